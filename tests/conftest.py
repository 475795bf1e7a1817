import importlib
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X GPU (runs the HIP kernels)")


def sea_module(name=None):
    """The product package (its directory name is not an identifier)."""
    full = "serving-engine_amd" + (f".{name}" if name else "")
    return importlib.import_module(full)


@pytest.fixture(scope="session")
def sea():
    return sea_module()


@pytest.fixture(scope="session")
def workloads():
    return sea_module("workloads")


@pytest.fixture(scope="session")
def cuda():
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no GPU visible")
    return torch.device("cuda:0")


GOLDEN = os.path.join(ROOT, "tests", "golden")


def load_golden(name):
    """A golden step fixture as a dict: numpy metadata/expected arrays plus
    torch CPU tensors q, new_k, new_v ([T, Hkv, D]) and the full pools
    k_cache / v_cache ([N, bs, Hkv, D]) rebuilt from the stored blocks."""
    import numpy as np
    import torch

    z = np.load(os.path.join(GOLDEN, name), allow_pickle=False)
    dtype = getattr(torch, str(z["dtype"]))
    hq, hkv, d, bs, n = (int(x) for x in z["heads"])

    def t(a):
        a = np.ascontiguousarray(a)
        if a.dtype == np.uint16:
            return torch.from_numpy(a.view(np.int16)).view(dtype)
        return torch.from_numpy(a)

    kc = torch.zeros(n, bs, hkv, d, dtype=dtype)
    vc = torch.zeros(n, bs, hkv, d, dtype=dtype)
    used = torch.from_numpy(z["used_blocks"])
    kc[used] = t(z["k_blocks"])
    vc[used] = t(z["v_blocks"])
    out = {k: z[k] for k in ("slot_mapping", "q_lens", "k_lens", "q_starts", "q_pos_offsets",
                             "block_table", "expected_o", "expected_lse", "used_blocks")}
    out.update(dtype=dtype, num_q_heads=hq, num_kv_heads=hkv, head_dim=d, block_size=bs, num_blocks=n,
               q=t(z["q"]), new_k=t(z["new_k"]), new_v=t(z["new_v"]), k_cache=kc, v_cache=vc)
    return out
