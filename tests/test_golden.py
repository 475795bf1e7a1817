"""The committed golden fixtures still agree with the oracle (CPU)."""
import math

import numpy as np
import pytest

from conftest import load_golden
from oracle import paged_ref


@pytest.mark.parametrize("name", ["config1_fp32.npz", "gqa_bf16_mixed.npz"])
def test_oracle_reproduces_golden(name):
    g = load_golden(name)
    kc, vc = paged_ref.reshape_and_cache(g["k_cache"].float().numpy(), g["v_cache"].float().numpy(),
                                         g["new_k"].float().numpy(), g["new_v"].float().numpy(),
                                         g["slot_mapping"])
    o, lse = paged_ref.paged_attention(g["q"].float().numpy(), kc, vc, g["q_lens"], g["k_lens"],
                                       g["q_starts"], g["q_pos_offsets"], g["block_table"],
                                       g["num_q_heads"], g["num_kv_heads"], 1.0 / math.sqrt(g["head_dim"]))
    np.testing.assert_allclose(o.astype(np.float32), g["expected_o"], rtol=1e-6, atol=1e-6)
    np.testing.assert_allclose(lse.astype(np.float32), g["expected_lse"], rtol=1e-6, atol=1e-6)
    # every query token wrote its own slot: its position in its row's table
    for r in range(len(g["q_lens"])):
        for i in range(int(g["q_lens"][r])):
            pos = int(g["q_pos_offsets"][r]) + i
            blk = int(g["block_table"][r][pos // 16])
            assert g["slot_mapping"][int(g["q_starts"][r]) + i] == blk * 16 + pos % 16
