"""Decode steps replayed from a recorded HIP graph (DecodeStepGraph) against
the same steps run eagerly, on a small random-weight Llama whose attention is
paged|hip.  Each replay is checked against its eager step, with the eager
work and synchronisations in between; a step whose launch list needs other
unit counts records the graph again and must still agree."""
import math

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

transformers = pytest.importorskip("transformers")


class _Row:
    """A decode request as build_paged_batch_metadata reads it."""

    def __init__(self, rid, total_len, table, phase):
        self.request_id = rid
        self.total_len = total_len
        self.num_computed_tokens = total_len - 1
        self.block_table = table
        self.phase = phase


def _model(sea, device):
    from transformers import LlamaConfig, LlamaForCausalLM

    cfg = LlamaConfig(vocab_size=1000, hidden_size=512, intermediate_size=1024, num_hidden_layers=2,
                      num_attention_heads=8, num_key_value_heads=2, head_dim=64,
                      max_position_embeddings=16384, rope_theta=10000.0)
    cfg._attn_implementation = sea.register_attention()
    torch.manual_seed(11)
    return LlamaForCausalLM(cfg).to(device=device, dtype=torch.bfloat16).eval()


def _eager_step(sea, model, cache, lens, tables, tok, device):
    so = sea.SchedulerOutput()
    for i, (ln, tb) in enumerate(zip(lens, tables)):
        so.scheduled_requests.append(_Row(f"r{i}", ln, tb, sea.RequestPhase.NEEDS_DECODE))
    meta = sea.build_paged_batch_metadata(so, device=device)
    with torch.no_grad():
        out = model(input_ids=tok.view(1, -1), position_ids=meta["positions"].view(1, -1), cache=cache,
                    write_index=meta["slot_mapping"], paged_metadata=meta, use_cache=False)
    logits = out.logits[0].float()
    return logits, logits.argmax(-1)


def test_decode_graph_replays_match_eager_steps(cuda, sea):
    print("[gpu-case] decode step graph vs eager, 8 rows, 2-layer Llama (D=64, G=4)", flush=True)
    model = _model(sea, cuda)
    rng = np.random.default_rng(5)
    start = [17, 30, 64, 100, 1, 16, 33, 200]
    steps = 4
    long_len = 6000  # one step with a row this long needs a cut launch list
    max_blocks = math.ceil((long_len + steps) / 16)
    need = [math.ceil((s + steps) / 16) for s in start]
    need[0] = max_blocks
    nblocks = sum(need) + 5
    perm = rng.permutation(nblocks)
    tables, k = [], 0
    for nb in need:
        tables.append([int(b) for b in perm[k:k + nb]])
        k += nb
    kv = sea.allocate_kv_cache(2, nblocks, 2, 64, dtype=torch.bfloat16, device=cuda)
    kv.normal_(0.0, 0.125, generator=torch.Generator(device=cuda).manual_seed(3))
    kv_eager = kv.clone()
    cache, cache_eager = sea._PagedKVCache(kv), sea._PagedKVCache(kv_eager)

    g = sea.DecodeStepGraph(model, cache, len(start), max_blocks, 8, 2, 64, cuda)
    tok = torch.tensor(rng.integers(0, 1000, len(start)), dtype=torch.int64, device=cuda)
    g.tokens.copy_(tok)
    lens = [s + 1 for s in start]
    for s in range(steps):
        if s == 2:
            lens[0] = long_len
        logits_e, tok_e = _eager_step(sea, model, cache_eager, lens, tables, tok, cuda)
        out = g.step(lens, tables)
        torch.cuda.synchronize()
        torch.testing.assert_close(g.logits.float(), logits_e, atol=5e-2, rtol=2e-2)
        # Tokens agree wherever the eager step's top two logits are apart by
        # more than the tolerance (a near tie may go either way: the
        # attention's summation order is set at run time).
        top2 = logits_e.topk(2, dim=-1).values
        clear = (top2[:, 0] - top2[:, 1]) > 0.1
        assert torch.equal(out[clear], tok_e[clear]), f"step {s}: tokens differ"
        g.tokens.copy_(tok_e)  # both continue from the eager tokens
        tok = tok_e
        lens = [x + 1 for x in lens]
    assert g.recordings >= 2  # the long row's step recorded again (and the next step back)
    torch.testing.assert_close(kv.float(), kv_eager.float(), atol=2e-2, rtol=1e-2)
