"""Copy-on-write end to end on the GPU: the scheduler forks a request whose
last block is partly filled, both rows decode a token into that block, the
step's block copy runs on the GPU (step_inputs -> _PagedKVCache.copy_blocks),
and each row appends its own token and attends over its own keys.  The
blocks are checked bit-exactly and the attention against the oracle."""
import math

import numpy as np
import pytest
import torch

from oracle import paged_ref
from parity import check_attention

pytestmark = pytest.mark.gpu


def test_forked_rows_decode_into_private_copies(cuda, sea):
    print("[gpu-case] copy-on-write: fork at 20 tokens, two decode rows, 2 layers, 8/2 heads, D=64, bf16",
          flush=True)
    layers, nblocks, hkv, hq, d, bs = 2, 16, 2, 8, 64, 16
    dt = torch.bfloat16
    gen = torch.Generator(device=cuda).manual_seed(5)
    kv = sea.allocate_kv_cache(layers, nblocks, hkv, d, dtype=dt, device=cuda)
    kv.normal_(0.0, 0.5, generator=gen)
    cache = sea._PagedKVCache(kv)
    sched = sea.Scheduler(sea.BlockManager(nblocks))

    # Prefill the parent's 20 prompt tokens (the last block is 4/16 full).
    parent = sea.Request("p", list(range(20)))
    sched.add_request(parent)
    out = sched.schedule()
    meta, slots, _ = sea.step_inputs(out, cuda, cache)
    pk = torch.randn(1, hkv, 20, d, generator=gen, device=cuda).to(dt)
    pv = torch.randn(1, hkv, 20, d, generator=gen, device=cuda).to(dt)
    for layer in range(layers):
        cache.write(pk, pv, layer, slots)
    parent.output_token_ids = [7]
    sched.update_after_step(out)
    assert parent.phase == sea.RequestPhase.NEEDS_DECODE and parent.block_table == [15, 14]

    # Fork: the child shares both blocks, then both decode position 20.
    child = sea.Request("c", list(range(20)))
    child.output_token_ids = list(parent.output_token_ids)
    child.num_computed_tokens = parent.num_computed_tokens
    child.phase, child.status = sea.RequestPhase.NEEDS_DECODE, sea.RequestStatus.RUNNING
    sched.block_manager.fork(parent, child)
    sched.running.append(child)
    torch.cuda.synchronize()
    before = kv.clone()
    out = sched.schedule()
    assert out.scheduled_requests == [parent, child]
    (src, dst), = out.blocks_to_copy
    assert src == 14 and parent.block_table == [15, dst] and child.block_table == [15, 14]
    meta, slots, pos = sea.step_inputs(out, cuda, cache)
    assert slots.tolist() == [dst * bs + 4, 14 * bs + 4] and pos.tolist() == [20, 20]
    nk = torch.randn(1, hkv, 2, d, generator=gen, device=cuda).to(dt)
    nv = torch.randn(1, hkv, 2, d, generator=gen, device=cuda).to(dt)
    q = torch.randn(2, hq, d, generator=gen, device=cuda).to(dt)
    outs = []
    for layer in range(layers):
        cache.write(nk, nv, layer, slots)
        kc, vc = cache.blocks(layer)
        outs.append(sea.paged_flash_attention(q, kc, vc, meta, hq, hkv, 1.0 / math.sqrt(d)))
    torch.cuda.synchronize()

    # Blocks, bit-exactly: the copy holds the shared block's tokens with the
    # parent's new token at offset 4; the original holds the child's.
    after, before = kv.cpu(), before.cpu()
    for layer in range(layers):
        for kvi, new in ((0, nk), (1, nv)):
            new = new.cpu()[0]  # [Hkv, 2, D]
            a, b = after[layer, kvi], before[layer, kvi]
            assert torch.equal(a[15], b[15])
            assert torch.equal(a[dst, :4], b[14, :4]) and torch.equal(a[14, :4], b[14, :4])
            assert torch.equal(a[dst, 4], new[:, 0]) and torch.equal(a[14, 4], new[:, 1])
            others = [i for i in range(nblocks) if i not in (14, 15, dst)]
            assert torch.equal(a[others], b[others])

    # Attention of each row over its own 21 keys, against the oracle.
    q_lens, k_lens = np.array([1, 1]), np.array([21, 21])
    q_starts, offs = np.array([0, 1]), np.array([20, 20])
    bt = np.array([parent.block_table, child.block_table], dtype=np.int32)
    for layer, (o, lse) in enumerate(outs):
        kc = after[layer, 0].float().numpy()
        vc = after[layer, 1].float().numpy()
        ref_o, ref_l = paged_ref.paged_attention(q.float().cpu().numpy(), kc, vc, q_lens, k_lens, q_starts, offs,
                                                 bt, hq, hkv, 1.0 / math.sqrt(d))
        check_attention(o.float().cpu().numpy(), lse.cpu().numpy(), ref_o, ref_l, torch.bfloat16)
    # the two rows differ only in their last key, and do differ
    assert not torch.equal(outs[0][0][0], outs[0][0][1])
