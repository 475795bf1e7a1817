"""torch-CPU restatement of the reference's eager ("paged|eager") attention
path, in the model dtype.  TEST INFRASTRUCTURE ONLY (see oracle/__init__.py);
bench.py times it as the CPU baseline.

One layer of one engine step:
1. append: k_cache.view(-1, Hkv, D).index_copy_(0, write_index, key[S, Hkv, D])
   and the same for V (serving_engine/model_runner.py:21-32);
2. read indices, key positions and the dense additive mask, 0 where
   same-request and key_pos <= query_pos, finfo(dtype).min elsewhere
   (serving_engine/model_runner.py:185-207);
3. index_select gather of every read slot (serving_engine/model_runner.py:34-40);
4. repeat_kv, Q.K^T * scaling + mask, softmax in fp32 cast back to the model
   dtype, P.V, transpose to [S, Hq, D] (transformers
   integrations/eager_paged.py:7-16, 43-73).

`per_row=True` evaluates step 2-4 one row at a time: cross-row entries of the
whole-batch form are masked to probability 0, so the result is the same
mathematics with O(max row) instead of O(batch^2) memory.
"""
from __future__ import annotations

import torch


def repeat_kv(x: torch.Tensor, n_rep: int) -> torch.Tensor:
    """[1, Hkv, L, D] -> [1, Hkv * n_rep, L, D]; head h reads kv head h // n_rep."""
    b, h, l, d = x.shape
    if n_rep == 1:
        return x
    return x[:, :, None, :, :].expand(b, h, n_rep, l, d).reshape(b, h * n_rep, l, d)


def _attend(query, key, value, mask, scaling, n_rep):
    """query [1, Hq, S, D], key/value [1, Hkv, L, D], mask [1, 1, S, L] or None."""
    key = repeat_kv(key, n_rep)
    value = repeat_kv(value, n_rep)
    w = torch.matmul(query, key.transpose(2, 3)) * scaling
    if mask is not None:
        w = w + mask
    w = torch.nn.functional.softmax(w, dim=-1, dtype=torch.float32).to(query.dtype)
    return torch.matmul(w, value).transpose(1, 2).contiguous()  # [1, S, Hq, D]


def eager_step(q, key_new, value_new, k_cache, v_cache, write_index, rows, scale,
               num_kv_heads, per_row=False):
    """q [T, Hq, D]; key_new/value_new [T, Hkv, D] (the step's new K/V);
    k_cache/v_cache [N, bs, Hkv, D] (modified in place by the append);
    write_index int64 [T]; rows: list of (q_len, k_len, q_pos_offset,
    block_table).  Returns o [T, Hq, D] in q's dtype."""
    hkv = num_kv_heads
    d = q.shape[-1]
    bs = k_cache.shape[1]
    kf = k_cache.view(-1, hkv, d)
    vf = v_cache.view(-1, hkv, d)
    kf.index_copy_(0, write_index, key_new)
    vf.index_copy_(0, write_index, value_new)
    n_rep = q.shape[1] // hkv
    dtype = q.dtype

    def row_reads(r):
        n_q, n_k, off, bt = r
        pos = torch.arange(n_k)
        bt_t = torch.as_tensor(bt, dtype=torch.int64)
        slots = bt_t[pos // bs] * bs + pos % bs
        return slots, pos

    if per_row:
        outs = []
        start = 0
        for r in rows:
            n_q, n_k, off, _ = r
            slots, kpos = row_reads(r)
            qpos = off + torch.arange(n_q)
            allowed = kpos[None, :] <= qpos[:, None]
            mask = torch.zeros(n_q, n_k, dtype=dtype)
            mask.masked_fill_(~allowed, torch.finfo(dtype).min)
            key = torch.index_select(kf, 0, slots).transpose(0, 1).unsqueeze(0)
            value = torch.index_select(vf, 0, slots).transpose(0, 1).unsqueeze(0)
            query = q[start:start + n_q].transpose(0, 1).unsqueeze(0)
            outs.append(_attend(query, key, value, mask[None, None], scale, n_rep)[0])
            start += n_q
        return torch.cat(outs, dim=0) if outs else q.new_empty(q.shape)

    read, kpos, kgrp, qpos, qgrp = [], [], [], [], []
    for gi, r in enumerate(rows):
        n_q, n_k, off, _ = r
        slots, pos = row_reads(r)
        read.append(slots)
        kpos.append(pos)
        kgrp.append(torch.full((n_k,), gi))
        qpos.append(off + torch.arange(n_q))
        qgrp.append(torch.full((n_q,), gi))
    read = torch.cat(read)
    kpos, kgrp = torch.cat(kpos), torch.cat(kgrp)
    qpos, qgrp = torch.cat(qpos), torch.cat(qgrp)
    allowed = (qgrp[:, None] == kgrp[None, :]) & (kpos[None, :] <= qpos[:, None])
    mask = torch.zeros(qpos.numel(), read.numel(), dtype=dtype)
    mask.masked_fill_(~allowed, torch.finfo(dtype).min)
    key = torch.index_select(kf, 0, read).transpose(0, 1).unsqueeze(0)
    value = torch.index_select(vf, 0, read).transpose(0, 1).unsqueeze(0)
    query = q.transpose(0, 1).unsqueeze(0)
    return _attend(query, key, value, mask[None, None], scale, n_rep)[0]


def workload_rows(w):
    """(q_len, k_len, q_pos_offset, block_table) rows of a workloads.Workload."""
    return [(x.q_len, x.k_len, x.q_pos_offset, x.block_table) for x in w.rows]
