"""The engine loop in bf16, on the MFMA kernels, against an independent
reference.

A small random-weight Llama (8 query / 2 kv heads, head_dim 64: the shape
class of the 64-row GQA workload, G = 4) runs in bf16 on paged|hip attention,
so the decode, merge and prefill MFMA kernels do the attention.  The
reference is the same weights (the bf16 values, held in fp32) in
transformers' dense eager attention on the CPU in fp32, run over each
request's whole token sequence.

* Scheduler + BlockManager drive chunked prefill, decode and a forked request
  whose first decode goes through copy-on-write; each step is sample_step
  (forward_step with logits_to_keep, argmax on the device, one host copy of
  the step's tokens).
* Decode-only steps run as replays of DecodeStepGraph after an eager
  prefill.
* A prefilled request forked five times: six decode rows share their
  leading blocks (copy-on-write of the last one), so the launch list
  attends the shared prefix once (shared-prefix units), eagerly and in
  graph replays.

Every sampled token's logits row is checked against the reference within
atol 2e-2 / rtol 1e-2, the bf16 bar of the attention parity tests (measured
here: at most 0.0075 off), and the token must be the reference's argmax
wherever the reference's top two logits are more than 0.04 apart (a near
tie may go either way: the attention's summation order is set at run
time).  Pattern of the reference's own check:
tests/test_correctness.py:249-279 (kernel path against the eager path).
"""
import copy

import pytest
import torch

pytestmark = pytest.mark.gpu

transformers = pytest.importorskip("transformers")

ATOL, RTOL, TIE = 2e-2, 1e-2, 0.04


def _models(sea, device):
    from transformers import LlamaConfig, LlamaForCausalLM

    cfg = LlamaConfig(vocab_size=500, hidden_size=256, intermediate_size=512, num_hidden_layers=2,
                      num_attention_heads=8, num_key_value_heads=2, head_dim=64,
                      max_position_embeddings=2048, rope_theta=10000.0)
    cfg._attn_implementation = sea.register_attention()
    torch.manual_seed(3)
    model = LlamaForCausalLM(cfg).to(torch.bfloat16).eval()
    dense = copy.deepcopy(model).float()
    dense.config._attn_implementation = "eager"
    for layer in dense.model.layers:
        layer.self_attn.config._attn_implementation = "eager"
    return model.to(device), dense


def _check_against_dense(dense, requests, logits_of):
    worst = 0.0
    for r in requests:
        seq = torch.tensor([r.all_token_ids()[:-1]])
        with torch.no_grad():
            ref = dense(input_ids=seq).logits[0, r.prompt_len - 1:].float()
        got = torch.stack(logits_of[r.request_id]).float().cpu()
        worst = max(worst, float((got - ref).abs().max()))
        torch.testing.assert_close(got, ref, atol=ATOL, rtol=RTOL)
        top2 = ref.topk(2, dim=-1).values
        clear = (top2[:, 0] - top2[:, 1]) > TIE
        toks = torch.tensor(r.output_token_ids)
        assert torch.equal(toks[clear], ref.argmax(-1)[clear]), r.request_id
    print(f"[gpu-case] largest logit difference from the dense fp32 reference: {worst:.4f}", flush=True)


def test_bf16_engine_loop_matches_dense_attention(cuda, sea):
    print("[gpu-case] bf16 engine loop: 3 requests + 1 fork, chunked prefill, sample_step", flush=True)
    model, dense = _models(sea, cuda)
    nblocks, new_tokens = 24, 6
    kv = sea.allocate_kv_cache(2, nblocks, 2, 64, dtype=torch.bfloat16, device=cuda)
    cache = sea._PagedKVCache(kv)
    bm = sea.BlockManager(nblocks)
    sched = sea.Scheduler(bm, max_num_batched_tokens=48, min_chunk_size=8)
    gen = torch.Generator().manual_seed(9)
    reqs = [sea.Request(f"r{i}", torch.randint(0, 500, (n,), generator=gen).tolist(), max_new_tokens=new_tokens)
            for i, n in enumerate((20, 61, 90))]
    for r in reqs:
        sched.add_request(r)
    logits_of, forked, copies = {}, None, 0
    for _ in range(60):
        if not sched.has_unfinished_requests():
            break
        out, logits = sea.sample_step(model, sched, cache, cuda)
        if logits is None:
            continue
        copies += len(out.blocks_to_copy)
        assert logits.shape == (len(out.scheduled_requests), 500)  # one row per request
        # sample_step has already moved the rows' phases on; record by what the step was
        for i, r in enumerate(out.scheduled_requests):
            sampled = r.request_id in out.prefill_final_chunk or (
                r.request_id not in out.prefill_chunk_sizes)
            if sampled:
                logits_of.setdefault(r.request_id, []).append(logits[i].float())
        if forked is None and reqs[0].phase == sea.RequestPhase.NEEDS_DECODE:
            p = reqs[0]
            forked = sea.Request("fork", list(p.prompt_token_ids), max_new_tokens=new_tokens,
                                 output_token_ids=list(p.output_token_ids))
            forked.num_computed_tokens = p.num_computed_tokens
            forked.phase, forked.status = p.phase, sea.RequestStatus.RUNNING
            bm.fork(p, forked)
            sched.running.append(forked)
            logits_of["fork"] = list(logits_of[p.request_id])
    assert not sched.has_unfinished_requests(), "the loop did not finish"
    assert copies >= 1, "the fork's shared last block was never copied"
    assert bm.get_num_free_blocks() == nblocks
    for r in reqs + [forked]:
        assert len(r.output_token_ids) == new_tokens
        assert len(logits_of[r.request_id]) == new_tokens
    _check_against_dense(dense, reqs + [forked], logits_of)


def test_bf16_graph_decode_matches_dense_attention(cuda, sea):
    print("[gpu-case] bf16 decode steps replayed from DecodeStepGraph after an eager prefill", flush=True)
    model, dense = _models(sea, cuda)
    nblocks, new_tokens = 40, 8
    kv = sea.allocate_kv_cache(2, nblocks, 2, 64, dtype=torch.bfloat16, device=cuda)
    cache = sea._PagedKVCache(kv)
    bm = sea.BlockManager(nblocks)
    sched = sea.Scheduler(bm, max_num_batched_tokens=512, min_chunk_size=8)
    gen = torch.Generator().manual_seed(21)
    reqs = [sea.Request(f"g{i}", torch.randint(0, 500, (n,), generator=gen).tolist(), max_new_tokens=new_tokens)
            for i, n in enumerate((33, 100, 16, 150))]
    for r in reqs:
        sched.add_request(r)
    logits_of = {}
    # Eager prefill (and decode steps until every request decodes).
    while any(r.phase != sea.RequestPhase.NEEDS_DECODE for r in reqs):
        out, logits = sea.sample_step(model, sched, cache, cuda)
        for i, r in enumerate(out.scheduled_requests):
            if r.request_id in out.prefill_final_chunk or r.request_id not in out.prefill_chunk_sizes:
                logits_of.setdefault(r.request_id, []).append(logits[i].float())
    max_blocks = (max(r.prompt_len for r in reqs) + new_tokens) // 16 + 1
    graph = sea.DecodeStepGraph(model, cache, len(reqs), max_blocks, 8, 2, 64, cuda)
    replays = 0
    while sched.has_unfinished_requests():
        out = sched.schedule()
        rows = out.scheduled_requests
        assert len(rows) == len(reqs) and not out.prefill_chunk_sizes  # decode-only steps
        graph.tokens.copy_(torch.tensor([r.output_token_ids[-1] for r in rows], device=cuda))
        toks = graph.step([r.total_len for r in rows], [list(r.block_table) for r in rows]).cpu().tolist()
        replays += 1
        for i, r in enumerate(rows):
            r.output_token_ids.append(int(toks[i]))
            logits_of.setdefault(r.request_id, []).append(graph.logits[i].float().clone())
        sched.update_after_step(out)
    assert replays >= new_tokens - 2
    for r in reqs:
        assert len(r.output_token_ids) == new_tokens
    _check_against_dense(dense, reqs, logits_of)


def test_bf16_shared_prefix_decode_matches_dense_attention(cuda, sea):
    print("[gpu-case] bf16 decode of six rows sharing 18 blocks (a request and five forks), eager then graph",
          flush=True)
    model, dense = _models(sea, cuda)
    nblocks, new_tokens = 48, 7
    kv = sea.allocate_kv_cache(2, nblocks, 2, 64, dtype=torch.bfloat16, device=cuda)
    cache = sea._PagedKVCache(kv)
    bm = sea.BlockManager(nblocks)
    sched = sea.Scheduler(bm, max_num_batched_tokens=512, min_chunk_size=8)
    gen = torch.Generator().manual_seed(33)
    base = sea.Request("p", torch.randint(0, 500, (300,), generator=gen).tolist(), max_new_tokens=new_tokens)
    sched.add_request(base)
    logits_of = {}
    while base.phase != sea.RequestPhase.NEEDS_DECODE:
        out, logits = sea.sample_step(model, sched, cache, cuda)
        if base.request_id in out.prefill_final_chunk:
            logits_of["p"] = [logits[0].float()]
    reqs = [base]
    for i in range(5):
        f = sea.Request(f"f{i}", list(base.prompt_token_ids), max_new_tokens=new_tokens,
                        output_token_ids=list(base.output_token_ids))
        f.num_computed_tokens = base.num_computed_tokens
        f.phase, f.status = base.phase, sea.RequestStatus.RUNNING
        bm.fork(base, f)
        sched.running.append(f)
        logits_of[f.request_id] = list(logits_of["p"])
        reqs.append(f)
    # one eager decode step: the shared partial last block is copied on write
    out, logits = sea.sample_step(model, sched, cache, cuda)
    assert len(out.blocks_to_copy) >= 5
    for i, r in enumerate(out.scheduled_requests):
        logits_of[r.request_id].append(logits[i].float())
    max_blocks = (300 + new_tokens) // 16 + 1
    graph = sea.DecodeStepGraph(model, cache, len(reqs), max_blocks, 8, 2, 64, cuda)
    while sched.has_unfinished_requests():
        out = sched.schedule()
        rows = out.scheduled_requests
        assert len(rows) == len(reqs) and not out.prefill_chunk_sizes
        if out.blocks_to_copy:
            cache.copy_blocks([s for s, _ in out.blocks_to_copy], [d for _, d in out.blocks_to_copy])
        graph.tokens.copy_(torch.tensor([r.output_token_ids[-1] for r in rows], device=cuda))
        toks = graph.step([r.total_len for r in rows], [list(r.block_table) for r in rows]).cpu().tolist()
        assert graph._recorded[4] > 0, "the launch list has no shared-prefix units"
        for i, r in enumerate(rows):
            r.output_token_ids.append(int(toks[i]))
            logits_of.setdefault(r.request_id, []).append(graph.logits[i].float().clone())
        sched.update_after_step(out)
    for r in reqs:
        assert len(r.output_token_ids) == new_tokens
    _check_against_dense(dense, reqs, logits_of)
