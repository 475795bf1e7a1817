"""The engine loop end to end on the GPU: Scheduler + BlockManager (chunked
prefill under a token cap, decode, a forked request whose first decode goes
through copy-on-write) drive a small random-weight Llama whose attention is
paged|hip, one greedy token per row and step; step_inputs builds each step's
metadata, slot mapping and positions and runs the block copies.  Every
sampled token and its logits are checked against transformers' own eager
attention over the whole sequence, in fp32 on the CPU."""
import copy

import pytest
import torch

pytestmark = pytest.mark.gpu

transformers = pytest.importorskip("transformers")


def _config(attn):
    from transformers import LlamaConfig

    cfg = LlamaConfig(vocab_size=500, hidden_size=256, intermediate_size=512, num_hidden_layers=2,
                      num_attention_heads=8, num_key_value_heads=2, head_dim=64,
                      max_position_embeddings=512, rope_theta=10000.0)
    cfg._attn_implementation = attn
    return cfg


def test_scheduler_driven_decode_matches_dense_attention(cuda, sea):
    print("[gpu-case] engine loop: 3 requests + 1 fork, chunked prefill, 2-layer fp32 Llama (8/2 heads, D=64)",
          flush=True)
    from transformers import LlamaForCausalLM

    torch.manual_seed(3)
    model = LlamaForCausalLM(_config(sea.register_attention())).eval()
    dense = copy.deepcopy(model)
    dense.config._attn_implementation = "eager"
    for layer in dense.model.layers:
        layer.self_attn.config._attn_implementation = "eager"
    model = model.to(cuda)

    nblocks, new_tokens = 16, 6
    kv = sea.allocate_kv_cache(2, nblocks, 2, 64, dtype=torch.float32, device=cuda)
    cache = sea._PagedKVCache(kv)
    bm = sea.BlockManager(nblocks)
    sched = sea.Scheduler(bm, max_num_batched_tokens=32, min_chunk_size=8)
    gen = torch.Generator().manual_seed(9)
    reqs = [sea.Request(f"r{i}", torch.randint(0, 500, (n,), generator=gen).tolist(), max_new_tokens=new_tokens)
            for i, n in enumerate((20, 37, 50))]
    for r in reqs:
        sched.add_request(r)
    logits_of = {}  # request id -> list of the logits rows that sampled its tokens
    forked = None
    copies = 0
    for step in range(40):
        if not sched.has_unfinished_requests():
            break
        out = sched.schedule()
        copies += len(out.blocks_to_copy)
        meta, slots, pos = sea.step_inputs(out, cuda, cache)
        ids = []
        for r in out.scheduled_requests:
            toks = r.all_token_ids()
            if r.phase == sea.RequestPhase.NEEDS_PREFILL:
                ids += toks[r.num_computed_tokens:r.num_computed_tokens + out.prefill_chunk_sizes[r.request_id]]
            else:
                ids.append(toks[-1])
        with torch.no_grad():
            logits = model(input_ids=torch.tensor([ids], device=cuda), position_ids=pos.view(1, -1), cache=cache,
                           write_index=slots, paged_metadata=meta, use_cache=False).logits[0].float().cpu()
        starts = meta["q_starts"].tolist()
        lens = meta["q_lens"].tolist()
        for i, r in enumerate(out.scheduled_requests):
            if r.phase == sea.RequestPhase.NEEDS_DECODE or r.request_id in out.prefill_final_chunk:
                row = logits[starts[i] + lens[i] - 1]
                r.output_token_ids.append(int(row.argmax()))
                logits_of.setdefault(r.request_id, []).append(row)
        sched.update_after_step(out)
        if forked is None and reqs[0].phase == sea.RequestPhase.NEEDS_DECODE:
            # Fork request 0 right after its prefill: the child shares every
            # block, including the partly filled last one both write next.
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
        seq = torch.tensor([r.all_token_ids()[:-1]])
        with torch.no_grad():
            ref = dense(input_ids=seq).logits[0, r.prompt_len - 1:].float()
        got = torch.stack(logits_of[r.request_id])
        torch.testing.assert_close(got, ref, atol=2e-3, rtol=1e-3)
        assert r.output_token_ids == ref.argmax(-1).tolist()
    assert forked.output_token_ids == reqs[0].output_token_ids
