"""CPU oracle for the KV-cache hot path -- TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
import this package, and only as the checker (or the timed CPU baseline),
never as a product code path.  The product (serving-engine_amd/) has no CPU
fallback: it fails loudly when libkvhot.so is missing.

Modules
* paged_ref -- numpy restatement, fp64 arithmetic, of the reference algorithm:
  slot mapping and step metadata (serving_engine/model_runner.py:127-170,
  serving_engine/paged_attention_kernel.py:163-200), KV append
  (serving_engine/model_runner.py:21-32), block copy (closed form; no
  reference implementation exists), and paged attention with causal offset,
  GQA mapping and natural-log LSE (serving_engine/paged_attention_kernel.py:16-122
  semantics, serving_engine/model_runner.py:185-207 mask,
  transformers integrations/eager_paged.py:43-73 arithmetic).
* eager -- torch-CPU restatement of the reference's eager ("paged|eager")
  path in the model dtype: index_copy_ append, index_select gather, repeat_kv,
  dense masked fp32 softmax cast back to the model dtype, matmul.  This is the
  "reference PyTorch/CPU path" the parity bar and the CPU baseline refer to.

How each function is pinned (beyond restating the formula) is listed in the
tests: tests/test_oracle.py checks paged_ref against torch's
scaled_dot_product_attention and index_copy_, against pure-Python brute force
on tiny inputs, against closed-form special cases and invariants, and shows
that planted mistakes (wrong GQA map, off-by-one causal mask, missing scale,
log base) are caught.
"""
