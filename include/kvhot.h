/*
 * kvhot.h -- C ABI of the MI355X (gfx950) KV-cache hot path of a paged-attention
 * serving engine.
 *
 * Every entry point is stateless and stream-ordered on the caller's hipStream_t
 * (passed as `void* stream`; NULL means the legacy default stream).  Device
 * buffers are plain device pointers owned by the caller; no entry point
 * allocates or frees device memory.  Sizes and strides are int64 and strides
 * are in ELEMENTS of the tensor they describe.  All arguments are validated on
 * the host before any launch.
 *
 * Return codes: 0 = success; negative = invalid argument (see KVHOT_E*; nothing
 * was launched); positive = a hipError_t from the launch.
 * kvhot_last_error() returns a human-readable description of the most recent
 * failure on the calling thread.
 *
 * Layouts (same as the reference engine):
 *   KV pool of one layer:  k_cache / v_cache [num_blocks, block_size, num_kv_heads, head_dim]
 *                          (serving_engine/model_runner.py:101-110, :42-45)
 *   Whole pool:            kv_cache [num_layers, 2, num_blocks, block_size, num_kv_heads, head_dim]
 *   Queries:               q [total_query, num_q_heads, head_dim]   (head_dim stride must be 1)
 *   Block table:           int32 [num_rows, bt_row_stride], padded with 0
 *                          (serving_engine/paged_attention_kernel.py:189-197)
 *   GQA: query head h reads kv head h / (num_q_heads / num_kv_heads)
 *        (serving_engine/paged_attention_kernel.py:81).
 * Those are the logical shapes: every entry point takes the pool's strides,
 * so a block may lie in memory token-major (the reference's [block_size,
 * num_kv_heads, head_dim]), head-major ([num_kv_heads, block_size,
 * head_dim]) or kv-interleaved (K and V of one block together,
 * [num_kv_heads, 2, block_size, head_dim]: the fastest for decode).
 */
#ifndef KVHOT_H
#define KVHOT_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Element types. */
enum {
  KVHOT_F32 = 0,
  KVHOT_F16 = 1,
  KVHOT_BF16 = 2
};

/* attn_flags bits of kvhot_paged_attention(_noalloc) and
 * kvhot_paged_attention_schedule.  1 and 0 keep the meaning of the
 * reference's is_causal argument (serving_engine/paged_attention_kernel.py:125). */
enum {
  KVHOT_CAUSAL = 1,        /* key j is visible to query i iff j <= q_pos_offset + i */
  KVHOT_DETERMINISTIC = 2, /* bitwise-repeatable out and lse: decode waves walk their
                              planned key ranges in order, with no run-time sharing */
  KVHOT_VERIFY_BLOCKS = 4  /* decode waves check the first block of their range that
                              the launch list took from the host copy of the block
                              table against the device table, and use the device
                              table's (for callers that edit only the device copy);
                              costs about 1-2% of a decode call */
};

/* Invalid-argument codes (negative return values). */
enum {
  KVHOT_EINVAL = -1,       /* a size, stride, pointer or dtype is invalid */
  KVHOT_EUNSUPPORTED = -2, /* the shape is valid but no kernel covers it */
  KVHOT_EWORKSPACE = -3    /* workspace missing or smaller than required */
};

/* Library version, for binding sanity checks: major*10000 + minor*100 + patch. */
int kvhot_version(void);

/* Description of the most recent error on the calling thread ("" if none). */
const char* kvhot_last_error(void);

/*
 * KV append ("reshape_and_cache"): for i in [0, num_tokens):
 *   s = slot_mapping[i]; if 0 <= s < num_blocks*block_size:
 *     k_cache[s / block_size, s % block_size, :, :] = key[i, :, :]
 *     v_cache[s / block_size, s % block_size, :, :] = value[i, :, :]
 * Negative or out-of-range slots are skipped (padding).  Bit-exact byte copy,
 * K and V in one launch.
 * key/value: [num_tokens, num_kv_heads, head_dim] with strides key_strides[3] /
 * value_strides[3] (the reference passes the transposed view
 * key_states.transpose(1, 2).squeeze(0)).  Cache strides are [4] (block, token,
 * head, dim).  slot_is_int64: 1 for int64 slots (the reference's write_index),
 * 0 for int32.
 * Replaces _PagedKVCache.write (serving_engine/model_runner.py:21-32), i.e.
 * k_cache.view(-1, Hkv, D).index_copy_(0, write_index, key_states) and the same
 * for V.
 */
int kvhot_reshape_and_cache(const void* key, const int64_t key_strides[3],
                            const void* value, const int64_t value_strides[3],
                            void* k_cache, const int64_t k_cache_strides[4],
                            void* v_cache, const int64_t v_cache_strides[4],
                            const void* slot_mapping, int slot_is_int64,
                            int64_t num_tokens, int64_t num_kv_heads,
                            int64_t head_dim, int64_t block_size,
                            int64_t num_blocks, int dtype, void* stream);

/*
 * Block copy for prefix-cache copy-on-write: for every pair i, every layer and
 * both K and V, copy the bytes of block src_block_ids[i] to block
 * dst_block_ids[i]:  kv_cache[:, :, dst[i]] = kv_cache[:, :, src[i]].
 * The whole-pool tensor is described by its base pointer and BYTE strides of
 * its first three dims (layer, K/V, block); each block's payload of
 * block_bytes bytes must be contiguous.  (A kv-interleaved pool, whose K and
 * V of one block are one range of 2 * block_bytes, is copied by passing half
 * of that range as block_bytes and its offset as the K/V stride.)  Destinations must be unique and must
 * not appear among the sources of the same call (the copies run in parallel).
 * Ids outside [0, num_blocks) are skipped.
 * The reference has no block copy: fork() shares blocks by reference count
 * (serving_engine/block_manager.py:129-132) and its copy-on-write branch was
 * removed (handoff.md:716-722, 842-853); this entry point is the data mover a
 * copy-on-write fork needs.
 */
int kvhot_copy_blocks(void* kv_cache, int64_t num_layers,
                      int64_t layer_stride_bytes, int64_t kv_stride_bytes,
                      int64_t block_stride_bytes, int64_t block_bytes,
                      int64_t num_blocks, const int64_t* src_block_ids,
                      const int64_t* dst_block_ids, int64_t num_pairs,
                      void* stream);

/*
 * Device-side slot mapping and RoPE positions for one engine step.  For row r
 * and i in [0, q_lens[r]):
 *   pos = q_pos_offsets[r] + i
 *   positions[q_starts[r] + i]    = pos
 *   slot_mapping[q_starts[r] + i] = block_table[r, pos / block_size] * block_size
 *                                   + pos % block_size
 * (slot -1 if pos / block_size >= bt_row_stride).  Replaces the per-token
 * Python loop of ModelRunner.forward (serving_engine/model_runner.py:142-170)
 * and ModelRunner._flat_slot (:127-129).  max_q_len bounds q_lens; outputs
 * are written only at indices below total_query (their length).
 */
int kvhot_build_slot_mapping(const int32_t* block_table, int64_t bt_row_stride,
                             const int32_t* q_lens, const int32_t* q_starts,
                             const int32_t* q_pos_offsets, int64_t num_rows,
                             int64_t total_query, int64_t max_q_len,
                             int64_t block_size, int64_t* slot_mapping,
                             int64_t* positions, void* stream);

/*
 * Workspace bytes kvhot_paged_attention needs for these sizes when it is
 * called WITHOUT a schedule (0 if it needs none): split-K partition results
 * of decode rows, fully rewritten by each call before they are read, so a
 * workspace needs no initialisation and may be reused by calls of any shape
 * that fits.  Calls sharing a workspace must be ordered on one stream.
 * Returns a negative KVHOT_E* code for invalid sizes.  (With a schedule, the
 * size comes from kvhot_paged_attention_schedule.)
 */
int64_t kvhot_paged_attention_workspace_bytes(
    int64_t num_rows, int64_t total_query, int64_t max_q_len,
    int64_t max_k_len, int64_t num_q_heads, int64_t num_kv_heads,
    int64_t head_dim, int64_t block_size, int64_t partition_tokens, int dtype);

/*
 * Launch list ("schedule") for kvhot_paged_attention, built on the host from
 * HOST copies of q_lens, k_lens, q_starts, q_pos_offsets and the block table,
 * with the head counts, head_dim, block_size, attn_flags (KVHOT_CAUSAL; the
 * KVHOT_DETERMINISTIC and KVHOT_VERIFY_BLOCKS bits are accepted and do not
 * change the plan) and dtype
 * the attention call will get.  The (row, kv head) key ranges of decode rows are
 * laid end to end and cut into equal numbers of 16-token slices per decode
 * work-group, one device-full of work-groups; a range cut in two becomes
 * "parts" in different work-groups.  Units of 8 int32, in order:
 * num_decode_units range descriptors (whole work-groups: one per wave, or
 * with partition_tokens > 0 up to four per wave; each carries its row's
 * metadata and first block, so the wave's first K/V loads depend on nothing
 * else; with KVHOT_VERIFY_BLOCKS in the attention call's attn_flags the
 * kernel checks that block against the device block table before using it), num_prefill_units per-work-group prefill units (longest
 * first), num_merge_units units, one per decode range cut into parts.
 * Shared prefixes: when at least 4 decode rows (with causal masking or not)
 * read the same first 256 or more keys through the same physical blocks, the
 * keys of that common prefix are attended once, for all of those rows'
 * queries together, by prefix units on the MFMA prefill path; each row's
 * decode work-group then reads only its own tail and folds the prefix
 * partials into its output (a row whose tail is cut across work-groups
 * has them folded in by its merge unit instead).  The first
 * *num_prefix_units of the prefill units are such prefix units (they run
 * before the decode launch).
 * partition_tokens > 0 (a multiple of 32 up to 2^20) first cuts every decode
 * row into partitions of that many keys, which are then never cut further;
 * 0 leaves the cuts to the planner.  *workspace_bytes receives the workspace
 * the attention call needs with this schedule (0: none).  Returns the total
 * unit count (units are written when `units` is non-NULL and capacity_units
 * suffices) or a negative KVHOT_E* code.  A schedule depends only on the
 * step's lengths, so one upload serves every layer of an engine step.
 * Without a schedule the attention launch covers the padded grid of (row,
 * partition, head group), and work-groups without work still cost a launch
 * slot each.
 */
int64_t kvhot_paged_attention_schedule(
    const int32_t* q_lens, const int32_t* k_lens, const int32_t* q_starts,
    const int32_t* q_pos_offsets, const int32_t* block_table,
    int64_t bt_row_stride, int64_t num_rows, int64_t num_q_heads, int64_t num_kv_heads,
    int64_t head_dim, int64_t block_size, int64_t partition_tokens,
    int attn_flags, int dtype, int32_t* units, int64_t capacity_units,
    int64_t* num_decode_units, int64_t* num_prefill_units,
    int64_t* num_merge_units, int64_t* workspace_bytes,
    int64_t* num_prefix_units);

/*
 * Paged attention forward over a ragged batch of rows (prefill chunks and
 * decode rows mixed), one call per layer.  For row r with n_q = q_lens[r],
 * n_k = k_lens[r], off = q_pos_offsets[r], and each query i < n_q (global
 * token t = q_starts[r] + i) and query head h:
 *   keys j in [0, n_k) are read through block_table[r, j / block_size];
 *   with KVHOT_CAUSAL in attn_flags, key j is visible iff j <= off + i;
 *   out[t, h, :] = softmax_j(scale * q[t,h,:] . k_j) @ v_j   (fp32 accumulate)
 *   lse[t, h]    = natural-log logsumexp_j(scale * q[t,h,:] . k_j)
 * A query with no visible key gets out = 0 and lse = -inf.
 * Rows with n_q == 1 run the split-K flash-decoding kernel, plus a merge
 * launch when a decode row was split across work-groups; rows with
 * n_q >= 2 run the chunked-prefill kernel.  max_q_len / max_k_len must bound
 * q_lens / k_lens (they size the grid; no device->host sync is made).
 * schedule: device copy of the units from kvhot_paged_attention_schedule for
 * exactly these lengths and sizes, with its four unit counts, the workspace
 * size it reported (schedule_workspace_bytes) and a workspace at least that
 * large (a shorter one fails with KVHOT_EWORKSPACE before any launch); or
 * NULL, and then partition_tokens (keys per decode partition; 0 picks a
 * size, otherwise a multiple of 32 up to 2^20) and
 * kvhot_paged_attention_workspace_bytes apply.  Decode waves of one
 * work-group share out their slices at run time (the waves of a CU stream at
 * different rates), so the summation order, and with it the last bits of out
 * and lse, can differ from call to call; with KVHOT_DETERMINISTIC in
 * attn_flags every wave walks its planned range alone and repeated calls
 * give the same bits (the work-group then ends with its slowest wave).
 * Other attn_flags bits are invalid.  lse may be NULL.  out has the dtype of
 * q, k_cache and v_cache; lse is fp32.  Replaces paged_flash_attention +
 * paged_flash_fwd_kernel (serving_engine/paged_attention_kernel.py:16-160).
 */
int kvhot_paged_attention(
    const void* q, const int64_t q_strides[3],
    const void* k_cache, const int64_t k_cache_strides[4],
    const void* v_cache, const int64_t v_cache_strides[4],
    void* out, const int64_t out_strides[3],
    float* lse, const int64_t lse_strides[2],
    const int32_t* block_table, int64_t bt_row_stride,
    const int32_t* q_lens, const int32_t* k_lens, const int32_t* q_starts,
    const int32_t* q_pos_offsets, int64_t num_rows, int64_t total_query,
    int64_t max_q_len, int64_t max_k_len, int64_t num_q_heads,
    int64_t num_kv_heads, int64_t head_dim, int64_t block_size,
    int64_t num_blocks, float scale, int attn_flags, int dtype,
    int64_t partition_tokens, const int32_t* schedule,
    int64_t num_decode_units, int64_t num_prefill_units,
    int64_t num_merge_units, int64_t num_prefix_units,
    int64_t schedule_workspace_bytes,
    void* workspace, int64_t workspace_bytes,
    void* stream);

/* Bytes of split-K partials kvhot_paged_attention_noalloc can hold (64 MiB). */
#define KVHOT_NOALLOC_SCRATCH_BYTES (64LL << 20)

/*
 * kvhot_paged_attention for callers that cannot allocate device memory (code
 * under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc); it has no counterpart in the reference.  Same arguments and
 * results as kvhot_paged_attention, without workspace / workspace_bytes: the
 * split-K partials go to a device-global array of
 * KVHOT_NOALLOC_SCRATCH_BYTES, one on each device the library runs on, held
 * until the process ends.  A call that needs more (the schedule's
 * schedule_workspace_bytes, or kvhot_paged_attention_workspace_bytes without
 * a schedule) fails with KVHOT_EWORKSPACE before any launch.  Allocates
 * nothing: no device memory, and no stream or event (a mixed batch's prefill
 * and decode launches both go to the caller's stream).  Every call on a
 * device shares that device's array, so calls that overlap on one device (on
 * different streams, or from threads without ordering) race; calls ordered
 * on one stream do not.  A call writes every partial it reads, so nothing
 * needs clearing between calls.
 */
int kvhot_paged_attention_noalloc(
    const void* q, const int64_t q_strides[3],
    const void* k_cache, const int64_t k_cache_strides[4],
    const void* v_cache, const int64_t v_cache_strides[4],
    void* out, const int64_t out_strides[3],
    float* lse, const int64_t lse_strides[2],
    const int32_t* block_table, int64_t bt_row_stride,
    const int32_t* q_lens, const int32_t* k_lens, const int32_t* q_starts,
    const int32_t* q_pos_offsets, int64_t num_rows, int64_t total_query,
    int64_t max_q_len, int64_t max_k_len, int64_t num_q_heads,
    int64_t num_kv_heads, int64_t head_dim, int64_t block_size,
    int64_t num_blocks, float scale, int attn_flags, int dtype,
    int64_t partition_tokens, const int32_t* schedule,
    int64_t num_decode_units, int64_t num_prefill_units,
    int64_t num_merge_units, int64_t num_prefix_units,
    int64_t schedule_workspace_bytes,
    void* stream);

#ifdef __cplusplus
}
#endif

#endif /* KVHOT_H */
