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
 * block_bytes bytes must be contiguous.  Destinations must be unique and must
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
 * Every workspace starts with this many bytes of counters used by scheduled
 * decode calls (rows whose keys were cut across work-groups).  They must be
 * zero before a workspace's first call, and every call leaves them zero, so
 * allocate workspaces zero-filled.  Split-K partials follow them.
 */
#define KVHOT_WORKSPACE_COUNTER_BYTES 16384

/*
 * Workspace bytes kvhot_paged_attention needs for these sizes when it is
 * called WITHOUT a schedule (0 if it needs none): the counter bytes above,
 * then split-K partition results of decode rows, fully rewritten by each call
 * before they are read.  A workspace may be reused by calls of any shape that
 * fits.  Calls sharing a workspace must be ordered on one stream.  Returns a
 * negative KVHOT_E* code for invalid sizes.  (With a schedule, the size comes
 * from kvhot_paged_attention_schedule.)
 */
int64_t kvhot_paged_attention_workspace_bytes(
    int64_t num_rows, int64_t total_query, int64_t max_q_len,
    int64_t max_k_len, int64_t num_q_heads, int64_t num_kv_heads,
    int64_t head_dim, int64_t block_size, int64_t partition_tokens, int dtype);

/* Entries of the description kvhot_paged_attention_schedule writes beside a
 * launch list; kvhot_paged_attention takes it back unchanged. */
enum {
  KVHOT_SCHED_UNITS = 0,           /* units in the list (8 int32 each) */
  KVHOT_SCHED_PREFILL_UNITS = 1,   /* prefill work-groups: units [0, n) */
  KVHOT_SCHED_DECODE_UNITS = 2,    /* the decode section: the n units after them */
  KVHOT_SCHED_DECODE_GROUPS = 3,   /* work-groups of the decode launch */
  KVHOT_SCHED_WORKSPACE_BYTES = 4, /* workspace the attention call needs (0: none) */
  KVHOT_SCHED_CUT_ROWS = 5,        /* decode rows whose keys are cut across work-groups */
  KVHOT_SCHED_DECODE_LDS_BYTES = 6,/* LDS of a decode work-group */
  KVHOT_SCHED_DECODE_BANKS = 7,    /* its per-piece accumulators (| 256: one slot per wave) */
  KVHOT_SCHED_INFO_LEN = 8
};

/*
 * Launch list ("schedule") for kvhot_paged_attention, built on the host from
 * HOST copies of q_lens, k_lens, q_starts and q_pos_offsets, with the head
 * counts, head_dim, block_size, is_causal and dtype the attention call will
 * get.  Units of 8 int32: the prefill work-groups (row, kv head, query block;
 * longest key range first), then the decode section.  Decode rows run as
 * head groups: the 16-token slices of all decode rows, rows in order, are cut
 * into equal ranges, one per group of num_kv_heads work-groups, and work-group
 * q * num_kv_heads + i streams kv head (i + q) % num_kv_heads of range q, so a
 * group's work-groups read every block of the range at about the same time.  A row cut between
 * two ranges is combined inside the launch by whichever of its pieces
 * finishes last (through the workspace).  partition_tokens > 0 (a multiple of
 * 32 up to 2^20) makes every such cut fall on a multiple of that many keys
 * into the row; 0 lets the planner cut anywhere (at least 64 keys from
 * either end of a piece).  info (KVHOT_SCHED_INFO_LEN entries) receives the
 * unit counts, the decode launch's work-groups and the workspace the
 * attention call needs.  Returns the total unit count (units are written when
 * `units` is non-NULL and capacity_units suffices) or a negative KVHOT_E*
 * code; 0 units means no schedule (shapes the MFMA kernels do not take, or
 * counts beyond the list's fields): call kvhot_paged_attention without one.
 * A schedule depends only on the step's lengths, so one upload serves every
 * layer of an engine step.  Without a schedule the attention launch covers
 * the padded grid of (row, partition, head group), and work-groups without
 * work still cost a launch slot each.
 */
int64_t kvhot_paged_attention_schedule(
    const int32_t* q_lens, const int32_t* k_lens, const int32_t* q_starts,
    const int32_t* q_pos_offsets, int64_t num_rows, int64_t num_q_heads,
    int64_t num_kv_heads, int64_t head_dim, int64_t block_size,
    int64_t partition_tokens, int is_causal, int dtype, int32_t* units,
    int64_t capacity_units, int64_t info[KVHOT_SCHED_INFO_LEN]);

/*
 * Paged attention forward over a ragged batch of rows (prefill chunks and
 * decode rows mixed), one call per layer.  For row r with n_q = q_lens[r],
 * n_k = k_lens[r], off = q_pos_offsets[r], and each query i < n_q (global
 * token t = q_starts[r] + i) and query head h:
 *   keys j in [0, n_k) are read through block_table[r, j / block_size];
 *   when is_causal, key j is visible iff j <= off + i;
 *   out[t, h, :] = softmax_j(scale * q[t,h,:] . k_j) @ v_j   (fp32 accumulate)
 *   lse[t, h]    = natural-log logsumexp_j(scale * q[t,h,:] . k_j)
 * A query with no visible key gets out = 0 and lse = -inf.
 * Rows with n_q == 1 run the flash-decoding kernel, rows with n_q >= 2 the
 * chunked-prefill kernel.  max_q_len / max_k_len must bound q_lens / k_lens
 * (they size the grid; no device->host sync is made).
 * schedule: device copy of the units from kvhot_paged_attention_schedule for
 * exactly these lengths and sizes, schedule_info its description (host
 * memory), and a workspace of at least its KVHOT_SCHED_WORKSPACE_BYTES (a
 * shorter one fails with KVHOT_EWORKSPACE before any launch); or NULL, and
 * then partition_tokens (keys per decode partition; 0 picks a size,
 * otherwise a multiple of 32 up to 2^20) and
 * kvhot_paged_attention_workspace_bytes apply (plus a merge launch for rows
 * of several partitions).  With a schedule, the waves of a work-group claim
 * slices at run time, so the summation order, and with it the last bits of
 * out and lse, can differ from call to call.  lse may be NULL.  out has the
 * dtype of q, k_cache and v_cache; lse is fp32.  Replaces
 * paged_flash_attention + paged_flash_fwd_kernel
 * (serving_engine/paged_attention_kernel.py:16-160).
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
    int64_t num_blocks, float scale, int is_causal, int dtype,
    int64_t partition_tokens, const int32_t* schedule,
    const int64_t* schedule_info, void* workspace, int64_t workspace_bytes,
    void* stream);

#ifdef __cplusplus
}
#endif

#endif /* KVHOT_H */
