// KV append (reshape_and_cache), copy-on-write block copy and device-side
// slot-mapping construction.  All three are byte/integer work bound by HBM
// bandwidth (or by launch latency at decode sizes): every lane moves 16-byte
// vectors when the layout allows, and no arithmetic touches the payload, so
// results are bit-exact copies.
#include "kvhot_internal.h"

#include <cstring>

namespace kvhot {

static thread_local std::string g_last_error;

int set_error(int code, const std::string& msg) {
  g_last_error = msg;
  return code;
}

void clear_error() { g_last_error.clear(); }

// ------------------------------------------------------------------ append --

// A lane copies U W-sized units of (token, head) rows, K (kv = 0) or V
// (kv = 1): unit j of the lane is unit idx0 + j * blockDim.x of the call, so
// each of its U loads is coalesced across the block.  All U units and their
// tokens' slots are loaded before the first store (the units' addresses do
// not depend on the slots), so a lane has U loads in flight and its stores
// wait for one round trip.  Strides are in units of W.  Lane indices and
// slots are of type I: 32-bit (cheaper divisions) whenever the call's units
// and the pool's slots fit.
template <typename W, typename SlotT, typename I, int U>
__global__ void __launch_bounds__(256)
reshape_and_cache_kernel(const W* __restrict__ key, const W* __restrict__ value,
                         W* __restrict__ k_cache, W* __restrict__ v_cache,
                         const SlotT* __restrict__ slots, I per_kv, I num_heads,
                         I units_per_row, int64_t k_st, int64_t k_sh, int64_t v_st,
                         int64_t v_sh, int64_t kc_sb, int64_t kc_st, int64_t kc_sh,
                         int64_t vc_sb, int64_t vc_st, int64_t vc_sh,
                         int32_t block_size, int64_t num_slots) {
  const I idx0 = static_cast<I>(blockIdx.x) * static_cast<I>(blockDim.x) * U + static_cast<I>(threadIdx.x);
  W x[U];
  int64_t s[U], h[U];
  I u[U];
  bool kvs[U], live[U];
#pragma unroll
  for (int j = 0; j < U; ++j) {
    I idx = idx0 + static_cast<I>(j) * static_cast<I>(blockDim.x);
    live[j] = idx < 2 * per_kv;
    if (!live[j]) idx = 0;
    kvs[j] = idx >= per_kv;
    if (kvs[j]) idx -= per_kv;
    u[j] = idx % units_per_row;
    const I th = idx / units_per_row;
    h[j] = static_cast<int64_t>(th % num_heads);
    const int64_t t = static_cast<int64_t>(th / num_heads);
    x[j] = kvs[j] ? value[t * v_st + h[j] * v_sh + u[j]] : key[t * k_st + h[j] * k_sh + u[j]];
    s[j] = static_cast<int64_t>(slots[t]);
  }
#pragma unroll
  for (int j = 0; j < U; ++j) __asm__ volatile("" : "+v"(x[j]));  // keeps the loads ahead of the slot tests
#pragma unroll
  for (int j = 0; j < U; ++j) {
    if (!live[j] || s[j] < 0 || s[j] >= num_slots) continue;
    int64_t blk, off;
    if constexpr (sizeof(I) == 4) {  // the pool's slots fit 32 bits too
      const uint32_t b = static_cast<uint32_t>(s[j]) / static_cast<uint32_t>(block_size);
      blk = b;
      off = static_cast<uint32_t>(s[j]) - b * static_cast<uint32_t>(block_size);
    } else {
      blk = s[j] / block_size;
      off = s[j] - blk * block_size;
    }
    // Non-temporal stores: the pool's new rows are not read again by this
    // launch, and keeping them out of the caches' way lets the writes stream
    // (the 4,152-token append: 8.1 -> 6.4 us, 52% -> 66% of 8 TB/s).
    if (!kvs[j])
      __builtin_nontemporal_store(x[j], &k_cache[blk * kc_sb + off * kc_st + h[j] * kc_sh + u[j]]);
    else
      __builtin_nontemporal_store(x[j], &v_cache[blk * vc_sb + off * vc_st + h[j] * vc_sh + u[j]]);
  }
}

// Units per lane of an append: 4 once the call has a device-full of lanes
// or more (the 4,152-token chunked-prefill append moves 34 MB), else 1 (a
// decode step's append is launch-bound, and one unit per lane starts soonest).
constexpr int64_t kAppendMultiUnits = 256 * 2048;

template <typename W, typename SlotT, typename I, int U>
static void launch_append_u(const W* k, const W* v, W* kc, W* vc, const SlotT* sl, int64_t per_kv, int64_t H,
                            int64_t upr, const int64_t* ks, const int64_t* vs, const int64_t* kcs,
                            const int64_t* vcs, int64_t f, int64_t bs, int64_t nslots, hipStream_t stream) {
  const int64_t grid = (2 * per_kv + 256 * U - 1) / (256 * U);
  hipLaunchKernelGGL((reshape_and_cache_kernel<W, SlotT, I, U>), dim3(static_cast<uint32_t>(grid)), dim3(256), 0,
                     stream, k, v, kc, vc, sl, static_cast<I>(per_kv), static_cast<I>(H), static_cast<I>(upr),
                     ks[0] / f, ks[1] / f, vs[0] / f, vs[1] / f, kcs[0] / f, kcs[1] / f, kcs[2] / f, vcs[0] / f,
                     vcs[1] / f, vcs[2] / f, static_cast<int32_t>(bs), nslots);
}

template <typename W, typename SlotT>
static int launch_append(const void* key, const int64_t* ks, const void* value,
                         const int64_t* vs, void* kc, const int64_t* kcs,
                         void* vc, const int64_t* vcs, const void* slots,
                         int64_t T, int64_t H, int64_t D, int64_t bs,
                         int64_t nblocks, int64_t es, hipStream_t stream) {
  const int64_t f = static_cast<int64_t>(sizeof(W)) / es;  // elements per unit
  const int64_t upr = D / f;
  const int64_t per_kv = T * H * upr;
  const W* k = static_cast<const W*>(key);
  const W* v = static_cast<const W*>(value);
  const SlotT* sl = static_cast<const SlotT*>(slots);
  W* kcw = static_cast<W*>(kc);
  W* vcw = static_cast<W*>(vc);
  const bool multi = 2 * per_kv >= kAppendMultiUnits;
  if (2 * per_kv + 1024 < (int64_t{1} << 31) && nblocks * bs < (int64_t{1} << 31)) {
    if (multi)
      launch_append_u<W, SlotT, uint32_t, 4>(k, v, kcw, vcw, sl, per_kv, H, upr, ks, vs, kcs, vcs, f, bs, nblocks * bs,
                                             stream);
    else
      launch_append_u<W, SlotT, uint32_t, 1>(k, v, kcw, vcw, sl, per_kv, H, upr, ks, vs, kcs, vcs, f, bs, nblocks * bs,
                                             stream);
  } else {
    launch_append_u<W, SlotT, int64_t, 4>(k, v, kcw, vcw, sl, per_kv, H, upr, ks, vs, kcs, vcs, f, bs, nblocks * bs,
                                          stream);
  }
  return launch_status("reshape_and_cache");
}

// Largest copy unit (16, 8, 4, 2 or 1 bytes) that divides every row start.
static int64_t pick_unit(int64_t row_bytes, const uintptr_t* ptrs, int nptr,
                         const int64_t* strides_bytes, int nstr) {
  for (int64_t u : {16, 8, 4, 2, 1}) {
    bool ok = (row_bytes % u) == 0;
    for (int i = 0; ok && i < nptr; ++i) ok = (ptrs[i] % u) == 0;
    for (int i = 0; ok && i < nstr; ++i) ok = (strides_bytes[i] % u) == 0;
    if (ok) return u;
  }
  return 1;
}

}  // namespace kvhot

using namespace kvhot;

extern "C" int kvhot_version(void) { return 100; }

extern "C" const char* kvhot_last_error(void) { return g_last_error.c_str(); }

extern "C" int kvhot_reshape_and_cache(
    const void* key, const int64_t key_strides[3], const void* value,
    const int64_t value_strides[3], void* k_cache,
    const int64_t k_cache_strides[4], void* v_cache,
    const int64_t v_cache_strides[4], const void* slot_mapping,
    int slot_is_int64, int64_t num_tokens, int64_t num_kv_heads,
    int64_t head_dim, int64_t block_size, int64_t num_blocks, int dtype,
    void* stream) {
  clear_error();
  const int64_t es = dtype_size(dtype);
  if (es == 0) return set_error(KVHOT_EINVAL, "reshape_and_cache: bad dtype");
  if (num_tokens < 0 || num_kv_heads <= 0 || head_dim <= 0 || block_size <= 0 ||
      num_blocks < 0)
    return set_error(KVHOT_EINVAL, "reshape_and_cache: bad sizes");
  if (num_tokens == 0) return 0;
  if (!key || !value || !k_cache || !v_cache || !slot_mapping || !key_strides ||
      !value_strides || !k_cache_strides || !v_cache_strides)
    return set_error(KVHOT_EINVAL, "reshape_and_cache: null pointer");
  if (key_strides[2] != 1 || value_strides[2] != 1 || k_cache_strides[3] != 1 ||
      v_cache_strides[3] != 1)
    return set_error(KVHOT_EINVAL,
                     "reshape_and_cache: head_dim must be the innermost, unit-stride dim");
  const uintptr_t ptrs[4] = {reinterpret_cast<uintptr_t>(key),
                             reinterpret_cast<uintptr_t>(value),
                             reinterpret_cast<uintptr_t>(k_cache),
                             reinterpret_cast<uintptr_t>(v_cache)};
  const int64_t sb[10] = {key_strides[0] * es,     key_strides[1] * es,
                          value_strides[0] * es,   value_strides[1] * es,
                          k_cache_strides[0] * es, k_cache_strides[1] * es,
                          k_cache_strides[2] * es, v_cache_strides[0] * es,
                          v_cache_strides[1] * es, v_cache_strides[2] * es};
  const int64_t unit = pick_unit(head_dim * es, ptrs, 4, sb, 10);
  hipStream_t s = static_cast<hipStream_t>(stream);
#define KVHOT_APPEND(W)                                                          \
  (slot_is_int64                                                                 \
       ? launch_append<W, int64_t>(key, key_strides, value, value_strides,       \
                                   k_cache, k_cache_strides, v_cache,            \
                                   v_cache_strides, slot_mapping, num_tokens,    \
                                   num_kv_heads, head_dim, block_size,           \
                                   num_blocks, es, s)                            \
       : launch_append<W, int32_t>(key, key_strides, value, value_strides,       \
                                   k_cache, k_cache_strides, v_cache,            \
                                   v_cache_strides, slot_mapping, num_tokens,    \
                                   num_kv_heads, head_dim, block_size,           \
                                   num_blocks, es, s))
  if (unit < es) return set_error(KVHOT_EINVAL, "reshape_and_cache: misaligned tensors");
  switch (unit) {
    case 16: return KVHOT_APPEND(u32x4);
    case 8: return KVHOT_APPEND(u32x2);
    case 4: return KVHOT_APPEND(uint32_t);
    default: return KVHOT_APPEND(uint16_t);
  }
#undef KVHOT_APPEND
}

// ------------------------------------------------------------- block copy --

namespace kvhot {

// Work-group (pair i, layer*2 + kv) copies one block payload: each lane
// loads 8 units (a whole 32 KiB block at 16-byte units) before storing them,
// with nontemporal loads and stores (the data is touched once).  On MI355X
// this copy runs at 96% of the rate of a contiguous device-to-device copy of
// the same volume (210 against 203 us for 512 MiB each way).
template <typename W>
__global__ void __launch_bounds__(256)
copy_blocks_kernel(char* __restrict__ base, int64_t layer_stride,
                   int64_t kv_stride, int64_t block_stride, int64_t block_bytes,
                   int64_t num_blocks, const int64_t* __restrict__ src,
                   const int64_t* __restrict__ dst) {
  const int64_t i = blockIdx.x;
  const int64_t lk = blockIdx.y;
  const int64_t s = src[i], d = dst[i];
  if (s < 0 || s >= num_blocks || d < 0 || d >= num_blocks) return;
  const int64_t plane = (lk >> 1) * layer_stride + (lk & 1) * kv_stride;
  const W* __restrict__ from = reinterpret_cast<const W*>(base + plane + s * block_stride);
  W* __restrict__ to = reinterpret_cast<W*>(base + plane + d * block_stride);
  const int64_t n = block_bytes / static_cast<int64_t>(sizeof(W));
  constexpr int kUnroll = 8;
  int64_t j = threadIdx.x;
  for (; j + (kUnroll - 1) * 256 < n; j += kUnroll * 256) {
    W r[kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) r[u] = __builtin_nontemporal_load(from + j + u * 256);
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) __builtin_nontemporal_store(r[u], to + j + u * 256);
  }
  for (; j < n; j += 256) __builtin_nontemporal_store(__builtin_nontemporal_load(from + j), to + j);
}

}  // namespace kvhot

extern "C" int kvhot_copy_blocks(void* kv_cache, int64_t num_layers,
                                 int64_t layer_stride_bytes,
                                 int64_t kv_stride_bytes,
                                 int64_t block_stride_bytes, int64_t block_bytes,
                                 int64_t num_blocks, const int64_t* src_block_ids,
                                 const int64_t* dst_block_ids, int64_t num_pairs,
                                 void* stream) {
  clear_error();
  if (num_pairs < 0 || num_layers <= 0 || block_bytes < 0 || num_blocks < 0)
    return set_error(KVHOT_EINVAL, "copy_blocks: bad sizes");
  if (num_pairs == 0 || block_bytes == 0) return 0;
  if (!kv_cache || !src_block_ids || !dst_block_ids)
    return set_error(KVHOT_EINVAL, "copy_blocks: null pointer");
  if (num_layers > 32768 || num_pairs > 0x7fffffff)
    return set_error(KVHOT_EINVAL, "copy_blocks: too many layers or pairs");
  const uintptr_t ptrs[1] = {reinterpret_cast<uintptr_t>(kv_cache)};
  const int64_t strides[3] = {layer_stride_bytes, kv_stride_bytes, block_stride_bytes};
  const int64_t unit = pick_unit(block_bytes, ptrs, 1, strides, 3);
  hipStream_t s = static_cast<hipStream_t>(stream);
  dim3 grid(static_cast<uint32_t>(num_pairs), static_cast<uint32_t>(2 * num_layers));
  char* base = static_cast<char*>(kv_cache);
#define KVHOT_COPY(W)                                                              \
  hipLaunchKernelGGL(copy_blocks_kernel<W>, grid, dim3(256), 0, s, base,           \
                     layer_stride_bytes, kv_stride_bytes, block_stride_bytes,      \
                     block_bytes, num_blocks, src_block_ids, dst_block_ids)
  switch (unit) {
    case 16: KVHOT_COPY(u32x4); break;
    case 8: KVHOT_COPY(u32x2); break;
    case 4: KVHOT_COPY(uint32_t); break;
    case 2: KVHOT_COPY(uint16_t); break;
    default: KVHOT_COPY(uint8_t); break;
  }
#undef KVHOT_COPY
  return launch_status("copy_blocks");
}

// ----------------------------------------------------------- slot mapping --

namespace kvhot {

__global__ void __launch_bounds__(256)
slot_mapping_kernel(const int32_t* __restrict__ bt, int64_t bt_stride,
                    const int32_t* __restrict__ q_lens,
                    const int32_t* __restrict__ q_starts,
                    const int32_t* __restrict__ q_offs, int32_t block_size,
                    int64_t total, int64_t* __restrict__ slots,
                    int64_t* __restrict__ positions) {
  const int64_t r = blockIdx.y;
  const int32_t i = blockIdx.x * 256 + threadIdx.x;
  if (i >= q_lens[r]) return;
  const int64_t t = static_cast<int64_t>(q_starts[r]) + i;
  if (t < 0 || t >= total) return;
  const int64_t pos = static_cast<int64_t>(q_offs[r]) + i;
  const int64_t lb = pos / block_size;
  int64_t slot = -1;
  if (pos >= 0 && lb < bt_stride)
    slot = static_cast<int64_t>(bt[r * bt_stride + lb]) * block_size + (pos - lb * block_size);
  if (slots) slots[t] = slot;
  if (positions) positions[t] = pos;
}

}  // namespace kvhot

extern "C" int kvhot_build_slot_mapping(const int32_t* block_table,
                                        int64_t bt_row_stride,
                                        const int32_t* q_lens,
                                        const int32_t* q_starts,
                                        const int32_t* q_pos_offsets,
                                        int64_t num_rows, int64_t total_query,
                                        int64_t max_q_len, int64_t block_size,
                                        int64_t* slot_mapping,
                                        int64_t* positions, void* stream) {
  clear_error();
  if (num_rows < 0 || total_query < 0 || max_q_len < 0 || block_size <= 0 || bt_row_stride < 0)
    return set_error(KVHOT_EINVAL, "build_slot_mapping: bad sizes");
  if (num_rows == 0 || max_q_len == 0 || total_query == 0) return 0;
  if (!q_lens || !q_starts || !q_pos_offsets || (!slot_mapping && !positions) ||
      (bt_row_stride > 0 && !block_table))
    return set_error(KVHOT_EINVAL, "build_slot_mapping: null pointer");
  if (num_rows > 65535)
    return set_error(KVHOT_EUNSUPPORTED, "build_slot_mapping: more than 65535 rows");
  dim3 grid(static_cast<uint32_t>((max_q_len + 255) / 256), static_cast<uint32_t>(num_rows));
  hipLaunchKernelGGL(slot_mapping_kernel, grid, dim3(256), 0,
                     static_cast<hipStream_t>(stream), block_table, bt_row_stride,
                     q_lens, q_starts, q_pos_offsets, static_cast<int32_t>(block_size),
                     total_query, slot_mapping, positions);
  return launch_status("build_slot_mapping");
}
