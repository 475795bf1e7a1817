// Paged attention over a ragged batch of prefill chunks and decode rows.
//
// Kernel map:
//  * WaveAttn<T, D, NM>: one wavefront attends 16*NM "m-rows" -- (query, head)
//    pairs of one GQA group, so every K/V byte it loads serves all
//    G = Hq/Hkv query heads of that kv head -- over a key range.  Keys are
//    walked in 16-token block slices.  Scores are formed transposed,
//    S^T = K . Q^T, with v_mfma_f32_16x16x32: K rows (token-major, head_dim
//    contiguous) are already the MFMA A-operand layout, so K goes HBM -> VGPR
//    with no LDS round trip.  The accumulator layout of S^T (lane = m-row,
//    4 tokens per lane) is exactly the B-operand layout P^T needs for
//    O^T = V^T . P^T on v_mfma_f32_16x16x16, so probabilities never leave
//    registers.  V^T is formed in registers with v_perm_b32 from 16-byte row
//    loads.  Softmax statistics live in the lane that owns the m-row, so
//    rescaling O needs no cross-lane traffic.
//  * attn_decode_kernel<T, D, W>: rows with q_len == 1.  The host planner
//    cuts every (row, kv head) into a segment of 16-token slices and packs
//    the segments into work-groups of W = 8 waves, longest first, splitting a
//    segment only where a work-group's load demands it.  Inside a work-group
//    each wave claims slices one at a time from LDS counters and steals from
//    the ranges with the most left, so waves that stream slower than their
//    neighbours do not set the end time.  Per-(wave, segment) (LSE, O) pieces
//    are merged through LDS; a segment split across work-groups stores
//    partials to HBM that attn_merge_kernel combines in a second launch.  K/V
//    loads are non-temporal: every byte of a call is read by one wave once.
//  * attn_prefill_kernel<T, D, NM>: rows with q_len >= 2, and the key splits
//    of a prefix shared by many decode rows (one unit serves all those rows'
//    queries; the decode segments fold its partials in).  A work-group of 4
//    waves (two per CU; 8 waves at head_dim 256) per (row, kv head, query
//    block) copies 32-key K/V tiles from the paged cache into LDS through a
//    four-slot ring and shares them; both products use the 16x16x32 MFMA
//    (P^T keeps S^T's key order as the K dimension), and at head_dim <= 128
//    the QK of the next tile runs beside the softmax of this one.  Causal
//    mask from q_pos_offset; tiles past the work-group's last query are never
//    loaded.
//  * attn_generic_kernel<T>: VALU kernel for fp32 (exact fp32 arithmetic) and
//    for shapes the MFMA kernels do not cover.
#include "kvhot_internal.h"

#include <algorithm>
#include <cfloat>
#include <climits>
#include <functional>
#include <mutex>
#include <type_traits>
#include <vector>

namespace kvhot {

struct AttnArgs {
  const void* q;
  int64_t q_st, q_sh;
  const void* k;
  int64_t k_sb, k_st, k_sh;
  const void* v;
  int64_t v_sb, v_st, v_sh;
  void* o;
  int64_t o_st, o_sh;
  float* lse;
  int64_t l_st, l_sh;
  const int32_t* bt;
  int64_t bt_stride;
  const int32_t* q_lens;
  const int32_t* k_lens;
  const int32_t* q_starts;
  const int32_t* q_offs;
  // Split-K partials, P = num_partials of them: ws_o [P][G][D] normalised
  // output, ws_lse [P][G] log2-domain LSE of a (row, kv head, part) piece.
  float* ws_lse;
  float* ws_o;
  int64_t num_partials;
  int64_t num_blocks;
  int32_t Hq, Hkv, G, bs;
  int32_t part_tokens, max_parts;
  float scale_log2;
  int32_t causal;
  int32_t D;        // head_dim (generic kernel)
  int64_t total_q;  // rows of q / out / lse: outputs are only written below it
  // Launch list from kvhot_paged_attention_schedule (decode: two int4 per wave,
  // prefill: two int4 per work-group), or null: then the grid enumerates every
  // (row, partition, head group) and work-groups without work exit.
  const int4* sched;
  const int4* merge_units;  // schedule: two int4 per split decode segment
  int32_t dec_slots;  // LDS (LSE, O) slots of a decode work-group, >= its ranges
  int32_t dec_ranges; // range descriptors per decode work-group (its waves, or 4x them)
  // KVHOT_DETERMINISTIC: every decode wave walks exactly its planned range,
  // in order (no claiming from other waves), so each partial sum, and with it
  // out and lse, is the same bits on every call.
  int32_t fixed;
  // KVHOT_VERIFY_BLOCKS: decode waves check a launch list's first block.
  int32_t verify;
};

__device__ inline float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

typedef __attribute__((address_space(3))) void* lds_ptr_t;

// 16 bytes per lane from r at byte offset off into LDS at dst + 16 * lane
// (buffer_load_dwordx4 ... lds; offsets past the descriptor's range give
// zeros).  A plain device function: the builtin needs a device target
// feature, and inside a kernel template the host pass would drop the kernel.
__device__ inline void dma16(__amdgpu_buffer_rsrc_t r, void* dst, int off) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_ptr_t)dst, 16, off, 0, 0, 0);
}

// The words of the buffer descriptor block_rsrc builds: base, stride 0,
// `bytes` records, the same flags.
typedef uint32_t rsrc_words_t __attribute__((ext_vector_type(4)));
__device__ inline rsrc_words_t rsrc_words(const void* base, int bytes) {
  const uint64_t b = reinterpret_cast<uint64_t>(base);
  return rsrc_words_t{static_cast<uint32_t>(b), static_cast<uint32_t>(b >> 32) & 0xffffu,
                      static_cast<uint32_t>(bytes), 0x00020000u};
}

// dma16 as inline assembly.  The compiler's wait insertion treats every LDS
// read without alias-scope metadata (the ds_read_tr builtins have none) as
// possibly reading what an LDS DMA in flight writes, and drains every DMA
// before it; issued this way the DMA is invisible to it.  A caller orders its
// DMAs itself: the issuing wave waits with s_waitcnt vmcnt, then a
// work-group barrier, before any wave reads what they wrote.  (The
// compiler's own vmcnt waits stay correct: DMAs it does not know of only make
// them wait longer.)  It sets M0, which the compiler treats as reserved and
// does not track across asm: a kernel that uses it may hold nothing of its
// own in M0 (the prefill kernel uses M0 for these DMAs only).
__device__ inline void dma16_asm(rsrc_words_t r, void* dst, int off) {
  const uint32_t lds = static_cast<uint32_t>(reinterpret_cast<uintptr_t>((lds_ptr_t)dst));
  asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dwordx4 %1, %2, 0 offen lds" ::"s"(lds), "v"(off), "s"(r)
               : "memory");
}

// A pointer every lane holds, broadcast from lane 0 so the compiler keeps it
// (and descriptors built from it) in scalar registers.
template <typename T>
__device__ inline const T* uniform_ptr(const T* p) {
  const uint64_t v = reinterpret_cast<uint64_t>(p);
  const uint32_t lo = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(v));
  const uint32_t hi = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(v >> 32));
  return reinterpret_cast<const T*>((static_cast<uint64_t>(hi) << 32) | lo);
}

// Buffer resource over [base, base + bytes): loads through it take a 32-bit
// lane offset (no 64-bit per-lane address registers), and the hardware returns
// zeros for any offset past `bytes`.  Word 3 = 0x00020000: raw dword access
// for CDNA.
__device__ inline __amdgpu_buffer_rsrc_t block_rsrc(const void* base, int bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, bytes, 0x00020000);
}

// Cache policy of the decode kernel's K/V loads: non-temporal (the nt bit).
// Each K/V byte of a decode launch is read by one wave (a slice serves every
// query head of its kv head), and rows whose tables share a long prefix have
// it attended once by prefix units, so the loads leave no reuse to keep.
// (Rows that share blocks outside a prefix unit, e.g. a few forks, each read
// them from HBM.)
#ifndef KVHOT_KV_LOAD_POLICY
#define KVHOT_KV_LOAD_POLICY 2
#endif
constexpr int kKvLoadPolicy = KVHOT_KV_LOAD_POLICY;

// Loads N dwords (N in {2, 4, 8}) at byte offset off (+ uniform soff) of r.
template <int N>
__device__ inline void buffer_dwords(__amdgpu_buffer_rsrc_t r, int off, int soff, uint32_t* out) {
  if constexpr (N == 2) {
    const u32x2 v = __builtin_bit_cast(u32x2, __builtin_amdgcn_raw_buffer_load_b64(r, off, soff, kKvLoadPolicy));
    out[0] = v.x; out[1] = v.y;
  } else {
#pragma unroll
    for (int c = 0; c < N / 4; ++c) {
      const u32x4 v = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, off + 16 * c, soff, kKvLoadPolicy));
      out[4 * c + 0] = v.x; out[4 * c + 1] = v.y;
      out[4 * c + 2] = v.z; out[4 * c + 3] = v.w;
    }
  }
}

// Loads N dwords (N in {2, 4, 8}) from a 16-bit element pointer.
template <int N>
__device__ inline void load_dwords(const uint16_t* p, uint32_t* out) {
  if constexpr (N == 2) {
    u32x2 v = *reinterpret_cast<const u32x2*>(p);
    out[0] = v.x; out[1] = v.y;
  } else {
#pragma unroll
    for (int c = 0; c < N / 4; ++c) {
      u32x4 v = *reinterpret_cast<const u32x4*>(p + 8 * c);
      out[4 * c + 0] = v.x; out[4 * c + 1] = v.y;
      out[4 * c + 2] = v.z; out[4 * c + 3] = v.w;
    }
  }
}

template <int D>
struct KVSlice {
  static constexpr int NC = D / 32;   // 32-wide head_dim chunks of Q.K
  static constexpr int VW = D / 32;   // dwords per V row per lane (D/16 elements)
  u32x4 k[NC];                        // token n, dims 8*(4c+g)..+8
  uint32_t v[4][VW];                  // token 4g+j, dims (D/16)*n..+D/16
};

// Key partition a decode row is cut into, shared by the split and merge
// kernels: visible keys, clamped to what the grid and workspace were sized for.
__device__ inline int decode_visible_keys(const AttnArgs& a, int row) {
  const int klen = a.k_lens[row];
  int kend = a.causal ? min(klen, a.q_offs[row] + 1) : klen;
  kend = max(kend, 0);
  return static_cast<int>(min(static_cast<int64_t>(kend),
                              static_cast<int64_t>(a.max_parts) * a.part_tokens));
}

// Prefill tiles move their softmax reference only when a score exceeds it by
// more than this many log2 units, so P <= 2^15: finite as an fp16 operand
// (largest 65504), and with up to 2^31 keys and |V| < 2^70 the fp32 sums stay
// finite.
constexpr float kLazyRescale = 15.f;


// One wavefront's attention state and key loop.
template <class TT, int D, int NM>
struct WaveAttn {
  static constexpr int NC = D / 32;
  static constexpr int EPL = D / 16;  // head_dim values per lane per V row; PV MFMAs per tile
  static constexpr int VW = EPL / 2;
  using st = uint16_t;

  int n, g;
  // m-row s*16 + n of this lane: causal limit (key positions up to it are visible) and validity
  int kvh_;                  // the work's kv head (uniform)
  int qbase_, lg_g_;         // causal limit of query 0 (INT_MAX: none), log2 G (uniform)
  int qpos[NM];
  bool mval[NM];
  u32x4 qf[NM][NC];  // Q as the B operand of S^T = K . Q^T
  float m[NM], l[NM];
  float thr[NM];     // prefill tiles: raw score above which m[s] has to move
  f32x4 o[NM][EPL];  // O^T: lane (n, g) holds head_dim EPL*(4g+j)+e of m-row n

  // m-rows are the (query, head) pairs q0 + i / G, kvh * G + i % G of a row
  // whose first query is global token qs; nq queries are valid.
  __device__ void setup(const AttnArgs& a, int lane, int kvh, int64_t qs, int q0, int nq,
                        int off) {
    n = lane & 15;
    g = lane >> 4;
    kvh_ = kvh;
    const int G = a.G;
    qbase_ = a.causal ? off + q0 : INT_MAX;
    lg_g_ = __builtin_ctz(static_cast<unsigned>(G));
#pragma unroll
    for (int s = 0; s < NM; ++s) {
      const int i = 16 * s + n;
      const int mq = i / G, mh = kvh * G + (i % G);
      mval[s] = mq < nq && qs + q0 + mq < a.total_q;
      qpos[s] = mval[s] ? (a.causal ? off + q0 + mq : INT_MAX) : -1;
#pragma unroll
      for (int c = 0; c < NC; ++c) qf[s][c] = u32x4{0, 0, 0, 0};
      if (mval[s]) {
        const st* qp = static_cast<const st*>(a.q) + (qs + q0 + mq) * a.q_st +
                       static_cast<int64_t>(mh) * a.q_sh;
#pragma unroll
        for (int c = 0; c < NC; ++c)
          qf[s][c] = *reinterpret_cast<const u32x4*>(qp + 8 * (4 * c + g));
      }
      m[s] = -INFINITY;
      l[s] = 0.f;
#pragma unroll
      for (int e = 0; e < EPL; ++e) o[s][e] = f32x4{0.f, 0.f, 0.f, 0.f};
    }
  }

  // Query (within the block), query head and causal limit of m-row s of
  // this lane, recomputed where needed rather than held in registers through
  // the loop (G a power of two).
  __device__ int qlimit(int s) const {
    return mval[s] ? (qbase_ == INT_MAX ? INT_MAX : qbase_ + ((16 * s + n) >> lg_g_)) : -1;
  }
  __device__ int row_query(const AttnArgs& a, int s) const { return (16 * s + n) / a.G; }
  __device__ int row_head(const AttnArgs& a, int s) const { return kvh_ * a.G + (16 * s + n) % a.G; }

  // Issues the loads of one 16-token slice of kv head kvh: tokens bo..bo+15
  // of physical block id.
  // With live false the descriptors cover no bytes (zeros, no memory read).
  __device__ void load_slice(const AttnArgs& a, int kvh, int64_t id, int bo, KVSlice<D>& T,
                             bool live = true) const {
    // Per-lane byte offsets inside the slice; one descriptor per block, over
    // this kv head's rows and bounded by the block stride.
    const int k_lane = 2 * (n * static_cast<int>(a.k_st) + 8 * g);
    const st* kb = static_cast<const st*>(a.k) + static_cast<int64_t>(kvh) * a.k_sh + id * a.k_sb;
    const st* vb = static_cast<const st*>(a.v) + static_cast<int64_t>(kvh) * a.v_sh + id * a.v_sb;
    const __amdgpu_buffer_rsrc_t kr = block_rsrc(kb, live ? static_cast<int>(2 * a.k_sb) : 0);
    const __amdgpu_buffer_rsrc_t vr = block_rsrc(vb, live ? static_cast<int>(2 * a.v_sb) : 0);
    const int ks = 2 * bo * static_cast<int>(a.k_st);
    const int vs = 2 * bo * static_cast<int>(a.v_st);
#pragma unroll
    for (int c = 0; c < NC; ++c)
      T.k[c] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(kr, k_lane + 64 * c, ks, kKvLoadPolicy));
#pragma unroll
    for (int j = 0; j < 4; ++j)
      buffer_dwords<VW>(vr, 2 * ((4 * g + j) * static_cast<int>(a.v_st) + EPL * n), vs, T.v[j]);
  }

  // The loads of load_slice from the slice's block bases kb, vb (uniform).
  // With live false the descriptors cover no bytes: every lane reads zeros
  // and no memory is touched, but the loads still count in vmcnt.
  __device__ void load_slice_from(const AttnArgs& a, const st* kb, const st* vb, int bo, KVSlice<D>& T,
                                  bool live = true) const {
    const int k_lane = 2 * (n * static_cast<int>(a.k_st) + 8 * g);
    const __amdgpu_buffer_rsrc_t kr = block_rsrc(kb, live ? static_cast<int>(2 * a.k_sb) : 0);
    const __amdgpu_buffer_rsrc_t vr = block_rsrc(vb, live ? static_cast<int>(2 * a.v_sb) : 0);
    const int ks = 2 * bo * static_cast<int>(a.k_st);
    const int vs = 2 * bo * static_cast<int>(a.v_st);
#pragma unroll
    for (int c = 0; c < NC; ++c)
      T.k[c] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(kr, k_lane + 64 * c, ks, kKvLoadPolicy));
#pragma unroll
    for (int j = 0; j < 4; ++j)
      buffer_dwords<VW>(vr, 2 * ((4 * g + j) * static_cast<int>(a.v_st) + EPL * n), vs, T.v[j]);
  }

  // Folds the slice of keys ts..ts+15 into the online softmax.  Keys at or
  // past kstop, and keys past an m-row's causal limit, are masked; qpos_min is
  // the smallest causal limit of the valid m-rows (keys up to it are visible
  // to all of them).
  __device__ void compute_slice(const AttnArgs& a, int ts, int kstop, int qpos_min, KVSlice<D>& T) {
    // S^T: lane (n, g) gets tokens ts + 4g + j of m-row n.
    f32x4 sc[NM];
#pragma unroll
    for (int s = 0; s < NM; ++s) {
      f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int c = 0; c < NC; ++c) acc = TT::mfma(T.k[c], qf[s][c], acc);
      sc[s] = acc;
    }
    const bool tail = ts + 16 > kstop;
    const bool full = !tail && (ts + 15 <= qpos_min);
#pragma unroll
    for (int s = 0; s < NM; ++s)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        float x = sc[s][j] * a.scale_log2;
        if (!full) {
          const int tk = ts + 4 * g + j;
          x = (tk < kstop && tk <= qpos[s]) ? x : -INFINITY;
        }
        sc[s][j] = x;
      }
    if (tail) {
      // Keys past the end may hold any bit pattern; zero them so 0 * V stays 0.
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const bool ok = ts + 4 * g + j < kstop;
#pragma unroll
        for (int w = 0; w < VW; ++w) T.v[j][w] = ok ? T.v[j][w] : 0u;
      }
    }
    // Online softmax (base 2); P^T packed as the B operand of O^T += V^T . P^T.
    u32x2 pb[NM];
#pragma unroll
    for (int s = 0; s < NM; ++s) {
      float mx = fmaxf(fmaxf(sc[s][0], sc[s][1]), fmaxf(sc[s][2], sc[s][3]));
      mx = fmaxf(mx, __shfl_xor(mx, 16, kWave));
      mx = fmaxf(mx, __shfl_xor(mx, 32, kWave));
      const float mnew = fmaxf(m[s], mx);
      const float muse = (mnew == -INFINITY) ? 0.f : mnew;
      const float corr = fast_exp2(m[s] - muse);
      float pr[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) pr[j] = fast_exp2(sc[s][j] - muse);
      l[s] = l[s] * corr + ((pr[0] + pr[1]) + (pr[2] + pr[3]));
      m[s] = mnew;
      pb[s] = u32x2{TT::pack2(pr[0], pr[1]), TT::pack2(pr[2], pr[3])};
#pragma unroll
      for (int e = 0; e < EPL; ++e) o[s][e] *= corr;
    }
    // V^T A operand for head_dim values EPL*n + e, then O^T += V^T . P^T.
#pragma unroll
    for (int e = 0; e < EPL; ++e) {
      const int w = e >> 1;
      const uint32_t sel = (e & 1) ? 0x07060302u : 0x05040100u;
      const u32x2 vt = {__builtin_amdgcn_perm(T.v[1][w], T.v[0][w], sel),
                        __builtin_amdgcn_perm(T.v[3][w], T.v[2][w], sel)};
#pragma unroll
      for (int s = 0; s < NM; ++s) o[s][e] = TT::mfma16(vt, pb[s], o[s][e]);
    }
  }

  // ---- 32-key LDS tiles (PreTile layout, rows of Tile::RB bytes) ----
  // Both products use v_mfma_f32_16x16x32.  The 32 keys are the K dimension
  // of O^T += V^T . P^T in the order lane group g holds them in S^T -- keys
  // 4g..4g+3 of the first 16, then 4g..4g+3 of the second -- so P^T is the B
  // operand as it stands; V^T is gathered in that same key order.
  //
  // m[s] is a reference, not the exact running max: P = 2^(x - m) with x the
  // score in log2 units, and m only moves when some score exceeds it by more
  // than kLazyRescale, so P stays below 2^kLazyRescale.  While no lane sees
  // such a score (the usual case once a row's first keys are in) a tile needs
  // no cross-lane reduction and no rescale of O.  m starts at -FLT_MAX, so
  // masked scores (-inf) give P = 0 and the first visible score moves it.
  // sl = scale * log2(e) > 0 (a negative scale is folded into Q).

  // Raw S^T of a tile in two parts, so that the reads can be issued well
  // ahead of the products: the K operands (K row 16h + n, logical chunk
  // 4c + g), then lane (n, g) gets keys 4g+j (sc[s][0]) and 16+4g+j
  // (sc[s][1]) of m-row n.
  template <class Tile>
  __device__ void k_operands(const char* kt, int h, u32x4 (&kop)[NC]) const {
#pragma unroll
    for (int c = 0; c < NC; ++c) kop[c] = *reinterpret_cast<const u32x4*>(kt + Tile::offset(16 * h + n, 4 * c + g));
  }
  __device__ void qk_ops(const u32x4 (&kop)[NC], int h, f32x4 (&sc)[NM][2]) const {
#pragma unroll
    for (int s = 0; s < NM; ++s) sc[s][h] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int c = 0; c < NC; ++c)
#pragma unroll
      for (int s = 0; s < NM; ++s) sc[s][h] = TT::mfma(kop[c], qf[s][c], sc[s][h]);
  }

  // Local (per-lane) max of each m-row's raw scores, and whether any exceeds
  // its threshold thr[s] = (m[s] + kLazyRescale) / sl.  IEEE maximum (NaN in,
  // NaN out) needs no canonicalising of the MFMA results and pairs into
  // v_maximum3_f32: four instructions and one compare per m-row.  A NaN
  // score leaves m alone and makes the row's P, and so its output, NaN.
  __device__ static float max3(float x, float y, float z) {
    return __builtin_elementwise_maximum(__builtin_elementwise_maximum(x, y), z);
  }
  __device__ bool lazy_check(const f32x4 (&sc)[NM][2], float (&mloc)[NM]) const {
    bool need = false;
#pragma unroll
    for (int s = 0; s < NM; ++s) {
      const f32x4 x = sc[s][0], y = sc[s][1];
      mloc[s] = __builtin_elementwise_maximum(max3(x[3], y[0], y[1]), max3(y[2], y[3], max3(x[0], x[1], x[2])));
      need = need || mloc[s] > thr[s];
    }
    return need;
  }

  // P = 2^(S sl - m) as the packed B operand of the PV product, and this
  // lane's sums of P per m-row (ls, not yet added to l).
  __device__ void probs(float sl, const f32x4 (&sc)[NM][2], u32x4 (&pb)[NM], float (&ls)[NM]) const {
#pragma unroll
    for (int s = 0; s < NM; ++s) {
      float p[2][4];
#pragma unroll
      for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int j = 0; j < 4; ++j) p[h][j] = fast_exp2(__builtin_fmaf(sc[s][h][j], sl, -m[s]));
      ls[s] = ((p[0][0] + p[0][1]) + (p[0][2] + p[0][3])) + ((p[1][0] + p[1][1]) + (p[1][2] + p[1][3]));
      pb[s] = u32x4{TT::pack2(p[0][0], p[0][1]), TT::pack2(p[0][2], p[0][3]),
                    TT::pack2(p[1][0], p[1][1]), TT::pack2(p[1][2], p[1][3])};
    }
  }

  // Moves the references of the m-rows whose scores call for it (mloc: this
  // lane's raw maxima from lazy_check): the new reference is the row's
  // maximum in log2 units, O and the row sums are rescaled to it.
  __device__ void move_refs(float sl, const float (&mloc)[NM]) {
#pragma unroll
    for (int s = 0; s < NM; ++s) {
      float mx = fmaxf(mloc[s], __shfl_xor(mloc[s], 16, kWave));
      mx = fmaxf(mx, __shfl_xor(mx, 32, kWave)) * sl;
      const float mnew = fmaxf(m[s], mx);
      const float corr = fast_exp2(m[s] - mnew);
      m[s] = mnew;
      thr[s] = (mnew + kLazyRescale) / sl;
      l[s] *= corr;
#pragma unroll
      for (int e = 0; e < EPL; ++e) o[s][e] *= corr;
    }
  }

  // Softmax of a tile with no masked key: P formed with the current
  // references first, so that everything up to the rare move of a
  // reference is one branch-free block the scheduler can interleave with
  // MFMAs, and formed again after a move.
  __device__ void softmax_nomask(float sl, const f32x4 (&sc)[NM][2], u32x4 (&pb)[NM]) {
    float mloc[NM], ls[NM];
    const bool need = lazy_check(sc, mloc);
    probs(sl, sc, pb, ls);
    if (__builtin_amdgcn_ballot_w64(need) != 0) {
      move_refs(sl, mloc);
      probs(sl, sc, pb, ls);
    }
#pragma unroll
    for (int s = 0; s < NM; ++s) l[s] += ls[s];
  }

  // V^T operands of a tile, read with ds_read_b64_tr_b16.  Within a 16-lane
  // group, lane l of the read gets element l % 4 of the 8-byte pieces the
  // lanes 4j + l/4 address (j = 0..3).  Lane n (group g) addresses V row
  // key (4g + n/4, plus 16 for the second read) at head_dim 16e + 4(n % 4), so
  // it receives V[key 4g+j (+16)][16e + n] for j = 0..3: the A operand of
  // O^T += V^T . P^T for head_dim rows 16e .. 16e+15, in the key order of P^T
  // (slots 8g..8g+3 = keys 4g..4g+3, slots 8g+4.. = keys 16+4g..).  VB blocks of
  // 16 head_dim values from block e0.
  static constexpr int VB = EPL < 8 ? EPL : 8;
  template <class Tile>
  __device__ void read_vt(const char* vt, int e0, u32x4 (&va)[VB]) const {
    typedef __attribute__((address_space(3))) s16x4* lds4_t;
    const int r = 4 * g + (n >> 2);
#pragma unroll
    for (int e = 0; e < VB; ++e) {
      const int d0 = 16 * (e0 + e) + 4 * (n & 3);
      const char* p = vt + Tile::offset(r, d0 >> 3) + 2 * (d0 & 7);
      const s16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds4_t)(p));
      const s16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds4_t)(p + 16 * Tile::RB));
      const u32x2 l2 = __builtin_bit_cast(u32x2, lo), h2 = __builtin_bit_cast(u32x2, hi);
      va[e] = u32x4{l2.x, l2.y, h2.x, h2.y};
    }
  }

  // O^T += V^T . P^T with O^T in head_dim blocks: o[s][e] row i is head_dim
  // 16e + i (lane (n, g) holds 16e + 4g + j of m-row n).  va holds blocks
  // 0 .. VB-1 on entry.
  template <class Tile>
  __device__ void pv_lds(const char* vt, u32x4 (&va)[VB], const u32x4 (&pb)[NM]) {
    // (va is overwritten when EPL > VB.)
#pragma unroll
    for (int e0 = 0; e0 < EPL; e0 += VB) {
      if (e0 > 0) read_vt<Tile>(vt, e0, va);
#pragma unroll
      for (int e = 0; e < VB; ++e)
#pragma unroll
        for (int s = 0; s < NM; ++s) o[s][e0 + e] = TT::mfma(va[e], pb[s], o[s][e0 + e]);
    }
  }

  // Final O (q dtype) and natural-log LSE of m-row s in the head_dim-block
  // layout of pv_lds, to token t.
  __device__ void store_final_blocks(const AttnArgs& a, int s, int64_t t, float ltot) const {
    const float inv = ltot > 0.f ? 1.f / ltot : 0.f;
    st* op = static_cast<st*>(a.o) + t * a.o_st + static_cast<int64_t>(row_head(a, s)) * a.o_sh + 4 * g;
#pragma unroll
    for (int e = 0; e < EPL; ++e)
      *reinterpret_cast<u32x2*>(op + 16 * e) =
          u32x2{TT::pack2(o[s][e][0] * inv, o[s][e][1] * inv), TT::pack2(o[s][e][2] * inv, o[s][e][3] * inv)};
    if (a.lse && g == 0)
      a.lse[t * a.l_st + static_cast<int64_t>(row_head(a, s)) * a.l_sh] =
          ltot > 0.f ? (m[s] + __log2f(ltot)) * kLn2 : -INFINITY;
  }

  // Normalised O (fp32) and log2-domain LSE of m-row s to split-K partial
  // `slot`, query head hh of its kv head, in the layout of the decode
  // partials.
  __device__ void store_partial_blocks(const AttnArgs& a, int s, int64_t slot, int hh, float ltot) const {
    const float inv = ltot > 0.f ? 1.f / ltot : 0.f;
    float* op = a.ws_o + (slot * a.G + hh) * D + 4 * g;
#pragma unroll
    for (int e = 0; e < EPL; ++e)
      *reinterpret_cast<f32x4*>(op + 16 * e) = f32x4{o[s][e][0] * inv, o[s][e][1] * inv, o[s][e][2] * inv,
                                                     o[s][e][3] * inv};
    if (g == 0) a.ws_lse[slot * a.G + hh] = ltot > 0.f ? m[s] + __log2f(ltot) : -INFINITY;
  }

  // Softmax of a tile's raw scores sc (from qk_ops): keys at or past kstop
  // or past an m-row's causal limit masked when `mask`, references moved and
  // O and the row sums rescaled when a score calls for it, row sums added;
  // P packed as the B operand of the tile's PV product.
  __device__ void mask_tile(f32x4 (&sc)[NM][2], int ts, int kstop) const {
#pragma unroll
    for (int s = 0; s < NM; ++s)
#pragma unroll
      for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int tk = ts + 16 * h + 4 * g + j;
          sc[s][h][j] = (tk < kstop && tk <= qlimit(s)) ? sc[s][h][j] : -INFINITY;
        }
  }
  __device__ void softmax_tile(float sl, f32x4 (&sc)[NM][2], bool mask, int ts, int kstop, u32x4 (&pb)[NM]) {
    if (mask) mask_tile(sc, ts, kstop);
    float mloc[NM], ls[NM];
    if (__builtin_amdgcn_ballot_w64(lazy_check(sc, mloc)) != 0) move_refs(sl, mloc);
    probs(sl, sc, pb, ls);
#pragma unroll
    for (int s = 0; s < NM; ++s) l[s] += ls[s];
  }

  // Row sums over the four lane groups that share an m-row.
  __device__ void row_sums(float (&ltot)[NM]) const {
#pragma unroll
    for (int s = 0; s < NM; ++s) {
      const float t = l[s] + __shfl_xor(l[s], 16, kWave);
      ltot[s] = t + __shfl_xor(t, 32, kWave);
    }
  }
};

// --------------------------------------------------------------- decode --
// A decode row's keys are cut into (row, kv head, partition) segments, and a
// segment into "ranges" of 16-token slices, one range per wave of a
// work-group (host schedule from kvhot_paged_attention_schedule, or the grid:
// work-group (group, partition, row) takes W/S kv heads of one row, S waves
// each, S from decode_splits).
//
// Waves of one CU stream at very different rates (measured: equal ranges end
// up to 20 us apart inside one work-group, while work-group means agree to a
// few percent), so ranges are only a starting point.  Each wave claims its
// slices one at a time from an LDS counter; when its range is used up it
// claims slices from the range with the most left, first among waves of its
// own segment (the online softmax takes keys in any order), then from other
// segments.  Every (wave, segment) pair a wave worked on leaves a normalised
// (LSE, O) in an LDS slot: its own slot first, then slots from a pool of
// `dec_slots - W` (when the pool is empty the wave stops taking new segments).
// After a barrier the first wave of each segment merges that segment's slots.
// With KVHOT_DETERMINISTIC (AttnArgs::fixed) a wave claims from its own range
// only and stops when it is used up: slices are summed in the same order on
// every call.
// A segment that is one of several partitions of its row stores an (LSE, O)
// partial to HBM instead, and attn_merge_kernel combines the partitions in a
// second launch.  (Merging across work-groups inside one launch needs a
// device-scope release per wave, which on gfx950 is an L2 write-back per wave
// -- far slower than a launch.)

// Slices in flight per decode wave: 1 (load the next slice after computing
// this one) or 2 (double-buffered).
#ifndef KVHOT_DECODE_DEPTH
#define KVHOT_DECODE_DEPTH 1
#endif

#ifndef KVHOT_SLICES_PER_WAVE
#define KVHOT_SLICES_PER_WAVE 8
#endif

// Waves per kv head in grid mode for a partition of nslices slices: the
// smallest power of two up to W that keeps each wave near
// KVHOT_SLICES_PER_WAVE slices and leaves no more than Hkv kv heads to a
// work-group (no idle waves).
__host__ __device__ inline int decode_splits(int nslices, int W, int Hkv) {
  int S = 1;
  while (S < W && (S * KVHOT_SLICES_PER_WAVE < nslices || W / S > Hkv)) S *= 2;
  return S;
}

// LDS of a decode work-group with P ranges and S slots, in 4-byte words: per
// slot the normalised O [G][D] and base-2 LSE [G] of its query heads and its
// segment key (row, kv head, part); per range the claim counter, range end
// and segment description [8]; the slot-pool counter.
constexpr int kDecInfo = 8;
// Bit of a decode descriptor's part field: the segment folds in its row's
// shared-prefix partials.
constexpr int kPrefixFold = 0x8000;
// Prefix partials a fold reads per round trip.
constexpr int kFoldBatch = 8;
__host__ __device__ constexpr int64_t decode_lds_words(int64_t P, int64_t S, int64_t G, int64_t D) {
  return S * G * D + S * G + 4 * S + (2 + kDecInfo) * P + 1;
}

__device__ inline int wave_max_int(int x) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) x = max(x, __shfl_xor(x, o, kWave));
  return x;
}

// One decode work-group: launch-list work-group bx (decode descriptors at
// sched), or without a launch list grid work-group (bx, by, bz).
// MR: the launch list gives a work-group more ranges than waves (fixed
// partitions, decode_ranges); otherwise one range per wave, and P is W.
// VB: KVHOT_VERIFY_BLOCKS (below).
template <class TT, int D, int W, bool MR, bool VB>
__device__ __attribute__((always_inline)) inline void decode_wg(const AttnArgs& a, const int4* sched, int bx, int by,
                                                                int bz) {
  extern __shared__ float smem[];
  using st = uint16_t;
  // Wave-uniform values are pinned to SGPRs with readfirstlane: derived from
  // threadIdx they would otherwise count as divergent, putting block ids and
  // buffer descriptors in VGPRs (a waterfall loop around every load).
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int G = a.G;
  const int PT = a.part_tokens;
  const int S = a.dec_slots;
  const int P = MR ? a.dec_ranges : W;  // ranges: wave w starts on range w (w < W <= P)
  const bool fixed = a.fixed != 0;

  // ---- this wave's range: slices [s0, s1) of part `part` of (row, kvh) ----
  int row = -1, kvh = 0, s0 = 0, s1 = 0, part = 0, nparts = 0, kend = 0;
  int64_t qs = 0, pidx = 0;
  int d_first = -1;
  if (sched) {
    // (row | parts << 16, kvh | part << 16, s0, s1), (query token, visible
    // keys, physical block of slice s0 or -1, partial index).  part with bit
    // 15 set (kPrefixFold): the row's shared prefix left `parts` partials
    // from index pidx in an earlier launch; this segment, the rest of the
    // row, folds them in and writes the row's output.
    const int4* u = sched + 2 * (static_cast<int64_t>(bx) * P + wave);
    const int4 u0 = u[0], u1 = u[1];
    const int x = __builtin_amdgcn_readfirstlane(u0.x);
    const int y = __builtin_amdgcn_readfirstlane(u0.y);
    if (x >= 0) {
      row = x & 0xffff;
      nparts = (x >> 16) & 0xffff;
      kvh = y & 0xffff;
      part = (y >> 16) & 0xffff;
    }
    s0 = __builtin_amdgcn_readfirstlane(u0.z);
    s1 = __builtin_amdgcn_readfirstlane(u0.w);
    qs = __builtin_amdgcn_readfirstlane(u1.x);
    kend = __builtin_amdgcn_readfirstlane(u1.y);
    d_first = __builtin_amdgcn_readfirstlane(u1.z);
    pidx = __builtin_amdgcn_readfirstlane(u1.w);
  } else {
    const int r = bz;
    const int p = by;
    if (a.q_lens[r] != 1) return;
    const int ke_r = decode_visible_keys(a, r);
    const int np = max((ke_r + PT - 1) / PT, 1);
    if (p >= np) return;
    const int kbeg = p * PT;
    const int nsl = max((min(ke_r, kbeg + PT) - kbeg + 15) / 16, 0);
    const int Sp = decode_splits(nsl, W, a.Hkv);
    const int HW = W / Sp;
    if (static_cast<int>(bx) * HW >= a.Hkv) return;
    const int h = bx * HW + wave / Sp;
    const int split = wave % Sp;
    if (h < a.Hkv) {
      row = r;
      kvh = h;
      s0 = kbeg / 16 + (nsl * split) / Sp;
      s1 = kbeg / 16 + (nsl * (split + 1)) / Sp;
      part = p;
      nparts = np;
      kend = ke_r;
      qs = a.q_starts[r];
      pidx = (static_cast<int64_t>(r) * a.Hkv + h) * a.max_parts + p;
      // The first slice's block, as a launch list would give it.
      const int64_t lb = (16 * static_cast<int64_t>(s0)) / a.bs;
      if (s1 > s0 && lb < a.bt_stride) {
        const int64_t id = a.bt[static_cast<int64_t>(r) * a.bt_stride + lb];
        d_first = static_cast<int>(id < 0 ? 0 : (id >= a.num_blocks ? a.num_blocks - 1 : id));
      }
    }
  }
  row = __builtin_amdgcn_readfirstlane(row);
  kvh = __builtin_amdgcn_readfirstlane(kvh);
  s0 = __builtin_amdgcn_readfirstlane(s0);
  s1 = __builtin_amdgcn_readfirstlane(s1);
  const bool fold = (part & kPrefixFold) != 0;
  const bool valid = row >= 0 && kvh >= 0 && kvh < a.Hkv && qs >= 0 && qs < a.total_q && s0 >= 0 &&
                     nparts >= 1 &&
                     (fold ? part == kPrefixFold && pidx >= 0 && pidx + nparts <= a.num_partials
                           : part < nparts && (nparts == 1 || (pidx >= 0 && pidx < a.num_partials)));
  const int kb = 16 * s0;
  const int ke = min(kend, 16 * s1);
  const int nsl = valid && ke > kb ? (ke - kb + 15) / 16 : 0;

  float* so = smem;                                      // [S][G][D]
  float* sl = so + static_cast<int64_t>(S) * G * D;      // [S][G]
  int* skey = reinterpret_cast<int*>(sl + S * G);        // [S][4] row, kvh, part, -
  int* cnt = skey + 4 * S;                               // [P] next slice to claim
  int* dend = cnt + P;                                   // [P] end of the range
  int* info = dend + P;                                  // [P][kDecInfo]
  int* nslot = info + kDecInfo * P;                      // slots handed out

  const int bs = a.bs;
  auto block_of = [&](int r, int slice) -> int64_t {     // physical block of a slice
    const int64_t lb = (16 * static_cast<int64_t>(slice)) / bs;
    int64_t id = lb < a.bt_stride ? a.bt[static_cast<int64_t>(r) * a.bt_stride + lb] : 0;
    return id < 0 ? 0 : (id >= a.num_blocks ? a.num_blocks - 1 : id);
  };

  // The current segment (starts as this wave's own).  A decode row's causal
  // limit is already in kend (its one query sees keys [0, kend)), so the
  // query position passed to the m-row setup is kend - 1.
  int krow = valid ? row : -1, kkvh = kvh, kpart = part, kkend = kend;

  WaveAttn<TT, D, 1> wa;
  wa.setup(a, lane, valid ? kvh : 0, qs, 0, valid ? 1 : 0, kend - 1);
  KVSlice<D> T;
  int i = s0;              // slice whose loads are in flight, if `have`
  bool have = nsl > 0;     // the first slice of the range is taken without a claim
#if KVHOT_DECODE_DEPTH < 2
  // The first slice's block comes from the launch list, built from the host
  // copy of the block table, so that its loads wait for nothing.  With
  // KVHOT_VERIFY_BLOCKS the device table's entry is read before them and
  // compared before the slice is used: a caller that edited only the device
  // table gets the slice loaded again from the block the device table names.
  // (Off by default: waiting for that entry before the first claim cost
  // 1-2% of a decode call.)
  // (A buffer load: its wait is counted with the slice's vector loads, in
  // order, rather than with LDS operations.  The check is made once, before
  // the loop, so that nothing of it is carried through the loop.)
  const bool check_first = VB && sched && have && d_first >= 0;
  int dev_first = 0;
  if (check_first) {
    const int64_t lb = (16 * static_cast<int64_t>(s0)) / bs;
    const __amdgpu_buffer_rsrc_t br =
        block_rsrc(a.bt + static_cast<int64_t>(row) * a.bt_stride, static_cast<int>(4 * a.bt_stride));
    dev_first = __builtin_amdgcn_raw_buffer_load_b32(br, static_cast<int>(4 * lb), 0, 0);
  }
  if (have)
    wa.load_slice(a, kvh, d_first >= 0 ? min(static_cast<int64_t>(d_first), a.num_blocks - 1) : block_of(row, s0),
                  kb % bs, T);
#endif
  if (lane == 0) {
    cnt[wave] = s0 + (have ? 1 : 0);
    dend[wave] = s0 + nsl;
    int* d = info + kDecInfo * wave;
    d[0] = krow; d[1] = kvh; d[2] = part; d[3] = nparts;
    d[4] = static_cast<int>(qs); d[5] = kend; d[6] = static_cast<int>(pidx); d[7] = 1;
    skey[4 * wave] = -1;
    if (wave == 0) *nslot = P;
  }
  // Ranges past the first W (launch lists of fixed partitions): wave w sets up
  // ranges w + W, w + 2W, ...; they start untouched (d[7] = 0), each with its
  // own slot, the one of the same index.
  if constexpr (MR)
  for (int r = wave + W; r < P; r += W) {
    const int4* u = sched + 2 * (static_cast<int64_t>(bx) * P + r);
    const int4 u0 = u[0], u1 = u[1];
    const int x = __builtin_amdgcn_readfirstlane(u0.x);
    const int y = __builtin_amdgcn_readfirstlane(u0.y);
    const int rr = x >= 0 ? (x & 0xffff) : -1, rnp = (x >> 16) & 0xffff;
    const int rh = y & 0xffff, rp = (y >> 16) & 0xffff;
    const int rs0 = __builtin_amdgcn_readfirstlane(u0.z), rs1 = __builtin_amdgcn_readfirstlane(u0.w);
    const int rqs = __builtin_amdgcn_readfirstlane(u1.x), rke = __builtin_amdgcn_readfirstlane(u1.y);
    const int rpi = __builtin_amdgcn_readfirstlane(u1.w);
    const bool rfold = (rp & kPrefixFold) != 0;
    const bool rvalid = x >= 0 && rh < a.Hkv && rqs >= 0 && rqs < a.total_q && rs0 >= 0 && rnp >= 1 &&
                        (rfold ? rp == kPrefixFold && rpi >= 0 && static_cast<int64_t>(rpi) + rnp <= a.num_partials
                               : rp < rnp && (rnp == 1 || (rpi >= 0 && rpi < a.num_partials)));
    const int rke2 = min(rke, 16 * rs1);
    const int rn = rvalid && rke2 > 16 * rs0 ? (rke2 - 16 * rs0 + 15) / 16 : 0;
    if (lane == 0) {
      cnt[r] = rs0;
      dend[r] = rs0 + rn;
      int* d = info + kDecInfo * r;
      d[0] = rvalid ? rr : -1; d[1] = rh; d[2] = rp; d[3] = rnp;
      d[4] = rqs; d[5] = rke; d[6] = rpi; d[7] = 0;
      skey[4 * r] = -1;
    }
  }
  // LDS-only barrier: the first slice's loads stay in flight across it.
  __asm__ volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
#if KVHOT_DECODE_DEPTH < 2
  if (check_first) {
    const int raw = __builtin_amdgcn_readfirstlane(dev_first);
    const int64_t want = raw < 0 ? 0 : (raw >= a.num_blocks ? a.num_blocks - 1 : raw);
    if (want != min(static_cast<int64_t>(d_first), a.num_blocks - 1)) wa.load_slice(a, kvh, want, kb % bs, T);
  }
#endif

  // Claims one slice of range v (-1 when the range is used up).
  auto claim = [&](int v) -> int {
    int r = 0;
    if (lane == 0) r = atomicAdd(&cnt[v], 1);
    r = __builtin_amdgcn_readlane(r, 0);
    return r < __builtin_amdgcn_readfirstlane(dend[v]) ? r : -1;
  };
  // Range with the most slices left (only ranges of the current segment when
  // same_segment), or -1.
  auto pick = [&](bool same_segment) -> int {
    int best = -1;
    if (lane < P) {
      const int left = dend[lane] - cnt[lane];
      const int* d = info + kDecInfo * lane;
      bool ok = left > 0;
      if (same_segment) ok = ok && d[0] == krow && d[1] == kkvh && d[2] == kpart;
      best = ok ? (min(left, 1 << 24) << 6) | lane : -1;
    }
    best = wave_max_int(best);
    return best < 0 ? -1 : (best & 63);
  };
  int slot = wave;
  bool used = false;       // the slot holds work
  auto flush = [&]() {
    float lt[1];
    wa.row_sums(lt);
    if (wa.mval[0]) {
      const float inv = lt[0] > 0.f ? 1.f / lt[0] : 0.f;
      float* dst = so + (static_cast<int64_t>(slot) * G + wa.n) * D;
#pragma unroll
      for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int e = 0; e < D / 16; e += 4)
          *reinterpret_cast<f32x4*>(dst + (D / 16) * (4 * wa.g + j) + e) =
              f32x4{wa.o[0][e][j] * inv, wa.o[0][e + 1][j] * inv, wa.o[0][e + 2][j] * inv,
                    wa.o[0][e + 3][j] * inv};
      if (wa.g == 0) sl[slot * G + wa.n] = lt[0] > 0.f ? wa.m[0] + __log2f(lt[0]) : -INFINITY;
    }
    if (lane == 0) {
      skey[4 * slot + 0] = krow;
      skey[4 * slot + 1] = kkvh;
      skey[4 * slot + 2] = kpart;
      skey[4 * slot + 3] = 0;
    }
  };

#if KVHOT_DECODE_DEPTH < 2
  int cv = wave;           // range being claimed from
  int own = wave;          // the last of this wave's own ranges it entered (deterministic order)
  bool live = nsl > 0;     // the current segment may still have slices
  for (;;) {
    int j = -1;
    if (live) {
      j = claim(cv);
      while (j < 0 && !fixed) {
        const int v = pick(true);
        if (v < 0) break;
        cv = v;
        j = claim(cv);
      }
      live = j >= 0;
    }
    // The next slice's block id is fetched while this slice's loads land.
    const int64_t jb = j >= 0 ? block_of(__builtin_amdgcn_readfirstlane(krow), __builtin_amdgcn_readfirstlane(j)) : 0;
    if (have) {
      wa.compute_slice(a, 16 * i, kkend, INT_MAX, T);
      used = true;
    }
    if (j >= 0) {
      i = j;
      // The slice's bases and offset are broadcast: they are uniform, but are
      // carried out of claim loops the compiler cannot prove uniform, and a
      // per-lane buffer descriptor puts each load in a loop over the distinct
      // descriptors that waits for the load before it.
      wa.load_slice_from(a, uniform_ptr(static_cast<const st*>(a.k) + static_cast<int64_t>(kkvh) * a.k_sh + jb * a.k_sb),
                         uniform_ptr(static_cast<const st*>(a.v) + static_cast<int64_t>(kkvh) * a.v_sh + jb * a.v_sb),
                         __builtin_amdgcn_readfirstlane((16 * j) % bs), T);
      have = true;
      continue;
    }
    have = false;
    // Segment exhausted: park its state, then take slices of another one:
    // the range with the most left, or with KVHOT_DETERMINISTIC the wave's
    // own next range (ranges w + W, w + 2W, ... of a launch list of fixed
    // partitions), in order.
    if (used) flush();
    int v = -1;
    if (fixed) {
      if constexpr (MR) {
        for (own += W; own < P; own += W)
          if (__builtin_amdgcn_readfirstlane(dend[own] - cnt[own]) > 0) {
            v = own;
            break;
          }
      }
    } else {
      v = pick(false);
    }
    if (v < 0) break;
    // The first wave to enter a range parks its state in the range's own
    // slot; a later one takes a slot from the pool (none left: it stops,
    // and the range's other waves finish it).  (One range per wave: every
    // range was entered by its wave at the start.)
    int first = 0;
    if constexpr (MR) {
      if (lane == 0) first = atomicExch(&info[kDecInfo * v + 7], 1) == 0 ? 1 : 0;
      first = __builtin_amdgcn_readlane(first, 0);
    }
    if (first) {
      slot = v;
      used = false;
    } else if (used) {
      int ns = 0;
      if (lane == 0) ns = atomicAdd(nslot, 1);
      ns = __builtin_amdgcn_readlane(ns, 0);
      if (ns >= S) break;
      slot = ns;
      if (lane == 0) skey[4 * slot] = -1;
      used = false;
    }
    const int* d = info + kDecInfo * v;
    krow = __builtin_amdgcn_readfirstlane(d[0]);
    kkvh = __builtin_amdgcn_readfirstlane(d[1]);
    kpart = __builtin_amdgcn_readfirstlane(d[2]);
    kkend = __builtin_amdgcn_readfirstlane(d[5]);
    wa.setup(a, lane, kkvh, __builtin_amdgcn_readfirstlane(d[4]), 0, 1, kkend - 1);
    cv = v;
    live = true;
  }
#else
  // Two slices in flight per wave: the older in one buffer, the newer in the
  // other, and the block-table entry of the next claimed slice (iz) loading
  // behind them.  A half-step computes the older buffer, claims one more
  // slice and issues its block-table load, then refills the computed buffer
  // with iz.  iz's entry was loaded before the newer buffer's K/V, so waiting
  // for it leaves that buffer in flight (vector loads complete in order).
  KVSlice<D> T1;
  int ix = i, iy = 0, iz = 0, zraw = 0;
  bool hx = have, hy = false, hz = false;
  int cv = wave;           // range being claimed from
  bool live = nsl > 0;     // the current segment may still have slices
  auto claim_next = [&]() {
    hz = false;
    int j = -1;
    if (live) {
      j = claim(cv);
      while (j < 0 && !fixed) {
        const int v = pick(true);
        if (v < 0) break;
        cv = v;
        j = claim(cv);
      }
      live = j >= 0;
    }
    // The entry is loaded on every path (entry 0 of the row when nothing was
    // claimed), so the vector loads of each half-step come in one order.
    const int64_t lb = j >= 0 ? (16 * static_cast<int64_t>(j)) / bs : 0;
    const int r = max(__builtin_amdgcn_readfirstlane(krow), 0);
    const int64_t e = lb < a.bt_stride ? lb : a.bt_stride - 1;
    zraw = a.bt[static_cast<int64_t>(r) * a.bt_stride + (e > 0 ? e : 0)];
    iz = max(j, 0);
    hz = j >= 0;
  };
  // Computes the older buffer X, then refills it with slice iz.  The refill is
  // issued on every path (no bytes when nothing was claimed): the waits the
  // compiler places before a compute then always leave the other buffer's
  // loads in flight.
  auto half = [&](KVSlice<D>& X, int& ix_, bool& hx_) {
    if (hx_) {
      wa.compute_slice(a, 16 * ix_, kkend, INT_MAX, X);
      used = true;
    }
    const bool take = __builtin_amdgcn_readfirstlane(static_cast<int>(hz)) != 0;
    const int j = __builtin_amdgcn_readfirstlane(iz);
    const int64_t jr = __builtin_amdgcn_readfirstlane(zraw);
    const int64_t jb = jr < 0 ? 0 : (jr >= a.num_blocks ? a.num_blocks - 1 : jr);
    claim_next();
    wa.load_slice_from(a, uniform_ptr(static_cast<const st*>(a.k) + static_cast<int64_t>(kkvh) * a.k_sh + jb * a.k_sb),
                       uniform_ptr(static_cast<const st*>(a.v) + static_cast<int64_t>(kkvh) * a.v_sh + jb * a.v_sb),
                       __builtin_amdgcn_readfirstlane((16 * j) % bs), X, take);
    ix_ = j;
    hx_ = take;
  };
  // Segment exhausted and both buffers computed: park its state, then take
  // slices of another one.
  auto next_segment = [&]() -> bool {
    if (used) flush();
    if (fixed) return false;
    const int v = pick(false);
    if (v < 0) return false;
    if (used) {
      int ns = 0;
      if (lane == 0) ns = atomicAdd(nslot, 1);
      ns = __builtin_amdgcn_readlane(ns, 0);
      if (ns >= S) return false;
      slot = ns;
      if (lane == 0) skey[4 * slot] = -1;
      used = false;
    }
    const int* d = info + kDecInfo * v;
    krow = __builtin_amdgcn_readfirstlane(d[0]);
    kkvh = __builtin_amdgcn_readfirstlane(d[1]);
    kpart = __builtin_amdgcn_readfirstlane(d[2]);
    kkend = __builtin_amdgcn_readfirstlane(d[5]);
    wa.setup(a, lane, kkvh, __builtin_amdgcn_readfirstlane(d[4]), 0, 1, kkend - 1);
    cv = v;
    live = true;
    claim_next();
    // Both buffers are computed here: waiting for the new Q and block-table
    // entry now costs nothing, and keeps the loop's waits (which must hold on
    // every path into it) from draining the other buffer after each half-step.
    __builtin_amdgcn_s_waitcnt((7 << 4) | (15 << 8));  // vmcnt(0)
    return true;
  };
  // The slice after the range's first, then the first (taken without a
  // claim) into T, always issued: the loads enter the loop in the order each
  // half-step leaves them (a block-table entry, then a buffer's K/V).
  claim_next();
  {
    // (The first block from the device table, which the launch list's copy
    // may not match.)
    const bool h0 = __builtin_amdgcn_readfirstlane(static_cast<int>(have)) != 0;
    wa.load_slice(a, kvh, h0 ? block_of(row, s0) : 0, kb % bs, T, h0);
  }
  for (;;) {
    half(T1, iy, hy);
    half(T, ix, hx);
    if (!hx && !hy && !hz && !next_segment()) break;
  }
#endif
  __syncthreads();

  // ---- merge: each range's slots are combined by the wave that set the
  // range up (a segment split over several ranges: by the first of them) ----
  const int nused = min(__builtin_amdgcn_readfirstlane(*nslot), S);
  auto merge = [&](int mrow, int mkvh, int mpart, int mnp, int64_t mpidx, int64_t mqs) {
    const bool mfold = (mpart & kPrefixFold) != 0;
    const bool mine = lane < nused && skey[4 * lane] == mrow && skey[4 * lane + 1] == mkvh &&
                      skey[4 * lane + 2] == mpart;
    const uint64_t slots = __ballot(mine);
    for (int it = lane; it < G * (D / 4); it += 64) {
      const int hh = it / (D / 4);
      const int d0 = 4 * (it % (D / 4));
      // The slots' states, weighted against their maximum.
      float mx = -INFINITY;
      for (uint64_t b = slots; b; b &= b - 1) mx = fmaxf(mx, sl[__builtin_ctzll(b) * G + hh]);
      f32x4 acc = {0.f, 0.f, 0.f, 0.f};
      float lsum = 0.f;
      if (mx != -INFINITY) {
        for (uint64_t b = slots; b; b &= b - 1) {
          const int w = __builtin_ctzll(b);
          const float wt = fast_exp2(sl[w * G + hh] - mx);
          lsum += wt;
          acc += wt * *reinterpret_cast<const f32x4*>(so + (static_cast<int64_t>(w) * G + hh) * D + d0);
        }
      }
      if (mfold) {
        // The prefix partials, kFoldBatch at a time with all their loads in
        // flight together (indices past the last partial re-read it, weight 0),
        // combined with a running maximum.
        for (int p0 = 0; p0 < mnp; p0 += kFoldBatch) {
          float lp[kFoldBatch];
          f32x4 ov[kFoldBatch];
#pragma unroll
          for (int k = 0; k < kFoldBatch; ++k) {
            const int64_t pi = mpidx + min(p0 + k, mnp - 1);
            lp[k] = a.ws_lse[pi * G + hh];
            ov[k] = *reinterpret_cast<const f32x4*>(a.ws_o + (pi * G + hh) * D + d0);
          }
          float cm = mx;
#pragma unroll
          for (int k = 0; k < kFoldBatch; ++k) {
            if (p0 + k >= mnp) lp[k] = -INFINITY;
            cm = fmaxf(cm, lp[k]);
          }
          if (cm == -INFINITY) continue;
          const float sc = mx == -INFINITY ? 0.f : fast_exp2(mx - cm);
          acc *= sc;
          lsum *= sc;
#pragma unroll
          for (int k = 0; k < kFoldBatch; ++k) {
            const float wt = lp[k] == -INFINITY ? 0.f : fast_exp2(lp[k] - cm);
            lsum += wt;
            acc += wt * ov[k];
          }
          mx = cm;
        }
      }
      const float inv = lsum > 0.f ? 1.f / lsum : 0.f;
      const int h = mkvh * G + hh;
      const float lse2 = lsum > 0.f ? mx + __log2f(lsum) : -INFINITY;
      if (mnp == 1 || mfold) {
        st* dp = static_cast<st*>(a.o) + mqs * a.o_st + static_cast<int64_t>(h) * a.o_sh + d0;
        *reinterpret_cast<u32x2*>(dp) =
            u32x2{TT::pack2(acc.x * inv, acc.y * inv), TT::pack2(acc.z * inv, acc.w * inv)};
        if (a.lse && d0 == 0) a.lse[mqs * a.l_st + static_cast<int64_t>(h) * a.l_sh] = lse2 * kLn2;
      } else {
        *reinterpret_cast<f32x4*>(a.ws_o + (mpidx * G + hh) * D + d0) = acc * inv;
        if (d0 == 0) a.ws_lse[mpidx * G + hh] = lse2;
      }
    }
  };
  if constexpr (!MR) {
    // One range per wave: the first wave of each segment merges it.
    if (!valid) return;
    if (wave > 0) {
      const int* d = info + kDecInfo * (wave - 1);
      if (d[0] == row && d[1] == kvh && d[2] == part) return;
    }
    merge(row, kvh, part, nparts, pidx, qs);
    return;
  }
  // (Each range's description is read back from LDS rather than held in
  // registers through the loop; without a launch list the partial index is
  // recomputed, as it may not fit the table's 32 bits.)
  for (int r = wave; r < P; r += W) {
    const int* d = info + kDecInfo * r;
    const int mrow = __builtin_amdgcn_readfirstlane(d[0]);
    if (mrow < 0) continue;
    const int mkvh = __builtin_amdgcn_readfirstlane(d[1]);
    const int mpart = __builtin_amdgcn_readfirstlane(d[2]);
    const int mnp = __builtin_amdgcn_readfirstlane(d[3]);
    const int64_t mqs = __builtin_amdgcn_readfirstlane(d[4]);
    const int64_t mpidx = sched ? static_cast<int64_t>(__builtin_amdgcn_readfirstlane(d[6]))
                                : (static_cast<int64_t>(mrow) * a.Hkv + mkvh) * a.max_parts + mpart;
    // Ranges of one segment are consecutive (the planner gives a segment's
    // waves consecutive ranges; a range of fixed partitions is its own
    // segment): the first of them merges.
    if (r > 0) {
      const int* d2 = info + kDecInfo * (r - 1);
      if (__builtin_amdgcn_readfirstlane(static_cast<int>(d2[0] == mrow && d2[1] == mkvh && d2[2] == mpart)) != 0)
        continue;
    }
    merge(mrow, mkvh, mpart, mnp, mpidx, mqs);
  }
}

template <class TT, int D, int W, bool MR = false, bool VB = false>
__global__ void __launch_bounds__(64 * W)
attn_decode_kernel(const AttnArgs a) {
  decode_wg<TT, D, W, MR, VB>(a, a.sched, blockIdx.x, blockIdx.y, blockIdx.z);
}

// Combines the parts of split decode segments: (row, kv head) pieces that
// ran in different work-groups and left (LSE, O) partials.  With a schedule,
// work-group u takes merge unit u = (query token, kv head, parts, first
// partial index), (first extra partial, extra partials) -- the extras are the
// key splits of a shared prefix the row reads, written by prefix units --
// each lane 8 head_dim values of one of the G query heads;
// the kMergeWaves waves of the work-group fold a share of the parts each and
// combine their states through LDS.  Without one, the grid is (head_dim
// chunks, rows) of one-wave work-groups, and a row's parts are the fixed
// partitions of part_tokens keys, recomputed as the decode kernel did.
constexpr int kMergeWaves = 4;

template <class TT, int D>
__global__ void __launch_bounds__(64 * kMergeWaves)
attn_merge_kernel(const AttnArgs a) {
  using st = uint16_t;
  constexpr int CH = D / 8;
  const int G = a.G;
  const int wv = static_cast<int>(threadIdx.x >> 6), nwv = static_cast<int>(blockDim.x >> 6);
  int64_t t, base, xbase = 0;
  int kvh, nparts, xparts = 0, it0, step;
  if (a.merge_units) {
    // (query token, kv head, parts, first partial), (first extra partial,
    // extra partials, 0, 0): the extra ones are a shared prefix's key splits.
    const int4 u = a.merge_units[2 * static_cast<int64_t>(blockIdx.x)];
    const int4 u1 = a.merge_units[2 * static_cast<int64_t>(blockIdx.x) + 1];
    t = u.x;
    kvh = u.y;
    nparts = u.z;
    base = u.w;
    xbase = u1.x;
    xparts = u1.y;
    it0 = threadIdx.x & 63;
    step = 64;
  } else {
    const int row = blockIdx.y;
    if (a.q_lens[row] != 1) return;
    const int idx = blockIdx.x * 64 + threadIdx.x;
    if (idx >= a.Hq * CH) return;
    const int PT = a.part_tokens;
    nparts = (decode_visible_keys(a, row) + PT - 1) / PT;
    if (nparts <= 1) return;
    t = a.q_starts[row];
    kvh = (idx / CH) / G;
    base = (static_cast<int64_t>(row) * a.Hkv + kvh) * a.max_parts;
    it0 = idx - kvh * G * CH;  // (head in group, chunk) of this lane
    step = G * CH;             // one item per lane
  }
  if (t < 0 || t >= a.total_q || kvh < 0 || kvh >= a.Hkv || nparts < 1 || base < 0 ||
      base + nparts > a.num_partials || xparts < 0 || xbase < 0 || xbase + xparts > a.num_partials)
    return;
  // Partial of the i-th input: the parts, then the extra ones.
  const int total = nparts + xparts;
  auto input = [&](int i) -> int64_t { return i < nparts ? base + i : xbase + (i - nparts); };
  constexpr int kFew = 4;  // up to this many inputs, every load is issued at once
  if (total <= kFew && wv > 0) return;  // one wave folds a few inputs
  __shared__ float part_state[kMergeWaves][64][10];  // max, sum, O (8 values) per wave and lane
  for (int it = it0; it < G * CH; it += step) {
    const int hh = it / CH;
    const int c = it % CH;
    float mmax = -INFINITY;
    f32x4 acc0 = {0.f, 0.f, 0.f, 0.f}, acc1 = {0.f, 0.f, 0.f, 0.f};
    float lsum = 0.f;
    if (total <= kFew) {
      float lv[kFew];
      f32x4 p0[kFew], p1[kFew];
#pragma unroll
      for (int pp = 0; pp < kFew; ++pp) {
        lv[pp] = -INFINITY;
        p0[pp] = p1[pp] = f32x4{0.f, 0.f, 0.f, 0.f};
        if (pp < total) {
          const int64_t pi = input(pp);
          lv[pp] = a.ws_lse[pi * G + hh];
          const f32x4* src = reinterpret_cast<const f32x4*>(a.ws_o + (pi * G + hh) * D + 8 * c);
          p0[pp] = src[0];
          p1[pp] = src[1];
        }
      }
#pragma unroll
      for (int pp = 0; pp < kFew; ++pp) mmax = fmaxf(mmax, lv[pp]);
      if (mmax != -INFINITY) {
#pragma unroll
        for (int pp = 0; pp < kFew; ++pp) {
          const float w = pp < total ? fast_exp2(lv[pp] - mmax) : 0.f;
          lsum += w;
          acc0 += w * p0[pp];
          acc1 += w * p1[pp];
        }
      }
    } else {
      // One pass, kBatch parts at a time: a batch's loads are issued
      // together, then folded in with the running max moved (long rows have
      // tens of parts, and a part-by-part loop waits for each load in turn).
      constexpr int kBatch = 8;
      const int lo = static_cast<int>((static_cast<int64_t>(total) * wv) / nwv);
      const int hi = static_cast<int>((static_cast<int64_t>(total) * (wv + 1)) / nwv);
      for (int b0 = lo; b0 < hi; b0 += kBatch) {
        float lv[kBatch];
        f32x4 p0[kBatch], p1[kBatch];
#pragma unroll
        for (int k = 0; k < kBatch; ++k) {
          lv[k] = -INFINITY;
          p0[k] = p1[k] = f32x4{0.f, 0.f, 0.f, 0.f};
          if (b0 + k < hi) {
            const int64_t pi = input(b0 + k);
            lv[k] = a.ws_lse[pi * G + hh];
            const f32x4* src = reinterpret_cast<const f32x4*>(a.ws_o + (pi * G + hh) * D + 8 * c);
            p0[k] = src[0];
            p1[k] = src[1];
          }
        }
        float bmax = -INFINITY;
#pragma unroll
        for (int k = 0; k < kBatch; ++k) bmax = fmaxf(bmax, lv[k]);
        if (bmax == -INFINITY) continue;
        const float mnew = fmaxf(mmax, bmax);
        const float corr = fast_exp2(mmax - mnew);  // 0 while mmax is -inf
        lsum *= corr;
        acc0 *= corr;
        acc1 *= corr;
#pragma unroll
        for (int k = 0; k < kBatch; ++k) {
          const float w = fast_exp2(lv[k] - mnew);
          lsum += w;
          acc0 += w * p0[k];
          acc1 += w * p1[k];
        }
        mmax = mnew;
      }
      if (nwv > 1) {
        // The waves' states meet in LDS; wave 0 combines them.
        float* my = part_state[wv][threadIdx.x & 63];
        my[0] = mmax;
        my[1] = lsum;
        my[2] = acc0.x; my[3] = acc0.y; my[4] = acc0.z; my[5] = acc0.w;
        my[6] = acc1.x; my[7] = acc1.y; my[8] = acc1.z; my[9] = acc1.w;
        __syncthreads();
        if (wv == 0) {
          float m2 = -INFINITY;
          for (int w = 0; w < nwv; ++w) m2 = fmaxf(m2, part_state[w][threadIdx.x][0]);
          lsum = 0.f;
          acc0 = acc1 = f32x4{0.f, 0.f, 0.f, 0.f};
          if (m2 != -INFINITY) {
            for (int w = 0; w < nwv; ++w) {
              const float* q = part_state[w][threadIdx.x];
              const float c2 = fast_exp2(q[0] - m2);  // 0 for a wave that saw no part
              lsum += c2 * q[1];
              acc0 += c2 * f32x4{q[2], q[3], q[4], q[5]};
              acc1 += c2 * f32x4{q[6], q[7], q[8], q[9]};
            }
          }
          mmax = m2;
        }
        __syncthreads();  // the states are read before the next item writes them
        if (wv > 0) continue;
      }
    }
    const float inv = lsum > 0.f ? 1.f / lsum : 0.f;
    const int h = kvh * G + hh;
    st* dp = static_cast<st*>(a.o) + t * a.o_st + static_cast<int64_t>(h) * a.o_sh + 8 * c;
    *reinterpret_cast<u32x4*>(dp) =
        u32x4{TT::pack2(acc0.x * inv, acc0.y * inv), TT::pack2(acc0.z * inv, acc0.w * inv),
              TT::pack2(acc1.x * inv, acc1.y * inv), TT::pack2(acc1.z * inv, acc1.w * inv)};
    if (a.lse && c == 0)
      a.lse[t * a.l_st + static_cast<int64_t>(h) * a.l_sh] =
          lsum > 0.f ? (mmax + __log2f(lsum)) * kLn2 : -INFINITY;
  }
}

// -------------------------------------------------------------- prefill --
// A work-group of prefill_waves(D) waves takes consecutive query blocks of
// one (row, kv head): wave w the 16*NM/G queries q0 + w*16*NM/G ... (all G
// heads of each).  Keys are walked in 32-key tiles that the work-group copies
// from the paged cache straight into LDS (buffer_load ... lds, no register
// staging) through a ring of four slots, three tiles ahead of the one being
// computed, so each K/V byte is read from HBM once per work-group and from
// LDS once per wave.  A wave skips tiles wholly past its own causal limit.
//
// At head_dim 64 and 128 a work-group is 4 waves, one per SIMD, and two
// work-groups share a CU (64 KiB of ring each, at most 256 VGPRs a wave).
// Their barriers are their own, so the two waves of a SIMD drift apart and
// one's MFMAs run while the other forms its softmax; with one 8-wave
// work-group per CU the two waves of a SIMD meet at every tile's barrier and
// their softmax phases coincide (measured on the mixed workload's prefill
// rows: 158 us with two 4-wave work-groups per CU against 172 us with one
// 8-wave work-group).  At head_dim 256 (a 128 KiB ring) one 8-wave
// work-group takes the CU.
constexpr int prefill_waves(int64_t D) { return D == 256 ? 8 : 4; }
constexpr int kPreIssuers = 4;  // waves 0-3 issue the DMA, one per SIMD
constexpr int kPreKeys = 32;
// Interleave of the pipelined prefill phase: softmax VALU instructions
// before the first QK MFMA, and after each QK MFMA.
#ifndef KVHOT_PRE_SCHED
#define KVHOT_PRE_SCHED 1
#endif
#ifndef KVHOT_PRE_VALU_LEAD
#define KVHOT_PRE_VALU_LEAD 8
#endif
#ifndef KVHOT_PRE_VALU_PER_MFMA
#define KVHOT_PRE_VALU_PER_MFMA 4
#endif

// A K (or V) tile in LDS: 32 key rows of 2*D bytes.  The 16-byte chunks of a
// row are XOR-swizzled (chunk lc of row r sits at lc ^ swz(r)), so the MFMA
// operand reads -- 16 rows at one logical chunk for K, one row at 16
// consecutive chunks for V -- fall in distinct banks of the 64.  A DMA
// instruction fills 64 consecutive chunks (1 KiB); each lane picks the global
// chunk that belongs at its position.
template <int D>
struct PreTile {
  static constexpr int CPR = D / 8;              // 16-byte chunks per key row
  static constexpr int RB = 2 * D;               // bytes per key row
  static constexpr int BYTES = kPreKeys * RB;    // bytes per K (or V) tile
  static constexpr int CHUNKS = kPreKeys * CPR;  // chunks per tile
  // DMA instructions per issuing wave (K or V): kPreIssuers waves issue a tile.
  static constexpr int NI = CHUNKS / (64 * kPreIssuers);
  static_assert(CHUNKS % (64 * kPreIssuers) == 0, "a tile splits evenly over the issuing waves");
  // 128-byte rows (D = 64) share a 256-byte bank line in pairs.
  __host__ __device__ static constexpr int swz(int r) { return D == 64 ? (r >> 1) & 7 : r & 15; }
  __host__ __device__ static constexpr int offset(int r, int lc) { return r * RB + 16 * (lc ^ swz(r)); }
};

// s_waitcnt vmcnt(N) alone (expcnt and lgkmcnt at their no-wait maximum).
template <int N>
__device__ inline void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (15 << 8) | ((N >> 4) << 14));
}

// Work-group barrier for LDS filled by DMA: the caller has waited for its own
// DMA (vmcnt); LDS reads are drained first so a slot can be refilled after.
// The empty asm statements keep the compiler from moving memory accesses
// across it (the s_barrier intrinsic alone does not order them).
__device__ inline void lds_barrier() {
  __builtin_amdgcn_s_waitcnt((15) | (7 << 4) | (0 << 8) | (3 << 14));  // lgkmcnt(0)
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// lds_barrier that also ends an instruction-scheduling region: nothing moves
// across it, so the half-steps of the prefill loop stay apart.
__device__ inline void half_barrier() {
  __builtin_amdgcn_sched_barrier(0);
  lds_barrier();
  __builtin_amdgcn_sched_barrier(0);
}

// One prefill work-group: launch-list unit bx (prefill units at sched), or
// without a launch list grid work-group (bx, by, bz).
template <class TT, int D, int NM>
__device__ __attribute__((always_inline)) inline void prefill_wg(const AttnArgs& a, const int4* sched, int bx, int by,
                                                                 int bz) {
  (void)by;
  using Tile = PreTile<D>;
  using WA = WaveAttn<TT, D, NM>;
  constexpr int PW = prefill_waves(D);
  // Ring slots, K tile then V tile.  Separate arrays: the compiler can tell
  // that reads of one slot do not alias the DMA into another, and so does
  // not wait for every DMA in flight before each LDS read.
  __shared__ __attribute__((aligned(16))) char slot0[2 * Tile::BYTES];
  __shared__ __attribute__((aligned(16))) char slot1[2 * Tile::BYTES];
  __shared__ __attribute__((aligned(16))) char slot2[2 * Tile::BYTES];
  __shared__ __attribute__((aligned(16))) char slot3[2 * Tile::BYTES];
  // Every call passes a constant slot, so after inlining each access names
  // one array.
  auto slot = [&](int S) -> char* {
    switch (S) {
      case 0: return slot0;
      case 1: return slot1;
      case 2: return slot2;
      default: return slot3;
    }
  };
  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63;
  const int QPW = 16 * NM / a.G;  // queries per wave
  // A unit is a query block of a prefill row (keys from 0, causal), or a
  // shared-prefix unit: the queries of consecutive decode rows (tokens
  // qt0 .. qt0 + nqg - 1, one per row) over keys [k0, kend_g) of the prefix
  // they share, read through `row`'s block table; every such key is visible
  // to every such query, and the normalised output of query i goes to the
  // split-K partial pbase + i * pstride instead of the output.
  int row, kvh, qblk = 0, k0 = 0, kend_g = 0, nqg = 0, off = 0, pbase = 0, pstride = 0;
  int64_t qs = 0;
  int q0g = 0;
  bool prefix = false;
  if (sched) {
    const int4 u = sched[2 * static_cast<int64_t>(bx)];
    const int4 u1 = sched[2 * static_cast<int64_t>(bx) + 1];
    row = u.x;
    kvh = u.y;
    prefix = __builtin_amdgcn_readfirstlane(u1.y) > 0;
    if (prefix) {
      k0 = u.z;
      kend_g = u.w;
      qs = u1.x;
      nqg = min(u1.y, QPW * PW);
      pbase = u1.z;
      pstride = u1.w;
    } else {
      qblk = u.z;
    }
  } else {
    row = bz;
    kvh = bx % a.Hkv;
    qblk = bx / a.Hkv;
  }
  row = __builtin_amdgcn_readfirstlane(row);
  kvh = __builtin_amdgcn_readfirstlane(kvh);
  qblk = __builtin_amdgcn_readfirstlane(qblk);
  if (row < 0 || kvh < 0 || kvh >= a.Hkv || qblk < 0) return;
  if (prefix) {
    k0 = __builtin_amdgcn_readfirstlane(k0);
    kend_g = __builtin_amdgcn_readfirstlane(kend_g);
    qs = __builtin_amdgcn_readfirstlane(static_cast<int>(qs));
    nqg = __builtin_amdgcn_readfirstlane(nqg);
    pbase = __builtin_amdgcn_readfirstlane(pbase);
    pstride = __builtin_amdgcn_readfirstlane(pstride);
    if (k0 < 0 || k0 % kPreKeys != 0 || kend_g <= k0 || kend_g > a.k_lens[row] || qs < 0 || pbase < 0 ||
        pstride <= 0 || static_cast<int64_t>(pbase) + static_cast<int64_t>(nqg - 1) * pstride >= a.num_partials)
      return;
    off = 1 << 29;  // past every key: the prefix is wholly visible
  } else {
    const int qlen = a.q_lens[row];
    if (qlen < 2) return;
    q0g = qblk * QPW * PW;
    if (q0g >= qlen) return;
    nqg = min(QPW * PW, qlen - q0g);
    off = a.q_offs[row];
    const int klen = a.k_lens[row];
    kend_g = max(a.causal ? min(klen, off + q0g + nqg) : klen, 0);
    qs = a.q_starts[row];
  }
  const bool causal = a.causal && !prefix;
  const int klen = prefix ? kend_g : a.k_lens[row];
  // This wave's queries and the keys they see.
  const int q0 = q0g + wave * QPW;
  const int nq = max(min(QPW, nqg - wave * QPW), 0);
  const int kend = nq > 0 ? max(causal ? min(klen, off + q0 + nq) : klen, 0) : 0;
  const int qpos_min = causal ? off + q0 : INT_MAX;

  // DMA: issuing wave w (the leading group), instruction i fills chunks
  // 64 (NI w + i) .. of a tile; all of a wave's chunks lie in the one 16-key
  // half hw.  Lane L's chunk is physical chunk pc of row pr; it loads logical
  // chunk pc ^ swz(pr) of that key.
  constexpr int NI = Tile::NI;
  const bool issuer = wave < kPreIssuers;
  const int hw = __builtin_amdgcn_readfirstlane(issuer ? (64 * NI * wave) / (16 * Tile::CPR) : 0);
  uint32_t koff[NI], voff[NI];
#pragma unroll
  for (int i = 0; i < NI; ++i) {
    const int p = 64 * (NI * (issuer ? wave : 0) + i) + lane;
    const int pr = p / Tile::CPR, pc = p % Tile::CPR;
    const int lc = pc ^ Tile::swz(pr);
    koff[i] = 2u * ((pr & 15) * static_cast<uint32_t>(a.k_st) + 8u * lc);
    voff[i] = 2u * ((pr & 15) * static_cast<uint32_t>(a.v_st) + 8u * lc);
  }
  const int bs = a.bs;
  const int32_t* btrow = a.bt + static_cast<int64_t>(row) * a.bt_stride;
  const int nb_row = static_cast<int>(min(static_cast<int64_t>((kend_g + bs - 1) / bs), a.bt_stride));
  const char* kbase = static_cast<const char*>(a.k) + 2 * static_cast<int64_t>(kvh) * a.k_sh;
  const char* vbase = static_cast<const char*>(a.v) + 2 * static_cast<int64_t>(kvh) * a.v_sh;
  // Byte strides; a block and the rows of a block fit 32 bits (checked on
  // the host: block strides below 2^31 bytes).
  const uint32_t ksb = 2u * static_cast<uint32_t>(a.k_sb), vsb = 2u * static_cast<uint32_t>(a.v_sb);
  const uint32_t kst = 2u * static_cast<uint32_t>(a.k_st), vst = 2u * static_cast<uint32_t>(a.v_st);
  const uint32_t nblocks = static_cast<uint32_t>(a.num_blocks);
  // Block ids come through scalar loads (constant address space): nblk is
  // the logical block holding this wave's half of the next tile to load,
  // nbo its first row there.  (A vector load here would make the compiler
  // wait for every DMA in flight before using it.  Staging the unit's ids in
  // LDS before the first DMA instead measured the same.)
  const __attribute__((address_space(4))) int32_t* btc =
      (const __attribute__((address_space(4))) int32_t*)btrow;
  auto bt_at = [&](int blk) -> int { return btc[min(blk, max(nb_row - 1, 0))]; };
  int nblk = (k0 + 16 * hw) / bs, nbo = (k0 + 16 * hw) % bs;

  // DMA of tile t (the next in order) into ring slot S.  The descriptor of
  // the half starts at its first key and covers only keys below kend_g: the
  // rows past it read as zeros.
  auto issue = [&](int S, int t) {
    const int nid = bt_at(nblk);
    const uint32_t b = min(static_cast<uint32_t>(max(nid, 0)), nblocks - 1);
    const int rows = min(max(kend_g - (k0 + kPreKeys * t + 16 * hw), 0), 16);
    const char* kb = kbase + (static_cast<uint64_t>(b) * ksb + static_cast<uint32_t>(nbo) * kst);
    const char* vb = vbase + (static_cast<uint64_t>(b) * vsb + static_cast<uint32_t>(nbo) * vst);
    const int nrk = __builtin_amdgcn_readfirstlane(rows * static_cast<int>(kst));
    const int nrv = __builtin_amdgcn_readfirstlane(rows * static_cast<int>(vst));
    // This half of tile t + 1 (32 keys on).
    if (bs == 16) {
      nblk += 2;
    } else {
      nbo += kPreKeys;
      if (nbo >= bs) {
        nbo -= bs;
        ++nblk;
      }
    }
    char* dst = slot(S) + 1024 * NI * wave;
    const rsrc_words_t kr = rsrc_words(kb, nrk), vr = rsrc_words(vb, nrv);
#pragma unroll
    for (int i = 0; i < NI; ++i) {
      dma16_asm(kr, dst + 1024 * i, koff[i]);
      dma16_asm(vr, dst + Tile::BYTES + 1024 * i, voff[i]);
    }
  };

  // One phase per tile, each ending in one work-group barrier (see the
  // loops below).  The issuing waves put tile t+LEAD in flight at the start
  // of phase t; tile t sits in slot t % 4, and the loop body is unrolled
  // four times so that every LDS access names a fixed slot.  (Two barriers
  // per tile, pinning the two waves of a SIMD half a tile apart, measured
  // 187.5 us against 182.6 for one, on the mixed workload's prefill rows
  // with 8-wave work-groups.)
  constexpr int PER_TILE = 2 * NI;  // DMA instructions per issuing wave and tile
  constexpr int LEAD = WA::NC <= 4 ? 3 : 2;
  const int ntiles = (kend_g - k0 + kPreKeys - 1) / kPreKeys;
  // Tiles [0, nfull) have no key masked for this wave; tiles from kend on
  // have no key it sees.
  const int nfull = ((causal ? min(kend, qpos_min + 1) : kend) - k0) / kPreKeys;
  // Prologue: tiles 0 .. LEAD-1, then Q; one wait for all of it.  (Q's loads
  // are the only vector loads the compiler knows of: waited for here, none
  // is pending inside the loop, so it adds no wait there that would also
  // drain the DMAs.)
  if (issuer && ntiles > 0) issue(0, 0);
  if (issuer && ntiles > 1) issue(1, 1);
  if (LEAD > 2 && issuer && ntiles > 2) issue(2, 2);
  WA wa;
  wa.setup(a, lane, kvh, qs, q0, nq, off);
  wait_vmcnt<0>();
  // Scores in log2 units are S * sl with sl > 0: a negative scale flips the
  // sign of Q (exact), a zero scale becomes a negligible positive one.
  float sl = a.scale_log2;
  if (sl < 0.f) {
#pragma unroll
    for (int s = 0; s < NM; ++s)
#pragma unroll
      for (int c = 0; c < WA::NC; ++c) wa.qf[s][c] ^= u32x4{0x80008000u, 0x80008000u, 0x80008000u, 0x80008000u};
    sl = -sl;
  }
  sl = fmaxf(sl, 1e-30f);
#pragma unroll
  for (int s = 0; s < NM; ++s) {
    wa.m[s] = -FLT_MAX;
    wa.thr[s] = -INFINITY;  // the first visible score moves m
  }
  half_barrier();

  constexpr bool kVAhead = WA::NC <= 4;
  if constexpr (kVAhead) {
    // head_dim 64 and 128, software-pipelined: phase t reads K(t+1) and
    // V^T(t), runs QK(t+1) while it forms P(t) from the scores QK(t) left in
    // scc one phase earlier, then PV(t).  The QK MFMAs and the softmax VALU
    // of one wave are independent, so they interleave (sched_group_barrier
    // below) instead of the softmax waiting for the QK results.  At its start
    // the issuing waves put tile t+3 in flight into the slot of tile t-1
    // (its K read in phase t-2, its V^T in phase t-1, both before the last
    // barrier); before the barrier an issuing wave waits for its part of
    // tile t+2, whose K phase t+1 reads: its DMAs complete in issue order,
    // and the only vector memory operations in the loop are these DMAs, so
    // vmcnt <= PER_TILE (tile t+3 alone still in flight) or 0 means tile
    // t+2's PER_TILE instructions have landed.
    f32x4 scc[NM][2];  // raw S of tile t
    if (ntiles > 0) {
      u32x4 kop[2][WA::NC];
      wa.template k_operands<Tile>(slot(0), 0, kop[0]);
      wa.template k_operands<Tile>(slot(0), 1, kop[1]);
      wa.qk_ops(kop[0], 0, scc);
      wa.qk_ops(kop[1], 1, scc);
    }
    // Every wave runs every tile of the unit: a tile wholly past a wave's
    // causal limit is masked like the diagonal one (P = 0), which keeps the
    // phase one straight block.  Such tiles are at most one per wave, the
    // waves of a work-group being 16*NM/G queries apart.
    auto phase = [&](auto S_, int t) {
      constexpr int S = decltype(S_)::value;
      if (issuer && t + LEAD < ntiles) issue((S + LEAD) & 3, t + LEAD);
      const int ts = k0 + kPreKeys * t;
      if (t >= nfull) wa.mask_tile(scc, ts, kend);
      const char* vt = slot(S) + Tile::BYTES;
      const char* kn = slot((S + 1) & 3);
      u32x4 va[WA::VB];
      u32x4 pb[NM];
      f32x4 scn[NM][2];
      // References first (rare move, before the block), then one block:
      // K(t+1) and V^T(t) reads, QK(t+1) and P(t).
      float mloc[NM], ls[NM];
      if (__builtin_amdgcn_ballot_w64(wa.lazy_check(scc, mloc)) != 0) wa.move_refs(sl, mloc);
      u32x4 kop[2][WA::NC];
      wa.template k_operands<Tile>(kn, 0, kop[0]);
      wa.template k_operands<Tile>(kn, 1, kop[1]);
      wa.template read_vt<Tile>(vt, 0, va);
      wa.qk_ops(kop[0], 0, scn);
      wa.qk_ops(kop[1], 1, scn);
      wa.probs(sl, scc, pb, ls);
#if KVHOT_PRE_SCHED
      // The LDS reads first, then each QK MFMA followed by a few softmax
      // VALU instructions.
      __builtin_amdgcn_sched_group_barrier(0x100, 2 * WA::NC, 0);
      __builtin_amdgcn_sched_group_barrier(0x002, KVHOT_PRE_VALU_LEAD, 0);
#pragma unroll
      for (int i = 0; i < 4 * NM * WA::NC; ++i) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        if (i < 2 * WA::VB) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
        __builtin_amdgcn_sched_group_barrier(0x002, KVHOT_PRE_VALU_PER_MFMA, 0);
      }
#endif
#pragma unroll
      for (int s2 = 0; s2 < NM; ++s2) {
        wa.l[s2] += ls[s2];
        scc[s2][0] = scn[s2][0];
        scc[s2][1] = scn[s2][1];
      }
      wa.template pv_lds<Tile>(vt, va, pb);
      if (issuer && t + 2 < ntiles) {
        // This wave's vector memory operations in flight, oldest first: its
        // PER_TILE DMAs of tile t+2 (issued in phase t-1), then, when it
        // exists, its PER_TILE of tile t+3 (issued in this phase); nothing
        // else (Q was waited for in the prologue).  Tile t+2 has landed once
        // at most the newer PER_TILE remain.
        if (t + 3 < ntiles) wait_vmcnt<PER_TILE>();
        else wait_vmcnt<0>();
      }
      half_barrier();
    };
    // The last tile: softmax and PV only (no tile after it, no barrier).
    auto last = [&](auto S_, int t) {
      constexpr int S = decltype(S_)::value;
      const int ts = k0 + kPreKeys * t;
      if (t >= nfull) wa.mask_tile(scc, ts, kend);
      const char* vt = slot(S) + Tile::BYTES;
      u32x4 va[WA::VB];
      u32x4 pb[NM];
      wa.template read_vt<Tile>(vt, 0, va);
      wa.softmax_tile(sl, scc, false, ts, kend, pb);
      wa.template pv_lds<Tile>(vt, va, pb);
    };
    const int nlast = ntiles - 1;
    for (int t = 0; t < nlast; t += 4) {
      phase(std::integral_constant<int, 0>{}, t);
      if (t + 1 >= nlast) break;
      phase(std::integral_constant<int, 1>{}, t + 1);
      if (t + 2 >= nlast) break;
      phase(std::integral_constant<int, 2>{}, t + 2);
      if (t + 3 >= nlast) break;
      phase(std::integral_constant<int, 3>{}, t + 3);
    }
    switch (ntiles > 0 ? nlast & 3 : -1) {
      case -1: break;  // no key: O = 0
      case 0: last(std::integral_constant<int, 0>{}, nlast); break;
      case 1: last(std::integral_constant<int, 1>{}, nlast); break;
      case 2: last(std::integral_constant<int, 2>{}, nlast); break;
      default: last(std::integral_constant<int, 3>{}, nlast); break;
    }
  } else {
    // head_dim 256 (K operands in halves, V^T read in the phase of its PV):
    // phase t issues tile t+2 into the slot of tile t-2, reads K(t) half by
    // half around PV(t-1), runs QK(t) and forms P(t); before the barrier an
    // issuing wave waits for its part of tile t+1 (vmcnt <= PER_TILE while
    // tile t+2 is in flight).
    u32x4 pb[NM];      // P of the previous tile, for its PV
    u32x4 va[WA::VB];  // its V^T operands
    bool pv_due = false;
    auto step = [&](auto S_, int t) {
      constexpr int S = decltype(S_)::value;
      if (issuer && t + LEAD < ntiles) issue((S + LEAD) & 3, t + LEAD);
      const int ts = k0 + kPreKeys * t;
      const bool live = t < ntiles && ts < kend;
      f32x4 sc[NM][2];
      u32x4 kh[WA::NC];
      if (live) wa.template k_operands<Tile>(slot(S), 0, kh);
      if (pv_due) {
        wa.template read_vt<Tile>(slot((S + 3) & 3) + Tile::BYTES, 0, va);
        wa.template pv_lds<Tile>(slot((S + 3) & 3) + Tile::BYTES, va, pb);
      }
      if (live) {
        wa.qk_ops(kh, 0, sc);
        wa.template k_operands<Tile>(slot(S), 1, kh);
        wa.qk_ops(kh, 1, sc);
        wa.softmax_tile(sl, sc, t >= nfull, ts, kend, pb);
      }
      pv_due = live;
      if (issuer && t + 1 < ntiles) {
        // In flight, oldest first: this wave's PER_TILE DMAs of tile t+1
        // (issued in phase t-1), then its PER_TILE of tile t+2 (this phase)
        // when it exists; tile t+1 has landed once at most PER_TILE remain.
        if (t + 2 < ntiles) wait_vmcnt<PER_TILE>();
        else wait_vmcnt<0>();
      }
      half_barrier();
    };
    for (int t = 0; t <= ntiles; t += 4) {
      step(std::integral_constant<int, 0>{}, t);
      if (t + 1 > ntiles) break;
      step(std::integral_constant<int, 1>{}, t + 1);
      if (t + 2 > ntiles) break;
      step(std::integral_constant<int, 2>{}, t + 2);
      if (t + 3 > ntiles) break;
      step(std::integral_constant<int, 3>{}, t + 3);
    }
  }
  float ltot[NM];
  wa.row_sums(ltot);
#pragma unroll
  for (int s = 0; s < NM; ++s) {
    if (!wa.mval[s]) continue;
    if (prefix)
      wa.store_partial_blocks(a, s, static_cast<int64_t>(pbase) + static_cast<int64_t>(q0 + wa.row_query(a, s)) * pstride,
                              wa.row_head(a, s) - kvh * a.G, ltot[s]);
    else
      wa.store_final_blocks(a, s, qs + q0 + wa.row_query(a, s), ltot[s]);
  }
}

// Two waves per SIMD at every head_dim (at most 256 VGPRs a wave).
template <class TT, int D, int NM>
__global__ void __launch_bounds__(64 * prefill_waves(D)) __attribute__((amdgpu_waves_per_eu(2)))
attn_prefill_kernel(const AttnArgs a) {
  prefill_wg<TT, D, NM>(a, a.sched, blockIdx.x, blockIdx.y, blockIdx.z);
}

// ----------------------------------------------------------- VALU kernel --
// One wave per (row, query, query head).  Lanes take 64 keys at a time for the
// scores; for P.V each lane owns head_dim values lane, lane+64, ...
constexpr int kGenericMaxD = 256;

template <class TT>
__global__ void __launch_bounds__(64)
attn_generic_kernel(const AttnArgs a) {
  using st = typename TT::storage;
  const int lane = threadIdx.x;
  const int h = blockIdx.x;
  const int qi = blockIdx.y;
  const int row = blockIdx.z;
  const int qlen = a.q_lens[row];
  if (qi >= qlen) return;
  if (static_cast<int64_t>(a.q_starts[row]) + qi >= a.total_q) return;
  const int D = a.D;
  const int kvh = h / a.G;
  const int64_t t = static_cast<int64_t>(a.q_starts[row]) + qi;
  const int klen = a.k_lens[row];
  const int qpos = a.q_offs[row] + qi;
  int kend = a.causal ? min(klen, qpos + 1) : klen;
  kend = max(kend, 0);
  const int bs = a.bs;
  const int32_t* btrow = a.bt + static_cast<int64_t>(row) * a.bt_stride;
  const int64_t max_tok = a.bt_stride * bs;
  if (kend > max_tok) kend = static_cast<int>(max_tok);

  __shared__ float qsh[kGenericMaxD];
  __shared__ float psh[64];
  __shared__ int64_t vsh[64];
  const st* qp = static_cast<const st*>(a.q) + t * a.q_st + static_cast<int64_t>(h) * a.q_sh;
  for (int d = lane; d < D; d += 64) qsh[d] = TT::to_float(qp[d]);
  __syncthreads();

  const st* kbase = static_cast<const st*>(a.k) + static_cast<int64_t>(kvh) * a.k_sh;
  const st* vbase = static_cast<const st*>(a.v) + static_cast<int64_t>(kvh) * a.v_sh;
  float m = -INFINITY, l = 0.f;
  float acc[kGenericMaxD / 64];
#pragma unroll
  for (int k = 0; k < kGenericMaxD / 64; ++k) acc[k] = 0.f;

  for (int ts = 0; ts < kend; ts += 64) {
    const int tok = ts + lane;
    const bool valid = tok < kend;
    float x = -INFINITY;
    if (valid) {
      int64_t id = btrow[tok / bs];
      id = id < 0 ? 0 : (id >= a.num_blocks ? a.num_blocks - 1 : id);
      const int bo = tok % bs;
      const st* kp = kbase + id * a.k_sb + static_cast<int64_t>(bo) * a.k_st;
      float dot = 0.f;
      for (int d = 0; d < D; ++d) dot = fmaf(qsh[d], TT::to_float(kp[d]), dot);
      x = dot * a.scale_log2;
      vsh[lane] = id * a.v_sb + static_cast<int64_t>(bo) * a.v_st;
    }
    const float mnew = fmaxf(m, wave_max(x));
    const float muse = (mnew == -INFINITY) ? 0.f : mnew;
    const float corr = exp2f(m - muse);
    const float pv = valid ? exp2f(x - muse) : 0.f;
    l = l * corr + wave_sum(pv);
    m = mnew;
    psh[lane] = pv;
    __syncthreads();
#pragma unroll
    for (int k = 0; k < kGenericMaxD / 64; ++k) acc[k] *= corr;
    const int cnt = min(64, kend - ts);
    for (int j = 0; j < cnt; ++j) {
      const float pj = psh[j];
      const st* vp = vbase + vsh[j];
#pragma unroll
      for (int k = 0; k < kGenericMaxD / 64; ++k) {
        const int d = lane + 64 * k;
        if (d < D) acc[k] = fmaf(pj, TT::to_float(vp[d]), acc[k]);
      }
    }
    __syncthreads();
  }
  const float inv = l > 0.f ? 1.f / l : 0.f;
  st* op = static_cast<st*>(a.o) + t * a.o_st + static_cast<int64_t>(h) * a.o_sh;
#pragma unroll
  for (int k = 0; k < kGenericMaxD / 64; ++k) {
    const int d = lane + 64 * k;
    if (d < D) op[d] = TT::from_float(acc[k] * inv);
  }
  if (a.lse && lane == 0)
    a.lse[t * a.l_st + static_cast<int64_t>(h) * a.l_sh] =
        l > 0.f ? (m + log2f(l)) * kLn2 : -INFINITY;
}


// ------------------------------------------------------------------ host --

// LDS of a decode work-group: 64 KiB, or up to the 160 KiB of a gfx950 CU when
// one slot per wave needs more (query groups of 16 heads at head_dim 128, 8 or
// more at 256; 8 waves then fit at every head_dim and group size).
constexpr int64_t kMaxLdsBytes = 64 * 1024;
constexpr int64_t kCuLdsBytes = 160 * 1024;
#ifndef KVHOT_MAX_DECODE_WAVES
#define KVHOT_MAX_DECODE_WAVES 8
#endif

// Waves per decode work-group: 8 (KVHOT_MAX_DECODE_WAVES=16 builds a 16-wave
// variant for head_dim <= 128 when one slot per wave fits in 64 KiB of LDS).
// At head_dim 128 the 8-wave kernel takes 135 VGPRs, so a CU holds one such
// work-group: with non-temporal K/V loads, 8 waves per CU streamed faster
// than 16 (measured on MI355X, one box, 64-row GQA workload: 52.2 against
// 54.1 us per call; 55.7 us with 16 waves and cached loads).
static int decode_waves(int64_t G, int64_t D) {
  if (KVHOT_MAX_DECODE_WAVES >= 16 && D <= 128 && decode_lds_words(16, 16, G, D) * 4 <= kMaxLdsBytes)
    return 16;
  return 8;
}

// LDS bytes a decode work-group of P ranges may use (see kMaxLdsBytes).
static int64_t decode_lds_limit(int P, int64_t G, int64_t D) {
  return decode_lds_words(P, P, G, D) * 4 <= kMaxLdsBytes ? kMaxLdsBytes : kCuLdsBytes;
}

// LDS slots of a decode work-group of W waves and P ranges: one per range
// plus a pool of up to 3W more for waves that move on to ranges another wave
// entered first, as LDS allows; 0 when one slot per range does not fit.  (A
// wave that finds the pool empty stops taking slices of other segments.
// With many short segments per work-group -- 256 rows' private tails after
// a shared prefix -- a pool of 3W rather than W took the call from 75.1 to
// 74.4 us, one box; P + 3W <= 64 keeps the merge's 64-lane ballot over the
// slots.)
static int decode_slots(int W, int P, int64_t G, int64_t D) {
  const int64_t limit = decode_lds_limit(P, G, D);
  const int64_t base = decode_lds_words(P, P, G, D);
  if (base * 4 > limit) return 0;
  const int64_t spare = limit / 4 - base;
  const int64_t per_slot = G * D + G + 4;
  return P + static_cast<int>(std::max<int64_t>(0, std::min<int64_t>(3 * W, spare / per_slot)));
}

// Range descriptors per decode work-group of W waves.  A launch list of
// fixed partitions (partition_tokens > 0) gives a work-group up to
// kFixedRangesPerWave ranges per wave, one partition each: a wave starts on
// one and, when it is used up, enters the range with the most slices left,
// parking each partition's state in that range's own slot; so a device-full
// of work-groups takes a long-context call in one round, where one
// partition per wave took four (16 rows x 32,768 tokens, 512-token
// partitions: 1,024 work-groups of 8 one-partition waves).  Other launch
// lists, the grid path and two-slice waves keep one range per wave.
constexpr int kFixedRangesPerWave = 4;
static int decode_ranges(int W, int64_t G, int64_t D, bool fixed_partitions) {
  const int P = kFixedRangesPerWave * W;
  if (!fixed_partitions || KVHOT_DECODE_DEPTH >= 2 || P + 3 * W > 64) return W;
  if (decode_slots(W, P, G, D) < P) return W;
  return P;
}

// Bytes of one split-K partial: the normalised O and LSE of G query heads.
static int64_t partial_bytes(int64_t G, int64_t D) { return G * (D + 1) * 4; }

struct Plan {
  bool mfma = false;     // the MFMA kernels take this shape
  bool grid_ok = false;  // ... also without a schedule (partition count fits the grid)
  int waves = 0;         // waves per decode work-group
  int part_tokens = 0;   // keys per decode partition (no schedule)
  int max_parts = 1;
  int64_t partials = 0;  // split-K partials without a schedule
  int64_t workspace_bytes(int64_t G, int64_t D) const { return partials * partial_bytes(G, D); }
};

static bool mfma_shape_ok(int64_t Hq, int64_t Hkv, int64_t D, int64_t bs, int dtype) {
  if (dtype != KVHOT_BF16 && dtype != KVHOT_F16) return false;
  if (D != 64 && D != 128 && D != 256) return false;
  if (bs % 16 != 0) return false;
  const int64_t G = Hq / Hkv;
  return G == 1 || G == 2 || G == 4 || G == 8 || G == 16;
}

// Without a schedule, decode rows are cut into partitions of part_tokens keys
// (0: W * KVHOT_SLICES_PER_WAVE slices, so no wave walks more than that many)
// and the grid enumerates (head group, partition, row).
static Plan make_plan(int64_t rows, int64_t max_q, int64_t max_k, int64_t Hq,
                      int64_t Hkv, int64_t D, int64_t bs, int64_t part_tokens,
                      int dtype) {
  Plan pl;
  pl.mfma = mfma_shape_ok(Hq, Hkv, D, bs, dtype);
  if (!pl.mfma || max_q < 1) return pl;
  pl.waves = decode_waves(Hq / Hkv, D);
  pl.part_tokens = part_tokens > 0 ? static_cast<int>(part_tokens)
                                   : 16 * pl.waves * KVHOT_SLICES_PER_WAVE;
  const int64_t parts = std::max<int64_t>((max_k + pl.part_tokens - 1) / pl.part_tokens, 1);
  if (parts > 65535) return pl;
  pl.grid_ok = true;
  pl.max_parts = static_cast<int>(parts);
  if (pl.max_parts > 1) pl.partials = rows * Hkv * pl.max_parts;
  return pl;
}

// 16-row tiles of (query, head) pairs per prefill wave: O^T takes 64 VGPRs
// and Q 32 at every head_dim, so two waves fit on a SIMD.
#ifndef KVHOT_PRE_NM128
#define KVHOT_PRE_NM128 2
#endif
constexpr int prefill_nm(int64_t D) { return D == 64 ? 4 : (D == 128 ? KVHOT_PRE_NM128 : 1); }

// Decode work-groups the current device holds at once, times their waves
// (one work-group on each of 256 CUs when no device can be queried).
template <class TT, int D, int W>
static int decode_groups_per_cu(int64_t G) {
  int n = 0;
  const size_t lds = static_cast<size_t>(decode_lds_words(W, decode_slots(W, W, G, D), G, D) * 4);
  if ((lds > kMaxLdsBytes &&
       hipFuncSetAttribute(reinterpret_cast<const void*>(&attn_decode_kernel<TT, D, W>),
                           hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(lds)) != hipSuccess) ||
      hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, attn_decode_kernel<TT, D, W>, 64 * W, lds) !=
          hipSuccess)
    n = 0;
  return n;
}

template <class TT>
static int decode_groups_per_cu(int64_t D, int W, int64_t G) {
#if KVHOT_MAX_DECODE_WAVES >= 16
  if (W == 16) {
    if (D == 64) return decode_groups_per_cu<TT, 64, 16>(G);
    return decode_groups_per_cu<TT, 128, 16>(G);
  }
#else
  (void)W;
#endif
  if (D == 64) return decode_groups_per_cu<TT, 64, 8>(G);
  if (D == 128) return decode_groups_per_cu<TT, 128, 8>(G);
  return decode_groups_per_cu<TT, 256, 8>(G);
}

static int64_t resident_decode_waves(int dtype, int64_t D, int W, int64_t G) {
  int dev = 0, cus = 0;
  int per = 0;
  if (hipGetDevice(&dev) == hipSuccess &&
      hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess)
    per = dtype == KVHOT_BF16 ? decode_groups_per_cu<BF16>(D, W, G)
                              : decode_groups_per_cu<F16>(D, W, G);
  if (cus <= 0 || per <= 0) {
    (void)hipGetLastError();
    return 256 * static_cast<int64_t>(W);
  }
  return static_cast<int64_t>(cus) * per * W;
}

struct Piece {
  int row, kvh, s0, s1, part, seg;
};

// Minimum slices per decode work-group: below it, a split costs more (partial
// stores and a merge) than the parallelism gains.
constexpr int64_t kMinGroupSlicesPerWave = 2;
// Split pieces shorter than this are not cut off a segment.
constexpr int64_t kMinPieceSlices = 4;
// Cost model for choosing a plan that cuts no segment (and so needs no merge
// launch): the merge launch and its gap cost about kMergeLaunchUs, and a
// work-group streams K/V at about kDecodeRateGBs / (work-groups) GB/s
// (measured on MI355X: 5.5-6 TB/s in the decode kernel's steady state).
constexpr double kMergeLaunchUs = 5.0;
constexpr double kDecodeRateGBs = 5500.0;
// Kv heads stream at different rates: which HBM channels a head's rows hit
// follows from the row's byte offset inside a token's [Hkv, D] row, and on
// MI355X two of eight 256-byte offsets read about 16% slower in every XCD
// (shifting the pool by 256 bytes moves the slow heads along; the slow pair
// is h and h + 4, and which pair it is changes from one process to the next:
// heads 1 and 5 at 2.66 against 3.22 slices per us in one, 3 and 7 in
// another).  A work-group
// of one head's segments then ends late or early with its head; one that
// holds a mix of heads averages the rates (its waves share the slices).  So
// the packing below places a segment, among the up to kMixCandidates
// work-groups within kMixSlack slices of the least loaded, in the one that
// holds the fewest segments of its kv head.
constexpr int kMixCandidates = 8;
constexpr int64_t kMixSlack = 2;

// Decode launch list.  Work-groups of one device-full are given equal numbers
// of 16-token slices (inside a work-group the waves balance themselves by
// claiming slices, so only the per-work-group total matters): the (row, kv
// head) segments are laid end to end and cut every `target` slices, a
// segment that straddles a cut becoming parts in several work-groups (joined
// by attn_merge_kernel).  A work-group holds at most W pieces.  Its waves are
// shared among its pieces in proportion to their slices, and each wave's
// starting range is an even share of its piece.  With given_pt > 0 segments
// are first cut at multiples of given_pt keys and those partitions are never
// split further.  Otherwise, when that plan cuts some segment, the uncut
// alternative is tried too: whole segments, longest first, each to the
// least-loaded work-group with a free wave (LPT).  It is taken when its
// longest work-group holds fewer extra slices than a merge launch costs
// (slice_bytes per slice at the per-work-group rate).
//
// Per wave two int4: (row | parts << 16, kvh | part << 16, first slice, end
// slice) and (query token, visible keys, physical block of the first slice
// or -1, partial index).  Per split segment two int4: (query token, kv head,
// parts, first partial index) and zeros.  Returns false when a count does not
// fit its 16-bit field.
// Shared prefixes: runs of at least kMinPrefixRows consecutive decode rows
// (one query each, consecutive query tokens) whose block tables start with
// the same blocks, over at least kMinPrefixKeys keys that precede every
// row's own last key.  Such a run's prefix keys are attended once for all its
// queries (prefill-kernel units, cut into key splits of at least
// kMinSplitKeys), and each row's decode segment covers only its own keys.
constexpr int64_t kMinPrefixRows = 4;
constexpr int64_t kMinPrefixKeys = 256;
constexpr int64_t kMinSplitKeys = 128;

struct PrefixGroup {
  int64_t r0, nrows, keys;  // rows [r0, r0 + nrows) share keys [0, keys)
};

// kend[r]: visible keys of decode row r (-1 for other rows).
static std::vector<PrefixGroup> find_prefix_groups(const int32_t* q_starts, const int32_t* bt, int64_t bt_stride,
                                                   int64_t bs, int64_t rows, const std::vector<int64_t>& kend) {
  std::vector<PrefixGroup> out;
  for (int64_t r = 0; r < rows;) {
    if (kend[r] < 1 || !bt) {
      ++r;
      continue;
    }
    // Blocks wholly before row r's last key.
    int64_t lcp = std::min<int64_t>(bt_stride, (kend[r] - 1) / bs);
    int64_t e = r + 1;
    while (e < rows && kend[e] >= 1 && q_starts[e] == q_starts[e - 1] + 1) {
      const int64_t lim = std::min<int64_t>(lcp, (kend[e] - 1) / bs);
      int64_t l = 0;
      while (l < lim && bt[r * bt_stride + l] == bt[e * bt_stride + l]) ++l;
      if (l * bs < kMinPrefixKeys) break;
      // n rows sharing lcp blocks read them once instead of n times.  A row
      // that would shorten the prefix joins a group that is already large
      // enough only if the group then saves more block reads.
      const int64_t n = e - r;
      if (l < lcp && n >= kMinPrefixRows && n * l <= (n - 1) * lcp) break;
      lcp = l;
      ++e;
    }
    const int64_t keys = lcp * bs / kPreKeys * kPreKeys;
    if (e - r >= kMinPrefixRows && keys >= kMinPrefixKeys) {
      out.push_back(PrefixGroup{r, e - r, keys});
      r = e;
    } else {
      ++r;
    }
  }
  return out;
}

static bool plan_decode(const int32_t* q_lens, const int32_t* k_lens, const int32_t* q_offs,
                        const int32_t* q_starts, const int32_t* bt, int64_t bt_stride, int64_t bs,
                        int64_t rows, int64_t Hkv, bool causal, int W, int ranges, int64_t groups,
                        int64_t given_pt, int64_t slice_bytes, int64_t prefix_queries, std::vector<int4>& dec,
                        std::vector<int4>& mrg, std::vector<int4>& pfx, int64_t& partials) {
  dec.clear();
  mrg.clear();
  pfx.clear();
  partials = 0;
  std::vector<int64_t> kend(rows, -1);
  for (int64_t r = 0; r < rows; ++r) {
    if (q_lens[r] != 1) continue;
    const int64_t klen = k_lens[r], off = q_offs[r];
    kend[r] = std::max<int64_t>(causal ? std::min(klen, off + 1) : klen, 0);
  }
  // Shared prefixes (none under fixed partitions): the rows' decode segments
  // start after the prefix and fold in the ks partials of the prefix's key
  // splits (kPrefixFold), which an earlier launch writes.
  std::vector<PrefixGroup> pgroups;
  if (given_pt == 0 && prefix_queries > 0) pgroups = find_prefix_groups(q_starts, bt, bt_stride, bs, rows, kend);
  std::vector<int64_t> pfx_sl(rows, 0), pfx_splits(rows, 0);
  for (const PrefixGroup& pg : pgroups) {
    const int64_t qblocks = (pg.nrows + prefix_queries - 1) / prefix_queries;
    // Key splits for a device-fill of prefix work-groups (a CU holds two
    // 4-wave prefill work-groups where it holds one decode work-group): on
    // 256 rows sharing 1024 keys (D=128, G=4), 512 units (8 splits) took
    // 74.7 us per call against 76.2 with 256 and 78.2 with 128 (one box):
    // shorter units outweigh the more fp32 partials to write and fold.
    const int64_t units = std::max<int64_t>(2 * groups, 1);
    const int64_t want = (units + qblocks * Hkv - 1) / (qblocks * Hkv);
    const int64_t ks = std::max<int64_t>(1, std::min<int64_t>(want, pg.keys / kMinSplitKeys));
    for (int64_t r = pg.r0; r < pg.r0 + pg.nrows; ++r) {
      pfx_sl[r] = pg.keys / 16;
      pfx_splits[r] = ks;
    }
  }
  int64_t total = 0;
  for (int64_t r = 0; r < rows; ++r)
    if (kend[r] >= 0) total += ((kend[r] + 15) / 16 - pfx_sl[r]) * Hkv;
  const int64_t target = std::max<int64_t>((total + std::max<int64_t>(groups, 1) - 1) / std::max<int64_t>(groups, 1),
                                           kMinGroupSlicesPerWave * W);
  const int64_t slack = std::max<int64_t>(2, target / 32);

  std::vector<std::vector<Piece>> wgs;
  std::vector<Piece> cur;
  int64_t load = 0;
  auto close = [&]() {
    if (!cur.empty()) wgs.push_back(cur);
    cur.clear();
    load = 0;
  };
  std::vector<int> seg_parts;  // parts per segment (row, kv head)
  std::vector<int> seg_row, seg_kvh;
  std::vector<int64_t> seg_start(rows, -1);  // first segment of each decode row
  // Adds slices [s, s + rem) of segment seg (row r, kv head h) to the open
  // work-groups: whole when it is a fixed partition p, else cut at the
  // work-group loads.
  // Pieces per work-group: one per wave, or with fixed partitions one per
  // range (decode_ranges).
  const int cap = given_pt > 0 ? ranges : W;
  auto place = [&](int seg, int64_t r, int64_t h, int64_t s, int64_t rem, int64_t p, bool splittable) {
    for (;;) {
      if (static_cast<int>(cur.size()) == cap) close();
      const int64_t space = target - load;
      if (rem <= space + slack || (!splittable && cur.empty())) {
        const int part = splittable ? seg_parts[seg]++ : static_cast<int>(p);
        cur.push_back(Piece{static_cast<int>(r), static_cast<int>(h), static_cast<int>(s),
                            static_cast<int>(s + rem), part, seg});
        load += rem;
        return;
      }
      if (!splittable || space < kMinPieceSlices) {
        close();
        continue;
      }
      int64_t take = space;
      if (rem - take < kMinPieceSlices) take = rem - kMinPieceSlices;
      cur.push_back(Piece{static_cast<int>(r), static_cast<int>(h), static_cast<int>(s),
                          static_cast<int>(s + take), seg_parts[seg]++, seg});
      s += take;
      rem -= take;
      close();
    }
  };
  const int64_t pt_sl = given_pt > 0 ? given_pt / 16 : 0;
  for (int64_t r = 0; r < rows; ++r) {
    if (kend[r] < 0) continue;
    const int64_t n = (kend[r] + 15) / 16;
    const int seg0 = static_cast<int>(seg_parts.size());
    seg_start[r] = seg0;
    for (int64_t h = 0; h < Hkv; ++h) {
      seg_parts.push_back(0);
      seg_row.push_back(static_cast<int>(r));
      seg_kvh.push_back(static_cast<int>(h));
    }
    if (pfx_splits[r] > 0) {
      // The row's own keys after the shared prefix.  Cut like any other
      // segment: a segment left whole folds the prefix's partials in itself
      // (kPrefixFold); the parts of a cut one meet them in its merge unit.
      for (int64_t h = 0; h < Hkv; ++h) place(seg0 + static_cast<int>(h), r, h, pfx_sl[r], n - pfx_sl[r], 0, true);
    } else if (pt_sl > 0) {
      // Fixed partitions, partition-major over the row's kv heads: a
      // work-group's run of partitions spans the heads, whose streaming
      // rates differ (see kMixCandidates).
      const int64_t natoms = std::max<int64_t>((n + pt_sl - 1) / pt_sl, 1);
      for (int64_t p = 0; p < natoms; ++p) {
        const int64_t s = p * pt_sl;
        for (int64_t h = 0; h < Hkv; ++h) place(seg0 + static_cast<int>(h), r, h, s, std::min(n, s + pt_sl) - s, p, false);
      }
      for (int64_t h = 0; h < Hkv; ++h) seg_parts[seg0 + h] = static_cast<int>(natoms);
    } else {
      for (int64_t h = 0; h < Hkv; ++h) place(seg0 + static_cast<int>(h), r, h, 0, n, 0, true);
    }
  }
  close();

  // Uncut plan: whole segments, longest first, onto the least loaded of
  // `groups` work-groups.  Taken when the cut plan cut a segment and the
  // uncut one is within a merge launch of balanced, and when segments that
  // fold shared-prefix partials are in the plan and nothing was cut (its
  // packing mixes kv heads; see kMixCandidates).  On the 64-row GQA decode
  // workload it leaves work-groups at 118-140 slices against an even 131, and
  // no packing of whole segments does better there (best-fit decreasing under
  // a cap and a simulated-annealing search over moves and swaps both stop at
  // 140).  Measured and not kept: listing the fullest work-groups first (no
  // change there, +14 us on the mixed batch), and idling waves of the lighter
  // work-groups in proportion (no change: a CU's rate did not follow its
  // waves in flight).
  bool any_cut = false, any_fold = false;
  for (size_t sg = 0; sg < seg_parts.size(); ++sg) {
    any_cut = any_cut || seg_parts[sg] > 1;
    any_fold = any_fold || pfx_splits[seg_row[sg]] > 0;
  }
  if (given_pt == 0 && (any_cut || any_fold)) {
    const int nseg = static_cast<int>(seg_parts.size());
    std::vector<int64_t> n(nseg);
    std::vector<int> order(nseg);
    for (int sg = 0; sg < nseg; ++sg) {
      n[sg] = (kend[seg_row[sg]] + 15) / 16 - pfx_sl[seg_row[sg]];
      order[sg] = sg;
    }
    std::stable_sort(order.begin(), order.end(), [&](int x, int y) { return n[x] > n[y]; });
    const int64_t ng = std::max<int64_t>(std::max<int64_t>(groups, 1), (nseg + W - 1) / W);
    // Min-heap of (slices, work-group); a work-group leaves it when full.
    std::vector<std::pair<int64_t, int64_t>> heap;
    heap.reserve(ng);
    for (int64_t g2 = 0; g2 < ng; ++g2) heap.emplace_back(0, g2);
    std::vector<std::vector<Piece>> lpt(ng);
    std::vector<int> held(static_cast<size_t>(ng * Hkv), 0);  // segments of each kv head per work-group
    std::vector<std::pair<int64_t, int64_t>> cand;
    int64_t lmax = 0;
    for (int sg : order) {
      const int h = seg_kvh[sg];
      cand.clear();
      std::pop_heap(heap.begin(), heap.end(), std::greater<>());
      cand.push_back(heap.back());
      heap.pop_back();
      while (static_cast<int>(cand.size()) < kMixCandidates && !heap.empty() &&
             heap.front().first <= cand[0].first + kMixSlack) {
        std::pop_heap(heap.begin(), heap.end(), std::greater<>());
        cand.push_back(heap.back());
        heap.pop_back();
      }
      size_t c = 0;
      for (size_t k = 1; k < cand.size(); ++k)
        if (held[cand[k].second * Hkv + h] < held[cand[c].second * Hkv + h]) c = k;
      for (size_t k = 0; k < cand.size(); ++k) {
        if (k == c) continue;
        heap.push_back(cand[k]);
        std::push_heap(heap.begin(), heap.end(), std::greater<>());
      }
      auto [ld, g2] = cand[c];
      const int64_t s0 = pfx_sl[seg_row[sg]];
      lpt[g2].push_back(Piece{seg_row[sg], seg_kvh[sg], static_cast<int>(s0), static_cast<int>(s0 + n[sg]), 0, sg});
      ++held[g2 * Hkv + h];
      ld += n[sg];
      lmax = std::max(lmax, ld);
      if (static_cast<int>(lpt[g2].size()) < W) {
        heap.push_back({ld, g2});
        std::push_heap(heap.begin(), heap.end(), std::greater<>());
      }
    }
    const double slice_us = static_cast<double>(slice_bytes) * ng / (kDecodeRateGBs * 1e3);
    if (!any_cut || static_cast<double>(lmax - target) * slice_us <= kMergeLaunchUs) {
      wgs.clear();
      for (auto& g2 : lpt)
        if (!g2.empty()) wgs.push_back(std::move(g2));
      std::fill(seg_parts.begin(), seg_parts.end(), 1);
    }
  }

  // Partial indices: first the prefix partials of every segment whose row
  // shares a prefix (ks per segment, so the rows of a group lie at a fixed
  // stride, as the prefix units write them), then the parts of cut segments.
  // A cut segment's merge unit is (query token, kv head, parts, first part
  // partial), (first prefix partial, ks, 0, 0) -- ks 0 when its row shares
  // none.  A segment left whole that shares a prefix folds its ks prefix
  // partials itself.
  std::vector<int64_t> seg_base(seg_parts.size(), -1), pfx_base(seg_parts.size(), -1);
  for (size_t sg = 0; sg < seg_parts.size(); ++sg) {
    const int64_t ks = pfx_splits[seg_row[sg]];
    // both counts fill bits 16-30 of a wave descriptor's first int
    if (seg_parts[sg] > 32767 || ks > 32767) return false;
    if (ks > 0) {
      pfx_base[sg] = partials;
      partials += ks;
    }
  }
  for (size_t sg = 0; sg < seg_parts.size(); ++sg) {
    if (seg_parts[sg] > 1) {
      seg_base[sg] = partials;
      const int64_t ks = pfx_splits[seg_row[sg]];
      mrg.push_back(int4{q_starts[seg_row[sg]], seg_kvh[sg], seg_parts[sg], static_cast<int>(partials)});
      mrg.push_back(int4{ks > 0 ? static_cast<int>(pfx_base[sg]) : 0, static_cast<int>(ks), 0, 0});
      partials += seg_parts[sg];
    }
  }
  if (partials > 0x7fffffff) return false;

  // Shared-prefix units: (row holding the prefix, kv head, first key, end
  // key), (first query token, queries, partial of the first query, partial
  // stride): query block b of a group, kv head h, key split k.  The rows of a
  // group have consecutive segments with ks partials each, so a block's
  // partials lie at a fixed stride.
  for (const PrefixGroup& pg : pgroups) {
    const int64_t ks = pfx_splits[pg.r0];
    const int64_t tiles = pg.keys / kPreKeys;
    for (int64_t b = 0; b * prefix_queries < pg.nrows; ++b) {
      const int64_t r = pg.r0 + b * prefix_queries;
      const int64_t nq = std::min(prefix_queries, pg.nrows - b * prefix_queries);
      for (int64_t h = 0; h < Hkv; ++h) {
        const int64_t base = pfx_base[seg_start[r] + h];
        const int64_t stride = nq > 1 ? pfx_base[seg_start[r + 1] + h] - base : 1;
        for (int64_t i = 0; i < nq; ++i)
          if (pfx_base[seg_start[r + i] + h] != base + i * stride) return false;
        for (int64_t k = 0; k < ks; ++k) {
          const int64_t k0 = kPreKeys * (tiles * k / ks), k1 = kPreKeys * (tiles * (k + 1) / ks);
          if (k1 <= k0) return false;
          pfx.push_back(int4{static_cast<int>(pg.r0), static_cast<int>(h), static_cast<int>(k0), static_cast<int>(k1)});
          pfx.push_back(int4{q_starts[r], static_cast<int>(nq), static_cast<int>(base + k), static_cast<int>(stride)});
        }
      }
    }
  }

  // Descriptors per work-group: W (one range per wave), or `ranges` when the
  // plan has fixed partitions (padded with empty ranges).
  const int per_wg = given_pt > 0 ? ranges : W;
  for (const auto& g : wgs) {
    // Waves per piece: one each, the rest to the piece with most slices per
    // wave (more pieces than waves: one range each).
    const int k = static_cast<int>(g.size());
    std::vector<int> w(k, 1);
    for (int extra = W - k; extra > 0; --extra) {
      int best = 0;
      for (int i = 1; i < k; ++i)
        if (static_cast<int64_t>(g[i].s1 - g[i].s0) * w[best] > static_cast<int64_t>(g[best].s1 - g[best].s0) * w[i])
          best = i;
      ++w[best];
    }
    for (int i = 0; i < k; ++i) {
      const Piece& pc = g[i];
      const int n = pc.s1 - pc.s0;
      const int r = pc.row;
      // A whole segment of a row that shares a prefix folds the prefix's
      // partials: its descriptor carries their count and first index.
      const bool fold = pfx_splits[r] > 0 && seg_parts[pc.seg] == 1;
      const int nparts = fold ? static_cast<int>(pfx_splits[r]) : seg_parts[pc.seg];
      const int part = fold ? kPrefixFold : pc.part;
      const int pidx = fold ? static_cast<int>(pfx_base[pc.seg])
                            : (nparts > 1 ? static_cast<int>(seg_base[pc.seg] + pc.part) : 0);
      for (int j = 0; j < w[i]; ++j) {
        const int a0 = pc.s0 + static_cast<int>((static_cast<int64_t>(n) * j) / w[i]);
        const int a1 = pc.s0 + static_cast<int>((static_cast<int64_t>(n) * (j + 1)) / w[i]);
        const int64_t lb = 16 * static_cast<int64_t>(a0) / bs;
        const int first = (a0 < a1 && lb < bt_stride) ? bt[r * bt_stride + lb] : -1;
        dec.push_back(int4{r | (nparts << 16), pc.kvh | (part << 16), a0, a1});
        dec.push_back(int4{q_starts[r], static_cast<int>(kend[r]), first, pidx});
      }
    }
    const int emitted = std::max(k, W);
    for (int e = emitted; e < per_wg; ++e) {
      dec.push_back(int4{-1, 0, 0, 0});
      dec.push_back(int4{0, 0, -1, 0});
    }
  }
  return true;
}

// Prefill launch list: (row, kv head, query block) units, longest key range first.
static void plan_prefill(const int32_t* q_lens, const int32_t* k_lens, const int32_t* q_offs,
                         int64_t rows, int64_t Hkv, int64_t G, int64_t D, bool causal,
                         std::vector<int4>& pre) {
  for (int64_t r = 0; r < rows; ++r) {
    const int64_t qlen = q_lens[r], klen = k_lens[r], off = q_offs[r];
    if (qlen < 2) continue;
    const int64_t qpw = prefill_waves(D) * 16 * prefill_nm(D) / G;  // queries per work-group
    for (int64_t qb = 0; qb * qpw < qlen; ++qb) {
      const int64_t q0 = qb * qpw, nq = std::min(qpw, qlen - q0);
      const int64_t kend = std::max<int64_t>(causal ? std::min(klen, off + q0 + nq) : klen, 0);
      for (int64_t h = 0; h < Hkv; ++h)
        pre.push_back(int4{static_cast<int>(r), static_cast<int>(h), static_cast<int>(qb),
                           static_cast<int>((kend + kPreKeys - 1) / kPreKeys)});
    }
  }
  std::stable_sort(pre.begin(), pre.end(), [](const int4& x, const int4& y) { return x.w > y.w; });
  // Two int4 per work-group, like the decode descriptors (second one unused).
  std::vector<int4> wide;
  wide.reserve(2 * pre.size());
  for (const int4& u : pre) {
    wide.push_back(u);
    wide.push_back(int4{0, 0, 0, 0});
  }
  pre.swap(wide);
}

template <class TT, int D, int W>
static void launch_decode(const AttnArgs& a, int64_t rows, int64_t n_dec, hipStream_t stream) {
  AttnArgs da = a;
  da.dec_ranges = a.sched && a.dec_ranges > W && n_dec % a.dec_ranges == 0 ? a.dec_ranges : W;
  dim3 grid = a.sched ? dim3(static_cast<uint32_t>(n_dec / da.dec_ranges))
                      : dim3(static_cast<uint32_t>(a.Hkv), static_cast<uint32_t>(a.max_parts),
                             static_cast<uint32_t>(rows));
  da.dec_slots = decode_slots(W, da.dec_ranges, a.G, D);
  const size_t lds = static_cast<size_t>(decode_lds_words(da.dec_ranges, da.dec_slots, a.G, D) * 4);
  auto go = [&](auto kernel) {
    if (lds > kMaxLdsBytes)
      (void)hipFuncSetAttribute(reinterpret_cast<const void*>(kernel), hipFuncAttributeMaxDynamicSharedMemorySize,
                                static_cast<int>(lds));
    hipLaunchKernelGGL(kernel, grid, dim3(64 * W), lds, stream, da);
  };
  // One instantiation per mode, so that the common one carries none of the
  // others' code.
  const bool mr = da.dec_ranges > W, vb = a.verify && a.sched;
  if (mr && vb) go(attn_decode_kernel<TT, D, W, true, true>);
  else if (mr) go(attn_decode_kernel<TT, D, W, true, false>);
  else if (vb) go(attn_decode_kernel<TT, D, W, false, true>);
  else go(attn_decode_kernel<TT, D, W, false, false>);
}

template <class TT, int D>
static void launch_mfma(const AttnArgs& a, int waves, int64_t rows, int64_t max_q, int64_t n_dec,
                        int64_t n_pre, int64_t n_merge, int64_t n_pfx, hipStream_t stream) {
  constexpr int NM = prefill_nm(D);
  if (a.sched && n_pfx > 0) {
    // Shared-prefix units, the first n_pfx of the prefill section, before
    // anything else on the caller's stream: the decode launch folds in the
    // partials they write.
    AttnArgs xa = a;
    xa.sched = a.sched + 2 * n_dec;
    hipLaunchKernelGGL((attn_prefill_kernel<TT, D, NM>), dim3(static_cast<uint32_t>(n_pfx)), dim3(64 * prefill_waves(D)), 0,
                       stream, xa);
  }
  // Prefill units, then the decode work-groups, in launch order on the
  // caller's stream.  (One launch holding both -- prefill units first,
  // decode work-groups taking the CUs the prefill tail leaves idle -- needs
  // one work-group size for both; with 8-wave prefill work-groups it saved
  // 6 us on the mixed workload, less than two 4-wave prefill work-groups per
  // CU save in the prefill alone.)
  const bool dec = !a.sched || n_dec > 0;
  const bool pre = a.sched ? n_pre > n_pfx : max_q >= 2;
  if (pre) {
    const int64_t qpw = prefill_waves(D) * 16 * NM / a.G;
    const int64_t nqb = (max_q + qpw - 1) / qpw;
    dim3 grid = a.sched ? dim3(static_cast<uint32_t>(n_pre - n_pfx))
                        : dim3(static_cast<uint32_t>(a.Hkv * nqb), 1u, static_cast<uint32_t>(rows));
    AttnArgs pa = a;
    if (a.sched) pa.sched = a.sched + 2 * (n_dec + n_pfx);
    hipLaunchKernelGGL((attn_prefill_kernel<TT, D, NM>), grid, dim3(64 * prefill_waves(D)), 0, stream, pa);
  }
  if (dec) {
    bool launched = false;
#if KVHOT_MAX_DECODE_WAVES >= 16
    if constexpr (D <= 128) {
      if (waves == 16) {
        launch_decode<TT, D, 16>(a, rows, n_dec, stream);
        launched = true;
      }
    }
#else
    (void)waves;
#endif
    if (!launched) launch_decode<TT, D, 8>(a, rows, n_dec, stream);
  }
  if (a.sched ? n_merge > 0 : (!a.sched || n_dec > 0) && a.max_parts > 1) {
    dim3 mgrid = a.sched ? dim3(static_cast<uint32_t>(n_merge))
                         : dim3(static_cast<uint32_t>((a.Hq * (D / 8) + 63) / 64), static_cast<uint32_t>(rows));
    hipLaunchKernelGGL((attn_merge_kernel<TT, D>), mgrid, dim3(a.sched ? 64 * kMergeWaves : 64), 0, stream, a);
  }
}

}  // namespace kvhot

using namespace kvhot;

extern "C" int64_t kvhot_paged_attention_workspace_bytes(
    int64_t num_rows, int64_t total_query, int64_t max_q_len, int64_t max_k_len,
    int64_t num_q_heads, int64_t num_kv_heads, int64_t head_dim,
    int64_t block_size, int64_t partition_tokens, int dtype) {
  (void)total_query;
  if (num_rows < 0 || max_q_len < 0 || max_k_len < 0 || num_q_heads <= 0 ||
      num_kv_heads <= 0 || head_dim <= 0 || block_size <= 0 || partition_tokens < 0 ||
      num_q_heads % num_kv_heads != 0 || dtype_size(dtype) == 0)
    return KVHOT_EINVAL;
  const Plan pl = make_plan(num_rows, max_q_len, max_k_len, num_q_heads, num_kv_heads,
                            head_dim, block_size, partition_tokens, dtype);
  return pl.grid_ok ? pl.workspace_bytes(num_q_heads / num_kv_heads, head_dim) : 0;
}

extern "C" int64_t kvhot_paged_attention_schedule(
    const int32_t* q_lens, const int32_t* k_lens, const int32_t* q_starts,
    const int32_t* q_pos_offsets, const int32_t* block_table, int64_t bt_row_stride,
    int64_t num_rows, int64_t num_q_heads, int64_t num_kv_heads, int64_t head_dim,
    int64_t block_size, int64_t partition_tokens, int attn_flags, int dtype,
    int32_t* units, int64_t capacity_units, int64_t* num_decode_units,
    int64_t* num_prefill_units, int64_t* num_merge_units, int64_t* workspace_bytes,
    int64_t* num_prefix_units) {
  clear_error();
  if (num_rows < 0 || num_q_heads <= 0 || num_kv_heads <= 0 || head_dim <= 0 ||
      block_size <= 0 || partition_tokens < 0 || num_q_heads % num_kv_heads != 0 ||
      dtype_size(dtype) == 0 || capacity_units < 0 || bt_row_stride < 0)
    return set_error(KVHOT_EINVAL, "paged_attention_schedule: bad sizes");
  if (attn_flags & ~(KVHOT_CAUSAL | KVHOT_DETERMINISTIC | KVHOT_VERIFY_BLOCKS))
    return set_error(KVHOT_EINVAL, "paged_attention_schedule: unknown attn_flags bits");
  const bool is_causal = (attn_flags & KVHOT_CAUSAL) != 0;
  if (num_rows > 65535 || num_q_heads > 65535)
    return set_error(KVHOT_EUNSUPPORTED, "paged_attention_schedule: rows or heads too large");
  if (num_rows > 0 && (!q_lens || !k_lens || !q_starts || !q_pos_offsets ||
                       (bt_row_stride > 0 && !block_table)))
    return set_error(KVHOT_EINVAL, "paged_attention_schedule: null host arrays");
  if (partition_tokens != 0 && (partition_tokens % 32 != 0 || partition_tokens > (1 << 20)))
    return set_error(KVHOT_EINVAL, "paged_attention_schedule: bad partition_tokens");
  int64_t max_q = 0, max_k = 0;
  for (int64_t r = 0; r < num_rows; ++r) {
    if (q_lens[r] < 0 || k_lens[r] < 0)
      return set_error(KVHOT_EINVAL, "paged_attention_schedule: negative length");
    max_q = std::max<int64_t>(max_q, q_lens[r]);
    max_k = std::max<int64_t>(max_k, k_lens[r]);
  }
  std::vector<int4> dec, pre, mrg, pfx;
  int64_t partials = 0;
  const Plan pl = make_plan(num_rows, max_q, max_k, num_q_heads, num_kv_heads, head_dim,
                            block_size, partition_tokens, dtype);
  if (pl.mfma) {
    const int64_t G = num_q_heads / num_kv_heads;
    const int64_t groups = resident_decode_waves(dtype, head_dim, pl.waves, G) / pl.waves;
    const int64_t prefix_queries = prefill_waves(head_dim) * 16 * prefill_nm(head_dim) / G;  // per prefill work-group
    const int ranges = decode_ranges(pl.waves, G, head_dim, partition_tokens > 0);
    if (plan_decode(q_lens, k_lens, q_pos_offsets, q_starts, block_table, bt_row_stride, block_size,
                    num_rows, num_kv_heads, is_causal, pl.waves, ranges, groups, partition_tokens,
                    32 * head_dim * dtype_size(dtype), prefix_queries, dec, mrg, pfx, partials)) {
      plan_prefill(q_lens, k_lens, q_pos_offsets, num_rows, num_kv_heads, G, head_dim, is_causal, pre);
      pre.insert(pre.begin(), pfx.begin(), pfx.end());  // shared-prefix units first
    } else {  // counts beyond the descriptor fields: no schedule
      dec.clear();
      mrg.clear();
      partials = 0;
    }
  }
  // Units are 8 int32 (two int4) each: decode waves, prefill work-groups,
  // merge units.
  const int64_t n_dec = static_cast<int64_t>(dec.size() / 2);
  const int64_t n_pre = static_cast<int64_t>(pre.size() / 2);
  const int64_t n_mrg = static_cast<int64_t>(mrg.size() / 2);
  if (num_decode_units) *num_decode_units = n_dec;
  if (num_prefill_units) *num_prefill_units = n_pre;
  if (num_merge_units) *num_merge_units = n_mrg;
  if (num_prefix_units) *num_prefix_units = static_cast<int64_t>(pfx.size() / 2);
  if (workspace_bytes) *workspace_bytes = partials * partial_bytes(num_q_heads / num_kv_heads, head_dim);
  if (units && capacity_units >= n_dec + n_pre + n_mrg) {
    int4* out = reinterpret_cast<int4*>(units);
    std::copy(dec.begin(), dec.end(), out);
    std::copy(pre.begin(), pre.end(), out + dec.size());
    std::copy(mrg.begin(), mrg.end(), out + dec.size() + pre.size());
  }
  return n_dec + n_pre + n_mrg;
}

// kvhot_paged_attention's body: validation, then the launches, all on the
// caller's stream.
static int paged_attention_impl(
    const void* q, const int64_t q_strides[3], const void* k_cache,
    const int64_t k_cache_strides[4], const void* v_cache,
    const int64_t v_cache_strides[4], void* out, const int64_t out_strides[3],
    float* lse, const int64_t lse_strides[2], const int32_t* block_table,
    int64_t bt_row_stride, const int32_t* q_lens, const int32_t* k_lens,
    const int32_t* q_starts, const int32_t* q_pos_offsets, int64_t num_rows,
    int64_t total_query, int64_t max_q_len, int64_t max_k_len,
    int64_t num_q_heads, int64_t num_kv_heads, int64_t head_dim,
    int64_t block_size, int64_t num_blocks, float scale, int attn_flags,
    int dtype, int64_t partition_tokens, const int32_t* schedule,
    int64_t num_decode_units, int64_t num_prefill_units, int64_t num_merge_units,
    int64_t num_prefix_units, int64_t schedule_workspace_bytes, void* workspace, int64_t workspace_bytes,
    void* stream) {
  clear_error();
  const int64_t es = dtype_size(dtype);
  if (es == 0) return set_error(KVHOT_EINVAL, "paged_attention: bad dtype");
  if (num_rows < 0 || total_query < 0 || max_q_len < 0 || max_k_len < 0 ||
      num_q_heads <= 0 || num_kv_heads <= 0 || head_dim <= 0 || block_size <= 0 ||
      num_blocks < 0 || bt_row_stride < 0 || partition_tokens < 0 || workspace_bytes < 0)
    return set_error(KVHOT_EINVAL, "paged_attention: bad sizes");
  if (num_q_heads % num_kv_heads != 0)
    return set_error(KVHOT_EINVAL, "paged_attention: num_q_heads % num_kv_heads != 0");
  if (attn_flags & ~(KVHOT_CAUSAL | KVHOT_DETERMINISTIC | KVHOT_VERIFY_BLOCKS))
    return set_error(KVHOT_EINVAL, "paged_attention: unknown attn_flags bits");
  if (num_rows == 0 || total_query == 0 || max_q_len == 0) return 0;
  if (!q || !k_cache || !v_cache || !out || !q_lens || !k_lens || !q_starts ||
      !q_pos_offsets || !q_strides || !k_cache_strides || !v_cache_strides ||
      !out_strides || (lse && !lse_strides))
    return set_error(KVHOT_EINVAL, "paged_attention: null pointer");
  if (max_k_len > 0 && (num_blocks == 0 || bt_row_stride == 0 || !block_table))
    return set_error(KVHOT_EINVAL, "paged_attention: keys requested but no blocks / block table");
  if (q_strides[2] != 1 || k_cache_strides[3] != 1 || v_cache_strides[3] != 1 ||
      out_strides[2] != 1)
    return set_error(KVHOT_EINVAL, "paged_attention: head_dim must be unit-stride");
  if (num_rows > 65535 || max_q_len > 65535 || max_k_len > (1LL << 30) ||
      num_q_heads > 65535)
    return set_error(KVHOT_EUNSUPPORTED, "paged_attention: rows, max_q_len or heads too large");
  if (partition_tokens != 0 &&
      (partition_tokens % 32 != 0 || partition_tokens > (1 << 20)))
    return set_error(KVHOT_EINVAL,
                     "paged_attention: partition_tokens must be a multiple of 32 and <= 2^20");

  AttnArgs a{};
  a.q = q; a.q_st = q_strides[0]; a.q_sh = q_strides[1];
  a.k = k_cache; a.k_sb = k_cache_strides[0]; a.k_st = k_cache_strides[1]; a.k_sh = k_cache_strides[2];
  a.v = v_cache; a.v_sb = v_cache_strides[0]; a.v_st = v_cache_strides[1]; a.v_sh = v_cache_strides[2];
  a.o = out; a.o_st = out_strides[0]; a.o_sh = out_strides[1];
  a.lse = lse;
  a.l_st = lse ? lse_strides[0] : 0;
  a.l_sh = lse ? lse_strides[1] : 0;
  a.bt = block_table; a.bt_stride = bt_row_stride;
  // A launch with no keys may have no table; the decode loop still reads one
  // entry ahead of its claims (row 0, entry 0 when nothing is claimed), so
  // k_lens, which every launch has, stands in for it.
  if (!a.bt || a.bt_stride == 0) {
    a.bt = k_lens;
    a.bt_stride = 0;
  }
  a.q_lens = q_lens; a.k_lens = k_lens; a.q_starts = q_starts; a.q_offs = q_pos_offsets;
  a.num_blocks = num_blocks;
  a.Hq = static_cast<int32_t>(num_q_heads);
  a.Hkv = static_cast<int32_t>(num_kv_heads);
  a.G = static_cast<int32_t>(num_q_heads / num_kv_heads);
  a.bs = static_cast<int32_t>(block_size);
  a.scale_log2 = scale * kLog2e;
  a.causal = (attn_flags & KVHOT_CAUSAL) ? 1 : 0;
  a.fixed = (attn_flags & KVHOT_DETERMINISTIC) ? 1 : 0;
  a.verify = (attn_flags & KVHOT_VERIFY_BLOCKS) ? 1 : 0;
  a.D = static_cast<int32_t>(head_dim);
  a.total_q = total_query;
  const int64_t n_dec = schedule ? num_decode_units : 0;
  const int64_t n_pre = schedule ? num_prefill_units : 0;
  const int64_t n_mrg = schedule ? num_merge_units : 0;
  const int64_t n_pfx = schedule ? num_prefix_units : 0;
  if (schedule && (n_dec < 0 || n_pre < 0 || n_mrg < 0 || n_dec > 0x7fffffff ||
                   n_pre > 0x7fffffff || n_mrg > 0x7fffffff || schedule_workspace_bytes < 0 ||
                   n_pfx < 0 || n_pfx > n_pre))
    return set_error(KVHOT_EINVAL, "paged_attention: bad schedule unit counts");
  a.sched = reinterpret_cast<const int4*>(schedule);
  a.merge_units = (schedule && n_mrg > 0) ? a.sched + 2 * (n_dec + n_pre) : nullptr;
  a.max_parts = 1;
  hipStream_t s = static_cast<hipStream_t>(stream);

  Plan pl = make_plan(num_rows, max_q_len, max_k_len, num_q_heads, num_kv_heads, head_dim,
                      block_size, partition_tokens, dtype);
  if (!schedule && !pl.grid_ok) pl.mfma = false;
  if (schedule && pl.mfma && n_dec % pl.waves != 0)
    return set_error(KVHOT_EINVAL, "paged_attention: decode schedule is not whole work-groups");
  if (pl.mfma) {
    // 16-byte vector loads/stores need 16-byte aligned rows.
    const int64_t al = 16 / es;
    const uintptr_t ptr_or = reinterpret_cast<uintptr_t>(q) | reinterpret_cast<uintptr_t>(k_cache) |
                             reinterpret_cast<uintptr_t>(v_cache) | reinterpret_cast<uintptr_t>(out);
    const int64_t str[10] = {a.q_st, a.q_sh, a.k_sb, a.k_st, a.k_sh,
                             a.v_sb, a.v_st, a.v_sh, a.o_st, a.o_sh};
    bool aligned = (ptr_or % 16) == 0;
    for (int64_t x : str) aligned = aligned && (x % al) == 0;
    // Buffer descriptors cover one block: its stride (and the token stride
    // inside it) must fit their 32-bit ranges.
    const bool fits = a.k_sb > 0 && a.v_sb > 0 && es * a.k_sb < (1LL << 31) && es * a.v_sb < (1LL << 31) &&
                      a.k_st > 0 && a.v_st > 0 && 16 * es * a.k_st < (1LL << 31) && 16 * es * a.v_st < (1LL << 31);
    if (!aligned || !fits) pl.mfma = false;
  }
  if (pl.mfma) {
    const int64_t pb = partial_bytes(a.G, head_dim);
    if (schedule && (n_mrg > 0 || n_pfx > 0) && schedule_workspace_bytes < pb)
      return set_error(KVHOT_EINVAL, "paged_attention: a schedule with merge or prefix units needs partials");
    const int64_t need = schedule ? (n_mrg > 0 || n_pfx > 0 ? schedule_workspace_bytes : 0)
                                  : pl.workspace_bytes(a.G, head_dim);
    if (need > 0) {
      if (!workspace || workspace_bytes < need)
        return set_error(KVHOT_EWORKSPACE,
                         "paged_attention: workspace of " + std::to_string(need) + " bytes required");
      a.num_partials = schedule ? workspace_bytes / pb : pl.partials;
      a.ws_o = static_cast<float*>(workspace);
      a.ws_lse = a.ws_o + a.num_partials * a.G * head_dim;
    }
    if (!schedule) {
      a.part_tokens = pl.part_tokens;
      a.max_parts = pl.max_parts;
    }
    // A launch list of fixed partitions groups its decode ranges as the
    // planner did (the same partition_tokens is passed to both calls; with
    // another value the ranges come in groups of one per wave, which gives
    // the same results).
    a.dec_ranges = schedule ? decode_ranges(pl.waves, a.G, head_dim, partition_tokens > 0) : pl.waves;
#define KVHOT_MFMA(TT, DD) \
  launch_mfma<TT, DD>(a, pl.waves, num_rows, max_q_len, n_dec, n_pre, n_mrg, n_pfx, s)
    if (dtype == KVHOT_BF16) {
      if (head_dim == 64) KVHOT_MFMA(BF16, 64);
      else if (head_dim == 128) KVHOT_MFMA(BF16, 128);
      else KVHOT_MFMA(BF16, 256);
    } else {
      if (head_dim == 64) KVHOT_MFMA(F16, 64);
      else if (head_dim == 128) KVHOT_MFMA(F16, 128);
      else KVHOT_MFMA(F16, 256);
    }
#undef KVHOT_MFMA
    return launch_status("paged_attention");
  }

  if (head_dim > kGenericMaxD)
    return set_error(KVHOT_EUNSUPPORTED, "paged_attention: head_dim > 256");
  dim3 grid(static_cast<uint32_t>(num_q_heads), static_cast<uint32_t>(max_q_len),
            static_cast<uint32_t>(num_rows));
  if (dtype == KVHOT_F32)
    hipLaunchKernelGGL(attn_generic_kernel<F32>, grid, dim3(64), 0, s, a);
  else if (dtype == KVHOT_BF16)
    hipLaunchKernelGGL(attn_generic_kernel<BF16>, grid, dim3(64), 0, s, a);
  else
    hipLaunchKernelGGL(attn_generic_kernel<F16>, grid, dim3(64), 0, s, a);
  return launch_status("paged_attention");
}

extern "C" int kvhot_paged_attention(
    const void* q, const int64_t q_strides[3], const void* k_cache,
    const int64_t k_cache_strides[4], const void* v_cache,
    const int64_t v_cache_strides[4], void* out, const int64_t out_strides[3],
    float* lse, const int64_t lse_strides[2], const int32_t* block_table,
    int64_t bt_row_stride, const int32_t* q_lens, const int32_t* k_lens,
    const int32_t* q_starts, const int32_t* q_pos_offsets, int64_t num_rows,
    int64_t total_query, int64_t max_q_len, int64_t max_k_len,
    int64_t num_q_heads, int64_t num_kv_heads, int64_t head_dim,
    int64_t block_size, int64_t num_blocks, float scale, int attn_flags,
    int dtype, int64_t partition_tokens, const int32_t* schedule,
    int64_t num_decode_units, int64_t num_prefill_units, int64_t num_merge_units,
    int64_t num_prefix_units, int64_t schedule_workspace_bytes, void* workspace, int64_t workspace_bytes, void* stream) {
  return paged_attention_impl(q, q_strides, k_cache, k_cache_strides, v_cache, v_cache_strides, out, out_strides,
                              lse, lse_strides, block_table, bt_row_stride, q_lens, k_lens, q_starts,
                              q_pos_offsets, num_rows, total_query, max_q_len, max_k_len, num_q_heads,
                              num_kv_heads, head_dim, block_size, num_blocks, scale, attn_flags, dtype,
                              partition_tokens, schedule, num_decode_units, num_prefill_units, num_merge_units,
                              num_prefix_units, schedule_workspace_bytes, workspace, workspace_bytes, stream);
}

// ------------------------------------------------------------ no-alloc --
// Split-K partials of kvhot_paged_attention_noalloc: a device-global array,
// one copy on every device the library runs on, held until the process ends.
// In host code `scratch` names a host-side stand-in, not device memory: its
// device address comes from hipGetSymbolAddress, once per device.
static __device__ __align__(256) unsigned char scratch[KVHOT_NOALLOC_SCRATCH_BYTES];

constexpr int kMaxDevices = 64;
static std::mutex g_scratch_mutex;
static void* g_scratch_addr[kMaxDevices];

// Device address of the current device's `scratch`, looked up on the
// device's first call.  0, or a positive hipError_t.  That first call may come
// while the caller's stream is being captured into a graph: the lookup is not
// a stream operation, and it runs with this thread's capture mode relaxed so
// that a global-mode capture does not treat it as an unsafe call.
static int scratch_address(void** out) {
  int dev = -1;
  const hipError_t de = hipGetDevice(&dev);
  if (de != hipSuccess || dev < 0 || dev >= kMaxDevices) {
    (void)hipGetLastError();
    return set_error(de != hipSuccess ? static_cast<int>(de) : static_cast<int>(hipErrorInvalidDevice),
                     "paged_attention_noalloc: no usable current device");
  }
  std::lock_guard<std::mutex> guard(g_scratch_mutex);
  if (!g_scratch_addr[dev]) {
    void* p = nullptr;
    hipStreamCaptureMode mode = hipStreamCaptureModeRelaxed;
    const bool exchanged = hipThreadExchangeStreamCaptureMode(&mode) == hipSuccess;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (exchanged) (void)hipThreadExchangeStreamCaptureMode(&mode);
    if (e != hipSuccess || !p) {
      (void)hipGetLastError();
      return set_error(e != hipSuccess ? static_cast<int>(e) : static_cast<int>(hipErrorInvalidSymbol),
                       std::string("paged_attention_noalloc: hipGetSymbolAddress(scratch): ") +
                           hipGetErrorString(e));
    }
    g_scratch_addr[dev] = p;
  }
  *out = g_scratch_addr[dev];
  return 0;
}

extern "C" int kvhot_paged_attention_noalloc(
    const void* q, const int64_t q_strides[3], const void* k_cache,
    const int64_t k_cache_strides[4], const void* v_cache,
    const int64_t v_cache_strides[4], void* out, const int64_t out_strides[3],
    float* lse, const int64_t lse_strides[2], const int32_t* block_table,
    int64_t bt_row_stride, const int32_t* q_lens, const int32_t* k_lens,
    const int32_t* q_starts, const int32_t* q_pos_offsets, int64_t num_rows,
    int64_t total_query, int64_t max_q_len, int64_t max_k_len,
    int64_t num_q_heads, int64_t num_kv_heads, int64_t head_dim,
    int64_t block_size, int64_t num_blocks, float scale, int attn_flags,
    int dtype, int64_t partition_tokens, const int32_t* schedule,
    int64_t num_decode_units, int64_t num_prefill_units, int64_t num_merge_units,
    int64_t num_prefix_units, int64_t schedule_workspace_bytes, void* stream) {
  clear_error();
  int64_t need = 0;
  if (schedule) {
    need = num_merge_units > 0 || num_prefix_units > 0 ? schedule_workspace_bytes : 0;
  } else {
    need = kvhot_paged_attention_workspace_bytes(num_rows, total_query, max_q_len, max_k_len, num_q_heads,
                                                 num_kv_heads, head_dim, block_size, partition_tokens, dtype);
    if (need < 0) return set_error(static_cast<int>(need), "paged_attention_noalloc: bad sizes");
  }
  if (need > KVHOT_NOALLOC_SCRATCH_BYTES)
    return set_error(KVHOT_EWORKSPACE, "paged_attention_noalloc: the call needs " + std::to_string(need) +
                                           " bytes of split-K partials, more than its scratch of " +
                                           std::to_string(static_cast<int64_t>(KVHOT_NOALLOC_SCRATCH_BYTES)));
  void* ws = nullptr;
  if (need > 0) {
    const int rc = scratch_address(&ws);
    if (rc != 0) return rc;
  }
  return paged_attention_impl(q, q_strides, k_cache, k_cache_strides, v_cache, v_cache_strides, out, out_strides,
                              lse, lse_strides, block_table, bt_row_stride, q_lens, k_lens, q_starts,
                              q_pos_offsets, num_rows, total_query, max_q_len, max_k_len, num_q_heads,
                              num_kv_heads, head_dim, block_size, num_blocks, scale, attn_flags, dtype,
                              partition_tokens, schedule, num_decode_units, num_prefill_units, num_merge_units,
                              num_prefix_units, schedule_workspace_bytes, ws, need > 0 ? int64_t{KVHOT_NOALLOC_SCRATCH_BYTES} : 0,
                              stream);
}
