// Paged attention over a ragged batch of prefill chunks and decode rows.
//
// Kernel map (one wavefront per work-group throughout):
//  * attn_mfma_kernel<T, D, NM>, bf16/f16.  A wave owns one (row, kv head,
//    query block, key partition).  Its 16*NM "m-rows" are (query, head) pairs
//    of one GQA group, so every K/V byte it loads serves all G = Hq/Hkv query
//    heads of that kv head.  Keys are walked in tiles of 32 tokens (two
//    16-token block slices).  Scores are formed transposed, S^T = K . Q^T, with
//    v_mfma_f32_16x16x32: K rows (token-major, head_dim contiguous) are already
//    the MFMA A-operand layout, so K goes HBM -> VGPR with no LDS round trip.
//    The accumulator layout of S^T (lane = m-row, 4 tokens per lane) is exactly
//    the B-operand layout P^T needs for O^T = V^T . P^T, so probabilities never
//    leave registers.  V^T is formed in registers with v_perm_b32 from 16-byte
//    row loads.  Softmax statistics live in the lane that owns the m-row, so
//    rescaling O needs no cross-lane traffic.
//    - decode launch (role 0, rows with q_len == 1, NM = 1): split-K over key
//      partitions.  A row with one partition is finished in place; otherwise
//      each partition stores (LSE, normalised O) with plain stores and
//      attn_merge_kernel combines them in a second launch.  (Merging inside
//      the first launch needs a device-scope release per wave, which on
//      gfx950 is an L2 write-back per wave: far slower than a launch.)
//    - prefill launch (role 1, rows with q_len >= 2, NM = 4): 16*4/G queries
//      per wave, causal mask from q_pos_offset, tiles past the diagonal skipped.
//  * attn_generic_kernel<T>: VALU kernel for fp32 (exact fp32 arithmetic) and
//    for shapes the MFMA kernel does not cover.
#include "kvhot_internal.h"

#include <algorithm>
#include <climits>

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
  float* ws_lse;  // [rows, Hq, max_parts] log2-domain partition LSE
  float* ws_o;    // [rows, Hq, max_parts, D] normalised partition output
  int64_t num_blocks;
  int32_t Hq, Hkv, G, bs;
  int32_t part_tokens, max_parts;
  float scale_log2;
  int32_t causal;
  int32_t role;  // 0: rows with q_len == 1; 1: rows with q_len >= 2; 2: all rows
  int32_t D;     // head_dim (generic kernel)
  int64_t total_q;  // rows of q / out / lse: outputs are only written below it
};

__device__ inline float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

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
struct KVTile {
  static constexpr int NC = D / 32;   // 32-wide head_dim chunks of Q.K
  static constexpr int VW = D / 32;   // dwords per V row slice per lane (D/16 elements)
  u32x4 k[2][NC];                     // [slice][chunk]: token n, dims 8*(4c+g)..+8
  uint32_t v[8][VW];                  // [k-slot]: token tok(g, slot), dims (D/16)*n..+D/16
};

// Which key token (0..31 within a tile) k-slot s8 of lane group g holds.
__device__ inline int slot_token(int g, int s8) {
  return (s8 < 4) ? (4 * g + s8) : (16 + 4 * g + (s8 - 4));
}

template <class TT, int D, int NM, bool DB>
__global__ void __launch_bounds__(64)
attn_mfma_kernel(const AttnArgs a) {
  constexpr int NC = D / 32;
  constexpr int EPL = D / 16;   // head_dim values per lane per V row; PV MFMAs per tile
  constexpr int VW = EPL / 2;
  constexpr int MR = 16 * NM;   // m-rows per wave
  using st = uint16_t;

  const int lane = threadIdx.x;
  const int n = lane & 15;
  const int g = lane >> 4;
  const int row = blockIdx.z;
  const int qlen = a.q_lens[row];
  if (a.role == 0 ? (qlen != 1) : (qlen < 2)) return;
  const int kvh = blockIdx.x % a.Hkv;
  const int qblk = blockIdx.x / a.Hkv;
  const int G = a.G;
  const int QPW = MR / G;
  const int q0 = qblk * QPW;
  if (q0 >= qlen) return;
  const int nq = min(QPW, qlen - q0);
  const int off = a.q_offs[row];
  const int klen = a.k_lens[row];
  int kend = a.causal ? min(klen, off + q0 + nq) : klen;
  kend = max(kend, 0);
  const int PT = a.part_tokens;
  // Never more partitions than the grid and the workspace were sized for.
  kend = static_cast<int>(min(static_cast<int64_t>(kend), static_cast<int64_t>(a.max_parts) * PT));
  const int nparts = max((kend + PT - 1) / PT, 1);
  const int p = blockIdx.y;
  if (p >= nparts) return;
  const int kbeg = p * PT;
  const int kstop = min(kend, kbeg + PT);
  const int qs = a.q_starts[row];

  // ---- per-lane m-rows and Q (B operand of S^T = K . Q^T) ----
  int mq[NM], mh[NM], qpos[NM];
  bool mval[NM];
  u32x4 qf[NM][NC];
#pragma unroll
  for (int s = 0; s < NM; ++s) {
    const int i = 16 * s + n;
    mq[s] = i / G;
    mh[s] = kvh * G + (i % G);
    mval[s] = mq[s] < nq && static_cast<int64_t>(qs) + q0 + mq[s] < a.total_q;
    qpos[s] = mval[s] ? (a.causal ? off + q0 + mq[s] : INT_MAX) : -1;
#pragma unroll
    for (int c = 0; c < NC; ++c) qf[s][c] = u32x4{0, 0, 0, 0};
    if (mval[s]) {
      const st* qp = static_cast<const st*>(a.q) +
                     (static_cast<int64_t>(qs) + q0 + mq[s]) * a.q_st +
                     static_cast<int64_t>(mh[s]) * a.q_sh;
#pragma unroll
      for (int c = 0; c < NC; ++c)
        qf[s][c] = *reinterpret_cast<const u32x4*>(qp + 8 * (4 * c + g));
    }
  }
  // Smallest query position of the wave: keys up to it are visible to all m-rows.
  const int qpos_min = a.causal ? off + q0 : INT_MAX;

  // ---- block table: lane j holds the id of logical block win + j, for a
  // window of 64 blocks loaded once before its tiles are walked ----
  const int bs = a.bs;
  const int32_t* btrow = a.bt + static_cast<int64_t>(row) * a.bt_stride;
  const int nb_row = min(static_cast<int64_t>((kstop + bs - 1) / bs), a.bt_stride);
  int win = 0;
  int bt_reg = 0;
  auto block_of = [&](int lb) -> int64_t {
    int64_t id = __builtin_amdgcn_readlane(bt_reg, lb - win);
    id = id < 0 ? 0 : (id >= a.num_blocks ? a.num_blocks - 1 : id);
    return id;
  };

  // Loop-invariant per-lane element offsets inside a 16-token block slice.
  const int k_lane = n * static_cast<int>(a.k_st) + 8 * g;
  int v_lane[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) v_lane[j] = (4 * g + j) * static_cast<int>(a.v_st) + EPL * n;

  const st* kbase = static_cast<const st*>(a.k) + static_cast<int64_t>(kvh) * a.k_sh;
  const st* vbase = static_cast<const st*>(a.v) + static_cast<int64_t>(kvh) * a.v_sh;

  auto load_tile = [&](int ts, KVTile<D>& T) {
    const int64_t id0 = block_of(ts / bs);
    const int bo0 = ts % bs;
    int64_t id1 = id0;
    int bo1 = bo0;
    if (ts + 16 < kstop) {
      id1 = block_of((ts + 16) / bs);
      bo1 = (ts + 16) % bs;
    }
    const st* kp[2] = {kbase + id0 * a.k_sb + static_cast<int64_t>(bo0) * a.k_st,
                       kbase + id1 * a.k_sb + static_cast<int64_t>(bo1) * a.k_st};
    const st* vp[2] = {vbase + id0 * a.v_sb + static_cast<int64_t>(bo0) * a.v_st,
                       vbase + id1 * a.v_sb + static_cast<int64_t>(bo1) * a.v_st};
#pragma unroll
    for (int sl = 0; sl < 2; ++sl)
#pragma unroll
      for (int c = 0; c < NC; ++c)
        T.k[sl][c] = *reinterpret_cast<const u32x4*>(kp[sl] + k_lane + 32 * c);
#pragma unroll
    for (int s8 = 0; s8 < 8; ++s8) load_dwords<VW>(vp[s8 >> 2] + v_lane[s8 & 3], T.v[s8]);
  };

  float m[NM], l[NM];
  f32x4 o[NM][EPL];
#pragma unroll
  for (int s = 0; s < NM; ++s) {
    m[s] = -INFINITY;
    l[s] = 0.f;
#pragma unroll
    for (int e = 0; e < EPL; ++e) o[s][e] = f32x4{0.f, 0.f, 0.f, 0.f};
  }

  auto compute_tile = [&](int ts, KVTile<D>& T) {
    // S^T for the two 16-token slices.
    f32x4 sc[2][NM];
#pragma unroll
    for (int sl = 0; sl < 2; ++sl)
#pragma unroll
      for (int s = 0; s < NM; ++s) {
        f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int c = 0; c < NC; ++c) acc = TT::mfma(T.k[sl][c], qf[s][c], acc);
        sc[sl][s] = acc;
      }
    const bool tail = ts + 32 > kstop;
    const bool full = !tail && (ts + 31 <= qpos_min);
#pragma unroll
    for (int sl = 0; sl < 2; ++sl)
#pragma unroll
      for (int s = 0; s < NM; ++s)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          float x = sc[sl][s][j] * a.scale_log2;
          if (!full) {
            const int tk = ts + 16 * sl + 4 * g + j;
            x = (tk < kstop && tk <= qpos[s]) ? x : -INFINITY;
          }
          sc[sl][s][j] = x;
        }
    if (tail) {
      // Keys past the end may hold any bit pattern; zero them so 0 * V stays 0.
#pragma unroll
      for (int s8 = 0; s8 < 8; ++s8) {
        const bool ok = ts + slot_token(g, s8) < kstop;
#pragma unroll
        for (int w = 0; w < VW; ++w) T.v[s8][w] = ok ? T.v[s8][w] : 0u;
      }
    }
    // Online softmax (base 2); P^T packed as the B operand of O^T += V^T . P^T.
    u32x4 pb[NM];
#pragma unroll
    for (int s = 0; s < NM; ++s) {
      float mx = fmaxf(fmaxf(fmaxf(sc[0][s][0], sc[0][s][1]), fmaxf(sc[0][s][2], sc[0][s][3])),
                       fmaxf(fmaxf(sc[1][s][0], sc[1][s][1]), fmaxf(sc[1][s][2], sc[1][s][3])));
      mx = fmaxf(mx, __shfl_xor(mx, 16, kWave));
      mx = fmaxf(mx, __shfl_xor(mx, 32, kWave));
      const float mnew = fmaxf(m[s], mx);
      const float muse = (mnew == -INFINITY) ? 0.f : mnew;
      const float corr = fast_exp2(m[s] - muse);
      float pr[8];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        pr[j] = fast_exp2(sc[0][s][j] - muse);
        pr[4 + j] = fast_exp2(sc[1][s][j] - muse);
      }
      float sum = ((pr[0] + pr[1]) + (pr[2] + pr[3])) + ((pr[4] + pr[5]) + (pr[6] + pr[7]));
      l[s] = l[s] * corr + sum;
      m[s] = mnew;
      pb[s] = u32x4{TT::pack2(pr[0], pr[1]), TT::pack2(pr[2], pr[3]),
                    TT::pack2(pr[4], pr[5]), TT::pack2(pr[6], pr[7])};
#pragma unroll
      for (int e = 0; e < EPL; ++e) o[s][e] *= corr;
    }
    // V^T A operand for head_dim values EPL*n + e, then O^T += V^T . P^T.
#pragma unroll
    for (int e = 0; e < EPL; ++e) {
      const int w = e >> 1;
      const uint32_t sel = (e & 1) ? 0x07060302u : 0x05040100u;
      const u32x4 vt = {__builtin_amdgcn_perm(T.v[1][w], T.v[0][w], sel),
                        __builtin_amdgcn_perm(T.v[3][w], T.v[2][w], sel),
                        __builtin_amdgcn_perm(T.v[5][w], T.v[4][w], sel),
                        __builtin_amdgcn_perm(T.v[7][w], T.v[6][w], sel)};
#pragma unroll
      for (int s = 0; s < NM; ++s) o[s][e] = TT::mfma(vt, pb[s], o[s][e]);
    }
  };

  // ---- key loop over windows of 64 blocks; with DB, tile i+1 is in flight
  // while tile i computes ----
  for (int wbeg = kbeg; wbeg < kstop; wbeg += 64 * bs) {
    const int wend = min(kstop, wbeg + 64 * bs);
    win = wbeg / bs;
    bt_reg = (win + lane < nb_row) ? btrow[win + lane] : 0;
    if constexpr (!DB) {
      for (int ts = wbeg; ts < wend; ts += 32) {
        KVTile<D> T;
        load_tile(ts, T);
        compute_tile(ts, T);
      }
    } else {
      KVTile<D> A, B;
      int ts = wbeg;
      load_tile(ts, A);
      while (true) {
        bool more = ts + 32 < wend;
        if (more) load_tile(ts + 32, B);
        compute_tile(ts, A);
        ts += 32;
        if (!more) break;
        more = ts + 32 < wend;
        if (more) load_tile(ts + 32, A);
        compute_tile(ts, B);
        ts += 32;
        if (!more) break;
      }
    }
  }

  // ---- finish: lane (n, g) holds O^T rows d = EPL*(4g+j)+e of m-row n ----
  float ltot[NM];
#pragma unroll
  for (int s = 0; s < NM; ++s) {
    float t = l[s] + __shfl_xor(l[s], 16, kWave);
    ltot[s] = t + __shfl_xor(t, 32, kWave);
  }

  if (nparts == 1) {
#pragma unroll
    for (int s = 0; s < NM; ++s) {
      if (!mval[s]) continue;
      const int64_t t = static_cast<int64_t>(qs) + q0 + mq[s];
      const float inv = ltot[s] > 0.f ? 1.f / ltot[s] : 0.f;
      st* op = static_cast<st*>(a.o) + t * a.o_st + static_cast<int64_t>(mh[s]) * a.o_sh;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        uint32_t w[VW];
#pragma unroll
        for (int e2 = 0; e2 < VW; ++e2)
          w[e2] = TT::pack2(o[s][2 * e2][j] * inv, o[s][2 * e2 + 1][j] * inv);
        st* dp = op + EPL * (4 * g + j);
        if constexpr (VW == 2) {
          *reinterpret_cast<u32x2*>(dp) = u32x2{w[0], w[1]};
        } else {
#pragma unroll
          for (int c = 0; c < VW / 4; ++c)
            *reinterpret_cast<u32x4*>(dp + 8 * c) =
                u32x4{w[4 * c], w[4 * c + 1], w[4 * c + 2], w[4 * c + 3]};
        }
      }
      if (a.lse && g == 0)
        a.lse[t * a.l_st + static_cast<int64_t>(mh[s]) * a.l_sh] =
            ltot[s] > 0.f ? (m[s] + __log2f(ltot[s])) * kLn2 : -INFINITY;
    }
    return;
  }

  // ---- split-K: store this partition for attn_merge_kernel ----
  // Only the decode launch splits, so a row holds exactly one query.
#pragma unroll
  for (int s = 0; s < NM; ++s) {
    if (!mval[s]) continue;
    const int64_t pidx = (static_cast<int64_t>(row) * a.Hq + mh[s]) * a.max_parts + p;
    const float inv = ltot[s] > 0.f ? 1.f / ltot[s] : 0.f;
    float* wp = a.ws_o + pidx * D;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      float* dp = wp + EPL * (4 * g + j);
#pragma unroll
      for (int c = 0; c < EPL / 4; ++c)
        *reinterpret_cast<f32x4*>(dp + 4 * c) =
            f32x4{o[s][4 * c][j] * inv, o[s][4 * c + 1][j] * inv,
                  o[s][4 * c + 2][j] * inv, o[s][4 * c + 3][j] * inv};
    }
    if (g == 0) a.ws_lse[pidx] = ltot[s] > 0.f ? m[s] + __log2f(ltot[s]) : -INFINITY;
  }
}

// Combines the split-K partitions of decode rows: one lane per (row, query
// head, 8 head_dim values).  Rows finished by a single partition are skipped;
// the partition count is recomputed exactly as the split kernel did.
template <class TT, int D>
__global__ void __launch_bounds__(256)
attn_merge_kernel(const AttnArgs a) {
  using st = uint16_t;
  constexpr int CH = D / 8;
  const int row = blockIdx.y;
  if (a.q_lens[row] != 1) return;
  const int idx = blockIdx.x * 256 + threadIdx.x;
  if (idx >= a.Hq * CH) return;
  const int h = idx / CH;
  const int c = idx % CH;
  const int off = a.q_offs[row];
  const int klen = a.k_lens[row];
  int kend = a.causal ? min(klen, off + 1) : klen;
  kend = max(kend, 0);
  const int PT = a.part_tokens;
  kend = static_cast<int>(min(static_cast<int64_t>(kend), static_cast<int64_t>(a.max_parts) * PT));
  const int nparts = (kend + PT - 1) / PT;
  if (nparts <= 1) return;
  const int64_t t = a.q_starts[row];
  if (t < 0 || t >= a.total_q) return;

  const int64_t base = (static_cast<int64_t>(row) * a.Hq + h) * a.max_parts;
  float mmax = -INFINITY;
  for (int pp = 0; pp < nparts; ++pp) mmax = fmaxf(mmax, a.ws_lse[base + pp]);
  float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  float lsum = 0.f;
  if (mmax != -INFINITY) {
    for (int pp = 0; pp < nparts; ++pp) {
      const float w = fast_exp2(a.ws_lse[base + pp] - mmax);
      lsum += w;
      const f32x4* src = reinterpret_cast<const f32x4*>(a.ws_o + (base + pp) * D + 8 * c);
      const f32x4 x0 = src[0], x1 = src[1];
      acc[0] += w * x0.x; acc[1] += w * x0.y; acc[2] += w * x0.z; acc[3] += w * x0.w;
      acc[4] += w * x1.x; acc[5] += w * x1.y; acc[6] += w * x1.z; acc[7] += w * x1.w;
    }
  }
  const float inv = lsum > 0.f ? 1.f / lsum : 0.f;
  st* dp = static_cast<st*>(a.o) + t * a.o_st + static_cast<int64_t>(h) * a.o_sh + 8 * c;
  *reinterpret_cast<u32x4*>(dp) =
      u32x4{TT::pack2(acc[0] * inv, acc[1] * inv), TT::pack2(acc[2] * inv, acc[3] * inv),
            TT::pack2(acc[4] * inv, acc[5] * inv), TT::pack2(acc[6] * inv, acc[7] * inv)};
  if (a.lse && c == 0)
    a.lse[t * a.l_st + static_cast<int64_t>(h) * a.l_sh] =
        lsum > 0.f ? (mmax + __log2f(lsum)) * kLn2 : -INFINITY;
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

struct Plan {
  bool mfma = false;
  int part_tokens = 0;  // decode partition size (mfma path)
  int max_parts = 1;
  int64_t lse_bytes = 0, o_bytes = 0;
  int64_t workspace_bytes() const { return lse_bytes + o_bytes; }
};

static int64_t round_up(int64_t x, int64_t m) { return (x + m - 1) / m * m; }

static bool mfma_shape_ok(int64_t Hq, int64_t Hkv, int64_t D, int64_t bs, int dtype) {
  if (dtype != KVHOT_BF16 && dtype != KVHOT_F16) return false;
  if (D != 64 && D != 128 && D != 256) return false;
  if (bs % 16 != 0) return false;
  const int64_t G = Hq / Hkv;
  return G == 1 || G == 2 || G == 4 || G == 8 || G == 16;
}

// Decode partition size: the largest of 512/256/128/64 keys that still gives
// about 4096 (row, kv head, partition) waves over the batch.
static int pick_partition(int64_t rows, int64_t Hkv, int64_t max_k) {
  int pt = 512;
  while (pt > 64 && rows * Hkv * ((max_k + pt - 1) / pt) < 4096) pt /= 2;
  return pt;
}

static Plan make_plan(int64_t rows, int64_t max_q, int64_t max_k, int64_t Hq,
                      int64_t Hkv, int64_t D, int64_t bs, int64_t part_tokens,
                      int dtype) {
  Plan pl;
  pl.mfma = mfma_shape_ok(Hq, Hkv, D, bs, dtype);
  if (!pl.mfma || max_q < 1 || max_k < 1) return pl;
  pl.part_tokens = part_tokens > 0 ? static_cast<int>(part_tokens)
                                   : pick_partition(rows, Hkv, max_k);
  pl.max_parts = static_cast<int>((max_k + pl.part_tokens - 1) / pl.part_tokens);
  if (pl.max_parts > 65535) {
    pl.mfma = false;
    pl.max_parts = 1;
    return pl;
  }
  if (pl.max_parts > 1) {
    pl.lse_bytes = round_up(rows * Hq * pl.max_parts * 4, 256);
    pl.o_bytes = rows * Hq * pl.max_parts * D * 4;
  }
  return pl;
}

#ifndef KVHOT_DECODE_DB
#define KVHOT_DECODE_DB 1
#endif
constexpr bool kDecodeDB = KVHOT_DECODE_DB != 0;

template <class TT, int D>
static void launch_mfma(const AttnArgs& a, int64_t rows, int64_t max_q,
                        int max_parts_dec, hipStream_t stream) {
  // Decode rows: NM = 1, split-K.
  {
    AttnArgs d = a;
    d.role = 0;
    d.max_parts = max_parts_dec;
    dim3 grid(static_cast<uint32_t>(a.Hkv), static_cast<uint32_t>(max_parts_dec),
              static_cast<uint32_t>(rows));
    hipLaunchKernelGGL((attn_mfma_kernel<TT, D, 1, kDecodeDB>), grid, dim3(64), 0, stream, d);
    if (max_parts_dec > 1) {
      dim3 mgrid(static_cast<uint32_t>((a.Hq * (D / 8) + 255) / 256),
                 static_cast<uint32_t>(rows));
      hipLaunchKernelGGL((attn_merge_kernel<TT, D>), mgrid, dim3(256), 0, stream, d);
    }
  }
  if (max_q >= 2) {
    constexpr int NM = 4;
    AttnArgs pf = a;
    pf.role = 1;
    pf.max_parts = 1;
    pf.part_tokens = INT_MAX / 2;
    const int64_t qpw = 16 * NM / a.G;
    const int64_t nqb = (max_q + qpw - 1) / qpw;
    dim3 grid(static_cast<uint32_t>(a.Hkv * nqb), 1u, static_cast<uint32_t>(rows));
    hipLaunchKernelGGL((attn_mfma_kernel<TT, D, NM, false>), grid, dim3(64), 0, stream, pf);
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
  return pl.workspace_bytes();
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
    int64_t block_size, int64_t num_blocks, float scale, int is_causal,
    int dtype, int64_t partition_tokens, void* workspace,
    int64_t workspace_bytes, void* stream) {
  clear_error();
  const int64_t es = dtype_size(dtype);
  if (es == 0) return set_error(KVHOT_EINVAL, "paged_attention: bad dtype");
  if (num_rows < 0 || total_query < 0 || max_q_len < 0 || max_k_len < 0 ||
      num_q_heads <= 0 || num_kv_heads <= 0 || head_dim <= 0 || block_size <= 0 ||
      num_blocks < 0 || bt_row_stride < 0 || partition_tokens < 0)
    return set_error(KVHOT_EINVAL, "paged_attention: bad sizes");
  if (num_q_heads % num_kv_heads != 0)
    return set_error(KVHOT_EINVAL, "paged_attention: num_q_heads % num_kv_heads != 0");
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
      (partition_tokens % 32 != 0 || partition_tokens > 64 * block_size))
    return set_error(KVHOT_EINVAL,
                     "paged_attention: partition_tokens must be a multiple of 32 and <= 64*block_size");

  AttnArgs a{};
  a.q = q; a.q_st = q_strides[0]; a.q_sh = q_strides[1];
  a.k = k_cache; a.k_sb = k_cache_strides[0]; a.k_st = k_cache_strides[1]; a.k_sh = k_cache_strides[2];
  a.v = v_cache; a.v_sb = v_cache_strides[0]; a.v_st = v_cache_strides[1]; a.v_sh = v_cache_strides[2];
  a.o = out; a.o_st = out_strides[0]; a.o_sh = out_strides[1];
  a.lse = lse;
  a.l_st = lse ? lse_strides[0] : 0;
  a.l_sh = lse ? lse_strides[1] : 0;
  a.bt = block_table; a.bt_stride = bt_row_stride;
  a.q_lens = q_lens; a.k_lens = k_lens; a.q_starts = q_starts; a.q_offs = q_pos_offsets;
  a.num_blocks = num_blocks;
  a.Hq = static_cast<int32_t>(num_q_heads);
  a.Hkv = static_cast<int32_t>(num_kv_heads);
  a.G = static_cast<int32_t>(num_q_heads / num_kv_heads);
  a.bs = static_cast<int32_t>(block_size);
  a.scale_log2 = scale * kLog2e;
  a.causal = is_causal ? 1 : 0;
  a.D = static_cast<int32_t>(head_dim);
  a.total_q = total_query;
  a.max_parts = 1;
  hipStream_t s = static_cast<hipStream_t>(stream);

  Plan pl = make_plan(num_rows, max_q_len, max_k_len, num_q_heads, num_kv_heads, head_dim,
                      block_size, partition_tokens, dtype);
  if (pl.mfma) {
    // 16-byte vector loads/stores need 16-byte aligned rows.
    const int64_t al = 16 / es;
    const uintptr_t ptr_or = reinterpret_cast<uintptr_t>(q) | reinterpret_cast<uintptr_t>(k_cache) |
                             reinterpret_cast<uintptr_t>(v_cache) | reinterpret_cast<uintptr_t>(out);
    const int64_t str[10] = {a.q_st, a.q_sh, a.k_sb, a.k_st, a.k_sh,
                             a.v_sb, a.v_st, a.v_sh, a.o_st, a.o_sh};
    bool aligned = (ptr_or % 16) == 0;
    for (int64_t x : str) aligned = aligned && (x % al) == 0;
    if (!aligned) pl.mfma = false;
  }
  if (pl.mfma) {
    if (pl.max_parts > 1) {
      if (!workspace || workspace_bytes < pl.workspace_bytes())
        return set_error(KVHOT_EWORKSPACE,
                         "paged_attention: workspace of " + std::to_string(pl.workspace_bytes()) +
                             " bytes required");
      char* ws = static_cast<char*>(workspace);
      a.ws_lse = reinterpret_cast<float*>(ws);
      a.ws_o = reinterpret_cast<float*>(ws + pl.lse_bytes);
    }
    a.part_tokens = pl.part_tokens;
#define KVHOT_MFMA(TT, DD) launch_mfma<TT, DD>(a, num_rows, max_q_len, pl.max_parts, s)
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
  a.role = 2;
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
