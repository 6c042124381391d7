// Score tables for reference-format attention over coded segments (the
// score_tables mode of rfsn_ref_attention), gfx950.
//
// The exact path (ref_attention.hip) rebuilds every coded K and V vector in
// registers, as RFSNHybridAttentionMLX.__call__ (attention.py:150-171) does
// through the decode of quantization.py:310-319, and attends it.  Here the
// decode step's attention over the coded tokens is regrouped around the
// codebooks instead:
//
//   score(t) = sum over t's entries e of tab[e],   tab[e] = scale log2(e) q . c_e
//   out      = sum_e H[e] V_e / sum_t p_t,         H[e] = sum of p_t over tokens using V entry e
//
// with c_e every PQ entry (on its subspace's coordinates) and every gated
// RVQ codeword, p_t = 2^(score(t) - m) for the block's largest score m.
// Four launches:
//   ref_tab_scores_kernel  tab [BH][Ep] (v_mfma_f32_32x32x16_f16: 32 query
//                          heads x 32 entries per wave, K = 16 coordinates)
//   ref_tab_hist_kernel    one block per (query head, token split): the
//                          head's table in LDS, per token one LDS read per
//                          entry, then p into an integer histogram of the V
//                          entries (LDS u32 atomics, p in steps of 2^-19;
//                          fp32 LDS atomics run at a quarter of the u32 rate)
//   ref_tab_values_kernel  per 64-entry chunk: H over the splits (rescaled
//                          to a common maximum) times the chunk's V rows
//   ref_tab_out_kernel     per (query, KV head) group: the chunk sums, the
//                          drift estimate of each head, and the group's
//                          partial slot for merge_partials_kernel (empty
//                          when the group falls back to the exact decode)
// The fp16 rounding of the decoded K and V is skipped (tables and codebook
// products are fp32); the drift guard's estimate per query head is
//   scale sqrt(var s2) sqrt(Q) / L * 2 vmax      (K rounding -> scores)
// + sqrt(Q) / L * sqrt(var Wv)                   (V rounding)
// + sqrt(QE) / L * vmax                          (fixed-point steps)
// with var = 2^-20 / 12 (uniform rounding of at most 2^-10 |x|), s2 =
// sum_i q_i^2 WK_i, Q = sum p^2, L = sum p, QE = sum (p~ - p)^2 over the
// tokens, WK / WV / vmax from rfsn_ref_table_stats.
#include "rfsn_common.h"
#include "rfsn_internal.h"

#include <type_traits>

namespace rfsn {
namespace {

typedef _Float16 th8 __attribute__((ext_vector_type(8)));
typedef float tf16 __attribute__((ext_vector_type(16)));
typedef const rfsn_ref_segment __attribute__((address_space(4)))* tcref;

constexpr int kChunk = 64;           // codebook entries per chunk (within one section)
constexpr int kHistThreads = 1024;
constexpr int kHistWaves = kHistThreads / 64;  // red[] holds 4 values per wave: 64 floats
constexpr int kHistF = 19;           // fraction bits of the fixed-point weights
constexpr int kMaxHistSplits = 256;  // token splits per query head
constexpr float kTabDriftVar = 1.0f / (12.0f * 1048576.0f);

// tokens per thread of a histogram block (its codes stay in registers from
// the score pass to the histogram pass)
constexpr int hist_tokens(int M) { return M <= 8 ? 4 : (M == 16 ? 2 : 1); }

__device__ __forceinline__ _Float16 hbits(uint16_t b) { return __builtin_bit_cast(_Float16, b); }

// chunk c -> (section, first entry, entries): M PQ sections of C entries,
// then L gated layers of Cr entries, each cut into chunks of 64
__host__ __device__ __forceinline__ void chunk_of(const RefTabGeom& g, int c, int& sec, int& e0, int& n) {
  if (c < g.M * g.cpq) {
    sec = c / g.cpq;
    const int k = c - sec * g.cpq;
    e0 = sec * g.C + k * kChunk;
    n = min(kChunk, g.C - k * kChunk);
  } else {
    const int c2 = c - g.M * g.cpq, l = c2 / g.crv, k = c2 - l * g.crv;
    sec = g.M + l;
    e0 = g.M * g.C + l * g.Cr + k * kChunk;
    n = min(kChunk, g.Cr - k * kChunk);
  }
}

// tab[bh][e] = scale2 q_bh . c_e for the chunk's entries and 32 query heads
// bh0 ..: wave w takes entries 32 w .. 32 w + 31 of the chunk; A = 32 query
// rows (lane (i, hi) holds q[bh0 + i][16 st + 8 hi .. + 7]), B = 32 entry
// rows; D[i][j] sits in lane j + 32 hi, register r, i = 8 (r / 4) + 4 hi + r % 4.
template <int D>
__global__ void __launch_bounds__(128) ref_tab_scores_kernel(const uint16_t* __restrict__ q, int BH,
                                                             const uint16_t* __restrict__ pq_cb,
                                                             const uint16_t* __restrict__ rvq_cb, RefTabGeom g,
                                                             float scale2, float* __restrict__ tab) {
  int sec, e0, n;
  chunk_of(g, blockIdx.x, sec, e0, n);
  const int bh0 = blockIdx.y * 32;
  const int lane = threadIdx.x & 63, col = lane & 31, hi = lane >> 5;
  const int j = 32 * (threadIdx.x >> 6) + col;
  const bool ent = j < n;
  const int qa = bh0 + col;
  const bool pq = sec < g.M;
  const int lo = pq ? sec * g.dsub : 0;
  // PQ entries are zero outside their subspace: only its K steps
  const int st0 = pq ? lo / 16 : 0, st1 = pq ? (lo + g.dsub + 15) / 16 : D / 16;
  const uint16_t* row = !ent ? nullptr
                        : pq ? pq_cb + (int64_t)(e0 + j) * g.dsub
                             : rvq_cb + (int64_t)(e0 + j - g.M * g.C) * D;
  tf16 acc = {};
  for (int st = st0; st < st1; ++st) {
    const int d0 = 16 * st + 8 * hi;
    th8 a, b;
    if (qa < BH && reinterpret_cast<uintptr_t>(q) % 16 == 0) {  // uniform alignment: one 16-byte load
      const uint4 w = *reinterpret_cast<const uint4*>(q + (int64_t)qa * D + d0);
      const uint32_t ww[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
      for (int u = 0; u < 8; ++u) a[u] = hbits((uint16_t)(ww[u >> 1] >> (16 * (u & 1))));
    } else if (qa < BH) {
#pragma unroll
      for (int u = 0; u < 8; ++u) a[u] = hbits(q[(int64_t)qa * D + d0 + u]);
    } else {
#pragma unroll
      for (int u = 0; u < 8; ++u) a[u] = (_Float16)0.0f;
    }
#pragma unroll
    for (int u = 0; u < 8; ++u) b[u] = (_Float16)0.0f;
    if (ent) {
      if (!pq) {
        // gated rows: 8-byte aligned codebook, d0 a multiple of 8
        const uint2 w0 = *reinterpret_cast<const uint2*>(row + d0);
        const uint2 w1 = *reinterpret_cast<const uint2*>(row + d0 + 4);
        const uint32_t w[4] = {w0.x, w0.y, w1.x, w1.y};
#pragma unroll
        for (int u = 0; u < 8; ++u) b[u] = hbits((uint16_t)(w[u >> 1] >> (16 * (u & 1))));
      } else if (g.dsub % 8 == 0) {
        // the 8 coordinates are all inside the subspace or all outside it
        if (d0 >= lo && d0 < lo + g.dsub) {
          const uint4 w = *reinterpret_cast<const uint4*>(row + (d0 - lo));
          const uint32_t ww[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
          for (int u = 0; u < 8; ++u) b[u] = hbits((uint16_t)(ww[u >> 1] >> (16 * (u & 1))));
        }
      } else {
#pragma unroll
        for (int u = 0; u < 8; ++u) {
          const int dd = d0 + u;
          if (dd >= lo && dd < lo + g.dsub) b[u] = hbits(row[dd - lo]);
        }
      }
    }
    acc = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, acc, 0, 0, 0);
  }
  if (!ent) return;
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    const int bh = bh0 + 8 * (r >> 2) + 4 * hi + (r & 3);
    const float z = acc[r];
    if (bh < BH) tab[(int64_t)bh * g.Ep + blockIdx.x * kChunk + j] = scale2 * z;
  }
}

// The gated stage of a segment's K or V codes, as the histogram kernel
// loads them: none, dense rows (row r's codes are row r), an active map, or
// anything else (codes not in 8-byte aligned groups of 4 layers; blocks over
// segments of different kinds), which takes the per-token loads.
constexpr int kGNone = 0, kGDense = 1, kGMapped = 2, kGMixed = 3;
__device__ __forceinline__ int gated_kind(const int32_t* act, const uint16_t* rvq, int L) {
  if (rvq == nullptr) return act ? kGMixed : kGNone;
  if (L % 4 != 0 || reinterpret_cast<uintptr_t>(rvq) % 8 != 0) return kGMixed;
  return act ? kGMapped : kGDense;
}
__device__ __forceinline__ int merge_kind(int a, int b) { return a < 0 || a == b ? b : kGMixed; }

// row of (store token t, KV head h) in a coded segment's arrays: its code
// strides, or (both 0) the stores' [T][heads] order
__device__ __forceinline__ int64_t code_row(int64_t cts, int64_t chs, int64_t t, int h, int kv_heads) {
  return (cts | chs) == 0 ? t * kv_heads + h : t * cts + h * chs;
}

// The window's coded tokens, in window order, split S ways per query head
// (S a multiple of 8); BH * S blocks, each one (query head row bh, split).
// A thread holds KT tokens: their codes, then their scores.
// pst[bh][split] = {m, L, Q, QE}: m the block's largest score (base 2), L =
// sum p, Q = sum p^2, QE = sum (p~ - p)^2 (p~ = p rounded to 2^-19); hbuf
// [chunk][bh][split][64]: H[e] = sum of p~ over the tokens whose V uses entry
// e, chunk-major so that a chunk's sums over every head and split are one
// contiguous run for ref_tab_values_kernel.
template <int M, int LQ>
__global__ void __launch_bounds__(kHistThreads) ref_tab_hist_kernel(const rfsn_ref_params p, RefTabGeom g, int S,
                                                                    const float* __restrict__ tab,
                                                                    float* __restrict__ pst,
                                                                    float* __restrict__ hbuf) {
  constexpr int KT = hist_tokens(M);
  constexpr int MW = M / 4;  // code words per token
  extern __shared__ __align__(16) float tsm[];
  float* tl = tsm;                                          // [Ep] the head's table
  uint32_t* hist = reinterpret_cast<uint32_t*>(tsm + g.Ep);  // [Ep]
  float* red = tsm + 2 * g.Ep;                              // [64]
  const tcref segs = (tcref)p.segments;
  // Blocks run on XCD blockIdx.x % 8.  Over head-major codes (every coded
  // segment with code strides) the blocks of a (query, KV head) unit share an
  // XCD when there are a multiple of 8 units -- its L2 then holds the unit's
  // codes once for its G query heads and each head's table once for its S
  // splits (blockIdx.x = (split G + g) NKV + unit) -- else those of a query
  // head (blockIdx.x = split BH + bh).  Over the stores' own [T][heads] codes
  // the blocks of a split share one, and with them the 128-byte lines of the
  // split's codes (blockIdx.x = bh S + split).
  int coded = 0;
  bool head_rows = true;
  for (int s = 0; s < p.num_segments; ++s)
    if (segs[s].k.pq != nullptr) {
      coded += segs[s].len;
      head_rows = head_rows && (segs[s].code_token_stride | segs[s].code_head_stride) != 0;
    }
  const int G = p.q_heads / p.kv_heads;
  const int NKV = p.batch * p.kv_heads, BHn = p.batch * p.q_heads;
  int bh, split;
  if (head_rows && NKV % 8 == 0) {
    const int t = (int)blockIdx.x / NKV;
    bh = ((int)blockIdx.x % NKV) * G + t % G;
    split = t / G;
  } else if (head_rows) {
    bh = (int)blockIdx.x % BHn;
    split = (int)blockIdx.x / BHn;
  } else {
    bh = (int)blockIdx.x / S;
    split = (int)blockIdx.x % S;
  }
  const int hq = bh % p.q_heads, h = hq / G;
  const int qp = (p.causal && p.qpos) ? p.qpos[bh] : 0x7fffffff;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  // chunk-space indices: section s starts at chunk boundary (PQ sections of
  // Cp = 64 ceil(C / 64) slots, then gated layers of Crp = 64 ceil(Cr / 64))
  const int C = g.C, Cr = g.Cr, L = g.L, Cp = g.cpq * kChunk, Crp = g.crv * kChunk, MC = g.M * Cp;

  // stage the table, zero the histogram (Ep is a multiple of 4)
  {
    const float4* src = reinterpret_cast<const float4*>(tab + (int64_t)bh * g.Ep);
    const int n4 = g.Ep / 4;
    for (int i0 = threadIdx.x; i0 < n4; i0 += 8 * kHistThreads) {
      float4 v[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        const int i = i0 + u * kHistThreads;
        v[u] = i < n4 ? src[i] : make_float4(0.f, 0.f, 0.f, 0.f);
      }
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        const int i = i0 + u * kHistThreads;
        if (i < n4) {
          reinterpret_cast<float4*>(tl)[i] = v[u];
          reinterpret_cast<uint4*>(hist)[i] = make_uint4(0u, 0u, 0u, 0u);
        }
      }
    }
  }

  const int tps = (coded + S - 1) / S;
  const int ci0 = min(coded, split * tps), ci1 = min(coded, ci0 + tps);

  // codes of the thread's tokens ci0 + threadIdx.x + kHistThreads u.  A wave-uniform
  // walk over the segments (scalar loads of their fields) finds each token's
  // segment; the code loads follow in straight-line code, reading segment
  // fields as scalars where the wave's tokens share one segment, so a thread
  // issues the loads of all its tokens before its first wait.  (A per-token
  // walk read the fields with vector loads and waited on them: one memory
  // round trip per token.)
  uint32_t kc[KT][MW], vc[KT][MW];
  int ka[KT], va[KT], sg[KT], tt[KT];
  bool live[KT];
  // the gated codes of the active rows: LQ groups of 4 layers (u16 each),
  // read only where ka / va >= 0 (so they need no initial value: a zero
  // merged across the map / dense branches made the compiler wait on loads)
  constexpr int LQ1 = LQ > 0 ? LQ : 1;
  uint2 kr[KT][LQ1], vr[KT][LQ1];
  int kam[KT], vam[KT];  // active-map entries of the fast tokens
#pragma unroll
  for (int u = 0; u < KT; ++u) {
    live[u] = false;
    ka[u] = va[u] = -1;
    sg[u] = tt[u] = 0;
#pragma unroll
    for (int w = 0; w < MW; ++w) kc[u][w] = vc[u][w] = 0u;
  }
  // the gated stage of the block's segments, K and V (uniform): kGNone,
  // kGDense, kGMapped, or kGMixed (mixed kinds, or codes not in 8-byte
  // aligned groups of 4 layers)
  int kkind = LQ > 0 ? -1 : kGNone, vkind = LQ > 0 ? -1 : kGNone;
  {
    int cpre = 0;  // coded tokens before segment s
    for (int s = 0; s < p.num_segments && cpre < ci1; ++s) {
      if (segs[s].k.pq == nullptr) continue;
      const int lo = cpre;
      cpre += segs[s].len;
      if (cpre <= ci0) continue;  // before the block's tokens
      if constexpr (LQ > 0) {
        kkind = merge_kind(kkind, gated_kind(segs[s].k.active, segs[s].k.rvq, L));
        vkind = merge_kind(vkind, gated_kind(segs[s].v.active, segs[s].v.rvq, L));
      }
      const int pos0 = segs[s].pos0;
#pragma unroll
      for (int u = 0; u < KT; ++u) {
        const int ci = ci0 + (int)threadIdx.x + u * kHistThreads;
        const int t = ci - lo, pos = pos0 + t;
        if (ci >= lo && ci < cpre && ci < ci1 && pos >= 0 && pos <= qp) {  // else outside or masked
          live[u] = true;
          sg[u] = s;
          tt[u] = t;
        }
      }
    }
  }
  // Fast issue, straight-line and specialized on the block's gated kinds:
  // token u of every lane of the wave, where the wave's live tokens u share
  // one segment s0 (scalar fields).  The rest goes per token below.
  bool done[KT];
  int s0u[KT];  // uniform: the fast segment of token u, or -1
#pragma unroll
  for (int u = 0; u < KT; ++u) {
    done[u] = !live[u];
    s0u[u] = -1;
  }
  auto fast = [&](auto kk, auto vk) __attribute__((always_inline)) {
    constexpr int KK = decltype(kk)::value, VK = decltype(vk)::value;
#pragma unroll
    for (int u = 0; u < KT; ++u) {
      const uint64_t lm = __ballot(live[u]);
      if (lm == 0) continue;
      const int s0 = __builtin_amdgcn_readlane(sg[u], __builtin_ctzll(lm));
      if (__ballot(live[u] && sg[u] != s0) != 0) continue;
      s0u[u] = s0;
      done[u] = true;
      if (!live[u]) continue;
      const int64_t row = code_row(segs[s0].code_token_stride, segs[s0].code_head_stride, segs[s0].token0 + tt[u], h, p.kv_heads);
      const uint32_t* kp = reinterpret_cast<const uint32_t*>(segs[s0].k.pq + row * M);
      const uint32_t* vp = reinterpret_cast<const uint32_t*>(segs[s0].v.pq + row * M);
#pragma unroll
      for (int w = 0; w < MW; ++w) {
        kc[u][w] = kp[w];
        vc[u][w] = vp[w];
      }
      // dense rows: row r's gated codes are row r; an active map: read here,
      // its rows' codes load below
      if constexpr (KK == kGDense) {
        ka[u] = (int)row;
#pragma unroll
        for (int k = 0; k < LQ1; ++k) kr[u][k] = *reinterpret_cast<const uint2*>(segs[s0].k.rvq + row * L + 4 * k);
      } else if constexpr (KK == kGMapped) {
        kam[u] = segs[s0].k.active[row];
      }
      if constexpr (VK == kGDense) {
        va[u] = (int)row;
#pragma unroll
        for (int k = 0; k < LQ1; ++k) vr[u][k] = *reinterpret_cast<const uint2*>(segs[s0].v.rvq + row * L + 4 * k);
      } else if constexpr (VK == kGMapped) {
        vam[u] = segs[s0].v.active[row];
      }
    }
    if constexpr (KK == kGMapped || VK == kGMapped) {  // one round trip after the maps
#pragma unroll
      for (int u = 0; u < KT; ++u) {
        const int s0 = s0u[u];
        if (s0 < 0 || !live[u]) continue;
        if constexpr (KK == kGMapped) {
          ka[u] = kam[u];
          if (ka[u] >= 0) {
#pragma unroll
            for (int k = 0; k < LQ1; ++k)
              kr[u][k] = *reinterpret_cast<const uint2*>(segs[s0].k.rvq + (int64_t)ka[u] * L + 4 * k);
          }
        }
        if constexpr (VK == kGMapped) {
          va[u] = vam[u];
          if (va[u] >= 0) {
#pragma unroll
            for (int k = 0; k < LQ1; ++k)
              vr[u][k] = *reinterpret_cast<const uint2*>(segs[s0].v.rvq + (int64_t)va[u] * L + 4 * k);
          }
        }
      }
    }
  };
  using G0 = std::integral_constant<int, kGNone>;
  using G1 = std::integral_constant<int, kGDense>;
  using G2 = std::integral_constant<int, kGMapped>;
  auto fast_v = [&](auto kk) __attribute__((always_inline)) {
    if (vkind == kGNone) fast(kk, G0{});
    else if (vkind == kGDense) fast(kk, G1{});
    else if (vkind == kGMapped) fast(kk, G2{});
  };
  if (LQ == 0 || kkind == kGNone) fast_v(G0{});
  else if (kkind == kGDense) fast_v(G1{});
  else if (kkind == kGMapped) fast_v(G2{});
  // The rest, per token (a wave whose tokens u span segments; gated codes
  // not in aligned groups of 4), after every fast load is issued.
  bool rest = false;
#pragma unroll
  for (int u = 0; u < KT; ++u) rest |= !done[u];
  if (__ballot(rest) != 0) {
#pragma unroll
    for (int u = 0; u < KT; ++u) {
      if (done[u]) continue;
      const int sx = sg[u];
      const int64_t row = code_row(segs[sx].code_token_stride, segs[sx].code_head_stride, segs[sx].token0 + tt[u], h, p.kv_heads);
      const uint32_t* kp = reinterpret_cast<const uint32_t*>(segs[sx].k.pq + row * M);
      const uint32_t* vp = reinterpret_cast<const uint32_t*>(segs[sx].v.pq + row * M);
#pragma unroll
      for (int w = 0; w < MW; ++w) {
        kc[u][w] = kp[w];
        vc[u][w] = vp[w];
      }
      if constexpr (LQ > 0) {
        const int32_t* kact = segs[sx].k.active;
        const int32_t* vact = segs[sx].v.active;
        ka[u] = kact ? kact[row] : segs[sx].k.rvq ? (int)row : -1;
        va[u] = vact ? vact[row] : segs[sx].v.rvq ? (int)row : -1;
#pragma unroll
        for (int pass = 0; pass < 2; ++pass) {
          const int a = pass ? va[u] : ka[u];
          if (a < 0) continue;
          const uint16_t* rc = (pass ? segs[sx].v.rvq : segs[sx].k.rvq) + (int64_t)a * L;
          uint2 w[LQ];
          if (L % 4 == 0 && reinterpret_cast<uintptr_t>(rc) % 8 == 0) {
#pragma unroll
            for (int k = 0; k < LQ; ++k) w[k] = *reinterpret_cast<const uint2*>(rc + 4 * k);
          } else {
#pragma unroll
            for (int k = 0; k < LQ; ++k) {
              uint32_t x[2] = {0u, 0u};
#pragma unroll
              for (int j = 0; j < 4; ++j)
                if (4 * k + j < L) x[j >> 1] |= (uint32_t)rc[4 * k + j] << (16 * (j & 1));
              w[k] = make_uint2(x[0], x[1]);
            }
          }
#pragma unroll
          for (int k = 0; k < LQ; ++k) {
            if (pass)
              vr[u][k] = w[k];
            else
              kr[u][k] = w[k];
          }
        }
      }
    }
  }
  __syncthreads();  // the table is staged

  // scores; codes past the codebook sizes are clamped (codes are < C, < C_r)
  float sc[KT];
  float mx = -__builtin_inff();
#pragma unroll
  for (int u = 0; u < KT; ++u) {
    float x = 0.f;
#pragma unroll
    for (int m = 0; m < M; ++m) x += tl[m * Cp + min((int)((kc[u][m >> 2] >> (8 * (m & 3))) & 0xFFu), C - 1)];
    if constexpr (LQ > 0) {
      if (ka[u] >= 0) {
#pragma unroll
        for (int l = 0; l < 4 * LQ; ++l) {
          if (l >= L) break;
          const uint32_t w = (l & 2) ? kr[u][l >> 2].y : kr[u][l >> 2].x;
          x += tl[MC + l * Crp + min((int)((w >> (16 * (l & 1))) & 0xFFFFu), Cr - 1)];
        }
      }
    }
    sc[u] = live[u] ? x : -__builtin_inff();
    mx = fmaxf(mx, sc[u]);
  }
  mx = wave_max(mx);
  if (lane == 0) red[wave] = mx;
  __syncthreads();
  mx = red[0];
#pragma unroll
  for (int w = 1; w < kHistWaves; ++w) mx = fmaxf(mx, red[w]);

  float ls = 0.f, q2 = 0.f, qe = 0.f;
  if (mx > -__builtin_inff()) {  // uniform
#pragma unroll
    for (int u = 0; u < KT; ++u) {
      if (!(sc[u] > -__builtin_inff())) continue;
      const float pr = exp2f(sc[u] - mx);
      const uint32_t qi = __float2uint_rn(pr * (float)(1 << kHistF));
      const float d = (float)qi * (1.0f / (float)(1 << kHistF)) - pr;
      ls += pr;
      q2 += pr * pr;
      qe += d * d;
#pragma unroll
      for (int m = 0; m < M; ++m)
        atomicAdd(&hist[m * Cp + min((int)((vc[u][m >> 2] >> (8 * (m & 3))) & 0xFFu), C - 1)], qi);
      if constexpr (LQ > 0) {
        if (va[u] >= 0) {
#pragma unroll
          for (int l = 0; l < 4 * LQ; ++l) {
            if (l >= L) break;
            const uint32_t w = (l & 2) ? vr[u][l >> 2].y : vr[u][l >> 2].x;
            atomicAdd(&hist[MC + l * Crp + min((int)((w >> (16 * (l & 1))) & 0xFFFFu), Cr - 1)], qi);
          }
        }
      }
    }
  }
  ls = wave_sum(ls);
  q2 = wave_sum(q2);
  qe = wave_sum(qe);
  __syncthreads();  // every histogram add is done; red is read
  if (lane == 0) {
    red[kHistWaves + wave] = ls;
    red[2 * kHistWaves + wave] = q2;
    red[3 * kHistWaves + wave] = qe;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    float a = 0.f, b2 = 0.f, c2 = 0.f;
    for (int w = 0; w < kHistWaves; ++w) {
      a += red[kHistWaves + w];
      b2 += red[2 * kHistWaves + w];
      c2 += red[3 * kHistWaves + w];
    }
    *reinterpret_cast<float4*>(pst + ((int64_t)bh * S + split) * 4) = make_float4(mx, a, b2, c2);
  }
  // the sums in chunk space are [chunk][64]: 16-byte units, unit u = chunk
  // u / 16, entries 4 (u % 16) ..; slots past a section's end hold zeros
  constexpr float f = 1.0f / (float)(1 << kHistF);
  const int64_t BH = (int64_t)p.batch * p.q_heads;
  for (int u = threadIdx.x; u < g.nch * (kChunk / 4); u += kHistThreads) {
    const int c = u / (kChunk / 4), j4 = u - c * (kChunk / 4);
    const uint4 hv = reinterpret_cast<const uint4*>(hist)[u];
    reinterpret_cast<float4*>(hbuf + ((c * BH + bh) * S + split) * kChunk)[j4] =
        make_float4((float)hv.x * f, (float)hv.y * f, (float)hv.z * f, (float)hv.w * f);
  }
}

// part2[c][bh][d] = sum over chunk c's entries e of H_bh[e] V_e[d], H_bh =
// sum over splits k of 2^(m_k - max m) H_k.  Block: chunk x 32 query heads,
// 2 D threads (D / 32 waves).  The chunk's V rows, its first 8 splits' sums
// (one contiguous run of [32][S][64], 16-byte units) and the split maxima
// load together; the first 32 threads turn the maxima into weights; further
// splits load 8 at a time.  The product runs on v_mfma_f32_32x32x16_f16, wave
// w taking coordinates 32 w .. 32 w + 31: A = H of the 32 heads, 16 entries
// per step, as fp16 hi + lo of s_bh H (s_bh a power of 2 that puts the head's
// largest sum of the chunk in [2^14, 2^15); hi + lo holds 22 bits of it), B =
// the V rows (fp16, exact), and the fp32 result is divided by s_bh.
constexpr int kValHs = kChunk + 4;  // LDS row of a head's sums (floats; +4: rows start 4 banks apart)
constexpr int kValRt = kChunk + 8;  // LDS row of a coordinate's V entries (halves; +8: 4 banks apart)
template <int D>
constexpr size_t values_lds_bytes(int S) {
  return ((size_t)32 * kValHs + 32 + 32 * S) * sizeof(float) + (size_t)D * kValRt * sizeof(uint16_t);
}

template <int D, int HB>
__global__ void __launch_bounds__(D * HB / 16) ref_tab_values_kernel(const float* __restrict__ pst,
                                                               const float* __restrict__ hbuf, int S, int BH,
                                                               const uint16_t* __restrict__ pq_cb,
                                                               const uint16_t* __restrict__ rvq_cb, RefTabGeom g,
                                                               float* __restrict__ part2) {
  static_assert(HB == 32, "the query heads are the 32 rows of one MFMA tile");
  constexpr int NT = D * HB / 16;  // 2 D: D / 32 waves of 32 coordinates
  constexpr int RU = kChunk * (D / 4) / NT;  // 4-coordinate units of the rows per thread (8)
  constexpr int HU = HB * (kChunk / 4) / NT;  // (head, 4 entries) units per thread: 256 / D
  extern __shared__ __align__(16) float vsm[];
  float* hs = vsm;                     // [HB][kValHs] scaled sums
  float* hinv = hs + HB * kValHs;      // [HB] 1 / s_bh
  float* wk = hinv + HB;               // [HB][S]
  uint16_t* rt = reinterpret_cast<uint16_t*>(wk + HB * S);  // [D][kValRt] fp16 V rows, transposed
  int sec, e0, n;
  chunk_of(g, blockIdx.x, sec, e0, n);
  const int bh0 = blockIdx.y * HB;
  const bool pq = sec < g.M;
  const int lo = pq ? sec * g.dsub : 0;

  // V rows in units of 4 coordinates (8 bytes): gated rows (8-byte aligned
  // codebook), PQ rows on their subspace when it holds whole units (dsub a
  // multiple of 4; 16-byte aligned codebook), zeros elsewhere
  const bool pq4 = pq && g.dsub % 4 == 0;
  uint2 rw[RU];
  if (!pq || pq4) {
#pragma unroll
    for (int u = 0; u < RU; ++u) {
      const int idx = threadIdx.x + u * NT, j = idx / (D / 4), c4 = idx - j * (D / 4);
      const int dd = 4 * c4;
      const uint16_t* src = !pq ? rvq_cb + (int64_t)(e0 + j - g.M * g.C) * D + dd
                                : pq_cb + (int64_t)(e0 + j) * g.dsub + (dd - lo);
      rw[u] = j < n && (!pq || (dd >= lo && dd < lo + g.dsub)) ? *reinterpret_cast<const uint2*>(src)
                                                                : make_uint2(0u, 0u);
    }
  }
  // the first 8 splits' sums: unit (r, j4) = entries 4 j4 .. 4 j4 + 3 of head row r
  const float4* hsrc = reinterpret_cast<const float4*>(hbuf + ((int64_t)blockIdx.x * BH + bh0) * S * kChunk);
  float4 x[HU][8];
  auto load_h = [&](int k0) __attribute__((always_inline)) {
#pragma unroll
    for (int a = 0; a < HU; ++a) {
      const int i = threadIdx.x + a * NT, r = i / (kChunk / 4), j4 = i - r * (kChunk / 4);
      const bool ok = bh0 + r < BH && 4 * j4 < n;
#pragma unroll
      for (int u = 0; u < 8; ++u)
        x[a][u] = ok && k0 + u < S ? hsrc[((int64_t)r * S + k0 + u) * (kChunk / 4) + j4] : make_float4(0.f, 0.f, 0.f, 0.f);
    }
  };
  load_h(0);
  // split weights of head row r = threadIdx.x < HB
  if (threadIdx.x < HB) {
    const int r = threadIdx.x;
    const float* src = pst + (int64_t)(bh0 + r) * S * 4;
    float mx = -__builtin_inff();
    if (bh0 + r < BH)
      for (int k = 0; k < S; ++k) mx = fmaxf(mx, src[4 * k]);
    for (int k = 0; k < S; ++k) {
      const float m = bh0 + r < BH ? src[4 * k] : -__builtin_inff();
      wk[r * S + k] = m > -__builtin_inff() ? exp2f(m - mx) : 0.f;
    }
  }
  if (!pq || pq4) {
#pragma unroll
    for (int u = 0; u < RU; ++u) {
      const int idx = threadIdx.x + u * NT, j = idx / (D / 4), c4 = idx - j * (D / 4);
      uint16_t* col = rt + (4 * c4) * kValRt + j;
      col[0] = (uint16_t)rw[u].x;
      col[kValRt] = (uint16_t)(rw[u].x >> 16);
      col[2 * kValRt] = (uint16_t)rw[u].y;
      col[3 * kValRt] = (uint16_t)(rw[u].y >> 16);
    }
  } else {
    // 2-wide PQ subspaces: the subspace's coordinates, zero elsewhere
    for (int i = threadIdx.x; i < kChunk * D; i += NT) {
      const int j = i / D, dd = i - j * D;
      rt[dd * kValRt + j] = (j < n && dd >= lo && dd < lo + g.dsub) ? pq_cb[(int64_t)(e0 + j) * g.dsub + (dd - lo)]
                                                                     : (uint16_t)0;
    }
  }
  __syncthreads();
  // H over the splits: unit (r, j4) = entries 4 j4 .. 4 j4 + 3 of head row r,
  // r's 16 units in 16 consecutive lanes
  {
    float4 v[HU];
#pragma unroll
    for (int a = 0; a < HU; ++a) v[a] = make_float4(0.f, 0.f, 0.f, 0.f);
    for (int k0 = 0; k0 < S; k0 += 8) {
      if (k0 > 0) load_h(k0);
#pragma unroll
      for (int a = 0; a < HU; ++a) {
        const int r = (threadIdx.x + a * NT) / (kChunk / 4);
#pragma unroll
        for (int u = 0; u < 8; ++u) {
          if (k0 + u >= S) break;
          const float w = wk[r * S + k0 + u];
          v[a].x = __builtin_fmaf(w, x[a][u].x, v[a].x);
          v[a].y = __builtin_fmaf(w, x[a][u].y, v[a].y);
          v[a].z = __builtin_fmaf(w, x[a][u].z, v[a].z);
          v[a].w = __builtin_fmaf(w, x[a][u].w, v[a].w);
        }
      }
    }
#pragma unroll
    for (int a = 0; a < HU; ++a) {
      const int i = threadIdx.x + a * NT, r = i / (kChunk / 4), j4 = i - r * (kChunk / 4);
      // entries past the chunk's n hold stale values: zero them
      float4 h = v[a];
      h.x = 4 * j4 + 0 < n ? h.x : 0.f;
      h.y = 4 * j4 + 1 < n ? h.y : 0.f;
      h.z = 4 * j4 + 2 < n ? h.z : 0.f;
      h.w = 4 * j4 + 3 < n ? h.w : 0.f;
      // the head's largest sum (sums are >= 0) and its scale 2^(15 - e), with
      // largest = f 2^e, f in [0.5, 1): s H < 2^15, clamped to normal scales
      float mx = fmaxf(fmaxf(h.x, h.y), fmaxf(h.z, h.w));
#pragma unroll
      for (int o = 1; o < kChunk / 4; o <<= 1) mx = fmaxf(mx, __shfl_xor(mx, o, 64));
      int e = 0;
      (void)frexpf(mx, &e);
      const int k = mx > 0.f ? min(126, max(-126, 15 - e)) : 0;
      const float sc = ldexpf(1.0f, k);
      *reinterpret_cast<float4*>(hs + r * kValHs + 4 * j4) = make_float4(h.x * sc, h.y * sc, h.z * sc, h.w * sc);
      if (j4 == 0) hinv[r] = ldexpf(1.0f, -k);
    }
  }
  __syncthreads();
  {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int col = lane & 31, hi = lane >> 5;
    const int d = 32 * wave + col;
    tf16 acc = {};
#pragma unroll
    for (int st = 0; st < kChunk / 16; ++st) {
      const int e = 16 * st + 8 * hi;
      const float4 h0 = *reinterpret_cast<const float4*>(hs + col * kValHs + e);
      const float4 h1 = *reinterpret_cast<const float4*>(hs + col * kValHs + e + 4);
      const float hv[8] = {h0.x, h0.y, h0.z, h0.w, h1.x, h1.y, h1.z, h1.w};
      th8 ah, al;
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        ah[u] = (_Float16)hv[u];
        al[u] = (_Float16)(hv[u] - (float)ah[u]);
      }
      const th8 bv = __builtin_bit_cast(th8, *reinterpret_cast<const uint4*>(rt + d * kValRt + e));
      acc = __builtin_amdgcn_mfma_f32_32x32x16_f16(al, bv, acc, 0, 0, 0);
      acc = __builtin_amdgcn_mfma_f32_32x32x16_f16(ah, bv, acc, 0, 0, 0);
    }
    // D[i][j]: lane (j, hi), register r holds head i = 8 (r / 4) + 4 hi + r % 4, coordinate j
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int i = 8 * (r >> 2) + 4 * hi + (r & 3);
      if (bh0 + i < BH) part2[((int64_t)blockIdx.x * BH + bh0 + i) * D + d] = acc[r] * hinv[i];
    }
  }
}

// Block (query b, KV head h; tile y of 64 of the group's G D outputs): the
// tile's chunk sums (64 outputs x 16 chunk slices); every tile computes the
// G heads' split statistics and drift estimates (tile 0 writes them).  The
// group's partial slot (the last of `slots`) holds (m, L, sum) unless one
// head's estimate exceeds the tolerance: then the exact pass decodes the
// group's coded tokens and the slot is empty (m = -inf, L = 0, zeros).
template <int D>
__global__ void __launch_bounds__(1024) ref_tab_out_kernel(const rfsn_ref_params p, RefTabGeom g, int S, int nch,
                                                           const float* __restrict__ pst,
                                                           const float* __restrict__ part2, int slots,
                                                           float* __restrict__ partial, float* __restrict__ est) {
  __shared__ float red[1024];
  __shared__ float gm[8], gl[8], ge[8];
  const int G = p.q_heads / p.kv_heads;
  const int b = blockIdx.x / p.kv_heads, h = blockIdx.x % p.kv_heads;
  const int BH = p.batch * p.q_heads, bhb = b * p.q_heads + h * G;
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const int o = blockIdx.y * 64 + lane;  // output g D + c of the group
  const bool oo = o < G * D;
  {
    float v = 0.f;
    if (oo) {
      const float* src = part2 + (int64_t)bhb * D + o;
      // 24 chunks' loads in flight per thread: one round trip for up to 384 chunks
      for (int k = wave; k < nch; k += 16 * 24) {
        float x[24];
#pragma unroll
        for (int u = 0; u < 24; ++u) x[u] = k + 16 * u < nch ? src[(int64_t)(k + 16 * u) * BH * D] : 0.f;
#pragma unroll
        for (int u = 0; u < 24; ++u) v += x[u];
      }
    }
    red[t] = v;
  }
  // wave w < G: head w's split statistics and drift estimate
  if (wave < G) {
    const int bh = bhb + wave;
    float m = -__builtin_inff();
    for (int k = lane; k < S; k += 64) m = fmaxf(m, pst[((int64_t)bh * S + k) * 4]);
    m = wave_max(m);
    float Ls = 0.f, Q = 0.f, QE = 0.f;
    if (m > -__builtin_inff()) {
      for (int k = lane; k < S; k += 64) {
        const float* ps = pst + ((int64_t)bh * S + k) * 4;
        const float mk = ps[0];
        const float w = mk > -__builtin_inff() ? exp2f(mk - m) : 0.f;
        Ls += w * ps[1];
        Q += w * w * ps[2];
        QE += w * w * ps[3];
      }
    }
    Ls = wave_sum(Ls);
    Q = wave_sum(Q);
    QE = wave_sum(QE);
    const uint16_t* qrow = (const uint16_t*)p.q + (int64_t)bh * D;
    float s2 = 0.f, wv = 0.f, vm = 0.f;
    for (int i = lane; i < D; i += 64) {
      const float qv = h2f(qrow[i]);
      s2 += qv * qv * p.table_stats[i];
      wv = fmaxf(wv, p.table_stats[D + i]);
      vm = fmaxf(vm, p.table_stats[2 * D + i]);
    }
    s2 = wave_sum(s2);
    wv = wave_max(wv);
    vm = wave_max(vm);
    float e = 0.f;
    if (Ls > 0.f) {
      const float sq = sqrtf(Q) / Ls;
      e = p.scale * sqrtf(kTabDriftVar * s2) * sq * 2.f * vm + sq * sqrtf(kTabDriftVar * wv) + sqrtf(QE) / Ls * vm;
    }
    if (lane == 0) {
      gm[wave] = m;
      gl[wave] = Ls;
      ge[wave] = e;
      if (blockIdx.y == 0) {
        est[bh] = e;
        if (p.drift) p.drift[bh] = e;
      }
    }
  }
  __syncthreads();
  if (wave == 0 && oo) {
    float sum = 0.f;
#pragma unroll
    for (int k = 0; k < 16; ++k) sum += red[k * 64 + lane];
    bool exact = false;
    for (int j = 0; j < G; ++j) exact = exact || !(ge[j] <= p.table_tol);
    const int j = o / D, c = o - j * D;
    float* slot = partial + ((int64_t)(bhb + j) * slots + slots - 1) * (D + 2);
    const bool use = !exact && gl[j] > 0.f;
    if (c == 0) {
      slot[0] = use ? gm[j] : -__builtin_inff();
      slot[1] = use ? gl[j] : 0.f;
    }
    slot[2 + c] = use ? sum : 0.f;
  }
}

// stats[w][i]: see rfsn_ref_table_stats.  Block (codebook w in {K, V},
// coordinate i); 256 threads over the entries.
__global__ void __launch_bounds__(256) ref_tab_stats_kernel(const uint16_t* __restrict__ kpq,
                                                            const uint16_t* __restrict__ krvq,
                                                            const uint16_t* __restrict__ vpq,
                                                            const uint16_t* __restrict__ vrvq, RefTabGeom g,
                                                            float* __restrict__ stats) {
  __shared__ float red[3][4];
  const int w = blockIdx.x / g.D, i = blockIdx.x % g.D;
  const uint16_t* pq = w ? vpq : kpq;
  const uint16_t* rv = w ? vrvq : krvq;
  const int m = i / g.dsub, ii = i - m * g.dsub;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  auto block3 = [&](float a, float b2, float c2) {
    a = wave_sum(a);
    b2 = wave_max(b2);
    c2 = wave_sum(c2);
    if (lane == 0) {
      red[0][wave] = a;
      red[1][wave] = b2;
      red[2][wave] = c2;
    }
    __syncthreads();
    float3 r = make_float3(0.f, 0.f, 0.f);
    for (int k = 0; k < 4; ++k) {
      r.x += red[0][k];
      r.y = fmaxf(r.y, red[1][k]);
      r.z += red[2][k];
    }
    __syncthreads();
    return r;
  };
  float s = 0.f, mx = 0.f;
  for (int c = threadIdx.x; c < g.C; c += 256) {
    const float x = h2f(pq[((int64_t)m * g.C + c) * g.dsub + ii]);
    s += x * x;
    mx = fmaxf(mx, fabsf(x));
  }
  const float3 rp = block3(s, mx, 0.f);
  float wsum = rp.x / (float)g.C, vmax = rp.y;
  for (int l = 0; l < g.L; ++l) {
    float s2 = 0.f, m2 = 0.f;
    for (int c = threadIdx.x; c < g.Cr; c += 256) {
      const float x = h2f(rv[((int64_t)l * g.Cr + c) * g.D + i]);
      s2 += x * x;
      m2 = fmaxf(m2, fabsf(x));
    }
    const float3 rl = block3(s2, m2, 0.f);
    wsum += 2.f * rl.x / (float)g.Cr;
    vmax += rl.y;
  }
  if (threadIdx.x == 0) {
    stats[w * g.D + i] = wsum;
    if (w) stats[2 * g.D + i] = vmax;
  }
}

template <int M>
int launch_hist(const rfsn_ref_params* p, const RefTabGeom& g, int S, const float* tab, float* pst, float* hbuf,
                hipStream_t s) {
  const size_t lds = ((size_t)2 * g.Ep + 64) * sizeof(float);
  const int BH = p->batch * p->q_heads;
  auto kern = g.L == 0 ? ref_tab_hist_kernel<M, 0> : g.L <= 4 ? ref_tab_hist_kernel<M, 1> : ref_tab_hist_kernel<M, 2>;
  (void)hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
  hipLaunchKernelGGL(kern, dim3((unsigned)(BH * S)), dim3(kHistThreads), lds, s, *p, g, S, tab, pst, hbuf);
  return check_launch("ref_tables hist");
}

template <int D>
int launch_tables_d(const rfsn_ref_params* p, const RefTabGeom& g, const RefTabLayout& w, hipStream_t s) {
  const int BH = p->batch * p->q_heads, S = w.hist_splits;
  const dim3 cg((unsigned)g.nch, (unsigned)((BH + 31) / 32));
  const float scale2 = p->scale * 1.4426950408889634f;
  hipLaunchKernelGGL(ref_tab_scores_kernel<D>, cg, dim3(128), 0, s, (const uint16_t*)p->q, BH,
                     (const uint16_t*)p->k_pq_cb, (const uint16_t*)p->k_rvq_cb, g, scale2, w.tab);
  int st = check_launch("ref_tables scores");
  if (st) return st;
  switch (p->pq_subspaces) {
    case 4: st = launch_hist<4>(p, g, S, w.tab, w.pst, w.part, s); break;
    case 8: st = launch_hist<8>(p, g, S, w.tab, w.pst, w.part, s); break;
    case 16: st = launch_hist<16>(p, g, S, w.tab, w.pst, w.part, s); break;
    default: st = launch_hist<32>(p, g, S, w.tab, w.pst, w.part, s); break;
  }
  if (st) return st;
  constexpr int HB = 32;  // query heads per values block (16 measured the same, 8 slower)
  const dim3 vg((unsigned)g.nch, (unsigned)((BH + HB - 1) / HB));
  const size_t vlds = values_lds_bytes<D>(S);
  (void)hipFuncSetAttribute((const void*)ref_tab_values_kernel<D, HB>, hipFuncAttributeMaxDynamicSharedMemorySize,
                            (int)vlds);
  hipLaunchKernelGGL((ref_tab_values_kernel<D, HB>), vg, dim3(D * HB / 16), vlds, s, w.pst, w.part, S, BH,
                     (const uint16_t*)p->v_pq_cb, (const uint16_t*)p->v_rvq_cb, g, w.part2);
  st = check_launch("ref_tables values");
  if (st) return st;
  const int G = p->q_heads / p->kv_heads;
  hipLaunchKernelGGL(ref_tab_out_kernel<D>, dim3((unsigned)(p->batch * p->kv_heads), (unsigned)((G * D + 63) / 64)),
                     dim3(1024), 0, s, *p, g, S, g.nch, w.pst, w.part2, w.slots, w.partial, w.est);
  return check_launch("ref_tables out");
}

}  // namespace

RefTabGeom ref_tab_geom(const rfsn_ref_params* p) {
  RefTabGeom g{};
  g.D = p->head_dim;
  g.M = p->pq_subspaces;
  g.C = p->pq_centroids;
  g.L = p->rvq_layers;
  g.Cr = p->rvq_layers > 0 ? p->rvq_centroids : 0;
  g.dsub = g.M > 0 ? g.D / g.M : 0;
  g.cpq = (g.C + kChunk - 1) / kChunk;
  g.crv = g.L > 0 ? (g.Cr + kChunk - 1) / kChunk : 0;
  g.E = g.M * g.C + g.L * g.Cr;
  g.nch = g.M * g.cpq + g.L * g.crv;
  g.Ep = g.nch * kChunk;  // chunk space: every section padded to a multiple of 64 slots
  return g;
}

bool ref_tables_shape_ok(const rfsn_ref_params* p) {
  if (p == nullptr) return false;
  const int D = p->head_dim, M = p->pq_subspaces;
  if (!(D == 64 || D == 128 || D == 256) || !(M == 4 || M == 8 || M == 16 || M == 32) || D % M) return false;
  if (p->pq_centroids < 1 || p->pq_centroids > 256) return false;
  if (p->rvq_subspaces != 0 || p->sparse_k != 0) return false;  // the long-context stages
  if (p->rvq_layers < 0 || p->rvq_layers > 8 || (p->rvq_layers > 0 && (p->rvq_centroids < 1 || p->rvq_centroids > 65536)))
    return false;
  if (p->batch <= 0 || p->q_heads <= 0 || p->kv_heads <= 0 || p->q_heads % p->kv_heads || p->q_heads / p->kv_heads > 8)
    return false;
  const RefTabGeom g = ref_tab_geom(p);
  if (((size_t)2 * g.Ep + 64) * sizeof(float) > 160 * 1024) return false;
  const int64_t per_block = (int64_t)hist_tokens(M) * kHistThreads;
  return p->total_tokens >= 0 && (int64_t)p->total_tokens <= per_block * kMaxHistSplits;
}

int ref_tab_hist_splits(const rfsn_ref_params* p) {
  const int BH = p->batch * p->q_heads;
  const int64_t per_block = (int64_t)hist_tokens(p->pq_subspaces) * kHistThreads;
  int64_t s = ceil_div(p->total_tokens, per_block);
  const int64_t fill = ceil_div(256, BH);  // one block per CU
  if (s < fill) s = fill;
  s = (s + 7) / 8 * 8;  // a split's blocks share an XCD
  if (s > kMaxHistSplits) s = kMaxHistSplits;
  return (int)s;
}

size_t ref_tab_bytes(const rfsn_ref_params* p, int slots, RefTabLayout* w, void* base) {
  const RefTabGeom g = ref_tab_geom(p);
  const int64_t BH = (int64_t)p->batch * p->q_heads;
  const int S = ref_tab_hist_splits(p);
  auto al = [](size_t x) { return (x + 255) / 256 * 256; };
  size_t off = 0;
  const size_t o_partial = off;
  off += al((size_t)BH * slots * (p->head_dim + 2) * sizeof(float));
  const size_t o_est = off;
  off += al((size_t)BH * sizeof(float));
  const size_t o_tab = off;
  off += al((size_t)BH * g.Ep * sizeof(float));
  const size_t o_pst = off;
  off += al((size_t)BH * S * 4 * sizeof(float));
  const size_t o_part = off;
  off += al((size_t)g.nch * BH * S * kChunk * sizeof(float));
  const size_t o_part2 = off;
  off += al((size_t)g.nch * BH * p->head_dim * sizeof(float));
  if (w != nullptr) {
    char* b = reinterpret_cast<char*>(base);
    w->partial = reinterpret_cast<float*>(b + o_partial);
    w->est = reinterpret_cast<float*>(b + o_est);
    w->tab = reinterpret_cast<float*>(b + o_tab);
    w->pst = reinterpret_cast<float*>(b + o_pst);
    w->part = reinterpret_cast<float*>(b + o_part);
    w->part2 = reinterpret_cast<float*>(b + o_part2);
    w->slots = slots;
    w->hist_splits = S;
  }
  return off;
}

int launch_ref_tables(const rfsn_ref_params* p, const RefTabLayout& w, hipStream_t s) {
  const RefTabGeom g = ref_tab_geom(p);
  switch (p->head_dim) {
    case 64: return launch_tables_d<64>(p, g, w, s);
    case 128: return launch_tables_d<128>(p, g, w, s);
    default: return launch_tables_d<256>(p, g, w, s);
  }
}

}  // namespace rfsn

using namespace rfsn;

extern "C" int rfsn_ref_tables_ok(const rfsn_ref_params* p) { return ref_tables_shape_ok(p) ? 1 : 0; }

extern "C" int rfsn_ref_table_stats(const rfsn_ref_params* p, float* stats_dev, void* stream) {
  RFSN_REQUIRE(p != nullptr && stats_dev != nullptr, "ref_table_stats: null pointer");
  RFSN_REQUIRE(ref_tables_shape_ok(p) || (p->head_dim > 0 && p->pq_subspaces > 0 && p->rvq_subspaces == 0 &&
                                          p->sparse_k == 0 && p->head_dim % p->pq_subspaces == 0 &&
                                          p->rvq_layers >= 0 && p->rvq_layers <= 8),
               "ref_table_stats: the score tables serve the gated reference format (or PQ only)");
  RFSN_REQUIRE(p->k_pq_cb && p->v_pq_cb && (p->rvq_layers == 0 || (p->k_rvq_cb && p->v_rvq_cb)),
               "ref_table_stats: null codebook");
  RFSN_REQUIRE(p->pq_centroids >= 1 && (p->rvq_layers == 0 || p->rvq_centroids >= 1), "ref_table_stats: empty codebook");
  const RefTabGeom g = ref_tab_geom(p);
  hipLaunchKernelGGL(ref_tab_stats_kernel, dim3((unsigned)(2 * g.D)), dim3(256), 0, (hipStream_t)stream,
                     (const uint16_t*)p->k_pq_cb, (const uint16_t*)p->k_rvq_cb, (const uint16_t*)p->v_pq_cb,
                     (const uint16_t*)p->v_rvq_cb, g, stats_dev);
  return check_launch("ref_table_stats");
}
