// Fused decode attention over compressed stores in CompressedTensorMLX's
// layout for gfx950: PQ codes with the gated full-dimension RVQ correction
// (quantization.py:99-319), or with a subspace RVQ stage and top-k sparse
// residuals (the long-context format), head_dim 64, 128 or 256.
//
// Replaces the decode-then-attend of RFSNHybridAttentionMLX.__call__
// (attention.py:150-171) and of RFSNv10KVCacheMLX.attention_forward over
// tiers the tiled fused kernel does not serve (cache.py:395-428: materialize_window, then
// _blockwise_exact_attention), without writing the decoded window to HBM.
//
// One block = (query b, KV head h, token split), 8 waves.  The PQ codebooks
// of K and V sit in LDS (entry-major rows of d fp16 per subspace).  A wave
// holds P token groups (P = 4, 2, 1 at head_dim 64, 128, 256), and lane ll of
// a group owns DPL = 4 coordinates (one PQ subspace), so one instruction
// serves P tokens.  A lane reads its token's code byte for its subspace and
// gathers its slice of the PQ entry from LDS.  For an active row of the
// reference format it adds its slice of the L RVQ codewords from global
// memory (a group's lanes read one codeword row: coalesced) with the
// reference's rounding chain: corr = fp16(sum_l fl32(C_l[code_l])) in stage
// order, K = fp16(fl32(base) + fl32(corr)) (corr = 0 for inactive rows).  The
// long-context format reads its subspace RVQ entries from global memory
// (L2-resident codebooks) and adds the sparse residuals to the coordinates
// they name.  A token's score is its group's sum of q . K partials in fp32;
// the online softmax runs on the wave (uniform), and the lane accumulates
// p * V on its coordinates.  The groups, then the 8 waves, combine in LDS;
// splits write (m, l, acc) partials that merge_partials_kernel combines.
#include "rfsn_common.h"
#include "rfsn_internal.h"

#include <type_traits>

namespace rfsn {
namespace {

constexpr int kRefWaves = 8;
constexpr int kRefThreads = kRefWaves * 64;
constexpr int kRefMaxG = 8;  // query heads per KV head
// exact rows: token slots per lane in units of U (2: 0.0693 -> 0.0684 ms at
// the reference default's table step; 4: 0.0698 ms; at one block per CU 3 and
// 4 tie there and lose 2-7% with 8 or 4 KV heads)
constexpr int kExactSlots = 2;
constexpr int kRefMaxL = 8;  // gated RVQ layers

typedef const rfsn_ref_segment __attribute__((address_space(4)))* cref;

// Sums over the P token groups of a wave (64 / P lanes each): DPP adds
// within each row of 16 lanes (quad_perm [1,0,3,2], [2,3,0,1],
// row_half_mirror, row_mirror leave every lane holding its row's sum), then
// the row sums of each group, returned as uniform scalars s[0..P).
template <int P>
__device__ __forceinline__ void group_sums(float v, float (&s)[P]) {
  auto f = [](int x) { return __builtin_bit_cast(float, x); };
  auto i = [](float x) { return __builtin_bit_cast(int, x); };
  v += f(__builtin_amdgcn_mov_dpp(i(v), 0xB1, 0xF, 0xF, true));
  v += f(__builtin_amdgcn_mov_dpp(i(v), 0x4E, 0xF, 0xF, true));
  v += f(__builtin_amdgcn_mov_dpp(i(v), 0x141, 0xF, 0xF, true));
  v += f(__builtin_amdgcn_mov_dpp(i(v), 0x140, 0xF, 0xF, true));
  const float r0 = f(__builtin_amdgcn_readlane(i(v), 0)), r1 = f(__builtin_amdgcn_readlane(i(v), 16));
  const float r2 = f(__builtin_amdgcn_readlane(i(v), 32)), r3 = f(__builtin_amdgcn_readlane(i(v), 48));
  if constexpr (P == 4) {
    s[0] = r0;
    s[1] = r1;
    s[2] = r2;
    s[3] = r3;
  } else if constexpr (P == 2) {
    s[0] = r0 + r1;
    s[1] = r2 + r3;
  } else {
    s[0] = (r0 + r1) + (r2 + r3);
  }
}

// The value of x for this lane's token group (tg < P), from uniform x[0..P),
// blended with bit masks: a chain of selects on tg becomes an indexed load
// through scratch memory at P = 4.
template <int P>
__device__ __forceinline__ float pick(const float (&x)[P], int tg) {
  uint32_t r = __builtin_bit_cast(uint32_t, x[0]);
#pragma unroll
  for (int p = 1; p < P; ++p) {
    const uint32_t m = 0u - (uint32_t)(tg == p);
    r = (r & ~m) | (__builtin_bit_cast(uint32_t, x[p]) & m);
  }
  return __builtin_bit_cast(float, r);
}

// Sum of v over the lanes that hold the same coordinates in the P token
// groups (lanes l, l ^ 16, l ^ 32, l ^ 48 for P = 4; l, l ^ 32 for P = 2).
template <int P>
__device__ __forceinline__ float across_groups(float v) {
  auto f = [](uint32_t x) { return __builtin_bit_cast(float, x); };
  auto u = [](float x) { return __builtin_bit_cast(uint32_t, x); };
  if constexpr (P == 4) {
    const auto r16 = __builtin_amdgcn_permlane16_swap(u(v), u(v), false, false);
    v = f(r16[0]) + f(r16[1]);
  }
  if constexpr (P >= 2) {
    const auto r32 = __builtin_amdgcn_permlane32_swap(u(v), u(v), false, false);
    v = f(r32[0]) + f(r32[1]);
  }
  return v;
}

// DPL consecutive fp16 values at p (DPL * 2-byte aligned when vec).
template <int DPL>
__device__ __forceinline__ void load_h(const uint16_t* p, uint16_t (&w)[DPL], bool vec = true) {
  if constexpr (DPL == 4) {
    if (vec) {
      const uint2 x = *reinterpret_cast<const uint2*>(p);
      w[0] = (uint16_t)x.x;
      w[1] = (uint16_t)(x.x >> 16);
      w[2] = (uint16_t)x.y;
      w[3] = (uint16_t)(x.y >> 16);
      return;
    }
  } else if constexpr (DPL == 2) {
    if (vec) {
      const uint32_t x = *reinterpret_cast<const uint32_t*>(p);
      w[0] = (uint16_t)x;
      w[1] = (uint16_t)(x >> 16);
      return;
    }
  }
#pragma unroll
  for (int v = 0; v < DPL; ++v) w[v] = p[v];
}

struct RvqShape {
  int L, Cr;   // gated full-dimension layers
  int Mr, dr;  // subspace stage (Mr = 0: none)
  int k;       // sparse residuals
};

// The lane's DPL coordinates c0 .. c0 + DPL - 1 of U stored vectors (rows
// row[u] of a store, one per lane: the lane's token group picks its token):
// PQ base, then the gated full-dimension correction (reference format) or
// the subspace RVQ stage and the sparse residuals (long-context format).
// Every load of the U vectors is issued before the first is consumed: the
// PQ code bytes and row indices, then the gated codes of every layer, then
// the codewords.
template <int D, int DPL, int U, bool EXT>
__device__ __forceinline__ void rebuild(float (&out)[U][DPL], const rfsn_ref_store_codes& sc, const int64_t (&row)[U],
                                        const uint16_t* __restrict__ tab, int M, int C, int dsub,
                                        const uint16_t* __restrict__ rvq_cb, const RvqShape& r, int c0) {
  // the lane's DPL coordinates sit in one PQ subspace (dsub is a multiple of DPL)
  const int m = c0 / dsub;
  const int off = c0 - m * dsub;
  int code[U];
#pragma unroll
  for (int u = 0; u < U; ++u) code[u] = sc.pq[row[u] * M + m];
  float corr[U][DPL];
#pragma unroll
  for (int u = 0; u < U; ++u)
#pragma unroll
    for (int v = 0; v < DPL; ++v) corr[u][v] = 0.0f;
  if (EXT && sc.rvq_sub != nullptr) {
    if (r.dr % DPL == 0) {  // uniform: the lane's coordinates sit in one subspace, one code
      const int mr = c0 / r.dr;
      int cr[U];
#pragma unroll
      for (int u = 0; u < U; ++u) cr[u] = sc.rvq_sub[row[u] * r.Mr + mr];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        uint16_t e[DPL];
        load_h<DPL>(rvq_cb + ((int64_t)mr * r.Cr + cr[u]) * r.dr + (c0 - mr * r.dr), e,
                    reinterpret_cast<uintptr_t>(rvq_cb) % (2 * DPL) == 0);
#pragma unroll
        for (int v = 0; v < DPL; ++v) corr[u][v] = h2f(e[v]);
      }
    } else {
      // the lane's coordinates span several subspaces
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const uint8_t* codes = sc.rvq_sub + row[u] * r.Mr;
#pragma unroll
        for (int v = 0; v < DPL; ++v) {
          const int dd = c0 + v;
          const int mr = dd / r.dr;
          corr[u][v] = h2f(rvq_cb[((int64_t)mr * r.Cr + codes[mr]) * r.dr + (dd - mr * r.dr)]);
        }
      }
    }
  } else if (!EXT && (sc.active != nullptr || sc.rvq != nullptr)) {
    // a row's index into the gated codes: the active map, or the row itself
    // when every row is active (no map)
    int a[U];
#pragma unroll
    for (int u = 0; u < U; ++u) a[u] = sc.active != nullptr ? sc.active[row[u]] : (int)row[u];
    int64_t base[U];
#pragma unroll
    for (int u = 0; u < U; ++u) base[u] = (int64_t)(a[u] < 0 ? 0 : a[u]) * r.L;  // the store holds >= 1 active row
    float tot[U][DPL];
#pragma unroll
    for (int u = 0; u < U; ++u)
#pragma unroll
      for (int v = 0; v < DPL; ++v) tot[u][v] = 0.0f;
    // four layers' codes in one 8-byte load when every row's codes start
    // 8-byte aligned (L a multiple of 4, an aligned code array; uniform)
    const bool quad = r.L % 4 == 0 && reinterpret_cast<uintptr_t>(sc.rvq) % 8 == 0;
    // layers four at a time: their codes, then their codewords of the U
    // rows in flight together; summed in stage order
    for (int l = 0; l < r.L; l += 4) {
      const int nl = min(4, r.L - l);
      int c[4][U];
      if (quad) {
#pragma unroll
        for (int u = 0; u < U; ++u) {
          const uint2 w = *reinterpret_cast<const uint2*>(sc.rvq + base[u] + l);
          const bool on = a[u] >= 0;
          c[0][u] = on ? (int)(w.x & 0xFFFFu) : 0;
          c[1][u] = on ? (int)(w.x >> 16) : 0;
          c[2][u] = on ? (int)(w.y & 0xFFFFu) : 0;
          c[3][u] = on ? (int)(w.y >> 16) : 0;
        }
      } else {
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
          for (int u = 0; u < U; ++u) c[j][u] = (a[u] < 0 || j >= nl) ? 0 : (int)sc.rvq[base[u] + l + j];
      }
      uint16_t w[4][U][DPL];
#pragma unroll
      for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int u = 0; u < U; ++u)
          load_h<DPL>(rvq_cb + ((int64_t)(j < nl ? l + j : l) * r.Cr + c[j][u]) * D + c0, w[j][u]);
#pragma unroll
      for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int u = 0; u < U; ++u)
#pragma unroll
          for (int v = 0; v < DPL; ++v)
            if (j < nl) tot[u][v] = __fadd_rn(tot[u][v], h2f(w[j][u][v]));
    }
#pragma unroll
    for (int u = 0; u < U; ++u)
#pragma unroll
      for (int v = 0; v < DPL; ++v) corr[u][v] = a[u] < 0 ? 0.0f : h2f(f2h(tot[u][v]));
  }
#pragma unroll
  for (int u = 0; u < U; ++u) {
    uint16_t e[DPL];
    load_h<DPL>(tab + ((int64_t)m * C + code[u]) * dsub + off, e);
#pragma unroll
    for (int v = 0; v < DPL; ++v) out[u][v] = h2f(f2h(__fadd_rn(h2f(e[v]), corr[u][v])));  // fp16(base + corr)
  }
  if (EXT && sc.sparse_idx != nullptr) {
    // K[idx] = fp16(fl32(K[idx]) + fl32(val)); the indices of a row are distinct
    const bool quad = r.k == 4 && reinterpret_cast<uintptr_t>(sc.sparse_idx) % 4 == 0 &&
                      reinterpret_cast<uintptr_t>(sc.sparse_val) % 8 == 0;  // uniform: one load per array
#pragma unroll
    for (int u = 0; u < U; ++u) {
      if (quad) {
        const uint32_t iw = *reinterpret_cast<const uint32_t*>(sc.sparse_idx + row[u] * 4);
        const uint2 vw = *reinterpret_cast<const uint2*>(sc.sparse_val + row[u] * 4);
        const uint32_t vh[4] = {vw.x & 0xFFFFu, vw.x >> 16, vw.y & 0xFFFFu, vw.y >> 16};
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int idx = (int)((iw >> (8 * j)) & 0xFFu);
          const float val = h2f((uint16_t)vh[j]);
#pragma unroll
          for (int v = 0; v < DPL; ++v)
            if (idx == c0 + v) out[u][v] = h2f(f2h(__fadd_rn(out[u][v], val)));
        }
      } else {
        for (int j = 0; j < r.k; ++j) {
          const int idx = sc.sparse_idx[row[u] * r.k + j];
          const float val = h2f(sc.sparse_val[row[u] * r.k + j]);
#pragma unroll
          for (int v = 0; v < DPL; ++v)
            if (idx == c0 + v) out[u][v] = h2f(f2h(__fadd_rn(out[u][v], val)));
        }
      }
    }
  }
}

// Splits balance the work, not the tokens: an exact (hot) token costs
// kExactCost and a coded one kCodedCost (at the reference's default config
// one block's coded tokens took 2.6x its exact ones: 214 us for 24,576 coded
// tokens per head against 28 us for 8,192 exact ones).  Split s covers the
// tokens t with bound(s) <= t < bound(s + 1), bound(s) = the first token
// whose cost prefix reaches s / splits of the total: a partition of the
// window whatever the segments (uniform scalar arithmetic).
// With score tables, the coded tokens of a group that keeps the tables'
// result cost 0: the splits partition its exact tokens.
constexpr int kExactCost = 2, kCodedCost = 5;

__device__ __forceinline__ int split_bound(cref segs, int nseg, int64_t total_cost, int splits, int s,
                                           int coded_cost) {
  if (s <= 0) return 0;
  const int64_t target = (int64_t)s * total_cost;  // prefix * splits >= target
  int64_t prefix = 0;
  int base = 0;
  for (int i = 0; i < nseg; ++i) {
    const int len = segs[i].len;
    const int64_t c = segs[i].k.pq != nullptr ? coded_cost : kExactCost;
    if (c == 0) {
      base += len;
      continue;
    }
    const int64_t need = target - prefix * splits;
    if (need <= 0) return base;
    const int64_t k = (need + c * splits - 1) / (c * splits);  // tokens of this segment before the bound
    if (k < len) return base + (int)k;
    prefix += (int64_t)len * c;
    base += len;
  }
  return base;
}

// Lane geometry: a wave holds P token groups of 64 / P lanes, and lane ll of
// a group owns coordinates c0 = DPL * ll .. c0 + DPL - 1 (DPL = D * P / 64),
// so one instruction serves P tokens.  A wave takes U * P consecutive tokens
// per step.  EXT: the long-context format (subspace RVQ stage, sparse
// residuals); otherwise the reference format (gated RVQ) or PQ only.
template <int D, int P, int U, int GMAX, bool EXT>
__global__ void __launch_bounds__(kRefThreads) __attribute__((amdgpu_waves_per_eu(GMAX == 1 ? 4 : 1))) ref_attn_kernel(const rfsn_ref_params p, int splits, int slots,
                                                               int kv_tab_shared, const float* __restrict__ tab_est) {
  extern __shared__ __align__(16) uint16_t tabs[];
  constexpr int DPL = D * P / 64;
  constexpr int LG = 64 / P;  // lanes per token group
  const int M = p.pq_subspaces, C = p.pq_centroids, dsub = D / M;
  const int G = p.q_heads / p.kv_heads;
  const int split = blockIdx.x % splits;
  const int h = (blockIdx.x / splits) % p.kv_heads;
  const int b = blockIdx.x / (splits * p.kv_heads);
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // uniform: keeps token indices scalar
  const int tg = lane / LG;        // the lane's token group
  const int c0 = DPL * (lane % LG);  // its first coordinate

  const cref segs = (cref)p.segments;
  // score tables: the group's coded tokens are the tables' unless the drift
  // estimate of one of its heads exceeds the tolerance (uniform)
  bool skip_coded = false;
  if (tab_est != nullptr) {
    bool redo = false;
    for (int g = 0; g < G; ++g) redo = redo || !(tab_est[(int64_t)b * p.q_heads + h * G + g] <= p.table_tol);
    skip_coded = !redo;
  }
  const int coded_cost = skip_coded ? 0 : kCodedCost;
  int64_t total_cost = 0;
  for (int s = 0; s < p.num_segments; ++s)
    total_cost += (int64_t)segs[s].len * (segs[s].k.pq != nullptr ? coded_cost : kExactCost);
  const int begin = split_bound(segs, p.num_segments, total_cost, splits, split, coded_cost);
  const int end = min(p.total_tokens, split_bound(segs, p.num_segments, total_cost, splits, split + 1, coded_cost));
  // whether the split decodes coded tokens (uniform): else the tables stay unstaged
  bool coded_here = false;
  if (!skip_coded) {
    int base = 0;
    for (int s = 0; s < p.num_segments && base < end; ++s) {
      const int len = segs[s].len;
      if (segs[s].k.pq != nullptr && max(begin, base) < min(end, base + len)) coded_here = true;
      base += len;
    }
  }

  // PQ tables: [M][C][dsub] for K, then V (unless they share one), copied in
  // 16-byte units (C * D * 2 bytes, a multiple of 16), up to 8 loads per
  // thread in flight before their stores
  const int tab_elems = M * C * dsub;
  if (coded_here) {
    const int units = tab_elems / 8;
    uint4* dst = reinterpret_cast<uint4*>(tabs);
    for (int t = 0; t < (kv_tab_shared ? 1 : 2); ++t) {
      const uint4* src = reinterpret_cast<const uint4*>(t ? p.v_pq_cb : p.k_pq_cb);
      for (int i0 = threadIdx.x; i0 < units; i0 += 8 * kRefThreads) {
        uint4 v[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) {
          const int i = i0 + u * kRefThreads;
          v[u] = i < units ? src[i] : make_uint4(0u, 0u, 0u, 0u);
        }
#pragma unroll
        for (int u = 0; u < 8; ++u) {
          const int i = i0 + u * kRefThreads;
          if (i < units) dst[t * units + i] = v[u];
        }
      }
    }
  }
  const uint16_t* ktab = tabs;
  const uint16_t* vtab = kv_tab_shared ? tabs : tabs + tab_elems;

  float qv[GMAX][DPL], acc[GMAX][DPL], m_run[GMAX], l_run[GMAX];
  int qpos[GMAX];
#pragma unroll
  for (int g = 0; g < GMAX; ++g) {
    const int hq = h * G + (g < G ? g : 0);
    const uint16_t* qrow = (const uint16_t*)p.q + ((int64_t)b * p.q_heads + hq) * D;
#pragma unroll
    for (int v = 0; v < DPL; ++v) {
      qv[g][v] = g < G ? h2f(qrow[c0 + v]) * p.scale : 0.0f;
      acc[g][v] = 0.0f;
    }
    m_run[g] = -__builtin_inff();
    l_run[g] = 0.0f;
    qpos[g] = (p.causal && p.qpos && g < G) ? p.qpos[(int64_t)b * p.q_heads + hq] : 0x7fffffff;
  }
  __syncthreads();

  RvqShape rs;
  rs.L = p.rvq_layers;
  rs.Cr = p.rvq_centroids;
  rs.Mr = p.rvq_subspaces;
  rs.dr = p.rvq_subspaces > 0 ? D / p.rvq_subspaces : 0;
  rs.k = p.sparse_k;
  int seg_base = 0;
  for (int s = 0; s < p.num_segments; ++s) {
    const int len = segs[s].len;
    const int lo = max(begin, seg_base), hi = min(end, seg_base + len);
    if (lo < hi && !(skip_coded && segs[s].k.pq != nullptr)) {
      rfsn_ref_store_codes kc{}, vc{};  // field by field: the table lives in the constant address space
      kc.pq = segs[s].k.pq;
      kc.rvq = segs[s].k.rvq;
      kc.active = segs[s].k.active;
      kc.rvq_sub = segs[s].k.rvq_sub;
      kc.sparse_idx = segs[s].k.sparse_idx;
      kc.sparse_val = segs[s].k.sparse_val;
      vc.pq = segs[s].v.pq;
      vc.rvq = segs[s].v.rvq;
      vc.active = segs[s].v.active;
      vc.rvq_sub = segs[s].v.rvq_sub;
      vc.sparse_idx = segs[s].v.sparse_idx;
      vc.sparse_val = segs[s].v.sparse_val;
      const int64_t tok0 = segs[s].token0;
      const int pos0 = segs[s].pos0;
      // code rows: the segment's strides, or the stores' [T][heads] order
      const int64_t cts = segs[s].code_token_stride, chs = segs[s].code_head_stride;
      const bool own = (cts | chs) == 0;
      const int64_t rts = own ? (int64_t)p.kv_heads : cts, rhs = own ? 1 : chs;
      const uint16_t* ek = (const uint16_t*)segs[s].exact_k;
      const uint16_t* ev = (const uint16_t*)segs[s].exact_v;
      const int64_t ets = segs[s].exact_token_stride, ehs = segs[s].exact_head_stride;
      // exact rows: DPL-wide loads when the rows and strides allow them (uniform)
      const bool evec = (((uintptr_t)ek | (uintptr_t)ev) % (2 * DPL) == 0) && ets % DPL == 0 && ehs % DPL == 0;
      // one step of UU * P consecutive tokens from g0 (token g0 + u * P + tg
      // is slot u of the lane's group): scores, online softmax, P.V
      auto attend = [&](auto uu, int g0, const auto& kk, const auto& vv) __attribute__((always_inline)) {
        constexpr int UU = decltype(uu)::value;
#pragma unroll
        for (int g = 0; g < GMAX; ++g) {
          if (g >= G) continue;  // uniform
          float sc[UU][P];
          float mx = -__builtin_inff();
#pragma unroll
          for (int u = 0; u < UU; ++u) {
            float part = 0.0f;
#pragma unroll
            for (int v = 0; v < DPL; ++v) part = __builtin_fmaf(qv[g][v], (float)kk[u][v], part);
            group_sums<P>(part, sc[u]);  // q was scaled on load
#pragma unroll
            for (int q = 0; q < P; ++q) {
              const int tt = g0 + u * P + q;
              const int pos = pos0 + (tt - seg_base);
              if (tt >= hi || pos < 0 || pos > qpos[g]) sc[u][q] = -__builtin_inff();  // masked (uniform)
              mx = fmaxf(mx, sc[u][q]);
            }
          }
          if (mx == -__builtin_inff()) continue;  // no allowed token in the step (uniform)
          const float mn = fmaxf(m_run[g], mx);
          const float corr = __expf(m_run[g] - mn);
          float l = l_run[g] * corr;
#pragma unroll
          for (int v = 0; v < DPL; ++v) acc[g][v] *= corr;
#pragma unroll
          for (int u = 0; u < UU; ++u) {
            float pr[P];
#pragma unroll
            for (int q = 0; q < P; ++q) {
              pr[q] = __expf(sc[u][q] - mn);
              l += pr[q];
            }
            const float pl = pick<P>(pr, tg);
#pragma unroll
            for (int v = 0; v < DPL; ++v) acc[g][v] = __builtin_fmaf(pl, (float)vv[u][v], acc[g][v]);
          }
          l_run[g] = l;
          m_run[g] = mn;
        }
      };
      // wave w takes steps of U * P consecutive tokens, every kRefWaves-th
      // step; exact rows take steps of UE * P (no decode registers are live
      // there: more loads in flight per lane, the rows kept in fp16, which
      // the FMAs convert exactly)
      if (kc.pq == nullptr) {
        constexpr int UE = kExactSlots * U;
        for (int g0 = lo + wave * (UE * P); g0 < hi; g0 += kRefWaves * UE * P) {
          _Float16 kk[UE][DPL], vv[UE][DPL];
#pragma unroll
          for (int u = 0; u < UE; ++u) {
            const int tl = g0 + u * P + tg;
            const int t = (tl < hi ? tl : g0) - seg_base;  // past the end: re-read the step's first token
            const int64_t e = (tok0 + t) * ets + (int64_t)h * ehs + c0;
            uint16_t wk[DPL], wv[DPL];
            load_h<DPL>(ek + e, wk, evec);
            load_h<DPL>(ev + e, wv, evec);
#pragma unroll
            for (int v = 0; v < DPL; ++v) {
              kk[u][v] = __builtin_bit_cast(_Float16, wk[v]);
              vv[u][v] = __builtin_bit_cast(_Float16, wv[v]);
            }
          }
          attend(std::integral_constant<int, UE>{}, g0, kk, vv);
        }
      } else {
        for (int g0 = lo + wave * (U * P); g0 < hi; g0 += kRefWaves * U * P) {
          int64_t row[U];
#pragma unroll
          for (int u = 0; u < U; ++u) {
            const int tl = g0 + u * P + tg;
            const int t = (tl < hi ? tl : g0) - seg_base;  // past the end: re-read the step's first token
            row[u] = (tok0 + t) * rts + h * rhs;
          }
          float kk[U][DPL], vv[U][DPL];
          rebuild<D, DPL, U, EXT>(kk, kc, row, ktab, M, C, dsub, (const uint16_t*)p.k_rvq_cb, rs, c0);
          rebuild<D, DPL, U, EXT>(vv, vc, row, vtab, M, C, dsub, (const uint16_t*)p.v_rvq_cb, rs, c0);
          attend(std::integral_constant<int, U>{}, g0, kk, vv);
        }
      }
    }
    seg_base += len;
  }

  // the token groups of a wave hold partial sums of the same coordinates
#pragma unroll
  for (int g = 0; g < GMAX; ++g)
#pragma unroll
    for (int v = 0; v < DPL; ++v) acc[g][v] = across_groups<P>(acc[g][v]);
  // combine the waves: [w][g] m, l, then [w][g][D] acc
  __syncthreads();
  float* red = reinterpret_cast<float*>(tabs);
  float* red_m = red;
  float* red_l = red + kRefWaves * kRefMaxG;
  float* red_a = red + 2 * kRefWaves * kRefMaxG;
#pragma unroll
  for (int g = 0; g < GMAX; ++g) {
    if (g >= G) continue;
    if (lane == 0) {
      red_m[wave * kRefMaxG + g] = m_run[g];
      red_l[wave * kRefMaxG + g] = l_run[g];
    }
    if (tg == 0)
#pragma unroll
      for (int v = 0; v < DPL; ++v) red_a[(wave * kRefMaxG + g) * D + c0 + v] = acc[g][v];
  }
  __syncthreads();
  for (int idx = threadIdx.x; idx < G * D; idx += kRefThreads) {
    const int g = idx / D, c = idx % D;
    float Mx = -__builtin_inff();
    for (int w = 0; w < kRefWaves; ++w) Mx = fmaxf(Mx, red_m[w * kRefMaxG + g]);
    float Ls = 0.f, A = 0.f;
    for (int w = 0; w < kRefWaves; ++w) {
      const float mw = red_m[w * kRefMaxG + g];
      const float f = mw > -__builtin_inff() ? __expf(mw - Mx) : 0.f;
      Ls += red_l[w * kRefMaxG + g] * f;
      A += red_a[(w * kRefMaxG + g) * D + c] * f;
    }
    const int hq = h * G + g;
    if (slots == 1) {
      // a query with no allowed key returns zeros (attention.py:104-105)
      ((uint16_t*)p.out)[((int64_t)b * p.q_heads + hq) * D + c] = f2h(Ls > 0.f ? A / Ls : 0.f);
      continue;
    }
    float* o = reinterpret_cast<float*>(p.workspace) + (((int64_t)b * p.q_heads + hq) * slots + split) * (D + 2);
    if (c == 0) {
      // the merge works in base 2
      o[0] = Mx * 1.4426950408889634f;
      o[1] = Ls;
    }
    o[2 + c] = A;
  }
}

int ref_splits(const rfsn_ref_params* p) {
  if (p->splits > 0) return p->splits;
  // blocks to aim for: two per CU, or one where a block's fixed cost (its
  // heads' q, combine and partials) outweighs its tokens -- groups of query
  // heads, and the exact pass of the score tables, which holds the hot
  // tokens only.  Measured on the default format (32 query heads, D 128,
  // 10k-33k tokens), 256 blocks against 512: 8 or 4 KV heads 4-14% faster
  // (exact decode) and 11-23% (score tables); one query head per KV head
  // flat or slower in the exact decode (8 heads, 9k tokens: 15% slower).
  const int units = p->batch * p->kv_heads;
  const int target = (p->score_tables != 0 || p->q_heads > p->kv_heads) ? 256 : 512;
  int s = (target + units - 1) / units;
  const int max_s = (p->total_tokens + 63) / 64;  // at least 64 tokens per split
  if (s > max_s) s = max_s;
  return s < 1 ? 1 : s;
}

size_t ref_lds_bytes(const rfsn_ref_params* p, bool shared) {
  const size_t tab = (size_t)p->pq_subspaces * p->pq_centroids * (p->head_dim / p->pq_subspaces) * 2;
  const size_t combine = (size_t)(2 * kRefWaves * kRefMaxG + kRefWaves * kRefMaxG * p->head_dim) * 4;
  const size_t t = shared ? tab : 2 * tab;
  return t > combine ? t : combine;
}

// P token groups per wave: 4 coordinates per lane where the PQ subspace
// allows it (head_dim 64 with 32 subspaces of 2: 2 coordinates, P = 2)
template <int D, int P>
int launch_ref(const rfsn_ref_params* p, hipStream_t s) {
  const int splits = ref_splits(p);
  const bool tables = p->score_tables != 0;
  // score tables: their launches first (the last partial slot of every query
  // head and the drift estimates the exact pass reads), then the exact pass
  // over the exact segments (and the coded ones of groups the guard sends
  // back), then the merge of splits + 1 slots
  const int slots = tables ? splits + 1 : splits;
  RefTabLayout tw{};
  if (tables) {
    ref_tab_bytes(p, slots, &tw, p->workspace);
    const int st = launch_ref_tables(p, tw, s);
    if (st) return st;
  }
  const bool shared = p->k_pq_cb == p->v_pq_cb;
  const size_t lds = ref_lds_bytes(p, shared);
  const int blocks = p->batch * p->kv_heads * splits;
  // token slots per lane: 8 coordinates of K and of V in flight per lane,
  // 12 for the gated format with 4 coordinates per lane (its kernel has the
  // registers; measured best at the reference's default config)
  constexpr int DPL = D * P / 64;
  constexpr int U = 8 / DPL;
  constexpr int UG = DPL == 4 ? 3 : U;
  const int G = p->q_heads / p->kv_heads;
  const bool ext = p->rvq_subspaces > 0 || p->sparse_k > 0;
  auto pick_g = [G](auto k1, auto k2, auto k4, auto k8) { return G <= 1 ? k1 : G <= 2 ? k2 : G <= 4 ? k4 : k8; };
  auto kern = ext ? pick_g(ref_attn_kernel<D, P, U, 1, true>, ref_attn_kernel<D, P, U, 2, true>,
                           ref_attn_kernel<D, P, U, 4, true>, ref_attn_kernel<D, P, U, 8, true>)
                  : pick_g(ref_attn_kernel<D, P, UG, 1, false>, ref_attn_kernel<D, P, UG, 2, false>,
                           ref_attn_kernel<D, P, UG, 4, false>, ref_attn_kernel<D, P, UG, 8, false>);
  if (lds > 64 * 1024) (void)hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
  hipLaunchKernelGGL(kern, dim3((unsigned)blocks), dim3(kRefThreads), lds, s, *p, splits, slots, (int)shared,
                     tables ? (const float*)tw.est : nullptr);
  int st = check_launch("ref_attention");
  if (st || slots == 1) return st;
  return launch_merge(reinterpret_cast<const float*>(p->workspace), (int64_t)p->batch * p->q_heads, slots,
                      p->head_dim, p->out, s);
}

}  // namespace
}  // namespace rfsn

using namespace rfsn;

extern "C" size_t rfsn_ref_attention_workspace_bytes(const rfsn_ref_params* p) {
  if (p == nullptr || p->batch <= 0 || p->q_heads <= 0 || p->kv_heads <= 0 || p->total_tokens <= 0) return 0;
  const int splits = ref_splits(p);
  if (p->score_tables) return ref_tables_shape_ok(p) ? ref_tab_bytes(p, splits + 1, nullptr, nullptr) : 0;
  if (splits == 1) return 0;
  return (size_t)p->batch * p->q_heads * splits * (p->head_dim + 2) * sizeof(float);
}

extern "C" int rfsn_ref_attention(const rfsn_ref_params* p, void* stream) {
  RFSN_REQUIRE(p != nullptr, "ref_attention: null params");
  const int D = p->head_dim, M = p->pq_subspaces;
  RFSN_REQUIRE(D == 64 || D == 128 || D == 256, "ref_attention: head_dim must be 64, 128 or 256");
  RFSN_REQUIRE((M == 4 || M == 8 || M == 16 || M == 32) && D % M == 0,
               "ref_attention: num_subspaces must be 4, 8, 16 or 32 and divide head_dim");
  RFSN_REQUIRE(p->pq_centroids >= 1 && p->pq_centroids <= 256, "ref_attention: PQ codebook size must be in [1, 256]");
  RFSN_REQUIRE(p->rvq_layers >= 0 && p->rvq_layers <= kRefMaxL &&
                   (p->rvq_layers == 0 || (p->rvq_centroids >= 1 && p->rvq_centroids <= 65536)),
               "ref_attention: at most 8 gated RVQ layers of at most 65536 codewords");
  RFSN_REQUIRE(p->rvq_subspaces >= 0 && (p->rvq_subspaces == 0 || p->rvq_layers == 0),
               "ref_attention: gated RVQ layers and an RVQ subspace stage are exclusive");
  RFSN_REQUIRE(p->rvq_subspaces == 0 || (D % p->rvq_subspaces == 0 && p->rvq_centroids >= 1 && p->rvq_centroids <= 256),
               "ref_attention: rvq_subspaces must divide head_dim, with at most 256 centroids");
  RFSN_REQUIRE(p->sparse_k >= 0 && p->sparse_k <= 8, "ref_attention: sparse_k must be in [0, 8]");
  RFSN_REQUIRE(p->batch > 0 && p->q_heads > 0 && p->kv_heads > 0 && p->q_heads % p->kv_heads == 0 &&
                   p->q_heads / p->kv_heads <= kRefMaxG,
               "ref_attention: query heads must be a multiple of KV heads, at most 8 per KV head");
  RFSN_REQUIRE(p->q && p->out && p->k_pq_cb && p->v_pq_cb, "ref_attention: null pointer");
  RFSN_REQUIRE(reinterpret_cast<uintptr_t>(p->k_pq_cb) % 16 == 0 && reinterpret_cast<uintptr_t>(p->v_pq_cb) % 16 == 0,
               "ref_attention: PQ codebooks must be 16-byte aligned");
  RFSN_REQUIRE((p->rvq_layers == 0 && p->rvq_subspaces == 0) || (p->k_rvq_cb && p->v_rvq_cb),
               "ref_attention: RVQ codebooks missing");
  RFSN_REQUIRE(p->rvq_layers == 0 ||
                   (reinterpret_cast<uintptr_t>(p->k_rvq_cb) % 8 == 0 && reinterpret_cast<uintptr_t>(p->v_rvq_cb) % 8 == 0),
               "ref_attention: gated RVQ codebooks must be 8-byte aligned");
  RFSN_REQUIRE(p->num_segments >= 0 && p->total_tokens >= 0 && (p->num_segments == 0 || p->segments),
               "ref_attention: bad segment table");
  const size_t shared_lds = ref_lds_bytes(p, p->k_pq_cb == p->v_pq_cb);
  RFSN_REQUIRE(shared_lds <= 160 * 1024, "ref_attention: the PQ codebooks do not fit the LDS (head_dim x centroids too large)");
  RFSN_REQUIRE(p->total_tokens > 0, "ref_attention: empty window (the caller returns zeros, attention.py:104-105)");
  RFSN_REQUIRE(p->splits >= 0 && p->splits <= 8192, "ref_attention: splits must be in [0, 8192]");
  RFSN_REQUIRE(p->score_tables == 0 || p->score_tables == 1, "ref_attention: score_tables must be 0 or 1");
  RFSN_REQUIRE(!p->score_tables || ref_tables_shape_ok(p),
               "ref_attention: score tables need the gated reference format (or PQ only), (2 E + 64) * 4 bytes "
               "of LDS for E = M C + L C_r entries and a window within the tables' token limit");
  RFSN_REQUIRE(!p->score_tables || (p->table_tol >= 0.f && p->table_stats != nullptr),
               "ref_attention: score tables need table_tol >= 0 and table_stats");
  hipStream_t s = (hipStream_t)stream;
  const size_t wsb = rfsn_ref_attention_workspace_bytes(p);
  RFSN_REQUIRE(wsb == 0 || (p->workspace && p->workspace_bytes >= wsb), "ref_attention: workspace too small");
  switch (D) {
    case 64: return M == 32 ? launch_ref<64, 2>(p, s) : launch_ref<64, 4>(p, s);
    case 128: return launch_ref<128, 2>(p, s);
    default: return launch_ref<256, 1>(p, s);
  }
}
