// Standalone decode kernels (materialize_window compatibility path) and the
// k-means centroid update, for gfx950.
//
// Warm format (quantization.py:146-157 and the subspace-RVQ / sparse
// extension): base = C_pq[code]; with an RVQ stage K = fp16(base + C_rvq[code_r]);
// then K[idx] = fp16(K[idx] + val) for each sparse coordinate.
// Reference format (quantization.py:254-275, 310-319): corr = fp16(sum_l
// fl32(C_l[code_l])) in stage order from +0.0 on active rows, 0 elsewhere;
// out = fp16(base + corr).
#include "rfsn_common.h"

#include <algorithm>

namespace rfsn {
namespace {

// One thread per (vector, group of 4 coordinates).
__global__ void __launch_bounds__(256)
decode_ext_kernel(int64_t n, int D, const uint8_t* __restrict__ pq, int M, int C, const uint16_t* __restrict__ pq_cb,
                  const uint8_t* __restrict__ rvq, int Mr, int Cr, const uint16_t* __restrict__ rvq_cb,
                  const uint8_t* __restrict__ sidx, const uint16_t* __restrict__ sval, int k, int add_zero,
                  uint16_t* __restrict__ out, int64_t ldo) {
  const int groups = D / 4;
  const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (gid >= n * groups) return;
  const int64_t v = gid / groups;
  const int i0 = (int)(gid - v * groups) * 4;
  const int d = D / M;
  const int dr = Mr > 0 ? D / Mr : 1;
  uint16_t r[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const int i = i0 + e;
    const int m = i / d;
    uint16_t val = pq_cb[((size_t)m * C + min((int)pq[v * M + m], C - 1)) * d + (i - m * d)];
    if (Mr > 0) {
      const int mr = i / dr;
      val = hadd_bits(val, rvq_cb[((size_t)mr * Cr + min((int)rvq[v * Mr + mr], Cr - 1)) * dr + (i - mr * dr)]);
    } else if (add_zero) {
      val = hadd_bits(val, 0);
    }
    for (int j = 0; j < k; ++j) {
      if ((int)sidx[v * k + j] == i) val = hadd_bits(val, sval[v * k + j]);
    }
    r[e] = val;
  }
  uint16_t* o = out + v * ldo + i0;
#pragma unroll
  for (int e = 0; e < 4; ++e) o[e] = r[e];
}

// One thread per sparse entry (vector v, slot j): the corrected coordinate
// fp16(K[idx] + val) with K = fp16(base + rvq), i.e. the value the warm decode
// leaves at coordinate idx (the indices of one vector are distinct).
// DELTA = false: the corrected coordinate c = fp16(fp16(base + rvq) + val);
// DELTA = true: the score delta fp16(c - (float(base) + float(rvq))).
// Sparse entry (index byte sidx_e, residual sval_e) of the vector whose codes
// are pq_v[M] and rvq_v[Mr]: writes the corrected coordinate to *cc and the
// score delta to *delta (either may be NULL).
__device__ __forceinline__ void fold_entry(int D, const uint8_t* __restrict__ pq_v, int M, int C,
                                           const uint16_t* __restrict__ pq_cb, const uint8_t* __restrict__ rvq_v,
                                           int Mr, int Cr, const uint16_t* __restrict__ rvq_cb, uint8_t sidx_e,
                                           uint16_t sval_e, uint16_t* cc, uint16_t* delta) {
  const int i = min((int)sidx_e, D - 1);
  const int d = D / M;
  const int m = i / d;
  const uint16_t base = pq_cb[((size_t)m * C + min((int)pq_v[m], C - 1)) * d + (i - m * d)];
  uint16_t corr = 0, val = base;
  if (Mr > 0) {
    const int dr = D / Mr;
    const int mr = i / dr;
    corr = rvq_cb[((size_t)mr * Cr + min((int)rvq_v[mr], Cr - 1)) * dr + (i - mr * dr)];
    val = hadd_bits(base, corr);
  }
  const uint16_t c = hadd_bits(val, sval_e);
  if (cc) *cc = c;
  if (delta) {
    const float exact = h2f(base) + (Mr > 0 ? h2f(corr) : 0.f);
    *delta = f2h(h2f(c) - exact);
  }
}

template <bool DELTA>
__global__ void __launch_bounds__(256)
sparse_fold_kernel(int64_t n, int D, const uint8_t* __restrict__ pq, int M, int C, const uint16_t* __restrict__ pq_cb,
                   const uint8_t* __restrict__ rvq, int Mr, int Cr, const uint16_t* __restrict__ rvq_cb,
                   const uint8_t* __restrict__ sidx, const uint16_t* __restrict__ sval, int k,
                   uint16_t* __restrict__ out) {
  const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (gid >= n * k) return;
  const int64_t v = gid / k;
  fold_entry(D, pq + v * M, M, C, pq_cb, Mr > 0 ? rvq + v * Mr : nullptr, Mr, Cr, rvq_cb, sidx[gid], sval[gid],
             DELTA ? nullptr : out + gid, DELTA ? out + gid : nullptr);
}

// The warm append of one K/V block in one launch (16 PQ + 16 RVQ subspaces,
// k sparse entries): plain head-major codes [H][T][16] and sparse entries
// [H][T][k] of K and V into tokens t_base .. of their tiled stores.  V, and K
// without KSCORE, go to the tiled layout (rfsn_pack_codes) with the corrected
// coordinates at the plain positions [H][dst_tokens][k]; K with KSCORE goes
// to the score-table layout (rfsn_pack_score_codes) with the score deltas as
// sparse values and, when kcc is given, the corrected coordinates in the
// plane kcc at the same positions.  One thread per (head, token, row byte
// j); the threads j < k also fold sparse entry j of K and of V.
// Token-major rows [cap][H][*] of a reference-layout store (pq, rvq codes,
// the all-ones RVQ mask of the subspace formats, sparse index / residual);
// pq == NULL: none.
struct RingRows {
  uint8_t* pq;
  uint8_t* rvq;
  uint8_t* mask;
  uint8_t* sidx;
  uint16_t* sval;
};

// Copy one token's codes (row byte j, sparse entry j < k) into row rr of a ring.
__device__ __forceinline__ void ring_put(const RingRows& rg, int64_t rr, int H, int h, int j, int k,
                                         const uint8_t* __restrict__ pq, const uint8_t* __restrict__ rvq,
                                         const uint8_t* __restrict__ si, const uint16_t* __restrict__ sv, int64_t row,
                                         int64_t se) {
  const int64_t o = rr * H + h;
  rg.pq[o * 16 + j] = pq[row * 16 + j];
  rg.rvq[o * 16 + j] = rvq[row * 16 + j];
  if (j == 0) rg.mask[o] = 1;
  if (j < k) {
    rg.sidx[o * k + j] = si[se];
    rg.sval[o * k + j] = sv[se];
  }
}

template <bool KSCORE>
__global__ void __launch_bounds__(256)
warm_append_pair_kernel(int64_t T, int C, int Cr, int k, const uint8_t* __restrict__ kpq,
                        const uint8_t* __restrict__ krvq, const uint8_t* __restrict__ ksi,
                        const uint16_t* __restrict__ ksv, const uint8_t* __restrict__ vpq,
                        const uint8_t* __restrict__ vrvq, const uint8_t* __restrict__ vsi,
                        const uint16_t* __restrict__ vsv, const uint16_t* __restrict__ kpq_cb,
                        const uint16_t* __restrict__ krvq_cb, const uint16_t* __restrict__ vpq_cb,
                        const uint16_t* __restrict__ vrvq_cb, uint8_t* __restrict__ dkpq, uint8_t* __restrict__ dkrvq,
                        uint8_t* __restrict__ dksi, uint16_t* __restrict__ dksv, uint16_t* __restrict__ dkcc,
                        uint8_t* __restrict__ dvpq, uint8_t* __restrict__ dvrvq, uint8_t* __restrict__ dvsi,
                        uint16_t* __restrict__ dvsv, int64_t dst_tokens, int64_t t_base, RingRows kring,
                        RingRows vring, int64_t ring_row) {
  constexpr int kM = 16, kDim = 64;
  const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int h = blockIdx.y;
  if (gid >= T * kM) return;
  const int64_t tl = gid >> 4;
  const int j = (int)(gid & 15);
  const int64_t t = t_base + tl;
  const int64_t row = (int64_t)h * T + tl;  // plain code row of (head, token)
  const int64_t tau = t >> 5;
  const int u = (int)((t >> 4) & 1), r = (int)(t & 15);
  // tiled rows: subspace j of token t (TPI = 4 tokens per gather, IPT = 8)
  const int64_t to = (int64_t)h * dst_tokens * kM + tau * 32 * kM + ((t % 4) * kM + j) * 8 + (t % 32) / 4;
  const int64_t pe = (int64_t)h * dst_tokens * k + t * k + j;  // plain sparse position (j < k)
  if constexpr (KSCORE) {
    const int m = (j & 12) | ((j & 3) ^ ((r >> 2) & 3));
    const uint8_t a = kpq[row * kM + m], c = krvq[row * kM + m];
    const int64_t dst = (int64_t)h * dst_tokens * kM + tau * 512 + r * 32 + (j >> 2) * 8 + u * 4 + (j & 3);
    const bool odd = (r & 1) != 0;
    dkpq[dst] = odd ? c : a;
    dkrvq[dst] = odd ? a : c;
  } else {
    dkpq[to] = kpq[row * kM + j];
    dkrvq[to] = krvq[row * kM + j];
  }
  dvpq[to] = vpq[row * kM + j];
  dvrvq[to] = vrvq[row * kM + j];
  if (j < k) {
    const int64_t se = row * k + j;
    if constexpr (KSCORE) {
      const int64_t de = (int64_t)h * dst_tokens * k + tau * 32 * k + r * 2 * k + 2 * j + u;
      dksi[de] = ksi[se];
      fold_entry(kDim, kpq + row * kM, kM, C, kpq_cb, krvq + row * kM, kM, Cr, krvq_cb, ksi[se], ksv[se],
                 dkcc ? dkcc + de : nullptr, dksv + de);
    } else {
      dksi[pe] = ksi[se];
      fold_entry(kDim, kpq + row * kM, kM, C, kpq_cb, krvq + row * kM, kM, Cr, krvq_cb, ksi[se], ksv[se], dksv + pe,
                 nullptr);
    }
    dvsi[pe] = vsi[se];
    fold_entry(kDim, vpq + row * kM, kM, C, vpq_cb, vrvq + row * kM, kM, Cr, vrvq_cb, vsi[se], vsv[se], dvsv + pe,
               nullptr);
  }
  if (kring.pq) {
    const int H = (int)gridDim.y;
    const int64_t se = row * k + j;
    ring_put(kring, ring_row + tl, H, h, j, k, kpq, krvq, ksi, ksv, row, se);
    ring_put(vring, ring_row + tl, H, h, j, k, vpq, vrvq, vsi, vsv, row, se);
  }
}

__global__ void __launch_bounds__(256)
decode_ref_base_kernel(int64_t n, int D, const uint8_t* __restrict__ pq, int M, int C,
                       const uint16_t* __restrict__ pq_cb, uint16_t* __restrict__ out) {
  const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (gid >= n * D) return;
  const int64_t v = gid / D;
  const int i = (int)(gid - v * D);
  const int d = D / M;
  const int m = i / d;
  out[gid] = hadd_bits(pq_cb[((size_t)m * C + min((int)pq[v * M + m], C - 1)) * d + (i - m * d)], 0);
}

__global__ void __launch_bounds__(256)
decode_ref_corr_kernel(int64_t n, int64_t active, int D, const uint8_t* __restrict__ pq, int M, int C,
                       const uint16_t* __restrict__ pq_cb, const uint16_t* __restrict__ codes,
                       const int32_t* __restrict__ offsets, int L, int Cr, const uint16_t* __restrict__ rvq_cb,
                       uint16_t* __restrict__ out) {
  const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (gid >= active * D) return;
  const int64_t a = gid / D;
  const int i = (int)(gid - a * D);
  const int64_t v = offsets[a];
  if (v < 0 || v >= n) return;  // offsets outside the decoded rows are ignored
  float total = 0.0f;
  for (int l = 0; l < L; ++l) {
    const int c = min((int)codes[a * L + l], Cr - 1);
    total = __fadd_rn(total, h2f(rvq_cb[((size_t)l * Cr + c) * D + i]));
  }
  const uint16_t corr = f2h(total);
  const int d = D / M;
  const int m = i / d;
  out[v * D + i] = hadd_bits(pq_cb[((size_t)m * C + min((int)pq[v * M + m], C - 1)) * d + (i - m * d)], corr);
}

// k-means: per-(subspace, centroid) sums in float64 via atomics, then mean.
__global__ void kmeans_accum_kernel(const uint16_t* __restrict__ x, int64_t n, int D, int64_t ldx,
                                    const uint8_t* __restrict__ codes, int M, int C, double* __restrict__ sums,
                                    unsigned int* __restrict__ counts) {
  const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (gid >= n * M) return;
  const int64_t v = gid / M;
  const int m = (int)(gid - v * M);
  const int d = D / M;
  const int c = codes[v * M + m];
  double* s = sums + ((size_t)m * C + c) * d;
  for (int u = 0; u < d; ++u) atomicAdd(s + u, (double)h2f(x[v * ldx + m * d + u]));
  atomicAdd(counts + (size_t)m * C + c, 1u);
}

__global__ void kmeans_finish_kernel(int M, int C, int d, const double* __restrict__ sums,
                                     const unsigned int* __restrict__ counts, uint16_t* __restrict__ cb) {
  const int gid = blockIdx.x * blockDim.x + threadIdx.x;
  if (gid >= M * C * d) return;
  const int mc = gid / d;
  const unsigned int cnt = counts[mc];
  if (cnt == 0) return;
  cb[gid] = f2h((float)(sums[gid] / (double)cnt));
}

// k-means member sums in two levels.  Each block accumulates the (subspace,
// centroid) sums of its range of vectors in LDS, then writes them to its own
// slice of the workspace; kmeans_reduce_kernel adds the slices in block order
// in float64.  No global atomics: the single-level kernel above contends on
// the hot centroids' addresses.  A centroid's slot holds its d sums and its
// member count (fp32, exact below 2^24), d + 1 floats: with d = 4 the odd
// stride spreads 64 random centroids over all 64 banks.
constexpr int kKmeansMaxParts = 256;

template <int W>  // LDS words of the table, M * C * (d + 1) <= W
__global__ void __launch_bounds__(1024)
kmeans_partial_kernel(const uint16_t* __restrict__ x, int64_t n, int D, int64_t ldx, const uint8_t* __restrict__ codes,
                      int M, int C, int64_t per_block, float* __restrict__ parts) {
  __shared__ float sm[W];
  const int d = D / M, e = d + 1;
  const int S = M * C * e;
  for (int i = threadIdx.x; i < S; i += blockDim.x) sm[i] = 0.f;
  __syncthreads();
  const int64_t v0 = (int64_t)blockIdx.x * per_block;
  const int64_t v1 = min(n, v0 + per_block);
  const int64_t end = v1 * M;
  int64_t idx = v0 * M + threadIdx.x;
  if (d == 4 && (ldx & 3) == 0 && ((uintptr_t)x & 7) == 0) {
    // 8 (vector, subspace) pairs per thread per step: every load of the step
    // is issued before its atomics, so the memory latency is paid once per step
    constexpr int U = 8;
    const int64_t stride = (int64_t)blockDim.x;
    for (; idx + (U - 1) * stride < end; idx += U * stride) {
      int c[U];
      uint2 xv[U];
#pragma unroll
      for (int k = 0; k < U; ++k) {
        const int64_t id = idx + k * stride;
        const int64_t v = id / M;
        c[k] = codes[id];
        xv[k] = *reinterpret_cast<const uint2*>(x + v * ldx + (id - v * M) * 4);
      }
#pragma unroll
      for (int k = 0; k < U; ++k) {
        const int m = (int)((idx + k * stride) % M);
        float* sp = sm + (m * C + min(c[k], C - 1)) * 5;  // codes come from an encode against these C rows
        atomicAdd(sp + 0, h2f((uint16_t)(xv[k].x & 0xFFFFu)));
        atomicAdd(sp + 1, h2f((uint16_t)(xv[k].x >> 16)));
        atomicAdd(sp + 2, h2f((uint16_t)(xv[k].y & 0xFFFFu)));
        atomicAdd(sp + 3, h2f((uint16_t)(xv[k].y >> 16)));
        atomicAdd(sp + 4, 1.f);
      }
    }
  }
  for (; idx < end; idx += blockDim.x) {
    const int64_t v = idx / M;
    const int m = (int)(idx - v * M);
    const int c = min((int)codes[idx], C - 1);
    const uint16_t* xr = x + v * ldx + m * d;
    float* sp = sm + (m * C + c) * e;
    for (int u = 0; u < d; ++u) atomicAdd(sp + u, h2f(xr[u]));
    atomicAdd(sp + d, 1.f);
  }
  __syncthreads();
  float* ps = parts + (int64_t)blockIdx.x * S;
  for (int i = threadIdx.x; i < S; i += blockDim.x) ps[i] = sm[i];
}

__global__ void kmeans_reduce_kernel(int M, int C, int d, int nparts, const float* __restrict__ parts,
                                     uint16_t* __restrict__ cb) {
  const int gid = blockIdx.x * blockDim.x + threadIdx.x;
  const int e = d + 1, S = M * C * e;
  if (gid >= M * C * d) return;
  const int mc = gid / d, u = gid - mc * d;
  double cnt = 0.0, sum = 0.0;
#pragma unroll 8
  for (int p = 0; p < nparts; ++p) {
    cnt += (double)parts[(int64_t)p * S + mc * e + d];
    sum += (double)parts[(int64_t)p * S + mc * e + u];
  }
  if (cnt == 0.0) return;  // empty cluster keeps its row
  cb[gid] = f2h((float)(sum / cnt));
}

__global__ void zero_kernel(uint32_t* __restrict__ p, int64_t words) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < words) p[i] = 0u;
}

}  // namespace
}  // namespace rfsn

using namespace rfsn;

extern "C" int rfsn_decode(const rfsn_format* f, const rfsn_codes* codes, int64_t n, const void* pq_cb,
                           const void* rvq_cb, void* out, int64_t ldo, int32_t add_zero, void* stream) {
  RFSN_REQUIRE(f && codes && codes->pq && pq_cb && out, "decode: null pointer");
  RFSN_REQUIRE(f->head_dim % 4 == 0 && f->head_dim % f->pq_subspaces == 0, "decode: head_dim must be a multiple of 4");
  RFSN_REQUIRE(f->rvq_subspaces == 0 || (codes->rvq && rvq_cb && f->head_dim % f->rvq_subspaces == 0),
               "decode: RVQ stage needs codes and codebooks");
  RFSN_REQUIRE(f->sparse_k == 0 || (codes->sparse_idx && codes->sparse_val), "decode: sparse stage needs codes");
  RFSN_REQUIRE(ldo >= f->head_dim, "decode: bad leading dimension");
  if (n == 0) return RFSN_OK;
  const int64_t total = n * (f->head_dim / 4);
  hipLaunchKernelGGL(decode_ext_kernel, dim3((unsigned)ceil_div(total, 256)), dim3(256), 0, (hipStream_t)stream, n,
                     f->head_dim, codes->pq, f->pq_subspaces, f->pq_centroids, (const uint16_t*)pq_cb, codes->rvq,
                     f->rvq_subspaces, f->rvq_centroids, (const uint16_t*)rvq_cb, codes->sparse_idx,
                     (const uint16_t*)codes->sparse_val, f->sparse_k, add_zero, (uint16_t*)out, ldo);
  return check_launch("decode");
}

namespace rfsn {
namespace {
int sparse_fold_launch(bool delta, const char* name, const rfsn_format* f, const rfsn_codes* codes, int64_t n,
                       const void* pq_cb, const void* rvq_cb, void* out, void* stream) {
  RFSN_REQUIRE(f && codes && codes->pq && pq_cb && out, "sparse_fold: null pointer");
  RFSN_REQUIRE(f->sparse_k > 0 && codes->sparse_idx && codes->sparse_val, "sparse_fold: no sparse stage");
  RFSN_REQUIRE(f->head_dim % f->pq_subspaces == 0, "sparse_fold: head_dim must be a multiple of num_subspaces");
  RFSN_REQUIRE(f->rvq_subspaces == 0 || (codes->rvq && rvq_cb && f->head_dim % f->rvq_subspaces == 0),
               "sparse_fold: RVQ stage needs codes and codebooks");
  if (n == 0) return RFSN_OK;
  const int64_t total = n * f->sparse_k;
  auto kern = delta ? sparse_fold_kernel<true> : sparse_fold_kernel<false>;
  hipLaunchKernelGGL(kern, dim3((unsigned)ceil_div(total, 256)), dim3(256), 0, (hipStream_t)stream, n,
                     f->head_dim, codes->pq, f->pq_subspaces, f->pq_centroids, (const uint16_t*)pq_cb, codes->rvq,
                     f->rvq_subspaces, f->rvq_centroids, (const uint16_t*)rvq_cb, codes->sparse_idx,
                     (const uint16_t*)codes->sparse_val, f->sparse_k, (uint16_t*)out);
  return check_launch(name);
}
}  // namespace
}  // namespace rfsn

extern "C" int rfsn_sparse_fold(const rfsn_format* f, const rfsn_codes* codes, int64_t n, const void* pq_cb,
                                const void* rvq_cb, void* out, void* stream) {
  return sparse_fold_launch(false, "sparse_fold", f, codes, n, pq_cb, rvq_cb, out, stream);
}

extern "C" int rfsn_sparse_delta(const rfsn_format* f, const rfsn_codes* codes, int64_t n, const void* pq_cb,
                                 const void* rvq_cb, void* out, void* stream) {
  return sparse_fold_launch(true, "sparse_delta", f, codes, n, pq_cb, rvq_cb, out, stream);
}

extern "C" int rfsn_warm_append_pair(const rfsn_format* f, const rfsn_codes* k_src, const rfsn_codes* v_src, int64_t T,
                                     int32_t heads, const void* k_pq_cb, const void* k_rvq_cb, const void* v_pq_cb,
                                     const void* v_rvq_cb, const rfsn_codes* k_dst, int32_t k_score_rows, void* k_cc,
                                     const rfsn_codes* v_dst, int64_t dst_tokens, int64_t t_base,
                                     const rfsn_codes* k_ring, uint8_t* k_ring_mask, const rfsn_codes* v_ring,
                                     uint8_t* v_ring_mask, int64_t ring_row, void* stream) {
  RFSN_REQUIRE(k_score_rows == 0 || k_score_rows == 1, "warm_append_pair: k_score_rows must be 0 or 1");
  RFSN_REQUIRE(k_cc == nullptr || k_score_rows, "warm_append_pair: a corrected-coordinate plane needs score rows");
  RFSN_REQUIRE(f && k_src && v_src && k_dst && v_dst, "warm_append_pair: null pointer");
  RFSN_REQUIRE(f->head_dim == 64 && f->pq_subspaces == 16 && f->rvq_subspaces == 16 && f->sparse_k > 0 &&
                   f->sparse_k <= 16,
               "warm_append_pair: needs head_dim 64, 16 PQ and 16 RVQ subspaces and 1..16 sparse entries");
  RFSN_REQUIRE(f->pq_centroids >= 1 && f->pq_centroids <= 256 && f->rvq_centroids >= 1 && f->rvq_centroids <= 256,
               "warm_append_pair: codebook sizes must be in [1, 256]");
  RFSN_REQUIRE(heads > 0 && T >= 0 && t_base >= 0, "warm_append_pair: bad arguments");
  RFSN_REQUIRE(dst_tokens % 32 == 0 && dst_tokens >= ceil_div(t_base + T, 32) * 32,
               "warm_append_pair: destination too small (whole 32-token tiles)");
  const rfsn_codes* all[4] = {k_src, v_src, k_dst, v_dst};
  for (const rfsn_codes* c : all)
    RFSN_REQUIRE(c->pq && c->rvq && c->sparse_idx && c->sparse_val, "warm_append_pair: missing code arrays");
  RFSN_REQUIRE(k_pq_cb && k_rvq_cb && v_pq_cb && v_rvq_cb, "warm_append_pair: missing codebooks");
  RFSN_REQUIRE((k_ring == nullptr) == (v_ring == nullptr) && ring_row >= 0, "warm_append_pair: rings come as a pair");
  RingRows kr = {}, vr = {};
  if (k_ring) {
    RFSN_REQUIRE(k_ring->pq && k_ring->rvq && k_ring->sparse_idx && k_ring->sparse_val && k_ring_mask && v_ring->pq &&
                     v_ring->rvq && v_ring->sparse_idx && v_ring->sparse_val && v_ring_mask,
                 "warm_append_pair: missing ring arrays");
    kr = {k_ring->pq, k_ring->rvq, k_ring_mask, k_ring->sparse_idx, (uint16_t*)k_ring->sparse_val};
    vr = {v_ring->pq, v_ring->rvq, v_ring_mask, v_ring->sparse_idx, (uint16_t*)v_ring->sparse_val};
  }
  if (T == 0) return RFSN_OK;
  auto kern = k_score_rows ? warm_append_pair_kernel<true> : warm_append_pair_kernel<false>;
  hipLaunchKernelGGL(kern, dim3((unsigned)ceil_div(T * 16, 256), (unsigned)heads), dim3(256), 0,
                     (hipStream_t)stream, T, f->pq_centroids, f->rvq_centroids, f->sparse_k, k_src->pq, k_src->rvq,
                     k_src->sparse_idx, (const uint16_t*)k_src->sparse_val, v_src->pq, v_src->rvq, v_src->sparse_idx,
                     (const uint16_t*)v_src->sparse_val, (const uint16_t*)k_pq_cb, (const uint16_t*)k_rvq_cb,
                     (const uint16_t*)v_pq_cb, (const uint16_t*)v_rvq_cb, k_dst->pq, k_dst->rvq, k_dst->sparse_idx,
                     (uint16_t*)k_dst->sparse_val, (uint16_t*)k_cc, v_dst->pq, v_dst->rvq, v_dst->sparse_idx,
                     (uint16_t*)v_dst->sparse_val, dst_tokens, t_base, kr, vr, ring_row);
  return check_launch("warm_append_pair");
}

extern "C" int rfsn_decode_ref(const uint8_t* pq, int64_t n, int32_t D, int32_t M, int32_t C, const void* pq_cb,
                               const uint16_t* rvq_codes, const int32_t* offsets, int64_t active, int32_t L,
                               int32_t Cr, const void* rvq_cb, void* out, void* stream) {
  RFSN_REQUIRE(pq && pq_cb && out && D > 0 && M > 0 && D % M == 0, "decode_ref: bad arguments");
  RFSN_REQUIRE(active == 0 || (rvq_codes && offsets && rvq_cb && L >= 1), "decode_ref: RVQ arguments missing");
  hipStream_t s = (hipStream_t)stream;
  if (n > 0) {
    hipLaunchKernelGGL(decode_ref_base_kernel, dim3((unsigned)ceil_div(n * D, 256)), dim3(256), 0, s, n, D, pq, M, C,
                       (const uint16_t*)pq_cb, (uint16_t*)out);
  }
  if (active > 0) {
    hipLaunchKernelGGL(decode_ref_corr_kernel, dim3((unsigned)ceil_div(active * D, 256)), dim3(256), 0, s, n, active, D,
                       pq, M, C, (const uint16_t*)pq_cb, rvq_codes, offsets, L, Cr, (const uint16_t*)rvq_cb,
                       (uint16_t*)out);
  }
  return check_launch("decode_ref");
}

extern "C" size_t rfsn_kmeans_workspace_bytes(int32_t M, int32_t C, int32_t d) {
  const size_t single = (size_t)M * C * d * sizeof(double) + (size_t)M * C * sizeof(unsigned int) + 256;
  const size_t parts = (size_t)kKmeansMaxParts * (size_t)M * C * (d + 1) * 4 + 256;
  return (size_t)M * C * (d + 1) <= 40 * 1024 ? parts : single;
}

extern "C" int rfsn_kmeans_update(const void* x, int64_t n, int32_t D, int64_t ldx, const uint8_t* codes, int32_t M,
                                  int32_t C, void* cb, void* ws, size_t ws_bytes, void* stream) {
  RFSN_REQUIRE(x && codes && cb && ws && M > 0 && D % M == 0 && C >= 1 && C <= 256, "kmeans_update: bad arguments");
  const int d = D / M;
  RFSN_REQUIRE(ws_bytes >= rfsn_kmeans_workspace_bytes(M, C, d), "kmeans_update: workspace too small");
  hipStream_t s = (hipStream_t)stream;
  const int64_t table_words = (int64_t)M * C * (d + 1);
  if (table_words <= 40 * 1024) {
    if (n == 0) return RFSN_OK;  // every cluster empty: the codebooks stay
    // at least about 1,024 vectors per block, at most kKmeansMaxParts blocks
    const int parts = (int)std::min<int64_t>(kKmeansMaxParts, std::max<int64_t>(1, ceil_div(n, 1024)));
    const int64_t per_block = ceil_div(n, parts);
    float* psums = (float*)ws;
    if (table_words <= 20 * 1024)  // 80 KB: two blocks per CU
      hipLaunchKernelGGL(kmeans_partial_kernel<20 * 1024>, dim3((unsigned)parts), dim3(1024), 0, s,
                         (const uint16_t*)x, n, D, ldx, codes, M, C, per_block, psums);
    else
      hipLaunchKernelGGL(kmeans_partial_kernel<40 * 1024>, dim3((unsigned)parts), dim3(1024), 0, s,
                         (const uint16_t*)x, n, D, ldx, codes, M, C, per_block, psums);
    hipLaunchKernelGGL(kmeans_reduce_kernel, dim3((unsigned)ceil_div((int64_t)M * C * d, 256)), dim3(256), 0, s, M, C,
                       d, parts, psums, (uint16_t*)cb);
    return check_launch("kmeans_update");
  }
  double* sums = (double*)ws;
  unsigned int* counts = (unsigned int*)(sums + (size_t)M * C * d);
  const int64_t words = ((int64_t)M * C * d * 2 + (int64_t)M * C);
  hipLaunchKernelGGL(zero_kernel, dim3((unsigned)ceil_div(words, 256)), dim3(256), 0, s, (uint32_t*)ws, words);
  if (n > 0) {
    hipLaunchKernelGGL(kmeans_accum_kernel, dim3((unsigned)ceil_div(n * M, 256)), dim3(256), 0, s,
                       (const uint16_t*)x, n, D, ldx, codes, M, C, sums, counts);
  }
  hipLaunchKernelGGL(kmeans_finish_kernel, dim3((unsigned)ceil_div((int64_t)M * C * d, 256)), dim3(256), 0, s, M, C, d,
                     sums, counts, (uint16_t*)cb);
  return check_launch("kmeans_update");
}

// ---------------------------------------------------------------- hot-tier append
namespace rfsn {
namespace {

// One thread per 8 fp16 (16 bytes) of a (token, head) row of K or V:
// hot[h][t0 + t][:] = src[t][h][:]; the V rows also fold max |v| into *vabs
// (float bits compared as integers: |v| >= 0; NaN bits order above +inf).
__global__ void __launch_bounds__(256)
hot_append_kernel(const uint16_t* __restrict__ k, const uint16_t* __restrict__ v, int64_t ld_t, int T, int H, int D,
                  uint16_t* __restrict__ hot_k, uint16_t* __restrict__ hot_v, int64_t hot_cap, int64_t t0,
                  uint32_t* __restrict__ vabs) {
  const int units = D / 8;
  const int64_t per = (int64_t)T * H * units;
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= 2 * per) return;
  const bool is_v = i >= per;
  const int64_t j = is_v ? i - per : i;
  const int u = (int)(j % units), h = (int)((j / units) % H);
  const int64_t t = j / ((int64_t)units * H);
  const uint16_t* src = (is_v ? v : k) + t * ld_t + (int64_t)h * D + 8 * u;
  uint16_t* dst = (is_v ? hot_v : hot_k) + ((int64_t)h * hot_cap + t0 + t) * D + 8 * u;
  const uint4 w = *reinterpret_cast<const uint4*>(src);
  *reinterpret_cast<uint4*>(dst) = w;
  if (is_v && vabs != nullptr) {
    uint32_t m = 0;
    const uint32_t ww[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      m = max(m, (uint32_t)__builtin_bit_cast(uint32_t, fabsf(h2f((uint16_t)(ww[e] & 0xFFFFu)))));
      m = max(m, (uint32_t)__builtin_bit_cast(uint32_t, fabsf(h2f((uint16_t)(ww[e] >> 16)))));
    }
    atomicMax(vabs, m);
  }
}

}  // namespace
}  // namespace rfsn

extern "C" int rfsn_hot_append(const void* k, const void* v, int64_t ld_t, int32_t T, int32_t heads, int32_t D,
                               void* hot_k, void* hot_v, int64_t hot_cap, int64_t t0, float* vabs, void* stream) {
  RFSN_REQUIRE(T >= 0 && heads > 0 && D > 0 && D % 8 == 0, "hot_append: head_dim must be a multiple of 8");
  RFSN_REQUIRE(T == 0 || (k && v && hot_k && hot_v), "hot_append: null pointer");
  RFSN_REQUIRE(ld_t >= (int64_t)heads * D && ld_t % 8 == 0, "hot_append: bad token stride");
  RFSN_REQUIRE(t0 >= 0 && t0 + T <= hot_cap, "hot_append: tokens past the hot buffers' capacity");
  RFSN_REQUIRE(reinterpret_cast<uintptr_t>(k) % 16 == 0 && reinterpret_cast<uintptr_t>(v) % 16 == 0 &&
                   reinterpret_cast<uintptr_t>(hot_k) % 16 == 0 && reinterpret_cast<uintptr_t>(hot_v) % 16 == 0,
               "hot_append: rows must be 16-byte aligned");
  if (T == 0) return RFSN_OK;
  const int64_t work = 2 * (int64_t)T * heads * (D / 8);
  hipLaunchKernelGGL(hot_append_kernel, dim3((unsigned)ceil_div(work, 256)), dim3(256), 0, (hipStream_t)stream,
                     (const uint16_t*)k, (const uint16_t*)v, ld_t, (int)T, (int)heads, (int)D, (uint16_t*)hot_k,
                     (uint16_t*)hot_v, hot_cap, t0, reinterpret_cast<uint32_t*>(vabs));
  return check_launch("hot_append");
}
