// Exact blockwise decode attention over fp16 K/V (attention.py:39-105) with a
// split-K log-sum-exp merge, and the code-layout pack kernel.
//
// Scores are computed in base-2 units (s * scale * log2 e) so that exp2 is a
// single v_exp_f32; masked positions contribute exactly zero, as
// exp_scores * allowed does in the reference (attention.py:93-95); a query
// with no allowed key returns zeros (safe_sum, attention.py:104-105).
#include "rfsn_common.h"
#include "rfsn_internal.h"

namespace rfsn {

namespace {

constexpr float kLog2e = 1.4426950408889634f;

// One block = (split, KV head, sequence); 4 waves; lane = token for scores,
// lane = coordinate for P.V.
template <int D, int G>
__global__ void __launch_bounds__(256)
exact_attn_kernel(const uint16_t* __restrict__ q, int Hq, const uint16_t* __restrict__ K,
                  const uint16_t* __restrict__ V, int64_t T, int64_t stride_t, int64_t stride_h,
                  int64_t stride_b, float scale_log2, int causal, const int32_t* __restrict__ qpos,
                  int splits, int64_t tokens_per_split, float* __restrict__ partial) {
  constexpr int kWaves = 4;
  constexpr int DPL = D / 64;  // coordinates per lane in P.V
  __shared__ float qs[G][D];
  __shared__ float pbuf[kWaves][G][64];
  __shared__ float red_m[kWaves][G], red_l[kWaves][G];
  __shared__ float red_acc[kWaves][G][D];
  const int split = blockIdx.x, h = blockIdx.y, b = blockIdx.z;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
  for (int i = threadIdx.x; i < G * D; i += blockDim.x) {
    const int g = i / D, c = i % D;
    qs[g][c] = h2f(q[((int64_t)b * Hq + h * G + g) * D + c]) * scale_log2;
  }
  int qp[G];
#pragma unroll
  for (int g = 0; g < G; ++g) qp[g] = qpos ? qpos[(int64_t)b * Hq + h * G + g] : (int)(T - 1);
  __syncthreads();

  const int64_t t0 = (int64_t)split * tokens_per_split;
  const int64_t t1 = t0 + tokens_per_split < T ? t0 + tokens_per_split : T;
  const uint16_t* Kb = K + (int64_t)b * stride_b + (int64_t)h * stride_h;
  const uint16_t* Vb = V + (int64_t)b * stride_b + (int64_t)h * stride_h;
  float m_run[G], l_run[G], acc[G][DPL];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    m_run[g] = -__builtin_inff();
    l_run[g] = 0.f;
#pragma unroll
    for (int e = 0; e < DPL; ++e) acc[g][e] = 0.f;
  }
  for (int64_t base = t0 + (int64_t)wave * 64; base < t1; base += kWaves * 64) {
    const int64_t tok = base + lane;
    const bool valid = tok < t1;
    float s[G];
#pragma unroll
    for (int g = 0; g < G; ++g) s[g] = 0.f;
    if (valid) {
      const uint4* row = reinterpret_cast<const uint4*>(Kb + tok * stride_t);
#pragma unroll
      for (int c = 0; c < D / 8; ++c) {
        const uint4 w = row[c];
        const uint32_t ws[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const float lo = h2f((uint16_t)(ws[e] & 0xffff));
          const float hi = h2f((uint16_t)(ws[e] >> 16));
#pragma unroll
          for (int g = 0; g < G; ++g) s[g] = fmaf(qs[g][c * 8 + 2 * e + 1], hi, fmaf(qs[g][c * 8 + 2 * e], lo, s[g]));
        }
      }
    }
    float corr[G];
#pragma unroll
    for (int g = 0; g < G; ++g) {
      const bool allowed = valid && (!causal || tok <= (int64_t)qp[g]);
      const float sv = allowed ? s[g] : -__builtin_inff();
      const float mt = wave_max(sv);
      const float mn = fmaxf(m_run[g], mt);
      const float p = (allowed && mn > -__builtin_inff()) ? exp2f(sv - mn) : 0.f;
      corr[g] = (m_run[g] > -__builtin_inff()) ? exp2f(m_run[g] - mn) : (mn > -__builtin_inff() ? 0.f : 1.f);
      l_run[g] = l_run[g] * corr[g] + wave_sum(p);
      m_run[g] = mn;
      pbuf[wave][g][lane] = p;
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
    for (int g = 0; g < G; ++g)
#pragma unroll
      for (int e = 0; e < DPL; ++e) acc[g][e] *= corr[g];
    const int ntok = (int)((t1 - base) < 64 ? (t1 - base) : 64);
    for (int t = 0; t < ntok; ++t) {
      const uint16_t* vr = Vb + (base + t) * stride_t;
      float vv[DPL];
#pragma unroll
      for (int e = 0; e < DPL; ++e) vv[e] = h2f(vr[lane * DPL + e]);
#pragma unroll
      for (int g = 0; g < G; ++g) {
        const float p = pbuf[wave][g][t];
#pragma unroll
        for (int e = 0; e < DPL; ++e) acc[g][e] = fmaf(p, vv[e], acc[g][e]);
      }
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  }
  // combine the four waves
#pragma unroll
  for (int g = 0; g < G; ++g) {
    if (lane == 0) {
      red_m[wave][g] = m_run[g];
      red_l[wave][g] = l_run[g];
    }
#pragma unroll
    for (int e = 0; e < DPL; ++e) red_acc[wave][g][lane * DPL + e] = acc[g][e];
  }
  __syncthreads();
  if (wave == 0) {
#pragma unroll
    for (int g = 0; g < G; ++g) {
      float M = -__builtin_inff();
      for (int w = 0; w < kWaves; ++w) M = fmaxf(M, red_m[w][g]);
      float L = 0.f, a[DPL];
#pragma unroll
      for (int e = 0; e < DPL; ++e) a[e] = 0.f;
      for (int w = 0; w < kWaves; ++w) {
        const float f = (red_m[w][g] > -__builtin_inff()) ? exp2f(red_m[w][g] - M) : 0.f;
        L += red_l[w][g] * f;
#pragma unroll
        for (int e = 0; e < DPL; ++e) a[e] += red_acc[w][g][lane * DPL + e] * f;
      }
      float* out = partial + (((int64_t)b * Hq + h * G + g) * splits + split) * (D + 2);
      if (lane == 0) {
        out[0] = M;
        out[1] = L;
      }
#pragma unroll
      for (int e = 0; e < DPL; ++e) out[2 + lane * DPL + e] = a[e];
    }
  }
}

}  // namespace

// Merge split partials (m, l, acc[D]) into fp16 outputs: one block of 256
// threads per (sequence, query head).  The split weights exp2(m_s - max) go
// to LDS once; then 256/D groups of D threads each sum a share of the splits
// with independent loads, and the groups are added in LDS.  A split with
// m_s = -inf (no allowed key) has weight 0.  Every thread issues its first
// split header and its first kMergePre partial sums together at the start,
// so a merge of up to 256 splits (kMergePre per group) waits for one memory
// round trip; the sums are formed in the same order either way.
constexpr int kMergeThreads = 256;
constexpr int kMergeMaxSplits = 8192;
constexpr int kMergePre = 16;

__device__ __forceinline__ float block_reduce(float v, float* red, bool is_max) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    const float y = __shfl_xor(v, o);
    v = is_max ? fmaxf(v, y) : v + y;
  }
  const int wave = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) red[wave] = v;
  __syncthreads();
  float r = red[0];
#pragma unroll
  for (int w = 1; w < kMergeThreads / 64; ++w) r = is_max ? fmaxf(r, red[w]) : r + red[w];
  __syncthreads();
  return r;
}

__global__ void __launch_bounds__(kMergeThreads) merge_partials_kernel(const float* __restrict__ partial, int splits,
                                                                      int D, uint16_t* __restrict__ out) {
  extern __shared__ float weight[];  // [splits]
  __shared__ float red[kMergeThreads / 64];
  __shared__ float part[kMergeThreads];
  const int64_t bh = blockIdx.x;
  const int t = threadIdx.x;
  const float* p = partial + bh * splits * (D + 2);
  const int groups = kMergeThreads / D, g = t / D, c = t % D;
  // the loads of one round trip: header t, sums g, g + groups, ...
  const bool h0 = t < splits;
  const float m0 = h0 ? p[t * (D + 2)] : -__builtin_inff();
  const float l0 = h0 ? p[t * (D + 2) + 1] : 0.f;
  float av[kMergePre];
#pragma unroll
  for (int u = 0; u < kMergePre; ++u) {
    const int s = g + u * groups;
    av[u] = g < groups && s < splits ? p[s * (D + 2) + 2 + c] : 0.f;
  }
  float mx = m0;
  for (int s = t + kMergeThreads; s < splits; s += kMergeThreads) mx = fmaxf(mx, p[s * (D + 2)]);
  mx = block_reduce(mx, red, true);
  float l = 0.f;
  if (h0) {
    const float w = m0 > -__builtin_inff() ? exp2f(m0 - mx) : 0.f;
    weight[t] = w;
    l += l0 * w;
  }
  for (int s = t + kMergeThreads; s < splits; s += kMergeThreads) {
    const float m = p[s * (D + 2)];
    const float w = m > -__builtin_inff() ? exp2f(m - mx) : 0.f;
    weight[s] = w;
    l += p[s * (D + 2) + 1] * w;
  }
  l = block_reduce(l, red, false);  // its barriers also publish weight[]
  float a = 0.f;
  if (g < groups) {
#pragma unroll
    for (int u = 0; u < kMergePre; ++u) {
      const int s = g + u * groups;
      if (s < splits) a += weight[s] * av[u];
    }
#pragma unroll 8
    for (int s = g + kMergePre * groups; s < splits; s += groups) a += weight[s] * p[s * (D + 2) + 2 + c];
  }
  part[t] = a;
  __syncthreads();
  if (t < D) {
    float sum = 0.f;
    for (int k = 0; k < groups; ++k) sum += part[k * D + t];
    out[bh * D + t] = f2h(l > 0.f ? sum / l : 0.f);
  }
}

int launch_merge(const float* partial, int64_t bh, int splits, int D, void* out, hipStream_t s) {
  RFSN_REQUIRE(D > 0 && D <= kMergeThreads && kMergeThreads % D == 0, "merge: head_dim must divide 256");
  RFSN_REQUIRE(splits > 0 && splits <= kMergeMaxSplits, "merge: at most 8192 split partials per row");
  hipLaunchKernelGGL(merge_partials_kernel, dim3((unsigned)bh), dim3(kMergeThreads), (size_t)splits * sizeof(float),
                     s, partial, splits, D, (uint16_t*)out);
  return check_launch("merge_partials");
}

// Pack plain code rows [H][T][M] (row stride M) into the tiled layout the
// fused kernel streams: per head a block of cap*M bytes; within 32-token
// tile tau, byte (t, m) sits at tau*32*M + ((t % TPI)*M + m)*IPT + (t%32)/TPI
// with TPI = 64/M tokens per gather instruction and IPT = 32/TPI.
__global__ void pack_codes_kernel(const uint8_t* __restrict__ src, int64_t src_head_stride, int64_t T,
                                  int M, uint8_t* __restrict__ dst, int64_t dst_head_stride, int64_t t_base) {
  const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int h = blockIdx.y;
  if (gid >= T * M) return;
  const int64_t tl = gid / M;
  const int m = (int)(gid - tl * M);
  const int64_t t = t_base + tl;
  const int tpi = 64 / M, ipt = 32 / tpi;
  const int64_t off = (t / 32) * 32 * M + ((t % tpi) * M + m) * ipt + (t % 32) / tpi;
  dst[(int64_t)h * dst_head_stride + off] = src[(int64_t)h * src_head_stride + gid];
}

// Score-table K layout (16 PQ + 16 RVQ subspaces, k sparse entries): token
// t = 32 tau + 16 u + r of a head's stream.  Code byte j = 4 beta + b of its
// row (in each array) sits at 512 tau + 32 r + 8 beta + 4 u + b and holds
// subspace 4 beta + (b ^ ((r >> 2) & 3)); odd tokens keep their RVQ codes in
// the PQ array and their PQ codes in the RVQ array.  Sparse entry e sits at
// entry 32 k tau + 2 k r + 2 e + u.  One thread per (token, row byte j); the
// threads j < k also move sparse entry j.
__global__ void pack_score_codes_kernel(const uint8_t* __restrict__ pq, const uint8_t* __restrict__ rvq,
                                        const uint8_t* __restrict__ sidx, const uint16_t* __restrict__ sval, int k,
                                        int64_t T, uint8_t* __restrict__ dpq, uint8_t* __restrict__ drvq,
                                        uint8_t* __restrict__ dsidx, uint16_t* __restrict__ dsval,
                                        int64_t dst_tokens, int64_t t_base) {
  const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int h = blockIdx.y;
  if (gid >= T * 16) return;
  const int64_t tl = gid >> 4;
  const int j = (int)(gid & 15);
  const int64_t t = t_base + tl;
  const int64_t tau = t >> 5;
  const int u = (int)((t >> 4) & 1), r = (int)(t & 15);
  const int m = (j & 12) | ((j & 3) ^ ((r >> 2) & 3));
  const int64_t src = ((int64_t)h * T + tl) * 16 + m;
  const uint8_t a = pq[src], c = rvq[src];
  const int64_t dst = (int64_t)h * dst_tokens * 16 + tau * 512 + r * 32 + (j >> 2) * 8 + u * 4 + (j & 3);
  const bool odd = (r & 1) != 0;
  dpq[dst] = odd ? c : a;
  drvq[dst] = odd ? a : c;
  if (j < k) {
    const int64_t se = ((int64_t)h * T + tl) * k + j;
    const int64_t de = (int64_t)h * dst_tokens * k + tau * 32 * k + r * 2 * k + 2 * j + u;
    dsidx[de] = sidx[se];
    dsval[de] = sval[se];
  }
}

}  // namespace rfsn

using namespace rfsn;

extern "C" size_t rfsn_attention_workspace_bytes(int32_t B, int32_t Hq, int32_t D, int32_t splits) {
  if (B <= 0 || Hq <= 0 || D <= 0 || splits <= 0) return 0;
  return (size_t)B * Hq * splits * (D + 2) * sizeof(float);
}

static int choose_splits(int64_t T, int64_t blocks_per_split) {
  // enough blocks to fill 256 CUs several times over, at least 256 tokens each
  int64_t s = ceil_div(1024, blocks_per_split > 0 ? blocks_per_split : 1);
  const int64_t max_s = ceil_div(T, 256);
  if (s > max_s) s = max_s;
  if (s < 1) s = 1;
  if (s > 1024) s = 1024;
  return (int)s;
}

extern "C" int rfsn_blockwise_attention(const void* q, int32_t B, int32_t Hq, int32_t D, const void* k, const void* v,
                                        int64_t T, int32_t Hkv, int64_t stride_t, int64_t stride_h, float scale,
                                        int32_t causal, const int32_t* qpos, void* out, void* ws, size_t ws_bytes,
                                        void* stream) {
  RFSN_REQUIRE(q && out && B > 0 && Hq > 0 && Hkv > 0, "blockwise_attention: bad arguments");
  RFSN_REQUIRE(Hq % Hkv == 0, "blockwise_attention: query heads must be a multiple of KV heads");
  RFSN_REQUIRE(D == 64 || D == 128, "blockwise_attention: head_dim must be 64 or 128");
  RFSN_REQUIRE(T >= 0 && (T == 0 || (k && v)), "blockwise_attention: bad K/V");
  RFSN_REQUIRE(stride_t % 8 == 0 && stride_h % 8 == 0, "blockwise_attention: K/V rows must be 16-byte aligned");
  const int G = Hq / Hkv;
  hipStream_t s = (hipStream_t)stream;
  int splits = T > 0 ? choose_splits(T, (int64_t)B * Hkv) : 1;
  if (ws_bytes < rfsn_attention_workspace_bytes(B, Hq, D, splits)) {
    splits = 1;
    RFSN_REQUIRE(ws && ws_bytes >= rfsn_attention_workspace_bytes(B, Hq, D, 1),
                 "blockwise_attention: workspace too small");
  }
  const int64_t tps = T > 0 ? ceil_div(ceil_div(T, splits), 64) * 64 : 64;
  dim3 grid((unsigned)splits, (unsigned)Hkv, (unsigned)B);
  const float sl2 = scale * 1.4426950408889634f;
  // the batch axis of q/out is separate; K/V are shared by the batch of queries
  // (attention.py:48: q [B,H,D] are queries over one cache)
#define RFSN_EXACT(DD, GG)                                                                                       \
  hipLaunchKernelGGL((exact_attn_kernel<DD, GG>), grid, dim3(256), 0, s, (const uint16_t*)q, Hq, (const uint16_t*)k, \
                     (const uint16_t*)v, T, stride_t, stride_h, (int64_t)0, sl2, causal, qpos, splits, tps, (float*)ws)
  if (D == 64) {
    switch (G) {
      case 1: RFSN_EXACT(64, 1); break;
      case 2: RFSN_EXACT(64, 2); break;
      case 4: RFSN_EXACT(64, 4); break;
      case 8: RFSN_EXACT(64, 8); break;
      default: return fail(RFSN_ERR_UNSUPPORTED, "blockwise_attention: Hq/Hkv must be 1, 2, 4 or 8");
    }
  } else {
    switch (G) {
      case 1: RFSN_EXACT(128, 1); break;
      case 2: RFSN_EXACT(128, 2); break;
      case 4: RFSN_EXACT(128, 4); break;
      case 8: RFSN_EXACT(128, 8); break;
      default: return fail(RFSN_ERR_UNSUPPORTED, "blockwise_attention: Hq/Hkv must be 1, 2, 4 or 8");
    }
  }
#undef RFSN_EXACT
  int st = check_launch("blockwise_attention");
  if (st) return st;
  return launch_merge((const float*)ws, (int64_t)B * Hq, splits, D, out, s);
}

extern "C" int rfsn_pack_codes(const uint8_t* src, int64_t src_head_stride, int64_t T, int32_t M, int32_t heads,
                               uint8_t* dst, int64_t dst_head_stride, int64_t t_base, void* stream) {
  RFSN_REQUIRE(src && dst && heads > 0 && T >= 0 && t_base >= 0, "pack_codes: bad arguments");
  RFSN_REQUIRE(M == 8 || M == 16, "pack_codes: M must be 8 or 16");
  RFSN_REQUIRE(dst_head_stride >= ceil_div(t_base + T, 32) * 32 * M, "pack_codes: destination too small");
  if (T == 0) return RFSN_OK;
  hipLaunchKernelGGL(pack_codes_kernel, dim3((unsigned)ceil_div(T * M, 256), (unsigned)heads), dim3(256), 0,
                     (hipStream_t)stream, src, src_head_stride, T, M, dst, dst_head_stride, t_base);
  return check_launch("pack_codes");
}

extern "C" int rfsn_pack_score_codes(const uint8_t* pq, const uint8_t* rvq, const uint8_t* sidx,
                                     const uint16_t* sval, int32_t k, int64_t T, int32_t heads, uint8_t* dpq,
                                     uint8_t* drvq, uint8_t* dsidx, uint16_t* dsval, int64_t dst_tokens,
                                     int64_t t_base, void* stream) {
  RFSN_REQUIRE(pq && rvq && dpq && drvq && heads > 0 && T >= 0 && t_base >= 0, "pack_score_codes: bad arguments");
  RFSN_REQUIRE(k >= 0 && k <= 16 && (k == 0 || (sidx && sval && dsidx && dsval)),
               "pack_score_codes: sparse entries need 0 <= k <= 16 and all four arrays");
  RFSN_REQUIRE(dst_tokens % 32 == 0 && dst_tokens >= ceil_div(t_base + T, 32) * 32,
               "pack_score_codes: destination too small (whole 32-token tiles)");
  if (T == 0) return RFSN_OK;
  hipLaunchKernelGGL(pack_score_codes_kernel, dim3((unsigned)ceil_div(T * 16, 256), (unsigned)heads), dim3(256), 0,
                     (hipStream_t)stream, pq, rvq, sidx, sval, k, T, dpq, drvq, dsidx, dsval, dst_tokens, t_base);
  return check_launch("pack_score_codes");
}
