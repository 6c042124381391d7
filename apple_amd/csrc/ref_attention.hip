// Fused decode attention over reference-format compressed stores for gfx950:
// PQ codes with the gated full-dimension RVQ correction
// (quantization.py:99-319), any head_dim that is a multiple of 64 up to 256.
//
// Replaces the decode-then-attend of RFSNHybridAttentionMLX.__call__
// (attention.py:150-171) and of RFSNv10KVCacheMLX.attention_forward over
// reference-format tiers (cache.py:395-428: materialize_window, then
// _blockwise_exact_attention), without writing the decoded window to HBM.
//
// One block = (query b, KV head h, token split), 4 waves.  The PQ codebooks
// of K and V sit in LDS (entry-major rows of d fp16 per subspace).  A wave
// streams the split's tokens one at a time with the token's codes in scalar
// registers (uniform loads); lane l owns coordinates DPL*l .. DPL*l+DPL-1, so
// it gathers its slice of the token's PQ entry from LDS and, for an active
// row, its slice of the L RVQ codewords from global memory (64 lanes read one
// codeword row: coalesced), and rebuilds the reference's rounding chain:
// corr = fp16(sum_l fl32(C_l[code_l])) in stage order, K = fp16(fl32(base) +
// fl32(corr)) (corr = 0 for inactive rows).  Scores are the wave's sum of
// q . K partials in fp32; the online softmax runs on the wave (uniform), and
// the lane accumulates p * V on its coordinates.  The 4 waves combine in LDS;
// splits write (m, l, acc) partials that merge_partials_kernel combines.
#include "rfsn_common.h"
#include "rfsn_internal.h"

namespace rfsn {
namespace {

constexpr int kRefWaves = 4;
constexpr int kRefThreads = kRefWaves * 64;
constexpr int kRefMaxG = 8;  // query heads per KV head

typedef const rfsn_ref_segment __attribute__((address_space(4)))* cref;

__device__ __forceinline__ float wave_sum64(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

// code byte m (0 <= m < M <= 32) of a row whose M bytes are the uniform
// words w[0 .. M/4)
template <int MW>
__device__ __forceinline__ int code_byte(const uint32_t (&w)[MW], int m) {
  uint32_t x = w[0];
#pragma unroll
  for (int i = 1; i < MW; ++i) x = (m >> 2) == i ? w[i] : x;
  return (int)((x >> (8 * (m & 3))) & 0xFFu);
}

// The lane's DPL coordinates of one stored vector (PQ base + gated RVQ
// correction) or of an exact row.
template <int DPL, int MW>
__device__ __forceinline__ void rebuild(float (&out)[DPL], const rfsn_ref_store_codes& sc, const uint16_t* exact_row,
                                        int64_t row, const uint16_t* __restrict__ tab, int M, int C, int dsub,
                                        const uint16_t* rvq_cb, int L, int Cr, int D, int lane) {
  if (exact_row != nullptr) {
#pragma unroll
    for (int u = 0; u < DPL; ++u) out[u] = h2f(exact_row[DPL * lane + u]);
    return;
  }
  uint32_t w[MW];
#pragma unroll
  for (int i = 0; i < MW; ++i) w[i] = reinterpret_cast<const uint32_t*>(sc.pq + row * M)[i];  // M = 4 MW bytes
  const int a = sc.active ? sc.active[row] : -1;  // uniform
  float corr[DPL];
#pragma unroll
  for (int u = 0; u < DPL; ++u) corr[u] = 0.0f;
  if (a >= 0) {
    float tot[DPL];
#pragma unroll
    for (int u = 0; u < DPL; ++u) tot[u] = 0.0f;
    for (int l = 0; l < L; ++l) {
      const int c = sc.rvq[(int64_t)a * L + l];
      const uint16_t* cw = rvq_cb + ((int64_t)l * Cr + c) * D + DPL * lane;
#pragma unroll
      for (int u = 0; u < DPL; ++u) tot[u] = __fadd_rn(tot[u], h2f(cw[u]));
    }
#pragma unroll
    for (int u = 0; u < DPL; ++u) corr[u] = h2f(f2h(tot[u]));
  }
#pragma unroll
  for (int u = 0; u < DPL; ++u) {
    const int dd = DPL * lane + u;
    const int m = dd / dsub;
    const int code = code_byte<MW>(w, m);
    const float base = h2f(tab[((int64_t)m * C + code) * dsub + (dd - m * dsub)]);
    out[u] = h2f(f2h(__fadd_rn(base, corr[u])));  // fp16(fl32(base) + fl32(corr))
  }
}

template <int DPL, int MW>
__global__ void __launch_bounds__(kRefThreads) ref_attn_kernel(const rfsn_ref_params p, int splits, int tps,
                                                               int kv_tab_shared) {
  extern __shared__ __align__(16) uint16_t tabs[];
  constexpr int D = 64 * DPL;
  const int M = p.pq_subspaces, C = p.pq_centroids, dsub = D / M;
  const int G = p.q_heads / p.kv_heads;
  const int split = blockIdx.x % splits;
  const int h = (blockIdx.x / splits) % p.kv_heads;
  const int b = blockIdx.x / (splits * p.kv_heads);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;

  // PQ tables: [M][C][dsub] for K, then V (unless they share one)
  const int tab_elems = M * C * dsub;
  for (int i = threadIdx.x; i < tab_elems; i += kRefThreads) tabs[i] = ((const uint16_t*)p.k_pq_cb)[i];
  if (!kv_tab_shared)
    for (int i = threadIdx.x; i < tab_elems; i += kRefThreads) tabs[tab_elems + i] = ((const uint16_t*)p.v_pq_cb)[i];
  const uint16_t* ktab = tabs;
  const uint16_t* vtab = kv_tab_shared ? tabs : tabs + tab_elems;

  float qv[kRefMaxG][DPL], acc[kRefMaxG][DPL], m_run[kRefMaxG], l_run[kRefMaxG];
  int qpos[kRefMaxG];
#pragma unroll
  for (int g = 0; g < kRefMaxG; ++g) {
    const int hq = h * G + (g < G ? g : 0);
    const uint16_t* qrow = (const uint16_t*)p.q + ((int64_t)b * p.q_heads + hq) * D;
#pragma unroll
    for (int u = 0; u < DPL; ++u) {
      qv[g][u] = g < G ? h2f(qrow[DPL * lane + u]) : 0.0f;
      acc[g][u] = 0.0f;
    }
    m_run[g] = -__builtin_inff();
    l_run[g] = 0.0f;
    qpos[g] = (p.causal && p.qpos && g < G) ? p.qpos[(int64_t)b * p.q_heads + hq] : 0x7fffffff;
  }
  __syncthreads();

  const cref segs = (cref)p.segments;
  const int begin = split * tps, end = min(p.total_tokens, begin + tps);
  int seg_base = 0;
  for (int s = 0; s < p.num_segments; ++s) {
    const int len = segs[s].len;
    const int lo = max(begin, seg_base), hi = min(end, seg_base + len);
    if (lo < hi) {
      rfsn_ref_store_codes kc, vc;  // field by field: the table lives in the constant address space
      kc.pq = segs[s].k.pq;
      kc.rvq = segs[s].k.rvq;
      kc.active = segs[s].k.active;
      vc.pq = segs[s].v.pq;
      vc.rvq = segs[s].v.rvq;
      vc.active = segs[s].v.active;
      const int64_t tok0 = segs[s].token0;
      const int pos0 = segs[s].pos0;
      const uint16_t* ek = (const uint16_t*)segs[s].exact_k;
      const uint16_t* ev = (const uint16_t*)segs[s].exact_v;
      const int first = lo + (((wave - (lo - begin)) % kRefWaves) + kRefWaves) % kRefWaves;
      for (int i = first; i < hi; i += kRefWaves) {
        const int t = i - seg_base;
        const int64_t row = (tok0 + t) * p.kv_heads + h;
        const int pos = pos0 + t;
        float kk[DPL], vv[DPL];
        const int64_t erow = (tok0 + t) * segs[s].exact_token_stride + (int64_t)h * segs[s].exact_head_stride;
        rebuild<DPL, MW>(kk, kc, kc.pq ? nullptr : ek + erow, row, ktab, M, C, dsub,
                         (const uint16_t*)p.k_rvq_cb, p.rvq_layers, p.rvq_centroids, D, lane);
        rebuild<DPL, MW>(vv, vc, vc.pq ? nullptr : ev + erow, row, vtab, M, C, dsub,
                         (const uint16_t*)p.v_rvq_cb, p.rvq_layers, p.rvq_centroids, D, lane);
#pragma unroll
        for (int g = 0; g < kRefMaxG; ++g) {
          if (g >= G) continue;  // uniform
          float part = 0.0f;
#pragma unroll
          for (int u = 0; u < DPL; ++u) part = __builtin_fmaf(qv[g][u], kk[u], part);
          const float sc = wave_sum64(part) * p.scale;
          if (pos < 0 || pos > qpos[g]) continue;  // masked (uniform)
          const float mn = fmaxf(m_run[g], sc);
          const float corr = __expf(m_run[g] - mn);
          const float pr = __expf(sc - mn);
          l_run[g] = l_run[g] * corr + pr;
#pragma unroll
          for (int u = 0; u < DPL; ++u) acc[g][u] = __builtin_fmaf(pr, vv[u], acc[g][u] * corr);
          m_run[g] = mn;
        }
      }
    }
    seg_base += len;
  }

  // combine the 4 waves: [w][g] m, l, then [w][g][D] acc
  __syncthreads();
  float* red = reinterpret_cast<float*>(tabs);
  float* red_m = red;
  float* red_l = red + kRefWaves * kRefMaxG;
  float* red_a = red + 2 * kRefWaves * kRefMaxG;
#pragma unroll
  for (int g = 0; g < kRefMaxG; ++g) {
    if (g >= G) continue;
    if (lane == 0) {
      red_m[wave * kRefMaxG + g] = m_run[g];
      red_l[wave * kRefMaxG + g] = l_run[g];
    }
#pragma unroll
    for (int u = 0; u < DPL; ++u) red_a[(wave * kRefMaxG + g) * D + DPL * lane + u] = acc[g][u];
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
    if (splits == 1) {
      // a query with no allowed key returns zeros (attention.py:104-105)
      ((uint16_t*)p.out)[((int64_t)b * p.q_heads + hq) * D + c] = f2h(Ls > 0.f ? A / Ls : 0.f);
      continue;
    }
    float* o = reinterpret_cast<float*>(p.workspace) + (((int64_t)b * p.q_heads + hq) * splits + split) * (D + 2);
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
  const int units = p->batch * p->kv_heads;
  int s = (512 + units - 1) / units;
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

template <int DPL>
int launch_ref(const rfsn_ref_params* p, int mw, hipStream_t s) {
  const int splits = ref_splits(p);
  const int tps = (p->total_tokens + splits - 1) / splits;
  const bool shared = p->k_pq_cb == p->v_pq_cb;
  const size_t lds = ref_lds_bytes(p, shared);
  const int blocks = p->batch * p->kv_heads * splits;
#define RFSN_REF(MW)                                                                                       \
  do {                                                                                                     \
    auto kern = ref_attn_kernel<DPL, MW>;                                                                  \
    if (lds > 64 * 1024) (void)hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds); \
    hipLaunchKernelGGL(kern, dim3((unsigned)blocks), dim3(kRefThreads), lds, s, *p, splits, tps, (int)shared); \
  } while (0)
  switch (mw) {
    case 1: RFSN_REF(1); break;
    case 2: RFSN_REF(2); break;
    case 4: RFSN_REF(4); break;
    default: RFSN_REF(8); break;
  }
#undef RFSN_REF
  int st = check_launch("ref_attention");
  if (st || splits == 1) return st;
  return launch_merge(reinterpret_cast<const float*>(p->workspace), (int64_t)p->batch * p->q_heads, splits,
                      p->head_dim, p->out, s);
}

}  // namespace
}  // namespace rfsn

using namespace rfsn;

extern "C" size_t rfsn_ref_attention_workspace_bytes(const rfsn_ref_params* p) {
  if (p == nullptr || p->batch <= 0 || p->q_heads <= 0 || p->kv_heads <= 0 || p->total_tokens <= 0) return 0;
  const int splits = ref_splits(p);
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
  RFSN_REQUIRE(p->rvq_layers >= 0 && (p->rvq_layers == 0 || (p->rvq_centroids >= 1 && p->rvq_centroids <= 65536)),
               "ref_attention: bad RVQ shape");
  RFSN_REQUIRE(p->batch > 0 && p->q_heads > 0 && p->kv_heads > 0 && p->q_heads % p->kv_heads == 0 &&
                   p->q_heads / p->kv_heads <= kRefMaxG,
               "ref_attention: query heads must be a multiple of KV heads, at most 8 per KV head");
  RFSN_REQUIRE(p->q && p->out && p->k_pq_cb && p->v_pq_cb, "ref_attention: null pointer");
  RFSN_REQUIRE(p->rvq_layers == 0 || (p->k_rvq_cb && p->v_rvq_cb), "ref_attention: RVQ codebooks missing");
  RFSN_REQUIRE(p->num_segments >= 0 && p->total_tokens >= 0 && (p->num_segments == 0 || p->segments),
               "ref_attention: bad segment table");
  const size_t shared_lds = ref_lds_bytes(p, p->k_pq_cb == p->v_pq_cb);
  RFSN_REQUIRE(shared_lds <= 160 * 1024, "ref_attention: the PQ codebooks do not fit the LDS (head_dim x centroids too large)");
  RFSN_REQUIRE(p->total_tokens > 0, "ref_attention: empty window (the caller returns zeros, attention.py:104-105)");
  RFSN_REQUIRE(p->splits >= 0 && p->splits <= 8192, "ref_attention: splits must be in [0, 8192]");
  hipStream_t s = (hipStream_t)stream;
  const size_t wsb = rfsn_ref_attention_workspace_bytes(p);
  RFSN_REQUIRE(wsb == 0 || (p->workspace && p->workspace_bytes >= wsb), "ref_attention: workspace too small");
  switch (D) {
    case 64: return launch_ref<1>(p, M / 4, s);
    case 128: return launch_ref<2>(p, M / 4, s);
    default: return launch_ref<4>(p, M / 4, s);
  }
}
