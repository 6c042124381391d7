// Nearest-centroid encode kernels (PQ, subspace RVQ, reference-mode gated
// full-dimension RVQ) and the top-k sparse residual, for gfx950.
//
// Distances follow the canonical chain of quantization.py:92-96:
//   L = fl32(S x*x), X_j = fl32(S x*c_j), R_j = fl32(S c_j*c_j),
//   dist_j = fl32(fl32(L - 2 X_j) + R_j),
// where S is a float64 sum in coordinate order from +0.0.  Products of fp16
// (or fp32) values with fp16 values are exact in float64, so v_fma_f64 in
// coordinate order reproduces S exactly.  Ties go to the lowest index
// (mx.argmin, quantization.py:139; strict-< chunk merge, quantization.py:244).
#include "rfsn_common.h"

#include <type_traits>

namespace rfsn {

namespace {

constexpr int kEncodeThreads = 256;

// One block: 256 vectors x one subspace m of one group.  The subspace
// codebook is staged in LDS as float64 (exact), together with R_j.
template <int DSUB>
__global__ void __launch_bounds__(kEncodeThreads)
pq_encode_kernel(const uint16_t* __restrict__ x, int64_t n, int64_t ldx, int64_t x_gstride,
                 const uint16_t* __restrict__ cb, int M, int C, int dsub_rt, int64_t cb_gstride,
                 uint8_t* __restrict__ codes, int64_t ldc, int64_t codes_gstride,
                 uint16_t* __restrict__ resid, int64_t ldr, int64_t resid_gstride) {
  extern __shared__ double smem[];
  const int d = DSUB > 0 ? DSUB : dsub_rt;
  const int m = blockIdx.y;
  const int g = blockIdx.z;
  double* c64 = smem;                                  // [C][d]
  float* R = reinterpret_cast<float*>(smem + (size_t)C * d);  // [C]
  const uint16_t* cbm = cb + (size_t)g * cb_gstride + (size_t)m * C * d;
  for (int i = threadIdx.x; i < C * d; i += blockDim.x) c64[i] = (double)h2f(cbm[i]);
  __syncthreads();
  for (int j = threadIdx.x; j < C; j += blockDim.x) {
    double acc = 0.0;
    for (int u = 0; u < d; ++u) acc = __builtin_fma(c64[j * d + u], c64[j * d + u], acc);
    R[j] = (float)acc;
  }
  __syncthreads();

  const int64_t v = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (v >= n) return;
  const uint16_t* xv = x + (size_t)g * x_gstride + v * ldx + (size_t)m * d;
  double xs[DSUB > 0 ? DSUB : 32];
  double lacc = 0.0;
#pragma unroll
  for (int u = 0; u < (DSUB > 0 ? DSUB : 32); ++u) {
    if (DSUB == 0 && u >= d) break;
    xs[u] = (double)h2f(xv[u]);
    lacc = __builtin_fma(xs[u], xs[u], lacc);
  }
  const float L = (float)lacc;
  float best = __builtin_inff();
  int bi = 0;
  for (int j = 0; j < C; ++j) {
    const double* cj = c64 + j * d;
    double acc = 0.0;
#pragma unroll
    for (int u = 0; u < (DSUB > 0 ? DSUB : 32); ++u) {
      if (DSUB == 0 && u >= d) break;
      acc = __builtin_fma(xs[u], cj[u], acc);
    }
    const float X = (float)acc;
    const float t = __fsub_rn(L, 2.0f * X);
    const float dist = __fadd_rn(t, R[j]);
    if (dist < best) {
      best = dist;
      bi = j;
    }
  }
  codes[(size_t)g * codes_gstride + v * ldc + m] = (uint8_t)bi;
  if (resid != nullptr) {
    uint16_t* rv = resid + (size_t)g * resid_gstride + v * ldr + (size_t)m * d;
    for (int u = 0; u < d; ++u) {
      const float diff = __fsub_rn((float)xs[u], (float)c64[bi * d + u]);
      rv[u] = f2h(diff);
    }
  }
}

// Reference-mode RVQ gate: fl32(sqrt(fl32(S r^2))) > thr, S summed in
// float64 in coordinate order.  Rows of 16-byte aligned fp16 load 8
// coordinates per instruction (a lane's row is two 128-byte lines, read
// whole), others one at a time.
__global__ void rvq_gate_kernel(const uint16_t* __restrict__ r, int64_t n, int D, int64_t ld, float thr,
                                uint8_t* __restrict__ mask) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const uint16_t* row = r + i * ld;
  double acc = 0.0;
  if (D % 8 == 0 && ld % 8 == 0 && reinterpret_cast<uintptr_t>(r) % 16 == 0) {  // uniform
    for (int u0 = 0; u0 < D; u0 += 32) {
      uint4 w[4];
#pragma unroll
      for (int k = 0; k < 4; ++k) w[k] = u0 + 8 * k < D ? reinterpret_cast<const uint4*>(row + u0)[k] : make_uint4(0u, 0u, 0u, 0u);
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        if (u0 + 8 * k >= D) break;
        const uint32_t ww[4] = {w[k].x, w[k].y, w[k].z, w[k].w};
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const double v = (double)h2f((uint16_t)(ww[e >> 1] >> (16 * (e & 1))));
          acc = __builtin_fma(v, v, acc);
        }
      }
    }
  } else {
    for (int u = 0; u < D; ++u) {
      const double v = (double)h2f(row[u]);
      acc = __builtin_fma(v, v, acc);
    }
  }
  const float s = (float)acc;
  // correctly rounded float sqrt: the f64 square root of an f32 input rounded
  // to f32 is the correctly rounded f32 square root (53 >= 2*24+2).
  const float norm = (float)__builtin_sqrt((double)s);
  mask[i] = norm > thr ? 1 : 0;
}

// Stream compaction of a 0/1 mask into ascending offsets (single pass per
// 1024-element tile: tile counts, then tile prefix, then scatter).
constexpr int kScanTile = 1024;

__global__ void mask_count_kernel(const uint8_t* __restrict__ mask, int64_t n, int32_t* __restrict__ tile_counts) {
  __shared__ int32_t wsum[kScanTile / 64];
  const int64_t i = (int64_t)blockIdx.x * kScanTile + threadIdx.x;
  int v = (i < n && mask[i]) ? 1 : 0;
  int s = v;
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) s += __shfl_xor(s, o, 64);
  if ((threadIdx.x & 63) == 0) wsum[threadIdx.x >> 6] = s;
  __syncthreads();
  if (threadIdx.x == 0) {
    int t = 0;
    for (int w = 0; w < kScanTile / 64; ++w) t += wsum[w];
    tile_counts[blockIdx.x] = t;
  }
}

__global__ void tile_prefix_kernel(int32_t* __restrict__ tile_counts, int64_t tiles, int32_t* __restrict__ count) {
  // one wave: exclusive prefix over 64 tiles at a time (shuffle scan), the
  // running total carried from chunk to chunk
  if (blockIdx.x != 0 || threadIdx.x >= 64) return;
  const int lane = threadIdx.x;
  int32_t carry = 0;
  for (int64_t t0 = 0; t0 < tiles; t0 += 64) {
    const int64_t t = t0 + lane;
    const int32_t c = t < tiles ? tile_counts[t] : 0;
    int32_t inc = c;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      const int32_t y = __shfl_up(inc, o, 64);
      if (lane >= o) inc += y;
    }
    if (t < tiles) tile_counts[t] = carry + inc - c;
    carry += __shfl(inc, 63, 64);
  }
  if (lane == 0) count[0] = carry;
}

__global__ void mask_scatter_kernel(const uint8_t* __restrict__ mask, int64_t n, const int32_t* __restrict__ tile_base,
                                    int32_t* __restrict__ offsets) {
  __shared__ int32_t wpre[kScanTile / 64];
  const int64_t i = (int64_t)blockIdx.x * kScanTile + threadIdx.x;
  const int v = (i < n && mask[i]) ? 1 : 0;
  const int lane = threadIdx.x & 63;
  const uint64_t ballot = __ballot(v);
  const int before = __popcll(ballot & ((lane == 0) ? 0ull : (~0ull >> (64 - lane))));
  if (lane == 0) wpre[threadIdx.x >> 6] = __popcll(ballot);
  __syncthreads();
  if (threadIdx.x == 0) {
    int acc = 0;
    for (int w = 0; w < kScanTile / 64; ++w) {
      const int c = wpre[w];
      wpre[w] = acc;
      acc += c;
    }
  }
  __syncthreads();
  if (v) offsets[tile_base[blockIdx.x] + wpre[threadIdx.x >> 6] + before] = (int32_t)i;
}

// Reference-mode full-dimension RVQ: one wave per active row; lanes split the
// centroids, argmin merged across the wave with lowest index on ties.
__global__ void __launch_bounds__(256)
rvq_full_kernel(const uint16_t* __restrict__ resid, int64_t ld, int D, const int32_t* __restrict__ offsets,
                int64_t active, const uint16_t* __restrict__ cb, int L, int C, uint16_t* __restrict__ codes) {
  extern __shared__ double run_all[];  // [waves][D] running residual as f64 (values are fp32)
  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  const int64_t a = (int64_t)blockIdx.x * (blockDim.x >> 6) + wave;
  double* run = run_all + (size_t)wave * D;
  const bool live = a < active;
  if (live) {
    const uint16_t* row = resid + (int64_t)offsets[a] * ld;
    for (int u = lane; u < D; u += 64) run[u] = (double)h2f(row[u]);
  }
  __syncthreads();
  for (int layer = 0; layer < L; ++layer) {
    float best = __builtin_inff();
    int bi = 0x7fffffff;
    if (live) {
      double lacc = 0.0;
      for (int u = 0; u < D; ++u) lacc = __builtin_fma(run[u], run[u], lacc);
      const float Lf = (float)lacc;
      const uint16_t* cbl = cb + (size_t)layer * C * D;
      for (int j = lane; j < C; j += 64) {
        const uint16_t* cj = cbl + (size_t)j * D;
        double xacc = 0.0, racc = 0.0;
        for (int u = 0; u < D; ++u) {
          const double c = (double)h2f(cj[u]);
          xacc = __builtin_fma(run[u], c, xacc);
          racc = __builtin_fma(c, c, racc);
        }
        const float t = __fsub_rn(Lf, 2.0f * (float)xacc);
        const float dist = __fadd_rn(t, (float)racc);
        if (dist < best) {  // ascending j per lane: first min kept
          best = dist;
          bi = j;
        }
      }
      // wave argmin, ties -> lowest index
#pragma unroll
      for (int o = 32; o > 0; o >>= 1) {
        const float ob = __shfl_xor(best, o, 64);
        const int oi = __shfl_xor(bi, o, 64);
        if (ob < best || (ob == best && oi < bi)) {
          best = ob;
          bi = oi;
        }
      }
      if (bi == 0x7fffffff) bi = 0;  // all-NaN row: mx.argmin would return 0
      if (lane == 0) codes[a * L + layer] = (uint16_t)bi;
    }
    __syncthreads();
    if (live) {
      const uint16_t* cj = cb + (size_t)layer * C * D + (size_t)bi * D;
      for (int u = lane; u < D; u += 64) run[u] = (double)__fsub_rn((float)run[u], h2f(cj[u]));
    }
    __syncthreads();
  }
}

// Top-k |r2| of r2 = fl32(x - fp16(base + rvq)) per vector; descending |r2|,
// ties to the lower coordinate.  One thread per vector; codebooks are read
// through the cache (they are a few KB and shared by all vectors).
template <int K>
__global__ void __launch_bounds__(256)
sparse_topk_kernel(const uint16_t* __restrict__ x, int64_t n, int D, int64_t ldx,
                   const uint8_t* __restrict__ pq, int M, int C, const uint16_t* __restrict__ pq_cb,
                   const uint8_t* __restrict__ rvq, int Mr, int Cr, const uint16_t* __restrict__ rvq_cb,
                   uint8_t* __restrict__ idx_out, uint16_t* __restrict__ val_out) {
  const int64_t v = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (v >= n) return;
  const int d = D / M;
  const int dr = Mr > 0 ? D / Mr : 1;
  float bmag[K];
  float bval[K];
  int bidx[K];
#pragma unroll
  for (int j = 0; j < K; ++j) {
    bmag[j] = -1.0f;
    bval[j] = 0.0f;
    bidx[j] = 0;
  }
  const uint16_t* xv = x + v * ldx;
  for (int i = 0; i < D; ++i) {
    const int m = i / d;
    uint16_t rec = pq_cb[((size_t)m * C + pq[v * M + m]) * d + (i - m * d)];
    if (Mr > 0) {
      const int mr = i / dr;
      rec = hadd_bits(rec, rvq_cb[((size_t)mr * Cr + rvq[v * Mr + mr]) * dr + (i - mr * dr)]);
    }
    const float r2 = __fsub_rn(h2f(xv[i]), h2f(rec));
    const float mag = fabsf(r2);
    if (mag > bmag[K - 1]) {
      // insert keeping earlier (lower-index) entries ahead of equal magnitudes
      int pos = K - 1;
#pragma unroll
      for (int j = K - 1; j > 0; --j) {
        if (j <= pos && mag > bmag[j - 1]) {
          bmag[j] = bmag[j - 1];
          bval[j] = bval[j - 1];
          bidx[j] = bidx[j - 1];
          pos = j - 1;
        }
      }
      bmag[pos] = mag;
      bval[pos] = r2;
      bidx[pos] = i;
    }
  }
#pragma unroll
  for (int j = 0; j < K; ++j) {
    idx_out[v * K + j] = (uint8_t)bidx[j];
    val_out[v * K + j] = f2h(bval[j]);
  }
}

// ---------------------------------------------------------------------------
// Nearest-centroid search on MFMA (subspace dims d = 4, 8 and 16).
//
// Half the squared distance is one MFMA dot product of augmented operands:
//   centroid row  [ c_j (d) | rh_j  rl_j  1  1 | 0 ... ]   (A, 32 centroids)
//   vector column [ -x  (d) | 1     1  lh  ll  | 0 ... ]   (B, 32 vectors)
//   z_j = -x.c_j + (rh_j + rl_j) + (lh + ll) ~= (L - 2 X_j + R_j) / 2
// with R_j / 2 = rh_j + rl_j and L / 2 = lh + ll split into fp16 pairs
// (22 significant bits).  The products are exact in fp32 and the MFMA
// accumulates in fp32, so |z_j - dist_j / 2| <= E with dist_j the canonical
// distance and E = 2^-17 (L + R_max) + 2^-22, four times the worst-case sum
// of the accumulation (d + 4 terms), split-representation and canonical
// rounding errors.
//
// Each lane keeps the three smallest keys (z with its low byte replaced by
// the centroid index) of its 128 (vector, centroid) pairs; the two lanes of a
// vector merge theirs.  With v1 <= v2 <= v3 the key values and t the key
// truncation (2^-14 |v|):
//   v2 - v1 > 2E + t  -> the smallest key's centroid is the canonical code;
//   v3 - v1 > 2E + t  -> only the two smallest can be the code: both are
//                        rescored exactly (the duplicate-centroid case);
//   otherwise (or non-finite values) the exact canonical scan over all C.
// The exact rescoring uses the float64 chain of pq_encode_kernel, so codes
// are identical to it (and to the oracle) by construction.
constexpr int kMfmaVecsPerWave = 32;
constexpr int kMfmaThreads = 256;
constexpr int kMfmaVecsPerBlock = (kMfmaThreads / 64) * kMfmaVecsPerWave;

typedef _Float16 mh4 __attribute__((ext_vector_type(4)));
typedef _Float16 mh8 __attribute__((ext_vector_type(8)));
typedef float mf16 __attribute__((ext_vector_type(16)));

__device__ __forceinline__ int med3i(int a, int b, int c) { return max(min(a, b), min(max(a, b), c)); }
// insert key k into the sorted triple (m1 <= m2 <= m3)
__device__ __forceinline__ void top3_insert(int& m1, int& m2, int& m3, int k) {
  const int n3 = med3i(m2, m3, k);
  const int n2 = med3i(m1, m2, k);
  m1 = min(m1, k);
  m2 = n2;
  m3 = n3;
}
__device__ __forceinline__ float key_value(int k) { return __builtin_bit_cast(float, k & (int)0xFFFFFF00); }
constexpr int kNoKey = 0x7F8000FF;  // value +inf, above every finite key

template <int DS>
__global__ void __launch_bounds__(kMfmaThreads)
pq_encode_mfma_kernel(const uint16_t* __restrict__ x, int64_t n, int64_t ldx, int64_t x_gstride,
                      const uint16_t* __restrict__ cb, int M, int C, int64_t cb_gstride,
                      uint8_t* __restrict__ codes, int64_t ldc, int64_t codes_gstride,
                      uint16_t* __restrict__ resid, int64_t ldr, int64_t resid_gstride) {
  // row depth: 32x32x8 (d = 4), one 32x32x16 (d = 8) or two (d = 16: the
  // coordinates, then the augmented group)
  constexpr int K = DS == 4 ? 8 : (DS == 8 ? 16 : 32);
  constexpr int KH = DS == 16 ? 8 : K / 2;  // operand halves per lane and MFMA
  constexpr int NSTEP = DS == 16 ? 2 : 1;
  constexpr int AUG = DS == 16 ? 16 : KH;   // first element of the augmented group
  __shared__ __align__(16) _Float16 tab[256 * K];  // augmented centroid rows
  __shared__ float Rs[256];                        // canonical R_j
  __shared__ uint32_t rmax_s[kMfmaThreads / 64];
  const int m = blockIdx.y, g = blockIdx.z;
  const uint16_t* cbm = cb + (size_t)g * cb_gstride + (size_t)m * C * DS;
  const int nch = (C + 31) / 32;  // 32-centroid chunks
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int col = lane & 31, hi = lane >> 5;
  // the block's first tile of vectors: its slices load ahead of the codebook staging
  const int64_t ntiles = (n + kMfmaVecsPerBlock - 1) / kMfmaVecsPerBlock;
  uint16_t xr[DS];
  auto load_slice = [&](int64_t tile) {
    const int64_t v = (tile * (kMfmaThreads / 64) + wave) * kMfmaVecsPerWave + col;
    const bool live = v < n;
    const uint16_t* xv = x + (size_t)g * x_gstride + (live ? v : 0) * ldx + (size_t)m * DS;
#pragma unroll
    for (int u = 0; u < DS; ++u) xr[u] = live ? xv[u] : (uint16_t)0;
  };
  load_slice(blockIdx.x);

  uint32_t rmax_t = 0;  // this thread's largest R_j, as bits (R >= 0; NaN above +inf)
  for (int j = threadIdx.x; j < 32 * nch; j += kMfmaThreads) {
    _Float16 row[K];  // built in registers, stored as 16-byte units
#pragma unroll
    for (int u = 0; u < K; ++u) row[u] = (_Float16)0.0f;
    if (j < C) {
      double acc = 0.0;
#pragma unroll
      for (int u = 0; u < DS; ++u) {
        const uint16_t cu = cbm[j * DS + u];
        const double c = (double)h2f(cu);
        acc = __builtin_fma(c, c, acc);
        row[u] = __builtin_bit_cast(_Float16, cu);
      }
      const float R = (float)acc;
      const float half_r = 0.5f * R;
      const _Float16 rh = (_Float16)half_r;
      const _Float16 rl = (_Float16)(half_r - (float)rh);
      row[AUG] = rh;
      row[AUG + 1] = rl;
      row[AUG + 2] = (_Float16)1.0f;
      row[AUG + 3] = (_Float16)1.0f;
      Rs[j] = R;
      rmax_t = max(rmax_t, __builtin_bit_cast(uint32_t, R) & 0x7FFFFFFFu);
    }
#pragma unroll
    for (int c = 0; c < K / 8; ++c) {
      mh8 w;
#pragma unroll
      for (int u = 0; u < 8; ++u) w[u] = row[8 * c + u];
      *reinterpret_cast<mh8*>(tab + j * K + 8 * c) = w;
    }
  }
  // block max of R_j (a NaN R makes every lane take the exact path)
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) rmax_t = max(rmax_t, (uint32_t)__shfl_xor((int)rmax_t, o, 64));
  if ((threadIdx.x & 63) == 0) rmax_s[threadIdx.x >> 6] = rmax_t;
  __syncthreads();
  uint32_t rmax_b = rmax_s[0];
#pragma unroll
  for (int w = 1; w < kMfmaThreads / 64; ++w) rmax_b = max(rmax_b, rmax_s[w]);
  const float rmax = __builtin_bit_cast(float, rmax_b);

  // residual rows take one DS*2-byte store when the output is aligned for it
  const bool vec_ok = resid != nullptr && ldr % DS == 0 && (reinterpret_cast<uintptr_t>(resid) % (2 * DS)) == 0 &&
                      (resid_gstride % DS) == 0;
  // the block's tiles of vectors: blockIdx.x, + gridDim.x, ... (the staged
  // codebook serves them all)
  for (int64_t tile = blockIdx.x; tile < ntiles; tile += gridDim.x) {
  if (tile != blockIdx.x) load_slice(tile);
  const int64_t v = (tile * (kMfmaThreads / 64) + wave) * kMfmaVecsPerWave + col;
  const bool live = v < n;
  // the lane's vector: canonical L and the B operand
  double xs[DS];
  double lacc = 0.0;
#pragma unroll
  for (int u = 0; u < DS; ++u) {
    xs[u] = (double)h2f(xr[u]);
    lacc = __builtin_fma(xs[u], xs[u], lacc);
  }
  const float L = (float)lacc;
  const float half_l = 0.5f * L;
  const _Float16 lh = (_Float16)half_l;
  const _Float16 ll = (_Float16)(half_l - (float)lh);
  // B of MFMA step st: lane (col, hi) holds k = 16 st + KH hi .. + KH - 1
  _Float16 bop[NSTEP][KH];
#pragma unroll
  for (int st = 0; st < NSTEP; ++st)
#pragma unroll
    for (int u = 0; u < KH; ++u) bop[st][u] = (_Float16)0.0f;
  if constexpr (DS == 16) {
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      // -fp16(x) of coordinate 8 hi + u: the half's sign flipped, chosen by a
      // bit mask (a select between xs[u] and xs[8 + u] became an indexed
      // access that kept xs in scratch memory)
      const uint32_t msk = 0u - (uint32_t)hi;
      const uint32_t w = ((uint32_t)xr[u] ^ (((uint32_t)xr[u] ^ (uint32_t)xr[8 + u]) & msk)) ^ 0x8000u;
      bop[0][u] = __builtin_bit_cast(_Float16, (uint16_t)w);
    }
    if (hi == 0) {
      bop[1][0] = (_Float16)1.0f;
      bop[1][1] = (_Float16)1.0f;
      bop[1][2] = lh;
      bop[1][3] = ll;
    }
  } else if (hi == 0) {
#pragma unroll
    for (int u = 0; u < DS; ++u) bop[0][u] = (_Float16)(-(float)xs[u]);
  } else {
    bop[0][0] = (_Float16)1.0f;
    bop[0][1] = (_Float16)1.0f;
    bop[0][2] = lh;
    bop[0][3] = ll;
  }

  // screen: the three smallest keys of the lane's rows 8(r/4) + 4 hi + r%4
  // two independent lists (even / odd accumulator registers) for more ILP
  int m1 = kNoKey, m2 = kNoKey, m3 = kNoKey;
  int n1 = kNoKey, n2 = kNoKey, n3 = kNoKey;
  auto chunk = [&](int t, bool partial) {
    mf16 acc = {};
    const _Float16* arow = tab + (32 * t + col) * K + KH * hi;
    if constexpr (DS == 4) {
      mh4 a, b;
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        a[u] = arow[u];
        b[u] = bop[0][u];
      }
      acc = __builtin_amdgcn_mfma_f32_32x32x8f16(a, b, acc, 0, 0, 0);
    } else {
#pragma unroll
      for (int st = 0; st < NSTEP; ++st) {
        mh8 a, b;
#pragma unroll
        for (int u = 0; u < 8; ++u) {
          a[u] = arow[16 * st + u];
          b[u] = bop[st][u];
        }
        acc = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, acc, 0, 0, 0);
      }
    }
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int jl = 32 * t + 8 * (r >> 2) + (r & 3);  // centroid index without the lane's 4 hi
      // the element goes through a scalar first: bit-casting a vector element
      // subscript in place reads element 0 with this compiler
      const float z = acc[r];
      int key = (__builtin_bit_cast(int, z) & (int)0xFFFFFF00) | jl;
      if (partial && jl + 4 * hi >= C) key = kNoKey;
      if (r & 1)
        top3_insert(n1, n2, n3, key);
      else
        top3_insert(m1, m2, m3, key);
    }
  };
  const int nfull = C / 32;
  for (int t = 0; t < nfull; ++t) chunk(t, false);
  if (nfull < nch) chunk(nfull, true);  // uniform: the last, partial chunk
  top3_insert(m1, m2, m3, n1);
  top3_insert(m1, m2, m3, n2);
  top3_insert(m1, m2, m3, n3);
  // add the lane's row offset, then merge with the other lane of the vector
  if (m1 != kNoKey) m1 |= 4 * hi;
  if (m2 != kNoKey) m2 |= 4 * hi;
  if (m3 != kNoKey) m3 |= 4 * hi;
  {
    const int o1 = __shfl_xor(m1, 32, 64), o2 = __shfl_xor(m2, 32, 64), o3 = __shfl_xor(m3, 32, 64);
    top3_insert(m1, m2, m3, o1);
    top3_insert(m1, m2, m3, o2);
    top3_insert(m1, m2, m3, o3);
  }
  const float v1 = key_value(m1), v2 = key_value(m2), v3 = key_value(m3);
  // (d + 6) 2^-23 (L + R) covers the accumulation, split and canonical errors;
  // E keeps at least a 4x margin over it (d = 16: 2^-16)
  const float E = (DS == 16 ? 0x1p-16f : 0x1p-17f) * (L + rmax) + 0x1p-22f;
  const bool unique = v2 - v1 > 2.0f * E + 0x1p-14f * (fabsf(v1) + fabsf(v2));
  const bool pair = v3 - v1 > 2.0f * E + 0x1p-14f * (fabsf(v1) + fabsf(v3));
  const bool safe = rmax < 120000.0f;  // R / 2 representable in fp16 for every centroid

  // canonical distance of centroid j (the float64 chain of pq_encode_kernel)
  auto exact = [&](int j) {
    double acc = 0.0;
#pragma unroll
    for (int u = 0; u < DS; ++u) acc = __builtin_fma(xs[u], (double)(float)tab[j * K + u], acc);
    const float X = (float)acc;
    return __fadd_rn(__fsub_rn(L, 2.0f * X), Rs[j]);
  };
  int code;
  if (safe && unique) {
    code = m1 & 0xFF;
  } else if (safe && pair) {
    const int ja = min(m1 & 0xFF, m2 & 0xFF), jb = max(m1 & 0xFF, m2 & 0xFF);
    const float da = exact(ja), db = exact(jb);
    code = db < da ? jb : ja;  // first min: ties keep the lower index
  } else {
    float best = __builtin_inff();
    code = 0;
    for (int j = 0; j < C; ++j) {
      const float dj = exact(j);
      if (dj < best) {
        best = dj;
        code = j;
      }
    }
  }
  if (!live || hi != 0) continue;
  codes[(size_t)g * codes_gstride + v * ldc + m] = (uint8_t)code;
  if (resid != nullptr) {
    uint16_t* rv = resid + (size_t)g * resid_gstride + v * ldr + (size_t)m * DS;
    uint16_t r[DS];
#pragma unroll
    for (int u = 0; u < DS; ++u) r[u] = f2h(__fsub_rn((float)xs[u], (float)tab[code * K + u]));
    if (vec_ok) {
      if constexpr (DS == 4) {
        *reinterpret_cast<uint2*>(rv) = make_uint2(r[0] | ((uint32_t)r[1] << 16), r[2] | ((uint32_t)r[3] << 16));
      } else {
#pragma unroll
        for (int h = 0; h < DS / 8; ++h)
          reinterpret_cast<uint4*>(rv)[h] =
              make_uint4(r[8 * h] | ((uint32_t)r[8 * h + 1] << 16), r[8 * h + 2] | ((uint32_t)r[8 * h + 3] << 16),
                         r[8 * h + 4] | ((uint32_t)r[8 * h + 5] << 16), r[8 * h + 6] | ((uint32_t)r[8 * h + 7] << 16));
      }
    } else {
#pragma unroll
      for (int u = 0; u < DS; ++u) rv[u] = r[u];
    }
  }
  }  // tiles
}

template <int DS>
int launch_pq_mfma(const void* x, int64_t n, int64_t ldx, int64_t xg, const void* cb, int M, int C, int64_t cbg,
                   uint8_t* codes, int64_t ldc, int64_t cg, void* resid, int64_t ldr, int64_t rg, int groups,
                   hipStream_t s) {
  // about 16 blocks per CU in all: each block stages its subspace's codebook
  // once and takes every gridDim.x-th tile of 128 vectors
  const int64_t tiles = ceil_div(n, kMfmaVecsPerBlock);
  const int64_t want = ceil_div(4096, (int64_t)M * groups);
  dim3 grid((unsigned)std::max<int64_t>(1, std::min(tiles, want)), (unsigned)M, (unsigned)groups);
  hipLaunchKernelGGL(pq_encode_mfma_kernel<DS>, grid, dim3(kMfmaThreads), 0, s, (const uint16_t*)x, n, ldx, xg,
                     (const uint16_t*)cb, M, C, cbg, codes, ldc, cg, (uint16_t*)resid, ldr, rg);
  return check_launch("pq_encode");
}

// Top-k |r2| for head_dim 64: four lanes per vector, 16 coordinates each,
// then the lanes' lists merge across the quad.  Order and tie rule are those
// of sparse_topk_kernel (|r2| descending, ties to the lower coordinate, NaN
// never enters, unused slots (index 0, value 0)).  An entry is one 64-bit key
//   |r2| bits (32) | 64 - index (16) | fp16(r2) (16),
// so the rank order is the unsigned key order (|r2| >= 0; the index field
// breaks ties toward the lower coordinate) and the stored value rides along;
// every entry is nonzero, so 0 marks an unused slot.  A sorted insert is then
// a max/min network with static indices.
template <int K>
__device__ __forceinline__ void topk_insert(uint64_t (&t)[K], uint64_t x) {
#pragma unroll
  for (int j = K - 1; j > 0; --j) t[j] = __builtin_elementwise_max(t[j], __builtin_elementwise_min(t[j - 1], x));
  t[0] = __builtin_elementwise_max(t[0], x);
}

template <int K, int DS, bool RVQ>
__global__ void __launch_bounds__(256)
sparse_topk64_kernel(const uint16_t* __restrict__ x, int64_t n, int64_t ldx, const uint8_t* __restrict__ pq, int M,
                     int C, const uint16_t* __restrict__ pq_cb, const uint8_t* __restrict__ rvq, int Cr,
                     const uint16_t* __restrict__ rvq_cb, uint8_t* __restrict__ idx_out,
                     uint16_t* __restrict__ val_out) {
  constexpr int NS = 16 / DS;  // subspaces of the lane's 16 coordinates (same split for both stages)
  typedef typename std::conditional<DS == 4, uint2, uint4>::type E;
  const int64_t v = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) >> 2;
  const int q = threadIdx.x & 3;  // quarter: coordinates 16q .. 16q + 15
  const bool live = v < n;
  const int64_t vv = live ? v : 0;
  const int m0 = q * NS;
  // all loads first: the vector's 16 coordinates, its codes and the centroid entries
  const uint4* xq = reinterpret_cast<const uint4*>(x + vv * ldx + 16 * q);
  const uint4 xa = xq[0], xb = xq[1];
  E pe[NS], re[NS];
#pragma unroll
  for (int s = 0; s < NS; ++s) {
    pe[s] = *reinterpret_cast<const E*>(pq_cb + ((size_t)(m0 + s) * C + pq[vv * M + m0 + s]) * DS);
    if constexpr (RVQ) re[s] = *reinterpret_cast<const E*>(rvq_cb + ((size_t)(m0 + s) * Cr + rvq[vv * M + m0 + s]) * DS);
  }
  const uint32_t xw[8] = {xa.x, xa.y, xa.z, xa.w, xb.x, xb.y, xb.z, xb.w};
  uint32_t pw[8], rw[8];
#pragma unroll
  for (int s = 0; s < NS; ++s) {
    if constexpr (DS == 4) {
      pw[2 * s] = pe[s].x;
      pw[2 * s + 1] = pe[s].y;
      if constexpr (RVQ) {
        rw[2 * s] = re[s].x;
        rw[2 * s + 1] = re[s].y;
      }
    } else {
      pw[4 * s] = pe[s].x;
      pw[4 * s + 1] = pe[s].y;
      pw[4 * s + 2] = pe[s].z;
      pw[4 * s + 3] = pe[s].w;
      if constexpr (RVQ) {
        rw[4 * s] = re[s].x;
        rw[4 * s + 1] = re[s].y;
        rw[4 * s + 2] = re[s].z;
        rw[4 * s + 3] = re[s].w;
      }
    }
  }
  uint64_t t[K];
#pragma unroll
  for (int j = 0; j < K; ++j) t[j] = 0;  // unused slot, below every entry
#pragma unroll
  for (int u = 0; u < 16; ++u) {
    const uint16_t xh = (uint16_t)(xw[u >> 1] >> (16 * (u & 1)));
    uint16_t rec = (uint16_t)(pw[u >> 1] >> (16 * (u & 1)));
    if constexpr (RVQ) rec = hadd_bits(rec, (uint16_t)(rw[u >> 1] >> (16 * (u & 1))));
    const float r2 = __fsub_rn(h2f(xh), h2f(rec));
    const uint32_t mb = __builtin_bit_cast(uint32_t, r2) & 0x7FFFFFFFu;
    if (mb <= 0x7F800000u) {  // NaN never enters
      const int i = 16 * q + u;
      topk_insert(t, ((uint64_t)mb << 32) | ((uint64_t)(64 - i) << 16) | f2h(r2));
    }
  }
  // merge across the quad (lanes 4v' .. 4v'+3 of the wave)
#pragma unroll
  for (int o = 1; o < 4; o <<= 1) {
    uint64_t ot[K];
#pragma unroll
    for (int j = 0; j < K; ++j) ot[j] = __shfl_xor(t[j], o, 64);
#pragma unroll
    for (int j = 0; j < K; ++j) topk_insert(t, ot[j]);
  }
  if (!live || q != 0) return;
#pragma unroll
  for (int j = 0; j < K; ++j) {
    const bool real = t[j] != 0;
    idx_out[v * K + j] = real ? (uint8_t)(64 - (int)((t[j] >> 16) & 0xFFFF)) : (uint8_t)0;
    val_out[v * K + j] = real ? (uint16_t)(t[j] & 0xFFFF) : (uint16_t)0;
  }
}

// ---------------------------------------------------------------- fused warm encode
// One launch encodes up to kMaxJobs vector sets (a chunk's K and V): PQ, the
// subspace RVQ stage on the register-resident fp16 PQ residual, then the
// top-k |r2|, head_dim 64.  A block (16 waves) holds 256 vectors of one job
// and first writes the augmented centroid rows of every (stage, subspace)
// into LDS: coordinates in 8-byte groups, then (R/2 hi, R/2 lo, 1, 1), with
// R the canonical fl32(S c*c); rows past the codebook get R/2 = +inf.  A wave
// takes 16 vectors through every subspace: v_mfma_f32_16x16x16_f16 with
// A = 16 centroid rows (lane l: row l % 16, k-group l / 16) and B = the 16
// vectors (-x in the coordinate groups, (1, 1, L/2 hi, L/2 lo) in the next)
// gives dist/2 of centroid 16t + 4(l / 16) + i and vector l % 16 in
// accumulator i, so the four lanes of a vector screen 64 centroids each with
// the keys and certificate of pq_encode_mfma_kernel, merge their top three,
// and settle uncertain cases with the canonical float64 chain.  The residual
// never leaves registers; each lane folds its share of the vector's r2 into a
// running top-k, and the codes are written once per vector at the end.
constexpr int kMaxJobs = 4;
constexpr int kFeWaves = 16;
constexpr int kFeThreads = kFeWaves * 64;
constexpr int kFeVecs = kFeWaves * 16;  // vectors per block

struct EncodeJob {
  const uint16_t* x;
  int64_t n;
  int64_t ldx;
  const uint16_t* pq_cb;
  const uint16_t* rvq_cb;
  uint8_t* pq;
  uint8_t* rvq;
  uint8_t* sidx;
  uint16_t* sval;
  int32_t block0;  // first block of the job in the grid
};
struct EncodeJobs {
  EncodeJob j[kMaxJobs];
  int32_t count;
  int32_t C;   // PQ centroids
  int32_t Cr;  // RVQ centroids
};

typedef _Float16 fh4 __attribute__((ext_vector_type(4)));
typedef float ff4 __attribute__((ext_vector_type(4)));

// Insert keys a, b into the sorted pair m1 <= m2 in three VALU ops: the new
// second smallest is min(m2, med3(m1, a, b)) (m2 >= m1, so the second of
// {m1, m2, a, b} is the smaller of m2 and the second of {m1, a, b}).
__device__ __forceinline__ void key_insert2x2(int& m1, int& m2, int a, int b) {
  int t;
  asm("v_med3_i32 %2, %0, %3, %4\n\t"
      "v_min3_i32 %0, %0, %3, %4\n\t"
      "v_min_i32_e32 %1, %1, %2"
      : "+v"(m1), "+v"(m2), "=&v"(t)
      : "v"(a), "v"(b));
}
// Insert key k into the sorted triple m1 <= m2 <= m3 in three VALU ops.
// Written out because the compiler, knowing m1 <= m2, turns the middle
// median into a min / max pair.  k must be an ordinary VALU result, never an
// MFMA destination read directly: the compiler pads MFMA -> VALU read hazards
// only for reads it can see.
__device__ __forceinline__ void key_insert3(int& m1, int& m2, int& m3, int k) {
  asm("v_med3_i32 %2, %1, %2, %3\n\t"
      "v_med3_i32 %1, %0, %1, %3\n\t"
      "v_min_i32_e32 %0, %0, %3"
      : "+v"(m1), "+v"(m2), "+v"(m3)
      : "v"(k));
}
// The value of lane l ^ 16: ds_swizzle in bit-mask mode (and 0x1F, xor 0x10)
// within each half of the wave; of lane l ^ 32: ds_bpermute from byte address
// xor32_addr = 4 (l ^ 32).  Both run on the LDS crossbar, not the VALU.
__device__ __forceinline__ int lane_xor16(int v) { return __builtin_amdgcn_ds_swizzle(v, 0x401F); }
__device__ __forceinline__ int lane_xor32(int v, int xor32_addr) { return __builtin_amdgcn_ds_bpermute(xor32_addr, v); }

template <int DS, bool RVQ, int KS>
__global__ void __launch_bounds__(kFeThreads, 1) warm_encode_fused_kernel(const EncodeJobs jobs) {
  constexpr int M = 64 / DS;
  constexpr int S = RVQ ? 2 : 1;       // stages
  constexpr int CG = DS / 4;           // coordinate k-groups of a row
  constexpr int RB = (CG + 1) * 8;     // row bytes: coordinate groups, then the R/2 group
  constexpr int TB = 256 * RB;         // one (stage, subspace) table
  __shared__ __align__(16) uint8_t tab[S * M * TB];
  __shared__ uint32_t rmax_s[S * M];
  // the block's job (uniform)
  int ji = 0;
#pragma unroll
  for (int i = 1; i < kMaxJobs; ++i)
    if (i < jobs.count && (int)blockIdx.x >= jobs.j[i].block0) ji = i;
  const EncodeJob& job = jobs.j[ji];
  const int C = jobs.C, Cr = jobs.Cr;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;

  // ---- tables: row r of (stage s, subspace m) at tab + (s*M + m)*TB + r*RB.
  // Thread tid builds rows i = tid + kFeThreads * it; every centroid load is
  // issued before the first row is formed, so the set-up waits for one memory
  // round trip.
  constexpr int kRows = S * M * 256 / kFeThreads;
  static_assert(S * M * 256 % kFeThreads == 0, "table rows per thread");
  for (int i = tid; i < S * M; i += kFeThreads) rmax_s[i] = 0u;
  uint2 cw[kRows][CG];  // the centroids' coordinates, 4 fp16 per group
#pragma unroll
  for (int it = 0; it < kRows; ++it) {
    const int i = tid + kFeThreads * it;
    const int r = i & 255, sm = i >> 8, s = sm / M, m = sm % M;
    const int nc = s == 0 ? C : Cr;
    const uint16_t* cb = (s == 0 ? job.pq_cb : job.rvq_cb) + ((size_t)m * nc + (r < nc ? r : 0)) * DS;
#pragma unroll
    for (int gq = 0; gq < CG; ++gq)
      cw[it][gq] = r < nc ? reinterpret_cast<const uint2*>(cb)[gq] : make_uint2(0u, 0u);
  }
  __syncthreads();  // rmax_s cleared
#pragma unroll
  for (int it = 0; it < kRows; ++it) {
    const int i = tid + kFeThreads * it;
    const int r = i & 255, sm = i >> 8, s = sm / M;
    const int nc = s == 0 ? C : Cr;
    // R for the screening rows and the certificate's rmax: a float sum, whose
    // error (< 2^-21 R) the certificate's 2^-17 R margin covers; the exact
    // distances form the canonical float64 R themselves
    float R = 0.0f;
#pragma unroll
    for (int gq = 0; gq < CG; ++gq) {
      const fh4 c4 = __builtin_bit_cast(fh4, cw[it][gq]);
#pragma unroll
      for (int u = 0; u < 4; ++u) R = __builtin_fmaf((float)c4[u], (float)c4[u], R);
    }
    uint8_t* row = tab + (size_t)sm * TB + r * RB;
#pragma unroll
    for (int gq = 0; gq < CG; ++gq) *reinterpret_cast<uint2*>(row + 8 * gq) = cw[it][gq];
    _Float16 rh, rl;
    if (r < nc) {
      const float half_r = 0.5f * R;
      rh = (_Float16)half_r;
      rl = (_Float16)(half_r - (float)rh);
    } else {  // past the codebook: never the minimum
      rh = (_Float16)__builtin_inff();
      rl = (_Float16)0.0f;
    }
    const fh4 aug = {rh, rl, (_Float16)1.0f, (_Float16)1.0f};
    *reinterpret_cast<fh4*>(row + 8 * CG) = aug;
    // largest R of the table (a wave's 64 rows share (s, m)): the wave's max
    // by DPP within rows of 16 lanes, then the four row maxima
    uint32_t rb = r < nc ? (__builtin_bit_cast(uint32_t, R) & 0x7FFFFFFFu) : 0u;
    rb = max(rb, (uint32_t)__builtin_amdgcn_mov_dpp((int)rb, 0xB1, 0xF, 0xF, true));   // quad_perm [1,0,3,2]
    rb = max(rb, (uint32_t)__builtin_amdgcn_mov_dpp((int)rb, 0x4E, 0xF, 0xF, true));   // quad_perm [2,3,0,1]
    rb = max(rb, (uint32_t)__builtin_amdgcn_mov_dpp((int)rb, 0x141, 0xF, 0xF, true));  // row_half_mirror
    rb = max(rb, (uint32_t)__builtin_amdgcn_mov_dpp((int)rb, 0x140, 0xF, 0xF, true));  // row_mirror
    const uint32_t w0 = (uint32_t)__builtin_amdgcn_readlane((int)rb, 0), w1 = (uint32_t)__builtin_amdgcn_readlane((int)rb, 16);
    const uint32_t w2 = (uint32_t)__builtin_amdgcn_readlane((int)rb, 32), w3 = (uint32_t)__builtin_amdgcn_readlane((int)rb, 48);
    if (lane == 0) atomicMax(&rmax_s[sm], max(max(w0, w1), max(w2, w3)));
  }
  __syncthreads();

  const int vi = lane & 15, g = lane >> 4;
  const int64_t v = (int64_t)((int)blockIdx.x - job.block0) * kFeVecs + wave * 16 + vi;
  const bool live = v < job.n;
  const uint16_t* xv = job.x + (live ? v : 0) * job.ldx;

  uint64_t codes[S][M / 8];  // the vector's code bytes, packed (byte m % 8 of word m / 8)
#pragma unroll
  for (int s = 0; s < S; ++s)
#pragma unroll
    for (int w = 0; w < M / 8; ++w) codes[s][w] = 0u;
  // add code c of subspace m (m uniform: a shift, never a register index by m)
  auto put_code = [&](int s, int m, int c) {
    const uint64_t bits = (uint64_t)c << (8 * (m & 7));
    if (M == 8 || m < 8) codes[s][0] |= bits;
    else codes[s][M / 8 - 1] |= bits;
  };
  uint64_t top[KS > 0 ? KS : 1];
#pragma unroll
  for (int j = 0; j < (KS > 0 ? KS : 1); ++j) top[j] = 0;

  // fl32(a - b) of two fp16 halves (v_fma_mix: a * 1 - b rounded once)
  auto sub_h = [](_Float16 a, _Float16 b) { return __builtin_fmaf((float)a, 1.0f, -(float)b); };
  typedef _Float16 h2 __attribute__((ext_vector_type(2)));
  auto pair = [](uint32_t w) { return __builtin_bit_cast(h2, w); };
  auto pack = [](float lo, float hi) { return __builtin_bit_cast(uint32_t, h2{(_Float16)lo, (_Float16)hi}); };

  // one nearest-centroid search of stage s, subspace m for the lane's vector
  // slice xw (DS fp16 values, packed in pairs); returns the code
  auto search = [&](int s, int m, const uint32_t (&xw)[DS / 2]) -> int {
    const int nc = s == 0 ? C : Cr;
    const uint8_t* tb = tab + (size_t)(s * M + m) * TB;
    // screening L: a float sum (its error sits far inside the certificate's
    // 2^-17 L); the canonical float64 chain is formed only for exact distances
    float Ls = 0.0f;
#pragma unroll
    for (int k = 0; k < DS / 2; ++k) {
      const h2 x2 = pair(xw[k]);
      Ls = __builtin_fmaf((float)x2[0], (float)x2[0], Ls);
      Ls = __builtin_fmaf((float)x2[1], (float)x2[1], Ls);
    }
    const float half_l = 0.5f * Ls;
    const _Float16 lh = (_Float16)half_l;
    const _Float16 ll = (_Float16)(half_l - (float)lh);
    uint2 bw = make_uint2(0u, 0u);  // B: -x of k-group g, or (1, 1, L/2 hi, L/2 lo)
    if (g < CG) {
      uint32_t b0 = xw[0], b1 = xw[1];
      if constexpr (CG == 2) {
        b0 = g ? xw[2] : b0;
        b1 = g ? xw[3] : b1;
      }
      bw = make_uint2(b0 ^ 0x80008000u, b1 ^ 0x80008000u);  // exact: fp16 negation
    } else if (g == CG) {
      bw = make_uint2(0x3C003C00u, __builtin_bit_cast(uint32_t, h2{lh, ll}));
    }
    const fh4 b = __builtin_bit_cast(fh4, bw);
    int maskv;  // 0xFFFFFF00 in a VGPR (the key build's other operand is the SGPR index)
    asm("v_mov_b32 %0, 0xffffff00" : "=v"(maskv));
    // k-groups past the R/2 group have B = 0: those lanes read the (finite)
    // coordinate group instead, so that every lane loads and nothing branches
    const uint8_t* arow = tb + vi * RB + 8 * (g <= CG ? g : 0);
    // the lane's keys of chunk t, computed again by the exact rescreen below
    auto screen = [&](auto&& insert) {
      fh4 a[16];
#pragma unroll
      for (int t = 0; t < 16; ++t) a[t] = *reinterpret_cast<const fh4*>(arow + 16 * t * RB);
      ff4 acc = __builtin_amdgcn_mfma_f32_16x16x16f16(a[0], b, ff4{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
#pragma unroll
      for (int t = 0; t < 16; ++t) {  // MFMA t + 1 issued before the keys of t
        ff4 next = acc;
        if (t + 1 < 16) next = __builtin_amdgcn_mfma_f32_16x16x16f16(a[t + 1], b, ff4{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
        int key[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {  // centroid 16t + 4g + i, keyed 4t + i
          // 4t + i < 64 is an inline constant and the mask sits in a VGPR:
          // one v_and_or_b32 per key (the index orders the lane's centroids
          // as 16t + 4g + i does; widen restores the centroid)
          const float z = acc[i];
          key[i] = (__builtin_bit_cast(int, z) & maskv) | (4 * t + i);
        }
        insert(key);
        acc = next;
      }
    };
    const int x32 = 4 * (lane ^ 32);
    // a lane key's index 4t + i -> centroid 16t + 4g + i (kNoKey stays)
    auto widen = [&](int k) { return k == kNoKey ? k : (k & ~0x3F) | ((k & 0x3C) << 2) | (4 * g) | (k & 3); };
    // screening: the two smallest keys (two lists for independent chains)
    int m1 = kNoKey, m2 = kNoKey, n1 = kNoKey, n2 = kNoKey;
    screen([&](const int (&key)[4]) {
      key_insert2x2(m1, m2, key[0], key[1]);
      key_insert2x2(n1, n2, key[2], key[3]);
    });
    key_insert2x2(m1, m2, n1, n2);
    m1 = widen(m1);
    m2 = widen(m2);
    {  // the vector's four lanes l, l ^ 16, l ^ 32, l ^ 48
      int o1 = lane_xor16(m1), o2 = lane_xor16(m2);
      key_insert2x2(m1, m2, o1, o2);
      o1 = lane_xor32(m1, x32);
      o2 = lane_xor32(m2, x32);
      key_insert2x2(m1, m2, o1, o2);
    }
    const float rmax = __builtin_bit_cast(float, rmax_s[s * M + m]);
    const float v1 = key_value(m1), v2 = key_value(m2);
    const float E = 0x1p-17f * (Ls + rmax) + 0x1p-22f;
    const bool safe = rmax < 120000.0f;  // R / 2 representable in fp16 for every centroid
    const bool unique = safe && v2 - v1 > 2.0f * E + 0x1p-14f * (fabsf(v1) + fabsf(v2));
    if (__builtin_amdgcn_ballot_w64(!unique) == 0) return m1 & 0xFF;  // uniform: every vector settled
    // some vector of the wave is uncertain: its three smallest keys, then
    // the canonical float64 distances (x and L as float64 chains)
    int p3 = kNoKey, p1 = kNoKey, p2 = kNoKey;
    screen([&](const int (&key)[4]) {
#pragma unroll
      for (int i = 0; i < 4; ++i) key_insert3(p1, p2, p3, key[i]);
    });
    p1 = widen(p1);
    p2 = widen(p2);
    p3 = widen(p3);
    {
      int o1 = lane_xor16(p1), o2 = lane_xor16(p2), o3 = lane_xor16(p3);
      key_insert3(p1, p2, p3, o1);
      key_insert3(p1, p2, p3, o2);
      key_insert3(p1, p2, p3, o3);
      o1 = lane_xor32(p1, x32);
      o2 = lane_xor32(p2, x32);
      o3 = lane_xor32(p3, x32);
      key_insert3(p1, p2, p3, o1);
      key_insert3(p1, p2, p3, o2);
      key_insert3(p1, p2, p3, o3);
    }
    if (unique) return m1 & 0xFF;
    double xs[DS];
    double lacc = 0.0;
#pragma unroll
    for (int k = 0; k < DS / 2; ++k) {
      const h2 x2 = pair(xw[k]);
      xs[2 * k] = (double)(float)x2[0];
      xs[2 * k + 1] = (double)(float)x2[1];
      lacc = __builtin_fma(xs[2 * k], xs[2 * k], lacc);
      lacc = __builtin_fma(xs[2 * k + 1], xs[2 * k + 1], lacc);
    }
    const float L = (float)lacc;
    const float w1 = key_value(p1), w3 = key_value(p3);
    const bool pair3 = safe && w3 - w1 > 2.0f * E + 0x1p-14f * (fabsf(w1) + fabsf(w3));
    // canonical distance of centroid j: fl32(fl32(L - 2X) + R), X and R float64 chains
    auto exact = [&](int j) {
      const uint8_t* row = tb + j * RB;
      double xa = 0.0, ra = 0.0;
#pragma unroll
      for (int u = 0; u < DS; ++u) {
        const double c = (double)h2f(reinterpret_cast<const uint16_t*>(row)[u]);
        xa = __builtin_fma(xs[u], c, xa);
        ra = __builtin_fma(c, c, ra);
      }
      return __fadd_rn(__fsub_rn(L, 2.0f * (float)xa), (float)ra);
    };
    int code;
    if (pair3) {
      const int ja = min(p1 & 0xFF, p2 & 0xFF), jb = max(p1 & 0xFF, p2 & 0xFF);
      const float da = exact(ja), db = exact(jb);
      code = db < da ? jb : ja;  // first min: ties keep the lower index
    } else {
      float best = __builtin_inff();
      code = 0;
      for (int j = 0; j < nc; ++j) {
        const float dj = exact(j);
        if (dj < best) {
          best = dj;
          code = j;
        }
      }
    }
    return code;
  };

  // the vector's subspace slices, fp16 pairs, loaded one subspace ahead
  auto load_x = [&](int m, uint32_t (&w)[DS / 2]) {
    if constexpr (DS == 8) {
      const uint4 v4 = *reinterpret_cast<const uint4*>(xv + m * DS);
      w[0] = v4.x;
      w[1] = v4.y;
      w[2] = v4.z;
      w[3] = v4.w;
    } else {
      const uint2 v2 = *reinterpret_cast<const uint2*>(xv + m * DS);
      w[0] = v2.x;
      w[1] = v2.y;
    }
  };
  uint32_t xnext[DS / 2];
  load_x(0, xnext);
#pragma unroll 1
  for (int m = 0; m < M; ++m) {
    uint32_t xw[DS / 2];
#pragma unroll
    for (int k = 0; k < DS / 2; ++k) xw[k] = xnext[k];
    if (m + 1 < M) load_x(m + 1, xnext);  // uniform
    const int c0 = search(0, m, xw);
    put_code(0, m, c0);
    const uint32_t* base = reinterpret_cast<const uint32_t*>(tab + (size_t)m * TB + c0 * RB);
    uint32_t rec[DS / 2];  // fp16(base + rvq) pairs
#pragma unroll
    for (int k = 0; k < DS / 2; ++k) rec[k] = base[k];
    if constexpr (RVQ) {
      uint32_t r1[DS / 2];  // PQ residual fp16(fl32(x) - fl32(c))
#pragma unroll
      for (int k = 0; k < DS / 2; ++k) {
        const h2 x2 = pair(xw[k]), c2 = pair(rec[k]);
        r1[k] = pack(sub_h(x2[0], c2[0]), sub_h(x2[1], c2[1]));
      }
      const int c1 = search(1, m, r1);
      put_code(1, m, c1);
      const uint32_t* cr = reinterpret_cast<const uint32_t*>(tab + (size_t)(M + m) * TB + c1 * RB);
#pragma unroll
      for (int k = 0; k < DS / 2; ++k) {  // fp16(fl32(base) + fl32(rvq))
        const h2 a2 = pair(rec[k]), c2 = pair(cr[k]);
        rec[k] = pack(__builtin_fmaf((float)a2[0], 1.0f, (float)c2[0]), __builtin_fmaf((float)a2[1], 1.0f, (float)c2[1]));
      }
    }
    if constexpr (KS > 0) {
      // this lane's share of the subspace: coordinates g * DS/4 + e, e < DS/4
      // (pair word g for DS = 8, a half of word g >> 1 for DS = 4), selected
      // without indexing registers by lane
      uint32_t xs2 = xw[0], rs2 = rec[0];
#pragma unroll
      for (int k = 1; k < DS / 2; ++k) {
        const bool sel = DS == 8 ? g == k : (g >> 1) == k;
        xs2 = sel ? xw[k] : xs2;
        rs2 = sel ? rec[k] : rs2;
      }
#pragma unroll
      for (int e = 0; e < DS / 4; ++e) {
        const int hsel = DS == 8 ? e : (g & 1);
        const h2 x2 = pair(xs2), q2 = pair(rs2);
        const float r2 = hsel ? sub_h(x2[1], q2[1]) : sub_h(x2[0], q2[0]);
        const uint32_t mb = __builtin_bit_cast(uint32_t, r2) & 0x7FFFFFFFu;
        if (mb <= 0x7F800000u) {  // NaN never enters
          const int i = m * DS + g * (DS / 4) + e;
          topk_insert(top, ((uint64_t)mb << 32) | ((uint64_t)(64 - i) << 16) | f2h(r2));
        }
      }
    }
  }
  if constexpr (KS > 0) {
#pragma unroll
    for (int o = 16; o <= 32; o <<= 1) {
      uint64_t ot[KS];
#pragma unroll
      for (int j = 0; j < KS; ++j) ot[j] = __shfl_xor(top[j], o, 64);
#pragma unroll
      for (int j = 0; j < KS; ++j) topk_insert(top, ot[j]);
    }
  }
  if (!live || g != 0) return;
#pragma unroll
  for (int s = 0; s < S; ++s) {
    uint8_t* dst = (s == 0 ? job.pq : job.rvq) + v * M;
    const uint64_t lo = codes[s][0];
    if constexpr (M == 8) {
      *reinterpret_cast<uint2*>(dst) = make_uint2((uint32_t)lo, (uint32_t)(lo >> 32));
    } else {
      const uint64_t hi = codes[s][M / 8 - 1];
      *reinterpret_cast<uint4*>(dst) =
          make_uint4((uint32_t)lo, (uint32_t)(lo >> 32), (uint32_t)hi, (uint32_t)(hi >> 32));
    }
  }
  if constexpr (KS > 0) {
    uint32_t iw = 0;
    uint16_t vals[KS];
#pragma unroll
    for (int j = 0; j < KS; ++j) {
      const bool real = top[j] != 0;
      iw |= (uint32_t)(real ? (uint8_t)(64 - (int)((top[j] >> 16) & 0xFFFF)) : 0u) << (8 * j);
      vals[j] = real ? (uint16_t)(top[j] & 0xFFFF) : (uint16_t)0;
    }
    *reinterpret_cast<uint32_t*>(job.sidx + v * KS) = iw;
    *reinterpret_cast<uint2*>(job.sval + v * KS) =
        make_uint2(vals[0] | ((uint32_t)vals[1] << 16), vals[2] | ((uint32_t)vals[3] << 16));
  }
}

// ---------------------------------------------------------------- reference-mode RVQ on MFMA
// ResidualVQMLX.encode (quantization.py:206-252) over the gated rows, for
// head_dim D in {64, 128, 256} and 3 <= C <= 16384 centroids per stage.  One
// launch runs every stage; a row's running residual stays in a float32
// workspace [A][D] between stages (stage 0 reads the fp16 PQ residual).
//
// Screening: a block (4 waves) holds 4 * kRvqSets * 16 rows; each wave holds
// kRvqSets B operands of 16 rows as -fp16(x) (v_mfma_f32_16x16x32_f16: lane l
// has row l % 16, coordinates 32 ks + 8 (l / 16) + e).  The stage's codebook
// streams through LDS in chunks of 64 centroid rows (16-byte groups XOR-
// swizzled by the row, so the 16 rows of an A operand hit distinct banks),
// double-buffered, with R_j / 2 beside them.  Each A operand feeds kRvqSets
// MFMAs, whose accumulators start at R_j / 2: accumulator i of lane l holds
//   z = R_j / 2 - x . c_j   (j = 16 T + 4 (l / 16) + i of tile T, row l % 16),
// i.e. (dist_j - L) / 2 up to the screening error.  A key is z with its low
// F = ceil(log2 C) bits replaced by the lane's local centroid order; keys
// compare as floats (denormals are preserved), and each lane keeps its four
// smallest (v_med3_f32 / v_min_f32), merged over the row's four lanes.
//
// Certificate (every j): |z_j - (dist_j - L) / 2| <= E with
//   E = split + mfma + canon,
//   split = |x - fp16(x)| Cn                  (x rounded to fp16 for the B
//           operand; 0 at stage 0, where x is the fp16 residual itself),
//   mfma  = (D + 2) 2^-24 (|x| Cn + Rmax / 2) (fp32 accumulation of exact
//           fp16 products),
//   canon = 2^-21 (L + Rmax)                  (the canonical chain's roundings),
// Cn = sqrt(Rmax) bounding every |c_j|, plus the keys' truncation t.  With
// v1 <= .. <= v4 the four smallest keys: v2 - v1 > 2E + t proves the first
// key's centroid is the canonical first-min; v(k+1) - v1 > 2E + t (k = 2, 3)
// proves it is one of the first k, which are rescored with the float64 chain
// (ties to the lower index), the wave's rescoring sums spread over its lanes;
// anything else, non-finite values or |x| beyond fp16 take the canonical
// float64 scan over all C, spread over the wave.
constexpr int kRvqWaves = 4;
constexpr int kRvqThreads = kRvqWaves * 64;
constexpr int kRvqChunk = 64;          // centroid rows per LDS chunk
constexpr float kRvqPadHalfR = 1.0e38f;  // R / 2 of rows past the codebook: never a minimum

template <int D>
struct RvqShape {
  static constexpr int KS = D / 32;               // 16x16x32 k-steps
  static constexpr int G16 = D / 8;               // 16-byte groups of a row
  static constexpr int RB = D * 2;                // row bytes
  static constexpr int SETS = D <= 128 ? 4 : 2;   // B operands per wave
  static constexpr int VECS = kRvqWaves * SETS * 16;
};

typedef _Float16 rh8 __attribute__((ext_vector_type(8)));
typedef float rf4 __attribute__((ext_vector_type(4)));

// canonical R_j = fl32(S c_j * c_j) per (stage, centroid) into r[L][Cp]
// (rows past C: +inf): one thread per row, the row in 16-byte loads
template <int D>
__global__ void __launch_bounds__(256) rvq_norms_kernel(const uint16_t* __restrict__ cb, int C, int Cp,
                                                        float* __restrict__ r) {
  const int layer = blockIdx.y;
  const int j = blockIdx.x * 256 + threadIdx.x;
  if (j >= Cp) return;
  float R = __builtin_inff();
  if (j < C) {
    const uint4* row = reinterpret_cast<const uint4*>(cb + ((size_t)layer * C + j) * D);
    uint4 w[D / 8];
#pragma unroll
    for (int q = 0; q < D / 8; ++q) w[q] = row[q];
    double acc = 0.0;
#pragma unroll
    for (int q = 0; q < D / 8; ++q) {
      const uint32_t pw[4] = {w[q].x, w[q].y, w[q].z, w[q].w};
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const double c = (double)h2f((uint16_t)(pw[e >> 1] >> (16 * (e & 1))));
        acc = __builtin_fma(c, c, acc);
      }
    }
    R = (float)acc;
  }
  r[(size_t)layer * Cp + j] = R;
}

// the stage's largest R over its C rows (+inf when some R is not finite): one block per stage
__global__ void __launch_bounds__(256) rvq_rmax_kernel(const float* __restrict__ r, int C, int Cp,
                                                       float* __restrict__ rmax) {
  __shared__ float red[256];
  const int layer = blockIdx.x;
  float mx = 0.0f;
  for (int j = threadIdx.x; j < C; j += 256) {
    const float R = r[(size_t)layer * Cp + j];
    mx = R <= 3.0e38f ? fmaxf(mx, R) : __builtin_inff();  // NaN or inf: the stage is unsafe
  }
  red[threadIdx.x] = mx;
  __syncthreads();
  for (int o = 128; o > 0; o >>= 1) {
    if ((int)threadIdx.x < o) red[threadIdx.x] = fmaxf(red[threadIdx.x], red[threadIdx.x + o]);
    __syncthreads();
  }
  if (threadIdx.x == 0) rmax[layer] = red[0];
}

// insert float key k into the sorted m1 <= m2 <= m3 <= m4 (as floats): each new
// entry is the median of its old value, the one below it and k
__device__ __forceinline__ void fkey_insert4(float& m1, float& m2, float& m3, float& m4, float k) {
  asm("v_med3_f32 %3, %2, %3, %4\n\t"
      "v_med3_f32 %2, %1, %2, %4\n\t"
      "v_med3_f32 %1, %0, %1, %4\n\t"
      "v_min_f32_e32 %0, %0, %4"
      : "+v"(m1), "+v"(m2), "+v"(m3), "+v"(m4)
      : "v"(k));
}

template <int D>
__global__ void __launch_bounds__(kRvqThreads) __attribute__((amdgpu_waves_per_eu(2)))
rvq_mfma_kernel(const uint16_t* __restrict__ resid, int64_t ld, const int32_t* __restrict__ offsets,
                int64_t active, const uint16_t* __restrict__ cb, int L, int C, int Cp, int F,
                const float* __restrict__ rr, const float* __restrict__ rmax_all, float* __restrict__ run,
                uint16_t* __restrict__ codes) {
  using S = RvqShape<D>;
  constexpr int KS = S::KS, G16 = S::G16, RB = S::RB, SETS = S::SETS;
  __shared__ __align__(16) uint8_t tab[2][kRvqChunk * RB];
  __shared__ __align__(16) float rs[2][kRvqChunk];
  __shared__ float xsc[kRvqWaves][D];  // one row's coordinates for the wave's float64 scans
  __shared__ int pitem[kRvqWaves][SETS * 16][3];     // rows to rescore: their candidates
  __shared__ int pslot[kRvqWaves][SETS * 16];        // item -> row (16 s + vi)
  __shared__ double pres[kRvqWaves][SETS * 16][4];   // L, then X of each candidate
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int vi = lane & 15, g = lane >> 4;
  const int64_t v0 = (int64_t)blockIdx.x * S::VECS + wave * (SETS * 16);
  int64_t vid[SETS];
  bool live[SETS];
#pragma unroll
  for (int s = 0; s < SETS; ++s) {
    vid[s] = v0 + 16 * s + vi;
    live[s] = vid[s] < active;
  }
  const int fmask = (1 << F) - 1;
  const int keep = ~fmask;  // key bits kept from z (in a VGPR: the key build's other operand is an SGPR)
  int keepv;
  asm("v_mov_b32 %0, %1" : "=v"(keepv) : "s"(keep));

  // the row's coordinate u at the current stage: the fp16 PQ residual at stage 0, then the workspace
  auto x_at = [&](int64_t v, int layer, int u) -> float {
    return layer == 0 ? h2f(resid[(int64_t)offsets[v] * ld + u]) : run[v * D + u];
  };
  // coordinates 8 q .. 8 q + 7 of row v
  auto load_row8 = [&](int64_t v, int layer, int q, float (&x)[8]) {
    const int k0 = 8 * q;
    if (layer == 0) {
      const uint4 h = *reinterpret_cast<const uint4*>(resid + (int64_t)offsets[v] * ld + k0);
      const uint32_t w[4] = {h.x, h.y, h.z, h.w};
#pragma unroll
      for (int e = 0; e < 8; ++e) x[e] = h2f((uint16_t)(w[e >> 1] >> (16 * (e & 1))));
    } else {
      const float4 a = *reinterpret_cast<const float4*>(run + v * D + k0);
      const float4 b = *reinterpret_cast<const float4*>(run + v * D + k0 + 4);
      x[0] = a.x; x[1] = a.y; x[2] = a.z; x[3] = a.w;
      x[4] = b.x; x[5] = b.y; x[6] = b.z; x[7] = b.w;
    }
  };
  // the lane's 8 coordinates 32 ks + 8 g .. + 7 of row v
  auto load8 = [&](int64_t v, int layer, int ks, float (&x)[8]) {
    const int k0 = 32 * ks + 8 * g;
    if (layer == 0) {
      const uint4 h = *reinterpret_cast<const uint4*>(resid + (int64_t)offsets[v] * ld + k0);
      const uint32_t w[4] = {h.x, h.y, h.z, h.w};
#pragma unroll
      for (int e = 0; e < 8; ++e) x[e] = h2f((uint16_t)(w[e >> 1] >> (16 * (e & 1))));
    } else {
      const float4 a = *reinterpret_cast<const float4*>(run + v * D + k0);
      const float4 b = *reinterpret_cast<const float4*>(run + v * D + k0 + 4);
      x[0] = a.x; x[1] = a.y; x[2] = a.z; x[3] = a.w;
      x[4] = b.x; x[5] = b.y; x[6] = b.z; x[7] = b.w;
    }
  };

  rh8 b[SETS][KS];
  float lsq[SETS], esq[SETS];  // |x|^2 and |x - fp16(x)|^2 (the lane's share, then the row's)
  bool fin[SETS];
  // the B operand -fp16(x) of 8 coordinates, with their shares of |x|^2 and of the rounding error
  auto to_b = [](const float (&x)[8], rh8& bo, float& l2, float& e2, bool& ok) {
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const _Float16 h = (_Float16)x[e];
      bo[e] = -h;
      const float d = x[e] - (float)h;  // exact in float32
      l2 = __builtin_fmaf(x[e], x[e], l2);
      e2 = __builtin_fmaf(d, d, e2);
      ok = ok && fabsf(x[e]) <= 65504.0f;
    }
  };
  // B operands and the screening L of each row at stage 0
#pragma unroll
  for (int s = 0; s < SETS; ++s) {
    float l2 = 0.0f, e2 = 0.0f;
    bool ok = true;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      float x[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
      if (live[s]) load8(vid[s], 0, ks, x);
      to_b(x, b[s][ks], l2, e2, ok);
    }
    lsq[s] = l2;
    esq[s] = e2;
    fin[s] = ok;
  }
  auto quad_sum = [&](float v) {  // sum over the row's four lanes l, l ^ 16, l ^ 32, l ^ 48
    v += __builtin_bit_cast(float, lane_xor16(__builtin_bit_cast(int, v)));
    return v + __builtin_bit_cast(float, lane_xor32(__builtin_bit_cast(int, v), 4 * (lane ^ 32)));
  };
  auto quad_all = [&](bool p) {
    int v = p ? 1 : 0;
    v &= lane_xor16(v);
    return (v & lane_xor32(v, 4 * (lane ^ 32))) != 0;
  };

  const int nchunks = Cp / kRvqChunk;
  constexpr int kLoads = kRvqChunk * G16 / kRvqThreads;  // 16-byte staging loads per thread and chunk
  static_assert(kRvqChunk * G16 % kRvqThreads == 0, "staging loads per thread");

  for (int layer = 0; layer < L; ++layer) {
    const uint16_t* cbl = cb + (size_t)layer * C * D;
    const float* rl = rr + (size_t)layer * Cp;
    const float rmax = rmax_all[layer];
#pragma unroll
    for (int s = 0; s < SETS; ++s) {
      lsq[s] = quad_sum(lsq[s]);
      esq[s] = quad_sum(esq[s]);
      fin[s] = quad_all(fin[s]);
    }
    // ---- staging of chunk c into buffer c & 1: loads, then stores
    uint4 stg[kLoads];
    float rstg = 0.0f;
    auto stage_load = [&](int c) {
#pragma unroll
      for (int it = 0; it < kLoads; ++it) {
        const int q = tid + kRvqThreads * it;
        const int row = q / G16, grp = q % G16;
        const int j = c * kRvqChunk + row;
        stg[it] = j < C ? *reinterpret_cast<const uint4*>(cbl + (size_t)j * D + 8 * grp) : make_uint4(0u, 0u, 0u, 0u);
      }
      if (tid < kRvqChunk) {
        const int j = c * kRvqChunk + tid;
        rstg = j < C ? 0.5f * rl[j] : kRvqPadHalfR;
      }
    };
    auto stage_store = [&](int c) {
      uint8_t* tb = tab[c & 1];
#pragma unroll
      for (int it = 0; it < kLoads; ++it) {
        const int q = tid + kRvqThreads * it;
        const int row = q / G16, grp = q % G16;
        *reinterpret_cast<uint4*>(tb + row * RB + 16 * (grp ^ (row & (G16 - 1)))) = stg[it];
      }
      if (tid < kRvqChunk) rs[c & 1][tid] = rstg;
    };
    __syncthreads();  // the previous stage's last chunk is no longer read
    stage_load(0);
    stage_store(0);
    __syncthreads();

    float m1[SETS], m2[SETS], m3[SETS], m4[SETS];
    const float nokey = __builtin_inff();
#pragma unroll
    for (int s = 0; s < SETS; ++s) m1[s] = m2[s] = m3[s] = m4[s] = nokey;
#pragma unroll 1
    for (int c = 0; c < nchunks; ++c) {
      if (c + 1 < nchunks) stage_load(c + 1);
      const uint8_t* tb = tab[c & 1];
#pragma unroll
      for (int tile = 0; tile < kRvqChunk / 16; ++tile) {
        const int row = tile * 16 + vi;
        const uint8_t* trow = tb + row * RB;
        rh8 a[KS];
#pragma unroll
        for (int ks = 0; ks < KS; ++ks)
          a[ks] = *reinterpret_cast<const rh8*>(trow + 16 * ((4 * ks + g) ^ (row & (G16 - 1))));
        const rf4 rinit = *reinterpret_cast<const rf4*>(&rs[c & 1][tile * 16 + 4 * g]);
        const int base = 4 * (c * (kRvqChunk / 16) + tile);  // local order 4 T + i
#pragma unroll
        for (int s = 0; s < SETS; ++s) {
          rf4 acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[0], b[s][0], rinit, 0, 0, 0);
#pragma unroll
          for (int ks = 1; ks < KS; ++ks) acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[ks], b[s][ks], acc, 0, 0, 0);
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const float z = acc[i];  // through a scalar: a bit_cast of the vector element reads element 0
            // one v_and_or_b32 with the order in an SGPR (readfirstlane keeps the
            // compiler from splitting it into an and plus an or3 of base | i);
            // built in C++ so that the compiler sees, and pads, the read of the
            // MFMA result
            const int idx = __builtin_amdgcn_readfirstlane(base + i);
            const float key = __builtin_bit_cast(float, (__builtin_bit_cast(int, z) & keepv) | idx);
            fkey_insert4(m1[s], m2[s], m3[s], m4[s], key);
          }
        }
      }
      if (c + 1 < nchunks) stage_store(c + 1);
      __syncthreads();
    }

    // ---- merge the row's four lanes: local order 4 T + i -> centroid 16 T + 4 g + i
    const int gq = 4 * g;
    auto widen = [&](float k) {
      const int b = __builtin_bit_cast(int, k);
      const int li = b & fmask;
      return __builtin_bit_cast(float, (b & ~fmask) | ((li & ~3) << 2) | gq | (li & 3));
    };
    const float Cn = sqrtf(rmax) * 1.0001f;
    int code[SETS];
    int how[SETS];  // 0 unique, 1 rescore the first two, 2 full scan
    int pa[SETS], pb[SETS], pc[SETS];  // the rescored candidates, ascending (pc = pb for two)
#pragma unroll
    for (int s = 0; s < SETS; ++s) {
      float p[4] = {widen(m1[s]), widen(m2[s]), widen(m3[s]), widen(m4[s])};
      auto merge_from = [&](auto&& other) {
        float o[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) o[k] = __builtin_bit_cast(float, other(__builtin_bit_cast(int, p[k])));
#pragma unroll
        for (int k = 0; k < 4; ++k) fkey_insert4(p[0], p[1], p[2], p[3], o[k]);
      };
      merge_from([](int v) { return lane_xor16(v); });
      const int x32 = 4 * (lane ^ 32);
      merge_from([&](int v) { return lane_xor32(v, x32); });
      const float xn = sqrtf(lsq[s]) * 1.0001f;
      const float split = sqrtf(esq[s]) * 1.0001f * Cn;  // |(x - fp16(x)) . c_j| <= |x - fp16(x)| Cn
      const float mf = (float)(D + 2) * 0x1p-24f * (xn * Cn + 0.5f * rmax);
      const float canon = 0x1p-21f * (lsq[s] + rmax);
      const float E = 1.25f * (split + mf + canon) + 0x1p-100f;
      const float tq = __builtin_bit_cast(float, (127 + F - 22) << 23);  // 2^(F - 22)
      const bool safe = fin[s] && lsq[s] <= 1.0e30f && rmax <= 1.0e30f && C >= 3;
      // candidates: the keys within 2E + t of the first; 1 -> settled, 2 or 3 ->
      // rescored with the canonical chain, 4 (or unsafe values) -> the full scan
      auto apart = [&](float a, float b) { return b - a > 2.0f * E + tq * (fabsf(a) + fabsf(b)); };
      const int ncand = apart(p[0], p[1]) ? 1 : apart(p[0], p[2]) ? 2 : apart(p[0], p[3]) ? 3 : 4;
      how[s] = !safe || ncand == 4 ? 2 : (ncand == 1 ? 0 : 1);
      code[s] = __builtin_bit_cast(int, p[0]) & fmask;
      // the rescored candidates in ascending index order (the third repeats the second for a pair)
      int j0 = code[s], j1 = __builtin_bit_cast(int, p[1]) & fmask, j2 = __builtin_bit_cast(int, p[2]) & fmask;
      if (ncand < 3) j2 = j1;
      const int lo = min(j0, min(j1, j2)), hi = max(j0, max(j1, j2));
      pa[s] = lo;
      pb[s] = j0 + j1 + j2 - lo - hi;
      pc[s] = hi;
      if (!live[s]) how[s] = 0;
    }
    // ---- rows whose first two candidates need the canonical chain: three
    // float64 sums in coordinate order each (L, X_a, X_b), spread over the
    // wave's lanes as independent units, then each row picks its code
    {
      int nitems = 0;
      int myitem[SETS];
#pragma unroll
      for (int s = 0; s < SETS; ++s) {
        const uint64_t want = __builtin_amdgcn_ballot_w64(g == 0 && how[s] == 1);
        // every lane of row vi takes the row's rank among the set's wanting rows
        const int rank = __builtin_popcountll(want & ((1ull << vi) - 1));
        myitem[s] = ((want >> vi) & 1) ? nitems + rank : -1;
        if (g == 0 && myitem[s] >= 0) {
          pitem[wave][myitem[s]][0] = pa[s];
          pitem[wave][myitem[s]][1] = pb[s];
          pitem[wave][myitem[s]][2] = pc[s];
          pslot[wave][myitem[s]] = 16 * s + vi;
        }
        nitems += __builtin_popcountll(want);
      }
      if (nitems) {  // uniform
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        for (int u = lane; u < 4 * nitems; u += 64) {
          const int it = u >> 2, comp = u & 3;
          const int slot = pslot[wave][it];
          const int64_t v = v0 + slot;
          const uint4* crow = reinterpret_cast<const uint4*>(cbl + (size_t)pitem[wave][it][comp == 0 ? 0 : comp - 1] * D);
          double acc = 0.0;
#pragma unroll 4
          for (int q = 0; q < D / 8; ++q) {
            float x8[8];
            load_row8(v, layer, q, x8);
            const uint4 w = crow[q];  // unused for L
            const uint32_t pw[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
            for (int e = 0; e < 8; ++e) {
              const double xu = (double)x8[e];
              const double y = comp == 0 ? xu : (double)h2f((uint16_t)(pw[e >> 1] >> (16 * (e & 1))));
              acc = __builtin_fma(xu, y, acc);
            }
          }
          pres[wave][it][comp] = acc;
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
        for (int s = 0; s < SETS; ++s) {
          if (myitem[s] >= 0) {
            const int it = myitem[s];
            const float Lc = (float)pres[wave][it][0];
            const float da = __fadd_rn(__fsub_rn(Lc, 2.0f * (float)pres[wave][it][1]), rl[pa[s]]);
            const float db = __fadd_rn(__fsub_rn(Lc, 2.0f * (float)pres[wave][it][2]), rl[pb[s]]);
            const float dc = __fadd_rn(__fsub_rn(Lc, 2.0f * (float)pres[wave][it][3]), rl[pc[s]]);
            // first min in ascending index order: ties keep the lower index
            int best = pa[s];
            float bd = da;
            if (db < bd) { bd = db; best = pb[s]; }
            if (dc < bd) best = pc[s];
            code[s] = best;
          }
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();  // the item tables are rewritten at the next stage
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
      }
    }
    // ---- rows left uncertain: the canonical scan over all C, one row at a time
    // across the wave (lane j scans centroids j, j + 64, ...)
#pragma unroll
    for (int s = 0; s < SETS; ++s) {
      uint64_t todo = __builtin_amdgcn_ballot_w64(g == 0 && live[s] && how[s] == 2);
      while (todo) {  // uniform
        const int r0 = __builtin_ctzll(todo);
        todo &= todo - 1;
        const int64_t v = v0 + 16 * s + r0;
        for (int u = lane; u < D; u += 64) xsc[wave][u] = x_at(v, layer, u);
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        double lacc = 0.0;
        for (int u = 0; u < D; ++u) {
          const double xu = (double)xsc[wave][u];
          lacc = __builtin_fma(xu, xu, lacc);
        }
        const float Lc = (float)lacc;
        float best = __builtin_inff();
        int bi = 0x7fffffff;
        for (int j = lane; j < C; j += 64) {
          const uint4* cj = reinterpret_cast<const uint4*>(cbl + (size_t)j * D);
          double xacc = 0.0;
#pragma unroll 4
          for (int q = 0; q < D / 8; ++q) {  // the row's loads issued together
            const uint4 w = cj[q];
            const uint32_t pw[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
            for (int e = 0; e < 8; ++e)
              xacc = __builtin_fma((double)xsc[wave][8 * q + e], (double)h2f((uint16_t)(pw[e >> 1] >> (16 * (e & 1)))),
                                   xacc);
          }
          const float dist = __fadd_rn(__fsub_rn(Lc, 2.0f * (float)xacc), rl[j]);
          if (dist < best) {  // ascending j per lane: first min kept
            best = dist;
            bi = j;
          }
        }
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) {
          const float ob = __shfl_xor(best, o, 64);
          const int oi = __shfl_xor(bi, o, 64);
          if (ob < best || (ob == best && oi < bi)) {
            best = ob;
            bi = oi;
          }
        }
        if (bi == 0x7fffffff) bi = 0;  // no finite distance: index 0, as the reference's merge leaves it
        if (vi == r0) code[s] = bi;
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();  // xsc is rewritten by the next row
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
      }
    }
    // ---- codes, then the next stage's running residual fl32(run - c) and B operands
#pragma unroll
    for (int s = 0; s < SETS; ++s) {
      if (live[s] && g == 0) codes[vid[s] * L + layer] = (uint16_t)code[s];
      if (layer + 1 == L) continue;
      const uint16_t* crow = cbl + (size_t)code[s] * D;
      float l2 = 0.0f, e2 = 0.0f;
      bool ok = true;
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        const int k0 = 32 * ks + 8 * g;
        float x[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
        if (live[s]) {
          load8(vid[s], layer, ks, x);
          const uint4 cw = *reinterpret_cast<const uint4*>(crow + k0);
          const uint32_t w[4] = {cw.x, cw.y, cw.z, cw.w};
#pragma unroll
          for (int e = 0; e < 8; ++e) x[e] = __fsub_rn(x[e], h2f((uint16_t)(w[e >> 1] >> (16 * (e & 1)))));
          *reinterpret_cast<float4*>(run + vid[s] * D + k0) = make_float4(x[0], x[1], x[2], x[3]);
          *reinterpret_cast<float4*>(run + vid[s] * D + k0 + 4) = make_float4(x[4], x[5], x[6], x[7]);
        }
        to_b(x, b[s][ks], l2, e2, ok);
      }
      lsq[s] = l2;
      esq[s] = e2;
      fin[s] = ok;
    }
  }
}

size_t rvq_mfma_ws_bytes(int64_t active, int D, int L, int C) {
  const int64_t Cp = (C + kRvqChunk - 1) / kRvqChunk * kRvqChunk;
  const auto up = [](int64_t n) { return (size_t)((n + 255) / 256 * 256); };
  return up(4 * L * Cp) + up(4 * L) + up(4 * (active > 0 ? active : 1) * D);
}

bool rvq_mfma_ok(int D, int C) { return (D == 64 || D == 128 || D == 256) && C >= 3 && C <= 16384; }

template <int D>
int launch_rvq_mfma(const void* resid, int64_t ld, const int32_t* offsets, int64_t active, const void* cb, int L,
                    int C, uint16_t* codes, void* ws, hipStream_t s) {
  const int Cp = (C + kRvqChunk - 1) / kRvqChunk * kRvqChunk;
  int F = 0;
  while ((1 << F) < Cp) ++F;
  const auto up = [](int64_t n) { return (size_t)((n + 255) / 256 * 256); };
  float* r = (float*)ws;
  float* rmax = (float*)((uint8_t*)ws + up(4 * L * (int64_t)Cp));
  float* run = (float*)((uint8_t*)rmax + up(4 * L));
  hipLaunchKernelGGL(rvq_norms_kernel<D>, dim3((unsigned)ceil_div(Cp, 256), (unsigned)L), dim3(256), 0, s,
                     (const uint16_t*)cb, C, Cp, r);
  hipLaunchKernelGGL(rvq_rmax_kernel, dim3(L), dim3(256), 0, s, (const float*)r, C, Cp, rmax);
  const int64_t blocks = ceil_div(active, (int64_t)RvqShape<D>::VECS);
  hipLaunchKernelGGL(rvq_mfma_kernel<D>, dim3((unsigned)blocks), dim3(kRvqThreads), 0, s, (const uint16_t*)resid, ld,
                     offsets, active, (const uint16_t*)cb, L, C, Cp, F, (const float*)r, (const float*)rmax, run, codes);
  return check_launch("rvq_encode_full");
}

// The fused encode serves head_dim 64, 4- or 8-dim subspaces, an RVQ stage of
// the same split or none, k in {0, 4}, and aligned rows (16-byte x rows,
// code and sparse rows at their natural alignment).
bool fused_encode_ok(const rfsn_format* f, const EncodeJob& j) {
  const int d = f->head_dim / f->pq_subspaces;
  const auto al = [](const void* p, uintptr_t a) { return p == nullptr || reinterpret_cast<uintptr_t>(p) % a == 0; };
  return f->head_dim == 64 && (d == 4 || d == 8) && (f->rvq_subspaces == 0 || f->rvq_subspaces == f->pq_subspaces) &&
         (f->sparse_k == 0 || f->sparse_k == 4) && j.ldx % 8 == 0 && al(j.x, 16) && al(j.pq_cb, 8) &&
         al(j.rvq_cb, 8) && al(j.pq, f->pq_subspaces) && al(j.rvq, f->pq_subspaces) && al(j.sidx, 4) &&
         al(j.sval, 8);
}

int launch_warm_encode_fused(const rfsn_format* f, EncodeJobs& jobs, hipStream_t s) {
  int blocks = 0;
  for (int i = 0; i < jobs.count; ++i) {
    jobs.j[i].block0 = blocks;
    blocks += (int)ceil_div(jobs.j[i].n, kFeVecs);
  }
  if (blocks == 0) return RFSN_OK;
  jobs.C = f->pq_centroids;
  jobs.Cr = f->rvq_subspaces ? f->rvq_centroids : 1;
  const int d = f->head_dim / f->pq_subspaces;
  const bool rvq = f->rvq_subspaces > 0;
  const bool ks = f->sparse_k > 0;
#define RFSN_FE(DS, R, K) hipLaunchKernelGGL((warm_encode_fused_kernel<DS, R, K>), dim3(blocks), dim3(kFeThreads), 0, s, jobs)
  if (d == 8) {
    if (rvq) { if (ks) RFSN_FE(8, true, 4); else RFSN_FE(8, true, 0); }
    else { if (ks) RFSN_FE(8, false, 4); else RFSN_FE(8, false, 0); }
  } else {
    if (rvq) { if (ks) RFSN_FE(4, true, 4); else RFSN_FE(4, true, 0); }
    else { if (ks) RFSN_FE(4, false, 4); else RFSN_FE(4, false, 0); }
  }
#undef RFSN_FE
  return check_launch("warm_encode_fused");
}

template <int DSUB>
int launch_pq(const void* x, int64_t n, int64_t ldx, int64_t xg, const void* cb, int M, int C, int d, int64_t cbg,
              uint8_t* codes, int64_t ldc, int64_t cg, void* resid, int64_t ldr, int64_t rg, int groups,
              hipStream_t s) {
  dim3 grid((unsigned)ceil_div(n, kEncodeThreads), (unsigned)M, (unsigned)groups);
  const size_t lds = (size_t)C * d * sizeof(double) + (size_t)C * sizeof(float);
  if (lds > 64 * 1024) {
    hipFuncSetAttribute((const void*)pq_encode_kernel<DSUB>, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
  }
  hipLaunchKernelGGL(pq_encode_kernel<DSUB>, grid, dim3(kEncodeThreads), lds, s,
                     (const uint16_t*)x, n, ldx, xg, (const uint16_t*)cb, M, C, d, cbg, codes, ldc, cg,
                     (uint16_t*)resid, ldr, rg);
  return check_launch("pq_encode");
}

}  // namespace

int pq_encode_impl(const void* x, int64_t n, int D, int64_t ldx, int64_t xg, const void* cb, int M, int C,
                   int64_t cbg, uint8_t* codes, int64_t ldc, int64_t cg, void* resid, int64_t ldr, int64_t rg,
                   int groups, hipStream_t s) {
  RFSN_REQUIRE(x && cb && codes, "pq_encode: null pointer");
  RFSN_REQUIRE(M > 0 && D > 0 && D % M == 0, "pq_encode: head_dim must equal num_subspaces * subspace_dim");
  RFSN_REQUIRE(C > 0 && C <= 256, "pq_encode: codebook size must be in [1, 256] (uint8 codes)");
  RFSN_REQUIRE(n >= 0 && groups >= 1, "pq_encode: bad n / groups");
  RFSN_REQUIRE(ldx >= D && ldc >= M && (resid == nullptr || ldr >= D), "pq_encode: bad leading dimension");
  const int d = D / M;
  RFSN_REQUIRE(d <= 32, "pq_encode: subspace_dim > 32 unsupported");
  if (n == 0) return RFSN_OK;
  switch (d) {
    case 4: return launch_pq_mfma<4>(x, n, ldx, xg, cb, M, C, cbg, codes, ldc, cg, resid, ldr, rg, groups, s);
    case 8: return launch_pq_mfma<8>(x, n, ldx, xg, cb, M, C, cbg, codes, ldc, cg, resid, ldr, rg, groups, s);
    case 16: return launch_pq_mfma<16>(x, n, ldx, xg, cb, M, C, cbg, codes, ldc, cg, resid, ldr, rg, groups, s);
    default: return launch_pq<0>(x, n, ldx, xg, cb, M, C, d, cbg, codes, ldc, cg, resid, ldr, rg, groups, s);
  }
}

int sparse_topk_impl(const void* x, int64_t n, int D, int64_t ldx, const uint8_t* pq, int M, int C,
                     const void* pq_cb, const uint8_t* rvq, int Mr, int Cr, const void* rvq_cb, int k,
                     uint8_t* idx, void* val, hipStream_t s) {
  // head_dim 64, 4- or 8-dim subspaces, an RVQ stage of the same split or
  // none, k = 4, 16-byte aligned rows: four lanes per vector
  const int d = D / M;
  const bool fast = D == 64 && k == 4 && (d == 4 || d == 8) && (Mr == 0 || Mr == M) && ldx % 8 == 0 &&
                    reinterpret_cast<uintptr_t>(x) % 16 == 0 && reinterpret_cast<uintptr_t>(pq_cb) % 16 == 0 &&
                    (Mr == 0 || reinterpret_cast<uintptr_t>(rvq_cb) % 16 == 0);
  if (fast) {
    dim3 grid4((unsigned)ceil_div(n * 4, 256));
#define RFSN_TOPK64(DS, R)                                                                                          \
  hipLaunchKernelGGL((sparse_topk64_kernel<4, DS, R>), grid4, dim3(256), 0, s, (const uint16_t*)x, n, ldx, pq, M, C, \
                     (const uint16_t*)pq_cb, rvq, Cr, (const uint16_t*)rvq_cb, idx, (uint16_t*)val)
    if (d == 4) {
      if (Mr) RFSN_TOPK64(4, true); else RFSN_TOPK64(4, false);
    } else {
      if (Mr) RFSN_TOPK64(8, true); else RFSN_TOPK64(8, false);
    }
#undef RFSN_TOPK64
    return check_launch("sparse_topk");
  }
  dim3 grid((unsigned)ceil_div(n, 256));
#define RFSN_TOPK(KK)                                                                                  \
  hipLaunchKernelGGL(sparse_topk_kernel<KK>, grid, dim3(256), 0, s, (const uint16_t*)x, n, D, ldx, pq, M, C, \
                     (const uint16_t*)pq_cb, rvq, Mr, Cr, (const uint16_t*)rvq_cb, idx, (uint16_t*)val)
  switch (k) {
    case 1: RFSN_TOPK(1); break;
    case 2: RFSN_TOPK(2); break;
    case 3: RFSN_TOPK(3); break;
    case 4: RFSN_TOPK(4); break;
    case 5: RFSN_TOPK(5); break;
    case 6: RFSN_TOPK(6); break;
    case 7: RFSN_TOPK(7); break;
    case 8: RFSN_TOPK(8); break;
    default: return fail(RFSN_ERR_UNSUPPORTED, "sparse_k must be in [0, 8]");
  }
#undef RFSN_TOPK
  return check_launch("sparse_topk");
}

}  // namespace rfsn

using namespace rfsn;

extern "C" int rfsn_pq_encode(const void* x, int64_t n, int32_t D, int64_t ldx, int64_t x_gstride,
                              const void* cb, int32_t M, int32_t C, int64_t cb_gstride, uint8_t* codes, int64_t ldc,
                              int64_t codes_gstride, void* resid, int64_t ldr, int64_t resid_gstride, int32_t groups,
                              void* stream) {
  return pq_encode_impl(x, n, D, ldx, x_gstride, cb, M, C, cb_gstride, codes, ldc, codes_gstride, resid, ldr,
                        resid_gstride, groups, (hipStream_t)stream);
}

static int validate_format(const rfsn_format* f) {
  RFSN_REQUIRE(f != nullptr, "null format");
  RFSN_REQUIRE(f->head_dim > 0 && f->pq_subspaces > 0 && f->head_dim % f->pq_subspaces == 0,
               "head_dim must equal num_subspaces * subspace_dim");
  RFSN_REQUIRE(f->pq_centroids >= 1 && f->pq_centroids <= 256, "PQ codebook size must be in [1, 256]");
  RFSN_REQUIRE(f->rvq_subspaces >= 0, "rvq_subspaces must be >= 0");
  if (f->rvq_subspaces > 0) {
    RFSN_REQUIRE(f->head_dim % f->rvq_subspaces == 0, "head_dim must be a multiple of rvq_subspaces");
    RFSN_REQUIRE(f->rvq_centroids >= 1 && f->rvq_centroids <= 256, "RVQ codebook size must be in [1, 256]");
  }
  RFSN_REQUIRE(f->sparse_k >= 0 && f->sparse_k <= 8 && f->sparse_k <= f->head_dim, "sparse_k must be in [0, 8]");
  RFSN_REQUIRE(f->head_dim <= 256, "head_dim must be <= 256 (uint8 sparse indices)");
  return RFSN_OK;
}

extern "C" size_t rfsn_warm_encode_workspace_bytes(const rfsn_format* f, int64_t n) {
  if (f == nullptr || n <= 0) return 0;
  return (size_t)n * f->head_dim * 2 + 256;
}

extern "C" int rfsn_warm_encode(const rfsn_format* f, const void* x, int64_t n, int64_t ldx, const void* pq_cb,
                                const void* rvq_cb, rfsn_codes out, void* ws, size_t ws_bytes, void* stream) {
  int st = validate_format(f);
  if (st) return st;
  RFSN_REQUIRE(x && pq_cb && out.pq, "warm_encode: null pointer");
  RFSN_REQUIRE(ldx >= f->head_dim, "warm_encode: bad leading dimension");
  if (n == 0) return RFSN_OK;
  RFSN_REQUIRE(f->rvq_subspaces == 0 || (rvq_cb && out.rvq), "warm_encode: RVQ stage needs codebooks and an output");
  RFSN_REQUIRE(f->sparse_k == 0 || (out.sparse_idx && out.sparse_val), "warm_encode: sparse stage needs outputs");
  hipStream_t s = (hipStream_t)stream;
  EncodeJobs jobs = {};
  jobs.count = 1;
  jobs.j[0] = EncodeJob{(const uint16_t*)x, n, ldx, (const uint16_t*)pq_cb, (const uint16_t*)rvq_cb, out.pq, out.rvq,
                        out.sparse_idx, (uint16_t*)out.sparse_val, 0};
  if (fused_encode_ok(f, jobs.j[0])) return launch_warm_encode_fused(f, jobs, s);
  // other formats: PQ, RVQ and top-k as separate launches, the PQ residual in the workspace
  const size_t need = rfsn_warm_encode_workspace_bytes(f, n);
  RFSN_REQUIRE(ws != nullptr && ws_bytes >= need, "warm_encode: workspace too small");
  const int D = f->head_dim;
  uint16_t* r1 = (uint16_t*)ws;  // [n][D] PQ residual
  st = pq_encode_impl(x, n, D, ldx, 0, pq_cb, f->pq_subspaces, f->pq_centroids, 0, out.pq, f->pq_subspaces, 0, r1,
                      D, 0, 1, s);
  if (st) return st;
  if (f->rvq_subspaces > 0) {
    st = pq_encode_impl(r1, n, D, D, 0, rvq_cb, f->rvq_subspaces, f->rvq_centroids, 0, out.rvq, f->rvq_subspaces, 0,
                        nullptr, D, 0, 1, s);
    if (st) return st;
  }
  if (f->sparse_k > 0) {
    st = sparse_topk_impl(x, n, D, ldx, out.pq, f->pq_subspaces, f->pq_centroids, pq_cb, out.rvq, f->rvq_subspaces,
                          f->rvq_centroids, rvq_cb, f->sparse_k, out.sparse_idx, out.sparse_val, s);
    if (st) return st;
  }
  return RFSN_OK;
}

extern "C" int rfsn_warm_encode_batch(const rfsn_format* f, const rfsn_encode_job* jobs, int32_t count,
                                      void* stream) {
  int st = validate_format(f);
  if (st) return st;
  RFSN_REQUIRE(count >= 0 && (count == 0 || jobs != nullptr), "warm_encode_batch: bad job list");
  auto as_job = [](const rfsn_encode_job& j) {
    return EncodeJob{(const uint16_t*)j.x, j.n, j.ldx, (const uint16_t*)j.pq_cb, (const uint16_t*)j.rvq_cb, j.out.pq,
                     j.out.rvq, j.out.sparse_idx, (uint16_t*)j.out.sparse_val, 0};
  };
  // every job is checked before the first launch: a refused call writes no output
  for (int i = 0; i < count; ++i) {
    const rfsn_encode_job& j = jobs[i];
    RFSN_REQUIRE(j.n >= 0 && j.ldx >= f->head_dim, "warm_encode_batch: bad job " + std::to_string(i));
    if (j.n == 0) continue;  // an empty set launches nothing
    RFSN_REQUIRE(j.x && j.pq_cb && j.out.pq, "warm_encode_batch: null pointer in job " + std::to_string(i));
    RFSN_REQUIRE(f->rvq_subspaces == 0 || (j.rvq_cb && j.out.rvq),
                 "warm_encode_batch: RVQ stage needs codebooks and an output");
    RFSN_REQUIRE(f->sparse_k == 0 || (j.out.sparse_idx && j.out.sparse_val),
                 "warm_encode_batch: sparse stage needs outputs");
    if (!fused_encode_ok(f, as_job(j)))
      return fail(RFSN_ERR_UNSUPPORTED, "warm_encode_batch: the one-launch encode serves head_dim 64, 4- or 8-dim "
                                        "subspaces, an RVQ stage of the same split or none, k in {0, 4} and aligned rows");
  }
  hipStream_t s = (hipStream_t)stream;
  for (int i0 = 0; i0 < count; i0 += kMaxJobs) {
    EncodeJobs batch = {};
    for (int i = i0; i < count && i < i0 + kMaxJobs; ++i)
      if (jobs[i].n > 0) batch.j[batch.count++] = as_job(jobs[i]);
    st = launch_warm_encode_fused(f, batch, s);
    if (st) return st;
  }
  return RFSN_OK;
}

extern "C" int rfsn_rvq_gate(const void* r, int64_t n, int32_t D, int64_t ld, float thr, uint8_t* mask, void* stream) {
  RFSN_REQUIRE(r && mask && D > 0 && ld >= D, "rvq_gate: bad arguments");
  if (n == 0) return RFSN_OK;
  hipLaunchKernelGGL(rvq_gate_kernel, dim3((unsigned)ceil_div(n, 256)), dim3(256), 0, (hipStream_t)stream,
                     (const uint16_t*)r, n, D, ld, thr, mask);
  return check_launch("rvq_gate");
}

extern "C" size_t rfsn_mask_compact_workspace_bytes(int64_t n) {
  return (size_t)(ceil_div(n > 0 ? n : 1, kScanTile)) * sizeof(int32_t) + 256;
}

extern "C" int rfsn_mask_compact(const uint8_t* mask, int64_t n, int32_t* offsets, int32_t* count, void* ws,
                                 size_t ws_bytes, void* stream) {
  RFSN_REQUIRE(mask && offsets && count && ws, "mask_compact: null pointer");
  RFSN_REQUIRE(ws_bytes >= rfsn_mask_compact_workspace_bytes(n), "mask_compact: workspace too small");
  RFSN_REQUIRE(n >= 0 && n < (int64_t)0x7fffffff, "mask_compact: n out of range");
  hipStream_t s = (hipStream_t)stream;
  const int64_t tiles = ceil_div(n > 0 ? n : 1, kScanTile);
  int32_t* tile = (int32_t*)ws;
  if (n == 0) {
    hipLaunchKernelGGL(tile_prefix_kernel, dim3(1), dim3(64), 0, s, tile, (int64_t)0, count);
    return check_launch("mask_compact");
  }
  hipLaunchKernelGGL(mask_count_kernel, dim3((unsigned)tiles), dim3(kScanTile), 0, s, mask, n, tile);
  hipLaunchKernelGGL(tile_prefix_kernel, dim3(1), dim3(64), 0, s, tile, tiles, count);
  hipLaunchKernelGGL(mask_scatter_kernel, dim3((unsigned)tiles), dim3(kScanTile), 0, s, mask, n, tile, offsets);
  return check_launch("mask_compact");
}

extern "C" size_t rfsn_rvq_encode_full_workspace_bytes(int64_t active, int32_t D, int32_t L, int32_t C) {
  if (active < 0 || D <= 0 || L <= 0 || C <= 0) return 0;
  return rvq_mfma_ok(D, C) ? rvq_mfma_ws_bytes(active, D, L, C) : 0;
}

extern "C" int rfsn_rvq_encode_full(const void* resid, int64_t ld, int32_t D, const int32_t* offsets, int64_t active,
                                    const void* cb, int32_t L, int32_t C, uint16_t* codes, void* ws, size_t ws_bytes,
                                    void* stream) {
  RFSN_REQUIRE(resid && offsets && cb && codes, "rvq_encode_full: null pointer");
  RFSN_REQUIRE(D > 0 && D <= 1024 && ld >= D && L >= 1 && C >= 1 && C <= 65535, "rvq_encode_full: bad shape");
  RFSN_REQUIRE(active >= 0, "rvq_encode_full: negative row count");
  if (active == 0) return RFSN_OK;
  if (rvq_mfma_ok(D, C)) {
    RFSN_REQUIRE(ws != nullptr && ws_bytes >= rvq_mfma_ws_bytes(active, D, L, C),
                 "rvq_encode_full: workspace too small (rfsn_rvq_encode_full_workspace_bytes)");
    RFSN_REQUIRE(reinterpret_cast<uintptr_t>(ws) % 16 == 0 && reinterpret_cast<uintptr_t>(resid) % 16 == 0 &&
                     reinterpret_cast<uintptr_t>(cb) % 16 == 0 && ld % 8 == 0,
                 "rvq_encode_full: residual rows, codebooks and workspace must be 16-byte aligned");
    hipStream_t s = (hipStream_t)stream;
    switch (D) {
      case 64: return launch_rvq_mfma<64>(resid, ld, offsets, active, cb, L, C, codes, ws, s);
      case 128: return launch_rvq_mfma<128>(resid, ld, offsets, active, cb, L, C, codes, ws, s);
      default: return launch_rvq_mfma<256>(resid, ld, offsets, active, cb, L, C, codes, ws, s);
    }
  }
  const int waves = 4;
  const size_t lds = (size_t)waves * D * sizeof(double);
  hipLaunchKernelGGL(rvq_full_kernel, dim3((unsigned)ceil_div(active, waves)), dim3(64 * waves), lds,
                     (hipStream_t)stream, (const uint16_t*)resid, ld, D, offsets, active, (const uint16_t*)cb, L, C,
                     codes);
  return check_launch("rvq_encode_full");
}
