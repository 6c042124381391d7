// Fused warm-tier dequant + exact decode attention for gfx950 (CDNA4).
//
// Replaces RFSNv10KVCacheMLX.attention_forward (cache.py:395-428):
// materialize_window (cache.py:344-393) followed by
// _blockwise_exact_attention (attention.py:39-105), without ever writing the
// reconstructed window to HBM.
//
// Work decomposition: one block = (sequence b, KV head h, token split);
// 4 waves; each wave streams 32-token tiles of the split.  Per tile:
//   1. K^ tile: PQ and RVQ codebook entries are gathered from LDS with one
//      lane per (token, subspace) -- the codebooks are stored entry-major,
//      [entry][subspace][d], so the 16 (or 8) lanes that one LDS pass serves
//      read 16 distinct bank pairs -- summed as fp16(base + rvq)
//      (quantization.py:317-319) and written to a per-wave LDS tile
//      (8-byte chunks XOR-swizzled by row); the sparse residual is applied in
//      place, K[idx] = fp16(K[idx] + val).
//   2. Scores on MFMA 4x4x4 f16 (16 blocks): B = K^ rows (lane = token),
//      A = the 4 query heads of this KV head; fp32 accumulation.
//   3. Online softmax in base 2 (lane = token, one register per head).
//   4. V^ tile built like K^.
//   5. P.V on MFMA 16x16x16 f16 with A = V^ rows read as (subspace group x
//      (token, coordinate)) and B = P placed on the coordinate diagonal, so
//      that no transpose of V^ is needed; P is scaled by 2^14 before the fp16
//      conversion to keep small weights out of the fp16 subnormal range.
// Split partials (m, l, acc) are merged by merge_partials_kernel.
#include "rfsn_common.h"
#include "rfsn_internal.h"

#include <type_traits>

namespace rfsn {
namespace {

typedef _Float16 half4_t __attribute__((ext_vector_type(4)));
typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
typedef float float4_t __attribute__((ext_vector_type(4)));

constexpr int kTile = 32;                 // tokens per wave tile
constexpr int kWaves = 4;                 // waves per block
constexpr int kD = 64;                    // head_dim of the fused kernel
constexpr int kTileHalves = kTile * kD;   // 4 KB per wave
constexpr int kDepth = 4;                 // tiles whose codes are in flight per wave
constexpr int kCbHalves = 256 * kD;       // one codebook table in LDS (256 entries x D halves)
constexpr size_t kDummyBytes = 4096;      // workspace head read by idle prefetch slots
constexpr float kPScale = 16384.0f;       // 2^14
constexpr float kPScaleInv = 1.0f / 16384.0f;
constexpr float kLog2e = 1.4426950408889634f;

// Order LDS traffic between the lanes of one wave.  A wave's LDS instructions
// execute in issue order, so it is enough that the compiler keeps program
// order (signal fences) and that earlier LDS operations have returned
// (lgkmcnt(0)); global loads in flight (vmcnt) are deliberately not waited on,
// so the tiles prefetched ahead keep streaming.
__device__ __forceinline__ void wave_sync() {
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0); vmcnt and expcnt unconstrained
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
}

// Offset (in halves) of 8-byte chunk c (0..15) of tile row t.
__device__ __forceinline__ int chunk_off(int t, int c) { return t * kD + ((c ^ (t & 15)) << 2); }

// DPP lane exchanges (VALU, no LDS round trip)
template <int Ctrl>
__device__ __forceinline__ float dpp(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), Ctrl, 0xf, 0xf, false));
}
__device__ __forceinline__ float swz16(float v) {
  // ds_swizzle bit mode: lane i reads lane i ^ 16 inside each group of 32
  return __builtin_bit_cast(float, __builtin_amdgcn_ds_swizzle(__builtin_bit_cast(int, v), 0x401f));
}

// max / sum over each group of 32 lanes: quad xor 1, quad xor 2, half-row
// mirror, row mirror (16 lanes), then the swizzle across the two rows
__device__ __forceinline__ float max32(float v) {
  v = fmaxf(v, dpp<0xb1>(v));
  v = fmaxf(v, dpp<0x4e>(v));
  v = fmaxf(v, dpp<0x141>(v));
  v = fmaxf(v, dpp<0x140>(v));
  return fmaxf(v, swz16(v));
}
__device__ __forceinline__ float sum32(float v) {
  v += dpp<0xb1>(v);
  v += dpp<0x4e>(v);
  v += dpp<0x141>(v);
  v += dpp<0x140>(v);
  return v + swz16(v);
}

__device__ __forceinline__ uint32_t add_h2(uint32_t a, uint32_t b) {
  half2_t x = __builtin_bit_cast(half2_t, a);
  half2_t y = __builtin_bit_cast(half2_t, b);
  return __builtin_bit_cast(uint32_t, x + y);  // v_pk_add_f16, IEEE round to nearest even
}

struct TileSrc {
  int kind;        // 0 hot, 1 segment
  int seg;         // segment index
  int off;         // first token of the tile inside its source
  int count;       // valid tokens (1..32)
  int pos0;        // window position of the tile's first token
};

__device__ __forceinline__ int uni(int v) { return __builtin_amdgcn_readfirstlane(v); }
__device__ __forceinline__ const void* uni(const void* p) {
  const uint64_t v = reinterpret_cast<uint64_t>(p);
  const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)v);
  const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(v >> 32));
  return reinterpret_cast<const void*>(((uint64_t)hi << 32) | lo);
}

// Global-address-space views: loads through these are global_load (counted by
// vmcnt only), never flat loads, which would also count against lgkmcnt and
// make every LDS wait drain the prefetched tiles.
typedef const uint8_t __attribute__((address_space(1)))* gbytes;
template <class T>
__device__ __forceinline__ T gload(gbytes base, int64_t off) {
  return *reinterpret_cast<const T __attribute__((address_space(1)))*>(base + off);
}
__device__ __forceinline__ gbytes gview(const void* p) { return (gbytes)(p); }

// The segment table is read through the constant address space: uniform
// indices there compile to scalar loads (SGPR results, lgkmcnt), so looking a
// tile up never waits on the vector-memory counter of the prefetched tiles.
typedef const rfsn_segment __attribute__((address_space(4)))* cseg;

// Tile tt of this (sequence, KV head): hot tiles first, then the segments in order.
__device__ __forceinline__ TileSrc locate_tile(const rfsn_fused_params& p, cseg segs, int tt, int hot_tiles,
                                               int nseg) {
  TileSrc s;
  if (tt < hot_tiles) {
    s.kind = 0;
    s.seg = 0;
    s.off = tt * kTile;
    s.count = min(kTile, p.hot_len - s.off);
    s.pos0 = p.hot_pos0 + s.off;
    return s;
  }
  int r = tt - hot_tiles;
  s.kind = 1;
  s.seg = 0;
  s.off = 0;
  s.count = 0;
  s.pos0 = 0;
  for (int i = 0; i < nseg; ++i) {
    const int len = segs[i].len;
    const int nt = (len + kTile - 1) / kTile;
    if (r < nt) {
      s.seg = i;
      s.off = r * kTile;
      s.count = min(kTile, len - s.off);
      s.pos0 = segs[i].pos0 + s.off;
      return s;
    }
    r -= nt;
  }
  return s;
}

// One tile's encoded data for one lane (K or V): IPT code bytes of the PQ and
// RVQ streams in the tiled layout, and this lane's half of the token's sparse
// entries (lane = token t = lane & 31, entries (lane >> 5)*KS/2 ...).  Loaded
// kDepth tiles ahead of use so that HBM latency overlaps the reconstruction.
template <int M, bool RVQ, int KS>
struct TileRegs {
  static constexpr int IPT = kTile * M / 64;
  static constexpr int NW = IPT / 4;
  uint32_t pq[NW];
  uint32_t rvq[RVQ ? NW : 1];
  uint32_t sidx;  // KS/2 index bytes
  uint32_t sval;  // KS/2 fp16 values
};

// Issue one tile's loads.  The same loads are issued for every slot (invalid
// and hot slots read a dummy address), so the compiler can count outstanding
// loads exactly and wait only for the tile about to be used.
template <int M, bool RVQ, int KS>
__device__ __forceinline__ void load_tile(TileRegs<M, RVQ, KS>& r, const TileSrc& src, cseg sg, bool is_k, int h,
                                          int lane, const uint8_t* dummy) {
  constexpr int IPT = TileRegs<M, RVQ, KS>::IPT;
  const bool real = src.kind == 1;
  const gbytes pq = gview(real ? (const void*)(is_k ? sg->k.pq : sg->v.pq) : (const void*)dummy);
  const gbytes rq = gview(real && RVQ ? (const void*)(is_k ? sg->k.rvq : sg->v.rvq) : (const void*)dummy);
  const int64_t hs = real ? sg->head_stride : 0;
  const int tile_in_seg = real ? src.off / kTile : 0;
  const int hh = real ? h : 0;
  const int64_t base = (int64_t)hh * hs * M + (int64_t)tile_in_seg * kTile * M + lane * IPT;
  if constexpr (IPT == 8) {
    const uint64_t a = gload<uint64_t>(pq, base);
    r.pq[0] = (uint32_t)a;
    r.pq[1] = (uint32_t)(a >> 32);
    if constexpr (RVQ) {
      const uint64_t c = gload<uint64_t>(rq, base);
      r.rvq[0] = (uint32_t)c;
      r.rvq[1] = (uint32_t)(c >> 32);
    }
  } else {
    r.pq[0] = gload<uint32_t>(pq, base);
    if constexpr (RVQ) r.rvq[0] = gload<uint32_t>(rq, base);
  }
  if constexpr (KS > 0) {
    static_assert(KS == 4, "fused kernel carries 4 sparse entries");
    const gbytes si = gview(real ? (const void*)(is_k ? sg->k.sparse_idx : sg->v.sparse_idx) : (const void*)dummy);
    const gbytes sv = gview(real ? (const void*)(is_k ? sg->k.sparse_val : sg->v.sparse_val) : (const void*)dummy);
    const int t = lane & (kTile - 1);
    const int tc = real ? min(t, src.count - 1) : t;  // rows past count re-read the last row
    const int64_t e0 = ((int64_t)hh * hs + (real ? src.off : 0) + tc) * KS + (lane >> 5) * 2;
    r.sidx = gload<uint16_t>(si, e0);
    r.sval = gload<uint32_t>(sv, e0 * 2);
  }
}

// Copy one exact (hot) tile into the wave's LDS tile: rows [off, off+count)
// of hot[...][D]; rows past count -> 0.  All four loads are issued before any
// is used (rows past count re-read the last valid row and are zeroed after).
__device__ __forceinline__ void build_hot_tile(uint16_t* __restrict__ tile, const TileSrc& src,
                                               const uint16_t* __restrict__ hot, int lane) {
  uint4 v[4];
  const int c16 = lane & 7;
#pragma unroll
  for (int k4 = 0; k4 < 4; ++k4) {
    const int row = min((lane >> 3) + 8 * k4, src.count - 1);
    v[k4] = *reinterpret_cast<const uint4*>(hot + (int64_t)(src.off + row) * kD + c16 * 8);
  }
#pragma unroll
  for (int k4 = 0; k4 < 4; ++k4) {
    const int row = (lane >> 3) + 8 * k4;
    if (row >= src.count) v[k4] = make_uint4(0, 0, 0, 0);
    *reinterpret_cast<uint2*>(tile + chunk_off(row, 2 * c16)) = make_uint2(v[k4].x, v[k4].y);
    *reinterpret_cast<uint2*>(tile + chunk_off(row, 2 * c16 + 1)) = make_uint2(v[k4].z, v[k4].w);
  }
}

// Build one reconstructed K^ or V^ tile in LDS (per wave) from prefetched codes.
template <int M, bool RVQ, int KS>
__device__ __forceinline__ void build_tile(uint16_t* __restrict__ tile, const TileSrc& src,
                                           const TileRegs<M, RVQ, KS>& regs, const uint16_t* __restrict__ cb_pq,
                                           const uint16_t* __restrict__ cb_rvq, int C, int Cr, int lane) {
  constexpr int d = kD / M;
  constexpr int TPI = 64 / M;
  constexpr int IPT = kTile / TPI;
  const uint32_t* pc = regs.pq;
  const uint32_t* rc = regs.rvq;
  const int j = lane / M;
  const int m = lane % M;
#pragma unroll
  for (int i = 0; i < IPT; ++i) {
    const int t = TPI * i + j;
    // every code byte indexes a 256-entry LDS table (entries >= C are zero)
    const uint32_t code = (pc[i >> 2] >> ((i & 3) * 8)) & 0xffu;
    const uint16_t* ep = cb_pq + (code * M + m) * d;
    if constexpr (d == 4) {
      uint2 e = *reinterpret_cast<const uint2*>(ep);
      if (RVQ) {
        const uint32_t rcode = (rc[i >> 2] >> ((i & 3) * 8)) & 0xffu;
        const uint2 r = *reinterpret_cast<const uint2*>(cb_rvq + (rcode * M + m) * d);
        e.x = add_h2(e.x, r.x);
        e.y = add_h2(e.y, r.y);
      }
      *reinterpret_cast<uint2*>(tile + chunk_off(t, m)) = e;
    } else {
      uint4 e = *reinterpret_cast<const uint4*>(ep);
      if (RVQ) {
        const uint32_t rcode = (rc[i >> 2] >> ((i & 3) * 8)) & 0xffu;
        const uint4 r = *reinterpret_cast<const uint4*>(cb_rvq + (rcode * M + m) * d);
        e.x = add_h2(e.x, r.x);
        e.y = add_h2(e.y, r.y);
        e.z = add_h2(e.z, r.z);
        e.w = add_h2(e.w, r.w);
      }
      *reinterpret_cast<uint2*>(tile + chunk_off(t, 2 * m)) = make_uint2(e.x, e.y);
      *reinterpret_cast<uint2*>(tile + chunk_off(t, 2 * m + 1)) = make_uint2(e.z, e.w);
    }
  }
  if constexpr (KS > 0) {
    // sparse residual in place: K[idx] = fp16(K[idx] + val); the indices of
    // one token are distinct, so the two lanes of a token never collide
    wave_sync();
    const int t = lane & (kTile - 1);
    if (t < src.count) {
#pragma unroll
      for (int e = 0; e < 2; ++e) {
        const int idx = (regs.sidx >> (8 * e)) & (kD - 1);
        const int o = chunk_off(t, idx >> 2) + (idx & 3);
        tile[o] = hadd_bits(tile[o], (uint16_t)(regs.sval >> (16 * e)));
      }
    }
  }
}

template <int M, bool RVQ, int KS, int NHG>
__global__ void __launch_bounds__(256, 1)
fused_decode_attn_kernel(const rfsn_fused_params p, int splits, int tiles_per_split, int blocks_total) {
  extern __shared__ uint16_t lds[];
  // XCD-aware block mapping: consecutive hardware block ids go to different
  // XCDs; give each XCD a contiguous range of (sequence, head, split) units so
  // that one sequence's codebooks are fetched into one L2.
  const int L = blockIdx.x;
  const int per = blocks_total / 8, rem = blocks_total % 8;
  const int xcd = L % 8, k = L / 8;
  const int vid = xcd * per + min(xcd, rem) + k;
  const int split = vid % splits;
  const int h = (vid / splits) % p.kv_heads;
  const int b = vid / (splits * p.kv_heads);

  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
  const int G = p.q_heads / p.kv_heads;
  const int C = p.fmt.pq_centroids, Cr = RVQ ? p.fmt.rvq_centroids : 0;
  (void)C;
  (void)Cr;

  // LDS: 256-entry codebook tables (K-PQ, V-PQ[, K-RVQ, V-RVQ]), then the
  // per-wave tiles and P buffers
  uint16_t* cbKp = lds;
  uint16_t* cbVp = cbKp + kCbHalves;
  uint16_t* cbKr = cbVp + kCbHalves;
  uint16_t* cbVr = cbKr + (RVQ ? kCbHalves : 0);
  uint16_t* tiles = cbVr + (RVQ ? kCbHalves : 0);
  uint16_t* tile = tiles + wave * kTileHalves;
  uint16_t* pb = tiles + kWaves * kTileHalves + wave * (NHG * 128);
  const uint8_t* dummy = reinterpret_cast<const uint8_t*>(p.workspace);  // readable scratch for idle slots
  const cseg segs = (cseg)(p.segments + (int64_t)b * p.max_segments);
  const int nseg = p.num_segments ? p.num_segments[b] : 0;

  // ---- stage this sequence's codebooks: HBM [m][e][d] -> LDS [e][m][d]
  {
    constexpr int d = kD / M;
    const uint16_t* srcs[4] = {(const uint16_t*)p.k_pq_cb + (int64_t)b * p.pq_cb_stride,
                               (const uint16_t*)p.v_pq_cb + (int64_t)b * p.pq_cb_stride,
                               RVQ ? (const uint16_t*)p.k_rvq_cb + (int64_t)b * p.rvq_cb_stride : nullptr,
                               RVQ ? (const uint16_t*)p.v_rvq_cb + (int64_t)b * p.rvq_cb_stride : nullptr};
    uint16_t* dsts[4] = {cbKp, cbVp, cbKr, cbVr};
#pragma unroll
    for (int c = 0; c < (RVQ ? 4 : 2); ++c) {
      const int n = c < 2 ? C : Cr;
      for (int idx = threadIdx.x; idx < M * 256; idx += blockDim.x) {
        const int m = idx / 256, e = idx % 256;
        uint16_t* t = dsts[c] + (e * M + m) * d;
        if constexpr (d == 4) {
          uint2 v = make_uint2(0, 0);
          if (e < n) v = *reinterpret_cast<const uint2*>(srcs[c] + ((int64_t)m * n + e) * d);
          *reinterpret_cast<uint2*>(t) = v;
        } else {
          uint4 v = make_uint4(0, 0, 0, 0);
          if (e < n) v = *reinterpret_cast<const uint4*>(srcs[c] + ((int64_t)m * n + e) * d);
          *reinterpret_cast<uint4*>(t) = v;
        }
      }
    }
  }

  // ---- query registers (4x4x4 A operand): lane l -> head group hgl, head r = l & 3
  const int hgl = (NHG == 2) ? (lane >> 5) : 0;
  const int myhead = hgl * 4 + (lane & 3);
  half4_t qa[16];
  {
    const bool qv = myhead < G;
    const uint16_t* qrow = (const uint16_t*)p.q + ((int64_t)b * p.q_heads + h * G + (qv ? myhead : 0)) * kD;
#pragma unroll
    for (int s = 0; s < 16; ++s) {
      uint2 w = qv ? *reinterpret_cast<const uint2*>(qrow + 4 * s) : make_uint2(0, 0);
      qa[s] = __builtin_bit_cast(half4_t, w);
    }
  }
  int qp[4];
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int hh = hgl * 4 + r;
    qp[r] = (p.causal && p.qpos && hh < G) ? p.qpos[(int64_t)b * p.q_heads + h * G + hh] : 0x7fffffff;
  }
  const float scale_log2 = p.scale * kLog2e;
  const int hot_tiles = (p.hot_len + kTile - 1) / kTile;
  int total_tiles = hot_tiles;
  for (int i = 0; i < nseg; ++i) total_tiles += (segs[i].len + kTile - 1) / kTile;
  const int t_begin = split * tiles_per_split;
  const int t_end = min(total_tiles, t_begin + tiles_per_split);
  const uint16_t* hotk = (const uint16_t*)p.hot_k + (int64_t)b * p.hot_seq_stride + (int64_t)h * p.hot_cap * kD;
  const uint16_t* hotv = (const uint16_t*)p.hot_v + (int64_t)b * p.hot_seq_stride + (int64_t)h * p.hot_cap * kD;

  float m_run[4], l_run[4];
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    m_run[r] = -__builtin_inff();
    l_run[r] = 0.f;
  }
  float4_t acc[NHG];
#pragma unroll
  for (int g = 0; g < NHG; ++g) acc[g] = float4_t{0.f, 0.f, 0.f, 0.f};

  __syncthreads();

  const int jq = lane >> 4;  // k-group of the 16x16x16 operands
  const int cq = lane & 15;  // column (B) / row (A)
  using Regs = TileRegs<M, RVQ, KS>;
  // kDepth tiles in flight per wave: slot s holds tile tt + s*kWaves
  TileSrc srcs[kDepth];
  Regs kr[kDepth], vr[kDepth];
  auto fetch = [&](TileSrc& s, Regs& rk, Regs& rv, int tt) {
    if (tt < t_end) {
      s = locate_tile(p, segs, tt, hot_tiles, nseg);
    } else {
      s.kind = -1;
      s.seg = 0;
    }
    const cseg sg = segs + s.seg;
    load_tile<M, RVQ, KS>(rk, s, sg, true, h, lane, dummy);
    load_tile<M, RVQ, KS>(rv, s, sg, false, h, lane, dummy);
  };
  auto process = [&](auto hot_tag, const TileSrc& src, const Regs& rk, const Regs& rv) {
    constexpr bool HOT = decltype(hot_tag)::value;
    // ---- K^ tile and scores
    if constexpr (HOT) {
      build_hot_tile(tile, src, hotk, lane);
    } else {
      build_tile<M, RVQ, KS>(tile, src, rk, cbKp, cbKr, C, Cr, lane);
    }
    wave_sync();
    float4_t sc = float4_t{0.f, 0.f, 0.f, 0.f};
    const int trow = lane & (kTile - 1);
#pragma unroll
    for (int s = 0; s < 16; ++s) {
      const half4_t kv = __builtin_bit_cast(half4_t, *reinterpret_cast<const uint2*>(tile + chunk_off(trow, s)));
      sc = __builtin_amdgcn_mfma_f32_4x4x4f16(qa[s], kv, sc, 0, 0, 0);
    }
    // ---- online softmax (lane = token trow, register r = head hgl*4 + r)
    const int pos = src.pos0 + trow;
    float corr[4];
    uint16_t p16[4];
    bool rescaled = false;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const bool allowed = trow < src.count && (hgl * 4 + r) < G && pos >= 0 && pos <= qp[r];
      const float sv = allowed ? sc[r] * scale_log2 : -__builtin_inff();
      // The running max only moves when some lane exceeds it; most tiles skip
      // the cross-lane reduction and the rescale (any max gives the same
      // softmax, the running one only keeps exp2 in range).
      float mn = m_run[r];
      corr[r] = 1.f;
      if (__ballot(sv > mn)) {
        mn = fmaxf(m_run[r], max32(sv));
        corr[r] = (m_run[r] > -__builtin_inff()) ? __builtin_amdgcn_exp2f(m_run[r] - mn) : 0.f;
        rescaled = true;
      }
      const float pv = allowed ? __builtin_amdgcn_exp2f(sv - mn) : 0.f;
      p16[r] = f2h(pv * kPScale);
      const float pr = h2f(p16[r]) * kPScaleInv;
      l_run[r] = l_run[r] * corr[r] + pr;  // per-lane partial sum, reduced once at the end
      m_run[r] = mn;
    }
    if (NHG == 2 || lane < 32) {
#pragma unroll
      for (int r = 0; r < 4; ++r) pb[((hgl * 4 + (trow & 3)) * 4 + r) * 8 + (trow >> 2)] = p16[r];
    }
    wave_sync();
    // ---- V^ tile
    if constexpr (HOT) {
      build_hot_tile(tile, src, hotv, lane);
    } else {
      build_tile<M, RVQ, KS>(tile, src, rv, cbVp, cbVr, C, Cr, lane);
    }
    wave_sync();
    // ---- rescale accumulators and P.V
#pragma unroll
    for (int g = 0; g < NHG; ++g) {
      const int hr = cq >> 2;
      if (rescaled) {
        float cg[4];
#pragma unroll
        for (int r = 0; r < 4; ++r)
          cg[r] = (NHG == 1) ? corr[r]
                             : __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, corr[r]), g * 32));
        const float f = hr == 0 ? cg[0] : hr == 1 ? cg[1] : hr == 2 ? cg[2] : cg[3];
        acc[g] *= f;
      }
      const uint4 pw = *reinterpret_cast<const uint4*>(pb + ((g * 4 + jq) * 4 + hr) * 8);
      const uint32_t pws[4] = {pw.x, pw.y, pw.z, pw.w};
      const int u = cq & 3;
#pragma unroll
      for (int i = 0; i < kTile / 4; ++i) {
        const half4_t av =
            __builtin_bit_cast(half4_t, *reinterpret_cast<const uint2*>(tile + chunk_off(4 * i + jq, cq)));
        const uint32_t ph = (pws[i >> 1] >> ((i & 1) * 16)) & 0xffffu;
        const uint32_t sh = ph << ((u & 1) * 16);
        const uint2 bw = (u < 2) ? make_uint2(sh, 0u) : make_uint2(0u, sh);
        acc[g] = __builtin_amdgcn_mfma_f32_16x16x16f16(av, __builtin_bit_cast(half4_t, bw), acc[g], 0, 0, 0);
      }
    }
    wave_sync();
  };
  // Phase 1: exact (hot) tiles, loaded synchronously (a few percent of tiles).
  const int hot_end = min(t_end, hot_tiles);
  for (int tt = t_begin + wave; tt < hot_end; tt += kWaves) {
    const TileSrc src = locate_tile(p, segs, tt, hot_tiles, nseg);
    process(std::true_type{}, src, kr[0], vr[0]);
  }
  // Phase 2: encoded tiles, kDepth tiles of codes in flight per wave.
  const int seg_begin = max(t_begin, hot_tiles);
#pragma unroll
  for (int s = 0; s < kDepth; ++s) fetch(srcs[s], kr[s], vr[s], seg_begin + wave + s * kWaves);
  for (int tt = seg_begin + wave; tt < t_end; tt += kDepth * kWaves) {
#pragma unroll
    for (int s = 0; s < kDepth; ++s) {
      if (srcs[s].kind >= 0) process(std::false_type{}, srcs[s], kr[s], vr[s]);
      fetch(srcs[s], kr[s], vr[s], tt + (s + kDepth) * kWaves);
    }
  }

  // ---- combine the waves of this block and write the split partial
  __syncthreads();
  float* red = reinterpret_cast<float*>(lds);  // [w][8] m, [w][8] l, [w][8][64] acc
  float* red_m = red;
  float* red_l = red + kWaves * 8;
  float* red_a = red + kWaves * 16;
#pragma unroll
  for (int r = 0; r < 4; ++r) l_run[r] = sum32(l_run[r]);
  if (lane == 0 || (NHG == 2 && lane == 32)) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      red_m[wave * 8 + hgl * 4 + r] = m_run[r];
      red_l[wave * 8 + hgl * 4 + r] = l_run[r];
    }
  }
#pragma unroll
  for (int g = 0; g < NHG; ++g) {
    const int head = g * 4 + (cq >> 2);
#pragma unroll
    for (int r = 0; r < 4; ++r) red_a[(wave * 8 + head) * kD + 16 * jq + 4 * r + (cq & 3)] = acc[g][r] * kPScaleInv;
  }
  __syncthreads();
  for (int idx = threadIdx.x; idx < G * kD; idx += blockDim.x) {
    const int head = idx / kD, c = idx % kD;
    float Mx = -__builtin_inff();
    for (int w = 0; w < kWaves; ++w) Mx = fmaxf(Mx, red_m[w * 8 + head]);
    float Ls = 0.f, A = 0.f;
    for (int w = 0; w < kWaves; ++w) {
      const float mw = red_m[w * 8 + head];
      const float f = mw > -__builtin_inff() ? exp2f(mw - Mx) : 0.f;
      Ls += red_l[w * 8 + head] * f;
      A += red_a[(w * 8 + head) * kD + c] * f;
    }
    if (splits == 1) {
      // whole (sequence, KV head) in this block: normalise and write fp16 directly
      // (a query with no allowed key returns zeros, attention.py:104-105)
      uint16_t* o = (uint16_t*)p.out + ((int64_t)b * p.q_heads + h * G + head) * kD;
      o[c] = f2h(Ls > 0.f ? A / Ls : 0.f);
      continue;
    }
    float* out = reinterpret_cast<float*>(reinterpret_cast<char*>(p.workspace) + kDummyBytes) +
                 (((int64_t)b * p.q_heads + h * G + head) * splits + split) * (kD + 2);
    if (c == 0) {
      out[0] = Mx;
      out[1] = Ls;
    }
    out[2 + c] = A;
  }
}

size_t fused_lds_bytes(const rfsn_format& f, int nhg) {
  size_t cb = (size_t)(f.rvq_subspaces > 0 ? 4 : 2) * kCbHalves * 2;
  size_t t = (size_t)kWaves * kTileHalves * 2 + (size_t)kWaves * nhg * 128 * 2;
  size_t red = (size_t)kWaves * 16 * 4 + (size_t)kWaves * 8 * kD * 4;
  return (cb + t) > red ? (cb + t) : red;
}

int total_tiles_host(const rfsn_fused_params* p) {
  // upper bound: hot tiles + tiles of max_tokens encoded tokens split over segments
  const int hot_tiles = (p->hot_len + kTile - 1) / kTile;
  const int enc = p->max_tokens - p->hot_len;
  return hot_tiles + (enc > 0 ? (enc + kTile - 1) / kTile : 0) + p->max_segments;
}

int auto_splits(const rfsn_fused_params* p) {
  if (p->splits > 0) return p->splits;
  const int units = p->batch * p->kv_heads;
  const int tiles = total_tiles_host(p);
  int s = (256 + units - 1) / units;          // one block per CU (LDS-bound occupancy)
  const int max_s = (tiles + kWaves - 1) / kWaves;  // at least one tile per wave
  if (s > max_s) s = max_s;
  if (s < 1) s = 1;
  return s;
}

template <int M, bool RVQ, int KS, int NHG>
int launch_fused(const rfsn_fused_params* p, hipStream_t s) {
  const int splits = auto_splits(p);
  const int tiles = total_tiles_host(p);
  const int tps = (tiles + splits - 1) / splits;
  const int blocks = p->batch * p->kv_heads * splits;
  const size_t lds = fused_lds_bytes(p->fmt, NHG);
  auto kern = fused_decode_attn_kernel<M, RVQ, KS, NHG>;
  hipError_t e = hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
  if (e != hipSuccess) return fail(RFSN_ERR_HIP, std::string("fused: hipFuncSetAttribute: ") + hipGetErrorString(e));
  hipLaunchKernelGGL(kern, dim3((unsigned)blocks), dim3(256), lds, s, *p, splits, tps, blocks);
  int st = check_launch("fused_decode_attention");
  if (st || splits == 1) return st;
  return launch_merge(reinterpret_cast<const float*>(reinterpret_cast<const char*>(p->workspace) + kDummyBytes),
                      (int64_t)p->batch * p->q_heads, splits, kD, p->out, s);
}

template <int M, bool RVQ, int KS>
int dispatch_nhg(const rfsn_fused_params* p, hipStream_t s) {
  const int G = p->q_heads / p->kv_heads;
  if (G <= 4) return launch_fused<M, RVQ, KS, 1>(p, s);
  return launch_fused<M, RVQ, KS, 2>(p, s);
}

template <int M, bool RVQ>
int dispatch_ks(const rfsn_fused_params* p, hipStream_t s) {
  switch (p->fmt.sparse_k) {
    case 0: return dispatch_nhg<M, RVQ, 0>(p, s);
    case 4: return dispatch_nhg<M, RVQ, 4>(p, s);
    default: return fail(RFSN_ERR_UNSUPPORTED, "fused: sparse_k must be 0 or 4");
  }
}

}  // namespace
}  // namespace rfsn

using namespace rfsn;

extern "C" size_t rfsn_fused_workspace_bytes(const rfsn_fused_params* p) {
  if (p == nullptr || p->batch <= 0 || p->q_heads <= 0 || p->kv_heads <= 0) return 0;
  const int splits = auto_splits(p);
  return kDummyBytes + (size_t)p->batch * p->q_heads * splits * (kD + 2) * sizeof(float);
}

extern "C" int rfsn_fused_decode_attention(const rfsn_fused_params* p, void* stream) {
  RFSN_REQUIRE(p != nullptr, "fused: null params");
  const rfsn_format& f = p->fmt;
  RFSN_REQUIRE(f.head_dim == kD, "fused: head_dim must be 64");
  RFSN_REQUIRE(f.pq_subspaces == 8 || f.pq_subspaces == 16, "fused: num_subspaces must be 8 or 16");
  RFSN_REQUIRE(f.rvq_subspaces == 0 || f.rvq_subspaces == f.pq_subspaces,
               "fused: rvq_subspaces must be 0 or equal to num_subspaces");
  RFSN_REQUIRE(f.pq_centroids >= 1 && f.pq_centroids <= 256, "fused: PQ codebook size must be in [1, 256]");
  RFSN_REQUIRE(f.rvq_subspaces == 0 || (f.rvq_centroids >= 1 && f.rvq_centroids <= 256),
               "fused: RVQ codebook size must be in [1, 256]");
  RFSN_REQUIRE(p->batch > 0 && p->q_heads > 0 && p->kv_heads > 0 && p->q_heads % p->kv_heads == 0,
               "fused: query heads must be a multiple of KV heads");
  RFSN_REQUIRE(p->q_heads / p->kv_heads <= 8, "fused: at most 8 query heads per KV head");
  RFSN_REQUIRE(p->q && p->out && p->k_pq_cb && p->v_pq_cb, "fused: null pointer");
  RFSN_REQUIRE(f.rvq_subspaces == 0 || (p->k_rvq_cb && p->v_rvq_cb), "fused: RVQ codebooks missing");
  RFSN_REQUIRE(p->hot_len >= 0 && (p->hot_len == 0 || (p->hot_k && p->hot_v && p->hot_cap >= p->hot_len)),
               "fused: bad hot tier");
  RFSN_REQUIRE(p->max_segments >= 0 && (p->max_segments == 0 || (p->segments && p->num_segments)),
               "fused: bad segment table");
  RFSN_REQUIRE(p->max_tokens >= p->hot_len, "fused: max_tokens must cover the hot tier");
  RFSN_REQUIRE(p->workspace && p->workspace_bytes >= rfsn_fused_workspace_bytes(p), "fused: workspace too small");
  hipStream_t s = (hipStream_t)stream;
  const bool rvq = f.rvq_subspaces > 0;
  if (f.pq_subspaces == 16) return rvq ? dispatch_ks<16, true>(p, s) : dispatch_ks<16, false>(p, s);
  return rvq ? dispatch_ks<8, true>(p, s) : dispatch_ks<8, false>(p, s);
}
