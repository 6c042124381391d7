// Fused warm-tier dequant + exact decode attention for gfx950 (CDNA4).
//
// Replaces RFSNv10KVCacheMLX.attention_forward (cache.py:395-428):
// materialize_window (cache.py:344-393) followed by
// _blockwise_exact_attention (attention.py:39-105), without ever writing the
// reconstructed window to HBM.
//
// Work decomposition: one block = (sequence b, KV head h, token split) with
// 16 waves, four per SIMD (12 when a KV head serves 8 query heads); each
// wave streams 32-token tiles of the split and
// passes each through a 2 KB LDS buffer in 16-token halves.  LDS holds the
// sequence's codebooks as two 64 KB tables (K, V), entry-major with 256-byte
// entries [PQ entries of the M subspaces | RVQ entries], then the waves'
// half-tile buffers (up to 160 KB in total).  Per tile:
//   1. K^ rows, per half: one lane per (token, subspace) and gather; the LDS
//      address of a codebook entry is built from the code byte with one
//      v_perm_b32 (code * 256 + subspace slot), and each LDS pass reads all 64
//      banks.  fp16(base + rvq) on v_pk_add_f16 (quantization.py:317-319)
//      goes to the wave's buffer (16-byte units XOR-swizzled by row); the
//      sparse stage stores the segment's corrected coordinates
//      fp16(K[idx] + val) over the reconstructed ones.
//   2. Scores on MFMA 16x16x32 f16: A = the 16 buffer rows ordered so that
//      token 16u+4i+g of half u lands in row 4g+i, B = the query heads
//      replicated over 4 columns each; fp32 accumulation.  Lane (g, n)
//      receives the scores of tokens 16u+4i+g (i = 0..3) for query head n/4.
//   3. Online softmax in base 2 on those registers; the running max is only
//      reduced across lanes when some score exceeds it by more than the fp16
//      headroom of P.
//   4. V^ halves built like K^; with 16 subspaces the gather registers are
//      already the P.V A operands and only pass through the buffer (lane-major,
//      one 16-byte store and load per operand) for the sparse stage.
//   5. P.V on MFMA 16x16x32 f16: A = V^ rows read as (subspace x (token,
//      coordinate)), B = the lane's own probabilities placed on the coordinate
//      diagonal (the score layout of step 2 is already the B layout, so P
//      never moves between lanes); a second MFMA with A = 1 accumulates the
//      softmax denominator.  P is produced as p * 2^14 before the fp16
//      conversion, keeping small weights out of the fp16 subnormal range;
//      the factor cancels in out = acc / l.
// The steps are software-pipelined: every gather is issued one step before
// the store that consumes it.
// Score tables (k_layout 1: 16 PQ + 16 RVQ subspaces, at most 4 query heads
// per KV head): the block first writes T[code][slot][head] = fp16(q_head .
// centroid) over the 32 slots (PQ subspaces, then RVQ) into the K table's
// place, same 256-byte entries.  K codes then arrive in the
// rfsn_pack_score_codes layout and a lane (row r, k-group kg) gathers 8 table
// entries of one token (4 slots x both stages), which are directly two
// 16x16x32 A operands with k = (slot, head); B selects head = k % 4 into the
// replicated score columns, so four MFMAs per half tile sum the 32 slots in
// fp32 and K^ is never built.  The sparse stage adds fp16(q[idx] * delta)
// through a 16x16x16 MFMA, q[idx] taken from other lanes' registers by
// ds_bpermute.
// Split partials (m, l, acc) are merged by merge_partials_kernel.
#include "rfsn_common.h"
#include "rfsn_internal.h"

#include <mutex>
#include <type_traits>

namespace rfsn {
namespace {

typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
typedef _Float16 half4_t __attribute__((ext_vector_type(4)));
typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef float float4_t __attribute__((ext_vector_type(4)));

constexpr int kTile = 32;                           // tokens per wave tile
constexpr int kD = 64;                              // head_dim of the fused kernel
constexpr int kDepth = 2;                           // tiles whose codes are in flight per wave
constexpr int kTableMinTilesPerWave = 16;           // tiles per wave for which the score tables pay off
constexpr int kEntryBytes = 256;                    // one codebook entry: PQ slots, then RVQ slots
constexpr int kRvqSlot = 128;                       // byte offset of the RVQ slots in an entry
constexpr int kTableBytes = 256 * kEntryBytes;      // one K or V table, 64 KB
constexpr int kHalf = 16;                           // tokens per LDS half tile
constexpr int kBufBytes = kHalf * kD * 2;           // 2 KB half-tile buffer per wave
constexpr int kTilesBase = 2 * kTableBytes;         // tiles follow the K and V tables
// Waves per block: 16 (4 per SIMD, 160 KB of LDS) when a KV head serves at
// most 4 query heads; 12 when it serves 8 (the second head group's registers
// must fit 170 VGPRs instead of 128).
template <int NHG>
struct BlockShape {
  static constexpr int W = NHG == 1 ? 16 : 12;
  static constexpr int T = W * 64;
  static constexpr size_t L = (size_t)kTilesBase + (size_t)W * kBufBytes;
  static_assert(L <= 160 * 1024, "LDS per CU");
  static_assert((size_t)W * 24 * 4 + (size_t)W * 8 * kD * 4 + 8 * 4 <= L, "the wave combine reuses the codebook LDS");
};
constexpr float kPScaleLog2 = 14.0f;                // P is produced as p * 2^14
// A score may exceed the running max by this much (log2 units) before the max
// is moved: P then stays below 2^15.75 < 65504, the fp16 maximum.
constexpr float kSlackLog2 = 1.75f;
constexpr float kLog2e = 1.4426950408889634f;
// Variance of a uniform rounding error of at most half an fp16 ulp, per unit
// x^2: ulp(x) <= 2^-10 |x|, so ulp^2 / 12 <= 2^-20 x^2 / 12.
constexpr float kDriftVar = 1.0f / (12.0f * 1048576.0f);

__device__ __forceinline__ uint32_t fbits(float v) { return __builtin_bit_cast(uint32_t, v); }
__device__ __forceinline__ float bitsf(uint32_t v) { return __builtin_bit_cast(float, v); }

// max over lanes l, l^16 (resp. l^32): v_permlane16/32_swap exchange the rows
// (halves) of the wave in one VALU op each.
__device__ __forceinline__ float xmax16(float v) {
  const auto r = __builtin_amdgcn_permlane16_swap(fbits(v), fbits(v), false, false);
  return fmaxf(bitsf(r[0]), bitsf(r[1]));
}
__device__ __forceinline__ float xmax32(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(fbits(v), fbits(v), false, false);
  return fmaxf(bitsf(r[0]), bitsf(r[1]));
}

__device__ __forceinline__ uint32_t add_h2(uint32_t a, uint32_t b) {
  half2_t x = __builtin_bit_cast(half2_t, a);
  half2_t y = __builtin_bit_cast(half2_t, b);
  return __builtin_bit_cast(uint32_t, x + y);  // v_pk_add_f16, IEEE round to nearest even
}

// Tile layout: row t (token) holds 64 fp16 = 8 units of 16 bytes; unit c of
// row t sits at unit c ^ row_swz(t).  LDS serves 64 banks (256 bytes) per
// pass, so a row's parity picks the bank half and row_swz must spread the
// units of same-parity rows: every pass below is then conflict-free -- two
// adjacent rows' chunks (gather stores, V operand reads, hot stores) and the
// 16 rows 4(n&3)+(n>>2) of a score operand read.
__device__ __forceinline__ int row_swz(int t) { return (t >> 1) & 7; }

// LDS byte address of the codebook entry selected by byte k of the code word
// w: code * 256 + lc.byte0 (the lane's subspace slot) + lc.byte2 * 65536 (the
// K or V table).  v_perm_b32 byte selectors: 4 -> lc.byte0, k -> w.byte k,
// 6 -> lc.byte2, 12 -> 0x00.
__device__ __forceinline__ uint32_t entry_addr(uint32_t w, uint32_t lc, int k) {
  return __builtin_amdgcn_perm(lc, w, 0x0C060004u | ((uint32_t)k << 8));
}

struct TileSrc {
  int kind;        // 0 hot, 1 segment, -1 idle slot
  int seg;         // segment index
  int off;         // first token of the tile inside its source
  int count;       // valid tokens (1..32)
  int pos0;        // window position of the tile's first token
};

// Global-address-space views: loads through these are global_load (counted by
// vmcnt only), never flat loads, which would also count against lgkmcnt and
// make every LDS wait drain the prefetched tiles.
typedef const uint8_t __attribute__((address_space(1)))* gbytes;
template <class T>
__device__ __forceinline__ T gload(gbytes base, uint32_t off) {  // base uniform, off per lane
  return *reinterpret_cast<const T __attribute__((address_space(1)))*>(base + off);
}
__device__ __forceinline__ gbytes gview(const void* p) { return (gbytes)(p); }

// The segment table is read through the constant address space: uniform
// indices there compile to scalar loads (SGPR results, lgkmcnt), so looking a
// tile up never waits on the vector-memory counter of the prefetched tiles.
typedef const rfsn_segment __attribute__((address_space(4)))* cseg;

// This KV head's rows of one segment: base addresses of its code and sparse
// streams [K, V] (scalar registers) and the segment's extent.  Tiles of the
// segment are then addressed with 32-bit offsets from these bases.
struct WarmBase {
  gbytes pq[2];
  gbytes rvq[2];
  gbytes si[2];
  gbytes sv[2];
  int len;
  int pos0;
  uint32_t kplane;  // bytes from K's score deltas to its corrected-coordinate plane (exact pass over score rows)
};
template <int M, bool RVQ, int KS, bool PLANE = false>
__device__ __forceinline__ WarmBase warm_base(cseg sg, int h, int kv_heads = 0) {
  WarmBase w;
  w.kplane = PLANE ? (uint32_t)((int64_t)kv_heads * sg->head_stride * KS * 2) : 0u;
  const int64_t row = (int64_t)h * sg->head_stride;  // first token row of head h
  const void* pq[2] = {sg->k.pq, sg->v.pq};
  const void* rvq[2] = {sg->k.rvq, sg->v.rvq};
  const void* si[2] = {sg->k.sparse_idx, sg->v.sparse_idx};
  const void* sv[2] = {sg->k.sparse_val, sg->v.sparse_val};
#pragma unroll
  for (int kv = 0; kv < 2; ++kv) {
    w.pq[kv] = gview(pq[kv]) + row * M;
    w.rvq[kv] = RVQ ? gview(rvq[kv]) + row * M : w.pq[kv];
    w.si[kv] = KS ? gview(si[kv]) + row * KS : w.pq[kv];
    w.sv[kv] = KS ? gview(sv[kv]) + row * KS * 2 : w.pq[kv];
  }
  w.len = sg->len;
  w.pos0 = sg->pos0;
  return w;
}

// Hot tile tt of this (sequence, KV head).
__device__ __forceinline__ TileSrc hot_tile(const rfsn_fused_params& p, int tt) {
  TileSrc s;
  s.kind = 0;
  s.seg = 0;
  s.off = tt * kTile;
  s.count = min(kTile, p.hot_len - s.off);
  s.pos0 = p.hot_pos0 + s.off;
  return s;
}

// Encoded tile r of segments 1..nseg-1 (r counted from the first tile of
// segment 1), walking the table (uniform).  The lengths of 8 segments are read
// per step, with no data dependence between the reads, so a walk costs one
// scalar-memory round trip per 8 segments.  r must lie inside the table.
__device__ __forceinline__ TileSrc walk_segments(cseg segs, int nseg, int r) {
  TileSrc s;
  s.kind = 1;
  s.seg = nseg - 1;
  s.off = 0;
  s.count = 0;
  s.pos0 = 0;
  for (int i0 = 1; i0 < nseg; i0 += 8) {
    int nt[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int i = min(i0 + j, nseg - 1);  // entries past the table count no tiles
      const int n = (segs[i].len + kTile - 1) / kTile;
      nt[j] = i0 + j < nseg ? n : 0;
    }
    int found = -1;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      if (found < 0) {
        if (r < nt[j]) found = j;
        else r -= nt[j];
      }
    }
    if (found >= 0) {
      const int seg = i0 + found;
      const int len = segs[seg].len;
      s.seg = seg;
      s.off = r * kTile;
      s.count = min(kTile, len - s.off);
      s.pos0 = segs[seg].pos0 + s.off;
      return s;
    }
  }
  return s;
}

// Encoded tile r of segments 1..nseg-1 from the host's tile map (uniform):
// one scalar load, then the segment's fields.  Entries are clamped to the
// table (a segment index past it reads the last segment; a tile past its
// segment counts no tokens).
typedef const uint32_t __attribute__((address_space(4)))* cmap;
__device__ __forceinline__ TileSrc map_tile(cseg segs, int nseg, cmap row, int r) {
  const uint32_t e = row[r];
  TileSrc s;
  s.kind = 1;
  s.seg = min((int)(e >> 16), nseg - 1);
  s.off = (int)(e & 0xFFFFu) * kTile;
  s.count = max(0, min(kTile, segs[s.seg].len - s.off));
  s.pos0 = segs[s.seg].pos0 + s.off;
  return s;
}

// Tiles of segments 1..nseg-1, 8 independent reads per step.
__device__ __forceinline__ int tail_tiles(cseg segs, int nseg) {
  int total = 0;
  for (int i0 = 1; i0 < nseg; i0 += 8) {
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int i = min(i0 + j, nseg - 1);
      const int n = (segs[i].len + kTile - 1) / kTile;
      total += i0 + j < nseg ? n : 0;
    }
  }
  return total;
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

// Issue one tile's loads: the tile starting at token off (a multiple of 32)
// of the segment whose bases are w, count valid tokens.  Bases are uniform
// (scalar registers); lanes add 32-bit offsets.  Every slot issues the same
// loads (idle slots re-read a real tile), so the compiler counts outstanding
// loads exactly and waits only for the tile about to be used.
template <int M, bool RVQ, int KS>
__device__ __forceinline__ void load_tile(TileRegs<M, RVQ, KS>& r, const WarmBase& w, int kv, int off, int count,
                                          int lane) {
  constexpr int IPT = TileRegs<M, RVQ, KS>::IPT;
  // tiled codes: tile off/32 starts at byte off * M of the head's stream
  const uint32_t lo = (uint32_t)(off * M) + (uint32_t)(lane * IPT);
  if constexpr (IPT == 8) {
    const uint64_t a = gload<uint64_t>(w.pq[kv], lo);
    r.pq[0] = (uint32_t)a;
    r.pq[1] = (uint32_t)(a >> 32);
    if constexpr (RVQ) {
      const uint64_t c = gload<uint64_t>(w.rvq[kv], lo);
      r.rvq[0] = (uint32_t)c;
      r.rvq[1] = (uint32_t)(c >> 32);
    }
  } else {
    r.pq[0] = gload<uint32_t>(w.pq[kv], lo);
    if constexpr (RVQ) r.rvq[0] = gload<uint32_t>(w.rvq[kv], lo);
  }
  if constexpr (KS > 0) {
    static_assert(KS == 4, "fused kernel carries 4 sparse entries");
    const int t = min(lane & (kTile - 1), count - 1);  // rows past count re-read the last row
    const uint32_t e0 = (uint32_t)((off + t) * KS + (lane >> 5) * 2);
    r.sidx = gload<uint16_t>(w.si[kv], e0);
    r.sval = gload<uint32_t>(w.sv[kv], e0 * 2);
  }
}

// Rows [16u, 16u+16) of one exact (hot) tile, this lane's two 16-byte units:
// rows [off, off+count) of hot[...][D] (rows past count re-read the last valid
// row and are zeroed when stored).  Hot tokens from app_first on are the
// launch's appended tokens, read from the caller's rows app + j*app_ld (j =
// token - app_first) instead of the hot buffers.  A tile's four halves (K and
// V) are loaded together, so that it waits for one memory round trip.
__device__ __forceinline__ void load_hot_half(uint4 (&v)[2], const TileSrc& src, const uint16_t* __restrict__ hot,
                                              int lane, int u, const uint16_t* __restrict__ app, int app_first,
                                              int64_t app_ld) {
  const int u16 = lane & 7;  // 16-byte unit of the row
#pragma unroll
  for (int k2 = 0; k2 < 2; ++k2) {
    const int row = src.off + min(16 * u + (lane >> 3) + 8 * k2, src.count - 1);
    const uint16_t* a = row >= app_first ? app + (int64_t)(row - app_first) * app_ld : hot + (int64_t)row * kD;
    v[k2] = *reinterpret_cast<const uint4*>(a + u16 * 8);
  }
}
// Store a loaded half into the wave's half-tile buffer (rows past count -> 0).
__device__ __forceinline__ void store_hot_half(uint8_t* __restrict__ lds, int tbase, const TileSrc& src,
                                               const uint4 (&v)[2], int lane, int u) {
  const int u16 = lane & 7;
#pragma unroll
  for (int k2 = 0; k2 < 2; ++k2) {
    const int r = (lane >> 3) + 8 * k2;  // buffer row
    const uint4 w = 16 * u + r >= src.count ? make_uint4(0, 0, 0, 0) : v[k2];
    *reinterpret_cast<uint4*>(lds + tbase + r * 128 + ((u16 ^ row_swz(r)) << 4)) = w;
  }
}

// Codebook entries gathered for one half (16 tokens) of a K^ or V^ tile, held
// in registers until they are summed and stored: the gathers are issued one
// pipeline step ahead of their use.
template <int M, bool RVQ>
struct RawHalf {
  static constexpr int N = M == 16 ? 4 : 2;  // gathers per lane and stream
  typedef typename std::conditional<M == 16, uint2, uint4>::type E;
  E a[N];
  E b[RVQ ? N : 1];
};

// Gather half u of one tile's codebook entries.  M = 16: lane (j, m) =
// (lane / 16, lane % 16) reads the 8-byte entry of subspace m for tokens 4i + j
// (i = 4u .. 4u+3); M = 8: lane (lane / 8, lane % 8) reads 16-byte entries for
// tokens 8i + j (i = 2u, 2u+1).  One LDS pass serves two adjacent j, which
// share subspace slots; lanes with odd j therefore read their RVQ entry first
// (slot half lc1 = +128) and their PQ entry second (lc2), so each pass covers
// all 64 banks (fp16 addition commutes, the sum is the same).  Without an RVQ
// stage the upper slot half holds a copy of the PQ table for the odd lanes.
template <int M, bool RVQ, int KS>
__device__ __forceinline__ void gather_half(const uint8_t* __restrict__ lds, const TileRegs<M, RVQ, KS>& regs, int u,
                                            uint32_t lc1, uint32_t lc2, bool odd, RawHalf<M, RVQ>& raw) {
  using E = typename RawHalf<M, RVQ>::E;
  constexpr int N = RawHalf<M, RVQ>::N;
#pragma unroll
  for (int k = 0; k < N; ++k) {
    const int i = N * u + k;  // gather group in the tile
    const uint32_t pw = regs.pq[i >> 2];
    uint32_t wa = pw, wb = 0;
    if constexpr (RVQ) {
      const uint32_t rw = regs.rvq[i >> 2];
      wa = odd ? rw : pw;
      wb = odd ? pw : rw;
    }
    raw.a[k] = *reinterpret_cast<const E*>(lds + entry_addr(wa, lc1, i & 3));
    if constexpr (RVQ) raw.b[k] = *reinterpret_cast<const E*>(lds + entry_addr(wb, lc2, i & 3));
  }
}

// K codes of one tile for the score-table path (rfsn_pack_score_codes
// layout): the lane's token row r = tokr (tokens 16u + tokr of the halves,
// the score layout's row order) and code block beta: one 8-byte load per code
// array gives bytes [4 beta, 4 beta + 4) of both halves' rows (u = 0 low word),
// and one load each gives sparse entry kg = lane >> 4 of both tokens (index
// bytes, delta halves; u = 0 low).
struct LutRegs {
  uint2 pq;
  uint2 rvq;
  uint32_t sidx;
  uint32_t sval;
};

template <int KS>
__device__ __forceinline__ void load_tile_lut(LutRegs& r, const WarmBase& w, int off, int tokr, uint32_t blk8,
                                              int kg) {
  // tile off / 32 of the head's block: 512 code bytes per array
  const uint32_t co = (uint32_t)off * 16u + (uint32_t)tokr * 32u + blk8;
  const uint64_t a = gload<uint64_t>(w.pq[0], co), c = gload<uint64_t>(w.rvq[0], co);
  r.pq = make_uint2((uint32_t)a, (uint32_t)(a >> 32));
  r.rvq = make_uint2((uint32_t)c, (uint32_t)(c >> 32));
  if constexpr (KS > 0) {
    // rows past count lie inside the tile (codes are allocated in whole
    // tiles) and their scores are masked before the exponential
    const uint32_t e = (uint32_t)off * (uint32_t)KS + (uint32_t)(tokr * 2 * KS + 2 * kg);
    r.sidx = gload<uint16_t>(w.si[0], e);
    r.sval = gload<uint32_t>(w.sv[0], e * 2);
  }
}

// K codes of one tile for the exact pass over score-table rows: the registers
// load_tile gives the codebook path (lane (j, m) = (lane / 16, lane % 16);
// byte i of its 8 bytes per code array = subspace m of token 4i + j), read
// from the rfsn_pack_score_codes rows.  Token 4i + j is row r = 4(i & 3) + j
// of half u = i >> 2, and its subspace m sits at byte (m & 3) ^ (i & 3) of the
// row's word 2(m >> 2) + u, so one 8-byte load per a = i & 3 brings the bytes
// of tokens a and a + 4 (low and high word) and v_perm_b32 picks them: sel01
// and sel23 take byte (m & 3) ^ a of words a = 0, 1 and 2, 3.  Odd tokens keep
// their RVQ code in the PQ array, and an odd lane's first gather reads its
// RVQ slot anyway, so the codes go to the gathers unswapped.  The sparse
// entries 2 (lane >> 5), +1 of token lane & 31 (row r, half u) sit at
// positions 8r + 4 (lane >> 5) + {u, 2 + u} of the tile's 128 (k = 4): the
// index bytes come from the shared index array, the values from the
// corrected-coordinate plane kplane bytes after the score deltas.
template <int KS>
__device__ __forceinline__ void load_tile_rows_exact(TileRegs<16, true, KS>& r, const WarmBase& w, int off,
                                                     int count, int lane, uint32_t sel01, uint32_t sel23) {
  const uint32_t co = (uint32_t)off * 16u + 32u * (uint32_t)(lane >> 4) + 8u * (uint32_t)((lane & 15) >> 2);
  uint32_t a[2][4][2];  // [array][i & 3][word]
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const uint64_t x = gload<uint64_t>(w.pq[0], co + 128u * k), y = gload<uint64_t>(w.rvq[0], co + 128u * k);
    a[0][k][0] = (uint32_t)x;
    a[0][k][1] = (uint32_t)(x >> 32);
    a[1][k][0] = (uint32_t)y;
    a[1][k][1] = (uint32_t)(y >> 32);
  }
#pragma unroll
  for (int s = 0; s < 2; ++s) {
#pragma unroll
    for (int wd = 0; wd < 2; ++wd) {
      const uint32_t x01 = __builtin_amdgcn_perm(a[s][1][wd], a[s][0][wd], sel01);
      const uint32_t x23 = __builtin_amdgcn_perm(a[s][3][wd], a[s][2][wd], sel23);
      const uint32_t word = __builtin_amdgcn_perm(x23, x01, 0x05040100u);
      if (s == 0) r.pq[wd] = word;
      else r.rvq[wd] = word;
    }
  }
  if constexpr (KS > 0) {
    static_assert(KS == 4, "fused kernel carries 4 sparse entries");
    const int t = min(lane & (kTile - 1), count - 1);
    const uint32_t u = (uint32_t)t >> 4;
    const uint32_t e = (uint32_t)off * KS + 8u * (uint32_t)(t & 15) + 4u * (uint32_t)(lane >> 5);
    const uint32_t ib = gload<uint32_t>(w.si[0], e);
    r.sidx = __builtin_amdgcn_perm(ib, ib, u ? 0x0C0C0301u : 0x0C0C0200u);
    const uint64_t vb = gload<uint64_t>(w.sv[0], w.kplane + 2u * e);
    r.sval = __builtin_amdgcn_perm((uint32_t)(vb >> 32), (uint32_t)vb, u ? 0x07060302u : 0x05040100u);
  }
}

// Gather the 8 score-table entries of half u: for k = 0..3 the entries of
// code byte k of the lane's PQ-array word and of its RVQ-array word.  The
// row layout permutes and swaps the codes so that byte k of a word is the
// same subspace slot for every token of the lane: lca / lcb hold those slot
// offsets (32 beta + 8 (k ^ ((t >> 2) & 3)) + stage * 128) in byte k, and one
// v_perm_b32 builds code * 256 + offset.  Per LDS pass the 32 lanes read 32
// distinct slots (all 64 banks).
// e[2k] (PQ-array byte k) and e[2k + 1] (RVQ-array byte k) form the A
// operand of score MFMA k.
struct LutHalf {
  uint4 e[4];
};
__device__ __forceinline__ void lut_gather(const uint8_t* __restrict__ lds, const LutRegs& r, int u, uint32_t lca,
                                           uint32_t lcb, LutHalf& raw) {
  const uint32_t wp = u ? r.pq.y : r.pq.x, wr = u ? r.rvq.y : r.rvq.x;
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const uint32_t sel = 0x0C0C0000u | ((uint32_t)k << 8) | (4u + (uint32_t)k);
    const uint2 a = *reinterpret_cast<const uint2*>(lds + __builtin_amdgcn_perm(lca, wp, sel));
    const uint2 b = *reinterpret_cast<const uint2*>(lds + __builtin_amdgcn_perm(lcb, wr, sel));
    raw.e[k] = make_uint4(a.x, a.y, b.x, b.y);
  }
}

// Sparse operand of half u for a 16x16x16 MFMA: fp16(q_j[idx] * delta) for
// heads j = 0..3 at k = 4kg + j (entry kg of the lane's token).  Lane l holds
// (q_0[l], q_1[l]) in qc0 and (q_2[l], q_3[l]) in qc1; ds_bpermute reads them
// from lane idx.
template <int KS>
__device__ __forceinline__ half4_t lut_sparse(const LutRegs& r, int u, uint32_t qc0, uint32_t qc1) {
  if constexpr (KS > 0) {
    const int a = (int)(((r.sidx >> (8 * u)) & 63u) << 2);
    const half2_t q01 = __builtin_bit_cast(half2_t, (uint32_t)__builtin_amdgcn_ds_bpermute(a, (int)qc0));
    const half2_t q23 = __builtin_bit_cast(half2_t, (uint32_t)__builtin_amdgcn_ds_bpermute(a, (int)qc1));
    const _Float16 dv = __builtin_bit_cast(_Float16, (uint16_t)(r.sval >> (16 * u)));
    const half2_t dd = {dv, dv};
    const half2_t p01 = q01 * dd, p23 = q23 * dd;  // v_pk_mul_f16
    return half4_t{p01[0], p01[1], p23[0], p23[1]};
  } else {
    return half4_t{};
  }
}

// Scores of both halves of a tile from their gathered score-table entries:
// MFMA k of a half sums e[k] (k = (slot, head) pairs), B selects head k % 4
// into the replicated score columns, and a 16x16x16 MFMA adds the sparse
// operand (B = the first 4 rows of the same selection).  The two halves'
// accumulation chains are interleaved, so that consecutive MFMAs are
// independent.
template <int KS>
__device__ __forceinline__ void lut_mfma2(const LutHalf& h0, const LutHalf& h1, const half4_t& sp0,
                                          const half4_t& sp1, const half8_t& bsel, float4_t& c0, float4_t& c1) {
  c0 = float4_t{0.f, 0.f, 0.f, 0.f};
  c1 = float4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    c0 = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(half8_t, h0.e[k]), bsel, c0, 0, 0, 0);
    c1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(half8_t, h1.e[k]), bsel, c1, 0, 0, 0);
  }
  if constexpr (KS > 0) {
    const half4_t b4 = {bsel[0], bsel[1], bsel[2], bsel[3]};
    c0 = __builtin_amdgcn_mfma_f32_16x16x16f16(sp0, b4, c0, 0, 0, 0);
    c1 = __builtin_amdgcn_mfma_f32_16x16x16f16(sp1, b4, c1, 0, 0, 0);
  }
}

// The sparse stage of half u: the segment carries the corrected coordinates
// fp16(X[idx] + val), stored over the reconstructed ones by the lanes of
// this half's tokens (two entries each, addresses from sparse_addrs).  The
// indices of one token are distinct, so the two lanes of a token never
// collide; rows past count repeat the last row's entries and get zero weight.
template <int M, bool RVQ, int KS>
__device__ __forceinline__ void sparse_stage(uint8_t* __restrict__ lds, const TileRegs<M, RVQ, KS>& regs, int u,
                                             const uint32_t (&saddr)[2], bool shalf) {
  if constexpr (KS > 0) {
    if (shalf == (u != 0)) {
#pragma unroll
      for (int e = 0; e < 2; ++e) *reinterpret_cast<uint16_t*>(lds + saddr[e]) = (uint16_t)(regs.sval >> (16 * e));
    }
  }
}

// Sum the gathered entries of half u (fp16(base + rvq), quantization.py:
// 317-319), store them to the wave's buffer, then run the sparse stage over
// them.  waddr holds the lane's LDS store addresses for the row patterns of
// consecutive gathers (4 for M = 16, 2 for M = 8).  A wave's LDS operations
// execute in issue order, so no wait separates these stores from earlier
// reads of the buffer or later reads of these values.
template <int M, bool RVQ, int KS>
__device__ __forceinline__ void store_half(uint8_t* __restrict__ lds, const TileRegs<M, RVQ, KS>& regs,
                                           const RawHalf<M, RVQ>& raw, int u, const int (&waddr)[4],
                                           const uint32_t (&saddr)[2], bool shalf) {
  if constexpr (M == 16) {
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      uint2 e = raw.a[k];
      if constexpr (RVQ) {
        e.x = add_h2(e.x, raw.b[k].x);
        e.y = add_h2(e.y, raw.b[k].y);
      }
      *reinterpret_cast<uint2*>(lds + waddr[k] + k * 512) = e;
    }
  } else {
#pragma unroll
    for (int k = 0; k < 2; ++k) {
      uint4 e = raw.a[k];
      if constexpr (RVQ) {
        e.x = add_h2(e.x, raw.b[k].x);
        e.y = add_h2(e.y, raw.b[k].y);
        e.z = add_h2(e.z, raw.b[k].z);
        e.w = add_h2(e.w, raw.b[k].w);
      }
      *reinterpret_cast<uint4*>(lds + waddr[k] + k * 1024) = e;
    }
  }
  sparse_stage<M, RVQ, KS>(lds, regs, u, saddr, shalf);
}

// M = 16 without a sparse stage: the gathered entries of half u are already
// the P.V MFMA's A operands (lane (j, m) holds subspace m of token
// 16u + 4k + j for gather k, the 16x16x32 A layout of MFMA k/2), so V^ skips
// the buffer: av[j] = fp16(base + rvq) of gathers 2j, 2j + 1.
template <bool RVQ>
__device__ __forceinline__ void direct_half(const RawHalf<16, RVQ>& raw, half8_t (&av)[2]) {
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    uint2 lo = raw.a[2 * j], hi = raw.a[2 * j + 1];
    if constexpr (RVQ) {
      lo = make_uint2(add_h2(lo.x, raw.b[2 * j].x), add_h2(lo.y, raw.b[2 * j].y));
      hi = make_uint2(add_h2(hi.x, raw.b[2 * j + 1].x), add_h2(hi.y, raw.b[2 * j + 1].y));
    }
    av[j] = __builtin_bit_cast(half8_t, make_uint4(lo.x, lo.y, hi.x, hi.y));
  }
}

// M = 16 with a sparse stage: V^ halves pass through the buffer lane-major
// (the gather lane already holds the P.V A operands, only the sparse stage
// needs the buffer): lane l's slots k = 0..3 (tokens 16u + 4k + l/16 of
// subspace l%16) sit at byte (k >> 1) * 1024 + 16 l + 8 (k & 1), so a lane
// stores and reloads each 16x16x32 A operand with one 16-byte access (64
// lanes x 16 B contiguous: no bank conflicts).
__device__ __forceinline__ void store_lanes(uint8_t* __restrict__ lds, int tbase, int lane, const half8_t (&av)[2]) {
#pragma unroll
  for (int j = 0; j < 2; ++j) *reinterpret_cast<half8_t*>(lds + tbase + j * 1024 + lane * 16) = av[j];
}
__device__ __forceinline__ void load_lanes(const uint8_t* __restrict__ lds, int tbase, int lane, half8_t (&av)[2]) {
  // A lane reloads the bytes it stored, which other lanes' sparse stores may
  // have changed: keep the compiler from forwarding the stored registers
  // (the wave's LDS operations execute in order, so no wait is needed).
  asm volatile("" ::: "memory");
#pragma unroll
  for (int j = 0; j < 2; ++j) av[j] = *reinterpret_cast<const half8_t*>(lds + tbase + j * 1024 + lane * 16);
}
// Sparse entry addresses in that layout: token t' = 4k + g of the half and
// coordinate idx land in lane 16 g + idx / 4, slot k, so the byte is
//   vtok(t') | 16 (idx >> 2) | 2 (idx & 3),
//   vtok(t') = buffer + 1024 (t' >> 3) + 256 (t' & 3) + 8 ((t' >> 2) & 1)
// (disjoint bits).  Both entries of the lane at once from the two index bytes.
template <int M, bool RVQ, int KS>
__device__ __forceinline__ void sparse_addrs_lanes(const TileRegs<M, RVQ, KS>& regs, uint32_t vtok, uint32_t (&sa)[2]) {
  const uint32_t x = regs.sidx;  // two index bytes
  const uint32_t y = ((x & 0x3C3Cu) << 2) | ((x & 0x0303u) << 1);
  sa[0] = vtok | (y & 0xFFu);
  sa[1] = vtok | (y >> 8);
}

// LDS addresses of the lane's two sparse entries in the half-tile buffer.
// Coordinate idx of buffer row r sits at byte
//   128 r + 16 ((idx >> 3) ^ row_swz(r)) + 2 (idx & 7) = sbase ^ (2 idx)
// with sbase = buffer base + 128 r + 16 row_swz(r): the index bits land below
// the row bits, and bits 4-6 of 2 idx XOR into the unit swizzle.
template <int M, bool RVQ, int KS>
__device__ __forceinline__ void sparse_addrs(const TileRegs<M, RVQ, KS>& regs, uint32_t sbase, uint32_t (&sa)[2]) {
  sa[0] = sbase ^ ((regs.sidx << 1) & 0x7Eu);
  sa[1] = sbase ^ ((regs.sidx >> 7) & 0x7Eu);
}

// Wave issue priority 0..3 (s_setprio takes an immediate; p is wave-uniform).
__device__ __forceinline__ void set_prio(int p) {
  switch (p) {
    case 0: __builtin_amdgcn_s_setprio(0); break;
    case 1: __builtin_amdgcn_s_setprio(1); break;
    case 2: __builtin_amdgcn_s_setprio(2); break;
    default: __builtin_amdgcn_s_setprio(3); break;
  }
}

// K paths of the kernel body.
enum KMode : int {
  kCodebook = 0,  // K^ rebuilt from the codebooks (k_layout 0)
  kTables = 1,    // score tables (k_layout 1)
  kExactRows = 2  // K^ rebuilt from the codebooks, codes read from the score-table rows (k_layout 1)
};

// XCD-aware block mapping: consecutive hardware block ids go to different
// XCDs; give each XCD a contiguous range of (sequence, head, split) units so
// that one sequence's codebooks are fetched into one L2.
__device__ __forceinline__ void block_unit(int blocks_total, int splits, int kv_heads, int& b, int& h, int& split) {
  const int L = blockIdx.x;
  const int per = blocks_total / 8, rem = blocks_total % 8;
  const int xcd = L % 8, k = L / 8;
  const int vid = xcd * per + min(xcd, rem) + k;
  split = vid % splits;
  h = (vid / splits) % kv_heads;
  b = vid / (splits * kv_heads);
}

// One block's attention over its split: stage, stream the tiles, combine and
// write the output (or the split partial).  With score tables and a drift
// guard it returns true, without writing, when some head's drift estimate
// exceeds the tolerance: the caller then runs the kExactRows body.  The
// estimate needs sum_t p_t^2, which the table body accumulates beside the
// softmax denominator.
template <int M, bool RVQ, int KS, int NHG, int KM>
__device__ __forceinline__ bool attn_body(const rfsn_fused_params& p, int splits, int tiles_per_split,
                                          int blocks_total, uint8_t* __restrict__ lds) {
  constexpr bool LUT = KM == kTables;
  constexpr bool SX = KM == kExactRows;
  // codes in flight per wave: the exact pass reads K's codes from the
  // score-table rows (4 loads per array for a tile) and keeps one tile ahead,
  // which holds its loop within the registers a call leaves it
  constexpr int kDep = SX ? 1 : kDepth;
  static_assert(KM == kCodebook || (M == 16 && RVQ && NHG == 1),
                "score-table rows: 16 + 16 subspaces, <= 4 heads per KV head");
  constexpr int kWaves = BlockShape<NHG>::W;
  constexpr int kThreads = BlockShape<NHG>::T;
  int b, h, split;
  block_unit(blocks_total, splits, p.kv_heads, b, h, split);

  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
  set_prio(3);  // lowered with the wave's progress through its encoded tiles
  const int G = p.q_heads / p.kv_heads;
  const int C = p.fmt.pq_centroids, Cr = RVQ ? p.fmt.rvq_centroids : 0;
  constexpr int d = kD / M;

  const int tbase = kTilesBase + wave * kBufBytes;  // this wave's half-tile buffer (LDS byte address)
  const cseg segs = (cseg)(p.segments + (int64_t)b * p.max_segments);
  // a count beyond the table's row would read the next sequence's segments
  const int nseg = p.num_segments ? min(max(p.num_segments[b], 0), p.max_segments) : 0;

  const int g = lane >> 4;   // k-group of the 16x16 MFMA operands
  const int n = lane & 15;   // column (B, D) / row (A)
  // score-table lanes: row n holds token row tokr of each half (tokens
  // t = 16u + tokr, so (t >> 2) & 3 = n & 3 and t & 1 = (n >> 2) & 1), k-group
  // g the code block beta (4 subspaces of both stages), chosen so that the 8
  // lanes of a block in one LDS pass differ in (n & 3, (n >> 2) & 1) and read
  // 8 distinct slots
  const int tokr = 4 * (n & 3) + (n >> 2);
  const int beta = (g + 2 * (n >> 3)) & 3;
  const uint32_t blk8 = 8u * (uint32_t)beta;
  // exact pass over score-table rows: v_perm_b32 selectors taking byte
  // (m & 3) ^ a of words a = 0, 1 (sel01) and 2, 3 (sel23), m = lane % 16
  const uint32_t m3 = (uint32_t)lane & 3u;
  const uint32_t sel01 = 0x0C0C0000u | m3 | ((4u + (m3 ^ 1u)) << 8);
  const uint32_t sel23 = 0x0C0C0000u | (m3 ^ 2u) | ((4u + (m3 ^ 3u)) << 8);

  const int hot_tiles = (p.hot_len + kTile - 1) / kTile;
  WarmBase w0 = {};
  if (nseg > 0) w0 = warm_base<M, RVQ, KS, SX>(segs, h, p.kv_heads);
  const int seg0_tiles = nseg > 0 ? (w0.len + kTile - 1) / kTile : 0;
  int total_tiles = hot_tiles + seg0_tiles;
  const cmap tmap = p.tile_map ? (cmap)(p.tile_map + (int64_t)b * p.tile_map_stride) : nullptr;
  total_tiles += tmap ? min(max(p.tile_map_count[b], 0), (int)p.tile_map_stride) : tail_tiles(segs, nseg);
  const int t_begin = split * tiles_per_split;
  const int t_end = min(total_tiles, t_begin + tiles_per_split);
  const uint16_t* hotk = (const uint16_t*)p.hot_k + (int64_t)b * p.hot_seq_stride + (int64_t)h * p.hot_cap * kD;
  const uint16_t* hotv = (const uint16_t*)p.hot_v + (int64_t)b * p.hot_seq_stride + (int64_t)h * p.hot_cap * kD;
  // the launch's appended tokens: hot tokens app_first .. hot_len - 1
  const int app_first = p.hot_len - p.app_count;
  const uint16_t* appk = p.app_count ? (const uint16_t*)p.app_k + (int64_t)h * kD : hotk;
  const uint16_t* appv = p.app_count ? (const uint16_t*)p.app_v + (int64_t)h * kD : hotv;


  using Regs = TileRegs<M, RVQ, KS>;
  using KRegs = typename std::conditional<LUT, LutRegs, Regs>::type;
  // kDepth tiles in flight per wave: slot s holds tile tt + s*kWaves.  Only
  // encoded tiles go through slots (tt >= hot_tiles); a slot past the split
  // is idle and re-reads the split's last tile, which is encoded.
  TileSrc srcs[kDep];
  KRegs kr[kDep];
  Regs vr[kDep];
  auto load_k = [&](KRegs& rk, const WarmBase& w, int off, int count) __attribute__((always_inline)) {
    if constexpr (LUT) load_tile_lut<KS>(rk, w, off, tokr, blk8, g);
    else if constexpr (SX) load_tile_rows_exact<KS>(rk, w, off, count, lane, sel01, sel23);
    else load_tile<M, RVQ, KS>(rk, w, 0, off, count, lane);
  };
  auto fetch = [&](TileSrc& s, KRegs& rk, Regs& rv, int tt) {
    const int r = min(tt, t_end - 1) - hot_tiles;
    if (r < seg0_tiles) {  // uniform; segment 0 from registers
      s.kind = 1;
      s.seg = 0;
      s.off = r * kTile;
      s.count = min(kTile, w0.len - s.off);
      s.pos0 = w0.pos0 + s.off;
      load_k(rk, w0, s.off, s.count);
      load_tile<M, RVQ, KS>(rv, w0, 1, s.off, s.count, lane);
    } else {
      s = tmap ? map_tile(segs, nseg, tmap, r - seg0_tiles) : walk_segments(segs, nseg, r - seg0_tiles);
      const WarmBase w = warm_base<M, RVQ, KS, SX>(segs + s.seg, h, p.kv_heads);
      load_k(rk, w, s.off, s.count);
      load_tile<M, RVQ, KS>(rv, w, 1, s.off, s.count, lane);
    }
    if (tt >= t_end) s.kind = -1;
  };
  const int seg_begin = max(t_begin, hot_tiles);

  // ---- stage this sequence's codebooks: HBM [m][e][d] -> LDS [table][e][PQ m | RVQ m][d]
  // (without an RVQ stage the upper slot half holds a second copy of the PQ table)
  {
    const uint16_t* kp = (const uint16_t*)p.k_pq_cb + (int64_t)b * p.pq_cb_stride;
    const uint16_t* vp = (const uint16_t*)p.v_pq_cb + (int64_t)b * p.pq_cb_stride;
    const uint16_t* cbp[4] = {kp, vp, RVQ ? (const uint16_t*)p.k_rvq_cb + (int64_t)b * p.rvq_cb_stride : kp,
                              RVQ ? (const uint16_t*)p.v_rvq_cb + (int64_t)b * p.rvq_cb_stride : vp};
    // every load of this thread is issued before its first LDS store, so the
    // block waits for one memory round trip rather than one per entry
    using Vec = typename std::conditional<d == 4, uint2, uint4>::type;
    constexpr int kIters = (M * 256 + kThreads - 1) / kThreads;
    constexpr int kTabVecs = kTableBytes / 16;                      // uint4 units of one table
    constexpr int kTabIters = (kTabVecs + kThreads - 1) / kThreads;
    const bool pre = p.v_tab != nullptr;  // uniform: entry-major tables from the host
    Vec v[4][kIters];
    uint4 tv[2][kTabIters];
    if (pre) {
      // contiguous copies of the K (codebook path) and V tables
#pragma unroll
      for (int c = 0; c < 2; ++c) {
        if (LUT && c == 0) continue;  // the K tables become score tables below
        const uint4* src = reinterpret_cast<const uint4*>((const uint8_t*)(c ? p.v_tab : p.k_tab) + (int64_t)b * p.tab_stride);
#pragma unroll
        for (int i = 0; i < kTabIters; ++i) {
          const int idx = threadIdx.x + i * kThreads;
          tv[c][i] = idx < kTabVecs ? src[idx] : make_uint4(0u, 0u, 0u, 0u);
        }
      }
    } else {
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        if (LUT && (c & 1) == 0) continue;  // the K tables become score tables below
        const int n = (c < 2 || !RVQ) ? C : Cr;
#pragma unroll
        for (int i = 0; i < kIters; ++i) {
          const int idx = threadIdx.x + i * kThreads;
          const int e = idx / M, m = idx % M;  // consecutive lanes store consecutive slots of one entry
          v[c][i] = Vec{};
          if (idx < M * 256 && e < n) v[c][i] = *reinterpret_cast<const Vec*>(cbp[c] + ((int64_t)m * n + e) * d);
        }
      }
    }
    // Every wave requests the codes of its first encoded tiles now, after the
    // codebook loads: HBM streams while the set-up runs, and the stores below
    // wait only for the (L2-resident) codebook loads issued before them.
    if (seg_begin < t_end) {  // uniform: the split has encoded tiles
#pragma unroll
      for (int s = 0; s < kDep; ++s) fetch(srcs[s], kr[s], vr[s], seg_begin + wave + s * kWaves);
    }
    if (pre) {
#pragma unroll
      for (int c = 0; c < 2; ++c) {
        if (LUT && c == 0) continue;
        uint4* dst = reinterpret_cast<uint4*>(lds + c * kTableBytes);
#pragma unroll
        for (int i = 0; i < kTabIters; ++i) {
          const int idx = threadIdx.x + i * kThreads;
          if (idx < kTabVecs) dst[idx] = tv[c][i];
        }
      }
    } else {
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        if (LUT && (c & 1) == 0) continue;
        uint8_t* dst = lds + (c & 1) * kTableBytes + (c >> 1) * kRvqSlot;
#pragma unroll
        for (int i = 0; i < kIters; ++i) {
          const int idx = threadIdx.x + i * kThreads;
          const int e = idx / M, m = idx % M;
          if (idx < M * 256) *reinterpret_cast<Vec*>(dst + e * kEntryBytes + m * d * 2) = v[c][i];
        }
      }
    }
  }
  if constexpr (LUT) {
    // score table T[c][s][j] = fp16(q_j . centroid c of slot s) in fp32
    // (slot s < 16: PQ subspace s, else RVQ subspace s - 16; heads j >= G
    // give 0, codes past the codebook 0).  Thread: slot tid % 32, codes
    // tid / 32 + kRows * i; every load is issued before the first store.
    constexpr int kRows = kThreads / 32;
    constexpr int kPasses = 256 / kRows;
    static_assert(256 % kRows == 0, "score table passes");
    const int s = threadIdx.x & 31, m = s & 15;
    const bool rv = s >= 16;
    const uint16_t* cb = rv ? (const uint16_t*)p.k_rvq_cb + (int64_t)b * p.rvq_cb_stride
                            : (const uint16_t*)p.k_pq_cb + (int64_t)b * p.pq_cb_stride;
    const int nc = rv ? Cr : C;
    uint2 qw[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const uint16_t* qrow = (const uint16_t*)p.q + ((int64_t)b * p.q_heads + h * G + min(j, G - 1)) * kD;
      qw[j] = j < G ? *reinterpret_cast<const uint2*>(qrow + 4 * m) : make_uint2(0, 0);
    }
    uint2 e[kPasses];
    const uint8_t* ktab = p.k_tab ? (const uint8_t*)p.k_tab + (int64_t)b * p.tab_stride : nullptr;
#pragma unroll
    for (int i = 0; i < kPasses; ++i) {
      const int c = (threadIdx.x >> 5) + kRows * i;
      if (ktab)  // entry-major: consecutive lanes read consecutive slots of one entry
        e[i] = *reinterpret_cast<const uint2*>(ktab + c * kEntryBytes + s * 8);
      else
        e[i] = c < nc ? *reinterpret_cast<const uint2*>(cb + ((int64_t)m * nc + c) * 4) : make_uint2(0, 0);
    }
    float qf[4][4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const half4_t hq = __builtin_bit_cast(half4_t, qw[j]);
#pragma unroll
      for (int t = 0; t < 4; ++t) qf[j][t] = (float)hq[t];
    }
#pragma unroll
    for (int i = 0; i < kPasses; ++i) {
      const int c = (threadIdx.x >> 5) + kRows * i;
      const half4_t x = __builtin_bit_cast(half4_t, e[i]);
      half4_t o;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        float a = qf[j][0] * (float)x[0];
        a = fmaf(qf[j][1], (float)x[1], a);
        a = fmaf(qf[j][2], (float)x[2], a);
        a = fmaf(qf[j][3], (float)x[3], a);
        o[j] = (_Float16)a;
      }
      *reinterpret_cast<uint2*>(lds + c * kEntryBytes + s * 8) = __builtin_bit_cast(uint2, o);
    }
  }

  // ---- lane constants
  // gather lane (jg, mg) and its codebook slot; store offsets for the row
  // patterns of consecutive gathers
  const int jg = lane / M, mg = lane % M;
  const bool odd = (jg & 1) != 0;
  const uint32_t slot = (uint32_t)(mg * d * 2);
  const uint32_t lc1_k = slot | (odd ? kRvqSlot : 0u), lc2_k = slot | (odd ? 0u : kRvqSlot);
  const uint32_t lc1_v = lc1_k | (1u << 16), lc2_v = lc2_k | (1u << 16);
  // Store addresses of gather k of a half: buffer row 4k + j (M = 16), with
  // row_swz = 2k + (j>>1); row 8k + j (M = 8), with row_swz = 4k + (j>>1).
  int waddr[4];
  if constexpr (M == 16) {
#pragma unroll
    for (int a = 0; a < 4; ++a)
      waddr[a] = tbase + jg * 128 + ((((mg >> 1) ^ (2 * a + (jg >> 1))) << 4) | ((mg & 1) << 3));
  } else {
#pragma unroll
    for (int a = 0; a < 2; ++a) waddr[a] = tbase + jg * 128 + ((mg ^ (4 * a + (jg >> 1))) << 4);
    waddr[2] = waddr[0];
    waddr[3] = waddr[1];
  }
  // sparse stores: token t = lane & 31 lives in half t >> 4
  const bool shalf = (lane & 16) != 0;
  const uint32_t sbase = (uint32_t)(tbase + (lane & 15) * 128 + (row_swz(lane & 15) << 4));
  const int tq = lane & 15;  // the sparse lane's token within its half
  const uint32_t vtok = (uint32_t)(tbase + 1024 * (tq >> 3) + 256 * (tq & 3) + 8 * ((tq >> 2) & 1));
  // V operand reads of P.V MFMA k of a half: buffer row 4k + g, chunk n (the M = 16 store pattern)
  int paddr[4];
#pragma unroll
  for (int a = 0; a < 4; ++a)
    paddr[a] = tbase + g * 128 + ((((n >> 1) ^ (2 * a + (g >> 1))) << 4) | ((n & 1) << 3));
  // score operand reads: buffer row 4(n&3) + (n>>2) (row_swz = 2(n&3) + (n>>3)), 16-byte unit 4c + g
  int raddr[2];
  {
    const int f = 2 * (n & 3) + (n >> 3);
#pragma unroll
    for (int c = 0; c < 2; ++c) raddr[c] = tbase + (4 * (n & 3) + (n >> 2)) * 128 + (((4 * c + g) ^ f) << 4);
  }
  // B operands of P.V: the probabilities X = (p_t0, p_t1) of a token pair,
  // packed in one dword, go to coordinate ep = n & 3 of each token's half of
  // the lane's k-group: dwords 0 (t0) and 2 (t1) for ep = 0, 1, dwords 1 and
  // 3 for ep = 2, 3, in the low half for even ep and the high half for odd.
  const int ep = n & 3;
  uint32_t psel[4];
  {
    const uint32_t s0 = (ep & 1) ? 0x01000C0Cu : 0x0C0C0100u, s1 = (ep & 1) ? 0x03020C0Cu : 0x0C0C0302u;
    const bool lo = ep < 2;
    psel[0] = lo ? s0 : 0x0C0C0C0Cu;
    psel[1] = lo ? 0x0C0C0C0Cu : s0;
    psel[2] = lo ? s1 : 0x0C0C0C0Cu;
    psel[3] = lo ? 0x0C0C0C0Cu : s1;
  }
  const bool todd = ((n >> 2) & 1) != 0;
  uint32_t lca = 0, lcb = 0;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int slot8 = 32 * beta + 8 * (i ^ (n & 3));
    lca |= (uint32_t)(slot8 + (todd ? kRvqSlot : 0)) << (8 * i);
    lcb |= (uint32_t)(slot8 + (todd ? 0 : kRvqSlot)) << (8 * i);
  }
  // B operand of the score-table MFMAs: k index 8g + e carries head e & 3,
  // column n scores head n >> 2
  half8_t bsel;
#pragma unroll
  for (int e2 = 0; e2 < 8; ++e2) bsel[e2] = (_Float16)((e2 & 3) == (n >> 2) ? 1.0f : 0.0f);

  // ---- query operands and per-head state: lane column n serves head hg*4 + n/4
  half8_t qb[NHG][2];
  float bias[NHG], bias_m[NHG], m_run[NHG];
  int qpl[NHG];
  float4_t acc[NHG];
  float lsum[NHG];  // this lane's share of the softmax denominator (its tokens, its head)
  float lsq[NHG];   // and of sum p^2 (score tables: the drift estimate)
#pragma unroll
  for (int hg = 0; hg < NHG; ++hg) {
    const int hh = hg * 4 + (n >> 2);
    const bool valid = hh < G;
    const uint16_t* qrow = (const uint16_t*)p.q + ((int64_t)b * p.q_heads + h * G + (valid ? hh : 0)) * kD;
#pragma unroll
    for (int c = 0; c < 2; ++c) {
      uint4 w = valid ? *reinterpret_cast<const uint4*>(qrow + 32 * c + 8 * g) : make_uint4(0, 0, 0, 0);
      qb[hg][c] = __builtin_bit_cast(half8_t, w);
    }
    bias[hg] = valid ? 0.f : -__builtin_inff();
    bias_m[hg] = valid ? __builtin_inff() : -__builtin_inff();  // forces the first max update
    m_run[hg] = -__builtin_inff();
    qpl[hg] = (p.causal && p.qpos && valid) ? p.qpos[(int64_t)b * p.q_heads + h * G + hh] : 0x7fffffff;
    acc[hg] = float4_t{0.f, 0.f, 0.f, 0.f};
    lsum[hg] = 0.f;
    lsq[hg] = 0.f;
  }
  // smallest query position of this KV head's query heads (uniform)
  int qmin = 0x7fffffff;
  if (p.causal && p.qpos)
    for (int hh = 0; hh < G; ++hh) qmin = min(qmin, p.qpos[(int64_t)b * p.q_heads + h * G + hh]);
  const float scale_log2 = p.scale * kLog2e;
  // q columns of the score-table sparse stage: lane l holds q_j[l], j < 4
  uint32_t qc0 = 0, qc1 = 0;
  if constexpr (LUT && KS > 0) {
    uint32_t qv[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const uint16_t* qrow = (const uint16_t*)p.q + ((int64_t)b * p.q_heads + h * G + min(j, G - 1)) * kD;
      qv[j] = j < G ? (uint32_t)qrow[lane] : 0u;
    }
    qc0 = qv[0] | (qv[1] << 16);
    qc1 = qv[2] | (qv[3] << 16);
  }


  __syncthreads();

  // score operands of the half in the buffer, then the scores: lane (g, n),
  // register i of half u = token 16u + 4i + g
  // Operand reads of data other lanes stored: a compiler barrier first, so
  // that no lane's own stored registers are forwarded past the other lanes'
  // stores (the wave's LDS operations execute in order: no wait is needed).
  auto score_operands = [&](half8_t (&a)[2]) {
    asm volatile("" ::: "memory");
#pragma unroll
    for (int c = 0; c < 2; ++c) a[c] = *reinterpret_cast<const half8_t*>(lds + raddr[c]);
  };
  auto scores = [&](const half8_t (&a)[2], float4_t (&sc)[NHG][2], int u) {
#pragma unroll
    for (int hg = 0; hg < NHG; ++hg) {
      sc[hg][u] = float4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int c = 0; c < 2; ++c) sc[hg][u] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[c], qb[hg][c], sc[hg][u], 0, 0, 0);
    }
  };
  // scores of both halves from their gathered score-table entries (+ the sparse operands)
  using KHalf = typename std::conditional<LUT, LutHalf, RawHalf<M, RVQ>>::type;
  auto lut_scores = [&](const KHalf& h0, const KHalf& h1, const half4_t& sp0, const half4_t& sp1,
                        float4_t (&sc)[NHG][2]) __attribute__((always_inline)) {
    if constexpr (LUT) lut_mfma2<KS>(h0, h1, sp0, sp1, bsel, sc[0][0], sc[0][1]);
  };
  // K half u of the tile in slot ks: score-table or codebook gathers
  auto gather_k = [&](const KRegs& rk, int u, KHalf& raw) __attribute__((always_inline)) {
    if constexpr (LUT) lut_gather(lds, rk, u, lca, lcb, raw);
    else gather_half<M, RVQ, KS>(lds, rk, u, lc1_k, lc2_k, odd && !SX, raw);
  };
  // online softmax in base 2; produces the B operands of P.V (probability at
  // coordinate n & 3 of the lane's k-group)
  auto softmax = [&](const TileSrc& src, const float4_t (&sc)[NHG][2], uint32_t (&pb)[NHG][4][4]) {
    // uniform: nothing masked (a segment may start before the window, with
    // negative positions for the tokens to skip)
    const bool full = src.count == kTile && src.pos0 >= 0 && src.pos0 + kTile - 1 <= qmin;
#pragma unroll
    for (int hg = 0; hg < NHG; ++hg) {
      // masked scores -> -inf (uniform branch: partial tile or causal boundary)
      auto mask = [&](float (&v)[8]) {
        if (!full) {
#pragma unroll
          for (int r = 0; r < 8; ++r) {
            const int tok = 16 * (r >> 2) + 4 * (r & 3) + g;
            const int pos = src.pos0 + tok;
            v[r] = (tok < src.count && pos >= 0 && pos <= qpl[hg]) ? v[r] : -__builtin_inff();
          }
        }
      };
      float arg[8];
#pragma unroll
      for (int r = 0; r < 8; ++r) arg[r] = fmaf(sc[hg][r >> 2][r & 3], scale_log2, bias_m[hg]);
      mask(arg);
      // The running max only moves when some score exceeds it by more than
      // the fp16 headroom of P (any max gives the same softmax, the running
      // one only keeps exp2 in range); most tiles skip the cross-lane
      // reduction and the rescale.  The test takes a signed-integer max of
      // the float bits: values above the (positive) threshold keep their
      // order, negative ones compare below it, and no float max (which
      // quiets NaN inputs first) is needed.
      int ibits = (int)fbits(arg[0]);
#pragma unroll
      for (int r = 1; r < 8; ++r) ibits = max(ibits, (int)fbits(arg[r]));
      if (__builtin_amdgcn_ballot_w64(ibits > (int)fbits(kPScaleLog2 + kSlackLog2))) {
        float sv[8];
#pragma unroll
        for (int r = 0; r < 8; ++r) sv[r] = fmaf(sc[hg][r >> 2][r & 3], scale_log2, bias[hg]);
        mask(sv);
        float mx = fmaxf(fmaxf(fmaxf(sv[0], sv[1]), fmaxf(sv[2], sv[3])),
                         fmaxf(fmaxf(sv[4], sv[5]), fmaxf(sv[6], sv[7])));
        mx = xmax32(xmax16(mx));  // the 4 k-groups holding this head's tokens
        const float mn = fmaxf(m_run[hg], mx);
        // a head with nothing allowed yet keeps m = -inf, probabilities 0 and
        // bias_m (+inf for a real head, so its first allowed score rescales)
        const bool none = mn == -__builtin_inff();
        const float corr = none ? 1.f : __builtin_amdgcn_exp2f(m_run[hg] - mn);
        acc[hg] *= corr;
        lsum[hg] *= corr;
        if constexpr (LUT) lsq[hg] *= corr * corr;
        m_run[hg] = mn;
        // exp2 argument = score - max + 14
        const float dm = none ? 0.f : kPScaleLog2 - mn;
        bias_m[hg] = none ? bias_m[hg] : bias[hg] + dm;
#pragma unroll
        for (int r = 0; r < 8; ++r) arg[r] = sv[r] + dm;
      }
      // score registers 2q, 2q + 1 are the two tokens of P.V operand q; the
      // denominator sums the same fp16 probabilities that P.V weights
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const half2_t ph = {(_Float16)__builtin_amdgcn_exp2f(arg[2 * q]),
                            (_Float16)__builtin_amdgcn_exp2f(arg[2 * q + 1])};  // v_cvt_pk_f16_f32
        const uint32_t x = __builtin_bit_cast(uint32_t, ph);
        lsum[hg] = __builtin_amdgcn_fdot2(ph, half2_t{(_Float16)1.0f, (_Float16)1.0f}, lsum[hg], false);
        if constexpr (LUT) lsq[hg] = __builtin_amdgcn_fdot2(ph, ph, lsq[hg], false);
#pragma unroll
        for (int k = 0; k < 4; ++k) pb[hg][q][k] = __builtin_amdgcn_perm(x, x, psel[k]);
      }
    }
  };
  // P.V and the denominator over the V^ half in the buffer on MFMA 16x16x32:
  // MFMA j of half u covers tokens 16u + 8j + 4t + g (t = 0, 1), k index
  // 8g + 4t + c (coordinate c); lane (n, g) holds V^ rows of subspace n for
  // its two tokens, and the B operand the lane's probabilities of the same
  // two tokens (score registers 4u + 2j + t) on the coordinate diagonal.
  auto pv_operands = [&](half8_t (&av)[2]) {
    asm volatile("" ::: "memory");
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const uint2 lo = *reinterpret_cast<const uint2*>(lds + paddr[2 * j] + 2 * j * 512);
      const uint2 hi = *reinterpret_cast<const uint2*>(lds + paddr[2 * j + 1] + (2 * j + 1) * 512);
      av[j] = __builtin_bit_cast(half8_t, make_uint4(lo.x, lo.y, hi.x, hi.y));
    }
  };
  auto pv = [&](const half8_t (&av)[2], const uint32_t (&pb)[NHG][4][4], int u) {
#pragma unroll
    for (int j = 0; j < 2; ++j) {
#pragma unroll
      for (int hg = 0; hg < NHG; ++hg) {
        const uint32_t* b4 = pb[hg][2 * u + j];
        const half8_t bw = __builtin_bit_cast(half8_t, make_uint4(b4[0], b4[1], b4[2], b4[3]));
        acc[hg] = __builtin_amdgcn_mfma_f32_16x16x32_f16(av[j], bw, acc[hg], 0, 0, 0);
      }
    }
  };

  // Phase 1: exact (hot) tiles, loaded synchronously (a few percent of tiles).
  const int hot_end = min(t_end, hot_tiles);
  for (int tt = t_begin + wave; tt < hot_end; tt += kWaves) {
    const TileSrc src = hot_tile(p, tt);
    float4_t sc[NHG][2];
    uint32_t pb[NHG][4][4];
    half8_t a[2];
    half8_t av[2];
    uint4 hk[2][2], hv[2][2];
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      load_hot_half(hk[u], src, hotk, lane, u, appk, app_first, p.app_ld);
      load_hot_half(hv[u], src, hotv, lane, u, appv, app_first, p.app_ld);
    }
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      store_hot_half(lds, tbase, src, hk[u], lane, u);
      score_operands(a);
      scores(a, sc, u);
    }
    softmax(src, sc, pb);
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      store_hot_half(lds, tbase, src, hv[u], lane, u);
      pv_operands(av);
      pv(av, pb, u);
    }
  }

  // Phase 2: encoded tiles, kDepth tiles of codes in flight per wave, and a
  // software pipeline over the tile's LDS steps: every gather is issued one
  // step ahead of the store that consumes it (the next tile's first K^ half
  // under this tile's last P.V MFMAs).  LDS operations of a wave execute in
  // order, so the buffer is reused without waits; the compiler's counters
  // only wait for the data each step consumes.
  // With 16 subspaces V^ goes from the gather registers into P.V (through
  // the buffer lane-major only for its sparse stage); with 8 its halves pass
  // through the buffer like K^.
  if (seg_begin < t_end) {
    RawHalf<M, RVQ> ra, rb;
    KHalf ka, kb;  // K halves of the score-table path (the codebook path gathers K into ra, rb)
    if constexpr (LUT) gather_k(kr[0], 0, ka);
    else gather_k(kr[0], 0, ra);
    // Issue priority falls as a wave works through its tiles.  With equal
    // priorities a SIMD issues oldest-first: the block's youngest waves then
    // finish about a third of the loop after its oldest (measured with
    // per-wave timestamps at batch 32 x 32K), and the CU runs the tail with
    // fewer waves.  A wave that is ahead yields to the ones behind it.
    // Priority 3 - stage, stage = floor(4 * done / my_tiles) capped at 3; it
    // changes at most three times, so a tile only compares done with the
    // count at which the next stage begins.
    const int my_tiles = max((t_end - seg_begin - wave + kWaves - 1) / kWaves, 1);
    int done = 0, stage = 0;
    int next_at = (my_tiles + 3) >> 2;  // ceil(my_tiles / 4)
    for (int tt = seg_begin + wave; tt < t_end; tt += kDep * kWaves) {
#pragma unroll
      for (int s = 0; s < kDep; ++s) {
        if (srcs[s].kind >= 0) {
          if (++done >= next_at) {  // uniform
            while (stage < 3 && 4 * done >= (stage + 1) * my_tiles) ++stage;
            set_prio(3 - stage);
            next_at = stage < 3 ? ((stage + 1) * my_tiles + 3) >> 2 : 0x7fffffff;
          }
          float4_t sc[NHG][2];
          uint32_t pb[NHG][4][4];
          half8_t a[2];
          half8_t av[2];
          uint32_t sav[2] = {0, 0};
          if constexpr (KS > 0 && M != 16) sparse_addrs(vr[s], sbase, sav);
          if constexpr (LUT) {
            gather_k(kr[s], 1, kb);
            const half4_t sp0 = lut_sparse<KS>(kr[s], 0, qc0, qc1);
            const half4_t sp1 = lut_sparse<KS>(kr[s], 1, qc0, qc1);
            gather_half<M, RVQ, KS>(lds, vr[s], 0, lc1_v, lc2_v, odd, ra);
            lut_scores(ka, kb, sp0, sp1, sc);
          } else {
            uint32_t sak[2] = {0, 0};
            if constexpr (KS > 0) sparse_addrs(kr[s], sbase, sak);
            store_half<M, RVQ, KS>(lds, kr[s], ra, 0, waddr, sak, shalf);
            score_operands(a);
            gather_k(kr[s], 1, rb);
            scores(a, sc, 0);
            store_half<M, RVQ, KS>(lds, kr[s], rb, 1, waddr, sak, shalf);
            score_operands(a);
            gather_half<M, RVQ, KS>(lds, vr[s], 0, lc1_v, lc2_v, odd, ra);
            scores(a, sc, 1);
          }
          softmax(srcs[s], sc, pb);
          if constexpr (M == 16 && KS == 0) {
            direct_half<RVQ>(ra, av);
            gather_half<M, RVQ, KS>(lds, vr[s], 1, lc1_v, lc2_v, odd, rb);
            pv(av, pb, 0);
            direct_half<RVQ>(rb, av);
          } else if constexpr (M == 16) {
            uint32_t svl[2];
            sparse_addrs_lanes(vr[s], vtok, svl);
            direct_half<RVQ>(ra, av);
            store_lanes(lds, tbase, lane, av);
            sparse_stage<M, RVQ, KS>(lds, vr[s], 0, svl, shalf);
            load_lanes(lds, tbase, lane, av);
            gather_half<M, RVQ, KS>(lds, vr[s], 1, lc1_v, lc2_v, odd, rb);
            pv(av, pb, 0);
            direct_half<RVQ>(rb, av);
            store_lanes(lds, tbase, lane, av);
            sparse_stage<M, RVQ, KS>(lds, vr[s], 1, svl, shalf);
            load_lanes(lds, tbase, lane, av);
          } else {
            store_half<M, RVQ, KS>(lds, vr[s], ra, 0, waddr, sav, shalf);
            pv_operands(av);
            gather_half<M, RVQ, KS>(lds, vr[s], 1, lc1_v, lc2_v, odd, rb);
            pv(av, pb, 0);
            store_half<M, RVQ, KS>(lds, vr[s], rb, 1, waddr, sav, shalf);
            pv_operands(av);
          }
          if constexpr (kDep > 1) {  // the next tile's codes are in the other slot
            if constexpr (LUT) gather_k(kr[(s + 1) % kDep], 0, ka);
            else gather_k(kr[(s + 1) % kDep], 0, ra);
          }
          pv(av, pb, 1);
        }
        fetch(srcs[s], kr[s], vr[s], tt + (s + kDep) * kWaves);
        if constexpr (kDep == 1) {  // one slot: the next tile's first gather follows its fetch
          if (srcs[0].kind >= 0) {
            if constexpr (LUT) gather_k(kr[0], 0, ka);
            else gather_k(kr[0], 0, ra);
          }
        }
      }
    }
  }

  set_prio(0);
  // ---- combine the waves of this block and write the split partial
  __syncthreads();
  // [w][8] m, [w][8] l, [w][8][64] acc, then (score tables) [w][8] sum p^2 and 8 drift estimates
  float* red = reinterpret_cast<float*>(lds);
  float* red_m = red;
  float* red_l = red + kWaves * 8;
  float* red_a = red + kWaves * 16;
  float* red_q = red_a + kWaves * 8 * kD;
  float* est = red_q + kWaves * 8;
#pragma unroll
  for (int hg = 0; hg < NHG; ++hg) {
    const int hh = hg * 4 + (n >> 2);
    // the head's denominator: the lanes of its 4 k-groups (l, l ^ 16, l ^ 32, l ^ 48)
    float ls = lsum[hg];
    {
      const auto r16 = __builtin_amdgcn_permlane16_swap(fbits(ls), fbits(ls), false, false);
      ls = bitsf(r16[0]) + bitsf(r16[1]);
      const auto r32 = __builtin_amdgcn_permlane32_swap(fbits(ls), fbits(ls), false, false);
      ls = bitsf(r32[0]) + bitsf(r32[1]);
    }
    float lq = lsq[hg];
    if constexpr (LUT) {
      const auto r16 = __builtin_amdgcn_permlane16_swap(fbits(lq), fbits(lq), false, false);
      lq = bitsf(r16[0]) + bitsf(r16[1]);
      const auto r32 = __builtin_amdgcn_permlane32_swap(fbits(lq), fbits(lq), false, false);
      lq = bitsf(r32[0]) + bitsf(r32[1]);
    }
    if (g == 0 && ep == 0) {
      red_m[wave * 8 + hh] = m_run[hg];
      red_l[wave * 8 + hh] = ls;
      if constexpr (LUT) red_q[wave * 8 + hh] = lq;
    }
    // D rows 4g + r = subspace m, column n = (head, coordinate ep): dim 4m + ep
#pragma unroll
    for (int r = 0; r < 4; ++r) red_a[(wave * 8 + hh) * kD + 4 * (4 * g + r) + ep] = acc[hg][r];
  }
  __syncthreads();
  const int slots = p.part_slots ? p.part_slots : splits;
  bool redo = false;
  if constexpr (LUT) {
    if (p.guard) {  // uniform
      // drift estimate of head j = wave (< G <= 4): sigma^2 = scale^2 2^-20/12
      // sum_i q_i^2 W_i (fp16 rounding of K^ and of the table entries, as
      // uniform errors of at most 2^-10 |x| per ulp), times sqrt(sum p^2) / l
      // (the first-order output change per unit logit noise) and 2 vmax
      // (|v_t - out| <= 2 max |V^|)
      const float* gw = p.guard + (p.pq_cb_stride ? (int64_t)b * 65 : 0);  // shared codebooks: one row
      if (wave < G) {
        const uint16_t* qrow = (const uint16_t*)p.q + ((int64_t)b * p.q_heads + h * G + wave) * kD;
        const float qv = h2f(qrow[lane]);
        float s2 = qv * qv * gw[lane];
#pragma unroll
        for (int o = 32; o >= 1; o >>= 1) s2 += __shfl_xor(s2, o, 64);
        // vmax also covers the launch's appended V rows (their fold into
        // the guard row may land after this read)
        uint32_t vb = __builtin_bit_cast(uint32_t, gw[64]);
        for (int i = lane; i < p.app_count * p.kv_heads * kD; i += 64) {
          const int j = i / (p.kv_heads * kD), r = i - j * (p.kv_heads * kD);
          vb = max(vb, __builtin_bit_cast(uint32_t, fabsf(h2f(((const uint16_t*)p.app_v)[(int64_t)j * p.app_ld + r]))));
        }
#pragma unroll
        for (int o = 32; o >= 1; o >>= 1) vb = max(vb, (uint32_t)__shfl_xor((int)vb, o, 64));
        const float vmax = __builtin_bit_cast(float, vb);
        if (lane == 0) {
          float Mx = -__builtin_inff();
          for (int w = 0; w < kWaves; ++w) Mx = fmaxf(Mx, red_m[w * 8 + wave]);
          float Ls = 0.f, Q = 0.f;
          for (int w = 0; w < kWaves; ++w) {
            const float mw = red_m[w * 8 + wave];
            const float f = mw > -__builtin_inff() ? exp2f(mw - Mx) : 0.f;
            Ls += red_l[w * 8 + wave] * f;
            Q += red_q[w * 8 + wave] * f * f;
          }
          const float sigma = p.scale * sqrtf(kDriftVar * s2);
          const float e = Ls > 0.f ? sigma * sqrtf(Q) / Ls * 2.f * vmax : 0.f;
          est[wave] = e;
          if (p.drift) p.drift[((int64_t)b * p.q_heads + h * G + wave) * slots + p.part_base + split] = e;
        }
      }
      __syncthreads();
      for (int j = 0; j < G; ++j) redo = redo || !(est[j] <= p.guard_tol);
    }
  }
  if (redo) return true;  // uniform: the exact pass writes this block's output
  for (int idx = threadIdx.x; idx < G * kD; idx += kThreads) {
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
    if (splits == 1 && p.part_slots == 0) {
      // whole (sequence, KV head) in this block: normalise and write fp16 directly
      // (a query with no allowed key returns zeros, attention.py:104-105)
      uint16_t* o = (uint16_t*)p.out + ((int64_t)b * p.q_heads + h * G + head) * kD;
      o[c] = f2h(Ls > 0.f ? A / Ls : 0.f);
      continue;
    }
    // partial slot: this call's split, after the slots of earlier calls in partial mode
    float* out = reinterpret_cast<float*>(p.workspace) +
                 (((int64_t)b * p.q_heads + h * G + head) * slots + p.part_base + split) * (kD + 2);
    if (c == 0) {
      out[0] = Mx;
      out[1] = Ls;
    }
    out[2 + c] = A;
  }
  return false;
}

// The exact pass out of line: its registers are allocated apart from the
// table pass's loop, which it would otherwise crowd into spills.
template <int M, bool RVQ, int KS, int NHG>
__device__ __noinline__ void exact_rows_pass(const rfsn_fused_params p, int splits, int tiles_per_split,
                                             int blocks_total, uint8_t* lds) {
  attn_body<M, RVQ, KS, NHG, kExactRows>(p, splits, tiles_per_split, blocks_total, lds);
}

// The launch's appended tokens (app_count of them, rows in the caller's
// buffers) into their hot slots hot_len - app_count .. for KV head h, and
// max |v| over them into *app_vabs.  Run by the first split of sequence 0 of
// each KV head; the launch itself reads these tokens from the caller's rows,
// so no block waits for the copy.
__device__ __forceinline__ void append_hot_tokens(const rfsn_fused_params& p, int h) {
  constexpr int kUnits = kD / 8;  // 16-byte units of a row
  const int per = p.app_count * kUnits;
  const int i = threadIdx.x;
  if (i >= 2 * per) return;
  const bool is_v = i >= per;
  const int j = (is_v ? i - per : i) / kUnits, u = i % kUnits;
  const uint16_t* src = (const uint16_t*)(is_v ? p.app_v : p.app_k) + (int64_t)j * p.app_ld + h * kD + u * 8;
  uint16_t* dst = (uint16_t*)(is_v ? p.hot_v : p.hot_k) +
                  ((int64_t)h * p.hot_cap + (p.hot_len - p.app_count) + j) * kD + u * 8;
  const uint4 w = *reinterpret_cast<const uint4*>(src);
  *reinterpret_cast<uint4*>(dst) = w;
  if (is_v && p.app_vabs) {
    // float bits compared as integers: |v| >= 0, NaN bits order above +inf
    uint32_t m = 0;
    const uint32_t ww[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      m = max(m, __builtin_bit_cast(uint32_t, fabsf(h2f((uint16_t)(ww[e] & 0xFFFFu)))));
      m = max(m, __builtin_bit_cast(uint32_t, fabsf(h2f((uint16_t)(ww[e] >> 16)))));
    }
    atomicMax(p.app_vabs, m);
  }
}

template <int M, bool RVQ, int KS, int NHG, int KM>
__global__ void __launch_bounds__(BlockShape<NHG>::T, 1)
fused_decode_attn_kernel(const rfsn_fused_params p, int splits, int tiles_per_split, int blocks_total) {
  // static allocation: its base address is known at compile time, so LDS
  // addresses built in registers need no base add
  __shared__ __align__(16) uint8_t lds[BlockShape<NHG>::L];
  if (p.app_count > 0) {  // uniform
    int b, h, split;
    block_unit(blocks_total, splits, p.kv_heads, b, h, split);
    if (b == 0 && split == 0) append_hot_tokens(p, h);
  }
  const bool redo = attn_body<M, RVQ, KS, NHG, KM>(p, splits, tiles_per_split, blocks_total, lds);
  if constexpr (KM == kTables) {
    if (redo) {  // uniform
      __syncthreads();  // every wave has read the combine area the exact pass restages over
      exact_rows_pass<M, RVQ, KS, NHG>(p, splits, tiles_per_split, blocks_total, lds);
    }
  }
  if constexpr (KM == kExactRows) {
    // launched instead of the table body: no table drift to report
    if (p.drift && threadIdx.x < p.q_heads / p.kv_heads) {
      int b, h, split;
      block_unit(blocks_total, splits, p.kv_heads, b, h, split);
      const int slots = p.part_slots ? p.part_slots : splits;
      p.drift[((int64_t)b * p.q_heads + h * (p.q_heads / p.kv_heads) + threadIdx.x) * slots + p.part_base + split] = 0.f;
    }
  }
}

int waves_for(const rfsn_fused_params* p) {
  return p->q_heads / p->kv_heads <= 4 ? BlockShape<1>::W : BlockShape<2>::W;
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
  int s = (256 + units - 1) / units;                // one block per CU (LDS-bound occupancy)
  const int waves = waves_for(p);
  const int max_s = (tiles + waves - 1) / waves;    // at least one tile per wave
  if (s > max_s) s = max_s;
  if (s < 1) s = 1;
  return s;
}

template <int M, bool RVQ, int KS, int NHG, int KM>
int launch_fused(const rfsn_fused_params* p, hipStream_t s) {
  const int splits = auto_splits(p);
  const int tiles = total_tiles_host(p);
  const int tps = (tiles + splits - 1) / splits;
  const int blocks = p->batch * p->kv_heads * splits;
  auto kern = fused_decode_attn_kernel<M, RVQ, KS, NHG, KM>;  // 160 KB of static LDS
  hipLaunchKernelGGL(kern, dim3((unsigned)blocks), dim3(BlockShape<NHG>::T), 0, s, *p, splits, tps, blocks);
  int st = check_launch("fused_decode_attention");
  if (st) return st;
  if (p->part_slots > 0) {
    if (!p->merge) return RFSN_OK;
    return launch_merge(reinterpret_cast<const float*>(p->workspace),
                        (int64_t)p->batch * p->q_heads, p->part_slots, kD, p->out, s);
  }
  if (splits == 1) return RFSN_OK;
  return launch_merge(reinterpret_cast<const float*>(p->workspace),
                      (int64_t)p->batch * p->q_heads, splits, kD, p->out, s);
}

// How a call scores K: kCodebook (K^ rebuilt from the codebooks, k_layout
// 0), kTables, or kExactRows (the drift guard's exact pass alone).
//
// The guard estimates a block's drift over its split, not over the
// whole window: with S splits of similar weight the estimate is about
// sqrt(S) times the window's, and a block that fires recomputes its
// split after the table pass.  With the guard on, a launch of several
// splits so short that a wave streams fewer than kTableMinTilesPerWave
// tiles runs the exact pass alone (from the codebooks): measured on
// one MI355X it is faster there (batch 4 x 32K, 8 splits: 0.032 ms
// against 0.097 ms), while at 16 tiles per wave and more the tables win.
int k_route(const rfsn_fused_params* p) {
  if (p->k_layout != 1) return kCodebook;
  if (p->guard) {
    const int splits = auto_splits(p);
    const int tps = (total_tiles_host(p) + splits - 1) / splits;
    if (splits > 1 && tps < kTableMinTilesPerWave * BlockShape<1>::W) return kExactRows;
  }
  return kTables;
}

template <int M, bool RVQ, int KS>
int dispatch_nhg(const rfsn_fused_params* p, hipStream_t s) {
  const int G = p->q_heads / p->kv_heads;
  if constexpr (M == 16 && RVQ) {
    switch (k_route(p)) {
      case kTables: return launch_fused<M, RVQ, KS, 1, kTables>(p, s);
      case kExactRows: return launch_fused<M, RVQ, KS, 1, kExactRows>(p, s);
      default: break;
    }
  }
  if (G <= 4) return launch_fused<M, RVQ, KS, 1, kCodebook>(p, s);
  return launch_fused<M, RVQ, KS, 2, kCodebook>(p, s);
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

extern "C" int32_t rfsn_fused_splits(const rfsn_fused_params* p) {
  if (p == nullptr || p->batch <= 0 || p->q_heads <= 0 || p->kv_heads <= 0) return 0;
  return auto_splits(p);
}

extern "C" int32_t rfsn_fused_k_scoring(const rfsn_fused_params* p) {
  if (p == nullptr || p->batch <= 0 || p->q_heads <= 0 || p->kv_heads <= 0) return -1;
  return k_route(p);
}

extern "C" size_t rfsn_fused_workspace_bytes(const rfsn_fused_params* p) {
  if (p == nullptr || p->batch <= 0 || p->q_heads <= 0 || p->kv_heads <= 0) return 0;
  const int splits = auto_splits(p);
  const int slots = p->part_slots > 0 ? p->part_slots : splits;
  if (p->part_slots <= 0 && splits == 1) return 0;  // one split writes the output directly
  return (size_t)p->batch * p->q_heads * slots * (kD + 2) * sizeof(float);
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
  RFSN_REQUIRE(p->part_slots >= 0 && p->part_base >= 0 && (p->merge == 0 || p->merge == 1),
               "fused: bad partial-mode fields");
  RFSN_REQUIRE(p->part_slots > 0 || (p->part_base == 0 && p->merge == 0),
               "fused: part_base and merge need part_slots > 0");
  RFSN_REQUIRE(p->part_slots <= 8192 && auto_splits(p) <= 8192, "fused: at most 8192 split partials");
  if (p->part_slots > 0) {
    const int splits = auto_splits(p);
    RFSN_REQUIRE(p->part_base + splits <= p->part_slots, "fused: part_base + splits exceeds part_slots");
    RFSN_REQUIRE(!p->merge || p->part_base + splits == p->part_slots,
                 "fused: the merging call must fill the last slots (part_base + splits == part_slots)");
  }
  RFSN_REQUIRE(p->k_layout == 0 || p->k_layout == 1, "fused: k_layout must be 0 or 1");
  RFSN_REQUIRE(p->k_layout == 0 || (f.pq_subspaces == 16 && f.rvq_subspaces == 16 && p->q_heads / p->kv_heads <= 4),
               "fused: k_layout 1 needs 16 PQ and 16 RVQ subspaces and at most 4 query heads per KV head");
  RFSN_REQUIRE(p->guard == nullptr || p->k_layout == 1, "fused: the drift guard serves k_layout 1 only");
  RFSN_REQUIRE(p->guard == nullptr || p->guard_tol >= 0.f, "fused: guard_tol must be >= 0");
  RFSN_REQUIRE(p->drift == nullptr || p->guard != nullptr, "fused: drift estimates need the guard");
  RFSN_REQUIRE(p->tile_map == nullptr || (p->tile_map_count && p->tile_map_stride > 0 && p->max_segments > 0),
               "fused: a tile map needs its counts, a positive stride and a segment table");
  RFSN_REQUIRE((p->k_tab == nullptr) == (p->v_tab == nullptr) && p->tab_stride >= 0 &&
                   (p->tab_stride == 0 || p->tab_stride >= 65536) &&
                   reinterpret_cast<uintptr_t>(p->k_tab) % 16 == 0 && reinterpret_cast<uintptr_t>(p->v_tab) % 16 == 0 &&
                   p->tab_stride % 16 == 0,
               "fused: entry tables come as a 16-byte aligned K and V pair of 64 KB per sequence (stride 0 or >= 65536)");
  const size_t wsb = rfsn_fused_workspace_bytes(p);
  RFSN_REQUIRE(wsb == 0 || (p->workspace && p->workspace_bytes >= wsb), "fused: workspace too small");
  RFSN_REQUIRE(p->app_count >= 0 && p->app_count <= kTile && p->app_count <= p->hot_len,
               "fused: app_count must be in [0, 32] and within hot_len");
  RFSN_REQUIRE(p->app_count == 0 ||
                   (p->app_k && p->app_v && p->app_ld >= (int64_t)p->kv_heads * kD && p->app_ld % 8 == 0 &&
                    reinterpret_cast<uintptr_t>(p->app_k) % 16 == 0 &&
                    reinterpret_cast<uintptr_t>(p->app_v) % 16 == 0 &&
                    reinterpret_cast<uintptr_t>(p->hot_k) % 16 == 0 &&
                    reinterpret_cast<uintptr_t>(p->hot_v) % 16 == 0 && p->hot_cap % 8 == 0),
               "fused: appended rows need K and V pointers, a token stride of at least kv_heads * 64 (a multiple "
               "of 8) and 16-byte alignment of them and of the hot buffers");
  RFSN_REQUIRE(p->app_count == 0 || p->hot_seq_stride == 0 || p->batch == 1,
               "fused: appending in the launch needs one hot tier shared by the sequences (hot_seq_stride 0)");
  hipStream_t s = (hipStream_t)stream;
  const bool rvq = f.rvq_subspaces > 0;
  if (f.pq_subspaces == 16) return rvq ? dispatch_ks<16, true>(p, s) : dispatch_ks<16, false>(p, s);
  return rvq ? dispatch_ks<8, true>(p, s) : dispatch_ks<8, false>(p, s);
}

// ---------------------------------------------------------------- allocation-free variant
// Split partials of rfsn_fused_decode_attention_noalloc live in this
// file-scope device array instead of a caller workspace.  Each device that
// runs the library holds its own copy (RFSN_FUSED_SCRATCH_BYTES) until the
// process ends.  Host code never passes `scratch` itself to a kernel (in host
// code the name is a host-side stand-in): the device address comes from
// hipGetSymbolAddress, looked up once per device with that device current.
static __device__ __align__(256) uint8_t scratch[RFSN_FUSED_SCRATCH_BYTES];

namespace {
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

int scratch_address(void** out) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return fail(RFSN_ERR_HIP, std::string("hipGetDevice: ") + hipGetErrorString(e));
  if (dev < 0 || dev >= kMaxDevices) return fail(RFSN_ERR_UNSUPPORTED, "fused_noalloc: device index beyond 63");
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    void* ptr = nullptr;
    e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess || ptr == nullptr)
      return fail(RFSN_ERR_HIP, std::string("hipGetSymbolAddress(scratch): ") + hipGetErrorString(e));
    g_scratch_ptr[dev] = ptr;
  }
  *out = g_scratch_ptr[dev];
  return RFSN_OK;
}
}  // namespace

extern "C" int rfsn_fused_decode_attention_noalloc(const rfsn_fused_params* p, void* stream) {
  RFSN_REQUIRE(p != nullptr, "fused_noalloc: null params");
  rfsn_fused_params q = *p;
  q.workspace = nullptr;
  q.workspace_bytes = 0;
  const size_t need = rfsn_fused_workspace_bytes(&q);
  if (need > (size_t)RFSN_FUSED_SCRATCH_BYTES)
    return fail(RFSN_ERR_INVALID, "fused_noalloc: the call's split partials need " + std::to_string(need) +
                                      " bytes, more than the " + std::to_string((size_t)RFSN_FUSED_SCRATCH_BYTES) +
                                      "-byte scratch (fewer splits, query heads or sequences per call)");
  if (need > 0) {
    void* ptr = nullptr;
    const int st = scratch_address(&ptr);
    if (st) return st;
    // every partial slot is written by the launch before the merge reads it:
    // nothing in the scratch has to start at zero
    q.workspace = ptr;
    q.workspace_bytes = (size_t)RFSN_FUSED_SCRATCH_BYTES;
  }
  return rfsn_fused_decode_attention(&q, stream);
}
