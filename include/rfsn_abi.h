/*
 * rfsn_abi.h -- C ABI of the MI355X (gfx950) warm-tier quantized-KV decode
 * library (librfsn_hip.so).
 *
 * Conventions
 *  - Every entry point returns int: RFSN_OK (0) or a negative RFSN_ERR_*;
 *    rfsn_last_error() returns the message of the last failure on the
 *    calling thread.  No C++ exception crosses this boundary.
 *  - Every pointer is caller-owned.  Pointers named *_dev are device
 *    (HBM) pointers; nothing here allocates device memory: scratch space is
 *    passed in as a workspace sized by the matching *_workspace_bytes().
 *  - Every kernel is asynchronous on the caller's hipStream_t (passed as
 *    void*; NULL = the legacy default stream).  No global mutable state,
 *    except the per-GPU scratch array of rfsn_fused_decode_attention_noalloc.
 *  - fp16 tensors are passed as void* and hold IEEE binary16 bit patterns.
 *  - Shapes use the reference's names: N vectors, D = head_dim,
 *    M PQ subspaces of d = D/M dims with C centroids, M_r RVQ subspaces of
 *    d_r = D/M_r dims with C_r centroids, k sparse residual coordinates.
 *
 * Reference interfaces replaced (files of dawsonblock/apple):
 *  see the comment above each entry point.
 */
#ifndef RFSN_ABI_H
#define RFSN_ABI_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define RFSN_ABI_VERSION 8

#define RFSN_OK 0
#define RFSN_ERR_INVALID (-1)     /* shape / contract violation -> ValueError   */
#define RFSN_ERR_STATE (-2)       /* use before set-up          -> RuntimeError */
#define RFSN_ERR_HIP (-3)         /* HIP runtime failure        -> RuntimeError */
#define RFSN_ERR_UNSUPPORTED (-4) /* shape outside the compiled kernels          */

int rfsn_abi_version(void);
const char* rfsn_last_error(void);

/* Warm-tier format: PQ base, optional subspace RVQ stage, optional top-k
 * sparse residual.  The reference's PQ (quantization.py:99-157) is the case
 * rvq_subspaces = 0, sparse_k = 0. */
typedef struct rfsn_format {
  int32_t head_dim;      /* D                                   */
  int32_t pq_subspaces;  /* M  (D % M == 0)                     */
  int32_t pq_centroids;  /* C  (<= 256, uint8 codes)            */
  int32_t rvq_subspaces; /* M_r, 0 = no RVQ stage               */
  int32_t rvq_centroids; /* C_r (<= 256)                        */
  int32_t sparse_k;      /* k, 0 = no sparse residual (<= 8)    */
} rfsn_format;

/* Codes of N vectors in the warm format, row-major, contiguous rows:
 * pq [N][M] u8, rvq [N][M_r] u8, sparse_idx [N][k] u8, sparse_val [N][k] fp16. */
typedef struct rfsn_codes {
  uint8_t* pq;
  uint8_t* rvq;
  uint8_t* sparse_idx;
  void* sparse_val;
} rfsn_codes;

/* ---------------------------------------------------------------- encode
 * Nearest-centroid PQ encode with the canonical distance
 * fl32(fl32(L - 2X) + R) and first-min argmin; residual fp16(x - c).
 * Replaces ProductQuantizerMLX.quantize (quantization.py:124-144) and
 * _squared_l2_distance (quantization.py:92-96).
 * x_dev [groups][N][ldx] fp16 (group stride x_gstride elements);
 * codebooks_dev [groups][M][C][d] fp16 (stride cb_gstride elements);
 * codes_dev [groups][N][ldc] u8 (stride codes_gstride); resid_dev may be NULL,
 * else [groups][N][ldr] fp16 (stride resid_gstride). */
int rfsn_pq_encode(const void* x_dev, int64_t n, int32_t D, int64_t ldx, int64_t x_gstride,
                   const void* codebooks_dev, int32_t M, int32_t C, int64_t cb_gstride,
                   uint8_t* codes_dev, int64_t ldc, int64_t codes_gstride,
                   void* resid_dev, int64_t ldr, int64_t resid_gstride,
                   int32_t groups, void* stream);

/* Fused warm-format encode: PQ, then (if fmt->rvq_subspaces) PQ of the fp16
 * residual with the RVQ codebooks, then (if fmt->sparse_k) the top-k |r2|
 * coordinates of r2 = fl32(x - fp16(base + rvq)).  No reference symbol: the
 * RVQ stage generalises ResidualVQMLX.encode (quantization.py:206-252) to
 * subspaces; the sparse stage is new.  Output rows go to out.* (rows of the
 * same vector order as x).  workspace_dev: rfsn_warm_encode_workspace_bytes. */
size_t rfsn_warm_encode_workspace_bytes(const rfsn_format* fmt, int64_t n);
int rfsn_warm_encode(const rfsn_format* fmt, const void* x_dev, int64_t n, int64_t ldx,
                     const void* pq_cb_dev, const void* rvq_cb_dev, rfsn_codes out,
                     void* workspace_dev, size_t workspace_bytes, void* stream);

/* Several vector sets of one format in one launch (a chunk's K and V, as
 * the warm append of cache.py:122-132 encodes them): each job is
 * rfsn_warm_encode's x / n / ldx / codebooks / out.  Needs head_dim 64, 4- or
 * 8-dim subspaces, an RVQ stage of the same split or none, sparse_k 0 or 4,
 * 16-byte aligned x rows and naturally aligned code and sparse rows, and no
 * workspace: the PQ residual stays in registers (RFSN_ERR_UNSUPPORTED for
 * other formats; rfsn_warm_encode serves every format).  The same codes as
 * rfsn_warm_encode, bit for bit. */
typedef struct rfsn_encode_job {
  const void* x;
  int64_t n;
  int64_t ldx;
  const void* pq_cb;
  const void* rvq_cb;
  rfsn_codes out;
} rfsn_encode_job;
int rfsn_warm_encode_batch(const rfsn_format* fmt, const rfsn_encode_job* jobs, int32_t count, void* stream);

/* Reference-mode RVQ (quantization.py:206-252), three steps:
 * (1) gate: mask[i] = fl32(sqrt(fl32(sum r^2))) > threshold (u8 0/1);
 * (2) compaction: offsets[0..A) = ascending indices with mask set,
 *     count_dev[0] = A  (np.flatnonzero, quantization.py:218);
 * (3) L-stage full-dimension encode of the active rows (running residual in
 *     fp32, first-min argmin over C <= 65535 centroids, which equals the
 *     reference's 512-centroid chunks merged with a strict <), codes [A][L]
 *     u16.  For D in {64, 128, 256} and 3 <= C <= 16384 the search screens
 *     on MFMA and needs a workspace of
 *     rfsn_rvq_encode_full_workspace_bytes(A, D, L, C) bytes (16-byte
 *     aligned; 0 = none needed), and the residual rows and codebooks must be
 *     16-byte aligned (ld a multiple of 8). */
int rfsn_rvq_gate(const void* resid_dev, int64_t n, int32_t D, int64_t ld, float threshold,
                  uint8_t* mask_dev, void* stream);
size_t rfsn_mask_compact_workspace_bytes(int64_t n);
int rfsn_mask_compact(const uint8_t* mask_dev, int64_t n, int32_t* offsets_dev, int32_t* count_dev,
                      void* workspace_dev, size_t workspace_bytes, void* stream);
size_t rfsn_rvq_encode_full_workspace_bytes(int64_t active, int32_t D, int32_t L, int32_t C);
int rfsn_rvq_encode_full(const void* resid_dev, int64_t ld, int32_t D, const int32_t* offsets_dev,
                         int64_t active, const void* codebooks_dev, int32_t L, int32_t C,
                         uint16_t* codes_dev, void* workspace_dev, size_t workspace_bytes, void* stream);

/* ---------------------------------------------------------------- decode
 * Warm-format decode to fp16 [N][ldo]: fp16(base + rvq) then sparse
 * K[idx] = fp16(K[idx] + val).  Replaces ProductQuantizerMLX.decode
 * (quantization.py:146-157) for the PQ-only format and
 * _decode_compressed_tensor (quantization.py:394-403) for the warm format. */
int rfsn_decode(const rfsn_format* fmt, const rfsn_codes* codes, int64_t n,
                const void* pq_cb_dev, const void* rvq_cb_dev, void* out_dev, int64_t ldo,
                int32_t add_zero_correction, void* stream);

/* Corrected coordinates of the sparse stage: out[v][j] = fp16(K[idx] + val)
 * with K = fp16(base + rvq) and idx = sparse_idx[v][j], val = sparse_val[v][j],
 * i.e. the value rfsn_decode leaves at coordinate idx.  out is [N][k] fp16.
 * The fused kernel's segments carry these values in place of the residuals
 * (rfsn_segment), so that it applies the sparse stage by one store per entry.
 * No reference symbol (the sparse stage extends quantization.py:317-319). */
int rfsn_sparse_fold(const rfsn_format* fmt, const rfsn_codes* codes, int64_t n,
                     const void* pq_cb_dev, const void* rvq_cb_dev, void* out_dev, void* stream);

/* Score deltas of the sparse stage: out[v][j] = fp16(c - (float(base[idx]) +
 * float(rvq[idx]))) in fp32 arithmetic, c = the corrected coordinate of
 * rfsn_sparse_fold.  A kernel that scores codes through q . centroid tables
 * (which sum base + rvq unrounded) adds q[idx] * out[v][j] to reach q . K of
 * the decoded key.  out is [N][k] fp16.  No reference symbol (see
 * rfsn_sparse_fold). */
int rfsn_sparse_delta(const rfsn_format* fmt, const rfsn_codes* codes, int64_t n,
                      const void* pq_cb_dev, const void* rvq_cb_dev, void* out_dev, void* stream);

/* The warm append of one block of K and V in one launch, for the 16 + 16
 * subspace formats of head_dim 64 with 1..16 sparse entries: plain
 * head-major codes k_src / v_src ([heads][T][16] codes, [heads][T][k] sparse
 * index bytes and fp16 residuals, contiguous) into tokens t_base ..
 * t_base+T-1 of blocks of dst_tokens tokens (a multiple of 32) per head.  V,
 * and K with k_score_rows = 0, go to the rfsn_pack_codes layout with the
 * corrected coordinates of rfsn_sparse_fold at [heads][dst_tokens][k]; K
 * with k_score_rows = 1 goes to the rfsn_pack_score_codes layout with the
 * score deltas of rfsn_sparse_delta as its sparse values and, when k_cc is
 * not NULL, the corrected coordinates in the array k_cc at the same
 * positions.  With k_ring / v_ring (NULL: none) the plain codes also go to
 * rows ring_row .. ring_row+T-1 of token-major stores in the reference
 * layout (CompressedTensorMLX: pq and rvq codes [cap][heads][16], the RVQ
 * mask [cap][heads] set to 1, sparse index and residual [cap][heads][k]).
 * The same bytes as those calls and copies, in one launch instead of up to
 * twelve.  Replaces the warm append of cache.py:122-132. */
int rfsn_warm_append_pair(const rfsn_format* fmt, const rfsn_codes* k_src, const rfsn_codes* v_src, int64_t T,
                          int32_t heads, const void* k_pq_cb_dev, const void* k_rvq_cb_dev, const void* v_pq_cb_dev,
                          const void* v_rvq_cb_dev, const rfsn_codes* k_dst, int32_t k_score_rows, void* k_cc_dev,
                          const rfsn_codes* v_dst, int64_t dst_tokens, int64_t t_base,
                          const rfsn_codes* k_ring, uint8_t* k_ring_mask_dev, const rfsn_codes* v_ring,
                          uint8_t* v_ring_mask_dev, int64_t ring_row, void* stream);

/* Reference-format hybrid decode (quantization.py:310-319): base =
 * C_pq[pq_codes]; corr = fp16(sum_l C_l[rvq_codes[a][l]]) scattered to rows
 * offsets[a]; out = fp16(base + corr) (corr = +0 for inactive rows). */
int rfsn_decode_ref(const uint8_t* pq_codes_dev, int64_t n, int32_t D, int32_t M, int32_t C,
                    const void* pq_cb_dev, const uint16_t* rvq_codes_dev, const int32_t* offsets_dev,
                    int64_t active, int32_t L, int32_t C_r, const void* rvq_cb_dev,
                    void* out_dev, void* stream);

/* ---------------------------------------------------------------- attention
 * Exact blockwise decode attention over fp16 K/V (attention.py:39-105,
 * _blockwise_exact_attention), split over the token axis with an LSE merge.
 * q [B][Hq][D] fp16, K/V element (t, h, i) at base + t*stride_t + h*stride_h + i,
 * Hq % Hkv == 0 (query head h reads KV head h / (Hq/Hkv)),
 * qpos_dev [B][Hq] int32 or NULL (= every query at T-1), causal masks
 * positions > qpos; out [B][Hq][D] fp16 = q.dtype.  Any block size gives the
 * same result up to fp32 rounding. */
size_t rfsn_attention_workspace_bytes(int32_t B, int32_t Hq, int32_t D, int32_t splits);
int rfsn_blockwise_attention(const void* q_dev, int32_t B, int32_t Hq, int32_t D,
                             const void* k_dev, const void* v_dev, int64_t T, int32_t Hkv,
                             int64_t stride_t, int64_t stride_h, float scale, int32_t causal,
                             const int32_t* qpos_dev, void* out_dev,
                             void* workspace_dev, size_t workspace_bytes, void* stream);

/* Code layout the fused kernel streams ("tiled"): codes of one KV head live
 * in a block of cap*M bytes (cap a multiple of 32); inside 32-token tile
 * tau, the code of (token t, subspace m) sits at byte
 *   tau*32*M + ((t % TPI)*M + m)*IPT + (t % 32)/TPI,  TPI = 64/M, IPT = 32/TPI,
 * so that one 64-lane gather instruction reads TPI tokens x M subspaces.
 * rfsn_pack_codes converts plain rows [heads][T][M] (head stride
 * src_head_stride bytes) into tokens t_base .. t_base+T-1 of the tiled
 * layout (head stride dst_head_stride bytes).  M must be 8 or 16. */
int rfsn_pack_codes(const uint8_t* src_dev, int64_t src_head_stride, int64_t T, int32_t M, int32_t heads,
                    uint8_t* dst_dev, int64_t dst_head_stride, int64_t t_base, void* stream);

/* K layout of k_layout = 1 (16 PQ + 16 RVQ subspaces, k <= 16 sparse
 * entries).  Token t = 32*tau + 16*u + r of a head: code byte j = 4*g + b of
 * its row (in each code array) sits at byte 512*tau + 32*r + 8*g + 4*u + b of
 * the head's block and holds subspace 4*g + (b ^ ((r >> 2) & 3)); odd tokens
 * keep their RVQ codes in the PQ array and their PQ codes in the RVQ array.
 * Sparse entry e of the token sits at entry 32*k*tau + 2*k*r + 2*e + u of the
 * head's block in both sparse arrays.  Converts plain rows [heads][T][16]
 * (codes) and [heads][T][k] (sparse index / value) into tokens
 * t_base .. t_base+T-1 of blocks of dst_tokens tokens (a multiple of 32) per
 * head.  No reference symbol: lays codes out for the fused kernel's score
 * tables (the warm append of cache.py:122-132). */
int rfsn_pack_score_codes(const uint8_t* pq_src_dev, const uint8_t* rvq_src_dev, const uint8_t* sparse_idx_dev,
                          const uint16_t* sparse_val_dev, int32_t k, int64_t T, int32_t heads,
                          uint8_t* pq_dst_dev, uint8_t* rvq_dst_dev, uint8_t* sparse_idx_dst_dev,
                          uint16_t* sparse_val_dst_dev, int64_t dst_tokens, int64_t t_base, void* stream);

/* Hot-tier append: hot_k[h][t0 + t][:] = k[t][h][:] (and the same for V) for
 * t < T, with the hot tier as [heads][hot_cap][D] fp16 and the new tokens as
 * rows of stride ld_t elements; vabs (may be NULL) receives max(|vabs|, |v|)
 * over the new values (the score tables' drift guard bounds |V| by it).  One
 * launch.  Replaces the hot-tier write of the decode step's append
 * (cache.py:89-120: mx.concatenate of the new tokens onto the hot arrays). */
int rfsn_hot_append(const void* k_dev, const void* v_dev, int64_t ld_t, int32_t T, int32_t heads, int32_t D,
                    void* hot_k_dev, void* hot_v_dev, int64_t hot_cap, int64_t t0, float* vabs_dev, void* stream);

/* Fused warm-tier dequant + exact decode attention over [hot | segments] (or
 * [segments | hot]).  Replaces RFSNv10KVCacheMLX.attention_forward
 * (cache.py:395-428) = materialize_window (cache.py:344-393) +
 * _blockwise_exact_attention, without writing the window to HBM.
 *
 * A segment is a run of encoded tokens of one sequence for all KV heads.
 * PQ and RVQ codes are in the tiled layout (head h at byte h*head_stride*M
 * resp. h*head_stride*M_r; K codes and sparse entries in the
 * rfsn_pack_score_codes layout when k_layout = 1);
 * sparse arrays are plain rows, (head h, token t) at row h*head_stride + t.
 * head_stride is a multiple of 32.  The sparse values of a segment are the
 * corrected coordinates of rfsn_sparse_fold (fp16(K[idx] + residual)), or
 * for K with k_layout = 1 the score deltas of rfsn_sparse_delta, not the
 * residuals.
 * Segment window positions are pos0 .. pos0+len-1 (used by causal masking;
 * tokens at negative positions are skipped). */
typedef struct rfsn_segment {
  rfsn_codes k;
  rfsn_codes v;
  int64_t head_stride; /* token rows between KV heads (multiple of 32) */
  int32_t len;         /* tokens                  */
  int32_t pos0;        /* window position of token 0 */
} rfsn_segment;

typedef struct rfsn_fused_params {
  rfsn_format fmt;
  int32_t batch;       /* B sequences                                   */
  int32_t q_heads;     /* Hq                                            */
  int32_t kv_heads;    /* Hkv                                           */
  const void* q;       /* [B][Hq][D] fp16                               */
  void* out;           /* [B][Hq][D] fp16                               */
  float scale;
  int32_t causal;
  const int32_t* qpos; /* [B][Hq] int32 window positions, or NULL       */
  /* exact (hot) tier: sequence b, KV head h, token t at
   * hot_k + b*hot_seq_stride + (h*hot_cap + t)*D  (fp16 elements);
   * hot_seq_stride = 0 lets B queries share one cache. */
  const void* hot_k;
  const void* hot_v;
  int64_t hot_cap;
  int64_t hot_seq_stride;
  int32_t hot_len;     /* tokens, same for every sequence               */
  int32_t hot_pos0;    /* window position of hot token 0                */
  /* encoded tiers: segments[b*max_segments + s], s < num_segments[b] */
  const rfsn_segment* segments;   /* device array                       */
  const int32_t* num_segments;    /* device [B]                         */
  int32_t max_segments;
  /* codebooks per sequence: pq [B][M][C][d], rvq [B][M_r][C_r][d_r], for K and V */
  const void* k_pq_cb;
  const void* k_rvq_cb;
  const void* v_pq_cb;
  const void* v_rvq_cb;
  int64_t pq_cb_stride;   /* elements between sequences (0 = shared)  */
  int64_t rvq_cb_stride;
  int32_t max_tokens;     /* upper bound on hot_len + sum of segment lengths */
  int32_t splits;         /* token splits per (sequence, KV head); 0 = auto  */
  void* workspace;        /* split partials; may be NULL when           */
  size_t workspace_bytes; /* rfsn_fused_workspace_bytes() returns 0     */
  /* Partial mode (part_slots > 0): one window attended over several calls
   * on one stream, e.g. the resident segments while a side stream copies
   * cold chunks in, then the copied chunks.  The call writes its split
   * partials (running max, sum, unnormalised output) into slots
   * [part_base, part_base + splits) of part_slots per (sequence, query head)
   * of the workspace; with merge = 1 (only when part_base + splits ==
   * part_slots) it then merges all part_slots slots into out.  Every slot
   * must have been written by a call queued earlier on the stream.  Calls
   * that share one workspace share B and Hq.  part_slots = 0: one call. */
  int32_t part_base;
  int32_t part_slots;
  int32_t merge;
  /* Layout of the K streams of every segment:
   * 0: PQ/RVQ codes tiled (rfsn_pack_codes), sparse values the corrected
   *    coordinates of rfsn_sparse_fold;
   * 1: PQ/RVQ codes and sparse entries in the rfsn_pack_score_codes
   *    layout, sparse values the score deltas of rfsn_sparse_delta.  Needs M = M_r = 16 and at most 4 query heads per
   *    KV head: the kernel then scores codes through a per-call table of
   *    q . centroid (fp16) instead of reconstructing K.
   * V streams are always layout 0. */
  int32_t k_layout;
  /* Drift guard of the score tables (k_layout = 1 only; guard = NULL: off).
   * The tables sum q . centroid per subspace without rounding K^ =
   * fp16(base + rvq) to fp16 as the decode does, so their scores drift from
   * q . K^ by about one fp16 rounding of K^ per coordinate.  Each block
   * estimates the drift of its output per query head,
   *   est = scale * sqrt(2^-20/12 * sum_i q_i^2 W_i) * sqrt(sum_t p_t^2) / sum_t p_t * 2 * vmax
   * (the logit noise of uniform roundings of at most 2^-10 |x| per ulp,
   * times the first-order output change per unit of it), from guard[b] =
   * {W_0 .. W_63, vmax} (one row for all sequences when the codebooks are
   * shared, pq_cb_stride = 0; W_i = the second moment of K^_i over the
   * codebooks plus those of the PQ and RVQ centroids of coordinate i's
   * subspace, vmax >= |V^|), and a block where some head's est exceeds
   * guard_tol recomputes its
   * output exactly (K^ rebuilt from the codebooks) before writing it.  That
   * pass reads the corrected coordinates fp16(K[idx] + residual) of K's
   * sparse entries from a second plane of each K sparse-value array, at
   * kv_heads * head_stride * k values after the score deltas, in the same
   * positions.  drift (may be NULL): est per (sequence, query head, split
   * slot), [B][Hq][slots] with slots = part_slots or the call's splits.
   * A guarded call of several splits whose blocks hold fewer than 256
   * tiles of 32 tokens (16 per wave) runs that exact pass alone, with no
   * tables; its drift entries are 0. */
  const float* guard;
  float* drift;
  float guard_tol;
  /* Tile map (optional; NULL: the kernel walks the segment table to find a
   * tile, one scalar-memory round trip per 8 segments).  For row b,
   * tile_map[b * tile_map_stride + r] = (segment << 16) | tile within the
   * segment, for the encoded tiles r = 0, 1, ... of segments 1..nseg-1 in
   * order, and tile_map_count[b] = their number (<= tile_map_stride). */
  const uint32_t* tile_map;
  const int32_t* tile_map_count;
  int64_t tile_map_stride;
  /* Entry-major codebook tables (optional; NULL: the kernel gathers its LDS
   * tables from the [M][C][d] codebooks above).  256 entries of 256 bytes:
   * entry e = [the PQ entries e of subspaces 0..M-1, d fp16 each | the RVQ
   * entries e (the PQ entries again without an RVQ stage)], zeros past a
   * codebook's size.  Sequence b's tables start tab_stride bytes after
   * sequence b-1's (0: shared).  They must hold what the codebooks hold; the
   * kernel then stages them with contiguous loads. */
  const void* k_tab;
  const void* v_tab;
  int64_t tab_stride;
  /* Append in the launch (optional; app_count = 0: none).  The hot range
   * [0, hot_len) ends with app_count (<= 32) new tokens whose K and V rows
   * are still in the caller's buffers, token j of KV head h at
   * app_k + j*app_ld + h*D (fp16 elements, 16-byte aligned rows), not in the
   * hot buffers yet: the launch attends them from there, writes them to hot
   * tokens hot_len - app_count .. hot_len - 1 (blocks of sequence 0, so the
   * next launch finds them in place), and folds max |v| over them into
   * *app_vabs (float bits as an unsigned maximum; may be NULL), which the
   * drift guard's vmax also takes.  Needs hot_seq_stride = 0 (the sequences
   * share one hot tier).  The reference appends in cache.py:89-120 and
   * attends in cache.py:395-428; this fuses the two for a decode loop's
   * one-token step (rfsn_v10_mlx_ane_complete.py:138-158). */
  const void* app_k;
  const void* app_v;
  int64_t app_ld;
  uint32_t* app_vabs;
  int32_t app_count;
} rfsn_fused_params;

/* Token splits the call would use (p->splits, or the automatic choice when 0);
 * sizes partial-mode slots.  Part of the attention_forward replacement
 * (cache.py:395-428). */
int32_t rfsn_fused_splits(const rfsn_fused_params* p);
/* How the call would score K: 0 = K^ rebuilt from the codebooks (k_layout
 * 0), 1 = score tables (with the drift guard's recompute where it fires),
 * 2 = the guard's exact pass alone (see guard above); -1 for a malformed
 * shape.  No counterpart in the reference, whose attention always
 * materializes K (cache.py:395-428); for hosts that report the route. */
int32_t rfsn_fused_k_scoring(const rfsn_fused_params* p);
size_t rfsn_fused_workspace_bytes(const rfsn_fused_params* p);
int rfsn_fused_decode_attention(const rfsn_fused_params* p, void* stream);

/* Allocation-free variant of rfsn_fused_decode_attention.  No counterpart in
 * the reference: it is for callers that cannot allocate device memory (code
 * under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc).  It ignores p->workspace / p->workspace_bytes and keeps the
 * split partials in a library-owned device array of RFSN_FUSED_SCRATCH_BYTES
 * per GPU (held until the process ends); it calls no hipMalloc or hipFree.
 * A call whose partials (rfsn_fused_workspace_bytes with the same params)
 * exceed that size returns RFSN_ERR_INVALID without launching.  Every call on
 * one GPU shares that GPU's array: calls that overlap on one GPU (other
 * streams, other threads) race, and partial-mode calls of one window must
 * not interleave with other calls of this entry point. */
#define RFSN_FUSED_SCRATCH_BYTES (4u << 20)
int rfsn_fused_decode_attention_noalloc(const rfsn_fused_params* p, void* stream);

/* ---------------------------------------------------------------- reference-layout attention
 * Fused decode attention over compressed stores in the layout
 * CompressedTensorMLX holds them (storage.py:75-98, token-major rows of
 * [T][heads]), decoding each K/V vector in registers, never to HBM:
 *  - reference format: PQ codes [T][heads][M] u8 with the gated
 *    full-dimension RVQ correction (codes [A][L] u16 of the active rows),
 *    decoded as quantization.py:310-319 does (corr = fp16(sum_l
 *    fl32(C_l[code_l])), K = fp16(fl32(base) + fl32(corr)), corr = 0 for
 *    inactive rows);
 *  - long-context format: PQ codes, then subspace RVQ codes [T][heads][M_r]
 *    u8 (K = fp16(fl32(base) + fl32(rvq))), then k sparse residuals
 *    (K[idx] = fp16(fl32(K[idx]) + fl32(val)));
 *  - exact segments (the hot tier).
 * Replaces RFSNHybridAttentionMLX.__call__ (attention.py:150-171) and
 * attention_forward over tiers the tiled fused kernel does not serve
 * (cache.py:395-428, materialize_window + _blockwise_exact_attention).
 * head_dim 64, 128 or 256; M in {4, 8, 16, 32} dividing head_dim, C <= 256
 * PQ centroids (the PQ codebooks of K and V must fit 160 KB of LDS together,
 * or one when K and V share it); either L gated RVQ layers of C_r <= 65536
 * codewords or M_r RVQ subspaces (dividing head_dim, C_r <= 256); k <= 8
 * sparse residuals; at most 8 query heads per KV head.  B queries share the
 * segments; segments are in window order. */
typedef struct rfsn_ref_store_codes {
  const uint8_t* pq;          /* [T][heads][M] u8 (4-byte aligned); NULL: an exact segment  */
  const uint16_t* rvq;        /* gated format: [A][L] u16 codes of the active rows          */
  const int32_t* active;      /* gated format: [T][heads] index into rvq, or -1.  NULL with rvq
                                 non-NULL: every row active, row r's codes at rvq + r L (dense);
                                 NULL with rvq NULL: no gated stage */
  const uint8_t* rvq_sub;     /* long-context format: [T][heads][M_r] u8, or NULL            */
  const uint8_t* sparse_idx;  /* long-context format: [T][heads][k] u8, or NULL              */
  const uint16_t* sparse_val; /* long-context format: [T][heads][k] fp16 residuals           */
} rfsn_ref_store_codes;

typedef struct rfsn_ref_segment {
  rfsn_ref_store_codes k;
  rfsn_ref_store_codes v;
  const void* exact_k;         /* exact segments: fp16 (t, h, d) at exact + t*token_stride + h*head_stride + d */
  const void* exact_v;
  int64_t exact_token_stride;  /* elements */
  int64_t exact_head_stride;   /* elements */
  int64_t token0;              /* the segment's first window token is token token0 of its store */
  int32_t len;                 /* tokens */
  int32_t pos0;                /* window position of the segment's first token */
  /* Coded segments: the codes of (token t, KV head h) are row
   * t * code_token_stride + h * code_head_stride of every per-row array (pq,
   * active, dense rvq, rvq_sub, sparse_idx, sparse_val; active entries still
   * index rvq).  0 and 0: the stores' own [T][heads] order, row t * kv_heads + h.
   * A head-major copy ([heads][T]: strides 1 and T) gives a head's consecutive
   * tokens consecutive codes, which the decode kernels read in whole lines.
   * The segment table lives in device memory, so the library cannot check
   * these rows: the caller keeps every row of tokens token0 .. token0 + len - 1
   * and heads 0 .. kv_heads - 1 inside the arrays. */
  int64_t code_token_stride;
  int64_t code_head_stride;
} rfsn_ref_segment;

typedef struct rfsn_ref_params {
  int32_t head_dim;
  int32_t pq_subspaces;
  int32_t pq_centroids;
  int32_t rvq_layers;     /* L gated full-dimension layers, 0 = none */
  int32_t rvq_centroids;  /* C_r (gated layers, or the subspace stage) */
  int32_t rvq_subspaces;  /* M_r subspace-RVQ subspaces, 0 = none (exclusive with rvq_layers) */
  int32_t sparse_k;       /* k sparse residuals per vector, 0 = none */
  int32_t batch;          /* B queries */
  int32_t q_heads;
  int32_t kv_heads;
  const void* q;          /* [B][Hq][D] fp16 */
  void* out;              /* [B][Hq][D] fp16 */
  float scale;
  int32_t causal;
  const int32_t* qpos;    /* [B][Hq] window positions, or NULL */
  const rfsn_ref_segment* segments;  /* device array, window order */
  int32_t num_segments;
  int32_t total_tokens;   /* sum of the segments' lengths (> 0) */
  const void* k_pq_cb;    /* [M][C][d] fp16 */
  const void* v_pq_cb;
  const void* k_rvq_cb;   /* [L][C_r][D] fp16, or [M_r][C_r][D/M_r] for the subspace stage */
  const void* v_rvq_cb;
  int32_t splits;         /* token splits per (query, KV head); 0 = auto */
  void* workspace;        /* split partials: rfsn_ref_attention_workspace_bytes */
  size_t workspace_bytes;
  /* Score tables for the coded segments (0 = decode every coded vector).
   * With 1, each query head gets a table of scale log2(e) q . c over every
   * PQ entry c (on its subspace) and every gated RVQ codeword: a coded
   * token's score is the sum of its entries; its weight p = 2^(score - the
   * block's largest) goes, in fixed point of 2^-19, into a sum per V
   * codeword, and the output is those sums times the V codebooks over the
   * sum of p.  This skips the fp16 rounding of the decoded K and V
   * (quantization.py:310-319); a drift guard estimates the output change
   * per query head from it and from the fixed-point steps, and a (query,
   * KV head) group whose estimate exceeds table_tol for one of its heads
   * decodes its coded tokens instead (exact segments are always exact).
   * Needs the reference format without the long-context stages (gated RVQ,
   * or PQ only), E = M C + L C_r entries with (2 E + 64) * 4 <= 160 KB of
   * LDS, and at most 1,048,576 window tokens (rfsn_ref_tables_ok). */
  int32_t score_tables;
  float table_tol;           /* >= 0 */
  const float* table_stats;  /* [3][head_dim] fp32 from rfsn_ref_table_stats */
  float* drift;              /* [B][Hq] the guard's estimates, or NULL */
} rfsn_ref_params;

size_t rfsn_ref_attention_workspace_bytes(const rfsn_ref_params* p);
int rfsn_ref_attention(const rfsn_ref_params* p, void* stream);
/* 1 when the params' format and shape allow score_tables (ignoring the
 * flag itself), else 0. */
int rfsn_ref_tables_ok(const rfsn_ref_params* p);
/* The drift guard's codebook statistics, [3][head_dim] fp32 into stats_dev:
 * row 0 = mean_c PQ_K(c, i)^2 + 2 sum_l mean_c RVQ_K(l, c, i)^2 (the second
 * moment of the decoded K coordinate and of its correction, whose fp16
 * roundings the tables skip), row 1 the same for V, row 2 = max_c
 * |PQ_V(c, i)| + sum_l max_c |RVQ_V(l, c, i)| (a bound on |V_i|).  Reads
 * the params' format and codebooks only; depends on nothing else. */
int rfsn_ref_table_stats(const rfsn_ref_params* p, float* stats_dev, void* stream);

/* ---------------------------------------------------------------- k-means
 * One Lloyd update of PQ codebooks (rfsn_v10_mlx_ane_complete.py:197-207):
 * every centroid with members becomes fp16(fp32 mean of its members); empty
 * clusters keep their row.  workspace: rfsn_kmeans_workspace_bytes. */
size_t rfsn_kmeans_workspace_bytes(int32_t M, int32_t C, int32_t d);
int rfsn_kmeans_update(const void* x_dev, int64_t n, int32_t D, int64_t ldx, const uint8_t* codes_dev,
                       int32_t M, int32_t C, void* codebooks_dev, void* workspace_dev,
                       size_t workspace_bytes, void* stream);

/* ---------------------------------------------------------------- cold tier
 * Pinned host pool + asynchronous host-to-device chunk prefetch on a side
 * stream.  Replaces the NPZ chunk files and the router's executor-thread
 * loads (cache.py:134-197, storage.py:113-151, storage.py:203-234). */
int rfsn_host_alloc(size_t bytes, void** ptr_out);
int rfsn_host_free(void* ptr);
typedef struct rfsn_copy {
  void* dst_dev;
  const void* src_host;
  size_t bytes;
} rfsn_copy;
int rfsn_prefetch_h2d(const rfsn_copy* copies, int32_t count, void* stream);
int rfsn_stream_create(void** stream_out);   /* default priority, non-blocking */
int rfsn_stream_destroy(void* stream);
int rfsn_event_create(void** event_out);
int rfsn_event_destroy(void* event);
int rfsn_event_record(void* event, void* stream);
int rfsn_stream_wait_event(void* stream, void* event);
int rfsn_event_synchronize(void* event);
/* 1 when the work recorded before the event has finished, 0 when not yet, <0 on error. */
int rfsn_event_query(void* event);
/* 1 when every operation queued on the stream has finished, 0 when not yet, <0 on error. */
int rfsn_stream_query(void* stream);

/* ---------------------------------------------------------------- measurement
 * A read-only stream over `bytes` (a positive multiple of 16, 16-byte
 * aligned) with `blocks` blocks of 256 threads; out_dev receives one word
 * per block.  No counterpart in the reference: it measures the HBM read
 * ceiling that the decode kernels' roofline fractions are compared with. */
int rfsn_read_stream(const void* src_dev, int64_t bytes, uint32_t* out_dev, int32_t blocks, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* RFSN_ABI_H */
