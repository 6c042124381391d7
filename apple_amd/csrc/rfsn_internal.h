// Declarations shared between the library's translation units (not ABI).
#pragma once

#include "rfsn_common.h"

namespace rfsn {

int launch_merge(const float* partial, int64_t bh, int splits, int D, void* out, hipStream_t s);

// ---- score tables of rfsn_ref_attention (ref_tables.hip) ----
// Codebook entries of the tables: M PQ sections of C entries, then L gated
// layers of Cr (E in all), cut into nch chunks of at most 64 within
// sections; tables and sums live in chunk space, Ep = 64 nch slots (each
// section padded to a multiple of 64).
struct RefTabGeom {
  int D, M, C, L, Cr, dsub, cpq, crv, E, Ep, nch;
};
// Workspace of a score-table call: the exact pass's split partials with one
// more slot per query head (the tables' slot, the last), the drift
// estimates, the tables, the histogram blocks' statistics and sums
// (chunk-major), and the chunk products.
struct RefTabLayout {
  float* partial;
  float* est;
  float* tab;
  float* pst;
  float* part;
  float* part2;
  int slots;
  int hist_splits;
};
RefTabGeom ref_tab_geom(const rfsn_ref_params* p);
bool ref_tables_shape_ok(const rfsn_ref_params* p);
int ref_tab_hist_splits(const rfsn_ref_params* p);
// bytes of the workspace (and, with w, its layout at base)
size_t ref_tab_bytes(const rfsn_ref_params* p, int slots, RefTabLayout* w, void* base);
// the four table launches; the exact pass and the merge follow
int launch_ref_tables(const rfsn_ref_params* p, const RefTabLayout& w, hipStream_t s);

}  // namespace rfsn
