// Pieces shared by the paged decode kernels (decode.hip, decode_gqa.hip):
// packed key row loads and the per-chunk page metadata.
#pragma once

#include "fdi4_device.hpp"
#include "fdi4_internal.hpp"

namespace fdi4 {

template <int KW>
struct KVec {
  unsigned w[KW];
};

template <int KW>
__device__ __forceinline__ KVec<KW> load_k(const uint8_t* p) {
  KVec<KW> r;
  if constexpr (KW == 4) {
    const U32x4 v = ld16_stream(p);
    r.w[0] = v.x; r.w[1] = v.y; r.w[2] = v.z; r.w[3] = v.w;
  } else if constexpr (KW == 2) {
    const uint2 v = ld8_stream(p);
    r.w[0] = v.x; r.w[1] = v.y;
  } else {
    static_assert(KW == 1, "KW");
    r.w[0] = __builtin_nontemporal_load(reinterpret_cast<const unsigned*>(p));
  }
  return r;
}

struct ChunkMeta {
  int64_t phys;
  int r0;
  int nval;
  int group;
};

__device__ __forceinline__ ChunkMeta chunk_meta(const DecodeArgs& a, int b, int T, int cpp,
                                                int c) {
  ChunkMeta m;
  const int lp = c / cpp;
  const int j = c - lp * cpp;
  int rows;
  if (a.page_lens) {
    rows = min(max(a.page_lens[(int64_t)b * a.pl_b + lp], 0), a.page_rows);
  } else {
    rows = min(a.page_rows, T - lp * a.page_rows);
  }
  m.r0 = j * 16;
  m.nval = min(16, rows - m.r0);
  const int pg = a.page_table ? a.page_table[(int64_t)b * a.pt_b + lp] : lp;
  m.phys = (int64_t)min(max(pg, 0), a.num_pages - 1);
  m.group = lp / a.pages_per_group;
  return m;
}

}  // namespace fdi4
