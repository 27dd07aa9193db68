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

// Valid rows of sequence b (every sequence spans max_pages pages when no
// lengths are given).
__device__ __forceinline__ int seq_len_of(const DecodeArgs& a, int b) {
  return a.seq_lens ? max(a.seq_lens[b], 0) : a.max_pages * a.page_rows;
}

// exp(x) for x <= ~0 in double: the exponent x*log2(e) is formed in double,
// rounded once to float (relative 2^-24, so 6e-8 absolute where |x| < 1, where
// the terms that matter lie) and raised with the hardware 2^y (v_exp_f32, ~1
// ulp); -inf gives 0.
__device__ __forceinline__ float exp2_of(double x) {
  return __builtin_amdgcn_exp2f((float)(x * 1.4426950408889634));
}

}  // namespace fdi4
