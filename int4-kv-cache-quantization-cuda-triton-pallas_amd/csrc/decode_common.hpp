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

// One element of a query or output tensor of type dt (EDtype), as float32:
// float16 and bfloat16 widen exactly.
__device__ __forceinline__ float load_elem(const void* p, int64_t i, int dt) {
  if (dt == kEF32) return static_cast<const float*>(p)[i];
  const unsigned short u = static_cast<const unsigned short*>(p)[i];
  if (dt == kEF16) return (float)__builtin_bit_cast(_Float16, u);
  return __uint_as_float((unsigned)u << 16);
}

// float32 -> bfloat16 bits, round to nearest even; NaN becomes the canonical
// quiet NaN 0x7FC0 (as torch's conversion gives).
__device__ __forceinline__ unsigned short bf16_rne(float x) {
  const unsigned u = __float_as_uint(x);
  if ((u & 0x7FFFFFFFu) > 0x7F800000u) return (unsigned short)0x7FC0u;
  return (unsigned short)((u + 0x7FFFu + ((u >> 16) & 1u)) >> 16);
}

// Store x into element i of an output tensor of type dt, rounded to nearest
// even for the 16-bit types.
__device__ __forceinline__ void store_elem(void* p, int64_t i, int dt, float x) {
  if (dt == kEF32) {
    static_cast<float*>(p)[i] = x;
  } else if (dt == kEF16) {
    static_cast<_Float16*>(p)[i] = (_Float16)x;
  } else {
    static_cast<unsigned short*>(p)[i] = bf16_rne(x);
  }
}

// Four values packed in 16 bytes of a value row as float32: float32 (4
// channels), float16 or bfloat16 (8 channels, two per 32-bit word).
template <int VDT>
__device__ __forceinline__ void widen_values(const U32x4& v, float* f) {
  if constexpr (VDT == kVF32) {
    f[0] = u2f(v.x); f[1] = u2f(v.y); f[2] = u2f(v.z); f[3] = u2f(v.w);
  } else {
    const unsigned u[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      if constexpr (VDT == kVF16) {
        f[2 * k] = (float)__builtin_bit_cast(_Float16, (unsigned short)(u[k] & 0xFFFFu));
        f[2 * k + 1] = (float)__builtin_bit_cast(_Float16, (unsigned short)(u[k] >> 16));
      } else {
        f[2 * k] = __uint_as_float(u[k] << 16);
        f[2 * k + 1] = __uint_as_float(u[k] & 0xFFFF0000u);
      }
    }
  }
}

// Element i of a read-only int32 kernel input (page table, page lengths,
// sequence lengths) through the constant address space: at a wave-uniform
// index a scalar-unit load, also in a kernel that stores to the cache before
// its chunk loop (the fused serving step), where the compiler would otherwise
// treat the arrays as possibly overwritten and load them as vectors, each
// load followed by a full vmcnt drain.
__device__ __forceinline__ int ld_ro(const int32_t* p, int64_t i) {
  return ((const __attribute__((address_space(4))) int32_t*)p)[i];
}

struct ChunkMeta {
  int64_t phys;
  int r0;
  int nval;
  int group;
  int tok0;        // logical row of the chunk's first row
};

__device__ __forceinline__ ChunkMeta chunk_meta(const DecodeArgs& a, int b, int T, int cpp,
                                                int c) {
  ChunkMeta m;
  const int lp = c / cpp;
  const int j = c - lp * cpp;
  int rows;
  if (a.page_lens) {
    rows = min(max(ld_ro(a.page_lens, (int64_t)b * a.pl_b + lp), 0), a.page_rows);
  } else {
    rows = min(a.page_rows, T - lp * a.page_rows);
  }
  m.r0 = j * 16;
  m.nval = min(16, rows - m.r0);
  const int pg = a.page_table ? ld_ro(a.page_table, (int64_t)b * a.pt_b + lp) : lp;
  m.phys = (int64_t)min(max(pg, 0), a.num_pages - 1);
  m.group = lp / a.pages_per_group;
  m.tok0 = lp * a.page_rows + m.r0;
  return m;
}

// Valid rows of sequence b, clamped to the max_pages * page_rows the cache
// holds (the host checks that this product fits in 32 bits), so no count
// derived from a length overflows; every sequence spans max_pages pages when
// no lengths are given.
__device__ __forceinline__ int seq_len_of(const DecodeArgs& a, int b) {
  const int cap = a.max_pages * a.page_rows;
  return a.seq_lens ? min(max(ld_ro(a.seq_lens, b), 0), cap) : cap;
}

// The serving step's length hand-back, at the end of the decode: workgroup
// (split 0, first head group) of sequence b copies the length it read to
// lens_out[b]. No workgroup of the decode reads lens_out, a different array
// from seq_lens (the host checks both). (At the start of the kernel the
// store would make the compiler treat the page-table reads of the chunk loop
// as possibly clobbered and turn them into vector loads.)
__device__ __forceinline__ void hand_back_length(const DecodeArgs& a, int b) {
  if (a.lens_out && blockIdx.x == 0 && blockIdx.y == 0 && threadIdx.x == 0)
    a.lens_out[b] = a.seq_lens[b];
}

// Logical pages holding the first T rows (T <= max_pages * page_rows).
__device__ __forceinline__ int pages_of(const DecodeArgs& a, int T) {
  return T / a.page_rows + (T % a.page_rows != 0);
}

// Chunks of wave w of `waves` (4 or 8) over the chunks [begin, end) of a
// split, as one contiguous range per wave. Wave w runs on SIMD w % 4; every
// SIMD takes span / 4 consecutive chunks (the first span % 4 SIMDs one more).
// With eight waves, waves w and w + 4 share a SIMD, and the older wave w is
// issued ahead of w + 4: with equal ranges at B8 H32 D128 T2048 (16 chunks
// each), waves 0-3 finished their loops 6.5 us before waves 4-7 (38.6 against
// 45.1 us), leaving one wave per SIMD, with half the loads in flight, for the
// rest of the decode. The older wave therefore takes kFirstShare32 / 32 of
// its SIMD's chunks (rounded to nearest) and the younger one the rest; the
// per-head decode with float32 values at D = 128 (512-byte value rows) gives
// it kFirstShare32F32 / 32. In-process A/B against 18/32, one box, eight
// waves: B8 H32 T2048 -0.8 to -1.1 %, T1024 -2 %, T8192 -0.5 %, B32 H32
// T2048 -0.8 %, B64 H32 T4096 -0.3 %, ragged B32 within 0.5 %; slower with
// other rows: float16 values at D = 128 +1.5 %, float32 at D = 64 +3 %, at
// D = 256 +0.6 %; 16/32 slower everywhere.
#ifndef FDI4_FIRST_SHARE32
#define FDI4_FIRST_SHARE32 18
#endif
constexpr int kFirstShare32 = FDI4_FIRST_SHARE32;
#ifndef FDI4_FIRST_SHARE32_F32
#define FDI4_FIRST_SHARE32_F32 20
#endif
constexpr int kFirstShare32F32 = FDI4_FIRST_SHARE32_F32;

struct WaveRange {
  int c0, c1;      // the wave's chunks [c0, c1)
};

__device__ __forceinline__ WaveRange wave_chunks(int begin, int end, int w, int waves) {
  const int span = max(end - begin, 0);
  const int simds = min(waves, 4);
  const int s = w % simds;
  const int base = span / simds, rem = span - base * simds;
  WaveRange r;
  r.c0 = begin + s * base + min(s, rem);
  const int n = base + (s < rem ? 1 : 0);
  r.c1 = r.c0 + n;
  if (waves > simds) {
    const int first = (n * kFirstShare32 + 16) / 32;
    if (w < simds) r.c1 = r.c0 + first;
    else r.c0 += first;
  }
  return r;
}

// The decode kernel's (decode_kernel) chunks of wave w of `waves` (4 or 8)
// over the chunks [begin, end) of a split, as up to two segments, each with
// an online-softmax partial of its own (LDS slot s1, and s2 when s2 >= 0).
// SIMD s = w % 4 takes the same consecutive chunks [S, E) as in wave_chunks
// (n of them). With four waves that is the wave's one segment (slot w). With
// eight, [S, E) is cut into three ranges: A = the first (n * first32 + 16) /
// 32 chunks, C = the last (n * kTailShare32 + 16) / 32 of the rest, B
// between; A's partial goes to slot s, B's to 4 + s, C's to 8 + s (12 slots,
// merged in slot order). The older wave w < 4 takes A, the younger wave w + 4
// takes B; C goes to the younger wave (then its segments B, C are contiguous)
// unless `lend_tail`, when the older wave takes it after A. A wave's partial
// for a range is the same whichever wave computes it, so the two assignments
// give the same bits; the serving step (whose younger waves first
// re-quantize the open group) lends C to the older waves.
#ifndef FDI4_TAIL_SHARE32
#define FDI4_TAIL_SHARE32 2
#endif
constexpr int kTailShare32 = FDI4_TAIL_SHARE32;

struct WaveSegs {
  int p0, p1;      // segment 1: chunks [p0, p1), partial in slot s1
  int q0, q1;      // segment 2: chunks [q0, q1), partial in slot s2
  int s1, s2;      // s2 < 0: no segment 2 (q0 == q1)
};

__device__ __forceinline__ WaveSegs wave_segments(int begin, int end, int w, int waves,
                                                  bool lend_tail, int first32) {
  const int span = max(end - begin, 0);
  const int simds = min(waves, 4);
  const int s = w % simds;
  const int base = span / simds, rem = span - base * simds;
  const int S = begin + s * base + min(s, rem);
  const int n = base + (s < rem ? 1 : 0);
  const int E = S + n;
  WaveSegs r;
  if (waves <= simds) {
    r.p0 = S; r.p1 = E; r.q0 = r.q1 = E; r.s1 = w; r.s2 = -1;
    return r;
  }
  const int first = (n * first32 + 16) / 32;
  const int tail = min((n * kTailShare32 + 16) / 32, n - first);
  const int a1 = S + first, c0 = E - tail;
  if (w < simds) {
    r.p0 = S; r.p1 = a1; r.s1 = s;
    if (lend_tail) { r.q0 = c0; r.q1 = E; } else { r.q0 = r.q1 = E; }
  } else {
    r.p0 = a1; r.p1 = c0; r.s1 = 4 + s;
    if (lend_tail) { r.q0 = r.q1 = E; } else { r.q0 = c0; r.q1 = E; }
  }
  // C's partial is written by the wave that owns C, also when C is empty.
  r.s2 = ((w >= simds) != lend_tail) ? 8 + s : -1;
  return r;
}

// exp(x) for x <= ~0 in double: the exponent x*log2(e) is formed in double,
// rounded once to float (relative 2^-24, so 6e-8 absolute where |x| < 1, where
// the terms that matter lie) and raised with the hardware 2^y (v_exp_f32, ~1
// ulp); -inf gives 0.
__device__ __forceinline__ float exp2_of(double x) {
  return __builtin_amdgcn_exp2f((float)(x * 1.4426950408889634));
}

}  // namespace fdi4
