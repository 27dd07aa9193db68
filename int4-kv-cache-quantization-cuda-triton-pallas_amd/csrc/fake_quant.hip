// INT4 quantize-dequantize ("fake quantization") of keys for quality studies.
//
// The device form of fake_quantize_keys (reference
// scripts/validate_llama.py:126-154): the key tensor a perplexity run hands to
// attention in place of the full-precision keys. For every (sequence b,
// kv-head h, block of `block` positions, channel c), over the block's valid
// rows (the reference pads a partial last block with copies of its last row,
// :145-147, which moves neither extreme):
//   mn, mx = min, max                              (:150-151, exact)
//   scale  = fmaxf(mx - mn, 1e-8f) / 15.0f         (:152, IEEE division: NumPy,
//            torch on the CPU), or with scale_recip
//            fmaxf(mx - mn, 1e-8f) * (1.0f / 15.0f) (what eager torch on a GPU
//            computes for a tensor divided by a Python scalar: it multiplies
//            by the float32 reciprocal, which moves some scales by one ulp)
//   half-up   (:153-154, the script's rule):
//       q  = clamp(floorf((x - mn) / scale + 0.5f), 0, 15)
//       dq = q * scale + mn
//   half-even (the stored scheme: quantize_and_dequantize_ref of
//              src/quantize_int4_ref.py:139-158 applied per block):
//       zp = (-mn) / scale
//       q  = clamp(rintf((x - mn) / scale), 0, 15)
//       dq = q * scale - zp * scale
// each one correctly rounded float32 operation (this file is compiled with
// -ffp-contract=off), then dq is converted to the key type (fp32, fp16 or
// bf16) with round-to-nearest-even. Keys are read as float32 exactly (fp16 and
// bf16 upcasts are exact). Inputs are finite: an infinite or NaN key gives bin
// 0 where the reference's float arithmetic gives NaN.
//
// fake_quant_kernel<KT, RND, NC>: one workgroup of 256 threads per (channel
// slice, block, kv-head, sequence); a slice is cw channels of every row of the
// block (128 bytes of each row by default). Thread t owns the 16-byte vector
// t % VPR of the slice (EPV = 16 / element size channels) in rows t / VPR +
// p * RPP of the block, p < ceil(rows / RPP). The first NC of its vectors stay
// in registers between the min/max pass and the quantize pass; further ones
// (blocks longer than NC * RPP rows) are read again. Keys are read and the
// result written with non-temporal 16-byte accesses (each byte moves once).
// Per-channel extremes meet in LDS. The
// quotient (x - mn) / scale is formed from the channel reciprocal with one FMA
// correction (Markstein), which is the correctly rounded IEEE quotient for
// 0 <= x - mn <= span, scale >= 1e-8 / 15.

#include <limits.h>
#include <stdlib.h>

#include "../../include/fdi4.h"
#include "fdi4_device.hpp"
#include "fdi4_internal.hpp"

namespace fdi4 {

namespace {

constexpr int kFqThreads = 256;
constexpr int kFqMaxD = 512;

// ---- key element types: 16-byte vector <-> float32 ----------------------------

struct F32Key {
  static constexpr int EPV = 4, ESZ = 4;
  static __device__ __forceinline__ void unpack(const U32x4& v, float* f) {
    f[0] = u2f(v.x);
    f[1] = u2f(v.y);
    f[2] = u2f(v.z);
    f[3] = u2f(v.w);
  }
  static __device__ __forceinline__ U32x4 pack(const float* f) {
    return U32x4{f2u(f[0]), f2u(f[1]), f2u(f[2]), f2u(f[3])};
  }
};

struct F16Key {
  static constexpr int EPV = 8, ESZ = 2;
  static __device__ __forceinline__ float lo(unsigned w) {
    return (float)__builtin_bit_cast(_Float16, (unsigned short)(w & 0xFFFFu));
  }
  static __device__ __forceinline__ float hi(unsigned w) {
    return (float)__builtin_bit_cast(_Float16, (unsigned short)(w >> 16));
  }
  static __device__ __forceinline__ unsigned two(float a, float b) {
    // float -> half conversion in the default round-to-nearest-even mode.
    const unsigned ua = __builtin_bit_cast(unsigned short, (_Float16)a);
    const unsigned ub = __builtin_bit_cast(unsigned short, (_Float16)b);
    return ua | (ub << 16);
  }
  static __device__ __forceinline__ void unpack(const U32x4& v, float* f) {
    f[0] = lo(v.x); f[1] = hi(v.x);
    f[2] = lo(v.y); f[3] = hi(v.y);
    f[4] = lo(v.z); f[5] = hi(v.z);
    f[6] = lo(v.w); f[7] = hi(v.w);
  }
  static __device__ __forceinline__ U32x4 pack(const float* f) {
    return U32x4{two(f[0], f[1]), two(f[2], f[3]), two(f[4], f[5]), two(f[6], f[7])};
  }
};

struct BF16Key {
  static constexpr int EPV = 8, ESZ = 2;
  // bf16 is the upper half of a float32.
  static __device__ __forceinline__ unsigned rne(float x) {
    const unsigned u = f2u(x);
    if ((u & 0x7FFFFFFFu) > 0x7F800000u) return 0x7FC0u;  // NaN: canonical quiet NaN
    return (u + 0x7FFFu + ((u >> 16) & 1u)) >> 16;
  }
  static __device__ __forceinline__ unsigned two(float a, float b) { return rne(a) | (rne(b) << 16); }
  static __device__ __forceinline__ void unpack(const U32x4& v, float* f) {
    f[0] = u2f(v.x << 16); f[1] = u2f(v.x & 0xFFFF0000u);
    f[2] = u2f(v.y << 16); f[3] = u2f(v.y & 0xFFFF0000u);
    f[4] = u2f(v.z << 16); f[5] = u2f(v.z & 0xFFFF0000u);
    f[6] = u2f(v.w << 16); f[7] = u2f(v.w & 0xFFFF0000u);
  }
  static __device__ __forceinline__ U32x4 pack(const float* f) {
    return U32x4{two(f[0], f[1]), two(f[2], f[3]), two(f[4], f[5]), two(f[6], f[7])};
  }
};

// Correctly rounded (x - mn) / scale from rc = 1.0f / scale.
__device__ __forceinline__ float fq_quot(float x, float mn, float scale, float rc) {
  const float y = x - mn;
  const float q0 = y * rc;
  return __builtin_fmaf(__builtin_fmaf(-q0, scale, y), rc, q0);
}

template <int RND>
__device__ __forceinline__ float fq_one(float x, float mn, float scale, float rc, float zp) {
  const float t = fq_quot(x, mn, scale, rc);
  if constexpr (RND == FDI4_ROUND_HALF_UP) {
    const float q = fminf(fmaxf(floorf(t + 0.5f), 0.0f), 15.0f);
    return q * scale + mn;
  } else {
    const float q = fminf(fmaxf(rintf(t), 0.0f), 15.0f);
    return q * scale - zp * scale;
  }
}

template <typename KT, int RND, int NC>
__global__ __launch_bounds__(kFqThreads) void fake_quant_kernel(FakeQuantArgs a) {
  constexpr int EPV = KT::EPV;
  // blockIdx.x = block index * nsplit + channel slice; the workgroup owns
  // channels [cs * cw, (cs + 1) * cw) of its block.
  const int cs = blockIdx.x % a.nsplit, blk = blockIdx.x / a.nsplit;
  const int h = blockIdx.y, b = blockIdx.z;
  const int r0 = blk * a.block;
  const int nrows = min(a.block, a.seq_len - r0);  // >= 1: the grid covers ceil(T / block)
  const int tid = threadIdx.x;
  const int vpr = a.vpr, rpp = a.rpp, D = a.cw;
  const int cv = tid % vpr, rsub = tid / vpr;
  const bool active = rsub < rpp;
  const int sweeps = (nrows + rpp - 1) / rpp;

  const int64_t cbyte = (int64_t)cs * a.cw * KT::ESZ + 16 * cv;
  const uint8_t* src = a.k + (int64_t)b * a.k_b + (int64_t)h * a.k_h + (int64_t)r0 * a.k_t + cbyte;
  uint8_t* dst = a.out + (int64_t)b * a.o_b + (int64_t)h * a.o_h + (int64_t)r0 * a.o_t + cbyte;

  float mn[EPV], mx[EPV];
#pragma unroll
  for (int e = 0; e < EPV; ++e) {
    mn[e] = INFINITY;
    mx[e] = -INFINITY;
  }
  // Pass 1: extremes. Rows past the block's end read its last row again (same
  // lines; duplicates move neither extreme).
  U32x4 x[NC];
  float f[EPV];
#pragma unroll
  for (int p = 0; p < NC; ++p) {
    if (active && p < sweeps) {
      const int r = min(rsub + p * rpp, nrows - 1);
      x[p] = ld16_stream(src + (int64_t)r * a.k_t);
      KT::unpack(x[p], f);
#pragma unroll
      for (int e = 0; e < EPV; ++e) {
        mn[e] = fminf(mn[e], f[e]);
        mx[e] = fmaxf(mx[e], f[e]);
      }
    }
  }
  for (int p = NC; active && p < sweeps; ++p) {
    const int r = min(rsub + p * rpp, nrows - 1);
    KT::unpack(ld16_stream(src + (int64_t)r * a.k_t), f);
#pragma unroll
    for (int e = 0; e < EPV; ++e) {
      mn[e] = fminf(mn[e], f[e]);
      mx[e] = fmaxf(mx[e], f[e]);
    }
  }

  // Per-channel extremes across the row slots, then the channel parameters.
  __shared__ float s_mn[kFqThreads * 8], s_mx[kFqThreads * 8];
  __shared__ float s_par[4][kFqMaxD];  // mn, scale, 1/scale, zp
  if (active) {
#pragma unroll
    for (int e = 0; e < EPV; ++e) {
      s_mn[rsub * D + cv * EPV + e] = mn[e];
      s_mx[rsub * D + cv * EPV + e] = mx[e];
    }
  }
  __syncthreads();
  for (int c = tid; c < D; c += kFqThreads) {
    float lo = INFINITY, hi = -INFINITY;
    for (int j = 0; j < rpp; ++j) {
      lo = fminf(lo, s_mn[j * D + c]);
      hi = fmaxf(hi, s_mx[j * D + c]);
    }
    const float span = fmaxf(hi - lo, 1e-8f);
    const float sc = a.scale_recip ? span * (1.0f / 15.0f) : span / 15.0f;
    s_par[0][c] = lo;
    s_par[1][c] = sc;
    s_par[2][c] = 1.0f / sc;
    s_par[3][c] = (-lo) / sc;
  }
  __syncthreads();
  if (!active) return;

  float cmn[EPV], csc[EPV], crc[EPV], czp[EPV];
#pragma unroll
  for (int e = 0; e < EPV; ++e) {
    const int c = cv * EPV + e;
    cmn[e] = s_par[0][c];
    csc[e] = s_par[1][c];
    crc[e] = s_par[2][c];
    czp[e] = s_par[3][c];
  }

  // Pass 2: bins and dequantized values.
  float o[EPV];
#pragma unroll
  for (int p = 0; p < NC; ++p) {
    const int r = rsub + p * rpp;
    if (p < sweeps && r < nrows) {
      KT::unpack(x[p], f);
#pragma unroll
      for (int e = 0; e < EPV; ++e) o[e] = fq_one<RND>(f[e], cmn[e], csc[e], crc[e], czp[e]);
      st16_stream(dst + (int64_t)r * a.o_t, KT::pack(o));
    }
  }
  for (int p = NC; p < sweeps; ++p) {
    const int r = rsub + p * rpp;
    if (r >= nrows) break;
    KT::unpack(ld16_stream(src + (int64_t)r * a.k_t), f);
#pragma unroll
    for (int e = 0; e < EPV; ++e) o[e] = fq_one<RND>(f[e], cmn[e], csc[e], crc[e], czp[e]);
    st16_stream(dst + (int64_t)r * a.o_t, KT::pack(o));
  }
}

template <typename KT, int RND>
hipError_t launch_typed(const FakeQuantArgs& a, dim3 grid, hipStream_t st) {
  const int sweeps = (min(a.block, a.seq_len) + a.rpp - 1) / a.rpp;
  const dim3 blk(kFqThreads);
  if (sweeps <= 4)
    hipLaunchKernelGGL((fake_quant_kernel<KT, RND, 4>), grid, blk, 0, st, a);
  else if (sweeps <= 8)
    hipLaunchKernelGGL((fake_quant_kernel<KT, RND, 8>), grid, blk, 0, st, a);
  else if (sweeps <= 16)
    hipLaunchKernelGGL((fake_quant_kernel<KT, RND, 16>), grid, blk, 0, st, a);
  else
    hipLaunchKernelGGL((fake_quant_kernel<KT, RND, 32>), grid, blk, 0, st, a);
  return hipGetLastError();
}

template <typename KT>
hipError_t launch_rounding(const FakeQuantArgs& a, int rounding, dim3 grid, hipStream_t st) {
  return rounding == FDI4_ROUND_HALF_UP ? launch_typed<KT, FDI4_ROUND_HALF_UP>(a, grid, st)
                                        : launch_typed<KT, FDI4_ROUND_HALF_EVEN>(a, grid, st);
}


}  // namespace

int fake_quant_max_head_dim() { return kFqMaxD; }

// The caller has checked: head_dim * element size a multiple of 16 and
// head_dim <= kFqMaxD, 16-byte aligned base and strides, block >= 1,
// seq_len >= 1, heads and batch <= 65535.
hipError_t launch_fake_quant(const FakeQuantArgs& args, int key_dtype, int rounding, int batch,
                             int heads, hipStream_t st) {
  FakeQuantArgs a = args;
  const int esz = key_dtype == FDI4_K_F32 ? 4 : 2;
  const int64_t nblk = ((int64_t)a.seq_len + a.block - 1) / a.block;
  // Channel slices of 128 bytes per row (one cache line): on MI355X they
  // beat whole rows and narrower slices for float32 and float16 keys at
  // head_dim 64 and 128 (8 x 32 x 2048 x 128 float32 in 128-row blocks:
  // 93 us against 103 us for whole rows and 96 us for 256-byte slices; a
  // Llama-2-7B window, 32 x 2048 x 128 float16 in 256-row blocks: 11.4 us
  // against 15.2 and 12.2 us). FDI4_TUNE_FAKE_QUANT_SPLIT overrides it.
  const int row_bytes = a.head_dim * esz;
  const int forced = tuning(FDI4_TUNE_FAKE_QUANT_SPLIT);
  int split = forced > 0 ? forced : (row_bytes >= 128 ? row_bytes / 128 : 1);
  while (split > 1 && (a.head_dim % split || (a.head_dim / split * esz) % 16 ||
                       nblk * split > INT32_MAX))
    --split;
  a.nsplit = max(split, 1);
  a.cw = a.head_dim / a.nsplit;
  a.vpr = a.cw * esz / 16;
  a.rpp = kFqThreads / a.vpr;
  const dim3 grid((unsigned)(nblk * a.nsplit), (unsigned)heads, (unsigned)batch);
  switch (key_dtype) {
    case FDI4_K_F32: return launch_rounding<F32Key>(a, rounding, grid, st);
    case FDI4_K_F16: return launch_rounding<F16Key>(a, rounding, grid, st);
    default: return launch_rounding<BF16Key>(a, rounding, grid, st);
  }
}

}  // namespace fdi4
