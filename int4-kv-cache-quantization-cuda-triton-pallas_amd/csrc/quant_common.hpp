// Quantizer arithmetic shared by the quantizer kernels (quantize.hip) and
// the decode kernel's fused serving step (decode.hip): the bin and scale
// formulas, bit-exact with the NumPy quantizer (reference
// src/quantize_int4_ref.py:46-84), and the re-quantization of a sequence's
// open scale group by one workgroup of any size.
#pragma once

#include "fdi4_device.hpp"
#include "fdi4_internal.hpp"

namespace fdi4 {

__device__ __forceinline__ unsigned quant_bin(float x, float mn, float scale) {
  float b = rintf((x - mn) / scale);
  b = fminf(fmaxf(b, 0.0f), 15.0f);
  return (unsigned)b;
}

// The same bin with the division done from the reciprocal rc = 1.0f / scale
// (one IEEE division per channel): q0 = y * rc, then one FMA residual step
// q = fma(fma(-q0, scale, y), rc, q0) yields the correctly rounded quotient
// RN(y / scale) (Markstein's correction: rc is the correctly rounded
// reciprocal, the residual y - q0 * scale is exact under FMA, and no
// intermediate under- or overflows for 0 <= y <= span and scale >= 1e-8/15).
// Infinite or NaN inputs give a NaN quotient and bin 0, as the division does.
__device__ __forceinline__ float quant_bin_rc(float x, float mn, float scale, float rc) {
  const float y = x - mn;
  const float q0 = y * rc;
  const float q = __builtin_fmaf(__builtin_fmaf(-q0, scale, y), rc, q0);
  return fminf(fmaxf(rintf(q), 0.0f), 15.0f);
}

__device__ __forceinline__ void scale_zp(float mn, float mx, float* s, float* z) {
  const float span = fmaxf(mx - mn, 1e-8f);
  *s = span / 15.0f;
  *z = (-mn) / *s;
}

// Largest scale group a fused serving step re-quantizes.
constexpr int kStepMaxGroup = 256;

// Word 3 of a raw buffer resource on gfx9 parts (untyped 32-bit data): with
// stride 0, a load at or past num_records bytes returns zeros and touches no
// memory.
constexpr int kBufferRsrcWord3 = 0x00020000;

// One quarter of the fused serving step's append, by one wave (lane
// 0..63): token t of (sequence b, kv-head h) is appended and its open group
// g = t / group_rows re-quantized over the group's t % group_rows + 1 rows,
// for channels [slice * D / 4, (slice + 1) * D / 4). Four waves with slices
// 0..3 make the whole append with no workgroup barrier; the other waves of
// the workgroup decode meanwhile. Each quarter: the slice of the group's rows
// in registers (batches of 16-byte loads, all of a batch in flight; rows
// 0..rnew-1 from the staging rows through a range-checked buffer load, which
// reads zeros past them without touching memory, replaced by the new row,
// row rnew), per-channel min/max by a lane butterfly, the slice's scale and
// zero-point, and the slice's D / 8 bytes of every packed row of the group
// (built in LDS, k_open, then stored with one store per row). The arithmetic
// is that of the grouped quantizer (quant_bin_rc, scale_zp), so the stored
// bytes equal the append kernel's. The slice's share of the new key row goes
// to the staging rows and its share of the new value row to the value page.
// The group's packed rows (row r at byte r * D / 2 of k_open), scale and
// zero-point (scale of channel d at d, zero-point at D + d) and the new value
// row are also left in the workgroup's LDS, k_open, sz_open and v_open; the
// caller publishes them to the other waves once its LDS writes are done.
// The stores to the cache are issued, not awaited: until the kernel ends the
// workgroup reads the open group's keys and scales and the new value row
// from LDS, never from the cache. pt_w: this wave's own LDS scratch of
// kStepMaxGroup ints (the group's page-table entries). k_pages/v_pages and
// the scales are the cache's (byte and element strides as in DecodeArgs;
// the group's rows lie in mapped pages).
template <int D, int VEB>
__device__ __forceinline__ void step_requant_slice(const StepAppend& s, uint8_t* k_pages,
                                                   int64_t kp_page, int64_t kp_head,
                                                   int64_t kp_row, uint8_t* v_pages,
                                                   int64_t vp_page, int64_t vp_head,
                                                   int64_t vp_row, float* k_scale, float* k_zp,
                                                   int64_t s_b, int64_t s_h, int64_t s_g,
                                                   const int32_t* page_table, int64_t pt_b,
                                                   int page_rows, int num_pages, int b, int h,
                                                   int t, int slice, int lane, uint16_t* k_open,
                                                   float* sz_open, U32x4* v_open, int* pt_w) {
  constexpr int DS = D / 4;            // channels of the slice
  constexpr int LPR = DS / 4;          // lanes per row (16 bytes = 4 channels each)
  constexpr int RPL = 64 / LPR;        // rows per wave-wide load
  constexpr int NI = kStepMaxGroup / RPL;   // row slots per lane, at most
  // Slots per batch: 16 (64 registers), 8 at D = 256, where the decode's
  // first chunk takes more of them meanwhile.
  constexpr int NBM = D == 256 ? 8 : 16;
  constexpr int NB = NI < NBM ? NI : NBM;
  constexpr int NBATCH = NI / NB;
  constexpr int VPS = D * VEB / 64;    // 16-byte pieces of the slice's value bytes
  static_assert(LPR >= 1 && 64 % LPR == 0 && NI % NB == 0 && VPS <= 64, "layout");
  const int cq = lane % LPR, rsub = lane / LPR;
  const int ch = slice * DS + 4 * cq;  // first channel of this lane
  const int G = s.group_rows;
  const int g = t / G, rnew = t - g * G, r0 = g * G;
  const int npg = rnew / page_rows + 1;     // pages holding rows 0..rnew
  const float* knew = s.k_new + (int64_t)b * s.kn_b + (int64_t)h * s.kn_h;
  float* stage = s.stage + (int64_t)b * s.st_b + (int64_t)h * s.st_h;
  const __amdgpu_buffer_rsrc_t srows = __builtin_amdgcn_make_buffer_rsrc(
      stage, (short)0, (int)((int64_t)rnew * s.st_r * 4), kBufferRsrcWord3);
  const float4 kcopy = *reinterpret_cast<const float4*>(knew + ch);
  // Slot i of batch bt holds row rsub + (bt * NB + i) * RPL as loaded (zeros
  // at and past row rnew); val() gives the row's keys, the new row's for rows
  // rnew and beyond (which leaves the min/max unchanged).
  float4 x[NB];
  auto load_batch = [&](int bt) {
#pragma unroll
    for (int i = 0; i < NB; ++i) {
      const int r = rsub + (bt * NB + i) * RPL;
      const auto v = __builtin_amdgcn_raw_buffer_load_b128(
          srows, (int)((int64_t)r * s.st_r * 4) + 4 * ch, 0, 0);
      x[i] = make_float4(__uint_as_float(v[0]), __uint_as_float(v[1]), __uint_as_float(v[2]),
                         __uint_as_float(v[3]));
    }
  };
  auto val = [&](int bt, int i) -> float4 {
    return rsub + (bt * NB + i) * RPL < rnew ? x[i] : kcopy;
  };
  auto minmax = [&](int bt, float* mn, float* mx) {
#pragma unroll
    for (int i = 0; i < NB; ++i) {
      const float4 y = val(bt, i);
      mn[0] = fminf(mn[0], y.x); mx[0] = fmaxf(mx[0], y.x);
      mn[1] = fminf(mn[1], y.y); mx[1] = fmaxf(mx[1], y.y);
      mn[2] = fminf(mn[2], y.z); mx[2] = fmaxf(mx[2], y.z);
      mn[3] = fminf(mn[3], y.w); mx[3] = fmaxf(mx[3], y.w);
    }
  };
  // One memory round: the first batch of rows, this slice's piece of the
  // new value row and the group's page-table entries (lane j: page j) are
  // all in flight before anything waits for them.
  load_batch(0);
  const uint8_t* vsrc = s.v_new + (int64_t)b * s.vn_b + (int64_t)h * s.vn_h;
  const int vpc = slice * VPS + min(lane, VPS - 1);
  const U32x4 vcopy = ld16(vsrc + 16 * vpc);
  const int64_t pt0 = (int64_t)b * pt_b + r0 / page_rows;
  int pg = r0 / page_rows + lane;
  if (page_table && lane < npg) pg = page_table[pt0 + lane];
  if (lane < npg) pt_w[lane] = min(max(pg, 0), num_pages - 1);
  // Groups of more than 64 pages (pages of fewer than four rows).
  for (int j = lane + 64; j < npg; j += 64) {
    const int pj = page_table ? page_table[pt0 + j] : r0 / page_rows + j;
    pt_w[j] = min(max(pj, 0), num_pages - 1);
  }

  float mn[4], mx[4];
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    mn[k] = INFINITY;
    mx[k] = -INFINITY;
  }
  minmax(0, mn, mx);
  const int nbu = rnew / (NB * RPL) + 1;   // batches holding rows 0..rnew
  if constexpr (NBATCH > 1) {
#pragma unroll 1
    for (int bt = 1; bt < nbu; ++bt) {
      load_batch(bt);
      minmax(bt, mn, mx);
    }
  }
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    mn[k] = allreduce_min_f<LPR, 64>(mn[k]);
    mx[k] = allreduce_max_f<LPR, 64>(mx[k]);
  }
  float sc[4], zp[4], rc[4];
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    scale_zp(mn[k], mx[k], &sc[k], &zp[k]);
    rc[k] = 1.0f / sc[k];
  }
  if (rsub == 0) {
    const int64_t so = (int64_t)b * s_b + (int64_t)h * s_h + (int64_t)g * s_g + ch;
    *reinterpret_cast<float4*>(k_scale + so) = make_float4(sc[0], sc[1], sc[2], sc[3]);
    *reinterpret_cast<float4*>(k_zp + so) = make_float4(zp[0], zp[1], zp[2], zp[3]);
    *reinterpret_cast<float4*>(sz_open + ch) = make_float4(sc[0], sc[1], sc[2], sc[3]);
    *reinterpret_cast<float4*>(sz_open + D + ch) = make_float4(zp[0], zp[1], zp[2], zp[3]);
    *reinterpret_cast<float4*>(stage + (int64_t)rnew * s.st_r + ch) = kcopy;
  }
  // pt_w was written by this wave's lanes; make it visible to all of them.
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  if (lane < VPS) {
    st16(v_pages + (int64_t)pt_w[rnew / page_rows] * vp_page + (int64_t)h * vp_head +
             (int64_t)(t % page_rows) * vp_row + 16 * vpc,
         vcopy);
    v_open[vpc] = vcopy;
  }

  // Bins of the valid rows: this lane's 4 channels of each of its rows, two
  // bytes of the packed row, into k_open. The last batch is still in
  // registers; earlier ones (groups of more rows than one batch) are loaded
  // again.
#pragma unroll 1
  for (int bt = nbu - 1; bt >= 0; --bt) {
    if (NBATCH > 1 && bt != nbu - 1) load_batch(bt);
#pragma unroll
    for (int i = 0; i < NB; ++i) {
      const int r = rsub + (bt * NB + i) * RPL;
      if (r <= rnew) {
        const float4 y = val(bt, i);
        const float n0 = quant_bin_rc(y.x, mn[0], sc[0], rc[0]);
        const float n1 = quant_bin_rc(y.y, mn[1], sc[1], rc[1]);
        const float n2 = quant_bin_rc(y.z, mn[2], sc[2], rc[2]);
        const float n3 = quant_bin_rc(y.w, mn[3], sc[3], rc[3]);
        const uint16_t pk = (uint16_t)(unsigned)__builtin_fmaf(
            n3, 4096.0f, __builtin_fmaf(n2, 256.0f, __builtin_fmaf(n1, 16.0f, n0)));
        k_open[r * (D / 4) + ch / 4] = pk;
      }
    }
  }
  // The slice's D / 8 bytes of every packed row, gathered from k_open: one
  // store of up to 16 bytes per row and piece (lane j: row j, j + 64, ...),
  // instead of one 2-byte store per lane and row.
  constexpr int SB = D / 8;
  constexpr int PB = SB < 16 ? SB : 16;
  constexpr int PPR = SB / PB;
  static_assert(PB == 8 || PB == 16, "piece");
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  for (int j = lane; j < (rnew + 1) * PPR; j += 64) {
    const int r = j / PPR, off = slice * SB + (j % PPR) * PB;
    const uint8_t* src = reinterpret_cast<const uint8_t*>(k_open) + r * (D / 2) + off;
    uint8_t* dst = k_pages + (int64_t)pt_w[r / page_rows] * kp_page + (int64_t)h * kp_head +
                   (int64_t)((r0 + r) % page_rows) * kp_row + off;
    if constexpr (PB == 16) {
      st16(dst, *reinterpret_cast<const U32x4*>(src));
    } else {
      *reinterpret_cast<uint2*>(dst) = *reinterpret_cast<const uint2*>(src);
    }
  }
}

}  // namespace fdi4
