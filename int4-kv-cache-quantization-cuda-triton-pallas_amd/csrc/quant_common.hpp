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

// Appends token t of (sequence b, kv-head h) and re-quantizes its open group
// g = t / group_rows over the group's t % group_rows + 1 rows, with the
// workgroup's NT threads: the key row goes to the staging rows, the value row
// to its page; the group's rows are held in registers (16-byte loads, all in
// flight at once), per-channel min/max by a lane butterfly then LDS across
// waves, the group's scale and zero-point, and the packed rows of the group
// to their pages. The arithmetic is that of the grouped quantizer
// (quant_bin_rc, scale_zp), so the stored bytes equal the append kernel's.
// k_pages/v_pages and the scales are the cache's (byte and element strides
// as in DecodeArgs; the group's rows lie in mapped pages). The group's packed
// rows (row r at byte r * D / 2), its scale and zero-point (scale of channel
// d at d, zero-point at D + d) and the new value row are also left in the
// workgroup's LDS, k_open, sz_open and v_open, visible to every wave on
// return. The stores to the cache are issued, not awaited: until the kernel
// ends, the workgroup reads the open group's keys and scales and the new
// value row from LDS, never from the cache.
//
// issue() is called once, right after this function's own loads of the
// first batch of rows, the new rows and the group's page-table entries: the
// caller's loads issued there stay in flight while the rows are reduced.
// Every load and store issued after issue() is unconditional and their
// number fixed (indices past the data are clamped, and repeated stores write
// equal bytes to the same place), so a wait for the caller's loads counts
// exactly the memory operations issued after them instead of draining them
// all.
template <int D, int NT, int VEB, typename Issue>
__device__ __forceinline__ void step_requant(Issue&& issue, const StepAppend& s, uint8_t* k_pages,
                                             int64_t kp_page, int64_t kp_head, int64_t kp_row,
                                             uint8_t* v_pages, int64_t vp_page, int64_t vp_head,
                                             int64_t vp_row, float* k_scale, float* k_zp,
                                             int64_t s_b, int64_t s_h, int64_t s_g,
                                             const int32_t* page_table, int64_t pt_b,
                                             int page_rows, int num_pages, int b, int h, int t,
                                             uint16_t* k_open, float* sz_open, U32x4* v_open) {
  constexpr int VPR = D / 4;          // threads per staged row (16 bytes each)
  constexpr int RPI = NT / VPR;       // rows per sweep of the workgroup
  constexpr int NI = kStepMaxGroup / RPI;   // rows per thread, at most
  constexpr int RB = D / 2;           // packed bytes per row
  constexpr int PPR = RB / 16;        // 16-byte pieces per packed row
  constexpr int VPC = D * VEB / 16;   // 16-byte pieces of a value row
  constexpr int NWAVE = NT / 64;
  static_assert(VPR <= 64 && NT % VPR == 0 && kStepMaxGroup % RPI == 0, "layout");
  static_assert(VPC <= NT, "one value piece per thread");
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int cq = tid % VPR, rsub = tid / VPR;
  const int G = s.group_rows;
  const int g = t / G, rnew = t - g * G, r0 = g * G;
  const int npg = rnew / page_rows + 1;   // pages of the group holding rows 0..rnew
  const float* knew = s.k_new + (int64_t)b * s.kn_b + (int64_t)h * s.kn_h;
  const uint8_t* vsrc = s.v_new + (int64_t)b * s.vn_b + (int64_t)h * s.vn_h;
  float* stage = s.stage + (int64_t)b * s.st_b + (int64_t)h * s.st_h;
  __shared__ int pt_grp[kStepMaxGroup];
  __shared__ float4 q_mn[NWAVE][VPR], q_mx[NWAVE][VPR];

  // The group's rows 0..rnew in batches of NB rows per thread, each batch's
  // loads in flight together; with one batch the rows stay in registers for
  // the bins, otherwise the bins re-read them (from the L2). 16 rows per
  // thread in a batch with eight waves at D <= 128, 8 otherwise (the
  // decode's first chunk is in registers meanwhile; more would spill). Rows
  // 0..rnew-1 come from the staging rows through a range-checked buffer load:
  // a row at or past rnew reads zeros without touching memory, and is
  // replaced by the new row (row rnew itself; the rows past it repeat it, so
  // they leave the min/max unchanged). The loads are unconditional: under a
  // branch, waits for anything issued after them would be conservative.
  constexpr int NBMAX = (NT == 512 && D <= 128) ? 16 : (D == 256 ? 4 : 8);
  constexpr int NB = NI < NBMAX ? NI : NBMAX;
  constexpr int NBATCH = NI / NB;
  static_assert(NI % NB == 0, "batches");
  const __amdgpu_buffer_rsrc_t srows = __builtin_amdgcn_make_buffer_rsrc(
      stage, (short)0, (int)((int64_t)rnew * s.st_r * 4), kBufferRsrcWord3);
  const float4 kcopy = *reinterpret_cast<const float4*>(knew + 4 * cq);
  auto row = [&](int i) -> float4 {
    const int r = rsub + i * RPI;
    const auto v = __builtin_amdgcn_raw_buffer_load_b128(
        srows, (int)((int64_t)r * s.st_r * 4) + 16 * cq, 0, 0);
    const float4 f = make_float4(__uint_as_float(v[0]), __uint_as_float(v[1]),
                                 __uint_as_float(v[2]), __uint_as_float(v[3]));
    return r < rnew ? f : kcopy;
  };
  float4 x[NB];
  float mn[4], mx[4];
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    mn[k] = INFINITY;
    mx[k] = -INFINITY;
  }
  auto load_batch = [&](int bt) {
#pragma unroll
    for (int i = 0; i < NB; ++i) x[i] = row(bt * NB + i);
  };
  auto reduce_batch = [&]() {
#pragma unroll
    for (int i = 0; i < NB; ++i) {
      mn[0] = fminf(mn[0], x[i].x); mx[0] = fmaxf(mx[0], x[i].x);
      mn[1] = fminf(mn[1], x[i].y); mx[1] = fmaxf(mx[1], x[i].y);
      mn[2] = fminf(mn[2], x[i].z); mx[2] = fmaxf(mx[2], x[i].z);
      mn[3] = fminf(mn[3], x[i].w); mx[3] = fmaxf(mx[3], x[i].w);
    }
  };
  load_batch(0);
  // The page-table entries of the group's pages up to row rnew (one per
  // thread, clamped) and a piece of the new value row.
  const int lp_e = r0 / page_rows + min(tid, npg - 1);
  const int pg_e = page_table ? page_table[(int64_t)b * pt_b + lp_e] : lp_e;
  const int vpiece = tid % VPC;
  const U32x4 vcopy = ld16(vsrc + 16 * vpiece);
  issue();
  if (tid < npg) pt_grp[tid] = min(max(pg_e, 0), num_pages - 1);
  reduce_batch();
#pragma unroll 1
  for (int bt = 1; bt < NBATCH; ++bt) {
    if (bt * NB * RPI <= rnew) {
      load_batch(bt);
      reduce_batch();
    }
  }
  // The new key row into the staging rows (every thread of a channel slice
  // writes the same 16 bytes).
  *reinterpret_cast<float4*>(stage + (int64_t)rnew * s.st_r + 4 * cq) = kcopy;
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    mn[k] = allreduce_min_f<VPR, 64>(mn[k]);
    mx[k] = allreduce_max_f<VPR, 64>(mx[k]);
  }
  if (lane < VPR) {
    q_mn[wv][lane] = make_float4(mn[0], mn[1], mn[2], mn[3]);
    q_mx[wv][lane] = make_float4(mx[0], mx[1], mx[2], mx[3]);
  }
  __syncthreads();
  // The new value row into its page (every thread stores a piece; pieces
  // repeat when NT > VPC).
  st16(v_pages + (int64_t)pt_grp[rnew / page_rows] * vp_page + (int64_t)h * vp_head +
           (int64_t)(t % page_rows) * vp_row + 16 * vpiece,
       vcopy);
  if (tid < VPC) v_open[tid] = vcopy;
#pragma unroll
  for (int w = 0; w < NWAVE; ++w) {
    const float4 pm = q_mn[w][cq], px = q_mx[w][cq];
    mn[0] = fminf(mn[0], pm.x); mx[0] = fmaxf(mx[0], px.x);
    mn[1] = fminf(mn[1], pm.y); mx[1] = fmaxf(mx[1], px.y);
    mn[2] = fminf(mn[2], pm.z); mx[2] = fmaxf(mx[2], px.z);
    mn[3] = fminf(mn[3], pm.w); mx[3] = fmaxf(mx[3], px.w);
  }
  float sc[4], zp[4], rc[4];
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    scale_zp(mn[k], mx[k], &sc[k], &zp[k]);
    rc[k] = 1.0f / sc[k];
  }
  {
    // Every thread of a channel slice holds the same scale and zero-point.
    const int64_t so = (int64_t)b * s_b + (int64_t)h * s_h + (int64_t)g * s_g + 4 * cq;
    *reinterpret_cast<float4*>(k_scale + so) = make_float4(sc[0], sc[1], sc[2], sc[3]);
    *reinterpret_cast<float4*>(k_zp + so) = make_float4(zp[0], zp[1], zp[2], zp[3]);
    if (rsub == 0) {
      *reinterpret_cast<float4*>(sz_open + 4 * cq) = make_float4(sc[0], sc[1], sc[2], sc[3]);
      *reinterpret_cast<float4*>(sz_open + D + 4 * cq) = make_float4(zp[0], zp[1], zp[2], zp[3]);
    }
  }

  // Bins of the valid rows, nibble pairs into k_open, then whole 16-byte
  // pieces of packed rows to the pages.
  uint16_t* q_out = k_open;
#pragma unroll 1
  for (int bt = 0; bt < NBATCH; ++bt) {
    if (bt * NB * RPI <= rnew) {
      if (NBATCH > 1) load_batch(bt);
#pragma unroll
      for (int i = 0; i < NB; ++i) {
        const int r = rsub + (bt * NB + i) * RPI;
        if (r <= rnew) {
          const float n0 = quant_bin_rc(x[i].x, mn[0], sc[0], rc[0]);
          const float n1 = quant_bin_rc(x[i].y, mn[1], sc[1], rc[1]);
          const float n2 = quant_bin_rc(x[i].z, mn[2], sc[2], rc[2]);
          const float n3 = quant_bin_rc(x[i].w, mn[3], sc[3], rc[3]);
          const float pk = __builtin_fmaf(
              n3, 4096.0f, __builtin_fmaf(n2, 256.0f, __builtin_fmaf(n1, 16.0f, n0)));
          q_out[r * (RB / 2) + cq] = (uint16_t)(unsigned)pk;
        }
      }
    }
  }
  __syncthreads();
  // A fixed number of pieces per thread: piece indices past the group's
  // valid rows repeat the last valid piece.
  constexpr int NPC = (kStepMaxGroup * PPR + NT - 1) / NT;
  const int npieces = (rnew + 1) * PPR;
#pragma unroll
  for (int i = 0; i < NPC; ++i) {
    const int pc = min(tid + i * NT, npieces - 1);
    const int r = pc / PPR, part = pc - r * PPR;
    const int tok = r0 + r;
    uint8_t* dst = k_pages + (int64_t)pt_grp[r / page_rows] * kp_page + (int64_t)h * kp_head +
                   (int64_t)(tok % page_rows) * kp_row + part * 16;
    st16(dst, *reinterpret_cast<const U32x4*>(reinterpret_cast<const uint8_t*>(q_out) +
                                              r * RB + part * 16));
  }
}

}  // namespace fdi4
