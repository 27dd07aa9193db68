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

// Appends token t of (sequence b, kv-head h) and re-quantizes its open group
// g = t / group_rows over the group's t % group_rows + 1 rows, with the
// workgroup's NT threads: the key row goes to the staging rows, the value row
// to its page; the group's rows are held in registers (16-byte loads, all in
// flight at once), per-channel min/max by a lane butterfly then LDS across
// waves, the group's scale and zero-point, and the packed rows of the group
// to their pages. The arithmetic is that of the grouped quantizer
// (quant_bin_rc, scale_zp), so the stored bytes equal the append kernel's.
// k_pages/v_pages and the scales are the cache's (byte and element strides
// as in DecodeArgs). Ends with the workgroup's stores complete and visible to
// its own later loads (a workgroup release: every vector memory operation the
// waves issued before, loads included, has completed).
template <int D, int NT, int VEB>
__device__ __forceinline__ void step_requant(const StepAppend& s, uint8_t* k_pages,
                                             int64_t kp_page, int64_t kp_head, int64_t kp_row,
                                             uint8_t* v_pages, int64_t vp_page, int64_t vp_head,
                                             int64_t vp_row, float* k_scale, float* k_zp,
                                             int64_t s_b, int64_t s_h, int64_t s_g,
                                             const int32_t* page_table, int64_t pt_b,
                                             int page_rows, int num_pages, int b, int h, int t) {
  constexpr int VPR = D / 4;          // threads per staged row (16 bytes each)
  constexpr int RPI = NT / VPR;       // rows per sweep of the workgroup
  constexpr int NI = kStepMaxGroup / RPI;   // rows per thread, at most
  constexpr int RB = D / 2;           // packed bytes per row
  constexpr int NWAVE = NT / 64;
  static_assert(VPR <= 64 && NT % VPR == 0 && kStepMaxGroup % RPI == 0, "layout");
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int cq = tid % VPR, rsub = tid / VPR;
  const int G = s.group_rows;
  const int g = t / G, rnew = t - g * G, r0 = g * G;
  const float* knew = s.k_new + (int64_t)b * s.kn_b + (int64_t)h * s.kn_h;
  float* stage = s.stage + (int64_t)b * s.st_b + (int64_t)h * s.st_h;
  auto phys_of = [&](int tok) {
    const int pg = page_table ? page_table[(int64_t)b * pt_b + tok / page_rows] : tok / page_rows;
    return (int64_t)min(max(pg, 0), num_pages - 1);
  };

  // The group's rows (row rnew from k_new itself; rows past it repeat it, so
  // they leave the min/max unchanged) in batches of NB rows per thread, each
  // batch's loads in flight together; with one batch the rows stay in
  // registers for the bins, otherwise the bins re-read them (from the L2).
  // 16 rows per thread in a batch with eight waves at D <= 128, 8 otherwise
  // (the decode's first chunk is in registers meanwhile; more would spill).
  constexpr int NBMAX = (NT == 512 && D <= 128) ? 16 : 8;
  constexpr int NB = NI < NBMAX ? NI : NBMAX;
  constexpr int NBATCH = NI / NB;
  static_assert(NI % NB == 0, "batches");
  auto row = [&](int i) -> float4 {
    const int r = min(rsub + i * RPI, rnew);
    const float* src = (r == rnew) ? knew : stage + (int64_t)r * s.st_r;
    return *reinterpret_cast<const float4*>(src + 4 * cq);
  };
  float4 x[NB];
  float mn[4], mx[4];
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    mn[k] = INFINITY;
    mx[k] = -INFINITY;
  }
#pragma unroll 1
  for (int bt = 0; bt < NBATCH; ++bt) {
    if (bt * NB * RPI <= rnew) {
#pragma unroll
      for (int i = 0; i < NB; ++i)
        if ((bt * NB + i) * RPI < G) x[i] = row(bt * NB + i);
#pragma unroll
      for (int i = 0; i < NB; ++i) {
        if ((bt * NB + i) * RPI < G) {
          mn[0] = fminf(mn[0], x[i].x); mx[0] = fmaxf(mx[0], x[i].x);
          mn[1] = fminf(mn[1], x[i].y); mx[1] = fmaxf(mx[1], x[i].y);
          mn[2] = fminf(mn[2], x[i].z); mx[2] = fmaxf(mx[2], x[i].z);
          mn[3] = fminf(mn[3], x[i].w); mx[3] = fmaxf(mx[3], x[i].w);
        }
      }
    }
  }
  // The new key row into the staging rows, the new value row into its page.
  if (tid < VPR)
    *reinterpret_cast<float4*>(stage + (int64_t)rnew * s.st_r + 4 * tid) =
        *reinterpret_cast<const float4*>(knew + 4 * tid);
  {
    const uint8_t* vsrc = s.v_new + (int64_t)b * s.vn_b + (int64_t)h * s.vn_h;
    uint8_t* vdst = v_pages + phys_of(t) * vp_page + (int64_t)h * vp_head +
                    (int64_t)(t % page_rows) * vp_row;
    for (int o = 16 * tid; o < D * VEB; o += 16 * NT) st16(vdst + o, ld16(vsrc + o));
  }
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    mn[k] = allreduce_min_f<VPR, 64>(mn[k]);
    mx[k] = allreduce_max_f<VPR, 64>(mx[k]);
  }
  __shared__ float4 q_mn[NWAVE][VPR], q_mx[NWAVE][VPR];
  if (lane < VPR) {
    q_mn[wv][lane] = make_float4(mn[0], mn[1], mn[2], mn[3]);
    q_mx[wv][lane] = make_float4(mx[0], mx[1], mx[2], mx[3]);
  }
  __syncthreads();
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
  if (rsub == 0) {
    const int64_t so = (int64_t)b * s_b + (int64_t)h * s_h + (int64_t)g * s_g + 4 * cq;
    *reinterpret_cast<float4*>(k_scale + so) = make_float4(sc[0], sc[1], sc[2], sc[3]);
    *reinterpret_cast<float4*>(k_zp + so) = make_float4(zp[0], zp[1], zp[2], zp[3]);
  }

  // Bins of the valid rows, nibble pairs staged in LDS, then whole 16-byte
  // pieces of packed rows.
  __shared__ uint16_t q_out[kStepMaxGroup * RB / 2];
#pragma unroll 1
  for (int bt = 0; bt < NBATCH; ++bt) {
    if (bt * NB * RPI <= rnew) {
      if (NBATCH > 1) {
#pragma unroll
        for (int i = 0; i < NB; ++i)
          if ((bt * NB + i) * RPI < G) x[i] = row(bt * NB + i);
      }
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
  constexpr int PPR = RB / 16;        // 16-byte pieces per packed row
  for (int pc = tid; pc < (rnew + 1) * PPR; pc += NT) {
    const int r = pc / PPR, part = pc - r * PPR;
    const int tok = r0 + r;
    uint8_t* dst = k_pages + phys_of(tok) * kp_page + (int64_t)h * kp_head +
                   (int64_t)(tok % page_rows) * kp_row + part * 16;
    st16(dst, *reinterpret_cast<const U32x4*>(reinterpret_cast<const uint8_t*>(q_out) +
                                              r * RB + part * 16));
  }
  // The workgroup's stores complete before any of its waves loads the group.
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
  __syncthreads();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
}

}  // namespace fdi4
