// Fused INT4 flash decoding with the key products on the int8 matrix cores
// (gfx950, D = 64 or 128). Same semantics as decode_kernel and
// decode_gqa_kernel (reference src/flash_decode_ref.py:30-139 per (sequence,
// q-head) stream, q-head h reading kv-head h // (Hq/Hkv), src/ops.py:189-192):
// unscaled logits sum_d (q_d*s_d)*nib_d - sum_d q_d*(zp_d*s_d), online softmax,
// float32 value accumulation, split partials or the final output. One
// workgroup serves HG (2, 4 or 8) q-heads of one kv-head.
//
// Logits, exactly: per head m and scale group, the products q_d*s_d (exact
// in double) are scaled by 2^(41-E_m), E_m the binary exponent of the head's
// largest |q_d*s_d|, and rounded to integers v_d, |v_d| <= 2^41, written as
// six 7-bit digits v = d0*2^35 + d1*2^28 + ... + d5 (d0 signed, d1..d5 in
// 0..127: all int8). One v_mfma_i32_16x16x64_i8 per digit and 64 channels
// multiplies the 16 key rows' nibbles (A, 16 x 64) by the digits of up to 16
// heads (B, 64 x 16) with exact int32 sums; the six sums recombine exactly in
// double as (P0*2^28 + P1*2^14 + P2) * 2^(E_m-41), P0 = acc0*128 + acc1 etc.
// The only rounding is v_d's: |error| <= 2^(E_m-42) per product, below 1e-9
// of the largest |q_d*s_d| summed over D=128 channels and nibbles <= 15.
//
// Lane roles (lane l, g = l / 16): A rows are key rows n = l % 16, each lane
// holding its row's channels of group g (D/8 packed bytes, one 16- or 8-byte
// load); B columns are heads m = l % 16 with the same channels; the result
// lane holds rows 4g .. 4g+3 of head m, so the softmax of head m runs across
// the four lanes l % 16 == m. Probabilities and rescale factors go through
// LDS to the value lanes, whose loads and float32 FMAs are those of
// decode_gqa_kernel. Loads are pipelined as in decode_kernel (two buffers,
// exact wait counts).

#include "decode_common.hpp"

namespace fdi4 {

typedef int v4i __attribute__((ext_vector_type(4)));

template <int D, int VDT>
struct MfmaGeo {
  static constexpr int NB = D / 64;                // 64-channel MFMA blocks
  static constexpr int KW = D / 32;                // packed key words per lane per row
  static constexpr int VEB = VDT == kVF32 ? 4 : 2; // bytes per value element
  static constexpr int VCL = 16 / VEB;             // value channels per lane
  static constexpr int VPR = D / VCL;              // lanes per value row
  static constexpr int RPL = 64 / VPR;             // value rows per sweep
  static constexpr int VLD = 16 / RPL;             // value sweeps per chunk
  static constexpr int SZI = D / 2;                // 16-byte items in a scale+zp block
  static constexpr int SZL = (SZI + 63) / 64;      // scale+zp loads per lane
  static constexpr int DIGITS = 6;
  static_assert(D == 64 || D == 128, "int8 MFMA decode: D = 64 or 128");
};

// Channel layout of the MFMA operands: lane group g (lanes 16g .. 16g+15)
// holds the 16-channel piece kb of channels base = 16g (D = 64) or 32g + 16kb
// (D = 128); slot j (byte j of the B operand) is channel base + 2j for
// j < 8 (the low nibbles of the packed bytes) and base + 2(j-8) + 1 for
// j >= 8 (the high nibbles), matching the A operand built from the packed
// key words.

template <int HG>
struct HeadF {
  float v[HG];
};

template <int D, int VDT, int WAVES, int HG>
__global__ __launch_bounds__(WAVES * 64) void decode_mfma_kernel(DecodeArgs a) {
  using G = MfmaGeo<D, VDT>;
  constexpr int NT = WAVES * 64;
  static_assert(HG >= 2 && HG <= 8, "heads per workgroup");

  const int split = blockIdx.x, b = blockIdx.z;
  const int h0 = blockIdx.y * HG;           // first q-head of this workgroup
  const int hk = h0 / a.hq_per_kv;          // HG divides hq_per_kv: one kv-head
  const int tid = threadIdx.x, lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int n16 = lane & 15;                // key row (A) and head (B, result)
  const int grp = lane >> 4;                // channel group; result rows 4*grp..+3
  const bool head_lane = n16 < HG;
  const int vrow = lane / G::VPR;
  const int vcol = lane % G::VPR;

  __shared__ float q_s[HG][D];
  __shared__ HeadF<HG> p_s[WAVES][16];
  __shared__ HeadF<HG> corr_s[WAVES];
  __shared__ float sz_s[WAVES][2 * D];
  __shared__ float acc_s[WAVES][HG][D];
  __shared__ double m_s[WAVES][HG];
  __shared__ float l_s[WAVES][HG];
  // Per wave: the HG heads' B operands in MFMA lane layout [digit][block]
  // [channel group][head][byte], their exponents and group constants.
  __shared__ __attribute__((aligned(16))) uint8_t dig_s[WAVES][G::DIGITS][G::NB][4][HG][16];
  __shared__ int hex_s[WAVES][HG];
  __shared__ double hcg_s[WAVES][HG];

  const int cpp = (a.page_rows + 15) >> 4;
  const int T = seq_len_of(a, b);
  const int n_chunks = pages_of(a, T) * cpp;
  const int c_begin = split * a.chunks_per_split;
  const int c_end = min(c_begin + a.chunks_per_split, n_chunks);
  const WaveRange wr = wave_chunks(c_begin, c_end, w, WAVES);
  const int wc0 = wr.c0, wc1 = wr.c1;

  // Softmax state of head n16 (meaningful on head lanes).
  double m_run = -INFINITY;
  float l_run = 0.f;
  double cg = 0.0;
  int e_head = 0;
  // Value accumulators of all HG heads for this lane's value channels.
  float acc[HG][G::VCL];
#pragma unroll
  for (int h = 0; h < HG; ++h)
#pragma unroll
    for (int k = 0; k < G::VCL; ++k) acc[h][k] = 0.f;
  // Digits of head n16's scaled q*s for this lane's channels (B operands).
  v4i bq[G::DIGITS][G::NB];
  int cur_group = -1;

  const float* sbase = a.k_scale + (int64_t)b * a.s_b + (int64_t)hk * a.s_h;
  const float* zbase = a.k_zp + (int64_t)b * a.s_b + (int64_t)hk * a.s_h;
  // Page bases are wave-uniform (scalar registers); each lane adds a 32-bit
  // byte offset (its channel slice and row), so the loads take the
  // scalar-base + vector-offset form with no 64-bit address arithmetic per
  // lane (row strides are checked on the host: 16 rows fit in 31 bits).
  const uint8_t* kbase_h = a.k_pages + (int64_t)hk * a.k_head;
  const uint8_t* vbase_h = reinterpret_cast<const uint8_t*>(a.v_pages) +
                           (int64_t)hk * a.v_head * G::VEB;
  const unsigned k_lane = grp * (D / 8), v_lane = vcol * 16;
  const unsigned krow_b = (unsigned)a.k_row, vrow_b = (unsigned)(a.v_row * G::VEB);

  auto load_sz = [&](const ChunkMeta& m, U32x4* sz) {
    const int64_t off = (int64_t)m.group * a.s_g + m.phys * a.s_p;
#pragma unroll
    for (int i = 0; i < G::SZL; ++i) {
      const int e = (i * 64 + lane) % G::SZI;
      const float* src = (e < D / 4) ? (sbase + off + 4 * e) : (zbase + off + 4 * (e - D / 4));
      sz[i] = ld16(src);
    }
  };

  auto load_chunk = [&](const ChunkMeta& m, KVec<G::KW>* kr, U32x4* vr) {
    const uint8_t* kb = kbase_h + m.phys * a.k_page + (int64_t)m.r0 * a.k_row;
    const int t = max(min(n16, m.nval - 1), 0);
    kr[0] = load_k<G::KW>(kb + (k_lane + (unsigned)t * krow_b));
    const uint8_t* vb = vbase_h + (m.phys * a.v_page + (int64_t)m.r0 * a.v_row) * G::VEB;
#pragma unroll
    for (int i = 0; i < G::VLD; ++i) {
      const int r = max(min(i * G::RPL + vrow, m.nval - 1), 0);
      vr[i] = ld16_stream(vb + (v_lane + (unsigned)r * vrow_b));
    }
  };

  // Rebuild the B operands (digits), exponents and group constants of the HG
  // heads from the staged scale/zero-point block. The products are spread
  // densely: lane l computes PPL channels of head l / LPH (every lane busy,
  // whatever HG), and the digit bytes go through LDS into the MFMA lane
  // layout (lane l's B operand: head l % 16, channel group l / 16), where a
  // head lane reads them back as 16-byte words.
  auto rebuild = [&](const float* szw) {
    constexpr int LPH = 64 / HG;        // lanes per head
    constexpr int PPL = HG * D / 64;    // channels per lane
    const int hh = lane / LPH;
    const int d0 = (lane % LPH) * PPL;
    const float* qh = q_s[hh];
    // Pass 1: the head's largest |q*s| (its exponent) and the group constant.
    double mx = 0.0, cgp = 0.0;
#pragma unroll
    for (int i = 0; i < PPL; ++i) {
      const int d = d0 + i;
      const double qd = (double)qh[d];
      const double sd = (double)szw[d];
      mx = fmax(mx, fabs(qd * sd));
      cgp = __builtin_fma(qd, (double)szw[D + d] * sd, cgp);
    }
    mx = allreduce_max<1, LPH>(mx);
    const double cgh = allreduce_sum<1, LPH>(cgp);
    int ex = 0;
    if (mx > 0.0) (void)frexp(mx, &ex);
    // Pass 2: the products again (cheaper than keeping them), as digits at
    // their B-operand byte: channel d is byte j of group g's block kb.
#pragma unroll
    for (int i = 0; i < PPL; ++i) {
      const int d = d0 + i;
      const double qsd = (double)qh[d] * (double)szw[d];
      // v = rint(q*s * 2^(41 - e)), |v| <= 2^41; v = hi * 2^21 + lo, 0 <= lo < 2^21.
      const double v = rint(ldexp(qsd, 41 - ex));
      const double hi = floor(v * 0x1p-21);
      const int hi_i = (int)hi;
      const int lo_i = (int)(v - hi * 0x1p21);
      const unsigned dig[G::DIGITS] = {
          (unsigned)(hi_i >> 14) & 255u, (unsigned)(hi_i >> 7) & 127u, (unsigned)hi_i & 127u,
          (unsigned)(lo_i >> 14) & 127u, (unsigned)(lo_i >> 7) & 127u, (unsigned)lo_i & 127u};
      const int g = (D == 64) ? d / 16 : d / 32;
      const int kb = (D == 64) ? 0 : (d / 16) & 1;
      const int o = d & 15;
      const int jb = (o & 1) ? 8 + (o >> 1) : (o >> 1);
#pragma unroll
      for (int dg = 0; dg < G::DIGITS; ++dg) dig_s[w][dg][kb][g][hh][jb] = (uint8_t)dig[dg];
    }
    if (lane % LPH == 0) {
      hex_s[w][hh] = ex;
      hcg_s[w][hh] = cgh;
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    if (head_lane) {
#pragma unroll
      for (int dg = 0; dg < G::DIGITS; ++dg)
#pragma unroll
        for (int kb = 0; kb < G::NB; ++kb)
          bq[dg][kb] = *reinterpret_cast<const v4i*>(&dig_s[w][dg][kb][grp][n16][0]);
      e_head = hex_s[w][n16];
      cg = hcg_s[w][n16];
    } else {
#pragma unroll
      for (int dg = 0; dg < G::DIGITS; ++dg)
#pragma unroll
        for (int kb = 0; kb < G::NB; ++kb) bq[dg][kb] = v4i{0, 0, 0, 0};
      e_head = 0;
      cg = 0.0;
    }
  };

  int c = wc0;
  ChunkMeta cm, nm;
  U32x4 sz[G::SZL];
  auto meta_at = [&](int ci) { return chunk_meta(a, b, T, cpp, min(ci, wc1 - 1)); };
  auto step = [&](const KVec<G::KW>* ck, const U32x4* cv, KVec<G::KW>* nk, U32x4* nv) -> bool {
    if (cm.group != cur_group) {
      float* szw = sz_s[w];
#pragma unroll
      for (int i = 0; i < G::SZL; ++i) {
        const int e = i * 64 + lane;
        if (e < G::SZI) *reinterpret_cast<U32x4*>(szw + 4 * e) = sz[i];
      }
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
      rebuild(szw);
      cur_group = cm.group;
      __builtin_amdgcn_wave_barrier();
    }

    const bool last = c + 1 >= wc1;
    ChunkMeta pf = nm;
    pf.nval = last ? 1 : nm.nval;
    load_sz(pf, sz);
    load_chunk(pf, nk, nv);
    const ChunkMeta nnm = meta_at(c + 2);
    if (cm.nval > 0) {
      // Key rows x digits: acc[dg][r] = sum over channels of nib * digit for
      // row 4*grp + r of head n16.
      v4i accd[G::DIGITS];
#pragma unroll
      for (int kb = 0; kb < G::NB; ++kb) {
        const unsigned w0 = ck[0].w[2 * kb], w1 = ck[0].w[2 * kb + 1];
        const v4i ak = v4i{(int)(w0 & 0x0F0F0F0Fu), (int)(w1 & 0x0F0F0F0Fu),
                           (int)((w0 >> 4) & 0x0F0F0F0Fu), (int)((w1 >> 4) & 0x0F0F0F0Fu)};
#pragma unroll
        for (int dg = 0; dg < G::DIGITS; ++dg)
          accd[dg] = __builtin_amdgcn_mfma_i32_16x16x64_i8(
              ak, bq[dg][kb], kb == 0 ? v4i{0, 0, 0, 0} : accd[dg], 0, 0, 0);
      }
      double lg[4];
      float mloc = -INFINITY;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int p0 = accd[0][r] * 128 + accd[1][r];
        const int p1 = accd[2][r] * 128 + accd[3][r];
        const int p2 = accd[4][r] * 128 + accd[5][r];
        const double s = __builtin_fma((double)p0, 0x1p28,
                                       __builtin_fma((double)p1, 0x1p14, (double)p2));
        lg[r] = (4 * grp + r < cm.nval) ? ldexp(s, e_head - 41) - cg : -INFINITY;
        mloc = fmaxf(mloc, (float)lg[r]);
      }
      // The float32 maximum of the rounded logits (exact as a double) is the
      // shift; lg - m_new stays <= half a float ulp of lg.
      const float mc = allreduce_max_f<16, 64>(mloc);
      const double m_new = fmax(m_run, (double)mc);
      const float corr = exp2_of(m_run - m_new);
      m_run = m_new;
      float psum = 0.f;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const float p = exp2_of(lg[r] - m_new);
        psum += p;
        if (head_lane) p_s[w][4 * grp + r].v[head_lane ? n16 : 0] = p;
      }
      l_run = l_run * corr + psum;
      if (head_lane && grp == 0) corr_s[w].v[head_lane ? n16 : 0] = corr;
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");

      const HeadF<HG> cr = corr_s[w];
#pragma unroll
      for (int h = 0; h < HG; ++h)
#pragma unroll
        for (int k = 0; k < G::VCL; ++k) acc[h][k] *= cr.v[h];
#pragma unroll
      for (int i = 0; i < G::VLD; ++i) {
        // Rows past the valid count hold probability 0 and a copy of a valid row.
        const HeadF<HG> pr = p_s[w][i * G::RPL + vrow];
        float vf[G::VCL];
        widen_values<VDT>(cv[i], vf);
#pragma unroll
        for (int h = 0; h < HG; ++h)
#pragma unroll
          for (int k = 0; k < G::VCL; ++k) acc[h][k] = __builtin_fmaf(pr.v[h], vf[k], acc[h][k]);
      }
      __builtin_amdgcn_wave_barrier();
    }
    c += 1;
    cm = nm;
    nm = nnm;
    return last;
  };

  // q rows of the HG heads: into registers first, then the first chunk's
  // loads, then q to LDS (as in decode_kernel).
  constexpr int QPT = (HG * D + NT - 1) / NT;
  float qv[QPT];
#pragma unroll
  for (int j = 0; j < QPT; ++j) {
    const int idx = tid + j * NT;
    qv[j] = (idx < HG * D)
                ? load_elem(a.q, (int64_t)b * a.q_b + (int64_t)(h0 + idx / D) * a.q_h + idx % D,
                            a.q_dtype)
                : 0.f;
  }
  const bool has_work = c < wc1;
  KVec<G::KW> ka[1], kb[1];
  U32x4 va[G::VLD], vb[G::VLD];
  if (has_work) {
    cm = meta_at(c);
    nm = meta_at(c + 1);
    load_sz(cm, sz);
    load_chunk(cm, ka, va);
  }
#pragma unroll
  for (int j = 0; j < QPT; ++j) {
    const int idx = tid + j * NT;
    if (idx < HG * D) q_s[idx / D][idx % D] = qv[j];
  }
  __syncthreads();
  if (has_work) {
    while (true) {
      if (step(ka, va, kb, vb)) break;
      if (step(kb, vb, ka, va)) break;
    }
  }

  // Wave totals per head, then the log-sum-exp merge of the waves.
  const float l_tot = allreduce_sum<16, 64>(l_run);
  if (head_lane && grp == 0) {
    m_s[w][head_lane ? n16 : 0] = m_run;
    l_s[w][head_lane ? n16 : 0] = l_tot;
  }
#pragma unroll
  for (int h = 0; h < HG; ++h) {
#pragma unroll
    for (int k = 0; k < G::VCL; ++k) acc[h][k] = allreduce_sum<G::VPR, 64>(acc[h][k]);
    if (lane < G::VPR) {
#pragma unroll
      for (int k = 0; k < G::VCL; ++k) acc_s[w][h][lane * G::VCL + k] = acc[h][k];
    }
  }
  __syncthreads();

  for (int idx = tid; idx < HG * D; idx += NT) {
    const int h = idx / D, d = idx % D;
    double ms = -INFINITY;
#pragma unroll
    for (int i = 0; i < WAVES; ++i) ms = fmax(ms, m_s[i][h]);
    float o = 0.f, l = 0.f;
#pragma unroll
    for (int i = 0; i < WAVES; ++i) {
      const float e = (m_s[i][h] == -INFINITY) ? 0.f : exp2_of(m_s[i][h] - ms);
      l = __builtin_fmaf(e, l_s[i][h], l);
      o = __builtin_fmaf(e, acc_s[i][h][d], o);
    }
    const int hq = h0 + h;
    const int64_t pi = ((int64_t)b * a.num_q_heads + hq) * a.num_splits + split;
    if (a.final_out) {
      store_elem(a.out, (int64_t)b * a.o_b + (int64_t)hq * a.o_h + d, a.out_dtype,
                 o / fmaxf(l, 1e-10f));
    } else {
      a.ws_acc[pi * D + d] = o;
      if (d == 0) {
        a.ws_ml[2 * pi] = ms;
        a.ws_ml[2 * pi + 1] = (double)l;
      }
    }
  }
  hand_back_length(a, b);
}

hipError_t launch_decode_mfma(const DecodeArgs& a, int D, int v_dtype, int batch, int hg,
                              hipStream_t st) {
  dim3 grid(a.num_splits, a.num_q_heads / hg, batch);
#define FDI4_MF(DD, VV, WW, HH)                                                            \
  if (D == DD && v_dtype == VV && a.waves == WW && hg == HH) {                             \
    hipLaunchKernelGGL((decode_mfma_kernel<DD, VV, WW, HH>), grid, dim3(WW * 64), 0, st, a); \
    return hipGetLastError();                                                              \
  }
#define FDI4_MF_H(WW, HH)                                                                 \
  FDI4_MF(64, kVF32, WW, HH) FDI4_MF(128, kVF32, WW, HH)                                  \
  FDI4_MF(64, kVF16, WW, HH) FDI4_MF(128, kVF16, WW, HH)                                  \
  FDI4_MF(64, kVBF16, WW, HH) FDI4_MF(128, kVBF16, WW, HH)
  FDI4_MF_H(4, 2) FDI4_MF_H(8, 2) FDI4_MF_H(4, 4) FDI4_MF_H(8, 4)
  // Eight heads per workgroup.
  FDI4_MF_H(4, 8) FDI4_MF_H(8, 8)
#undef FDI4_MF_H
#undef FDI4_MF
  return hipErrorInvalidValue;
}

}  // namespace fdi4
