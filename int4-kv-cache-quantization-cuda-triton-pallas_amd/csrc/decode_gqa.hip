// Fused INT4 flash decoding for grouped-query attention (gfx950): one
// workgroup serves HG query heads that share one kv-head, so every packed key
// and value byte of a split is read from HBM once per HG heads instead of once
// per head. Same semantics as decode_kernel (reference src/flash_decode_ref.py
// :30-139 applied per (sequence, q-head) stream with the kv-head h // (Hq/Hkv),
// the construction of src/ops.py:189-192): unscaled fp64 logits
// sum_d (q_d*s_d)*nib_d - sum_d q_d*(zp_d*s_d), online softmax per head,
// float32 value accumulation, split partials or the final output.
//
// Per 16-row chunk and wave:
//   K: LPT = D/8 lanes per key row, 8 channels (one 4-byte word of nibbles)
//      per lane. The (q*s) products of the HG heads live in LDS (8 doubles
//      per lane and head, rebuilt when the scale group changes) so that the
//      registers hold one head at a time; the nibbles are converted to double
//      once per chunk and multiplied into every head's slice; the KLD row
//      sums of a lane are combined by a reduce-scatter over the lane bits
//      LPT/2 .. 4 and an all-reduce over
//      bits 1 and 2, leaving each lane with the logit of row
//      (kq >> 2) * TPW + ktok (four lanes per row).
//   softmax: per head, fp64 chunk maximum across the wave, float32 exp;
//      the probabilities of the HG heads go to LDS as [row][head].
//   V: as decode_kernel (fully coalesced 16-byte loads), one LDS read of the
//      HG probabilities per row, HG float32 FMAs per value element.
//   The next chunk's loads are in flight while the current one is computed
//   (two-buffer ping-pong, wait counts exact as in decode_kernel).

#include "decode_common.hpp"

namespace fdi4 {

template <int D, int VDT>
struct GqaGeo {
  static constexpr int CPL = 8;                    // channels per lane (K)
  static constexpr int LPT = D / CPL;              // lanes per key row: 8, 16, 32
  static constexpr int TPW = 64 / LPT;             // key rows per sweep
  static constexpr int KLD = 16 / TPW;             // key sweeps per chunk
  static constexpr int VEB = VDT == kVF32 ? 4 : 2; // bytes per value element
  static constexpr int VCL = 16 / VEB;             // value channels per lane
  static constexpr int VPR = D / VCL;              // lanes per value row
  static constexpr int RPL = 64 / VPR;             // value rows per sweep
  static constexpr int VLD = 16 / RPL;             // value sweeps per chunk
  static constexpr int SZI = D / 2;                // 16-byte items in a scale+zp block
  static constexpr int SZL = (SZI + 63) / 64;      // scale+zp loads per lane
  static_assert(LPT / KLD == 4, "four lanes share each reduced logit");
  static_assert(RPL >= 1 && 16 % RPL == 0, "value geometry");
};

// s[0 .. N) are partial sums over this lane's channels for N rows; lanes
// differing in bit BIT hold the same rows. Afterwards s[0] holds the sum over
// the lane pair of row index (lane & BIT ? N/2 : 0) + ..., recursively.
template <int N, int BIT>
__device__ __forceinline__ void reduce_scatter(double* s, int lane) {
  if constexpr (N > 1) {
    const bool up = (lane & BIT) != 0;
#pragma unroll
    for (int j = 0; j < N / 2; ++j) {
      const double send = up ? s[j] : s[j + N / 2];
      const double keep = up ? s[j + N / 2] : s[j];
      s[j] = keep + xchg<BIT>(send);
    }
    reduce_scatter<N / 2, BIT / 2>(s, lane);
  }
}

template <int HG>
struct HeadP {
  float p[HG];
};

template <int D, int VDT, int WAVES, int HG>
__global__ __launch_bounds__(WAVES * 64) void decode_gqa_kernel(DecodeArgs a) {
  using G = GqaGeo<D, VDT>;
  constexpr int NT = WAVES * 64;

  const int split = blockIdx.x, b = blockIdx.z;
  const int h0 = blockIdx.y * HG;           // first q-head of this workgroup
  const int hk = h0 / a.hq_per_kv;          // HG divides hq_per_kv: one kv-head
  const int tid = threadIdx.x, lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int kq = lane % G::LPT;             // channel slice of this lane (K)
  const int ktok = lane / G::LPT;           // key row within a sweep
  const int krow = (kq >> 2) * G::TPW + ktok;  // row whose logit the lane ends with
  const bool kwriter = (kq & 3) == 0;          // one of the four lanes holding it
  const int vrow = lane / G::VPR;
  const int vcol = lane % G::VPR;

  __shared__ float q_s[HG][D];
  // [ci][kq]: the lanes of a key row read consecutive doubles (no bank
  // conflicts; lanes of the same slice get a broadcast).
  __shared__ double qs_s[WAVES][HG][G::CPL][G::LPT];
  __shared__ double cg_s[WAVES][HG];
  __shared__ HeadP<HG> p_s[WAVES][16];
  __shared__ float sz_s[WAVES][2 * D];
  __shared__ float acc_s[WAVES][HG][D];
  __shared__ double m_s[WAVES][HG];
  __shared__ float l_s[WAVES][HG];

  const int cpp = (a.page_rows + 15) >> 4;
  const int T = seq_len_of(a, b);
  const int n_chunks = pages_of(a, T) * cpp;
  const int c_begin = split * a.chunks_per_split;
  const int c_end = min(c_begin + a.chunks_per_split, n_chunks);
  const WaveRange wr = wave_chunks(c_begin, c_end, w, WAVES);
  const int wc0 = wr.c0, wc1 = wr.c1;

  double m_run[HG];
  float l_lane[HG];
  float acc[HG][G::VCL];
#pragma unroll
  for (int h = 0; h < HG; ++h) {
    m_run[h] = -INFINITY;
    l_lane[h] = 0.f;
#pragma unroll
    for (int k = 0; k < G::VCL; ++k) acc[h][k] = 0.f;
  }
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
  const unsigned k_lane = kq * (G::CPL / 2), v_lane = vcol * 16;
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

  auto load_chunk = [&](const ChunkMeta& m, KVec<1>* kr, U32x4* vr) {
    const uint8_t* kb = kbase_h + m.phys * a.k_page + (int64_t)m.r0 * a.k_row;
#pragma unroll
    for (int i = 0; i < G::KLD; ++i) {
      const int t = max(min(i * G::TPW + ktok, m.nval - 1), 0);
      kr[i] = load_k<1>(kb + (k_lane + (unsigned)t * krow_b));
    }
    const uint8_t* vb = vbase_h + (m.phys * a.v_page + (int64_t)m.r0 * a.v_row) * G::VEB;
#pragma unroll
    for (int i = 0; i < G::VLD; ++i) {
      const int r = max(min(i * G::RPL + vrow, m.nval - 1), 0);
      vr[i] = ld16_stream(vb + (v_lane + (unsigned)r * vrow_b));
    }
  };

  // The same step structure as decode_kernel: stage a new scale group,
  // prefetch chunk c+1 (one row of the last chunk on the last step), read the
  // page-table entry of chunk c+2, consume chunk c.
  int c = wc0;
  ChunkMeta cm, nm;
  U32x4 sz[G::SZL];
  auto meta_at = [&](int ci) { return chunk_meta(a, b, T, cpp, min(ci, wc1 - 1)); };
  auto step = [&](const KVec<1>* ck, const U32x4* cv, KVec<1>* nk, U32x4* nv) -> bool {
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
#pragma unroll
      for (int h = 0; h < HG; ++h) {
        double cgp = 0.0;
        double qsv[G::CPL];
#pragma unroll
        for (int ci = 0; ci < G::CPL; ++ci) {
          const int d = kq * G::CPL + ci;
          const double qd = (double)q_s[h][d];
          const double sd = (double)szw[d];
          qsv[ci] = qd * sd;
          cgp = __builtin_fma(qd, (double)szw[D + d] * sd, cgp);
        }
        const double cgh = allreduce_sum<1, G::LPT>(cgp);
        if (ktok == 0) {
#pragma unroll
          for (int ci = 0; ci < G::CPL; ++ci) qs_s[w][h][ci][kq] = qsv[ci];
          if (kq == 0) cg_s[w][h] = cgh;
        }
      }
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
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
      // The chunk's nibbles as doubles, shared by the heads.
      double f[G::KLD][G::CPL];
#pragma unroll
      for (int i = 0; i < G::KLD; ++i) {
        const unsigned x = ck[i].w[0];
#pragma unroll
        for (int ci = 0; ci < G::CPL; ++ci) f[i][ci] = (double)((x >> (4 * ci)) & 15u);
      }
      float corr[HG];
#pragma unroll
      for (int h = 0; h < HG; ++h) {
        double qv[G::CPL];
#pragma unroll
        for (int ci = 0; ci < G::CPL; ++ci) qv[ci] = qs_s[w][h][ci][kq];
        double s[G::KLD];
#pragma unroll
        for (int i = 0; i < G::KLD; ++i) {
          double s0 = f[i][0] * qv[0], s1 = f[i][1] * qv[1];
          s0 = __builtin_fma(f[i][2], qv[2], s0);
          s1 = __builtin_fma(f[i][3], qv[3], s1);
          s0 = __builtin_fma(f[i][4], qv[4], s0);
          s1 = __builtin_fma(f[i][5], qv[5], s1);
          s0 = __builtin_fma(f[i][6], qv[6], s0);
          s1 = __builtin_fma(f[i][7], qv[7], s1);
          s[i] = s0 + s1;
        }
        reduce_scatter<G::KLD, G::LPT / 2>(s, lane);
        const double dot = allreduce_sum<1, 4>(s[0]);
        const double lg = (krow < cm.nval) ? dot - cg_s[w][h] : -INFINITY;
        // The running maximum only shifts the exponentials: the float32
        // maximum of the rounded logits (exact as a double) serves, and
        // lg - m_new stays <= half a float ulp of lg.
        const float mc = allreduce_max_f<4, 64>((float)lg);
        const double m_new = fmax(m_run[h], (double)mc);
        corr[h] = exp2_of(m_run[h] - m_new);
        m_run[h] = m_new;
        const float p = exp2_of(lg - m_new);
        if (kwriter) p_s[w][krow].p[h] = p;
        l_lane[h] = l_lane[h] * corr[h] + (kwriter ? p : 0.f);
      }
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");

#pragma unroll
      for (int h = 0; h < HG; ++h) {
#pragma unroll
        for (int k = 0; k < G::VCL; ++k) acc[h][k] *= corr[h];
      }
#pragma unroll
      for (int i = 0; i < G::VLD; ++i) {
        const int r = i * G::RPL + vrow;
        // Rows past the valid count hold probability 0 (their logits are
        // -inf), and their value registers hold a copy of a valid row.
        const HeadP<HG> pr = p_s[w][r];
        float vf[G::VCL];
        widen_values<VDT>(cv[i], vf);
#pragma unroll
        for (int h = 0; h < HG; ++h) {
#pragma unroll
          for (int k = 0; k < G::VCL; ++k) acc[h][k] = __builtin_fmaf(pr.p[h], vf[k], acc[h][k]);
        }
      }
      __builtin_amdgcn_wave_barrier();
    }
    c += 1;
    cm = nm;
    nm = nnm;
    return last;
  };

  // q rows of the HG heads: loaded into registers first, then the first
  // chunk's loads are issued, then q goes to LDS (as in decode_kernel).
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
  KVec<1> ka[G::KLD], kb[G::KLD];
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
#pragma unroll
  for (int h = 0; h < HG; ++h) {
    const float lw = allreduce_sum<1, 64>(l_lane[h]);
#pragma unroll
    for (int k = 0; k < G::VCL; ++k) acc[h][k] = allreduce_sum<G::VPR, 64>(acc[h][k]);
    if (lane < G::VPR) {
#pragma unroll
      for (int k = 0; k < G::VCL; ++k) acc_s[w][h][lane * G::VCL + k] = acc[h][k];
    }
    if (lane == 0) {
      m_s[w][h] = m_run[h];
      l_s[w][h] = lw;
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

hipError_t launch_decode_gqa(const DecodeArgs& a, int D, int v_dtype, int batch, int hg,
                             hipStream_t st) {
  dim3 grid(a.num_splits, a.num_q_heads / hg, batch);
#define FDI4_GQA(DD, VV, WW, HH)                                                          \
  if (D == DD && v_dtype == VV && a.waves == WW && hg == HH) {                            \
    hipLaunchKernelGGL((decode_gqa_kernel<DD, VV, WW, HH>), grid, dim3(WW * 64), 0, st, a); \
    return hipGetLastError();                                                             \
  }
#define FDI4_GQA_D(WW, HH)                                                               \
  FDI4_GQA(64, kVF32, WW, HH) FDI4_GQA(128, kVF32, WW, HH)                               \
  FDI4_GQA(64, kVF16, WW, HH) FDI4_GQA(128, kVF16, WW, HH)                               \
  FDI4_GQA(64, kVBF16, WW, HH) FDI4_GQA(128, kVBF16, WW, HH)
  FDI4_GQA_D(4, 2) FDI4_GQA_D(8, 2) FDI4_GQA_D(4, 4) FDI4_GQA_D(8, 4)
  // Eight heads per workgroup at D=64 only, and D=256 with four waves only:
  // other shapes would spill registers or overflow LDS.
  FDI4_GQA(64, kVF32, 4, 8) FDI4_GQA(64, kVF32, 8, 8) FDI4_GQA(64, kVF16, 4, 8)
  FDI4_GQA(64, kVF16, 8, 8) FDI4_GQA(64, kVBF16, 4, 8) FDI4_GQA(64, kVBF16, 8, 8)
  FDI4_GQA(256, kVF32, 4, 2) FDI4_GQA(256, kVF32, 4, 4) FDI4_GQA(256, kVF16, 4, 2)
  FDI4_GQA(256, kVF16, 4, 4) FDI4_GQA(256, kVBF16, 4, 2) FDI4_GQA(256, kVBF16, 4, 4)
#undef FDI4_GQA_D
#undef FDI4_GQA
  return hipErrorInvalidValue;
}

}  // namespace fdi4
