// Fused INT4 flash-decoding over paged, nibble-packed keys (gfx950).
//
// Semantics follow the reference page loop (src/flash_decode_ref.py:30-139,
// the CUDA kernel csrc/flash_decode_int4.cu:104-221): unscaled logits q.k
// with k = nib*scale - zp*scale, online softmax over the valid rows of every
// page in logical order, empty pages skipped, out = acc / max(l, 1e-10).
//
// Work decomposition (split-K flash decoding):
//   grid (num_splits, Hq, B); a workgroup of WAVES (4 or 8) wave64s owns
//   one split, a contiguous range of 16-row chunks of one (sequence,
//   q-head); each SIMD takes a quarter of the range, which its one wave
//   computes (four waves) or which is cut into ranges of its two waves
//   (eight: about 20:12 between the SIMD's older and younger wave with
//   float32 values at D = 128, 18:14 otherwise, the younger wave's last
//   chunks a range of their own, see wave_segments); every range keeps its
//   own (m, l, acc) and the ranges are merged through LDS in a fixed order.
//   (The fused serving step with four decode waves adds four helper waves
//   that re-quantize the open group and own no chunks.)
//   With one split the workgroup writes the output,
//   otherwise (m, l, acc[D]) goes to the workspace and merge_kernel combines
//   the splits with a log-sum-exp weighting.
//
// Per 16-row chunk and wave:
//   K: LPT lanes per row, each lane one 8/16-byte load of packed nibbles
//      (CPL channels). The logit is an fp64 dot product
//          sum_d (q_d*s_d) * nib_d  -  sum_d q_d*(zp_d*s_d)
//      whose products are exact in fp64; fp64 keeps the logit error ~1e-16
//      relative, far below the float32 oracle's own ~1e-6 noise at D=128.
//      (q_d*s_d) and the group constant are recomputed when the scale group
//      changes; the scale/zero-point block of the next group is prefetched
//      with one 16-byte load per lane and staged through LDS.
//   softmax: wave-wide fp64 max over the chunk (DPP / ds_swizzle / permlane
//      swaps), the hardware 2^x of the fp64 differences times log2(e)
//      (exp2_of; also in the LDS merge of the waves' partials and in the
//      split merge).
//   V: fully coalesced 16-byte loads (VPR lanes per row); the probabilities
//      go through a 16-entry LDS row per wave; float32 FMA accumulation.
//   The K and V loads of the next chunk are issued before the current chunk
//   is computed (one chunk of software prefetch per wave). Rows past the
//   valid count are loaded from the last valid row (never out of bounds) and
//   masked to probability 0.

#include <limits.h>

#include "decode_common.hpp"
#include "quant_common.hpp"

namespace fdi4 {

template <int D, int VDT>
struct Geo {
  static constexpr int LPT = (D == 256) ? 8 : 4;   // lanes per key row
  static constexpr int CPL = D / LPT;              // channels per lane (K)
  static constexpr int KBL = CPL / 2;              // packed bytes per lane per row
  static constexpr int KW = KBL / 4;               // 32-bit words per lane per row
  static constexpr int TPW = 64 / LPT;             // key rows per sweep
  static constexpr int KLD = 16 / TPW;             // key sweeps per chunk
  static constexpr int VEB = VDT == kVF32 ? 4 : 2; // bytes per value element (f16, bf16: 2)
  static constexpr int VCL = 16 / VEB;             // value channels per lane
  static constexpr int VPR = D / VCL;              // lanes per value row
  static constexpr int RPL = 64 / VPR;             // value rows per sweep
  static constexpr int VLD = 16 / RPL;             // value sweeps per chunk
  static constexpr int SZI = D / 2;                // 16-byte items in a scale+zp block
  static constexpr int SZL = (SZI + 63) / 64;      // scale+zp loads per lane
  static_assert(RPL >= 1 && 16 % RPL == 0 && 16 % TPW == 0, "geometry");
};

// The fused serving step's append (STEP instantiations): the calling wave
// re-quantizes channel quarter `slice` of the open group of token t of its
// (sequence, kv-head) (step_requant_slice); four waves make the whole append.
template <int D, int VEB>
__device__ __forceinline__ void step_append(const DecodeArgs& a, int b, int hk, int t, int slice,
                                            int lane, uint16_t* k_open, float* sz_open,
                                            U32x4* v_open, int* pt_w) {
  step_requant_slice<D, VEB>(a.step, const_cast<uint8_t*>(a.k_pages), a.k_page, a.k_head,
                             a.k_row, reinterpret_cast<uint8_t*>(const_cast<void*>(a.v_pages)),
                             a.v_page * VEB, a.v_head * VEB, a.v_row * VEB,
                             const_cast<float*>(a.k_scale), const_cast<float*>(a.k_zp), a.s_b,
                             a.s_h, a.s_g, a.page_table, a.pt_b, a.page_rows, a.num_pages, b, hk,
                             t, slice, lane, k_open, sz_open, v_open, pt_w);
}

// The fused serving step's length advance: every workgroup of sequence b
// counts its arrival once all its waves have read the old length; the last to
// arrive writes the new length and clears the counter for the next step. A
// relaxed device-scope atomic: the count is all the arrivals need to agree
// on. Called by one wave (its lane 0): with helper waves and 16-bit values the
// first helper, once its re-quantization is done (after the first workgroup
// barrier, every wave having used the length before it), so that the
// atomic's round trip passes under the decode; otherwise wave 0 at the
// workgroup's end. (On a streaming wave a returning atomic would hold up the
// waits of every later chunk load, which the hardware counts in order. In
// process A/B of the step, one box: the early count from the helper gains with
// 16-bit values, B8 H32 D128 float16 38.9 -> 37.8 us, bfloat16 37.3 -> 36.5,
// D64 float16 28.1 -> 23.8 with the helper waves, and loses with float32
// values, D128 53.3-54.0 -> 54.2-54.3 us.)
__device__ __forceinline__ void step_arrive(const DecodeArgs& a, int b, int lane,
                                            int len_after) {
  if (lane != 0) return;
  const int n = gridDim.x * gridDim.y;
  const int prev =
      __hip_atomic_fetch_add(a.step.arrive + b, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  if (prev == n - 1) {
    __hip_atomic_store(a.step.arrive + b, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    a.step.lens[b] = len_after;
  }
}

// One split's term of the log-sum-exp merge of an output element: split
// maximum m (-inf: the split holds no rows and adds nothing), its sum of
// probabilities lraw and weighted value acc, against the maximum ms over the
// splits.
__device__ __forceinline__ void merge_term(double m, double ms, float acc, double lraw, float& o,
                                           float& l) {
  if (m == -INFINITY) return;
  const float e = exp2_of(m - ms);
  o = __builtin_fmaf(e, acc, o);
  l = __builtin_fmaf(e, (float)lraw, l);
}

// Waves of a decode workgroup that only re-quantize: the fused serving step
// adds four, which re-quantize the open group while the decode waves stream,
// with four decode waves, and with eight where three waves per SIMD fit in
// the registers (16-bit values at head_dim <= 128, float32 values at 64).
// Otherwise (eight decode waves at head_dim 256, or float32 values at 128)
// the younger four decode waves re-quantize first, then decode.
template <int D, int VDT, int WAVES, bool STEP>
constexpr int helper_waves() {
  if (!STEP) return 0;
  if (WAVES == 4) return 4;
  return (VDT == kVF32 ? D == 64 : D <= 128) ? 4 : 0;
}

template <int D, int VDT, int WAVES, bool STEP>
__global__ __launch_bounds__((WAVES + helper_waves<D, VDT, WAVES, STEP>()) * 64) void
decode_kernel(DecodeArgs a) {
  using G = Geo<D, VDT>;
  constexpr int HW = helper_waves<D, VDT, WAVES, STEP>();
  // Where the serving step counts its arrival (step_arrive).
  constexpr bool kEarlyArrive = STEP && HW > 0 && VDT != kVF32;
  constexpr int NT = (WAVES + HW) * 64;

  const int split = blockIdx.x, h = blockIdx.y, b = blockIdx.z;
  const int hk = h / a.hq_per_kv;
  const int tid = threadIdx.x, lane = tid & 63;
  // The wave index is uniform across the wave; saying so keeps the chunk loop
  // counters in scalar registers and the page-table reads on the scalar unit.
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const bool helper = w >= WAVES;     // a re-quantizing helper wave (no chunks)
  const int kq = lane % G::LPT;       // channel slice of this lane (K)
  const int ktok = lane / G::LPT;     // key row within a sweep
  const int vrow = lane / G::VPR;     // value row within a sweep
  const int vcol = lane % G::VPR;     // value channel slice

  __shared__ float q_s[D];
  __shared__ float p_s[WAVES][16];
  __shared__ float sz_s[WAVES][2 * D];
  // Partials of the wave_segments ranges (12 with eight waves).
  static_assert(WAVES == 4 || WAVES == 8, "wave_segments assumes 4 or 8 waves");
  constexpr int NS = WAVES > 4 ? WAVES + 4 : WAVES;
  __shared__ float acc_s[NS][D];
  __shared__ double m_s[NS];
  __shared__ float l_s[NS];
  // With STEP: the open group's packed rows and scale/zero-point, as the
  // re-quantization left them (step_requant_slice).
  __shared__ __align__(16) uint16_t k_open[STEP ? kStepMaxGroup * D / 4 : 1];
  __shared__ float sz_open[STEP ? 2 * D : 1];
  __shared__ U32x4 v_open[STEP ? D * G::VEB / 16 : 1];
  // With STEP: each re-quantizing wave's copy of the group's page-table
  // entries, and the count of waves whose quarter of the append is in LDS.
  __shared__ int pt_w[STEP ? 4 : 1][STEP ? kStepMaxGroup : 1];
  __shared__ int open_done;

  const int cpp = (a.page_rows + 15) >> 4;
  // With STEP, token t_app = seq_lens[b] is appended when 0 <= t_app < cap
  // and the decode attends over t_app + 1 rows, the length advancing to
  // t_app + 1. A length outside [0, cap) appends nothing, is left as read,
  // and the decode attends over it clamped to [0, cap] -- what the append
  // kernel and the two-launch step do with such a length.
  int T, t_app = -1, len_after = 0;
  if constexpr (STEP) {
    const int cap = a.max_pages * a.page_rows;
    const int raw = ld_ro(a.seq_lens, b);
    const bool fits = raw >= 0 && raw < cap;
    t_app = fits ? raw : -1;
    T = fits ? raw + 1 : min(max(raw, 0), cap);
    len_after = fits ? raw + 1 : raw;
    // Where a helper wave counts the workgroup's arrival after the first
    // workgroup barrier (step_arrive), every wave holds the length read
    // before that barrier; a helper would otherwise first use it after it.
    if constexpr (kEarlyArrive) asm volatile("" ::"s"(raw));
  } else {
    T = seq_len_of(a, b);
  }
  // With a token to append, the open group's keys and scales come from
  // k_open / sz_open and row t_app's values from v_open while the cache's
  // copies are being written.
  const bool append = STEP && t_app >= 0;
  const int open_g = append ? t_app / a.step.group_rows : -1;
  const int n_chunks = pages_of(a, T) * cpp;
  const int c_begin = split * a.chunks_per_split;
  const int c_end = min(c_begin + a.chunks_per_split, n_chunks);
  // The split that holds the open group re-quantizes it (with several splits
  // the host fuses the append only where every split holds whole scale
  // groups, so the group lies in one split); the others only decode.
  const int c_open = open_g * a.pages_per_group * cpp;
  const bool owns_open = append && c_open >= c_begin && c_open < c_begin + a.chunks_per_split;
  // Where the serving step's younger decode waves re-quantize first, the
  // older waves take the last range of each SIMD (the same partials,
  // computed by other waves).
  const WaveSegs ws = wave_segments(c_begin, c_end, helper ? 0 : w, WAVES, owns_open && HW == 0,
                                    VDT == kVF32 && D == 128 ? kFirstShare32F32
                                                             : kFirstShare32);
  const int len1 = helper ? 0 : ws.p1 - ws.p0, len2 = helper ? 0 : ws.q1 - ws.q0;
  const int wlen = len1 + len2;
  // The wave's i-th chunk.
  auto cidx = [&](int i) { return i < len1 ? ws.p0 + i : ws.q0 + (i - len1); };
  // Segment 1's partial is written when the loop reaches segment 2.
  const bool seg_flush = ws.s2 >= 0 && len2 > 0;

  double m_run = -INFINITY;
  float l_lane = 0.f;
  float acc[G::VCL];
#pragma unroll
  for (int k = 0; k < G::VCL; ++k) acc[k] = 0.f;
  double qs[G::CPL];
  double cg = 0.0;
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
  const unsigned k_lane = kq * G::KBL, v_lane = vcol * 16;
  const unsigned krow_b = (unsigned)a.k_row, vrow_b = (unsigned)(a.v_row * G::VEB);

  // Scale/zero-point block of one group: items 0..D/4-1 are scale[4e..4e+3],
  // items D/4..D/2-1 are zp. Lanes past the block reload an in-range item.
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
#pragma unroll
    for (int i = 0; i < G::KLD; ++i) {
      const int t = max(min(i * G::TPW + ktok, m.nval - 1), 0);
      kr[i] = load_k<G::KW>(kb + (k_lane + (unsigned)t * krow_b));
    }
    const uint8_t* vb = vbase_h + (m.phys * a.v_page + (int64_t)m.r0 * a.v_row) * G::VEB;
#pragma unroll
    for (int i = 0; i < G::VLD; ++i) {
      const int r = max(min(i * G::RPL + vrow, m.nval - 1), 0);
      vr[i] = ld16_stream(vb + (v_lane + (unsigned)r * vrow_b));
    }
  };

  // One step: (1) stage a new scale group, (2) prefetch chunk c+1 into
  // `nk/nv` (chunk c again on the last step, an L2-resident reload, so that
  // every step issues the same loads and the wait counts stay exact),
  // (3) read the page-table entry of chunk c+2 on the scalar unit,
  // (4)-(6) consume chunk c from `ck/cv`. Called alternately with the two
  // buffers swapped (a two-way unrolled ping-pong), so no register copy waits
  // on the prefetch. An empty chunk (page_lens 0) is loaded from row 0 of its
  // page and skipped.
  int c = 0;
  ChunkMeta cm{}, nm{};
  U32x4 sz[G::SZL];
  auto meta_at = [&](int ci) { return chunk_meta(a, b, T, cpp, cidx(min(ci, wlen - 1))); };
  // Writes the wave's running partial (max logit, probability sum, weighted
  // values, each reduced over the wave) to LDS slot `slot` and restarts the
  // online softmax.
  auto flush = [&](int slot) {
    const float lw = allreduce_sum<1, 64>(l_lane);
    float at[G::VCL];
#pragma unroll
    for (int k = 0; k < G::VCL; ++k) at[k] = allreduce_sum<G::VPR, 64>(acc[k]);
    if (lane < G::VPR) {
#pragma unroll
      for (int k = 0; k < G::VCL; ++k) acc_s[slot][lane * G::VCL + k] = at[k];
    }
    if (lane == 0) {
      m_s[slot] = m_run;
      l_s[slot] = lw;
    }
    m_run = -INFINITY;
    l_lane = 0.f;
#pragma unroll
    for (int k = 0; k < G::VCL; ++k) acc[k] = 0.f;
  };
  auto step = [&](KVec<G::KW>* ck, U32x4* cv, KVec<G::KW>* nk, U32x4* nv) -> bool {
    if (seg_flush && c == len1) flush(ws.s1);
    if (cm.group != cur_group) {
      const bool open = STEP && cm.group == open_g;
      // The open group's keys, scales and new value row are read from LDS
      // once all four quarters of the append are there (each re-quantizing
      // wave counts itself in after its last LDS write; none of them waits
      // on another wave first, so the count always reaches four).
      if (open) {
        while (__hip_atomic_load(&open_done, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_WORKGROUP) < 4)
          __builtin_amdgcn_s_sleep(2);
      }
      float* szw = open ? sz_open : sz_s[w];
      if (!open) {
#pragma unroll
        for (int i = 0; i < G::SZL; ++i) {
          const int e = i * 64 + lane;
          if (e < G::SZI) *reinterpret_cast<U32x4*>(szw + 4 * e) = sz[i];
        }
      }
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
      double cgp = 0.0;
#pragma unroll
      for (int ci = 0; ci < G::CPL; ++ci) {
        const int d = kq * G::CPL + ci;
        const double qd = (double)q_s[d];
        const double sd = (double)szw[d];
        qs[ci] = qd * sd;
        cgp = __builtin_fma(qd, (double)szw[D + d] * sd, cgp);
      }
      cg = allreduce_sum<1, G::LPT>(cgp);
      cur_group = cm.group;
      __builtin_amdgcn_wave_barrier();
    }

    const bool last = c + 1 >= wlen;
    // Unconditional loads: a conditional load here makes the wait counts at
    // the loop back-edge conservative (a full drain of the prefetch). On the
    // last step nm is the current chunk; with one valid row every lane reads
    // that chunk's first row, so the dummy prefetch costs one row, not a page.
    ChunkMeta pf = nm;
    pf.nval = last ? 1 : nm.nval;
    load_sz(pf, sz);
    load_chunk(pf, nk, nv);
    const ChunkMeta nnm = meta_at(c + 2);
    if (cm.nval > 0) {

    // Keys of the open group (STEP) from k_open: the cache's copy is being
    // written meanwhile, and the loads of it into ck are not used.
    if constexpr (STEP) {
      if (cm.group == open_g) {
#pragma unroll
        for (int i = 0; i < G::KLD; ++i) {
          const int t = max(min(i * G::TPW + ktok, cm.nval - 1), 0);
          const int row = cm.tok0 + t - open_g * a.step.group_rows;
          ck[i] = *reinterpret_cast<const KVec<G::KW>*>(
              reinterpret_cast<const uint8_t*>(k_open) + row * (D / 2) + k_lane);
        }
      }
    }
    double lg[G::KLD];
#pragma unroll
    for (int i = 0; i < G::KLD; ++i) {
      double s0 = 0.0, s1 = 0.0, s2 = 0.0, s3 = 0.0;
#pragma unroll
      for (int wi = 0; wi < G::KW; ++wi) {
        const unsigned x = ck[i].w[wi];
        s0 = __builtin_fma((double)(x & 15u), qs[wi * 8 + 0], s0);
        s1 = __builtin_fma((double)((x >> 4) & 15u), qs[wi * 8 + 1], s1);
        s2 = __builtin_fma((double)((x >> 8) & 15u), qs[wi * 8 + 2], s2);
        s3 = __builtin_fma((double)((x >> 12) & 15u), qs[wi * 8 + 3], s3);
        s0 = __builtin_fma((double)((x >> 16) & 15u), qs[wi * 8 + 4], s0);
        s1 = __builtin_fma((double)((x >> 20) & 15u), qs[wi * 8 + 5], s1);
        s2 = __builtin_fma((double)((x >> 24) & 15u), qs[wi * 8 + 6], s2);
        s3 = __builtin_fma((double)(x >> 28), qs[wi * 8 + 7], s3);
      }
      double s = (s0 + s1) + (s2 + s3);
      s = allreduce_sum<1, G::LPT>(s);
      const int t = i * G::TPW + ktok;
      lg[i] = (t < cm.nval) ? s - cg : -INFINITY;
    }

    double mc = lg[0];
#pragma unroll
    for (int i = 1; i < G::KLD; ++i) mc = fmax(mc, lg[i]);
    mc = allreduce_max<G::LPT, 64>(mc);
    const double m_new = fmax(m_run, mc);
    const float corr = exp2_of(m_run - m_new);
    m_run = m_new;
    float psum = 0.f;
#pragma unroll
    for (int i = 0; i < G::KLD; ++i) {
      const float p = exp2_of(lg[i] - m_new);
      if (kq == 0) p_s[w][i * G::TPW + ktok] = p;
      psum += p;
    }
    l_lane = l_lane * corr + (kq == 0 ? psum : 0.f);
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");

    // Row t_app's values (STEP) from v_open: the cache's row is being written
    // meanwhile, and the loads of it into cv (also those of lanes past the
    // valid rows, which load the last valid row) are not used.
    if constexpr (STEP) {
      if ((unsigned)(t_app - cm.tok0) < (unsigned)cm.nval) {
        const U32x4 vo = v_open[v_lane / 16];
#pragma unroll
        for (int i = 0; i < G::VLD; ++i) {
          const int r = max(min(i * G::RPL + vrow, cm.nval - 1), 0);
          if (cm.tok0 + r == t_app) cv[i] = vo;
        }
      }
    }
#pragma unroll
    for (int k = 0; k < G::VCL; ++k) acc[k] *= corr;
#pragma unroll
    for (int i = 0; i < G::VLD; ++i) {
      const int r = i * G::RPL + vrow;
      const float p = (r < cm.nval) ? p_s[w][r] : 0.f;
      float vf[G::VCL];
      widen_values<VDT>(cv[i], vf);
#pragma unroll
      for (int k = 0; k < G::VCL; ++k) acc[k] = __builtin_fmaf(p, vf[k], acc[k]);
    }
    __builtin_amdgcn_wave_barrier();
    }
    c += 1;
    cm = nm;
    nm = nnm;
    return last;
  };

  // q is loaded first (one element per thread, D <= NT), then the first
  // chunk's loads are issued, then q is staged in LDS: the chunk latency
  // overlaps the q load and the workgroup barrier, and waiting for q (the
  // oldest load) does not wait for the chunk.
  static_assert(D <= NT, "one query element per thread");
  const float qv =
      (tid < D) ? load_elem(a.q, (int64_t)b * a.q_b + (int64_t)h * a.q_h + tid, a.q_dtype) : 0.f;
  const bool has_work = wlen > 0;
  KVec<G::KW> ka[G::KLD], kb[G::KLD];
  U32x4 va[G::VLD], vb[G::VLD];
  // A re-quantizing wave (STEP) loads its first chunk after its quarter of
  // the append where the chunk's registers would not fit beside the rows
  // (head_dim 256, float32 values).
  constexpr bool kLateFirst = STEP && D == 256 && VDT == kVF32;
  const bool rq_wave = STEP && owns_open && w >= WAVES + HW - 4;
  auto first_loads = [&]() {
    cm = meta_at(c);
    nm = meta_at(c + 1);
    load_sz(cm, sz);
    load_chunk(cm, ka, va);
  };
  if (has_work && !(kLateFirst && rq_wave)) first_loads();
  if constexpr (STEP) {
    if (tid == 0) open_done = 0;
  }
  if (tid < D) q_s[tid] = qv;
  __syncthreads();
  // With a token to append, the last four waves (the helpers, or with eight
  // decode waves the second wave of each SIMD, whose delay the first waves'
  // streaming absorbs) each re-quantize a quarter of the open group's
  // channels, then decode what they own.
  if constexpr (STEP) {
    if (rq_wave) {
      const int slice = w - (WAVES + HW - 4);
      step_append<D, G::VEB>(a, b, hk, t_app, slice, lane, k_open, sz_open, v_open, pt_w[slice]);
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
      if (lane == 0)
        __hip_atomic_fetch_add(&open_done, 1, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_WORKGROUP);
      if (kLateFirst && has_work) first_loads();
    }
    if constexpr (kEarlyArrive) {
      if (w == WAVES) step_arrive(a, b, lane, len_after);
    }
  }
  if (has_work) {
    while (true) {
      if (step(ka, va, kb, vb)) break;
      if (step(kb, vb, ka, va)) break;
    }
  }

  // The last segment's partial; a range that this wave owns but that is
  // empty (C with no chunks) gets the empty partial. Helpers own none.
  if (!helper) {
    flush(seg_flush ? ws.s2 : ws.s1);
    if (ws.s2 >= 0 && !seg_flush) flush(ws.s2);
  }
  __syncthreads();

  double ms = -INFINITY;
#pragma unroll
  for (int i = 0; i < NS; ++i) ms = fmax(ms, m_s[i]);
  float ew[NS];
  float l = 0.f;
#pragma unroll
  for (int i = 0; i < NS; ++i) {
    ew[i] = (m_s[i] == -INFINITY) ? 0.f : exp2_of(m_s[i] - ms);
    l = __builtin_fmaf(ew[i], l_s[i], l);
  }
  const int64_t pi = ((int64_t)b * a.num_q_heads + h) * a.num_splits + split;
  for (int d = tid; d < D; d += NT) {
    float o = 0.f;
#pragma unroll
    for (int i = 0; i < NS; ++i) o = __builtin_fmaf(ew[i], acc_s[i][d], o);
    if (a.final_out) {
      store_elem(a.out, (int64_t)b * a.o_b + (int64_t)h * a.o_h + d, a.out_dtype,
                 o / fmaxf(l, 1e-10f));
    } else {
      a.ws_acc[pi * D + d] = o;
    }
  }
  if (!a.final_out && tid == 0) {
    a.ws_ml[2 * pi] = ms;
    a.ws_ml[2 * pi + 1] = (double)l;
  }
  hand_back_length(a, b);
  if constexpr (STEP && !kEarlyArrive) {
    if (w == 0) step_arrive(a, b, lane, len_after);
  }
}

// Log-sum-exp merge of the split partials: grid (Hq, B), one thread per
// channel. Split s adds nothing when its maximum is -inf (no rows); the
// others add exp(m_s - max) times their values and sums, in split order. Up
// to eight splits every partial a thread needs is loaded in one round
// (indices clamped to the last split, the extra loads unused); more splits
// take the loop.
template <int D>
__global__ __launch_bounds__(D) void merge_kernel(const float* __restrict__ ws_acc,
                                                  const double* __restrict__ ws_ml, int hq,
                                                  int splits, void* __restrict__ out,
                                                  int out_dtype, int64_t o_b, int64_t o_h) {
  const int h = blockIdx.x, b = blockIdx.y, d = threadIdx.x;
  const int64_t p0 = ((int64_t)b * hq + h) * splits;
  double ms = -INFINITY;
  float o = 0.f, l = 0.f;
  if (splits <= 8) {
    double mv[8], lv[8];
    float av[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int64_t p = p0 + min(j, splits - 1);
      mv[j] = ws_ml[2 * p];
      lv[j] = ws_ml[2 * p + 1];
      av[j] = ws_acc[p * D + d];
    }
    // Each value is used only under its split's condition; without this the
    // compiler moves every load into its branch, one memory round per split.
#pragma unroll
    for (int j = 0; j < 8; ++j) asm volatile("" ::"v"(av[j]));
#pragma unroll
    for (int j = 0; j < 8; ++j)
      if (j < splits) ms = fmax(ms, mv[j]);
#pragma unroll
    for (int j = 0; j < 8; ++j)
      if (j < splits) merge_term(mv[j], ms, av[j], lv[j], o, l);
  } else {
    for (int s = 0; s < splits; ++s) ms = fmax(ms, ws_ml[2 * (p0 + s)]);
    for (int s = 0; s < splits; ++s)
      merge_term(ws_ml[2 * (p0 + s)], ms, ws_acc[(p0 + s) * D + d], ws_ml[2 * (p0 + s) + 1], o,
                 l);
  }
  store_elem(out, (int64_t)b * o_b + (int64_t)h * o_h + d, out_dtype, o / fmaxf(l, 1e-10f));
}

hipError_t launch_decode(const DecodeArgs& a, int D, int v_dtype, int batch, hipStream_t st) {
  dim3 grid(a.num_splits, a.num_q_heads, batch);
#define FDI4_DEC(DD, VV, WW)                                                             \
  if (D == DD && v_dtype == VV && a.waves == WW) {                                       \
    if (a.step.k_new)                                                                    \
      hipLaunchKernelGGL((decode_kernel<DD, VV, WW, true>), grid,                        \
                         dim3((WW + helper_waves<DD, VV, WW, true>()) * 64), 0, st, a);      \
    else                                                                                 \
      hipLaunchKernelGGL((decode_kernel<DD, VV, WW, false>), grid, dim3(WW * 64), 0, st, a); \
    return hipGetLastError();                                                            \
  }
  FDI4_DEC(64, kVF32, 4) FDI4_DEC(128, kVF32, 4) FDI4_DEC(256, kVF32, 4)
  FDI4_DEC(64, kVF16, 4) FDI4_DEC(128, kVF16, 4) FDI4_DEC(256, kVF16, 4)
  FDI4_DEC(64, kVF32, 8) FDI4_DEC(128, kVF32, 8) FDI4_DEC(256, kVF32, 8)
  FDI4_DEC(64, kVF16, 8) FDI4_DEC(128, kVF16, 8) FDI4_DEC(256, kVF16, 8)
  FDI4_DEC(64, kVBF16, 4) FDI4_DEC(128, kVBF16, 4) FDI4_DEC(256, kVBF16, 4)
  FDI4_DEC(64, kVBF16, 8) FDI4_DEC(128, kVBF16, 8) FDI4_DEC(256, kVBF16, 8)
#undef FDI4_DEC
  return hipErrorInvalidValue;
}

hipError_t launch_merge(const float* ws_acc, const double* ws_ml, int batch, int hq, int D,
                        int splits, void* out, int out_dtype, int64_t o_b, int64_t o_h,
                        hipStream_t st) {
  dim3 grid(hq, batch);
#define FDI4_MRG(DD)                                                                         \
  if (D == DD) {                                                                             \
    hipLaunchKernelGGL((merge_kernel<DD>), grid, dim3(DD), 0, st, ws_acc, ws_ml, hq, splits, \
                       out, out_dtype, o_b, o_h);                                            \
    return hipGetLastError();                                                                \
  }
  FDI4_MRG(64) FDI4_MRG(128) FDI4_MRG(256)
#undef FDI4_MRG
  return hipErrorInvalidValue;
}

// Copy rows of `cols` floats into rows of `d_cols` floats, zero-filling the tail.
__global__ __launch_bounds__(256) void pad_rows_kernel(const float* __restrict__ src, int64_t rows,
                                                       int cols, int64_t s_stride,
                                                       float* __restrict__ dst, int64_t d_stride,
                                                       int d_cols) {
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (idx >= rows * d_cols) return;
  const int64_t r = idx / d_cols;
  const int c = (int)(idx % d_cols);
  dst[r * d_stride + c] = (c < cols) ? src[r * s_stride + c] : 0.f;
}

hipError_t launch_pad_rows(const float* src, int64_t rows, int cols, int64_t s_stride, float* dst,
                           int64_t d_stride, int d_cols, hipStream_t st) {
  const int64_t total = rows * d_cols;
  if (total == 0) return hipSuccess;
  hipLaunchKernelGGL(pad_rows_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, st,
                     src, rows, cols, s_stride, dst, d_stride, d_cols);
  return hipGetLastError();
}

}  // namespace fdi4
