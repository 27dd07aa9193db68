// INT4 key quantizer kernels for gfx950.
//
// Arithmetic (bit-exact with the NumPy quantizer, reference
// src/quantize_int4_ref.py:46-84): per channel over the group's valid rows,
//   mn, mx = min, max                     (exact)
//   span   = fmaxf(mx - mn, 1e-8f)        (float32 floor, as NumPy casts 1e-8)
//   scale  = span / 15.0f                 (IEEE division)
//   zp     = (-mn) / scale                (IEEE division)
//   q      = clamp(rintf((x - mn) / scale), 0, 15)   (round half to even)
// This file is compiled with -ffp-contract=off and without fast-math so that
// every operation above is one correctly rounded float32 operation. The
// grouped kernel forms the quotient (x - mn) / scale from the channel's
// reciprocal with one FMA correction step (quant_bin_rc), which returns the
// same correctly rounded quotient for a third of the instructions.
//
// Kernels
//   rows_minmax_kernel / rows_finalize_kernel / rows_quantize_kernel
//       the 2-D contract: one scale group over all rows of [rows, C]
//       (reference csrc/flash_decode_int4.cu:27-83), split over row tiles so
//       that any row count fills the chip; unpacked or nibble-packed output.
//   quantize_paged_kernel<D, GROUP>
//       one workgroup per (group, kv-head, sequence), dealt to the XCDs in
//       runs of consecutive groups of a (sequence, kv-head): 16-byte token-major
//       non-temporal loads held in registers, wave64 min/max reduction,
//       quantize from registers, nibble pack, and 16-byte non-temporal stores
//       of whole page rows through the page table.
//   append_paged_kernel<D, GROUP>
//       decode-time append: one workgroup per (kv-head, sequence) writes the
//       token at position seq_lens[b] (value row to its page, key row to the
//       staging rows of the open group) and re-quantizes that group over its
//       valid rows, exactly what the grouped quantizer gives for the whole
//       sequence; optionally writes the advanced length to a second array.
//   pack_kernel   device form of the nibble packing (reference src/int4_pack.py:14-29)

#include "fdi4_device.hpp"
#include "fdi4_internal.hpp"
#include "quant_common.hpp"

namespace fdi4 {

// ---------------------------------------------------------------------------
// 2-D contract: [rows, C] row-major, one group over all rows.
// ---------------------------------------------------------------------------

constexpr int kRowsThreads = 256;
constexpr int kRowsTile = 256;  // rows per partial

// grid (ceil(C/64), n_tiles); lane -> channel, wave -> row phase.
__global__ __launch_bounds__(kRowsThreads) void rows_minmax_kernel(
    const float* __restrict__ kv, int64_t rows, int C, int64_t stride,
    float2* __restrict__ partial) {
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const int c = blockIdx.x * 64 + lane;
  const int64_t r0 = (int64_t)blockIdx.y * kRowsTile;
  const int64_t r1 = min(r0 + kRowsTile, rows);
  float mn = INFINITY, mx = -INFINITY;
  if (c < C) {
    for (int64_t r = r0 + wv; r < r1; r += kRowsThreads / 64) {
      const float x = kv[r * stride + c];
      mn = fminf(mn, x);
      mx = fmaxf(mx, x);
    }
  }
  __shared__ float smn[kRowsThreads / 64][64], smx[kRowsThreads / 64][64];
  smn[wv][lane] = mn;
  smx[wv][lane] = mx;
  __syncthreads();
  if (wv == 0 && c < C) {
#pragma unroll
    for (int w = 1; w < kRowsThreads / 64; ++w) {
      mn = fminf(mn, smn[w][lane]);
      mx = fmaxf(mx, smx[w][lane]);
    }
    partial[(int64_t)blockIdx.y * C + c] = make_float2(mn, mx);
  }
}

// grid ceil(C/256): thread -> channel.
__global__ __launch_bounds__(256) void rows_finalize_kernel(
    const float2* __restrict__ partial, int n_tiles, int C, float* __restrict__ scale_out,
    float* __restrict__ zp_out, float2* __restrict__ mn_scale) {
  const int c = blockIdx.x * 256 + threadIdx.x;
  if (c >= C) return;
  float mn = INFINITY, mx = -INFINITY;
  for (int t = 0; t < n_tiles; ++t) {
    const float2 p = partial[(int64_t)t * C + c];
    mn = fminf(mn, p.x);
    mx = fmaxf(mx, p.y);
  }
  float s, z;
  scale_zp(mn, mx, &s, &z);
  scale_out[c] = s;
  zp_out[c] = z;
  mn_scale[c] = make_float2(mn, s);
}

// Unpacked: grid (ceil(C/64), ceil(rows/kRowsTile)); lane -> channel.
// Packed:   grid (ceil(ceil(C/2)/64), ...);           lane -> output byte.
template <bool PACKED>
__global__ __launch_bounds__(kRowsThreads) void rows_quantize_kernel(
    const float* __restrict__ kv, int64_t rows, int C, int64_t stride,
    const float2* __restrict__ mn_scale, uint8_t* __restrict__ q, int64_t q_stride) {
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const int j = blockIdx.x * 64 + lane;
  const int64_t r0 = (int64_t)blockIdx.y * kRowsTile;
  const int64_t r1 = min(r0 + kRowsTile, rows);
  if (!PACKED) {
    if (j >= C) return;
    const float2 ms = mn_scale[j];
    for (int64_t r = r0 + wv; r < r1; r += kRowsThreads / 64)
      q[r * q_stride + j] = (uint8_t)quant_bin(kv[r * stride + j], ms.x, ms.y);
  } else {
    const int c0 = 2 * j, c1 = 2 * j + 1;
    if (c0 >= C) return;
    const float2 m0 = mn_scale[c0];
    const bool has1 = c1 < C;
    const float2 m1 = has1 ? mn_scale[c1] : make_float2(0.f, 1.f);
    for (int64_t r = r0 + wv; r < r1; r += kRowsThreads / 64) {
      const unsigned lo = quant_bin(kv[r * stride + c0], m0.x, m0.y);
      const unsigned hi = has1 ? quant_bin(kv[r * stride + c1], m1.x, m1.y) : 0u;
      q[r * q_stride + j] = (uint8_t)(lo | (hi << 4));
    }
  }
}

// ---- 2-D contract, 16-byte path (C % 4 == 0, 16-byte aligned rows) -------------
//
// A row's channels are cut into slices of 32 (128 bytes, one cache line);
// eight lanes cover a slice of one row with one 16-byte load each, so a wave
// reads 8 rows of a slice and every load instruction is independent of the
// others (the scalar kernels above make one dependent 4-byte load per row and
// are latency-bound). Lanes of an idle slice tail (C not a multiple of 32)
// load the last full 4-channel group and store nothing.

constexpr int kSliceCh = 32;

struct RowsVecArgs {
  const float* kv;
  int64_t rows, stride;                  // elements
  int C;
  uint8_t* q;
  int64_t q_stride;                      // bytes
  int packed;                            // nibble pairs, else one bin per byte
  int q_word;                            // q and q_stride allow 4-byte (2-byte packed) stores
  float* scale;
  float* zp;
};

// Extremes of this thread's NI float4 into mn/mx (4 channels each).
template <int NI>
__device__ __forceinline__ void minmax4(const float4* x, float* mn, float* mx) {
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    mn[k] = INFINITY;
    mx[k] = -INFINITY;
  }
#pragma unroll
  for (int i = 0; i < NI; ++i) {
    mn[0] = fminf(mn[0], x[i].x); mx[0] = fmaxf(mx[0], x[i].x);
    mn[1] = fminf(mn[1], x[i].y); mx[1] = fmaxf(mx[1], x[i].y);
    mn[2] = fminf(mn[2], x[i].z); mx[2] = fmaxf(mx[2], x[i].z);
    mn[3] = fminf(mn[3], x[i].w); mx[3] = fmaxf(mx[3], x[i].w);
  }
}

// Bins of one row's 4 channels c0..c0+3, stored unpacked (4 bytes) or packed
// (2 bytes) at row r.
__device__ __forceinline__ void store_bins4(const RowsVecArgs& a, int64_t r, int c0, float4 x,
                                            const float* mn, const float* sc, const float* rc) {
  const unsigned n0 = (unsigned)quant_bin_rc(x.x, mn[0], sc[0], rc[0]);
  const unsigned n1 = (unsigned)quant_bin_rc(x.y, mn[1], sc[1], rc[1]);
  const unsigned n2 = (unsigned)quant_bin_rc(x.z, mn[2], sc[2], rc[2]);
  const unsigned n3 = (unsigned)quant_bin_rc(x.w, mn[3], sc[3], rc[3]);
  uint8_t* row = a.q + r * a.q_stride;
  if (!a.packed) {
    if (a.q_word) {
      *reinterpret_cast<unsigned*>(row + c0) = n0 | (n1 << 8) | (n2 << 16) | (n3 << 24);
    } else {
      row[c0] = (uint8_t)n0; row[c0 + 1] = (uint8_t)n1;
      row[c0 + 2] = (uint8_t)n2; row[c0 + 3] = (uint8_t)n3;
    }
  } else {
    const unsigned lo = n0 | (n1 << 4), hi = n2 | (n3 << 4);
    if (a.q_word) {
      *reinterpret_cast<uint16_t*>(row + c0 / 2) = (uint16_t)(lo | (hi << 8));
    } else {
      row[c0 / 2] = (uint8_t)lo;
      row[c0 / 2 + 1] = (uint8_t)hi;
    }
  }
}

// Whole contract in one launch: one workgroup per slice of SW channels (SW/4
// lanes per row, NT*4/SW rows per sweep) holds every row of its slice in
// registers (NI rows per thread), reduces the extremes (lane butterflies over
// the row bits, then LDS across the waves), writes scale and zero-point and
// stores the bins. The input is read once. Narrow slices give small inputs
// more workgroups (more CUs pulling data).
template <int NT, int NI, int SW>
__global__ __launch_bounds__(NT) void rows_single_kernel(RowsVecArgs a) {
  constexpr int LPR = SW / 4, RPS = NT / LPR, NWAVE = NT / 64;
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int sub = tid % LPR, rsub = tid / LPR;
  const int c0 = blockIdx.x * SW + sub * 4;
  const bool cval = c0 < a.C;
  const int cl = cval ? c0 : a.C - 4;
  float4 x[NI];
#pragma unroll
  for (int i = 0; i < NI; ++i) {
    const int64_t r = min((int64_t)(rsub + i * RPS), a.rows - 1);
    x[i] = ld16f_stream(a.kv + r * a.stride + cl);
  }
  float mn[4], mx[4];
  minmax4<NI>(x, mn, mx);
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    mn[k] = allreduce_min_f<LPR, 64>(mn[k]);
    mx[k] = allreduce_max_f<LPR, 64>(mx[k]);
  }
  __shared__ float4 s_mn[NWAVE][LPR], s_mx[NWAVE][LPR];
  if (lane < LPR) {
    s_mn[wv][lane] = make_float4(mn[0], mn[1], mn[2], mn[3]);
    s_mx[wv][lane] = make_float4(mx[0], mx[1], mx[2], mx[3]);
  }
  __syncthreads();
#pragma unroll
  for (int w = 0; w < NWAVE; ++w) {
    const float4 pm = s_mn[w][sub], px = s_mx[w][sub];
    mn[0] = fminf(mn[0], pm.x); mx[0] = fmaxf(mx[0], px.x);
    mn[1] = fminf(mn[1], pm.y); mx[1] = fmaxf(mx[1], px.y);
    mn[2] = fminf(mn[2], pm.z); mx[2] = fmaxf(mx[2], px.z);
    mn[3] = fminf(mn[3], pm.w); mx[3] = fmaxf(mx[3], px.w);
  }
  if (!cval) return;
  float sc[4], zp[4], rc[4];
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    scale_zp(mn[k], mx[k], &sc[k], &zp[k]);
    rc[k] = 1.0f / sc[k];
  }
  if (rsub == 0) {
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      a.scale[c0 + k] = sc[k];
      a.zp[c0 + k] = zp[k];
    }
  }
#pragma unroll
  for (int i = 0; i < NI; ++i) {
    const int r = rsub + i * RPS;
    if (r < a.rows) store_bins4(a, r, c0, x[i], mn, sc, rc);
  }
}

// Multi-pass form for more rows: tiles of kRowsTile rows; 256 threads cover
// 32 rows of a slice per sweep, 8 sweeps per tile.
constexpr int kVecSweeps = kRowsTile / (kRowsThreads / 8);

// Pass 1: per-tile extremes, partial[tile * C + c] = (min, max).
__global__ __launch_bounds__(kRowsThreads) void rows_minmax_vec_kernel(RowsVecArgs a,
                                                                       float2* __restrict__ partial) {
  constexpr int RPS = kRowsThreads / 8;
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int sub = tid & 7, rsub = tid >> 3;
  const int c0 = blockIdx.x * kSliceCh + sub * 4;
  const bool cval = c0 < a.C;
  const int cl = cval ? c0 : a.C - 4;
  const int64_t r0 = (int64_t)blockIdx.y * kRowsTile;
  const int64_t rlast = min(r0 + kRowsTile, a.rows) - 1;
  float4 x[kVecSweeps];
#pragma unroll
  for (int i = 0; i < kVecSweeps; ++i) {
    const int64_t r = min(r0 + rsub + i * RPS, rlast);
    x[i] = ld16f_stream(a.kv + r * a.stride + cl);
  }
  float mn[4], mx[4];
  minmax4<kVecSweeps>(x, mn, mx);
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    mn[k] = allreduce_min_f<8, 64>(mn[k]);
    mx[k] = allreduce_max_f<8, 64>(mx[k]);
  }
  __shared__ float4 s_mn[kRowsThreads / 64][8], s_mx[kRowsThreads / 64][8];
  if (lane < 8) {
    s_mn[wv][lane] = make_float4(mn[0], mn[1], mn[2], mn[3]);
    s_mx[wv][lane] = make_float4(mx[0], mx[1], mx[2], mx[3]);
  }
  __syncthreads();
  if (wv != 0 || lane >= 8 || !cval) return;
#pragma unroll
  for (int w = 1; w < kRowsThreads / 64; ++w) {
    const float4 pm = s_mn[w][lane], px = s_mx[w][lane];
    mn[0] = fminf(mn[0], pm.x); mx[0] = fmaxf(mx[0], px.x);
    mn[1] = fminf(mn[1], pm.y); mx[1] = fmaxf(mx[1], px.y);
    mn[2] = fminf(mn[2], pm.z); mx[2] = fmaxf(mx[2], px.z);
    mn[3] = fminf(mn[3], pm.w); mx[3] = fmaxf(mx[3], px.w);
  }
  float2* dst = partial + (int64_t)blockIdx.y * a.C + c0;
#pragma unroll
  for (int k = 0; k < 4; ++k) dst[k] = make_float2(mn[k], mx[k]);
}

// Pass 2: one workgroup per 64 channels; wave w combines tiles w, w + 4, ...
// (8 independent loads in flight per lane), the waves meet in LDS; writes
// scale, zero-point and (min, scale) for pass 3.
__global__ __launch_bounds__(kRowsThreads) void rows_finalize_vec_kernel(
    const float2* __restrict__ partial, int n_tiles, int C, float* __restrict__ scale_out,
    float* __restrict__ zp_out, float2* __restrict__ mn_scale) {
  constexpr int NW = kRowsThreads / 64, U = 8;
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const int c = blockIdx.x * 64 + lane;
  float mn = INFINITY, mx = -INFINITY;
  if (c < C) {
    for (int t0 = wv; t0 < n_tiles; t0 += NW * U) {
      float2 p[U];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int t = min(t0 + u * NW, n_tiles - 1);
        p[u] = partial[(int64_t)t * C + c];
      }
#pragma unroll
      for (int u = 0; u < U; ++u) {
        mn = fminf(mn, p[u].x);
        mx = fmaxf(mx, p[u].y);
      }
    }
  }
  __shared__ float s_mn[NW][64], s_mx[NW][64];
  s_mn[wv][lane] = mn;
  s_mx[wv][lane] = mx;
  __syncthreads();
  if (wv != 0 || c >= C) return;
#pragma unroll
  for (int w = 1; w < NW; ++w) {
    mn = fminf(mn, s_mn[w][lane]);
    mx = fmaxf(mx, s_mx[w][lane]);
  }
  float s, z;
  scale_zp(mn, mx, &s, &z);
  scale_out[c] = s;
  zp_out[c] = z;
  mn_scale[c] = make_float2(mn, s);
}

// Pass 3: bins of one tile (layout of pass 1).
__global__ __launch_bounds__(kRowsThreads) void rows_quantize_vec_kernel(
    RowsVecArgs a, const float2* __restrict__ mn_scale) {
  constexpr int RPS = kRowsThreads / 8;
  const int tid = threadIdx.x, sub = tid & 7, rsub = tid >> 3;
  const int c0 = blockIdx.x * kSliceCh + sub * 4;
  if (c0 >= a.C) return;
  const int64_t r0 = (int64_t)blockIdx.y * kRowsTile;
  const int64_t rlast = min(r0 + kRowsTile, a.rows) - 1;
  float4 x[kVecSweeps];
#pragma unroll
  for (int i = 0; i < kVecSweeps; ++i) {
    const int64_t r = min(r0 + rsub + i * RPS, rlast);
    x[i] = ld16f_stream(a.kv + r * a.stride + c0);
  }
  float mn[4], sc[4], rc[4];
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const float2 m = mn_scale[c0 + k];
    mn[k] = m.x;
    sc[k] = m.y;
    rc[k] = 1.0f / m.y;
  }
#pragma unroll
  for (int i = 0; i < kVecSweeps; ++i) {
    const int64_t r = r0 + rsub + i * RPS;
    if (r <= rlast) store_bins4(a, r, c0, x[i], mn, sc, rc);
  }
}

// Passes 2 and 3 in one launch for few tiles (graph-replayed GPU time on
// MI355X against three launches: 2048 x 128 7.2 against 8.5 us, 16384 x 128
// 8.6 against 10.7, 32768 x 128 12.4 against 14.8):
// every workgroup reduces the tile extremes of its 32 channels itself (at
// most MAXT x 32 partials, L2-resident after the first reads), the workgroups
// of tile 0 write scale and zero-point, and each quantizes its tile. The
// tile's rows are loaded first so that their latency overlaps the reduction.
// Every workgroup reads all tiles' partials of its slice, tiles^2 * C * 8 / 32
// bytes in all, so the fused form is limited to 64 tiles, or 128 for rows of
// at most kFused128MaxC channels (at C = 1024 and 128 tiles three launches
// are faster: 67.2 against 68.8 us).
constexpr int kFused128MaxC = 256;

template <int MAXT>
__global__ __launch_bounds__(kRowsThreads) void rows_finalize_quantize_vec_kernel(
    RowsVecArgs a, const float2* __restrict__ partial, int n_tiles) {
  constexpr int RPS = kRowsThreads / 8, TG = kRowsThreads / kSliceCh;
  const int tid = threadIdx.x, sub = tid & 7, rsub = tid >> 3;
  const int c0 = blockIdx.x * kSliceCh + sub * 4;
  const bool cval = c0 < a.C;
  const int cl = cval ? c0 : a.C - 4;
  const int64_t r0 = (int64_t)blockIdx.y * kRowsTile;
  const int64_t rlast = min(r0 + kRowsTile, a.rows) - 1;
  float4 x[kVecSweeps];
#pragma unroll
  for (int i = 0; i < kVecSweeps; ++i) {
    const int64_t r = min(r0 + rsub + i * RPS, rlast);
    x[i] = ld16f_stream(a.kv + r * a.stride + cl);
  }
  // Thread t reduces channel t % 32 of the slice over tiles t / 32 + TG * j.
  const int ch = blockIdx.x * kSliceCh + (tid % kSliceCh);
  const int chl = min(ch, a.C - 1);
  float mn = INFINITY, mx = -INFINITY;
  float2 p[MAXT / TG];
#pragma unroll
  for (int j = 0; j < MAXT / TG; ++j) {
    const int t = min(tid / kSliceCh + TG * j, n_tiles - 1);
    p[j] = partial[(int64_t)t * a.C + chl];
  }
#pragma unroll
  for (int j = 0; j < MAXT / TG; ++j) {
    mn = fminf(mn, p[j].x);
    mx = fmaxf(mx, p[j].y);
  }
  __shared__ float s_mn[TG][kSliceCh], s_mx[TG][kSliceCh];
  s_mn[tid / kSliceCh][tid % kSliceCh] = mn;
  s_mx[tid / kSliceCh][tid % kSliceCh] = mx;
  __syncthreads();
  if (!cval) return;
  float cmn[4], sc[4], zp[4], rc[4];
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    float lo = INFINITY, hi = -INFINITY;
#pragma unroll
    for (int g = 0; g < TG; ++g) {
      lo = fminf(lo, s_mn[g][sub * 4 + k]);
      hi = fmaxf(hi, s_mx[g][sub * 4 + k]);
    }
    cmn[k] = lo;
    scale_zp(lo, hi, &sc[k], &zp[k]);
    rc[k] = 1.0f / sc[k];
  }
  if (blockIdx.y == 0 && rsub == 0) {
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      a.scale[c0 + k] = sc[k];
      a.zp[c0 + k] = zp[k];
    }
  }
#pragma unroll
  for (int i = 0; i < kVecSweeps; ++i) {
    const int64_t r = r0 + rsub + i * RPS;
    if (r <= rlast) store_bins4(a, r, c0, x[i], cmn, sc, rc);
  }
}

constexpr int kSingleThreads = 512;

// The one-launch kernel runs up to kSingleMaxRows rows (kSingleMaxRowsNarrow
// for rows of at most kNarrowC channels); beyond, the passes are faster. GPU
// time of graph-replayed calls on MI355X, one launch against extremes +
// fused finalize-and-bins: 128 x 128 3.4 against 5.3 us, 512 x 128 6.1
// against 6.1, 768 x 128 7.1 against 6.4, 1024 x 128 8.1 against 6.6 (C = 64
// and 1024 alike); 1024 x 8 3.5 against 6.5. The one-launch kernel's threads
// walk long columns of narrow slices, which for wide rows fetch each line
// from several workgroups; the passes spread any row count over the chip.
constexpr int64_t kSingleMaxRows = 512;
constexpr int64_t kSingleMaxRowsNarrow = 1024;
constexpr int kNarrowC = 16;

// Slice width of the one-launch kernel: the widest of 32, 16, 8, 4 channels
// that still gives kSingleMinGroups workgroups (else 4), and the rows per
// thread it then needs (at most 16 within the row limits); 0 beyond 16.
constexpr int kSingleMinGroups = 64;

void pick_single(int64_t rows, int C, int* sw, int* ni) {
  int w = 4;
  for (int c : {32, 16, 8})
    if ((C + c - 1) / c >= kSingleMinGroups) { w = c; break; }
  const int64_t rps = kSingleThreads / (w / 4);
  const int64_t per = (rows + rps - 1) / rps;
  *sw = w;
  *ni = per <= 1 ? 1 : per <= 2 ? 2 : per <= 4 ? 4 : per <= 8 ? 8 : per <= 16 ? 16 : 0;
}

template <int SW>
hipError_t launch_single(const RowsVecArgs& a, int ni, hipStream_t st) {
  const dim3 grid((unsigned)((a.C + SW - 1) / SW)), blk(kSingleThreads);
  switch (ni) {
    case 1: hipLaunchKernelGGL((rows_single_kernel<kSingleThreads, 1, SW>), grid, blk, 0, st, a); break;
    case 2: hipLaunchKernelGGL((rows_single_kernel<kSingleThreads, 2, SW>), grid, blk, 0, st, a); break;
    case 4: hipLaunchKernelGGL((rows_single_kernel<kSingleThreads, 4, SW>), grid, blk, 0, st, a); break;
    case 8: hipLaunchKernelGGL((rows_single_kernel<kSingleThreads, 8, SW>), grid, blk, 0, st, a); break;
    default: hipLaunchKernelGGL((rows_single_kernel<kSingleThreads, 16, SW>), grid, blk, 0, st, a); break;
  }
  return hipGetLastError();
}

hipError_t launch_quantize_rows_vec(const RowsVecArgs& a, void* ws, hipStream_t st) {
  const unsigned slices = (unsigned)((a.C + kSliceCh - 1) / kSliceCh);
  int sw, ni;
  pick_single(a.rows, a.C, &sw, &ni);
  const int64_t single_max = a.C <= kNarrowC ? kSingleMaxRowsNarrow : kSingleMaxRows;
  if (ni > 0 && a.rows <= single_max) {
    switch (sw) {
      case 32: return launch_single<32>(a, ni, st);
      case 16: return launch_single<16>(a, ni, st);
      case 8: return launch_single<8>(a, ni, st);
      default: return launch_single<4>(a, ni, st);
    }
  }
  const int64_t tiles = (a.rows + kRowsTile - 1) / kRowsTile;
  float2* partial = reinterpret_cast<float2*>(ws);
  float2* mn_scale = partial + tiles * a.C;
  hipLaunchKernelGGL(rows_minmax_vec_kernel, dim3(slices, (unsigned)tiles), dim3(kRowsThreads), 0,
                     st, a, partial);
  if (tiles <= 64) {
    hipLaunchKernelGGL(rows_finalize_quantize_vec_kernel<64>, dim3(slices, (unsigned)tiles),
                       dim3(kRowsThreads), 0, st, a, partial, (int)tiles);
    return hipGetLastError();
  }
  if (tiles <= 128 && a.C <= kFused128MaxC) {
    hipLaunchKernelGGL(rows_finalize_quantize_vec_kernel<128>, dim3(slices, (unsigned)tiles),
                       dim3(kRowsThreads), 0, st, a, partial, (int)tiles);
    return hipGetLastError();
  }
  hipLaunchKernelGGL(rows_finalize_vec_kernel, dim3((unsigned)((a.C + 63) / 64)),
                     dim3(kRowsThreads), 0, st, partial, (int)tiles, a.C, a.scale, a.zp, mn_scale);
  hipLaunchKernelGGL(rows_quantize_vec_kernel, dim3(slices, (unsigned)tiles), dim3(kRowsThreads),
                     0, st, a, mn_scale);
  return hipGetLastError();
}

size_t rows_workspace_bytes(int64_t rows, int C) {
  const int64_t tiles = (rows + kRowsTile - 1) / kRowsTile;
  return (size_t)(tiles * C + C) * sizeof(float2);
}

hipError_t launch_quantize_rows(const float* kv, int64_t rows, int C, int64_t stride,
                                uint8_t* q, int64_t q_stride, bool packed, float* scale_out,
                                float* zp_out, void* ws, hipStream_t st) {
  // 16-byte path when every row is 16-byte aligned and C is a multiple of 4.
  if (C % 4 == 0 && stride % 4 == 0 && (reinterpret_cast<uintptr_t>(kv) & 15) == 0) {
    RowsVecArgs va;
    va.kv = kv;
    va.rows = rows;
    va.stride = stride;
    va.C = C;
    va.q = q;
    va.q_stride = q_stride;
    va.packed = packed ? 1 : 0;
    const uintptr_t wmask = packed ? 1 : 3;
    va.q_word = ((reinterpret_cast<uintptr_t>(q) | (uintptr_t)q_stride) & wmask) == 0;
    va.scale = scale_out;
    va.zp = zp_out;
    return launch_quantize_rows_vec(va, ws, st);
  }
  const int64_t tiles = (rows + kRowsTile - 1) / kRowsTile;
  float2* partial = reinterpret_cast<float2*>(ws);
  float2* mn_scale = partial + tiles * C;
  dim3 g1((C + 63) / 64, (unsigned)tiles);
  hipLaunchKernelGGL(rows_minmax_kernel, g1, dim3(kRowsThreads), 0, st, kv, rows, C, stride,
                     partial);
  hipLaunchKernelGGL(rows_finalize_kernel, dim3((C + 255) / 256), dim3(256), 0, st, partial,
                     (int)tiles, C, scale_out, zp_out, mn_scale);
  if (packed) {
    const int nbytes = (C + 1) / 2;
    dim3 g3((nbytes + 63) / 64, (unsigned)tiles);
    hipLaunchKernelGGL(rows_quantize_kernel<true>, g3, dim3(kRowsThreads), 0, st, kv, rows, C,
                       stride, mn_scale, q, q_stride);
  } else {
    dim3 g3((C + 63) / 64, (unsigned)tiles);
    hipLaunchKernelGGL(rows_quantize_kernel<false>, g3, dim3(kRowsThreads), 0, st, kv, rows, C,
                       stride, mn_scale, q, q_stride);
  }
  return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Grouped, paged, packed quantizer.
// ---------------------------------------------------------------------------

constexpr int kQThreads = 256;

// Thread t of a grouped-quantizer workgroup owns channels 4*(t % VPR) .. +3
// of the group rows t / VPR + i * RPI, i < NI, one 16-byte load per owned row.
template <int D, int GROUP>
struct QGeo {
  static constexpr int VPR = D / 4;              // threads per row (16 B each)
  static constexpr int RPI = kQThreads / VPR;    // rows covered per sweep
  static constexpr int NI = GROUP / RPI;         // rows per thread
  static constexpr int RB = D / 2;               // packed bytes per row
  static constexpr int NWAVE = kQThreads / 64;
  static_assert(VPR <= 64 && GROUP % RPI == 0, "layout");
};

// Quantizes the rows [r0, r0 + nrows) of one (sequence b, kv-head h) whose
// values the calling threads hold in x (QGeo layout; rows past nrows hold
// copies of valid rows): per-channel min/max (wave64 butterfly, then LDS
// across the waves), scale and zero-point of group g, bins from the channel
// reciprocal (quant_bin_rc), nibble pairs staged in LDS, and whole 16-byte
// pieces of packed rows stored to their pages through the page table.
template <int D, int GROUP>
__device__ __forceinline__ void quantize_group(const QuantPagedArgs& a, int b, int h, int g,
                                               int r0, int nrows, const float4* x) {
  using G = QGeo<D, GROUP>;
  constexpr int VPR = G::VPR, RPI = G::RPI, NI = G::NI, RB = G::RB, NWAVE = G::NWAVE;
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int cq = tid % VPR, rsub = tid / VPR;

  float mn[4], mx[4];
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    mn[k] = INFINITY;
    mx[k] = -INFINITY;
  }
#pragma unroll
  for (int i = 0; i < NI; ++i) {
    mn[0] = fminf(mn[0], x[i].x); mx[0] = fmaxf(mx[0], x[i].x);
    mn[1] = fminf(mn[1], x[i].y); mx[1] = fmaxf(mx[1], x[i].y);
    mn[2] = fminf(mn[2], x[i].z); mx[2] = fmaxf(mx[2], x[i].z);
    mn[3] = fminf(mn[3], x[i].w); mx[3] = fmaxf(mx[3], x[i].w);
  }
  // Lanes of one wave that own the same channels differ in the bits >= VPR.
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    mn[k] = allreduce_min_f<VPR, 64>(mn[k]);
    mx[k] = allreduce_max_f<VPR, 64>(mx[k]);
  }
  __shared__ float4 s_mn[NWAVE][VPR], s_mx[NWAVE][VPR];
  if (lane < VPR) {
    s_mn[wv][lane] = make_float4(mn[0], mn[1], mn[2], mn[3]);
    s_mx[wv][lane] = make_float4(mx[0], mx[1], mx[2], mx[3]);
  }
  __syncthreads();
#pragma unroll
  for (int w = 0; w < NWAVE; ++w) {
    const float4 pm = s_mn[w][cq], px = s_mx[w][cq];
    mn[0] = fminf(mn[0], pm.x); mx[0] = fmaxf(mx[0], px.x);
    mn[1] = fminf(mn[1], pm.y); mx[1] = fmaxf(mx[1], px.y);
    mn[2] = fminf(mn[2], pm.z); mx[2] = fmaxf(mx[2], px.z);
    mn[3] = fminf(mn[3], pm.w); mx[3] = fmaxf(mx[3], px.w);
  }
  float sc[4], zp[4];
#pragma unroll
  for (int k = 0; k < 4; ++k) scale_zp(mn[k], mx[k], &sc[k], &zp[k]);
  if (rsub == 0) {
    const int64_t so = (int64_t)b * a.s_b + (int64_t)h * a.s_h + (int64_t)g * a.s_g + 4 * cq;
    *reinterpret_cast<float4*>(a.scale + so) = make_float4(sc[0], sc[1], sc[2], sc[3]);
    *reinterpret_cast<float4*>(a.zp + so) = make_float4(zp[0], zp[1], zp[2], zp[3]);
  }

  // Quantize from registers; two bytes (channels 4cq..4cq+3) per owned row.
  __shared__ uint16_t s_out[GROUP * RB / 2];
  float rc[4];
#pragma unroll
  for (int k = 0; k < 4; ++k) rc[k] = 1.0f / sc[k];
#pragma unroll
  for (int i = 0; i < NI; ++i) {
    const int r = rsub + i * RPI;
    if (r < nrows) {
      const float n0 = quant_bin_rc(x[i].x, mn[0], sc[0], rc[0]);
      const float n1 = quant_bin_rc(x[i].y, mn[1], sc[1], rc[1]);
      const float n2 = quant_bin_rc(x[i].z, mn[2], sc[2], rc[2]);
      const float n3 = quant_bin_rc(x[i].w, mn[3], sc[3], rc[3]);
      // n0 | n1 << 4 | n2 << 8 | n3 << 12 in exact float arithmetic (< 2^16).
      const float pk = __builtin_fmaf(
          n3, 4096.0f, __builtin_fmaf(n2, 256.0f, __builtin_fmaf(n1, 16.0f, n0)));
      s_out[r * (RB / 2) + cq] = (uint16_t)(unsigned)pk;
    }
  }
  __syncthreads();

  // Whole 16-byte pieces of packed rows to their pages.
  constexpr int PPR = RB / 16;            // 16-byte pieces per packed row
  constexpr int NPIECE = GROUP * PPR;
  for (int pc = tid; pc < NPIECE; pc += kQThreads) {
    const int r = pc / PPR, part = pc % PPR;
    if (r >= nrows) continue;
    const int tok = r0 + r;
    const int lp = tok / a.page_rows, row = tok % a.page_rows;
    const int64_t phys =
        (int64_t)min(max(a.page_table[(int64_t)b * a.pt_b + lp], 0), a.num_pages - 1);
    uint8_t* dst = a.k_pages + phys * a.kp_page + (int64_t)h * a.kp_head + (int64_t)row * a.kp_row +
                   part * 16;
    // Non-temporal. Measured against default stores on MI355X (same box, per
    // call, D = 128): B8 H32 T512 6 % faster, T8192 1 %, T32768 5 %, ragged
    // B32 1 %, B64 H32 T4096 8 %; only B8 H32 T2048 is 3 % slower.
    st16_stream(dst, *reinterpret_cast<const U32x4*>(reinterpret_cast<const uint8_t*>(s_out) +
                                                     r * RB + part * 16));
  }
}

// Scale groups per XCD run: the groups of one (sequence, kv-head) are
// consecutive work items, so a run of 16 keeps up to 16 x 64 KiB (D = 128) of
// contiguous key rows on one XCD. Measured on MI355X against the plain
// (group, head, sequence) grid: anchor keys 56.8 -> 55.8 us, Llama-sized keys
// 934 -> 895 us, bit-identical output.
constexpr unsigned kQRun = 16;

// One workgroup quantizes the rows [g*GROUP, min((g+1)*GROUP, T_b)) of one
// (sequence b, kv-head h) of the key tensor. One-dimensional grid over the
// work items g + ngroups * (h + heads * b), dealt to the XCDs in runs.
template <int D, int GROUP>
__global__ __launch_bounds__(kQThreads) void quantize_paged_kernel(QuantPagedArgs a, int ngroups,
                                                                   int heads) {
  using G = QGeo<D, GROUP>;
  const unsigned wi = xcd_run_item(blockIdx.x, gridDim.x, kQRun);
  const int g = (int)(wi % (unsigned)ngroups);
  const int h = (int)(wi / (unsigned)ngroups % (unsigned)heads);
  const int b = (int)(wi / ((unsigned)ngroups * (unsigned)heads));
  const int T = min(a.seq_lens[b], a.max_tokens);
  const int r0 = g * GROUP;
  if (r0 >= T) return;
  const int nrows = min(GROUP, T - r0);
  const int cq = threadIdx.x % G::VPR, rsub = threadIdx.x / G::VPR;

  const float* src = a.k + (int64_t)b * a.k_b + (int64_t)h * a.k_h + (int64_t)r0 * a.k_t + 4 * cq;
  // Rows past the valid count load the last valid row again (same lines, no
  // extra HBM traffic): every register holds a valid value, and duplicates
  // change neither the minimum nor the maximum.
  float4 x[G::NI];
#pragma unroll
  for (int i = 0; i < G::NI; ++i) {
    const int r = min(rsub + i * G::RPI, nrows - 1);
    x[i] = ld16f_stream(src + (int64_t)r * a.k_t);
  }
  quantize_group<D, GROUP>(a, b, h, g, r0, nrows, x);
}

// Decode-time append: one workgroup per (kv-head, sequence) writes the new
// token at position t = seq_lens[b] -- its value row into the value page and
// its key row into the staging rows of the open scale group -- and
// re-quantizes that group over its t % GROUP + 1 valid rows, which is the
// grouped quantizer applied to the whole sequence (a partial group is
// quantized over its valid rows). The new row is taken from k_new, the older
// rows from the staging buffer, so nothing written here is read back.
template <int D, int GROUP>
__global__ __launch_bounds__(kQThreads) void append_paged_kernel(AppendArgs a) {
  using G = QGeo<D, GROUP>;
  const int h = blockIdx.x, b = blockIdx.y;
  const int t = a.q.seq_lens[b];
  const bool fits = t >= 0 && t < a.capacity;
  // The serving step's length advance: one workgroup per sequence writes the
  // length after this append to a separate array (no workgroup of this
  // kernel reads it, so the other heads of the sequence still read t).
  if (a.lens_next && h == 0 && threadIdx.x == 0) a.lens_next[b] = fits ? t + 1 : t;
  if (!fits) return;
  const int g = t / GROUP, rnew = t % GROUP;
  const int tid = threadIdx.x;
  const int cq = tid % G::VPR, rsub = tid / G::VPR;

  const float* knew = a.k_new + (int64_t)b * a.kn_b + (int64_t)h * a.kn_h;
  float* stage = a.stage + (int64_t)b * a.st_b + (int64_t)h * a.st_h;
  if (tid < G::VPR)
    *reinterpret_cast<float4*>(stage + (int64_t)rnew * a.st_r + 4 * tid) =
        *reinterpret_cast<const float4*>(knew + 4 * tid);
  {
    const int lp = t / a.q.page_rows, row = t % a.q.page_rows;
    const int64_t phys =
        (int64_t)min(max(a.q.page_table[(int64_t)b * a.q.pt_b + lp], 0), a.q.num_pages - 1);
    const uint8_t* vsrc = a.v_new + (int64_t)b * a.vn_b + (int64_t)h * a.vn_h;
    uint8_t* vdst = a.v_pages + phys * a.vp_page + (int64_t)h * a.vp_head + (int64_t)row * a.vp_row;
    for (int o = 16 * tid; o < a.v_row_bytes; o += 16 * kQThreads) st16(vdst + o, ld16(vsrc + o));
  }

  float4 x[G::NI];
#pragma unroll
  for (int i = 0; i < G::NI; ++i) {
    const int r = min(rsub + i * G::RPI, rnew);
    const float* src = (r == rnew) ? knew : stage + (int64_t)r * a.st_r;
    x[i] = *reinterpret_cast<const float4*>(src + 4 * cq);
  }
  quantize_group<D, GROUP>(a.q, b, h, g, g * GROUP, rnew + 1, x);
}

hipError_t launch_quantize_paged(const QuantPagedArgs& a, int D, int group, int batch, int heads,
                                 int max_tokens, hipStream_t st) {
  const int ngroups = (max_tokens + group - 1) / group;
  if (ngroups == 0 || batch == 0 || heads == 0) return hipSuccess;
  const int64_t items = (int64_t)ngroups * heads * batch;
  if (items > INT32_MAX) return hipErrorInvalidValue;
  dim3 grid((unsigned)items);
#define FDI4_QP(DD, GG)                                                             \
  if (D == DD && group == GG) {                                                     \
    hipLaunchKernelGGL((quantize_paged_kernel<DD, GG>), grid, dim3(kQThreads), 0, st, a, \
                       ngroups, heads);                                             \
    return hipGetLastError();                                                       \
  }
  FDI4_QP(64, 64) FDI4_QP(64, 128) FDI4_QP(64, 256)
  FDI4_QP(128, 64) FDI4_QP(128, 128) FDI4_QP(128, 256)
  FDI4_QP(256, 64) FDI4_QP(256, 128) FDI4_QP(256, 256)
#undef FDI4_QP
  return hipErrorInvalidValue;
}

hipError_t launch_append_paged(const AppendArgs& a, int D, int group, int batch, int heads,
                               hipStream_t st) {
  if (batch == 0 || heads == 0) return hipSuccess;
  dim3 grid(heads, batch);
#define FDI4_AP(DD, GG)                                                                  \
  if (D == DD && group == GG) {                                                          \
    hipLaunchKernelGGL((append_paged_kernel<DD, GG>), grid, dim3(kQThreads), 0, st, a);   \
    return hipGetLastError();                                                            \
  }
  FDI4_AP(64, 64) FDI4_AP(64, 128) FDI4_AP(64, 256)
  FDI4_AP(128, 64) FDI4_AP(128, 128) FDI4_AP(128, 256)
  FDI4_AP(256, 64) FDI4_AP(256, 128) FDI4_AP(256, 256)
#undef FDI4_AP
  return hipErrorInvalidValue;
}

// ---------------------------------------------------------------------------
// Device nibble packing: out[r, j] = q[r, 2j] | q[r, 2j+1] << 4 for
// j < ceil(C/2); bytes ceil(C/2) .. out_cols-1 are zero (row padding).
// ---------------------------------------------------------------------------

__global__ __launch_bounds__(256) void pack_kernel(const uint8_t* __restrict__ q, int64_t rows,
                                                   int C, int64_t q_stride,
                                                   uint8_t* __restrict__ out, int64_t o_stride,
                                                   int out_cols) {
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int64_t total = rows * out_cols;
  if (idx >= total) return;
  const int64_t r = idx / out_cols;
  const int j = (int)(idx % out_cols);
  const int c0 = 2 * j, c1 = 2 * j + 1;
  unsigned v = 0;
  if (c0 < C) v = q[r * q_stride + c0] & 0xF;
  if (c1 < C) v |= (q[r * q_stride + c1] & 0xF) << 4;
  out[r * o_stride + j] = (uint8_t)v;
}

hipError_t launch_pack(const uint8_t* q, int64_t rows, int C, int64_t q_stride, uint8_t* out,
                       int64_t o_stride, int out_cols, hipStream_t st) {
  const int64_t total = rows * out_cols;
  if (total == 0) return hipSuccess;
  const int64_t blocks = (total + 255) / 256;
  hipLaunchKernelGGL(pack_kernel, dim3((unsigned)blocks), dim3(256), 0, st, q, rows, C, q_stride,
                     out, o_stride, out_cols);
  return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Dequantization of stored INT4 values (reference dequantize_int4_ref,
// src/quantize_int4_ref.py:87-136): out[r, c] = q*s - zp*s with
// s = scale[r*s_rs + c*s_cs], zp likewise -- two float32 products, each
// rounded, then a rounded subtraction, as NumPy evaluates the formula. q is
// one value per byte (its full byte value, as the reference's astype) or two
// nibbles per byte (packed, channel c in the low nibble of byte c/2 when c is
// even, the high nibble when odd). One thread per output element.
// ---------------------------------------------------------------------------

__global__ __launch_bounds__(256) void dequant_kernel(const uint8_t* __restrict__ q, int64_t rows,
                                                      int C, int64_t q_stride, int packed,
                                                      const float* __restrict__ scale,
                                                      const float* __restrict__ zp, int64_t s_rs,
                                                      int64_t s_cs, float* __restrict__ out,
                                                      int64_t o_stride) {
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (idx >= rows * C) return;
  const int64_t r = idx / C;
  const int c = (int)(idx - r * C);
  unsigned v;
  if (packed) {
    v = (q[r * q_stride + (c >> 1)] >> (4 * (c & 1))) & 15u;
  } else {
    v = q[r * q_stride + c];
  }
  const int64_t si = r * s_rs + (int64_t)c * s_cs;
  const float sc = scale[si];
  out[r * o_stride + c] = __fsub_rn(__fmul_rn((float)v, sc), __fmul_rn(zp[si], sc));
}

hipError_t launch_dequantize(const uint8_t* q, int64_t rows, int C, int64_t q_stride, int packed,
                             const float* scale, const float* zp, int64_t s_rs, int64_t s_cs,
                             float* out, int64_t o_stride, hipStream_t st) {
  const int64_t total = rows * C;
  if (total == 0) return hipSuccess;
  const int64_t blocks = (total + 255) / 256;
  if (blocks > INT32_MAX) return hipErrorInvalidValue;
  hipLaunchKernelGGL(dequant_kernel, dim3((unsigned)blocks), dim3(256), 0, st, q, rows, C,
                     q_stride, packed, scale, zp, s_rs, s_cs, out, o_stride);
  return hipGetLastError();
}

}  // namespace fdi4
