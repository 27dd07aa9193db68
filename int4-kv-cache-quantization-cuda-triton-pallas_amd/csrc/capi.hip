// extern "C" entry points of libfdi4 (declared in include/fdi4.h).
//
// Host-side only: argument validation (every size and alignment the kernels
// assume is checked here, so a malformed call becomes hipErrorInvalidValue
// instead of an out-of-bounds device access), translation of the public
// layout into kernel argument blocks, split-count selection and workspace
// carving.

#include <limits.h>
#include <stdlib.h>

#include <algorithm>
#include <atomic>
#include <map>
#include <mutex>

#include "../../include/fdi4.h"
#include "fdi4_internal.hpp"

namespace {

using fdi4::DecodeArgs;
using fdi4::QuantPagedArgs;

// Decode launch shape. A workgroup has 4 or 8 wave64s; the split count is the
// smallest that gives about kTargetWaves resident waves (8 per CU on 256 CUs,
// the occupancy the decode kernel's ~200 VGPRs allow), so that with enough
// (sequence, head) streams no split -- and no merge kernel -- is needed.
// FDI4_TUNE_DECODE_WAVES and FDI4_TUNE_DECODE_TARGET_WAVES override the choice.
constexpr int kTargetWaves = 2048;
constexpr int kMinChunksPerWave = 4;
constexpr int kMaxGroupedSplits = 8;
constexpr size_t kAlign = 256;

inline size_t align_up(size_t x) { return (x + kAlign - 1) / kAlign * kAlign; }
inline bool aligned(const void* p, size_t a) { return ((uintptr_t)p % a) == 0; }
inline int ceil_div(int64_t a, int64_t b) { return (int)((a + b - 1) / b); }

bool valid_head_dim(int d) { return d == 64 || d == 128 || d == 256; }

int padded_head_dim(int d) { return d <= 64 ? 64 : (d <= 128 ? 128 : 256); }

int chunks_per_seq(const fdi4_paged_cache* c) {
  return c->max_pages * ceil_div(c->page_rows, 16);
}

// Launch-shape overrides set through fdi4_set_tuning (0 = automatic). Atomic
// so that a setting made on one thread is seen, whole, by launches on another.
std::atomic<int> g_tuning[FDI4_TUNE_COUNT];

bool tuning_value_ok(int knob, int v) {
  if (v == 0) return true;
  switch (knob) {
    case FDI4_TUNE_DECODE_VECTOR_ONLY: return v == 1;
    case FDI4_TUNE_DECODE_WAVES: return v == 4 || v == 8;
    case FDI4_TUNE_DECODE_HEADS_PER_WG: return v == 1 || v == 2 || v == 4 || v == 8;
    case FDI4_TUNE_DECODE_TARGET_WAVES: return v >= 1 && v <= (1 << 20);
    case FDI4_TUNE_FAKE_QUANT_SPLIT: return v >= 1 && v <= 512;
    default: return false;
  }
}

// Eight waves as soon as each gets kMinChunksPerWave chunks: more waves per
// workgroup merge in LDS, where more splits need the merge kernel (at B8 H32
// T512, 8 waves and one split take 16.5 us against 19.2 us for 4 waves, two
// splits and the merge).
int pick_waves(int chunks) {
  const int w = g_tuning[FDI4_TUNE_DECODE_WAVES].load(std::memory_order_relaxed);
  if (w == 4 || w == 8) return w;
  return chunks >= 8 * kMinChunksPerWave ? 8 : 4;
}

// Query heads one decode workgroup serves (heads of one kv-head, so their
// keys and values are read once for all of them): the largest of 8, 4, 2 that
// divides Hq/Hkv within what registers and LDS allow (8 at D=64, 4 at D=128
// and 256); 1 runs the per-head kernel. FDI4_TUNE_DECODE_HEADS_PER_WG caps the
// choice (1 disables grouping).
int heads_per_wg_cap() {
  const int c = g_tuning[FDI4_TUNE_DECODE_HEADS_PER_WG].load(std::memory_order_relaxed);
  return c > 0 ? c : 8;
}

int pick_heads_per_wg(int d, int hq_per_kv) {
  const int cap = std::min(heads_per_wg_cap(), d == 64 ? 8 : 4);
  for (int hg : {8, 4, 2})
    if (hg <= cap && hq_per_kv % hg == 0) return hg;
  return 1;
}

// Kernel family: with two or more q-heads per kv-head at D = 64 or 128 the
// int8 matrix-core kernel (2, 4 or 8 heads per workgroup, 8 only at D=64;
// B8 Hkv8 Hq32 T8192: 61 us against 75 us for the vector grouped kernel);
// with one head per kv-head the vector per-head kernel, which is faster there
// (anchor 51.9 against 54.2 us). FDI4_TUNE_DECODE_VECTOR_ONLY selects the
// vector kernels throughout (A/B measurement).
bool use_mfma(int d) {
  const bool off = g_tuning[FDI4_TUNE_DECODE_VECTOR_ONLY].load(std::memory_order_relaxed) == 1;
  return !off && (d == 64 || d == 128);
}

// Up to eight heads per workgroup (at D=128: 248 VGPRs with float32 values,
// 244 with float16, no spills).
int pick_heads_per_wg_mfma(int d, int v_dtype, int hq_per_kv) {
  (void)d;
  (void)v_dtype;
  const int cap = heads_per_wg_cap();
  for (int hg : {8, 4, 2})
    if (hg <= cap && hq_per_kv % hg == 0) return hg;
  return 1;
}

struct DecodePlan {
  int mfma;
  int heads_per_wg;
  int waves;
  int splits;
};

// The per-head decode with float32 values at D = 128 (512-byte value rows)
// runs four waves, one per SIMD, and aims at one wave per SIMD
// (kTargetWaves / 2) while the streams at four waves stay within kTargetWaves:
// one wave streams a 16-row chunk of 8 KB of values with enough loads in
// flight, and no SIMD is shared by an older and a younger wave that finish
// apart. In-process A/B against eight waves and kTargetWaves, one box: B8 H32
// T512 16.15 -> 15.61 us, T2048 48.8 -> 47.8, T8192 182.0 -> 181.4, B16 H32
// T2048 94.7 -> 93.4, B1 H8 T1024 13.5 -> 10.7 (four splits against two);
// slower with 256-byte rows (D=64: 27.8 -> 30.0 us; float16 values at D=128:
// 31.3 -> 35.7) and with more streams (B32 H32, ragged lengths to 8192:
// 321.5 -> 346.2 us; B64 H32 T4096: 713.2 -> 716.5). (At D = 256 the
// four-wave kernel needs more than 256 registers, one wave per SIMD.)
bool one_wave_per_simd(int d, int v_dtype, int64_t streams) {
  return d == 128 && v_dtype == FDI4_V_F32 && streams * 4 <= kTargetWaves;
}

// Launch shape of a decode: heads per workgroup, waves per workgroup (the
// grouped kernel at D=256 has registers for four), and the split count that
// gives about kTargetWaves waves over the (sequence, head group) streams. The
// fused serving step takes the same shape (and so gives the same bits as the
// append and the decode); with four decode waves its kernel adds four helper
// waves that re-quantize the open group meanwhile.
DecodePlan plan_decode(int batch, int hq, int hq_per_kv, int d, int v_dtype, int chunks) {
  DecodePlan p;
  p.mfma = use_mfma(d) ? 1 : 0;
  p.heads_per_wg = p.mfma ? pick_heads_per_wg_mfma(d, v_dtype, hq_per_kv)
                          : pick_heads_per_wg(d, hq_per_kv);
  if (p.heads_per_wg == 1) p.mfma = 0;
  const int64_t streams = (int64_t)batch * (hq / p.heads_per_wg);
  const bool per_simd = !p.mfma && p.heads_per_wg == 1 && one_wave_per_simd(d, v_dtype, streams);
  const int forced = g_tuning[FDI4_TUNE_DECODE_WAVES].load(std::memory_order_relaxed);
  if (!p.mfma && p.heads_per_wg > 1 && d == 256) p.waves = 4;
  else if (per_simd && forced == 0) p.waves = 4;
  else p.waves = pick_waves(chunks);
  if (chunks <= 0) {
    p.splits = 1;
    return p;
  }
  const int tw = g_tuning[FDI4_TUNE_DECODE_TARGET_WAVES].load(std::memory_order_relaxed);
  const int64_t target =
      tw > 0 ? tw : (per_simd && p.waves == 4 ? kTargetWaves / 2 : kTargetWaves);
  const int64_t per_split = (int64_t)batch * (hq / p.heads_per_wg) * p.waves;
  const int s = (int)((target + per_split - 1) / per_split);
  int smax = std::max(1, chunks / (p.waves * kMinChunksPerWave));
  // Grouped heads (several q-heads per workgroup, more work per chunk) split
  // down to one chunk per wave, up to eight splits (one merge round): in
  // process A/B against four chunks per wave, one box: B1 Hkv8 Hq32 T1024
  // 15.3 -> 12.0 us (8 splits against 2), B2 T2048 16.1 -> 13.8 (8 against
  // 4), D64 B2 Hq64 T2048 14.9 -> 13.4, the shared-stream call of 8 x 256
  // rows 19.1 -> 17.0; 16 and 32 splits were slower (B1 T4096 16.2 -> 22.3).
  if (p.heads_per_wg > 1) smax = std::max(smax, std::min(chunks / p.waves, kMaxGroupedSplits));
  p.splits = std::max(1, std::min(s, smax));
  return p;
}

size_t decode_ws_bytes(int batch, int hq, int d, int splits) {
  if (splits <= 0) return 0;
  const size_t n = (size_t)batch * hq * splits;
  return align_up(n * d * sizeof(float)) + align_up(n * 2 * sizeof(double));
}

int check_cache(const fdi4_paged_cache* c, bool need_values) {
  if (!c || !c->k_pages || !c->k_scale || !c->k_zp) return hipErrorInvalidValue;
  if (!valid_head_dim(c->head_dim)) return hipErrorInvalidValue;
  if (c->num_kv_heads < 1 || c->page_rows < 1 || c->pages_per_group < 1 || c->max_pages < 0 ||
      c->num_pages < 1)
    return hipErrorInvalidValue;
  if (c->s_page_stride != 0 && c->pages_per_group != 1) return hipErrorInvalidValue;
  // Token positions within a sequence are 32-bit in the kernels.
  if ((int64_t)c->max_pages * c->page_rows > INT32_MAX) return hipErrorInvalidValue;
  const int kbl = c->head_dim == 64 ? 8 : 16;  // bytes a lane loads from a key row
  if (!aligned(c->k_pages, kbl) || c->k_page_stride % kbl || c->k_head_stride % kbl ||
      c->k_row_stride % kbl || c->k_row_stride < c->head_dim / 2)
    return hipErrorInvalidValue;
  // The kernels address the rows of a 16-row chunk with 32-bit byte offsets.
  if ((int64_t)c->k_row_stride * 16 + c->head_dim > INT32_MAX) return hipErrorInvalidValue;
  if (!aligned(c->k_scale, 16) || !aligned(c->k_zp, 16) || c->s_batch_stride % 4 ||
      c->s_head_stride % 4 || c->s_group_stride % 4 || c->s_page_stride % 4)
    return hipErrorInvalidValue;
  if (need_values) {
    if (!c->v_pages ||
        (c->v_dtype != FDI4_V_F32 && c->v_dtype != FDI4_V_F16 && c->v_dtype != FDI4_V_BF16))
      return hipErrorInvalidValue;
    const int veb = c->v_dtype == FDI4_V_F32 ? 4 : 2;
    if (!aligned(c->v_pages, 16) || (c->v_page_stride * veb) % 16 ||
        (c->v_head_stride * veb) % 16 || (c->v_row_stride * veb) % 16 ||
        c->v_row_stride < c->head_dim)
      return hipErrorInvalidValue;
    if ((c->v_row_stride * veb) * 16 + (int64_t)c->head_dim * veb > INT32_MAX)
      return hipErrorInvalidValue;
  }
  return hipSuccess;
}

// Stream-ordered temporaries of the two entry points that keep the
// reference's argument lists (no workspace argument) come from a memory pool
// this library creates on each device at first use and keeps until the
// process ends; its release threshold keeps freed blocks for the next call.
// The process's default pool is left as the caller configured it.
hipError_t temp_alloc(void** ptr, size_t bytes, hipStream_t stream) {
  int dev = 0;
  hipError_t e = stream ? hipStreamGetDevice(stream, &dev) : hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  static std::mutex mu;
  static std::map<int, hipMemPool_t> pools;
  hipMemPool_t pool = nullptr;
  {
    std::lock_guard<std::mutex> lock(mu);
    auto it = pools.find(dev);
    if (it == pools.end()) {
      hipMemPoolProps props = {};
      props.allocType = hipMemAllocationTypePinned;
      props.handleTypes = hipMemHandleTypeNone;
      props.location.type = hipMemLocationTypeDevice;
      props.location.id = dev;
      if ((e = hipMemPoolCreate(&pool, &props)) != hipSuccess) return e;
      uint64_t keep = UINT64_MAX;
      (void)hipMemPoolSetAttribute(pool, hipMemPoolAttrReleaseThreshold, &keep);
      pools[dev] = pool;
    } else {
      pool = it->second;
    }
  }
  return hipMallocFromPoolAsync(ptr, bytes, pool, stream);
}

}  // namespace

int fdi4::tuning(int knob) {
  return (knob >= 0 && knob < FDI4_TUNE_COUNT) ? g_tuning[knob].load(std::memory_order_relaxed)
                                               : 0;
}

extern "C" {

int fdi4_set_tuning(int knob, int value) {
  if (knob < 0 || knob >= FDI4_TUNE_COUNT || !tuning_value_ok(knob, value))
    return hipErrorInvalidValue;
  g_tuning[knob].store(value, std::memory_order_relaxed);
  return hipSuccess;
}

int fdi4_get_tuning(int knob) {
  if (knob < 0 || knob >= FDI4_TUNE_COUNT) return -1;
  return g_tuning[knob].load(std::memory_order_relaxed);
}

int fdi4_abi_version(void) { return FDI4_ABI_VERSION; }

const char* fdi4_error_string(int status) { return hipGetErrorString((hipError_t)status); }

size_t fdi4_quantize_rows_workspace_bytes(int64_t num_rows, int num_channels) {
  if (num_rows <= 0 || num_channels <= 0) return 0;
  return fdi4::rows_workspace_bytes(num_rows, num_channels);
}

int fdi4_quantize_rows(const float* kv, int64_t num_rows, int num_channels, int64_t kv_row_stride,
                       uint8_t* q_out, int64_t q_row_stride, int packed, float* scale_out,
                       float* zp_out, void* workspace, size_t workspace_bytes,
                       hipStream_t stream) {
  if (!kv || !q_out || !scale_out || !zp_out) return hipErrorInvalidValue;
  if (num_rows <= 0 || num_channels <= 0) return hipErrorInvalidValue;
  if ((num_rows + 255) / 256 > 65535) return hipErrorInvalidValue;  // grid.y of the row tiles
  const int qcols = packed ? (num_channels + 1) / 2 : num_channels;
  if (kv_row_stride < num_channels || q_row_stride < qcols) return hipErrorInvalidValue;
  if (!workspace || !aligned(workspace, 8) ||
      workspace_bytes < fdi4::rows_workspace_bytes(num_rows, num_channels))
    return hipErrorInvalidValue;
  return fdi4::launch_quantize_rows(kv, num_rows, num_channels, kv_row_stride, q_out,
                                    q_row_stride, packed != 0, scale_out, zp_out, workspace,
                                    stream);
}

int fdi4_quantize_int4(const float* kv, int num_rows, int num_channels, uint8_t* q_out,
                       float* scale_out, float* zp_out, hipStream_t stream) {
  if (num_rows <= 0 || num_channels <= 0 || !kv || !q_out || !scale_out || !zp_out)
    return hipErrorInvalidValue;
  const size_t wsb = fdi4::rows_workspace_bytes(num_rows, num_channels);
  void* ws = nullptr;
  hipError_t e = temp_alloc(&ws, wsb, stream);
  if (e != hipSuccess) return e;
  int rc = fdi4_quantize_rows(kv, num_rows, num_channels, num_channels, q_out, num_channels, 0,
                              scale_out, zp_out, ws, wsb, stream);
  hipError_t f = hipFreeAsync(ws, stream);
  return rc != hipSuccess ? rc : f;
}

}  // extern "C"

namespace {

// Checks shared by the grouped writers (fdi4_quantize_paged, fdi4_append_paged):
// group-indexed scales, pages_per_group consistent with group_rows, lengths
// and page table present, 16-byte stores of packed rows.
int check_grouped_cache(const fdi4_paged_cache* cache, int group_rows, bool need_values) {
  int rc = check_cache(cache, need_values);
  if (rc != hipSuccess) return rc;
  if (!cache->seq_lens || !cache->page_table || cache->num_kv_heads > 65535)
    return hipErrorInvalidValue;
  if (group_rows != 64 && group_rows != 128 && group_rows != 256) return hipErrorInvalidValue;
  if (group_rows % cache->page_rows) return hipErrorInvalidValue;
  if (cache->pages_per_group != group_rows / cache->page_rows || cache->s_page_stride != 0)
    return hipErrorInvalidValue;
  if (cache->k_page_stride % 16 || cache->k_head_stride % 16 || cache->k_row_stride % 16 ||
      !aligned(cache->k_pages, 16))
    return hipErrorInvalidValue;
  return hipSuccess;
}

QuantPagedArgs quant_args(const fdi4_paged_cache* cache) {
  QuantPagedArgs a;
  a.k = nullptr;
  a.k_b = a.k_h = a.k_t = 0;
  a.seq_lens = cache->seq_lens;
  a.page_table = cache->page_table;
  a.pt_b = cache->pt_batch_stride;
  a.k_pages = cache->k_pages;
  a.kp_page = cache->k_page_stride;
  a.kp_head = cache->k_head_stride;
  a.kp_row = cache->k_row_stride;
  a.scale = cache->k_scale;
  a.zp = cache->k_zp;
  a.s_b = cache->s_batch_stride;
  a.s_h = cache->s_head_stride;
  a.s_g = cache->s_group_stride;
  a.page_rows = cache->page_rows;
  a.num_pages = cache->num_pages;
  a.max_tokens = 0;
  return a;
}

}  // namespace

extern "C" {

int fdi4_quantize_paged(const float* k, int batch, int max_tokens, int64_t k_batch_stride,
                        int64_t k_head_stride, int64_t k_row_stride, int group_rows,
                        const fdi4_paged_cache* cache, hipStream_t stream) {
  int rc = check_grouped_cache(cache, group_rows, false);
  if (rc != hipSuccess) return rc;
  if (!k || batch < 0 || max_tokens < 0 || batch > 65535) return hipErrorInvalidValue;
  if ((int64_t)cache->max_pages * cache->page_rows < max_tokens) return hipErrorInvalidValue;
  // 16-byte row loads of the keys.
  if (!aligned(k, 16) || k_batch_stride % 4 || k_head_stride % 4 || k_row_stride % 4 ||
      k_row_stride < cache->head_dim)
    return hipErrorInvalidValue;
  QuantPagedArgs a = quant_args(cache);
  a.k = k;
  a.k_b = k_batch_stride;
  a.k_h = k_head_stride;
  a.k_t = k_row_stride;
  a.max_tokens = max_tokens;
  return fdi4::launch_quantize_paged(a, cache->head_dim, group_rows, batch, cache->num_kv_heads,
                                     max_tokens, stream);
}

}  // extern "C"

namespace {

// The [0, n) int32 ranges at p and q do not overlap.
bool disjoint_lens(const int32_t* p, const int32_t* q, int n) {
  return p + n <= q || q + n <= p;
}

// The checks of fdi4_append_paged, and its kernel argument block.
int make_append_args(const float* k_new, int64_t kn_batch_stride, int64_t kn_head_stride,
                     const void* v_new, int64_t vn_batch_stride, int64_t vn_head_stride,
                     int batch, float* k_stage, int64_t st_batch_stride, int64_t st_head_stride,
                     int64_t st_row_stride, int group_rows, const fdi4_paged_cache* cache,
                     fdi4::AppendArgs* out) {
  int rc = check_grouped_cache(cache, group_rows, true);
  if (rc != hipSuccess) return rc;
  if (!k_new || !v_new || !k_stage || batch < 0 || batch > 65535) return hipErrorInvalidValue;
  const int D = cache->head_dim;
  const int veb = cache->v_dtype == FDI4_V_F32 ? 4 : 2;
  // 16-byte loads and stores of key rows (float4) and value rows.
  if (!aligned(k_new, 16) || kn_batch_stride % 4 || kn_head_stride % 4 || !aligned(k_stage, 16) ||
      st_batch_stride % 4 || st_head_stride % 4 || st_row_stride % 4 || st_row_stride < D ||
      !aligned(v_new, 16) || (vn_batch_stride * veb) % 16 || (vn_head_stride * veb) % 16)
    return hipErrorInvalidValue;
  fdi4::AppendArgs& a = *out;
  a.q = quant_args(cache);
  a.q.k = nullptr;
  a.q.k_b = a.q.k_h = a.q.k_t = 0;
  a.q.max_tokens = cache->max_pages * cache->page_rows;
  a.k_new = k_new;
  a.kn_b = kn_batch_stride;
  a.kn_h = kn_head_stride;
  a.v_new = static_cast<const uint8_t*>(v_new);
  a.vn_b = vn_batch_stride * veb;
  a.vn_h = vn_head_stride * veb;
  a.v_pages = static_cast<uint8_t*>(cache->v_pages);
  a.vp_page = cache->v_page_stride * veb;
  a.vp_head = cache->v_head_stride * veb;
  a.vp_row = cache->v_row_stride * veb;
  a.v_row_bytes = D * veb;
  a.stage = k_stage;
  a.st_b = st_batch_stride;
  a.st_h = st_head_stride;
  a.st_r = st_row_stride;
  a.capacity = cache->max_pages * cache->page_rows;
  a.lens_next = nullptr;
  return hipSuccess;
}

int append_paged_any(const float* k_new, int64_t kn_batch_stride, int64_t kn_head_stride,
                     const void* v_new, int64_t vn_batch_stride, int64_t vn_head_stride,
                     int batch, float* k_stage, int64_t st_batch_stride, int64_t st_head_stride,
                     int64_t st_row_stride, int group_rows, const fdi4_paged_cache* cache,
                     int32_t* lens_next, hipStream_t stream) {
  fdi4::AppendArgs a;
  const int rc = make_append_args(k_new, kn_batch_stride, kn_head_stride, v_new, vn_batch_stride,
                                  vn_head_stride, batch, k_stage, st_batch_stride,
                                  st_head_stride, st_row_stride, group_rows, cache, &a);
  if (rc != hipSuccess) return rc;
  a.lens_next = lens_next;
  return fdi4::launch_append_paged(a, cache->head_dim, group_rows, batch, cache->num_kv_heads,
                                   stream);
}

}  // namespace

extern "C" {

int fdi4_append_paged(const float* k_new, int64_t kn_batch_stride, int64_t kn_head_stride,
                      const void* v_new, int64_t vn_batch_stride, int64_t vn_head_stride,
                      int batch, float* k_stage, int64_t st_batch_stride, int64_t st_head_stride,
                      int64_t st_row_stride, int group_rows, const fdi4_paged_cache* cache,
                      hipStream_t stream) {
  return append_paged_any(k_new, kn_batch_stride, kn_head_stride, v_new, vn_batch_stride,
                          vn_head_stride, batch, k_stage, st_batch_stride, st_head_stride,
                          st_row_stride, group_rows, cache, nullptr, stream);
}

int fdi4_append_paged_advance(const float* k_new, int64_t kn_batch_stride,
                              int64_t kn_head_stride, const void* v_new,
                              int64_t vn_batch_stride, int64_t vn_head_stride, int batch,
                              float* k_stage, int64_t st_batch_stride, int64_t st_head_stride,
                              int64_t st_row_stride, int group_rows,
                              const fdi4_paged_cache* cache, int32_t* lens_next,
                              hipStream_t stream) {
  if (!cache || !cache->seq_lens || !lens_next || !aligned(lens_next, 4) || batch < 0 ||
      !disjoint_lens(lens_next, cache->seq_lens, batch))
    return hipErrorInvalidValue;
  return append_paged_any(k_new, kn_batch_stride, kn_head_stride, v_new, vn_batch_stride,
                          vn_head_stride, batch, k_stage, st_batch_stride, st_head_stride,
                          st_row_stride, group_rows, cache, lens_next, stream);
}

int fdi4_decode_num_splits(int batch, int num_q_heads, const fdi4_paged_cache* cache) {
  if (!cache || batch <= 0 || num_q_heads <= 0 || cache->page_rows < 1 ||
      cache->num_kv_heads < 1 || num_q_heads % cache->num_kv_heads)
    return 1;
  return plan_decode(batch, num_q_heads, num_q_heads / cache->num_kv_heads, cache->head_dim,
                     cache->v_dtype, chunks_per_seq(cache))
      .splits;
}

size_t fdi4_decode_workspace_bytes(int batch, int num_q_heads, int head_dim, int num_splits) {
  if (batch <= 0 || num_q_heads <= 0 || head_dim <= 0 || num_splits <= 1) return 0;
  return decode_ws_bytes(batch, num_q_heads, head_dim, num_splits);
}

size_t fdi4_decode_partials_bytes(int batch, int num_q_heads, int head_dim, int num_splits) {
  if (batch <= 0 || num_q_heads <= 0 || head_dim <= 0 || num_splits <= 0) return 0;
  return decode_ws_bytes(batch, num_q_heads, head_dim, num_splits);
}

int fdi4_merge_splits(const float* part_acc, const double* part_ml, int batch, int num_q_heads,
                      int head_dim, int num_splits, float* out, int64_t out_batch_stride,
                      int64_t out_head_stride, hipStream_t stream) {
  if (!part_acc || !part_ml || !out || batch <= 0 || num_q_heads <= 0 || num_splits <= 0)
    return hipErrorInvalidValue;
  if (!valid_head_dim(head_dim) || batch > 65535 || num_q_heads > 65535)
    return hipErrorInvalidValue;
  return fdi4::launch_merge(part_acc, part_ml, batch, num_q_heads, head_dim, num_splits, out,
                            FDI4_K_F32, out_batch_stride, out_head_stride, stream);
}

}  // extern "C"

namespace {

// Validate and fill the kernel argument block shared by the decode entry points.
hipError_t launch_decode_any(const DecodeArgs& a, int d, int v_dtype, int batch,
                             hipStream_t stream) {
  if (a.mfma) return fdi4::launch_decode_mfma(a, d, v_dtype, batch, a.heads_per_wg, stream);
  if (a.heads_per_wg > 1)
    return fdi4::launch_decode_gqa(a, d, v_dtype, batch, a.heads_per_wg, stream);
  return fdi4::launch_decode(a, d, v_dtype, batch, stream);
}

bool valid_elem_dtype(int dt) {
  return dt == FDI4_K_F32 || dt == FDI4_K_F16 || dt == FDI4_K_BF16;
}

int make_decode_args(const void* query, int q_dtype, int batch, int num_q_heads,
                     int64_t q_batch_stride, int64_t q_head_stride,
                     const fdi4_paged_cache* cache, int num_splits, DecodeArgs* a) {
  int rc = check_cache(cache, true);
  if (rc != hipSuccess) return rc;
  if (!query || batch <= 0 || num_q_heads <= 0 || !valid_elem_dtype(q_dtype))
    return hipErrorInvalidValue;
  if (batch > 65535 || num_q_heads > 65535) return hipErrorInvalidValue;
  if (num_q_heads % cache->num_kv_heads) return hipErrorInvalidValue;
  if (cache->page_table && cache->pt_batch_stride < 0) return hipErrorInvalidValue;
  const int chunks = chunks_per_seq(cache);
  const DecodePlan plan = plan_decode(batch, num_q_heads, num_q_heads / cache->num_kv_heads,
                                      cache->head_dim, cache->v_dtype, chunks);
  int splits = num_splits > 0 ? num_splits : plan.splits;
  splits = std::max(1, std::min(splits, std::max(chunks, 1)));
  a->q = query;
  a->q_dtype = q_dtype;
  a->q_b = q_batch_stride;
  a->q_h = q_head_stride;
  a->k_pages = cache->k_pages;
  a->k_page = cache->k_page_stride;
  a->k_head = cache->k_head_stride;
  a->k_row = cache->k_row_stride;
  a->v_pages = cache->v_pages;
  a->v_page = cache->v_page_stride;
  a->v_head = cache->v_head_stride;
  a->v_row = cache->v_row_stride;
  a->k_scale = cache->k_scale;
  a->k_zp = cache->k_zp;
  a->s_b = cache->s_batch_stride;
  a->s_h = cache->s_head_stride;
  a->s_g = cache->s_group_stride;
  a->s_p = cache->s_page_stride;
  a->page_table = cache->page_table;
  a->pt_b = cache->pt_batch_stride;
  a->seq_lens = cache->seq_lens;
  a->page_lens = cache->page_lens;
  a->pl_b = cache->pl_batch_stride;
  a->page_rows = cache->page_rows;
  a->pages_per_group = cache->pages_per_group;
  a->max_pages = cache->max_pages;
  a->hq_per_kv = num_q_heads / cache->num_kv_heads;
  a->num_pages = cache->num_pages;
  a->chunks_per_split = std::max(1, ceil_div(chunks, splits));
  a->num_splits = splits;
  a->num_q_heads = num_q_heads;
  a->out = nullptr;
  a->out_dtype = FDI4_K_F32;
  a->o_b = a->o_h = 0;
  a->ws_acc = nullptr;
  a->ws_ml = nullptr;
  a->final_out = 0;
  a->waves = plan.waves;
  a->heads_per_wg = plan.heads_per_wg;
  a->mfma = plan.mfma;
  a->lens_out = nullptr;
  a->step = fdi4::StepAppend{};
  return hipSuccess;
}

int carve_partials(void* workspace, size_t workspace_bytes, int batch, int hq, int d,
                   DecodeArgs* a) {
  const size_t need = decode_ws_bytes(batch, hq, d, a->num_splits);
  if (!workspace || workspace_bytes < need || !aligned(workspace, kAlign))
    return hipErrorInvalidValue;
  const size_t n = (size_t)batch * hq * a->num_splits;
  a->ws_acc = reinterpret_cast<float*>(workspace);
  a->ws_ml = reinterpret_cast<double*>(reinterpret_cast<char*>(workspace) +
                                       align_up(n * d * sizeof(float)));
  return hipSuccess;
}

}  // namespace

namespace {

int decode_paged_any(const void* query, int q_dtype, int batch, int num_q_heads,
                     int64_t q_batch_stride, int64_t q_head_stride,
                     const fdi4_paged_cache* cache, void* out, int out_dtype,
                     int64_t out_batch_stride, int64_t out_head_stride, int num_splits,
                     void* workspace, size_t workspace_bytes, int32_t* lens_out,
                     hipStream_t stream) {
  DecodeArgs a;
  int rc = make_decode_args(query, q_dtype, batch, num_q_heads, q_batch_stride, q_head_stride,
                            cache, num_splits, &a);
  if (rc != hipSuccess) return rc;
  a.lens_out = lens_out;
  if (!out || !valid_elem_dtype(out_dtype)) return hipErrorInvalidValue;
  const int d = cache->head_dim;
  a.out = out;
  a.out_dtype = out_dtype;
  a.o_b = out_batch_stride;
  a.o_h = out_head_stride;
  if (a.num_splits == 1) {
    a.final_out = 1;
    return launch_decode_any(a, d, cache->v_dtype, batch, stream);
  }
  rc = carve_partials(workspace, workspace_bytes, batch, num_q_heads, d, &a);
  if (rc != hipSuccess) return rc;
  hipError_t e = launch_decode_any(a, d, cache->v_dtype, batch, stream);
  if (e != hipSuccess) return e;
  return fdi4::launch_merge(a.ws_acc, a.ws_ml, batch, num_q_heads, d, a.num_splits, out,
                            out_dtype, out_batch_stride, out_head_stride, stream);
}

}  // namespace

extern "C" {

int fdi4_decode_paged(const float* query, int batch, int num_q_heads, int64_t q_batch_stride,
                      int64_t q_head_stride, const fdi4_paged_cache* cache, float* out,
                      int64_t out_batch_stride, int64_t out_head_stride, int num_splits,
                      void* workspace, size_t workspace_bytes, hipStream_t stream) {
  return decode_paged_any(query, FDI4_K_F32, batch, num_q_heads, q_batch_stride, q_head_stride,
                          cache, out, FDI4_K_F32, out_batch_stride, out_head_stride, num_splits,
                          workspace, workspace_bytes, nullptr, stream);
}

int fdi4_decode_paged_ex(const void* query, int query_dtype, int batch, int num_q_heads,
                         int64_t q_batch_stride, int64_t q_head_stride,
                         const fdi4_paged_cache* cache, void* out, int out_dtype,
                         int64_t out_batch_stride, int64_t out_head_stride, int num_splits,
                         void* workspace, size_t workspace_bytes, hipStream_t stream) {
  return decode_paged_any(query, query_dtype, batch, num_q_heads, q_batch_stride, q_head_stride,
                          cache, out, out_dtype, out_batch_stride, out_head_stride, num_splits,
                          workspace, workspace_bytes, nullptr, stream);
}

int fdi4_decode_paged_advance(const void* query, int query_dtype, int batch, int num_q_heads,
                              int64_t q_batch_stride, int64_t q_head_stride,
                              const fdi4_paged_cache* cache, void* out, int out_dtype,
                              int64_t out_batch_stride, int64_t out_head_stride, int num_splits,
                              void* workspace, size_t workspace_bytes, int32_t* lens_out,
                              hipStream_t stream) {
  if (!cache || !cache->seq_lens || !lens_out || !aligned(lens_out, 4) || batch < 0 ||
      !disjoint_lens(lens_out, cache->seq_lens, batch))
    return hipErrorInvalidValue;
  return decode_paged_any(query, query_dtype, batch, num_q_heads, q_batch_stride, q_head_stride,
                          cache, out, out_dtype, out_batch_stride, out_head_stride, num_splits,
                          workspace, workspace_bytes, lens_out, stream);
}

int fdi4_decode_step(const void* query, int query_dtype, int batch, int num_q_heads,
                     int64_t q_batch_stride, int64_t q_head_stride, const float* k_new,
                     int64_t kn_batch_stride, int64_t kn_head_stride, const void* v_new,
                     int64_t vn_batch_stride, int64_t vn_head_stride, float* k_stage,
                     int64_t st_batch_stride, int64_t st_head_stride, int64_t st_row_stride,
                     int group_rows, const fdi4_paged_cache* cache, void* out, int out_dtype,
                     int64_t out_batch_stride, int64_t out_head_stride, int32_t* counters,
                     int32_t* lens_next, void* workspace, size_t workspace_bytes,
                     hipStream_t stream) {
  fdi4::AppendArgs ap;
  int rc = make_append_args(k_new, kn_batch_stride, kn_head_stride, v_new, vn_batch_stride,
                            vn_head_stride, batch, k_stage, st_batch_stride, st_head_stride,
                            st_row_stride, group_rows, cache, &ap);
  if (rc != hipSuccess) return rc;
  const int32_t* lens = cache->seq_lens;
  if (!counters || !lens_next || !aligned(counters, 4) || !aligned(lens_next, 4) ||
      !disjoint_lens(counters, lens, batch) || !disjoint_lens(lens_next, lens, batch) ||
      !disjoint_lens(counters, lens_next, batch))
    return hipErrorInvalidValue;
  DecodeArgs a;
  rc = make_decode_args(query, query_dtype, batch, num_q_heads, q_batch_stride, q_head_stride,
                        cache, 0, &a);
  if (rc != hipSuccess) return rc;
  if (!out || !valid_elem_dtype(out_dtype)) return hipErrorInvalidValue;
  // One q-head per kv-head and splits of whole scale groups (one split, or
  // chunks_per_split a multiple of a group's chunks, so that the open group
  // lies in one split): the append fuses into the decode (whose reads of a
  // group's staging rows take 32-bit byte offsets); with several splits the
  // merge follows it.
  const int group_chunks = cache->pages_per_group * ceil_div(cache->page_rows, 16);
  const bool fused = !a.mfma && a.heads_per_wg == 1 && a.hq_per_kv == 1 &&
                     (a.num_splits == 1 || a.chunks_per_split % group_chunks == 0) &&
                     (int64_t)group_rows * st_row_stride * 4 <= INT32_MAX;
  // Both forms check the workspace before anything is launched, so a rejected
  // call leaves the cache as it was.
  if (a.num_splits > 1 &&
      (!workspace || !aligned(workspace, kAlign) ||
       workspace_bytes < decode_ws_bytes(batch, num_q_heads, cache->head_dim, a.num_splits)))
    return hipErrorInvalidValue;
  if (!fused) {
    // Two launches: the append writes the advanced lengths to lens_next, the
    // decode attends over them and copies them back to the cache's lengths.
    // Everything the decode checks is checked before the append writes the
    // cache. The decode's plan (and so its split count and workspace)
    // depends on the shapes only.
    ap.lens_next = lens_next;
    hipError_t e = fdi4::launch_append_paged(ap, cache->head_dim, group_rows, batch,
                                             cache->num_kv_heads, stream);
    if (e != hipSuccess) return e;
    fdi4_paged_cache next = *cache;
    next.seq_lens = lens_next;
    return decode_paged_any(query, query_dtype, batch, num_q_heads, q_batch_stride,
                            q_head_stride, &next, out, out_dtype, out_batch_stride,
                            out_head_stride, 0, workspace, workspace_bytes,
                            const_cast<int32_t*>(lens), stream);
  }
  a.out = out;
  a.out_dtype = out_dtype;
  a.o_b = out_batch_stride;
  a.o_h = out_head_stride;
  a.final_out = a.num_splits == 1 ? 1 : 0;
  if (a.num_splits > 1) {
    rc = carve_partials(workspace, workspace_bytes, batch, num_q_heads, cache->head_dim, &a);
    if (rc != hipSuccess) return rc;
  }
  fdi4::StepAppend& st = a.step;
  st.k_new = k_new;
  st.kn_b = ap.kn_b;
  st.kn_h = ap.kn_h;
  st.v_new = ap.v_new;
  st.vn_b = ap.vn_b;
  st.vn_h = ap.vn_h;
  st.stage = k_stage;
  st.st_b = st_batch_stride;
  st.st_h = st_head_stride;
  st.st_r = st_row_stride;
  st.group_rows = group_rows;
  st.arrive = counters;
  st.lens = const_cast<int32_t*>(lens);
  hipError_t e = fdi4::launch_decode(a, cache->head_dim, cache->v_dtype, batch, stream);
  if (e != hipSuccess || a.num_splits == 1) return e;
  return fdi4::launch_merge(a.ws_acc, a.ws_ml, batch, num_q_heads, cache->head_dim, a.num_splits,
                            out, out_dtype, out_batch_stride, out_head_stride, stream);
}

int fdi4_decode_paged_partials(const float* query, int batch, int num_q_heads,
                               int64_t q_batch_stride, int64_t q_head_stride,
                               const fdi4_paged_cache* cache, int num_splits, void* partials,
                               size_t partials_bytes, hipStream_t stream) {
  DecodeArgs a;
  int rc = make_decode_args(query, FDI4_K_F32, batch, num_q_heads, q_batch_stride,
                            q_head_stride, cache, num_splits, &a);
  if (rc != hipSuccess) return rc;
  if (a.num_splits != num_splits) return hipErrorInvalidValue;  // the layout must be exact
  rc = carve_partials(partials, partials_bytes, batch, num_q_heads, cache->head_dim, &a);
  if (rc != hipSuccess) return rc;
  return launch_decode_any(a, cache->head_dim, cache->v_dtype, batch, stream);
}

}  // extern "C"

// ---- decode with its split partials in a static device array ------------------

namespace {

// Split partials of fdi4_decode_paged_noalloc. Every GPU the library runs on
// holds its own copy of this array until the process ends. In host code the
// name stands for a host-side shadow, not a device address: kernels and
// copies get the per-device address from scratch_address() instead.
static __device__ __align__(256) unsigned char scratch[FDI4_NOALLOC_SCRATCH_BYTES];

// Device address of `scratch` on device `dev`, looked up once per device
// (hipGetSymbolAddress with that device current) and kept.
hipError_t scratch_address(int dev, void** out) {
  static std::mutex mu;
  static std::map<int, void*> addrs;
  std::lock_guard<std::mutex> lock(mu);
  auto it = addrs.find(dev);
  if (it != addrs.end()) {
    *out = it->second;
    return hipSuccess;
  }
  int cur = 0;
  hipError_t e = hipGetDevice(&cur);
  if (e != hipSuccess) return e;
  if (cur != dev && (e = hipSetDevice(dev)) != hipSuccess) return e;
  void* p = nullptr;
  e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
  if (cur != dev) {
    const hipError_t r = hipSetDevice(cur);
    if (e == hipSuccess) e = r;
  }
  if (e != hipSuccess) return e;
  if (!p) return hipErrorInvalidSymbol;
  addrs[dev] = p;
  *out = p;
  return hipSuccess;
}

}  // namespace

extern "C" {

int fdi4_decode_paged_noalloc(const float* query, int batch, int num_q_heads,
                              int64_t q_batch_stride, int64_t q_head_stride,
                              const fdi4_paged_cache* cache, float* out,
                              int64_t out_batch_stride, int64_t out_head_stride, int num_splits,
                              hipStream_t stream) {
  DecodeArgs a;
  int rc = make_decode_args(query, FDI4_K_F32, batch, num_q_heads, q_batch_stride,
                            q_head_stride, cache, num_splits, &a);
  if (rc != hipSuccess) return rc;
  if (!out) return hipErrorInvalidValue;
  const int d = cache->head_dim;
  a.out = out;
  a.out_dtype = FDI4_K_F32;
  a.o_b = out_batch_stride;
  a.o_h = out_head_stride;
  if (a.num_splits == 1) {
    a.final_out = 1;
    return launch_decode_any(a, d, cache->v_dtype, batch, stream);
  }
  // Checked before any device call: partials beyond the array are refused.
  const size_t need = decode_ws_bytes(batch, num_q_heads, d, a.num_splits);
  if (need > (size_t)FDI4_NOALLOC_SCRATCH_BYTES) return hipErrorInvalidValue;
  int dev = 0;
  hipError_t e = stream ? hipStreamGetDevice(stream, &dev) : hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  void* base = nullptr;
  if ((e = scratch_address(dev, &base)) != hipSuccess) return e;
  // Every split writes its (m, l, acc) whether or not it holds rows, so the
  // array needs no clearing between calls.
  rc = carve_partials(base, need, batch, num_q_heads, d, &a);
  if (rc != hipSuccess) return rc;
  e = launch_decode_any(a, d, cache->v_dtype, batch, stream);
  if (e != hipSuccess) return e;
  return fdi4::launch_merge(a.ws_acc, a.ws_ml, batch, num_q_heads, d, a.num_splits, out,
                            FDI4_K_F32, out_batch_stride, out_head_stride, stream);
}

// ---- the reference's dense, shared-stream attention call ----------------------

}  // extern "C"

namespace {

struct DenseLayout {
  int dp;
  size_t off_k, off_q, off_v, off_s, off_z, off_o, off_part, total;
  int splits;
};

DenseLayout dense_layout(int B, int H, int D, int nb, int bs) {
  DenseLayout L;
  L.dp = padded_head_dim(D);
  const bool pad = L.dp != D;
  size_t off = 0;
  L.off_k = off;
  off += align_up((size_t)nb * bs * (L.dp / 2));
  L.off_q = L.off_v = L.off_s = L.off_z = L.off_o = 0;
  if (pad) {
    L.off_q = off;
    off += align_up((size_t)B * H * L.dp * sizeof(float));
    L.off_v = off;
    off += align_up((size_t)nb * bs * L.dp * sizeof(float));
    L.off_s = off;
    off += align_up((size_t)nb * L.dp * sizeof(float));
    L.off_z = off;
    off += align_up((size_t)nb * L.dp * sizeof(float));
    L.off_o = off;
    off += align_up((size_t)B * H * L.dp * sizeof(float));
  }
  // Every (sequence, head) attends the one shared page stream (kv-heads = 1).
  L.splits = plan_decode(B, H, H, L.dp, FDI4_V_F32, nb * ceil_div(bs, 16)).splits;
  L.off_part = off;
  off += decode_ws_bytes(B, H, L.dp, L.splits);
  L.total = std::max<size_t>(off, kAlign);
  return L;
}

bool dense_args_ok(int B, int H, int D, int nb, int bs) {
  return B > 0 && H > 0 && D >= 1 && D <= 256 && nb >= 0 && bs >= 0 && B <= 65535 &&
         H <= 65535;
}

}  // namespace

extern "C" {

size_t fdi4_flash_decode_int4_workspace_bytes(int batch_size, int num_heads, int head_dim,
                                              int num_blocks, int block_size) {
  if (!dense_args_ok(batch_size, num_heads, head_dim, num_blocks, block_size)) return 0;
  return dense_layout(batch_size, num_heads, head_dim, num_blocks, block_size).total;
}

int fdi4_flash_decode_int4_ws(const float* query, const uint8_t* k_q, const float* k_scale,
                              const float* k_zp, const float* value, const int* block_lens,
                              int B, int H, int D, int nb, int bs, float* output,
                              void* workspace, size_t workspace_bytes, hipStream_t stream) {
  if (!dense_args_ok(B, H, D, nb, bs) || !query || !output) return hipErrorInvalidValue;
  if (nb == 0 || bs == 0) {
    // No rows: the all-pages-empty case, exact zeros (a fill kernel, so the
    // call stays capturable into a graph).
    return fdi4::launch_pad_rows(output, (int64_t)B * H, 0, D, output, D, D, stream);
  }
  if (!k_q || !k_scale || !k_zp || !value || !block_lens) return hipErrorInvalidValue;
  const DenseLayout L = dense_layout(B, H, D, nb, bs);
  if (!workspace || workspace_bytes < L.total || !aligned(workspace, kAlign))
    return hipErrorInvalidValue;
  char* ws = reinterpret_cast<char*>(workspace);
  const int dp = L.dp;
  uint8_t* kp = reinterpret_cast<uint8_t*>(ws + L.off_k);
  hipError_t e = fdi4::launch_pack(k_q, (int64_t)nb * bs, D, D, kp, dp / 2, dp / 2, stream);
  if (e != hipSuccess) return e;
  const float* q = query;
  const float* v = value;
  const float* s = k_scale;
  const float* z = k_zp;
  float* o = output;
  if (dp != D) {
    float* qp = reinterpret_cast<float*>(ws + L.off_q);
    float* vp = reinterpret_cast<float*>(ws + L.off_v);
    float* sp = reinterpret_cast<float*>(ws + L.off_s);
    float* zp = reinterpret_cast<float*>(ws + L.off_z);
    if ((e = fdi4::launch_pad_rows(query, (int64_t)B * H, D, D, qp, dp, dp, stream))) return e;
    if ((e = fdi4::launch_pad_rows(value, (int64_t)nb * bs, D, D, vp, dp, dp, stream))) return e;
    if ((e = fdi4::launch_pad_rows(k_scale, nb, D, D, sp, dp, dp, stream))) return e;
    if ((e = fdi4::launch_pad_rows(k_zp, nb, D, D, zp, dp, dp, stream))) return e;
    q = qp;
    v = vp;
    s = sp;
    z = zp;
    o = reinterpret_cast<float*>(ws + L.off_o);
  }
  fdi4_paged_cache c = {};
  c.k_pages = kp;
  c.k_page_stride = (int64_t)bs * (dp / 2);
  c.k_head_stride = 0;
  c.k_row_stride = dp / 2;
  c.v_pages = const_cast<float*>(v);
  c.v_dtype = FDI4_V_F32;
  c.v_page_stride = (int64_t)bs * dp;
  c.v_head_stride = 0;
  c.v_row_stride = dp;
  c.k_scale = const_cast<float*>(s);
  c.k_zp = const_cast<float*>(z);
  c.s_page_stride = dp;
  c.page_table = nullptr;
  c.seq_lens = nullptr;
  c.page_lens = block_lens;
  c.pl_batch_stride = 0;
  c.num_kv_heads = 1;
  c.head_dim = dp;
  c.page_rows = bs;
  c.pages_per_group = 1;
  c.max_pages = nb;
  c.num_pages = nb;
  int rc = fdi4_decode_paged(q, B, H, (int64_t)H * dp, dp, &c, o, (int64_t)H * dp, dp, L.splits,
                             ws + L.off_part, L.total - L.off_part, stream);
  if (rc != hipSuccess) return rc;
  if (dp != D) {
    // Keep the first D channels: rows of dp floats back to rows of D floats.
    return fdi4::launch_pad_rows(o, (int64_t)B * H, D, dp, output, D, D, stream);
  }
  return hipSuccess;
}

int fdi4_flash_decode_int4(const float* query, const uint8_t* k_q, const float* k_scale,
                           const float* k_zp, const float* value, const int* block_lens,
                           int batch_size, int num_heads, int head_dim, int num_blocks,
                           int block_size, float* output, hipStream_t stream) {
  if (!dense_args_ok(batch_size, num_heads, head_dim, num_blocks, block_size))
    return hipErrorInvalidValue;
  const size_t wsb = fdi4_flash_decode_int4_workspace_bytes(batch_size, num_heads, head_dim,
                                                            num_blocks, block_size);
  void* ws = nullptr;
  hipError_t e = temp_alloc(&ws, wsb, stream);
  if (e != hipSuccess) return e;
  int rc = fdi4_flash_decode_int4_ws(query, k_q, k_scale, k_zp, value, block_lens, batch_size,
                                     num_heads, head_dim, num_blocks, block_size, output, ws, wsb,
                                     stream);
  hipError_t f = hipFreeAsync(ws, stream);
  return rc != hipSuccess ? rc : f;
}

int fdi4_fake_quantize(const void* k, int key_dtype, int batch, int heads, int seq_len,
                       int head_dim, int64_t k_batch_stride, int64_t k_head_stride,
                       int64_t k_row_stride, void* out, int64_t out_batch_stride,
                       int64_t out_head_stride, int64_t out_row_stride, int block_size,
                       int rounding, int scale_op, hipStream_t stream) {
  if (key_dtype != FDI4_K_F32 && key_dtype != FDI4_K_F16 && key_dtype != FDI4_K_BF16)
    return hipErrorInvalidValue;
  if (rounding != FDI4_ROUND_HALF_UP && rounding != FDI4_ROUND_HALF_EVEN)
    return hipErrorInvalidValue;
  if (scale_op != FDI4_SCALE_DIVIDE && scale_op != FDI4_SCALE_RECIPROCAL)
    return hipErrorInvalidValue;
  if (batch < 0 || heads < 0 || seq_len < 0 || batch > 65535 || heads > 65535 ||
      block_size < 1 || head_dim < 1 || head_dim > fdi4::fake_quant_max_head_dim())
    return hipErrorInvalidValue;
  if (batch == 0 || heads == 0 || seq_len == 0) return hipSuccess;
  if (!k || !out) return hipErrorInvalidValue;
  const int64_t esz = key_dtype == FDI4_K_F32 ? 4 : 2;
  // 16-byte vector loads and stores of whole row pieces.
  if ((head_dim * esz) % 16 || !aligned(k, 16) || !aligned(out, 16) ||
      (k_batch_stride * esz) % 16 || (k_head_stride * esz) % 16 || (k_row_stride * esz) % 16 ||
      (out_batch_stride * esz) % 16 || (out_head_stride * esz) % 16 ||
      (out_row_stride * esz) % 16)
    return hipErrorInvalidValue;
  fdi4::FakeQuantArgs a;
  a.k = static_cast<const uint8_t*>(k);
  a.k_b = k_batch_stride * esz;
  a.k_h = k_head_stride * esz;
  a.k_t = k_row_stride * esz;
  a.out = static_cast<uint8_t*>(out);
  a.o_b = out_batch_stride * esz;
  a.o_h = out_head_stride * esz;
  a.o_t = out_row_stride * esz;
  a.seq_len = seq_len;
  a.head_dim = head_dim;
  a.block = block_size;
  a.scale_recip = scale_op == FDI4_SCALE_RECIPROCAL ? 1 : 0;
  a.nsplit = a.cw = a.vpr = a.rpp = 0;
  return fdi4::launch_fake_quant(a, key_dtype, rounding, batch, heads, stream);
}

int fdi4_dequantize_int4(const uint8_t* q, int64_t rows, int num_channels, int64_t q_row_stride,
                         int packed, const float* scale, const float* zp,
                         int64_t s_row_stride, int64_t s_channel_stride, float* out,
                         int64_t out_row_stride, hipStream_t stream) {
  if (rows < 0 || num_channels <= 0 || s_row_stride < 0 || s_channel_stride < 0)
    return hipErrorInvalidValue;
  if (rows == 0) return hipSuccess;
  if (!q || !scale || !zp || !out) return hipErrorInvalidValue;
  const int64_t qcols = packed ? (num_channels + 1) / 2 : num_channels;
  if (q_row_stride < qcols || out_row_stride < num_channels) return hipErrorInvalidValue;
  return fdi4::launch_dequantize(q, rows, num_channels, q_row_stride, packed != 0, scale, zp,
                                 s_row_stride, s_channel_stride, out, out_row_stride, stream);
}

int fdi4_pack_int4(const uint8_t* q, int64_t rows, int num_channels, int64_t q_row_stride,
                   uint8_t* out, int64_t out_row_stride, int out_cols, hipStream_t stream) {
  if (!q || !out || rows < 0 || num_channels <= 0) return hipErrorInvalidValue;
  if (out_cols < (num_channels + 1) / 2 || out_row_stride < out_cols ||
      q_row_stride < num_channels)
    return hipErrorInvalidValue;
  return fdi4::launch_pack(q, rows, num_channels, q_row_stride, out, out_row_stride, out_cols,
                           stream);
}

}  // extern "C"
