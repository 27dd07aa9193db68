/*
 * fdi4 -- C ABI of the MI355X (gfx950) INT4 key quantizer and fused INT4
 * flash-decoding kernels.
 *
 * Every entry point is a plain C function over device pointers, sizes and
 * strides, enqueued asynchronously on the given HIP stream (0 = the null
 * stream); none synchronizes the host. Return value: a hipError_t code
 * (0 = hipSuccess, 1 = hipErrorInvalidValue for rejected sizes, otherwise the
 * launch error). Inputs are borrowed for the duration of the enqueued work;
 * nothing is retained between calls.
 *
 * The library is libfdi4.so in the package directory
 * int4-kv-cache-quantization-cuda-triton-pallas_amd/flash_decode_int4/.
 */
#ifndef FDI4_H_
#define FDI4_H_

#include <stddef.h>
#include <stdint.h>
#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

#define FDI4_ABI_VERSION 1

enum fdi4_value_dtype { FDI4_V_F32 = 0, FDI4_V_F16 = 1, FDI4_V_BF16 = 2 };
/* Element types of key tensors (fdi4_fake_quantize) and of the queries and
 * outputs of fdi4_decode_paged_ex. */
enum fdi4_key_dtype { FDI4_K_F32 = 0, FDI4_K_F16 = 1, FDI4_K_BF16 = 2 };
enum fdi4_rounding { FDI4_ROUND_HALF_UP = 0, FDI4_ROUND_HALF_EVEN = 1 };
enum fdi4_scale_op { FDI4_SCALE_DIVIDE = 0, FDI4_SCALE_RECIPROCAL = 1 };

/* Device layout of a paged INT4 key/value cache.
 *
 *   k_pages   packed keys, byte j of a row = channel 2j (low nibble) |
 *             channel 2j+1 (high nibble); address of row r of physical page p,
 *             kv-head h: k_pages + p*k_page_stride + h*k_head_stride +
 *             r*k_row_stride (bytes). A row holds head_dim/2 bytes.
 *   v_pages   values (fp32, fp16 or bf16), same addressing in elements.
 *   k_scale,  per-channel scale and zero-point of the scale group of logical
 *   k_zp      page lp of sequence b: element offset
 *             b*s_batch_stride + h*s_head_stride + (lp/pages_per_group)*s_group_stride
 *             + p*s_page_stride (+ channel). s_page_stride != 0 (scales attached to
 *             physical pages) requires pages_per_group == 1.
 *   page_table [B, pt_batch_stride] int32 physical page of each logical page;
 *             NULL means logical page == physical page. Entries are clamped to
 *             [0, num_pages) on the device, so a bad table cannot address
 *             memory outside the pool (the results are then meaningless).
 *   seq_lens  [B] int32 valid tokens; NULL means every sequence spans max_pages
 *             full pages (then page_lens gives the valid rows).
 *   page_lens [B, pl_batch_stride] int32 valid rows of each logical page, or NULL;
 *             values are clamped to [0, page_rows].
 * head_dim is 64, 128 or 256 for the paged entry points. page_rows and
 * pages_per_group are >= 1. Strides of 0 share one stream between sequences or
 * heads (the reference's shared-page-stream semantics).
 */
typedef struct fdi4_paged_cache {
  uint8_t* k_pages;
  int64_t k_page_stride, k_head_stride, k_row_stride;
  void* v_pages;
  int32_t v_dtype;
  int64_t v_page_stride, v_head_stride, v_row_stride;
  float* k_scale;
  float* k_zp;
  int64_t s_batch_stride, s_head_stride, s_group_stride, s_page_stride;
  const int32_t* page_table;
  int64_t pt_batch_stride;
  const int32_t* seq_lens;
  const int32_t* page_lens;
  int64_t pl_batch_stride;
  int32_t num_kv_heads;
  int32_t head_dim;
  int32_t page_rows;
  int32_t pages_per_group;
  int32_t max_pages;  /* logical pages per sequence (columns of page_table) */
  int32_t num_pages;  /* physical pages in the pool */
} fdi4_paged_cache;

/* Launch-shape overrides, for measurement and tests; production callers
 * need none of them. The library reads no environment variables: the
 * automatic choices below apply unless a caller sets a knob here. Settings
 * are process-wide and take effect for calls made after fdi4_set_tuning
 * returns; value 0 restores the automatic choice.
 *
 *   FDI4_TUNE_DECODE_VECTOR_ONLY   1: grouped-head decodes at head_dim 64/128
 *                                  run on the vector kernels instead of the
 *                                  int8 matrix-core kernel
 *   FDI4_TUNE_DECODE_WAVES         4 or 8 decode wave64s per workgroup (the
 *                                  fused serving step adds 4 re-quantizing
 *                                  waves to 4-wave workgroups, and to 8-wave
 *                                  ones where registers allow)
 *   FDI4_TUNE_DECODE_HEADS_PER_WG  cap on q-heads per decode workgroup: 1
 *                                  (per-head kernel), 2, 4 or 8
 *   FDI4_TUNE_DECODE_TARGET_WAVES  resident waves the split count aims for
 *                                  (1 .. 1<<20)
 *   FDI4_TUNE_FAKE_QUANT_SPLIT     channel slices per key row of
 *                                  fdi4_fake_quantize (1 .. 512)
 */
enum fdi4_tuning_knob {
  FDI4_TUNE_DECODE_VECTOR_ONLY = 0,
  FDI4_TUNE_DECODE_WAVES = 1,
  FDI4_TUNE_DECODE_HEADS_PER_WG = 2,
  FDI4_TUNE_DECODE_TARGET_WAVES = 3,
  FDI4_TUNE_FAKE_QUANT_SPLIT = 4,
  FDI4_TUNE_COUNT = 5
};

/* Set a knob (hipErrorInvalidValue for an unknown knob or a value outside
 * its range; the setting is then unchanged). No counterpart in the
 * reference, whose launch shapes are fixed. */
int fdi4_set_tuning(int knob, int value);

/* Current value of a knob (0 = automatic; -1 for an unknown knob). */
int fdi4_get_tuning(int knob);

/* ABI version of the loaded library (FDI4_ABI_VERSION). */
int fdi4_abi_version(void);

/* Human-readable text of a status code returned by this library. */
const char* fdi4_error_string(int status);

/* Per-channel asymmetric INT4 quantization of kv[num_rows, num_channels]
 * (row-major, contiguous) as ONE scale group over all rows; q_out is one
 * value per byte [num_rows, num_channels], scale_out/zp_out are [num_channels].
 * Bit-exact with NumPy: round half to even, IEEE float32 division.
 * Replaces cu_quantize_int4 (reference csrc/flash_decode_int4.cu:228-247,
 * declared at csrc/bindings.cpp:17-18); same arguments. Takes a stream-ordered
 * temporary for the row-tile partials from a memory pool the library keeps on
 * the stream's device (hipMallocFromPoolAsync). */
int fdi4_quantize_int4(const float* kv, int num_rows, int num_channels, uint8_t* q_out,
                       float* scale_out, float* zp_out, hipStream_t stream);

/* Workspace needed by fdi4_quantize_rows. */
size_t fdi4_quantize_rows_workspace_bytes(int64_t num_rows, int num_channels);

/* General form of fdi4_quantize_int4 with row strides (elements / bytes),
 * nibble-packed output when packed != 0 (q_out row = ceil(C/2) bytes), and a
 * caller-provided workspace (no allocation). Serves the reference's
 * ops.quantize_int4 (src/ops.py:111-161) and the paged cache's block writes
 * (src/vllm_integration.py:48-56). */
int fdi4_quantize_rows(const float* kv, int64_t num_rows, int num_channels,
                       int64_t kv_row_stride, uint8_t* q_out, int64_t q_row_stride, int packed,
                       float* scale_out, float* zp_out, void* workspace,
                       size_t workspace_bytes, hipStream_t stream);

/* Grouped quantization of keys k[b, h, t, :] (element strides, channel stride
 * 1, 16-byte aligned rows) for t < cache->seq_lens[b]: every group_rows tokens
 * of one (sequence, kv-head) form one scale group (a partial last group uses
 * its valid rows only); packed rows are written through cache->page_table
 * and the group scales to cache->k_scale / k_zp. group_rows is 64, 128 or 256
 * and a multiple of cache->page_rows; head_dim is 64, 128 or 256. Counterpart
 * of the reference's per-group quantize_int4_ref + pack_int4
 * (src/quantize_int4_ref.py:23-84, src/int4_pack.py:14-29) on device. */
int fdi4_quantize_paged(const float* k, int batch, int max_tokens, int64_t k_batch_stride,
                        int64_t k_head_stride, int64_t k_row_stride, int group_rows,
                        const fdi4_paged_cache* cache, hipStream_t stream);

/* Decode-time append of one token per sequence b < batch at position
 * t = cache->seq_lens[b] (t < max_pages * page_rows; the caller has mapped
 * the page holding t in cache->page_table and advances seq_lens afterwards):
 * the value row v_new[b, h, :] (the cache's value type, element strides) goes
 * to its page, the key row k_new[b, h, :] (float32) to row t % group_rows of
 * k_stage[b, h, :, :] (float32, element strides), and the open scale group
 * g = t / group_rows is re-quantized over its t % group_rows + 1 valid rows
 * from k_stage -- packed rows to the pages, scale and zero-point to group g.
 * The result equals fdi4_quantize_paged over the whole sequence of t + 1
 * tokens (the reference quantizes a partial group over its valid rows,
 * tests/test_perplexity_harness.py:122-131). k_stage must hold the open
 * group's earlier key rows (after a prefill: rows g*group_rows .. t-1). The
 * device form of the cache write (reference src/vllm_integration.py:48-56)
 * for one token per step. */
int fdi4_append_paged(const float* k_new, int64_t kn_batch_stride, int64_t kn_head_stride,
                      const void* v_new, int64_t vn_batch_stride, int64_t vn_head_stride,
                      int batch, float* k_stage, int64_t st_batch_stride, int64_t st_head_stride,
                      int64_t st_row_stride, int group_rows, const fdi4_paged_cache* cache,
                      hipStream_t stream);

/* fdi4_append_paged that also writes lens_next[b] = cache->seq_lens[b] + 1
 * for every sequence b < batch whose token it appended (seq_lens[b] when the
 * position falls outside the cache), from one workgroup per sequence; the
 * cache's own lengths are not changed. lens_next is int32 [batch], 4-byte
 * aligned, and must not overlap cache->seq_lens[0, batch) (hipErrorInvalidValue
 * otherwise; cache->seq_lens must be given). With fdi4_decode_paged_advance
 * reading lens_next and writing the lengths back, one decode step of a
 * serving loop is two launches with no separate length update, the same
 * launches every step (so a captured HIP graph replays them unchanged). No
 * counterpart in the reference, whose cache appends on the host. */
int fdi4_append_paged_advance(const float* k_new, int64_t kn_batch_stride,
                              int64_t kn_head_stride, const void* v_new,
                              int64_t vn_batch_stride, int64_t vn_head_stride, int batch,
                              float* k_stage, int64_t st_batch_stride, int64_t st_head_stride,
                              int64_t st_row_stride, int group_rows,
                              const fdi4_paged_cache* cache, int32_t* lens_next,
                              hipStream_t stream);

/* Fused INT4 flash decoding with the reference's exact arguments: query
 * [B, H, D], k_q [nb, bs, D] one INT4 value per byte, k_scale/k_zp [nb, D],
 * value [nb, bs, D] fp32, block_lens [nb]; every (b, h) query attends the same
 * page stream; 1 <= D <= 256. Replaces cu_flash_decode_int4 (reference
 * csrc/flash_decode_int4.cu:249-284, declared at csrc/bindings.cpp:19-21).
 * Packs keys into a stream-ordered temporary from the library's memory pool on
 * the stream's device, then runs the split-K decode. */
int fdi4_flash_decode_int4(const float* query, const uint8_t* k_q, const float* k_scale,
                           const float* k_zp, const float* value, const int* block_lens,
                           int batch_size, int num_heads, int head_dim, int num_blocks,
                           int block_size, float* output, hipStream_t stream);

/* Workspace for fdi4_flash_decode_int4_ws. */
size_t fdi4_flash_decode_int4_workspace_bytes(int batch_size, int num_heads, int head_dim,
                                              int num_blocks, int block_size);

/* fdi4_flash_decode_int4 with a caller-provided workspace (no allocation);
 * serves the reference's _C.flash_decode_int4 binding (csrc/bindings.cpp:56-127). */
int fdi4_flash_decode_int4_ws(const float* query, const uint8_t* k_q, const float* k_scale,
                              const float* k_zp, const float* value, const int* block_lens,
                              int batch_size, int num_heads, int head_dim, int num_blocks,
                              int block_size, float* output, void* workspace,
                              size_t workspace_bytes, hipStream_t stream);

/* Split count the decode would choose for this shape when num_splits <= 0
 * (reads cache->num_kv_heads, head_dim, max_pages and page_rows only; 1 when
 * num_kv_heads does not divide num_q_heads). */
int fdi4_decode_num_splits(int batch, int num_q_heads, const fdi4_paged_cache* cache);

/* Workspace for fdi4_decode_paged with the given split count (0 when 1). */
size_t fdi4_decode_workspace_bytes(int batch, int num_q_heads, int head_dim, int num_splits);

/* Split-K paged decode: out[b, h, :] = softmax(q[b,h].K^T) V over the valid
 * rows of sequence b, kv-head h / (num_q_heads / num_kv_heads) (up to eight
 * q-heads of one kv-head share a workgroup and one read of its pages); unscaled
 * logits; empty pages skipped; a sequence with no valid row gives exact
 * zeros. num_splits <= 0 selects fdi4_decode_num_splits. With more than one
 * split the partials go to the workspace and the merge kernel runs on the
 * same stream. Counterpart of the reference's flash_decode_int4_kernel
 * (csrc/flash_decode_int4.cu:104-221) generalized to per-sequence page
 * tables, group scales and packed keys. */
int fdi4_decode_paged(const float* query, int batch, int num_q_heads, int64_t q_batch_stride,
                      int64_t q_head_stride, const fdi4_paged_cache* cache, float* out,
                      int64_t out_batch_stride, int64_t out_head_stride, int num_splits,
                      void* workspace, size_t workspace_bytes, hipStream_t stream);

/* fdi4_decode_paged with queries and outputs of any element type
 * (fdi4_key_dtype: FDI4_K_F32, FDI4_K_F16, FDI4_K_BF16). The queries are
 * widened to float32 exactly, the arithmetic is that of fdi4_decode_paged,
 * and each output element is rounded once, to nearest even, from its float32
 * value. The fp16/bf16 query and output side of the cache's 16-bit storage
 * (the reference stores fp16 values, src/vllm_integration.py:45, 55). */
int fdi4_decode_paged_ex(const void* query, int query_dtype, int batch, int num_q_heads,
                         int64_t q_batch_stride, int64_t q_head_stride,
                         const fdi4_paged_cache* cache, void* out, int out_dtype,
                         int64_t out_batch_stride, int64_t out_head_stride, int num_splits,
                         void* workspace, size_t workspace_bytes, hipStream_t stream);

/* fdi4_decode_paged_ex that also copies the lengths it reads
 * (cache->seq_lens[b], b < batch) to lens_out[b] when the decode kernel ends
 * (int32 [batch], 4-byte aligned, not overlapping cache->seq_lens[0, batch);
 * cache->seq_lens must be given). The second launch of a serving step:
 * after fdi4_append_paged_advance(seq_lens = L, lens_next = N), this call
 * with seq_lens = N and lens_out = L attends over the advanced lengths and
 * leaves L == N. No counterpart in the reference. */
int fdi4_decode_paged_advance(const void* query, int query_dtype, int batch, int num_q_heads,
                              int64_t q_batch_stride, int64_t q_head_stride,
                              const fdi4_paged_cache* cache, void* out, int out_dtype,
                              int64_t out_batch_stride, int64_t out_head_stride, int num_splits,
                              void* workspace, size_t workspace_bytes, int32_t* lens_out,
                              hipStream_t stream);

/* One decode step of a serving loop: append token t = cache->seq_lens[b]
 * of every sequence b < batch (k_new float32 and v_new in the cache's value
 * type, [batch, num_kv_heads, head_dim] with element strides; the staging
 * rows k_stage as in fdi4_append_paged), attend with query over the t + 1
 * rows, and advance cache->seq_lens[b] to t + 1. A length outside
 * [0, capacity) (capacity = max_pages * page_rows; a sequence already full,
 * or a corrupt length) appends nothing, stays as it is, and the decode
 * attends over it clamped to [0, capacity]. The result equals
 * fdi4_append_paged, that length update and fdi4_decode_paged_ex, bit for
 * bit. Every argument is checked before anything is enqueued: a rejected
 * call (hipErrorInvalidValue) leaves the cache unchanged.
 * With num_q_heads == num_kv_heads and splits of whole scale groups (a single
 * split, or a split length that is a multiple of a group's 16-row chunks)
 * this is ONE launch, then the split merge when there are several: the
 * workgroup of the split that holds the open group appends its token and
 * re-quantizes the group before it decodes it, and the last workgroup of a
 * sequence to count itself advances its length (counters: int32 [batch],
 * zero before the first call, left zero by every call). Otherwise it is
 * fdi4_append_paged_advance into lens_next (int32 [batch] scratch) and
 * fdi4_decode_paged_advance back. Both use the library's split count
 * (workspace of fdi4_decode_workspace_bytes). counters,
 * lens_next and cache->seq_lens must not overlap. No counterpart in the
 * reference, whose cache appends on the host. */
int fdi4_decode_step(const void* query, int query_dtype, int batch, int num_q_heads,
                     int64_t q_batch_stride, int64_t q_head_stride, const float* k_new,
                     int64_t kn_batch_stride, int64_t kn_head_stride, const void* v_new,
                     int64_t vn_batch_stride, int64_t vn_head_stride, float* k_stage,
                     int64_t st_batch_stride, int64_t st_head_stride, int64_t st_row_stride,
                     int group_rows, const fdi4_paged_cache* cache, void* out, int out_dtype,
                     int64_t out_batch_stride, int64_t out_head_stride, int32_t* counters,
                     int32_t* lens_next, void* workspace, size_t workspace_bytes,
                     hipStream_t stream);

/* Bytes of the split partials for fdi4_decode_paged_partials: part_acc
 * float [B, Hq, S, D] at offset 0, then part_ml double [B, Hq, S, 2] = (m, l)
 * at offset round_up(B*Hq*S*D*4, 256). */
size_t fdi4_decode_partials_bytes(int batch, int num_q_heads, int head_dim, int num_splits);

/* The decode kernel alone: writes the per-split partials (the layout of
 * fdi4_decode_partials_bytes) instead of the output; num_splits >= 1 and at
 * most one split per 16-row chunk of the longest sequence. With
 * fdi4_merge_splits this is fdi4_decode_paged in two calls -- for timing the
 * kernels separately, and for split-K across devices (gather the partials,
 * then merge once). */
int fdi4_decode_paged_partials(const float* query, int batch, int num_q_heads,
                               int64_t q_batch_stride, int64_t q_head_stride,
                               const fdi4_paged_cache* cache, int num_splits, void* partials,
                               size_t partials_bytes, hipStream_t stream);

/* Largest split-partials size fdi4_decode_paged_noalloc holds:
 * fdi4_decode_workspace_bytes(batch, num_q_heads, head_dim, splits) must not
 * exceed it (at head_dim 128: 528 bytes per (sequence, q-head, split), about
 * 15,800 of them). */
#define FDI4_NOALLOC_SCRATCH_BYTES (8u << 20)

/* fdi4_decode_paged without a workspace argument and without any allocation:
 * with more than one split the partials go to a static device array of
 * FDI4_NOALLOC_SCRATCH_BYTES that the library holds on each GPU (its address
 * is looked up, with hipGetSymbolAddress, on the first multi-split call on a
 * device: make that call once eagerly, outside any HIP graph capture, before
 * capturing the entry point; later calls only enqueue kernels and can be
 * captured). A call whose partials would
 * exceed the array returns hipErrorInvalidValue before any device work. The
 * caller still passes the inputs and the output. Calls that overlap on one GPU
 * (concurrent streams, or threads) share the array and race; serialize them.
 * No counterpart in the reference: for callers that cannot allocate device
 * memory (code under HIP graph capture, allocation-free serving loops). */
int fdi4_decode_paged_noalloc(const float* query, int batch, int num_q_heads,
                              int64_t q_batch_stride, int64_t q_head_stride,
                              const fdi4_paged_cache* cache, float* out,
                              int64_t out_batch_stride, int64_t out_head_stride, int num_splits,
                              hipStream_t stream);

/* Log-sum-exp merge of split partials part_acc [B, Hq, S, D] fp32 and
 * part_ml [B, Hq, S, 2] fp64 (m, l), as written by fdi4_decode_paged, into
 * out. Exposed so that partials gathered from several devices can be merged.
 * Counterpart of the cross-warp merge of the reference kernel
 * (csrc/flash_decode_int4.cu:186-220). */
int fdi4_merge_splits(const float* part_acc, const double* part_ml, int batch, int num_q_heads,
                      int head_dim, int num_splits, float* out, int64_t out_batch_stride,
                      int64_t out_head_stride, hipStream_t stream);

/* INT4 quantize-dequantize ("fake quantization") of keys k[b, h, t, :]
 * (b < batch, h < heads, t < seq_len; element strides, channel stride 1) into
 * out (same dtype, its own element strides): per (sequence, head, block of
 * block_size positions, channel) over the block's valid rows, mn/mx,
 * scale = max(mx - mn, 1e-8f) / 15 (FDI4_SCALE_DIVIDE, IEEE division, as
 * NumPy and torch on the CPU evaluate the reference's formula) or
 * max(mx - mn, 1e-8f) * float(1/15) (FDI4_SCALE_RECIPROCAL, as eager torch on
 * a GPU evaluates it: a tensor divided by a Python scalar is multiplied by
 * the reciprocal), and
 *   FDI4_ROUND_HALF_UP:   q = clamp(floor((x - mn) / scale + 0.5), 0, 15),
 *                         out = q*scale + mn
 *   FDI4_ROUND_HALF_EVEN: q = clamp(rint((x - mn) / scale), 0, 15),
 *                         zp = -mn / scale, out = q*scale - zp*scale
 * in float32 (one rounding per operation), converted to the key dtype
 * (FDI4_K_F32 / F16 / BF16) with round-to-nearest-even. Finite keys only.
 * head_dim * element size is a multiple of 16 bytes and head_dim <= 512; k,
 * out and their strides are 16-byte aligned; block_size >= 1; heads and
 * batch <= 65535. out must not overlap k. Half-up is fake_quantize_keys of
 * the reference's quality study (scripts/validate_llama.py:126-154);
 * half-even is its stored scheme, quantize_and_dequantize_ref
 * (src/quantize_int4_ref.py:139-158), per block. */
int fdi4_fake_quantize(const void* k, int key_dtype, int batch, int heads, int seq_len,
                       int head_dim, int64_t k_batch_stride, int64_t k_head_stride,
                       int64_t k_row_stride, void* out, int64_t out_batch_stride,
                       int64_t out_head_stride, int64_t out_row_stride, int block_size,
                       int rounding, int scale_op, hipStream_t stream);

/* Dequantization of stored INT4 values: out[r, c] = q*s - zp*s in float32
 * (two rounded products, then a rounded subtraction) with s = scale[r *
 * s_row_stride + c * s_channel_stride] and zp at the same offset: strides
 * (0, 1) for per-channel scales [num_channels], (1, 0) for per-row scales
 * [rows], (num_channels, 1) for one scale per element. q is one value per
 * byte (the whole byte is the value) or, with packed != 0, two per byte
 * (channel c in the low nibble of byte c/2 when c is even, the high nibble
 * when odd); row strides in bytes (q) and elements (out). Bit-exact with the
 * reference's dequantize_int4_ref (src/quantize_int4_ref.py:87-136), which
 * the decode kernels fuse into their logits instead. */
int fdi4_dequantize_int4(const uint8_t* q, int64_t rows, int num_channels, int64_t q_row_stride,
                         int packed, const float* scale, const float* zp,
                         int64_t s_row_stride, int64_t s_channel_stride, float* out,
                         int64_t out_row_stride, hipStream_t stream);

/* Device nibble packing: out[r, j] = q[r, 2j] | q[r, 2j+1] << 4 for
 * j < ceil(C/2) (odd C zero-padded), zero for ceil(C/2) <= j < out_cols.
 * Values are taken modulo 16. Counterpart of pack_int4 (reference
 * src/int4_pack.py:14-29). */
int fdi4_pack_int4(const uint8_t* q, int64_t rows, int num_channels, int64_t q_row_stride,
                   uint8_t* out, int64_t out_row_stride, int out_cols, hipStream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* FDI4_H_ */
