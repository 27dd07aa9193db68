// Kernel argument blocks and launcher declarations shared by the HIP
// translation units and the C-ABI layer. Not part of the public interface.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace fdi4 {

enum VDtype : int { kVF32 = 0, kVF16 = 1, kVBF16 = 2 };

// Element types of queries and outputs (the codes of fdi4_key_dtype).
enum EDtype : int { kEF32 = 0, kEF16 = 1, kEBF16 = 2 };

// Grouped paged quantizer: keys [B, H, T, D] (any strides, channel stride 1)
// into packed pages and group scales.
struct QuantPagedArgs {
  const float* k;
  int64_t k_b, k_h, k_t;                // elements
  const int32_t* seq_lens;              // [B]
  const int32_t* page_table;            // [B, pt_b]
  int64_t pt_b;
  uint8_t* k_pages;
  int64_t kp_page, kp_head, kp_row;     // bytes
  float* scale;
  float* zp;
  int64_t s_b, s_h, s_g;                // elements
  int page_rows;
  int num_pages;                        // physical pages; table entries are clamped
  int max_tokens;                       // rows of k; sequence lengths are clamped to it
};

// Decode-time append of one token per sequence (grouped quantizer re-run over
// the open group from a staging copy of its key rows).
struct AppendArgs {
  QuantPagedArgs q;                     // pages, scales, table, lengths (k unused)
  const float* k_new;
  int64_t kn_b, kn_h;                   // elements
  const uint8_t* v_new;
  int64_t vn_b, vn_h;                   // bytes
  uint8_t* v_pages;
  int64_t vp_page, vp_head, vp_row;     // bytes
  int v_row_bytes;                      // head_dim * value element size
  float* stage;
  int64_t st_b, st_h, st_r;             // elements
  int capacity;                         // max_pages * page_rows
  int32_t* lens_next;                   // null, or [B]: the length after this append
};

// Where the fused serving step of the decode writes one token (k_new null:
// no step): the new key row (float32),
// the new value row (the cache's value type, as bytes) and the staging rows
// of the open group, per (sequence, kv-head).
struct StepAppend {
  const float* k_new;
  int64_t kn_b, kn_h;                   // elements
  const uint8_t* v_new;
  int64_t vn_b, vn_h;                   // bytes
  float* stage;
  int64_t st_b, st_h, st_r;             // elements
  int group_rows;                       // 64, 128 or 256, a multiple of page_rows
  int32_t* arrive;                      // [B] arrival counters, zero between steps
  int32_t* lens;                        // [B] the lengths, advanced by the last arriver
};

// Split-K paged decode.
struct DecodeArgs {
  const void* q;
  int q_dtype;                          // EDtype of q
  int64_t q_b, q_h;                     // elements
  const uint8_t* k_pages;
  int64_t k_page, k_head, k_row;        // bytes
  const void* v_pages;
  int64_t v_page, v_head, v_row;        // elements
  const float* k_scale;
  const float* k_zp;
  int64_t s_b, s_h, s_g, s_p;           // elements
  const int32_t* page_table;            // null: logical page == physical page
  int64_t pt_b;
  const int32_t* seq_lens;              // null: every sequence spans max_pages pages
  const int32_t* page_lens;             // null: rows from seq_lens
  int64_t pl_b;
  int page_rows, pages_per_group, max_pages, hq_per_kv, num_pages;
  int chunks_per_split, num_splits, num_q_heads;
  int final_out;                        // 1: normalized output; 0: split partials
  int waves;                            // wave64s per workgroup (4 or 8)
  int heads_per_wg;                     // q-heads per workgroup (1: per-head kernel)
  int mfma;                             // int8 matrix-core kernel (D = 64 or 128)
  void* out;
  int out_dtype;                        // EDtype of out
  int64_t o_b, o_h;
  float* ws_acc;                        // [B, Hq, S, D]
  double* ws_ml;                        // [B, Hq, S, 2] = (m, l)
  int32_t* lens_out;                    // null, or [B]: receives the lengths read
  StepAppend step;                      // the fused serving step (step.k_new != null)
};

// Quantize-dequantize of keys [B, H, T, D] (channel stride 1) in blocks of
// `block` positions into out (same type and shape, own strides).
struct FakeQuantArgs {
  const uint8_t* k;
  int64_t k_b, k_h, k_t;                // bytes
  uint8_t* out;
  int64_t o_b, o_h, o_t;                // bytes
  int seq_len, head_dim, block;
  int scale_recip;                      // 1: scale = span * (1/15); 0: span / 15
  // Set by the launcher: channel slices per block, channels per slice,
  // 16-byte vectors per slice row, rows per sweep.
  int nsplit, cw, vpr, rpp;
};

// Value of a launch-shape override (fdi4_set_tuning; 0 = automatic).
int tuning(int knob);

hipError_t launch_quantize_rows(const float* kv, int64_t rows, int C, int64_t stride, uint8_t* q,
                                int64_t q_stride, bool packed, float* scale_out, float* zp_out,
                                void* ws, hipStream_t st);
size_t rows_workspace_bytes(int64_t rows, int C);

hipError_t launch_quantize_paged(const QuantPagedArgs& a, int D, int group, int batch, int heads,
                                 int max_tokens, hipStream_t st);

hipError_t launch_append_paged(const AppendArgs& a, int D, int group, int batch, int heads,
                               hipStream_t st);

hipError_t launch_pack(const uint8_t* q, int64_t rows, int C, int64_t q_stride, uint8_t* out,
                       int64_t o_stride, int out_cols, hipStream_t st);

hipError_t launch_dequantize(const uint8_t* q, int64_t rows, int C, int64_t q_stride, int packed,
                             const float* scale, const float* zp, int64_t s_rs, int64_t s_cs,
                             float* out, int64_t o_stride, hipStream_t st);

hipError_t launch_decode(const DecodeArgs& a, int D, int v_dtype, int batch, hipStream_t st);

hipError_t launch_decode_gqa(const DecodeArgs& a, int D, int v_dtype, int batch, int hg,
                             hipStream_t st);

hipError_t launch_decode_mfma(const DecodeArgs& a, int D, int v_dtype, int batch, int hg,
                              hipStream_t st);

hipError_t launch_merge(const float* ws_acc, const double* ws_ml, int batch, int hq, int D,
                        int splits, void* out, int out_dtype, int64_t o_b, int64_t o_h,
                        hipStream_t st);

hipError_t launch_fake_quant(const FakeQuantArgs& a, int key_dtype, int rounding, int batch,
                             int heads, hipStream_t st);
int fake_quant_max_head_dim();

hipError_t launch_pad_rows(const float* src, int64_t rows, int cols, int64_t s_stride, float* dst,
                           int64_t d_stride, int d_cols, hipStream_t st);

}  // namespace fdi4
