// Thin PyTorch-ROCm binding over the fdi4 C ABI (include/fdi4.h).
//
// Replaces the reference's csrc/bindings.cpp: the same Python names
// (quantize_int4, flash_decode_int4), argument order, shape/dtype checks and
// error-message substrings, plus the paged entry points. This file holds no
// device code: it validates tensors, allocates outputs and workspaces with
// torch's caching allocator, takes the current HIP stream and calls the C
// functions, which enqueue asynchronously.

#include <ATen/hip/impl/HIPGuardImplMasqueradingAsCUDA.h>
#include <c10/hip/HIPStream.h>
#include <torch/extension.h>

#include <cstdint>
#include <vector>

#include "../../include/fdi4.h"

namespace {

// The attention kernel's head_dim limit (reference csrc/bindings.cpp:13-15).
constexpr int64_t kMaxHeadDim = 256;

// The current stream of the current device; every entry point first makes
// the device of its tensors current (DeviceGuard), so the work is enqueued
// there whatever device the caller has current.
hipStream_t stream() { return c10::hip::getCurrentHIPStream().stream(); }

using DeviceGuard = c10::hip::OptionalHIPGuardMasqueradingAsCUDA;

#define CHECK_DEV(x) TORCH_CHECK((x).is_cuda(), #x " must be a GPU (cuda device) tensor")
#define CHECK_CONTIGUOUS(x) TORCH_CHECK((x).is_contiguous(), #x " must be contiguous")
#define CHECK_INPUT(x) \
  CHECK_DEV(x);        \
  CHECK_CONTIGUOUS(x)
#define CHECK_SAME_DEVICE(ref, x) \
  TORCH_CHECK((x).device() == (ref).device(), #x " must be on the device of " #ref)

void check_rc(int rc, const char* what) {
  TORCH_CHECK(rc == 0, what, " failed: ", fdi4_error_string(rc));
}

torch::Tensor workspace(const torch::Tensor& like, size_t bytes) {
  return torch::empty({(int64_t)std::max<size_t>(bytes, 256)},
                      torch::TensorOptions().dtype(torch::kUInt8).device(like.device()));
}

// reference csrc/bindings.cpp:26-54
std::vector<torch::Tensor> quantize_int4(torch::Tensor kv) {
  CHECK_INPUT(kv);
  TORCH_CHECK(kv.dim() == 2, "kv must be 2D [num_rows, num_channels]");
  TORCH_CHECK(kv.scalar_type() == torch::kFloat32, "kv must be float32");
  TORCH_CHECK(kv.size(0) > 0 && kv.size(1) > 0, "kv must be non-empty, got [", kv.size(0), ", ",
              kv.size(1), "]");
  TORCH_CHECK(kv.size(0) <= INT32_MAX && kv.size(1) <= INT32_MAX,
              "kv dimensions must fit in int32");
  const DeviceGuard guard(kv.device());
  const int64_t rows = kv.size(0);
  const int c = (int)kv.size(1);
  auto q = torch::empty({rows, c}, kv.options().dtype(torch::kUInt8));
  auto scale = torch::empty({c}, kv.options());
  auto zp = torch::empty({c}, kv.options());
  const size_t wsb = fdi4_quantize_rows_workspace_bytes(rows, c);
  auto ws = workspace(kv, wsb);
  check_rc(fdi4_quantize_rows(kv.data_ptr<float>(), rows, c, c, q.data_ptr<uint8_t>(), c, 0,
                              scale.data_ptr<float>(), zp.data_ptr<float>(), ws.data_ptr(),
                              ws.numel(), stream()),
           "quantize_int4");
  return {q, scale, zp};
}

// One scale group over all rows of kv, written into caller-provided views
// (q_out rows may be strided, e.g. a slot of a page pool); packed != 0 writes
// nibble pairs (q_out width ceil(C/2)).
void quantize_rows_into(torch::Tensor kv, torch::Tensor q_out, torch::Tensor scale_out,
                        torch::Tensor zp_out, bool packed) {
  CHECK_DEV(kv);
  CHECK_DEV(q_out);
  CHECK_INPUT(scale_out);
  CHECK_INPUT(zp_out);
  CHECK_SAME_DEVICE(kv, q_out);
  CHECK_SAME_DEVICE(kv, scale_out);
  CHECK_SAME_DEVICE(kv, zp_out);
  const DeviceGuard guard(kv.device());
  TORCH_CHECK(kv.dim() == 2 && kv.stride(1) == 1, "kv must be 2D with contiguous rows");
  TORCH_CHECK(kv.scalar_type() == torch::kFloat32, "kv must be float32");
  TORCH_CHECK(kv.size(0) > 0 && kv.size(1) > 0, "kv must be non-empty");
  const int64_t rows = kv.size(0);
  const int c = (int)kv.size(1);
  const int64_t qcols = packed ? (c + 1) / 2 : c;
  TORCH_CHECK(q_out.scalar_type() == torch::kUInt8 && q_out.dim() == 2 && q_out.stride(1) == 1 &&
                  q_out.size(0) == rows && q_out.size(1) >= qcols,
              "q_out must be uint8 [rows, >= ", qcols, "] with contiguous rows");
  TORCH_CHECK(scale_out.scalar_type() == torch::kFloat32 && scale_out.numel() >= c,
              "scale_out must be float32 with >= C entries");
  TORCH_CHECK(zp_out.scalar_type() == torch::kFloat32 && zp_out.numel() >= c,
              "zp_out must be float32 with >= C entries");
  const size_t wsb = fdi4_quantize_rows_workspace_bytes(rows, c);
  auto ws = workspace(kv, wsb);
  check_rc(fdi4_quantize_rows(kv.data_ptr<float>(), rows, c, kv.stride(0),
                              q_out.data_ptr<uint8_t>(), q_out.stride(0), packed ? 1 : 0,
                              scale_out.data_ptr<float>(), zp_out.data_ptr<float>(),
                              ws.data_ptr(), ws.numel(), stream()),
           "quantize_rows");
}

// reference csrc/bindings.cpp:56-127
torch::Tensor flash_decode_int4(torch::Tensor query, torch::Tensor k_q, torch::Tensor k_scale,
                                torch::Tensor k_zp, torch::Tensor value,
                                torch::Tensor block_lens) {
  CHECK_INPUT(query);
  CHECK_INPUT(k_q);
  CHECK_INPUT(k_scale);
  CHECK_INPUT(k_zp);
  CHECK_INPUT(value);
  CHECK_INPUT(block_lens);
  CHECK_SAME_DEVICE(query, k_q);
  CHECK_SAME_DEVICE(query, k_scale);
  CHECK_SAME_DEVICE(query, k_zp);
  CHECK_SAME_DEVICE(query, value);
  CHECK_SAME_DEVICE(query, block_lens);
  const DeviceGuard guard(query.device());
  TORCH_CHECK(query.dim() == 3, "query must be 3D [batch, heads, head_dim]");
  TORCH_CHECK(k_q.dim() == 3, "k_q must be 3D [num_blocks, block_size, head_dim]");
  TORCH_CHECK(query.scalar_type() == torch::kFloat32, "query must be float32");
  TORCH_CHECK(k_q.scalar_type() == torch::kUInt8, "k_q must be uint8");
  TORCH_CHECK(k_scale.scalar_type() == torch::kFloat32, "k_scale must be float32");
  TORCH_CHECK(k_zp.scalar_type() == torch::kFloat32, "k_zp must be float32");
  TORCH_CHECK(value.scalar_type() == torch::kFloat32, "value must be float32");
  TORCH_CHECK(block_lens.scalar_type() == torch::kInt32, "block_lens must be int32");
  const int64_t hd = query.size(2);
  const int64_t nb = k_q.size(0);
  const int64_t bs = k_q.size(1);
  TORCH_CHECK(query.size(0) > 0 && query.size(1) > 0,
              "query must have at least one batch entry and one head");
  TORCH_CHECK(hd >= 1 && hd <= kMaxHeadDim, "head_dim must be in [1, ", kMaxHeadDim, "], got ",
              hd);
  TORCH_CHECK(k_q.size(2) == hd, "k_q last dim must equal head_dim");
  TORCH_CHECK(value.dim() == 3 && value.size(0) == nb && value.size(1) == bs &&
                  value.size(2) == hd,
              "value must be [num_blocks, block_size, head_dim] matching k_q");
  TORCH_CHECK(k_scale.dim() == 2 && k_scale.size(0) == nb && k_scale.size(1) == hd,
              "k_scale must be [num_blocks, head_dim]");
  TORCH_CHECK(k_zp.dim() == 2 && k_zp.size(0) == nb && k_zp.size(1) == hd,
              "k_zp must be [num_blocks, head_dim]");
  TORCH_CHECK(block_lens.dim() == 1 && block_lens.size(0) == nb,
              "block_lens must be [num_blocks]");
  TORCH_CHECK(nb <= INT32_MAX && bs <= INT32_MAX, "sizes must fit in int32");
  const int B = (int)query.size(0), H = (int)query.size(1), D = (int)hd;
  auto out = torch::empty({B, H, D}, query.options());
  const size_t wsb = fdi4_flash_decode_int4_workspace_bytes(B, H, D, (int)nb, (int)bs);
  auto ws = workspace(query, wsb);
  check_rc(fdi4_flash_decode_int4_ws(query.data_ptr<float>(), k_q.data_ptr<uint8_t>(),
                                     k_scale.data_ptr<float>(), k_zp.data_ptr<float>(),
                                     value.data_ptr<float>(), block_lens.data_ptr<int>(), B, H,
                                     D, (int)nb, (int)bs, out.data_ptr<float>(), ws.data_ptr(),
                                     ws.numel(), stream()),
           "flash_decode_int4");
  return out;
}

int dtype_code(const torch::Tensor& v) {
  if (v.scalar_type() == torch::kFloat32) return FDI4_V_F32;
  if (v.scalar_type() == torch::kFloat16) return FDI4_V_F16;
  if (v.scalar_type() == torch::kBFloat16) return FDI4_V_BF16;
  TORCH_CHECK(false, "v_pages must be float32, float16 or bfloat16");
  return -1;
}

// Element type code (fdi4_key_dtype) of a query / output tensor.
int elem_code(const torch::Tensor& t, const char* what) {
  if (t.scalar_type() == torch::kFloat32) return FDI4_K_F32;
  if (t.scalar_type() == torch::kFloat16) return FDI4_K_F16;
  if (t.scalar_type() == torch::kBFloat16) return FDI4_K_BF16;
  TORCH_CHECK(false, what, " must be float32, float16 or bfloat16");
  return -1;
}

// Build the C-ABI cache descriptor from tensors. k_pages [P, Hkv, R, D/2] u8,
// v_pages [P, Hkv, R, D] (may be undefined for the quantizer), k_scale/k_zp
// either [B, Hkv, G, D] (group mode) or [P, D] (scales attached to physical
// pages). Strides are taken from the tensors (0 for broadcast dimensions).
fdi4_paged_cache make_cache(const torch::Tensor& k_pages, const torch::Tensor* v_pages,
                            const torch::Tensor& k_scale, const torch::Tensor& k_zp,
                            const c10::optional<torch::Tensor>& page_table,
                            const c10::optional<torch::Tensor>& seq_lens,
                            const c10::optional<torch::Tensor>& page_lens, int64_t page_rows_ppg,
                            int64_t max_pages) {
  CHECK_DEV(k_pages);
  CHECK_DEV(k_scale);
  CHECK_DEV(k_zp);
  CHECK_SAME_DEVICE(k_pages, k_scale);
  CHECK_SAME_DEVICE(k_pages, k_zp);
  TORCH_CHECK(k_pages.scalar_type() == torch::kUInt8 && k_pages.dim() == 4 &&
                  k_pages.stride(3) == 1,
              "k_pages must be uint8 [pages, kv_heads, page_rows, head_dim/2]");
  const int64_t D = k_pages.size(3) * 2;
  TORCH_CHECK(D == 64 || D == 128 || D == 256, "head_dim must be 64, 128 or 256, got ", D);
  TORCH_CHECK(k_scale.scalar_type() == torch::kFloat32 && k_zp.scalar_type() == torch::kFloat32,
              "k_scale and k_zp must be float32");
  TORCH_CHECK(k_scale.sizes() == k_zp.sizes() && k_scale.strides() == k_zp.strides(),
              "k_scale and k_zp must have the same shape and strides");
  TORCH_CHECK(k_scale.size(-1) == D && k_scale.stride(-1) == 1,
              "k_scale last dim must be head_dim and contiguous");
  fdi4_paged_cache c = {};
  c.k_pages = k_pages.data_ptr<uint8_t>();
  c.k_page_stride = k_pages.stride(0);
  c.k_head_stride = k_pages.stride(1);
  c.k_row_stride = k_pages.stride(2);
  if (v_pages) {
    CHECK_DEV(*v_pages);
    CHECK_SAME_DEVICE(k_pages, *v_pages);
    TORCH_CHECK(v_pages->dim() == 4 && v_pages->size(0) == k_pages.size(0) &&
                    v_pages->size(1) == k_pages.size(1) && v_pages->size(2) == k_pages.size(2) &&
                    v_pages->size(3) == D && v_pages->stride(3) == 1,
                "v_pages must be [pages, kv_heads, page_rows, head_dim] matching k_pages");
    c.v_pages = v_pages->data_ptr();
    c.v_dtype = dtype_code(*v_pages);
    c.v_page_stride = v_pages->stride(0);
    c.v_head_stride = v_pages->stride(1);
    c.v_row_stride = v_pages->stride(2);
  }
  c.k_scale = k_scale.data_ptr<float>();
  c.k_zp = k_zp.data_ptr<float>();
  if (k_scale.dim() == 4) {
    c.s_batch_stride = k_scale.stride(0);
    c.s_head_stride = k_scale.stride(1);
    c.s_group_stride = k_scale.stride(2);
    c.pages_per_group = (int32_t)page_rows_ppg;
  } else {
    TORCH_CHECK(k_scale.dim() == 2 && k_scale.size(0) == k_pages.size(0),
                "k_scale must be [batch, kv_heads, groups, head_dim] or [pages, head_dim]");
    c.s_page_stride = k_scale.stride(0);
    c.pages_per_group = 1;
  }
  if (page_table && page_table->defined()) {
    CHECK_DEV(*page_table);
    CHECK_SAME_DEVICE(k_pages, *page_table);
    TORCH_CHECK(page_table->scalar_type() == torch::kInt32 && page_table->dim() == 2 &&
                    page_table->stride(1) == 1,
                "page_table must be int32 [batch, max_pages] with contiguous rows");
    c.page_table = page_table->data_ptr<int32_t>();
    c.pt_batch_stride = page_table->stride(0);
    TORCH_CHECK(page_table->size(1) >= max_pages, "page_table has fewer than max_pages columns");
  }
  if (seq_lens && seq_lens->defined()) {
    CHECK_DEV(*seq_lens);
    CHECK_SAME_DEVICE(k_pages, *seq_lens);
    TORCH_CHECK(seq_lens->scalar_type() == torch::kInt32 && seq_lens->dim() == 1 &&
                    seq_lens->stride(0) == 1,
                "seq_lens must be contiguous int32 [batch]");
    c.seq_lens = seq_lens->data_ptr<int32_t>();
  }
  if (page_lens && page_lens->defined()) {
    CHECK_DEV(*page_lens);
    CHECK_SAME_DEVICE(k_pages, *page_lens);
    TORCH_CHECK(page_lens->scalar_type() == torch::kInt32 && page_lens->dim() == 2 &&
                    page_lens->stride(1) == 1,
                "page_lens must be int32 [batch, max_pages] with contiguous rows");
    TORCH_CHECK(page_lens->size(1) >= max_pages, "page_lens has fewer than max_pages columns");
    c.page_lens = page_lens->data_ptr<int32_t>();
    c.pl_batch_stride = page_lens->stride(0);
  }
  c.num_kv_heads = (int32_t)k_pages.size(1);
  c.head_dim = (int32_t)D;
  c.page_rows = (int32_t)k_pages.size(2);
  c.max_pages = (int32_t)max_pages;
  c.num_pages = (int32_t)k_pages.size(0);
  return c;
}

void quantize_paged(torch::Tensor k, torch::Tensor seq_lens, torch::Tensor page_table,
                    torch::Tensor k_pages, torch::Tensor k_scale, torch::Tensor k_zp,
                    int64_t group_rows) {
  CHECK_DEV(k);
  TORCH_CHECK(k.scalar_type() == torch::kFloat32 && k.dim() == 4 && k.stride(3) == 1,
              "k must be float32 [batch, kv_heads, tokens, head_dim] with contiguous rows");
  TORCH_CHECK(k_scale.dim() == 4, "k_scale must be [batch, kv_heads, groups, head_dim]");
  TORCH_CHECK(seq_lens.dim() == 1 && seq_lens.size(0) == k.size(0) &&
                  page_table.size(0) == k.size(0),
              "seq_lens and page_table must have one row per sequence");
  TORCH_CHECK(page_table.size(1) * k_pages.size(2) >= k.size(2),
              "page_table has too few pages for the key length");
  TORCH_CHECK(k.size(1) == k_pages.size(1), "k and k_pages must have the same kv_heads");
  TORCH_CHECK(k.size(3) == k_pages.size(3) * 2, "k head_dim must match k_pages");
  TORCH_CHECK(group_rows % k_pages.size(2) == 0, "group_rows must be a multiple of page_rows");
  const int64_t G = (k.size(2) + group_rows - 1) / group_rows;
  TORCH_CHECK(k_scale.size(0) == k.size(0) && k_scale.size(1) == k.size(1) && k_scale.size(2) >= G,
              "k_scale must be [batch, kv_heads, >= ceil(tokens/group_rows), head_dim]");
  const int64_t max_pages = page_table.size(1);
  CHECK_SAME_DEVICE(k, k_pages);
  fdi4_paged_cache c = make_cache(k_pages, nullptr, k_scale, k_zp, page_table, seq_lens,
                                  c10::nullopt, group_rows / k_pages.size(2), max_pages);
  const DeviceGuard guard(k.device());
  check_rc(fdi4_quantize_paged(k.data_ptr<float>(), (int)k.size(0), (int)k.size(2), k.stride(0),
                               k.stride(1), k.stride(2), (int)group_rows, &c, stream()),
           "quantize_paged");
}

// One token per sequence appended at seq_lens[b] (see fdi4_append_paged);
// seq_lens is left for the caller to advance, or, with lens_next (int32,
// [>= batch], not seq_lens), the advanced lengths are written there
// (fdi4_append_paged_advance).
void append_paged_impl(torch::Tensor k_new, torch::Tensor v_new, torch::Tensor k_stage,
                       torch::Tensor k_pages, torch::Tensor v_pages, torch::Tensor k_scale,
                       torch::Tensor k_zp, torch::Tensor page_table, torch::Tensor seq_lens,
                       int64_t group_rows, c10::optional<torch::Tensor> lens_next) {
  CHECK_DEV(k_new);
  CHECK_DEV(v_new);
  CHECK_DEV(k_stage);
  TORCH_CHECK(k_new.scalar_type() == torch::kFloat32 && k_new.dim() == 3 && k_new.stride(2) == 1,
              "k_new must be float32 [batch, kv_heads, head_dim] with contiguous rows");
  TORCH_CHECK(v_new.scalar_type() == v_pages.scalar_type() && v_new.dim() == 3 &&
                  v_new.stride(2) == 1 && v_new.sizes() == k_new.sizes(),
              "v_new must be [batch, kv_heads, head_dim] in the cache's value dtype");
  TORCH_CHECK(k_stage.scalar_type() == torch::kFloat32 && k_stage.dim() == 4 &&
                  k_stage.stride(3) == 1 && k_stage.size(2) >= group_rows,
              "k_stage must be float32 [batch, kv_heads, >= group_rows, head_dim]");
  TORCH_CHECK(k_new.size(1) == k_pages.size(1) && k_new.size(2) == k_pages.size(3) * 2 &&
                  k_stage.size(1) == k_pages.size(1) && k_stage.size(3) == k_new.size(2),
              "k_new / k_stage heads and head_dim must match the cache");
  const int64_t B = k_new.size(0);
  TORCH_CHECK(k_stage.size(0) >= B && seq_lens.size(0) >= B && page_table.size(0) >= B &&
                  k_scale.dim() == 4 && k_scale.size(0) >= B,
              "k_stage, seq_lens, page_table and k_scale need a row per sequence");
  TORCH_CHECK(group_rows % k_pages.size(2) == 0, "group_rows must be a multiple of page_rows");
  const int64_t max_pages = page_table.size(1);
  TORCH_CHECK(k_scale.size(2) * (group_rows / k_pages.size(2)) >= max_pages,
              "k_scale has fewer than ceil(max_pages / pages_per_group) groups");
  CHECK_SAME_DEVICE(k_new, v_new);
  CHECK_SAME_DEVICE(k_new, k_stage);
  CHECK_SAME_DEVICE(k_new, k_pages);
  fdi4_paged_cache c = make_cache(k_pages, &v_pages, k_scale, k_zp, page_table, seq_lens,
                                  c10::nullopt, group_rows / k_pages.size(2), max_pages);
  const DeviceGuard guard(k_new.device());
  if (lens_next) {
    const torch::Tensor& next = *lens_next;
    CHECK_INPUT(next);
    CHECK_SAME_DEVICE(k_new, next);
    TORCH_CHECK(next.scalar_type() == torch::kInt32 && next.dim() == 1 && next.size(0) >= B,
                "lens_next must be int32 [>= batch]");
    check_rc(fdi4_append_paged_advance(k_new.data_ptr<float>(), k_new.stride(0),
                                       k_new.stride(1), v_new.data_ptr(), v_new.stride(0),
                                       v_new.stride(1), (int)B, k_stage.data_ptr<float>(),
                                       k_stage.stride(0), k_stage.stride(1), k_stage.stride(2),
                                       (int)group_rows, &c, lens_next->data_ptr<int32_t>(),
                                       stream()),
             "append_paged_advance");
    return;
  }
  check_rc(fdi4_append_paged(k_new.data_ptr<float>(), k_new.stride(0), k_new.stride(1),
                             v_new.data_ptr(), v_new.stride(0), v_new.stride(1), (int)B,
                             k_stage.data_ptr<float>(), k_stage.stride(0), k_stage.stride(1),
                             k_stage.stride(2), (int)group_rows, &c, stream()),
           "append_paged");
}

// One decode step of a serving loop on the device (see fdi4_decode_step):
// append k_new/v_new at each sequence's length, attend with query over the
// advanced lengths, advance seq_lens. counters (int32 [>= batch], zero) and
// lens_next (int32 [>= batch]) belong to the cache; returns [B, Hq, D] in the
// query's dtype.
torch::Tensor decode_step(torch::Tensor query, torch::Tensor k_new, torch::Tensor v_new,
                          torch::Tensor k_stage, torch::Tensor k_pages, torch::Tensor v_pages,
                          torch::Tensor k_scale, torch::Tensor k_zp, torch::Tensor page_table,
                          torch::Tensor seq_lens, int64_t group_rows, torch::Tensor counters,
                          torch::Tensor lens_next) {
  CHECK_DEV(query);
  CHECK_DEV(k_new);
  CHECK_DEV(v_new);
  CHECK_DEV(k_stage);
  const int qcode = elem_code(query, "query");
  TORCH_CHECK(query.dim() == 3 && query.stride(2) == 1,
              "query must be [batch, heads, head_dim] with contiguous rows");
  TORCH_CHECK(k_new.scalar_type() == torch::kFloat32 && k_new.dim() == 3 && k_new.stride(2) == 1,
              "k_new must be float32 [batch, kv_heads, head_dim] with contiguous rows");
  TORCH_CHECK(v_new.scalar_type() == v_pages.scalar_type() && v_new.dim() == 3 &&
                  v_new.stride(2) == 1 && v_new.sizes() == k_new.sizes(),
              "v_new must be [batch, kv_heads, head_dim] in the cache's value dtype");
  TORCH_CHECK(k_stage.scalar_type() == torch::kFloat32 && k_stage.dim() == 4 &&
                  k_stage.stride(3) == 1 && k_stage.size(2) >= group_rows,
              "k_stage must be float32 [batch, kv_heads, >= group_rows, head_dim]");
  TORCH_CHECK(k_new.size(1) == k_pages.size(1) && k_new.size(2) == k_pages.size(3) * 2 &&
                  k_stage.size(1) == k_pages.size(1) && k_stage.size(3) == k_new.size(2) &&
                  query.size(2) == k_new.size(2),
              "k_new / k_stage / query heads and head_dim must match the cache");
  const int64_t B = k_new.size(0);
  TORCH_CHECK(query.size(0) == B, "query and k_new must have the same batch");
  TORCH_CHECK(query.size(1) % k_pages.size(1) == 0,
              "query heads must be a multiple of kv_heads");
  TORCH_CHECK(k_stage.size(0) >= B && seq_lens.size(0) >= B && page_table.size(0) >= B &&
                  k_scale.dim() == 4 && k_scale.size(0) >= B,
              "k_stage, seq_lens, page_table and k_scale need a row per sequence");
  TORCH_CHECK(group_rows % k_pages.size(2) == 0, "group_rows must be a multiple of page_rows");
  const int64_t max_pages = page_table.size(1);
  TORCH_CHECK(k_scale.size(2) * (group_rows / k_pages.size(2)) >= max_pages,
              "k_scale has fewer than ceil(max_pages / pages_per_group) groups");
  for (const torch::Tensor* t : {&counters, &lens_next}) {
    CHECK_INPUT(*t);
    TORCH_CHECK(t->scalar_type() == torch::kInt32 && t->dim() == 1 && t->size(0) >= B,
                "counters and lens_next must be int32 [>= batch]");
  }
  CHECK_SAME_DEVICE(query, k_new);
  CHECK_SAME_DEVICE(query, v_new);
  CHECK_SAME_DEVICE(query, k_stage);
  CHECK_SAME_DEVICE(query, k_pages);
  CHECK_SAME_DEVICE(query, counters);
  CHECK_SAME_DEVICE(query, lens_next);
  fdi4_paged_cache c = make_cache(k_pages, &v_pages, k_scale, k_zp, page_table, seq_lens,
                                  c10::nullopt, group_rows / k_pages.size(2), max_pages);
  const DeviceGuard guard(query.device());
  const int Hq = (int)query.size(1), D = (int)query.size(2);
  auto out = torch::empty({B, Hq, D}, query.options());
  const int splits = fdi4_decode_num_splits((int)B, Hq, &c);
  auto ws = workspace(query, fdi4_decode_workspace_bytes((int)B, Hq, D, splits));
  check_rc(fdi4_decode_step(query.data_ptr(), qcode, (int)B, Hq, query.stride(0),
                            query.stride(1), k_new.data_ptr<float>(), k_new.stride(0),
                            k_new.stride(1), v_new.data_ptr(), v_new.stride(0), v_new.stride(1),
                            k_stage.data_ptr<float>(), k_stage.stride(0), k_stage.stride(1),
                            k_stage.stride(2), (int)group_rows, &c, out.data_ptr(), qcode,
                            out.stride(0), out.stride(1), counters.data_ptr<int32_t>(),
                            lens_next.data_ptr<int32_t>(), ws.data_ptr(), ws.numel(),
                            stream()),
           "decode_step");
  return out;
}

void append_paged(torch::Tensor k_new, torch::Tensor v_new, torch::Tensor k_stage,
                  torch::Tensor k_pages, torch::Tensor v_pages, torch::Tensor k_scale,
                  torch::Tensor k_zp, torch::Tensor page_table, torch::Tensor seq_lens,
                  int64_t group_rows) {
  append_paged_impl(k_new, v_new, k_stage, k_pages, v_pages, k_scale, k_zp, page_table,
                    seq_lens, group_rows, c10::nullopt);
}

void append_paged_advance(torch::Tensor k_new, torch::Tensor v_new, torch::Tensor k_stage,
                          torch::Tensor k_pages, torch::Tensor v_pages, torch::Tensor k_scale,
                          torch::Tensor k_zp, torch::Tensor page_table, torch::Tensor seq_lens,
                          int64_t group_rows, torch::Tensor lens_next) {
  append_paged_impl(k_new, v_new, k_stage, k_pages, v_pages, k_scale, k_zp, page_table,
                    seq_lens, group_rows, lens_next);
}

torch::Tensor decode_paged_impl(torch::Tensor query, torch::Tensor k_pages,
                                torch::Tensor v_pages, torch::Tensor k_scale, torch::Tensor k_zp,
                                c10::optional<torch::Tensor> page_table,
                                c10::optional<torch::Tensor> seq_lens,
                                c10::optional<torch::Tensor> page_lens, int64_t pages_per_group,
                                int64_t max_pages, int64_t num_splits,
                                c10::optional<torch::Tensor> lens_out) {
  CHECK_DEV(query);
  const int qcode = elem_code(query, "query");
  TORCH_CHECK(query.dim() == 3 && query.stride(2) == 1,
              "query must be [batch, heads, head_dim] with contiguous rows");
  TORCH_CHECK(query.size(2) == k_pages.size(3) * 2, "query head_dim must match the cache");
  CHECK_SAME_DEVICE(query, k_pages);
  fdi4_paged_cache c = make_cache(k_pages, &v_pages, k_scale, k_zp, page_table, seq_lens,
                                  page_lens, pages_per_group, max_pages);
  const DeviceGuard guard(query.device());
  const int B = (int)query.size(0), Hq = (int)query.size(1), D = (int)query.size(2);
  // Every row the kernel may index must exist: batch rows of the per-sequence
  // tensors, and one scale group per pages_per_group logical pages.
  if (k_scale.dim() == 4) {
    TORCH_CHECK(k_scale.size(0) >= B && k_scale.size(1) == k_pages.size(1),
                "k_scale must be [batch, kv_heads, groups, head_dim]");
    TORCH_CHECK(k_scale.size(2) * pages_per_group >= max_pages,
                "k_scale has fewer than ceil(max_pages / pages_per_group) groups");
  }
  if (page_table && page_table->defined())
    TORCH_CHECK(page_table->size(0) >= B, "page_table must have a row per sequence");
  if (seq_lens && seq_lens->defined())
    TORCH_CHECK(seq_lens->size(0) >= B, "seq_lens must have an entry per sequence");
  if (page_lens && page_lens->defined())
    TORCH_CHECK(page_lens->size(0) >= B, "page_lens must have a row per sequence");
  TORCH_CHECK(Hq % k_pages.size(1) == 0, "query heads must be a multiple of kv_heads");
  auto out = torch::empty({B, Hq, D}, query.options());
  const int splits = num_splits > 0 ? (int)num_splits : fdi4_decode_num_splits(B, Hq, &c);
  auto ws = workspace(query, fdi4_decode_workspace_bytes(B, Hq, D, splits));
  if (lens_out) {
    const torch::Tensor& back = *lens_out;
    CHECK_INPUT(back);
    CHECK_SAME_DEVICE(query, back);
    TORCH_CHECK(back.scalar_type() == torch::kInt32 && back.dim() == 1 && back.size(0) >= B,
                "lens_out must be int32 [>= batch]");
    TORCH_CHECK(seq_lens && seq_lens->defined(), "lens_out needs seq_lens");
    check_rc(fdi4_decode_paged_advance(query.data_ptr(), qcode, B, Hq, query.stride(0),
                                       query.stride(1), &c, out.data_ptr(), qcode,
                                       out.stride(0), out.stride(1), splits, ws.data_ptr(),
                                       ws.numel(), lens_out->data_ptr<int32_t>(), stream()),
             "decode_paged_advance");
    return out;
  }
  check_rc(fdi4_decode_paged_ex(query.data_ptr(), qcode, B, Hq, query.stride(0), query.stride(1),
                                &c, out.data_ptr(), qcode, out.stride(0), out.stride(1), splits,
                                ws.data_ptr(), ws.numel(), stream()),
           "decode_paged");
  return out;
}

torch::Tensor decode_paged(torch::Tensor query, torch::Tensor k_pages, torch::Tensor v_pages,
                           torch::Tensor k_scale, torch::Tensor k_zp,
                           c10::optional<torch::Tensor> page_table,
                           c10::optional<torch::Tensor> seq_lens,
                           c10::optional<torch::Tensor> page_lens, int64_t pages_per_group,
                           int64_t max_pages, int64_t num_splits) {
  return decode_paged_impl(query, k_pages, v_pages, k_scale, k_zp, page_table, seq_lens,
                           page_lens, pages_per_group, max_pages, num_splits, c10::nullopt);
}

// decode_paged that also copies the lengths it reads to lens_out (the
// second launch of a serving step; see fdi4_decode_paged_advance).
torch::Tensor decode_paged_advance(torch::Tensor query, torch::Tensor k_pages,
                                   torch::Tensor v_pages, torch::Tensor k_scale,
                                   torch::Tensor k_zp, c10::optional<torch::Tensor> page_table,
                                   torch::Tensor seq_lens, int64_t pages_per_group,
                                   int64_t max_pages, int64_t num_splits,
                                   torch::Tensor lens_out) {
  return decode_paged_impl(query, k_pages, v_pages, k_scale, k_zp, page_table, seq_lens,
                           c10::nullopt, pages_per_group, max_pages, num_splits, lens_out);
}

// Decode kernel alone into a caller-provided partials buffer (uint8 tensor of
// at least fdi4_decode_partials_bytes); see merge_splits.
void decode_paged_partials(torch::Tensor query, torch::Tensor k_pages, torch::Tensor v_pages,
                           torch::Tensor k_scale, torch::Tensor k_zp,
                           c10::optional<torch::Tensor> page_table,
                           c10::optional<torch::Tensor> seq_lens,
                           c10::optional<torch::Tensor> page_lens, int64_t pages_per_group,
                           int64_t max_pages, int64_t num_splits, torch::Tensor partials) {
  CHECK_DEV(query);
  CHECK_INPUT(partials);
  TORCH_CHECK(query.scalar_type() == torch::kFloat32 && query.dim() == 3 && query.stride(2) == 1,
              "query must be float32 [batch, heads, head_dim] with contiguous rows");
  TORCH_CHECK(query.size(2) == k_pages.size(3) * 2, "query head_dim must match the cache");
  TORCH_CHECK(num_splits >= 1, "num_splits must be >= 1");
  CHECK_SAME_DEVICE(query, k_pages);
  fdi4_paged_cache c = make_cache(k_pages, &v_pages, k_scale, k_zp, page_table, seq_lens,
                                  page_lens, pages_per_group, max_pages);
  const DeviceGuard guard(query.device());
  const int B = (int)query.size(0), Hq = (int)query.size(1), D = (int)query.size(2);
  if (k_scale.dim() == 4) {
    TORCH_CHECK(k_scale.size(0) >= B && k_scale.size(2) * pages_per_group >= max_pages,
                "k_scale too small for the batch / pages");
  }
  if (page_table && page_table->defined())
    TORCH_CHECK(page_table->size(0) >= B, "page_table must have a row per sequence");
  if (seq_lens && seq_lens->defined())
    TORCH_CHECK(seq_lens->size(0) >= B, "seq_lens must have an entry per sequence");
  if (page_lens && page_lens->defined())
    TORCH_CHECK(page_lens->size(0) >= B, "page_lens must have a row per sequence");
  TORCH_CHECK(Hq % k_pages.size(1) == 0, "query heads must be a multiple of kv_heads");
  CHECK_SAME_DEVICE(query, partials);
  const size_t need = fdi4_decode_partials_bytes(B, Hq, D, (int)num_splits);
  TORCH_CHECK(partials.scalar_type() == torch::kUInt8 && (size_t)partials.numel() >= need,
              "partials must be a uint8 buffer of at least ", need, " bytes");
  check_rc(fdi4_decode_paged_partials(query.data_ptr<float>(), B, Hq, query.stride(0),
                                      query.stride(1), &c, (int)num_splits, partials.data_ptr(),
                                      partials.numel(), stream()),
           "decode_paged_partials");
}

torch::Tensor merge_splits(torch::Tensor partials, int64_t batch, int64_t q_heads,
                           int64_t head_dim, int64_t num_splits) {
  CHECK_INPUT(partials);
  const size_t need =
      fdi4_decode_partials_bytes((int)batch, (int)q_heads, (int)head_dim, (int)num_splits);
  TORCH_CHECK(need > 0 && partials.scalar_type() == torch::kUInt8 &&
                  (size_t)partials.numel() >= need,
              "partials must be a uint8 buffer of at least ", need, " bytes");
  const DeviceGuard guard(partials.device());
  auto out = torch::empty({batch, q_heads, head_dim},
                          partials.options().dtype(torch::kFloat32));
  const size_t acc_bytes = (size_t)batch * q_heads * num_splits * head_dim * sizeof(float);
  const size_t ml_off = (acc_bytes + 255) / 256 * 256;
  const auto* base = reinterpret_cast<const char*>(partials.data_ptr());
  check_rc(fdi4_merge_splits(reinterpret_cast<const float*>(base),
                             reinterpret_cast<const double*>(base + ml_off), (int)batch,
                             (int)q_heads, (int)head_dim, (int)num_splits, out.data_ptr<float>(),
                             out.stride(0), out.stride(1), stream()),
           "merge_splits");
  return out;
}

int64_t decode_partials_bytes(int64_t batch, int64_t q_heads, int64_t head_dim,
                              int64_t num_splits) {
  return (int64_t)fdi4_decode_partials_bytes((int)batch, (int)q_heads, (int)head_dim,
                                             (int)num_splits);
}

int64_t decode_num_splits(int64_t batch, int64_t q_heads, int64_t kv_heads, int64_t head_dim,
                          int64_t max_pages, int64_t page_rows) {
  fdi4_paged_cache c = {};
  c.num_kv_heads = (int32_t)kv_heads;
  c.head_dim = (int32_t)head_dim;
  c.max_pages = (int32_t)max_pages;
  c.page_rows = (int32_t)page_rows;
  return fdi4_decode_num_splits((int)batch, (int)q_heads, &c);
}

torch::Tensor pack_int4(torch::Tensor q, int64_t out_cols) {
  CHECK_DEV(q);
  TORCH_CHECK(q.scalar_type() == torch::kUInt8 && q.dim() == 2 && q.stride(1) == 1,
              "q must be uint8 [rows, channels] with contiguous rows");
  const int64_t rows = q.size(0);
  const int c = (int)q.size(1);
  if (out_cols <= 0) out_cols = (c + 1) / 2;
  const DeviceGuard guard(q.device());
  auto out = torch::empty({rows, out_cols}, q.options());
  check_rc(fdi4_pack_int4(q.data_ptr<uint8_t>(), rows, c, q.stride(0), out.data_ptr<uint8_t>(),
                          out_cols, (int)out_cols, stream()),
           "pack_int4");
  return out;
}

// Dequantization of stored INT4 values q [rows, bytes] (one value per byte,
// or two nibbles per byte when packed) with scale / zp viewed as [rows,
// num_channels] through their strides (0 for a broadcast axis; the two must
// share strides): float32 [rows, num_channels] = q*s - zp*s.
torch::Tensor dequantize_int4(torch::Tensor q, torch::Tensor scale, torch::Tensor zp,
                              int64_t num_channels, bool packed) {
  CHECK_DEV(q);
  CHECK_DEV(scale);
  CHECK_DEV(zp);
  CHECK_SAME_DEVICE(q, scale);
  CHECK_SAME_DEVICE(q, zp);
  TORCH_CHECK(q.scalar_type() == torch::kUInt8 && q.dim() == 2 && q.stride(1) == 1,
              "q must be uint8 [rows, bytes] with contiguous rows");
  const int64_t rows = q.size(0);
  TORCH_CHECK(num_channels >= 1 && num_channels <= INT32_MAX, "num_channels must be >= 1");
  TORCH_CHECK(q.size(1) == (packed ? (num_channels + 1) / 2 : num_channels),
              "q has ", q.size(1), " bytes per row for ", num_channels,
              packed ? " packed channels" : " channels");
  TORCH_CHECK(scale.scalar_type() == torch::kFloat32 && zp.scalar_type() == torch::kFloat32,
              "scale and zp must be float32");
  TORCH_CHECK(scale.dim() == 2 && scale.size(0) == rows && scale.size(1) == num_channels &&
                  zp.sizes() == scale.sizes() && zp.strides() == scale.strides(),
              "scale and zp must be [rows, num_channels] views with the same strides");
  TORCH_CHECK(scale.stride(0) >= 0 && scale.stride(1) >= 0, "negative scale strides");
  const DeviceGuard guard(q.device());
  auto out = torch::empty({rows, num_channels}, q.options().dtype(torch::kFloat32));
  check_rc(fdi4_dequantize_int4(q.data_ptr<uint8_t>(), rows, (int)num_channels, q.stride(0),
                                packed ? 1 : 0, scale.data_ptr<float>(), zp.data_ptr<float>(),
                                scale.stride(0), scale.stride(1), out.data_ptr<float>(),
                                num_channels, stream()),
           "dequantize_int4");
  return out;
}

// INT4 quantize-dequantize of keys [batch, heads, seq, head_dim] into `out`
// (same dtype and shape; see fdi4_fake_quantize). rounding: 0 half-up, 1
// half-even; scale_op: 0 divide, 1 reciprocal.
void fake_quantize(torch::Tensor k, torch::Tensor out, int64_t block_size, int64_t rounding,
                   int64_t scale_op) {
  CHECK_DEV(k);
  CHECK_DEV(out);
  TORCH_CHECK(k.dim() == 4, "k must be 4D [batch, heads, seq, head_dim], got ", k.dim(), "D");
  const auto dt = k.scalar_type();
  int code;
  if (dt == torch::kFloat32) code = FDI4_K_F32;
  else if (dt == torch::kFloat16) code = FDI4_K_F16;
  else if (dt == torch::kBFloat16) code = FDI4_K_BF16;
  else TORCH_CHECK(false, "k must be float32, float16 or bfloat16, got ", dt);
  TORCH_CHECK(out.scalar_type() == dt && out.sizes() == k.sizes(),
              "out must have the dtype and shape of k");
  TORCH_CHECK(k.stride(3) == 1 && out.stride(3) == 1, "k and out need contiguous rows");
  TORCH_CHECK(block_size >= 1 && block_size <= INT32_MAX, "block_size must be >= 1");
  TORCH_CHECK(rounding == FDI4_ROUND_HALF_UP || rounding == FDI4_ROUND_HALF_EVEN,
              "rounding must be 0 (half-up) or 1 (half-even)");
  TORCH_CHECK(scale_op == FDI4_SCALE_DIVIDE || scale_op == FDI4_SCALE_RECIPROCAL,
              "scale_op must be 0 (divide) or 1 (reciprocal)");
  TORCH_CHECK(k.size(0) <= 65535 && k.size(1) <= 65535 && k.size(2) <= INT32_MAX,
              "k has too many sequences, heads or positions");
  CHECK_SAME_DEVICE(k, out);
  const DeviceGuard guard(k.device());
  check_rc(fdi4_fake_quantize(k.data_ptr(), code, (int)k.size(0), (int)k.size(1), (int)k.size(2),
                              (int)k.size(3), k.stride(0), k.stride(1), k.stride(2),
                              out.data_ptr(), out.stride(0), out.stride(1), out.stride(2),
                              (int)block_size, (int)rounding, (int)scale_op, stream()),
           "fake_quantize");
}

}  // namespace

PYBIND11_MODULE(TORCH_EXTENSION_NAME, m) {
  m.def("quantize_int4", &quantize_int4,
        "Per-channel asymmetric INT4 quantization, one group over all rows (HIP)");
  m.def("flash_decode_int4", &flash_decode_int4,
        "Fused online softmax + INT4 dequant attention over a shared page stream (HIP)");
  m.def("quantize_rows_into", &quantize_rows_into, "One-group INT4 quantization into views (HIP)");
  m.def("quantize_paged", &quantize_paged, "Grouped INT4 key quantization into packed pages (HIP)");
  m.def("append_paged", &append_paged,
        "Decode-time append: one token per sequence, open group re-quantized (HIP)");
  m.def("decode_paged", &decode_paged, "Split-K INT4 flash decoding over paged keys (HIP)");
  m.def("decode_step", &decode_step,
        "One serving step: append, decode over the advanced lengths, advance them (HIP)");
  m.def("append_paged_advance", &append_paged_advance,
        "Decode-time append that writes the advanced lengths to a second array (HIP)");
  m.def("decode_paged_advance", &decode_paged_advance,
        "decode_paged that copies the lengths it reads to a second array (HIP)");
  m.def("decode_paged_partials", &decode_paged_partials,
        "Decode kernel alone, writing split partials (HIP)");
  m.def("merge_splits", &merge_splits, "Log-sum-exp merge of split partials (HIP)");
  m.def("decode_partials_bytes", &decode_partials_bytes, "Bytes of the split partials");
  m.def("decode_num_splits", &decode_num_splits, "Split count chosen for a decode shape");
  m.def("pack_int4", &pack_int4, "Device nibble packing (HIP)");
  m.def("dequantize_int4", &dequantize_int4, "Dequantization of stored INT4 values (HIP)");
  m.def("fake_quantize", &fake_quantize, "INT4 quantize-dequantize of keys in blocks (HIP)");
  m.def("abi_version", &fdi4_abi_version, "C ABI version of the loaded libfdi4");
}
