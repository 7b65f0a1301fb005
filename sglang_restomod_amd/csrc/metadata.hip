// On-device metadata: token-table rows translated through a slot mapping.
//
// Replaces the sliding-window page-table build of the reference's backend
// (sglang_restomod/attention/v100/flash_attn_v100_backend.py:460-503: req_to_token rows
// gathered up to the batch's longest sequence, read from the host with .item(), and passed
// through the pool's translate_loc_from_full_to_swa). Here every row is translated up to
// its own length, read on the device, into a table of fixed width, so no host value is
// needed and a captured graph replays it:
//   out[b * out_stride + j] = mapping[table[r * table_stride + j]],  j < min(seq_lens[b], width)
//   r = row_index ? row_index[b] : b
// A slot outside [0, mapping_len) translates to 0, the pool's padding slot. Positions
// from seq_lens[b] on are not written (no kernel reads them).
//
// Integer gather work, HBM-bound: 4 bytes of table and 8 bytes of mapping read, 4 bytes
// written per position. One thread per position; a workgroup covers 1024 positions of
// one row and leaves at once when the row is shorter.
//
// Also the key rows of a multi-step speculative draft (draft_table_kernel): replaces the
// engine's per-step draft KV-index build that the reference's draft container reuses
// (sglang_restomod/attention/v100/draft_decode.py:172-208, the engine container's
// common_template) followed by the page-table conversion of every step
// (draft_decode_plan.py:42-78). Row r = b * topk + k lists the slots that branch k of
// request b attends over: the request's prefix, then the branch's draft tokens, which the
// engine places at req_to_token positions seq_lens[b] + k * num_steps onwards. One table
// serves every draft step: step i reads the first seq_lens[b] + i + 1 entries of a row.

#include "common.h"
#include "capi_internal.h"

namespace ma {

constexpr int kXlateThreads = 256;
constexpr int kXlatePerThread = 4;
constexpr int kXlateSpan = kXlateThreads * kXlatePerThread;  // positions per workgroup

struct TranslateArgs {
  const int32_t* table;
  int64_t table_stride;
  const int64_t* row_index;
  const int32_t* seq_lens;
  const int64_t* mapping;
  int64_t mapping_len;
  int32_t* out;
  int64_t out_stride;
  int width;
};

__global__ __launch_bounds__(kXlateThreads) void translate_slots_kernel(const TranslateArgs a) {
  const int b = blockIdx.y;
  const int n = min(cptr(a.seq_lens)[b], a.width);
  const int j0 = blockIdx.x * kXlateSpan;
  if (j0 >= n) return;
  const int64_t r = a.row_index ? cptr(a.row_index)[b] : (int64_t)b;
  const int32_t MA_GLOBAL* src = gptr(a.table) + r * a.table_stride;
  int32_t MA_GLOBAL* dst = gptr_mut(a.out) + (int64_t)b * a.out_stride;
  const int64_t MA_GLOBAL* map = gptr(a.mapping);
#pragma unroll
  for (int i = 0; i < kXlatePerThread; ++i) {
    const int j = j0 + i * kXlateThreads + (int)threadIdx.x;
    if (j < n) {
      const int32_t slot = src[j];
      dst[j] = (slot >= 0 && slot < a.mapping_len) ? (int32_t)map[slot] : 0;
    }
  }
}

struct DraftTableArgs {
  const int32_t* table;
  int64_t table_stride;
  int table_width;
  const int64_t* row_index;
  const int32_t* seq_lens;
  int topk, num_steps;
  const int64_t* mapping;  // null: slots as they are
  int64_t mapping_len;
  int32_t* out;
  int64_t out_stride;
  int width;
};

// Grid: (position blocks of kXlateSpan, batch * topk rows).
__global__ __launch_bounds__(kXlateThreads) void draft_table_kernel(const DraftTableArgs a) {
  const int r = blockIdx.y;
  const int b = r / a.topk;
  const int k = r - b * a.topk;
  const int seq = max(cptr(a.seq_lens)[b], 0);
  const int n = min(seq + a.num_steps, a.width);
  const int j0 = blockIdx.x * kXlateSpan;
  if (j0 >= n) return;
  const int64_t row = a.row_index ? cptr(a.row_index)[b] : (int64_t)b;
  const int32_t MA_GLOBAL* src = gptr(a.table) + row * a.table_stride;
  int32_t MA_GLOBAL* dst = gptr_mut(a.out) + (int64_t)r * a.out_stride;
  const int64_t MA_GLOBAL* map = gptr(a.mapping);
  const int gap = k * a.num_steps;  // draft positions of branch k follow those of branches 0..k-1
#pragma unroll
  for (int i = 0; i < kXlatePerThread; ++i) {
    const int j = j0 + i * kXlateThreads + (int)threadIdx.x;
    if (j < n) {
      const int p = j < seq ? j : j + gap;
      int32_t slot = p < a.table_width ? src[p] : 0;
      if (map) slot = (slot >= 0 && slot < a.mapping_len) ? (int32_t)map[slot] : 0;
      dst[j] = slot;
    }
  }
}

}  // namespace ma

using namespace ma;

extern "C" int ma_translate_slots(const int32_t* table, int64_t table_stride, const int64_t* row_index,
                                  const int32_t* seq_lens, int batch, const int64_t* mapping, int64_t mapping_len,
                                  int32_t* out, int64_t out_stride, int width, void* stream) {
  if (batch < 0 || width < 0 || mapping_len < 0) return set_error(MA_EINVAL, "sizes must be >= 0");
  if (batch > 65535) return set_error(MA_EINVAL, "batch %d exceeds 65535 rows", batch);
  if (batch == 0 || width == 0) return MA_OK;
  if (!table || !seq_lens || !mapping || !out) return set_error(MA_EINVAL, "null pointer argument");
  if (out_stride < width) return set_error(MA_EINVAL, "out_stride %lld is below the width %d",
                                            (long long)out_stride, width);
  TranslateArgs a{};
  a.table = table; a.table_stride = table_stride; a.row_index = row_index; a.seq_lens = seq_lens;
  a.mapping = mapping; a.mapping_len = mapping_len; a.out = out; a.out_stride = out_stride; a.width = width;
  const dim3 grid((unsigned)((width + kXlateSpan - 1) / kXlateSpan), (unsigned)batch);
  hipLaunchKernelGGL(translate_slots_kernel, grid, dim3(kXlateThreads), 0, (hipStream_t)stream, a);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return set_error(MA_ELAUNCH, "slot translation launch failed: %s", hipGetErrorString(e));
  return MA_OK;
}

extern "C" int ma_draft_table(const int32_t* table, int64_t table_stride, int table_width, const int64_t* row_index,
                              const int32_t* seq_lens, int batch, int topk, int num_steps, const int64_t* mapping,
                              int64_t mapping_len, int32_t* out, int64_t out_stride, int width, void* stream) {
  if (batch < 0 || width < 0 || table_width < 0 || mapping_len < 0) return set_error(MA_EINVAL, "sizes must be >= 0");
  if (topk <= 0 || num_steps <= 0) return set_error(MA_EINVAL, "topk %d and num_steps %d must be positive", topk, num_steps);
  if ((int64_t)batch * topk > 65535) return set_error(MA_EINVAL, "%d draft rows exceed 65535", batch * topk);
  if ((int64_t)topk * num_steps > (1 << 24)) return set_error(MA_EINVAL, "topk * num_steps too large");
  if (batch == 0 || width == 0) return MA_OK;
  if (!table || !seq_lens || !out) return set_error(MA_EINVAL, "null pointer argument");
  if (out_stride < width) return set_error(MA_EINVAL, "out_stride %lld is below the width %d", (long long)out_stride, width);
  if (table_stride < table_width) return set_error(MA_EINVAL, "table_stride is below the table width");
  DraftTableArgs a{};
  a.table = table; a.table_stride = table_stride; a.table_width = table_width; a.row_index = row_index;
  a.seq_lens = seq_lens; a.topk = topk; a.num_steps = num_steps; a.mapping = mapping; a.mapping_len = mapping_len;
  a.out = out; a.out_stride = out_stride; a.width = width;
  const dim3 grid((unsigned)((width + kXlateSpan - 1) / kXlateSpan), (unsigned)(batch * topk));
  hipLaunchKernelGGL(draft_table_kernel, grid, dim3(kXlateThreads), 0, (hipStream_t)stream, a);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return set_error(MA_ELAUNCH, "draft table launch failed: %s", hipGetErrorString(e));
  return MA_OK;
}
