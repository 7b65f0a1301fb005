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
