// Paged attention for the head dims the tuned kernels do not take (every multiple of 16
// from 16 to 512 other than 64, 128 and 256): one kernel for decode, linear verify and
// extend rows. Shared by the decode/verify and extend entry points.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "common.h"

namespace ma {

constexpr int kAnyWaves = 4;        // waves per workgroup
constexpr int kAnyRows = 16;        // query rows per wave
constexpr int kAnyKeys = 16;        // keys per tile
constexpr int kAnyPlanRows = 128;   // rows of one work-list entry (the extend plan's smallest tile)
constexpr int kAnyMaxDim = 512;

struct AnyArgs {
  const void* q;
  int64_t q_stride_tok, q_stride_head;    // elements
  const void* k;
  const void* v;
  int64_t kv_stride_row, kv_stride_head;  // elements (fp8: bytes)
  TokenTable tt;
  const int64_t* row_index;  // request row of each sequence, or null (row b)
  const int32_t* seq_lens;
  const int32_t* qsl;        // [B+1] query start per sequence, or null (one row per sequence)
  const int32_t* prefix;     // [B] cached prefix per sequence, or null (seq_len - query count)
  int num_tokens;            // rows of q and out: query rows are clamped into [0, num_tokens)
  int batch, hq, hkv, group;
  int head_dim;              // D: the kernel's width is the next of 64, 128, 256, 512
  const int64_t* items;      // work list of 128-row tiles (extend), or null: workgroup
  int row_blocks;            //   item -> (kv head, 16-row block of row_blocks, sequence)
  int causal, window;
  float scale_log2;          // softmax_scale * k_scale * log2(e)
  float v_scale;
  void* out;
  int64_t out_stride_tok, out_stride_head;  // elements of the output dtype
  int out_f32;
};

// True for the head dims this path serves.
inline bool any_head_dim(int d) {
  return d >= 16 && d <= kAnyMaxDim && d % 16 == 0 && d != 64 && d != 128 && d != 256;
}

// Launch on `a` (validated by the caller, items already planned when set); returns the
// launch status. q_dtype DT_F16/DT_BF16, kv_dtype the same or fp8.
hipError_t any_launch(const AnyArgs& a, int q_dtype, int kv_dtype, int64_t work_items, hipStream_t stream);

}  // namespace ma
