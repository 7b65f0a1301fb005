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
  int row_blocks;            //   item -> (kv head, key piece, 16-row block of row_blocks, sequence)
  int pieces;                // decode: workgroups per row block, each over a contiguous piece of
                             //   the keys (1: one workgroup takes them all)
  float* part_o;             // pieces > 1: each piece's normalised O, [slot][16 rows][DP] fp32,
  float* part_lse;           //   and its log2 LSE [slot][16], slot = (row block item) * pieces + piece
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
// launch status. q_dtype DT_F16/DT_BF16, kv_dtype the same or fp8. With pieces > 1 (decode
// only) the grid is row-block items x pieces and a merge kernel follows.
hipError_t any_launch(const AnyArgs& a, int q_dtype, int kv_dtype, int64_t work_items, hipStream_t stream);

// The padded width of the kernel at head dim d (64, 128, 256 or 512).
inline int any_padded_dim(int d) { return d <= 64 ? 64 : d <= 128 ? 128 : d <= 256 ? 256 : 512; }

// Bytes of the piece partials for up to `slots` pieces at head dim d (each region 256-byte
// aligned): O then LSE.
constexpr size_t any_piece_o_bytes_c(int64_t slots, int dp) {
  return ((size_t)slots * 16 * dp * sizeof(float) + 255) & ~(size_t)255;
}
constexpr size_t any_piece_bytes_c(int64_t slots, int dp) {
  return any_piece_o_bytes_c(slots, dp) + (((size_t)slots * 16 * sizeof(float) + 255) & ~(size_t)255);
}
inline size_t any_piece_o_bytes(int64_t slots, int d) { return any_piece_o_bytes_c(slots, any_padded_dim(d)); }
inline size_t any_piece_bytes(int64_t slots, int d) { return any_piece_bytes_c(slots, any_padded_dim(d)); }

}  // namespace ma
