// fp8 paged KV -> fp16 logical pages.
//
// Replaces gather_fp8_paged_kv (sglang_restomod/attention/v100/tilelang/_paged_adapter.py:527-564,
// kernel _kernels_fp8_bridge.py:20-70): for sequence b and logical page p below
// ceil(seq_lens[b] / page_size), physical page page_table[b, p] of the fp8 K and V caches
// ([pages, page_size, heads, head_dim] bytes) is decoded into page b * max_blocks + p of
// the fp16 outputs ([batch * max_blocks, page_size, heads, head_dim], contiguous). Other
// output pages are left untouched.
//
// Decoding is exact: e5m2 is the high byte of the fp16 with the same value (the byte
// shifted left by eight, every code including NaN payloads, as the reference does);
// e4m3fn goes through v_cvt_scalef32_pk_f16_fp8 with scale 1, which gives torch's cast
// for every finite code and a NaN for the two NaN codes.
//
// The attention kernels here read fp8 pools directly; this op serves callers that want
// an fp16 copy. Byte work, HBM-bound: 1 byte read and 2 bytes written per element; one
// workgroup per (sequence, logical page), each thread converting 16 bytes at a time.

#include "common.h"
#include "capi_internal.h"

namespace ma {

constexpr int kGatherThreads = 256;

struct Fp8GatherArgs {
  const unsigned char* k;
  const unsigned char* v;
  int64_t stride_page, stride_tok, stride_head;  // bytes
  const int32_t* page_table;
  int64_t table_stride;
  const int32_t* seq_lens;
  int max_blocks, page_size, heads, head_dim;
  int64_t num_pages;
  uint16_t* k_out;
  uint16_t* v_out;
};

// 8 fp8 bytes -> 8 fp16 values (cvt8_fp8: e5m2 by byte permute, e4m3fn by the hardware
// conversion)
template <int KV>
__device__ __forceinline__ u32x4 decode8(uint32_t w0, uint32_t w1) {
  return cvt8_fp8<KV, false>(w0, w1);
}

template <int KV>
__global__ __launch_bounds__(kGatherThreads) void fp8_gather_kernel(const Fp8GatherArgs a) {
  const int p = blockIdx.x;
  const int b = blockIdx.y;
  const int seq = cptr(a.seq_lens)[b];
  if (p >= (seq + a.page_size - 1) / a.page_size) return;
  const int64_t phys = cptr(a.page_table)[(int64_t)b * a.table_stride + p];
  if (phys < 0 || phys >= a.num_pages) return;
  const int64_t out_page = (int64_t)b * a.max_blocks + p;
  const int chunks_per_row = a.head_dim / 16;              // 16 fp8 bytes per chunk
  const int chunks = a.page_size * a.heads * chunks_per_row;
  const int64_t out_base = out_page * a.page_size * a.heads * a.head_dim;
  for (int c = threadIdx.x; c < 2 * chunks; c += kGatherThreads) {
    const bool is_v = c >= chunks;
    const int cc = is_v ? c - chunks : c;
    const int row = cc / chunks_per_row;  // (token, head)
    const int col = cc - row * chunks_per_row;
    const int tok = row / a.heads;
    const int head = row - tok * a.heads;
    const unsigned char MA_GLOBAL* src = gptr(is_v ? a.v : a.k) + phys * a.stride_page + tok * a.stride_tok +
                                         head * a.stride_head + col * 16;
    const u32x4 raw = *reinterpret_cast<const u32x4 MA_GLOBAL*>(src);
    uint16_t MA_GLOBAL* dst = gptr_mut(is_v ? a.v_out : a.k_out) + out_base + (int64_t)row * a.head_dim + col * 16;
    *reinterpret_cast<u32x4 MA_GLOBAL*>(dst) = decode8<KV>(raw[0], raw[1]);
    *reinterpret_cast<u32x4 MA_GLOBAL*>(dst + 8) = decode8<KV>(raw[2], raw[3]);
  }
}

}  // namespace ma

using namespace ma;

extern "C" int ma_gather_fp8_paged_kv(const void* k_cache, const void* v_cache, int64_t stride_page,
                                      int64_t stride_tok, int64_t stride_head, int kv_dtype, int64_t num_pages,
                                      const int32_t* page_table, int64_t table_stride, const int32_t* seq_lens,
                                      int batch, int max_blocks, int page_size, int num_kv_heads, int head_dim,
                                      void* k_out, void* v_out, void* stream) {
  if (kv_dtype != DT_E4M3 && kv_dtype != DT_E5M2)
    return set_error(MA_EINVAL, "gather_fp8_paged_kv expects an e4m3 or e5m2 cache (dtype %d)", kv_dtype);
  if (batch < 0 || max_blocks < 0 || page_size <= 0 || num_kv_heads <= 0 || num_pages < 0)
    return set_error(MA_EINVAL, "bad sizes");
  if (head_dim <= 0 || head_dim % 16) return set_error(MA_EINVAL, "head_dim %d must be a multiple of 16", head_dim);
  if ((int64_t)page_size * num_kv_heads * head_dim > (1 << 24)) return set_error(MA_EINVAL, "page too large");
  if (batch > 65535 || max_blocks > 0x7fffffff) return set_error(MA_EINVAL, "grid too large");
  if (batch == 0 || max_blocks == 0) return MA_OK;
  if (!k_cache || !v_cache || !page_table || !seq_lens || !k_out || !v_out)
    return set_error(MA_EINVAL, "null pointer argument");
  if ((reinterpret_cast<uintptr_t>(k_cache) | reinterpret_cast<uintptr_t>(v_cache) |
       reinterpret_cast<uintptr_t>(k_out) | reinterpret_cast<uintptr_t>(v_out) | (uintptr_t)stride_page |
       (uintptr_t)stride_tok | (uintptr_t)stride_head) & 15)
    return set_error(MA_EINVAL, "caches, outputs and cache strides must be 16-byte aligned");
  if (table_stride < max_blocks) return set_error(MA_EINVAL, "page table stride below max_blocks");
  Fp8GatherArgs a{};
  a.k = reinterpret_cast<const unsigned char*>(k_cache); a.v = reinterpret_cast<const unsigned char*>(v_cache);
  a.stride_page = stride_page; a.stride_tok = stride_tok; a.stride_head = stride_head;
  a.page_table = page_table; a.table_stride = table_stride; a.seq_lens = seq_lens;
  a.max_blocks = max_blocks; a.page_size = page_size; a.heads = num_kv_heads; a.head_dim = head_dim;
  a.num_pages = num_pages;
  a.k_out = reinterpret_cast<uint16_t*>(k_out); a.v_out = reinterpret_cast<uint16_t*>(v_out);
  const dim3 grid((unsigned)max_blocks, (unsigned)batch);
  if (kv_dtype == DT_E4M3)
    hipLaunchKernelGGL(fp8_gather_kernel<DT_E4M3>, grid, dim3(kGatherThreads), 0, (hipStream_t)stream, a);
  else
    hipLaunchKernelGGL(fp8_gather_kernel<DT_E5M2>, grid, dim3(kGatherThreads), 0, (hipStream_t)stream, a);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return set_error(MA_ELAUNCH, "fp8 gather launch failed: %s", hipGetErrorString(e));
  return MA_OK;
}
