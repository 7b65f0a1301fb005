// KV write into the token pool (set_kv_buffer), with fp8 quantisation on write.
//
// Replaces the pool write the reference's backend issues before every attention call
// (sglang_restomod/attention/v100/flash_attn_v100_backend.py:1174-1182, 1038-1046;
// draft_decode.py:132-139), with the semantics of SGLang's token pool: row t of the new
// K (and V) lands at pool slot loc[t]; when the cache dtype differs from the source dtype
// the source is first divided by the per-tensor scale in the source dtype (fp32 quotient,
// rounded to nearest even in bf16/fp16) and then cast: round to nearest even onto the
// fp8 grid, overflow past the largest finite value becoming NaN (e4m3fn, which has no
// infinity) or infinity (e5m2). The division stays an IEEE fp32 division: the stored
// byte depends on its exact rounding.
//
// Same source and cache dtype: a plain copy. HBM-bound: one thread per 16 source bytes,
// 16-byte loads and 16- or 8-byte stores per thread; each (token, head) row of K or V is
// read once and written once.

#include "common.h"
#include "capi_internal.h"

namespace ma {

struct KvWriteArgs {
  const void* k;
  const void* v;
  int64_t src_stride_tok, src_stride_head;  // elements
  const int64_t* loc;
  int64_t num_tokens;
  int hkv;
  int chunks;       // 16-byte source chunks per row (head_dim / 8)
  int chunk_shift;  // log2(chunks) when chunks is a power of two, else -1
  int per_block;    // whole rows per 256-thread block
  void* k_cache;
  void* v_cache;
  int64_t cache_stride_row, cache_stride_head;  // elements of the cache dtype (bytes for fp8)
  int64_t num_slots;
  float k_div, v_div;  // divisors (1 when no scale is applied)
  float k_rcp, v_rcp;  // their reciprocals, rounded to fp32
  int apply_scale;
};

// Two floats -> two fp8 codes in byte pair `hi` of `old` (v_cvt_pk_fp8_f32 / _bf8_f32:
// round to nearest even; past the largest finite value e4m3fn gives NaN, e5m2 infinity,
// which is the cast's convention, checked over every 16-bit input by the tests).
template <int KV>
__device__ __forceinline__ uint32_t cvt_pk_fp8(float a, float b, uint32_t old, bool hi) {
  if constexpr (KV == DT_E4M3) {
    if (hi) return (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(a, b, (int)old, true);
    return (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(a, b, (int)old, false);
  } else {
    if (hi) return (uint32_t)__builtin_amdgcn_cvt_pk_bf8_f32(a, b, (int)old, true);
    return (uint32_t)__builtin_amdgcn_cvt_pk_bf8_f32(a, b, (int)old, false);
  }
}

template <int SRC>
__device__ __forceinline__ float load16(uint32_t word, int hi) {
  const uint32_t bits = hi ? (word >> 16) : (word & 0xffffu);
  return h2f<SRC == DT_BF16>(bits);
}

// float -> 16-bit bits, round to nearest even (hardware conversions)
template <int SRC>
__device__ __forceinline__ uint32_t store16(float x) {
  if constexpr (SRC == DT_BF16) return __builtin_bit_cast(uint16_t, (__bf16)x);
  else return __builtin_bit_cast(uint16_t, (_Float16)x);
}

// x / div in fp32, then rounded to the source dtype, exactly as the IEEE division and the
// cast give it. q = x * rcp (rcp = 1 / div rounded to fp32) is within 3 fp32 ulps of the
// IEEE quotient (two roundings of relative size 2^-24 each, against the quotient's own
// half ulp), so both round to the same 16-bit value unless a 16-bit rounding boundary
// lies within 3 ulps of q; then (rarely) the division is done. The boundaries: bf16 rounds
// at the low 16 bits of the fp32 pattern (boundary 0x8000), fp16 at the low 13 bits
// (0x1000) in its normal range; below fp16's smallest normal the division is always done.
template <int SRC>
__device__ __forceinline__ float div_to_src(float x, float div, float rcp) {
  const float q = x * rcp;
  const uint32_t b = __builtin_bit_cast(uint32_t, q);
  bool near;
  if constexpr (SRC == DT_BF16) {
    const int low = (int)(b & 0xffffu) - 0x8000;
    near = low >= -3 && low <= 3;
  } else {
    const int low = (int)(b & 0x1fffu) - 0x1000;
    near = (low >= -3 && low <= 3) || (b & 0x7f800000u) < (113u << 23);
  }
  float exact = q;
  if (__builtin_expect(near, 0)) exact = x / div;  // lanes near a boundary only
  return h2f<SRC == DT_BF16>(store16<SRC>(exact));
}

// One 16-byte chunk of 8 source values -> cache values.
template <int SRC, int DST>
__device__ __forceinline__ void convert_chunk(const u32x4 in, float div, float rcp, bool apply, u32x4& out16,
                                              u32x2& out8) {
  if constexpr (SRC == DST) {
    out16 = in;  // same dtype: a copy (no scale is applied, as in the pool)
    return;
  }
  float x[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) x[i] = load16<SRC>(in[i >> 1], i & 1);
  if (apply) {
    // divide in fp32 and round to the source dtype, as the source-dtype division does
#pragma unroll
    for (int i = 0; i < 8; ++i) x[i] = div_to_src<SRC>(x[i], div, rcp);
  }
  if constexpr (DST == DT_E4M3 || DST == DT_E5M2) {
#pragma unroll
    for (int w = 0; w < 2; ++w) {
      const uint32_t lo = cvt_pk_fp8<DST>(x[4 * w], x[4 * w + 1], 0u, false);
      out8[w] = cvt_pk_fp8<DST>(x[4 * w + 2], x[4 * w + 3], lo, true);
    }
  } else {
#pragma unroll
    for (int w = 0; w < 4; ++w) out16[w] = store16<DST>(x[2 * w]) | (store16<DST>(x[2 * w + 1]) << 16);
  }
}

// Grid: x = blocks of 256 / (head_dim / 8) tokens (threads past whole rows idle), y = kv
// head, z = K (0) or V (1).
template <int SRC, int DST>
__global__ __launch_bounds__(256) void kv_write_kernel(const KvWriteArgs args) {
  const KvWriteArgs a = args;
  constexpr bool kFp8 = (DST == DT_E4M3 || DST == DT_E5M2);
  const int which = blockIdx.z;
  const int h = blockIdx.y;
  const int per_block = a.per_block;
  int row, part;
  if (a.chunk_shift >= 0) {  // the common head dims: shifts, not a division
    row = (int)threadIdx.x >> a.chunk_shift;
    part = (int)threadIdx.x & (a.chunks - 1);
  } else {
    row = (int)threadIdx.x / a.chunks;
    part = (int)threadIdx.x - row * a.chunks;
  }
  if (row >= per_block) return;
  const int64_t t = (int64_t)blockIdx.x * per_block + row;
  if (t >= a.num_tokens) return;
  const int64_t slot = gptr(a.loc)[t];
  if (slot < 0 || slot >= a.num_slots) return;  // not a slot of this pool: nothing is written
  const uint16_t MA_GLOBAL* src = gptr(reinterpret_cast<const uint16_t*>(which ? a.v : a.k)) +
                                  t * a.src_stride_tok + (int64_t)h * a.src_stride_head + part * 8;
  const u32x4 in = *reinterpret_cast<const u32x4 MA_GLOBAL*>(src);
  u32x4 o16;
  u32x2 o8;
  convert_chunk<SRC, DST>(in, which ? a.v_div : a.k_div, which ? a.v_rcp : a.k_rcp, a.apply_scale != 0, o16, o8);
  const int64_t off = slot * a.cache_stride_row + (int64_t)h * a.cache_stride_head + part * 8;
  if constexpr (kFp8) {
    unsigned char MA_GLOBAL* dst = gptr_mut(reinterpret_cast<unsigned char*>(which ? a.v_cache : a.k_cache)) + off;
    *reinterpret_cast<u32x2 MA_GLOBAL*>(dst) = o8;
  } else {
    uint16_t MA_GLOBAL* dst = gptr_mut(reinterpret_cast<uint16_t*>(which ? a.v_cache : a.k_cache)) + off;
    *reinterpret_cast<u32x4 MA_GLOBAL*>(dst) = o16;
  }
}

template <int SRC>
static hipError_t launch_kv_write(int dst, dim3 grid, hipStream_t st, const KvWriteArgs& a) {
  switch (dst) {
    case DT_F16: hipLaunchKernelGGL((kv_write_kernel<SRC, DT_F16>), grid, dim3(256), 0, st, a); break;
    case DT_BF16: hipLaunchKernelGGL((kv_write_kernel<SRC, DT_BF16>), grid, dim3(256), 0, st, a); break;
    case DT_E4M3: hipLaunchKernelGGL((kv_write_kernel<SRC, DT_E4M3>), grid, dim3(256), 0, st, a); break;
    default: hipLaunchKernelGGL((kv_write_kernel<SRC, DT_E5M2>), grid, dim3(256), 0, st, a); break;
  }
  return hipGetLastError();
}

}  // namespace ma

using namespace ma;

extern "C" int ma_set_kv_buffer(const void* k, const void* v, int64_t src_stride_tok, int64_t src_stride_head,
                                int src_dtype, const int64_t* loc, int64_t num_tokens, int num_kv_heads,
                                int head_dim, void* k_cache, void* v_cache, int64_t cache_stride_row,
                                int64_t cache_stride_head, int cache_dtype, int64_t num_slots, float k_scale,
                                float v_scale, int apply_scale, void* stream) {
  if (src_dtype != DT_F16 && src_dtype != DT_BF16) return set_error(MA_EINVAL, "source dtype %d must be f16 or bf16", src_dtype);
  if (cache_dtype < DT_F16 || cache_dtype > DT_E5M2) return set_error(MA_EINVAL, "cache dtype %d unknown", cache_dtype);
  if (num_tokens < 0 || num_kv_heads <= 0 || num_slots < 0) return set_error(MA_EINVAL, "bad sizes");
  if (head_dim < 8 || head_dim > 2048 || (head_dim % 8))
    return set_error(MA_EUNSUPPORTED, "head_dim %d must be a multiple of 8 in 8..2048", head_dim);
  if (apply_scale && !(k_scale > 0.f && v_scale > 0.f)) return set_error(MA_EINVAL, "scales must be positive");
  if (num_tokens == 0) return MA_OK;
  if (!k || !v || !loc || !k_cache || !v_cache) return set_error(MA_EINVAL, "null pointer argument");
  const int elt = cache_dtype >= DT_E4M3 ? 1 : 2;
  const int store_align = cache_dtype >= DT_E4M3 ? 8 : 16;
  if ((reinterpret_cast<uintptr_t>(k) | reinterpret_cast<uintptr_t>(v)) & 15)
    return set_error(MA_EINVAL, "k and v must be 16-byte aligned");
  if ((reinterpret_cast<uintptr_t>(k_cache) | reinterpret_cast<uintptr_t>(v_cache)) & (store_align - 1))
    return set_error(MA_EINVAL, "caches must be %d-byte aligned", store_align);
  if (((src_stride_tok * 2) & 15) || ((src_stride_head * 2) & 15))
    return set_error(MA_EINVAL, "source strides must keep rows 16-byte aligned");
  if (((cache_stride_row * elt) & (store_align - 1)) || ((cache_stride_head * elt) & (store_align - 1)))
    return set_error(MA_EINVAL, "cache strides must keep rows %d-byte aligned", store_align);
  KvWriteArgs a{};
  a.k = k; a.v = v; a.src_stride_tok = src_stride_tok; a.src_stride_head = src_stride_head;
  a.loc = loc; a.num_tokens = num_tokens; a.hkv = num_kv_heads; a.chunks = head_dim / 8;
  a.k_cache = k_cache; a.v_cache = v_cache; a.cache_stride_row = cache_stride_row;
  a.cache_stride_head = cache_stride_head; a.num_slots = num_slots;
  a.apply_scale = apply_scale ? 1 : 0;
  a.k_div = apply_scale ? k_scale : 1.f;
  a.v_div = apply_scale ? v_scale : 1.f;
  a.k_rcp = 1.f / a.k_div;  // IEEE fp32 on the host
  a.v_rcp = 1.f / a.v_div;
  const int64_t per_block = 256 / a.chunks;  // tokens per block (head_dim <= 2048: at least 1)
  a.per_block = (int)per_block;
  a.chunk_shift = (a.chunks & (a.chunks - 1)) ? -1 : __builtin_ctz((unsigned)a.chunks);
  const int64_t blocks = (num_tokens + per_block - 1) / per_block;
  if (blocks > 0x7fffffff || num_kv_heads > 65535) return set_error(MA_EINVAL, "too many tokens or heads");
  const dim3 grid((unsigned)blocks, (unsigned)num_kv_heads, 2);
  hipError_t e = (src_dtype == DT_BF16) ? launch_kv_write<DT_BF16>(cache_dtype, grid, (hipStream_t)stream, a)
                                        : launch_kv_write<DT_F16>(cache_dtype, grid, (hipStream_t)stream, a);
  if (e != hipSuccess) return set_error(MA_ELAUNCH, "kv write launch failed: %s", hipGetErrorString(e));
  return MA_OK;
}
