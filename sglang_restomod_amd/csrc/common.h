// Shared device helpers for the gfx950 attention kernels.
//
// Everything here is written for CDNA4 (gfx950): wave64, MFMA 16x16x32 with
// 8 sixteen-bit operands per lane, packed fp8 -> 16-bit conversions.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "query_rows.h"

namespace ma {

typedef __attribute__((__vector_size__(8 * sizeof(__bf16)))) __bf16 bf16x8;
typedef __attribute__((__vector_size__(8 * sizeof(_Float16)))) _Float16 f16x8;
typedef __attribute__((__vector_size__(4 * sizeof(float)))) float f32x4;
typedef __attribute__((__vector_size__(2 * sizeof(_Float16)))) _Float16 f16x2;
typedef __attribute__((__vector_size__(2 * sizeof(__bf16)))) __bf16 bf16x2;
typedef __attribute__((__vector_size__(4 * sizeof(uint32_t)))) uint32_t u32x4;
typedef __attribute__((__vector_size__(2 * sizeof(uint32_t)))) uint32_t u32x2;
typedef __attribute__((__vector_size__(2 * sizeof(int)))) int i32x2;
typedef __attribute__((__vector_size__(4 * sizeof(short)))) short i16x4;

// Global-memory pointers. Pointers that reach a kernel inside a by-value argument
// struct are generic (flat) to the compiler; casting them to address space 1 makes
// it emit global_load/global_store, whose completion counts stay exact (flat accesses
// count against both the vector-memory and the LDS counters and make every wait
// conservative).
#define MA_GLOBAL __attribute__((address_space(1)))
template <typename T>
__device__ __forceinline__ const T MA_GLOBAL* gptr(const T* p) {
  return (const T MA_GLOBAL*)p;
}
template <typename T>
__device__ __forceinline__ T MA_GLOBAL* gptr_mut(T* p) {
  return (T MA_GLOBAL*)p;
}

// Read-only metadata indexed by a wave-uniform value: through the constant address
// space the compiler can use scalar loads, which complete on the LDS/scalar counter and
// never wait behind in-flight vector loads.
#define MA_CONST __attribute__((address_space(4)))
template <typename T>
__device__ __forceinline__ const T MA_CONST* cptr(const T* p) {
  return (const T MA_CONST*)p;
}

// Cache policies of the inline-assembly loads of decode and verify (appended to the
// mnemonic). K and V rows (whole rows per instruction) stream with the nontemporal hint: on random-slot gathers of 256-byte and 2 KiB rows, nt loads of whole
// rows reach 6.4-6.5 TB/s against 5.7-5.8 TB/s for default-policy loads, sequential or
// random alike. Slot lookups keep the default policy (each (sequence, kv head) segment
// re-reads its sequence's slots).
#ifndef MA_V_POLICY
#define MA_V_POLICY " nt"
#endif
#ifndef MA_K_POLICY
#define MA_K_POLICY " nt"
#endif
#ifndef MA_SLOT_POLICY
#define MA_SLOT_POLICY ""
#endif

// dtype codes shared with the C ABI (include/mi355x_attn.h)
enum DType : int { DT_F16 = 0, DT_BF16 = 1, DT_E4M3 = 2, DT_E5M2 = 3, DT_F32 = 4 };

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kEmptyLse = -1073741824.0f;  // -2^30: LSE of a split that saw no key

__device__ __forceinline__ int lane_id() { return threadIdx.x & 63; }

// ---------------------------------------------------------------------------
// MFMA wrappers. 16x16x32: A is 16(M) x 32(K), B is 32(K) x 16(N), C/D 16x16 f32.
// Lane l supplies row/col (l & 15) and 8 consecutive K values of group (l >> 4);
// the accumulator lane l holds column (l & 15), rows 4*(l >> 4) .. +3.
// ---------------------------------------------------------------------------
__device__ __forceinline__ f32x4 mfma16(const u32x4& a, const u32x4& b, f32x4 c, bool is_bf16) {
  if (is_bf16)
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a),
                                                   __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a),
                                                __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
}

template <bool BF16>
__device__ __forceinline__ f32x4 mfma16t(const u32x4& a, const u32x4& b, f32x4 c) {
  if constexpr (BF16)
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a),
                                                   __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a),
                                                  __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
}

// ---------------------------------------------------------------------------
// Online softmax helpers.
// ---------------------------------------------------------------------------
// A row's exponent base moves only when its max has grown by more than this (log2 of the
// largest p between two rescales of O). p stays exact to fp16's relative precision and
// the sums are fp32, so the result is the same up to rounding; O is rescaled rarely.
constexpr float kLazyRescale = 8.f;

// Max of three floats; the compiler makes it one v_max3_f32 (also straight from MFMA
// results, with no quieting v_max first). It must stay compiler code, not inline
// assembly: the hardware does not interlock a VALU read of an MFMA result, and the
// compiler inserts the wait states that read needs only for instructions it knows. An
// inline-assembly v_max3 placed right after the score MFMAs read partly accumulated
// scores (a row max from a stale accumulator, seen as run-to-run differences of the
// fp16 extend at head dim 256).
__device__ __forceinline__ float max3f(float x, float y, float z) {
  return __builtin_fmaxf(__builtin_fmaxf(x, y), z);
}

// Maximum of N scores by three-input maxima.
template <int N>
__device__ __forceinline__ float max_tree(const float* v) {
  if constexpr (N == 1) {
    return v[0];
  } else if constexpr (N == 2) {
    return max3f(v[0], v[1], -INFINITY);
  } else {
    constexpr int M = (N + 2) / 3;
    float w[M];
#pragma unroll
    for (int i = 0; i < M; ++i)
      w[i] = 3 * i + 2 < N ? max3f(v[3 * i], v[3 * i + 1], v[3 * i + 2])
                           : (3 * i + 1 < N ? max3f(v[3 * i], v[3 * i + 1], -INFINITY) : v[3 * i]);
    return max_tree<M>(w);
  }
}

// ---------------------------------------------------------------------------
// fp8 -> 16-bit, two values per instruction (exact: every e4m3fn / e5m2 value is
// representable in both fp16 and bf16). `w` holds four fp8 bytes; `hi` selects
// bytes 2..3 instead of 0..1. Result: low half = first byte, high half = second.
// ---------------------------------------------------------------------------
template <int KV, bool TO_BF16>
__device__ __forceinline__ uint32_t cvt2_fp8(uint32_t w, bool hi) {
  if constexpr (KV == DT_E4M3) {
    if constexpr (TO_BF16) {
      if (hi) return __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w, 1.0f, true));
      return __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w, 1.0f, false));
    } else {
      if (hi) return __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w, 1.0f, true));
      return __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w, 1.0f, false));
    }
  } else {
    if constexpr (TO_BF16) {
      if (hi) return __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_bf8(w, 1.0f, true));
      return __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_bf8(w, 1.0f, false));
    } else {
      // e5m2 is the high byte of the fp16 with the same value: one byte permute
      // (selector 0x0c gives a zero byte)
      return __builtin_amdgcn_perm(0u, w, hi ? 0x030c020cu : 0x010c000cu);
    }
  }
}

// 16 fp8 bytes (u32x4) -> 16 sixteen-bit values (two u32x4, element order kept).
template <int KV, bool TO_BF16>
__device__ __forceinline__ void cvt16_fp8(const u32x4& in, u32x4& lo, u32x4& hi) {
  lo[0] = cvt2_fp8<KV, TO_BF16>(in[0], false);
  lo[1] = cvt2_fp8<KV, TO_BF16>(in[0], true);
  lo[2] = cvt2_fp8<KV, TO_BF16>(in[1], false);
  lo[3] = cvt2_fp8<KV, TO_BF16>(in[1], true);
  hi[0] = cvt2_fp8<KV, TO_BF16>(in[2], false);
  hi[1] = cvt2_fp8<KV, TO_BF16>(in[2], true);
  hi[2] = cvt2_fp8<KV, TO_BF16>(in[3], false);
  hi[3] = cvt2_fp8<KV, TO_BF16>(in[3], true);
}

// 8 fp8 bytes (u32x2) -> 8 sixteen-bit values (u32x4).
template <int KV, bool TO_BF16>
__device__ __forceinline__ u32x4 cvt8_fp8(uint32_t w0, uint32_t w1) {
  u32x4 r;
  r[0] = cvt2_fp8<KV, TO_BF16>(w0, false);
  r[1] = cvt2_fp8<KV, TO_BF16>(w0, true);
  r[2] = cvt2_fp8<KV, TO_BF16>(w1, false);
  r[3] = cvt2_fp8<KV, TO_BF16>(w1, true);
  return r;
}

// ---------------------------------------------------------------------------
// Packing helpers.
// ---------------------------------------------------------------------------
// v_perm_b32 byte select: result byte i = byte sel[i] of {hi_word:lo_word} (bytes 0-3 = lo).
__device__ __forceinline__ uint32_t perm(uint32_t hi_word, uint32_t lo_word, uint32_t sel) {
  return __builtin_amdgcn_perm(hi_word, lo_word, sel);
}
// low halves of a and b -> (a.lo | b.lo << 16)
__device__ __forceinline__ uint32_t pack_lo(uint32_t a, uint32_t b) { return perm(b, a, 0x05040100u); }
// high halves of a and b -> (a.hi | b.hi << 16)
__device__ __forceinline__ uint32_t pack_hi(uint32_t a, uint32_t b) { return perm(b, a, 0x07060302u); }

// Two floats -> packed fp16 (round toward zero; exact for values already representable).
__device__ __forceinline__ uint32_t pack_f16(float a, float b) {
  return __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_pkrtz(a, b));
}

// Two floats -> packed bf16 by truncation, and the two truncation remainders.
__device__ __forceinline__ void split_bf16(float a, float b, uint32_t& hi, uint32_t& lo) {
  uint32_t ua = __builtin_bit_cast(uint32_t, a), ub = __builtin_bit_cast(uint32_t, b);
  hi = pack_hi(ua, ub);
  float ra = a - __builtin_bit_cast(float, ua & 0xffff0000u);
  float rb = b - __builtin_bit_cast(float, ub & 0xffff0000u);
  lo = pack_hi(__builtin_bit_cast(uint32_t, ra), __builtin_bit_cast(uint32_t, rb));
}

// Convert one 16-bit value (bits in low half) to float.
template <bool BF16>
__device__ __forceinline__ float h2f(uint32_t bits16) {
  if constexpr (BF16) return __builtin_bit_cast(float, bits16 << 16);
  else return (float)__builtin_bit_cast(_Float16, (uint16_t)bits16);
}

template <bool BF16>
__device__ __forceinline__ uint16_t f2h(float x) {
  if constexpr (BF16) {
    // round to nearest even; NaN stays NaN
    uint32_t u = __builtin_bit_cast(uint32_t, x);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40);
    u += 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
  } else {
    return __builtin_bit_cast(uint16_t, (_Float16)x);
  }
}

// Four consecutive output values of one row, scaled by s, at element `off` of out: fp32
// when out_f32 (the kernels' pre-cast result, for checking), else the query's 16-bit dtype.
template <bool BF16>
__device__ __forceinline__ void store_out4(void* out, int64_t off, f32x4 v, float s, bool out_f32) {
  if (out_f32) {
    *reinterpret_cast<f32x4 MA_GLOBAL*>(gptr_mut(reinterpret_cast<float*>(out)) + off) = v * s;
  } else {
    u32x2 w;
    w[0] = (uint32_t)f2h<BF16>(v[0] * s) | ((uint32_t)f2h<BF16>(v[1] * s) << 16);
    w[1] = (uint32_t)f2h<BF16>(v[2] * s) | ((uint32_t)f2h<BF16>(v[3] * s) << 16);
    *reinterpret_cast<u32x2 MA_GLOBAL*>(gptr_mut(reinterpret_cast<uint16_t*>(out)) + off) = w;
  }
}

// ---------------------------------------------------------------------------
// Cross-lane reductions within a wave.
// ---------------------------------------------------------------------------
__device__ __forceinline__ float shfl_xor_f(float v, int mask) {
  int src = lane_id() ^ mask;
  return __builtin_bit_cast(float, __builtin_amdgcn_ds_bpermute(src << 2, __builtin_bit_cast(int, v)));
}

__device__ __forceinline__ int shfl_i(int v, int src_lane) {
  return __builtin_amdgcn_ds_bpermute(src_lane << 2, v);
}

// ---------------------------------------------------------------------------
// Token -> KV row. row = table[row_of_seq * table_stride + (pos >> page_shift)] << page_shift
//                        | (pos & page_mask)
// With page_shift 0 and table = req_to_token this is the token-pool slot.
// ---------------------------------------------------------------------------
struct TokenTable {
  const int32_t* table;
  int64_t stride;
  int page_shift;
};

__device__ __forceinline__ int64_t kv_row(const TokenTable& t, int64_t seq_row, int pos) {
  const int32_t page = gptr(t.table)[seq_row * t.stride + (pos >> t.page_shift)];
  return ((int64_t)page << t.page_shift) | (int64_t)(pos & ((1 << t.page_shift) - 1));
}

}  // namespace ma
