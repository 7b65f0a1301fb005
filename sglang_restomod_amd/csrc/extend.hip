// Prefix-aware paged extend (chunked prefill) attention for gfx950.
//
// Replaces the reference's paged extend kernel
// (sglang_restomod/attention/v100/tilelang/_kernels_paged.py:55-393, launched from
// _paged_adapter.py:567-759): query token i of sequence b sees key j when
//   j < seq_lens[b]  and (causal: j <= prefix[b] + i)  and (window W >= 0: j >= prefix[b] + i - W).
//
// Decomposition: one workgroup = 4 waves = 128 query rows of ONE kv head, where row
// r of a sequence is (query token r / G, GQA head r % G). All G heads that share a
// kv head therefore share each K/V tile staged in LDS (GQA read once per tile).
// Row tiles are launched heaviest-first (the last tokens of a causal sequence see
// the most keys).
//
// Per 64-key tile, per wave (32 rows = two 16-row blocks), MFMA 16x16x32:
//   S^T[key, row] = K[key, :] . Q[row, :]   A = K from LDS (row-major, padded rows),
//                                           B = Q^T held in registers for the whole kernel.
//   O^T[d, row] += V^T[d, key] P^T[key, row] A = V^T from LDS (head-dim rows, keys in the
//                                           order the S^T accumulator holds them), B = P^T
//                                           straight from the S^T accumulators (fp16).
// K/V rows of tile n+1 are gathered from HBM into registers while tile n computes.
// bf16/fp16 K stays in the query dtype (exact products); V is converted to fp16 when
// staged (exact for |v| < 65504) and P is fp16, fp32 accumulate, fp32 softmax state.

#include "common.h"
#include "capi_internal.h"

namespace ma {

constexpr int kXBM = 128;              // query rows per workgroup
constexpr int kXBN = 64;               // keys per tile
constexpr int kXD = 128;               // head dim
constexpr int kKRow = kXD * 2 + 16;    // bytes per K row in LDS (padded)
constexpr int kVRow = kXBN * 2 + 16;   // bytes per V^T row in LDS (padded)

struct ExtendArgs {
  const void* q;
  int64_t q_stride_tok, q_stride_head;
  const void* k;
  const void* v;
  int64_t kv_stride_row, kv_stride_head;
  TokenTable tt;
  const int64_t* row_index;
  const int32_t* seq_lens;
  const int32_t* qsl;
  const int32_t* prefix;
  int batch, hq, hkv, group;
  int row_tiles;      // row tiles per (sequence, kv head) in the grid
  int causal, window;
  float scale_log2;
  float v_scale;
  void* out;
  int64_t out_stride_tok, out_stride_head;
};

// Column of the V^T tile that holds tile-local key `key` (0..63): within each 32-key
// step, keys 4j..4j+3 -> columns 8j..8j+3 and keys 16+4j..16+4j+3 -> columns 8j+4..8j+7,
// the order in which the S^T accumulators of lane group j hold them.
__device__ __forceinline__ int vt_col(int key) {
  const int step = key >> 5, k = key & 31;
  const int blk = k >> 4, jj = (k >> 2) & 3, i = k & 3;
  return step * 32 + jj * 8 + blk * 4 + i;
}

template <bool QBF16, int KV>
__global__ __launch_bounds__(256) void extend_kernel(const ExtendArgs a) {
  constexpr bool kFp8 = (KV == DT_E4M3 || KV == DT_E5M2);
  __shared__ __attribute__((aligned(16))) unsigned char ks[kXBN * kKRow];
  __shared__ __attribute__((aligned(16))) unsigned char vs[kXD * kVRow];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int c = lane & 15;
  const int j = lane >> 4;

  const int rt = a.row_tiles - 1 - (int)blockIdx.x;  // heaviest row tiles first
  const int h = blockIdx.y;
  const int b = blockIdx.z;
  const int tok0 = a.qsl[b];
  const int ntok = a.qsl[b + 1] - tok0;
  const int r0 = rt * kXBM;
  if (r0 >= ntok * a.group) return;
  const int seq = a.seq_lens[b];
  const int prefix = a.prefix ? a.prefix[b] : seq - ntok;
  const int64_t seq_row = a.row_index ? a.row_index[b] : (int64_t)b;

  // ---- rows of this lane (one per 16-row block of the wave) ----
  int lo_r[2], hi_r[2];
  bool real[2];
  u32x4 qv[2][4];
  const uint16_t* qbase = reinterpret_cast<const uint16_t*>(a.q);
#pragma unroll
  for (int rb = 0; rb < 2; ++rb) {
    const int r = r0 + wave * 32 + rb * 16 + c;
    const int t = r / a.group;
    const int g = r - t * a.group;
    real[rb] = t < ntok;
    const int qpos = prefix + t;
    lo_r[rb] = (real[rb] && a.window >= 0) ? max(0, qpos - a.window) : 0;
    hi_r[rb] = real[rb] ? (a.causal ? min(seq, qpos + 1) : seq) : 0;
    const uint16_t* qp = qbase + (int64_t)(tok0 + t) * a.q_stride_tok + (int64_t)(h * a.group + g) * a.q_stride_head + j * 32;
#pragma unroll
    for (int kk = 0; kk < 4; ++kk)
      qv[rb][kk] = real[rb] ? *reinterpret_cast<const u32x4*>(qp + kk * 8) : u32x4{0, 0, 0, 0};
  }
  // key range of the whole workgroup and the window in which no row needs masking
  const int t_first = r0 / a.group;
  const int t_last = min(ntok - 1, (r0 + kXBM - 1) / a.group);
  const int key_lo = a.window >= 0 ? max(0, prefix + t_first - a.window) : 0;
  const int key_hi = a.causal ? min(seq, prefix + t_last + 1) : seq;
  const int full_lo = a.window >= 0 ? max(0, prefix + t_last - a.window) : 0;
  const int full_hi = a.causal ? min(seq, prefix + t_first + 1) : seq;

  float m_run[2] = {-INFINITY, -INFINITY};
  float l_run[2] = {0.f, 0.f};
  f32x4 o[2][8];
#pragma unroll
  for (int rb = 0; rb < 2; ++rb)
#pragma unroll
    for (int db = 0; db < 8; ++db) o[rb][db] = f32x4{0.f, 0.f, 0.f, 0.f};

  const unsigned char* kbase = reinterpret_cast<const unsigned char*>(a.k);
  const unsigned char* vbase = reinterpret_cast<const unsigned char*>(a.v);
  constexpr int kElt = kFp8 ? 1 : 2;
  const int64_t row_bytes = a.kv_stride_row * kElt;
  const int64_t head_off = (int64_t)h * a.kv_stride_head * kElt;

  // ---- global -> register staging of one tile ----
  // 16-bit: K: thread loads chunk (tid & 15) of keys (tid >> 4) + 16 i;
  //         V: thread loads chunk (tid & 15) of keys 4 (tid >> 4) + i.
  // fp8:    K: chunk (tid & 7) of keys (tid >> 3) + 32 i (i < 2);
  //         V: chunk (tid & 7) of keys 2 (tid >> 3) + i (i < 2).
  u32x4 kreg[4], vreg[4];
  auto load_tile = [&](int base) {
    if constexpr (kFp8) {
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        const int key = (tid >> 3) + 32 * i;
        const int pos = base + key;
        if (pos < key_hi) {
          const int64_t row = kv_row(a.tt, seq_row, pos);
          kreg[i] = *reinterpret_cast<const u32x4*>(kbase + row * row_bytes + head_off + (tid & 7) * 16);
        } else {
          kreg[i] = u32x4{0, 0, 0, 0};
        }
        const int vkey = 2 * (tid >> 3) + i;
        const int vpos = base + vkey;
        if (vpos < key_hi) {
          const int64_t row = kv_row(a.tt, seq_row, vpos);
          vreg[i] = *reinterpret_cast<const u32x4*>(vbase + row * row_bytes + head_off + (tid & 7) * 16);
        } else {
          vreg[i] = u32x4{0, 0, 0, 0};
        }
      }
    } else {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int key = (tid >> 4) + 16 * i;
        const int pos = base + key;
        if (pos < key_hi) {
          const int64_t row = kv_row(a.tt, seq_row, pos);
          kreg[i] = *reinterpret_cast<const u32x4*>(kbase + row * row_bytes + head_off + (tid & 15) * 16);
        } else {
          kreg[i] = u32x4{0, 0, 0, 0};
        }
        const int vkey = 4 * (tid >> 4) + i;
        const int vpos = base + vkey;
        if (vpos < key_hi) {
          const int64_t row = kv_row(a.tt, seq_row, vpos);
          vreg[i] = *reinterpret_cast<const u32x4*>(vbase + row * row_bytes + head_off + (tid & 15) * 16);
        } else {
          vreg[i] = u32x4{0, 0, 0, 0};
        }
      }
    }
  };

  // ---- register -> LDS (K row-major in the query dtype, V^T in fp16) ----
  auto store_tile = [&]() {
    if constexpr (kFp8) {
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        const int key = (tid >> 3) + 32 * i;
        u32x4 lo, hi;
        cvt16_fp8<KV, QBF16>(kreg[i], lo, hi);
        unsigned char* dst = ks + key * kKRow + (tid & 7) * 32;
        *reinterpret_cast<u32x4*>(dst) = lo;
        *reinterpret_cast<u32x4*>(dst + 16) = hi;
      }
      // V: two keys x 16 head-dim entries -> 16 packed pairs
      u32x4 v0l, v0h, v1l, v1h;
      cvt16_fp8<KV, false>(vreg[0], v0l, v0h);
      cvt16_fp8<KV, false>(vreg[1], v1l, v1h);
      const int col = vt_col(2 * (tid >> 3));
      const int d0 = (tid & 7) * 16;
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int w = e >> 1;
        const uint32_t a0 = (w < 4) ? v0l[w] : v0h[w - 4];
        const uint32_t a1 = (w < 4) ? v1l[w] : v1h[w - 4];
        const uint32_t pk = (e & 1) ? pack_hi(a0, a1) : pack_lo(a0, a1);
        *reinterpret_cast<uint32_t*>(vs + (d0 + e) * kVRow + col * 2) = pk;
      }
    } else {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int key = (tid >> 4) + 16 * i;
        *reinterpret_cast<u32x4*>(ks + key * kKRow + (tid & 15) * 16) = kreg[i];
      }
      // V: 4 keys x 8 head-dim entries; bf16 -> fp16 (exact in range), transpose in registers
      uint32_t vh[4][4];
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int w = 0; w < 4; ++w) {
          if constexpr (QBF16) {
            const uint32_t x = vreg[i][w];
            vh[i][w] = pack_f16(__builtin_bit_cast(float, x << 16), __builtin_bit_cast(float, x & 0xffff0000u));
          } else {
            vh[i][w] = vreg[i][w];
          }
        }
      const int col = vt_col(4 * (tid >> 4));
      const int d0 = (tid & 15) * 8;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int w = e >> 1;
        u32x2 pk;
        if (e & 1) { pk[0] = pack_hi(vh[0][w], vh[1][w]); pk[1] = pack_hi(vh[2][w], vh[3][w]); }
        else { pk[0] = pack_lo(vh[0][w], vh[1][w]); pk[1] = pack_lo(vh[2][w], vh[3][w]); }
        *reinterpret_cast<u32x2*>(vs + (d0 + e) * kVRow + col * 2) = pk;
      }
    }
  };

  if (key_lo < key_hi) load_tile(key_lo);
  for (int base = key_lo; base < key_hi; base += kXBN) {
    __syncthreads();
    store_tile();
    __syncthreads();
    if (base + kXBN < key_hi) load_tile(base + kXBN);

    // ---- S^T = K Q^T : 4 key blocks x 2 row blocks ----
    f32x4 s[2][4];
#pragma unroll
    for (int rb = 0; rb < 2; ++rb)
#pragma unroll
      for (int kb = 0; kb < 4; ++kb) s[rb][kb] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
#pragma unroll
      for (int kb = 0; kb < 4; ++kb) {
        const u32x4 kf = *reinterpret_cast<const u32x4*>(ks + (kb * 16 + c) * kKRow + (j * 32 + kk * 8) * 2);
#pragma unroll
        for (int rb = 0; rb < 2; ++rb) s[rb][kb] = mfma16t<QBF16>(kf, qv[rb][kk], s[rb][kb]);
      }
    }

    // ---- online softmax per row (lane column) ----
    const bool full = (base >= full_lo) && (base + kXBN <= full_hi);
    u32x4 pk[2][2];
    float alpha[2];
    bool grew = false;
#pragma unroll
    for (int rb = 0; rb < 2; ++rb) {
      if (!full) {
#pragma unroll
        for (int kb = 0; kb < 4; ++kb)
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const int pos = base + kb * 16 + 4 * j + i;
            if (pos < lo_r[rb] || pos >= hi_r[rb]) s[rb][kb][i] = -INFINITY;
          }
      }
      float mx = -INFINITY;
#pragma unroll
      for (int kb = 0; kb < 4; ++kb)
        mx = fmaxf(mx, fmaxf(fmaxf(s[rb][kb][0], s[rb][kb][1]), fmaxf(s[rb][kb][2], s[rb][kb][3])));
      mx = fmaxf(mx, shfl_xor_f(mx, 16));
      mx = fmaxf(mx, shfl_xor_f(mx, 32));
      const float m_new = fmaxf(m_run[rb], mx);
      const float m_use = (m_new == -INFINITY) ? 0.f : m_new;
      grew |= (m_new != m_run[rb]);
      alpha[rb] = __builtin_amdgcn_exp2f((m_run[rb] - m_use) * a.scale_log2);
      m_run[rb] = m_new;
      const float msc = m_use * a.scale_log2;
      float p[16];
#pragma unroll
      for (int kb = 0; kb < 4; ++kb)
#pragma unroll
        for (int i = 0; i < 4; ++i) p[kb * 4 + i] = __builtin_amdgcn_exp2f(s[rb][kb][i] * a.scale_log2 - msc);
      float ps = 0.f;
#pragma unroll
      for (int x = 0; x < 16; ++x) ps += p[x];
      l_run[rb] = l_run[rb] * alpha[rb] + ps;
      // P^T operand for key step ks: keys (2ks block, i) then (2ks+1 block, i)
#pragma unroll
      for (int st = 0; st < 2; ++st) {
        pk[rb][st][0] = pack_f16(p[(2 * st) * 4 + 0], p[(2 * st) * 4 + 1]);
        pk[rb][st][1] = pack_f16(p[(2 * st) * 4 + 2], p[(2 * st) * 4 + 3]);
        pk[rb][st][2] = pack_f16(p[(2 * st + 1) * 4 + 0], p[(2 * st + 1) * 4 + 1]);
        pk[rb][st][3] = pack_f16(p[(2 * st + 1) * 4 + 2], p[(2 * st + 1) * 4 + 3]);
      }
    }
    if (__builtin_amdgcn_ballot_w64(grew)) {
#pragma unroll
      for (int rb = 0; rb < 2; ++rb)
#pragma unroll
        for (int db = 0; db < 8; ++db) o[rb][db] *= alpha[rb];
    }

    // ---- O^T += V^T P^T : 8 head-dim blocks x 2 key steps x 2 row blocks ----
#pragma unroll
    for (int db = 0; db < 8; ++db) {
#pragma unroll
      for (int st = 0; st < 2; ++st) {
        const u32x4 vf = *reinterpret_cast<const u32x4*>(vs + (db * 16 + c) * kVRow + (st * 32 + j * 8) * 2);
#pragma unroll
        for (int rb = 0; rb < 2; ++rb) o[rb][db] = mfma16t<false>(vf, pk[rb][st], o[rb][db]);
      }
    }
  }

  // ---- epilogue: normalise and write this lane's row ----
#pragma unroll
  for (int rb = 0; rb < 2; ++rb) {
    float lt = l_run[rb];
    lt += shfl_xor_f(lt, 16);
    lt += shfl_xor_f(lt, 32);
    if (!real[rb]) continue;
    const int r = r0 + wave * 32 + rb * 16 + c;
    const int t = r / a.group;
    const int g = r - t * a.group;
    const float inv = (lt > 0.f) ? a.v_scale / lt : 0.f;
    uint16_t* op = reinterpret_cast<uint16_t*>(a.out) + (int64_t)(tok0 + t) * a.out_stride_tok +
                   (int64_t)(h * a.group + g) * a.out_stride_head;
#pragma unroll
    for (int db = 0; db < 8; ++db) {
      u32x2 w;
      w[0] = (uint32_t)f2h<QBF16>(o[rb][db][0] * inv) | ((uint32_t)f2h<QBF16>(o[rb][db][1] * inv) << 16);
      w[1] = (uint32_t)f2h<QBF16>(o[rb][db][2] * inv) | ((uint32_t)f2h<QBF16>(o[rb][db][3] * inv) << 16);
      *reinterpret_cast<u32x2*>(op + db * 16 + 4 * j) = w;
    }
  }
}

template <bool QBF16>
static hipError_t launch_extend_q(int kv, dim3 grid, hipStream_t st, const ExtendArgs& a) {
  switch (kv) {
    case DT_E4M3: hipLaunchKernelGGL((extend_kernel<QBF16, DT_E4M3>), grid, dim3(256), 0, st, a); break;
    case DT_E5M2: hipLaunchKernelGGL((extend_kernel<QBF16, DT_E5M2>), grid, dim3(256), 0, st, a); break;
    default: hipLaunchKernelGGL((extend_kernel<QBF16, QBF16 ? DT_BF16 : DT_F16>), grid, dim3(256), 0, st, a);
  }
  return hipGetLastError();
}

}  // namespace ma

using namespace ma;

extern "C" int ma_paged_extend(
    const void* q, int64_t q_stride_tok, int64_t q_stride_head, int q_dtype, int64_t num_tokens,
    const void* k_cache, const void* v_cache, int64_t kv_stride_row, int64_t kv_stride_head, int kv_dtype,
    const int32_t* table, int64_t table_stride, const int64_t* row_index, int page_size,
    const int32_t* seq_lens, const int32_t* query_start_loc, const int32_t* prefix_lens,
    int batch, int max_q_per_seq, int num_q_heads, int num_kv_heads, int head_dim,
    int causal, int sliding_window, float softmax_scale, float k_scale, float v_scale,
    void* out, int64_t out_stride_tok, int64_t out_stride_head, void* stream) {
  if (head_dim != kXD) return set_error(MA_EUNSUPPORTED, "head_dim %d not supported (128)", head_dim);
  if (q_dtype != DT_F16 && q_dtype != DT_BF16) return set_error(MA_EINVAL, "q dtype %d must be f16 or bf16", q_dtype);
  if (kv_dtype < 0 || kv_dtype > DT_E5M2) return set_error(MA_EINVAL, "kv dtype %d unknown", kv_dtype);
  if ((kv_dtype == DT_F16 || kv_dtype == DT_BF16) && kv_dtype != q_dtype)
    return set_error(MA_EINVAL, "16-bit KV dtype must equal the query dtype");
  if (batch < 0 || num_q_heads <= 0 || num_kv_heads <= 0 || num_q_heads % num_kv_heads)
    return set_error(MA_EINVAL, "bad head counts hq=%d hkv=%d", num_q_heads, num_kv_heads);
  if (page_size <= 0 || (page_size & (page_size - 1))) return set_error(MA_EINVAL, "page size %d must be a power of two", page_size);
  if (!(softmax_scale * k_scale > 0.f)) return set_error(MA_EINVAL, "softmax scale must be positive");
  if (max_q_per_seq < 0) return set_error(MA_EINVAL, "max query rows per sequence must be >= 0");
  if (batch == 0 || max_q_per_seq == 0 || num_tokens == 0) return MA_OK;
  if (!q || !k_cache || !v_cache || !table || !seq_lens || !query_start_loc || !out)
    return set_error(MA_EINVAL, "null pointer argument");
  if ((reinterpret_cast<uintptr_t>(q) | reinterpret_cast<uintptr_t>(k_cache) | reinterpret_cast<uintptr_t>(v_cache) |
       reinterpret_cast<uintptr_t>(out)) & 15)
    return set_error(MA_EINVAL, "q, k, v and out must be 16-byte aligned");
  const int elt = (kv_dtype >= DT_E4M3) ? 1 : 2;
  if (((kv_stride_row * elt) & 15) || ((kv_stride_head * elt) & 15) || ((q_stride_tok * 2) & 15) ||
      ((q_stride_head * 2) & 15) || ((out_stride_tok * 2) & 7) || ((out_stride_head * 2) & 7))
    return set_error(MA_EINVAL, "strides must keep rows 16-byte aligned");
  ExtendArgs a{};
  a.q = q; a.q_stride_tok = q_stride_tok; a.q_stride_head = q_stride_head;
  a.k = k_cache; a.v = v_cache; a.kv_stride_row = kv_stride_row; a.kv_stride_head = kv_stride_head;
  a.tt.table = table; a.tt.stride = table_stride; a.tt.page_shift = __builtin_ctz(page_size);
  a.row_index = row_index; a.seq_lens = seq_lens; a.qsl = query_start_loc; a.prefix = prefix_lens;
  a.batch = batch; a.hq = num_q_heads; a.hkv = num_kv_heads; a.group = num_q_heads / num_kv_heads;
  a.row_tiles = (int)(((int64_t)max_q_per_seq * a.group + kXBM - 1) / kXBM);
  a.causal = causal ? 1 : 0; a.window = sliding_window < 0 ? -1 : sliding_window;
  a.scale_log2 = softmax_scale * k_scale * kLog2e; a.v_scale = v_scale;
  a.out = out; a.out_stride_tok = out_stride_tok; a.out_stride_head = out_stride_head;
  if (batch > 65535 || num_kv_heads > 65535) return set_error(MA_EINVAL, "grid too large");
  dim3 grid(a.row_tiles, num_kv_heads, batch);
  hipError_t e = (q_dtype == DT_BF16) ? launch_extend_q<true>(kv_dtype, grid, (hipStream_t)stream, a)
                                      : launch_extend_q<false>(kv_dtype, grid, (hipStream_t)stream, a);
  if (e != hipSuccess) return set_error(MA_ELAUNCH, "extend launch failed: %s", hipGetErrorString(e));
  return MA_OK;
}
