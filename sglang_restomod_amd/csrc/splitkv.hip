// Grouped split-KV attention for few query rows per sequence: decode (one row)
// and linear-chain target verify (a handful of draft rows under a causal mask).
//
// Replaces the reference's grouped decode partial + combine
// (sglang_restomod/attention/v100/tilelang/_kernels_paged_decode.py:41-312) and
// the grouped verify partial + combine (_kernels_paged_verify.py:52-433).
//
// Work decomposition (one workgroup = 4 waves):
//   blockIdx.x = kv_head * row_groups + row_group,  blockIdx.y = split,  blockIdx.z = sequence.
//   A row group is 16*NB query rows of one kv head: row R -> (query token R / G, head R % G),
//   so every GQA head of a kv head is served from one read of its K/V.
//   The split's key range is cut into 32-token tiles; wave w takes tiles w, w+4, ...
//   Each wave keeps its own online-softmax state; the four are merged in LDS at the end.
//
// Per 32-token tile and wave (all MFMA 16x16x32, fp32 accumulate):
//   S^T[t, r] = K[t, :] . Q[r, :]     M = tokens (two 16-token blocks), N = rows, K = head dim.
//               K rows are loaded from HBM straight into the A-operand layout (16 B per lane
//               per step); Q^T sits in registers for the whole kernel.
//   O^T[d, r] += V^T[d, t] P^T[t, r]  M = head dim (16 per step), N = rows, K = 32 tokens.
//               The S^T accumulator already holds, per lane, the 8 tokens the P^T B-operand
//               needs (tokens 4j..4j+3 and 16+4j..16+4j+3 of lane group j), so P never moves
//               between lanes. V is transposed through a per-wave LDS tile whose rows are
//               head-dim entries and whose 32 columns are the tokens in that same order.
//   16-bit V: P is split into bf16/fp16 hi + lo halves (two MFMAs) for bf16, or cast to fp16.
//   fp8 V: dequantized to fp16 in registers, P cast to fp16.
//
// Numerics: scores and softmax in fp32 (exp2 domain, scale folded in), partial outputs and
// LSE (log2 domain, -2^30 for an empty split) in fp32, output in the query dtype.

#include "common.h"
#include "capi_internal.h"

namespace ma {

constexpr int kWaves = 4;
constexpr int kTile = 32;
constexpr int kVtRow = 80;  // bytes per head-dim row of the V^T tile: 32 tokens * 2 B + 16 B pad

struct SplitKVArgs {
  const void* q;
  int64_t q_stride_tok, q_stride_head;  // elements
  const void* k;
  const void* v;
  int64_t kv_stride_row, kv_stride_head;  // elements (fp8: bytes)
  TokenTable tt;
  const int64_t* row_index;  // request row of each sequence, or null (row b)
  const int32_t* seq_lens;   // keys visible to the last query row of each sequence
  const int32_t* qsl;        // [B+1] query start per sequence, or null (one row per sequence)
  const int32_t* prefix;     // [B] cached prefix per sequence, or null (seq_len - 1)
  int batch, hq, hkv, group;
  int row_groups;
  int max_splits, min_tokens;
  int causal, window;
  float scale_log2;  // softmax_scale * k_scale * log2(e)
  float v_scale;
  float* part_o;     // [max_splits][qrows][D]
  float* part_lse;   // [max_splits][qrows]
  int64_t qrows;     // total query rows (tokens * hq)
  void* out;
  int64_t out_stride_tok, out_stride_head;
};

struct SeqInfo {
  int seq, prefix, tok0, ntok, lo_min, span, active, split_len;
};

// Identical in the partial and the combine kernel: the combine re-derives how many
// splits a sequence used from its lengths alone (no extra metadata, graph-safe).
__device__ __forceinline__ SeqInfo seq_info(const SplitKVArgs& a, int b) {
  SeqInfo s;
  s.seq = a.seq_lens[b];
  if (a.qsl) {
    s.tok0 = a.qsl[b];
    s.ntok = a.qsl[b + 1] - s.tok0;
    s.prefix = a.prefix ? a.prefix[b] : s.seq - s.ntok;
  } else {
    s.tok0 = b;
    s.ntok = 1;
    s.prefix = s.seq - 1;
  }
  s.lo_min = a.window >= 0 ? max(0, s.prefix - a.window) : 0;
  s.lo_min = min(s.lo_min, max(s.seq, 0));
  s.span = max(s.seq - s.lo_min, 0);
  int want = (s.span + a.min_tokens - 1) / a.min_tokens;
  s.active = min(a.max_splits, max(1, want));
  s.split_len = (s.span + s.active - 1) / s.active;
  return s;
}

template <bool BF16>
__device__ __forceinline__ void store_out(void* out, int64_t off, float x) {
  reinterpret_cast<uint16_t*>(out)[off] = f2h<BF16>(x);
}

// ---------------------------------------------------------------------------
// Partial kernel.
//   D: head dim (multiple of 64). NB: 16-row blocks per workgroup.
//   QBF16: query (and 16-bit KV) is bf16. KV: DT_F16 / DT_BF16 / DT_E4M3 / DT_E5M2.
// ---------------------------------------------------------------------------
template <int D, int NB, bool QBF16, int KV>
__global__ __launch_bounds__(256) void splitkv_partial(const SplitKVArgs a) {
  constexpr bool kFp8 = (KV == DT_E4M3 || KV == DT_E5M2);
  constexpr int KK = D / 32;        // QK MFMA steps (32 head-dim entries each)
  constexpr int DB = D / 16;        // PV MFMA steps (16 head-dim rows each)
  constexpr int DQ = D / 4;         // head-dim entries owned by one lane group in QK
  constexpr int kRows = 16 * NB;
  // fp8 V is dequantized to fp16 and multiplied with fp16 P; bf16 V keeps bf16 and
  // multiplies P split in two bf16 halves.
  constexpr bool kPvBf16 = (!kFp8) && QBF16;
  constexpr bool kSplitP = kPvBf16;

  __shared__ __attribute__((aligned(16))) unsigned char smem[kWaves * D * kVtRow];
  __shared__ float sm_m[kWaves][kRows];
  __shared__ float sm_l[kWaves][kRows];

  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int c = lane & 15;
  const int j = lane >> 4;

  const int h = blockIdx.x / a.row_groups;
  const int rg = blockIdx.x - h * a.row_groups;
  const int split = blockIdx.y;
  const int b = blockIdx.z;

  const SeqInfo si = seq_info(a, b);
  if (split >= si.active) return;
  const int s0 = si.lo_min + split * si.split_len;
  const int s1 = min(si.lo_min + si.span, s0 + si.split_len);
  const int64_t seq_row = a.row_index ? a.row_index[b] : (int64_t)b;

  // ---- this lane's query row in each 16-row block: bounds and Q^T operand ----
  int lo_r[NB], hi_r[NB];
  bool real[NB];
  u32x4 qv[NB][KK];
  const uint16_t* qbase = reinterpret_cast<const uint16_t*>(a.q);
#pragma unroll
  for (int nb = 0; nb < NB; ++nb) {
    const int R = rg * kRows + nb * 16 + c;
    const int t = R / a.group;
    const int g = R - t * a.group;
    real[nb] = t < si.ntok;
    const int qpos = si.prefix + t;
    int hi = a.causal ? min(si.seq, qpos + 1) : si.seq;
    int lo = a.window >= 0 ? max(0, qpos - a.window) : 0;
    lo_r[nb] = real[nb] ? max(lo, s0) : 0;
    hi_r[nb] = real[nb] ? min(hi, s1) : 0;
    const uint16_t* qp = qbase + (int64_t)(si.tok0 + t) * a.q_stride_tok +
                         (int64_t)(h * a.group + g) * a.q_stride_head + j * DQ;
#pragma unroll
    for (int kk = 0; kk < KK; ++kk) {
      if (real[nb]) qv[nb][kk] = *reinterpret_cast<const u32x4*>(qp + kk * 8);
      else qv[nb][kk] = u32x4{0, 0, 0, 0};
    }
  }
  // Wave-uniform window in which every real row sees every key (no masking needed).
  int lmax = -0x7fffffff, hmin = 0x7fffffff;
#pragma unroll
  for (int nb = 0; nb < NB; ++nb) {
    if (real[nb]) {
      lmax = max(lmax, lo_r[nb]);
      hmin = min(hmin, hi_r[nb]);
    }
  }
#pragma unroll
  for (int m = 1; m < 64; m <<= 1) {
    lmax = max(lmax, __builtin_amdgcn_ds_bpermute((lane ^ m) << 2, lmax));
    hmin = min(hmin, __builtin_amdgcn_ds_bpermute((lane ^ m) << 2, hmin));
  }

  // ---- online softmax state ----
  float m_run[NB], l_run[NB];
  f32x4 o[NB][DB];
#pragma unroll
  for (int nb = 0; nb < NB; ++nb) {
    m_run[nb] = -INFINITY;
    l_run[nb] = 0.f;
#pragma unroll
    for (int db = 0; db < DB; ++db) o[nb][db] = f32x4{0.f, 0.f, 0.f, 0.f};
  }

  unsigned char* vt = smem + wave * D * kVtRow;
  const unsigned char* kbase = reinterpret_cast<const unsigned char*>(a.k);
  const unsigned char* vbase = reinterpret_cast<const unsigned char*>(a.v);
  constexpr int kElt = kFp8 ? 1 : 2;
  const int64_t row_bytes = a.kv_stride_row * kElt;
  const int64_t head_off = (int64_t)h * a.kv_stride_head * kElt;

  for (int tb0 = s0 + kTile * wave; tb0 < s1; tb0 += kTile * kWaves) {
    // slot of token (lane & 31) of the tile, spread to the lanes that load it
    const int mypos = tb0 + (lane & 31);
    int myslot = 0;
    if (mypos < s1) myslot = (int)kv_row(a.tt, seq_row, mypos);

    // ---- K: straight into the A-operand layout ----
    u32x4 kr[2][KK];
#pragma unroll
    for (int tb = 0; tb < 2; ++tb) {
      const int tok = tb * 16 + c;
      const int slot = shfl_i(myslot, tok);
      const bool ok = tb0 + tok < s1;
      const unsigned char* kp = kbase + (int64_t)slot * row_bytes + head_off;
      if constexpr (kFp8) {
#pragma unroll
        for (int half = 0; half < KK / 2; ++half) {
          u32x4 raw = ok ? *reinterpret_cast<const u32x4*>(kp + j * DQ + half * 16) : u32x4{0, 0, 0, 0};
          cvt16_fp8<KV, QBF16>(raw, kr[tb][2 * half], kr[tb][2 * half + 1]);
        }
      } else {
#pragma unroll
        for (int kk = 0; kk < KK; ++kk)
          kr[tb][kk] = ok ? *reinterpret_cast<const u32x4*>(kp + (j * DQ + kk * 8) * 2) : u32x4{0, 0, 0, 0};
      }
    }

    // ---- V: load rows, convert to the PV operand type ----
    // 16-bit: lane holds head-dim chunk (lane & 15) of tokens 4j+i and 16+4j+i.
    // fp8:    lane holds head-dim chunk (lane & 7) (16 entries) of tokens 4(lane>>3)+i.
    u32x4 vr[8];
    if constexpr (kFp8) {
      const int ch = lane & 7, qd = lane >> 3;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int tok = 4 * qd + i;
        const int slot = shfl_i(myslot, tok);
        const bool ok = tb0 + tok < s1;
        u32x4 raw = ok ? *reinterpret_cast<const u32x4*>(vbase + (int64_t)slot * row_bytes + head_off + ch * 16)
                       : u32x4{0, 0, 0, 0};
        cvt16_fp8<KV, false>(raw, vr[2 * i], vr[2 * i + 1]);
      }
    } else {
#pragma unroll
      for (int hh = 0; hh < 2; ++hh) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int tok = 16 * hh + 4 * j + i;
          const int slot = shfl_i(myslot, tok);
          const bool ok = tb0 + tok < s1;
          vr[4 * hh + i] = ok ? *reinterpret_cast<const u32x4*>(vbase + (int64_t)slot * row_bytes + head_off + c * 16)
                              : u32x4{0, 0, 0, 0};
        }
      }
    }

    // ---- S^T = K Q^T ----
    f32x4 s[NB][2];
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) {
#pragma unroll
      for (int tb = 0; tb < 2; ++tb) {
        f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int kk = 0; kk < KK; ++kk) acc = mfma16t<QBF16>(kr[tb][kk], qv[nb][kk], acc);
        s[nb][tb] = acc;
      }
    }

    // ---- V^T tile into LDS (columns in the P^T token order) ----
    if constexpr (kFp8) {
      const int ch = lane & 7, qd = lane >> 3;
      const int col = (qd < 4) ? 8 * qd : 8 * (qd - 4) + 4;
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int w = e >> 1;  // dword inside the 16 converted values
        uint32_t a0 = (w < 4) ? vr[0][w] : vr[1][w - 4];
        uint32_t a1 = (w < 4) ? vr[2][w] : vr[3][w - 4];
        uint32_t a2 = (w < 4) ? vr[4][w] : vr[5][w - 4];
        uint32_t a3 = (w < 4) ? vr[6][w] : vr[7][w - 4];
        u32x2 pk;
        if (e & 1) { pk[0] = pack_hi(a0, a1); pk[1] = pack_hi(a2, a3); }
        else { pk[0] = pack_lo(a0, a1); pk[1] = pack_lo(a2, a3); }
        *reinterpret_cast<u32x2*>(vt + (ch * 16 + e) * kVtRow + col * 2) = pk;
      }
    } else {
#pragma unroll
      for (int hh = 0; hh < 2; ++hh) {
        const int col = 8 * j + 4 * hh;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const int w = e >> 1;
          uint32_t a0 = vr[4 * hh + 0][w], a1 = vr[4 * hh + 1][w];
          uint32_t a2 = vr[4 * hh + 2][w], a3 = vr[4 * hh + 3][w];
          u32x2 pk;
          if (e & 1) { pk[0] = pack_hi(a0, a1); pk[1] = pack_hi(a2, a3); }
          else { pk[0] = pack_lo(a0, a1); pk[1] = pack_lo(a2, a3); }
          *reinterpret_cast<u32x2*>(vt + (c * 8 + e) * kVtRow + col * 2) = pk;
        }
      }
    }

    // ---- online softmax (column = this lane's row) ----
    const bool full = (tb0 >= lmax) && (tb0 + kTile <= hmin);
    u32x4 pb[NB], pl[NB];
    bool grew = false;
    float alpha[NB];
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) {
      if (!full) {
#pragma unroll
        for (int tb = 0; tb < 2; ++tb)
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const int pos = tb0 + tb * 16 + 4 * j + i;
            if (pos < lo_r[nb] || pos >= hi_r[nb]) s[nb][tb][i] = -INFINITY;
          }
      }
      float mx = fmaxf(fmaxf(fmaxf(s[nb][0][0], s[nb][0][1]), fmaxf(s[nb][0][2], s[nb][0][3])),
                       fmaxf(fmaxf(s[nb][1][0], s[nb][1][1]), fmaxf(s[nb][1][2], s[nb][1][3])));
      mx = fmaxf(mx, shfl_xor_f(mx, 16));
      mx = fmaxf(mx, shfl_xor_f(mx, 32));
      const float m_new = fmaxf(m_run[nb], mx);
      const float m_use = (m_new == -INFINITY) ? 0.f : m_new;
      grew |= (m_new != m_run[nb]);
      alpha[nb] = __builtin_amdgcn_exp2f((m_run[nb] - m_use) * a.scale_log2);
      m_run[nb] = m_new;
      float p[8];
#pragma unroll
      for (int tb = 0; tb < 2; ++tb)
#pragma unroll
        for (int i = 0; i < 4; ++i) p[4 * tb + i] = __builtin_amdgcn_exp2f((s[nb][tb][i] - m_use) * a.scale_log2);
      float ps = ((p[0] + p[1]) + (p[2] + p[3])) + ((p[4] + p[5]) + (p[6] + p[7]));
      l_run[nb] = l_run[nb] * alpha[nb] + ps;
      if constexpr (kSplitP) {
#pragma unroll
        for (int w = 0; w < 4; ++w) {
          uint32_t hi, lo;
          split_bf16(p[2 * w], p[2 * w + 1], hi, lo);
          pb[nb][w] = hi;
          pl[nb][w] = lo;
        }
      } else {
#pragma unroll
        for (int w = 0; w < 4; ++w) pb[nb][w] = pack_f16(p[2 * w], p[2 * w + 1]);
      }
    }
    if (__builtin_amdgcn_ballot_w64(grew)) {
#pragma unroll
      for (int nb = 0; nb < NB; ++nb)
#pragma unroll
        for (int db = 0; db < DB; ++db) o[nb][db] *= alpha[nb];
    }

    // ---- O^T += V^T P^T ----
    __asm__ volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
#pragma unroll
    for (int db = 0; db < DB; ++db) {
      const u32x4 va = *reinterpret_cast<const u32x4*>(vt + (db * 16 + c) * kVtRow + j * 16);
#pragma unroll
      for (int nb = 0; nb < NB; ++nb) {
        o[nb][db] = mfma16t<kPvBf16>(va, pb[nb], o[nb][db]);
        if constexpr (kSplitP) o[nb][db] = mfma16t<kPvBf16>(va, pl[nb], o[nb][db]);
      }
    }
    __asm__ volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
  }

  // ---- merge the four waves ----
#pragma unroll
  for (int nb = 0; nb < NB; ++nb) {
    float lt = l_run[nb];
    lt += shfl_xor_f(lt, 16);
    lt += shfl_xor_f(lt, 32);
    l_run[nb] = lt;
    if (j == 0) {
      sm_m[wave][nb * 16 + c] = m_run[nb];
      sm_l[wave][nb * 16 + c] = lt;
    }
  }
  __syncthreads();
  float* acc = reinterpret_cast<float*>(smem);  // [kRows][D], reuses the V^T tiles
  for (int idx = threadIdx.x; idx < kRows * D; idx += 256) acc[idx] = 0.f;
  float M[NB], L[NB];
#pragma unroll
  for (int nb = 0; nb < NB; ++nb) {
    const int col = nb * 16 + c;
    float mm = -INFINITY;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) mm = fmaxf(mm, sm_m[w][col]);
    const float mu = (mm == -INFINITY) ? 0.f : mm;
    float ll = 0.f;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) ll += sm_l[w][col] * __builtin_amdgcn_exp2f((sm_m[w][col] - mu) * a.scale_log2);
    M[nb] = mm;
    L[nb] = ll;
  }
  __syncthreads();
#pragma unroll
  for (int nb = 0; nb < NB; ++nb) {
    const float mu = (M[nb] == -INFINITY) ? 0.f : M[nb];
    const float f = (L[nb] > 0.f) ? __builtin_amdgcn_exp2f((m_run[nb] - mu) * a.scale_log2) / L[nb] : 0.f;
    const int col = nb * 16 + c;
#pragma unroll
    for (int db = 0; db < DB; ++db)
#pragma unroll
      for (int i = 0; i < 4; ++i) atomicAdd(&acc[col * D + db * 16 + 4 * j + i], o[nb][db][i] * f);
  }
  __syncthreads();

  // ---- write: final output when this sequence has one split, else a partial ----
  const bool direct = (si.active == 1);
  for (int idx = threadIdx.x; idx < kRows * (D / 4); idx += 256) {
    const int col = idx / (D / 4);
    const int d4 = (idx - col * (D / 4)) * 4;
    const int R = rg * kRows + col;
    const int t = R / a.group;
    const int g = R - t * a.group;
    if (t >= si.ntok) continue;
    const int tok = si.tok0 + t;
    const int head = h * a.group + g;
    f32x4 val = *reinterpret_cast<const f32x4*>(&acc[col * D + d4]);
    if (direct) {
      const int64_t off = (int64_t)tok * a.out_stride_tok + (int64_t)head * a.out_stride_head + d4;
      uint16_t* op = reinterpret_cast<uint16_t*>(a.out) + off;
      u32x2 pk;
      pk[0] = (uint32_t)f2h<QBF16>(val[0] * a.v_scale) | ((uint32_t)f2h<QBF16>(val[1] * a.v_scale) << 16);
      pk[1] = (uint32_t)f2h<QBF16>(val[2] * a.v_scale) | ((uint32_t)f2h<QBF16>(val[3] * a.v_scale) << 16);
      *reinterpret_cast<u32x2*>(op) = pk;
    } else {
      const int64_t qrow = (int64_t)tok * a.hq + head;
      *reinterpret_cast<f32x4*>(a.part_o + ((int64_t)split * a.qrows + qrow) * D + d4) = val;
    }
  }
  if (!direct && threadIdx.x < kRows) {
    const int col = threadIdx.x;
    const int R = rg * kRows + col;
    const int t = R / a.group;
    const int g = R - t * a.group;
    if (t < si.ntok) {
      const int nbk = col >> 4;
      float mm = -INFINITY, ll = 0.f;
      // M/L for this column live in the lanes of wave 0 with c == col & 15
#pragma unroll
      for (int w = 0; w < kWaves; ++w) mm = fmaxf(mm, sm_m[w][col]);
      const float mu = (mm == -INFINITY) ? 0.f : mm;
#pragma unroll
      for (int w = 0; w < kWaves; ++w) ll += sm_l[w][col] * __builtin_amdgcn_exp2f((sm_m[w][col] - mu) * a.scale_log2);
      (void)nbk;
      const int64_t qrow = (int64_t)(si.tok0 + t) * a.hq + h * a.group + g;
      a.part_lse[(int64_t)split * a.qrows + qrow] = (ll > 0.f) ? __builtin_amdgcn_logf(ll) + mu * a.scale_log2 : kEmptyLse;
    }
  }
}

// ---------------------------------------------------------------------------
// Combine: LSE-weighted merge of the split partials (log2 domain).
// grid (ceil(hq / 8), max_tokens_per_seq, batch), 256 threads: 32 threads per head,
// 4 head-dim entries per thread.
// ---------------------------------------------------------------------------
template <int D, bool QBF16>
__global__ __launch_bounds__(256) void splitkv_combine(const SplitKVArgs a) {
  constexpr int TPH = D / 4;           // threads per head
  constexpr int HPB = 256 / TPH;       // heads per block
  const int b = blockIdx.z;
  const int t = blockIdx.y;
  const SeqInfo si = seq_info(a, b);
  if (si.active == 1 || t >= si.ntok) return;
  const int head = blockIdx.x * HPB + threadIdx.x / TPH;
  if (head >= a.hq) return;
  const int d4 = (threadIdx.x % TPH) * 4;
  const int tok = si.tok0 + t;
  const int64_t qrow = (int64_t)tok * a.hq + head;
  float mx = -INFINITY;
  for (int s = 0; s < si.active; ++s) mx = fmaxf(mx, a.part_lse[(int64_t)s * a.qrows + qrow]);
  float wsum = 0.f;
  f32x4 accv = {0.f, 0.f, 0.f, 0.f};
  for (int s = 0; s < si.active; ++s) {
    const float w = __builtin_amdgcn_exp2f(a.part_lse[(int64_t)s * a.qrows + qrow] - mx);
    wsum += w;
    const f32x4 po = *reinterpret_cast<const f32x4*>(a.part_o + ((int64_t)s * a.qrows + qrow) * D + d4);
    accv += po * w;
  }
  const float inv = a.v_scale / wsum;
  const int64_t off = (int64_t)tok * a.out_stride_tok + (int64_t)head * a.out_stride_head + d4;
  uint16_t* op = reinterpret_cast<uint16_t*>(a.out) + off;
  u32x2 pk;
  pk[0] = (uint32_t)f2h<QBF16>(accv[0] * inv) | ((uint32_t)f2h<QBF16>(accv[1] * inv) << 16);
  pk[1] = (uint32_t)f2h<QBF16>(accv[2] * inv) | ((uint32_t)f2h<QBF16>(accv[3] * inv) << 16);
  *reinterpret_cast<u32x2*>(op) = pk;
}

// ---------------------------------------------------------------------------
// Host-side dispatch.
// ---------------------------------------------------------------------------
template <int D, int NB, bool QBF16>
static hipError_t launch_partial_kv(int kv, dim3 grid, hipStream_t st, const SplitKVArgs& a) {
  switch (kv) {
    case DT_E4M3: hipLaunchKernelGGL((splitkv_partial<D, NB, QBF16, DT_E4M3>), grid, dim3(256), 0, st, a); break;
    case DT_E5M2: hipLaunchKernelGGL((splitkv_partial<D, NB, QBF16, DT_E5M2>), grid, dim3(256), 0, st, a); break;
    default:
      hipLaunchKernelGGL((splitkv_partial<D, NB, QBF16, QBF16 ? DT_BF16 : DT_F16>), grid, dim3(256), 0, st, a);
  }
  return hipGetLastError();
}

template <int D>
static hipError_t launch_partial_d(int nb, bool qbf16, int kv, dim3 grid, hipStream_t st, const SplitKVArgs& a) {
  if (qbf16) {
    if (nb == 1) return launch_partial_kv<D, 1, true>(kv, grid, st, a);
    if (nb == 2) return launch_partial_kv<D, 2, true>(kv, grid, st, a);
    return launch_partial_kv<D, 4, true>(kv, grid, st, a);
  }
  if (nb == 1) return launch_partial_kv<D, 1, false>(kv, grid, st, a);
  if (nb == 2) return launch_partial_kv<D, 2, false>(kv, grid, st, a);
  return launch_partial_kv<D, 4, false>(kv, grid, st, a);
}

template <int D>
static hipError_t launch_combine_d(bool qbf16, dim3 grid, hipStream_t st, const SplitKVArgs& a) {
  if (qbf16) hipLaunchKernelGGL((splitkv_combine<D, true>), grid, dim3(256), 0, st, a);
  else hipLaunchKernelGGL((splitkv_combine<D, false>), grid, dim3(256), 0, st, a);
  return hipGetLastError();
}

}  // namespace ma

using namespace ma;

// Common body of ma_grouped_decode and ma_paged_verify.
static int splitkv_run(SplitKVArgs a, int head_dim, int q_dtype, int kv_dtype, int max_q_per_seq,
                       size_t workspace_bytes, hipStream_t stream) {
  if (head_dim != 128) return set_error(MA_EUNSUPPORTED, "head_dim %d not supported (128)", head_dim);
  if (q_dtype != DT_F16 && q_dtype != DT_BF16) return set_error(MA_EINVAL, "q dtype %d must be f16 or bf16", q_dtype);
  if (kv_dtype < 0 || kv_dtype > DT_E5M2) return set_error(MA_EINVAL, "kv dtype %d unknown", kv_dtype);
  if ((kv_dtype == DT_F16 || kv_dtype == DT_BF16) && kv_dtype != q_dtype)
    return set_error(MA_EINVAL, "16-bit KV dtype must equal the query dtype");
  if (a.batch < 0 || a.hq <= 0 || a.hkv <= 0 || a.hq % a.hkv)
    return set_error(MA_EINVAL, "bad head counts hq=%d hkv=%d", a.hq, a.hkv);
  if (a.max_splits <= 0 || a.min_tokens <= 0) return set_error(MA_EINVAL, "max_splits and min_tokens must be positive");
  if (!(a.scale_log2 > 0.f)) return set_error(MA_EINVAL, "softmax scale must be positive");
  if (a.tt.page_shift < 0 || a.tt.page_shift > 16) return set_error(MA_EINVAL, "bad page shift");
  if (max_q_per_seq <= 0) return set_error(MA_EINVAL, "max query rows per sequence must be positive");
  if (a.batch == 0) return MA_OK;
  if (!a.q || !a.k || !a.v || !a.tt.table || !a.seq_lens || !a.out)
    return set_error(MA_EINVAL, "null pointer argument");
  if ((reinterpret_cast<uintptr_t>(a.q) | reinterpret_cast<uintptr_t>(a.k) | reinterpret_cast<uintptr_t>(a.v) |
       reinterpret_cast<uintptr_t>(a.out)) & 15)
    return set_error(MA_EINVAL, "q, k, v and out must be 16-byte aligned");
  const int elt = (kv_dtype >= DT_E4M3) ? 1 : 2;
  if (((a.kv_stride_row * elt) & 15) || ((a.kv_stride_head * elt) & 15) || ((a.q_stride_tok * 2) & 15) ||
      ((a.q_stride_head * 2) & 15) || ((a.out_stride_tok * 2) & 7) || ((a.out_stride_head * 2) & 7))
    return set_error(MA_EINVAL, "strides must keep rows 16-byte aligned");
  a.group = a.hq / a.hkv;
  const int rows = max_q_per_seq * a.group;
  const int nb = rows <= 16 ? 1 : (rows <= 32 ? 2 : 4);
  a.row_groups = (rows + 16 * nb - 1) / (16 * nb);
  const size_t need = ma_splitkv_workspace_bytes(a.max_splits, a.qrows / a.hq, a.hq, head_dim);
  if (a.max_splits > 1 && (!a.part_o || workspace_bytes < need))
    return set_error(MA_EINVAL, "workspace too small: %zu < %zu bytes", workspace_bytes, need);
  dim3 grid(a.hkv * a.row_groups, a.max_splits, a.batch);
  hipError_t e = launch_partial_d<128>(nb, q_dtype == DT_BF16, kv_dtype, grid, stream, a);
  if (e != hipSuccess) return set_error(MA_ELAUNCH, "partial launch failed: %s", hipGetErrorString(e));
  if (a.max_splits > 1) {
    dim3 cg((a.hq + 7) / 8, max_q_per_seq, a.batch);
    e = launch_combine_d<128>(q_dtype == DT_BF16, cg, stream, a);
    if (e != hipSuccess) return set_error(MA_ELAUNCH, "combine launch failed: %s", hipGetErrorString(e));
  }
  return MA_OK;
}

extern "C" size_t ma_splitkv_workspace_bytes(int max_splits, int64_t num_tokens, int num_q_heads, int head_dim) {
  if (max_splits <= 1) return 0;
  const int64_t rows = num_tokens * (int64_t)num_q_heads;
  // partial O then partial LSE, each 256-byte aligned
  size_t o = (size_t)max_splits * rows * head_dim * sizeof(float);
  o = (o + 255) & ~(size_t)255;
  size_t l = (size_t)max_splits * rows * sizeof(float);
  return o + ((l + 255) & ~(size_t)255);
}

static void split_workspace(SplitKVArgs& a, void* ws, int64_t rows, int head_dim) {
  if (!ws || a.max_splits <= 1) {
    a.part_o = nullptr;
    a.part_lse = nullptr;
    return;
  }
  size_t o = (size_t)a.max_splits * rows * head_dim * sizeof(float);
  o = (o + 255) & ~(size_t)255;
  a.part_o = reinterpret_cast<float*>(ws);
  a.part_lse = reinterpret_cast<float*>(reinterpret_cast<char*>(ws) + o);
}

extern "C" int ma_grouped_decode(
    const void* q, int64_t q_stride_tok, int64_t q_stride_head, int q_dtype,
    const void* k_cache, const void* v_cache, int64_t kv_stride_row, int64_t kv_stride_head, int kv_dtype,
    const int32_t* table, int64_t table_stride, const int64_t* row_index, int page_size,
    const int32_t* seq_lens, int batch, int num_q_heads, int num_kv_heads, int head_dim,
    int max_splits, int min_tokens_per_split, float softmax_scale, float k_scale, float v_scale,
    int sliding_window, void* workspace, size_t workspace_bytes,
    void* out, int64_t out_stride_tok, int64_t out_stride_head, void* stream) {
  if (page_size <= 0 || (page_size & (page_size - 1))) return set_error(MA_EINVAL, "page size %d must be a power of two", page_size);
  SplitKVArgs a{};
  a.q = q; a.q_stride_tok = q_stride_tok; a.q_stride_head = q_stride_head;
  a.k = k_cache; a.v = v_cache; a.kv_stride_row = kv_stride_row; a.kv_stride_head = kv_stride_head;
  a.tt.table = table; a.tt.stride = table_stride; a.tt.page_shift = __builtin_ctz(page_size);
  a.row_index = row_index; a.seq_lens = seq_lens; a.qsl = nullptr; a.prefix = nullptr;
  a.batch = batch; a.hq = num_q_heads; a.hkv = num_kv_heads;
  a.max_splits = max_splits; a.min_tokens = min_tokens_per_split;
  a.causal = 1; a.window = sliding_window < 0 ? -1 : sliding_window;
  a.scale_log2 = softmax_scale * k_scale * kLog2e; a.v_scale = v_scale;
  a.qrows = (int64_t)batch * num_q_heads;
  a.out = out; a.out_stride_tok = out_stride_tok; a.out_stride_head = out_stride_head;
  split_workspace(a, workspace, a.qrows, head_dim);
  return splitkv_run(a, head_dim, q_dtype, kv_dtype, 1, workspace_bytes, (hipStream_t)stream);
}

extern "C" int ma_paged_verify(
    const void* q, int64_t q_stride_tok, int64_t q_stride_head, int q_dtype, int64_t num_tokens,
    const void* k_cache, const void* v_cache, int64_t kv_stride_row, int64_t kv_stride_head, int kv_dtype,
    const int32_t* table, int64_t table_stride, const int64_t* row_index, int page_size,
    const int32_t* seq_lens, const int32_t* query_start_loc, const int32_t* prefix_lens,
    int batch, int max_q_per_seq, int num_q_heads, int num_kv_heads, int head_dim,
    int causal, int sliding_window, int max_splits, int min_tokens_per_split,
    float softmax_scale, float k_scale, float v_scale, void* workspace, size_t workspace_bytes,
    void* out, int64_t out_stride_tok, int64_t out_stride_head, void* stream) {
  if (page_size <= 0 || (page_size & (page_size - 1))) return set_error(MA_EINVAL, "page size %d must be a power of two", page_size);
  if (!query_start_loc) return set_error(MA_EINVAL, "query_start_loc is required");
  if (max_q_per_seq > 64) return set_error(MA_EUNSUPPORTED, "verify supports at most 64 query rows per sequence");
  SplitKVArgs a{};
  a.q = q; a.q_stride_tok = q_stride_tok; a.q_stride_head = q_stride_head;
  a.k = k_cache; a.v = v_cache; a.kv_stride_row = kv_stride_row; a.kv_stride_head = kv_stride_head;
  a.tt.table = table; a.tt.stride = table_stride; a.tt.page_shift = __builtin_ctz(page_size);
  a.row_index = row_index; a.seq_lens = seq_lens; a.qsl = query_start_loc; a.prefix = prefix_lens;
  a.batch = batch; a.hq = num_q_heads; a.hkv = num_kv_heads;
  a.max_splits = max_splits; a.min_tokens = min_tokens_per_split;
  a.causal = causal ? 1 : 0; a.window = sliding_window < 0 ? -1 : sliding_window;
  a.scale_log2 = softmax_scale * k_scale * kLog2e; a.v_scale = v_scale;
  a.qrows = num_tokens * num_q_heads;
  a.out = out; a.out_stride_tok = out_stride_tok; a.out_stride_head = out_stride_head;
  split_workspace(a, workspace, a.qrows, head_dim);
  return splitkv_run(a, head_dim, q_dtype, kv_dtype, max_q_per_seq, workspace_bytes, (hipStream_t)stream);
}
