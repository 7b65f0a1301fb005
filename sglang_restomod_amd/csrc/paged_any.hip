// Paged attention at the head dims the tuned kernels do not take: every multiple of 16
// from 16 to 512 other than 64, 128 and 256 (the reference's paged kernels take any head
// dim, with a default tile configuration and a tuned one for 512:
// sglang_restomod/attention/v100/tilelang/_kernels_paged.py:397-418; above 256 its linear
// verify also runs on the ordinary paged kernel, _paged_adapter.py:612-616).
//
// One kernel serves decode, linear verify and extend rows. A wave computes 16 query rows
// (token, GQA head) of one sequence and kv head over 16-key tiles:
//   - scores S^T = K Q^T on 16x16x32 MFMAs (the query's 16-bit type; fp8 K converted),
//     so each lane holds four keys of one row: the B operand of the 16x16x16 fp16 MFMA
//     of O^T += V^T P^T, whose A operand is read transposed (ds_read_b64_tr_b16) from
//     fp16 V rows in LDS,
//   - an online softmax with the tuned kernels' lazy rescale (kLazyRescale).
// Decode and verify (no work list): the four waves of a workgroup hold the same 16 rows
// and take a quarter of their key tiles each, K straight into operand registers and V
// through the wave's own LDS rows, then merge through LDS. Extend (the work list): the
// four waves hold 64 consecutive rows and share each K/V tile through a two-stage LDS
// ring, one barrier per tile.
// The kernel is as wide as the next of 64, 128, 256 and 512: lanes past the head dim
// read the row's last dims again (every load is unconditional), which meet Q's zeros in
// the scores and fill output dims that are never stored.
#include "capi_internal.h"
#include "paged_any.h"

namespace ma {

typedef __attribute__((__vector_size__(4 * sizeof(_Float16)))) _Float16 f16x4;

template <bool FP8>
struct AnyVRaw;  // one V unit (8 elements) as loaded
template <>
struct AnyVRaw<false> {
  typedef u32x4 type;
};
template <>
struct AnyVRaw<true> {
  typedef u32x2 type;
};

template <int DP, bool QBF16, int KV>
__global__ __launch_bounds__(kAnyWaves * 64, DP >= 256 ? 1 : 2) void any_kernel(const AnyArgs args) {
  const AnyArgs a = args;  // local copy: the lambdas capture by reference
  constexpr bool kFp8 = (KV == DT_E4M3 || KV == DT_E5M2);
  constexpr int KK = DP / 32;                   // QK MFMA steps
  constexpr int DB = DP / 16;                   // PV MFMA steps, 16 output dims each
  constexpr int kElt = kFp8 ? 1 : 2;            // bytes of one K/V element
  constexpr int kKL = kFp8 ? KK / 2 : KK;       // 16-byte K loads per lane per tile
  constexpr int kRowL = DP * 2 + 32;            // LDS bytes of one fp16 V row, padded: row t
                                                // starts 32 t bytes into a 256-byte bank period
  constexpr int kUnits = DP / 8;                // 8-element V units per row
  constexpr int kUL = kUnits * kAnyKeys / 64;   // V units per lane per tile
  static_assert(kUL >= 1 && (kUnits * kAnyKeys) % 64 == 0, "whole V units per lane");
  static_assert(!kFp8 || KK % 2 == 0, "fp8 K loads cover two QK steps");
  typedef typename AnyVRaw<kFp8>::type VRaw;

  // At the widest head dim with 16-bit KV, Q lives in LDS (rows padded by 16 bytes so the
  // 16 rows of an operand read fall in different banks): its 64 registers are what the
  // prefetched K and V need.
  constexpr bool kQLds = DP >= 512 && !kFp8;
  constexpr int kQRow = DP * 2 + 16;
  constexpr int kVBlock = kAnyKeys * kRowL;            // one wave's V rows
  constexpr int kQBlock = kQLds ? kAnyRows * kQRow : 0;  // one wave's Q rows
  constexpr int kSmem = kAnyWaves * (kVBlock + kQBlock);
  // When the four waves split one row block's keys, their partial O meet in the same
  // memory after the loop, kBPR 16-column blocks (1 KiB per wave each) at a time.
  constexpr int kBPR = (DB * kAnyWaves * 1024 <= kSmem) ? DB
                       : (DB / 2 * kAnyWaves * 1024 <= kSmem) ? DB / 2
                       : (DB / 4 * kAnyWaves * 1024 <= kSmem) ? DB / 4 : DB / 8;
  static_assert(kBPR >= 1 && kBPR * kAnyWaves * 1024 <= kSmem, "merge rounds fit the V/Q memory");
  // Extend rows: the four waves own 64 consecutive rows of one sequence and kv head and
  // share every K/V tile through a two-stage LDS ring (16-bit K rows padded by 16 bytes,
  // fp16 V rows as above), loaded once per workgroup; kUW 16-byte units per thread.
  constexpr int kRowK = DP * 2 + 16;
  constexpr int kKTile = kAnyKeys * kRowK;
  constexpr int kStageB = kKTile + kVBlock;
  constexpr int kTileUnits = kAnyKeys * kUnits;  // 16-byte units of one K (or V) tile
  constexpr int kUW = kTileUnits >= kAnyWaves * 64 ? kTileUnits / (kAnyWaves * 64) : 1;
  static_assert(2 * kStageB <= kAnyWaves * kVBlock, "the ring fits the per-wave V memory it replaces");
  __shared__ __attribute__((aligned(256))) unsigned char smem[kSmem];
  __shared__ float mrow[kAnyWaves][2][kAnyRows];  // each wave's row max and row sum of p

  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int c = lane & 15;
  const int j = lane >> 4;
  const int D = a.head_dim;
  const int G = a.group;
  const uint32_t smem_base = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) unsigned char*)smem;
  const uint32_t lds_base = smem_base + wave * kVBlock;                          // this wave's V rows
  const uint32_t q_base = smem_base + kAnyWaves * kVBlock + wave * kQBlock;      // and Q rows

  // first dim of QK step kk for lane group j (fp8: one 16-byte load covers two steps)
  auto qdim = [&](int kk) -> int {
    if constexpr (kFp8) return (kk >> 1) * 64 + j * 16 + (kk & 1) * 8;
    else return kk * 32 + j * 8;
  };
  const unsigned char MA_GLOBAL* kbase = gptr(reinterpret_cast<const unsigned char*>(a.k));
  const unsigned char MA_GLOBAL* vbase = gptr(reinterpret_cast<const unsigned char*>(a.v));
  const int64_t row_bytes = a.kv_stride_row * kElt;
  const int page_mask = (1 << a.tt.page_shift) - 1;

  // One wave's 16 rows r0 .. r0 + 15 of sequence b, kv head h. split < 0: the workgroup's
  // four waves own consecutive row blocks (rows r0 - 16 * wave ..) and walk the keys any
  // of them sees together, sharing each K/V tile. split >= 0: the four waves own the same
  // row block and take quarter `split` of its key tiles each, merging at the end.
  auto rows = [&](int b, int h, int r0, int split) __attribute__((always_inline)) {
    const bool shared = split < 0;
    const int rg0 = shared ? r0 - wave * kAnyRows : r0;  // first row of the workgroup's rows
    const int rgn = shared ? kAnyWaves * kAnyRows : kAnyRows;
    int tok0, ntok;
    if (a.qsl) {
      const QueryRows qr = clamp_query_rows(cptr(a.qsl)[b], cptr(a.qsl)[b + 1], a.num_tokens);
      tok0 = qr.tok0;
      ntok = qr.ntok;
    } else {
      tok0 = b;
      ntok = b < a.num_tokens ? 1 : 0;
    }
    if (rg0 >= ntok * G) return;  // the same for every wave of the workgroup
    const int seq = max(cptr(a.seq_lens)[b], 0);
    const int prefix = a.prefix ? cptr(a.prefix)[b] : seq - ntok;
    const int64_t seq_row = a.row_index ? cptr(a.row_index)[b] : (int64_t)b;
    const int64_t head_off = (int64_t)h * a.kv_stride_head * kElt;

    // this lane's row (column c of every MFMA result)
    const int r = r0 + c;
    const int t = r / G;
    const int g = r - t * G;
    const bool real = t < ntok;
    const int qpos = prefix + t;
    const int lo_r = (real && a.window >= 0) ? max(0, qpos - a.window) : 0;
    const int hi_r = real ? (a.causal ? min(seq, qpos + 1) : seq) : 0;
    u32x4 qv[kQLds ? 1 : KK];
    const uint32_t qa = q_base + c * kQRow + j * 16;
    {
      const uint16_t MA_GLOBAL* qp = gptr(reinterpret_cast<const uint16_t*>(a.q)) +
                                     (int64_t)(tok0 + (real ? t : 0)) * a.q_stride_tok +
                                     (int64_t)(h * G + g) * a.q_stride_head;
#pragma unroll
      for (int kk = 0; kk < KK; ++kk) {
        const int d0 = shared ? kk * 32 + j * 8 : qdim(kk);
        const u32x4 qf = (real && d0 < D) ? *reinterpret_cast<const u32x4 MA_GLOBAL*>(qp + d0) : u32x4{0, 0, 0, 0};
        if constexpr (kQLds) *reinterpret_cast<__attribute__((address_space(3))) u32x4*>((uintptr_t)(qa + kk * 64)) = qf;
        else qv[kk] = qf;
      }
    }
    // keys any of the rows (the wave's, or the workgroup's in shared mode) may see
    const int t_first = rg0 / G;
    const int t_last = min(ntok - 1, (rg0 + rgn - 1) / G);
    const int key_lo = a.window >= 0 ? max(0, prefix + t_first - a.window) : 0;
    const int key_hi = a.causal ? min(seq, prefix + t_last + 1) : seq;
    const int nt = key_hi > key_lo ? (key_hi - key_lo + kAnyKeys - 1) / kAnyKeys : 0;
    const int i_lo = shared ? 0 : split * nt / kAnyWaves;
    const int i_hi = shared ? nt : (split + 1) * nt / kAnyWaves;

    float m_run = -INFINITY;
    float lsum = 0.f;  // this lane's share of its row's sum of p (keys 4j .. 4j + 3 of each tile)
    f32x4 o[DB];
#pragma unroll
    for (int db = 0; db < DB; ++db) o[db] = f32x4{0.f, 0.f, 0.f, 0.f};

    // lane c holds tile i's key c: its page, then its slot
    auto key_pos = [&](int i) __attribute__((always_inline)) -> int {
      return min(key_lo + i * kAnyKeys + c, key_hi - 1);
    };
    auto page_load = [&](int i) __attribute__((always_inline)) -> int {
      return gptr(a.tt.table)[seq_row * a.tt.stride + (key_pos(i) >> a.tt.page_shift)];
    };
    // Loads are unconditional, so the compiler's wait counts stay exact (a load behind a
    // branch would make it wait for every load in flight): lanes past the head dim read the
    // row's last dims again. Those finite values meet Q's zeros in the scores and fill
    // output dims that are never stored.
    auto slot_of = [&](int i, int page) __attribute__((always_inline)) -> int {
      return (page << a.tt.page_shift) | (key_pos(i) & page_mask);
    };
    auto load_k = [&](int myslot, u32x4 (&kr)[kKL]) __attribute__((always_inline)) {
      const int kslot = shfl_i(myslot, c);
      const unsigned char MA_GLOBAL* krow = kbase + (int64_t)kslot * row_bytes + head_off;
#pragma unroll
      for (int x = 0; x < kKL; ++x) {
        const int d0 = min(kFp8 ? x * 64 + j * 16 : x * 32 + j * 8, D - (kFp8 ? 16 : 8));
        kr[x] = *reinterpret_cast<const u32x4 MA_GLOBAL*>(krow + d0 * kElt);
      }
    };
    auto load_v = [&](int myslot, VRaw (&vr)[kUL]) __attribute__((always_inline)) {
#pragma unroll
      for (int x = 0; x < kUL; ++x) {
        const int u = lane + 64 * x;
        const int tr = u / kUnits;
        const int q = min(u - tr * kUnits, D / 8 - 1);
        const int vs = shfl_i(myslot, tr);
        vr[x] = *reinterpret_cast<const VRaw MA_GLOBAL*>(vbase + (int64_t)vs * row_bytes + head_off + q * 8 * kElt);
      }
    };
    // V units -> fp16 -> this wave's LDS block, row-major with padded rows (the transposed
    // reads take 4 rows of one 32-byte column block per 16 lanes; the padding puts those
    // rows in different banks). Lane-constant base plus an immediate per unit.
    auto write_v = [&](const VRaw (&vr)[kUL]) __attribute__((always_inline)) {
      const uint32_t wa = lds_base + (lane / kUnits) * kRowL + (lane % kUnits) * 16;
#pragma unroll
      for (int x = 0; x < kUL; ++x) {
        u32x4 hv;
        if constexpr (kFp8) {
          hv = cvt8_fp8<KV, false>(vr[x][0], vr[x][1]);
        } else if constexpr (QBF16) {
#pragma unroll
          for (int w = 0; w < 4; ++w)
            hv[w] = pack_f16(__builtin_bit_cast(float, vr[x][w] << 16), __builtin_bit_cast(float, vr[x][w] & 0xffff0000u));
        } else {
          hv = vr[x];
        }
        *reinterpret_cast<__attribute__((address_space(3))) u32x4*>((uintptr_t)(wa + x * (64 / kUnits) * kRowL)) = hv;
      }
    };
    // scores of tile i: lane (c, j) holds keys 4j .. 4j + 3 of row c
    auto scores = [&](const u32x4 (&kr)[kKL]) __attribute__((always_inline)) -> f32x4 {
      f32x4 s = f32x4{0.f, 0.f, 0.f, 0.f};
      if constexpr (kFp8) {
#pragma unroll
        for (int x = 0; x < kKL; ++x) {
          u32x4 k0, k1;
          cvt16_fp8<KV, QBF16>(kr[x], k0, k1);
          s = mfma16t<QBF16>(k0, qv[2 * x], s);
          s = mfma16t<QBF16>(k1, qv[2 * x + 1], s);
        }
      } else {
#pragma unroll
        for (int kk = 0; kk < KK; ++kk) {
          if constexpr (kQLds) {
            const u32x4 qf = *reinterpret_cast<const __attribute__((address_space(3))) u32x4*>((uintptr_t)(qa + kk * 64));
            s = mfma16t<QBF16>(kr[kk], qf, s);
          } else
            s = mfma16t<QBF16>(kr[kk], qv[kk], s);
        }
      }
      return s;
    };
    // scores of tile i from a K tile in LDS (shared mode)
    // The operand reads run one batch of kFB steps ahead of the MFMAs; the scheduling
    // barriers keep the compiler from sinking each read down to its MFMA, which left every
    // MFMA waiting out a full LDS latency.
    auto scores_lds = [&](uint32_t kt) __attribute__((always_inline)) -> f32x4 {
      f32x4 s = f32x4{0.f, 0.f, 0.f, 0.f};
      const uint32_t ka0 = kt + c * kRowK + j * 16;
      constexpr int kFB = KK < 4 ? KK : 4;  // QK steps per batch
      constexpr int kNB = KK / kFB;
      u32x4 kf[2][kFB], qf[2][kFB];
      auto fetch = [&](int bb, int sl) __attribute__((always_inline)) {
#pragma unroll
        for (int x = 0; x < kFB; ++x) {
          const int kk = bb * kFB + x;
          kf[sl][x] = *reinterpret_cast<const __attribute__((address_space(3))) u32x4*>((uintptr_t)(ka0 + kk * 64));
          if constexpr (kQLds)
            qf[sl][x] = *reinterpret_cast<const __attribute__((address_space(3))) u32x4*>((uintptr_t)(qa + kk * 64));
        }
      };
      fetch(0, 0);
#pragma unroll
      for (int bb = 0; bb < kNB; ++bb) {
        if (bb + 1 < kNB) fetch(bb + 1, (bb + 1) & 1);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int x = 0; x < kFB; ++x) {
          if constexpr (kQLds) s = mfma16t<QBF16>(kf[bb & 1][x], qf[bb & 1][x], s);
          else s = mfma16t<QBF16>(kf[bb & 1][x], qv[bb * kFB + x], s);
        }
        __builtin_amdgcn_sched_barrier(0);
      }
      return s;
    };
    // softmax and PV of tile i (its V in LDS at vt)
    auto finish = [&](int i, f32x4 s, uint32_t vt) __attribute__((always_inline)) {
      const int kb0 = key_lo + i * kAnyKeys + 4 * j;
#pragma unroll
      for (int e = 0; e < 4; ++e)
        if (kb0 + e < lo_r || kb0 + e >= hi_r) s[e] = -INFINITY;
      float mx = fmaxf(fmaxf(s[0], s[1]), fmaxf(s[2], s[3]));
      // the exponent base moves only when some row's max grew by more than 2^kLazyRescale in p
      if (__builtin_amdgcn_ballot_w64((mx - m_run) * a.scale_log2 > kLazyRescale)) {
        mx = fmaxf(mx, shfl_xor_f(mx, 16));
        mx = fmaxf(mx, shfl_xor_f(mx, 32));
        const float m_new = fmaxf(m_run, mx);
        const float m_use = (m_new == -INFINITY) ? 0.f : m_new;
        const float alpha = __builtin_amdgcn_exp2f((m_run - m_use) * a.scale_log2);
        m_run = m_new;
#pragma unroll
        for (int db = 0; db < DB; ++db) o[db] *= alpha;
        lsum *= alpha;
      }
      const float msc = (m_run == -INFINITY ? 0.f : m_run) * a.scale_log2;
      float p[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) p[e] = __builtin_amdgcn_exp2f(s[e] * a.scale_log2 - msc);
      lsum += (p[0] + p[1]) + (p[2] + p[3]);
      const u32x2 pk = u32x2{pack_f16(p[0], p[1]), pack_f16(p[2], p[3])};
      // O^T[d][row] += V^T[d][key] P^T[key][row], 16 dims per step; the transposed V reads
      // run one batch of kVB steps ahead, as in the scores
      const uint32_t vb = vt + (4 * j + (c >> 2)) * kRowL + (c & 3) * 8;
      constexpr int kVB = DB < 8 ? DB : 8;
      constexpr int kVNB = DB / kVB;
      u32x2 vf[2][kVB];
      auto vfetch = [&](int bb, int sl) __attribute__((always_inline)) {
#pragma unroll
        for (int x = 0; x < kVB; ++x)
          vf[sl][x] = __builtin_bit_cast(u32x2, __builtin_amdgcn_ds_read_tr16_b64_v4i16(
              (__attribute__((address_space(3))) i16x4*)(uintptr_t)(vb + (bb * kVB + x) * 32)));
      };
      vfetch(0, 0);
#pragma unroll
      for (int bb = 0; bb < kVNB; ++bb) {
        if (bb + 1 < kVNB) vfetch(bb + 1, (bb + 1) & 1);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int x = 0; x < kVB; ++x)
          o[bb * kVB + x] = __builtin_amdgcn_mfma_f32_16x16x16f16(
              __builtin_bit_cast(f16x4, vf[bb & 1][x]), __builtin_bit_cast(f16x4, pk), o[bb * kVB + x], 0, 0, 0);
        __builtin_amdgcn_sched_barrier(0);
      }
    };

    if (shared && nt > 0) {
      // The workgroup's tile ring. Step i writes tile i+1 (loaded during step i-1) to stage
      // (i+1) % 2, loads tile i+2, computes tile i from stage i % 2, then meets the other
      // waves: the barrier publishes stage (i+1) % 2 and retires stage i % 2. Tiles past
      // the last are the last again (key positions clamp), every load is unconditional.
      u32x4 kraw0[kUW], kraw1[kUW];
      VRaw vraw0[kUW], vraw1[kUW];
      auto load_units = [&](int myslot, u32x4 (&kraw)[kUW], VRaw (&vraw)[kUW]) __attribute__((always_inline)) {
#pragma unroll
        for (int x = 0; x < kUW; ++x) {
          const int u = min((int)threadIdx.x + kAnyWaves * 64 * x, kTileUnits - 1);
          const int key = u / kUnits;
          const int q = min(u - key * kUnits, D / 8 - 1);
          const int64_t off = (int64_t)shfl_i(myslot, key) * row_bytes + head_off + q * 8 * kElt;
          if constexpr (kFp8) {
            const u32x2 w = *reinterpret_cast<const u32x2 MA_GLOBAL*>(kbase + off);
            kraw[x] = u32x4{w[0], w[1], 0u, 0u};
          } else {
            kraw[x] = *reinterpret_cast<const u32x4 MA_GLOBAL*>(kbase + off);
          }
          vraw[x] = *reinterpret_cast<const VRaw MA_GLOBAL*>(vbase + off);
        }
      };
      auto write_units = [&](uint32_t st, const u32x4 (&kraw)[kUW], const VRaw (&vraw)[kUW]) __attribute__((always_inline)) {
#pragma unroll
        for (int x = 0; x < kUW; ++x) {
          const int u = (int)threadIdx.x + kAnyWaves * 64 * x;
          if (kTileUnits % (kAnyWaves * 64) == 0 || u < kTileUnits) {
            const int key = u / kUnits;
            const int q = u - key * kUnits;
            u32x4 kh, vh;
            if constexpr (kFp8) {
              kh = cvt8_fp8<KV, QBF16>(kraw[x][0], kraw[x][1]);
              vh = cvt8_fp8<KV, false>(vraw[x][0], vraw[x][1]);
            } else {
              kh = kraw[x];
              if constexpr (QBF16) {
#pragma unroll
                for (int w = 0; w < 4; ++w)
                  vh[w] = pack_f16(__builtin_bit_cast(float, vraw[x][w] << 16),
                                   __builtin_bit_cast(float, vraw[x][w] & 0xffff0000u));
              } else {
                vh = vraw[x];
              }
            }
            *reinterpret_cast<__attribute__((address_space(3))) u32x4*>((uintptr_t)(st + key * kRowK + q * 16)) = kh;
            *reinterpret_cast<__attribute__((address_space(3))) u32x4*>((uintptr_t)(st + kKTile + key * kRowL + q * 16)) = vh;
          }
        }
      };
      auto stage = [&](int i) -> uint32_t { return smem_base + (i & 1) * kStageB; };
      // tile t's raw units live in buffer t % 2 from the step that loads them (t - 3) to
      // the step that writes them to LDS (t - 1): two tiles' compute to land in
      int pg = page_load(0);
      load_units(slot_of(0, pg), kraw0, vraw0);
      pg = page_load(1);
      load_units(slot_of(1, pg), kraw1, vraw1);
      pg = page_load(2);
      write_units(stage(0), kraw0, vraw0);
      load_units(slot_of(2, pg), kraw0, vraw0);
      pg = page_load(3);
      __syncthreads();
      auto tile_step = [&](int i, u32x4 (&kn)[kUW], VRaw (&vn)[kUW]) __attribute__((always_inline)) {
        write_units(stage(i + 1), kn, vn);       // tile i+1, buffer (i+1) % 2
        // the next page lookup goes out before the unit loads, so the step that uses it
        // waits for it alone, not for the units behind it
        const int pn = page_load(i + 4);
        load_units(slot_of(i + 3, pg), kn, vn);  // tile i+3 into the buffer just written
        pg = pn;
        finish(i, scores_lds(stage(i)), stage(i) + kKTile);
        __syncthreads();
      };
#pragma unroll 1
      for (int i = 0; i < nt; i += 2) {
        tile_step(i, kraw1, vraw1);
        if (i + 1 < nt) tile_step(i + 1, kraw0, vraw0);
      }
    }
    if (!shared && i_hi > i_lo) {
      // Step i issues the slot lookup of tile i+2, writes tile i's V to LDS and refills the
      // V registers with tile i+1, and loads tile i+1's K (into the other K buffer, or at
      // the widest head dims into the same one once tile i's scores have used it), so every
      // load has a tile's softmax and PV to land in. Tiles past the last are the last again
      // (key positions clamp), so every step issues the same loads on every path.
      constexpr bool kTwoK = DP <= 256;
      u32x4 ka[kKL], kb[kKL];
      VRaw vr[kUL];
      int page1 = page_load(i_lo);
      load_v(slot_of(i_lo, page1), vr);
      load_k(slot_of(i_lo, page1), ka);
      page1 = page_load(i_lo + 1);
      int page2;
      auto step = [&](int i, u32x4 (&kc)[kKL], u32x4 (&kn)[kKL]) __attribute__((always_inline)) {
        page2 = page_load(i + 2);
        write_v(vr);
        const int sn = slot_of(i + 1, page1);
        load_v(sn, vr);
        f32x4 s;
        if constexpr (kTwoK) {
          load_k(sn, kn);
          s = scores(kc);
        } else {
          s = scores(kc);
          load_k(sn, kc);
        }
        finish(i, s, lds_base);
        page1 = page2;
      };
#pragma unroll 1
      for (int i = i_lo; i < i_hi; i += 2) {
        if constexpr (kTwoK) {
          step(i, ka, kb);
          if (i + 1 < i_hi) step(i + 1, kb, ka);
        } else {
          step(i, ka, ka);
          if (i + 1 < i_hi) step(i + 1, ka, ka);
        }
      }
    }

    // normalise and store this lane's row: dims db * 16 + 4j .. + 3
    float lt = lsum + shfl_xor_f(lsum, 16);
    lt += shfl_xor_f(lt, 32);
    const int64_t off = (int64_t)(tok0 + t) * a.out_stride_tok + (int64_t)(h * G + g) * a.out_stride_head;
    if (shared) {
      if (real) {
        const float inv = (lt > 0.f) ? a.v_scale / lt : 0.f;
#pragma unroll
        for (int db = 0; db < DB; ++db) {
          if (db * 16 >= D) break;
          store_out4<QBF16>(a.out, off + db * 16 + 4 * j, o[db], inv, a.out_f32);
        }
      }
      return;
    }
    // merge of the four quarters: each O and row sum is relative to its wave's exponent
    // base (its row max, 0 when it saw no key), rescaled to the largest
    if (j == 0) {
      mrow[wave][0][c] = m_run;
      mrow[wave][1][c] = lt;
    }
    __syncthreads();  // every wave is done with its V/Q memory, which the merge reuses
    float mmax = -INFINITY;
#pragma unroll
    for (int u = 0; u < kAnyWaves; ++u) mmax = fmaxf(mmax, mrow[u][0][c]);
    float sc[kAnyWaves];
    float ltot = 0.f;
#pragma unroll
    for (int u = 0; u < kAnyWaves; ++u) {
      const float mu = mrow[u][0][c];
      sc[u] = (mu == -INFINITY) ? 0.f : __builtin_amdgcn_exp2f((mu - mmax) * a.scale_log2);
      ltot += mrow[u][1][c] * sc[u];
    }
    const float inv = (ltot > 0.f) ? a.v_scale / ltot : 0.f;
#pragma unroll
    for (int r = 0; r < DB; r += kBPR) {
#pragma unroll
      for (int blk = 0; blk < kBPR; ++blk)
        *reinterpret_cast<__attribute__((address_space(3))) f32x4*>(
            (uintptr_t)(smem_base + ((wave * kBPR + blk) * 64 + lane) * 16)) = o[r + blk];
      __syncthreads();
      // this wave finishes the round's blocks wave, wave + 4, ...
      for (int blk = wave; blk < kBPR; blk += kAnyWaves) {
        f32x4 acc = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int u = 0; u < kAnyWaves; ++u)
          acc += *reinterpret_cast<const __attribute__((address_space(3))) f32x4*>(
                     (uintptr_t)(smem_base + ((u * kBPR + blk) * 64 + lane) * 16)) * sc[u];
        if (real && (r + blk) * 16 < D) store_out4<QBF16>(a.out, off + (r + blk) * 16 + 4 * j, acc, inv, a.out_f32);
      }
      __syncthreads();  // before the next round (or the next row block) reuses the memory
    }
  };

  if (a.items) {
    // one 128-row work-list entry per workgroup and kv head, in two passes of 64 rows
    const int entry = (int)blockIdx.x / a.hkv;
    const int h = (int)blockIdx.x - entry * a.hkv;
    const int64_t work = cptr(a.items)[entry];
    const int b = (int)(uint32_t)work;
    if (b < 0) return;
    const int rt = (int)(work >> 32);
#pragma unroll 1
    for (int pass = 0; pass < kAnyPlanRows / (kAnyWaves * kAnyRows); ++pass)
      rows(b, h, rt * kAnyPlanRows + pass * (kAnyWaves * kAnyRows) + wave * kAnyRows, -1);
  } else {
    // decode and verify: workgroup item = (kv head, 16-row block, sequence), kv head
    // fastest; its four waves take the four quarters of the rows' key tiles. A sequence
    // with more rows than row_blocks blocks has its later blocks taken in turn.
    const int64_t item = blockIdx.x;
    const int h = (int)(item % a.hkv);
    const int64_t rest = item / a.hkv;
    const int b = (int)(rest / a.row_blocks);
    const int rb = (int)(rest - (int64_t)b * a.row_blocks);
    if (b >= a.batch) return;
    int rows_b;
    if (a.qsl) rows_b = clamp_query_rows(cptr(a.qsl)[b], cptr(a.qsl)[b + 1], a.num_tokens).ntok * a.group;
    else rows_b = (b < a.num_tokens ? 1 : 0) * a.group;
#pragma unroll 1
    for (int r0 = rb * kAnyRows; r0 < rows_b; r0 += a.row_blocks * kAnyRows) rows(b, h, r0, wave);
  }
}

template <int DP, bool QBF16>
static hipError_t launch_any_q(int kv, dim3 grid, hipStream_t st, const AnyArgs& a) {
  if (kv == DT_E4M3)
    hipLaunchKernelGGL((any_kernel<DP, QBF16, DT_E4M3>), grid, dim3(kAnyWaves * 64), 0, st, a);
  else if (kv == DT_E5M2)
    hipLaunchKernelGGL((any_kernel<DP, QBF16, DT_E5M2>), grid, dim3(kAnyWaves * 64), 0, st, a);
  else
    hipLaunchKernelGGL((any_kernel<DP, QBF16, QBF16 ? DT_BF16 : DT_F16>), grid, dim3(kAnyWaves * 64), 0, st, a);
  return hipGetLastError();
}

template <int DP>
static hipError_t launch_any_d(bool qbf16, int kv, dim3 grid, hipStream_t st, const AnyArgs& a) {
  return qbf16 ? launch_any_q<DP, true>(kv, grid, st, a) : launch_any_q<DP, false>(kv, grid, st, a);
}

hipError_t any_launch(const AnyArgs& a, int q_dtype, int kv_dtype, int64_t grid_x, hipStream_t st) {
  if (grid_x <= 0) return hipSuccess;
  const dim3 grid((unsigned)grid_x);
  const bool qbf16 = q_dtype == DT_BF16;
  const int d = a.head_dim;
  return d <= 64    ? launch_any_d<64>(qbf16, kv_dtype, grid, st, a)
         : d <= 128 ? launch_any_d<128>(qbf16, kv_dtype, grid, st, a)
         : d <= 256 ? launch_any_d<256>(qbf16, kv_dtype, grid, st, a)
                    : launch_any_d<512>(qbf16, kv_dtype, grid, st, a);
}

}  // namespace ma
