// Paged attention at the head dims the tuned kernels do not take: every multiple of 16
// from 16 to 512 other than 64, 128 and 256 (the reference's paged kernels take any head
// dim, with a default tile configuration and a tuned one for 512:
// sglang_restomod/attention/v100/tilelang/_kernels_paged.py:397-418; above 256 its linear
// verify also runs on the ordinary paged kernel, _paged_adapter.py:612-616).
//
// One kernel family serves decode, linear verify and extend rows. A wave computes the
// scores of 16 query rows (token, GQA head) of one sequence and kv head, 16 keys at a
// time:
//   - scores S^T = K Q^T on 16x16x32 MFMAs (the query's 16-bit type; fp8 K converted),
//     so each lane holds four keys of one row: the B operand of the 16x16x16 fp16 MFMA
//     of O^T += V^T P^T, whose A operand is read transposed (ds_read_b64_tr_b16) from
//     fp16 V rows in LDS,
//   - an online softmax with the tuned kernels' lazy rescale (kLazyRescale).
// Decode and verify (no work list): the four waves of a workgroup hold the same 16 rows
// and take a quarter of their 16-key tiles each, K straight into operand registers and V
// through the wave's own LDS rows, then merge through LDS. Extend (the work list, its own
// instantiation): the four waves hold 64 consecutive rows and share each K/V tile (32
// keys up to 128 dims, else 16) through a three-stage LDS ring; each wave publishes its
// rows' P and accumulates O for a quarter of the dims of all 64 rows, one barrier per
// tile.
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

// the mode of one call of the row routine, fixed at compile time
template <bool SHARED>
struct AnyMode {
  static constexpr bool shared = SHARED;
};
// a register buffer index, fixed at compile time
template <int N>
struct AnyIdx {
  static constexpr int v = N;
};

// SHARED: the extend kernel (work list, shared K/V ring); otherwise decode and verify
// (split keys). Two workgroups share a CU where the registers allow it.
template <bool SHARED, int DP>
constexpr int any_wg_per_cu() {
  return (DP >= 512 || (DP >= 256 && !SHARED)) ? 1 : 2;
}

template <int DP, bool QBF16, int KV, bool SHARED>
__global__ __launch_bounds__(kAnyWaves * 64, (any_wg_per_cu<SHARED, DP>())) void any_kernel(const AnyArgs args) {
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

  // Decode and verify at the widest head dim with fp16 Q and KV keep Q in LDS (rows padded
  // by 16 bytes so the 16 rows of an operand read fall in different banks): in registers
  // it spilled. bf16 and fp8 KV, and extend, keep Q in registers (1-3% faster at D=320
  // and 512 than reading it from LDS every tile).
  constexpr bool kQLds = DP >= 512 && !kFp8 && !QBF16;
  constexpr int kQRow = DP * 2 + 16;
  constexpr int kVBlock = kAnyKeys * kRowL;            // one wave's V rows
  constexpr int kQBlock = kQLds ? kAnyRows * kQRow : 0;  // one wave's Q rows
  // Extend rows: the four waves own 64 consecutive rows of one sequence and kv head and
  // share every K/V tile (kKT keys: 32 up to 128 dims, else 16) through a three-stage LDS
  // ring (16-bit K rows padded by 32 bytes, V rows padded as above: fp16, or bf16 that
  // becomes fp16 as its fragments are read), loaded once per workgroup; kUW 16-byte
  // units per thread. Each wave computes the scores and softmax of its own 16 rows, and
  // O for a quarter of the dims (kCB 16-dim blocks) of all 64 rows: P, the rescale
  // factors and their flags pass through the exchange memory behind the ring (two tiles
  // deep). Decode and verify tiles have 16 keys.
  constexpr int kKT = (SHARED && DP <= 128) ? 2 * kAnyKeys : kAnyKeys;
  constexpr int kNS = kKT / kAnyKeys;  // 16-key score blocks per tile
  // K row pitch: 32 bytes of padding. With 16, the score reads of the D = 512 extend batch
  // took 139 million bank-conflict cycles per launch (a quarter of the LDS's active
  // cycles); with 32, none, and the kernel ran 3.7% faster.
  constexpr int kRowK = DP * 2 + 32;
  constexpr int kKTile = kKT * kRowK;
  constexpr int kStageB = kKTile + kKT * kRowL;
  constexpr int kTileUnits = kKT * kUnits;  // 16-byte units of one K (or V) tile
  constexpr int kUW = kTileUnits >= kAnyWaves * 64 ? kTileUnits / (kAnyWaves * 64) : 1;
  constexpr int kCB = DB / kAnyWaves;
  static_assert(kCB >= 1 && DB % kAnyWaves == 0, "whole dim blocks per wave");
  constexpr int kXP = 0;                                   // P: [tile & 1][wave][block][lane] u32x2
  constexpr int kXA = kXP + 2 * kAnyWaves * kNS * 64 * 8;  // factors: [tile & 1][wave][row] f32
  constexpr int kXF = kXA + 2 * kAnyWaves * kAnyRows * 4;  // flags: [tile & 1][wave] u32
  constexpr int kXBytes = kXF + 2 * kAnyWaves * 4;
  constexpr int kRing = 3 * kStageB;
  constexpr int kSmem = SHARED ? kRing + kXBytes : kAnyWaves * (kVBlock + kQBlock);
  // When the four waves split one row block's keys, their partial O meet in the same
  // memory after the loop, kBPR 16-column blocks (1 KiB per wave each) at a time.
  constexpr int kBPR = (DB * kAnyWaves * 1024 <= kSmem) ? DB
                       : (DB / 2 * kAnyWaves * 1024 <= kSmem) ? DB / 2
                       : (DB / 4 * kAnyWaves * 1024 <= kSmem) ? DB / 4 : DB / 8;
  static_assert(kBPR >= 1 && kBPR * kAnyWaves * 1024 <= kSmem, "merge rounds fit the kernel's LDS");
  __shared__ __attribute__((aligned(256))) unsigned char smem[kSmem];
  __shared__ float mrow[kAnyWaves][2][kAnyRows];  // each wave's row max and row sum of p
  int64_t piece_slot = 0;  // decode with pieces > 1: where this workgroup's partial goes

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
  const uint32_t row_bytes32 = (uint32_t)(a.kv_stride_row * kElt);  // the hosts check it fits
  const int page_mask = (1 << a.tt.page_shift) - 1;

  // One wave's 16 rows r0 .. r0 + 15 of sequence b, kv head h. Shared mode: the
  // workgroup's four waves own consecutive row blocks (rows r0 - 16 * wave ..) and walk the
  // keys any of them sees together, sharing each K/V tile. Otherwise the four waves own the
  // same row block and take quarter `split` of its key tiles each, merging at the end.
  auto rows = [&](auto mode, int b, int h, int r0, int split) __attribute__((always_inline)) {
    constexpr bool shared = decltype(mode)::shared;
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
    constexpr bool kQInLds = kQLds && !shared;  // shared mode keeps Q in registers
    u32x4 qv[kQInLds ? 1 : KK];
    const uint32_t qa = q_base + c * kQRow + j * 16;
    {
      const uint16_t MA_GLOBAL* qp = gptr(reinterpret_cast<const uint16_t*>(a.q)) +
                                     (int64_t)(tok0 + (real ? t : 0)) * a.q_stride_tok +
                                     (int64_t)(h * G + g) * a.q_stride_head;
#pragma unroll
      for (int kk = 0; kk < KK; ++kk) {
        const int d0 = shared ? kk * 32 + j * 8 : qdim(kk);
        const u32x4 qf = (real && d0 < D) ? *reinterpret_cast<const u32x4 MA_GLOBAL*>(qp + d0) : u32x4{0, 0, 0, 0};
        if constexpr (kQInLds) *reinterpret_cast<__attribute__((address_space(3))) u32x4*>((uintptr_t)(qa + kk * 64)) = qf;
        else qv[kk] = qf;
      }
    }
    // keys any of the rows (the wave's, or the workgroup's in shared mode) may see
    const int t_first = rg0 / G;
    const int t_last = min(ntok - 1, (rg0 + rgn - 1) / G);
    const int key_lo = a.window >= 0 ? max(0, prefix + t_first - a.window) : 0;
    const int key_hi = a.causal ? min(seq, prefix + t_last + 1) : seq;
    const int nt = key_hi > key_lo ? (key_hi - key_lo + kKT - 1) / kKT : 0;
    // split: this wave's quarter of the workgroup's key piece (pieces x 4 equal shares)
    const int parts = kAnyWaves * a.pieces;
    const int i_lo = shared ? 0 : (int)((int64_t)split * nt / parts);
    const int i_hi = shared ? nt : (int)((int64_t)(split + 1) * nt / parts);

    float m_run = -INFINITY;
    float lsum = 0.f;  // this lane's share of its row's sum of p (keys 4j .. 4j + 3 of each tile)
    f32x4 o[DB];
#pragma unroll
    for (int db = 0; db < DB; ++db) o[db] = f32x4{0.f, 0.f, 0.f, 0.f};

    // lane l holds tile i's key l % kKT: its page, then its slot
    auto key_pos = [&](int i) __attribute__((always_inline)) -> int {
      return min(key_lo + i * kKT + (lane & (kKT - 1)), key_hi - 1);
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
      const unsigned char MA_GLOBAL* krow = kbase + (uint64_t)(uint32_t)kslot * row_bytes32 + head_off;
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
        vr[x] = *reinterpret_cast<const VRaw MA_GLOBAL*>(vbase + (uint64_t)(uint32_t)vs * row_bytes32 + head_off + q * 8 * kElt);
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
          if constexpr (kQInLds) {
            const u32x4 qf = *reinterpret_cast<const __attribute__((address_space(3))) u32x4*>((uintptr_t)(qa + kk * 64));
            s = mfma16t<QBF16>(kr[kk], qf, s);
          } else
            s = mfma16t<QBF16>(kr[kk], qv[kk], s);
        }
      }
      return s;
    };
    // scores of tile i from a K tile in LDS (shared mode, Q in registers)
    // The operand reads run one batch of kFB steps ahead of the MFMAs; the scheduling
    // barriers keep the compiler from sinking each read down to its MFMA, which left every
    // MFMA waiting out a full LDS latency.
    auto scores_lds = [&](uint32_t kt) __attribute__((always_inline)) -> f32x4 {
      f32x4 s2[2] = {f32x4{0.f, 0.f, 0.f, 0.f}, f32x4{0.f, 0.f, 0.f, 0.f}};  // two MFMA chains
      const uint32_t ka0 = kt + c * kRowK + j * 16;
      constexpr int kFB = KK < 4 ? KK : 4;  // QK steps per batch
      constexpr int kNB = KK / kFB;
      u32x4 kf[2][kFB];
      auto fetch = [&](int bb, int sl) __attribute__((always_inline)) {
#pragma unroll
        for (int x = 0; x < kFB; ++x)
          kf[sl][x] = *reinterpret_cast<const __attribute__((address_space(3))) u32x4*>((uintptr_t)(ka0 + (bb * kFB + x) * 64));
      };
      fetch(0, 0);
#pragma unroll
      for (int bb = 0; bb < kNB; ++bb) {
        if (bb + 1 < kNB) fetch(bb + 1, (bb + 1) & 1);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int x = 0; x < kFB; ++x) s2[x & 1] = mfma16t<QBF16>(kf[bb & 1][x], qv[bb * kFB + x], s2[x & 1]);
        __builtin_amdgcn_sched_barrier(0);
      }
      return s2[0] + s2[1];
    };
    // Online softmax of tile i's scores, kNS blocks of 16 keys (lane (c, j): keys
    // 16 sb + 4j .. + 3 of row c in block sb). Writes p in fp16; `moved` (the same in
    // every lane) says whether some row's exponent base moved, and then `alpha` is the
    // factor the row's earlier O takes (1 for the others). The base moves only when a
    // row's max grew by more than 2^kLazyRescale in p.
    auto softmax = [&](int i, f32x4 (&s)[kNS], u32x2 (&pk)[kNS], float& alpha, bool& moved) __attribute__((always_inline)) {
      float mx = -INFINITY;
#pragma unroll
      for (int sb = 0; sb < kNS; ++sb) {
        const int kb0 = key_lo + i * kKT + sb * kAnyKeys + 4 * j;
#pragma unroll
        for (int e = 0; e < 4; ++e)
          if (kb0 + e < lo_r || kb0 + e >= hi_r) s[sb][e] = -INFINITY;
        mx = fmaxf(mx, fmaxf(fmaxf(s[sb][0], s[sb][1]), fmaxf(s[sb][2], s[sb][3])));
      }
      alpha = 1.f;
      moved = __builtin_amdgcn_ballot_w64((mx - m_run) * a.scale_log2 > kLazyRescale) != 0;
      if (moved) {
        mx = fmaxf(mx, shfl_xor_f(mx, 16));
        mx = fmaxf(mx, shfl_xor_f(mx, 32));
        const float m_new = fmaxf(m_run, mx);
        const float m_use = (m_new == -INFINITY) ? 0.f : m_new;
        alpha = __builtin_amdgcn_exp2f((m_run - m_use) * a.scale_log2);
        m_run = m_new;
        lsum *= alpha;
      }
      const float msc = (m_run == -INFINITY ? 0.f : m_run) * a.scale_log2;
#pragma unroll
      for (int sb = 0; sb < kNS; ++sb) {
        float p[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) p[e] = __builtin_amdgcn_exp2f(s[sb][e] * a.scale_log2 - msc);
        lsum += (p[0] + p[1]) + (p[2] + p[3]);
        pk[sb] = u32x2{pack_f16(p[0], p[1]), pack_f16(p[2], p[3])};
      }
    };
    // softmax and PV of tile i in split mode (its V in this wave's LDS rows at vt)
    auto finish = [&](int i, f32x4 s, uint32_t vt) __attribute__((always_inline)) {
      float alpha;
      bool moved;
      f32x4 sa[kNS] = {s};
      u32x2 pka[kNS];
      softmax(i, sa, pka, alpha, moved);
      const u32x2 pk = pka[0];
      if (moved) {
#pragma unroll
        for (int db = 0; db < DB; ++db) o[db] *= alpha;
      }
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

    // LDS words of the shared mode's exchange memory
    const uint32_t xbase = smem_base + kRing;
    auto xp = [&](int i, int w, int sb) -> uint32_t { return xbase + kXP + (((i & 1) * kAnyWaves + w) * kNS + sb) * 512; };
    auto xa = [&](int i, int w) -> uint32_t { return xbase + kXA + ((i & 1) * kAnyWaves + w) * (kAnyRows * 4); };
    auto xf = [&](int i) -> uint32_t { return xbase + kXF + (i & 1) * (kAnyWaves * 4); };
    if (shared && nt > 0) {
      // The workgroup's tile ring. Step i writes tile i+1 (its units loaded kRB steps
      // earlier) to stage (i+1) % 3, loads tile i+kRB+1, computes the scores and softmax
      // of tile i from stage i % 3 and publishes P, then meets the other waves, then
      // accumulates PV for its dims from every wave's P. The barrier of step i publishes
      // stage (i+1) % 3 and tile i's P; stage (i+2) % 3, which step i+1 writes, was last
      // read before the barrier of step i-1, and so were the exchange words of tile i-2.
      // Tiles past the last are the last again (key positions clamp), every load is
      // unconditional.
      // tile t's raw units live in register buffer t % kRB from the step that loads them
      // (t - kRB - 1) to the step that writes them to LDS (t - 1): kRB tiles' compute to
      // land in (three at the widest head dim, where one wave per SIMD leaves the registers)
      constexpr int kRB = DP >= 512 ? 3 : 2;
      u32x4 kraw[kRB][kUW];
      VRaw vraw[kRB][kUW];
      auto load_units = [&](int myslot, u32x4 (&kraw)[kUW], VRaw (&vraw)[kUW]) __attribute__((always_inline)) {
#pragma unroll
        for (int x = 0; x < kUW; ++x) {
          const int u = min((int)threadIdx.x + kAnyWaves * 64 * x, kTileUnits - 1);
          const int key = u / kUnits;
          const int q = min(u - key * kUnits, D / 8 - 1);
          const int64_t off = (int64_t)((uint64_t)(uint32_t)shfl_i(myslot, key) * row_bytes32) + head_off + q * 8 * kElt;
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
              vh = vraw[x];  // bf16 V stays bf16 in LDS: its fragments are converted as read
            }
            *reinterpret_cast<__attribute__((address_space(3))) u32x4*>((uintptr_t)(st + key * kRowK + q * 16)) = kh;
            *reinterpret_cast<__attribute__((address_space(3))) u32x4*>((uintptr_t)(st + kKTile + key * kRowL + q * 16)) = vh;
          }
        }
      };
      auto stage = [&](int i) -> uint32_t { return smem_base + (uint32_t)(i % 3) * kStageB; };
      // Page lookups go out two steps before the units that use them: waiting for a lookup
      // then waits only for loads issued before it, which have had kRB steps to land. The
      // prologue issues its loads in the steps' order, so the loop starts with the load
      // counts its back edge brings.
      int pa = page_load(0);
      int pb = page_load(1);
      int pc = page_load(2);
#pragma unroll
      for (int t = 0; t < kRB; ++t) {
        load_units(slot_of(t, pa), kraw[t], vraw[t]);
        pa = pb;
        pb = pc;
        pc = page_load(t + 3);
      }
      write_units(stage(0), kraw[0], vraw[0]);
      load_units(slot_of(kRB, pa), kraw[0], vraw[0]);
      int pg1 = pb, pg2 = pc;  // the pages of tiles kRB + 1 and kRB + 2
      __syncthreads();
      // PV of tile t: the V^T fragments of this wave's kCB dim blocks (stage t % 3) meet
      // the P fragments of all four row blocks, after the rows whose exponent base moved
      // have taken their factor
      auto pv = [&](int t) __attribute__((always_inline)) {
        const uint32_t vb = stage(t) + kKTile + (4 * j + (c >> 2)) * kRowL + (c & 3) * 8 + wave * kCB * 32;
        u32x2 vf[kNS][kCB], pf[kNS][kAnyWaves];
#pragma unroll
        for (int sb = 0; sb < kNS; ++sb)
#pragma unroll
          for (int cb = 0; cb < kCB; ++cb)
            vf[sb][cb] = __builtin_bit_cast(u32x2, __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                (__attribute__((address_space(3))) i16x4*)(uintptr_t)(vb + sb * kAnyKeys * kRowL + cb * 32)));
        const u32x4 fl = *reinterpret_cast<const __attribute__((address_space(3))) u32x4*>((uintptr_t)xf(t));
#pragma unroll
        for (int sb = 0; sb < kNS; ++sb)
#pragma unroll
          for (int rb = 0; rb < kAnyWaves; ++rb)
            pf[sb][rb] = *reinterpret_cast<const __attribute__((address_space(3))) u32x2*>((uintptr_t)(xp(t, rb, sb) + lane * 8));
        if constexpr (QBF16 && !kFp8) {
          // bf16 V fragments to fp16 (each V element is read by one wave only, so this is
          // the same conversion count as converting the tile when it is written)
#pragma unroll
          for (int sb = 0; sb < kNS; ++sb)
#pragma unroll
            for (int cb = 0; cb < kCB; ++cb)
#pragma unroll
              for (int w = 0; w < 2; ++w)
                vf[sb][cb][w] = pack_f16(__builtin_bit_cast(float, vf[sb][cb][w] << 16),
                                         __builtin_bit_cast(float, vf[sb][cb][w] & 0xffff0000u));
        }
#pragma unroll
        for (int rb = 0; rb < kAnyWaves; ++rb) {
          if (__builtin_amdgcn_readfirstlane(fl[rb])) {
            const float al = *reinterpret_cast<const __attribute__((address_space(3))) float*>((uintptr_t)(xa(t, rb) + c * 4));
#pragma unroll
            for (int cb = 0; cb < kCB; ++cb) o[rb * kCB + cb] *= al;
          }
        }
#pragma unroll
        for (int sb = 0; sb < kNS; ++sb)
#pragma unroll
          for (int cb = 0; cb < kCB; ++cb)
#pragma unroll
            for (int rb = 0; rb < kAnyWaves; ++rb)
              o[rb * kCB + cb] = __builtin_amdgcn_mfma_f32_16x16x16f16(__builtin_bit_cast(f16x4, vf[sb][cb]),
                                                                       __builtin_bit_cast(f16x4, pf[sb][rb]),
                                                                       o[rb * kCB + cb], 0, 0, 0);
      };
      // Step i: the scores of tile i, then PV of tile i-1 (independent work for the MFMA
      // pipe while the scores land), then tile i's softmax, whose P the barrier publishes.
      auto tile_step = [&](int i, auto buf_t) __attribute__((always_inline)) {
        constexpr int cur = decltype(buf_t)::v;  // (i + 1) % kRB
        write_units(stage(i + 1), kraw[cur], vraw[cur]);  // tile i+1
        const int pn = page_load(i + kRB + 3);
        load_units(slot_of(i + kRB + 1, pg1), kraw[cur], vraw[cur]);  // into the buffer just written
        pg1 = pg2;
        pg2 = pn;
        float alpha;
        bool moved;
        f32x4 sc[kNS];
        u32x2 pk[kNS];
#pragma unroll
        for (int sb = 0; sb < kNS; ++sb) sc[sb] = scores_lds(stage(i) + sb * kAnyKeys * kRowK);
        if (i > 0) pv(i - 1);
        softmax(i, sc, pk, alpha, moved);
#pragma unroll
        for (int sb = 0; sb < kNS; ++sb)
          *reinterpret_cast<__attribute__((address_space(3))) u32x2*>((uintptr_t)(xp(i, wave, sb) + lane * 8)) = pk[sb];
        if (lane == 0) *reinterpret_cast<__attribute__((address_space(3))) uint32_t*>((uintptr_t)(xf(i) + wave * 4)) = moved;
        if (moved && j == 0) *reinterpret_cast<__attribute__((address_space(3))) float*>((uintptr_t)(xa(i, wave) + c * 4)) = alpha;
        __syncthreads();
      };
      // the last steps short of a whole round of buffers run after the loop, so the loop's
      // back edge is its only path to the next pass and the compiler's load counts stay
      // exact there
      int i = 0;
#pragma unroll 1
      for (; i + kRB - 1 < nt; i += kRB) {
        tile_step(i, AnyIdx<1 % kRB>{});
        tile_step(i + 1, AnyIdx<2 % kRB>{});
        if constexpr (kRB == 3) tile_step(i + 2, AnyIdx<0>{});
      }
      if (i < nt) tile_step(i, AnyIdx<1 % kRB>{});
      if constexpr (kRB == 3) {
        if (i + 1 < nt) tile_step(i + 1, AnyIdx<2 % kRB>{});
      }
      pv(nt - 1);
    }
    if (!shared && DP <= 128 && i_hi > i_lo) {
      // Up to 128 dims a tile is small and its compute short, so each wave keeps two tiles
      // in flight: step i issues the slot lookup of tile i+3, writes tile i's V to LDS,
      // loads tile i+2 into the buffers tile i-1 has left, and computes tile i. The
      // prologue issues its loads in the steps' order. Tiles past the last are the last
      // again (key positions clamp), so every step issues the same loads on every path.
      u32x4 kq[3][kKL];
      VRaw vq[3][kUL];
      const int pa = page_load(i_lo);
      const int pb = page_load(i_lo + 1);
      load_v(slot_of(i_lo, pa), vq[0]);
      load_k(slot_of(i_lo, pa), kq[0]);
      int pc = page_load(i_lo + 2);
      __builtin_amdgcn_sched_barrier(0);  // the lookup stays ahead of the loads after it
      load_v(slot_of(i_lo + 1, pb), vq[1]);
      load_k(slot_of(i_lo + 1, pb), kq[1]);
      auto step3 = [&](int i, auto cur_t) __attribute__((always_inline)) {
        constexpr int cur = decltype(cur_t)::v;
        constexpr int nx = (cur + 2) % 3;
        const int pn = page_load(i + 3);
        __builtin_amdgcn_sched_barrier(0);
        write_v(vq[cur]);
        const int sn = slot_of(i + 2, pc);
        load_v(sn, vq[nx]);
        load_k(sn, kq[nx]);
        finish(i, scores(kq[cur]), lds_base);
        pc = pn;
      };
      int i = i_lo;
#pragma unroll 1
      for (; i + 2 < i_hi; i += 3) {
        step3(i, AnyIdx<0>{});
        step3(i + 1, AnyIdx<1>{});
        step3(i + 2, AnyIdx<2>{});
      }
      if (i < i_hi) step3(i, AnyIdx<0>{});
      if (i + 1 < i_hi) step3(i + 1, AnyIdx<1>{});
    }
    if (!shared && DP > 128 && i_hi > i_lo) {
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
      int i = i_lo;
#pragma unroll 1
      for (; i + 1 < i_hi; i += 2) {
        if constexpr (kTwoK) {
          step(i, ka, kb);
          step(i + 1, kb, ka);
        } else {
          step(i, ka, ka);
          step(i + 1, ka, ka);
        }
      }
      if (i < i_hi) step(i, ka, kTwoK ? kb : ka);
    }

    // normalise and store: row sums first
    float lt = lsum + shfl_xor_f(lsum, 16);
    lt += shfl_xor_f(lt, 32);
    if constexpr (shared) {
      // Each row's owner publishes its sum of p (in the factor words of tile nt, whose last
      // readers were done before the barrier of step nt-1); this wave then stores its dims
      // of all 64 rows. The second barrier keeps the words until every wave has read them.
      if (j == 0) *reinterpret_cast<__attribute__((address_space(3))) float*>((uintptr_t)(xa(nt, wave) + c * 4)) = lt;
      __syncthreads();
      float ls[kAnyWaves];
#pragma unroll
      for (int rb = 0; rb < kAnyWaves; ++rb)
        ls[rb] = *reinterpret_cast<const __attribute__((address_space(3))) float*>((uintptr_t)(xa(nt, rb) + c * 4));
      __syncthreads();
#pragma unroll
      for (int rb = 0; rb < kAnyWaves; ++rb) {
        const int rr = rg0 + rb * kAnyRows + c;
        const int tr = rr / G;
        if (tr < ntok) {
          const int gr = rr - tr * G;
          const int64_t offr = (int64_t)(tok0 + tr) * a.out_stride_tok + (int64_t)(h * G + gr) * a.out_stride_head;
          const float inv = (ls[rb] > 0.f) ? a.v_scale / ls[rb] : 0.f;
#pragma unroll
          for (int cb = 0; cb < kCB; ++cb) {
            const int d0 = (wave * kCB + cb) * 16;
            if (d0 < D) store_out4<QBF16>(a.out, offr + d0 + 4 * j, o[rb * kCB + cb], inv, a.out_f32);
          }
        }
      }
      return;
    }
    const int64_t off = (int64_t)(tok0 + t) * a.out_stride_tok + (int64_t)(h * G + g) * a.out_stride_head;
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
    // one piece of several (pieces > 1): this workgroup's rows normalised over its keys,
    // in fp32, and their log2 LSE, for the merge kernel; every row is written (a row that
    // saw no key gets O = 0 and LSE -inf)
    const bool piece_out = a.pieces > 1;
    float MA_GLOBAL* po = nullptr;
    if (piece_out) {
      po = gptr_mut(a.part_o) + (int64_t)piece_slot * (16 * DP) + c * DP + 4 * j;
      if (wave == 0 && j == 0)
        gptr_mut(a.part_lse)[(int64_t)piece_slot * 16 + c] =
            (ltot > 0.f) ? __builtin_amdgcn_logf(ltot) + mmax * a.scale_log2 : -INFINITY;
    }
    const float pinv = (ltot > 0.f) ? 1.f / ltot : 0.f;
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
        if (piece_out)
          *reinterpret_cast<f32x4 MA_GLOBAL*>(po + (r + blk) * 16) = acc * pinv;
        else if (real && (r + blk) * 16 < D)
          store_out4<QBF16>(a.out, off + (r + blk) * 16 + 4 * j, acc, inv, a.out_f32);
      }
      __syncthreads();  // before the next round (or the next row block) reuses the memory
    }
  };

  if constexpr (SHARED) {
    // one 128-row work-list entry per workgroup and kv head, in two passes of 64 rows
    const int entry = (int)blockIdx.x / a.hkv;
    const int h = (int)blockIdx.x - entry * a.hkv;
    const int64_t work = cptr(a.items)[entry];
    const int b = (int)(uint32_t)work;
    if (b < 0) return;
    const int rt = (int)(work >> 32);
#pragma unroll 1
    for (int pass = 0; pass < kAnyPlanRows / (kAnyWaves * kAnyRows); ++pass)
      rows(AnyMode<true>{}, b, h, rt * kAnyPlanRows + pass * (kAnyWaves * kAnyRows) + wave * kAnyRows, -1);
  } else {
    // decode and verify: workgroup = (kv head, key piece, 16-row block, sequence), kv head
    // fastest; its four waves take the four quarters of its piece of the rows' key tiles.
    // A sequence with more rows than row_blocks blocks has its later blocks taken in turn
    // (verify, whose calls have one piece).
    const int64_t item = blockIdx.x;
    const int h = (int)(item % a.hkv);
    const int64_t rest = item / a.hkv;
    const int piece = (int)(rest % a.pieces);
    const int64_t blk_item = rest / a.pieces;
    const int b = (int)(blk_item / a.row_blocks);
    const int rb = (int)(blk_item - (int64_t)b * a.row_blocks);
    if (b >= a.batch) return;
    piece_slot = (blk_item * a.hkv + h) * a.pieces + piece;
    int rows_b;
    if (a.qsl) rows_b = clamp_query_rows(cptr(a.qsl)[b], cptr(a.qsl)[b + 1], a.num_tokens).ntok * a.group;
    else rows_b = (b < a.num_tokens ? 1 : 0) * a.group;
#pragma unroll 1
    for (int r0 = rb * kAnyRows; r0 < rows_b; r0 += a.row_blocks * kAnyRows)
      rows(AnyMode<false>{}, b, h, r0, piece * kAnyWaves + wave);
  }
}

// Merge of the key pieces of a decode (pieces > 1): one workgroup per (sequence, 16-row
// block, kv head), 16 threads per row, each thread four dims of every 64. The row's 16
// threads read the pieces' log2 LSEs 16 at a time and reduce them across lanes, so every
// load of a round is in flight together; a piece's weight is 2^(lse - max), and its O
// chunks are then read eight pieces at a time. Pieces that saw no key have weight 0.
template <int DP, bool QBF16>
__global__ __launch_bounds__(256) void any_merge(const AnyArgs args) {
  const AnyArgs a = args;
  constexpr int kNC = DP / 64;  // f32x4 chunks per thread
  const int item = (int)blockIdx.x;  // (b * row_blocks + rb) * hkv + h
  const int h = item % a.hkv;
  const int blk_item = item / a.hkv;
  const int b = blk_item / a.row_blocks;
  const int rb = blk_item - b * a.row_blocks;
  const int row = threadIdx.x >> 4;
  const int part = threadIdx.x & 15;
  const int lane16 = (threadIdx.x & 63) & ~15;  // first lane of this row's 16 in the wave
  const int R = rb * kAnyRows + row;  // decode: rows 0 .. G-1 of one token
  // the row's 16 threads stay together (rows are whole 16-lane groups of a wave)
  const bool live = b < a.batch && b < a.num_tokens && R < a.group;
  const int np = a.pieces;
  const int64_t slot0 = (int64_t)item * np;
  const float MA_GLOBAL* lse = gptr(a.part_lse) + slot0 * 16 + row;
  const float MA_GLOBAL* po = gptr(a.part_o) + slot0 * (16 * DP) + row * DP + part * 4;
  // 1. max LSE over the pieces: thread `part` reads pieces part, part + 16, ...
  float lv[4];  // up to 64 pieces per row in registers
  float m = -INFINITY;
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const int p = part + 16 * k;
    lv[k] = (live && p < np) ? lse[(int64_t)p * 16] : -INFINITY;
    m = fmaxf(m, lv[k]);
  }
  for (int p = part + 64; p < np; p += 16) m = fmaxf(m, live ? lse[(int64_t)p * 16] : -INFINITY);
#pragma unroll
  for (int d = 1; d < 16; d <<= 1) m = fmaxf(m, __shfl_xor(m, d, 64));
  // 2. weights of this thread's pieces and their sum over the row
  float wv[4];
  float wsum = 0.f;
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    wv[k] = (lv[k] == -INFINITY) ? 0.f : __builtin_amdgcn_exp2f(lv[k] - m);
    wsum += wv[k];
  }
  for (int p = part + 64; p < np; p += 16) {
    const float l = live ? lse[(int64_t)p * 16] : -INFINITY;
    wsum += (l == -INFINITY) ? 0.f : __builtin_amdgcn_exp2f(l - m);
  }
#pragma unroll
  for (int d = 1; d < 16; d <<= 1) wsum += __shfl_xor(wsum, d, 64);
  // 3. the weighted sum of the pieces' O, eight pieces' loads in flight at a time
  f32x4 acc[kNC];
#pragma unroll
  for (int x = 0; x < kNC; ++x) acc[x] = f32x4{0.f, 0.f, 0.f, 0.f};
  if (live && wsum > 0.f) {
    for (int p0 = 0; p0 < np; p0 += 8) {
      f32x4 ov[8][kNC];
      float w8[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        const int p = p0 + u;
        // the weight of piece p sits in lane (p % 16) of the row's group, register p / 16
        const int k = (p >> 4) & 3;
        const float wk = k == 0 ? wv[0] : k == 1 ? wv[1] : k == 2 ? wv[2] : wv[3];
        float w = __shfl(wk, lane16 + (p & 15), 64);
        if (p >= 64) {
          const float l = p < np ? lse[(int64_t)p * 16] : -INFINITY;
          w = (l == -INFINITY) ? 0.f : __builtin_amdgcn_exp2f(l - m);
        }
        w8[u] = p < np ? w : 0.f;
#pragma unroll
        for (int x = 0; x < kNC; ++x)
          ov[u][x] = (p < np && w8[u] > 0.f)
                         ? *reinterpret_cast<const f32x4 MA_GLOBAL*>(po + (int64_t)p * (16 * DP) + x * 64)
                         : f32x4{0.f, 0.f, 0.f, 0.f};
      }
#pragma unroll
      for (int u = 0; u < 8; ++u)
#pragma unroll
        for (int x = 0; x < kNC; ++x) acc[x] += ov[u][x] * w8[u];
    }
  }
  if (!live) return;
  const float inv = (wsum > 0.f) ? a.v_scale / wsum : 0.f;
  const int g = R;
  const int64_t off = (int64_t)b * a.out_stride_tok + (int64_t)(h * a.group + g) * a.out_stride_head;
#pragma unroll
  for (int x = 0; x < kNC; ++x) {
    const int d0 = x * 64 + part * 4;
    if (d0 < a.head_dim) store_out4<QBF16>(a.out, off + d0, acc[x], inv, a.out_f32);
  }
}

template <int DP, bool QBF16, bool SHARED>
static hipError_t launch_any_m(int kv, dim3 grid, hipStream_t st, const AnyArgs& a) {
  if (kv == DT_E4M3)
    hipLaunchKernelGGL((any_kernel<DP, QBF16, DT_E4M3, SHARED>), grid, dim3(kAnyWaves * 64), 0, st, a);
  else if (kv == DT_E5M2)
    hipLaunchKernelGGL((any_kernel<DP, QBF16, DT_E5M2, SHARED>), grid, dim3(kAnyWaves * 64), 0, st, a);
  else
    hipLaunchKernelGGL((any_kernel<DP, QBF16, QBF16 ? DT_BF16 : DT_F16, SHARED>), grid, dim3(kAnyWaves * 64), 0, st, a);
  return hipGetLastError();
}

template <int DP, bool QBF16>
static hipError_t launch_any_q(int kv, dim3 grid, hipStream_t st, const AnyArgs& a) {
  // extend rows reach this kernel above 256 dims only (the tiled extend kernels take the rest)
  if (a.items) {
    if constexpr (DP == 512) return launch_any_m<DP, QBF16, true>(kv, grid, st, a);
    else return hipErrorInvalidValue;
  }
  return launch_any_m<DP, QBF16, false>(kv, grid, st, a);
}

template <int DP>
static hipError_t launch_any_d(bool qbf16, int kv, dim3 grid, hipStream_t st, const AnyArgs& a) {
  hipError_t e = qbf16 ? launch_any_q<DP, true>(kv, grid, st, a) : launch_any_q<DP, false>(kv, grid, st, a);
  if (e != hipSuccess || a.pieces <= 1) return e;
  const dim3 mgrid(grid.x / (unsigned)a.pieces);
  if (qbf16) hipLaunchKernelGGL((any_merge<DP, true>), mgrid, dim3(256), 0, st, a);
  else hipLaunchKernelGGL((any_merge<DP, false>), mgrid, dim3(256), 0, st, a);
  return hipGetLastError();
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
