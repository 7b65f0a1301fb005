// Grouped split-KV attention for few query rows per sequence: decode (one row) and
// linear-chain target verify (a handful of draft rows under a causal mask).
//
// Replaces the reference's grouped decode partial + combine
// (sglang_restomod/attention/v100/tilelang/_kernels_paged_decode.py:41-312) and the
// grouped verify partial + combine (_kernels_paged_verify.py:52-433).
//
// Work decomposition (stream-K): the key axis of every (sequence, kv head, row group)
// "segment" is cut into 32-token tiles (16 for 16-bit KV at D = 256). All tiles of all
// segments form one list, and a persistent grid (one 4-wave workgroup per CU) hands
// every wave an equal, contiguous range of that list. A wave walks its range, keeps an online-softmax state per segment
// piece, writes the output directly when it covered a whole segment and a partial
// (normalised O + log2 LSE) when the segment continues in a neighbouring wave's range.
// Every wave gets at least kMinTiles tiles (small problems use fewer waves), so a segment
// is shared by few waves. Ragged lengths cost nothing in balance, and a wave leaves at
// most two partials: its first and its last piece.
//
// Merging: a shared segment ends in the first piece of the wave that holds its last
// tile. That wave writes a small descriptor (segment, first wave, slot) for it; every
// other wave writes an empty one. A second kernel with one wave per partial-kernel wave
// reads its descriptor and, for a shared segment, merges the pieces of the waves that
// shared it. The kernel boundary orders the partials before the merge (device-scope
// fences inside one kernel would write back and invalidate whole L2 caches while other
// waves still stream). Rows of sequences that see no key at all (no tile covers them)
// are zeroed during the initial scan.
//
// A row group is 16*NB query rows of one kv head: row R -> (query token R / G,
// GQA head R % G), so every head of a kv head is served from one read of its K/V.
//
// Per 32-token tile (MFMA 16x16x32, fp32 accumulate):
//   S^T[t, r] = K[t, :] . Q[r, :]     A = K rows straight from HBM in operand layout,
//                                     B = Q^T (registers, reloaded per segment).
//   O^T[d, r] += V^T[d, t] P^T[t, r]  P^T comes straight from the S^T accumulators; V is
//                                     written row-major into a per-wave LDS tile and read
//                                     back transposed (ds_read_b64_tr_b16 / _tr_b8).
//   bf16 V: P split into two bf16 halves (exact to ~16 bits); fp16 / fp8 V: fp16 P.
//
// Head dims 64, 128 and 256; the configuration measured and tuned is D = 128.
//
// Memory pipeline: K and V of up to S-1 tiles ahead are issued before a tile computes
// (S = 2 for 8 KB tiles: 16-bit KV at D = 128 and 256, fp8 at D = 256; 4 for smaller
// ones: fp8 at D = 128, D = 64); 16-bit KV at S >= 4 waits for all of them before the
// compute, the others keep them in flight through it.
// Every load instruction reads whole rows (1 KB: 64 / (row bytes / 16) rows) with the
// nontemporal hint, and lands them in a per-wave LDS ring by DMA (global_load_lds): V
// rows in row-major order, K rows with their 16-byte chunks permuted by lane so that the
// ring holds the swizzled layout the QK operand reads. Slots are looked up 2S-3 tiles
// ahead of compute. All of these are issued as inline assembly and waited for with
// explicit counts. The issue cursor clamps at the wave's last tile, so the pipelined
// loop has no data-dependent branches around loads and the counts stay exact.

#include <algorithm>
#include <mutex>
#include <type_traits>

#include "common.h"
#include "paged_any.h"

// MA_ASM_PIPELINE: the build verifies the generated code of this file for accesses to
// registers whose inline-assembly loads are still in flight.
#include "capi_internal.h"

namespace ma {

constexpr int kWaves = 4;
constexpr int kMaxRows = 32;  // 16 * NB, NB <= 2

// Keys per tile: 32, and 16 for 16-bit KV at D = 256, whose 32-key tile would take 33 of
// the 63 vector memory instructions a wave can have outstanding, and 16 KB of K plus 16 KB
// of V per wave and stage, one stage of LDS; with 16 keys two stages fit.
template <int D, bool FP8>
constexpr int kTileKeys() {
  return (D == 256 && !FP8) ? 16 : 32;
}
constexpr int kMinTiles = 2;  // least tiles per active wave
constexpr int kDescInts = 8;  // per wave: valid, sequence, kv head, row group, first wave, its slot

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
  const int32_t* prefix;     // [B] cached prefix per sequence, or null (seq_len - query count)
  int num_tokens;            // rows of q and out: query rows are clamped into [0, num_tokens)
  int batch, hq, hkv, group;
  int row_groups;            // row groups per (sequence, kv head) at the host's longest-chain hint
  int rows;                  // rows per row group (16 * NB)
  int causal, window;
  float scale_log2;          // softmax_scale * k_scale * log2(e)
  float v_scale;
  int nwaves;                // waves of the persistent grid
  int merge_split;           // merge workgroups per wave: 1, or one per row set of a row group
  int* desc;                 // [nwaves][kDescInts] shared segment ending in each wave's first piece
  float* part_o;             // [nwaves][2][kMaxRows][D]
  float* part_lse;           // [nwaves][2][kMaxRows]
  void* out;
  int64_t out_stride_tok, out_stride_head;  // elements of the output dtype
  int out_f32;                              // out holds fp32 (else the query dtype)
};

// Geometry of one sequence.
struct Geom {
  int b, seq, ntok, prefix, tok0, lo_min, span, nt, rg_real;
  int64_t seq_row;
};

// Loads go through the constant address space: with a wave-uniform `b` they become
// scalar loads (geom_u), with a per-lane `b` vector loads (scan over sequences).
// TS: log2 of the keys per tile (a constant of the partial kernel, see kTileKeys).
template <int TS>
__device__ __forceinline__ Geom geom(const SplitKVArgs& a, int b) {
  Geom g;
  g.b = b;
  g.seq = max(cptr(a.seq_lens)[b], 0);
  if (a.qsl) {
    const QueryRows qr = clamp_query_rows(cptr(a.qsl)[b], cptr(a.qsl)[b + 1], a.num_tokens);
    g.tok0 = qr.tok0;
    g.ntok = qr.ntok;
    g.prefix = a.prefix ? cptr(a.prefix)[b] : g.seq - g.ntok;
  } else {
    g.tok0 = b;
    g.ntok = 1;
    g.prefix = g.seq - 1;
  }
  g.lo_min = a.window >= 0 ? max(0, g.prefix - a.window) : 0;
  g.lo_min = min(g.lo_min, g.seq);
  g.span = g.seq - g.lo_min;
  g.nt = (g.span + (1 << TS) - 1) / (1 << TS);
  const int real_rows = max(g.ntok, 0) * a.group;
  g.rg_real = (int)(((int64_t)real_rows + a.rows - 1) / a.rows);  // every query row, whatever the host's hint
  g.seq_row = a.row_index ? cptr(a.row_index)[b] : (int64_t)b;
  return g;
}

template <int TS>
__device__ __forceinline__ Geom geom_u(const SplitKVArgs& a, int b) {
  return geom<TS>(a, __builtin_amdgcn_readfirstlane(b));
}

// tiles of sequence b over all its kv heads and row groups (64-bit: a verify sequence's
// row groups are not capped, so rows x keys can pass 2^31)
template <int TS>
__device__ __forceinline__ int64_t seq_work(const SplitKVArgs& a, int b) {
  const Geom g = geom<TS>(a, b);
  return (int64_t)g.nt * g.rg_real * a.hkv;
}

__device__ __forceinline__ int64_t shfl_up_i64(int64_t v, int delta) {
  const int lane = lane_id();
  const int src = (lane >= delta ? lane - delta : lane) << 2;
  const int lo = __builtin_amdgcn_ds_bpermute(src, (int)(uint32_t)v);
  const int hi = __builtin_amdgcn_ds_bpermute(src, (int)(v >> 32));
  return (int64_t)(((uint64_t)(uint32_t)hi << 32) | (uint32_t)lo);
}

__device__ __forceinline__ int64_t readlane_i64(int64_t v, int lane) {
  const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)v, lane);
  const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(v >> 32), lane);
  return (int64_t)(((uint64_t)hi << 32) | lo);
}

// Total tiles, and (when t >= 0) the sequence holding global tile t and t's offset in it.
template <int TS>
__device__ __forceinline__ void scan_work(const SplitKVArgs& a, int64_t t, int64_t& total, int& b_at, int64_t& off_at) {
  const int lane = lane_id();
  int64_t base = 0;
  b_at = -1;
  off_at = 0;
  for (int b0 = 0; b0 < a.batch; b0 += 64) {
    const int b = b0 + lane;
    const int64_t w = b < a.batch ? seq_work<TS>(a, b) : 0;
    int64_t inc = w;
#pragma unroll
    for (int m = 1; m < 64; m <<= 1) {
      const int64_t y = shfl_up_i64(inc, m);
      if (lane >= m) inc += y;
    }
    const int64_t chunk = readlane_i64(inc, 63);
    if (b_at < 0 && t >= 0 && base + chunk > t) {
      const uint64_t hit = __builtin_amdgcn_ballot_w64(base + inc > t);
      const int L = __builtin_ctzll(hit);
      b_at = b0 + L;
      off_at = t - (base + readlane_i64(inc - w, L));
    }
    base += chunk;
  }
  total = base;
}

// Zeros for every real row of sequence b (a sequence whose rows see no key: no tile
// covers it).
template <int D, int TS>
__device__ __forceinline__ void write_zero_rows(const SplitKVArgs& a, int b) {
  const Geom g = geom_u<TS>(a, b);
  const int lane = lane_id();
  const int n = g.ntok * a.hq * (D / 4);
  for (int idx = lane; idx < n; idx += 64) {
    const int row = idx / (D / 4);
    const int d4 = (idx - row * (D / 4)) * 4;
    const int t = row / a.hq;
    const int h = row - t * a.hq;
    const int64_t off = (int64_t)(g.tok0 + t) * a.out_stride_tok + (int64_t)h * a.out_stride_head + d4;
    store_out4<false>(a.out, off, f32x4{0.f, 0.f, 0.f, 0.f}, 0.f, a.out_f32);
  }
}

// Total tiles over all sequences. Wave W also zeroes the rows of the key-less sequences
// b with b mod nwaves == W.
template <int D, int TS>
__device__ __forceinline__ int64_t scan_total(const SplitKVArgs& a, int W) {
  const int lane = lane_id();
  int64_t base = 0;
  for (int b0 = 0; b0 < a.batch; b0 += 64) {
    const int b = b0 + lane;
    int64_t w = 0;
    bool zero = false;
    if (b < a.batch) {
      const Geom g = geom<TS>(a, b);
      w = (int64_t)g.nt * g.rg_real * a.hkv;
      zero = g.nt == 0 && g.ntok > 0 && (b % a.nwaves) == W;
    }
#pragma unroll
    for (int m = 1; m < 64; m <<= 1) {
      const int src = (lane ^ m) << 2;
      const int lo = __builtin_amdgcn_ds_bpermute(src, (int)(uint32_t)w);
      const int hi = __builtin_amdgcn_ds_bpermute(src, (int)(w >> 32));
      w += (int64_t)(((uint64_t)(uint32_t)hi << 32) | (uint32_t)lo);
    }
    base += readlane_i64(w, 0);
    uint64_t zm = __builtin_amdgcn_ballot_w64(zero);
    while (zm) {
      const int L = __builtin_ctzll(zm);
      zm &= zm - 1;
      write_zero_rows<D, TS>(a, b0 + L);
    }
  }
  return base;
}

// Waves that take part: all of them, unless that would leave a wave fewer than
// kMinTiles tiles.
__device__ __forceinline__ int active_waves(int64_t total, int nwaves) {
  const int64_t want = (total + kMinTiles - 1) / kMinTiles;
  return (int)max((int64_t)1, min((int64_t)nwaves, want));
}

// Position of a wave in its tile range: sequence geometry, kv head, row group, tile.
struct Cursor {
  Geom g;
  int h, rg, tile;
  int t;  // wave-local tile number
};

template <int TS>
__device__ __forceinline__ void cursor_at(const SplitKVArgs& a, Cursor& c, int b, int64_t off) {
  c.g = geom_u<TS>(a, b);
  const int per_seg = c.g.nt;
  const int seg = (int)(off / per_seg);  // < rg_real * hkv
  c.tile = (int)(off - (int64_t)seg * per_seg);
  c.h = seg / c.g.rg_real;
  c.rg = seg - c.h * c.g.rg_real;
  c.t = 0;
}

// Next tile of the range; stays on the last tile once the range is exhausted.
template <int TS>
__device__ __forceinline__ void cursor_next(const SplitKVArgs& a, Cursor& c, int count) {
  if (c.t + 1 >= count) return;
  ++c.t;
  if (++c.tile < c.g.nt) return;
  c.tile = 0;
  if (++c.rg < c.g.rg_real) return;
  c.rg = 0;
  if (++c.h < a.hkv) return;
  c.h = 0;
  int b = c.g.b;
  do {
    ++b;
    c.g = geom_u<TS>(a, b);
  } while (c.g.nt == 0 || c.g.rg_real == 0);
}

// Wave index holding global tile t in a grid of nw waves over `total` tiles.
__device__ __forceinline__ int wave_of(int64_t t, int64_t total, int nw) {
  return (int)(((t + 1) * nw - 1) / total);
}
__device__ __forceinline__ int64_t wave_begin(int w, int64_t total, int nw) { return (int64_t)w * total / nw; }

// ---------------------------------------------------------------------------
// Partial kernel (persistent).
// ---------------------------------------------------------------------------
template <int D, int NB, bool QBF16, int KV>
__global__ __launch_bounds__(256, 1) void splitkv_partial(const SplitKVArgs args) {
  // A local copy: the lambdas below capture by reference, and a reference to the kernel
  // argument itself would force it into scratch memory.
  const SplitKVArgs a = args;
  static_assert(D == 64 || D == 128 || D == 256, "head dim 64, 128 or 256");
  constexpr bool kFp8 = (KV == DT_E4M3 || KV == DT_E5M2);
  constexpr int KK = D / 32;          // QK MFMA steps
  constexpr int DB = D / 16;          // PV MFMA steps
  constexpr int kRows = 16 * NB;
  constexpr bool kPvBf16 = (!kFp8) && QBF16;
  constexpr bool kSplitP = kPvBf16;
  constexpr int kElt = kFp8 ? 1 : 2;
  constexpr int kRowB = D * kElt;           // bytes of one head row
  constexpr int kCPR = kRowB / 16;          // 16-byte chunks per row
  constexpr int kTile = kTileKeys<D, kFp8>();  // keys per tile
  constexpr int TB = kTile / 16;            // 16-key blocks per tile
  constexpr int kTS = kTile == 16 ? 4 : 5;  // log2(kTile)
  static_assert(TB == 2 || !kFp8, "fp8 V^T reads assume 32-key tiles");
  constexpr int kStage = kTile * kRowB;     // bytes of one K (or V) tile
  constexpr int kVL = kStage / 1024;        // 16-byte K (or V) loads per lane per tile
  constexpr int OPS = 1 + 2 * kVL;          // vector memory instructions per pipeline step
  // Pipeline stages: K and V of S tiles in per-wave LDS rings. Each step issues OPS
  // vector memory instructions (one slot lookup, the V DMA, the K DMA); a wave can have
  // at most 63 outstanding, which bounds S (kSMax), and the two rings of four waves must
  // fit the CU's 160 KB of LDS (kSLds: 2 stages of 8 KB tiles, 5 of 4 KB tiles). Fewer
  // stages than the counter allows measured faster: at D = 128, 2 for the one-row-group
  // 16-bit kernels (3 measured 1.2-1.5% slower on bf16 decode and 4 about 2% slower),
  // and 4 for the fp8 kernels (8 measured 6.6% slower on fp8 verify and 0.8-1.4% on fp8
  // decode, 2 much slower). The two-row-group 16-bit kernels measured the same on verify
  // at 2 stages as at 4 when K still came through registers, where 4 fitted. 16-bit KV
  // at D = 64 has fp8 D = 128's 4 KB tiles and takes its 4 stages (its decode ran 5%
  // faster than at 8 stages with K through registers).
  constexpr int kSMax = 63 / OPS + 1;
  constexpr int kSLds = 160 * 1024 / (2 * kWaves * kStage);
  constexpr int kSWant = kStage <= 4096 ? 4 : 2;
  constexpr int S = std::min(std::min(kSMax, kSLds), kSWant);
  constexpr int A = 2 * S - 3;  // slots are looked up A tiles ahead of compute
  // Tiles kept in flight through a 16-bit tile's compute at S >= 4: none. Measured on
  // decode and verify with whole-row nontemporal loads, keeping 1, 2 or 3 in flight is
  // 2-3% slower there.
  constexpr int kInFlight16 = 0;
  static_assert(S >= 2 && (S - 1) * OPS <= 63, "more outstanding loads than the counter holds");
  static_assert(kVL >= 1 && 64 % kCPR == 0, "a V load covers whole rows");

  __shared__ __attribute__((aligned(16))) unsigned char vring[kWaves][S][kStage];
  __shared__ __attribute__((aligned(16))) unsigned char kring[kWaves][S][kStage];

  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int c = lane & 15;
  const int j = lane >> 4;
  const int W = blockIdx.x * kWaves + wave;
  // Head-dim order of the QK contraction: MFMA step kk of lane group j holds the K row's
  // 16-byte chunk 4*kk + j (16-bit KV; fp8: chunk 4*(kk/2) + j, half kk%2), that is
  // dims qdim(kk) .. +8, and the query rows are loaded in the same order.
  auto qdim = [&](int kk) -> int {
    if constexpr (kFp8) return (kk >> 1) * 64 + j * 16 + (kk & 1) * 8;
    else return kk * 32 + j * 8;
  };

  const int64_t total = scan_total<D, kTS>(a, W);
  const int nA = active_waves(total, a.nwaves);
  int MA_GLOBAL* my_desc = gptr_mut(a.desc) + (int64_t)W * kDescInts;
  if (W >= nA) {
    if (lane == 0) my_desc[0] = 0;
    return;
  }
  const int64_t t0 = wave_begin(W, total, nA);
  const int count = (int)(wave_begin(W + 1, total, nA) - t0);
  if (count <= 0) {
    if (lane == 0) my_desc[0] = 0;
    return;
  }
  int b0;
  int64_t off0;
  {
    int64_t tot_again;
    scan_work<kTS>(a, t0, tot_again, b0, off0);
  }

  const unsigned char MA_GLOBAL* kbase = gptr(reinterpret_cast<const unsigned char*>(a.k));
  const unsigned char MA_GLOBAL* vbase = gptr(reinterpret_cast<const unsigned char*>(a.v));
  const uint32_t row_bytes32 = (uint32_t)(a.kv_stride_row * kElt);  // the host checks it fits
  const int64_t head_bytes = a.kv_stride_head * kElt;

  // XOR swizzle of the 16-byte chunks of V row t in LDS (spreads the transposed reads
  // over the banks); it stays below the row's chunk count. fp8: each 32-lane half of a
  // transposed read takes one chunk of 16 rows, {0..7, 16..23} (+8 for the upper half);
  // the row's index among them, (t & 7) | ((t >> 1) & 8), picks its 16-byte column of the
  // 256-byte bank period (256 / kRowB rows share a period), so the 16 chunks fall in 16
  // distinct columns.
  auto swz = [](int t) -> int {
    if constexpr (kFp8) return (((t & 7) | ((t >> 1) & 8)) * kCPR) >> 4;
    else return (2 * t) & (kCPR - 2);
  };
  // XOR swizzle of the 16-byte chunks of K row t in the K ring: the 16 rows an
  // operand read takes one chunk from land in 16 different 16-byte columns of a 256-byte
  // bank period (a row of kRowB bytes spans 256 / kRowB rows of a period).
  auto swzk = [](int t) -> int {
    constexpr int kRowsPerPeriod = kRowB >= 256 ? 1 : 256 / kRowB;
    constexpr int kCols = kCPR < 16 ? kCPR : 16;
    return (t / kRowsPerPeriod) & (kCols - 1);
  };

  int sreg[S];  // slot lookups in flight, one per stage

  // The pipeline's vector memory instructions are issued as inline assembly and waited
  // for with explicit counts (wait_vm below): the compiler's own wait insertion cannot
  // follow the slot lookups across the loop back edge, and it drains all outstanding
  // loads before any LDS read once it has seen an LDS DMA. The build checks the generated
  // code for any access to a register whose load is still in flight.
  auto load_slot = [&](const Cursor& cu) __attribute__((always_inline)) -> int {
    const int key0 = cu.g.lo_min + cu.tile * kTile;
    const int pos = min(key0 + (lane & (kTile - 1)), cu.g.seq - 1);
    const int32_t MA_GLOBAL* tp =
        gptr(a.tt.table) + cu.g.seq_row * a.tt.stride + (pos >> a.tt.page_shift);
    int page;
    __asm__ volatile("global_load_dword %0, %1, off" MA_SLOT_POLICY : "=v"(page) : "v"(tp) : "memory");
    return page;
  };
  // slot = page << page_shift | offset in page; applied after the load has landed
  auto slot_of = [&](const Cursor& cu, int page) __attribute__((always_inline)) -> int {
    const int key0 = cu.g.lo_min + cu.tile * kTile;
    const int pos = min(key0 + (lane & (kTile - 1)), cu.g.seq - 1);
    return (page << a.tt.page_shift) | (pos & ((1 << a.tt.page_shift) - 1));
  };

  // V rows, then K rows, go straight to LDS stage `stage` of their rings (global_load_lds).
  auto issue = [&](const Cursor& cu, int myslot, int stage) __attribute__((always_inline)) {
    const uint64_t hoff = (uint64_t)cu.h * (uint64_t)head_bytes;
    const uint32_t lds0 = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) unsigned char*)vring[wave][stage];
    // Byte offset of the row that load x of this lane reads (its slot times the row
    // stride, plus the head): K and V read the same rows, so one lookup and one 32 x 32
    // -> 64-bit multiply serve both (the host keeps the row stride below 4 GiB).
    uint64_t roff[kVL];
#pragma unroll
    for (int x = 0; x < kVL; ++x) {
      const int tok = (64 / kCPR) * x + lane / kCPR;
      roff[x] = (uint64_t)(uint32_t)shfl_i(myslot, tok) * row_bytes32 + hoff;
    }
#pragma unroll
    for (int x = 0; x < kVL; ++x) {
      // one instruction: 64 / kCPR whole rows, lane -> (row, 16-byte chunk)
      const int tok = (64 / kCPR) * x + lane / kCPR;
      const int pos = lane % kCPR;
      const unsigned char MA_GLOBAL* src = vbase + roff[x] + ((pos ^ swz(tok)) << 4);
      const uint32_t m0 = __builtin_amdgcn_readfirstlane(lds0 + x * 1024);
      __asm__ volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dwordx4 %1, off" MA_V_POLICY : : "s"(m0), "v"(src) : "memory", "m0");
    }
    // K: whole rows per instruction, like V. The DMA writes lane chunks in lane order, so
    // lane chunk `pos` fetching the row's chunk pos ^ swzk(tok) lands the swizzled layout.
    const uint32_t kl0 = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) unsigned char*)kring[wave][stage];
#pragma unroll
    for (int x = 0; x < kVL; ++x) {
      const int tok = (64 / kCPR) * x + lane / kCPR;
      const int pos = lane % kCPR;
      const unsigned char MA_GLOBAL* kp = kbase + roff[x] + ((pos ^ swzk(tok)) << 4);
      const uint32_t m0 = __builtin_amdgcn_readfirstlane(kl0 + x * 1024);
      __asm__ volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dwordx4 %1, off" MA_K_POLICY : : "s"(m0), "v"(kp) : "memory", "m0");
    }
  };

  // Wait until at most N of this wave's vector memory instructions are outstanding; the
  // memory clobber keeps the ring's LDS reads below the wait.
  auto wait_vm = [&](auto N_) __attribute__((always_inline)) {
    constexpr int N = decltype(N_)::value;
    __asm__ volatile("s_waitcnt vmcnt(%0)" : : "n"(N) : "memory");
  };

  // ---- per-segment state ----
  int lo_r[NB], hi_r[NB];
  bool real[NB];
  u32x4 qv[NB][KK];
  float m_run[NB], l_run[NB];
  f32x4 o[NB][DB];
  int lmax = 0, hmin = 0;
  bool first_piece = true;  // the current piece is the first piece of this wave's range
  int piece_start_t = 0;    // wave-local tile where the current piece began
  // the shared segment that ends in this wave's first piece, if any
  bool ends_shared = false;
  int end_b = 0, end_h = 0, end_rg = 0;
  int64_t end_first = 0;

  auto begin_segment = [&](const Cursor& cu) __attribute__((always_inline)) {
    const uint16_t MA_GLOBAL* qbase = gptr(reinterpret_cast<const uint16_t*>(a.q));
    const int s_end = cu.g.seq;
    lmax = -0x7fffffff;
    hmin = 0x7fffffff;
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) {
      const int R = cu.rg * kRows + nb * 16 + c;
      const int t = R / a.group;
      const int g = R - t * a.group;
      real[nb] = t < cu.g.ntok;
      const int qpos = cu.g.prefix + t;
      const int hi = a.causal ? min(s_end, qpos + 1) : s_end;
      const int lo = a.window >= 0 ? max(0, qpos - a.window) : 0;
      lo_r[nb] = real[nb] ? lo : 0;
      hi_r[nb] = real[nb] ? hi : 0;
      if (real[nb]) {
        lmax = max(lmax, lo);
        hmin = min(hmin, hi);
      }
      // padding rows load the segment's first row (every segment has one) and are
      // zeroed below
      const int tq = real[nb] ? t : 0;
      const int gq = real[nb] ? g : 0;
      const uint16_t MA_GLOBAL* qp = qbase + (int64_t)(cu.g.tok0 + tq) * a.q_stride_tok +
                                     (int64_t)(cu.h * a.group + gq) * a.q_stride_head;
#pragma unroll
      for (int kk = 0; kk < KK; ++kk)
        __asm__ volatile("global_load_dwordx4 %0, %1, off" : "=v"(qv[nb][kk]) : "v"(qp + qdim(kk)) : "memory");
      m_run[nb] = -INFINITY;
      l_run[nb] = 0.f;
#pragma unroll
      for (int db = 0; db < DB; ++db) o[nb][db] = f32x4{0.f, 0.f, 0.f, 0.f};
    }
    // The query rows are inline-assembly loads waited for here, where a segment begins.
    // Loaded by the compiler, their wait would sit at their first use, a join that every
    // step passes, and be vmcnt(0) there (the compiler cannot count the pipeline's
    // inline-assembly loads): a drain of the K/V loads issued ahead on every step.
    __asm__ volatile("s_waitcnt vmcnt(0)" ::: "memory");
#pragma unroll
    for (int nb = 0; nb < NB; ++nb)
#pragma unroll
      for (int kk = 0; kk < KK; ++kk) {
        __asm__ volatile("" : "+v"(qv[nb][kk]));
        if (!real[nb]) qv[nb][kk] = u32x4{0, 0, 0, 0};
      }
#pragma unroll
    for (int m = 1; m < 64; m <<= 1) {
      lmax = max(lmax, __builtin_amdgcn_ds_bpermute((lane ^ m) << 2, lmax));
      hmin = min(hmin, __builtin_amdgcn_ds_bpermute((lane ^ m) << 2, hmin));
    }
  };

  // Write this piece: the final output when it covers the whole segment, else a partial.
  auto end_segment = [&](const Cursor& cu, bool whole, int slot_sel) __attribute__((always_inline)) {
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) {
      float lt = l_run[nb];
      lt += shfl_xor_f(lt, 16);
      lt += shfl_xor_f(lt, 32);
      if (!real[nb]) continue;
      const int R = cu.rg * kRows + nb * 16 + c;
      const int t = R / a.group;
      const int g = R - t * a.group;
      const float inv = lt > 0.f ? 1.f / lt : 0.f;
      if (whole) {
        const int64_t off = (int64_t)(cu.g.tok0 + t) * a.out_stride_tok + (int64_t)(cu.h * a.group + g) * a.out_stride_head;
        const float sc = inv * a.v_scale;
#pragma unroll
        for (int db = 0; db < DB; ++db) store_out4<QBF16>(a.out, off + db * 16 + 4 * j, o[nb][db], sc, a.out_f32);
      } else {
        const int64_t pidx = ((int64_t)W * 2 + slot_sel) * kMaxRows + nb * 16 + c;
        float MA_GLOBAL* po = gptr_mut(a.part_o) + pidx * D;
#pragma unroll
        for (int db = 0; db < DB; ++db) *reinterpret_cast<f32x4 MA_GLOBAL*>(po + db * 16 + 4 * j) = o[nb][db] * inv;
        if (j == 0) {
          const float mu = (m_run[nb] == -INFINITY) ? 0.f : m_run[nb];
          gptr_mut(a.part_lse)[pidx] = lt > 0.f ? __builtin_amdgcn_logf(lt) + mu * a.scale_log2 : kEmptyLse;
        }
      }
    }
    if (!whole && slot_sel == 0 && cu.tile == cu.g.nt - 1) {
      // first piece of this range and last tile of its segment, which began earlier
      ends_shared = true;
      end_b = cu.g.b;
      end_h = cu.h;
      end_rg = cu.rg;
      end_first = t0 + cu.t - cu.tile;
    }
  };

  auto compute = [&](const Cursor& cu, int stage) __attribute__((always_inline)) {
    const int tb0 = cu.g.lo_min + cu.tile * kTile;
    const unsigned char* vt = vring[wave][stage];
    // ---- K operand: the tile's rows from the K ring, unswizzled into operand order ----
    const unsigned char* ks = kring[wave][stage];
    u32x4 kr[TB][KK];
#pragma unroll
    for (int tb = 0; tb < TB; ++tb) {
      const int t = tb * 16 + c;
      auto chunk = [&](int q) -> u32x4 {
        return *reinterpret_cast<const u32x4*>(ks + t * kRowB + (((4 * q + j) ^ swzk(t)) << 4));
      };
      if constexpr (kFp8) {
#pragma unroll
        for (int half = 0; half < KK / 2; ++half) cvt16_fp8<KV, QBF16>(chunk(half), kr[tb][2 * half], kr[tb][2 * half + 1]);
      } else {
#pragma unroll
        for (int kk = 0; kk < KK; ++kk) kr[tb][kk] = chunk(kk);
      }
    }
    // ---- S^T = K Q^T ----
    f32x4 s[NB][TB];
#pragma unroll
    for (int nb = 0; nb < NB; ++nb)
#pragma unroll
      for (int tb = 0; tb < TB; ++tb) {
        f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int kk = 0; kk < KK; ++kk) acc = mfma16t<QBF16>(kr[tb][kk], qv[nb][kk], acc);
        s[nb][tb] = acc;
      }
    // ---- online softmax ----
    const bool full = (tb0 >= lmax) && (tb0 + kTile <= hmin);
    u32x4 pb[NB], pl[NB];
    bool grew = false;
    float alpha[NB];
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) {
      if (!full) {
#pragma unroll
        for (int tb = 0; tb < TB; ++tb)
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const int pos = tb0 + tb * 16 + 4 * j + i;
            if (pos < lo_r[nb] || pos >= hi_r[nb]) s[nb][tb][i] = -INFINITY;
          }
      }
      float mx;
      if constexpr (TB == 2) {
        const f32x4* sr = s[nb];
        mx = max3f(max3f(sr[0][0], sr[0][1], sr[0][2]), max3f(sr[0][3], sr[1][0], sr[1][1]),
                   max3f(sr[1][2], sr[1][3], -INFINITY));
      } else {
        mx = max3f(max3f(s[nb][0][0], s[nb][0][1], s[nb][0][2]), s[nb][0][3], -INFINITY);
      }
      alpha[nb] = 1.f;
      // fp8 KV (more VALU per tile for the conversions): the exponent base moves only when
      // some row's max has grown by more than 2^kLazyRescale in p, so the cross-lane max
      // and the rescale of O are rare. 16-bit KV measured faster with the update each tile.
      if (!kFp8 || __builtin_amdgcn_ballot_w64((mx - m_run[nb]) * a.scale_log2 > kLazyRescale)) {
        mx = fmaxf(mx, shfl_xor_f(mx, 16));
        mx = fmaxf(mx, shfl_xor_f(mx, 32));
        const float m_new = fmaxf(m_run[nb], mx);
        const float m_use = (m_new == -INFINITY) ? 0.f : m_new;
        grew |= (m_new != m_run[nb]);
        alpha[nb] = __builtin_amdgcn_exp2f((m_run[nb] - m_use) * a.scale_log2);
        m_run[nb] = m_new;
      }
      const float msc = ((m_run[nb] == -INFINITY) ? 0.f : m_run[nb]) * a.scale_log2;
      // P^T of the PV MFMA holds 32 keys; a 16-key tile leaves the upper 16 at zero
      float p[8];
      float ps;
      if constexpr (TB == 2) {
#pragma unroll
        for (int tb = 0; tb < 2; ++tb)
#pragma unroll
          for (int i = 0; i < 4; ++i) p[4 * tb + i] = __builtin_amdgcn_exp2f(s[nb][tb][i] * a.scale_log2 - msc);
        ps = ((p[0] + p[1]) + (p[2] + p[3])) + ((p[4] + p[5]) + (p[6] + p[7]));
      } else {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          p[i] = __builtin_amdgcn_exp2f(s[nb][0][i] * a.scale_log2 - msc);
          p[4 + i] = 0.f;
        }
        ps = (p[0] + p[1]) + (p[2] + p[3]);
      }
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
#pragma unroll
    for (int db = 0; db < DB; ++db) {
      u32x4 va;
      if constexpr (kFp8) {
        const int e = c >> 1, cc = lane & 1;
        const int t = (e < 4) ? (4 * j + e) : (16 + 4 * j + e - 4);
        const unsigned char* ptr = vt + t * kRowB + ((db ^ swz(t)) << 4) + cc * 8;
        const u32x2 raw = __builtin_bit_cast(u32x2, __builtin_amdgcn_ds_read_tr8_b64_v2i32(
            (__attribute__((address_space(3))) i32x2*)(ptr)));
        va = cvt8_fp8<KV, false>(raw[0], raw[1]);
      } else {
        const int e = c >> 2, cc = lane & 3;
        const int chunk = 2 * db + (cc >> 1);
#pragma unroll
        for (int half = 0; half < 2; ++half) {
          if (half >= TB) {  // keys past a 16-key tile: zero, like their P
            va[2 * half] = 0u;
            va[2 * half + 1] = 0u;
            continue;
          }
          const int t = 16 * half + 4 * j + e;
          const unsigned char* ptr = vt + t * kRowB + ((chunk ^ swz(t)) << 4) + (cc & 1) * 8;
          const u32x2 raw = __builtin_bit_cast(u32x2, __builtin_amdgcn_ds_read_tr16_b64_v4i16(
              (__attribute__((address_space(3))) i16x4*)(ptr)));
          va[2 * half] = raw[0];
          va[2 * half + 1] = raw[1];
        }
      }
#pragma unroll
      for (int nb = 0; nb < NB; ++nb) {
        o[nb][db] = mfma16t<kPvBf16>(va, pb[nb], o[nb][db]);
        if constexpr (kSplitP) o[nb][db] = mfma16t<kPvBf16>(va, pl[nb], o[nb][db]);
      }
    }
    __asm__ volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
  };

  // ---- cursors: slots run A tiles ahead of compute, K/V issue S-1 tiles ahead ----
  // A = 2S-3 is the largest lead the S-entry slot ring allows, and it keeps the wait for a
  // slot register from forcing any tile newer than the one about to be computed.
  Cursor cc, ci, cs;
  cursor_at<kTS>(a, cc, b0, off0);
  ci = cc;
  cs = cc;
  // Schedule. Step n: look up the slots of tile n+A, issue tile n+S-1 (its slots were
  // looked up at step n+S-1-A), compute tile n (issued at step n-S+1). Steps -A..-1 form
  // the prologue (no compute; tiles are issued from step 1-S on).
  // Vector memory instructions issued at step k: one slot lookup, plus OPS-1 tile loads
  // from step 1-S on. A wait for an instruction issued at step k0 keeps the instructions
  // of later steps in flight.
  auto ops_at = [](int k) constexpr -> int { return k >= 1 - S ? OPS : 1; };
  auto ops_between = [ops_at](int k0, int k1) constexpr -> int {  // steps k0..k1 inclusive
    int n = 0;
    for (int k = k0; k <= k1; ++k) n += ops_at(k);
    return n;
  };
  auto vstep = [&](auto N_) __attribute__((always_inline)) {
    constexpr int N = decltype(N_)::value - A;
    constexpr int SI = ((N + A) % S + S) % S;
    sreg[SI] = load_slot(cs);
    cursor_next<kTS>(a, cs, count);
    if constexpr (N + S - 1 >= 0) {
      constexpr int RI = ((N + S - 1) % S + S) % S;
      // the slot lookup of tile N+S-1 was issued at step N+S-1-A, first in its step
      constexpr int W = ops_between(N + S - 1 - A, N - 1);
      wait_vm(std::integral_constant<int, W>{});
      __asm__ volatile("" : "+v"(sreg[RI]));
      issue(ci, slot_of(ci, sreg[RI]), RI);
      cursor_next<kTS>(a, ci, count);
    }
  };
  [&]<int... Is>(std::integer_sequence<int, Is...>) __attribute__((always_inline)) {
    (vstep(std::integral_constant<int, Is>{}), ...);
  }(std::make_integer_sequence<int, A>{});

  auto step = [&](auto I_, int n) __attribute__((always_inline)) {
    constexpr int I = decltype(I_)::value;
    constexpr int RI = (I + S - 1) % S;
    // slot of tile n+A -> sreg[(n+A) % S] (that register's previous tile is already issued)
    sreg[(I + A) % S] = load_slot(cs);
    cursor_next<kTS>(a, cs, count);
    // K/V of tile n+S-1, once its slot lookup (A-S+1 steps ago) has landed
    wait_vm(std::integral_constant<int, OPS * (A - S + 1)>{});
    __asm__ volatile("" : "+v"(sreg[RI]));
    issue(ci, slot_of(ci, sreg[RI]), RI);
    cursor_next<kTS>(a, ci, count);
    if (n < count) {
      if (cc.t == 0 || cc.tile == 0) {
        begin_segment(cc);
        piece_start_t = cc.t;
      }
      // tile n was issued at step n-S+1; the S-1 steps since then keep their loads in flight
      // 16-bit KV at S >= 4 (D = 64): every load issued so far, the newest tile's included.
      // Measured on decode and verify at S = 4 (with K through registers), that was
      // 1.5-2.5% faster than keeping 1, 2 or S-1 tiles in flight through the compute: no
      // DMA then writes the LDS rings while the tile's operand reads run. With S = 2
      // (16-bit KV at D = 128 and 256) the wait for the slot above has already drained
      // tile n, and tile n+1 stays in flight. fp8 KV, half the bytes per tile:
      // only tile n, so S-1 tiles stay in flight, which is 12% faster than waiting for all.
      wait_vm(std::integral_constant<int, (kFp8 || S < 4) ? (S - 1) * OPS : kInFlight16 * OPS>{});
      compute(cc, I);
      const bool seg_last = (cc.tile == cc.g.nt - 1);
      const bool range_last = (n == count - 1);
      if (seg_last || range_last) {
        const bool whole = seg_last && (cc.tile == cc.t - piece_start_t);
        // slot 0: the first piece of the range (also a single-piece range); slot 1: the last
        end_segment(cc, whole, first_piece ? 0 : 1);
        first_piece = false;
      }
      cursor_next<kTS>(a, cc, count);
    }
  };

  auto group = [&]<int... Is>(std::integer_sequence<int, Is...>, int n) __attribute__((always_inline)) {
    (step(std::integral_constant<int, Is>{}, n + Is), ...);
  };
  for (int n = 0; n < count; n += S) group(std::make_integer_sequence<int, S>{}, n);

  // ---- descriptor of the shared segment ending here (read by splitkv_merge) ----
  if (lane == 0) {
    int MA_GLOBAL* dsc = my_desc;
    if (ends_shared) {
      const int w1 = wave_of(end_first, total, nA);
      dsc[1] = end_b;
      dsc[2] = end_h;
      dsc[3] = end_rg;
      dsc[4] = w1;
      dsc[5] = end_first > wave_begin(w1, total, nA) ? 1 : 0;  // slot of the first piece
      dsc[0] = 1;
    } else {
      dsc[0] = 0;
    }
  }
}

// ---------------------------------------------------------------------------
// Merge: one workgroup per partial-kernel wave W (for 32-row groups, one per 8-row set of
// W's row group). If W's first piece ended a shared segment, combine the pieces of waves
// w1..W into the output: a running maximum of the log2 LSEs rescales the sum of the
// normalised partial outputs, so one pass reads each piece once and the loads of
// successive pieces do not wait for each other's math. 256 threads cover 1024 / D rows x
// D head-dim entries per pass.
// ---------------------------------------------------------------------------
// Row sets (1024 / D rows: one pass of a 256-thread merge workgroup) of a row group.
template <int D, int NB>
constexpr int merge_passes() {
  return (16 * NB) / (1024 / D) > 0 ? (16 * NB) / (1024 / D) : 1;
}
// Merge workgroups per partial-kernel wave: one per row set when more than one row set
// holds real rows (they then merge in parallel), else one for the whole row group.
template <int D, int NB>
static int merge_split(int rows_total) {
  const int real_rows = rows_total < 16 * NB ? rows_total : 16 * NB;
  return real_rows > 1024 / D ? merge_passes<D, NB>() : 1;
}

template <int D, int NB, bool QBF16>
__global__ __launch_bounds__(256) void splitkv_merge(const SplitKVArgs args) {
  const SplitKVArgs a = args;
  constexpr int kRows = 16 * NB;
  const int split = a.merge_split;  // workgroups per partial-kernel wave: 1 or kPass
  const int W = blockIdx.x / split;
  const int part = blockIdx.x - W * split;
  const int MA_CONST* dsc = cptr(a.desc) + (int64_t)W * kDescInts;
  if (dsc[0] == 0) return;
  const int b = dsc[1], h = dsc[2], rg = dsc[3], w1 = dsc[4], sel1 = dsc[5];
  const Geom g = geom_u<5>(a, b);  // only its token range is read here, not the tile count
  const float MA_GLOBAL* plse = gptr(a.part_lse);
  const float MA_GLOBAL* po = gptr(a.part_o);
  constexpr int kTPR = D / 4;       // threads per row, four head-dim entries each
  constexpr int kRPP = 256 / kTPR;  // rows per pass of the workgroup
  const int d4 = (threadIdx.x % kTPR) * 4;
  const int r_base = threadIdx.x / kTPR;
  // thread: rows r_base + kRPP i, head-dim entries d4..d4+3. Each row set has a workgroup
  // of its own (one whose rows are all GQA padding returns at once). Within a row set the pieces
  // are the outer loop (unrolled by four), so the loads of four pieces are in flight
  // together. Measured at D=128 on a verify batch of 32 x 4 tokens: 13 us with one row
  // set at a time in one workgroup, 10 us with all four together, 8.0 us with a
  // workgroup per row set; about 5 us on a decode batch of 64.
  constexpr int kPass = merge_passes<D, NB>();
  static_assert(kPass == (kRows / kRPP > 0 ? kRows / kRPP : 1), "a row set is one pass");
  constexpr int kChunk = 1;
  for (int c0 = split == 1 ? 0 : part; c0 < (split == 1 ? kPass : part + 1); c0 += kChunk) {
    bool live = false;  // rows past the last query token (GQA padding) are not read
#pragma unroll
    for (int i = 0; i < kChunk; ++i) {
      const int row = r_base + kRPP * (c0 + i);
      live |= row < kRows && (rg * kRows + row) / a.group < g.ntok;
    }
    if (!live) continue;
    float m[kChunk], wsum[kChunk];
    f32x4 acc[kChunk];
#pragma unroll
    for (int i = 0; i < kChunk; ++i) {
      m[i] = -INFINITY;
      wsum[i] = 0.f;
      acc[i] = f32x4{0.f, 0.f, 0.f, 0.f};
    }
#pragma unroll 4
    for (int w = w1; w <= W; ++w) {
      const int64_t pbase = ((int64_t)w * 2 + (w == w1 ? sel1 : 0)) * kMaxRows + r_base + kRPP * c0;
      float lse[kChunk];
      f32x4 o[kChunk];
#pragma unroll
      for (int i = 0; i < kChunk; ++i) {
        lse[i] = plse[pbase + kRPP * i];
        o[i] = *reinterpret_cast<const f32x4 MA_GLOBAL*>(po + (pbase + kRPP * i) * D + d4);
      }
#pragma unroll
      for (int i = 0; i < kChunk; ++i) {
        const float m_new = fmaxf(m[i], lse[i]);  // every LSE is finite (empty pieces: -2^30)
        const float s_old = __builtin_amdgcn_exp2f(m[i] - m_new);
        const float s_new = __builtin_amdgcn_exp2f(lse[i] - m_new);
        acc[i] = acc[i] * s_old + o[i] * s_new;
        wsum[i] = wsum[i] * s_old + s_new;
        m[i] = m_new;
      }
    }
#pragma unroll
    for (int i = 0; i < kChunk; ++i) {
      const int row = r_base + kRPP * (c0 + i);
      const int R = rg * kRows + row;
      const int t = R / a.group;
      const int gg = R - t * a.group;
      if (row >= kRows || t >= g.ntok) continue;
      const int64_t off = (int64_t)(g.tok0 + t) * a.out_stride_tok + (int64_t)(h * a.group + gg) * a.out_stride_head + d4;
      store_out4<QBF16>(a.out, off, acc[i], a.v_scale / wsum[i], a.out_f32);
    }
  }
}
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

// Row blocks per row group: at D = 256 only one (two would spill registers that in-flight
// loads still target); the host then uses more row groups of 16 rows.
template <int D>
constexpr int kMaxNB = D == 256 ? 1 : 2;

template <int D>
static hipError_t launch_partial_d(int nb, bool qbf16, int kv, dim3 grid, hipStream_t st, const SplitKVArgs& a) {
  if constexpr (kMaxNB<D> == 1) {
    return qbf16 ? launch_partial_kv<D, 1, true>(kv, grid, st, a) : launch_partial_kv<D, 1, false>(kv, grid, st, a);
  } else {
    if (qbf16) return nb == 1 ? launch_partial_kv<D, 1, true>(kv, grid, st, a) : launch_partial_kv<D, 2, true>(kv, grid, st, a);
    return nb == 1 ? launch_partial_kv<D, 1, false>(kv, grid, st, a) : launch_partial_kv<D, 2, false>(kv, grid, st, a);
  }
}

template <int D>
static hipError_t launch_merge_d(int nb, bool qbf16, int nwaves, hipStream_t st, const SplitKVArgs& a) {
  constexpr int NB2 = kMaxNB<D>;
  const dim3 grid((unsigned)(nwaves * a.merge_split));
  if (qbf16) {
    if (nb == 1) hipLaunchKernelGGL((splitkv_merge<D, 1, true>), grid, dim3(256), 0, st, a);
    else hipLaunchKernelGGL((splitkv_merge<D, NB2, true>), grid, dim3(256), 0, st, a);
  } else {
    if (nb == 1) hipLaunchKernelGGL((splitkv_merge<D, 1, false>), grid, dim3(256), 0, st, a);
    else hipLaunchKernelGGL((splitkv_merge<D, NB2, false>), grid, dim3(256), 0, st, a);
  }
  return hipGetLastError();
}

}  // namespace ma

using namespace ma;

static int device_workgroups(int requested) {
  if (requested > 0) return requested;
  int dev = 0, cus = 0;
  if (hipGetDevice(&dev) != hipSuccess) return -1;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) return -1;
  return cus;
}

// Workspace: [descriptors: nwaves x kDescInts int32][partial O: nwaves x 2 x 32 x D fp32]
// [LSE: nwaves x 2 x 32 fp32], each region 256-byte aligned. Every call rewrites the
// descriptors of all its waves, so the workspace needs no initialisation.
constexpr int kMaxWorkgroups = 16384;
static constexpr size_t ws_desc_bytes(int num_workgroups) {
  return ((size_t)num_workgroups * kWaves * kDescInts * sizeof(int) + 255) & ~(size_t)255;
}
static constexpr size_t ws_o_bytes(int num_workgroups, int head_dim) {
  const size_t pieces = (size_t)num_workgroups * kWaves * 2 * kMaxRows;
  return (pieces * head_dim * sizeof(float) + 255) & ~(size_t)255;
}

static constexpr size_t ws_bytes(int num_workgroups, int head_dim) {
  return ws_desc_bytes(num_workgroups) + ws_o_bytes(num_workgroups, head_dim) +
         (((size_t)num_workgroups * kWaves * 2 * kMaxRows * sizeof(float) + 255) & ~(size_t)255);
}

// Decode on the any-head-dim kernel splits each row block's keys over up to this many
// workgroups per compute unit in all (the piece partials the workspace holds).
constexpr int kPieceWgPerCu = 2;
// ... but only when the longest row known is longer than this many keys: up to it one
// workgroup per row block in a single launch is as fast on the device and one launch
// cheaper on the host. Measured at D=128, 32 / 8 heads, fp16, B=1 and 4: 512 keys 9.8
// against 12.6 us per call (wall clock), 1,024 keys 13.8 against 13.0 (pieces ahead).
constexpr int64_t kPieceMinKeys = 512;

extern "C" size_t ma_splitkv_workspace_bytes(int num_workgroups, int head_dim) {
  if (num_workgroups <= 0 || head_dim <= 0) return 0;
  // the any-head-dim kernel keeps only the pieces of a split decode
  if (any_head_dim(head_dim)) return any_piece_bytes((int64_t)num_workgroups * kPieceWgPerCu, head_dim);
  return ws_bytes(num_workgroups, head_dim);
}

// A decode whose split-KV tile count (32-key tiles over every sequence, kv head and row
// group, at the longest length the caller knows) is at most this runs on the any-head-dim
// kernel as one pass over key pieces plus a merge: for so little work the persistent
// kernel's start (a scan of every sequence) and its merge over every wave's descriptor
// cost more than they save. Measured at D = 128, 32 / 8 heads, B 1-32 and contexts of
// 512-8192: the pieces are faster up to 16384 tiles (B = 8 at 8192 keys: 51.8 against
// 61.5 us per call; B = 32 at 2048: 45.6 against 59.4) and slower beyond (B = 16 at 8192:
// 110 against 101); B = 1 at 512 keys takes 16.5 us per call either way.
#ifndef MA_SMALL_DECODE_TILES
#define MA_SMALL_DECODE_TILES 16384
#endif
constexpr int64_t kSmallDecodeTiles = MA_SMALL_DECODE_TILES;

// ---------------------------------------------------------------------------
// Static scratch of the allocation-free decode (ma_grouped_decode_noalloc): the split-KV
// workspace of a persistent grid of up to kScratchWorkgroups workgroups at the largest
// head dim, in device memory that the code object itself carries. Each device the
// library runs on holds one copy from the module's load until the process ends. The
// kernels never read this symbol: host code passes the copy's device address, taken once
// per device with hipGetSymbolAddress (the name itself is a host-side stand-in, not a
// device address).
// ---------------------------------------------------------------------------
constexpr int kScratchWorkgroups = MA_NOALLOC_MAX_WORKGROUPS;
constexpr size_t kScratchBytes = ws_bytes(kScratchWorkgroups, 256);
static __device__ __align__(256) unsigned char scratch[kScratchBytes];

namespace {
constexpr int kMaxDevices = 64;
std::mutex g_scratch_lock;
void* g_scratch_ptr[kMaxDevices] = {};
}  // namespace

// This device's copy of `scratch`, looked up on its first use with the device current.
static int scratch_of_current_device(void** out) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return set_error(MA_ELAUNCH, "hipGetDevice failed");
  if (dev < 0 || dev >= kMaxDevices) return set_error(MA_EUNSUPPORTED, "device %d beyond %d devices", dev, kMaxDevices);
  std::lock_guard<std::mutex> guard(g_scratch_lock);
  if (!g_scratch_ptr[dev]) {
    void* ptr = nullptr;
    const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !ptr)
      return set_error(MA_ELAUNCH, "hipGetSymbolAddress(scratch) failed on device %d: %s", dev, hipGetErrorString(e));
    g_scratch_ptr[dev] = ptr;
  }
  *out = g_scratch_ptr[dev];
  return MA_OK;
}

extern "C" int ma_device_workgroups(void) { return device_workgroups(0); }

static int splitkv_run(SplitKVArgs a, int head_dim, int q_dtype, int kv_dtype, int max_q_per_seq,
                       int num_workgroups, int max_seq_len, void* workspace, size_t workspace_bytes,
                       hipStream_t stream) {
  const bool generic = any_head_dim(head_dim);  // served by the any-head-dim kernel
  if (!generic && head_dim != 64 && head_dim != 128 && head_dim != 256)
    return set_error(MA_EUNSUPPORTED, "head_dim %d not supported (multiples of 16 up to %d)", head_dim, kAnyMaxDim);
  if (q_dtype != DT_F16 && q_dtype != DT_BF16) return set_error(MA_EINVAL, "q dtype %d must be f16 or bf16", q_dtype);
  if (kv_dtype < 0 || kv_dtype > DT_E5M2) return set_error(MA_EINVAL, "kv dtype %d unknown", kv_dtype);
  if ((kv_dtype == DT_F16 || kv_dtype == DT_BF16) && kv_dtype != q_dtype)
    return set_error(MA_EINVAL, "16-bit KV dtype must equal the query dtype");
  if (a.batch < 0 || a.hq <= 0 || a.hkv <= 0 || a.hq % a.hkv)
    return set_error(MA_EINVAL, "bad head counts hq=%d hkv=%d", a.hq, a.hkv);
  if (!(a.scale_log2 > 0.f)) return set_error(MA_EINVAL, "softmax scale must be positive");
  if (a.tt.page_shift < 0 || a.tt.page_shift > 16) return set_error(MA_EINVAL, "bad page shift");
  if (max_q_per_seq <= 0) return set_error(MA_EINVAL, "max query rows per sequence must be positive");
  if (num_workgroups <= 0 || num_workgroups > kMaxWorkgroups)
    return set_error(MA_EINVAL, "num_workgroups must be in 1..%d (ma_device_workgroups())", kMaxWorkgroups);
  if (a.batch == 0) return MA_OK;
  if (!a.q || !a.k || !a.v || !a.tt.table || !a.seq_lens || !a.out)
    return set_error(MA_EINVAL, "null pointer argument");
  if ((reinterpret_cast<uintptr_t>(a.q) | reinterpret_cast<uintptr_t>(a.k) | reinterpret_cast<uintptr_t>(a.v) |
       reinterpret_cast<uintptr_t>(a.out)) & 15)
    return set_error(MA_EINVAL, "q, k, v and out must be 16-byte aligned");
  const int elt = (kv_dtype >= DT_E4M3) ? 1 : 2;
  const int out_elt = a.out_f32 ? 4 : 2;
  const int out_align = a.out_f32 ? 15 : 7;  // f32x4 or 4 x 16-bit stores
  if (((a.kv_stride_row * elt) & 15) || ((a.kv_stride_head * elt) & 15) || ((a.q_stride_tok * 2) & 15) ||
      ((a.q_stride_head * 2) & 15) || ((a.out_stride_tok * out_elt) & out_align) ||
      ((a.out_stride_head * out_elt) & out_align))
    return set_error(MA_EINVAL, "strides must keep rows 16-byte aligned");
  if (a.kv_stride_row * elt >= ((int64_t)1 << 32))
    return set_error(MA_EUNSUPPORTED, "KV row stride of %lld bytes exceeds 4 GiB", (long long)(a.kv_stride_row * elt));
  a.group = a.hq / a.hkv;
  if ((int64_t)a.num_tokens * a.group > 0x7fffffff) return set_error(MA_EINVAL, "num_tokens x GQA group exceeds 2^31");
  if (max_seq_len < 0) return set_error(MA_EINVAL, "max_seq_len must be >= 0 (0: not known)");
  const bool decode = a.qsl == nullptr;
  // a small decode: the split-KV tiles at the longest length the caller knows
  bool small = false;
  if (!generic && decode && max_seq_len > 0) {
    const int rows_total = a.group;
    const int64_t row_groups = (rows_total + 31) / 32;
    const int64_t tiles = (int64_t)a.batch * a.hkv * row_groups * ((max_seq_len + 31) / 32);
    small = tiles <= kSmallDecodeTiles;
  }
  if (generic || small) {
    // one workgroup per 16 rows (token, GQA head), its four waves splitting the keys and
    // merging through LDS; a decode also splits each row block's keys over `pieces`
    // workgroups when the grid would leave compute units idle, merged by a second kernel
    AnyArgs g{};
    g.q = a.q; g.q_stride_tok = a.q_stride_tok; g.q_stride_head = a.q_stride_head;
    g.k = a.k; g.v = a.v; g.kv_stride_row = a.kv_stride_row; g.kv_stride_head = a.kv_stride_head;
    g.tt = a.tt; g.row_index = a.row_index; g.seq_lens = a.seq_lens; g.qsl = a.qsl; g.prefix = a.prefix;
    g.num_tokens = a.num_tokens; g.batch = a.batch; g.hq = a.hq; g.hkv = a.hkv; g.group = a.group;
    g.head_dim = head_dim; g.items = nullptr;
    g.row_blocks = (int)(((int64_t)max_q_per_seq * a.group + kAnyRows - 1) / kAnyRows);
    g.causal = a.causal; g.window = a.window; g.scale_log2 = a.scale_log2; g.v_scale = a.v_scale;
    g.out = a.out; g.out_stride_tok = a.out_stride_tok; g.out_stride_head = a.out_stride_head; g.out_f32 = a.out_f32;
    g.pieces = 1;
    const int64_t base = (int64_t)a.batch * a.hkv * g.row_blocks;  // one workgroup per row block
    const int64_t cap_slots = (int64_t)num_workgroups * kPieceWgPerCu;
    if (decode && base < num_workgroups && workspace && workspace_bytes >= any_piece_bytes(cap_slots, head_dim) &&
        !(reinterpret_cast<uintptr_t>(workspace) & 255)) {
      // pieces: enough workgroups to cover the chip twice, no more than one 16-key tile per
      // wave at the longest length known (the caller's bound, else the table's width),
      // within the workspace's piece slots; each piece is an equal share of its sequence's
      // own keys, so any bound gives the same result
      const int64_t width = max_seq_len > 0 ? (int64_t)max_seq_len : (a.tt.stride << a.tt.page_shift);
      const int64_t by_len = (width + kAnyWaves * kAnyKeys - 1) / (kAnyWaves * kAnyKeys);
      const int64_t want = (cap_slots + base - 1) / base;
      const int64_t pieces = width > kPieceMinKeys ? std::min(std::min(want, by_len), cap_slots / base) : 1;
      if (pieces > 1) {
        g.pieces = (int)pieces;
        char* ws = reinterpret_cast<char*>(workspace);
        g.part_o = reinterpret_cast<float*>(ws);
        g.part_lse = reinterpret_cast<float*>(ws + any_piece_o_bytes(cap_slots, head_dim));
      }
    }
    const int64_t grid = base * g.pieces;
    if (grid > 0x7fffffff) return set_error(MA_EINVAL, "grid too large");
    const hipError_t e = any_launch(g, q_dtype, kv_dtype, grid, stream);
    if (e != hipSuccess) return set_error(MA_ELAUNCH, "any-head-dim launch failed: %s", hipGetErrorString(e));
    return MA_OK;
  }
  const int rows_total = max_q_per_seq * a.group;
  const int nb = (rows_total <= 16 || head_dim == 256) ? 1 : 2;
  a.rows = 16 * nb;
  a.row_groups = (rows_total + a.rows - 1) / a.rows;
  a.nwaves = num_workgroups * kWaves;
  a.merge_split = head_dim == 64    ? (nb == 1 ? merge_split<64, 1>(rows_total) : merge_split<64, 2>(rows_total))
                  : head_dim == 128 ? (nb == 1 ? merge_split<128, 1>(rows_total) : merge_split<128, 2>(rows_total))
                                    : merge_split<256, 1>(rows_total);
  const size_t need = ma_splitkv_workspace_bytes(num_workgroups, head_dim);
  if (!workspace || workspace_bytes < need)
    return set_error(MA_EINVAL, "workspace too small: %zu < %zu bytes", workspace_bytes, need);
  char* ws = reinterpret_cast<char*>(workspace);
  if (reinterpret_cast<uintptr_t>(ws) & 255) return set_error(MA_EINVAL, "workspace must be 256-byte aligned");
  a.desc = reinterpret_cast<int*>(ws);
  a.part_o = reinterpret_cast<float*>(ws + ws_desc_bytes(num_workgroups));
  a.part_lse = reinterpret_cast<float*>(ws + ws_desc_bytes(num_workgroups) + ws_o_bytes(num_workgroups, head_dim));
  const int64_t segs = (int64_t)a.batch * a.hkv * a.row_groups;
  if (segs > 0x7fffffff) return set_error(MA_EINVAL, "too many segments");
  const bool qbf16 = q_dtype == DT_BF16;
  const dim3 grid((unsigned)num_workgroups);
  hipError_t e = head_dim == 64    ? launch_partial_d<64>(nb, qbf16, kv_dtype, grid, stream, a)
                 : head_dim == 128 ? launch_partial_d<128>(nb, qbf16, kv_dtype, grid, stream, a)
                                   : launch_partial_d<256>(nb, qbf16, kv_dtype, grid, stream, a);
  if (e != hipSuccess) return set_error(MA_ELAUNCH, "split-KV launch failed: %s", hipGetErrorString(e));
  e = head_dim == 64    ? launch_merge_d<64>(nb, qbf16, a.nwaves, stream, a)
      : head_dim == 128 ? launch_merge_d<128>(nb, qbf16, a.nwaves, stream, a)
                        : launch_merge_d<256>(nb, qbf16, a.nwaves, stream, a);
  if (e != hipSuccess) return set_error(MA_ELAUNCH, "merge launch failed: %s", hipGetErrorString(e));
  return MA_OK;
}

extern "C" int ma_grouped_decode(
    const void* q, int64_t q_stride_tok, int64_t q_stride_head, int q_dtype,
    const void* k_cache, const void* v_cache, int64_t kv_stride_row, int64_t kv_stride_head, int kv_dtype,
    const int32_t* table, int64_t table_stride, const int64_t* row_index, int page_size,
    const int32_t* seq_lens, int batch, int num_q_heads, int num_kv_heads, int head_dim,
    int num_workgroups, float softmax_scale, float k_scale, float v_scale,
    int sliding_window, int max_seq_len, void* workspace, size_t workspace_bytes,
    void* out, int out_dtype, int64_t out_stride_tok, int64_t out_stride_head, void* stream) {
  if (page_size <= 0 || (page_size & (page_size - 1))) return set_error(MA_EINVAL, "page size %d must be a power of two", page_size);
  if ((q_dtype == DT_F16 || q_dtype == DT_BF16) && out_dtype != q_dtype && out_dtype != DT_F32)
    return set_error(MA_EINVAL, "out dtype %d must be the query dtype or f32", out_dtype);
  SplitKVArgs a{};
  a.q = q; a.q_stride_tok = q_stride_tok; a.q_stride_head = q_stride_head;
  a.k = k_cache; a.v = v_cache; a.kv_stride_row = kv_stride_row; a.kv_stride_head = kv_stride_head;
  a.tt.table = table; a.tt.stride = table_stride; a.tt.page_shift = __builtin_ctz(page_size);
  a.row_index = row_index; a.seq_lens = seq_lens; a.qsl = nullptr; a.prefix = nullptr;
  a.num_tokens = batch;
  a.batch = batch; a.hq = num_q_heads; a.hkv = num_kv_heads;
  a.causal = 1; a.window = sliding_window < 0 ? -1 : sliding_window;
  a.scale_log2 = softmax_scale * k_scale * kLog2e; a.v_scale = v_scale;
  a.out = out; a.out_stride_tok = out_stride_tok; a.out_stride_head = out_stride_head;
  a.out_f32 = out_dtype == DT_F32;
  return splitkv_run(a, head_dim, q_dtype, kv_dtype, 1, num_workgroups, max_seq_len, workspace, workspace_bytes,
                     (hipStream_t)stream);
}

extern "C" int ma_paged_verify(
    const void* q, int64_t q_stride_tok, int64_t q_stride_head, int q_dtype, int64_t num_tokens,
    const void* k_cache, const void* v_cache, int64_t kv_stride_row, int64_t kv_stride_head, int kv_dtype,
    const int32_t* table, int64_t table_stride, const int64_t* row_index, int page_size,
    const int32_t* seq_lens, const int32_t* query_start_loc, const int32_t* prefix_lens,
    int batch, int max_q_per_seq, int num_q_heads, int num_kv_heads, int head_dim,
    int causal, int sliding_window, int num_workgroups,
    float softmax_scale, float k_scale, float v_scale, void* workspace, size_t workspace_bytes,
    void* out, int out_dtype, int64_t out_stride_tok, int64_t out_stride_head, void* stream) {
  if ((q_dtype == DT_F16 || q_dtype == DT_BF16) && out_dtype != q_dtype && out_dtype != DT_F32)
    return set_error(MA_EINVAL, "out dtype %d must be the query dtype or f32", out_dtype);
  if (num_tokens < 0 || num_tokens > 0x7fffffff) return set_error(MA_EINVAL, "num_tokens %lld out of range", (long long)num_tokens);
  if (page_size <= 0 || (page_size & (page_size - 1))) return set_error(MA_EINVAL, "page size %d must be a power of two", page_size);
  if (!query_start_loc) return set_error(MA_EINVAL, "query_start_loc is required");
  if (max_q_per_seq > 64) return set_error(MA_EUNSUPPORTED, "verify supports at most 64 query rows per sequence");
  SplitKVArgs a{};
  a.q = q; a.q_stride_tok = q_stride_tok; a.q_stride_head = q_stride_head;
  a.k = k_cache; a.v = v_cache; a.kv_stride_row = kv_stride_row; a.kv_stride_head = kv_stride_head;
  a.tt.table = table; a.tt.stride = table_stride; a.tt.page_shift = __builtin_ctz(page_size);
  a.row_index = row_index; a.seq_lens = seq_lens; a.qsl = query_start_loc; a.prefix = prefix_lens;
  a.num_tokens = (int)num_tokens;
  a.batch = batch; a.hq = num_q_heads; a.hkv = num_kv_heads;
  a.causal = causal ? 1 : 0; a.window = sliding_window < 0 ? -1 : sliding_window;
  a.scale_log2 = softmax_scale * k_scale * kLog2e; a.v_scale = v_scale;
  a.out = out; a.out_stride_tok = out_stride_tok; a.out_stride_head = out_stride_head;
  a.out_f32 = out_dtype == DT_F32;
  return splitkv_run(a, head_dim, q_dtype, kv_dtype, max_q_per_seq, num_workgroups, 0, workspace, workspace_bytes,
                     (hipStream_t)stream);
}

extern "C" int ma_grouped_decode_noalloc(
    const void* q, int64_t q_stride_tok, int64_t q_stride_head, int q_dtype,
    const void* k_cache, const void* v_cache, int64_t kv_stride_row, int64_t kv_stride_head, int kv_dtype,
    const int32_t* table, int64_t table_stride, const int64_t* row_index, int page_size,
    const int32_t* seq_lens, int batch, int num_q_heads, int num_kv_heads, int head_dim,
    int num_workgroups, float softmax_scale, float k_scale, float v_scale, int sliding_window,
    int max_seq_len, void* out, int out_dtype, int64_t out_stride_tok, int64_t out_stride_head, void* stream) {
  if (num_workgroups <= 0 || num_workgroups > kScratchWorkgroups)
    return set_error(MA_EINVAL, "num_workgroups %d: the static scratch serves 1..%d", num_workgroups, kScratchWorkgroups);
  // the scratch holds the split-KV workspace of the largest grid at head dim 256, which also
  // covers the key pieces of the any-head-dim kernel at every head dim up to 512
  static_assert(any_piece_bytes_c(kScratchWorkgroups * kPieceWgPerCu, 512) <= kScratchBytes, "scratch too small");
  void* ws = nullptr;
  const int rc = scratch_of_current_device(&ws);
  if (rc != MA_OK) return rc;
  return ma_grouped_decode(q, q_stride_tok, q_stride_head, q_dtype, k_cache, v_cache, kv_stride_row, kv_stride_head,
                           kv_dtype, table, table_stride, row_index, page_size, seq_lens, batch, num_q_heads,
                           num_kv_heads, head_dim, num_workgroups, softmax_scale, k_scale, v_scale, sliding_window,
                           max_seq_len, ws, kScratchBytes, out, out_dtype, out_stride_tok, out_stride_head, stream);
}
