// Prefix-aware paged extend (chunked prefill) attention for gfx950.
//
// Replaces the reference's paged extend kernel
// (sglang_restomod/attention/v100/tilelang/_kernels_paged.py:55-393, launched from
// _paged_adapter.py:567-759): query token i of sequence b sees key j when
//   j < seq_lens[b]  and (causal: j <= prefix[b] + i)  and (window W >= 0: j >= prefix[b] + i - W).
//
// Decomposition (head dims 64 and 128; XShape below gives D = 256's): one workgroup =
// 8 waves = 256 query rows of ONE kv head, where row r of a sequence is (query token
// r / G, GQA head r % G); each wave owns 32 rows (two 16-row blocks), two waves per SIMD
// so that one's softmax overlaps the other's MFMAs. All G heads that share a kv head are
// served from one copy of each K/V tile in LDS. At D = 256 a wave owns 16 rows and a
// tile has 32 keys.
//
// Work list: a one-workgroup plan kernel lists the row tiles (sequence, tile) of the
// batch from query_start_loc on the device, ordered by their key-tile count, heaviest
// first (a longest-processing-time order over the CUs), so no host-side maximum of the
// query lengths is needed. The extend grid is 1-D, (list entry) x (kv head) with the kv
// head fastest: workgroup i runs on XCD i % 8, so with 8 kv heads each XCD streams one
// head's K/V through its own L2.
//
// Per 64-key tile, per wave (scores of all its keys, then one online-softmax update, then
// PV), MFMA 16x16x32 with fp32 accumulate; the softmax's VALU work is what bounds the
// kernel, so the row sums of P also come from an MFMA (a block of V^T whose row 0 is
// ones), the row max uses three-input maxima, and O is rescaled only when a row's max
// has grown by more than a factor 2^8 in p:
//   S^T[key, row] = K[key, :] . Q[row, :]     A = K from LDS, B = Q^T (registers, whole kernel)
//   O^T[d, row] += V^T[d, key] P^T[key, row]  A = V^T read transposed from LDS
//                                             (ds_read_b64_tr_b16 / _tr_b8), B = P^T straight
//                                             from the S^T accumulators, in fp16.
// K stays in the query dtype (exact products; fp8 converted exactly). V is used in fp16:
// bf16 V is converted in LDS once per tile (each wave converts the part it loaded, exact
// for |v| in fp16's normal range), fp8 V exactly while it is read. P is fp16, the
// softmax state fp32.
//
// Memory pipeline: K and V tiles travel HBM -> LDS by DMA (global_load_lds) into an
// S-stage ring (4 stages for 16-bit KV, 8 for fp8), with S-1 tiles in flight while one
// computes; each wave moves an eighth of every tile (for an fp8 tile at D = 64, half the
// waves move K and half V). K lands as MFMA fragment blocks (a 1 KB block holds 16 keys
// x 16 bytes per lane, lane l's 16 bytes at l * 16), so each operand read is one
// conflict-free ds_read_b128; V lands row-major with an XOR swizzle of its 16-byte
// chunks. Slots are
// looked up S+1 tiles ahead. The loads are inline assembly with explicit wait counts,
// and one barrier per tile both publishes a tile and retires the stage it replaces.

#include <type_traits>

#include "common.h"
#include "paged_any.h"

// MA_ASM_PIPELINE: the build verifies the generated code of this file for accesses to
// registers whose inline-assembly loads are still in flight.
#include "capi_internal.h"

namespace ma {

constexpr int kXWaves = 8;  // waves per workgroup

// Tile shape per head dim (64, 128 or 256). Q and O take registers in proportion to the
// head dim, so at D = 256 a wave holds one 16-row block and a tile has 32 keys; the K
// and V stages keep their size in LDS.
template <int D>
struct XShape {
  static constexpr int BN = D == 256 ? 32 : 64;  // keys per tile
  static constexpr int RB = D == 256 ? 1 : 2;    // 16-row blocks per wave
  static constexpr int BM = kXWaves * RB * 16;   // query rows per workgroup
};
constexpr int kXBMMin = XShape<256>::BM;  // the smallest row tile: it sizes the work list

// One entry of the work list: sequence in the low 32 bits, row tile in the high 32;
// -1 (sequence -1) past the last tile.
__host__ __device__ constexpr int64_t row_tile_item(int seq, int tile) {
  return (int64_t)(((uint64_t)(uint32_t)tile << 32) | (uint32_t)seq);
}

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
  int num_tokens;        // rows of q and out: query rows are clamped into [0, num_tokens)
  int batch, hq, hkv, group;
  const int64_t* items;  // work list (row_tile_item)
  int causal, window;
  float scale_log2;
  float v_scale;
  void* out;
  int64_t out_stride_tok, out_stride_head;  // elements of the output dtype
  int out_f32;                              // out holds fp32 (else the query dtype)
  int head_dim;                             // the rows' head dim (<= the kernel's D when padded)
  int chunks;                               // 16-byte chunks of one K/V row at head_dim
};

// Keys [lo, hi) that some row of the bm-row tile starting at row r0 of a sequence may see.
struct KeyRange {
  int lo, hi;
};
__device__ __forceinline__ KeyRange row_tile_keys(int r0, int bm, int ntok, int group, int prefix, int seq,
                                                  int causal, int window) {
  const int t_first = r0 / group;
  const int t_last = min(ntok - 1, (r0 + bm - 1) / group);
  KeyRange k;
  k.lo = window >= 0 ? max(0, prefix + t_first - window) : 0;
  k.hi = causal ? min(seq, prefix + t_last + 1) : seq;
  return k;
}

// ---- work list ----
constexpr int kPlanThreads = 1024;
constexpr int kPlanBuckets = 1024;      // cost classes of the counting sort
constexpr int kPlanMaxBatch = 16384;    // per-sequence tile offsets kept in LDS
constexpr int kPlanFixedCost = 2;       // a row tile's set-up, in key tiles

struct ExtendPlanArgs {
  const int32_t* qsl;
  const int32_t* seq_lens;
  const int32_t* prefix;
  int num_tokens;
  int batch, group, causal, window;
  int tile_rows, tile_keys;  // the extend kernel's rows per workgroup and keys per tile
  int capacity;              // entries of items
  int64_t* items;
};

// Row tiles of bm rows of a sequence with ntok query tokens.
__device__ __forceinline__ int seq_row_tiles(int ntok, int group, int bm) {
  return ntok > 0 ? (int)(((int64_t)ntok * group + bm - 1) / bm) : 0;
}

// Block-wide exclusive prefix sum of one value per thread (kPlanThreads threads);
// returns this thread's offset and sets *total. Uses sums[kPlanThreads / 64].
__device__ __forceinline__ int block_exclusive_scan(int x, int* sums, int* total) {
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  int incl = x;
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    const int y = __shfl_up(incl, d, 64);
    if (lane >= d) incl += y;
  }
  if (lane == 63) sums[wave] = incl;
  __syncthreads();
  int before = 0, all = 0;
#pragma unroll
  for (int w = 0; w < kPlanThreads / 64; ++w) {
    const int s = sums[w];
    before += (w < wave) ? s : 0;
    all += s;
  }
  __syncthreads();  // sums is free again
  *total = all;
  return before + incl - x;
}

// One workgroup: list every row tile of the batch as {sequence, tile}, the ones with the
// most key tiles first (a counting sort over kPlanBuckets cost classes), and fill the
// rest of items with {-1, -1}. The order within a class is arbitrary; each row tile's
// result does not depend on it.
__global__ __launch_bounds__(kPlanThreads, 1) void extend_plan_kernel(const ExtendPlanArgs a) {
  __shared__ int start[kPlanMaxBatch + 1];
  __shared__ int hist[kPlanBuckets];
  __shared__ int sums[kPlanThreads / 64];
  static_assert(kPlanBuckets == kPlanThreads, "one cost class per thread in the scan");
  const int tid = threadIdx.x;
  const int32_t MA_GLOBAL* qsl = gptr(a.qsl);
  const int32_t MA_GLOBAL* seq_lens = gptr(a.seq_lens);

  // 1. first list index of each sequence's row tiles
  int carry = 0;
  for (int base = 0; base < a.batch; base += kPlanThreads) {
    const int b = base + tid;
    const int n = b < a.batch ? seq_row_tiles(clamp_query_rows(qsl[b], qsl[b + 1], a.num_tokens).ntok, a.group,
                                              a.tile_rows)
                              : 0;
    int total;
    const int off = block_exclusive_scan(n, sums, &total);
    if (b < a.batch) start[b] = carry + off;
    carry += total;
  }
  const int m = carry;  // the same in every thread
  if (tid == 0) start[a.batch] = m;
  hist[tid] = 0;
  __syncthreads();

  // list index t -> (sequence, row tile) and its cost in key tiles
  auto decode = [&](int t, int* b_out, int* rt_out) -> int {
    int lo = 0, hi = a.batch;  // the last b with start[b] <= t (start[batch] = m > t)
    while (hi - lo > 1) {
      const int mid = (lo + hi) >> 1;
      if (start[mid] <= t) lo = mid; else hi = mid;
    }
    const int b = lo;
    const int rt = t - start[b];
    const int ntok = clamp_query_rows(qsl[b], qsl[b + 1], a.num_tokens).ntok;
    const int seq = seq_lens[b];
    const int prefix = a.prefix ? gptr(a.prefix)[b] : seq - ntok;
    const KeyRange k = row_tile_keys(rt * a.tile_rows, a.tile_rows, ntok, a.group, prefix, seq, a.causal, a.window);
    *b_out = b;
    *rt_out = rt;
    return (k.hi > k.lo ? (k.hi - k.lo + a.tile_keys - 1) / a.tile_keys : 0) + kPlanFixedCost;
  };

  // 2. the largest cost, which scales the classes
  int cmax = 0;
  for (int t = tid; t < m; t += kPlanThreads) {
    int b, rt;
    cmax = max(cmax, decode(t, &b, &rt));
  }
#pragma unroll
  for (int d = 32; d >= 1; d >>= 1) cmax = max(cmax, __shfl_xor(cmax, d, 64));
  if ((tid & 63) == 0) sums[tid >> 6] = cmax;
  __syncthreads();
#pragma unroll
  for (int w = 0; w < kPlanThreads / 64; ++w) cmax = max(cmax, sums[w]);
  __syncthreads();

  // 3. class sizes (class 0 holds the heaviest tiles), 4. their first list index
  auto cls = [&](int cost) -> int {
    return kPlanBuckets - 1 - (int)(((int64_t)cost * kPlanBuckets) / ((int64_t)cmax + 1));
  };
  for (int t = tid; t < m; t += kPlanThreads) {
    int b, rt;
    atomicAdd(&hist[cls(decode(t, &b, &rt))], 1);
  }
  __syncthreads();
  int unused;
  const int first = block_exclusive_scan(hist[tid], sums, &unused);
  hist[tid] = first;
  __syncthreads();

  // 5. scatter, 6. pad
  int64_t MA_GLOBAL* items = gptr_mut(a.items);
  for (int t = tid; t < m; t += kPlanThreads) {
    int b, rt;
    const int pos = atomicAdd(&hist[cls(decode(t, &b, &rt))], 1);
    if (pos < a.capacity) items[pos] = row_tile_item(b, rt);
  }
  for (int i = m + tid; i < a.capacity; i += kPlanThreads) items[i] = row_tile_item(-1, -1);
}

// HD: the rows' head dim. HD == D: exact. Otherwise the head dim is below D (a multiple of
// 16 that has no kernel of its own): every load stays in its row, the chunks past head_dim
// reading the row's last chunk again; those K dims meet Q dims that are zero, and the
// output dims they feed are not stored. HD == 0 takes the head dim from the arguments and
// runs every MFMA step of D; a head dim fixed at compile time (0 < HD < D) also skips the
// score steps and output blocks that lie wholly past it.
template <int D, bool QBF16, int KV, int HD>
__global__ __launch_bounds__(kXWaves * 64, 1) void extend_kernel(const ExtendArgs args) {
  const ExtendArgs a = args;  // local copy: the lambdas capture by reference
  constexpr bool PAD = HD != D;
  constexpr int kSkipFrom = (PAD && HD != 0) ? HD : 0;  // first dim with no work, or 0
  constexpr int kXD = D;
  constexpr bool kFp8 = (KV == DT_E4M3 || KV == DT_E5M2);
  constexpr int kXBN = XShape<D>::BN;
  constexpr int kXRB = XShape<D>::RB;
  constexpr int kXBM = XShape<D>::BM;
  constexpr int KK = D / 32;                     // QK MFMA steps (16-bit operands)
  constexpr int KB = kXBN / 16;                  // 16-key blocks per tile
  constexpr int DB = D / 16;                     // PV MFMA steps
  constexpr int HF = kXBN / 32;                  // 32-key halves of a tile (PV contraction)
  constexpr bool kConvV = (!kFp8) && QBF16;      // bf16 V: converted to fp16 in LDS
  constexpr int kElt = kFp8 ? 1 : 2;
  constexpr int kRowB = kXD * kElt;              // bytes of one K/V row
  constexpr int kKSub = kRowB / 64;              // K DMA blocks (1 KB) per 16-key block
  constexpr int kCPR = kRowB / 16;               // 16-byte chunks per row
  constexpr int kStageB = kXBN * kRowB;          // bytes of the K (or V) part of a tile
  // DMA blocks (1 KB) of K, and of V, per tile. Each wave moves an equal share of both;
  // when a tile has fewer blocks than waves (fp8 at D = 64: 4), half the waves move K
  // and the other half V, one block each, so every wave issues the same count.
  constexpr int kTileBlk = kStageB / 1024;
  constexpr bool kSplitDMA = kTileBlk < kXWaves;
  static_assert(!kSplitDMA || 2 * kTileBlk == kXWaves, "K and V blocks must cover the waves");
  static_assert(!kSplitDMA || !kConvV, "the V conversion assumes every wave loaded V");
  constexpr int kKBlk = kSplitDMA ? 1 : kTileBlk / kXWaves;  // K DMA blocks per moving wave
  constexpr int kVBlk = kSplitDMA ? 1 : kTileBlk / kXWaves;  // V DMA blocks per moving wave
  constexpr int ND = kSplitDMA ? 1 : kKBlk + kVBlk;          // DMA instructions per wave per tile
  constexpr int OPS = 1 + ND;                    // plus one slot lookup
  // pipeline stages: 4 x 32 KB for 16-bit KV, 8 x 16 KB for fp8. Five 16-bit stages (all
  // 160 KB of LDS) measured 1.8% slower on the D = 128 extend batch, and five fp8 stages
  // the same as eight.
  constexpr int S = kFp8 ? 8 : 4;
  constexpr int A = S + 1;                       // slot lookahead (tiles)
  static_assert((S - 1) * ND + 2 <= 63, "outstanding loads exceed the counter");
  // the wait before a tile's barrier counts on its loads preceding the slot lookup of
  // step k-2 (tile k is issued at step k-S+1 <= k-3)
  static_assert(S >= 4, "the schedule needs at least four stages");
  static_assert(kKBlk >= 1 && kKSub % kKBlk == 0, "a wave's K blocks share one key block");
  static_assert(kVBlk >= 1 && 64 % kCPR == 0, "a V DMA block holds whole rows");

  __shared__ __attribute__((aligned(1024))) unsigned char kring[S][kStageB];
  __shared__ __attribute__((aligned(1024))) unsigned char vring[S][kStageB];

  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int c = lane & 15;
  const int j = lane >> 4;
  // Head-dim order of the QK contraction: MFMA step kk of lane group j holds dims
  // qdim(kk) .. +8, the 16-byte chunk 4*kk + j of a K row (fp8: steps 2h and 2h+1 split
  // chunk 4*h + j), so that each step covers 32 consecutive dims (fp8: a pair of steps
  // covers 64) and steps past a padded head dim hold only zeros.
  auto qdim = [&](int kk) -> int {
    if constexpr (kFp8) return (kk >> 1) * 64 + j * 16 + (kk & 1) * 8;
    else return kk * 32 + j * 8;
  };

  const int item = (int)blockIdx.x / a.hkv;
  const int h = (int)blockIdx.x - item * a.hkv;
  const int64_t work = cptr(a.items)[item];
  const int b = (int)(uint32_t)work;
  if (b < 0) return;
  const int rt = (int)(work >> 32);
  const QueryRows qr = clamp_query_rows(cptr(a.qsl)[b], cptr(a.qsl)[b + 1], a.num_tokens);
  const int tok0 = qr.tok0;
  const int ntok = qr.ntok;
  const int r0 = rt * kXBM;
  if (r0 >= ntok * a.group) return;
  const int seq = cptr(a.seq_lens)[b];
  const int prefix = a.prefix ? cptr(a.prefix)[b] : seq - ntok;
  const int64_t seq_row = a.row_index ? cptr(a.row_index)[b] : (int64_t)b;

  // ---- this lane's rows (one per 16-row block) ----
  int lo_r[kXRB], hi_r[kXRB];
  bool real[kXRB];
  u32x4 qv[kXRB][KK];
  const uint16_t MA_GLOBAL* qbase = gptr(reinterpret_cast<const uint16_t*>(a.q));
#pragma unroll
  for (int rb = 0; rb < kXRB; ++rb) {
    const int r = r0 + wave * (kXRB * 16) + rb * 16 + c;
    const int t = r / a.group;
    const int g = r - t * a.group;
    real[rb] = t < ntok;
    const int qpos = prefix + t;
    lo_r[rb] = (real[rb] && a.window >= 0) ? max(0, qpos - a.window) : 0;
    hi_r[rb] = real[rb] ? (a.causal ? min(seq, qpos + 1) : seq) : 0;
    const uint16_t MA_GLOBAL* qp =
        qbase + (int64_t)(tok0 + t) * a.q_stride_tok + (int64_t)(h * a.group + g) * a.q_stride_head;
#pragma unroll
    for (int kk = 0; kk < KK; ++kk) {
      const bool in_dim = !PAD || qdim(kk) < a.head_dim;
      qv[rb][kk] = (real[rb] && in_dim) ? *reinterpret_cast<const u32x4 MA_GLOBAL*>(qp + qdim(kk)) : u32x4{0, 0, 0, 0};
    }
  }
  // Q is waited for here, once. The compiler cannot count the loads issued by inline
  // assembly below, so a Q load still outstanding at the first score MFMA in the loop
  // is waited for with vmcnt(0), which drains every K/V tile in flight, once per pass.
#pragma unroll
  for (int rb = 0; rb < kXRB; ++rb)
#pragma unroll
    for (int kk = 0; kk < KK; ++kk) __asm__ volatile("" : "+v"(qv[rb][kk]));
  // keys any row of the workgroup may see, and the window in which no row needs masking
  const int t_first = r0 / a.group;
  const int t_last = min(ntok - 1, (r0 + kXBM - 1) / a.group);
  const KeyRange keys = row_tile_keys(r0, kXBM, ntok, a.group, prefix, seq, a.causal, a.window);
  const int key_lo = keys.lo;
  const int key_hi = keys.hi;
  const int full_lo = a.window >= 0 ? max(0, prefix + t_last - a.window) : 0;
  const int full_hi = a.causal ? min(seq, prefix + t_first + 1) : seq;
  const int ntiles = key_hi > key_lo ? (key_hi - key_lo + kXBN - 1) / kXBN : 0;

  float m_run[kXRB];
  f32x4 o[kXRB][DB];
  // row sums of P, by MFMA: A = a 16 x 32 block whose row 0 is ones, so D[0][row] = sum_k P[row][k]
  f32x4 lacc[kXRB];
  const uint32_t one2 = (c == 0) ? 0x3C003C00u : 0u;
  const u32x4 ones = u32x4{one2, one2, one2, one2};
#pragma unroll
  for (int rb = 0; rb < kXRB; ++rb) {
    m_run[rb] = -INFINITY;
    lacc[rb] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int db = 0; db < DB; ++db) o[rb][db] = f32x4{0.f, 0.f, 0.f, 0.f};
  }

  const unsigned char MA_GLOBAL* kbase = gptr(reinterpret_cast<const unsigned char*>(a.k));
  const unsigned char MA_GLOBAL* vbase = gptr(reinterpret_cast<const unsigned char*>(a.v));
  const int64_t row_bytes = a.kv_stride_row * kElt;
  const uint32_t row_bytes32 = (uint32_t)row_bytes;  // the host checks it fits
  const int64_t head_off = (int64_t)h * a.kv_stride_head * kElt;
  // XOR swizzle of the 16-byte chunks of V row t in LDS (spreads the transposed reads
  // over the banks); it stays below the row's chunk count
  auto swz = [](int t) -> int {
    if constexpr (kFp8) return kCPR >= 8 ? ((t & 3) | ((t >> 2) & 4)) : (t & (kCPR - 1));
    else return (2 * t) & (kCPR - 2);
  };
  // the row's 16-byte chunk a DMA lane reads: chunk c, or the row's last one past head_dim
  auto src_chunk = [&](int c) __attribute__((always_inline)) -> int {
    if constexpr (PAD) return min(c, a.chunks - 1);
    else return c;
  };

  // ---- memory pipeline ----
  // Lane l looks up the slot of key l of a tile; tiles past the last are clamped to it
  // (their loads are issued and ignored, so every step issues the same instructions).
  auto key_of = [&](int tile) __attribute__((always_inline)) -> int {
    return min(key_lo + min(tile, ntiles - 1) * kXBN + lane, key_hi - 1);
  };
  auto load_slot = [&](int tile) __attribute__((always_inline)) -> int {
    const int pos = key_of(tile);
    const int32_t MA_GLOBAL* tp = gptr(a.tt.table) + seq_row * a.tt.stride + (pos >> a.tt.page_shift);
    int page;
    __asm__ volatile("global_load_dword %0, %1, off" : "=v"(page) : "v"(tp) : "memory");
    return page;
  };
  auto slot_of = [&](int tile, int page) __attribute__((always_inline)) -> int {
    const int pos = key_of(tile);
    return (page << a.tt.page_shift) | (pos & ((1 << a.tt.page_shift) - 1));
  };
  auto dma = [&](const unsigned char MA_GLOBAL* src, uint32_t lds) __attribute__((always_inline)) {
    const uint32_t m0 = __builtin_amdgcn_readfirstlane(lds);
    __asm__ volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dwordx4 %1, off" : : "s"(m0), "v"(src) : "memory", "m0");
  };
  auto issue = [&](int myslot, int st) __attribute__((always_inline)) {
    const uint32_t kl = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) unsigned char*)kring[st];
    const uint32_t vl = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) unsigned char*)vring[st];
    if constexpr (kSplitDMA) {
      // waves below kTileBlk move one K block, the others one V block; the source and
      // destination are selected, not branched on, so that every wave runs the same
      // instructions around the in-flight slot registers
      const bool is_k = wave < kTileBlk;
      const int xb = is_k ? wave : wave - kTileBlk;
      const int tok = (64 / kCPR) * xb + lane / kCPR;  // V row of this lane
      const int pos = lane % kCPR;
      const int sl = shfl_i(myslot, is_k ? xb * 16 + c : tok);
      const unsigned char MA_GLOBAL* row = (is_k ? kbase : vbase) + (uint64_t)(uint32_t)sl * row_bytes32 + head_off;
      // K: lane l -> key 16 * xb + (l & 15), 16-byte chunk j (one 64-byte block per row)
      const int chunk = src_chunk(is_k ? j : (pos ^ swz(tok)));
      dma(row + chunk * 16, (is_k ? kl : vl) + xb * 1024);
    } else {
      // all slot shuffles first, so that their LDS round trips overlap; this wave's K blocks
      // (kb, sub) = divmod(wave * kKBlk + x, kKSub) all lie in key block kb
      const int kb_w = (wave * kKBlk) / kKSub;
      const int kslot = shfl_i(myslot, kb_w * 16 + c);
      int vslot[kVBlk];
#pragma unroll
      for (int x = 0; x < kVBlk; ++x) {
        const int xb = wave * kVBlk + x;
        vslot[x] = shfl_i(myslot, (64 / kCPR) * xb + lane / kCPR);
      }
      // K: lane l -> key kb_w*16 + (l & 15), 16-byte chunk 4*sub + j
      const unsigned char MA_GLOBAL* kp = kbase + (uint64_t)(uint32_t)kslot * row_bytes32 + head_off;
#pragma unroll
      for (int x = 0; x < kKBlk; ++x) {
        const int blk = wave * kKBlk + x;
        dma(kp + src_chunk(4 * (blk % kKSub) + j) * 16, kl + blk * 1024);
      }
      // V: rows of this wave's blocks, row-major, 16-byte chunks XOR-swizzled by row
#pragma unroll
      for (int x = 0; x < kVBlk; ++x) {
        const int xb = wave * kVBlk + x;
        const int tok = (64 / kCPR) * xb + lane / kCPR;
        const int pos = lane % kCPR;
        dma(vbase + (uint64_t)(uint32_t)vslot[x] * row_bytes32 + head_off + (src_chunk(pos ^ swz(tok)) << 4),
            vl + xb * 1024);
      }
    }
  };
  auto wait_vm = [&](auto N_) __attribute__((always_inline)) {
    constexpr int N = decltype(N_)::value;
    __asm__ volatile("s_waitcnt vmcnt(%0)" : : "n"(N) : "memory");
  };
  auto barrier = [&]() __attribute__((always_inline)) { __asm__ volatile("s_barrier" : : : "memory"); };
  // bf16 V -> fp16 in place, the 16 bytes per block that this lane loaded
  auto convert_v = [&](int st) __attribute__((always_inline)) {
#pragma unroll
    for (int x = 0; x < kVBlk; ++x) {
      u32x4* pv = reinterpret_cast<u32x4*>(vring[st] + (wave * kVBlk + x) * 1024 + lane * 16);
      u32x4 v = *pv;
#pragma unroll
      for (int w = 0; w < 4; ++w)
        v[w] = pack_f16(__builtin_bit_cast(float, v[w] << 16), __builtin_bit_cast(float, v[w] & 0xffff0000u));
      *pv = v;
    }
  };
  // per-lane part of the V^T read addresses (16-bit V): row 4j + e, column bits of cc
  const int vrow = (4 * j + (c >> 2)) * kRowB + ((lane & 3) >> 1) * 16 + (lane & 1) * 8;
  const int vs1 = (4 * j + (c >> 2)) & (kCPR / 2 - 1);

  // ---- one tile: scores for all 64 keys, then mid() (work that overlaps the score
  // MFMAs), one softmax update, PV ----
  auto compute = [&](int tile, int st, auto&& mid) __attribute__((always_inline)) {
    const unsigned char* kt = kring[st];
    const unsigned char* vt = vring[st];
    const int base = key_lo + tile * kXBN;
    f32x4 s[kXRB][KB];
#pragma unroll
    for (int rb = 0; rb < kXRB; ++rb)
#pragma unroll
      for (int kb = 0; kb < KB; ++kb) s[rb][kb] = f32x4{0.f, 0.f, 0.f, 0.f};
    if constexpr (kFp8) {
#pragma unroll
      for (int hh = 0; hh < kKSub; ++hh) {
        if (kSkipFrom && hh * 64 >= kSkipFrom) continue;  // dims past the head dim: zeros in Q
#pragma unroll
        for (int kb = 0; kb < KB; ++kb) {
          const u32x4 raw = *reinterpret_cast<const u32x4*>(kt + (kb * kKSub + hh) * 1024 + lane * 16);
          u32x4 k0, k1;
          cvt16_fp8<KV, QBF16>(raw, k0, k1);
#pragma unroll
          for (int rb = 0; rb < kXRB; ++rb) {
            s[rb][kb] = mfma16t<QBF16>(k0, qv[rb][2 * hh], s[rb][kb]);
            s[rb][kb] = mfma16t<QBF16>(k1, qv[rb][2 * hh + 1], s[rb][kb]);
          }
        }
      }
    } else {
#pragma unroll
      for (int kk = 0; kk < KK; ++kk) {
        if (kSkipFrom && kk * 32 >= kSkipFrom) continue;  // dims past the head dim: zeros in Q
#pragma unroll
        for (int kb = 0; kb < KB; ++kb) {
          const u32x4 kf = *reinterpret_cast<const u32x4*>(kt + (kb * kKSub + kk) * 1024 + lane * 16);
#pragma unroll
          for (int rb = 0; rb < kXRB; ++rb) s[rb][kb] = mfma16t<QBF16>(kf, qv[rb][kk], s[rb][kb]);
        }
      }
    }
    mid();
    const bool full = (base >= full_lo) && (base + kXBN <= full_hi);
    u32x4 pk[kXRB][HF];
    float alpha[kXRB];
    bool grew = false;
#pragma unroll
    for (int rb = 0; rb < kXRB; ++rb) {
      if (!full) {
#pragma unroll
        for (int kb = 0; kb < KB; ++kb)
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const int pos = base + kb * 16 + 4 * j + i;
            if (pos < lo_r[rb] || pos >= hi_r[rb]) s[rb][kb][i] = -INFINITY;
          }
      }
      float sv[4 * KB];
#pragma unroll
      for (int kb = 0; kb < KB; ++kb)
#pragma unroll
        for (int i = 0; i < 4; ++i) sv[kb * 4 + i] = s[rb][kb][i];
      float mx = max_tree<4 * KB>(sv);
      alpha[rb] = 1.f;
      // the exponent base only moves when some row's max has grown by more than
      // 2^kLazyRescale in p: until then p stays <= 2^kLazyRescale (exact in fp16's
      // relative precision, fp32 sums) and O is not rescaled
      if (__builtin_amdgcn_ballot_w64((mx - m_run[rb]) * a.scale_log2 > kLazyRescale)) {
        mx = fmaxf(mx, shfl_xor_f(mx, 16));
        mx = fmaxf(mx, shfl_xor_f(mx, 32));
        const float m_new = fmaxf(m_run[rb], mx);
        const float m_use = (m_new == -INFINITY) ? 0.f : m_new;
        grew |= (m_new != m_run[rb]);
        alpha[rb] = __builtin_amdgcn_exp2f((m_run[rb] - m_use) * a.scale_log2);
        m_run[rb] = m_new;
      }
      const float m_use = (m_run[rb] == -INFINITY) ? 0.f : m_run[rb];
      const float msc = m_use * a.scale_log2;
      float p[4 * KB];
#pragma unroll
      for (int kb = 0; kb < KB; ++kb)
#pragma unroll
        for (int i = 0; i < 4; ++i) p[kb * 4 + i] = __builtin_amdgcn_exp2f(s[rb][kb][i] * a.scale_log2 - msc);

#pragma unroll
      for (int st2 = 0; st2 < HF; ++st2)
#pragma unroll
        for (int w = 0; w < 4; ++w) pk[rb][st2][w] = pack_f16(p[8 * st2 + 2 * w], p[8 * st2 + 2 * w + 1]);
    }
    if (__builtin_amdgcn_ballot_w64(grew)) {
#pragma unroll
      for (int rb = 0; rb < kXRB; ++rb)
#pragma unroll
        for (int db = 0; db < DB; ++db) o[rb][db] *= alpha[rb];
#pragma unroll
      for (int rb = 0; rb < kXRB; ++rb) lacc[rb] *= alpha[rb];
    }
#pragma unroll
    for (int hf = 0; hf < HF; ++hf)
#pragma unroll
      for (int db = 0; db < DB; ++db) {
        if (kSkipFrom && db * 16 >= kSkipFrom) continue;  // output dims past the head dim: never stored
        u32x4 va;
        if constexpr (kFp8) {
          const int e = c >> 1, cc = lane & 1;
          const int t = hf * 32 + ((e < 4) ? (4 * j + e) : (16 + 4 * j + e - 4));
          const unsigned char* ptr = vt + t * kRowB + ((db ^ swz(t)) << 4) + cc * 8;
          const u32x2 raw = __builtin_bit_cast(u32x2, __builtin_amdgcn_ds_read_tr8_b64_v2i32(
              (__attribute__((address_space(3))) i32x2*)(ptr)));
          va = cvt8_fp8<KV, false>(raw[0], raw[1]);
        } else {
          const unsigned char* pcol = vt + vrow + ((db ^ vs1) << 5);
#pragma unroll
          for (int half = 0; half < 2; ++half) {
            const unsigned char* ptr = pcol + (hf * 32 + 16 * half) * kRowB;
            const u32x2 raw = __builtin_bit_cast(u32x2, __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                (__attribute__((address_space(3))) i16x4*)(ptr)));
            va[2 * half] = raw[0];
            va[2 * half + 1] = raw[1];
          }
        }
#pragma unroll
        for (int rb = 0; rb < kXRB; ++rb) o[rb][db] = mfma16t<false>(va, pk[rb][hf], o[rb][db]);
      }
#pragma unroll
    for (int hf = 0; hf < HF; ++hf)
#pragma unroll
      for (int rb = 0; rb < kXRB; ++rb) lacc[rb] = mfma16t<false>(ones, pk[rb][hf], lacc[rb]);
  };

  // ---- schedule ----
  // Step k: look up the slots of tile k+A; once the slots of tile k+S-1 (looked up at
  // step k-2) have landed, and at k >= 0 after a barrier, issue tile k+S-1 into stage
  // (k+S-1) % S; at k >= 0 compute tile k from stage k % S, converting tile k+1's bf16 V
  // while the scores' MFMAs run. Steps -A..-1 are the prologue. Instructions issued per
  // step: one slot lookup, plus ND from step 1-S on.
  auto nd_at = [](int k) constexpr -> int { return k >= 1 - S ? ND : 0; };
  auto wait_at = [nd_at](int k) constexpr -> int {  // issued after the slot lookup of step k-2
    int n = 0;
    if (k - 2 >= -A) n += nd_at(k - 2);
    if (k - 1 >= -A) n += 1 + nd_at(k - 1);
    return n + 1;
  };
  int sreg[S];
  auto step = [&](auto K_, int kbase) __attribute__((always_inline)) {
    constexpr int KC = decltype(K_)::value;  // step index modulo S (steady state) or exact (prologue)
    const int k = kbase + KC;
    constexpr int SL = ((KC + A) % S + S) % S;
    constexpr int DI = ((KC + S - 1) % S + S) % S;
    sreg[SL] = load_slot(k + A);
    if (k + S - 1 >= 0) {
      // wait counts: exact per prologue step, 2 * OPS from step -1 on
      wait_vm(std::integral_constant<int, wait_at(KC < 0 ? KC : 2)>{});
      __asm__ volatile("" : "+v"(sreg[DI]));
      if (k >= 0) barrier();
      issue(slot_of(k + S - 1, sreg[DI]), DI);
    }
    // bf16 V of tile k+1 -> fp16, inside tile k's compute after its score MFMAs are
    // issued (or on its own where no tile is computed); its LDS writes are waited for
    // before the next barrier. Tile k+1 (issued at step k+2-S) has landed once at most
    // (S-2)*OPS newer instructions (those of steps k+3-S .. k) remain.
    auto conv = [&]() __attribute__((always_inline)) {
      if constexpr (kConvV) {
        if (k >= -1) {
          wait_vm(std::integral_constant<int, (S - 2) * OPS>{});
          convert_v(((KC + 1) % S + S) % S);
        }
      }
    };
    if (k >= 0 && k < ntiles) compute(k, ((KC % S) + S) % S, conv);
    else conv();
    __asm__ volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
  };

  if (ntiles > 0) {
    // prologue: steps -A .. -1
    [&]<int... Is>(std::integer_sequence<int, Is...>) __attribute__((always_inline)) {
      (step(std::integral_constant<int, Is - A>{}, 0), ...);
    }(std::make_integer_sequence<int, A>{});
    auto group = [&]<int... Is>(std::integer_sequence<int, Is...>, int n) __attribute__((always_inline)) {
      (step(std::integral_constant<int, Is>{}, n), ...);
    };
    for (int n = 0; n < ntiles; n += S) group(std::make_integer_sequence<int, S>{}, n);
    wait_vm(std::integral_constant<int, 0>{});  // no DMA may land after the workgroup ends
  }

  // ---- epilogue: normalise and write this lane's rows ----
#pragma unroll
  for (int rb = 0; rb < kXRB; ++rb) {
    // D[0][row] sits in element 0 of lane `row` (0..15)
    const float lt = __builtin_bit_cast(float, shfl_i(__builtin_bit_cast(int, lacc[rb][0]), c));
    if (!real[rb]) continue;
    const int r = r0 + wave * (kXRB * 16) + rb * 16 + c;
    const int t = r / a.group;
    const int g = r - t * a.group;
    const float inv = (lt > 0.f) ? a.v_scale / lt : 0.f;
    const int64_t off = (int64_t)(tok0 + t) * a.out_stride_tok + (int64_t)(h * a.group + g) * a.out_stride_head;
#pragma unroll
    for (int db = 0; db < DB; ++db)
      if (!PAD || db * 16 + 4 * j < a.head_dim)
        store_out4<QBF16>(a.out, off + db * 16 + 4 * j, o[rb][db], inv, a.out_f32);
  }
}

template <int D, bool QBF16, int HD>
static hipError_t launch_extend_q(int kv, dim3 grid, hipStream_t st, const ExtendArgs& a) {
  if (kv == DT_E4M3)
    hipLaunchKernelGGL((extend_kernel<D, QBF16, DT_E4M3, HD>), grid, dim3(kXWaves * 64), 0, st, a);
  else if (kv == DT_E5M2)
    hipLaunchKernelGGL((extend_kernel<D, QBF16, DT_E5M2, HD>), grid, dim3(kXWaves * 64), 0, st, a);
  else
    hipLaunchKernelGGL((extend_kernel<D, QBF16, QBF16 ? DT_BF16 : DT_F16, HD>), grid, dim3(kXWaves * 64), 0, st, a);
  return hipGetLastError();
}

// Padded head dims with kernels of their own (their zero score steps and output blocks
// skipped at compile time): 96 on the 128 kernel, 192 on the 256 kernel.
template <int D>
constexpr int kStaticPad = D == 128 ? 96 : D == 256 ? 192 : 0;

template <int D>
static hipError_t launch_extend_d(bool qbf16, int kv, dim3 grid, hipStream_t st, const ExtendArgs& a) {
  if (a.head_dim == D)
    return qbf16 ? launch_extend_q<D, true, D>(kv, grid, st, a) : launch_extend_q<D, false, D>(kv, grid, st, a);
  if constexpr (kStaticPad<D> != 0) {
    if (a.head_dim == kStaticPad<D>)
      return qbf16 ? launch_extend_q<D, true, kStaticPad<D>>(kv, grid, st, a)
                   : launch_extend_q<D, false, kStaticPad<D>>(kv, grid, st, a);
  }
  return qbf16 ? launch_extend_q<D, true, 0>(kv, grid, st, a) : launch_extend_q<D, false, 0>(kv, grid, st, a);
}

}  // namespace ma

using namespace ma;

static int64_t extend_items(int64_t num_tokens, int group, int batch, int bm) {
  // sum over sequences of ceil(ntok * G / bm) <= num_tokens * G / bm + batch
  return (num_tokens * group + bm - 1) / bm + batch;
}

// The tiled extend kernel that serves a head dim: 64, 128 or 256, padded up from the
// multiples of 16 below (their MFMA work is that of the padded dim), or 0 above 256 (the
// any-head-dim kernel).
static int extend_kernel_dim(int head_dim) {
  if (head_dim < 16 || head_dim % 16) return 0;
  return head_dim <= 64 ? 64 : head_dim <= 128 ? 128 : head_dim <= 256 ? 256 : 0;
}

// Rows per workgroup of the extend kernel at a head dim (0 if unsupported).
static int extend_tile_rows(int head_dim) {
  const int d = extend_kernel_dim(head_dim);
  return d == 64 ? XShape<64>::BM : d == 128 ? XShape<128>::BM : d == 256 ? XShape<256>::BM : 0;
}

extern "C" size_t ma_extend_workspace_bytes(int64_t num_tokens, int num_q_heads, int num_kv_heads, int batch) {
  if (num_tokens < 0 || batch < 0 || num_q_heads <= 0 || num_kv_heads <= 0 || num_q_heads % num_kv_heads) return 0;
  // sized for the smallest row tile, so one workspace serves every head dim
  const int64_t n = extend_items(num_tokens, num_q_heads / num_kv_heads, batch, kXBMMin);
  return ((size_t)n * sizeof(int64_t) + 255) & ~(size_t)255;
}

extern "C" int ma_paged_extend(
    const void* q, int64_t q_stride_tok, int64_t q_stride_head, int q_dtype, int64_t num_tokens,
    const void* k_cache, const void* v_cache, int64_t kv_stride_row, int64_t kv_stride_head, int kv_dtype,
    const int32_t* table, int64_t table_stride, const int64_t* row_index, int page_size,
    const int32_t* seq_lens, const int32_t* query_start_loc, const int32_t* prefix_lens,
    int batch, int num_q_heads, int num_kv_heads, int head_dim,
    int causal, int sliding_window, float softmax_scale, float k_scale, float v_scale,
    void* workspace, size_t workspace_bytes, void* out, int out_dtype, int64_t out_stride_tok,
    int64_t out_stride_head, void* stream) {
  // head dims up to 256 run on the tiled kernels (padded up to 64, 128 or 256), the
  // wider ones on the any-head-dim kernel
  const int kdim = extend_kernel_dim(head_dim);
  const bool generic = kdim == 0 && any_head_dim(head_dim);
  const int bm = generic ? kAnyPlanRows : extend_tile_rows(head_dim);
  if (bm == 0) return set_error(MA_EUNSUPPORTED, "head_dim %d not supported (multiples of 16 up to %d)", head_dim, kAnyMaxDim);
  if (q_dtype != DT_F16 && q_dtype != DT_BF16) return set_error(MA_EINVAL, "q dtype %d must be f16 or bf16", q_dtype);
  if (kv_dtype < 0 || kv_dtype > DT_E5M2) return set_error(MA_EINVAL, "kv dtype %d unknown", kv_dtype);
  if ((kv_dtype == DT_F16 || kv_dtype == DT_BF16) && kv_dtype != q_dtype)
    return set_error(MA_EINVAL, "16-bit KV dtype must equal the query dtype");
  if (out_dtype != q_dtype && out_dtype != DT_F32) return set_error(MA_EINVAL, "out dtype %d must be the query dtype or f32", out_dtype);
  if (batch < 0 || num_q_heads <= 0 || num_kv_heads <= 0 || num_q_heads % num_kv_heads)
    return set_error(MA_EINVAL, "bad head counts hq=%d hkv=%d", num_q_heads, num_kv_heads);
  if (page_size <= 0 || (page_size & (page_size - 1))) return set_error(MA_EINVAL, "page size %d must be a power of two", page_size);
  if (!(softmax_scale * k_scale > 0.f)) return set_error(MA_EINVAL, "softmax scale must be positive");
  if (num_tokens < 0 || num_tokens > 0x7fffffff) return set_error(MA_EINVAL, "num_tokens %lld out of range", (long long)num_tokens);
  if (batch > kPlanMaxBatch) return set_error(MA_EUNSUPPORTED, "batch %d exceeds %d sequences", batch, kPlanMaxBatch);
  if (batch == 0 || num_tokens == 0) return MA_OK;
  if (!q || !k_cache || !v_cache || !table || !seq_lens || !query_start_loc || !out)
    return set_error(MA_EINVAL, "null pointer argument");
  if ((reinterpret_cast<uintptr_t>(q) | reinterpret_cast<uintptr_t>(k_cache) | reinterpret_cast<uintptr_t>(v_cache) |
       reinterpret_cast<uintptr_t>(out)) & 15)
    return set_error(MA_EINVAL, "q, k, v and out must be 16-byte aligned");
  const int elt = (kv_dtype >= DT_E4M3) ? 1 : 2;
  if (kv_stride_row * elt >= ((int64_t)1 << 32))
    return set_error(MA_EUNSUPPORTED, "KV row stride of %lld bytes exceeds 4 GiB", (long long)(kv_stride_row * elt));
  const int out_elt = out_dtype == DT_F32 ? 4 : 2;
  const int out_align = out_dtype == DT_F32 ? 15 : 7;  // f32x4 or 4 x 16-bit stores
  if (((kv_stride_row * elt) & 15) || ((kv_stride_head * elt) & 15) || ((q_stride_tok * 2) & 15) ||
      ((q_stride_head * 2) & 15) || ((out_stride_tok * out_elt) & out_align) || ((out_stride_head * out_elt) & out_align))
    return set_error(MA_EINVAL, "strides must keep rows 16-byte aligned");
  const int group = num_q_heads / num_kv_heads;
  const int64_t items = extend_items(num_tokens, group, batch, bm);
  if (items * num_kv_heads > 0x7fffffff / (kXWaves * 64)) return set_error(MA_EINVAL, "grid too large");
  const size_t need = ma_extend_workspace_bytes(num_tokens, num_q_heads, num_kv_heads, batch);
  if (!workspace || workspace_bytes < need)
    return set_error(MA_EINVAL, "workspace too small: %zu < %zu bytes", workspace_bytes, need);
  if (reinterpret_cast<uintptr_t>(workspace) & 255) return set_error(MA_EINVAL, "workspace must be 256-byte aligned");
  ExtendPlanArgs p{};
  p.qsl = query_start_loc; p.seq_lens = seq_lens; p.prefix = prefix_lens;
  p.num_tokens = (int)num_tokens;
  p.batch = batch; p.group = group; p.causal = causal ? 1 : 0; p.window = sliding_window < 0 ? -1 : sliding_window;
  p.tile_rows = bm;
  p.tile_keys = generic ? kAnyKeys : kdim == 256 ? XShape<256>::BN : XShape<128>::BN;
  p.capacity = (int)items; p.items = reinterpret_cast<int64_t*>(workspace);
  hipLaunchKernelGGL(extend_plan_kernel, dim3(1), dim3(kPlanThreads), 0, (hipStream_t)stream, p);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return set_error(MA_ELAUNCH, "extend plan launch failed: %s", hipGetErrorString(e));
  if (generic) {
    AnyArgs g{};
    g.q = q; g.q_stride_tok = q_stride_tok; g.q_stride_head = q_stride_head;
    g.k = k_cache; g.v = v_cache; g.kv_stride_row = kv_stride_row; g.kv_stride_head = kv_stride_head;
    g.tt.table = table; g.tt.stride = table_stride; g.tt.page_shift = __builtin_ctz(page_size);
    g.row_index = row_index; g.seq_lens = seq_lens; g.qsl = query_start_loc; g.prefix = prefix_lens;
    g.num_tokens = (int)num_tokens; g.batch = batch; g.hq = num_q_heads; g.hkv = num_kv_heads; g.group = group;
    g.head_dim = head_dim; g.items = p.items; g.row_blocks = 0; g.pieces = 1;
    g.causal = p.causal; g.window = p.window;
    g.scale_log2 = softmax_scale * k_scale * kLog2e; g.v_scale = v_scale;
    g.out = out; g.out_stride_tok = out_stride_tok; g.out_stride_head = out_stride_head;
    g.out_f32 = out_dtype == DT_F32;
    e = any_launch(g, q_dtype, kv_dtype, items * num_kv_heads, (hipStream_t)stream);
    if (e != hipSuccess) return set_error(MA_ELAUNCH, "any-head-dim launch failed: %s", hipGetErrorString(e));
    return MA_OK;
  }
  ExtendArgs a{};
  a.q = q; a.q_stride_tok = q_stride_tok; a.q_stride_head = q_stride_head;
  a.k = k_cache; a.v = v_cache; a.kv_stride_row = kv_stride_row; a.kv_stride_head = kv_stride_head;
  a.tt.table = table; a.tt.stride = table_stride; a.tt.page_shift = __builtin_ctz(page_size);
  a.row_index = row_index; a.seq_lens = seq_lens; a.qsl = query_start_loc; a.prefix = prefix_lens;
  a.num_tokens = (int)num_tokens;
  a.batch = batch; a.hq = num_q_heads; a.hkv = num_kv_heads; a.group = group;
  a.items = p.items;
  a.causal = p.causal; a.window = p.window;
  a.scale_log2 = softmax_scale * k_scale * kLog2e; a.v_scale = v_scale;
  a.out = out; a.out_stride_tok = out_stride_tok; a.out_stride_head = out_stride_head;
  a.out_f32 = out_dtype == DT_F32;
  const dim3 grid((unsigned)(items * num_kv_heads));
  const bool qbf16 = q_dtype == DT_BF16;
  a.head_dim = head_dim;
  a.chunks = head_dim * elt / 16;  // >= 1: head_dim is a multiple of 16
  e = kdim == 64    ? launch_extend_d<64>(qbf16, kv_dtype, grid, (hipStream_t)stream, a)
      : kdim == 128 ? launch_extend_d<128>(qbf16, kv_dtype, grid, (hipStream_t)stream, a)
                    : launch_extend_d<256>(qbf16, kv_dtype, grid, (hipStream_t)stream, a);
  if (e != hipSuccess) return set_error(MA_ELAUNCH, "extend launch failed: %s", hipGetErrorString(e));
  return MA_OK;
}
