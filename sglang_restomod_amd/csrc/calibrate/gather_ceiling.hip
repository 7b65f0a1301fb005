// Measurement kernel (not part of the attention library): the HBM read bandwidth of
// gathering rows of a token pool [num_tokens, heads, row_bytes] from random slots, with
// no arithmetic. It gives an attainable rate for the KV access pattern of paged decode
// with page size 1: rows of one kv head (64 to 1024 B: D=128 in 16 bits is 256 B) at
// random pool slots, each row read once per kv head, in the decode's head-major order.
//
// Workgroup (x, h): 4 waves; a wave reads the rows of head h for chunks_per_wave chunks of
// 64 consecutive entries of `perm` (its slots). Each lane loads one slot per chunk, and
// the rows of each 1 KB load instruction take their slots by ds_bpermute, so the row
// loads of a chunk (row_bytes / 16 loads of 1 KB) are in flight together while
// the next chunk's slots load. The XOR of everything read goes to one word per thread.
// Rows load with the nontemporal hint, like the attention kernels' K and V rows (on
// this pattern that reaches 6.4-6.5 TB/s where default-policy loads reach 5.7-5.8).

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
constexpr int kThreads = 256;
constexpr int kChunk = 64;  // slots per chunk: one per lane

template <int ROW>
__global__ __launch_bounds__(kThreads) void gather_ceiling_kernel(const unsigned char* pool, const int32_t* perm,
                                                                  int64_t num_tokens, int heads,
                                                                  int chunks_per_wave, uint32_t* sink) {
  constexpr int kLanesPerRow = ROW / 16;
  constexpr int kRowsPerInst = 64 / kLanesPerRow;
  constexpr int kInsts = kChunk / kRowsPerInst;
  const int lane = threadIdx.x & 63;
  const int64_t wave = (int64_t)blockIdx.x * (kThreads / 64) + (threadIdx.x >> 6);
  const int h = blockIdx.y;
  const int64_t token_bytes = (int64_t)heads * ROW;
  const unsigned char* base = pool + (int64_t)h * ROW + (lane % kLanesPerRow) * 16;
  const int64_t nchunks = (num_tokens + kChunk - 1) / kChunk;
  int64_t c = wave * chunks_per_wave;
  int64_t t = c * kChunk + lane;
  int slot = perm[t < num_tokens ? t : num_tokens - 1];
  uint32_t acc = 0;
  for (int k = 0; k < chunks_per_wave && c < nchunks; ++k, ++c) {
    const int64_t tn = (c + 1) * kChunk + lane;
    const int next = perm[tn < num_tokens ? tn : num_tokens - 1];
    u32x4 v[kInsts];
#pragma unroll
    for (int u = 0; u < kInsts; ++u) {
      const int s = __shfl(slot, u * kRowsPerInst + lane / kLanesPerRow, 64);
      v[u] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(base + (int64_t)(uint32_t)s * token_bytes));
    }
#pragma unroll
    for (int u = 0; u < kInsts; ++u) acc ^= v[u][0] ^ v[u][1] ^ v[u][2] ^ v[u][3];
    slot = next;
  }
  sink[((int64_t)blockIdx.y * gridDim.x + blockIdx.x) * kThreads + threadIdx.x] = acc;
}

}  // namespace

// Sink words needed for the given sizes; 0 on bad sizes.
extern "C" int64_t ma_gather_ceiling_sink_words(int64_t num_tokens, int heads, int chunks_per_wave) {
  if (num_tokens <= 0 || heads <= 0 || heads > 65535 || chunks_per_wave <= 0) return 0;
  const int64_t nchunks = (num_tokens + kChunk - 1) / kChunk;
  const int64_t waves = (nchunks + chunks_per_wave - 1) / chunks_per_wave;
  const int64_t bx = (waves + kThreads / 64 - 1) / (kThreads / 64);
  return bx * heads * kThreads;
}

// perm: num_tokens slots in [0, num_tokens); pool: num_tokens * heads * row_bytes bytes.
extern "C" int ma_gather_ceiling(const void* pool, const int32_t* perm, int64_t num_tokens, int heads, int row_bytes,
                                 int chunks_per_wave, uint32_t* sink, int64_t sink_words, void* stream) {
  const int64_t words = ma_gather_ceiling_sink_words(num_tokens, heads, chunks_per_wave);
  if (words <= 0 || !pool || !perm || !sink || sink_words < words) return -1;
  const int64_t bx = words / ((int64_t)heads * kThreads);
  if (bx > 0x7fffffff) return -1;
  const dim3 grid((unsigned)bx, (unsigned)heads);
  const unsigned char* p = reinterpret_cast<const unsigned char*>(pool);
  hipStream_t st = (hipStream_t)stream;
  if (row_bytes == 1024)
    hipLaunchKernelGGL(gather_ceiling_kernel<1024>, grid, dim3(kThreads), 0, st, p, perm, num_tokens, heads,
                       chunks_per_wave, sink);
  else if (row_bytes == 512)
    hipLaunchKernelGGL(gather_ceiling_kernel<512>, grid, dim3(kThreads), 0, st, p, perm, num_tokens, heads,
                       chunks_per_wave, sink);
  else if (row_bytes == 256)
    hipLaunchKernelGGL(gather_ceiling_kernel<256>, grid, dim3(kThreads), 0, st, p, perm, num_tokens, heads,
                       chunks_per_wave, sink);
  else if (row_bytes == 128)
    hipLaunchKernelGGL(gather_ceiling_kernel<128>, grid, dim3(kThreads), 0, st, p, perm, num_tokens, heads,
                       chunks_per_wave, sink);
  else if (row_bytes == 64)
    hipLaunchKernelGGL(gather_ceiling_kernel<64>, grid, dim3(kThreads), 0, st, p, perm, num_tokens, heads,
                       chunks_per_wave, sink);
  else
    return -1;
  return hipGetLastError() == hipSuccess ? 0 : -2;
}
