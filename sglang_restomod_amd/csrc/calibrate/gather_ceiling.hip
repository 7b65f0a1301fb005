// Measurement kernel (not part of the attention library): the HBM read bandwidth of
// gathering rows of a token pool [num_tokens, heads, row_bytes] through a permutation,
// with no compute. It gives the attainable ceiling for the KV access pattern of paged
// decode with page size 1: rows of one kv head (256 B for D=128 in 16 bits, 128 B in
// fp8) at random pool slots.
//   order 0: head-major, the order of the decode's segments: row i -> head i / N,
//            token perm[i % N]
//   order 1: head-minor: row i -> head i % heads, token perm[i / heads]
//   order 2: in order: row i -> head i % heads, token i / heads (a streaming read)
// Each lane reads 16 bytes; a wave reads 1 KB per instruction and keeps 8 in flight.
// The XOR of everything read goes to one word per thread so that no load is dropped.

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
constexpr int kThreads = 256;
constexpr int kInFlight = 8;

__global__ __launch_bounds__(kThreads) void gather_ceiling_kernel(const unsigned char* pool, const int32_t* perm,
                                                                  int64_t num_tokens, int heads, int row_bytes,
                                                                  int order, int rows_per_wave, uint32_t* sink) {
  const int lane = threadIdx.x & 63;
  const int64_t wave = ((int64_t)blockIdx.x * kThreads + threadIdx.x) >> 6;
  const int lanes_per_row = row_bytes / 16;
  const int rows_per_inst = 64 / lanes_per_row;
  const int64_t total = num_tokens * heads;
  const int64_t token_bytes = (int64_t)heads * row_bytes;
  const int64_t first = wave * rows_per_wave;
  uint32_t acc = 0;
  for (int it = 0; it < rows_per_wave; it += kInFlight * rows_per_inst) {
    u32x4 v[kInFlight];
#pragma unroll
    for (int u = 0; u < kInFlight; ++u) {
      int64_t row = first + it + u * rows_per_inst + lane / lanes_per_row;
      row = row < total ? row : total - 1;
      int64_t tok, head;
      if (order == 0) {
        head = row / num_tokens;
        tok = perm[row - head * num_tokens];
      } else {
        head = row % heads;
        tok = (order == 1) ? perm[row / heads] : row / heads;
      }
      v[u] = *reinterpret_cast<const u32x4*>(pool + tok * token_bytes + head * row_bytes + (lane % lanes_per_row) * 16);
    }
#pragma unroll
    for (int u = 0; u < kInFlight; ++u) acc ^= v[u][0] ^ v[u][1] ^ v[u][2] ^ v[u][3];
  }
  sink[(int64_t)blockIdx.x * kThreads + threadIdx.x] = acc;
}

}  // namespace

// Grid blocks needed for the given sizes (sink holds blocks * 256 words); 0 on bad sizes.
extern "C" int64_t ma_gather_ceiling_blocks(int64_t num_tokens, int heads, int row_bytes, int rows_per_wave) {
  if (num_tokens <= 0 || heads <= 0 || (row_bytes != 64 && row_bytes != 128 && row_bytes != 256 &&
                                        row_bytes != 512 && row_bytes != 1024))
    return 0;
  const int rows_per_step = kInFlight * (64 / (row_bytes / 16));
  if (rows_per_wave <= 0 || rows_per_wave % rows_per_step) return 0;
  const int64_t waves = (num_tokens * heads + rows_per_wave - 1) / rows_per_wave;
  return (waves + kThreads / 64 - 1) / (kThreads / 64);
}

extern "C" int ma_gather_ceiling(const void* pool, const int32_t* perm, int64_t num_tokens, int heads, int row_bytes,
                                 int order, int rows_per_wave, uint32_t* sink, int64_t sink_words, void* stream) {
  const int64_t blocks = ma_gather_ceiling_blocks(num_tokens, heads, row_bytes, rows_per_wave);
  if (blocks <= 0 || blocks > 0x7fffffff || order < 0 || order > 2 || !pool || !sink ||
      (order != 2 && !perm) || sink_words < blocks * kThreads)
    return -1;
  hipLaunchKernelGGL(gather_ceiling_kernel, dim3((unsigned)blocks), dim3(kThreads), 0, (hipStream_t)stream,
                     reinterpret_cast<const unsigned char*>(pool), perm, num_tokens, heads, row_bytes, order,
                     rows_per_wave, sink);
  return hipGetLastError() == hipSuccess ? 0 : -2;
}
