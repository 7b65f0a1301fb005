// Query rows of one sequence from query_start_loc, clamped into the rows the caller's q
// and out actually have. Kept free of HIP headers so that a host-only build of this exact
// code can be tested on the CPU (tests/test_query_rows.py).
#pragma once

#include <stdint.h>

#if defined(__HIPCC__)
#define MA_HD __host__ __device__ __forceinline__
#else
#define MA_HD inline
#endif

namespace ma {

struct QueryRows {
  int tok0;  // first query row of the sequence
  int ntok;  // query rows of the sequence (>= 0)
};

// Sequence b owns rows [qsl[b], qsl[b+1]) by its metadata; the kernels read q and write
// out only inside [0, num_tokens), so the range is cut to that window: inconsistent
// metadata (qsl[batch] > num_tokens, a decreasing or negative entry) can shorten or
// empty a sequence but never address a row outside the buffers.
MA_HD QueryRows clamp_query_rows(int start, int end, int num_tokens) {
  const int n = num_tokens < 0 ? 0 : num_tokens;
  const int lo = start < 0 ? 0 : (start > n ? n : start);
  const int hi = end < lo ? lo : (end > n ? n : end);
  return QueryRows{lo, hi - lo};
}

}  // namespace ma

#undef MA_HD
