// Threshold-select routing kernel (route_select.hip): the bf16 top-k routing
// path for archives whose keys fit one CU's LDS.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace grmhip {

struct RouteSelArgs {
  const void* q;      // [batch, n_query, dim] bf16
  const void* keys;   // [batch, n_keys, dim] bf16
  int64_t* idx;       // [batch, n_query, k]
  float* scores;
  float* gates;
  int64_t n_query;
  int64_t n_keys;
  int dim;
  int k;              // selected per row (< n_keys without windows)
  float scale;
  float inv_temp;
  // seg_len > 0: row t sees the keys [lo, hi), hi = min(n_keys, base + t / seg_len),
  // lo = max(0, hi - cap); a window of at most k keys is taken whole in index order.
  int seg_len;
  int64_t base;
  int64_t cap;
};

// One row's top k, kept descending in ts / ti, written out: a slot whose score is
// not above -inf (NaN or -inf: never selected) or that was never filled is
// empty, (-1, -inf, 0); the gates are the softmax of the filled slots' scores
// over the temperature.  The filled slots come first (the list is descending).
template <int KMAX>
__device__ __forceinline__ void write_topk_row(int64_t* idx, float* scores, float* gates, int64_t obase, int k,
                                               float inv_temp, const float (&ts)[KMAX], const int (&ti)[KMAX]) {
  const bool any = ts[0] > -INFINITY;
  const float mx = any ? ts[0] * inv_temp : 0.f;
  float e[KMAX];
  float sum = 0.f;
#pragma unroll
  for (int m = 0; m < KMAX; ++m) {
    e[m] = (m < k && ts[m] > -INFINITY) ? expf(ts[m] * inv_temp - mx) : 0.f;
    sum += e[m];
  }
#pragma unroll
  for (int m = 0; m < KMAX; ++m) {
    if (m < k) {
      const bool f = ts[m] > -INFINITY;
      idx[obase + m] = f ? ti[m] : -1;
      scores[obase + m] = f ? ts[m] : -INFINITY;
      gates[obase + m] = f ? e[m] / sum : 0.f;
    }
  }
}

// Launches the threshold-select kernel when it covers these arguments and
// returns 1 with *rc the launch status; returns 0 (nothing launched) otherwise.
int try_route_select(const RouteSelArgs& a, int dtype, int64_t batch, hipStream_t s, int* rc);

}  // namespace grmhip
