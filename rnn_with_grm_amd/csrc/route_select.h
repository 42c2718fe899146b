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

// Launches the threshold-select kernel when it covers these arguments and
// returns 1 with *rc the launch status; returns 0 (nothing launched) otherwise.
int try_route_select(const RouteSelArgs& a, int dtype, int64_t batch, hipStream_t s, int* rc);

}  // namespace grmhip
