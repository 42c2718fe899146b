// Segment routing (score -> top-k -> softmax) and residual fusion, gfx950.
//
// Routing follows SegmentRecurrentMemoryModel._route_chunk
// (reference grm/core/paper_grm.py:566-589) and TopKMemoryRetriever.forward
// (grm/core/gating_unit.py:54-91):
//   score[q, s] = scale * <query_q, key_s>;  k' = min(top_k, S)
//   k' < S : the k' largest scores, descending      (torch.topk, sorted)
//   k' == S: all scores in index order, idx = arange  (the arange branch)
//   gates  = softmax(selected / temperature)
// torch.topk leaves the order of equal scores unspecified; here ties go to the
// lower segment index, and every score is a single fp32 FMA chain over d in
// increasing order, so the result is reproducible on any IEEE machine.
//
// One thread owns one query row: it streams the keys of its batch entry from
// LDS (16-byte broadcast reads, one per 8 FMAs) and keeps its running top-k
// sorted in registers.
//
// Fusion follows RetrievedStateFusion residual mode
// (reference grm/core/aggregator.py:67-145): LayerNorm(h + sum_r g_r * r_r),
// biased variance, eps inside the square root; one wave per row.
#include <stdint.h>
#include <string.h>

#include <cmath>

#include "grm_hip.h"
#include "grm_hip_common.h"

namespace grmhip {
namespace {

constexpr int RT = 256;  // threads (= query rows) per routing workgroup
constexpr int SC = 32;   // keys per LDS tile
constexpr int DT = 128;  // key dims per LDS tile

struct RouteArgs {
  const void* q;
  const void* keys;
  int64_t* idx;
  float* scores;
  float* gates;
  int64_t n_query;
  int64_t n_keys;
  int dim;
  int k;        // selected per query (k <= n_keys)
  int natural;  // k == n_keys: index order, no selection
  int vec;      // 16-byte loads of query rows legal
  float scale;
  float inv_temp;
};

template <class E, int KMAX>
__global__ __launch_bounds__(RT) void route_kernel(const RouteArgs a) {
  using raw = typename ET<E>::raw;
  constexpr int V = 16 / sizeof(raw);  // elements per 16-byte LDS read
  __shared__ __align__(16) raw ktile[SC * DT];
  __shared__ float sbuf[SC * RT];  // per-thread columns of one tile's scores

  const int64_t b = blockIdx.y;
  const int64_t qi = static_cast<int64_t>(blockIdx.x) * RT + threadIdx.x;
  const bool active = qi < a.n_query;
  const int D = a.dim;
  const int64_t S = a.n_keys;
  const raw* qrow = static_cast<const raw*>(a.q) + (b * a.n_query + (active ? qi : 0)) * D;
  const raw* kb = static_cast<const raw*>(a.keys) + b * S * D;
  const int64_t obase = (b * a.n_query + qi) * a.k;

  // Running top-k, descending.  Slots at or past k only receive entries
  // shifted out of the top k; the k-th best score is kept in thr for the
  // cheap reject test, so a candidate enters the network only if it belongs
  // in the top k.
  float top_s[KMAX];
  int top_i[KMAX];
  const int k = a.k;
#pragma unroll
  for (int m = 0; m < KMAX; ++m) {
    top_s[m] = (m < k) ? -INFINITY : INFINITY;
    top_i[m] = -1;
  }
  float thr = -INFINITY;

  for (int64_t s0 = 0; s0 < S; s0 += SC) {
    float acc[SC];
#pragma unroll
    for (int s = 0; s < SC; ++s) acc[s] = 0.f;
    for (int d0 = 0; d0 < D; d0 += DT) {
      const int dl = min(DT, D - d0);
      __syncthreads();
      for (int e = threadIdx.x; e < SC * DT; e += RT) {
        const int s = e / DT, d = e % DT;
        ktile[e] = (s0 + s < S && d < dl) ? kb[(s0 + s) * D + d0 + d] : static_cast<raw>(0);
      }
      __syncthreads();
      if (active) {
        for (int dd = 0; dd < dl; dd += V) {
          float x[V];
          if (a.vec && dd + V <= dl) {
            if constexpr (V == 8) {
              const U8<E> u = *reinterpret_cast<const U8<E>*>(qrow + d0 + dd);
#pragma unroll
              for (int i = 0; i < 8; ++i) x[i] = ET<E>::to_f(u.e[i]);
            } else {
              const float4 f = *reinterpret_cast<const float4*>(qrow + d0 + dd);
              x[0] = f.x; x[1] = f.y; x[2] = f.z; x[3] = f.w;
            }
          } else {
#pragma unroll
            for (int i = 0; i < V; ++i) x[i] = (dd + i < dl) ? ET<E>::to_f(qrow[d0 + dd + i]) : 0.f;
          }
          const int nv = min(V, dl - dd);
#pragma unroll
          for (int s = 0; s < SC; ++s) {
            struct KV { raw e[V]; };
            const KV kv = __builtin_bit_cast(KV, *reinterpret_cast<const uint4*>(ktile + s * DT + dd));
            if (nv == V) {
#pragma unroll
              for (int i = 0; i < V; ++i) acc[s] = fmaf(x[i], ET<E>::to_f(kv.e[i]), acc[s]);
            } else {
#pragma unroll
              for (int i = 0; i < V; ++i)
                if (i < nv) acc[s] = fmaf(x[i], ET<E>::to_f(kv.e[i]), acc[s]);
            }
          }
        }
      }
    }
    if (active) {
      const int ns = static_cast<int>(min(static_cast<int64_t>(SC), S - s0));
      if (a.natural) {
#pragma unroll
        for (int s = 0; s < SC; ++s) {
          if (s < ns) {
            a.scores[obase + s0 + s] = acc[s] * a.scale;
            a.idx[obase + s0 + s] = s0 + s;
          }
        }
      } else {
        // Park the tile's scores in this thread's LDS column, then insert them
        // with one (not unrolled) pass so the network is emitted once.
#pragma unroll
        for (int s = 0; s < SC; ++s) sbuf[s * RT + threadIdx.x] = acc[s] * a.scale;
#pragma unroll 1
        for (int s = 0; s < ns; ++s) {
          const float v = sbuf[s * RT + threadIdx.x];
          if (v > thr) {
            // The new entry lands after every kept entry with an equal score
            // (those have lower indices); from there on every entry shifts
            // down one slot, keeping equal scores in index order.
            float cs = v;
            int ci = static_cast<int>(s0 + s);
            bool shift = false;
#pragma unroll
            for (int m = 0; m < KMAX; ++m) {
              shift = shift || (cs > top_s[m]);
              if (shift) {
                const float ts = top_s[m];
                const int ti = top_i[m];
                top_s[m] = cs;
                top_i[m] = ci;
                cs = ts;
                ci = ti;
              }
            }
#pragma unroll
            for (int m = 0; m < KMAX; ++m) thr = (m == k - 1) ? top_s[m] : thr;
          }
        }
      }
    }
  }
  if (!active) return;
  if (a.natural) {
    float mx = -INFINITY;
    for (int64_t s = 0; s < k; ++s) mx = fmaxf(mx, a.scores[obase + s] * a.inv_temp);
    float sum = 0.f;
    for (int64_t s = 0; s < k; ++s) sum += expf(a.scores[obase + s] * a.inv_temp - mx);
    for (int64_t s = 0; s < k; ++s)
      a.gates[obase + s] = expf(a.scores[obase + s] * a.inv_temp - mx) / sum;
    return;
  }
  const float mx = top_s[0] * a.inv_temp;
  float e[KMAX];
  float sum = 0.f;
#pragma unroll
  for (int m = 0; m < KMAX; ++m) {
    e[m] = (m < k) ? expf(top_s[m] * a.inv_temp - mx) : 0.f;
    sum += e[m];
  }
#pragma unroll
  for (int m = 0; m < KMAX; ++m) {
    if (m < k) {
      a.idx[obase + m] = top_i[m];
      a.scores[obase + m] = top_s[m];
      a.gates[obase + m] = e[m] / sum;
    }
  }
}

template <class E>
int launch_route(const RouteArgs& a, int64_t batch, hipStream_t s) {
  const dim3 grid(static_cast<unsigned>((a.n_query + RT - 1) / RT), static_cast<unsigned>(batch));
  const int km = a.natural ? 1 : a.k;
  if (km <= 8) {
    hipLaunchKernelGGL((route_kernel<E, 8>), grid, dim3(RT), 0, s, a);
  } else if (km <= 16) {
    hipLaunchKernelGGL((route_kernel<E, 16>), grid, dim3(RT), 0, s, a);
  } else {
    hipLaunchKernelGGL((route_kernel<E, 32>), grid, dim3(RT), 0, s, a);
  }
  return check_launch("topk_route");
}

// ---------------------------------------------------------------------------
struct FuseArgs {
  const void* h;
  const void* ret;
  const float* gates;
  const void* w;
  const void* bias;
  void* out;
  int64_t rows;
  int routes;
  int hidden;
  float eps;
};

constexpr int FMAX = 32;  // hidden elements per lane -> hidden <= 2048

template <class E>
__global__ __launch_bounds__(256) void fuse_kernel(const FuseArgs a) {
  using raw = typename ET<E>::raw;
  const int lane = threadIdx.x & 63;
  const int64_t row = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  if (row >= a.rows) return;
  const int H = a.hidden;
  const raw* h = static_cast<const raw*>(a.h) + row * H;
  const raw* ret = static_cast<const raw*>(a.ret) + row * a.routes * H;
  const float* g = a.gates + row * a.routes;
  float x[FMAX];
  float sum = 0.f;
#pragma unroll
  for (int i = 0; i < FMAX; ++i) {
    const int c = lane + 64 * i;
    x[i] = 0.f;
    if (c < H) {
      float v = ET<E>::to_f(h[c]);
      float r = 0.f;
      for (int j = 0; j < a.routes; ++j) r = fmaf(g[j], ET<E>::to_f(ret[j * H + c]), r);
      x[i] = v + r;
      sum += x[i];
    }
  }
  for (int off = 32; off > 0; off >>= 1) sum += __shfl_xor(sum, off, 64);
  raw* out = static_cast<raw*>(a.out) + row * H;
  if (a.w == nullptr) {
#pragma unroll
    for (int i = 0; i < FMAX; ++i) {
      const int c = lane + 64 * i;
      if (c < H) out[c] = ET<E>::from_f(x[i]);
    }
    return;
  }
  const float mean = sum / static_cast<float>(H);
  float var = 0.f;
#pragma unroll
  for (int i = 0; i < FMAX; ++i) {
    const int c = lane + 64 * i;
    if (c < H) {
      const float d = x[i] - mean;
      var = fmaf(d, d, var);
    }
  }
  for (int off = 32; off > 0; off >>= 1) var += __shfl_xor(var, off, 64);
  const float rstd = 1.0f / sqrtf(var / static_cast<float>(H) + a.eps);
  const raw* w = static_cast<const raw*>(a.w);
  const raw* bias = static_cast<const raw*>(a.bias);
#pragma unroll
  for (int i = 0; i < FMAX; ++i) {
    const int c = lane + 64 * i;
    if (c < H) {
      const float y = (x[i] - mean) * rstd * ET<E>::to_f(w[c]) +
                      (bias != nullptr ? ET<E>::to_f(bias[c]) : 0.f);
      out[c] = ET<E>::from_f(y);
    }
  }
}

bool aligned(const void* p, size_t n) { return (reinterpret_cast<uintptr_t>(p) % n) == 0; }

}  // namespace
}  // namespace grmhip

using namespace grmhip;

extern "C" int grm_hip_topk_route(const void* queries, const void* keys, int64_t* topk_indices,
                                  float* topk_scores, float* gates, int64_t batch, int64_t n_query,
                                  int64_t n_keys, int64_t dim, int dtype, int64_t top_k,
                                  float scale, float temperature, void* stream) {
  if (batch < 0 || n_query < 0 || n_keys < 0 || dim < 0 || top_k < 1) {
    set_error("topk_route: bad sizes");
    return GRM_HIP_EINVAL;
  }
  if (dtype < GRM_HIP_F32 || dtype > GRM_HIP_BF16) {
    set_error("topk_route: unsupported dtype %d", dtype);
    return GRM_HIP_EUNSUPPORTED;
  }
  if (!(temperature > 0.f) || !std::isfinite(scale)) {
    set_error("topk_route: temperature must be > 0 and scale finite");
    return GRM_HIP_EINVAL;
  }
  const int64_t k = top_k < n_keys ? top_k : n_keys;
  const bool natural = k == n_keys;
  if (!natural && k > 32) {
    set_error("topk_route: top_k %lld > 32", (long long)k);
    return GRM_HIP_EUNSUPPORTED;
  }
  if (batch == 0 || n_query == 0 || k == 0) return GRM_HIP_OK;
  if (batch > 65535 || dim > INT32_MAX || n_keys > INT32_MAX) {
    set_error("topk_route: batch > 65535 or dims too large");
    return GRM_HIP_EUNSUPPORTED;
  }
  if (queries == nullptr || keys == nullptr || topk_indices == nullptr || topk_scores == nullptr ||
      gates == nullptr) {
    set_error("topk_route: null pointer");
    return GRM_HIP_EINVAL;
  }
  RouteArgs a;
  memset(&a, 0, sizeof(a));
  a.q = queries;
  a.keys = keys;
  a.idx = topk_indices;
  a.scores = topk_scores;
  a.gates = gates;
  a.n_query = n_query;
  a.n_keys = n_keys;
  a.dim = static_cast<int>(dim);
  a.k = static_cast<int>(k);
  a.natural = natural ? 1 : 0;
  const int eb = dtype == GRM_HIP_F32 ? 4 : 2;
  a.vec = (dim * eb) % 16 == 0 && aligned(queries, 16);
  a.scale = scale;
  a.inv_temp = 1.0f / temperature;
  hipStream_t s = static_cast<hipStream_t>(stream);
  switch (dtype) {
    case GRM_HIP_F32: return launch_route<F32>(a, batch, s);
    case GRM_HIP_F16: return launch_route<F16>(a, batch, s);
    default: return launch_route<BF16>(a, batch, s);
  }
}

extern "C" int grm_hip_fuse_residual(const void* h_online, const void* retrieved,
                                     const float* gates, const void* ln_weight,
                                     const void* ln_bias, void* out, int64_t rows, int64_t routes,
                                     int64_t hidden_size, int dtype, float eps, void* stream) {
  if (rows < 0 || routes < 0 || hidden_size < 0) {
    set_error("fuse_residual: negative size");
    return GRM_HIP_EINVAL;
  }
  if (dtype < GRM_HIP_F32 || dtype > GRM_HIP_BF16) {
    set_error("fuse_residual: unsupported dtype %d", dtype);
    return GRM_HIP_EUNSUPPORTED;
  }
  if (hidden_size > 64 * FMAX || routes > INT32_MAX) {
    set_error("fuse_residual: hidden_size %lld > %d", (long long)hidden_size, 64 * FMAX);
    return GRM_HIP_EUNSUPPORTED;
  }
  if (rows == 0 || hidden_size == 0) return GRM_HIP_OK;
  if (h_online == nullptr || out == nullptr || (routes > 0 && (retrieved == nullptr || gates == nullptr))) {
    set_error("fuse_residual: null pointer");
    return GRM_HIP_EINVAL;
  }
  FuseArgs a;
  a.h = h_online;
  a.ret = retrieved;
  a.gates = gates;
  a.w = ln_weight;
  a.bias = ln_bias;
  a.out = out;
  a.rows = rows;
  a.routes = static_cast<int>(routes);
  a.hidden = static_cast<int>(hidden_size);
  a.eps = eps;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const dim3 grid(static_cast<unsigned>((rows + 3) / 4));
  switch (dtype) {
    case GRM_HIP_F32: hipLaunchKernelGGL(fuse_kernel<F32>, grid, dim3(256), 0, s, a); break;
    case GRM_HIP_F16: hipLaunchKernelGGL(fuse_kernel<F16>, grid, dim3(256), 0, s, a); break;
    default: hipLaunchKernelGGL(fuse_kernel<BF16>, grid, dim3(256), 0, s, a); break;
  }
  return check_launch("fuse_residual");
}
