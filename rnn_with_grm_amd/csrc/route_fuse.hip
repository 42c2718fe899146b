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

#include <cfloat>
#include <cmath>
#include <cstdlib>
#include <type_traits>

#include "grm_hip.h"
#include "grm_hip_common.h"
#include "route_select.h"

namespace grmhip {
namespace {

constexpr int RT = 256;  // threads (= query rows) per routing workgroup
constexpr int kRouteMaxK = 128;  // largest top_k routed on the GPU
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
  int k;        // selected per query (k <= n_keys; the output width when seg_len > 0)
  int natural;  // k == n_keys: index order, no selection
  int vec;      // 16-byte loads of query rows legal
  float scale;
  float inv_temp;
  // Segment windows (seg_len > 0): query row t belongs to segment
  // s = t / seg_len and sees the keys [lo, hi), hi = base + s,
  // lo = max(0, hi - cap): the archive as it stood when segment s ran.
  int seg_len;
  int64_t base;
  int64_t cap;
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

  // Keys this row may select, [lo, hi), and the keys the workgroup streams,
  // [blk_lo, blk_hi) (windows only move forward with the row index).  A row
  // whose window holds at most k keys takes all of them in index order.
  int64_t lo = 0, hi = S, blk_lo = 0, blk_hi = S;
  bool row_nat = false;
  if (a.seg_len > 0) {
    const int64_t r0 = static_cast<int64_t>(blockIdx.x) * RT;
    const int64_t r1 = min(a.n_query, r0 + RT) - 1;
    auto win_hi = [&](int64_t r) { return min(S, a.base + r / a.seg_len); };
    auto win_lo = [&](int64_t h) { return h > a.cap ? h - a.cap : int64_t{0}; };
    blk_hi = win_hi(r1);
    blk_lo = win_lo(win_hi(r0));
    hi = win_hi(active ? qi : r0);
    lo = win_lo(hi);
    row_nat = hi - lo <= a.k;
  }

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

  for (int64_t s0 = blk_lo; s0 < blk_hi; s0 += SC) {
    float acc[SC];
#pragma unroll
    for (int s = 0; s < SC; ++s) acc[s] = 0.f;
    for (int d0 = 0; d0 < D; d0 += DT) {
      const int dl = min(DT, D - d0);
      __syncthreads();
      for (int e = threadIdx.x; e < SC * DT; e += RT) {
        const int s = e / DT, d = e % DT;
        ktile[e] = (s0 + s < blk_hi && d < dl) ? kb[(s0 + s) * D + d0 + d] : static_cast<raw>(0);
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
      const int ns = static_cast<int>(min(static_cast<int64_t>(SC), blk_hi - s0));
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
          const int64_t key = s0 + s;
          if (a.seg_len > 0) {
            if (key < lo || key >= hi) continue;
            if (row_nat) {  // index order: slot key - lo
              const int slot = static_cast<int>(key - lo);
#pragma unroll
              for (int m = 0; m < KMAX; ++m) {
                if (m == slot) {
                  top_s[m] = v;
                  top_i[m] = static_cast<int>(key);
                }
              }
              continue;
            }
          }
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
  if (row_nat) {
    // Window of n <= k keys in index order; slots n .. k-1 stay empty
    // (index -1, score -inf, gate 0).
    const int n = static_cast<int>(hi - lo);
    float mx = -INFINITY;
#pragma unroll
    for (int m = 0; m < KMAX; ++m) mx = (m < n) ? fmaxf(mx, top_s[m] * a.inv_temp) : mx;
    float e[KMAX];
    float sum = 0.f;
#pragma unroll
    for (int m = 0; m < KMAX; ++m) {
      e[m] = (m < n) ? expf(top_s[m] * a.inv_temp - mx) : 0.f;
      sum += e[m];
    }
#pragma unroll
    for (int m = 0; m < KMAX; ++m) {
      if (m < k) {
        a.idx[obase + m] = (m < n) ? top_i[m] : -1;
        a.scores[obase + m] = (m < n) ? top_s[m] : -INFINITY;
        a.gates[obase + m] = (m < n) ? e[m] / sum : 0.f;
      }
    }
    return;
  }
  write_topk_row<KMAX>(a.idx, a.scores, a.gates, obase, k, a.inv_temp, top_s, top_i);
}

template <class E>
int launch_route(const RouteArgs& a, int64_t batch, hipStream_t s) {
  const dim3 grid(static_cast<unsigned>((a.n_query + RT - 1) / RT), static_cast<unsigned>(batch));
  const int km = a.natural ? 1 : a.k;
  if (km <= 8) {
    hipLaunchKernelGGL((route_kernel<E, 8>), grid, dim3(RT), 0, s, a);
  } else if (km <= 16) {
    hipLaunchKernelGGL((route_kernel<E, 16>), grid, dim3(RT), 0, s, a);
  } else if (km <= 32) {
    hipLaunchKernelGGL((route_kernel<E, 32>), grid, dim3(RT), 0, s, a);
  } else if (km <= 64) {  // lists past 32 entries: correct, not fast (registers spill)
    hipLaunchKernelGGL((route_kernel<E, 64>), grid, dim3(RT), 0, s, a);
  } else {
    hipLaunchKernelGGL((route_kernel<E, kRouteMaxK>), grid, dim3(RT), 0, s, a);
  }
  return check_launch("topk_route");
}

// ---------------------------------------------------------------------------
// Segment routing with short windows (grm_hip_segment_route when every
// workgroup's key range fits WR_MAXK keys).  Same result as route_kernel's
// window mode, bit for bit: every score is the same fp32 FMA chain.
//
// A workgroup owns WR_ROWS query rows with WR_LANES lanes per row; lane l of a
// row computes the chains of keys l, l + WR_LANES, ... of the workgroup's key
// range, so a row's keys are scored in parallel instead of by one thread.  Key
// and query slices are staged in LDS.  The top k then follow from ranks: a
// key's rank is the number of window keys that beat it (greater score, or an
// equal score and a lower index), so slot = rank for every key with rank < k,
// the order "score descending, ties to the lower index" with no serial
// insertion.  Keys whose score is NaN or -inf are never selected, as in
// route_kernel.
constexpr int WR_ROWS = 32;
constexpr int WR_LANES = 8;
constexpr int WR_THREADS = WR_ROWS * WR_LANES;
constexpr int WR_MAXK = 128;                  // keys per workgroup (score buffer)
constexpr int WR_DT = 64;                     // dims per staged slice

__device__ __forceinline__ void window_write_gates(const RouteArgs& a, const float (*out_s)[32],
                                                   const int (*out_i)[32], int rl, int lane, bool row_nat,
                                                   bool active, int64_t b, int64_t row);

// The end of route_window_kernel, with every window key's exact score in sc:
// each lane places its keys (index order in a short window, rank otherwise: a
// key's rank is the number of window keys that beat it), then lane 0 of each
// row writes indices, scores and gates.  Every thread of the workgroup calls it
// (one barrier inside).
__device__ __forceinline__ void window_select_write(const RouteArgs& a, const float (*sc)[WR_MAXK + 1],
                                                    float (*out_s)[32], int (*out_i)[32], int rl, int lane, int nk,
                                                    int64_t blk_lo, int64_t lo, int64_t hi, bool row_nat,
                                                    bool active, int64_t b, int64_t row) {
  const int k = a.k;
  // Place this lane's keys: index order in a short window, rank otherwise.
  if (active) {
    for (int kl = lane; kl < nk; kl += WR_LANES) {
      const int64_t key = blk_lo + kl;
      if (key < lo || key >= hi) continue;
      const float v = sc[rl][kl];
      int slot;
      if (row_nat) {
        slot = static_cast<int>(key - lo);
      } else {
        if (!(v > -INFINITY)) continue;  // NaN or -inf: never selected
        int rank = 0;
        const int wl = static_cast<int>(lo - blk_lo), wh = static_cast<int>(hi - blk_lo);
        for (int i = wl; i < wh && rank < k; ++i) {
          const float u = sc[rl][i];
          rank += (u > v || (u == v && i < kl)) ? 1 : 0;
        }
        if (rank >= k) continue;
        slot = rank;
      }
      out_s[rl][slot] = v;
      out_i[rl][slot] = static_cast<int>(key);
    }
  }
  __syncthreads();
  window_write_gates(a, out_s, out_i, rl, lane, row_nat, active, b, row);
}

// Lane 0 of each row: indices, scores and gates over the filled slots (a
// prefix), in slot order as route_kernel sums them.
__device__ __forceinline__ void window_write_gates(const RouteArgs& a, const float (*out_s)[32],
                                                   const int (*out_i)[32], int rl, int lane, bool row_nat,
                                                   bool active, int64_t b, int64_t row) {
  const int k = a.k;
  if (!active || lane != 0) return;
  const int64_t obase = (b * a.n_query + row) * k;
  int n = 0;
  for (int m = 0; m < k; ++m) n += out_i[rl][m] >= 0 ? 1 : 0;
  float mx = -INFINITY;
  if (row_nat) {
    for (int m = 0; m < n; ++m) mx = fmaxf(mx, out_s[rl][m] * a.inv_temp);
  } else if (n > 0) {
    mx = out_s[rl][0] * a.inv_temp;
  }
  float sum = 0.f;
  for (int m = 0; m < n; ++m) sum += expf(out_s[rl][m] * a.inv_temp - mx);
  for (int m = 0; m < k; ++m) {
    const bool f = m < n;
    a.idx[obase + m] = f ? out_i[rl][m] : -1;
    a.scores[obase + m] = f ? out_s[rl][m] : -INFINITY;
    a.gates[obase + m] = f ? expf(out_s[rl][m] * a.inv_temp - mx) / sum : 0.f;
  }
}

// KPT keys per lane per key chunk: 8 when every workgroup's range is at most
// 64 keys, else 16.
template <class E, int KPT>
__global__ __launch_bounds__(WR_THREADS) void route_window_kernel(const RouteArgs a) {
  using raw = typename ET<E>::raw;
  constexpr int WR_KPT = KPT;
  constexpr int WR_KC = WR_LANES * KPT;  // keys per chunk
  constexpr int V = 16 / sizeof(raw);         // elements per 16-byte read
  // Row stride WR_DT + 16 bytes: the 8 key rows a wave reads at one offset
  // start in 8 distinct 4-bank groups.
  constexpr int RS = WR_DT + V;
  __shared__ __align__(16) raw ktile[WR_KC * RS];
  __shared__ __align__(16) raw qtile[WR_ROWS * RS];
  __shared__ float sc[WR_ROWS][WR_MAXK + 1];
  __shared__ float out_s[WR_ROWS][32];
  __shared__ int out_i[WR_ROWS][32];

  const int tid = threadIdx.x;
  const int lane = tid % WR_LANES;
  const int rl = tid / WR_LANES;
  const int64_t b = blockIdx.y;
  const int64_t S = a.n_keys;
  const int D = a.dim;
  const int k = a.k;
  const int64_t r0 = static_cast<int64_t>(blockIdx.x) * WR_ROWS;
  const int64_t rlast = min(a.n_query, r0 + WR_ROWS) - 1;
  const int64_t row = r0 + rl;
  const bool active = row < a.n_query;
  auto win_hi = [&](int64_t r) { return min(S, a.base + r / a.seg_len); };
  auto win_lo = [&](int64_t h) { return h > a.cap ? h - a.cap : int64_t{0}; };
  const int64_t blk_hi = win_hi(rlast);
  const int64_t blk_lo = win_lo(win_hi(r0));
  const int nk = static_cast<int>(blk_hi - blk_lo);  // <= WR_MAXK, checked on the host
  const int64_t hi = win_hi(active ? row : r0);
  const int64_t lo = win_lo(hi);
  const bool row_nat = hi - lo <= k;

  const raw* qb = static_cast<const raw*>(a.q) + (b * a.n_query + r0) * D;
  const raw* kb = static_cast<const raw*>(a.keys) + (b * S + blk_lo) * D;

  for (int m = tid; m < WR_ROWS * 32; m += WR_THREADS) {
    out_s[m / 32][m % 32] = -INFINITY;
    out_i[m / 32][m % 32] = -1;
  }
  // 16-byte units of one staged slice (WR_KC key rows and WR_ROWS query rows of
  // WR_DT dims), and how many each thread moves.
  constexpr int UNITS = (WR_KC + WR_ROWS) * (WR_DT / V);
  constexpr int UPT = (UNITS + WR_THREADS - 1) / WR_THREADS;
  for (int kc0 = 0; kc0 < nk; kc0 += WR_KC) {
    float acc[WR_KPT];
#pragma unroll
    for (int j = 0; j < WR_KPT; ++j) acc[j] = 0.f;
    // The next slice's loads are issued before the current slice is computed.
    uint4 st[UPT];
    auto load_slice = [&](int d0) {
#pragma unroll
      for (int i = 0; i < UPT; ++i) {
        const int u = tid + WR_THREADS * i;
        const int r = u / (WR_DT / V);
        const int c = (u % (WR_DT / V)) * V;
        st[i] = make_uint4(0, 0, 0, 0);
        if (u < UNITS && d0 + c < D) {
          if (r < WR_KC) {
            if (kc0 + r < nk) st[i] = *reinterpret_cast<const uint4*>(kb + (kc0 + r) * static_cast<int64_t>(D) + d0 + c);
          } else if (r0 + (r - WR_KC) < a.n_query) {
            st[i] = *reinterpret_cast<const uint4*>(qb + (r - WR_KC) * static_cast<int64_t>(D) + d0 + c);
          }
        }
      }
    };
    load_slice(0);
    for (int d0 = 0; d0 < D; d0 += WR_DT) {
      __syncthreads();  // previous slice consumed
#pragma unroll
      for (int i = 0; i < UPT; ++i) {
        const int u = tid + WR_THREADS * i;
        const int r = u / (WR_DT / V);
        const int c = (u % (WR_DT / V)) * V;
        if (u < UNITS) *reinterpret_cast<uint4*>((r < WR_KC ? ktile + r * RS : qtile + (r - WR_KC) * RS) + c) = st[i];
      }
      __syncthreads();
      if (d0 + WR_DT < D) load_slice(d0 + WR_DT);
      const int dl = min(WR_DT, D - d0);
      for (int dd = 0; dd < dl; dd += V) {
        struct RV { raw e[V]; };
        const RV qv = __builtin_bit_cast(RV, *reinterpret_cast<const uint4*>(qtile + rl * RS + dd));
        float x[V];
#pragma unroll
        for (int e = 0; e < V; ++e) x[e] = ET<E>::to_f(qv.e[e]);
#pragma unroll
        for (int j = 0; j < WR_KPT; ++j) {
          const RV kv = __builtin_bit_cast(RV, *reinterpret_cast<const uint4*>(ktile + (lane + WR_LANES * j) * RS + dd));
#pragma unroll
          for (int e = 0; e < V; ++e) acc[j] = fmaf(x[e], ET<E>::to_f(kv.e[e]), acc[j]);
        }
      }
    }
#pragma unroll
    for (int j = 0; j < WR_KPT; ++j) {
      const int kl = kc0 + lane + WR_LANES * j;
      if (kl < nk) sc[rl][kl] = acc[j] * a.scale;
    }
  }
  __syncthreads();  // every score of the row in sc

  window_select_write(a, sc, out_s, out_i, rl, lane, nk, blk_lo, lo, hi, row_nat, active, b, row);
}

// Segment routing with short windows, 16-bit inputs: route_window_kernel's
// result, bit for bit, with an MFMA pass that narrows the exact chains to a few
// candidates per row (reference grm/core/paper_grm.py:566-589, 702-728).
//
//  1. 16x16x32 MFMAs give A, the approximate dot product of every (row, key)
//     of the workgroup.  A and the exact chain add the same exact 16-bit
//     products in fp32, so |A - chain| <= e = 4 max(dim, 64) 2^-23 |q| max|key|
//     (norms from the staged slices, scaled up by 1.001).
//  2. A window key is a candidate of its row when A_key >= L - W, L the k-th
//     largest A of the window and W twice 2e plus the ties the final
//     multiplication by `scale` can create and the flushed-denormal terms (as in
//     route_select.hip).  A key below that is beaten by k keys after the exact
//     chain and the scaling, so every key of the exact top k is a candidate.
//     For k <= KPT, L comes from a bitonic sort of each lane's KPT values and
//     three merges across the row's 8 lanes; otherwise each key counts the
//     window keys with A > A_key + W (the same test: fewer than k).  Rows whose
//     window holds at most k keys, or whose bound is not finite, take every
//     window key.
//  3. The workgroup's candidates, row after row, are dealt to all 256 lanes
//     (candidate c to thread c mod 256), so a wave runs a second round only for
//     the candidates past the first 256; each lane runs the exact chain (the
//     same fp32 FMA chain over d in increasing order, times scale) over the
//     restaged slices.
//  4. Slots by rank among the row's candidates (a key that is not a candidate
//     is beaten by k keys, so it beats no key of the top k and changes none of
//     their ranks), then the gates as in route_window_kernel.
constexpr int WS_ROUNDS = 2;  // candidate rounds per pass (256 candidates a round)

__device__ __forceinline__ float ws_max(float a, float b) { return __builtin_amdgcn_fmed3f(a, b, FLT_MAX); }
__device__ __forceinline__ float ws_min(float a, float b) { return __builtin_amdgcn_fmed3f(a, b, -FLT_MAX); }

// x sorted descending in place (bitonic network; NaN-free input, -inf may come
// out as -FLT_MAX).
template <int N>
__device__ __forceinline__ void ws_sort_desc(float (&x)[N]) {
#pragma unroll
  for (int size = 2; size <= N; size <<= 1)
#pragma unroll
    for (int stride = size / 2; stride > 0; stride >>= 1)
#pragma unroll
      for (int i = 0; i < N; ++i) {
        const int j = i ^ stride;
        if (j > i) {
          const float hi = ws_max(x[i], x[j]), lo = ws_min(x[i], x[j]);
          const bool desc = (i & size) == 0 || size == N;
          x[i] = desc ? hi : lo;
          x[j] = desc ? lo : hi;
        }
      }
}

// Descending x := the N largest of x and the partner lane's x (lane ^ off),
// descending: max(x_i, y_{N-1-i}) is bitonic and holds them; half-cleaners sort.
template <int N>
__device__ __forceinline__ void ws_merge_desc(float (&x)[N], int off) {
  float y[N];
#pragma unroll
  for (int i = 0; i < N; ++i) y[i] = __shfl_xor(x[i], off, 64);
#pragma unroll
  for (int i = 0; i < N; ++i) x[i] = ws_max(x[i], y[N - 1 - i]);
#pragma unroll
  for (int stride = N / 2; stride > 0; stride >>= 1)
#pragma unroll
    for (int i = 0; i < N; ++i) {
      const int j = i ^ stride;
      if (j > i) {
        const float hi = ws_max(x[i], x[j]), lo = ws_min(x[i], x[j]);
        x[i] = hi;
        x[j] = lo;
      }
    }
}

template <class E, int KPT>
__global__ __launch_bounds__(WR_THREADS) void route_wsel_kernel(const RouteArgs a) {
  using raw = typename ET<E>::raw;
  static_assert(sizeof(raw) == 2, "16-bit inputs");
  constexpr int V = 8;                    // elements per 16-byte granule
  constexpr int RS = WR_DT + V;           // staged row stride, elements
  constexpr int KC = WR_LANES * KPT;      // key rows staged (>= the workgroup's range)
  constexpr int NKT = KC / 16;            // 16-key MFMA tiles
  constexpr int TPW = NKT / 2;            // key tiles per wave (4 waves: 2 row tiles x 2)
  constexpr int UNITS = (KC + WR_ROWS) * (WR_DT / V);
  constexpr int UPT = (UNITS + WR_THREADS - 1) / WR_THREADS;
  // The key slices; after the last sweep, the rows' output slots.
  __shared__ __align__(16) raw ktile[KC * RS];
  static_assert(sizeof(ktile) >= WR_ROWS * 32 * (sizeof(float) + sizeof(int)), "slots fit the key tile");
  __shared__ __align__(16) raw qtile[WR_ROWS * RS];
  // Approximations by key, then exact scores by candidate; rows 16-byte
  // aligned, 4 banks apart.
  __shared__ __align__(16) float sc[WR_ROWS][WR_MAXK + 4];
  __shared__ uint8_t clist[WR_ROWS][WR_MAXK];
  __shared__ int rowoff[WR_ROWS + 1];  // first workgroup candidate of each row
  __shared__ float kred[WR_THREADS / 64];

  const int tid = threadIdx.x;
  const int lane = tid % WR_LANES;
  const int rl = tid / WR_LANES;
  const int lane64 = tid & 63;
  const int g = lane64 >> 4, n = lane64 & 15;
  const int w = tid >> 6;
  const int64_t b = blockIdx.y;
  const int64_t S = a.n_keys;
  const int D = a.dim;
  const int k = a.k;
  const int64_t r0 = static_cast<int64_t>(blockIdx.x) * WR_ROWS;
  const int64_t rlast = min(a.n_query, r0 + WR_ROWS) - 1;
  const int64_t row = r0 + rl;
  const bool active = row < a.n_query;
  auto win_hi = [&](int64_t r) { return min(S, a.base + r / a.seg_len); };
  auto win_lo = [&](int64_t h) { return h > a.cap ? h - a.cap : int64_t{0}; };
  const int64_t blk_hi = win_hi(rlast);
  const int64_t blk_lo = win_lo(win_hi(r0));
  const int nk = static_cast<int>(blk_hi - blk_lo);  // <= KC, checked on the host
  const int64_t hi = win_hi(active ? row : r0);
  const int64_t lo = win_lo(hi);
  const bool row_nat = hi - lo <= k;

  const raw* qb = static_cast<const raw*>(a.q) + (b * a.n_query + r0) * D;
  const raw* kb = static_cast<const raw*>(a.keys) + (b * S + blk_lo) * D;

  // One sweep over d: each slice of WR_DT dims (key rows past nk, query rows
  // past n_query and dims past D zero) staged, then body(d0, dims in slice).
  // The next slice's loads are issued before the current one is used.
  auto load_slice = [&](uint4 (&st)[UPT], int d0) {
#pragma unroll
    for (int i = 0; i < UPT; ++i) {
      const int u = tid + WR_THREADS * i;
      const int r = u / (WR_DT / V);
      const int c = (u % (WR_DT / V)) * V;
      st[i] = make_uint4(0, 0, 0, 0);
      if (u < UNITS && d0 + c < D) {
        if (r < KC) {
          if (r < nk) st[i] = *reinterpret_cast<const uint4*>(kb + r * static_cast<int64_t>(D) + d0 + c);
        } else if (r0 + (r - KC) < a.n_query) {
          st[i] = *reinterpret_cast<const uint4*>(qb + (r - KC) * static_cast<int64_t>(D) + d0 + c);
        }
      }
    }
  };
  auto sweep = [&](auto&& body) {
    uint4 st[UPT];
    load_slice(st, 0);
    for (int d0 = 0; d0 < D; d0 += WR_DT) {
      __syncthreads();  // previous slice consumed
#pragma unroll
      for (int i = 0; i < UPT; ++i) {
        const int u = tid + WR_THREADS * i;
        const int r = u / (WR_DT / V);
        const int c = (u % (WR_DT / V)) * V;
        if (u < UNITS) *reinterpret_cast<uint4*>((r < KC ? ktile + r * RS : qtile + (r - KC) * RS) + c) = st[i];
      }
      __syncthreads();
      if (d0 + WR_DT < D) load_slice(st, d0 + WR_DT);
      body(d0, min(WR_DT, D - d0));
    }
  };

  // ---- 1. approximations and norms.  Wave w: row tile w & 1, key tiles
  // (w >> 1) + 2 i; acc[i][r] is key 16 kt + 4 g + r of row 16 (w & 1) + n.
  const int rt = w & 1;
  f32x4 acc[TPW];
#pragma unroll
  for (int i = 0; i < TPW; ++i) acc[i] = f32x4{0.f, 0.f, 0.f, 0.f};
  float qn2 = 0.f;           // partial squared norm of row rl (granule `lane` of each slice)
  float kn2[KC / WR_ROWS];   // partial squared norms of keys rl + 32 j
#pragma unroll
  for (int j = 0; j < KC / WR_ROWS; ++j) kn2[j] = 0.f;
  sweep([&](int, int) {
#pragma unroll
    for (int c = 0; c < WR_DT / 32; ++c) {
      const Frag8<E> bq = __builtin_bit_cast(Frag8<E>, *reinterpret_cast<const uint4*>(qtile + (16 * rt + n) * RS + 32 * c + 8 * g));
#pragma unroll
      for (int i = 0; i < TPW; ++i) {
        const int kt = (w >> 1) + 2 * i;
        if (16 * kt < nk) {  // wave-uniform
          const Frag8<E> ak = __builtin_bit_cast(Frag8<E>, *reinterpret_cast<const uint4*>(ktile + (16 * kt + n) * RS + 32 * c + 8 * g));
          acc[i] = mfma8(ak, bq, acc[i]);
        }
      }
    }
    const U8<E> qv = __builtin_bit_cast(U8<E>, *reinterpret_cast<const uint4*>(qtile + rl * RS + V * lane));
#pragma unroll
    for (int e = 0; e < V; ++e) {
      const float x = ET<E>::to_f(qv.e[e]);
      qn2 = fmaf(x, x, qn2);
    }
#pragma unroll
    for (int j = 0; j < KC / WR_ROWS; ++j) {
      const U8<E> kv = __builtin_bit_cast(U8<E>, *reinterpret_cast<const uint4*>(ktile + (rl + WR_ROWS * j) * RS + V * lane));
#pragma unroll
      for (int e = 0; e < V; ++e) {
        const float x = ET<E>::to_f(kv.e[e]);
        kn2[j] = fmaf(x, x, kn2[j]);
      }
    }
  });
#pragma unroll
  for (int i = 0; i < TPW; ++i) {
    const int kt = (w >> 1) + 2 * i;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int key = 16 * kt + 4 * g + r;
      if (key < nk) sc[16 * rt + n][key] = acc[i][r];
    }
  }
  // Row norms over the row's 8 lanes; the largest key norm over the workgroup
  // (NaN when any is not finite: every row then takes the exact path).
#pragma unroll
  for (int off = 1; off < WR_LANES; off <<= 1) qn2 += __shfl_xor(qn2, off, 64);
  float kmx = 0.f;
#pragma unroll
  for (int j = 0; j < KC / WR_ROWS; ++j) {
    float t = kn2[j];
#pragma unroll
    for (int off = 1; off < WR_LANES; off <<= 1) t += __shfl_xor(t, off, 64);
    kmx = (t <= INFINITY && kmx <= INFINITY) ? fmaxf(kmx, t) : NAN;
  }
#pragma unroll
  for (int off = 8; off < 64; off <<= 1) {
    const float o = __shfl_xor(kmx, off, 64);
    kmx = (o <= INFINITY && kmx <= INFINITY) ? fmaxf(kmx, o) : NAN;
  }
  if (lane64 == 0) kred[w] = kmx;
  __syncthreads();  // sc holds every approximation, kred every wave's maximum
  float kmax2 = kred[0];
#pragma unroll
  for (int i = 1; i < WR_THREADS / 64; ++i)
    kmax2 = (kred[i] <= INFINITY && kmax2 <= INFINITY) ? fmaxf(kmax2, kred[i]) : NAN;

  // ---- 2. candidates.  Bit j of cmask: key lane + 8 j of the workgroup's range.
  const float qn = sqrtf(qn2) * 1.001f;
  const float km = sqrtf(kmax2) * 1.001f;
  const float e_mfma = 4.f * static_cast<float>(max(D, 64)) * 0x1p-23f * qn * km;
  const float mag = qn * km + 4.f * e_mfma;  // >= |A| and |chain| of every key
  const float wl = 2.f * (2.f * e_mfma + 0x1p-21f * (mag + 2.f * e_mfma) + 0x1p-148f / a.scale +
                          4.f * static_cast<float>(D) * 0x1p-126f * (qn + km));
  const bool sound = qn * km < 1e30f && wl <= 1e30f;  // false for NaN and inf
  const bool take_all = row_nat || !sound;
  const int wlo = static_cast<int>(lo - blk_lo), whi = static_cast<int>(hi - blk_lo);
  uint32_t cmask = 0u;
  {
    float x[KPT];
#pragma unroll
    for (int j = 0; j < KPT; ++j) {
      const int kl = lane + WR_LANES * j;
      x[j] = (kl >= wlo && kl < whi) ? sc[rl][kl] : -INFINITY;
    }
    if (k <= KPT) {
      // L: the row's KPT largest in every lane of the row (the merges run in
      // every lane; the inputs of rows that take every key do not matter).
      float y[KPT];
#pragma unroll
      for (int j = 0; j < KPT; ++j) y[j] = sound ? x[j] : -INFINITY;  // NaN-free
      ws_sort_desc(y);
#pragma unroll
      for (int off = 1; off < WR_LANES; off <<= 1) ws_merge_desc(y, off);
      float lk = y[0];
#pragma unroll
      for (int i = 1; i < KPT; ++i) lk = (i == k - 1) ? y[i] : lk;
      const float thr = lk - wl;
#pragma unroll
      for (int j = 0; j < KPT; ++j) {
        const int kl = lane + WR_LANES * j;
        const bool cand = active && kl >= wlo && kl < whi && (take_all || x[j] >= thr);
        cmask |= cand ? (1u << j) : 0u;
      }
    } else if (active) {
      // Each lane counts, for all its keys at once, the window keys whose A
      // exceeds theirs by more than W (16-byte reads of the row).
      float t[KPT];
      int cnt[KPT];
#pragma unroll
      for (int j = 0; j < KPT; ++j) {
        t[j] = x[j] > -INFINITY ? x[j] + wl : INFINITY;
        cnt[j] = 0;
      }
      if (!take_all) {
        for (int i = wlo & ~3; i < whi; i += 4) {
          const float4 u4 = *reinterpret_cast<const float4*>(&sc[rl][i]);
          const float uu[4] = {u4.x, u4.y, u4.z, u4.w};
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const float u = (i + e >= wlo && i + e < whi) ? uu[e] : -INFINITY;
#pragma unroll
            for (int j = 0; j < KPT; ++j) cnt[j] += u > t[j] ? 1 : 0;
          }
        }
      }
#pragma unroll
      for (int j = 0; j < KPT; ++j) {
        const int kl = lane + WR_LANES * j;
        const bool cand = kl >= wlo && kl < whi && (take_all || cnt[j] < k);
        cmask |= cand ? (1u << j) : 0u;
      }
    }
  }
  // The row's candidates in lane order: an exclusive prefix over its 8 lanes.
  const int mine = __builtin_popcount(cmask);
  int incl = mine;
#pragma unroll
  for (int off = 1; off < WR_LANES; off <<= 1) {
    const int o = __shfl_up(incl, off, WR_LANES);
    incl += lane >= off ? o : 0;
  }
  const int total = __shfl(incl, WR_LANES - 1, WR_LANES);
  {
    int pos = incl - mine;
#pragma unroll
    for (int j = 0; j < KPT; ++j)
      if (cmask & (1u << j)) clist[rl][pos++] = static_cast<uint8_t>(lane + WR_LANES * j);
  }
  if (lane == 0) rowoff[rl + 1] = total;
  __syncthreads();  // every approximation read; the lists and row totals written
  if (tid < 64) {
    // rowoff := exclusive prefix of the row totals (32 rows, one wave)
    int v = tid < WR_ROWS ? rowoff[tid + 1] : 0;
#pragma unroll
    for (int off = 1; off < WR_ROWS; off <<= 1) {
      const int o = __shfl_up(v, off, 64);
      v += tid >= off ? o : 0;
    }
    if (tid < WR_ROWS) rowoff[tid + 1] = v;
    if (tid == 0) rowoff[0] = 0;
  }
  __syncthreads();
  const int ctot = rowoff[WR_ROWS];

  // ---- 3. exact chains: workgroup candidate c (rows in order) on thread c mod
  // 256, pass c / (256 WS_ROUNDS).
  for (int pass0 = 0; pass0 < ctot; pass0 += WR_THREADS * WS_ROUNDS) {
    int crow[WS_ROUNDS], ckey[WS_ROUNDS], cpos[WS_ROUNDS];
    float ex[WS_ROUNDS];
#pragma unroll
    for (int r = 0; r < WS_ROUNDS; ++r) {
      const int c = pass0 + WR_THREADS * r + tid;
      int rr = 0;  // the row whose candidates hold c: rowoff[rr] <= c < rowoff[rr + 1]
#pragma unroll
      for (int step = WR_ROWS / 2; step > 0; step >>= 1) rr += (c >= rowoff[rr + step]) ? step : 0;
      crow[r] = rr;
      cpos[r] = c - rowoff[rr];
      ckey[r] = c < ctot ? clist[rr][cpos[r]] : 0;
      ex[r] = 0.f;
    }
    sweep([&](int, int dl) {
#pragma unroll
      for (int r = 0; r < WS_ROUNDS; ++r) {
        if (pass0 + WR_THREADS * r + 64 * w < ctot) {  // wave-uniform: a candidate in this wave
          const raw* qr = qtile + crow[r] * RS;
          const raw* kr = ktile + ckey[r] * RS;
          for (int dd = 0; dd < dl; dd += V) {
            const U8<E> qv = __builtin_bit_cast(U8<E>, *reinterpret_cast<const uint4*>(qr + dd));
            const U8<E> kv = __builtin_bit_cast(U8<E>, *reinterpret_cast<const uint4*>(kr + dd));
#pragma unroll
            for (int e = 0; e < V; ++e) ex[r] = fmaf(ET<E>::to_f(qv.e[e]), ET<E>::to_f(kv.e[e]), ex[r]);
          }
        }
      }
    });
#pragma unroll
    for (int r = 0; r < WS_ROUNDS; ++r)
      if (pass0 + WR_THREADS * r + tid < ctot) sc[crow[r]][cpos[r]] = ex[r] * a.scale;
  }
  __syncthreads();  // every candidate's exact score in sc, in candidate order; ktile free

  // ---- 4. slots in the key tile's memory.
  float (*out_s)[32] = reinterpret_cast<float (*)[32]>(ktile);
  int (*out_i)[32] = reinterpret_cast<int (*)[32]>(reinterpret_cast<unsigned char*>(ktile) + WR_ROWS * 32 * sizeof(float));
  for (int m = tid; m < WR_ROWS * 32; m += WR_THREADS) {
    out_s[m / 32][m % 32] = -INFINITY;
    out_i[m / 32][m % 32] = -1;
  }
  __syncthreads();
  if (active) {
    for (int c = lane; c < total; c += WR_LANES) {
      const int kl = clist[rl][c];
      const int64_t key = blk_lo + kl;
      const float v = sc[rl][c];
      int slot;
      if (row_nat) {
        slot = static_cast<int>(key - lo);
      } else {
        if (!(v > -INFINITY)) continue;  // NaN or -inf: never selected
        int rank = 0;
        for (int i = 0; i < total && rank < k; ++i) {
          const float u = sc[rl][i];
          const int ki = clist[rl][i];
          rank += (u > v || (u == v && ki < kl)) ? 1 : 0;
        }
        if (rank >= k) continue;
        slot = rank;
      }
      out_s[rl][slot] = v;
      out_i[rl][slot] = static_cast<int>(key);
    }
  }
  __syncthreads();
  window_write_gates(a, out_s, out_i, rl, lane, row_nat, active, b, row);
}

template <class E>
int launch_route_window(const RouteArgs& a, int64_t batch, int64_t span, hipStream_t s) {
  const dim3 grid(static_cast<unsigned>((a.n_query + WR_ROWS - 1) / WR_ROWS), static_cast<unsigned>(batch));
  if constexpr (!std::is_same_v<E, F32>) {
    // The MFMA-narrowed kernel needs a positive finite scale (the candidate
    // bound assumes scores keep the chains' order); GRM_HIP_ROUTE_WSEL=0 keeps
    // every window on the all-exact kernel.
    const char* env = getenv("GRM_HIP_ROUTE_WSEL");
    if ((env == nullptr || env[0] != '0') && a.scale > 0.f && a.scale <= FLT_MAX) {
      if (span <= WR_LANES * 8) {
        hipLaunchKernelGGL((route_wsel_kernel<E, 8>), grid, dim3(WR_THREADS), 0, s, a);
      } else {
        hipLaunchKernelGGL((route_wsel_kernel<E, 16>), grid, dim3(WR_THREADS), 0, s, a);
      }
      return check_launch("segment_route");
    }
  }
  if (span <= WR_LANES * 8) {
    hipLaunchKernelGGL((route_window_kernel<E, 8>), grid, dim3(WR_THREADS), 0, s, a);
  } else {
    hipLaunchKernelGGL((route_window_kernel<E, 16>), grid, dim3(WR_THREADS), 0, s, a);
  }
  return check_launch("segment_route");
}

// MFMA routing for bf16 inputs with k < n_keys.  Same result as route_kernel,
// bit for bit: the MFMA only narrows the search.
//
// 1. Each wave owns 64 query rows.  bf16 MFMAs give approximate scores A for
//    32 keys at a time; every lane keeps the KN = KMAX + 4 best approximate
//    scores of its row in a sorted register list of packed words
//    (order-preserving float bits, low `ib` bits replaced by the key index).
// 2. With S the exact score (the fp32 FMA chain of route_kernel), any key in
//    the exact top k has A' >= tau - W, where tau is the k-th best packed
//    score and W bounds |A' - S| twice over plus the ties the final
//    multiplication by `scale` can create:
//      |A - S| <= 4 * max(dim, 64) * 2^-23 * |q| * max_s |key_s|
//    (both are fp32 sums of the same exact bf16 products; each rounding or
//    truncation costs at most 2^-23 of the running sum of magnitudes, and a
//    flushed denormal product at most 2^-126 * (|q| + |key|) per term).
// 3. When the KN-th kept entry is below tau - W, the kept entries at or
//    above tau - W are a superset of the exact top k: only they get the exact
//    FMA chain, and the exact top k is chosen among them (ties to the lower
//    index).  Otherwise (near-ties over more than four places, or inputs
//    that are not finite) the lane scans every key exactly.
constexpr int RM_THREADS = 256;  // four independent waves
constexpr int RM_KT = 32;        // keys per tile
constexpr int RM_ROW = RM_KT + 4;
constexpr int RM_KC = 256;       // keys per LDS chunk of the exact pass

__device__ __forceinline__ uint32_t order_bits(float f) {
  const uint32_t u = __float_as_uint(f);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

__device__ __forceinline__ float unorder_bits(uint32_t u) {
  return __uint_as_float((u & 0x80000000u) ? (u ^ 0x80000000u) : ~u);
}

// Exact scores: each the fp32 FMA chain over d in increasing order, times
// scale.  NCH chains at once (independent accumulators, the query converted
// once per element); chain t reads the LDS key row rows[t].
template <int DKP, int NCH>
__device__ __forceinline__ void exact_scores_lds(const uint4 (&qv)[DKP / 8], const uint16_t* const (&rows)[NCH],
                                                 int dim, float scale, float (&out)[NCH]) {
  float acc[NCH];
#pragma unroll
  for (int t = 0; t < NCH; ++t) acc[t] = 0.f;
#pragma unroll
  for (int u = 0; u < DKP / 8; ++u) {
    if (8 * u < dim) {
      U8<BF16> kv[NCH];
#pragma unroll
      for (int t = 0; t < NCH; ++t) kv[t] = __builtin_bit_cast(U8<BF16>, *reinterpret_cast<const uint4*>(rows[t] + 8 * u));
      const U8<BF16> qq = __builtin_bit_cast(U8<BF16>, qv[u]);
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float x = ET<BF16>::to_f(qq.e[e]);
#pragma unroll
        for (int t = 0; t < NCH; ++t) acc[t] = fmaf(x, ET<BF16>::to_f(kv[t].e[e]), acc[t]);
      }
    }
  }
#pragma unroll
  for (int t = 0; t < NCH; ++t) out[t] = acc[t] * scale;
}

template <int KMAX>
__device__ __forceinline__ void exact_insert(float (&ts)[KMAX], int (&ti)[KMAX], float cs, int ci) {
#pragma unroll
  for (int m = 0; m < KMAX; ++m) {
    const bool better = cs > ts[m] || (cs == ts[m] && ci < ti[m]);
    const float s0 = better ? cs : ts[m];
    const int i0 = better ? ci : ti[m];
    cs = better ? ts[m] : cs;
    ci = better ? ti[m] : ci;
    ts[m] = s0;
    ti[m] = i0;
  }
}

template <int DKP, int KMAX>
__global__ __launch_bounds__(RM_THREADS, 2) void route_mfma_kernel(const RouteArgs a, const int ib) {
  constexpr int NC = DKP / 32;  // 32-element MFMA steps over d
  constexpr int KN = KMAX + 4;
  constexpr int KLS = DKP + 8;  // LDS key row stride (elements)
  constexpr int TILE_BYTES = 4 * 64 * RM_ROW * 4;
  constexpr int KEY_BYTES = RM_KC * KLS * 2;
  // Score tiles during the MFMA pass; afterwards 256-key chunks for the exact chains.
  __shared__ __align__(16) unsigned char smem[TILE_BYTES > KEY_BYTES ? TILE_BYTES : KEY_BYTES];
  __shared__ float red[4];

  const int tid = threadIdx.x;
  const int lane = tid & 63, g = lane >> 4, n = lane & 15;
  const int w = tid >> 6;
  const int64_t b = blockIdx.y;
  const int D = a.dim;
  const int S = static_cast<int>(a.n_keys);
  const int k = a.k;
  const uint16_t* kb = static_cast<const uint16_t*>(a.keys) + b * a.n_keys * D;
  const __amdgpu_buffer_rsrc_t rk = make_rsrc(kb, static_cast<uint32_t>(a.n_keys * D * 2));

  // Largest key norm of this batch entry (NaN if any key is not finite).
  float kn2 = 0.f;
  for (int s = tid; s < S; s += RM_THREADS) {
    float t = 0.f;
#pragma unroll
    for (int u = 0; u < DKP / 8; ++u) {
      if (8 * u < D) {
        const U8<BF16> kv = buf_load8<BF16>(rk, (s * D + 8 * u) * 2);
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const float x = ET<BF16>::to_f(kv.e[e]);
          t = fmaf(x, x, t);
        }
      }
    }
    kn2 = (t <= INFINITY) ? fmaxf(kn2, t) : NAN;  // false for NaN
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    const float o = __shfl_xor(kn2, off, 64);
    kn2 = (o <= INFINITY && kn2 <= INFINITY) ? fmaxf(kn2, o) : NAN;
  }
  if (lane == 0) red[w] = kn2;
  __syncthreads();
  float kmax2 = red[0];
#pragma unroll
  for (int i = 1; i < 4; ++i) kmax2 = (red[i] <= INFINITY && kmax2 <= INFINITY) ? fmaxf(kmax2, red[i]) : NAN;

  const int64_t qw = static_cast<int64_t>(blockIdx.x) * RM_THREADS + 64 * w;  // first row of this wave
  // Every wave stays to the end: the exact chains stage keys with the whole workgroup.
  const bool wave_live = qw < a.n_query;
  const int64_t qi = qw + lane;
  const bool active = qi < a.n_query;

  // Key windows (segment routing, seg_len > 0): row r sees [lo(r), hi(r)),
  // hi = base + r / seg_len, lo = max(0, hi - cap); both move forward with r.
  // Without windows every row sees [0, S).  A row whose window holds at most
  // k keys takes all of them in index order.
  auto win_hi = [&](int64_t r) -> int {
    return a.seg_len > 0 ? static_cast<int>(min(a.n_keys, a.base + min(r, a.n_query - 1) / a.seg_len)) : S;
  };
  auto win_lo = [&](int h) -> int {
    return a.seg_len > 0 ? static_cast<int>(h > a.cap ? h - a.cap : int64_t{0}) : 0;
  };
  const int row_hi = win_hi(qi), row_lo = win_lo(row_hi);
  const int row_n = row_hi - row_lo;
  const bool row_nat = a.seg_len > 0 && row_n <= k;
  // Keys the wave scores (rows qw .. qw + 63) and keys the workgroup stages.
  const int wave_lo = win_lo(win_hi(qw)) & ~(RM_KT - 1), wave_hi = win_hi(qw + 63);
  const int64_t qb0 = static_cast<int64_t>(blockIdx.x) * RM_THREADS;
  const int blk_lo = win_lo(win_hi(qb0)), blk_hi = win_hi(qb0 + RM_THREADS - 1);
  const uint16_t* qb = static_cast<const uint16_t*>(a.q) + b * a.n_query * D;
  const __amdgpu_buffer_rsrc_t rq = make_rsrc(qb, static_cast<uint32_t>(a.n_query * D * 2));

  // B operands: rows qw + 16 qt + n, d = 32 c + 8 g .. + 7.
  Frag8<BF16> bq[4][NC];
  float qp[4];
#pragma unroll
  for (int qt = 0; qt < 4; ++qt) {
    const int64_t row = qw + 16 * qt + n;
    qp[qt] = 0.f;
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      const int d = 32 * c + 8 * g;
      const U8<BF16> v = buf_load8<BF16>(rq, (row < a.n_query && d < D) ? static_cast<int>((row * D + d) * 2) : kBufOOB);
      bq[qt][c] = __builtin_bit_cast(Frag8<BF16>, v);
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float x = ET<BF16>::to_f(v.e[e]);
        qp[qt] = fmaf(x, x, qp[qt]);
      }
    }
    qp[qt] += __shfl_xor(qp[qt], 16, 64);
    qp[qt] += __shfl_xor(qp[qt], 32, 64);
  }
  // Lane 16 g + n owns row qw + 16 g + n, whose norm sits in qp[g].
  const float qn2 = g == 0 ? qp[0] : g == 1 ? qp[1] : g == 2 ? qp[2] : qp[3];
  // Windows of the rows this lane packs scores for: qw + 16 qt + n.
  int pk_lo[4], pk_hi[4];
#pragma unroll
  for (int qt = 0; qt < 4; ++qt) {
    pk_hi[qt] = win_hi(qw + 16 * qt + n);
    pk_lo[qt] = win_lo(pk_hi[qt]);
  }

  const uint32_t imask = (1u << ib) - 1u;
  uint32_t net[KN];
#pragma unroll
  for (int i = 0; i < KN; ++i) net[i] = 0u;
  uint32_t* srow = reinterpret_cast<uint32_t*>(smem) + w * 64 * RM_ROW;

  Frag8<BF16> ak[2][NC];
  auto load_keys = [&](int s0) {
#pragma unroll
    for (int kt = 0; kt < 2; ++kt) {
      const int row = s0 + 16 * kt + n;
#pragma unroll
      for (int c = 0; c < NC; ++c) {
        const int d = 32 * c + 8 * g;
        ak[kt][c] = __builtin_bit_cast(Frag8<BF16>, buf_load8<BF16>(rk, (row < S && d < D) ? (row * D + d) * 2 : kBufOOB));
      }
    }
  };
  load_keys(wave_lo);
  const int s_scan = wave_live ? wave_hi : 0;
  for (int s0 = wave_lo; s0 < s_scan; s0 += RM_KT) {
    f32x4 acc[4][2];
#pragma unroll
    for (int qt = 0; qt < 4; ++qt)
#pragma unroll
      for (int kt = 0; kt < 2; ++kt) {
        acc[qt][kt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int c = 0; c < NC; ++c) acc[qt][kt] = mfma8(ak[kt][c], bq[qt][c], acc[qt][kt]);
      }
    if (s0 + RM_KT < s_scan) load_keys(s0 + RM_KT);
    // acc[qt][kt][r] = A(key s0 + 16 kt + 4 g + r, row 16 qt + n)
#pragma unroll
    for (int qt = 0; qt < 4; ++qt)
#pragma unroll
      for (int kt = 0; kt < 2; ++kt) {
        uint4 pk;
        uint32_t* pe = reinterpret_cast<uint32_t*>(&pk);
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int key = s0 + 16 * kt + 4 * g + r;
          pe[r] = (key >= pk_lo[qt] && key < pk_hi[qt])
                      ? ((order_bits(acc[qt][kt][r]) & ~imask) | static_cast<uint32_t>(key)) : 0u;
        }
        *reinterpret_cast<uint4*>(srow + (16 * qt + n) * RM_ROW + 16 * kt + 4 * g) = pk;
      }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    const uint32_t thr = net[KN - 1];
    uint32_t m = 0u;
#pragma unroll
    for (int j4 = 0; j4 < RM_KT / 4; ++j4) {
      const uint4 v = *reinterpret_cast<const uint4*>(srow + lane * RM_ROW + 4 * j4);
      m |= (v.x > thr ? 1u : 0u) << (4 * j4);
      m |= (v.y > thr ? 1u : 0u) << (4 * j4 + 1);
      m |= (v.z > thr ? 1u : 0u) << (4 * j4 + 2);
      m |= (v.w > thr ? 1u : 0u) << (4 * j4 + 3);
    }
    if (!active) m = 0u;
    while (m != 0u) {
      const int j = __builtin_ctz(m);
      m &= m - 1u;
      uint32_t p = srow[lane * RM_ROW + j];
#pragma unroll
      for (int i = 0; i < KN; ++i) {
        const uint32_t hi = max(net[i], p);
        p = min(net[i], p);
        net[i] = hi;
      }
    }
    // The next tile's writes must not pass this tile's reads.
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  }
  // This row, packed, for the exact chains.
  uint4 qv[DKP / 8];
#pragma unroll
  for (int u = 0; u < DKP / 8; ++u)
    qv[u] = __builtin_bit_cast(uint4, buf_load8<BF16>(rq, (active && 8 * u < D) ? static_cast<int>((qi * D + 8 * u) * 2)
                                                                               : kBufOOB));

  float top_s[KMAX];
  int top_i[KMAX];
#pragma unroll
  for (int m = 0; m < KMAX; ++m) {
    top_s[m] = -INFINITY;
    top_i[m] = INT32_MAX;
  }
  uint32_t tau_u = net[0];
#pragma unroll
  for (int i = 1; i < KN; ++i) tau_u = (i == k - 1) ? net[i] : tau_u;
  const float tau = unorder_bits(tau_u & ~imask);
  const float a0 = unorder_bits(net[0] & ~imask);
  const float qn = sqrtf(qn2) * 1.001f, km = sqrtf(kmax2) * 1.001f;
  const float e_mfma = 4.f * static_cast<float>(max(D, 64)) * 0x1p-23f * qn * km;
  const float eta = __uint_as_float(static_cast<uint32_t>(127 + ib - 22) << 23);  // 2^(ib-22): packing
  const float r_abs = fmaxf(fabsf(tau), fabsf(a0)) + 4.f * e_mfma;
  const float w0 = 2.f * e_mfma + 4.f * eta * (r_abs + 2.f * e_mfma);
  const float wide = w0 + 0x1p-21f * (fabsf(tau) + 2.f * w0) + 0x1p-148f / a.scale +
                     4.f * static_cast<float>(D) * 0x1p-126f * (qn + km);
  const float theta = tau - wide;
  const bool sound = qn * km < 1e30f && wide <= 1e30f;  // false for NaN and inf
  const bool complete = row_n <= KN || unorder_bits(net[KN - 1] & ~imask) < theta;
  // A short window (row_nat) is scored key by key in index order, like scan_all.
  const bool scan_all = active && (row_nat || !(sound && complete));

  // Candidate keys in ascending order (0xffffffff past the last), so that the
  // candidates inside one key chunk are a contiguous run.
  uint32_t ck[KN];
#pragma unroll
  for (int i = 0; i < KN; ++i) ck[i] = 0xffffffffu;
#pragma unroll
  for (int i = 0; i < KN; ++i) {
    const bool take = active && !scan_all && i < row_n && unorder_bits(net[i] & ~imask) >= theta;
    uint32_t x = take ? (net[i] & imask) : 0xffffffffu;
#pragma unroll
    for (int m = 0; m < KN; ++m) {
      const uint32_t lo = min(ck[m], x);
      x = max(ck[m], x);
      ck[m] = lo;
    }
  }

  // Key chunks through LDS; each lane walks its candidates in the chunk (or,
  // for a row that needs it, every key of the chunk) with one copy of the chain.
  const uint16_t* kl = reinterpret_cast<const uint16_t*>(smem);
  for (int c0 = blk_lo; c0 < blk_hi; c0 += RM_KC) {
    const int c1 = min(blk_hi, c0 + RM_KC);
    __syncthreads();  // score tiles / the previous chunk are no longer read
    constexpr int UPR = DKP / 8;  // 16-byte units per padded row
    for (int e = tid; e < RM_KC * UPR; e += RM_THREADS) {
      const int r = e / UPR, u = e % UPR;
      const int key = c0 + r;
      const uint4 v = __builtin_bit_cast(
          uint4, buf_load8<BF16>(rk, (key < c1 && 8 * u < D) ? (key * D + 8 * u) * 2 : kBufOOB));
      *reinterpret_cast<uint4*>(reinterpret_cast<uint16_t*>(smem) + r * KLS + 8 * u) = v;
    }
    __syncthreads();
    int lo = 0, hi = 0;
#pragma unroll
    for (int i = 0; i < KN; ++i) {
      lo += ck[i] < static_cast<uint32_t>(c0) ? 1 : 0;
      hi += ck[i] < static_cast<uint32_t>(c1) ? 1 : 0;
    }
    // scan_all rows walk their window's keys of this chunk, [w0, w1)
    const int w0 = max(c0, row_lo), w1 = min(c1, row_hi);
    const int count = scan_all ? max(w1 - w0, 0) : hi - lo;
    constexpr int NCH = 2;  // chains per step
#pragma unroll 1
    for (int j = 0; j < count; j += NCH) {
      int key[NCH];
      const uint16_t* rows[NCH];
#pragma unroll
      for (int t = 0; t < NCH; ++t) {
        key[t] = w0 + j + t;
        if (!scan_all) {
          uint32_t word = 0u;
#pragma unroll
          for (int i = 0; i < KN; ++i) word = (i == lo + j + t) ? ck[i] : word;
          key[t] = static_cast<int>(word);
        }
        rows[t] = kl + (j + t < count ? key[t] - c0 : 0) * KLS;
      }
      float sc4[NCH];
      exact_scores_lds<DKP, NCH>(qv, rows, D, a.scale, sc4);
#pragma unroll
      for (int t = 0; t < NCH; ++t) {
        if (j + t >= count) continue;
        if (row_nat) {  // index order: slot key - row_lo
#pragma unroll
          for (int m = 0; m < KMAX; ++m) {
            if (m == key[t] - row_lo) {
              top_s[m] = sc4[t];
              top_i[m] = key[t];
            }
          }
        } else {
          exact_insert<KMAX>(top_s, top_i, sc4[t], key[t]);
        }
      }
    }
  }
  if (!active) return;

  const int64_t obase = (b * a.n_query + qi) * k;
  if (row_nat) {
    // n <= k window keys in index order; slots n .. k-1 empty (-1, -inf, 0).
    float mxn = -INFINITY;
#pragma unroll
    for (int m = 0; m < KMAX; ++m) mxn = (m < row_n) ? fmaxf(mxn, top_s[m] * a.inv_temp) : mxn;
    float en[KMAX];
    float sumn = 0.f;
#pragma unroll
    for (int m = 0; m < KMAX; ++m) {
      en[m] = (m < row_n) ? expf(top_s[m] * a.inv_temp - mxn) : 0.f;
      sumn += en[m];
    }
#pragma unroll
    for (int m = 0; m < KMAX; ++m) {
      if (m < k) {
        a.idx[obase + m] = (m < row_n) ? top_i[m] : -1;
        a.scores[obase + m] = (m < row_n) ? top_s[m] : -INFINITY;
        a.gates[obase + m] = (m < row_n) ? en[m] / sumn : 0.f;
      }
    }
    return;
  }
  write_topk_row<KMAX>(a.idx, a.scores, a.gates, obase, k, a.inv_temp, top_s, top_i);
}

// Whether route_mfma_kernel covers these arguments; ib = index bits.
bool mfma_route_ok(const RouteArgs& a, int dtype, const void* queries, const void* keys, int* ib) {
  if (dtype != GRM_HIP_BF16 || a.natural || !(a.scale > 0.f) || a.dim > 128 || a.dim % 8 != 0 ||
      a.n_keys > 2048 || a.k > 32 || (reinterpret_cast<uintptr_t>(queries) | reinterpret_cast<uintptr_t>(keys)) % 16 != 0 ||
      a.n_query * a.dim * 2 > INT32_MAX || a.n_keys * a.dim * 2 > INT32_MAX)
    return false;
  int bits = 1;
  while ((int64_t{1} << bits) < a.n_keys) ++bits;
  *ib = bits;
  return true;
}

template <int DKP>
int launch_route_mfma_dk(const RouteArgs& a, int64_t batch, int ib, hipStream_t s) {
  const dim3 grid(static_cast<unsigned>((a.n_query + RM_THREADS - 1) / RM_THREADS), static_cast<unsigned>(batch));
  if (a.k <= 8) {
    hipLaunchKernelGGL((route_mfma_kernel<DKP, 8>), grid, dim3(RM_THREADS), 0, s, a, ib);
  } else if (a.k <= 16) {
    hipLaunchKernelGGL((route_mfma_kernel<DKP, 16>), grid, dim3(RM_THREADS), 0, s, a, ib);
  } else {
    hipLaunchKernelGGL((route_mfma_kernel<DKP, 32>), grid, dim3(RM_THREADS), 0, s, a, ib);
  }
  return check_launch("topk_route");
}

int launch_route_mfma(const RouteArgs& a, int64_t batch, int ib, hipStream_t s) {
  if (a.dim <= 32) return launch_route_mfma_dk<32>(a, batch, ib, s);
  if (a.dim <= 64) return launch_route_mfma_dk<64>(a, batch, ib, s);
  return launch_route_mfma_dk<128>(a, batch, ib, s);
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

// Vector form of fuse_kernel for 16-byte aligned rows (hidden a multiple of 8 /
// 4 elements): `lpr` lanes (a power of two) share one row, each holding NV
// 16-byte groups of it, so every access is a 16-byte load or store and all
// routes' loads of a lane are in flight together.  Same arithmetic order per
// element as fuse_kernel (the route sum, then the residual add).
// One 16-byte group (8 16-bit or 4 fp32 elements) as floats; OOB -> zeros.
template <class E>
__device__ __forceinline__ void load_group(__amdgpu_buffer_rsrc_t r, int off, float (&f)[16 / sizeof(typename ET<E>::raw)]) {
  typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
  const u32x4 q = __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0);
  if constexpr (sizeof(typename ET<E>::raw) == 2) {
    const U8<E> u = __builtin_bit_cast(U8<E>, q);
#pragma unroll
    for (int e = 0; e < 8; ++e) f[e] = ET<E>::to_f(u.e[e]);
  } else {
#pragma unroll
    for (int e = 0; e < 4; ++e) f[e] = __uint_as_float(q[e]);
  }
}

template <class E, int NV>
__global__ __launch_bounds__(256) void fuse_vec_kernel(const FuseArgs a, const int lpr) {
  using raw = typename ET<E>::raw;
  constexpr int VE = 16 / sizeof(raw);
  typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
  const int tid = threadIdx.x;
  const int sub = tid & (lpr - 1);
  const WaveRows wr = wave_rows(static_cast<int64_t>(blockIdx.x) * (256 / lpr), lpr, a.rows);
  const bool live = wr.row < a.rows;
  const int H = a.hidden;
  const int64_t rr = live ? wr.row : 0;
  const int hb = H * static_cast<int>(sizeof(raw)), retb = a.routes * hb;  // row bytes of h / out and of ret
  const __amdgpu_buffer_rsrc_t rh = wave_rows_rsrc(a.h, wr, hb);
  const __amdgpu_buffer_rsrc_t rret = wave_rows_rsrc(a.ret, wr, retb);
  const float* g = a.gates + rr * a.routes;
  float x[NV][VE];
#pragma unroll
  for (int v = 0; v < NV; ++v) {
    const int c = (sub + lpr * v) * VE;
    const int off = (live && c < H) ? wr.local * hb + c * static_cast<int>(sizeof(raw)) : kBufOOB;
    float hv[VE];
    load_group<E>(rh, off, hv);
    float r[VE];
#pragma unroll
    for (int e = 0; e < VE; ++e) r[e] = 0.f;
#pragma unroll 8
    for (int j = 0; j < a.routes; ++j) {
      const float gj = g[j];
      const int o2 = (live && c < H) ? wr.local * retb + (j * H + c) * static_cast<int>(sizeof(raw)) : kBufOOB;
      float rv[VE];
      load_group<E>(rret, o2, rv);
#pragma unroll
      for (int e = 0; e < VE; ++e) r[e] = fmaf(gj, rv[e], r[e]);
    }
#pragma unroll
    for (int e = 0; e < VE; ++e) x[v][e] = (c < H) ? hv[e] + r[e] : 0.f;
  }
  const __amdgpu_buffer_rsrc_t ro = wave_rows_rsrc(a.out, wr, hb);
  auto store = [&](int v, const float (&y)[VE]) {
    const int c = (sub + lpr * v) * VE;
    const int off = (live && c < H) ? wr.local * hb + c * static_cast<int>(sizeof(raw)) : kBufOOB;
    if constexpr (VE == 8) {
      uint4 pk;
      pk.x = ET<E>::from_f(y[0]) | (static_cast<uint32_t>(ET<E>::from_f(y[1])) << 16);
      pk.y = ET<E>::from_f(y[2]) | (static_cast<uint32_t>(ET<E>::from_f(y[3])) << 16);
      pk.z = ET<E>::from_f(y[4]) | (static_cast<uint32_t>(ET<E>::from_f(y[5])) << 16);
      pk.w = ET<E>::from_f(y[6]) | (static_cast<uint32_t>(ET<E>::from_f(y[7])) << 16);
      __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, pk), ro, off, 0, 0);
    } else {
      __builtin_amdgcn_raw_buffer_store_b128(
          u32x4{__float_as_uint(y[0]), __float_as_uint(y[1]), __float_as_uint(y[2]), __float_as_uint(y[3])}, ro, off, 0, 0);
    }
  };
  if (a.w == nullptr) {
#pragma unroll
    for (int v = 0; v < NV; ++v) store(v, x[v]);
    return;
  }
  float sum = 0.f;
#pragma unroll
  for (int v = 0; v < NV; ++v)
#pragma unroll
    for (int e = 0; e < VE; ++e) sum += x[v][e];
  for (int off = lpr >> 1; off > 0; off >>= 1) sum += __shfl_xor(sum, off, 64);
  const float mean = sum / static_cast<float>(H);
  float var = 0.f;
#pragma unroll
  for (int v = 0; v < NV; ++v) {
    const int c = (sub + lpr * v) * VE;
#pragma unroll
    for (int e = 0; e < VE; ++e) {
      const float d = x[v][e] - mean;
      var = (c < H) ? fmaf(d, d, var) : var;
    }
  }
  for (int off = lpr >> 1; off > 0; off >>= 1) var += __shfl_xor(var, off, 64);
  const float rstd = 1.0f / sqrtf(var / static_cast<float>(H) + a.eps);
  const __amdgpu_buffer_rsrc_t rw = make_rsrc(a.w, H * sizeof(raw));
  const __amdgpu_buffer_rsrc_t rb = make_rsrc(a.bias, a.bias != nullptr ? H * sizeof(raw) : 0u);
#pragma unroll
  for (int v = 0; v < NV; ++v) {
    const int c = (sub + lpr * v) * VE;
    const int off = c < H ? c * static_cast<int>(sizeof(raw)) : kBufOOB;
    float wv[VE], bv[VE];
    load_group<E>(rw, off, wv);
    load_group<E>(rb, off, bv);  // zeros without a bias
    float y[VE];
#pragma unroll
    for (int e = 0; e < VE; ++e) y[e] = (x[v][e] - mean) * rstd * wv[e] + bv[e];
    store(v, y);
  }
}

bool aligned(const void* p, size_t n) { return (reinterpret_cast<uintptr_t>(p) % n) == 0; }

RouteSelArgs select_args(const RouteArgs& a) {
  RouteSelArgs r;
  memset(&r, 0, sizeof(r));
  r.q = a.q;
  r.keys = a.keys;
  r.idx = a.idx;
  r.scores = a.scores;
  r.gates = a.gates;
  r.n_query = a.n_query;
  r.n_keys = a.n_keys;
  r.dim = a.dim;
  r.k = a.k;
  r.scale = a.scale;
  r.inv_temp = a.inv_temp;
  r.seg_len = a.seg_len;
  r.base = a.base;
  r.cap = a.cap;
  return r;
}

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
  if (!natural && k > kRouteMaxK) {
    set_error("topk_route: top_k %lld > %d", (long long)k, kRouteMaxK);
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
  if (!natural) {
    int rc = GRM_HIP_OK;
    if (try_route_select(select_args(a), dtype, batch, s, &rc)) return rc;
  }
  int ib = 0;
  if (mfma_route_ok(a, dtype, queries, keys, &ib)) return launch_route_mfma(a, batch, ib, s);
  switch (dtype) {
    case GRM_HIP_F32: return launch_route<F32>(a, batch, s);
    case GRM_HIP_F16: return launch_route<F16>(a, batch, s);
    default: return launch_route<BF16>(a, batch, s);
  }
}

extern "C" int grm_hip_segment_route(const void* queries, const void* keys, int64_t* topk_indices,
                                     float* topk_scores, float* gates, int64_t batch, int64_t n_query,
                                     int64_t n_keys, int64_t dim, int dtype, int64_t top_k,
                                     int64_t segment_len, int64_t base, int64_t capacity, float scale,
                                     float temperature, void* stream) {
  if (batch < 0 || n_query < 0 || n_keys < 0 || dim < 0 || top_k < 1 || top_k > kRouteMaxK || segment_len < 1 ||
      base < 0 || capacity < 1) {
    set_error("segment_route: bad sizes (1 <= top_k <= %d, segment_len >= 1, base >= 0, capacity >= 1)",
              kRouteMaxK);
    return GRM_HIP_EINVAL;
  }
  if (dtype < GRM_HIP_F32 || dtype > GRM_HIP_BF16) {
    set_error("segment_route: unsupported dtype %d", dtype);
    return GRM_HIP_EUNSUPPORTED;
  }
  if (!(temperature > 0.f) || !std::isfinite(scale)) {
    set_error("segment_route: temperature must be > 0 and scale finite");
    return GRM_HIP_EINVAL;
  }
  if (batch == 0 || n_query == 0) return GRM_HIP_OK;
  if (base + (n_query - 1) / segment_len > n_keys) {
    set_error("segment_route: the last segment's window ends past n_keys");
    return GRM_HIP_EINVAL;
  }
  if (batch > 65535 || dim > INT32_MAX || n_keys > INT32_MAX || segment_len > INT32_MAX) {
    set_error("segment_route: batch > 65535 or dims too large");
    return GRM_HIP_EUNSUPPORTED;
  }
  if (queries == nullptr || (keys == nullptr && n_keys > 0) || topk_indices == nullptr ||
      topk_scores == nullptr || gates == nullptr) {
    set_error("segment_route: null pointer");
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
  a.k = static_cast<int>(top_k);
  a.natural = 0;
  const int eb = dtype == GRM_HIP_F32 ? 4 : 2;
  a.vec = (dim * eb) % 16 == 0 && aligned(queries, 16);
  a.scale = scale;
  a.inv_temp = 1.0f / temperature;
  a.seg_len = static_cast<int>(segment_len);
  a.base = base;
  a.cap = capacity;
  hipStream_t s = static_cast<hipStream_t>(stream);
  // Keys of one workgroup of WR_ROWS rows (r0 a multiple of WR_ROWS): hi runs
  // from h0 = base + r0 / segment_len to h1 = base + r1 / segment_len, so the
  // range is h1 - max(0, h0 - capacity) <= (h1 - h0) + min(n_keys, capacity).
  // Without a segment boundary inside a workgroup (segment_len a multiple of
  // WR_ROWS) h1 == h0; otherwise h1 - h0 <= (WR_ROWS - 1) / segment_len + 1.
  const int64_t crossings = segment_len % WR_ROWS == 0 ? 0 : (WR_ROWS - 1) / segment_len + 1;
  const int64_t span = std::min(n_keys, capacity) + crossings;
  {
    int rc = GRM_HIP_OK;
    if (try_route_select(select_args(a), dtype, batch, s, &rc)) return rc;
  }
  int ib = 0;
  if (mfma_route_ok(a, dtype, queries, keys, &ib)) return launch_route_mfma(a, batch, ib, s);
  const bool window_ok = span <= WR_MAXK && a.vec && aligned(keys, 16) && top_k <= 32;
  if (window_ok) {
    switch (dtype) {
      case GRM_HIP_F32: return launch_route_window<F32>(a, batch, span, s);
      case GRM_HIP_F16: return launch_route_window<F16>(a, batch, span, s);
      default: return launch_route_window<BF16>(a, batch, span, s);
    }
  }
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
  const int eb = dtype == GRM_HIP_F32 ? 4 : 2;
  const int ve = 16 / eb;
  const bool vec = hidden_size % ve == 0 && aligned(h_online, 16) && aligned(out, 16) &&
                   (routes == 0 || aligned(retrieved, 16)) && (ln_weight == nullptr || aligned(ln_weight, 16)) &&
                   (ln_bias == nullptr || aligned(ln_bias, 16)) && routes * hidden_size * eb <= INT32_MAX;
  if (vec) {
    // lanes per row: the power of two covering the row's 16-byte groups, at most 64
    const int64_t groups = hidden_size / ve;
    int lpr = 1;
    while (lpr < 64 && lpr < groups) lpr <<= 1;
    const int64_t nv = (groups + lpr - 1) / lpr;
    const dim3 vgrid(static_cast<unsigned>((rows + 256 / lpr - 1) / (256 / lpr)));
    auto go = [&](auto tag, auto nvc) {
      using E = decltype(tag);
      hipLaunchKernelGGL((fuse_vec_kernel<E, decltype(nvc)::value>), vgrid, dim3(256), 0, s, a, lpr);
    };
    auto by_nv = [&](auto tag) {
      if (nv <= 1) go(tag, std::integral_constant<int, 1>{});
      else if (nv <= 2) go(tag, std::integral_constant<int, 2>{});
      else if (nv <= 4) go(tag, std::integral_constant<int, 4>{});
      else go(tag, std::integral_constant<int, 8>{});
    };
    switch (dtype) {
      case GRM_HIP_F32: by_nv(F32{}); break;
      case GRM_HIP_F16: by_nv(F16{}); break;
      default: by_nv(BF16{}); break;
    }
    return check_launch("fuse_residual");
  }
  const dim3 grid(static_cast<unsigned>((rows + 3) / 4));
  switch (dtype) {
    case GRM_HIP_F32: hipLaunchKernelGGL(fuse_kernel<F32>, grid, dim3(256), 0, s, a); break;
    case GRM_HIP_F16: hipLaunchKernelGGL(fuse_kernel<F16>, grid, dim3(256), 0, s, a); break;
    default: hipLaunchKernelGGL(fuse_kernel<BF16>, grid, dim3(256), 0, s, a); break;
  }
  return check_launch("fuse_residual");
}
