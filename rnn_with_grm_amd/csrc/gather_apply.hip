// Batched gather of archived segment states and query application, gfx950.
//
// Both are HBM-bound streams with no reuse worth tiling for:
//   gather:      out[b, i, :] = memories[b, idx[b, i], :]
//                (reference grm/csrc/batched_gather.cu:14-77, grm_cuda.cpp:156-179)
//   apply fwd:   hidden[row] = sum_k M[row, k] * q[row / (R*H), k]
//                (reference grm/csrc/apply_query.cu:14-75, grm_cuda.cpp:128-134)
//   apply bwd:   dM[row, k] = dh[row] * q[row / (R*H), k]
//                dq[bq, k]  = sum_{rh} dh[bq*R*H + rh] * M[bq*R*H + rh, k]
//                (reference grm/csrc/apply_query.cu:77-169, grm_cuda.cpp:136-154)
// The gather has two kernels, both with 16-byte accesses:
//   - column-tiled, when every archived state is referenced about once or more
//     (n_index >= segments): one workgroup per (sequence, row chunk, column
//     slice) keeps that slice of all the sequence's states in LDS and writes it
//     into its output rows, so the archive crosses HBM once and the kernel runs
//     at the HBM write rate;
//   - row-wise otherwise: one row per workgroup pass, rows split into eight
//     contiguous ranges, one per XCD, so one XCD's L2 sees the archive of only
//     a few sequences at a time; non-temporal stores for large outputs (the
//     materialised output is never re-read here).
#include <stdint.h>
#include <string.h>

#include <algorithm>

#include "grm_hip.h"
#include "grm_hip_common.h"

namespace grmhip {
namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int GT = 256;  // threads per workgroup

struct GatherArgs {
  const void* mem;
  const int64_t* idx;
  void* out;
  int64_t batch;
  int64_t segments;
  int64_t n_index;     // indices per batch entry
  int64_t total_rows;  // batch * n_index
  int64_t row_units;   // units per row
  int tpr;             // threads per row (power of two, <= GT)
  int xcd_split;       // grid is a multiple of 8: XCD x copies rows [x R/8, (x+1) R/8)
  int32_t* bad;
};

template <typename U, bool NT>
__device__ __forceinline__ void put(U* p, U v) {
  if constexpr (NT) {
    __builtin_nontemporal_store(v, p);
  } else {
    *p = v;
  }
}

template <typename U, bool NT>
__global__ __launch_bounds__(GT) void gather_kernel(const GatherArgs a) {
  const int tpr = a.tpr;
  const int rows_per_wg = GT / tpr;
  const int sub = threadIdx.x / tpr;
  const int lane = threadIdx.x % tpr;
  int64_t lo = 0, hi = a.total_rows;
  int64_t wg = blockIdx.x, nwg = gridDim.x;
  if (a.xcd_split) {
    const int64_t x = blockIdx.x & 7;
    wg = blockIdx.x >> 3;
    nwg = gridDim.x >> 3;
    lo = a.total_rows * x / 8;
    hi = a.total_rows * (x + 1) / 8;
  }
  const U* mem = static_cast<const U*>(a.mem);
  U* out = static_cast<U*>(a.out);
  const int64_t ru = a.row_units;
  for (int64_t row = lo + wg * rows_per_wg + sub; row < hi; row += nwg * rows_per_wg) {
    const int64_t b = row / a.n_index;
    const int64_t s = a.idx[row];
    const bool ok = s >= 0 && s < a.segments;
    if (!ok && lane == 0 && a.bad != nullptr) atomicAdd(a.bad, 1);
    const U* src = mem + (b * a.segments + (ok ? s : 0)) * ru;
    U* dst = out + row * ru;
    int64_t u = lane;
    if (ok) {
      for (; u + 3 * tpr < ru; u += 4 * tpr) {
        const U v0 = src[u], v1 = src[u + tpr], v2 = src[u + 2 * tpr], v3 = src[u + 3 * tpr];
        put<U, NT>(dst + u, v0);
        put<U, NT>(dst + u + tpr, v1);
        put<U, NT>(dst + u + 2 * tpr, v2);
        put<U, NT>(dst + u + 3 * tpr, v3);
      }
      for (; u < ru; u += tpr) put<U, NT>(dst + u, src[u]);
    } else {
      U z;
      memset(&z, 0, sizeof(z));
      for (; u < ru; u += tpr) put<U, NT>(dst + u, z);
    }
  }
}

// Column-tiled gather for the many-queries case (n_index >= segments): workgroup
// (b, row chunk, t) stages units [t*W, (t+1)*W) of every archived state of
// sequence b in LDS (S*W*16 bytes; the archive crosses HBM once, the second row
// chunk re-reads it from L2), then writes that W-unit slice of its output rows.
// Workgroups of one (b, row chunk) are adjacent in launch order, so the rows
// being written at any time form a narrow band of memory.  Plain stores: on
// this path they sustain a higher HBM write rate than non-temporal ones.
constexpr int GC_THREADS = 1024;
constexpr int GC_UNROLL = 4;
constexpr int GC_ROW_CHUNKS = 2;
constexpr int64_t GC_MAX_LDS = 128 * 1024;

template <int W>
__global__ __launch_bounds__(GC_THREADS) void gather_cols_kernel(const GatherArgs a, int64_t tiles, int64_t chunks) {
  extern __shared__ u32x4 cols[];
  const int64_t t = blockIdx.x % tiles;
  const int64_t rest = blockIdx.x / tiles;
  const int64_t ch = rest % chunks;
  const int64_t b = rest / chunks;
  const int64_t S = a.segments, ru = a.row_units;
  const u32x4* src = static_cast<const u32x4*>(a.mem) + b * S * ru + t * W;
  for (int64_t e = threadIdx.x; e < S * W; e += GC_THREADS) {
    const int64_t s = e / W;
    cols[e] = src[s * ru + (e - s * W)];
  }
  __syncthreads();
  constexpr int RPP = GC_THREADS / W;  // output rows per pass
  const int w = threadIdx.x % W;
  const int64_t rows = (a.n_index + chunks - 1) / chunks;
  const int64_t r0 = ch * rows;
  const int64_t r1 = min(a.n_index, r0 + rows);
  const int64_t* ib = a.idx + b * a.n_index;
  u32x4* ob = static_cast<u32x4*>(a.out) + b * a.n_index * ru + t * W + w;
  const bool count = a.bad != nullptr && t == 0 && w == 0;
  const u32x4 zero = {0u, 0u, 0u, 0u};
  int64_t i = r0 + threadIdx.x / W;
  for (; i + (GC_UNROLL - 1) * RPP < r1; i += GC_UNROLL * RPP) {
    int64_t s[GC_UNROLL];
#pragma unroll
    for (int r = 0; r < GC_UNROLL; ++r) s[r] = ib[i + r * RPP];
#pragma unroll
    for (int r = 0; r < GC_UNROLL; ++r) {
      const bool ok = s[r] >= 0 && s[r] < S;
      if (!ok && count) atomicAdd(a.bad, 1);
      ob[(i + r * RPP) * ru] = ok ? cols[s[r] * W + w] : zero;
    }
  }
  for (; i < r1; i += RPP) {
    const int64_t s = ib[i];
    const bool ok = s >= 0 && s < S;
    if (!ok && count) atomicAdd(a.bad, 1);
    ob[i * ru] = ok ? cols[s * W + w] : zero;
  }
}

template <int W>
int launch_gather_cols(GatherArgs a, hipStream_t s) {
  static bool attr_set = false;
  if (!attr_set) {
    hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(&gather_cols_kernel<W>),
                                       hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(GC_MAX_LDS));
    if (e != hipSuccess) {
      set_error("batched_gather: hipFuncSetAttribute failed: %s", hipGetErrorString(e));
      return static_cast<int>(e);
    }
    attr_set = true;
  }
  const int64_t tiles = a.row_units / W;
  const int64_t chunks = a.n_index >= GC_ROW_CHUNKS * GC_THREADS ? GC_ROW_CHUNKS : 1;
  const size_t lds = static_cast<size_t>(a.segments * W * 16);
  hipLaunchKernelGGL((gather_cols_kernel<W>), dim3(static_cast<unsigned>(a.batch * chunks * tiles)),
                     dim3(GC_THREADS), lds, s, a, tiles, chunks);
  return check_launch("batched_gather");
}

// Widest column tile whose LDS slice fits, or 0 when the row kernel is the better
// (or only) choice: few references per state, a row not divisible into tiles, or
// too few workgroups to fill the chip.
int cols_width(const GatherArgs& a) {
  if (a.segments < 1 || a.n_index < a.segments) return 0;
  for (int w : {32, 16, 8}) {
    if (a.row_units % w != 0 || a.segments * w * 16 > GC_MAX_LDS) continue;
    const int64_t grid = a.batch * (a.row_units / w);
    if (grid < 1024 || grid * GC_ROW_CHUNKS > INT32_MAX) continue;
    return w;
  }
  return 0;
}

int launch_cols_any(GatherArgs a, int w, hipStream_t s) {
  if (w == 32) return launch_gather_cols<32>(a, s);
  if (w == 16) return launch_gather_cols<16>(a, s);
  return launch_gather_cols<8>(a, s);
}

template <typename U, bool NT>
int launch_gather(GatherArgs a, hipStream_t s) {
  int tpr = 1;
  while (tpr < GT && tpr < a.row_units) tpr <<= 1;
  a.tpr = tpr;
  const int64_t rows_per_wg = GT / tpr;
  int64_t want = (a.total_rows + rows_per_wg - 1) / rows_per_wg;
  // Enough workgroups to fill 256 CUs many times over; the loop covers the rest.
  const int64_t cap = 256 * 32;
  int64_t grid = want < cap ? want : cap;
  a.xcd_split = 0;
  if (grid >= 64) {
    grid -= grid % 8;
    a.xcd_split = 1;
  }
  if (grid < 1) grid = 1;
  hipLaunchKernelGGL((gather_kernel<U, NT>), dim3(static_cast<unsigned>(grid)), dim3(GT), 0, s, a);
  return check_launch("batched_gather");
}

bool aligned(const void* p, size_t n) { return (reinterpret_cast<uintptr_t>(p) % n) == 0; }

// ---------------------------------------------------------------------------
// apply_query forward: a group of G lanes per row, VEC elements per lane per step.
struct ApplyArgs {
  const void* mem;
  const void* q;
  void* out;
  const void* dh;    // backward only
  void* dmem;        // backward only
  void* dq;          // backward only
  int64_t rows;      // batch * n_query * routes * hidden
  int64_t rh;        // routes * hidden (rows per query vector)
  int64_t nq;        // batch * n_query
  int kdim;
  int group;         // lanes per row (power of two <= 64)
  int vec;           // 16-byte vector path legal
};

template <class E>
__device__ __forceinline__ void load_vec(const typename ET<E>::raw* p, int k, int K, bool vec,
                                         float (&x)[8], int& cnt) {
  // Loads up to 16 bytes starting at element k.
  constexpr int V = (sizeof(typename ET<E>::raw) == 2) ? 8 : 4;
  cnt = V;
  if (vec && k + V <= K) {
    if constexpr (V == 8) {
      const U8<E> u = *reinterpret_cast<const U8<E>*>(p + k);
#pragma unroll
      for (int i = 0; i < 8; ++i) x[i] = ET<E>::to_f(u.e[i]);
    } else {
      const float4 f = *reinterpret_cast<const float4*>(p + k);
      x[0] = f.x; x[1] = f.y; x[2] = f.z; x[3] = f.w;
    }
  } else {
#pragma unroll
    for (int i = 0; i < V; ++i) x[i] = (k + i < K) ? ET<E>::to_f(p[k + i]) : 0.f;
  }
}

template <class E>
__global__ __launch_bounds__(GT) void apply_fwd_kernel(const ApplyArgs a) {
  using raw = typename ET<E>::raw;
  constexpr int V = (sizeof(raw) == 2) ? 8 : 4;
  constexpr int RPI = 4;  // rows per group per iteration (independent loads in flight)
  const int G = a.group;
  const int lane = threadIdx.x % G;
  const int grp = threadIdx.x / G;
  const int groups_per_wg = GT / G;
  const int K = a.kdim;
  const raw* mem = static_cast<const raw*>(a.mem);
  const raw* q = static_cast<const raw*>(a.q);
  raw* out = static_cast<raw*>(a.out);
  const int64_t step = static_cast<int64_t>(gridDim.x) * groups_per_wg * RPI;
  for (int64_t base = (static_cast<int64_t>(blockIdx.x) * groups_per_wg + grp) * RPI; base < a.rows;
       base += step) {
    float acc[RPI];
#pragma unroll
    for (int r = 0; r < RPI; ++r) acc[r] = 0.f;
    for (int k0 = 0; k0 < K; k0 += G * V) {
      const int k = k0 + lane * V;
#pragma unroll
      for (int r = 0; r < RPI; ++r) {
        const int64_t row = base + r;
        if (row < a.rows && k < K) {
          float m[8], x[8];
          int cnt;
          load_vec<E>(mem + row * K, k, K, a.vec, m, cnt);
          load_vec<E>(q + (row / a.rh) * K, k, K, a.vec, x, cnt);
#pragma unroll
          for (int i = 0; i < V; ++i) acc[r] = fmaf(m[i], x[i], acc[r]);
        }
      }
    }
#pragma unroll
    for (int r = 0; r < RPI; ++r) {
      float v = acc[r];
      for (int off = G >> 1; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
      const int64_t row = base + r;
      if (lane == 0 && row < a.rows) out[row] = ET<E>::from_f(v);
    }
  }
}

// dM[row, k] = dh[row] * q[row / rh, k]
template <class E>
__global__ __launch_bounds__(GT) void apply_bwd_dmem_kernel(const ApplyArgs a) {
  using raw = typename ET<E>::raw;
  constexpr int V = (sizeof(raw) == 2) ? 8 : 4;
  const int G = a.group;
  const int lane = threadIdx.x % G;
  const int grp = threadIdx.x / G;
  const int groups_per_wg = GT / G;
  const int K = a.kdim;
  const raw* q = static_cast<const raw*>(a.q);
  const raw* dh = static_cast<const raw*>(a.dh);
  raw* dmem = static_cast<raw*>(a.dmem);
  const int64_t step = static_cast<int64_t>(gridDim.x) * groups_per_wg;
  for (int64_t row = static_cast<int64_t>(blockIdx.x) * groups_per_wg + grp; row < a.rows;
       row += step) {
    const float d = ET<E>::to_f(dh[row]);
    const raw* qr = q + (row / a.rh) * K;
    raw* dst = dmem + row * K;
    for (int k = lane * V; k < K; k += G * V) {
      float x[8];
      int cnt;
      load_vec<E>(qr, k, K, a.vec, x, cnt);
      if (a.vec && k + V <= K) {
        U8<E> u;
        if constexpr (V == 8) {
#pragma unroll
          for (int i = 0; i < 8; ++i) u.e[i] = ET<E>::from_f(d * x[i]);
          *reinterpret_cast<U8<E>*>(dst + k) = u;
        } else {
          *reinterpret_cast<float4*>(dst + k) = make_float4(d * x[0], d * x[1], d * x[2], d * x[3]);
        }
      } else {
#pragma unroll
        for (int i = 0; i < V; ++i)
          if (k + i < K) dst[k + i] = ET<E>::from_f(d * x[i]);
      }
    }
  }
}

// dq[bq, k] = sum_rh dh[bq*rh + i] * M[bq*rh + i, k]; one workgroup per bq,
// threads = KT k-lanes x P row-partitions, fixed-order partial sums.
template <class E>
__global__ __launch_bounds__(GT) void apply_bwd_dq_kernel(const ApplyArgs a) {
  using raw = typename ET<E>::raw;
  __shared__ float part[GT];
  const int K = a.kdim;
  int KT = 1;
  while (KT < K && KT < GT) KT <<= 1;
  const int P = GT / KT;
  const int kl = threadIdx.x % KT;
  const int pi = threadIdx.x / KT;
  const raw* mem = static_cast<const raw*>(a.mem);
  const raw* dh = static_cast<const raw*>(a.dh);
  raw* dq = static_cast<raw*>(a.dq);
  for (int64_t bq = blockIdx.x; bq < a.nq; bq += gridDim.x) {
    for (int k0 = 0; k0 < K; k0 += KT) {
      const int k = k0 + kl;
      float acc = 0.f;
      if (k < K) {
        for (int64_t i = pi; i < a.rh; i += P) {
          const int64_t row = bq * a.rh + i;
          acc = fmaf(ET<E>::to_f(dh[row]), ET<E>::to_f(mem[row * K + k]), acc);
        }
      }
      part[threadIdx.x] = acc;
      __syncthreads();
      if (pi == 0 && k < K) {
        float s = 0.f;
        for (int p = 0; p < P; ++p) s += part[p * KT + kl];
        dq[bq * K + k] = ET<E>::from_f(s);
      }
      __syncthreads();
    }
  }
}

int lanes_per_row(int64_t K, int elem_bytes) {
  const int V = elem_bytes == 2 ? 8 : 4;
  const int64_t need = (K + V - 1) / V;
  int g = 1;
  while (g < 64 && g < need) g <<= 1;
  return g;
}

// Zero fill of n 16-bit units, grid-stride: the degenerate shapes of the
// apply entry points clear their output with a kernel rather than hipMemsetAsync,
// so that no entry point records a memset node into a captured graph.
__global__ __launch_bounds__(256) void zero16_kernel(uint16_t* __restrict__ p, int64_t n) {
  const int64_t stride = static_cast<int64_t>(gridDim.x) * 256;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; i < n; i += stride) p[i] = 0;
}

int launch_zero16(void* p, int64_t n, hipStream_t s, const char* what) {
  if (n <= 0) return GRM_HIP_OK;
  const int64_t blocks = std::min<int64_t>((n + 255) / 256, 4096);
  hipLaunchKernelGGL(zero16_kernel, dim3(static_cast<unsigned>(blocks)), dim3(256), 0, s, static_cast<uint16_t*>(p),
                     n);
  return check_launch(what);
}

template <class E>
int launch_apply_fwd(ApplyArgs a, hipStream_t s) {
  const int64_t groups_per_wg = GT / a.group;
  const int64_t want = (a.rows + groups_per_wg * 4 - 1) / (groups_per_wg * 4);
  const int64_t grid = want < 256 * 64 ? want : 256 * 64;
  hipLaunchKernelGGL(apply_fwd_kernel<E>, dim3(static_cast<unsigned>(grid < 1 ? 1 : grid)), dim3(GT),
                     0, s, a);
  return check_launch("apply_query_fwd");
}

template <class E>
int launch_apply_bwd(ApplyArgs a, hipStream_t s) {
  if (a.dmem != nullptr) {  // NULL: the caller needs grad_queries only
    const int64_t groups_per_wg = GT / a.group;
    const int64_t want = (a.rows + groups_per_wg - 1) / groups_per_wg;
    const int64_t g = want < 256 * 64 ? want : 256 * 64;
    hipLaunchKernelGGL(apply_bwd_dmem_kernel<E>, dim3(static_cast<unsigned>(g < 1 ? 1 : g)), dim3(GT), 0, s, a);
    const int rc = check_launch("apply_query_bwd(grad_memories)");
    if (rc != GRM_HIP_OK) return rc;
  }
  const int64_t grid = a.nq < 256 * 64 ? a.nq : 256 * 64;
  hipLaunchKernelGGL(apply_bwd_dq_kernel<E>, dim3(static_cast<unsigned>(grid < 1 ? 1 : grid)),
                     dim3(GT), 0, s, a);
  return check_launch("apply_query_bwd(grad_queries)");
}

int check_apply_sizes(const char* what, int64_t batch, int64_t n_query, int64_t routes,
                      int64_t hidden_size, int64_t key_dim, int dtype) {
  if (batch < 0 || n_query < 0 || routes < 0 || hidden_size < 0 || key_dim < 0) {
    set_error("%s: negative size", what);
    return GRM_HIP_EINVAL;
  }
  if (key_dim > INT32_MAX) {
    set_error("%s: key_dim too large", what);
    return GRM_HIP_EINVAL;
  }
  if (dtype < GRM_HIP_F32 || dtype > GRM_HIP_BF16) {
    set_error("%s: unsupported dtype %d", what, dtype);
    return GRM_HIP_EUNSUPPORTED;
  }
  return GRM_HIP_OK;
}

}  // namespace
}  // namespace grmhip

using namespace grmhip;

extern "C" int grm_hip_batched_gather(const void* memories, const int64_t* indices, void* out,
                                      int64_t batch, int64_t segments, int64_t n_index,
                                      int64_t row_elems, int elem_bytes, int32_t* bad_index_count,
                                      void* stream) {
  if (batch < 0 || segments < 0 || n_index < 0 || row_elems < 0) {
    set_error("batched_gather: negative size");
    return GRM_HIP_EINVAL;
  }
  if (elem_bytes != 1 && elem_bytes != 2 && elem_bytes != 4 && elem_bytes != 8) {
    set_error("batched_gather: unsupported element size %d", elem_bytes);
    return GRM_HIP_EUNSUPPORTED;
  }
  const int64_t total_rows = batch * n_index;
  if (total_rows == 0 || row_elems == 0) return GRM_HIP_OK;
  if (memories == nullptr && segments > 0) {
    set_error("batched_gather: null memories");
    return GRM_HIP_EINVAL;
  }
  if (indices == nullptr || out == nullptr) {
    set_error("batched_gather: null pointer");
    return GRM_HIP_EINVAL;
  }
  hipStream_t s = static_cast<hipStream_t>(stream);
  GatherArgs a;
  memset(&a, 0, sizeof(a));
  a.mem = memories;
  a.idx = indices;
  a.out = out;
  a.batch = batch;
  a.segments = segments;
  a.n_index = n_index;
  a.total_rows = total_rows;
  a.bad = bad_index_count;
  const int64_t row_bytes = row_elems * elem_bytes;
  if (row_bytes % 16 == 0 && aligned(memories, 16) && aligned(out, 16)) {
    a.row_units = row_bytes / 16;
    // Non-temporal stores only pay for outputs far larger than L2.
    const bool nt = total_rows * row_bytes >= (int64_t(64) << 20);
    const int w = cols_width(a);
    if (w > 0) return launch_cols_any(a, w, s);
    if (nt) return launch_gather<u32x4, true>(a, s);
    return launch_gather<u32x4, false>(a, s);
  }
  a.row_units = row_elems;
  switch (elem_bytes) {
    case 1: return launch_gather<uint8_t, false>(a, s);
    case 2: return launch_gather<uint16_t, false>(a, s);
    case 4: return launch_gather<uint32_t, false>(a, s);
    default: return launch_gather<uint64_t, false>(a, s);
  }
}

extern "C" int grm_hip_apply_query_fwd(const void* memories, const void* queries, void* hidden,
                                       int64_t batch, int64_t n_query, int64_t routes,
                                       int64_t hidden_size, int64_t key_dim, int dtype,
                                       void* stream) {
  int rc = check_apply_sizes("apply_query_fwd", batch, n_query, routes, hidden_size, key_dim, dtype);
  if (rc != GRM_HIP_OK) return rc;
  const int64_t rows = batch * n_query * routes * hidden_size;
  if (rows == 0) return GRM_HIP_OK;
  if (memories == nullptr || queries == nullptr || hidden == nullptr) {
    set_error("apply_query_fwd: null pointer");
    return GRM_HIP_EINVAL;
  }
  const int eb = dtype == GRM_HIP_F32 ? 4 : 2;
  ApplyArgs a;
  memset(&a, 0, sizeof(a));
  a.mem = memories;
  a.q = queries;
  a.out = hidden;
  a.rows = rows;
  a.rh = routes * hidden_size;
  a.nq = batch * n_query;
  a.kdim = static_cast<int>(key_dim);
  a.group = lanes_per_row(key_dim, eb);
  a.vec = (key_dim * eb) % 16 == 0 && aligned(memories, 16) && aligned(queries, 16);
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (key_dim == 0) return launch_zero16(hidden, rows * eb / 2, s, "apply_query_fwd");
  switch (dtype) {
    case GRM_HIP_F32: return launch_apply_fwd<F32>(a, s);
    case GRM_HIP_F16: return launch_apply_fwd<F16>(a, s);
    default: return launch_apply_fwd<BF16>(a, s);
  }
}

extern "C" int grm_hip_apply_query_bwd(const void* grad_hidden, const void* memories,
                                       const void* queries, void* grad_memories,
                                       void* grad_queries, int64_t batch, int64_t n_query,
                                       int64_t routes, int64_t hidden_size, int64_t key_dim,
                                       int dtype, void* stream) {
  int rc = check_apply_sizes("apply_query_bwd", batch, n_query, routes, hidden_size, key_dim, dtype);
  if (rc != GRM_HIP_OK) return rc;
  const int64_t rows = batch * n_query * routes * hidden_size;
  const int64_t nq = batch * n_query;
  const int eb = dtype == GRM_HIP_F32 ? 4 : 2;
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (nq == 0 || key_dim == 0) return GRM_HIP_OK;
  if (queries == nullptr || grad_queries == nullptr || (rows > 0 && (grad_hidden == nullptr ||
                                                                     memories == nullptr))) {
    set_error("apply_query_bwd: null pointer");
    return GRM_HIP_EINVAL;
  }
  if (rows == 0) return launch_zero16(grad_queries, nq * key_dim * eb / 2, s, "apply_query_bwd");
  ApplyArgs a;
  memset(&a, 0, sizeof(a));
  a.mem = memories;
  a.q = queries;
  a.dh = grad_hidden;
  a.dmem = grad_memories;
  a.dq = grad_queries;
  a.rows = rows;
  a.rh = routes * hidden_size;
  a.nq = nq;
  a.kdim = static_cast<int>(key_dim);
  a.group = lanes_per_row(key_dim, eb);
  a.vec = (key_dim * eb) % 16 == 0 && aligned(grad_memories, 16) && aligned(queries, 16);
  switch (dtype) {
    case GRM_HIP_F32: return launch_apply_bwd<F32>(a, s);
    case GRM_HIP_F16: return launch_apply_bwd<F16>(a, s);
    default: return launch_apply_bwd<BF16>(a, s);
  }
}
