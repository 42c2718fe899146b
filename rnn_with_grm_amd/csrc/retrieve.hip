// Gather + query application over archived segment states, without
// materialising the gathered states, gfx950.
//
//   out[b, q, r, h] = sum_k memories[b, idx[b, q, r], h, k] * q'[b, q, k]
//
// which is the reference's apply_query_forward(batched_memory_gather(M, idx), q)
// (grm/core/cuda_ops.py:370-402; apply_query.cu:14-75 and batched_gather.cu:14-77
// for the two kernels it chains, paper_grm.py:229,301-313 for the composition),
// with q' = q cast to the memories' dtype as the caller does (paper_grm.py:301).
//
// The reference materialises [B, Q, R, d_v, d_k] (64 GiB at BASELINE config 3)
// and reads it back.  Here the (q, r) pairs of each sequence are first sorted by
// segment (one workgroup per sequence: LDS histogram, exclusive scan, scatter);
// then one workgroup per (sequence, segment, 128-row value tile) reads that
// archived state once into LDS and applies it to every query that selected it
// with fp32 MFMA (16x16x4), 64 pairs at a time.  Each pair's output row is
// written whole by exactly one workgroup, so the result does not depend on the
// order in which the sort placed pairs.
#include <stdint.h>
#include <string.h>

#include <type_traits>

#include "grm_hip.h"
#include "grm_hip_common.h"
#include "retrieve.h"

namespace grmhip {
namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int BK_THREADS = 1024;     // bucket kernels
constexpr int BK_ITEMS = 16384;      // pairs per workgroup when one sequence's pairs are split
constexpr int64_t kMultiBucketPairs = 4 * BK_ITEMS;  // from this many pairs per sequence
constexpr int64_t kMaxSegments = 16384;
constexpr int AP_THREADS = 256;      // apply kernel: 4 waves
constexpr int AP_V = kScaledTile;    // value rows per workgroup
constexpr int AP_N = 64;             // (q, r) pairs per tile

struct RetrieveArgs {
  const void* mem;
  const int64_t* idx;
  const void* queries;
  void* out;
  int32_t* offsets;  // [batch, segments + 1]
  int32_t* list;     // [batch, n_index]
  int32_t* bad;
  int64_t batch;
  int64_t segments;
  int64_t n_query;
  int64_t routes;
  int64_t n_index;  // n_query * routes
  int dv;
  int dk;
  int v_tiles;
  int32_t* partial;  // [batch, bk_chunks, segments]: per-chunk counts, then bases (multi-workgroup bucketing)
  int bk_chunks;     // pair groups of about BK_ITEMS per sequence (strided blocks of BK_THREADS pairs)
  // Work tiles of the apply kernels: at most tile_pairs consecutive pairs of
  // one segment each, so a segment that many queries selected is spread over
  // several workgroups.  tiles [batch, tb_max] of (segment, first pair, end, 0);
  // n_tiles [batch]; tile_base [batch, segments + 1] is the scan's scratch.
  int4* tiles;
  int32_t* n_tiles;
  int32_t* tile_base;
  int tb_max;
  int tile_pairs;
  // Gate-weighted, row-scaled 16-bit output (retrieve_fuse): out holds float16
  // rows of g * M q scaled by 2^sh per (pair, 128-value tile), scales[pair,
  // tile] = 2^-sh.  nullptr: the plain [pairs, dv] output of gather_apply.
  const float* gates;  // [batch, n_index]
  float* scales;       // [batch, n_index, v_tiles]
  int out_row;         // elements per output row (dv; dk for the queries' gradient)
};

// ---------------------------------------------------------------------------
// Exclusive scan of hist[0..S) in LDS, in place, by one workgroup of
// BK_THREADS; offsets[s] gets the same values and offsets[S] the total.
__device__ void bucket_offsets(int* hist, int64_t S, int32_t* offsets) {
  __shared__ int wave_sum[BK_THREADS / 64];
  const int tid = threadIdx.x;
  // thread t owns bins [t per, (t + 1) per)
  const int per = static_cast<int>((S + BK_THREADS - 1) / BK_THREADS);
  const int lo = min(static_cast<int64_t>(tid) * per, S);
  const int hi = min(static_cast<int64_t>(lo) + per, S);
  int local = 0;
  for (int s = lo; s < hi; ++s) local += hist[s];
  const int lane = tid & 63, wave = tid >> 6;
  int incl = local;
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    const int y = __shfl_up(incl, d, 64);
    if (lane >= d) incl += y;
  }
  if (lane == 63) wave_sum[wave] = incl;
  __syncthreads();
  int base = 0;
  for (int w = 0; w < wave; ++w) base += wave_sum[w];
  if (tid == 0) {
    int t = 0;
    for (int w = 0; w < BK_THREADS / 64; ++w) t += wave_sum[w];
    offsets[S] = t;
  }
  int run = base + incl - local;
  for (int s = lo; s < hi; ++s) {
    const int c = hist[s];
    offsets[s] = run;
    hist[s] = run;
    run += c;
  }
  __syncthreads();
}

// Lane index of the r-th set bit of mask (r < popcount(mask)).
__device__ __forceinline__ int nth_set_bit(uint64_t mask, int r) {
  int pos = 0;
#pragma unroll
  for (int w = 32; w >= 1; w >>= 1) {
    const int c = __popcll(mask & ((1ull << w) - 1u));
    if (r >= c) {
      r -= c;
      mask >>= w;
      pos += w;
    }
  }
  return pos;
}

// A row whose index is outside [0, segments): zeros, and one count.  Called
// by every lane of a wave together (bad: this lane's pair i is invalid).  With
// 16-byte rows the wave writes several whole rows per store instruction,
// coalesced (the first segments' short windows can leave most of a pair chunk
// empty); otherwise one row after another, consecutive lanes on consecutive
// elements.
template <class EM>
__device__ __forceinline__ void zero_rows_wave(const RetrieveArgs& a, int64_t b, int64_t i, bool bad) {
  using raw = typename ET<EM>::raw;
  uint64_t mask = __ballot(bad);
  const int lane = threadIdx.x & 63;
  if (mask != 0u && lane == 0 && a.bad != nullptr) atomicAdd(a.bad, static_cast<int>(__popcll(mask)));
  if (mask == 0u) return;
  const int64_t row_bytes = static_cast<int64_t>(a.out_row) * sizeof(raw);
  if (row_bytes % 16 == 0 && reinterpret_cast<uintptr_t>(a.out) % 16 == 0) {
    // Whole rows in 16-byte pieces: lpr lanes per row, 64 / lpr rows per store
    // instruction, the rows taken in ballot order (i < n_index <= INT32_MAX).
    const int pieces = static_cast<int>(row_bytes / 16);
    int lpr = 1;
    while (lpr < pieces && lpr < 64) lpr <<= 1;
    const int m = __popcll(mask);
    const int i32 = static_cast<int>(i);
    for (int r0 = 0; r0 < m; r0 += 64 / lpr) {
      const int r = r0 + lane / lpr;
      const int row = __shfl(i32, nth_set_bit(mask, r < m ? r : 0), 64);
      if (r < m) {
        uint4* ob = reinterpret_cast<uint4*>(static_cast<raw*>(a.out) + (b * a.n_index + row) * a.out_row);
        for (int p = lane % lpr; p < pieces; p += lpr) ob[p] = uint4{0u, 0u, 0u, 0u};
        if (a.scales != nullptr)
          for (int t = lane % lpr; t < a.v_tiles; t += lpr) a.scales[(b * a.n_index + row) * a.v_tiles + t] = 0.f;
      }
    }
    return;
  }
  while (mask != 0u) {
    const int l = __ffsll(static_cast<unsigned long long>(mask)) - 1;
    mask &= mask - 1u;
    const int64_t row = __shfl(i, l, 64);
    typename ET<EM>::raw* ob = static_cast<typename ET<EM>::raw*>(a.out) + (b * a.n_index + row) * a.out_row;
    for (int h = lane; h < a.out_row; h += 64) ob[h] = ET<EM>::from_f(0.f);
    if (a.scales != nullptr)
      for (int t = lane; t < a.v_tiles; t += 64) a.scales[(b * a.n_index + row) * a.v_tiles + t] = 0.f;
  }
}

// Pairs of one sequence sorted by segment, one workgroup per sequence.  Rows
// with an invalid index are zeroed here and never enter a bucket.
template <class EM>
__global__ __launch_bounds__(BK_THREADS) void bucket_kernel(const RetrieveArgs a) {
  extern __shared__ int hist[];  // [segments]
  const int tid = threadIdx.x;
  const int64_t b = blockIdx.x;
  const int64_t S = a.segments, n = a.n_index;
  const int64_t* ib = a.idx + b * n;
  for (int64_t s = tid; s < S; s += BK_THREADS) hist[s] = 0;
  __syncthreads();
  for (int64_t i = tid; i < n; i += BK_THREADS) {
    const int64_t s = ib[i];
    if (s >= 0 && s < S) atomicAdd(&hist[s], 1);
  }
  __syncthreads();
  bucket_offsets(hist, S, a.offsets + b * (S + 1));
  int32_t* lb = a.list + b * n;
  for (int64_t i0 = 0; i0 < n; i0 += BK_THREADS) {  // uniform trip count: whole waves zero rows
    const int64_t i = i0 + tid;
    const int64_t s = i < n ? ib[i] : 0;
    const bool valid = s >= 0 && s < S;
    if (i < n && valid) lb[atomicAdd(&hist[s], 1)] = static_cast<int32_t>(i);
    zero_rows_wave<EM>(a, b, i, i < n && !valid);
  }
}

// The same sort over many workgroups per sequence (three launches): counts per
// pair group, per-(group, segment) bases, then the scatter.  Group c holds the
// blocks of BK_THREADS pairs c, c + bk_chunks, c + 2 bk_chunks, ... (about
// BK_ITEMS pairs): strided rather than contiguous, so that the empty slots of
// the first segments' short windows, which can fill most of the first 16384
// pairs, are zeroed by every group instead of one or two.  The order of pairs
// inside a segment does not change any result.
template <class EM>
__global__ __launch_bounds__(BK_THREADS) void bucket_count_kernel(const RetrieveArgs a) {
  extern __shared__ int hist[];  // [segments]
  const int tid = threadIdx.x;
  const int64_t b = blockIdx.y, chunk = blockIdx.x;
  const int64_t S = a.segments, n = a.n_index;
  const int64_t n_blocks = (n + BK_THREADS - 1) / BK_THREADS;
  const int64_t* ib = a.idx + b * n;
  for (int64_t s = tid; s < S; s += BK_THREADS) hist[s] = 0;
  __syncthreads();
  for (int64_t blk = chunk; blk < n_blocks; blk += a.bk_chunks) {  // uniform trip count: whole waves zero rows
    const int64_t i = blk * BK_THREADS + tid;
    const int64_t s = i < n ? ib[i] : 0;
    const bool valid = s >= 0 && s < S;
    if (i < n && valid) atomicAdd(&hist[s], 1);
    zero_rows_wave<EM>(a, b, i, i < n && !valid);
  }
  __syncthreads();
  int32_t* pc = a.partial + (b * a.bk_chunks + chunk) * S;
  for (int64_t s = tid; s < S; s += BK_THREADS) pc[s] = hist[s];
}

__global__ __launch_bounds__(BK_THREADS) void bucket_bases_kernel(const RetrieveArgs a) {
  extern __shared__ int hist[];  // [segments]: totals, then segment offsets
  const int tid = threadIdx.x;
  const int64_t b = blockIdx.x;
  const int64_t S = a.segments;
  int32_t* pb = a.partial + b * a.bk_chunks * S;
  for (int64_t s = tid; s < S; s += BK_THREADS) {
    int run = 0;
    for (int c = 0; c < a.bk_chunks; ++c) {
      const int v = pb[c * S + s];
      pb[c * S + s] = run;
      run += v;
    }
    hist[s] = run;
  }
  __syncthreads();
  bucket_offsets(hist, S, a.offsets + b * (S + 1));
  for (int64_t s = tid; s < S; s += BK_THREADS) {
    const int off = hist[s];
    for (int c = 0; c < a.bk_chunks; ++c) pb[c * S + s] += off;
  }
}

__global__ __launch_bounds__(BK_THREADS) void bucket_scatter_kernel(const RetrieveArgs a) {
  extern __shared__ int cur[];  // [segments]: next slot of each segment for this chunk
  const int tid = threadIdx.x;
  const int64_t b = blockIdx.y, chunk = blockIdx.x;
  const int64_t S = a.segments, n = a.n_index;
  const int64_t n_blocks = (n + BK_THREADS - 1) / BK_THREADS;
  const int64_t* ib = a.idx + b * n;
  const int32_t* pc = a.partial + (b * a.bk_chunks + chunk) * S;
  for (int64_t s = tid; s < S; s += BK_THREADS) cur[s] = pc[s];
  __syncthreads();
  int32_t* lb = a.list + b * n;
  for (int64_t blk = chunk; blk < n_blocks; blk += a.bk_chunks) {  // the count kernel's pair group
    const int64_t i = blk * BK_THREADS + tid;
    if (i >= n) continue;
    const int64_t s = ib[i];
    if (s >= 0 && s < S) lb[atomicAdd(&cur[s], 1)] = static_cast<int32_t>(i);
  }
}

// The apply kernels' work list of one sequence: segment s with c pairs gives
// ceil(c / tile_pairs) tiles, in segment order (one workgroup per sequence).
__global__ __launch_bounds__(BK_THREADS) void tile_list_kernel(const RetrieveArgs a) {
  extern __shared__ int hist[];  // [segments]: tiles per segment, then their first slot
  const int tid = threadIdx.x;
  const int64_t b = blockIdx.x;
  const int64_t S = a.segments;
  const int32_t* off = a.offsets + b * (S + 1);
  const int tp = a.tile_pairs;
  for (int64_t s = tid; s < S; s += BK_THREADS) hist[s] = (off[s + 1] - off[s] + tp - 1) / tp;
  __syncthreads();
  int32_t* base = a.tile_base + b * (S + 1);
  bucket_offsets(hist, S, base);
  int4* tl = a.tiles + b * a.tb_max;
  for (int64_t s = tid; s < S; s += BK_THREADS) {
    const int p0 = off[s], p1 = off[s + 1];
    int slot = hist[s];
    for (int p = p0; p < p1; p += tp) tl[slot++] = make_int4(static_cast<int>(s), p, min(p1, p + tp), 0);
  }
  if (tid == 0) a.n_tiles[b] = base[S];
}

// Sixteen bytes of a row-major tile as fp32 values (8 elements for 16-bit types,
// 4 for float32); an OOB offset reads zeros.
template <class E>
__device__ __forceinline__ void load16_f32(__amdgpu_buffer_rsrc_t r, int off, float* dst) {
  const u32x4 u = __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0);
  if constexpr (sizeof(typename ET<E>::raw) == 2) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      dst[2 * i] = ET<E>::to_f(static_cast<typename ET<E>::raw>(u[i] & 0xffffu));
      dst[2 * i + 1] = ET<E>::to_f(static_cast<typename ET<E>::raw>(u[i] >> 16));
    }
  } else {
#pragma unroll
    for (int i = 0; i < 4; ++i) dst[i] = __uint_as_float(u[i]);
  }
}

// ---------------------------------------------------------------------------
// One workgroup per (sequence, segment, 128-row value tile).  Wave w computes
// value rows [32w, 32w + 32) for 64 pairs: D[v][p] = sum_k M[v][k] q'[p][k]
// with A = state rows v, B = query rows p (lane (g, n) of a 16x16x4 operand
// holds row n, key 4kk + g).
template <class EL, class EM, class EQ, int DKP, bool VEC>
__global__ __launch_bounds__(AP_THREADS) void apply_bucket_kernel(const RetrieveArgs a) {
  using rawl = typename ET<EL>::raw;  // stored memories
  using rawm = typename ET<EM>::raw;  // arithmetic / output type
  using rawq = typename ET<EQ>::raw;
  constexpr int MS = DKP + 4;                            // state tile row stride (floats)
  constexpr int QS = (DKP > AP_V ? DKP : AP_V) + 4;      // query / output tile row stride
  constexpr int EPU_M = 16 / sizeof(rawl);               // elements per 16-byte unit
  constexpr int EPU_Q = 16 / sizeof(rawq);
  constexpr int UPR_M = DKP / EPU_M;                     // units per padded row
  constexpr int UPR_Q = DKP / EPU_Q;
  constexpr int M_UNITS = AP_V * UPR_M / AP_THREADS;     // per thread
  constexpr int Q_UNITS = (AP_N * UPR_Q + AP_THREADS - 1) / AP_THREADS;
  static_assert(M_UNITS * AP_THREADS == AP_V * UPR_M, "state tile splits evenly");
  extern __shared__ __align__(16) float sm[];
  float* Ms = sm;              // [AP_V][MS]
  float* QO = Ms + AP_V * MS;  // [AP_N][QS]: queries, then the output tile
  __shared__ int pair_id[AP_N];

  const int tid = threadIdx.x;
  const int lane = tid & 63, g = lane >> 4, n = lane & 15;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int64_t vt = blockIdx.x % a.v_tiles;
  const int64_t tile = blockIdx.x / a.v_tiles;
  const int64_t b = blockIdx.y;
  if (tile >= a.n_tiles[b]) return;
  const int4 te = a.tiles[b * a.tb_max + tile];
  const int64_t s = te.x;
  const int p_begin = te.y, p_end = te.z;
  const int dk = a.dk, dv = a.dv;
  const int v0 = static_cast<int>(vt) * AP_V;

  // State rows v0 .. v0 + 127 as fp32, zero past d_v and d_k.
  const rawl* msrc = static_cast<const rawl*>(a.mem) + (b * a.segments + s) * dv * dk;
  if constexpr (VEC) {
    const __amdgpu_buffer_rsrc_t rm = make_rsrc(msrc, static_cast<uint32_t>(dv * dk * sizeof(rawl)));
    float x[M_UNITS][EPU_M];
#pragma unroll
    for (int u = 0; u < M_UNITS; ++u) {
      const int e = tid + AP_THREADS * u;
      const int v = e / UPR_M, c = (e % UPR_M) * EPU_M;
      load16_f32<EL>(rm, (v0 + v < dv && c < dk) ? ((v0 + v) * dk + c) * static_cast<int>(sizeof(rawl)) : kBufOOB,
                     x[u]);
    }
#pragma unroll
    for (int u = 0; u < M_UNITS; ++u) {
      const int e = tid + AP_THREADS * u;
      const int v = e / UPR_M, c = (e % UPR_M) * EPU_M;
#pragma unroll
      for (int i = 0; i < EPU_M; i += 4)
        *reinterpret_cast<f32x4*>(Ms + v * MS + c + i) = f32x4{x[u][i], x[u][i + 1], x[u][i + 2], x[u][i + 3]};
    }
  } else {
    for (int e = tid; e < AP_V * DKP; e += AP_THREADS) {
      const int v = e / DKP, k = e % DKP;
      Ms[v * MS + k] = (v0 + v < dv && k < dk) ? ET<EL>::to_f(msrc[(v0 + v) * dk + k]) : 0.f;
    }
  }
  const int32_t* lb = a.list + b * a.n_index;
  const rawq* qsrc = static_cast<const rawq*>(a.queries) + b * a.n_query * dk;
  const __amdgpu_buffer_rsrc_t rq = make_rsrc(qsrc, static_cast<uint32_t>(a.n_query * dk * sizeof(rawq)));
  rawm* obase = static_cast<rawm*>(a.out) + b * a.n_index * dv;

  for (int p0 = p_begin; p0 < p_end; p0 += AP_N) {
    const int np = min(AP_N, p_end - p0);
    __syncthreads();  // state tile in place; previous output tile written out
    if (tid < AP_N) pair_id[tid] = tid < np ? lb[p0 + tid] : -1;
    __syncthreads();
    // Query rows of the tile's pairs, cast to the memories' dtype (the caller's
    // cast of q), as fp32.
    if constexpr (VEC) {
      float x[Q_UNITS][EPU_Q];
#pragma unroll
      for (int u = 0; u < Q_UNITS; ++u) {
        const int e = tid + AP_THREADS * u;
        const int p = min(e / UPR_Q, AP_N - 1), c = (e % UPR_Q) * EPU_Q;
        const int pid = pair_id[p];
        const int qoff = (e < AP_N * UPR_Q && pid >= 0 && c < dk)
                             ? (static_cast<int>(pid / a.routes) * dk + c) * static_cast<int>(sizeof(rawq))
                             : kBufOOB;
        load16_f32<EQ>(rq, qoff, x[u]);
      }
#pragma unroll
      for (int u = 0; u < Q_UNITS; ++u) {
        const int e = tid + AP_THREADS * u;
        if (e >= AP_N * UPR_Q) continue;
        const int p = e / UPR_Q, c = (e % UPR_Q) * EPU_Q;
#pragma unroll
        for (int i = 0; i < EPU_Q; i += 4) {
          f32x4 y;
#pragma unroll
          for (int j = 0; j < 4; ++j) y[j] = ET<EM>::to_f(ET<EM>::from_f(x[u][i + j]));
          *reinterpret_cast<f32x4*>(QO + p * QS + c + i) = y;
        }
      }
    } else {
      for (int e = tid; e < AP_N * DKP; e += AP_THREADS) {
        const int p = e / DKP, k = e % DKP;
        const int pid = pair_id[p];
        float x = 0.f;
        if (pid >= 0 && k < dk) x = ET<EM>::to_f(ET<EM>::from_f(ET<EQ>::to_f(qsrc[(pid / a.routes) * dk + k])));
        QO[p * QS + k] = x;
      }
    }
    __syncthreads();
    f32x4 acc[2][4];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll 4
    for (int kk = 0; kk < DKP / 4; ++kk) {
      float av[2], bv[4];
#pragma unroll
      for (int i = 0; i < 2; ++i) av[i] = Ms[(32 * w + 16 * i + n) * MS + 4 * kk + g];
#pragma unroll
      for (int j = 0; j < 4; ++j) bv[j] = QO[(16 * j + n) * QS + 4 * kk + g];
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(av[i], bv[j], acc[i][j], 0, 0, 0);
    }
    __syncthreads();  // query tile consumed
    // lane (g, n) holds D[v = 32w + 16i + 4g + r][p = 16j + n]
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j)
        *reinterpret_cast<f32x4*>(QO + (16 * j + n) * QS + 32 * w + 16 * i + 4 * g) = acc[i][j];
    __syncthreads();
    // whole output rows: pair p -> out[b, pair_id[p], v0 .. v0 + 127]
    const int vcols = min(AP_V, dv - v0);
    for (int e = tid; e < np * AP_V; e += AP_THREADS) {
      const int p = e / AP_V, v = e % AP_V;
      if (v < vcols) obase[static_cast<int64_t>(pair_id[p]) * dv + v0 + v] = ET<EM>::from_f(QO[p * QS + v]);
    }
  }
}

// Register-operand variant (16-byte aligned rows): no input tiles in LDS.  The
// key order of every 4-deep fp32 MFMA step is permuted so that lane group g
// owns keys [g*KG, (g+1)*KG), KG = DKP / 4: step t uses key g*KG + t in group g.
// A lane then holds 32 (for d_k = 128) consecutive keys of its state row and of
// its pair's query row, both loaded with 16-byte vector loads straight into the
// operand registers.  Only the output tile goes through LDS (for whole-row
// stores), so two or three workgroups share a CU and hide each other's latency.
template <class EL, class EM, class EQ, int DKP>
__global__ __launch_bounds__(AP_THREADS) void apply_reg_kernel(const RetrieveArgs a) {
  using rawl = typename ET<EL>::raw;  // stored memories
  using rawm = typename ET<EM>::raw;  // arithmetic / output type
  using rawq = typename ET<EQ>::raw;
  constexpr int KG = DKP / 4;                       // keys per lane group
  constexpr int OS = AP_V + 4;                      // output tile row stride (floats)
  constexpr int EPU_M = 16 / sizeof(rawl);
  constexpr int EPU_Q = 16 / sizeof(rawq);
  static_assert(KG % EPU_M == 0 && KG % EPU_Q == 0, "a lane's keys are whole 16-byte units");
  __shared__ __align__(16) float Os[AP_N * OS];

  const int tid = threadIdx.x;
  const int lane = tid & 63, g = lane >> 4, n = lane & 15;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int64_t vt = blockIdx.x % a.v_tiles;
  const int64_t tile = blockIdx.x / a.v_tiles;
  const int64_t b = blockIdx.y;
  if (tile >= a.n_tiles[b]) return;
  const int4 te = a.tiles[b * a.tb_max + tile];
  const int64_t s = te.x;
  const int p_begin = te.y, p_end = te.z;
  const int dk = a.dk, dv = a.dv;
  const int v0 = static_cast<int>(vt) * AP_V;
  const int k0 = g * KG;

  // A operands: state rows v = v0 + 32w + 16i + n, keys k0 .. k0 + KG - 1.
  const rawl* msrc = static_cast<const rawl*>(a.mem) + (b * a.segments + s) * dv * dk;
  const __amdgpu_buffer_rsrc_t rm = make_rsrc(msrc, static_cast<uint32_t>(dv * dk * sizeof(rawl)));
  float am[2][KG];
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int v = v0 + 32 * w + 16 * i + n;
#pragma unroll
    for (int u = 0; u < KG / EPU_M; ++u) {
      const int k = k0 + u * EPU_M;
      load16_f32<EL>(rm, (v < dv && k < dk) ? (v * dk + k) * static_cast<int>(sizeof(rawl)) : kBufOOB,
                     &am[i][u * EPU_M]);
    }
  }
  const int32_t* lb = a.list + b * a.n_index;
  const rawq* qsrc = static_cast<const rawq*>(a.queries) + b * a.n_query * dk;
  const __amdgpu_buffer_rsrc_t rq = make_rsrc(qsrc, static_cast<uint32_t>(a.n_query * dk * sizeof(rawq)));
  rawm* obase = static_cast<rawm*>(a.out) + b * a.n_index * dv;
  const int vcols = min(AP_V, dv - v0);

  for (int p0 = p_begin; p0 < p_end; p0 += AP_N) {
    const int np = min(AP_N, p_end - p0);
    f32x4 acc[2][4];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      // B operand: the query of pair 16j + n, keys k0 .. k0 + KG - 1, cast to
      // the memories' dtype (the caller's cast of q).
      const int p = 16 * j + n;
      const int pid = p < np ? lb[p0 + p] : -1;
      float bq[KG];
#pragma unroll
      for (int u = 0; u < KG / EPU_Q; ++u) {
        const int k = k0 + u * EPU_Q;
        load16_f32<EQ>(rq, (pid >= 0 && k < dk) ? (static_cast<int>(pid / a.routes) * dk + k) *
                                                      static_cast<int>(sizeof(rawq))
                                                : kBufOOB,
                       &bq[u * EPU_Q]);
      }
#pragma unroll
      for (int t = 0; t < KG; ++t) bq[t] = ET<EM>::to_f(ET<EM>::from_f(bq[t]));
#pragma unroll
      for (int t = 0; t < KG; ++t) {
#pragma unroll
        for (int i = 0; i < 2; ++i) acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(am[i][t], bq[t], acc[i][j], 0, 0, 0);
      }
    }
    __syncthreads();  // previous output tile written out
    // lane (g, n) holds D[v = 32w + 16i + 4g + r][p = 16j + n]
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j)
        *reinterpret_cast<f32x4*>(Os + (16 * j + n) * OS + 32 * w + 16 * i + 4 * g) = acc[i][j];
    __syncthreads();
    // whole output rows, four values per thread: pair p -> out[b, pair, v0 .. v0 + 127]
    for (int e = tid; e < np * (AP_V / 4); e += AP_THREADS) {
      const int p = e / (AP_V / 4), v = (e % (AP_V / 4)) * 4;
      const int pid = lb[p0 + p];
      const f32x4 val = *reinterpret_cast<const f32x4*>(Os + p * OS + v);
      rawm* dst = obase + static_cast<int64_t>(pid) * dv + v0 + v;
      if (v + 4 <= vcols) {
        store4_raw<EM>(dst, val);
      } else {
#pragma unroll
        for (int r = 0; r < 4; ++r)
          if (v + r < vcols) dst[r] = ET<EM>::from_f(val[r]);
      }
    }
  }
}

// 16-bit MFMA variant, exact: the memories are split into NPART parts of the
// MFMA input type EF (one part when EM is EF; hi + mid + lo bf16 parts, which
// together hold all 24 mantissa bits, when EM is float32), and the query cast
// to EM is exact in EF, so every product is exact and only the float32
// accumulation rounds, as in a float32 dot product.  MFMA step c (16x16x32)
// takes keys 32c + 8g .. + 7 from lane group g, so the four groups of a row
// read consecutive bytes: each state load instruction covers whole 128-byte
// lines of 16 rows (fp32 states) instead of 16-byte pieces of 64 lines.
template <class EL, class EM, class EQ, int DKP, class EF, int NPART, bool SCALED = false>
__global__ __launch_bounds__(AP_THREADS) void apply_mfma16_kernel(const RetrieveArgs a) {
  using rawl = typename ET<EL>::raw;  // stored memories
  using rawm = typename ET<EM>::raw;  // arithmetic / output type
  using rawq = typename ET<EQ>::raw;
  constexpr int KG = DKP / 4;
  constexpr int NSTEP = KG / 8;
  constexpr int OS = AP_V + 4;
  constexpr int EPU_M = 16 / sizeof(rawl);
  constexpr int EPU_Q = 16 / sizeof(rawq);
  static_assert(KG % 8 == 0 && KG % EPU_M == 0 && KG % EPU_Q == 0, "a lane's keys are whole MFMA slots");
  static_assert(AP_N == 64, "one pair per lane");
  __shared__ __align__(16) float Os[AP_N * OS];

  const int tid = threadIdx.x;
  const int lane = tid & 63, g = lane >> 4, n = lane & 15;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int64_t vt = blockIdx.x % a.v_tiles;
  const int64_t tile = blockIdx.x / a.v_tiles;
  const int64_t b = blockIdx.y;
  if (tile >= a.n_tiles[b]) return;
  const int4 te = a.tiles[b * a.tb_max + tile];
  const int64_t s = te.x;
  const int p_begin = te.y, p_end = te.z;
  const int dk = a.dk, dv = a.dv;
  const int v0 = static_cast<int>(vt) * AP_V;
  // Register slot x (0 .. KG - 1) of a lane's state row / query holds key key_of(x).
  auto key_of = [&](int x) { return 32 * (x >> 3) + 8 * g + (x & 7); };
  static_assert(EPU_M <= 8 && EPU_Q <= 8, "a 16-byte load stays inside one MFMA slot group");
  const int32_t* lb = a.list + b * a.n_index;
  // Pair ids of the first tile, one per lane (issued before the state loads so
  // that waiting for them does not wait for the state).
  int pid_l = lane < p_end - p_begin ? lb[p_begin + lane] : -1;

  const rawl* msrc = static_cast<const rawl*>(a.mem) + (b * a.segments + s) * dv * dk;
  const __amdgpu_buffer_rsrc_t rm = make_rsrc(msrc, static_cast<uint32_t>(dv * dk * sizeof(rawl)));
  float xm[2][KG];
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int v = v0 + 32 * w + 16 * i + n;
#pragma unroll
    for (int u = 0; u < KG / EPU_M; ++u) {
      const int k = key_of(u * EPU_M);
      load16_f32<EL>(rm, (v < dv && k < dk) ? (v * dk + k) * static_cast<int>(sizeof(rawl)) : kBufOOB,
                     &xm[i][u * EPU_M]);
    }
  }
  const rawq* qsrc = static_cast<const rawq*>(a.queries) + b * a.n_query * dk;
  const __amdgpu_buffer_rsrc_t rq = make_rsrc(qsrc, static_cast<uint32_t>(a.n_query * dk * sizeof(rawq)));
  rawm* obase = static_cast<rawm*>(a.out) + b * a.n_index * dv;
  const int vcols = min(AP_V, dv - v0);

  Frag8<EF> am[2][NPART][NSTEP];
  bool split = false;
  // The query's MFMA operand: q cast to EM, then to EF.  When both casts are
  // exact (a 16-bit query of type EF, EM float32 or EF) the operand is the
  // query's own bits, loaded as they are (half the registers of float32).
  constexpr bool kRawQ = std::is_same_v<EQ, EF> && (std::is_same_v<EM, F32> || std::is_same_v<EM, EQ>);
  float xq[kRawQ ? 1 : 4][kRawQ ? 1 : KG];
  Frag8<EF> rq8[4][kRawQ ? NSTEP : 1];
  // Query rows of a 64-pair step: lane 16 j + n holds pair j's row in slot j.
  // The loads of step s + 1 are issued right after step s's products, so they
  // overlap its output tile instead of opening the next step.
  auto load_q = [&](int pid_src) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int pid = __shfl(pid_src, 16 * j + n, 64);
      if constexpr (kRawQ) {
#pragma unroll
        for (int c = 0; c < NSTEP; ++c) {
          const int k = key_of(8 * c);
          const int off = (pid >= 0 && k < dk) ? (static_cast<int>(pid / a.routes) * dk + k) *
                                                     static_cast<int>(sizeof(rawq))
                                               : kBufOOB;
          rq8[j][c] = __builtin_bit_cast(Frag8<EF>, __builtin_amdgcn_raw_buffer_load_b128(rq, off, 0, 0));
        }
      } else {
#pragma unroll
        for (int u = 0; u < KG / EPU_Q; ++u) {
          const int k = key_of(u * EPU_Q);
          load16_f32<EQ>(rq, (pid >= 0 && k < dk) ? (static_cast<int>(pid / a.routes) * dk + k) *
                                                        static_cast<int>(sizeof(rawq))
                                                  : kBufOOB,
                         &xq[j][u * EPU_Q]);
        }
      }
    }
  };
  load_q(pid_l);
  for (int p0 = p_begin; p0 < p_end; p0 += AP_N) {
    const int np = min(AP_N, p_end - p0);
    const int pid_cur = pid_l;
    const bool more = p0 + AP_N < p_end;
    const int pid_next = (more && lane < p_end - p0 - AP_N) ? lb[p0 + AP_N + lane] : -1;
    // The gate of this lane's pair, loaded while the tile's products run.
    float gate_cur = 0.f;
    if constexpr (SCALED) gate_cur = pid_cur >= 0 ? a.gates[b * a.n_index + pid_cur] : 0.f;
    if (!split) {
      split = true;
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int c = 0; c < NSTEP; ++c)
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            float rest = xm[i][8 * c + e];
#pragma unroll
            for (int part = 0; part < NPART; ++part) {
              const typename ET<EF>::raw h = ET<EF>::from_f(rest);
              am[i][part][c].e[e] = h;
              rest -= ET<EF>::to_f(h);
            }
          }
    }
    f32x4 acc[2][4];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      Frag8<EF> bq[NSTEP];
#pragma unroll
      for (int c = 0; c < NSTEP; ++c) {
        if constexpr (kRawQ) {
          bq[c] = rq8[j][c];
        } else {
#pragma unroll
          for (int e = 0; e < 8; ++e) bq[c].e[e] = ET<EF>::from_f(ET<EM>::to_f(ET<EM>::from_f(xq[j][8 * c + e])));
        }
      }
#pragma unroll
      for (int c = 0; c < NSTEP; ++c)
#pragma unroll
        for (int part = 0; part < NPART; ++part)
#pragma unroll
          for (int i = 0; i < 2; ++i) acc[i][j] = mfma8(am[i][part][c], bq[c], acc[i][j]);
    }
    if (more) load_q(pid_next);
    pid_l = pid_next;
    __syncthreads();  // previous output tile written out
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j)
        *reinterpret_cast<f32x4*>(Os + (16 * j + n) * OS + 32 * w + 16 * i + 4 * g) = acc[i][j];
    __syncthreads();
    constexpr int PER = AP_N * (AP_V / 4) / AP_THREADS;  // stores per thread per full tile
#pragma unroll
    for (int it = 0; it < PER; ++it) {
      const int e = tid + AP_THREADS * it;
      const int p = e / (AP_V / 4), v = (e % (AP_V / 4)) * 4;
      const int pid = __shfl(pid_cur, p, 64);
      if constexpr (SCALED) {
        // The 32 lanes of one half-wave hold pair p's 128 values of this tile:
        // scale the gate-weighted row so its largest magnitude lies in
        // [2^14, 2^15) and store it as float16 with the inverse power of two.
        const float gp = __shfl(gate_cur, p, 64);
        const f32x4 val = *reinterpret_cast<const f32x4*>(Os + p * OS + v) * gp;
        float m = fmaxf(fmaxf(fabsf(val[0]), fabsf(val[1])), fmaxf(fabsf(val[2]), fabsf(val[3])));
        // maximum over the 32 lanes of the half-wave without LDS: quad swaps, the
        // half-row and row mirrors (DPP), then the 16-lane row swap
        m = fmaxf(m, __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(m), 0xb1, 0xf, 0xf, false)));
        m = fmaxf(m, __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(m), 0x4e, 0xf, 0xf, false)));
        m = fmaxf(m, __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(m), 0x141, 0xf, 0xf, false)));
        m = fmaxf(m, __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(m), 0x140, 0xf, 0xf, false)));
        {
          const auto sw = __builtin_amdgcn_permlane16_swap(__float_as_uint(m), __float_as_uint(m), false, false);
          m = fmaxf(__uint_as_float(sw[0]), __uint_as_float(sw[1]));
        }
        int ex = 0;
        (void)frexpf(m, &ex);
        const int sh = min(max(15 - ex, -100), 100);
        if (p < np) {
          uint16_t* dst = static_cast<uint16_t*>(a.out) + (b * a.n_index + pid) * static_cast<int64_t>(dv) + v0 + v;
          if (v + 4 <= vcols) {
            uint2 q;
            q.x = pack2<F16>(ldexpf(val[0], sh), ldexpf(val[1], sh));
            q.y = pack2<F16>(ldexpf(val[2], sh), ldexpf(val[3], sh));
            *reinterpret_cast<uint2*>(dst) = q;
          } else {
#pragma unroll
            for (int r = 0; r < 4; ++r)
              if (v + r < vcols) dst[r] = ET<F16>::from_f(ldexpf(val[r], sh));
          }
          if ((tid & 31) == 0) a.scales[(b * a.n_index + pid) * a.v_tiles + vt] = ldexpf(1.f, -sh);
        }
        continue;
      }
      if (p < np) {
        const f32x4 val = *reinterpret_cast<const f32x4*>(Os + p * OS + v);
        rawm* dst = obase + static_cast<int64_t>(pid) * dv + v0 + v;
        if (v + 4 <= vcols) {
          store4_raw<EM>(dst, val);
        } else {
#pragma unroll
          for (int r = 0; r < 4; ++r)
            if (v + r < vcols) dst[r] = ET<EM>::from_f(val[r]);
        }
      }
    }
  }
}

template <class EL, class EM, class EQ, int DKP, class EF, int NPART, bool SCALED = false>
int launch_apply_mfma16(const RetrieveArgs& a, hipStream_t s) {
  const dim3 grid(static_cast<unsigned>(static_cast<int64_t>(a.tb_max) * a.v_tiles), static_cast<unsigned>(a.batch));
  hipLaunchKernelGGL((apply_mfma16_kernel<EL, EM, EQ, DKP, EF, NPART, SCALED>), grid,
                     dim3(AP_THREADS), 0, s, a);
  return check_launch("gather_apply");
}

template <class EL, class EM, class EQ, int DKP>
int launch_apply_reg(const RetrieveArgs& a, hipStream_t s) {
  const dim3 grid(static_cast<unsigned>(static_cast<int64_t>(a.tb_max) * a.v_tiles), static_cast<unsigned>(a.batch));
  hipLaunchKernelGGL((apply_reg_kernel<EL, EM, EQ, DKP>), grid, dim3(AP_THREADS), 0, s,
                     a);
  return check_launch("gather_apply");
}

template <class EL, class EM, class EQ, int DKP, bool VEC>
int launch_apply(const RetrieveArgs& a, hipStream_t s) {
  constexpr int MS = DKP + 4;
  constexpr int QS = (DKP > AP_V ? DKP : AP_V) + 4;
  constexpr size_t lds = (static_cast<size_t>(AP_V) * MS + static_cast<size_t>(AP_N) * QS) * sizeof(float);
  static_assert(lds <= 160 * 1024, "apply tiles fit one CU's LDS");
  static bool attr_set = false;
  if (!attr_set) {
    hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(&apply_bucket_kernel<EL, EM, EQ, DKP, VEC>),
                                       hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(lds));
    if (e != hipSuccess) {
      set_error("gather_apply: hipFuncSetAttribute failed: %s", hipGetErrorString(e));
      return static_cast<int>(e);
    }
    attr_set = true;
  }
  const dim3 grid(static_cast<unsigned>(static_cast<int64_t>(a.tb_max) * a.v_tiles), static_cast<unsigned>(a.batch));
  hipLaunchKernelGGL((apply_bucket_kernel<EL, EM, EQ, DKP, VEC>), grid,
                     dim3(AP_THREADS), lds, s, a);
  return check_launch("gather_apply");
}

// 16-byte tile loads need whole units per row and 16-byte aligned bases.
template <class EL, class EQ>
bool vec_ok(const RetrieveArgs& a) {
  const int el = 16 / static_cast<int>(sizeof(typename ET<EL>::raw));
  const int eq = 16 / static_cast<int>(sizeof(typename ET<EQ>::raw));
  return a.dk % el == 0 && a.dk % eq == 0 && reinterpret_cast<uintptr_t>(a.mem) % 16 == 0 &&
         reinterpret_cast<uintptr_t>(a.queries) % 16 == 0 &&
         a.dv * static_cast<int64_t>(a.dk) * static_cast<int64_t>(sizeof(typename ET<EL>::raw)) < INT32_MAX &&
         a.n_query * static_cast<int64_t>(a.dk) * static_cast<int64_t>(sizeof(typename ET<EQ>::raw)) < INT32_MAX;
}

template <class EL, class EM, class EQ>
int dispatch_dk(const RetrieveArgs& a, hipStream_t s) {
  if (vec_ok<EL, EQ>(a)) {
    using Plan = MfmaPlan<EL, EM, EQ>;
    if constexpr (Plan::ok) {
      using EF = typename Plan::EF;
      constexpr int NPART = Plan::parts;
      if (a.dk <= 32) return launch_apply_mfma16<EL, EM, EQ, 32, EF, NPART>(a, s);
      if (a.dk <= 64) return launch_apply_mfma16<EL, EM, EQ, 64, EF, NPART>(a, s);
      return launch_apply_mfma16<EL, EM, EQ, 128, EF, NPART>(a, s);
    } else {
      if (a.dk <= 32) return launch_apply_reg<EL, EM, EQ, 32>(a, s);
      if (a.dk <= 64) return launch_apply_reg<EL, EM, EQ, 64>(a, s);
      return launch_apply_reg<EL, EM, EQ, 128>(a, s);
    }
  }
  if (a.dk <= 32) return launch_apply<EL, EM, EQ, 32, false>(a, s);
  if (a.dk <= 64) return launch_apply<EL, EM, EQ, 64, false>(a, s);
  return launch_apply<EL, EM, EQ, 128, false>(a, s);
}

template <class EL, class EM>
int dispatch_q(const RetrieveArgs& a, int q_dtype, hipStream_t s) {
  switch (q_dtype) {
    case GRM_HIP_F32: return dispatch_dk<EL, EM, F32>(a, s);
    case GRM_HIP_F16: return dispatch_dk<EL, EM, F16>(a, s);
    default: return dispatch_dk<EL, EM, BF16>(a, s);
  }
}

// ---------------------------------------------------------------------------
// Residual + LayerNorm over the scaled rows of retrieve_fuse:
//   out[t] = LN(h[t] + sum_r scales[t, r, c / 128] * rows[t, r, c])
// h and out in E, the LayerNorm weight and bias in float32,
// with r in order 0 .. R-1 (the gates are already in the rows), a two-pass
// mean / variance in fp32.  lpr lanes share a row, each covering NV groups of
// 8 consecutive columns (16-byte float16 loads of the rows).

template <class E>
__device__ __forceinline__ void load8(__amdgpu_buffer_rsrc_t r, int off, float (&f)[8]) {
  if constexpr (sizeof(typename ET<E>::raw) == 2) {
    const U8<E> u = __builtin_bit_cast(U8<E>, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0));
#pragma unroll
    for (int e = 0; e < 8; ++e) f[e] = ET<E>::to_f(u.e[e]);
  } else {
    const u32x4 lo = __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0);
    const u32x4 hi = __builtin_amdgcn_raw_buffer_load_b128(r, off == kBufOOB ? kBufOOB : off + 16, 0, 0);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      f[e] = __uint_as_float(lo[e]);
      f[4 + e] = __uint_as_float(hi[e]);
    }
  }
}

template <class E>
__device__ __forceinline__ void store8(__amdgpu_buffer_rsrc_t r, int off, const float (&y)[8]) {
  if constexpr (sizeof(typename ET<E>::raw) == 2) {
    const u32x4 q = u32x4{pack2<E>(y[0], y[1]), pack2<E>(y[2], y[3]), pack2<E>(y[4], y[5]), pack2<E>(y[6], y[7])};
    __builtin_amdgcn_raw_buffer_store_b128(q, r, off, 0, 0);
  } else {
    __builtin_amdgcn_raw_buffer_store_b128(
        u32x4{__float_as_uint(y[0]), __float_as_uint(y[1]), __float_as_uint(y[2]), __float_as_uint(y[3])}, r, off, 0, 0);
    __builtin_amdgcn_raw_buffer_store_b128(
        u32x4{__float_as_uint(y[4]), __float_as_uint(y[5]), __float_as_uint(y[6]), __float_as_uint(y[7])}, r,
        off == kBufOOB ? kBufOOB : off + 16, 0, 0);
  }
}

template <class E, int NV>
__global__ __launch_bounds__(256) void fuse_scaled_kernel(const FuseScaledArgs a, const int lpr) {
  using raw = typename ET<E>::raw;
  const int tid = threadIdx.x;
  const int sub = tid & (lpr - 1);
  const WaveRows wr = wave_rows(static_cast<int64_t>(blockIdx.x) * (256 / lpr), lpr, a.n_rows);
  const bool live = wr.row < a.n_rows;
  const int H = a.hidden;
  const int64_t rr = live ? wr.row : 0;
  const int hb = H * static_cast<int>(sizeof(raw)), rowb = a.routes * H * 2;  // row bytes of h / out, of rows
  const __amdgpu_buffer_rsrc_t rh = wave_rows_rsrc(a.h, wr, hb);
  const __amdgpu_buffer_rsrc_t rrow = wave_rows_rsrc(a.rows, wr, rowb);
  const float* sc = a.scales + rr * a.routes * a.v_tiles;
  float x[NV][8];
#pragma unroll
  for (int v = 0; v < NV; ++v) {
    const int c = (sub + lpr * v) * 8;
    const bool in = live && c < H;
    float hv[8];
    load8<E>(rh, in ? wr.local * hb + c * static_cast<int>(sizeof(raw)) : kBufOOB, hv);
    float r[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) r[e] = 0.f;
    const int tile = c / AP_V;
#pragma unroll 4
    for (int j = 0; j < a.routes; ++j) {
      const float sj = in ? sc[j * a.v_tiles + tile] : 0.f;
      float rv[8];
      load8<F16>(rrow, in ? wr.local * rowb + (j * H + c) * 2 : kBufOOB, rv);
#pragma unroll
      for (int e = 0; e < 8; ++e) r[e] = fmaf(sj, rv[e], r[e]);
    }
#pragma unroll
    for (int e = 0; e < 8; ++e) x[v][e] = c < H ? hv[e] + r[e] : 0.f;
  }
  const __amdgpu_buffer_rsrc_t ro = wave_rows_rsrc(a.out, wr, hb);
  auto out_off = [&](int v) {
    const int c = (sub + lpr * v) * 8;
    return (live && c < H) ? wr.local * hb + c * static_cast<int>(sizeof(raw)) : kBufOOB;
  };
  if (a.w == nullptr) {
#pragma unroll
    for (int v = 0; v < NV; ++v) store8<E>(ro, out_off(v), x[v]);
    return;
  }
  float sum = 0.f;
#pragma unroll
  for (int v = 0; v < NV; ++v)
#pragma unroll
    for (int e = 0; e < 8; ++e) sum += x[v][e];
  for (int off = lpr >> 1; off > 0; off >>= 1) sum += __shfl_xor(sum, off, 64);
  const float mean = sum / static_cast<float>(H);
  float var = 0.f;
#pragma unroll
  for (int v = 0; v < NV; ++v) {
    const int c = (sub + lpr * v) * 8;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float d = x[v][e] - mean;
      var = c < H ? fmaf(d, d, var) : var;
    }
  }
  for (int off = lpr >> 1; off > 0; off >>= 1) var += __shfl_xor(var, off, 64);
  const float rstd = 1.0f / sqrtf(var / static_cast<float>(H) + a.eps);
  const __amdgpu_buffer_rsrc_t rw = make_rsrc(a.w, H * 4);
  const __amdgpu_buffer_rsrc_t rb = make_rsrc(a.bias, a.bias != nullptr ? H * 4 : 0u);
#pragma unroll
  for (int v = 0; v < NV; ++v) {
    const int c = (sub + lpr * v) * 8;
    const int off = c < H ? c * 4 : kBufOOB;
    float wv[8], bv[8];
    load8<F32>(rw, off, wv);  // LayerNorm parameters are float32
    load8<F32>(rb, off, bv);  // zeros without a bias
    float y[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) y[e] = (x[v][e] - mean) * rstd * wv[e] + bv[e];
    store8<E>(ro, out_off(v), y);
  }
}

template <class E>
int launch_fuse_scaled(const FuseScaledArgs& a, hipStream_t s) {
  const int groups = a.hidden / 8;
  int lpr = 1;
  while (lpr < 64 && lpr < groups) lpr <<= 1;
  const int nv = (groups + lpr - 1) / lpr;
  const dim3 grid(static_cast<unsigned>((a.n_rows + 256 / lpr - 1) / (256 / lpr)));
  auto go = [&](auto nvc) {
    hipLaunchKernelGGL((fuse_scaled_kernel<E, decltype(nvc)::value>), grid, dim3(256), 0, s, a, lpr);
  };
  if (nv <= 1) go(std::integral_constant<int, 1>{});
  else if (nv <= 2) go(std::integral_constant<int, 2>{});
  else if (nv <= 4) go(std::integral_constant<int, 4>{});
  else go(std::integral_constant<int, 8>{});
  return check_launch("retrieve_fuse(fuse)");
}

}  // namespace

int fuse_scaled(const FuseScaledArgs& a, int h_dtype, hipStream_t s) {
  switch (h_dtype) {
    case GRM_HIP_F32: return launch_fuse_scaled<F32>(a, s);
    case GRM_HIP_F16: return launch_fuse_scaled<F16>(a, s);
    default: return launch_fuse_scaled<BF16>(a, s);
  }
}

namespace {

// The scaled apply runs the exact 16-bit MFMA kernel with float32 arithmetic;
// other dtype pairs and unaligned shapes are not supported by retrieve_fuse.
template <class EL, class EQ>
int launch_apply_scaled(const RetrieveArgs& a, hipStream_t s) {
  using Plan = MfmaPlan<EL, F32, EQ>;
  if constexpr (Plan::ok) {
    using EF = typename Plan::EF;
    constexpr int NPART = Plan::parts;
    if (a.dk <= 32) return launch_apply_mfma16<EL, F32, EQ, 32, EF, NPART, true>(a, s);
    if (a.dk <= 64) return launch_apply_mfma16<EL, F32, EQ, 64, EF, NPART, true>(a, s);
    return launch_apply_mfma16<EL, F32, EQ, 128, EF, NPART, true>(a, s);
  } else {
    set_error("retrieve_fuse: no exact 16-bit MFMA plan for these dtypes");
    return GRM_HIP_EUNSUPPORTED;
  }
}

template <class EL>
bool scaled_ok_q(const RetrieveArgs& a, int q_dtype) {
  switch (q_dtype) {
    case GRM_HIP_F16: return MfmaPlan<EL, F32, F16>::ok && vec_ok<EL, F16>(a);
    case GRM_HIP_BF16: return MfmaPlan<EL, F32, BF16>::ok && vec_ok<EL, BF16>(a);
    default: return false;
  }
}

bool scaled_supported(const RetrieveArgs& a, int mem_dtype, int q_dtype) {
  switch (mem_dtype) {
    case GRM_HIP_F32: return scaled_ok_q<F32>(a, q_dtype);
    case GRM_HIP_F16: return scaled_ok_q<F16>(a, q_dtype);
    default: return scaled_ok_q<BF16>(a, q_dtype);
  }
}

template <class EL>
int apply_scaled_q(const RetrieveArgs& a, int q_dtype, hipStream_t s) {
  return q_dtype == GRM_HIP_F16 ? launch_apply_scaled<EL, F16>(a, s) : launch_apply_scaled<EL, BF16>(a, s);
}

// ---------------------------------------------------------------------------
// The queries' gradient of gather_apply: for every pair (q, r) with a valid
// index, dqp[b, q, r, :] = M[b, idx[b, q, r]]^T g[b, q, r, :] (float32 grad_out
// rows of d_v, float32 result rows of d_k); the caller sums over r.  One
// workgroup of 8 waves per (sequence, work tile) stages its segment's state in
// LDS as float32, rows of d_v padded to a multiple of 16 with zeros, row stride
// DKP + 4 floats, and applies its transpose with float32 MFMA (16x16x4).  Wave
// w takes 16 pairs at a time: in MFMA j of value block v0, lane (kq, n) gives
// A = M[v0 + 4 kq + j][16 kb + n] and B = g[pair n][v0 + 4 kq + j], so each
// lane's gradient values of a block are one float4 (loaded a 128-value chunk
// ahead of the MFMAs), and the four rows one A read touches (4 apart) start
// 16 banks apart.  Each output row is written by one wave: deterministic, no
// atomics.
constexpr int AT_THREADS = 512;
constexpr int AT_CHUNK = 8;  // value blocks of 16 per prefetched chunk

template <int DKP>
__host__ __device__ constexpr int at_row_stride() { return DKP + 4; }

__host__ __device__ inline int at_rows(int dv) { return (dv + 15) / 16 * 16; }

template <class EL, int DKP>
__global__ __launch_bounds__(AT_THREADS) void apply_t_kernel(const RetrieveArgs a, const float* grad, float* dqp,
                                                             int vec_state, int vec_grad, int token_rows) {
  using rawl = typename ET<EL>::raw;
  extern __shared__ float Ms[];  // [at_rows(dv)][DKP + 4]
  constexpr int MSK = at_row_stride<DKP>();
  constexpr int KB = DKP / 16;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int64_t tile = blockIdx.x;
  const int64_t b = blockIdx.y;
  if (tile >= a.n_tiles[b]) return;
  const int4 te = a.tiles[b * a.tb_max + tile];
  const int64_t s = te.x;
  const int p_begin = te.y, p_end = te.z;
  const int dk = a.dk, dv = a.dv, dv16 = at_rows(dv);
  const rawl* msrc = static_cast<const rawl*>(a.mem) + (b * a.segments + s) * dv * dk;
  if (vec_state) {
    // dk == DKP and 16-byte aligned rows: 16 bytes of the state per thread and step
    constexpr int PER = 16 / sizeof(rawl);
    const int nvec = dv * DKP / PER;
    for (int e = tid; e < nvec; e += AT_THREADS) {
      const int idx = e * PER;
      const int v = idx / DKP, k = idx % DKP;
      rawl t[PER];
      *reinterpret_cast<uint4*>(t) = *reinterpret_cast<const uint4*>(msrc + idx);
#pragma unroll
      for (int i = 0; i < PER; i += 4)
        *reinterpret_cast<f32x4*>(Ms + v * MSK + k + i) =
            f32x4{ET<EL>::to_f(t[i]), ET<EL>::to_f(t[i + 1]), ET<EL>::to_f(t[i + 2]), ET<EL>::to_f(t[i + 3])};
    }
    for (int e = dv * DKP + tid; e < dv16 * DKP; e += AT_THREADS) Ms[(e / DKP) * MSK + e % DKP] = 0.f;
  } else {
    for (int e = tid; e < dv16 * DKP; e += AT_THREADS) {
      const int v = e / DKP, k = e % DKP;
      Ms[v * MSK + k] = (v < dv && k < dk) ? ET<EL>::to_f(msrc[v * dk + k]) : 0.f;
    }
  }
  __syncthreads();
  const int32_t* lb = a.list + b * a.n_index;
  const int n = lane & 15, kq = lane >> 4;
  const int n_chunks = (dv16 / 16 + AT_CHUNK - 1) / AT_CHUNK;
  int p0 = p_begin + 16 * w;
  int pid = p0 < p_end && p0 + n < p_end ? lb[p0 + n] : -1;
  for (; p0 < p_end; p0 += 16 * (AT_THREADS / 64)) {
    const int pn = p0 + 16 * (AT_THREADS / 64);
    const int pid_next = pn + n < p_end ? lb[pn + n] : -1;
    // grad rows per pair, or (token_rows) one row per query shared by its routes
    const int64_t grow_i = token_rows ? b * a.n_query + (pid >= 0 ? pid : 0) / a.routes
                                      : b * a.n_index + (pid >= 0 ? pid : 0);
    const float* grow = grad + grow_i * static_cast<int64_t>(dv);
    auto load_chunk = [&](f32x4* g, int c) {
#pragma unroll
      for (int u = 0; u < AT_CHUNK; ++u) {
        const int vq = 16 * (AT_CHUNK * c + u) + 4 * kq;
        f32x4 x{0.f, 0.f, 0.f, 0.f};
        if (pid >= 0) {
          if (vec_grad) {
            if (vq < dv) x = *reinterpret_cast<const f32x4*>(grow + vq);
          } else {
#pragma unroll
            for (int r = 0; r < 4; ++r)
              if (vq + r < dv) x[r] = grow[vq + r];
          }
        }
        g[u] = x;
      }
    };
    f32x4 acc[KB];
#pragma unroll
    for (int kb = 0; kb < KB; ++kb) acc[kb] = f32x4{0.f, 0.f, 0.f, 0.f};
    f32x4 cur[AT_CHUNK], nxt[AT_CHUNK];
    load_chunk(cur, 0);
    for (int c = 0; c < n_chunks; ++c) {
      if (c + 1 < n_chunks) load_chunk(nxt, c + 1);
#pragma unroll
      for (int u = 0; u < AT_CHUNK; ++u) {
        const int v0 = 16 * (AT_CHUNK * c + u);
        if (v0 < dv16) {
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            const float* mrow = Ms + (v0 + 4 * kq + j) * MSK + n;
#pragma unroll
            for (int kb = 0; kb < KB; ++kb)
              acc[kb] = __builtin_amdgcn_mfma_f32_16x16x4f32(mrow[16 * kb], cur[u][j], acc[kb], 0, 0, 0);
          }
        }
      }
      if (c + 1 < n_chunks) {
#pragma unroll
        for (int u = 0; u < AT_CHUNK; ++u) cur[u] = nxt[u];
      }
    }
    // lane (kq, n) holds keys 16 kb + 4 kq + r of pair n (the pair its pid names)
    if (pid >= 0) {
      float* orow = dqp + (b * a.n_index + pid) * static_cast<int64_t>(dk);
#pragma unroll
      for (int kb = 0; kb < KB; ++kb) {
        const int k = 16 * kb + 4 * kq;
        if (k + 4 <= dk && (dk & 3) == 0) {
          *reinterpret_cast<f32x4*>(orow + k) = acc[kb];
        } else {
#pragma unroll
          for (int r = 0; r < 4; ++r)
            if (k + r < dk) orow[k + r] = acc[kb][r];
        }
      }
    }
    pid = pid_next;
  }
}

// The same per-pair product M[idx]^T g for float16 archives on 16-bit MFMA.
// The state sits in LDS transposed ([DKP][value index], float16, rows padded by
// 8 values so the 16 rows of one fragment read start 4 banks apart).  Each
// 32-value chunk of a pair's float32 gradient row is scaled by the power of two
// that puts its largest magnitude in [2^14, 2^15) and split into float16 parts
// hi = round(g s) and lo = round(g s - hi); two 16x16x32 MFMAs (products of
// float16 values are exact in fp32) and one multiply by 1/s per chunk.  Error
// per chunk about 2^-22 of its largest magnitude times sum_v |M[v][k]|, the size
// of the fp32 accumulation's own rounding.  Chunks of 4 are loaded one group
// ahead, as apply_t_kernel does.
__host__ __device__ inline int at16_stride(int dv) { return (dv + 31) / 32 * 32 + 8; }

template <int DKP>
__global__ __launch_bounds__(AT_THREADS) void apply_t16_kernel(const RetrieveArgs a, const float* grad, float* dqp,
                                                               int vec_state, int vec_grad, int token_rows) {
  extern __shared__ uint16_t MsT[];  // [DKP][at16_stride(dv)]
  constexpr int KB = DKP / 16;
  constexpr int GC = 4;  // 32-value chunks per prefetched group
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int64_t tile = blockIdx.x;
  const int64_t b = blockIdx.y;
  if (tile >= a.n_tiles[b]) return;
  const int4 te = a.tiles[b * a.tb_max + tile];
  const int64_t s = te.x;
  const int p_begin = te.y, p_end = te.z;
  const int dk = a.dk, dv = a.dv;
  const int VS = at16_stride(dv);
  const int dv32 = VS - 8;
  const uint16_t* msrc = static_cast<const uint16_t*>(a.mem) + (b * a.segments + s) * dv * dk;
  if (vec_state) {
    // 16 bytes (8 key values of one value row) per thread and step, written transposed
    const int nvec = dv * dk / 8;
    for (int e = tid; e < nvec; e += AT_THREADS) {
      const int idx = 8 * e;
      const int v = idx / dk, k = idx % dk;
      const uint4 t = *reinterpret_cast<const uint4*>(msrc + idx);
      const uint32_t wds[4] = {t.x, t.y, t.z, t.w};
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        MsT[(k + 2 * j) * VS + v] = static_cast<uint16_t>(wds[j] & 0xffffu);
        MsT[(k + 2 * j + 1) * VS + v] = static_cast<uint16_t>(wds[j] >> 16);
      }
    }
  } else {
    for (int e = tid; e < dv * dk; e += AT_THREADS) MsT[(e % dk) * VS + e / dk] = msrc[e];
  }
  if (dk < DKP || dv < dv32) {
    for (int e = tid; e < DKP * dv32; e += AT_THREADS) {
      const int k = e / dv32, v = e % dv32;
      if (k >= dk || v >= dv) MsT[k * VS + v] = 0;
    }
  }
  __syncthreads();
  const int32_t* lb = a.list + b * a.n_index;
  const int n = lane & 15, kq = lane >> 4;
  const int nch = dv32 / 32;
  const int ngr = (nch + GC - 1) / GC;
  int p0 = p_begin + 16 * w;
  int pid = p0 < p_end && p0 + n < p_end ? lb[p0 + n] : -1;
  for (; p0 < p_end; p0 += 16 * (AT_THREADS / 64)) {
    const int pn = p0 + 16 * (AT_THREADS / 64);
    const int pid_next = pn + n < p_end ? lb[pn + n] : -1;
    // grad rows per pair, or (token_rows) one row per query shared by its routes
    const int64_t grow_i = token_rows ? b * a.n_query + (pid >= 0 ? pid : 0) / a.routes
                                      : b * a.n_index + (pid >= 0 ? pid : 0);
    const float* grow = grad + grow_i * static_cast<int64_t>(dv);
    // values 32 c + 8 kq .. + 7 of this lane's pair, chunks of group gi
    auto load_group = [&](float (&x)[GC][8], int gi) {
#pragma unroll
      for (int u = 0; u < GC; ++u) {
        const int v = 32 * (GC * gi + u) + 8 * kq;
#pragma unroll
        for (int j = 0; j < 8; ++j) x[u][j] = 0.f;
        if (pid >= 0) {
          if (vec_grad) {
            if (v < dv) {
              const f32x4 lo4 = *reinterpret_cast<const f32x4*>(grow + v);
#pragma unroll
              for (int j = 0; j < 4; ++j) x[u][j] = lo4[j];
            }
            if (v + 4 < dv) {
              const f32x4 hi4 = *reinterpret_cast<const f32x4*>(grow + v + 4);
#pragma unroll
              for (int j = 0; j < 4; ++j) x[u][4 + j] = hi4[j];
            }
          } else {
#pragma unroll
            for (int j = 0; j < 8; ++j)
              if (v + j < dv) x[u][j] = grow[v + j];
          }
        }
      }
    };
    f32x4 acc[KB];
#pragma unroll
    for (int kb = 0; kb < KB; ++kb) acc[kb] = f32x4{0.f, 0.f, 0.f, 0.f};
    float cur[GC][8], nxt[GC][8];
    load_group(cur, 0);
    for (int gi = 0; gi < ngr; ++gi) {
      if (gi + 1 < ngr) load_group(nxt, gi + 1);
#pragma unroll
      for (int u = 0; u < GC; ++u) {
        const int c = GC * gi + u;
        if (c < nch) {
          // the chunk's scale: its largest magnitude over the pair's 4 lanes
          float m = 0.f;
#pragma unroll
          for (int j = 0; j < 8; ++j) m = fmaxf(m, fabsf(cur[u][j]));
          m = fmaxf(m, __shfl_xor(m, 16, 64));
          m = fmaxf(m, __shfl_xor(m, 32, 64));
          const int ex = static_cast<int>((__float_as_uint(m) >> 23) & 0xffu);
          // s = 2^(14 - floor(log2 m)) as a biased exponent in [1, 253]; 1 for 0 or inf
          const int es = (m > 0.f && ex < 255) ? min(max(268 - ex, 1), 253) : 127;
          const float sc = __uint_as_float(static_cast<uint32_t>(es) << 23);
          const float inv = __uint_as_float(static_cast<uint32_t>(254 - es) << 23);
          Frag8<F16> hi, lo;
#pragma unroll
          for (int j = 0; j < 8; ++j) {
            const float x = cur[u][j] * sc;
            hi.e[j] = ET<F16>::from_f(x);
            lo.e[j] = ET<F16>::from_f(x - ET<F16>::to_f(hi.e[j]));
          }
          const int vA = 32 * c + 8 * kq;
#pragma unroll
          for (int kb = 0; kb < KB; ++kb) {
            const Frag8<F16> am =
                __builtin_bit_cast(Frag8<F16>, *reinterpret_cast<const uint4*>(MsT + (16 * kb + n) * VS + vA));
            f32x4 t = mfma8(am, hi, f32x4{0.f, 0.f, 0.f, 0.f});
            t = mfma8(am, lo, t);
#pragma unroll
            for (int r = 0; r < 4; ++r) acc[kb][r] = fmaf(t[r], inv, acc[kb][r]);
          }
        }
      }
      if (gi + 1 < ngr) {
#pragma unroll
        for (int u = 0; u < GC; ++u)
#pragma unroll
          for (int j = 0; j < 8; ++j) cur[u][j] = nxt[u][j];
      }
    }
    // lane (kq, n) holds keys 16 kb + 4 kq + r of pair n (the pair its pid names)
    if (pid >= 0) {
      float* orow = dqp + (b * a.n_index + pid) * static_cast<int64_t>(dk);
#pragma unroll
      for (int kb = 0; kb < KB; ++kb) {
        const int k = 16 * kb + 4 * kq;
        if (k + 4 <= dk && (dk & 3) == 0) {
          *reinterpret_cast<f32x4*>(orow + k) = acc[kb];
        } else {
#pragma unroll
          for (int r = 0; r < 4; ++r)
            if (k + r < dk) orow[k + r] = acc[kb][r];
        }
      }
    }
    pid = pid_next;
  }
}

inline size_t apply_t16_lds(int dv, int dkp) { return static_cast<size_t>(dkp) * at16_stride(dv) * sizeof(uint16_t); }

template <int DKP>
int launch_apply_t16(const RetrieveArgs& a, const float* grad, float* dqp, int token_rows, hipStream_t s) {
  const size_t lds = apply_t16_lds(a.dv, DKP);
  static bool attr_set = false;
  if (!attr_set) {
    hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(&apply_t16_kernel<DKP>),
                                       hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
    if (e != hipSuccess) {
      set_error("gather_apply_bwd: hipFuncSetAttribute failed: %s", hipGetErrorString(e));
      return static_cast<int>(e);
    }
    attr_set = true;
  }
  const int vec_state = a.dk % 8 == 0 && reinterpret_cast<uintptr_t>(a.mem) % 16 == 0;
  const int vec_grad = a.dv % 4 == 0 && reinterpret_cast<uintptr_t>(grad) % 16 == 0;
  const dim3 grid(static_cast<unsigned>(a.tb_max), static_cast<unsigned>(a.batch));
  hipLaunchKernelGGL((apply_t16_kernel<DKP>), grid, dim3(AT_THREADS), lds, s, a, grad, dqp, vec_state, vec_grad,
                     token_rows);
  return check_launch("gather_apply_bwd");
}

inline size_t apply_t_lds(int dv, int dkp) {
  return static_cast<size_t>(at_rows(dv)) * (dkp + 4) * sizeof(float);
}

template <class EL, int DKP>
int launch_apply_t(const RetrieveArgs& a, const float* grad, float* dqp, int token_rows, hipStream_t s) {
  using rawl = typename ET<EL>::raw;
  const size_t lds = apply_t_lds(a.dv, DKP);
  static bool attr_set = false;
  if (!attr_set) {
    hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(&apply_t_kernel<EL, DKP>),
                                       hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
    if (e != hipSuccess) {
      set_error("gather_apply_bwd: hipFuncSetAttribute failed: %s", hipGetErrorString(e));
      return static_cast<int>(e);
    }
    attr_set = true;
  }
  const int vec_state = a.dk == DKP && (DKP * sizeof(rawl)) % 16 == 0 &&
                        reinterpret_cast<uintptr_t>(a.mem) % 16 == 0;
  const int vec_grad = a.dv % 4 == 0 && reinterpret_cast<uintptr_t>(grad) % 16 == 0;
  const dim3 grid(static_cast<unsigned>(a.tb_max), static_cast<unsigned>(a.batch));
  hipLaunchKernelGGL((apply_t_kernel<EL, DKP>), grid, dim3(AT_THREADS), lds, s, a, grad, dqp, vec_state, vec_grad,
                     token_rows);
  return check_launch("gather_apply_bwd");
}

template <class EL>
int dispatch_apply_t(const RetrieveArgs& a, const float* grad, float* dqp, int token_rows, hipStream_t s) {
  if constexpr (std::is_same_v<EL, F16>) {
    // float16 archives: the 16-bit MFMA form (GRM_HIP_APPLY_T16=0 keeps the fp32 one)
    const char* env = getenv("GRM_HIP_APPLY_T16");
    if (env == nullptr || env[0] != '0') {
      if (a.dk <= 16) return launch_apply_t16<16>(a, grad, dqp, token_rows, s);
      if (a.dk <= 32) return launch_apply_t16<32>(a, grad, dqp, token_rows, s);
      if (a.dk <= 64) return launch_apply_t16<64>(a, grad, dqp, token_rows, s);
      return launch_apply_t16<128>(a, grad, dqp, token_rows, s);
    }
  }
  if (a.dk <= 16) return launch_apply_t<EL, 16>(a, grad, dqp, token_rows, s);
  if (a.dk <= 32) return launch_apply_t<EL, 32>(a, grad, dqp, token_rows, s);
  if (a.dk <= 64) return launch_apply_t<EL, 64>(a, grad, dqp, token_rows, s);
  return launch_apply_t<EL, 128>(a, grad, dqp, token_rows, s);
}

int allow_segment_lds(const void* fn) {
  const hipError_t e = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize,
                                           static_cast<int>(kMaxSegments * sizeof(int)));
  if (e != hipSuccess) {
    set_error("gather_apply: hipFuncSetAttribute failed: %s", hipGetErrorString(e));
    return static_cast<int>(e);
  }
  return GRM_HIP_OK;
}

template <class EM>
int launch_bucket(const RetrieveArgs& a, hipStream_t s) {
  const size_t lds = static_cast<size_t>(a.segments) * sizeof(int);
  static int attr_rc = -1;
  if (attr_rc != GRM_HIP_OK) {
    attr_rc = allow_segment_lds(reinterpret_cast<const void*>(&bucket_kernel<EM>));
    if (attr_rc == GRM_HIP_OK) attr_rc = allow_segment_lds(reinterpret_cast<const void*>(&bucket_count_kernel<EM>));
    if (attr_rc == GRM_HIP_OK) attr_rc = allow_segment_lds(reinterpret_cast<const void*>(&bucket_bases_kernel));
    if (attr_rc == GRM_HIP_OK) attr_rc = allow_segment_lds(reinterpret_cast<const void*>(&bucket_scatter_kernel));
    if (attr_rc == GRM_HIP_OK) attr_rc = allow_segment_lds(reinterpret_cast<const void*>(&tile_list_kernel));
    if (attr_rc != GRM_HIP_OK) return attr_rc;
  }
  int rc;
  if (a.bk_chunks <= 1) {
    hipLaunchKernelGGL((bucket_kernel<EM>), dim3(static_cast<unsigned>(a.batch)), dim3(BK_THREADS), lds, s, a);
    rc = check_launch("gather_apply(sort)");
  } else {
    const dim3 grid(static_cast<unsigned>(a.bk_chunks), static_cast<unsigned>(a.batch));
    hipLaunchKernelGGL((bucket_count_kernel<EM>), grid, dim3(BK_THREADS), lds, s, a);
    rc = check_launch("gather_apply(sort counts)");
    if (rc != GRM_HIP_OK) return rc;
    hipLaunchKernelGGL(bucket_bases_kernel, dim3(static_cast<unsigned>(a.batch)), dim3(BK_THREADS), lds, s, a);
    rc = check_launch("gather_apply(sort bases)");
    if (rc != GRM_HIP_OK) return rc;
    hipLaunchKernelGGL(bucket_scatter_kernel, grid, dim3(BK_THREADS), lds, s, a);
    rc = check_launch("gather_apply(sort scatter)");
  }
  if (rc != GRM_HIP_OK || a.segments == 0) return rc;
  hipLaunchKernelGGL(tile_list_kernel, dim3(static_cast<unsigned>(a.batch)), dim3(BK_THREADS), lds, s, a);
  return check_launch("gather_apply(tile list)");
}

int64_t offsets_bytes(int64_t batch, int64_t segments) { return (batch * (segments + 1) * 4 + 15) / 16 * 16; }

// Pair chunks per sequence for the multi-workgroup sort (1: one workgroup per sequence).
int64_t bucket_chunks(int64_t batch, int64_t n_index) {
  return n_index >= kMultiBucketPairs && batch <= 65535 ? (n_index + BK_ITEMS - 1) / BK_ITEMS : 1;
}

int64_t list_bytes(int64_t batch, int64_t n_index) { return (batch * n_index * 4 + 15) / 16 * 16; }

int64_t partial_bytes(int64_t batch, int64_t segments, int64_t n_index) {
  const int64_t c = bucket_chunks(batch, n_index);
  return c > 1 ? (batch * c * segments * 4 + 15) / 16 * 16 : 0;
}

// Pairs per apply work tile: the mean pairs per segment (at least 512, a
// multiple of the 64-pair MFMA tile), so balanced selections keep about one
// tile per segment and a heavily selected segment is split.
int64_t tile_pairs_for(int64_t segments, int64_t n_index) {
  const int64_t mean = segments > 0 ? (n_index + segments - 1) / segments : n_index;
  const int64_t tp = (mean + AP_N - 1) / AP_N * AP_N;
  return tp > 8 * AP_N ? tp : 8 * AP_N;
}

// Tiles per sequence at most: sum_s ceil(c_s / tp) <= n_index / tp + segments.
int64_t tiles_max(int64_t segments, int64_t n_index) {
  const int64_t tp = tile_pairs_for(segments, n_index);
  return (n_index + tp - 1) / tp + segments;
}

int64_t tiles_bytes(int64_t batch, int64_t segments, int64_t n_index) {
  return batch * tiles_max(segments, n_index) * 16 + (batch * 4 + 15) / 16 * 16 + offsets_bytes(batch, segments);
}

}  // namespace
}  // namespace grmhip

using namespace grmhip;

namespace grmhip {
namespace {

// The sort's workspace carve-up and the sizes, shared by gather_apply and
// retrieve_fuse (the workspace of grm_hip_gather_apply_workspace comes first).
void init_retrieve_args(RetrieveArgs& a, const void* memories, const int64_t* indices, const void* queries, void* out,
                        void* workspace, int64_t batch, int64_t segments, int64_t n_query, int64_t routes,
                        int64_t n_index, int64_t hidden_size, int64_t key_dim, int32_t* bad_index_count) {
  memset(&a, 0, sizeof(a));
  a.mem = memories;
  a.idx = indices;
  a.queries = queries;
  a.out = out;
  a.offsets = static_cast<int32_t*>(workspace);
  a.list = reinterpret_cast<int32_t*>(static_cast<unsigned char*>(workspace) + offsets_bytes(batch, segments));
  a.partial = reinterpret_cast<int32_t*>(static_cast<unsigned char*>(workspace) + offsets_bytes(batch, segments) +
                                         list_bytes(batch, n_index));
  a.bk_chunks = static_cast<int>(bucket_chunks(batch, n_index));
  {
    unsigned char* t0 = static_cast<unsigned char*>(workspace) + offsets_bytes(batch, segments) +
                        list_bytes(batch, n_index) + partial_bytes(batch, segments, n_index);
    a.tile_pairs = static_cast<int>(tile_pairs_for(segments, n_index));
    a.tb_max = static_cast<int>(tiles_max(segments, n_index));
    a.tiles = reinterpret_cast<int4*>(t0);
    t0 += batch * a.tb_max * 16;
    a.n_tiles = reinterpret_cast<int32_t*>(t0);
    t0 += (batch * 4 + 15) / 16 * 16;
    a.tile_base = reinterpret_cast<int32_t*>(t0);
  }
  a.bad = bad_index_count;
  a.batch = batch;
  a.segments = segments;
  a.n_query = n_query;
  a.routes = routes;
  a.n_index = n_index;
  a.dv = static_cast<int>(hidden_size);
  a.dk = static_cast<int>(key_dim);
  a.out_row = a.dv;
  a.v_tiles = static_cast<int>((hidden_size + AP_V - 1) / AP_V);
}

}  // namespace
}  // namespace grmhip

extern "C" int64_t grm_hip_gather_apply_workspace(int64_t batch, int64_t segments, int64_t n_index) {
  if (batch <= 0 || segments < 0 || n_index <= 0) return 0;
  return offsets_bytes(batch, segments) + list_bytes(batch, n_index) + partial_bytes(batch, segments, n_index) +
         tiles_bytes(batch, segments, n_index);
}

extern "C" int grm_hip_gather_apply(const void* memories, const int64_t* indices, const void* queries, void* out,
                                    void* workspace, int64_t workspace_bytes, int64_t batch, int64_t segments,
                                    int64_t n_query, int64_t routes, int64_t hidden_size, int64_t key_dim,
                                    int mem_dtype, int q_dtype, int out_dtype, int32_t* bad_index_count,
                                    void* stream) {
  if (batch < 0 || segments < 0 || n_query < 0 || routes < 0 || hidden_size < 0 || key_dim < 1) {
    set_error("gather_apply: negative size or key_dim < 1");
    return GRM_HIP_EINVAL;
  }
  if (mem_dtype < GRM_HIP_F32 || mem_dtype > GRM_HIP_BF16 || q_dtype < GRM_HIP_F32 || q_dtype > GRM_HIP_BF16) {
    set_error("gather_apply: unsupported dtypes mem=%d q=%d", mem_dtype, q_dtype);
    return GRM_HIP_EUNSUPPORTED;
  }
  if (out_dtype != mem_dtype && out_dtype != GRM_HIP_F32) {
    set_error("gather_apply: out_dtype %d must be the memories' dtype %d or float32", out_dtype, mem_dtype);
    return GRM_HIP_EINVAL;
  }
  if (key_dim > 128 || segments > kMaxSegments) {
    set_error("gather_apply: key_dim %lld > 128 or segments %lld > %lld", (long long)key_dim, (long long)segments,
              (long long)kMaxSegments);
    return GRM_HIP_EUNSUPPORTED;
  }
  const int64_t n_index = n_query * routes;
  if (batch == 0 || n_index == 0 || hidden_size == 0) return GRM_HIP_OK;
  if (n_index > INT32_MAX || hidden_size > INT32_MAX / 2 || batch > 65535 ||
      tiles_max(segments, n_index) * ((hidden_size + AP_V - 1) / AP_V) * AP_THREADS > UINT32_MAX) {
    set_error("gather_apply: sizes exceed one launch");
    return GRM_HIP_EINVAL;
  }
  if (indices == nullptr || queries == nullptr || out == nullptr || (segments > 0 && memories == nullptr)) {
    set_error("gather_apply: null pointer");
    return GRM_HIP_EINVAL;
  }
  const int64_t need = grm_hip_gather_apply_workspace(batch, segments, n_index);
  if (workspace == nullptr || workspace_bytes < need || reinterpret_cast<uintptr_t>(workspace) % 16 != 0) {
    set_error("gather_apply: workspace of %lld bytes (16-byte aligned) required", (long long)need);
    return GRM_HIP_EINVAL;
  }
  RetrieveArgs a;
  init_retrieve_args(a, memories, indices, queries, out, workspace, batch, segments, n_query, routes, n_index,
                     hidden_size, key_dim, bad_index_count);
  hipStream_t s = static_cast<hipStream_t>(stream);
  int rc;
  switch (out_dtype) {
    case GRM_HIP_F32: rc = launch_bucket<F32>(a, s); break;
    case GRM_HIP_F16: rc = launch_bucket<F16>(a, s); break;
    default: rc = launch_bucket<BF16>(a, s); break;
  }
  if (rc != GRM_HIP_OK || segments == 0) return rc;
  if (out_dtype == GRM_HIP_F32) {
    // float32 arithmetic and output; 16-bit memories are widened exactly on load
    switch (mem_dtype) {
      case GRM_HIP_F32: return dispatch_q<F32, F32>(a, q_dtype, s);
      case GRM_HIP_F16: return dispatch_q<F16, F32>(a, q_dtype, s);
      default: return dispatch_q<BF16, F32>(a, q_dtype, s);
    }
  }
  switch (mem_dtype) {
    case GRM_HIP_F16: return dispatch_q<F16, F16>(a, q_dtype, s);
    default: return dispatch_q<BF16, BF16>(a, q_dtype, s);
  }
}

namespace {

int64_t align16(int64_t n) { return (n + 15) / 16 * 16; }

}  // namespace

extern "C" int64_t grm_hip_retrieve_fuse_workspace(int64_t batch, int64_t segments, int64_t n_index,
                                                   int64_t value_dim) {
  if (batch <= 0 || segments < 0 || n_index <= 0 || value_dim <= 0) return 0;
  const int64_t tiles = (value_dim + AP_V - 1) / AP_V;
  return grm_hip_gather_apply_workspace(batch, segments, n_index) + align16(batch * n_index * value_dim * 2) +
         align16(batch * n_index * tiles * 4);
}

extern "C" int grm_hip_retrieve_fuse(const void* memories, const int64_t* indices, const void* queries,
                                     const float* gates, const void* h_online, const void* ln_weight,
                                     const void* ln_bias, void* out, void* workspace, int64_t workspace_bytes,
                                     int64_t batch, int64_t segments, int64_t n_query, int64_t routes,
                                     int64_t value_dim, int64_t key_dim, int mem_dtype, int q_dtype, int h_dtype,
                                     float eps, int32_t* bad_index_count, void* stream) {
  if (batch < 0 || segments < 0 || n_query < 0 || routes < 0 || value_dim < 0 || key_dim < 1) {
    set_error("retrieve_fuse: negative size or key_dim < 1");
    return GRM_HIP_EINVAL;
  }
  if (mem_dtype < GRM_HIP_F32 || mem_dtype > GRM_HIP_BF16 || q_dtype < GRM_HIP_F32 || q_dtype > GRM_HIP_BF16 ||
      h_dtype < GRM_HIP_F32 || h_dtype > GRM_HIP_BF16) {
    set_error("retrieve_fuse: unsupported dtypes mem=%d q=%d h=%d", mem_dtype, q_dtype, h_dtype);
    return GRM_HIP_EUNSUPPORTED;
  }
  if (key_dim > 128 || segments > kMaxSegments || value_dim % 8 != 0 || value_dim > 2048) {
    set_error("retrieve_fuse: needs key_dim <= 128, segments <= %lld, value_dim a multiple of 8 and <= 2048",
              (long long)kMaxSegments);
    return GRM_HIP_EUNSUPPORTED;
  }
  const int64_t rows = batch * n_query;
  const int64_t n_index = n_query * routes;
  if (rows == 0 || value_dim == 0) return GRM_HIP_OK;
  if (h_online == nullptr || out == nullptr || (n_index > 0 && (indices == nullptr || queries == nullptr ||
                                                                gates == nullptr)) ||
      (segments > 0 && memories == nullptr)) {
    set_error("retrieve_fuse: null pointer");
    return GRM_HIP_EINVAL;
  }
  if (n_index > INT32_MAX || batch > 65535 || routes * value_dim * 2 > INT32_MAX ||
      tiles_max(segments, n_index) * ((value_dim + AP_V - 1) / AP_V) * AP_THREADS > UINT32_MAX) {
    set_error("retrieve_fuse: sizes exceed one launch");
    return GRM_HIP_EINVAL;
  }
  const int64_t need = grm_hip_retrieve_fuse_workspace(batch, segments, n_index, value_dim);
  if (n_index > 0 &&
      (workspace == nullptr || workspace_bytes < need || reinterpret_cast<uintptr_t>(workspace) % 16 != 0)) {
    set_error("retrieve_fuse: workspace of %lld bytes (16-byte aligned) required", (long long)need);
    return GRM_HIP_EINVAL;
  }
  const int hb = h_dtype == GRM_HIP_F32 ? 4 : 2;
  if (reinterpret_cast<uintptr_t>(h_online) % 16 != 0 || reinterpret_cast<uintptr_t>(out) % 16 != 0 ||
      (ln_weight != nullptr && reinterpret_cast<uintptr_t>(ln_weight) % 16 != 0) ||
      (ln_bias != nullptr && reinterpret_cast<uintptr_t>(ln_bias) % 16 != 0) || (value_dim * hb) % 16 != 0) {
    set_error("retrieve_fuse: h_online, out and the LayerNorm parameters must be 16-byte aligned");
    return GRM_HIP_EUNSUPPORTED;
  }
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int v_tiles = static_cast<int>((value_dim + AP_V - 1) / AP_V);
  unsigned char* rows16 = nullptr;
  float* scales = nullptr;
  if (n_index > 0) {
    rows16 = static_cast<unsigned char*>(workspace) + grm_hip_gather_apply_workspace(batch, segments, n_index);
    scales = reinterpret_cast<float*>(rows16 + align16(batch * n_index * value_dim * 2));
    RetrieveArgs a;
    init_retrieve_args(a, memories, indices, queries, rows16, workspace, batch, segments, n_query, routes, n_index,
                       value_dim, key_dim, bad_index_count);
    a.gates = gates;
    a.scales = scales;
    if (!scaled_supported(a, mem_dtype, q_dtype)) {
      set_error("retrieve_fuse: needs bf16 queries (or f16 queries with f16 memories), 16-byte rows and "
                "16-byte aligned memories and queries");
      return GRM_HIP_EUNSUPPORTED;
    }
    int rc = launch_bucket<F16>(a, s);  // invalid pairs: zero rows and zero scales
    if (rc != GRM_HIP_OK) return rc;
    if (segments > 0) {
      switch (mem_dtype) {
        case GRM_HIP_F32: rc = apply_scaled_q<F32>(a, q_dtype, s); break;
        case GRM_HIP_F16: rc = apply_scaled_q<F16>(a, q_dtype, s); break;
        default: rc = apply_scaled_q<BF16>(a, q_dtype, s); break;
      }
      if (rc != GRM_HIP_OK) return rc;
    }
  }
  FuseScaledArgs f;
  f.h = h_online;
  f.rows = reinterpret_cast<const uint16_t*>(rows16);
  f.scales = scales;
  f.w = ln_weight;
  f.bias = ln_bias;
  f.out = out;
  f.n_rows = rows;
  f.routes = static_cast<int>(routes);
  f.hidden = static_cast<int>(value_dim);
  f.v_tiles = v_tiles;
  f.eps = eps;
  return fuse_scaled(f, h_dtype, s);
}

namespace {
int gather_apply_bwd_impl(const void* memories, const int64_t* indices, const float* grad_out, float* grad_pairs,
                          void* workspace, int64_t workspace_bytes, int64_t batch, int64_t segments, int64_t n_query,
                          int64_t routes, int64_t hidden_size, int64_t key_dim, int mem_dtype,
                          int32_t* bad_index_count, int token_rows, void* stream) {
  if (batch < 0 || segments < 0 || n_query < 0 || routes < 0 || hidden_size < 0 || key_dim < 1) {
    set_error("gather_apply_bwd: negative size or key_dim < 1");
    return GRM_HIP_EINVAL;
  }
  if (mem_dtype < GRM_HIP_F32 || mem_dtype > GRM_HIP_BF16) {
    set_error("gather_apply_bwd: unsupported memories dtype %d", mem_dtype);
    return GRM_HIP_EUNSUPPORTED;
  }
  const int64_t dkp = key_dim <= 16 ? 16 : key_dim <= 32 ? 32 : key_dim <= 64 ? 64 : 128;
  if (key_dim > 128 || segments > kMaxSegments || hidden_size > (1 << 20) ||
      apply_t_lds(static_cast<int>(hidden_size), static_cast<int>(dkp)) > 160 * 1024) {
    set_error("gather_apply_bwd: needs key_dim <= 128, segments <= %lld and the float32 state in LDS",
              (long long)kMaxSegments);
    return GRM_HIP_EUNSUPPORTED;
  }
  const int64_t n_index = n_query * routes;
  if (batch == 0 || n_index == 0 || key_dim == 0) return GRM_HIP_OK;
  if (n_index > INT32_MAX || batch > 65535 || tiles_max(segments, n_index) > UINT32_MAX) {
    set_error("gather_apply_bwd: sizes exceed one launch");
    return GRM_HIP_EINVAL;
  }
  if (indices == nullptr || grad_pairs == nullptr || (hidden_size > 0 && grad_out == nullptr) ||
      (segments > 0 && memories == nullptr)) {
    set_error("gather_apply_bwd: null pointer");
    return GRM_HIP_EINVAL;
  }
  const int64_t need = grm_hip_gather_apply_workspace(batch, segments, n_index);
  if (workspace == nullptr || workspace_bytes < need || reinterpret_cast<uintptr_t>(workspace) % 16 != 0 ||
      reinterpret_cast<uintptr_t>(grad_pairs) % 16 != 0) {
    set_error("gather_apply_bwd: workspace of %lld bytes and 16-byte aligned buffers required", (long long)need);
    return GRM_HIP_EINVAL;
  }
  RetrieveArgs a;
  init_retrieve_args(a, memories, indices, nullptr, grad_pairs, workspace, batch, segments, n_query, routes, n_index,
                     hidden_size, key_dim, bad_index_count);
  a.out_row = static_cast<int>(key_dim);  // invalid pairs: zero gradient rows
  hipStream_t s = static_cast<hipStream_t>(stream);
  int rc = launch_bucket<F32>(a, s);
  if (rc != GRM_HIP_OK || segments == 0) return rc;
  if (hidden_size == 0) {
    set_error("gather_apply_bwd: value_dim 0 with valid pairs");
    return GRM_HIP_EUNSUPPORTED;
  }
  switch (mem_dtype) {
    case GRM_HIP_F32: return dispatch_apply_t<F32>(a, grad_out, grad_pairs, token_rows, s);
    case GRM_HIP_F16: return dispatch_apply_t<F16>(a, grad_out, grad_pairs, token_rows, s);
    default: return dispatch_apply_t<BF16>(a, grad_out, grad_pairs, token_rows, s);
  }
}
}  // namespace

extern "C" int grm_hip_gather_apply_bwd_queries(const void* memories, const int64_t* indices, const float* grad_out,
                                                float* grad_pairs, void* workspace, int64_t workspace_bytes,
                                                int64_t batch, int64_t segments, int64_t n_query, int64_t routes,
                                                int64_t hidden_size, int64_t key_dim, int mem_dtype,
                                                int32_t* bad_index_count, void* stream) {
  return gather_apply_bwd_impl(memories, indices, grad_out, grad_pairs, workspace, workspace_bytes, batch, segments,
                               n_query, routes, hidden_size, key_dim, mem_dtype, bad_index_count, 0, stream);
}

extern "C" int grm_hip_gather_apply_bwd_tokens(const void* memories, const int64_t* indices, const float* grad_tokens,
                                               float* grad_pairs, void* workspace, int64_t workspace_bytes,
                                               int64_t batch, int64_t segments, int64_t n_query, int64_t routes,
                                               int64_t hidden_size, int64_t key_dim, int mem_dtype,
                                               int32_t* bad_index_count, void* stream) {
  return gather_apply_bwd_impl(memories, indices, grad_tokens, grad_pairs, workspace, workspace_bytes, batch, segments,
                               n_query, routes, hidden_size, key_dim, mem_dtype, bad_index_count, 1, stream);
}
