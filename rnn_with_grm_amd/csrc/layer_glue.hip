// Per-layer glue of the whole-sequence models, gfx950: the passes around the
// projection GEMM and after the layer's output, each one read and one write of
// the rows instead of a chain of elementwise launches.
//
//   project_split        the concatenated k | v | q | extra projection output of
//                        LinearMemoryCell.project (reference grm/core/paper_grm.py:
//                        491-493: key_proj / value_proj / query_proj, F.normalize of
//                        keys and queries; 570-574: the gating query projection) ->
//                        contiguous keys and queries L2-normalised, values and extra.
//   residual_layer_norm  LayerNorm(x + residual), SegmentRecurrentMemoryLayer's
//                        block output (grm/core/multilayer_grm.py:92-97).
//   archive_cast         float32 states rounded to the model dtype and then to the
//                        archive's storage dtype (push(), grm/core/paper_grm.py:
//                        139-140), one pass instead of two casts.
//
// Both follow the rounding of the torch ops they replace for 16-bit rows: the
// norm and its eps clamp are rounded to the row dtype before the division
// (F.normalize divides by a norm tensor of that dtype), and x + residual is
// rounded to the row dtype before the LayerNorm, whose statistics are float32.
// One wavefront per row, 16-byte accesses.
#include <stdint.h>
#include <string.h>

#include <algorithm>

#include "grm_hip.h"
#include "grm_hip_common.h"

namespace grmhip {
namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int GL_THREADS = 256;  // 4 rows per workgroup

template <class E>
__device__ __forceinline__ float round_to(float x) {
  return ET<E>::to_f(ET<E>::from_f(x));
}

// Eight elements at byte offset off of a buffer as float (zeros past its end).
template <class E>
__device__ __forceinline__ void ld8(__amdgpu_buffer_rsrc_t r, int off, float (&f)[8]) {
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
__device__ __forceinline__ void st8(__amdgpu_buffer_rsrc_t r, int off, const float (&y)[8]) {
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

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}

// N independent wave sums, one butterfly level for all of them at a time.
template <int N>
__device__ __forceinline__ void wave_sum_n(float (&v)[N]) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    float t[N];
#pragma unroll
    for (int i = 0; i < N; ++i) t[i] = __shfl_xor(v[i], off, 64);
#pragma unroll
    for (int i = 0; i < N; ++i) v[i] += t[i];
  }
}

struct SplitArgs {
  const void* proj;
  void* keys;
  void* values;
  void* queries;
  void* extra;
  int64_t rows;
  int dk, dv, de;  // multiples of 8
  float eps;
};

// One row segment [c0, c0 + n) of the projection row into out (n a multiple of 8),
// L2-normalised when NORM.
template <class E, bool NORM>
__device__ __forceinline__ void split_segment(const SplitArgs& a, int64_t row, int lane, int c0, int n, void* out) {
  using raw = typename ET<E>::raw;
  constexpr int ES = sizeof(raw);
  const int W = 2 * a.dk + a.dv + a.de;
  const __amdgpu_buffer_rsrc_t rs = make_rsrc(static_cast<const raw*>(a.proj) + row * W + c0, n * ES);
  const __amdgpu_buffer_rsrc_t rd = make_rsrc(static_cast<raw*>(out) + row * n, n * ES);
  const int units = n / 8;
  if constexpr (!NORM) {
    for (int u = lane; u < units; u += 64) {
      float x[8];
      ld8<E>(rs, u * 8 * ES, x);
      st8<E>(rd, u * 8 * ES, x);
    }
  } else {
    float ss = 0.f;
    for (int u = lane; u < units; u += 64) {
      float x[8];
      ld8<E>(rs, u * 8 * ES, x);
#pragma unroll
      for (int e = 0; e < 8; ++e) ss = fmaf(x[e], x[e], ss);
    }
    ss = wave_sum(ss);
    // x / clamp_min(||x||, eps) with the norm and the clamp in the row dtype
    const float den = round_to<E>(fmaxf(round_to<E>(sqrtf(ss)), a.eps));
    for (int u = lane; u < units; u += 64) {
      float x[8];
      ld8<E>(rs, u * 8 * ES, x);
#pragma unroll
      for (int e = 0; e < 8; ++e) x[e] = x[e] / den;
      st8<E>(rd, u * 8 * ES, x);
    }
  }
}

template <class E>
__global__ __launch_bounds__(GL_THREADS) void project_split_kernel(const SplitArgs a) {
  const int lane = threadIdx.x & 63;
  // (readfirstlane: the row is wave-uniform, and the compiler then knows it, so the row's
  // buffer resources stay scalar)
  const int64_t row = static_cast<int64_t>(blockIdx.x) * (GL_THREADS / 64) +
                      __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x) >> 6);
  if (row >= a.rows) return;  // wave-uniform
  split_segment<E, true>(a, row, lane, 0, a.dk, a.keys);
  split_segment<E, false>(a, row, lane, a.dk, a.dv, a.values);
  split_segment<E, true>(a, row, lane, a.dk + a.dv, a.dk, a.queries);
  if (a.de > 0) split_segment<E, false>(a, row, lane, 2 * a.dk + a.dv, a.de, a.extra);
}

struct ResLnArgs {
  const void* x;
  const void* res;
  const void* w;
  const void* b;
  void* out;
  int64_t rows;
  int hidden;  // multiple of 8, at most 64 * 8 * RLN_MAX
  float eps;
};

constexpr int RLN_MAX = 4;  // 16-byte units per lane: hidden <= 2048

template <class E, class P>
__global__ __launch_bounds__(GL_THREADS) void residual_layer_norm_kernel(const ResLnArgs a) {
  using raw = typename ET<E>::raw;
  using rawp = typename ET<P>::raw;
  constexpr int ES = sizeof(raw), PS = sizeof(rawp);
  const int lane = threadIdx.x & 63;
  // (readfirstlane: the row is wave-uniform, and the compiler then knows it, so the row's
  // buffer resources stay scalar)
  const int64_t row = static_cast<int64_t>(blockIdx.x) * (GL_THREADS / 64) +
                      __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x) >> 6);
  if (row >= a.rows) return;  // wave-uniform
  const int H = a.hidden, units = H / 8;
  const __amdgpu_buffer_rsrc_t rx = make_rsrc(static_cast<const raw*>(a.x) + row * H, H * ES);
  const __amdgpu_buffer_rsrc_t rr = make_rsrc(static_cast<const raw*>(a.res) + row * H, H * ES);
  float s[RLN_MAX][8];
  float sum = 0.f;
#pragma unroll
  for (int i = 0; i < RLN_MAX; ++i) {
    const int u = lane + 64 * i;
    const int off = u < units ? u * 8 * ES : kBufOOB;
    float xv[8], rv[8];
    ld8<E>(rx, off, xv);
    ld8<E>(rr, off, rv);
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      s[i][e] = round_to<E>(xv[e] + rv[e]);  // x + residual in the row dtype
      sum += s[i][e];
    }
  }
  const float mean = wave_sum(sum) / static_cast<float>(H);
  float var = 0.f;
#pragma unroll
  for (int i = 0; i < RLN_MAX; ++i) {
    const bool in = lane + 64 * i < units;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float d = s[i][e] - mean;
      var = in ? fmaf(d, d, var) : var;
    }
  }
  const float rstd = 1.0f / sqrtf(wave_sum(var) / static_cast<float>(H) + a.eps);
  const __amdgpu_buffer_rsrc_t rw = make_rsrc(a.w, a.w != nullptr ? H * PS : 0u);
  const __amdgpu_buffer_rsrc_t rb = make_rsrc(a.b, a.b != nullptr ? H * PS : 0u);
  const __amdgpu_buffer_rsrc_t ro = make_rsrc(static_cast<raw*>(a.out) + row * H, H * ES);
#pragma unroll
  for (int i = 0; i < RLN_MAX; ++i) {
    const int u = lane + 64 * i;
    if (u >= units) continue;
    float wv[8], bv[8], y[8];
    ld8<P>(rw, u * 8 * PS, wv);
    ld8<P>(rb, u * 8 * PS, bv);  // zeros without a bias
#pragma unroll
    for (int e = 0; e < 8; ++e) y[e] = (s[i][e] - mean) * rstd * (a.w != nullptr ? wv[e] : 1.f) + bv[e];
    st8<E>(ro, u * 8 * ES, y);
  }
}

bool aligned16(const void* p) { return reinterpret_cast<uintptr_t>(p) % 16 == 0; }

// The main loop of the two glue GEMMs, C = A W^T over a 512-thread workgroup's
// BM x BN tile (A: BM rows of K 16-bit values, W: BN rows of K): K in steps of
// 32, two LDS stages (64-byte rows whose four 16-byte granules are XOR-swizzled
// by bits 2-3 of the row, gl_at: both the staging writes, 16 consecutive
// granules per 16 lanes, and the fragment reads, 16 rows of one granule per
// 16 lanes, fall on 16 distinct 4-bank groups), and the global loads of step
// k + 2 issued while step k is multiplied, into one of two register slots, so
// a load has two steps of MFMAs to arrive.  Loads past K or past the tile's
// rows read zeros from the buffer resources (every step issues the same
// instructions, which keeps the compiler's load-wait counts exact).  One
// barrier per step: a stage is written one step after its last read.
// Wave w owns rows [wr0, + 16 TM) and columns [wc0, + 16 TN) of the tile as
// acc[ti][tj] (16x16x32 MFMA: lane (g, n), register r = row 16 ti + 4 g + r,
// column 16 tj + n).
constexpr int GL_BK = 32;
constexpr int GL_GEMM_THREADS = 512;

// Element offset of 16-byte granule j of row `row` in a staged tile.
__device__ __forceinline__ int gl_at(int row, int j) { return row * GL_BK + 8 * (j ^ ((row >> 2) & 3)); }

template <int BM, int BN>
struct GemmTile {
  static constexpr int UA = BM * (GL_BK / 8) / GL_GEMM_THREADS;  // 16-byte A units per thread per step
  static constexpr int UW = BN * (GL_BK / 8) / GL_GEMM_THREADS;
  static constexpr int STAGE = (BM + BN) * GL_BK;                // elements per LDS stage
  static_assert(UA * GL_GEMM_THREADS == BM * (GL_BK / 8) && UW * GL_GEMM_THREADS == BN * (GL_BK / 8),
                "tiles split evenly over the threads");
};

template <class E, int BM, int BN, int TM, int TN>
__device__ __forceinline__ void gemm_mainloop(typename ET<E>::raw* smem, __amdgpu_buffer_rsrc_t ra_rsrc,
                                              __amdgpu_buffer_rsrc_t rw_rsrc, int K, int w_rows, int wr0, int wc0,
                                              bool wave_on, f32x4 (&acc)[TM][TN]) {
  using raw = typename ET<E>::raw;
  using T = GemmTile<BM, BN>;
  const int tid = threadIdx.x, lane = tid & 63, g = lane >> 4, n = lane & 15;
  u32x4 ra[2][T::UA], rwv[2][T::UW];
  const int nk = K / GL_BK;
  auto gload = [&](int slot, int step) {
    const int k0 = step * GL_BK;
#pragma unroll
    for (int i = 0; i < T::UA; ++i) {
      const int u = tid + GL_GEMM_THREADS * i;
      const int off = k0 < K ? ((u >> 2) * K + k0 + 8 * (u & 3)) * 2 : kBufOOB;
      ra[slot][i] = __builtin_amdgcn_raw_buffer_load_b128(ra_rsrc, off, 0, 0);
    }
#pragma unroll
    for (int i = 0; i < T::UW; ++i) {
      const int u = tid + GL_GEMM_THREADS * i;
      const int row = u >> 2;
      const int off = (k0 < K && row < w_rows) ? (row * K + k0 + 8 * (u & 3)) * 2 : kBufOOB;
      rwv[slot][i] = __builtin_amdgcn_raw_buffer_load_b128(rw_rsrc, off, 0, 0);
    }
  };
  auto sstore = [&](int slot, int stage) {
    raw* As = smem + stage * T::STAGE;
    raw* Ws = As + BM * GL_BK;
#pragma unroll
    for (int i = 0; i < T::UA; ++i) {
      const int u = tid + GL_GEMM_THREADS * i;
      *reinterpret_cast<u32x4*>(As + gl_at(u >> 2, u & 3)) = ra[slot][i];
    }
#pragma unroll
    for (int i = 0; i < T::UW; ++i) {
      const int u = tid + GL_GEMM_THREADS * i;
      *reinterpret_cast<u32x4*>(Ws + gl_at(u >> 2, u & 3)) = rwv[slot][i];
    }
  };
  auto compute = [&](int stage) {
    if (!wave_on) return;
    const raw* As = smem + stage * T::STAGE;
    const raw* Ws = As + BM * GL_BK;
    Frag8<E> af[TM], bf[TN];
#pragma unroll
    for (int ti = 0; ti < TM; ++ti)
      af[ti] = __builtin_bit_cast(Frag8<E>, *reinterpret_cast<const u32x4*>(As + gl_at(wr0 + 16 * ti + n, g)));
#pragma unroll
    for (int tj = 0; tj < TN; ++tj)
      bf[tj] = __builtin_bit_cast(Frag8<E>, *reinterpret_cast<const u32x4*>(Ws + gl_at(wc0 + 16 * tj + n, g)));
#pragma unroll
    for (int ti = 0; ti < TM; ++ti)
#pragma unroll
      for (int tj = 0; tj < TN; ++tj) acc[ti][tj] = mfma8(af[ti], bf[tj], acc[ti][tj]);
  };
#pragma unroll
  for (int ti = 0; ti < TM; ++ti)
#pragma unroll
    for (int tj = 0; tj < TN; ++tj) acc[ti][tj] = f32x4{0.f, 0.f, 0.f, 0.f};
  gload(0, 0);
  gload(1, 1);
  sstore(0, 0);
  __syncthreads();
  for (int k = 0; k < nk; k += 2) {
    gload(0, k + 2);  // slot 0 was staged at the end of the previous step
    compute(0);       // step k
    sstore(1, 1);     // step k + 1 (zeros past K)
    __syncthreads();
    if (k + 1 >= nk) break;
    gload(1, k + 3);
    compute(1);                 // step k + 1
    sstore(0, 0);               // step k + 2
    __syncthreads();
  }
}

// project_gemm: LinearMemoryCell.project's GEMM (the concatenated k | v | q | extra
// projection, reference grm/core/paper_grm.py:491-493, 570-574) with project_split
// as its epilogue.  Y = X W^T + bias on 16x16x32 MFMA, 128 x 256 output tiles,
// on gemm_mainloop.  Eight waves: wave w owns rows [m0 + 64 (w >> 2), + 64) and
// columns [n0 + 64 (w & 3), + 64); at key_dim 64 a key or query block is one
// wave's columns, so its row norms need no other wave.  Epilogue: Y + bias
// rounded to the model dtype (F.linear's output), keys and queries
// L2-normalised with project_split's roundings, every part written contiguous
// through an LDS transpose (16-byte row stores).
constexpr int PG_BM = 128, PG_BN = 256, PG_THREADS = GL_GEMM_THREADS;

struct GemmArgs {
  const void* x;
  const void* w;
  const void* bias;
  void* keys;
  void* values;
  void* queries;
  void* extra;
  int64_t rows;
  int K;
  int dk, dv, de;  // dk == 64; dv, de multiples of 64
  float eps;
};

template <class E>
__global__ __launch_bounds__(PG_THREADS) void project_gemm_kernel(const GemmArgs a) {
  using raw = typename ET<E>::raw;
  static_assert(sizeof(raw) == 2, "16-bit inputs");
  // The two LDS stages; afterwards the epilogue's staging (8 waves x 4 KB).
  __shared__ __align__(16) raw smem[2 * GemmTile<PG_BM, PG_BN>::STAGE];
  const int tid = threadIdx.x, lane = tid & 63, g = lane >> 4, n = lane & 15;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int N = 2 * a.dk + a.dv + a.de;
  const int K = a.K;
  const int64_t m0 = static_cast<int64_t>(blockIdx.x) * PG_BM;
  const int n0 = static_cast<int>(blockIdx.y) * PG_BN;
  const int wr = w >> 2;              // row half
  const int c0 = n0 + 64 * (w & 3);  // this wave's first column
  const bool wave_on = c0 < N;
  const __amdgpu_buffer_rsrc_t rx =
      make_rsrc(static_cast<const raw*>(a.x) + m0 * K, static_cast<uint32_t>(min_i64(a.rows - m0, PG_BM) * K * 2));
  const __amdgpu_buffer_rsrc_t rw =
      make_rsrc(static_cast<const raw*>(a.w) + static_cast<int64_t>(n0) * K,
                static_cast<uint32_t>(static_cast<int64_t>(min(N - n0, PG_BN)) * K * 2));
  f32x4 acc[4][4];
  gemm_mainloop<E, PG_BM, PG_BN, 4, 4>(smem, rx, rw, K, min(N - n0, PG_BN), 64 * wr, 64 * (w & 3), wave_on, acc);
  if (!wave_on) return;  // (the main loop ends on a barrier: every wave is done with the stages)
  // acc[ti][tj][r]: row m0 + 64 wr + 16 ti + 4 g + r, column c0 + 16 tj + n.  Y + bias in the
  // model dtype, as F.linear returns it.
  float bcol[4];
#pragma unroll
  for (int tj = 0; tj < 4; ++tj)
    bcol[tj] = a.bias != nullptr ? ET<E>::to_f(static_cast<const raw*>(a.bias)[c0 + 16 * tj + n]) : 0.f;
#pragma unroll
  for (int ti = 0; ti < 4; ++ti)
#pragma unroll
    for (int tj = 0; tj < 4; ++tj)
#pragma unroll
      for (int r = 0; r < 4; ++r) acc[ti][tj][r] = round_to<E>(acc[ti][tj][r] + bcol[tj]);
  const int dk = a.dk, dv = a.dv, de = a.de;
  void* out;
  int col, ld;
  bool norm = false;
  if (c0 < dk) {
    out = a.keys; col = c0; ld = dk; norm = true;
  } else if (c0 < dk + dv) {
    out = a.values; col = c0 - dk; ld = dv;
  } else if (c0 < 2 * dk + dv) {
    out = a.queries; col = c0 - dk - dv; ld = dk; norm = true;
  } else {
    out = a.extra; col = c0 - 2 * dk - dv; ld = de;
  }
  if (norm) {
    // x / clamp_min(||x||, eps), the norm and the clamp rounded to the row dtype; the 16
    // rows' sums over the 16 lanes of a column group run together (one butterfly level
    // for all of them at a time)
    float ss[16];
#pragma unroll
    for (int ti = 0; ti < 4; ++ti)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        ss[4 * ti + r] = 0.f;
#pragma unroll
        for (int tj = 0; tj < 4; ++tj) ss[4 * ti + r] = fmaf(acc[ti][tj][r], acc[ti][tj][r], ss[4 * ti + r]);
      }
#pragma unroll
    for (int off = 1; off < 16; off <<= 1) {
      float t[16];
#pragma unroll
      for (int i = 0; i < 16; ++i) t[i] = __shfl_xor(ss[i], off, 64);
#pragma unroll
      for (int i = 0; i < 16; ++i) ss[i] += t[i];
    }
#pragma unroll
    for (int ti = 0; ti < 4; ++ti)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const float inv = 1.0f / round_to<E>(fmaxf(round_to<E>(sqrtf(ss[4 * ti + r])), a.eps));
#pragma unroll
        for (int tj = 0; tj < 4; ++tj) acc[ti][tj][r] = acc[ti][tj][r] * inv;
      }
  }
  // Two halves of 32 rows through this wave's 4 KB of LDS, then 16-byte row stores.
  raw* st = smem + w * 32 * 64;
  static_assert(sizeof(smem) >= 8 * 32 * 64 * sizeof(raw), "staging fits");
  raw* ob = static_cast<raw*>(out);
#pragma unroll
  for (int h = 0; h < 2; ++h) {
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int tj = 0; tj < 4; ++tj)
#pragma unroll
        for (int r = 0; r < 4; ++r)
          st[(16 * t + 4 * g + r) * 64 + 16 * tj + n] = ET<E>::from_f(acc[2 * h + t][tj][r]);
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int u = lane + 64 * i;
      const int rr = u >> 3, cu = 8 * (u & 7);
      const int64_t row = m0 + 64 * wr + 32 * h + rr;
      if (row < a.rows)
        *reinterpret_cast<u32x4*>(ob + row * ld + col + cu) = *reinterpret_cast<const u32x4*>(st + rr * 64 + cu);
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  }
}

// linear_residual_layer_norm: SegmentRecurrentMemoryModel's output projection
// (reference grm/core/paper_grm.py:709, y = output_proj(h)) and the block output
// of SegmentRecurrentMemoryLayer (grm/core/multilayer_grm.py:92-97,
// layer_norm(y + x)) in one kernel: the GEMM's epilogue is the residual add and
// the LayerNorm, so y never goes to HBM.  A workgroup owns 128 whole rows
// (every output column, N <= 512), so the LayerNorm's row statistics stay
// inside it; wave w owns the 128 x 64 block at columns [64 w, + 64), on
// gemm_mainloop.  Epilogue: y + bias rounded to the model dtype (F.linear's
// output) into LDS, the residual rows of each wave loaded meanwhile; then each
// wave walks its 16 rows: s = y + x rounded to the model dtype (the torch add),
// mean and variance in float32 (two passes), (s - mean) rstd w + b.  On
// request it also writes s, mean and rstd, the saved tensors of LayerNorm's
// backward (aten native_layer_norm).
constexpr int OL_BM = 128, OL_MAXN = 512, OL_THREADS = GL_GEMM_THREADS;
constexpr int OL_YS = OL_MAXN + 8;  // LDS row stride of the y tile, elements
constexpr int OL_RPW = OL_BM / 8;   // rows per wave in the row pass
constexpr int OL_RB = 8;            // rows whose reductions run together

struct OutLnArgs {
  const void* h;     // [rows, K]
  const void* w;     // [N, K]
  const void* bias;  // [N] or null
  const void* res;   // [rows, N]
  const void* ln_w;  // [N] or null
  const void* ln_b;  // [N] or null
  void* out;         // [rows, N]
  void* pre;         // [rows, N] or null: y + x, the LayerNorm input
  float* mean;       // [rows] or null
  float* rstd;       // [rows] or null
  int64_t rows;
  int K, N;
  float eps;
};

template <class E, class P, bool FULL>
__global__ __launch_bounds__(OL_THREADS) void out_ln_kernel(const OutLnArgs a) {
  using raw = typename ET<E>::raw;
  using rawp = typename ET<P>::raw;
  static_assert(sizeof(raw) == 2, "16-bit inputs");
  constexpr int PSZ = sizeof(rawp);
  constexpr int STAGES = 2 * GemmTile<OL_BM, OL_MAXN>::STAGE;
  __shared__ __align__(16) raw smem[STAGES > OL_BM * OL_YS ? STAGES : OL_BM * OL_YS];
  const int tid = threadIdx.x, lane = tid & 63, g = lane >> 4, n = lane & 15;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int N = a.N, K = a.K;
  const int64_t m0 = static_cast<int64_t>(blockIdx.x) * OL_BM;
  const int c0 = 64 * w;
  const bool wave_on = c0 < N;
  const int tile_rows = static_cast<int>(min_i64(a.rows - m0, OL_BM));
  const __amdgpu_buffer_rsrc_t rx = make_rsrc(static_cast<const raw*>(a.h) + m0 * K,
                                              static_cast<uint32_t>(tile_rows * K * 2));
  const __amdgpu_buffer_rsrc_t rw = make_rsrc(a.w, static_cast<uint32_t>(static_cast<int64_t>(N) * K * 2));
  f32x4 acc[8][4];
  gemm_mainloop<E, OL_BM, OL_MAXN, 8, 4>(smem, rx, rw, K, N, 0, c0, wave_on, acc);
  // (the main loop ends on a barrier: the stages become the y tile)
  raw* const Y = smem;
  if (wave_on) {
    // acc[ti][tj][r]: row 16 ti + 4 g + r, column c0 + 16 tj + n
#pragma unroll
    for (int tj = 0; tj < 4; ++tj) {
      const int col = c0 + 16 * tj + n;
      const float bcol = a.bias != nullptr ? ET<E>::to_f(static_cast<const raw*>(a.bias)[col]) : 0.f;
#pragma unroll
      for (int ti = 0; ti < 8; ++ti)
#pragma unroll
        for (int r = 0; r < 4; ++r) Y[(16 * ti + 4 * g + r) * OL_YS + col] = ET<E>::from_f(acc[ti][tj][r] + bcol);
    }
  }
  // Row pass: wave w takes rows OL_RPW w .. + OL_RPW; lane l holds columns 8 l .. 8 l + 7.  The
  // residual rows are loaded before the barrier, so their latency overlaps it.
  const bool lane_on = FULL || 8 * lane < N;  // FULL: N == OL_MAXN, every lane holds 8 columns
  const __amdgpu_buffer_rsrc_t rres = make_rsrc(static_cast<const raw*>(a.res) + m0 * N,
                                                static_cast<uint32_t>(tile_rows * N * 2));
  u32x4 xr[OL_RPW];
#pragma unroll
  for (int rr = 0; rr < OL_RPW; ++rr) {
    const int row = OL_RPW * w + rr;
    xr[rr] = __builtin_amdgcn_raw_buffer_load_b128(rres, lane_on ? (row * N + 8 * lane) * 2 : kBufOOB, 0, 0);
  }
  const __amdgpu_buffer_rsrc_t rlw = make_rsrc(a.ln_w, a.ln_w != nullptr ? N * PSZ : 0u);
  const __amdgpu_buffer_rsrc_t rlb = make_rsrc(a.ln_b, a.ln_b != nullptr ? N * PSZ : 0u);
  float wv[8], bv[8];
  ld8<P>(rlw, lane_on ? 8 * lane * PSZ : kBufOOB, wv);
  ld8<P>(rlb, lane_on ? 8 * lane * PSZ : kBufOOB, bv);  // zeros without a bias
  if (a.ln_w == nullptr) {
#pragma unroll
    for (int e = 0; e < 8; ++e) wv[e] = 1.f;  // no affine map
  }
  __syncthreads();
  const __amdgpu_buffer_rsrc_t ro = make_rsrc(static_cast<raw*>(a.out) + m0 * N,
                                              static_cast<uint32_t>(tile_rows * N * 2));
  const __amdgpu_buffer_rsrc_t rp = make_rsrc(static_cast<raw*>(a.pre) + (a.pre != nullptr ? m0 * N : 0),
                                              a.pre != nullptr ? static_cast<uint32_t>(tile_rows * N * 2) : 0u);
  // OL_RB rows at a time: their cross-lane sums run together, so the shuffles' LDS
  // latencies overlap instead of adding up row after row.  Rows past the tile
  // compute on zeros and store nothing (their offsets are out of the resources).
  const float inv_n = 1.0f / static_cast<float>(N);
#pragma unroll
  for (int r0 = 0; r0 < OL_RPW; r0 += OL_RB) {
    float s[OL_RB][8], red[OL_RB];
#pragma unroll
    for (int q = 0; q < OL_RB; ++q) {
      const int row = OL_RPW * w + r0 + q;
      const U8<E> xv = __builtin_bit_cast(U8<E>, xr[r0 + q]);
      const U8<E> yv = __builtin_bit_cast(
          U8<E>, *reinterpret_cast<const u32x4*>(Y + row * OL_YS + (lane_on ? 8 * lane : 0)));
      red[q] = 0.f;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float v = round_to<E>(ET<E>::to_f(yv.e[e]) + ET<E>::to_f(xv.e[e]));  // y + x in the row dtype
        s[q][e] = FULL ? v : (lane_on ? v : 0.f);
        red[q] += s[q][e];
      }
    }
    wave_sum_n(red);
    float mean[OL_RB];
#pragma unroll
    for (int q = 0; q < OL_RB; ++q) {
      mean[q] = red[q] * inv_n;
      red[q] = 0.f;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float d = s[q][e] - mean[q];
        red[q] = (FULL || lane_on) ? fmaf(d, d, red[q]) : red[q];
      }
    }
    wave_sum_n(red);
#pragma unroll
    for (int q = 0; q < OL_RB; ++q) {
      const int row = OL_RPW * w + r0 + q;
      const float rstd = 1.0f / sqrtf(red[q] * inv_n + a.eps);
      float y[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) y[e] = fmaf((s[q][e] - mean[q]) * rstd, wv[e], bv[e]);
      const int off = (lane_on && row < tile_rows) ? (row * N + 8 * lane) * 2 : kBufOOB;
      st8<E>(ro, off, y);
      if (a.pre != nullptr) st8<E>(rp, off, s[q]);
      if (lane == 0 && a.mean != nullptr && row < tile_rows) {
        a.mean[m0 + row] = mean[q];
        a.rstd[m0 + row] = rstd;
      }
    }
  }
}

// archive_cast: float32 states in the form the archive stores them, rounded
// to the model dtype and then to the storage dtype, as push() stores a state
// the model computed (reference grm/core/paper_grm.py:139-140: the state in
// the model's dtype, then memory_storage_dtype).  One read, one write.
template <class M, class St>
__global__ __launch_bounds__(GL_THREADS) void archive_cast_kernel(const float* __restrict__ src,
                                                                  typename ET<St>::raw* __restrict__ dst,
                                                                  int64_t n) {
  using raw = typename ET<St>::raw;
  auto cvt = [](float f) -> raw { return ET<St>::from_f(ET<M>::to_f(ET<M>::from_f(f))); };
  const int64_t n8 = n / 8;
  const int64_t stride = static_cast<int64_t>(gridDim.x) * GL_THREADS;
  const int64_t t0 = static_cast<int64_t>(blockIdx.x) * GL_THREADS + threadIdx.x;
  for (int64_t i = t0; i < n8; i += stride) {
    const float4 a = reinterpret_cast<const float4*>(src)[2 * i];
    const float4 b = reinterpret_cast<const float4*>(src)[2 * i + 1];
    const float f[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
    if constexpr (sizeof(raw) == 2) {
      raw r[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) r[e] = cvt(f[e]);
      reinterpret_cast<uint4*>(dst)[i] = __builtin_bit_cast(uint4, r);
    } else {
      reinterpret_cast<float4*>(dst)[2 * i] = make_float4(cvt(f[0]), cvt(f[1]), cvt(f[2]), cvt(f[3]));
      reinterpret_cast<float4*>(dst)[2 * i + 1] = make_float4(cvt(f[4]), cvt(f[5]), cvt(f[6]), cvt(f[7]));
    }
  }
  for (int64_t i = 8 * n8 + t0; i < n; i += stride) dst[i] = cvt(src[i]);
}

}  // namespace
}  // namespace grmhip

using namespace grmhip;

extern "C" int grm_hip_project_split(const void* proj, void* keys, void* values, void* queries, void* extra,
                                     int64_t rows, int64_t key_dim, int64_t value_dim, int64_t extra_dim,
                                     int dtype, float eps, void* stream) {
  if (rows < 0 || key_dim < 0 || value_dim < 0 || extra_dim < 0) {
    set_error("project_split: negative size");
    return GRM_HIP_EINVAL;
  }
  if (dtype < GRM_HIP_F32 || dtype > GRM_HIP_BF16) {
    set_error("project_split: unsupported dtype %d", dtype);
    return GRM_HIP_EUNSUPPORTED;
  }
  if (key_dim % 8 || value_dim % 8 || extra_dim % 8) {
    set_error("project_split: key_dim, value_dim and extra_dim must be multiples of 8");
    return GRM_HIP_EUNSUPPORTED;
  }
  const int eb = dtype == GRM_HIP_F32 ? 4 : 2;
  if ((2 * key_dim + value_dim + extra_dim) * eb > INT32_MAX / 2) {
    set_error("project_split: rows too wide");
    return GRM_HIP_EINVAL;
  }
  if (rows == 0) return GRM_HIP_OK;
  if (proj == nullptr || keys == nullptr || values == nullptr || queries == nullptr ||
      (extra_dim > 0 && extra == nullptr)) {
    set_error("project_split: null pointer");
    return GRM_HIP_EINVAL;
  }
  if (!aligned16(proj) || !aligned16(keys) || !aligned16(values) || !aligned16(queries) ||
      (extra_dim > 0 && !aligned16(extra))) {
    set_error("project_split: buffers must be 16-byte aligned");
    return GRM_HIP_EUNSUPPORTED;
  }
  SplitArgs a;
  a.proj = proj;
  a.keys = keys;
  a.values = values;
  a.queries = queries;
  a.extra = extra;
  a.rows = rows;
  a.dk = static_cast<int>(key_dim);
  a.dv = static_cast<int>(value_dim);
  a.de = static_cast<int>(extra_dim);
  a.eps = eps;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const dim3 grid(static_cast<unsigned>((rows + GL_THREADS / 64 - 1) / (GL_THREADS / 64)));
  switch (dtype) {
    case GRM_HIP_F32: hipLaunchKernelGGL(project_split_kernel<F32>, grid, dim3(GL_THREADS), 0, s, a); break;
    case GRM_HIP_F16: hipLaunchKernelGGL(project_split_kernel<F16>, grid, dim3(GL_THREADS), 0, s, a); break;
    default: hipLaunchKernelGGL(project_split_kernel<BF16>, grid, dim3(GL_THREADS), 0, s, a); break;
  }
  return check_launch("project_split");
}

extern "C" int grm_hip_residual_layer_norm(const void* x, const void* residual, const void* weight,
                                           const void* bias, void* out, int64_t rows, int64_t hidden_size,
                                           int dtype, int param_dtype, float eps, void* stream) {
  if (rows < 0 || hidden_size < 0) {
    set_error("residual_layer_norm: negative size");
    return GRM_HIP_EINVAL;
  }
  if (dtype < GRM_HIP_F32 || dtype > GRM_HIP_BF16 || param_dtype < GRM_HIP_F32 || param_dtype > GRM_HIP_BF16) {
    set_error("residual_layer_norm: unsupported dtypes %d / %d", dtype, param_dtype);
    return GRM_HIP_EUNSUPPORTED;
  }
  if (hidden_size % 8 || hidden_size > 64 * 8 * RLN_MAX) {
    set_error("residual_layer_norm: hidden_size must be a multiple of 8 and at most %d", 64 * 8 * RLN_MAX);
    return GRM_HIP_EUNSUPPORTED;
  }
  if (rows == 0 || hidden_size == 0) return GRM_HIP_OK;
  if (x == nullptr || residual == nullptr || out == nullptr || (bias != nullptr && weight == nullptr)) {
    set_error("residual_layer_norm: null pointer (a bias needs a weight)");
    return GRM_HIP_EINVAL;
  }
  if (!aligned16(x) || !aligned16(residual) || !aligned16(out) || (weight != nullptr && !aligned16(weight)) ||
      (bias != nullptr && !aligned16(bias))) {
    set_error("residual_layer_norm: buffers must be 16-byte aligned");
    return GRM_HIP_EUNSUPPORTED;
  }
  ResLnArgs a;
  a.x = x;
  a.res = residual;
  a.w = weight;
  a.b = bias;
  a.out = out;
  a.rows = rows;
  a.hidden = static_cast<int>(hidden_size);
  a.eps = eps;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const dim3 grid(static_cast<unsigned>((rows + GL_THREADS / 64 - 1) / (GL_THREADS / 64)));
  auto go = [&](auto et) {
    using E = decltype(et);
    switch (param_dtype) {
      case GRM_HIP_F32:
        hipLaunchKernelGGL((residual_layer_norm_kernel<E, F32>), grid, dim3(GL_THREADS), 0, s, a);
        break;
      case GRM_HIP_F16:
        hipLaunchKernelGGL((residual_layer_norm_kernel<E, F16>), grid, dim3(GL_THREADS), 0, s, a);
        break;
      default:
        hipLaunchKernelGGL((residual_layer_norm_kernel<E, BF16>), grid, dim3(GL_THREADS), 0, s, a);
        break;
    }
  };
  switch (dtype) {
    case GRM_HIP_F32: go(F32{}); break;
    case GRM_HIP_F16: go(F16{}); break;
    default: go(BF16{}); break;
  }
  return check_launch("residual_layer_norm");
}

extern "C" int grm_hip_archive_cast(const float* states, void* out, int64_t n, int model_dtype, int storage_dtype,
                                    void* stream) {
  if (n < 0) {
    set_error("archive_cast: negative size");
    return GRM_HIP_EINVAL;
  }
  if (model_dtype < GRM_HIP_F32 || model_dtype > GRM_HIP_BF16 || storage_dtype < GRM_HIP_F32 ||
      storage_dtype > GRM_HIP_BF16) {
    set_error("archive_cast: unsupported dtypes %d / %d", model_dtype, storage_dtype);
    return GRM_HIP_EUNSUPPORTED;
  }
  if (n == 0) return GRM_HIP_OK;
  if (states == nullptr || out == nullptr) {
    set_error("archive_cast: null pointer");
    return GRM_HIP_EINVAL;
  }
  if (!aligned16(states) || !aligned16(out)) {
    set_error("archive_cast: buffers must be 16-byte aligned");
    return GRM_HIP_EUNSUPPORTED;
  }
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int64_t groups = (n + 7) / 8;
  const dim3 grid(static_cast<unsigned>(std::min<int64_t>((groups + GL_THREADS - 1) / GL_THREADS, 4096)));
  auto go = [&](auto mt) {
    using M = decltype(mt);
    switch (storage_dtype) {
      case GRM_HIP_F32:
        hipLaunchKernelGGL((archive_cast_kernel<M, F32>), grid, dim3(GL_THREADS), 0, s, states,
                           static_cast<float*>(out), n);
        break;
      case GRM_HIP_F16:
        hipLaunchKernelGGL((archive_cast_kernel<M, F16>), grid, dim3(GL_THREADS), 0, s, states,
                           static_cast<uint16_t*>(out), n);
        break;
      default:
        hipLaunchKernelGGL((archive_cast_kernel<M, BF16>), grid, dim3(GL_THREADS), 0, s, states,
                           static_cast<uint16_t*>(out), n);
        break;
    }
  };
  switch (model_dtype) {
    case GRM_HIP_F32: go(F32{}); break;
    case GRM_HIP_F16: go(F16{}); break;
    default: go(BF16{}); break;
  }
  return check_launch("archive_cast");
}

extern "C" int grm_hip_project_gemm(const void* x, const void* weight, const void* bias, void* keys, void* values,
                                    void* queries, void* extra, int64_t rows, int64_t in_dim, int64_t key_dim,
                                    int64_t value_dim, int64_t extra_dim, int dtype, float eps, void* stream) {
  if (rows < 0 || in_dim < 0 || key_dim < 0 || value_dim < 0 || extra_dim < 0) {
    set_error("project_gemm: negative size");
    return GRM_HIP_EINVAL;
  }
  if (dtype != GRM_HIP_F16 && dtype != GRM_HIP_BF16) {
    set_error("project_gemm: 16-bit inputs only (dtype %d)", dtype);
    return GRM_HIP_EUNSUPPORTED;
  }
  const int64_t N = 2 * key_dim + value_dim + extra_dim;
  if (key_dim != 64 || value_dim % 64 || extra_dim % 64 || in_dim % GL_BK || in_dim == 0 ||
      rows * in_dim * 2 > INT32_MAX || static_cast<int64_t>(PG_BN) * in_dim * 2 > INT32_MAX ||
      N * in_dim * 2 > INT32_MAX || (rows + PG_BM - 1) / PG_BM > INT32_MAX) {
    set_error("project_gemm: needs key_dim 64, value_dim and extra_dim multiples of 64, in_dim a multiple of %d, "
              "and operands under 2 GiB",
              GL_BK);
    return GRM_HIP_EUNSUPPORTED;
  }
  if (rows == 0) return GRM_HIP_OK;
  if (x == nullptr || weight == nullptr || keys == nullptr || values == nullptr || queries == nullptr ||
      (extra_dim > 0 && extra == nullptr)) {
    set_error("project_gemm: null pointer");
    return GRM_HIP_EINVAL;
  }
  if (!aligned16(x) || !aligned16(weight) || !aligned16(keys) || !aligned16(values) || !aligned16(queries) ||
      (extra_dim > 0 && !aligned16(extra))) {
    set_error("project_gemm: buffers must be 16-byte aligned");
    return GRM_HIP_EUNSUPPORTED;
  }
  GemmArgs a;
  a.x = x;
  a.w = weight;
  a.bias = bias;
  a.keys = keys;
  a.values = values;
  a.queries = queries;
  a.extra = extra;
  a.rows = rows;
  a.K = static_cast<int>(in_dim);
  a.dk = static_cast<int>(key_dim);
  a.dv = static_cast<int>(value_dim);
  a.de = static_cast<int>(extra_dim);
  a.eps = eps;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const dim3 grid(static_cast<unsigned>((rows + PG_BM - 1) / PG_BM), static_cast<unsigned>((N + PG_BN - 1) / PG_BN));
  if (dtype == GRM_HIP_F16) {
    hipLaunchKernelGGL(project_gemm_kernel<F16>, grid, dim3(PG_THREADS), 0, s, a);
  } else {
    hipLaunchKernelGGL(project_gemm_kernel<BF16>, grid, dim3(PG_THREADS), 0, s, a);
  }
  return check_launch("project_gemm");
}

extern "C" int grm_hip_linear_residual_layer_norm(const void* x, const void* weight, const void* bias,
                                                  const void* residual, const void* ln_weight, const void* ln_bias,
                                                  void* out, void* pre, float* mean, float* rstd, int64_t rows,
                                                  int64_t in_dim, int64_t out_dim, int dtype, int param_dtype,
                                                  float eps, void* stream) {
  if (rows < 0 || in_dim < 0 || out_dim < 0) {
    set_error("linear_residual_layer_norm: negative size");
    return GRM_HIP_EINVAL;
  }
  if ((dtype != GRM_HIP_F16 && dtype != GRM_HIP_BF16) || param_dtype < GRM_HIP_F32 || param_dtype > GRM_HIP_BF16) {
    set_error("linear_residual_layer_norm: 16-bit inputs only (dtype %d, param_dtype %d)", dtype, param_dtype);
    return GRM_HIP_EUNSUPPORTED;
  }
  if (in_dim % GL_BK || in_dim == 0 || out_dim % 64 || out_dim == 0 || out_dim > OL_MAXN ||
      out_dim * in_dim * 2 > INT32_MAX || static_cast<int64_t>(OL_BM) * in_dim * 2 > INT32_MAX ||
      (rows + OL_BM - 1) / OL_BM > INT32_MAX) {
    set_error("linear_residual_layer_norm: needs in_dim a positive multiple of %d, out_dim a positive multiple of "
              "64 and at most %d, and the weight under 2 GiB", GL_BK, OL_MAXN);
    return GRM_HIP_EUNSUPPORTED;
  }
  if (rows == 0) return GRM_HIP_OK;
  if (x == nullptr || weight == nullptr || residual == nullptr || out == nullptr ||
      (ln_bias != nullptr && ln_weight == nullptr) || ((mean == nullptr) != (rstd == nullptr))) {
    set_error("linear_residual_layer_norm: null pointer (an ln_bias needs an ln_weight, mean and rstd go together)");
    return GRM_HIP_EINVAL;
  }
  if (!aligned16(x) || !aligned16(weight) || !aligned16(residual) || !aligned16(out) ||
      (pre != nullptr && !aligned16(pre)) || (ln_weight != nullptr && !aligned16(ln_weight)) ||
      (ln_bias != nullptr && !aligned16(ln_bias))) {
    set_error("linear_residual_layer_norm: buffers must be 16-byte aligned");
    return GRM_HIP_EUNSUPPORTED;
  }
  OutLnArgs a;
  a.h = x;
  a.w = weight;
  a.bias = bias;
  a.res = residual;
  a.ln_w = ln_weight;
  a.ln_b = ln_bias;
  a.out = out;
  a.pre = pre;
  a.mean = mean;
  a.rstd = rstd;
  a.rows = rows;
  a.K = static_cast<int>(in_dim);
  a.N = static_cast<int>(out_dim);
  a.eps = eps;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const dim3 grid(static_cast<unsigned>((rows + OL_BM - 1) / OL_BM));
  auto go = [&](auto et) {
    using E = decltype(et);
    auto launch = [&](auto pt) {
      using P = decltype(pt);
      if (a.N == OL_MAXN) {
        hipLaunchKernelGGL((out_ln_kernel<E, P, true>), grid, dim3(OL_THREADS), 0, s, a);
      } else {
        hipLaunchKernelGGL((out_ln_kernel<E, P, false>), grid, dim3(OL_THREADS), 0, s, a);
      }
    };
    switch (param_dtype) {
      case GRM_HIP_F32: launch(F32{}); break;
      case GRM_HIP_F16: launch(F16{}); break;
      default: launch(BF16{}); break;
    }
  };
  if (dtype == GRM_HIP_F16) {
    go(F16{});
  } else {
    go(BF16{});
  }
  return check_launch("linear_residual_layer_norm");
}
