// Top-k routing by threshold selection, bf16 inputs, gfx950.
//
// Same result as route_kernel in route_fuse.hip, bit for bit: every selected
// score is the fp32 FMA chain over d = 0 .. dim-1 in order, times `scale`;
// the k best are taken by (score descending, index ascending); gates are the
// softmax of the selected scores over the temperature.  Routing of
// SegmentRecurrentMemoryModel._route_chunk (reference grm/core/paper_grm.py:
// 566-589) and TopKMemoryRetriever.forward (grm/core/gating_unit.py:54-91).
//
// The MFMA narrows the search; only a handful of keys per row get the exact
// chain.  With A the bf16 MFMA approximation of the unscaled dot product and
// e = 4 max(dim, 64) 2^-23 |q| max|key| a bound on |A - chain| (both are fp32
// sums of the same exact bf16 products):
//
//  pass 1  MFMA scores of every key; in the accumulator layout each lane keeps
//          the two largest A of 8 key classes (key mod 32) of its rows, so a row
//          holds 32 classes x 2 = 64 values, each the A of a distinct key.
//          L = k-th largest of those 64 <= k-th largest A of the row.
//  pass 2  the MFMA scores again; keys with A >= L - W are appended to the
//          row's candidate list in LDS.  Every key of the exact top k is a
//          candidate: its chain is >= the k-th best chain up to the ties that
//          the final multiplication by `scale` can create (d), the k-th best
//          chain is >= the k-th best A - e, so its A >= L - 2e - d; W is twice
//          2e + d plus the terms for flushed denormal products.
//  pass 3  one lane per row computes the exact chain of each candidate (keys
//          from LDS) and keeps the k best exactly.  A row whose list overflows,
//          whose inputs are not finite, or whose window holds at most k keys is
//          scored exactly over every key of its window instead.
//
// All keys of one batch entry are staged in LDS once per workgroup, and each
// workgroup walks several 512-row blocks of its batch entry, so keys cross
// HBM/L2 once per workgroup.  Eight waves per workgroup, 64 rows per wave.
#include <stdint.h>
#include <string.h>

#include <cfloat>
#include <cmath>

#include "grm_hip.h"
#include "grm_hip_common.h"
#include "route_select.h"

namespace grmhip {
namespace {

constexpr int SW = 8;            // waves per workgroup
constexpr int ST = 64 * SW;      // threads per workgroup
constexpr int SROWS = 64 * SW;   // query rows per block
constexpr int SKT = 32;          // keys per MFMA step
constexpr int kLdsMax = 163840;  // LDS bytes one workgroup may use on gfx950
constexpr int kTransBytes = 16 * 64 * 4;  // one 16-row round of the class maxima

struct SelParams {
  RouteSelArgs a;
  int s_pad;    // key rows staged in LDS (a multiple of SKT)
  int scratch;  // LDS bytes per wave: the class-maxima transposition, then the candidate lists
  int cap;      // candidate slots per row
  int nblk;     // row blocks per batch entry
};

// max / min as one med3 against +-FLT_MAX (fmaxf would add NaN-quieting
// instructions, and a med3 against an infinity is folded back into it).  Exact
// for the values met here, which are below FLT_MAX: max_num is the maximum;
// min_num is the minimum, except that a -inf paired with a larger value comes
// out as -FLT_MAX, which stays below every score.
__device__ __forceinline__ float max_num(float a, float b) { return __builtin_amdgcn_fmed3f(a, b, FLT_MAX); }
__device__ __forceinline__ float min_num(float a, float b) { return __builtin_amdgcn_fmed3f(a, b, -FLT_MAX); }

__device__ __forceinline__ void cs_desc(float& a, float& b) {
  const float hi = max_num(a, b), lo = min_num(a, b);
  a = hi;
  b = lo;
}

// x[off .. off + N) sorted descending (bitonic network).
template <int N, int TOT>
__device__ __forceinline__ void sort_block_desc(float (&x)[TOT], int off) {
#pragma unroll
  for (int size = 2; size <= N; size <<= 1) {
#pragma unroll
    for (int stride = size >> 1; stride > 0; stride >>= 1) {
#pragma unroll
      for (int i = 0; i < N; ++i) {
        const int j = i ^ stride;
        if (j > i) {
          if ((i & size) == 0) {
            cs_desc(x[off + i], x[off + j]);
          } else {
            cs_desc(x[off + j], x[off + i]);
          }
        }
      }
    }
  }
}

// The N largest of the descending blocks at oa and ob, descending, at oa:
// max(A_i, B_{N-1-i}) is bitonic and holds them; half-cleaners sort it.
template <int N, int TOT>
__device__ __forceinline__ void merge_top_desc(float (&x)[TOT], int oa, int ob) {
#pragma unroll
  for (int i = 0; i < N; ++i) x[oa + i] = max_num(x[oa + i], x[ob + N - 1 - i]);
#pragma unroll
  for (int stride = N >> 1; stride > 0; stride >>= 1) {
#pragma unroll
    for (int i = 0; i < N; ++i) {
      if ((i & stride) == 0) cs_desc(x[oa + i], x[oa + i + stride]);
    }
  }
}

// x[0 .. KM) = the KM largest of x[0 .. 64), descending.
template <int KM>
__device__ __forceinline__ void top_of_64(float (&x)[64]) {
  constexpr int NB = 64 / KM;
#pragma unroll
  for (int blk = 0; blk < NB; ++blk) sort_block_desc<KM, 64>(x, blk * KM);
#pragma unroll
  for (int width = 1; width < NB; width <<= 1) {
#pragma unroll
    for (int blk = 0; blk < NB; blk += 2 * width) merge_top_desc<KM, 64>(x, blk * KM, (blk + width) * KM);
  }
}

template <int KMAX>
__device__ __forceinline__ void exact_insert_sel(float (&ts)[KMAX], int (&ti)[KMAX], float cs, int ci) {
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

// LDS element offset of 16-byte granule u of staged key row r: granules are
// XOR-swizzled by row so that the fragment reads of 16 rows spread over banks.
template <int NG>
__device__ __forceinline__ int key_off(int r, int u) {
  return (r * NG + (u ^ (r & (NG - 1)))) * 8;
}

// Exact score of one key: the fp32 FMA chain over d in increasing order, times
// scale.  qf holds the row's query converted to fp32 once.  FULL (dim == DKP):
// one straight-line body, so the key loads of every granule are in flight
// together; otherwise granules past dim are skipped (they are zero, but an
// extra fma(0, 0, -0) would turn a -0 chain into +0).  One chain per call: the
// chain's FMAs issue back to back, and the key conversions fill the gaps.
template <int DKP, bool FULL>
__device__ __forceinline__ float exact_one(const float (&qf)[DKP], const uint16_t* klds, int key, int dim,
                                           float scale) {
  constexpr int NG = DKP / 8;
  float acc = 0.f;
#pragma unroll
  for (int u = 0; u < NG; ++u) {
    if (FULL || 8 * u < dim) {
      const U8<BF16> kv = __builtin_bit_cast(U8<BF16>, *reinterpret_cast<const uint4*>(klds + key_off<NG>(key, u)));
#pragma unroll
      for (int e = 0; e < 8; ++e) acc = fmaf(qf[8 * u + e], ET<BF16>::to_f(kv.e[e]), acc);
    }
  }
  return acc * scale;
}

__device__ __forceinline__ void wave_sync_lds() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

template <int DKP, int KMAX, bool WIN, bool FULL>
__global__ __launch_bounds__(ST) void route_select_kernel(const SelParams p) {
  constexpr int NC = DKP / 32;  // 32-element MFMA steps over d
  constexpr int NG = DKP / 8;   // 16-byte granules per key row
  extern __shared__ __align__(16) unsigned char lds[];
  uint16_t* klds = reinterpret_cast<uint16_t*>(lds);
  const RouteSelArgs& a = p.a;

  const int tid = threadIdx.x;
  const int lane0 = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform: scalar loop control
  const int64_t b = blockIdx.y;
  const int D = a.dim;
  const int S = static_cast<int>(a.n_keys);
  const int k = a.k;
  unsigned char* const scratch0 = lds + static_cast<size_t>(p.s_pad) * DKP * 2;
  unsigned char* const wscr = scratch0 + static_cast<size_t>(w) * p.scratch;

  // ---- keys of this batch entry into LDS (rows past S and dims past D are zero)
  const uint16_t* kb = static_cast<const uint16_t*>(a.keys) + b * a.n_keys * D;
  const __amdgpu_buffer_rsrc_t rk = make_rsrc(kb, static_cast<uint32_t>(a.n_keys * D * 2));
  for (int e = tid; e < p.s_pad * NG; e += ST) {
    const int r = e / NG, u = e % NG;
    const uint4 v = __builtin_bit_cast(uint4, buf_load8<BF16>(rk, (r < S && 8 * u < D) ? (r * D + 8 * u) * 2 : kBufOOB));
    *reinterpret_cast<uint4*>(klds + key_off<NG>(r, u)) = v;
  }
  __syncthreads();
  // Largest squared key norm (NaN if any key is not finite).
  float kn2 = 0.f;
  for (int r = tid; r < S; r += ST) {
    float t = 0.f;
#pragma unroll
    for (int u = 0; u < NG; ++u) {
      const U8<BF16> kv = __builtin_bit_cast(U8<BF16>, *reinterpret_cast<const uint4*>(klds + key_off<NG>(r, u)));
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float x = ET<BF16>::to_f(kv.e[e]);
        t = fmaf(x, x, t);
      }
    }
    kn2 = (t <= INFINITY) ? fmaxf(kn2, t) : NAN;  // false for NaN
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    const float o = __shfl_xor(kn2, off, 64);
    kn2 = (o <= INFINITY && kn2 <= INFINITY) ? fmaxf(kn2, o) : NAN;
  }
  float* red = reinterpret_cast<float*>(scratch0);
  if (lane0 == 0) red[w] = kn2;
  __syncthreads();
  float kmax2 = red[0];
#pragma unroll
  for (int i = 1; i < SW; ++i) kmax2 = (red[i] <= INFINITY && kmax2 <= INFINITY) ? fmaxf(kmax2, red[i]) : NAN;
  __syncthreads();  // red is read before wave 0 reuses its scratch
  const float km = sqrtf(kmax2) * 1.001f;

  const uint16_t* qb = static_cast<const uint16_t*>(a.q) + b * a.n_query * D;
  const __amdgpu_buffer_rsrc_t rq = make_rsrc(qb, static_cast<uint32_t>(a.n_query * D * 2));
  auto win_hi = [&](int64_t r) -> int {
    return WIN ? static_cast<int>(min(a.n_keys, a.base + min(r, a.n_query - 1) / a.seg_len)) : S;
  };
  auto win_lo = [&](int h) -> int { return WIN ? static_cast<int>(h > a.cap ? h - a.cap : int64_t{0}) : 0; };
  float* trans = reinterpret_cast<float*>(wscr);
  uint16_t* lst = reinterpret_cast<uint16_t*>(wscr + 256);
  const int cap = p.cap;

  for (int blk = blockIdx.x; blk < p.nblk; blk += gridDim.x) {
    // The lane index is made opaque per block, so that the compiler does not
    // hoist every lane-dependent address out of this loop (and spill them).
    int lane = lane0;
    asm volatile("" : "+v"(lane));
    const int g = lane >> 4, n = lane & 15;
    const int64_t qw = static_cast<int64_t>(blk) * SROWS + 64 * w;  // first row of this wave
    if (qw >= a.n_query) continue;                                   // wave-uniform
    const int64_t qi = qw + lane;
    const bool active = qi < a.n_query;
    const int row_hi = win_hi(qi), row_lo = win_lo(row_hi);
    const int row_n = row_hi - row_lo;
    const bool row_nat = WIN && row_n <= k;

    // B operands: rows qw + 16 qt + n, d = 32 c + 8 g .. + 7.  Loaded for each
    // MFMA pass (L2 hits the second time), so they are not live across the
    // selection network.
    Frag8<BF16> bq[4][NC];
    auto load_bq = [&]() {
#pragma unroll
      for (int qt = 0; qt < 4; ++qt) {
        const int64_t row = qw + 16 * qt + n;
#pragma unroll
        for (int c = 0; c < NC; ++c) {
          const int d = 32 * c + 8 * g;
          bq[qt][c] = __builtin_bit_cast(
              Frag8<BF16>,
              buf_load8<BF16>(rq, (row < a.n_query && d < D) ? static_cast<int>((row * D + d) * 2) : kBufOOB));
        }
      }
    };
    load_bq();
    // Squared row norms.
    float qp[4];
#pragma unroll
    for (int qt = 0; qt < 4; ++qt) {
      qp[qt] = 0.f;
#pragma unroll
      for (int c = 0; c < NC; ++c) {
        const U8<BF16> v = __builtin_bit_cast(U8<BF16>, bq[qt][c]);
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
    int pk_lo[4], pk_hi[4];
#pragma unroll
    for (int qt = 0; qt < 4; ++qt) {
      pk_hi[qt] = win_hi(qw + 16 * qt + n);
      pk_lo[qt] = win_lo(pk_hi[qt]);
    }
    // Keys the wave scores, and the steps that lie inside every row's window:
    // [wave_lo, in_a) and [in_b, wave_hi) are masked per key, [in_a, in_b) not.
    const int wave_lo = win_lo(win_hi(qw)) & ~(SKT - 1);
    const int wave_hi = win_hi(qw + 63);
    const int in_a = min(max((win_lo(win_hi(qw + 63)) + SKT - 1) & ~(SKT - 1), wave_lo), wave_hi);
    const int in_b = max(min(win_hi(qw) & ~(SKT - 1), wave_hi), in_a);

    auto scores = [&](int s0, f32x4 (&acc)[4][2]) {
      Frag8<BF16> ak[2][NC];
#pragma unroll
      for (int kt = 0; kt < 2; ++kt) {
        const int row = s0 + 16 * kt + n;
#pragma unroll
        for (int c = 0; c < NC; ++c)
          ak[kt][c] = __builtin_bit_cast(Frag8<BF16>, *reinterpret_cast<const uint4*>(klds + key_off<NG>(row, 4 * c + g)));
      }
#pragma unroll
      for (int qt = 0; qt < 4; ++qt)
#pragma unroll
        for (int kt = 0; kt < 2; ++kt) {
          acc[qt][kt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
          for (int c = 0; c < NC; ++c) acc[qt][kt] = mfma8(ak[kt][c], bq[qt][c], acc[qt][kt]);
        }
    };
    // Keys outside a row's window score -inf (acc[qt][kt][r] is key s0 + 16 kt + 4 g + r
    // of row 16 qt + n).
    auto mask = [&](int s0, f32x4 (&acc)[4][2]) {
#pragma unroll
      for (int qt = 0; qt < 4; ++qt)
#pragma unroll
        for (int kt = 0; kt < 2; ++kt)
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const int key = s0 + 16 * kt + 4 * g + r;
            acc[qt][kt][r] = (key >= pk_lo[qt] && key < pk_hi[qt]) ? acc[qt][kt][r] : -INFINITY;
          }
    };

    // ---- pass 1: the two largest A of each key class.
    float m1[4][2][4], m2[4][2][4];
#pragma unroll
    for (int qt = 0; qt < 4; ++qt)
#pragma unroll
      for (int kt = 0; kt < 2; ++kt)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          m1[qt][kt][r] = -INFINITY;
          m2[qt][kt][r] = -INFINITY;
        }
    auto keep2 = [&](const f32x4 (&acc)[4][2]) {
#pragma unroll
      for (int qt = 0; qt < 4; ++qt)
#pragma unroll
        for (int kt = 0; kt < 2; ++kt)
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const float v = acc[qt][kt][r];
            m2[qt][kt][r] = __builtin_amdgcn_fmed3f(m1[qt][kt][r], m2[qt][kt][r], v);
            m1[qt][kt][r] = max_num(m1[qt][kt][r], v);
          }
    };
    // Only the steps inside every row's window: the maxima over a subset of a
    // row's keys still bound its k-th best from below, and no masking is needed.
    for (int s0 = in_a; s0 < in_b; s0 += SKT) {
      f32x4 acc[4][2];
      scores(s0, acc);
      keep2(acc);
    }

    // ---- each row's 64 class values to the lane that owns the row, 16 rows a round.
    // Row n' of a round holds 16 granules of 4 floats; granule p sits at p ^ n'.
    float x[64];
#pragma unroll
    for (int i = 0; i < 64; ++i) x[i] = -INFINITY;
#pragma unroll
    for (int qt = 0; qt < 4; ++qt) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        // granule 4 g + i of row n: classes (kt, r) = (i >> 1, 2 (i & 1) + {0, 1}), both maxima
        const int kt = i >> 1, r0 = 2 * (i & 1);
        const float4 v = make_float4(m1[qt][kt][r0], m2[qt][kt][r0], m1[qt][kt][r0 + 1], m2[qt][kt][r0 + 1]);
        *reinterpret_cast<float4*>(trans + (n * 16 + ((4 * g + i) ^ n)) * 4) = v;
      }
      wave_sync_lds();
      // Every lane reads and keeps the round of its own row (a select, not a
      // branch: the values stay in place in registers).
      const bool mine = g == qt;
#pragma unroll
      for (int pp = 0; pp < 16; ++pp) {
        const float4 v = *reinterpret_cast<const float4*>(trans + (n * 16 + (pp ^ n)) * 4);
        x[4 * pp] = mine ? v.x : x[4 * pp];
        x[4 * pp + 1] = mine ? v.y : x[4 * pp + 1];
        x[4 * pp + 2] = mine ? v.z : x[4 * pp + 2];
        x[4 * pp + 3] = mine ? v.w : x[4 * pp + 3];
      }
      wave_sync_lds();
    }
    top_of_64<KMAX>(x);
    float lk = x[0];
#pragma unroll
    for (int i = 1; i < KMAX; ++i) lk = (i == k - 1) ? x[i] : lk;

    // Candidate threshold L - W (W as in the header comment, doubled).
    const float qn = sqrtf(qn2) * 1.001f;
    const float e_mfma = 4.f * static_cast<float>(max(D, 64)) * 0x1p-23f * qn * km;
    // |A| <= |q| |key| + e for every key (pass 1 may have skipped the largest)
    const float mag = max_num(fabsf(lk), qn * km) + 4.f * e_mfma;
    const float wl = 2.f * (2.f * e_mfma + 0x1p-21f * (mag + 2.f * e_mfma) + 0x1p-148f / a.scale +
                            4.f * static_cast<float>(D) * 0x1p-126f * (qn + km));
    const bool sound = qn * km < 1e30f && wl <= 1e30f;  // false for NaN and inf (L = -inf too)
    const bool exact_all = row_nat || !sound;
    const float thr = (active && !exact_all) ? lk - wl : INFINITY;
    float thr_q[4];
#pragma unroll
    for (int qt = 0; qt < 4; ++qt) thr_q[qt] = __shfl(thr, 16 * qt + n, 64);

    // ---- pass 2: candidates A >= L - W into the rows' lists.  Each lane marks its
    // hits in one 64-bit mask per row tile over up to kFlush steps; the marks are
    // then appended together.  The four lanes of a row (lanes n, n + 16, n + 32,
    // n + 48) count their hits; a prefix over them gives each its slots, so the
    // lists are filled without atomics, and one loop takes every lane's hits of
    // the group (its trip count is the largest number of hits one lane holds, not
    // a sum over the steps of each step's largest).
    asm volatile("" ::: "memory");  // reload the B operands rather than keep them
    load_bq();
    int filled[4] = {0, 0, 0, 0};  // list length of row 16 qt + n, the same in its four lanes
    constexpr int kFlush = 8;      // steps per group: 8 bits each
    // bit 8 i + 4 kt + r of hq[qt]: key s0g + SKT i + 16 kt + 4 g + r of row 16 qt + n
    uint64_t hq[4] = {0u, 0u, 0u, 0u};
    auto mark = [&](int i, const f32x4 (&acc)[4][2]) {
#pragma unroll
      for (int qt = 0; qt < 4; ++qt) {
        uint32_t b = 0u;
#pragma unroll
        for (int kt = 0; kt < 2; ++kt)
#pragma unroll
          for (int r = 0; r < 4; ++r) b |= (acc[qt][kt][r] >= thr_q[qt] ? 1u : 0u) << (4 * kt + r);
        hq[qt] |= static_cast<uint64_t>(b) << (8 * i);
      }
    };
    auto flush = [&](int s0g) {
      int base[4];
#pragma unroll
      for (int qt = 0; qt < 4; ++qt) {
        const int mine = __builtin_popcountll(hq[qt]);
        // Exclusive prefix over g and the total, with lane swaps (no LDS): the
        // 16-lane swap pairs g = 0 with 1 and 2 with 3, the 32-lane swap the halves.
        const auto p16 = __builtin_amdgcn_permlane16_swap(mine, mine, false, false);
        const int even = static_cast<int>(p16[0]), odd = static_cast<int>(p16[1]);
        const int pair = even + odd;
        const auto p32 = __builtin_amdgcn_permlane32_swap(pair, pair, false, false);
        const int low = static_cast<int>(p32[0]), high = static_cast<int>(p32[1]);
        base[qt] = filled[qt] + ((g & 1) ? even : 0) + (g >= 2 ? low : 0);
        filled[qt] += low + high;
      }
      while ((hq[0] | hq[1] | hq[2] | hq[3]) != 0u) {
        // the lowest hit of the first non-empty mask
        const int qt = hq[0] != 0u ? 0 : hq[1] != 0u ? 1 : hq[2] != 0u ? 2 : 3;
        const uint64_t m = qt == 0 ? hq[0] : qt == 1 ? hq[1] : qt == 2 ? hq[2] : hq[3];
        const int j = __builtin_ctzll(m);
        const uint64_t rest = m & (m - 1u);
        const int row = 16 * qt + n;
        const int key = s0g + SKT * (j >> 3) + 16 * ((j >> 2) & 1) + 4 * g + (j & 3);
        const int pos = qt == 0 ? base[0] : qt == 1 ? base[1] : qt == 2 ? base[2] : base[3];
        if (pos < cap) lst[row * cap + pos] = static_cast<uint16_t>(key);
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          base[t] += (t == qt) ? 1 : 0;
          hq[t] = (t == qt) ? rest : hq[t];
        }
      }
    };
    // Steps in groups of kFlush over a contiguous range of key steps; `masked`
    // for the steps at the window boundaries.
    auto pass2 = [&](int lo, int hi, bool masked) {
      int i = 0, s0g = lo;
      for (int s0 = lo; s0 < hi; s0 += SKT) {
        f32x4 acc[4][2];
        scores(s0, acc);
        if (masked) mask(s0, acc);
        mark(i, acc);
        if (++i == kFlush) {
          flush(s0g);
          i = 0;
          s0g = s0 + SKT;
        }
      }
      if (i != 0) flush(s0g);
    };
    pass2(in_a, in_b, false);
    pass2(wave_lo, min(in_a, wave_hi), true);      // the boundary steps below the interior
    pass2(max(in_b, in_a), wave_hi, true);         // and above it
    // the row owner (lane 16 g + n owns row 16 g + n) takes its row's length
    const int c = g == 0 ? filled[0] : g == 1 ? filled[1] : g == 2 ? filled[2] : filled[3];
    wave_sync_lds();

    // ---- pass 3: exact chains of the candidates (or of the whole window).
    float qf[DKP];
#pragma unroll
    for (int u = 0; u < NG; ++u) {
      const U8<BF16> v =
          buf_load8<BF16>(rq, (active && 8 * u < D) ? static_cast<int>((qi * D + 8 * u) * 2) : kBufOOB);
#pragma unroll
      for (int e = 0; e < 8; ++e) qf[8 * u + e] = ET<BF16>::to_f(v.e[e]);
    }
    float top_s[KMAX];
    int top_i[KMAX];
#pragma unroll
    for (int m = 0; m < KMAX; ++m) {
      top_s[m] = -INFINITY;
      top_i[m] = INT32_MAX;
    }
    const bool scan_all = exact_all || c > cap || c < min(k, row_n);
    const int count = !active ? 0 : scan_all ? max(row_n, 0) : c;
#pragma unroll 1
    for (int j = 0; j < count; ++j) {
      const int key = scan_all ? row_lo + j : static_cast<int>(lst[lane * cap + j]);
      const float sc = exact_one<DKP, FULL>(qf, klds, key, D, a.scale);
      if (row_nat) {
#pragma unroll
        for (int m = 0; m < KMAX; ++m) {
          if (m == key - row_lo) {
            top_s[m] = sc;
            top_i[m] = key;
          }
        }
      } else {
        exact_insert_sel<KMAX>(top_s, top_i, sc, key);
      }
    }
    wave_sync_lds();  // the lists are read before the next block reuses the scratch
    if (!active) continue;

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
      continue;
    }
    write_topk_row<KMAX>(a.idx, a.scores, a.gates, obase, k, a.inv_temp, top_s, top_i);
  }
}

template <int DKP, int KMAX, bool WIN, bool FULL>
int launch_sel(const SelParams& p, int64_t batch, int lds_bytes, hipStream_t s) {
  static bool attr_set = false;
  if (!attr_set) {
    hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(&route_select_kernel<DKP, KMAX, WIN, FULL>),
                                       hipFuncAttributeMaxDynamicSharedMemorySize, kLdsMax);
    if (e != hipSuccess) {
      set_error("topk_route: hipFuncSetAttribute failed: %s", hipGetErrorString(e));
      return static_cast<int>(e);
    }
    attr_set = true;
  }
  // Enough workgroups to give every CU one, each walking several blocks of its batch entry.
  const int64_t per_batch = std::max<int64_t>(1, (256 + batch - 1) / batch);
  const int nx = static_cast<int>(std::min<int64_t>(p.nblk, per_batch));
  hipLaunchKernelGGL((route_select_kernel<DKP, KMAX, WIN, FULL>),
                     dim3(static_cast<unsigned>(nx), static_cast<unsigned>(batch)), dim3(ST), lds_bytes, s, p);
  return check_launch("topk_route");
}

template <int DKP, bool WIN, bool FULL>
int launch_sel_k(const SelParams& p, int64_t batch, int lds_bytes, hipStream_t s) {
  if (p.a.k <= 8) return launch_sel<DKP, 8, WIN, FULL>(p, batch, lds_bytes, s);
  if (p.a.k <= 16) return launch_sel<DKP, 16, WIN, FULL>(p, batch, lds_bytes, s);
  return launch_sel<DKP, 32, WIN, FULL>(p, batch, lds_bytes, s);
}

template <int DKP, bool WIN>
int launch_sel_full(const SelParams& p, int64_t batch, int lds_bytes, hipStream_t s) {
  return p.a.dim == DKP ? launch_sel_k<DKP, WIN, true>(p, batch, lds_bytes, s)
                        : launch_sel_k<DKP, WIN, false>(p, batch, lds_bytes, s);
}

template <bool WIN>
int launch_sel_win(const SelParams& p, int64_t batch, int dkp, int lds_bytes, hipStream_t s) {
  if (dkp == 32) return launch_sel_full<32, WIN>(p, batch, lds_bytes, s);
  if (dkp == 64) return launch_sel_full<64, WIN>(p, batch, lds_bytes, s);
  return launch_sel_full<128, WIN>(p, batch, lds_bytes, s);
}

}  // namespace

int try_route_select(const RouteSelArgs& a, int dtype, int64_t batch, hipStream_t s, int* rc) {
  const bool win = a.seg_len > 0;
  if (dtype != GRM_HIP_BF16 || !(a.scale > 0.f) || a.dim < 1 || a.dim > 128 || a.dim % 8 != 0 || a.k < 1 ||
      a.k > 32 || a.n_keys < 1 || a.n_keys > 65535 || (!win && a.k >= a.n_keys) || batch > 65535)
    return 0;
  if ((reinterpret_cast<uintptr_t>(a.q) | reinterpret_cast<uintptr_t>(a.keys)) % 16 != 0) return 0;
  if (a.n_query * a.dim * 2 > INT32_MAX || a.n_keys * a.dim * 2 > INT32_MAX) return 0;
  const int dkp = a.dim <= 32 ? 32 : a.dim <= 64 ? 64 : 128;
  const int s_pad = static_cast<int>((a.n_keys + SKT - 1) / SKT * SKT);
  const int64_t key_bytes = static_cast<int64_t>(s_pad) * dkp * 2;
  const int64_t avail = ((kLdsMax - key_bytes) / SW) & ~int64_t{15};
  if (avail < kTransBytes) return 0;
  const int cap = static_cast<int>(std::min<int64_t>(2 * a.k + 8, (avail - 256) / 128));
  if (cap < a.k + 4) return 0;
  const int scratch = std::max(kTransBytes, (256 + 128 * cap + 15) & ~15);
  const int lds_bytes = static_cast<int>(key_bytes) + SW * scratch;
  SelParams p;
  memset(&p, 0, sizeof(p));
  p.a = a;
  p.s_pad = s_pad;
  p.scratch = scratch;
  p.cap = cap;
  const int64_t nblk = (a.n_query + SROWS - 1) / SROWS;
  if (nblk > INT32_MAX) return 0;
  p.nblk = static_cast<int>(nblk);
  *rc = win ? launch_sel_win<true>(p, batch, dkp, lds_bytes, s) : launch_sel_win<false>(p, batch, dkp, lds_bytes, s);
  return 1;
}

}  // namespace grmhip
