// Gradient of the chunked linear-memory update + query application, gfx950.
//
// Adjoint of  M_t = decay M_{t-1} + c v_t k_t^T,  h_t = M_t q_t   (c = (1-decay)/sqrt(d_k))
// (reference grm/csrc/chunk_update.cu:137-278 and :588-716; CPU autograd in
// grm_cuda.cpp:92-126).  With G_t = dL/dM_t:
//   G_t     = decay G_{t+1} + dh_t q_t^T     (G at the last token starts from grad_memory_out)
//   dv_t[v] = c <G_t[v, :], k_t>
//   dk_t[k] = c sum_v G_t[v, k] v_t[v]
//   dq_t[k] = sum_v dh_t[v] M_t[v, k]
//   dM_0    = decay G_0
// Instead of the reference's per-token state history, the forward kernel is
// re-run to store only the state at every 64-token chunk boundary; each chunk
// is then replayed forward (rebuilding M_t for dq) and swept backward (G, dk, dv).
//
// One wavefront owns 16 value rows of one sequence, lanes hold d_k in steps
// of 64.  dq and dk are summed over those 16 rows in registers and written as
// per-tile partials; a second kernel adds the tiles in a fixed order, so the
// result is deterministic and atomic-free like the reference's partial-buffer
// reduction.  dv is a reduction over k done with a 16-value transposing
// butterfly (17 shuffles per token).
#include <stdint.h>
#include <string.h>

#include <cmath>
#include <cstdlib>

#include "grm_hip.h"
#include "grm_hip_common.h"

namespace grmhip {
namespace {

constexpr int RB = 16;   // value rows per wavefront
constexpr int BCT = 64;  // tokens per chunk (chunk_states granularity)

struct BwdArgs {
  const void* dh;
  const void* dmo;     // grad_memory_out
  const void* keys;
  const void* values;
  const void* queries;
  const void* memory;  // initial state
  const float* states; // [B, n_chunks, dv, dk] state after each chunk
  void* dv_out;
  void* dm_out;        // grad_memory
  float* part_k;       // [B, tiles, T, dk]
  float* part_q;       // [B, tiles, T, dk]
  int64_t batch;
  int64_t T;
  int dk;
  int dv;
  int tiles;
  int n_chunks;
  int mem_f32;
  float decay;
  float c;
};

template <class E>
__device__ __forceinline__ float ld(const void* p, int64_t i) {
  return ET<E>::to_f(static_cast<const typename ET<E>::raw*>(p)[i]);
}

template <class E, int KR>
__global__ __launch_bounds__(64) void chunk_bwd_kernel(const BwdArgs a) {
  const int lane = threadIdx.x;
  const int64_t b = blockIdx.x / a.tiles;
  const int tile = blockIdx.x % a.tiles;
  const int v0 = tile * RB;
  const int dk = a.dk, dv = a.dv;
  const int64_t T = a.T;
  // 32-bit chunk lengths (a 64-bit min would be a VALU compare in the loop)
  const int last_len = static_cast<int>(T - static_cast<int64_t>(a.n_chunks - 1) * BCT);
  const float lam = a.decay, c = a.c;
  const bool f32m = a.mem_f32 != 0;

  auto mem_ld = [&](const void* p, int64_t i) -> float {
    return f32m ? static_cast<const float*>(p)[i] : ld<E>(p, i);
  };

  // Carried adjoint E = dL/dM at the end of the current chunk.
  float G[RB][KR];
#pragma unroll
  for (int r = 0; r < RB; ++r) {
    const int v = v0 + r;
#pragma unroll
    for (int e = 0; e < KR; ++e) {
      const int k = lane + 64 * e;
      G[r][e] = (v < dv && k < dk) ? mem_ld(a.dmo, (b * dv + v) * dk + k) : 0.f;
    }
  }

  for (int ch = a.n_chunks - 1; ch >= 0; --ch) {
    const int64_t t0 = static_cast<int64_t>(ch) * BCT;
    const int L = ch == a.n_chunks - 1 ? last_len : BCT;
    // ---- forward replay of the chunk: rebuild M_t rows, emit dq partials
    {
      float m[RB][KR];
#pragma unroll
      for (int r = 0; r < RB; ++r) {
        const int v = v0 + r;
#pragma unroll
        for (int e = 0; e < KR; ++e) {
          const int k = lane + 64 * e;
          float x = 0.f;
          if (v < dv && k < dk) {
            x = (ch == 0) ? mem_ld(a.memory, (b * dv + v) * dk + k)
                          : a.states[((b * a.n_chunks + ch - 1) * dv + v) * dk + k];
          }
          m[r][e] = x;
        }
      }
      for (int t = 0; t < L; ++t) {
        const int64_t tt = t0 + t;
        float kt[KR];
#pragma unroll
        for (int e = 0; e < KR; ++e) {
          const int k = lane + 64 * e;
          kt[e] = (k < dk) ? ld<E>(a.keys, (b * T + tt) * dk + k) : 0.f;
        }
        float dq[KR];
#pragma unroll
        for (int e = 0; e < KR; ++e) dq[e] = 0.f;
#pragma unroll
        for (int r = 0; r < RB; ++r) {
          const int v = v0 + r;
          const float vv = (v < dv) ? ld<E>(a.values, (b * T + tt) * dv + v) : 0.f;
          const float dh = (v < dv) ? ld<E>(a.dh, (b * T + tt) * dv + v) : 0.f;
          const float cv = c * vv;
#pragma unroll
          for (int e = 0; e < KR; ++e) {
            m[r][e] = fmaf(m[r][e], lam, cv * kt[e]);
            dq[e] = fmaf(dh, m[r][e], dq[e]);
          }
        }
        float* pq = a.part_q + ((b * a.tiles + tile) * T + tt) * dk;
#pragma unroll
        for (int e = 0; e < KR; ++e) {
          const int k = lane + 64 * e;
          if (k < dk) pq[k] = dq[e];
        }
      }
    }
    // ---- backward sweep: G, dk partials, dv
    for (int t = L - 1; t >= 0; --t) {
      const int64_t tt = t0 + t;
      const bool first = (t == L - 1);
      float kt[KR], qt[KR];
#pragma unroll
      for (int e = 0; e < KR; ++e) {
        const int k = lane + 64 * e;
        kt[e] = (k < dk) ? ld<E>(a.keys, (b * T + tt) * dk + k) : 0.f;
        qt[e] = (k < dk) ? ld<E>(a.queries, (b * T + tt) * dk + k) : 0.f;
      }
      float dkacc[KR];
#pragma unroll
      for (int e = 0; e < KR; ++e) dkacc[e] = 0.f;
      float dvp[RB];
#pragma unroll
      for (int r = 0; r < RB; ++r) {
        const int v = v0 + r;
        const float vv = (v < dv) ? ld<E>(a.values, (b * T + tt) * dv + v) : 0.f;
        const float dh = (v < dv) ? ld<E>(a.dh, (b * T + tt) * dv + v) : 0.f;
        float acc = 0.f;
#pragma unroll
        for (int e = 0; e < KR; ++e) {
          const float gp = first ? G[r][e] : G[r][e] * lam;
          G[r][e] = fmaf(dh, qt[e], gp);
          dkacc[e] = fmaf(G[r][e], vv, dkacc[e]);
          acc = fmaf(G[r][e], kt[e], acc);
        }
        dvp[r] = acc;
      }
      float* pk = a.part_k + ((b * a.tiles + tile) * T + tt) * dk;
#pragma unroll
      for (int e = 0; e < KR; ++e) {
        const int k = lane + 64 * e;
        if (k < dk) pk[k] = c * dkacc[e];
      }
      // 16 row sums over 64 lanes: halve the value count per exchange.
#pragma unroll
      for (int half = RB / 2, d = 32; half >= 1; half >>= 1, d >>= 1) {
        const bool up = (lane & d) != 0;
#pragma unroll
        for (int i = 0; i < half; ++i) {
          const float send = up ? dvp[i] : dvp[i + half];
          const float keep = up ? dvp[i + half] : dvp[i];
          dvp[i] = keep + __shfl_xor(send, d, 64);
        }
      }
      float tot = dvp[0];
      tot += __shfl_xor(tot, 2, 64);
      tot += __shfl_xor(tot, 1, 64);
      if ((lane & 3) == 0) {
        const int r = ((lane >> 5) & 1) * 8 + ((lane >> 4) & 1) * 4 + ((lane >> 3) & 1) * 2 +
                      ((lane >> 2) & 1);
        const int v = v0 + r;
        if (v < dv) {
          static_cast<typename ET<E>::raw*>(a.dv_out)[(b * T + tt) * dv + v] = ET<E>::from_f(c * tot);
        }
      }
    }
    // G now holds G_0 of this chunk; carry decay * G_0 into the previous chunk.
#pragma unroll
    for (int r = 0; r < RB; ++r)
#pragma unroll
      for (int e = 0; e < KR; ++e) G[r][e] *= lam;
  }

#pragma unroll
  for (int r = 0; r < RB; ++r) {
    const int v = v0 + r;
#pragma unroll
    for (int e = 0; e < KR; ++e) {
      const int k = lane + 64 * e;
      if (v < dv && k < dk) {
        const int64_t i = (b * dv + v) * dk + k;
        if (f32m) {
          static_cast<float*>(a.dm_out)[i] = G[r][e];
        } else {
          static_cast<typename ET<E>::raw*>(a.dm_out)[i] = ET<E>::from_f(G[r][e]);
        }
      }
    }
  }
}

// out[b, t, k] = sum over tiles of part[b, tile, t, k], tiles in order.
template <class E>
__global__ __launch_bounds__(256) void tile_sum_kernel(const float* part, void* out, int64_t batch,
                                                       int tiles, int64_t T, int dk) {
  const int64_t n = batch * T * dk;
  const int64_t plane = T * dk;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; i < n;
       i += static_cast<int64_t>(gridDim.x) * 256) {
    const int64_t b = i / plane;
    const int64_t rest = i % plane;
    const float* p = part + b * tiles * plane + rest;
    float s = 0.f;
    for (int t = 0; t < tiles; ++t) s += p[t * plane];
    static_cast<typename ET<E>::raw*>(out)[i] = ET<E>::from_f(s);
  }
}

template <class E>
int launch_bwd(const BwdArgs& a, void* grad_keys, void* grad_queries, hipStream_t s) {
  const dim3 grid(static_cast<unsigned>(a.batch * a.tiles));
  if (a.dk <= 64) {
    hipLaunchKernelGGL((chunk_bwd_kernel<E, 1>), grid, dim3(64), 0, s, a);
  } else if (a.dk <= 128) {
    hipLaunchKernelGGL((chunk_bwd_kernel<E, 2>), grid, dim3(64), 0, s, a);
  } else {
    hipLaunchKernelGGL((chunk_bwd_kernel<E, 4>), grid, dim3(64), 0, s, a);
  }
  int rc = check_launch("chunk_update_bwd");
  if (rc != GRM_HIP_OK) return rc;
  const int64_t n = a.batch * a.T * a.dk;
  const int64_t want = (n + 255) / 256;
  const unsigned g = static_cast<unsigned>(want < 256 * 64 ? want : 256 * 64);
  hipLaunchKernelGGL(tile_sum_kernel<E>, dim3(g < 1 ? 1 : g), dim3(256), 0, s, a.part_k, grad_keys,
                     a.batch, a.tiles, a.T, a.dk);
  rc = check_launch("chunk_update_bwd(grad_keys)");
  if (rc != GRM_HIP_OK) return rc;
  hipLaunchKernelGGL(tile_sum_kernel<E>, dim3(g < 1 ? 1 : g), dim3(256), 0, s, a.part_q,
                     grad_queries, a.batch, a.tiles, a.T, a.dk);
  return check_launch("chunk_update_bwd(grad_queries)");
}


// ---------------------------------------------------------------------------
// Chunk-parallel MFMA backward for 16-bit inputs (key_dim <= 128, value_dim a
// multiple of 32, 16-byte rows), two kernels.  Per 64-token chunk, from the
// chunk's starting state M (the forward's chunk states) and the adjoint G at its
// end (dL/dM after its last token), with D[i][j] = decay^{i-j} (j <= i),
// P = c (Q K^T) o D and dS = c (dH V^T) o D:
//   dQ = decay^{i+1} dH M + dS K
//   dK = dS^T Q + c decay^{L-1-j} V G
//   dV = P^T dH + c decay^{L-1-j} K G^T
//   G  <- decay^L G + dH^T diag(decay^{i+1}) Q      (the adjoint at the chunk's start)
// Only the last line carries from chunk to chunk.  bwd_adjoint_kernel walks it
// backwards over one part of the chunks (one workgroup per sequence, 64 value
// rows and part, G in fp32 MFMA accumulators; eight waves, each 16 value rows
// and half of the key columns, so each chunk's MFMA chain per wave is half as
// long as with four: config 2's backward 238 -> 232 us) and stores G at every
// chunk end.
// The recurrence is linear: a part walked from a zero adjoint gives local
// values, and the true adjoint at the end of chunk ch of part p is
// local(ch) + decay^(tokens from the end of ch to the end of p) B_p, B_p the
// true adjoint at the part's end, B_p = start(p + 1) + decay^(tokens of p + 1)
// B_(p+1), the last part starting from dL/dM_out.  bwd_adjoint_join_kernel
// forms the B_p and bwd_adjoint_fix_kernel adds those terms (parts walked in
// parallel: sequences x value tiles alone are 32 workgroups at config 4).  bwd_grad_kernel then
// takes one (sequence, chunk) per workgroup and all of its value columns, in
// 32-column tiles: dQ and dK are summed over the whole value dimension in
// registers and written once, dV tile by tile, so there are no partial sums to
// add afterwards and the chunks run in parallel.  The fp32 operands of the
// products (G, M and the decay-weighted dH of the adjoint update) enter the
// MFMAs as hi + lo pairs of 16-bit values (hi = x rounded, lo = x - hi
// rounded), two MFMAs per product, so each carries ~16 (bf16) or ~22 (f16)
// significant bits instead of 8 / 11: rounding them to one 16-bit value costs
// bf16 inputs ~1e-3 absolute error on grad_memory over a few hundred tokens.
// Wave w owns query/key block w (tokens [16w, +16)) of every per-chunk product.
constexpr int MB_DV = 32;  // value columns per tile of bwd_grad_kernel
constexpr int MB_NT = 256;
constexpr int AJ_V = 64;   // value rows per bwd_adjoint_kernel workgroup
constexpr int AJ_NT = 512; // bwd_adjoint_kernel: 8 waves, wave w owns value rows 16 (w & 3) .. + 16 and key half w >> 2

struct BwdMArgs {
  const void* dh;
  const void* dmo;
  const void* keys;
  const void* values;
  const void* queries;
  const void* memory;
  const float* states;  // [B, n_chunks, dv, dk] state after each chunk
  float* gbuf;          // [B, n_chunks, dv, dk] adjoint at each chunk's end
  float* lstart;        // [B, n_parts, dv, dk] each part's local adjoint at its start (n_parts > 1)
  void* dq_out;
  void* dk_out;
  void* dv_out;
  void* dm_out;
  int64_t batch;
  int64_t T;
  int dk;
  int dv;
  int n_chunks;
  int n_parts;          // parts of the adjoint walk
  int cpp;              // chunks per part (the last part may hold fewer)
  int mem_f32;
  int xcd_remap;
  float c;
  float pw[BCT + 1];  // decay^0 .. decay^64
};

template <int DKP>
struct AjShape {
  static constexpr int KS = DKP + 8;   // Q rows (4 banks mod 64)
  static constexpr int HS = AJ_V + 8;  // dH rows of the tile
  static constexpr int KT = DKP / 16;
  static constexpr int KU = DKP / 8;
  static constexpr int KTW = KT / 2;   // key tiles of one wave
  static constexpr int K_UNITS = BCT * KU / AJ_NT;
  static constexpr int H_UNITS = BCT * (AJ_V / 8) / AJ_NT;
  static constexpr size_t lds_bytes = static_cast<size_t>(BCT * KS + BCT * HS) * 2 + (BCT + 1) * 4;
  static_assert(K_UNITS * AJ_NT == BCT * KU && H_UNITS * AJ_NT == BCT * (AJ_V / 8), "tiles split evenly");
};

template <int DKP>
struct GrShape {
  static constexpr int KS = DKP + 8;    // K, Q and 16-bit M, G rows (4 banks mod 64)
  static constexpr int VS = MB_DV + 8;  // V, dH rows
  static constexpr int PS = BCT + 8;    // P, dS rows
  static constexpr int KT = DKP / 16;   // 16-wide key tiles
  static constexpr int NKK = DKP / 32;  // 32-deep key steps
  static constexpr int KU = DKP / 8;    // 16-byte units per K/Q row
  static constexpr int K_UNITS = BCT * KU / MB_NT;
  static constexpr int M_UNITS = MB_DV * KU / MB_NT;
  // P (before the first value tile) and dS (after the last) share the value
  // tile region: key_dim 128 fits two workgroups per CU.
  static constexpr int TILE_ELEMS = 2 * BCT * VS + 4 * MB_DV * KS;
  static_assert(TILE_ELEMS >= BCT * PS, "P / dS fit the value tile region");
  static constexpr size_t lds_bytes = static_cast<size_t>(2 * BCT * KS + TILE_ELEMS) * 2 + (BCT + 1) * 4;
  static_assert(K_UNITS * MB_NT == BCT * KU && M_UNITS * MB_NT == MB_DV * KU, "tiles split evenly");
};

template <class E>
__device__ __forceinline__ Frag8<E> bw_frag_tr(const typename ET<E>::raw* p_lo, const typename ET<E>::raw* p_hi) {
  // Four 16-bit elements of a row-major tile, transposed across each 16-lane
  // block: lane i of the block receives X[r0 + e][c0 + i] (e = 0..3) when lane
  // s of the block passes &X[r0 + (s >> 2)][c0 + 4 (s & 3)].
  typedef short s16x4 __attribute__((ext_vector_type(4)));
  typedef __attribute__((address_space(3))) s16x4 lds_s16x4;
  const s16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(p_lo));
  const s16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(p_hi));
  Frag8<E> f;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    f.e[e] = static_cast<typename ET<E>::raw>(static_cast<uint16_t>(lo[e]));
    f.e[4 + e] = static_cast<typename ET<E>::raw>(static_cast<uint16_t>(hi[e]));
  }
  return f;
}

// Four fp32 values as hi + lo 16-bit pairs: hi rounded as from_f, lo the
// rounded remainder.
template <class E>
__device__ __forceinline__ void store4_split(typename ET<E>::raw* hi, typename ET<E>::raw* lo, f32x4 v) {
  f32x4 r;
#pragma unroll
  for (int i = 0; i < 4; ++i) r[i] = v[i] - ET<E>::to_f(ET<E>::from_f(v[i]));
  store4_raw<E>(hi, v);
  store4_raw<E>(lo, r);
}

// The adjoint recurrence.  Lane (g, n) of wave w holds gacc[t][r] =
// G[v][k], v = v0 + 16 w + n, k = 16 t + 4 g + r.  Chunk staging: the loads of
// chunk ch - 1 are in flight while chunk ch is processed.
template <class E, int DKP>
__global__ __launch_bounds__(AJ_NT) void bwd_adjoint_kernel(const BwdMArgs a) {
  using S = AjShape<DKP>;
  using raw = typename ET<E>::raw;
  typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
  typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
  constexpr int KS = S::KS, HS = S::HS, KT = S::KTW, KU = S::KU;
  constexpr int ES = 2;

  extern __shared__ __align__(16) unsigned char smem[];
  raw* Qs = reinterpret_cast<raw*>(smem);  // [BCT][KS]
  raw* Hs = Qs + BCT * KS;                  // [BCT][HS] grad_hidden, the tile's value columns
  float* pw = reinterpret_cast<float*>(Hs + BCT * HS);

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int g = lane >> 4;
  const int n = lane & 15;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int vtiles = (a.dv + AJ_V - 1) / AJ_V;
  int wg = blockIdx.x;
  if (a.xcd_remap) {  // the value tiles of one sequence (same queries) on one XCD
    const int per = gridDim.x >> 3;
    wg = (wg & 7) * per + (wg >> 3);
  }
  const int tile = wg % vtiles;
  const int part = (wg / vtiles) % a.n_parts;
  const int64_t b = wg / vtiles / a.n_parts;
  const int c0 = part * a.cpp, c1 = min(a.n_chunks, c0 + a.cpp);  // chunks [c0, c1)
  const bool last_part = part == a.n_parts - 1;
  const int v0 = tile * AJ_V;
  const int dk = a.dk, dv = a.dv;
  const int64_t T = a.T;
  const int last_len = static_cast<int>(T - static_cast<int64_t>(a.n_chunks - 1) * BCT);
  const raw* queries = static_cast<const raw*>(a.queries) + b * T * dk;
  const raw* dh = static_cast<const raw*>(a.dh) + b * T * dv;
  if (tid <= BCT) pw[tid] = a.pw[tid];
  const int wr = w & 3, kt0 = KT * (w >> 2);  // value block, first key tile of this wave
  const int vrow = v0 + 16 * wr + n;
  const int64_t mem_b = a.mem_f32 ? 4 : ES;
  auto g_off = [&](int t) -> int {
    const int k = 16 * (kt0 + t) + 4 * g;
    return (vrow < dv && k < dk) ? vrow * dk + k : -1;
  };
  f32x4 gacc[KT];
  {
    // The last part's walk starts from dL/dM_out, earlier parts' from zero: a
    // zero-sized buffer for them, whose loads return zeros (no branch here; the
    // branch cost the walk its load scheduling, 72 -> 89 us at config 2).
    const __amdgpu_buffer_rsrc_t rg = make_rsrc(static_cast<const unsigned char*>(a.dmo) + b * dv * dk * mem_b,
                                                last_part ? static_cast<uint32_t>(dv * dk * mem_b) : 0u);
#pragma unroll
    for (int t = 0; t < KT; ++t) {
      const int off = g_off(t);
      if (a.mem_f32) {
        const u32x4 u = __builtin_amdgcn_raw_buffer_load_b128(rg, off < 0 ? kBufOOB : off * 4, 0, 0);
#pragma unroll
        for (int i = 0; i < 4; ++i) gacc[t][i] = __uint_as_float(u[i]);
      } else {
        const u32x2 u = __builtin_amdgcn_raw_buffer_load_b64(rg, off < 0 ? kBufOOB : off * ES, 0, 0);
        gacc[t][0] = ET<E>::to_f(static_cast<raw>(u[0] & 0xffffu));
        gacc[t][1] = ET<E>::to_f(static_cast<raw>(u[0] >> 16));
        gacc[t][2] = ET<E>::to_f(static_cast<raw>(u[1] & 0xffffu));
        gacc[t][3] = ET<E>::to_f(static_cast<raw>(u[1] >> 16));
      }
    }
  }
  __syncthreads();  // pw
  // decay^{i+1} of the token slots i = 32p + 16 (s / 4) + 4g + s % 4
  float gw[2][8];
#pragma unroll
  for (int p = 0; p < 2; ++p)
#pragma unroll
    for (int s = 0; s < 8; ++s) gw[p][s] = pw[32 * p + 16 * (s >> 2) + 4 * g + (s & 3) + 1];

  struct Stage {
    U8<E> q[S::K_UNITS];
    U8<E> h[S::H_UNITS];
  };
  auto load_chunk = [&](int ch, Stage& sg) {
    const int64_t t0 = static_cast<int64_t>(ch) * BCT;
    const int L = ch == a.n_chunks - 1 ? last_len : BCT;
    const __amdgpu_buffer_rsrc_t rq = make_rsrc(queries + t0 * dk, static_cast<uint32_t>(L * dk * ES));
    const __amdgpu_buffer_rsrc_t rh = make_rsrc(dh + t0 * dv, static_cast<uint32_t>(L * dv * ES));
#pragma unroll
    for (int u = 0; u < S::K_UNITS; ++u) {
      const int l = tid + AJ_NT * u;
      const int row = l / KU, col = 8 * (l % KU);
      sg.q[u] = buf_load8<E>(rq, col < dk ? (row * dk + col) * ES : kBufOOB);
    }
#pragma unroll
    for (int u = 0; u < S::H_UNITS; ++u) {
      const int l = tid + AJ_NT * u;
      const int row = l / (AJ_V / 8), col = 8 * (l % (AJ_V / 8));
      sg.h[u] = buf_load8<E>(rh, v0 + col < dv ? (row * dv + v0 + col) * ES : kBufOOB);
    }
  };
  auto store_chunk = [&](const Stage& sg) {
#pragma unroll
    for (int u = 0; u < S::K_UNITS; ++u) {
      const int l = tid + AJ_NT * u;
      *reinterpret_cast<U8<E>*>(Qs + (l / KU) * KS + 8 * (l % KU)) = sg.q[u];
    }
#pragma unroll
    for (int u = 0; u < S::H_UNITS; ++u) {
      const int l = tid + AJ_NT * u;
      *reinterpret_cast<U8<E>*>(Hs + (l / (AJ_V / 8)) * HS + 8 * (l % (AJ_V / 8))) = sg.h[u];
    }
  };

  // (Loading two chunks ahead, in two register stages, measured slower: 84
  // against 71 us at config 2.)
  Stage stage;
  load_chunk(c1 - 1, stage);
  for (int ch = c1 - 1; ch >= c0; --ch) {
    const int L = ch == a.n_chunks - 1 ? last_len : BCT;
    store_chunk(stage);
    if (ch > c0) load_chunk(ch - 1, stage);
    __syncthreads();  // chunk in LDS
    {
      // the adjoint at this chunk's end, for bwd_grad_kernel
      const __amdgpu_buffer_rsrc_t rs =
          make_rsrc(a.gbuf + (b * a.n_chunks + ch) * dv * dk, static_cast<uint32_t>(dv * dk * 4));
#pragma unroll
      for (int t = 0; t < KT; ++t) {
        const int off = g_off(t);
        buf_store4<F32>(rs, off < 0 ? kBufOOB : off * 4, gacc[t]);
      }
    }
    Frag8<E> hw[2], hwl[2];
#pragma unroll
    for (int p = 0; p < 2; ++p) {
      const raw* hb = Hs + (32 * p + 4 * g + (n >> 2)) * HS + 16 * wr + 4 * (n & 3);
      const Frag8<E> h = bw_frag_tr<E>(hb, hb + 16 * HS);
#pragma unroll
      for (int s = 0; s < 8; ++s) {
        const float x = ET<E>::to_f(h.e[s]) * gw[p][s];
        hw[p].e[s] = ET<E>::from_f(x);
        hwl[p].e[s] = ET<E>::from_f(x - ET<E>::to_f(hw[p].e[s]));
      }
    }
    const float decay_L = pw[L];
#pragma unroll
    for (int t = 0; t < KT; ++t) {
      f32x4 acc = gacc[t] * decay_L;
#pragma unroll
      for (int p = 0; p < 2; ++p) {
        const raw* qb = Qs + (32 * p + 4 * g + (n >> 2)) * KS + 16 * (kt0 + t) + 4 * (n & 3);
        const Frag8<E> qT = bw_frag_tr<E>(qb, qb + 16 * KS);
        acc = mfma8(qT, hw[p], acc);
        acc = mfma8(qT, hwl[p], acc);
      }
      gacc[t] = acc;
    }
    __syncthreads();  // every read of this chunk's tiles done
  }
  if (a.n_parts > 1) {
    // the part's local adjoint at its start, for bwd_adjoint_fix_kernel
    const __amdgpu_buffer_rsrc_t rl =
        make_rsrc(a.lstart + (b * a.n_parts + part) * dv * dk, static_cast<uint32_t>(dv * dk * 4));
#pragma unroll
    for (int t = 0; t < KT; ++t) {
      const int off = g_off(t);
      buf_store4<F32>(rl, off < 0 ? kBufOOB : off * 4, gacc[t]);
    }
    return;
  }
  // grad_memory: the adjoint at the sequence's start.
  const __amdgpu_buffer_rsrc_t ro = make_rsrc(static_cast<unsigned char*>(a.dm_out) + b * dv * dk * mem_b,
                                              static_cast<uint32_t>(dv * dk * mem_b));
#pragma unroll
  for (int t = 0; t < KT; ++t) {
    const int off = g_off(t);
    if (a.mem_f32) {
      buf_store4<F32>(ro, off < 0 ? kBufOOB : off * 4, gacc[t]);
    } else {
      buf_store4<E>(ro, off < 0 ? kBufOOB : off * ES, gacc[t]);
    }
  }
}

// The walked parts joined (n_parts > 1), two launches.  Thread t of a
// workgroup owns float4 columns of one 64-row value tile; no LDS.
struct AjTile {
  static constexpr int UMAX = AJ_V * 128 / 4 / MB_NT;  // float4 units per thread at key_dim 128
  int off[UMAX];
  __device__ AjTile(int v0, int dv, int dk) {
    const int qpr = dk / 4;  // dk is a multiple of 8
#pragma unroll
    for (int i = 0; i < UMAX; ++i) {
      const int u = threadIdx.x + MB_NT * i;
      const int v = v0 + u / qpr;
      off[i] = (u < AJ_V * qpr && v < dv) ? v * dk + 4 * (u % qpr) : -1;
    }
  }
  __device__ float4 ld(const float* base, int i) const {
    return off[i] < 0 ? make_float4(0.f, 0.f, 0.f, 0.f) : *reinterpret_cast<const float4*>(base + off[i]);
  }
};

__device__ __forceinline__ float4 axpy4(float4 x, float f, float4 y) {  // x + f y
  return make_float4(x.x + f * y.x, x.y + f * y.y, x.z + f * y.z, x.w + f * y.w);
}

// Join: workgroup (sequence, value tile) turns the local starts into the parts'
// boundary adjoints in place, slot p + 1 := B_p = start(p + 1) + decay^(64 cpp)
// B_(p+1) for p = n_parts - 3 .. 0 (slot n_parts - 1 already is B_(n_parts-2):
// the last part started from dL/dM_out), then writes grad_memory = start(0) +
// decay^(64 cpp) B_0.  Every part but the last holds cpp full chunks.
__global__ __launch_bounds__(MB_NT) void bwd_adjoint_join_kernel(const BwdMArgs a, int mem_dtype) {
  const int vtiles = (a.dv + AJ_V - 1) / AJ_V;
  const int tile = blockIdx.x % vtiles;
  const int64_t b = blockIdx.x / vtiles;
  const int dk = a.dk, dv = a.dv;
  const AjTile tl(tile * AJ_V, dv, dk);
  float f = 1.f;
  for (int c = 0; c < a.cpp; ++c) f *= a.pw[BCT];
  float* ls = a.lstart + b * a.n_parts * dv * dk;
  float4 bt[AjTile::UMAX];
#pragma unroll
  for (int i = 0; i < AjTile::UMAX; ++i) bt[i] = tl.ld(ls + (a.n_parts - 1) * dv * dk, i);
  for (int q = a.n_parts - 2; q >= 1; --q) {
#pragma unroll
    for (int i = 0; i < AjTile::UMAX; ++i) {
      bt[i] = axpy4(tl.ld(ls + q * dv * dk, i), f, bt[i]);
      if (tl.off[i] >= 0) *reinterpret_cast<float4*>(ls + q * dv * dk + tl.off[i]) = bt[i];
    }
  }
  unsigned char* dm = static_cast<unsigned char*>(a.dm_out) + b * dv * dk * (a.mem_f32 ? 4 : 2);
#pragma unroll
  for (int i = 0; i < AjTile::UMAX; ++i) {
    if (tl.off[i] < 0) continue;
    const float4 y = axpy4(tl.ld(ls, i), f, bt[i]);
    if (a.mem_f32) {
      *reinterpret_cast<float4*>(reinterpret_cast<float*>(dm) + tl.off[i]) = y;
    } else {
      uint16_t* o = reinterpret_cast<uint16_t*>(dm) + tl.off[i];
      if (mem_dtype == GRM_HIP_F16) {
        o[0] = ET<F16>::from_f(y.x); o[1] = ET<F16>::from_f(y.y); o[2] = ET<F16>::from_f(y.z); o[3] = ET<F16>::from_f(y.w);
      } else {
        o[0] = ET<BF16>::from_f(y.x); o[1] = ET<BF16>::from_f(y.y); o[2] = ET<BF16>::from_f(y.z); o[3] = ET<BF16>::from_f(y.w);
      }
    }
  }
}

// Fix-up: workgroup (sequence, value tile, chunk ch of parts 0 .. n_parts - 2)
// adds decay^(64 (c1 - 1 - ch)) B_p to the adjoint stored at the end of ch
// (part p = ch / cpp ends at chunk c1 - 1 = (p + 1) cpp - 1; B_p in slot p + 1).
__global__ __launch_bounds__(MB_NT) void bwd_adjoint_fix_kernel(const BwdMArgs a) {
  const int vtiles = (a.dv + AJ_V - 1) / AJ_V;
  const int nfix = (a.n_parts - 1) * a.cpp;
  const int tile = blockIdx.x % vtiles;
  const int ch = (blockIdx.x / vtiles) % nfix;
  const int64_t b = blockIdx.x / vtiles / nfix;
  const int dk = a.dk, dv = a.dv;
  const int part = ch / a.cpp;
  const AjTile tl(tile * AJ_V, dv, dk);
  float f = 1.f;
  for (int c = ch; c < (part + 1) * a.cpp - 1; ++c) f *= a.pw[BCT];
  const float* bp = a.lstart + (b * a.n_parts + part + 1) * dv * dk;
  float* gb = a.gbuf + (b * a.n_chunks + ch) * dv * dk;
  float4 x[AjTile::UMAX], y[AjTile::UMAX];
#pragma unroll
  for (int i = 0; i < AjTile::UMAX; ++i) {
    x[i] = tl.ld(gb, i);
    y[i] = tl.ld(bp, i);
  }
#pragma unroll
  for (int i = 0; i < AjTile::UMAX; ++i)
    if (tl.off[i] >= 0) *reinterpret_cast<float4*>(gb + tl.off[i]) = axpy4(x[i], f, y[i]);
}

// The gradients of one chunk from its starting state and the adjoint at its end.
template <class E, int DKP>
__global__ __launch_bounds__(MB_NT, 2) void bwd_grad_kernel(const BwdMArgs a) {
  using S = GrShape<DKP>;
  using raw = typename ET<E>::raw;
  typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
  constexpr int KS = S::KS, VS = S::VS, PS = S::PS, KT = S::KT, NKK = S::NKK, KU = S::KU;
  constexpr int ES = 2;

  extern __shared__ __align__(16) unsigned char smem[];
  raw* Ks = reinterpret_cast<raw*>(smem);  // [BCT][KS]
  raw* Qs = Ks + BCT * KS;                  // [BCT][KS]
  raw* Vs = Qs + BCT * KS;                  // [BCT][VS] value tile columns
  raw* Hs = Vs + BCT * VS;                  // [BCT][VS] grad_hidden tile columns
  raw* Ms = Hs + BCT * VS;                  // [MB_DV][KS] the chunk's starting state, hi
  raw* Ml = Ms + MB_DV * KS;                // [MB_DV][KS] ... lo
  raw* Gs = Ml + MB_DV * KS;                // [MB_DV][KS] adjoint at the chunk's end, hi
  raw* Gl = Gs + MB_DV * KS;                // [MB_DV][KS] ... lo
  raw* Ps = Vs;                             // [BCT][PS] P, before the first value tile
  raw* Ds = Vs;                             // [BCT][PS] dS, after the last
  float* pw = reinterpret_cast<float*>(Qs + BCT * KS + S::TILE_ELEMS);

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int g = lane >> 4;
  const int n = lane & 15;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int ch = static_cast<int>(blockIdx.x % static_cast<unsigned>(a.n_chunks));
  const int64_t b = blockIdx.x / static_cast<unsigned>(a.n_chunks);
  const int dk = a.dk, dv = a.dv;
  const int64_t T = a.T;
  const int64_t t0 = static_cast<int64_t>(ch) * BCT;
  const int L = ch == a.n_chunks - 1 ? static_cast<int>(T - t0) : BCT;
  const float c = a.c;
  const bool f32m = a.mem_f32 != 0;
  const raw* keys = static_cast<const raw*>(a.keys) + (b * T + t0) * dk;
  const raw* queries = static_cast<const raw*>(a.queries) + (b * T + t0) * dk;
  const raw* values = static_cast<const raw*>(a.values) + (b * T + t0) * dv;
  const raw* dh = static_cast<const raw*>(a.dh) + (b * T + t0) * dv;
  if (tid <= BCT) pw[tid] = a.pw[tid];
  {
    const __amdgpu_buffer_rsrc_t rk = make_rsrc(keys, static_cast<uint32_t>(L * dk * ES));
    const __amdgpu_buffer_rsrc_t rq = make_rsrc(queries, static_cast<uint32_t>(L * dk * ES));
    U8<E> kx[S::K_UNITS], qx[S::K_UNITS];
#pragma unroll
    for (int u = 0; u < S::K_UNITS; ++u) {
      const int l = tid + MB_NT * u;
      const int row = l / KU, col = 8 * (l % KU);
      const int off = col < dk ? (row * dk + col) * ES : kBufOOB;
      kx[u] = buf_load8<E>(rk, off);
      qx[u] = buf_load8<E>(rq, off);
    }
#pragma unroll
    for (int u = 0; u < S::K_UNITS; ++u) {
      const int l = tid + MB_NT * u;
      const int row = l / KU, col = 8 * (l % KU);
      *reinterpret_cast<U8<E>*>(Ks + row * KS + col) = kx[u];
      *reinterpret_cast<U8<E>*>(Qs + row * KS + col) = qx[u];
    }
  }

  // Value tile staging: V / dH unit of thread t is row t / 4, columns 8 (t % 4)
  // of the tile; state / adjoint unit u is row (t + 256 u) / KU of the tile, 8
  // key columns (fp32, or 16-bit in m[u][0] for a 16-bit initial memory).
  struct Stage {
    U8<E> v, h;
    u32x4 m[S::M_UNITS][2];
    u32x4 gg[S::M_UNITS][2];
  };
  const unsigned char* msrc = ch == 0 ? static_cast<const unsigned char*>(a.memory) + b * dv * dk * (f32m ? 4 : ES)
                                      : reinterpret_cast<const unsigned char*>(
                                            a.states + (b * a.n_chunks + ch - 1) * dv * dk);
  const bool m32 = ch != 0 || f32m;
  const __amdgpu_buffer_rsrc_t rm = make_rsrc(msrc, static_cast<uint32_t>(dv * dk * (m32 ? 4 : ES)));
  const __amdgpu_buffer_rsrc_t rg =
      make_rsrc(a.gbuf + (b * a.n_chunks + ch) * dv * dk, static_cast<uint32_t>(dv * dk * 4));
  const __amdgpu_buffer_rsrc_t rv = make_rsrc(values, static_cast<uint32_t>(L * dv * ES));
  const __amdgpu_buffer_rsrc_t rh = make_rsrc(dh, static_cast<uint32_t>(L * dv * ES));
  auto load_vtile = [&](int vt, Stage& sg) {
    const int v0 = vt * MB_DV;
    const int off = ((tid >> 2) * dv + v0 + 8 * (tid & 3)) * ES;
    sg.v = buf_load8<E>(rv, off);
    sg.h = buf_load8<E>(rh, off);
#pragma unroll
    for (int u = 0; u < S::M_UNITS; ++u) {
      const int l = tid + MB_NT * u;
      const int row = l / KU, col = 8 * (l % KU);
      const int el = col < dk ? (v0 + row) * dk + col : -1;
      if (m32) {
        sg.m[u][0] = __builtin_amdgcn_raw_buffer_load_b128(rm, el < 0 ? kBufOOB : el * 4, 0, 0);
        sg.m[u][1] = __builtin_amdgcn_raw_buffer_load_b128(rm, el < 0 ? kBufOOB : el * 4 + 16, 0, 0);
      } else {
        sg.m[u][0] = __builtin_amdgcn_raw_buffer_load_b128(rm, el < 0 ? kBufOOB : el * ES, 0, 0);
      }
      sg.gg[u][0] = __builtin_amdgcn_raw_buffer_load_b128(rg, el < 0 ? kBufOOB : el * 4, 0, 0);
      sg.gg[u][1] = __builtin_amdgcn_raw_buffer_load_b128(rg, el < 0 ? kBufOOB : el * 4 + 16, 0, 0);
    }
  };
  auto split8 = [&](raw* hi, raw* lo, const u32x4* x) {
    f32x4 x0, x1;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      x0[i] = __uint_as_float(x[0][i]);
      x1[i] = __uint_as_float(x[1][i]);
    }
    store4_split<E>(hi, lo, x0);
    store4_split<E>(hi + 4, lo + 4, x1);
  };
  auto store_vtile = [&](const Stage& sg) {
    *reinterpret_cast<U8<E>*>(Vs + (tid >> 2) * VS + 8 * (tid & 3)) = sg.v;
    *reinterpret_cast<U8<E>*>(Hs + (tid >> 2) * VS + 8 * (tid & 3)) = sg.h;
#pragma unroll
    for (int u = 0; u < S::M_UNITS; ++u) {
      const int l = tid + MB_NT * u;
      const int o = (l / KU) * KS + 8 * (l % KU);
      if (m32) {
        split8(Ms + o, Ml + o, sg.m[u]);
      } else {
        *reinterpret_cast<U8<E>*>(Ms + o) = __builtin_bit_cast(U8<E>, sg.m[u][0]);
        *reinterpret_cast<uint4*>(Ml + o) = make_uint4(0u, 0u, 0u, 0u);
      }
      split8(Gs + o, Gl + o, sg.gg[u]);
    }
  };

  Stage stage;
  load_vtile(0, stage);
  __syncthreads();  // K, Q, pw

  // Causal coefficients c decay^{i-j} of this wave's P / dS rows i = 16w + n
  // against keys j = 16 jb + 4g + r (read from LDS where used).
  auto coef4 = [&](int jb) {
    f32x4 cf;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int i = 16 * w + n, j = 16 * jb + 4 * g + r;
      cf[r] = (j <= i) ? c * pw[max(i - j, 0)] : 0.f;
    }
    return cf;
  };
  const int jrow = 16 * w + n;  // this lane's key / query row
  const float sq = pw[jrow + 1];
  const float wl = (jrow < L) ? c * pw[max(L - 1 - jrow, 0)] : 0.f;

  // ---- P rows of query block w (blocks right of the diagonal are zeros)
  {
    Frag8<E> qf[NKK];
#pragma unroll
    for (int kk = 0; kk < NKK; ++kk)
      qf[kk] = *reinterpret_cast<const Frag8<E>*>(Qs + jrow * KS + 32 * kk + 8 * g);
#pragma unroll
    for (int jb = 0; jb < 4; ++jb) {
      f32x4 sacc = f32x4{0.f, 0.f, 0.f, 0.f};
      if (jb <= w) {
#pragma unroll
        for (int kk = 0; kk < NKK; ++kk) {
          const Frag8<E> kf = *reinterpret_cast<const Frag8<E>*>(Ks + (16 * jb + n) * KS + 32 * kk + 8 * g);
          sacc = mfma8(kf, qf[kk], sacc);
        }
      }
      store4_raw<E>(Ps + jrow * PS + 16 * jb + 4 * g, sacc * coef4(jb));
    }
  }
  __syncthreads();  // P complete
  // Columns j = 16w + n of P: lane n holds rows i = 32p + 4g + e (+16).
  Frag8<E> pT[2];
#pragma unroll
  for (int p = 0; p < 2; ++p) {
    const int off = (32 * p + 4 * g + (n >> 2)) * PS + 16 * w + 4 * (n & 3);
    pT[p] = bw_frag_tr<E>(Ps + off, Ps + off + 16 * PS);
  }
  __syncthreads();  // P read: the region takes the value tiles

  f32x4 dsacc[4], dq[KT], dkk[KT];
#pragma unroll
  for (int jb = 0; jb < 4; ++jb) dsacc[jb] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int kt = 0; kt < KT; ++kt) dq[kt] = dkk[kt] = f32x4{0.f, 0.f, 0.f, 0.f};
  const __amdgpu_buffer_rsrc_t rdv = make_rsrc(static_cast<raw*>(a.dv_out) + (b * T + t0) * dv,
                                               static_cast<uint32_t>(L * dv * ES));
  const int n_vt = dv / MB_DV;
  for (int vt = 0; vt < n_vt; ++vt) {
    store_vtile(stage);
    if (vt + 1 < n_vt) load_vtile(vt + 1, stage);
    __syncthreads();  // value tile in LDS
    // dS rows of block w, this tile's share of the sum over value columns
    {
      const Frag8<E> hf = *reinterpret_cast<const Frag8<E>*>(Hs + jrow * VS + 8 * g);
#pragma unroll
      for (int jb = 0; jb < 4; ++jb) {
        if (jb <= w) {
          const Frag8<E> vfj = *reinterpret_cast<const Frag8<E>*>(Vs + (16 * jb + n) * VS + 8 * g);
          dsacc[jb] = mfma8(vfj, hf, dsacc[jb]);
        }
      }
    }
    // dQ (sum_v dH[i][v] M[v][k]) and dK (sum_v G[v][k] V[j][v]) over this tile
    {
      const Frag8<E> hq = lds_frag_4x2<E>(Hs + jrow * VS + 4 * g, Hs + jrow * VS + 4 * g + 16);
      const Frag8<E> vj = lds_frag_4x2<E>(Vs + jrow * VS + 4 * g, Vs + jrow * VS + 4 * g + 16);
#pragma unroll
      for (int kt = 0; kt < KT; ++kt) {
        const int mo = (4 * g + (n >> 2)) * KS + 16 * kt + 4 * (n & 3);
        dq[kt] = mfma8(bw_frag_tr<E>(Ms + mo, Ms + mo + 16 * KS), hq, dq[kt]);
        dq[kt] = mfma8(bw_frag_tr<E>(Ml + mo, Ml + mo + 16 * KS), hq, dq[kt]);
        dkk[kt] = mfma8(bw_frag_tr<E>(Gs + mo, Gs + mo + 16 * KS), vj, dkk[kt]);
        dkk[kt] = mfma8(bw_frag_tr<E>(Gl + mo, Gl + mo + 16 * KS), vj, dkk[kt]);
      }
    }
    // dV rows of block w for this tile: c decay^{L-1-j} sum_k G[v][k] K[j][k] + sum_i dH[i][v] P[i][j]
    {
      const int v0 = vt * MB_DV;
#pragma unroll
      for (int vb = 0; vb < 2; ++vb) {
        f32x4 acc = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int kk = 0; kk < NKK; ++kk) {
          const int go = (16 * vb + n) * KS + 32 * kk + 8 * g;
          const Frag8<E> kr = *reinterpret_cast<const Frag8<E>*>(Ks + jrow * KS + 32 * kk + 8 * g);
          acc = mfma8(*reinterpret_cast<const Frag8<E>*>(Gs + go), kr, acc);
          acc = mfma8(*reinterpret_cast<const Frag8<E>*>(Gl + go), kr, acc);
        }
        acc *= wl;
#pragma unroll
        for (int p = 0; p < 2; ++p) {
          if (32 * p + 31 < 16 * w) continue;
          const raw* hb = Hs + (32 * p + 4 * g + (n >> 2)) * VS + 16 * vb + 4 * (n & 3);
          acc = mfma8(bw_frag_tr<E>(hb, hb + 16 * VS), pT[p], acc);
        }
        buf_store4<E>(rdv, (jrow * dv + v0 + 16 * vb + 4 * g) * ES, acc);
      }
    }
    __syncthreads();  // every read of this tile done
  }

  // ---- dS complete: c (dH V^T) o D, rounded to the MFMA type like P
#pragma unroll
  for (int jb = 0; jb < 4; ++jb) store4_raw<E>(Ds + jrow * PS + 16 * jb + 4 * g, dsacc[jb] * coef4(jb));
  __syncthreads();
  // ---- dQ rows of block w: decay^{i+1} sum_v dH M + sum_j dS[i][j] K[j][k]
  {
    const __amdgpu_buffer_rsrc_t rqo = make_rsrc(static_cast<raw*>(a.dq_out) + (b * T + t0) * dk,
                                                 static_cast<uint32_t>(L * dk * ES));
    Frag8<E> dsf[2];
#pragma unroll
    for (int p = 0; p < 2; ++p)
      dsf[p] = lds_frag_4x2<E>(Ds + jrow * PS + 32 * p + 4 * g, Ds + jrow * PS + 32 * p + 4 * g + 16);
#pragma unroll
    for (int kt = 0; kt < KT; ++kt) {
      f32x4 acc = dq[kt] * sq;
#pragma unroll
      for (int p = 0; p < 2; ++p) {
        if (32 * p > 16 * w + 15) continue;
        const raw* kb = Ks + (32 * p + 4 * g + (n >> 2)) * KS + 16 * kt + 4 * (n & 3);
        acc = mfma8(bw_frag_tr<E>(kb, kb + 16 * KS), dsf[p], acc);
      }
      const int kc = 16 * kt + 4 * g;
      buf_store4<E>(rqo, kc < dk ? (jrow * dk + kc) * ES : kBufOOB, acc);
    }
  }
  // ---- dK rows of block w: c decay^{L-1-j} sum_v G V + sum_i Q[i][k] dS[i][j]
  {
    const __amdgpu_buffer_rsrc_t rko = make_rsrc(static_cast<raw*>(a.dk_out) + (b * T + t0) * dk,
                                                 static_cast<uint32_t>(L * dk * ES));
    Frag8<E> dsT[2];
#pragma unroll
    for (int p = 0; p < 2; ++p) {
      const int off = (32 * p + 4 * g + (n >> 2)) * PS + 16 * w + 4 * (n & 3);
      dsT[p] = bw_frag_tr<E>(Ds + off, Ds + off + 16 * PS);
    }
#pragma unroll
    for (int kt = 0; kt < KT; ++kt) {
      f32x4 acc = dkk[kt] * wl;
#pragma unroll
      for (int p = 0; p < 2; ++p) {
        if (32 * p + 31 < 16 * w) continue;
        const raw* qb = Qs + (32 * p + 4 * g + (n >> 2)) * KS + 16 * kt + 4 * (n & 3);
        acc = mfma8(bw_frag_tr<E>(qb, qb + 16 * KS), dsT[p], acc);
      }
      const int kc = 16 * kt + 4 * g;
      buf_store4<E>(rko, kc < dk ? (jrow * dk + kc) * ES : kBufOOB, acc);
    }
  }
}

template <class K>
int allow_lds(K* fn, size_t bytes, bool& done) {
  if (done || bytes <= 64 * 1024) return GRM_HIP_OK;
  hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(fn), hipFuncAttributeMaxDynamicSharedMemorySize,
                                     static_cast<int>(bytes));
  if (e != hipSuccess) {
    set_error("chunk_update_bwd: hipFuncSetAttribute failed: %s", hipGetErrorString(e));
    return static_cast<int>(e);
  }
  done = true;
  return GRM_HIP_OK;
}

template <class E, int DKP>
int launch_bwd_mfma(BwdMArgs a, int mem_dtype, hipStream_t s) {
  static bool attr_a = false, attr_g = false;
  int rc = allow_lds(&bwd_adjoint_kernel<E, DKP>, AjShape<DKP>::lds_bytes, attr_a);
  if (rc == GRM_HIP_OK) rc = allow_lds(&bwd_grad_kernel<E, DKP>, GrShape<DKP>::lds_bytes, attr_g);
  if (rc != GRM_HIP_OK) return rc;
  const int64_t grid_a = a.batch * ((a.dv + AJ_V - 1) / AJ_V) * a.n_parts;
  a.xcd_remap = (grid_a % 8 == 0) ? 1 : 0;
  hipLaunchKernelGGL((bwd_adjoint_kernel<E, DKP>), dim3(static_cast<unsigned>(grid_a)), dim3(AJ_NT),
                     AjShape<DKP>::lds_bytes, s, a);
  rc = check_launch("chunk_update_bwd(adjoint)");
  if (rc != GRM_HIP_OK) return rc;
  if (a.n_parts > 1) {
    const int64_t vt = (a.dv + AJ_V - 1) / AJ_V;
    hipLaunchKernelGGL(bwd_adjoint_join_kernel, dim3(static_cast<unsigned>(a.batch * vt)), dim3(MB_NT), 0, s, a,
                       mem_dtype);
    rc = check_launch("chunk_update_bwd(adjoint join)");
    if (rc != GRM_HIP_OK) return rc;
    const int64_t grid_f = a.batch * vt * (a.n_parts - 1) * a.cpp;
    hipLaunchKernelGGL(bwd_adjoint_fix_kernel, dim3(static_cast<unsigned>(grid_f)), dim3(MB_NT), 0, s, a);
    rc = check_launch("chunk_update_bwd(adjoint fix-up)");
    if (rc != GRM_HIP_OK) return rc;
  }
  const int64_t grid_g = a.batch * a.n_chunks;
  hipLaunchKernelGGL((bwd_grad_kernel<E, DKP>), dim3(static_cast<unsigned>(grid_g)), dim3(MB_NT),
                     GrShape<DKP>::lds_bytes, s, a);
  return check_launch("chunk_update_bwd(gradients)");
}

}  // namespace
}  // namespace grmhip

using namespace grmhip;

namespace {
bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }
}  // namespace

extern "C" int grm_hip_chunk_update_bwd(const void* grad_hidden, const void* grad_memory_out,
                                        const void* keys, const void* values, const void* queries,
                                        const void* memory, void* grad_keys, void* grad_values,
                                        void* grad_queries, void* grad_memory, float* chunk_states,
                                        int states_given, float* dkq_partial, int64_t batch, int64_t seq_len,
                                        int64_t key_dim, int64_t value_dim, int in_dtype,
                                        int mem_dtype, double memory_decay, void* stream) {
  if (batch < 0 || seq_len < 0 || key_dim < 1 || value_dim < 1) {
    set_error("chunk_update_bwd: bad sizes");
    return GRM_HIP_EINVAL;
  }
  if (in_dtype < GRM_HIP_F32 || in_dtype > GRM_HIP_BF16 ||
      (mem_dtype != GRM_HIP_F32 && mem_dtype != in_dtype)) {
    set_error("chunk_update_bwd: unsupported dtypes in=%d mem=%d", in_dtype, mem_dtype);
    return GRM_HIP_EUNSUPPORTED;
  }
  if (key_dim > 256 || (in_dtype == GRM_HIP_F32 && key_dim > 128)) {
    set_error("chunk_update_bwd: key_dim %lld exceeds %d for this dtype", (long long)key_dim,
              in_dtype == GRM_HIP_F32 ? 128 : 256);
    return GRM_HIP_EUNSUPPORTED;
  }
  if (!std::isfinite(memory_decay)) {
    set_error("chunk_update_bwd: memory_decay is not finite");
    return GRM_HIP_EINVAL;
  }
  if (batch == 0) return GRM_HIP_OK;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const size_t mem_b = (mem_dtype == GRM_HIP_F32) ? 4 : 2;
  if (grad_memory_out == nullptr || grad_memory == nullptr) {
    set_error("chunk_update_bwd: null pointer");
    return GRM_HIP_EINVAL;
  }
  if (seq_len == 0) {
    hipError_t e = hipMemcpyAsync(grad_memory, grad_memory_out, batch * value_dim * key_dim * mem_b,
                                  hipMemcpyDeviceToDevice, s);
    if (e != hipSuccess) {
      set_error("chunk_update_bwd: hipMemcpyAsync failed: %s", hipGetErrorString(e));
      return static_cast<int>(e);
    }
    return GRM_HIP_OK;
  }
  if (grad_hidden == nullptr || keys == nullptr || values == nullptr || queries == nullptr ||
      memory == nullptr || grad_keys == nullptr || grad_values == nullptr ||
      grad_queries == nullptr || chunk_states == nullptr || dkq_partial == nullptr) {
    set_error("chunk_update_bwd: null pointer");
    return GRM_HIP_EINVAL;
  }
  const int64_t n_chunks = (seq_len + BCT - 1) / BCT;
  const int tiles = static_cast<int>((value_dim + RB - 1) / RB);
  if (batch * tiles > INT32_MAX || n_chunks > INT32_MAX) {
    set_error("chunk_update_bwd: problem too large for one launch");
    return GRM_HIP_EINVAL;
  }
  // Without the forward's chunk states, run the forward again to store the
  // state after every 64-token chunk; its hidden output and final state are not needed.
  if (!states_given) {
    const int rc = grm_hip_chunk_update_fwd(keys, values, queries, memory, nullptr, nullptr, chunk_states,
                                            nullptr, 0, batch, seq_len, key_dim, value_dim, in_dtype,
                                            mem_dtype, memory_decay, BCT, stream);
    if (rc != GRM_HIP_OK) return rc;
  }

  const char* env = getenv("GRM_HIP_BWD_MFMA");
  // The MFMA kernels keep the adjoint at every chunk end, [batch, n_chunks,
  // value_dim, key_dim] float32, in dkq_partial: used where that fits the
  // buffer's documented size (from about ten tokens on; shorter sequences take
  // the scalar kernel).
  const bool gbuf_fits = n_chunks * value_dim <= 2 * ((value_dim + RB - 1) / RB) * seq_len;
  const bool mfma = (env == nullptr || env[0] != '0') && (in_dtype == GRM_HIP_BF16 || in_dtype == GRM_HIP_F16) &&
                    key_dim <= 128 && key_dim % 8 == 0 && value_dim % MB_DV == 0 && gbuf_fits &&
                    batch * n_chunks <= INT32_MAX &&
                    aligned16(grad_hidden) && aligned16(keys) && aligned16(values) && aligned16(queries) &&
                    aligned16(grad_values) && aligned16(dkq_partial) && aligned16(memory) &&
                    aligned16(grad_memory_out) && aligned16(grad_memory) && aligned16(chunk_states);
  if (mfma) {
    BwdMArgs m;
    memset(&m, 0, sizeof(m));
    m.dh = grad_hidden;
    m.dmo = grad_memory_out;
    m.keys = keys;
    m.values = values;
    m.queries = queries;
    m.memory = memory;
    m.states = chunk_states;
    m.gbuf = dkq_partial;
    // Parts of the adjoint walk when sequences x value tiles are fewer than 128
    // workgroups: enough for the chip (about 256), at least 4 chunks a part,
    // their local starts after the chunk-end adjoints in dkq_partial (within its
    // documented size).  (At config 2, 128 workgroups, two parts plus the join
    // took longer than one walk.)
    {
      const int64_t vt = (value_dim + AJ_V - 1) / AJ_V;
      int64_t parts = batch * vt >= 128 ? 1 : std::min<int64_t>((256 + batch * vt - 1) / (batch * vt), n_chunks / 4);
      parts = std::max<int64_t>(parts, 1);
      const int64_t cpp = (n_chunks + parts - 1) / parts;
      parts = (n_chunks + cpp - 1) / cpp;
      const bool fits = (n_chunks + parts) * value_dim <= 2 * ((value_dim + RB - 1) / RB) * seq_len &&
                        batch * vt * n_chunks <= INT32_MAX;
      const char* penv = getenv("GRM_HIP_BWD_PARTS");
      m.n_parts = (fits && (penv == nullptr || penv[0] != '0')) ? static_cast<int>(parts) : 1;
      m.cpp = m.n_parts > 1 ? static_cast<int>(cpp) : static_cast<int>(n_chunks);
      m.lstart = dkq_partial + batch * n_chunks * value_dim * key_dim;
    }
    m.dq_out = grad_queries;
    m.dk_out = grad_keys;
    m.dv_out = grad_values;
    m.dm_out = grad_memory;
    m.batch = batch;
    m.T = seq_len;
    m.dk = static_cast<int>(key_dim);
    m.dv = static_cast<int>(value_dim);
    m.n_chunks = static_cast<int>(n_chunks);
    m.mem_f32 = mem_dtype == GRM_HIP_F32;
    m.c = static_cast<float>((1.0 - memory_decay) / std::sqrt(static_cast<double>(key_dim)));
    for (int i = 0; i <= BCT; ++i) m.pw[i] = static_cast<float>(std::pow(memory_decay, i));
    if (in_dtype == GRM_HIP_F16) {
      return key_dim <= 64 ? launch_bwd_mfma<F16, 64>(m, mem_dtype, s) : launch_bwd_mfma<F16, 128>(m, mem_dtype, s);
    }
    return key_dim <= 64 ? launch_bwd_mfma<BF16, 64>(m, mem_dtype, s) : launch_bwd_mfma<BF16, 128>(m, mem_dtype, s);
  }

  BwdArgs a;
  memset(&a, 0, sizeof(a));
  a.dh = grad_hidden;
  a.dmo = grad_memory_out;
  a.keys = keys;
  a.values = values;
  a.queries = queries;
  a.memory = memory;
  a.states = chunk_states;
  a.dv_out = grad_values;
  a.dm_out = grad_memory;
  a.part_k = dkq_partial;
  a.part_q = dkq_partial + batch * tiles * seq_len * key_dim;
  a.batch = batch;
  a.T = seq_len;
  a.dk = static_cast<int>(key_dim);
  a.dv = static_cast<int>(value_dim);
  a.tiles = tiles;
  a.n_chunks = static_cast<int>(n_chunks);
  a.mem_f32 = mem_dtype == GRM_HIP_F32;
  a.decay = static_cast<float>(memory_decay);
  a.c = static_cast<float>((1.0 - memory_decay) / std::sqrt(static_cast<double>(key_dim)));
  switch (in_dtype) {
    case GRM_HIP_F32: return launch_bwd<F32>(a, grad_keys, grad_queries, s);
    case GRM_HIP_F16: return launch_bwd<F16>(a, grad_keys, grad_queries, s);
    default: return launch_bwd<BF16>(a, grad_keys, grad_queries, s);
  }
}
