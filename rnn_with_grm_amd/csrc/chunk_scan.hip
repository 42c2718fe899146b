// Fused chunked linear-memory update + query application (forward), gfx950.
//
// Maths (reference grm/core/cuda_ops.py:218-254 chunked form; the per-token
// recurrence of grm/csrc/chunk_update.cu:82-123 and grm_cuda.cpp:74-83 is the
// same map): for a chunk of L tokens starting from state M (rows = value
// index v, columns = key index k), with c = (1 - decay) / sqrt(d_k),
//   h_i  = decay^{i+1} M q_i + c * sum_{j<=i} decay^{i-j} (q_i . k_j) v_j
//   M'   = decay^L M + c * sum_j decay^{L-1-j} v_j k_j^T
//
// Work decomposition.  One workgroup (4 waves) per (sequence, 16- or 32-wide
// value tile) walks every 64-token chunk of its sequence in order, keeping
// its d_k x DV slice of the state in fp32 MFMA accumulators the whole time.
// Value columns are independent given k and q, so tiles never talk to each
// other.  Per chunk, wave w owns query rows [16w, 16w+16):
//   S   = Q K^T              (MFMA, only the causal j-blocks <= w)
//   P   = S * c * decay^{i-j} (masked; stays in registers, it is already in
//                              the operand layout of the next MFMA)
//   O^T = decay^{i+1} M Q^T + V^T P^T   (MFMA; written as 4 contiguous v)
//   M^T = decay^L M^T + (w K)^T V      (MFMA, state tiles split over waves)
// K, V^T and a bf16/f16/f32 copy of the state live in LDS; the next chunk's
// K, V and Q are loaded into registers while the current one computes.
// Workgroups of one sequence are placed on one XCD so its Q and K are read
// from HBM once and hit that XCD's L2 for the other value tiles.
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#include <cmath>
#include <mutex>

#include "chunk_scan.h"
#include "grm_hip.h"
#include "grm_hip_common.h"

namespace grmhip {
namespace {

constexpr int NW = 4;          // waves per workgroup
constexpr int NTHR = 64 * NW;  // threads per workgroup

template <class E>
__device__ __forceinline__ void store4(typename ET<E>::raw* row, int col, f32x4 v, int ncols,
                                       bool vec) {
  using raw = typename ET<E>::raw;
  if (vec && col + 4 <= ncols) {
    if constexpr (sizeof(raw) == 2) {
      uint2 p;
      p.x = static_cast<uint32_t>(ET<E>::from_f(v[0])) |
            (static_cast<uint32_t>(ET<E>::from_f(v[1])) << 16);
      p.y = static_cast<uint32_t>(ET<E>::from_f(v[2])) |
            (static_cast<uint32_t>(ET<E>::from_f(v[3])) << 16);
      *reinterpret_cast<uint2*>(row + col) = p;
    } else {
      *reinterpret_cast<float4*>(row + col) = make_float4(v[0], v[1], v[2], v[3]);
    }
  } else {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      if (col + r < ncols) row[col + r] = ET<E>::from_f(v[r]);
    }
  }
}

// State rows live in memory as float32 or as the input dtype.
template <class E>
__device__ __forceinline__ f32x4 load_state4(const void* base, int64_t off, int col, int ncols,
                                             bool row_ok, bool f32, bool vec) {
  f32x4 out = {0.f, 0.f, 0.f, 0.f};
  if (!row_ok) return out;
  if (f32) {
    const float* p = static_cast<const float*>(base) + off;
    if (vec && col + 4 <= ncols) {
      float4 v = *reinterpret_cast<const float4*>(p + col);
      out[0] = v.x; out[1] = v.y; out[2] = v.z; out[3] = v.w;
    } else {
#pragma unroll
      for (int r = 0; r < 4; ++r) out[r] = (col + r < ncols) ? p[col + r] : 0.f;
    }
  } else {
    const typename ET<E>::raw* p = static_cast<const typename ET<E>::raw*>(base) + off;
#pragma unroll
    for (int r = 0; r < 4; ++r) out[r] = (col + r < ncols) ? ET<E>::to_f(p[col + r]) : 0.f;
  }
  return out;
}

template <class E>
__device__ __forceinline__ void store_state4(void* base, int64_t off, int col, int ncols,
                                             bool row_ok, bool f32, bool vec, f32x4 v) {
  if (!row_ok) return;
  if (f32) {
    float* p = static_cast<float*>(base) + off;
    if (vec && col + 4 <= ncols) {
      *reinterpret_cast<float4*>(p + col) = make_float4(v[0], v[1], v[2], v[3]);
    } else {
#pragma unroll
      for (int r = 0; r < 4; ++r)
        if (col + r < ncols) p[col + r] = v[r];
    }
  } else {
    typename ET<E>::raw* p = static_cast<typename ET<E>::raw*>(base) + off;
#pragma unroll
    for (int r = 0; r < 4; ++r)
      if (col + r < ncols) p[col + r] = ET<E>::from_f(v[r]);
  }
}

template <class E, int DKP, int DV>
struct FwdShape {
  using raw = typename ET<E>::raw;
  static constexpr int KS = DKP + 8;  // LDS row stride (elements) of K, Q and the state copy
  static constexpr int TS = CT + 4;   // LDS row stride (elements) of K^T, V^T and weighted V^T
  static constexpr int NKK = DKP / 32;
  static constexpr int VT = DV / 16;
  static constexpr int KT = DKP / 16;
  static constexpr int KTW = (KT + NW - 1) / NW;  // state key-tiles per wave
  static constexpr int NJP = CT / 32;             // 32-token slices of a chunk
  static constexpr int NCU = DKP / 8;             // 8-element units per K/Q row
  static constexpr int K_UNITS = CT * DKP / 8 / NTHR;
  static constexpr int V_UNITS = CT * DV / 8;     // <= NTHR
  static constexpr size_t lds_elems = 2 * static_cast<size_t>(CT) * KS  // Ks, Qs
                                      + static_cast<size_t>(DKP) * TS    // Kt
                                      + static_cast<size_t>(DV) * KS     // Mb
                                      + 2 * static_cast<size_t>(DV) * TS;  // Vt, Vw
  static constexpr size_t lds_bytes = lds_elems * sizeof(raw) + PW_N * sizeof(float);
  static_assert(K_UNITS * NTHR * 8 == CT * DKP, "K tile must split evenly over the workgroup");
  static_assert(V_UNITS <= NTHR, "V tile must fit one unit per thread");
  static_assert(NTHR % (16 * NCU) == 0 || (16 * NCU) % NTHR == 0, "row/unit map");
};

// Staging depth: the loads for chunk c+PF are issued while chunk c computes,
// so each load has PF chunk-times to arrive (global latency is about 3 us,
// a chunk computes in about 1 us).  32-wide tiles stage 2 deep so that two
// waves fit per SIMD (VGPR + AGPR <= 256); 16-wide tiles fit with 3.
template <int DV>
constexpr int prefetch_depth() { return DV >= 32 ? 2 : 3; }

// FULL = true: the fused scan (hidden, snapshots, final state) over one time
// part, starting from the state the earlier parts leave behind.
// FULL = false: the state-only pass that gives each part's end-state
// contribution from a zero start (keys and values only; no S, no outputs).
template <class E, int DKP, int DV, bool VEC, bool FULL>
__global__ __launch_bounds__(NTHR) void chunk_fwd_kernel(const ChunkFwdArgs a) {
  using S = FwdShape<E, DKP, DV>;
  using raw = typename ET<E>::raw;
  constexpr int KS = S::KS, TS = S::TS, NKK = S::NKK, VT = S::VT, KT = S::KT, KTW = S::KTW,
                NJP = S::NJP, NCU = S::NCU, K_UNITS = S::K_UNITS, V_UNITS = S::V_UNITS;
  constexpr int ES = static_cast<int>(sizeof(raw));
  constexpr int PF = prefetch_depth<DV>();

  extern __shared__ __align__(16) unsigned char smem[];
  raw* Ks = reinterpret_cast<raw*>(smem);  // [CT][KS]   keys, row = token
  raw* Qs = Ks + CT * KS;                  // [CT][KS]   queries, row = token
  raw* Kt = Qs + CT * KS;                  // [DKP][TS]  keys transposed, row = key index
  raw* Mb = Kt + DKP * TS;                 // [DV][KS]   state copy, row = value index
  raw* Vt = Mb + DV * KS;                  // [DV][TS]   values transposed, row = value index
  raw* Vw = Vt + DV * TS;                  // [DV][TS]   c * decay^{L-1-j} * values, transposed
  float* pw = reinterpret_cast<float*>(Vw + DV * TS);  // [PW_N]

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int g = lane >> 4;
  const int n = lane & 15;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);

  int wg = blockIdx.x;
  if (a.xcd_remap) {
    const int per = gridDim.x >> 3;
    wg = (wg & 7) * per + (wg >> 3);
  }
  // workgroup -> (sequence b, time part, value tile); tiles of one (b, part)
  // are adjacent so they share an XCD and its L2.
  const int parts_in_grid = FULL ? a.n_parts : a.n_parts - 1;
  const int seq = wg / a.v_tiles;
  const int64_t b = seq / parts_in_grid;
  const int part = seq % parts_in_grid;
  const int v0 = (wg % a.v_tiles) * DV;
  const int dk = a.dk, dv = a.dv;
  const int64_t T = a.seq_len;
  const int chunk = a.chunk;
  const int n_chunks = a.n_chunks;
  const int c_begin = part * a.part_chunks;
  const int c_end = min(c_begin + a.part_chunks, n_chunks);
  const bool f32m = a.mem_f32 != 0;
  const bool vec_m = a.vec_m != 0;

  const raw* keys = static_cast<const raw*>(a.keys) + b * T * dk;
  const raw* queries = static_cast<const raw*>(a.queries) + b * T * dk;
  const raw* values = static_cast<const raw*>(a.values) + b * T * dv;
  raw* hidden = static_cast<raw*>(a.hidden) + b * T * dv;

  for (int i = tid; i < PW_N; i += NTHR) pw[i] = a.pw[i];

  // ---- initial state: tile (kt, vt), lane (g, n), register r holds M[v][k]
  //      with v = v0 + 16 vt + n and k = 16 kt + 4 g + r.
  f32x4 st[KTW][VT];
#pragma unroll
  for (int q = 0; q < KTW; ++q) {
    const int kt = w + NW * q;
#pragma unroll
    for (int vt = 0; vt < VT; ++vt) {
      const int v = v0 + 16 * vt + n;
      st[q][vt] = (FULL && kt < KT) ? load_state4<E>(a.memory, (b * dv + v) * dk, 16 * kt + 4 * g,
                                                     dk, v < dv, f32m, vec_m)
                                    : f32x4{0.f, 0.f, 0.f, 0.f};
      // Start of part p: M_p = part_decay * M_{p-1} + D_{p-1}, from M_0 = memory.
      if (FULL && kt < KT) {
        for (int pp = 0; pp < part; ++pp) {
          const f32x4 d = load_state4<F32>(a.part_states, ((b * (a.n_parts - 1) + pp) * dv + v) * dk,
                                           16 * kt + 4 * g, dk, v < dv, true, vec_m);
          st[q][vt] = st[q][vt] * a.part_decay + d;
        }
      }
    }
  }

  const int i_loc = 16 * w + n;  // this lane's query row within a chunk
  // Tokens of chunk c; 0 outside this workgroup's part, so prefetches past
  // the part read nothing.
  // (32-bit scalar arithmetic: a 64-bit min is a VALU compare whose temporary
  // VGPRs can alias a prefetch in flight and force a wait for it.)
  const int last_c = static_cast<int>((T - 1) / chunk);
  const int last_len = static_cast<int>(T - static_cast<int64_t>(last_c) * chunk);
  auto chunk_len = [&](int c) -> int { return c >= c_end ? 0 : c == last_c ? last_len : chunk; };
  // Unit u of this thread covers K/Q row unit_row(u), elements unit_col(u) .. +8.
  // A wave's 64 units span 16 rows x 4 column units, so the transposed LDS
  // writes of K land on distinct banks.
  auto unit_row = [&](int u) {
    const int l = tid + NTHR * u;
    return (l & 15) + 16 * (l / (16 * NCU));
  };
  auto unit_col = [&](int u) { return ((tid + NTHR * u) / 16 % NCU) * 8; };

  // ---- staging (global -> registers -> LDS).  Each chunk gets buffer
  // resources that end at its last valid row, so rows past the chunk (and
  // every row past the last chunk) read as zero; columns past d_k / d_v are
  // sent out of range with an offset select.
  struct Stage {
    U8<E> k[K_UNITS];
    U8<E> q[K_UNITS];
    U8<E> v;
  };
  auto load8 = [&](__amdgpu_buffer_rsrc_t r, int row_off, int col, int ncols) -> U8<E> {
    if constexpr (VEC) {
      return buf_load8<E>(r, col < ncols ? row_off + col * ES : kBufOOB);
    } else {
      U8<E> u;
#pragma unroll
      for (int i = 0; i < 8; ++i) u.e[i] = buf_load1<E>(r, col + i < ncols ? row_off + (col + i) * ES : kBufOOB);
      return u;
    }
  };
  auto load_chunk = [&](int c, Stage& sg) {
    const int64_t t0 = static_cast<int64_t>(c) * chunk;
    const int L = chunk_len(c);
    const __amdgpu_buffer_rsrc_t rk = make_rsrc(keys + t0 * dk, static_cast<uint32_t>(L * dk * ES));
    const __amdgpu_buffer_rsrc_t rq = make_rsrc(queries + t0 * dk, static_cast<uint32_t>(L * dk * ES));
    const __amdgpu_buffer_rsrc_t rv = make_rsrc(values + t0 * dv, static_cast<uint32_t>(L * dv * ES));
#pragma unroll
    for (int u = 0; u < K_UNITS; ++u) {
      sg.k[u] = load8(rk, unit_row(u) * dk * ES, unit_col(u), dk);
      if constexpr (FULL) sg.q[u] = load8(rq, unit_row(u) * dk * ES, unit_col(u), dk);
    }
    // Threads past the V tile load an out-of-range unit (zeros) so the load
    // stays unconditional and never forces an early wait.
    const int row = (tid % 16) + 16 * (tid / (16 * (DV / 8)));
    const int col = v0 + ((tid / 16) % (DV / 8)) * 8;
    sg.v = load8(rv, row * dv * ES, (V_UNITS == NTHR || tid < V_UNITS) ? col : dv, dv);
  };
  // K and Q go to LDS row-major (S / O operands), K also transposed
  // (state-update operand); V goes transposed, plain (O operand) and scaled
  // by c * decay^{L-1-j} (state-update operand), L being the staged chunk's length.
  auto store_chunk = [&](int c, const Stage& sg) {
#pragma unroll
    for (int u = 0; u < K_UNITS; ++u) {
      const int row = unit_row(u), col = unit_col(u);
      if constexpr (FULL) {
        *reinterpret_cast<U8<E>*>(Ks + row * KS + col) = sg.k[u];
        *reinterpret_cast<U8<E>*>(Qs + row * KS + col) = sg.q[u];
      }
#pragma unroll
      for (int e = 0; e < 8; ++e) Kt[(col + e) * TS + row] = sg.k[u].e[e];
    }
    if (V_UNITS == NTHR || tid < V_UNITS) {
      const int L = chunk_len(c);
      const int row = (tid % 16) + 16 * (tid / (16 * (DV / 8)));
      const int c8 = (tid / 16) % (DV / 8);
      const float wj = (row < L) ? a.c * pw[max(L - 1 - row, 0)] : 0.f;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        if constexpr (FULL) Vt[(8 * c8 + e) * TS + row] = sg.v.e[e];
        Vw[(8 * c8 + e) * TS + row] = ET<E>::from_f(ET<E>::to_f(sg.v.e[e]) * wj);
      }
    }
  };
  auto store_state_copy = [&]() {
#pragma unroll
    for (int q = 0; q < KTW; ++q) {
      const int kt = w + NW * q;
      if (kt < KT) {
#pragma unroll
        for (int vt = 0; vt < VT; ++vt) {
          store4_raw<E>(Mb + (16 * vt + n) * KS + 16 * kt + 4 * g, st[q][vt]);
        }
      }
    }
  };

  Stage sg0, sg1, sg2;
  load_chunk(c_begin, sg0);
  load_chunk(c_begin + 1, sg1);
  if constexpr (PF == 3) load_chunk(c_begin + 2, sg2);
  __syncthreads();  // pw visible before store_chunk reads it
  store_chunk(c_begin, sg0);
  if constexpr (FULL) store_state_copy();
  __syncthreads();

  // Causal decay coefficients of S, fixed for every chunk: lane row i = i_loc,
  // column j = 16 jb + 4 g + r.
  float coef[4][4];
#pragma unroll
  for (int jb = 0; jb < 4; ++jb) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int j = 16 * jb + 4 * g + r;
      const float pv = pw[max(i_loc - j, 0)];
      coef[jb][r] = (j <= i_loc) ? a.c * pv : 0.f;
    }
  }

  // One chunk.  `ld` receives chunk c+PF (it held chunk c, already in LDS);
  // `st_next` holds chunk c+1 and goes to LDS at the end.  Everything between
  // the two barriers is branch-free so operand reads batch ahead of MFMAs.
  auto step = [&](int c, Stage& ld, const Stage& st_next) {
    const int64_t t0 = static_cast<int64_t>(c) * chunk;
    const int L = chunk_len(c);
    if (c > c_begin) __syncthreads();  // LDS operands and state copy of chunk c are in place
    load_chunk(c + PF, ld);

    if constexpr (FULL) {
    Frag8<E> qf[NKK];
#pragma unroll
    for (int kk = 0; kk < NKK; ++kk)
      qf[kk] = *reinterpret_cast<const Frag8<E>*>(Qs + i_loc * KS + 32 * kk + 8 * g);

    // S^T blocks: A = K rows j, B = Q rows i -> lane holds S[i = i_loc][j = 16jb + 4g + r].
    // All four j-blocks are computed; the causal mask lives in coef.
    f32x4 sacc[4];
#pragma unroll
    for (int jb = 0; jb < 4; ++jb) sacc[jb] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int kk = 0; kk < NKK; ++kk) {
      Frag8<E> kf[4];
#pragma unroll
      for (int jb = 0; jb < 4; ++jb)
        kf[jb] = *reinterpret_cast<const Frag8<E>*>(Ks + (16 * jb + n) * KS + 32 * kk + 8 * g);
#pragma unroll
      for (int jb = 0; jb < 4; ++jb) sacc[jb] = mfma8(kf[jb], qf[kk], sacc[jb]);
    }
    Frag8<E> pf[NJP];
#pragma unroll
    for (int p = 0; p < NJP; ++p) {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        pf[p].e[r] = ET<E>::from_f(sacc[2 * p][r] * coef[2 * p][r]);
        pf[p].e[4 + r] = ET<E>::from_f(sacc[2 * p + 1][r] * coef[2 * p + 1][r]);
      }
    }

    // O^T: A = state rows v, B = Q rows i, then A = V^T rows v, B = P rows i
    // -> lane holds O[i_loc][16vt + 4g + r].
    f32x4 o[VT];
#pragma unroll
    for (int vt = 0; vt < VT; ++vt) o[vt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int kk = 0; kk < NKK; ++kk) {
      Frag8<E> mf[VT];
#pragma unroll
      for (int vt = 0; vt < VT; ++vt)
        mf[vt] = *reinterpret_cast<const Frag8<E>*>(Mb + (16 * vt + n) * KS + 32 * kk + 8 * g);
#pragma unroll
      for (int vt = 0; vt < VT; ++vt) o[vt] = mfma8(mf[vt], qf[kk], o[vt]);
    }
    Frag8<E> vf[VT][NJP];
#pragma unroll
    for (int vt = 0; vt < VT; ++vt)
#pragma unroll
      for (int p = 0; p < NJP; ++p) {
        const raw* src = Vt + (16 * vt + n) * TS + 32 * p + 4 * g;
        vf[vt][p] = lds_frag_4x2<E>(src, src + 16);
      }
    const float s_start = (i_loc < L) ? pw[i_loc + 1] : 0.f;
    const __amdgpu_buffer_rsrc_t rh =
        make_rsrc(hidden + t0 * dv, static_cast<uint32_t>(a.hidden != nullptr ? L * dv * ES : 0));
#pragma unroll
    for (int vt = 0; vt < VT; ++vt) {
      o[vt] *= s_start;
#pragma unroll
      for (int p = 0; p < NJP; ++p) o[vt] = mfma8(vf[vt][p], pf[p], o[vt]);
      const int col = v0 + 16 * vt + 4 * g;
      const int row_off = i_loc * dv * ES;
      if constexpr (VEC) {
        buf_store4<E>(rh, col < dv ? row_off + col * ES : kBufOOB, o[vt]);
      } else {
#pragma unroll
        for (int r = 0; r < 4; ++r)
          buf_store1<E>(rh, col + r < dv ? row_off + (col + r) * ES : kBufOOB, o[vt][r]);
      }
    }

    }  // FULL

    // State update: M^T = decay^L M^T + K^T (w V), A = K^T rows k, B = (wV)^T rows v.
    Frag8<E> wf[VT][NJP];
#pragma unroll
    for (int vt = 0; vt < VT; ++vt)
#pragma unroll
      for (int p = 0; p < NJP; ++p) {
        const raw* src = Vw + (16 * vt + n) * TS + 32 * p + 4 * g;
        wf[vt][p] = lds_frag_4x2<E>(src, src + 16);
      }
    const float decay_L = pw[L];
#pragma unroll
    for (int q = 0; q < KTW; ++q) {
      const int kt = w + NW * q;
      if (kt < KT) {
        Frag8<E> kf[NJP];
#pragma unroll
        for (int p = 0; p < NJP; ++p) {
          const raw* src = Kt + (16 * kt + n) * TS + 32 * p + 4 * g;
          kf[p] = lds_frag_4x2<E>(src, src + 16);
        }
#pragma unroll
        for (int vt = 0; vt < VT; ++vt) {
          f32x4 acc = st[q][vt] * decay_L;
#pragma unroll
          for (int p = 0; p < NJP; ++p) acc = mfma8(kf[p], wf[vt][p], acc);
          st[q][vt] = acc;
        }
      }
    }

    if (FULL && a.snap_every > 0 && ((c + 1) % a.snap_every == 0 || c + 1 == n_chunks)) {
      const int si = c / a.snap_every;
      const __amdgpu_buffer_rsrc_t rs =
          make_rsrc(a.snapshots + (b * a.n_snap + si) * dv * dk, static_cast<uint32_t>(dv * dk * 4));
#pragma unroll
      for (int q = 0; q < KTW; ++q) {
        const int kt = w + NW * q;
        if (kt < KT) {
#pragma unroll
          for (int vt = 0; vt < VT; ++vt) {
            const int v = v0 + 16 * vt + n;
            const int k = 16 * kt + 4 * g;
            if constexpr (VEC) {
              // Key tiles past d_k (padding of the 16-wide tiles) are not stored: their
              // offsets would land in the next state row.
              buf_store4<F32>(rs, (v < dv && k < dk) ? (v * dk + k) * 4 : kBufOOB, st[q][vt]);
            } else {
#pragma unroll
              for (int r = 0; r < 4; ++r)
                buf_store1<F32>(rs, (v < dv && k + r < dk) ? (v * dk + k + r) * 4 : kBufOOB, st[q][vt][r]);
            }
          }
        }
      }
    }

    __syncthreads();  // every wave is done with chunk c's LDS
    store_chunk(c + 1, st_next);
    if constexpr (FULL) store_state_copy();
  };

  for (int c = c_begin; c < c_end; c += PF) {
    if constexpr (PF == 3) {
      step(c, sg0, sg1);
      if (c + 1 < c_end) step(c + 1, sg1, sg2);
      if (c + 2 < c_end) step(c + 2, sg2, sg0);
    } else {
      step(c, sg0, sg1);
      if (c + 1 < c_end) step(c + 1, sg1, sg0);
    }
  }

  if constexpr (!FULL) {
#pragma unroll
    for (int q = 0; q < KTW; ++q) {
      const int kt = w + NW * q;
      if (kt < KT) {
#pragma unroll
        for (int vt = 0; vt < VT; ++vt) {
          const int v = v0 + 16 * vt + n;
          store_state4<F32>(a.part_states, ((b * (a.n_parts - 1) + part) * dv + v) * dk, 16 * kt + 4 * g,
                            dk, v < dv, true, vec_m, st[q][vt]);
        }
      }
    }
    return;
  }
  if (a.memory_out == nullptr || part != a.n_parts - 1) return;
#pragma unroll
  for (int q = 0; q < KTW; ++q) {
    const int kt = w + NW * q;
    if (kt < KT) {
#pragma unroll
      for (int vt = 0; vt < VT; ++vt) {
        const int v = v0 + 16 * vt + n;
        store_state4<E>(a.memory_out, (b * dv + v) * dk, 16 * kt + 4 * g, dk, v < dv, f32m, vec_m,
                        st[q][vt]);
      }
    }
  }
}

template <class E, int DKP, int DV, bool VEC, bool FULL>
int launch_pass(ChunkFwdArgs a, hipStream_t stream) {
  using S = FwdShape<E, DKP, DV>;
  static_assert(S::lds_bytes <= kMaxLds, "tile does not fit the LDS of one CU");
  static bool attr_set = false;
  if (!attr_set) {
    hipError_t e = hipFuncSetAttribute(
        reinterpret_cast<const void*>(&chunk_fwd_kernel<E, DKP, DV, VEC, FULL>),
        hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(S::lds_bytes));
    if (e != hipSuccess) {
      set_error("chunk_update_fwd: hipFuncSetAttribute failed: %s", hipGetErrorString(e));
      return static_cast<int>(e);
    }
    attr_set = true;
  }
  const int64_t grid = a.batch * (FULL ? a.n_parts : a.n_parts - 1) * a.v_tiles;
  a.xcd_remap = (grid % 8 == 0) ? 1 : 0;
  hipLaunchKernelGGL((chunk_fwd_kernel<E, DKP, DV, VEC, FULL>), dim3(static_cast<unsigned>(grid)),
                     dim3(NTHR), S::lds_bytes, stream, a);
  return check_launch(FULL ? "chunk_update_fwd" : "chunk_update_fwd(part states)");
}

template <class E, int DKP, int DV, bool VEC>
int launch_fwd(const ChunkFwdArgs& a, hipStream_t stream) {
  if (a.n_parts > 1) {
    const int rc = launch_pass<E, DKP, DV, VEC, false>(a, stream);
    if (rc != GRM_HIP_OK) return rc;
  }
  return launch_pass<E, DKP, DV, VEC, true>(a, stream);
}

template <class E, int DV, bool VEC>
int dispatch_dk(const ChunkFwdArgs& a, hipStream_t s) {
  if (a.dk <= 32) return launch_fwd<E, 32, DV, VEC>(a, s);
  if (a.dk <= 64) return launch_fwd<E, 64, DV, VEC>(a, s);
  if (a.dk <= 128) return launch_fwd<E, 128, DV, VEC>(a, s);
  if constexpr (FwdShape<E, 256, DV>::lds_bytes <= kMaxLds) {
    return launch_fwd<E, 256, DV, VEC>(a, s);
  } else {
    set_error("chunk_update_fwd: key_dim %d needs more LDS than a CU has for this dtype", a.dk);
    return GRM_HIP_EUNSUPPORTED;
  }
}

// 16-byte accesses need every row of keys/queries/values/hidden to start on
// a 16-byte boundary; otherwise the element-wise variant (16-wide tiles) runs.
template <class E>
int dispatch_dv(const ChunkFwdArgs& a, int dv_tile, bool vec, hipStream_t s) {
  if (!vec) return dispatch_dk<E, 16, false>(a, s);
  return dv_tile == 32 ? dispatch_dk<E, 32, true>(a, s) : dispatch_dk<E, 16, true>(a, s);
}

bool aligned(const void* p, size_t n) { return (reinterpret_cast<uintptr_t>(p) % n) == 0; }

// Largest chunk length <= 64 that divides the snapshot interval, so snapshots
// always land on chunk boundaries.
int chunk_for_snapshot(int64_t snapshot_len) {
  if (snapshot_len % CT == 0) return CT;
  if (snapshot_len < CT) return static_cast<int>(snapshot_len);
  for (int c = CT; c >= 1; --c)
    if (snapshot_len % c == 0) return c;
  return 1;
}

// Time parts per sequence.  Splitting costs an extra state pass over K and V,
// so it is used only when (sequence, tile) workgroups would leave CUs idle:
// the grid is grown to about one workgroup per CU (256), keeping at least 8
// chunks per part.
int parts_for(int64_t wgs, int64_t n_chunks) {
  const char* env = getenv("GRM_HIP_CHUNK_PARTS");
  if (env != nullptr) {
    const int v = atoi(env);
    if (v >= 1) return static_cast<int>(min(static_cast<int64_t>(v), n_chunks));
  }
  if (wgs >= 192) return 1;
  int64_t p = (256 + wgs - 1) / wgs;
  p = min(p, n_chunks / 8);
  p = min(p, static_cast<int64_t>(64));
  return static_cast<int>(max(p, static_cast<int64_t>(1)));
}

}  // namespace

int tile_dv_for(int64_t batch, int64_t value_dim) {
  const char* env = getenv("GRM_HIP_CHUNK_DV");
  if (env != nullptr) {
    const int v = atoi(env);
    if (v == 16 || v == 32) return v;
  }
  // The wider tile halves the redundant Q K^T work per sequence; time parts
  // (parts_for) supply the parallelism it gives up.
  (void)batch;
  return value_dim >= 32 ? 32 : 16;
}

}  // namespace grmhip

using namespace grmhip;

namespace {

bool vec_ok(const void* keys, const void* values, const void* queries, const void* hidden,
            const float* snapshots, int64_t key_dim, int64_t value_dim) {
  return (key_dim % 8 == 0) && (value_dim % 8 == 0) && aligned(keys, 16) && aligned(queries, 16) &&
         aligned(values, 16) && aligned(hidden, 16) && (snapshots == nullptr || aligned(snapshots, 16));
}

struct Plan {
  bool wide;      // 128-wide value tiles (chunk_scan_wide.hip)
  bool vsplit;    // 32-wide value tiles, whole sequence per workgroup (chunk_scan_vsplit.hip)
  int chunk;
  int64_t n_chunks;
  int dv_tile;
  int v_tiles;
  int n_parts;
  int part_chunks;
  int64_t workspace_bytes;
};

// The wide kernel unless GRM_HIP_CHUNK_DV asks for the 16/32-column tiles.
bool use_wide(int in_dtype, int64_t key_dim, int64_t value_dim, bool vec) {
  const char* env = getenv("GRM_HIP_CHUNK_DV");
  if (env != nullptr && (atoi(env) == 16 || atoi(env) == 32)) return false;
  return wide_supported(in_dtype, key_dim, value_dim, vec);
}

// The value-split kernel where the wide kernel would need time parts (fewer
// than 192 sequence x 128-column workgroups) and 32-column tiles give at least
// as many workgroups instead.  GRM_HIP_CHUNK_VSPLIT=0 turns it off, =1 uses it
// wherever it is supported.
bool use_vsplit(int in_dtype, int64_t batch, int64_t key_dim, int64_t value_dim, bool vec, bool wide) {
  if (!wide || !vsplit_supported(in_dtype, key_dim, value_dim, vec)) return false;
  const char* env = getenv("GRM_HIP_CHUNK_VSPLIT");
  if (env != nullptr && (env[0] == '0' || env[0] == '1')) return env[0] == '1';
  const int64_t wide_wgs = batch * ((value_dim + kWideDv - 1) / kWideDv);
  return wide_wgs < 192 && batch * (value_dim / kVsplitDv) >= 192;
}

Plan make_plan(int64_t batch, int64_t seq_len, int64_t value_dim, int64_t key_dim,
               int64_t snapshot_len, bool vec, bool wide, bool vsplit = false) {
  Plan p;
  p.wide = wide && !vsplit;
  p.vsplit = vsplit;
  p.chunk = snapshot_len > 0 ? chunk_for_snapshot(snapshot_len) : CT;
  p.n_chunks = (seq_len + p.chunk - 1) / p.chunk;
  p.dv_tile = vsplit ? kVsplitDv : wide ? kWideDv : (vec ? tile_dv_for(batch, value_dim) : 16);
  p.v_tiles = static_cast<int>((value_dim + p.dv_tile - 1) / p.dv_tile);
  p.n_parts = vsplit ? 1 : parts_for(batch * p.v_tiles, p.n_chunks);
  p.part_chunks = static_cast<int>((p.n_chunks + p.n_parts - 1) / p.n_parts);
  p.n_parts = static_cast<int>((p.n_chunks + p.part_chunks - 1) / p.part_chunks);
  if (p.n_parts < 1) p.n_parts = 1;
  p.workspace_bytes = batch * (p.n_parts - 1) * value_dim * key_dim * 4;
  return p;
}

}  // namespace

extern "C" int64_t grm_hip_chunk_update_fwd_workspace(int64_t batch, int64_t seq_len,
                                                      int64_t key_dim, int64_t value_dim,
                                                      int64_t snapshot_len) {
  if (batch <= 0 || seq_len <= 0 || key_dim < 1 || value_dim < 1) return 0;
  // The dtype is not known here: size for whichever kernel needs more (the
  // element-wise path never needs more than the 16-byte one).
  const bool vec = key_dim % 8 == 0 && value_dim % 8 == 0;
  const Plan narrow = make_plan(batch, seq_len, value_dim, key_dim, snapshot_len, vec, false);
  const Plan wide = make_plan(batch, seq_len, value_dim, key_dim, snapshot_len, vec,
                              use_wide(GRM_HIP_BF16, key_dim, value_dim, vec));
  return narrow.workspace_bytes > wide.workspace_bytes ? narrow.workspace_bytes : wide.workspace_bytes;
}

extern "C" int grm_hip_chunk_update_fwd(const void* keys, const void* values, const void* queries,
                                        const void* memory, void* hidden, void* memory_out,
                                        float* snapshots, void* workspace, int64_t workspace_bytes,
                                        int64_t batch, int64_t seq_len, int64_t key_dim,
                                        int64_t value_dim, int in_dtype, int mem_dtype,
                                        double memory_decay, int64_t snapshot_len, void* stream) {
  if (batch < 0 || seq_len < 0 || key_dim < 1 || value_dim < 1) {
    set_error("chunk_update_fwd: bad sizes batch=%lld seq_len=%lld key_dim=%lld value_dim=%lld",
              (long long)batch, (long long)seq_len, (long long)key_dim, (long long)value_dim);
    return GRM_HIP_EINVAL;
  }
  if (in_dtype < GRM_HIP_F32 || in_dtype > GRM_HIP_BF16 ||
      (mem_dtype != GRM_HIP_F32 && mem_dtype != in_dtype)) {
    set_error("chunk_update_fwd: unsupported dtypes in=%d mem=%d", in_dtype, mem_dtype);
    return GRM_HIP_EUNSUPPORTED;
  }
  if (key_dim > 256 || (in_dtype == GRM_HIP_F32 && key_dim > 128)) {
    set_error("chunk_update_fwd: key_dim %lld exceeds %d for this dtype", (long long)key_dim,
              in_dtype == GRM_HIP_F32 ? 128 : 256);
    return GRM_HIP_EUNSUPPORTED;
  }
  if (!std::isfinite(memory_decay)) {
    set_error("chunk_update_fwd: memory_decay is not finite");
    return GRM_HIP_EINVAL;
  }
  if (snapshots != nullptr && snapshot_len <= 0) {
    set_error("chunk_update_fwd: snapshot_len must be > 0 when snapshots are requested");
    return GRM_HIP_EINVAL;
  }
  if (batch == 0) return GRM_HIP_OK;
  if (memory == nullptr || (seq_len > 0 && (keys == nullptr || values == nullptr ||
                                             queries == nullptr))) {
    set_error("chunk_update_fwd: null input pointer");
    return GRM_HIP_EINVAL;
  }
  if (memory_out == nullptr && snapshots == nullptr) {
    set_error("chunk_update_fwd: memory_out may be NULL only when snapshots are requested");
    return GRM_HIP_EINVAL;
  }
  if (memory_out != nullptr && memory_out == memory) {
    set_error("chunk_update_fwd: memory_out must not alias memory");
    return GRM_HIP_EINVAL;
  }
  hipStream_t s = static_cast<hipStream_t>(stream);
  const size_t in_b = (in_dtype == GRM_HIP_F32) ? 4 : 2;
  const size_t mem_b = (mem_dtype == GRM_HIP_F32) ? 4 : 2;

  ChunkFwdArgs a;
  memset(&a, 0, sizeof(a));
  a.keys = keys;
  a.values = values;
  a.queries = queries;
  a.memory = memory;
  a.hidden = hidden;
  a.memory_out = memory_out;
  a.snapshots = snapshots;
  a.batch = batch;
  a.seq_len = seq_len;
  a.dk = static_cast<int>(key_dim);
  a.dv = static_cast<int>(value_dim);
  const bool vec = vec_ok(keys, values, queries, hidden, snapshots, key_dim, value_dim);
  const bool vec_m = (key_dim % 4 == 0) && aligned(memory, 4 * mem_b) && aligned(memory_out, 4 * mem_b) &&
                     (snapshots == nullptr || aligned(snapshots, 16)) && aligned(workspace, 16);
  const bool wide = vec_m && use_wide(in_dtype, key_dim, value_dim, vec);
  const bool vsplit = use_vsplit(in_dtype, batch, key_dim, value_dim, vec, wide);
  Plan plan = make_plan(batch, seq_len, value_dim, key_dim, snapshots != nullptr ? snapshot_len : 0, vec, wide,
                        vsplit);
  if (plan.n_chunks > INT32_MAX) {
    set_error("chunk_update_fwd: seq_len too large");
    return GRM_HIP_EINVAL;
  }
  // Without room for the per-part states, one workgroup walks each whole sequence.
  if (plan.n_parts > 1 && (workspace == nullptr || workspace_bytes < plan.workspace_bytes ||
                           !aligned(workspace, 16))) {
    plan.n_parts = 1;
    plan.part_chunks = static_cast<int>(plan.n_chunks);
  }
  const int dv_tile = plan.dv_tile;
  a.chunk = plan.chunk;
  a.n_chunks = static_cast<int>(plan.n_chunks);
  if (snapshots != nullptr) {
    a.snap_every = static_cast<int>(snapshot_len / a.chunk);
    a.n_snap = static_cast<int>((seq_len + snapshot_len - 1) / snapshot_len);
  }
  a.v_tiles = plan.v_tiles;
  a.n_parts = plan.n_parts;
  a.part_chunks = plan.part_chunks;
  a.part_states = static_cast<float*>(workspace);
  a.part_decay = static_cast<float>(std::pow(memory_decay, static_cast<double>(plan.part_chunks) * a.chunk));
  const int64_t grid = batch * a.n_parts * a.v_tiles;
  if (grid > INT32_MAX) {
    set_error("chunk_update_fwd: batch too large for one launch");
    return GRM_HIP_EINVAL;
  }
  a.mem_f32 = mem_dtype == GRM_HIP_F32;
  a.vec_m = vec_m;
  {
    const int64_t snap_bytes = snapshots != nullptr ? batch * a.n_snap * value_dim * key_dim * 4 : 0;
    a.snap_full_lines = snap_bytes >= kFullLineSnapBytes;
    if (const char* env = getenv("GRM_HIP_SNAP_FULL_LINES")) a.snap_full_lines = env[0] == '1';
  }
  a.c = static_cast<float>((1.0 - memory_decay) / std::sqrt(static_cast<double>(key_dim)));
  for (int i = 0; i < PW_N; ++i) a.pw[i] = static_cast<float>(std::pow(memory_decay, i));

  if (seq_len == 0) {
    // Nothing to scan: memory_out = memory (reference returns the input state).
    if (memory_out == nullptr) return GRM_HIP_OK;
    hipError_t e = hipMemcpyAsync(memory_out, memory, batch * value_dim * key_dim * mem_b,
                                  hipMemcpyDeviceToDevice, s);
    if (e != hipSuccess) {
      set_error("chunk_update_fwd: hipMemcpyAsync failed: %s", hipGetErrorString(e));
      return static_cast<int>(e);
    }
    return GRM_HIP_OK;
  }
  if (plan.vsplit) return launch_scan_vsplit(a, in_dtype, s);
  if (plan.wide) return launch_scan_wide(a, in_dtype, mem_dtype, s);
  switch (in_dtype) {
    case GRM_HIP_F32: return dispatch_dv<F32>(a, dv_tile, vec, s);
    case GRM_HIP_F16: return dispatch_dv<F16>(a, dv_tile, vec, s);
    default: return dispatch_dv<BF16>(a, dv_tile, vec, s);
  }
}

// ---------------------------------------------------------------------------
// The same forward with no allocation at all: the time-split workspace is a
// file-scope device array, one per GPU, instead of caller memory.
namespace {

constexpr int64_t kNoAllocScratchBytes = GRM_HIP_NOALLOC_SCRATCH_BYTES;
constexpr int kMaxDevices = 64;

// Device-side scratch of the no-alloc forward.  In host code this name is not
// a device address: host code uses the per-device pointer from
// hipGetSymbolAddress below, never the name itself.
static __device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];

std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};
// Per device: an event recorded on the stream of the last call (after its
// launches) and that stream, so that a call on another stream first waits for
// it.  Created with the address lookup, once per device, and kept.
hipEvent_t g_scratch_done[kMaxDevices] = {};
hipStream_t g_scratch_stream[kMaxDevices] = {};
bool g_scratch_recorded[kMaxDevices] = {};

// The current device's index and copy of `scratch`, looked up once per device
// (with that device current) and kept.  Called with g_scratch_mu held.
int scratch_for_current_device(int* dev_out, void** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) {
    set_error("chunk_update_fwd_noalloc: hipGetDevice failed: %s", hipGetErrorString(e));
    return static_cast<int>(e);
  }
  if (dev < 0 || dev >= kMaxDevices) {
    set_error("chunk_update_fwd_noalloc: device %d beyond the %d this library tracks", dev, kMaxDevices);
    return GRM_HIP_EUNSUPPORTED;
  }
  if (g_scratch_ptr[dev] == nullptr) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || p == nullptr) {
      set_error("chunk_update_fwd_noalloc: hipGetSymbolAddress(scratch) failed on device %d: %s", dev,
                hipGetErrorString(e));
      return e != hipSuccess ? static_cast<int>(e) : GRM_HIP_EINVAL;
    }
    hipEvent_t ev = nullptr;
    e = hipEventCreateWithFlags(&ev, hipEventDisableTiming);
    if (e != hipSuccess) {
      set_error("chunk_update_fwd_noalloc: hipEventCreateWithFlags failed on device %d: %s", dev,
                hipGetErrorString(e));
      return static_cast<int>(e);
    }
    g_scratch_done[dev] = ev;
    g_scratch_ptr[dev] = p;
  }
  *dev_out = dev;
  *out = g_scratch_ptr[dev];
  return GRM_HIP_OK;
}

}  // namespace

extern "C" int64_t grm_hip_chunk_update_fwd_noalloc_limit(void) { return kNoAllocScratchBytes; }

extern "C" int grm_hip_chunk_update_fwd_noalloc(const void* keys, const void* values, const void* queries,
                                                const void* memory, void* hidden, void* memory_out,
                                                float* snapshots, int64_t batch, int64_t seq_len,
                                                int64_t key_dim, int64_t value_dim, int in_dtype, int mem_dtype,
                                                double memory_decay, int64_t snapshot_len, void* stream) {
  const int64_t need = grm_hip_chunk_update_fwd_workspace(batch, seq_len, key_dim, value_dim,
                                                          snapshots != nullptr ? snapshot_len : 0);
  if (need > kNoAllocScratchBytes) {
    set_error("chunk_update_fwd_noalloc: these sizes need %lld bytes of time-split scratch, beyond the "
              "library's fixed %lld (use grm_hip_chunk_update_fwd with a caller workspace)",
              (long long)need, (long long)kNoAllocScratchBytes);
    return GRM_HIP_EINVAL;
  }
  if (need == 0) {  // no time split: the scratch is not used
    return grm_hip_chunk_update_fwd(keys, values, queries, memory, hidden, memory_out, snapshots, nullptr, 0, batch,
                                    seq_len, key_dim, value_dim, in_dtype, mem_dtype, memory_decay, snapshot_len,
                                    stream);
  }
  hipStream_t s = static_cast<hipStream_t>(stream);
  hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
  hipError_t e = hipStreamIsCapturing(s, &cap);
  if (e != hipSuccess) {
    set_error("chunk_update_fwd_noalloc: hipStreamIsCapturing failed: %s", hipGetErrorString(e));
    return static_cast<int>(e);
  }
  const bool capturing = cap != hipStreamCaptureStatusNone;
  // Held over the wait, the launches and the record: calls from several host
  // threads take the scratch one after another.
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  int dev = -1;
  void* ws = nullptr;
  int rc = scratch_for_current_device(&dev, &ws);
  if (rc != GRM_HIP_OK) return rc;
  // A call on another stream than the last one waits for the last one's kernels, so
  // calls on different streams take the scratch in turn instead of racing on it.
  // Under stream capture the library orders nothing: the caller orders replays.
  if (!capturing && g_scratch_recorded[dev] && g_scratch_stream[dev] != s) {
    e = hipStreamWaitEvent(s, g_scratch_done[dev], 0);
    if (e != hipSuccess) {
      set_error("chunk_update_fwd_noalloc: hipStreamWaitEvent failed: %s", hipGetErrorString(e));
      return static_cast<int>(e);
    }
  }
  rc = grm_hip_chunk_update_fwd(keys, values, queries, memory, hidden, memory_out, snapshots, ws,
                                kNoAllocScratchBytes, batch, seq_len, key_dim, value_dim, in_dtype, mem_dtype,
                                memory_decay, snapshot_len, stream);
  if (rc == GRM_HIP_OK && !capturing) {
    e = hipEventRecord(g_scratch_done[dev], s);
    if (e != hipSuccess) {
      set_error("chunk_update_fwd_noalloc: hipEventRecord failed: %s", hipGetErrorString(e));
      return static_cast<int>(e);
    }
    g_scratch_stream[dev] = s;
    g_scratch_recorded[dev] = true;
  }
  return rc;
}
