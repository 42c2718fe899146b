// Fused chunked linear-memory update + query application (forward), wide
// variant for bf16 / f16 inputs with key_dim <= 128, gfx950.
//
// Maths (reference grm/core/cuda_ops.py:218-254 chunked form; the per-token
// recurrence of grm/csrc/chunk_update.cu:82-123 and grm_cuda.cpp:74-83 is the
// same map): for a chunk of L tokens starting from state M (rows = value
// index v, columns = key index k), with c = (1 - decay) / sqrt(d_k),
//   h_i  = decay^{i+1} M q_i + c * sum_{j<=i} decay^{i-j} (q_i . k_j) v_j
//   M'   = decay^L M + c * sum_j decay^{L-1-j} v_j k_j^T
//
// Work decomposition.  One workgroup of 8 waves per (sequence, time part,
// 128-wide value tile) walks the 64-token chunks of its part in order.  Wave w
// owns state rows v in [16w, 16w + 16) for every key column, as fp32 MFMA
// accumulators that never leave registers.  Per chunk:
//   S = Q K^T      wave w computes query rows [16(w%4), +16) against key
//                  columns [32(w/4), +32) once for the whole value tile and
//                  publishes P = S * c * decay^{i-j} (causal) to LDS;
//   O^T = decay^{i+1} M Q^T + V^T P^T
//                  wave w computes its 16 value rows for all 64 queries; the
//                  M Q^T operand comes straight from the state accumulators
//                  (two 16x16 accumulator tiles form one 32-deep operand);
//   M^T = decay^L M^T + K^T (w V)
//                  K^T and V^T operands are read from the row-major K and V
//                  tiles with the LDS transpose read (ds_read_b64_tr_b16), so
//                  every LDS write is a plain 16-byte row write.
// K, Q and V arrive with full-row 16-byte buffer loads two chunks ahead and
// alternate between two LDS buffers; the output tile is staged in LDS and
// leaves as full rows.  A state-only pass over the earlier time parts gives
// each part its starting state (M_p = decay^{len} M_{p-1} + D_{p-1}).
#include <stdint.h>
#include <string.h>

#include <cmath>
#include <type_traits>

#include "chunk_scan.h"
#include "grm_hip.h"
#include "grm_hip_common.h"

namespace grmhip {
namespace {

constexpr int VB = 1;  // 16-wide value blocks per wave

typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) s16x4 lds_s16x4;

// Both passes run 8 waves (two per SIMD) on a 128-wide value tile; the state
// pass keeps only K and V in LDS.
constexpr int pass_threads(bool) { return 512; }

// Up to this many parts the full pass combines M_0 and the earlier parts'
// contributions itself; beyond it a combine step writes each part's starting
// state and the full pass reads just that.
constexpr int kCombineInPlaceParts = 4;

template <class E, int DKP, bool FULL>
struct WideShape {
  using raw = typename ET<E>::raw;
  static constexpr int NW = 8;                  // waves per workgroup
  static constexpr int NT = 64 * NW;            // threads per workgroup
  static_assert(NT == pass_threads(FULL), "launch bound matches the tile");
  static constexpr int DVT = 16 * VB * NW;      // value columns per workgroup
  static_assert(!FULL || DVT == kWideDv, "full pass covers kWideDv value columns");
  // Row strides (elements) are 4 banks mod 64 (K, Q, V, output) or a distinct
  // multiple of 4 banks for each of 16 rows (P): 16-byte reads of 16 rows are
  // conflict-free and 8-byte reads of 16 consecutive rows (the transposed
  // reads) hit every bank exactly twice, the minimum for 512 bytes.
  static constexpr int KS = DKP + 8;   // K and Q tiles [CT][KS]
  static constexpr int VS = DVT + 8;   // V tile and output tile [CT][VS]
  static constexpr int PS = CT + 8;    // P tile [CT][PS]
  static constexpr int KT = DKP / 16;  // 16-wide key tiles
  static constexpr int NKK = DKP / 32; // 32-deep key steps
  static constexpr int KU = DKP / 8;   // 16-byte units per K/Q row
  static constexpr int VU = DVT / 8;   // 16-byte units per V / output row
  static constexpr int K_UNITS = CT * KU / NT;
  static constexpr int V_UNITS = CT * VU / NT;
  static constexpr int KQ = FULL ? 2 : 1;            // K (and Q) tiles per buffer
  static constexpr int BUF = CT * (KQ * KS + VS);    // one K/Q/V buffer, elements
  static constexpr int EXTRA = FULL ? CT * (PS + VS) : 0;  // P and output tiles
  static constexpr size_t lds_bytes =
      static_cast<size_t>(2 * BUF + EXTRA) * sizeof(raw) + PW_N * sizeof(float);
  static_assert(K_UNITS * NT == CT * KU && V_UNITS * NT == CT * VU, "tiles split evenly");
  static_assert(lds_bytes <= kMaxLds, "tile set must fit one CU's LDS");
};

// Four 16-bit elements of a row-major tile, transposed across each 16-lane
// block: lane i of the block receives X[r0 + e][c0 + i] (e = 0..3) when lane s
// of the block passes &X[r0 + (s >> 2)][c0 + 4 (s & 3)].
template <class E>
__device__ __forceinline__ s16x4 tr4(const typename ET<E>::raw* p) {
  return __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(p));
}

template <class E>
__device__ __forceinline__ Frag8<E> frag_tr(const typename ET<E>::raw* p_lo, const typename ET<E>::raw* p_hi) {
  const s16x4 lo = tr4<E>(p_lo);
  const s16x4 hi = tr4<E>(p_hi);
  Frag8<E> f;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    f.e[e] = static_cast<typename ET<E>::raw>(static_cast<uint16_t>(lo[e]));
    f.e[4 + e] = static_cast<typename ET<E>::raw>(static_cast<uint16_t>(hi[e]));
  }
  return f;
}

// Four state values at element offset `off` of a [v][k] row-major state
// (fp32 or the input dtype); OOB offsets read zeros.
template <class E>
__device__ __forceinline__ f32x4 ld_state4(__amdgpu_buffer_rsrc_t r, int off, bool f32) {
  f32x4 out;
  if (f32) {
    const u32x4 u = __builtin_amdgcn_raw_buffer_load_b128(r, off == kBufOOB ? kBufOOB : off * 4, 0, 0);
#pragma unroll
    for (int i = 0; i < 4; ++i) out[i] = __uint_as_float(u[i]);
  } else {
    constexpr int ES = static_cast<int>(sizeof(typename ET<E>::raw));
    const u32x2 u = __builtin_amdgcn_raw_buffer_load_b64(r, off == kBufOOB ? kBufOOB : off * ES, 0, 0);
    out[0] = ET<E>::to_f(static_cast<typename ET<E>::raw>(u[0] & 0xffffu));
    out[1] = ET<E>::to_f(static_cast<typename ET<E>::raw>(u[0] >> 16));
    out[2] = ET<E>::to_f(static_cast<typename ET<E>::raw>(u[1] & 0xffffu));
    out[3] = ET<E>::to_f(static_cast<typename ET<E>::raw>(u[1] >> 16));
  }
  return out;
}

template <class E>
__device__ __forceinline__ void st_state4(__amdgpu_buffer_rsrc_t r, int off, bool f32, f32x4 v) {
  if (f32) {
    buf_store4<F32>(r, off == kBufOOB ? kBufOOB : off * 4, v);
  } else {
    constexpr int ES = static_cast<int>(sizeof(typename ET<E>::raw));
    buf_store4<E>(r, off == kBufOOB ? kBufOOB : off * ES, v);
  }
}

// FULL = true: hidden, snapshots and the final state over one time part,
// starting from M_p.  With a.part_starts the state pass's combine step has
// already written M_p (p >= 1) to part_states[p - 1]; otherwise part_states
// holds each earlier part's contribution D_q and the workgroup combines
//   M_p = pd^p M_0 + sum_{q < p} pd^{p-1-q} D_q,  pd = decay^{part length}.
// FULL = false: the state pass, D_q of each earlier part from a zero start
// (keys and values only).
template <class E, int DKP, bool FULL>
__global__ __launch_bounds__(pass_threads(FULL), 1) void scan_wide_kernel(const ChunkFwdArgs a) {
  using S = WideShape<E, DKP, FULL>;
  constexpr int WNT = S::NT, DVT = S::DVT;
  using raw = typename ET<E>::raw;
  constexpr int KS = S::KS, VS = S::VS, PS = S::PS, KT = S::KT, NKK = S::NKK, KU = S::KU, VU = S::VU,
                K_UNITS = S::K_UNITS, V_UNITS = S::V_UNITS, BUF = S::BUF;
  constexpr int ES = static_cast<int>(sizeof(raw));
  // Chunks in flight between global memory and LDS: the full pass has no
  // registers for more than two staging sets; the state pass stages K and V
  // only and keeps four in flight.
  constexpr int PF = FULL ? 2 : 4;
  static_assert(PF % 2 == 0, "staging sets pair with the two LDS buffers");
  using FullStep = std::integral_constant<bool, true>;
  using StateStep = std::integral_constant<bool, false>;

  extern __shared__ __align__(16) unsigned char smem[];
  raw* bufs = reinterpret_cast<raw*>(smem);  // 2 x { K [CT][KS], Q [CT][KS] (full pass), V [CT][VS] }
  raw* Ps = bufs + 2 * BUF;                   // [CT][PS]  P = S * coef, row = query (full pass)
  raw* Os = Ps + CT * PS;                     // [CT][VS]  output tile, row = query (full pass)
  float* pw = reinterpret_cast<float*>(bufs + 2 * BUF + S::EXTRA);  // [PW_N]

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
  // workgroup -> (sequence b, time part, value tile); the parts of a sequence
  // are adjacent, so they share an XCD and earlier parts dispatch first.
  const int parts_in_grid = FULL ? a.n_parts : a.n_parts - 1;
  const int v_tiles = (a.dv + DVT - 1) / DVT;
  const int vtile = wg % v_tiles;
  const int seq = wg / v_tiles;
  const int64_t b = seq / parts_in_grid;
  const int part = seq % parts_in_grid;
  const int v0 = vtile * DVT;
  const int dk = a.dk, dv = a.dv;
  const int64_t T = a.seq_len;
  const int chunk = a.chunk;
  const int n_chunks = a.n_chunks;
  const int c_begin = part * a.part_chunks;
  const int c_end = min(c_begin + a.part_chunks, n_chunks);
  const bool f32m = a.mem_f32 != 0;

  const raw* keys = static_cast<const raw*>(a.keys) + b * T * dk;
  const raw* queries = static_cast<const raw*>(a.queries) + b * T * dk;
  const raw* values = static_cast<const raw*>(a.values) + b * T * dv;
  raw* hidden = a.hidden != nullptr ? static_cast<raw*>(a.hidden) + b * T * dv : nullptr;

  // The power table is the first load issued, so waiting for it later does
  // not wait for the state and chunk loads issued after it.
  static_assert(PW_N <= WNT, "one power per thread");
  const float pw_first = tid < PW_N ? a.pw[tid] : 0.f;

  // ---- state: st[vb][kt], lane (g, n), register r = M[v][k] with
  //      v = v0 + 16 (VB w + vb) + n and k = 16kt + 4g + r.
  const int vl = 16 * VB * w + n;  // local value row of block 0 for this lane
  f32x4 st[VB][KT];
  auto state_off = [&](int vb, int kt) -> int {
    const int v = v0 + vl + 16 * vb;
    const int k = 16 * kt + 4 * g;
    return (v < dv && k < dk) ? v * dk + k : kBufOOB;
  };
  auto zero_state = [&]() {
#pragma unroll
    for (int vb = 0; vb < VB; ++vb)
#pragma unroll
      for (int kt = 0; kt < KT; ++kt) st[vb][kt] = f32x4{0.f, 0.f, 0.f, 0.f};
  };
  const int64_t mem_b = f32m ? 4 : ES;
  const __amdgpu_buffer_rsrc_t rmem =
      make_rsrc(static_cast<const unsigned char*>(a.memory) + b * dv * dk * mem_b, static_cast<uint32_t>(dv * dk * mem_b));
  auto part_rsrc = [&](int q) {
    return make_rsrc(a.part_states + (b * (a.n_parts - 1) + q) * dv * dk, static_cast<uint32_t>(dv * dk * 4));
  };
  // st = pd^q_end M_0 + sum_{q < q_end} pd^{q_end-1-q} D_q, pd = decay^{part length}.
  // issue_start() only issues the loads (M_0 into st, up to
  // kCombineInPlaceParts - 1 contributions into d; D slots past q_end read as
  // zero); finish_start() combines them once the chunk loads are out too.
  // M_0 arrives as raw words (four fp32, or four 16-bit values in .xy) and is
  // converted in finish_start(): one branch around all loads, so they issue
  // back to back instead of each waiting for its conversion.
  constexpr int NQ = FULL ? kCombineInPlaceParts - 1 : 1;
  f32x4 d[NQ][VB][KT];
  u32x4 m0raw[VB][KT];
  auto issue_start = [&](int q_end, bool from_slot) {
    if (from_slot) {  // the combine step wrote M_p into slot p - 1
      const __amdgpu_buffer_rsrc_t rp = part_rsrc(q_end - 1);
#pragma unroll
      for (int vb = 0; vb < VB; ++vb)
#pragma unroll
        for (int kt = 0; kt < KT; ++kt) st[vb][kt] = ld_state4<F32>(rp, state_off(vb, kt), true);
      return;
    }
    if (f32m) {
#pragma unroll
      for (int vb = 0; vb < VB; ++vb)
#pragma unroll
        for (int kt = 0; kt < KT; ++kt) {
          const int off = state_off(vb, kt);
          m0raw[vb][kt] = __builtin_amdgcn_raw_buffer_load_b128(rmem, off == kBufOOB ? kBufOOB : off * 4, 0, 0);
        }
    } else {
#pragma unroll
      for (int vb = 0; vb < VB; ++vb)
#pragma unroll
        for (int kt = 0; kt < KT; ++kt) {
          const int off = state_off(vb, kt);
          const u32x2 u = __builtin_amdgcn_raw_buffer_load_b64(rmem, off == kBufOOB ? kBufOOB : off * ES, 0, 0);
          m0raw[vb][kt] = u32x4{u[0], u[1], 0u, 0u};
        }
    }
#pragma unroll
    for (int q = 0; q < NQ; ++q) {
      const __amdgpu_buffer_rsrc_t rp = part_rsrc(q < q_end ? q : 0);
#pragma unroll
      for (int vb = 0; vb < VB; ++vb)
#pragma unroll
        for (int kt = 0; kt < KT; ++kt) {
          const int off = state_off(vb, kt);
          d[q][vb][kt] = ld_state4<F32>(rp, q < q_end ? off : kBufOOB, true);
        }
    }
  };
  auto finish_start = [&](int q_end, bool from_slot) {
    if (from_slot) return;
    // Opaque register moves pin the first use of the loaded words here, after
    // the barrier: otherwise the compiler hoists the sums above the chunk
    // loads and every load waits for the state's latency first.
#pragma unroll
    for (int vb = 0; vb < VB; ++vb)
#pragma unroll
      for (int kt = 0; kt < KT; ++kt) {
        asm volatile("" : "+v"(m0raw[vb][kt]));
#pragma unroll
        for (int q = 0; q < NQ; ++q) asm volatile("" : "+v"(d[q][vb][kt]));
      }
    float m = 1.f;  // pd^(q_end - 1 - q) for q = q_end - 1, q_end - 2, ...
    f32x4 acc[VB][KT];
#pragma unroll
    for (int vb = 0; vb < VB; ++vb)
#pragma unroll
      for (int kt = 0; kt < KT; ++kt) acc[vb][kt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int q = NQ - 1; q >= 0; --q) {
      if (q >= q_end) continue;
#pragma unroll
      for (int vb = 0; vb < VB; ++vb)
#pragma unroll
        for (int kt = 0; kt < KT; ++kt) acc[vb][kt] += m * d[q][vb][kt];
      m *= a.part_decay;
    }
#pragma unroll
    for (int vb = 0; vb < VB; ++vb)
#pragma unroll
      for (int kt = 0; kt < KT; ++kt) {
        const u32x4 u = m0raw[vb][kt];
        f32x4 m0;
        if (f32m) {
#pragma unroll
          for (int i = 0; i < 4; ++i) m0[i] = __uint_as_float(u[i]);
        } else {
          m0[0] = ET<E>::to_f(static_cast<raw>(u[0] & 0xffffu));
          m0[1] = ET<E>::to_f(static_cast<raw>(u[0] >> 16));
          m0[2] = ET<E>::to_f(static_cast<raw>(u[1] & 0xffffu));
          m0[3] = ET<E>::to_f(static_cast<raw>(u[1] >> 16));
        }
        st[vb][kt] = acc[vb][kt] + m * m0;
      }
  };
  auto store_state = [&](__amdgpu_buffer_rsrc_t r) {
#pragma unroll
    for (int vb = 0; vb < VB; ++vb)
#pragma unroll
      for (int kt = 0; kt < KT; ++kt) {
        const int off = state_off(vb, kt);
        buf_store4<F32>(r, off == kBufOOB ? kBufOOB : off * 4, st[vb][kt]);
      }
  };

  // Tokens of chunk c; 0 at or past the end of the chunk window being
  // scanned, so loads past it read nothing.
  int ce_cur = c_end;
  // (32-bit scalar arithmetic: a 64-bit min is a VALU compare whose temporary
  // VGPRs can alias a prefetch in flight and force a wait for it.)
  const int last_c = static_cast<int>((T - 1) / chunk);
  const int last_len = static_cast<int>(T - static_cast<int64_t>(last_c) * chunk);
  auto chunk_len = [&](int c) -> int { return c >= ce_cur ? 0 : c == last_c ? last_len : chunk; };

  // ---- staging: unit u of this thread is row (tid + WNT u) / KU, 16-byte
  // column (tid + WNT u) % KU, so a wave reads whole rows.
  struct Stage {
    U8<E> k[K_UNITS];
    U8<E> q[K_UNITS];
    U8<E> v[V_UNITS];
  };
  auto load_chunk = [&](int c, Stage& sg, auto full) {
    constexpr bool F = decltype(full)::value;
    const int64_t t0 = static_cast<int64_t>(c) * chunk;
    const int L = chunk_len(c);
    const __amdgpu_buffer_rsrc_t rk = make_rsrc(keys + t0 * dk, static_cast<uint32_t>(L * dk * ES));
    const __amdgpu_buffer_rsrc_t rq = make_rsrc(queries + t0 * dk, static_cast<uint32_t>(L * dk * ES));
    const __amdgpu_buffer_rsrc_t rv = make_rsrc(values + t0 * dv, static_cast<uint32_t>(L * dv * ES));
#pragma unroll
    for (int u = 0; u < K_UNITS; ++u) {
      const int l = tid + WNT * u;
      const int row = l / KU, col = 8 * (l % KU);
      const int off = col < dk ? (row * dk + col) * ES : kBufOOB;
      sg.k[u] = buf_load8<E>(rk, off);
      if constexpr (F) sg.q[u] = buf_load8<E>(rq, off);
    }
#pragma unroll
    for (int u = 0; u < V_UNITS; ++u) {
      const int l = tid + WNT * u;
      const int row = l / VU, col = v0 + 8 * (l % VU);
      sg.v[u] = buf_load8<E>(rv, col < dv ? (row * dv + col) * ES : kBufOOB);
    }
  };
  auto store_chunk = [&](int buf, const Stage& sg, auto full) {
    constexpr bool F = decltype(full)::value;
    raw* Kb = bufs + buf * BUF;
    raw* Qb = Kb + CT * KS;
    raw* Vb = Kb + S::KQ * CT * KS;
#pragma unroll
    for (int u = 0; u < K_UNITS; ++u) {
      const int l = tid + WNT * u;
      const int row = l / KU, col = 8 * (l % KU);
      *reinterpret_cast<U8<E>*>(Kb + row * KS + col) = sg.k[u];
      if constexpr (F) *reinterpret_cast<U8<E>*>(Qb + row * KS + col) = sg.q[u];
    }
#pragma unroll
    for (int u = 0; u < V_UNITS; ++u) {
      const int l = tid + WNT * u;
      const int row = l / VU, col = 8 * (l % VU);
      *reinterpret_cast<U8<E>*>(Vb + row * VS + col) = sg.v[u];
    }
  };
  // Output tile of a chunk (Os) -> hidden rows, whole rows per wave.
  auto flush_out = [&](int c) {
    const int64_t t0 = static_cast<int64_t>(c) * chunk;
    const int L = chunk_len(c);
    const __amdgpu_buffer_rsrc_t rh = make_rsrc(hidden + (hidden != nullptr ? t0 * dv : 0),
                                                static_cast<uint32_t>(hidden != nullptr ? L * dv * ES : 0));
#pragma unroll
    for (int u = 0; u < V_UNITS; ++u) {
      const int l = tid + WNT * u;
      const int row = l / VU, col = 8 * (l % VU);
      const u32x4 val = *reinterpret_cast<const u32x4*>(Os + row * VS + col);
      __builtin_amdgcn_raw_buffer_store_b128(val, rh, v0 + col < dv ? (row * dv + v0 + col) * ES : kBufOOB, 0, 0);
    }
  };

  static_assert(!FULL || S::NW == 8, "S blocks are split as 4 query blocks x 2 key halves");
  // This wave's S block: query rows i = 16 i_blk + n, key columns
  // j = 32 j_half + 16 jj + 4g + r (jj = 0, 1), with causal coefficients.
  const int i_blk = w & 3;
  const int j_half = w >> 2;
  const int i_loc = 16 * i_blk + n;
  float coef[2][4];
  // decay^{i+1} for the query rows i = 16 ib + n of this lane's output tiles.
  float s_start[4];
  // State-update weights c * decay^{L-1-j} for this lane's slots
  // j = 32p + 16 (s / 4) + 4g + s % 4 (the token order of every 64-deep operand).
  float wgt[2][8];
  auto set_weights = [&](int L) {
#pragma unroll
    for (int p = 0; p < 2; ++p) {
#pragma unroll
      for (int s = 0; s < 8; ++s) {
        const int j = 32 * p + 16 * (s >> 2) + 4 * g + (s & 3);
        wgt[p][s] = (j < L) ? a.c * pw[max(L - 1 - j, 0)] : 0.f;
      }
    }
  };
  int snap_phase = 1;  // == 0: a snapshot follows the current chunk

  auto step = [&](int c, int cb, int cur, Stage& ld, const Stage& nx, auto full) {
    constexpr bool F = decltype(full)::value;
    const int L = chunk_len(c);
    const raw* Kb = bufs + cur * BUF;
    const raw* Qb = Kb + CT * KS;
    const raw* Vb = Kb + S::KQ * CT * KS;
    if (c > cb) __syncthreads();  // chunk c in LDS; the previous output tile is complete
    load_chunk(c + PF, ld, full);
    if (F && c > cb) flush_out(c - 1);
    if (L != CT) set_weights(L);

    f32x4 o[4][VB];
    if constexpr (F) {
      // S^T blocks: A = K rows j, B = Q rows i -> lane holds S[i_loc][j] for
      // j = 32 j_half + 16 jj + 4g + r.  Blocks wholly above the diagonal are
      // neither computed nor read.
      if (32 * j_half <= 16 * i_blk + 15) {
        Frag8<E> qf[NKK];
#pragma unroll
        for (int kk = 0; kk < NKK; ++kk)
          qf[kk] = *reinterpret_cast<const Frag8<E>*>(Qb + i_loc * KS + 32 * kk + 8 * g);
        f32x4 sacc[2];
#pragma unroll
        for (int jj = 0; jj < 2; ++jj) sacc[jj] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int kk = 0; kk < NKK; ++kk) {
          Frag8<E> kf[2];
#pragma unroll
          for (int jj = 0; jj < 2; ++jj)
            kf[jj] = *reinterpret_cast<const Frag8<E>*>(Kb + (32 * j_half + 16 * jj + n) * KS + 32 * kk + 8 * g);
#pragma unroll
          for (int jj = 0; jj < 2; ++jj) sacc[jj] = mfma8(kf[jj], qf[kk], sacc[jj]);
        }
#pragma unroll
        for (int jj = 0; jj < 2; ++jj)
          store4_raw<E>(Ps + i_loc * PS + 32 * j_half + 16 * jj + 4 * g,
                        sacc[jj] * f32x4{coef[jj][0], coef[jj][1], coef[jj][2], coef[jj][3]});
      }
      // O^T = M Q^T: A = state rows v (two accumulator tiles = one 32-deep
      // operand, key slots 32p + 4g + {0..3}, 32p + 16 + 4g + {0..3}), B = Q rows i.
#pragma unroll
      for (int ib = 0; ib < 4; ++ib)
#pragma unroll
        for (int vb = 0; vb < VB; ++vb) o[ib][vb] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int p = 0; p < NKK; ++p) {
        Frag8<E> mf[VB];
#pragma unroll
        for (int vb = 0; vb < VB; ++vb) {
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            mf[vb].e[r] = ET<E>::from_f(st[vb][2 * p][r]);
            mf[vb].e[4 + r] = ET<E>::from_f(st[vb][2 * p + 1][r]);
          }
        }
#pragma unroll
        for (int ib = 0; ib < 4; ++ib) {
          const raw* src = Qb + (16 * ib + n) * KS + 32 * p + 4 * g;
          const Frag8<E> qf = lds_frag_4x2<E>(src, src + 16);
#pragma unroll
          for (int vb = 0; vb < VB; ++vb) o[ib][vb] = mfma8(mf[vb], qf, o[ib][vb]);
        }
      }
#pragma unroll
      for (int ib = 0; ib < 4; ++ib)
#pragma unroll
        for (int vb = 0; vb < VB; ++vb) o[ib][vb] *= s_start[ib];
    }

    // V^T fragments (rows v, slots j = 32p + 16 (s / 4) + 4g + s % 4) for both
    // products; each transposed read covers 16 consecutive token rows.
    Frag8<E> vf[VB][2];
#pragma unroll
    for (int vb = 0; vb < VB; ++vb) {
#pragma unroll
      for (int p = 0; p < 2; ++p) {
        const raw* base = Vb + (32 * p + 4 * g + (n >> 2)) * VS + 16 * VB * w + 16 * vb + 4 * (n & 3);
        vf[vb][p] = frag_tr<E>(base, base + 16 * VS);
      }
    }
    // State update: M^T = decay^L M^T + K^T (w V); A = K^T rows k, B = (w V)^T rows v.
    {
      Frag8<E> wf[VB][2];
#pragma unroll
      for (int vb = 0; vb < VB; ++vb)
#pragma unroll
        for (int p = 0; p < 2; ++p)
#pragma unroll
          for (int s = 0; s < 8; ++s) wf[vb][p].e[s] = ET<E>::from_f(ET<E>::to_f(vf[vb][p].e[s]) * wgt[p][s]);
      const float decay_L = pw[L];
#pragma unroll
      for (int kt = 0; kt < KT; ++kt) {
        Frag8<E> kf[2];
#pragma unroll
        for (int p = 0; p < 2; ++p) {
          const raw* base = Kb + (32 * p + 4 * g + (n >> 2)) * KS + 16 * kt + 4 * (n & 3);
          kf[p] = frag_tr<E>(base, base + 16 * KS);
        }
#pragma unroll
        for (int vb = 0; vb < VB; ++vb) {
          f32x4 acc = st[vb][kt] * decay_L;
#pragma unroll
          for (int p = 0; p < 2; ++p) acc = mfma8(kf[p], wf[vb][p], acc);
          st[vb][kt] = acc;
        }
      }
    }

    store_chunk(cur ^ 1, nx, full);  // chunk c + 1 into the other buffer
    __syncthreads();                 // P complete; the previous output tile has left

    if constexpr (F) {
      // O^T += V^T P^T: A = V^T rows v, B = P rows i; P[i][j] = 0 for j > i.
#pragma unroll
      for (int ib = 0; ib < 4; ++ib) {
#pragma unroll
        for (int p = 0; p < 2; ++p) {
          if (32 * p > 16 * ib + 15) continue;
          const raw* src = Ps + (16 * ib + n) * PS + 32 * p + 4 * g;
          const Frag8<E> pf = lds_frag_4x2<E>(src, src + 16);
#pragma unroll
          for (int vb = 0; vb < VB; ++vb) o[ib][vb] = mfma8(vf[vb][p], pf, o[ib][vb]);
        }
#pragma unroll
        for (int vb = 0; vb < VB; ++vb)
          store4_raw<E>(Os + (16 * ib + n) * VS + 16 * VB * w + 16 * vb + 4 * g, o[ib][vb]);
      }
      if (a.snap_every > 0 && (snap_phase == 0 || c + 1 == n_chunks)) {
        const int si = c / a.snap_every;
        store_state(make_rsrc(a.snapshots + (b * a.n_snap + si) * dv * dk, static_cast<uint32_t>(dv * dk * 4)));
      }
      if (a.snap_every > 0) snap_phase = (snap_phase + 1 == a.snap_every) ? 0 : snap_phase + 1;
    }
  };

  // Per-token weights of a full chunk, causal coefficients and query decays,
  // from the power table in LDS.
  auto prepare_weights = [&]() {
    set_weights(CT);
    if constexpr (FULL) {
#pragma unroll
      for (int jj = 0; jj < 2; ++jj) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int j = 32 * j_half + 16 * jj + 4 * g + r;
          coef[jj][r] = (j <= i_loc) ? a.c * pw[max(i_loc - j, 0)] : 0.f;
        }
      }
#pragma unroll
      for (int ib = 0; ib < 4; ++ib) s_start[ib] = pw[16 * ib + n + 1];
    }
  };

  // Scans chunks [cb, ce) from the state in st.  issue() sends the starting
  // state's loads, then the first chunks' loads go out; only then does the
  // workgroup wait (for the power table, the oldest load) and finish() combine
  // the state while the chunks land.
  auto scan = [&](auto full, int cb, int ce, auto issue, auto finish) {
    constexpr bool F = decltype(full)::value;
    ce_cur = ce;
    Stage sg[PF];
    issue();
#pragma unroll
    for (int i = 0; i < PF; ++i) load_chunk(cb + i, sg[i], full);
    if (tid < PW_N) pw[tid] = pw_first;
    __syncthreads();  // pw visible
    prepare_weights();
    finish();
    store_chunk(0, sg[0], full);
    if (F) snap_phase = a.snap_every > 0 ? (cb + 1) % a.snap_every : 1;
    __syncthreads();
    for (int c = cb; c < ce; c += PF) {
#pragma unroll
      for (int i = 0; i < PF; ++i) {
        if (c + i < ce) step(c + i, cb, i & 1, sg[i], sg[(i + 1) % PF], full);
      }
    }
    if constexpr (F) {
      __syncthreads();
      flush_out(ce - 1);
    }
  };

  if constexpr (!FULL) {
    zero_state();
    scan(StateStep{}, c_begin, c_end, []() {}, []() {});
    store_state(part_rsrc(part));
    return;
  } else {
    const bool from_slot = a.part_starts && part > 0;
    scan(FullStep{}, c_begin, c_end, [&]() { issue_start(part, from_slot); },
         [&]() { finish_start(part, from_slot); });
    if (a.memory_out == nullptr || part != a.n_parts - 1) return;
    const __amdgpu_buffer_rsrc_t ro = make_rsrc(static_cast<unsigned char*>(a.memory_out) + b * dv * dk * mem_b,
                                                static_cast<uint32_t>(dv * dk * mem_b));
#pragma unroll
    for (int vb = 0; vb < VB; ++vb)
#pragma unroll
      for (int kt = 0; kt < KT; ++kt) st_state4<E>(ro, state_off(vb, kt), f32m, st[vb][kt]);
  }
}

template <class E, int DKP, bool FULL>
int launch_wide_pass(ChunkFwdArgs a, hipStream_t stream) {
  using S = WideShape<E, DKP, FULL>;
  static bool attr_set = false;
  if (!attr_set) {
    hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(&scan_wide_kernel<E, DKP, FULL>),
                                       hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(S::lds_bytes));
    if (e != hipSuccess) {
      set_error("chunk_update_fwd: hipFuncSetAttribute failed: %s", hipGetErrorString(e));
      return static_cast<int>(e);
    }
    attr_set = true;
  }
  const int64_t v_tiles = (a.dv + S::DVT - 1) / S::DVT;
  const int64_t grid = a.batch * (FULL ? a.n_parts : a.n_parts - 1) * v_tiles;
  if (grid > INT32_MAX) {
    set_error("chunk_update_fwd: batch too large for one launch");
    return GRM_HIP_EINVAL;
  }
  a.xcd_remap = (grid % 8 == 0) ? 1 : 0;
  hipLaunchKernelGGL((scan_wide_kernel<E, DKP, FULL>), dim3(static_cast<unsigned>(grid)), dim3(S::NT),
                     S::lds_bytes, stream, a);
  return check_launch(FULL ? "chunk_update_fwd" : "chunk_update_fwd(part states)");
}

// Part starting states in place of the contributions: slot q of part_states
// becomes M_{q+1} = pd M_q + D_q, one thread per four state elements.
__global__ void combine_parts_kernel(const void* memory, float* part_states, int64_t batch, int64_t n_parts,
                                     int64_t elems, int mem_f32, int mem_dtype, float part_decay) {
  const int64_t units = elems / 4;
  const int64_t total = batch * units;
  for (int64_t i = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; i < total;
       i += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    const int64_t b = i / units, u = i - b * units;
    f32x4 m;
    if (mem_f32) {
      m = reinterpret_cast<const f32x4*>(static_cast<const float*>(memory) + b * elems)[u];
    } else {
      const uint16_t* src = static_cast<const uint16_t*>(memory) + b * elems + 4 * u;
#pragma unroll
      for (int r = 0; r < 4; ++r) m[r] = mem_dtype == GRM_HIP_F16 ? ET<F16>::to_f(src[r]) : ET<BF16>::to_f(src[r]);
    }
    f32x4* slots = reinterpret_cast<f32x4*>(part_states + b * (n_parts - 1) * elems) + u;
    for (int64_t q = 0; q + 1 < n_parts; ++q) {
      m = m * part_decay + slots[q * units];
      slots[q * units] = m;
    }
  }
}

template <class E, int DKP>
int launch_wide(ChunkFwdArgs a, int mem_dtype, hipStream_t stream) {
  a.part_starts = 0;
  if (a.n_parts > 1) {
    const int rc = launch_wide_pass<E, DKP, false>(a, stream);
    if (rc != GRM_HIP_OK) return rc;
    if (a.n_parts > kCombineInPlaceParts) {
      const int64_t units = a.batch * (static_cast<int64_t>(a.dv) * a.dk / 4);
      const int64_t blocks = (units + 255) / 256 < 4096 ? (units + 255) / 256 : 4096;
      hipLaunchKernelGGL(combine_parts_kernel, dim3(static_cast<unsigned>(blocks)), dim3(256), 0, stream, a.memory,
                         a.part_states, a.batch, static_cast<int64_t>(a.n_parts),
                         static_cast<int64_t>(a.dv) * a.dk, a.mem_f32, mem_dtype, a.part_decay);
      const int rc2 = check_launch("chunk_update_fwd(part starts)");
      if (rc2 != GRM_HIP_OK) return rc2;
      a.part_starts = 1;
    }
  }
  return launch_wide_pass<E, DKP, true>(a, stream);
}

}  // namespace

bool wide_supported(int in_dtype, int64_t key_dim, int64_t value_dim, bool vec) {
  return vec && (in_dtype == GRM_HIP_BF16 || in_dtype == GRM_HIP_F16) && key_dim <= 128 && key_dim % 8 == 0 &&
         value_dim % 8 == 0;
}

int launch_scan_wide(const ChunkFwdArgs& a, int in_dtype, int mem_dtype, hipStream_t stream) {
  if (in_dtype == GRM_HIP_F16) {
    return a.dk <= 64 ? launch_wide<F16, 64>(a, mem_dtype, stream) : launch_wide<F16, 128>(a, mem_dtype, stream);
  }
  return a.dk <= 64 ? launch_wide<BF16, 64>(a, mem_dtype, stream) : launch_wide<BF16, 128>(a, mem_dtype, stream);
}

}  // namespace grmhip
