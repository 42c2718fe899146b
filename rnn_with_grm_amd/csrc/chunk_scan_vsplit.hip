// Fused chunked linear-memory update + query application (forward), value-split
// variant for bf16 / f16 inputs with key_dim <= 128, gfx950.
//
// Maths (reference grm/core/cuda_ops.py:218-254 chunked form; the per-token
// recurrence of grm/csrc/chunk_update.cu:82-123 and grm_cuda.cpp:74-83 is the
// same map): for a chunk of L tokens starting from state M (rows = value
// index v, columns = key index k), with c = (1 - decay) / sqrt(d_k),
//   h_i  = decay^{i+1} M q_i + c * sum_{j<=i} decay^{i-j} (q_i . k_j) v_j
//   M'   = decay^L M + c * sum_j decay^{L-1-j} v_j k_j^T
//
// Work decomposition.  Value columns are independent given K and Q, so each
// sequence is split into 32-column value tiles, one workgroup each, and every
// workgroup walks the whole sequence: no time split, no state pass, no re-read
// of K and V.  The tiles of one sequence run on one XCD and read the same K
// and Q rows, which the XCD's L2 serves after the first.
//
// The eight waves form a two-stage pipeline with one barrier per chunk; each
// half runs its own loop (same barrier count), so neither carries the other's
// registers.  In the step that scans chunk c:
//   P waves (0-3)  issue the loads of chunk c + PF (registers hold PF chunks),
//                  stage chunk c + 2 into LDS, flush the output tile of chunk
//                  c - 1, and compute S = Q K^T of chunk c + 1 (wave p: query block p against the
//                  key blocks at or below the diagonal), publishing
//                  P = S * c * decay^{i-j};
//   M waves (4-7)  waves 4-5 form O^T = decay^{i+1} M Q^T + V^T P^T for all
//                  32 value rows and 32 queries each, M read from a 16-bit copy
//                  in LDS; waves 6-7 hold the state (32 value rows x d/2 key
//                  columns each, fp32 MFMA accumulators), update it,
//                  M^T = decay^L M^T + K^T (w V), write the 16-bit copy the next
//                  step reads, and store the snapshot.
// Chunk data lives in three LDS stage buffers (written two steps ahead, read
// by the P waves one step ahead and by the M waves in their step); P, the
// output tile and the 16-bit state copy are double-buffered.  K^T and V^T
// operands come from the row-major tiles through the LDS transpose read
// (ds_read_b64_tr_b16).  K, Q, V and the output tile have unpadded rows whose
// 16-byte granules are XOR-swizzled by row, so that both the 16-byte reads of
// 16 rows and the transposed 8-byte reads of 8 rows x 32 bytes (one half-wave)
// land on distinct banks.
//
// Key width 128 (SO) moves the stores off the update waves' chain.  Issuing a
// snapshot's stores stalled those waves, the step's critical path, for about
// a third of the step once the snapshots go to HBM (64 sequences x 8192
// tokens), while the other six waves waited at the barrier.  There the state
// copy is fp32 (the output waves round their operand from it), the output
// waves store the hidden rows straight from their accumulators (two lane
// swaps give each lane 8 consecutive values; no output tile, no flush), and
// each snapshot is stored from the fp32 copy in whole lines: rows 16 vb +
// [0, 8) by the output waves in the next step, rows 16 vb + [8, 16) by the
// update waves right after writing the copy.  Splitting it so measured faster
// than either role storing all of it (or the update waves storing from their
// accumulators through a lane permutation), with the same bytes written.
#include <stdint.h>
#include <string.h>

#include "chunk_scan.h"
#include "grm_hip.h"
#include "grm_hip_common.h"

#include <type_traits>

namespace grmhip {
namespace {

typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) s16x4 lds_s16x4;

constexpr int kVsThreads = 512;   // 8 waves, two per SIMD
constexpr int kVsPThreads = 256;  // the P waves
constexpr int kVsStages = 3;      // LDS stage buffers

template <class E, int DKP>
struct VsShape {
  using raw = typename ET<E>::raw;
  static constexpr int DVT = kVsplitDv;  // value columns per workgroup
  // Row strides (elements): K, Q, V and the output tile unpadded and
  // swizzled (kq_at, v_at, o_at); the 16-bit state unpadded with 8-byte
  // pieces swizzled (m_at) at key_dim 128, 4 banks mod 64 otherwise; P 34
  // banks, the 8-byte reads of 16 rows on 32 distinct banks.
  static constexpr int KS = DKP;
  static constexpr int MS = DKP == 128 ? DKP : DKP + 8;
  static constexpr int VS = DVT;
  static constexpr int PS = CT + 4;
  static constexpr int OS = DVT;
  static constexpr int KH = DKP / 2;   // key columns of one state wave
  static constexpr int KT = KH / 16;   // 16-wide key tiles per state wave
  static constexpr int NKK = DKP / 32; // 32-deep key steps
  static constexpr int KU = DKP / 8;   // 16-byte units per K/Q row
  static constexpr int VU = DVT / 8;   // 16-byte units per V / output row
  static constexpr int K_UNITS = CT * KU / kVsPThreads;
  static constexpr int BUF = CT * (2 * KS + VS);  // K, Q, V of one chunk
  static constexpr int MB = DVT * MS;             // one 16-bit state copy
  // SO (key_dim 128): the state copy between the update and output waves is fp32, the
  // output waves store the snapshots from it and the hidden rows from their accumulators
  // (no output tile in LDS).
  static constexpr bool SO = DKP == 128;
  static constexpr int MFB = DVT * 128;  // floats in one fp32 state copy
  static constexpr size_t lds_elems =
      SO ? static_cast<size_t>(kVsStages * BUF + 2 * CT * PS)
         : static_cast<size_t>(kVsStages * BUF + 2 * CT * PS + 2 * CT * OS + 2 * MB);
  static constexpr size_t lds_bytes =
      lds_elems * sizeof(raw) + (SO ? 2 * MFB * sizeof(float) : 0) + PW_N * sizeof(float);
  static_assert(K_UNITS * kVsPThreads == CT * KU && CT * VU == kVsPThreads, "tiles split evenly");
  static_assert(lds_bytes <= kMaxLds, "tile set must fit one CU's LDS");
};

// Element offsets in the swizzled tiles; col is a multiple of 4 (an 8- or
// 16-byte piece inside one 16-byte granule).  K/Q rows of DKP elements:
// granule (col / 8) ^ s(row), s(row) = row & 15 for 16 granules per row (the
// 16-byte reads of 16 rows x 4 granules conflict-free; the transposed 8-byte
// reads of the state update pay 2-way, 32 of them against 72 16-byte reads a
// step), 2 ((row >> 1) & 3) | bit 3 of row for 8; rows 16 apart share s, so
// the two halves of a transposed fragment are 16 rows apart.
// V rows (32 elements): granule ^ 2 * bit 2 of row.
// LDS on gfx950, as measured with SQ_LDS_BANK_CONFLICT: 8-byte writes go in
// four passes of 16 consecutive lanes over 32 banks of 4 bytes, 8-byte reads
// in two passes of 32 consecutive lanes over 64 banks; a pass costs one cycle
// per distinct dword in its busiest bank.  The 16-bit state copy (key_dim 128:
// 32 pieces of 8 bytes per row) and the output tile (8 pieces per 64-byte
// row) are written as 8-byte columns of 16 rows and read as 8-byte pieces, so
// their pieces are swizzled by row for both: m_at spreads 16 rows of one
// column over 16 bank pairs and keeps a read pass's two lane groups (pieces
// 2 apart) apart by bit 4; o_at spreads the 8 rows of one parity over 8
// pieces and flips bit 0 between rows r and r + 4, which a read pass pairs.
__device__ __forceinline__ int m_at(int row, int col) {
  const int f = (row & 15) ^ ((row & 2) << 3);
  return row * 128 + ((((col >> 2) ^ f)) << 2) + (col & 3);
}
__device__ __forceinline__ int o_at(int row, int col) {
  const int f = ((row >> 1) & 7) ^ ((row >> 2) & 1);
  return row * kVsplitDv + ((((col >> 2) ^ f)) << 2) + (col & 3);
}

// fp32 state copy (SO): rows of 128 floats, 16-byte granule G (keys 4G .. 4G + 3)
// at G ^ (row & 15): the update waves' writes (16 rows x one granule per 16
// lanes), the output waves' operand reads (the same) and the snapshot reads (32
// consecutive granules of one row per 32 lanes) fall on distinct bank groups.
__device__ __forceinline__ int mf_at(int row, int G) { return row * 128 + 4 * (G ^ (row & 15)); }

template <int DKP>
__device__ __forceinline__ int kq_at(int row, int col) {
  const int s = DKP == 128 ? (row & 15) : ((((row >> 1) & 3) << 1) | ((row >> 3) & 1));
  return row * DKP + ((((col >> 3) ^ s)) << 3) + (col & 7);
}
__device__ __forceinline__ int v_at(int row, int col) {
  return row * kVsplitDv + (((col >> 3) ^ (((row >> 2) & 1) << 1)) << 3) + (col & 7);
}

// Stores of results nothing in this kernel reads again (hidden rows,
// snapshots, the final state) carry the non-temporal policy: without it the
// 20 KB a workgroup writes per chunk displace, in the XCD's L2, the K and Q
// lines its sibling value tiles are about to read, and the scan runs ~25%
// slower.  (Loads keep the default policy: K, Q and the 64-byte V slices are
// shared between the tiles of a sequence.)
constexpr int kStreamStore = 2;  // cache-policy bit NT


__device__ __forceinline__ void store_stream(__amdgpu_buffer_rsrc_t r, int off, u32x4 v) {
  __builtin_amdgcn_raw_buffer_store_b128(v, r, off, 0, kStreamStore);
}
__device__ __forceinline__ void store_stream_f32x4(__amdgpu_buffer_rsrc_t r, int off, f32x4 v) {
  u32x4 q;
#pragma unroll
  for (int i = 0; i < 4; ++i) q[i] = __float_as_uint(v[i]);
  store_stream(r, off, q);
}

template <class E>
__device__ __forceinline__ Frag8<E> vs_frag_tr(const typename ET<E>::raw* p_lo, const typename ET<E>::raw* p_hi) {
  // Four 16-bit elements of a row-major tile, transposed across each 16-lane
  // block: lane i of the block receives X[r0 + e][c0 + i] (e = 0..3) when lane
  // s of the block passes &X[r0 + (s >> 2)][c0 + 4 (s & 3)].
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

template <class E, int DKP, int PF>
__global__ __launch_bounds__(kVsThreads, 1) void scan_vsplit_kernel(const ChunkFwdArgs a) {
  using S = VsShape<E, DKP>;
  constexpr int DVT = S::DVT;
  using raw = typename ET<E>::raw;
  constexpr int KS = S::KS, MS = S::MS, PS = S::PS, OS = S::OS, KH = S::KH, KT = S::KT, NKK = S::NKK,
                KU = S::KU, VU = S::VU, K_UNITS = S::K_UNITS, BUF = S::BUF, MB = S::MB;
  constexpr int ES = static_cast<int>(sizeof(raw));
  static_assert(PF >= 3, "chunk c + 2 is staged in step c from registers loaded earlier");

  extern __shared__ __align__(16) unsigned char smem[];
  raw* stages = reinterpret_cast<raw*>(smem);     // 3 x { K [CT][KS], Q [CT][KS], V [CT][VS] }
  raw* Pbuf = stages + kVsStages * BUF;            // 2 x [CT][PS]  P = S * coef, row = query
  raw* Obuf = Pbuf + 2 * CT * PS;                  // 2 x [CT][OS]  output tile, row = query
  raw* Mbuf = Obuf + 2 * CT * OS;                  // 2 x [DVT][MS] state before a chunk, 16-bit
  float* Mf = reinterpret_cast<float*>(Pbuf + 2 * CT * PS);  // SO: 2 x [DVT][128] fp32 state
  float* pw = S::SO ? Mf + 2 * S::MFB : reinterpret_cast<float*>(Mbuf + 2 * MB);  // [PW_N]

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int g = lane >> 4;
  const int n = lane & 15;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const bool p_wave = w < 4;
  const int mw = w & 3;

  int wg = blockIdx.x;
  if (a.xcd_remap) {
    const int per = gridDim.x >> 3;
    wg = (wg & 7) * per + (wg >> 3);
  }
  // workgroup -> (sequence b, value tile); the tiles of a sequence are
  // adjacent, so after the remap they share an XCD (and its L2).
  const int v_tiles = a.v_tiles;
  const int vtile = wg % v_tiles;
  const int64_t b = wg / v_tiles;
  const int v0 = vtile * DVT;
  const int dk = a.dk, dv = a.dv;
  const int64_t T = a.seq_len;
  const int chunk = a.chunk;
  const int n_chunks = a.n_chunks;
  const bool f32m = a.mem_f32 != 0;

  const raw* keys = static_cast<const raw*>(a.keys) + b * T * dk;
  const raw* queries = static_cast<const raw*>(a.queries) + b * T * dk;
  const raw* values = static_cast<const raw*>(a.values) + b * T * dv;
  raw* hidden = a.hidden != nullptr ? static_cast<raw*>(a.hidden) + b * T * dv : nullptr;
  // Without hidden rows (the backward's recompute of the chunk states) nothing reads
  // Q, S or the output tiles: the queries are not loaded and S and O^T are skipped.
  const bool want_out = a.hidden != nullptr;

  // Chunk lengths in 32-bit scalar arithmetic: a 64-bit min here is a VALU
  // compare whose temporary VGPR pair the register allocator may take from a
  // prefetch destination still in flight, and the wait for that load then
  // drains the prefetch queue once per unrolled loop iteration.
  const int last_len = static_cast<int>(T - static_cast<int64_t>(n_chunks - 1) * chunk);
  auto chunk_len = [&](int c) -> int { return c < n_chunks - 1 ? chunk : c == n_chunks - 1 ? last_len : 0; };
  auto stage_k = [&](int c) { return stages + (c % kVsStages) * BUF; };

  // ======================= P waves: staging, S, output flush
  // K/Q unit u of P thread t is row (t + 256 u) / KU, 16-byte column
  // (t + 256 u) % KU (a wave reads whole rows); its V / output unit is row
  // t / VU of this workgroup's 32 columns.
  struct Stage {
    U8<E> k[K_UNITS];
    U8<E> q[K_UNITS];
    U8<E> v;
  };
  auto load_chunk = [&](int c, Stage& sg) {
    const int64_t t0 = static_cast<int64_t>(c) * chunk;
    const int L = chunk_len(c);
    const __amdgpu_buffer_rsrc_t rk = make_rsrc(keys + t0 * dk, static_cast<uint32_t>(L * dk * ES));
    const __amdgpu_buffer_rsrc_t rq = make_rsrc(queries + t0 * dk, static_cast<uint32_t>(want_out ? L * dk * ES : 0));
    const __amdgpu_buffer_rsrc_t rv = make_rsrc(values + t0 * dv, static_cast<uint32_t>(L * dv * ES));
#pragma unroll
    for (int u = 0; u < K_UNITS; ++u) {
      const int l = tid + kVsPThreads * u;
      const int row = l / KU, col = 8 * (l % KU);
      const int off = col < dk ? (row * dk + col) * ES : kBufOOB;
      sg.k[u] = buf_load8<E>(rk, off);
      sg.q[u] = buf_load8<E>(rq, off);
    }
    sg.v = buf_load8<E>(rv, ((tid / VU) * dv + v0 + 8 * (tid % VU)) * ES);
  };
  auto store_chunk = [&](int c, const Stage& sg) {
    raw* Kb = stage_k(c);
    raw* Qb = Kb + CT * KS;
    raw* Vb = Qb + CT * KS;
#pragma unroll
    for (int u = 0; u < K_UNITS; ++u) {
      const int l = tid + kVsPThreads * u;
      const int row = l / KU, col = 8 * (l % KU);
      *reinterpret_cast<U8<E>*>(Kb + kq_at<DKP>(row, col)) = sg.k[u];
      *reinterpret_cast<U8<E>*>(Qb + kq_at<DKP>(row, col)) = sg.q[u];
    }
    *reinterpret_cast<U8<E>*>(Vb + v_at(tid / VU, 8 * (tid % VU))) = sg.v;
  };
  // Chunk -1 stores nothing (an empty resource): every step then issues the
  // same memory instructions, which keeps the compiler's load-wait counts exact.
  auto flush_out = [&](int c) {
    const int64_t t0 = static_cast<int64_t>(max(c, 0)) * chunk;
    const int L = c >= 0 ? chunk_len(c) : 0;
    const __amdgpu_buffer_rsrc_t rh = make_rsrc(hidden + (hidden != nullptr ? t0 * dv : 0),
                                                static_cast<uint32_t>(hidden != nullptr ? L * dv * ES : 0));
    const int row = tid / VU, col = 8 * (tid % VU);
    const raw* Ob = Obuf + (c & 1) * CT * OS;
    const u32x2 lo = *reinterpret_cast<const u32x2*>(Ob + o_at(row, col));
    const u32x2 hi = *reinterpret_cast<const u32x2*>(Ob + o_at(row, col + 4));
    store_stream(rh, (row * dv + v0 + col) * ES, u32x4{lo[0], lo[1], hi[0], hi[1]});
  };
  // P wave p: S rows i = 16 p + n against key blocks jb <= p (lane holds
  // S[i][16 jb + 4g + r]); the blocks right of the diagonal are written as
  // zeros, so the M waves read whole P rows without branches.  The wave index
  // is a compile-time constant here: every K fragment the wave multiplies is
  // read first and its p + 1 block chains interleave.
  const int i_loc = 16 * mw + n;
  float coef[4][4];
  auto s_chunk = [&](int c, auto mw_c) {
    constexpr int MW = decltype(mw_c)::value;
    const raw* Kb = stage_k(c);
    const raw* Qb = Kb + CT * KS;
    raw* Pb = Pbuf + (c & 1) * CT * PS;
    Frag8<E> qf[NKK], kf[MW + 1][NKK];
#pragma unroll
    for (int kk = 0; kk < NKK; ++kk) qf[kk] = *reinterpret_cast<const Frag8<E>*>(Qb + kq_at<DKP>(16 * MW + n, 32 * kk + 8 * g));
#pragma unroll
    for (int jb = 0; jb <= MW; ++jb)
#pragma unroll
      for (int kk = 0; kk < NKK; ++kk)
        kf[jb][kk] = *reinterpret_cast<const Frag8<E>*>(Kb + kq_at<DKP>(16 * jb + n, 32 * kk + 8 * g));
    f32x4 sacc[MW + 1];
#pragma unroll
    for (int jb = 0; jb <= MW; ++jb) sacc[jb] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int kk = 0; kk < NKK; ++kk)
#pragma unroll
      for (int jb = 0; jb <= MW; ++jb) sacc[jb] = mfma8(kf[jb][kk], qf[kk], sacc[jb]);
#pragma unroll
    for (int jb = 0; jb < 4; ++jb) {
      const f32x4 val = jb <= MW ? sacc[jb <= MW ? jb : 0] * f32x4{coef[jb][0], coef[jb][1], coef[jb][2], coef[jb][3]}
                                 : f32x4{0.f, 0.f, 0.f, 0.f};
      store4_raw<E>(Pb + (16 * MW + n) * PS + 16 * jb + 4 * g, val);
    }
  };

  // ======================= M waves: output (waves 4-5) and state (waves 6-7)
  // O wave oq: O^T for all 32 value rows and the queries [32 oq, +32), from the
  //   16-bit state copy (M before the chunk), Q, V^T and P.
  // U wave uk: the state rows v in [0, 32) and key columns [KH uk, +KH) as fp32
  //   MFMA accumulators st[vb][kt], lane (g, n), register r = M[v][k] with
  //   v = v0 + 16 vb + n and k = KH uk + 16 kt + 4g + r; it updates them, writes
  //   them to the other 16-bit copy and stores the snapshot.
  // The two read different data, so each reads only what it multiplies.
  const bool o_wave = mw < 2;
  const int uk = mw & 1;
  f32x4 st[2][KT];
  auto state_off = [&](int vb, int kt) -> int {
    const int k = KH * uk + 16 * kt + 4 * g;
    return k < dk ? (v0 + 16 * vb + n) * dk + k : kBufOOB;
  };
  const int64_t mem_b = f32m ? 4 : ES;
  auto publish_state = [&](int slot) {
    if constexpr (S::SO) {
      float* M = Mf + slot * S::MFB;
#pragma unroll
      for (int vb = 0; vb < 2; ++vb)
#pragma unroll
        for (int kt = 0; kt < KT; ++kt)
          *reinterpret_cast<f32x4*>(M + mf_at(16 * vb + n, 16 * uk + 4 * kt + g)) = st[vb][kt];
      return;
    }
    raw* Mb = Mbuf + slot * MB;
#pragma unroll
    for (int vb = 0; vb < 2; ++vb)
#pragma unroll
      for (int kt = 0; kt < KT; ++kt) {
        const int row = 16 * vb + n, col = KH * uk + 16 * kt + 4 * g;
        store4_raw<E>(Mb + (DKP == 128 ? m_at(row, col) : row * MS + col), st[vb][kt]);
      }
  };
  // O waves: decay^{i+1} for the query rows i = 32 oq + 16 ib + n of this lane's output tiles.
  float s_start[2];
  // U waves: state-update weights c * decay^{L-1-j} for this lane's slots
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
  // V^T fragments (rows v, slots j = 32p + 16 (s / 4) + 4g + s % 4) for both
  // products; each transposed read covers 16 consecutive token rows.  P rows
  // and K^T fragments use the same slot order.
  auto v_frags = [&](const raw* Vb, Frag8<E>(&vf)[2][2]) {
#pragma unroll
    for (int vb = 0; vb < 2; ++vb)
#pragma unroll
      for (int p = 0; p < 2; ++p) {
        const raw* base = Vb + v_at(32 * p + 4 * g + (n >> 2), 16 * vb + 4 * (n & 3));
        vf[vb][p] = vs_frag_tr<E>(base, base + 16 * S::VS);
      }
  };
  // SO: output wave oq stores state rows [16 oq, + 8) of a snapshot from the fp32
  // copy in slot `slot`, two whole 512-byte rows per store; update wave uk stores
  // rows 16 vb + [8, 16) of its key half [64 uk, + 64), four 256-byte row halves
  // per store, right after writing them to the copy.
  auto o_snap = [&](int si, int slot, int oq) {
    const float* M = Mf + slot * S::MFB;
    const __amdgpu_buffer_rsrc_t rs =
        make_rsrc(a.snapshots + (b * a.n_snap + si) * dv * dk, static_cast<uint32_t>(dv * dk * 4));
    const int G = lane & 31, h = lane >> 5;
    // one lane offset; the row offsets 2j apart go in the scalar offset
    const int voff = 4 * G < dk ? ((v0 + 16 * oq + h) * dk + 4 * G) * 4 : kBufOOB;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const f32x4 v = *reinterpret_cast<const f32x4*>(M + mf_at(16 * oq + 2 * j + h, G));
      u32x4 q;
#pragma unroll
      for (int i = 0; i < 4; ++i) q[i] = __float_as_uint(v[i]);
      __builtin_amdgcn_raw_buffer_store_b128(q, rs, voff, 8 * dk * j, kStreamStore);
    }
  };
  // Every LDS operand of a step is read first, so the reads overlap one another
  // instead of each waiting for the product before it.
  auto o_chunk = [&](int c, auto oq_c) {
    constexpr int oq = decltype(oq_c)::value;
    const raw* Qb = stage_k(c) + CT * KS;
    const raw* Vb = Qb + CT * KS;
    const raw* Pb = Pbuf + (c & 1) * CT * PS;
    const raw* Mb = Mbuf + (c & 1) * MB;
    raw* Ob = Obuf + (c & 1) * CT * OS;
    Frag8<E> mf[2][NKK], qf[2][NKK], vf[2][2], pf[2][2];
#pragma unroll
    for (int kk = 0; kk < NKK; ++kk) {
#pragma unroll
      for (int vb = 0; vb < 2; ++vb) {
        const int row = 16 * vb + n, col = 32 * kk + 8 * g;
        if constexpr (S::SO) {
          const float* M = Mf + (c & 1) * S::MFB;
          const f32x4 lo = *reinterpret_cast<const f32x4*>(M + mf_at(row, 8 * kk + 2 * g));
          const f32x4 hi = *reinterpret_cast<const f32x4*>(M + mf_at(row, 8 * kk + 2 * g + 1));
          mf[vb][kk] = __builtin_bit_cast(Frag8<E>, u32x4{pack2<E>(lo[0], lo[1]), pack2<E>(lo[2], lo[3]),
                                                          pack2<E>(hi[0], hi[1]), pack2<E>(hi[2], hi[3])});
        } else if constexpr (DKP == 128) {
          mf[vb][kk] = lds_frag_4x2<E>(Mb + m_at(row, col), Mb + m_at(row, col + 4));
        } else {
          mf[vb][kk] = *reinterpret_cast<const Frag8<E>*>(Mb + row * MS + col);
        }
      }
#pragma unroll
      for (int ib = 0; ib < 2; ++ib)
        qf[ib][kk] = *reinterpret_cast<const Frag8<E>*>(Qb + kq_at<DKP>(32 * oq + 16 * ib + n, 32 * kk + 8 * g));
    }
    v_frags(Vb, vf);
    // P slots 0-3 of fragment p are key block 2p, slots 4-7 key block 2p + 1;
    // blocks right of the diagonal (never written) are taken as zeros, and a
    // fragment wholly right of it is skipped.
#pragma unroll
    for (int ib = 0; ib < 2; ++ib) {
      const int iblk = 2 * oq + ib;
#pragma unroll
      for (int p = 0; p < 2; ++p) {
        if (2 * p > iblk) continue;
        const raw* src = Pb + (16 * iblk + n) * PS + 32 * p + 4 * g;
        pf[ib][p] = lds_frag_4x2<E>(src, src + 16);
        if (2 * p + 1 > iblk) {
#pragma unroll
          for (int e = 4; e < 8; ++e) pf[ib][p].e[e] = 0;
        }
      }
    }
    // O^T = decay^{i+1} M Q^T + V^T P^T: A = state rows v (16-bit, from the copy) then
    // V^T rows v; B = Q rows i then P rows i.
    __amdgpu_buffer_rsrc_t rh;
    if constexpr (S::SO) {
      const int64_t t0 = static_cast<int64_t>(c) * chunk;
      rh = make_rsrc(hidden + (hidden != nullptr ? t0 * dv : 0),
                     static_cast<uint32_t>(hidden != nullptr ? chunk_len(c) * dv * ES : 0));
    }
#pragma unroll
    for (int ib = 0; ib < 2; ++ib) {
      const int iblk = 2 * oq + ib;
      f32x4 ov[2];
#pragma unroll
      for (int vb = 0; vb < 2; ++vb) {
        f32x4 o = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int kk = 0; kk < NKK; ++kk) o = mfma8(mf[vb][kk], qf[ib][kk], o);
        o *= s_start[ib];
#pragma unroll
        for (int p = 0; p < 2; ++p) {
          if (2 * p > iblk) continue;
          o = mfma8(vf[vb][p], pf[ib][p], o);
        }
        if constexpr (S::SO) {
          ov[vb] = o;
        } else {
          store4_raw<E>(Ob + o_at(16 * iblk + n, 16 * vb + 4 * g), o);
        }
      }
      if constexpr (S::SO) {
        // Lane (g, n) holds values 4g .. 4g + 3 of both 16-value halves of token
        // 16 iblk + n; two swaps give it values 8g .. 8g + 7, one 16-byte store.
        const auto s0 = __builtin_amdgcn_permlane32_swap(pack2<E>(ov[0][0], ov[0][1]), pack2<E>(ov[1][0], ov[1][1]),
                                                         false, false);
        const auto s1 = __builtin_amdgcn_permlane32_swap(pack2<E>(ov[0][2], ov[0][3]), pack2<E>(ov[1][2], ov[1][3]),
                                                         false, false);
        const auto t0 = __builtin_amdgcn_permlane16_swap(s0[0], s0[1], false, false);
        const auto t1 = __builtin_amdgcn_permlane16_swap(s1[0], s1[1], false, false);
        store_stream(rh, ((16 * iblk + n) * dv + v0 + 8 * g) * ES, u32x4{t0[0], t1[0], t0[1], t1[1]});
      }
    }
    if constexpr (S::SO) {
      if (a.snap_every > 0 && c > 0 && c % a.snap_every == 0) o_snap(c / a.snap_every - 1, c & 1, oq);
    }
  };
  int snap_phase = a.snap_every > 0 ? 1 % a.snap_every : 1;  // == 0: a snapshot follows the current chunk
  auto u_chunk = [&](int c) {
    const int L = chunk_len(c);
    const raw* Kb = stage_k(c);
    const raw* Vb = Kb + 2 * CT * KS;
    if (L != CT) set_weights(L);
    Frag8<E> vf[2][2], kf[KT][2];
    v_frags(Vb, vf);
#pragma unroll
    for (int p = 0; p < 2; ++p)
#pragma unroll
      for (int kt = 0; kt < KT; ++kt) {
        const raw* kb = Kb + kq_at<DKP>(32 * p + 4 * g + (n >> 2), KH * uk + 16 * kt + 4 * (n & 3));
        kf[kt][p] = vs_frag_tr<E>(kb, kb + 16 * KS);
      }
    // State update: M^T = decay^L M^T + K^T (w V); A = K^T rows k, B = (w V)^T rows v.
    Frag8<E> wf[2][2];
#pragma unroll
    for (int vb = 0; vb < 2; ++vb)
#pragma unroll
      for (int p = 0; p < 2; ++p)
#pragma unroll
        for (int s = 0; s < 8; ++s) wf[vb][p].e[s] = ET<E>::from_f(ET<E>::to_f(vf[vb][p].e[s]) * wgt[p][s]);
    const float decay_L = pw[L];
#pragma unroll
    for (int vb = 0; vb < 2; ++vb)
#pragma unroll
      for (int kt = 0; kt < KT; ++kt) {
        f32x4 acc = st[vb][kt] * decay_L;
#pragma unroll
        for (int p = 0; p < 2; ++p) acc = mfma8(kf[kt][p], wf[vb][p], acc);
        st[vb][kt] = acc;
      }
    // The snapshot's stores go out before the 16-bit copy for the output waves
    // (measured about 1% faster at 64 x 8192 tokens, same results).
    if (!S::SO && a.snap_every > 0 && (snap_phase == 0 || c + 1 == n_chunks)) {
      const int si = c / a.snap_every;
      const __amdgpu_buffer_rsrc_t rs =
          make_rsrc(a.snapshots + (b * a.n_snap + si) * dv * dk, static_cast<uint32_t>(dv * dk * 4));
      if (a.snap_full_lines && KT % 2 == 0) {
        // Whole 128-byte lines per store (full_line_pair): key tiles 2p and 2p + 1
        // hold the two halves of every line of the wave's rows.
        const int half = n >> 3;
#pragma unroll
        for (int vb = 0; vb < 2; ++vb)
#pragma unroll
          for (int p = 0; p < KT / 2; ++p) {
            f32x4 oa, ob;
            full_line_pair(st[vb][2 * p], st[vb][2 * p + 1], n, oa, ob);
            const int k = KH * uk + 32 * p + 4 * (2 * g + half);
            const int offa = k < dk ? (v0 + 16 * vb + (n & 7)) * dk + k : kBufOOB;
            const int offb = k < dk ? (v0 + 16 * vb + 8 + (n & 7)) * dk + k : kBufOOB;
            store_stream_f32x4(rs, offa == kBufOOB ? kBufOOB : offa * 4, oa);
            store_stream_f32x4(rs, offb == kBufOOB ? kBufOOB : offb * 4, ob);
          }
      } else {
#pragma unroll
        for (int vb = 0; vb < 2; ++vb)
#pragma unroll
          for (int kt = 0; kt < KT; ++kt) {
            const int off = state_off(vb, kt);
            store_stream_f32x4(rs, off == kBufOOB ? kBufOOB : off * 4, st[vb][kt]);
          }
      }
    }
    publish_state((c + 1) & 1);
    if constexpr (S::SO) {
      // Rows 16 vb + [8, 16) of this wave's key half, read back from the copy it has
      // just written (its own writes: no barrier needed), four rows x 256 bytes per
      // store; the row offsets 4 and 16 apart go in the scalar offset.
      if (a.snap_every > 0 && (snap_phase == 0 || c + 1 == n_chunks)) {
        const float* M = Mf + ((c + 1) & 1) * S::MFB;
        const __amdgpu_buffer_rsrc_t rs = make_rsrc(a.snapshots + (b * a.n_snap + c / a.snap_every) * dv * dk,
                                                    static_cast<uint32_t>(dv * dk * 4));
        const int G = 16 * uk + (lane & 15), q = lane >> 4;
        const int voff = 4 * G < dk ? ((v0 + 8 + q) * dk + 4 * G) * 4 : kBufOOB;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int dr = 16 * (j >> 1) + 4 * (j & 1);
          const f32x4 v = *reinterpret_cast<const f32x4*>(M + mf_at(8 + dr + q, G));
          u32x4 qv;
#pragma unroll
          for (int i = 0; i < 4; ++i) qv[i] = __float_as_uint(v[i]);
          __builtin_amdgcn_raw_buffer_store_b128(qv, rs, voff, 4 * dk * dr, kStreamStore);
        }
      }
    }
    if (a.snap_every > 0) snap_phase = (snap_phase + 1 == a.snap_every) ? 0 : snap_phase + 1;
  };

  // ======================= the two loops
  // Barriers: one after the prologue, one at the top of each step, one before
  // the last flush; both halves pass the same number.  In step c the barrier
  // orders every LDS producer before its consumers, and each buffer's next
  // writer runs at least one step after its last reader.
  static_assert(PW_N <= kVsPThreads, "one power per P thread");
  auto p_loop = [&](auto mw_c) {
    const float pw_first = tid < PW_N ? a.pw[tid] : 0.f;
    Stage sg[PF];
#pragma unroll
    for (int i = 0; i < PF; ++i) load_chunk(i, sg[i]);
    if (tid < PW_N) pw[tid] = pw_first;
    store_chunk(0, sg[0]);
    store_chunk(1, sg[1]);
    __syncthreads();  // pw, chunks 0 and 1, M_0
#pragma unroll
    for (int jb = 0; jb < 4; ++jb) {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int j = 16 * jb + 4 * g + r;
        coef[jb][r] = (j <= i_loc) ? a.c * pw[max(i_loc - j, 0)] : 0.f;
      }
    }
    if (want_out) s_chunk(0, mw_c);
    // Step c: load chunk c + PF into the slot chunk c held, stage chunk c + 2,
    // flush chunk c - 1's output, S of chunk c + 1.
    for (int c = 0; c < n_chunks; c += PF) {
#pragma unroll
      for (int i = 0; i < PF; ++i) {
        if (c + i >= n_chunks) break;
        __syncthreads();
        load_chunk(c + i + PF, sg[i]);
        store_chunk(c + i + 2, sg[(i + 2) % PF]);
        if constexpr (!S::SO) flush_out(c + i - 1);
        if (want_out && c + i + 1 < n_chunks) s_chunk(c + i + 1, mw_c);
      }
    }
    __syncthreads();
    if constexpr (!S::SO) flush_out(n_chunks - 1);
  };
  if (p_wave) {
    if (mw == 0) {
      p_loop(std::integral_constant<int, 0>{});
    } else if (mw == 1) {
      p_loop(std::integral_constant<int, 1>{});
    } else if (mw == 2) {
      p_loop(std::integral_constant<int, 2>{});
    } else {
      p_loop(std::integral_constant<int, 3>{});
    }
    return;
  }

  if (!o_wave) {
    const __amdgpu_buffer_rsrc_t rmem = make_rsrc(static_cast<const unsigned char*>(a.memory) + b * dv * dk * mem_b,
                                                  static_cast<uint32_t>(dv * dk * mem_b));
#pragma unroll
    for (int vb = 0; vb < 2; ++vb)
#pragma unroll
      for (int kt = 0; kt < KT; ++kt) {
        const int off = state_off(vb, kt);
        if (f32m) {
          const u32x4 u = __builtin_amdgcn_raw_buffer_load_b128(rmem, off == kBufOOB ? kBufOOB : off * 4, 0, 0);
#pragma unroll
          for (int i = 0; i < 4; ++i) st[vb][kt][i] = __uint_as_float(u[i]);
        } else {
          const u32x2 u = __builtin_amdgcn_raw_buffer_load_b64(rmem, off == kBufOOB ? kBufOOB : off * ES, 0, 0);
          st[vb][kt][0] = ET<E>::to_f(static_cast<raw>(u[0] & 0xffffu));
          st[vb][kt][1] = ET<E>::to_f(static_cast<raw>(u[0] >> 16));
          st[vb][kt][2] = ET<E>::to_f(static_cast<raw>(u[1] & 0xffffu));
          st[vb][kt][3] = ET<E>::to_f(static_cast<raw>(u[1] >> 16));
        }
      }
    publish_state(0);
  }
  // The M waves carry the step's dependency chain: when an M wave and a P
  // wave of one SIMD are both ready, the M wave issues first.
  __builtin_amdgcn_s_setprio(2);
  __syncthreads();  // pw, chunks 0 and 1, M_0
  if (o_wave) {
#pragma unroll
    for (int ib = 0; ib < 2; ++ib) s_start[ib] = pw[32 * (mw & 1) + 16 * ib + n + 1];
  } else {
    set_weights(CT);
  }
  // Step c: scan chunk c.
  for (int c = 0; c < n_chunks; ++c) {
    __syncthreads();
    if (mw >= 2) {
      u_chunk(c);
    } else if (want_out) {
      if (mw == 0) {
        o_chunk(c, std::integral_constant<int, 0>{});
      } else {
        o_chunk(c, std::integral_constant<int, 1>{});
      }
    } else if constexpr (S::SO) {
      if (a.snap_every > 0 && c > 0 && c % a.snap_every == 0) o_snap(c / a.snap_every - 1, c & 1, mw & 1);
    }
  }
  __syncthreads();
  if constexpr (S::SO) {
    if (o_wave && a.snap_every > 0) o_snap((n_chunks - 1) / a.snap_every, n_chunks & 1, mw & 1);
  }
  if (o_wave || a.memory_out == nullptr) return;
  const __amdgpu_buffer_rsrc_t ro = make_rsrc(static_cast<unsigned char*>(a.memory_out) + b * dv * dk * mem_b,
                                              static_cast<uint32_t>(dv * dk * mem_b));
#pragma unroll
  for (int vb = 0; vb < 2; ++vb)
#pragma unroll
    for (int kt = 0; kt < KT; ++kt) {
      const int off = state_off(vb, kt);
      if (f32m) {
        store_stream_f32x4(ro, off == kBufOOB ? kBufOOB : off * 4, st[vb][kt]);
      } else {
        buf_store4<E>(ro, off == kBufOOB ? kBufOOB : off * ES, st[vb][kt]);
      }
    }
}

template <class E, int DKP>
int launch_vsplit(ChunkFwdArgs a, hipStream_t stream) {
  using S = VsShape<E, DKP>;
  constexpr int PF = kVsplitPrefetch;
  static bool attr_set = false;
  if (!attr_set) {
    hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(&scan_vsplit_kernel<E, DKP, PF>),
                                       hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(S::lds_bytes));
    if (e != hipSuccess) {
      set_error("chunk_update_fwd: hipFuncSetAttribute failed: %s", hipGetErrorString(e));
      return static_cast<int>(e);
    }
    attr_set = true;
  }
  if (a.n_parts != 1 || a.v_tiles * S::DVT != a.dv) {
    set_error("chunk_update_fwd: value-split scan needs one part and value_dim = %d x tiles", S::DVT);
    return GRM_HIP_EINVAL;
  }
  const int64_t grid = a.batch * a.v_tiles;
  if (grid > INT32_MAX) {
    set_error("chunk_update_fwd: batch too large for one launch");
    return GRM_HIP_EINVAL;
  }
  a.xcd_remap = (grid % 8 == 0) ? 1 : 0;
  hipLaunchKernelGGL((scan_vsplit_kernel<E, DKP, PF>), dim3(static_cast<unsigned>(grid)), dim3(kVsThreads),
                     S::lds_bytes, stream, a);
  return check_launch("chunk_update_fwd");
}

}  // namespace

bool vsplit_supported(int in_dtype, int64_t key_dim, int64_t value_dim, bool vec) {
  return wide_supported(in_dtype, key_dim, value_dim, vec) && value_dim % kVsplitDv == 0;
}

int launch_scan_vsplit(const ChunkFwdArgs& a, int in_dtype, hipStream_t stream) {
  if (in_dtype == GRM_HIP_F16) {
    return a.dk <= 64 ? launch_vsplit<F16, 64>(a, stream) : launch_vsplit<F16, 128>(a, stream);
  }
  return a.dk <= 64 ? launch_vsplit<BF16, 64>(a, stream) : launch_vsplit<BF16, 128>(a, stream);
}

}  // namespace grmhip
