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

#include "grm_hip.h"
#include "grm_hip_common.h"

namespace grmhip {
namespace {

constexpr int CT = 64;         // token rows per chunk tile
constexpr int NW = 4;          // waves per workgroup
constexpr int NTHR = 64 * NW;  // threads per workgroup
constexpr int PW_N = CT + 1;   // decay^0 .. decay^64

struct ChunkFwdArgs {
  const void* keys;
  const void* values;
  const void* queries;
  const void* memory;
  void* hidden;
  void* memory_out;
  float* snapshots;
  int64_t batch;
  int64_t seq_len;
  int dk;
  int dv;
  int chunk;       // tokens per chunk, 1..64
  int n_chunks;
  int snap_every;  // chunks per snapshot; 0 = no snapshots
  int n_snap;
  int v_tiles;     // workgroups per sequence
  int mem_f32;     // memory / memory_out are float32 (else the input dtype)
  int vec_k;       // keys/queries rows allow 8-element vector loads
  int vec_v;       // values rows allow 8-element vector loads
  int vec_o;       // hidden rows allow 4-element vector stores
  int vec_m;       // memory/memory_out/snapshot rows allow 4-element vector access
  int xcd_remap;   // grid is a multiple of 8: place a sequence's tiles on one XCD
  float c;         // (1 - decay) / sqrt(d_k)
  float pw[PW_N];  // decay^n rounded from double
};

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
  static constexpr int KS = DKP + 8;  // LDS row stride (elements) of K and of the state copy
  static constexpr int VS = CT + 4;   // LDS row stride (elements) of V^T
  static constexpr int NKK = DKP / 32;
  static constexpr int VT = DV / 16;
  static constexpr int KT = DKP / 16;
  static constexpr int KTW = (KT + NW - 1) / NW;  // state key-tiles per wave
  static constexpr int NJP = CT / 32;             // 32-token slices of a chunk
  static constexpr int K_UNITS = CT * DKP / 8 / NTHR;
  static constexpr int V_UNITS = CT * DV / 8;     // <= NTHR
  static constexpr size_t lds_bytes =
      (static_cast<size_t>(CT) * KS + static_cast<size_t>(DV) * KS + static_cast<size_t>(DV) * VS) *
          sizeof(raw) +
      PW_N * sizeof(float);
  static_assert(K_UNITS * NTHR * 8 == CT * DKP, "K tile must split evenly over the workgroup");
  static_assert(V_UNITS <= NTHR, "V tile must fit one unit per thread");
};

template <class E, int DKP, int DV>
__global__ __launch_bounds__(NTHR) void chunk_fwd_kernel(const ChunkFwdArgs a) {
  using S = FwdShape<E, DKP, DV>;
  using raw = typename ET<E>::raw;
  constexpr int KS = S::KS, VS = S::VS, NKK = S::NKK, VT = S::VT, KT = S::KT, KTW = S::KTW,
                NJP = S::NJP, K_UNITS = S::K_UNITS, V_UNITS = S::V_UNITS;

  extern __shared__ __align__(16) unsigned char smem[];
  raw* Ks = reinterpret_cast<raw*>(smem);        // [CT][KS]   keys of the chunk
  raw* Mb = Ks + CT * KS;                        // [DV][KS]   state copy, row = value index
  raw* Vt = Mb + DV * KS;                        // [DV][VS]   values of the chunk, transposed
  float* pw = reinterpret_cast<float*>(Vt + DV * VS);  // [PW_N]

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
  const int64_t b = wg / a.v_tiles;
  const int v0 = (wg % a.v_tiles) * DV;
  const int dk = a.dk, dv = a.dv;
  const int64_t T = a.seq_len;
  const int chunk = a.chunk;
  const bool f32m = a.mem_f32 != 0;
  const bool vec_k = a.vec_k != 0, vec_v = a.vec_v != 0, vec_o = a.vec_o != 0,
             vec_m = a.vec_m != 0;

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
      st[q][vt] = (kt < KT) ? load_state4<E>(a.memory, (b * dv + v) * dk, 16 * kt + 4 * g, dk,
                                             v < dv, f32m, vec_m)
                            : f32x4{0.f, 0.f, 0.f, 0.f};
    }
  }

  // ---- chunk staging (global -> registers -> LDS)
  U8<E> kst[K_UNITS];
  U8<E> vst;
  Frag8<E> qf[NKK], qn[NKK];
  const int i_loc = 16 * w + n;  // this lane's query row within a chunk

  auto load_chunk = [&](int c, U8<E>* kd, U8<E>& vd, Frag8<E>* qd) {
    const int64_t t0 = static_cast<int64_t>(c) * chunk;
    const int L = static_cast<int>(min(static_cast<int64_t>(chunk), T - t0));
#pragma unroll
    for (int u = 0; u < K_UNITS; ++u) {
      const int idx = tid + NTHR * u;
      const int row = idx / (DKP / 8);
      const int col = (idx % (DKP / 8)) * 8;
      kd[u] = load_u8<E>(keys + (t0 + row) * dk, col, dk, row < L, vec_k);
    }
    if (V_UNITS == NTHR || tid < V_UNITS) {
      const int row = tid / (DV / 8);
      const int col = v0 + (tid % (DV / 8)) * 8;
      vd = load_u8<E>(values + (t0 + row) * dv, col, dv, row < L, vec_v);
    }
#pragma unroll
    for (int kk = 0; kk < NKK; ++kk) {
      U8<E> u = load_u8<E>(queries + (t0 + i_loc) * dk, 32 * kk + 8 * g, dk, i_loc < L, vec_k);
      qd[kk] = __builtin_bit_cast(Frag8<E>, u);
    }
  };
  auto store_chunk = [&](const U8<E>* kd, const U8<E>& vd) {
#pragma unroll
    for (int u = 0; u < K_UNITS; ++u) {
      const int idx = tid + NTHR * u;
      const int row = idx / (DKP / 8);
      const int col = (idx % (DKP / 8)) * 8;
      *reinterpret_cast<U8<E>*>(Ks + row * KS + col) = kd[u];
    }
    if (V_UNITS == NTHR || tid < V_UNITS) {
      const int row = tid / (DV / 8);
      const int c8 = tid % (DV / 8);
#pragma unroll
      for (int e = 0; e < 8; ++e) Vt[(8 * c8 + e) * VS + row] = vd.e[e];
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

  if (a.n_chunks > 0) {
    load_chunk(0, kst, vst, qf);
    store_chunk(kst, vst);
  }
  store_state_copy();
  __syncthreads();

  // Causal decay coefficients of S, fixed for every chunk: lane row i = i_loc,
  // column j = 16 jb + 4 g + r.
  float coef[4][4];
#pragma unroll
  for (int jb = 0; jb < 4; ++jb) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int j = 16 * jb + 4 * g + r;
      coef[jb][r] = (jb <= w && j <= i_loc) ? a.c * pw[i_loc - j] : 0.f;
    }
  }

  for (int c = 0; c < a.n_chunks; ++c) {
    const int64_t t0 = static_cast<int64_t>(c) * chunk;
    const int L = static_cast<int>(min(static_cast<int64_t>(chunk), T - t0));
    if (c > 0) __syncthreads();  // LDS K, V^T and state copy of chunk c are in place
    const bool has_next = c + 1 < a.n_chunks;
    if (has_next) load_chunk(c + 1, kst, vst, qn);

    // V^T fragments: rows v = 16 vt + n; slot s < 4 -> j = 32p + 4g + s,
    // s >= 4 -> j = 32p + 16 + 4g + (s - 4).  Shared by O and the state update.
    Frag8<E> vf[VT][NJP];
#pragma unroll
    for (int vt = 0; vt < VT; ++vt) {
#pragma unroll
      for (int p = 0; p < NJP; ++p) {
        const raw* src = Vt + (16 * vt + n) * VS + 32 * p + 4 * g;
        vf[vt][p] = lds_frag_4x2<E>(src, src + 16);
      }
    }

    if (16 * w < L) {
      // S^T blocks: A = K rows j, B = Q rows i -> lane holds S[i = i_loc][j = 16jb + 4g + r].
      f32x4 sacc[4];
#pragma unroll
      for (int jb = 0; jb < 4; ++jb) {
        sacc[jb] = f32x4{0.f, 0.f, 0.f, 0.f};
        if (jb <= w) {
#pragma unroll
          for (int kk = 0; kk < NKK; ++kk) {
            const Frag8<E> kf =
                *reinterpret_cast<const Frag8<E>*>(Ks + (16 * jb + n) * KS + 32 * kk + 8 * g);
            sacc[jb] = mfma8(kf, qf[kk], sacc[jb]);
          }
        }
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
      const float s_start = (i_loc < L) ? pw[i_loc + 1] : 0.f;
#pragma unroll
      for (int vt = 0; vt < VT; ++vt) {
        // O^T: A = state rows v, B = Q rows i -> lane holds O[i_loc][16vt + 4g + r].
        f32x4 o = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int kk = 0; kk < NKK; ++kk) {
          const Frag8<E> mf =
              *reinterpret_cast<const Frag8<E>*>(Mb + (16 * vt + n) * KS + 32 * kk + 8 * g);
          o = mfma8(mf, qf[kk], o);
        }
        o *= s_start;
#pragma unroll
        for (int p = 0; p < NJP; ++p) {
          if (32 * p < 16 * (w + 1)) o = mfma8(vf[vt][p], pf[p], o);
        }
        if (i_loc < L && a.hidden != nullptr)
          store4<E>(hidden + (t0 + i_loc) * dv, v0 + 16 * vt + 4 * g, o, dv, vec_o);
      }
    }

    // State update.  Weights c * decay^{L-1-j} ride on the K^T operand.
    float wt[NJP][8];
#pragma unroll
    for (int p = 0; p < NJP; ++p) {
#pragma unroll
      for (int s = 0; s < 8; ++s) {
        const int j = 32 * p + (s < 4 ? 4 * g + s : 16 + 4 * g + (s - 4));
        wt[p][s] = (j < L) ? a.c * pw[L - 1 - j] : 0.f;
      }
    }
    const float decay_L = pw[L];
#pragma unroll
    for (int q = 0; q < KTW; ++q) {
      const int kt = w + NW * q;
      if (kt < KT) {
        Frag8<E> kf[NJP];
#pragma unroll
        for (int p = 0; p < NJP; ++p) {
#pragma unroll
          for (int s = 0; s < 8; ++s) {
            const int j = 32 * p + (s < 4 ? 4 * g + s : 16 + 4 * g + (s - 4));
            kf[p].e[s] = ET<E>::from_f(ET<E>::to_f(Ks[j * KS + 16 * kt + n]) * wt[p][s]);
          }
        }
#pragma unroll
        for (int vt = 0; vt < VT; ++vt) {
          f32x4 acc = st[q][vt] * decay_L;
#pragma unroll
          for (int p = 0; p < NJP; ++p) acc = mfma8(kf[p], vf[vt][p], acc);
          st[q][vt] = acc;
        }
      }
    }

    if (a.snap_every > 0 && ((c + 1) % a.snap_every == 0 || c + 1 == a.n_chunks)) {
      const int si = c / a.snap_every;
#pragma unroll
      for (int q = 0; q < KTW; ++q) {
        const int kt = w + NW * q;
        if (kt < KT) {
#pragma unroll
          for (int vt = 0; vt < VT; ++vt) {
            const int v = v0 + 16 * vt + n;
            store_state4<F32>(a.snapshots, ((b * a.n_snap + si) * dv + v) * dk, 16 * kt + 4 * g,
                              dk, v < dv, true, vec_m, st[q][vt]);
          }
        }
      }
    }

    __syncthreads();  // every wave is done with chunk c's LDS
    if (has_next) {
      store_chunk(kst, vst);
#pragma unroll
      for (int kk = 0; kk < NKK; ++kk) qf[kk] = qn[kk];
      store_state_copy();
    }
  }

  if (a.memory_out == nullptr) return;
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

template <class E, int DKP, int DV>
int launch_fwd(const ChunkFwdArgs& a, hipStream_t stream) {
  using S = FwdShape<E, DKP, DV>;
  static bool attr_set = false;
  if (!attr_set) {
    hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(&chunk_fwd_kernel<E, DKP, DV>),
                                       hipFuncAttributeMaxDynamicSharedMemorySize,
                                       static_cast<int>(S::lds_bytes));
    if (e != hipSuccess) {
      set_error("chunk_update_fwd: hipFuncSetAttribute failed: %s", hipGetErrorString(e));
      return static_cast<int>(e);
    }
    attr_set = true;
  }
  const int64_t grid = a.batch * a.v_tiles;
  hipLaunchKernelGGL((chunk_fwd_kernel<E, DKP, DV>), dim3(static_cast<unsigned>(grid)), dim3(NTHR),
                     S::lds_bytes, stream, a);
  return check_launch("chunk_update_fwd");
}

template <class E, int DV>
int dispatch_dk(const ChunkFwdArgs& a, hipStream_t s) {
  if (a.dk <= 32) return launch_fwd<E, 32, DV>(a, s);
  if (a.dk <= 64) return launch_fwd<E, 64, DV>(a, s);
  if (a.dk <= 128) return launch_fwd<E, 128, DV>(a, s);
  return launch_fwd<E, 256, DV>(a, s);
}

template <class E>
int dispatch_dv(const ChunkFwdArgs& a, int dv_tile, hipStream_t s) {
  return dv_tile == 32 ? dispatch_dk<E, 32>(a, s) : dispatch_dk<E, 16>(a, s);
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

}  // namespace

int tile_dv_for(int64_t batch, int64_t value_dim) {
  const char* env = getenv("GRM_HIP_CHUNK_DV");
  if (env != nullptr) {
    const int v = atoi(env);
    if (v == 16 || v == 32) return v;
  }
  // Prefer the wider tile only when it still gives every CU a workgroup.
  return (batch * ((value_dim + 31) / 32) >= 512) ? 32 : 16;
}

}  // namespace grmhip

using namespace grmhip;

extern "C" int grm_hip_chunk_update_fwd(const void* keys, const void* values, const void* queries,
                                        const void* memory, void* hidden, void* memory_out,
                                        float* snapshots, int64_t batch, int64_t seq_len,
                                        int64_t key_dim, int64_t value_dim, int in_dtype,
                                        int mem_dtype, double memory_decay, int64_t snapshot_len,
                                        void* stream) {
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
  if (key_dim > 256) {
    set_error("chunk_update_fwd: key_dim %lld > 256", (long long)key_dim);
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
  a.chunk = snapshots != nullptr ? chunk_for_snapshot(snapshot_len) : CT;
  const int64_t n_chunks = (seq_len + a.chunk - 1) / a.chunk;
  if (n_chunks > INT32_MAX) {
    set_error("chunk_update_fwd: seq_len too large");
    return GRM_HIP_EINVAL;
  }
  a.n_chunks = static_cast<int>(n_chunks);
  if (snapshots != nullptr) {
    a.snap_every = static_cast<int>(snapshot_len / a.chunk);
    a.n_snap = static_cast<int>((seq_len + snapshot_len - 1) / snapshot_len);
  }
  const int dv_tile = tile_dv_for(batch, value_dim);
  a.v_tiles = static_cast<int>((value_dim + dv_tile - 1) / dv_tile);
  const int64_t grid = batch * a.v_tiles;
  if (grid > INT32_MAX) {
    set_error("chunk_update_fwd: batch too large for one launch");
    return GRM_HIP_EINVAL;
  }
  a.mem_f32 = mem_dtype == GRM_HIP_F32;
  a.vec_k = (key_dim % 8 == 0) && aligned(keys, 16) && aligned(queries, 16);
  a.vec_v = (value_dim % 8 == 0) && aligned(values, 16);
  a.vec_o = (value_dim % 4 == 0) && aligned(hidden, 4 * in_b);
  a.vec_m = (key_dim % 4 == 0) && aligned(memory, 4 * mem_b) && aligned(memory_out, 4 * mem_b) &&
            (snapshots == nullptr || aligned(snapshots, 16));
  a.xcd_remap = (grid % 8 == 0) ? 1 : 0;
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
  switch (in_dtype) {
    case GRM_HIP_F32: return dispatch_dv<F32>(a, dv_tile, s);
    case GRM_HIP_F16: return dispatch_dv<F16>(a, dv_tile, s);
    default: return dispatch_dv<BF16>(a, dv_tile, s);
  }
}
