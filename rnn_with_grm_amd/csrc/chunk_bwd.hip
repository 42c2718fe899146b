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
    const int L = static_cast<int>(min(static_cast<int64_t>(BCT), T - t0));
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

}  // namespace
}  // namespace grmhip

using namespace grmhip;

extern "C" int grm_hip_chunk_update_bwd(const void* grad_hidden, const void* grad_memory_out,
                                        const void* keys, const void* values, const void* queries,
                                        const void* memory, void* grad_keys, void* grad_values,
                                        void* grad_queries, void* grad_memory, float* chunk_states,
                                        float* dkq_partial, int64_t batch, int64_t seq_len,
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
  // Re-run the forward to store the state after every 64-token chunk; its
  // hidden output and final state are not needed.
  int rc = grm_hip_chunk_update_fwd(keys, values, queries, memory, nullptr, nullptr, chunk_states,
                                    nullptr, 0, batch, seq_len, key_dim, value_dim, in_dtype,
                                    mem_dtype, memory_decay, BCT, stream);
  if (rc != GRM_HIP_OK) return rc;

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
