/*
 * grm_oracle.c - CPU restatement of the GRM hot path.  TEST INFRASTRUCTURE ONLY.
 *
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
 * load this; the product path (rnn_with_grm_amd) never does.
 *
 * Float maths runs in double on the caller's inputs (already rounded to the
 * input dtype), so it is the exact map the kernels approximate.  The routing
 * score is the exception: it is restated in float32 with one fused
 * multiply-add chain per score in d order, the canonical score that makes
 * top-k indices comparable bit for bit.
 *
 * Layouts: keys/queries [B, T, K], values/hidden [B, T, H], memory [B, H, K]
 * (row = value index), all row-major.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

/* Per-token recurrence (reference grm/csrc/grm_cuda.cpp:71-83 and the CUDA
 * kernel grm/csrc/chunk_update.cu:82-123):
 *   M <- decay M + (1 - decay) / sqrt(K) v_t k_t^T ;  h_t = M q_t
 * snapshots (may be NULL): state after every snapshot_len tokens and at the end,
 * [B, ceil(T / snapshot_len), H, K]. */
void grm_oracle_chunk_update_seq(const double* keys, const double* values, const double* queries,
                                 const double* memory, double decay, int64_t B, int64_t T,
                                 int64_t K, int64_t H, double* hidden, double* memory_out,
                                 double* snapshots, int64_t snapshot_len) {
  const double inv_scale = 1.0 / sqrt((double)K);
  const double beta = 1.0 - decay;
  const int64_t n_snap = (snapshots && snapshot_len > 0) ? (T + snapshot_len - 1) / snapshot_len : 0;
  double* m = (double*)malloc(sizeof(double) * (size_t)(H * K));
  for (int64_t b = 0; b < B; ++b) {
    memcpy(m, memory + b * H * K, sizeof(double) * (size_t)(H * K));
    for (int64_t t = 0; t < T; ++t) {
      const double* kt = keys + (b * T + t) * K;
      const double* qt = queries + (b * T + t) * K;
      const double* vt = values + (b * T + t) * H;
      for (int64_t h = 0; h < H; ++h) {
        double acc = 0.0;
        for (int64_t k = 0; k < K; ++k) {
          const double u = vt[h] * kt[k] * inv_scale;
          m[h * K + k] = m[h * K + k] * decay + u * beta;
          acc += m[h * K + k] * qt[k];
        }
        hidden[(b * T + t) * H + h] = acc;
      }
      if (n_snap > 0 && ((t + 1) % snapshot_len == 0 || t + 1 == T)) {
        const int64_t si = t / snapshot_len;
        memcpy(snapshots + (b * n_snap + si) * H * K, m, sizeof(double) * (size_t)(H * K));
      }
    }
    memcpy(memory_out + b * H * K, m, sizeof(double) * (size_t)(H * K));
  }
  free(m);
}

/* Chunked closed form (reference grm/core/cuda_ops.py:218-254), applied to
 * consecutive chunks of `chunk` tokens with the state carried:
 *   h_i = decay^{i+1} M q_i + beta * sum_{j<=i} decay^{i-j} (q_i.k_j / sqrt K) v_j
 *   M'  = decay^L M + sum_j beta decay^{L-1-j} / sqrt K  v_j k_j^T            */
void grm_oracle_chunk_update_chunked(const double* keys, const double* values,
                                     const double* queries, const double* memory, double decay,
                                     int64_t B, int64_t T, int64_t K, int64_t H, int64_t chunk,
                                     double* hidden, double* memory_out) {
  const double sq = sqrt((double)K);
  const double beta = 1.0 - decay;
  double* m = (double*)malloc(sizeof(double) * (size_t)(H * K));
  double* dm = (double*)malloc(sizeof(double) * (size_t)(H * K));
  for (int64_t b = 0; b < B; ++b) {
    memcpy(m, memory + b * H * K, sizeof(double) * (size_t)(H * K));
    for (int64_t t0 = 0; t0 < T; t0 += chunk) {
      const int64_t L = (T - t0 < chunk) ? (T - t0) : chunk;
      for (int64_t i = 0; i < L; ++i) {
        const double* qi = queries + (b * T + t0 + i) * K;
        double* hi = hidden + (b * T + t0 + i) * H;
        const double start = pow(decay, (double)(i + 1));
        for (int64_t h = 0; h < H; ++h) {
          double acc = 0.0;
          for (int64_t k = 0; k < K; ++k) acc += m[h * K + k] * qi[k];
          hi[h] = start * acc;
        }
        for (int64_t j = 0; j <= i; ++j) {
          const double* kj = keys + (b * T + t0 + j) * K;
          const double* vj = values + (b * T + t0 + j) * H;
          double s = 0.0;
          for (int64_t k = 0; k < K; ++k) s += qi[k] * kj[k];
          const double wgt = beta * (s / sq) * pow(decay, (double)(i - j));
          for (int64_t h = 0; h < H; ++h) hi[h] += wgt * vj[h];
        }
      }
      memset(dm, 0, sizeof(double) * (size_t)(H * K));
      for (int64_t j = 0; j < L; ++j) {
        const double* kj = keys + (b * T + t0 + j) * K;
        const double* vj = values + (b * T + t0 + j) * H;
        const double wgt = beta * pow(decay, (double)(L - 1 - j)) / sq;
        for (int64_t h = 0; h < H; ++h)
          for (int64_t k = 0; k < K; ++k) dm[h * K + k] += wgt * vj[h] * kj[k];
      }
      const double dl = pow(decay, (double)L);
      for (int64_t e = 0; e < H * K; ++e) m[e] = dl * m[e] + dm[e];
    }
    memcpy(memory_out + b * H * K, m, sizeof(double) * (size_t)(H * K));
  }
  free(m);
  free(dm);
}

/* Gradient of the recurrence by reverse-mode differentiation of the
 * per-token loop above (the reference differentiates its forward with
 * autograd, grm/csrc/grm_cuda.cpp:92-126).  Keeps every per-token state. */
void grm_oracle_chunk_update_bwd(const double* grad_hidden, const double* grad_memory_out,
                                 const double* keys, const double* values, const double* queries,
                                 const double* memory, double decay, int64_t B, int64_t T,
                                 int64_t K, int64_t H, double* gk, double* gv, double* gq,
                                 double* gm) {
  const double c = (1.0 - decay) / sqrt((double)K);
  const size_t HK = (size_t)(H * K);
  double* states = (double*)malloc(sizeof(double) * HK * (size_t)(T + 1));
  double* G = (double*)malloc(sizeof(double) * HK);
  for (int64_t b = 0; b < B; ++b) {
    /* forward, keeping M_{-1} .. M_{T-1} */
    memcpy(states, memory + b * HK, sizeof(double) * HK);
    for (int64_t t = 0; t < T; ++t) {
      const double* kt = keys + (b * T + t) * K;
      const double* vt = values + (b * T + t) * H;
      const double* prev = states + (size_t)t * HK;
      double* cur = states + (size_t)(t + 1) * HK;
      for (int64_t h = 0; h < H; ++h)
        for (int64_t k = 0; k < K; ++k) cur[h * K + k] = decay * prev[h * K + k] + c * vt[h] * kt[k];
    }
    memcpy(G, grad_memory_out + b * HK, sizeof(double) * HK);
    for (int64_t t = T - 1; t >= 0; --t) {
      const double* kt = keys + (b * T + t) * K;
      const double* qt = queries + (b * T + t) * K;
      const double* vt = values + (b * T + t) * H;
      const double* dh = grad_hidden + (b * T + t) * H;
      const double* cur = states + (size_t)(t + 1) * HK;
      /* h_t = M_t q_t */
      for (int64_t k = 0; k < K; ++k) {
        double acc = 0.0;
        for (int64_t h = 0; h < H; ++h) acc += dh[h] * cur[h * K + k];
        gq[(b * T + t) * K + k] = acc;
      }
      for (int64_t h = 0; h < H; ++h)
        for (int64_t k = 0; k < K; ++k) G[h * K + k] += dh[h] * qt[k];
      /* M_t = decay M_{t-1} + c v k^T */
      for (int64_t h = 0; h < H; ++h) {
        double acc = 0.0;
        for (int64_t k = 0; k < K; ++k) acc += G[h * K + k] * kt[k];
        gv[(b * T + t) * H + h] = c * acc;
      }
      for (int64_t k = 0; k < K; ++k) {
        double acc = 0.0;
        for (int64_t h = 0; h < H; ++h) acc += G[h * K + k] * vt[h];
        gk[(b * T + t) * K + k] = c * acc;
      }
      for (size_t e = 0; e < HK; ++e) G[e] *= decay;
    }
    memcpy(gm + b * HK, G, sizeof(double) * HK);
  }
  free(states);
  free(G);
}

/* hidden[n, r, h] = sum_k mem[n, r, h, k] q[n, k] with n = b*Q + q
 * (reference grm/core/cuda_ops.py:257-262, grm/csrc/grm_cuda.cpp:128-134). */
void grm_oracle_apply_query(const double* mem, const double* q, int64_t NQ, int64_t RH, int64_t K,
                            double* out) {
  for (int64_t n = 0; n < NQ; ++n)
    for (int64_t r = 0; r < RH; ++r) {
      double acc = 0.0;
      const double* row = mem + (n * RH + r) * K;
      for (int64_t k = 0; k < K; ++k) acc += row[k] * q[n * K + k];
      out[n * RH + r] = acc;
    }
}

/* Gradient of the above: dM = dh (x) q, dq = sum_r dh_r M_r
 * (reference grm/csrc/grm_cuda.cpp:136-154). */
void grm_oracle_apply_query_bwd(const double* dh, const double* mem, const double* q, int64_t NQ,
                                int64_t RH, int64_t K, double* gmem, double* gq) {
  for (int64_t n = 0; n < NQ; ++n) {
    for (int64_t k = 0; k < K; ++k) gq[n * K + k] = 0.0;
    for (int64_t r = 0; r < RH; ++r) {
      const double d = dh[n * RH + r];
      const double* row = mem + (n * RH + r) * K;
      for (int64_t k = 0; k < K; ++k) {
        gmem[(n * RH + r) * K + k] = d * q[n * K + k];
        gq[n * K + k] += d * row[k];
      }
    }
  }
}

/* out[b, i, :] = mem[b, idx[b, i], :], rows of row_bytes bytes
 * (reference grm/core/cuda_ops.py:265-284, grm/csrc/grm_cuda.cpp:156-179).
 * Returns the number of indices outside [0, S) (those rows are left zero). */
int64_t grm_oracle_gather(const uint8_t* mem, const int64_t* idx, uint8_t* out, int64_t B,
                          int64_t S, int64_t n_index, int64_t row_bytes) {
  int64_t bad = 0;
  for (int64_t b = 0; b < B; ++b)
    for (int64_t i = 0; i < n_index; ++i) {
      const int64_t s = idx[b * n_index + i];
      uint8_t* dst = out + (b * n_index + i) * row_bytes;
      if (s < 0 || s >= S) {
        memset(dst, 0, (size_t)row_bytes);
        ++bad;
        continue;
      }
      memcpy(dst, mem + (b * S + s) * row_bytes, (size_t)row_bytes);
    }
  return bad;
}

/* Routing (reference grm/core/paper_grm.py:566-589, grm/core/gating_unit.py:54-91).
 * score = scale * (float32 FMA chain over d = 0..D-1); k = min(top_k, S);
 * k < S: best k, descending, ties to the lower index; k == S: index order.
 * gates = softmax(score / temperature) in double. */
void grm_oracle_topk_route(const float* q, const float* keys, int64_t B, int64_t Q, int64_t S,
                           int64_t D, int64_t top_k, float scale, double temperature,
                           int64_t* idx, float* scores, double* gates) {
  const int64_t k = top_k < S ? top_k : S;
  float* all = (float*)malloc(sizeof(float) * (size_t)(S > 0 ? S : 1));
  int64_t* order = (int64_t*)malloc(sizeof(int64_t) * (size_t)(S > 0 ? S : 1));
  for (int64_t b = 0; b < B; ++b)
    for (int64_t qi = 0; qi < Q; ++qi) {
      const float* qr = q + (b * Q + qi) * D;
      for (int64_t s = 0; s < S; ++s) {
        const float* kr = keys + (b * S + s) * D;
        float acc = 0.0f;
        for (int64_t d = 0; d < D; ++d) acc = fmaf(qr[d], kr[d], acc);
        all[s] = acc * scale;
        order[s] = s;
      }
      if (k < S) {
        /* selection of the k best by (score desc, index asc) */
        for (int64_t m = 0; m < k; ++m) {
          int64_t best = m;
          for (int64_t j = m + 1; j < S; ++j) {
            const float a = all[order[j]], c = all[order[best]];
            if (a > c || (a == c && order[j] < order[best])) best = j;
          }
          const int64_t tmp = order[m];
          order[m] = order[best];
          order[best] = tmp;
        }
      }
      double mx = -INFINITY;
      for (int64_t m = 0; m < k; ++m) {
        const double v = (double)all[order[m]] / temperature;
        if (v > mx) mx = v;
      }
      double sum = 0.0;
      for (int64_t m = 0; m < k; ++m) sum += exp((double)all[order[m]] / temperature - mx);
      const int64_t o = (b * Q + qi) * k;
      for (int64_t m = 0; m < k; ++m) {
        idx[o + m] = order[m];
        scores[o + m] = all[order[m]];
        gates[o + m] = exp((double)all[order[m]] / temperature - mx) / sum;
      }
    }
  free(all);
  free(order);
}

/* Residual fusion (reference grm/core/aggregator.py:67-145, residual mode):
 * x = h + sum_r g_r ret_r ; out = LayerNorm(x) * w + b (biased variance);
 * w == NULL: out = x. */
void grm_oracle_fuse_residual(const double* h, const double* ret, const double* gates,
                              const double* w, const double* bias, int64_t N, int64_t R,
                              int64_t H, double eps, double* out) {
  for (int64_t n = 0; n < N; ++n) {
    double* o = out + n * H;
    for (int64_t c = 0; c < H; ++c) {
      double x = h[n * H + c];
      for (int64_t r = 0; r < R; ++r) x += gates[n * R + r] * ret[(n * R + r) * H + c];
      o[c] = x;
    }
    if (w == NULL) continue;
    double mean = 0.0;
    for (int64_t c = 0; c < H; ++c) mean += o[c];
    mean /= (double)H;
    double var = 0.0;
    for (int64_t c = 0; c < H; ++c) var += (o[c] - mean) * (o[c] - mean);
    var /= (double)H;
    const double rstd = 1.0 / sqrt(var + eps);
    for (int64_t c = 0; c < H; ++c) o[c] = (o[c] - mean) * rstd * w[c] + (bias ? bias[c] : 0.0);
  }
}
