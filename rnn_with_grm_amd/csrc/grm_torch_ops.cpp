// torch.ops.grm_cuda registration for the MI355X library (module grm_cuda_ext).
//
// The five schemas are the reference's, character for character
// (reference grm/csrc/bindings.cpp:5-11), so grm.core.cuda_ops and every model
// above it bind to this library unchanged.  Fifteen more ops live in the same
// namespace: segment_scan_forward (whole-sequence update with per-segment
// state snapshots), topk_route (score -> top-k -> softmax), segment_route (the
// same routing for every segment of a sequence against the archive as it
// grows), fuse_residual, gather_apply (gather + query application without
// materialising the states), retrieve_fuse (gather_apply, the gate-weighted
// sum and fuse_residual in one call), segment_retrieve_fuse (the same for the
// windows of segment routing, summing the routes without per-route rows), the
// layer glue project_split (the
// projection's split with L2-normalised keys and queries),
// residual_layer_norm (the block's LayerNorm(out + x)), project_gemm (the
// projection GEMM with project_split as its epilogue),
// linear_residual_layer_norm (the output projection GEMM with the block's
// residual add and LayerNorm as its epilogue) and archive_cast (the
// archive's stored form of float32 states), and three gradients
// without gathered states: apply_query_backward_queries,
// gather_apply_backward_queries (one gradient row per pair) and
// gather_apply_backward_tokens (one row per query, shared by its routes).
//
// CUDA-key kernels (HIP devices dispatch on the CUDA key in PyTorch-ROCm)
// check the inputs, allocate outputs with ATen on the input's device and call
// the C ABI of libgrm_hip.so on the current stream.  Like the reference
// (chunk_update.cu:529-531, apply_query.cu:187-189, batched_gather.cu:92-94),
// inputs the kernels do not cover (e.g. float64) run the generic ATen
// implementation on the same device; grm_hip_launch_count() shows which path
// ran.  CPU-key kernels are the generic ATen implementations.
#include <torch/extension.h>

#include <c10/core/DeviceGuard.h>
#include <c10/hip/HIPStream.h>

#include <atomic>
#include <cmath>
#include <cstdlib>
#include <tuple>
#include <vector>

#include "grm_hip.h"

namespace grm {
namespace {

using at::Tensor;

std::atomic<int64_t> g_generic_calls{0};

int dtype_code(at::ScalarType t) {
  switch (t) {
    case at::kFloat: return GRM_HIP_F32;
    case at::kHalf: return GRM_HIP_F16;
    case at::kBFloat16: return GRM_HIP_BF16;
    default: return -1;
  }
}

void check_rc(int rc, const char* op) {
  TORCH_CHECK(rc == GRM_HIP_OK, op, " failed (", rc, "): ", grm_hip_last_error());
}

void* current_stream(const Tensor& t) {
  return static_cast<void*>(c10::hip::getCurrentHIPStream(t.device().index()).stream());
}

// Scratch for the time-split scan (per-part end states), allocated on the
// tensor's device through the caching allocator.
Tensor scan_workspace(const Tensor& like, int64_t B, int64_t T, int64_t K, int64_t H, int64_t snap) {
  const int64_t bytes = grm_hip_chunk_update_fwd_workspace(B, T, K, H, snap);
  return at::empty({(bytes + 3) / 4}, like.options().dtype(at::kFloat));
}

// ---------------------------------------------------------------------------
// Argument checks (same conditions and error class as the reference,
// grm/csrc/grm_cuda.cpp:13-42,159-161).
void check_chunk_inputs(const Tensor& keys, const Tensor& values, const Tensor& queries,
                        const Tensor& memory) {
  TORCH_CHECK(keys.dim() == 3, "keys must have shape [B, T, K]");
  TORCH_CHECK(values.dim() == 3, "values must have shape [B, T, H]");
  TORCH_CHECK(queries.dim() == 3, "queries must have shape [B, T, K]");
  TORCH_CHECK(memory.dim() == 3, "memory must have shape [B, H, K]");
  TORCH_CHECK(keys.size(0) == values.size(0) && keys.size(1) == values.size(1),
              "keys and values batch/time dims must match");
  TORCH_CHECK(keys.sizes() == queries.sizes(), "keys and queries must have the same shape");
  TORCH_CHECK(values.size(0) == memory.size(0), "memory batch dim must match values batch dim");
  TORCH_CHECK(values.size(2) == memory.size(1), "memory hidden dim must match values hidden dim");
  TORCH_CHECK(keys.size(2) == memory.size(2), "memory key dim must match keys key dim");
}

void check_apply_inputs(const Tensor& memories, const Tensor& queries) {
  TORCH_CHECK(memories.dim() == 4 || memories.dim() == 5,
              "memories must have shape [B, R, H, K] or [B, Q, R, H, K]");
  if (memories.dim() == 4) {
    TORCH_CHECK(queries.dim() == 2, "queries must have shape [B, K] when memories rank is 4");
    TORCH_CHECK(memories.size(0) == queries.size(0), "batch dim mismatch between memories and queries");
    TORCH_CHECK(memories.size(3) == queries.size(1), "key dim mismatch between memories and queries");
    return;
  }
  TORCH_CHECK(queries.dim() == 3, "queries must have shape [B, Q, K] when memories rank is 5");
  TORCH_CHECK(memories.size(0) == queries.size(0), "batch dim mismatch between memories and queries");
  TORCH_CHECK(memories.size(1) == queries.size(1), "query dim mismatch between memories and queries");
  TORCH_CHECK(memories.size(4) == queries.size(2), "key dim mismatch between memories and queries");
}

void check_gather_inputs(const Tensor& memories, const Tensor& indices) {
  TORCH_CHECK(memories.dim() == 4, "memories_per_batch must have shape [B, S, H, K]");
  TORCH_CHECK(indices.dim() == 2 || indices.dim() == 3,
              "topk_indices must have shape [B, R] or [B, Q, R]");
  TORCH_CHECK(memories.size(0) == indices.size(0),
              "batch dim mismatch between memories_per_batch and topk_indices");
}

// ---------------------------------------------------------------------------
// Generic ATen implementations (CPU key, and CUDA inputs outside the kernels).

// Chunked closed form, 64 tokens at a time, computed in float32 (float64 for
// float64 inputs).
std::tuple<Tensor, Tensor, std::vector<Tensor>> chunk_math(const Tensor& keys, const Tensor& values,
                                                           const Tensor& queries,
                                                           const Tensor& memory, double decay,
                                                           int64_t snapshot_len) {
  const auto cdt = keys.scalar_type() == at::kDouble ? at::kDouble : at::kFloat;
  const auto opts = keys.options().dtype(cdt);
  Tensor k = keys.to(cdt), v = values.to(cdt), q = queries.to(cdt);
  Tensor m = memory.to(cdt);
  const int64_t T = keys.size(1);
  const double c = (1.0 - decay) / std::sqrt(static_cast<double>(keys.size(2)));
  const Tensor base = at::scalar_tensor(decay, opts);
  const int64_t step = snapshot_len > 0 ? std::min<int64_t>(snapshot_len, 64) : 64;
  std::vector<Tensor> outs, snaps;
  int64_t since_snap = 0;
  int64_t t0 = 0;
  while (t0 < T) {
    int64_t L = std::min(step, T - t0);
    if (snapshot_len > 0) L = std::min(L, snapshot_len - since_snap);
    Tensor kc = k.narrow(1, t0, L), vc = v.narrow(1, t0, L), qc = q.narrow(1, t0, L);
    Tensor pos = at::arange(L, opts);
    Tensor rel = pos.unsqueeze(1) - pos.unsqueeze(0);
    Tensor dmask = at::where(rel >= 0, at::pow(base, rel.clamp_min(0)), at::zeros_like(rel));
    Tensor s = at::bmm(qc, kc.transpose(1, 2)) * (dmask * c).unsqueeze(0);
    Tensor h = at::bmm(qc, m.transpose(1, 2)) * at::pow(base, pos + 1).view({1, L, 1}) +
               at::bmm(s, vc);
    outs.push_back(h);
    Tensor w = at::pow(base, (L - 1) - pos) * c;
    m = at::pow(base, static_cast<double>(L)) * m +
        at::bmm((vc * w.view({1, L, 1})).transpose(1, 2), kc);
    since_snap += L;
    t0 += L;
    if (snapshot_len > 0 && (since_snap == snapshot_len || t0 == T)) {
      snaps.push_back(m);
      since_snap = 0;
    }
  }
  Tensor hidden = outs.empty() ? at::zeros({keys.size(0), 0, values.size(2)}, opts) : at::cat(outs, 1);
  return {hidden, m, snaps};
}

std::tuple<Tensor, Tensor, Tensor> chunk_update_forward_generic(const Tensor& keys,
                                                                const Tensor& values,
                                                                const Tensor& queries,
                                                                const Tensor& memory,
                                                                double decay) {
  check_chunk_inputs(keys, values, queries, memory);
  if (keys.size(1) == 0) {
    return {at::zeros({keys.size(0), 0, values.size(2)}, values.options()), memory.contiguous(),
            at::empty({0}, memory.options())};
  }
  auto res = chunk_math(keys, values, queries, memory, decay, 0);
  return {std::get<0>(res).to(values.scalar_type()).contiguous(),
          std::get<1>(res).to(memory.scalar_type()).contiguous(), at::empty({0}, memory.options())};
}

std::tuple<Tensor, Tensor, Tensor, Tensor> chunk_update_backward_generic(
    const Tensor& grad_hidden, const Tensor& grad_memory_out, const Tensor& keys,
    const Tensor& values, const Tensor& queries, const Tensor& memory, double decay) {
  at::AutoGradMode grad_on(true);
  Tensor k = keys.detach().clone().requires_grad_(true);
  Tensor v = values.detach().clone().requires_grad_(true);
  Tensor q = queries.detach().clone().requires_grad_(true);
  Tensor m = memory.detach().clone().requires_grad_(true);
  auto out = chunk_update_forward_generic(k, v, q, m, decay);
  auto grads = torch::autograd::grad({std::get<0>(out), std::get<1>(out)}, {k, v, q, m},
                                     {grad_hidden.to(values.scalar_type()).contiguous(),
                                      grad_memory_out.to(memory.scalar_type()).contiguous()},
                                     false, false, /*allow_unused=*/true);
  auto fix = [](const Tensor& g, const Tensor& like) {
    return g.defined() ? g.contiguous() : at::zeros_like(like);
  };
  return {fix(grads[0], keys), fix(grads[1], values), fix(grads[2], queries), fix(grads[3], memory)};
}

Tensor apply_query_forward_generic(const Tensor& memories, const Tensor& queries) {
  check_apply_inputs(memories, queries);
  if (memories.dim() == 5) return at::einsum("bqrhk,bqk->bqrh", {memories, queries}).contiguous();
  return at::einsum("brhk,bk->brh", {memories, queries}).contiguous();
}

std::tuple<Tensor, Tensor> apply_query_backward_generic(const Tensor& grad_hidden,
                                                        const Tensor& memories,
                                                        const Tensor& queries) {
  check_apply_inputs(memories, queries);
  Tensor dh = grad_hidden.to(memories.scalar_type());
  if (memories.dim() == 5) {
    Tensor gm = (dh.unsqueeze(-1) * queries.unsqueeze(2).unsqueeze(2)).contiguous();
    Tensor gq = at::einsum("bqrh,bqrhk->bqk", {dh, memories}).contiguous();
    return {gm, gq};
  }
  Tensor gm = (dh.unsqueeze(-1) * queries.unsqueeze(1).unsqueeze(1)).contiguous();
  Tensor gq = at::einsum("brh,brhk->bk", {dh, memories}).contiguous();
  return {gm, gq};
}

Tensor batched_memory_gather_generic(const Tensor& memories, const Tensor& indices) {
  check_gather_inputs(memories, indices);
  const int64_t B = memories.size(0);
  Tensor idx = indices.to(at::kLong).reshape({B, -1});
  std::vector<int64_t> shape{B};
  for (int64_t d = 1; d < indices.dim(); ++d) shape.push_back(indices.size(d));
  shape.push_back(memories.size(2));
  shape.push_back(memories.size(3));
  std::vector<Tensor> rows;
  rows.reserve(B);
  for (int64_t b = 0; b < B; ++b) rows.push_back(memories[b].index_select(0, idx[b]));
  if (B == 0) return at::empty(shape, memories.options());
  return at::stack(rows, 0).reshape(shape).contiguous();
}

// gather_apply: the reference's composition apply_query_forward(
// batched_memory_gather(memories, indices), queries.to(memories.dtype))
// (grm/core/cuda_ops.py:370-402, paper_grm.py:229,301-313) in one op.  With
// dtype=float32 the gathered 16-bit states are widened first, as the
// retriever's .to(torch.float32) of the fp16 archive (paper_grm.py:227).
void check_gather_apply_inputs(const Tensor& memories, const Tensor& indices, const Tensor& queries) {
  check_gather_inputs(memories, indices);
  TORCH_CHECK(queries.dim() == indices.dim(),
              "gather_apply: queries must be [B, K] with indices [B, R], or [B, Q, K] with indices [B, Q, R]");
  TORCH_CHECK(queries.size(0) == memories.size(0), "gather_apply: batch dim mismatch");
  TORCH_CHECK(queries.size(-1) == memories.size(3), "gather_apply: key dim mismatch");
  if (indices.dim() == 3) TORCH_CHECK(queries.size(1) == indices.size(1), "gather_apply: query dim mismatch");
}

at::ScalarType gather_apply_dtype(const Tensor& memories, std::optional<at::ScalarType> dtype) {
  const at::ScalarType t = dtype.value_or(memories.scalar_type());
  TORCH_CHECK(t == memories.scalar_type() || t == at::kFloat,
              "gather_apply: dtype must be the memories' dtype or float32");
  return t;
}

Tensor gather_apply_generic(const Tensor& memories, const Tensor& indices, const Tensor& queries,
                            std::optional<at::ScalarType> dtype) {
  check_gather_apply_inputs(memories, indices, queries);
  const at::ScalarType t = gather_apply_dtype(memories, dtype);
  return apply_query_forward_generic(batched_memory_gather_generic(memories, indices).to(t), queries.to(t));
}

// Canonical routing on the host: one float32 FMA chain per score, ties to the
// lower index; softmax in float32.
std::tuple<Tensor, Tensor, Tensor> topk_route_cpu(const Tensor& queries, const Tensor& keys,
                                                  int64_t top_k, double scale, double temperature) {
  TORCH_CHECK(queries.dim() == 3 && keys.dim() == 3, "topk_route: queries [B, Q, D], keys [B, S, D]");
  TORCH_CHECK(queries.size(0) == keys.size(0) && queries.size(2) == keys.size(2),
              "topk_route: batch/dim mismatch");
  TORCH_CHECK(top_k >= 1, "topk_route: top_k must be >= 1");
  TORCH_CHECK(temperature > 0, "topk_route: temperature must be > 0");
  const int64_t B = queries.size(0), Q = queries.size(1), S = keys.size(1), D = queries.size(2);
  const int64_t k = std::min(top_k, S);
  Tensor qf = queries.to(at::kFloat).contiguous(), kf = keys.to(at::kFloat).contiguous();
  auto fopt = queries.options().dtype(at::kFloat);
  Tensor idx = at::empty({B, Q, k}, queries.options().dtype(at::kLong));
  Tensor sc = at::empty({B, Q, k}, fopt), gt = at::empty({B, Q, k}, fopt);
  const float* qp = qf.data_ptr<float>();
  const float* kp = kf.data_ptr<float>();
  int64_t* ip = idx.data_ptr<int64_t>();
  float* sp = sc.data_ptr<float>();
  float* gp = gt.data_ptr<float>();
  const float fs = static_cast<float>(scale), inv_t = 1.0f / static_cast<float>(temperature);
  at::parallel_for(0, B * Q, 1, [&](int64_t lo, int64_t hi) {
    std::vector<float> all(S);
    std::vector<int64_t> order(S);
    for (int64_t r = lo; r < hi; ++r) {
      const int64_t b = r / Q;
      const float* qr = qp + r * D;
      for (int64_t s = 0; s < S; ++s) {
        const float* kr = kp + (b * S + s) * D;
        float acc = 0.f;
        for (int64_t d = 0; d < D; ++d) acc = std::fma(qr[d], kr[d], acc);
        all[s] = acc * fs;
        order[s] = s;
      }
      // k < S: a NaN or -inf score is never selected (NaN sorts as -inf; slots left
      // at -inf are empty, (-1, -inf, 0)).  k >= S: every key in index order.
      const bool select = k < S;
      if (select) {
        for (int64_t s = 0; s < S; ++s) all[s] = std::isnan(all[s]) ? -INFINITY : all[s];
        std::stable_sort(order.begin(), order.end(),
                         [&](int64_t x, int64_t y) { return all[x] > all[y]; });
      }
      auto filled = [&](int64_t m) { return !select || all[order[m]] > -INFINITY; };
      float mx = -INFINITY;
      for (int64_t m = 0; m < k; ++m) mx = filled(m) ? std::max(mx, all[order[m]] * inv_t) : mx;
      float sum = 0.f;
      for (int64_t m = 0; m < k; ++m) sum += filled(m) ? std::exp(all[order[m]] * inv_t - mx) : 0.f;
      for (int64_t m = 0; m < k; ++m) {
        const bool f = filled(m);
        ip[r * k + m] = f ? order[m] : -1;
        sp[r * k + m] = f ? all[order[m]] : -INFINITY;
        gp[r * k + m] = f ? std::exp(all[order[m]] * inv_t - mx) / sum : 0.f;
      }
    }
  });
  return {gt, idx, sc};
}

// Segment routing over the archive as it grows (grm_hip_segment_route): row t
// of segment s = t / segment_len is routed over keys [lo, hi), hi = base + s,
// lo = max(0, hi - capacity), with topk_route's rule inside the window.
void check_segment_route(const Tensor& queries, const Tensor& keys, int64_t top_k, int64_t segment_len,
                         int64_t base, int64_t capacity, double temperature) {
  TORCH_CHECK(queries.dim() == 3 && keys.dim() == 3, "segment_route: queries [B, Q, D], keys [B, S, D]");
  TORCH_CHECK(queries.size(0) == keys.size(0) && queries.size(2) == keys.size(2),
              "segment_route: batch/dim mismatch");
  TORCH_CHECK(top_k >= 1 && top_k <= 128, "segment_route: top_k must be in [1, 128]");
  TORCH_CHECK(segment_len >= 1 && base >= 0 && capacity >= 1,
              "segment_route: segment_len >= 1, base >= 0 and capacity >= 1 required");
  TORCH_CHECK(temperature > 0, "segment_route: temperature must be > 0");
  TORCH_CHECK(queries.size(1) == 0 || base + (queries.size(1) - 1) / segment_len <= keys.size(1),
              "segment_route: the last segment's window ends past the keys");
}

std::tuple<Tensor, Tensor, Tensor> segment_route_cpu(const Tensor& queries, const Tensor& keys, int64_t top_k,
                                                     int64_t segment_len, int64_t base, int64_t capacity,
                                                     double scale, double temperature) {
  check_segment_route(queries, keys, top_k, segment_len, base, capacity, temperature);
  const int64_t B = queries.size(0), Q = queries.size(1), S = keys.size(1), D = queries.size(2);
  const int64_t k = top_k;
  Tensor qf = queries.to(at::kFloat).contiguous(), kf = keys.to(at::kFloat).contiguous();
  auto fopt = queries.options().dtype(at::kFloat);
  Tensor idx = at::empty({B, Q, k}, queries.options().dtype(at::kLong));
  Tensor sc = at::empty({B, Q, k}, fopt), gt = at::empty({B, Q, k}, fopt);
  const float* qp = qf.data_ptr<float>();
  const float* kp = kf.data_ptr<float>();
  int64_t* ip = idx.data_ptr<int64_t>();
  float* sp = sc.data_ptr<float>();
  float* gp = gt.data_ptr<float>();
  const float fs = static_cast<float>(scale), inv_t = 1.0f / static_cast<float>(temperature);
  at::parallel_for(0, B * Q, 1, [&](int64_t r0, int64_t r1) {
    std::vector<float> all;
    std::vector<int64_t> order;
    for (int64_t r = r0; r < r1; ++r) {
      const int64_t b = r / Q, t = r % Q;
      const int64_t hi = std::min(S, base + t / segment_len);
      const int64_t lo = std::max<int64_t>(0, hi - capacity);
      const int64_t n = hi - lo;
      all.assign(n, 0.f);
      order.resize(n);
      const float* qr = qp + r * D;
      for (int64_t j = 0; j < n; ++j) {
        const float* kr = kp + (b * S + lo + j) * D;
        float acc = 0.f;
        for (int64_t d = 0; d < D; ++d) acc = std::fma(qr[d], kr[d], acc);
        all[j] = acc * fs;
        order[j] = j;
      }
      const int64_t kk = std::min(k, n);
      if (kk < n) {
        std::stable_sort(order.begin(), order.end(), [&](int64_t x, int64_t y) { return all[x] > all[y]; });
      }
      float mx = -INFINITY;
      for (int64_t m = 0; m < kk; ++m) mx = std::max(mx, all[order[m]] * inv_t);
      float sum = 0.f;
      for (int64_t m = 0; m < kk; ++m) sum += std::exp(all[order[m]] * inv_t - mx);
      for (int64_t m = 0; m < k; ++m) {
        const bool filled = m < kk;
        ip[r * k + m] = filled ? lo + order[m] : -1;
        sp[r * k + m] = filled ? all[order[m]] : -INFINITY;
        gp[r * k + m] = filled ? std::exp(all[order[m]] * inv_t - mx) / sum : 0.f;
      }
    }
  });
  return {gt, idx, sc};
}

Tensor fuse_residual_generic(const Tensor& h, const Tensor& retrieved, const Tensor& gates,
                             const c10::optional<Tensor>& weight, const c10::optional<Tensor>& bias,
                             double eps) {
  Tensor x = h.to(at::kFloat);
  if (retrieved.size(1) > 0) {
    x = x + (retrieved.to(at::kFloat) * gates.to(at::kFloat).unsqueeze(-1)).sum(1);
  }
  if (weight.has_value() && weight->defined()) {
    x = at::layer_norm(x, {h.size(-1)}, weight->to(at::kFloat),
                       bias.has_value() && bias->defined() ? bias->to(at::kFloat) : Tensor(), eps);
  }
  return x.to(h.scalar_type()).contiguous();
}

// retrieve_fuse: LN(h + sum_r gates_r (M[idx_r] q)) over [B, Q] rows, the
// retriever's float32 gather + apply followed by the aggregator's residual +
// LayerNorm (paper_grm.py:229,301-313,604-611; aggregator.py:67-145).
void check_retrieve_fuse_inputs(const Tensor& memories, const Tensor& indices, const Tensor& queries,
                                const Tensor& gates, const Tensor& h) {
  TORCH_CHECK(indices.dim() == 3, "retrieve_fuse: indices must be [B, Q, R]");
  check_gather_apply_inputs(memories, indices, queries);
  TORCH_CHECK(gates.sizes() == indices.sizes(), "retrieve_fuse: gates must match indices [B, Q, R]");
  TORCH_CHECK(h.dim() == 3 && h.size(0) == memories.size(0) && h.size(1) == indices.size(1) &&
                  h.size(2) == memories.size(2),
              "retrieve_fuse: h_online must be [B, Q, H]");
}

Tensor retrieve_fuse_generic(const Tensor& memories, const Tensor& indices, const Tensor& queries,
                             const Tensor& gates, const Tensor& h, const c10::optional<Tensor>& weight,
                             const c10::optional<Tensor>& bias, double eps) {
  check_retrieve_fuse_inputs(memories, indices, queries, gates, h);
  const int64_t B = h.size(0), Q = h.size(1), H = h.size(2), R = indices.size(2);
  Tensor r = gather_apply_generic(memories, indices, queries, at::kFloat).reshape({B * Q, R, H});
  // float32 sum and LayerNorm, one rounding to h's dtype at the end
  return fuse_residual_generic(h.reshape({B * Q, H}).to(at::kFloat), r, gates.reshape({B * Q, R}), weight, bias, eps)
      .to(h.scalar_type())
      .reshape({B, Q, H});
}

// segment_retrieve_fuse: retrieve_fuse for the indices of segment routing
// (paper_grm.py:702-728 -> _route_chunk, :566-589): query t sees the archive
// entries [lo(t), hi(t)), hi(t) = base + t / segment_len, lo(t) = max(0, hi(t) -
// capacity).  A negative index is an empty slot; an index outside the query's
// window, or repeating an earlier route of the same query, contributes nothing
// (and is reported when GRM_HIP_CHECK_INDICES is set).
bool check_indices_requested();

void check_segment_window(int64_t segment_len, int64_t base, int64_t capacity) {
  TORCH_CHECK(segment_len >= 1 && base >= 0 && capacity >= 1,
              "segment_retrieve_fuse: needs segment_len >= 1, base >= 0 and capacity >= 1");
}

// [B, Q, R] bool: the pairs that contribute.
Tensor segment_window_valid(const Tensor& indices, int64_t segment_len, int64_t base, int64_t capacity) {
  const int64_t Q = indices.size(1), R = indices.size(2);
  Tensor t = at::arange(Q, indices.options().dtype(at::kLong));
  Tensor hi = (at::floor_divide(t, segment_len) + base).view({1, Q, 1});
  Tensor lo = at::clamp_min(hi - capacity, 0);
  Tensor idx = indices.to(at::kLong);
  Tensor valid = idx.ge(lo).logical_and(idx.lt(hi));
  if (R > 1) {
    Tensor eq = idx.unsqueeze(-1).eq(idx.unsqueeze(-2));  // [B, Q, R, R]: route r against route r2
    Tensor earlier = at::ones({R, R}, indices.options().dtype(at::kBool)).tril(-1);
    valid = valid.logical_and(eq.logical_and(earlier).any(-1).logical_not());
  }
  return valid;
}

void check_window_indices(const Tensor& indices, const Tensor& valid) {
  if (!check_indices_requested()) return;
  const int64_t nbad = indices.ge(0).logical_and(valid.logical_not()).sum().item<int64_t>();
  TORCH_CHECK_INDEX(nbad == 0, "segment_retrieve_fuse: ", nbad,
                    " index values outside their query's window or repeated");
}

Tensor segment_retrieve_fuse_generic(const Tensor& memories, const Tensor& indices, const Tensor& queries,
                                     const Tensor& gates, const Tensor& h, const c10::optional<Tensor>& weight,
                                     const c10::optional<Tensor>& bias, double eps, int64_t segment_len, int64_t base,
                                     int64_t capacity) {
  check_retrieve_fuse_inputs(memories, indices, queries, gates, h);
  check_segment_window(segment_len, base, capacity);
  const int64_t B = h.size(0), Q = h.size(1), H = h.size(2), R = indices.size(2), S = memories.size(1);
  TORCH_CHECK(Q == 0 || base + (Q - 1) / segment_len <= S,
              "segment_retrieve_fuse: windows past the archive (base + (Q - 1) / segment_len > segments)");
  Tensor valid = segment_window_valid(indices, segment_len, base, capacity);
  check_window_indices(indices, valid);
  Tensor r;
  if (S == 0 || R == 0) {
    r = at::zeros({B * Q, R, H}, h.options().dtype(at::kFloat));
  } else {
    Tensor idx = indices.to(at::kLong).masked_fill(valid.logical_not(), 0);
    r = gather_apply_generic(memories, idx, queries, at::kFloat).reshape({B * Q, R, H});
    r = r.masked_fill(valid.logical_not().reshape({B * Q, R, 1}), 0.0);
  }
  Tensor g = gates.to(at::kFloat).masked_fill(valid.logical_not(), 0.0).reshape({B * Q, R});
  return fuse_residual_generic(h.reshape({B * Q, H}).to(at::kFloat), r, g, weight, bias, eps)
      .to(h.scalar_type())
      .reshape({B, Q, H});
}

// gather_apply_backward_queries: d(gather_apply(M, idx, q))/dq for a grad of the
// output, sum_r M[idx_r]^T grad_r, in the queries' dtype (the cast of q to the
// arithmetic type passes the gradient through unchanged, as autograd's .to()).
Tensor gather_apply_backward_queries_generic(const Tensor& memories, const Tensor& indices, const Tensor& grad_out,
                                             const Tensor& queries) {
  check_gather_apply_inputs(memories, indices, queries);
  Tensor sel = batched_memory_gather_generic(memories, indices).to(at::kFloat);  // [B, (Q,) R, H, K]
  Tensor g = grad_out.to(at::kFloat);
  Tensor dq = indices.dim() == 3 ? at::einsum("bqrhk,bqrh->bqk", {sel, g}) : at::einsum("brhk,brh->bk", {sel, g});
  return dq.to(queries.scalar_type());
}

// gather_apply_backward_tokens: per (query, route) pair, M[idx]^T g[q] for one
// float32 gradient row g per query shared by its routes ([B, Q, R, K] float32).
// With g = dL/d(h + sum_r gates_r r_r) it gives both the queries' gradient
// (sum_r gates_r rows) and the gates' (rows . q) without the [B, Q, R, H] rows.
void check_bwd_tokens(const Tensor& memories, const Tensor& indices, const Tensor& grad_tokens) {
  TORCH_CHECK(memories.dim() == 4 && indices.dim() == 3 && grad_tokens.dim() == 3,
              "gather_apply_backward_tokens: memories [B, S, H, K], indices [B, Q, R], grad_tokens [B, Q, H]");
  TORCH_CHECK(indices.size(0) == memories.size(0) && grad_tokens.size(0) == memories.size(0) &&
                  grad_tokens.size(1) == indices.size(1) && grad_tokens.size(2) == memories.size(2),
              "gather_apply_backward_tokens: shape mismatch");
}

Tensor gather_apply_backward_tokens_generic(const Tensor& memories, const Tensor& indices, const Tensor& grad_tokens) {
  check_bwd_tokens(memories, indices, grad_tokens);
  Tensor sel = batched_memory_gather_generic(memories, indices).to(at::kFloat);  // [B, Q, R, H, K]
  return at::einsum("bqrhk,bqh->bqrk", {sel, grad_tokens.to(at::kFloat)}).contiguous();
}

// project_split: LinearMemoryCell.project's split of the concatenated
// projection, F.normalize of keys and queries (paper_grm.py:491-493).
void check_project_split(const Tensor& proj, int64_t dk, int64_t dv, int64_t de) {
  TORCH_CHECK(proj.dim() >= 1 && dk >= 0 && dv >= 0 && de >= 0 && proj.size(-1) == 2 * dk + dv + de,
              "project_split: last dim must be key_dim + value_dim + key_dim + extra_dim");
}

std::tuple<Tensor, Tensor, Tensor, Tensor> project_split_generic(const Tensor& proj, int64_t key_dim,
                                                                 int64_t value_dim, int64_t extra_dim, double eps) {
  check_project_split(proj, key_dim, value_dim, extra_dim);
  auto parts = proj.split_with_sizes({key_dim, value_dim, key_dim, extra_dim}, -1);
  auto normalise = [&](const Tensor& t) { return (t / t.norm(2, {-1}, true).clamp_min(eps)).contiguous(); };
  return {normalise(parts[0]), parts[1].contiguous(), normalise(parts[2]), parts[3].contiguous()};
}

// project_gemm: the projection GEMM and its split in one op, F.linear(x, weight,
// bias) then project_split (paper_grm.py:491-493, 570-574).
std::tuple<Tensor, Tensor, Tensor, Tensor> project_gemm_generic(const Tensor& x, const Tensor& weight,
                                                                const c10::optional<Tensor>& bias, int64_t key_dim,
                                                                int64_t value_dim, int64_t extra_dim, double eps) {
  TORCH_CHECK(x.dim() >= 1 && weight.dim() == 2 && weight.size(1) == x.size(-1) &&
                  weight.size(0) == 2 * key_dim + value_dim + extra_dim,
              "project_gemm: weight must be [2 key_dim + value_dim + extra_dim, in_dim]");
  const Tensor proj = at::linear(x, weight, bias.has_value() ? *bias : Tensor());
  return project_split_generic(proj, key_dim, value_dim, extra_dim, eps);
}

// residual_layer_norm: layer_norm(x + residual) (multilayer_grm.py:92-97).
Tensor residual_layer_norm_generic(const Tensor& x, const Tensor& residual, const c10::optional<Tensor>& weight,
                                   const c10::optional<Tensor>& bias, double eps) {
  TORCH_CHECK(x.sizes() == residual.sizes() && x.dim() >= 1, "residual_layer_norm: x and residual must match");
  return at::layer_norm(x + residual, {x.size(-1)}, weight.has_value() ? *weight : Tensor(),
                        bias.has_value() ? *bias : Tensor(), eps);
}

// linear_residual_layer_norm: the layer's output projection and its block output,
// layer_norm(linear(x, weight, bias) + residual) (paper_grm.py:709,
// multilayer_grm.py:92-97).  With save, also the LayerNorm input and its float32
// row statistics (native_layer_norm's saved tensors, flattened to [rows]).
std::tuple<Tensor, Tensor, Tensor, Tensor> linear_residual_layer_norm_generic(
    const Tensor& x, const Tensor& weight, const c10::optional<Tensor>& bias, const Tensor& residual,
    const c10::optional<Tensor>& ln_weight, const c10::optional<Tensor>& ln_bias, double eps, bool save) {
  TORCH_CHECK(x.dim() >= 1 && weight.dim() == 2 && weight.size(1) == x.size(-1) && residual.dim() == x.dim() &&
                  residual.size(-1) == weight.size(0) && residual.numel() / residual.size(-1) == x.numel() / x.size(-1),
              "linear_residual_layer_norm: weight must be [out_dim, in_dim] and residual [..., out_dim] like x");
  const Tensor s = at::linear(x, weight, bias.has_value() ? *bias : Tensor()) + residual;
  const Tensor w = ln_weight.has_value() ? *ln_weight : Tensor(), b = ln_bias.has_value() ? *ln_bias : Tensor();
  if (!save) return {at::layer_norm(s, {s.size(-1)}, w, b, eps), Tensor(), Tensor(), Tensor()};
  auto res = at::native_layer_norm(s, {s.size(-1)}, w, b, eps);
  return {std::get<0>(res), s, std::get<1>(res).reshape({-1}).to(at::kFloat),
          std::get<2>(res).reshape({-1}).to(at::kFloat)};
}

// archive_cast: float32 states rounded to the model dtype, then to the storage
// dtype, as push() stores them (paper_grm.py:139-140).
Tensor archive_cast_generic(const Tensor& states, at::ScalarType model_dtype, at::ScalarType storage_dtype) {
  TORCH_CHECK(states.scalar_type() == at::kFloat, "archive_cast: states must be float32");
  return states.to(model_dtype).to(storage_dtype);
}

// ---------------------------------------------------------------------------
// HIP (CUDA-key) implementations.

bool same_cuda_device(std::initializer_list<const Tensor*> ts) {
  const Tensor* first = *ts.begin();
  for (const Tensor* t : ts) {
    if (!t->is_cuda() || t->device() != first->device()) return false;
  }
  return true;
}

bool chunk_supported(const Tensor& keys, const Tensor& values, const Tensor& queries,
                     const Tensor& memory) {
  if (!same_cuda_device({&keys, &values, &queries, &memory})) return false;
  const int in = dtype_code(keys.scalar_type());
  if (in < 0 || values.scalar_type() != keys.scalar_type() ||
      queries.scalar_type() != keys.scalar_type())
    return false;
  if (memory.scalar_type() != keys.scalar_type() && memory.scalar_type() != at::kFloat) return false;
  const int64_t max_k = keys.scalar_type() == at::kFloat ? 128 : 256;
  return keys.size(2) >= 1 && keys.size(2) <= max_k && values.size(2) >= 1;
}

std::tuple<Tensor, Tensor, Tensor> chunk_update_forward_hip(const Tensor& keys, const Tensor& values,
                                                            const Tensor& queries,
                                                            const Tensor& memory, double decay) {
  check_chunk_inputs(keys, values, queries, memory);
  if (!chunk_supported(keys, values, queries, memory)) {
    g_generic_calls.fetch_add(1);
    return chunk_update_forward_generic(keys, values, queries, memory, decay);
  }
  c10::OptionalDeviceGuard guard(keys.device());
  if (keys.size(1) == 0) {
    return {at::zeros({keys.size(0), 0, values.size(2)}, values.options()), memory.contiguous(),
            at::empty({0}, memory.options())};
  }
  Tensor k = keys.contiguous(), v = values.contiguous(), q = queries.contiguous();
  Tensor m = memory.contiguous();
  Tensor hidden = at::empty({k.size(0), k.size(1), v.size(2)}, v.options());
  Tensor memory_out = at::empty_like(m);
  Tensor ws = scan_workspace(k, k.size(0), k.size(1), k.size(2), v.size(2), 0);
  check_rc(grm_hip_chunk_update_fwd(k.data_ptr(), v.data_ptr(), q.data_ptr(), m.data_ptr(),
                                    hidden.data_ptr(), memory_out.data_ptr(), nullptr,
                                    ws.numel() ? ws.data_ptr() : nullptr, ws.numel() * 4, k.size(0),
                                    k.size(1), k.size(2), v.size(2), dtype_code(k.scalar_type()),
                                    dtype_code(m.scalar_type()), decay, 0, current_stream(k)),
           "chunk_update_forward");
  return {hidden, memory_out, at::empty({0}, m.options())};
}

std::tuple<Tensor, Tensor, Tensor, Tensor> chunk_update_backward_hip(
    const Tensor& grad_hidden, const Tensor& grad_memory_out, const Tensor& keys,
    const Tensor& values, const Tensor& queries, const Tensor& memory, const Tensor& aux,
    double decay) {
  check_chunk_inputs(keys, values, queries, memory);
  if (!chunk_supported(keys, values, queries, memory) ||
      !same_cuda_device({&keys, &grad_hidden, &grad_memory_out})) {
    g_generic_calls.fetch_add(1);
    return chunk_update_backward_generic(grad_hidden, grad_memory_out, keys, values, queries,
                                         memory, decay);
  }
  c10::OptionalDeviceGuard guard(keys.device());
  Tensor k = keys.contiguous(), v = values.contiguous(), q = queries.contiguous();
  Tensor m = memory.contiguous();
  Tensor gh = grad_hidden.to(v.scalar_type()).contiguous();
  Tensor gmo = grad_memory_out.to(m.scalar_type()).contiguous();
  const int64_t B = k.size(0), T = k.size(1), K = k.size(2), H = v.size(2);
  if (T == 0) return {at::zeros_like(k), at::zeros_like(v), at::zeros_like(q), gmo.clone()};
  Tensor gk = at::empty_like(k), gv = at::empty_like(v), gq = at::empty_like(q);
  Tensor gm = at::empty_like(m);
  auto f32 = k.options().dtype(at::kFloat);
  // aux from this library's forward under autograd holds the state after every
  // 64-token chunk (float32 [B, ceil(T/64), H, K]); anything else (the reference's
  // empty aux) means the backward scans again to produce them.
  const std::vector<int64_t> state_shape = {B, (T + 63) / 64, H, K};
  const bool given = aux.defined() && aux.is_cuda() && aux.device() == k.device() &&
                     aux.scalar_type() == at::kFloat && aux.sizes().vec() == state_shape && aux.is_contiguous();
  Tensor states = given ? aux : at::empty(state_shape, f32);
  Tensor partial = at::empty({2, B, (H + 15) / 16, T, K}, f32);
  check_rc(grm_hip_chunk_update_bwd(gh.data_ptr(), gmo.data_ptr(), k.data_ptr(), v.data_ptr(),
                                    q.data_ptr(), m.data_ptr(), gk.data_ptr(), gv.data_ptr(),
                                    gq.data_ptr(), gm.data_ptr(), states.data_ptr<float>(), given ? 1 : 0,
                                    partial.data_ptr<float>(), B, T, K, H,
                                    dtype_code(k.scalar_type()), dtype_code(m.scalar_type()), decay,
                                    current_stream(k)),
           "chunk_update_backward");
  return {gk, gv, gq, gm};
}

Tensor apply_query_forward_hip(const Tensor& memories, const Tensor& queries) {
  check_apply_inputs(memories, queries);
  const int dt = dtype_code(memories.scalar_type());
  if (!same_cuda_device({&memories, &queries}) || dt < 0 ||
      queries.scalar_type() != memories.scalar_type()) {
    g_generic_calls.fetch_add(1);
    return apply_query_forward_generic(memories, queries);
  }
  c10::OptionalDeviceGuard guard(memories.device());
  Tensor mm = memories.contiguous(), q = queries.contiguous();
  const bool r5 = mm.dim() == 5;
  const int64_t B = mm.size(0), Q = r5 ? mm.size(1) : 1;
  const int64_t R = mm.size(r5 ? 2 : 1), H = mm.size(r5 ? 3 : 2), K = mm.size(r5 ? 4 : 3);
  Tensor out = r5 ? at::empty({B, Q, R, H}, mm.options()) : at::empty({B, R, H}, mm.options());
  check_rc(grm_hip_apply_query_fwd(mm.data_ptr(), q.data_ptr(), out.data_ptr(), B, Q, R, H, K, dt,
                                   current_stream(mm)),
           "apply_query_forward");
  return out;
}

// grad_queries of apply_query_forward alone (the memories need no gradient).
Tensor apply_query_backward_queries_generic(const Tensor& grad_hidden, const Tensor& memories,
                                            const Tensor& queries) {
  check_apply_inputs(memories, queries);
  Tensor dh = grad_hidden.to(memories.scalar_type());
  if (memories.dim() == 5) return at::einsum("bqrh,bqrhk->bqk", {dh, memories}).contiguous();
  return at::einsum("brh,brhk->bk", {dh, memories}).contiguous();
}

Tensor apply_query_backward_queries_hip(const Tensor& grad_hidden, const Tensor& memories,
                                        const Tensor& queries) {
  check_apply_inputs(memories, queries);
  const int dt = dtype_code(memories.scalar_type());
  if (!same_cuda_device({&memories, &queries, &grad_hidden}) || dt < 0 ||
      queries.scalar_type() != memories.scalar_type()) {
    g_generic_calls.fetch_add(1);
    return apply_query_backward_queries_generic(grad_hidden, memories, queries);
  }
  c10::OptionalDeviceGuard guard(memories.device());
  Tensor mm = memories.contiguous(), q = queries.contiguous();
  Tensor dh = grad_hidden.to(mm.scalar_type()).contiguous();
  const bool r5 = mm.dim() == 5;
  const int64_t B = mm.size(0), Q = r5 ? mm.size(1) : 1;
  const int64_t R = mm.size(r5 ? 2 : 1), H = mm.size(r5 ? 3 : 2), K = mm.size(r5 ? 4 : 3);
  Tensor gq = at::empty_like(q);
  check_rc(grm_hip_apply_query_bwd(dh.data_ptr(), mm.data_ptr(), q.data_ptr(), nullptr, gq.data_ptr(), B, Q,
                                   R, H, K, dt, current_stream(mm)),
           "apply_query_backward_queries");
  return gq;
}

std::tuple<Tensor, Tensor> apply_query_backward_hip(const Tensor& grad_hidden,
                                                    const Tensor& memories, const Tensor& queries) {
  check_apply_inputs(memories, queries);
  const int dt = dtype_code(memories.scalar_type());
  if (!same_cuda_device({&memories, &queries, &grad_hidden}) || dt < 0 ||
      queries.scalar_type() != memories.scalar_type()) {
    g_generic_calls.fetch_add(1);
    return apply_query_backward_generic(grad_hidden, memories, queries);
  }
  c10::OptionalDeviceGuard guard(memories.device());
  Tensor mm = memories.contiguous(), q = queries.contiguous();
  Tensor dh = grad_hidden.to(mm.scalar_type()).contiguous();
  const bool r5 = mm.dim() == 5;
  const int64_t B = mm.size(0), Q = r5 ? mm.size(1) : 1;
  const int64_t R = mm.size(r5 ? 2 : 1), H = mm.size(r5 ? 3 : 2), K = mm.size(r5 ? 4 : 3);
  Tensor gm = at::empty_like(mm), gq = at::empty_like(q);
  check_rc(grm_hip_apply_query_bwd(dh.data_ptr(), mm.data_ptr(), q.data_ptr(), gm.data_ptr(),
                                   gq.data_ptr(), B, Q, R, H, K, dt, current_stream(mm)),
           "apply_query_backward");
  return {gm, gq};
}

bool check_indices_requested() {
  const char* e = std::getenv("GRM_HIP_CHECK_INDICES");
  return e != nullptr && e[0] != '\0' && e[0] != '0';
}

Tensor batched_memory_gather_hip(const Tensor& memories, const Tensor& indices) {
  check_gather_inputs(memories, indices);
  if (!same_cuda_device({&memories, &indices})) {
    g_generic_calls.fetch_add(1);
    return batched_memory_gather_generic(memories, indices);
  }
  c10::OptionalDeviceGuard guard(memories.device());
  Tensor mm = memories.contiguous();
  Tensor idx = indices.to(at::kLong).contiguous();
  const int64_t B = mm.size(0), S = mm.size(1);
  std::vector<int64_t> shape{B};
  for (int64_t d = 1; d < idx.dim(); ++d) shape.push_back(idx.size(d));
  shape.push_back(mm.size(2));
  shape.push_back(mm.size(3));
  Tensor out = at::empty(shape, mm.options());
  const int64_t n_index = B > 0 ? idx.numel() / B : 0;
  Tensor bad;
  const bool check = check_indices_requested();
  if (check) bad = at::zeros({1}, mm.options().dtype(at::kInt));
  check_rc(grm_hip_batched_gather(mm.data_ptr(), idx.data_ptr<int64_t>(), out.data_ptr(), B, S,
                                  n_index, mm.size(2) * mm.size(3),
                                  static_cast<int>(mm.element_size()),
                                  check ? bad.data_ptr<int32_t>() : nullptr, current_stream(mm)),
           "batched_memory_gather");
  if (check) {
    const int64_t nbad = bad.item<int32_t>();
    TORCH_CHECK_INDEX(nbad == 0, "batched_memory_gather: ", nbad,
                      " index values outside [0, ", S, ")");
  }
  return out;
}

Tensor gather_apply_hip(const Tensor& memories, const Tensor& indices, const Tensor& queries,
                        std::optional<at::ScalarType> dtype) {
  check_gather_apply_inputs(memories, indices, queries);
  const at::ScalarType t = gather_apply_dtype(memories, dtype);
  if (!same_cuda_device({&memories, &indices, &queries}) || dtype_code(memories.scalar_type()) < 0 ||
      dtype_code(queries.scalar_type()) < 0 || memories.size(3) > 128 || memories.size(1) > 16384) {
    g_generic_calls.fetch_add(1);
    return gather_apply_generic(memories, indices, queries, dtype);
  }
  c10::OptionalDeviceGuard guard(memories.device());
  Tensor mm = memories.contiguous();
  Tensor idx = indices.to(at::kLong).contiguous();
  Tensor q = queries.contiguous();
  const int64_t B = mm.size(0), S = mm.size(1), H = mm.size(2), K = mm.size(3);
  const int64_t Q = idx.dim() == 3 ? idx.size(1) : 1;
  const int64_t R = idx.size(-1);
  std::vector<int64_t> shape{B};
  if (idx.dim() == 3) shape.push_back(Q);
  shape.push_back(R);
  shape.push_back(H);
  Tensor out = at::empty(shape, mm.options().dtype(t));
  const int64_t wsb = grm_hip_gather_apply_workspace(B, S, Q * R);
  Tensor ws = at::empty({std::max<int64_t>(wsb, 16)}, mm.options().dtype(at::kByte));
  Tensor bad;
  const bool check = check_indices_requested();
  if (check) bad = at::zeros({1}, mm.options().dtype(at::kInt));
  check_rc(grm_hip_gather_apply(mm.data_ptr(), idx.data_ptr<int64_t>(), q.data_ptr(), out.data_ptr(), ws.data_ptr(),
                                wsb, B, S, Q, R, H, K, dtype_code(mm.scalar_type()), dtype_code(q.scalar_type()),
                                dtype_code(t), check ? bad.data_ptr<int32_t>() : nullptr, current_stream(mm)),
           "gather_apply");
  if (check) {
    const int64_t nbad = bad.item<int32_t>();
    TORCH_CHECK_INDEX(nbad == 0, "gather_apply: ", nbad, " index values outside [0, ", S, ")");
  }
  return out;
}

// ---- new ops --------------------------------------------------------------

std::tuple<Tensor, Tensor, Tensor> segment_scan_forward_generic(const Tensor& keys,
                                                                const Tensor& values,
                                                                const Tensor& queries,
                                                                const Tensor& memory, double decay,
                                                                int64_t segment_len) {
  check_chunk_inputs(keys, values, queries, memory);
  TORCH_CHECK(segment_len >= 1, "segment_len must be >= 1");
  auto res = chunk_math(keys, values, queries, memory, decay, segment_len);
  auto& snaps = std::get<2>(res);
  Tensor snap = snaps.empty()
                    ? at::empty({keys.size(0), 0, values.size(2), keys.size(2)},
                                keys.options().dtype(at::kFloat))
                    : at::stack(snaps, 1).to(at::kFloat).contiguous();
  return {std::get<0>(res).to(values.scalar_type()).contiguous(),
          std::get<1>(res).to(memory.scalar_type()).contiguous(), snap};
}

std::tuple<Tensor, Tensor, Tensor> segment_scan_forward_hip(const Tensor& keys, const Tensor& values,
                                                            const Tensor& queries,
                                                            const Tensor& memory, double decay,
                                                            int64_t segment_len) {
  check_chunk_inputs(keys, values, queries, memory);
  TORCH_CHECK(segment_len >= 1, "segment_len must be >= 1");
  if (!chunk_supported(keys, values, queries, memory)) {
    g_generic_calls.fetch_add(1);
    return segment_scan_forward_generic(keys, values, queries, memory, decay, segment_len);
  }
  c10::OptionalDeviceGuard guard(keys.device());
  Tensor k = keys.contiguous(), v = values.contiguous(), q = queries.contiguous();
  Tensor m = memory.contiguous();
  const int64_t B = k.size(0), T = k.size(1), K = k.size(2), H = v.size(2);
  const int64_t n_snap = (T + segment_len - 1) / segment_len;
  Tensor hidden = at::empty({B, T, H}, v.options());
  Tensor memory_out = at::empty_like(m);
  Tensor snaps = at::empty({B, n_snap, H, K}, k.options().dtype(at::kFloat));
  if (T == 0) {
    memory_out.copy_(m);
    return {hidden, memory_out, snaps};
  }
  Tensor ws = scan_workspace(k, B, T, K, H, segment_len);
  check_rc(grm_hip_chunk_update_fwd(k.data_ptr(), v.data_ptr(), q.data_ptr(), m.data_ptr(),
                                    hidden.data_ptr(), memory_out.data_ptr(),
                                    snaps.data_ptr<float>(), ws.numel() ? ws.data_ptr() : nullptr,
                                    ws.numel() * 4, B, T, K, H, dtype_code(k.scalar_type()),
                                    dtype_code(m.scalar_type()), decay, segment_len,
                                    current_stream(k)),
           "segment_scan_forward");
  return {hidden, memory_out, snaps};
}

// Queries and keys in one arithmetic type on their device: a mixed or unsupported
// pair is widened to float32 there (bf16 and f16 values are exact in float32, and
// the score is a float32 FMA chain either way).  Routing never leaves the GPU.
std::pair<Tensor, Tensor> route_operands(const char* what, const Tensor& queries, const Tensor& keys) {
  TORCH_CHECK(queries.is_cuda() && keys.is_cuda() && queries.device() == keys.device(),
              what, ": queries and keys must be on the same GPU");
  Tensor q = queries, kk = keys;
  if (q.scalar_type() != kk.scalar_type() || dtype_code(q.scalar_type()) < 0) {
    q = q.to(at::kFloat);
    kk = kk.to(at::kFloat);
  }
  return {q.contiguous(), kk.contiguous()};
}

std::tuple<Tensor, Tensor, Tensor> topk_route_hip(const Tensor& queries, const Tensor& keys,
                                                  int64_t top_k, double scale, double temperature) {
  TORCH_CHECK(queries.dim() == 3 && keys.dim() == 3, "topk_route: queries [B, Q, D], keys [B, S, D]");
  TORCH_CHECK(queries.size(0) == keys.size(0) && queries.size(2) == keys.size(2),
              "topk_route: batch/dim mismatch");
  TORCH_CHECK(top_k >= 1, "topk_route: top_k must be >= 1");
  TORCH_CHECK(temperature > 0, "topk_route: temperature must be > 0");
  const int64_t k = std::min(top_k, keys.size(1));
  if (k > 128 && k < keys.size(1)) {
    // Beyond the select kernels' k: every key's exact score in index order (the
    // k == n_keys branch), then a stable descending sort on the device, which
    // orders equal scores by index as the kernels do.  As in the kernels, a NaN or
    // -inf score is never selected: NaN sorts as -inf, and slots left at -inf are
    // empty (-1, -inf, 0).  Gates as softmax in float64 over the filled slots.
    auto all = topk_route_hip(queries, keys, keys.size(1), scale, temperature);
    Tensor all_sc = std::get<2>(all);
    all_sc = at::where(at::isnan(all_sc), at::full({}, -INFINITY, all_sc.options()), all_sc);
    auto sorted = at::sort(all_sc, /*stable=*/true, /*dim=*/-1, /*descending=*/true);
    Tensor sc = std::get<0>(sorted).narrow(-1, 0, k).contiguous();
    Tensor idx = std::get<1>(all).gather(-1, std::get<1>(sorted).narrow(-1, 0, k)).contiguous();
    const Tensor empty = sc == -INFINITY;
    idx.masked_fill_(empty, -1);
    Tensor gt = at::softmax(sc.to(at::kDouble) / temperature, -1).to(at::kFloat);
    gt.masked_fill_(empty, 0.0);
    return {gt, idx, sc};
  }
  c10::OptionalDeviceGuard guard(queries.device());
  auto [q, kk] = route_operands("topk_route", queries, keys);
  const int64_t B = q.size(0), Q = q.size(1), S = kk.size(1), D = q.size(2);
  Tensor idx = at::empty({B, Q, k}, q.options().dtype(at::kLong));
  Tensor sc = at::empty({B, Q, k}, q.options().dtype(at::kFloat));
  Tensor gt = at::empty({B, Q, k}, q.options().dtype(at::kFloat));
  if (k > 0 && Q > 0 && B > 0) {
    check_rc(grm_hip_topk_route(q.data_ptr(), kk.data_ptr(), idx.data_ptr<int64_t>(),
                                sc.data_ptr<float>(), gt.data_ptr<float>(), B, Q, S, D,
                                dtype_code(q.scalar_type()), top_k, static_cast<float>(scale),
                                static_cast<float>(temperature), current_stream(q)),
             "topk_route");
  }
  return {gt, idx, sc};
}

std::tuple<Tensor, Tensor, Tensor> segment_route_hip(const Tensor& queries, const Tensor& keys, int64_t top_k,
                                                     int64_t segment_len, int64_t base, int64_t capacity,
                                                     double scale, double temperature) {
  check_segment_route(queries, keys, top_k, segment_len, base, capacity, temperature);
  c10::OptionalDeviceGuard guard(queries.device());
  auto [q, kk] = route_operands("segment_route", queries, keys);
  const int64_t B = q.size(0), Q = q.size(1), S = kk.size(1), D = q.size(2);
  Tensor idx = at::empty({B, Q, top_k}, q.options().dtype(at::kLong));
  Tensor sc = at::empty({B, Q, top_k}, q.options().dtype(at::kFloat));
  Tensor gt = at::empty({B, Q, top_k}, q.options().dtype(at::kFloat));
  if (Q > 0 && B > 0) {
    check_rc(grm_hip_segment_route(q.data_ptr(), S > 0 ? kk.data_ptr() : nullptr, idx.data_ptr<int64_t>(),
                                   sc.data_ptr<float>(), gt.data_ptr<float>(), B, Q, S, D,
                                   dtype_code(q.scalar_type()), top_k, segment_len, base, capacity,
                                   static_cast<float>(scale), static_cast<float>(temperature),
                                   current_stream(q)),
             "segment_route");
  }
  return {gt, idx, sc};
}

Tensor fuse_residual_hip(const Tensor& h, const Tensor& retrieved, const Tensor& gates,
                         const c10::optional<Tensor>& weight, const c10::optional<Tensor>& bias,
                         double eps) {
  TORCH_CHECK(h.dim() == 2 && retrieved.dim() == 3 && gates.dim() == 2,
              "fuse_residual: h [N, H], retrieved [N, R, H], gates [N, R]");
  TORCH_CHECK(retrieved.size(0) == h.size(0) && retrieved.size(2) == h.size(1) &&
                  gates.size(0) == h.size(0) && gates.size(1) == retrieved.size(1),
              "fuse_residual: shape mismatch");
  const bool has_w = weight.has_value() && weight->defined();
  const bool has_b = bias.has_value() && bias->defined();
  const int dt = dtype_code(h.scalar_type());
  bool ok = same_cuda_device({&h, &retrieved, &gates}) && dt >= 0 &&
            retrieved.scalar_type() == h.scalar_type() && h.size(1) <= 2048;
  if (has_w) ok = ok && weight->is_cuda() && weight->scalar_type() == h.scalar_type();
  if (has_b) ok = ok && has_w && bias->is_cuda() && bias->scalar_type() == h.scalar_type();
  if (!ok) {
    if (h.is_cuda()) g_generic_calls.fetch_add(1);
    return fuse_residual_generic(h, retrieved, gates, weight, bias, eps);
  }
  c10::OptionalDeviceGuard guard(h.device());
  Tensor hc = h.contiguous(), rc = retrieved.contiguous();
  Tensor gc = gates.to(at::kFloat).contiguous();
  Tensor wc = has_w ? weight->contiguous() : Tensor();
  Tensor bc = has_b ? bias->contiguous() : Tensor();
  Tensor out = at::empty_like(hc);
  check_rc(grm_hip_fuse_residual(hc.data_ptr(), rc.data_ptr(), gc.data_ptr<float>(),
                                 has_w ? wc.data_ptr() : nullptr, has_b ? bc.data_ptr() : nullptr,
                                 out.data_ptr(), hc.size(0), rc.size(1), hc.size(1), dt,
                                 static_cast<float>(eps), current_stream(hc)),
           "fuse_residual");
  return out;
}

bool aligned16(const Tensor& t) { return reinterpret_cast<uintptr_t>(t.data_ptr()) % 16 == 0; }

Tensor retrieve_fuse_hip(const Tensor& memories, const Tensor& indices, const Tensor& queries, const Tensor& gates,
                         const Tensor& h, const c10::optional<Tensor>& weight, const c10::optional<Tensor>& bias,
                         double eps) {
  check_retrieve_fuse_inputs(memories, indices, queries, gates, h);
  const bool has_w = weight.has_value() && weight->defined();
  const bool has_b = bias.has_value() && bias->defined();
  const int64_t B = memories.size(0), S = memories.size(1), H = memories.size(2), K = memories.size(3);
  const int64_t Q = indices.size(1), R = indices.size(2);
  const int md = dtype_code(memories.scalar_type()), qd = dtype_code(queries.scalar_type());
  const int hd = dtype_code(h.scalar_type());
  const bool q16 = queries.scalar_type() == at::kBFloat16 ||
                   (queries.scalar_type() == at::kHalf && memories.scalar_type() == at::kHalf);
  bool ok = same_cuda_device({&memories, &indices, &queries, &gates, &h}) && md >= 0 && qd >= 0 && hd >= 0 && q16 &&
            K <= 128 && (K * 2) % 16 == 0 && H % 8 == 0 && H <= 2048 && S <= 16384 && B <= 65535;
  if (has_w) ok = ok && weight->is_cuda() && weight->numel() == H;
  if (has_b) ok = ok && has_w && bias->is_cuda() && bias->numel() == H;
  if (!ok) {
    // The two-kernel composition (gather_apply in float32, then fuse_residual).
    const Tensor r = gather_apply_hip(memories, indices, queries, at::kFloat).reshape({B * Q, R, H});
    c10::optional<Tensor> wf, bf;
    if (has_w) wf = weight->to(at::kFloat);
    if (has_b) bf = bias->to(at::kFloat);
    return fuse_residual_hip(h.reshape({B * Q, H}).to(at::kFloat), r, gates.reshape({B * Q, R}), wf, bf, eps)
        .to(h.scalar_type())
        .reshape({B, Q, H});
  }
  c10::OptionalDeviceGuard guard(memories.device());
  Tensor mm = memories.contiguous(), idx = indices.to(at::kLong).contiguous(), q = queries.contiguous();
  Tensor gc = gates.to(at::kFloat).contiguous(), hc = h.contiguous();
  Tensor wc = has_w ? weight->to(at::kFloat).contiguous() : Tensor();
  Tensor bc = has_b ? bias->to(at::kFloat).contiguous() : Tensor();
  if (!aligned16(mm) || !aligned16(q) || !aligned16(hc) || (has_w && !aligned16(wc)) || (has_b && !aligned16(bc))) {
    mm = mm.clone();
    q = q.clone();
    hc = hc.clone();
    if (has_w) wc = wc.clone();
    if (has_b) bc = bc.clone();
  }
  Tensor out = at::empty_like(hc);
  const int64_t wsb = grm_hip_retrieve_fuse_workspace(B, S, Q * R, H);
  Tensor ws = at::empty({std::max<int64_t>(wsb, 16)}, mm.options().dtype(at::kByte));
  Tensor bad;
  const bool check = check_indices_requested();
  if (check) bad = at::zeros({1}, mm.options().dtype(at::kInt));
  check_rc(grm_hip_retrieve_fuse(mm.data_ptr(), idx.data_ptr<int64_t>(), q.data_ptr(), gc.data_ptr<float>(),
                                 hc.data_ptr(), has_w ? wc.data_ptr() : nullptr, has_b ? bc.data_ptr() : nullptr,
                                 out.data_ptr(), ws.data_ptr(), wsb, B, S, Q, R, H, K, md, qd, hd,
                                 static_cast<float>(eps), check ? bad.data_ptr<int32_t>() : nullptr,
                                 current_stream(mm)),
           "retrieve_fuse");
  if (check) {
    const int64_t nbad = bad.item<int32_t>();
    TORCH_CHECK_INDEX(nbad == 0, "retrieve_fuse: ", nbad, " index values outside [0, ", S, ")");
  }
  return out;
}

Tensor segment_retrieve_fuse_hip(const Tensor& memories, const Tensor& indices, const Tensor& queries,
                                 const Tensor& gates, const Tensor& h, const c10::optional<Tensor>& weight,
                                 const c10::optional<Tensor>& bias, double eps, int64_t segment_len, int64_t base,
                                 int64_t capacity) {
  check_retrieve_fuse_inputs(memories, indices, queries, gates, h);
  check_segment_window(segment_len, base, capacity);
  const bool has_w = weight.has_value() && weight->defined();
  const bool has_b = bias.has_value() && bias->defined();
  const int64_t B = memories.size(0), S = memories.size(1), H = memories.size(2), K = memories.size(3);
  const int64_t Q = indices.size(1), R = indices.size(2);
  TORCH_CHECK(Q == 0 || base + (Q - 1) / segment_len <= S,
              "segment_retrieve_fuse: windows past the archive (base + (Q - 1) / segment_len > segments)");
  const int md = dtype_code(memories.scalar_type()), qd = dtype_code(queries.scalar_type());
  const int hd = dtype_code(h.scalar_type());
  const bool q16 = queries.scalar_type() == at::kBFloat16 ||
                   (queries.scalar_type() == at::kHalf && memories.scalar_type() == at::kHalf);
  bool ok = same_cuda_device({&memories, &indices, &queries, &gates, &h}) && md >= 0 && qd >= 0 && hd >= 0 && q16 &&
            K <= 128 && K % 8 == 0 && H % 8 == 0 && H <= 2048 && R <= 32;
  if (has_w) ok = ok && weight->is_cuda() && weight->numel() == H;
  if (has_b) ok = ok && has_w && bias->is_cuda() && bias->numel() == H;
  // retrieve_fuse over the masked pairs (an invalid pair: index 0, gate 0): the inputs the
  // window kernel does not cover, including windows wider than one workgroup's entries
  auto masked = [&]() {
    Tensor valid = segment_window_valid(indices, segment_len, base, capacity);
    check_window_indices(indices, valid);
    if (S == 0) return segment_retrieve_fuse_generic(memories, indices, queries, gates, h, weight, bias, eps,
                                                     segment_len, base, capacity);
    return retrieve_fuse_hip(memories, indices.to(at::kLong).masked_fill(valid.logical_not(), 0), queries,
                             gates.to(at::kFloat).masked_fill(valid.logical_not(), 0.0), h, weight, bias, eps);
  };
  if (!ok) return masked();
  c10::OptionalDeviceGuard guard(memories.device());
  Tensor mm = memories.contiguous(), idx = indices.to(at::kLong).contiguous(), q = queries.contiguous();
  Tensor gc = gates.to(at::kFloat).contiguous(), hc = h.contiguous();
  Tensor wc = has_w ? weight->to(at::kFloat).contiguous() : Tensor();
  Tensor bc = has_b ? bias->to(at::kFloat).contiguous() : Tensor();
  if (!aligned16(mm) || !aligned16(q) || !aligned16(hc) || (has_w && !aligned16(wc)) || (has_b && !aligned16(bc))) {
    mm = mm.clone();
    q = q.clone();
    hc = hc.clone();
    if (has_w) wc = wc.clone();
    if (has_b) bc = bc.clone();
  }
  Tensor out = at::empty_like(hc);
  const int64_t wsb = grm_hip_segment_retrieve_fuse_workspace(B, Q, H, K, segment_len, base, capacity, md);
  Tensor ws = at::empty({std::max<int64_t>(wsb, 16)}, mm.options().dtype(at::kByte));
  Tensor bad;
  const bool check = check_indices_requested();
  if (check) bad = at::zeros({1}, mm.options().dtype(at::kInt));
  const int rc = grm_hip_segment_retrieve_fuse(mm.data_ptr(), idx.data_ptr<int64_t>(), q.data_ptr(),
                                               gc.data_ptr<float>(), hc.data_ptr(), has_w ? wc.data_ptr() : nullptr,
                                               has_b ? bc.data_ptr() : nullptr, out.data_ptr(), ws.data_ptr(), wsb, B,
                                               S, Q, R, H, K, segment_len, base, capacity, md, qd, hd,
                                               static_cast<float>(eps), check ? bad.data_ptr<int32_t>() : nullptr,
                                               current_stream(mm));
  if (rc == GRM_HIP_EUNSUPPORTED) return masked();  // rejected before any launch
  check_rc(rc, "segment_retrieve_fuse");
  if (check) {
    const int64_t nbad = bad.item<int32_t>();
    TORCH_CHECK_INDEX(nbad == 0, "segment_retrieve_fuse: ", nbad,
                      " index values outside their query's window or repeated");
  }
  return out;
}

Tensor gather_apply_backward_queries_hip(const Tensor& memories, const Tensor& indices, const Tensor& grad_out,
                                         const Tensor& queries) {
  check_gather_apply_inputs(memories, indices, queries);
  const int64_t B = memories.size(0), S = memories.size(1), H = memories.size(2), K = memories.size(3);
  const int64_t kp = K <= 16 ? 16 : K <= 32 ? 32 : K <= 64 ? 64 : 128;
  if (!same_cuda_device({&memories, &indices, &grad_out, &queries}) || dtype_code(memories.scalar_type()) < 0 ||
      K > 128 || S > 16384 || (H + 15) / 16 * 16 * (kp + 4) * 4 > 160 * 1024) {
    if (memories.is_cuda()) g_generic_calls.fetch_add(1);
    return gather_apply_backward_queries_generic(memories, indices, grad_out, queries);
  }
  c10::OptionalDeviceGuard guard(memories.device());
  Tensor mm = memories.contiguous();
  Tensor idx = indices.to(at::kLong).contiguous();
  Tensor g = grad_out.to(at::kFloat).contiguous();
  const int64_t Q = idx.dim() == 3 ? idx.size(1) : 1;
  const int64_t R = idx.size(-1);
  Tensor gp = at::empty({B, Q, R, K}, mm.options().dtype(at::kFloat));
  const int64_t wsb = grm_hip_gather_apply_workspace(B, S, Q * R);
  Tensor ws = at::empty({std::max<int64_t>(wsb, 16)}, mm.options().dtype(at::kByte));
  Tensor bad;
  const bool check = check_indices_requested();
  if (check) bad = at::zeros({1}, mm.options().dtype(at::kInt));
  check_rc(grm_hip_gather_apply_bwd_queries(mm.data_ptr(), idx.data_ptr<int64_t>(), g.data_ptr<float>(),
                                            gp.data_ptr<float>(), ws.data_ptr(), wsb, B, S, Q, R, H, K,
                                            dtype_code(mm.scalar_type()), check ? bad.data_ptr<int32_t>() : nullptr,
                                            current_stream(mm)),
           "gather_apply_backward_queries");
  if (check) {
    const int64_t nbad = bad.item<int32_t>();
    TORCH_CHECK_INDEX(nbad == 0, "gather_apply: ", nbad, " index values outside [0, ", S, ")");
  }
  Tensor dq = gp.sum(2);  // fixed-order reduction over the routes
  if (idx.dim() == 2) dq = dq.squeeze(1);
  return dq.to(queries.scalar_type());
}

Tensor gather_apply_backward_tokens_hip(const Tensor& memories, const Tensor& indices, const Tensor& grad_tokens) {
  check_bwd_tokens(memories, indices, grad_tokens);
  const int64_t B = memories.size(0), S = memories.size(1), H = memories.size(2), K = memories.size(3);
  const int64_t kp = K <= 16 ? 16 : K <= 32 ? 32 : K <= 64 ? 64 : 128;
  if (!same_cuda_device({&memories, &indices, &grad_tokens}) || dtype_code(memories.scalar_type()) < 0 ||
      K > 128 || S > 16384 || (H + 15) / 16 * 16 * (kp + 4) * 4 > 160 * 1024) {
    if (memories.is_cuda()) g_generic_calls.fetch_add(1);
    return gather_apply_backward_tokens_generic(memories, indices, grad_tokens);
  }
  c10::OptionalDeviceGuard guard(memories.device());
  Tensor mm = memories.contiguous();
  Tensor idx = indices.to(at::kLong).contiguous();
  Tensor g = grad_tokens.to(at::kFloat).contiguous();
  const int64_t Q = idx.size(1), R = idx.size(2);
  Tensor gp = at::empty({B, Q, R, K}, mm.options().dtype(at::kFloat));
  const int64_t wsb = grm_hip_gather_apply_workspace(B, S, Q * R);
  Tensor ws = at::empty({std::max<int64_t>(wsb, 16)}, mm.options().dtype(at::kByte));
  Tensor bad;
  const bool check = check_indices_requested();
  if (check) bad = at::zeros({1}, mm.options().dtype(at::kInt));
  check_rc(grm_hip_gather_apply_bwd_tokens(mm.data_ptr(), idx.data_ptr<int64_t>(), g.data_ptr<float>(),
                                           gp.data_ptr<float>(), ws.data_ptr(), wsb, B, S, Q, R, H, K,
                                           dtype_code(mm.scalar_type()), check ? bad.data_ptr<int32_t>() : nullptr,
                                           current_stream(mm)),
           "gather_apply_backward_tokens");
  if (check) {
    const int64_t nbad = bad.item<int32_t>();
    TORCH_CHECK_INDEX(nbad == 0, "gather_apply: ", nbad, " index values outside [0, ", S, ")");
  }
  return gp;
}

std::tuple<Tensor, Tensor, Tensor, Tensor> project_split_hip(const Tensor& proj, int64_t key_dim, int64_t value_dim,
                                                             int64_t extra_dim, double eps) {
  check_project_split(proj, key_dim, value_dim, extra_dim);
  const int dt = dtype_code(proj.scalar_type());
  if (!proj.is_cuda() || dt < 0 || key_dim % 8 || value_dim % 8 || extra_dim % 8) {
    if (proj.is_cuda()) g_generic_calls.fetch_add(1);
    return project_split_generic(proj, key_dim, value_dim, extra_dim, eps);
  }
  c10::OptionalDeviceGuard guard(proj.device());
  Tensor p = proj.contiguous();
  if (!aligned16(p)) p = p.clone();
  auto lead = p.sizes().vec();
  lead.pop_back();
  auto mk = [&](int64_t d) {
    auto shape = lead;
    shape.push_back(d);
    return at::empty(shape, p.options());
  };
  Tensor k = mk(key_dim), v = mk(value_dim), q = mk(key_dim), e = mk(extra_dim);
  const int64_t rows = p.size(-1) > 0 ? p.numel() / p.size(-1) : 0;
  check_rc(grm_hip_project_split(p.data_ptr(), k.data_ptr(), v.data_ptr(), q.data_ptr(),
                                 extra_dim > 0 ? e.data_ptr() : nullptr, rows, key_dim, value_dim, extra_dim, dt,
                                 static_cast<float>(eps), current_stream(p)),
           "project_split");
  return {k, v, q, e};
}

std::tuple<Tensor, Tensor, Tensor, Tensor> project_gemm_hip(const Tensor& x, const Tensor& weight,
                                                            const c10::optional<Tensor>& bias, int64_t key_dim,
                                                            int64_t value_dim, int64_t extra_dim, double eps) {
  TORCH_CHECK(x.dim() >= 1 && weight.dim() == 2 && weight.size(1) == x.size(-1) &&
                  weight.size(0) == 2 * key_dim + value_dim + extra_dim,
              "project_gemm: weight must be [2 key_dim + value_dim + extra_dim, in_dim]");
  const bool has_b = bias.has_value() && bias->defined();
  const int dt = dtype_code(x.scalar_type());
  const int64_t K = x.size(-1);
  const int64_t rows = K > 0 ? x.numel() / K : 0;
  bool ok = x.is_cuda() && weight.is_cuda() && (dt == 1 || dt == 2) && weight.scalar_type() == x.scalar_type() &&
            key_dim == 64 && value_dim % 64 == 0 && extra_dim % 64 == 0 && K % 64 == 0 && K > 0 &&
            rows * K * 2 <= INT32_MAX && weight.numel() * 2 <= INT32_MAX;
  if (has_b) ok = ok && bias->is_cuda() && bias->scalar_type() == x.scalar_type() && bias->numel() == weight.size(0);
  if (!ok) {
    // Shapes the fused kernel does not take: the library GEMM, then the split's own kernel
    // (which counts a generic call only where it falls back itself).
    return project_split_hip(at::linear(x, weight, has_b ? *bias : Tensor()), key_dim, value_dim, extra_dim, eps);
  }
  c10::OptionalDeviceGuard guard(x.device());
  Tensor xc = x.contiguous(), wc = weight.contiguous();
  Tensor bc = has_b ? bias->contiguous() : Tensor();
  if (!aligned16(xc)) xc = xc.clone();
  if (!aligned16(wc)) wc = wc.clone();
  auto lead = xc.sizes().vec();
  lead.pop_back();
  auto mk = [&](int64_t d) {
    auto shape = lead;
    shape.push_back(d);
    return at::empty(shape, xc.options());
  };
  Tensor k = mk(key_dim), v = mk(value_dim), q = mk(key_dim), e = mk(extra_dim);
  check_rc(grm_hip_project_gemm(xc.data_ptr(), wc.data_ptr(), has_b ? bc.data_ptr() : nullptr, k.data_ptr(),
                                v.data_ptr(), q.data_ptr(), extra_dim > 0 ? e.data_ptr() : nullptr, rows, K, key_dim,
                                value_dim, extra_dim, dt, static_cast<float>(eps), current_stream(xc)),
           "project_gemm");
  return {k, v, q, e};
}

Tensor residual_layer_norm_hip(const Tensor& x, const Tensor& residual, const c10::optional<Tensor>& weight,
                               const c10::optional<Tensor>& bias, double eps) {
  TORCH_CHECK(x.sizes() == residual.sizes() && x.dim() >= 1, "residual_layer_norm: x and residual must match");
  const bool has_w = weight.has_value() && weight->defined();
  const bool has_b = bias.has_value() && bias->defined();
  const int dt = dtype_code(x.scalar_type());
  const int pd = has_w ? dtype_code(weight->scalar_type()) : dt;
  const int64_t H = x.size(-1);
  bool ok = same_cuda_device({&x, &residual}) && residual.scalar_type() == x.scalar_type() && dt >= 0 && pd >= 0 &&
            H % 8 == 0 && H <= 2048;
  if (has_w) ok = ok && weight->is_cuda() && weight->numel() == H;
  if (has_b) ok = ok && has_w && bias->is_cuda() && bias->numel() == H && bias->scalar_type() == weight->scalar_type();
  if (!ok) {
    if (x.is_cuda()) g_generic_calls.fetch_add(1);
    return residual_layer_norm_generic(x, residual, weight, bias, eps);
  }
  c10::OptionalDeviceGuard guard(x.device());
  Tensor xc = x.contiguous(), rc = residual.contiguous();
  Tensor wc = has_w ? weight->contiguous() : Tensor(), bc = has_b ? bias->contiguous() : Tensor();
  if (!aligned16(xc)) xc = xc.clone();
  if (!aligned16(rc)) rc = rc.clone();
  if (has_w && !aligned16(wc)) wc = wc.clone();
  if (has_b && !aligned16(bc)) bc = bc.clone();
  Tensor out = at::empty_like(xc);
  check_rc(grm_hip_residual_layer_norm(xc.data_ptr(), rc.data_ptr(), has_w ? wc.data_ptr() : nullptr,
                                       has_b ? bc.data_ptr() : nullptr, out.data_ptr(), xc.numel() / H, H, dt, pd,
                                       static_cast<float>(eps), current_stream(xc)),
           "residual_layer_norm");
  return out;
}

std::tuple<Tensor, Tensor, Tensor, Tensor> linear_residual_layer_norm_hip(
    const Tensor& x, const Tensor& weight, const c10::optional<Tensor>& bias, const Tensor& residual,
    const c10::optional<Tensor>& ln_weight, const c10::optional<Tensor>& ln_bias, double eps, bool save) {
  TORCH_CHECK(x.dim() >= 1 && weight.dim() == 2 && weight.size(1) == x.size(-1) && residual.dim() == x.dim() &&
                  residual.size(-1) == weight.size(0) && residual.numel() / residual.size(-1) == x.numel() / x.size(-1),
              "linear_residual_layer_norm: weight must be [out_dim, in_dim] and residual [..., out_dim] like x");
  const bool has_b = bias.has_value() && bias->defined();
  const bool has_w = ln_weight.has_value() && ln_weight->defined();
  const bool has_lb = ln_bias.has_value() && ln_bias->defined();
  const int dt = dtype_code(x.scalar_type());
  const int pd = has_w ? dtype_code(ln_weight->scalar_type()) : dt;
  const int64_t K = x.size(-1), N = weight.size(0);
  const int64_t rows = K > 0 ? x.numel() / K : 0;
  bool ok = same_cuda_device({&x, &weight, &residual}) && (dt == 1 || dt == 2) &&
            weight.scalar_type() == x.scalar_type() && residual.scalar_type() == x.scalar_type() && pd >= 0 &&
            K % 64 == 0 && K > 0 && N % 64 == 0 && N > 0 && N <= 512 && weight.numel() * 2 <= INT32_MAX;
  if (has_b) ok = ok && bias->is_cuda() && bias->scalar_type() == x.scalar_type() && bias->numel() == N;
  if (has_w) ok = ok && ln_weight->is_cuda() && ln_weight->numel() == N;
  if (has_lb) ok = ok && has_w && ln_bias->is_cuda() && ln_bias->numel() == N &&
                   ln_bias->scalar_type() == ln_weight->scalar_type();
  if (!ok) {
    if (x.is_cuda()) g_generic_calls.fetch_add(1);
    return linear_residual_layer_norm_generic(x, weight, bias, residual, ln_weight, ln_bias, eps, save);
  }
  c10::OptionalDeviceGuard guard(x.device());
  Tensor xc = x.contiguous(), wc = weight.contiguous(), rc = residual.contiguous();
  Tensor bc = has_b ? bias->contiguous() : Tensor();
  Tensor lw = has_w ? ln_weight->contiguous() : Tensor(), lb = has_lb ? ln_bias->contiguous() : Tensor();
  if (!aligned16(xc)) xc = xc.clone();
  if (!aligned16(wc)) wc = wc.clone();
  if (!aligned16(rc)) rc = rc.clone();
  if (has_w && !aligned16(lw)) lw = lw.clone();
  if (has_lb && !aligned16(lb)) lb = lb.clone();
  Tensor out = at::empty_like(rc);
  Tensor pre = save ? at::empty_like(rc) : Tensor();
  Tensor mean = save ? at::empty({rows}, xc.options().dtype(at::kFloat)) : Tensor();
  Tensor rstd = save ? at::empty({rows}, xc.options().dtype(at::kFloat)) : Tensor();
  check_rc(grm_hip_linear_residual_layer_norm(
               xc.data_ptr(), wc.data_ptr(), has_b ? bc.data_ptr() : nullptr, rc.data_ptr(),
               has_w ? lw.data_ptr() : nullptr, has_lb ? lb.data_ptr() : nullptr, out.data_ptr(),
               save ? pre.data_ptr() : nullptr, save ? mean.data_ptr<float>() : nullptr,
               save ? rstd.data_ptr<float>() : nullptr, rows, K, N, dt, pd, static_cast<float>(eps),
               current_stream(xc)),
           "linear_residual_layer_norm");
  return {out, pre, mean, rstd};
}

// CPU-key wrappers for the generic forms.
std::tuple<Tensor, Tensor, Tensor, Tensor> chunk_update_backward_cpu(
    const Tensor& grad_hidden, const Tensor& grad_memory_out, const Tensor& keys,
    const Tensor& values, const Tensor& queries, const Tensor& memory, const Tensor& aux,
    double decay) {
  (void)aux;
  check_chunk_inputs(keys, values, queries, memory);
  return chunk_update_backward_generic(grad_hidden, grad_memory_out, keys, values, queries, memory,
                                       decay);
}

}  // namespace
Tensor archive_cast_hip(const Tensor& states, at::ScalarType model_dtype, at::ScalarType storage_dtype) {
  TORCH_CHECK(states.scalar_type() == at::kFloat, "archive_cast: states must be float32");
  const int md = dtype_code(model_dtype), sd = dtype_code(storage_dtype);
  Tensor x = states.contiguous();
  if (md < 0 || sd < 0 || !states.is_cuda() || !aligned16(x)) {
    if (states.is_cuda()) g_generic_calls.fetch_add(1);
    return archive_cast_generic(states, model_dtype, storage_dtype);
  }
  c10::OptionalDeviceGuard guard(states.device());
  Tensor out = at::empty(x.sizes(), x.options().dtype(storage_dtype));
  check_rc(grm_hip_archive_cast(x.data_ptr<float>(), out.data_ptr(), x.numel(), md, sd, current_stream(x)),
           "archive_cast");
  return out;
}

}  // namespace grm

TORCH_LIBRARY(grm_cuda, m) {
  m.def("chunk_update_forward(Tensor keys, Tensor values, Tensor queries, Tensor memory, float memory_decay) -> (Tensor hidden, Tensor memory_out, Tensor aux)");
  m.def("chunk_update_backward(Tensor grad_hidden, Tensor grad_memory_out, Tensor keys, Tensor values, Tensor queries, Tensor memory, Tensor aux, float memory_decay) -> (Tensor grad_keys, Tensor grad_values, Tensor grad_queries, Tensor grad_memory)");
  m.def("apply_query_forward(Tensor memories, Tensor queries) -> Tensor");
  m.def("apply_query_backward(Tensor grad_hidden, Tensor memories, Tensor queries) -> (Tensor grad_memories, Tensor grad_queries)");
  m.def("apply_query_backward_queries(Tensor grad_hidden, Tensor memories, Tensor queries) -> Tensor");
  m.def("batched_memory_gather(Tensor memories_per_batch, Tensor topk_indices) -> Tensor");
  m.def("segment_scan_forward(Tensor keys, Tensor values, Tensor queries, Tensor memory, float memory_decay, int segment_len) -> (Tensor hidden, Tensor memory_out, Tensor snapshots)");
  m.def("topk_route(Tensor queries, Tensor keys, int top_k, float scale, float temperature) -> (Tensor gates, Tensor indices, Tensor scores)");
  m.def("fuse_residual(Tensor h_online, Tensor retrieved, Tensor gates, Tensor? weight, Tensor? bias, float eps) -> Tensor");
  m.def("gather_apply(Tensor memories, Tensor indices, Tensor queries, ScalarType? dtype=None) -> Tensor");
  m.def("segment_route(Tensor queries, Tensor keys, int top_k, int segment_len, int base, int capacity, float scale, float temperature) -> (Tensor gates, Tensor indices, Tensor scores)");
  m.def("retrieve_fuse(Tensor memories, Tensor indices, Tensor queries, Tensor gates, Tensor h_online, Tensor? weight, Tensor? bias, float eps) -> Tensor");
  m.def("project_split(Tensor proj, int key_dim, int value_dim, int extra_dim, float eps) -> (Tensor keys, Tensor values, Tensor queries, Tensor extra)");
  m.def("gather_apply_backward_queries(Tensor memories, Tensor indices, Tensor grad_out, Tensor queries) -> Tensor");
  m.def("gather_apply_backward_tokens(Tensor memories, Tensor indices, Tensor grad_tokens) -> Tensor");
  m.def("residual_layer_norm(Tensor x, Tensor residual, Tensor? weight, Tensor? bias, float eps) -> Tensor");
  m.def("archive_cast(Tensor states, ScalarType model_dtype, ScalarType storage_dtype) -> Tensor");
  m.def("project_gemm(Tensor x, Tensor weight, Tensor? bias, int key_dim, int value_dim, int extra_dim, float eps) "
        "-> (Tensor, Tensor, Tensor, Tensor)");
  m.def("linear_residual_layer_norm(Tensor x, Tensor weight, Tensor? bias, Tensor residual, Tensor? ln_weight, "
        "Tensor? ln_bias, float eps, bool save) -> (Tensor out, Tensor pre, Tensor mean, Tensor rstd)");
  m.def("segment_retrieve_fuse(Tensor memories, Tensor indices, Tensor queries, Tensor gates, Tensor h_online, "
        "Tensor? weight, Tensor? bias, float eps, int segment_len, int base, int capacity) -> Tensor");
}

TORCH_LIBRARY_IMPL(grm_cuda, CPU, m) {
  m.impl("chunk_update_forward", grm::chunk_update_forward_generic);
  m.impl("chunk_update_backward", grm::chunk_update_backward_cpu);
  m.impl("apply_query_forward", grm::apply_query_forward_generic);
  m.impl("apply_query_backward", grm::apply_query_backward_generic);
  m.impl("apply_query_backward_queries", grm::apply_query_backward_queries_generic);
  m.impl("batched_memory_gather", grm::batched_memory_gather_generic);
  m.impl("segment_scan_forward", grm::segment_scan_forward_generic);
  m.impl("topk_route", grm::topk_route_cpu);
  m.impl("fuse_residual", grm::fuse_residual_generic);
  m.impl("gather_apply", grm::gather_apply_generic);
  m.impl("segment_route", grm::segment_route_cpu);
  m.impl("retrieve_fuse", grm::retrieve_fuse_generic);
  m.impl("project_split", grm::project_split_generic);
  m.impl("gather_apply_backward_queries", grm::gather_apply_backward_queries_generic);
  m.impl("gather_apply_backward_tokens", grm::gather_apply_backward_tokens_generic);
  m.impl("residual_layer_norm", grm::residual_layer_norm_generic);
  m.impl("archive_cast", grm::archive_cast_generic);
  m.impl("project_gemm", grm::project_gemm_generic);
  m.impl("linear_residual_layer_norm", grm::linear_residual_layer_norm_generic);
  m.impl("segment_retrieve_fuse", grm::segment_retrieve_fuse_generic);
}

TORCH_LIBRARY_IMPL(grm_cuda, CUDA, m) {
  m.impl("chunk_update_forward", grm::chunk_update_forward_hip);
  m.impl("chunk_update_backward", grm::chunk_update_backward_hip);
  m.impl("apply_query_forward", grm::apply_query_forward_hip);
  m.impl("apply_query_backward", grm::apply_query_backward_hip);
  m.impl("apply_query_backward_queries", grm::apply_query_backward_queries_hip);
  m.impl("batched_memory_gather", grm::batched_memory_gather_hip);
  m.impl("segment_scan_forward", grm::segment_scan_forward_hip);
  m.impl("topk_route", grm::topk_route_hip);
  m.impl("fuse_residual", grm::fuse_residual_hip);
  m.impl("gather_apply", grm::gather_apply_hip);
  m.impl("segment_route", grm::segment_route_hip);
  m.impl("retrieve_fuse", grm::retrieve_fuse_hip);
  m.impl("project_split", grm::project_split_hip);
  m.impl("gather_apply_backward_queries", grm::gather_apply_backward_queries_hip);
  m.impl("gather_apply_backward_tokens", grm::gather_apply_backward_tokens_hip);
  m.impl("residual_layer_norm", grm::residual_layer_norm_hip);
  m.impl("archive_cast", grm::archive_cast_hip);
  m.impl("project_gemm", grm::project_gemm_hip);
  m.impl("linear_residual_layer_norm", grm::linear_residual_layer_norm_hip);
  m.impl("segment_retrieve_fuse", grm::segment_retrieve_fuse_hip);
}

PYBIND11_MODULE(TORCH_EXTENSION_NAME, m) {
  m.doc() = "GRM hot-path ops for MI355X (gfx950): torch.ops.grm_cuda backed by libgrm_hip.so";
  m.attr("__grm_cuda_with_kernels__") = pybind11::bool_(true);
  m.attr("__grm_hip_arch__") = "gfx950";
  m.def("hip_launch_count", []() { return static_cast<uint64_t>(grm_hip_launch_count()); },
        "Kernels launched by libgrm_hip.so in this process");
  m.def("generic_path_calls", []() { return static_cast<int64_t>(grm::g_generic_calls.load()); },
        "CUDA-key calls that ran the generic ATen implementation");
  m.def("abi_version", []() { return grm_hip_abi_version(); });
}
