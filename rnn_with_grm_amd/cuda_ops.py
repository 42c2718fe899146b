"""GRM hot-path op wrappers over the MI355X extension (torch.ops.grm_cuda).

Public surface of the reference's ``grm.core.cuda_ops`` (reference
grm/core/cuda_ops.py:405-413): the lazily loaded op library, per-op
``auto/native/fallback`` policies read from the same environment variables
with the same precedence, the runtime-status dictionary with the same keys,
autograd wrappers, and PyTorch fallbacks (``debug_fallback=True`` or a
``fallback`` policy) with the same error messages.

Deliberate differences:
  * On a GPU tensor the native path is mandatory: if the extension cannot be
    loaded the call raises instead of running PyTorch code.
  * ``auto`` runs the native apply-query kernel for rank-5 inputs too (the
    reference's auto policy sends rank 5 to einsum, cuda_ops.py:154-155).
  * Under autograd, the forward scan also returns the state after every
    64-token chunk as ``aux``; the backward reads it instead of re-running the
    scan (the schema allows it, bindings.cpp:6-7; the reference's aux is empty).
  * New entry points: ``cuda_segment_scan``, ``cuda_topk_route``,
    ``cuda_segment_route``, ``cuda_gather_apply`` and ``cuda_fuse_residual``.
"""

from __future__ import annotations

import importlib
import math
import os
from typing import Any, Dict, Optional, Tuple

import torch
from torch import Tensor

# The reference's five op schemas (bindings.cpp:6-10) and this library's additions.
SCHEMA_OPS = (
    "chunk_update_forward",
    "chunk_update_backward",
    "apply_query_forward",
    "apply_query_backward",
    "batched_memory_gather",
)
EXTRA_OPS = ("segment_scan_forward", "topk_route", "fuse_residual", "gather_apply", "segment_route",
             "retrieve_fuse", "project_split", "residual_layer_norm", "gather_apply_backward_queries",
             "gather_apply_backward_tokens", "apply_query_backward_queries", "archive_cast", "project_gemm",
             "linear_residual_layer_norm", "segment_retrieve_fuse")

# Environment variables of the reference (cuda_ops.py:26-32): one per op and a global one.
GLOBAL_POLICY_ENV = "GRM_CUDA_KERNEL_POLICY"
OP_POLICY_ENV = {
    "chunk_update": "GRM_CUDA_CHUNK_UPDATE_POLICY",
    "apply_query": "GRM_CUDA_APPLY_QUERY_POLICY",
    "batched_memory_gather": "GRM_CUDA_BATCHED_GATHER_POLICY",
}
POLICIES = ("auto", "native", "fallback")

# Chunk length of the backward's state checkpoints (BCT in csrc/chunk_bwd.hip).
_STATE_CHUNK = 64


class GrmExtensionUnavailable(RuntimeError):
    """The HIP extension is required for a GPU tensor but could not be loaded."""


class _OpLibrary:
    """The compiled op library, imported on first use.  A failed import is not
    retried unless forced, and its reasons are kept for the status report."""

    module_names = ("rnn_with_grm_amd.grm_cuda_ext", "grm_cuda_ext", "grm.grm_cuda_ext")

    def __init__(self) -> None:
        self.module: Optional[Any] = None
        self.attempted = False
        self.error = ""

    @staticmethod
    def namespace():
        return getattr(torch.ops, "grm_cuda", None)

    def schemas_present(self) -> bool:
        ns = self.namespace()
        return ns is not None and all(hasattr(ns, op) for op in SCHEMA_OPS)

    def load(self, force: bool = False) -> bool:
        if self.module is not None and not force:
            return True
        if self.attempted and not force:
            return False
        self.attempted, self.module, self.error = True, None, ""
        reasons = []
        for name in self.module_names:
            try:
                candidate = importlib.import_module(name)
            except Exception as exc:  # recorded, reported by the status dictionary
                reasons.append(f"{name}: {type(exc).__name__}: {exc}")
                continue
            if self.schemas_present():
                self.module = candidate
                return True
            reasons.append(f"{name}: torch.ops.grm_cuda registration missing")
        self.error = "; ".join(reasons)
        return False

    @staticmethod
    def has_kernel(op: str, key: str) -> bool:
        probe = getattr(torch._C, "_dispatch_has_kernel_for_dispatch_key", None)
        if probe is None:
            return False
        try:
            return bool(probe(f"grm_cuda::{op}", key))
        except Exception:
            return False

    def kernel_table(self) -> Dict[str, Dict[str, bool]]:
        return {op: {"cuda": self.has_kernel(op, "CUDA"),
                     "composite_explicit_autograd": self.has_kernel(op, "CompositeExplicitAutograd")}
                for op in SCHEMA_OPS}


_LIB = _OpLibrary()


def extension_module() -> Optional[Any]:
    """The loaded op-library module (None before a successful load)."""
    return _LIB.module


def extension_load_error() -> str:
    """Why the last load attempt failed ('' after a success)."""
    return _LIB.error


def load_grm_cuda_extension(force: bool = False) -> bool:
    """Import the op library once (``force`` tries again); True when its ops are registered."""
    return _LIB.load(force)


def is_grm_cpp_extension_available() -> bool:
    return _LIB.load()


def is_grm_cuda_available() -> bool:
    if not _LIB.load():
        return False
    return torch.cuda.is_available() and all(entry["cuda"] for entry in _LIB.kernel_table().values())


def kernel_policy(op_name: str) -> str:
    """The op's own variable wins over the global one; unset or unknown values are skipped."""
    for env in (OP_POLICY_ENV.get(op_name), GLOBAL_POLICY_ENV):
        value = os.environ.get(env, "").strip().lower() if env else ""
        if value in POLICIES:
            return value
    return "auto"


def get_grm_cuda_runtime_status() -> Dict[str, Any]:
    """The reference's status keys (cuda_ops.py:198-215), plus ``hip``."""
    loaded = _LIB.load()
    ns = _LIB.namespace()
    table = _LIB.kernel_table() if loaded else {op: {"cuda": False, "composite_explicit_autograd": False}
                                                for op in SCHEMA_OPS}
    with_sources = loaded and bool(getattr(_LIB.module, "__grm_cuda_with_kernels__", False))
    with_kernels = with_sources and all(entry["cuda"] for entry in table.values())
    gpu = torch.cuda.is_available()
    status: Dict[str, Any] = dict(
        load_attempted=_LIB.attempted,
        extension_loaded=loaded,
        compiled_with_cuda_sources=with_sources,
        compiled_with_cuda_kernels=with_kernels,
        torch_cuda_available=gpu,
        cuda_backend_available=with_kernels and gpu,
        load_error=_LIB.error,
        module_name=_LIB.module.__name__ if loaded else "",
        registered_ops={op: ns is not None and hasattr(ns, op) for op in SCHEMA_OPS},
        dispatch_kernels=table,
        kernel_policy={"global": kernel_policy(""), **{op: kernel_policy(op) for op in OP_POLICY_ENV}},
    )
    if loaded:
        status["hip"] = {
            "arch": getattr(_LIB.module, "__grm_hip_arch__", ""),
            "launch_count": int(_LIB.module.hip_launch_count()),
            "generic_path_calls": int(_LIB.module.generic_path_calls()),
            "extra_ops": {op: ns is not None and hasattr(ns, op) for op in EXTRA_OPS},
        }
    return status


def _native_required(device: torch.device) -> bool:
    """True when the op library is there.  A GPU tensor needs it; on the CPU its
    absence means the PyTorch path, as in the reference."""
    if _LIB.load():
        return True
    if device.type == "cuda":
        raise GrmExtensionUnavailable(
            "GRM HIP extension (grm_cuda_ext / libgrm_hip.so) is not loaded; build it with "
            f"`python -m rnn_with_grm_amd.build`. Load error: {_LIB.error}")
    return False


def _run_native(op_name: str, device: torch.device, *, enabled: bool, debug_fallback: bool,
                auto_on_cpu: bool = False) -> bool:
    """Which path a call takes: disabled or debug calls and a ``fallback`` policy take
    PyTorch; ``native`` takes the library; ``auto`` takes it on the GPU (and on the CPU
    where the reference's auto rule does)."""
    if debug_fallback or not enabled:
        return False
    policy = kernel_policy(op_name)
    if policy == "fallback" or not _native_required(device):
        return False
    return policy == "native" or device.type == "cuda" or auto_on_cpu


# ---------------------------------------------------------------------------
# PyTorch paths (the maths of the reference's fallbacks, cuda_ops.py:218-284).

def _decay_powers(decay: float, n: int, like: Tensor) -> Tensor:
    """decay ** [0, 1, ..., n] in like's dtype and device."""
    base = torch.full((n + 1,), float(decay), dtype=like.dtype, device=like.device)
    return base.pow(torch.arange(n + 1, dtype=like.dtype, device=like.device))


def _torch_chunk_update(keys: Tensor, values: Tensor, queries: Tensor, memory: Tensor,
                        memory_decay: float) -> Tuple[Tensor, Tensor]:
    """One chunk of L tokens from state M in closed form, c = (1 - decay) / sqrt(d_k):
    h_i = decay^(i+1) M q_i + c sum_{j<=i} decay^(i-j) (q_i . k_j) v_j,
    M'  = decay^L M + c sum_j decay^(L-1-j) v_j k_j^T."""
    B, L, K = keys.shape
    if L == 0:
        return values.new_zeros(B, 0, values.size(-1)), memory
    powers = _decay_powers(memory_decay, L, memory)
    c = (1.0 - float(memory_decay)) / math.sqrt(float(K))
    step = torch.arange(L, device=memory.device)
    lag = step.view(L, 1) - step.view(1, L)
    causal = torch.where(lag >= 0, powers[lag.clamp_min(0)], torch.zeros((), dtype=memory.dtype,
                                                                           device=memory.device))
    carried = torch.bmm(queries, memory.transpose(1, 2)) * powers[1:].view(1, L, 1)
    within = torch.bmm(torch.bmm(queries, keys.transpose(1, 2)) * causal, values) * c
    tail = powers[:L].flip(0) * c                                   # c decay^(L-1-j)
    memory_out = powers[L] * memory + torch.bmm((values * tail.view(1, L, 1)).transpose(1, 2), keys)
    return carried + within, memory_out


def _torch_apply_query(memories: Tensor, queries: Tensor) -> Tensor:
    if memories.ndim == 5:                      # [B, Q, R, H, K] x [B, Q, K]
        return torch.matmul(memories, queries[:, :, None, :, None]).squeeze(-1)
    if memories.ndim == 4:                      # [B, R, H, K] x [B, K]
        return torch.matmul(memories, queries[:, None, :, None]).squeeze(-1)
    raise ValueError(f"Unsupported memory rank for apply-query: {memories.ndim}")


def _torch_batched_gather(memories_per_batch: Tensor, topk_indices: Tensor) -> Tensor:
    if memories_per_batch.ndim != 4:
        raise ValueError(f"Expected memories_per_batch rank 4, got {memories_per_batch.ndim}")
    if topk_indices.ndim not in (2, 3):
        raise ValueError(f"Expected topk_indices rank 2 or 3, got {topk_indices.ndim}")
    B, S = memories_per_batch.shape[:2]
    flat = topk_indices.reshape(B, -1).long()
    if flat.numel() and bool(((flat < 0) | (flat >= S)).any()):
        raise IndexError("index out of range in self")  # what index_select raises there
    rows = torch.arange(B, device=memories_per_batch.device).view(B, 1).expand_as(flat)
    picked = memories_per_batch[rows, flat]
    return picked.reshape(B, *topk_indices.shape[1:], *memories_per_batch.shape[2:]).contiguous()


# ---------------------------------------------------------------------------
# Autograd wrappers.

def _scan_grads(ctx, grad_hidden: Optional[Tensor], grad_memory_out: Optional[Tensor], chunk_states: Tensor):
    """chunk_update_backward with missing output gradients as zeros, each gradient cast
    to the dtype of its input (cuda_ops.py:304-309)."""
    keys, values, queries, memory = ctx.saved_tensors[:4]
    if grad_hidden is None:
        grad_hidden = values.new_zeros(keys.size(0), keys.size(1), values.size(2))
    if grad_memory_out is None:
        grad_memory_out = torch.zeros_like(memory)
    return torch.ops.grm_cuda.chunk_update_backward(
        grad_hidden.to(values.dtype).contiguous(), grad_memory_out.to(memory.dtype).contiguous(),
        keys, values, queries, memory, chunk_states, ctx.decay)


class _ChunkScanFn(torch.autograd.Function):
    """The fused scan.  When gradients are wanted, the forward also keeps the state
    after every 64-token chunk (the whole-sequence op with 64-token snapshots), and
    the backward reads those instead of scanning again."""

    @staticmethod
    def forward(ctx, keys: Tensor, values: Tensor, queries: Tensor, memory: Tensor, memory_decay: float):
        ctx.decay = float(memory_decay)
        if any(ctx.needs_input_grad[:4]):
            hidden, memory_out, states = torch.ops.grm_cuda.segment_scan_forward(
                keys, values, queries, memory, ctx.decay, _STATE_CHUNK)
            if memory_out.dtype != memory.dtype:
                memory_out = memory_out.to(memory.dtype)
        else:
            hidden, memory_out, states = torch.ops.grm_cuda.chunk_update_forward(
                keys, values, queries, memory, ctx.decay)
        ctx.save_for_backward(keys, values, queries, memory, states)
        return hidden, memory_out

    @staticmethod
    def backward(ctx, grad_hidden: Tensor, grad_memory_out: Tensor):
        return (*_scan_grads(ctx, grad_hidden, grad_memory_out, ctx.saved_tensors[4]), None)


class _SegmentScanFn(torch.autograd.Function):
    """Whole-sequence scan with per-segment snapshots; snapshots carry no gradient.
    With 64-token segments the snapshots are the backward's chunk states."""

    @staticmethod
    def forward(ctx, keys, values, queries, memory, memory_decay: float, segment_len: int):
        ctx.decay = float(memory_decay)
        hidden, memory_out, snapshots = torch.ops.grm_cuda.segment_scan_forward(
            keys, values, queries, memory, ctx.decay, int(segment_len))
        states = snapshots if int(segment_len) == _STATE_CHUNK else memory.new_empty(0)
        ctx.save_for_backward(keys, values, queries, memory, states)
        ctx.mark_non_differentiable(snapshots)
        return hidden, memory_out, snapshots

    @staticmethod
    def backward(ctx, grad_hidden, grad_memory_out, _grad_snapshots):
        return (*_scan_grads(ctx, grad_hidden, grad_memory_out, ctx.saved_tensors[4]), None, None)


class _ApplyQueryFn(torch.autograd.Function):
    """Native apply-query.  The backward forms grad_memories only when the memories
    need it (a retrieved archive never does)."""

    @staticmethod
    def forward(ctx, memories: Tensor, queries: Tensor):
        ctx.save_for_backward(memories, queries)
        return torch.ops.grm_cuda.apply_query_forward(memories, queries)

    @staticmethod
    def backward(ctx, grad_hidden: Tensor):
        memories, queries = ctx.saved_tensors
        grad_hidden = grad_hidden.to(memories.dtype).contiguous()
        if not ctx.needs_input_grad[0]:
            return None, torch.ops.grm_cuda.apply_query_backward_queries(grad_hidden, memories, queries)
        return torch.ops.grm_cuda.apply_query_backward(grad_hidden, memories, queries)


class _GatherApplyFn(torch.autograd.Function):
    """Native gather + apply with the queries' gradient from the transposed apply
    (sum_r M[idx_r]^T g_r): neither direction forms the gathered [.., R, d_v, d_k] states.
    The memories get no gradient (a detached archive)."""

    @staticmethod
    def forward(ctx, memories: Tensor, indices: Tensor, queries: Tensor, dtype):
        ctx.save_for_backward(memories, indices, queries)
        return torch.ops.grm_cuda.gather_apply(memories, indices, queries, dtype)

    @staticmethod
    def backward(ctx, grad_out: Tensor):
        memories, indices, queries = ctx.saved_tensors
        grad_q = None
        if ctx.needs_input_grad[2]:
            grad_q = torch.ops.grm_cuda.gather_apply_backward_queries(memories, indices, grad_out.contiguous(),
                                                                      queries)
        return None, None, grad_q, None


class _RetrieveFuseFn(torch.autograd.Function):
    """Training form of the fused retrieval, LN(h + sum_r g_r M[idx_r] q) with float32
    arithmetic (the retriever's gather + apply, paper_grm.py:227-229,301-313, then the
    aggregator's residual fusion, aggregator.py:67-145).  Forward: x = h + sum_r g_r rows_r
    in float32, then LayerNorm; only x ([B, Q, H] float32) and LayerNorm's mean and 1/std are
    kept, not the [B, Q, R, H] rows.  A 16-bit model (16-bit h and queries) takes x from
    retrieve_fuse without LayerNorm weights, whose rows are row-scaled float16 (rounding 2^-11
    of each row's largest value, as at inference); a float32 model takes the float32 rows of
    gather_apply and fuse_residual's weighted sum.  Backward: LayerNorm's gradient dx, then per pair
    u_r = M[idx_r]^T dx (gather_apply_backward_tokens, one dx row per query shared by its
    routes), dq = sum_r g_r u_r (fuse_residual again, on zero rows) and dg_r = u_r . q.  The
    memories get no gradient (a detached archive)."""

    @staticmethod
    def _weighted_sum(base: Tensor, rows: Tensor, gates: Tensor) -> Tensor:
        """base + sum_r gates_r rows_r for float32 [N, H] base, [N, R, H] rows, [N, R] gates."""
        if rows.size(-1) <= 2048:
            return torch.ops.grm_cuda.fuse_residual(base, rows, gates, None, None, 1e-5)
        return base + (rows * gates.unsqueeze(-1)).sum(1)

    @staticmethod
    def forward(ctx, memories: Tensor, indices: Tensor, queries: Tensor, gates: Tensor, h_online: Tensor,
                weight: Optional[Tensor], bias: Optional[Tensor], eps: float):
        B, Q, H = h_online.shape
        R = indices.size(-1)
        gf = gates.float().reshape(B * Q, R).contiguous()
        q16 = queries.dtype == torch.bfloat16 or (queries.dtype == torch.float16 and memories.dtype == torch.float16)
        if q16 and h_online.dtype in (torch.bfloat16, torch.float16):
            x = torch.ops.grm_cuda.retrieve_fuse(memories, indices, queries, gf.view(B, Q, R), h_online.float(),
                                                 None, None, eps)
        else:
            rows = torch.ops.grm_cuda.gather_apply(memories, indices, queries, torch.float32)  # [B, Q, R, H]
            x = _RetrieveFuseFn._weighted_sum(h_online.float().reshape(B * Q, H), rows.reshape(B * Q, R, H), gf)
            del rows
            x = x.reshape(B, Q, H)
        mean = rstd = None
        if weight is None:
            out = x
        else:
            out, mean, rstd = torch.native_layer_norm(x, (H,), weight.float(),
                                                      None if bias is None else bias.float(), eps)
        ctx.save_for_backward(memories, indices, queries, gf, x, mean, rstd, weight, bias)
        ctx.h_dtype = h_online.dtype
        ctx.gates_dtype = gates.dtype
        return out.to(h_online.dtype)

    @staticmethod
    def backward(ctx, grad_out: Tensor):
        memories, indices, queries, gf, x, mean, rstd, weight, bias = ctx.saved_tensors
        B, Q, H = x.shape
        R, K = gf.size(1), queries.size(-1)
        dw = db = None
        if weight is None:
            dx = grad_out.float()
        else:
            mask = [True, ctx.needs_input_grad[5], bias is not None and ctx.needs_input_grad[6]]
            dx, dwf, dbf = torch.ops.aten.native_layer_norm_backward(
                grad_out.float().contiguous(), x, (H,), mean, rstd, weight.float(),
                None if bias is None else bias.float(), mask)
            dw = None if dwf is None else dwf.to(weight.dtype)
            db = None if dbf is None else dbf.to(bias.dtype)
        dq = dg = dh = None
        if ctx.needs_input_grad[2] or ctx.needs_input_grad[3]:
            u = torch.ops.grm_cuda.gather_apply_backward_tokens(memories, indices, dx.contiguous())  # [B, Q, R, K]
            u = u.reshape(B * Q, R, K)
            if ctx.needs_input_grad[2]:
                dq = _RetrieveFuseFn._weighted_sum(u.new_zeros(B * Q, K), u, gf)
                dq = dq.reshape(queries.shape).to(queries.dtype)
            if ctx.needs_input_grad[3]:
                dg = (u * queries.float().reshape(B * Q, 1, K)).sum(-1)
                dg = dg.reshape(B, Q, R).to(ctx.gates_dtype)
        if ctx.needs_input_grad[4]:
            dh = dx.to(ctx.h_dtype)
        return None, None, dq, dg, dh, dw, db, None


# ---------------------------------------------------------------------------
# Entry points (the reference's cuda_ops.py:347-402, then this library's own).

def cuda_chunk_update(keys: Tensor, values: Tensor, queries: Tensor, memory: Tensor, memory_decay: float, *,
                      enabled: bool = True, debug_fallback: bool = False) -> Tuple[Tensor, Tensor]:
    if _run_native("chunk_update", memory.device, enabled=enabled, debug_fallback=debug_fallback):
        return _ChunkScanFn.apply(keys, values, queries, memory, float(memory_decay))
    return _torch_chunk_update(keys, values, queries, memory, memory_decay)


def cuda_apply_query(memories: Tensor, queries: Tensor, *, enabled: bool = True,
                     debug_fallback: bool = False) -> Tensor:
    if _run_native("apply_query", memories.device, enabled=enabled, debug_fallback=debug_fallback):
        return _ApplyQueryFn.apply(memories, queries)
    return _torch_apply_query(memories, queries)


def cuda_batched_memory_gather(memories_per_batch: Tensor, topk_indices: Tensor, *, enabled: bool = True,
                               debug_fallback: bool = False) -> Tensor:
    # The reference's auto rule uses the library on the CPU too (cuda_ops.py:158-174).
    if _run_native("batched_memory_gather", memories_per_batch.device, enabled=enabled,
                   debug_fallback=debug_fallback, auto_on_cpu=True):
        # The op has no backward (as the reference's native gather): the archive gets no
        # gradient, stated here by detaching rather than left to autograd's fallback.
        return torch.ops.grm_cuda.batched_memory_gather(memories_per_batch.detach(), topk_indices)
    return _torch_batched_gather(memories_per_batch, topk_indices)


def cuda_segment_scan(keys: Tensor, values: Tensor, queries: Tensor, memory: Tensor, memory_decay: float,
                      segment_len: int, *, enabled: bool = True,
                      debug_fallback: bool = False) -> Tuple[Tensor, Tensor, Tensor]:
    """Whole sequence in one call.  Returns (hidden [B,T,H], memory_out [B,H,K],
    snapshots float32 [B, ceil(T/segment_len), H, K] = state after each segment)."""
    if _run_native("chunk_update", memory.device, enabled=enabled, debug_fallback=debug_fallback):
        return _SegmentScanFn.apply(keys, values, queries, memory, float(memory_decay), int(segment_len))
    T = keys.size(1)
    hiddens, snapshots, state = [], [], memory
    for t0 in range(0, T, segment_len):
        part = slice(t0, t0 + segment_len)
        h, state = _torch_chunk_update(keys[:, part], values[:, part], queries[:, part], state, memory_decay)
        hiddens.append(h)
        snapshots.append(state.float())
    if not hiddens:
        return (values.new_zeros(values.size(0), 0, values.size(2)), memory,
                memory.new_zeros(memory.size(0), 0, *memory.shape[1:]).float())
    return torch.cat(hiddens, 1), state, torch.stack(snapshots, 1)


def cuda_topk_route(queries: Tensor, keys: Tensor, top_k: int, scale: float, temperature: float = 1.0, *,
                    enabled: bool = True, debug_fallback: bool = False) -> Tuple[Tensor, Tensor, Tensor]:
    """Score -> top-k -> softmax (paper_grm.py:566-589).  Returns (gates, indices, scores).
    Native scores are one float32 FMA chain per score; ties go to the lower index."""
    if _run_native("topk_route", queries.device, enabled=enabled, debug_fallback=debug_fallback,
                   auto_on_cpu=True):
        return torch.ops.grm_cuda.topk_route(queries, keys, int(top_k), float(scale), float(temperature))
    scores = torch.matmul(queries, keys.transpose(1, 2)) * scale
    S = keys.size(1)
    if min(top_k, S) < S:
        top, idx = torch.topk(scores, k=min(top_k, S), dim=-1)
    else:  # every key, in index order
        top = scores
        idx = torch.arange(S, device=queries.device).expand(queries.size(0), queries.size(1), S)
    return torch.softmax(top / temperature, dim=-1), idx, top


def cuda_segment_route(queries: Tensor, keys: Tensor, top_k: int, segment_len: int, base: int, capacity: int,
                       scale: float, temperature: float = 1.0, *, enabled: bool = True,
                       debug_fallback: bool = False) -> Tuple[Tensor, Tensor, Tensor]:
    """Routing of every segment of a sequence in one call, as the reference's
    segment loop routes each segment over the archive of the moment
    (paper_grm.py:702-728 -> _route_chunk, :566-589).  Query row t of segment
    s = t // segment_len sees keys [lo, hi), hi = base + s, lo = max(0, hi - capacity).
    Returns (gates, indices, scores), each [B, Q, top_k]; indices are absolute key
    positions, and a window of n <= top_k keys fills slots n.. with index -1,
    score -inf and gate 0."""
    native = _run_native("topk_route", queries.device, enabled=enabled, debug_fallback=debug_fallback,
                         auto_on_cpu=True)
    if native and top_k <= 128:
        return torch.ops.grm_cuda.segment_route(queries, keys, int(top_k), int(segment_len), int(base),
                                                int(capacity), float(scale), float(temperature))
    B, Q, _ = queries.shape
    gates = queries.new_zeros((B, Q, top_k), dtype=torch.float32)
    idx = torch.full((B, Q, top_k), -1, dtype=torch.long, device=queries.device)
    scores = torch.full((B, Q, top_k), float("-inf"), dtype=torch.float32, device=queries.device)
    for seg, t0 in enumerate(range(0, Q, segment_len)):
        hi = min(keys.size(1), base + seg)
        lo = max(0, hi - capacity)
        if hi > lo:
            rows = slice(t0, t0 + segment_len)
            # top_k beyond the one-launch kernel's 128: each window through topk_route's own op
            g, i, sc = cuda_topk_route(queries[:, rows], keys[:, lo:hi], top_k, scale, temperature, enabled=native)
            n = g.size(-1)
            gates[:, rows, :n], idx[:, rows, :n], scores[:, rows, :n] = g.float(), i + lo, sc.float()
    return gates, idx, scores


def cuda_fuse_residual(h_online: Tensor, retrieved: Tensor, gates: Tensor, weight: Optional[Tensor] = None,
                       bias: Optional[Tensor] = None, eps: float = 1e-5, *, enabled: bool = True,
                       debug_fallback: bool = False) -> Tensor:
    """LayerNorm(h + sum_r g_r r_r) (aggregator.py:67-145, residual mode); no LN when weight is None."""
    if _run_native("fuse_residual", h_online.device, enabled=enabled, debug_fallback=debug_fallback):
        return torch.ops.grm_cuda.fuse_residual(h_online, retrieved, gates, weight, bias, float(eps))
    x = h_online
    if retrieved.size(1) > 0:
        x = x + torch.einsum("nr,nrh->nh", gates.to(retrieved.dtype), retrieved)
    if weight is not None:
        x = torch.nn.functional.layer_norm(x, (h_online.size(-1),), weight, bias, eps)
    return x


def cuda_gather_apply(memories_per_batch: Tensor, topk_indices: Tensor, queries: Tensor,
                      dtype: Optional[torch.dtype] = None, *, enabled: bool = True,
                      debug_fallback: bool = False) -> Tensor:
    """apply_query(batched_memory_gather(M, idx).to(dtype), q.to(dtype)) without materialising
    the gathered states (cuda_ops.py:370-402, composed as in paper_grm.py:227-229,301-313).
    ``dtype`` is M's dtype by default; float32 widens 16-bit archives as the retriever does.
    Under autograd, when only the queries need a gradient (a detached archive, as in the
    models) the native op runs with the transposed apply as its backward; when the memories
    need one too, the composition runs."""
    needs_grad = torch.is_grad_enabled() and (memories_per_batch.requires_grad or queries.requires_grad)
    native = _run_native("gather_apply", memories_per_batch.device, enabled=enabled, debug_fallback=debug_fallback)
    if native and not needs_grad:
        return torch.ops.grm_cuda.gather_apply(memories_per_batch, topk_indices, queries, dtype)
    if native and not memories_per_batch.requires_grad:
        # only the queries need a gradient: the transposed apply gives it without the gathered states
        return _GatherApplyFn.apply(memories_per_batch, topk_indices, queries, dtype)
    gathered = cuda_batched_memory_gather(memories_per_batch, topk_indices, enabled=enabled,
                                          debug_fallback=debug_fallback)
    if dtype is not None:
        gathered = gathered.to(dtype)
    return cuda_apply_query(gathered, queries.to(gathered.dtype), enabled=enabled, debug_fallback=debug_fallback)


def cuda_retrieve_fuse(memories_per_batch: Tensor, topk_indices: Tensor, queries: Tensor, gates: Tensor,
                       h_online: Tensor, weight: Optional[Tensor] = None, bias: Optional[Tensor] = None,
                       eps: float = 1e-5, *, enabled: bool = True, debug_fallback: bool = False) -> Tensor:
    """LayerNorm(h + sum_r gates_r (M[idx_r] q)) for [B, Q] rows: the retriever's float32 gather +
    apply (paper_grm.py:227-229,301-313) followed by the aggregator's residual fusion
    (aggregator.py:67-145, paper_grm.py:604-611), without the [B, Q, R, H] retrieved rows.
    Without gradients the op keeps the per-route rows as row-scaled float16 in its workspace;
    under autograd (queries, gates, h or the LayerNorm parameters; a detached archive) the
    native _RetrieveFuseFn runs with float32 rows and keeps only [B, Q, H] for its backward.
    Memories that need a gradient take the torch composition."""
    needs_grad = torch.is_grad_enabled() and any(
        t is not None and t.requires_grad for t in (memories_per_batch, queries, gates, h_online, weight, bias))
    native = _run_native("retrieve_fuse", h_online.device, enabled=enabled, debug_fallback=debug_fallback)
    if native and not needs_grad:
        return torch.ops.grm_cuda.retrieve_fuse(memories_per_batch, topk_indices, queries, gates, h_online, weight,
                                                bias, float(eps))
    if native and not memories_per_batch.requires_grad and topk_indices.dim() == 3:
        return _RetrieveFuseFn.apply(memories_per_batch, topk_indices, queries, gates, h_online, weight, bias,
                                     float(eps))
    B, Q, H = h_online.shape
    R = topk_indices.size(-1)
    retrieved = cuda_gather_apply(memories_per_batch, topk_indices, queries, torch.float32, enabled=enabled,
                                  debug_fallback=debug_fallback)
    fused = cuda_fuse_residual(h_online.reshape(B * Q, H).float(), retrieved.reshape(B * Q, R, H),
                               gates.reshape(B * Q, R).float(), None if weight is None else weight.float(),
                               None if bias is None else bias.float(), eps, enabled=enabled,
                               debug_fallback=debug_fallback)
    return fused.reshape(B, Q, H).to(h_online.dtype)


def _segment_window_valid(indices: Tensor, segment_len: int, base: int, capacity: int) -> Tensor:
    """[B, Q, R] bool: the (query, route) pairs inside the query's routing window
    [max(0, hi - capacity), hi), hi = base + t // segment_len, and not repeating an
    earlier route of the same query."""
    Q, R = indices.shape[1], indices.shape[2]
    hi = (torch.arange(Q, device=indices.device) // segment_len + base).view(1, Q, 1)
    lo = (hi - capacity).clamp(min=0)
    valid = (indices >= lo) & (indices < hi)
    if R > 1:
        earlier = torch.ones(R, R, dtype=torch.bool, device=indices.device).tril(-1)
        valid = valid & ~((indices.unsqueeze(-1) == indices.unsqueeze(-2)) & earlier).any(-1)
    return valid


def cuda_segment_retrieve_fuse(memories_per_batch: Tensor, topk_indices: Tensor, queries: Tensor, gates: Tensor,
                               h_online: Tensor, weight: Optional[Tensor], bias: Optional[Tensor], eps: float,
                               segment_len: int, base: int, capacity: int, *, enabled: bool = True,
                               debug_fallback: bool = False) -> Tensor:
    """cuda_retrieve_fuse for the indices of segment routing (paper_grm.py:702-728 ->
    _route_chunk, :566-589): query t routes over the archive entries [lo(t), hi(t)),
    hi(t) = base + t // segment_len, lo(t) = max(0, hi(t) - capacity).  A negative index
    is an empty slot; an index outside the window or repeated within a query contributes
    nothing.  The native op sums each query's routes inside the kernel, one workgroup per
    block of queries walking the block's window, so no per-route rows are written.
    Inference only (no autograd)."""
    if _run_native("retrieve_fuse", h_online.device, enabled=enabled, debug_fallback=debug_fallback):
        return torch.ops.grm_cuda.segment_retrieve_fuse(memories_per_batch, topk_indices, queries, gates, h_online,
                                                        weight, bias, float(eps), int(segment_len), int(base),
                                                        int(capacity))
    B, Q, H = h_online.shape
    R = topk_indices.size(-1)
    valid = _segment_window_valid(topk_indices, segment_len, base, capacity)
    if memories_per_batch.size(1) == 0 or R == 0:
        retrieved = h_online.new_zeros(B, Q, R, H, dtype=torch.float32)
    else:
        retrieved = cuda_gather_apply(memories_per_batch, topk_indices.masked_fill(~valid, 0), queries, torch.float32,
                                      enabled=enabled, debug_fallback=debug_fallback)
        retrieved = retrieved.masked_fill(~valid.unsqueeze(-1), 0.0)
    fused = cuda_fuse_residual(h_online.reshape(B * Q, H).float(), retrieved.reshape(B * Q, R, H),
                               gates.float().masked_fill(~valid, 0.0).reshape(B * Q, R),
                               None if weight is None else weight.float(), None if bias is None else bias.float(),
                               eps, enabled=enabled, debug_fallback=debug_fallback)
    return fused.reshape(B, Q, H).to(h_online.dtype)


def cuda_archive_cast(states: Tensor, model_dtype: torch.dtype, storage_dtype: torch.dtype, *,
                      enabled: bool = True, debug_fallback: bool = False) -> Tensor:
    """float32 states as the archive stores them: rounded to the model dtype, then to the
    storage dtype (push() storing the model's state, paper_grm.py:139-140), in one pass."""
    if states.dtype == torch.float32 and _run_native("archive_cast", states.device, enabled=enabled,
                                                     debug_fallback=debug_fallback):
        return torch.ops.grm_cuda.archive_cast(states, model_dtype, storage_dtype)
    return states.to(model_dtype).to(storage_dtype)


def cuda_project_split(proj: Tensor, key_dim: int, value_dim: int, extra_dim: int = 0, eps: float = 1e-6, *,
                       enabled: bool = True, debug_fallback: bool = False) -> Tuple[Tensor, ...]:
    """(keys, values, queries[, extra]) of the concatenated projection rows, keys and queries
    F.normalize'd (paper_grm.py:491-493; the extra part is the gating query projection,
    paper_grm.py:570-574).  Inference only: under autograd the split views and
    F.normalize run."""
    if not (torch.is_grad_enabled() and proj.requires_grad) and _run_native(
            "project_split", proj.device, enabled=enabled, debug_fallback=debug_fallback):
        k, v, q, e = torch.ops.grm_cuda.project_split(proj, int(key_dim), int(value_dim), int(extra_dim), float(eps))
        return (k, v, q) + ((e,) if extra_dim else ())
    parts = proj.split([key_dim, value_dim, key_dim, extra_dim], dim=-1)
    k = torch.nn.functional.normalize(parts[0], p=2, dim=-1, eps=eps)
    q = torch.nn.functional.normalize(parts[2], p=2, dim=-1, eps=eps)
    return (k, parts[1], q) + ((parts[3],) if extra_dim else ())


class _ProjectGemmFn(torch.autograd.Function):
    """project_gemm under autograd: the fused GEMM + split + normalise forward; the backward
    takes the normalisation's gradient in float32 (dp = (dy - y (y . dy)) / ||p||, or dy / eps
    where the norm is clamped: F.normalize's derivative) from the key and query projections'
    norms, recomputed with two GEMMs of key_dim columns, then the GEMM's gradients on the
    library (dx = dP W, dW = dP^T x, db = sum dP)."""

    @staticmethod
    def forward(ctx, x, weight, bias, key_dim, value_dim, extra_dim, eps):
        k, v, q, e = torch.ops.grm_cuda.project_gemm(x, weight, bias, key_dim, value_dim, extra_dim, eps)
        ctx.save_for_backward(x, weight, bias)
        ctx.dims = (key_dim, value_dim, extra_dim, eps)
        return k, v, q, e

    @staticmethod
    def backward(ctx, dk, dv, dq, de):
        x, weight, bias = ctx.saved_tensors
        dkd, dvd, ded, eps = ctx.dims
        K = x.size(-1)
        x2 = x.reshape(-1, K)
        rows = x2.size(0)
        dt = x.dtype

        def grad_or_zeros(g, d):
            return torch.zeros(rows, d, dtype=dt, device=x.device) if g is None else g.reshape(rows, d)

        def normalize_grad(lo, g):
            p = torch.nn.functional.linear(x2, weight[lo:lo + dkd], None if bias is None else bias[lo:lo + dkd])
            p = p.float()
            norm = p.norm(dim=-1, keepdim=True)
            den = norm.clamp_min(eps)
            y = p / den
            gf = g.float()
            dp = torch.where(norm > eps, (gf - y * (y * gf).sum(-1, keepdim=True)) / den, gf / eps)
            return dp.to(dt)

        parts = [normalize_grad(0, grad_or_zeros(dk, dkd)), grad_or_zeros(dv, dvd),
                 normalize_grad(dkd + dvd, grad_or_zeros(dq, dkd))]
        if ded:
            parts.append(grad_or_zeros(de, ded))
        dP = torch.cat(parts, -1)
        dx = dW = db = None
        if ctx.needs_input_grad[0]:
            dx = (dP @ weight).reshape(x.shape)
        if ctx.needs_input_grad[1]:
            dW = dP.t() @ x2
        if bias is not None and ctx.needs_input_grad[2]:
            db = dP.sum(0)
        return dx, dW, db, None, None, None, None


def _project_gemm_fused(x: Tensor, weight: Tensor, bias: Optional[Tensor], key_dim: int, value_dim: int,
                        extra_dim: int) -> bool:
    """Shapes the fused projection kernel takes (the op runs the library GEMM otherwise)."""
    return (x.is_cuda and x.dtype in (torch.bfloat16, torch.float16) and weight.dtype == x.dtype
            and (bias is None or bias.dtype == x.dtype) and key_dim == 64 and value_dim % 64 == 0
            and extra_dim % 64 == 0 and x.size(-1) % 64 == 0 and x.size(-1) > 0)


def cuda_project_gemm(x: Tensor, weight: Tensor, bias: Optional[Tensor], key_dim: int, value_dim: int,
                      extra_dim: int = 0, eps: float = 1e-6, *, enabled: bool = True,
                      debug_fallback: bool = False) -> Tuple[Tensor, ...]:
    """cuda_project_split(F.linear(x, weight, bias), ...) as one op: the projection GEMM with the
    split and the keys' and queries' L2 normalisation as its epilogue (paper_grm.py:491-493,
    570-574).  Under autograd, 16-bit inputs take _ProjectGemmFn (the fused forward, a native
    backward on library GEMMs); other dtypes F.linear and cuda_project_split."""
    needs_grad = torch.is_grad_enabled() and any(
        t is not None and t.requires_grad for t in (x, weight, bias))
    if _run_native("project_gemm", x.device, enabled=enabled, debug_fallback=debug_fallback):
        if not needs_grad:
            k, v, q, e = torch.ops.grm_cuda.project_gemm(x, weight, bias, int(key_dim), int(value_dim),
                                                         int(extra_dim), float(eps))
            return (k, v, q) + ((e,) if extra_dim else ())
        if _project_gemm_fused(x, weight, bias, key_dim, value_dim, extra_dim):
            k, v, q, e = _ProjectGemmFn.apply(x, weight, bias, int(key_dim), int(value_dim), int(extra_dim),
                                              float(eps))
            return (k, v, q) + ((e,) if extra_dim else ())
    return cuda_project_split(torch.nn.functional.linear(x, weight, bias), key_dim, value_dim, extra_dim, eps,
                              enabled=enabled, debug_fallback=debug_fallback)


def cuda_residual_layer_norm(x: Tensor, residual: Tensor, weight: Optional[Tensor] = None,
                             bias: Optional[Tensor] = None, eps: float = 1e-5, *, enabled: bool = True,
                             debug_fallback: bool = False) -> Tensor:
    """layer_norm(x + residual) (multilayer_grm.py:92-97).  Inference only: under autograd
    the add and torch's layer_norm run."""
    needs_grad = torch.is_grad_enabled() and any(
        t is not None and t.requires_grad for t in (x, residual, weight, bias))
    if not needs_grad and _run_native("residual_layer_norm", x.device, enabled=enabled,
                                      debug_fallback=debug_fallback):
        return torch.ops.grm_cuda.residual_layer_norm(x, residual, weight, bias, float(eps))
    return torch.nn.functional.layer_norm(x + residual, (x.size(-1),), weight, bias, eps)


class _LinearResidualLayerNormFn(torch.autograd.Function):
    """linear_residual_layer_norm under autograd: the fused forward also writes the LayerNorm's
    input s = linear(x) + residual and its float32 row statistics; the backward is aten's
    native_layer_norm_backward on them (ds and the LayerNorm parameters' gradients), then
    ds flows to the residual unchanged and through the linear map on the library
    (dx = ds W, dW = ds^T x, db = sum ds)."""

    @staticmethod
    def forward(ctx, x, weight, bias, residual, ln_weight, ln_bias, eps):
        out, pre, mean, rstd = torch.ops.grm_cuda.linear_residual_layer_norm(x, weight, bias, residual, ln_weight,
                                                                            ln_bias, eps, True)
        ctx.save_for_backward(x, weight, pre, mean, rstd, ln_weight, ln_bias)
        ctx.has_bias = bias is not None
        return out

    @staticmethod
    def backward(ctx, dout):
        x, weight, pre, mean, rstd, ln_weight, ln_bias = ctx.saved_tensors
        N, K = weight.shape
        rows = pre.numel() // N
        mask = [True, ln_weight is not None and ctx.needs_input_grad[4],
                ln_bias is not None and ctx.needs_input_grad[5]]
        ds, dlw, dlb = torch.ops.aten.native_layer_norm_backward(
            dout.reshape(rows, N).contiguous(), pre.reshape(rows, N), [N], mean.view(rows, 1), rstd.view(rows, 1),
            ln_weight, ln_bias, mask)
        x2 = x.reshape(rows, K)
        dx = dW = db = dres = None
        if ctx.needs_input_grad[0]:
            dx = (ds @ weight).reshape(x.shape)
        if ctx.needs_input_grad[1]:
            dW = ds.t() @ x2
        if ctx.has_bias and ctx.needs_input_grad[2]:
            db = ds.sum(0)
        if ctx.needs_input_grad[3]:
            dres = ds.reshape(pre.shape)
        return dx, dW, db, dres, dlw if mask[1] else None, dlb if mask[2] else None, None


def _linear_res_ln_fused(x: Tensor, weight: Tensor, bias: Optional[Tensor], residual: Tensor) -> bool:
    N, K = weight.shape
    return (x.is_cuda and x.dtype in (torch.bfloat16, torch.float16) and weight.dtype == x.dtype
            and residual.dtype == x.dtype and (bias is None or bias.dtype == x.dtype) and K % 64 == 0 and K > 0
            and N % 64 == 0 and 0 < N <= 512)


def cuda_linear_residual_layer_norm(x: Tensor, weight: Tensor, bias: Optional[Tensor], residual: Tensor,
                                    ln_weight: Optional[Tensor] = None, ln_bias: Optional[Tensor] = None,
                                    eps: float = 1e-5, *, enabled: bool = True,
                                    debug_fallback: bool = False) -> Tensor:
    """layer_norm(F.linear(x, weight, bias) + residual): the model's output projection
    (paper_grm.py:709) and the block output (multilayer_grm.py:92-97) as one GEMM whose epilogue
    is the residual add and the LayerNorm.  Under autograd, 16-bit inputs take
    _LinearResidualLayerNormFn; other dtypes the torch composition."""
    needs_grad = torch.is_grad_enabled() and any(
        t is not None and t.requires_grad for t in (x, weight, bias, residual, ln_weight, ln_bias))
    if _run_native("linear_residual_layer_norm", x.device, enabled=enabled, debug_fallback=debug_fallback):
        if not needs_grad:
            return torch.ops.grm_cuda.linear_residual_layer_norm(x, weight, bias, residual, ln_weight, ln_bias,
                                                                 float(eps), False)[0]
        if _linear_res_ln_fused(x, weight, bias, residual):
            return _LinearResidualLayerNormFn.apply(x, weight, bias, residual, ln_weight, ln_bias, float(eps))
    y = torch.nn.functional.linear(x, weight, bias)
    return torch.nn.functional.layer_norm(y + residual, (y.size(-1),), ln_weight, ln_bias, eps)


__all__ = [
    "GrmExtensionUnavailable",
    "cuda_apply_query",
    "cuda_batched_memory_gather",
    "cuda_chunk_update",
    "cuda_fuse_residual",
    "cuda_gather_apply",
    "cuda_linear_residual_layer_norm",
    "cuda_project_gemm",
    "cuda_project_split",
    "cuda_residual_layer_norm",
    "cuda_retrieve_fuse",
    "cuda_segment_retrieve_fuse",
    "cuda_segment_route",
    "cuda_segment_scan",
    "cuda_topk_route",
    "extension_load_error",
    "extension_module",
    "get_grm_cuda_runtime_status",
    "is_grm_cpp_extension_available",
    "is_grm_cuda_available",
    "kernel_policy",
    "load_grm_cuda_extension",
]
