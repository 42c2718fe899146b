"""GRM hot-path op wrappers over the MI355X extension (torch.ops.grm_cuda).

Same public surface as the reference's ``grm.core.cuda_ops``
(reference grm/core/cuda_ops.py:405-413): lazy extension loading,
per-op ``auto/native/fallback`` policies read from the same environment
variables with the same precedence, the same runtime-status dictionary, the
same autograd wrappers and the same pure-PyTorch fallbacks (selected by
``debug_fallback=True`` or a ``fallback`` policy).

Differences, all deliberate:
  * On a GPU tensor the native path is mandatory: if the extension cannot be
    loaded the call raises instead of silently running PyTorch code.
  * ``auto`` runs the native apply-query kernel for rank-5 inputs too (the
    reference's auto policy sends rank 5 to einsum, cuda_ops.py:154-155).
  * New whole-sequence / routing / retrieval / fusion entry points:
    ``cuda_segment_scan``, ``cuda_topk_route``, ``cuda_gather_apply`` and
    ``cuda_fuse_residual``.
"""

from __future__ import annotations

import importlib
import math
import os
from typing import Any, Dict, Optional, Tuple

import torch
from torch import Tensor

_IMPORT_CANDIDATES = ("rnn_with_grm_amd.grm_cuda_ext", "grm_cuda_ext", "grm.grm_cuda_ext")
_REGISTERED_OPS = (
    "chunk_update_forward",
    "chunk_update_backward",
    "apply_query_forward",
    "apply_query_backward",
    "batched_memory_gather",
)
_EXTRA_OPS = ("segment_scan_forward", "topk_route", "fuse_residual", "gather_apply", "segment_route")

_EXTENSION_MODULE: Optional[Any] = None
_EXTENSION_LOAD_ATTEMPTED = False
_EXTENSION_LOAD_ERROR = ""
_KERNEL_POLICY_ENV = "GRM_CUDA_KERNEL_POLICY"
_KERNEL_POLICY_OP_ENVS = {
    "chunk_update": "GRM_CUDA_CHUNK_UPDATE_POLICY",
    "apply_query": "GRM_CUDA_APPLY_QUERY_POLICY",
    "batched_memory_gather": "GRM_CUDA_BATCHED_GATHER_POLICY",
}
_VALID_KERNEL_POLICIES = {"auto", "native", "fallback"}


class GrmExtensionUnavailable(RuntimeError):
    """The HIP extension is required for a GPU tensor but could not be loaded."""


def _has_registered_ops() -> bool:
    namespace = getattr(torch.ops, "grm_cuda", None)
    if namespace is None:
        return False
    return all(hasattr(namespace, name) for name in _REGISTERED_OPS)


def _has_dispatch_kernel(op_name: str, dispatch_key: str) -> bool:
    checker = getattr(torch._C, "_dispatch_has_kernel_for_dispatch_key", None)
    if checker is None:
        return False
    try:
        return bool(checker(f"grm_cuda::{op_name}", dispatch_key))
    except Exception:
        return False


def _get_dispatch_kernel_status() -> Dict[str, Dict[str, bool]]:
    return {
        name: {
            "cuda": _has_dispatch_kernel(name, "CUDA"),
            "composite_explicit_autograd": _has_dispatch_kernel(name, "CompositeExplicitAutograd"),
        }
        for name in _REGISTERED_OPS
    }


def load_grm_cuda_extension(force: bool = False) -> bool:
    """Import the extension once; ``force`` retries.  Mirrors cuda_ops.py:62-89."""
    global _EXTENSION_MODULE, _EXTENSION_LOAD_ATTEMPTED, _EXTENSION_LOAD_ERROR
    if _EXTENSION_MODULE is not None and not force:
        return True
    if _EXTENSION_LOAD_ATTEMPTED and not force:
        return False
    _EXTENSION_LOAD_ATTEMPTED = True
    _EXTENSION_MODULE = None
    _EXTENSION_LOAD_ERROR = ""
    errors = []
    for module_name in _IMPORT_CANDIDATES:
        try:
            module = importlib.import_module(module_name)
        except Exception as exc:  # import failure is recorded, as in the reference
            errors.append(f"{module_name}: {type(exc).__name__}: {exc}")
            continue
        if not _has_registered_ops():
            errors.append(f"{module_name}: torch.ops.grm_cuda registration missing")
            continue
        _EXTENSION_MODULE = module
        _EXTENSION_LOAD_ERROR = ""
        return True
    _EXTENSION_LOAD_ERROR = "; ".join(errors)
    return False


def is_grm_cpp_extension_available() -> bool:
    return load_grm_cuda_extension()


def is_grm_cuda_available() -> bool:
    if not load_grm_cuda_extension():
        return False
    status = _get_dispatch_kernel_status()
    return all(s["cuda"] for s in status.values()) and torch.cuda.is_available()


def _get_kernel_policy(op_name: str) -> str:
    for env_name in (_KERNEL_POLICY_OP_ENVS.get(op_name, ""), _KERNEL_POLICY_ENV):
        if not env_name:
            continue
        value = os.environ.get(env_name, "").strip().lower()
        if value and value in _VALID_KERNEL_POLICIES:
            return value
    return "auto"


def get_grm_cuda_runtime_status() -> Dict[str, Any]:
    """Same keys as the reference (cuda_ops.py:185-215), plus ``hip``."""
    extension_loaded = load_grm_cuda_extension()
    namespace = getattr(torch.ops, "grm_cuda", None)
    registered_ops = {name: bool(namespace and hasattr(namespace, name)) for name in _REGISTERED_OPS}
    compiled_with_cuda_sources = bool(
        getattr(_EXTENSION_MODULE, "__grm_cuda_with_kernels__", False) if _EXTENSION_MODULE is not None else False
    )
    dispatch_kernels = _get_dispatch_kernel_status() if extension_loaded else {
        name: {"cuda": False, "composite_explicit_autograd": False} for name in _REGISTERED_OPS
    }
    compiled_with_cuda_kernels = compiled_with_cuda_sources and all(s["cuda"] for s in dispatch_kernels.values())
    status: Dict[str, Any] = {
        "load_attempted": _EXTENSION_LOAD_ATTEMPTED,
        "extension_loaded": extension_loaded,
        "compiled_with_cuda_sources": compiled_with_cuda_sources,
        "compiled_with_cuda_kernels": compiled_with_cuda_kernels,
        "torch_cuda_available": torch.cuda.is_available(),
        "cuda_backend_available": compiled_with_cuda_kernels and torch.cuda.is_available(),
        "load_error": _EXTENSION_LOAD_ERROR,
        "module_name": getattr(_EXTENSION_MODULE, "__name__", "") if _EXTENSION_MODULE is not None else "",
        "registered_ops": registered_ops,
        "dispatch_kernels": dispatch_kernels,
        "kernel_policy": {
            "global": _get_kernel_policy(""),
            "chunk_update": _get_kernel_policy("chunk_update"),
            "apply_query": _get_kernel_policy("apply_query"),
            "batched_memory_gather": _get_kernel_policy("batched_memory_gather"),
        },
    }
    if _EXTENSION_MODULE is not None:
        status["hip"] = {
            "arch": getattr(_EXTENSION_MODULE, "__grm_hip_arch__", ""),
            "launch_count": int(_EXTENSION_MODULE.hip_launch_count()),
            "generic_path_calls": int(_EXTENSION_MODULE.generic_path_calls()),
            "extra_ops": {name: bool(namespace and hasattr(namespace, name)) for name in _EXTRA_OPS},
        }
    return status


def _require_extension(device: torch.device) -> bool:
    """True when the native op should run.  On a GPU the extension is
    mandatory; on CPU its absence falls back like the reference."""
    if load_grm_cuda_extension():
        return True
    if device.type == "cuda":
        raise GrmExtensionUnavailable(
            "GRM HIP extension (grm_cuda_ext / libgrm_hip.so) is not loaded; build it with "
            f"`python -m rnn_with_grm_amd.build`. Load error: {_EXTENSION_LOAD_ERROR}"
        )
    return False


def _use_native(op_name: str, device: torch.device, *, enabled: bool, debug_fallback: bool,
                auto_on_cpu: bool = False) -> bool:
    if not enabled or debug_fallback:
        return False
    policy = _get_kernel_policy(op_name)
    if policy == "fallback":
        return False
    if not _require_extension(device):
        return False
    if policy == "native":
        return True
    return device.type == "cuda" or auto_on_cpu


# ---------------------------------------------------------------------------
# Pure-PyTorch fallbacks (same maths as cuda_ops.py:218-284).

def _vectorized_chunk_update(keys: Tensor, values: Tensor, queries: Tensor, memory: Tensor,
                             memory_decay: float) -> Tuple[Tensor, Tensor]:
    batch, length, key_dim = keys.shape
    if length == 0:
        return values.new_zeros(batch, 0, values.size(-1)), memory
    lam = torch.as_tensor(memory_decay, device=memory.device, dtype=memory.dtype)
    pos = torch.arange(length, device=memory.device, dtype=memory.dtype)
    inv_sqrt = 1.0 / math.sqrt(float(key_dim))
    carried = torch.matmul(queries, memory.transpose(1, 2)) * torch.pow(lam, pos + 1.0).view(1, length, 1)
    gap = pos.view(-1, 1) - pos.view(1, -1)
    decay_tri = torch.pow(lam, gap.clamp_min(0)) * (gap >= 0).to(memory.dtype)
    attn = torch.matmul(queries, keys.transpose(1, 2)) * inv_sqrt * decay_tri
    hidden = carried + (1.0 - lam) * torch.matmul(attn, values)
    tail = (1.0 - lam) * torch.pow(lam, (length - 1) - pos) * inv_sqrt
    delta = torch.matmul((values * tail.view(1, length, 1)).transpose(1, 2), keys)
    memory_out = torch.pow(lam, torch.tensor(float(length), device=memory.device, dtype=memory.dtype)) * memory + delta
    return hidden, memory_out


def _fallback_apply_query(memories: Tensor, queries: Tensor) -> Tensor:
    if memories.ndim == 5:
        return torch.einsum("bqrhk,bqk->bqrh", memories, queries)
    if memories.ndim == 4:
        return torch.einsum("brhk,bk->brh", memories, queries)
    raise ValueError(f"Unsupported memory rank for apply-query: {memories.ndim}")


def _fallback_batched_memory_gather(memories_per_batch: Tensor, topk_indices: Tensor) -> Tensor:
    if memories_per_batch.ndim != 4:
        raise ValueError(f"Expected memories_per_batch rank 4, got {memories_per_batch.ndim}")
    if topk_indices.ndim not in (2, 3):
        raise ValueError(f"Expected topk_indices rank 2 or 3, got {topk_indices.ndim}")
    rows = [memories_per_batch[b].index_select(0, topk_indices[b].reshape(-1))
            for b in range(memories_per_batch.size(0))]
    shape = (memories_per_batch.size(0), *topk_indices.shape[1:], *memories_per_batch.shape[2:])
    if not rows:
        return memories_per_batch.new_empty(shape)
    return torch.stack(rows, 0).reshape(shape).contiguous()


# ---------------------------------------------------------------------------
# Autograd wrappers.

class ChunkUpdateCudaFn(torch.autograd.Function):
    """Native forward/backward (cuda_ops.py:287-321); grads come back in the
    dtype of the tensor they belong to."""

    @staticmethod
    def forward(ctx, keys: Tensor, values: Tensor, queries: Tensor, memory: Tensor, memory_decay: float):
        hidden, memory_out, aux = torch.ops.grm_cuda.chunk_update_forward(keys, values, queries, memory,
                                                                            float(memory_decay))
        ctx.memory_decay = float(memory_decay)
        ctx.save_for_backward(keys, values, queries, memory, aux)
        return hidden, memory_out

    @staticmethod
    def backward(ctx, grad_hidden: Tensor, grad_memory_out: Tensor):
        keys, values, queries, memory, aux = ctx.saved_tensors
        if grad_hidden is None:
            grad_hidden = torch.zeros((keys.size(0), keys.size(1), values.size(2)), dtype=values.dtype,
                                      device=values.device)
        if grad_memory_out is None:
            grad_memory_out = torch.zeros_like(memory)
        gk, gv, gq, gm = torch.ops.grm_cuda.chunk_update_backward(
            grad_hidden.to(values.dtype).contiguous(), grad_memory_out.to(memory.dtype).contiguous(),
            keys, values, queries, memory, aux, float(ctx.memory_decay))
        return gk, gv, gq, gm, None


class SegmentScanCudaFn(torch.autograd.Function):
    """Whole-sequence scan with per-segment snapshots; snapshots carry no gradient."""

    @staticmethod
    def forward(ctx, keys, values, queries, memory, memory_decay: float, segment_len: int):
        hidden, memory_out, snapshots = torch.ops.grm_cuda.segment_scan_forward(
            keys, values, queries, memory, float(memory_decay), int(segment_len))
        ctx.memory_decay = float(memory_decay)
        ctx.save_for_backward(keys, values, queries, memory)
        ctx.mark_non_differentiable(snapshots)
        return hidden, memory_out, snapshots

    @staticmethod
    def backward(ctx, grad_hidden, grad_memory_out, _grad_snapshots):
        keys, values, queries, memory = ctx.saved_tensors
        if grad_hidden is None:
            grad_hidden = torch.zeros((keys.size(0), keys.size(1), values.size(2)), dtype=values.dtype,
                                      device=values.device)
        if grad_memory_out is None:
            grad_memory_out = torch.zeros_like(memory)
        aux = memory.new_empty(0)
        gk, gv, gq, gm = torch.ops.grm_cuda.chunk_update_backward(
            grad_hidden.to(values.dtype).contiguous(), grad_memory_out.to(memory.dtype).contiguous(),
            keys, values, queries, memory, aux, float(ctx.memory_decay))
        return gk, gv, gq, gm, None, None


class ApplyQueryCudaFn(torch.autograd.Function):
    @staticmethod
    def forward(ctx, memories: Tensor, queries: Tensor):
        hidden = torch.ops.grm_cuda.apply_query_forward(memories, queries)
        ctx.save_for_backward(memories, queries)
        return hidden

    @staticmethod
    def backward(ctx, grad_hidden: Tensor):
        memories, queries = ctx.saved_tensors
        grad_memories, grad_queries = torch.ops.grm_cuda.apply_query_backward(
            grad_hidden.to(memories.dtype).contiguous(), memories, queries)
        return grad_memories, grad_queries


# ---------------------------------------------------------------------------
# Entry points (cuda_ops.py:347-402 and the new ones).

def cuda_chunk_update(keys: Tensor, values: Tensor, queries: Tensor, memory: Tensor, memory_decay: float, *,
                      enabled: bool = True, debug_fallback: bool = False) -> Tuple[Tensor, Tensor]:
    if _use_native("chunk_update", memory.device, enabled=enabled, debug_fallback=debug_fallback):
        return ChunkUpdateCudaFn.apply(keys, values, queries, memory, float(memory_decay))
    return _vectorized_chunk_update(keys, values, queries, memory, memory_decay)


def cuda_apply_query(memories: Tensor, queries: Tensor, *, enabled: bool = True,
                     debug_fallback: bool = False) -> Tensor:
    if _use_native("apply_query", memories.device, enabled=enabled, debug_fallback=debug_fallback):
        return ApplyQueryCudaFn.apply(memories, queries)
    return _fallback_apply_query(memories, queries)


def cuda_batched_memory_gather(memories_per_batch: Tensor, topk_indices: Tensor, *, enabled: bool = True,
                               debug_fallback: bool = False) -> Tensor:
    # The reference's auto policy uses the extension on CPU too (cuda_ops.py:158-174).
    if _use_native("batched_memory_gather", memories_per_batch.device, enabled=enabled,
                   debug_fallback=debug_fallback, auto_on_cpu=True):
        return torch.ops.grm_cuda.batched_memory_gather(memories_per_batch, topk_indices)
    return _fallback_batched_memory_gather(memories_per_batch, topk_indices)


def cuda_segment_scan(keys: Tensor, values: Tensor, queries: Tensor, memory: Tensor, memory_decay: float,
                      segment_len: int, *, enabled: bool = True,
                      debug_fallback: bool = False) -> Tuple[Tensor, Tensor, Tensor]:
    """Whole sequence in one call.  Returns (hidden [B,T,H], memory_out [B,H,K],
    snapshots float32 [B, ceil(T/segment_len), H, K] = state after each segment)."""
    if _use_native("chunk_update", memory.device, enabled=enabled, debug_fallback=debug_fallback):
        return SegmentScanCudaFn.apply(keys, values, queries, memory, float(memory_decay), int(segment_len))
    outs, snaps = [], []
    state = memory
    for t0 in range(0, keys.size(1), segment_len):
        sl = slice(t0, t0 + segment_len)
        h, state = _vectorized_chunk_update(keys[:, sl], values[:, sl], queries[:, sl], state, memory_decay)
        outs.append(h)
        snaps.append(state.float())
    hidden = torch.cat(outs, 1) if outs else values.new_zeros(values.size(0), 0, values.size(2))
    snapshots = torch.stack(snaps, 1) if snaps else memory.new_zeros(memory.size(0), 0, *memory.shape[1:]).float()
    return hidden, state, snapshots


def cuda_topk_route(queries: Tensor, keys: Tensor, top_k: int, scale: float, temperature: float = 1.0, *,
                    enabled: bool = True, debug_fallback: bool = False) -> Tuple[Tensor, Tensor, Tensor]:
    """Score -> top-k -> softmax (paper_grm.py:566-589).  Returns (gates, indices, scores).
    Native scores are one float32 FMA chain per score; ties go to the lower index."""
    if _use_native("topk_route", queries.device, enabled=enabled, debug_fallback=debug_fallback,
                   auto_on_cpu=True):
        return torch.ops.grm_cuda.topk_route(queries, keys, int(top_k), float(scale), float(temperature))
    scores = torch.matmul(queries, keys.transpose(1, 2)) * scale
    k = min(top_k, keys.size(1))
    if k < keys.size(1):
        top, idx = torch.topk(scores, k=k, dim=-1)
    else:
        top = scores
        idx = torch.arange(keys.size(1), device=queries.device).view(1, 1, -1).expand(
            queries.size(0), queries.size(1), -1)
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
    if _use_native("topk_route", queries.device, enabled=enabled, debug_fallback=debug_fallback,
                   auto_on_cpu=True):
        return torch.ops.grm_cuda.segment_route(queries, keys, int(top_k), int(segment_len), int(base),
                                                int(capacity), float(scale), float(temperature))
    B, Q, _ = queries.shape
    gates = queries.new_zeros((B, Q, top_k), dtype=torch.float32)
    idx = torch.full((B, Q, top_k), -1, dtype=torch.long, device=queries.device)
    scores = torch.full((B, Q, top_k), float("-inf"), dtype=torch.float32, device=queries.device)
    for t0 in range(0, Q, segment_len):
        hi = min(keys.size(1), base + t0 // segment_len)
        lo = max(0, hi - capacity)
        if hi <= lo:
            continue
        sl = slice(t0, t0 + segment_len)
        g, i, sc = cuda_topk_route(queries[:, sl], keys[:, lo:hi], top_k, scale, temperature, enabled=False)
        n = g.size(-1)
        gates[:, sl, :n] = g.float()
        idx[:, sl, :n] = i + lo
        scores[:, sl, :n] = sc.float()
    return gates, idx, scores


def cuda_fuse_residual(h_online: Tensor, retrieved: Tensor, gates: Tensor, weight: Optional[Tensor] = None,
                       bias: Optional[Tensor] = None, eps: float = 1e-5, *, enabled: bool = True,
                       debug_fallback: bool = False) -> Tensor:
    """LayerNorm(h + sum_r g_r r_r) (aggregator.py:67-145, residual mode); no LN when weight is None."""
    if _use_native("fuse_residual", h_online.device, enabled=enabled, debug_fallback=debug_fallback):
        return torch.ops.grm_cuda.fuse_residual(h_online, retrieved, gates, weight, bias, float(eps))
    x = h_online
    if retrieved.size(1) > 0:
        x = x + (retrieved * gates.to(retrieved.dtype).unsqueeze(-1)).sum(1)
    if weight is not None:
        x = torch.nn.functional.layer_norm(x, (h_online.size(-1),), weight, bias, eps)
    return x


def cuda_gather_apply(memories_per_batch: Tensor, topk_indices: Tensor, queries: Tensor,
                      dtype: Optional[torch.dtype] = None, *, enabled: bool = True,
                      debug_fallback: bool = False) -> Tensor:
    """apply_query(batched_memory_gather(M, idx).to(dtype), q.to(dtype)) without materialising
    the gathered states (cuda_ops.py:370-402, composed as in paper_grm.py:227-229,301-313).
    ``dtype`` is M's dtype by default; float32 widens 16-bit archives as the retriever does.
    The fused op has no backward: when autograd needs gradients the composition runs."""
    needs_grad = torch.is_grad_enabled() and (memories_per_batch.requires_grad or queries.requires_grad)
    if not needs_grad and _use_native("gather_apply", memories_per_batch.device, enabled=enabled,
                                      debug_fallback=debug_fallback):
        return torch.ops.grm_cuda.gather_apply(memories_per_batch, topk_indices, queries, dtype)
    gathered = cuda_batched_memory_gather(memories_per_batch, topk_indices, enabled=enabled,
                                          debug_fallback=debug_fallback)
    if dtype is not None:
        gathered = gathered.to(dtype)
    return cuda_apply_query(gathered, queries.to(gathered.dtype), enabled=enabled, debug_fallback=debug_fallback)


__all__ = [
    "GrmExtensionUnavailable",
    "cuda_apply_query",
    "cuda_batched_memory_gather",
    "cuda_chunk_update",
    "cuda_fuse_residual",
    "cuda_gather_apply",
    "cuda_segment_route",
    "cuda_segment_scan",
    "cuda_topk_route",
    "get_grm_cuda_runtime_status",
    "is_grm_cpp_extension_available",
    "is_grm_cuda_available",
    "load_grm_cuda_extension",
]
