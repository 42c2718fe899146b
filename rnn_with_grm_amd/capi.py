"""ctypes binding of libgrm_hip.so (the C ABI declared in include/grm_hip.h).

This is what a non-torch host (or the reference's own FFI) binds.  The helpers
below take torch tensors only to read their device pointers and the current
HIP stream; the library itself sees raw pointers and sizes.  torch is
imported before the library is loaded so both share one HIP runtime.
"""

from __future__ import annotations

import ctypes
from pathlib import Path
from typing import Optional

import torch

LIB_PATH = Path(__file__).resolve().parent / "libgrm_hip.so"

F32, F16, BF16 = 0, 1, 2
OK, EINVAL, EUNSUPPORTED = 0, -1, -2

_P = ctypes.c_void_p
_I = ctypes.c_int64
_C = ctypes.c_int

# name -> (restype, argtypes); must match include/grm_hip.h
SIGNATURES = {
    "grm_hip_abi_version": (ctypes.c_int, []),
    "grm_hip_last_error": (ctypes.c_char_p, []),
    "grm_hip_launch_count": (ctypes.c_uint64, []),
    "grm_hip_chunk_update_fwd": (_C, [_P, _P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _C, _C, ctypes.c_double,
                                      _I, _P]),
    "grm_hip_chunk_update_fwd_workspace": (_I, [_I, _I, _I, _I, _I]),
    "grm_hip_chunk_update_fwd_noalloc_limit": (_I, []),
    "grm_hip_chunk_update_fwd_noalloc": (_C, [_P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _C, _C, ctypes.c_double,
                                              _I, _P]),
    "grm_hip_chunk_update_bwd": (_C, [_P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _C, _P, _I, _I, _I, _I, _C, _C,
                                      ctypes.c_double, _P]),
    "grm_hip_apply_query_fwd": (_C, [_P, _P, _P, _I, _I, _I, _I, _I, _C, _P]),
    "grm_hip_apply_query_bwd": (_C, [_P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _C, _P]),
    "grm_hip_batched_gather": (_C, [_P, _P, _P, _I, _I, _I, _I, _C, _P, _P]),
    "grm_hip_gather_apply_workspace": (_I, [_I, _I, _I]),
    "grm_hip_gather_apply": (_C, [_P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _I, _C, _C, _C, _P, _P]),
    "grm_hip_retrieve_fuse_workspace": (_I, [_I, _I, _I, _I]),
    "grm_hip_gather_apply_bwd_queries": (_C, [_P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _I, _C, _P, _P]),
    "grm_hip_gather_apply_bwd_tokens": (_C, [_P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _I, _C, _P, _P]),
    "grm_hip_project_split": (_C, [_P, _P, _P, _P, _P, _I, _I, _I, _I, _C, ctypes.c_float, _P]),
    "grm_hip_residual_layer_norm": (_C, [_P, _P, _P, _P, _P, _I, _I, _C, _C, ctypes.c_float, _P]),
    "grm_hip_archive_cast": (_C, [_P, _P, _I, _C, _C, _P]),
    "grm_hip_project_gemm": (_C, [_P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _C, ctypes.c_float, _P]),
    "grm_hip_linear_residual_layer_norm": (_C, [_P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _C, _C,
                                                ctypes.c_float, _P]),
    "grm_hip_retrieve_fuse": (_C, [_P, _P, _P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _I, _C, _C, _C,
                                   ctypes.c_float, _P, _P]),
    "grm_hip_segment_retrieve_fuse_workspace": (_I, [_I, _I, _I, _I, _I, _I, _I, _C]),
    "grm_hip_segment_retrieve_fuse": (_C, [_P, _P, _P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _I, _I, _I,
                                           _I, _C, _C, _C, ctypes.c_float, _P, _P]),
    "grm_hip_topk_route": (_C, [_P, _P, _P, _P, _P, _I, _I, _I, _I, _C, _I, ctypes.c_float, ctypes.c_float, _P]),
    "grm_hip_segment_route": (_C, [_P, _P, _P, _P, _P, _I, _I, _I, _I, _C, _I, _I, _I, _I, ctypes.c_float,
                                   ctypes.c_float, _P]),
    "grm_hip_fuse_residual": (_C, [_P, _P, _P, _P, _P, _P, _I, _I, _I, _C, ctypes.c_float, _P]),
}

_lib: Optional[ctypes.CDLL] = None


def load(path: Optional[Path] = None) -> ctypes.CDLL:
    """Load libgrm_hip.so and declare every exported signature.  Raises if the
    library or a symbol is missing."""
    global _lib
    if _lib is not None and path is None:
        return _lib
    p = Path(path) if path else LIB_PATH
    if not p.exists():
        raise FileNotFoundError(f"{p} not built; run `python -m rnn_with_grm_amd.build`")
    lib = ctypes.CDLL(str(p))
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    if path is None:
        _lib = lib
    return lib


def dtype_code(dtype: torch.dtype) -> int:
    return {torch.float32: F32, torch.float16: F16, torch.bfloat16: BF16}[dtype]


def last_error() -> str:
    return (load().grm_hip_last_error() or b"").decode()


def launch_count() -> int:
    return int(load().grm_hip_launch_count())


def _ptr(t: Optional[torch.Tensor]):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def _stream(t: torch.Tensor):
    return ctypes.c_void_p(torch.cuda.current_stream(t.device).cuda_stream)


def _check(rc: int, what: str) -> None:
    if rc != OK:
        raise RuntimeError(f"{what} failed ({rc}): {last_error()}")


def fwd_workspace_bytes(B: int, T: int, K: int, H: int, snapshot_len: int = 0) -> int:
    return int(load().grm_hip_chunk_update_fwd_workspace(B, T, K, H, snapshot_len))


def chunk_update_fwd(keys, values, queries, memory, decay: float, snapshot_len: int = 0, split: bool = True,
                     want_hidden: bool = True, want_memory_out: bool = True):
    """Returns (hidden, memory_out, snapshots), each None when not requested; inputs must be
    contiguous device tensors.  split=False withholds the workspace, so each sequence is
    scanned by one workgroup chain.  want_hidden / want_memory_out=False pass NULL for that
    output (memory_out may be NULL only when snapshots are requested)."""
    B, T, K = keys.shape
    H = values.shape[2]
    hidden = torch.empty((B, T, H), dtype=values.dtype, device=values.device) if want_hidden else None
    memory_out = torch.empty_like(memory) if want_memory_out else None
    snaps = None
    if snapshot_len > 0:
        snaps = torch.empty((B, (T + snapshot_len - 1) // snapshot_len, H, K), dtype=torch.float32,
                            device=keys.device)
    wsb = fwd_workspace_bytes(B, T, K, H, snapshot_len) if split else 0
    ws = torch.empty((max(wsb, 4) + 3) // 4, dtype=torch.float32, device=keys.device) if wsb else None
    rc = load().grm_hip_chunk_update_fwd(_ptr(keys), _ptr(values), _ptr(queries), _ptr(memory), _ptr(hidden),
                                         _ptr(memory_out), _ptr(snaps), _ptr(ws), wsb, B, T, K, H,
                                         dtype_code(keys.dtype), dtype_code(memory.dtype), float(decay),
                                         int(snapshot_len), _stream(keys))
    _check(rc, "grm_hip_chunk_update_fwd")
    return hidden, memory_out, snaps


def chunk_update_fwd_noalloc(keys, values, queries, memory, decay: float, snapshot_len: int = 0, hidden=None,
                             memory_out=None, snapshots=None):
    """grm_hip_chunk_update_fwd_noalloc into caller-given outputs (allocated here when not
    given, before the call): the library itself allocates nothing.  Returns (hidden,
    memory_out, snapshots)."""
    B, T, K = keys.shape
    H = values.shape[2]
    if hidden is None:
        hidden = torch.empty((B, T, H), dtype=values.dtype, device=values.device)
    if memory_out is None:
        memory_out = torch.empty_like(memory)
    if snapshots is None and snapshot_len > 0:
        snapshots = torch.empty((B, (T + snapshot_len - 1) // snapshot_len, H, K), dtype=torch.float32,
                                device=keys.device)
    rc = load().grm_hip_chunk_update_fwd_noalloc(_ptr(keys), _ptr(values), _ptr(queries), _ptr(memory),
                                                 _ptr(hidden), _ptr(memory_out), _ptr(snapshots), B, T, K, H,
                                                 dtype_code(keys.dtype), dtype_code(memory.dtype), float(decay),
                                                 int(snapshot_len), _stream(keys))
    _check(rc, "grm_hip_chunk_update_fwd_noalloc")
    return hidden, memory_out, snapshots


def noalloc_limit() -> int:
    return int(load().grm_hip_chunk_update_fwd_noalloc_limit())


def chunk_update_bwd(grad_hidden, grad_memory_out, keys, values, queries, memory, decay: float,
                     chunk_states=None):
    """chunk_states: the forward's float32 64-token snapshots [B, ceil(T/64), H, K], or None
    (the backward scans again to produce them)."""
    B, T, K = keys.shape
    H = values.shape[2]
    gk, gv, gq, gm = (torch.empty_like(keys), torch.empty_like(values), torch.empty_like(queries),
                      torch.empty_like(memory))
    given = chunk_states is not None
    states = chunk_states if given else torch.empty((B, max(1, (T + 63) // 64), H, K), dtype=torch.float32,
                                                     device=keys.device)
    partial = torch.empty((2, B, (H + 15) // 16, max(T, 1), K), dtype=torch.float32, device=keys.device)
    rc = load().grm_hip_chunk_update_bwd(_ptr(grad_hidden), _ptr(grad_memory_out), _ptr(keys), _ptr(values),
                                         _ptr(queries), _ptr(memory), _ptr(gk), _ptr(gv), _ptr(gq), _ptr(gm),
                                         _ptr(states), int(given), _ptr(partial), B, T, K, H, dtype_code(keys.dtype),
                                         dtype_code(memory.dtype), float(decay), _stream(keys))
    _check(rc, "grm_hip_chunk_update_bwd")
    return gk, gv, gq, gm


def apply_query_fwd(memories, queries):
    r5 = memories.dim() == 5
    B = memories.shape[0]
    Q = memories.shape[1] if r5 else 1
    R, H, K = memories.shape[-3:]
    out = torch.empty(memories.shape[:-1], dtype=memories.dtype, device=memories.device)
    rc = load().grm_hip_apply_query_fwd(_ptr(memories), _ptr(queries), _ptr(out), B, Q, R, H, K,
                                        dtype_code(memories.dtype), _stream(memories))
    _check(rc, "grm_hip_apply_query_fwd")
    return out


def apply_query_bwd(grad_hidden, memories, queries):
    r5 = memories.dim() == 5
    B = memories.shape[0]
    Q = memories.shape[1] if r5 else 1
    R, H, K = memories.shape[-3:]
    gm, gq = torch.empty_like(memories), torch.empty_like(queries)
    rc = load().grm_hip_apply_query_bwd(_ptr(grad_hidden), _ptr(memories), _ptr(queries), _ptr(gm), _ptr(gq),
                                        B, Q, R, H, K, dtype_code(memories.dtype), _stream(memories))
    _check(rc, "grm_hip_apply_query_bwd")
    return gm, gq


def batched_gather(memories, indices, bad_count=None, out=None):
    B, S = memories.shape[:2]
    n_index = indices[0].numel() if B > 0 else 0
    if out is None:
        out = torch.empty((B,) + tuple(indices.shape[1:]) + tuple(memories.shape[2:]), dtype=memories.dtype,
                          device=memories.device)
    row = memories[0, 0].numel() if B > 0 and S > 0 else int(torch.tensor(memories.shape[2:]).prod())
    rc = load().grm_hip_batched_gather(_ptr(memories), _ptr(indices), _ptr(out), B, S, n_index, row,
                                       memories.element_size(), _ptr(bad_count), _stream(memories))
    _check(rc, "grm_hip_batched_gather")
    return out


def gather_apply(memories, indices, queries, bad_count=None, out=None, dtype=None):
    """out[b, q, r, :] = memories[b, indices[b, q, r]] @ queries[b, q] in `dtype` (the memories'
    dtype by default, or float32: widened 16-bit memories), without materialising the gathered
    states."""
    B, S, H, K = memories.shape
    Q, R = indices.shape[1], indices.shape[2]
    dtype = dtype or memories.dtype
    if out is None:
        out = torch.empty((B, Q, R, H), dtype=dtype, device=memories.device)
    wsb = int(load().grm_hip_gather_apply_workspace(B, S, Q * R))
    ws = torch.empty(max(wsb, 16), dtype=torch.uint8, device=memories.device)
    rc = load().grm_hip_gather_apply(_ptr(memories), _ptr(indices), _ptr(queries), _ptr(out), _ptr(ws), wsb, B, S,
                                     Q, R, H, K, dtype_code(memories.dtype), dtype_code(queries.dtype),
                                     dtype_code(dtype), _ptr(bad_count), _stream(memories))
    _check(rc, "grm_hip_gather_apply")
    return out


def gather_apply_bwd_queries(memories, indices, grad_out, bad_count=None):
    """Per-pair queries' gradient of gather_apply: [B, Q, R, K] float32 = M[idx]^T grad_out."""
    B, S, H, K = memories.shape
    Q, R = indices.shape[1], indices.shape[2]
    gp = torch.empty((B, Q, R, K), dtype=torch.float32, device=memories.device)
    wsb = int(load().grm_hip_gather_apply_workspace(B, S, Q * R))
    ws = torch.empty(max(wsb, 16), dtype=torch.uint8, device=memories.device)
    rc = load().grm_hip_gather_apply_bwd_queries(_ptr(memories), _ptr(indices), _ptr(grad_out), _ptr(gp), _ptr(ws), wsb,
                                                 B, S, Q, R, H, K, dtype_code(memories.dtype), _ptr(bad_count),
                                                 _stream(memories))
    _check(rc, "grm_hip_gather_apply_bwd_queries")
    return gp


def gather_apply_bwd_tokens(memories, indices, grad_tokens, bad_count=None):
    """Per-pair rows M[idx]^T g[q] for one float32 gradient row per query: [B, Q, R, K] float32."""
    B, S, H, K = memories.shape
    Q, R = indices.shape[1], indices.shape[2]
    gp = torch.empty((B, Q, R, K), dtype=torch.float32, device=memories.device)
    wsb = int(load().grm_hip_gather_apply_workspace(B, S, Q * R))
    ws = torch.empty(max(wsb, 16), dtype=torch.uint8, device=memories.device)
    rc = load().grm_hip_gather_apply_bwd_tokens(_ptr(memories), _ptr(indices), _ptr(grad_tokens), _ptr(gp), _ptr(ws),
                                                wsb, B, S, Q, R, H, K, dtype_code(memories.dtype), _ptr(bad_count),
                                                _stream(memories))
    _check(rc, "grm_hip_gather_apply_bwd_tokens")
    return gp


def retrieve_fuse(memories, indices, queries, gates, h_online, ln_weight=None, ln_bias=None, eps=1e-5,
                  bad_count=None, out=None):
    """out[b, q] = LN(h_online[b, q] + sum_r gates[b, q, r] * memories[b, indices[b, q, r]] @ queries[b, q]):
    gather_apply (float32) + fuse_residual in one call, without the float32 [B, Q, R, H] rows."""
    B, S, H, K = memories.shape
    Q, R = indices.shape[1], indices.shape[2]
    if out is None:
        out = torch.empty_like(h_online)
    wsb = int(load().grm_hip_retrieve_fuse_workspace(B, S, Q * R, H))
    ws = torch.empty(max(wsb, 16), dtype=torch.uint8, device=memories.device)
    rc = load().grm_hip_retrieve_fuse(_ptr(memories), _ptr(indices), _ptr(queries), _ptr(gates), _ptr(h_online),
                                      _ptr(ln_weight), _ptr(ln_bias), _ptr(out), _ptr(ws), wsb, B, S, Q, R, H, K,
                                      dtype_code(memories.dtype), dtype_code(queries.dtype),
                                      dtype_code(h_online.dtype), float(eps), _ptr(bad_count), _stream(memories))
    _check(rc, "grm_hip_retrieve_fuse")
    return out


def segment_retrieve_fuse(memories, indices, queries, gates, h_online, segment_len: int, base: int, capacity: int,
                          ln_weight=None, ln_bias=None, eps=1e-5, bad_count=None, out=None):
    """retrieve_fuse for the indices of segment routing: query t sees the entries [lo(t), hi(t)),
    hi(t) = base + t // segment_len, lo(t) = max(0, hi(t) - capacity); negative indices are empty
    slots, indices outside the window (or repeated within a query) contribute nothing and are
    counted in bad_count.  Each query's routes are summed in the kernel (no per-route rows)."""
    B, S, H, K = memories.shape
    Q, R = indices.shape[1], indices.shape[2]
    if out is None:
        out = torch.empty_like(h_online)
    wsb = int(load().grm_hip_segment_retrieve_fuse_workspace(B, Q, H, K, int(segment_len), int(base), int(capacity),
                                                              dtype_code(memories.dtype)))
    ws = torch.empty(max(wsb, 16), dtype=torch.uint8, device=memories.device)
    rc = load().grm_hip_segment_retrieve_fuse(_ptr(memories), _ptr(indices), _ptr(queries), _ptr(gates),
                                              _ptr(h_online), _ptr(ln_weight), _ptr(ln_bias), _ptr(out), _ptr(ws),
                                              wsb, B, S, Q, R, H, K, int(segment_len), int(base), int(capacity),
                                              dtype_code(memories.dtype), dtype_code(queries.dtype),
                                              dtype_code(h_online.dtype), float(eps), _ptr(bad_count),
                                              _stream(memories))
    _check(rc, "grm_hip_segment_retrieve_fuse")
    return out


def project_split(proj, key_dim: int, value_dim: int, extra_dim: int = 0, eps: float = 1e-6):
    """(keys, values, queries, extra) from [..., key_dim + value_dim + key_dim + extra_dim] rows;
    keys and queries L2-normalised."""
    lead = proj.shape[:-1]
    rows = int(proj.numel() // proj.shape[-1]) if proj.shape[-1] else 0
    mk = lambda d: torch.empty(lead + (d,), dtype=proj.dtype, device=proj.device)  # noqa: E731
    k, v, q = mk(key_dim), mk(value_dim), mk(key_dim)
    e = mk(extra_dim) if extra_dim else None
    rc = load().grm_hip_project_split(_ptr(proj), _ptr(k), _ptr(v), _ptr(q), _ptr(e), rows, key_dim, value_dim,
                                      extra_dim, dtype_code(proj.dtype), float(eps), _stream(proj))
    _check(rc, "grm_hip_project_split")
    return k, v, q, e


def residual_layer_norm(x, residual, weight=None, bias=None, eps: float = 1e-5, out=None):
    H = x.shape[-1]
    out = torch.empty_like(x) if out is None else out
    pd = dtype_code(weight.dtype) if weight is not None else dtype_code(x.dtype)
    rc = load().grm_hip_residual_layer_norm(_ptr(x), _ptr(residual), _ptr(weight), _ptr(bias), _ptr(out),
                                            int(x.numel() // H) if H else 0, H, dtype_code(x.dtype), pd, float(eps),
                                            _stream(x))
    _check(rc, "grm_hip_residual_layer_norm")
    return out


def project_gemm(x, weight, bias, key_dim: int, value_dim: int, extra_dim: int = 0, eps: float = 1e-6):
    """(keys, values, queries, extra) of x weight^T + bias, keys and queries L2-normalised."""
    K = x.shape[-1]
    rows = x.numel() // K
    mk = lambda d: torch.empty(x.shape[:-1] + (d,), dtype=x.dtype, device=x.device)  # noqa: E731
    k, v, q, e = mk(key_dim), mk(value_dim), mk(key_dim), mk(extra_dim)
    rc = load().grm_hip_project_gemm(_ptr(x), _ptr(weight), _ptr(bias), _ptr(k), _ptr(v), _ptr(q),
                                     _ptr(e) if extra_dim else None, rows, K, key_dim, value_dim, extra_dim,
                                     dtype_code(x.dtype), float(eps), _stream(x))
    _check(rc, "grm_hip_project_gemm")
    return k, v, q, e


def linear_residual_layer_norm(x, weight, bias, residual, ln_weight=None, ln_bias=None, eps: float = 1e-5,
                               save: bool = False):
    """LayerNorm(round(x weight^T + bias) + residual) in one kernel.  Returns out, or with save
    (out, pre, mean, rstd): the LayerNorm input and its float32 row statistics."""
    K, N = x.shape[-1], weight.shape[0]
    rows = x.numel() // K if K else 0
    out = torch.empty(x.shape[:-1] + (N,), dtype=x.dtype, device=x.device)
    pre = torch.empty_like(out) if save else None
    mean = torch.empty(rows, dtype=torch.float32, device=x.device) if save else None
    rstd = torch.empty(rows, dtype=torch.float32, device=x.device) if save else None
    pd = dtype_code(ln_weight.dtype) if ln_weight is not None else dtype_code(x.dtype)
    rc = load().grm_hip_linear_residual_layer_norm(_ptr(x), _ptr(weight), _ptr(bias), _ptr(residual),
                                                   _ptr(ln_weight), _ptr(ln_bias), _ptr(out), _ptr(pre), _ptr(mean),
                                                   _ptr(rstd), rows, K, N, dtype_code(x.dtype), pd, float(eps),
                                                   _stream(x))
    _check(rc, "grm_hip_linear_residual_layer_norm")
    return (out, pre, mean, rstd) if save else out


def archive_cast(states, model_dtype, storage_dtype, out=None):
    """float32 states rounded to model_dtype, then to storage_dtype (the archive's stored form)."""
    out = torch.empty(states.shape, dtype=storage_dtype, device=states.device) if out is None else out
    rc = load().grm_hip_archive_cast(_ptr(states), _ptr(out), int(states.numel()), dtype_code(model_dtype),
                                     dtype_code(storage_dtype), _stream(states))
    _check(rc, "grm_hip_archive_cast")
    return out


def topk_route(queries, keys, top_k: int, scale: float, temperature: float = 1.0):
    B, Q, D = queries.shape
    S = keys.shape[1]
    k = min(top_k, S)
    idx = torch.empty((B, Q, k), dtype=torch.int64, device=queries.device)
    sc = torch.empty((B, Q, k), dtype=torch.float32, device=queries.device)
    gt = torch.empty((B, Q, k), dtype=torch.float32, device=queries.device)
    rc = load().grm_hip_topk_route(_ptr(queries), _ptr(keys), _ptr(idx), _ptr(sc), _ptr(gt), B, Q, S, D,
                                   dtype_code(queries.dtype), int(top_k), float(scale), float(temperature),
                                   _stream(queries))
    _check(rc, "grm_hip_topk_route")
    return gt, idx, sc


def segment_route(queries, keys, top_k: int, segment_len: int, base: int, capacity: int, scale: float,
                  temperature: float = 1.0):
    B, Q, D = queries.shape
    S = keys.shape[1]
    idx = torch.empty((B, Q, top_k), dtype=torch.int64, device=queries.device)
    sc = torch.empty((B, Q, top_k), dtype=torch.float32, device=queries.device)
    gt = torch.empty((B, Q, top_k), dtype=torch.float32, device=queries.device)
    rc = load().grm_hip_segment_route(_ptr(queries), _ptr(keys), _ptr(idx), _ptr(sc), _ptr(gt), B, Q, S, D,
                                      dtype_code(queries.dtype), int(top_k), int(segment_len), int(base),
                                      int(capacity), float(scale), float(temperature), _stream(queries))
    _check(rc, "grm_hip_segment_route")
    return gt, idx, sc


def fuse_residual(h, retrieved, gates, weight=None, bias=None, eps: float = 1e-5):
    N, H = h.shape
    R = retrieved.shape[1]
    out = torch.empty_like(h)
    rc = load().grm_hip_fuse_residual(_ptr(h), _ptr(retrieved), _ptr(gates), _ptr(weight), _ptr(bias), _ptr(out),
                                      N, R, H, dtype_code(h.dtype), float(eps), _stream(h))
    _check(rc, "grm_hip_fuse_residual")
    return out
