"""ctypes front end of the C oracle (grm_oracle.c).  TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg import
this module; the product path never does.  Every function takes numpy arrays
(any float dtype is converted to float64 first, so pass values already
rounded to the dtype under test) and returns numpy arrays.

Reference files each function restates are cited in grm_oracle.c.
"""

from __future__ import annotations

import ctypes
import subprocess
from pathlib import Path
from typing import Optional, Tuple

import numpy as np

ORACLE_DIR = Path(__file__).resolve().parent
SRC = ORACLE_DIR / "grm_oracle.c"
LIB = ORACLE_DIR / "_build" / "libgrm_oracle.so"

_lib: Optional[ctypes.CDLL] = None


def build(force: bool = False) -> Path:
    """Compile grm_oracle.c with gcc (no fused contraction, so float32 code is
    exactly what the source says)."""
    LIB.parent.mkdir(exist_ok=True)
    if force or not LIB.exists() or LIB.stat().st_mtime < SRC.stat().st_mtime:
        tmp = LIB.with_suffix(".so.tmp")
        subprocess.run(["gcc", "-O2", "-fPIC", "-shared", "-ffp-contract=off", "-o", str(tmp), str(SRC), "-lm"],
                       check=True)
        tmp.replace(LIB)
    return LIB


def _load() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        lib = ctypes.CDLL(str(build()))
        lib.grm_oracle_gather.restype = ctypes.c_int64
        _lib = lib
    return _lib


def _d(a) -> np.ndarray:
    return np.ascontiguousarray(np.asarray(a, dtype=np.float64))


def _p(a: np.ndarray):
    return a.ctypes.data_as(ctypes.c_void_p)


_I = ctypes.c_int64
_D = ctypes.c_double


def chunk_update_seq(keys, values, queries, memory, decay: float,
                     snapshot_len: int = 0) -> Tuple[np.ndarray, np.ndarray, Optional[np.ndarray]]:
    """Per-token recurrence; returns (hidden [B,T,H], memory_out [B,H,K], snapshots or None)."""
    k, v, q, m = _d(keys), _d(values), _d(queries), _d(memory)
    B, T, K = k.shape
    H = v.shape[2]
    hid = np.zeros((B, T, H))
    mo = np.zeros((B, H, K))
    snaps = None
    if snapshot_len > 0:
        snaps = np.zeros((B, (T + snapshot_len - 1) // snapshot_len, H, K))
    _load().grm_oracle_chunk_update_seq(_p(k), _p(v), _p(q), _p(m), _D(decay), _I(B), _I(T), _I(K), _I(H),
                                        _p(hid), _p(mo), _p(snaps) if snaps is not None else None,
                                        _I(snapshot_len))
    return hid, mo, snaps


def chunk_update_chunked(keys, values, queries, memory, decay: float, chunk: int) -> Tuple[np.ndarray, np.ndarray]:
    """Chunked closed form with the state carried between chunks."""
    k, v, q, m = _d(keys), _d(values), _d(queries), _d(memory)
    B, T, K = k.shape
    H = v.shape[2]
    hid = np.zeros((B, T, H))
    mo = np.zeros((B, H, K))
    _load().grm_oracle_chunk_update_chunked(_p(k), _p(v), _p(q), _p(m), _D(decay), _I(B), _I(T), _I(K), _I(H),
                                            _I(chunk), _p(hid), _p(mo))
    return hid, mo


def chunk_update_bwd(grad_hidden, grad_memory_out, keys, values, queries, memory, decay: float):
    """Returns (grad_keys, grad_values, grad_queries, grad_memory)."""
    dh, dmo = _d(grad_hidden), _d(grad_memory_out)
    k, v, q, m = _d(keys), _d(values), _d(queries), _d(memory)
    B, T, K = k.shape
    H = v.shape[2]
    gk, gv, gq, gm = np.zeros((B, T, K)), np.zeros((B, T, H)), np.zeros((B, T, K)), np.zeros((B, H, K))
    _load().grm_oracle_chunk_update_bwd(_p(dh), _p(dmo), _p(k), _p(v), _p(q), _p(m), _D(decay), _I(B), _I(T),
                                        _I(K), _I(H), _p(gk), _p(gv), _p(gq), _p(gm))
    return gk, gv, gq, gm


def apply_query(memories, queries) -> np.ndarray:
    """Rank 4 ([B,R,H,K] x [B,K]) or rank 5 ([B,Q,R,H,K] x [B,Q,K])."""
    mm, q = _d(memories), _d(queries)
    K = mm.shape[-1]
    lead = mm.shape[:-3]
    NQ = int(np.prod(lead))
    RH = mm.shape[-3] * mm.shape[-2]
    out = np.zeros(mm.shape[:-1])
    _load().grm_oracle_apply_query(_p(mm), _p(q), _I(NQ), _I(RH), _I(K), _p(out))
    return out


def apply_query_bwd(grad_hidden, memories, queries) -> Tuple[np.ndarray, np.ndarray]:
    dh, mm, q = _d(grad_hidden), _d(memories), _d(queries)
    K = mm.shape[-1]
    NQ = int(np.prod(mm.shape[:-3]))
    RH = mm.shape[-3] * mm.shape[-2]
    gm = np.zeros(mm.shape)
    gq = np.zeros(q.shape)
    _load().grm_oracle_apply_query_bwd(_p(dh), _p(mm), _p(q), _I(NQ), _I(RH), _I(K), _p(gm), _p(gq))
    return gm, gq


def gather(memories: np.ndarray, indices: np.ndarray) -> Tuple[np.ndarray, int]:
    """Byte-exact gather; returns (out, number of out-of-range indices)."""
    mm = np.ascontiguousarray(memories)
    idx = np.ascontiguousarray(indices, dtype=np.int64)
    B, S = mm.shape[:2]
    row_shape = mm.shape[2:]
    n_index = int(np.prod(idx.shape[1:])) if idx.ndim > 1 else 0
    out = np.zeros((B,) + idx.shape[1:] + row_shape, dtype=mm.dtype)
    row_bytes = int(np.prod(row_shape)) * mm.itemsize
    bad = _load().grm_oracle_gather(_p(mm), _p(idx), _p(out), _I(B), _I(S), _I(n_index), _I(row_bytes))
    return out, int(bad)


def topk_route(queries, keys, top_k: int, scale: float, temperature: float = 1.0):
    """Canonical routing; inputs are cast to float32 (exact for bf16/f16 values).
    Returns (gates float64, indices int64, scores float32)."""
    q = np.ascontiguousarray(np.asarray(queries, dtype=np.float32))
    kk = np.ascontiguousarray(np.asarray(keys, dtype=np.float32))
    B, Q, D = q.shape
    S = kk.shape[1]
    k = min(top_k, S)
    idx = np.zeros((B, Q, k), dtype=np.int64)
    sc = np.zeros((B, Q, k), dtype=np.float32)
    gt = np.zeros((B, Q, k), dtype=np.float64)
    lib = _load()
    lib.grm_oracle_topk_route.argtypes = [ctypes.c_void_p, ctypes.c_void_p, _I, _I, _I, _I, _I, ctypes.c_float,
                                          _D, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p]
    lib.grm_oracle_topk_route(_p(q), _p(kk), B, Q, S, D, top_k, ctypes.c_float(scale), float(temperature),
                              _p(idx), _p(sc), _p(gt))
    return gt, idx, sc


def segment_route(queries, keys, top_k: int, segment_len: int, base: int, capacity: int, scale: float,
                  temperature: float = 1.0):
    """Routing of each segment over the archive of its moment, as the
    reference's segment loop does it (grm/core/paper_grm.py:702-728 calling
    _route_chunk, :566-589, with get_segment_summaries, :148-160): the rows of
    segment s see keys [lo, hi), hi = base + s, lo = max(0, hi - capacity), and
    are routed by topk_route over exactly those keys.  Indices are returned as
    absolute key positions; slots past a short window hold -1 / -inf / 0."""
    q = np.asarray(queries, dtype=np.float32)
    kk = np.asarray(keys, dtype=np.float32)
    B, Q, _ = q.shape
    idx = np.full((B, Q, top_k), -1, dtype=np.int64)
    sc = np.full((B, Q, top_k), -np.inf, dtype=np.float32)
    gt = np.zeros((B, Q, top_k), dtype=np.float64)
    for t0 in range(0, Q, segment_len):
        hi = min(kk.shape[1], base + t0 // segment_len)
        lo = max(0, hi - capacity)
        if hi <= lo:
            continue
        sl = slice(t0, min(Q, t0 + segment_len))
        g, i, s_ = topk_route(q[:, sl], kk[:, lo:hi], top_k, scale, temperature)
        n = g.shape[-1]
        gt[:, sl, :n], idx[:, sl, :n], sc[:, sl, :n] = g, i + lo, s_
    return gt, idx, sc


def fuse_residual(h, retrieved, gates, weight=None, bias=None, eps: float = 1e-5) -> np.ndarray:
    hh, rr, gg = _d(h), _d(retrieved), _d(gates)
    N, H = hh.shape
    R = rr.shape[1]
    w = _d(weight) if weight is not None else None
    b = _d(bias) if bias is not None else None
    out = np.zeros((N, H))
    _load().grm_oracle_fuse_residual(_p(hh), _p(rr), _p(gg), _p(w) if w is not None else None,
                                     _p(b) if b is not None else None, _I(N), _I(R), _I(H), _D(eps), _p(out))
    return out
