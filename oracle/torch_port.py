"""Torch-CPU restatement of the reference's CPU path.  TEST INFRASTRUCTURE ONLY.

This is what the reference runs for these ops on CPU tensors under the
default ``auto`` policy (its cuda_ops falls back to PyTorch on CPU,
grm/core/cuda_ops.py:117-135), restated in this repository so it can be timed
on the GPU box's host as bench.py's cpu_baseline leg ("port").  It is never on
the product path.

  chunk_update      grm/core/cuda_ops.py:218-254 (_vectorized_chunk_update),
                    called once per segment with the state carried, as the
                    models do (grm/core/paper_grm.py:486-504, 702-728)
  route             grm/core/paper_grm.py:566-589 (matmul * scale, topk, softmax)
  gather            grm/core/cuda_ops.py:265-284 (index_select per batch entry)
  apply_query       grm/core/cuda_ops.py:257-262 (einsum)
  fuse_residual     grm/core/aggregator.py:67-145 (weighted sum + LayerNorm)
"""

from __future__ import annotations

import math
from typing import List, Tuple

import torch
from torch import Tensor


def vectorized_chunk_update(keys: Tensor, values: Tensor, queries: Tensor, memory: Tensor,
                            decay: float) -> Tuple[Tensor, Tensor]:
    """One segment of the chunked closed form, in memory's dtype."""
    B, L, K = keys.shape
    if L == 0:
        return values.new_zeros(B, 0, values.size(-1)), memory
    base = torch.as_tensor(decay, dtype=memory.dtype)
    pos = torch.arange(L, dtype=memory.dtype)
    start = torch.pow(base, pos + 1.0).view(1, L, 1)
    h_start = torch.matmul(memory, queries.transpose(1, 2)).transpose(1, 2) * start
    s = torch.matmul(queries, keys.transpose(1, 2)) / math.sqrt(float(K))
    rel = pos.unsqueeze(1) - pos.unsqueeze(0)
    dmask = torch.pow(base, rel.clamp_min(0)) * (rel >= 0).to(s.dtype)
    h = h_start + (1.0 - base) * torch.matmul(s * dmask.unsqueeze(0), values)
    end = torch.pow(base, (L - 1) - pos)
    wv = values * ((1.0 - base) * end / math.sqrt(float(K))).view(1, L, 1)
    m = torch.pow(base, torch.tensor(float(L), dtype=memory.dtype)) * memory + torch.einsum("bch,bck->bhk", wv, keys)
    return h, m


def segment_scan(keys: Tensor, values: Tensor, queries: Tensor, memory: Tensor, decay: float,
                 segment_len: int) -> Tuple[Tensor, Tensor, Tensor]:
    """Whole sequence, one call per segment, computed in float32.
    Returns (hidden, final state, per-segment snapshots)."""
    k, v, q = keys.float(), values.float(), queries.float()
    m = memory.float()
    outs: List[Tensor] = []
    snaps: List[Tensor] = []
    for t0 in range(0, k.size(1), segment_len):
        h, m = vectorized_chunk_update(k[:, t0:t0 + segment_len], v[:, t0:t0 + segment_len],
                                       q[:, t0:t0 + segment_len], m, decay)
        outs.append(h)
        snaps.append(m)
    return torch.cat(outs, 1), m, torch.stack(snaps, 1)


def route(queries: Tensor, keys: Tensor, top_k: int, scale: float, temperature: float = 1.0):
    """Scores, top-k (torch.topk) and softmax gates, float32."""
    scores = torch.matmul(queries.float(), keys.float().transpose(1, 2)) * scale
    k = min(top_k, keys.size(1))
    if k < keys.size(1):
        top, idx = torch.topk(scores, k=k, dim=-1)
    else:
        top = scores
        idx = torch.arange(keys.size(1)).view(1, 1, -1).expand(scores.size(0), scores.size(1), -1)
    return torch.softmax(top / temperature, dim=-1), idx, top


def gather(memories: Tensor, indices: Tensor) -> Tensor:
    out = memories.new_empty((memories.size(0),) + tuple(indices.shape[1:]) + tuple(memories.shape[2:]))
    for b in range(memories.size(0)):
        out[b].copy_(memories[b].index_select(0, indices[b].reshape(-1)).reshape(out[b].shape))
    return out


def apply_query(memories: Tensor, queries: Tensor) -> Tensor:
    if memories.ndim == 5:
        return torch.einsum("bqrhk,bqk->bqrh", memories, queries)
    return torch.einsum("brhk,bk->brh", memories, queries)


def fuse_residual(h_online: Tensor, retrieved: Tensor, gates: Tensor, weight: Tensor, bias: Tensor,
                  eps: float = 1e-5) -> Tensor:
    """LayerNorm(h + sum_r gates_r retrieved_r): the residual fusion of
    grm/core/aggregator.py:67-145 as the models call it (paper_grm.py:604-611)."""
    contribution = (retrieved * gates.unsqueeze(-1)).sum(dim=-2)
    return torch.nn.functional.layer_norm(h_online + contribution, (h_online.size(-1),), weight, bias, eps)
