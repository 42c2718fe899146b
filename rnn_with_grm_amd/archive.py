"""Device ring-buffer archive of segment states, a drop-in for the reference's
``SegmentMemoryArchive`` (grm/core/paper_grm.py:47-349).

The reference keeps each batch-size group as three ``deque(maxlen=capacity)``
of per-segment tensors and, on every segment, stacks the whole deque into a
fresh ``[B, S, d_v, d_k]`` float32 tensor (``torch.stack(...).to(float32)
.permute(1, 0, 2, 3).contiguous()``, paper_grm.py:227-228) before gathering
from it.  Here each group owns two device rings allocated once:

  memories  [B, capacity, d_v, d_k]  in the storage dtype (float16 by default)
  summaries [B, capacity, D_in]      in the storage dtype

A push writes one slot; the oldest entry is overwritten once the ring is
full, which is the deque's eviction.  Position j of the reference's stacked
deque (0 = oldest kept) is ring slot ``(start + j) % capacity``, so retrieval
remaps the router's indices and reads the ring in place:

  retrieve_from_indices -> one fused gather + query application
                           (torch.ops.grm_cuda.gather_apply, dtype=float32:
                           the float16 states are widened on load, exactly as
                           the reference's .to(float32)), no stacked copy and
                           no [B, Q, R, d_v, d_k] tensor;
  retrieve_memories     -> the gathered states, as the reference returns them
                           (memory_soup mode needs them).

``get_extra_state`` / ``set_extra_state`` read and write the reference's
format (paper_grm.py:98-133): per group, lists of per-segment tensors oldest
first, so checkpoints written by either implementation load in the other.
Selective recompute (``recomputation_ratio > 0``, paper_grm.py:169-201) is not
provided; the hierarchical model and every benchmark configuration use 0.
"""

from __future__ import annotations

from collections import deque
from dataclasses import dataclass
from typing import Deque, Dict, List, Optional

import torch
import torch.nn as nn
import torch.nn.functional as F
from torch import Tensor

from . import cuda_ops


@dataclass
class SegmentCheckpoint:
    """Inputs and starting state of one segment (the reference's
    SegmentReconstructionState, paper_grm.py:25-28), kept for the state format."""

    inputs: Tensor
    memory_start: Tensor


class _Ring:
    """One batch-size group: fixed-capacity device rings plus a checkpoint deque."""

    def __init__(self, capacity: int):
        self.capacity = capacity
        self.memories: Optional[Tensor] = None   # [B, capacity, d_v, d_k]
        self.summaries: Optional[Tensor] = None  # [B, capacity, D]
        self.checkpoints: Deque[SegmentCheckpoint] = deque(maxlen=capacity)
        self.count = 0  # entries kept (<= capacity)
        self.head = 0   # next slot written

    def __len__(self) -> int:
        return self.count

    def start(self) -> int:
        """Ring slot of the oldest kept entry (deque position 0)."""
        return (self.head - self.count) % self.capacity

    def order(self, device: torch.device) -> Tensor:
        """Ring slots in deque order, oldest first."""
        return (torch.arange(self.count, device=device) + self.start()) % self.capacity

    def allocate(self, memory: Tensor, summary: Tensor, dtype: torch.dtype) -> None:
        if self.memories is None:
            b = memory.size(0)
            self.memories = torch.zeros((b, self.capacity) + tuple(memory.shape[1:]), dtype=dtype,
                                        device=memory.device)
            self.summaries = torch.zeros((b, self.capacity) + tuple(summary.shape[1:]), dtype=dtype,
                                         device=summary.device)

    def write(self, memories: Tensor, summaries: Tensor) -> None:
        """Append n entries ([B, n, ...]); only the last `capacity` survive."""
        n = memories.size(1)
        if n > self.capacity:
            memories, summaries = memories[:, n - self.capacity:], summaries[:, n - self.capacity:]
            self.head = (self.head + n - self.capacity) % self.capacity
            n = self.capacity
        # The slots head .. head + n - 1 (mod capacity) are at most two runs: two slice copies.
        first = min(n, self.capacity - self.head)
        for dst, src in ((self.memories, memories), (self.summaries, summaries)):
            dst[:, self.head:self.head + first].copy_(src[:, :first])
            if first < n:
                dst[:, :n - first].copy_(src[:, first:])
        self.head = (self.head + n) % self.capacity
        self.count = min(self.capacity, self.count + n)


class DeviceSegmentArchive(nn.Module):
    """Same constructor, methods and state format as the reference's
    SegmentMemoryArchive (paper_grm.py:47-349); storage is a device ring."""

    def __init__(self, hidden_size: int, memory_key_dim: int, summary_size: int, max_segments: int,
                 memory_storage_dtype: torch.dtype = torch.float16, recomputation_ratio: float = 0.0):
        super().__init__()
        if recomputation_ratio > 0.0:
            raise NotImplementedError("DeviceSegmentArchive does not recompute segments (recomputation_ratio must be 0)")
        self.hidden_size = hidden_size
        self.memory_key_dim = memory_key_dim
        self.summary_size = summary_size
        self.max_segments = max_segments
        self.memory_storage_dtype = memory_storage_dtype
        self.recomputation_ratio = recomputation_ratio
        self._groups: Dict[int, _Ring] = {}
        self.register_buffer("total_pushed", torch.tensor(0, dtype=torch.long))
        self.register_buffer("total_recomputed", torch.tensor(0, dtype=torch.long))
        self.register_buffer("total_retrieved", torch.tensor(0, dtype=torch.long))
        # Host mirror of (total_retrieved, total_recomputed) for get_recompute_rate, so
        # that a forward's report reads no device value (a forward then has no host
        # synchronisation and can be captured in a graph).  None: read the buffers
        # once (after a state-dict load or a change made outside this class).
        self._host_counts: Optional[List[int]] = [0, 0]
        self.register_load_state_dict_post_hook(lambda module, keys: setattr(module, "_host_counts", None))

    # ------------------------------------------------------------- bookkeeping
    def _group(self, batch_size: int) -> _Ring:
        if batch_size not in self._groups:
            self._groups[batch_size] = _Ring(self.max_segments)
        return self._groups[batch_size]

    def clear(self) -> None:
        self._groups.clear()
        # one launch for the three counters
        torch._foreach_zero_([self.total_pushed, self.total_recomputed, self.total_retrieved])
        self._host_counts = [0, 0]

    def _count_retrieved(self, n: int) -> None:
        self.total_retrieved.add_(n)
        if self._host_counts is not None:
            self._host_counts[0] += n

    def _apply(self, fn):
        super()._apply(fn)
        for ring in self._groups.values():
            if ring.memories is not None:
                ring.memories = fn(ring.memories)
                ring.summaries = fn(ring.summaries)
            ring.checkpoints = deque((SegmentCheckpoint(fn(c.inputs), fn(c.memory_start)) for c in ring.checkpoints),
                                     maxlen=self.max_segments)
        return self

    def get_num_segments(self, batch_size: Optional[int] = None) -> int:
        if batch_size is not None:
            ring = self._groups.get(batch_size)
            return 0 if ring is None else len(ring)
        if not self._groups:
            return 0
        return max(len(ring) for ring in self._groups.values())

    # ------------------------------------------------------------- state format
    def get_extra_state(self):
        groups = {}
        for batch_size, ring in self._groups.items():
            if ring.memories is None or ring.count == 0:
                mem_list, sum_list = [], []
            else:
                order = ring.order(ring.memories.device)
                mem_list = list(ring.memories.index_select(1, order).unbind(1))
                sum_list = list(ring.summaries.index_select(1, order).unbind(1))
            groups[batch_size] = {
                "memories": [m.clone() for m in mem_list],
                "summaries": [s.clone() for s in sum_list],
                "checkpoints": [{"inputs": c.inputs, "memory_start": c.memory_start} for c in ring.checkpoints],
            }
        return {"groups": groups}

    def set_extra_state(self, state):
        self._groups = {}
        groups_state = {} if state is None else state.get("groups", {})
        for batch_size, g in groups_state.items():
            ring = _Ring(self.max_segments)
            mems, sums = list(g.get("memories", [])), list(g.get("summaries", []))
            if mems:
                ring.allocate(mems[0], sums[0], mems[0].dtype)
                ring.write(torch.stack(mems, 1), torch.stack(sums, 1))
            for c in g.get("checkpoints", []):
                ring.checkpoints.append(SegmentCheckpoint(c["inputs"], c["memory_start"]))
            self._groups[int(batch_size)] = ring

    # ------------------------------------------------------------- writes
    def push(self, memory: Tensor, summary: Tensor, checkpoint) -> None:
        """One segment: memory [B, d_v, d_k], summary [B, D] (paper_grm.py:135-146)."""
        ring = self._group(memory.size(0))
        ring.allocate(memory, summary, self.memory_storage_dtype)
        ring.write(memory.detach().unsqueeze(1), summary.detach().unsqueeze(1))
        ring.checkpoints.append(SegmentCheckpoint(checkpoint.inputs.detach().clone(),
                                                  checkpoint.memory_start.detach().to(self.memory_storage_dtype).clone()))
        self.total_pushed.add_(1)

    def push_segments(self, memories: Tensor, summaries: Tensor, checkpoints=None, owned: bool = False) -> None:
        """n segments at once (the whole-sequence path): memories [B, n, d_v, d_k],
        summaries [B, n, D], oldest first; equal to n calls of push.  With
        owned=True the checkpoints' tensors are fresh copies the archive may keep
        as they are (memory_start already in the storage dtype), so no per-segment
        copies are made."""
        n = memories.size(1)
        if n == 0:
            return
        ring = self._group(memories.size(0))
        ring.allocate(memories[:, 0], summaries[:, 0], self.memory_storage_dtype)
        ring.write(memories.detach(), summaries.detach())
        for c in checkpoints or []:
            if owned:
                ring.checkpoints.append(SegmentCheckpoint(c.inputs, c.memory_start))
            else:
                ring.checkpoints.append(SegmentCheckpoint(
                    c.inputs.detach().clone(), c.memory_start.detach().to(self.memory_storage_dtype).clone()))
        self.total_pushed.add_(n)

    # ------------------------------------------------------------- reads
    def get_segment_summaries(self, query_batch_size: int, device: torch.device,
                              dtype: Optional[torch.dtype] = None) -> Tensor:
        """[B, S, D] oldest first (paper_grm.py:148-160)."""
        ring = self._groups.get(query_batch_size)
        target = dtype or torch.float32
        if ring is None or len(ring) == 0:
            return torch.zeros(query_batch_size, 0, self.summary_size, device=device, dtype=target)
        return ring.summaries.index_select(1, ring.order(ring.summaries.device)).to(device=device, dtype=target)

    def slots(self, topk_indices: Tensor, batch_size: int) -> Tensor:
        """Deque positions (0 = oldest kept) -> ring slots, for reading the ring in place.
        A position outside [0, len) (such as the -1 of an empty routing slot) stays
        invalid (-1): the gather kernels then write a zero row and count it, instead of
        reading whatever state the ring holds in that slot."""
        ring = self._groups[batch_size]
        pos = topk_indices.to(torch.long)
        valid = (pos >= 0) & (pos < len(ring))
        return torch.where(valid, (pos + ring.start()) % ring.capacity, torch.full_like(pos, -1))

    def _empty_retrieval(self, topk_indices: Tensor, device, last: tuple) -> Tensor:
        lead = (topk_indices.size(0),) + ((topk_indices.size(1),) if topk_indices.ndim == 3 else ())
        return torch.zeros(lead + (0,) + last, device=device, dtype=torch.float32)

    def retrieve_memories(self, topk_indices: Tensor, gates: Tensor, memory_cell, device: torch.device,
                          memory_decay: float, cuda_cpp_debug_fallback: bool = False) -> Tensor:
        """Gathered states, float32, [B, (Q,) R, d_v, d_k] (paper_grm.py:203-236)."""
        batch_size = topk_indices.size(0)
        ring = self._groups.get(batch_size)
        if ring is None or topk_indices.numel() == 0 or len(ring) == 0:
            return self._empty_retrieval(topk_indices, device, (self.hidden_size, self.memory_key_dim))
        slots = self.slots(topk_indices, batch_size)
        selected = cuda_ops.cuda_batched_memory_gather(ring.memories, slots, enabled=True,
                                                       debug_fallback=cuda_cpp_debug_fallback)
        self._count_retrieved(int(topk_indices.numel()))
        return selected.to(device=device, dtype=torch.float32)

    def retrieve_from_indices(self, query_inputs: Tensor, topk_indices: Tensor, gates: Tensor, memory_cell,
                              device: torch.device, memory_decay: float,
                              cuda_cpp_debug_fallback: bool = False) -> Tensor:
        """M_selected q for every route, float32 [B, (Q,) R, d_v] (paper_grm.py:271-313),
        as one fused gather + apply over the ring."""
        batch_size = topk_indices.size(0)
        ring = self._groups.get(batch_size)
        if ring is None or topk_indices.numel() == 0 or len(ring) == 0:
            return self._empty_retrieval(topk_indices, device, (self.hidden_size,))
        q_t = F.normalize(memory_cell.query_proj(query_inputs), p=2, dim=-1, eps=1e-6).to(torch.float32)
        slots = self.slots(topk_indices, batch_size)
        self._count_retrieved(int(topk_indices.numel()))
        return cuda_ops.cuda_gather_apply(ring.memories, slots, q_t, torch.float32,
                                          debug_fallback=cuda_cpp_debug_fallback).to(device)

    # ------------------------------------------------------------- reporting
    def refresh_counters(self) -> None:
        """Read the counter buffers again at the next report.  The host mirror advances when
        Python code runs a forward; a captured graph replayed N times advances the device
        buffers N times and the mirror not at all, so call this after replaying a graph
        that contains a forward."""
        self._host_counts = None

    def get_recompute_rate(self) -> float:
        """total_recomputed / total_retrieved from the host mirror (no device read), or from
        the buffers after a state-dict load or refresh_counters()."""
        if self._host_counts is None:
            self._host_counts = [int(self.total_retrieved.item()), int(self.total_recomputed.item())]
        total, recomputed = self._host_counts
        return 0.0 if total == 0 else float(recomputed) / total

    def get_memory_info(self) -> Dict[str, float]:
        """Same keys as paper_grm.py:322-349; bytes count the kept entries."""
        memory_bytes = summary_bytes = checkpoint_bytes = 0
        num_segments = 0
        for ring in self._groups.values():
            num_segments += len(ring)
            if ring.memories is not None and ring.count:
                memory_bytes += ring.count * ring.memories[:, 0].numel() * ring.memories.element_size()
                summary_bytes += ring.count * ring.summaries[:, 0].numel() * ring.summaries.element_size()
            for c in ring.checkpoints:
                checkpoint_bytes += c.inputs.numel() * c.inputs.element_size()
                checkpoint_bytes += c.memory_start.numel() * c.memory_start.element_size()
        mb = 1024 ** 2
        return {
            "cached_states_mb": round(memory_bytes / mb, 2),
            "summaries_mb": round(summary_bytes / mb, 2),
            "checkpoints_mb": round(checkpoint_bytes / mb, 2),
            "total_mb": round((memory_bytes + summary_bytes + checkpoint_bytes) / mb, 2),
            "num_segments": num_segments,
            "num_groups": len(self._groups),
            "recompute_rate": self.get_recompute_rate(),
        }


__all__ = ["DeviceSegmentArchive", "SegmentCheckpoint"]
