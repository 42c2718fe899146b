"""Segment-memory models running the whole sequence through the MI355X path.

Drop-in counterparts of the reference's model classes, with the same
constructor arguments, submodule names (so state dicts load either way) and
forward signatures:

  LinearMemoryCell                (reference grm/core/linear_attention.py:21-60)
  TopKMemoryRetriever             (grm/core/gating_unit.py:14-92)
  RetrievedStateFusion            (grm/core/aggregator.py:12-176)
  SegmentRecurrentMemoryModel     (grm/core/paper_grm.py:350-784)
  SegmentRecurrentMemoryLayer     (grm/core/multilayer_grm.py:12-102)
  HierarchicalSegmentMemoryModel  (grm/core/multilayer_grm.py:105-240)

The reference walks a sequence segment by segment (paper_grm.py:702-728):
update the memory over the segment, route the segment's tokens over the
archive as it stands, gather and apply the selected states, fuse, then push
the segment's end state and mean input.  Nothing the retrieval produces flows
back into the memory recurrence, and the archive a segment sees is fixed by
the segments before it, so one layer runs as five launches over the whole
sequence instead of five per segment:

  segment_scan_forward  every segment's outputs and end state (the snapshots)
  segment_route         each token routed over the archive of its segment's
                        moment: base + s entries, the last `capacity` kept
  gather_apply          selected archived states applied to the query
  fuse_residual         LayerNorm(h_online + sum_r g_r r_r)
                        (a 16-bit model runs the two as one retrieve_fuse)
  (projections and the output Linear stay library GEMMs)

Archive contents and the state format are the reference's: states are stored
in memory_storage_dtype after passing through the model dtype, summaries are
the segment means in the storage dtype, and the segment's starting state and
inputs are kept as checkpoints.

Differences, by design:
  - the memory state is carried in float32 between segments; a 16-bit model
    in the reference rounds it to the model dtype at every segment end;
  - routing ranks float32 scores (one FMA chain each, ties to the lower
    index); the reference ranks scores rounded to the model dtype with
    torch.topk, whose tie order is unspecified;
  - selective recompute (recomputation_ratio > 0) is not provided: the
    constructor raises, and the default is 0 (the reference's
    SegmentRecurrentMemoryModel defaults to 0.02; its hierarchical model and
    every benchmark configuration use 0).
With autograd enabled the fused retrieval ops, which have no backward, are
replaced by their differentiable compositions.
"""

from __future__ import annotations

import math
from dataclasses import dataclass
from typing import Any, Dict, List, Literal, Optional, Tuple

import torch
import torch.nn as nn
import torch.nn.functional as F
from torch import Tensor

from . import cuda_ops
from .archive import DeviceSegmentArchive, SegmentCheckpoint

_NORM_EPS = 1e-6

# Phase timing for benchmarks: when a list, every phase boundary of the
# whole-sequence forward appends (name, event) with an event recorded on the
# current stream; None (the default) records nothing.
PHASE_EVENTS: Optional[List[Tuple[str, Any]]] = None


def _mark(name: str, like: Tensor) -> None:
    if PHASE_EVENTS is not None and like.is_cuda:
        ev = torch.cuda.Event(enable_timing=True)
        ev.record()
        PHASE_EVENTS.append((name, ev))


def phase_times_ms() -> Dict[str, float]:
    """Milliseconds per phase name between consecutive marks of PHASE_EVENTS (after a
    synchronisation), summed over layers."""
    out: Dict[str, float] = {}
    evs = PHASE_EVENTS or []
    for (_, e0), (name, e1) in zip(evs, evs[1:]):
        out[name] = out.get(name, 0.0) + e0.elapsed_time(e1)
    return out


@dataclass
class LinearMemoryState:
    """Memory state of the linear cell (linear_attention.py:13-18)."""

    memory: Tensor
    h: Optional[Tensor] = None


class LinearMemoryCell(nn.Module):
    """The linear memory cell (linear_attention.py:21-167); same parameters and
    initialisation order as the reference.  Its recurrence runs on the chunked
    scan: a whole sequence is one launch instead of one step per token."""

    def __init__(self, input_size: int, hidden_size: int, memory_key_dim: Optional[int] = None,
                 use_bias: bool = True, memory_init: Literal["zeros", "eye", "random"] = "zeros",
                 memory_decay: float = 0.97):
        super().__init__()
        self.input_size = input_size
        self.hidden_size = hidden_size
        self.memory_key_dim = memory_key_dim or hidden_size
        self.use_bias = use_bias
        self.memory_init = memory_init
        self.memory_decay = memory_decay
        self.key_proj = nn.Linear(input_size, self.memory_key_dim, bias=use_bias)
        self.value_proj = nn.Linear(input_size, hidden_size, bias=use_bias)
        self.query_proj = nn.Linear(input_size, self.memory_key_dim, bias=use_bias)
        self.output_proj = nn.Linear(hidden_size, input_size, bias=use_bias)
        for proj in (self.key_proj, self.value_proj, self.query_proj):
            nn.init.xavier_uniform_(proj.weight)
            if proj.bias is not None:
                nn.init.zeros_(proj.bias)
        nn.init.xavier_uniform_(self.output_proj.weight)
        if self.output_proj.bias is not None:
            nn.init.zeros_(self.output_proj.bias)

    def init_memory(self, batch_size: int, device: torch.device,
                    dtype: torch.dtype = torch.float32) -> LinearMemoryState:
        shape = (batch_size, self.hidden_size, self.memory_key_dim)
        if self.memory_init == "zeros":
            memory = torch.zeros(shape, device=device, dtype=dtype)
        elif self.memory_init == "eye":
            eye = torch.eye(self.hidden_size, self.memory_key_dim, device=device, dtype=dtype)
            memory = eye.unsqueeze(0).expand(batch_size, -1, -1).clone()
        elif self.memory_init == "random":
            memory = torch.randn(shape, device=device, dtype=dtype) * 0.02
        else:
            raise ValueError(f"Unknown memory_init: {self.memory_init}")
        return LinearMemoryState(memory=memory)

    def forward(self, x_t: Tensor, state: Optional[LinearMemoryState] = None) -> Tuple[Tensor, LinearMemoryState]:
        """One token: M <- decay M + (1 - decay) v k^T / sqrt(d_k), h = M q, output_proj(h)
        (linear_attention.py:97-121)."""
        out, new_state = self.forward_sequence(x_t.unsqueeze(1), state)
        return out[:, 0], new_state

    def forward_sequence(self, x_seq: Tensor, state: Optional[LinearMemoryState] = None,
                         return_all_outputs: bool = True) -> Tuple[Tensor, LinearMemoryState]:
        """The per-token recurrence over x_seq [B, T, input] (linear_attention.py:123-167),
        as one chunked scan."""
        batch_size, seq_len, _ = x_seq.shape
        if state is None:
            state = self.init_memory(batch_size, x_seq.device, x_seq.dtype)
        memory = state.memory
        if seq_len == 0:
            hidden = torch.zeros(batch_size, self.hidden_size, device=x_seq.device, dtype=x_seq.dtype)
            output = self.output_proj(hidden)
            outputs = x_seq.new_zeros(batch_size, 0, self.input_size) if return_all_outputs else output
            return outputs, LinearMemoryState(memory=memory, h=hidden)
        k, v, q = self.project(x_seq)
        hidden, memory = cuda_ops.cuda_chunk_update(k, v, q, memory, self.memory_decay)
        outputs = self.output_proj(hidden)
        return (outputs if return_all_outputs else outputs[:, -1]), LinearMemoryState(memory=memory,
                                                                                     h=hidden[:, -1])

    def project(self, x: Tensor, extra: Optional[nn.Linear] = None) -> Tuple[Tensor, ...]:
        """Normalised keys, values and normalised queries of every token, as one
        GEMM over the concatenated weights; `extra` (a Linear on the same input)
        joins the same GEMM and its output is returned last."""
        mods = [self.key_proj, self.value_proj, self.query_proj] + ([extra] if extra is not None else [])
        weight, bias = self._concat_params(mods)
        extra_dim = extra.out_features if extra is not None else 0
        return cuda_ops.cuda_project_gemm(x, weight, bias, self.memory_key_dim, self.hidden_size, extra_dim, _NORM_EPS)

    def _concat_params(self, mods: List[nn.Linear]) -> Tuple[Tensor, Optional[Tensor]]:
        """The projections' weights and biases concatenated for one GEMM; without autograd
        the concatenation is kept until a parameter changes (in place or replaced)."""
        params = [p for m in mods for p in (m.weight, m.bias) if p is not None]
        cacheable = not (torch.is_grad_enabled() and any(p.requires_grad for p in params))
        key = tuple((id(p), p.data_ptr(), p._version, p.dtype, p.device) for p in params)
        cached = getattr(self, "_concat_cache", None)
        if cacheable and cached is not None and cached[0] == key:
            return cached[1], cached[2]
        weight = torch.cat([m.weight for m in mods], 0)
        if all(m.bias is None for m in mods):
            bias = None
        else:
            bias = torch.cat([m.bias if m.bias is not None else m.weight.new_zeros(m.out_features) for m in mods])
        if cacheable:
            self._concat_cache = (key, weight, bias)
        else:
            self._concat_cache = None
        return weight, bias


class TopKMemoryRetriever(nn.Module):
    """Top-k retriever over segment summary keys (gating_unit.py:14-116): same
    parameters, aliases and initialisation as the reference.  The models route
    whole sequences through `cuda_segment_route`; `forward` is the reference's
    per-query form."""

    def __init__(self, query_dim: int, key_dim: Optional[int] = None, hidden_dim: Optional[int] = None,
                 retrieval_top_k: int = 16, temperature: float = 1.0, use_causal_mask: bool = True,
                 dropout: float = 0.1) -> None:
        super().__init__()
        self.query_dim = query_dim
        self.key_dim = key_dim or query_dim
        self.hidden_dim = hidden_dim or query_dim
        self.retrieval_top_k = retrieval_top_k
        self.temperature = temperature
        self.use_causal_mask = use_causal_mask
        self.query_projection = nn.Linear(self.query_dim, self.hidden_dim, bias=False)
        self.key_projection = nn.Linear(self.key_dim, self.hidden_dim, bias=False)
        self.query_proj = self.query_projection
        self.key_proj = self.key_projection
        self.output_projection = (nn.Linear(self.hidden_dim, self.query_dim, bias=False)
                                  if self.hidden_dim != self.query_dim else None)
        self.dropout = nn.Dropout(dropout) if dropout > 0 else nn.Identity()
        self.scale = 1.0 / math.sqrt(self.hidden_dim)
        nn.init.xavier_uniform_(self.query_projection.weight)
        nn.init.xavier_uniform_(self.key_projection.weight)
        if self.output_projection is not None:
            nn.init.xavier_uniform_(self.output_projection.weight)

    def _scores(self, query: Tensor, keys: Tensor, segment_offset: int) -> Tensor:
        """Scaled projected dot products [B, S]; keys at or after segment_offset
        masked out when 0 < segment_offset < S (gating_unit.py:63-80)."""
        if keys.ndim == 2:
            keys = keys.unsqueeze(0).expand(query.size(0), -1, -1)
        pq = self.query_projection(query).unsqueeze(1)
        pk = self.key_projection(keys)
        scores = torch.matmul(pq, pk.transpose(-2, -1)).squeeze(1) * self.scale
        num_keys = keys.size(1)
        if self.use_causal_mask and 0 < segment_offset < num_keys:
            later = torch.arange(num_keys, device=query.device) >= segment_offset
            scores = scores.masked_fill(later.unsqueeze(0), float("-inf"))
        return scores

    def forward(self, query: Tensor, keys: Tensor, segment_offset: int = 0,
                attention_mask: Optional[Tensor] = None) -> Tuple[Tensor, Tensor, Tensor]:
        """One query per batch row against S keys: (routing weights, indices, scores)
        (gating_unit.py:54-91).  k < S: the top k, descending; k >= S: every key in index order."""
        scores = self._scores(query, keys, 0)
        if attention_mask is not None:
            scores = scores.masked_fill(~attention_mask.bool(), float("-inf"))
        num_keys = scores.size(1)
        if self.use_causal_mask and 0 < segment_offset < num_keys:
            later = torch.arange(num_keys, device=query.device) >= segment_offset
            scores = scores.masked_fill(later.unsqueeze(0), float("-inf"))
        routes = min(self.retrieval_top_k, num_keys)
        if routes < num_keys:
            top, idx = torch.topk(scores, k=routes, dim=-1)
        else:
            top = scores
            idx = torch.arange(num_keys, device=query.device).unsqueeze(0).expand(query.size(0), -1)
        weights = self.dropout(F.softmax(top / self.temperature, dim=-1))
        return weights, idx, scores

    def compute_dense_routing_weights(self, query: Tensor, keys: Tensor, segment_offset: int = 0) -> Tensor:
        """Softmax over every (unmasked) key (gating_unit.py:93-116)."""
        return F.softmax(self._scores(query, keys, segment_offset) / self.temperature, dim=-1)


class RetrievedStateFusion(nn.Module):
    """Fusion rules of aggregator.py:12-176, same parameters.  Residual mode
    without an output projection runs as one fused kernel; the other rules
    are the reference's torch compositions."""

    def __init__(self, hidden_size: int,
                 retrieval_fusion_mode: Literal["residual", "concat", "gate", "linear", "memory_soup"] = "residual",
                 use_layer_norm: bool = True, use_output_projection: bool = False, dropout: float = 0.1) -> None:
        super().__init__()
        self.hidden_size = hidden_size
        self.retrieval_fusion_mode = retrieval_fusion_mode
        self.use_layer_norm = use_layer_norm
        self.layer_norm = nn.LayerNorm(hidden_size) if use_layer_norm else nn.Identity()
        self.dropout = nn.Dropout(dropout) if dropout > 0 else nn.Identity()
        self.output_projection: Optional[nn.Linear] = None
        self.gate_projection: Optional[nn.Linear] = None
        self.online_projection: Optional[nn.Linear] = None
        self.memory_projection: Optional[nn.Linear] = None
        self.soup_projection: Optional[nn.Linear] = None
        if retrieval_fusion_mode == "residual":
            if use_output_projection:
                self.output_projection = nn.Linear(hidden_size, hidden_size)
        elif retrieval_fusion_mode == "concat":
            self.output_projection = nn.Linear(hidden_size * 2, hidden_size)
        elif retrieval_fusion_mode == "gate":
            self.gate_projection = nn.Linear(hidden_size * 2, hidden_size)
        elif retrieval_fusion_mode == "linear":
            self.online_projection = nn.Linear(hidden_size, hidden_size, bias=False)
            self.memory_projection = nn.Linear(hidden_size, hidden_size, bias=False)
        elif retrieval_fusion_mode == "memory_soup":
            self.soup_projection = nn.Linear(hidden_size, hidden_size, bias=False)
        else:
            raise ValueError(f"Unknown retrieval_fusion_mode: {retrieval_fusion_mode}")
        for module in (self.output_projection, self.gate_projection, self.online_projection,
                       self.memory_projection, self.soup_projection):
            if module is None:
                continue
            nn.init.xavier_uniform_(module.weight)
            if getattr(module, "bias", None) is not None:
                nn.init.zeros_(module.bias)

    def fused_kernel_applies(self) -> bool:
        return self.retrieval_fusion_mode == "residual" and self.output_projection is None

    def combine(self, online: Tensor, retrieved: Tensor,
                routing_weights: Optional[Tensor] = None) -> Tuple[Tensor, Optional[Tensor]]:
        """Weighted sum of [B, R, H] retrieved states (aggregator.py:67-104): uniform weights when
        none are given; weights of another width are zero-padded or cut, then renormalised."""
        if retrieved.size(1) == 0:
            return torch.zeros_like(online), None
        batch, routes, _ = retrieved.shape
        w = routing_weights
        if w is None:
            w = torch.full((batch, routes), 1.0 / routes, device=online.device, dtype=online.dtype)
        if w.dim() == 1:
            w = w.unsqueeze(0)
        if w.size(0) == 1 and batch > 1:
            w = w.expand(batch, -1)
        if w.size(1) != routes:
            if w.size(1) < routes:
                w = torch.cat([w, w.new_zeros(batch, routes - w.size(1))], dim=-1)
            else:
                w = w[:, :routes]
            w = w / w.sum(dim=-1, keepdim=True).clamp(min=1e-9)
        return (retrieved * w.unsqueeze(-1)).sum(dim=1), w

    @staticmethod
    def _states(online_state, retrieved_states, routing_weights, legacy: dict):
        online_state = legacy.pop("h_online", None) if online_state is None else online_state
        retrieved_states = legacy.pop("cached_states", None) if retrieved_states is None else retrieved_states
        routing_weights = legacy.pop("gates", None) if routing_weights is None else routing_weights
        if legacy:
            raise TypeError(f"Unexpected keyword arguments: {', '.join(sorted(legacy))}")
        if online_state is None or retrieved_states is None:
            raise TypeError("`online_state` and `retrieved_states` must be provided.")
        return online_state, retrieved_states, routing_weights

    def forward(self, online_state: Optional[Tensor] = None, retrieved_states: Optional[Tensor] = None,
                routing_weights: Optional[Tensor] = None, **legacy_kwargs) -> Tensor:
        """Fused state [B, H] (aggregator.py:147-176); accepts the legacy names h_online,
        cached_states and gates."""
        online, retrieved, weights = self._states(online_state, retrieved_states, routing_weights, legacy_kwargs)
        contribution, weights = self.combine(online, retrieved, weights)
        return self.apply_rule(online, contribution, retrieved, weights)

    def forward_with_auxiliary_statistics(self, online_state: Optional[Tensor] = None,
                                          retrieved_states: Optional[Tensor] = None,
                                          routing_weights: Optional[Tensor] = None,
                                          **legacy_kwargs) -> Tuple[Tensor, Dict[str, float]]:
        """The fused state plus norms, route count and routing entropy (aggregator.py:178-218)."""
        online, retrieved, weights = self._states(online_state, retrieved_states, routing_weights, legacy_kwargs)
        contribution, weights = self.combine(online, retrieved, weights)
        fused = self.apply_rule(online, contribution, retrieved, weights)
        entropy = 0.0 if weights is None else float(
            (-(weights * torch.log(weights.clamp(min=1e-10))).sum(dim=-1).mean()).item())
        stats = {"online_norm": float(online.norm().item()), "retrieved_norm": float(contribution.norm().item()),
                 "num_retrieved": int(retrieved.size(1)), "routing_entropy": entropy}
        return fused, stats

    def apply_rule(self, online: Tensor, contribution: Tensor, retrieved: Tensor, gates: Tensor) -> Tensor:
        """_apply_fusion_rule (aggregator.py:106-145) on [..., hidden] rows; retrieved [..., R, hidden]."""
        mode = self.retrieval_fusion_mode
        if mode == "residual":
            fused = online + contribution
            if self.output_projection is not None:
                fused = self.output_projection(fused)
        elif mode == "concat":
            fused = self.output_projection(torch.cat([online, contribution], dim=-1))
        elif mode == "gate":
            gate = torch.sigmoid(self.gate_projection(torch.cat([online, contribution], dim=-1)))
            fused = gate * online + (1.0 - gate) * contribution
        elif mode == "linear":
            fused = self.online_projection(online) + self.memory_projection(contribution)
        else:  # memory_soup
            if retrieved.size(-2) == 0:
                soup_input = online
            else:
                w = gates
                if w is None:
                    w = torch.full(retrieved.shape[:-1], 1.0 / max(1, retrieved.size(-2)), device=online.device,
                                   dtype=online.dtype)
                soup_input = online + (retrieved * w.unsqueeze(-1)).sum(dim=-2)
            fused = self.soup_projection(soup_input)
        return self.dropout(self.layer_norm(fused))


class ParameterMixtureFusion(nn.Module):
    """LayerNorm(h + mean over layers l of sum_r g_r (w_l * r_r)) (aggregator.py:221-264)."""

    def __init__(self, hidden_size: int, num_memory_layers: int = 2, segment_pooling_mode: str = "mean",
                 use_layer_norm: bool = True, dropout: float = 0.1) -> None:
        super().__init__()
        self.hidden_size = hidden_size
        self.num_memory_layers = num_memory_layers
        self.segment_pooling_mode = segment_pooling_mode
        self.segment_weights = nn.ParameterList(
            [nn.Parameter(torch.full((hidden_size,), 0.1)) for _ in range(num_memory_layers)])
        self.layer_norm = nn.LayerNorm(hidden_size) if use_layer_norm else nn.Identity()
        self.dropout = nn.Dropout(dropout) if dropout > 0 else nn.Identity()

    def forward(self, online_state: Tensor, retrieved_states: Tensor,
                routing_weights: Optional[Tensor] = None) -> Tensor:
        if retrieved_states.size(1) == 0:
            return self.dropout(self.layer_norm(online_state))
        batch, routes, _ = retrieved_states.shape
        w = routing_weights
        if w is None:
            w = torch.full((batch, routes), 1.0 / routes, device=online_state.device, dtype=online_state.dtype)
        mixed = [((retrieved_states * sw.view(1, 1, -1)) * w.unsqueeze(-1)).sum(dim=1) for sw in self.segment_weights]
        mixture = mixed[0] if len(mixed) == 1 else torch.stack(mixed, dim=0).mean(dim=0)
        return self.dropout(self.layer_norm(online_state + mixture))


def _segment_means(x: Tensor, seg: int) -> Tensor:
    """Mean input of every segment, [B, n_seg, D] (paper_grm.py:546-547)."""
    B, T, D = x.shape
    full = T // seg
    parts = []
    if full:
        parts.append(x[:, :full * seg].reshape(B, full, seg, D).mean(dim=2))
    if T % seg:
        parts.append(x[:, full * seg:].mean(dim=1, keepdim=True))
    return torch.cat(parts, dim=1)


class SegmentRecurrentMemoryModel(nn.Module):
    """Same constructor and forward contract as the reference's
    SegmentRecurrentMemoryModel (paper_grm.py:350-784); one sequence runs as
    whole-sequence launches (module docstring)."""

    def __init__(self, input_size: int, hidden_size: int, output_size: int, rnn_type: Literal["linear"] = "linear",
                 segment_length: int = 64, memory_capacity_segments: int = 64, retrieval_top_k: int = 4,
                 memory_storage_dtype: torch.dtype = torch.float16, recomputation_ratio: float = 0.0,
                 segment_pooling_mode: Literal["mean", "max", "attention", "weighted"] = "mean",
                 retrieval_fusion_mode: Literal["residual", "concat", "gate", "linear", "memory_soup"] = "residual",
                 use_layer_norm: bool = True, dropout: float = 0.0, batch_first: bool = True,
                 memory_key_dim: Optional[int] = None,
                 memory_initialization_mode: Literal["checkpoint", "independent"] = "checkpoint",
                 retrieval_query_source: Literal["input"] = "input",
                 segment_summary_source: Literal["input_mean"] = "input_mean", memory_decay: float = 0.97,
                 **kwargs):
        super().__init__()
        if rnn_type != "linear":
            raise ValueError("The active GRM architecture only supports rnn_type='linear'. "
                             "Legacy GRU/LSTM/RNN backends have been retired.")
        if retrieval_query_source != "input" or segment_summary_source != "input_mean":
            raise ValueError("The active paper backend supports only retrieval_query_source='input' and "
                             "segment_summary_source='input_mean'.")
        if segment_pooling_mode != "mean":
            raise ValueError("The active paper backend supports only mean segment summaries.")
        if recomputation_ratio > 0.0:
            raise NotImplementedError("selective recompute (recomputation_ratio > 0) is not provided; use 0")
        self.input_size = input_size
        self.hidden_size = hidden_size
        self.output_size = output_size
        self.rnn_type = rnn_type
        self.segment_length = segment_length
        self.memory_capacity_segments = memory_capacity_segments
        self.retrieval_top_k = retrieval_top_k
        self.batch_first = batch_first
        self.memory_key_dim = memory_key_dim or max(16, hidden_size // 8)
        self.memory_initialization_mode = memory_initialization_mode
        self.retrieval_query_source = retrieval_query_source
        self.segment_summary_source = segment_summary_source
        self.memory_decay = memory_decay
        self.retrieval_fusion_mode = retrieval_fusion_mode
        self.enable_activation_checkpointing = bool(kwargs.pop("enable_activation_checkpointing", False))
        removed = [k for k in ("use_torch_compile", "torch_compile_mode", "use_triton_kernels", "use_cuda_cpp_kernels")
                   if k in kwargs]
        if removed:
            raise TypeError(f"Removed runtime arguments: {', '.join(sorted(removed))}. "
                            "The active GRM runtime always uses the CUDA C++ op wrapper path.")
        self.cuda_cpp_debug_fallback = bool(kwargs.pop("cuda_cpp_debug_fallback", False))

        self.memory_cell = LinearMemoryCell(input_size=input_size, hidden_size=hidden_size,
                                            memory_key_dim=self.memory_key_dim, memory_init="zeros")
        self.gating_unit = TopKMemoryRetriever(query_dim=input_size, key_dim=input_size, hidden_dim=input_size,
                                               retrieval_top_k=retrieval_top_k, use_causal_mask=True, dropout=dropout)
        self.aggregator = RetrievedStateFusion(
            hidden_size=hidden_size,
            retrieval_fusion_mode=retrieval_fusion_mode if retrieval_fusion_mode != "memory_soup" else "residual",
            use_layer_norm=use_layer_norm, dropout=dropout)
        self.memory_soup_norm = (nn.LayerNorm(hidden_size) if retrieval_fusion_mode == "memory_soup" and use_layer_norm
                                 else nn.Identity())
        self.output_proj = nn.Linear(hidden_size, output_size)
        self.memory_bank = DeviceSegmentArchive(hidden_size=hidden_size, memory_key_dim=self.memory_key_dim,
                                                summary_size=input_size, max_segments=memory_capacity_segments,
                                                memory_storage_dtype=memory_storage_dtype,
                                                recomputation_ratio=recomputation_ratio)
        self.dropout = nn.Dropout(dropout) if dropout > 0 else nn.Identity()

    # ------------------------------------------------------------- reference API
    def get_runtime_optimization_status(self, device_type: Optional[str] = None) -> Dict[str, Any]:
        return {
            "runtime_path": "cuda_cpp",
            "cuda_cpp_enabled": True,
            "cuda_cpp_debug_fallback": self.cuda_cpp_debug_fallback,
            "cuda_cpp_runtime": cuda_ops.get_grm_cuda_runtime_status(),
            "device_type": device_type or str(self.output_proj.weight.device.type),
        }

    def _init_memory(self, batch_size: int, device: torch.device, dtype: torch.dtype) -> Tensor:
        return self.memory_cell.init_memory(batch_size, device, dtype).memory

    def clear_memory(self) -> None:
        self.memory_bank.clear()

    def get_num_segments(self) -> int:
        return self.memory_bank.get_num_segments()

    def get_memory_info(self) -> Dict[str, float]:
        return self.memory_bank.get_memory_info()

    def init_hidden(self, batch_size: int, device: torch.device) -> Tuple[Tensor, Tensor]:
        h_init = torch.zeros(batch_size, self.hidden_size, device=device)
        return h_init, self._init_memory(batch_size, device, h_init.dtype)

    # ------------------------------------------------------------- sequence path
    def _scan(self, k: Tensor, v: Tensor, q: Tensor, memory: Tensor) -> Tuple[Tensor, Tensor, Tensor]:
        """Online outputs, final memory and the end state of every segment."""
        seg = self.segment_length
        run = lambda kk, vv, qq, mm: cuda_ops.cuda_segment_scan(  # noqa: E731
            kk, vv, qq, mm, self.memory_decay, seg, debug_fallback=self.cuda_cpp_debug_fallback)
        if self.memory_initialization_mode != "independent":
            return run(k, v, q, memory)
        # Every segment after the first starts from the initial memory again
        # (paper_grm.py:726-727): segments become independent sequences.
        B, T, _ = k.shape
        outs, snaps = [], []
        h0, _, s0 = run(k[:, :seg], v[:, :seg], q[:, :seg], memory)
        outs.append(h0)
        snaps.append(s0)
        full = T // seg
        if full > 1:
            n = full - 1
            fold = lambda t: t[:, seg:full * seg].reshape(B * n, seg, t.size(-1))  # noqa: E731
            zero = self._init_memory(B * n, memory.device, memory.dtype)
            h1, _, s1 = run(fold(k), fold(v), fold(q), zero)
            outs.append(h1.reshape(B, n * seg, -1))
            snaps.append(s1.reshape(B, n, *s1.shape[2:]))
        if T > seg and T % seg:
            t0 = full * seg
            h2, _, s2 = run(k[:, t0:], v[:, t0:], q[:, t0:], self._init_memory(B, memory.device, memory.dtype))
            outs.append(h2)
            snaps.append(s2)
        return torch.cat(outs, 1), self._init_memory(B, memory.device, memory.dtype), torch.cat(snaps, 1)

    def _float32_norm_params(self, weight: Optional[Tensor],
                             bias: Optional[Tensor]) -> Tuple[Optional[Tensor], Optional[Tensor]]:
        """float32 copies of 16-bit LayerNorm parameters for the fused kernel, made again
        only when a parameter changed (its storage or its in-place version), so that a
        forward does not convert them on every call."""
        key = tuple((t.data_ptr(), t._version, t.dtype) if t is not None else None for t in (weight, bias))
        cached = getattr(self, "_norm_f32", None)
        if cached is None or cached[0] != key:
            # the sources are held too, so that no other tensor can take their addresses
            # while the copies are in use
            src = tuple(None if t is None else t.detach() for t in (weight, bias))
            cached = (key, None if weight is None else weight.detach().float(),
                      None if bias is None else bias.detach().float(), src)
            self._norm_f32 = cached
        return cached[1], cached[2]

    def _retrieve(self, x: Tensor, q: Tensor, q_r: Tensor, h_online: Tensor, states: Tensor, summaries: Tensor,
                  base: int) -> Tensor:
        """Routing, retrieval and fusion for every token at once
        (paper_grm.py:613-643 per segment).  states/summaries hold the archive
        before this sequence (base entries) followed by this sequence's segments."""
        B, T, _ = x.shape
        seg, cap = self.segment_length, self.memory_capacity_segments
        gu = self.gating_unit
        grad = torch.is_grad_enabled() and any(p.requires_grad for p in self.parameters())
        k_r = gu.key_proj(summaries.to(x.dtype))
        top_k = min(self.retrieval_top_k, cap)
        _mark("routing key projection", x)
        gates, idx, _ = cuda_ops.cuda_segment_route(q_r, k_r, top_k, seg, base, cap, gu.scale, gu.temperature,
                                                    debug_fallback=self.cuda_cpp_debug_fallback)
        _mark("segment routing (score, top-k, softmax)", x)
        idx0 = idx.clamp(min=0)
        if grad:
            filled = idx >= 0
            # Differentiable gates: the selected scores again, as torch ops.  All scores
            # as one product (paper_grm.py:573), then the selected ones gathered: the
            # backward is a scatter into [B, T, S] and two GEMMs.  (Indexing k_r by the
            # [B, T, k] indices instead makes the backward an index_put with many
            # repeated indices, tens of ms per layer at 4 x 8192 tokens.)  float32
            # operands, with the keys' transpose materialised, keep the batched
            # products and their backward off 16-bit transposed views.
            scores_all = torch.matmul(q_r.float(), k_r.float().transpose(1, 2).contiguous())
            scores = scores_all.gather(-1, idx0) * gu.scale
            scores = scores.masked_fill(~filled, float("-inf"))
            gates = torch.softmax(scores.float() / gu.temperature, dim=-1).masked_fill(~filled, 0.0)
        gates = gu.dropout(gates)
        # Retrieval in float32 (paper_grm.py:227,301): a 16-bit q is passed as is, its
        # values exact in float32, which lets the kernel use exact 16-bit MFMA.
        q_in = q if q.dtype in (torch.bfloat16, torch.float16) else q.to(torch.float32)
        soup = self.retrieval_fusion_mode == "memory_soup"
        if soup or self.aggregator.fused_kernel_applies():
            norm = self.memory_soup_norm if soup else self.aggregator.layer_norm
            weight = norm.weight if isinstance(norm, nn.LayerNorm) else None
            bias = norm.bias if isinstance(norm, nn.LayerNorm) else None
            eps = norm.eps if isinstance(norm, nn.LayerNorm) else 1e-5
            if grad:
                # Training: float32 retrieval rows, residual and LayerNorm in one autograd
                # function whose backward takes M^T dx per query and route on the GPU; only
                # the [B, T, H] pre-norm sum is kept for it, not the [B, T, k, H] rows.
                fused = cuda_ops.cuda_retrieve_fuse(states, idx0, q_in, gates, h_online, weight, bias, eps,
                                                    debug_fallback=self.cuda_cpp_debug_fallback)
            elif q.dtype in (torch.bfloat16, torch.float16):
                # A 16-bit model: retrieval, gate-weighted sum, residual and LayerNorm in one
                # op over the routing windows: each block of tokens walks its window of
                # archive entries and sums its routes in float32, the sums kept as
                # tile-scaled float16 (relative rounding 2^-11) for the LayerNorm pass.
                w32, b32 = self._float32_norm_params(weight, bias)
                fused = cuda_ops.cuda_segment_retrieve_fuse(states, idx, q_in, gates.float(), h_online, w32, b32,
                                                            eps, seg, base, cap,
                                                            debug_fallback=self.cuda_cpp_debug_fallback)
            else:
                H = h_online.size(-1)
                retrieved = cuda_ops.cuda_gather_apply(states, idx0, q_in, torch.float32,
                                                       debug_fallback=self.cuda_cpp_debug_fallback)
                fused = cuda_ops.cuda_fuse_residual(h_online.float().reshape(B * T, H),
                                                    retrieved.reshape(B * T, -1, H), gates.reshape(B * T, -1),
                                                    None if weight is None else weight.float(),
                                                    None if bias is None else bias.float(), eps,
                                                    debug_fallback=self.cuda_cpp_debug_fallback).view(B, T, H)
            fused = (self.dropout if soup else self.aggregator.dropout)(fused)
        else:
            retrieved = cuda_ops.cuda_gather_apply(states, idx0, q_in, torch.float32,
                                                   debug_fallback=self.cuda_cpp_debug_fallback)
            contribution = (retrieved * gates.unsqueeze(-1)).sum(dim=2)
            if h_online.dtype != contribution.dtype:
                # A 16-bit model: its fusion layers hold 16-bit parameters, so the float32
                # retrieval enters them in the model's dtype.
                contribution, retrieved, gates = (t.to(h_online.dtype) for t in (contribution, retrieved, gates))
            if soup:
                fused = self.dropout(self.memory_soup_norm(h_online + contribution))
            else:
                fused = self.aggregator.apply_rule(h_online, contribution, retrieved, gates)
        _mark("retrieval (gather, apply, fuse, residual + LayerNorm)", x)
        fused = fused.to(h_online.dtype)
        if base == 0:  # the first segment found an empty archive: h_online unchanged
            if fused.requires_grad:
                fused = torch.cat([h_online[:, :seg], fused[:, seg:]], dim=1)
            else:
                fused[:, :seg] = h_online[:, :seg]
        return fused

    def forward(self, x_seq: Tensor, h_init: Optional[Tensor] = None, c_init: Optional[Tensor] = None,
                return_all_outputs: bool = True, return_hidden_states: bool = False,
                reset_memory: bool = False) -> Tuple[Tensor, Tensor, Optional[Tensor], Optional[Dict[str, Any]]]:
        return self._forward_impl(x_seq, h_init, c_init, return_all_outputs, return_hidden_states, reset_memory)

    def _forward_impl(self, x_seq: Tensor, h_init: Optional[Tensor], c_init: Optional[Tensor],
                      return_all_outputs: bool, return_hidden_states: bool, reset_memory: bool,
                      out_norm: Optional[Tuple[Tensor, nn.LayerNorm]] = None
                      ) -> Tuple[Tensor, Tensor, Optional[Tensor], Optional[Dict[str, Any]]]:
        """forward(); with out_norm = (residual, norm) and all outputs returned, the output is
        norm(output_proj(h) + residual) instead of output_proj(h): SegmentRecurrentMemoryLayer's
        block output (multilayer_grm.py:92-97) as the epilogue of the output projection's GEMM."""
        if x_seq.ndim == 2:
            x_seq = x_seq.unsqueeze(1 if self.batch_first else 0)
        x = x_seq if self.batch_first else x_seq.transpose(0, 1)
        B, T, _ = x.shape
        device, dtype = x.device, x.dtype
        if reset_memory:
            self.clear_memory()
        memory = c_init if (c_init is not None and c_init.ndim == 3) else self._init_memory(B, device, dtype)
        last_hidden = (h_init if (h_init is not None and h_init.ndim == 2)
                       else torch.zeros(B, self.hidden_size, device=device, dtype=dtype))

        def aux_dict(hidden: Optional[Tensor]) -> Dict[str, Any]:
            aux = {"memory_info": self.memory_bank.get_memory_info(),
                   "num_segments": self.memory_bank.get_num_segments(B),
                   "recompute_rate": self.memory_bank.get_recompute_rate()}
            if return_hidden_states:
                aux["hidden_states"] = hidden if self.batch_first else hidden.transpose(0, 1)
            return aux

        if T == 0:
            if return_all_outputs:
                out = x.new_zeros(B, 0, self.output_size)
                out = out if self.batch_first else out.transpose(0, 1)
            else:
                out = torch.zeros(B, self.output_size, device=device, dtype=dtype)
            return out, last_hidden, memory, aux_dict(x.new_zeros(B, 0, self.hidden_size))

        seg = self.segment_length
        _mark("other (between phases)", x)
        k, v, q, q_r = self.memory_cell.project(x, self.gating_unit.query_proj)
        _mark("projection GEMM + k/q normalise", x)
        h_online, memory_end, snaps = self._scan(k, v, q, memory)
        h_online = self.dropout(h_online)
        _mark("scan (chunk update + query, snapshots)", x)

        # The archive every segment of this sequence reads from: what was kept
        # before (deque order) followed by this sequence's segments, each state
        # through the model dtype into the storage dtype as push() stores it,
        # detached as the archive holds it (paper_grm.py:139-140): retrieval
        # passes no gradient back into the scan or the summaries' inputs.
        bank = self.memory_bank
        storage = bank.memory_storage_dtype
        new_states = cuda_ops.cuda_archive_cast(snaps.detach(), dtype, storage,
                                                debug_fallback=self.cuda_cpp_debug_fallback)  # what push() stores
        new_summaries = _segment_means(x.detach(), seg).to(storage)
        ring = bank._groups.get(B)
        base = 0 if ring is None else len(ring)
        if base:
            order = ring.order(ring.memories.device)
            states = torch.cat([ring.memories.index_select(1, order), new_states], dim=1)
            summaries = torch.cat([ring.summaries.index_select(1, order), new_summaries], dim=1)
        else:
            states, summaries = new_states, new_summaries
        n_seg = new_states.size(1)
        _mark("archive states and summaries (conversions, segment means)", x)
        if base + n_seg > 1:
            h_enhanced = self._retrieve(x, q, q_r, h_online, states, summaries, base)
        else:
            h_enhanced = h_online
        if out_norm is not None:
            residual, norm = out_norm
            if not self.batch_first:
                residual = residual.transpose(0, 1)
            y = cuda_ops.cuda_linear_residual_layer_norm(h_enhanced, self.output_proj.weight, self.output_proj.bias,
                                                         residual, norm.weight, norm.bias, norm.eps,
                                                         debug_fallback=self.cuda_cpp_debug_fallback)
            _mark("output projection GEMM + layer residual + LayerNorm", x)
        else:
            y = self.output_proj(h_enhanced)
            _mark("output projection GEMM", x)

        # Push every segment (paper_grm.py:718-724); only the last `capacity` survive.
        # Checkpoints of the kept segments: one time-major copy of their inputs
        # and one stack of their starting states, sliced per segment.
        cap = self.memory_capacity_segments
        first = max(0, n_seg - cap)
        inputs = x.detach()[:, first * seg:].transpose(0, 1).contiguous()
        if self.memory_initialization_mode == "independent":
            starts = torch.zeros((n_seg - first,) + tuple(memory.shape), dtype=storage, device=device)
        else:
            # the end states of the previous segments, as stored (views of new_states)
            prev = new_states[:, max(first - 1, 0):n_seg - 1].transpose(0, 1)
            starts = torch.cat([memory.detach().to(dtype).to(storage).unsqueeze(0), prev], 0) if first == 0 else prev
        if first == 0:
            starts[0].copy_(memory.detach())
        checkpoints = [SegmentCheckpoint(inputs[(s - first) * seg:(s - first + 1) * seg], starts[s - first])
                       for s in range(first, n_seg)]
        bank.push_segments(new_states, new_summaries, checkpoints, owned=True)
        _mark("archive push (ring writes, checkpoints)", x)
        # Routes handed out, as the reference counts them per segment (paper_grm.py:230).
        routes = sum(B * (min(T, (s + 1) * seg) - s * seg) * min(self.retrieval_top_k, min(base + s, cap))
                     for s in range(n_seg))
        bank._count_retrieved(routes)

        last_hidden = h_enhanced[:, -1]
        if return_all_outputs:
            out = y if self.batch_first else y.transpose(0, 1).contiguous()
        else:
            out = y[:, -1]
        return out, last_hidden, memory_end, aux_dict(h_enhanced)

    def forward_incremental(self, x_seq: Tensor, incremental_state: Optional[Dict[str, Any]] = None,
                            h_init: Optional[Tensor] = None, c_init: Optional[Tensor] = None,
                            return_all_outputs: bool = True, reset_memory: bool = False,
                            **kwargs) -> Tuple[Tensor, Tensor, Optional[Tensor], Dict[str, Any]]:
        outputs, h_final, memory_final, _ = self.forward(x_seq=x_seq, h_init=h_init, c_init=c_init,
                                                         return_all_outputs=return_all_outputs,
                                                         return_hidden_states=False, reset_memory=reset_memory)
        state = dict(incremental_state or {})
        state["last_memory"] = memory_final
        return outputs, h_final, memory_final, state


class SegmentRecurrentMemoryLayer(nn.Module):
    """One block: segment-memory model, residual, LayerNorm, dropout (multilayer_grm.py:12-102)."""

    def __init__(self, input_size: int, hidden_size: int, rnn_type: Literal["linear"] = "linear",
                 segment_length: int = 64, memory_capacity_segments: int = 64, retrieval_top_k: int = 8,
                 memory_storage_dtype: torch.dtype = torch.float16, recomputation_ratio: float = 0.0,
                 retrieval_fusion_mode: str = "residual", use_layer_norm: bool = True, dropout: float = 0.1,
                 batch_first: bool = True, memory_key_dim: Optional[int] = None,
                 memory_initialization_mode: str = "checkpoint", retrieval_query_source: str = "input",
                 segment_summary_source: str = "input_mean", memory_decay: float = 0.97,
                 enable_activation_checkpointing: bool = False, cuda_cpp_debug_fallback: bool = False):
        super().__init__()
        if rnn_type != "linear":
            raise ValueError("SegmentRecurrentMemoryLayer currently supports only the linear-memory backend.")
        self.input_size = input_size
        self.hidden_size = hidden_size
        self.segment_length = segment_length
        self.batch_first = batch_first
        self.grm = SegmentRecurrentMemoryModel(
            input_size=input_size, hidden_size=hidden_size, output_size=input_size, rnn_type="linear",
            segment_length=segment_length, memory_capacity_segments=memory_capacity_segments,
            retrieval_top_k=retrieval_top_k, memory_storage_dtype=memory_storage_dtype,
            recomputation_ratio=recomputation_ratio, retrieval_fusion_mode=retrieval_fusion_mode,
            use_layer_norm=use_layer_norm, dropout=dropout, batch_first=batch_first, memory_key_dim=memory_key_dim,
            memory_initialization_mode=memory_initialization_mode, retrieval_query_source=retrieval_query_source,
            segment_summary_source=segment_summary_source, memory_decay=memory_decay,
            enable_activation_checkpointing=enable_activation_checkpointing,
            cuda_cpp_debug_fallback=cuda_cpp_debug_fallback)
        self.layer_norm = nn.LayerNorm(input_size) if use_layer_norm else nn.Identity()
        self.dropout = nn.Dropout(dropout) if dropout > 0 else nn.Identity()

    def forward(self, x: Tensor, h_init: Optional[Tensor] = None, c_init: Optional[Tensor] = None,
                return_all_outputs: bool = False, return_hidden_states: bool = False,
                reset_memory: bool = False) -> Tuple[Tensor, Tensor, Optional[Tensor], Optional[Dict]]:
        if x.ndim == 2:
            x = x.unsqueeze(1 if self.batch_first else 0)
        if return_all_outputs and isinstance(self.layer_norm, nn.LayerNorm):
            # the residual add and the LayerNorm run as the output projection's epilogue
            outputs, h_final, memory_final, aux = self.grm._forward_impl(
                x, h_init, c_init, True, return_hidden_states, reset_memory, out_norm=(x, self.layer_norm))
            return self.dropout(outputs), h_final, memory_final, aux
        outputs, h_final, memory_final, aux = self.grm(x, h_init=h_init, c_init=c_init,
                                                       return_all_outputs=return_all_outputs,
                                                       return_hidden_states=return_hidden_states,
                                                       reset_memory=reset_memory)
        _mark("other (between phases)", x)
        residual = x if return_all_outputs else (x[:, -1, :] if self.batch_first else x[-1, :, :])
        if isinstance(self.layer_norm, nn.LayerNorm):
            ln = self.layer_norm
            outputs = cuda_ops.cuda_residual_layer_norm(outputs, residual, ln.weight, ln.bias, ln.eps,
                                                        debug_fallback=self.grm.cuda_cpp_debug_fallback)
        else:
            outputs = self.layer_norm(outputs + residual)
        _mark("layer residual + LayerNorm", x)
        return self.dropout(outputs), h_final, memory_final, aux

    @property
    def memory_bank(self):
        return self.grm.memory_bank


class HierarchicalSegmentMemoryModel(nn.Module):
    """Stacked blocks and an output projection (multilayer_grm.py:105-240)."""

    def __init__(self, input_size: int, hidden_size: int, output_size: int, num_layers: int = 6,
                 rnn_type: Literal["linear"] = "linear", segment_length: int = 64,
                 memory_capacity_segments: int = 64, retrieval_top_k: int = 8,
                 memory_storage_dtype: torch.dtype = torch.float16, recomputation_ratio: float = 0.0,
                 retrieval_fusion_mode: str = "residual", use_layer_norm: bool = True, dropout: float = 0.1,
                 batch_first: bool = True, memory_key_dim: Optional[int] = None,
                 memory_initialization_mode: str = "checkpoint", retrieval_query_source: str = "input",
                 segment_summary_source: str = "input_mean", memory_decay: float = 0.97,
                 enable_activation_checkpointing: bool = False, cuda_cpp_debug_fallback: bool = False):
        super().__init__()
        if rnn_type != "linear":
            raise ValueError("HierarchicalSegmentMemoryModel currently supports only the linear-memory backend.")
        self.input_size = input_size
        self.hidden_size = hidden_size
        self.output_size = output_size
        self.num_layers = num_layers
        self.rnn_type = rnn_type
        self.batch_first = batch_first
        self.layers = nn.ModuleList([
            SegmentRecurrentMemoryLayer(
                input_size=input_size, hidden_size=hidden_size, rnn_type="linear", segment_length=segment_length,
                memory_capacity_segments=memory_capacity_segments, retrieval_top_k=retrieval_top_k,
                memory_storage_dtype=memory_storage_dtype, recomputation_ratio=recomputation_ratio,
                retrieval_fusion_mode=retrieval_fusion_mode, use_layer_norm=use_layer_norm, dropout=dropout,
                batch_first=batch_first, memory_key_dim=memory_key_dim,
                memory_initialization_mode=memory_initialization_mode,
                retrieval_query_source=retrieval_query_source, segment_summary_source=segment_summary_source,
                memory_decay=memory_decay, enable_activation_checkpointing=enable_activation_checkpointing,
                cuda_cpp_debug_fallback=cuda_cpp_debug_fallback)
            for _ in range(num_layers)
        ])
        self.output_proj = nn.Linear(input_size, output_size)
        self.dropout = nn.Dropout(dropout) if dropout > 0 else nn.Identity()

    def forward(self, x: Tensor, h_init: Optional[Tensor] = None, c_init: Optional[Tensor] = None,
                return_all_outputs: bool = True, return_hidden_states: bool = False,
                reset_memory: bool = False) -> Tuple[Tensor, Tensor, Optional[Tensor], Optional[Dict]]:
        batch_size = x.size(0) if self.batch_first else x.size(1)
        device = x.device
        if reset_memory:
            self.clear_memory()
        if h_init is None:
            h_init = torch.zeros(self.num_layers, batch_size, self.hidden_size, device=device, dtype=x.dtype)
        if c_init is None:
            c_init = torch.zeros(self.num_layers, batch_size, self.hidden_size, self.layers[0].grm.memory_key_dim,
                                 device=device, dtype=x.dtype)
        h_list: List[Tensor] = []
        c_list: List[Tensor] = []
        current, aux = x, None
        for i, layer in enumerate(self.layers):
            current, h_final, memory_final, aux = layer(current, h_init=h_init[i], c_init=c_init[i],
                                                        return_all_outputs=return_all_outputs,
                                                        return_hidden_states=return_hidden_states,
                                                        reset_memory=False)
            h_list.append(h_final)
            c_list.append(memory_final)
        outputs = self.dropout(self.output_proj(current))
        return outputs, torch.stack(h_list, dim=0), torch.stack(c_list, dim=0), aux

    def clear_memory(self) -> None:
        for layer in self.layers:
            layer.memory_bank.clear()

    def get_memory_info(self):
        return [layer.memory_bank.get_memory_info() for layer in self.layers]

    def get_runtime_optimization_status(self, device_type: Optional[str] = None) -> Dict[str, object]:
        return self.layers[0].grm.get_runtime_optimization_status(device_type=device_type)

    @property
    def memory_bank(self):
        return self.layers[0].memory_bank


def build_topk_memory_retriever(query_dim: int, key_dim: Optional[int] = None, retrieval_top_k: int = 16,
                                **kwargs) -> TopKMemoryRetriever:
    return TopKMemoryRetriever(query_dim=query_dim, key_dim=key_dim, retrieval_top_k=retrieval_top_k, **kwargs)


def build_retrieved_state_fusion(hidden_size: int, retrieval_fusion_mode: str = "residual",
                                 **kwargs) -> RetrievedStateFusion:
    return RetrievedStateFusion(hidden_size=hidden_size, retrieval_fusion_mode=retrieval_fusion_mode, **kwargs)


def build_segment_memory_model(input_size: int, hidden_size: int, output_size: int,
                               **kwargs) -> SegmentRecurrentMemoryModel:
    return SegmentRecurrentMemoryModel(input_size=input_size, hidden_size=hidden_size, output_size=output_size,
                                       **kwargs)


def build_hierarchical_segment_memory_model(input_size: int, hidden_size: int, output_size: int, num_layers: int = 6,
                                            **kwargs) -> HierarchicalSegmentMemoryModel:
    return HierarchicalSegmentMemoryModel(input_size=input_size, hidden_size=hidden_size, output_size=output_size,
                                          num_layers=num_layers, **kwargs)


__all__ = [
    "HierarchicalSegmentMemoryModel",
    "LinearMemoryCell",
    "LinearMemoryState",
    "ParameterMixtureFusion",
    "RetrievedStateFusion",
    "SegmentRecurrentMemoryLayer",
    "SegmentRecurrentMemoryModel",
    "TopKMemoryRetriever",
    "build_hierarchical_segment_memory_model",
    "build_retrieved_state_fusion",
    "build_segment_memory_model",
    "build_topk_memory_retriever",
]
