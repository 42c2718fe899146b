"""Write tests/golden/reference_cpu_ops.npz from the reference's own CPU ops.

Runs in this container only: it imports oracle/_ref/grm_ref_harness.so, which
oracle/ref/build_ref.py compiles from the reference's grm/csrc/grm_cuda.cpp
(the reference's CPU implementations: per-token at::bmm recurrence,
autograd backward, einsum apply-query, index_select gather).  The fixture
holds seeded inputs and the reference outputs, float64, so the oracle can be
pinned against the reference on machines without the reference.

Usage: python tests/golden/make_golden.py
"""

from __future__ import annotations

import importlib.util
import sys
from pathlib import Path

import numpy as np
import torch

HERE = Path(__file__).resolve().parent
REPO = HERE.parents[1]
HARNESS = REPO / "oracle" / "_ref" / "grm_ref_harness.so"
OUT = HERE / "reference_cpu_ops.npz"


def load_harness():
    spec = importlib.util.spec_from_file_location("grm_ref_harness", HARNESS)
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def main() -> int:
    if not HARNESS.exists():
        print(f"{HARNESS} missing; run python oracle/ref/build_ref.py first", file=sys.stderr)
        return 1
    ref = load_harness()
    torch.manual_seed(0)
    data = {}
    dt = torch.float64
    # chunk update: the reference's test shape (B=2, d_v=16, d_k=8) at several lengths and decays
    cases = [(2, 8, 8, 16, 0.97), (2, 64, 8, 16, 0.97), (3, 70, 32, 24, 0.9), (1, 130, 64, 64, 0.97),
             (2, 5, 4, 3, 0.0), (2, 9, 6, 5, 1.0)]
    for i, (B, T, K, H, decay) in enumerate(cases):
        g = torch.Generator().manual_seed(100 + i)
        k = torch.nn.functional.normalize(torch.randn(B, T, K, generator=g, dtype=dt), dim=-1)
        v = torch.randn(B, T, H, generator=g, dtype=dt)
        q = torch.nn.functional.normalize(torch.randn(B, T, K, generator=g, dtype=dt), dim=-1)
        m = torch.randn(B, H, K, generator=g, dtype=dt)
        dh = torch.randn(B, T, H, generator=g, dtype=dt)
        dm = torch.randn(B, H, K, generator=g, dtype=dt)
        h, mo, _ = ref.chunk_update_forward(k, v, q, m, decay)
        gk, gv, gq, gm = ref.chunk_update_backward(dh, dm, k, v, q, m, torch.empty(0, dtype=dt), decay)
        p = f"chunk{i}_"
        for name, t in (("keys", k), ("values", v), ("queries", q), ("memory", m), ("grad_hidden", dh),
                        ("grad_memory_out", dm), ("hidden", h), ("memory_out", mo), ("grad_keys", gk),
                        ("grad_values", gv), ("grad_queries", gq), ("grad_memory", gm)):
            data[p + name] = t.numpy()
        data[p + "decay"] = np.array(decay)
    # apply query: rank 5 at the reference's test shape, rank 4
    for i, shape in enumerate([(2, 3, 4, 5, 6), (3, 4, 7, 5)]):
        g = torch.Generator().manual_seed(200 + i)
        mm = torch.randn(*shape, generator=g, dtype=dt)
        qs = shape[:2] + shape[-1:] if len(shape) == 5 else (shape[0], shape[-1])
        qq = torch.nn.functional.normalize(torch.randn(*qs, generator=g, dtype=dt), dim=-1)
        dh = torch.randn(*shape[:-1], generator=g, dtype=dt)
        out = ref.apply_query_forward(mm, qq)
        gmm, gqq = ref.apply_query_backward(dh, mm, qq)
        p = f"apply{i}_"
        for name, t in (("memories", mm), ("queries", qq), ("grad_hidden", dh), ("hidden", out),
                        ("grad_memories", gmm), ("grad_queries", gqq)):
            data[p + name] = t.numpy()
    # gather: the fixed index tensors of the reference's own test (examples/test_grm.py:202-210)
    g = torch.Generator().manual_seed(300)
    mem = torch.randn(2, 7, 4, 5, generator=g, dtype=dt)
    idx3 = torch.tensor([[[1, 3], [2, 5], [0, 6]], [[4, 2], [1, 0], [3, 5]]], dtype=torch.long)
    idx2 = torch.tensor([[0, 2, 4], [1, 3, 5]], dtype=torch.long)
    data["gather_memories"] = mem.numpy()
    data["gather_idx3"] = idx3.numpy()
    data["gather_idx2"] = idx2.numpy()
    data["gather_out3"] = ref.batched_memory_gather(mem, idx3).numpy()
    data["gather_out2"] = ref.batched_memory_gather(mem, idx2).numpy()
    np.savez_compressed(OUT, **data)
    print(f"wrote {OUT} ({OUT.stat().st_size} bytes, {len(data)} arrays)")
    return 0


if __name__ == "__main__":
    sys.exit(main())
