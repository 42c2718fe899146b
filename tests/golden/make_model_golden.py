"""Write tests/golden/reference_models.npz: end-to-end forwards of the
reference's own segment-memory models at tiny shapes.

The closed forms pin every op on the hot path, but not how the reference's
models compose them: which archive entries a segment sees, when entries are
evicted, the float16 round trip of archived states and summaries, where the
LayerNorms and residuals sit, the first segment's bypass, the arange branch
of short archives, independent-memory mode and memory-soup fusion.  This
script runs the reference's models (grm/core/multilayer_grm.py,
grm/core/paper_grm.py) on the CPU of this container, in float32 with their
PyTorch fallbacks, and stores the seeded inputs, the models' weights and
their outputs, so the tests can load the same weights into the models of
this repository and compare, with no reference present.

Runs in this container only (the reference is not shipped).  Only the
reference's grm.core modules are imported: the grm package's own __init__,
which also imports its training utilities, is bypassed.

Usage: python tests/golden/make_model_golden.py
"""

from __future__ import annotations

import os
import sys
import types
from pathlib import Path

import numpy as np
import torch

HERE = Path(__file__).resolve().parent
OUT = HERE / "reference_models.npz"
REFERENCE = Path("/root/reference")


def import_reference_core():
    os.environ["GRM_CUDA_KERNEL_POLICY"] = "fallback"
    pkg = types.ModuleType("grm")
    pkg.__path__ = [str(REFERENCE / "grm")]
    sys.modules["grm"] = pkg
    from grm.core import multilayer_grm, paper_grm  # noqa: E402

    return multilayer_grm, paper_grm


def flat_state(prefix: str, module: torch.nn.Module, data: dict) -> None:
    for name, t in module.state_dict().items():
        if isinstance(t, torch.Tensor):
            data[f"{prefix}w:{name}"] = t.detach().numpy()


def archive_state(prefix: str, bank, data: dict) -> None:
    for bsz, group in bank.get_extra_state()["groups"].items():
        data[f"{prefix}arch_mem"] = torch.stack(group["memories"], 1).float().numpy()
        data[f"{prefix}arch_sum"] = torch.stack(group["summaries"], 1).float().numpy()
        data[f"{prefix}arch_ckpt_in"] = torch.cat([c["inputs"] for c in group["checkpoints"]], 0).numpy()
        data[f"{prefix}arch_ckpt_len"] = np.array([c["inputs"].size(0) for c in group["checkpoints"]])
        data[f"{prefix}arch_ckpt_m0"] = torch.stack([c["memory_start"] for c in group["checkpoints"]], 0).float().numpy()


def run_cases(multilayer_grm, paper_grm, storage: torch.dtype, tag: str, data: dict) -> None:
    """The three cases below with archived states and summaries kept in `storage`."""
    # Case A: hierarchical stack, residual fusion, checkpoint memory, two calls
    # (the second starts from a full archive: eviction and base > 0).
    torch.manual_seed(0)
    model = multilayer_grm.HierarchicalSegmentMemoryModel(
        input_size=32, hidden_size=24, output_size=16, num_layers=2, segment_length=8, memory_capacity_segments=5,
        retrieval_top_k=3, memory_key_dim=8, dropout=0.0, recomputation_ratio=0.0,
        memory_storage_dtype=storage).eval()
    p = f"A{tag}_"
    flat_state(p, model, data)
    g = torch.Generator().manual_seed(1)
    x1 = torch.randn(2, 61, 32, generator=g)
    x2 = torch.randn(2, 27, 32, generator=g)
    with torch.no_grad():
        o1, h1, c1, _ = model(x1)
        o2, h2, c2, _ = model(x2)
    for name, t in (("x1", x1), ("x2", x2), ("out1", o1), ("h1", h1), ("c1", c1), ("out2", o2), ("h2", h2),
                    ("c2", c2)):
        data[p + name] = t.numpy()
    archive_state(p + "L1_", model.layers[1].memory_bank, data)

    # Case B: one SegmentRecurrentMemoryModel, time-major input, memory-soup
    # fusion, independent memory per segment, hidden states returned.
    torch.manual_seed(3)
    single = paper_grm.SegmentRecurrentMemoryModel(
        input_size=20, hidden_size=16, output_size=12, segment_length=6, memory_capacity_segments=4,
        retrieval_top_k=2, memory_key_dim=8, dropout=0.0, recomputation_ratio=0.0,
        retrieval_fusion_mode="memory_soup", memory_initialization_mode="independent", batch_first=False,
        memory_storage_dtype=storage).eval()
    p = f"B{tag}_"
    flat_state(p, single, data)
    x = torch.randn(40, 3, 20, generator=g)
    c0 = torch.randn(3, 16, 8, generator=g) * 0.1
    with torch.no_grad():
        o, h, c, aux = single(x, c_init=c0, return_hidden_states=True)
    for name, t in (("x", x), ("c0", c0), ("out", o), ("h", h), ("c", c), ("hidden", aux["hidden_states"])):
        data[p + name] = t.numpy()
    data[p + "num_segments"] = np.array(aux["num_segments"])

    # Case C: the last output only, for a sequence shorter than one segment
    # after a longer one (a one-segment call reading a part-full archive).
    torch.manual_seed(5)
    short = paper_grm.SegmentRecurrentMemoryModel(
        input_size=16, hidden_size=16, output_size=8, segment_length=10, memory_capacity_segments=8,
        retrieval_top_k=4, memory_key_dim=16, dropout=0.0, recomputation_ratio=0.0,
        memory_storage_dtype=storage).eval()
    p = f"C{tag}_"
    flat_state(p, short, data)
    xa = torch.randn(2, 35, 16, generator=g)
    xb = torch.randn(2, 7, 16, generator=g)
    with torch.no_grad():
        oa, ha, ca, _ = short(xa)
        ob, hb, cb, _ = short(xb, return_all_outputs=False)
    for name, t in (("xa", xa), ("xb", xb), ("outa", oa), ("outb", ob), ("hb", hb), ("cb", cb)):
        data[p + name] = t.numpy()


def main() -> int:
    multilayer_grm, paper_grm = import_reference_core()
    data = {}
    # float16 archives (the reference's default) and float32 archives (its
    # trainer's stage 1): the float32 ones pin the composition without the
    # float16 round trip, whose rounding boundaries a different float32
    # evaluation order can cross.
    run_cases(multilayer_grm, paper_grm, torch.float16, "16", data)
    run_cases(multilayer_grm, paper_grm, torch.float32, "32", data)
    np.savez_compressed(OUT, **data)
    print(f"wrote {OUT} ({OUT.stat().st_size} bytes, {len(data)} arrays)")
    return 0


if __name__ == "__main__":
    sys.exit(main())
