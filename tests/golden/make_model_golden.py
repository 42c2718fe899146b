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


def gradient_case(multilayer_grm, data: dict) -> None:
    """Case G: the hierarchical model of case A in training mode (dropout 0,
    float32 archive), two calls, the second reading the first's archive; the
    gradient of the summed squared outputs for every parameter."""
    torch.manual_seed(7)
    model = multilayer_grm.HierarchicalSegmentMemoryModel(
        input_size=32, hidden_size=24, output_size=16, num_layers=2, segment_length=8, memory_capacity_segments=5,
        retrieval_top_k=3, memory_key_dim=8, dropout=0.0, recomputation_ratio=0.0,
        memory_storage_dtype=torch.float32).train()
    flat_state("G_", model, data)
    g = torch.Generator().manual_seed(8)
    x1 = torch.randn(2, 43, 32, generator=g)
    x2 = torch.randn(2, 21, 32, generator=g)
    o1, _, _, _ = model(x1)
    o2, _, _, _ = model(x2)
    (o1.square().mean() + o2.square().mean()).backward()
    data["G_x1"], data["G_x2"] = x1.numpy(), x2.numpy()
    data["G_out1"], data["G_out2"] = o1.detach().numpy(), o2.detach().numpy()
    for name, prm in model.named_parameters():
        if prm.grad is not None:
            data[f"G_grad:{name}"] = prm.grad.numpy()


def submodule_cases(data: dict) -> None:
    """The building blocks the models are made of, called directly: the linear
    memory cell, the per-query retriever (with the causal segment mask), every
    fusion rule with and without routing weights, and the parameter-mixture fusion."""
    from grm.core.aggregator import ParameterMixtureFusion, RetrievedStateFusion
    from grm.core.gating_unit import TopKMemoryRetriever
    from grm.core.linear_attention import LinearMemoryCell

    g = torch.Generator().manual_seed(9)
    torch.manual_seed(11)
    cell = LinearMemoryCell(16, 12, memory_key_dim=8, memory_decay=0.9)
    flat_state("Dcell_", cell, data)
    xs = torch.randn(2, 9, 16, generator=g)
    with torch.no_grad():
        outs, st = cell.forward_sequence(xs)
        last, st1 = cell.forward(xs[:, 0], st)
        last_only, _ = cell.forward_sequence(xs, return_all_outputs=False)
    for name, t in (("xs", xs), ("outs", outs), ("mem", st.memory), ("h", st.h), ("step_out", last),
                    ("step_mem", st1.memory), ("step_h", st1.h), ("last_only", last_only)):
        data["Dcell_" + name] = t.numpy()

    torch.manual_seed(12)
    ret = TopKMemoryRetriever(12, retrieval_top_k=3, dropout=0.0)
    flat_state("Dret_", ret, data)
    q = torch.randn(3, 12, generator=g)
    keys = torch.randn(3, 7, 12, generator=g)
    keys2 = torch.randn(7, 12, generator=g)
    mask = torch.rand(3, 7, generator=g) > 0.3
    with torch.no_grad():
        cases = {"off5": ret(q, keys, segment_offset=5), "off0": ret(q, keys), "k2d": ret(q, keys2, segment_offset=2),
                 "mask": ret(q, keys, attention_mask=mask)}
        dense = ret.compute_dense_routing_weights(q, keys, segment_offset=4)
    ret8 = TopKMemoryRetriever(12, retrieval_top_k=8, dropout=0.0)
    ret8.load_state_dict(ret.state_dict())
    with torch.no_grad():
        cases["all"] = ret8(q, keys, segment_offset=3)
    data["Dret_q"], data["Dret_keys"], data["Dret_keys2"] = q.numpy(), keys.numpy(), keys2.numpy()
    data["Dret_mask"] = mask.numpy()
    for name, (w, i, sc) in cases.items():
        data[f"Dret_{name}_w"], data[f"Dret_{name}_i"], data[f"Dret_{name}_s"] = w.numpy(), i.numpy(), sc.numpy()
    data["Dret_dense"] = dense.numpy()

    online = torch.randn(4, 10, generator=g)
    retrieved = torch.randn(4, 3, 10, generator=g)
    weights = torch.softmax(torch.randn(4, 3, generator=g), -1)
    data["Dfus_online"], data["Dfus_retrieved"], data["Dfus_weights"] = (online.numpy(), retrieved.numpy(),
                                                                          weights.numpy())
    modes = [("residual", False), ("residual", True), ("concat", False), ("gate", False), ("linear", False),
             ("memory_soup", False)]
    for n, (mode, proj) in enumerate(modes):
        torch.manual_seed(20 + n)
        fus = RetrievedStateFusion(10, retrieval_fusion_mode=mode, use_output_projection=proj, dropout=0.0)
        pre = f"Dfus{n}_"
        flat_state(pre, fus, data)
        with torch.no_grad():
            out, stats = fus.forward_with_auxiliary_statistics(online, retrieved, weights)
            short = fus(online_state=online, retrieved_states=retrieved, routing_weights=weights[:, :2])
            none_w = fus(h_online=online, cached_states=retrieved)
            empty = fus(online, retrieved[:, :0], None)
        data[pre + "out"], data[pre + "short"], data[pre + "none"], data[pre + "empty"] = (
            out.numpy(), short.numpy(), none_w.numpy(), empty.numpy())
        data[pre + "stats"] = np.array([stats["online_norm"], stats["retrieved_norm"], stats["num_retrieved"],
                                        stats["routing_entropy"]])
    torch.manual_seed(30)
    mix = ParameterMixtureFusion(10, num_memory_layers=2, dropout=0.0)
    with torch.no_grad():
        mix.segment_weights[1].add_(torch.randn(10, generator=g) * 0.1)
        data["Dmix_out"] = mix(online, retrieved, weights).numpy()
        data["Dmix_none"] = mix(online, retrieved).numpy()
        data["Dmix_empty"] = mix(online, retrieved[:, :0]).numpy()
    flat_state("Dmix_", mix, data)


def main() -> int:
    multilayer_grm, paper_grm = import_reference_core()
    data = {}
    submodule_cases(data)
    gradient_case(multilayer_grm, data)
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
