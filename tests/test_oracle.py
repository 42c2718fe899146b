"""Pins the CPU oracle (oracle/grm_oracle.c) before anything is compared with it.

Each check is independent of the oracle's own formulas:
  * the reference's CPU ops, through fixtures written from oracle/_ref
    (tests/golden/make_golden.py) and, when built here, live;
  * a second algorithm (per-token recurrence vs chunked closed form);
  * closed forms: decay 1 is a plain GEMM, decay 0 a scaled dot product,
    one token from a zero state an outer product;
  * finite differences for the gradients;
  * library routines (numpy einsum / take, torch.topk on float64, torch layer_norm)
    and a float32 loop that reproduces the FMA chain exactly for bf16 inputs.
"""

import importlib.util
from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import oracle as orc

GOLDEN = Path(__file__).resolve().parent / "golden" / "reference_cpu_ops.npz"
REF_HARNESS = Path(__file__).resolve().parents[1] / "oracle" / "_ref" / "grm_ref_harness.so"


def rnd(*shape, seed=0, normalize=False):
    x = np.random.default_rng(seed).standard_normal(shape)
    if normalize:
        x = x / np.linalg.norm(x, axis=-1, keepdims=True)
    return x


def chunk_case(B=2, T=37, K=8, H=16, seed=0):
    return (rnd(B, T, K, seed=seed, normalize=True), rnd(B, T, H, seed=seed + 1),
            rnd(B, T, K, seed=seed + 2, normalize=True), rnd(B, H, K, seed=seed + 3))


# ---------------------------------------------------------------- chunk update
def test_golden_fixtures_chunk_update():
    """Oracle vs the reference's own CPU recurrence and autograd backward (fixtures)."""
    d = np.load(GOLDEN)
    i = 0
    while f"chunk{i}_keys" in d:
        p = f"chunk{i}_"
        decay = float(d[p + "decay"])
        h, mo, _ = orc.chunk_update_seq(d[p + "keys"], d[p + "values"], d[p + "queries"], d[p + "memory"], decay)
        np.testing.assert_allclose(h, d[p + "hidden"], rtol=1e-12, atol=1e-12)
        np.testing.assert_allclose(mo, d[p + "memory_out"], rtol=1e-12, atol=1e-12)
        grads = orc.chunk_update_bwd(d[p + "grad_hidden"], d[p + "grad_memory_out"], d[p + "keys"],
                                     d[p + "values"], d[p + "queries"], d[p + "memory"], decay)
        for name, g in zip(("grad_keys", "grad_values", "grad_queries", "grad_memory"), grads):
            np.testing.assert_allclose(g, d[p + name], rtol=1e-10, atol=1e-11, err_msg=f"{p}{name}")
        i += 1
    assert i >= 6


@pytest.mark.skipif(not REF_HARNESS.exists(), reason="oracle/_ref not built (needs /root/reference)")
def test_live_reference_chunk_update():
    spec = importlib.util.spec_from_file_location("grm_ref_harness", REF_HARNESS)
    ref = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(ref)
    k, v, q, m = chunk_case(3, 129, 32, 24, seed=4)
    t = lambda x: torch.from_numpy(x)  # noqa: E731
    h, mo, _ = ref.chunk_update_forward(t(k), t(v), t(q), t(m), 0.93)
    oh, om, _ = orc.chunk_update_seq(k, v, q, m, 0.93)
    np.testing.assert_allclose(oh, h.numpy(), rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(om, mo.numpy(), rtol=1e-12, atol=1e-12)


@pytest.mark.parametrize("chunk", [1, 5, 16, 64, 1000])
def test_sequential_equals_chunked(chunk):
    k, v, q, m = chunk_case(2, 150, 12, 7, seed=chunk)
    h1, m1, _ = orc.chunk_update_seq(k, v, q, m, 0.97)
    h2, m2 = orc.chunk_update_chunked(k, v, q, m, 0.97, chunk)
    np.testing.assert_allclose(h1, h2, rtol=1e-11, atol=1e-13)
    np.testing.assert_allclose(m1, m2, rtol=1e-11, atol=1e-13)


def test_decay_one_is_plain_gemm():
    k, v, q, m = chunk_case(3, 20, 9, 5, seed=1)
    h, mo, _ = orc.chunk_update_seq(k, v, q, m, 1.0)
    np.testing.assert_allclose(h, np.einsum("bhk,btk->bth", m, q), rtol=1e-13, atol=1e-13)
    np.testing.assert_array_equal(mo, m)


def test_decay_zero_is_scaled_dot():
    k, v, q, m = chunk_case(2, 11, 6, 4, seed=2)
    h, mo, _ = orc.chunk_update_seq(k, v, q, m, 0.0)
    expect = (np.sum(q * k, -1, keepdims=True) / np.sqrt(6)) * v
    np.testing.assert_allclose(h, expect, rtol=1e-13, atol=1e-13)
    np.testing.assert_allclose(mo, np.einsum("bh,bk->bhk", v[:, -1], k[:, -1]) / np.sqrt(6), rtol=1e-13)


def test_one_token_from_zero_is_outer_product():
    k, v, q, _ = chunk_case(2, 1, 8, 3, seed=3)
    m = np.zeros((2, 3, 8))
    h, mo, _ = orc.chunk_update_seq(k, v, q, m, 0.9)
    outer = 0.1 / np.sqrt(8) * np.einsum("bh,bk->bhk", v[:, 0], k[:, 0])
    np.testing.assert_allclose(mo, outer, rtol=1e-13)
    np.testing.assert_allclose(h[:, 0], np.einsum("bhk,bk->bh", outer, q[:, 0]), rtol=1e-13)


def test_linearity_in_values_and_state():
    k, v1, q, m1 = chunk_case(2, 40, 8, 6, seed=5)
    _, v2, _, m2 = chunk_case(2, 40, 8, 6, seed=9)
    a, b = 0.7, -1.3
    h1, o1, _ = orc.chunk_update_seq(k, v1, q, m1, 0.95)
    h2, o2, _ = orc.chunk_update_seq(k, v2, q, m2, 0.95)
    h, o, _ = orc.chunk_update_seq(k, a * v1 + b * v2, q, a * m1 + b * m2, 0.95)
    np.testing.assert_allclose(h, a * h1 + b * h2, rtol=1e-11, atol=1e-13)
    np.testing.assert_allclose(o, a * o1 + b * o2, rtol=1e-11, atol=1e-13)


def test_snapshots_are_prefix_states():
    k, v, q, m = chunk_case(2, 100, 8, 6, seed=6)
    _, _, snaps = orc.chunk_update_seq(k, v, q, m, 0.97, snapshot_len=30)
    assert snaps.shape == (2, 4, 6, 8)
    for i, end in enumerate((30, 60, 90, 100)):
        _, mo, _ = orc.chunk_update_seq(k[:, :end], v[:, :end], q[:, :end], m, 0.97)
        np.testing.assert_allclose(snaps[:, i], mo, rtol=1e-13)


def test_backward_finite_differences():
    k, v, q, m = chunk_case(1, 9, 4, 3, seed=7)
    dh = rnd(1, 9, 3, seed=8)
    dm = rnd(1, 3, 4, seed=9)

    def loss(kk, vv, qq, mm):
        h, mo, _ = orc.chunk_update_seq(kk, vv, qq, mm, 0.8)
        return float(np.sum(h * dh) + np.sum(mo * dm))

    grads = orc.chunk_update_bwd(dh, dm, k, v, q, m, 0.8)
    eps = 1e-6
    for gi, arg in enumerate((k, v, q, m)):
        num = np.zeros_like(arg)
        for idx in np.ndindex(arg.shape):
            args = [k.copy(), v.copy(), q.copy(), m.copy()]
            args[gi][idx] += eps
            up = loss(*args)
            args[gi][idx] -= 2 * eps
            num[idx] = (up - loss(*args)) / (2 * eps)
        np.testing.assert_allclose(grads[gi], num, rtol=1e-6, atol=1e-8)


# ---------------------------------------------------------------- apply / gather
def test_golden_apply_and_gather():
    d = np.load(GOLDEN)
    for i in range(2):
        p = f"apply{i}_"
        np.testing.assert_allclose(orc.apply_query(d[p + "memories"], d[p + "queries"]), d[p + "hidden"],
                                   rtol=1e-13, atol=1e-14)
        gm, gq = orc.apply_query_bwd(d[p + "grad_hidden"], d[p + "memories"], d[p + "queries"])
        np.testing.assert_allclose(gm, d[p + "grad_memories"], rtol=1e-13, atol=1e-14)
        np.testing.assert_allclose(gq, d[p + "grad_queries"], rtol=1e-12, atol=1e-13)
    for r in ("3", "2"):
        out, bad = orc.gather(d["gather_memories"], d["gather_idx" + r])
        assert bad == 0 and np.array_equal(out, d["gather_out" + r])


def test_apply_query_einsum():
    mm = rnd(2, 3, 4, 5, 6, seed=1)
    q = rnd(2, 3, 6, seed=2)
    np.testing.assert_allclose(orc.apply_query(mm, q), np.einsum("bqrhk,bqk->bqrh", mm, q), rtol=1e-13)
    mm4 = rnd(3, 4, 5, 7, seed=3)
    q4 = rnd(3, 7, seed=4)
    np.testing.assert_allclose(orc.apply_query(mm4, q4), np.einsum("brhk,bk->brh", mm4, q4), rtol=1e-13)


def test_gather_take_and_bad_indices():
    mem = np.arange(2 * 5 * 3 * 2, dtype=np.float32).reshape(2, 5, 3, 2)
    idx = np.array([[4, 0, 2], [1, 1, 3]])
    out, bad = orc.gather(mem, idx)
    assert bad == 0
    assert np.array_equal(out, np.stack([np.take(mem[b], idx[b], axis=0) for b in range(2)]))
    out, bad = orc.gather(mem, np.array([[5, -1, 2], [0, 0, 0]]))
    assert bad == 2 and not out[0, :2].any() and np.array_equal(out[0, 2], mem[0, 2])


# ---------------------------------------------------------------- routing
def bf16_round(x):
    return torch.from_numpy(np.asarray(x, dtype=np.float32)).to(torch.bfloat16).float().numpy()


def fp32_chain_scores(q, keys, scale):
    """float32 sequential dot products; exact FMA emulation for bf16-valued inputs
    (their products are exact in float32, so fma == add of the product)."""
    B, Q, D = q.shape
    S = keys.shape[1]
    out = np.zeros((B, Q, S), dtype=np.float32)
    prods = q[:, :, None, :].astype(np.float32) * keys[:, None, :, :].astype(np.float32)
    acc = np.zeros((B, Q, S), dtype=np.float32)
    for d in range(D):
        acc = (acc + prods[..., d]).astype(np.float32)
    out[:] = acc * np.float32(scale)
    return out


@pytest.mark.parametrize("S,k", [(64, 8), (30, 30), (12, 20), (257, 16)])
def test_topk_route_against_brute_force(S, k):
    q = bf16_round(rnd(2, 23, 32, seed=S, normalize=True))
    keys = bf16_round(rnd(2, S, 32, seed=S + 1, normalize=True))
    scale = 1.0 / np.sqrt(32)
    gates, idx, sc = orc.topk_route(q, keys, k, scale)
    ref = fp32_chain_scores(q, keys, scale)
    kk = min(k, S)
    if kk < S:
        order = np.argsort(-ref, axis=-1, kind="stable")[..., :kk]  # stable: ties to the lower index
    else:
        order = np.broadcast_to(np.arange(S), ref.shape)
    assert np.array_equal(idx, order)
    assert np.array_equal(sc, np.take_along_axis(ref, order, -1))
    sel = np.take_along_axis(ref, order, -1).astype(np.float64)
    e = np.exp(sel - sel.max(-1, keepdims=True))
    np.testing.assert_allclose(gates, e / e.sum(-1, keepdims=True), rtol=1e-12)


def test_topk_route_ties_and_torch_topk():
    base = bf16_round(rnd(1, 6, 16, seed=1, normalize=True))
    keys = np.concatenate([base, base, base], axis=1)
    q = bf16_round(rnd(1, 9, 16, seed=2, normalize=True))
    _, idx, sc = orc.topk_route(q, keys, 7, 0.25)
    eq = sc[..., 1:] == sc[..., :-1]
    assert (idx[..., 1:][eq] > idx[..., :-1][eq]).all()
    # away from ties the selection agrees with torch.topk on float64 scores
    q2 = rnd(2, 15, 24, seed=3, normalize=True).astype(np.float32)
    k2 = rnd(2, 80, 24, seed=4, normalize=True).astype(np.float32)
    _, idx2, _ = orc.topk_route(q2, k2, 8, 0.2)
    s64 = torch.from_numpy(q2.astype(np.float64)) @ torch.from_numpy(k2.astype(np.float64)).transpose(1, 2)
    top = torch.topk(s64, 9, dim=-1)
    clear = (top.values[..., 7] - top.values[..., 8]) > 1e-5
    assert np.array_equal(np.sort(idx2, -1)[clear.numpy()], np.sort(top.indices[..., :8].numpy(), -1)[clear.numpy()])


# ---------------------------------------------------------------- fusion
def test_fuse_residual_against_torch_layer_norm():
    h, r = rnd(7, 33, seed=1), rnd(7, 4, 33, seed=2)
    g = np.abs(rnd(7, 4, seed=3))
    w, b = rnd(33, seed=4), rnd(33, seed=5)
    out = orc.fuse_residual(h, r, g, w, b, eps=1e-5)
    x = torch.from_numpy(h) + (torch.from_numpy(r) * torch.from_numpy(g)[..., None]).sum(1)
    ref = torch.nn.functional.layer_norm(x, (33,), torch.from_numpy(w), torch.from_numpy(b), 1e-5)
    np.testing.assert_allclose(out, ref.numpy(), rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(orc.fuse_residual(h, r[:, :0], g[:, :0]), h, rtol=0, atol=0)
