"""The Python op surface on CPU: runtime status, kernel policies, the CPU-key
implementations of torch.ops.grm_cuda and the PyTorch fallbacks, all checked
against the oracle.  Mirrors the reference's own checks in
examples/test_grm.py:29-221 where they apply to CPU tensors."""

import numpy as np
import pytest
import torch

from oracle import oracle as orc
from rnn_with_grm_amd import cuda_ops


def make_chunk_case(T, B=2, H=16, K=8, dtype=torch.float32, seed=0):
    g = torch.Generator().manual_seed(seed)
    k = torch.nn.functional.normalize(torch.randn(B, T, K, generator=g), dim=-1).to(dtype)
    v = torch.randn(B, T, H, generator=g).to(dtype)
    q = torch.nn.functional.normalize(torch.randn(B, T, K, generator=g), dim=-1).to(dtype)
    m = torch.randn(B, H, K, generator=g).to(dtype)
    return k, v, q, m


@pytest.fixture(autouse=True, scope="module")
def _extension_loaded():
    """The tests below call torch.ops.grm_cuda directly, so the extension is
    loaded before the first of them, whatever order they run in."""
    assert cuda_ops.load_grm_cuda_extension(), cuda_ops.get_grm_cuda_runtime_status()["load_error"]


def np64(t):
    return t.detach().double().numpy()


def test_runtime_status_payload():
    """Same keys, policy values and dispatch consistency as examples/test_grm.py:116-151."""
    status = cuda_ops.get_grm_cuda_runtime_status()
    for key in ("load_attempted", "extension_loaded", "compiled_with_cuda_sources", "compiled_with_cuda_kernels",
                "torch_cuda_available", "cuda_backend_available", "load_error", "module_name", "registered_ops",
                "dispatch_kernels", "kernel_policy"):
        assert key in status
    assert set(status["kernel_policy"]) == {"global", "chunk_update", "apply_query", "batched_memory_gather"}
    assert all(p in {"auto", "native", "fallback"} for p in status["kernel_policy"].values())
    assert status["extension_loaded"], status["load_error"]
    assert status["compiled_with_cuda_sources"] and status["compiled_with_cuda_kernels"]
    assert all(d["cuda"] for d in status["dispatch_kernels"].values())
    assert all(status["registered_ops"].values())
    assert status["hip"]["arch"] == "gfx950"
    assert all(status["hip"]["extra_ops"].values())
    assert status["cuda_backend_available"] == torch.cuda.is_available()


def test_policy_precedence(monkeypatch):
    monkeypatch.setenv("GRM_CUDA_KERNEL_POLICY", "fallback")
    monkeypatch.setenv("GRM_CUDA_CHUNK_UPDATE_POLICY", "native")
    monkeypatch.setenv("GRM_CUDA_APPLY_QUERY_POLICY", "bogus")
    assert cuda_ops.kernel_policy("chunk_update") == "native"  # per-op beats global
    assert cuda_ops.kernel_policy("apply_query") == "fallback"  # invalid per-op value is ignored
    assert cuda_ops.kernel_policy("batched_memory_gather") == "fallback"
    assert cuda_ops.kernel_policy("") == "fallback"
    monkeypatch.delenv("GRM_CUDA_KERNEL_POLICY")
    assert cuda_ops.kernel_policy("batched_memory_gather") == "auto"


def test_gpu_tensor_without_extension_raises(monkeypatch):
    monkeypatch.setattr(cuda_ops._LIB, "module", None)
    monkeypatch.setattr(cuda_ops._LIB, "attempted", True)
    monkeypatch.setattr(cuda_ops._LIB, "error", "simulated import failure")
    with pytest.raises(cuda_ops.GrmExtensionUnavailable, match="simulated import failure"):
        cuda_ops._native_required(torch.device("cuda"))
    assert cuda_ops._native_required(torch.device("cpu")) is False
    status = cuda_ops.get_grm_cuda_runtime_status()
    assert status["extension_loaded"] is False and status["load_error"] == "simulated import failure"


@pytest.mark.parametrize("T", [0, 1, 8, 64, 100])
@pytest.mark.parametrize("dtype,tol", [(torch.float64, 1e-12), (torch.float32, 1e-5)])
def test_cpu_chunk_update_forward(T, dtype, tol):
    k, v, q, m = make_chunk_case(T, dtype=dtype, seed=T)
    h, mo, aux = torch.ops.grm_cuda.chunk_update_forward(k, v, q, m, 0.97)
    assert aux.numel() == 0 and h.dtype == dtype and mo.dtype == dtype
    rh, rm, _ = orc.chunk_update_seq(np64(k), np64(v), np64(q), np64(m), 0.97)
    np.testing.assert_allclose(np64(h), rh, rtol=tol, atol=tol)
    np.testing.assert_allclose(np64(mo), rm, rtol=tol, atol=tol)


def test_cpu_chunk_update_backward():
    k, v, q, m = make_chunk_case(70, H=12, K=6, dtype=torch.float64, seed=3)
    g = torch.Generator().manual_seed(4)
    dh = torch.randn(2, 70, 12, generator=g, dtype=torch.float64)
    dm = torch.randn(2, 12, 6, generator=g, dtype=torch.float64)
    grads = torch.ops.grm_cuda.chunk_update_backward(dh, dm, k, v, q, m, torch.empty(0), 0.9)
    ref = orc.chunk_update_bwd(np64(dh), np64(dm), np64(k), np64(v), np64(q), np64(m), 0.9)
    for got, want in zip(grads, ref):
        np.testing.assert_allclose(np64(got), want, rtol=1e-10, atol=1e-12)


def test_entrypoint_parity_reference_case():
    """examples/test_grm.py:40-113 on CPU: chunk 8, native (CPU op) vs fallback, forward and grads at 1e-5."""
    k, v, q, m = make_chunk_case(8, seed=11)

    def run(debug, policy):
        ins = [t.clone().requires_grad_(True) for t in (k, v, q, m)]
        h, mo = cuda_ops.cuda_chunk_update(*ins, memory_decay=0.97, debug_fallback=debug)
        (h.square().mean() + mo.square().mean()).backward()
        return [h.detach(), mo.detach()] + [t.grad for t in ins]

    ref = run(True, None)
    import os
    os.environ["GRM_CUDA_CHUNK_UPDATE_POLICY"] = "native"
    try:
        live = run(False, "native")
    finally:
        del os.environ["GRM_CUDA_CHUNK_UPDATE_POLICY"]
    for a, b in zip(live, ref):
        torch.testing.assert_close(a, b, atol=1e-5, rtol=1e-5)


def test_fallback_chunk_update_matches_oracle():
    k, v, q, m = make_chunk_case(64, dtype=torch.float64, seed=5)
    h, mo = cuda_ops._torch_chunk_update(k, v, q, m, 0.97)
    rh, rm, _ = orc.chunk_update_seq(np64(k), np64(v), np64(q), np64(m), 0.97)
    np.testing.assert_allclose(np64(h), rh, rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(np64(mo), rm, rtol=1e-12, atol=1e-12)


@pytest.mark.parametrize("seg", [64, 30, 1])
def test_cpu_segment_scan(seg):
    k, v, q, m = make_chunk_case(130, H=8, K=16, dtype=torch.float64, seed=seg)
    h, mo, snaps = torch.ops.grm_cuda.segment_scan_forward(k, v, q, m, 0.97, seg)
    rh, rm, rs = orc.chunk_update_seq(np64(k), np64(v), np64(q), np64(m), 0.97, seg)
    np.testing.assert_allclose(np64(h), rh, rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(np64(snaps), rs, rtol=1e-6, atol=1e-7)  # snapshots are float32
    h2, mo2, snaps2 = cuda_ops.cuda_segment_scan(k, v, q, m, 0.97, seg, debug_fallback=True)
    np.testing.assert_allclose(np64(h2), rh, rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(np64(snaps2), rs, rtol=1e-6, atol=1e-7)


def test_cpu_gather_reference_cases():
    g = torch.Generator().manual_seed(0)
    mem = torch.randn(2, 7, 4, 5, generator=g)
    for idx in (torch.tensor([[[1, 3], [2, 5], [0, 6]], [[4, 2], [1, 0], [3, 5]]]),
                torch.tensor([[0, 2, 4], [1, 3, 5]])):
        live = cuda_ops.cuda_batched_memory_gather(mem, idx)
        ref = cuda_ops.cuda_batched_memory_gather(mem, idx, debug_fallback=True)
        torch.testing.assert_close(live, ref, atol=0.0, rtol=0.0)
        assert np.array_equal(live.numpy(), orc.gather(mem.numpy(), idx.numpy())[0])


def test_cpu_apply_query_and_backward():
    g = torch.Generator().manual_seed(1)
    mem = torch.randn(2, 3, 4, 5, 6, generator=g, dtype=torch.float64)
    q = torch.nn.functional.normalize(torch.randn(2, 3, 6, generator=g, dtype=torch.float64), dim=-1)
    out = torch.ops.grm_cuda.apply_query_forward(mem, q)
    np.testing.assert_allclose(np64(out), orc.apply_query(np64(mem), np64(q)), rtol=1e-13)
    dh = torch.randn(2, 3, 4, 5, generator=g, dtype=torch.float64)
    gm, gq = torch.ops.grm_cuda.apply_query_backward(dh, mem, q)
    rgm, rgq = orc.apply_query_bwd(np64(dh), np64(mem), np64(q))
    np.testing.assert_allclose(np64(gm), rgm, rtol=1e-13)
    np.testing.assert_allclose(np64(gq), rgq, rtol=1e-12)


@pytest.mark.parametrize("S,k", [(50, 8), (6, 8), (40, 32)])
def test_cpu_topk_route_bit_exact(S, k):
    g = torch.Generator().manual_seed(S)
    q = torch.nn.functional.normalize(torch.randn(3, 21, 24, generator=g), dim=-1).to(torch.bfloat16)
    keys = torch.nn.functional.normalize(torch.randn(3, S, 24, generator=g), dim=-1).to(torch.bfloat16)
    gates, idx, sc = cuda_ops.cuda_topk_route(q, keys, k, 24 ** -0.5)
    og, oi, osc = orc.topk_route(q.float().numpy(), keys.float().numpy(), k, 24 ** -0.5)
    assert np.array_equal(idx.numpy(), oi) and np.array_equal(sc.numpy(), osc)
    np.testing.assert_allclose(gates.numpy(), og, rtol=1e-6)


@pytest.mark.parametrize("T,seg,base,cap,k,S", [(200, 16, 0, 64, 8, 13), (96, 8, 5, 6, 4, 16), (64, 64, 0, 64, 8, 1),
                                                 (70, 10, 3, 4, 32, 10)])
def test_cpu_segment_route_matches_oracle(T, seg, base, cap, k, S):
    """One call routes every segment over the archive of its moment: the oracle's
    per-window topk_route, absolute indices, empty slots -1 / -inf / 0."""
    g = torch.Generator().manual_seed(T + k)
    q = torch.nn.functional.normalize(torch.randn(2, T, 24, generator=g), dim=-1).to(torch.bfloat16)
    keys = torch.nn.functional.normalize(torch.randn(2, S, 24, generator=g), dim=-1).to(torch.bfloat16)
    gates, idx, sc = cuda_ops.cuda_segment_route(q, keys, k, seg, base, cap, 24 ** -0.5)
    og, oi, osc = orc.segment_route(q.float().numpy(), keys.float().numpy(), k, seg, base, cap, 24 ** -0.5)
    assert np.array_equal(idx.numpy(), oi) and np.array_equal(sc.numpy(), osc)
    np.testing.assert_allclose(gates.numpy(), og, rtol=1e-6, atol=1e-7)
    # segment s sees min(base + s, cap) keys: every filled index lies in its window
    for t in range(T):
        hi = min(S, base + t // seg)
        lo = max(0, hi - cap)
        row = idx[:, t].numpy()
        assert ((row == -1) | ((row >= lo) & (row < hi))).all()
        assert (row >= 0).sum(-1).tolist() == [min(k, hi - lo)] * 2
    # the PyTorch fallback (torch.topk per window) agrees away from near-ties
    fg, fi, _ = cuda_ops.cuda_segment_route(q.float(), keys.float(), k, seg, base, cap, 24 ** -0.5, enabled=False)
    assert np.array_equal(fi.numpy(), oi)
    np.testing.assert_allclose(fg.numpy(), og, rtol=1e-5, atol=1e-7)


def test_cpu_segment_route_rejects():
    q = torch.zeros(1, 10, 4)
    with pytest.raises(RuntimeError, match="window ends past"):
        torch.ops.grm_cuda.segment_route(q, torch.zeros(1, 2, 4), 2, 3, 0, 8, 1.0, 1.0)
    with pytest.raises(RuntimeError, match="top_k must be in"):
        torch.ops.grm_cuda.segment_route(q, torch.zeros(1, 4, 4), 129, 3, 0, 8, 1.0, 1.0)


def test_cpu_fuse_residual():
    g = torch.Generator().manual_seed(2)
    h, r = torch.randn(5, 32, generator=g), torch.randn(5, 3, 32, generator=g)
    gt = torch.softmax(torch.randn(5, 3, generator=g), -1)
    w, b = torch.randn(32, generator=g), torch.randn(32, generator=g)
    out = cuda_ops.cuda_fuse_residual(h, r, gt, w, b)
    ref = orc.fuse_residual(np64(h), np64(r), np64(gt), np64(w), np64(b))
    np.testing.assert_allclose(out.numpy(), ref, rtol=1e-5, atol=1e-5)


def test_cpu_gather_apply_is_the_composition():
    """The generic gather_apply (CPU key) equals the oracle's gather then apply with the
    queries cast to the memories' dtype; the CUDA-key kernel is checked against it on GPU."""
    g = torch.Generator().manual_seed(3)
    mem = torch.randn(2, 6, 10, 12, generator=g)
    q = torch.randn(2, 4, 12, generator=g).to(torch.bfloat16)
    idx = torch.randint(0, 6, (2, 4, 3), generator=g)
    out = torch.ops.grm_cuda.gather_apply(mem, idx, q)
    gathered, bad = orc.gather(mem.numpy(), idx.numpy())
    ref = orc.apply_query(gathered, np64(q.float()))
    assert bad == 0 and out.dtype == torch.float32 and out.shape == (2, 4, 3, 10)
    np.testing.assert_allclose(out.numpy(), ref, rtol=1e-5, atol=1e-6)
    with pytest.raises(RuntimeError, match="key dim mismatch"):
        torch.ops.grm_cuda.gather_apply(mem, idx, q[..., :5])
    # dtype=float32 on a float16 archive: widened states, float32 queries and output
    m16 = mem.to(torch.float16)
    wide = torch.ops.grm_cuda.gather_apply(m16, idx, q, torch.float32)
    g16, _ = orc.gather(m16.double().numpy(), idx.numpy())
    assert wide.dtype == torch.float32
    np.testing.assert_allclose(wide.numpy(), orc.apply_query(g16, np64(q.float())), rtol=1e-5, atol=1e-6)
    with pytest.raises(RuntimeError, match="memories' dtype or float32"):
        torch.ops.grm_cuda.gather_apply(m16, idx, q, torch.bfloat16)


def test_cpu_segment_retrieve_fuse_window_rule(monkeypatch):
    """The generic segment_retrieve_fuse (CPU key): only the pairs inside the query's routing
    window [max(0, hi - capacity), hi), hi = base + t // segment_len, that do not repeat an
    earlier route contribute; against the oracle's gather -> apply -> residual + LayerNorm over
    exactly those pairs, the PyTorch fallback of cuda_segment_retrieve_fuse, and the index
    check (GRM_HIP_CHECK_INDICES) naming the bad pairs."""
    g = torch.Generator().manual_seed(9)
    B, Q, S, H, K, R, seg, base, cap = 2, 40, 8, 16, 8, 4, 6, 2, 3
    mem = torch.randn(B, S, H, K, generator=g)
    q = torch.randn(B, Q, K, generator=g)
    h = torch.randn(B, Q, H, generator=g)
    gates = torch.softmax(torch.randn(B, Q, R, generator=g), -1)
    w, b = 1 + 0.1 * torch.randn(H, generator=g), 0.1 * torch.randn(H, generator=g)
    idx = torch.randint(-1, S, (B, Q, R), generator=g)
    idx[0, 5, 2] = idx[0, 5, 1] = base + 5 // seg - 1  # a repeat inside the window
    out = torch.ops.grm_cuda.segment_retrieve_fuse(mem, idx, q, gates, h, w, b, 1e-5, seg, base, cap)
    t = np.arange(Q)[None, :, None]
    hi = base + t // seg
    lo = np.maximum(hi - cap, 0)
    ix = idx.numpy()
    valid = (ix >= lo) & (ix < hi)
    for r in range(R):
        for r2 in range(r):
            valid[:, :, r] &= ix[:, :, r] != ix[:, :, r2]
    assert not valid[0, 5, 2] and valid[0, 5, 1]
    gathered, _ = orc.gather(np64(mem), np.where(valid, ix, 0))
    rows = orc.apply_query(gathered, np64(q)) * valid[..., None]
    ref = orc.fuse_residual(np64(h).reshape(B * Q, H), rows.reshape(B * Q, R, H),
                            (np64(gates) * valid).reshape(B * Q, R), np64(w), np64(b)).reshape(B, Q, H)
    np.testing.assert_allclose(out.numpy(), ref, rtol=1e-5, atol=1e-5)
    fb = cuda_ops.cuda_segment_retrieve_fuse(mem, idx, q, gates, h, w, b, 1e-5, seg, base, cap, debug_fallback=True)
    np.testing.assert_allclose(fb.numpy(), ref, rtol=1e-5, atol=1e-5)
    nbad = int(((ix >= 0) & ~valid).sum())
    assert nbad > 0
    monkeypatch.setenv("GRM_HIP_CHECK_INDICES", "1")
    with pytest.raises(IndexError, match=f"{nbad} index values outside their query's window or repeated"):
        torch.ops.grm_cuda.segment_retrieve_fuse(mem, idx, q, gates, h, w, b, 1e-5, seg, base, cap)
    with pytest.raises(RuntimeError, match="windows past the archive"):
        torch.ops.grm_cuda.segment_retrieve_fuse(mem, idx, q, gates, h, w, b, 1e-5, seg, base + S, cap)


def test_shape_errors_raise_like_reference():
    k, v, q, m = make_chunk_case(4)
    with pytest.raises(RuntimeError, match="keys must have shape"):
        torch.ops.grm_cuda.chunk_update_forward(k[0], v, q, m, 0.9)
    with pytest.raises(RuntimeError, match="memory hidden dim"):
        torch.ops.grm_cuda.chunk_update_forward(k, v, q, m[:, :3], 0.9)
    with pytest.raises(RuntimeError, match="topk_indices must have shape"):
        torch.ops.grm_cuda.batched_memory_gather(torch.randn(2, 3, 4, 5), torch.zeros(2, dtype=torch.long))


def test_glue_ops_cpu_match_torch():
    """The CPU kernels of project_split and residual_layer_norm are the torch compositions."""
    import torch.nn.functional as F

    from rnn_with_grm_amd import cuda_ops as co

    if not co.load_grm_cuda_extension():
        pytest.skip("extension not built")
    g = torch.Generator().manual_seed(5)
    for dtype in (torch.float32, torch.bfloat16):
        proj = torch.randn(2, 7, 8 + 16 + 8 + 8, generator=g).to(dtype)
        k, v, q, e = torch.ops.grm_cuda.project_split(proj, 8, 16, 8, 1e-6)
        parts = proj.split([8, 16, 8, 8], dim=-1)
        assert torch.equal(k, F.normalize(parts[0], p=2, dim=-1, eps=1e-6))
        assert torch.equal(q, F.normalize(parts[2], p=2, dim=-1, eps=1e-6))
        assert torch.equal(v, parts[1]) and torch.equal(e, parts[3])
        x, r = torch.randn(5, 16, generator=g).to(dtype), torch.randn(5, 16, generator=g).to(dtype)
        w, b = torch.randn(16, generator=g).to(dtype), torch.randn(16, generator=g).to(dtype)
        y = torch.ops.grm_cuda.residual_layer_norm(x, r, w, b, 1e-5)
        assert torch.equal(y, F.layer_norm(x + r, (16,), w, b, 1e-5))


def _pair_bwd_ref(mem, idx, grad_tokens):
    """Per (query, route) pair M[idx]^T g[q] from the oracle: each pair is its own rank-4
    apply-query backward with one route, so the sum over routes cannot hide a wrong route."""
    B, Q, R = idx.shape
    H, K = mem.shape[2], mem.shape[3]
    ok = (idx >= 0).numpy()
    gathered, _ = orc.gather(mem.double().numpy(), np.where(ok, idx.numpy(), 0))
    gathered = (gathered * ok[..., None, None]).reshape(B * Q * R, 1, H, K)
    g = np.repeat(grad_tokens.double().numpy()[:, :, None, :], R, axis=2).reshape(B * Q * R, 1, H)
    _, gq = orc.apply_query_bwd(g, gathered, np.zeros((B * Q * R, K)))
    return gq.reshape(B, Q, R, K)


def test_cpu_gather_apply_backward_tokens():
    """The generic (CPU-key) token gradient per pair against the oracle (the generic gather, like
    the reference's fallback, rejects out-of-range indices; the kernel's zero rows for them are
    checked on the GPU)."""
    if not cuda_ops.load_grm_cuda_extension():
        pytest.skip("extension not built")
    g = torch.Generator().manual_seed(11)
    mem = torch.randn(2, 5, 12, 9, generator=g).to(torch.bfloat16)
    idx = torch.randint(0, 5, (2, 7, 3), generator=g)
    gx = torch.randn(2, 7, 12, generator=g)
    out = torch.ops.grm_cuda.gather_apply_backward_tokens(mem, idx, gx)
    assert out.dtype == torch.float32 and out.shape == (2, 7, 3, 9)
    np.testing.assert_allclose(out.numpy(), _pair_bwd_ref(mem, idx, gx), rtol=1e-5, atol=1e-5)
    with pytest.raises(RuntimeError, match="shape mismatch"):
        torch.ops.grm_cuda.gather_apply_backward_tokens(mem, idx, gx[..., :5])


@pytest.mark.parametrize("ln", [True, False])
def test_cpu_retrieve_fuse_training_function(monkeypatch, ln):
    """The training form of the fused retrieval (policy "native" on CPU tensors runs it through
    the CPU-key ops): output and the gradients of queries, gates, h and the LayerNorm
    parameters equal autograd through the float64 composition gather -> apply -> weighted sum ->
    residual -> LayerNorm."""
    monkeypatch.setenv(cuda_ops.GLOBAL_POLICY_ENV, "native")
    if not cuda_ops.load_grm_cuda_extension():
        pytest.skip("extension not built")
    g = torch.Generator().manual_seed(12)
    B, S, Q, R, H, K = 2, 6, 9, 3, 16, 8
    mem = torch.randn(B, S, H, K, generator=g) * 0.3
    idx = torch.randint(0, S, (B, Q, R), generator=g)
    q = torch.nn.functional.normalize(torch.randn(B, Q, K, generator=g), dim=-1).requires_grad_(True)
    gates = torch.softmax(torch.randn(B, Q, R, generator=g), -1).requires_grad_(True)
    h = torch.randn(B, Q, H, generator=g).requires_grad_(True)
    w = (1 + 0.1 * torch.randn(H, generator=g)).requires_grad_(ln)
    b = (0.1 * torch.randn(H, generator=g)).requires_grad_(ln)
    lw, lb = (w, b) if ln else (None, None)
    gout = torch.randn(B, Q, H, generator=g)
    out = cuda_ops.cuda_retrieve_fuse(mem, idx, q, gates, h, lw, lb, 1e-5)
    assert out.grad_fn is not None and "RetrieveFuse" in type(out.grad_fn).__name__
    wrt = [q, gates, h] + ([w, b] if ln else [])
    grads = torch.autograd.grad(out, wrt, gout)
    d = [t.detach().double().requires_grad_(True) for t in wrt]
    sel = mem.double()[torch.arange(B)[:, None, None], idx]
    x = d[2] + torch.einsum("bqr,bqrh->bqh", d[1], torch.einsum("bqrhk,bqk->bqrh", sel, d[0]))
    ref = torch.nn.functional.layer_norm(x, (H,), d[3], d[4], 1e-5) if ln else x
    rgrads = torch.autograd.grad(ref, d, gout.double())
    torch.testing.assert_close(out.double(), ref.detach(), rtol=1e-5, atol=1e-5)
    for got, want in zip(grads, rgrads):
        torch.testing.assert_close(got.double(), want, rtol=1e-4, atol=1e-5)


def test_cpu_archive_cast():
    """archive_cast (CPU key and the cuda_ops wrapper) is the two torch casts, model dtype first."""
    if not cuda_ops.load_grm_cuda_extension():
        pytest.skip("extension not built")
    g = torch.Generator().manual_seed(13)
    x = torch.randn(3, 5, 7, generator=g) * 1e3
    for md in (torch.float32, torch.bfloat16, torch.float16):
        for sd in (torch.float32, torch.bfloat16, torch.float16):
            want = x.to(md).to(sd)
            assert torch.equal(torch.ops.grm_cuda.archive_cast(x, md, sd), want)
            assert torch.equal(cuda_ops.cuda_archive_cast(x, md, sd), want)
    with pytest.raises(RuntimeError, match="float32"):
        torch.ops.grm_cuda.archive_cast(x.half(), torch.bfloat16, torch.float16)


def test_cpu_project_gemm_is_linear_then_split():
    """project_gemm's CPU kernel and the cuda_ops wrapper are F.linear followed by project_split."""
    import torch.nn.functional as F

    if not cuda_ops.load_grm_cuda_extension():
        pytest.skip("extension not built")
    g = torch.Generator().manual_seed(14)
    x = torch.randn(3, 5, 16, generator=g)
    w, b = torch.randn(2 * 8 + 24 + 8, 16, generator=g), torch.randn(2 * 8 + 24 + 8, generator=g)
    got = torch.ops.grm_cuda.project_gemm(x, w, b, 8, 24, 8, 1e-6)
    want = torch.ops.grm_cuda.project_split(F.linear(x, w, b), 8, 24, 8, 1e-6)
    assert all(torch.equal(a, c) for a, c in zip(got, want))
    wrapped = cuda_ops.cuda_project_gemm(x, w, b, 8, 24, 8, 1e-6)
    assert len(wrapped) == 4 and all(torch.equal(a, c) for a, c in zip(wrapped, want))
    with pytest.raises(RuntimeError, match="weight must be"):
        torch.ops.grm_cuda.project_gemm(x, w[:-1], None, 8, 24, 8, 1e-6)


def test_cpu_linear_residual_layer_norm_is_linear_then_layer_norm():
    """linear_residual_layer_norm's CPU kernel is layer_norm(F.linear(x, w, b) + residual); with
    save it also returns the LayerNorm input and native_layer_norm's row statistics."""
    import torch.nn.functional as F

    if not cuda_ops.load_grm_cuda_extension():
        pytest.skip("extension not built")
    g = torch.Generator().manual_seed(15)
    x, res = torch.randn(3, 7, 24, generator=g), torch.randn(3, 7, 16, generator=g)
    w, b = torch.randn(16, 24, generator=g), torch.randn(16, generator=g)
    lw, lb = torch.randn(16, generator=g), torch.randn(16, generator=g)
    s = F.linear(x, w, b) + res
    want = F.layer_norm(s, (16,), lw, lb, 1e-5)
    out, pre, mean, rstd = torch.ops.grm_cuda.linear_residual_layer_norm(x, w, b, res, lw, lb, 1e-5, True)
    torch.testing.assert_close(out, want)
    torch.testing.assert_close(pre, s)
    _, m, r = torch.ops.aten.native_layer_norm(s, [16], lw, lb, 1e-5)
    torch.testing.assert_close(mean, m.reshape(-1))
    torch.testing.assert_close(rstd, r.reshape(-1))
    assert torch.equal(torch.ops.grm_cuda.linear_residual_layer_norm(x, w, b, res, lw, lb, 1e-5, False)[0], out)
    torch.testing.assert_close(cuda_ops.cuda_linear_residual_layer_norm(x, w, b, res, lw, lb, 1e-5), want)
    with pytest.raises(RuntimeError, match="weight must be"):
        torch.ops.grm_cuda.linear_residual_layer_norm(x, w[:, :-1], b, res, lw, lb, 1e-5, False)


@pytest.mark.parametrize("affine", [True, False])
def test_linear_residual_layer_norm_backward_matches_autograd(affine):
    """_LinearResidualLayerNormFn's backward (aten's layer-norm backward on the saved input and
    statistics, then the linear map's gradients) equals torch autograd of F.linear + add +
    layer_norm, float32 on the CPU, for every input."""
    import torch.nn.functional as F

    if not cuda_ops.load_grm_cuda_extension():
        pytest.skip("extension not built")
    g = torch.Generator().manual_seed(16)
    ins = [torch.randn(2, 9, 24, generator=g), torch.randn(16, 24, generator=g), torch.randn(16, generator=g),
           torch.randn(2, 9, 16, generator=g)]
    ln = [torch.randn(16, generator=g), torch.randn(16, generator=g)] if affine else [None, None]
    dout = torch.randn(2, 9, 16, generator=g)
    a = [t.clone().requires_grad_(True) for t in ins] + [None if t is None else t.clone().requires_grad_(True)
                                                          for t in ln]
    out = cuda_ops._LinearResidualLayerNormFn.apply(*a, 1e-5)
    got = torch.autograd.grad(out, [t for t in a if t is not None], dout)
    r = [t.clone().requires_grad_(True) for t in ins] + [None if t is None else t.clone().requires_grad_(True)
                                                          for t in ln]
    ref_out = F.layer_norm(F.linear(r[0], r[1], r[2]) + r[3], (16,), r[4], r[5], 1e-5)
    want = torch.autograd.grad(ref_out, [t for t in r if t is not None], dout)
    torch.testing.assert_close(out, ref_out)
    for x, y in zip(got, want):
        torch.testing.assert_close(x, y, rtol=1e-5, atol=1e-5)


def test_project_gemm_backward_matches_autograd():
    """_ProjectGemmFn's backward (F.normalize's derivative from recomputed norms, then the GEMM's
    gradients) equals torch autograd of F.linear + split + F.normalize, float32 on the CPU, with
    an extra part, unused outputs, and one row whose key projection is below the eps clamp."""
    import torch.nn.functional as F

    if not cuda_ops.load_grm_cuda_extension():
        pytest.skip("extension not built")
    g = torch.Generator().manual_seed(17)
    dk, dv, de, K = 8, 24, 16, 20
    x = torch.randn(3, 5, K, generator=g)
    w = torch.randn(2 * dk + dv + de, K, generator=g)
    b = torch.randn(2 * dk + dv + de, generator=g)
    w[:dk] *= 1e-9  # key projections of tiny norm ...
    b[:dk] *= 1e-9  # ... below eps for every row: the clamped branch
    grads = [torch.randn(3, 5, d, generator=g) for d in (dk, dv, dk, de)]
    for used in ((0, 1, 2, 3), (1, 2)):
        a = [t.clone().requires_grad_(True) for t in (x, w, b)]
        outs = cuda_ops._ProjectGemmFn.apply(a[0], a[1], a[2], dk, dv, de, 1e-6)
        got = torch.autograd.grad([outs[i] for i in used], a, [grads[i] for i in used])
        r = [t.clone().requires_grad_(True) for t in (x, w, b)]
        p = F.linear(r[0], r[1], r[2]).split([dk, dv, dk, de], -1)
        ref = (F.normalize(p[0], dim=-1, eps=1e-6), p[1], F.normalize(p[2], dim=-1, eps=1e-6), p[3])
        want = torch.autograd.grad([ref[i] for i in used], r, [grads[i] for i in used])
        for o, rr in zip(outs, ref):
            torch.testing.assert_close(o, rr)
        for gg, ww in zip(got, want):
            torch.testing.assert_close(gg, ww, rtol=1e-4, atol=1e-5)


def test_cpu_topk_route_non_finite_rule():
    """The CPU kernel's rule for non-finite scores (the GPU paths share it): a NaN or -inf score is
    never selected, slots left over are (-1, -inf, 0), gates the softmax of the filled slots;
    with k >= n_keys every key comes back in index order, as in the reference's branch."""
    if not cuda_ops.load_grm_cuda_extension():
        pytest.skip("extension not built")
    g = torch.Generator().manual_seed(18)
    q = torch.nn.functional.normalize(torch.randn(1, 4, 16, generator=g), dim=-1)
    keys = torch.nn.functional.normalize(torch.randn(1, 6, 16, generator=g), dim=-1)
    q[0, 1] = float("nan")
    keys[0, 2, 3] = float("nan")
    gates, idx, sc = torch.ops.grm_cuda.topk_route(q, keys, 3, 0.25, 1.0)
    assert (idx[0, 1] == -1).all() and torch.isinf(sc[0, 1]).all() and (gates[0, 1] == 0).all()
    assert not (idx == 2).any()
    full = (q[0, 0] @ keys[0].T * 0.25)
    full[2] = -float("inf")
    top = torch.sort(full, descending=True, stable=True)
    assert torch.equal(idx[0, 0], top.indices[:3])
    torch.testing.assert_close(gates[0, 0], torch.softmax(top.values[:3], -1), rtol=1e-5, atol=1e-6)
    gates_all, idx_all, _ = torch.ops.grm_cuda.topk_route(q, keys, 6, 0.25, 1.0)
    assert torch.equal(idx_all[0, 0], torch.arange(6))
