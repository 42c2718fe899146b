"""GPU parity of the retrieval path: gather (bit-exact), apply-query, routing
(bit-exact indices and scores) and residual fusion, against the CPU oracle."""

import numpy as np
import pytest
import torch

from oracle import oracle as orc
from rnn_with_grm_amd import capi, cuda_ops

pytestmark = pytest.mark.gpu


def norm(x):
    return torch.nn.functional.normalize(x, dim=-1)


# ---------------------------------------------------------------- gather
def test_gather_reference_cases(dev):
    """The fixed index tensors of the reference's gather test
    (examples/test_grm.py:197-221), bit-exact."""
    g = torch.Generator().manual_seed(0)
    mem = torch.randn(2, 7, 4, 5, generator=g)
    chunk_idx = torch.tensor([[[1, 3], [2, 5], [0, 6]], [[4, 2], [1, 0], [3, 5]]], dtype=torch.long)
    flat_idx = torch.tensor([[0, 2, 4], [1, 3, 5]], dtype=torch.long)
    for idx in (chunk_idx, flat_idx):
        out = torch.ops.grm_cuda.batched_memory_gather(mem.to(dev), idx.to(dev))
        ref, bad = orc.gather(mem.numpy(), idx.numpy())
        assert bad == 0
        assert np.array_equal(out.cpu().numpy(), ref)
        out2 = capi.batched_gather(mem.to(dev), idx.to(dev))
        assert torch.equal(out, out2)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16, torch.float64, torch.int32])
@pytest.mark.parametrize("shape", [(3, 11, 5, 3), (2, 9, 128, 128), (4, 6, 1, 1)])
def test_gather_dtypes(dev, dtype, shape):
    g = torch.Generator().manual_seed(1)
    mem = (torch.randn(*shape, generator=g) * 100).to(dtype)
    B, S = shape[:2]
    idx = torch.randint(0, S, (B, 13, 3), generator=g)
    out = cuda_ops.cuda_batched_memory_gather(mem.to(dev), idx.to(dev))
    ref, _ = orc.gather(mem.numpy() if dtype != torch.bfloat16 else mem.view(torch.int16).numpy(), idx.numpy())
    got = out.cpu()
    got = got.view(torch.int16).numpy() if dtype == torch.bfloat16 else got.numpy()
    assert np.array_equal(got, ref)


def test_gather_int32_indices_and_bad_index(dev):
    mem = torch.arange(2 * 4 * 3 * 2, dtype=torch.float32).reshape(2, 4, 3, 2)
    idx = torch.tensor([[0, 3, 9], [-1, 2, 1]], dtype=torch.int32)
    bad = torch.zeros(1, dtype=torch.int32, device=dev)
    out = capi.batched_gather(mem.to(dev), idx.to(torch.int64).to(dev), bad_count=bad)
    ref, nbad = orc.gather(mem.numpy(), idx.numpy())
    assert int(bad.item()) == nbad == 2
    assert np.array_equal(out.cpu().numpy(), ref)
    # int32 indices through the op are widened to int64 like the reference
    good = torch.tensor([[0, 3, 1], [2, 2, 1]], dtype=torch.int32)
    out = torch.ops.grm_cuda.batched_memory_gather(mem.to(dev), good.to(dev))
    assert np.array_equal(out.cpu().numpy(), orc.gather(mem.numpy(), good.numpy())[0])


def test_gather_config3_slice(dev):
    """BASELINE config 3 geometry with Q reduced to 256: 128x128 fp32 states,
    S=256, k=8; bit-exact against index_select plus a checksum of checksums."""
    B, S, Q, R, D = 64, 256, 256, 8, 128
    g = torch.Generator().manual_seed(4)
    mem = (torch.randn(B, S, D, D, generator=g) * 0.02).to(dev)
    idx = torch.randint(0, S, (B, Q, R), generator=g).to(dev)
    out = capi.batched_gather(mem, idx)
    ref = torch.stack([mem[b].index_select(0, idx[b].reshape(-1)) for b in range(B)]).reshape(out.shape)
    assert torch.equal(out, ref)
    per_row = out.double().sum(dim=(-1, -2))
    expect = mem.double().sum(dim=(-1, -2))
    expect = torch.gather(expect, 1, idx.reshape(B, -1)).reshape(B, Q, R)
    assert torch.equal(per_row, expect)


@pytest.mark.parametrize("B,S,N,D,dtype", [
    (8, 16, 32, 128, torch.float32),     # 32-unit column tiles, 16 MiB out (regular stores)
    (8, 64, 256, 128, torch.bfloat16),   # 16-unit column tiles, 64 MiB out (non-temporal stores)
    (16, 600, 700, 64, torch.float32),   # 8-unit column tiles (600 states need the narrow slice)
])
def test_gather_column_tiles_with_bad_indices(dev, B, S, N, D, dtype):
    """Shapes where every archived state is referenced about once or more, so the
    column-tiled kernel runs; out-of-range indices give zero rows and are counted
    once each."""
    g = torch.Generator().manual_seed(5)
    mem = (torch.randn(B, S, D, D, generator=g) * 0.02).to(dtype).to(dev)
    idx = torch.randint(0, S, (B, N), generator=g)
    idx[0, 3] = -1
    idx[B - 1, N - 1] = S
    idx[B // 2, 0] = 1 << 40
    bad = torch.zeros(1, dtype=torch.int32, device=dev)
    out = capi.batched_gather(mem, idx.to(dev), bad_count=bad)
    ok = (idx >= 0) & (idx < S)
    ref = torch.stack([mem[b].index_select(0, idx[b].clamp(0, S - 1).to(dev)) for b in range(B)])
    ref[~ok.to(dev)] = 0
    assert int(bad.item()) == 3
    assert torch.equal(out, ref)


# ---------------------------------------------------------------- fused gather + apply
def _cast_like(q, dtype):
    return q.to(dtype).to(torch.float64)


@pytest.mark.parametrize("mem_dtype,q_dtype", [(torch.float32, torch.bfloat16), (torch.float32, torch.float32),
                                               (torch.bfloat16, torch.bfloat16), (torch.float16, torch.float32)])
@pytest.mark.parametrize("B,S,Q,R,H,K", [(3, 7, 13, 3, 20, 8), (2, 40, 5, 50, 200, 64), (2, 256, 300, 8, 128, 128),
                                         (1, 1, 4, 2, 8, 33)])
def test_gather_apply_matches_composition(dev, mem_dtype, q_dtype, B, S, Q, R, H, K):
    """gather_apply == apply_query(batched_gather(M, idx), q cast to M's dtype), the
    reference's composition, against the oracle's gather and apply."""
    g = torch.Generator().manual_seed(B * 100 + S)
    mem = (torch.randn(B, S, H, K, generator=g) * 0.02).to(mem_dtype)
    q = norm(torch.randn(B, Q, K, generator=g)).to(q_dtype)
    idx = torch.randint(0, S, (B, Q, R), generator=g)
    out = capi.gather_apply(mem.to(dev), idx.to(dev), q.to(dev))
    gathered, bad = orc.gather(mem.float().numpy(), idx.numpy())
    assert bad == 0
    ref = orc.apply_query(gathered, _cast_like(q, mem_dtype).numpy())
    assert out.dtype == mem_dtype and out.shape == (B, Q, R, H)
    tol = (1e-5, 1e-6) if mem_dtype == torch.float32 else (2e-2, 2e-3)
    np.testing.assert_allclose(out.float().cpu().double().numpy(), ref, rtol=tol[0], atol=tol[1])


@pytest.mark.parametrize("mem_dtype,q_dtype", [(torch.float16, torch.bfloat16), (torch.float16, torch.float32),
                                               (torch.float16, torch.float16), (torch.bfloat16, torch.bfloat16),
                                               (torch.bfloat16, torch.float16), (torch.float32, torch.float32)])
@pytest.mark.parametrize("B,S,Q,R,H,K", [(3, 7, 13, 3, 20, 8), (2, 64, 90, 8, 128, 64), (1, 5, 4, 2, 8, 33)])
def test_gather_apply_widened(dev, mem_dtype, q_dtype, B, S, Q, R, H, K):
    """dtype=float32: 16-bit archives widened on load, queries cast to float32, float32 out,
    i.e. the retriever's stack(...).to(float32) then apply (paper_grm.py:227-229,301)."""
    g = torch.Generator().manual_seed(B * 31 + K)
    mem = (torch.randn(B, S, H, K, generator=g) * 0.05).to(mem_dtype)
    q = norm(torch.randn(B, Q, K, generator=g)).to(q_dtype)
    idx = torch.randint(0, S, (B, Q, R), generator=g)
    out = capi.gather_apply(mem.to(dev), idx.to(dev), q.to(dev), dtype=torch.float32)
    gathered, bad = orc.gather(mem.double().numpy(), idx.numpy())
    ref = orc.apply_query(gathered, q.double().numpy())
    assert out.dtype == torch.float32 and out.shape == (B, Q, R, H)
    np.testing.assert_allclose(out.cpu().double().numpy(), ref, rtol=1e-5, atol=1e-6)
    op = torch.ops.grm_cuda.gather_apply(mem.to(dev), idx.to(dev), q.to(dev), torch.float32)
    assert torch.equal(op, out)


@pytest.mark.parametrize("mem_dtype,q_dtype,H,K", [(torch.float32, torch.bfloat16, 128, 128),
                                                   (torch.float16, torch.bfloat16, 256, 64),
                                                   (torch.float32, torch.float32, 96, 32),
                                                   (torch.float32, torch.float32, 40, 30)])
def test_gather_apply_skewed_selection(dev, mem_dtype, q_dtype, H, K):
    """Causal routing selects early segments far more often than late ones: segments
    selected by many pairs are split over several work tiles.  Here segment 0 takes
    every pair of most queries, segment 1 a third, the rest a thin random tail, and
    some pairs are empty (-1)."""
    g = torch.Generator().manual_seed(H + K)
    B, S, Q, R = 2, 40, 3000, 4
    mem = (torch.randn(B, S, H, K, generator=g) * 0.05).to(mem_dtype)
    q = norm(torch.randn(B, Q, K, generator=g)).to(q_dtype)
    idx = torch.randint(0, S, (B, Q, R), generator=g)
    u = torch.rand(B, Q, R, generator=g)
    idx[u < 0.6] = 0
    idx[(u >= 0.6) & (u < 0.8)] = 1
    idx[:, :50, 2:] = -1
    out = capi.gather_apply(mem.to(dev), idx.to(dev), q.to(dev), dtype=torch.float32)
    ok = idx >= 0
    gathered, bad = orc.gather(mem.double().numpy(), idx.clamp(min=0).numpy())
    ref = orc.apply_query(gathered, q.double().numpy())
    ref[~ok.numpy()] = 0.0
    np.testing.assert_allclose(out.cpu().double().numpy(), ref, rtol=1e-5, atol=1e-6)


def test_gather_apply_bad_indices_and_rank2(dev):
    """Out-of-range indices give zero rows and are counted; rank-2 indices ([B, R]
    with queries [B, K]) go through the torch op like the reference's rank-4 apply."""
    g = torch.Generator().manual_seed(11)
    mem = torch.randn(2, 5, 16, 24, generator=g)
    q = torch.randn(2, 6, 24, generator=g)
    idx = torch.randint(0, 5, (2, 6, 3), generator=g)
    idx[0, 1, 2] = 5
    idx[1, 0, 0] = -3
    bad = torch.zeros(1, dtype=torch.int32, device=dev)
    out = capi.gather_apply(mem.to(dev), idx.to(dev), q.to(dev), bad_count=bad)
    assert int(bad.item()) == 2
    assert torch.count_nonzero(out[0, 1, 2]) == 0 and torch.count_nonzero(out[1, 0, 0]) == 0
    ok = (idx >= 0) & (idx < 5)
    ref = torch.einsum("bqrhk,bqk->bqrh", mem[torch.arange(2)[:, None, None], idx.clamp(0, 4)], q)
    ref[~ok] = 0
    torch.testing.assert_close(out.cpu(), ref, rtol=1e-5, atol=1e-6)
    idx2 = torch.randint(0, 5, (2, 4), generator=g)
    q2 = torch.randn(2, 24, generator=g)
    out2 = torch.ops.grm_cuda.gather_apply(mem.to(dev), idx2.to(dev), q2.to(dev))
    ref2 = torch.einsum("brhk,bk->brh", mem[torch.arange(2)[:, None], idx2], q2)
    assert out2.shape == (2, 4, 16)
    torch.testing.assert_close(out2.cpu(), ref2, rtol=1e-5, atol=1e-6)


def test_gather_apply_config3_slice(dev):
    """BASELINE config 3 geometry (128x128 fp32 states, S=256, k=8, bf16 queries) on 8 of
    the 64 sequences with all 2048 queries, against the materialised composition on the GPU."""
    B, S, Q, R, D = 8, 256, 2048, 8, 128
    g = torch.Generator().manual_seed(12)
    mem = (torch.randn(B, S, D, D, generator=g) * 0.02).to(dev)
    q = norm(torch.randn(B, Q, D, generator=g)).to(torch.bfloat16).to(dev)
    keys = norm(torch.randn(B, S, D, generator=g)).to(torch.bfloat16).to(dev)
    gates, idx, _ = torch.ops.grm_cuda.topk_route(q, keys, R, 1.0 / D ** 0.5, 1.0)
    fused = torch.ops.grm_cuda.gather_apply(mem, idx, q)
    composed = torch.ops.grm_cuda.apply_query_forward(torch.ops.grm_cuda.batched_memory_gather(mem, idx),
                                                      q.to(mem.dtype))
    torch.testing.assert_close(fused, composed, rtol=1e-5, atol=1e-6)


def test_gather_apply_many_pairs_per_sequence(dev):
    """72000 pairs per sequence take the multi-workgroup sort (chunks of 16384 pairs); with
    invalid indices among them, against the composition on the CPU."""
    B, S, Q, R, H, K = 2, 37, 9000, 8, 8, 16
    g = torch.Generator().manual_seed(14)
    mem = torch.randn(B, S, H, K, generator=g)
    q = torch.randn(B, Q, K, generator=g)
    idx = torch.randint(0, S, (B, Q, R), generator=g)
    idx[0, 17, 3] = S
    idx[1, 8999, 7] = -1
    idx[1, 4000, :] = 36
    bad = torch.zeros(1, dtype=torch.int32, device=dev)
    out = capi.gather_apply(mem.to(dev), idx.to(dev), q.to(dev), bad_count=bad)
    assert int(bad.item()) == 2
    ok = (idx >= 0) & (idx < S)
    ref = torch.einsum("bqrhk,bqk->bqrh", mem[torch.arange(B)[:, None, None], idx.clamp(0, S - 1)], q)
    ref[~ok] = 0
    torch.testing.assert_close(out.cpu(), ref, rtol=1e-5, atol=1e-5)


def test_gather_apply_autograd_falls_back(dev):
    """With gradients required, cuda_gather_apply runs the differentiable composition:
    the queries get their gradient through apply_query; like the reference's native
    batched_memory_gather (cuda_ops.py:388-402, no autograd), the archive gets none."""
    g = torch.Generator().manual_seed(13)
    mem = torch.randn(2, 6, 8, 16, generator=g).to(dev).requires_grad_(True)
    q = torch.randn(2, 5, 16, generator=g).to(dev).requires_grad_(True)
    idx = torch.randint(0, 6, (2, 5, 3), generator=g).to(dev)
    out = cuda_ops.cuda_gather_apply(mem, idx, q)
    out.square().sum().backward()
    assert mem.grad is None
    q2 = q.detach().cpu().requires_grad_(True)
    ref = torch.einsum("bqrhk,bqk->bqrh", mem.detach().cpu()[torch.arange(2)[:, None, None], idx.cpu()], q2)
    ref.square().sum().backward()
    torch.testing.assert_close(q.grad.cpu(), q2.grad, rtol=1e-4, atol=1e-5)
    with torch.no_grad():
        before = capi.launch_count()
        fused = cuda_ops.cuda_gather_apply(mem, idx, q)
        assert capi.launch_count() > before
        torch.testing.assert_close(fused, out.detach(), rtol=1e-5, atol=1e-6)


# ---------------------------------------------------------------- apply query
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("shape", [(2, 3, 4, 5, 6), (4, 7, 8, 128, 128), (3, 5, 2, 9, 33), (2, 4, 16, 64)])
def test_apply_query(dev, dtype, shape):
    g = torch.Generator().manual_seed(2)
    mem = torch.randn(*shape, generator=g).to(dtype)
    qshape = shape[:2] + shape[-1:] if len(shape) == 5 else (shape[0], shape[-1])
    q = norm(torch.randn(*qshape, generator=g)).to(dtype)
    out = capi.apply_query_fwd(mem.to(dev), q.to(dev))
    out_op = torch.ops.grm_cuda.apply_query_forward(mem.to(dev), q.to(dev))
    assert torch.equal(out, out_op)
    ref = orc.apply_query(mem.double().numpy(), q.double().numpy())
    rtol, atol = (1e-5, 1e-5) if dtype == torch.float32 else (2e-2, 2e-3)
    np.testing.assert_allclose(out.double().cpu().numpy(), ref, rtol=rtol, atol=atol)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("shape", [(2, 3, 4, 5, 6), (2, 3, 8, 64, 128), (3, 4, 16, 64), (2, 5, 3, 32, 40)])
def test_apply_query_backward(dev, dtype, shape):
    """grad_memories (outer products dh q^T) and grad_queries (sum over slots and rows of
    dh M) against the oracle on the same 16-bit inputs: 1e-5 for float32, element by element
    at rtol 2e-2 / atol 2e-3 for bf16 / f16 (float32 accumulation, one rounding at the end)."""
    g = torch.Generator().manual_seed(3)
    mem = torch.randn(*shape, generator=g).to(dtype)
    qshape = shape[:2] + shape[-1:] if len(shape) == 5 else (shape[0], shape[-1])
    q = norm(torch.randn(*qshape, generator=g)).to(dtype)
    dh = torch.randn(*shape[:-1], generator=g).to(dtype)
    gm, gq = capi.apply_query_bwd(dh.to(dev), mem.to(dev), q.to(dev))
    assert gm.dtype == dtype and gq.dtype == dtype
    rgm, rgq = orc.apply_query_bwd(dh.double().numpy(), mem.double().numpy(), q.double().numpy())
    if dtype == torch.float32:
        np.testing.assert_allclose(gm.double().cpu().numpy(), rgm, rtol=1e-5, atol=1e-6)
        np.testing.assert_allclose(gq.double().cpu().numpy(), rgq, rtol=1e-5, atol=1e-5)
    else:
        np.testing.assert_allclose(gm.double().cpu().numpy(), rgm, rtol=2e-2, atol=2e-3)
        np.testing.assert_allclose(gq.double().cpu().numpy(), rgq, rtol=2e-2, atol=2e-3)


def test_apply_query_autograd_reference_case(dev):
    """examples/test_grm.py:167-194: native vs fallback forward and grads at 1e-5."""
    g = torch.Generator().manual_seed(9)
    mem = torch.randn(2, 3, 4, 5, 6, generator=g)
    q = norm(torch.randn(2, 3, 6, generator=g))

    def run(debug):
        mm = mem.to(dev).clone().requires_grad_(True)
        qq = q.to(dev).clone().requires_grad_(True)
        h = cuda_ops.cuda_apply_query(mm, qq, debug_fallback=debug)
        h.square().mean().backward()
        return h.detach(), mm.grad, qq.grad

    for a, b in zip(run(False), run(True)):
        torch.testing.assert_close(a, b, atol=1e-5, rtol=1e-5)


# ---------------------------------------------------------------- routing
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32, torch.float16])
@pytest.mark.parametrize("B,Q,S,D,k", [(2, 37, 256, 128, 8), (3, 300, 64, 512, 8), (1, 50, 512, 128, 16),
                                       (2, 20, 5, 16, 8), (2, 33, 40, 24, 32), (1, 10, 9, 130, 1)])
def test_topk_route_bit_exact(dev, dtype, B, Q, S, D, k):
    g = torch.Generator().manual_seed(B * 7 + S)
    q = norm(torch.randn(B, Q, D, generator=g)).to(dtype)
    keys = norm(torch.randn(B, S, D, generator=g)).to(dtype)
    scale = 1.0 / D ** 0.5
    gates, idx, sc = capi.topk_route(q.to(dev), keys.to(dev), k, scale)
    og, oi, osc = orc.topk_route(q.float().numpy(), keys.float().numpy(), k, scale)
    assert np.array_equal(idx.cpu().numpy(), oi)
    assert np.array_equal(sc.cpu().numpy(), osc)
    np.testing.assert_allclose(gates.cpu().numpy(), og, rtol=1e-5, atol=1e-6)
    g2, i2, s2 = torch.ops.grm_cuda.topk_route(q.to(dev), keys.to(dev), k, scale, 1.0)
    assert torch.equal(i2, idx) and torch.equal(s2, sc) and torch.equal(g2, gates)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32, torch.float16])
@pytest.mark.parametrize("B,T,seg,base,cap,S,D,k", [
    (2, 1000, 64, 0, 64, 16, 512, 8),     # config 4's shape class: windows grow from 0 to 15 keys
    (1, 8192, 64, 0, 64, 128, 64, 8),     # a full config-4 layer sequence, capacity 64 caps the window
    (3, 300, 7, 12, 20, 55, 96, 16),      # earlier archive entries (base), short partial last segment
    (2, 130, 13, 2, 5, 12, 40, 32),       # windows never longer than k: index order throughout
    (1, 64, 64, 0, 64, 1, 32, 8),         # one segment, empty archive: every slot empty
    (1, 600, 64, 0, 200, 10, 64, 8),      # capacity beyond one workgroup's key buffer: per-row kernel
    (2, 90, 9, 0, 16, 11, 30, 4),         # rows not 16-byte multiples: per-row kernel
    (1, 2048, 4, 0, 512, 512, 128, 16),   # config 5's causal windows in miniature: up to 511 keys, 2 key chunks
    (2, 700, 2, 100, 300, 450, 64, 8),    # base and capacity both bind; windows slide
])
def test_segment_route_bit_exact(dev, dtype, B, T, seg, base, cap, S, D, k):
    """Every segment routed over the archive of its moment in one launch,
    bit-exact against the oracle's per-window routing."""
    g = torch.Generator().manual_seed(T + S)
    q = norm(torch.randn(B, T, D, generator=g)).to(dtype)
    keys = norm(torch.randn(B, S, D, generator=g)).to(dtype)
    scale = 1.0 / D ** 0.5
    print(f"segment_route {dtype} B={B} T={T} seg={seg} base={base} cap={cap} S={S} D={D} k={k}", flush=True)
    gates, idx, sc = capi.segment_route(q.to(dev), keys.to(dev), k, seg, base, cap, scale)
    og, oi, osc = orc.segment_route(q.float().numpy(), keys.float().numpy(), k, seg, base, cap, scale)
    assert np.array_equal(idx.cpu().numpy(), oi)
    assert np.array_equal(sc.cpu().numpy(), osc)
    np.testing.assert_allclose(gates.cpu().numpy(), og, rtol=1e-5, atol=1e-6)
    g2, i2, s2 = torch.ops.grm_cuda.segment_route(q.to(dev), keys.to(dev), k, seg, base, cap, scale, 1.0)
    assert torch.equal(i2, idx) and torch.equal(s2, sc) and torch.equal(g2, gates)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_topk_route_beyond_128(dev, dtype):
    """top_k = 150 of 300 keys (beyond the select kernels' 128, with duplicate keys for
    ties): every key's exact score, then a stable sort on the device; indices and scores
    bit-exact against the oracle, no host round trip; and the per-window segment routing
    built on it matches the oracle's."""
    g = torch.Generator().manual_seed(15)
    base = norm(torch.randn(2, 150, 64, generator=g))
    keys = torch.cat([base, base], dim=1).to(dtype)  # every score appears twice
    q = norm(torch.randn(2, 70, 64, generator=g)).to(dtype)
    print(f"topk_route k=150 of 300 {dtype}", flush=True)
    generic = cuda_ops.extension_module().generic_path_calls()
    gates, idx, sc = torch.ops.grm_cuda.topk_route(q.to(dev), keys.to(dev), 150, 0.125, 1.0)
    assert cuda_ops.extension_module().generic_path_calls() == generic
    og, oi, osc = orc.topk_route(q.float().numpy(), keys.float().numpy(), 150, 0.125)
    assert np.array_equal(idx.cpu().numpy(), oi)
    assert np.array_equal(sc.cpu().numpy(), osc)
    np.testing.assert_allclose(gates.cpu().numpy(), og, rtol=1e-5, atol=1e-6)
    print(f"segment routing k=150 {dtype}", flush=True)
    # windows of 100-134 keys (at most k: index order), then of 160-194 keys (beyond k: the sort)
    for seg_base, cap in ((100, 180), (160, 250)):
        gates, idx, sc = cuda_ops.cuda_segment_route(q.to(dev), keys.to(dev), 150, 2, seg_base, cap, 0.125)
        og, oi, osc = orc.segment_route(q.float().numpy(), keys.float().numpy(), 150, 2, seg_base, cap, 0.125)
        assert np.array_equal(idx.cpu().numpy(), oi), (seg_base, cap)
        assert np.array_equal(sc.cpu().numpy(), osc), (seg_base, cap)
        np.testing.assert_allclose(gates.cpu().numpy(), og, rtol=1e-5, atol=1e-6)


def test_topk_route_ties(dev):
    """Duplicate keys give equal scores; the lower index must win every tie."""
    g = torch.Generator().manual_seed(6)
    base = norm(torch.randn(2, 8, 64, generator=g))
    keys = torch.cat([base, base, base[:, :3]], dim=1)  # each score appears 2-3 times
    q = norm(torch.randn(2, 25, 64, generator=g))
    gates, idx, sc = capi.topk_route(q.to(dev), keys.to(dev), 5, 0.125)
    og, oi, osc = orc.topk_route(q.numpy(), keys.numpy(), 5, 0.125)
    assert np.array_equal(idx.cpu().numpy(), oi)
    i = idx.cpu()
    s = sc.cpu()
    # within equal scores, indices ascend
    eq = s[..., 1:] == s[..., :-1]
    assert bool((i[..., 1:][eq] > i[..., :-1][eq]).all())


def test_topk_route_config3_slice(dev):
    """BASELINE config 3 routing geometry (S=256, d=128, k=8, bf16) on 8 of the 64 (b,h) pairs."""
    B, Q, S, D = 8, 2048, 256, 128
    g = torch.Generator().manual_seed(0)
    q = norm(torch.randn(B, Q, D, generator=g)).to(torch.bfloat16)
    keys = norm(torch.randn(B, S, D, generator=g)).to(torch.bfloat16)
    gates, idx, sc = capi.topk_route(q.to(dev), keys.to(dev), 8, 1.0 / D ** 0.5)
    og, oi, osc = orc.topk_route(q.float().numpy(), keys.float().numpy(), 8, 1.0 / D ** 0.5)
    assert np.array_equal(idx.cpu().numpy(), oi)
    assert np.array_equal(sc.cpu().numpy(), osc)


def _near_tie_route_inputs(B, Q, S, D, hot, copies, seed):
    """Keys that are element permutations of a few hot base keys, and queries whose
    elements are all equal: such scores are equal in exact arithmetic and differ only
    by the rounding of the FMA chain, so the top k is decided at the last bit."""
    g = torch.Generator().manual_seed(seed)
    keys = norm(torch.randn(B, S, D, generator=g))
    pos = torch.randperm(S, generator=g)[: hot * copies].view(hot, copies)
    for h in range(hot):
        base = norm(torch.ones(D) + 0.5 * torch.randn(D, generator=g))
        for c in range(copies):
            keys[:, pos[h, c]] = base[torch.randperm(D, generator=g)]
    q = norm(torch.randn(B, Q, D, generator=g))
    q[:, ::2] = 1.0 / D ** 0.5  # every other row: equal elements
    return q.to(torch.bfloat16), keys.to(torch.bfloat16)


@pytest.mark.parametrize("S,D,k,hot,copies", [(256, 128, 8, 3, 5), (256, 128, 3, 1, 4), (512, 128, 16, 4, 6),
                                              (100, 64, 8, 2, 3), (40, 24, 32, 3, 9), (300, 96, 1, 1, 30)])
def test_topk_route_near_ties(dev, S, D, k, hot, copies):
    """Rows whose best scores agree to the last few bits: the MFMA narrowing must keep
    every key the exact FMA chain ranks in the top k (and scan all keys when more than
    a few places are tied), so indices and scores still match the oracle bit for bit."""
    B, Q = 2, 70
    q, keys = _near_tie_route_inputs(B, Q, S, D, hot, copies, seed=S + k)
    scale = 1.0 / D ** 0.5
    gates, idx, sc = capi.topk_route(q.to(dev), keys.to(dev), k, scale)
    og, oi, osc = orc.topk_route(q.float().numpy(), keys.float().numpy(), k, scale)
    assert np.array_equal(idx.cpu().numpy(), oi)
    assert np.array_equal(sc.cpu().numpy(), osc)
    np.testing.assert_allclose(gates.cpu().numpy(), og, rtol=1e-5, atol=1e-6)


@pytest.mark.parametrize("S,D,k,copies", [(256, 128, 8, 256), (512, 128, 16, 60), (300, 64, 8, 40), (90, 32, 32, 90)])
def test_topk_route_candidate_overflow(dev, S, D, k, copies):
    """Rows with more near-best keys than the candidate lists hold (every key equal, or
    many copies of the best key): those rows are scored exactly over all keys; ties go
    to the lower index."""
    g = torch.Generator().manual_seed(S + copies)
    keys = norm(torch.randn(2, S, D, generator=g))
    best = norm(torch.randn(D, generator=g))
    pos = torch.randperm(S, generator=g)[:copies]
    keys[:, pos] = best
    q = norm(torch.randn(2, 600, D, generator=g))
    q[:, ::3] = best  # these rows score every copy of the best key highest, all tied
    q, keys = q.to(torch.bfloat16), keys.to(torch.bfloat16)
    scale = 1.0 / D ** 0.5
    gates, idx, sc = capi.topk_route(q.to(dev), keys.to(dev), k, scale)
    og, oi, osc = orc.topk_route(q.float().numpy(), keys.float().numpy(), k, scale)
    assert np.array_equal(idx.cpu().numpy(), oi)
    assert np.array_equal(sc.cpu().numpy(), osc)
    np.testing.assert_allclose(gates.cpu().numpy(), og, rtol=1e-5, atol=1e-6)


@pytest.mark.parametrize("B,Q,S,D,k", [(1, 70000, 100, 64, 8), (3, 1500, 33, 128, 16), (2, 2000, 257, 96, 4),
                                       (1, 1200, 2000, 32, 8)])
def test_topk_route_block_shapes(dev, B, Q, S, D, k):
    """Row counts that leave partial 512-row blocks and partial 64-row waves, key counts
    that are not multiples of 32, several blocks per workgroup (70000 rows of one batch
    entry), and an archive of 2000 keys."""
    g = torch.Generator().manual_seed(Q + S)
    q = norm(torch.randn(B, Q, D, generator=g)).to(torch.bfloat16)
    keys = norm(torch.randn(B, S, D, generator=g)).to(torch.bfloat16)
    scale = 1.0 / D ** 0.5
    gates, idx, sc = capi.topk_route(q.to(dev), keys.to(dev), k, scale)
    rows = torch.cat([torch.arange(0, 300), torch.arange(Q - 300, Q)]) if Q > 600 else torch.arange(Q)
    og, oi, osc = orc.topk_route(q[:, rows].float().numpy(), keys.float().numpy(), k, scale)
    assert np.array_equal(idx[:, rows].cpu().numpy(), oi)
    assert np.array_equal(sc[:, rows].cpu().numpy(), osc)
    np.testing.assert_allclose(gates[:, rows].cpu().numpy(), og, rtol=1e-5, atol=1e-6)


def test_topk_route_unit_scale_and_large_norms(dev):
    """Unnormalised bf16 inputs (norms up to ~1e3) and scale 1: the error bound of the
    narrowing scales with the norms, the indices stay exact."""
    g = torch.Generator().manual_seed(21)
    q = (torch.randn(3, 90, 128, generator=g) * torch.rand(3, 90, 1, generator=g) * 100).to(torch.bfloat16)
    keys = (torch.randn(3, 333, 128, generator=g) * 10).to(torch.bfloat16)
    gates, idx, sc = capi.topk_route(q.to(dev), keys.to(dev), 12, 1.0)
    og, oi, osc = orc.topk_route(q.float().numpy(), keys.float().numpy(), 12, 1.0)
    assert np.array_equal(idx.cpu().numpy(), oi)
    assert np.array_equal(sc.cpu().numpy(), osc)


# ---------------------------------------------------------------- fusion
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("N,R,H,ln", [(37, 8, 128, True), (5, 3, 512, True), (9, 0, 64, True), (12, 4, 100, False),
                                      (70, 16, 2048, True), (33, 5, 24, True), (300, 8, 128, False), (3, 1, 1000, True)])
def test_fuse_residual(dev, dtype, N, R, H, ln):
    g = torch.Generator().manual_seed(N)
    h = torch.randn(N, H, generator=g).to(dtype)
    r = torch.randn(N, R, H, generator=g).to(dtype)
    gt = torch.softmax(torch.randn(N, R, generator=g), -1) if R > 0 else torch.zeros(N, 0)
    w = (1 + 0.1 * torch.randn(H, generator=g)).to(dtype) if ln else None
    b = (0.1 * torch.randn(H, generator=g)).to(dtype) if ln else None
    out = capi.fuse_residual(h.to(dev), r.to(dev), gt.to(dev), None if w is None else w.to(dev),
                             None if b is None else b.to(dev))
    ref = orc.fuse_residual(h.double().numpy(), r.double().numpy(), gt.double().numpy(),
                            None if w is None else w.double().numpy(), None if b is None else b.double().numpy())
    rtol, atol = (1e-5, 1e-5) if dtype == torch.float32 else (2e-2, 2e-2)
    np.testing.assert_allclose(out.double().cpu().numpy(), ref, rtol=rtol, atol=atol)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("shape", [(2, 3, 8, 64, 128), (3, 4, 16, 64)])
def test_apply_query_backward_queries_only(dev, dtype, shape):
    """Memories that need no gradient (a retrieved archive): the backward computes grad_queries
    only, equal to apply_query_backward's, and never forms grad_memories."""
    g = torch.Generator().manual_seed(17)
    mem = torch.randn(*shape, generator=g).to(dtype).to(dev)
    qshape = shape[:2] + shape[-1:] if len(shape) == 5 else (shape[0], shape[-1])
    q = norm(torch.randn(*qshape, generator=g)).to(dtype).to(dev).requires_grad_(True)
    dh = torch.randn(*shape[:-1], generator=g).to(dtype).to(dev)
    _, gq_full = torch.ops.grm_cuda.apply_query_backward(dh, mem, q.detach())
    gq_only = torch.ops.grm_cuda.apply_query_backward_queries(dh, mem, q.detach())
    assert torch.equal(gq_only, gq_full)
    out = cuda_ops.cuda_apply_query(mem, q)
    (gq_auto,) = torch.autograd.grad(out, (q,), dh)
    assert torch.equal(gq_auto, gq_full)


@pytest.mark.parametrize("k,S", [(40, 300), (100, 257), (128, 2000)])
def test_topk_route_wide_k(dev, k, S):
    """top_k beyond 32 (up to 128) is routed on the GPU, bit-exact; both entry points."""
    g = torch.Generator().manual_seed(k + S)
    q = norm(torch.randn(2, 90, 64, generator=g)).to(torch.bfloat16)
    keys = norm(torch.randn(2, S, 64, generator=g)).to(torch.bfloat16)
    scale = 0.125
    gates, idx, sc = capi.topk_route(q.to(dev), keys.to(dev), k, scale)
    og, oi, osc = orc.topk_route(q.float().numpy(), keys.float().numpy(), k, scale)
    assert np.array_equal(idx.cpu().numpy(), oi) and np.array_equal(sc.cpu().numpy(), osc)
    np.testing.assert_allclose(gates.cpu().numpy(), og, rtol=1e-5, atol=1e-6)
    seg = 30
    gates, idx, sc = capi.segment_route(q.to(dev), keys.to(dev), k, seg, S - 3, S, scale)
    og, oi, osc = orc.segment_route(q.float().numpy(), keys.float().numpy(), k, seg, S - 3, S, scale)
    assert np.array_equal(idx.cpu().numpy(), oi) and np.array_equal(sc.cpu().numpy(), osc)


def test_routing_mixed_dtypes_stays_on_device(dev):
    """float32 queries against bf16 keys: both widened to float32 on the GPU (the values are
    exact), no host round trip; bit-exact against the oracle."""
    g = torch.Generator().manual_seed(77)
    q = norm(torch.randn(2, 50, 32, generator=g))
    keys = norm(torch.randn(2, 70, 32, generator=g)).to(torch.bfloat16)
    ext = cuda_ops.extension_module()
    before = ext.generic_path_calls()
    gates, idx, sc = torch.ops.grm_cuda.topk_route(q.to(dev), keys.to(dev), 8, 0.25, 1.0)
    g2, i2, s2 = torch.ops.grm_cuda.segment_route(q.to(dev), keys.to(dev), 8, 5, 60, 40, 0.25, 1.0)
    torch.cuda.synchronize()
    assert ext.generic_path_calls() == before
    og, oi, osc = orc.topk_route(q.numpy(), keys.float().numpy(), 8, 0.25)
    assert np.array_equal(idx.cpu().numpy(), oi) and np.array_equal(sc.cpu().numpy(), osc)
    og, oi, osc = orc.segment_route(q.numpy(), keys.float().numpy(), 8, 5, 60, 40, 0.25)
    assert np.array_equal(i2.cpu().numpy(), oi) and np.array_equal(s2.cpu().numpy(), osc)


# ---------------------------------------------------------------- fused retrieval
def _retrieve_fuse_ref(mem, idx, q, gates, h, w, b, eps=1e-5):
    """The oracle's gather -> apply (float64) -> residual + LayerNorm, with zero rows for
    indices outside [0, S)."""
    B, Q, R = idx.shape
    S, H = mem.shape[1], mem.shape[2]
    mem64 = mem.double().numpy()
    idx_np = idx.numpy()
    valid = (idx_np >= 0) & (idx_np < S)
    gathered, _ = orc.gather(mem64, np.where(valid, idx_np, 0))
    r = orc.apply_query(gathered, q.double().numpy()) * valid[..., None]
    return orc.fuse_residual(h.double().numpy().reshape(B * Q, H), r.reshape(B * Q, R, H),
                             gates.double().numpy().reshape(B * Q, R),
                             None if w is None else w.double().numpy(), None if b is None else b.double().numpy(),
                             eps).reshape(B, Q, H)


@pytest.mark.parametrize("mem_dtype", [torch.float32, torch.float16, torch.bfloat16])
@pytest.mark.parametrize("h_dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("B,Q,S,R,H,K,ln", [(2, 300, 37, 5, 128, 128, True), (3, 64, 8, 8, 512, 64, True),
                                            (1, 129, 300, 16, 200, 32, False), (2, 50, 5, 3, 8, 64, True),
                                            (1, 70, 3, 8, 264, 128, True)])
def test_retrieve_fuse(dev, mem_dtype, h_dtype, B, Q, S, R, H, K, ln):
    """retrieve_fuse (gather + apply + gate-weighted sum + residual + LayerNorm in one call)
    against the oracle's composition element by element at rtol 2e-2 / atol 2e-3 (the
    retrieved rows are kept as row-scaled float16: measured error ~1e-4), against the
    float32 two-kernel composition (gather_apply + fuse_residual), and run to run bit for
    bit: value widths of one to five 128-column tiles with a partial last tile, invalid
    indices (-1, S) contributing nothing, no LayerNorm."""
    g = torch.Generator().manual_seed(B * 7 + Q + H)
    q_dtype = torch.float16 if mem_dtype == torch.float16 and Q % 2 == 0 else torch.bfloat16
    mem = (torch.randn(B, S, H, K, generator=g) * 0.3).to(mem_dtype)
    idx = torch.randint(0, S, (B, Q, R), generator=g)
    idx[0, 1, 0] = -1
    idx[-1, -1, -1] = S
    q = norm(torch.randn(B, Q, K, generator=g)).to(q_dtype)
    gates = torch.softmax(torch.randn(B, Q, R, generator=g), dim=-1)
    h = torch.randn(B, Q, H, generator=g).to(h_dtype)
    w = (1 + 0.1 * torch.randn(H, generator=g)) if ln else None  # float32 LayerNorm parameters
    b = (0.1 * torch.randn(H, generator=g)) if ln else None
    print(f"retrieve_fuse B={B} Q={Q} S={S} R={R} H={H} K={K} mem {mem_dtype} q {q_dtype} h {h_dtype} ln={ln}",
          flush=True)
    D = lambda t: None if t is None else t.to(dev)  # noqa: E731
    bad = torch.zeros(1, dtype=torch.int32, device=dev)
    args = (D(mem), D(idx), D(q), D(gates), D(h), D(w), D(b))
    out = capi.retrieve_fuse(*args, bad_count=bad)
    out2 = capi.retrieve_fuse(*args)
    rows = capi.gather_apply(D(mem), D(idx), D(q), dtype=torch.float32)
    comp = capi.fuse_residual(D(h).float().reshape(B * Q, H), rows.reshape(B * Q, R, H), D(gates).reshape(B * Q, R),
                              D(w), D(b)).reshape(B, Q, H).to(h_dtype)
    torch.cuda.synchronize()
    assert out.dtype == h_dtype and out.shape == (B, Q, H)
    assert int(bad.item()) == 2
    assert torch.equal(out, out2), "retrieve_fuse is not deterministic"
    ref = _retrieve_fuse_ref(mem, idx, q, gates, h, w, b)
    got = out.float().cpu().double().numpy()
    np.testing.assert_allclose(got, ref, rtol=2e-2, atol=2e-3)
    if h_dtype == torch.float32:
        err = np.abs(got - ref).max() / max(np.abs(ref).max(), 1e-30)
        assert err < 2e-3, err
        torch.testing.assert_close(out, comp, rtol=2e-3, atol=2e-3)
    else:
        # the float32 composition rounded once to bf16: at most one bf16 step apart, mostly equal
        torch.testing.assert_close(out.float(), comp.float(), rtol=1e-2, atol=1e-2)


def test_retrieve_fuse_op_and_model_path(dev):
    """torch.ops.grm_cuda.retrieve_fuse on [B, Q, ...] tensors equals capi.retrieve_fuse, runs no
    generic path, and its unsupported inputs (float32 queries) take the two-kernel HIP
    composition with the same result as gather_apply + fuse_residual."""
    from rnn_with_grm_amd import cuda_ops

    g = torch.Generator().manual_seed(41)
    B, Q, S, R, H, K = 2, 100, 20, 8, 256, 64
    mem = (torch.randn(B, S, H, K, generator=g) * 0.1).to(dev)
    idx = torch.randint(0, S, (B, Q, R), generator=g).to(dev)
    q = norm(torch.randn(B, Q, K, generator=g)).to(torch.bfloat16).to(dev)
    gates = torch.softmax(torch.randn(B, Q, R, generator=g), -1).to(dev)
    h = torch.randn(B, Q, H, generator=g).to(dev)
    w, b = torch.ones(H, device=dev), torch.zeros(H, device=dev)
    ext = cuda_ops.extension_module()
    generic = ext.generic_path_calls()
    with torch.no_grad():
        a = cuda_ops.cuda_retrieve_fuse(mem, idx, q, gates, h, w, b)
    c = capi.retrieve_fuse(mem, idx, q, gates, h, w, b)
    assert torch.equal(a, c) and ext.generic_path_calls() == generic
    qf = q.float()
    with torch.no_grad():
        d = cuda_ops.cuda_retrieve_fuse(mem, idx, qf, gates, h, w, b)
    rows = capi.gather_apply(mem, idx, qf, dtype=torch.float32)
    e = capi.fuse_residual(h.reshape(B * Q, H), rows.reshape(B * Q, R, H), gates.reshape(B * Q, R), w, b)
    assert torch.equal(d, e.reshape(B, Q, H))


# ---------------------------------------------------------------- segment-window retrieval
def _window_indices(g, B, Q, R, S, seg, base, cap):
    """Routing-like indices: query t takes up to R distinct entries of its window
    [max(0, hi - cap), hi), hi = base + t // seg, the rest -1; then three bad pairs are
    planted (an entry past the window, one before it, and a repeat of an earlier route)
    where the window allows.  Returns the indices and the number of bad pairs."""
    idx = torch.full((B, Q, R), -1, dtype=torch.long)
    for bb in range(B):
        for t in range(Q):
            hi = base + t // seg
            lo = max(0, hi - cap)
            n = min(R, hi - lo)
            if n > 0:
                idx[bb, t, :n] = lo + torch.randperm(hi - lo, generator=g)[:n]
    bad = 0
    t = Q - 1
    hi = base + t // seg
    if hi < S and R >= 1:
        idx[0, t, 0] = hi  # past the window
        bad += 1
    t = Q // 2
    hi = base + t // seg
    if hi - cap > 0 and R >= 2:
        idx[-1, t, 1] = hi - cap - 1  # before the window
        bad += 1
    for t in range(Q):
        if R >= 3 and int(idx[0, t, 0]) >= 0 and int(idx[0, t, 2]) >= 0 and int(idx[0, t, 0]) < base + t // seg:
            idx[0, t, 2] = idx[0, t, 0]  # a repeat
            bad += 1
            break
    return idx, bad


def _window_valid_np(idx, seg, base, cap):
    B, Q, R = idx.shape
    hi = base + np.arange(Q)[None, :, None] // seg
    lo = np.maximum(hi - cap, 0)
    valid = (idx >= lo) & (idx < hi)
    for r in range(R):
        for r2 in range(r):
            valid[:, :, r] &= idx[:, :, r] != idx[:, :, r2]
    return valid


@pytest.mark.parametrize("mem_dtype,q_dtype", [(torch.float16, torch.bfloat16), (torch.bfloat16, torch.bfloat16),
                                               (torch.float32, torch.bfloat16), (torch.float16, torch.float16)])
@pytest.mark.parametrize("h_dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("B,Q,H,K,seg,base,cap,R,ln", [(2, 300, 128, 64, 64, 0, 64, 8, True),
                                                       (1, 1000, 512, 64, 64, 3, 64, 8, True),
                                                       (2, 257, 200, 32, 7, 5, 20, 4, False),
                                                       (1, 130, 40, 48, 1, 0, 100, 16, True),
                                                       (3, 64, 264, 128, 16, 2, 9, 8, True)])
def test_segment_retrieve_fuse(dev, mem_dtype, q_dtype, h_dtype, B, Q, H, K, seg, base, cap, R, ln):
    """segment_retrieve_fuse (each query block walks its routing window, the routes summed in
    the kernel) against the oracle's gather -> apply -> residual + LayerNorm over the window's
    valid pairs, at retrieve_fuse's bars (rtol 2e-2 / atol 2e-3; the sums leave as tile-scaled
    float16); against the float32 two-kernel composition over the same pairs; bad pairs
    (outside the window, repeated) counted and contributing nothing, empty slots (-1) not
    counted; run to run bit for bit.  Windows of one entry per token (segment_len 1), partial
    value tiles, key widths 32 / 48 / 64 / 128."""
    g = torch.Generator().manual_seed(B * 11 + Q + H + K)
    S = base + (Q - 1) // seg + 1
    mem = (torch.randn(B, S, H, K, generator=g) * 0.3).to(mem_dtype)
    idx, nbad = _window_indices(g, B, Q, R, S, seg, base, cap)
    q = norm(torch.randn(B, Q, K, generator=g)).to(q_dtype)
    gates = torch.softmax(torch.randn(B, Q, R, generator=g), dim=-1)
    h = torch.randn(B, Q, H, generator=g).to(h_dtype)
    w = (1 + 0.1 * torch.randn(H, generator=g)) if ln else None
    b = (0.1 * torch.randn(H, generator=g)) if ln else None
    print(f"segment_retrieve_fuse B={B} Q={Q} H={H} K={K} seg={seg} base={base} cap={cap} R={R} mem {mem_dtype} "
          f"q {q_dtype} h {h_dtype} ln={ln}", flush=True)
    D = lambda t: None if t is None else t.to(dev)  # noqa: E731
    bad = torch.zeros(1, dtype=torch.int32, device=dev)
    args = (D(mem), D(idx), D(q), D(gates), D(h), seg, base, cap, D(w), D(b))
    out = capi.segment_retrieve_fuse(*args, bad_count=bad)
    out2 = capi.segment_retrieve_fuse(*args)
    valid = _window_valid_np(idx.numpy(), seg, base, cap)
    vt = torch.from_numpy(valid)
    idx_m = torch.where(vt, idx, torch.zeros_like(idx))
    rows = capi.gather_apply(D(mem), D(idx_m), D(q), dtype=torch.float32) * D(vt).unsqueeze(-1)
    comp = capi.fuse_residual(D(h).float().reshape(B * Q, H), rows.reshape(B * Q, R, H),
                              (D(gates) * D(vt)).reshape(B * Q, R), D(w), D(b)).reshape(B, Q, H).to(h_dtype)
    torch.cuda.synchronize()
    assert out.dtype == h_dtype and out.shape == (B, Q, H)
    assert int(bad.item()) == nbad
    assert torch.equal(out, out2), "segment_retrieve_fuse is not deterministic"
    ref = _retrieve_fuse_ref(mem, torch.where(vt, idx, torch.full_like(idx, -1)), q, gates, h, w, b)
    got = out.float().cpu().double().numpy()
    np.testing.assert_allclose(got, ref, rtol=2e-2, atol=2e-3)
    if h_dtype == torch.float32:
        err = np.abs(got - ref).max() / max(np.abs(ref).max(), 1e-30)
        assert err < 2e-3, err
        torch.testing.assert_close(out, comp, rtol=2e-3, atol=2e-3)
    else:
        torch.testing.assert_close(out.float(), comp.float(), rtol=1e-2, atol=1e-2)


def test_segment_retrieve_fuse_config4_geometry(dev):
    """One config-4 layer's retrieval at full size (4 x 8192 tokens, 64-token segments, capacity
    64, top-8, float16 archive 512 x 64, bf16 queries and rows, LayerNorm) with the indices and
    gates of segment routing: the window kernel against retrieve_fuse over the same pairs (both
    keep tile-scaled float16 intermediates) and against the float32 two-kernel composition on
    two sequences."""
    g = torch.Generator().manual_seed(44)
    B, T, H, K, seg, cap, R = 4, 8192, 512, 64, 64, 64, 8
    S = T // seg
    mem = (torch.randn(B, S, H, K, generator=g) * 0.05).to(torch.float16).to(dev)
    q = norm(torch.randn(B, T, K, generator=g)).to(torch.bfloat16).to(dev)
    keys = norm(torch.randn(B, S, K, generator=g)).to(torch.bfloat16).to(dev)
    h = torch.randn(B, T, H, generator=g).to(torch.bfloat16).to(dev)
    w = (1 + 0.1 * torch.randn(H, generator=g)).to(dev)
    b = (0.1 * torch.randn(H, generator=g)).to(dev)
    print("segment_retrieve_fuse config-4 geometry", flush=True)
    gates, idx, _ = capi.segment_route(q, keys, R, seg, 0, cap, K ** -0.5, 1.0)
    bad = torch.zeros(1, dtype=torch.int32, device=dev)
    out = capi.segment_retrieve_fuse(mem, idx, q, gates, h, seg, 0, cap, w, b, bad_count=bad)
    ref = capi.retrieve_fuse(mem, idx.clamp(min=0), q, gates, h, w, b)
    torch.cuda.synchronize()
    assert int(bad.item()) == 0
    torch.testing.assert_close(out.float(), ref.float(), rtol=1e-2, atol=1e-2)
    assert (out != ref).float().mean().item() < 0.05
    for bb in (0, 3):
        rows = capi.gather_apply(mem[bb:bb + 1], idx[bb:bb + 1].clamp(min=0), q[bb:bb + 1], dtype=torch.float32)
        comp = capi.fuse_residual(h[bb].float(), rows.reshape(T, R, H), gates[bb].reshape(T, R), w, b)
        torch.testing.assert_close(out[bb].float(), comp, rtol=1e-2, atol=1e-2)


def test_segment_retrieve_fuse_op_and_fallbacks(dev):
    """torch.ops.grm_cuda.segment_retrieve_fuse equals capi.segment_retrieve_fuse with no generic
    path; float32 queries take retrieve_fuse over the masked pairs (same result as the float32
    composition over the window's pairs); cuda_segment_retrieve_fuse's PyTorch fallback agrees."""
    from rnn_with_grm_amd import cuda_ops

    g = torch.Generator().manual_seed(43)
    B, Q, H, K, seg, base, cap, R = 2, 500, 256, 64, 32, 4, 12, 8
    S = base + (Q - 1) // seg + 1
    idx, _ = _window_indices(g, B, Q, R, S, seg, base, cap)
    mem = (torch.randn(B, S, H, K, generator=g) * 0.1).to(dev)
    idx = idx.to(dev)
    q = norm(torch.randn(B, Q, K, generator=g)).to(torch.bfloat16).to(dev)
    gates = torch.softmax(torch.randn(B, Q, R, generator=g), -1).to(dev)
    h = torch.randn(B, Q, H, generator=g).to(dev)
    w, b = torch.ones(H, device=dev), torch.zeros(H, device=dev)
    ext = cuda_ops.extension_module()
    generic = ext.generic_path_calls()
    with torch.no_grad():
        a = cuda_ops.cuda_segment_retrieve_fuse(mem, idx, q, gates, h, w, b, 1e-5, seg, base, cap)
    c = capi.segment_retrieve_fuse(mem, idx, q, gates, h, seg, base, cap, w, b)
    assert torch.equal(a, c) and ext.generic_path_calls() == generic
    with torch.no_grad():
        fb = cuda_ops.cuda_segment_retrieve_fuse(mem, idx, q, gates, h, w, b, 1e-5, seg, base, cap,
                                                 debug_fallback=True)
    torch.testing.assert_close(fb, a, rtol=2e-3, atol=2e-3)
    qf = q.float()
    with torch.no_grad():
        d = cuda_ops.cuda_segment_retrieve_fuse(mem, idx, qf, gates, h, w, b, 1e-5, seg, base, cap)
    valid = torch.from_numpy(_window_valid_np(idx.cpu().numpy(), seg, base, cap)).to(dev)
    rows = capi.gather_apply(mem, torch.where(valid, idx, torch.zeros_like(idx)), qf, dtype=torch.float32)
    e = capi.fuse_residual(h.reshape(B * Q, H), (rows * valid.unsqueeze(-1)).reshape(B * Q, R, H),
                           (gates * valid).reshape(B * Q, R), w, b)
    torch.testing.assert_close(d, e.reshape(B, Q, H), rtol=1e-5, atol=1e-5)


def test_segment_retrieve_fuse_wide_window_falls_back(dev):
    """A capacity wider than one block of queries can hold (capacity + 95 / segment_len + 1 > 256
    entries): the C entry rejects it before any launch (GRM_HIP_EUNSUPPORTED) and the op runs
    retrieve_fuse over the masked pairs, with the same result as the float32 composition over the
    window's valid pairs."""
    from rnn_with_grm_amd import cuda_ops

    g = torch.Generator().manual_seed(45)
    B, Q, H, K, seg, base, cap, R = 1, 600, 128, 64, 2, 0, 300, 8
    S = base + (Q - 1) // seg + 1
    idx, _ = _window_indices(g, B, Q, R, S, seg, base, cap)
    mem = (torch.randn(B, S, H, K, generator=g) * 0.1).to(torch.float16).to(dev)
    q = norm(torch.randn(B, Q, K, generator=g)).to(torch.bfloat16).to(dev)
    gates = torch.softmax(torch.randn(B, Q, R, generator=g), -1).to(dev)
    h = torch.randn(B, Q, H, generator=g).to(torch.bfloat16).to(dev)
    w, b = torch.ones(H, device=dev), torch.zeros(H, device=dev)
    idx = idx.to(dev)
    with pytest.raises(RuntimeError, match="use retrieve_fuse"):
        capi.segment_retrieve_fuse(mem, idx, q, gates, h, seg, base, cap, w, b)
    print("segment_retrieve_fuse wide window", flush=True)
    with torch.no_grad():
        out = cuda_ops.cuda_segment_retrieve_fuse(mem, idx, q, gates, h, w, b, 1e-5, seg, base, cap)
    valid = torch.from_numpy(_window_valid_np(idx.cpu().numpy(), seg, base, cap)).to(dev)
    rows = capi.gather_apply(mem, torch.where(valid, idx, torch.zeros_like(idx)), q, dtype=torch.float32)
    comp = capi.fuse_residual(h.float().reshape(B * Q, H), (rows * valid.unsqueeze(-1)).reshape(B * Q, R, H),
                              (gates * valid).reshape(B * Q, R), w, b).reshape(B, Q, H).to(torch.bfloat16)
    torch.cuda.synchronize()
    torch.testing.assert_close(out.float(), comp.float(), rtol=1e-2, atol=1e-2)


# ---------------------------------------------------------------- gather_apply backward (queries)
@pytest.mark.parametrize("mem_dtype", [torch.float32, torch.float16, torch.bfloat16])
@pytest.mark.parametrize("B,Q,S,R,H,K", [(2, 100, 37, 5, 128, 128), (3, 64, 8, 8, 512, 64), (1, 129, 300, 16, 200, 32),
                                         (2, 50, 5, 3, 8, 64), (1, 70, 3, 8, 40, 20), (1, 33, 6, 4, 30, 64),
                                         (1, 1000, 4, 4, 64, 64)])
def test_gather_apply_bwd_queries(dev, mem_dtype, B, Q, S, R, H, K):
    """The transposed apply (per pair M[idx]^T g, float32) summed over routes against the oracle's
    apply-query backward on the gathered states, at 1e-5 of the gradient's scale; invalid
    indices give zero rows and are counted."""
    g = torch.Generator().manual_seed(B + Q + H + K)
    mem = (torch.randn(B, S, H, K, generator=g) * 0.3).to(mem_dtype)
    idx = torch.randint(0, S, (B, Q, R), generator=g)
    idx[0, 2, 1] = -1
    grad = torch.randn(B, Q, R, H, generator=g)
    q = norm(torch.randn(B, Q, K, generator=g))
    bad = torch.zeros(1, dtype=torch.int32, device=dev)
    print(f"gather_apply_bwd_queries B={B} Q={Q} S={S} R={R} H={H} K={K} {mem_dtype}", flush=True)
    gp = capi.gather_apply_bwd_queries(mem.to(dev), idx.to(dev), grad.to(dev), bad_count=bad)
    torch.cuda.synchronize()
    assert int(bad.item()) == 1
    assert not gp[0, 2, 1].any()
    valid = (idx >= 0).numpy()
    gathered, _ = orc.gather(mem.double().numpy(), np.where(valid, idx.numpy(), 0))
    gathered = gathered * valid[..., None, None]
    _, ref = orc.apply_query_bwd(grad.double().numpy(), gathered, q.double().numpy())
    # float32 sums of H products per pair and R pairs: 1e-5 of the gradient's scale
    np.testing.assert_allclose(gp.sum(2).double().cpu().numpy(), ref, rtol=1e-5,
                               atol=1e-5 * max(1.0, float(np.abs(ref).max())))


def test_gather_apply_native_queries_gradient(dev):
    """With a detached archive and queries that need a gradient, cuda_gather_apply runs the native
    op with the transposed apply as its backward (no gathered states, no generic path); the
    queries' gradient equals the composition's on the CPU."""
    g = torch.Generator().manual_seed(23)
    mem = (torch.randn(2, 9, 64, 32, generator=g) * 0.2).to(torch.float16).to(dev)
    idx = torch.randint(0, 9, (2, 40, 4), generator=g).to(dev)
    q = norm(torch.randn(2, 40, 32, generator=g)).to(torch.bfloat16).to(dev).requires_grad_(True)
    ext = cuda_ops.extension_module()
    generic = ext.generic_path_calls()
    out = cuda_ops.cuda_gather_apply(mem, idx, q, torch.float32)
    (out.square().sum()).backward()
    torch.cuda.synchronize()
    assert ext.generic_path_calls() == generic
    q2 = q.detach().cpu().float().requires_grad_(True)
    sel = mem.cpu().float()[torch.arange(2)[:, None, None], idx.cpu()]
    ref = torch.einsum("bqrhk,bqk->bqrh", sel, q2)
    ref.square().sum().backward()
    torch.testing.assert_close(out.detach().cpu(), ref.detach(), rtol=1e-5, atol=1e-5)
    torch.testing.assert_close(q.grad.float().cpu(), q2.grad, rtol=1e-2, atol=1e-2)  # q.grad is bf16


@pytest.mark.parametrize("Q", [700, 8200])
def test_empty_slot_blocks(dev, Q):
    """The short windows of the first segments leave whole blocks of empty slots (-1), which
    a wave zeroes one row per lane.  gather_apply (float32 rows), retrieve_fuse (row-scaled
    float16 rows and their scales) and the queries' gradient, through the one-workgroup sort
    (5600 pairs) and the chunked sort (65600 pairs), against the oracle; empty slots counted."""
    B, S, R, H, K = 2, 37, 8, 128, 16
    g = torch.Generator().manual_seed(Q)
    mem = (torch.randn(B, S, H, K, generator=g) * 0.3).to(torch.float16)
    idx = torch.randint(0, S, (B, Q, R), generator=g)
    idx[:, : Q // 3, 2:] = -1           # 48 of every 64 consecutive pairs empty
    idx[1, Q // 2:Q // 2 + 40, :] = -1  # whole queries empty
    n_bad = int((idx < 0).sum())
    q = norm(torch.randn(B, Q, K, generator=g)).to(torch.bfloat16)
    gates = torch.softmax(torch.randn(B, Q, R, generator=g), dim=-1)
    h = torch.randn(B, Q, H, generator=g)
    w, b = 1 + 0.1 * torch.randn(H, generator=g), 0.1 * torch.randn(H, generator=g)
    grad = torch.randn(B, Q, R, H, generator=g)
    print(f"empty slot blocks Q={Q} bad={n_bad}", flush=True)
    ok = (idx >= 0).numpy()
    gathered, _ = orc.gather(mem.double().numpy(), np.where(ok, idx.numpy(), 0))
    gathered = gathered * ok[..., None, None]
    D = lambda t: t.to(dev)  # noqa: E731
    for name in ("gather_apply", "retrieve_fuse", "bwd_queries"):
        bad = torch.zeros(1, dtype=torch.int32, device=dev)
        if name == "gather_apply":
            out = capi.gather_apply(D(mem), D(idx), D(q), bad_count=bad, dtype=torch.float32)
            ref = orc.apply_query(gathered, q.double().numpy())
            np.testing.assert_allclose(out.cpu().double().numpy(), ref, rtol=1e-5, atol=1e-6)
        elif name == "retrieve_fuse":
            out = capi.retrieve_fuse(D(mem), D(idx), D(q), D(gates), D(h), D(w), D(b), bad_count=bad)
            ref = _retrieve_fuse_ref(mem, idx, q, gates, h, w, b)
            np.testing.assert_allclose(out.cpu().double().numpy(), ref, rtol=2e-3, atol=2e-3)
        else:
            out = capi.gather_apply_bwd_queries(D(mem), D(idx), D(grad), bad_count=bad)
            assert not out[:, : Q // 3, 2:].any()
            _, ref = orc.apply_query_bwd(grad.double().numpy(), gathered, q.double().numpy())
            np.testing.assert_allclose(out.sum(2).double().cpu().numpy(), ref, rtol=1e-5,
                                       atol=1e-5 * max(1.0, float(np.abs(ref).max())))
        torch.cuda.synchronize()
        assert int(bad.item()) == n_bad, name


# ---------------------------------------------------------------- gather_apply backward (tokens)
def _pair_bwd_ref(mem, idx, grad_tokens):
    """Per (query, route) pair M[idx]^T g[q] from the oracle, each pair a one-route rank-4
    apply-query backward; invalid indices give zero rows."""
    B, Q, R = idx.shape
    H, K = mem.shape[2], mem.shape[3]
    ok = (idx >= 0).numpy()
    gathered, _ = orc.gather(mem.double().numpy(), np.where(ok, idx.numpy(), 0))
    gathered = (gathered * ok[..., None, None]).reshape(B * Q * R, 1, H, K)
    g = np.repeat(grad_tokens.double().numpy()[:, :, None, :], R, axis=2).reshape(B * Q * R, 1, H)
    _, gq = orc.apply_query_bwd(g, gathered, np.zeros((B * Q * R, K)))
    return gq.reshape(B, Q, R, K)


@pytest.mark.parametrize("mem_dtype", [torch.float32, torch.float16, torch.bfloat16])
@pytest.mark.parametrize("B,Q,S,R,H,K", [(2, 100, 37, 5, 128, 128), (3, 64, 8, 8, 512, 64), (1, 129, 300, 16, 200, 32),
                                         (1, 70, 3, 8, 40, 20), (1, 1000, 4, 4, 64, 64)])
def test_gather_apply_bwd_tokens(dev, mem_dtype, B, Q, S, R, H, K):
    """One float32 gradient row per query shared by its routes: every pair's M[idx]^T g[q]
    against the oracle at 1e-5 of the gradient's scale, invalid indices zero and counted, and
    bit-identical to the per-pair entry point given that row repeated for each route."""
    g = torch.Generator().manual_seed(B * Q + S + H + K)
    mem = (torch.randn(B, S, H, K, generator=g) * 0.3).to(mem_dtype)
    idx = torch.randint(0, S, (B, Q, R), generator=g)
    idx[0, 2, 1] = -1
    gx = torch.randn(B, Q, H, generator=g)
    bad = torch.zeros(1, dtype=torch.int32, device=dev)
    print(f"gather_apply_bwd_tokens B={B} Q={Q} S={S} R={R} H={H} K={K} {mem_dtype}", flush=True)
    md, idd, gd = mem.to(dev), idx.to(dev), gx.to(dev)
    gp = capi.gather_apply_bwd_tokens(md, idd, gd, bad_count=bad)
    pairs = capi.gather_apply_bwd_queries(md, idd, gd.unsqueeze(2).expand(B, Q, R, H).contiguous())
    torch.cuda.synchronize()
    assert int(bad.item()) == 1
    assert not gp[0, 2, 1].any()
    ref = _pair_bwd_ref(mem, idx, gx)
    np.testing.assert_allclose(gp.double().cpu().numpy(), ref, rtol=1e-5,
                               atol=1e-5 * max(1.0, float(np.abs(ref).max())))
    assert torch.equal(gp, pairs)


@pytest.mark.parametrize("h_dtype,ln", [(torch.bfloat16, True), (torch.float32, True), (torch.float32, False)])
def test_retrieve_fuse_training_gradients(dev, h_dtype, ln):
    """The training form of cuda_retrieve_fuse (float32 rows, residual, LayerNorm, and a backward
    through the token-gradient kernel): no generic-path call, and the output and the gradients of
    queries, gates, h and the LayerNorm parameters against autograd through the float64
    composition on the CPU.  16-bit q and h enter both sides with the same values; the 16-bit
    results carry one rounding of their own dtype."""
    g = torch.Generator().manual_seed(31)
    B, S, Q, R, H, K = 2, 11, 300, 8, 128, 64
    mem = (torch.randn(B, S, H, K, generator=g) * 0.2).to(torch.float16)
    idx = torch.randint(0, S, (B, Q, R), generator=g)
    q0 = norm(torch.randn(B, Q, K, generator=g)).to(h_dtype)
    g0 = torch.softmax(torch.randn(B, Q, R, generator=g), -1)
    h0 = torch.randn(B, Q, H, generator=g).to(h_dtype)
    w0, b0 = 1 + 0.1 * torch.randn(H, generator=g), 0.1 * torch.randn(H, generator=g)
    gout = torch.randn(B, Q, H, generator=g).to(h_dtype)
    print(f"retrieve_fuse training gradients {h_dtype} ln={ln}", flush=True)
    leaves = [t.to(dev).requires_grad_(True) for t in (q0, g0, h0, w0, b0)]
    q, gates, h, w, b = leaves
    ext = cuda_ops.extension_module()
    generic = ext.generic_path_calls()
    out = cuda_ops.cuda_retrieve_fuse(mem.to(dev), idx.to(dev), q, gates, h, w if ln else None, b if ln else None)
    assert "RetrieveFuse" in type(out.grad_fn).__name__
    wrt = leaves if ln else leaves[:3]
    grads = torch.autograd.grad(out, wrt, gout.to(dev))
    torch.cuda.synchronize()
    assert ext.generic_path_calls() == generic
    d = [t.detach().double().requires_grad_(True) for t in (q0, g0, h0, w0, b0)]
    sel = mem.double()[torch.arange(B)[:, None, None], idx]
    x = d[2] + torch.einsum("bqr,bqrh->bqh", d[1], torch.einsum("bqrhk,bqk->bqrh", sel, d[0]))
    ref = torch.nn.functional.layer_norm(x, (H,), d[3], d[4], 1e-5) if ln else x
    rgrads = torch.autograd.grad(ref, d if ln else d[:3], gout.double())
    tol = 1e-4 if h_dtype == torch.float32 else 1e-2
    torch.testing.assert_close(out.detach().double().cpu(), ref.detach(), rtol=tol, atol=tol)
    for name, got, want in zip("q gates h w b".split(), grads, rgrads):
        assert got.dtype == (torch.float32 if name in ("gates", "w", "b") else h_dtype), name
        scale = max(1.0, float(want.abs().max()))
        torch.testing.assert_close(got.double().cpu(), want, rtol=tol, atol=tol * scale, msg=name)


# ---------------------------------------------------------------- segment routing, MFMA-narrowed windows
def _route_both(dev, monkeypatch, q, keys, k, seg, base, cap, scale):
    """segment_route through the MFMA-narrowed window kernel and through the all-exact one
    (GRM_HIP_ROUTE_WSEL=0), on the device."""
    qd, kd = q.to(dev), keys.to(dev)
    out = capi.segment_route(qd, kd, k, seg, base, cap, scale)
    monkeypatch.setenv("GRM_HIP_ROUTE_WSEL", "0")
    ref = capi.segment_route(qd, kd, k, seg, base, cap, scale)
    monkeypatch.delenv("GRM_HIP_ROUTE_WSEL")
    torch.cuda.synchronize()
    return out, ref


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("B,T,seg,base,cap,S,D,k", [
    (2, 2048, 64, 0, 64, 32, 512, 8),      # config 4's routing: hidden 512, 64-token segments, top-8 of 64
    (1, 1500, 64, 40, 64, 63, 512, 8),     # a filled archive: every window 64 keys
    (2, 700, 50, 3, 100, 17, 256, 16),     # segments straddle 32-row workgroups; up to 101 keys a workgroup
    (1, 900, 24, 0, 120, 37, 136, 32),     # k = 32, windows of 120 keys
    (1, 333, 7, 60, 16, 107, 512, 8),      # short segments: several windows per workgroup
    (1, 400, 64, 0, 64, 7, 1024, 4),       # d = 1024, windows below and above k
])
def test_segment_route_window_select(dev, monkeypatch, dtype, B, T, seg, base, cap, S, D, k):
    """Segment routing with 16-bit inputs whose windows fit one workgroup: the MFMA-narrowed
    window kernel, bit-exact against the oracle's per-window routing and equal to the all-exact
    window kernel (indices, scores and gates)."""
    g = torch.Generator().manual_seed(T + S + D)
    q = torch.randn(B, T, D, generator=g).to(dtype)
    keys = (torch.randn(B, S, D, generator=g) * 0.5).to(dtype)
    scale = 1.0 / D ** 0.5
    print(f"window select {dtype} B={B} T={T} seg={seg} base={base} cap={cap} S={S} D={D} k={k}", flush=True)
    (gates, idx, sc), (g0, i0, s0) = _route_both(dev, monkeypatch, q, keys, k, seg, base, cap, scale)
    og, oi, osc = orc.segment_route(q.float().numpy(), keys.float().numpy(), k, seg, base, cap, scale)
    assert np.array_equal(idx.cpu().numpy(), oi)
    assert np.array_equal(sc.cpu().numpy(), osc)
    np.testing.assert_allclose(gates.cpu().numpy(), og, rtol=1e-5, atol=1e-6)
    assert torch.equal(idx, i0) and torch.equal(sc, s0) and torch.equal(gates, g0)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_segment_route_window_select_ties(dev, monkeypatch, dtype):
    """Windows full of exact and near ties: duplicated keys (equal scores: the lower index wins),
    keys one 16-bit step apart, and rows whose every window key is a candidate (all keys equal),
    which takes several passes of exact chains per row; against the oracle and the all-exact
    kernel."""
    g = torch.Generator().manual_seed(77)
    B, T, seg, cap, S, D, k = 2, 640, 32, 128, 100, 384, 32  # base 81: windows of 81 .. 100 keys
    base_keys = torch.randn(B, 6, D, generator=g)
    keys = base_keys[:, torch.randint(0, 6, (S,), generator=g)].clone()  # many exact duplicates
    keys[:, ::3, 5] += 2.0 ** -6                                          # near duplicates
    keys[1] = base_keys[1, 0]                                             # batch 1: all keys equal
    keys = keys.to(dtype)
    q = (base_keys[:, torch.randint(0, 6, (T,), generator=g)] + 0.01 * torch.randn(B, T, D, generator=g)).to(dtype)
    scale = 0.05
    print(f"window select ties {dtype}", flush=True)
    (gates, idx, sc), (g0, i0, s0) = _route_both(dev, monkeypatch, q, keys, k, seg, 81, cap, scale)
    og, oi, osc = orc.segment_route(q.float().numpy(), keys.float().numpy(), k, seg, 81, cap, scale)
    assert np.array_equal(idx.cpu().numpy(), oi)
    assert np.array_equal(sc.cpu().numpy(), osc)
    assert torch.equal(idx, i0) and torch.equal(sc, s0) and torch.equal(gates, g0)


def test_segment_route_window_select_nonfinite(dev, monkeypatch):
    """A NaN query row and an infinite key take the exact path (the candidate bound is not
    finite): the same indices, scores and gates as the all-exact window kernel, NaN for NaN."""
    g = torch.Generator().manual_seed(78)
    q = torch.randn(1, 256, 512, generator=g)
    keys = torch.randn(1, 12, 512, generator=g)
    q[0, 70, 3] = float("nan")
    q = q.to(torch.bfloat16)
    for bad_key in (False, True):
        kk = keys.clone()
        if bad_key:
            kk[0, 2, 9] = float("inf")
        print(f"window select non-finite bad_key={bad_key}", flush=True)
        (gates, idx, sc), (g0, i0, s0) = _route_both(dev, monkeypatch, q, kk.to(torch.bfloat16), 4, 32, 0, 64,
                                                     0.04)
        assert torch.equal(idx, i0)
        assert torch.equal(torch.nan_to_num(sc, nan=7.0), torch.nan_to_num(s0, nan=7.0))
        assert torch.equal(torch.nan_to_num(gates, nan=7.0), torch.nan_to_num(g0, nan=7.0))


@pytest.mark.parametrize("B,Q,S,R,H,K", [(4, 2048, 128, 8, 512, 64), (2, 300, 9, 5, 200, 40), (1, 129, 30, 16, 72, 128),
                                         (2, 64, 3, 4, 36, 8)])
def test_transposed_apply_f16_split(dev, monkeypatch, B, Q, S, R, H, K):
    """Float16 archives: the 16-bit MFMA transposed apply (each 32-value chunk of a gradient row
    scaled by a power of two and split into two float16 parts) against the fp32 MFMA kernel
    (GRM_HIP_APPLY_T16=0) at 1e-5 of the gradient's scale, per pair and in the token form, with
    gradient rows spanning 30 binary orders of magnitude, an all-zero row and ragged hidden and
    key widths; and against the oracle."""
    g = torch.Generator().manual_seed(B + Q + H)
    mem = (torch.randn(B, S, H, K, generator=g) * 0.3).to(torch.float16)
    idx = torch.randint(0, S, (B, Q, R), generator=g)
    idx[0, 1, 0] = -1
    gx = torch.randn(B, Q, H, generator=g) * torch.exp2(torch.randint(-15, 15, (B, Q, 1), generator=g).float())
    gx[0, 3] = 0.0
    gp = torch.randn(B, Q, R, H, generator=g)
    print(f"f16 split transposed apply B={B} Q={Q} S={S} R={R} H={H} K={K}", flush=True)
    md, idd = mem.to(dev), idx.to(dev)
    tok = capi.gather_apply_bwd_tokens(md, idd, gx.to(dev))
    pair = capi.gather_apply_bwd_queries(md, idd, gp.to(dev))
    monkeypatch.setenv("GRM_HIP_APPLY_T16", "0")
    tok32 = capi.gather_apply_bwd_tokens(md, idd, gx.to(dev))
    pair32 = capi.gather_apply_bwd_queries(md, idd, gp.to(dev))
    monkeypatch.delenv("GRM_HIP_APPLY_T16")
    torch.cuda.synchronize()
    assert not tok[0, 1, 0].any() and not pair[0, 1, 0].any()
    for got, ref32 in ((tok, tok32), (pair, pair32)):
        got, ref32 = got.cpu().double(), ref32.cpu().double()
        # per query row: the error is relative to that row's scale
        scale = ref32.abs().amax(dim=(2, 3), keepdim=True).clamp(min=1e-30)
        assert float(((got - ref32).abs() / scale).max()) <= 1e-5
    ref = _pair_bwd_ref(mem, idx, gx)
    scale = np.abs(ref).max(axis=(2, 3), keepdims=True).clip(1e-30)
    assert float((np.abs(tok.cpu().double().numpy() - ref) / scale).max()) <= 1e-5


def test_bucket_order_does_not_reach_outputs(dev):
    """The segment sort places pairs in their buckets with LDS atomics, so the order inside a
    bucket varies from run to run; every output is a function of one pair (or, in
    retrieve_fuse, of one query's routes in route order), so repeated calls are bit-identical:
    gather_apply, retrieve_fuse and both transposed applies, with thousands of pairs per segment
    (7200 pairs: the one-workgroup sort; 72000: the chunked sort)."""
    g = torch.Generator().manual_seed(99)
    for B, Q, S, R in ((2, 900, 5, 8), (1, 9000, 7, 8)):
        H, K = 128, 64
        mem = (torch.randn(B, S, H, K, generator=g) * 0.3).to(torch.float16).to(dev)
        idx = torch.randint(0, S, (B, Q, R), generator=g).to(dev)
        q = norm(torch.randn(B, Q, K, generator=g)).to(torch.bfloat16).to(dev)
        gates = torch.softmax(torch.randn(B, Q, R, generator=g), -1).to(dev)
        h = torch.randn(B, Q, H, generator=g).to(dev)
        gx = torch.randn(B, Q, H, generator=g).to(dev)
        gp = torch.randn(B, Q, R, H, generator=g).to(dev)
        print(f"bucket order B={B} Q={Q} S={S} R={R}", flush=True)

        def run():
            return (capi.gather_apply(mem, idx, q, dtype=torch.float32),
                    capi.retrieve_fuse(mem, idx, q, gates, h),
                    capi.gather_apply_bwd_tokens(mem, idx, gx),
                    capi.gather_apply_bwd_queries(mem, idx, gp))

        first = [t.clone() for t in run()]
        for _ in range(3):
            again = run()
            torch.cuda.synchronize()
            for a, b in zip(first, again):
                assert torch.equal(a, b)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
def test_apply_degenerate_shapes_clear_outputs(dev, dtype):
    """key_dim 0 (apply_query forward) and no routes (apply_query backward) clear the output with
    the library's fill kernel, not a memset: buffers filled with 7 before the call read zero after
    it, in every dtype, with odd element counts."""
    import ctypes

    lib = capi.load()
    sp = ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)
    P = lambda t: ctypes.c_void_p(t.data_ptr())  # noqa: E731
    B, Q, R, H = 3, 5, 2, 7
    dummy = torch.zeros(8, dtype=dtype, device=dev)  # inputs of zero elements, never read
    mem, q = dummy, dummy
    out = torch.full((B, Q, R, H), 7.0, dtype=dtype, device=dev)
    rc = lib.grm_hip_apply_query_fwd(P(mem), P(q), P(out), B, Q, R, H, 0, capi.dtype_code(dtype), sp)
    assert rc == 0, capi.last_error()
    K = 9
    q = torch.randn(B, Q, K, device=dev).to(dtype)
    gq = torch.full((B, Q, K), 7.0, dtype=dtype, device=dev)
    rc = lib.grm_hip_apply_query_bwd(P(dummy), P(dummy), P(q), P(dummy), P(gq), B, Q, 0, H, K, capi.dtype_code(dtype),
                                     sp)
    assert rc == 0, capi.last_error()
    torch.cuda.synchronize()
    assert int(torch.count_nonzero(out)) == 0 and int(torch.count_nonzero(gq)) == 0


def _nonfinite_expect(q, keys, k, scale):
    """topk_route's rule for non-finite scores, from the oracle's canonical scores in index order:
    a NaN or -inf score is never selected, the rest by (score descending, index ascending); slots
    left over are (-1, -inf, 0); gates are the softmax of the filled slots."""
    S = keys.shape[1]
    _, _, all_sc = orc.topk_route(q, keys, S, scale)          # k == S: every score, index order
    B, Q = all_sc.shape[:2]
    idx = np.full((B, Q, k), -1, dtype=np.int64)
    sc = np.full((B, Q, k), -np.inf, dtype=np.float32)
    gt = np.zeros((B, Q, k))
    for b in range(B):
        for r in range(Q):
            s = all_sc[b, r]
            ok = np.flatnonzero(s > -np.inf)                   # False for NaN
            order = ok[np.argsort(-s[ok], kind="stable")][:k]
            idx[b, r, :len(order)] = order
            sc[b, r, :len(order)] = s[order]
            if len(order):
                e = np.exp(s[order].astype(np.float64) - s[order].max())
                gt[b, r, :len(order)] = e / e.sum()
    return gt, idx, sc


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("S,k", [(40, 3), (40, 8), (300, 150)])
def test_topk_route_non_finite(dev, dtype, S, k):
    """One rule for non-finite scores on every routing path (the select kernels at k <= 32 and
    k <= 128, the sort beyond 128): a NaN or -inf score is never selected, empty slots are
    (-1, -inf, 0), gates the softmax of the filled slots.  A query row of NaN (no slot filled),
    a key with a NaN (never selected by any row of its batch entry), and a key scoring -inf for
    every row."""
    g = torch.Generator().manual_seed(S + k)
    q = torch.randn(2, 30, 64, generator=g)
    q[..., 0] = q[..., 0].abs() + 0.1   # positive first component: key 9 below scores -inf
    q = norm(q)
    keys = norm(torch.randn(2, S, 64, generator=g))
    q[0, 3] = float("nan")
    keys[1, 5, 7] = float("nan")
    keys[0, 9, 0] = float("-inf")
    q, keys = q.to(dtype), keys.to(dtype)
    print(f"topk_route non-finite S={S} k={k} {dtype}", flush=True)
    gates, idx, sc = torch.ops.grm_cuda.topk_route(q.to(dev), keys.to(dev), k, 0.125, 1.0)
    og, oi, osc = _nonfinite_expect(q.float().numpy(), keys.float().numpy(), k, 0.125)
    assert np.array_equal(idx.cpu().numpy(), oi)
    assert np.array_equal(sc.cpu().numpy(), osc)
    np.testing.assert_allclose(gates.cpu().numpy(), og, rtol=1e-5, atol=1e-6)
    assert bool((idx[0, 3] == -1).all()) and not bool((idx[1] == 5).any()) and not bool((idx[0] == 9).any())
