"""The per-layer glue kernels (layer_glue.hip) against the torch ops they replace:
project_split (split of the concatenated projection, F.normalize of keys and queries;
reference grm/core/paper_grm.py:491-493,570-574) and residual_layer_norm
(layer_norm(x + residual), grm/core/multilayer_grm.py:92-97)."""

import pytest
import torch
import torch.nn.functional as F

from rnn_with_grm_amd import capi, cuda_ops

pytestmark = pytest.mark.gpu


def ulps_apart(a, b, dtype):
    """Largest distance between a and b in units in the last place of dtype at |b|."""
    a, b = a.double(), b.double()
    eps = {torch.bfloat16: 2.0 ** -7, torch.float16: 2.0 ** -10, torch.float32: 2.0 ** -23}[dtype]
    scale = torch.clamp(b.abs(), min=torch.finfo(dtype).tiny) * eps
    return float(((a - b).abs() / scale).max())


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("lead,dk,dv,de", [((4, 300), 64, 512, 512), ((7,), 8, 24, 0), ((2, 33), 128, 128, 16),
                                           ((1, 5), 32, 8, 8)])
def test_project_split(dev, dtype, lead, dk, dv, de):
    """Keys and queries within two units in the last place of F.normalize's (the kernel sums
    the squares in another order, so the norm can differ by one unit before the same
    roundings and the division), values and extra bit for bit; zero rows stay zero (the eps
    clamp)."""
    g = torch.Generator().manual_seed(dk + dv + de)
    proj = torch.randn(*lead, 2 * dk + dv + de, generator=g).to(dtype)
    proj.view(-1, proj.shape[-1])[0, :dk] = 0  # a zero key row
    pd = proj.to(dev)
    print(f"project_split lead={lead} dk={dk} dv={dv} de={de} {dtype}", flush=True)
    k, v, q, e = capi.project_split(pd, dk, dv, de, 1e-6)
    torch.cuda.synchronize()
    parts = pd.split([dk, dv, dk, de], dim=-1)
    rk = F.normalize(parts[0], p=2, dim=-1, eps=1e-6)
    rq = F.normalize(parts[2], p=2, dim=-1, eps=1e-6)
    assert k.is_contiguous() and v.is_contiguous() and q.is_contiguous()
    assert torch.equal(v, parts[1]) and (de == 0 or torch.equal(e, parts[3]))
    assert not k.view(-1, dk)[0].any()
    for name, got, ref in (("keys", k, rk), ("queries", q, rq)):
        assert ulps_apart(got, ref, dtype) <= 2.0, name
        if dtype != torch.float32:  # the 16-bit rounding of the norm hides most sum-order differences
            assert (got != ref).float().mean() < 0.02, name


@pytest.mark.parametrize("dtype,pdtype", [(torch.float32, torch.float32), (torch.bfloat16, torch.bfloat16),
                                          (torch.float16, torch.float16), (torch.bfloat16, torch.float32)])
@pytest.mark.parametrize("rows,H,affine", [(1000, 512, True), (37, 8, True), (5, 2048, False), (64, 200, True)])
def test_residual_layer_norm(dev, dtype, pdtype, rows, H, affine):
    """Against F.layer_norm(x + residual): the sum rounded to the row dtype as torch's add
    does, float32 statistics; 16-bit outputs within one unit in the last place (the
    statistics are summed in another order), float32 within 1e-5."""
    g = torch.Generator().manual_seed(rows + H)
    x = (torch.randn(rows, H, generator=g) * 2 + 0.5).to(dtype).to(dev)
    r = torch.randn(rows, H, generator=g).to(dtype).to(dev)
    w = (1 + 0.1 * torch.randn(H, generator=g)).to(pdtype).to(dev) if affine else None
    b = (0.1 * torch.randn(H, generator=g)).to(pdtype).to(dev) if affine else None
    print(f"residual_layer_norm rows={rows} H={H} {dtype} params {pdtype} affine={affine}", flush=True)
    out = capi.residual_layer_norm(x, r, w, b, 1e-5)
    torch.cuda.synchronize()
    s = (x + r)
    ref = F.layer_norm(s.float(), (H,), None if w is None else w.float(), None if b is None else b.float(), 1e-5)
    if dtype == torch.float32:
        torch.testing.assert_close(out, ref, rtol=1e-5, atol=1e-5)
    else:
        assert (out.double() - ref.double()).abs().max() <= 2 ** -7 * ref.abs().max().item() + 1e-3


def test_glue_ops_through_cuda_ops(dev):
    """cuda_ops' wrappers take the native ops without autograd (no generic path) and the
    torch compositions under autograd, with gradients."""
    ext = cuda_ops.extension_module()
    g = torch.Generator().manual_seed(2)
    proj = torch.randn(3, 50, 64 + 128 + 64 + 32, generator=g).to(torch.bfloat16).to(dev)
    x = torch.randn(3, 50, 256, generator=g).to(dev)
    r = torch.randn(3, 50, 256, generator=g).to(dev)
    ln = torch.nn.LayerNorm(256).to(dev)
    generic = ext.generic_path_calls()
    launches = capi.launch_count()
    with torch.no_grad():
        k, v, q, e = cuda_ops.cuda_project_split(proj, 64, 128, 32)
        y = cuda_ops.cuda_residual_layer_norm(x, r, ln.weight, ln.bias, ln.eps)
    assert ext.generic_path_calls() == generic and capi.launch_count() >= launches + 2
    assert e.shape == (3, 50, 32) and k.shape == (3, 50, 64)
    xr = x.clone().requires_grad_(True)
    y2 = cuda_ops.cuda_residual_layer_norm(xr, r, ln.weight, ln.bias, ln.eps)
    y2.sum().backward()
    assert xr.grad is not None and ln.weight.grad is not None
    torch.testing.assert_close(y, y2.detach(), rtol=1e-5, atol=1e-5)


@pytest.mark.parametrize("n", [8 * 4096 + 5, 1, 7, 64 * 512 * 64 * 3])
def test_archive_cast(dev, n):
    """archive_cast (grm_hip_archive_cast) against torch's two casts, bit for bit, for every
    (model dtype, storage dtype) pair: values that round differently through bfloat16 than
    straight to float16, float16 overflow and underflow, zeros of both signs, infinities and
    NaN; sizes with a ragged tail."""
    g = torch.Generator().manual_seed(n % 1000)
    x = torch.randn(n, generator=g) * torch.exp2(torch.randint(-30, 30, (n,), generator=g).float())
    special = torch.tensor([0.0, -0.0, float("inf"), -float("inf"), float("nan"), 65520.0, 1e-8, -3e-41,
                            1.0 + 2.0 ** -8 + 2.0 ** -12, 1.0 + 2.0 ** -9 + 2.0 ** -11])
    x[: min(n, special.numel())] = special[: min(n, special.numel())]
    print(f"archive_cast n={n}", flush=True)
    xd = x.to(dev)
    for md in (torch.float32, torch.bfloat16, torch.float16):
        for sd in (torch.float32, torch.bfloat16, torch.float16):
            want = x.to(md).to(sd)
            got = capi.archive_cast(xd, md, sd)
            op = torch.ops.grm_cuda.archive_cast(xd, md, sd)
            torch.cuda.synchronize()
            it = torch.int32 if sd == torch.float32 else torch.int16
            wnan = want.float().isnan()
            for out in (got.cpu(), op.cpu()):
                # the bits of every value, and NaN where NaN (payloads may differ)
                assert out.dtype == sd
                assert torch.equal(out.float().isnan(), wnan), (md, sd)
                assert torch.equal(out.view(it)[~wnan], want.view(it)[~wnan]), (md, sd)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("rows,K,dv,de,with_bias", [(32768, 512, 512, 512, False), (1000, 64, 64, 0, True),
                                                    (37, 128, 128, 64, True), (300, 192, 256, 128, False)])
def test_project_gemm(dev, dtype, rows, K, dv, de, with_bias):
    """project_gemm (the projection GEMM with project_split as its epilogue) against F.linear then
    F.normalize in the same dtype.  The GEMM sums in another order than the library, so an
    element may round to the neighbouring 16-bit value: values and extra within 2^-7 of each
    element plus 2^-14 of the tensor's largest magnitude (cancellation near zero), keys and
    queries within 2^-6 plus 2^-12; and at most 3% of the elements differ at all."""
    g = torch.Generator().manual_seed(rows + K)
    dk = 64
    N = 2 * dk + dv + de
    x = torch.randn(rows, K, generator=g).to(dtype)
    w = (torch.randn(N, K, generator=g) / K ** 0.5).to(dtype)
    b = (0.1 * torch.randn(N, generator=g)).to(dtype) if with_bias else None
    print(f"project_gemm rows={rows} K={K} dv={dv} de={de} bias={with_bias} {dtype}", flush=True)
    xd, wd, bd = x.to(dev), w.to(dev), (b.to(dev) if b is not None else None)
    ext = cuda_ops.extension_module()
    generic = ext.generic_path_calls()
    got = capi.project_gemm(xd, wd, bd, dk, dv, de)
    op = torch.ops.grm_cuda.project_gemm(xd, wd, bd, dk, dv, de, 1e-6)
    torch.cuda.synchronize()
    assert ext.generic_path_calls() == generic
    proj = F.linear(xd, wd, bd)
    parts = proj.split([dk, dv, dk, de], dim=-1)
    ref = (F.normalize(parts[0], p=2, dim=-1, eps=1e-6), parts[1], F.normalize(parts[2], p=2, dim=-1, eps=1e-6),
           parts[3])
    for name, a_, o_, r_, rel, ab in zip(("keys", "values", "queries", "extra"), got, op, ref,
                                         (2.0 ** -6, 2.0 ** -7, 2.0 ** -6, 2.0 ** -7),
                                         (2.0 ** -12, 2.0 ** -14, 2.0 ** -12, 2.0 ** -14)):
        assert torch.equal(a_, o_), name
        if r_.numel() == 0:
            continue
        a64, r64 = a_.double().cpu(), r_.double().cpu()
        scale = float(r64.abs().max())
        assert bool(((a64 - r64).abs() <= rel * r64.abs() + ab * scale).all()), name
        assert float((a64 != r64).double().mean()) <= 0.03, name


def test_project_gemm_shapes_outside_the_kernel(dev):
    """Shapes the fused kernel does not take (key_dim 32) run the library GEMM and the split's own
    kernel (no generic call), with the same results as F.linear then project_split."""
    g = torch.Generator().manual_seed(5)
    x = torch.randn(50, 64, generator=g).to(torch.bfloat16).to(dev)
    w = torch.randn(2 * 32 + 96, 64, generator=g).to(torch.bfloat16).to(dev)
    ext = cuda_ops.extension_module()
    generic = ext.generic_path_calls()
    k, v, q, e = torch.ops.grm_cuda.project_gemm(x, w, None, 32, 96, 0, 1e-6)
    assert ext.generic_path_calls() == generic
    k2, v2, q2, e2 = torch.ops.grm_cuda.project_split(F.linear(x, w), 32, 96, 0, 1e-6)
    assert torch.equal(k, k2) and torch.equal(v, v2) and torch.equal(q, q2)
