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


# ---------------------------------------------------------------- output projection + residual + LayerNorm
@pytest.mark.parametrize("dtype,pdtype", [(torch.bfloat16, torch.bfloat16), (torch.float16, torch.float16),
                                          (torch.bfloat16, torch.float32)])
@pytest.mark.parametrize("rows,K,N,with_bias,affine", [(32768, 512, 512, True, True), (1000, 64, 64, True, True),
                                                       (37, 128, 192, False, True), (130, 256, 512, True, False),
                                                       (65, 512, 448, False, False)])
def test_linear_residual_layer_norm(dev, dtype, pdtype, rows, K, N, with_bias, affine):
    """linear_residual_layer_norm (the output projection GEMM with the block's residual add and
    LayerNorm as its epilogue) against torch's F.linear, add and F.layer_norm in the same dtype:
    the LayerNorm input (pre) within one unit in the last place of torch's F.linear + residual and
    at most 3% of its elements different (the GEMM sums in another order); the output within one
    unit of F.layer_norm of that same input, float32 statistics within 1e-5 of
    native_layer_norm's; the whole output at relative L2 below 1e-2 of the float32 composition;
    save=False writes the same output.  (32768, 512, 512) is config 4's layer."""
    g = torch.Generator().manual_seed(rows + K + N)
    x = torch.randn(rows, K, generator=g).to(dtype).to(dev)
    w = (torch.randn(N, K, generator=g) / K ** 0.5).to(dtype).to(dev)
    b = (0.1 * torch.randn(N, generator=g)).to(dtype).to(dev) if with_bias else None
    r = torch.randn(rows, N, generator=g).to(dtype).to(dev)
    lw = (1 + 0.1 * torch.randn(N, generator=g)).to(pdtype).to(dev) if affine else None
    lb = (0.1 * torch.randn(N, generator=g)).to(pdtype).to(dev) if affine else None
    print(f"linear_residual_layer_norm rows={rows} K={K} N={N} bias={with_bias} affine={affine} {dtype}/{pdtype}",
          flush=True)
    ext = cuda_ops.extension_module()
    generic, launches = ext.generic_path_calls(), ext.hip_launch_count()
    out, pre, mean, rstd = capi.linear_residual_layer_norm(x, w, b, r, lw, lb, 1e-5, save=True)
    out2 = torch.ops.grm_cuda.linear_residual_layer_norm(x, w, b, r, lw, lb, 1e-5, False)[0]
    torch.cuda.synchronize()
    assert ext.generic_path_calls() == generic and ext.hip_launch_count() > launches
    assert torch.equal(out, out2)
    e = {torch.bfloat16: 2.0 ** -7, torch.float16: 2.0 ** -10}[dtype]  # one unit in the last place at 1
    y_ref = F.linear(x, w, b)
    s_ref = y_ref + r
    # y may round to the neighbouring value (another summation order): s moves by one step of y,
    # then rounds once more
    bound = e * (y_ref.double().abs() + s_ref.double().abs()) + 1e-6
    assert bool(((pre.double() - s_ref.double()).abs() <= bound).all())
    assert float((pre != s_ref).double().mean()) <= 0.03
    # the LayerNorm of that same input: float32 statistics, one rounding of the output
    ln32, m_ref, r_ref = torch.ops.aten.native_layer_norm(pre.float(), [N], None if lw is None else lw.float(),
                                                          None if lb is None else lb.float(), 1e-5)
    assert bool(((out.double() - ln32.double()).abs() <= e * ln32.double().abs() + 1e-4).all())
    torch.testing.assert_close(mean, m_ref.reshape(-1), rtol=1e-5, atol=1e-5)
    torch.testing.assert_close(rstd, r_ref.reshape(-1), rtol=1e-5, atol=1e-5)
    f32 = F.layer_norm(F.linear(x.float(), w.float(), None if b is None else b.float()) + r.float(), (N,),
                       None if lw is None else lw.float(), None if lb is None else lb.float(), 1e-5)
    rel = float((out.float() - f32).norm() / f32.norm())
    assert rel < 1e-2, rel


def test_linear_residual_layer_norm_outside_the_kernel(dev):
    """Shapes the kernel does not take (out_dim 576, float32) run the generic composition on the
    device and count a generic call; the C ABI refuses them with a message."""
    g = torch.Generator().manual_seed(9)
    x = torch.randn(10, 64, generator=g).to(torch.bfloat16).to(dev)
    w = torch.randn(576, 64, generator=g).to(torch.bfloat16).to(dev)
    r = torch.randn(10, 576, generator=g).to(torch.bfloat16).to(dev)
    ext = cuda_ops.extension_module()
    generic = ext.generic_path_calls()
    out = torch.ops.grm_cuda.linear_residual_layer_norm(x, w, None, r, None, None, 1e-5, False)[0]
    assert ext.generic_path_calls() == generic + 1
    torch.testing.assert_close(out, F.layer_norm(F.linear(x, w) + r, (576,)))
    with pytest.raises(RuntimeError, match="out_dim"):
        capi.linear_residual_layer_norm(x, w, None, r)


def _bf16_grad_close(name, got, ref):
    got, ref = got.double().cpu(), ref.double().cpu()
    rel = float((got - ref).norm() / ref.norm().clamp_min(1e-30))
    assert rel < 1e-2, (name, rel)
    scale = float(ref.abs().max())
    assert bool(((got - ref).abs() <= 3e-2 * ref.abs() + 1e-2 * scale).all()), name


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_linear_residual_layer_norm_training_form(dev, dtype):
    """cuda_linear_residual_layer_norm under autograd (_LinearResidualLayerNormFn: the fused
    forward, aten's LayerNorm backward on its saved input and statistics, the linear map's
    gradients on the library): output and every gradient against float32 autograd of
    F.linear + add + F.layer_norm on the same 16-bit inputs, relative L2 below 1e-2."""
    g = torch.Generator().manual_seed(23)
    rows, K, N = 4096, 512, 512
    vals = [torch.randn(rows, K, generator=g), torch.randn(N, K, generator=g) / K ** 0.5,
            0.1 * torch.randn(N, generator=g), torch.randn(rows, N, generator=g),
            1 + 0.1 * torch.randn(N, generator=g), 0.1 * torch.randn(N, generator=g)]
    dout = torch.randn(rows, N, generator=g).to(dtype).to(dev)
    a = [v.to(dtype).to(dev).requires_grad_(True) for v in vals]
    out = cuda_ops.cuda_linear_residual_layer_norm(*a, 1e-5)
    got = torch.autograd.grad(out, a, dout)
    f = [v.to(dtype).float().to(dev).requires_grad_(True) for v in vals]
    ref_out = F.layer_norm(F.linear(f[0], f[1], f[2]) + f[3], (N,), f[4], f[5], 1e-5)
    want = torch.autograd.grad(ref_out, f, dout.float())
    _bf16_grad_close("out", out.detach(), ref_out.detach())
    for name, x_, y_ in zip(("x", "weight", "bias", "residual", "ln_weight", "ln_bias"), got, want):
        assert x_.dtype == dtype
        _bf16_grad_close(name, x_, y_)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_project_gemm_training_form(dev, dtype):
    """cuda_project_gemm under autograd (_ProjectGemmFn: the fused forward, F.normalize's
    derivative in float32 from recomputed norms, the GEMM's gradients on the library) against
    float32 autograd of F.linear + split + F.normalize on the same 16-bit inputs, relative L2
    below 1e-2, with config 4's layer shape (key 64, value 512, gating query 512)."""
    g = torch.Generator().manual_seed(29)
    rows, K, dk, dv, de = 4096, 512, 64, 512, 512
    N = 2 * dk + dv + de
    vals = [torch.randn(rows, K, generator=g), torch.randn(N, K, generator=g) / K ** 0.5,
            0.1 * torch.randn(N, generator=g)]
    douts = [torch.randn(rows, d, generator=g).to(dtype).to(dev) for d in (dk, dv, dk, de)]
    a = [v.to(dtype).to(dev).requires_grad_(True) for v in vals]
    outs = cuda_ops.cuda_project_gemm(a[0], a[1], a[2], dk, dv, de, 1e-6)
    got = torch.autograd.grad(outs, a, douts)
    f = [v.to(dtype).float().to(dev).requires_grad_(True) for v in vals]
    p = F.linear(f[0], f[1], f[2]).split([dk, dv, dk, de], -1)
    ref = (F.normalize(p[0], dim=-1, eps=1e-6), p[1], F.normalize(p[2], dim=-1, eps=1e-6), p[3])
    want = torch.autograd.grad(ref, f, [d.float() for d in douts])
    for o, rr in zip(outs, ref):
        _bf16_grad_close("forward", o.detach(), rr.detach())
    for name, x_, y_ in zip(("x", "weight", "bias"), got, want):
        assert x_.dtype == dtype
        _bf16_grad_close(name, x_, y_)


def test_model_training_uses_fused_glue(dev, monkeypatch):
    """A bf16 two-layer hierarchical model's training step (forward, loss, backward) runs the
    fused projection and output forms under autograd, and its parameter gradients agree with the
    same step through the torch compositions of those two ops (everything else unchanged) to
    relative L2 2e-2 per parameter."""
    from rnn_with_grm_amd.segment_model import HierarchicalSegmentMemoryModel

    torch.manual_seed(31)
    model = HierarchicalSegmentMemoryModel(128, 128, 128, num_layers=2, segment_length=64, memory_capacity_segments=8,
                                           retrieval_top_k=4, memory_key_dim=64, dropout=0.0,
                                           recomputation_ratio=0.0).to(dev, torch.bfloat16)
    x = torch.randn(2, 512, 128, generator=torch.Generator().manual_seed(32)).to(dev, torch.bfloat16)
    tgt = torch.randn(2, 512, 128, generator=torch.Generator().manual_seed(33)).to(dev, torch.bfloat16)
    calls = {"proj": 0, "out": 0}
    pg, lr = cuda_ops._ProjectGemmFn.apply, cuda_ops._LinearResidualLayerNormFn.apply

    def count(key, fn):
        def wrapped(*args):
            calls[key] += 1
            return fn(*args)
        return wrapped

    def step():
        model.zero_grad(set_to_none=True)
        out, _, _, _ = model(x, reset_memory=True)
        (out.float() - tgt.float()).square().mean().backward()
        return {n: p.grad.detach().clone() for n, p in model.named_parameters() if p.grad is not None}

    monkeypatch.setattr(cuda_ops._ProjectGemmFn, "apply", count("proj", pg))
    monkeypatch.setattr(cuda_ops._LinearResidualLayerNormFn, "apply", count("out", lr))
    fused = step()
    assert calls["proj"] == 2 and calls["out"] == 2, calls
    monkeypatch.setattr(cuda_ops, "_project_gemm_fused", lambda *a: False)
    monkeypatch.setattr(cuda_ops, "_linear_res_ln_fused", lambda *a: False)
    plain = step()
    assert calls["proj"] == 2 and calls["out"] == 2, calls
    assert fused.keys() == plain.keys() and len(fused) > 10
    for n in fused:
        a_, b_ = fused[n].double(), plain[n].double()
        rel = float((a_ - b_).norm() / b_.norm().clamp_min(1e-30))
        assert rel < 2e-2, (n, rel)
