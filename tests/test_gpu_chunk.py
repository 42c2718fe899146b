"""GPU parity of the fused chunk-update + query kernel and its gradient.

Compares libgrm_hip.so (through the C ABI and through torch.ops.grm_cuda) with
the double-precision oracle on the same seeded inputs.  Tolerances: rtol 2e-2 /
atol 2e-3 for bf16/f16 inputs with fp32 accumulation, 1e-5 for fp32 (the
bounds the task's north star states), plus a relative-L2 bound.
"""

import numpy as np
import pytest
import torch

from oracle import oracle as orc
from rnn_with_grm_amd import capi, cuda_ops

pytestmark = pytest.mark.gpu

TOL = {torch.float32: (1e-5, 1e-5), torch.bfloat16: (2e-2, 2e-3), torch.float16: (2e-2, 2e-3)}
REL_L2 = {torch.float32: 1e-5, torch.bfloat16: 1e-2, torch.float16: 5e-3}


def make_case(B, T, K, H, dtype, mem_dtype, seed=0, m_std=0.02):
    g = torch.Generator().manual_seed(seed)
    q = torch.nn.functional.normalize(torch.randn(B, T, K, generator=g), dim=-1).to(dtype)
    k = torch.nn.functional.normalize(torch.randn(B, T, K, generator=g), dim=-1).to(dtype)
    v = torch.randn(B, T, H, generator=g).to(dtype)
    m = (torch.randn(B, H, K, generator=g) * m_std).to(mem_dtype)
    return k, v, q, m


def close(name, got, ref, dtype):
    rtol, atol = TOL[dtype]
    got = got.float().cpu().double().numpy()
    np.testing.assert_allclose(got, ref, rtol=rtol, atol=atol, err_msg=name)
    den = np.linalg.norm(ref)
    if den > 0:
        rel = np.linalg.norm(got - ref) / den
        assert rel < REL_L2[dtype], f"{name}: relative L2 error {rel:.3e}"


def oracle_fwd(k, v, q, m, decay, snap=0):
    return orc.chunk_update_seq(k.double().numpy(), v.double().numpy(), q.double().numpy(), m.double().numpy(),
                                decay, snap)


@pytest.mark.parametrize("dtype,mem_dtype", [
    (torch.bfloat16, torch.float32),
    (torch.float16, torch.float32),
    (torch.float32, torch.float32),
    (torch.bfloat16, torch.bfloat16),
    (torch.float16, torch.float16),
])
@pytest.mark.parametrize("B,T,K,H", [(2, 8, 8, 16), (3, 200, 64, 48), (2, 130, 128, 128), (1, 64, 256, 40),
                                     (2, 77, 33, 20)])
def test_chunk_forward_capi(dev, dtype, mem_dtype, B, T, K, H):
    if dtype == torch.float32 and K > 128:
        pytest.skip("float32 inputs take key_dim <= 128 (test_fp32_wide_keys covers the rejection)")
    k, v, q, m = make_case(B, T, K, H, dtype, mem_dtype, seed=B * 1000 + T)
    decay = 0.97
    hid, mo, _ = capi.chunk_update_fwd(k.to(dev), v.to(dev), q.to(dev), m.to(dev), decay)
    torch.cuda.synchronize()
    rh, rm, _ = oracle_fwd(k, v, q, m, decay)
    close("hidden", hid, rh, dtype)
    close("memory_out", mo, rm, mem_dtype if mem_dtype != torch.float32 else dtype)


def test_fp32_wide_keys(dev):
    """float32 with key_dim > 128 exceeds one CU's LDS: the C ABI refuses it and the
    torch op runs the generic ATen path on the GPU, as the reference does for d_k > 128."""
    k, v, q, m = make_case(1, 40, 192, 16, torch.float32, torch.float32, seed=1)
    with pytest.raises(RuntimeError, match="exceeds 128"):
        capi.chunk_update_fwd(k.to(dev), v.to(dev), q.to(dev), m.to(dev), 0.97)
    hid, mo, _ = torch.ops.grm_cuda.chunk_update_forward(k.to(dev), v.to(dev), q.to(dev), m.to(dev), 0.97)
    rh, rm, _ = oracle_fwd(k, v, q, m, 0.97)
    close("hidden", hid, rh, torch.float32)
    close("memory_out", mo, rm, torch.float32)


def test_reference_case_fp32(dev):
    """The reference's own parity shape (examples/test_grm.py:29-37,154-164:
    B=2, d_v=16, d_k=8, chunk 64, unit-normal memory) at fp32."""
    k, v, q, m = make_case(2, 64, 8, 16, torch.float32, torch.float32, seed=7, m_std=1.0)
    hid, mo, aux = torch.ops.grm_cuda.chunk_update_forward(k.to(dev), v.to(dev), q.to(dev), m.to(dev), 0.97)
    rh, rm, _ = oracle_fwd(k, v, q, m, 0.97)
    close("hidden", hid, rh, torch.float32)
    close("memory_out", mo, rm, torch.float32)
    assert aux.numel() == 0


@pytest.mark.parametrize("decay", [0.0, 0.5, 0.97, 1.0])
def test_decay_edges(dev, decay):
    k, v, q, m = make_case(2, 150, 64, 32, torch.float32, torch.float32, seed=3, m_std=0.5)
    hid, mo, _ = capi.chunk_update_fwd(k.to(dev), v.to(dev), q.to(dev), m.to(dev), decay)
    rh, rm, _ = oracle_fwd(k, v, q, m, decay)
    close("hidden", hid, rh, torch.float32)
    close("memory_out", mo, rm, torch.float32)


@pytest.mark.parametrize("seg", [64, 128, 32, 100, 1])
def test_segment_snapshots(dev, seg):
    T = 300 if seg != 1 else 40
    k, v, q, m = make_case(2, T, 128, 64, torch.bfloat16, torch.float32, seed=seg)
    hid, mo, snaps = cuda_ops.cuda_segment_scan(k.to(dev), v.to(dev), q.to(dev), m.to(dev), 0.97, seg)
    rh, rm, rs = oracle_fwd(k, v, q, m, 0.97, seg)
    assert snaps.shape == (2, (T + seg - 1) // seg, 64, 128) and snaps.dtype == torch.float32
    close("hidden", hid, rh, torch.bfloat16)
    close("memory_out", mo, rm, torch.bfloat16)
    close("snapshots", snaps, rs, torch.bfloat16)
    # the last snapshot is the final state, bit for bit
    assert torch.equal(snaps[:, -1], mo)


def test_config2_shape(dev):
    """BASELINE config 2 at full size (B*H=64, T=2048, d=128, C=64, bf16 in / fp32 state):
    4 sequences against the oracle, plus size-independent properties on all 64."""
    B, T, D = 64, 2048, 128
    g = torch.Generator().manual_seed(0)
    q = torch.nn.functional.normalize(torch.randn(B, T, D, generator=g), dim=-1).to(torch.bfloat16)
    k = torch.nn.functional.normalize(torch.randn(B, T, D, generator=g), dim=-1).to(torch.bfloat16)
    v = torch.randn(B, T, D, generator=g).to(torch.bfloat16)
    m = torch.randn(B, D, D, generator=g) * 0.02
    kd, vd, qd, md = k.to(dev), v.to(dev), q.to(dev), m.to(dev)
    hid, mo, snaps = capi.chunk_update_fwd(kd, vd, qd, md, 0.97, 64)
    hid2, mo2, _ = capi.chunk_update_fwd(kd, vd, qd, md, 0.97)
    torch.cuda.synchronize()
    assert torch.equal(hid, hid2) and torch.equal(mo, mo2), "snapshot output must not change the scan"
    assert torch.equal(snaps[:, -1], mo)
    assert torch.isfinite(hid.float()).all() and torch.isfinite(snaps).all()
    for b in (0, 17, 40, 63):
        rh, rm, rs = oracle_fwd(k[b:b + 1], v[b:b + 1], q[b:b + 1], m[b:b + 1], 0.97, 64)
        close(f"hidden[{b}]", hid[b:b + 1], rh, torch.bfloat16)
        close(f"snapshots[{b}]", snaps[b:b + 1], rs, torch.bfloat16)
    # run-to-run determinism (no atomics)
    hid3, _, snaps3 = capi.chunk_update_fwd(kd, vd, qd, md, 0.97, 64)
    assert torch.equal(hid, hid3) and torch.equal(snaps, snaps3)


@pytest.mark.parametrize("parts", [2, 3, 5, 9])
@pytest.mark.parametrize("seg", [0, 64, 100, 128])
def test_time_split(dev, monkeypatch, parts, seg):
    """Sequences split into time parts match the oracle and the single-chain scan
    (up to 4 parts each part combines the earlier contributions itself, beyond
    that a combine step writes the starting states); ragged last part and odd
    snapshot lengths included."""
    B, T, K, H = 3, 700, 128, 96
    k, v, q, m = make_case(B, T, K, H, torch.bfloat16, torch.float32, seed=parts * 7 + seg)
    kd, vd, qd, md = k.to(dev), v.to(dev), q.to(dev), m.to(dev)
    monkeypatch.setenv("GRM_HIP_CHUNK_PARTS", str(parts))
    assert capi.fwd_workspace_bytes(B, T, K, H, seg) > 0
    hid, mo, snaps = capi.chunk_update_fwd(kd, vd, qd, md, 0.97, seg)
    hid1, mo1, snaps1 = capi.chunk_update_fwd(kd, vd, qd, md, 0.97, seg, split=False)
    torch.cuda.synchronize()
    rh, rm, rs = oracle_fwd(k, v, q, m, 0.97, seg)
    close("hidden", hid, rh, torch.bfloat16)
    close("memory_out", mo, rm, torch.bfloat16)
    if seg:
        close("snapshots", snaps, rs, torch.bfloat16)
        assert torch.equal(snaps[:, -1], mo)
    # the split only reassociates fp32 sums of the state
    torch.testing.assert_close(hid.float(), hid1.float(), rtol=2e-2, atol=2e-3)
    torch.testing.assert_close(mo, mo1, rtol=1e-4, atol=1e-6)


@pytest.mark.parametrize("B,T,K,H", [(2, 300, 128, 256), (3, 129, 64, 200), (1, 640, 96, 136), (4, 64, 16, 8)])
def test_wide_and_narrow_tiles_agree(dev, monkeypatch, B, T, K, H):
    """16-bit inputs run on 128-wide value tiles by default (several tiles and a
    ragged last tile here); the 32-wide tiles (GRM_HIP_CHUNK_DV=32) compute the
    same map.  Both against the oracle, and against each other."""
    k, v, q, m = make_case(B, T, K, H, torch.bfloat16, torch.float32, seed=B * 31 + H)
    kd, vd, qd, md = k.to(dev), v.to(dev), q.to(dev), m.to(dev)
    hw, mw, sw = capi.chunk_update_fwd(kd, vd, qd, md, 0.97, 64)
    monkeypatch.setenv("GRM_HIP_CHUNK_DV", "32")
    hn, mn, sn = capi.chunk_update_fwd(kd, vd, qd, md, 0.97, 64)
    torch.cuda.synchronize()
    rh, rm, rs = oracle_fwd(k, v, q, m, 0.97, 64)
    for tag, (h, mo, s) in (("wide", (hw, mw, sw)), ("narrow", (hn, mn, sn))):
        close(f"{tag} hidden", h, rh, torch.bfloat16)
        close(f"{tag} memory_out", mo, rm, torch.bfloat16)
        close(f"{tag} snapshots", s, rs, torch.bfloat16)
    torch.testing.assert_close(hw.float(), hn.float(), rtol=1e-2, atol=1e-3)
    torch.testing.assert_close(mw, mn, rtol=1e-4, atol=1e-6)


@pytest.mark.parametrize("dtype,mem_dtype", [(torch.bfloat16, torch.float32), (torch.float16, torch.float32),
                                             (torch.bfloat16, torch.bfloat16), (torch.float16, torch.float16)])
@pytest.mark.parametrize("B,T,K,H,seg", [(2, 300, 128, 128, 64), (3, 129, 64, 64, 0), (1, 640, 96, 256, 100),
                                         (2, 64, 128, 32, 128), (5, 1000, 32, 96, 32), (1, 7, 128, 128, 1)])
def test_value_split_scan(dev, monkeypatch, dtype, mem_dtype, B, T, K, H, seg):
    """The value-split scan (32-column value tiles, one workgroup per sequence and
    tile, GRM_HIP_CHUNK_VSPLIT=1) against the oracle and against the 128-column
    kernel (=0): ragged last chunks, key widths below the padded 64/128, one to
    eight value tiles, snapshot lengths that set shorter chunks, 16-bit states."""
    k, v, q, m = make_case(B, T, K, H, dtype, mem_dtype, seed=B * 97 + T + K)
    kd, vd, qd, md = k.to(dev), v.to(dev), q.to(dev), m.to(dev)
    print(f"value split B={B} T={T} K={K} H={H} seg={seg} {dtype} state {mem_dtype}", flush=True)
    monkeypatch.setenv("GRM_HIP_CHUNK_VSPLIT", "1")
    hs, ms, ss = capi.chunk_update_fwd(kd, vd, qd, md, 0.97, seg)
    monkeypatch.setenv("GRM_HIP_CHUNK_VSPLIT", "0")
    hw, mw, sw = capi.chunk_update_fwd(kd, vd, qd, md, 0.97, seg)
    torch.cuda.synchronize()
    rh, rm, rs = oracle_fwd(k, v, q, m, 0.97, seg)
    close("hidden", hs, rh, dtype)
    close("memory_out", ms, rm, dtype)
    if seg:
        close("snapshots", ss, rs, dtype)
        if mem_dtype == torch.float32:
            assert torch.equal(ss[:, -1], ms)
    torch.testing.assert_close(hs.float(), hw.float(), rtol=1e-2, atol=1e-3)
    torch.testing.assert_close(ms.float(), mw.float(), rtol=1e-2 if mem_dtype != torch.float32 else 1e-4,
                               atol=1e-3 if mem_dtype != torch.float32 else 1e-6)


@pytest.mark.parametrize("B,T,K,H,seg", [(2, 300, 128, 128, 64), (3, 129, 64, 64, 64), (1, 640, 96, 256, 100),
                                         (2, 200, 32, 96, 32), (4, 1000, 128, 128, 128)])
def test_full_line_snapshots(dev, monkeypatch, B, T, K, H, seg):
    """The value-split scan's full-line snapshot stores (a lane permutation that gives each
    store whole 128-byte lines, chosen from 320 MB of snapshots, forced here with
    GRM_HIP_SNAP_FULL_LINES=1) write the same bytes as the per-tile stores (=0): key widths
    below the padded 64 (partial last lines), ragged chunks, fp32 and bf16 states.  At key
    widths 65-128 the kernel stores snapshots from its fp32 state copy whatever the flag,
    so both calls take that path and are checked against the oracle."""
    for mem_dtype in (torch.float32, torch.bfloat16):
        k, v, q, m = make_case(B, T, K, H, torch.bfloat16, mem_dtype, seed=B * 31 + T + K)
        kd, vd, qd, md = k.to(dev), v.to(dev), q.to(dev), m.to(dev)
        print(f"full-line snapshots B={B} T={T} K={K} H={H} seg={seg} state {mem_dtype}", flush=True)
        monkeypatch.setenv("GRM_HIP_CHUNK_VSPLIT", "1")
        monkeypatch.setenv("GRM_HIP_SNAP_FULL_LINES", "1")
        h1, m1, s1 = capi.chunk_update_fwd(kd, vd, qd, md, 0.97, seg)
        monkeypatch.setenv("GRM_HIP_SNAP_FULL_LINES", "0")
        h0, m0, s0 = capi.chunk_update_fwd(kd, vd, qd, md, 0.97, seg)
        torch.cuda.synchronize()
        assert torch.equal(s1, s0) and torch.equal(h1, h0) and torch.equal(m1, m0)
        if mem_dtype == torch.float32:
            rh, rm, rs = oracle_fwd(k, v, q, m, 0.97, seg)
            close("snapshots", s1, rs, torch.bfloat16)


@pytest.mark.parametrize("vsplit", ["1", "0"])
def test_optional_outputs(dev, monkeypatch, vsplit):
    """hidden may be NULL, and memory_out may be NULL when snapshots are requested; the outputs
    that are written equal those of the full call, on both 16-bit scan kernels."""
    B, T, K, H, seg = 2, 300, 128, 128, 64
    k, v, q, m = make_case(B, T, K, H, torch.bfloat16, torch.float32, seed=29)
    kd, vd, qd, md = k.to(dev), v.to(dev), q.to(dev), m.to(dev)
    monkeypatch.setenv("GRM_HIP_CHUNK_VSPLIT", vsplit)
    h, mo, s = capi.chunk_update_fwd(kd, vd, qd, md, 0.97, seg)
    h1, mo1, s1 = capi.chunk_update_fwd(kd, vd, qd, md, 0.97, seg, want_hidden=False)
    h2, mo2, s2 = capi.chunk_update_fwd(kd, vd, qd, md, 0.97, seg, want_memory_out=False)
    torch.cuda.synchronize()
    assert h1 is None and mo2 is None
    assert torch.equal(mo1, mo) and torch.equal(s1, s)
    assert torch.equal(h2, h) and torch.equal(s2, s)
    with pytest.raises(RuntimeError):
        capi.chunk_update_fwd(kd, vd, qd, md, 0.97, 0, want_memory_out=False)


def test_value_split_is_default_at_config2_shape(dev, monkeypatch):
    """Config 2's shape (64 sequences x 128 value columns) takes the value-split scan
    by default; it and the time-split 128-column scan agree, and it is deterministic."""
    B, T, D = 64, 512, 128
    k, v, q, m = make_case(B, T, D, D, torch.bfloat16, torch.float32, seed=11)
    kd, vd, qd, md = k.to(dev), v.to(dev), q.to(dev), m.to(dev)
    h0, m0, s0 = capi.chunk_update_fwd(kd, vd, qd, md, 0.97, 64)
    monkeypatch.setenv("GRM_HIP_CHUNK_VSPLIT", "1")
    h1, m1, s1 = capi.chunk_update_fwd(kd, vd, qd, md, 0.97, 64)
    monkeypatch.setenv("GRM_HIP_CHUNK_VSPLIT", "0")
    h2, m2, s2 = capi.chunk_update_fwd(kd, vd, qd, md, 0.97, 64)
    torch.cuda.synchronize()
    assert torch.equal(h0, h1) and torch.equal(s0, s1), "default path must be the value split here"
    torch.testing.assert_close(h1.float(), h2.float(), rtol=1e-2, atol=1e-3)
    torch.testing.assert_close(s1, s2, rtol=1e-4, atol=1e-6)
    for b in (0, 63):
        rh, rm, rs = oracle_fwd(k[b:b + 1], v[b:b + 1], q[b:b + 1], m[b:b + 1], 0.97, 64)
        close(f"hidden[{b}]", h1[b:b + 1], rh, torch.bfloat16)
        close(f"snapshots[{b}]", s1[b:b + 1], rs, torch.bfloat16)


def test_long_context_split_fp32(dev, monkeypatch):
    """fp32 long sequence, automatic part count, against the oracle at fp32 tolerance."""
    B, T, K, H = 2, 4096, 64, 64
    k, v, q, m = make_case(B, T, K, H, torch.float32, torch.float32, seed=5)
    assert capi.fwd_workspace_bytes(B, T, K, H, 0) > 0
    hid, mo, _ = capi.chunk_update_fwd(k.to(dev), v.to(dev), q.to(dev), m.to(dev), 0.97)
    rh, rm, _ = oracle_fwd(k, v, q, m, 0.97)
    close("hidden", hid, rh, torch.float32)
    close("memory_out", mo, rm, torch.float32)


def test_empty_and_zero_batch(dev):
    k, v, q, m = make_case(2, 0, 16, 8, torch.float32, torch.float32)
    hid, mo, aux = torch.ops.grm_cuda.chunk_update_forward(k.to(dev), v.to(dev), q.to(dev), m.to(dev), 0.9)
    assert hid.shape == (2, 0, 8) and torch.equal(mo.cpu(), m)
    k, v, q, m = make_case(0, 5, 16, 8, torch.float32, torch.float32)
    hid, mo, _ = torch.ops.grm_cuda.chunk_update_forward(k.to(dev), v.to(dev), q.to(dev), m.to(dev), 0.9)
    assert hid.shape == (0, 5, 8)


def test_native_path_runs(dev):
    ext = cuda_ops.extension_module()
    before = ext.hip_launch_count()
    k, v, q, m = make_case(2, 64, 32, 16, torch.bfloat16, torch.float32)
    cuda_ops.cuda_chunk_update(k.to(dev), v.to(dev), q.to(dev), m.to(dev), 0.97)
    assert ext.hip_launch_count() > before
    status = cuda_ops.get_grm_cuda_runtime_status()
    assert status["extension_loaded"] and status["compiled_with_cuda_kernels"] and status["cuda_backend_available"]


@pytest.mark.parametrize("dtype,mem_dtype", [(torch.float32, torch.float32), (torch.bfloat16, torch.float32),
                                             (torch.bfloat16, torch.bfloat16)])
@pytest.mark.parametrize("B,T,K,H", [(2, 8, 8, 16), (2, 150, 64, 40), (1, 70, 128, 128)])
def test_chunk_backward(dev, dtype, mem_dtype, B, T, K, H):
    k, v, q, m = make_case(B, T, K, H, dtype, mem_dtype, seed=11)
    g = torch.Generator().manual_seed(5)
    dh = torch.randn(B, T, H, generator=g).to(dtype)
    dm = torch.randn(B, H, K, generator=g).to(mem_dtype)
    gk, gv, gq, gm = capi.chunk_update_bwd(dh.to(dev), dm.to(dev), k.to(dev), v.to(dev), q.to(dev), m.to(dev), 0.97)
    torch.cuda.synchronize()
    rk, rv, rq, rm = orc.chunk_update_bwd(dh.double().numpy(), dm.double().numpy(), k.double().numpy(),
                                          v.double().numpy(), q.double().numpy(), m.double().numpy(), 0.97)
    tol_dtype = torch.float32 if dtype == torch.float32 else torch.bfloat16
    for name, got, ref in (("grad_keys", gk, rk), ("grad_values", gv, rv), ("grad_queries", gq, rq),
                           ("grad_memory", gm, rm)):
        if tol_dtype == torch.float32:
            # the north star's float32 bar, element by element (the reference's own CUDA test holds 5e-4)
            got64 = got.double().cpu().numpy()
            worst = float(np.max(np.abs(got64 - ref) / (1e-5 + 1e-5 * np.abs(ref))))
            print(f"{name}: float32 error / (1e-5 + 1e-5 |ref|) at most {worst:.3f}", flush=True)
            np.testing.assert_allclose(got64, ref, rtol=1e-5, atol=1e-5, err_msg=name)
        else:
            close(name, got, ref, torch.bfloat16)


def close_elementwise(name, got, ref, rtol=2e-2, atol=2e-3):
    """|got - ref| <= atol + rtol |ref| for every element (the bar of the 16-bit paths)."""
    got = got.float().cpu().double().numpy() if torch.is_tensor(got) else got
    np.testing.assert_allclose(got, ref, rtol=rtol, atol=atol, err_msg=name)


@pytest.mark.parametrize("dtype,mem_dtype", [(torch.bfloat16, torch.float32), (torch.float16, torch.float32),
                                             (torch.bfloat16, torch.bfloat16), (torch.float16, torch.float16)])
@pytest.mark.parametrize("B,T,K,H", [(2, 300, 128, 128), (3, 129, 64, 64), (1, 640, 96, 96), (2, 64, 128, 32),
                                     (1, 7, 128, 32), (1, 12, 128, 32), (2, 200, 32, 64), (1, 200, 64, 512),
                                     (1, 2000, 64, 512), (2, 1000, 64, 96)])
def test_mfma_backward(dev, monkeypatch, dtype, mem_dtype, B, T, K, H):
    """The chunk-parallel MFMA backward (16-bit inputs, value_dim a multiple of 32: the adjoint
    pass, then the per-chunk gradients over every value tile) against the double-precision
    oracle and against the scalar per-token kernel (GRM_HIP_BWD_MFMA=0), element by element at
    rtol 2e-2 / atol 2e-3: ragged last chunks, key widths below the padded 64/128, one to
    sixteen value tiles, a half-filled 64-row adjoint tile (96 values), one chunk (12 tokens),
    7 tokens, where the adjoint buffer would not fit the workspace and the scalar kernel runs,
    and adjoint walks split into 2, 4 and 8 parts (640, 1000 and 2000 tokens)."""
    k, v, q, m = make_case(B, T, K, H, dtype, mem_dtype, seed=B * 13 + T)
    g = torch.Generator().manual_seed(7)
    dh = torch.randn(B, T, H, generator=g).to(dtype)
    dm = torch.randn(B, H, K, generator=g).to(mem_dtype)
    args = [t.to(dev) for t in (dh, dm, k, v, q, m)]
    print(f"mfma backward B={B} T={T} K={K} H={H} {dtype} state {mem_dtype}", flush=True)
    got = capi.chunk_update_bwd(*args, 0.97)
    monkeypatch.setenv("GRM_HIP_BWD_MFMA", "0")
    scalar = capi.chunk_update_bwd(*args, 0.97)
    torch.cuda.synchronize()
    ref = orc.chunk_update_bwd(dh.double().numpy(), dm.double().numpy(), k.double().numpy(), v.double().numpy(),
                               q.double().numpy(), m.double().numpy(), 0.97)
    for name, x, y, r in zip(("grad_keys", "grad_values", "grad_queries", "grad_memory"), got, scalar, ref):
        assert torch.isfinite(x.float()).all(), name
        close_elementwise(name, x, r)
        close_elementwise(name + " vs scalar kernel", x, y.float().cpu().double().numpy())


@pytest.mark.parametrize("B,T,K,H,mem_dtype", [(1, 2000, 64, 512, torch.float32), (2, 1000, 64, 96, torch.bfloat16),
                                               (4, 8192, 64, 512, torch.float32)])
def test_mfma_backward_parts(dev, monkeypatch, B, T, K, H, mem_dtype):
    """The adjoint walk split into parts (run in parallel, then joined) against the unsplit
    walk (GRM_HIP_BWD_PARTS=0): only the rounding order of the fp32 adjoint differs, so a
    float32 grad_memory agrees to 1e-5 of its largest magnitude and every 16-bit gradient to
    one rounding step of its own (2^-7 of the element, plus 1e-6 of the largest magnitude).
    (4, 8192, 64, 512) is config 4's layer shape, eight parts of 16 chunks."""
    k, v, q, m = make_case(B, T, K, H, torch.bfloat16, mem_dtype, seed=T + H)
    g = torch.Generator().manual_seed(8)
    dh = torch.randn(B, T, H, generator=g).to(torch.bfloat16)
    dm = torch.randn(B, H, K, generator=g).to(mem_dtype)
    args = [t.to(dev) for t in (dh, dm, k, v, q, m)]
    print(f"mfma backward parts B={B} T={T} K={K} H={H} state {mem_dtype}", flush=True)
    got = capi.chunk_update_bwd(*args, 0.97)
    monkeypatch.setenv("GRM_HIP_BWD_PARTS", "0")
    one = capi.chunk_update_bwd(*args, 0.97)
    torch.cuda.synchronize()
    for name, x, y in zip(("grad_keys", "grad_values", "grad_queries", "grad_memory"), got, one):
        sixteen = x.dtype != torch.float32
        x, y = x.float().cpu(), y.float().cpu()
        scale = max(float(y.abs().max()), 1e-30)
        if sixteen:
            assert bool(((x - y).abs() <= 2.0 ** -7 * y.abs() + 1e-6 * scale).all()), name
        else:
            assert float((x - y).abs().max()) <= 1e-5 * scale, name


def test_autograd_through_cuda_ops(dev):
    """cuda_chunk_update under autograd matches the fallback's autograd (the
    reference's check, examples/test_grm.py:72-113)."""
    k, v, q, m = make_case(2, 64, 8, 16, torch.float32, torch.float32, seed=2, m_std=1.0)

    def run(debug):
        ins = [t.to(dev).clone().requires_grad_(True) for t in (k, v, q, m)]
        h, mo = cuda_ops.cuda_chunk_update(*ins, memory_decay=0.97, debug_fallback=debug)
        (h.square().mean() + mo.square().mean()).backward()
        return [t.grad for t in ins]

    for a, b in zip(run(False), run(True)):
        torch.testing.assert_close(a, b, atol=5e-4, rtol=5e-4)


def test_autograd_fp32_against_oracle(dev):
    """cuda_chunk_update under autograd in float32: the gradients autograd returns for given
    output gradients equal the double-precision oracle's backward at 1e-5 (rtol and atol), on the
    reference test's shape (B=2, d_v=16, d_k=8, examples/test_grm.py:29-37) with a 64-token chunk
    and on a config-1 sized case (8 x 512, d=64)."""
    for B, T, K, H, m_std in ((2, 64, 8, 16, 1.0), (8, 512, 64, 64, 0.0)):
        k, v, q, m = make_case(B, T, K, H, torch.float32, torch.float32, seed=T + K, m_std=m_std)
        g = torch.Generator().manual_seed(3)
        dh = torch.randn(B, T, H, generator=g)
        dm = torch.randn(B, H, K, generator=g)
        ins = [t.to(dev).requires_grad_(True) for t in (k, v, q, m)]
        h, mo = cuda_ops.cuda_chunk_update(*ins, memory_decay=0.97)
        grads = torch.autograd.grad((h, mo), ins, (dh.to(dev), dm.to(dev)))
        torch.cuda.synchronize()
        ref = orc.chunk_update_bwd(dh.double().numpy(), dm.double().numpy(), k.double().numpy(), v.double().numpy(),
                                   q.double().numpy(), m.double().numpy(), 0.97)
        for name, got, r in zip(("grad_keys", "grad_values", "grad_queries", "grad_memory"), grads, ref):
            got64 = got.double().cpu().numpy()
            worst = float(np.max(np.abs(got64 - r) / (1e-5 + 1e-5 * np.abs(r))))
            print(f"autograd B={B} T={T} {name}: error / (1e-5 + 1e-5 |ref|) at most {worst:.3f}", flush=True)
            np.testing.assert_allclose(got64, r, rtol=1e-5, atol=1e-5, err_msg=f"{name} B={B} T={T}")


@pytest.mark.parametrize("dtype,mem_dtype,T", [(torch.bfloat16, torch.float32, 300), (torch.float32, torch.float32, 70),
                                               (torch.bfloat16, torch.bfloat16, 64)])
def test_autograd_passes_chunk_states(dev, dtype, mem_dtype, T):
    """Under autograd the forward keeps the state after every 64-token chunk as aux and the
    backward reads it instead of scanning again: the gradients are bit-identical to the
    backward that scans again, and the backward launches fewer kernels."""
    k, v, q, m = make_case(2, T, 64, 96, dtype, mem_dtype, seed=T)
    ins = [t.to(dev).requires_grad_(True) for t in (k, v, q, m)]
    h, mo = cuda_ops.cuda_chunk_update(*ins, memory_decay=0.97)
    g = torch.Generator().manual_seed(1)
    dh = torch.randn(h.shape, generator=g).to(dtype).to(dev)
    dm = torch.randn(mo.shape, generator=g).to(mem_dtype).to(dev)
    before = capi.launch_count()
    gk, gv, gq, gm = torch.autograd.grad((h, mo), ins, (dh, dm))
    torch.cuda.synchronize()
    with_states = capi.launch_count() - before
    before = capi.launch_count()
    rk, rv, rq, rm = capi.chunk_update_bwd(dh, dm, *[t.detach() for t in ins], 0.97)
    torch.cuda.synchronize()
    rescan = capi.launch_count() - before
    assert with_states < rescan
    for a, b in zip((gk, gv, gq, gm), (rk, rv, rq, rm)):
        assert torch.equal(a, b)
    # and the forward under autograd is the plain forward's
    h0, mo0, _ = capi.chunk_update_fwd(*[t.detach() for t in ins], 0.97)
    assert torch.equal(h.detach(), h0) and torch.equal(mo.detach(), mo0)
