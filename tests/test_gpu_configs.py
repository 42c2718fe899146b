"""GPU parity at the full sizes of the benchmark configurations.

Each test runs the HIP path on the whole workload of one configuration and checks
it three ways:
  - against the double-precision / canonical-fp32 oracle on sampled sequences,
    tokens or heads (the oracle finishes each in seconds);
  - through size-independent properties over the whole output (the last snapshot is
    the final state, run-to-run bit equality, agreement of the time-split and
    single-chain scans, linearity checksums of the retrieval);
  - for the model, the 16-bit forward against the same weights in float32.

Shapes (folded B = batch x heads):
  north star  B=64, T=8192, d_k=d_v=128, chunk 64, bf16 inputs / fp32 state
  config 5    B=16, T=65536, d=128, snapshots every 128 tokens (512 per sequence),
              top-16 of 512 routing per token, gather + apply, residual + LayerNorm
  config 4    B=4, T=8192, d_k=64, d_v=512 (one memory per layer), segments of 64,
              capacity 64, top-8 routing over 512-wide summaries, float16 archive,
              and the 4-layer bf16 model forward
Tolerances: rtol 2e-2 / atol 2e-3 plus relative L2 1e-2 for bf16 inputs with fp32
accumulation, 1e-5 for float32 arithmetic, indices and routing scores bit-exact.
"""

import numpy as np
import pytest
import torch

from oracle import oracle as orc
from rnn_with_grm_amd import capi

pytestmark = pytest.mark.gpu

BF16_TOL = (2e-2, 2e-3)
BF16_REL_L2 = 1e-2


def nrm(x):
    return torch.nn.functional.normalize(x, dim=-1)


def close16(name, got, ref):
    got = got.float().cpu().double().numpy()
    np.testing.assert_allclose(got, ref, rtol=BF16_TOL[0], atol=BF16_TOL[1], err_msg=name)
    den = np.linalg.norm(ref)
    if den > 0:
        rel = np.linalg.norm(got - ref) / den
        assert rel < BF16_REL_L2, f"{name}: relative L2 error {rel:.3e}"


def scan_inputs(B, T, K, H, mem_dtype, seed):
    g = torch.Generator().manual_seed(seed)
    q = nrm(torch.randn(B, T, K, generator=g)).to(torch.bfloat16)
    k = nrm(torch.randn(B, T, K, generator=g)).to(torch.bfloat16)
    v = torch.randn(B, T, H, generator=g).to(torch.bfloat16)
    m = (torch.randn(B, H, K, generator=g) * 0.02).to(mem_dtype)
    return k, v, q, m


def oracle_rows(k, v, q, m, rows, seg):
    for b in rows:
        sl = slice(b, b + 1)
        yield b, orc.chunk_update_seq(k[sl].double().numpy(), v[sl].double().numpy(), q[sl].double().numpy(),
                                      m[sl].double().numpy(), 0.97, seg)


# ---------------------------------------------------------------- north star
def test_north_star_scan(dev, monkeypatch):
    """B*H=64, T=8192, d=128, chunk 64: three sequences against the oracle; on all 64, the
    snapshot-free call gives the same hidden rows, the last snapshot is the final state,
    a second call is bit-identical, and the time-split 128-column scan agrees."""
    B, T, D, SEG = 64, 8192, 128, 64
    k, v, q, m = scan_inputs(B, T, D, D, torch.float32, seed=8192)
    kd, vd, qd, md = k.to(dev), v.to(dev), q.to(dev), m.to(dev)
    print(f"north star scan B={B} T={T} D={D}", flush=True)
    hid, mo, snaps = capi.chunk_update_fwd(kd, vd, qd, md, 0.97, SEG)
    hid2, mo2, _ = capi.chunk_update_fwd(kd, vd, qd, md, 0.97)
    hid3, mo3, snaps3 = capi.chunk_update_fwd(kd, vd, qd, md, 0.97, SEG)
    monkeypatch.setenv("GRM_HIP_CHUNK_VSPLIT", "0")
    hw, mw, sw = capi.chunk_update_fwd(kd, vd, qd, md, 0.97, SEG)
    torch.cuda.synchronize()
    assert snaps.shape == (B, T // SEG, D, D)
    assert torch.equal(hid, hid2) and torch.equal(mo, mo2), "snapshot output must not change the scan"
    assert torch.equal(hid, hid3) and torch.equal(snaps, snaps3), "run-to-run results differ"
    assert torch.equal(snaps[:, -1], mo)
    torch.testing.assert_close(hw.float(), hid.float(), rtol=1e-2, atol=1e-3)
    torch.testing.assert_close(sw, snaps, rtol=1e-4, atol=1e-6)
    for b, (rh, rm, rs) in oracle_rows(k, v, q, m, (0, 31, 63), SEG):
        close16(f"hidden[{b}]", hid[b:b + 1], rh)
        close16(f"snapshots[{b}]", snaps[b:b + 1], rs)
        close16(f"memory_out[{b}]", mo[b:b + 1], rm)


# ---------------------------------------------------------------- config 5
@pytest.fixture(scope="module")
def c5(dev):
    """Config 5 inputs and the whole-sequence scan (one call, 512 snapshots per sequence)."""
    BH, T, D, SEG = 16, 65536, 128, 128
    k, v, q, m = scan_inputs(BH, T, D, D, torch.float32, seed=5)
    g = torch.Generator().manual_seed(55)
    summaries = nrm(torch.randn(BH, T // SEG, D, generator=g)).to(torch.bfloat16)
    kd, vd, qd, md = k.to(dev), v.to(dev), q.to(dev), m.to(dev)
    print(f"config 5 scan BH={BH} T={T} D={D} seg={SEG}", flush=True)
    hid, mo, snaps = capi.chunk_update_fwd(kd, vd, qd, md, 0.97, SEG)
    torch.cuda.synchronize()
    return dict(BH=BH, T=T, D=D, SEG=SEG, k=k, v=v, q=q, m=m, kd=kd, vd=vd, qd=qd, md=md, hid=hid, mo=mo,
                snaps=snaps, summaries=summaries, sd=summaries.to(dev))


def test_c5_scan(c5):
    """Two sequences against the oracle over all 65536 tokens and 512 snapshots; on all 16,
    the last snapshot is the final state, a second call is bit-identical, and the
    single-chain scan (no time split) agrees with the time-split one."""
    hid, mo, snaps = c5["hid"], c5["mo"], c5["snaps"]
    assert snaps.shape == (16, 512, 128, 128)
    assert torch.equal(snaps[:, -1], mo)
    h2, m2, s2 = capi.chunk_update_fwd(c5["kd"], c5["vd"], c5["qd"], c5["md"], 0.97, c5["SEG"])
    h1, m1, s1 = capi.chunk_update_fwd(c5["kd"], c5["vd"], c5["qd"], c5["md"], 0.97, c5["SEG"], split=False)
    torch.cuda.synchronize()
    assert torch.equal(h2, hid) and torch.equal(s2, snaps), "run-to-run results differ"
    torch.testing.assert_close(h1.float(), hid.float(), rtol=1e-2, atol=1e-3)
    torch.testing.assert_close(s1, snaps, rtol=1e-4, atol=1e-6)
    del h1, m1, s1, h2, m2, s2
    for b, (rh, rm, rs) in oracle_rows(c5["k"], c5["v"], c5["q"], c5["m"], (0, 11), c5["SEG"]):
        print(f"config 5 oracle sequence {b}", flush=True)
        close16(f"hidden[{b}]", hid[b:b + 1], rh)
        close16(f"snapshots[{b}]", snaps[b:b + 1], rs)


def test_c5_route(c5):
    """Top-16 of 512 for all 16 x 65536 tokens; a 2048-token slice of four heads bit-exact
    against the oracle (indices and scores), gates within 1e-5."""
    D = c5["D"]
    scale = 1.0 / D ** 0.5
    gates, idx, sc = capi.topk_route(c5["qd"], c5["sd"], 16, scale)
    torch.cuda.synchronize()
    heads, t0 = [0, 5, 9, 15], 30000
    qs = c5["q"][heads, t0:t0 + 2048].float().numpy()
    og, oi, osc = orc.topk_route(qs, c5["summaries"][heads].float().numpy(), 16, scale)
    assert np.array_equal(idx[heads, t0:t0 + 2048].cpu().numpy(), oi)
    assert np.array_equal(sc[heads, t0:t0 + 2048].cpu().numpy(), osc)
    np.testing.assert_allclose(gates[heads, t0:t0 + 2048].cpu().numpy(), og, rtol=1e-5, atol=1e-6)


@pytest.mark.parametrize("t0,n", [(0, 1024), (12800, 1024), (64512, 1024)])
def test_c5_causal_route(c5, t0, n):
    """Causal windows (segment s over snapshots 0..s-1) for all 16 x 65536 tokens in one
    launch; token slices at the start (windows shorter than k: index order and empty
    slots), the middle and the end (511 keys) bit-exact against the oracle's per-window
    routing."""
    D, SEG, S = c5["D"], c5["SEG"], c5["T"] // c5["SEG"]
    scale = 1.0 / D ** 0.5
    gates, idx, sc = capi.segment_route(c5["qd"], c5["sd"], 16, SEG, 0, S, scale)
    torch.cuda.synchronize()
    heads = [2, 7]
    og, oi, osc = orc.segment_route(c5["q"][heads, t0:t0 + n].float().numpy(), c5["summaries"][heads].float().numpy(),
                                    16, SEG, t0 // SEG, S, scale)
    assert np.array_equal(idx[heads, t0:t0 + n].cpu().numpy(), oi)
    assert np.array_equal(sc[heads, t0:t0 + n].cpu().numpy(), osc)
    np.testing.assert_allclose(gates[heads, t0:t0 + n].cpu().numpy(), og, rtol=1e-5, atol=1e-6)


def test_c5_retrieval(c5):
    """gather_apply over the 512 float32 snapshots per head (k=16 per token, bf16 queries,
    float32 out: [16, 65536, 16, 128], 8.6 GB) and the residual + LayerNorm fusion.
    Sampled tokens of two heads against the oracle's gather and apply and its fusion;
    over every token, a linearity checksum: the sum of each output row equals the
    selected state's column sums applied to the query."""
    BH, T, D = c5["BH"], c5["T"], c5["D"]
    snaps, qd = c5["snaps"], c5["qd"]
    gates, idx, _ = capi.topk_route(qd, c5["sd"], 16, 1.0 / D ** 0.5)
    out = capi.gather_apply(snaps, idx, qd, dtype=torch.float32)
    torch.cuda.synchronize()
    assert out.shape == (BH, T, 16, D)
    g = torch.Generator().manual_seed(3)
    for b in (4, 13):
        toks = torch.randint(0, T, (48,), generator=g)
        mem = snaps[b:b + 1].cpu().numpy()
        sel = idx[b:b + 1, toks].cpu().numpy()
        gathered, bad = orc.gather(mem, sel)
        assert bad == 0
        ref = orc.apply_query(gathered, c5["q"][b:b + 1, toks].double().numpy())
        np.testing.assert_allclose(out[b:b + 1, toks].cpu().double().numpy(), ref, rtol=1e-5, atol=1e-6,
                                   err_msg=f"gather_apply head {b}")
    colsum = snaps.double().sum(dim=2)                                   # [BH, S, D]
    for b in range(BH):
        sel_cs = colsum[b].index_select(0, idx[b].reshape(-1)).view(T, 16, D)
        expect = (sel_cs * qd[b].double().unsqueeze(1)).sum(-1)          # [T, 16]
        got = out[b].double().sum(-1)
        torch.testing.assert_close(got, expect, rtol=1e-4, atol=1e-6)
    # residual + LayerNorm over every token; sampled rows against the oracle
    h_online = c5["hid"].float().reshape(BH * T, D)
    w = (1 + 0.1 * torch.randn(D, generator=g)).to(dev_of(snaps))
    bias = (0.1 * torch.randn(D, generator=g)).to(dev_of(snaps))
    fused = capi.fuse_residual(h_online, out.view(BH * T, 16, D), gates.view(BH * T, 16), w, bias)
    torch.cuda.synchronize()
    rows = torch.randint(0, BH * T, (512,), generator=g)
    ref = orc.fuse_residual(h_online[rows].cpu().double().numpy(), out.view(BH * T, 16, D)[rows].cpu().double().numpy(),
                            gates.view(BH * T, 16)[rows].cpu().double().numpy(), w.cpu().double().numpy(),
                            bias.cpu().double().numpy())
    np.testing.assert_allclose(fused[rows].cpu().double().numpy(), ref, rtol=1e-5, atol=1e-5)


def test_c5_retrieve_fuse(c5):
    """The fused retrieval at config 5 (16 heads x 65536 tokens, top-16 of 512 float32 snapshots,
    bf16 queries): retrieve_fuse against the float32 two-kernel composition over every token,
    and sampled tokens of two heads against the oracle's gather, apply and fusion, at the
    north-star tolerance."""
    BH, T, D = c5["BH"], c5["T"], c5["D"]
    snaps, qd = c5["snaps"], c5["qd"]
    gates, idx, _ = capi.topk_route(qd, c5["sd"], 16, 1.0 / D ** 0.5)
    g = torch.Generator().manual_seed(8)
    w = (1 + 0.1 * torch.randn(D, generator=g)).to(snaps.device)
    bias = (0.1 * torch.randn(D, generator=g)).to(snaps.device)
    h_online = c5["hid"].float()
    fused = capi.retrieve_fuse(snaps, idx, qd, gates, h_online, w, bias)
    rows = capi.gather_apply(snaps, idx, qd, dtype=torch.float32)
    comp = capi.fuse_residual(h_online.view(BH * T, D), rows.view(BH * T, 16, D), gates.view(BH * T, 16), w, bias)
    torch.cuda.synchronize()
    del rows
    diff = (fused.view(BH * T, D) - comp).abs().max().item()
    assert diff < 2e-3, diff
    for b in (2, 11):
        toks = torch.randint(0, T, (32,), generator=g)
        gathered, bad = orc.gather(snaps[b:b + 1].cpu().numpy(), idx[b:b + 1, toks].cpu().numpy())
        assert bad == 0
        r = orc.apply_query(gathered, c5["q"][b:b + 1, toks].double().numpy())
        ref = orc.fuse_residual(h_online[b, toks].cpu().double().numpy(), r[0], gates[b, toks].cpu().double().numpy(),
                                w.cpu().double().numpy(), bias.cpu().double().numpy())
        np.testing.assert_allclose(fused[b, toks].cpu().double().numpy(), ref, rtol=2e-2, atol=2e-3,
                                   err_msg=f"retrieve_fuse head {b}")


def dev_of(t):
    return t.device


# ---------------------------------------------------------------- config 4
@pytest.mark.parametrize("mem_dtype", [torch.bfloat16, torch.float32])
def test_c4_scan(dev, mem_dtype):
    """One layer's scan at config 4 (B=4, T=8192, d_k=64, d_v=512, 64-token segments; the
    bf16 model carries a bf16 state): two batch rows against the oracle, the last snapshot
    is the final state, and a second call is bit-identical."""
    B, T, K, H, SEG = 4, 8192, 64, 512, 64
    k, v, q, m = scan_inputs(B, T, K, H, mem_dtype, seed=44)
    kd, vd, qd, md = k.to(dev), v.to(dev), q.to(dev), m.to(dev)
    print(f"config 4 scan state {mem_dtype}", flush=True)
    hid, mo, snaps = capi.chunk_update_fwd(kd, vd, qd, md, 0.97, SEG)
    hid2, mo2, snaps2 = capi.chunk_update_fwd(kd, vd, qd, md, 0.97, SEG)
    torch.cuda.synchronize()
    assert torch.equal(hid, hid2) and torch.equal(snaps, snaps2) and torch.equal(mo, mo2)
    if mem_dtype == torch.float32:
        assert torch.equal(snaps[:, -1], mo)
    else:
        assert torch.equal(snaps[:, -1].to(mem_dtype), mo)
    for b, (rh, rm, rs) in oracle_rows(k, v, q, m, (1, 3), SEG):
        close16(f"hidden[{b}]", hid[b:b + 1], rh)
        close16(f"snapshots[{b}]", snaps[b:b + 1], rs)
        close16(f"memory_out[{b}]", mo[b:b + 1], rm)


@pytest.mark.parametrize("base", [0, 64])
def test_c4_route_and_retrieval(dev, base):
    """One layer's retrieval at config 4: 4 x 8192 routing queries (bf16, 512 wide) over the
    summaries of the archive (base entries kept from an earlier call, then the 128 segments
    of this one; capacity 64), top-8; then gather + apply from the float16 archive
    [4, base + 128, 512, 64] widened to float32 with bf16 queries.  Routing of two whole
    batch rows bit-exact against the oracle's per-segment routing, retrieval of sampled
    tokens against the oracle's gather and apply."""
    B, T, D, K, H, SEG, CAP, TOP = 4, 8192, 512, 64, 512, 64, 64, 8
    S = base + T // SEG
    g = torch.Generator().manual_seed(400 + base)
    q_r = nrm(torch.randn(B, T, D, generator=g)).to(torch.bfloat16)
    k_r = nrm(torch.randn(B, S, D, generator=g)).to(torch.bfloat16)
    q = nrm(torch.randn(B, T, K, generator=g)).to(torch.bfloat16)
    states = (torch.randn(B, S, H, K, generator=g) * 0.05).to(torch.float16)
    scale = 1.0 / D ** 0.5
    print(f"config 4 routing base={base}", flush=True)
    gates, idx, sc = capi.segment_route(q_r.to(dev), k_r.to(dev), TOP, SEG, base, CAP, scale)
    torch.cuda.synchronize()
    for b in (0, 2):
        og, oi, osc = orc.segment_route(q_r[b:b + 1].float().numpy(), k_r[b:b + 1].float().numpy(), TOP, SEG, base,
                                        CAP, scale)
        assert np.array_equal(idx[b:b + 1].cpu().numpy(), oi), f"indices of row {b}"
        assert np.array_equal(sc[b:b + 1].cpu().numpy(), osc), f"scores of row {b}"
        np.testing.assert_allclose(gates[b:b + 1].cpu().numpy(), og, rtol=1e-5, atol=1e-6)
    filled = idx >= 0
    idx0 = idx.clamp(min=0)
    out = capi.gather_apply(states.to(dev), idx0, q.to(dev), dtype=torch.float32)
    torch.cuda.synchronize()
    assert out.shape == (B, T, TOP, H)
    for b in (1, 3):
        toks = torch.randint(0, T, (64,), generator=g)
        gathered, bad = orc.gather(states[b:b + 1].double().numpy(), idx0[b:b + 1, toks].cpu().numpy())
        assert bad == 0
        ref = orc.apply_query(gathered, q[b:b + 1, toks].double().numpy())
        np.testing.assert_allclose(out[b:b + 1, toks].cpu().double().numpy(), ref, rtol=1e-5, atol=1e-6,
                                   err_msg=f"gather_apply row {b}")
    if base == 0:
        # the first segment's tokens found an empty archive: no route is filled
        assert not bool(filled[:, :SEG].any())


def test_c4_model_forward_tracks_float32(dev):
    """The config-4 stack (Embedding 32000x512 -> 4 segment-memory layers, hidden 512, d_k 64,
    segments of 64, capacity 64, top-8, float16 archive) on 4 x 8192 token ids, bf16 against
    the same weights in float32 on the GPU.  Routing may pick another segment where two
    summaries score within bf16 rounding of each other, which moves that token's output by
    the LayerNorm's scale, so the bar is the relative L2 error of the whole output."""
    from rnn_with_grm_amd.segment_model import HierarchicalSegmentMemoryModel
    from rnn_with_grm_amd import cuda_ops

    B, T, V, DIM = 4, 8192, 32000, 512
    torch.manual_seed(0)
    emb = torch.nn.Embedding(V, DIM)
    grm = HierarchicalSegmentMemoryModel(DIM, DIM, DIM, num_layers=4, segment_length=64, memory_capacity_segments=64,
                                         retrieval_top_k=8, memory_key_dim=64, dropout=0.0, recomputation_ratio=0.0)
    g = torch.Generator().manual_seed(7)
    ids = torch.randint(0, V, (B, T), generator=g).to(dev)
    outs = {}
    before = cuda_ops.extension_module().hip_launch_count()
    for dt in (torch.float32, torch.bfloat16):
        print(f"config 4 model forward {dt}", flush=True)
        e = emb.to(device=dev, dtype=dt).eval()
        m = grm.to(device=dev, dtype=dt).eval()
        with torch.no_grad():
            o, _, _, _ = m(e(ids), reset_memory=True)
        torch.cuda.synchronize()
        outs[dt] = o.float()
        assert torch.isfinite(outs[dt]).all()
    assert cuda_ops.extension_module().hip_launch_count() > before
    a, r = outs[torch.bfloat16], outs[torch.float32]
    rel = float((a - r).norm() / r.norm())
    per_tok = ((a - r).norm(dim=-1) / r.norm(dim=-1).clamp_min(1e-12))
    frac_far = float((per_tok > 0.1).float().mean())
    print(f"config 4 model bf16 vs fp32: relative L2 {rel:.3e}, tokens beyond 0.1: {frac_far:.4f}", flush=True)
    assert rel < 5e-2, rel
    assert frac_far < 0.02, frac_far


# ---------------------------------------------------------------- config 1
def c1_inputs():
    """Config 1 exactly: fp32, B=2 x H=4 -> 8 sequences, T=512, d_k=d_v=64, q, k, v ~ N(0,1) from
    seed 0 (drawn in that order) with q and k L2-normalised per row, zero initial state."""
    g = torch.Generator().manual_seed(0)
    q = nrm(torch.randn(2, 4, 512, 64, generator=g)).reshape(8, 512, 64)
    k = nrm(torch.randn(2, 4, 512, 64, generator=g)).reshape(8, 512, 64)
    v = torch.randn(2, 4, 512, 64, generator=g).reshape(8, 512, 64)
    m = torch.zeros(8, 64, 64)
    return k, v, q, m


def test_config1_hip_path(dev):
    """Config 1 on the HIP path, against the double-precision oracle at 1e-5 (rtol and atol), every
    sequence and every element: the C ABI with 64-token snapshots, torch.ops.grm_cuda's
    chunk_update_forward (the reference's op, one call over all 512 tokens), cuda_segment_scan, and
    the reference model's granularity, cuda_chunk_update once per 64-token chunk carrying the
    state.  The native kernels must run (launch counter), with no generic-path call."""
    from rnn_with_grm_amd import cuda_ops

    k, v, q, m = c1_inputs()
    rh, rm, rs = orc.chunk_update_seq(k.double().numpy(), v.double().numpy(), q.double().numpy(),
                                      m.double().numpy(), 0.97, 64)
    kd, vd, qd, md = k.to(dev), v.to(dev), q.to(dev), m.to(dev)
    ext = cuda_ops.extension_module()
    launches, generic = ext.hip_launch_count(), ext.generic_path_calls()
    print("config 1: fp32 8 x 512, d=64, chunk 64", flush=True)
    outs = {}
    outs["capi"] = capi.chunk_update_fwd(kd, vd, qd, md, 0.97, 64)
    h, mo, aux = torch.ops.grm_cuda.chunk_update_forward(kd, vd, qd, md, 0.97)
    outs["op"] = (h, mo, None)
    outs["segment_scan"] = cuda_ops.cuda_segment_scan(kd, vd, qd, md, 0.97, 64)
    state, hs, snaps = md, [], []
    for t0 in range(0, 512, 64):
        hh, state = cuda_ops.cuda_chunk_update(kd[:, t0:t0 + 64], vd[:, t0:t0 + 64], qd[:, t0:t0 + 64], state, 0.97)
        hs.append(hh)
        snaps.append(state)
    outs["per_chunk"] = (torch.cat(hs, 1), state, torch.stack(snaps, 1))
    torch.cuda.synchronize()
    assert ext.hip_launch_count() > launches and ext.generic_path_calls() == generic
    for name, (hid, mout, sn) in outs.items():
        assert hid.dtype == torch.float32 and mout.dtype == torch.float32
        np.testing.assert_allclose(hid.cpu().double().numpy(), rh, rtol=1e-5, atol=1e-5, err_msg=f"{name} hidden")
        np.testing.assert_allclose(mout.cpu().double().numpy(), rm, rtol=1e-5, atol=1e-5, err_msg=f"{name} memory")
        if sn is not None:
            assert sn.shape == (8, 8, 64, 64)
            np.testing.assert_allclose(sn.cpu().double().numpy(), rs, rtol=1e-5, atol=1e-5,
                                       err_msg=f"{name} snapshots")


# ---------------------------------------------------------------- config 3, fused retrieval
def test_config3_retrieve_fuse(dev):
    """The launch the bench times for config 3's fused retrieval, at its geometry: 64 sequences x
    2048 bf16 queries, S=256 fp32 128x128 states, top-8 routing, h_online = M_online q, residual +
    LayerNorm (affine).  Four whole sequences (all 2048 queries each) element by element against
    the oracle's gather -> apply -> residual + LayerNorm in double precision at rtol 2e-2 /
    atol 2e-3 and relative L2 1e-3; the routing of those sequences bit-exact against the
    oracle's; every sequence against the float32 two-kernel composition."""
    BH, Q, S, D, K = 64, 2048, 256, 128, 8
    g = torch.Generator().manual_seed(1)
    q = nrm(torch.randn(BH, Q, D, generator=g)).to(torch.bfloat16)
    keys = nrm(torch.randn(BH, S, D, generator=g)).to(torch.bfloat16)
    states = torch.randn(BH, S, D, D, generator=g) * 0.02
    online = torch.randn(BH, D, D, generator=g) * 0.02
    w = 1 + 0.1 * torch.randn(D, generator=g)
    bias = 0.1 * torch.randn(D, generator=g)
    qd, kd, sd = q.to(dev), keys.to(dev), states.to(dev)
    h = torch.bmm(qd.float(), online.to(dev).transpose(1, 2).contiguous())       # h_online = M_online q
    print("config 3 retrieve_fuse: 64 x 2048 queries, S=256, k=8", flush=True)
    gates, idx, _ = capi.topk_route(qd, kd, K, 1.0 / D ** 0.5)
    fused = capi.retrieve_fuse(sd, idx, qd, gates, h, w.to(dev), bias.to(dev))
    rows = capi.gather_apply(sd, idx, qd, dtype=torch.float32)
    comp = capi.fuse_residual(h.view(BH * Q, D), rows.view(BH * Q, K, D), gates.view(BH * Q, K), w.to(dev),
                              bias.to(dev)).view(BH, Q, D)
    torch.cuda.synchronize()
    del rows
    torch.testing.assert_close(fused, comp, rtol=2e-3, atol=2e-3)
    hc, gc, ic = h.cpu().double().numpy(), gates.cpu().double().numpy(), idx.cpu().numpy()
    for b in (0, 21, 42, 63):
        og, oi, _ = orc.topk_route(q[b:b + 1].float().numpy(), keys[b:b + 1].float().numpy(), K, 1.0 / D ** 0.5)
        assert np.array_equal(ic[b:b + 1], oi), f"routing of sequence {b}"
        ref = np.empty((Q, D))
        for q0 in range(0, Q, 256):
            gathered, bad = orc.gather(states[b:b + 1].double().numpy(), ic[b:b + 1, q0:q0 + 256])
            assert bad == 0
            r = orc.apply_query(gathered, q[b:b + 1, q0:q0 + 256].double().numpy())[0]
            ref[q0:q0 + 256] = orc.fuse_residual(hc[b, q0:q0 + 256], r, gc[b, q0:q0 + 256], w.double().numpy(),
                                                 bias.double().numpy())
        got = fused[b].cpu().double().numpy()
        np.testing.assert_allclose(got, ref, rtol=2e-2, atol=2e-3, err_msg=f"retrieve_fuse sequence {b}")
        rel = np.linalg.norm(got - ref) / np.linalg.norm(ref)
        print(f"config 3 retrieve_fuse sequence {b}: relative L2 {rel:.3e}, max abs {np.abs(got - ref).max():.3e}",
              flush=True)
        assert rel < 1e-3, rel


@pytest.mark.parametrize("storage", [torch.float32, torch.float16])
def test_c4_model_forward_against_fallback_arithmetic(dev, storage):
    """The config-4 stack at full size (4 x 8192 token ids, 4 layers, hidden 512, d_k 64, segments of 64,
    capacity 64, top-8) in float32 on the native kernels against the same model and weights with
    cuda_cpp_debug_fallback=True, where the scan, routing, gather + apply and fusion run the torch
    restatements of the reference's fallbacks (cuda_ops.py:218-284) segment by segment, layer by layer.
    float32 archive: every token of every layer within 1e-5 relative (measured: at most 1.0e-6).
    float16 archive (the reference's default): the archive's rounding of states that differ in their
    last float32 bits can flip a float16 bit, and a near-tie routing decision in a later layer then
    differs for a few tokens and cascades; layer 0 is held per token at 1e-4 (measured: 7.9e-6), the
    final output at relative L2 1e-2 (measured: 3.3e-3)."""
    from rnn_with_grm_amd.segment_model import HierarchicalSegmentMemoryModel

    B, T, V, DIM = 4, 8192, 32000, 512
    torch.manual_seed(0)
    emb = torch.nn.Embedding(V, DIM).to(dev).eval()
    kw = dict(num_layers=4, segment_length=64, memory_capacity_segments=64, retrieval_top_k=8, memory_key_dim=64,
              dropout=0.0, recomputation_ratio=0.0, memory_storage_dtype=storage)
    native = HierarchicalSegmentMemoryModel(DIM, DIM, DIM, **kw).to(dev).eval()
    slow = HierarchicalSegmentMemoryModel(DIM, DIM, DIM, cuda_cpp_debug_fallback=True, **kw).to(dev).eval()
    slow.load_state_dict(native.state_dict())
    g = torch.Generator().manual_seed(11)
    ids = torch.randint(0, V, (B, T), generator=g).to(dev)
    with torch.no_grad():
        x = emb(ids)
        outs = {}
        for name, m in (("native", native), ("fallback", slow)):
            print(f"config 4 float32 layers, {storage} archive: {name}", flush=True)
            cur = x
            for i, layer in enumerate(m.layers):
                cur, _, _, _ = layer(cur, return_all_outputs=True, reset_memory=True)
                outs[(name, i)] = cur
    torch.cuda.synchronize()
    for i in range(4):
        a, r = outs[("native", i)], outs[("fallback", i)]
        per_tok = ((a - r).norm(dim=-1) / r.norm(dim=-1).clamp_min(1e-12))
        rel = float((a - r).norm() / r.norm())
        print(f"config 4 {storage} layer {i}: largest per-token relative error {float(per_tok.max()):.3e}, "
              f"relative L2 {rel:.3e}", flush=True)
        if storage == torch.float32:
            assert float(per_tok.max()) < 1e-5, (i, float(per_tok.max()))
        elif i == 0:
            assert float(per_tok.max()) < 1e-4, float(per_tok.max())
        elif i == 3:
            assert rel < 1e-2, rel
