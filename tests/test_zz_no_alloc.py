"""grm_hip_chunk_update_fwd_noalloc: the forward scan with its time-split scratch in a
fixed device array of the library instead of caller memory.  Through the C ABI, against
grm_hip_chunk_update_fwd with a caller workspace on the same inputs: the same kernels
and the same plan, so the results are bit-identical.  Two calls in a row, the second
with smaller inputs; two calls on two streams at once; then a call whose sizes need more
scratch than the library holds."""

import pytest
import torch

from rnn_with_grm_amd import capi

pytestmark = pytest.mark.gpu


def inputs(B, T, K, H, mem_dtype, seed):
    g = torch.Generator().manual_seed(seed)
    q = torch.nn.functional.normalize(torch.randn(B, T, K, generator=g), dim=-1).to(torch.bfloat16)
    k = torch.nn.functional.normalize(torch.randn(B, T, K, generator=g), dim=-1).to(torch.bfloat16)
    v = torch.randn(B, T, H, generator=g).to(torch.bfloat16)
    m = (torch.randn(B, H, K, generator=g) * 0.02).to(mem_dtype)
    return k, v, q, m


@pytest.mark.parametrize("mem_dtype", [torch.float32, torch.bfloat16])
def test_noalloc_matches_workspace_entry_point(dev, mem_dtype):
    cases = [(4, 4096, 128, 128, 64), (2, 1000, 64, 96, 100)]   # second call: smaller input
    for B, T, K, H, seg in cases:
        need = capi.fwd_workspace_bytes(B, T, K, H, seg)
        assert 0 < need <= capi.noalloc_limit(), "the case must use the time-split scratch"
        kd, vd, qd, md = (t.to(dev) for t in inputs(B, T, K, H, mem_dtype, seed=B * 7 + T))
        print(f"noalloc B={B} T={T} K={K} H={H} seg={seg} state {mem_dtype}", flush=True)
        before = capi.launch_count()
        h0, m0, s0 = capi.chunk_update_fwd_noalloc(kd, vd, qd, md, 0.97, seg)
        torch.cuda.synchronize()
        assert capi.launch_count() >= before + 2, "time split runs a state pass and a full pass"
        h1, m1, s1 = capi.chunk_update_fwd(kd, vd, qd, md, 0.97, seg)
        torch.cuda.synchronize()
        assert torch.equal(h0, h1) and torch.equal(m0, m1) and torch.equal(s0, s1)
        # and with no snapshots (memory_out only)
        h2, m2, _ = capi.chunk_update_fwd_noalloc(kd, vd, qd, md, 0.97, 0)
        h3, m3, _ = capi.chunk_update_fwd(kd, vd, qd, md, 0.97, 0)
        torch.cuda.synchronize()
        assert torch.equal(h2, h3) and torch.equal(m2, m3)


def test_noalloc_calls_on_two_streams_take_the_scratch_in_turn(dev):
    """Two calls that both need the time-split scratch, issued back to back on two streams
    while the first stream is still busy with a long matrix product: the second call's
    stream waits for the first call, so both results equal the workspace entry point's
    (without the wait the two calls would write their part states into the same array)."""
    B, T, K, H, seg = 4, 8192, 128, 128, 64
    assert 0 < capi.fwd_workspace_bytes(B, T, K, H, seg) <= capi.noalloc_limit()
    a_in = [t.to(dev) for t in inputs(B, T, K, H, torch.float32, seed=11)]
    b_in = [t.to(dev) for t in inputs(B, T, K, H, torch.float32, seed=12)]
    busy = torch.randn(4096, 4096, device=dev)
    torch.cuda.synchronize()
    sa, sb = torch.cuda.Stream(dev), torch.cuda.Stream(dev)
    print(f"noalloc two streams B={B} T={T} K={K} H={H} seg={seg}", flush=True)
    with torch.cuda.stream(sa):
        for _ in range(8):
            busy = busy @ busy * 1e-3  # keeps stream A busy for a while
        ha, ma, sna = capi.chunk_update_fwd_noalloc(*a_in, 0.97, seg)
    with torch.cuda.stream(sb):
        hb, mb, snb = capi.chunk_update_fwd_noalloc(*b_in, 0.97, seg)
    torch.cuda.synchronize()
    for (k, v, q, m), (h0, m0, s0) in ((a_in, (ha, ma, sna)), (b_in, (hb, mb, snb))):
        h1, m1, s1 = capi.chunk_update_fwd(k, v, q, m, 0.97, seg)
        torch.cuda.synchronize()
        assert torch.equal(h0, h1) and torch.equal(m0, m1) and torch.equal(s0, s1)


def test_noalloc_rejects_beyond_limit(dev, monkeypatch):
    """Every part count the library picks by itself fits the fixed scratch (at most about
    17 MiB); a forced part count (GRM_HIP_CHUNK_PARTS) can ask for more, and that call is
    refused before any launch."""
    B, T, K, H = 16, 65536, 128, 128
    assert capi.fwd_workspace_bytes(B, T, K, H, 0) <= capi.noalloc_limit()
    monkeypatch.setenv("GRM_HIP_CHUNK_PARTS", "200")
    need = capi.fwd_workspace_bytes(B, T, K, H, 0)
    assert need > capi.noalloc_limit()
    kd = torch.zeros((B, T, K), dtype=torch.bfloat16, device=dev)
    vd = torch.zeros((B, T, H), dtype=torch.bfloat16, device=dev)
    md = torch.zeros((B, H, K), dtype=torch.float32, device=dev)
    before = capi.launch_count()
    with pytest.raises(RuntimeError, match="beyond the library's fixed"):
        capi.chunk_update_fwd_noalloc(kd, vd, kd, md, 0.97, 0)
    assert capi.launch_count() == before
