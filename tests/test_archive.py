"""DeviceSegmentArchive against a deque restatement of the reference's
SegmentMemoryArchive (grm/core/paper_grm.py:30-349): push/eviction, summaries,
retrieval of states and of applied queries, and the extra-state format.

The restatement below follows the reference line by line in behaviour:
deques with maxlen (paper_grm.py:30-45), storage-dtype copies on push
(:135-146), stacked oldest-first summaries (:148-160), stacked float32 states
gathered per index (:203-236) and the normalised query applied to them
(:271-313).  It is test infrastructure only."""

from collections import deque
from types import SimpleNamespace

import pytest
import torch
import torch.nn as nn
import torch.nn.functional as F

from rnn_with_grm_amd.archive import DeviceSegmentArchive, SegmentCheckpoint


class DequeArchive:
    def __init__(self, cap, dtype):
        self.cap, self.dtype = cap, dtype
        self.groups = {}

    def push(self, memory, summary, ckpt):
        g = self.groups.setdefault(memory.size(0), (deque(maxlen=self.cap), deque(maxlen=self.cap),
                                                    deque(maxlen=self.cap)))
        g[0].append(memory.detach().to(self.dtype).clone())
        g[1].append(summary.detach().to(self.dtype).clone())
        g[2].append((ckpt.inputs.detach().clone(), ckpt.memory_start.detach().to(self.dtype).clone()))

    def summaries(self, b, dtype):
        return torch.stack(list(self.groups[b][1]), 0).to(dtype).permute(1, 0, 2).contiguous()

    def memories(self, idx):
        allm = torch.stack(list(self.groups[idx.size(0)][0]), 0).to(torch.float32).permute(1, 0, 2, 3).contiguous()
        bi = torch.arange(idx.size(0)).view(-1, *([1] * (idx.ndim - 1)))
        return allm[bi, idx]

    def applied(self, query_inputs, idx, cell):
        mem = self.memories(idx)
        q = F.normalize(cell.query_proj(query_inputs), p=2, dim=-1, eps=1e-6).to(mem.dtype)
        if idx.ndim == 3:
            return torch.einsum("bqrhk,bqk->bqrh", mem, q)
        return torch.einsum("brhk,bk->brh", mem, q)


def make_cell(d_in, d_k, seed=0):
    torch.manual_seed(seed)
    return SimpleNamespace(query_proj=nn.Linear(d_in, d_k))


@pytest.mark.parametrize("store", [torch.float16, torch.float32])
def test_archive_matches_deque_restatement(store):
    B, H, K, D, cap = 3, 24, 16, 20, 5
    cell = make_cell(D, K)
    arch = DeviceSegmentArchive(H, K, D, cap, store)
    ref = DequeArchive(cap, store)
    g = torch.Generator().manual_seed(1)
    for step in range(12):  # more pushes than the capacity: eviction
        mem = torch.randn(B, H, K, generator=g)
        summ = torch.randn(B, D, generator=g)
        ck = SegmentCheckpoint(torch.randn(7, B, D, generator=g), torch.randn(B, H, K, generator=g))
        arch.push(mem, summ, ck)
        ref.push(mem, summ, ck)
        n = min(step + 1, cap)
        assert arch.get_num_segments(B) == n
        s = arch.get_segment_summaries(B, torch.device("cpu"), torch.float32)
        assert torch.equal(s, ref.summaries(B, torch.float32))
        idx = torch.randint(0, n, (B, 6, 3), generator=g)
        x = torch.randn(B, 6, D, generator=g)
        got = arch.retrieve_from_indices(x, idx, None, cell, torch.device("cpu"), 0.97)
        torch.testing.assert_close(got, ref.applied(x, idx, cell), rtol=1e-5, atol=1e-6)
        states = arch.retrieve_memories(idx, None, cell, torch.device("cpu"), 0.97)
        assert states.dtype == torch.float32 and torch.equal(states, ref.memories(idx))
        idx2 = torch.randint(0, n, (B, 4), generator=g)  # rank-2 routing
        x2 = torch.randn(B, D, generator=g)
        torch.testing.assert_close(arch.retrieve_from_indices(x2, idx2, None, cell, torch.device("cpu"), 0.97),
                                   ref.applied(x2, idx2, cell), rtol=1e-5, atol=1e-6)
    assert int(arch.total_pushed) == 12


def test_extra_state_is_the_reference_format():
    B, H, K, D, cap = 2, 8, 4, 6, 3
    arch = DeviceSegmentArchive(H, K, D, cap, torch.float16)
    pushed = []
    for i in range(5):
        m, s = torch.full((B, H, K), float(i)), torch.full((B, D), float(10 + i))
        arch.push(m, s, SegmentCheckpoint(torch.zeros(4, B, D), m))
        pushed.append((m, s))
    st = arch.get_extra_state()
    grp = st["groups"][B]
    assert set(grp) == {"memories", "summaries", "checkpoints"}
    assert [float(t[0, 0, 0]) for t in grp["memories"]] == [2.0, 3.0, 4.0]  # oldest first, deque eviction
    assert [float(t[0, 0]) for t in grp["summaries"]] == [12.0, 13.0, 14.0]
    assert all(t.dtype == torch.float16 and t.shape == (B, H, K) for t in grp["memories"])
    assert [set(c) for c in grp["checkpoints"]] == [{"inputs", "memory_start"}] * 3
    # a state written in that format (by either implementation) loads and reads back the same
    other = DeviceSegmentArchive(H, K, D, cap, torch.float16)
    other.set_extra_state(st)
    assert other.get_num_segments(B) == 3
    assert torch.equal(other.get_segment_summaries(B, torch.device("cpu")), arch.get_segment_summaries(B, torch.device("cpu")))
    idx = torch.tensor([[0, 2], [1, 1]])
    assert torch.equal(other.retrieve_memories(idx, None, None, torch.device("cpu"), 0.97),
                       arch.retrieve_memories(idx, None, None, torch.device("cpu"), 0.97))
    # and pushing on after a load continues the ring in deque order
    other.push(torch.full((B, H, K), 9.0), torch.zeros(B, D), SegmentCheckpoint(torch.zeros(1), torch.zeros(1)))
    assert [float(t[0, 0, 0]) for t in other.get_extra_state()["groups"][B]["memories"]] == [3.0, 4.0, 9.0]


def test_push_segments_equals_repeated_push():
    B, H, K, D, cap = 2, 8, 4, 6, 4
    g = torch.Generator().manual_seed(3)
    mems, sums = torch.randn(B, 7, H, K, generator=g), torch.randn(B, 7, D, generator=g)
    a = DeviceSegmentArchive(H, K, D, cap, torch.float16)
    b = DeviceSegmentArchive(H, K, D, cap, torch.float16)
    a.push(torch.randn(B, H, K, generator=g), torch.randn(B, D, generator=g), SegmentCheckpoint(torch.zeros(1), torch.zeros(1)))
    b.set_extra_state(a.get_extra_state())
    a.push_segments(mems[:, :2], sums[:, :2])
    a.push_segments(mems[:, 2:], sums[:, 2:])
    for i in range(7):
        b.push(mems[:, i], sums[:, i], SegmentCheckpoint(torch.zeros(1), torch.zeros(1)))
    sa, sb = a.get_extra_state()["groups"][B], b.get_extra_state()["groups"][B]
    assert all(torch.equal(x, y) for x, y in zip(sa["memories"], sb["memories"]))
    assert all(torch.equal(x, y) for x, y in zip(sa["summaries"], sb["summaries"]))


def test_groups_empty_reads_and_limits():
    arch = DeviceSegmentArchive(8, 4, 6, 3, torch.float16)
    cpu = torch.device("cpu")
    assert arch.get_segment_summaries(5, cpu).shape == (5, 0, 6)
    idx = torch.zeros(5, 2, 3, dtype=torch.long)
    assert arch.retrieve_from_indices(torch.zeros(5, 2, 6), idx, None, None, cpu, 0.97).shape == (5, 2, 0, 8)
    assert arch.retrieve_memories(idx, None, None, cpu, 0.97).shape == (5, 2, 0, 8, 4)
    arch.push(torch.ones(2, 8, 4), torch.ones(2, 6), SegmentCheckpoint(torch.zeros(1), torch.zeros(1)))
    arch.push(torch.ones(3, 8, 4), torch.ones(3, 6), SegmentCheckpoint(torch.zeros(1), torch.zeros(1)))
    assert arch.get_num_segments(2) == 1 and arch.get_num_segments(3) == 1 and arch.get_num_segments() == 1
    info = arch.get_memory_info()
    assert info["num_segments"] == 2 and info["num_groups"] == 2
    arch.clear()
    assert arch.get_num_segments() == 0 and int(arch.total_pushed) == 0
    with pytest.raises(NotImplementedError):
        DeviceSegmentArchive(8, 4, 6, 3, torch.float16, recomputation_ratio=0.02)


@pytest.mark.gpu
def test_archive_on_device_matches_restatement():
    """The ring on the GPU (fused gather_apply with float32 widening of the float16 ring)
    against the deque restatement on the CPU."""
    dev = torch.device("cuda:0")
    B, H, K, D, cap = 4, 512, 64, 96, 64
    cell = make_cell(D, K, seed=2)
    cell_dev = SimpleNamespace(query_proj=nn.Linear(D, K).to(dev))
    cell_dev.query_proj.load_state_dict(cell.query_proj.state_dict())
    arch = DeviceSegmentArchive(H, K, D, cap, torch.float16).to(dev)
    ref = DequeArchive(cap, torch.float16)
    g = torch.Generator().manual_seed(4)
    mems = torch.randn(B, 70, H, K, generator=g) * 0.02
    sums = torch.randn(B, 70, D, generator=g)
    arch.push_segments(mems.to(dev), sums.to(dev))
    for i in range(70):
        ref.push(mems[:, i], sums[:, i], SegmentCheckpoint(torch.zeros(1), torch.zeros(1)))
    assert torch.equal(arch.get_segment_summaries(B, dev).cpu(), ref.summaries(B, torch.float32))
    idx = torch.randint(0, cap, (B, 64, 8), generator=g)
    x = torch.randn(B, 64, D, generator=g)
    got = arch.retrieve_from_indices(x.to(dev), idx.to(dev), None, cell_dev, dev, 0.97)
    want = ref.applied(x, idx, cell)
    torch.testing.assert_close(got.cpu(), want, rtol=1e-4, atol=1e-5)
    assert torch.equal(arch.retrieve_memories(idx.to(dev), None, None, dev, 0.97).cpu(), ref.memories(idx))


def test_invalid_positions_stay_invalid():
    """A position outside the kept deque (the -1 of an empty routing slot, or one past the
    end) is not remapped onto a ring slot: on the CPU the gather raises, as index_select
    does in the reference's CPU path."""
    arch = DeviceSegmentArchive(8, 4, 6, 3, torch.float32)
    g = torch.Generator().manual_seed(9)
    arch.push_segments(torch.randn(2, 5, 8, 4, generator=g), torch.randn(2, 5, 6, generator=g))
    slots = arch.slots(torch.tensor([[0, 2, -1, 3]]), 2)
    assert slots[0, 2] == -1 and slots[0, 3] == -1 and bool((slots[0, :2] >= 0).all())
    with pytest.raises((IndexError, RuntimeError)):
        arch.retrieve_memories(torch.tensor([[0, -1], [1, 2]]), None, None, torch.device("cpu"), 0.97)


@pytest.mark.gpu
def test_invalid_positions_read_zero_on_device():
    """On the GPU the gather writes a zero row for an invalid position (and counts it)."""
    dev = torch.device("cuda:0")
    arch = DeviceSegmentArchive(8, 4, 6, 3, torch.float32).to(dev)
    g = torch.Generator().manual_seed(9)
    mems = torch.randn(2, 5, 8, 4, generator=g)
    arch.push_segments(mems.to(dev), torch.randn(2, 5, 6, generator=g).to(dev))
    got = arch.retrieve_memories(torch.tensor([[0, -1], [2, 3]], device=dev), None, None, dev, 0.97).cpu()
    assert torch.count_nonzero(got[0, 1]) == 0 and torch.count_nonzero(got[1, 1]) == 0
    assert torch.equal(got[0, 0], mems[0, 2]) and torch.equal(got[1, 0], mems[1, 4])


def test_recompute_rate_counters_mirrored_on_host():
    """get_recompute_rate reads a host mirror of the counters (no device read in a forward);
    it agrees with the buffers after retrievals, re-reads them after a state-dict load or
    direct writes detected by the load hook, and resets with clear()."""
    B, H, K, D, cap = 2, 8, 4, 6, 3
    arch = DeviceSegmentArchive(H, K, D, cap, torch.float16)
    for i in range(3):
        arch.push(torch.full((B, H, K), float(i)), torch.zeros(B, D), SegmentCheckpoint(torch.zeros(1), torch.zeros(1)))
    idx = torch.tensor([[0, 2], [1, 1]])
    arch.retrieve_memories(idx, None, None, torch.device("cpu"), 0.97)
    arch.retrieve_memories(idx, None, None, torch.device("cpu"), 0.97)
    assert int(arch.total_retrieved) == 8 and arch._host_counts == [8, 0]
    assert arch.get_recompute_rate() == 0.0
    other = DeviceSegmentArchive(H, K, D, cap, torch.float16)
    sd = arch.state_dict()
    sd["total_recomputed"] = torch.tensor(2)
    other.load_state_dict(sd)
    assert other._host_counts is None
    assert other.get_recompute_rate() == 0.25 and other._host_counts == [8, 2]
    other.clear()
    assert other._host_counts == [0, 0] and other.get_recompute_rate() == 0.0 and int(other.total_retrieved) == 0


def test_push_segments_wraps_like_repeated_push():
    """Whole-sequence pushes of ragged sizes whose slots wrap around the ring (two runs of
    slots), and pushes longer than the capacity, keep the same ring as one push per segment."""
    B, H, K, D, cap = 2, 4, 3, 5, 5
    g = torch.Generator().manual_seed(9)
    sizes = [3, 3, 1, 4, 7, 2, 5, 6]
    total = sum(sizes)
    mems, sums = torch.randn(B, total, H, K, generator=g), torch.randn(B, total, D, generator=g)
    a = DeviceSegmentArchive(H, K, D, cap, torch.float16)
    b = DeviceSegmentArchive(H, K, D, cap, torch.float16)
    i0 = 0
    for n in sizes:
        a.push_segments(mems[:, i0:i0 + n], sums[:, i0:i0 + n])
        for i in range(i0, i0 + n):
            b.push(mems[:, i], sums[:, i], SegmentCheckpoint(torch.zeros(1), torch.zeros(1)))
        i0 += n
        sa, sb = a.get_extra_state()["groups"][B], b.get_extra_state()["groups"][B]
        assert len(sa["memories"]) == len(sb["memories"]) == min(cap, i0)
        assert all(torch.equal(x, y) for x, y in zip(sa["memories"], sb["memories"]))
        assert all(torch.equal(x, y) for x, y in zip(sa["summaries"], sb["summaries"]))
