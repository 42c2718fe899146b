"""C ABI checks that need no GPU: libgrm_hip.so loads, exports every entry point
declared in include/grm_hip.h, and rejects bad arguments before touching the device."""

import ctypes
import re
from pathlib import Path

import pytest

from rnn_with_grm_amd import capi

HEADER = Path(__file__).resolve().parents[1] / "include" / "grm_hip.h"


def declared_symbols():
    text = HEADER.read_text()
    return sorted(set(re.findall(r"^\s*(?:int|int64_t|const char\*|uint64_t)\s+(grm_hip_\w+)\s*\(", text, re.M)))


def test_header_declares_all_bound_symbols():
    assert declared_symbols() == sorted(capi.SIGNATURES)


def test_library_exports_every_declared_symbol():
    lib = ctypes.CDLL(str(capi.LIB_PATH))
    for name in declared_symbols():
        assert hasattr(lib, name), name


def test_workspace_query():
    lib = capi.load()
    assert lib.grm_hip_chunk_update_fwd_workspace(0, 10, 8, 8, 0) == 0
    assert lib.grm_hip_chunk_update_fwd_workspace(4, 64, 64, 512, 0) == 0  # one chunk: no split
    ws = lib.grm_hip_chunk_update_fwd_workspace(16, 65536, 128, 128, 128)  # long context splits
    assert ws > 0 and ws % (16 * 128 * 128 * 4) == 0


def test_abi_version_and_counters():
    lib = capi.load()
    assert lib.grm_hip_abi_version() == 109
    assert capi.launch_count() >= 0


def _null():
    return None


@pytest.mark.parametrize("kwargs,code", [
    (dict(key_dim=0), capi.EINVAL),
    (dict(key_dim=300), capi.EUNSUPPORTED),
    (dict(in_dtype=7), capi.EUNSUPPORTED),
    (dict(mem_dtype=capi.F16, in_dtype=capi.BF16), capi.EUNSUPPORTED),
    (dict(batch=-1), capi.EINVAL),
    (dict(decay=float("nan")), capi.EINVAL),
    (dict(snapshot=True, snapshot_len=0), capi.EINVAL),
])
def test_chunk_fwd_rejects(kwargs, code):
    a = dict(batch=2, seq_len=4, key_dim=8, value_dim=4, in_dtype=capi.F32, mem_dtype=capi.F32, decay=0.9,
             snapshot=False, snapshot_len=0)
    a.update(kwargs)
    fake = ctypes.c_void_p(16)  # never dereferenced: validation fails first
    rc = capi.load().grm_hip_chunk_update_fwd(fake, fake, fake, fake, fake, ctypes.c_void_p(32),
                                              fake if a["snapshot"] else None, None, 0, a["batch"], a["seq_len"],
                                              a["key_dim"], a["value_dim"], a["in_dtype"], a["mem_dtype"],
                                              a["decay"], a["snapshot_len"], None)
    assert rc == code
    assert capi.last_error()


def test_chunk_fwd_zero_batch_is_noop():
    assert capi.load().grm_hip_chunk_update_fwd(None, None, None, None, None, None, None, None, 0, 0, 5, 8, 4,
                                                capi.BF16, capi.F32, 0.97, 0, None) == capi.OK


def test_chunk_fwd_null_pointers_rejected():
    rc = capi.load().grm_hip_chunk_update_fwd(None, None, None, None, None, None, None, None, 0, 1, 5, 8, 4,
                                              capi.BF16, capi.F32, 0.97, 0, None)
    assert rc == capi.EINVAL


def test_other_entry_points_reject():
    lib = capi.load()
    fake = ctypes.c_void_p(16)
    assert lib.grm_hip_batched_gather(fake, fake, fake, 1, 2, 3, 4, 3, None, None) == capi.EUNSUPPORTED
    assert lib.grm_hip_batched_gather(fake, fake, fake, -1, 2, 3, 4, 4, None, None) == capi.EINVAL
    assert lib.grm_hip_batched_gather(None, None, None, 0, 2, 3, 4, 4, None, None) == capi.OK
    assert lib.grm_hip_apply_query_fwd(fake, fake, fake, 1, 1, 1, 1, 4, 9, None) == capi.EUNSUPPORTED
    assert lib.grm_hip_apply_query_fwd(fake, fake, fake, -2, 1, 1, 1, 4, 0, None) == capi.EINVAL
    assert lib.grm_hip_topk_route(fake, fake, fake, fake, fake, 1, 1, 4, 4, 0, 0, 1.0, 1.0, None) == capi.EINVAL
    assert lib.grm_hip_topk_route(fake, fake, fake, fake, fake, 1, 1, 4, 4, 0, 2, 1.0, 0.0, None) == capi.EINVAL
    assert lib.grm_hip_topk_route(fake, fake, fake, fake, fake, 1, 1, 1000, 4, 0, 200, 1.0, 1.0,
                                  None) == capi.EUNSUPPORTED
    assert lib.grm_hip_segment_route(fake, fake, fake, fake, fake, 1, 10, 2, 4, 0, 2, 3, 0, 8, 1.0, 1.0,
                                     None) == capi.EINVAL  # window past the keys
    assert lib.grm_hip_segment_route(fake, fake, fake, fake, fake, 1, 10, 4, 4, 0, 200, 3, 0, 8, 1.0, 1.0,
                                     None) == capi.EINVAL  # top_k > 128
    assert lib.grm_hip_segment_route(fake, fake, fake, fake, fake, 1, 10, 4, 4, 0, 2, 0, 0, 8, 1.0, 1.0,
                                     None) == capi.EINVAL  # segment_len 0
    assert lib.grm_hip_fuse_residual(fake, fake, fake, None, None, fake, 1, 1, 4096, 0, 1e-5,
                                     None) == capi.EUNSUPPORTED
    assert lib.grm_hip_chunk_update_bwd(fake, fake, fake, fake, fake, fake, fake, fake, fake, fake, fake, 0, fake,
                                        1, 4, 512, 4, 0, 0, 0.9, None) == capi.EUNSUPPORTED
