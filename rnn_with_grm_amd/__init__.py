"""MI355X-native GRM hot path: chunked linear-memory update + query
application, top-k routing, archived-state gather and residual fusion.

``rnn_with_grm_amd.cuda_ops`` mirrors the reference's ``grm.core.cuda_ops``
surface; ``rnn_with_grm_amd.archive.DeviceSegmentArchive`` is a device ring
drop-in for the reference's ``SegmentMemoryArchive``;
``rnn_with_grm_amd.capi`` binds the C ABI of libgrm_hip.so directly.
"""

from .archive import DeviceSegmentArchive, SegmentCheckpoint  # noqa: F401

from .cuda_ops import (  # noqa: F401
    GrmExtensionUnavailable,
    cuda_apply_query,
    cuda_batched_memory_gather,
    cuda_chunk_update,
    cuda_fuse_residual,
    cuda_gather_apply,
    cuda_segment_scan,
    cuda_topk_route,
    get_grm_cuda_runtime_status,
    is_grm_cpp_extension_available,
    is_grm_cuda_available,
    load_grm_cuda_extension,
)

__all__ = [
    "DeviceSegmentArchive",
    "GrmExtensionUnavailable",
    "SegmentCheckpoint",
    "cuda_apply_query",
    "cuda_batched_memory_gather",
    "cuda_chunk_update",
    "cuda_fuse_residual",
    "cuda_gather_apply",
    "cuda_segment_scan",
    "cuda_topk_route",
    "get_grm_cuda_runtime_status",
    "is_grm_cpp_extension_available",
    "is_grm_cuda_available",
    "load_grm_cuda_extension",
]
