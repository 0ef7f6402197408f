"""swiftllm_amd — MI355X (gfx950) implementation of SwiftLLM's decode hot path.

The compute lives in libswiftllm_hip.so (hand-written HIP kernels behind the
C ABI declared in include/swiftllm_hip.h). This package is the host side:
library loading, device memory through the HIP runtime, and the
reference-named interface (paged_attention.py, moe.py).
"""

from ._lib import LIB_PATH, LibraryMissing, lib  # noqa: F401
from .paged_attention import (  # noqa: F401
    BatchedCacheMetadata,
    CudaError,
    DeviceMemoryError,
    DeviceNotFound,
    InitError,
    InvalidParameter,
    KernelError,
    KvCacheConfig,
    NotSupported,
    PagedAttention,
    PagedAttentionConfig,
    PagedAttentionParams,
    ReshapeCacheParams,
    SequenceCacheMetadata,
    blocks_needed,
    get_slot_mapping,
    paged_attention_decode,
    reshape_and_cache,
)

__version__ = "0.1.0"
