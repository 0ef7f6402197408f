"""The C ABI of libswiftllm_hip.so: it loads, exports every function that
include/swiftllm_hip.h declares, and validates arguments on the host before
touching a device (no GPU needed for these tests)."""

import ctypes
import re
from pathlib import Path

import numpy as np
import pytest

from swiftllm_amd import _hip, _lib
from swiftllm_amd import paged_attention as pa

HEADER = Path(__file__).resolve().parents[1] / "include" / "swiftllm_hip.h"

# Status values mirror CudaError (crates/swiftllm-cuda/src/lib.rs:16-42).
OK, INIT, KERNEL, MEMORY, INVALID, NODEV, UNSUP = 0, -1, -2, -3, -4, -5, -6


def declared_functions():
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    names = re.findall(r"^\s*(?:const\s+)?[A-Za-z_][\w\s\*]*?\b([A-Za-z_]\w*)\s*\(", text, flags=re.M)
    return sorted({n for n in names if n not in ("defined", "__has_include", "if")})


def test_header_declares_the_reference_launchers():
    names = declared_functions()
    # paged_attention.cu:232, :271 — same names as the reference launchers
    assert "launch_paged_attention_v1" in names
    assert "launch_reshape_and_cache" in names
    assert len(names) >= 20


def test_every_declared_function_is_exported():
    L = _lib.lib()
    missing = [n for n in declared_functions() if not hasattr(L, n)]
    assert not missing, missing


def test_loader_signatures_cover_the_header():
    assert set(declared_functions()) == set(_lib.SIGNATURES)


def test_dropin_launcher_argument_lists():
    """Parameter lists of the drop-in names equal the reference launchers'
    (paged_attention.cu:232-247, :271-282) with hipStream_t for cudaStream_t."""
    text = HEADER.read_text()
    v1 = re.search(r"void launch_paged_attention_v1\((.*?)\);", text, flags=re.S).group(1)
    params = [p.strip().split()[-1].lstrip("*") for p in v1.split(",")]
    assert params == ["output", "query", "key_cache", "value_cache", "block_tables", "context_lens",
                      "scale", "num_seqs", "num_heads", "num_kv_heads", "head_dim", "block_size",
                      "max_num_blocks_per_seq", "stream"]
    rc = re.search(r"void launch_reshape_and_cache\((.*?)\);", text, flags=re.S).group(1)
    params = [p.strip().split()[-1].lstrip("*") for p in rc.split(",")]
    assert params == ["key", "value", "key_cache", "value_cache", "slot_mapping", "num_tokens",
                      "num_kv_heads", "head_dim", "block_size", "stream"]


def test_version_and_status_strings():
    L = _lib.lib()
    assert L.swiftllm_hip_version().decode().startswith("0.1.0")
    assert isinstance(L.swiftllm_hip_last_error_message(), bytes)


FAKE = 0x1000  # never dereferenced: validation fails first


def _v1(**kw):
    a = dict(output=FAKE, query=FAKE, key_cache=FAKE, value_cache=FAKE, block_tables=FAKE,
             context_lens=FAKE, scale=0.1, num_seqs=2, num_heads=32, num_kv_heads=8, head_dim=128,
             block_size=16, max_num_blocks_per_seq=4, num_blocks=0)
    a.update(kw)
    L = _lib.lib()
    return L.swiftllm_hip_launch_paged_attention_v1(
        a["output"], a["query"], a["key_cache"], a["value_cache"], a["block_tables"],
        a["context_lens"], a["scale"], a["num_seqs"], a["num_heads"], a["num_kv_heads"],
        a["head_dim"], a["block_size"], a["max_num_blocks_per_seq"], a["num_blocks"], None)


@pytest.mark.parametrize("kw,code", [
    (dict(head_dim=96), UNSUP),           # the reference dispatches only 128 (cu:252)
    (dict(head_dim=256), UNSUP),
    (dict(block_size=8), UNSUP),
    (dict(num_heads=30), INVALID),        # not a multiple of num_kv_heads
    (dict(num_kv_heads=0), INVALID),
    (dict(num_seqs=-1), INVALID),
    (dict(max_num_blocks_per_seq=-3), INVALID),
    (dict(query=0), INVALID),             # null pointer
    (dict(key_cache=FAKE + 2), INVALID),  # misaligned
    (dict(num_seqs=70000), UNSUP),
])
def test_decode_validation(kw, code):
    assert _v1(**kw) == code
    status, msg = _lib.last_error()
    assert status == code and msg


def test_void_launcher_reports_through_last_error():
    L = _lib.lib()
    L.launch_paged_attention_v1(FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, 0.1, 2, 32, 8, 96, 16, 4, None)
    assert L.swiftllm_hip_last_error() == UNSUP
    L.launch_reshape_and_cache(FAKE, FAKE, FAKE, FAKE, FAKE, 3, 0, 128, 16, None)
    assert L.swiftllm_hip_last_error() == INVALID


def test_v2_workspace_size_and_validation():
    L = _lib.lib()
    n = L.swiftllm_hip_paged_attention_v2_workspace_size(8, 64, 8, 128, 16, 2048, 512)
    # counters + max + sum (S*H*MP floats each) + partial outputs (S*H*MP*D floats)
    S, H, MP, D = 8, 64, 4, 128
    assert n >= S * H * MP * 4 * 2 + S * H * MP * D * 4
    assert L.swiftllm_hip_paged_attention_v2_workspace_size(8, 64, 8, 128, 16, 2048, 500) == 0
    rc = L.swiftllm_hip_launch_paged_attention_v2(FAKE, 0x100000, 16, FAKE, FAKE, FAKE, FAKE, FAKE,
                                                  0.1, 8, 64, 8, 128, 16, 2048, 512, 0, None)
    assert rc == INVALID  # workspace too small
    rc = L.swiftllm_hip_launch_paged_attention_v2(FAKE, 0x100000, n, FAKE, FAKE, FAKE, FAKE, FAKE,
                                                  0.1, 8, 64, 8, 128, 16, 2048, 24, 0, None)
    assert rc == INVALID  # partition not a multiple of 16


def test_v2_noalloc_validation_before_any_device_call():
    """The no-allocation split-K entry refuses bad shapes and sizes beyond its
    static scratch on the host, before it looks for a device."""
    L = _lib.lib()
    assert _lib.NOALLOC_SCRATCH_BYTES == 64 << 20
    # 256 x 64 heads x 4096 partitions of 16 tokens x 128 floats: ~34 GB
    rc = L.swiftllm_hip_launch_paged_attention_v2_noalloc(
        FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, 0.1, 256, 64, 8, 128, 16, 4096, 16, 0, None)
    assert rc == INVALID and "static scratch" in _lib.last_error()[1]
    rc = L.swiftllm_hip_launch_paged_attention_v2_noalloc(
        FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, 0.1, 8, 64, 8, 128, 16, 2048, 24, 0, None)
    assert rc == INVALID  # partition not a multiple of 16
    rc = L.swiftllm_hip_launch_paged_attention_v2_noalloc(
        FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, 0.1, 8, 64, 8, 96, 16, 2048, 512, 0, None)
    assert rc == UNSUP  # head_dim 96


def test_params_struct_twins_validate():
    p = pa.PagedAttentionParams(2, 32, 8, 96, 16, 0.1, 64)
    with pytest.raises(pa.NotSupported):
        pa.paged_attention_decode(FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, p)
    with pytest.raises(pa.InvalidParameter):
        pa.reshape_and_cache(FAKE, FAKE, FAKE, FAKE, FAKE, pa.ReshapeCacheParams(4, 0, 128, 16))


def test_moe_validation():
    L = _lib.lib()
    assert L.swiftllm_hip_moe_route(FAKE, 16, 8, 9, FAKE, FAKE, None) == UNSUP   # K > E
    assert L.swiftllm_hip_moe_route(FAKE, 16, 300, 2, FAKE, FAKE, None) == UNSUP  # E > 256
    assert L.swiftllm_hip_moe_route(FAKE, -1, 8, 2, FAKE, FAKE, None) == INVALID
    assert L.swiftllm_hip_moe_dispatch_workspace_size(4096, 8, 2) > 4096 * 2 * 4
    rc = L.swiftllm_hip_moe_dispatch(FAKE, FAKE, 4096, 2, 8, 4096, FAKE, FAKE, FAKE, FAKE, FAKE,
                                     0x100000, 64, None)
    assert rc == INVALID  # workspace too small


def test_expert_gemm_validation():
    """Shapes the grouped expert GEMM does not take are refused before any
    device work: n not a multiple of the tile's output columns (128 with w2,
    256 without), k not a multiple of 64 or above 2^21, E > 256."""
    L = _lib.lib()
    gemm = L.swiftllm_hip_moe_expert_gemm
    assert gemm(FAKE, FAKE, FAKE, FAKE, 8, 64, 14336 + 64, 4096, FAKE, None) == UNSUP
    assert gemm(FAKE, FAKE, None, FAKE, 8, 64, 4096 + 128, 4096, FAKE, None) == UNSUP
    assert gemm(FAKE, FAKE, None, FAKE, 8, 64, 4096, 4096 + 32, FAKE, None) == UNSUP
    assert gemm(FAKE, FAKE, None, FAKE, 8, 64, 4096, (1 << 21) + 64, FAKE, None) == UNSUP
    assert gemm(FAKE, FAKE, None, FAKE, 300, 64, 4096, 4096, FAKE, None) == UNSUP
    assert gemm(FAKE, FAKE, None, FAKE, 8, -1, 4096, 4096, FAKE, None) == INVALID
    assert gemm(FAKE, None, None, FAKE, 8, 64, 4096, 4096, FAKE, None) == INVALID


def test_prefill_validation():
    """Prefill arguments refused before any device work: head_dim other than
    64 / 128, heads not a multiple of kv heads, a negative length, a null
    pointer, and a max_context_len whose grid would need 2^21 or more
    workgroups per sequence (G = 4: 32 query tokens per workgroup)."""
    L = _lib.lib()

    def call(S=2, H=32, Hkv=8, D=128, max_len=64, q=FAKE):
        return L.swiftllm_hip_launch_paged_prefill(FAKE, q, FAKE, FAKE, FAKE, FAKE, 0.1, S, H,
                                                   Hkv, D, 16, max_len, 0, None)

    assert call(D=96) == UNSUP
    assert call(H=30) == INVALID
    assert call(max_len=-1) == INVALID
    assert call(q=None) == INVALID
    assert call(max_len=32 << 21) == UNSUP
    # Just under the limit passes validation (no sequences: nothing launches).
    assert call(S=0, max_len=(32 << 21) - 32) in (OK, NODEV)


@pytest.mark.skipif(_hip.device_count() > 0, reason="checks the no-device path")
def test_device_not_found_without_gpu():
    """Valid arguments on a host without a HIP device: DeviceNotFound, the
    behaviour of bindings.rs:72-75 when CUDA is absent."""
    assert _lib.lib().swiftllm_hip_device_check() == NODEV
    assert _v1() == NODEV
    with pytest.raises(pa.DeviceNotFound):
        pa.paged_attention_decode(FAKE, FAKE, FAKE, FAKE, FAKE, FAKE,
                                  pa.PagedAttentionParams(2, 32, 8, 128, 16, 0.1, 64))


def test_copy_blocks_dropin_argument_list():
    """launch_copy_blocks keeps the parameter list of paged_attention.cu:302-311."""
    text = HEADER.read_text()
    cb = re.search(r"void launch_copy_blocks\((.*?)\);", text, flags=re.S).group(1)
    params = [p.strip().split()[-1].lstrip("*") for p in cb.split(",")]
    assert params == ["block_mapping", "key_cache", "value_cache", "num_pairs", "num_kv_heads",
                      "head_dim", "block_size", "stream"]


def test_block_copy_validation():
    L = _lib.lib()
    # null cache list / null mapping / misaligned mapping / bad sizes
    assert L.swiftllm_hip_copy_blocks(None, None, FAKE, 2, 1, 8, 128, 16, None) == INVALID
    kc = (ctypes.c_void_p * 1)(FAKE)
    assert L.swiftllm_hip_copy_blocks(kc, kc, None, 2, 1, 8, 128, 16, None) == INVALID
    assert L.swiftllm_hip_launch_copy_blocks(FAKE + 4, FAKE, FAKE, 2, 8, 128, 16, 0, None) == INVALID
    assert L.swiftllm_hip_launch_copy_blocks(FAKE, FAKE, FAKE, 2, 0, 128, 16, 0, None) == INVALID
    assert L.swiftllm_hip_launch_copy_blocks(FAKE, FAKE, FAKE, -1, 8, 128, 16, 0, None) == INVALID
    assert L.swiftllm_hip_swap_blocks(FAKE, None, FAKE, 3, 4096, None) == INVALID
    assert L.swiftllm_hip_swap_blocks(FAKE, FAKE, FAKE, 3, 0, None) == INVALID
    L.launch_copy_blocks(FAKE, None, FAKE, 2, 8, 128, 16, None)
    assert L.swiftllm_hip_last_error() == INVALID


@pytest.mark.skipif(_hip.device_count() > 0, reason="checks the no-device path")
def test_block_copies_without_gpu():
    L = _lib.lib()
    kc = (ctypes.c_void_p * 1)(FAKE)
    assert L.swiftllm_hip_copy_blocks(kc, kc, FAKE, 2, 1, 8, 128, 16, None) == NODEV
    assert L.swiftllm_hip_swap_blocks(FAKE, FAKE, FAKE, 3, 4096, None) == NODEV
