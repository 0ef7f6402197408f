"""libswiftllm_ceilings.so (include/swiftllm_ceilings.h), the measurement
kernels bench.py times beside the path: it loads, exports every function
its header declares with the signatures the loader uses, and refuses bad
arguments on the host before any launch (no GPU needed)."""

import re
from pathlib import Path

from swiftllm_amd import ceilings

HEADER = Path(__file__).resolve().parents[1] / "include" / "swiftllm_ceilings.h"
FAKE = 0x1000  # never dereferenced: validation fails first


def _declared():
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    text = re.sub(r"^\s*#.*$", "", text, flags=re.M)
    return sorted(set(re.findall(r"\b(swiftllm_ceil_\w+)\s*\(", text)))


def test_exports_every_declared_function():
    L = ceilings.lib()
    names = _declared()
    assert len(names) == 5
    assert sorted(ceilings.SIGNATURES) == names
    assert all(hasattr(L, n) for n in names)


def test_argument_counts_match_header():
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    for name, (_, args) in ceilings.SIGNATURES.items():
        params = re.search(name + r"\s*\((.*?)\)\s*;", text, flags=re.S).group(1)
        assert len(params.split(",")) == len(args), name


def test_validation_before_launch():
    L = ceilings.lib()
    assert L.swiftllm_ceil_read_stream(FAKE + 8, 4096, FAKE, None) == -4          # misaligned
    assert L.swiftllm_ceil_read_stream(FAKE, 4095, FAKE, None) == -4              # not 16-byte sized
    assert L.swiftllm_ceil_tile_gather(FAKE, FAKE, FAKE, FAKE, 4, 2, 8, 96, 16, 0, 16, FAKE,
                                       None) == -6                                # head_dim 96
    assert L.swiftllm_ceil_tile_gather(FAKE, FAKE, FAKE, FAKE, 4, 2, 8, 128, 16, 0, 4, FAKE,
                                       None) == -6                                # 4-byte loads
    assert L.swiftllm_ceil_tile_gather(FAKE, FAKE, FAKE, FAKE, 4, -1, 8, 128, 16, 0, 16, FAKE,
                                       None) == -4                                # negative num_seqs
    assert L.swiftllm_ceil_cache_store(FAKE, FAKE, FAKE, 4, 8, 128, 0, 3, None) == -4  # mode 3
    assert L.swiftllm_ceil_row_copy(FAKE, FAKE, FAKE, 4, 2, 4000, 8, None) == -6  # hidden % 512
    assert L.swiftllm_ceil_mfma_stream(FAKE, 512, 4, 4, FAKE, None) == -4         # < one fragment
    assert L.swiftllm_ceil_mfma_stream(FAKE + 8, 4096, 4, 4, FAKE, None) == -4    # misaligned
    assert L.swiftllm_ceil_mfma_stream(FAKE, 4096, -1, 4, FAKE, None) == -4       # negative grid
    for fn, args in [(L.swiftllm_ceil_read_stream, (FAKE, 0, FAKE, None)),
                     (L.swiftllm_ceil_row_copy, (FAKE, FAKE, FAKE, 0, 2, 4096, 8, None)),
                     (L.swiftllm_ceil_mfma_stream, (FAKE, 4096, 0, 64, FAKE, None))]:
        assert fn(*args) == 0                                                     # nothing to do


def test_unit_order_longest_first_snake():
    order = ceilings.unit_order([5, 9, 7, 1], 2, cus=4)
    # longest first: seq 1, 2, 0, 3 -> units (1,0)(1,1)(2,0)(2,1) | (0,0)(0,1)(3,0)(3,1) reversed
    assert order.tolist() == [2, 3, 4, 5, 7, 6, 1, 0]


def test_gather_items_cover_every_block_once():
    """Single-pass items are whole (sequence, kv head) units; split-K items
    cut them into partitions; either way every valid block of every unit is
    read exactly once."""
    import numpy as np

    lens = [1, 16, 17, 700, 0, 4096]
    for P in (0, 512, 1024):
        items = ceilings.gather_items(lens, 4, P, cus=8)
        seen = {}
        for unit, b0, b1 in items.tolist():
            assert b1 > b0 or (b1 == b0 == 0)
            if P:
                assert b1 - b0 <= P // 16
            for b in range(b0, b1):
                seen[(unit, b)] = seen.get((unit, b), 0) + 1
        want = {(s * 4 + h, b) for s, L in enumerate(lens) for h in range(4) for b in range((L + 15) // 16)}
        assert set(seen) == want and set(seen.values()) == {1}
        if P:
            lengths = items[:, 2] - items[:, 1]
            assert np.all(np.diff(lengths) <= 0)   # longest first
