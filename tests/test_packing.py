"""CPU checks of the numpy model of the tile-packed activation layout (tests/_packing.py) and of
the library's size / routing functions for it."""
from __future__ import annotations

import numpy as np
import pytest

from _packing import pack_a, packed_elems, packed_index


@pytest.mark.parametrize("M,K", [(1, 8), (255, 40), (256, 32), (300, 136), (513, 72)])
def test_pack_a_places_every_element_and_zero_pads(M, K):
    y = (np.arange(M * K, dtype=np.float32).reshape(M, K) % 2000 + 1).astype(np.float16)
    p = pack_a(y)
    assert p.shape == (packed_elems(M, K),)
    idx = np.array([[packed_index(r, c, K) for c in range(K)] for r in range(M)])
    assert len(np.unique(idx)) == M * K                      # a bijection onto its image
    assert np.array_equal(p[idx], y)                         # every element where the formula says
    mask = np.ones(p.shape, dtype=bool)
    mask[idx.reshape(-1)] = False
    assert not p[mask].any()                                 # padding rows / columns are zero


def test_pack_a_block_is_the_stage_image():
    # Block (0, 0), chunk q*64 + i holds local row 16q + i//4; its four chunks permute the four
    # 8-column groups of that row by XOR with (row // 2) % 4.
    y = np.zeros((256, 32), dtype=np.float16)
    for r in range(256):
        for c in range(4):
            y[r, 8 * c:8 * c + 8] = r * 4 + c
    p = pack_a(y).reshape(1024, 8)
    for q in range(16):
        for i in range(64):
            r = 16 * q + i // 4
            c = (i % 4) ^ ((r // 2) % 4)
            assert (p[q * 64 + i] == r * 4 + c).all()


def test_library_packed_sizes_and_routing():
    from gtx16_fp16 import _clib

    lib = _clib.load()
    for M, K in [(1, 8), (300, 136), (4096, 4096), (65536, 768)]:
        assert lib.g16_packed_a_bytes(M, K) == 2 * packed_elems(M, K)
    assert lib.g16_packed_a_bytes(0, 64) == 0
    assert lib.g16_hgemm_use_packed(4096, 4096, 4096, 256) == 1
    assert lib.g16_hgemm_use_packed(65536, 3072, 768, 256) == 1
    assert lib.g16_hgemm_use_packed(64, 1024, 4096, 256) == 0     # split-K shape
    assert lib.g16_hgemm_use_packed(300, 264, 136, 256) == 0      # small: 128x128 tiles


def test_library_packed_weight_size():
    from gtx16_fp16 import _clib

    lib = _clib.load()
    for K, N in [(8, 8), (136, 264), (4096, 4096), (768, 3072)]:
        assert lib.g16_packed_b_bytes(K, N) == 2 * packed_elems(N, K)
    assert lib.g16_packed_b_bytes(0, 8) == 0
    assert lib.g16_pack_weight(None, None, 12, 8, None) == -1   # K % 8
