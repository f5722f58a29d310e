"""The CX_LAYOUT_TILE16 gate/up layout on the host side: tile16 / untile16
(constellation_amd/engine.py) against hand-computed byte positions and each
other.  The device side (the generator, the tiled upload and every gate/up
kernel) is checked against these in tests/test_gpu_layout.py."""
import numpy as np

from constellation_amd.engine import tile16, untile16


def test_roundtrip():
    a = np.random.default_rng(0).integers(0, 256, (48, 384), dtype=np.uint8)
    t = tile16(a)
    assert t.shape == a.shape and not np.array_equal(t, a)
    assert np.array_equal(untile16(t), a)


def test_known_positions():
    # 32 x 256: 2 row groups x 2 k-blocks, one 2 KB tile each, in row-group
    # then k-block order; inside a tile the 32 bytes of row r (mod 16),
    # columns 32q .. 32q + 31 (q = quarter of the k-block) at (16q + r) * 32
    cases = {(0, 0): 0, (0, 31): 31, (0, 32): 512, (1, 0): 32, (15, 127): 2047,
             (0, 128): 2048, (16, 0): 4096, (17, 130): 3 * 2048 + 32 + 2,
             (31, 255): 4 * 2048 - 1, (5, 100): 3 * 512 + 5 * 32 + 4}
    for (r, c), off in cases.items():
        a = np.zeros((32, 256), np.uint8)
        a[r, c] = 1
        assert np.flatnonzero(tile16(a)).tolist() == [off], (r, c)
