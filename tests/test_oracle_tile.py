"""The oracle's tiled forward (src/tile.rs:50-107, restated in oracle.tile_forward)
pinned by the properties the reference's own tiling tests assert
(tests/tiling.rs:65-144) on the oracle's whole forward, each shown to fail on a
planted mistake in the tile loop. The GPU's hat_tile_forward is compared with
this oracle in test_gpu_cli.py."""
import numpy as np
import pytest

import oracle
from conftest import make_weights


@pytest.fixture(scope="module")
def model(tmp_path_factory):
    # the same seeded network as the GPU tiling tests (HAT-S x4, two stages of two HABs)
    wp = make_weights(tmp_path_factory.mktemp("tilew"), "hat-s", 4, 21, [2, 2])
    return oracle.OracleModel(wp)


def _img(seed, h, w):
    return np.random.default_rng(seed).random((3, h, w), dtype=np.float32)


def test_one_tile_is_the_whole_pass(model):
    """tests/tiling.rs:65-83: a tile that covers the image runs one forward."""
    img = _img(1, 40, 56)
    whole = model.forward(40, 56, img)
    for tile in (56, 64, 1000):
        got, (tiles, step, _, lh, lw) = oracle.tile_forward(model, 40, 56, img, tile, 32)
        assert tiles == 1 and step % 16 == 0 and (lh, lw) == (40, 56)
        assert np.array_equal(got, whole)


@pytest.mark.parametrize("plant", [None, "origin"])
def test_a_covering_margin_is_exact(model, plant):
    """tests/tiling.rs:86-107: cores of one window with a margin wider than the
    image make every sub-image the whole image, so the assembly must be exact;
    copying each core from the sub-image's corner breaks it."""
    h = w = 32
    img = _img(2, h, w)
    whole = model.forward(h, w, img)
    got, (tiles, *_rest) = oracle.tile_forward(model, h, w, img, 16, 48, _plant=plant)
    assert tiles == 4
    if plant is None:
        assert np.array_equal(got, whole)
    else:
        assert np.abs(got - whole).max() > 1e-2


def test_the_margin_bounds_the_seam(model):
    """tests/tiling.rs:110-144: with no margin the seams differ visibly from the
    whole pass, and two windows of margin cut the error by an order of magnitude."""
    h = w = 64
    img = _img(3, h, w)
    whole = model.forward(h, w, img)
    rows = []
    for margin in (0, 16, 32, 64):
        got, (tiles, _, m, lh, lw) = oracle.tile_forward(model, h, w, img, 32, margin)
        assert tiles == 4 and m == margin and lh == lw == min(32 + margin, 64)
        d = np.abs(got - whole)
        rows.append((margin, d.max(), d.mean()))
        print(f"  margin {margin:2d}: worst {d.max():.3e}, mean {d.mean():.3e}")
    assert rows[0][1] > 1e-4
    assert rows[2][1] < rows[0][1] / 10
    assert rows[3][1] == 0.0  # 32 + 64 covers the 64-pixel image from every core


def test_an_unrounded_margin_is_not_the_reference_geometry(model):
    """tile.rs:65 rounds the margin up to the window; a margin of 8 kept as 8
    puts the sub-image's window grid off the whole image's and changes the
    output, which the rounded loop does not (it equals margin 16)."""
    h = w = 64
    img = _img(4, h, w)
    m16, _ = oracle.tile_forward(model, h, w, img, 32, 16)
    m8, info = oracle.tile_forward(model, h, w, img, 32, 8)
    assert info[2] == 16 and np.array_equal(m8, m16)
    bad, _ = oracle.tile_forward(model, h, w, img, 32, 8, _plant="unrounded")
    assert not np.array_equal(bad, m16)
