"""The rows around the path on the GPU: tiling (src/tile.rs, the reference's
tests/tiling.rs), multi-image batching, and the `hat` CLI end to end (PNG in,
PNG out, --verify, --cuda-selftest; src/main.rs)."""
import os
import subprocess

import numpy as np
import pytest

from conftest import FWD_MEAN_TOL, FWD_TOL, GOLDEN, make_weights

pytestmark = pytest.mark.gpu


def _say(msg):
    print(msg, flush=True)


@pytest.fixture(scope="module")
def hl():
    import hat_amd
    assert hat_amd.gpu_available(), "the HIP runtime or the GPU is missing"
    return hat_amd


@pytest.fixture(scope="module")
def small(hl, tmp_path_factory):
    wp = make_weights(tmp_path_factory.mktemp("cliw"), "hat-s", 4, 21, [2, 2])
    W = hl.Weights(wp)
    return wp, W, hl.Backend(W)


def test_admission_counts_the_weights_the_upload_allocates(small):
    """The memory plan's weights term is what the backend's upload allocated
    (packed tensors and split-bf16 copies), computed without a device."""
    wp, W, be = small
    assert be.weight_bytes() == W.gpu_plan(64, 64)["weights"] > 2 * W.file_bytes()


def test_a_tile_that_covers_the_image_is_one_tile(small):
    """tests/tiling.rs:65-83: one tile reproduces the whole-image pass bit for bit."""
    _, W, be = small
    img = np.random.default_rng(1).random((3, 40, 56), dtype=np.float32)
    whole = be.forward(40, 56, img)
    for tile in (56, 64, 1000):
        got, info = be.tile_forward(40, 56, img, tile, 32)
        assert info["tiles"] == 1 and info["tile"] % 16 == 0
        assert np.array_equal(got, whole)


def _fwd_ok(got, exp, what):
    d = np.abs(got - exp)
    _say(f"  {what}: worst {d.max():.3e}, mean {d.mean():.3e}")
    assert d.max() < FWD_TOL and d.mean() < FWD_MEAN_TOL, what


def test_a_covering_margin_is_exact_and_the_margin_bounds_the_seam(small):
    """tests/tiling.rs:86-144: a margin that reaches the image's edges from every
    core reproduces the whole image exactly; with less margin the seams differ,
    and more margin differs less. The seams themselves (margin 0 and 16, where
    the tiled output is not the whole pass) are held to the whole-forward bars
    against the oracle's tiled forward (tile.rs:50-107 geometry over the oracle's
    forward per sub-image), so a halo or core placement that differs from the
    reference's shows up."""
    import oracle
    wp, W, be = small
    h, w = 64, 64
    img = np.random.default_rng(2).random((3, h, w), dtype=np.float32)
    whole = be.forward(h, w, img)
    got, info = be.tile_forward(h, w, img, 32, 64)
    assert info["tiles"] == 4 and info["largest_h"] == 64
    assert np.array_equal(got, whole)
    M = oracle.OracleModel(wp)
    errs = []
    for margin in (0, 16):
        got, info = be.tile_forward(h, w, img, 32, margin)
        assert info["tiles"] == 4 and info["margin"] == margin
        exp, oinfo = oracle.tile_forward(M, h, w, img, 32, margin)
        assert (info["tiles"], info["tile"], info["margin"], info["largest_h"], info["largest_w"]) == oinfo
        _fwd_ok(got, exp, f"tiled margin {margin} vs the oracle's tiled forward")
        errs.append(float(np.abs(got - whole).max()))
    _say(f"  seam worst |diff| vs the whole pass: margin 0 {errs[0]:.3e}, margin 16 {errs[1]:.3e}")
    assert errs[0] > 1e-4 and errs[1] < errs[0]


def test_a_non_square_tiling_matches_the_oracle(small):
    """Ragged cores (the last row and column of tiles shorter than the step) on a
    non-square, non-window-multiple image, against the oracle's tiled forward."""
    import oracle
    wp, W, be = small
    h, w = 45, 70
    img = np.random.default_rng(6).random((3, h, w), dtype=np.float32)
    got, info = be.tile_forward(h, w, img, 20, 10)
    exp, oinfo = oracle.tile_forward(oracle.OracleModel(wp), h, w, img, 20, 10)
    assert (info["tiles"], info["tile"], info["margin"], info["largest_h"], info["largest_w"]) == oinfo
    # step round_up(20, 16) = 32, margin 16: 2 x 3 cores, the last ones 13 and 6 wide
    assert (info["tiles"], info["tile"], info["margin"]) == (6, 32, 16)
    _fwd_ok(got, exp, "45x70 tile 20 margin 10 vs the oracle")


@pytest.mark.parametrize("n,h,w", [(5, 48, 32), (2, 16, 16), (9, 17, 23)])
def test_batch_equals_one_image_at_a_time(small, n, h, w):
    """forward_batch runs up to 4 images at once on separate streams with their
    own buffers: each result is bit-identical to that image's own forward, and
    every image of the batch is held to the whole-forward bars against the
    oracle's forward of that image."""
    import oracle
    wp, W, be = small
    M = oracle.OracleModel(wp)
    imgs = np.random.default_rng(n).random((n, 3, h, w), dtype=np.float32)
    got = be.forward_batch(n, h, w, imgs)
    for i in range(n):
        assert np.array_equal(got[i], be.forward(h, w, imgs[i])), i
        _fwd_ok(got[i], M.forward(h, w, imgs[i]), f"batch image {i} of {n} ({h}x{w}) vs the oracle")


def _cli(hl, *args):
    r = subprocess.run([hl.CLI_PATH, *args], capture_output=True, text=True, timeout=300)
    _say(r.stdout + r.stderr)
    return r


def test_cli_upscales_a_png(hl, small, tmp_path):
    wp, W, be = small
    img = np.random.default_rng(3).random((3, 37, 45), dtype=np.float32)
    src = str(tmp_path / "in.png")
    hl.png_save(src, img)
    planes = hl.png_load(src)  # what the CLI sees: the 8-bit image
    dst = str(tmp_path / "out.png")
    r = _cli(hl, "-m", wp, "-i", src, "-o", dst)
    assert r.returncode == 0
    out = r.stdout.splitlines()
    assert out[1] == "  input  45x37 -> 180x148"
    assert "whole-image pass fits in free VRAM" in r.stdout
    assert any(l.startswith("  gpu forward in ") and l.endswith(" MP/s)") for l in out)
    assert out[-1] == f"  wrote {dst}"
    ref = str(tmp_path / "ref.png")
    hl.png_save(ref, be.forward(37, 45, planes))
    assert open(dst, "rb").read() == open(ref, "rb").read()
    # --mem picks a tile (the pick is pinned on the CPU by
    # test_mem_budget_picks_the_tile_from_this_backends_plan); the tiled line
    # names the largest sub-image as height x width, as main.rs:278-280 does
    r = _cli(hl, "-m", wp, "-i", src, "-o", dst, "--mem", "100")
    assert r.returncode == 0
    assert "  --mem 100 MiB -> tile 32px (margin 32)" in r.stdout.splitlines()
    assert "  tiled 45x37 into 4 tiles (32px cores, 32px margin, largest 37x45)" in r.stdout.splitlines()
    assert hl.png_load(dst).shape == (3, 148, 180)
    # the budget in bytes is main.rs:270's `as u64`, a saturating cast: NaN and
    # negative budgets hold no window, a huge one holds the whole image
    for m in ("nan", "-5"):
        r = _cli(hl, "-m", wp, "-i", src, "-o", dst, "--mem", m)
        assert r.returncode != 0 and "too small even for one window" in r.stderr, (m, r.stderr)
    r = _cli(hl, "-m", wp, "-i", src, "-o", dst, "--mem", "1e300")
    assert r.returncode == 0, r.stderr
    assert "  --mem 1e+300 MiB -> tile 45px (margin 32)" in r.stdout.splitlines()


def test_cli_verify_and_selftest(hl, tmp_path):
    import json
    with open(os.path.join(GOLDEN, "golden.json")) as f:
        fx = json.load(f)["forward"][0]
    wp = make_weights(tmp_path, fx["variant"], fx["scale"], fx["weight_seed"], fx["depths"])
    r = _cli(hl, "-m", wp, "--verify", os.path.join(GOLDEN, fx["file"]))
    assert r.returncode == 0 and "  verify worst |diff| " in r.stdout and r.stdout.rstrip().endswith("ok")
    other = next(f for f in json.load(open(os.path.join(GOLDEN, "golden.json")))["forward"]
                 if f["scale"] != fx["scale"])
    r = _cli(hl, "-m", wp, "--verify", os.path.join(GOLDEN, other["file"]))
    assert r.returncode == 1 and "hat: " in r.stderr
    r = _cli(hl, "--cuda-selftest")
    assert r.returncode == 0 and "  ok  " in r.stdout
