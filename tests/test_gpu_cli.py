"""The rows around the path on the GPU: tiling (src/tile.rs, the reference's
tests/tiling.rs), multi-image batching, and the `hat` CLI end to end (PNG in,
PNG out, --verify, --cuda-selftest; src/main.rs)."""
import os
import subprocess

import numpy as np
import pytest

from conftest import GOLDEN, make_weights

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


def test_a_tile_that_covers_the_image_is_one_tile(small):
    """tests/tiling.rs:65-83: one tile reproduces the whole-image pass bit for bit."""
    _, W, be = small
    img = np.random.default_rng(1).random((3, 40, 56), dtype=np.float32)
    whole = be.forward(40, 56, img)
    for tile in (56, 64, 1000):
        got, info = be.tile_forward(40, 56, img, tile, 32)
        assert info["tiles"] == 1 and info["tile"] % 16 == 0
        assert np.array_equal(got, whole)


def test_a_covering_margin_is_exact_and_the_margin_bounds_the_seam(small):
    """tests/tiling.rs:86-144: a margin that reaches the image's edges from every
    core reproduces the whole image exactly; with less margin the seams differ,
    and more margin differs less."""
    _, W, be = small
    h, w = 64, 64
    img = np.random.default_rng(2).random((3, h, w), dtype=np.float32)
    whole = be.forward(h, w, img)
    got, info = be.tile_forward(h, w, img, 32, 64)
    assert info["tiles"] == 4 and info["largest_h"] == 64
    assert np.array_equal(got, whole)
    errs = []
    for margin in (0, 16):
        got, info = be.tile_forward(h, w, img, 32, margin)
        assert info["tiles"] == 4 and info["margin"] == margin
        errs.append(float(np.abs(got - whole).max()))
    _say(f"  seam worst |diff|: margin 0 {errs[0]:.3e}, margin 16 {errs[1]:.3e}")
    assert errs[0] > 0 and errs[1] < errs[0]


@pytest.mark.parametrize("n,h,w", [(5, 48, 32), (2, 16, 16), (9, 17, 23)])
def test_batch_equals_one_image_at_a_time(small, n, h, w):
    """forward_batch runs up to 4 images at once on separate streams with their
    own buffers: each result is bit-identical to that image's own forward."""
    _, W, be = small
    imgs = np.random.default_rng(n).random((n, 3, h, w), dtype=np.float32)
    got = be.forward_batch(n, h, w, imgs)
    for i in range(n):
        assert np.array_equal(got[i], be.forward(h, w, imgs[i])), i


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
    # --mem picks a tile; the run still writes an image of the right size
    r = _cli(hl, "-m", wp, "-i", src, "-o", dst, "--mem", "300")
    assert r.returncode == 0 and "--mem 300 MiB -> tile" in r.stdout
    assert hl.png_load(dst).shape == (3, 148, 180)


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
