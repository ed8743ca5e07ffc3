"""Host-side checks of the rows around the path: PNG I/O (src/image.rs), the
tiling arithmetic (src/tile.rs), the memory plan (src/memguard.rs) and the
`hat` CLI's argument handling and exit codes (src/main.rs:182-195). No GPU.

PNG inputs are written here by an independent encoder (zlib + struct, with
every scanline filter and Adam7 interlacing), so the decoder is checked
against files it did not write."""
import os
import struct
import subprocess
import zlib

import numpy as np
import pytest

import hat_amd
from conftest import make_weights

ADAM7 = [(0, 0, 8, 8), (4, 0, 8, 8), (0, 4, 4, 8), (2, 0, 4, 4), (0, 2, 2, 4), (1, 0, 2, 2), (0, 1, 1, 2)]


def _chunk(t, d):
    return struct.pack(">I", len(d)) + t + d + struct.pack(">I", zlib.crc32(t + d) & 0xFFFFFFFF)


def _paeth(a, b, c):
    p = a + b - c
    pa, pb, pc = abs(p - a), abs(p - b), abs(p - c)
    return a if pa <= pb and pa <= pc else (b if pb <= pc else c)


def _filter_rows(rows, bpp):
    """Encode each row with filter (row index mod 5)."""
    out = b""
    prev = bytes(len(rows[0])) if rows else b""
    for y, row in enumerate(rows):
        ft = y % 5
        enc = bytearray()
        for i, v in enumerate(row):
            a = row[i - bpp] if i >= bpp else 0
            b = prev[i]
            c = prev[i - bpp] if i >= bpp else 0
            pred = [0, a, b, (a + b) // 2, _paeth(a, b, c)][ft]
            enc.append((v - pred) & 0xFF)
        out += bytes([ft]) + bytes(enc)
        prev = row
    return out


def write_png(path, pix, ctype, depth, interlace=False):
    """pix: uint array [h][w][channels] of the given depth."""
    h, w, ch = pix.shape
    bpp = ch * depth // 8
    dt = ">u2" if depth == 16 else "u1"

    def rows_of(sub):
        return [sub[y].astype(dt).tobytes() for y in range(sub.shape[0])]

    if interlace:
        raw = b""
        for x0, y0, dx, dy in ADAM7:
            sub = pix[y0::dy, x0::dx]
            if sub.shape[0] and sub.shape[1]:
                raw += _filter_rows(rows_of(sub), bpp)
    else:
        raw = _filter_rows(rows_of(pix), bpp)
    ihdr = struct.pack(">IIBBBBB", w, h, depth, ctype, 0, 0, 1 if interlace else 0)
    with open(path, "wb") as f:
        f.write(b"\x89PNG\r\n\x1a\n" + _chunk(b"IHDR", ihdr) + _chunk(b"tEXt", b"k\x00v")
                + _chunk(b"IDAT", zlib.compress(raw)) + _chunk(b"IEND", b""))


@pytest.mark.parametrize("ctype,ch", [(0, 1), (2, 3), (4, 2), (6, 4)])
@pytest.mark.parametrize("depth", [8, 16])
@pytest.mark.parametrize("interlace", [False, True])
def test_png_decode_matches_the_reference_rules(tmp_path, ctype, ch, depth, interlace):
    """image.rs:51-99: grey replicated to three planes, alpha dropped, samples
    over 255 or 65535."""
    rng = np.random.default_rng(ctype * 100 + depth + interlace)
    h, w = 13, 11
    top = 255 if depth == 8 else 65535
    pix = rng.integers(0, top + 1, size=(h, w, ch))
    p = str(tmp_path / "in.png")
    write_png(p, pix, ctype, depth, interlace)
    got = hat_amd.png_load(p)
    f = pix.astype(np.float32) * np.float32(1.0 / top)
    want = np.stack([f[..., 0]] * 3) if ch <= 2 else np.stack([f[..., 0], f[..., 1], f[..., 2]])
    assert got.shape == (3, h, w)
    assert np.array_equal(got, want)


def test_png_refuses_what_the_reference_refuses(tmp_path):
    p = str(tmp_path / "idx.png")
    write_png(p, np.zeros((4, 4, 1), dtype=np.int64), 3, 8)
    with pytest.raises(hat_amd.HatError) as e:
        hat_amd.png_load(p)
    assert "unsupported png colour type Indexed" in str(e.value)
    q = str(tmp_path / "crc.png")
    write_png(q, np.zeros((4, 4, 3), dtype=np.int64), 2, 8)
    b = bytearray(open(q, "rb").read())
    b[-20] ^= 0xFF  # inside the IDAT payload
    open(q, "wb").write(bytes(b))
    with pytest.raises(hat_amd.HatError) as e:
        hat_amd.png_load(q)
    assert "CRC" in str(e.value)
    with pytest.raises(hat_amd.HatError):
        hat_amd.png_load(str(tmp_path / "missing.png"))


def _read_png_rgb8(path):
    b = open(path, "rb").read()
    assert b[:8] == b"\x89PNG\r\n\x1a\n"
    off, idat, ihdr = 8, b"", None
    while off < len(b):
        n = struct.unpack(">I", b[off:off + 4])[0]
        t, d = b[off + 4:off + 8], b[off + 8:off + 8 + n]
        assert zlib.crc32(t + d) & 0xFFFFFFFF == struct.unpack(">I", b[off + 8 + n:off + 12 + n])[0]
        if t == b"IHDR":
            ihdr = struct.unpack(">IIBBBBB", d)
        elif t == b"IDAT":
            idat += d
        off += 12 + n
    w, h, depth, ctype, _, _, il = ihdr
    assert (depth, ctype, il) == (8, 2, 0)
    raw = zlib.decompress(idat)
    rows = [raw[y * (1 + 3 * w):(y + 1) * (1 + 3 * w)] for y in range(h)]
    assert all(r[0] == 0 for r in rows)
    return np.frombuffer(b"".join(r[1:] for r in rows), dtype=np.uint8).reshape(h, w, 3)


def test_png_encode_rounds_and_clamps_like_to_rgb8(tmp_path):
    """Image::to_rgb8 (image.rs:30-41): clamp to [0,1], x255, floor(v + 0.5),
    min 255 - so a NaN, whose clamp stays NaN, becomes 255."""
    rng = np.random.default_rng(3)
    x = rng.uniform(-0.2, 1.2, size=(3, 9, 14)).astype(np.float32)
    x[0, 0, :6] = [np.nan, -1.0, 0.5 / 255, 1.5 / 255, 254.5 / 255, np.inf]
    p = str(tmp_path / "out.png")
    hat_amd.png_save(p, x)
    got = _read_png_rgb8(p)
    v = np.clip(x, 0.0, 1.0) * np.float32(255.0)
    want = np.where(np.isnan(v), 255, np.minimum(np.floor(v + np.float32(0.5)), 255)).astype(np.uint8)
    assert np.array_equal(got, want.transpose(1, 2, 0))
    assert got[0, 0, 0] == 255 and got[0, 1, 0] == 0 and got[0, 5, 0] == 255
    # and the decoder reads back exactly k / 255
    assert np.array_equal(hat_amd.png_load(p), (got.transpose(2, 0, 1).astype(np.float32) * np.float32(1 / 255)))


def test_auto_tile_returns_a_window_multiple_that_fits_the_budget():
    """tile.rs:140-184 and the reference's tests/tiling.rs:146-206."""
    win, per_pixel, constant = 16, 300, 1 << 20
    assert hat_amd.auto_tile(1024, 1024, win, 32 << 20, 1 << 16, constant, 0) is None
    for budget in (64 << 20, 256 << 20, 1 << 30, 4 << 30):
        t = hat_amd.auto_tile(1024, 1024, win, budget, per_pixel, constant, 0)
        assert t % win == 0
        assert t * t * per_pixel * 4 + constant * 4 <= budget
        up = t + win
        assert up > 1024 or up * up * per_pixel * 4 + constant * 4 > budget
    assert hat_amd.auto_tile(1024, 1024, win, 64 << 30, per_pixel, constant, 0) == 1024
    assert hat_amd.auto_tile(64, 64, win, 64 << 30, per_pixel, constant, 0) == 64
    for margin in (16, 32):
        bare = hat_amd.auto_tile(1024, 1024, win, 1 << 30, per_pixel, constant, 0)
        t = hat_amd.auto_tile(1024, 1024, win, 1 << 30, per_pixel, constant, margin)
        sub = (t + 2 * margin) ** 2
        assert t % win == 0 and t <= bare
        assert sub * per_pixel * 4 + constant * 4 <= 1 << 30


def test_memory_plan_is_the_reference_formula(weights_dir):
    """memguard.rs:60-75: need = buffers * 1.05 + weights + 128 MiB; the
    buffers are this backend's own per-plan layout (host staging included), the
    weights what its upload allocates: the packed FP32 tensors and their
    split-bf16 copies, several times the 38.4 MiB HAT-S file (the reference
    uploads the file's tensors as they are, so it counts wt.bytes; the GPU test
    test_admission_counts_the_weights_the_upload_allocates holds this figure
    to what the upload allocated)."""
    W = hat_amd.Weights(make_weights(weights_dir, "hat-s", 4, 1, None))
    p = W.gpu_plan(512, 512)
    assert p["base"] == 128 << 20
    assert 3.0 * W.file_bytes() < p["weights"] < 5.0 * W.file_bytes()
    assert p["need"] == int(p["activations"] * 1.05) + p["weights"] + p["base"]
    # the 2.44 GiB a HAT-S 512 backend allocates (host staging included)
    assert abs(p["activations"] - 2.437 * 2**30) < 0.01 * 2**30
    q = W.gpu_plan(256, 256)
    assert 3.5 < p["activations"] / q["activations"] < 4.5
    if not hat_amd.gpu_available():
        assert p["have_avail"] == 0


def test_mem_budget_picks_the_tile_from_this_backends_plan(weights_dir):
    """The CLI's --mem rule (main.rs:268-274): auto_tile over the per-pixel cost,
    here the backend's per-plan device bytes over the padded pixels (the
    reference uses its CPU footprint; INTEGRATION.md records the difference).
    Pinned for the GPU CLI test's image and network: 45x37 under 100 MiB picks
    32 px cores, under 300 MiB the whole image."""
    W = hat_amd.Weights(make_weights(weights_dir, "hat-s", 4, 21, [2, 2]))
    per_pixel = W.gpu_plan(37, 45)["activations"] // 4 // (48 * 48)
    assert per_pixel == 2493
    assert hat_amd.auto_tile(37, 45, 16, 100 << 20, per_pixel, 0, 32) == 32
    assert hat_amd.auto_tile(37, 45, 16, 300 << 20, per_pixel, 0, 32) == 45
    assert hat_amd.auto_tile(37, 45, 16, 50 << 20, per_pixel, 0, 32) is None


def _cli(*args):
    return subprocess.run([hat_amd.CLI_PATH, *args], capture_output=True, text=True, timeout=120)


def test_cli_usage_and_exit_codes(weights_dir):
    r = _cli()
    assert r.returncode == 2 and "no model: -m is required" in r.stderr
    r = _cli("--bogus")
    assert r.returncode == 2 and "unknown argument `--bogus`" in r.stderr
    r = _cli("-m")
    assert r.returncode == 2 and "-m needs a value" in r.stderr
    r = _cli("-m", "x", "--tile", "abc")
    assert r.returncode == 2
    r = _cli("-h")
    assert r.returncode == 0 and "USAGE:" in r.stdout
    r = _cli("-m", "/nonexistent.safetensors", "--list-weights")
    assert r.returncode == 1 and r.stderr.startswith("hat: ")
    wp = make_weights(weights_dir, "hat-s", 4, 2, [1])
    r = _cli("-m", wp, "--list-weights")
    assert r.returncode == 0
    lines = r.stdout.splitlines()
    assert lines[0].startswith("hat ") and "hat-s (x4)" in lines[0]
    W = hat_amd.Weights(wp)
    assert len(lines) == 1 + len(W.names())
    assert "  conv_first.weight  [144, 3, 3, 3]" in lines
    r = _cli("-m", wp, "--device", "cpu", "-i", "a.png", "-o", "b.png")
    assert r.returncode == 1 and "has only `gpu`" in r.stderr
    r = _cli("-m", wp, "--device", "tpu", "-i", "a.png", "-o", "b.png")
    assert r.returncode == 1 and "device `tpu`" in r.stderr
    if not hat_amd.gpu_available():
        r = _cli("-m", wp, "-i", "a.png", "-o", "b.png")
        assert r.returncode == 1 and "no HIP device" in r.stderr
