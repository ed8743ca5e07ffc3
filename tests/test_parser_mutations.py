"""The host parsers against mutated inputs: PNG images (hat_png_load), safetensors
checkpoints (hat_weights_open) and HATF fixtures (hat_verify's reader), each
mutated from a valid file with a fixed seed - truncations, appended bytes, byte
and bit flips, extreme 32-bit values written over header fields, and JSON
numbers of the checkpoint header replaced by negative, fractional, huge and
non-finite ones. Every call must return (a value or a HatError); a crash or
hang of the parser ends this test process. (These inputs were also run
against an AddressSanitizer + UBSan build of the host library.)"""
import json
import random
import struct

import numpy as np
import pytest

import hat_amd
from conftest import make_weights


def _mutate(rng, b):
    b = bytearray(b)
    k = rng.randrange(6)
    if k == 0 and len(b) > 1:
        return bytes(b[:rng.randrange(len(b))])
    if k == 1:
        return bytes(b) + bytes(rng.randrange(256) for _ in range(rng.randrange(1, 64)))
    for _ in range(rng.choice([1, 1, 2, 4, 16])):
        i = rng.randrange(len(b)) if rng.random() < 0.5 else rng.randrange(min(len(b), 256))
        if k == 2:
            b[i] = rng.randrange(256)
        elif k == 3:
            b[i] ^= 1 << rng.randrange(8)
        elif k == 4:
            b[i] = rng.choice([0, 0xff, 0x7f, 0x80])
        else:
            b[i:i + 4] = struct.pack("<I", rng.choice([0, 1, 0xffffffff, 0x7fffffff, 0x80000000, 65536, 1 << 24]))
    return bytes(b)


def test_png_loader_survives_mutations(tmp_path):
    rng = random.Random(11)
    srcs = []
    for w, h in [(13, 7), (1, 1), (64, 3)]:
        p = str(tmp_path / f"v{w}x{h}.png")
        hat_amd.png_save(p, np.random.default_rng(1).random((3, h, w), dtype=np.float32))
        srcs.append(open(p, "rb").read())
    loaded = 0
    m = str(tmp_path / "m.png")
    for _ in range(600):
        open(m, "wb").write(_mutate(rng, rng.choice(srcs)))
        try:
            img = hat_amd.png_load(m)
            assert img.ndim == 3 and img.shape[0] == 3 and np.isfinite(img).all()
            loaded += 1
        except hat_amd.HatError:
            pass
    # chunks are CRC-checked, so what still loads is mostly bytes appended after IEND
    assert 0 < loaded < 300


def test_checkpoint_loader_survives_mutations(weights_dir, tmp_path):
    rng = random.Random(12)
    src = open(make_weights(weights_dir, "hat-s", 2, 3, [1]), "rb").read()
    (hlen,) = struct.unpack("<Q", src[:8])
    hdr = json.loads(src[8:8 + hlen])
    names = [k for k in hdr if k != "__metadata__"]
    vals = [-1, -2**63, 0.5, 1e300, float("nan"), 2**53, 2**64, 2**32, 0, 1, 3, 144, 10**18]
    m = str(tmp_path / "m.safetensors")
    for it in range(300):
        if it % 2:
            h2 = json.loads(json.dumps(hdr))
            t = h2[rng.choice(names)]
            k = rng.randrange(4)
            if k == 0:
                t["shape"] = [rng.choice(vals) for _ in range(rng.randrange(0, 5))]
            elif k == 1:
                t["data_offsets"] = [rng.choice(vals), rng.choice(vals)]
            elif k == 2 and t["shape"]:
                t["shape"][rng.randrange(len(t["shape"]))] = rng.choice(vals)
            else:
                meta = h2["__metadata__"]
                meta[rng.choice(list(meta))] = rng.choice(["nan", "-1", "0", "1e300", "2000000000", "", "x"])
            hj = json.dumps(h2).encode()
            data = struct.pack("<Q", len(hj)) + hj + src[8 + hlen:]
        else:
            data = _mutate(rng, src[:8 + hlen]) + src[8 + hlen:]
        open(m, "wb").write(data)
        try:
            hat_amd.Weights(m)
        except hat_amd.HatError:
            pass


def test_fixture_reader_survives_mutations(weights_dir, tmp_path):
    """Header fields of a HATF fixture overwritten with extreme values: each is
    refused by the reader (or, on a machine without a GPU, by the backend after
    it), never used to size or copy a buffer it does not describe."""
    rng = random.Random(13)
    W = hat_amd.Weights(make_weights(weights_dir, "hat-s", 2, 3, [1]))
    h, w, s = 5, 6, 2
    fx = struct.pack("<4sIIIIIIII", b"HATF", 1, h, w, 3, s, 0, 0, 0) + \
        np.zeros(3 * h * w + 3 * h * s * w * s, np.float32).tobytes()
    extremes = [0, 1, 2, 3, 4, 6, 0xffffffff, 0x80000000, 0x55555556, 1 << 30, 0xaaaaaaab]
    m = str(tmp_path / "m.hatf")
    for _ in range(300):
        b = bytearray(fx)
        for _ in range(rng.choice([1, 2, 3])):
            f = rng.randrange(9)
            b[4 + 4 * f:8 + 4 * f] = struct.pack("<I", rng.choice(extremes))
        if rng.random() < 0.3:
            b = bytearray(_mutate(rng, bytes(b)))
        open(m, "wb").write(bytes(b))
        try:
            hat_amd.verify(W, m)
        except hat_amd.HatError:
            pass


def test_png_errors_quote_chunk_bytes_as_text(tmp_path):
    """A corrupt chunk's type bytes come from the file: the error names them
    with non-printable bytes escaped, so the message is valid text."""
    p = str(tmp_path / "v.png")
    hat_amd.png_save(p, np.zeros((3, 4, 5), dtype=np.float32))
    b = bytearray(open(p, "rb").read())
    i = b.index(b"IDAT")
    b[i:i + 2] = b"\xff\xfe"
    bad = str(tmp_path / "bad.png")
    open(bad, "wb").write(bytes(b))
    with pytest.raises(hat_amd.HatError) as e:
        hat_amd.png_load(bad)
    assert "\\xff\\xfeAT" in str(e.value)


@pytest.mark.parametrize("raw", [b"\xc9(", b"\\udc00"])
def test_checkpoint_header_strings_must_be_utf8(weights_dir, tmp_path, raw):
    """safetensors headers are UTF-8 JSON: a raw byte that starts no valid
    sequence, or a lone surrogate escape, is refused."""
    src = open(make_weights(weights_dir, "hat-s", 2, 3, [1]), "rb").read()
    (hlen,) = struct.unpack("<Q", src[:8])
    hj = src[8:8 + hlen].replace(b'"source":"', b'"source":"' + raw, 1)
    assert hj != src[8:8 + hlen]
    m = str(tmp_path / "u.safetensors")
    open(m, "wb").write(struct.pack("<Q", len(hj)) + hj + src[8 + hlen:])
    with pytest.raises(hat_amd.HatError) as e:
        hat_amd.Weights(m)
    assert "not UTF-8" in str(e.value)
