"""The C ABI without a GPU: the library loads and exports every declared entry
point, the kernel list matches the kernel sources and the built code object in
both directions (the reference's build.rs:99-122 check), and the host-side
logic - the checkpoint reader, its validation (weights.rs:133-265), the seeded
generator, the device/fixture error paths - behaves."""
import json
import os
import re
import struct
import subprocess

import numpy as np
import pytest

import hat_amd
import oracle
from conftest import GOLDEN, REPO, make_weights

PKG = os.path.join(REPO, "hat-rs_amd")


def test_library_exports_every_declared_symbol():
    L = hat_amd.lib()
    declared = hat_amd.declared_symbols()
    assert len(declared) >= 30
    missing = [s for s in declared if not hasattr(L, s)]
    assert not missing, missing
    out = subprocess.run(["nm", "-D", "--defined-only", hat_amd.LIB_PATH], capture_output=True,
                         text=True, check=True).stdout
    exported = set(re.findall(r" T (hat_[a-z0-9_]+)$", out, flags=re.M))
    assert set(declared) <= exported
    # no link-time dependency on the HIP runtime: it is dlopened
    ldd = subprocess.run(["readelf", "-d", hat_amd.LIB_PATH], capture_output=True, text=True).stdout
    assert "libamdhip64" not in ldd


def _kernel_sources():
    names = set()
    for fn in os.listdir(os.path.join(PKG, "csrc", "kernels")):
        if not fn.endswith(".hip"):
            continue
        src = open(os.path.join(PKG, "csrc", "kernels", fn)).read()
        names |= set(re.findall(r"^[A-Z_]+_INST\((\w+),", src, flags=re.M))
        names |= set(re.findall(r'extern "C" __global__[^\n]*?\bvoid (hat_\w+)\(', src))
    return names


def test_kernel_list_matches_sources_and_code_object():
    src = open(os.path.join(PKG, "csrc", "hip_rt.cpp")).read()
    block = src[src.index("required_kernels()"):src.index("return k;")]
    listed = set(re.findall(r'"(hat_\w+)"', block))
    in_src = _kernel_sources()
    assert listed == in_src, (listed ^ in_src)
    co = os.path.join(PKG, "build", "hat_kernels.co")
    out = subprocess.run(["nm", co], capture_output=True, text=True, check=True).stdout
    in_co = set(re.findall(r" T (hat_\w+)$", out, flags=re.M))
    assert listed == in_co, (listed ^ in_co)


def test_no_gpu_reports_unavailable_without_failing():
    if hat_amd.gpu_available():
        pytest.skip("a GPU is present")
    assert hat_amd.gpu_available() is False


def test_generator_is_deterministic_and_seeded(weights_dir):
    a = str(weights_dir / "det_a.safetensors")
    b = str(weights_dir / "det_b.safetensors")
    c = str(weights_dir / "det_c.safetensors")
    for p, s in ((a, 9), (b, 9), (c, 10)):
        hat_amd.generate_weights(p, "hat-s", 4, s, [1])
    assert open(a, "rb").read() == open(b, "rb").read()
    assert open(a, "rb").read() != open(c, "rb").read()


def test_weights_metadata_and_statistics(weights_dir):
    wp = make_weights(weights_dir, "hat-s", 4, 1, None)
    W = hat_amd.Weights(wp)
    assert (W.embed, W.heads, W.head_dim, W.depths, W.compressed, W.squeezed, W.head_feat) == \
        (144, 6, 24, [6] * 6, 6, 6, 64)
    assert (W.scale, W.window, W.owin, W.mlp_ratio) == (4, 16, 24, 2)
    assert abs(W.conv_scale - 0.01) < 1e-9 and W.img_range == 1.0
    assert np.allclose(W.mean, [0.4488, 0.4371, 0.4040])
    # README.md:58 counts 864 tensors for hat-s: 862 float tensors + 2 index buffers
    assert len(W.names()) == 864
    t = W.tensor("layers.0.residual_group.blocks.0.attn.qkv.weight")
    assert t.size == 432 * 144 and abs(t.std() - 0.02) < 1e-3 and abs(t.mean()) < 1e-3
    assert np.all(W.tensor("norm.weight") == 1.0) and np.all(W.tensor("norm.bias") == 0.0)
    # the int64 buffers: rpi_sa as is, rpi_oca with negatives folded = the oracle's maps
    assert np.array_equal(W.i64("relative_position_index_SA"), oracle.rpi_sa(16).astype(np.int64))
    raw = W.i64("relative_position_index_OCA")
    assert raw.min() == -880 and raw.max() == 640
    assert np.array_equal(raw % 1521, oracle.rpi_oca(16, 24).astype(np.int64))


@pytest.mark.parametrize("variant,embed,stages", [("hat", 180, 6), ("hat-l", 180, 12)])
def test_other_variants(weights_dir, variant, embed, stages):
    wp = str(weights_dir / f"{variant}_v.safetensors")
    hat_amd.generate_weights(wp, variant, 2, 4, [1] * stages)
    W = hat_amd.Weights(wp)
    assert (W.embed, W.head_dim, W.compressed, W.squeezed, len(W.depths)) == (embed, 30, 60, 6, stages)
    assert W.scale == 2


def _rewrite_header(src, dst, edit):
    b = open(src, "rb").read()
    (n,) = struct.unpack("<Q", b[:8])
    hdr = json.loads(b[8:8 + n])
    edit(hdr)
    hj = json.dumps(hdr, separators=(",", ":")).encode()
    hj += b" " * ((8 - (8 + len(hj)) % 8) % 8)
    open(dst, "wb").write(struct.pack("<Q", len(hj)) + hj + b[8 + n:])


def test_validation_rejects_bad_checkpoints(weights_dir):
    good = make_weights(weights_dir, "hat-s", 4, 2, [1])
    cases = {
        "no_meta": (lambda h: h["__metadata__"].pop("depths"), "depths"),
        "bad_shape": (lambda h: h["layers.0.conv.weight"].__setitem__("shape", [144, 144, 1, 9]),
                      "layers.0.conv.weight"),
        "missing": (lambda h: h.pop("layers.0.residual_group.blocks.0.norm2.bias"), "norm2.bias"),
        "bad_scale": (lambda h: h["__metadata__"].__setitem__("scale", "5"), "scale 5"),
        "bad_heads": (lambda h: h["__metadata__"].__setitem__("num_heads", "7"), "divisible"),
    }
    for name, (edit, needle) in cases.items():
        p = str(weights_dir / f"bad_{name}.safetensors")
        _rewrite_header(good, p, edit)
        with pytest.raises(hat_amd.HatError) as e:
            hat_amd.Weights(p)
        assert needle in str(e.value), (name, str(e.value))
    trunc = str(weights_dir / "bad_trunc.safetensors")
    open(trunc, "wb").write(open(good, "rb").read()[:1000])
    with pytest.raises(hat_amd.HatError):
        hat_amd.Weights(trunc)
    with pytest.raises(hat_amd.HatError):
        hat_amd.Weights(str(weights_dir / "does_not_exist.safetensors"))


def _entry(name, shape, nbytes=None):
    """An edit that gives tensor `name` this shape, its data starting where it
    did and spanning nbytes (default: unchanged)."""
    def edit(h):
        t = h[name]
        b = t["data_offsets"][0]
        t["shape"] = shape
        if nbytes is not None:
            t["data_offsets"] = [b, b + nbytes]
    return edit


@pytest.mark.parametrize("case,edit,needle", [
    # [2^32, 2^32] F32 is 2^66 bytes: with a 64-bit product it wraps to 0 and
    # an empty byte range would match it
    ("wrap", _entry("layers.0.conv.weight", [2**32, 2**32], 0), "larger than any file"),
    ("negative", _entry("layers.0.conv.weight", [-1, 144, 3, 3]), "not a count"),
    ("fraction", lambda h: h["layers.0.conv.bias"].__setitem__("data_offsets", [0.5, 576.5]), "not a count"),
    ("huge_depth", lambda h: h["__metadata__"].__setitem__("depths", "2000000000"), "bad entry"),
    ("many_stages", lambda h: h["__metadata__"].__setitem__("depths", ",".join(["1"] * 33)), "33 stages"),
    ("nan_overlap", lambda h: h["__metadata__"].__setitem__("overlap_ratio", "nan"), "out of range"),
    ("huge_embed", lambda h: h["__metadata__"].__setitem__("embed_dim", "1000000002"), "out of range"),
    ("rank0_head", _entry("conv_before_upsample.0.weight", [], 4), "conv_before_upsample.0.weight"),
])
def test_checkpoint_counts_and_ranges_are_checked_before_use(weights_dir, case, edit, needle):
    """Shapes and offsets are JSON numbers and the architecture comes from
    string metadata: values that would wrap a size, are not integers, would
    make the shape table unbounded, or leave a dimension to read that is not
    there are refused with an error, not used."""
    good = make_weights(weights_dir, "hat-s", 4, 2, [1])
    p = str(weights_dir / f"range_{case}.safetensors")
    _rewrite_header(good, p, edit)
    with pytest.raises(hat_amd.HatError) as e:
        hat_amd.Weights(p)
    assert needle in str(e.value), (case, str(e.value))


def test_backend_refuses_a_cpu_device(weights_dir):
    W = hat_amd.Weights(make_weights(weights_dir, "hat-s", 4, 2, [1]))
    with pytest.raises(hat_amd.HatError) as e:
        hat_amd.Backend(W, "cpu")
    assert "only `gpu`" in str(e.value)


def test_verify_rejects_bad_fixtures(weights_dir):
    W = hat_amd.Weights(make_weights(weights_dir, "hat-s", 4, 2, [1]))
    with pytest.raises(hat_amd.HatError):
        hat_amd.verify(W, str(weights_dir / "nope.bin"))
    bad = str(weights_dir / "bad.hatf")
    b = bytearray(open(os.path.join(GOLDEN, "hats_x4_d22_32x32.hatf"), "rb").read())
    b[:4] = b"XXXX"
    open(bad, "wb").write(bytes(b))
    with pytest.raises(hat_amd.HatError) as e:
        hat_amd.verify(W, bad)
    assert "HATF" in str(e.value)
    short = str(weights_dir / "short.hatf")
    open(short, "wb").write(open(os.path.join(GOLDEN, "hats_x4_d22_32x32.hatf"), "rb").read()[:-4])
    with pytest.raises(hat_amd.HatError) as e:
        hat_amd.verify(W, short)
    assert "bytes expected" in str(e.value)


def test_verify_rejects_a_fixture_that_is_not_rgb(weights_dir):
    """A HATF header with c != 3 is refused before anything is sized by it (the
    backend takes 3-channel input and returns 3-channel output)."""
    W = hat_amd.Weights(make_weights(weights_dir, "hat-s", 4, 2, [1]))
    h, w, scale, c = 16, 16, 4, 1
    one = str(weights_dir / "c1.hatf")
    with open(one, "wb") as f:
        f.write(struct.pack("<4sIIIIIIII", b"HATF", 1, h, w, c, scale, 16, 0, 0))
        f.write(np.zeros(h * w * c + h * scale * w * scale * c, dtype="<f4").tobytes())
    with pytest.raises(hat_amd.HatError) as e:
        hat_amd.verify(W, one)
    assert "3-channel" in str(e.value)


def test_verify_refuses_sides_whose_sizes_would_wrap(weights_dir):
    """A HATF header's sides are 32-bit: 2154230017 x 2854344542 at x4 makes
    3 h w wrap to 26 values and the output to 416 in 64-bit arithmetic, so a
    1804-byte file would match its own size check while the forward ran at the
    real sides. Sides above 2^20 are refused before anything is sized."""
    W = hat_amd.Weights(make_weights(weights_dir, "hat-s", 4, 2, [1]))
    h, w, scale, c = 2154230017, 2854344542, 4, 3
    assert (3 * h * w) % 2**64 == 26 and (3 * h * scale * w * scale) % 2**64 == 416
    wrap = str(weights_dir / "wrap.hatf")
    with open(wrap, "wb") as f:
        f.write(struct.pack("<4sIIIIIIII", b"HATF", 1, h, w, c, scale, 0, 0, 0))
        f.write(np.zeros(26 + 416, dtype="<f4").tobytes())
    assert os.path.getsize(wrap) == 1804
    with pytest.raises(hat_amd.HatError) as e:
        hat_amd.verify(W, wrap)
    assert "above 2^20" in str(e.value)


@pytest.mark.parametrize("shift", [-8, 1, 4, 7, 9, 16, 32])
def test_swmsa_refuses_a_shift_the_kernels_do_not_build(shift):
    """The attention kernels roll by the plan's half window or not at all; any
    other shift is an error raised before any device work."""
    c, hh, ww = 144, 32, 32
    x = np.zeros((hh * ww, c), dtype=np.float32)
    w = [np.zeros(s, dtype=np.float32) for s in ((3 * c, c), (3 * c,), (c, c), (c,), (961, 6))]
    with pytest.raises(hat_amd.HatError) as e:
        hat_amd.op_swmsa(x, hh, ww, c, 6, shift, *w)
    assert "shift" in str(e.value)


def test_ops_refuse_planes_past_their_int_token_counts():
    """The isolated ops count tokens in ints: a 16384 x 16384 plane (2^28
    tokens) is refused before any buffer is read, not overflowed."""
    L = hat_amd.lib()
    x = np.zeros(16, dtype=np.float32)
    p = hat_amd._fp(x)
    rc = L.hat_op_swmsa(p, p, 16384, 16384, 144, 6, 0, p, p, p, p, p, 1, None, None)
    assert rc == -1 and "too large" in hat_amd._err()
    rc = L.hat_op_ocab(p, p, 16384, 16384, 144, 6, 2, *([p] * 13), 1, None, None)
    assert rc == -1 and "too large" in hat_amd._err()


def _tamper_i64(src, dst, name, index, value):
    b = bytearray(open(src, "rb").read())
    (n,) = struct.unpack("<Q", b[:8])
    hdr = json.loads(b[8:8 + n])
    begin = hdr[name]["data_offsets"][0]
    struct.pack_into("<q", b, 8 + n + begin + 8 * index, value)
    open(dst, "wb").write(bytes(b))


@pytest.mark.parametrize("name,index,value,ok", [
    ("relative_position_index_SA", 1000, 0, False),
    ("relative_position_index_OCA", 5, 3, False),
    # the same entry plus a whole table: PyTorch's indexing and the reference's
    # rem_euclid fold (gpu.rs:59-62) read the same row, so this one is accepted
    ("relative_position_index_OCA", 0, -280 + 1521, True),
])
def test_loader_checks_the_index_buffers(weights_dir, name, index, value, ok):
    good = make_weights(weights_dir, "hat-s", 4, 2, [1])
    assert hat_amd.Weights(good).i64("relative_position_index_OCA")[0] == -280
    p = str(weights_dir / f"idx_{name}_{index}.safetensors")
    _tamper_i64(good, p, name, index, value)
    if ok:
        hat_amd.Weights(p)
        return
    with pytest.raises(hat_amd.HatError) as e:
        hat_amd.Weights(p)
    assert name in str(e.value) and "relative-position index" in str(e.value)
