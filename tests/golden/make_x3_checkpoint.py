#!/usr/bin/env python3
"""Rebuild the checkpoint behind the reference's own x3 whole-forward fixture.

    python3 tests/golden/make_x3_checkpoint.py

The reference's `tests/data/hats_x3_48x48.bin` was made from a HAT-S x3 network
with torch-seeded random weights (the recipe at tests/parity.rs:30-37):

    make_fixture.py --config s --scale 3 --seed 5 --save-weights x3.pth
    convert.py x3.pth hat-s-x3.safetensors --variant hat-s
    make_fixture.py --model x3.pth --config s --scale 3 --h 48 --w 48 --seed 1 --out ...

This script runs the same recipe in this container only (it imports the
reference's upstream network, tools/hat_arch.py, which never travels to the GPU
box): torch.manual_seed(5), build HAT-S x3 exactly as make_fixture.py's `build`
does (tools/make_fixture.py:44-60), and write its state dict in convert.py's
format (tools/convert.py:120-250: float tensors as F32, the two relative-position
index buffers as I64, `.drop_path` and the patch_size-1 projection dropped, the
same __metadata__ keys). It then checks that

  * the fixture's input equals torch.rand(1, 3, 48, 48) from a generator seeded
    with 1 (make_fixture.py's input), bit for bit;
  * the rebuilt network reproduces the fixture's output (within 1e-5);

and only then writes

  * tests/golden/hats_x3_48x48.bin - the reference's fixture, copied unmodified
    (data: a HATF v1 input and expected output, fixture.rs:44-78);
  * tests/golden/hats_x3_seed5.safetensors - the 38 MB checkpoint, committed
    as data (random fp32 weights do not compress: gzip saves 14%), so that the
    tests that need it run on every checkout; its absence fails them.
"""
import os
import shutil
import struct
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
REF = "/root/reference"
FIXTURE = os.path.join(REF, "tests", "data", "hats_x3_48x48.bin")
OUT_FIXTURE = os.path.join(HERE, "hats_x3_48x48.bin")
OUT_CKPT = os.path.join(HERE, "hats_x3_seed5.safetensors")

sys.path.insert(0, os.path.join(REF, "tools"))
import timm_shim  # noqa: E402

timm_shim.install()
from hat_arch import HAT  # noqa: E402

# make_fixture.py's CONFIGS["s"] and COMMON (tools/make_fixture.py:44-58).
HAT_S = dict(depths=[6] * 6, embed_dim=144, num_heads=[6] * 6, mlp_ratio=2, compress_ratio=24,
             squeeze_factor=24)
COMMON = dict(in_chans=3, img_size=64, window_size=16, overlap_ratio=0.5, conv_scale=0.01,
              img_range=1., upsampler="pixelshuffle", resi_connection="1conv")


def read_hatf(path):
    b = open(path, "rb").read()
    magic, version, h, w, c, scale, win, flags, _ = struct.unpack("<4sIIIIIIII", b[:36])
    assert magic == b"HATF" and version == 1 and flags == 0 and c == 3
    n_in = h * w * c
    inp = np.frombuffer(b[36:36 + 4 * n_in], dtype="<f4").reshape(1, 3, h, w)
    out = np.frombuffer(b[36 + 4 * n_in:], dtype="<f4").reshape(1, 3, h * scale, w * scale)
    return h, w, scale, inp, out


def converted(sd):
    """convert.py's tensor selection (tools/convert.py:120-180)."""
    out = {}
    for k, v in sd.items():
        if k.startswith("relative_position_index"):
            out[k] = v.detach().numpy().astype(np.int64)
        elif v.is_floating_point():
            if k.endswith(".drop_path") or (k.startswith("patch_embed.")
                                            and not k.startswith("patch_embed.norm.")):
                continue
            out[k] = v.detach().to(torch.float32).contiguous().numpy()
    return out


def write_safetensors(path, tensors, metadata):
    from safetensors.numpy import save_file
    os.makedirs(os.path.dirname(path), exist_ok=True)
    save_file(dict(sorted(tensors.items())), path, metadata=metadata)


def main():
    torch.set_num_threads(8)
    torch.manual_seed(5)
    model = HAT(upscale=3, **HAT_S, **COMMON)
    model.eval()

    h, w, scale, inp, exp = read_hatf(FIXTURE)
    assert scale == 3 and (h, w) == (48, 48)
    x = torch.rand(1, 3, 48, 48, generator=torch.Generator().manual_seed(1))
    assert np.array_equal(x.numpy(), inp), "the fixture's input is not make_fixture.py's seed-1 input"
    with torch.no_grad():
        y = model(torch.from_numpy(inp.copy())).numpy()
    worst = float(np.abs(y - exp).max())
    print(f"rebuilt seed-5 HAT-S x3 vs {FIXTURE}: worst |diff| {worst:.3e}")
    assert worst < 1e-5, "the rebuilt network does not reproduce the reference's fixture"

    meta = {"variant": "hat-s", "scale": "3", "window_size": "16", "overlap_ratio": "0.5",
            "embed_dim": "144", "num_heads": "6", "mlp_ratio": "2",
            "depths": ",".join(str(d) for d in HAT_S["depths"]), "compress_ratio": "24",
            "squeeze_factor": "24", "conv_scale": "0.01", "img_range": "1.0",
            "rgb_mean": "0.4488,0.4371,0.4040", "source": "hats_x3_random.pth:params_ema",
            "format": "pt"}
    t = converted(model.state_dict())
    write_safetensors(OUT_CKPT, t, meta)
    shutil.copyfile(FIXTURE, OUT_FIXTURE)
    print(f"wrote {OUT_CKPT} ({os.path.getsize(OUT_CKPT)} bytes, {len(t)} tensors) and {OUT_FIXTURE}")


if __name__ == "__main__":
    main()
