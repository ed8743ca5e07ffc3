#!/usr/bin/env python3
"""Write compact oracle fixtures for the benchmark's full-size configurations.

    python3 tests/golden/make_large_parity.py [name ...]

The CPU oracle (oracle/, a C restatement of the reference's src/cpu.rs) takes
minutes per forward at these sizes, far too long for a test, so it is run once
here and a compact summary of its output is committed; the GPU test
(tests/test_gpu_large_parity.py) regenerates the same seeded weights and input,
runs the HIP path and compares against the summary:

  * ``idx`` / ``val``: 65 536 output values at flat indices drawn without
    replacement (the indices are stored, not regenerated), plus every value of
    the outermost output rows and columns of each channel (the padding, crop and
    border-tap paths);
  * ``block_sum``: float64 sums of every 64 x 64 block of each output channel,
    so an error anywhere in the image moves some block's sum;
  * ``chan_sum``: float64 sums of each output channel;
  * ``input_sha256`` / ``weights_sha256``: the test checks that it regenerated
    exactly the input and checkpoint used here.

Weights come from libhat's seeded generator (hat_weights_generate, host code
only, no GPU), the input from numpy's PCG64 at a fixed seed.
"""
import hashlib
import os
import sys
import tempfile
import time

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, os.path.join(REPO, "hat-rs_amd"))
sys.path.insert(0, os.path.join(REPO, "oracle"))

# name: (variant, scale, weight seed, input seed, h, w)
CONFIGS = {
    "hats_x4_512": ("hat-s", 4, 1, 512, 512, 512),
    "hat_x4_256": ("hat", 4, 4, 256, 256, 256),
    "hatl_x4_512": ("hat-l", 4, 5, 55, 512, 512),
}
N_SAMPLES = 65536
BLOCK = 64


def make_input(seed, h, w):
    return np.random.default_rng(seed).random((3, h, w), dtype=np.float32)


def sha256_file(path):
    hsh = hashlib.sha256()
    with open(path, "rb") as f:
        for chunk in iter(lambda: f.read(1 << 20), b""):
            hsh.update(chunk)
    return hsh.hexdigest()


def border_indices(oh, ow):
    """Flat indices of rows 0 and oh-1 and columns 0 and ow-1 of each channel."""
    out = []
    for c in range(3):
        base = c * oh * ow
        out.append(base + np.arange(ow))
        out.append(base + (oh - 1) * ow + np.arange(ow))
        out.append(base + np.arange(oh) * ow)
        out.append(base + np.arange(oh) * ow + (ow - 1))
    return np.unique(np.concatenate(out))


def summarise(y, seed):
    c, oh, ow = y.shape
    n = y.size
    rng = np.random.default_rng(seed)
    idx = np.union1d(rng.choice(n, size=N_SAMPLES, replace=False), border_indices(oh, ow))
    idx = idx.astype(np.uint32)
    flat = y.reshape(-1)
    yd = y.astype(np.float64)
    bs = yd.reshape(c, oh // BLOCK, BLOCK, ow // BLOCK, BLOCK).sum(axis=(2, 4))
    return dict(idx=idx, val=flat[idx].astype(np.float32), block_sum=bs,
                chan_sum=yd.sum(axis=(1, 2)))


def main():
    import hat_amd
    import oracle
    oracle.set_threads(os.cpu_count() or 8)
    names = sys.argv[1:] or list(CONFIGS)
    with tempfile.TemporaryDirectory() as td:
        for name in names:
            variant, scale, wseed, iseed, h, w = CONFIGS[name]
            wp = os.path.join(td, name + ".safetensors")
            hat_amd.generate_weights(wp, variant, scale, wseed, None)
            img = make_input(iseed, h, w)
            t0 = time.time()
            print(f"{name}: oracle forward {variant} x{scale} {h}x{w} on {oracle.threads()} threads",
                  flush=True)
            y = oracle.OracleModel(wp).forward(h, w, img)
            dt = time.time() - t0
            s = summarise(y, 1000 + iseed)
            out = os.path.join(HERE, f"large_{name}.npz")
            np.savez_compressed(
                out, variant=variant, scale=scale, weight_seed=wseed, input_seed=iseed, h=h, w=w,
                block=BLOCK, input_sha256=hashlib.sha256(img.tobytes()).hexdigest(),
                weights_sha256=sha256_file(wp), oracle_seconds=dt, **s)
            print(f"  {dt:.0f} s; wrote {out} ({os.path.getsize(out)} bytes, {s['idx'].size} values)",
                  flush=True)


if __name__ == "__main__":
    main()
