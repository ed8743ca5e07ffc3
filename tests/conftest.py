"""Shared test setup: import paths, the `gpu` marker, seeded weights."""
import json
import os
import struct
import sys

import numpy as np
import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
GOLDEN = os.path.join(REPO, "tests", "golden")
# Written by tests/golden/make_x3_checkpoint.py and committed as data: the
# checkpoint behind the reference's own x3 fixture (hats_x3_48x48.bin).
X3_CHECKPOINT = os.path.join(GOLDEN, "hats_x3_seed5.safetensors")
sys.path.insert(0, os.path.join(REPO, "hat-rs_amd"))
sys.path.insert(0, os.path.join(REPO, "oracle"))


# Parity bars.
# CONTRACT_TOL is the reference's own `--verify` bound: worst |diff| on the [0,1]
# image (src/main.rs:306-310). It is too loose to see a mistake deep in the
# trunk at the seeded N(0, 0.02) weights (a zeroed bias table of one block moves
# the HAT-S output by 3.4e-6), so the seeded whole-forward fixtures are held to
# FWD_TOL on the worst difference and FWD_MEAN_TOL on the mean difference, which
# tests/test_oracle_golden.py shows every planted single-block slip exceeds.
# OP_TOL bounds the isolated ops on N(0,1) inputs.
CONTRACT_TOL = 1e-4
FWD_TOL = 2e-6
FWD_MEAN_TOL = 1.5e-7
OP_TOL = 2e-5


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP path)")


@pytest.fixture(scope="session")
def golden_manifest():
    with open(os.path.join(GOLDEN, "golden.json")) as f:
        return json.load(f)


@pytest.fixture(scope="session")
def weights_dir(tmp_path_factory):
    return tmp_path_factory.mktemp("weights")


_made = {}


def make_weights(directory, variant, scale, seed, depths):
    """Regenerate a seeded checkpoint (the generator is deterministic)."""
    import hat_amd
    key = (variant, scale, seed, tuple(depths) if depths else None)
    if key not in _made:
        name = f"{variant}_x{scale}_s{seed}_d{'-'.join(map(str, depths or []))}.safetensors"
        path = os.path.join(str(directory), name)
        hat_amd.generate_weights(path, variant, scale, seed, depths)
        _made[key] = path
    return _made[key]


def read_hatf(path):
    """HATF v1 (src/fixture.rs:44-78)."""
    b = open(path, "rb").read()
    assert b[:4] == b"HATF"
    version, h, w, c, scale, win, flags = struct.unpack("<7I", b[4:32])
    assert version == 1 and flags == 0 and c == 3
    n_in = h * w * c
    inp = np.frombuffer(b[36:36 + 4 * n_in], dtype="<f4").reshape(3, h, w)
    out = np.frombuffer(b[36 + 4 * n_in:], dtype="<f4").reshape(3, h * scale, w * scale)
    return h, w, scale, inp, out


def op_input(seed, n, c):
    return np.random.default_rng(seed).standard_normal((n, c), dtype=np.float32)


OCAB_NAMES = (".norm1.weight", ".norm1.bias", ".qkv.weight", ".qkv.bias", ".proj.weight",
              ".proj.bias", ".relative_position_bias_table", ".norm2.weight", ".norm2.bias",
              ".mlp.fc1.weight", ".mlp.fc1.bias", ".mlp.fc2.weight", ".mlp.fc2.bias")
