"""The oracle against the golden vectors of the upstream network
(tests/golden/make_golden.py): whole forwards at three scales, two variants,
square, non-square and non-window-multiple inputs, and the isolated SW-MSA,
HAB and OCAB ops. The oracle keeps the reference CPU path's summation order,
and PyTorch's does not, so the bound is a few float32 ulps of the outputs.
"""
import os

import numpy as np
import pytest

import oracle
from conftest import (FWD_MEAN_TOL, FWD_TOL, GOLDEN, OCAB_NAMES, OP_TOL, X3_CHECKPOINT, make_weights,
                      op_input, read_hatf)


def _manifest():
    import json
    with open(os.path.join(GOLDEN, "golden.json")) as f:
        return json.load(f)


@pytest.mark.parametrize("fx", _manifest()["forward"], ids=lambda f: f["name"])
def test_oracle_forward_matches_upstream(weights_dir, fx):
    wp = make_weights(weights_dir, fx["variant"], fx["scale"], fx["weight_seed"], fx["depths"])
    h, w, scale, inp, exp = read_hatf(os.path.join(GOLDEN, fx["file"]))
    got = oracle.OracleModel(wp).forward(h, w, inp)
    assert got.shape == exp.shape
    d = np.abs(got - exp)
    assert d.max() < FWD_TOL and d.mean() < FWD_MEAN_TOL


@pytest.mark.parametrize("o", _manifest()["ops"], ids=lambda o: o["variant"])
def test_oracle_ops_match_upstream(weights_dir, o):
    wp = make_weights(weights_dir, o["variant"], 4, o["weight_seed"], o["depths"])
    M = oracle.OracleModel(wp)
    A = M.arrays
    hh, ww, c = o["h"], o["w"], o["c"]
    x = op_input(o["input_seed"], hh * ww, c)
    ref = np.load(os.path.join(GOLDEN, o["file"]))
    for blk, shift in ((0, 0), (1, 8)):
        p = f"layers.0.residual_group.blocks.{blk}.attn"
        got = oracle.swmsa_op(x, hh, ww, c, 6, shift, A[p + ".qkv.weight"], A[p + ".qkv.bias"],
                              A[p + ".proj.weight"], A[p + ".proj.bias"],
                              A[p + ".relative_position_bias_table"])
        assert np.abs(got - ref[f"swmsa_shift{shift}"]).max() < 2e-6
        if f"hab{blk}" in ref:
            assert np.abs(M.hab(x, hh, ww, 0, blk) - ref[f"hab{blk}"]).max() < 2e-6
    ws = [A["layers.0.residual_group.overlap_attn" + n] for n in OCAB_NAMES]
    assert np.abs(oracle.ocab_op(x, hh, ww, c, 6, 2, ws) - ref["ocab"]).max() < 2e-6


def test_oracle_detects_a_planted_mistake(weights_dir):
    """A checker that cannot fail pins nothing: with one block's qkv bias
    perturbed by 1e-3 (a smaller slip than any wrong index), the forward leaves
    the fixture's tolerance."""
    fx = _manifest()["forward"][0]
    wp = make_weights(weights_dir, fx["variant"], fx["scale"], fx["weight_seed"], fx["depths"])
    h, w, scale, inp, exp = read_hatf(os.path.join(GOLDEN, fx["file"]))
    M = oracle.OracleModel(wp)
    M.arrays["layers.0.residual_group.blocks.1.attn.qkv.bias"][:] += 1e-3
    assert np.abs(M.forward(h, w, inp) - exp).max() > 1e-5


# One deep block (stage 3, block 4) of the full-depth HAT-S fixture, slipped in
# ways a wrong kernel could slip: each must move the output past the bars the
# GPU's whole-forward tests use, or those tests could not see it.
PLANTS = {
    "zeroed SW bias table": ("layers.3.residual_group.blocks.4.attn.relative_position_bias_table",
                             lambda a: a * 0),
    "zeroed OCAB bias table": ("layers.3.residual_group.overlap_attn.relative_position_bias_table",
                               lambda a: a * 0),
    "dropped CAB conv2 weights": ("layers.3.residual_group.blocks.4.conv_block.cab.2.weight",
                                  lambda a: a * 0),
    "dropped CAB conv2 bias": ("layers.3.residual_group.blocks.4.conv_block.cab.2.bias", lambda a: a * 0),
    "qkv bias +1e-3": ("layers.3.residual_group.blocks.4.attn.qkv.bias", lambda a: a + 1e-3),
    "channel-attention gate shut": ("layers.3.residual_group.blocks.4.conv_block.cab.3.attention.3.bias",
                                    lambda a: a - 50),
}


@pytest.mark.parametrize("plant", sorted(PLANTS))
def test_forward_bars_see_a_slip_in_a_deep_block(weights_dir, plant):
    fx = next(f for f in _manifest()["forward"] if f["name"] == "hats_x4_full_32x48")
    wp = make_weights(weights_dir, fx["variant"], fx["scale"], fx["weight_seed"], fx["depths"])
    h, w, scale, inp, exp = read_hatf(os.path.join(GOLDEN, fx["file"]))
    M = oracle.OracleModel(wp)
    name, edit = PLANTS[plant]
    M.arrays[name][:] = edit(M.arrays[name])
    d = np.abs(M.forward(h, w, inp) - exp)
    print(f"{plant}: worst {d.max():.3e}, mean {d.mean():.3e}")
    # the mean bar alone catches every one of them
    assert d.mean() > FWD_MEAN_TOL


HAB_PLANTS = {
    "dropped CAB conv2 weights": ("conv_block.cab.2.weight", lambda a: a * 0),
    "dropped CAB conv2 bias": ("conv_block.cab.2.bias", lambda a: a * 0),
    "zeroed bias table": ("attn.relative_position_bias_table", lambda a: a * 0),
    "channel-attention gate shut": ("conv_block.cab.3.attention.3.bias", lambda a: a - 50),
}


@pytest.mark.parametrize("o", _manifest()["ops"], ids=lambda o: o["variant"])
@pytest.mark.parametrize("plant", sorted(HAB_PLANTS))
def test_hab_bar_sees_a_slip(weights_dir, o, plant):
    """The GPU's HAB op test compares whole blocks at OP_TOL: every slip in the
    CAB branch (scaled by conv_scale = 0.01 in the block's output) or the bias
    table moves that output by more than that, in both blocks."""
    wp = make_weights(weights_dir, o["variant"], 4, o["weight_seed"], o["depths"])
    hh, ww, c = o["h"], o["w"], o["c"]
    x = op_input(o["input_seed"], hh * ww, c)
    ref = np.load(os.path.join(GOLDEN, o["file"]))
    for blk in (0, 1):
        M = oracle.OracleModel(wp)
        name, edit = HAB_PLANTS[plant]
        k = f"layers.0.residual_group.blocks.{blk}." + name
        M.arrays[k][:] = edit(M.arrays[k])
        assert np.abs(M.hab(x, hh, ww, 0, blk) - ref[f"hab{blk}"]).max() > 5 * OP_TOL


def test_oracle_matches_the_reference_x3_fixture():
    """The reference's own whole-forward fixture (tests/data/hats_x3_48x48.bin,
    made by its tools/make_fixture.py from a torch-seeded HAT-S x3, recipe at
    tests/parity.rs:30-37), on the checkpoint rebuilt from that recipe."""
    assert os.path.exists(X3_CHECKPOINT), f"{X3_CHECKPOINT} is missing from the tree"
    h, w, scale, inp, exp = read_hatf(os.path.join(GOLDEN, "hats_x3_48x48.bin"))
    M = oracle.OracleModel(X3_CHECKPOINT)
    assert (M.scale, h, w) == (3, 48, 48)
    d = np.abs(M.forward(h, w, inp) - exp)
    print(f"oracle vs the reference's x3 fixture: worst {d.max():.3e}, mean {d.mean():.3e}")
    assert d.max() < FWD_TOL and d.mean() < FWD_MEAN_TOL
