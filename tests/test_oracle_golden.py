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
from conftest import GOLDEN, OCAB_NAMES, make_weights, op_input, read_hatf


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
    assert np.abs(got - exp).max() < 2e-6


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
