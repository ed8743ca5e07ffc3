"""The oracle's primitives against closed forms and library routines at tiny
shapes (numpy, float64), each chosen so a plausible slip - a transposed kernel,
a dropped bias, a wrong softmax axis, a backwards shuffle - fails."""
import math

import numpy as np
import pytest

import oracle

RNG = np.random.default_rng(1234)


def conv3x3_ref(x, w, b):
    ci, h, wd = x.shape
    co = w.shape[0]
    xp = np.pad(x.astype(np.float64), ((0, 0), (1, 1), (1, 1)))
    out = np.zeros((co, h, wd))
    for o in range(co):
        acc = np.full((h, wd), float(b[o]))
        for c in range(ci):
            for dy in range(3):
                for dx in range(3):
                    acc += xp[c, dy:dy + h, dx:dx + wd] * w[o, c, dy, dx]
        out[o] = acc
    return out


@pytest.mark.parametrize("ci,co,h,w", [(3, 5, 8, 16), (7, 4, 5, 7), (16, 3, 16, 24)])
def test_conv3x3_zero_padded(ci, co, h, w):
    x = RNG.standard_normal((ci, h, w)).astype(np.float32)
    wt = RNG.standard_normal((co, ci, 3, 3)).astype(np.float32)
    b = RNG.standard_normal(co).astype(np.float32)
    got = oracle.conv3x3(x, wt, b)
    want = conv3x3_ref(x, wt, b)
    assert np.abs(got - want).max() < 1e-4 * max(1.0, np.abs(want).max())
    # the kernel flipped (dy <-> dx): a plausible slip that must not pass
    bad = oracle.conv3x3(x, wt.transpose(0, 1, 3, 2).copy(), b)
    assert np.abs(bad - want).max() > 1e-2
    relu = oracle.conv3x3(x, wt, b, relu=True)
    assert np.array_equal(relu, np.maximum(got, 0))


def test_conv1x1_and_linear():
    x = RNG.standard_normal((9, 13)).astype(np.float32)
    w = RNG.standard_normal((5, 9)).astype(np.float32)
    b = RNG.standard_normal(5).astype(np.float32)
    assert np.allclose(oracle.conv1x1(x, w, b), w.astype(np.float64) @ x + b[:, None], atol=1e-5)
    xr = RNG.standard_normal((37, 20)).astype(np.float32)  # rows not a multiple of 8
    wr = RNG.standard_normal((11, 20)).astype(np.float32)  # outputs not a multiple of 8
    br = RNG.standard_normal(11).astype(np.float32)
    got = oracle.linear(xr, wr, br)
    assert np.allclose(got, xr.astype(np.float64) @ wr.T + br, atol=1e-5)
    # x W, not x W^T, would be wrong (square case so the shapes still fit)
    ws = RNG.standard_normal((20, 20)).astype(np.float32)
    assert np.abs(oracle.linear(xr, ws, np.zeros(20)) - xr @ ws).max() > 1e-2


def test_layer_norm_closed_form_and_invariants():
    x = (RNG.standard_normal((50, 144)) * 3 + 1).astype(np.float32)
    w = np.ones(144, np.float32)
    b = np.zeros(144, np.float32)
    y = oracle.layer_norm(x, w, b)
    assert np.abs(y.mean(1)).max() < 1e-5
    # biased variance with eps 1e-5: var(y) = var / (var + eps)
    v = x.astype(np.float64).var(1)
    assert np.allclose(y.astype(np.float64).var(1), v / (v + 1e-5), atol=1e-5)
    w2 = RNG.standard_normal(144).astype(np.float32)
    b2 = RNG.standard_normal(144).astype(np.float32)
    xd = x.astype(np.float64)
    want = (xd - xd.mean(1, keepdims=True)) / np.sqrt(xd.var(1, keepdims=True) + 1e-5) * w2 + b2
    assert np.abs(oracle.layer_norm(x, w2, b2) - want).max() < 1e-5


def test_erf_and_gelu_against_exact():
    worst = 0.0
    for v in np.linspace(-6, 6, 2401):
        worst = max(worst, abs(oracle.erf(v) - math.erf(v)))
    # A&S 7.1.26's bound is 1.5e-7 in exact arithmetic; evaluated in float32, as the
    # reference does (cpu.rs:597-603), 1 - poly*t*exp(-x^2) cancels near 0 and adds
    # a few ulps of 1.0.
    assert worst < 1.5e-7 + 3e-7
    for v in np.linspace(-8, 8, 801):
        exact = 0.5 * v * (1 + math.erf(v / math.sqrt(2)))
        assert abs(oracle.gelu(v) - exact) < 1e-6 * max(1.0, abs(v))
    # the tanh approximation differs by far more than the tolerance
    v = 1.5
    tanh = 0.5 * v * (1 + math.tanh(math.sqrt(2 / math.pi) * (v + 0.044715 * v ** 3)))
    assert abs(oracle.gelu(v) - tanh) > 1e-4


def attn_ref(q, k, v, bias, mask, nw, nq, nk, heads, d, scale):
    q = q.reshape(nw, nq, heads, d).astype(np.float64)
    k = k.reshape(nw, nk, heads, d).astype(np.float64)
    v = v.reshape(nw, nk, heads, d).astype(np.float64)
    s = np.einsum("wqhd,wkhd->whqk", q, k) * scale + bias[None]
    if mask is not None:
        s = s + mask[:, None]
    s = s - s.max(-1, keepdims=True)
    p = np.exp(s)
    p /= p.sum(-1, keepdims=True)
    return np.einsum("whqk,wkhd->wqhd", p, v).reshape(nw * nq, heads * d)


def test_window_attention_with_bias_and_mask():
    nw, win, heads, d = 2, 4, 3, 5
    nq = win * win
    q, k, v = (RNG.standard_normal((nw * nq, heads * d)).astype(np.float32) for _ in range(3))
    table = RNG.standard_normal(((2 * win - 1) ** 2, heads)).astype(np.float32)
    idx = np.zeros(nq * nq, np.uint32)
    for qi in range(nq):
        for ki in range(nq):
            idx[qi * nq + ki] = ((qi // win - ki // win + win - 1) * (2 * win - 1)
                                 + (qi % win - ki % win + win - 1))
    bias = table[idx.astype(np.int64)].reshape(nq, nq, heads).transpose(2, 0, 1)
    lab = RNG.integers(0, 3, (nw, nq))
    mask = np.where(lab[:, :, None] == lab[:, None, :], 0.0, -100.0).astype(np.float32)
    scale = d ** -0.5
    got = oracle.window_attention(q, k, v, idx, table, mask, nw, nq, heads, d, scale)
    want = attn_ref(q, k, v, bias, mask, nw, nq, nq, heads, d, scale)
    assert np.abs(got - want).max() < 1e-5
    nomask = oracle.window_attention(q, k, v, idx, table, None, nw, nq, heads, d, scale)
    assert np.abs(nomask - attn_ref(q, k, v, bias, None, nw, nq, nq, heads, d, scale)).max() < 1e-5
    # an all-(-100) row is a uniform softmax (finite mask): output = mean of v
    allmask = np.full((nw, nq, nq), -100.0, np.float32)
    u = oracle.window_attention(q, k, v, None, None, allmask, nw, nq, heads, d, 0.0)
    assert np.allclose(u.reshape(nw, nq, -1), v.reshape(nw, nq, -1).mean(1, keepdims=True), atol=1e-5)


def test_overlap_attention_more_keys_than_queries():
    nw, nq, nk, heads, d = 2, 9, 25, 2, 4
    q = RNG.standard_normal((nw * nq, heads * d)).astype(np.float32)
    k, v = (RNG.standard_normal((nw * nk, heads * d)).astype(np.float32) for _ in range(2))
    table = RNG.standard_normal((40, heads)).astype(np.float32)
    idx = RNG.integers(0, 40, nq * nk).astype(np.uint32)
    bias = table[idx.astype(np.int64)].reshape(nq, nk, heads).transpose(2, 0, 1)
    got = oracle.overlap_attention(q, k, v, idx, table, nw, nq, nk, heads, d, 0.5)
    assert np.abs(got - attn_ref(q, k, v, bias, None, nw, nq, nk, heads, d, 0.5)).max() < 1e-5


@pytest.mark.parametrize("r", [2, 3])
def test_pixel_shuffle_matches_depth_to_space(r):
    c, h, w = 3, 4, 5
    x = RNG.standard_normal((c * r * r, h, w)).astype(np.float32)
    # nn.PixelShuffle: (c, r, r, h, w) -> (c, h, r, w, r)
    want = x.reshape(c, r, r, h, w).transpose(0, 3, 1, 4, 2).reshape(c, h * r, w * r)
    assert np.array_equal(oracle.pixel_shuffle(x, r), want)
    # the subsampling axes swapped is a plausible, wrong variant
    bad = x.reshape(c, r, r, h, w).transpose(0, 3, 2, 4, 1).reshape(c, h * r, w * r)
    assert not np.array_equal(oracle.pixel_shuffle(x, r), bad)
