"""Geometry: the oracle's maps against the reference's own record, and the GPU
kernels' folded addressing against those maps.

`plan_oracle.bin` is the reference's fixture (tests/data/plan_oracle.bin,
written by its tools/make_plan_oracle.py from torch.roll + window_partition,
nn.Unfold and calculate_mask); the checks follow tests/plan.rs:244-354.
"""
import os
import struct

import numpy as np
import pytest

import oracle
from conftest import GOLDEN

WIN = 16
GEOMETRIES = [(16, 16), (32, 32), (48, 48), (32, 48), (64, 64), (64, 32)]


def load_plan_oracle():
    """HATPLAN1 container (tests/plan.rs:169-206)."""
    b = open(os.path.join(GOLDEN, "plan_oracle.bin"), "rb").read()
    assert b[:8] == b"HATPLAN1"
    off = 8
    (count,) = struct.unpack_from("<I", b, off)
    off += 4
    out = {}
    for _ in range(count):
        (nl,) = struct.unpack_from("<I", b, off)
        off += 4
        name = b[off:off + nl].decode()
        off += nl
        assert b[off] == 1
        off += 1
        (rank,) = struct.unpack_from("<I", b, off)
        off += 4
        dims = struct.unpack_from("<" + "I" * rank, b, off)
        off += 4 * rank
        n = int(np.prod(dims))
        out[name] = np.frombuffer(b, dtype="<u4", count=n, offset=off).copy()
        off += 4 * n
    return out


@pytest.fixture(scope="module")
def po():
    return load_plan_oracle()


@pytest.mark.parametrize("h,w", GEOMETRIES)
def test_window_map_matches_torch_roll_and_partition(po, h, w):
    p = oracle.plan(h, w, WIN)
    for shift, name in ((0, "window_index_plain"), (p.shift, "window_index_shifted")):
        assert np.array_equal(oracle.window_index(p, shift), po[f"{h}x{w}/{name}"]), name


@pytest.mark.parametrize("h,w", GEOMETRIES)
def test_unfold_map_and_keep_match_nn_unfold(po, h, w):
    p = oracle.plan(h, w, WIN)
    idx, keep = oracle.unfold_index(p)
    want_keep = po[f"{h}x{w}/unfold_keep"]
    want_idx = po[f"{h}x{w}/unfold_index"]
    assert np.array_equal(keep.astype(np.uint32), want_keep)
    live = want_keep == 1
    assert live.any()
    assert np.array_equal(idx[live], want_idx[live])


def test_shift_mask_matches_calculate_mask(po):
    nonzero = 0
    for h, w in GEOMETRIES:
        p = oracle.plan(h, w, WIN)
        lab = po[f"{h}x{w}/mask_labels"].reshape(-1, WIN * WIN)
        want = np.where(lab[:, :, None] == lab[:, None, :], 0.0, -100.0).astype(np.float32)
        got = oracle.shift_mask(p).reshape(want.shape)
        assert np.array_equal(got, want), f"{h}x{w}"
        assert np.array_equal(oracle.mask_label(p), po[f"{h}x{w}/mask_labels"])
        nonzero += int((want != 0).sum())
    assert nonzero > 0


def test_plan_pads_to_the_next_window_multiple():
    """tests/plan.rs:305-331"""
    assert oracle.plan(48, 48).hp == 48
    p = oracle.plan(33, 17)
    assert (p.hp, p.wp) == (48, 32)
    p = oracle.plan(48, 48)
    assert (p.hp * p.wp, oracle.nw(p), p.win ** 2, p.owin ** 2, (p.owin - p.win) // 2) == (2304, 9, 256, 576, 4)
    r = oracle.plan(32, 48)
    assert (r.hp // 16, r.wp // 16, oracle.nw(r)) == (2, 3, 6)
    assert oracle.nw(oracle.plan(48, 32)) == 6


def test_rpi_known_answers():
    """tests/plan.rs:337-354"""
    sa = oracle.rpi_sa(WIN)
    assert sa.size == WIN ** 4
    assert sa[0] == (WIN - 1) * (2 * WIN - 1) + (WIN - 1)
    assert list(sa[:4]) == [480, 479, 478, 477]
    oca = oracle.rpi_oca(WIN, 24)
    assert oca.size == WIN * WIN * 576
    assert list(oca[:4]) == [1241, 1242, 1243, 1244]
    assert (oca < 1521).all()


# ---- the GPU kernels' folded addressing, against the reference's maps ----------

@pytest.mark.parametrize("h,w", GEOMETRIES)
def test_kernel_mask_shortcut_equals_calculate_mask(po, h, w):
    """hat_attn_sw_*: in a shifted block a score is masked iff (last window row
    and the y halves of query and key differ) or (last window column and the x
    halves differ). Checked against the reference's label grid."""
    lab = po[f"{h}x{w}/mask_labels"].reshape(-1, WIN * WIN)
    ny, nx = h // WIN, w // WIN
    t = np.arange(256)
    ty, tx = t // 16, t % 16
    for wi in range(ny * nx):
        wy, wx = divmod(wi, nx)
        want = lab[wi][:, None] != lab[wi][None, :]
        got = np.zeros((256, 256), dtype=bool)
        if wy == ny - 1:
            got |= ((ty[:, None] ^ ty[None, :]) & 8) != 0
        if wx == nx - 1:
            got |= ((tx[:, None] ^ tx[None, :]) & 8) != 0
        assert np.array_equal(got, want), f"{h}x{w} window {wi}"


def test_kernel_bias_addressing_equals_rpi():
    """hat_attn_sw_*: idx = (qy+15)*31 + qx+15 - (ky*31 + kx) is rpi_sa.
    hat_attn_oca_*: the table rotated by 880 rows and indexed by
    (ky*39 + kx) - (qy*39 + qx) + 600 selects rpi_oca's folded row."""
    q = np.arange(256)
    qy, qx = q // 16, q % 16
    k = np.arange(256)
    ky, kx = k // 16, k % 16
    sw = (qy[:, None] + 15) * 31 + qx[:, None] + 15 - (ky[None, :] * 31 + kx[None, :])
    assert np.array_equal(sw.reshape(-1), oracle.rpi_sa(16).astype(np.int64))
    k = np.arange(576)
    ky, kx = k // 24, k % 24
    j = (ky[None, :] * 39 + kx[None, :]) - (qy[:, None] * 39 + qx[:, None]) + 600
    assert j.min() >= 0 and j.max() <= 1520
    rot = (np.arange(1521) - 880) % 1521  # Tb[j] = table[(j - 880) mod 1521]
    assert np.array_equal(rot[j].reshape(-1), oracle.rpi_oca(16, 24).astype(np.int64))
