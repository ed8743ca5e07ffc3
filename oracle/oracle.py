"""TEST INFRASTRUCTURE ONLY: ctypes wrapper of the CPU oracle (liboracle.so).

The oracle restates the reference CPU path (jacobsparts/hat-rs src/cpu.rs,
src/plan.rs, src/backend.rs) in C; see hat_oracle.h. Only tests/, the smoke()
entry of __graft_entry__.py and bench.py's cpu_baseline leg use it, as the
checker. Checkpoints are read with the `safetensors` package, independently of
the product's own reader.
"""
import ctypes as C
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")

_f32p = C.POINTER(C.c_float)
_u32p = C.POINTER(C.c_uint32)
_u8p = C.POINTER(C.c_uint8)


class Plan(C.Structure):
    _fields_ = [(n, C.c_int) for n in ("h", "w", "hp", "wp", "c", "win", "shift", "owin")]


class Model(C.Structure):
    _fields_ = [("scale", C.c_int), ("window", C.c_int), ("owin", C.c_int), ("embed", C.c_int),
                ("heads", C.c_int), ("head_dim", C.c_int), ("mlp_ratio", C.c_int),
                ("n_stages", C.c_int), ("depths", C.c_int * 32), ("compressed", C.c_int),
                ("squeezed", C.c_int), ("head_feat", C.c_int), ("conv_scale", C.c_float),
                ("img_range", C.c_float), ("mean", C.c_float * 3), ("n_tensors", C.c_int),
                ("names", C.POINTER(C.c_char_p)), ("data", C.POINTER(_f32p))]


_lib = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} missing: build it with `make -C oracle`")
        L = C.CDLL(LIB_PATH)
        L.or_erf.restype = C.c_float
        L.or_erf.argtypes = [C.c_float]
        L.or_gelu.restype = C.c_float
        L.or_gelu.argtypes = [C.c_float]
        L.or_get_threads.restype = C.c_int
        _lib = L
    return _lib


def f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


def fp(a):
    return a.ctypes.data_as(_f32p)


def set_threads(n):
    lib().or_set_threads(int(n))


def threads():
    return lib().or_get_threads()


# ---- geometry ---------------------------------------------------------------

def plan(h, w, win=16, c=4):
    p = Plan()
    lib().or_plan_new(C.byref(p), h, w, win, c)
    return p


def nw(p):
    return (p.hp // p.win) * (p.wp // p.win)


def window_index(p, shift):
    out = np.zeros(nw(p) * p.win * p.win, dtype=np.uint32)
    lib().or_window_index(C.byref(p), shift, out.ctypes.data_as(_u32p))
    return out


def unfold_index(p):
    n = nw(p) * p.owin * p.owin
    idx = np.zeros(n, dtype=np.uint32)
    keep = np.zeros(n, dtype=np.uint8)
    lib().or_unfold_index(C.byref(p), idx.ctypes.data_as(_u32p), keep.ctypes.data_as(_u8p))
    return idx, keep


def shift_mask(p):
    n = p.win * p.win
    out = np.zeros(nw(p) * n * n, dtype=np.float32)
    lib().or_shift_mask(C.byref(p), fp(out))
    return out


def mask_label(p):
    out = np.zeros(nw(p) * p.win * p.win, dtype=np.uint32)
    lib().or_mask_label(C.byref(p), out.ctypes.data_as(_u32p))
    return out


def rpi_sa(win=16):
    out = np.zeros(win ** 4, dtype=np.uint32)
    lib().or_rpi_sa(win, out.ctypes.data_as(_u32p))
    return out


def rpi_oca(win=16, owin=24):
    out = np.zeros(win * win * owin * owin, dtype=np.uint32)
    lib().or_rpi_oca(win, owin, out.ctypes.data_as(_u32p))
    return out


# ---- primitives ---------------------------------------------------------------

def conv3x3(x, w, b, relu=False):
    """x [ci][h][w], w [co][ci][3][3] -> [co][h][w]"""
    x, w, b = f32(x), f32(w), f32(b)
    ci, h, wd = x.shape
    co = w.shape[0]
    out = np.zeros((co, h, wd), dtype=np.float32)
    lib().or_conv3x3(fp(x), fp(out), fp(w), fp(b), ci, co, h, wd, int(relu))
    return out


def conv1x1(x, w, b):
    x, w, b = f32(x), f32(w), f32(b)
    ci, hw = x.shape
    co = w.shape[0]
    out = np.zeros((co, hw), dtype=np.float32)
    lib().or_conv1x1(fp(x), fp(out), fp(w), fp(b), ci, co, hw)
    return out


def linear(x, w, b):
    x, w, b = f32(x), f32(w), f32(b)
    rows, ci = x.shape
    co = w.shape[0]
    out = np.zeros((rows, co), dtype=np.float32)
    lib().or_linear(fp(x), fp(out), fp(w), fp(b), ci, co, C.c_long(rows))
    return out


def layer_norm(x, w, b, eps=1e-5):
    x = f32(x).copy()
    rows, c = x.shape
    lib().or_layer_norm(fp(x), fp(f32(w)), fp(f32(b)), c, C.c_long(rows), C.c_float(eps))
    return x


def erf(v):
    return lib().or_erf(float(v))


def gelu(v):
    return lib().or_gelu(float(v))


def pixel_shuffle(x, r):
    x = f32(x)
    cr, h, w = x.shape
    c = cr // (r * r)
    out = np.zeros((c, h * r, w * r), dtype=np.float32)
    lib().or_pixel_shuffle(fp(x), fp(out), c, h, w, r)
    return out


def window_attention(q, k, v, bias_idx, bias_tab, mask, nw_, nq, heads, d, scale):
    q, k, v = f32(q), f32(k), f32(v)
    out = np.zeros_like(q)
    bi = None if bias_idx is None else np.ascontiguousarray(bias_idx, dtype=np.uint32)
    bt = None if bias_tab is None else f32(bias_tab)
    mk = None if mask is None else f32(mask)
    lib().or_window_attention(fp(q), fp(k), fp(v), bi.ctypes.data_as(_u32p) if bi is not None else None,
                              fp(bt) if bt is not None else None, fp(mk) if mk is not None else None,
                              fp(out), nw_, nq, heads, d, C.c_float(scale), int(mk is not None))
    return out


def overlap_attention(q, k, v, bias_idx, bias_tab, nw_, nq, nk, heads, d, scale):
    q, k, v = f32(q), f32(k), f32(v)
    out = np.zeros_like(q)
    bi = np.ascontiguousarray(bias_idx, dtype=np.uint32)
    lib().or_overlap_attention(fp(q), fp(k), fp(v), bi.ctypes.data_as(_u32p), fp(f32(bias_tab)),
                               fp(out), nw_, nq, nk, heads, d, C.c_float(scale))
    return out


# ---- ops -------------------------------------------------------------------------

def swmsa_op(x, hp, wp, c, heads, shift, qkv_w, qkv_b, proj_w, proj_b, table, win=16):
    x = f32(x)
    out = np.zeros_like(x)
    a = [f32(t) for t in (qkv_w, qkv_b, proj_w, proj_b, table)]
    lib().or_swmsa_op(fp(x), fp(out), hp, wp, c, heads, win, shift, *[fp(t) for t in a])
    return out


def ocab_op(x, hp, wp, c, heads, mlp_ratio, ws, win=16, owin=24):
    """ws: norm1 w/b, qkv w/b, proj w/b, table, norm2 w/b, fc1 w/b, fc2 w/b."""
    x = f32(x)
    out = np.zeros_like(x)
    a = [f32(t) for t in ws]
    lib().or_ocab_op(fp(x), fp(out), hp, wp, c, heads, win, owin, mlp_ratio, *[fp(t) for t in a])
    return out


# ---- the whole model ---------------------------------------------------------------

class OracleModel:
    """The reference CPU forward over a converted checkpoint (safetensors)."""

    def __init__(self, path):
        from safetensors import safe_open
        from safetensors.numpy import load_file
        with safe_open(str(path), framework="numpy") as f:
            meta = f.metadata()
        tensors = load_file(str(path))
        self.arrays = {k: np.array(v, dtype=np.float32, copy=True)
                       for k, v in tensors.items() if v.dtype == np.float32}
        m = Model()
        self.scale = m.scale = int(meta["scale"])
        m.window = int(meta["window_size"])
        m.owin = m.window + int(m.window * float(meta["overlap_ratio"]))
        m.embed = int(meta["embed_dim"])
        m.heads = int(meta["num_heads"])
        m.head_dim = m.embed // m.heads
        m.mlp_ratio = int(meta["mlp_ratio"])
        depths = [int(d) for d in meta["depths"].split(",")]
        m.n_stages = len(depths)
        for i, d in enumerate(depths):
            m.depths[i] = d
        m.compressed = m.embed // int(meta["compress_ratio"])
        m.squeezed = m.embed // int(meta["squeeze_factor"])
        m.head_feat = self.arrays["conv_before_upsample.0.weight"].shape[0]
        m.conv_scale = float(meta["conv_scale"])
        m.img_range = float(meta["img_range"])
        for i, v in enumerate(meta["rgb_mean"].split(",")):
            m.mean[i] = float(v)
        names = list(self.arrays)
        self._names = (C.c_char_p * len(names))(*[n.encode() for n in names])
        self._data = (_f32p * len(names))(*[fp(self.arrays[n]) for n in names])
        m.n_tensors = len(names)
        m.names = self._names
        m.data = self._data
        self.m = m
        self.meta = meta

    def forward(self, h, w, img):
        img = f32(img).reshape(3, h, w)
        out = np.zeros((3, h * self.scale, w * self.scale), dtype=np.float32)
        rc = lib().or_forward(C.byref(self.m), h, w, fp(img), fp(out))
        if rc != 0:
            raise RuntimeError("oracle forward failed")
        return out

    def hab(self, x, hp, wp, stage, block):
        x = f32(x)
        out = np.zeros_like(x)
        lib().or_hab_op(C.byref(self.m), fp(x), fp(out), hp, wp, stage, block)
        return out


# ---- tiling -------------------------------------------------------------------------

def _round_up(v, to):
    return v if to == 0 else (v + to - 1) // to * to


def tile_forward(model, h, w, img, tile, margin, win=16, _plant=None):
    """tile::forward (src/tile.rs:50-107) over the oracle's whole forward.

    Cores of `tile` input pixels rounded up to the window, a halo of `margin`
    rounded up to the window and clamped to the image (tile.rs:62-66, 80-87),
    one forward per sub-image, and only each core copied back, at its own
    position scaled by the model (tile.rs:90-100); no blending. Returns the
    [3][h*s][w*s] image and (tiles, step, margin, largest_h, largest_w).
    `_plant` is for the tests that show the tiling checks can fail:
    "origin" copies each core from the sub-image's corner instead of its own
    offset, "unrounded" keeps the margin as given.
    """
    img = f32(img).reshape(3, h, w)
    s = model.scale
    step = max(_round_up(tile, win), win)
    margin = margin if _plant == "unrounded" else _round_up(margin, win)
    out = np.zeros((3, h * s, w * s), dtype=np.float32)
    tiles = largest_h = largest_w = 0
    for ty in range(-(-h // step)):
        for tx in range(-(-w // step)):
            y0, x0 = ty * step, tx * step
            y1, x1 = min(y0 + step, h), min(x0 + step, w)
            sy0, sx0 = max(y0 - margin, 0), max(x0 - margin, 0)
            sy1, sx1 = min(y1 + margin, h), min(x1 + margin, w)
            sh, sw = sy1 - sy0, sx1 - sx0
            largest_h, largest_w = max(largest_h, sh), max(largest_w, sw)
            planes = model.forward(sh, sw, img[:, sy0:sy1, sx0:sx1])
            dy0, dx0 = (0, 0) if _plant == "origin" else ((y0 - sy0) * s, (x0 - sx0) * s)
            ch, cw = (y1 - y0) * s, (x1 - x0) * s
            out[:, y0 * s:y0 * s + ch, x0 * s:x0 * s + cw] = planes[:, dy0:dy0 + ch, dx0:dx0 + cw]
            tiles += 1
    return out, (tiles, step, margin, largest_h, largest_w)
