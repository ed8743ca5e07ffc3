"""ctypes binding of libhat.so (include/hat.h) for the tests and the benchmark.

The product is the C ABI; this module only marshals numpy arrays across it.
It mirrors the reference's host interface: `Weights.load` (src/weights.rs:60),
`Backend.name` / `Backend.forward` (src/backend.rs:29-36), `verify`
(src/main.rs:312-326) and `selftest` (src/selftest.rs:437-523).

There is no CPU fallback: `Backend("gpu")` fails loudly when the library or a
device is missing.
"""
import ctypes as C
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "build", "libhat.so")
HEADER = os.path.join(os.path.dirname(HERE), "include", "hat.h")

_f32p = C.POINTER(C.c_float)


class HatError(RuntimeError):
    pass


class ModelInfo(C.Structure):
    _fields_ = [("scale", C.c_int), ("window", C.c_int), ("owin", C.c_int), ("embed", C.c_int),
                ("heads", C.c_int), ("head_dim", C.c_int), ("mlp_ratio", C.c_int),
                ("n_stages", C.c_int), ("depths", C.c_int * 32), ("compressed", C.c_int),
                ("squeezed", C.c_int), ("head_feat", C.c_int), ("conv_scale", C.c_float),
                ("img_range", C.c_float), ("mean", C.c_float * 3)]


class Tiling(C.Structure):
    _fields_ = [(n, C.c_size_t) for n in ("tile", "margin", "scale", "tiles", "largest_h", "largest_w")]


class MemPlan(C.Structure):
    _fields_ = [(n, C.c_ulonglong) for n in ("activations", "weights", "base", "need", "avail")] + \
               [("have_avail", C.c_int)]


_lib = None


def lib():
    """Load libhat.so (built by __graft_entry__.build / `make -C hat-rs_amd`)."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise HatError(f"{LIB_PATH} is missing: build it with `make -C hat-rs_amd`")
    L = C.CDLL(LIB_PATH)
    sig = {
        "hat_version": (C.c_char_p, []),
        "hat_last_error": (C.c_char_p, []),
        "hat_weights_open": (C.c_void_p, [C.c_char_p]),
        "hat_weights_close": (None, [C.c_void_p]),
        "hat_weights_info": (C.c_int, [C.c_void_p, C.POINTER(ModelInfo)]),
        "hat_weights_count": (C.c_int, [C.c_void_p]),
        "hat_weights_name": (C.c_char_p, [C.c_void_p, C.c_int]),
        "hat_weights_tensor": (_f32p, [C.c_void_p, C.c_char_p, C.POINTER(C.c_size_t)]),
        "hat_weights_index_i64": (C.c_long, [C.c_void_p, C.c_char_p, C.POINTER(C.c_longlong), C.c_size_t]),
        "hat_weights_generate": (C.c_int, [C.c_char_p, C.c_char_p, C.c_int, C.c_ulonglong,
                                           C.POINTER(C.c_int), C.c_int]),
        "hat_weights_variant": (C.c_char_p, [C.c_void_p]),
        "hat_weights_file_bytes": (C.c_ulonglong, [C.c_void_p]),
        "hat_weights_shape": (C.c_int, [C.c_void_p, C.c_char_p, C.POINTER(C.c_size_t), C.c_int]),
        "hat_backend_forward_batch": (C.c_int, [C.c_void_p, C.c_size_t, C.c_size_t, C.c_size_t, _f32p, _f32p]),
        "hat_tile_forward": (C.c_int, [C.c_void_p, C.c_size_t, C.c_size_t, _f32p, _f32p, C.c_size_t, C.c_size_t,
                                       C.POINTER(Tiling)]),
        "hat_auto_tile": (C.c_size_t, [C.c_size_t, C.c_size_t, C.c_size_t, C.c_ulonglong, C.c_ulonglong,
                                       C.c_ulonglong, C.c_size_t]),
        "hat_gpu_plan": (C.c_int, [C.c_void_p, C.c_size_t, C.c_size_t, C.POINTER(MemPlan)]),
        "hat_gpu_auto_tile": (C.c_long, [C.c_void_p, C.c_size_t, C.c_size_t]),
        "hat_png_load": (C.c_int, [C.c_char_p, C.POINTER(C.c_size_t), C.POINTER(C.c_size_t), _f32p, C.c_size_t]),
        "hat_png_save": (C.c_int, [C.c_char_p, C.c_size_t, C.c_size_t, _f32p]),
        "hat_gpu_available": (C.c_int, []),
        "hat_backend_new": (C.c_void_p, [C.c_void_p, C.c_char_p]),
        "hat_backend_name": (C.c_char_p, [C.c_void_p]),
        "hat_backend_forward": (C.c_int, [C.c_void_p, C.c_size_t, C.c_size_t, _f32p, _f32p]),
        "hat_backend_forward_device": (C.c_int, [C.c_void_p, C.c_size_t, C.c_size_t, C.c_void_p,
                                                 C.c_void_p]),
        "hat_backend_synchronize": (C.c_int, [C.c_void_p]),
        "hat_backend_forward_noalloc": (C.c_int, [C.c_void_p, C.c_size_t, C.c_size_t, C.c_void_p,
                                                  C.c_void_p]),
        "hat_backend_hab": (C.c_int, [C.c_void_p, C.c_int, C.c_int, C.c_size_t, C.c_size_t, _f32p, _f32p,
                                      C.c_int, _f32p]),
        "hat_backend_acts_bytes": (C.c_size_t, [C.c_void_p]),
        "hat_backend_weight_bytes": (C.c_size_t, [C.c_void_p]),
        "hat_backend_free": (None, [C.c_void_p]),
        "hat_verify": (C.c_int, [C.c_void_p, C.c_char_p, C.c_char_p]),
        "hat_gpu_selftest": (C.c_int, []),
        "hat_op_swmsa": (C.c_int, [_f32p, _f32p, C.c_int, C.c_int, C.c_int, C.c_int, C.c_int,
                                   _f32p, _f32p, _f32p, _f32p, _f32p, C.c_int, _f32p, _f32p]),
        "hat_op_ocab": (C.c_int, [_f32p, _f32p, C.c_int, C.c_int, C.c_int, C.c_int, C.c_int]
                        + [_f32p] * 13 + [C.c_int, _f32p, _f32p]),
        "hat_device_alloc": (C.c_void_p, [C.c_size_t]),
        "hat_device_free": (C.c_int, [C.c_void_p]),
        "hat_memcpy_h2d": (C.c_int, [C.c_void_p, C.c_void_p, C.c_size_t]),
        "hat_memcpy_d2h": (C.c_int, [C.c_void_p, C.c_void_p, C.c_size_t]),
        "hat_device_copy": (C.c_int, [C.c_void_p, C.c_void_p, C.c_size_t]),
        "hat_device_synchronize": (C.c_int, []),
        "hat_device_mem_info": (C.c_int, [C.POINTER(C.c_size_t), C.POINTER(C.c_size_t)]),
        "hat_device_name": (C.c_char_p, []),
        "hat_device_cu_count": (C.c_int, []),
        "hat_profile_begin": (C.c_int, []),
        "hat_profile_end": (C.c_int, []),
        "hat_profile_count": (C.c_int, []),
        "hat_profile_get": (C.c_int, [C.c_int, C.c_char_p, C.c_int, C.POINTER(C.c_long),
                                      C.POINTER(C.c_double)]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(L, name)
        fn.restype = res
        fn.argtypes = args
    _lib = L
    return L


def _err():
    # messages can quote names read from a file: never fail on their bytes
    return lib().hat_last_error().decode(errors="replace")


def _check(rc, what):
    if rc is None or (isinstance(rc, int) and rc < 0):
        raise HatError(f"{what}: {_err()}")
    return rc


def _fp(a):
    return a.ctypes.data_as(_f32p) if a is not None else None


def f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


def declared_symbols():
    """Every function name include/hat.h declares."""
    import re
    src = open(HEADER).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    return sorted(set(re.findall(r"\b(hat_[a-z0-9_]+)\s*\(", src)))


# ---------------------------------------------------------------------------

def generate_weights(path, variant="hat-s", scale=4, seed=0, depths=None):
    d = None
    n = 0
    if depths is not None:
        n = len(depths)
        d = (C.c_int * n)(*depths)
    _check(lib().hat_weights_generate(str(path).encode(), variant.encode(), scale, seed, d, n),
           "hat_weights_generate")
    return path


class Weights:
    """Weights::load (src/weights.rs:60)."""

    def __init__(self, path):
        self.path = str(path)
        h = lib().hat_weights_open(self.path.encode())
        if not h:
            raise HatError(_err())
        self.h = h
        info = ModelInfo()
        _check(lib().hat_weights_info(h, C.byref(info)), "hat_weights_info")
        self.info = info
        self.scale = info.scale
        self.window = info.window
        self.owin = info.owin
        self.embed = info.embed
        self.heads = info.heads
        self.head_dim = info.head_dim
        self.mlp_ratio = info.mlp_ratio
        self.depths = [info.depths[i] for i in range(info.n_stages)]
        self.compressed = info.compressed
        self.squeezed = info.squeezed
        self.head_feat = info.head_feat
        self.conv_scale = info.conv_scale
        self.img_range = info.img_range
        self.mean = [info.mean[i] for i in range(3)]

    def variant(self):
        return lib().hat_weights_variant(self.h).decode()

    def file_bytes(self):
        return lib().hat_weights_file_bytes(self.h)

    def shape(self, name):
        d = (C.c_size_t * 16)()
        n = _check(lib().hat_weights_shape(self.h, name.encode(), d, 16), "hat_weights_shape")
        return [d[i] for i in range(n)]

    def gpu_plan(self, h, w):
        p = MemPlan()
        _check(lib().hat_gpu_plan(self.h, h, w, C.byref(p)), "hat_gpu_plan")
        return {n: getattr(p, n) for n, _ in MemPlan._fields_}

    def names(self):
        L = lib()
        return [L.hat_weights_name(self.h, i).decode() for i in range(L.hat_weights_count(self.h))]

    def tensor(self, name):
        n = C.c_size_t(0)
        p = lib().hat_weights_tensor(self.h, name.encode(), C.byref(n))
        if not p:
            raise HatError(_err())
        return np.ctypeslib.as_array(p, shape=(n.value,))

    def i64(self, name):
        L = lib()
        n = L.hat_weights_index_i64(self.h, name.encode(), None, 0)
        _check(n, "hat_weights_index_i64")
        out = np.zeros(n, dtype=np.int64)
        L.hat_weights_index_i64(self.h, name.encode(), out.ctypes.data_as(C.POINTER(C.c_longlong)), n)
        return out

    def close(self):
        if self.h:
            lib().hat_weights_close(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def gpu_available():
    return bool(lib().hat_gpu_available())


class Backend:
    """The MI355X backend behind the reference's `Backend` trait (src/backend.rs:29-36)."""

    def __init__(self, weights, device="gpu"):
        self.weights = weights
        h = lib().hat_backend_new(weights.h, device.encode())
        if not h:
            raise HatError(_err())
        self.h = h

    def name(self):
        return lib().hat_backend_name(self.h).decode()

    def forward(self, h, w, img, out=None):
        """Backend::forward; `out` (optional) is a caller-allocated
        [3][h*s][w*s] float32 array, as the C ABI's output argument is."""
        img = f32(img).reshape(3, h, w)
        s = self.weights.scale
        if out is None:
            out = np.empty((3, h * s, w * s), dtype=np.float32)
        assert out.shape == (3, h * s, w * s) and out.dtype == np.float32 and out.flags["C_CONTIGUOUS"]
        _check(lib().hat_backend_forward(self.h, h, w, _fp(img), _fp(out)), "forward")
        return out

    def forward_device(self, h, w, d_in, d_out):
        _check(lib().hat_backend_forward_device(self.h, h, w, d_in, d_out), "forward_device")

    def forward_batch(self, n, h, w, imgs):
        imgs = f32(imgs).reshape(n, 3, h, w)
        s = self.weights.scale
        out = np.empty((n, 3, h * s, w * s), dtype=np.float32)
        _check(lib().hat_backend_forward_batch(self.h, n, h, w, _fp(imgs), _fp(out)), "forward_batch")
        return out

    def tile_forward(self, h, w, img, tile, margin):
        img = f32(img).reshape(3, h, w)
        s = self.weights.scale
        out = np.empty((3, h * s, w * s), dtype=np.float32)
        t = Tiling()
        _check(lib().hat_tile_forward(self.h, h, w, _fp(img), _fp(out), tile, margin, C.byref(t)),
               "tile_forward")
        return out, {n: getattr(t, n) for n, _ in Tiling._fields_}

    def forward_noalloc(self, h, w, d_in, d_out):
        _check(lib().hat_backend_forward_noalloc(self.h, h, w, d_in, d_out), "forward_noalloc")

    def synchronize(self):
        _check(lib().hat_backend_synchronize(self.h), "synchronize")

    def hab(self, stage, block, hp, wp, x, iters=0):
        """One HAB (gpu.rs:469-520) on a token-major [hp*wp][embed] plane; returns
        (out, mean ms over `iters` further runs)."""
        x = f32(x).reshape(hp * wp, self.weights.embed)
        out = np.empty_like(x)
        ms = C.c_float(0)
        _check(lib().hat_backend_hab(self.h, stage, block, hp, wp, _fp(x), _fp(out), iters,
                                     C.cast(C.byref(ms), _f32p)), "hat_backend_hab")
        return out, ms.value

    def acts_bytes(self):
        return lib().hat_backend_acts_bytes(self.h)

    def weight_bytes(self):
        return lib().hat_backend_weight_bytes(self.h)

    def close(self):
        if self.h:
            lib().hat_backend_free(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def verify(weights, fixture_path, device="gpu"):
    rc = lib().hat_verify(weights.h, device.encode(), str(fixture_path).encode())
    if rc < 0:
        raise HatError(_err())
    return rc


def auto_tile(h, w, win, budget_bytes, per_pixel_floats, constant_floats, margin):
    """tile::auto_tile; None when not even one window fits."""
    t = lib().hat_auto_tile(h, w, win, budget_bytes, per_pixel_floats, constant_floats, margin)
    return t or None


def png_load(path):
    w, h = C.c_size_t(0), C.c_size_t(0)
    _check(lib().hat_png_load(str(path).encode(), C.byref(w), C.byref(h), None, 0), "hat_png_load")
    out = np.empty((3, h.value, w.value), dtype=np.float32)
    _check(lib().hat_png_load(str(path).encode(), C.byref(w), C.byref(h), _fp(out), out.size), "hat_png_load")
    return out


def png_save(path, planes):
    planes = f32(planes)
    c, h, w = planes.shape
    assert c == 3
    _check(lib().hat_png_save(str(path).encode(), w, h, _fp(planes)), "hat_png_save")


CLI_PATH = os.path.join(HERE, "build", "hat")


def selftest():
    return _check(lib().hat_gpu_selftest(), "selftest")


def op_swmsa(x, hp, wp, c, heads, shift, qkv_w, qkv_b, proj_w, proj_b, table, iters=0):
    x = f32(x)
    out = np.empty_like(x)
    ms = C.c_float(0)
    ams = C.c_float(0)
    args = [f32(a) for a in (qkv_w, qkv_b, proj_w, proj_b, table)]
    _check(lib().hat_op_swmsa(_fp(x), _fp(out), hp, wp, c, heads, shift, *[_fp(a) for a in args],
                              iters, C.cast(C.byref(ms), _f32p), C.cast(C.byref(ams), _f32p)),
           "hat_op_swmsa")
    return out, ms.value, ams.value


def op_ocab(x, hp, wp, c, heads, mlp_ratio, ws, iters=0):
    """ws: the 13 OCAB tensors in the order of include/hat.h."""
    x = f32(x)
    out = np.empty_like(x)
    ms = C.c_float(0)
    ams = C.c_float(0)
    args = [f32(a) for a in ws]
    _check(lib().hat_op_ocab(_fp(x), _fp(out), hp, wp, c, heads, mlp_ratio,
                             *[_fp(a) for a in args], iters, C.cast(C.byref(ms), _f32p),
                             C.cast(C.byref(ams), _f32p)), "hat_op_ocab")
    return out, ms.value, ams.value


class DeviceBuffer:
    def __init__(self, nbytes):
        self.nbytes = nbytes
        self.ptr = lib().hat_device_alloc(nbytes)
        if not self.ptr:
            raise HatError(_err())

    def upload(self, arr):
        arr = np.ascontiguousarray(arr)
        assert arr.nbytes <= self.nbytes
        _check(lib().hat_memcpy_h2d(self.ptr, arr.ctypes.data, arr.nbytes), "h2d")

    def download(self, arr):
        assert arr.nbytes <= self.nbytes and arr.flags["C_CONTIGUOUS"]
        _check(lib().hat_memcpy_d2h(arr.ctypes.data, self.ptr, arr.nbytes), "d2h")
        return arr

    def free(self):
        if self.ptr:
            lib().hat_device_free(self.ptr)
            self.ptr = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


def synchronize():
    _check(lib().hat_device_synchronize(), "synchronize")


def device_copy(dst, src, nbytes):
    """Device-to-device copy with the library's copy kernel (DeviceBuffer or raw pointers)."""
    d = dst.ptr if isinstance(dst, DeviceBuffer) else dst
    s = src.ptr if isinstance(src, DeviceBuffer) else src
    _check(lib().hat_device_copy(d, s, nbytes), "device_copy")


def device_mem_info():
    """(free, total) device memory in bytes."""
    fr, tot = C.c_size_t(0), C.c_size_t(0)
    _check(lib().hat_device_mem_info(C.byref(fr), C.byref(tot)), "device_mem_info")
    return fr.value, tot.value


def device_name():
    return lib().hat_device_name().decode()


def device_cu_count():
    return lib().hat_device_cu_count()


def profile_begin():
    _check(lib().hat_profile_begin(), "profile_begin")


def profile_end():
    """Stop timing; return {kernel: (launches, total_ms)}."""
    L = lib()
    _check(L.hat_profile_end(), "profile_end")
    out = {}
    buf = C.create_string_buffer(128)
    for i in range(L.hat_profile_count()):
        cnt = C.c_long(0)
        tot = C.c_double(0)
        _check(L.hat_profile_get(i, buf, 128, C.byref(cnt), C.byref(tot)), "profile_get")
        out[buf.value.decode()] = (cnt.value, tot.value)
    return out
