"""hat_backend_forward_noalloc: the forward with every per-plan buffer carved
from the library's fixed scratch array instead of allocated. Checked through the
C ABI against hat_backend_forward_device on the same backend (same kernels,
same order: bit-identical), on two calls in a row, the second on a smaller
image, so the second runs over what the first left in the array."""
import numpy as np
import pytest

from conftest import make_weights

pytestmark = pytest.mark.gpu


def _say(msg):
    print(msg, flush=True)


def _run(hl, be, h, w, scale, img, noalloc):
    d_in = hl.DeviceBuffer(img.nbytes)
    out = np.empty((3, h * scale, w * scale), dtype=np.float32)
    d_out = hl.DeviceBuffer(out.nbytes)
    d_in.upload(img)
    if noalloc:
        be.forward_noalloc(h, w, d_in.ptr, d_out.ptr)
    else:
        be.forward_device(h, w, d_in.ptr, d_out.ptr)
    be.synchronize()
    return d_out.download(out)


@pytest.mark.parametrize("variant,sizes", [("hat-s", [(64, 64), (32, 48)]), ("hat", [(48, 48), (16, 32)])])
def test_noalloc_forward_equals_forward_device(weights_dir, variant, sizes):
    """HAT-S (C = 144: the folded CAB, the 144-channel tails) and HAT (C = 180:
    the unfolded CAB's Winograd convs, the 180-channel tails), each on two calls
    in a row, the second smaller."""
    import hat_amd as hl
    assert hl.gpu_available(), "the HIP runtime or the GPU is missing"
    wp = make_weights(weights_dir, variant, 4, 1, None)
    be = hl.Backend(hl.Weights(wp))
    rng = np.random.default_rng(77)
    for h, w in sizes:
        img = rng.random((3, h, w), dtype=np.float32)
        _say(f"forward_noalloc {variant} x4 {h}x{w}")
        got = _run(hl, be, h, w, 4, img, True)
        want = _run(hl, be, h, w, 4, img, False)
        assert np.isfinite(got).all()
        assert np.array_equal(got, want), f"{h}x{w}: worst |diff| {np.abs(got - want).max():.3e}"
    # a plan beyond the array is refused before anything runs
    big = hl.DeviceBuffer(3 * 512 * 512 * 4)
    big_out = hl.DeviceBuffer(3 * 2048 * 2048 * 4)
    with pytest.raises(hl.HatError) as e:
        be.forward_noalloc(512, 512, big.ptr, big_out.ptr)
    assert "scratch" in str(e.value)
    be.close()
