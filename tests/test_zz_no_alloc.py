"""navi_linear_noalloc (the entry point that allocates nothing) against navi_linear through the C
ABI: two calls in a row, the second with a smaller input, each bit-identical to navi_linear on the
same inputs (same split count and kernels; only the workspace differs), plus numpy f64 as a sanity
bound; a request whose partials exceed the fixed scratch is a clear error."""
import numpy as np
import pytest

from gpu_util import log

pytestmark = pytest.mark.gpu


def _case(abi, rng, M, K, N, act, bias, resid):
    x = (rng.standard_normal((M, K)) * 2).astype(np.float32)
    w = (rng.standard_normal((N, K)) * 0.05).astype(np.float16)
    b = rng.standard_normal(N).astype(np.float32) if bias else None
    r = rng.standard_normal((M, N)).astype(np.float32) if resid else None
    dx, dw = abi.DeviceBuffer(x.nbytes), abi.DeviceBuffer(w.nbytes)
    dx.upload(x)
    dw.upload(w.view(np.uint16))
    db = None
    if b is not None:
        db = abi.DeviceBuffer(b.nbytes)
        db.upload(b)
    outs = []
    for noalloc in (False, True):
        dy = abi.DeviceBuffer(4 * M * N)
        dy.upload(r if r is not None else np.full((M, N), np.nan, np.float32))
        abi.linear(dx.ptr, K, M, dw.ptr, K, N, dy.ptr, N, bias=db.ptr if db else None,
                   residual=dy.ptr if r is not None else None, act=act, noalloc=noalloc)
        outs.append(dy.download(np.float32, M * N).reshape(M, N))
    want = x.astype(np.float64) @ w.astype(np.float64).T
    if b is not None:
        want += b
    if act:
        want = want / (1 + np.exp(-want))
    if r is not None:
        want += r
    return outs[0], outs[1], want


def test_noalloc_linear_equals_linear_twice_second_smaller():
    from navi_amd import abi
    abi.device_open()
    rng = np.random.default_rng(7)
    for M, K, N, act, bias, resid in ((130, 2048, 2048, 1, True, False), (9, 1024, 1024, 0, False, True)):
        log(f"noalloc linear M={M} K={K} N={N}")
        ref, got, want = _case(abi, rng, M, K, N, act, bias, resid)
        assert np.array_equal(got, ref), f"M={M}: noalloc differs from navi_linear"
        scale = np.abs(want).max() + 1.0
        assert np.abs(got - want).max() / scale < 1e-5


def test_noalloc_linear_rejects_oversized_partials():
    from navi_amd import abi
    abi.device_open()
    M, K, N = 1024, 4096, 4096            # K-split partials far above the fixed scratch
    d = abi.DeviceBuffer(4 * M * K)
    w = abi.DeviceBuffer(2 * N * K)
    y = abi.DeviceBuffer(4 * M * N)
    with pytest.raises(abi.NaviError) as e:
        abi.linear(d.ptr, K, M, w.ptr, K, N, y.ptr, N, noalloc=True)
    assert e.value.status == abi.NAVI_ERR_INVALID and "fixed scratch" in str(e.value)
