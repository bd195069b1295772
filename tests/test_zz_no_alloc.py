"""fg_matmul_device_noalloc: the product of fg_matmul_device with the
activation pieces in the library's static device scratch instead of the
context workspace. Its output must equal fg_matmul_device's bit for bit
(the same kernels), on two calls in a row with the second on fewer rows,
for each weight format, through the multi-pass GEMVs (13 then 5 rows) and
the one-pass ones (4 then 1 row: the decode GEMVs, the int4 16-wave kernel
among them); inputs beyond its limits are refused, and a call at the limit
of one pass still equals fg_matmul_device.

Device buffers come from hipMalloc of the HIP runtime the library itself
uses (the caller's allocations, not the entry point's); the library's
stream is synchronised before they are read back."""
import ctypes as C

import numpy as np
import pytest

from ferrolm_amd import gpu
from ferrolm_amd.weights import BF16, INT4, INT8, Matrix

pytestmark = pytest.mark.gpu


def matrix(kind, rows, cols, seed):
    rng = np.random.default_rng(seed)
    w = (rng.standard_normal((rows, cols)) * 0.05).astype(np.float32)
    if kind == BF16:
        bits = (w.view(np.uint32) + 0x7FFF + ((w.view(np.uint32) >> 16) & 1)) >> 16
        return Matrix(BF16, rows, cols, bf16=bits.astype(np.uint16))
    from ferrolm_amd import host
    return host.quantize(kind, w)


class Hip:
    """hipMalloc / hipMemcpy / hipFree of the runtime the library loaded."""

    def __init__(self):
        self.rt = C.CDLL("libamdhip64.so")

    def alloc(self, nbytes):
        p = C.c_void_p()
        assert self.rt.hipMalloc(C.byref(p), C.c_size_t(nbytes)) == 0
        return p

    def put(self, dst, a):
        a = np.ascontiguousarray(a)
        assert self.rt.hipMemcpy(dst, a.ctypes.data_as(C.c_void_p), C.c_size_t(a.nbytes), 1) == 0

    def get(self, src, shape, dtype=np.float32):
        out = np.empty(shape, dtype)
        assert self.rt.hipMemcpy(out.ctypes.data_as(C.c_void_p), src, C.c_size_t(out.nbytes), 2) == 0
        return out

    def free(self, *ps):
        for p in ps:
            self.rt.hipFree(p)


def call(fn, ctx, mat, x, m, y):
    gpu.check(fn(ctx.h, mat.h, x, m, y))


@pytest.mark.parametrize("rows_pair", [(13, 5), (4, 1)])
@pytest.mark.parametrize("kind", [BF16, INT8, INT4])
def test_matches_the_allocating_entry_point(ctx, kind, rows_pair):
    hip = Hip()
    rows, cols = 768, 2048
    mat = gpu.Mat(ctx, matrix(kind, rows, cols, 7 + kind))
    lib = gpu.lib()
    nan = np.full((16, rows), np.nan, np.float32)
    for m in rows_pair:  # two calls in a row, the second on fewer rows
        x_np = np.random.default_rng(m).standard_normal((m, cols)).astype(np.float32)
        x, want, got = hip.alloc(x_np.nbytes), hip.alloc(nan.nbytes), hip.alloc(nan.nbytes)
        try:
            hip.put(x, x_np)
            hip.put(want, nan)
            hip.put(got, nan)
            call(lib.fg_matmul_device, ctx, mat, x, m, want)
            call(lib.fg_matmul_device_noalloc, ctx, mat, x, m, got)
            ctx.sync()
            w, g = hip.get(want, (m, rows)), hip.get(got, (m, rows))
        finally:
            hip.free(x, want, got)
        assert np.isfinite(w).all()
        assert np.array_equal(g.view(np.uint32), w.view(np.uint32)), (kind, m)


def test_refuses_beyond_its_limits(ctx):
    hip = Hip()
    lib = gpu.lib()
    wide = gpu.Mat(ctx, matrix(BF16, 32, 16384, 3))  # 512 k-blocks: 4 passes need 2.1 MB
    x, y, want = hip.alloc(16 * 16384 * 4), hip.alloc(16 * 32 * 4), hip.alloc(16 * 32 * 4)
    try:
        hip.put(x, np.random.default_rng(11).standard_normal((16, 16384)).astype(np.float32))
        with pytest.raises(gpu.FgError, match="2 MiB scratch"):
            call(lib.fg_matmul_device_noalloc, ctx, wide, x, 13, y)
        with pytest.raises(gpu.FgError, match="at most 15 rows"):
            call(lib.fg_matmul_device_noalloc, ctx, wide, x, 16, y)
        call(lib.fg_matmul_device_noalloc, ctx, wide, x, 4, y)  # one pass fits
        call(lib.fg_matmul_device, ctx, wide, x, 4, want)
        ctx.sync()
        g, w = hip.get(y, (4, 32)), hip.get(want, (4, 32))
        assert np.isfinite(w).all() and np.abs(w).max() > 0
        assert np.array_equal(g.view(np.uint32), w.view(np.uint32))
    finally:
        hip.free(x, y, want)
