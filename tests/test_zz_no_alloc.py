"""GPU: lq8_linear_forward_device_noalloc (the activation operand in the
library's static per-GPU scratch array, no allocation) against
lq8_linear_forward_device, bit for bit, on two calls in a row whose second
input is smaller, plus the GEMV path and the size limit."""
import numpy as np
import pytest

import lq8
import oracle

pytestmark = pytest.mark.gpu


def normal(shape, std, seed):
    return (np.random.default_rng(seed).standard_normal(shape) * std).astype(np.float32)


def run(ctx, fn, w, x, m, n):
    dx = lq8.DeviceBuffer.from_array(ctx, x)
    dy = lq8.DeviceBuffer(ctx, m * n * 4)
    try:
        lq8._check(getattr(lq8.lib(), fn)(ctx.handle, w.handle, dx.ptr, m, dy.ptr))
        lq8._check(lq8.lib().lq8_synchronize(ctx.handle))
        return dy.download(np.float32, m * n).reshape(m, n)
    finally:
        dx.free()
        dy.free()


def test_noalloc_equals_linear_forward_device(ctx):
    cases = [(512, 3072, 1024, 1), (37, 1024, 3072, 2), (1, 2048, 1024, 3)]  # second call smaller; then the GEMV
    for m, n, k, seed in cases:
        blocks = oracle.quantize_q8_0(normal((n, k), 0.02, seed))
        w = lq8.Q8Weight.from_blocks(ctx, blocks, n, k)
        x = normal((m, k), 1.0, 100 + seed)
        try:
            ref = run(ctx, "lq8_linear_forward_device", w, x, m, n)
            got = run(ctx, "lq8_linear_forward_device_noalloc", w, x, m, n)
        finally:
            w.free()
        assert np.array_equal(got.view(np.uint32), ref.view(np.uint32)), (m, n, k)
        assert np.array_equal(got.view(np.uint32), oracle.linear_forward(blocks, n, k, x).view(np.uint32)), (m, n, k)


def test_noalloc_rejects_operands_above_the_scratch(ctx):
    """2048 x 4096 needs 10 MiB of activation operand: refused on the host,
    nothing launched; 2048 x 3072 (7.5 MiB) fits."""
    w = lq8.Q8Weight.random(ctx, 64, 4096, seed=4)
    dx = lq8.DeviceBuffer(ctx, 2048 * 4096 * 4)
    dy = lq8.DeviceBuffer(ctx, 2048 * 64 * 4)
    try:
        with pytest.raises(lq8.ShapeMismatch):
            lq8._check(lq8.lib().lq8_linear_forward_device_noalloc(ctx.handle, w.handle, dx.ptr, 2048, dy.ptr))
    finally:
        dx.free(); dy.free(); w.free()
    blocks = oracle.quantize_q8_0(normal((64, 3072), 0.02, 5))
    w = lq8.Q8Weight.from_blocks(ctx, blocks, 64, 3072)
    x = normal((2048, 3072), 1.0, 6)
    try:
        got = run(ctx, "lq8_linear_forward_device_noalloc", w, x, 2048, 64)
        ref = run(ctx, "lq8_linear_forward_device", w, x, 2048, 64)
    finally:
        w.free()
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))
