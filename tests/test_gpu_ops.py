"""GPU decoder ops vs the oracle, bit for bit, over many rows: RmsNorm's
correctly rounded sqrt/divide and bf16 roundings, SiLU's exp."""
import numpy as np
import pytest

import lq8
import oracle

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("dim,rows", [(1024, 40000), (128, 200000)])
def test_rms_norm_rows_bit_exact(ctx, dim, rows):
    rng = np.random.default_rng(dim)
    scale = np.exp(rng.uniform(-6, 6, (rows, 1))).astype(np.float32)
    x = (rng.standard_normal((rows, dim)) * scale).astype(np.float32)
    w = (1.0 + 0.1 * rng.standard_normal(dim)).astype(np.float32)
    got = lq8.rms_norm_device(ctx, x, w, 1e-6)
    ref = oracle.rms_norm(x, w, 1e-6)
    bad = np.flatnonzero((got.view(np.uint32) != ref.view(np.uint32)).any(axis=1))
    assert bad.size == 0, f"{bad.size} rows differ, first {bad[:5]}"


def test_silu_exp_sweep_bit_exact(ctx):
    x = np.concatenate([np.linspace(-120, 120, 1_000_001, dtype=np.float32),
                        np.random.default_rng(0).standard_normal(500_000).astype(np.float32) * 4,
                        np.array([0.0, -0.0, 88.7, 89.5, -87.5, -103.9, -104.5, np.inf, -np.inf], np.float32)])
    got = lq8.silu_device(ctx, x)
    e = oracle.expf(-x)
    with np.errstate(over="ignore", invalid="ignore"):
        ref = (x / (np.float32(1.0) + e)).astype(np.float32)
    same = (got.view(np.uint32) == ref.view(np.uint32)) | (np.isnan(got) & np.isnan(ref))
    assert same.all(), f"{np.count_nonzero(~same)} differ, e.g. x={x[~same][:5]}"
