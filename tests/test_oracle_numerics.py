"""CPU: the oracle's scalar numerics pinned against numpy and closed forms."""
import numpy as np
import pytest

import oracle
from golden import numpy_q8


def test_f16_to_f32_exhaustive():
    h = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    got = oracle.f16_bits_to_f32(h)
    ref = h.view(np.float16).astype(np.float32)
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), ref[~nan].view(np.uint32))


def test_f32_to_f16_round_to_nearest_even():
    rng = np.random.default_rng(0)
    x = np.concatenate([
        (rng.standard_normal(200000) * np.exp(rng.uniform(-25, 12, 200000))).astype(np.float32),
        # exact midpoints between neighbouring f16 values (ties), normal and subnormal
        ((np.arange(0, 65504, 7, dtype=np.float32).astype(np.float16).astype(np.float32)
          + np.nextafter(np.arange(0, 65504, 7, dtype=np.float32).astype(np.float16), np.float16(np.inf)).astype(np.float32)) / 2),
        (np.arange(1, 2048, dtype=np.float32) * 2.0 ** -25),
        np.array([0.0, -0.0, 65504, 65519.99, 65520, 1e30, -1e30, np.inf, -np.inf, 2.0 ** -25, 2.0 ** -26], np.float32)])
    got = oracle.f32_to_f16_bits(x)
    with np.errstate(over="ignore"):
        ref = x.astype(np.float16).view(np.uint16)
    assert np.array_equal(got, ref)


def test_bf16_round_matches_reference_formula_and_tests():
    rng = np.random.default_rng(1)
    x = np.concatenate([rng.standard_normal(100000).astype(np.float32) * 1e3,
                        np.array([0.0, -0.0, 1.0, -1.0, np.inf, -np.inf], np.float32)])
    assert np.array_equal(oracle.bf16_round(x).view(np.uint32), numpy_q8.bf16_round(x).view(np.uint32))
    # src/bf16.rs:170 -0.0 keeps its sign; :238 the tie 0x3F808000 rounds to even (1.0)
    assert oracle.bf16_round(np.array([-0.0], np.float32)).view(np.uint32)[0] == 0x80000000
    tie = np.array([0x3F808000], np.uint32).view(np.float32)
    assert oracle.bf16_round(tie)[0] == 1.0
    tie_up = np.array([0x3F818000], np.uint32).view(np.float32)     # odd lsb -> rounds up
    assert oracle.bf16_round(tie_up).view(np.uint32)[0] == 0x3F820000
    # src/bf16.rs:224: the smallest subnormal becomes (signed) zero or stays tiny
    assert abs(oracle.bf16_round(np.array([np.float32(1e-45)]))[0]) < 1e-30


def test_expf_correctly_rounded_on_dense_grid():
    x = np.concatenate([np.linspace(-104, 89, 3_000_001, dtype=np.float32),
                        np.random.default_rng(2).standard_normal(500000).astype(np.float32) * 10])
    got = oracle.expf(x)
    with np.errstate(over="ignore"):
        ref = np.exp(x.astype(np.float64)).astype(np.float32)
    assert np.count_nonzero(got.view(np.uint32) != ref.view(np.uint32)) == 0


def test_expf_special_values():
    x = np.array([0.0, -0.0, np.inf, -np.inf, np.nan, 89.5, -120.0, 88.72283], np.float32)
    y = oracle.expf(x)
    assert y[0] == 1.0 and y[1] == 1.0 and np.isinf(y[2]) and y[3] == 0.0 and np.isnan(y[4])
    assert np.isinf(y[5]) and y[6] == 0.0 and np.isfinite(y[7])


@pytest.mark.parametrize("x,expected", [(0.0, 0.0), (1.0, 0.7310585786300049), (-1.0, -0.2689414213699951),
                                        (5.0, 4.966535745378576), (-5.0, -0.03346425462142428)])
def test_silu_known_values(x, expected):
    """SiLU closed form x * sigmoid(x) (src/mlp.rs:242-520 checks the same)."""
    assert abs(oracle.silu(x) - expected) <= 1e-6 * max(1.0, abs(expected))


def test_argmax_last_index_on_ties():
    """Iterator::max_by returns the last maximum (src/tensor.rs:2475-2480)."""
    assert oracle.argmax_last(np.array([1, 5, 2, 5, 0], np.float32)) == 3
    assert oracle.argmax_last(np.array([7, 7, 7], np.float32)) == 2
    assert oracle.argmax_last(np.array([1.0, 2.0, 5.0, 1.0, 0.5], np.float32)) == 2   # src/generate.rs:149
