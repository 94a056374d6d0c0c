"""The restated reference CPU Linear::forward (oracle/ref_linear_bf16.c), the
CPU baseline bench.py times: pinned against closed forms and a float64
product, independent of the restatement's own loops."""
import numpy as np
import pytest

import oracle


def bf16_bits(a):
    """Truncating f32 -> BF16 bits (values chosen BF16-exact where it matters)."""
    return (np.asarray(a, dtype=np.float32).view(np.uint32) >> 16).astype(np.uint16)


def bf16_value(bits):
    return (bits.astype(np.uint32) << 16).view(np.float32)


def test_integer_operands_give_the_exact_product():
    # small integers: every BF16 weight and every partial sum is exact, so the
    # result must equal the integer matrix product whatever the loop order
    rng = np.random.default_rng(1)
    w = rng.integers(-8, 9, (64, 96)).astype(np.float32)
    x = rng.integers(-8, 9, (3, 96)).astype(np.float32)
    y = oracle.ref_linear_forward_bf16(bf16_bits(w), x)
    assert np.array_equal(y, (x.astype(np.int64) @ w.T.astype(np.int64)).astype(np.float32))


def test_non_square_orientation():
    # distinct values in a 5 x 7 weight: a transposed or mis-strided read
    # lands on a different element and changes the result
    w = np.arange(35, dtype=np.float32).reshape(5, 7) - 17.0
    x = np.array([[1, 0, 0, 0, 0, 0, 2], [0, 3, 0, 0, 1, 0, 0]], dtype=np.float32)
    y = oracle.ref_linear_forward_bf16(bf16_bits(w), x)
    assert y.shape == (2, 5)
    assert np.array_equal(y, x @ w.T)


def test_bf16_bits_are_widened_not_rounded():
    # 0x3F81 is 1.0078125: the weight's BF16 bits become the f32 operand as is
    w = np.array([[0x3F81, 0xC000]], dtype=np.uint16)  # [1.0078125, -2.0]
    y = oracle.ref_linear_forward_bf16(w, np.array([[1.0, 0.25]], dtype=np.float32))
    assert y[0, 0] == np.float32(1.0078125 - 0.5)


@pytest.mark.parametrize("n,k", [(1024, 1024), (3072, 1024), (1024, 3072)])
def test_random_close_to_float64(n, k):
    rng = np.random.default_rng(n + k)
    wb = bf16_bits(rng.standard_normal((n, k)).astype(np.float32) * 0.02)
    x = rng.standard_normal((1, k)).astype(np.float32)
    y = oracle.ref_linear_forward_bf16(wb, x)
    w64 = bf16_value(wb).astype(np.float64)
    ref = x.astype(np.float64) @ w64.T
    scale = np.abs(x.astype(np.float64)) @ np.abs(w64).T
    # a sequential f32 sum over k terms: error below k * 2^-24 of the sum of |terms|
    assert np.all(np.abs(y - ref) <= k * 2.0 ** -24 * scale + 1e-30)


def test_shape_mismatch_is_an_error():
    with pytest.raises(ValueError):
        oracle.ref_linear_forward_bf16(np.zeros((4, 8), np.uint16), np.zeros((1, 9), np.float32))
