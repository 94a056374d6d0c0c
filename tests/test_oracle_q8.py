"""CPU: Q8_0 format and matmul of the oracle, pinned by an independent numpy
restatement, invariants, closed forms, brute force and golden fixtures."""
import os

import numpy as np
import pytest

import oracle
from golden import numpy_q8

GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "q8_0_golden.npz")


def normal(shape, std, seed):
    return (np.random.default_rng(seed).standard_normal(shape) * std).astype(np.float32)


def test_quantize_matches_numpy_restatement():
    x = np.concatenate([normal(32 * 20000, 1.0, 1), normal(32 * 5000, 0.02, 2),
                        normal(32 * 2000, 1e-5, 3), normal(32 * 2000, 1e4, 4)])
    assert np.array_equal(oracle.quantize_q8_0(x), numpy_q8.quantize_q8_0(x))


def test_quantize_invariants():
    x = normal(32 * 4096, 1.0, 7)
    b = oracle.quantize_q8_0(x).reshape(-1, 34)
    q = b[:, 2:].view(np.int8).astype(np.int32)
    xb = x.reshape(-1, 32)
    # the element of largest magnitude maps to +-127
    i = np.argmax(np.abs(xb), axis=1)
    assert np.all(np.abs(q[np.arange(len(i)), i]) == 127)
    # sign preserved (or zero), codes in [-127, 127]
    assert np.all((np.sign(q) == np.sign(xb)) | (q == 0))
    assert np.all(np.abs(q) <= 127)
    # reconstruction error bounded by half the (f32) step
    d32 = (np.abs(xb).max(axis=1) / np.float32(127)).astype(np.float64)
    err = np.abs(xb.astype(np.float64) - q * d32[:, None])
    assert np.all(err <= d32[:, None] * (0.5 + 1e-4))


def test_quantize_special_blocks():
    z = oracle.quantize_q8_0(np.zeros(32, np.float32))
    assert np.all(z == 0)                                      # d = 0, codes 0
    t = np.zeros(32, np.float32)
    t[0] = 127.0
    t[1:7] = [0.5, -0.5, 1.5, -1.5, 2.5, -2.5]
    q = oracle.quantize_q8_0(t)[2:].view(np.int8)
    assert q[:7].tolist() == [127, 1, -1, 2, -2, 3, -3]        # ties round away from zero
    t = np.random.default_rng(1).standard_normal(32).astype(np.float32)
    t[4] = np.nan
    assert oracle.quantize_q8_0(t)[2 + 4] == 0                 # NaN -> 0, ignored by amax
    with pytest.raises(ValueError):
        oracle.quantize_q8_0(np.zeros(33, np.float32))


def test_dequantize_exact():
    x = normal(32 * 1000, 0.5, 9)
    b = oracle.quantize_q8_0(x)
    y = oracle.dequantize_q8_0(b, x.size)
    assert np.array_equal(y, numpy_q8.dequantize_q8_0(b, x.size))
    # d (11-bit significand) * q (8-bit) is exact in f32: equal to the f64 product
    bb = b.reshape(-1, 34)
    d = bb[:, :2].copy().view(np.float16).astype(np.float64)
    q = bb[:, 2:].view(np.int8).astype(np.float64)
    assert np.array_equal(y.astype(np.float64), (d * q).reshape(-1))


@pytest.mark.parametrize("n,k", [(96, 256), (3, 32), (64, 1024), (33, 3072)])
def test_gemv_vs_f64_brute_force(n, k):
    b = oracle.quantize_q8_0(normal((n, k), 0.02, n + k))
    x = normal(k, 1.0, 2 * k)
    y = oracle.gemv_q8_0(b, n, k, x)
    ref = numpy_q8.gemv_f64(b, n, k, x)
    assert np.max(np.abs(y - ref)) <= 1e-5 * max(np.max(np.abs(ref)), 1e-30)


def test_gemv_known_answers():
    """test_linear_forward (src/attention.rs:605) -> [14, 32] and the GPU GEMV
    test (src/gpu/gemv.rs:543) -> [14, 32, 50, 68], on Q8_0-exact weights (a
    127 in each row makes d = 1; x is 0 there)."""
    W = np.zeros((4, 32), np.float32)
    W[:, :3] = [[1, 2, 3], [4, 5, 6], [7, 8, 9], [10, 11, 12]]
    W[:, -1] = 127
    x = np.zeros(32, np.float32)
    x[:3] = [1, 2, 3]
    b = oracle.quantize_q8_0(W)
    assert oracle.gemv_q8_0(b, 4, 32, x).tolist() == [14.0, 32.0, 50.0, 68.0]
    assert oracle.gemv_q8_0(b[:2 * 34], 2, 32, x).tolist() == [14.0, 32.0]


def test_gemv_one_hot_and_zero():
    n, k = 40, 128
    b = oracle.quantize_q8_0(normal((n, k), 0.02, 3))
    W = oracle.dequantize_q8_0(b, n * k).reshape(n, k)
    for col in (0, 31, 32, 127):
        e = np.zeros(k, np.float32)
        e[col] = 1.0
        assert np.array_equal(oracle.gemv_q8_0(b, n, k, e), W[:, col])
    assert np.all(oracle.gemv_q8_0(b, n, k, np.zeros(k, np.float32)) == 0)


def test_gemm_int32_blocks_exact():
    """With a 127 in every block (d = 1) the W8A8 result is the integer dot."""
    m, n, k = 7, 9, 96
    rng = np.random.default_rng(4)
    qw = rng.integers(-127, 128, (n, k)).astype(np.float32)
    qx = rng.integers(-127, 128, (m, k)).astype(np.float32)
    qw[:, ::32] = 127
    qx[:, ::32] = 127
    y = oracle.gemm_q8_0(oracle.quantize_q8_0(qw), n, k, qx)
    assert np.array_equal(y.astype(np.int64), qx.astype(np.int64) @ qw.astype(np.int64).T)


def test_gemm_equals_w8a8_f64():
    m, n, k = 6, 50, 256
    b = oracle.quantize_q8_0(normal((n, k), 0.02, 11))
    x = normal((m, k), 1.0, 12)
    y = oracle.gemm_q8_0(b, n, k, x)
    Xd = numpy_q8.dequantize_q8_0(numpy_q8.quantize_q8_0(x), m * k).reshape(m, k).astype(np.float64)
    W = numpy_q8.dequantize_q8_0(b, n * k).reshape(n, k).astype(np.float64)
    ref = Xd @ W.T
    assert np.max(np.abs(y - ref)) <= 1e-5 * np.max(np.abs(ref))
    # linear_forward dispatch: m == 1 is the W8A32 GEMV, m > 1 the W8A8 GEMM
    assert np.array_equal(oracle.linear_forward(b, n, k, x[:1])[0], oracle.gemv_q8_0(b, n, k, x[0]))
    assert np.array_equal(oracle.linear_forward(b, n, k, x), y)


def test_canonical_and_sequential_orders_agree():
    n, k = 256, 3072
    b = oracle.quantize_q8_0(normal((n, k), 0.02, 5))
    x = normal(k, 1.0, 6)
    y = oracle.gemv_q8_0(b, n, k, x)
    oracle.set_sequential_sums(True)
    try:
        ys = oracle.gemv_q8_0(b, n, k, x)
    finally:
        oracle.set_sequential_sums(False)
    assert np.max(np.abs(y - ys)) <= 1e-5 * np.max(np.abs(ys))


def test_golden_fixtures():
    g = np.load(GOLDEN)
    assert np.array_equal(oracle.quantize_q8_0(g["quant_x"]), g["quant_blocks"])
    assert np.array_equal(numpy_q8.quantize_q8_0(g["quant_x"]), g["quant_blocks"])
    n, k = g["gemv_y"].size, g["gemv_x"].size
    assert np.array_equal(oracle.gemv_q8_0(g["gemv_w"], n, k, g["gemv_x"]).view(np.uint32), g["gemv_y"].view(np.uint32))
    assert np.array_equal(oracle.gemm_q8_0(g["gemv_w"], n, k, g["gemm_x"]).view(np.uint32), g["gemm_y"].view(np.uint32))


@pytest.mark.parametrize("n,k", [(5, 1024), (3, 96), (4, 3072), (2, 32)])
def test_gemv_tree_order_exact(n, k):
    """The oracle's GEMV equals an exact rational restatement of its documented
    summation order (fmaf rounded once from the exact value), bit for bit."""
    b = oracle.quantize_q8_0(normal((n, k), 0.02, 40 + k))
    x = normal(k, 1.0, 41 + k)
    y = oracle.gemv_q8_0(b, n, k, x)
    ref = numpy_q8.gemv_tree_rows(b, n, k, x, range(n))
    assert np.array_equal(y.view(np.uint32), ref.view(np.uint32))


def test_gemv_tree_order_is_not_sequential():
    """The exact restatement separates the tree from a plain chain over blocks
    (a plausible mistake): on a row where the two differ, the oracle gives the
    tree's bits."""
    k = 256
    for seed in range(200):
        b = oracle.quantize_q8_0(normal((1, k), 0.02, 1000 + seed))
        x = normal(k, 1.0, 2000 + seed)
        bb = b.reshape(8, 34)
        vals = []
        for j in range(8):
            d = bb[j, :2].copy().view(np.float16).astype(np.float32)[0]
            q = bb[j, 2:].view(np.int8).astype(np.float32)
            h0 = np.float32(0)
            for t in range(16):
                h0 = numpy_q8.fmaf_exact(q[t], x[32 * j + t], h0)
            h1 = np.float32(0)
            for t in range(16, 32):
                h1 = numpy_q8.fmaf_exact(q[t], x[32 * j + t], h1)
            vals.append(np.float32(np.float32(h0 + h1) * d))
        chain = np.float32(0)
        for v in vals:
            chain = np.float32(chain + v)
        tree = numpy_q8.gemv_tree_rows(b, 1, k, x, [0])[0]
        if chain != tree:
            assert oracle.gemv_q8_0(b, 1, k, x)[0] == tree
            return
    pytest.fail("no row separating the two orders found")


# Known answers of the reference's matmul tests, made Q8_0-exact: the operands
# are padded to one 32-value block with a 127 in a column where the other
# operand is 0, so both block scales are exactly 1 and the codes are the
# integers themselves.
MATMUL_KNOWN = [
    ("src/tensor.rs:3360 test_matmul_2d_basic", [[1, 2], [3, 4]], [[5, 6], [7, 8]], [[19, 22], [43, 50]]),
    ("src/tensor.rs:3377 test_matmul_2d_non_square", [[1, 2], [3, 4], [5, 6]], [[1, 2, 3, 4], [5, 6, 7, 8]],
     [[11, 14, 17, 20], [23, 30, 37, 44], [35, 46, 57, 68]]),
    ("src/tensor.rs:3408 test_matmul_2d_identity", [[1, 2], [3, 4]], [[1, 0], [0, 1]], [[1, 2], [3, 4]]),
    ("src/tensor.rs:3420 test_matmul_2d_zero_matrix", [[1, 2], [3, 4]], [[0, 0], [0, 0]], [[0, 0], [0, 0]]),
    ("src/gpu/gemm.rs:530 test_gemm_small", [[1, 2, 3], [4, 5, 6], [7, 8, 9], [10, 11, 12]],
     [[1, 0, 0, 0, 1], [0, 1, 0, 1, 0], [0, 0, 1, 0, 0]],
     [[1, 2, 3, 2, 1], [4, 5, 6, 5, 4], [7, 8, 9, 8, 7], [10, 11, 12, 11, 10]]),
]


def exact_operands(a, b):
    """x [m, 32] and W [n, 32] (W = b^T) for x W^T = a b, Q8_0-exact."""
    a, b = np.asarray(a, np.float32), np.asarray(b, np.float32)
    m, k = a.shape
    n = b.shape[1]
    x = np.zeros((m, 32), np.float32)
    x[:, :k] = a
    x[:, 31] = 127.0
    w = np.zeros((n, 32), np.float32)
    w[:, :k] = b.T
    w[:, 30] = 127.0
    return x, w


@pytest.mark.parametrize("case", MATMUL_KNOWN, ids=[c[0].split()[1] for c in MATMUL_KNOWN])
def test_matmul_known_answers(case):
    _, a, b, want = case
    x, w = exact_operands(a, b)
    blocks = oracle.quantize_q8_0(w)
    n = w.shape[0]
    want = np.asarray(want, np.float32)
    assert np.array_equal(oracle.gemm_q8_0(blocks, n, 32, x), want)
    for r in range(x.shape[0]):
        assert np.array_equal(oracle.gemv_q8_0(blocks, n, 32, x[r]), want[r])
