"""GPU parity of the Q8_0 kernels against the CPU oracle, through the C ABI.

Bar: quantized codes and scales bit-exact; GEMV / GEMM outputs bit-exact with
the oracle (the kernels follow the oracle's accumulation order) and, as the
stated contract, within 1e-3 relative error (f32 accumulation).
"""
import numpy as np
import pytest

import lq8
import oracle
from test_oracle_q8 import MATMUL_KNOWN, exact_operands

pytestmark = pytest.mark.gpu

REL_TOL = 1e-3  # matvec/matmul tolerance of the contract (f32 accumulation)


def rel_err(y, ref):
    scale = max(float(np.max(np.abs(ref))), float(np.sqrt(np.mean(ref.astype(np.float64) ** 2))), 1e-30)
    return float(np.max(np.abs(y.astype(np.float64) - ref))) / scale


def assert_parity(y, ref):
    assert y.shape == ref.shape
    assert rel_err(y, ref) <= REL_TOL
    bad = np.flatnonzero(y.view(np.uint32) != ref.view(np.uint32))
    assert bad.size == 0, f"{bad.size} elements differ from the oracle, first at {bad[:5]}: {y.ravel()[bad[:5]]} vs {ref.ravel()[bad[:5]]}"


def normal(shape, std, seed):
    return (np.random.default_rng(seed).standard_normal(shape) * std).astype(np.float32)


def edge_blocks():
    """Blocks that pin the quantizer's special cases."""
    rows = []
    rows.append(np.zeros(32, np.float32))                                  # d = 0, codes 0
    t = np.zeros(32, np.float32); t[0] = 127.0; t[1:8] = [0.5, -0.5, 1.5, -1.5, 2.5, -2.5, 126.5]
    rows.append(t)                                                         # d = 1: ties round away from zero
    rows.append(np.full(32, -3.0, np.float32))                             # all equal negative -> -127
    t = np.linspace(-1e-6, 1e-6, 32).astype(np.float32); rows.append(t)   # f16 subnormal scale
    t = np.linspace(-1e-38, 2e-38, 32).astype(np.float32); rows.append(t) # f32-subnormal scale, 1/d overflows
    t = np.ones(32, np.float32) * 7e6; t[3] = -9e6; rows.append(t)         # f16 scale overflow to inf
    t = normal(32, 1.0, 5); t[7] = np.nan; rows.append(t)                  # NaN ignored by amax, coded 0
    t = normal(32, 1.0, 6); t[9] = np.inf; rows.append(t)                  # inf
    return np.concatenate(rows)


def test_device_quantizer_bit_exact(ctx):
    x = np.concatenate([normal(32 * 4096, 1.0, 1), normal(32 * 1024, 0.02, 2), edge_blocks()])
    ref = oracle.quantize_q8_0(x)
    host = lq8.quantize_q8_0(x)
    assert np.array_equal(host, ref)
    dx = lq8.DeviceBuffer.from_array(ctx, x)
    db = lq8.DeviceBuffer(ctx, ref.size)
    lq8._check(lq8.lib().lq8_quantize_q8_0_device(ctx.handle, dx.ptr, x.size, db.ptr))
    got = db.download(np.uint8, ref.size)
    dx.free(); db.free()
    bad = np.flatnonzero(got != ref)
    assert bad.size == 0, f"blocks differ at bytes {bad[:8]} (block {bad[0] // 34})"


def act_operand(ctx, source, x, m, k, w=None, eps=1e-6):
    """The GEMM's activation operand for rows x, as GGUF blocks."""
    dx = lq8.DeviceBuffer.from_array(ctx, x)
    dw = lq8.DeviceBuffer.from_array(ctx, w) if w is not None else None
    db = lq8.DeviceBuffer(ctx, m * k // 32 * 34)
    try:
        lq8._check(lq8.lib().lq8_quantize_activations_device(ctx.handle, source, dx.ptr, dw.ptr if dw else None, m, k,
                                                             eps, db.ptr))
        return db.download(np.uint8, m * k // 32 * 34)
    finally:
        dx.free(); db.free()
        if dw:
            dw.free()


def assert_blocks_equal(got, ref):
    bad = np.flatnonzero(got != ref)
    assert bad.size == 0, f"{bad.size} bytes differ, first in block {bad[0] // 34} (byte {bad[0] % 34})"


@pytest.mark.parametrize("m,k", [(512, 1024), (512, 3072), (37, 96), (130, 224)])
def test_activation_quantizer_codes_and_scales(ctx, m, k):
    """k_quantize_act -- the activation quantizer the W8A8 GEMM runs -- gives
    the codes and f16 scales of the Q8_0 quantizer (the oracle's, itself
    pinned by the numpy restatement) for every block, including ragged row
    counts, odd block counts and the special blocks."""
    x = normal((m, k), 1.0, m + k)
    e = edge_blocks()
    x.reshape(-1)[:e.size] = e                      # special blocks in the first rows
    assert_blocks_equal(act_operand(ctx, lq8.ACT_PLAIN, x, m, k), oracle.quantize_q8_0(x))


@pytest.mark.parametrize("m,k", [(512, 1024), (128, 1568), (33, 2112)])
def test_rmsnorm_activation_quantizer(ctx, m, k):
    """k_rms_quantize_act (RmsNorm fused into the quantizer; 2112 takes the
    RmsNorm-rows-then-quantize path of prefill): the blocks of
    quantize(RmsNorm(x)) exactly."""
    x = normal((m, k), 1.0, 7 * k)
    w = (1.0 + 0.1 * normal(k, 1.0, 8 * k)).astype(np.float32)
    ref = oracle.quantize_q8_0(oracle.rms_norm(x, w, 1e-6))
    assert_blocks_equal(act_operand(ctx, lq8.ACT_RMSNORM, x, m, k, w), ref)


@pytest.mark.parametrize("m,inter", [(512, 3072), (45, 800)])
def test_silu_activation_quantizer(ctx, m, inter):
    """k_silu_quantize_act (silu(gate) * up fused into the quantizer): the
    blocks of quantize(silu(g) * u), silu(g) = g / (1 + exp(-g)) with the
    oracle's exp, every step an f32 operation."""
    gu = normal((m, 2 * inter), 2.0, inter)
    g, u = gu[:, :inter], gu[:, inter:]
    e = oracle.expf(-g).reshape(g.shape)
    act = (g / (np.float32(1.0) + e)).astype(np.float32) * u
    assert_blocks_equal(act_operand(ctx, lq8.ACT_SILU_MUL, gu, m, inter), oracle.quantize_q8_0(act))


def test_weight_upload_download_roundtrip(ctx):
    n, k = 200, 96  # ragged: 200 rows is not a multiple of the 64-row tile
    blocks = oracle.quantize_q8_0(normal((n, k), 0.02, 3))
    w = lq8.Q8Weight.from_blocks(ctx, blocks, n, k)
    assert np.array_equal(w.download(), blocks)
    w.free()
    wf = normal((n, k), 0.5, 4)
    w2 = lq8.Q8Weight.quantize(ctx, wf)
    assert np.array_equal(w2.download(), oracle.quantize_q8_0(wf))
    w2.free()


def test_dequantize_rows_exact(ctx):
    n, k = 130, 64
    blocks = oracle.quantize_q8_0(normal((n, k), 0.02, 8))
    w = lq8.Q8Weight.from_blocks(ctx, blocks, n, k)
    y = lq8.DeviceBuffer(ctx, 5 * k * 4)
    lq8._check(lq8.lib().lq8_weight_dequantize_rows_device(ctx.handle, w.handle, 120, 5, y.ptr))
    got = y.download(np.float32, 5 * k)
    ref = oracle.dequantize_q8_0(blocks, n * k).reshape(n, k)[120:125].ravel()
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))
    y.free(); w.free()


def gemv_case(ctx, n, k, seed, x_std=1.0):
    blocks = oracle.quantize_q8_0(normal((n, k), 0.02, seed))
    x = normal(k, x_std, seed + 1000)
    w = lq8.Q8Weight.from_blocks(ctx, blocks, n, k)
    dx = lq8.DeviceBuffer.from_array(ctx, x)
    dy = lq8.DeviceBuffer(ctx, n * 4)
    lq8._check(lq8.lib().lq8_gemv_q8_0_device(ctx.handle, w.handle, dx.ptr, dy.ptr))
    y = dy.download(np.float32, n)
    dx.free(); dy.free(); w.free()
    return y, oracle.gemv_q8_0(blocks, n, k, x)


def test_gemv_3072x1024(ctx):
    y, ref = gemv_case(ctx, 3072, 1024, 11)
    assert_parity(y, ref)


@pytest.mark.parametrize("n,k", [(2048, 1024), (1024, 1024), (1024, 2048), (3072, 1024), (1024, 3072)])
def test_gemv_qwen3_layer_shapes(ctx, n, k):
    y, ref = gemv_case(ctx, n, k, n + k)
    assert_parity(y, ref)


def test_gemv_lm_head_151936x1024(ctx):
    y, ref = gemv_case(ctx, 151936, 1024, 99)
    assert_parity(y, ref)


@pytest.mark.parametrize("n,k", [(1, 32), (65, 96), (100, 288), (7, 8192), (64, 4096), (3, 160)])
def test_gemv_edge_shapes(ctx, n, k):
    y, ref = gemv_case(ctx, n, k, 7 * n + k)
    assert_parity(y, ref)


@pytest.mark.parametrize("n,k", [(48, 12288), (17, 12256)])
def test_gemv_maximum_k(ctx, n, k):
    """The largest input the GEMV stages (12288 = 384 blocks, and one block
    short of it: an odd block count at the limit)."""
    y, ref = gemv_case(ctx, n, k, 3 * n + k)
    assert_parity(y, ref)


@pytest.mark.parametrize("n,k", [(16, 12320), (1024, 17408), (37, 8224 * 3), (5, 131040)])
def test_gemv_above_staging_limit(ctx, n, k):
    """Inputs past the single-stage limit (12288) stream through LDS in
    8192-value stages with the same block tree: bit-exact with the oracle.
    17408 is a down_proj input (intermediate size) of the larger Qwen3
    models; 24672 = 771 blocks (odd, the padding block in the last stage);
    131040 sits one block under the staged limit."""
    y, ref = gemv_case(ctx, n, k, 5 * n + k)
    assert_parity(y, ref)


def test_gemv_limits_and_long_k_linear_forward(ctx):
    """k above 131072 is refused (ShapeMismatch), never run on a fallback;
    Linear::forward at m = 1 (host pointers) on a 17408-long input is the
    oracle's GEMV bit for bit, and the same weight runs the GEMM at m = 2."""
    k = 17408
    blocks = oracle.quantize_q8_0(normal((48, k), 0.02, 5))
    lin = lq8.Linear.new(lq8.Q8Weight.from_blocks(ctx, blocks, 48, k))
    big = lq8.Q8Weight.random(ctx, 16, 131072 + 32, seed=2)
    dx = lq8.DeviceBuffer(ctx, (131072 + 32) * 4)
    dy = lq8.DeviceBuffer(ctx, 16 * 4)
    try:
        with pytest.raises(lq8.ShapeMismatch):
            lq8._check(lq8.lib().lq8_gemv_q8_0_device(ctx.handle, big.handle, dx.ptr, dy.ptr))
        x = normal((2, k), 1.0, 6)
        assert_parity(lin.forward(x[:1]).reshape(48), oracle.gemv_q8_0(blocks, 48, k, x[0]))
        y2 = lin.forward(x)
        assert np.array_equal(y2.view(np.uint32), oracle.gemm_q8_0(blocks, 48, k, x).view(np.uint32))
    finally:
        dx.free(); dy.free(); big.free(); lin.weight.free()


def test_gemv_known_answer(ctx):
    """test_linear_forward (src/attention.rs:605) on Q8_0-exact weights.

    Each weight row holds 127 in its last slot, so d = 1 and the codes are the
    integers themselves; x is zero there.  x @ W^T = [14, 32] exactly, as in
    the reference test, and [14, 32, 50, 68] for src/gpu/gemv.rs:543.
    """
    k = 32
    W = np.zeros((4, k), np.float32)
    W[:, :3] = [[1, 2, 3], [4, 5, 6], [7, 8, 9], [10, 11, 12]]
    W[:, -1] = 127.0
    x = np.zeros(k, np.float32)
    x[:3] = [1, 2, 3]
    w = lq8.Q8Weight.quantize(ctx, W)
    y = lq8.Linear.new(w).forward(x.reshape(1, k))
    assert y.shape == (1, 4)
    assert y.ravel().tolist() == [14.0, 32.0, 50.0, 68.0]
    w.free()


def gemm_case(ctx, m, n, k, seed):
    blocks = oracle.quantize_q8_0(normal((n, k), 0.02, seed))
    x = normal((m, k), 1.0, seed + 1)
    w = lq8.Q8Weight.from_blocks(ctx, blocks, n, k)
    dx = lq8.DeviceBuffer.from_array(ctx, x)
    dy = lq8.DeviceBuffer(ctx, m * n * 4)
    lq8._check(lq8.lib().lq8_gemm_q8_0_device(ctx.handle, w.handle, dx.ptr, m, dy.ptr))
    y = dy.download(np.float32, m * n).reshape(m, n)
    dx.free(); dy.free(); w.free()
    return y, oracle.gemm_q8_0(blocks, n, k, x)


@pytest.mark.parametrize("n,k", [(3072, 1024), (1024, 3072)])
def test_gemm_m512(ctx, n, k):
    y, ref = gemm_case(ctx, 512, n, k, n)
    assert_parity(y, ref)


@pytest.mark.parametrize("m,n,k", [(2, 64, 32), (3, 100, 96), (63, 130, 288), (65, 64, 1024), (130, 192, 256),
                                   (1, 96, 64)])
def test_gemm_ragged(ctx, m, n, k):
    y, ref = gemm_case(ctx, m, n, k, m * 31 + n)
    assert_parity(y, ref)


@pytest.mark.parametrize("n,k", [(2048, 4096), (5120, 2048)])
def test_gemm_small_batch_kernels_agree(ctx, n, k):
    """A batch of 32 rows runs the 16 x 16-tile kernel, one of 96 rows the
    32 x 32 one: both give the oracle's bits, and since an output row depends
    only on its own activation row, the 32 rows they share are equal."""
    blocks = oracle.quantize_q8_0(normal((n, k), 0.02, n + k))
    x = normal((96, k), 1.0, 7)
    w = lq8.Q8Weight.from_blocks(ctx, blocks, n, k)
    out = {}
    for m in (32, 96):
        dx = lq8.DeviceBuffer.from_array(ctx, np.ascontiguousarray(x[:m]))
        dy = lq8.DeviceBuffer(ctx, m * n * 4)
        lq8._check(lq8.lib().lq8_gemm_q8_0_device(ctx.handle, w.handle, dx.ptr, m, dy.ptr))
        out[m] = dy.download(np.float32, m * n).reshape(m, n)
        dx.free(); dy.free()
    w.free()
    ref = oracle.gemm_q8_0(blocks, n, k, x[:32])
    assert np.array_equal(out[32].view(np.uint32), ref.view(np.uint32))
    assert np.array_equal(out[96][:32].view(np.uint32), out[32].view(np.uint32))


def test_gemm_scale_edge_cases(ctx):
    """Activation and weight blocks whose f16 scales are subnormal (amax
    below 127 * 2^-14) or zero, NaN entries (ignored by amax), and a block
    count that is neither even nor a multiple of the 8-block group."""
    m, n, k = 45, 70, 32 * 11
    wf = normal((n, k), 0.02, 40)
    wf[::3] *= np.float32(1e-3)          # weight scales ~5e-7: f16 subnormal
    wf[5, :64] = 0.0                    # two all-zero weight blocks
    x = normal((m, k), 1.0, 41)
    x *= np.float32(10.0) ** -(np.arange(m) % 7).astype(np.float32)[:, None]   # down to 1e-6
    x[3, 32:64] = 0.0                   # zero activation block
    x[4, 7] = np.nan                    # NaN is ignored by amax; its code follows the quantizer
    blocks = oracle.quantize_q8_0(wf)
    w = lq8.Q8Weight.from_blocks(ctx, blocks, n, k)
    dx = lq8.DeviceBuffer.from_array(ctx, x)
    dy = lq8.DeviceBuffer(ctx, m * n * 4)
    lq8._check(lq8.lib().lq8_gemm_q8_0_device(ctx.handle, w.handle, dx.ptr, m, dy.ptr))
    y = dy.download(np.float32, m * n).reshape(m, n)
    dx.free(); dy.free(); w.free()
    ref = oracle.gemm_q8_0(blocks, n, k, x)
    bad = np.flatnonzero(y.view(np.uint32) != ref.view(np.uint32))
    assert bad.size == 0, f"{bad.size} elements differ, first at {bad[:5]}: {y.ravel()[bad[:5]]} vs {ref.ravel()[bad[:5]]}"


def test_gemm_int_blocks_exact(ctx):
    """Per-block int32 sums are exact: with d_w = d_x = 1 (a 127 in every
    block) the f32 result is the integer dot product itself."""
    m, n, k = 64, 64, 256
    rng = np.random.default_rng(4)
    qw = rng.integers(-127, 128, (n, k)).astype(np.float32)
    qx = rng.integers(-127, 128, (m, k)).astype(np.float32)
    qw[:, ::32] = 127.0
    qx[:, ::32] = 127.0
    w = lq8.Q8Weight.quantize(ctx, qw)
    y = lq8.Linear.new(w).forward(qx)
    exact = qx.astype(np.int64) @ qw.astype(np.int64).T
    assert np.array_equal(y.astype(np.int64), exact)
    w.free()


def test_linear_forward_dispatch(ctx):
    n, k = 256, 512
    blocks = oracle.quantize_q8_0(normal((n, k), 0.02, 21))
    lin = lq8.Linear.new(lq8.Q8Weight.from_blocks(ctx, blocks, n, k))
    x1 = normal((1, 1, k), 1.0, 22)
    assert_parity(lin.forward(x1).reshape(1, n), oracle.linear_forward(blocks, n, k, x1))
    x5 = normal((1, 5, k), 1.0, 23)
    y5 = lin.forward(x5)
    assert y5.shape == (1, 5, n)
    assert_parity(y5.reshape(5, n), oracle.linear_forward(blocks, n, k, x5))
    with pytest.raises(lq8.ShapeMismatch):
        lin.forward(normal((2, k + 32), 1.0, 1))
    lin.weight.free()


def test_linear_forward_device_equals_host(ctx):
    """lq8_linear_forward_device (inputs and outputs already in HBM) gives the
    bits of lq8_linear_forward, on the GEMV (m = 1) and GEMM (m > 1) paths."""
    n, k = 384, 1024
    blocks = oracle.quantize_q8_0(normal((n, k), 0.02, 31))
    lin = lq8.Linear.new(lq8.Q8Weight.from_blocks(ctx, blocks, n, k))
    try:
        for m in (1, 5):
            x = normal((m, k), 1.0, 32 + m)
            host = lin.forward(x.reshape(1, m, k)).reshape(m, n)
            dx = lq8.DeviceBuffer.from_array(ctx, x)
            dy = lq8.DeviceBuffer(ctx, m * n * 4)
            try:
                lin.forward_device(dx, m, dy)
                dev = dy.download(np.float32, m * n).reshape(m, n)
            finally:
                dx.free()
                dy.free()
            assert np.array_equal(dev.view(np.uint32), host.view(np.uint32)), m
    finally:
        lin.weight.free()


def test_grouped_gemv(ctx):
    shapes = [(2048, 1024), (1024, 1024), (1024, 2048), (3072, 1024), (1024, 3072), (100, 96)]
    probs, refs, bufs, ws = [], [], [], []
    for i, (n, k) in enumerate(shapes):
        blocks = oracle.quantize_q8_0(normal((n, k), 0.02, 300 + i))
        x = normal(k, 1.0, 400 + i)
        w = lq8.Q8Weight.from_blocks(ctx, blocks, n, k)
        dx, dy = lq8.DeviceBuffer.from_array(ctx, x), lq8.DeviceBuffer(ctx, n * 4)
        probs.append((w, dx, dy))
        refs.append(oracle.gemv_q8_0(blocks, n, k, x))
        bufs += [dx, dy]
        ws.append(w)
    lq8.gemv_grouped_device(ctx, probs)
    for (w, dx, dy), ref in zip(probs, refs):
        assert_parity(dy.download(np.float32, w.n_out), ref)
    for b in bufs:
        b.free()
    for w in ws:
        w.free()


def test_errors_no_fallback(ctx):
    with pytest.raises(lq8.ShapeMismatch):
        lq8.Q8Weight.quantize(ctx, np.zeros((4, 33), np.float32))
    w = lq8.Q8Weight.random(ctx, 64, 64, seed=1)
    stale = w.handle
    w.free()
    with pytest.raises(lq8.InvalidArgument):
        lq8._check(lq8.lib().lq8_weight_free(stale))
    with pytest.raises(lq8.InvalidArgument):
        lq8._check(lq8.lib().lq8_gemv_q8_0_device(ctx.handle, stale, None, None))


def test_gemv_repeated_and_graph_calls(ctx):
    """Repeated calls, interleaved shapes and graph replays give the oracle's
    bits every time."""
    cases = []
    for i, (n, k) in enumerate([(1024, 3072), (64, 2048), (1024, 1024), (200, 768)]):
        blocks = oracle.quantize_q8_0(normal((n, k), 0.02, 500 + i))
        x = normal(k, 1.0, 600 + i)
        w = lq8.Q8Weight.from_blocks(ctx, blocks, n, k)
        cases.append((w, lq8.DeviceBuffer.from_array(ctx, x), lq8.DeviceBuffer(ctx, 4 * n),
                      oracle.gemv_q8_0(blocks, n, k, x)))
    for _ in range(3):
        for w, dx, dy, ref in cases:
            lq8._check(lq8.lib().lq8_gemv_q8_0_device(ctx.handle, w.handle, dx.ptr, dy.ptr))
        for w, dx, dy, ref in cases:
            assert_parity(dy.download(np.float32, w.n_out), ref)
    lq8.bench_gemv(ctx, [(w, dx, dy) for w, dx, dy, _ in cases], mode=2, reps=5)
    for w, dx, dy, ref in cases:
        assert_parity(dy.download(np.float32, w.n_out), ref)
        dx.free(); dy.free(); w.free()


@pytest.mark.parametrize("case", MATMUL_KNOWN, ids=[c[0].split()[1] for c in MATMUL_KNOWN])
def test_matmul_known_answers_gpu(ctx, case):
    """The reference's matmul known answers through Linear::forward: the
    W8A8 GEMM for m > 1 rows and the W8A32 GEMV for each row."""
    _, a, b, want = case
    x, w = exact_operands(a, b)
    q = lq8.Q8Weight.quantize(ctx, w)
    lin = lq8.Linear.new(q)
    want = np.asarray(want, np.float32)
    assert np.array_equal(lin.forward(x), want)
    for r in range(x.shape[0]):
        assert np.array_equal(lin.forward(x[r:r + 1]), want[r:r + 1])
    q.free()
