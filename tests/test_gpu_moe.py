"""GPU parity of the Qwen3-MoE decoder layers against the CPU oracle, through
the C ABI: hidden states and routing bit-exact with the oracle, for batch 1
(fused attention combine in the o-projection) and batched decode (combine
kernel, W8A8 GEMMs for the attention projections, multi-vector expert GEMVs),
across attention segment boundaries, and batch invariance (a token's bits do
not depend on the other tokens of its batch)."""
import numpy as np
import pytest

import lq8
import oracle
from test_oracle_moe import MoeCfg, moe_tensors

pytestmark = pytest.mark.gpu


def lq8_cfg(c):
    return lq8.MoeConfig(c.hidden_size, c.num_heads, c.num_kv_heads, c.head_dim, c.num_experts, c.top_k,
                         c.expert_intermediate_size, c.max_positions, c.max_batch, c.num_layers, c.rms_norm_eps,
                         c.rope_theta)


def assert_bits(a, b, what):
    bad = np.flatnonzero(a.view(np.uint32) != b.view(np.uint32))
    assert bad.size == 0, f"{what}: {bad.size} elements differ, first at {bad[:5]}: {a.ravel()[bad[:5]]} vs {b.ravel()[bad[:5]]}"


def run_steps(ctx, cfg, tens, T, pos0, steps, seed):
    gpu = lq8.Qwen3MoeLayers.load(ctx, lq8_cfg(cfg), tens)
    orc = oracle.MoeStack(cfg, tens)
    rng = np.random.default_rng(seed)
    pos = np.array(pos0, np.int32)
    for step in range(steps):
        x = rng.standard_normal((T, cfg.hidden_size)).astype(np.float32)
        scores = rng.standard_normal((cfg.num_layers, T, cfg.num_experts)).astype(np.float32)
        y = gpu.forward(x, scores, pos)
        ref = orc.forward(x, scores, pos.astype(np.uint32))
        assert np.isfinite(y).all() and not np.array_equal(y, x)
        assert_bits(y, ref, f"step {step} hidden")
        ids, w = gpu.routing(T)
        for l in range(cfg.num_layers):
            rid, rw = oracle.moe_route(scores[l], cfg.top_k)
            assert np.array_equal(ids[l], rid), f"step {step} layer {l} experts"
            assert_bits(w[l], rw, f"step {step} layer {l} weights")
        pos += 1
    gpu.free()
    orc.close()


def test_moe_batch1_across_segments(ctx):
    cfg = MoeCfg(num_experts=16, top_k=4, max_positions=200, max_batch=4, num_layers=2)
    tens = moe_tensors(cfg, 21)
    run_steps(ctx, cfg, tens, 1, [62], 4, 22)      # positions 62..65 cross the 64-position segment edge


@pytest.mark.parametrize("pos0,T", [([100], 1), ([4150], 1), ([4150, 90], 2)])
def test_moe_long_max_positions(ctx, pos0, T):
    """Qwen3-30B-A3B's heads (32 query, 4 kv) at max_positions 40960 (640
    attention segments): the batch-1 o projection's segment combine holds the
    coefficients of at most 64 segments in LDS at a time, so it fits; position
    4150 combines 65 segments in two batches (batch 1) or through the combine
    kernel (batch 2)."""
    cfg = MoeCfg(num_heads=32, num_kv_heads=4, num_experts=16, top_k=4, max_positions=40960, max_batch=2,
                 num_layers=2)
    run_steps(ctx, cfg, moe_tensors(cfg, 31), T, pos0, 2, 32)


def test_moe_batched_decode(ctx):
    cfg = MoeCfg(num_experts=16, top_k=4, max_positions=200, max_batch=8, num_layers=2)
    tens = moe_tensors(cfg, 23)
    run_steps(ctx, cfg, tens, 5, [0, 3, 63, 64, 130], 3, 24)


@pytest.mark.parametrize("hidden", [320, 288])
def test_moe_partial_groups_odd_blocks(ctx, hidden):
    """Shapes whose block-pair groups end part-way: hidden 320 (10 blocks, 5
    pairs in groups of 2: the last group holds one pair; 20 output tiles, so
    the batched down projection takes 4 tiles per workgroup) or 288 (9
    blocks, the last pair half padding; 18 tiles: one per workgroup), and
    expert intermediate 672 (21 blocks; 11 pairs in groups of 4: the last
    holds three), with 6 experts top-4 over 7 sequences so that experts see 3
    to 7 vectors (pairs of vectors, a vector left over, more than one staging
    pass)."""
    cfg = MoeCfg(hidden_size=hidden, expert_intermediate_size=672, num_experts=6, top_k=4, max_positions=96,
                 max_batch=8, num_layers=2)
    tens = moe_tensors(cfg, 41)
    run_steps(ctx, cfg, tens, 7, [0, 1, 2, 40, 63, 64, 90], 2, 42)
    run_steps(ctx, cfg, tens, 8, [3] * 8, 1, 43)


@pytest.mark.parametrize("hidden,inter,nh,nkv,ne,k", [
    (288, 160, 6, 2, 8, 2),    # gate|up: 40 tiles, the last workgroup takes one; odd block counts; 3 q heads per kv head
    (256, 1536, 4, 2, 16, 8),  # down: 8 ranks x 6 groups = 48 items, the prefetching path
    (320, 64, 4, 4, 4, 1),     # one routed expert, 8 tiles (3, 3, 2); one q head per kv head
    (288, 672, 4, 2, 6, 4),    # down with every item in flight, 21 blocks (11 pairs in groups of 4, a padding block)
])
def test_moe_batch1_shapes(ctx, hidden, inter, nh, nkv, ne, k):
    """Batch 1 through shapes at the edges of its kernels: the gate|up tile
    list (3 tiles per workgroup) ending part-way, block counts with a padding
    block, the down kernel within and past its every-item-in-flight limits
    (groups of 4 pairs, at most 32 items), and the
    attention's head groups falling back to whole kv-head groups (an odd or a
    single query head per kv head); bit-exact with the oracle across a
    segment edge."""
    cfg = MoeCfg(hidden_size=hidden, expert_intermediate_size=inter, num_heads=nh, num_kv_heads=nkv,
                 num_experts=ne, top_k=k, max_positions=96, max_batch=2, num_layers=2)
    tens = moe_tensors(cfg, 61 + inter)
    run_steps(ctx, cfg, tens, 1, [61], 4, 62 + hidden)


def test_moe_batch_invariance(ctx):
    """A token's bits do not depend on the other tokens of its batch: each
    sequence of a batch of 6 equals its result in a batch of 2 with another
    partner (the batched attention projections are per-row W8A8 GEMMs, the
    experts per-token GEMVs)."""
    cfg = MoeCfg(num_experts=16, top_k=4, max_positions=200, max_batch=8, num_layers=2)
    tens = moe_tensors(cfg, 25)
    T = 6
    rng = np.random.default_rng(26)
    x = rng.standard_normal((T, cfg.hidden_size)).astype(np.float32)
    scores = rng.standard_normal((cfg.num_layers, T, cfg.num_experts)).astype(np.float32)
    pos = np.array([5, 5, 70, 1, 0, 199], np.int32)
    gpu = lq8.Qwen3MoeLayers.load(ctx, lq8_cfg(cfg), tens)
    yb = gpu.forward(x, scores, pos)
    gpu.free()
    for t in range(T):
        u = (t + 3) % T
        pair = lq8.Qwen3MoeLayers.load(ctx, lq8_cfg(cfg), tens)
        yp = pair.forward(x[[t, u]], scores[:, [t, u]], pos[[t, u]])
        assert_bits(yp[0], yb[t], f"sequence {t}")
        pair.free()


def test_moe_forward_device_equals_host(ctx):
    """lq8_moe_forward_device (hidden state, scores and positions in HBM, the
    hidden state updated in place) gives the bits of lq8_moe_forward, at
    batch 1 and 5, from a cleared cache."""
    cfg = MoeCfg(num_experts=16, top_k=4, max_positions=96, max_batch=8, num_layers=2)
    gpu = lq8.Qwen3MoeLayers.load(ctx, lq8_cfg(cfg), moe_tensors(cfg, 51))
    rng = np.random.default_rng(52)
    try:
        for T, pos in ((1, [7]), (5, [0, 9, 63, 64, 90])):
            x = rng.standard_normal((T, cfg.hidden_size)).astype(np.float32)
            scores = rng.standard_normal((cfg.num_layers, T, cfg.num_experts)).astype(np.float32)
            p = np.array(pos, np.int32)
            gpu.clear_kv_cache()
            host = gpu.forward(x, scores, p)
            gpu.clear_kv_cache()
            dh = lq8.DeviceBuffer.from_array(ctx, x)
            ds = lq8.DeviceBuffer.from_array(ctx, scores)
            dp = lq8.DeviceBuffer.from_array(ctx, p)
            try:
                gpu.forward_device(dh, ds, dp, T)
                dev = dh.download(np.float32, T * cfg.hidden_size).reshape(T, cfg.hidden_size)
            finally:
                dh.free()
                ds.free()
                dp.free()
            assert_bits(dev, host, f"T={T}")
    finally:
        gpu.free()


def test_moe_rejects_bad_calls(ctx):
    cfg = MoeCfg(num_experts=16, top_k=4, max_positions=64, max_batch=2)
    gpu = lq8.Qwen3MoeLayers.load(ctx, lq8_cfg(cfg), moe_tensors(cfg, 27))
    x = np.zeros((3, cfg.hidden_size), np.float32)
    with pytest.raises(lq8.ShapeMismatch):
        gpu.forward(x, np.zeros((1, 3, 16), np.float32), [0, 0, 0])      # T above max_batch
    with pytest.raises(lq8.DimOutOfRange):
        gpu.forward(x[:1], np.zeros((1, 1, 16), np.float32), [64])       # position outside the cache
    gpu.free()
    bad = lq8_cfg(MoeCfg(num_experts=4, top_k=8))
    with pytest.raises(lq8.ShapeMismatch):
        lq8.Qwen3MoeLayers.random(ctx, bad, seed=1)


def test_moe_expert_weights_round_trip(ctx):
    """The expert gate and up weights are stored interleaved by 8 rows per
    16-row tile; loading host tensors and exporting them gives the same
    bytes (intermediate size 96: 12 such tiles per expert, 2 layers)."""
    cfg = MoeCfg(num_experts=8, top_k=2, expert_intermediate_size=96, max_positions=64, max_batch=2,
                 num_layers=2)
    tens = moe_tensors(cfg, 41)
    gpu = lq8.Qwen3MoeLayers.load(ctx, lq8_cfg(cfg), tens)
    back = gpu.export_all()
    assert len(back) == len(tens)
    for i, (a, b) in enumerate(zip(tens, back)):
        assert np.array_equal(np.asarray(a).view(np.uint8).ravel(), np.asarray(b).view(np.uint8).ravel()), f"tensor {i}"
    gpu.free()


@pytest.mark.parametrize("T,pos0", [(1, 0), (32, 0), (1, 126), (32, 126)])
def test_moe_qwen3_30b_a3b_layer(ctx, T, pos0):
    """One full-size Qwen3-30B-A3B-style layer (hidden 2048, 32/4 heads, 128
    experts, top-8, expert intermediate 768), random-init on the device,
    exported and replayed on the oracle: three decode steps bit-exact.  From
    position 126 the steps reach positions 126..134 (T = 32: position
    126 + t % 7 for sequence t), so attention combines three 64-position
    segments, as at the bench's position 128."""
    cfg = MoeCfg(hidden_size=2048, num_heads=32, num_kv_heads=4, num_experts=128, top_k=8,
                 expert_intermediate_size=768, max_positions=256, max_batch=32, num_layers=1)
    gpu = lq8.Qwen3MoeLayers.random(ctx, lq8_cfg(cfg), seed=2026)
    tens = gpu.export_all()
    orc = oracle.MoeStack(cfg, tens)
    rng = np.random.default_rng(31 + T + pos0)
    pos = (pos0 + np.arange(T) % 7).astype(np.int32)
    for step in range(3):
        x = rng.standard_normal((T, cfg.hidden_size)).astype(np.float32)
        scores = rng.standard_normal((1, T, cfg.num_experts)).astype(np.float32)
        y = gpu.forward(x, scores, pos)
        ref = orc.forward(x, scores, pos.astype(np.uint32))
        assert np.isfinite(y).all() and not np.array_equal(y, x)
        assert_bits(y, ref, f"T={T} step {step}")
        pos += 1
    orc.close()
    gpu.free()
