"""CPU: the oracle's Qwen3-MoE decoder layer, pinned.

- Router: expert choice against a brute-force sort of the scores (softmax is
  monotonic; ties go to the lower index) and the weights against a float64
  softmax renormalised over the chosen experts.
- Layer structure: with one expert and top-1 routing the MoE layer is the
  dense Qwen3 decoder layer (weight 1 exactly), so it must equal the dense
  oracle layer -- itself pinned against the reference's numerics -- bit for
  bit, position by position.
- Combine: identical experts with top_k = num_experts give h2 + y (the
  renormalised weights sum to 1), up to rounding.
- Batch: the attention projections of a batch of T > 1 tokens are one
  Linear::forward each (the W8A8 GEMM), so a token's bits do not depend on
  the other tokens of its batch; with the activation quantization switched
  off a batch equals its sequences run one by one.
"""
from dataclasses import dataclass

import numpy as np
import pytest

import oracle


@dataclass
class MoeCfg:
    hidden_size: int = 256
    num_heads: int = 4
    num_kv_heads: int = 2
    head_dim: int = 128
    num_experts: int = 8
    top_k: int = 2
    expert_intermediate_size: int = 96
    max_positions: int = 80
    max_batch: int = 4
    num_layers: int = 1
    rms_norm_eps: float = 1e-6
    rope_theta: float = 1e6


@dataclass
class DenseCfg:
    vocab_size: int = 64
    hidden_size: int = 256
    intermediate_size: int = 96
    num_hidden_layers: int = 1
    num_attention_heads: int = 4
    num_key_value_heads: int = 2
    head_dim: int = 128
    max_position_embeddings: int = 80
    rms_norm_eps: float = 1e-6
    rope_theta: float = 1e6


def q8(rng, shape, std=0.02):
    return oracle.quantize_q8_0((rng.standard_normal(shape) * std).astype(np.float32))


def moe_tensors(cfg, seed):
    rng = np.random.default_rng(seed)
    H, I, hd, E = cfg.hidden_size, cfg.expert_intermediate_size, cfg.head_dim, cfg.num_experts
    QD, KD = cfg.num_heads * hd, cfg.num_kv_heads * hd
    out = []
    for _ in range(cfg.num_layers):
        out += [1.0 + 0.1 * rng.standard_normal(H).astype(np.float32), 1.0 + 0.1 * rng.standard_normal(H).astype(np.float32),
                1.0 + 0.1 * rng.standard_normal(hd).astype(np.float32), 1.0 + 0.1 * rng.standard_normal(hd).astype(np.float32),
                q8(rng, (QD, H)), q8(rng, (KD, H)), q8(rng, (KD, H)), q8(rng, (H, QD))]
        out += [q8(rng, (I, H)) for _ in range(E)] + [q8(rng, (I, H)) for _ in range(E)] + \
               [q8(rng, (H, I)) for _ in range(E)]
    return [np.ascontiguousarray(t, dtype=np.float32) if t.dtype != np.uint8 else t for t in out]


def test_route_matches_sort_and_f64_softmax():
    rng = np.random.default_rng(1)
    T, E, K = 40, 128, 8
    s = rng.standard_normal((T, E)).astype(np.float32)
    ids, w = oracle.moe_route(s, K)
    for t in range(T):
        order = sorted(range(E), key=lambda i: (-float(s[t, i]), i))[:K]
        assert ids[t].tolist() == order
        p = np.exp(s[t].astype(np.float64) - s[t].max())
        p /= p.sum()
        ref = p[order] / p[order].sum()
        assert np.allclose(w[t], ref, rtol=2e-6, atol=0)
        assert abs(float(w[t].astype(np.float64).sum()) - 1.0) < 1e-6


def test_route_ties_go_to_lower_index():
    s = np.zeros((2, 16), np.float32)
    s[0, [3, 9, 12]] = 2.0
    s[1, :] = 1.0
    ids, w = oracle.moe_route(s, 4)
    assert ids[0].tolist() == [3, 9, 12, 0]
    assert ids[1].tolist() == [0, 1, 2, 3]
    assert np.all(w[1] == np.float32(0.25))


def test_route_all_experts_weights_are_softmax():
    rng = np.random.default_rng(2)
    s = rng.standard_normal((3, 8)).astype(np.float32)
    ids, w = oracle.moe_route(s, 8)
    for t in range(3):
        p = np.exp(s[t].astype(np.float64) - s[t].max())
        p /= p.sum()
        assert np.allclose(w[t], p[ids[t]], rtol=2e-6)


def test_single_expert_layer_equals_dense_layer():
    dense = DenseCfg()
    cfg = MoeCfg(num_experts=1, top_k=1, expert_intermediate_size=dense.intermediate_size, max_batch=1)
    mt = moe_tensors(cfg, 3)
    rng = np.random.default_rng(4)
    embed = q8(rng, (dense.vocab_size, dense.hidden_size), 1.0)
    # dense table: embed, final norm, then the layer's 11 tensors in the same order
    dt = [embed, np.ones(dense.hidden_size, np.float32)] + mt[:8] + [mt[8], mt[9], mt[10]]
    dm = oracle.Model(dense, dt)
    mm = oracle.MoeStack(cfg, mt)
    ids = [5, 17, 42, 9, 63, 1]
    for p, tok in enumerate(ids):
        hidden, _, _ = dm.forward_with_intermediates([tok], p)
        out = mm.forward(hidden[0], np.zeros((1, 1, 1), np.float32), [p])
        assert np.array_equal(out.view(np.uint32), hidden[1].view(np.uint32)), f"position {p}"
    dm.close()
    mm.close()


def test_identical_experts_combine_to_one_expert():
    cfg1 = MoeCfg(num_experts=1, top_k=1, max_batch=1)
    cfg4 = MoeCfg(num_experts=4, top_k=4, max_batch=1)
    t1 = moe_tensors(cfg1, 6)
    t4 = t1[:8] + [t1[8]] * 4 + [t1[9]] * 4 + [t1[10]] * 4
    m1, m4 = oracle.MoeStack(cfg1, t1), oracle.MoeStack(cfg4, t4)
    x = np.random.default_rng(7).standard_normal((1, cfg1.hidden_size)).astype(np.float32)
    scores = np.random.default_rng(8).standard_normal((1, 1, 4)).astype(np.float32)
    y1 = m1.forward(x, np.zeros((1, 1, 1), np.float32), [0])
    y4 = m4.forward(x, scores, [0])
    assert np.allclose(y4, y1, rtol=0, atol=1e-6 * float(np.abs(y1).max()))
    m1.close()
    m4.close()


def moe_batch_case(T=3):
    cfg = MoeCfg(num_layers=2)
    tens = moe_tensors(cfg, 9)
    rng = np.random.default_rng(10)
    x = rng.standard_normal((T, cfg.hidden_size)).astype(np.float32)
    scores = rng.standard_normal((cfg.num_layers, T, cfg.num_experts)).astype(np.float32)
    return cfg, tens, x, scores, [0, 7, 70][:T]


def test_batch_result_independent_of_the_other_tokens():
    """Each token of a batch of 3 gets the same bits in a batch of 2 with a
    different partner (per-row activation quantization, per-element GEMM)."""
    cfg, tens, x, scores, pos = moe_batch_case()
    batch = oracle.MoeStack(cfg, tens)
    yb = batch.forward(x, scores, pos)
    batch.close()
    T = len(pos)
    for t in range(T):
        u = (t + 1) % T
        pair = oracle.MoeStack(cfg, tens)
        yp = pair.forward(x[[t, u]], scores[:, [t, u]], [pos[t], pos[u]])
        pair.close()
        assert np.array_equal(yp[0].view(np.uint32), yb[t].view(np.uint32)), t


def test_batch_equals_sequences_one_by_one_without_activation_quantization():
    cfg, tens, x, scores, pos = moe_batch_case()
    oracle.set_activation_quantization(False)
    try:
        batch = oracle.MoeStack(cfg, tens)
        yb = batch.forward(x, scores, pos)
        batch.close()
        for t in range(len(pos)):
            one = oracle.MoeStack(cfg, tens)
            yt = one.forward(x[t:t + 1], scores[:, t:t + 1], [pos[t]])
            one.close()
            assert np.array_equal(yt[0].view(np.uint32), yb[t].view(np.uint32))
    finally:
        oracle.set_activation_quantization(True)


def test_batch_differs_from_single_only_by_activation_quantization():
    """With the quantization on, a token's batched result stays within the
    error Q8_0 activations add (~1e-2 relative) of its single-token result."""
    cfg, tens, x, scores, pos = moe_batch_case()
    batch = oracle.MoeStack(cfg, tens)
    yb = batch.forward(x, scores, pos)
    batch.close()
    for t in range(len(pos)):
        one = oracle.MoeStack(cfg, tens)
        yt = one.forward(x[t:t + 1], scores[:, t:t + 1], [pos[t]])
        one.close()
        err = np.max(np.abs(yt[0] - yb[t])) / np.max(np.abs(yt[0]))
        assert 0 < err < 2e-2, err
