"""CPU: the oracle's decoder numerics against the reference's own unit tests
(closed forms) and invariants, and the tiny-model golden tokens."""
import ctypes
import ctypes.util
import os

import numpy as np
import pytest

import lq8
import oracle

BF16_TOL = 1e-2  # rms_norm.rs tests compare bf16 outputs with this tolerance


def norm(x, w=None, eps=1e-6):
    x = np.asarray(x, np.float32).reshape(1, -1)
    w = np.ones(x.shape[1], np.float32) if w is None else np.asarray(w, np.float32)
    return oracle.rms_norm(x, w, eps)[0]


def test_rms_norm_reference_cases():
    """src/rms_norm.rs:199-440 known answers."""
    assert np.allclose(norm([1, 1, 1]), [1, 1, 1], atol=BF16_TOL)
    r = np.sqrt(np.float32(4.0 / 3.0))
    assert np.allclose(norm([2, 0, 0]), [2 / r, 0, 0], atol=BF16_TOL)
    assert np.allclose(norm([1, 1, 1], [2, 3, 4]), [2, 3, 4], atol=BF16_TOL)
    assert np.all(norm([0, 0, 0]) == 0)                                  # eps guards 0/0
    r = np.sqrt(np.float32((1e6 + 4e6 + 9e6) / 3))
    out = norm([1000, 2000, 3000])
    assert np.allclose(out, [1000 / r, 2000 / r, 3000 / r], atol=BF16_TOL) and np.all(np.isfinite(out))
    r = np.sqrt(np.float32(14.0 / 3.0))
    assert np.allclose(norm([-1, 2, -3]), [-1 / r, 2 / r, -3 / r], atol=BF16_TOL)


def test_rms_norm_output_is_bf16_and_unit_rms():
    x = np.random.default_rng(0).standard_normal(1024).astype(np.float32) * 37
    y = norm(x)
    assert np.array_equal(y, oracle.bf16_round(y))                       # bf16 outputs
    assert abs(np.sqrt(np.mean(y.astype(np.float64) ** 2)) - 1.0) < 5e-3


def test_rope_tables_reference_values():
    """src/rope.rs:514: head_dim 4, theta 1e4: cos[1,0] = cos[1,1] = cos(1)."""
    c, s = oracle.rope_tables(4, 100, 10000.0)
    assert c[0, 0] == 1.0 and s[0, 0] == 0.0
    assert c[1, 0] == np.float32(np.cos(1.0)) and c[1, 1] == np.float32(np.cos(1.0))
    assert s[1, 0] == np.float32(np.sin(1.0)) and s[1, 1] == np.float32(np.sin(1.0))
    # Qwen3 layout (head_dim 128): frequency i sits at columns 2i and 2i+1
    c, s = oracle.rope_tables(128, 8, 1e6)
    inv = 1.0 / (1e6 ** (np.arange(32) * 2 / 64.0))
    assert np.array_equal(c[5, 0::2], (np.cos(5 * inv)).astype(np.float32))
    assert np.array_equal(c[5, 1::2], c[5, 0::2])


def test_rope_identity_at_zero_and_norm_preserving():
    """src/rope.rs:341 (position 0 is the identity) and :373 (norm preserved)."""
    c, s = oracle.rope_tables(4, 10, 10000.0)
    x = np.array([1, 2, 3, 4], np.float32).reshape(1, 1, 4)
    assert np.array_equal(oracle.rope_apply(x, c, s, 0), x)
    c, s = oracle.rope_tables(128, 64, 1e6)
    x = np.random.default_rng(1).standard_normal((3, 5, 128)).astype(np.float32)
    y = oracle.rope_apply(x, c, s, 7)
    assert np.allclose(np.linalg.norm(y, axis=-1), np.linalg.norm(x, axis=-1), rtol=1e-5)
    # the rotate-half pairing: out[d] = x[d] c - x[d+64] s, with c from column 2*(d//2)
    d, pos = 5, 7 + 2
    assert y[0, 2, d] == np.float32(x[0, 2, d] * c[pos, 4] - x[0, 2, d + 64] * s[pos, 4])


TINY = lq8.Qwen3Config(vocab_size=512, hidden_size=128, intermediate_size=256, num_hidden_layers=2,
                       num_attention_heads=2, num_key_value_heads=1, head_dim=128, max_position_embeddings=64)


@pytest.fixture(scope="module")
def tiny():
    m = oracle.Model(TINY, oracle.random_q8_tensors(TINY, seed=77))
    yield m
    m.close()


def test_tiny_model_golden(tiny):
    g = np.load(os.path.join(os.path.dirname(__file__), "golden", "q8_0_golden.npz"))
    tiny.clear_kv_cache()
    assert np.array_equal(tiny.forward(g["tiny_prompt"], 0).view(np.uint32), g["tiny_logits0"].view(np.uint32))
    toks, margins = tiny.generate_greedy(g["tiny_prompt"], 12)
    assert toks.tolist() == g["tiny_tokens"].tolist()
    assert np.all(margins >= 0)


def test_generate_equals_manual_loop(tiny):
    """generate() = prefill, argmax, then one-token forwards at offset
    prefill_len + generated - 1 (src/generate.rs:611-664)."""
    prompt = np.array([3, 1, 4, 1, 5, 9, 2, 6], np.uint32)
    toks, _ = tiny.generate_greedy(prompt, 6)
    tiny.clear_kv_cache()
    logits = tiny.forward(prompt, 0)
    manual = [oracle.argmax_last(logits)]
    for t in range(1, 6):
        logits = tiny.forward([manual[-1]], len(prompt) + t - 1)
        manual.append(oracle.argmax_last(logits))
    assert toks.tolist() == manual


def test_kv_offset_and_vocab_checks(tiny):
    tiny.clear_kv_cache()
    tiny.forward([1, 2], 0)
    with pytest.raises(ValueError):
        tiny.forward([3], 5)            # offset must equal the cached length
    with pytest.raises(ValueError):
        tiny.forward([TINY.vocab_size], 2)


def test_intermediates_consistent(tiny):
    tiny.clear_kv_cache()
    ids = np.array([10, 20, 30, 40], np.uint32)
    hidden, fin, logits = tiny.forward_with_intermediates(ids, 0)
    assert hidden.shape == (TINY.num_hidden_layers + 1, 4, TINY.hidden_size)
    emb = oracle.dequantize_q8_0(oracle.random_q8_tensors(TINY, seed=77)[0], TINY.vocab_size * TINY.hidden_size)
    assert np.array_equal(hidden[0], emb.reshape(TINY.vocab_size, -1)[ids])
    assert np.array_equal(fin, oracle.rms_norm(hidden[-1], np.ones(TINY.hidden_size, np.float32), TINY.rms_norm_eps))


def test_sequential_sum_order_close_to_canonical():
    """The canonical summation orders stay within f32 rounding of the
    reference's plain sequential sums on the same model and prompt."""
    m = oracle.Model(TINY, oracle.random_q8_tensors(TINY, seed=78))
    ids = np.arange(5, dtype=np.uint32) * 11
    a = m.forward(ids, 0)
    oracle.set_sequential_sums(True)
    try:
        m.clear_kv_cache()
        b = m.forward(ids, 0)
    finally:
        oracle.set_sequential_sums(False)
        m.close()
    assert np.max(np.abs(a - b)) <= 1e-3 * np.max(np.abs(b))


def test_reference_arithmetic_mode_close_to_canonical():
    """The reference's own arithmetic -- plain sequential sums and the C
    library's expf for the softmax and SiLU (glibc's on linux-gnu, which
    Rust's f32::exp calls) -- against the canonical orders and orc_expf:
    logits within f32 rounding and the same greedy pick.  The switch is
    pinned by SiLU: in the mode, silu(x) is x / (1 + expf(-x)) with the
    library's expf, bit for bit."""
    libm = ctypes.CDLL(ctypes.util.find_library("m"))
    libm.expf.restype = ctypes.c_float
    libm.expf.argtypes = [ctypes.c_float]
    xs = np.linspace(-30.0, 30.0, 2001, dtype=np.float32)
    m = oracle.Model(TINY, oracle.random_q8_tensors(TINY, seed=79))
    ids = np.arange(6, dtype=np.uint32) * 13
    a = m.forward(ids, 0)
    oracle.set_sequential_sums(True)
    oracle.set_libm_exp(True)
    try:
        for x in xs:
            x = np.float32(x)
            want = np.float32(x / (np.float32(1.0) + np.float32(libm.expf(-x))))
            assert np.float32(oracle.silu(float(x))).view(np.uint32) == want.view(np.uint32), float(x)
        m.clear_kv_cache()
        b = m.forward(ids, 0)
    finally:
        oracle.set_libm_exp(False)
        oracle.set_sequential_sums(False)
        m.close()
    assert np.max(np.abs(a - b)) <= 1e-3 * np.max(np.abs(b))
    assert int(np.argmax(a)) == int(np.argmax(b))


VARIED = lq8.Qwen3Config(vocab_size=1024, hidden_size=256, intermediate_size=512, num_hidden_layers=2,
                         num_attention_heads=4, num_key_value_heads=2, head_dim=128, max_position_embeddings=96)


def test_reference_loop_as_written_diverges_from_feeding_the_latest_token():
    """src/generate.rs:632-650: the `let next_token` inside the loop body
    shadows the outer binding only for the rest of that iteration, so each
    decode step of the reference forwards the FIRST generated token.  On a
    model whose greedy tokens vary, that loop (feed_first) and the loop that
    forwards the latest token -- the library's default -- part after the
    second token; each equals its manual restatement."""
    m = oracle.Model(VARIED, oracle.random_q8_tensors(VARIED, seed=3, layer_std=0.08, norm_jitter=0.1))
    prompt = np.random.default_rng(1).integers(0, VARIED.vocab_size, 16).astype(np.uint32)
    try:
        latest, _ = m.generate_greedy(prompt, 24)
        first, _ = m.generate_greedy(prompt, 24, feed_first=True)
        m.clear_kv_cache()
        logits = m.forward(prompt, 0)
        manual = [oracle.argmax_last(logits)]
        for t in range(1, 24):
            manual.append(oracle.argmax_last(m.forward([manual[0]], prompt.size + t - 1)))
    finally:
        m.close()
    assert first.tolist() == manual
    assert latest[:2].tolist() == first[:2].tolist()      # same prefill token and first decode input
    assert latest.tolist() != first.tolist()
    assert len(set(latest.tolist())) >= 10                 # the model's tokens really vary
