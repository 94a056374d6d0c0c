"""GPU sampling (lq8_sample_device, lq8_generate) against the oracle's
restatement of the same rule: the chosen token is identical for every
configuration, step and seed, at the Qwen3 vocabulary (151936) and at small
vocabularies full of ties; sampled generation gives the oracle's tokens with
and without the captured graph."""
import os

import numpy as np
import pytest

import lq8
import oracle

pytestmark = pytest.mark.gpu

CONFIGS = [
    # temperature, top_k, top_p, repetition_penalty
    (1.0, 0, 1.0, 1.0),
    (0.7, 50, 0.9, 1.3),
    (1.5, 0, 0.95, 1.0),
    (0.8, 0, 0.5, 1.1),
    (1.0, 1, 1.0, 1.0),
    (2.0, 1000, 1.0, 1.0),
    (0.0, 0, 1.0, 1.5),
    (0.0, 0, 1.0, 1.0),
    (0.01, 0, 1.0, 1.0),
]


def run_pair(ctx, logits, counts, cfg, seed, step, dl=None, dc=None):
    t, k, p, pen = cfg
    own_l = dl is None
    dl = dl or lq8.DeviceBuffer.from_array(ctx, logits)
    own_c = dc is None and counts is not None
    if own_c:
        dc = lq8.DeviceBuffer.from_array(ctx, counts)
    try:
        g = lq8.sample_device(ctx, dl, logits.size, lq8.GenerationConfig(1, t, k, p, pen), seed, step, dc)
    finally:
        if own_l:
            dl.free()
        if own_c:
            dc.free()
    return g, oracle.sample(logits, counts, t, k, p, pen, seed, step)


@pytest.mark.parametrize("cfg", CONFIGS, ids=[str(c) for c in CONFIGS])
def test_sample_qwen3_vocab_matches_oracle(ctx, cfg):
    V = 151936
    rng = np.random.default_rng(hash(cfg) & 0xFFFF)
    logits = (rng.standard_normal(V) * 3.0).astype(np.float32)
    counts = np.zeros(V, np.uint32)
    counts[rng.integers(0, V, 300)] = rng.integers(1, 4, 300)
    # make some penalized tokens the strongest candidates
    top = np.argsort(logits)[-20:]
    counts[top[::2]] = 2
    dl, dc = lq8.DeviceBuffer.from_array(ctx, logits), lq8.DeviceBuffer.from_array(ctx, counts)
    try:
        for seed in (0, 12345, 2**63 + 7):
            for step in (0, 1, 17, 4096):
                g, o = run_pair(ctx, logits, counts, cfg, seed, step, dl, dc)
                assert g == o, (cfg, seed, step, g, o)
    finally:
        dl.free()
        dc.free()


@pytest.mark.parametrize("V", [1, 2, 5, 63, 64, 65, 130, 1023, 1024, 1025, 2047, 2048, 2049, 4097])
def test_sample_small_vocab_ties(ctx, V):
    """Integer logits (many ties), sizes around a wave, the 1024-entry sort
    tile (also the pick's per-thread span) and several tiles."""
    rng = np.random.default_rng(V)
    logits = rng.integers(-3, 4, V).astype(np.float32)
    counts = rng.integers(0, 2, V).astype(np.uint32)
    for cfg in [(1.0, 0, 1.0, 1.0), (1.0, 3, 1.0, 1.0), (0.5, 0, 0.6, 1.0), (0.0, 0, 1.0, 1.0),
                (0.0, 0, 1.0, 2.0), (1.0, 0, 0.3, 2.0)]:
        for step in range(6):
            g, o = run_pair(ctx, logits, counts if cfg[3] != 1.0 else None, cfg, 99, step)
            assert g == o, (V, cfg, step, g, o)


@pytest.mark.parametrize("case", ["flat", "integer", "dense"])
def test_sample_topk_exact_selection(ctx, case):
    """top_k up to 1024 selects candidates by the top 12 bits of the key; when
    the boundary bucket holds more than 4096 keys the pick selects the K keys
    exactly (two more histogram levels, ties by index).  Flat logits (every key
    tied), integer logits (few values) and 151936 distinct values packed into
    one bucket all take that route; top_k 1024 / 1025 sit on either side of
    the path boundary."""
    V = 151936
    rng = np.random.default_rng(17)
    if case == "flat":
        logits = np.zeros(V, np.float32)
    elif case == "integer":
        logits = rng.integers(-3, 4, V).astype(np.float32)
    else:
        logits = (np.float32(1.0) + rng.permutation(V).astype(np.float32) * np.float32(2.0**-23)).astype(np.float32)
    counts = np.zeros(V, np.uint32)
    counts[rng.integers(0, V, 200)] = 1
    dl, dc = lq8.DeviceBuffer.from_array(ctx, logits), lq8.DeviceBuffer.from_array(ctx, counts)
    try:
        for cfg in [(1.0, 50, 1.0, 1.0), (0.7, 1024, 0.9, 1.0), (1.3, 1, 1.0, 1.0), (1.0, 700, 0.5, 1.2),
                    (1.0, 1025, 1.0, 1.0)]:
            for step in range(3):
                g, o = run_pair(ctx, logits, counts, cfg, 3, step, dl, dc)
                assert g == o, (case, cfg, step, g, o)
    finally:
        dl.free()
        dc.free()


def test_sample_extreme_values(ctx):
    """Signed zeros, huge magnitudes and a single finite winner."""
    x = np.array([-0.0, 0.0, 3e38, -3e38, 1e-45, -1e-45, 5.0, 5.0], np.float32)
    for cfg in [(1.0, 0, 1.0, 1.0), (0.0, 0, 1.0, 1.0), (1e-3, 0, 0.9, 1.0), (3.0, 4, 1.0, 1.0)]:
        for step in range(4):
            g, o = run_pair(ctx, x, None, cfg, 5, step)
            assert g == o, (cfg, step, g, o)


def test_sample_device_rejects_bad_config(ctx):
    dl = lq8.DeviceBuffer.from_array(ctx, np.zeros(16, np.float32))
    try:
        for bad in [lq8.GenerationConfig(1, -1.0, 0, 1.0, 1.0), lq8.GenerationConfig(1, 1.0, 0, 1.5, 1.0),
                    lq8.GenerationConfig(1, 1.0, 0, 1.0, 0.5)]:
            with pytest.raises(lq8.InvalidArgument):
                lq8.sample_device(ctx, dl, 16, bad)
        # vocabulary bounds are checked before any device work
        for vocab in (0, 2**20 + 1):
            with pytest.raises(lq8.InvalidArgument):
                lq8.sample_device(ctx, dl, vocab, lq8.GenerationConfig(1, 1.0, 0, 1.0, 1.0))
    finally:
        dl.free()


SMALL = lq8.Qwen3Config(vocab_size=2048, hidden_size=256, intermediate_size=768, num_hidden_layers=3,
                        num_attention_heads=4, num_key_value_heads=2, head_dim=128, max_position_embeddings=128)


@pytest.fixture(scope="module")
def small_pair(ctx):
    model = lq8.Qwen3ForCausalLM.random(ctx, SMALL, seed=3)
    ref = oracle.Model(SMALL, model.export_all())
    yield model, ref
    model.free()
    ref.close()


def generate(model, prompt, cfg, seed, graph, eos=()):
    old = os.environ.pop("LQ8_NO_GRAPH", None)
    if not graph:
        os.environ["LQ8_NO_GRAPH"] = "1"
    try:
        return model.generate(prompt, cfg, seed, eos)
    finally:
        os.environ.pop("LQ8_NO_GRAPH", None)
        if old is not None:
            os.environ["LQ8_NO_GRAPH"] = old


@pytest.mark.parametrize("graph", [True, False])
@pytest.mark.parametrize("cfg", [(1.0, 0, 1.0, 1.0), (0.8, 40, 0.9, 1.3), (0.0, 0, 1.0, 1.6)])
def test_generate_sampled_matches_oracle(small_pair, graph, cfg):
    model, ref = small_pair
    prompt = np.random.default_rng(12).integers(0, SMALL.vocab_size, 20).astype(np.uint32)
    gc = lq8.GenerationConfig(30, *cfg)
    toks, stats = generate(model, prompt, gc, 77, graph)
    assert stats["used_graph"] == graph
    ref_toks = ref.generate_sampled(prompt, 30, *cfg, 77)
    assert toks.tolist() == ref_toks.tolist()


def test_generate_temperature_zero_is_greedy(small_pair):
    model, _ = small_pair
    prompt = np.arange(11, dtype=np.uint32)
    a, _ = model.generate(prompt, lq8.GenerationConfig(20), seed=4)
    b, _ = model.generate_greedy(prompt, 20)
    assert a.tolist() == b.tolist()


def test_generate_sampled_replays_repeatable(small_pair):
    """The same seed replays the same tokens across calls (graph replays of
    the decode step and the sampler); another seed differs."""
    model, _ = small_pair
    prompt = np.arange(9, dtype=np.uint32)
    cfg = lq8.GenerationConfig(24, 1.0, 0, 1.0, 1.2)
    a, _ = model.generate(prompt, cfg, seed=1)
    b, _ = model.generate(prompt, cfg, seed=1)
    c, _ = model.generate(prompt, cfg, seed=2)
    g, _ = model.generate_greedy(prompt, 5)
    d, _ = model.generate(prompt, cfg, seed=1)
    assert a.tolist() == b.tolist() == d.tolist()
    assert a.tolist() != c.tolist()
    assert g.size == 5


@pytest.mark.parametrize("graph", [True, False])
def test_generate_stops_at_eos(small_pair, graph):
    """generate() ends at the first EOS token (kept), as the reference's loop
    does; the cache is left at the early stop's length, so a forward at the
    next offset continues bit for bit like the oracle's."""
    model, ref = small_pair
    prompt = np.random.default_rng(31).integers(0, SMALL.vocab_size, 15).astype(np.uint32)
    cfg = (0.9, 0, 1.0, 1.2)
    full = ref.generate_sampled(prompt, 30, *cfg, 5)
    eos = [int(full[11]), 2047]  # a token first drawn at step 11, and one never drawn
    first = next(t for t in range(30) if int(full[t]) in eos)
    toks, _ = generate(model, prompt, lq8.GenerationConfig(30, *cfg), 5, graph, eos)
    ref_toks = ref.generate_sampled(prompt, 30, *cfg, 5, eos_token_ids=eos)
    assert toks.tolist() == ref_toks.tolist() == full[:first + 1].tolist()
    nxt = [int(toks[-1])]
    pos = prompt.size + toks.size - 1
    assert same_bits(model.forward(nxt, pos), ref.forward(nxt, pos))
    # no EOS among the tokens: all of them
    toks, _ = generate(model, prompt, lq8.GenerationConfig(30, *cfg), 5, graph, [2047] if 2047 not in full else [])
    assert toks.size == 30


def same_bits(a, b):
    return np.array_equal(np.asarray(a, np.float32).view(np.uint32), np.asarray(b, np.float32).view(np.uint32))


def test_generate_vocabulary_bound(ctx):
    """Sampling is bounded to vocabularies of 2^20 (checked before any device
    work); temperature 0 without a penalty is the greedy path, which is not."""
    cfg = lq8.Qwen3Config(vocab_size=2**20 + 1, hidden_size=64, intermediate_size=64, num_hidden_layers=1,
                          num_attention_heads=1, num_key_value_heads=1, head_dim=128, max_position_embeddings=16)
    model = lq8.Qwen3ForCausalLM.random(ctx, cfg, seed=1)
    try:
        with pytest.raises(lq8.InvalidArgument):
            model.generate([1, 2, 3], lq8.GenerationConfig(4, 1.0, 0, 1.0, 1.0))
        toks, _ = model.generate([1, 2, 3], lq8.GenerationConfig(4))
        greedy, _ = model.generate_greedy([1, 2, 3], 4)
        assert toks.tolist() == greedy.tolist()
    finally:
        model.free()


def test_generate_rejects_bad_config(small_pair):
    model, _ = small_pair
    with pytest.raises(lq8.InvalidArgument):
        model.generate([1, 2], lq8.GenerationConfig(4, 1.0, 0, 2.0, 1.0))
