"""GPU Qwen3 decoder vs the CPU oracle: prefill/decode logits bit for bit and
greedy tokens identical (the end-to-end bar), including the Qwen3-0.6B
random-init config with a 128-token prompt and 128 generated tokens."""
import os
import time

import numpy as np
import pytest

import lq8
import oracle

pytestmark = pytest.mark.gpu

SMALL = lq8.Qwen3Config(vocab_size=2048, hidden_size=256, intermediate_size=768, num_hidden_layers=3,
                        num_attention_heads=4, num_key_value_heads=2, head_dim=128, max_position_embeddings=128)


def same_bits(a, b):
    return np.array_equal(np.asarray(a, np.float32).view(np.uint32), np.asarray(b, np.float32).view(np.uint32))


@pytest.fixture(scope="module")
def small_pair(ctx):
    model = lq8.Qwen3ForCausalLM.random(ctx, SMALL, seed=3)
    ref = oracle.Model(SMALL, model.export_all())
    yield model, ref
    model.free()
    ref.close()


def test_load_from_host_tensors_matches_export(ctx):
    tensors = oracle.random_q8_tensors(SMALL, seed=5)
    m = lq8.Qwen3ForCausalLM.load(ctx, SMALL, tensors)
    for i, t in enumerate(tensors):
        assert np.array_equal(m.export_tensor(i).view(np.uint8), t.view(np.uint8)), f"tensor {i}"
    m.free()


def test_prefill_then_decode_logits_bit_exact(small_pair):
    model, ref = small_pair
    rng = np.random.default_rng(11)
    prompt = rng.integers(0, SMALL.vocab_size, 37).astype(np.uint32)
    model.clear_kv_cache()
    ref.clear_kv_cache()
    lg, lr = model.forward(prompt, 0), ref.forward(prompt, 0)
    assert same_bits(lg, lr), f"prefill max|d| {np.max(np.abs(lg - lr))}"
    pos = prompt.size
    for step in range(6):
        tok = [int(rng.integers(0, SMALL.vocab_size))]
        lg, lr = model.forward(tok, pos), ref.forward(tok, pos)
        assert same_bits(lg, lr), f"decode step {step}: max|d| {np.max(np.abs(lg - lr))}"
        pos += 1


def test_single_token_prompt(small_pair):
    model, ref = small_pair
    model.clear_kv_cache()
    ref.clear_kv_cache()
    assert same_bits(model.forward([5], 0), ref.forward([5], 0))


def test_offset_must_match_cache(small_pair):
    model, _ = small_pair
    model.clear_kv_cache()
    model.forward([1, 2, 3], 0)
    with pytest.raises(lq8.InvalidArgument):
        model.forward([4], 7)
    with pytest.raises(lq8.InvalidArgument):
        model.forward([SMALL.vocab_size], 3)


@pytest.mark.parametrize("graph", [True, False])
def test_generate_greedy_matches_oracle(small_pair, graph):
    model, ref = small_pair
    prompt = np.random.default_rng(12).integers(0, SMALL.vocab_size, 20).astype(np.uint32)
    old = os.environ.pop("LQ8_NO_GRAPH", None)
    if not graph:
        os.environ["LQ8_NO_GRAPH"] = "1"
    try:
        toks, stats = model.generate_greedy(prompt, 24)
    finally:
        os.environ.pop("LQ8_NO_GRAPH", None)
        if old is not None:
            os.environ["LQ8_NO_GRAPH"] = old
    ref_toks, _ = ref.generate_greedy(prompt, 24)
    assert stats["used_graph"] == graph
    assert toks.tolist() == ref_toks.tolist()


def test_graph_replays_repeatable(small_pair):
    """The captured decode step is replayed many times across calls."""
    model, _ = small_pair
    prompt = np.arange(9, dtype=np.uint32)
    a, _ = model.generate_greedy(prompt, 16)
    b, _ = model.generate_greedy(prompt, 16)
    assert a.tolist() == b.tolist()


def test_long_context_many_segments(ctx):
    """max_positions 8192 (128 attention segments launched, most idle) and a
    200-token prompt: decode attention combines 4-5 segments; tokens match."""
    cfg = lq8.Qwen3Config(vocab_size=1024, hidden_size=256, intermediate_size=512, num_hidden_layers=2,
                          num_attention_heads=4, num_key_value_heads=2, head_dim=128, max_position_embeddings=8192)
    model = lq8.Qwen3ForCausalLM.random(ctx, cfg, seed=9)
    ref = oracle.Model(cfg, model.export_all())
    prompt = np.random.default_rng(9).integers(0, cfg.vocab_size, 200).astype(np.uint32)
    toks, _ = model.generate_greedy(prompt, 70)
    ref_toks, _ = ref.generate_greedy(prompt, 70)
    assert toks.tolist() == ref_toks.tolist()
    model.clear_kv_cache()
    ref.clear_kv_cache()
    assert same_bits(model.forward(prompt[:129], 0), ref.forward(prompt[:129], 0))
    for t in range(3):
        assert same_bits(model.forward([int(prompt[129 + t])], 129 + t), ref.forward([int(prompt[129 + t])], 129 + t))
    model.free()
    ref.close()


def test_wide_gqa_and_odd_block_counts(ctx):
    """8 query heads per kv head (the MoE layer's grouping) and hidden /
    intermediate sizes with an odd number of Q8_0 blocks (224 = 7 blocks,
    352 = 11 blocks): logits bit-exact, tokens identical."""
    cfg = lq8.Qwen3Config(vocab_size=1000, hidden_size=224, intermediate_size=352, num_hidden_layers=2,
                          num_attention_heads=8, num_key_value_heads=1, head_dim=128, max_position_embeddings=160)
    model = lq8.Qwen3ForCausalLM.random(ctx, cfg, seed=21)
    ref = oracle.Model(cfg, model.export_all())
    prompt = np.random.default_rng(21).integers(0, cfg.vocab_size, 66).astype(np.uint32)
    assert same_bits(model.forward(prompt, 0), ref.forward(prompt, 0))
    assert same_bits(model.forward([7], 66), ref.forward([7], 66))
    toks, _ = model.generate_greedy(prompt, 20)
    ref_toks, _ = ref.generate_greedy(prompt, 20)
    assert toks.tolist() == ref_toks.tolist()
    model.free()
    ref.close()


@pytest.mark.parametrize("heads,kv", [(4, 2), (8, 1)])
def test_chunked_prefill_across_segments(ctx, heads, kv):
    """Prefill in chunks at offsets 0, 30 and 61: the later chunks' rows
    straddle 64-position segment boundaries, so rows of one attention
    workgroup end in different segments.  Logits bit-exact after every chunk
    and for a decode step."""
    cfg = lq8.Qwen3Config(vocab_size=700, hidden_size=256, intermediate_size=352, num_hidden_layers=2,
                          num_attention_heads=heads, num_key_value_heads=kv, head_dim=128,
                          max_position_embeddings=192)
    model = lq8.Qwen3ForCausalLM.random(ctx, cfg, seed=40 + heads)
    ref = oracle.Model(cfg, model.export_all())
    ids = np.random.default_rng(heads).integers(0, cfg.vocab_size, 140).astype(np.uint32)
    for a, b in [(0, 30), (30, 61), (61, 139)]:
        assert same_bits(model.forward(ids[a:b], a), ref.forward(ids[a:b], a)), (a, b)
    assert same_bits(model.forward([int(ids[139])], 139), ref.forward([int(ids[139])], 139))
    model.free()
    ref.close()


@pytest.mark.parametrize("hidden", [1568, 2112])
def test_wide_hidden_prefill_paths(ctx, hidden):
    """Prefill normalizes and quantizes GEMM inputs in one kernel for hidden
    sizes up to 2048 (1568: 49 blocks, odd, the widest register variant) and
    falls back to RmsNorm rows + quantize above it (2112); intermediate 800
    (25 blocks) takes silu(gate) * up straight into the quantizer.  Prefill
    and decode logits bit-exact either way."""
    cfg = lq8.Qwen3Config(vocab_size=640, hidden_size=hidden, intermediate_size=800, num_hidden_layers=2,
                          num_attention_heads=4, num_key_value_heads=2, head_dim=128, max_position_embeddings=96)
    model = lq8.Qwen3ForCausalLM.random(ctx, cfg, seed=hidden)
    ref = oracle.Model(cfg, model.export_all())
    prompt = np.random.default_rng(hidden).integers(0, cfg.vocab_size, 37).astype(np.uint32)
    assert same_bits(model.forward(prompt, 0), ref.forward(prompt, 0))
    assert same_bits(model.forward([5], 37), ref.forward([5], 37))
    model.free()
    ref.close()


def test_qwen3_0_6b_greedy_128_plus_128(ctx):
    """Qwen3-0.6B random-init Q8_0, 128 uniform-random prompt ids, 128 greedy
    tokens: identical to the oracle; the prefill logits are bit-identical."""
    cfg = lq8.qwen3_0_6b(max_positions=512)
    model = lq8.Qwen3ForCausalLM.random(ctx, cfg, seed=2026)
    t0 = time.time()
    ref = oracle.Model(cfg, model.export_all())
    prompt = np.random.default_rng(2026).integers(0, cfg.vocab_size, 128).astype(np.uint32)
    toks, stats = model.generate_greedy(prompt, 128)
    ref_toks, margins = ref.generate_greedy(prompt, 128)
    print(f"\noracle+export {time.time() - t0:.1f}s; gpu {stats}; min top-2 margin {float(margins.min()):.3g}")
    assert toks.tolist() == ref_toks.tolist()
    model.clear_kv_cache()
    ref.clear_kv_cache()
    assert same_bits(model.forward(prompt, 0), ref.forward(prompt, 0))
    model.free()
    ref.close()
