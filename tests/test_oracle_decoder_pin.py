"""CPU: the oracle's decoder forward (orc_model_forward) and MoE layer
(orc_moe_forward) pinned against an independent float64 numpy restatement
of the reference's numerics (tests/golden/numpy_decoder.py, written from
src/attention.rs:318-456, src/rms_norm.rs:143-176, src/rope.rs:77-128,245-303,
src/mlp.rs:151-164, src/transformer.rs:180-204, src/model.rs:345-372), and
against closed forms a plausible mistake fails.

Two kinds of comparison:
- Structure (tight, 1e-5 relative on the logits): RmsNorm's bf16 roundings
  and the W8A8 activation quantization are switched off in both, because
  both are discontinuous -- a one-ulp float32-vs-float64 difference can put a
  value on the other side of a rounding midpoint, and the ~1e-3 jump that
  follows would hide everything else.  What remains is the decoder's wiring:
  GQA head mapping, q/k-norm placement, RoPE tables and pairing, causal mask
  with offset, segment-order softmax, SwiGLU, residuals, final norm, KV cache.
  Planted mistakes in the restatement (the `mutation` modes) move the logits
  by 1e-2 or far more, so this bar tells them apart.
- Reference numerics (bf16 sites and W8A8 on, the contract the GPU
  implements): 1e-5 on a prefill + decode run whose roundings do not straddle
  a midpoint, and a looser bound plus the argmax on longer runs.
"""
from dataclasses import dataclass

import numpy as np
import pytest

import lq8
import oracle
from golden import numpy_decoder as ndm

TIGHT = 1e-5


@pytest.fixture
def structure_mode():
    oracle.set_bf16_rounding(False)
    oracle.set_activation_quantization(False)
    ndm.BF16_SITES[0] = False
    ndm.Q8_ACTIVATIONS[0] = False
    yield
    oracle.set_bf16_rounding(True)
    oracle.set_activation_quantization(True)
    ndm.BF16_SITES[0] = True
    ndm.Q8_ACTIVATIONS[0] = True


def rel(a, b):
    return float(np.max(np.abs(np.asarray(a, np.float64) - b)) / np.max(np.abs(b)))


def tensors(cfg, seed, norm_jitter=0.1):
    """Table-order tensors: N(0, 0.02) Q8_0 matrices, norm weights 1 + jitter
    N(0, 1) (so a norm weight applied in the wrong place shows)."""
    rng = np.random.default_rng(seed)
    out = []
    for i in range(cfg.tensor_count()):
        kind, shape = cfg.tensor_shape(i)
        if kind == "f32":
            out.append((1 + norm_jitter * rng.standard_normal(shape)).astype(np.float32))
        else:
            out.append(oracle.quantize_q8_0((rng.standard_normal(shape) * 0.02).astype(np.float32)))
    return out


def config(nh, nkv, layers=2, hidden=256, max_pos=160):
    return lq8.Qwen3Config(vocab_size=1024, hidden_size=hidden, intermediate_size=512, num_hidden_layers=layers,
                           num_attention_heads=nh, num_key_value_heads=nkv, head_dim=128,
                           max_position_embeddings=max_pos)


def run_pair(cfg, T, prompt, steps, chunks=1, mutation=None):
    """Prefill (in `chunks` pieces, each at its offset) then `steps` one-token
    decode forwards; returns the per-forward relative logit errors and
    whether every argmax agreed."""
    o = oracle.Model(cfg, T)
    nd = ndm.NumpyQwen3(cfg, T, mutation=mutation)
    try:
        errs, same = [], True
        parts = np.array_split(np.asarray(prompt, np.uint32), chunks)
        off = 0
        for p in parts:
            lo, ln = o.forward(p, off), nd.forward(p, off)
            errs.append(rel(lo, ln))
            same &= int(np.argmax(lo)) == int(np.argmax(ln))
            off += p.size
        tok = int(np.argmax(lo))
        for s in range(steps):
            lo, ln = o.forward([tok], off + s), nd.forward([tok], off + s)
            errs.append(rel(lo, ln))
            same &= int(np.argmax(lo)) == int(np.argmax(ln))
            tok = (tok * 7 + 3) % cfg.vocab_size
        return errs, same
    finally:
        o.close()


GQA = [(4, 2), (16, 2)]  # groups 2 and 8, each with kv heads that differ


@pytest.mark.parametrize("nh,nkv", GQA)
def test_structure_prefill_across_segment_edge(structure_mode, nh, nkv):
    """62-position prefill, then 6 decode steps through positions 62..67 (the
    64-position segment edge of the attention order)."""
    cfg = config(nh, nkv)
    T = tensors(cfg, 5)
    prompt = np.random.default_rng(1).integers(0, cfg.vocab_size, 62)
    errs, same = run_pair(cfg, T, prompt, 6)
    assert max(errs) <= TIGHT, errs
    assert same


@pytest.mark.parametrize("nh,nkv", GQA)
def test_structure_decode_only(structure_mode, nh, nkv):
    """One-token prompt then 70 KV-cached decode steps (every forward is a
    single position: no mask, the cache grows across the segment edge)."""
    cfg = config(nh, nkv)
    T = tensors(cfg, 6)
    errs, same = run_pair(cfg, T, [17], 70)
    assert max(errs) <= TIGHT, max(errs)
    assert same


def test_structure_chunked_prefill_uses_offset_mask(structure_mode):
    """A prompt forwarded in three chunks at offsets 0, 20, 40: the causal
    mask of a chunk is j > i + offset (src/causal_mask.rs:139-150)."""
    cfg = config(4, 2)
    T = tensors(cfg, 7)
    prompt = np.random.default_rng(2).integers(0, cfg.vocab_size, 60)
    errs, same = run_pair(cfg, T, prompt, 3, chunks=3)
    assert max(errs) <= TIGHT, errs
    assert same


MUTATIONS = ["gqa_mod", "rope_pairing", "rope_sign", "qnorm_after_rope", "no_final_norm", "mask_offset",
             "swiglu_swap", "residual_normed"]


@pytest.mark.parametrize("mutation", MUTATIONS)
def test_planted_mistakes_fail_the_pin(structure_mode, mutation):
    """Each planted mistake moves the logits far past the tight bar, so the
    comparisons above would catch it in the oracle."""
    cfg = config(16, 2)
    T = tensors(cfg, 5)
    prompt = np.random.default_rng(3).integers(0, cfg.vocab_size, 40)
    errs, _ = run_pair(cfg, T, prompt, 3, chunks=2, mutation=mutation)
    assert max(errs) > 100 * TIGHT, (mutation, errs)


def test_reference_numerics_prefill_and_decode():
    """bf16 roundings and W8A8 activations on (the contract itself): a 20-token
    prefill and 3 decode steps whose roundings land clear of midpoints agree
    to 1e-5."""
    cfg = config(4, 2)
    T = tensors(cfg, 5)
    prompt = np.random.default_rng(1).integers(0, cfg.vocab_size, 20)
    errs, same = run_pair(cfg, T, prompt, 3)
    assert max(errs) <= TIGHT, errs
    assert same


@pytest.mark.parametrize("nh,nkv", GQA)
def test_reference_numerics_long_run(nh, nkv):
    """bf16 roundings and W8A8 activations on over 62 + 8 positions: single
    roundings may land across a midpoint (each moves the logits by ~1e-3), so
    the bound here is 1e-2 and the argmax."""
    cfg = config(nh, nkv)
    T = tensors(cfg, 8)
    prompt = np.random.default_rng(4).integers(0, cfg.vocab_size, 62)
    errs, same = run_pair(cfg, T, prompt, 8)
    assert max(errs) <= 1e-2, errs
    assert same


# ---- closed forms --------------------------------------------------------------

def identity_q8(n):
    """Q8_0 blocks of the n x n identity: scale 1.0 (f16 0x3C00), code 1 on
    the diagonal."""
    b = np.zeros((n, n // 32, 34), np.uint8)
    b[:, :, 0:2] = np.frombuffer(np.float16(1.0).tobytes(), np.uint8)
    for r in range(n):
        b[r, r // 32, 2 + r % 32] = 1
    return b.reshape(-1)


def closed_form_model(zero_k):
    """One layer, hidden = num_heads * head_dim = 512 (4 query heads, 2 kv
    heads), o_proj the identity, gate/up/down zero (the MLP adds exactly 0):
    the layer output is h + attention output, concatenated over heads."""
    cfg = lq8.Qwen3Config(vocab_size=256, hidden_size=512, intermediate_size=64, num_hidden_layers=1,
                          num_attention_heads=4, num_key_value_heads=2, head_dim=128, max_position_embeddings=80)
    T = tensors(cfg, 11)
    H, I = 512, 64
    z = lambda r, c: np.zeros(r * c // 32 * 34, np.uint8)  # noqa: E731 (all-zero blocks: scale 0, codes 0)
    T[2 + 7] = identity_q8(H)
    T[2 + 8], T[2 + 9], T[2 + 10] = z(I, H), z(I, H), z(H, I)
    if zero_k:
        T[2 + 5] = z(256, H)
    return cfg, T


def v_rows(cfg, T, h0):
    """v = v_proj(input_layernorm(h)) from the oracle's pinned pieces
    (RmsNorm, GEMV), one row per position."""
    x = oracle.rms_norm(h0, T[2], cfg.rms_norm_eps)
    return np.stack([oracle.gemv_q8_0(T[2 + 6], 256, 512, r) for r in x])


def test_single_position_attention_is_v_exactly():
    """With one visible position the softmax weight is exactly 1, so each
    query head's output is the v of its kv head h // 2 (repeat_kv,
    src/attention.rs:442-452), bit for bit: layer output = h + [v0 v0 v1 v1]."""
    cfg, T = closed_form_model(zero_k=False)
    o = oracle.Model(cfg, T)
    try:
        hid, _, _ = o.forward_with_intermediates([9], 0)
    finally:
        o.close()
    h0 = hid[0]
    v = v_rows(cfg, T, h0)[0]
    tiled = np.concatenate([v[:128], v[:128], v[128:], v[128:]]).astype(np.float32)
    assert np.array_equal(hid[1][0].view(np.uint32), (h0[0] + tiled).view(np.uint32))
    # the h % n_kv mapping would give [v0 v1 v0 v1]: the kv heads really differ here
    assert not np.allclose(v[:128], v[128:], rtol=1e-2)


def test_equal_keys_average_the_values():
    """k_proj = 0 makes every key 0, so the scores are all equal and each
    head's output is the mean of V over the visible positions: checked at
    every step of 70 decode positions (across the segment edge)."""
    cfg, T = closed_form_model(zero_k=True)
    o = oracle.Model(cfg, T)
    try:
        rng = np.random.default_rng(12)
        ids = rng.integers(0, cfg.vocab_size, 70)
        h0s, outs = [], []
        for p, t in enumerate(ids):
            hid, _, _ = o.forward_with_intermediates([t], p)
            h0s.append(hid[0][0])
            outs.append(hid[1][0])
    finally:
        o.close()
    h0s = np.array(h0s)
    v = v_rows(cfg, T, h0s).astype(np.float64)
    for p in range(len(ids)):
        m = v[:p + 1].mean(axis=0)
        ref = h0s[p] + np.concatenate([m[:128], m[:128], m[128:], m[128:]])
        assert np.max(np.abs(outs[p] - ref)) <= 1e-6 * np.max(np.abs(ref)) + 1e-9, p


# ---- MoE layer ------------------------------------------------------------------

@dataclass
class MoeCfg:
    hidden_size: int = 256
    num_heads: int = 4
    num_kv_heads: int = 2
    head_dim: int = 128
    num_experts: int = 8
    top_k: int = 3
    expert_intermediate_size: int = 96
    max_positions: int = 80
    max_batch: int = 3
    num_layers: int = 2
    rms_norm_eps: float = 1e-6
    rope_theta: float = 1e6


def moe_tensors(cfg, seed):
    rng = np.random.default_rng(seed)
    H, I, hd, E = cfg.hidden_size, cfg.expert_intermediate_size, cfg.head_dim, cfg.num_experts
    QD, KD = cfg.num_heads * hd, cfg.num_kv_heads * hd
    q8 = lambda shape: oracle.quantize_q8_0((rng.standard_normal(shape) * 0.02).astype(np.float32))  # noqa: E731
    nw = lambda n: (1.0 + 0.1 * rng.standard_normal(n)).astype(np.float32)  # noqa: E731
    out = []
    for _ in range(cfg.num_layers):
        out += [nw(H), nw(H), nw(hd), nw(hd), q8((QD, H)), q8((KD, H)), q8((KD, H)), q8((H, QD))]
        out += [q8((I, H)) for _ in range(E)] + [q8((I, H)) for _ in range(E)] + [q8((H, I)) for _ in range(E)]
    return out


def test_moe_layers_pinned(structure_mode):
    """Two MoE layers, three sequences at different positions, 70 decode
    steps (every sequence crosses the segment edge): the oracle's hidden
    states equal the float64 restatement's to 1e-5, with the router scores
    spread so that no two experts tie."""
    cfg = MoeCfg()
    T = moe_tensors(cfg, 21)
    om = oracle.MoeStack(cfg, T)
    nm = ndm.NumpyMoeStack(cfg, T)
    rng = np.random.default_rng(22)
    try:
        start = np.array([0, 3, 9])
        for s in range(70):
            pos = start + s
            pos = pos[pos < cfg.max_positions]
            Tn = pos.size
            h = (rng.standard_normal((Tn, cfg.hidden_size)) * 0.5).astype(np.float32)
            sc = rng.standard_normal((cfg.num_layers, Tn, cfg.num_experts)).astype(np.float32)
            ho = om.forward(h, sc, pos)
            hn = nm.forward(h, sc, pos)
            assert rel(ho, hn) <= TIGHT, (s, rel(ho, hn))
    finally:
        om.close()
