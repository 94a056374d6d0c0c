"""Independent float64 numpy restatement of the Qwen3 decoder numerics of the
reference crate (lluda-inference), used to pin the C oracle's model forward.

Written from the reference's source, not from the oracle:
  - Embedding::forward (src/embedding.rs:105-153): a row gather; rows are the
    dequantized Q8_0 table (exact in float32, src of the tied lm_head).
  - RmsNorm::forward (src/rms_norm.rs:143-176): input and weight rounded to
    bf16 (src/bf16.rs:112-131), sum of squares, mean, 1/sqrt(mean + eps as f32),
    x * inv * w, output rounded to bf16.
  - RotaryEmbedding::new / apply_rope_to_tensor (src/rope.rs:77-128, 245-303):
    rope_dim = head_dim / 2, inv_freq[i] = 1 / theta^(2i / rope_dim) for
    i < rope_dim / 2, tables [pos][rope_dim] holding each frequency twice
    (cast to f32); out[d] = x[d] c - x[d + rope_dim] s and
    out[d + rope_dim] = x[d + rope_dim] c + x[d] s with c = cos[pos][d & ~1].
  - Attention::forward (src/attention.rs:318-403): q/k/v projections, per-head
    q/k RmsNorm before RoPE, KV cache append, repeat_kv (src/attention.rs:426-456:
    kv head k is repeated for query heads k*groups .. k*groups + groups - 1),
    scores q k^T times 1/sqrt(head_dim) (f32 scale), causal mask of -inf for
    j > i + offset (src/causal_mask.rs:104-164, none for one position),
    softmax over positions, P V, heads concatenated, o projection.
  - MLP::forward (src/mlp.rs:151-164): down(silu(gate x) * up x), silu(x) =
    x / (1 + exp(-x)) (src/tensor.rs:1955-1990).
  - DecoderLayer::forward (src/transformer.rs:180-204): pre-norm residual
    blocks; Qwen3ForCausalLM::forward (src/model.rs:345-372): final norm, the
    last position's logits through the tied embedding.
  - Linear::forward on a Q8_0 weight (the library's contract for the W8A8
    path): with more than one row the activation rows are quantized to Q8_0
    per 32-element block first (quantize_q8_0 of numpy_q8.py); one row uses
    the activations as they are.

Everything else is float64: the differences from the oracle are the oracle's
float32 rounding, so agreement to ~1e-6 relative pins what the oracle
computes, while a wrong head mapping, rotation pairing, norm placement or
residual wiring moves the logits by far more.

`mutation` plants one mistake (for the tests that show the pin notices it):
  "gqa_mod"      query head h reads kv head h % n_kv instead of h // groups
  "rope_pairing" rotate-half frequency index d instead of d // 2
  "qnorm_after_rope"  q/k RmsNorm applied after RoPE instead of before
  "no_final_norm"     lm_head on the un-normed hidden state
  "rope_sign"    out[d] = x[d] c + x[d + rope_dim] s (rotation the other way)
  "mask_offset"  causal mask j > i instead of j > i + offset
  "swiglu_swap"  silu(up x) * gate x instead of silu(gate x) * up x
  "residual_normed"   attention residual added to the normed input
"""
import numpy as np

from .numpy_q8 import bf16_round, dequantize_q8_0, quantize_q8_0


# RmsNorm's bf16 roundings and the W8A8 activation quantization; switched
# off together with the oracle's (oracle.set_bf16_rounding,
# oracle.set_activation_quantization) to compare the rest of the decoder
# tightly: both are discontinuous, so a float32-vs-float64 difference of one
# ulp can move a value across a rounding midpoint and hide everything else.
BF16_SITES = [True]
Q8_ACTIVATIONS = [True]


def bf16(x):
    """Value of the reference's BF16::from(f32) on the f32 cast of x, as f64."""
    x = np.asarray(x, np.float64)
    if not BF16_SITES[0]:
        return x
    return bf16_round(x.astype(np.float32)).reshape(x.shape).astype(np.float64)


def rms_norm(x, w, eps):
    """src/rms_norm.rs:143-176 over the last axis."""
    xb = bf16(x)
    wb = bf16(w)
    ms = np.sum(xb * xb, axis=-1, keepdims=True) / xb.shape[-1]
    inv = 1.0 / np.sqrt(ms + float(np.float32(eps)))
    return bf16(xb * inv * wb)


def rope_tables(head_dim, max_pos, theta):
    """src/rope.rs:89-118: [max_pos][head_dim / 2], each frequency twice, f32."""
    rope_dim = head_dim // 2
    half = rope_dim // 2
    inv = np.array([1.0 / theta ** ((2 * i) / rope_dim) for i in range(half)])
    freqs = np.arange(max_pos, dtype=np.float64)[:, None] * inv[None, :]
    c = np.repeat(np.cos(freqs).astype(np.float32), 2, axis=1).astype(np.float64)
    s = np.repeat(np.sin(freqs).astype(np.float32), 2, axis=1).astype(np.float64)
    return c, s


def rope(x, c, s, offset, mutation=None):
    """src/rope.rs:270-297 on x [heads, seq, head_dim] at positions offset + l."""
    heads, seq, hd = x.shape
    R = hd // 2
    cs = c[offset:offset + seq]
    sn = s[offset:offset + seq]
    if mutation == "rope_pairing":
        # frequency index d instead of d // 2 (a table without the repeat)
        cs = np.concatenate([cs[:, 0::2], cs[:, 0::2]], axis=1)[:, :R]
        sn = np.concatenate([sn[:, 0::2], sn[:, 0::2]], axis=1)[:, :R]
    x1, x2 = x[..., :R], x[..., R:]
    if mutation == "rope_sign":
        return np.concatenate([x1 * cs + x2 * sn, x2 * cs - x1 * sn], axis=-1)
    return np.concatenate([x1 * cs - x2 * sn, x2 * cs + x1 * sn], axis=-1)


def silu(x):
    return x / (1.0 + np.exp(-x))


def dequant(blocks, rows, cols):
    return dequantize_q8_0(blocks, rows * cols).reshape(rows, cols).astype(np.float64)


def linear(W, x, quantize_rows=True):
    """Linear::forward (src/attention.rs:101-136) with a Q8_0 weight W
    (dequantized, exact): x [M, K] -> [M, N].  M > 1 quantizes the
    activation rows to Q8_0 (the W8A8 path)."""
    x = np.asarray(x, np.float64)
    if x.shape[0] > 1 and quantize_rows and Q8_ACTIVATIONS[0]:
        M, K = x.shape
        x = dequantize_q8_0(quantize_q8_0(x.astype(np.float32)), M * K).reshape(M, K).astype(np.float64)
    return x @ W.T


def attention(q, K, V, offset, scale, mutation=None):
    """q [H, n, hd], K/V [H, L, hd] (after repeat_kv): softmax(q K^T * scale
    + mask) V with the causal mask for n > 1."""
    scores = np.einsum("hid,hjd->hij", q, K) * scale
    n, L = q.shape[1], K.shape[1]
    if n > 1:
        i = np.arange(n)[:, None]
        j = np.arange(L)[None, :]
        scores = np.where(j > i + (0 if mutation == "mask_offset" else offset), -np.inf, scores)
    mx = np.max(scores, axis=-1, keepdims=True)
    e = np.exp(scores - mx)
    p = e / np.sum(e, axis=-1, keepdims=True)
    return np.einsum("hij,hjd->hid", p, V)


def repeat_kv(x, groups, n_heads, mutation=None):
    """src/attention.rs:426-456: [n_kv, L, hd] -> [n_kv * groups, L, hd]."""
    if mutation == "gqa_mod":
        n_kv = x.shape[0]
        return x[np.arange(n_heads) % n_kv]
    return np.repeat(x, groups, axis=0)


class NumpyQwen3:
    """Qwen3ForCausalLM over host tensors in the include/lq8.h table order
    (Q8_0 blocks and f32 norms), with a KV cache."""

    def __init__(self, cfg, tensors, mutation=None):
        self.cfg = cfg
        self.mutation = mutation
        H, I, hd = cfg.hidden_size, cfg.intermediate_size, cfg.head_dim
        NH, NKV = cfg.num_attention_heads, cfg.num_key_value_heads
        self.E = dequant(tensors[0], cfg.vocab_size, H)
        self.final_norm = np.asarray(tensors[1], np.float64)
        self.layers = []
        for l in range(cfg.num_hidden_layers):
            t = tensors[2 + 11 * l: 13 + 11 * l]
            self.layers.append(dict(
                in_norm=np.asarray(t[0], np.float64), post_norm=np.asarray(t[1], np.float64),
                q_norm=np.asarray(t[2], np.float64), k_norm=np.asarray(t[3], np.float64),
                q=dequant(t[4], NH * hd, H), k=dequant(t[5], NKV * hd, H), v=dequant(t[6], NKV * hd, H),
                o=dequant(t[7], H, NH * hd), gate=dequant(t[8], I, H), up=dequant(t[9], I, H),
                down=dequant(t[10], H, I)))
        self.cos, self.sin = rope_tables(hd, cfg.max_position_embeddings, cfg.rope_theta)
        self.scale = float(np.float32(1.0) / np.sqrt(np.float32(hd)))
        self.clear_kv_cache()

    def clear_kv_cache(self):
        hd, NKV = self.cfg.head_dim, self.cfg.num_key_value_heads
        self.kc = [np.zeros((NKV, 0, hd)) for _ in self.layers]
        self.vc = [np.zeros((NKV, 0, hd)) for _ in self.layers]

    def forward(self, ids, offset, hidden_out=None):
        """Logits [vocab] (f64) of the last position; hidden_out (a list)
        receives the embedding output and each layer's output."""
        cfg, mu = self.cfg, self.mutation
        ids = np.asarray(ids, np.int64)
        if offset != self.kc[0].shape[1]:
            raise ValueError("offset must equal the cached length")
        n = ids.size
        hd, NH, NKV = cfg.head_dim, cfg.num_attention_heads, cfg.num_key_value_heads
        eps = cfg.rms_norm_eps
        h = self.E[ids].copy()
        if hidden_out is not None:
            hidden_out.append(h.copy())
        for li, L in enumerate(self.layers):
            x = rms_norm(h, L["in_norm"], eps)
            q = linear(L["q"], x).reshape(n, NH, hd).transpose(1, 0, 2)
            k = linear(L["k"], x).reshape(n, NKV, hd).transpose(1, 0, 2)
            v = linear(L["v"], x).reshape(n, NKV, hd).transpose(1, 0, 2)
            if mu == "qnorm_after_rope":
                q = rms_norm(rope(q, self.cos, self.sin, offset), L["q_norm"], eps)
                k = rms_norm(rope(k, self.cos, self.sin, offset), L["k_norm"], eps)
            else:
                q = rope(rms_norm(q, L["q_norm"], eps), self.cos, self.sin, offset, mu)
                k = rope(rms_norm(k, L["k_norm"], eps), self.cos, self.sin, offset, mu)
            self.kc[li] = np.concatenate([self.kc[li], k], axis=1)
            self.vc[li] = np.concatenate([self.vc[li], v], axis=1)
            K = repeat_kv(self.kc[li], NH // NKV, NH, mu)
            V = repeat_kv(self.vc[li], NH // NKV, NH, mu)
            a = attention(q, K, V, offset, self.scale, mu).transpose(1, 0, 2).reshape(n, NH * hd)
            h = (x if mu == "residual_normed" else h) + linear(L["o"], a)
            x = rms_norm(h, L["post_norm"], eps)
            g = linear(L["gate"], x)
            u = linear(L["up"], x)
            if mu == "swiglu_swap":
                g, u = u, g
            h = h + linear(L["down"], silu(g) * u)
            if hidden_out is not None:
                hidden_out.append(h.copy())
        last = h[-1:]
        x = last if mu == "no_final_norm" else rms_norm(last, self.final_norm, eps)
        return (x @ self.E.T)[0]


class NumpyMoeStack:
    """The library's Qwen3-MoE decoder layers (decode step of T independent
    sequences, sequence t in KV slot t at position pos[t]), in float64, from
    the same reference pieces: attention and norms as above, router
    p = softmax(scores), the top_k experts by p (ties to the lower index),
    weights renormalised over them, expert down(silu(gate x) * up x), combined
    as h2 + sum of w_e y_e.  Every projection is applied to one token at a
    time unless w8a8_batch is set (the library's rule, the default), in which
    case the attention projections of a batch of T > 1 tokens quantize their
    activation rows (W8A8)."""

    def __init__(self, cfg, tensors, w8a8_batch=True):
        self.cfg = cfg
        self.w8a8_batch = w8a8_batch
        H, hd, E, I = cfg.hidden_size, cfg.head_dim, cfg.num_experts, cfg.expert_intermediate_size
        NH, NKV = cfg.num_heads, cfg.num_kv_heads
        per = 8 + 3 * E
        self.layers = []
        for l in range(cfg.num_layers):
            t = tensors[per * l: per * (l + 1)]
            self.layers.append(dict(
                in_norm=np.asarray(t[0], np.float64), post_norm=np.asarray(t[1], np.float64),
                q_norm=np.asarray(t[2], np.float64), k_norm=np.asarray(t[3], np.float64),
                q=dequant(t[4], NH * hd, H), k=dequant(t[5], NKV * hd, H), v=dequant(t[6], NKV * hd, H),
                o=dequant(t[7], H, NH * hd),
                gate=[dequant(t[8 + e], I, H) for e in range(E)],
                up=[dequant(t[8 + E + e], I, H) for e in range(E)],
                down=[dequant(t[8 + 2 * E + e], H, I) for e in range(E)]))
        self.cos, self.sin = rope_tables(hd, cfg.max_positions, cfg.rope_theta)
        self.scale = float(np.float32(1.0) / np.sqrt(np.float32(hd)))
        self.kc = np.zeros((cfg.num_layers, cfg.max_batch, NKV, cfg.max_positions, hd))
        self.vc = np.zeros_like(self.kc)

    def route(self, s):
        s = np.asarray(s, np.float64)
        p = np.exp(s - s.max())
        p = p / p.sum()
        order = sorted(range(s.size), key=lambda e: (-p[e], e))[:self.cfg.top_k]
        w = p[order] / p[order].sum()
        return order, w

    def forward(self, hidden, scores, pos):
        cfg = self.cfg
        hd, NH, NKV, eps = cfg.head_dim, cfg.num_heads, cfg.num_kv_heads, cfg.rms_norm_eps
        h = np.asarray(hidden, np.float64).copy()
        T = h.shape[0]
        q8 = self.w8a8_batch and T > 1
        for li, L in enumerate(self.layers):
            x = rms_norm(h, L["in_norm"], eps)
            q = linear(L["q"], x, q8) if q8 else np.stack([linear(L["q"], x[t:t + 1])[0] for t in range(T)])
            k = linear(L["k"], x, q8) if q8 else np.stack([linear(L["k"], x[t:t + 1])[0] for t in range(T)])
            v = linear(L["v"], x, q8) if q8 else np.stack([linear(L["v"], x[t:t + 1])[0] for t in range(T)])
            a = np.zeros((T, NH * hd))
            for t in range(T):
                p = int(pos[t])
                qt = rope(rms_norm(q[t].reshape(NH, 1, hd), L["q_norm"], eps), self.cos, self.sin, p)
                kt = rope(rms_norm(k[t].reshape(NKV, 1, hd), L["k_norm"], eps), self.cos, self.sin, p)
                self.kc[li, t, :, p] = kt[:, 0]
                self.vc[li, t, :, p] = v[t].reshape(NKV, hd)
                K = repeat_kv(self.kc[li, t, :, :p + 1], NH // NKV, NH)
                V = repeat_kv(self.vc[li, t, :, :p + 1], NH // NKV, NH)
                a[t] = attention(qt, K, V, p, self.scale).reshape(NH * hd)
            o = linear(L["o"], a, q8) if q8 else np.stack([linear(L["o"], a[t:t + 1])[0] for t in range(T)])
            h2 = h + o
            x2 = rms_norm(h2, L["post_norm"], eps)
            out = h2.copy()
            for t in range(T):
                experts, w = self.route(scores[li][t])
                acc = np.zeros(cfg.hidden_size)
                for e, we in sorted(zip(experts, w)):
                    g = L["gate"][e] @ x2[t]
                    u = L["up"][e] @ x2[t]
                    acc = acc + we * (L["down"][e] @ (silu(g) * u))
                out[t] = h2[t] + acc
            h = out
        return h
