"""ctypes wrapper of the CPU oracle (TEST INFRASTRUCTURE).

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg import
this module, and only to check results against it.  The shipped library never
uses it.
Build with ``make -C oracle`` (done by __graft_entry__.build()).
"""
from __future__ import annotations

import ctypes as C
import os
from typing import Sequence

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
# LQ8_ORACLE_BUILD: another build directory (the sanitizer build, _build_san)
_BUILD = os.environ.get("LQ8_ORACLE_BUILD") or os.path.join(_HERE, "_build")
LIB_PATH = os.path.join(_BUILD, "liblq8_oracle.so")

QK = 32
BLOCK_BYTES = 34


class OrcConfig(C.Structure):
    _fields_ = [
        ("vocab_size", C.c_uint32), ("hidden_size", C.c_uint32), ("intermediate_size", C.c_uint32),
        ("num_layers", C.c_uint32), ("num_heads", C.c_uint32), ("num_kv_heads", C.c_uint32),
        ("head_dim", C.c_uint32), ("max_positions", C.c_uint32), ("rms_norm_eps", C.c_float),
        ("rope_theta", C.c_double),
    ]


class OrcMoeConfig(C.Structure):
    _fields_ = [
        ("hidden_size", C.c_uint32), ("num_heads", C.c_uint32), ("num_kv_heads", C.c_uint32),
        ("head_dim", C.c_uint32), ("num_experts", C.c_uint32), ("top_k", C.c_uint32),
        ("expert_intermediate_size", C.c_uint32), ("max_positions", C.c_uint32), ("max_batch", C.c_uint32),
        ("num_layers", C.c_uint32), ("rms_norm_eps", C.c_float), ("rope_theta", C.c_double),
    ]


_lib = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} not built (make -C oracle)")
        L = C.CDLL(LIB_PATH)
        vp, sz = C.c_void_p, C.c_size_t
        sigs = {
            "orc_f32_to_f16": (C.c_uint16, [C.c_float]),
            "orc_f16_to_f32": (C.c_float, [C.c_uint16]),
            "orc_bf16_round": (C.c_float, [C.c_float]),
            "orc_expf": (C.c_float, [C.c_float]),
            "orc_f32_to_f16_n": (None, [vp, vp, sz]),
            "orc_f16_to_f32_n": (None, [vp, vp, sz]),
            "orc_bf16_round_n": (None, [vp, vp, sz]),
            "orc_expf_n": (None, [vp, vp, sz]),
            "orc_set_sequential_sums": (None, [C.c_int]),
            "orc_set_libm_exp": (None, [C.c_int]),
            "orc_set_threads": (None, [C.c_int]),
            "orc_set_bf16_rounding": (None, [C.c_int]),
            "orc_set_activation_quantization": (None, [C.c_int]),
            "orc_quantize_q8_0": (C.c_int, [vp, sz, vp]),
            "orc_dequantize_q8_0": (C.c_int, [vp, sz, vp]),
            "orc_gemv_q8_0": (C.c_int, [vp, sz, sz, vp, vp]),
            "orc_gemm_q8_0": (C.c_int, [vp, sz, sz, vp, sz, vp]),
            "orc_linear_forward": (C.c_int, [vp, sz, sz, vp, sz, vp]),
            "orc_rms_norm": (C.c_int, [vp, vp, sz, sz, C.c_float, vp]),
            "orc_rope_tables": (C.c_int, [sz, sz, C.c_double, vp, vp]),
            "orc_rope_apply": (C.c_int, [vp, sz, sz, sz, vp, vp, sz, vp]),
            "orc_silu": (C.c_float, [C.c_float]),
            "orc_argmax_last": (C.c_uint32, [vp, sz]),
            "orc_sample": (C.c_int64, [vp, sz, vp, C.c_float, C.c_uint32, C.c_float, C.c_float, C.c_uint64,
                                       C.c_uint32]),
            "orc_model_new": (vp, [C.POINTER(OrcConfig), vp]),
            "orc_model_free": (None, [vp]),
            "orc_model_clear_kv_cache": (None, [vp]),
            "orc_model_forward": (C.c_int, [vp, vp, sz, sz, vp]),
            "orc_model_forward_with_intermediates": (C.c_int, [vp, vp, sz, sz, vp, vp, vp]),
            "orc_generate_greedy": (C.c_int, [vp, vp, sz, sz, vp, vp]),
            "orc_generate_greedy_ex": (C.c_int, [vp, vp, sz, sz, C.c_int, vp, vp]),
            "orc_moe_new": (vp, [C.POINTER(OrcMoeConfig), vp]),
            "orc_moe_free": (None, [vp]),
            "orc_moe_route": (C.c_int, [vp, sz, sz, sz, vp, vp]),
            "orc_moe_forward": (C.c_int, [vp, vp, vp, vp, sz]),
        }
        for name, (res, args) in sigs.items():
            f = getattr(L, name)
            f.restype = res
            f.argtypes = args
        _lib = L
    return _lib


def _p(a: np.ndarray):
    return C.c_void_p(a.ctypes.data)


def f32_to_f16_bits(x) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1)
    out = np.empty(x.size, dtype=np.uint16)
    lib().orc_f32_to_f16_n(_p(x), _p(out), x.size)
    return out


def f16_bits_to_f32(h) -> np.ndarray:
    h = np.ascontiguousarray(h, dtype=np.uint16).reshape(-1)
    out = np.empty(h.size, dtype=np.float32)
    lib().orc_f16_to_f32_n(_p(h), _p(out), h.size)
    return out


def bf16_round(x) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1)
    out = np.empty(x.size, dtype=np.float32)
    lib().orc_bf16_round_n(_p(x), _p(out), x.size)
    return out


def expf(x) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1)
    out = np.empty(x.size, dtype=np.float32)
    lib().orc_expf_n(_p(x), _p(out), x.size)
    return out


def set_sequential_sums(on: bool) -> None:
    lib().orc_set_sequential_sums(1 if on else 0)


def set_libm_exp(on: bool) -> None:
    """The decoder's softmax and SiLU exp: the C library's expf (on
    linux-gnu glibc's, which the reference's f32::exp calls) or orc_expf."""
    lib().orc_set_libm_exp(1 if on else 0)


def set_bf16_rounding(on: bool) -> None:
    """RmsNorm's bf16 roundings on (the default, the reference's numerics)
    or off (only to pin the decoder structure against a float64 restatement)."""
    lib().orc_set_bf16_rounding(1 if on else 0)


def set_activation_quantization(on: bool) -> None:
    """Rows > 1 through the W8A8 GEMM (the default) or every row through
    the W8A32 GEMV (only to pin the decoder structure)."""
    lib().orc_set_activation_quantization(1 if on else 0)


def set_threads(n: int) -> None:
    lib().orc_set_threads(int(n))


def quantize_q8_0(x) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1)
    out = np.empty(x.size // QK * BLOCK_BYTES, dtype=np.uint8)
    if lib().orc_quantize_q8_0(_p(x), x.size, _p(out)):
        raise ValueError("n must be a multiple of 32")
    return out


def dequantize_q8_0(blocks, n: int) -> np.ndarray:
    blocks = np.ascontiguousarray(blocks, dtype=np.uint8)
    out = np.empty(n, dtype=np.float32)
    if lib().orc_dequantize_q8_0(_p(blocks), n, _p(out)):
        raise ValueError("n must be a multiple of 32")
    return out


def gemv_q8_0(blocks, n_out: int, k_in: int, x) -> np.ndarray:
    blocks = np.ascontiguousarray(blocks, dtype=np.uint8)
    x = np.ascontiguousarray(x, dtype=np.float32)
    y = np.empty(n_out, dtype=np.float32)
    if lib().orc_gemv_q8_0(_p(blocks), n_out, k_in, _p(x), _p(y)):
        raise ValueError("bad shape")
    return y


def gemm_q8_0(blocks, n_out: int, k_in: int, x) -> np.ndarray:
    blocks = np.ascontiguousarray(blocks, dtype=np.uint8)
    x = np.ascontiguousarray(x, dtype=np.float32)
    m = x.size // k_in
    y = np.empty((m, n_out), dtype=np.float32)
    if lib().orc_gemm_q8_0(_p(blocks), n_out, k_in, _p(x), m, _p(y)):
        raise ValueError("bad shape")
    return y


def linear_forward(blocks, n_out: int, k_in: int, x) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    m = x.size // k_in
    y = np.empty((m, n_out), dtype=np.float32)
    blocks = np.ascontiguousarray(blocks, dtype=np.uint8)
    if lib().orc_linear_forward(_p(blocks), n_out, k_in, _p(x), m, _p(y)):
        raise ValueError("bad shape")
    return y


REF_LINEAR_PATH = os.path.join(_BUILD, "libref_linear_bf16.so")
_ref_lib = None


def ref_linear_forward_bf16(w_bf16, x) -> np.ndarray:
    """The reference's CPU Linear::forward on a BF16 weight (ref_linear_bf16.c):
    w_bf16 uint16 [n_out, k_in] (BF16 bits), x f32 [m, k_in] -> y f32 [m, n_out]."""
    global _ref_lib
    if _ref_lib is None:
        if not os.path.exists(REF_LINEAR_PATH):
            raise RuntimeError(f"{REF_LINEAR_PATH} not built (make -C oracle)")
        _ref_lib = C.CDLL(REF_LINEAR_PATH)
        _ref_lib.ref_linear_forward_bf16.restype = C.c_int
        _ref_lib.ref_linear_forward_bf16.argtypes = [C.c_void_p, C.c_size_t, C.c_size_t, C.c_void_p, C.c_size_t,
                                                     C.c_void_p]
    w = np.ascontiguousarray(w_bf16, dtype=np.uint16)
    xa = np.ascontiguousarray(x, dtype=np.float32)
    if xa.ndim == 1:
        xa = xa[None, :]
    n, k = w.shape
    if xa.shape[1] != k:
        raise ValueError(f"x has {xa.shape[1]} columns, the weight {k}")
    y = np.empty((xa.shape[0], n), dtype=np.float32)
    if _ref_lib.ref_linear_forward_bf16(_p(w), n, k, _p(xa), xa.shape[0], _p(y)) != 0:
        raise MemoryError("ref_linear_forward_bf16: allocation failed")
    return y


def rms_norm(x, weight, eps: float) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    w = np.ascontiguousarray(weight, dtype=np.float32)
    dim = w.size
    y = np.empty_like(x)
    lib().orc_rms_norm(_p(x), _p(w), x.size // dim, dim, eps, _p(y))
    return y


def rope_tables(head_dim: int, max_pos: int, theta: float):
    R = head_dim // 2
    c = np.empty((max_pos, R), dtype=np.float32)
    s = np.empty((max_pos, R), dtype=np.float32)
    if lib().orc_rope_tables(head_dim, max_pos, theta, _p(c), _p(s)):
        raise ValueError("head_dim must be a multiple of 4")
    return c, s


def rope_apply(x, cos_t, sin_t, offset: int) -> np.ndarray:
    """x: [heads, seq, head_dim]."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    h, l, d = x.shape
    y = np.empty_like(x)
    lib().orc_rope_apply(_p(x), h, l, d, _p(np.ascontiguousarray(cos_t)), _p(np.ascontiguousarray(sin_t)), offset,
                         _p(y))
    return y


def silu(x: float) -> float:
    return lib().orc_silu(x)


def argmax_last(x) -> int:
    x = np.ascontiguousarray(x, dtype=np.float32)
    return int(lib().orc_argmax_last(_p(x), x.size))


def sample(logits, counts, temperature: float, top_k: int, top_p: float, repetition_penalty: float, seed: int,
           step: int) -> int:
    """The library's sampling rule (lq8_sample_device), restated on the CPU."""
    x = np.ascontiguousarray(logits, dtype=np.float32)
    cnt = None if counts is None else np.ascontiguousarray(counts, dtype=np.uint32)
    t = lib().orc_sample(_p(x), x.size, _p(cnt) if cnt is not None else None, temperature, top_k, top_p,
                         repetition_penalty, seed & (2**64 - 1), step)
    if t < 0:
        raise ValueError("oracle sample failed")
    return int(t)


class Model:
    """Oracle Qwen3ForCausalLM over host tensors in the include/lq8.h table order."""

    def __init__(self, cfg, tensors: Sequence[np.ndarray]):
        self.cfg = cfg
        self._keep = [np.ascontiguousarray(t) for t in tensors]
        arr = (C.c_void_p * len(self._keep))(*[t.ctypes.data for t in self._keep])
        self._c = OrcConfig(cfg.vocab_size, cfg.hidden_size, cfg.intermediate_size, cfg.num_hidden_layers,
                            cfg.num_attention_heads, cfg.num_key_value_heads, cfg.head_dim,
                            cfg.max_position_embeddings, cfg.rms_norm_eps, cfg.rope_theta)
        self.h = lib().orc_model_new(C.byref(self._c), arr)
        if not self.h:
            raise MemoryError("oracle model allocation failed")

    def close(self):
        if self.h:
            lib().orc_model_free(self.h)
            self.h = None

    def __del__(self):
        self.close()

    def clear_kv_cache(self):
        lib().orc_model_clear_kv_cache(self.h)

    def forward(self, ids, offset: int) -> np.ndarray:
        ids = np.ascontiguousarray(ids, dtype=np.uint32)
        logits = np.empty(self.cfg.vocab_size, dtype=np.float32)
        rc = lib().orc_model_forward(self.h, _p(ids), ids.size, offset, _p(logits))
        if rc:
            raise ValueError(f"oracle forward failed ({rc})")
        return logits

    def forward_with_intermediates(self, ids, offset: int):
        ids = np.ascontiguousarray(ids, dtype=np.uint32)
        n, H = ids.size, self.cfg.hidden_size
        hidden = np.empty((self.cfg.num_hidden_layers + 1, n, H), dtype=np.float32)
        fin = np.empty((n, H), dtype=np.float32)
        logits = np.empty(self.cfg.vocab_size, dtype=np.float32)
        rc = lib().orc_model_forward_with_intermediates(self.h, _p(ids), n, offset, _p(hidden), _p(fin), _p(logits))
        if rc:
            raise ValueError(f"oracle forward failed ({rc})")
        return hidden, fin, logits

    def generate_greedy(self, prompt, max_new: int, feed_first: bool = False):
        """generate() with the greedy sampler.  feed_first: the reference's
        loop as written, where every decode step forwards the first
        generated token (src/generate.rs:632-650)."""
        ids = np.ascontiguousarray(prompt, dtype=np.uint32)
        toks = np.empty(max_new, dtype=np.uint32)
        margins = np.empty(max_new, dtype=np.float32)
        rc = lib().orc_generate_greedy_ex(self.h, _p(ids), ids.size, max_new, 1 if feed_first else 0, _p(toks),
                                          _p(margins))
        if rc:
            raise ValueError(f"oracle generate failed ({rc})")
        return toks, margins

    def generate_sampled(self, prompt, max_new: int, temperature: float, top_k: int, top_p: float,
                         repetition_penalty: float, seed: int, eos_token_ids=(), feed_first: bool = False) -> np.ndarray:
        """generate() (src/generate.rs:611-664) with the sampling rule:
        prefill, then one sampled token per step (step t draws with counter t;
        the penalty counts the tokens generated before it); the loop ends at
        the first token in eos_token_ids, which is kept and not forwarded.
        feed_first: every decode step forwards the first generated token (the
        reference's loop as written)."""
        ids = np.ascontiguousarray(prompt, dtype=np.uint32)
        eos = set(int(e) for e in eos_token_ids)
        self.clear_kv_cache()
        logits = self.forward(ids, 0)
        counts = np.zeros(self.cfg.vocab_size, dtype=np.uint32)
        toks = []
        for t in range(max_new):
            tok = sample(logits, counts, temperature, top_k, top_p, repetition_penalty, seed, t)
            toks.append(tok)
            counts[tok] += 1
            if tok in eos:
                break
            if t + 1 < max_new:
                logits = self.forward([toks[0] if feed_first else tok], ids.size + t)
        return np.array(toks, dtype=np.uint32)


def random_q8_tensors(cfg, seed: int, std: float = 0.02, layer_std: float = None, norm_jitter: float = 0.0):
    """Small random model in table order (numpy normal draws, oracle quantizer).
    layer_std: the std of the decoder layers' matrices (default std, the
    embedding keeps std); norm_jitter: norm weights 1 + jitter * N(0, 1)
    instead of 1.  A layer_std of 0.08 with norm_jitter 0.1 gives greedy
    tokens that vary from step to step (the plain N(0, 0.02) model repeats
    one token)."""
    rng = np.random.default_rng(seed)
    out = []
    for i in range(cfg.tensor_count()):
        kind, shape = cfg.tensor_shape(i)
        if kind == "f32":
            out.append((1.0 + norm_jitter * rng.standard_normal(shape)).astype(np.float32) if norm_jitter
                       else np.ones(shape, dtype=np.float32))
        else:
            sd = std if (i == 0 or layer_std is None) else layer_std
            w = (rng.standard_normal(shape) * sd).astype(np.float32)
            out.append(quantize_q8_0(w))
    return out


def moe_route(scores, top_k: int):
    """Router of the MoE layer: scores [T, E] -> (expert ids [T, k] in rank
    order, renormalised weights [T, k])."""
    scores = np.ascontiguousarray(scores, dtype=np.float32)
    T, E = scores.shape
    ids = np.empty((T, top_k), dtype=np.uint32)
    w = np.empty((T, top_k), dtype=np.float32)
    if lib().orc_moe_route(_p(scores), T, E, top_k, _p(ids), _p(w)):
        raise ValueError("bad router shape")
    return ids, w


class MoeStack:
    """Oracle Qwen3-MoE decoder layers over host tensors (table order of
    orc_moe_new: per layer 4 f32 norms, q/k/v/o, then gate[E], up[E], down[E]
    as Q8_0 blocks); one KV cache slot per sequence of the batch."""

    def __init__(self, cfg, tensors: Sequence[np.ndarray]):
        self.cfg = cfg
        self._keep = [np.ascontiguousarray(t) for t in tensors]
        self._arr = (C.c_void_p * len(self._keep))(*[t.ctypes.data for t in self._keep])
        self._c = OrcMoeConfig(cfg.hidden_size, cfg.num_heads, cfg.num_kv_heads, cfg.head_dim, cfg.num_experts,
                               cfg.top_k, cfg.expert_intermediate_size, cfg.max_positions, cfg.max_batch,
                               cfg.num_layers, cfg.rms_norm_eps, cfg.rope_theta)
        self.h = lib().orc_moe_new(C.byref(self._c), self._arr)
        if not self.h:
            raise MemoryError("oracle MoE allocation failed")

    def close(self):
        if self.h:
            lib().orc_moe_free(self.h)
            self.h = None

    def __del__(self):
        self.close()

    def forward(self, hidden, scores, pos):
        """hidden [T, H] (returned updated), scores [layers, T, E], pos [T]."""
        h = np.array(hidden, dtype=np.float32, copy=True, order="C")
        sc = np.ascontiguousarray(scores, dtype=np.float32)
        p = np.ascontiguousarray(pos, dtype=np.uint32)
        rc = lib().orc_moe_forward(self.h, _p(h), _p(sc), _p(p), p.size)
        if rc:
            raise ValueError(f"oracle MoE forward failed ({rc})")
        return h
