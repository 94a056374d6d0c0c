"""Host-side mirror of lluda-inference's linear-layer / model API over liblq8.so.

The reference exposes ``Linear::new(weight)`` / ``Linear::forward(x)``
(src/attention.rs:63-136), ``Tensor::matmul`` (src/tensor.rs:804),
``Qwen3ForCausalLM::{load, forward, clear_kv_cache}`` (src/model.rs:273-398)
and ``generate`` (src/generate.rs:611-664).  This module keeps those names and
argument meanings on top of the C ABI in include/lq8.h.  Errors surface as
``LludaError`` subclasses named after the reference's error kinds
(src/error.rs:17-97).  There is no CPU fallback: without the shared library or
without a gfx950 device every call raises.
"""
from __future__ import annotations

import ctypes as C
import os
from dataclasses import dataclass
from typing import Optional, Sequence

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
# LQ8_LIBRARY: another build of the library (the sanitizer or trace build)
LIB_PATH = os.environ.get("LQ8_LIBRARY") or os.path.join(_HERE, "liblq8.so")

QK = 32
BLOCK_BYTES = 34


class LludaError(RuntimeError):
    """Base error; ``status`` is the lq8_status code."""

    status = -1

    def __init__(self, msg: str, status: int | None = None):
        super().__init__(msg)
        if status is not None:
            self.status = status


class ShapeMismatch(LludaError):
    status = 1


class DTypeMismatch(LludaError):
    status = 2


class DimOutOfRange(LludaError):
    status = 3


class InvalidArgument(LludaError):
    status = 4


class NoDevice(LludaError):
    status = 5


class DeviceError(LludaError):
    status = 6


class OutOfMemory(LludaError):
    status = 7


class ModelError(LludaError):
    status = 8


DTYPE_Q8_0, DTYPE_F32, DTYPE_BF16 = 0, 1, 2  # lq8_dtype

_ERRORS = {c.status: c for c in (ShapeMismatch, DTypeMismatch, DimOutOfRange, InvalidArgument, NoDevice,
                                  DeviceError, OutOfMemory, ModelError)}


class Qwen3ConfigC(C.Structure):
    _fields_ = [
        ("vocab_size", C.c_uint32), ("hidden_size", C.c_uint32), ("intermediate_size", C.c_uint32),
        ("num_layers", C.c_uint32), ("num_heads", C.c_uint32), ("num_kv_heads", C.c_uint32),
        ("head_dim", C.c_uint32), ("max_positions", C.c_uint32), ("rms_norm_eps", C.c_float),
        ("rope_theta", C.c_double),
    ]


class GemvProblemC(C.Structure):
    _fields_ = [("w", C.c_void_p), ("x", C.c_void_p), ("y", C.c_void_p)]


class MoeConfigC(C.Structure):
    _fields_ = [
        ("hidden_size", C.c_uint32), ("num_heads", C.c_uint32), ("num_kv_heads", C.c_uint32),
        ("head_dim", C.c_uint32), ("num_experts", C.c_uint32), ("top_k", C.c_uint32),
        ("expert_intermediate_size", C.c_uint32), ("max_positions", C.c_uint32), ("max_batch", C.c_uint32),
        ("num_layers", C.c_uint32), ("rms_norm_eps", C.c_float), ("rope_theta", C.c_double),
    ]


class GenStatsC(C.Structure):
    _fields_ = [("prefill_ms", C.c_double), ("decode_ms", C.c_double), ("decode_tokens_per_s", C.c_double),
                ("used_graph", C.c_uint32), ("used_persistent", C.c_uint32)]


class PersistInfoC(C.Structure):
    _fields_ = [(n, C.c_uint32) for n in (
        "supported", "o_chunk_blocks", "o_chunks", "down_chunk_pairs", "down_chunks", "lds_bytes", "lds_gather_floats",
        "lds_xs_offset", "lds_gs_offset", "lds_red_offset", "lds_attention_floats", "lds_combine_floats",
        "direct_segments")]


class SamplingC(C.Structure):
    _fields_ = [("temperature", C.c_float), ("top_k", C.c_uint32), ("top_p", C.c_float),
                ("repetition_penalty", C.c_float), ("seed", C.c_uint64)]


# lq8_generate_ex flag: the reference's generate() loop as written
GEN_FEED_FIRST_TOKEN = 1
# lq8_quantize_activations_device sources
ACT_PLAIN, ACT_RMSNORM, ACT_SILU_MUL = 0, 1, 2

_lib: Optional[C.CDLL] = None

# (name, restype, argtypes) of every exported entry point.
_SIGS = [
    ("lq8_version", C.c_char_p, []),
    ("lq8_last_error", C.c_char_p, []),
    ("lq8_device_count", C.c_int, [C.POINTER(C.c_int)]),
    ("lq8_q8_0_bytes", C.c_size_t, [C.c_size_t]),
    ("lq8_quantize_q8_0", C.c_int, [C.c_void_p, C.c_size_t, C.c_void_p]),
    ("lq8_dequantize_q8_0", C.c_int, [C.c_void_p, C.c_size_t, C.c_void_p]),
    ("lq8_init", C.c_int, [C.c_int, C.POINTER(C.c_void_p)]),
    ("lq8_shutdown", C.c_int, [C.c_void_p]),
    ("lq8_synchronize", C.c_int, [C.c_void_p]),
    ("lq8_device_alloc", C.c_int, [C.c_void_p, C.c_size_t, C.POINTER(C.c_void_p)]),
    ("lq8_device_free", C.c_int, [C.c_void_p, C.c_void_p]),
    ("lq8_copy_to_device", C.c_int, [C.c_void_p, C.c_void_p, C.c_void_p, C.c_size_t]),
    ("lq8_copy_to_host", C.c_int, [C.c_void_p, C.c_void_p, C.c_void_p, C.c_size_t]),
    ("lq8_copy_device", C.c_int, [C.c_void_p, C.c_void_p, C.c_void_p, C.c_size_t]),
    ("lq8_timer_start", C.c_int, [C.c_void_p]),
    ("lq8_timer_stop", C.c_int, [C.c_void_p, C.POINTER(C.c_float)]),
    ("lq8_weight_upload", C.c_int, [C.c_void_p, C.c_void_p, C.c_size_t, C.c_size_t, C.POINTER(C.c_void_p)]),
    ("lq8_weight_quantize_upload", C.c_int,
     [C.c_void_p, C.c_void_p, C.c_size_t, C.c_size_t, C.POINTER(C.c_void_p)]),
    ("lq8_weight_quantize_upload_bf16", C.c_int,
     [C.c_void_p, C.c_void_p, C.c_size_t, C.c_size_t, C.POINTER(C.c_void_p)]),
    ("lq8_weight_random", C.c_int,
     [C.c_void_p, C.c_size_t, C.c_size_t, C.c_uint64, C.c_uint64, C.c_float, C.POINTER(C.c_void_p)]),
    ("lq8_weight_download", C.c_int, [C.c_void_p, C.c_void_p, C.c_void_p]),
    ("lq8_weight_shape", C.c_int, [C.c_void_p, C.POINTER(C.c_size_t), C.POINTER(C.c_size_t)]),
    ("lq8_weight_free", C.c_int, [C.c_void_p]),
    ("lq8_quantize_q8_0_device", C.c_int, [C.c_void_p, C.c_void_p, C.c_size_t, C.c_void_p]),
    ("lq8_weight_dequantize_rows_device", C.c_int, [C.c_void_p, C.c_void_p, C.c_size_t, C.c_size_t, C.c_void_p]),
    ("lq8_rms_norm_device", C.c_int, [C.c_void_p, C.c_void_p, C.c_void_p, C.c_size_t, C.c_size_t, C.c_float,
                                      C.c_void_p]),
    ("lq8_silu_device", C.c_int, [C.c_void_p, C.c_void_p, C.c_size_t, C.c_void_p]),
    ("lq8_linear_forward", C.c_int, [C.c_void_p, C.c_void_p, C.c_void_p, C.c_size_t, C.c_void_p]),
    ("lq8_linear_forward_device", C.c_int, [C.c_void_p, C.c_void_p, C.c_void_p, C.c_size_t, C.c_void_p]),
    ("lq8_gemv_q8_0_device", C.c_int, [C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p]),
    ("lq8_gemm_q8_0_device", C.c_int, [C.c_void_p, C.c_void_p, C.c_void_p, C.c_size_t, C.c_void_p]),
    ("lq8_gemv_grouped_device", C.c_int, [C.c_void_p, C.c_void_p, C.c_size_t]),
    ("lq8_bench_gemv", C.c_int, [C.c_void_p, C.c_void_p, C.c_size_t, C.c_int, C.c_int, C.POINTER(C.c_float)]),
    ("lq8_model_tensor_count", C.c_size_t, [C.POINTER(Qwen3ConfigC)]),
    ("lq8_model_tensor_bytes", C.c_int, [C.POINTER(Qwen3ConfigC), C.c_size_t, C.POINTER(C.c_size_t)]),
    ("lq8_model_create", C.c_int, [C.c_void_p, C.POINTER(Qwen3ConfigC), C.c_void_p, C.POINTER(C.c_void_p)]),
    ("lq8_model_create_typed", C.c_int,
     [C.c_void_p, C.POINTER(Qwen3ConfigC), C.c_void_p, C.c_void_p, C.POINTER(C.c_void_p)]),
    ("lq8_model_create_random", C.c_int,
     [C.c_void_p, C.POINTER(Qwen3ConfigC), C.c_uint64, C.c_float, C.POINTER(C.c_void_p)]),
    ("lq8_model_export_tensor", C.c_int, [C.c_void_p, C.c_size_t, C.c_void_p]),
    ("lq8_model_clear_kv_cache", C.c_int, [C.c_void_p]),
    ("lq8_model_forward", C.c_int, [C.c_void_p, C.c_void_p, C.c_size_t, C.c_size_t, C.c_void_p]),
    ("lq8_model_forward_with_intermediates", C.c_int,
     [C.c_void_p, C.c_void_p, C.c_size_t, C.c_size_t, C.c_void_p, C.c_void_p, C.c_void_p]),
    ("lq8_generate_greedy", C.c_int,
     [C.c_void_p, C.c_void_p, C.c_size_t, C.c_size_t, C.c_void_p, C.POINTER(GenStatsC)]),
    ("lq8_sample_device", C.c_int,
     [C.c_void_p, C.c_void_p, C.c_size_t, C.c_void_p, C.POINTER(SamplingC), C.c_uint32, C.c_void_p]),
    ("lq8_generate", C.c_int,
     [C.c_void_p, C.c_void_p, C.c_size_t, C.c_size_t, C.POINTER(SamplingC), C.c_void_p, C.c_size_t, C.c_void_p,
      C.POINTER(C.c_size_t), C.POINTER(GenStatsC)]),
    ("lq8_generate_ex", C.c_int,
     [C.c_void_p, C.c_void_p, C.c_size_t, C.c_size_t, C.POINTER(SamplingC), C.c_void_p, C.c_size_t, C.c_uint32,
      C.c_void_p, C.POINTER(C.c_size_t), C.POINTER(GenStatsC)]),
    ("lq8_quantize_activations_device", C.c_int,
     [C.c_void_p, C.c_int, C.c_void_p, C.c_void_p, C.c_size_t, C.c_size_t, C.c_float, C.c_void_p]),
    ("lq8_linear_forward_device_noalloc", C.c_int, [C.c_void_p, C.c_void_p, C.c_void_p, C.c_size_t, C.c_void_p]),
    ("lq8_bench_grid_sync", C.c_int,
     [C.c_void_p, C.c_int, C.c_int, C.c_int, C.POINTER(C.c_float), C.POINTER(C.c_uint32), C.POINTER(C.c_uint32)]),
    ("lq8_bench_floors", C.c_int, [C.c_void_p, C.c_int, C.c_int, C.c_size_t, C.c_int, C.POINTER(C.c_double)]),
    ("lq8_persist_trace", C.c_int, [C.c_void_p, C.c_void_p, C.c_size_t]),
    ("lq8_persist_plan", C.c_int, [C.POINTER(Qwen3ConfigC), C.c_uint32, C.POINTER(PersistInfoC)]),
    ("lq8_model_persist_picks", C.c_int,
     [C.c_void_p, C.c_uint32, C.c_void_p, C.c_void_p, C.c_size_t, C.POINTER(C.c_size_t)]),
    ("lq8_model_free", C.c_int, [C.c_void_p]),
    ("lq8_moe_tensor_count", C.c_size_t, [C.POINTER(MoeConfigC)]),
    ("lq8_moe_tensor_bytes", C.c_int, [C.POINTER(MoeConfigC), C.c_size_t, C.POINTER(C.c_size_t)]),
    ("lq8_moe_create", C.c_int, [C.c_void_p, C.POINTER(MoeConfigC), C.c_void_p, C.POINTER(C.c_void_p)]),
    ("lq8_moe_create_random", C.c_int,
     [C.c_void_p, C.POINTER(MoeConfigC), C.c_uint64, C.c_float, C.POINTER(C.c_void_p)]),
    ("lq8_moe_export_tensor", C.c_int, [C.c_void_p, C.c_size_t, C.c_void_p]),
    ("lq8_moe_weight_bytes", C.c_int, [C.c_void_p, C.POINTER(C.c_size_t)]),
    ("lq8_moe_forward_device", C.c_int, [C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p, C.c_size_t]),
    ("lq8_moe_forward", C.c_int, [C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p, C.c_size_t]),
    ("lq8_moe_routing", C.c_int, [C.c_void_p, C.c_void_p, C.c_void_p]),
    ("lq8_moe_clear_kv_cache", C.c_int, [C.c_void_p]),
    ("lq8_moe_free", C.c_int, [C.c_void_p]),
]

EXPORTED = [s[0] for s in _SIGS]


def lib() -> C.CDLL:
    """Load liblq8.so (built in-tree).  Raises if it was not built."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise LludaError(f"{LIB_PATH} not built (run __graft_entry__.build())")
        L = C.CDLL(LIB_PATH)
        for name, res, args in _SIGS:
            f = getattr(L, name)
            f.restype = res
            f.argtypes = args
        _lib = L
    return _lib


def _check(status: int) -> None:
    if status != 0:
        msg = lib().lq8_last_error().decode(errors="replace")
        raise _ERRORS.get(status, LludaError)(msg, status)


def _ptr(a: np.ndarray) -> C.c_void_p:
    return C.c_void_p(a.ctypes.data)


def version() -> str:
    return lib().lq8_version().decode()


def device_count() -> int:
    n = C.c_int(0)
    _check(lib().lq8_device_count(C.byref(n)))
    return n.value


# ---- host Q8_0 format ----------------------------------------------------------

def quantize_q8_0(x: np.ndarray) -> np.ndarray:
    """f32 array (size multiple of 32) -> uint8 AoS blocks (34 bytes each)."""
    x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1)
    out = np.empty(x.size // QK * BLOCK_BYTES, dtype=np.uint8)
    _check(lib().lq8_quantize_q8_0(_ptr(x), x.size, _ptr(out)))
    return out


def dequantize_q8_0(blocks: np.ndarray, n: int) -> np.ndarray:
    blocks = np.ascontiguousarray(blocks, dtype=np.uint8)
    y = np.empty(n, dtype=np.float32)
    _check(lib().lq8_dequantize_q8_0(_ptr(blocks), n, _ptr(y)))
    return y


# ---- device context and buffers ----------------------------------------------------

class Context:
    """One device + one stream (the reference's global GPU context, src/gpu/mod.rs:129-178)."""

    def __init__(self, device: int = 0):
        h = C.c_void_p()
        _check(lib().lq8_init(device, C.byref(h)))
        self.handle = h

    def close(self) -> None:
        if self.handle:
            _check(lib().lq8_shutdown(self.handle))
            self.handle = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def synchronize(self) -> None:
        _check(lib().lq8_synchronize(self.handle))

    def timer_start(self) -> None:
        _check(lib().lq8_timer_start(self.handle))

    def timer_stop(self) -> float:
        ms = C.c_float(0.0)
        _check(lib().lq8_timer_stop(self.handle, C.byref(ms)))
        return ms.value


class DeviceBuffer:
    """A device allocation with explicit host copies (no implicit transfers)."""

    def __init__(self, ctx: Context, nbytes: int):
        self.ctx = ctx
        self.nbytes = int(nbytes)
        p = C.c_void_p()
        _check(lib().lq8_device_alloc(ctx.handle, self.nbytes, C.byref(p)))
        self.ptr = p

    @classmethod
    def from_array(cls, ctx: Context, a: np.ndarray) -> "DeviceBuffer":
        a = np.ascontiguousarray(a)
        b = cls(ctx, a.nbytes)
        b.upload(a)
        return b

    def upload(self, a: np.ndarray) -> None:
        a = np.ascontiguousarray(a)
        if a.nbytes > self.nbytes:
            raise ShapeMismatch("upload larger than buffer")
        _check(lib().lq8_copy_to_device(self.ctx.handle, self.ptr, _ptr(a), a.nbytes))

    def download(self, dtype, count: int) -> np.ndarray:
        out = np.empty(count, dtype=dtype)
        if out.nbytes > self.nbytes:
            raise ShapeMismatch("download larger than buffer")
        _check(lib().lq8_copy_to_host(self.ctx.handle, _ptr(out), self.ptr, out.nbytes))
        return out

    def free(self) -> None:
        if self.ptr:
            _check(lib().lq8_device_free(self.ctx.handle, self.ptr))
            self.ptr = None


def rms_norm_device(ctx: "Context", x: np.ndarray, w: np.ndarray, eps: float) -> np.ndarray:
    """RmsNorm::forward on the device over the rows of x."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    w = np.ascontiguousarray(w, dtype=np.float32)
    dx, dw = DeviceBuffer.from_array(ctx, x), DeviceBuffer.from_array(ctx, w)
    dy = DeviceBuffer(ctx, x.nbytes)
    try:
        _check(lib().lq8_rms_norm_device(ctx.handle, dx.ptr, dw.ptr, x.size // w.size, w.size, eps, dy.ptr))
        return dy.download(np.float32, x.size).reshape(x.shape)
    finally:
        dx.free(); dw.free(); dy.free()


def silu_device(ctx: "Context", x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    dx, dy = DeviceBuffer.from_array(ctx, x), DeviceBuffer(ctx, x.nbytes)
    try:
        _check(lib().lq8_silu_device(ctx.handle, dx.ptr, x.size, dy.ptr))
        return dy.download(np.float32, x.size).reshape(x.shape)
    finally:
        dx.free(); dy.free()


class Q8Weight:
    """A Q8_0 weight [n_out, k_in] resident on the device (uploaded once)."""

    def __init__(self, ctx: Context, handle: C.c_void_p):
        self.ctx = ctx
        self.handle = handle
        n, k = C.c_size_t(), C.c_size_t()
        _check(lib().lq8_weight_shape(handle, C.byref(n), C.byref(k)))
        self.n_out, self.k_in = n.value, k.value

    @classmethod
    def from_blocks(cls, ctx: Context, blocks: np.ndarray, n_out: int, k_in: int) -> "Q8Weight":
        blocks = np.ascontiguousarray(blocks, dtype=np.uint8)
        if blocks.size != n_out * (k_in // QK) * BLOCK_BYTES:
            raise ShapeMismatch(f"expected {n_out * (k_in // QK) * BLOCK_BYTES} bytes, got {blocks.size}")
        h = C.c_void_p()
        _check(lib().lq8_weight_upload(ctx.handle, _ptr(blocks), n_out, k_in, C.byref(h)))
        return cls(ctx, h)

    @classmethod
    def quantize(cls, ctx: Context, w: np.ndarray) -> "Q8Weight":
        w = np.ascontiguousarray(w, dtype=np.float32)
        if w.ndim != 2:
            raise ShapeMismatch("weight must be 2-D [out_features, in_features]")
        h = C.c_void_p()
        _check(lib().lq8_weight_quantize_upload(ctx.handle, _ptr(w), w.shape[0], w.shape[1], C.byref(h)))
        return cls(ctx, h)

    @classmethod
    def random(cls, ctx: Context, n_out: int, k_in: int, seed: int, stream: int = 0, std: float = 0.02):
        h = C.c_void_p()
        _check(lib().lq8_weight_random(ctx.handle, n_out, k_in, seed, stream, std, C.byref(h)))
        return cls(ctx, h)

    def download(self) -> np.ndarray:
        out = np.empty(self.n_out * (self.k_in // QK) * BLOCK_BYTES, dtype=np.uint8)
        _check(lib().lq8_weight_download(self.ctx.handle, self.handle, _ptr(out)))
        return out

    def free(self) -> None:
        if self.handle:
            _check(lib().lq8_weight_free(self.handle))
            self.handle = None


class Linear:
    """``Linear`` of src/attention.rs:33-137 on a Q8_0 weight: y = x @ W^T."""

    def __init__(self, weight: Q8Weight):
        self.weight = weight

    @classmethod
    def new(cls, weight: Q8Weight) -> "Linear":
        return cls(weight)

    def forward(self, x: np.ndarray) -> np.ndarray:
        x = np.ascontiguousarray(x, dtype=np.float32)
        if x.ndim < 1 or x.shape[-1] != self.weight.k_in:
            raise ShapeMismatch(f"expected last dim {self.weight.k_in}, got {x.shape}")
        m = int(np.prod(x.shape[:-1])) if x.ndim > 1 else 1
        y = np.empty((m, self.weight.n_out), dtype=np.float32)
        _check(lib().lq8_linear_forward(self.weight.ctx.handle, self.weight.handle, _ptr(x), m, _ptr(y)))
        return y.reshape(tuple(x.shape[:-1]) + (self.weight.n_out,))

    def forward_device(self, x: DeviceBuffer, m: int, y: DeviceBuffer) -> None:
        _check(lib().lq8_linear_forward_device(self.weight.ctx.handle, self.weight.handle, x.ptr, m, y.ptr))


# ---- Qwen3 -------------------------------------------------------------------

@dataclass
class Qwen3Config:
    """The fields of Qwen3Config (src/config.rs:15-82) that the decoder uses."""

    vocab_size: int = 151936
    hidden_size: int = 1024
    intermediate_size: int = 3072
    num_hidden_layers: int = 28
    num_attention_heads: int = 16
    num_key_value_heads: int = 8
    head_dim: int = 128
    max_position_embeddings: int = 4096
    rms_norm_eps: float = 1e-6
    rope_theta: float = 1e6

    def c(self) -> Qwen3ConfigC:
        return Qwen3ConfigC(self.vocab_size, self.hidden_size, self.intermediate_size, self.num_hidden_layers,
                            self.num_attention_heads, self.num_key_value_heads, self.head_dim,
                            self.max_position_embeddings, self.rms_norm_eps, self.rope_theta)

    def tensor_count(self) -> int:
        return 2 + 11 * self.num_hidden_layers

    def tensor_shape(self, idx: int):
        """(kind, shape) of tensor ``idx`` in the table order of include/lq8.h."""
        H, I, hd = self.hidden_size, self.intermediate_size, self.head_dim
        QD, KD = self.num_attention_heads * hd, self.num_key_value_heads * hd
        if idx == 0:
            return "q8", (self.vocab_size, H)
        if idx == 1:
            return "f32", (H,)
        k = (idx - 2) % 11
        return [("f32", (H,)), ("f32", (H,)), ("f32", (hd,)), ("f32", (hd,)), ("q8", (QD, H)), ("q8", (KD, H)),
                ("q8", (KD, H)), ("q8", (H, QD)), ("q8", (I, H)), ("q8", (I, H)), ("q8", (H, I))][k]


def qwen3_0_6b(max_positions: int = 4096) -> Qwen3Config:
    return Qwen3Config(max_position_embeddings=max_positions)


def qwen3_1_7b(max_positions: int = 4096) -> Qwen3Config:
    """Qwen3-1.7B's shapes (its config.json): hidden 2048, intermediate 6144,
    28 layers, 16 query and 8 kv heads of 128, vocab 151936, tied embedding;
    the other fields as Qwen3-0.6B's."""
    return Qwen3Config(hidden_size=2048, intermediate_size=6144, max_position_embeddings=max_positions)


def qwen3_4b(max_positions: int = 4096) -> Qwen3Config:
    """Qwen3-4B's shapes (its config.json): hidden 2560, intermediate 9728,
    36 layers, 32 query and 8 kv heads of 128, vocab 151936, tied embedding;
    the other fields as Qwen3-0.6B's."""
    return Qwen3Config(hidden_size=2560, intermediate_size=9728, num_hidden_layers=36, num_attention_heads=32,
                       num_key_value_heads=8, max_position_embeddings=max_positions)


class Qwen3ForCausalLM:
    """src/model.rs:245-398 on Q8_0 weights."""

    def __init__(self, ctx: Context, cfg: Qwen3Config, handle: C.c_void_p):
        self.ctx, self.cfg, self.handle = ctx, cfg, handle
        self._c = cfg.c()

    @classmethod
    def load(cls, ctx: Context, cfg: Qwen3Config, tensors: Sequence[np.ndarray]) -> "Qwen3ForCausalLM":
        """From host tensors (Q8_0 AoS blocks or f32 norms) in table order."""
        if len(tensors) != cfg.tensor_count():
            raise ModelError(f"expected {cfg.tensor_count()} tensors, got {len(tensors)}")
        keep = [np.ascontiguousarray(t) for t in tensors]
        arr = (C.c_void_p * len(keep))(*[t.ctypes.data for t in keep])
        h = C.c_void_p()
        c = cfg.c()
        _check(lib().lq8_model_create(ctx.handle, C.byref(c), arr, C.byref(h)))
        return cls(ctx, cfg, h)

    @classmethod
    def random(cls, ctx: Context, cfg: Qwen3Config, seed: int, std: float = 0.02) -> "Qwen3ForCausalLM":
        h = C.c_void_p()
        c = cfg.c()
        _check(lib().lq8_model_create_random(ctx.handle, C.byref(c), seed, std, C.byref(h)))
        return cls(ctx, cfg, h)

    @classmethod
    def load_typed(cls, ctx: Context, cfg: Qwen3Config, tensors: Sequence[np.ndarray],
                   dtypes: Sequence[int]) -> "Qwen3ForCausalLM":
        """Table-order tensors with a dtype each (DTYPE_Q8_0 blocks, DTYPE_F32 or
        DTYPE_BF16 rows); BF16/F32 matrices are quantized on the device."""
        if len(tensors) != cfg.tensor_count() or len(dtypes) != cfg.tensor_count():
            raise ModelError(f"expected {cfg.tensor_count()} tensors and dtypes")
        keep = [np.ascontiguousarray(t) for t in tensors]
        arr = (C.c_void_p * len(keep))(*[t.ctypes.data for t in keep])
        dt = np.ascontiguousarray(dtypes, dtype=np.int32)
        h = C.c_void_p()
        c = cfg.c()
        _check(lib().lq8_model_create_typed(ctx.handle, C.byref(c), arr, _ptr(dt), C.byref(h)))
        return cls(ctx, cfg, h)

    @classmethod
    def from_safetensors(cls, ctx: Context, path: str, cfg: Optional[Qwen3Config] = None,
                         max_positions: Optional[int] = None) -> "Qwen3ForCausalLM":
        """A HF Qwen3 checkpoint (a directory with config.json and
        model.safetensors, or the .safetensors file plus cfg): BF16/F32
        weights quantized to Q8_0 on the device (ModelWeights::from_safetensors,
        src/loader.rs:68-188, then Qwen3ForCausalLM::load, src/model.rs:273-302)."""
        from . import checkpoint as ck
        st_path = path
        if os.path.isdir(path):
            st_path = os.path.join(path, "model.safetensors")
            if cfg is None:
                cfg = ck.qwen3_config_from_json(os.path.join(path, "config.json"), max_positions)
        if cfg is None:
            raise ModelError("a config is needed with a bare .safetensors file")
        f = ck.SafeTensorsFile(st_path)
        try:
            names = ck.hf_tensor_names(cfg)
            tens, dts, shapes = [], [], []
            for n in names:
                t = f.get(n)
                if t is None:
                    raise ModelError(f"Missing {n}")
                tens.append(t.data)
                dts.append(DTYPE_BF16 if t.dtype == "BF16" else DTYPE_F32)
                shapes.append(t.shape)
            ck.check_shapes(cfg, shapes, names)
            return cls.load_typed(ctx, cfg, tens, dts)
        finally:
            f.close()

    @classmethod
    def from_gguf(cls, ctx: Context, path: str, max_positions: Optional[int] = None) -> "Qwen3ForCausalLM":
        """A GGUF Q8_0 Qwen3 file (llama.cpp tensor names; F32/BF16 norms,
        Q8_0 or BF16/F32 matrices)."""
        from . import checkpoint as ck
        g = ck.GgufFile(path)
        try:
            cfg = ck.qwen3_config_from_gguf(g, max_positions)
            names = ck.gguf_tensor_names(cfg)
            tens, dts, shapes = [], [], []
            for n in names:
                t = g.tensors.get(n)
                if t is None:
                    raise ModelError(f"Missing {n}")
                if t.ggml_type == ck.GGML_Q8_0:
                    dts.append(DTYPE_Q8_0)
                elif t.ggml_type == ck.GGML_F32:
                    dts.append(DTYPE_F32)
                elif t.ggml_type == ck.GGML_BF16:
                    dts.append(DTYPE_BF16)
                else:
                    raise DTypeMismatch(f"{n}: ggml type {t.ggml_type} (expected Q8_0, F32 or BF16)")
                tens.append(t.data)
                shapes.append(t.shape)
            ck.check_shapes(cfg, shapes, names)
            return cls.load_typed(ctx, cfg, tens, dts)
        finally:
            g.close()

    def save_gguf(self, path: str) -> None:
        """The model's weights as a GGUF v3 file (Q8_0 matrices, F32 norms)."""
        from . import checkpoint as ck
        names = ck.gguf_tensor_names(self.cfg)
        tens = []
        for i, n in enumerate(names):
            kind, shape = self.cfg.tensor_shape(i)
            data = self.export_tensor(i)
            tens.append(ck.GgufTensor(n, ck.GGML_Q8_0 if kind == "q8" else ck.GGML_F32, tuple(shape), data))
        ck.write_gguf(path, ck.qwen3_gguf_metadata(self.cfg), tens)

    def export_tensor(self, idx: int) -> np.ndarray:
        nb = C.c_size_t()
        _check(lib().lq8_model_tensor_bytes(C.byref(self._c), idx, C.byref(nb)))
        kind, _ = self.cfg.tensor_shape(idx)
        out = np.empty(nb.value // 4 if kind == "f32" else nb.value, dtype=np.float32 if kind == "f32" else np.uint8)
        _check(lib().lq8_model_export_tensor(self.handle, idx, _ptr(out)))
        return out

    def export_all(self):
        return [self.export_tensor(i) for i in range(self.cfg.tensor_count())]

    def clear_kv_cache(self) -> None:
        _check(lib().lq8_model_clear_kv_cache(self.handle))

    def forward(self, input_ids: Sequence[int], offset: int) -> np.ndarray:
        ids = np.ascontiguousarray(input_ids, dtype=np.uint32)
        logits = np.empty(self.cfg.vocab_size, dtype=np.float32)
        _check(lib().lq8_model_forward(self.handle, _ptr(ids), ids.size, offset, _ptr(logits)))
        return logits

    def forward_with_intermediates(self, input_ids: Sequence[int], offset: int):
        """(hidden [layers+1, n, hidden], final_norm [n, hidden], logits [vocab])."""
        ids = np.ascontiguousarray(input_ids, dtype=np.uint32)
        n, H = ids.size, self.cfg.hidden_size
        hidden = np.empty((self.cfg.num_hidden_layers + 1, n, H), dtype=np.float32)
        fin = np.empty((n, H), dtype=np.float32)
        logits = np.empty(self.cfg.vocab_size, dtype=np.float32)
        _check(lib().lq8_model_forward_with_intermediates(self.handle, _ptr(ids), n, offset, _ptr(hidden), _ptr(fin),
                                                          _ptr(logits)))
        return hidden, fin, logits

    def generate_greedy(self, prompt: Sequence[int], max_new_tokens: int, feed_first: bool = False):
        """generate() with greedy sampling.  feed_first: every decode step
        forwards the first generated token, as the reference's loop does as
        written (src/generate.rs:632-650); otherwise the token generated last."""
        ids = np.ascontiguousarray(prompt, dtype=np.uint32)
        out = np.empty(max_new_tokens, dtype=np.uint32)
        st = GenStatsC()
        if feed_first:
            n = C.c_size_t(0)
            sc = SamplingC(0.0, 0, 1.0, 1.0, 0)
            _check(lib().lq8_generate_ex(self.handle, _ptr(ids), ids.size, max_new_tokens, C.byref(sc), None, 0,
                                         GEN_FEED_FIRST_TOKEN, _ptr(out), C.byref(n), C.byref(st)))
        else:
            _check(lib().lq8_generate_greedy(self.handle, _ptr(ids), ids.size, max_new_tokens, _ptr(out),
                                             C.byref(st)))
        return out, {"prefill_ms": st.prefill_ms, "decode_ms": st.decode_ms,
                     "decode_tokens_per_s": st.decode_tokens_per_s, "used_graph": bool(st.used_graph),
                     "used_persistent": bool(st.used_persistent)}

    def persist_picks(self, back: int = 0):
        """(values f32 [P], indices uint32 [P]): each of the P workgroups'
        greedy pick of the last persistent decode step (back 0) or the step
        before (back 1) -- its largest logit over its lm_head rows (16-row
        tiles t with (t // 8) % P == w), last index on ties
        (lq8_model_persist_picks)."""
        cap = 65536
        v = np.empty(cap, dtype=np.float32)
        i = np.empty(cap, dtype=np.uint32)
        n = C.c_size_t(0)
        _check(lib().lq8_model_persist_picks(self.handle, back, _ptr(v), _ptr(i), cap, C.byref(n)))
        return v[:n.value].copy(), i[:n.value].copy()

    def generate(self, prompt: Sequence[int], config: "GenerationConfig", seed: int = 0,
                 eos_token_ids: Sequence[int] = (), feed_first: bool = False):
        """generate() (src/generate.rs:611-664) with the configuration's
        sampling: up to config.max_new_tokens tokens, ending at the first one
        in eos_token_ids (kept); the loop stays on the device.  feed_first:
        the reference's loop as written (see generate_greedy)."""
        ids = np.ascontiguousarray(prompt, dtype=np.uint32)
        eos = np.ascontiguousarray(list(eos_token_ids), dtype=np.uint32)
        out = np.empty(config.max_new_tokens, dtype=np.uint32)
        n = C.c_size_t(0)
        st = GenStatsC()
        sc = config.sampling(seed)
        _check(lib().lq8_generate_ex(self.handle, _ptr(ids), ids.size, config.max_new_tokens, C.byref(sc),
                                     _ptr(eos) if eos.size else None, eos.size,
                                     GEN_FEED_FIRST_TOKEN if feed_first else 0, _ptr(out), C.byref(n),
                                     C.byref(st)))
        return out[:n.value].copy(), {"prefill_ms": st.prefill_ms, "decode_ms": st.decode_ms,
                                      "decode_tokens_per_s": st.decode_tokens_per_s, "used_graph": bool(st.used_graph),
                                      "used_persistent": bool(st.used_persistent)}

    def free(self) -> None:
        if self.handle:
            _check(lib().lq8_model_free(self.handle))
            self.handle = None


# ---- sampling --------------------------------------------------------------------

@dataclass
class GenerationConfig:
    """GenerationConfig (src/generate.rs:40-128): the defaults are greedy;
    ``new`` enforces the reference's ranges (InvalidArgument otherwise).  The
    sampling rule itself is the library's (include/lq8.h, lq8_sampling): the
    reference's samplers are argmax stubs."""

    max_new_tokens: int = 100
    temperature: float = 0.0
    top_k: int = 0
    top_p: float = 1.0
    repetition_penalty: float = 1.0

    @classmethod
    def new(cls, max_new_tokens: int, temperature: float, top_k: int, top_p: float,
            repetition_penalty: float) -> "GenerationConfig":
        if temperature < 0.0:
            raise InvalidArgument(f"temperature must be >= 0.0, got {temperature}", 0)
        if not 0.0 <= top_p <= 1.0:
            raise InvalidArgument(f"top_p must be in [0.0, 1.0], got {top_p}", 0)
        if repetition_penalty < 1.0:
            raise InvalidArgument(f"repetition_penalty must be >= 1.0, got {repetition_penalty}", 0)
        return cls(max_new_tokens, temperature, top_k, top_p, repetition_penalty)

    def sampling(self, seed: int) -> SamplingC:
        return SamplingC(self.temperature, self.top_k, self.top_p, self.repetition_penalty, seed & (2**64 - 1))


def sample_device(ctx: Context, logits: "DeviceBuffer", vocab: int, config: GenerationConfig, seed: int = 0,
                  step: int = 0, counts: Optional["DeviceBuffer"] = None) -> int:
    """sample_with_config (src/generate.rs:670-693) on device logits with the
    library's sampling rule; counts: device uint32 [vocab] of the tokens
    generated so far (repetition penalty)."""
    tok = DeviceBuffer(ctx, 4)
    try:
        sc = config.sampling(seed)
        _check(lib().lq8_sample_device(ctx.handle, logits.ptr, vocab, counts.ptr if counts is not None else None,
                                       C.byref(sc), step, tok.ptr))
        return int(tok.download(np.uint32, 1)[0])
    finally:
        tok.free()


# ---- Qwen3-MoE decoder layers --------------------------------------------------

@dataclass
class MoeConfig:
    """Qwen3-MoE decoder layer dimensions (Qwen3-30B-A3B defaults)."""

    hidden_size: int = 2048
    num_heads: int = 32
    num_kv_heads: int = 4
    head_dim: int = 128
    num_experts: int = 128
    top_k: int = 8
    expert_intermediate_size: int = 768
    max_positions: int = 256
    max_batch: int = 32
    num_layers: int = 1
    rms_norm_eps: float = 1e-6
    rope_theta: float = 1e6

    def c(self) -> MoeConfigC:
        return MoeConfigC(self.hidden_size, self.num_heads, self.num_kv_heads, self.head_dim, self.num_experts,
                          self.top_k, self.expert_intermediate_size, self.max_positions, self.max_batch,
                          self.num_layers, self.rms_norm_eps, self.rope_theta)

    def per_layer(self) -> int:
        return 8 + 3 * self.num_experts

    def tensor_count(self) -> int:
        return self.per_layer() * self.num_layers

    def tensor_shape(self, idx: int):
        """(kind, shape) of tensor ``idx`` in the table order of include/lq8.h."""
        H, I, hd, E = self.hidden_size, self.expert_intermediate_size, self.head_dim, self.num_experts
        QD, KD = self.num_heads * hd, self.num_kv_heads * hd
        k = idx % self.per_layer()
        if k < 8:
            return [("f32", (H,)), ("f32", (H,)), ("f32", (hd,)), ("f32", (hd,)), ("q8", (QD, H)), ("q8", (KD, H)),
                    ("q8", (KD, H)), ("q8", (H, QD))][k]
        return ("q8", (I, H)) if k - 8 < 2 * E else ("q8", (H, I))


def qwen3_30b_a3b_layers(num_layers: int = 1, max_positions: int = 256, max_batch: int = 32) -> MoeConfig:
    return MoeConfig(num_layers=num_layers, max_positions=max_positions, max_batch=max_batch)


class Qwen3MoeLayers:
    """A stack of Qwen3-MoE decoder layers decoding T independent sequences
    per call (sequence t owns KV cache slot t and writes position pos[t])."""

    def __init__(self, ctx: Context, cfg: MoeConfig, handle: C.c_void_p):
        self.ctx, self.cfg, self.handle = ctx, cfg, handle
        self._c = cfg.c()

    @classmethod
    def load(cls, ctx: Context, cfg: MoeConfig, tensors: Sequence[np.ndarray]) -> "Qwen3MoeLayers":
        if len(tensors) != cfg.tensor_count():
            raise ModelError(f"expected {cfg.tensor_count()} tensors, got {len(tensors)}")
        keep = [np.ascontiguousarray(t) for t in tensors]
        arr = (C.c_void_p * len(keep))(*[t.ctypes.data for t in keep])
        h = C.c_void_p()
        c = cfg.c()
        _check(lib().lq8_moe_create(ctx.handle, C.byref(c), arr, C.byref(h)))
        return cls(ctx, cfg, h)

    @classmethod
    def random(cls, ctx: Context, cfg: MoeConfig, seed: int, std: float = 0.02) -> "Qwen3MoeLayers":
        h = C.c_void_p()
        c = cfg.c()
        _check(lib().lq8_moe_create_random(ctx.handle, C.byref(c), seed, std, C.byref(h)))
        return cls(ctx, cfg, h)

    def export_tensor(self, idx: int) -> np.ndarray:
        nb = C.c_size_t()
        _check(lib().lq8_moe_tensor_bytes(C.byref(self._c), idx, C.byref(nb)))
        kind, _ = self.cfg.tensor_shape(idx)
        out = np.empty(nb.value // 4 if kind == "f32" else nb.value, dtype=np.float32 if kind == "f32" else np.uint8)
        _check(lib().lq8_moe_export_tensor(self.handle, idx, _ptr(out)))
        return out

    def export_all(self):
        return [self.export_tensor(i) for i in range(self.cfg.tensor_count())]

    def weight_bytes(self) -> int:
        nb = C.c_size_t()
        _check(lib().lq8_moe_weight_bytes(self.handle, C.byref(nb)))
        return nb.value

    def forward(self, hidden: np.ndarray, scores: np.ndarray, pos: Sequence[int]) -> np.ndarray:
        """hidden [T, H], scores [num_layers, T, E], pos [T] -> hidden after the last layer."""
        h = np.array(hidden, dtype=np.float32, copy=True, order="C")
        sc = np.ascontiguousarray(scores, dtype=np.float32)
        p = np.ascontiguousarray(pos, dtype=np.int32)
        _check(lib().lq8_moe_forward(self.handle, _ptr(h), _ptr(sc), _ptr(p), p.size))
        return h

    def forward_device(self, hidden: DeviceBuffer, scores: DeviceBuffer, pos: DeviceBuffer, T: int) -> None:
        _check(lib().lq8_moe_forward_device(self.handle, hidden.ptr, scores.ptr, pos.ptr, T))

    def routing(self, T: int):
        """(experts [layers, T, k], weights [layers, T, k]) of the last forward."""
        L, K = self.cfg.num_layers, self.cfg.top_k
        ids = np.empty((L, T, K), dtype=np.uint32)
        w = np.empty((L, T, K), dtype=np.float32)
        _check(lib().lq8_moe_routing(self.handle, _ptr(ids), _ptr(w)))
        return ids, w

    def clear_kv_cache(self) -> None:
        _check(lib().lq8_moe_clear_kv_cache(self.handle))

    def free(self) -> None:
        if self.handle:
            _check(lib().lq8_moe_free(self.handle))
            self.handle = None


def bench_grid_sync(ctx: "Context", kind: int, nwg: int, rounds: int):
    """(us per grid-wide synchronisation, values read wrong, waits given up)
    of lq8_bench_grid_sync."""
    us, bad, gave = C.c_float(0), C.c_uint32(0), C.c_uint32(0)
    _check(lib().lq8_bench_grid_sync(ctx.handle, kind, nwg, rounds, C.byref(us), C.byref(bad), C.byref(gave)))
    return float(us.value), int(bad.value), int(gave.value)


def persist_plan(cfg: "Qwen3Config", num_workgroups: int) -> dict:
    """lq8_persist_plan: whether greedy decode of this configuration runs as
    the persistent kernel on num_workgroups workgroups, and its plan (input
    chunks of the o and down projections, LDS map in floats).  No device."""
    info = PersistInfoC()
    c = cfg.c()
    _check(lib().lq8_persist_plan(C.byref(c), num_workgroups, C.byref(info)))
    out = {n: int(getattr(info, n)) for n, _ in PersistInfoC._fields_}
    out["supported"] = bool(out["supported"])
    return out


FLOOR_EMPTY, FLOOR_STREAM, FLOOR_CHASE, FLOOR_STREAM_CHUNKS, FLOOR_EMPTY_GRAPH = 0, 1, 2, 3, 4


def bench_floor(ctx: "Context", kind: int, nwg: int = 1, nbytes: int = 0, reps: int = 1) -> float:
    """lq8_bench_floors: us per empty-kernel launch (FLOOR_EMPTY), GB/s of a
    read-only stream (FLOOR_STREAM), or ns per dependent HBM load
    (FLOOR_CHASE)."""
    v = C.c_double(0.0)
    _check(lib().lq8_bench_floors(ctx.handle, kind, nwg, nbytes, reps, C.byref(v)))
    return float(v.value)


PTRACE_WG, PTRACE_LAYERS, PTRACE_POINTS = 512, 64, 25
PTRACE_MARKS = ("P1_START", "P1_NORMED", "P2_START", "P2_QKV_IN", "P2_SCORES", "P2_PARTIALS", "P3_START",
                "P3_STAGED", "P4_START", "P4_STAGED", "P5_START", "P5_STAGED", "P5_DONE", "P6_START", "P6_NORMED",
                "P6_DONE", "P2_COMBINED", "P2_COMB_FETCHED", "P2_COMB_COEF", "P1_GATHERED", "P1_DOT", "P2_ROPED",
                "P3_COMBINED", "P4_NORMED", "P4_DOT")
# the marks of a decoder layer, in phase order, and of the lm_head phase (layer 0's row)
PTRACE_LAYER_MARKS = ("P1_START", "P1_GATHERED", "P1_NORMED", "P1_DOT", "P2_START", "P2_QKV_IN", "P2_ROPED",
                      "P2_SCORES", "P2_PARTIALS", "P2_COMB_FETCHED", "P2_COMB_COEF", "P2_COMBINED",
                      "P3_START", "P3_STAGED", "P3_COMBINED", "P4_START", "P4_STAGED", "P4_NORMED", "P4_DOT",
                      "P5_START", "P5_STAGED", "P5_DONE")
PTRACE_HEAD_MARKS = ("P6_START", "P6_NORMED", "P6_DONE")


def persist_trace(ctx: "Context") -> np.ndarray:
    """The persistent decode's phase marks (lq8_persist_trace) as uint64
    [PTRACE_WG][PTRACE_LAYERS][PTRACE_POINTS], 100 MHz ticks (0: not passed)."""
    out = np.zeros(PTRACE_WG * PTRACE_LAYERS * PTRACE_POINTS, dtype=np.uint64)
    _check(lib().lq8_persist_trace(ctx.handle, _ptr(out), out.size))
    return out.reshape(PTRACE_WG, PTRACE_LAYERS, PTRACE_POINTS)


def gemv_grouped_device(ctx: Context, problems) -> None:
    """problems: iterable of (Q8Weight, DeviceBuffer x, DeviceBuffer y)."""
    arr = (GemvProblemC * len(problems))(*[GemvProblemC(w.handle, x.ptr, y.ptr) for (w, x, y) in problems])
    _check(lib().lq8_gemv_grouped_device(ctx.handle, arr, len(problems)))


def bench_gemv(ctx: Context, problems, mode: int, reps: int) -> float:
    """Device ms for ``reps`` passes over (Q8Weight, x, y) problems (see lq8_bench_gemv)."""
    arr = (GemvProblemC * len(problems))(*[GemvProblemC(w.handle, x.ptr, y.ptr) for (w, x, y) in problems])
    ms = C.c_float(0.0)
    _check(lib().lq8_bench_gemv(ctx.handle, arr, len(problems), mode, reps, C.byref(ms)))
    return ms.value
