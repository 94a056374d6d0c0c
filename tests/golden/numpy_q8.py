"""Independent numpy restatement of the Q8_0 quantizer and reductions, used to
cross-check the C oracle (and to generate the golden fixtures).

Q8_0 (GGUF block_q8_0): amax = max|x| ignoring NaN; d = f32(amax / 127);
id = f32(1 / d) or 0; q = round-half-away-from-zero(f32(x * id)) saturated to
int8 with NaN -> 0; the stored scale is float16(d) (round to nearest even).
"""
import numpy as np


def quantize_q8_0(x):
    x = np.asarray(x, np.float32).reshape(-1, 32)
    with np.errstate(invalid="ignore", over="ignore", divide="ignore"):
        amax = np.nanmax(np.where(np.isnan(x), np.float32(0), np.abs(x)), axis=1).astype(np.float32)
        d = (amax / np.float32(127)).astype(np.float32)
        inv = np.where(d != 0, np.float32(1) / np.where(d != 0, d, np.float32(1)), np.float32(0)).astype(np.float32)
        v = (x * inv[:, None]).astype(np.float32).astype(np.float64)
        r = np.sign(v) * np.floor(np.abs(v) + 0.5)                  # half away from zero
        r = np.where(np.isnan(r), 0.0, np.clip(r, -128, 127))
    q = r.astype(np.int8)
    d16 = d.astype(np.float16)                                      # numpy casts round to nearest even
    out = np.empty((x.shape[0], 34), np.uint8)
    out[:, :2] = d16.view(np.uint8).reshape(-1, 2)
    out[:, 2:] = q.view(np.uint8)
    return out.reshape(-1)


def dequantize_q8_0(blocks, n):
    b = np.asarray(blocks, np.uint8).reshape(-1, 34)
    d = b[:, :2].copy().view(np.float16).astype(np.float32)
    q = b[:, 2:].view(np.int8).astype(np.float32)
    return (d * q).reshape(-1)[:n]


def gemv_f64(blocks, n_out, k_in, x):
    """Exact-ish reference: dequantized W (exact in f32) times x, in float64."""
    W = dequantize_q8_0(blocks, n_out * k_in).reshape(n_out, k_in).astype(np.float64)
    return W @ np.asarray(x, np.float64)


def bf16_round(x):
    """src/bf16.rs:112-131 restated on uint32 bit patterns."""
    b = np.asarray(x, np.float32).view(np.uint32).astype(np.uint64)
    r = (b + 0x7FFF + ((b >> 16) & 1)) & 0xFFFFFFFF
    return ((r >> 16) << 16).astype(np.uint32).view(np.float32)
