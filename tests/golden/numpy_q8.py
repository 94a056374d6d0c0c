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


# ---- exact restatement of the GEMV canonical order (small shapes only) ----
from fractions import Fraction  # noqa: E402


def round_f32(q):
    """Rational -> float32, round to nearest, ties to even (finite results)."""
    if q == 0:
        return np.float32(0.0)
    f = np.float32(float(q))
    best = None
    for c in (np.nextafter(f, np.float32(-np.inf), dtype=np.float32), f,
              np.nextafter(f, np.float32(np.inf), dtype=np.float32)):
        if not np.isfinite(c):
            continue
        key = (abs(Fraction(float(c)) - q), int(np.array(c, np.float32).view(np.uint32)) & 1)
        if best is None or key < best[0]:
            best = (key, c)
    return np.float32(best[1])


def fmaf_exact(a, b, c):
    """fmaf(a, b, c) for finite float32 operands: one rounding of the exact value.
    An exact zero result is +0 (round to nearest; never both addends -0 here)."""
    return round_f32(Fraction(float(a)) * Fraction(float(b)) + Fraction(float(c)))


def gemv_tree_rows(blocks, n_out, k_in, x, rows):
    """GEMV canonical order for the given rows: per block, h0 = fmaf chain over
    codes 0..15, h1 over codes 16..31 (from +0), v_b = (h0 + h1) * d_b (float32
    ops); then the pairwise tree v[i] += v[i + s], s = 1, 2, 4, ..., i + s < nb."""
    nb = k_in // 32
    b = np.asarray(blocks, np.uint8).reshape(n_out, nb, 34)
    x = np.asarray(x, np.float32)
    out = []
    for r in rows:
        v = []
        for j in range(nb):
            d = b[r, j, :2].copy().view(np.float16).astype(np.float32)[0]
            q = b[r, j, 2:].view(np.int8)
            h0 = np.float32(0.0)
            for t in range(16):
                h0 = fmaf_exact(np.float32(q[t]), x[32 * j + t], h0)
            h1 = np.float32(0.0)
            for t in range(16, 32):
                h1 = fmaf_exact(np.float32(q[t]), x[32 * j + t], h1)
            v.append(np.float32(np.float32(h0 + h1) * d))
        s = 1
        while s < nb:
            for i in range(0, nb - s, 2 * s):
                v[i] = np.float32(v[i] + v[i + s])
            s *= 2
        out.append(v[0])
    return np.array(out, np.float32)
