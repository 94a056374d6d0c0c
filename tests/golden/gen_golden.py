"""Writes tests/golden/q8_0_golden.npz from the C oracle, after checking the
oracle against the independent numpy restatement (tests/golden/numpy_q8.py).

The reference repository ships no Q8_0 vectors (its Q8_0 path is a plan), so
these fixtures are the build's own: they freeze the oracle's outputs on
seeded inputs and edge blocks so that any change to the oracle shows up.
Run from the repository root:  python tests/golden/gen_golden.py
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path[:0] = [HERE, os.path.join(ROOT, "oracle"), os.path.join(ROOT, "qwen-omni-inference-rs_amd")]

import numpy_q8  # noqa: E402
import oracle  # noqa: E402


def edge_blocks():
    rows = [np.zeros(32, np.float32)]
    t = np.zeros(32, np.float32); t[0] = 127.0; t[1:8] = [0.5, -0.5, 1.5, -1.5, 2.5, -2.5, 126.5]; rows.append(t)
    rows.append(np.full(32, -3.0, np.float32))
    rows.append(np.linspace(-1e-6, 1e-6, 32).astype(np.float32))
    rows.append(np.linspace(-1e-38, 2e-38, 32).astype(np.float32))
    t = np.ones(32, np.float32) * 7e6; t[3] = -9e6; rows.append(t)
    t = np.random.default_rng(5).standard_normal(32).astype(np.float32); t[7] = np.nan; rows.append(t)
    t = np.random.default_rng(6).standard_normal(32).astype(np.float32); t[9] = np.inf; rows.append(t)
    return np.concatenate(rows)


def main():
    rng = np.random.default_rng(20261201)
    qx = np.concatenate([edge_blocks(), rng.standard_normal(32 * 64).astype(np.float32),
                         (rng.standard_normal(32 * 64) * 0.02).astype(np.float32)])
    qb = oracle.quantize_q8_0(qx)
    assert np.array_equal(qb, numpy_q8.quantize_q8_0(qx)), "oracle quantizer disagrees with numpy"

    n, k = 96, 256
    w = (rng.standard_normal((n, k)) * 0.02).astype(np.float32)
    wb = oracle.quantize_q8_0(w)
    x = rng.standard_normal(k).astype(np.float32)
    y = oracle.gemv_q8_0(wb, n, k, x)
    ref = numpy_q8.gemv_f64(wb, n, k, x)
    assert np.max(np.abs(y - ref)) <= 1e-5 * np.max(np.abs(ref))
    exact = numpy_q8.gemv_tree_rows(wb, n, k, x, range(n))
    assert np.array_equal(y.view(np.uint32), exact.view(np.uint32)), "oracle GEMV disagrees with its exact restatement"

    m = 5
    xm = rng.standard_normal((m, k)).astype(np.float32)
    ym = oracle.gemm_q8_0(wb, n, k, xm)

    import lq8
    cfg = lq8.Qwen3Config(vocab_size=512, hidden_size=128, intermediate_size=256, num_hidden_layers=2,
                          num_attention_heads=2, num_key_value_heads=1, head_dim=128, max_position_embeddings=64)
    tensors = oracle.random_q8_tensors(cfg, seed=77)
    model = oracle.Model(cfg, tensors)
    prompt = np.arange(1, 9, dtype=np.uint32) * 37 % cfg.vocab_size
    logits0 = model.forward(prompt, 0)
    toks, _ = model.generate_greedy(prompt, 12)
    model.close()

    np.savez_compressed(os.path.join(HERE, "q8_0_golden.npz"), quant_x=qx, quant_blocks=qb, gemv_w=wb,
                        gemv_x=x, gemv_y=y, gemm_x=xm, gemm_y=ym, tiny_prompt=prompt, tiny_logits0=logits0,
                        tiny_tokens=toks)
    print("wrote", os.path.join(HERE, "q8_0_golden.npz"))


if __name__ == "__main__":
    main()
