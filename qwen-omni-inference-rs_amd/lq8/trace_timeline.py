"""Phase timeline of the persistent greedy decode kernel.

Runs Qwen3-0.6B-shaped (or, with --shape 1.7b, Qwen3-1.7B-shaped) greedy
decode (random Q8_0 weights, a 128-token prompt) through the persistent kernel of the trace build (``make trace`` ->
liblq8_trace.so) and prints, per phase mark, when the workgroups pass it
relative to the moment the layer's input is complete (the last workgroup's
layer start, i.e. the last down tile of the previous layer).  Medians over
the layers 4 .. L-1 of one decode step.

    python -m lq8.trace_timeline [--layers 28] [--prompt 128] [--shape 0.6b|1.7b]
"""
import argparse
import contextlib
import os
import sys

import numpy as np

import lq8

TICK_US = 0.01  # s_memrealtime runs at 100 MHz


def timeline(tr: np.ndarray, n_layers: int, first: int = 4):
    """Rows (mark name, workgroups passing, [min, median, max] in us) and the
    median layer period, from a trace of shape [WG][LAYERS][POINTS]."""
    tr = tr.astype(np.int64)
    L = min(n_layers, lq8.PTRACE_LAYERS)
    rows = []
    refs = []
    for l in range(L):
        st = tr[:, l, lq8.PTRACE_MARKS.index("P1_START")]
        refs.append(st[st != 0].max() if (st != 0).any() else 0)
    refs = np.array(refs)
    for name in lq8.PTRACE_LAYER_MARKS:
        m = lq8.PTRACE_MARKS.index(name)
        per = []
        n = 0
        for l in range(first, L):
            col = tr[:, l, m]
            v = col[col != 0] - refs[l]
            if v.size == 0:
                continue
            n = max(n, v.size)
            per.append((v.min(), np.median(v), v.max()))
        if per:
            rows.append((name, n, np.median(np.array(per), axis=0) * TICK_US))
    period = np.median(np.diff(refs[first:])) * TICK_US if L > first + 1 else float("nan")
    p6 = tr[:, 0, [lq8.PTRACE_MARKS.index(n) for n in lq8.PTRACE_HEAD_MARKS]]
    p6_rows = []
    if (p6[:, 0] != 0).any():
        base = p6[p6[:, 0] != 0, 0].min()
        for k, name in enumerate(lq8.PTRACE_HEAD_MARKS):
            v = p6[p6[:, k] != 0, k] - base
            p6_rows.append((name, v.size, np.array([v.min(), np.median(v), v.max()]) * TICK_US))
    return rows, period, p6_rows


@contextlib.contextmanager
def trace_library():
    """Inside the block lq8's calls go to the trace build (liblq8_trace.so,
    loaded beside liblq8.so); objects made inside belong to it."""
    saved = lq8._lib, lq8.LIB_PATH
    lq8._lib = None
    lq8.LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(lq8.__file__)), "liblq8_trace.so")
    try:
        lq8.lib()
        yield
    finally:
        lq8._lib, lq8.LIB_PATH = saved


def collect(layers: int, prompt: int, new: int, shape: str = "0.6b"):
    """(generate statistics, trace) of Qwen3-0.6B- or 1.7B-shaped greedy decode with
    ``layers`` layers through the persistent kernel of the trace build; the
    second of two runs is the one traced."""
    prev = os.environ.get("LQ8_PERSIST")
    os.environ["LQ8_PERSIST"] = "1"
    try:
        with trace_library():
            cfg = (lq8.qwen3_1_7b if shape == "1.7b" else lq8.qwen3_0_6b)(max_positions=512)
            cfg.num_hidden_layers = layers
            with lq8.Context(0) as ctx:
                model = lq8.Qwen3ForCausalLM.random(ctx, cfg, seed=2026)
                ids = np.random.default_rng(2026).integers(0, cfg.vocab_size, prompt).astype(np.uint32)
                stats = None
                for _ in range(2):
                    _, stats = model.generate_greedy(ids, new)
                tr = lq8.persist_trace(ctx)
                model.free()
    finally:
        if prev is None:
            os.environ.pop("LQ8_PERSIST", None)
        else:
            os.environ["LQ8_PERSIST"] = prev
    return stats, tr


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--layers", type=int, default=28)
    ap.add_argument("--prompt", type=int, default=128)
    ap.add_argument("--new", type=int, default=9, help="generated tokens (the 4th decode step is traced)")
    ap.add_argument("--shape", choices=("0.6b", "1.7b"), default="0.6b", help="the model's layer shapes")
    args = ap.parse_args(argv)
    stats, tr = collect(args.layers, args.prompt, args.new, args.shape)
    if not stats["used_persistent"]:
        print("the persistent kernel did not run", file=sys.stderr)
        return 1
    rows, period, p6 = timeline(tr, args.layers)
    print(f"decode {stats['decode_tokens_per_s']:.1f} tok/s ({1e6 / stats['decode_tokens_per_s']:.0f} us/token), "
          f"layer period {period:.2f} us")
    print("mark            WGs   min(us)  median    max   (from the layer input's completion)")
    for name, n, (a, b, c) in rows:
        print(f"{name:14s} {n:4d} {a:8.2f} {b:8.2f} {c:8.2f}")
    print("lm_head (from its first workgroup's start)")
    for name, n, (a, b, c) in p6:
        print(f"{name:14s} {n:4d} {a:8.2f} {b:8.2f} {c:8.2f}")
    return 0


if __name__ == "__main__":
    sys.exit(main())
