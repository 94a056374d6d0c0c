"""Benchmark of the Q8_0 hot path on one MI355X.

Workload (one "step"): every linear layer of one Qwen3-0.6B decode token at
batch 1 as a Q8_0 GEMV -- 28 layers x {q 2048x1024, k 1024x1024, v 1024x1024,
o 1024x2048, gate 3072x1024, up 3072x1024, down 1024x3072} plus the lm_head
151936x1024 -- 197 GEMVs over distinct resident weights (633 MB, more than
twice the 256 MB Infinity Cache, so every step streams from HBM), each with
its own seeded N(0, 1) input.  Weights N(0, 0.02) from a seeded device
generator, quantized to Q8_0 on the device.

The headline value runs the step as one grouped launch (the 197 GEMVs are
independent, so one kernel streams them back to back); the same step with one
launch per GEMV replayed from a HIP graph, the lm_head alone, the single
3072x1024 GEMV, the M = 512 W8A8 MFMA GEMM, and batch-1 decode of the
random-init Q8_0 Qwen3-0.6B (128-token prompt, 128 new tokens; greedy, and
sampled with temperature 0.8, top-k 50, top-p 0.95, repetition penalty 1.1)
are reported beside it (greedy decode on its default path, the persistent
kernel, and on the replayed graph; the same greedy decode at Qwen3-1.7B and
Qwen3-4B shapes, random weights, on the default path -- the replayed graph
above hidden 1024 --, the graph, and the persistent kernel where the shape
fits it; Qwen3-0.6B again with its own max_positions, 40960), and so is the
host-pointer
Linear::forward per call at the seven layer shapes.  The CPU
baseline is a C restatement of the reference's own CPU Linear::forward (BF16
weight, per-call transpose, BF16 -> F32 copy, naive matmul_2d) timed on one
pinned host core over a bounded sample of the same workload; the CPU oracle's
Q8_0 GEMV is reported beside it.

Prints one JSON line on stdout; progress goes to stderr.
"""
import argparse
import json
import os
import re
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path[:0] = [os.path.join(ROOT, "qwen-omni-inference-rs_amd"), os.path.join(ROOT, "oracle")]

import lq8  # noqa: E402

HBM_PEAK_GBS = 8000.0
INT8_PEAK_TOPS = 5000.0
LAYER_SHAPES = [("q", 2048, 1024), ("k", 1024, 1024), ("v", 1024, 1024), ("o", 1024, 2048),
                ("gate", 3072, 1024), ("up", 3072, 1024), ("down", 1024, 3072)]
LM_HEAD = ("lm_head", 151936, 1024)
LAYERS = 28
CALIB_BYTES = 256 << 20
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "gemv_grouped_qwen3_decode_step_traffic.md")


def gemv_bytes(n, k):
    """Algorithmic bytes of one GEMV: Q8_0 weight (34 B per 32) + f32 x + f32 y."""
    return n * k * 34 // 32 + 4 * k + 4 * n


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def make_problems(ctx, seed):
    shapes = [s for _ in range(LAYERS) for s in LAYER_SHAPES] + [LM_HEAD]
    probs, bufs = [], []
    rng = np.random.default_rng(seed)
    for i, (_, n, k) in enumerate(shapes):
        w = lq8.Q8Weight.random(ctx, n, k, seed=seed, stream=i, std=0.02)
        x = lq8.DeviceBuffer.from_array(ctx, rng.standard_normal(k).astype(np.float32))
        y = lq8.DeviceBuffer(ctx, 4 * n)
        probs.append((w, x, y))
        bufs += [x, y]
    return shapes, probs, bufs


def measured_traffic():
    """HBM bytes per grouped launch from the committed rocprofv3 PMC summary
    (FETCH_SIZE + WRITE_SIZE, scaled by the same counters on a copy of known
    size), or None when the summary is absent."""
    try:
        with open(TRAFFIC_FILE) as f:
            m = re.search(r"^traffic_bytes_per_launch:\s*(\d+)", f.read(), re.M)
        return int(m.group(1)) if m else None
    except OSError:
        return None


def pinned_core():
    """One core this process may use (the lowest), for single-core baselines."""
    return min(os.sched_getaffinity(0))


def cpu_reference_linear(seconds_target=12.0):
    """The reference's CPU Linear::forward restated (oracle/ref_linear_bf16.c:
    BF16 weight, per-call transpose, BF16 -> F32, naive matmul_2d, one
    thread) over one decode layer's 7 linears at batch 1, pinned to one core,
    repeated for ~seconds_target.  value: the workload's algorithmic (Q8_0)
    bytes per second, so that it divides the GPU value directly."""
    import oracle

    rng = np.random.default_rng(5)
    mats = []
    for _, n, k in LAYER_SHAPES:
        w = (rng.standard_normal((n, k)).astype(np.float32) * 0.02).view(np.uint32)
        mats.append(((w >> 16).astype(np.uint16), rng.standard_normal((1, k)).astype(np.float32)))
    layer_bytes = sum(gemv_bytes(n, k) for _, n, k in LAYER_SHAPES)
    bf16_bytes = sum(2 * n * k for _, n, k in LAYER_SHAPES)
    aff = os.sched_getaffinity(0)
    core = pinned_core()
    os.sched_setaffinity(0, {core})
    try:
        oracle.ref_linear_forward_bf16(*mats[0])  # first touch
        passes, t0 = 0, time.perf_counter()
        while True:
            for w, x in mats:
                oracle.ref_linear_forward_bf16(w, x)
            passes += 1
            el = time.perf_counter() - t0
            if el >= seconds_target:
                break
    finally:
        os.sched_setaffinity(0, aff)
    layer_s = el / passes
    # a token: 28 such layers plus the 151936 x 1024 lm_head (its share scaled by weight count)
    lm_frac = LM_HEAD[1] * LM_HEAD[2] / sum(n * k for _, n, k in LAYER_SHAPES)
    token_s = layer_s * (LAYERS + lm_frac)
    return {"value": round(passes * layer_bytes / el / 1e9, 4), "unit": "GB/s", "cores": 1, "kind": "port",
            "sample": f"restatement of the reference's CPU Linear::forward (src/attention.rs:101-136, "
                      f"src/tensor.rs:439-467, 957-958, 2716-2753) on BF16 weights: {passes} passes over one "
                      f"Qwen3-0.6B decode layer's 7 linears at batch 1, {el:.1f} s on core {core} "
                      f"(value counts the workload's Q8_0 bytes, {layer_bytes} per pass)",
            "bf16_weight_gbs": round(passes * bf16_bytes / el / 1e9, 4),
            "layer_ms": round(layer_s * 1e3, 1), "token_s_extrapolated": round(token_s, 2)}


def cpu_baseline(seconds_target=12.0):
    """Oracle Q8_0 GEMV (1 thread) over one decode layer's 7 linears, repeated
    for ~seconds_target; reported as GB/s of algorithmic bytes."""
    import oracle

    oracle.set_threads(1)
    rng = np.random.default_rng(5)
    mats = []
    for _, n, k in LAYER_SHAPES:
        blocks = oracle.quantize_q8_0((rng.standard_normal((n, k)) * 0.02).astype(np.float32))
        mats.append((blocks, n, k, rng.standard_normal(k).astype(np.float32)))
    layer_bytes = sum(gemv_bytes(n, k) for _, n, k, _ in mats)
    aff = os.sched_getaffinity(0)
    core = pinned_core()
    os.sched_setaffinity(0, {core})
    try:
        passes, t0 = 0, time.perf_counter()
        while True:
            for blocks, n, k, x in mats:
                oracle.gemv_q8_0(blocks, n, k, x)
            passes += 1
            el = time.perf_counter() - t0
            if el >= seconds_target:
                break
    finally:
        os.sched_setaffinity(0, aff)
        oracle.set_threads(0)
    return {"value": round(passes * layer_bytes / el / 1e9, 3), "unit": "GB/s", "cores": 1, "kind": "port",
            "sample": f"the oracle's Q8_0 GEMV: {passes} passes over one Qwen3-0.6B decode layer's 7 Q8_0 GEMVs "
                      f"({layer_bytes} B each), {el:.1f} s on core {core}"}


def host_cpu():
    """Model name and logical cores available to this process."""
    name = None
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    name = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return {"model": name, "logical_cores": len(os.sched_getaffinity(0))}


def cpu_gemv_all_cores(seconds_target=4.0):
    """The oracle's GEMV with one OpenMP thread per available core (each output
    row still summed by one thread in the fixed order), labelled apart from
    the single-core baseline."""
    import oracle

    threads = len(os.sched_getaffinity(0))
    oracle.set_threads(threads)
    rng = np.random.default_rng(5)
    mats = []
    for _, n, k in LAYER_SHAPES:
        blocks = oracle.quantize_q8_0((rng.standard_normal((n, k)) * 0.02).astype(np.float32))
        mats.append((blocks, n, k, rng.standard_normal(k).astype(np.float32)))
    layer_bytes = sum(gemv_bytes(n, k) for _, n, k, _ in mats)
    passes, t0 = 0, time.perf_counter()
    while True:
        for blocks, n, k, x in mats:
            oracle.gemv_q8_0(blocks, n, k, x)
        passes += 1
        el = time.perf_counter() - t0
        if el >= seconds_target:
            break
    oracle.set_threads(0)
    return {"value": round(passes * layer_bytes / el / 1e9, 3), "unit": "GB/s", "cores": threads, "kind": "port",
            "sample": f"{passes} passes over one decode layer's 7 Q8_0 GEMVs, {el:.1f} s"}


def cpu_decode(cfg, tensors, prompt, steps=3):
    """Qwen3-0.6B batch-1 decode on the host: the oracle's forward (the
    reference's decoder numerics over Q8_0 weights), a few single-token steps
    on one core after a 128-token prefill run on all cores (not timed)."""
    import oracle

    ref = oracle.Model(cfg, tensors)
    try:
        oracle.set_threads(len(os.sched_getaffinity(0)))
        logits = ref.forward(prompt, 0)
        oracle.set_threads(1)
        tok, pos = int(np.argmax(logits)), prompt.size
        t0 = time.perf_counter()
        for _ in range(steps):
            logits = ref.forward([tok], pos)
            tok, pos = int(np.argmax(logits)), pos + 1
        el = time.perf_counter() - t0
    finally:
        oracle.set_threads(0)
        ref.close()
    return {"tokens_per_s": round(steps / el, 3), "cores": 1, "kind": "port",
            "sample": f"{steps} decode steps at positions 128..{127 + steps} on one core, {el:.2f} s"}


def rotating_gemv_us(ctx, n, k, copies):
    """Per-launch time of an n x k GEMV, graph-replayed over `copies` distinct
    weights (cold: the copies together exceed the Infinity Cache)."""
    ws = [lq8.Q8Weight.random(ctx, n, k, seed=11, stream=i) for i in range(copies)]
    x = lq8.DeviceBuffer.from_array(ctx, np.random.default_rng(1).standard_normal(k).astype(np.float32))
    y = lq8.DeviceBuffer(ctx, 4 * n)
    probs = [(w, x, y) for w in ws]
    lq8.bench_gemv(ctx, probs, mode=2, reps=2)
    us = lq8.bench_gemv(ctx, probs, mode=2, reps=10) * 1e3 / (10 * copies)
    for w in ws:
        w.free()
    x.free()
    y.free()
    return us


def linear_forward_host(ctx, calls=200):
    """Host-pointer Linear::forward (lq8_linear_forward: host x in, host y
    out, through the context's pinned staging) per call at batch 1, at the
    seven decoder-layer shapes: median wall time of `calls` calls each."""
    out = {}
    for name, n, k in LAYER_SHAPES:
        w = lq8.Q8Weight.random(ctx, n, k, seed=21, stream=n + k)
        lin = lq8.Linear.new(w)
        x = np.random.default_rng(n).standard_normal((1, k)).astype(np.float32)
        for _ in range(10):
            lin.forward(x)
        ts = []
        for _ in range(calls):
            t0 = time.perf_counter()
            lin.forward(x)
            ts.append(time.perf_counter() - t0)
        out[f"{name}_{n}x{k}_us"] = round(float(np.median(ts)) * 1e6, 1)
        w.free()
    out["layer_us"] = round(sum(v for v in out.values()), 1)
    return out


def decode_larger(ctx, cfg, label):
    """Greedy decode of a larger Qwen3 shape (random Q8_0 weights, 128-token
    prompt, 128 new tokens) on the default path, on the replayed graph and,
    where its shape is supported, on the persistent kernel: tok/s, medians of
    3; the tokens of all paths must agree."""
    model = lq8.Qwen3ForCausalLM.random(ctx, cfg, seed=2026)
    prompt = np.random.default_rng(2026).integers(0, cfg.vocab_size, 128).astype(np.uint32)

    def timed(persist):
        if persist is not None:
            os.environ["LQ8_PERSIST"] = persist
        try:
            model.generate_greedy(prompt, 8)
            return [model.generate_greedy(prompt, 128) for _ in range(3)]
        finally:
            os.environ.pop("LQ8_PERSIST", None)

    runs, gruns = timed(None), timed("0")
    pruns = timed("1")
    if not pruns[0][1]["used_persistent"]:  # a shape outside the kernel's limits
        pruns = []
    model.free()
    med = lambda rs: sorted(st["decode_tokens_per_s"] for _, st in rs)[1]
    tps, gtps = med(runs), med(gruns)
    st0 = runs[0][1]
    H, I, QD, KD = cfg.hidden_size, cfg.intermediate_size, cfg.num_attention_heads * 128, cfg.num_key_value_heads * 128
    wbytes = (cfg.num_hidden_layers * ((QD + 2 * KD) * H + H * QD + 3 * I * H) + cfg.vocab_size * H) * 34 // 32
    out = {"tokens_per_s": round(tps, 1), "weight_bytes_per_token": wbytes, "weight_gbs": round(wbytes * tps / 1e9, 1),
           "path": "persistent" if st0["used_persistent"] else ("graph" if st0["used_graph"] else "plain"),
           "graph_tokens_per_s": round(gtps, 1),
           "persistent_tokens_per_s": round(med(pruns), 1) if pruns else None,
           "tokens_agree": all(np.array_equal(t, runs[0][0]) for t, _ in runs + gruns + pruns),
           "config": {"hidden": cfg.hidden_size, "intermediate": cfg.intermediate_size,
                      "layers": cfg.num_hidden_layers, "heads": cfg.num_attention_heads,
                      "kv_heads": cfg.num_key_value_heads, "vocab": cfg.vocab_size}}
    log(f"decode {label}: {tps:.1f} tok/s ({out['path']}), graph {gtps:.1f} tok/s, persistent "
        f"{out['persistent_tokens_per_s']} tok/s, tokens agree: {out['tokens_agree']}")
    return out


def moe_stack(ctx, layers=48, reps=10):
    """Qwen3-30B-A3B-style MoE decoder stack (48 layers, ~31.8 GB of Q8_0
    weights resident), one decode step for T = 1 and T = 32 sequences at
    position 128, router scores N(0, 1).  Bytes per step = attention weights +
    the weights of every distinct routed expert of every layer."""
    cfg = lq8.MoeConfig(num_layers=layers, max_positions=256, max_batch=32)
    m = lq8.Qwen3MoeLayers.random(ctx, cfg, seed=5)
    H, E = cfg.hidden_size, cfg.num_experts
    q8 = lambda r, k: r * (k // 32) * 34
    attn_b = q8(cfg.num_heads * 128 + 2 * cfg.num_kv_heads * 128, H) + q8(H, cfg.num_heads * 128)
    exp_b = 2 * q8(cfg.expert_intermediate_size, H) + q8(H, cfg.expert_intermediate_size)
    out = {"weights_gb": round(m.weight_bytes() / 1e9, 2), "position": 128}
    for T in (1, 32):
        rng = np.random.default_rng(T)
        x = lq8.DeviceBuffer.from_array(ctx, rng.standard_normal((T, H)).astype(np.float32))
        sc = lq8.DeviceBuffer.from_array(ctx, rng.standard_normal((layers, T, E)).astype(np.float32))
        pos = lq8.DeviceBuffer.from_array(ctx, np.full(T, 128, np.int32))
        for _ in range(3):
            m.forward_device(x, sc, pos, T)
        ctx.synchronize()
        ids, _ = m.routing(T)
        nact = [len(set(ids[l].ravel().tolist())) for l in range(layers)]
        step_b = sum(attn_b + n * exp_b for n in nact)
        ctx.timer_start()
        for _ in range(reps):
            m.forward_device(x, sc, pos, T)
        ms = ctx.timer_stop() / reps
        gbs = step_b / (ms * 1e-3) / 1e9
        out[f"batch{T}"] = {"us_per_step": round(ms * 1e3, 1), "us_per_layer": round(ms * 1e3 / layers, 2),
                            "tokens_per_s": round(T / (ms * 1e-3), 1), "bytes_per_step": step_b,
                            "experts_per_layer": round(float(np.mean(nact)), 1), "gbs": round(gbs, 1),
                            "pct_hbm_peak": round(gbs / HBM_PEAK_GBS, 4)}
        log(f"MoE {layers} layers, T={T}: {ms * 1e3:.0f} us/step ({ms * 1e3 / layers:.1f} us/layer), "
            f"{gbs:.0f} GB/s, {T / (ms * 1e-3):.0f} tok/s")
        x.free(); sc.free(); pos.free()
    m.free()
    return out


def gemm_sweep(ctx):
    """W8A8 GEMM (activation quantize + int8 MFMA) of the gate/up (3072 x 1024)
    and down (1024 x 3072) weights at M = 512 ... 8192: per-call time by HIP
    events over 20 calls and the fraction of the dense int8 peak."""
    for n, k in ((3072, 1024), (1024, 3072)):
        w = lq8.Q8Weight.random(ctx, n, k, seed=3, stream=n)
        lin = lq8.Linear.new(w)
        for m in (512, 1024, 2048, 4096, 8192):
            x = lq8.DeviceBuffer.from_array(ctx, np.random.default_rng(m).standard_normal((m, k)).astype(np.float32))
            y = lq8.DeviceBuffer(ctx, m * n * 4)
            for _ in range(3):
                lin.forward_device(x, m, y)
            ctx.synchronize()
            ctx.timer_start()
            for _ in range(20):
                lin.forward_device(x, m, y)
            ms = ctx.timer_stop() / 20
            tops = 2 * m * n * k / (ms * 1e-3) / 1e12
            print(f"{n}x{k} M={m}: {ms * 1e3:8.2f} us  {tops:7.1f} TOPS  {tops / INT8_PEAK_TOPS * 100:5.2f} % of int8 peak",
                  flush=True)
            x.free()
            y.free()
        w.free()


def decode_only(ctx, path, new_tokens):
    """Config-4 greedy decode alone (Qwen3-0.6B shapes, random Q8_0 weights,
    128-token prompt) on one path: the replayed decode graph or the persistent
    kernel; one line with the decode rate (for hardware-counter runs)."""
    cfg = lq8.qwen3_0_6b(max_positions=512)
    model = lq8.Qwen3ForCausalLM.random(ctx, cfg, seed=2026)
    prompt = np.random.default_rng(2026).integers(0, cfg.vocab_size, 128).astype(np.uint32)
    prev = os.environ.get("LQ8_PERSIST")
    os.environ["LQ8_PERSIST"] = "1" if path == "persistent" else "0"
    try:
        model.generate_greedy(prompt, 8)
        st = model.generate_greedy(prompt, new_tokens)[1]
    finally:
        os.environ.pop("LQ8_PERSIST", None)
        if prev is not None:
            os.environ["LQ8_PERSIST"] = prev
    print(f"decode ({path}): {st['decode_tokens_per_s']:.1f} tok/s over {new_tokens} tokens, graph {st['used_graph']}, "
          f"persistent {st['used_persistent']}", flush=True)
    model.free()
    # a device copy of known size: calibrates FETCH_SIZE / WRITE_SIZE when profiled
    src, dst = lq8.DeviceBuffer(ctx, CALIB_BYTES), lq8.DeviceBuffer(ctx, CALIB_BYTES)
    lq8._check(lq8.lib().lq8_copy_device(ctx.handle, dst.ptr, src.ptr, CALIB_BYTES))
    ctx.synchronize()
    src.free()
    dst.free()


def floors(ctx, full=False):
    """The hardware floors (lq8_bench_floors): the read-only streaming rate of
    the whole chip over 1 GiB (best of the grid sizes tried), of one compute
    unit over 64 MiB, the period of back-to-back empty launches and the
    latency of one dependent HBM load (random lines of 1 GiB)."""
    gib = 1 << 30
    grids = (256, 512, 1024, 2048) if full else (256, 1024)
    stream = {}
    for kind, kname in ((lq8.FLOOR_STREAM, "grid-stride"), (lq8.FLOOR_STREAM_CHUNKS, "chunks")):
        for nwg in grids:
            lq8.bench_floor(ctx, kind, nwg, gib, 1)
            stream[f"{kname} {nwg}"] = lq8.bench_floor(ctx, kind, nwg, gib, 5)
    best = max(stream, key=stream.get)
    out = {"read_peak_gbs": round(stream[best], 1), "read_peak_pattern": best,
           "read_by_pattern_gbs": {k: round(v, 1) for k, v in stream.items()}}
    if full:
        # the config-1 GEMV against them: 3072 x 1024, cold (160 rotating copies), graph-replayed
        out["gemv_3072x1024_us"] = round(rotating_gemv_us(ctx, 3072, 1024, 160), 3)
        out["one_cu_read_gbs"] = round(lq8.bench_floor(ctx, lq8.FLOOR_STREAM, 1, 64 << 20, 3), 2)
        out["eight_cu_read_gbs"] = round(lq8.bench_floor(ctx, lq8.FLOOR_STREAM, 8, 256 << 20, 3), 2)
        out["empty_launch_us"] = {f"{nwg}x{thr}": round(lq8.bench_floor(ctx, lq8.FLOOR_EMPTY, nwg, thr, 2000), 3)
                                  for nwg, thr in ((1, 64), (192, 1024), (256, 64), (256, 512), (1024, 256))}
        out["empty_graph_node_us"] = {f"{nwg}x{thr}": round(lq8.bench_floor(ctx, lq8.FLOOR_EMPTY_GRAPH, nwg, thr, 1000), 3)
                                      for nwg, thr in ((1, 64), (96, 1024), (192, 1024), (256, 512), (1024, 256))}
        out["dependent_load_ns"] = round(lq8.bench_floor(ctx, lq8.FLOOR_CHASE, 1, gib, 20000), 1)
    return out


def sync_bench(ctx):
    """Grid-wide synchronisation (lq8_bench_grid_sync) per kind and grid size:
    device time per synchronisation over 2000 synchronisations with a data
    exchange checked every round."""
    names = {0: "one counter, release/acquire fences", 1: "one counter, data by agent-scope atomics",
             2: "per-XCD counters + global counter", 3: "per-XCD counters + per-XCD flags"}
    for kind in range(4):
        for nwg in (256, 512):
            us, bad, gave = lq8.bench_grid_sync(ctx, kind, nwg, 1000)
            print(f"kind {kind} ({names[kind]}), {nwg} workgroups x 256 threads: {us:6.2f} us per sync, "
                  f"{bad} values wrong, gave up: {gave}", flush=True)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--no-decode", action="store_true")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-moe", action="store_true")
    ap.add_argument("--only-step", action="store_true",
                    help="only the headline step and the calibration copy (for hardware-counter runs)")
    ap.add_argument("--gemm-sweep", action="store_true",
                    help="only the W8A8 GEMM at M = 512 ... 8192 (gate/up and down shapes), one line each")
    ap.add_argument("--decode-only", choices=("graph", "persistent"),
                    help="only the Qwen3-0.6B greedy decode on one path, one line (for hardware-counter runs)")
    ap.add_argument("--new-tokens", type=int, default=128, help="tokens generated by --decode-only")
    ap.add_argument("--sync-bench", action="store_true",
                    help="only the grid-wide synchronisation microbenchmark, one line per kind and grid size")
    ap.add_argument("--floors", action="store_true",
                    help="only the hardware floors (streaming read rates, launch period, HBM load latency), one line")
    ap.add_argument("--moe-only", action="store_true",
                    help="only the 48-layer MoE stack at batch 1 and 32, one line (for kernel traces)")
    args = ap.parse_args()
    if args.moe_only:
        print(json.dumps(moe_stack(lq8.Context(0))), flush=True)
        return
    if args.floors:
        print(json.dumps(floors(lq8.Context(0), full=True)), flush=True)
        return
    if args.gemm_sweep:
        gemm_sweep(lq8.Context(0))
        return
    if args.sync_bench:
        sync_bench(lq8.Context(0))
        return
    if args.decode_only:
        decode_only(lq8.Context(0), args.decode_only, args.new_tokens)
        return
    if args.only_step:
        args.no_decode = args.no_cpu = args.no_moe = True
    if args.gpus != 1:
        print(json.dumps({"error": "the Q8_0 path runs on one GPU (--gpus 1); sharding it across GPUs is "
                                   "designed, not built"}))
        sys.exit(2)

    ctx = lq8.Context(0)
    shapes, probs, bufs = make_problems(ctx, seed=1234)
    step_bytes = sum(gemv_bytes(n, k) for _, n, k in shapes)
    nlaunch = len(probs)
    log(f"step: {nlaunch} GEMVs, {step_bytes} algorithmic bytes")

    # headline: the step as one grouped launch.  The device first runs ~0.3 s
    # of steps so its clocks leave the idle state, then W warmup steps, then
    # exactly K steps between HIP events on the context stream (synchronized
    # both sides).
    t0 = time.perf_counter()
    while time.perf_counter() - t0 < 0.3:
        lq8.bench_gemv(ctx, probs, mode=1, reps=20)
    lq8.bench_gemv(ctx, probs, mode=1, reps=max(args.warmup, 1))
    ctx.synchronize()
    ms = lq8.bench_gemv(ctx, probs, mode=1, reps=args.steps)
    ctx.synchronize()
    ms_step = ms / args.steps
    value = step_bytes / (ms_step * 1e-3) / 1e9
    log(f"grouped launch: {ms_step * 1e3:.1f} us/step, {value:.1f} GB/s ({value / HBM_PEAK_GBS:.1%} of HBM peak)")

    ms_chain = ms_lm = float("nan")
    if not args.only_step:
        # the same step, one launch per GEMV (a Linear::forward each), replayed as a HIP graph
        lq8.bench_gemv(ctx, probs, mode=2, reps=2)
        ms_chain = lq8.bench_gemv(ctx, probs, mode=2, reps=max(5, args.steps // 5)) / max(5, args.steps // 5)
        log(f"one launch per GEMV (graph): {ms_chain * 1e3:.1f} us/step, "
            f"{step_bytes / (ms_chain * 1e-3) / 1e9:.1f} GB/s")
    chain_gbs = step_bytes / (ms_chain * 1e-3) / 1e9
    for w, _, _ in probs:
        w.free()
    for b in bufs:
        b.free()
    if not args.only_step:
        # lm_head alone (165 MB, the largest single GEMV), cold: graph-replayed
        # over 4 distinct copies (661 MB, beyond the 256 MB Infinity Cache)
        ms_lm = rotating_gemv_us(ctx, LM_HEAD[1], LM_HEAD[2], 4) * 1e-3
        log(f"lm_head (cold, 4 rotating copies): {ms_lm * 1e3:.1f} us, "
            f"{gemv_bytes(*LM_HEAD[1:]) / (ms_lm * 1e-3) / 1e9:.1f} GB/s")
    lm_gbs = gemv_bytes(*LM_HEAD[1:]) / (ms_lm * 1e-3) / 1e9

    # known-size copy: calibrates FETCH_SIZE / WRITE_SIZE when profiled
    # (also the measured stream-copy peak: read + write bytes per second)
    src, dst = lq8.DeviceBuffer(ctx, CALIB_BYTES), lq8.DeviceBuffer(ctx, CALIB_BYTES)
    for _ in range(3):
        lq8._check(lq8.lib().lq8_copy_device(ctx.handle, dst.ptr, src.ptr, CALIB_BYTES))
    ctx.synchronize()
    copy_gbs = None
    if not args.only_step:
        ctx.timer_start()
        for _ in range(10):
            lq8._check(lq8.lib().lq8_copy_device(ctx.handle, dst.ptr, src.ptr, CALIB_BYTES))
        copy_ms = ctx.timer_stop() / 10
        copy_gbs = 2 * CALIB_BYTES / (copy_ms * 1e-3) / 1e9
        log(f"device copy 256 MiB: {copy_ms * 1e3:.1f} us, {copy_gbs:.0f} GB/s read+write")
    src.free()
    dst.free()
    # the measured read-only streaming ceiling (the headline kernel only reads)
    read_peak = None
    if not args.only_step:
        read_peak = floors(ctx)
        log(f"read-only stream, 1 GiB: {read_peak['read_peak_gbs']} GB/s")

    # the single 3072 x 1024 GEMV (cold: 160 rotating copies, 535 MB)
    c1_us = float("nan")
    linear_host = None
    if not args.only_step:
        c1_us = rotating_gemv_us(ctx, 3072, 1024, 160)
        log(f"GEMV 3072x1024: {c1_us:.2f} us, {gemv_bytes(3072, 1024) / c1_us / 1e3:.1f} GB/s")
        linear_host = linear_forward_host(ctx)
        log(f"host-pointer Linear::forward per call: {linear_host}")

    # prefill-shaped W8A8 GEMM, M = 512 (activation quantize + int8 MFMA)
    gemm = {}
    for name, n, k in ([] if args.only_step else [("gate_up", 3072, 1024), ("down", 1024, 3072)]):
        w = lq8.Q8Weight.random(ctx, n, k, seed=3, stream=n)
        x = lq8.DeviceBuffer.from_array(ctx, np.random.default_rng(3).standard_normal((512, k)).astype(np.float32))
        y = lq8.DeviceBuffer(ctx, 512 * n * 4)
        lin = lq8.Linear.new(w)
        for _ in range(3):
            lin.forward_device(x, 512, y)
        ctx.synchronize()
        ctx.timer_start()
        for _ in range(20):
            lin.forward_device(x, 512, y)
        ms = ctx.timer_stop() / 20
        tops = 2 * 512 * n * k / (ms * 1e-3) / 1e12
        # compulsory bytes: Q8_0 weight + Q8_0 activations + f32 output
        gbytes = n * k * 34 // 32 + 512 * k * 34 // 32 + 4 * 512 * n
        floor_us = max(gbytes / HBM_PEAK_GBS / 1e3, 2 * 512 * n * k / INT8_PEAK_TOPS / 1e6)
        gemm[name] = {"us": round(ms * 1e3, 2), "TOPS": round(tops, 1), "mfma_frac": round(tops / INT8_PEAK_TOPS, 4),
                      "bytes": gbytes, "floor_us": round(floor_us, 2),
                      "mfma_ceiling_frac": round(2 * 512 * n * k / INT8_PEAK_TOPS / 1e6 / floor_us, 3)}
        log(f"GEMM {name} M=512: {ms * 1e3:.1f} us, {tops:.1f} TOPS (includes the activation quantize)")
        w.free(); x.free(); y.free()

    decode = None
    cpu_model = None
    if not args.no_decode:
        cfg = lq8.qwen3_0_6b(max_positions=512)
        model = lq8.Qwen3ForCausalLM.random(ctx, cfg, seed=2026)
        prompt = np.random.default_rng(2026).integers(0, cfg.vocab_size, 128).astype(np.uint32)
        model.generate_greedy(prompt, 8)
        runs = [model.generate_greedy(prompt, 128)[1] for _ in range(3)]
        tps = sorted(r["decode_tokens_per_s"] for r in runs)[1]
        # sampled decode: penalty, temperature, top-k and top-p on the device
        gc = lq8.GenerationConfig(128, 0.8, 50, 0.95, 1.1)
        model.generate(prompt, gc, seed=1)
        sruns = [model.generate(prompt, gc, seed=1 + i)[1] for i in range(3)]
        stps = sorted(r["decode_tokens_per_s"] for r in sruns)[1]
        # the replayed decode graph (LQ8_PERSIST=0), the path before the
        # persistent kernel became the default
        os.environ["LQ8_PERSIST"] = "0"
        try:
            model.generate_greedy(prompt, 8)
            gruns = [model.generate_greedy(prompt, 128)[1] for _ in range(3)]
        finally:
            del os.environ["LQ8_PERSIST"]
        gtps = sorted(r["decode_tokens_per_s"] for r in gruns)[1] if all(r["used_graph"] for r in gruns) else None
        # every Q8_0 matrix of the model is read once per token (the tied
        # embedding as the lm_head); the step is a chain of dependent kernels
        wbytes = LAYERS * sum(n * k * 34 // 32 for _, n, k in LAYER_SHAPES) + LM_HEAD[1] * LM_HEAD[2] * 34 // 32
        chain = 5 * LAYERS + 3
        path = "persistent" if runs[0]["used_persistent"] else ("graph" if runs[0]["used_graph"] else "plain")
        decode = {"tokens_per_s": round(tps, 1), "us_per_token": round(1e6 / tps, 1), "path": path,
                  "weight_bytes_per_token": wbytes, "weight_gbs": round(wbytes * tps / 1e9, 1),
                  "bound": "latency: one cooperative kernel for all steps of a generate() call; per layer five "
                           "phases whose values pass between workgroups as tagged words" if path == "persistent"
                           else "latency: a chain of dependent kernels per token",
                  "prefill_ms": round(runs[0]["prefill_ms"], 2), "prompt": 128, "new_tokens": 128,
                  "graph_tokens_per_s": None if gtps is None else round(gtps, 1),
                  "graph_kernels_per_token": chain,
                  "graph_us_per_kernel": None if gtps is None else round(1e6 / gtps / chain, 2),
                  "sampled_tokens_per_s": round(stps, 1),
                  "sampled_config": {"temperature": 0.8, "top_k": 50, "top_p": 0.95, "repetition_penalty": 1.1},
                  "sampler_us_over_greedy_graph": None if gtps is None else round(1e6 / stps - 1e6 / gtps, 1)}
        log(f"decode: {tps:.1f} tok/s ({path}, median of 3), prefill {runs[0]['prefill_ms']:.2f} ms; "
            f"graph {gtps} tok/s; sampled (graph) {stps:.1f} tok/s")
        if not args.no_cpu:
            cpu_model = (cfg, model.export_all(), prompt)
        model.free()
        # the same model with Qwen3-0.6B's own max_position_embeddings (a 9.4 GB
        # KV cache; 640 attention segments of capacity, 3 in use)
        decode["qwen3_0_6b_max_positions_40960"] = decode_larger(ctx, lq8.qwen3_0_6b(max_positions=40960),
                                                                 "Qwen3-0.6B, max_positions 40960")
        decode["qwen3_1_7b"] = decode_larger(ctx, lq8.qwen3_1_7b(max_positions=512), "Qwen3-1.7B")
        decode["qwen3_4b"] = decode_larger(ctx, lq8.qwen3_4b(max_positions=512), "Qwen3-4B")

    moe = None if args.no_moe else moe_stack(ctx)
    ctx.close()

    cpu = None if args.no_cpu else cpu_reference_linear()
    if cpu:
        log(f"cpu baseline: {cpu['value']} GB/s ({cpu['sample']}); {cpu['layer_ms']} ms per layer, "
            f"~{cpu['token_s_extrapolated']} s per token")
        cpu["q8_oracle"] = cpu_baseline(seconds_target=6.0)
        log(f"cpu Q8_0 oracle: {cpu['q8_oracle']['value']} GB/s on one core")
        cpu["host"] = host_cpu()
        cpu["all_cores"] = cpu_gemv_all_cores()
        log(f"cpu all cores: {cpu['all_cores']['value']} GB/s on {cpu['all_cores']['cores']} threads")
        if cpu_model is not None:
            cpu["decode"] = cpu_decode(*cpu_model)
            log(f"cpu decode: {cpu['decode']['tokens_per_s']} tok/s ({cpu['decode']['sample']})")

    traffic = measured_traffic()
    out = {
        "metric": "Q8_0 GEMV HBM GB/s (% peak) + batch-1 decode tokens/s, Qwen3-0.6B shapes",
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8 codes x f32 (W8A32), f32 accumulate",
        "data": "synthetic: seeded N(0,0.02) Q8_0 weights, N(0,1) inputs",
        "config": {"workload": "Qwen3-0.6B decode-token linear set, batch 1: 28 x {q 2048x1024, k 1024x1024, "
                               "v 1024x1024, o 1024x2048, gate 3072x1024, up 3072x1024, down 1024x3072} + lm_head "
                               "151936x1024, 197 independent Q8_0 GEMVs streamed by one grouped launch",
                   "gemvs_per_step": nlaunch, "bytes_per_step": step_bytes,
                   "pct_hbm_peak": round(value / HBM_PEAK_GBS, 4)},
        "roofline": {"bound": "hbm", "achieved": round(value, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(value / HBM_PEAK_GBS, 4), "traffic": traffic,
                     "kernel": "k_gemv_grouped", "launch_us": round(ms_step * 1e3, 2),
                     "bytes_per_launch": step_bytes,
                     "measured_read_peak_gbs": None if read_peak is None else read_peak["read_peak_gbs"],
                     "frac_of_measured_read_peak": None if read_peak is None else
                     round(value / read_peak["read_peak_gbs"], 4)},
        "copy_peak_gbs": None if copy_gbs is None else round(copy_gbs, 1),
        "one_launch_per_gemv_gbs": None if args.only_step else round(chain_gbs, 1),
        "one_launch_per_gemv_frac": None if args.only_step else round(chain_gbs / HBM_PEAK_GBS, 4),
        "one_launch_per_gemv_us_per_step": None if args.only_step else round(ms_chain * 1e3, 1),
        "lm_head_cold_gbs": None if args.only_step else round(lm_gbs, 1),
        "lm_head_cold_us": None if args.only_step else round(ms_lm * 1e3, 2),
        "gemv_3072x1024_us": None if args.only_step else round(c1_us, 3),
        "gemv_3072x1024_gbs": None if args.only_step else round(gemv_bytes(3072, 1024) / c1_us / 1e3, 1),
        "linear_forward_host_us": linear_host,
        "gemm_m512": gemm,
        "decode": decode,
        "moe_qwen3_30b_a3b_48_layers": moe,
        "cpu_baseline": cpu,
    }
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
