"""The persistent decode's phase timeline: the trace build (make trace) runs
the kernel with its marks and lq8.persist_trace reads and summarises them;
the ordinary build refuses the read."""
import os
import subprocess
import sys

import pytest

import lq8

pytestmark = pytest.mark.gpu

PKG = os.path.join(os.path.dirname(os.path.abspath(__file__)), "..", "qwen-omni-inference-rs_amd")


def test_ordinary_build_refuses_the_trace_read(ctx):
    with pytest.raises(lq8.InvalidArgument):
        lq8.persist_trace(ctx)


def test_trace_build_timeline():
    if not os.path.exists(os.path.join(PKG, "lq8", "liblq8_trace.so")):
        pytest.skip("trace build absent (make -C qwen-omni-inference-rs_amd trace)")
    # a process of its own: it loads the trace build in place of liblq8.so
    r = subprocess.run([sys.executable, "-u", "-m", "lq8.persist_trace", "--layers", "6", "--new", "6"], cwd=PKG,
                       capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stderr[-2000:]
    lines = r.stdout.splitlines()
    assert lines[0].startswith("decode ") and "layer period" in lines[0]
    marks = {l.split()[0]: [float(v) for v in l.split()[2:5]] for l in lines[2:] if l.split()[0].startswith("P")}
    for name in ("P1_NORMED", "P2_QKV_IN", "P3_STAGED", "P4_STAGED", "P5_STAGED", "P5_DONE", "P6_DONE"):
        assert name in marks, (name, r.stdout)
    # within a layer the phases follow each other
    assert marks["P1_NORMED"][1] < marks["P3_STAGED"][1] < marks["P4_STAGED"][1] < marks["P5_DONE"][1]
