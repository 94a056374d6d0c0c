"""The persistent decode's phase timeline: the trace build (make trace) runs
the kernel with its marks, lq8.persist_trace reads them and
lq8.trace_timeline summarises them; the ordinary build refuses the read."""
import os

import pytest

import lq8
from lq8 import trace_timeline as pt

pytestmark = pytest.mark.gpu

PKG = os.path.join(os.path.dirname(os.path.abspath(__file__)), "..", "qwen-omni-inference-rs_amd")


def test_ordinary_build_refuses_the_trace_read(ctx):
    with pytest.raises(lq8.InvalidArgument):
        lq8.persist_trace(ctx)


def test_trace_build_timeline():
    if not os.path.exists(os.path.join(PKG, "lq8", "liblq8_trace.so")):
        pytest.skip("trace build absent (make -C qwen-omni-inference-rs_amd trace)")
    layers = 6
    stats, tr = pt.collect(layers, prompt=128, new=6)
    assert stats["used_persistent"]
    assert tr.shape == (lq8.PTRACE_WG, lq8.PTRACE_LAYERS, lq8.PTRACE_POINTS)
    rows, period, p6 = pt.timeline(tr, layers)
    marks = {name: v for name, _, v in rows}
    for name in ("P1_NORMED", "P2_QKV_IN", "P3_STAGED", "P4_STAGED", "P5_STAGED", "P5_DONE"):
        assert name in marks, (name, sorted(marks))
    # within a layer the phases follow each other, and a layer takes its period
    assert marks["P1_NORMED"][1] < marks["P3_STAGED"][1] < marks["P4_STAGED"][1] < marks["P5_DONE"][1] < period
    assert [name for name, _, _ in p6] == ["P6_START", "P6_NORMED", "P6_DONE"]
    # the calls after the block go to liblq8.so again
    assert lq8.LIB_PATH.endswith("liblq8.so") and lq8.lib()._name.endswith("liblq8.so")
