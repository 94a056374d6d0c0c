"""CPU: the C-ABI library loads, exports every symbol include/lq8.h declares,
and rejects bad input without a device; the oracle library likewise."""
import ctypes
import os
import re

import numpy as np
import pytest

import lq8
import oracle

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared(header):
    text = open(header).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b((?:lq8|orc)_[a-z0-9_]+)\s*\(", text)))


def test_lq8_exports_every_declared_symbol():
    lib = lq8.lib()
    names = declared(os.path.join(ROOT, "include", "lq8.h"))
    assert len(names) > 30
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing
    assert set(names) == set(lq8.EXPORTED), set(names) ^ set(lq8.EXPORTED)


def test_oracle_exports_every_declared_symbol():
    lib = ctypes.CDLL(oracle.LIB_PATH)
    names = declared(os.path.join(ROOT, "oracle", "lq8_oracle.h"))
    assert [n for n in names if not hasattr(lib, n)] == []


def test_host_quantizer_matches_oracle():
    x = np.random.default_rng(3).standard_normal(32 * 5000).astype(np.float32)
    x[::997] = np.nan
    assert np.array_equal(lq8.quantize_q8_0(x), oracle.quantize_q8_0(x))
    b = lq8.quantize_q8_0(x)
    assert np.array_equal(lq8.dequantize_q8_0(b, x.size).view(np.uint32),
                          oracle.dequantize_q8_0(b, x.size).view(np.uint32))
    assert lq8.lib().lq8_q8_0_bytes(4096) == 4096 // 32 * 34


def test_host_errors():
    with pytest.raises(lq8.ShapeMismatch) as e:
        lq8.quantize_q8_0(np.zeros(33, np.float32))
    assert "multiple of 32" in str(e.value)
    assert lq8.lib().lq8_quantize_q8_0(None, 64, None) == lq8.InvalidArgument.status


def test_no_device_is_an_error_not_a_fallback():
    if lq8.device_count() > 0:
        pytest.skip("a GPU is present")
    with pytest.raises(lq8.NoDevice):
        lq8.Context(0)


def test_stale_handles_rejected():
    bogus = ctypes.c_void_p(0x1234)
    assert lq8.lib().lq8_weight_free(bogus) == lq8.InvalidArgument.status
    assert lq8.lib().lq8_shutdown(bogus) == lq8.InvalidArgument.status
    assert lq8.lib().lq8_model_free(bogus) == lq8.InvalidArgument.status
