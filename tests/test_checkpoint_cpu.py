"""CPU: checkpoint formats (no device).

- GGUF: a file assembled byte by byte from the GGUF v3 specification (not by
  our writer) parses to the expected metadata and tensors; writer -> reader
  round trips keep every byte; dimension order is ggml's (ne[0] innermost).
- safetensors: files written by the `safetensors` package (BF16 and F32)
  parse to the same bits; other dtypes are rejected as the reference's loader
  does (src/loader.rs:176-183).
- HF config.json -> Qwen3Config; tensor-name tables match the table order.
"""
import json
import struct

import numpy as np
import pytest

import lq8
from lq8 import checkpoint as ck
import oracle


def _s(x: str) -> bytes:
    b = x.encode()
    return struct.pack("<Q", len(b)) + b


def test_gguf_reader_on_spec_built_file(tmp_path):
    a = np.arange(6, dtype=np.float32).reshape(2, 3)           # [rows 2, cols 3] -> ne = [3, 2]
    q = oracle.quantize_q8_0(np.linspace(-1, 1, 64, dtype=np.float32))   # one row of 2 blocks: ne = [64, 1]
    kv = (_s("general.architecture") + struct.pack("<I", 8) + _s("qwen3") +
          _s("some.u32") + struct.pack("<II", 4, 7) +
          _s("some.f32") + struct.pack("<If", 6, 0.5) +
          _s("some.arr") + struct.pack("<IIQ", 9, 8, 2) + _s("x") + _s("yz"))
    info = (_s("a") + struct.pack("<I", 2) + struct.pack("<QQ", 3, 2) + struct.pack("<IQ", 0, 0) +
            _s("b") + struct.pack("<I", 2) + struct.pack("<QQ", 64, 1) + struct.pack("<IQ", 8, 32))
    head = b"GGUF" + struct.pack("<IQQ", 3, 2, 4) + kv + info
    head += b"\0" * ((-len(head)) % 32)
    data = a.tobytes() + b"\0" * (32 - 24) + q.tobytes()
    p = tmp_path / "spec.gguf"
    p.write_bytes(head + data)
    g = ck.GgufFile(str(p))
    assert g.metadata == {"general.architecture": "qwen3", "some.u32": 7, "some.f32": 0.5, "some.arr": ["x", "yz"]}
    assert g.tensors["a"].shape == (2, 3) and g.tensors["a"].ggml_type == ck.GGML_F32
    assert np.array_equal(g.tensors["a"].data.reshape(2, 3), a)
    assert g.tensors["b"].shape == (1, 64) and g.tensors["b"].ggml_type == ck.GGML_Q8_0
    assert g.tensors["b"].data.tobytes() == q.tobytes()
    g.close()


@pytest.mark.parametrize("alignment", [32, 64])
def test_gguf_write_read_round_trip(tmp_path, alignment):
    rng = np.random.default_rng(1)
    tens = [ck.GgufTensor("w", ck.GGML_Q8_0, (5, 96), oracle.quantize_q8_0(rng.standard_normal(5 * 96).astype(np.float32))),
            ck.GgufTensor("n", ck.GGML_F32, (7,), rng.standard_normal(7).astype(np.float32)),
            ck.GgufTensor("h", ck.GGML_BF16, (3, 4), rng.integers(0, 65535, 12).astype(np.uint16))]
    md = {"general.architecture": "qwen3", "k.u": 5, "k.big": 2 ** 40, "k.f": 1.25, "k.s": "abc", "k.b": True,
          "k.arr": ["p", "q"]}
    p = tmp_path / "rt.gguf"
    ck.write_gguf(str(p), md, tens, alignment=alignment)
    raw = p.read_bytes()
    assert raw[:4] == b"GGUF" and struct.unpack_from("<I", raw, 4)[0] == 3
    g = ck.GgufFile(str(p))
    want = dict(md)
    if alignment != 32:
        want["general.alignment"] = alignment
    assert g.metadata == want
    for t in tens:
        r = g.tensors[t.name]
        assert r.ggml_type == t.ggml_type and r.shape == t.shape
        assert r.data.tobytes() == np.ascontiguousarray(t.data).tobytes()
    g.close()


def test_gguf_rejects_bad_files(tmp_path):
    p = tmp_path / "bad.gguf"
    p.write_bytes(b"GGUX" + b"\0" * 40)
    with pytest.raises(ValueError):
        ck.GgufFile(str(p))
    t = ck.GgufTensor("x", 2, (1, 32), np.zeros(18, np.uint8))  # Q4_0: not supported here
    ck.write_gguf(str(p), {}, [t])
    with pytest.raises(ValueError, match="not supported"):
        ck.GgufFile(str(p))


def test_safetensors_reader_matches_writer(tmp_path):
    torch = pytest.importorskip("torch")
    st = pytest.importorskip("safetensors.torch")
    g = torch.Generator().manual_seed(3)
    a = torch.randn(4, 64, generator=g).to(torch.bfloat16)
    b = torch.randn(5, generator=g)
    p = tmp_path / "m.safetensors"
    st.save_file({"a": a, "b": b}, str(p))
    f = ck.SafeTensorsFile(str(p))
    assert sorted(f.tensor_names()) == ["a", "b"] and len(f) == 2
    ta, tb = f.get("a"), f.get("b")
    assert ta.dtype == "BF16" and ta.shape == (4, 64) and tb.dtype == "F32" and tb.shape == (5,)
    assert np.array_equal(ta.data, a.view(torch.int16).numpy().view(np.uint16).ravel())
    assert np.array_equal(tb.data, b.numpy())
    assert np.array_equal(ck.bf16_to_f32(ta.data), a.float().numpy().ravel())
    f.close()
    st.save_file({"c": torch.zeros(3, dtype=torch.float16)}, str(p))
    with pytest.raises(ValueError, match="Only BF16 and F32"):
        ck.SafeTensorsFile(str(p))


def test_config_json_and_name_tables(tmp_path):
    cfg_json = {"vocab_size": 151936, "hidden_size": 1024, "intermediate_size": 3072, "num_hidden_layers": 28,
                "num_attention_heads": 16, "num_key_value_heads": 8, "head_dim": 128,
                "max_position_embeddings": 40960, "rms_norm_eps": 1e-6, "rope_theta": 1000000,
                "tie_word_embeddings": True}
    p = tmp_path / "config.json"
    p.write_text(json.dumps(cfg_json))
    c = ck.qwen3_config_from_json(str(p), max_positions=512)
    assert c == lq8.qwen3_0_6b(max_positions=512)
    hf, gg = ck.hf_tensor_names(c), ck.gguf_tensor_names(c)
    assert len(hf) == len(gg) == c.tensor_count()
    for i, (h, g) in enumerate(zip(hf, gg)):
        kind, _ = c.tensor_shape(i)
        assert (kind == "f32") == ("norm" in h) == ("norm" in g)
    md = ck.qwen3_gguf_metadata(c)
    assert md["qwen3.block_count"] == 28 and md["qwen3.attention.head_count_kv"] == 8
