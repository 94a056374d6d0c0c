"""GPU: checkpoint ingestion through the C ABI.

A tiny Qwen3 checkpoint in the HF layout (config.json + BF16
model.safetensors) is loaded with quantize-on-load: every exported Q8_0
tensor must equal the oracle quantizer applied to the exactly widened bf16
values, and the logits must equal the oracle model's on those blocks.  The
loaded model saved as GGUF and read back gives the same tensors and logits.
"""
import dataclasses
import json

import numpy as np
import pytest

import lq8
from lq8 import checkpoint as ck
import oracle

pytestmark = pytest.mark.gpu


def tiny_cfg():
    return lq8.Qwen3Config(vocab_size=320, hidden_size=256, intermediate_size=96, num_hidden_layers=2,
                           num_attention_heads=4, num_key_value_heads=2, head_dim=128, max_position_embeddings=64)


def write_hf_checkpoint(d, cfg, seed):
    torch = pytest.importorskip("torch")
    st = pytest.importorskip("safetensors.torch")
    g = torch.Generator().manual_seed(seed)
    tensors = {}
    for i, name in enumerate(ck.hf_tensor_names(cfg)):
        kind, shape = cfg.tensor_shape(i)
        if kind == "f32":
            t = 1.0 + 0.1 * torch.randn(shape, generator=g)
        else:
            t = 0.02 * torch.randn(shape, generator=g)
        tensors[name] = t.to(torch.bfloat16)
    st.save_file(tensors, str(d / "model.safetensors"))
    (d / "config.json").write_text(json.dumps({
        "vocab_size": cfg.vocab_size, "hidden_size": cfg.hidden_size, "intermediate_size": cfg.intermediate_size,
        "num_hidden_layers": cfg.num_hidden_layers, "num_attention_heads": cfg.num_attention_heads,
        "num_key_value_heads": cfg.num_key_value_heads, "head_dim": cfg.head_dim,
        "max_position_embeddings": cfg.max_position_embeddings, "rms_norm_eps": cfg.rms_norm_eps,
        "rope_theta": cfg.rope_theta, "tie_word_embeddings": True}))
    return {k: v.view(torch.int16).numpy().view(np.uint16).ravel() for k, v in tensors.items()}


def expected_table(cfg, raw):
    out = []
    for i, name in enumerate(ck.hf_tensor_names(cfg)):
        kind, _ = cfg.tensor_shape(i)
        f = ck.bf16_to_f32(raw[name])
        out.append(f if kind == "f32" else oracle.quantize_q8_0(f))
    return out


def test_safetensors_quantize_on_load_and_gguf_round_trip(ctx, tmp_path):
    cfg = tiny_cfg()
    raw = write_hf_checkpoint(tmp_path, cfg, 7)
    model = lq8.Qwen3ForCausalLM.from_safetensors(ctx, str(tmp_path))
    assert model.cfg == cfg
    want = expected_table(cfg, raw)
    got = model.export_all()
    for i, (a, b) in enumerate(zip(got, want)):
        assert a.tobytes() == np.ascontiguousarray(b).tobytes(), f"tensor {i} {ck.hf_tensor_names(cfg)[i]}"
    ids = [3, 17, 255, 90, 4]
    ref = oracle.Model(cfg, want)
    logits = model.forward(ids, 0)
    ref_logits = ref.forward(ids, 0)
    assert np.array_equal(logits.view(np.uint32), ref_logits.view(np.uint32))

    path = tmp_path / "tiny.gguf"
    model.save_gguf(str(path))
    g = ck.GgufFile(str(path))
    assert g.metadata["general.architecture"] == "qwen3"
    assert g.tensors["blk.1.ffn_down.weight"].shape == (cfg.hidden_size, cfg.intermediate_size)
    g.close()
    back = lq8.Qwen3ForCausalLM.from_gguf(ctx, str(path), max_positions=cfg.max_position_embeddings)
    # GGUF stores the epsilon as float32, the precision the model uses
    assert np.float32(back.cfg.rms_norm_eps) == np.float32(cfg.rms_norm_eps)
    assert dataclasses.replace(back.cfg, rms_norm_eps=cfg.rms_norm_eps) == cfg
    for i, (a, b) in enumerate(zip(back.export_all(), got)):
        assert a.tobytes() == b.tobytes(), f"tensor {i}"
    assert np.array_equal(back.forward(ids, 0).view(np.uint32), logits.view(np.uint32))
    back.free()
    model.free()
    ref.close()


def test_weight_quantize_upload_bf16(ctx):
    rng = np.random.default_rng(5)
    f = (rng.standard_normal((48, 96)) * 0.05).astype(np.float32)
    bits = (f.view(np.uint32) >> 16).astype(np.uint16)          # truncate to bf16 bit patterns
    w = lq8.C.c_void_p()
    lq8._check(lq8.lib().lq8_weight_quantize_upload_bf16(ctx.handle, lq8._ptr(bits), 48, 96, lq8.C.byref(w)))
    q = lq8.Q8Weight(ctx, w)
    assert q.download().tobytes() == oracle.quantize_q8_0(ck.bf16_to_f32(bits)).tobytes()
    q.free()


def test_loader_errors(ctx, tmp_path):
    cfg = tiny_cfg()
    write_hf_checkpoint(tmp_path, cfg, 9)
    bad = lq8.Qwen3Config(**{**cfg.__dict__, "intermediate_size": 128})
    with pytest.raises(ValueError, match="shape"):
        lq8.Qwen3ForCausalLM.from_safetensors(ctx, str(tmp_path / "model.safetensors"), cfg=bad)
    tens = [np.zeros(1, np.uint8)] * cfg.tensor_count()
    with pytest.raises(lq8.DTypeMismatch):
        lq8.Qwen3ForCausalLM.load_typed(ctx, cfg, tens, [7] * cfg.tensor_count())
