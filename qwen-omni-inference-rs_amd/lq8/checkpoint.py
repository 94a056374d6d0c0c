"""Checkpoint ingestion: safetensors (BF16/F32, quantized to Q8_0 on load) and
GGUF (Q8_0 + F32, read and written).

Mirrors the reference's loader (lluda-inference/src/loader.rs:68-188,
ModelWeights::from_safetensors / get / tensor_names; only BF16 and F32 are
accepted, other dtypes are an error), its weight names
(src/model.rs:439-538) and its config parsing (src/config.rs:15-120), and
adds the GGUF block_q8_0 container the reference plans to read
(docs/architecture/arch-2026-01-31-qwen3-omni-q8-rust.md:140-146,275-279).

Both formats are parsed here without executing anything from the file:
safetensors is an 8-byte header length, a JSON header and raw little-endian
tensor bytes; GGUF v3 is the little-endian key/value + tensor-info layout of
the public GGUF specification.  Tensor data is memory-mapped.
"""
from __future__ import annotations

import json
import mmap
import os
import struct
from dataclasses import dataclass
from typing import Dict, List, Optional, Sequence, Tuple

import numpy as np

# ---- safetensors -------------------------------------------------------------

_ST_DTYPES = {"BF16": (np.uint16, 2), "F32": (np.float32, 4)}


@dataclass
class StTensor:
    dtype: str            # "BF16" or "F32"
    shape: Tuple[int, ...]
    data: np.ndarray      # uint16 (bf16 bits) or float32, flat, read-only view of the file


class SafeTensorsFile:
    """ModelWeights::from_safetensors: every tensor of the file, memory-mapped."""

    def __init__(self, path: str):
        self.path = path
        self._f = open(path, "rb")
        self._mm = mmap.mmap(self._f.fileno(), 0, access=mmap.ACCESS_READ)
        if len(self._mm) < 8:
            raise ValueError(f"{path}: not a safetensors file (too short)")
        (hlen,) = struct.unpack_from("<Q", self._mm, 0)
        if hlen > len(self._mm) - 8:
            raise ValueError(f"{path}: header length {hlen} beyond the file")
        header = json.loads(bytes(self._mm[8:8 + hlen]).decode("utf-8"))
        base = 8 + hlen
        self.tensors: Dict[str, StTensor] = {}
        for name, info in header.items():
            if name == "__metadata__":
                continue
            dt = info["dtype"]
            if dt not in _ST_DTYPES:
                raise ValueError(f"Unsupported dtype: {dt}. Only BF16 and F32 are supported.")
            np_dt, size = _ST_DTYPES[dt]
            shape = tuple(int(d) for d in info["shape"])
            begin, end = (int(v) for v in info["data_offsets"])
            count = int(np.prod(shape)) if shape else 1
            if end - begin != count * size:
                raise ValueError(f"{dt} tensor size mismatch for {name}: expected {count * size} bytes, "
                                 f"got {end - begin}")
            data = np.frombuffer(self._mm, dtype=np_dt, count=count, offset=base + begin)
            self.tensors[name] = StTensor(dt, shape, data)

    def get(self, name: str) -> Optional[StTensor]:
        return self.tensors.get(name)

    def tensor_names(self) -> List[str]:
        return list(self.tensors)

    def __len__(self) -> int:
        return len(self.tensors)

    def close(self) -> None:
        self.tensors = {}
        try:
            self._mm.close()
        except BufferError:  # arrays handed out still view the mapping; it ends with the last of them
            pass
        self._f.close()


def bf16_to_f32(bits: np.ndarray) -> np.ndarray:
    """Exact widening of bf16 bit patterns."""
    return (np.asarray(bits, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def qwen3_config_from_json(path: str, max_positions: Optional[int] = None):
    """Qwen3Config::from_file (src/config.rs:116-120) for the fields the decoder uses."""
    from . import Qwen3Config

    with open(path, "r", encoding="utf-8") as f:
        c = json.load(f)
    heads = int(c["num_attention_heads"])
    head_dim = int(c.get("head_dim", int(c["hidden_size"]) // heads))
    return Qwen3Config(vocab_size=int(c["vocab_size"]), hidden_size=int(c["hidden_size"]),
                       intermediate_size=int(c["intermediate_size"]),
                       num_hidden_layers=int(c["num_hidden_layers"]), num_attention_heads=heads,
                       num_key_value_heads=int(c.get("num_key_value_heads", heads)), head_dim=head_dim,
                       max_position_embeddings=int(max_positions or c.get("max_position_embeddings", 4096)),
                       rms_norm_eps=float(c.get("rms_norm_eps", 1e-6)),
                       rope_theta=float(c.get("rope_theta", 1e6)))


def hf_tensor_names(cfg) -> List[str]:
    """HF names in the table order of lq8_model_create (src/model.rs:439-538);
    the lm_head is tied to the embedding (tie_word_embeddings, src/config.rs:81)."""
    names = ["model.embed_tokens.weight", "model.norm.weight"]
    for l in range(cfg.num_hidden_layers):
        p = f"model.layers.{l}"
        names += [f"{p}.input_layernorm.weight", f"{p}.post_attention_layernorm.weight",
                  f"{p}.self_attn.q_norm.weight", f"{p}.self_attn.k_norm.weight",
                  f"{p}.self_attn.q_proj.weight", f"{p}.self_attn.k_proj.weight", f"{p}.self_attn.v_proj.weight",
                  f"{p}.self_attn.o_proj.weight", f"{p}.mlp.gate_proj.weight", f"{p}.mlp.up_proj.weight",
                  f"{p}.mlp.down_proj.weight"]
    return names


# ---- GGUF --------------------------------------------------------------------

GGUF_MAGIC = b"GGUF"
GGUF_VERSION = 3
GGUF_DEFAULT_ALIGNMENT = 32
# gguf_metadata_value_type
GV_UINT8, GV_INT8, GV_UINT16, GV_INT16, GV_UINT32, GV_INT32, GV_FLOAT32, GV_BOOL, GV_STRING, GV_ARRAY, \
    GV_UINT64, GV_INT64, GV_FLOAT64 = range(13)
_GV_SCALAR = {GV_UINT8: "<B", GV_INT8: "<b", GV_UINT16: "<H", GV_INT16: "<h", GV_UINT32: "<I", GV_INT32: "<i",
              GV_FLOAT32: "<f", GV_BOOL: "<?", GV_UINT64: "<Q", GV_INT64: "<q", GV_FLOAT64: "<d"}
# ggml_type
GGML_F32, GGML_F16, GGML_Q8_0, GGML_BF16 = 0, 1, 8, 30
_GGML_BLOCK = {GGML_F32: (1, 4), GGML_F16: (1, 2), GGML_Q8_0: (32, 34), GGML_BF16: (1, 2)}


@dataclass
class GgufTensor:
    name: str
    ggml_type: int
    shape: Tuple[int, ...]  # row-major (outermost first): [n_out, k_in] for a weight
    data: np.ndarray        # uint8 bytes (Q8_0 blocks) or float32 / uint16 values, flat


def _read_str(buf, off):
    (n,) = struct.unpack_from("<Q", buf, off)
    off += 8
    return bytes(buf[off:off + n]).decode("utf-8"), off + n


def _read_value(buf, off, vt):
    if vt == GV_STRING:
        return _read_str(buf, off)
    if vt == GV_ARRAY:
        (et,) = struct.unpack_from("<I", buf, off)
        (n,) = struct.unpack_from("<Q", buf, off + 4)
        off += 12
        out = []
        for _ in range(n):
            v, off = _read_value(buf, off, et)
            out.append(v)
        return out, off
    if vt not in _GV_SCALAR:
        raise ValueError(f"unknown GGUF value type {vt}")
    fmt = _GV_SCALAR[vt]
    (v,) = struct.unpack_from(fmt, buf, off)
    return v, off + struct.calcsize(fmt)


class GgufFile:
    """A GGUF v3 file: metadata key/values and memory-mapped tensors."""

    def __init__(self, path: str):
        self.path = path
        self._f = open(path, "rb")
        self._mm = mmap.mmap(self._f.fileno(), 0, access=mmap.ACCESS_READ)
        buf = self._mm
        if bytes(buf[0:4]) != GGUF_MAGIC:
            raise ValueError(f"{path}: not a GGUF file")
        version, n_tensors, n_kv = struct.unpack_from("<IQQ", buf, 4)
        if version not in (2, 3):
            raise ValueError(f"{path}: GGUF version {version} is not supported")
        off = 24
        self.metadata: Dict[str, object] = {}
        for _ in range(n_kv):
            key, off = _read_str(buf, off)
            (vt,) = struct.unpack_from("<I", buf, off)
            val, off = _read_value(buf, off + 4, vt)
            self.metadata[key] = val
        infos = []
        for _ in range(n_tensors):
            name, off = _read_str(buf, off)
            (nd,) = struct.unpack_from("<I", buf, off)
            dims = struct.unpack_from(f"<{nd}Q", buf, off + 4)
            off += 4 + 8 * nd
            gt, toff = struct.unpack_from("<IQ", buf, off)
            off += 12
            infos.append((name, dims, gt, toff))
        align = int(self.metadata.get("general.alignment", GGUF_DEFAULT_ALIGNMENT))
        base = (off + align - 1) // align * align
        self.tensors: Dict[str, GgufTensor] = {}
        for name, dims, gt, toff in infos:
            if gt not in _GGML_BLOCK:
                raise ValueError(f"{name}: ggml type {gt} is not supported (F32, F16, BF16, Q8_0)")
            shape = tuple(int(d) for d in reversed(dims))  # ne[0] is the innermost dimension
            count = int(np.prod(shape)) if shape else 1
            bv, bb = _GGML_BLOCK[gt]
            if count % bv:
                raise ValueError(f"{name}: {count} values is not a whole number of blocks")
            nbytes = count // bv * bb
            start = base + toff
            if start + nbytes > len(buf):
                raise ValueError(f"{name}: data beyond the end of the file")
            if gt == GGML_F32:
                data = np.frombuffer(buf, dtype=np.float32, count=count, offset=start)
            elif gt in (GGML_F16, GGML_BF16):
                data = np.frombuffer(buf, dtype=np.uint16, count=count, offset=start)
            else:
                data = np.frombuffer(buf, dtype=np.uint8, count=nbytes, offset=start)
            self.tensors[name] = GgufTensor(name, gt, shape, data)

    def close(self) -> None:
        self.tensors = {}
        try:
            self._mm.close()
        except BufferError:  # arrays handed out still view the mapping; it ends with the last of them
            pass
        self._f.close()


def _w_str(out: bytearray, s: str) -> None:
    b = s.encode("utf-8")
    out += struct.pack("<Q", len(b)) + b


def _w_value(out: bytearray, v) -> None:
    if isinstance(v, bool):
        out += struct.pack("<I?", GV_BOOL, v)
    elif isinstance(v, int):
        out += struct.pack("<Iq", GV_INT64, v) if v < 0 else struct.pack("<IQ", GV_UINT64, v) \
            if v >= 2 ** 32 else struct.pack("<II", GV_UINT32, v)
    elif isinstance(v, float):
        out += struct.pack("<If", GV_FLOAT32, v)
    elif isinstance(v, str):
        out += struct.pack("<I", GV_STRING)
        _w_str(out, v)
    elif isinstance(v, (list, tuple)):
        if not v or not all(isinstance(e, str) for e in v):
            raise ValueError("only non-empty string arrays are written")
        out += struct.pack("<IIQ", GV_ARRAY, GV_STRING, len(v))
        for e in v:
            _w_str(out, e)
    else:
        raise TypeError(f"metadata value {v!r} has no GGUF type here")


def write_gguf(path: str, metadata: Dict[str, object], tensors: Sequence[GgufTensor],
               alignment: int = GGUF_DEFAULT_ALIGNMENT) -> None:
    """GGUF v3: header, metadata, tensor infos, then each tensor's data at a
    multiple of `alignment` from the aligned start of the data section."""
    md = dict(metadata)
    if alignment != GGUF_DEFAULT_ALIGNMENT:
        md["general.alignment"] = int(alignment)
    head = bytearray()
    head += GGUF_MAGIC + struct.pack("<IQQ", GGUF_VERSION, len(tensors), len(md))
    for k, v in md.items():
        _w_str(head, k)
        _w_value(head, v)
    offsets, off = [], 0
    for t in tensors:
        off = (off + alignment - 1) // alignment * alignment
        offsets.append(off)
        off += t.data.nbytes
    for t, o in zip(tensors, offsets):
        _w_str(head, t.name)
        dims = tuple(reversed(t.shape))
        head += struct.pack("<I", len(dims)) + struct.pack(f"<{len(dims)}Q", *dims)
        head += struct.pack("<IQ", t.ggml_type, o)
    with open(path, "wb") as f:
        f.write(head)
        pos = len(head)
        pad = (-pos) % alignment
        f.write(b"\0" * pad)
        data_start = pos + pad
        for t, o in zip(tensors, offsets):
            cur = f.tell() - data_start
            f.write(b"\0" * (o - cur))
            f.write(np.ascontiguousarray(t.data).tobytes())


def gguf_tensor_names(cfg) -> List[str]:
    """llama.cpp's Qwen3 tensor names in the table order of lq8_model_create."""
    names = ["token_embd.weight", "output_norm.weight"]
    for l in range(cfg.num_hidden_layers):
        b = f"blk.{l}"
        names += [f"{b}.attn_norm.weight", f"{b}.ffn_norm.weight", f"{b}.attn_q_norm.weight",
                  f"{b}.attn_k_norm.weight", f"{b}.attn_q.weight", f"{b}.attn_k.weight", f"{b}.attn_v.weight",
                  f"{b}.attn_output.weight", f"{b}.ffn_gate.weight", f"{b}.ffn_up.weight", f"{b}.ffn_down.weight"]
    return names


def qwen3_gguf_metadata(cfg) -> Dict[str, object]:
    return {
        "general.architecture": "qwen3",
        "general.file_type": 7,  # LLAMA_FTYPE_MOSTLY_Q8_0
        "qwen3.context_length": int(cfg.max_position_embeddings),
        "qwen3.embedding_length": int(cfg.hidden_size),
        "qwen3.block_count": int(cfg.num_hidden_layers),
        "qwen3.feed_forward_length": int(cfg.intermediate_size),
        "qwen3.attention.head_count": int(cfg.num_attention_heads),
        "qwen3.attention.head_count_kv": int(cfg.num_key_value_heads),
        "qwen3.attention.key_length": int(cfg.head_dim),
        "qwen3.attention.value_length": int(cfg.head_dim),
        "qwen3.attention.layer_norm_rms_epsilon": float(cfg.rms_norm_eps),
        "qwen3.rope.freq_base": float(cfg.rope_theta),
    }


def qwen3_config_from_gguf(g: GgufFile, max_positions: Optional[int] = None):
    from . import Qwen3Config

    md = g.metadata
    if md.get("general.architecture") != "qwen3":
        raise ValueError(f"general.architecture is {md.get('general.architecture')!r}, not 'qwen3'")
    emb = g.tensors["token_embd.weight"]
    heads = int(md["qwen3.attention.head_count"])
    H = int(md["qwen3.embedding_length"])
    return Qwen3Config(vocab_size=int(emb.shape[0]), hidden_size=H,
                       intermediate_size=int(md["qwen3.feed_forward_length"]),
                       num_hidden_layers=int(md["qwen3.block_count"]), num_attention_heads=heads,
                       num_key_value_heads=int(md.get("qwen3.attention.head_count_kv", heads)),
                       head_dim=int(md.get("qwen3.attention.key_length", H // heads)),
                       max_position_embeddings=int(max_positions or md.get("qwen3.context_length", 4096)),
                       rms_norm_eps=float(md.get("qwen3.attention.layer_norm_rms_epsilon", 1e-6)),
                       rope_theta=float(md.get("qwen3.rope.freq_base", 1e6)))


def check_shapes(cfg, shapes: Sequence[Tuple[int, ...]], names: Sequence[str]) -> None:
    for i, (shape, name) in enumerate(zip(shapes, names)):
        _, want = cfg.tensor_shape(i)
        if tuple(shape) != tuple(want):
            raise ValueError(f"{name}: shape {tuple(shape)}, expected {tuple(want)}")
