"""A small GGUF v2/v3 writer for the tests (test infrastructure): metadata of
any of the thirteen value types and F32 / Q4_0 tensors, laid out as the GGUF
format specifies (little-endian header, key/value records, tensor
directory, data section at the alignment)."""
from __future__ import annotations

import struct

import numpy as np

MAGIC = b"GGUF"
U8, I8, U16, I16, U32, I32, F32, BOOL, STR, ARRAY, U64, I64, F64 = range(13)
GGML_F32, GGML_F16, GGML_Q4_0, GGML_Q8_0 = 0, 1, 2, 8
_FMT = {U8: "<B", I8: "<b", U16: "<H", I16: "<h", U32: "<I", I32: "<i", F32: "<f",
        BOOL: "<B", U64: "<Q", I64: "<q", F64: "<d"}


def gguf_str(s: str | bytes) -> bytes:
    b = s.encode() if isinstance(s, str) else s
    return struct.pack("<Q", len(b)) + b


def encode_value(vtype: int, value, elem_type: int | None = None) -> bytes:
    """A value record body (type code, then payload)."""
    out = struct.pack("<I", vtype)
    if vtype == STR:
        return out + gguf_str(value)
    if vtype == ARRAY:
        out += struct.pack("<IQ", elem_type, len(value))
        for v in value:
            out += gguf_str(v) if elem_type == STR else struct.pack(_FMT[elem_type], v)
        return out
    return out + struct.pack(_FMT[vtype], value)


class GgufWriter:
    def __init__(self, version: int = 3, alignment: int = 32):
        self.version = version
        self.alignment = alignment
        self.kv: list[tuple[str, bytes]] = []
        self.tensors: list[tuple[str, int, list[int], bytes]] = []

    def add(self, key: str, vtype: int, value, elem_type: int | None = None):
        self.kv.append((key, encode_value(vtype, value, elem_type)))

    def add_u32(self, key, v):
        self.add(key, U32, v)

    def add_f32(self, key, v):
        self.add(key, F32, v)

    def add_str(self, key, v):
        self.add(key, STR, v)

    def add_tensor_f32(self, name: str, dims: list[int], data: np.ndarray):
        self.tensors.append((name, GGML_F32, list(dims),
                             np.ascontiguousarray(data, dtype=np.float32).tobytes()))

    def add_tensor_q4_0(self, name: str, dims: list[int], blocks: np.ndarray):
        self.tensors.append((name, GGML_Q4_0, list(dims),
                             np.ascontiguousarray(blocks, dtype=np.uint8).tobytes()))

    def to_bytes(self) -> bytes:
        a = self.alignment
        buf = bytearray(MAGIC + struct.pack("<IQQ", self.version, len(self.tensors), len(self.kv)))
        for key, rec in self.kv:
            buf += gguf_str(key) + rec
        rel, offsets = 0, []
        for name, gtype, dims, raw in self.tensors:
            rel = (rel + a - 1) // a * a
            offsets.append(rel)
            buf += gguf_str(name) + struct.pack("<I", len(dims))
            buf += b"".join(struct.pack("<Q", d) for d in dims)
            buf += struct.pack("<IQ", gtype, rel)
            rel += len(raw)
        data_off = (len(buf) + a - 1) // a * a
        buf += bytes(data_off - len(buf))
        for (_, _, _, raw), off in zip(self.tensors, offsets):
            buf += bytes(data_off + off - len(buf))
            buf += raw
        return bytes(buf)

    def write(self, path) -> None:
        with open(path, "wb") as f:
            f.write(self.to_bytes())


def write_model(path, cfg: dict, w, tied: bool = False, arch: str = "llama",
                rope_theta: float | None = None, edit=None) -> None:
    """A whole model in the reference's tensor names (loader.rs:508-552) and
    metadata keys (main.rs:36-46); w is an oracle ModelWeights.  edit, when
    given, may change the writer (its tensor list) before the file is written."""
    g = GgufWriter()
    g.add_str("general.architecture", arch)
    g.add_u32(f"{arch}.block_count", cfg["num_layers"])
    g.add_u32(f"{arch}.embedding_length", cfg["dim"])
    g.add_u32(f"{arch}.feed_forward_length", cfg["hidden_dim"])
    g.add_u32(f"{arch}.attention.head_count", cfg["num_heads"])
    g.add_u32(f"{arch}.attention.head_count_kv", cfg["num_kv_heads"])
    g.add_u32(f"{arch}.rope.dimension_count", cfg["dim"] // cfg["num_heads"])
    g.add_u32(f"{arch}.context_length", cfg["max_seq_len"])
    g.add_f32(f"{arch}.attention.layer_norm_rms_epsilon", cfg["rms_eps"])
    if rope_theta is not None:
        g.add_f32(f"{arch}.rope.freq_base", rope_theta)
    dim, vocab = cfg["dim"], w.vocab_size
    g.add_tensor_q4_0("token_embd.weight", [dim, vocab], w.token_embd)
    for l, lw in enumerate(w.layers):
        p = f"blk.{l}."
        h = lw.hidden_dim
        kvd = lw.wk.size // 18 * 32 // dim
        g.add_tensor_f32(p + "attn_norm.weight", [len(lw.rms_att)], lw.rms_att)
        g.add_tensor_q4_0(p + "attn_q.weight", [dim, dim], lw.wq)
        g.add_tensor_q4_0(p + "attn_k.weight", [dim, kvd], lw.wk)
        g.add_tensor_q4_0(p + "attn_v.weight", [dim, kvd], lw.wv)
        g.add_tensor_q4_0(p + "attn_output.weight", [dim, dim], lw.wo)
        g.add_tensor_f32(p + "ffn_norm.weight", [len(lw.rms_ffn)], lw.rms_ffn)
        g.add_tensor_q4_0(p + "ffn_gate.weight", [dim, h], lw.w_gate)
        g.add_tensor_q4_0(p + "ffn_up.weight", [dim, h], lw.w_up)
        g.add_tensor_q4_0(p + "ffn_down.weight", [h, dim], lw.w_down)
    g.add_tensor_f32("output_norm.weight", [len(w.output_norm)], w.output_norm)
    if not tied:
        g.add_tensor_q4_0("output.weight", [dim, vocab], w.lm_head)
    if edit is not None:
        edit(g)
    g.write(path)
