"""The GGUF reader (include/slm_gguf.h) on the CPU: the reference's two
loader tests (loader.rs:706-927) restated, and the format's edge cases
(alignment, bounds, UTF-8, dimensions, repeated keys, the model config)."""
import struct

import numpy as np
import pytest

from gguf_writer import (ARRAY, BOOL, F32, F64, GGML_F32, GGML_Q4_0, I8, I16, I32, I64, STR,
                         U8, U16, U32, U64, GgufWriter, encode_value, gguf_str, write_model)
from oracle import py_oracle as orc
from slm_testlib import load_product

P = load_product()


def test_parse_metadata_and_tensor_views(tmp_path):
    # loader.rs:706-778: metadata round trip, tensors as views of the file,
    # and a GEMV on the mapped weights equal to the one on the originals
    rows, cols = 8, 64
    w_f32 = np.sin(np.arange(rows * cols, dtype=np.float32) * np.float32(0.01))
    norm = np.float32(1.0) + np.arange(cols, dtype=np.float32) * np.float32(0.001)
    x = np.cos(np.arange(cols, dtype=np.float32) * np.float32(0.05))
    w_q4 = orc.quantize_q4_0(w_f32)
    x_q8 = orc.quantize_q8_0(x)
    expected = orc.gemm_q4_0(w_q4, x_q8, 1, rows, cols)
    g = GgufWriter()
    g.add_str("general.architecture", "llama")
    g.add_u32("llama.embedding_length", cols)
    g.add_f32("llama.attention.layer_norm_rms_epsilon", 1e-5)
    g.add_tensor_f32("blk.0.attn_norm.weight", [cols], norm)
    g.add_tensor_q4_0("blk.0.attn_q.weight", [cols, rows], w_q4)
    path = tmp_path / "model.gguf"
    g.write(path)
    with P.GgufFile(path) as f:
        assert f.version == 3
        assert f.get_str("general.architecture") == "llama"
        assert f.get_u32("llama.embedding_length") == cols
        assert f.get_f32("llama.attention.layer_norm_rms_epsilon") == np.float32(1e-5)
        mapped_norm = np.frombuffer(f.tensor_bytes("blk.0.attn_norm.weight", P.GGML_F32),
                                    np.float32)
        np.testing.assert_array_equal(mapped_norm, norm)
        mapped_wq = np.frombuffer(f.tensor_bytes("blk.0.attn_q.weight", P.GGML_Q4_0),
                                  np.uint8).reshape(-1, 18)
        np.testing.assert_array_equal(mapped_wq, w_q4.reshape(-1, 18))
        # views into one mapping: addresses differ exactly by the file offsets
        a_norm, _ = f.tensor_view("blk.0.attn_norm.weight", P.GGML_F32)
        a_wq, _ = f.tensor_view("blk.0.attn_q.weight", P.GGML_Q4_0)
        t_norm = f.tensor_info("blk.0.attn_norm.weight")
        t_wq = f.tensor_info("blk.0.attn_q.weight")
        assert a_wq - a_norm == t_wq.offset - t_norm.offset
        assert (t_wq.dims[0], t_wq.dims[1], t_wq.n_dims) == (cols, rows, 2)
        actual = orc.gemm_q4_0(np.ascontiguousarray(mapped_wq).reshape(-1), x_q8, 1, rows, cols)
        np.testing.assert_array_equal(actual, expected)


def thirteen_types_file() -> bytes:
    """loader.rs:781-886: a v2 file with one value of each type and a tensor
    at data offset 1 (misaligned for f32)."""
    buf = bytearray(b"GGUF" + struct.pack("<IQQ", 2, 1, 13))
    recs = [("k_u8", U8, 42), ("k_i8", I8, -7), ("k_u16", U16, 1024), ("k_i16", I16, -512),
            ("k_u32", U32, 999), ("k_i32", I32, -999), ("k_f32", F32, 3.5), ("k_bool", BOOL, 1),
            ("k_str", STR, "hello")]
    for k, t, v in recs:
        buf += gguf_str(k) + encode_value(t, v)
    buf += gguf_str("k_arr") + encode_value(ARRAY, ["tok0", "tok1"], STR)
    for k, t, v in [("k_u64", U64, 123456), ("k_i64", I64, -123456), ("k_f64", F64, 2.25)]:
        buf += gguf_str(k) + encode_value(t, v)
    buf += gguf_str("misaligned.weight") + struct.pack("<IQIQ", 1, 4, GGML_F32, 1)
    data_off = (len(buf) + 31) // 32 * 32
    buf += bytes(data_off + 32 - len(buf))
    return bytes(buf)


def test_thirteen_value_types_and_error_paths(tmp_path):
    path = tmp_path / "types.gguf"
    path.write_bytes(thirteen_types_file())
    with P.GgufFile(path) as f:
        assert f.version == 2
        expect = {"k_u8": (U8, 42), "k_i8": (I8, -7), "k_u16": (U16, 1024),
                  "k_i16": (I16, -512), "k_i32": (I32, -999), "k_bool": (BOOL, 1),
                  "k_i64": (I64, -123456)}
        for key, (t, v) in expect.items():
            val = f.get(key)
            assert val.type == t and val.i64 == v, key
        assert f.get_u32("k_u32") == 999
        assert f.get_f32("k_f32") == 3.5
        assert f.get_str("k_str") == "hello"
        assert f.get_usize("k_u64") == 123456
        assert f.get_f32("k_f64") == 2.25
        arr = f.get("k_arr")
        assert (arr.type, arr.elem_type, arr.len) == (ARRAY, STR, 2)
        with pytest.raises(P.SlmAttnError) as ei:
            f.tensor_view("misaligned.weight", P.GGML_F32)
        assert ei.value.code == P.ERR_UNALIGNED
        with pytest.raises(P.SlmAttnError) as ei:
            f.tensor_view("misaligned.weight", P.GGML_Q4_0)
        assert ei.value.code == P.ERR_TYPE
        with pytest.raises(P.SlmAttnError) as ei:
            f.tensor_view("nonexistent.weight", P.GGML_F32)
        assert ei.value.code == P.ERR_NOT_FOUND
    cases = [(b"BAD!0000", P.ERR_MAGIC), (b"GGUF" + struct.pack("<I", 99), P.ERR_VERSION),
             (b"GGUF", P.ERR_EOF)]
    for raw, code in cases:
        path.write_bytes(raw)
        with pytest.raises(P.SlmAttnError) as ei:
            P.GgufFile(path)
        assert ei.value.code == code, raw


def test_missing_file_is_an_io_error(tmp_path):
    with pytest.raises(P.SlmAttnError) as ei:
        P.GgufFile(tmp_path / "absent.gguf")
    assert ei.value.code == P.ERR_IO


def header(n_tensors, n_kv, version=3):
    return b"GGUF" + struct.pack("<IQQ", version, n_tensors, n_kv)


@pytest.mark.parametrize("raw,code", [
    (header(0, 1) + gguf_str(b"\xff\xfe") + encode_value(U32, 1), "ERR_UTF8"),
    (header(0, 1) + gguf_str("k") + encode_value(STR, b"a\xc0\x80"), "ERR_UTF8"),  # overlong
    (header(0, 1) + gguf_str("k") + struct.pack("<I", 13) + b"\0" * 8, "ERR_VALUE_TYPE"),
    (header(1, 0) + gguf_str("t") + struct.pack("<I", 0), "ERR_DIMS"),
    (header(1, 0) + gguf_str("t") + struct.pack("<I", 5), "ERR_DIMS"),
    (header(0, 1) + gguf_str("k") + encode_value(ARRAY, [1, 2, 3], U32)[:-2], "ERR_EOF"),
])
def test_malformed_files(tmp_path, raw, code):
    path = tmp_path / "bad.gguf"
    path.write_bytes(raw)
    with pytest.raises(P.SlmAttnError) as ei:
        P.GgufFile(path)
    assert ei.value.code == getattr(P, code)


def test_alignment_bounds_and_repeated_keys(tmp_path):
    g = GgufWriter(alignment=64)
    g.add("general.alignment", U32, 64)
    g.add_u32("dup", 1)
    g.add_u32("dup", 2)
    g.add_tensor_f32("a", [3], np.arange(3, dtype=np.float32))
    g.add_tensor_f32("b", [5], np.arange(5, dtype=np.float32) + np.float32(10))
    raw = g.to_bytes()
    path = tmp_path / "al.gguf"
    path.write_bytes(raw)
    with P.GgufFile(path) as f:
        assert f.alignment == 64 and f.data_offset % 64 == 0
        assert f.get_u32("dup") == 2  # the last value wins
        assert f.tensor_info("b").offset == 64
        np.testing.assert_array_equal(np.frombuffer(f.tensor_bytes("b", P.GGML_F32), np.float32),
                                      np.arange(5, dtype=np.float32) + np.float32(10))
    # the last tensor cut short: OutOfBounds on its view, the rest still opens
    path.write_bytes(raw[:-4])
    with P.GgufFile(path) as f:
        with pytest.raises(P.SlmAttnError) as ei:
            f.tensor_view("b", P.GGML_F32)
        assert ei.value.code == P.ERR_BOUNDS
        assert f.tensor_bytes("a", P.GGML_F32)


def test_model_config_from_metadata(tmp_path):
    g = GgufWriter()
    g.add_str("general.architecture", "qwen2")
    g.add_u32("qwen2.block_count", 24)
    g.add("qwen2.embedding_length", U64, 896)
    g.add("qwen2.feed_forward_length", I32, 4864)
    g.add_u32("qwen2.attention.head_count", 14)
    g.add_u32("qwen2.attention.head_count_kv", 2)
    g.add_u32("qwen2.context_length", 32768)
    g.add("qwen2.attention.layer_norm_rms_epsilon", F64, 1e-6)
    g.add_f32("qwen2.rope.freq_base", 1e6)
    path = tmp_path / "cfg.gguf"
    g.write(path)
    with P.GgufFile(path) as f:
        c = f.model_config()
    assert c == {"dim": 896, "hidden_dim": 4864, "num_heads": 14, "num_kv_heads": 2,
                 "max_seq_len": 32768, "num_layers": 24, "rms_eps": np.float32(1e-6),
                 "rope_theta": 1e6}
    # main.rs's defaults when the keys are absent; theta the reference's 10000
    path.write_bytes(GgufWriter().to_bytes())
    with P.GgufFile(path) as f:
        c = f.model_config()
    assert c == {"dim": 256, "hidden_dim": 768, "num_heads": 8, "num_kv_heads": 8,
                 "max_seq_len": 64, "num_layers": 2, "rms_eps": np.float32(1e-5),
                 "rope_theta": 10000.0}


def _ref_model_meta():
    from test_oracle_layer import ref_model
    cfg, w = ref_model()
    meta = dict(dim=cfg.dim, hidden_dim=128, num_heads=cfg.num_heads,
                num_kv_heads=cfg.num_kv_heads, max_seq_len=cfg.max_seq_len,
                num_layers=cfg.num_layers, rms_eps=1e-5)
    return cfg, w, meta


@pytest.mark.parametrize("which", ["attn_norm", "ffn_norm", "output_norm"])
def test_model_load_rejects_short_norm_before_upload(tmp_path, which):
    # The norm kernels read dim floats from a bare device pointer; the
    # reference asserts weights.len() == dst.len (engine.rs:199).  A cut-down
    # norm tensor is refused with SLM_ERR_SHAPE while every tensor is checked,
    # before any device allocation, copy or launch (this runs without a GPU).
    import dataclasses
    cfg, w, meta = _ref_model_meta()
    short = np.ones(cfg.dim - 32, np.float32)
    if which == "output_norm":
        w = dataclasses.replace(w, output_norm=short)
    else:
        key = "rms_att" if which == "attn_norm" else "rms_ffn"
        w = dataclasses.replace(w, layers=[dataclasses.replace(w.layers[0], **{key: short}),
                                           w.layers[1]])
    path = tmp_path / "short_norm.gguf"
    write_model(path, meta, w)
    with P.GgufFile(path) as f:
        with pytest.raises(P.SlmAttnError) as ei:
            P.GgufModel(f, meta["num_layers"])
    assert ei.value.code == P.ERR_SHAPE
    assert "dimension" in str(ei.value)


def test_model_load_missing_tensor_and_wrong_type_before_upload(tmp_path):
    # a missing layer and a tensor of the wrong type are found by the check
    # pass before anything is uploaded (runs without a GPU)
    cfg, w, meta = _ref_model_meta()
    path = tmp_path / "model.gguf"
    write_model(path, meta, w)
    with P.GgufFile(path) as f:
        with pytest.raises(P.SlmAttnError) as ei:   # asks for a third layer
            P.GgufModel(f, 3)
        assert ei.value.code == P.ERR_NOT_FOUND
    g = GgufWriter()
    g.add_tensor_f32("token_embd.weight", [cfg.dim, 4], np.zeros(4 * cfg.dim, np.float32))
    path2 = tmp_path / "f32_embd.gguf"
    g.write(path2)
    with P.GgufFile(path2) as f:
        with pytest.raises(P.SlmAttnError) as ei:
            P.GgufModel(f, 1)
        assert ei.value.code == P.ERR_TYPE


@pytest.mark.parametrize("first,code", [("attn_q", "ERR_NOT_FOUND"),
                                        ("attn_norm", "ERR_TYPE")])
def test_model_load_reports_the_first_fault_in_the_reference_order(tmp_path, first, code):
    # Two faults in layer 1: attn_q missing and a norm of the wrong type.
    # layer_weights resolves attn_norm, attn_q, attn_k, attn_v, attn_output,
    # ffn_norm, gate, up, down in that order (loader.rs:508-520), so the error
    # is the first fault met: with ffn_norm mistyped, TensorNotFound for
    # attn_q; with attn_norm mistyped, TypeMismatch.
    cfg, w, meta = _ref_model_meta()
    bad_norm = "ffn_norm" if first == "attn_q" else "attn_norm"

    def edit(g):
        keep = []
        for name, gtype, dims, raw in g.tensors:
            if name == "blk.1.attn_q.weight":
                continue
            if name == f"blk.1.{bad_norm}.weight":
                blocks = orc.quantize_q4_0(np.ones(cfg.dim, np.float32))
                gtype, raw = GGML_Q4_0, blocks.tobytes()
            keep.append((name, gtype, dims, raw))
        g.tensors = keep

    path = tmp_path / "two_faults.gguf"
    write_model(path, meta, w, edit=edit)
    with P.GgufFile(path) as f:
        with pytest.raises(P.SlmAttnError) as ei:
            P.GgufModel(f, meta["num_layers"])
    assert ei.value.code == getattr(P, code), (ei.value.code, str(ei.value))
