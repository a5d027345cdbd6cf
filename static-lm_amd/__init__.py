"""static-lm attention hot path on MI355X (gfx950): Python binding of the
slm_attn C ABI (include/slm_attn.h).

The compute lives in libslm_attn.so (hand-written HIP kernels); this module
only marshals buffers through ctypes.  Nothing here computes attention on the
CPU: if the library is missing, loading it raises.

Names follow the reference (src/model/transformer.rs of static-lm):
``TransformerConfig`` mirrors transformer.rs:8-33 and ``AttentionContext``
exposes the attention block of ``TransformerLayer::forward_token_with_kv``
(transformer.rs:413-443) as ``decode`` and of ``forward_batch_with_kv``
(transformer.rs:530-593) as ``prefill``.
"""
from __future__ import annotations

import ctypes
import os
import sys
import weakref
from dataclasses import dataclass
from pathlib import Path

import numpy as np

PKG_DIR = Path(__file__).resolve().parent
LIB_PATH = PKG_DIR / "libslm_attn.so"
HEADER_PATH = PKG_DIR.parent / "include" / "slm_attn.h"
CALIB_HEADER_PATH = PKG_DIR / "calib" / "slm_calib.h"
CALIB_LIB_PATH = PKG_DIR / "calib" / "libslm_calib.so"
QUANT_HEADER_PATH = PKG_DIR.parent / "include" / "slm_quant.h"
LAYER_HEADER_PATH = PKG_DIR.parent / "include" / "slm_layer.h"
GGUF_HEADER_PATH = PKG_DIR.parent / "include" / "slm_gguf.h"

SLM_OK = 0
ERRORS = {
    -1: "SLM_ERR_CONFIG",
    -2: "SLM_ERR_POS",
    -3: "SLM_ERR_BATCH",
    -4: "SLM_ERR_LAYER",
    -5: "SLM_ERR_ALIAS",
    -6: "SLM_ERR_ARG",
    -7: "SLM_ERR_HIP",
    -8: "SLM_ERR_UNSUPPORTED",
    -9: "SLM_ERR_DEVICE",
    -10: "SLM_ERR_SHAPE",
    -11: "SLM_ERR_TOKEN",
    -12: "SLM_ERR_IO",
    -13: "SLM_ERR_EOF",
    -14: "SLM_ERR_MAGIC",
    -15: "SLM_ERR_VERSION",
    -16: "SLM_ERR_UTF8",
    -17: "SLM_ERR_VALUE_TYPE",
    -18: "SLM_ERR_DIMS",
    -19: "SLM_ERR_NOT_FOUND",
    -20: "SLM_ERR_TYPE",
    -21: "SLM_ERR_BOUNDS",
    -22: "SLM_ERR_UNALIGNED",
    -23: "SLM_ERR_CAPTURE",
}
(ERR_CONFIG, ERR_POS, ERR_BATCH, ERR_LAYER, ERR_ALIAS, ERR_ARG, ERR_HIP, ERR_UNSUPPORTED,
 ERR_DEVICE, ERR_SHAPE, ERR_TOKEN) = (-1, -2, -3, -4, -5, -6, -7, -8, -9, -10, -11)
(ERR_IO, ERR_EOF, ERR_MAGIC, ERR_VERSION, ERR_UTF8, ERR_VALUE_TYPE, ERR_DIMS, ERR_NOT_FOUND,
 ERR_TYPE, ERR_BOUNDS, ERR_UNALIGNED) = tuple(range(-12, -23, -1))
ERR_CAPTURE = -23
GGML_F32, GGML_F16, GGML_Q4_0, GGML_Q8_0 = 0, 1, 2, 8

KERNEL_KINDS = ("append", "decode", "combine", "prefill", "rope", "quant", "gemm", "norm",
                "elem")
# prefill kernels, numbered as SLM_PF_* (slm_attn_prefill_kernel)
PREFILL_KERNELS = ("four_heads", "three_heads", "two_heads", "one_head", "key_split",
                   "paired_four_heads", "dma", "dma_paired", "paired_two_heads",
                   "paired_one_head")


class SlmAttnError(RuntimeError):
    """A nonzero slm_attn return code; the reference would have panicked."""

    def __init__(self, code: int, message: str):
        super().__init__(f"{ERRORS.get(code, code)}: {message}")
        self.code = code
        self.message = message


@dataclass(frozen=True)
class TransformerConfig:
    """transformer.rs:8-33 (hidden_dim and rms_eps are unused by attention)."""

    dim: int
    hidden_dim: int
    num_heads: int
    num_kv_heads: int
    max_seq_len: int
    rms_eps: float = 1e-5

    def head_dim(self) -> int:
        return self.dim // self.num_heads

    def kv_dim(self) -> int:
        return (self.dim // self.num_heads) * self.num_kv_heads

    def kv_mul(self) -> int:
        return self.num_heads // self.num_kv_heads


class _Config(ctypes.Structure):
    _fields_ = [
        ("dim", ctypes.c_int32),
        ("num_heads", ctypes.c_int32),
        ("num_kv_heads", ctypes.c_int32),
        ("max_seq_len", ctypes.c_int32),
        ("num_layers", ctypes.c_int32),
        ("rope_theta", ctypes.c_float),
    ]


class _KernelStat(ctypes.Structure):
    _fields_ = [("launches", ctypes.c_int64), ("total_ms", ctypes.c_double)]


_F = ctypes.POINTER(ctypes.c_float)
_P = ctypes.c_void_p
_I = ctypes.c_int32

# name -> (restype, argtypes); every function the header declares
SIGNATURES = {
    "slm_attn_create": (ctypes.c_int, [ctypes.POINTER(_Config), ctypes.POINTER(_P)]),
    "slm_attn_destroy": (None, [_P]),
    "slm_attn_last_error": (ctypes.c_char_p, [_P]),
    "slm_attn_decode": (ctypes.c_int, [_P, _I, _I, _F, _F, _F, _F]),
    "slm_attn_prefill": (ctypes.c_int, [_P, _I, _I, _I, _F, _F, _F, _F]),
    "slm_attn_decode_dev": (ctypes.c_int, [_P, _I, _I, _P, _P, _P, _P]),
    "slm_attn_prefill_dev": (ctypes.c_int, [_P, _I, _I, _I, _P, _P, _P, _P]),
    "slm_rope_apply_dev": (ctypes.c_int, [_P, _P, _I, _I, _I]),
    "slm_kv_append_dev": (ctypes.c_int, [_P, _I, _I, _I, _P, _P]),
    "slm_attn_attend_dev": (ctypes.c_int, [_P, _I, _I, _P, _P]),
    "slm_attn_attend_batch_dev": (ctypes.c_int, [_P, _I, _I, _I, _P, _P]),
    "slm_attn_set_stream": (ctypes.c_int, [_P, _P]),
    "slm_attn_get_stream": (_P, [_P]),
    "slm_attn_sync": (ctypes.c_int, [_P]),
    "slm_attn_capture_begin": (ctypes.c_int, [_P]),
    "slm_attn_capture_end": (ctypes.c_int, [_P, ctypes.POINTER(_P)]),
    "slm_attn_graph_launch": (ctypes.c_int, [_P, _P]),
    "slm_attn_graph_destroy": (None, [_P]),
    "slm_kv_write": (ctypes.c_int, [_P, _I, _I, _I, _I, _F]),
    "slm_kv_read": (ctypes.c_int, [_P, _I, _I, _I, _I, _F]),
    "slm_kv_write_dev": (ctypes.c_int, [_P, _I, _I, _I, _I, _P]),
    "slm_kv_offset": (ctypes.c_size_t, [_P, _I, _I, _I]),
    "slm_kv_device_ptr": (_P, [_P]),
    "slm_rope_tables_read": (ctypes.c_int, [_P, _F, _F]),
    "slm_attn_profile": (ctypes.c_int, [_P, _I]),
    "slm_attn_profile_read": (ctypes.c_int, [_P, ctypes.POINTER(_KernelStat)]),
    "slm_attn_decode_splits": (ctypes.c_int, [_P, _I, ctypes.POINTER(_I), ctypes.POINTER(_I)]),
    "slm_attn_prefill_kernel": (ctypes.c_int, [_P, _I, _I, ctypes.POINTER(_I)]),
    "slm_attn_version": (ctypes.c_char_p, []),
    # slm_quant.h
    "slm_q4_matrix_create": (ctypes.c_int, [_I, ctypes.c_void_p, _I, _I, ctypes.POINTER(_P)]),
    "slm_q4_matrix_destroy": (None, [_P]),
    "slm_q4_matrix_shape": (ctypes.c_int, [_P, ctypes.POINTER(_I), ctypes.POINTER(_I)]),
    "slm_quantize_q8_0_dev": (ctypes.c_int, [_P, _P, ctypes.c_int64, _P]),
    "slm_gemm_q4_0_dev": (ctypes.c_int, [_P, _P, _P, _I, _P]),
    "slm_attn_decode_xb_dev": (ctypes.c_int, [_P, _I, _I, _P, _P, _P, _P, _P]),
    "slm_attn_decode_xb_dev_noalloc": (ctypes.c_int, [_P, _I, _I, _P, _P, _P, _P, _P]),
    "slm_attn_prefill_xb_dev": (ctypes.c_int, [_P, _I, _I, _I, _P, _P, _P, _P, _P]),
    "slm_gemm_q4_0_residual_dev": (ctypes.c_int, [_P, _P, _P, _I, _P, _P]),
    "slm_attn_decode_wo_dev": (ctypes.c_int, [_P, _I, _I, _P, _P, _P, _P, _P, _P, _P]),
    "slm_attn_prefill_wo_dev": (ctypes.c_int, [_P, _I, _I, _I, _P, _P, _P, _P, _P, _P, _P]),
    "slm_rmsnorm_dev": (ctypes.c_int, [_P, _P, _P, _I, _I, ctypes.c_float, _P]),
    "slm_l2_norm_dev": (ctypes.c_int, [_P, _P, _I, _I, ctypes.c_float, _P]),
    "slm_swiglu_dev": (ctypes.c_int, [_P, _P, _P, ctypes.c_int64, _P]),
    "slm_residual_add_dev": (ctypes.c_int, [_P, _P, _P, ctypes.c_int64, _P]),
    "slm_layer_forward_dev": (ctypes.c_int, [_P, _I, _I, _I, _P, ctypes.c_float, _P]),
    "slm_model_forward_token_dev": (ctypes.c_int, [_P, _P, ctypes.c_float, _I, _I, _P, _P]),
    "slm_model_prefill_dev": (ctypes.c_int, [_P, _P, ctypes.c_float, _P, _I, _I, _P, _P]),
    "slm_model_generate_dev": (ctypes.c_int, [_P, _P, ctypes.c_float, _P, _I, _P, _I, _I, _P]),
    "slm_model_embed_dev": (ctypes.c_int, [_P, _P, ctypes.c_float, _P, _I, _P]),
    "slm_gguf_open": (ctypes.c_int, [ctypes.c_char_p, _P]),
    "slm_gguf_close": (None, [_P]),
    "slm_gguf_version": (ctypes.c_int32, [_P]),
    "slm_gguf_alignment": (ctypes.c_int64, [_P]),
    "slm_gguf_data_offset": (ctypes.c_int64, [_P]),
    "slm_gguf_tensor_count": (ctypes.c_int64, [_P]),
    "slm_gguf_kv_count": (ctypes.c_int64, [_P]),
    "slm_gguf_get": (ctypes.c_int, [_P, ctypes.c_char_p, _P]),
    "slm_gguf_get_u32": (ctypes.c_int, [_P, ctypes.c_char_p, _P]),
    "slm_gguf_get_usize": (ctypes.c_int, [_P, ctypes.c_char_p, _P]),
    "slm_gguf_get_f32": (ctypes.c_int, [_P, ctypes.c_char_p, _P]),
    "slm_gguf_get_str": (ctypes.c_int, [_P, ctypes.c_char_p, _P, _P]),
    "slm_gguf_tensor_info": (ctypes.c_int, [_P, ctypes.c_char_p, _P]),
    "slm_gguf_tensor_data": (ctypes.c_int, [_P, ctypes.c_char_p, _I, _P, _P]),
    "slm_gguf_model_config": (ctypes.c_int, [_P, _P]),
    "slm_model_load_gguf": (ctypes.c_int, [_P, _I, _I, _P]),
    "slm_model_destroy": (None, [_P]),
    "slm_model_weights_view": (_P, [_P]),
    "slm_model_vocab_size": (ctypes.c_int32, [_P]),
}


class GgufValueC(ctypes.Structure):
    """slm_gguf_value (include/slm_gguf.h)."""
    _fields_ = [("type", ctypes.c_int32), ("i64", ctypes.c_int64), ("u64", ctypes.c_uint64),
                ("f64", ctypes.c_double), ("str", ctypes.c_void_p), ("str_len", ctypes.c_uint64),
                ("elem_type", ctypes.c_int32), ("len", ctypes.c_uint64),
                ("byte_offset", ctypes.c_uint64), ("byte_len", ctypes.c_uint64)]


class GgufTensorC(ctypes.Structure):
    """slm_gguf_tensor (include/slm_gguf.h)."""
    _fields_ = [("ggml_type", ctypes.c_int32), ("n_dims", ctypes.c_int32),
                ("dims", ctypes.c_uint64 * 4), ("offset", ctypes.c_uint64),
                ("n_elements", ctypes.c_uint64)]


class ModelConfigC(ctypes.Structure):
    """slm_model_config (include/slm_gguf.h)."""
    _fields_ = [("dim", ctypes.c_int32), ("hidden_dim", ctypes.c_int32),
                ("num_heads", ctypes.c_int32), ("num_kv_heads", ctypes.c_int32),
                ("max_seq_len", ctypes.c_int32), ("num_layers", ctypes.c_int32),
                ("rms_eps", ctypes.c_float), ("rope_theta", ctypes.c_float)]


class LayerWeightsC(ctypes.Structure):
    """slm_layer_weights (include/slm_layer.h)."""
    _fields_ = [("rms_att", _P), ("wq", _P), ("wk", _P), ("wv", _P), ("wo", _P),
                ("rms_ffn", _P), ("w_gate", _P), ("w_up", _P), ("w_down", _P)]


class ModelWeightsC(ctypes.Structure):
    """slm_model_weights (include/slm_layer.h)."""
    _fields_ = [("token_embd", _P), ("layers", ctypes.POINTER(LayerWeightsC)),
                ("num_layers", ctypes.c_int32), ("output_norm", _P), ("lm_head", _P)]

_lib = None


def _share_torch_hip_runtime() -> None:
    """Maps PyTorch's bundled HIP runtime before ours, when torch is installed.

    torch ships its own libamdhip64 (SONAME libamdhip64.so.7) and its
    libc10_hip asks for it as "libamdhip64.so".  If this library were loaded
    first, the system runtime would be mapped under the SONAME and torch would
    later map a second HIP runtime that finds no GPU.  Mapping torch's copy
    first makes our DT_NEEDED libamdhip64.so.7 resolve to it, so the process
    has one runtime in either import order.  SLM_ATTN_SYSTEM_HIP=1 skips this.
    """
    if os.environ.get("SLM_ATTN_SYSTEM_HIP") == "1" or "torch" in sys.modules:
        return
    import importlib.util

    spec = importlib.util.find_spec("torch")
    if spec is None or not spec.submodule_search_locations:
        return
    hip = Path(spec.submodule_search_locations[0]) / "lib" / "libamdhip64.so"
    if hip.exists():
        ctypes.CDLL(str(hip), mode=ctypes.RTLD_GLOBAL)


def load_library(path: os.PathLike | str | None = None) -> ctypes.CDLL:
    """Loads libslm_attn.so; raises if it has not been built."""
    global _lib
    if _lib is not None and path is None:
        return _lib
    p = Path(path) if path is not None else LIB_PATH
    if not p.exists():
        raise FileNotFoundError(
            f"{p} is missing: build the HIP library first "
            "(python static-lm_amd/build.py or __graft_entry__.build())")
    _share_torch_hip_runtime()
    lib = ctypes.CDLL(str(p))
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    if path is None:
        _lib = lib
    return lib


def _fptr(a: np.ndarray):
    return a.ctypes.data_as(_F)


def _f32(a, shape=None) -> np.ndarray:
    arr = np.ascontiguousarray(a, dtype=np.float32)
    if shape is not None and arr.size != int(np.prod(shape)):
        raise ValueError(f"expected {shape} floats, got {arr.shape}")
    return arr


class AttentionContext:
    """One slm_attn context: device KV region [L][K|V][msl][kv_dim] f32 plus
    RoPE tables, like the KV part of TransformerModel (transformer.rs:714-743)."""

    def __init__(self, dim: int, num_heads: int, num_kv_heads: int, max_seq_len: int,
                 num_layers: int = 1, rope_theta: float = 10000.0):
        self.lib = load_library()
        self.cfg = TransformerConfig(dim, dim, num_heads, num_kv_heads, max_seq_len)
        self.num_layers = num_layers
        self.rope_theta = rope_theta
        c = _Config(dim, num_heads, num_kv_heads, max_seq_len, num_layers, rope_theta)
        h = _P()
        rc = self.lib.slm_attn_create(ctypes.byref(c), ctypes.byref(h))
        if rc != SLM_OK:
            raise SlmAttnError(rc, self.lib.slm_attn_last_error(None).decode())
        self._h = h
        self._graphs = weakref.WeakSet()  # live recordings, closed before the context

    # -- lifetime -------------------------------------------------------------
    def close(self) -> None:
        if getattr(self, "_h", None):
            for g in list(getattr(self, "_graphs", ())):
                g.close()
            self.lib.slm_attn_destroy(self._h)
            self._h = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def _check(self, rc: int) -> None:
        if rc != SLM_OK:
            raise SlmAttnError(rc, self.lib.slm_attn_last_error(self._h).decode())

    @property
    def handle(self):
        return self._h

    # -- host-pointer attention block -------------------------------------------
    def decode(self, layer: int, pos: int, q, k, v) -> np.ndarray:
        cfg = self.cfg
        q = _f32(q, (cfg.dim,))
        k = _f32(k, (cfg.kv_dim(),))
        v = _f32(v, (cfg.kv_dim(),))
        out = np.empty(cfg.dim, np.float32)
        self._check(self.lib.slm_attn_decode(self._h, layer, pos, _fptr(q), _fptr(k), _fptr(v),
                                             _fptr(out)))
        return out

    def prefill(self, layer: int, start: int, q, k, v) -> np.ndarray:
        cfg = self.cfg
        q = np.ascontiguousarray(q, dtype=np.float32).reshape(-1, cfg.dim)
        n = q.shape[0]
        k = _f32(k, (n, cfg.kv_dim()))
        v = _f32(v, (n, cfg.kv_dim()))
        out = np.empty((n, cfg.dim), np.float32)
        self._check(self.lib.slm_attn_prefill(self._h, layer, start, n, _fptr(q), _fptr(k),
                                              _fptr(v), _fptr(out)))
        return out

    # -- device-pointer entry points (addresses as ints) ------------------------
    def decode_dev(self, layer, pos, q, k, v, out):
        self._check(self.lib.slm_attn_decode_dev(self._h, layer, pos, q, k, v, out))

    def prefill_dev(self, layer, start, n, q, k, v, out):
        self._check(self.lib.slm_attn_prefill_dev(self._h, layer, start, n, q, k, v, out))

    def attend_dev(self, layer, pos, q_rot, out):
        self._check(self.lib.slm_attn_attend_dev(self._h, layer, pos, q_rot, out))

    def attend_batch_dev(self, layer, start, n, q_rot, out):
        self._check(self.lib.slm_attn_attend_batch_dev(self._h, layer, start, n, q_rot, out))

    def rope_apply_dev(self, x, n, row_len, pos0):
        self._check(self.lib.slm_rope_apply_dev(self._h, x, n, row_len, pos0))

    def kv_append_dev(self, layer, pos0, n, k, v):
        self._check(self.lib.slm_kv_append_dev(self._h, layer, pos0, n, k, v))

    # -- quantized projections (slm_quant.h) -------------------------------------
    def quantize_q8_0_dev(self, x, n: int, blocks) -> None:
        self._check(self.lib.slm_quantize_q8_0_dev(self._h, x, n, blocks))

    def gemm_q4_0_dev(self, w: "Q4Matrix", x, batch: int, out) -> None:
        self._check(self.lib.slm_gemm_q4_0_dev(self._h, w.handle, x, batch, out))

    def decode_xb_dev(self, layer, pos, xb, wq: "Q4Matrix", wk: "Q4Matrix", wv: "Q4Matrix",
                      out) -> None:
        self._check(self.lib.slm_attn_decode_xb_dev(self._h, layer, pos, xb, wq.handle,
                                                    wk.handle, wv.handle, out))

    def decode_xb_dev_noalloc(self, layer, pos, xb, wq: "Q4Matrix", wk: "Q4Matrix",
                              wv: "Q4Matrix", out) -> None:
        self._check(self.lib.slm_attn_decode_xb_dev_noalloc(self._h, layer, pos, xb, wq.handle,
                                                            wk.handle, wv.handle, out))

    def prefill_xb_dev(self, layer, start, n, xb, wq: "Q4Matrix", wk: "Q4Matrix",
                       wv: "Q4Matrix", out) -> None:
        self._check(self.lib.slm_attn_prefill_xb_dev(self._h, layer, start, n, xb, wq.handle,
                                                     wk.handle, wv.handle, out))

    def gemm_q4_0_residual_dev(self, w: "Q4Matrix", x, batch: int, res, out) -> None:
        self._check(self.lib.slm_gemm_q4_0_residual_dev(self._h, w.handle, x, batch, res, out))

    def decode_wo_dev(self, layer, pos, xb, wq: "Q4Matrix", wk: "Q4Matrix", wv: "Q4Matrix",
                      wo: "Q4Matrix", x, x_mid) -> None:
        self._check(self.lib.slm_attn_decode_wo_dev(self._h, layer, pos, xb, wq.handle,
                                                    wk.handle, wv.handle, wo.handle, x, x_mid))

    def prefill_wo_dev(self, layer, start, n, xb, wq: "Q4Matrix", wk: "Q4Matrix",
                       wv: "Q4Matrix", wo: "Q4Matrix", x, x_mid) -> None:
        self._check(self.lib.slm_attn_prefill_wo_dev(self._h, layer, start, n, xb, wq.handle,
                                                     wk.handle, wv.handle, wo.handle, x,
                                                     x_mid))

    def rmsnorm_dev(self, x, w, rows: int, n: int, eps: float, out) -> None:
        self._check(self.lib.slm_rmsnorm_dev(self._h, x, w, rows, n, eps, out))

    def l2_norm_dev(self, x, rows: int, n: int, eps: float, out) -> None:
        self._check(self.lib.slm_l2_norm_dev(self._h, x, rows, n, eps, out))

    def swiglu_dev(self, gate, up, n: int, out) -> None:
        self._check(self.lib.slm_swiglu_dev(self._h, gate, up, n, out))

    def residual_add_dev(self, a, b, n: int, out) -> None:
        self._check(self.lib.slm_residual_add_dev(self._h, a, b, n, out))

    def layer_forward_dev(self, layer: int, start: int, n: int, weights: "LayerWeights",
                          rms_eps: float, x) -> None:
        c = weights.c()
        self._check(self.lib.slm_layer_forward_dev(self._h, layer, start, n, ctypes.byref(c),
                                                   rms_eps, x))

    # -- the whole model (TransformerModel) ---------------------------------------
    def model_forward_token_dev(self, weights: "ModelWeights", rms_eps: float, token: int,
                                pos: int, logits=0) -> int:
        nxt = ctypes.c_int32()
        c = weights.c()
        self._check(self.lib.slm_model_forward_token_dev(self._h, ctypes.byref(c), rms_eps,
                                                         token, pos, logits or None,
                                                         ctypes.byref(nxt)))
        return nxt.value

    def model_prefill_dev(self, weights: "ModelWeights", rms_eps: float, tokens, start: int = 0,
                          logits=0) -> int:
        toks = np.ascontiguousarray(tokens, dtype=np.int32)
        nxt = ctypes.c_int32()
        c = weights.c()
        self._check(self.lib.slm_model_prefill_dev(self._h, ctypes.byref(c), rms_eps,
                                                   toks.ctypes.data, toks.size, start,
                                                   logits or None, ctypes.byref(nxt)))
        return nxt.value

    def model_generate_dev(self, weights: "ModelWeights", rms_eps: float, prompt, max_out: int,
                           eos: int = -1) -> list[int]:
        p = np.ascontiguousarray(prompt, dtype=np.int32)
        out = np.zeros(max(max_out, 1), np.int32)
        n = ctypes.c_int32()
        c = weights.c()
        self._check(self.lib.slm_model_generate_dev(self._h, ctypes.byref(c), rms_eps,
                                                    p.ctypes.data, p.size, out.ctypes.data,
                                                    max_out, eos, ctypes.byref(n)))
        return [int(t) for t in out[:n.value]]

    def model_embed_dev(self, weights: "ModelWeights", rms_eps: float, tokens, out) -> None:
        toks = np.ascontiguousarray(tokens, dtype=np.int32)
        c = weights.c()
        self._check(self.lib.slm_model_embed_dev(self._h, ctypes.byref(c), rms_eps,
                                                 toks.ctypes.data, toks.size, out))

    # -- streams, cache access, timing ------------------------------------------
    def set_stream(self, stream: int | None) -> None:
        self._check(self.lib.slm_attn_set_stream(self._h, stream or None))

    def get_stream(self) -> int:
        return self.lib.slm_attn_get_stream(self._h) or 0

    def sync(self) -> None:
        self._check(self.lib.slm_attn_sync(self._h))

    # -- HIP graphs -------------------------------------------------------------
    def capture_begin(self) -> None:
        """Device-pointer calls from here to capture_end() are recorded, not run."""
        self._check(self.lib.slm_attn_capture_begin(self._h))

    def capture_end(self) -> "AttentionGraph":
        g = _P()
        self._check(self.lib.slm_attn_capture_end(self._h, ctypes.byref(g)))
        graph = AttentionGraph(self, g)
        self._graphs.add(graph)
        return graph

    def graph_launch(self, graph: "AttentionGraph") -> None:
        """Replays a recording on the context stream (asynchronous)."""
        self._check(self.lib.slm_attn_graph_launch(self._h, graph.handle))

    def kv_write(self, layer: int, which: int, pos0: int, rows) -> None:
        rows = np.ascontiguousarray(rows, dtype=np.float32).reshape(-1, self.cfg.kv_dim())
        self._check(self.lib.slm_kv_write(self._h, layer, which, pos0, rows.shape[0], _fptr(rows)))

    def kv_write_dev(self, layer: int, which: int, pos0: int, n: int, rows_ptr: int) -> None:
        self._check(self.lib.slm_kv_write_dev(self._h, layer, which, pos0, n, rows_ptr))

    def kv_read(self, layer: int, which: int, pos0: int, n: int) -> np.ndarray:
        out = np.empty((n, self.cfg.kv_dim()), np.float32)
        self._check(self.lib.slm_kv_read(self._h, layer, which, pos0, n, _fptr(out)))
        return out

    def kv_offset(self, layer: int, which: int, pos: int) -> int:
        return int(self.lib.slm_kv_offset(self._h, layer, which, pos))

    def kv_device_ptr(self) -> int:
        return self.lib.slm_kv_device_ptr(self._h) or 0

    def rope_tables(self) -> tuple[np.ndarray, np.ndarray]:
        half = self.cfg.head_dim() // 2
        c = np.empty((self.cfg.max_seq_len, half), np.float32)
        s = np.empty((self.cfg.max_seq_len, half), np.float32)
        self._check(self.lib.slm_rope_tables_read(self._h, _fptr(c), _fptr(s)))
        return c, s

    def profile(self, enable: bool) -> None:
        self._check(self.lib.slm_attn_profile(self._h, 1 if enable else 0))

    def profile_read(self) -> dict:
        arr = (_KernelStat * len(KERNEL_KINDS))()
        self._check(self.lib.slm_attn_profile_read(self._h, arr))
        return {name: (int(arr[i].launches), float(arr[i].total_ms))
                for i, name in enumerate(KERNEL_KINDS)}

    def decode_splits(self, seq_len: int) -> tuple[int, int]:
        """(n_splits, tile): split s reads tiles s, s + n_splits, ... of `tile` rows."""
        ns, tile = _I(), _I()
        self._check(self.lib.slm_attn_decode_splits(self._h, seq_len, ctypes.byref(ns),
                                                    ctypes.byref(tile)))
        return ns.value, tile.value

    def prefill_kernel(self, start: int, n: int) -> str:
        """Name (PREFILL_KERNELS) of the kernel a prefill of n rows from row
        start runs."""
        k = _I()
        self._check(self.lib.slm_attn_prefill_kernel(self._h, start, n, ctypes.byref(k)))
        return PREFILL_KERNELS[k.value]


class AttentionGraph:
    """A recording of device-pointer calls (slm_attn_capture_end).  It keeps
    its context alive, and is destroyed as slm_attn.h asks: after its replays
    have finished (the context's stream is synchronized first) and before the
    context (AttentionContext.close closes its live graphs)."""

    def __init__(self, ctx: "AttentionContext", handle):
        self.lib = ctx.lib
        self._ctx = ctx
        self._h = handle

    @property
    def handle(self):
        return self._h

    def close(self) -> None:
        if getattr(self, "_h", None):
            ctx = self._ctx
            if ctx.handle:
                rc = self.lib.slm_attn_sync(ctx.handle)
                if rc != SLM_OK:
                    raise SlmAttnError(rc, "graph not destroyed: " +
                                       self.lib.slm_attn_last_error(ctx.handle).decode())
            self.lib.slm_attn_graph_destroy(self._h)
            self._h = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class Q4Matrix:
    """A device-resident Q4_0 weight matrix (slm_q4_matrix_create) from
    rows*cols/32 BlockQ4_0 of 18 bytes (blocks.rs:11-19), e.g. as a
    [rows*cols/32, 18] uint8 array."""

    def __init__(self, blocks, rows: int, cols: int, device: int = 0):
        self.lib = load_library()
        blocks = np.ascontiguousarray(blocks, dtype=np.uint8)
        if blocks.size != rows * (cols // 32) * 18:
            raise ValueError("blocks must hold rows*cols/32 BlockQ4_0")
        h = _P()
        rc = self.lib.slm_q4_matrix_create(device, blocks.ctypes.data, rows, cols, ctypes.byref(h))
        if rc != SLM_OK:
            raise SlmAttnError(rc, self.lib.slm_attn_last_error(None).decode())
        self._h = h
        self.rows, self.cols = rows, cols

    @property
    def handle(self):
        return self._h

    def close(self) -> None:
        if getattr(self, "_h", None):
            self.lib.slm_q4_matrix_destroy(self._h)
            self._h = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class LayerWeights:
    """slm_layer_weights (include/slm_layer.h): the two RMSNorm scale vectors
    as device pointers (their memory is the caller's to keep alive) and the
    seven Q4Matrix projections of one layer."""

    def __init__(self, rms_att: int, wq: Q4Matrix, wk: Q4Matrix, wv: Q4Matrix, wo: Q4Matrix,
                 rms_ffn: int, w_gate: Q4Matrix, w_up: Q4Matrix, w_down: Q4Matrix):
        self.rms_att, self.rms_ffn = rms_att, rms_ffn
        self.mats = (wq, wk, wv, wo, w_gate, w_up, w_down)

    def c(self) -> "LayerWeightsC":
        wq, wk, wv, wo, w_gate, w_up, w_down = (m.handle for m in self.mats)
        return LayerWeightsC(self.rms_att, wq, wk, wv, wo, self.rms_ffn, w_gate, w_up, w_down)

    def close(self) -> None:
        for m in self.mats:
            m.close()


class ModelWeights:
    """slm_model_weights (include/slm_layer.h): per-layer LayerWeights, the
    token embedding and lm_head Q4Matrix, and the final RMSNorm scale as a
    device pointer the caller keeps alive."""

    def __init__(self, token_embd: Q4Matrix, layers: list, output_norm: int, lm_head: Q4Matrix):
        self.token_embd, self.layers = token_embd, list(layers)
        self.output_norm, self.lm_head = output_norm, lm_head
        self._arr = (LayerWeightsC * len(self.layers))(*[lw.c() for lw in self.layers])

    def c(self) -> ModelWeightsC:
        return ModelWeightsC(self.token_embd.handle, self._arr, len(self.layers),
                             self.output_norm, self.lm_head.handle)


def _raise(lib, rc: int) -> None:
    if rc != SLM_OK:
        raise SlmAttnError(rc, lib.slm_attn_last_error(None).decode())


class GgufFile:
    """A GGUF v2/v3 file, memory-mapped (slm_gguf_open; GgufFile::open,
    loader.rs:330-400)."""

    def __init__(self, path):
        self.lib = load_library()
        h = _P()
        _raise(self.lib, self.lib.slm_gguf_open(os.fsencode(path), ctypes.byref(h)))
        self._h = h

    @property
    def handle(self):
        return self._h

    @property
    def version(self) -> int:
        return self.lib.slm_gguf_version(self._h)

    @property
    def alignment(self) -> int:
        return self.lib.slm_gguf_alignment(self._h)

    @property
    def data_offset(self) -> int:
        return self.lib.slm_gguf_data_offset(self._h)

    @property
    def tensor_count(self) -> int:
        return self.lib.slm_gguf_tensor_count(self._h)

    @property
    def kv_count(self) -> int:
        return self.lib.slm_gguf_kv_count(self._h)

    def get(self, key: str) -> GgufValueC:
        v = GgufValueC()
        _raise(self.lib, self.lib.slm_gguf_get(self._h, key.encode(), ctypes.byref(v)))
        return v

    def get_u32(self, key: str) -> int:
        v = ctypes.c_uint32()
        _raise(self.lib, self.lib.slm_gguf_get_u32(self._h, key.encode(), ctypes.byref(v)))
        return v.value

    def get_usize(self, key: str) -> int:
        v = ctypes.c_uint64()
        _raise(self.lib, self.lib.slm_gguf_get_usize(self._h, key.encode(), ctypes.byref(v)))
        return v.value

    def get_f32(self, key: str) -> float:
        v = ctypes.c_float()
        _raise(self.lib, self.lib.slm_gguf_get_f32(self._h, key.encode(), ctypes.byref(v)))
        return v.value

    def get_str(self, key: str) -> str:
        p, n = ctypes.c_void_p(), ctypes.c_uint64()
        _raise(self.lib, self.lib.slm_gguf_get_str(self._h, key.encode(), ctypes.byref(p),
                                                   ctypes.byref(n)))
        return ctypes.string_at(p.value, n.value).decode() if n.value else ""

    def tensor_info(self, name: str) -> GgufTensorC:
        t = GgufTensorC()
        _raise(self.lib, self.lib.slm_gguf_tensor_info(self._h, name.encode(), ctypes.byref(t)))
        return t

    def tensor_view(self, name: str, ggml_type: int) -> tuple[int, int]:
        """(address in the mapping, byte length) of a checked tensor view."""
        p, n = ctypes.c_void_p(), ctypes.c_uint64()
        _raise(self.lib, self.lib.slm_gguf_tensor_data(self._h, name.encode(), ggml_type,
                                                       ctypes.byref(p), ctypes.byref(n)))
        return p.value or 0, n.value

    def tensor_bytes(self, name: str, ggml_type: int) -> bytes:
        addr, n = self.tensor_view(name, ggml_type)
        return ctypes.string_at(addr, n) if n else b""

    def model_config(self) -> dict:
        c = ModelConfigC()
        _raise(self.lib, self.lib.slm_gguf_model_config(self._h, ctypes.byref(c)))
        return {f: getattr(c, f) for f, _ in ModelConfigC._fields_}

    def close(self) -> None:
        if getattr(self, "_h", None):
            self.lib.slm_gguf_close(self._h)
            self._h = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class GgufModel:
    """A whole model uploaded from a GgufFile (slm_model_load_gguf); usable
    wherever a ModelWeights is (its c() is the library's own view)."""

    def __init__(self, gguf: GgufFile, num_layers: int, device: int = 0):
        self.lib = load_library()
        h = _P()
        _raise(self.lib, self.lib.slm_model_load_gguf(gguf.handle, device, num_layers,
                                                      ctypes.byref(h)))
        self._h = h

    @property
    def vocab_size(self) -> int:
        return self.lib.slm_model_vocab_size(self._h)

    def c(self) -> "ModelWeightsC":
        return ctypes.cast(self.lib.slm_model_weights_view(self._h),
                           ctypes.POINTER(ModelWeightsC)).contents

    def close(self) -> None:
        if getattr(self, "_h", None):
            self.lib.slm_model_destroy(self._h)
            self._h = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def header_functions(*headers: os.PathLike | str) -> list[str]:
    """Names of the functions the given headers (default: every include/*.h) declare."""
    import re

    paths = headers or (HEADER_PATH, QUANT_HEADER_PATH, LAYER_HEADER_PATH, GGUF_HEADER_PATH)
    names = set()
    for h in paths:
        names |= set(re.findall(r"\b(slm_[a-z0-9_]+)\s*\(", Path(h).read_text()))
    return sorted(names)


# the bench's measurement probes: libslm_calib.so, not part of the product
CALIB_SIGNATURES = {
    "slm_calib_mfma_f32": (ctypes.c_int, [_I, _I, ctypes.POINTER(ctypes.c_double),
                                          ctypes.POINTER(ctypes.c_double)]),
    "slm_calib_hbm_read": (ctypes.c_int, [_I, ctypes.c_int64, _I,
                                          ctypes.POINTER(ctypes.c_double)]),
}
_calib_lib = None


def load_calib_library() -> ctypes.CDLL:
    """Loads calib/libslm_calib.so (the bench's probes); raises if not built."""
    global _calib_lib
    if _calib_lib is not None:
        return _calib_lib
    if not CALIB_LIB_PATH.exists():
        raise FileNotFoundError(f"{CALIB_LIB_PATH} is missing: build the package first")
    _share_torch_hip_runtime()
    lib = ctypes.CDLL(str(CALIB_LIB_PATH))
    for name, (res, args) in CALIB_SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _calib_lib = lib
    return lib


def calibrate_mfma_f32(iters: int = 20000, device: int = 0) -> dict:
    """Measured v_mfma_f32_16x16x4_f32 rate of the device (slm_calib_mfma_f32)."""
    lib = load_calib_library()
    tf, ms = ctypes.c_double(), ctypes.c_double()
    rc = lib.slm_calib_mfma_f32(device, iters, ctypes.byref(tf), ctypes.byref(ms))
    if rc != SLM_OK:
        raise SlmAttnError(rc, "slm_calib_mfma_f32 failed")
    return {"tflops": tf.value, "ms": ms.value, "iters": iters}


def calibrate_hbm_read(nbytes: int = 4 << 30, nontemporal: bool = True, device: int = 0) -> float:
    """Rate of a plain streaming read in GB/s (slm_calib_hbm_read): a probe,
    not a ceiling (the decode kernel streams faster at long context)."""
    lib = load_calib_library()
    gbs = ctypes.c_double()
    rc = lib.slm_calib_hbm_read(device, nbytes, 1 if nontemporal else 0, ctypes.byref(gbs))
    if rc != SLM_OK:
        raise SlmAttnError(rc, "slm_calib_hbm_read failed")
    return gbs.value
