"""ctypes binding of the C oracle (liboracle.so) -- test infrastructure only.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg use
this module, as the checker.  Functions restate static-lm's CPU arithmetic;
see slm_oracle.h for the reference lines each one follows.
"""
from __future__ import annotations

import ctypes
import subprocess
from dataclasses import dataclass
from pathlib import Path

import numpy as np

ORACLE_DIR = Path(__file__).resolve().parent
LIB_PATH = ORACLE_DIR / "liboracle.so"


class OrcConfig(ctypes.Structure):
    _fields_ = [
        ("dim", ctypes.c_int32),
        ("num_heads", ctypes.c_int32),
        ("num_kv_heads", ctypes.c_int32),
        ("max_seq_len", ctypes.c_int32),
        ("num_layers", ctypes.c_int32),
        ("rope_theta", ctypes.c_float),
    ]


_F = ctypes.POINTER(ctypes.c_float)
_D = ctypes.POINTER(ctypes.c_double)
_C = ctypes.POINTER(OrcConfig)
_SZ = ctypes.c_size_t
_I = ctypes.c_int
_U8 = ctypes.POINTER(ctypes.c_uint8)

_SIGS = {
    "orc_validate": (ctypes.c_int, [_C]),
    "orc_rope_tables": (None, [_I, _I, ctypes.c_float, _F, _F]),
    "orc_apply_rope_cached": (None, [_F, _SZ, _F, _F, _I]),
    "orc_apply_rope_in_place": (None, [_F, _SZ, _I, _I, ctypes.c_float]),
    "orc_jit_exp": (ctypes.c_float, [ctypes.c_float]),
    "orc_jit_exp_array": (None, [_F, _F, _SZ]),
    "orc_softmax_jit": (None, [_F, _SZ]),
    "orc_softmax_scalar": (None, [_F, _SZ]),
    "orc_attention_jit": (None, [_F, _F, _F, _F, _F, _C, _I]),
    "orc_attention_scalar": (None, [_F, _F, _F, _F, _F, _C, _I]),
    "orc_kv_offset": (_SZ, [_C, _I, _I, _I]),
    "orc_decode": (None, [_C, _F, _F, _F, _I, _I, _F, _F, _F, _F, _F, _F]),
    "orc_prefill": (None, [_C, _F, _F, _F, _I, _I, _I, _F, _F, _F, _F, _F, _F]),
    "orc_attention_f64": (None, [_F, _F, _F, _D, _C, _I]),
    "orc_f32_to_f16": (ctypes.c_uint16, [ctypes.c_float]),
    "orc_f16_to_f32": (ctypes.c_float, [ctypes.c_uint16]),
    "orc_quantize_row_q4_0": (None, [_F, _SZ, _U8]),
    "orc_dequantize_row_q4_0": (None, [_U8, _SZ, _F]),
    "orc_quantize_row_q8_0": (None, [_F, _SZ, _U8]),
    "orc_dequantize_row_q8_0": (None, [_U8, _SZ, _F]),
    "orc_vec_dot_q4_0_q8_0_scalar": (ctypes.c_float, [_U8, _U8, _SZ]),
    "orc_vec_dot_q4_0_q8_0_avx2": (ctypes.c_float, [_U8, _U8, _SZ]),
    "orc_gemm_q4_0": (None, [_U8, _U8, _F, _I, _I, _I, _I]),
    "orc_jit_rmsnorm_scale": (ctypes.c_float, [_F, _SZ, ctypes.c_float]),
    "orc_jit_rmsnorm": (None, [_F, _F, _SZ, ctypes.c_float, _F]),
    "orc_jit_silu": (ctypes.c_float, [ctypes.c_float]),
    "orc_jit_swiglu": (None, [_F, _F, _SZ, _F]),
    "orc_jit_residual_add": (None, [_F, _F, _SZ, _F]),
    "orc_jit_l2_norm": (None, [_F, _SZ, ctypes.c_float, _F]),
    "orc_scalar_rmsnorm": (None, [_F, _F, _SZ, ctypes.c_float, _F]),
    "orc_layer_forward_batch": (None, [_C, _I, ctypes.c_float, ctypes.c_void_p, _F, _F, _F,
                                       _I, _I, _I, _F]),
}


class OrcLayerWeights(ctypes.Structure):
    _fields_ = [
        ("rms_att", _F), ("wq", _U8), ("wk", _U8), ("wv", _U8), ("wo", _U8),
        ("rms_ffn", _F), ("w_gate", _U8), ("w_up", _U8), ("w_down", _U8),
    ]

_lib = None


def build() -> Path:
    """Compiles liboracle.so with oracle/Makefile (gcc, no fast-math)."""
    subprocess.run(["make", "-s", "-C", str(ORACLE_DIR)], check=True)
    return LIB_PATH


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            build()
        L = ctypes.CDLL(str(LIB_PATH))
        for name, (res, args) in _SIGS.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def _p(a: np.ndarray):
    assert a.dtype == np.float32 and a.flags.c_contiguous
    return a.ctypes.data_as(_F)


def _f32(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32)


@dataclass(frozen=True)
class Cfg:
    dim: int
    num_heads: int
    num_kv_heads: int
    max_seq_len: int
    num_layers: int = 1
    rope_theta: float = 10000.0

    @property
    def head_dim(self) -> int:
        return self.dim // self.num_heads

    @property
    def kv_dim(self) -> int:
        return self.head_dim * self.num_kv_heads

    @property
    def kv_mul(self) -> int:
        return self.num_heads // self.num_kv_heads

    def c(self) -> OrcConfig:
        return OrcConfig(self.dim, self.num_heads, self.num_kv_heads, self.max_seq_len,
                         self.num_layers, self.rope_theta)


def validate(cfg: Cfg) -> int:
    c = cfg.c()
    return lib().orc_validate(ctypes.byref(c))


def rope_tables(head_dim: int, max_seq_len: int, theta: float = 10000.0):
    half = head_dim // 2
    c = np.empty((max_seq_len, half), np.float32)
    s = np.empty((max_seq_len, half), np.float32)
    lib().orc_rope_tables(head_dim, max_seq_len, theta, _p(c), _p(s))
    return c, s


def apply_rope_cached(vec, cos_row, sin_row, head_dim: int) -> np.ndarray:
    v = _f32(vec).copy()
    c, s = _f32(cos_row), _f32(sin_row)
    lib().orc_apply_rope_cached(_p(v), v.size, _p(c), _p(s), head_dim)
    return v


def apply_rope_in_place(vec, pos: int, head_dim: int, theta: float = 10000.0) -> np.ndarray:
    v = _f32(vec).copy()
    lib().orc_apply_rope_in_place(_p(v), v.size, pos, head_dim, theta)
    return v


def jit_exp(x) -> np.ndarray:
    x = _f32(x)
    out = np.empty_like(x)
    lib().orc_jit_exp_array(_p(x), _p(out), x.size)
    return out


def softmax_jit(x) -> np.ndarray:
    v = _f32(x).copy()
    lib().orc_softmax_jit(_p(v), v.size)
    return v


def softmax_scalar(x) -> np.ndarray:
    v = _f32(x).copy()
    lib().orc_softmax_scalar(_p(v), v.size)
    return v


def attention(q_rot, k_cache, v_cache, cfg: Cfg, pos: int, jit: bool = True) -> np.ndarray:
    """causal_multi_head_attention{_jit} over one layer's [msl][kv_dim] slices."""
    q = _f32(q_rot)
    kc, vc = _f32(k_cache), _f32(v_cache)
    att = np.empty(cfg.num_heads * cfg.max_seq_len, np.float32)
    out = np.empty(cfg.dim, np.float32)
    c = cfg.c()
    fn = lib().orc_attention_jit if jit else lib().orc_attention_scalar
    fn(_p(q), _p(kc), _p(vc), _p(att), _p(out), ctypes.byref(c), pos)
    return out


def attention_f64(q_rot, k_cache, v_cache, cfg: Cfg, pos: int) -> np.ndarray:
    q = _f32(q_rot)
    kc, vc = _f32(k_cache), _f32(v_cache)
    out = np.empty(cfg.dim, np.float64)
    c = cfg.c()
    lib().orc_attention_f64(_p(q), _p(kc), _p(vc), out.ctypes.data_as(_D), ctypes.byref(c), pos)
    return out


def kv_offset(cfg: Cfg, layer: int, which: int, pos: int) -> int:
    c = cfg.c()
    return int(lib().orc_kv_offset(ctypes.byref(c), layer, which, pos))


class OracleModel:
    """The reference's KV arena [L][K|V][msl][kv_dim] plus RoPE tables, driven
    like TransformerModel drives its layers (decode and prefill blocks)."""

    def __init__(self, cfg: Cfg):
        self.cfg = cfg
        self.kv = np.zeros(2 * cfg.num_layers * cfg.max_seq_len * cfg.kv_dim, np.float32)
        self.cos, self.sin = rope_tables(cfg.head_dim, cfg.max_seq_len, cfg.rope_theta)
        self._att = np.empty(cfg.num_heads * cfg.max_seq_len, np.float32)

    def k_cache(self, layer: int) -> np.ndarray:
        S = self.cfg.max_seq_len * self.cfg.kv_dim
        return self.kv[(2 * layer) * S:(2 * layer + 1) * S].reshape(self.cfg.max_seq_len, -1)

    def v_cache(self, layer: int) -> np.ndarray:
        S = self.cfg.max_seq_len * self.cfg.kv_dim
        return self.kv[(2 * layer + 1) * S:(2 * layer + 2) * S].reshape(self.cfg.max_seq_len, -1)

    def decode(self, layer: int, pos: int, q, k, v) -> np.ndarray:
        cfg = self.cfg
        q, k, v = _f32(q), _f32(k), _f32(v)
        q_rot = np.empty(cfg.dim, np.float32)
        out = np.empty(cfg.dim, np.float32)
        c = cfg.c()
        lib().orc_decode(ctypes.byref(c), _p(self.kv), _p(self.cos), _p(self.sin), layer, pos,
                         _p(q), _p(k), _p(v), _p(q_rot), _p(self._att), _p(out))
        return out

    def prefill(self, layer: int, start: int, q, k, v) -> np.ndarray:
        cfg = self.cfg
        q = _f32(q).reshape(-1, cfg.dim)
        n = q.shape[0]
        k, v = _f32(k), _f32(v)
        q_rot = np.empty_like(q)
        out = np.empty_like(q)
        c = cfg.c()
        lib().orc_prefill(ctypes.byref(c), _p(self.kv), _p(self.cos), _p(self.sin), layer, start,
                          n, _p(q), _p(k), _p(v), _p(q_rot), _p(self._att), _p(out))
        return out

    def append(self, layer: int, pos0: int, k_rows, v_rows) -> None:
        """Only the cache side of a decode/prefill block: K rows pos0.. get
        rope(k), V rows get v (transformer.rs:545-561 then 575-578)."""
        k_rows = _f32(k_rows).reshape(-1, self.cfg.kv_dim)
        v_rows = _f32(v_rows).reshape(-1, self.cfg.kv_dim)
        kc, vc = self.k_cache(layer), self.v_cache(layer)
        for r in range(k_rows.shape[0]):
            p = pos0 + r
            kc[p] = apply_rope_cached(k_rows[r], self.cos[p], self.sin[p], self.cfg.head_dim)
            vc[p] = v_rows[r]

    def layer_forward(self, layer: int, start: int, x, w: "LayerWeights", eps: float) -> np.ndarray:
        """forward_batch_with_kv (transformer.rs:491-651) of x [n][dim] at
        rows start..start+n-1; n = 1 is forward_token_with_kv.  Returns the
        new residual stream; the cache rows are written like the reference's."""
        x = np.array(_f32(x).reshape(-1, self.cfg.dim), copy=True)
        n = x.shape[0]
        c = self.cfg.c()
        cw = w.c()
        lib().orc_layer_forward_batch(ctypes.byref(c), w.hidden_dim, eps, ctypes.byref(cw),
                                      _p(self.kv), _p(self.cos), _p(self.sin), layer, start, n,
                                      _p(x))
        return x

    def rotated_q(self, q_row, pos: int) -> np.ndarray:
        return apply_rope_cached(q_row, self.cos[pos], self.sin[pos], self.cfg.head_dim)

    def attend(self, layer: int, q_row, pos: int) -> np.ndarray:
        """Attention of an un-rotated q row at `pos` over the current cache."""
        q_rot = self.rotated_q(q_row, pos)
        return attention(q_rot, self.k_cache(layer), self.v_cache(layer), self.cfg, pos)


# ---- quantized projections (src/quant/blocks.rs, src/quant/kernels.rs) ----

QK = 32
Q4_BYTES = 18
Q8_BYTES = 34


def _u8(a: np.ndarray):
    assert a.dtype == np.uint8 and a.flags.c_contiguous
    return a.ctypes.data_as(_U8)


def f32_to_f16_bits(x) -> np.ndarray:
    """half::f16::from_f32(x).to_bits() for every element (uint16)."""
    x = _f32(x).ravel()
    L = lib()
    return np.array([L.orc_f32_to_f16(float(v)) for v in x], dtype=np.uint16)


def f16_bits_to_f32(h) -> np.ndarray:
    L = lib()
    return np.array([L.orc_f16_to_f32(int(v)) for v in np.asarray(h).ravel()], dtype=np.float32)


def quantize_q4_0(x) -> np.ndarray:
    """quantize_row_q4_0 (blocks.rs:50-82): [n] f32 -> [n/32][18] bytes."""
    x = _f32(x).ravel()
    assert x.size % QK == 0
    out = np.zeros((x.size // QK, Q4_BYTES), np.uint8)
    lib().orc_quantize_row_q4_0(_p(x), x.size, _u8(out))
    return out


def dequantize_q4_0(blocks: np.ndarray) -> np.ndarray:
    blocks = np.ascontiguousarray(blocks, np.uint8).reshape(-1, Q4_BYTES)
    out = np.zeros(blocks.shape[0] * QK, np.float32)
    lib().orc_dequantize_row_q4_0(_u8(blocks), blocks.shape[0], _p(out))
    return out


def quantize_q8_0(x) -> np.ndarray:
    """quantize_row_q8_0 (blocks.rs:102-123): [n] f32 -> [n/32][34] bytes."""
    x = _f32(x).ravel()
    assert x.size % QK == 0
    out = np.zeros((x.size // QK, Q8_BYTES), np.uint8)
    lib().orc_quantize_row_q8_0(_p(x), x.size, _u8(out))
    return out


def dequantize_q8_0(blocks: np.ndarray) -> np.ndarray:
    blocks = np.ascontiguousarray(blocks, np.uint8).reshape(-1, Q8_BYTES)
    out = np.zeros(blocks.shape[0] * QK, np.float32)
    lib().orc_dequantize_row_q8_0(_u8(blocks), blocks.shape[0], _p(out))
    return out


def vec_dot_q4_0_q8_0(w: np.ndarray, a: np.ndarray, avx2: bool = False) -> float:
    """vec_dot_q4_0_q8_0_scalar (kernels.rs:145-161) or the AVX2 path (163-212)."""
    w = np.ascontiguousarray(w, np.uint8).reshape(-1, Q4_BYTES)
    a = np.ascontiguousarray(a, np.uint8).reshape(-1, Q8_BYTES)
    assert w.shape[0] == a.shape[0]
    fn = lib().orc_vec_dot_q4_0_q8_0_avx2 if avx2 else lib().orc_vec_dot_q4_0_q8_0_scalar
    return float(np.float32(fn(_u8(w), _u8(a), w.shape[0])))


def gemm_q4_0(w: np.ndarray, x_q8: np.ndarray, batch: int, rows: int, cols: int,
              avx2: bool = False) -> np.ndarray:
    """gemm_q4_0 (kernels.rs:308-394): [batch][rows] f32."""
    w = np.ascontiguousarray(w, np.uint8).reshape(-1, Q4_BYTES)
    x_q8 = np.ascontiguousarray(x_q8, np.uint8).reshape(-1, Q8_BYTES)
    assert cols % QK == 0 and w.shape[0] == rows * cols // QK
    assert x_q8.shape[0] == batch * cols // QK
    out = np.zeros((batch, rows), np.float32)
    lib().orc_gemm_q4_0(_u8(w), _u8(x_q8), _p(out), batch, rows, cols, 1 if avx2 else 0)
    return out


def gemm_q4_0_f32(w: np.ndarray, x, batch: int, rows: int, cols: int,
                  avx2: bool = False) -> np.ndarray:
    """gemm_q4_0_arena (kernels.rs:398-415): quantize x [batch][cols] to Q8_0,
    then gemm_q4_0."""
    return gemm_q4_0(w, quantize_q8_0(x), batch, rows, cols, avx2)


# ---- JIT normalisation / activation kernels and the block (layer.c) ----

def jit_rmsnorm(x, w, eps: float) -> np.ndarray:
    """FuseGraph::rmsnorm (graph.rs:141-156) over each row of x."""
    x = _f32(x)
    w = _f32(w)
    rows = x.reshape(-1, w.size)
    out = np.empty_like(rows)
    for r in range(rows.shape[0]):
        row = np.ascontiguousarray(rows[r])
        o = np.empty_like(row)
        lib().orc_jit_rmsnorm(_p(row), _p(w), w.size, eps, _p(o))
        out[r] = o
    return out.reshape(x.shape)


def jit_rmsnorm_scale(x, eps: float) -> float:
    x = _f32(x)
    return float(lib().orc_jit_rmsnorm_scale(_p(x), x.size, eps))


def scalar_rmsnorm(x, w, eps: float) -> np.ndarray:
    """The reference tests' scalar_rmsnorm (transformer.rs:978-985)."""
    x, w = _f32(x), _f32(w)
    out = np.empty_like(x)
    lib().orc_scalar_rmsnorm(_p(x), _p(w), x.size, eps, _p(out))
    return out


def jit_silu(v) -> np.ndarray:
    v = _f32(v)
    return np.array([lib().orc_jit_silu(float(t)) for t in v.ravel()], np.float32).reshape(v.shape)


def jit_swiglu(gate, up) -> np.ndarray:
    """FuseGraph::swiglu (graph.rs:131-139)."""
    gate, up = _f32(gate), _f32(up)
    out = np.empty_like(gate)
    lib().orc_jit_swiglu(_p(gate), _p(up), gate.size, _p(out))
    return out


def jit_residual_add(a, b) -> np.ndarray:
    a, b = _f32(a), _f32(b)
    out = np.empty_like(a)
    lib().orc_jit_residual_add(_p(a), _p(b), a.size, _p(out))
    return out


def jit_l2_norm(x, eps: float) -> np.ndarray:
    """FuseGraph::l2_norm (graph.rs:182-193)."""
    x = _f32(x)
    out = np.empty_like(x)
    lib().orc_jit_l2_norm(_p(x), x.size, eps, _p(out))
    return out


@dataclass
class LayerWeights:
    """TransformerWeights (transformer.rs:36-47): f32 norm scales and
    BlockQ4_0 matrices as uint8 arrays of 18-byte blocks."""
    rms_att: np.ndarray
    wq: np.ndarray
    wk: np.ndarray
    wv: np.ndarray
    wo: np.ndarray
    rms_ffn: np.ndarray
    w_gate: np.ndarray
    w_up: np.ndarray
    w_down: np.ndarray
    hidden_dim: int

    def c(self) -> OrcLayerWeights:
        for name in ("wq", "wk", "wv", "wo", "w_gate", "w_up", "w_down"):
            a = getattr(self, name)
            assert a.dtype == np.uint8 and a.flags.c_contiguous
        for name in ("rms_att", "rms_ffn"):
            a = getattr(self, name)
            assert a.dtype == np.float32 and a.flags.c_contiguous
        return OrcLayerWeights(_p(self.rms_att), _u8(self.wq), _u8(self.wk), _u8(self.wv),
                               _u8(self.wo), _p(self.rms_ffn), _u8(self.w_gate),
                               _u8(self.w_up), _u8(self.w_down))


# ---- the whole model (TransformerModel, transformer.rs:699-957) ----

def sample_argmax(logits) -> int:
    """sample_argmax (transformer.rs:655-667): scan from index 0 with a
    strict `>`, so the first maximum wins and a later NaN never does."""
    logits = _f32(logits)
    best, val = 0, logits[0]
    for i in range(1, logits.size):
        if logits[i] > val:
            best, val = i, logits[i]
    return best


@dataclass
class ModelWeights:
    """ModelWeights (transformer.rs:49-56): BlockQ4_0 token_embd and lm_head
    [vocab][dim], per-layer LayerWeights, f32 output_norm."""
    token_embd: np.ndarray
    layers: list
    output_norm: np.ndarray
    lm_head: np.ndarray
    vocab_size: int


def embed_rows(token_embd: np.ndarray, tokens, dim: int) -> np.ndarray:
    """dequantize_row_q4_0 of each token's row (transformer.rs:769-770)."""
    nb = dim // QK
    blocks = np.ascontiguousarray(token_embd).reshape(-1, Q4_BYTES)
    return np.stack([dequantize_q4_0(blocks[t * nb:(t + 1) * nb]) for t in tokens])


def model_forward(om: "OracleModel", w: ModelWeights, eps: float, tokens, start: int):
    """forward_token (n = 1, transformer.rs:746-796) / prefill_tokens (n > 1,
    :800-850): returns (logits of the last row, argmax, residual rows)."""
    dim = om.cfg.dim
    x = embed_rows(w.token_embd, tokens, dim)
    for layer, lw in enumerate(w.layers):
        x = om.layer_forward(layer, start, x, lw, eps)
    xb = jit_rmsnorm(x[-1], w.output_norm, eps)
    logits = gemm_q4_0_f32(w.lm_head, xb, 1, w.vocab_size, dim)[0]
    return logits, sample_argmax(logits), x


def model_generate(om: "OracleModel", w: ModelWeights, eps: float, prompt, max_out: int,
                   eos: int = -1) -> list:
    """generate (transformer.rs:853-899)."""
    if max_out <= 0 or len(prompt) == 0:
        return []
    _, nxt, _ = model_forward(om, w, eps, prompt, 0)
    out = [nxt]
    if nxt == eos:
        return out
    pos = len(prompt)
    while len(out) < max_out and pos < om.cfg.max_seq_len:
        _, nxt, _ = model_forward(om, w, eps, [nxt], pos)
        out.append(nxt)
        pos += 1
        if nxt == eos:
            break
    return out


def model_embed(om: "OracleModel", w: ModelWeights, eps: float, tokens) -> np.ndarray:
    """embed_tokens (transformer.rs:904-957): the batch at 0 through every
    layer, each row normed with output_norm, accum += row * (1/n) in order,
    then the L2 norm."""
    dim = om.cfg.dim
    x = embed_rows(w.token_embd, tokens, dim)
    for layer, lw in enumerate(w.layers):
        x = om.layer_forward(layer, 0, x, lw, eps)
    inv = np.float32(1.0) / np.float32(len(tokens))
    acc = np.zeros(dim, np.float32)
    for b in range(len(tokens)):
        acc = acc + jit_rmsnorm(x[b], w.output_norm, eps) * inv
    return jit_l2_norm(acc, eps)
