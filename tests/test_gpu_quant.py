"""GPU parity of the quantized Q/K/V projections (include/slm_quant.h) with the
oracle (oracle/quant.c).

Bar: Q8_0 activation blocks byte for byte (quantize_row_q8_0); GEMV / GEMM
outputs bit for bit against vec_dot_q4_0_q8_0_scalar (kernels.rs:145-161) and
within the reference's own 1e-5 (relative to max(1, |x|)) of its AVX2 path;
the attention block from xb: K/V cache rows bit for bit, outputs within the
attention tolerance (max-abs 1e-4, max-rel 1e-3).
"""
import sys

import numpy as np
import pytest

from oracle import py_oracle as orc
from slm_testlib import assert_bitwise, assert_close, gen, load_product

P = load_product()
pytestmark = pytest.mark.gpu
torch = pytest.importorskip("torch")


def log(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def dev(a: np.ndarray):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def weights(seed, rows, cols, scale=0.05):
    w = gen(seed, (rows, cols)) * np.float32(scale / 0.5)
    return orc.quantize_q4_0(w)


@pytest.fixture(scope="module")
def ctx():
    with P.AttentionContext(4096, 32, 8, 64, 1) as c:
        yield c


def test_quantize_q8_0_bytes_match_oracle(ctx):
    rng = np.random.default_rng(21)
    parts = [rng.standard_normal(32 * 500).astype(np.float32) * np.float32(s)
             for s in (1e-3, 1.0, 37.0, 3e4)]
    special = np.zeros(32 * 6, np.float32)
    special[32 + 7] = -5.0                       # one-hot block
    special[64:96] = np.float32(127.0) * (np.arange(32) % 2)  # exact integer products
    t = special[96:128]
    t[0] = 127.0
    t[1:16] = np.arange(15, dtype=np.float32) + np.float32(0.5)   # exact .5 products
    t[16:31] = -(np.arange(15, dtype=np.float32) + np.float32(0.5))
    special[128:160] = np.float32(1e-30) * rng.standard_normal(32).astype(np.float32)
    special[160:192] = -np.float32(65000.0)
    x = np.concatenate(parts + [special])
    n = x.size
    xd = dev(x)
    out = torch.zeros(n // 32 * 34, dtype=torch.uint8, device="cuda")
    ctx.quantize_q8_0_dev(xd.data_ptr(), n, out.data_ptr())
    ctx.sync()
    got = out.cpu().numpy().reshape(-1, 34)
    want = orc.quantize_q8_0(x)
    bad = np.nonzero((got != want).any(axis=1))[0]
    assert bad.size == 0, f"{bad.size} blocks differ, first {bad[:5]}"


GEMM_CASES = [
    # rows, cols, batch
    (256, 256, 1),      # C1 shape, one block-lane round
    (288, 288, 1),      # C2: nb 9, rows not a multiple of 64
    (192, 576, 3),      # C3 kv_dim x dim, GEMV batch 3
    (1024, 4096, 1),    # Llama-3-8B Wk
    (4096, 4096, 4),    # Llama-3-8B Wq, largest GEMV batch
    (96, 16384, 2),     # nb 512, the longest compiled row
    (1024, 4096, 5),    # smallest MFMA batch
    (288, 288, 17),     # ragged row and token tiles
    (4096, 4096, 64),
    (320, 8192, 100),
    (288, 288, 128),    # ragged row tile
    (1024, 4096, 300),  # ragged token tile
    (96, 16384, 130),   # nb 512
    # enough 128 x 128 tiles to fill 256 CUs, where the launcher picks them
    # over 64 x 64 (Llama-3-8B Q/K/V and gate/up at 4096 tokens do too)
    (8192, 256, 2048),
    (16380, 64, 1000),  # ragged row and token tiles of the 128 x 128 workgroups
]


@pytest.mark.parametrize("rows,cols,batch", GEMM_CASES)
def test_gemm_bit_exact_with_scalar_reference(ctx, rows, cols, batch):
    log(f"gemm rows {rows} cols {cols} batch {batch}")
    w = weights([31, rows, cols], rows, cols)
    x = gen([32, cols, batch], (batch, cols))
    with P.Q4Matrix(w, rows, cols) as W:
        xd = dev(x)
        out = torch.full((batch, rows), float("nan"), device="cuda")
        ctx.gemm_q4_0_dev(W, xd.data_ptr(), batch, out.data_ptr())
        ctx.sync()
        got = out.cpu().numpy()
    want = orc.gemm_q4_0_f32(w, x, batch, rows, cols)
    assert_bitwise(got, want, f"gemm {rows}x{cols} batch {batch}")
    avx = orc.gemm_q4_0_f32(w, x, batch, rows, cols, avx2=True)
    rel = np.abs(got - avx) / np.maximum(np.abs(avx), 1.0)
    assert rel.max() < 1e-5


@pytest.mark.parametrize("batch", [1, 70, 150])
def test_gemm_scales_across_the_f16_range(ctx, batch):
    """Rows and tokens scaled from 1e-7 to 1e3: weight and activation block
    scales from f16 subnormals (below 6.1e-5) to large normals, and zero rows
    and tokens (scale 0), all bit for bit."""
    rows, cols = 192, 512
    row_mag = np.float32(10.0) ** np.linspace(-7, 3, rows).astype(np.float32)
    row_mag[::17] = 0.0
    w = orc.quantize_q4_0(gen([35], (rows, cols)) * row_mag[:, None])
    tok_mag = np.float32(10.0) ** np.linspace(-6, 4, batch).astype(np.float32)
    x = gen([36, batch], (batch, cols)) * tok_mag[:, None]
    if batch > 3:
        x[3] = 0.0
    with P.Q4Matrix(w, rows, cols) as W:
        xd = dev(x)
        out = torch.full((batch, rows), float("nan"), device="cuda")
        ctx.gemm_q4_0_dev(W, xd.data_ptr(), batch, out.data_ptr())
        ctx.sync()
        got = out.cpu().numpy()
    want = orc.gemm_q4_0_f32(w, x, batch, rows, cols)
    assert_bitwise(got, want, f"gemm scales batch {batch}")


def test_gemm_batch_zero_is_a_no_op_and_shapes_are_checked(ctx):
    w = weights(41, 64, 64)
    with P.Q4Matrix(w, 64, 64) as W:
        ctx.gemm_q4_0_dev(W, 0, 0, 0)  # nothing to do, nothing read
    wq = weights(42, 64, 4096)
    with P.Q4Matrix(wq, 64, 4096) as W:
        xd = dev(np.zeros(4096, np.float32))
        out = torch.zeros(4096, device="cuda")
        with pytest.raises(P.SlmAttnError) as ei:
            ctx.decode_xb_dev(0, 0, xd.data_ptr(), W, W, W, out.data_ptr())
        assert ei.value.code == P.ERR_SHAPE
        with pytest.raises(P.SlmAttnError) as ei:
            ctx.gemm_q4_0_dev(W, xd.data_ptr(), 1, xd.data_ptr())
        assert ei.value.code == P.ERR_ALIAS


XB_SHAPES = [
    # dim, heads, kv_heads, msl, theta
    (256, 4, 4, 64, 1e4),        # C1 shape
    (576, 9, 3, 96, 1e5),        # C3 (SmolLM2-135M) shape
    (4096, 32, 8, 320, 5e5),     # C4 (Llama-3-8B) shape
]


@pytest.mark.parametrize("dim,heads,kv_heads,msl,theta", XB_SHAPES)
def test_attention_block_from_xb(dim, heads, kv_heads, msl, theta):
    cfg = orc.Cfg(dim, heads, kv_heads, msl, 1, theta)
    kvd = cfg.kv_dim
    log(f"xb path dim {dim} heads {heads}/{kv_heads}")
    wq = weights([51, dim], dim, dim)
    wk = weights([52, dim], kvd, dim)
    wv = weights([53, dim], kvd, dim)
    n_pre, n_dec = 37, 3
    xb = gen([54, dim], (n_pre + n_dec, dim))
    om = orc.OracleModel(cfg)
    q_all = orc.gemm_q4_0_f32(wq, xb, n_pre + n_dec, dim, dim)
    k_all = orc.gemm_q4_0_f32(wk, xb, n_pre + n_dec, kvd, dim)
    v_all = orc.gemm_q4_0_f32(wv, xb, n_pre + n_dec, kvd, dim)
    with P.AttentionContext(dim, heads, kv_heads, msl, 1, theta) as ctx, \
            P.Q4Matrix(wq, dim, dim) as Wq, P.Q4Matrix(wk, kvd, dim) as Wk, \
            P.Q4Matrix(wv, kvd, dim) as Wv:
        xd = dev(xb)
        out = torch.zeros((n_pre + n_dec, dim), device="cuda")
        # prefill rows 0..36 (MFMA GEMM path), then 3 decode steps (GEMV path)
        ctx.prefill_xb_dev(0, 0, n_pre, xd.data_ptr(), Wq, Wk, Wv, out.data_ptr())
        for s in range(n_dec):
            p = n_pre + s
            ctx.decode_xb_dev(0, p, xd[p].data_ptr(), Wq, Wk, Wv, out[p].data_ptr())
        ctx.sync()
        got = out.cpu().numpy()
        ref_pre = om.prefill(0, 0, q_all[:n_pre], k_all[:n_pre], v_all[:n_pre])
        ref_dec = np.stack([om.decode(0, n_pre + s, q_all[n_pre + s], k_all[n_pre + s],
                                      v_all[n_pre + s]) for s in range(n_dec)])
        rows = n_pre + n_dec
        assert_bitwise(ctx.kv_read(0, 0, 0, rows), om.k_cache(0)[:rows], "K rows")
        assert_bitwise(ctx.kv_read(0, 1, 0, rows), om.v_cache(0)[:rows], "V rows")
        assert_close(got[:n_pre], ref_pre, what="prefill from xb")
        assert_close(got[n_pre:], ref_dec, what="decode from xb")


def test_xb_prefill_gemv_and_gemm_paths_agree():
    # a 4-row prefill takes the GEMV, a 5-row one the MFMA GEMM: both are
    # bit-exact with the scalar dot, so the cache rows they write are equal
    dim, heads, kvh = 576, 9, 3
    kvd = dim // heads * kvh
    wq, wk, wv = weights(61, dim, dim), weights(62, kvd, dim), weights(63, kvd, dim)
    xb = gen(64, (9, dim))
    with P.AttentionContext(dim, heads, kvh, 16, 2) as ctx, \
            P.Q4Matrix(wq, dim, dim) as Wq, P.Q4Matrix(wk, kvd, dim) as Wk, \
            P.Q4Matrix(wv, kvd, dim) as Wv:
        xd = dev(xb)
        out = torch.zeros((9, dim), device="cuda")
        ctx.prefill_xb_dev(0, 0, 4, xd.data_ptr(), Wq, Wk, Wv, out.data_ptr())
        ctx.prefill_xb_dev(0, 4, 5, xd[4:].data_ptr(), Wq, Wk, Wv, out[4:].data_ptr())
        ctx.prefill_xb_dev(1, 0, 9, xd.data_ptr(), Wq, Wk, Wv, out.data_ptr())
        ctx.sync()
        assert_bitwise(ctx.kv_read(0, 0, 0, 9), ctx.kv_read(1, 0, 0, 9), "K rows")
        assert_bitwise(ctx.kv_read(0, 1, 0, 9), ctx.kv_read(1, 1, 0, 9), "V rows")


RESIDUAL_CASES = [
    # rows, cols, batch: Wo (dim x dim) and w_down (dim x hidden_dim) shapes
    (256, 256, 1),        # C1 Wo, GEMV
    (576, 1536, 1),       # SmolLM2-135M w_down, GEMV
    (4096, 4096, 1),      # Llama-3-8B Wo, GEMV
    (4096, 14336, 1),     # Llama-3-8B w_down: nb 448, the longest GEMV row in use
    (576, 576, 4),        # GEMV batch 4
    (288, 768, 7),        # MFMA GEMM, ragged row and token tiles
    (4096, 14336, 65),    # MFMA GEMM, two token tiles
    (4096, 4096, 130),    # MFMA GEMM, ragged last token tile
    (16380, 64, 1000),    # 128 x 128 workgroups (on 256 CUs), ragged row and token tiles
    (90, 256, 9),         # rows not a multiple of 4: the per-element epilogue
]


@pytest.mark.parametrize("rows,cols,batch", RESIDUAL_CASES)
@pytest.mark.parametrize("in_place", [False, True])
def test_projection_plus_residual_bit_exact(ctx, rows, cols, batch, in_place):
    log(f"residual rows {rows} cols {cols} batch {batch} in_place {in_place}")
    w = weights([71, rows, cols], rows, cols)
    x = gen([72, cols, batch], (batch, cols))
    res = gen([73, rows, batch], (batch, rows)) * np.float32(4.0)
    want = res + orc.gemm_q4_0_f32(w, x, batch, rows, cols)  # one f32 add per element
    with P.Q4Matrix(w, rows, cols) as W:
        xd, rd = dev(x), dev(res)
        out = rd if in_place else torch.full((batch, rows), float("nan"), device="cuda")
        ctx.gemm_q4_0_residual_dev(W, xd.data_ptr(), batch, rd.data_ptr(), out.data_ptr())
        ctx.sync()
        got = out.cpu().numpy()
    assert_bitwise(got, want, f"residual {rows}x{cols} batch {batch}")


def test_residual_alias_rules(ctx):
    w = weights(81, 256, 256)
    with P.Q4Matrix(w, 256, 256) as W:
        buf = torch.zeros(3 * 256, device="cuda")
        x, res, out = (buf[i * 256:(i + 1) * 256] for i in range(3))
        with pytest.raises(P.SlmAttnError) as ei:   # out overlapping x
            ctx.gemm_q4_0_residual_dev(W, x.data_ptr(), 1, res.data_ptr(), x.data_ptr())
        assert ei.value.code == P.ERR_ALIAS
        with pytest.raises(P.SlmAttnError) as ei:   # out partly overlapping res
            ctx.gemm_q4_0_residual_dev(W, x.data_ptr(), 1, res.data_ptr(),
                                       buf[300:556].data_ptr())
        assert ei.value.code == P.ERR_ALIAS
        ctx.gemm_q4_0_residual_dev(W, x.data_ptr(), 0, 0, 0)  # batch 0: nothing read
        ctx.sync()


@pytest.mark.parametrize("dim,heads,kv_heads,msl,theta", XB_SHAPES)
def test_attention_block_through_wo(dim, heads, kv_heads, msl, theta):
    """xb -> q/k/v -> attention (into xb) -> x_mid = x + Wo.xb.

    The attention rows are checked within the attention tolerance against the
    oracle, the cache rows and x_mid bit for bit (x_mid against the scalar
    dot of Wo with the attention rows the device produced)."""
    cfg = orc.Cfg(dim, heads, kv_heads, msl, 1, theta)
    kvd = cfg.kv_dim
    log(f"wo block dim {dim} heads {heads}/{kv_heads}")
    wq = weights([91, dim], dim, dim)
    wk = weights([92, dim], kvd, dim)
    wv = weights([93, dim], kvd, dim)
    wo = weights([94, dim], dim, dim)
    n_pre, n_dec = 21, 3
    n = n_pre + n_dec
    xb = gen([95, dim], (n, dim))
    x = gen([96, dim], (n, dim)) * np.float32(3.0)
    om = orc.OracleModel(cfg)
    q_all = orc.gemm_q4_0_f32(wq, xb, n, dim, dim)
    k_all = orc.gemm_q4_0_f32(wk, xb, n, kvd, dim)
    v_all = orc.gemm_q4_0_f32(wv, xb, n, kvd, dim)
    ref_pre = om.prefill(0, 0, q_all[:n_pre], k_all[:n_pre], v_all[:n_pre])
    ref_dec = np.stack([om.decode(0, n_pre + s, q_all[n_pre + s], k_all[n_pre + s],
                                  v_all[n_pre + s]) for s in range(n_dec)])
    with P.AttentionContext(dim, heads, kv_heads, msl, 1, theta) as ctx, \
            P.Q4Matrix(wq, dim, dim) as Wq, P.Q4Matrix(wk, kvd, dim) as Wk, \
            P.Q4Matrix(wv, kvd, dim) as Wv, P.Q4Matrix(wo, dim, dim) as Wo:
        xbd, xd = dev(xb), dev(x)
        x_mid = torch.full((n, dim), float("nan"), device="cuda")
        ctx.prefill_wo_dev(0, 0, n_pre, xbd.data_ptr(), Wq, Wk, Wv, Wo, xd.data_ptr(),
                           x_mid.data_ptr())
        for s in range(n_dec):
            p = n_pre + s
            if s == n_dec - 1:   # in place: x_mid is x itself
                x_mid[p].copy_(xd[p])
                ctx.decode_wo_dev(0, p, xbd[p].data_ptr(), Wq, Wk, Wv, Wo,
                                  x_mid[p].data_ptr(), x_mid[p].data_ptr())
            else:
                ctx.decode_wo_dev(0, p, xbd[p].data_ptr(), Wq, Wk, Wv, Wo, xd[p].data_ptr(),
                                  x_mid[p].data_ptr())
        ctx.sync()
        att = xbd.cpu().numpy()
        got = x_mid.cpu().numpy()
        assert_bitwise(ctx.kv_read(0, 0, 0, n), om.k_cache(0)[:n], "K rows")
        assert_bitwise(ctx.kv_read(0, 1, 0, n), om.v_cache(0)[:n], "V rows")
    assert_close(att[:n_pre], ref_pre, what="prefill attention rows")
    assert_close(att[n_pre:], ref_dec, what="decode attention rows")
    want = x + orc.gemm_q4_0_f32(wo, att, n, dim, dim)
    assert_bitwise(got, want, "x_mid = x + Wo.att")


def test_wo_block_argument_checks():
    dim, heads, kvh = 256, 4, 4
    w = weights(97, dim, dim)
    with P.AttentionContext(dim, heads, kvh, 16, 1) as ctx, P.Q4Matrix(w, dim, dim) as W, \
            P.Q4Matrix(weights(98, 128, dim), 128, dim) as Wbad:
        buf = torch.zeros(3 * dim, device="cuda")
        xb, x, xm = (buf[i * dim:(i + 1) * dim] for i in range(3))
        with pytest.raises(P.SlmAttnError) as ei:
            ctx.decode_wo_dev(0, 0, xb.data_ptr(), W, W, W, Wbad, x.data_ptr(), xm.data_ptr())
        assert ei.value.code == P.ERR_SHAPE
        with pytest.raises(P.SlmAttnError) as ei:   # x_mid on top of xb
            ctx.decode_wo_dev(0, 0, xb.data_ptr(), W, W, W, W, x.data_ptr(), xb.data_ptr())
        assert ei.value.code == P.ERR_ALIAS
        with pytest.raises(P.SlmAttnError) as ei:
            ctx.prefill_wo_dev(0, 10, 7, xb.data_ptr(), W, W, W, W, x.data_ptr(),
                               xm.data_ptr())
        assert ei.value.code == P.ERR_BATCH
