"""GPU parity of the JIT kernels and the transformer block (include/slm_layer.h).

Bars:
  * rmsnorm, l2_norm, swiglu, residual_add: bit for bit against the oracle's
    restatement of the JIT kernels (oracle/layer.c);
  * slm_layer_forward_dev: bit for bit against the same block composed from
    the separately checked entry points (rmsnorm, the Q/K/V + attention + Wo
    block, the projections, swiglu, the projection with residual), which
    share its arithmetic step by step; and, on the reference's own layer-test
    shapes, within the reference's 1e-4 of the oracle's block with K/V cache
    rows bit for bit.  (On large shapes a rounding flip of one Q8_0
    activation value, caused by the attention's last-bit differences, moves
    an output by up to d_a * |w| ~ 1e-3, so there the composition is the
    exact check and the attention itself is held to its own bar elsewhere.)
"""
import sys

import numpy as np
import pytest

from oracle import py_oracle as orc
from slm_testlib import assert_bitwise, gen, load_product

P = load_product()
pytestmark = pytest.mark.gpu
torch = pytest.importorskip("torch")


def log(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def dev(a: np.ndarray):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


@pytest.fixture(scope="module")
def ctx():
    with P.AttentionContext(256, 4, 4, 64, 1) as c:
        yield c


def special_rows(n):
    rows = [np.zeros(n, np.float32), np.ones(n, np.float32) * np.float32(3.0),
            np.full(n, 1e-20, np.float32), np.full(n, 2e15, np.float32)]
    r = np.zeros(n, np.float32)
    r[n // 2] = -7.5
    rows.append(r)
    return np.stack(rows)


NORM_SHAPES = [(1, 32), (7, 576), (33, 4096), (2, 16384), (512, 288), (3, 2048)]


@pytest.mark.parametrize("rows,n", NORM_SHAPES)
@pytest.mark.parametrize("eps", [1e-5, 1e-6])
def test_rmsnorm_bit_exact(ctx, rows, n, eps):
    log(f"rmsnorm rows {rows} n {n} eps {eps}")
    x = gen([11, rows, n], (rows, n)) * np.float32(3.0)
    x = np.concatenate([x, special_rows(n)])
    w = gen([12, n], (n,))
    xd, wd = dev(x), dev(w)
    out = torch.full(x.shape, float("nan"), device="cuda")
    ctx.rmsnorm_dev(xd.data_ptr(), wd.data_ptr(), x.shape[0], n, eps, out.data_ptr())
    ctx.sync()
    assert_bitwise(out.cpu().numpy(), orc.jit_rmsnorm(x, w, eps), f"rmsnorm {rows}x{n}")


@pytest.mark.parametrize("n", [1, 3, 7, 102, 4097])
def test_rmsnorm_tail_lengths_one_row(ctx, n):
    # lengths that are not a multiple of 4 exercise the scalar tail
    x = gen([13, n], (1, n)) * np.float32(2.0)
    w = gen([14, n], (n,))
    xd, wd = dev(x), dev(w)
    out = torch.full((1, n), float("nan"), device="cuda")
    ctx.rmsnorm_dev(xd.data_ptr(), wd.data_ptr(), 1, n, 1e-5, out.data_ptr())
    ctx.sync()
    assert_bitwise(out.cpu().numpy(), orc.jit_rmsnorm(x, w, 1e-5), f"rmsnorm tail n {n}")


@pytest.mark.parametrize("rows,n", [(9, 576), (4, 4096), (1, 102)])
def test_l2_norm_bit_exact(ctx, rows, n):
    x = np.concatenate([gen([15, rows, n], (rows, n)) * np.float32(5.0), special_rows(n)[:2]])
    if n % 4:
        x = x[:1]
    xd = dev(x)
    out = torch.full(x.shape, float("nan"), device="cuda")
    ctx.l2_norm_dev(xd.data_ptr(), x.shape[0], n, 1e-5, out.data_ptr())
    ctx.sync()
    want = np.stack([orc.jit_l2_norm(r, 1e-5) for r in x])
    assert_bitwise(out.cpu().numpy(), want, f"l2 norm {rows}x{n}")


def test_swiglu_and_residual_add_bit_exact(ctx):
    g = np.concatenate([np.linspace(-100, 100, 400001, dtype=np.float32),
                        gen(16, (100003,)) * np.float32(6.0),
                        np.float32([0.0, -0.0, 1e30, -1e30, 87.3, -87.3, 88.3, -88.3, 1e-30])])
    u = gen(17, g.shape) * np.float32(2.0)
    gd, ud = dev(g), dev(u)
    out = torch.full(g.shape, float("nan"), device="cuda")
    ctx.swiglu_dev(gd.data_ptr(), ud.data_ptr(), g.size, out.data_ptr())
    s = torch.full(g.shape, float("nan"), device="cuda")
    ctx.residual_add_dev(gd.data_ptr(), ud.data_ptr(), g.size, s.data_ptr())
    ctx.sync()
    assert_bitwise(out.cpu().numpy(), orc.jit_swiglu(g, u), "swiglu")
    assert_bitwise(s.cpu().numpy(), g + u, "residual add")


def test_norm_and_elementwise_argument_checks(ctx):
    buf = torch.zeros(4 * 64, device="cuda")
    x, w, out = buf[:64], buf[64:128], buf[128:192]
    with pytest.raises(P.SlmAttnError) as ei:   # out on top of x
        ctx.rmsnorm_dev(x.data_ptr(), w.data_ptr(), 1, 64, 1e-5, x.data_ptr())
    assert ei.value.code == P.ERR_ALIAS
    with pytest.raises(P.SlmAttnError) as ei:
        ctx.rmsnorm_dev(x.data_ptr(), w.data_ptr(), 1, 0, 1e-5, out.data_ptr())
    assert ei.value.code == P.ERR_SHAPE
    with pytest.raises(P.SlmAttnError) as ei:   # unaligned rows of 6
        ctx.rmsnorm_dev(x.data_ptr(), w.data_ptr(), 2, 6, 1e-5, out.data_ptr())
    assert ei.value.code == P.ERR_SHAPE
    with pytest.raises(P.SlmAttnError) as ei:
        ctx.rmsnorm_dev(x.data_ptr(), 0, 1, 64, 1e-5, out.data_ptr())
    assert ei.value.code == P.ERR_ARG
    with pytest.raises(P.SlmAttnError) as ei:
        ctx.swiglu_dev(x.data_ptr(), w.data_ptr(), 64, w.data_ptr())
    assert ei.value.code == P.ERR_ALIAS
    ctx.rmsnorm_dev(x.data_ptr(), w.data_ptr(), 0, 64, 1e-5, out.data_ptr())  # no rows
    ctx.swiglu_dev(0, 0, 0, 0)
    ctx.sync()


# ---- the transformer block ----

class Block:
    """Random Q4_0 weights of one layer, on the host (oracle) and the device."""

    def __init__(self, seed, dim, kvd, hidden, wscale=0.3):
        def mat(i, rows, cols):
            return orc.quantize_q4_0(gen([seed, i, rows, cols], (rows, cols)) *
                                     np.float32(wscale))
        self.dim, self.kvd, self.hidden = dim, kvd, hidden
        self.host = orc.LayerWeights(
            rms_att=(np.float32(1.0) + gen([seed, 20], (dim,)) * np.float32(0.2)),
            rms_ffn=(np.float32(1.0) + gen([seed, 21], (dim,)) * np.float32(0.2)),
            wq=mat(1, dim, dim), wk=mat(2, kvd, dim), wv=mat(3, kvd, dim), wo=mat(4, dim, dim),
            w_gate=mat(5, hidden, dim), w_up=mat(6, hidden, dim), w_down=mat(7, dim, hidden),
            hidden_dim=hidden)
        h = self.host
        self.rms_att, self.rms_ffn = dev(h.rms_att), dev(h.rms_ffn)
        self.m = {name: P.Q4Matrix(getattr(h, name), rows, cols) for name, rows, cols in [
            ("wq", dim, dim), ("wk", kvd, dim), ("wv", kvd, dim), ("wo", dim, dim),
            ("w_gate", hidden, dim), ("w_up", hidden, dim), ("w_down", dim, hidden)]}
        m = self.m
        self.dev = P.LayerWeights(self.rms_att.data_ptr(), m["wq"], m["wk"], m["wv"], m["wo"],
                                  self.rms_ffn.data_ptr(), m["w_gate"], m["w_up"], m["w_down"])

    def close(self):
        for m in self.m.values():
            m.close()


def composed_step(ctx, blk: Block, layer, start, n, x, eps):
    """The block from the separately checked entry points (x [n][dim] torch)."""
    dim, hidden = blk.dim, blk.hidden
    m = blk.m
    xb = torch.empty(n, dim, device="cuda")
    x_mid = torch.empty(n, dim, device="cuda")
    ctx.rmsnorm_dev(x.data_ptr(), blk.rms_att.data_ptr(), n, dim, eps, xb.data_ptr())
    if n == 1:
        ctx.decode_wo_dev(layer, start, xb.data_ptr(), m["wq"], m["wk"], m["wv"], m["wo"],
                          x.data_ptr(), x_mid.data_ptr())
    else:
        ctx.prefill_wo_dev(layer, start, n, xb.data_ptr(), m["wq"], m["wk"], m["wv"], m["wo"],
                           x.data_ptr(), x_mid.data_ptr())
    ctx.rmsnorm_dev(x_mid.data_ptr(), blk.rms_ffn.data_ptr(), n, dim, eps, xb.data_ptr())
    gate = torch.empty(n, hidden, device="cuda")
    up = torch.empty(n, hidden, device="cuda")
    act = torch.empty(n, hidden, device="cuda")
    ctx.gemm_q4_0_dev(m["w_gate"], xb.data_ptr(), n, gate.data_ptr())
    ctx.gemm_q4_0_dev(m["w_up"], xb.data_ptr(), n, up.data_ptr())
    ctx.swiglu_dev(gate.data_ptr(), up.data_ptr(), n * hidden, act.data_ptr())
    out = torch.empty(n, dim, device="cuda")
    ctx.gemm_q4_0_residual_dev(m["w_down"], act.data_ptr(), n, x_mid.data_ptr(), out.data_ptr())
    ctx.sync()  # the context's stream is not torch's: finish before the buffers go
    return out


BLOCK_SHAPES = [
    # dim, hidden, heads, kv_heads, msl
    (64, 128, 4, 4, 40),          # the reference's MHA layer test shape
    (128, 256, 8, 2, 40),         # the reference's GQA layer test shape
    (576, 1536, 9, 3, 64),        # SmolLM2-135M
    (2560, 1024, 20, 4, 40),      # rows of 80 blocks: a partial second chunk
    (4096, 14336, 32, 8, 40),     # Llama-3-8B
    (8192, 512, 64, 8, 32),       # Llama-3-70B's width, four chunks
    (12288, 256, 96, 8, 32),      # six chunks, above 64 KiB of LDS when normalizing
]
# (start, n) calls in order: prefill, decode steps, a later prefill chunk,
# small batches (n <= 4 take the MFMA GEMM), more decode
CALLS = [(0, 9), (9, 1), (10, 1), (11, 6), (17, 2), (19, 1), (20, 4), (24, 1)]


@pytest.mark.parametrize("dim,hidden,heads,kvh,msl", BLOCK_SHAPES)
def test_layer_forward_equals_composed_entry_points(dim, hidden, heads, kvh, msl):
    kvd = dim // heads * kvh
    eps = 1e-5
    log(f"block dim {dim} hidden {hidden} heads {heads}/{kvh}")
    blk = Block(31, dim, kvd, hidden)
    try:
        with P.AttentionContext(dim, heads, kvh, msl, 2, 1e4) as a, \
                P.AttentionContext(dim, heads, kvh, msl, 2, 1e4) as b:
            x0 = gen([32, dim], (msl, dim))
            xa = dev(x0)
            xb_ = dev(x0)
            for layer in (0, 1):
                for start, n in CALLS:
                    log(f"  layer {layer} start {start} n {n}")
                    rows = xa[start:start + n]
                    a.layer_forward_dev(layer, start, n, blk.dev, eps, rows.data_ptr())
                    out = composed_step(b, blk, layer, start, n, xb_[start:start + n], eps)
                    xb_[start:start + n].copy_(out)
                    torch.cuda.synchronize()
            a.sync()
            b.sync()
            assert_bitwise(xa.cpu().numpy(), xb_.cpu().numpy(), "residual stream")
            for layer in (0, 1):
                for which in (0, 1):
                    assert_bitwise(a.kv_read(layer, which, 0, msl), b.kv_read(layer, which, 0, msl),
                                   f"cache layer {layer} which {which}")
    finally:
        blk.close()


# Decode positions where the split-K merge runs (more tiles of cache rows than
# one split takes: 4 tiles at hd 128 and hd 64); the layer tests above decode
# within one split.
SPLIT_DECODE_SHAPES = [
    # dim, hidden, heads, kv_heads, msl, prefill rows (tiles of 32 rows for hd 128, 64 for hd 64)
    (1024, 512, 8, 2, 320, 290),
    (576, 1536, 9, 3, 640, 580),
]


@pytest.mark.parametrize("dim,hidden,heads,kvh,msl,pre", SPLIT_DECODE_SHAPES)
def test_layer_decode_with_split_merge_equals_composed(dim, hidden, heads, kvh, msl, pre):
    kvd = dim // heads * kvh
    eps = 1e-5
    log(f"split decode block dim {dim} heads {heads}/{kvh} after {pre} rows")
    blk = Block(51, dim, kvd, hidden)
    calls = [(0, pre), (pre, 1), (pre + 1, 1), (pre + 2, 3), (pre + 5, 1)]
    try:
        with P.AttentionContext(dim, heads, kvh, msl, 1, 1e4) as a, \
                P.AttentionContext(dim, heads, kvh, msl, 1, 1e4) as b:
            assert a.decode_splits(pre + 1)[0] > 1
            x0 = gen([52, dim], (msl, dim))
            xa = dev(x0)
            xb_ = dev(x0)
            for start, n in calls:
                log(f"  start {start} n {n}")
                rows = xa[start:start + n]
                a.layer_forward_dev(0, start, n, blk.dev, eps, rows.data_ptr())
                out = composed_step(b, blk, 0, start, n, xb_[start:start + n], eps)
                xb_[start:start + n].copy_(out)
                torch.cuda.synchronize()
            a.sync()
            b.sync()
            assert_bitwise(xa.cpu().numpy(), xb_.cpu().numpy(), "residual stream")
    finally:
        blk.close()


@pytest.mark.parametrize("dim,hidden,heads,kvh,msl", BLOCK_SHAPES[:2])
def test_layer_forward_against_oracle(dim, hidden, heads, kvh, msl):
    """Each call against the oracle's block from the device's state before it
    (its residual rows and cache): K/V rows bit for bit, the residual stream
    within the reference's own layer-test bound of 1e-4."""
    kvd = dim // heads * kvh
    eps = 1e-5
    cfg = orc.Cfg(dim, heads, kvh, msl, 1, 1e4)
    blk = Block(41, dim, kvd, hidden, wscale=0.25)
    try:
        with P.AttentionContext(dim, heads, kvh, msl, 1, 1e4) as c:
            om = orc.OracleModel(cfg)
            x = dev(gen([42, dim], (msl, dim)))
            for start, n in CALLS:
                before = x[start:start + n].cpu().numpy()
                om.k_cache(0)[:] = c.kv_read(0, 0, 0, msl)
                om.v_cache(0)[:] = c.kv_read(0, 1, 0, msl)
                rows = x[start:start + n]
                c.layer_forward_dev(0, start, n, blk.dev, eps, rows.data_ptr())
                c.sync()
                want = om.layer_forward(0, start, before, blk.host, eps)
                got = rows.cpu().numpy()
                assert_bitwise(c.kv_read(0, 0, start, n), om.k_cache(0)[start:start + n], "K rows")
                assert_bitwise(c.kv_read(0, 1, start, n), om.v_cache(0)[start:start + n], "V rows")
                err = np.abs(got - want).max()
                assert err < 1e-4, f"start {start} n {n}: max abs {err}"
    finally:
        blk.close()


def test_layer_forward_argument_checks():
    dim, heads, kvh, hidden = 64, 4, 4, 128
    blk = Block(51, dim, dim, hidden)
    try:
        with P.AttentionContext(dim, heads, kvh, 8, 1, 1e4) as c:
            x = torch.zeros(8, dim, device="cuda")
            with pytest.raises(P.SlmAttnError) as ei:
                c.layer_forward_dev(1, 0, 1, blk.dev, 1e-5, x.data_ptr())
            assert ei.value.code == P.ERR_LAYER
            with pytest.raises(P.SlmAttnError) as ei:
                c.layer_forward_dev(0, 6, 3, blk.dev, 1e-5, x.data_ptr())
            assert ei.value.code == P.ERR_BATCH
            bad = P.LayerWeights(blk.rms_att.data_ptr(), blk.m["wq"], blk.m["wk"], blk.m["wv"],
                                 blk.m["wo"], blk.rms_ffn.data_ptr(), blk.m["w_gate"],
                                 blk.m["w_up"], blk.m["wq"])  # w_down of the wrong shape
            with pytest.raises(P.SlmAttnError) as ei:
                c.layer_forward_dev(0, 0, 1, bad, 1e-5, x.data_ptr())
            assert ei.value.code == P.ERR_SHAPE
    finally:
        blk.close()
