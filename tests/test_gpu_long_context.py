"""Closed-form parity of the long paths on the GPU, tight enough to see one
dropped or duplicated row.

At 131,072 and 32,768 positions the attention outputs are ~1e-3, so the
1e-4 absolute bar of the oracle comparisons is a few percent of the signal:
a split-K tile read twice or not at all would pass it.  These tests choose
inputs whose result is known exactly instead:

- every score zero (K rows and the appended k zero, or q zero), so the
  softmax weights of causal_multi_head_attention_jit (transformer.rs:273-321)
  are exactly uniform: out_h = sum_{t<=p} V[t, g] / (p + 1);
- V rows of small non-negative integers that vary with the row, the tile and
  the column, so every partial sum is an exact f32 integer and the only
  rounding is the final division.

The expected value is the exact integer sum divided in f64; the bar is 1e-6
relative.  Dropping or duplicating any one row moves some output column by
at least ~15/(p+1) on a value of ~30, i.e. >= 3.8e-6 relative at p = 131072.

The same construction checks every row of a 4096-row prefill (row b's
expected value is sum_{t<=b} V[t] / (b + 1)).
"""
import sys

import numpy as np
import pytest

from slm_testlib import _note, err_report, gen, load_product

P = load_product()
pytestmark = pytest.mark.gpu
torch = pytest.importorskip("torch")

DIM, HEADS, KV_HEADS, HD = 4096, 32, 8, 128
KV_DIM = HD * KV_HEADS
REL_BAR = 1e-6


def log(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def v_int_rows(p0: int, n: int, kv_dim: int = KV_DIM, mod: int = 61) -> np.ndarray:
    """V rows p0..p0+n-1: integers 0..mod-1 that depend on the row, its
    32-row tile and the column."""
    t = np.arange(p0, p0 + n, dtype=np.int64)[:, None]
    d = np.arange(kv_dim, dtype=np.int64)[None, :]
    return (t * 7 + d * 13 + (t // 32) * 5) % mod


def v_int_rows_dev(p0: int, n: int, kv_dim: int = KV_DIM, mod: int = 61):
    t = torch.arange(p0, p0 + n, device="cuda", dtype=torch.int64)[:, None]
    d = torch.arange(kv_dim, device="cuda", dtype=torch.int64)[None, :]
    return ((t * 7 + d * 13 + torch.div(t, 32, rounding_mode="floor") * 5) % mod).to(torch.float32)


def prefix_sums(p_list, kv_dim: int = KV_DIM, mod: int = 61) -> dict:
    """Exact sum over rows 0..p of v_int_rows for each p in p_list (int64)."""
    out = {}
    acc = np.zeros(kv_dim, np.int64)
    done = 0
    blk = 8192
    for p in sorted(p_list):
        while done <= p:
            n = min(blk, p + 1 - done)
            acc += v_int_rows(done, n, kv_dim, mod).sum(axis=0)
            done += n
        out[p] = acc.copy()
    return out


def expected_out(s: np.ndarray, p: int, heads=HEADS, kv_heads=KV_HEADS, hd=HD) -> np.ndarray:
    """out[h*hd + i] = S[g*hd + i] / (p + 1), g = h / kv_mul, in f64."""
    kv_mul = heads // kv_heads
    per_head = s.reshape(kv_heads, hd).astype(np.float64) / float(p + 1)
    return np.repeat(per_head, kv_mul, axis=0).reshape(-1)


def check(got, want, what):
    got = np.asarray(got, np.float64)
    assert np.all(np.isfinite(got)), what
    rel = np.abs(got - want) / np.abs(want).clip(min=1.0)
    r = err_report(got, want)
    _note(r)
    log(f"{what}: closed form max-abs {r['max_abs']:.3e} max-rel {float(rel.max()):.3e}")
    assert float(rel.max()) <= REL_BAR, f"{what}: max-rel {float(rel.max()):.3e} > {REL_BAR}"


def fill_v(ctx, layer: int, rows: int, blk: int = 16384, mod: int = 61):
    for p0 in range(0, rows, blk):
        n = min(blk, rows - p0)
        v = v_int_rows_dev(p0, n, mod=mod)
        ctx.kv_write_dev(layer, 1, p0, n, v.data_ptr())
    ctx.sync()


@pytest.mark.parametrize("ctx_len,steps", [(131072, (0, 1, 31, 63)), (32768, (-1,))])
def test_decode_uniform_scores_exact_sum(ctx_len, steps):
    """Zero keys: decode at the C5 length (131,072 pre-filled rows, steps at
    131072+s) and at the 32k headline point (position 32767, msl 32768)."""
    if steps == (-1,):
        msl, positions = ctx_len, [ctx_len - 1]
    else:
        msl, positions = ctx_len + 64, [ctx_len + s for s in steps]
    log(f"uniform-score decode: msl {msl}, positions {positions}")
    sums = prefix_sums(positions)
    with P.AttentionContext(DIM, HEADS, KV_HEADS, msl, 1, 5e5) as ctx:
        first = positions[0]
        fill_v(ctx, 0, first)  # K rows stay zero (the region is zeroed at creation)
        knew = torch.zeros(KV_DIM, device="cuda")
        out = torch.empty(DIM, device="cuda")
        done = first
        for p in positions:
            # rows between the checked positions, appended by decode calls
            while done < p:
                vrow = v_int_rows_dev(done, 1)[0].contiguous()
                q = torch.from_numpy(gen([7, done], DIM)).cuda()
                ctx.decode_dev(0, done, q.data_ptr(), knew.data_ptr(), vrow.data_ptr(),
                               out.data_ptr())
                done += 1
            vrow = v_int_rows_dev(p, 1)[0].contiguous()
            q = torch.from_numpy(gen([7, p], DIM)).cuda()
            ctx.decode_dev(0, p, q.data_ptr(), knew.data_ptr(), vrow.data_ptr(), out.data_ptr())
            ctx.sync()
            done = p + 1
            ns, tile = ctx.decode_splits(p + 1)
            check(out.cpu().numpy(), expected_out(sums[p], p),
                  f"decode pos {p} ({ns} splits of {tile}-row tiles)")


def test_decode_zero_query_random_keys_exact_sum():
    """q = 0 gives zero scores whatever K holds: random K rows (N(0,1)*0.5),
    integer V rows, at 32768 positions."""
    msl = 32768
    p = msl - 1
    with P.AttentionContext(DIM, HEADS, KV_HEADS, msl, 1, 5e5) as ctx:
        fill_v(ctx, 0, p)
        g = torch.Generator(device="cuda")
        g.manual_seed(11)
        kbuf = torch.empty(16384 * KV_DIM, device="cuda")
        for p0 in range(0, p, 16384):
            n = min(16384, p - p0)
            torch.randn(16384 * KV_DIM, generator=g, device="cuda", out=kbuf)
            ctx.kv_write_dev(0, 0, p0, n, kbuf.data_ptr())
        q = torch.zeros(DIM, device="cuda")
        knew = torch.from_numpy(gen(12, KV_DIM)).cuda()
        vrow = v_int_rows_dev(p, 1)[0].contiguous()
        out = torch.empty(DIM, device="cuda")
        ctx.decode_dev(0, p, q.data_ptr(), knew.data_ptr(), vrow.data_ptr(), out.data_ptr())
        ctx.sync()
        check(out.cpu().numpy(), expected_out(prefix_sums([p])[p], p), f"q=0 decode pos {p}")


@pytest.mark.parametrize("start,n", [(0, 4096), (1000, 3096)])
def test_prefill_uniform_scores_every_row(start, n):
    """Zero keys through the batched prefill kernel: every one of its rows
    against the closed form (start > 0 continues an earlier prefill)."""
    msl = 8192
    total = start + n
    v_all = v_int_rows(0, total)
    cums = np.cumsum(v_all, axis=0)  # exact int64 prefix sums
    with P.AttentionContext(DIM, HEADS, KV_HEADS, msl, 1, 5e5) as ctx:
        q = torch.from_numpy(gen([21, start], (total, DIM))).cuda()
        k = torch.zeros(total, KV_DIM, device="cuda")
        v = torch.from_numpy(v_all.astype(np.float32)).cuda()
        out = torch.empty(total, DIM, device="cuda")
        if start:
            ctx.prefill_dev(0, 0, start, q.data_ptr(), k.data_ptr(), v.data_ptr(),
                            out.data_ptr())
        ctx.prefill_dev(0, start, n, q[start:].data_ptr(), k[start:].data_ptr(),
                        v[start:].data_ptr(), out[start:].data_ptr())
        ctx.sync()
        got = out[start:].cpu().numpy().astype(np.float64)
    rows = np.arange(start, total)
    kv_mul = HEADS // KV_HEADS
    want = (cums[rows].reshape(n, KV_HEADS, HD).astype(np.float64)
            / (rows + 1)[:, None, None].astype(np.float64))
    want = np.repeat(want, kv_mul, axis=1).reshape(n, DIM)
    check(got, want, f"prefill rows {start}..{total - 1}")


@pytest.mark.parametrize("dim,heads,kv_heads,start,n", [
    (4096, 32, 8, 7, 4111),   # 129 query blocks of 32: the last holds 15 rows, so its
                              # second 16-row wave has none but joins every DMA and barrier
    (8192, 64, 8, 0, 2100),   # kv_mul 8: two workgroups' head groups share each KV head
])
def test_dma_prefill_unaligned_every_row(dim, heads, kv_heads, start, n):
    """Zero keys through the DMA-fed prefill kernel (hd 128, four query heads
    per workgroup, at least four workgroups per CU on 256 CUs) at row counts
    that are not multiples of its 32-row query block: every row against the
    closed form."""
    hd = dim // heads
    kv_dim = hd * kv_heads
    total = start + n
    v_all = v_int_rows(0, total, kv_dim)
    cums = np.cumsum(v_all, axis=0)
    log(f"DMA prefill {heads}/{kv_heads} heads, rows {start}..{total - 1}")
    with P.AttentionContext(dim, heads, kv_heads, total, 1, 5e5) as ctx:
        q = torch.from_numpy(gen([23, start], (total, dim))).cuda()
        k = torch.zeros(total, kv_dim, device="cuda")
        v = torch.from_numpy(v_all.astype(np.float32)).cuda()
        out = torch.empty(total, dim, device="cuda")
        if start:
            ctx.prefill_dev(0, 0, start, q.data_ptr(), k.data_ptr(), v.data_ptr(),
                            out.data_ptr())
        ctx.prefill_dev(0, start, n, q[start:].data_ptr(), k[start:].data_ptr(),
                        v[start:].data_ptr(), out[start:].data_ptr())
        ctx.sync()
        got = out[start:].cpu().numpy().astype(np.float64)
    rows = np.arange(start, total)
    want = (cums[rows].reshape(n, kv_heads, hd).astype(np.float64)
            / (rows + 1)[:, None, None].astype(np.float64))
    want = np.repeat(want, heads // kv_heads, axis=1).reshape(n, dim)
    check(got, want, f"DMA prefill rows {start}..{total - 1}")

def test_prefill_and_decode_past_row_2_pow_20():
    """One layer's K slice past 4 GiB (1,048,600 rows of kv_dim 1024, an
    8.6 GB cache): zero keys and V integers 0..15 (every sum below 2^24
    stays exact).  The 32-row prefill takes the register-prefetch kernel,
    the 4096-row one the DMA kernel; both end at row 1,048,599, so their
    first tiles' buffer ranges would have wrapped in 32 bits (to 8 and 24
    rows), reading the other rows of those tiles as zeros.  Every row of
    both against the closed form, then one decode at the last position."""
    msl = (1 << 20) + 24
    mod = 16
    log(f"past 2^20: msl {msl}, KV {2 * msl * KV_DIM * 4 / 1e9:.1f} GB")
    last = msl - 1
    n_big = 4096
    s_big = msl - n_big
    base = prefix_sums([s_big - 1], mod=mod)[s_big - 1]
    tail = v_int_rows(s_big, n_big, mod=mod)
    cums = base[None, :] + np.cumsum(tail, axis=0)  # exact sums over rows 0..s_big+b
    kv_mul = HEADS // KV_HEADS

    def want_rows(b0, n):
        rows = np.arange(b0, b0 + n)  # positions
        s = cums[rows - s_big].reshape(n, KV_HEADS, HD).astype(np.float64)
        w = s / (rows + 1)[:, None, None].astype(np.float64)
        return np.repeat(w, kv_mul, axis=1).reshape(n, DIM)

    with P.AttentionContext(DIM, HEADS, KV_HEADS, msl, 1, 5e5) as ctx:
        fill_v(ctx, 0, msl, mod=mod)  # K rows stay zero
        for n in (32, n_big):
            start = msl - n
            log(f"past 2^20: prefill {n} rows at {start}")
            q = torch.from_numpy(gen([31, n], (n, DIM))).cuda()
            k = torch.zeros(n, KV_DIM, device="cuda")
            v = v_int_rows_dev(start, n, mod=mod).contiguous()
            out = torch.empty(n, DIM, device="cuda")
            ctx.prefill_dev(0, start, n, q.data_ptr(), k.data_ptr(), v.data_ptr(),
                            out.data_ptr())
            ctx.sync()
            check(out.cpu().numpy(), want_rows(start, n), f"prefill rows {start}..{last}")
        log(f"past 2^20: decode at {last}")
        q = torch.from_numpy(gen([32, last], DIM)).cuda()
        knew = torch.zeros(KV_DIM, device="cuda")
        vrow = v_int_rows_dev(last, 1, mod=mod)[0].contiguous()
        out = torch.empty(DIM, device="cuda")
        ctx.decode_dev(0, last, q.data_ptr(), knew.data_ptr(), vrow.data_ptr(), out.data_ptr())
        ctx.sync()
        check(out.cpu().numpy(), want_rows(last, 1)[0], f"decode pos {last}")
