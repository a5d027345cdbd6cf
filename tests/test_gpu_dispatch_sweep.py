"""GPU parity over a seeded sweep of shapes and batches.

Each case prefills rows start..start+n-1 of one layer (after a prefix prefill
of rows 0..start-1), then decodes two positions, on a context whose cache is
exactly that long, and checks against the oracle: K/V rows bit for bit, every
output within max-abs 1e-4 and max-rel 1e-3 (relative error floored at |ref| =
0.1).  The targeted cases take each prefill kernel the library has (checked
through slm_attn_prefill_kernel); the random ones draw head dims, GQA
groupings, starts and lengths from a fixed seed, so the dispatch thresholds
meet batch shapes nobody picked by hand.  Where the oracle's full prefill
would take more than a few seconds, stated rows are checked instead (the
first and last rows of the first blocks, rows around block boundaries, the
last rows, a few seeded ones), each as the oracle's single-row attention
over the filled cache: the reference's prefill computes every row that way
(transformer.rs:563-593 calls the attention once per row).
"""
import sys

import numpy as np
import pytest

from oracle import py_oracle as orc
from slm_testlib import (SWEEP_TARGETED, assert_bitwise, assert_close, gen, load_product,
                         sweep_random_cases)

P = load_product()
pytestmark = pytest.mark.gpu

FULL_ORACLE_FLOP = 7.5e9  # about 3 s of the oracle's prefill on one core

CASES = ([pytest.param(*c, id=f"{c[5]}-{c[0]}-{c[1]}-{c[2]}-{c[3]}-{c[4]}") for c in SWEEP_TARGETED]
         + [pytest.param(*c, None, id=f"random{i}-{c[0]}-{c[1]}-{c[2]}-{c[3]}-{c[4]}")
            for i, c in enumerate(sweep_random_cases())])


def log(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def sample_rows(n, seed):
    rows = {0, 1, 15, 16, 17, 31, 32, 33, n // 3, n // 2, n - 33, n - 32, n - 17, n - 16,
            n - 2, n - 1}
    rows |= set(np.random.default_rng(seed).integers(0, n, 4).tolist())
    return sorted(r for r in rows if 0 <= r < n)


@pytest.mark.parametrize("dim,heads,kv_heads,start,n,kernel", CASES)
def test_dispatch_sweep_against_oracle(dim, heads, kv_heads, start, n, kernel):
    hd = dim // heads
    rows = start + n + 2
    theta = 1e4 if (start + n) % 2 else 5e5
    cfg = orc.Cfg(dim, heads, kv_heads, rows, 1, theta)
    seed = [131, dim, heads, kv_heads, start, n]
    q = gen(seed + [0], (rows, dim))
    k = gen(seed + [1], (rows, cfg.kv_dim))
    v = gen(seed + [2], (rows, cfg.kv_dim))
    om = orc.OracleModel(cfg)
    with P.AttentionContext(dim, heads, kv_heads, rows, 1, theta) as ctx:
        took = ctx.prefill_kernel(start, n)
        splits = [ctx.decode_splits(p + 1) for p in (start + n, start + n + 1)]
        log(f"sweep hd {hd} heads {heads}/{kv_heads} start {start} n {n}: prefill {took}, "
            f"decode (splits, tile) {splits}")
        if kernel is not None:
            assert took == kernel
        if start:
            ctx.prefill(0, 0, q[:start], k[:start], v[:start])
            om.append(0, 0, k[:start], v[:start])
        b = slice(start, start + n)
        g = ctx.prefill(0, start, q[b], k[b], v[b])
        flop = 4.0 * heads * hd * n * (start + (n + 1) / 2)
        if flop <= FULL_ORACLE_FLOP:
            ref = om.prefill(0, start, q[b], k[b], v[b])
            assert_close(g, ref, what=f"prefill rows {start}..{start + n - 1}")
        else:
            om.append(0, start, k[b], v[b])
            for r in sample_rows(n, sum(seed)):
                p = start + r
                ref = om.decode(0, p, q[p], k[p], v[p])
                assert_close(g[r], ref, what=f"prefill row {p} (rows {start}..{start + n - 1})")
        for p in (start + n, start + n + 1):
            got = ctx.decode(0, p, q[p], k[p], v[p])
            ref = om.decode(0, p, q[p], k[p], v[p])
            assert_close(got, ref, what=f"decode at {p}")
        assert_bitwise(ctx.kv_read(0, 0, 0, rows), om.k_cache(0)[:rows], "K rows")
        assert_bitwise(ctx.kv_read(0, 1, 0, rows), om.v_cache(0)[:rows], "V rows")


def test_prefill_kernel_query_rejects_batches_the_prefill_rejects():
    # the same checks and codes as slm_attn_prefill (SLM_ERR_BATCH); a batch
    # ending at max_seq_len is accepted
    with P.AttentionContext(4096, 32, 8, 300, 1, 5e5) as ctx:
        assert ctx.prefill_kernel(0, 300) == "paired_two_heads"
        for start, n in ((0, 0), (-1, 4), (290, 11), (300, 1)):
            with pytest.raises(P.SlmAttnError) as e:
                ctx.prefill_kernel(start, n)
            assert e.value.code == P.ERR_BATCH, (start, n)
