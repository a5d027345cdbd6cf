"""The no-allocation decode entry point (slm_attn_decode_xb_dev_noalloc)
against the allocating one (slm_attn_decode_xb_dev) on the same inputs.

Both run the same kernels in the same order, so the outputs and the appended
K/V rows must be identical bit for bit.  Two calls in a row, the second at a
smaller position (fewer cache rows, fewer split partials in the shared
scratch), so stale contents of the first call would show.  A shape whose
split partials exceed the scratch is refused with SLM_ERR_SHAPE before any
launch.
"""
import sys

import numpy as np
import pytest

from oracle import py_oracle as orc
from slm_testlib import assert_bitwise, gen, load_product

P = load_product()
pytestmark = pytest.mark.gpu
torch = pytest.importorskip("torch")

SCRATCH_FLOATS = 1 << 18


def log(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def need_floats(ctx, dim, heads, kv_dim, hd, pos):
    ns, _ = ctx.decode_splits(pos + 1)
    return dim + 2 * kv_dim + ns * heads * (hd + 2), ns


def run_pair(dim, heads, kv_heads, msl, positions, seed):
    hd = dim // heads
    kvd = hd * kv_heads
    wq = orc.quantize_q4_0(gen([seed, 1], (dim, dim)) * np.float32(0.1))
    wk = orc.quantize_q4_0(gen([seed, 2], (kvd, dim)) * np.float32(0.1))
    wv = orc.quantize_q4_0(gen([seed, 3], (kvd, dim)) * np.float32(0.1))
    with P.Q4Matrix(wq, dim, dim) as Wq, P.Q4Matrix(wk, kvd, dim) as Wk, \
            P.Q4Matrix(wv, kvd, dim) as Wv, \
            P.AttentionContext(dim, heads, kv_heads, msl, 1, 5e5) as a, \
            P.AttentionContext(dim, heads, kv_heads, msl, 1, 5e5) as b:
        for pos in positions:
            need, ns = need_floats(a, dim, heads, kvd, hd, pos)
            log(f"dim {dim} heads {heads}/{kv_heads} pos {pos}: {ns} splits, "
                f"{need} scratch floats")
            kr, vr = gen([seed, 4, pos], (pos, kvd)), gen([seed, 5, pos], (pos, kvd))
            for ctx in (a, b):
                ctx.kv_write(0, 0, 0, kr)
                ctx.kv_write(0, 1, 0, vr)
            xb = torch.from_numpy(gen([seed, 6, pos], dim)).cuda()
            oa = torch.empty(dim, device="cuda")
            ob = torch.full((dim,), float("nan"), device="cuda")
            a.decode_xb_dev(0, pos, xb.data_ptr(), Wq, Wk, Wv, oa.data_ptr())
            a.sync()
            if need > SCRATCH_FLOATS:
                with pytest.raises(P.SlmAttnError) as e:
                    b.decode_xb_dev_noalloc(0, pos, xb.data_ptr(), Wq, Wk, Wv, ob.data_ptr())
                assert e.value.code == P.ERR_SHAPE and "scratch" in e.value.message
                assert torch.isnan(ob).all()
                continue
            b.decode_xb_dev_noalloc(0, pos, xb.data_ptr(), Wq, Wk, Wv, ob.data_ptr())
            b.sync()
            assert_bitwise(ob.cpu().numpy(), oa.cpu().numpy(), f"out at pos {pos}")
            assert_bitwise(b.kv_read(0, 0, pos, 1), a.kv_read(0, 0, pos, 1), f"K row {pos}")
            assert_bitwise(b.kv_read(0, 1, pos, 1), a.kv_read(0, 1, pos, 1), f"V row {pos}")


def test_noalloc_decode_matches_allocating_entry_point():
    # Llama-3-8B head shape: 6000 rows (split-K with a merge), then 700
    run_pair(4096, 32, 8, 8192, (6000, 700), 91)


def test_noalloc_decode_small_then_refused_when_scratch_too_small():
    # head_dim 256 over one KV head: one workgroup group, so the split count
    # grows to one split per CU and its partials outgrow the scratch at long
    # positions; the first position fits, the last is refused (or, on a part
    # with few CUs, fits and is compared)
    run_pair(1024, 4, 1, 8192, (100, 8191, 40), 92)
