"""GPU parity: the HIP path through the C ABI against the CPU oracle.

Bar: KV-cache rows and RoPE tables bit for bit; attention outputs within
max-abs 1e-4 and max-rel 1e-3 (relative error floored at |ref| = 0.1).
Small workloads run in full; the large ones (4096-row prefill, 131072-position
decode) are checked on stated rows/steps with the oracle over the same cache,
plus size-independent relations (prefill row == decode, split invariance,
determinism).
"""
import os
import subprocess
import sys
import tempfile

import numpy as np
import pytest

from oracle import py_oracle as orc
from slm_testlib import (WORKLOADS, Workload, assert_bitwise, assert_close, gen, layer_inputs,
                         load_product, paired_blocks, paired_dma, paired_register,
                         prefilled_rows, takes_key_splits)

P = load_product()
pytestmark = pytest.mark.gpu


def log(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def make_ctx(w):
    return P.AttentionContext(w.dim, w.num_heads, w.num_kv_heads, w.max_seq_len, w.num_layers,
                              w.theta)


@pytest.mark.parametrize("key", ["ref_mha", "ref_gqa", "c0", "c1", "c2"])
def test_workload_full_parity(key):
    w = WORKLOADS[key]
    log(f"workload {key}: {w}")
    cfg = w.cfg()
    with make_ctx(w) as ctx:
        om = orc.OracleModel(cfg)
        c, s = ctx.rope_tables()
        assert_bitwise(c, om.cos, "cos table")
        assert_bitwise(s, om.sin, "sin table")
        for layer in range(w.num_layers):
            q, k, v = layer_inputs(w, layer)
            n = w.prefill
            g = ctx.prefill(layer, 0, q[:n], k[:n], v[:n])
            r = om.prefill(layer, 0, q[:n], k[:n], v[:n])
            assert_close(g, r, what=f"{key} layer {layer} prefill")
            for st in range(w.decode):
                p = n + st
                g = ctx.decode(layer, p, q[p], k[p], v[p])
                r = om.decode(layer, p, q[p], k[p], v[p])
                assert_close(g, r, what=f"{key} layer {layer} decode pos {p}")
            rows = n + w.decode
            assert_bitwise(ctx.kv_read(layer, 0, 0, rows), om.k_cache(layer)[:rows], "K rows")
            assert_bitwise(ctx.kv_read(layer, 1, 0, rows), om.v_cache(layer)[:rows], "V rows")


def test_smollm2_shape_gqa3():
    # SmolLM2-135M shape (9 heads over 3 KV heads, hd 64, theta 1e5): the first
    # and last of its 30 layers, 512-row prefill then 256 decode steps
    w = WORKLOADS["c3"]
    cfg = w.cfg()
    with make_ctx(w) as ctx:
        om = orc.OracleModel(cfg)
        for layer in (0, w.num_layers - 1):
            log(f"c3 layer {layer}")
            q, k, v = layer_inputs(w, layer)
            n = w.prefill
            g = ctx.prefill(layer, 0, q[:n], k[:n], v[:n])
            r = om.prefill(layer, 0, q[:n], k[:n], v[:n])
            assert_close(g, r, what=f"c3 layer {layer} prefill")
            for st in range(w.decode):
                p = n + st
                g = ctx.decode(layer, p, q[p], k[p], v[p])
                if st % 16 == 0 or st == w.decode - 1:
                    r = om.decode(layer, p, q[p], k[p], v[p])
                    assert_close(g, r, what=f"c3 layer {layer} decode pos {p}")
                else:
                    om.append(layer, p, k[p], v[p])
            rows = n + w.decode
            assert_bitwise(ctx.kv_read(layer, 0, 0, rows), om.k_cache(layer)[:rows], "K rows")
            assert_bitwise(ctx.kv_read(layer, 1, 0, rows), om.v_cache(layer)[:rows], "V rows")


def test_llama3_shape_prefill4096_then_decode():
    w = WORKLOADS["c4"]
    cfg = w.cfg()
    q, k, v = layer_inputs(w, 0)
    n = w.prefill
    with make_ctx(w) as ctx:
        log("c4 prefill 4096")
        g = ctx.prefill(0, 0, q[:n], k[:n], v[:n])
        om = orc.OracleModel(cfg)
        om.append(0, 0, k[:n], v[:n])
        assert_bitwise(ctx.kv_read(0, 0, 0, n), om.k_cache(0)[:n], "K rows")
        assert_bitwise(ctx.kv_read(0, 1, 0, n), om.v_cache(0)[:n], "V rows")
        for b in (0, 1, 15, 16, 17, 63, 64, 127, 128, 255, 1000, 2047, 2048, 3333, 4095):
            assert_close(g[b], om.attend(0, q[b], b), what=f"c4 prefill row {b}")
        log("c4 decode 128")
        for st in range(w.decode):
            p = n + st
            gd = ctx.decode(0, p, q[p], k[p], v[p])
            om.append(0, p, k[p], v[p])
            if st in (0, 1, 63, w.decode - 1):
                assert_close(gd, om.attend(0, q[p], p), what=f"c4 decode pos {p}")
        rows = n + w.decode
        assert_bitwise(ctx.kv_read(0, 0, n, w.decode), om.k_cache(0)[n:rows], "K rows")


def test_llama3_shape_prefill4096_continued_at_300():
    # A 4096-row prefill continued at start 300: on 256 CUs this size and
    # shape take the prefill kernel that stages K/V tiles by DMA, whose key
    # range then starts past the first tile boundary.  K/V rows bit for bit,
    # sampled rows against the oracle over the same cache.
    w = WORKLOADS["c4"]
    cfg = w.cfg()
    s0, n = 300, 4096
    rows = s0 + n
    q = gen([91, w.dim], (rows, w.dim))
    k = gen([92, w.dim], (rows, w.kv_dim))
    v = gen([93, w.dim], (rows, w.kv_dim))
    with make_ctx(w) as ctx:
        log(f"c4 shape: prefill {s0} rows, then {n} more at start {s0}")
        ctx.prefill(0, 0, q[:s0], k[:s0], v[:s0])
        g = ctx.prefill(0, s0, q[s0:], k[s0:], v[s0:])
        om = orc.OracleModel(cfg)
        om.append(0, 0, k, v)
        assert_bitwise(ctx.kv_read(0, 0, 0, rows), om.k_cache(0)[:rows], "K rows")
        assert_bitwise(ctx.kv_read(0, 1, 0, rows), om.v_cache(0)[:rows], "V rows")
        for b in (0, 1, 15, 16, 19, 20, 31, 32, 1000, 2047, 4095):
            p = s0 + b
            assert_close(g[b], om.attend(0, q[p], p), what=f"continued prefill row {p}")


@pytest.mark.parametrize("dim,heads,kv_heads,start,n", [(4096, 32, 8, 7, 4111),
                                                        (8192, 64, 8, 0, 2100)])
def test_dma_prefill_unaligned_against_oracle(dim, heads, kv_heads, start, n):
    # The DMA-staged prefill kernel at row counts that leave a partial last
    # 32-row query block (4111 rows: 15 in the last block, whose second wave
    # has none) and with two head groups per KV head (kv_mul 8).  K/V rows bit
    # for bit; rows around the block edges and the last rows against the
    # oracle over the same cache.
    w = Workload("dma-unaligned", dim, heads, kv_heads, start + n, 1, 5e5, n, 0)
    cfg = w.cfg()
    rows = start + n
    q = gen([94, dim], (rows, dim))
    k = gen([95, dim], (rows, w.kv_dim))
    v = gen([96, dim], (rows, w.kv_dim))
    with make_ctx(w) as ctx:
        log(f"DMA prefill {heads}/{kv_heads} heads: {n} rows at start {start}")
        if start:
            ctx.prefill(0, 0, q[:start], k[:start], v[:start])
        g = ctx.prefill(0, start, q[start:], k[start:], v[start:])
        om = orc.OracleModel(cfg)
        om.append(0, 0, k, v)
        assert_bitwise(ctx.kv_read(0, 0, 0, rows), om.k_cache(0)[:rows], "K rows")
        assert_bitwise(ctx.kv_read(0, 1, 0, rows), om.v_cache(0)[:rows], "V rows")
        for b in (0, 1, 15, 16, 31, 32, 33, 1000, n - 33, n - 21, n - 20, n - 17, n - 16,
                  n - 15, n - 2, n - 1):
            p = start + b
            assert_close(g[b], om.attend(0, q[p], p), what=f"DMA prefill row {p}")


@pytest.mark.parametrize("start,n", [(0, 512), (0, 1000), (333, 700), (3000, 64), (40, 30),
                                     (31, 2)])
def test_llama3_shape_short_prefill_every_row(start, n):
    # Llama-3-8B-shape prefills below the size that takes the DMA-staged
    # kernel (the register-prefetch kernel, 16-row blocks of four heads),
    # from the start of the cache and continued past it at tile-unaligned
    # starts (a block's first rows then share their diagonal tile with the
    # previous call's rows).  Every row against the oracle, K/V rows bit for
    # bit.
    dim, heads, kvh = 4096, 32, 8
    rows = start + n
    cfg = orc.Cfg(dim, heads, kvh, rows, 1, 5e5)
    q = gen([94, start, n], (rows, dim))
    k = gen([95, start, n], (rows, cfg.kv_dim))
    v = gen([96, start, n], (rows, cfg.kv_dim))
    om = orc.OracleModel(cfg)
    with P.AttentionContext(dim, heads, kvh, rows, 1, 5e5) as ctx:
        log(f"llama3 shape: prefill {n} rows at start {start}")
        if start:
            ctx.prefill(0, 0, q[:start], k[:start], v[:start])
            om.append(0, 0, k[:start], v[:start])
        g = ctx.prefill(0, start, q[start:], k[start:], v[start:])
        ref = om.prefill(0, start, q[start:], k[start:], v[start:])
        assert_bitwise(ctx.kv_read(0, 0, 0, rows), om.k_cache(0)[:rows], "K rows")
        assert_bitwise(ctx.kv_read(0, 1, 0, rows), om.v_cache(0)[:rows], "V rows")
        assert_close(g, ref, what=f"prefill of {n} rows at {start}")


@pytest.mark.parametrize("dim,heads,kv_heads,start,n,variant", [
    (4096, 32, 8, 0, 256, "h1k4"),     # 16 blocks: 8 pairs of one head
    (4096, 32, 32, 17, 256, "h1k4"),   # MHA (the Llama-2-7B layout), unaligned start
    (2048, 16, 16, 0, 300, "h1k4"),    # MHA, 19 blocks: the middle pair's second block is its first
    (1024, 8, 4, 0, 700, "h1k4"),      # kv_mul 2, 44 blocks
    (4096, 32, 8, 0, 300, "h2k2"),     # 19 blocks, two heads
    (4096, 32, 8, 37, 471, "h2k2"),    # unaligned start and a partial last block
    (4096, 32, 8, 1000, 512, "h2k2"),  # a long prefix: every block's keys span 48 tiles
    (2048, 16, 2, 0, 777, "h2k2"),     # kv_mul 8: two head pairs per KV head, 49 blocks
    (1024, 8, 4, 13, 1500, "h2k2"),    # kv_mul 2
])
def test_prefill_paired_blocks_every_row(dim, heads, kv_heads, start, n, variant):
    # every row against the oracle, K/V rows bit for bit
    assert paired_blocks(dim, heads, kv_heads, n) == variant
    rows = start + n
    cfg = orc.Cfg(dim, heads, kv_heads, rows, 1, 5e5)
    q = gen([102, start, n], (rows, dim))
    k = gen([103, start, n], (rows, cfg.kv_dim))
    v = gen([104, start, n], (rows, cfg.kv_dim))
    om = orc.OracleModel(cfg)
    with P.AttentionContext(dim, heads, kv_heads, rows, 1, 5e5) as ctx:
        log(f"paired-block prefill {heads}/{kv_heads} heads: {n} rows at start {start}")
        assert ctx.prefill_kernel(start, n) == {"h1k4": "paired_one_head",
                                                "h2k2": "paired_two_heads"}[variant]
        if start:
            ctx.prefill(0, 0, q[:start], k[:start], v[:start])
            om.append(0, 0, k[:start], v[:start])
        g = ctx.prefill(0, start, q[start:], k[start:], v[start:])
        ref = om.prefill(0, start, q[start:], k[start:], v[start:])
        assert_bitwise(ctx.kv_read(0, 0, 0, rows), om.k_cache(0)[:rows], "K rows")
        assert_bitwise(ctx.kv_read(0, 1, 0, rows), om.v_cache(0)[:rows], "V rows")
        assert_close(g, ref, what=f"prefill of {n} rows at {start}")


@pytest.mark.parametrize("dim,heads,kv_heads,start,n", [
    (4096, 32, 8, 5, 2040),    # 128 blocks, 512 workgroups (two per CU), a partial last block
    (2048, 16, 4, 0, 1520),    # 95 blocks: the middle pair's second block is its first
    (2048, 16, 2, 19, 1100),   # kv_mul 8: two workgroups' heads share each KV head
])
def test_prefill_paired_dma_every_row(dim, heads, kv_heads, start, n):
    # every row against the oracle, K/V rows bit for bit
    assert paired_dma(dim, heads, kv_heads, n)
    rows = start + n
    cfg = orc.Cfg(dim, heads, kv_heads, rows, 1, 5e5)
    q = gen([105, start, n], (rows, dim))
    k = gen([106, start, n], (rows, cfg.kv_dim))
    v = gen([107, start, n], (rows, cfg.kv_dim))
    om = orc.OracleModel(cfg)
    with P.AttentionContext(dim, heads, kv_heads, rows, 1, 5e5) as ctx:
        log(f"paired-block DMA prefill {heads}/{kv_heads} heads: {n} rows at start {start}")
        assert ctx.prefill_kernel(start, n) == "dma_paired"
        if start:
            ctx.prefill(0, 0, q[:start], k[:start], v[:start])
            om.append(0, 0, k[:start], v[:start])
        g = ctx.prefill(0, start, q[start:], k[start:], v[start:])
        ref = om.prefill(0, start, q[start:], k[start:], v[start:])
        assert_bitwise(ctx.kv_read(0, 0, 0, rows), om.k_cache(0)[:rows], "K rows")
        assert_bitwise(ctx.kv_read(0, 1, 0, rows), om.v_cache(0)[:rows], "V rows")
        assert_close(g, ref, what=f"prefill of {n} rows at {start}")


@pytest.mark.parametrize("dim,heads,kv_heads,start,n", [
    (3072, 32, 8, 0, 1000),   # hd 96: 63 blocks, the middle pair's second block is its first
    (3072, 32, 8, 9, 2040),   # hd 96: 128 blocks, two workgroups per CU, partial last block
    (2048, 32, 8, 0, 2048),   # hd 64 (the Llama-3.2-1B layout)
    (1024, 32, 8, 3, 1015),   # hd 32: 64 blocks, the last partial
    (512, 32, 8, 0, 2048),    # hd 16
])
def test_prefill_paired_register_every_row(dim, heads, kv_heads, start, n):
    # every row against the oracle, K/V rows bit for bit
    assert paired_register(dim, heads, kv_heads, start, n)
    rows = start + n
    cfg = orc.Cfg(dim, heads, kv_heads, rows, 1, 5e5)
    q = gen([108, start, n], (rows, dim))
    k = gen([109, start, n], (rows, cfg.kv_dim))
    v = gen([110, start, n], (rows, cfg.kv_dim))
    om = orc.OracleModel(cfg)
    with P.AttentionContext(dim, heads, kv_heads, rows, 1, 5e5) as ctx:
        log(f"paired-block register prefill hd {dim // heads}: {n} rows at start {start}")
        assert ctx.prefill_kernel(start, n) == "paired_four_heads"
        if start:
            ctx.prefill(0, 0, q[:start], k[:start], v[:start])
            om.append(0, 0, k[:start], v[:start])
        g = ctx.prefill(0, start, q[start:], k[start:], v[start:])
        ref = om.prefill(0, start, q[start:], k[start:], v[start:])
        assert_bitwise(ctx.kv_read(0, 0, 0, rows), om.k_cache(0)[:rows], "K rows")
        assert_bitwise(ctx.kv_read(0, 1, 0, rows), om.v_cache(0)[:rows], "V rows")
        assert_close(g, ref, what=f"prefill of {n} rows at {start}")


def test_long_context_decode_131072():
    w = WORKLOADS["c5"]
    cfg = w.cfg()
    q, k, v = layer_inputs(w, 0)
    om = orc.OracleModel(cfg)
    pre = w.prefilled
    log("c5 prefill cache rows")
    blk = 16384
    with make_ctx(w) as ctx:
        for p0 in range(0, pre, blk):
            kr = prefilled_rows(w, 0, 0, p0, blk)
            vr = prefilled_rows(w, 0, 1, p0, blk)
            om.k_cache(0)[p0:p0 + blk] = kr
            om.v_cache(0)[p0:p0 + blk] = vr
            ctx.kv_write(0, 0, p0, kr)
            ctx.kv_write(0, 1, p0, vr)
        log("c5 decode 64 steps")
        for st in range(w.decode):
            p = pre + st
            gd = ctx.decode(0, p, q[st], k[st], v[st])
            if st in (0, w.decode - 1):
                r = om.decode(0, p, q[st], k[st], v[st])
                assert_close(gd, r, what=f"c5 decode pos {p}")
            else:
                om.append(0, p, k[st], v[st])
        assert_bitwise(ctx.kv_read(0, 0, pre, w.decode), om.k_cache(0)[pre:pre + w.decode])
        assert_bitwise(ctx.kv_read(0, 0, pre - 3, 3), om.k_cache(0)[pre - 3:pre])


def test_prefill_rows_equal_sequential_decode_and_chunked_prefill():
    # transformer.rs:1269-1358 relation, here elementwise: batched prefill rows
    # equal token-by-token decode; a prefill continued at start > 0 equals one
    # longer prefill; caches are bit-identical
    w = WORKLOADS["c0"]
    q, k, v = layer_inputs(w, 0)
    n = 40
    q, k, v = gen(7, (n, w.dim)), gen(8, (n, w.kv_dim)), gen(9, (n, w.kv_dim))
    with make_ctx(w) as a, make_ctx(w) as b, make_ctx(w) as c:
        ga = a.prefill(0, 0, q, k, v)
        gb = np.stack([b.decode(0, p, q[p], k[p], v[p]) for p in range(n)])
        assert_close(ga, gb, what="prefill vs decode")
        c.prefill(0, 0, q[:13], k[:13], v[:13])
        gc = c.prefill(0, 13, q[13:], k[13:], v[13:])
        assert_close(gc, ga[13:], what="chunked prefill")
        for ctx in (b, c):
            assert_bitwise(ctx.kv_read(0, 0, 0, n), a.kv_read(0, 0, 0, n))
            assert_bitwise(ctx.kv_read(0, 1, 0, n), a.kv_read(0, 1, 0, n))


def test_decode_deterministic_and_split_invariant():
    torch = pytest.importorskip("torch")
    w = WORKLOADS["c4"]
    pos = 6000
    with make_ctx(w) as ctx:
        ns, tile = ctx.decode_splits(pos + 1)
        log(f"splits at {pos + 1}: {ns}, tiles of {tile} rows")
        assert ns > 1
        for p0 in range(0, pos + 1, 2048):
            m = min(2048, pos + 1 - p0)
            ctx.kv_write(0, 0, p0, gen([1, p0], (m, w.kv_dim)))
            ctx.kv_write(0, 1, p0, gen([2, p0], (m, w.kv_dim)))
        q2 = torch.from_numpy(np.stack([gen(4, w.dim), gen(3, w.dim)])).cuda()
        qd = q2[1]
        out1 = torch.empty(w.dim, device="cuda")
        out2 = torch.empty(w.dim, device="cuda")
        out3 = torch.empty((2, w.dim), device="cuda")
        ctx.attend_dev(0, pos, qd.data_ptr(), out1.data_ptr())
        ctx.attend_dev(0, pos, qd.data_ptr(), out2.data_ptr())
        # the same row through the prefill kernel (no split): rows at pos-1, pos
        ctx.attend_batch_dev(0, pos - 1, 2, q2.data_ptr(), out3.data_ptr())
        ctx.sync()
        o1, o2, o3 = out1.cpu().numpy(), out2.cpu().numpy(), out3[1].cpu().numpy()
        assert_bitwise(o1, o2, "repeat")
        assert_close(o1, o3, what="split-K decode vs prefill row")
        kc = ctx.kv_read(0, 0, 0, pos + 1)
        vc = ctx.kv_read(0, 1, 0, pos + 1)
        cfg = w.cfg()
        kfull = np.zeros((cfg.max_seq_len, cfg.kv_dim), np.float32)
        vfull = np.zeros_like(kfull)
        kfull[:pos + 1], vfull[:pos + 1] = kc, vc
        assert_close(o1, orc.attention(gen(3, w.dim), kfull, vfull, cfg, pos), what="vs oracle")


def test_device_entry_points_match_oracle():
    torch = pytest.importorskip("torch")
    w = WORKLOADS["c1"]
    cfg = w.cfg()
    n = 24
    q, k, v = gen(51, (n, w.dim)), gen(52, (n, w.kv_dim)), gen(53, (n, w.kv_dim))
    om = orc.OracleModel(cfg)
    with make_ctx(w) as ctx:
        kd, vd = torch.from_numpy(k).cuda(), torch.from_numpy(v).cuda()
        ctx.kv_append_dev(1, 0, n, kd.data_ptr(), vd.data_ptr())
        om.append(1, 0, k, v)
        # apply_rope_cached on device rows, bit for bit
        qd = torch.from_numpy(q).cuda()
        ctx.rope_apply_dev(qd.data_ptr(), n, w.dim, 0)
        ctx.sync()
        q_rot = np.stack([om.rotated_q(q[b], b) for b in range(n)])
        assert_bitwise(qd.cpu().numpy(), q_rot, "rope_apply_dev")
        assert_bitwise(ctx.kv_read(1, 0, 0, n), om.k_cache(1)[:n], "kv_append_dev K")
        assert_bitwise(ctx.kv_read(1, 1, 0, n), om.v_cache(1)[:n], "kv_append_dev V")
        # causal_multi_head_attention_jit on the rotated q
        out = torch.empty(w.dim, device="cuda")
        ctx.attend_dev(1, n - 1, qd[n - 1].data_ptr(), out.data_ptr())
        ctx.sync()
        ref = orc.attention(q_rot[n - 1], om.k_cache(1), om.v_cache(1), cfg, n - 1)
        assert_close(out.cpu().numpy(), ref, what="attend_dev")
        # batched rows on rotated q
        outb = torch.empty((n, w.dim), device="cuda")
        ctx.attend_batch_dev(1, 0, n, qd.data_ptr(), outb.data_ptr())
        ctx.sync()
        for b in (0, 5, n - 1):
            ref = orc.attention(q_rot[b], om.k_cache(1), om.v_cache(1), cfg, b)
            assert_close(outb[b].cpu().numpy(), ref, what=f"attend_batch_dev row {b}")
        # whole block on device pointers, on a caller-provided torch stream
        s = torch.cuda.Stream()
        ctx.set_stream(s.cuda_stream)
        assert ctx.get_stream() == s.cuda_stream
        q2, k2, v2 = gen(54, w.dim), gen(55, w.kv_dim), gen(56, w.kv_dim)
        t = [torch.from_numpy(x).cuda() for x in (q2, k2, v2)]
        torch.cuda.synchronize()
        o = torch.empty(w.dim, device="cuda")
        ctx.decode_dev(1, n, t[0].data_ptr(), t[1].data_ptr(), t[2].data_ptr(), o.data_ptr())
        s.synchronize()
        ctx.set_stream(None)
        assert_close(o.cpu().numpy(), om.decode(1, n, q2, k2, v2), what="decode_dev")


@pytest.mark.parametrize("shape,positions", [
    ((256, 4, 4, 512), (0, 7, 300, 511)),          # C1's head shape (MHA, hd 64)
    ((576, 9, 3, 1024), (0, 33, 257, 1000)),       # SmolLM2-135M (GQA kv_mul 3, hd 64)
    ((4096, 32, 8, 1200), (0, 255, 256, 1199)),    # Llama-3-8B (GQA kv_mul 4, hd 128): 1 and 9+ splits
])
def test_attend_against_scalar_attention(shape, positions):
    """The device attention against causal_multi_head_attention, the
    reference's scalar path (transformer.rs:214-271: sequential max, libm
    expf, sequential sum), directly rather than through the JIT restatement:
    the reference holds its layer outputs to 1e-4 of that path
    (transformer.rs:1000-1099), and so does this test."""
    torch = pytest.importorskip("torch")
    dim, heads, kvh, msl = shape
    w = Workload("scalar-check", dim, heads, kvh, msl, 1, 1e4, 0, 0, seed=0x5EED0020 + dim)
    cfg = w.cfg()
    rows = max(positions) + 1
    kc = np.zeros((msl, w.kv_dim), np.float32)
    vc = np.zeros((msl, w.kv_dim), np.float32)
    kc[:rows] = prefilled_rows(w, 0, 0, 0, rows)
    vc[:rows] = prefilled_rows(w, 0, 1, 0, rows)
    with make_ctx(w) as ctx:
        ctx.kv_write(0, 0, 0, kc[:rows])
        ctx.kv_write(0, 1, 0, vc[:rows])
        for pos in positions:
            q = gen([w.seed, 7, pos], dim)
            qd = torch.from_numpy(q).cuda()
            out = torch.empty(dim, device="cuda")
            ctx.attend_dev(0, pos, qd.data_ptr(), out.data_ptr())
            ctx.sync()
            ref = orc.attention(q, kc, vc, cfg, pos, jit=False)
            ns, _ = ctx.decode_splits(pos + 1)
            log(f"{shape} pos {pos} ({ns} splits): vs scalar attention")
            assert_close(out.cpu().numpy(), ref, what=f"attend_dev vs scalar pos {pos}")


def test_error_codes_mirror_reference_asserts():
    torch = pytest.importorskip("torch")
    w = WORKLOADS["c1"]
    with make_ctx(w) as ctx:
        q, k, v = gen(1, w.dim), gen(2, w.kv_dim), gen(3, w.kv_dim)
        with pytest.raises(P.SlmAttnError) as e:
            ctx.decode(0, w.max_seq_len, q, k, v)
        assert e.value.code == P.ERR_POS
        with pytest.raises(P.SlmAttnError) as e:
            ctx.decode(w.num_layers, 0, q, k, v)
        assert e.value.code == P.ERR_LAYER
        with pytest.raises(P.SlmAttnError) as e:
            ctx.prefill(0, w.max_seq_len - 2, np.tile(q, (3, 1)), np.tile(k, (3, 1)),
                        np.tile(v, (3, 1)))
        assert e.value.code == P.ERR_BATCH
        buf = torch.zeros(4 * w.dim, device="cuda")
        base = buf.data_ptr()
        with pytest.raises(P.SlmAttnError) as e:  # out overlaps q
            ctx.decode_dev(0, 0, base, base + 4 * w.dim, base + 8 * w.dim, base + 64)
        assert e.value.code == P.ERR_ALIAS
        with pytest.raises(P.SlmAttnError) as e:  # out inside the KV region
            ctx.attend_dev(0, 0, base, ctx.kv_device_ptr())
        assert e.value.code == P.ERR_ALIAS
        with pytest.raises(P.SlmAttnError) as e:  # misaligned
            ctx.attend_dev(0, 0, base + 4, base + 8 * w.dim)
        assert e.value.code == P.ERR_ARG
        # inputs of appending calls must not be cache rows: k taken from the
        # row being appended would be rotated while other workgroups read it.
        # Staging slots 4*dim floats apart (c1: kv_dim == dim), so only the KV
        # overlap can be what is refused.
        st = torch.zeros(16 * w.dim, device="cuda")
        s0, s1, s2, s3 = (st.data_ptr() + 4 * i * 4 * w.dim for i in range(4))
        kv = ctx.kv_device_ptr()
        row3 = kv + 4 * ctx.kv_offset(0, 0, 3)
        with pytest.raises(P.SlmAttnError) as e:  # decode, k = K row 3
            ctx.decode_dev(0, 3, s0, row3, s2, s3)
        assert e.value.code == P.ERR_ALIAS and "KV cache" in e.value.message
        with pytest.raises(P.SlmAttnError) as e:  # decode, q inside the region
            ctx.decode_dev(0, 3, row3, s1, s2, s3)
        assert e.value.code == P.ERR_ALIAS and "KV cache" in e.value.message
        with pytest.raises(P.SlmAttnError) as e:  # prefill, v = V rows 0..1
            ctx.prefill_dev(0, 0, 2, s0, s1, kv + 4 * ctx.kv_offset(0, 1, 0), s3)
        assert e.value.code == P.ERR_ALIAS and "KV cache" in e.value.message
        with pytest.raises(P.SlmAttnError) as e:  # KV append from a cache row
            ctx.kv_append_dev(0, 5, 1, row3, s2)
        assert e.value.code == P.ERR_ALIAS and "KV cache" in e.value.message
        with pytest.raises(P.SlmAttnError) as e:
            ctx.kv_write(0, 2, 0, k)
        assert e.value.code == P.ERR_ARG
        assert ctx.kv_offset(1, 1, 3) == ((2 * 1 + 1) * w.max_seq_len + 3) * w.kv_dim
        assert ctx.kv_offset(2, 0, 0) == 2**64 - 1
        # the context still works after rejected calls
        out = ctx.decode(0, 0, q, k, v)
        assert_bitwise(out[:w.head_dim], v[:w.head_dim], "pos 0 output is V row 0")


def test_profile_counts_launches():
    w = WORKLOADS["c4"]
    with make_ctx(w) as ctx:
        ctx.profile(True)
        q, k, v = gen(1, (64, w.dim)), gen(2, (64, w.kv_dim)), gen(3, (64, w.kv_dim))
        ctx.prefill(0, 0, q, k, v)
        for p in range(64, 66):
            ctx.decode(0, p, q[0], k[0], v[0])
        st = ctx.profile_read()
        assert st["append"][0] == 1  # the prefill batch; decode appends in-kernel
        assert st["prefill"][0] == 1 and st["decode"][0] == 2
        assert all(ms >= 0.0 for _, ms in st.values())
        st2 = ctx.profile_read()
        assert all(cnt == 0 for cnt, _ in st2.values())


def test_cpp_host_mirror_binary():
    exe = P.PKG_DIR / "slm_host_demo"
    assert exe.exists(), "build the package first"
    w = WORKLOADS["ref_gqa"]
    cfg = w.cfg()
    npf, nd = 9, 5
    rows = npf + nd
    q, k, v = gen(61, (rows, w.dim)), gen(62, (rows, w.kv_dim)), gen(63, (rows, w.kv_dim))
    with tempfile.TemporaryDirectory() as td:
        fin, fout = os.path.join(td, "in.bin"), os.path.join(td, "out.bin")
        with open(fin, "wb") as f:
            f.write(q.tobytes() + k.tobytes() + v.tobytes())
        subprocess.run([str(exe), str(w.dim), str(w.num_heads), str(w.num_kv_heads),
                        str(w.max_seq_len), str(w.theta), str(npf), str(nd), fin, fout],
                       check=True, timeout=60)
        raw = np.fromfile(fout, dtype=np.float32)
    out = raw[:rows * w.dim].reshape(rows, w.dim)
    err = raw[rows * w.dim:].view(np.int32)[0]
    assert err == P.ERR_POS
    om = orc.OracleModel(cfg)
    ref = np.concatenate([om.prefill(0, 0, q[:npf], k[:npf], v[:npf]),
                          np.stack([om.decode(0, p, q[p], k[p], v[p]) for p in range(npf, rows)])])
    assert_close(out, ref, what="C++ host mirror")


@pytest.mark.parametrize("dim,heads,kv_heads", [
    (64, 4, 4),      # hd 16, MHA (the reference's layer test shape)
    (256, 8, 2),     # hd 32, kv_mul 4
    (288, 6, 6),     # hd 48
    (576, 9, 3),     # hd 64, kv_mul 3
    (512, 8, 4),     # hd 64, kv_mul 2
    (768, 8, 8),     # hd 96
    (2048, 16, 2),   # hd 128, kv_mul 8
    (1024, 4, 4),    # hd 256
])
@pytest.mark.parametrize("start,n", [(0, 2), (0, 37), (0, 130), (50, 5), (61, 67)])
def test_prefill_shapes_and_ragged_batches(dim, heads, kv_heads, start, n):
    msl = 200
    cfg = orc.Cfg(dim, heads, kv_heads, msl, 1, 1e4)
    log(f"prefill shape dim {dim} heads {heads}/{kv_heads} start {start} n {n}")
    kvd = cfg.kv_dim
    q = gen([71, dim, n], (start + n, dim))
    k = gen([72, dim, n], (start + n, kvd))
    v = gen([73, dim, n], (start + n, kvd))
    om = orc.OracleModel(cfg)
    with P.AttentionContext(dim, heads, kv_heads, msl, 1) as ctx:
        if start:
            ctx.prefill(0, 0, q[:start], k[:start], v[:start])
            om.append(0, 0, k[:start], v[:start])
        g = ctx.prefill(0, start, q[start:], k[start:], v[start:])
        om.append(0, start, k[start:], v[start:])
        assert_bitwise(ctx.kv_read(0, 0, 0, start + n), om.k_cache(0)[:start + n], "K rows")
        for b in sorted({0, 1, n // 2, n - 1}):
            if b < n:
                assert_close(g[b], om.attend(0, q[start + b], start + b),
                             what=f"row {b} at {start + b}")


@pytest.mark.parametrize("dim,heads,kv_heads", [
    (576, 9, 3),     # hd 64, kv_mul 3 (SmolLM2-135M)
    (1024, 16, 16),  # hd 64, MHA
    (288, 6, 6),     # hd 48 (Stories-15M)
    (512, 16, 4),    # hd 32, kv_mul 4
    (256, 16, 8),    # hd 16, kv_mul 2
])
@pytest.mark.parametrize("start,n", [(0, 300), (37, 290), (200, 77), (250, 1)])
def test_prefill_key_splits_every_row(dim, heads, kv_heads, start, n):
    # The short-prefill kernel that splits a query block's key tiles over
    # four waves (one head per workgroup): ragged row counts, a start past
    # the first tiles (so a split's first tile can mask every key of some
    # query), a single row; every row against the oracle, K/V rows bit for bit.
    assert takes_key_splits(dim, heads, kv_heads, start, n)
    rows = start + n
    cfg = orc.Cfg(dim, heads, kv_heads, rows, 1, 1e4)
    log(f"key-split prefill dim {dim} heads {heads}/{kv_heads} start {start} n {n}")
    q = gen([81, dim, n], (rows, dim))
    k = gen([82, dim, n], (rows, cfg.kv_dim))
    v = gen([83, dim, n], (rows, cfg.kv_dim))
    om = orc.OracleModel(cfg)
    with P.AttentionContext(dim, heads, kv_heads, rows, 1) as ctx:
        assert ctx.prefill_kernel(start, n) == "key_split"
        if start:
            ctx.prefill(0, 0, q[:start], k[:start], v[:start])
            om.prefill(0, 0, q[:start], k[:start], v[:start])
        g = ctx.prefill(0, start, q[start:], k[start:], v[start:])
        r = om.prefill(0, start, q[start:], k[start:], v[start:])
        assert_bitwise(ctx.kv_read(0, 0, 0, rows), om.k_cache(0)[:rows], "K rows")
        assert_bitwise(ctx.kv_read(0, 1, 0, rows), om.v_cache(0)[:rows], "V rows")
        assert_close(g, r, what=f"key-split prefill rows {start}..{rows - 1}")


DECODE_SHAPES = [
    (64, 4, 4),      # hd 16
    (256, 8, 2),     # hd 32, kv_mul 4
    (288, 6, 6),     # hd 48
    (576, 9, 3),     # hd 64, kv_mul 3
    (768, 8, 8),     # hd 96
    (4096, 32, 8),   # hd 128, kv_mul 4 (Llama-3-8B)
    (2048, 16, 2),   # hd 128, kv_mul 8
    (1536, 12, 4),   # hd 128, kv_mul 3: three heads per workgroup
    (1024, 8, 4),    # hd 128, kv_mul 2: two heads per workgroup
    (768, 6, 6),     # hd 128, MHA: one head per workgroup
    (1024, 4, 4),    # hd 256
]


@pytest.mark.parametrize("dim,heads,kv_heads", DECODE_SHAPES)
def test_decode_split_tiles_across_shapes(dim, heads, kv_heads):
    """Decode with append at positions where split ownership changes.

    Split s of n reads tiles s, s+n, ... of the cache; the split holding row p's
    tile writes row p and adds it to its state after its loop (with no cache
    tile at all when row p starts the split's only tile).  While the split count is
    below its cap there is one tile per split and the last split owns row p;
    beyond it ownership rotates.  Positions: the shortest sequence that splits,
    and, past the cap, the first row of a tile held by split 0 and by split 1,
    the last row of the last split's tile, and a row inside another split's.
    """
    with P.AttentionContext(dim, heads, kv_heads, 16, 1) as probe:
        cap, tile = probe.decode_splits(1 << 24)  # the tiling of long sequences
    msl = 3 * cap * tile + 2 * tile
    cfg = orc.Cfg(dim, heads, kv_heads, msl, 1, 1e4)
    kvd = cfg.kv_dim
    om = orc.OracleModel(cfg)
    with P.AttentionContext(dim, heads, kv_heads, msl, 1) as ctx:
        picks = {}
        for p in range(msl - 1):
            ns, t = ctx.decode_splits(p + 1)  # hd 64 picks its tile by length
            if ns == 1:
                continue
            picks.setdefault("shortest split sequence", p)
            if ns < p // t + 1:  # past the cap
                owner, row = (p // t) % ns, p % t
                for key, at in (("split 0 tile start", (0, 0)), ("split 1 tile start", (1, 0)),
                                ("last split, last row", (ns - 1, t - 1)),
                                ("another split", (min(3, ns - 1), 5 % t))):
                    if (owner, row) == at:
                        picks.setdefault(key, p)
        assert len(picks) == 5, picks
        cands = sorted(set(picks.values()))
        log(f"decode shape dim {dim} heads {heads}/{kv_heads} msl {msl}: positions {picks}")
        top = cands[-1]
        kr = gen([81, dim], (top, kvd))
        vr = gen([82, dim], (top, kvd))
        ctx.kv_write(0, 0, 0, kr)
        ctx.kv_write(0, 1, 0, vr)
        om.k_cache(0)[:top] = kr
        om.v_cache(0)[:top] = vr
        for p in cands:
            q1, k1, v1 = gen([83, p], dim), gen([84, p], kvd), gen([85, p], kvd)
            g = ctx.decode(0, p, q1, k1, v1)
            r = om.decode(0, p, q1, k1, v1)
            assert_close(g, r, what=f"decode at {p}")
            assert_bitwise(ctx.kv_read(0, 0, p, 1), om.k_cache(0)[p:p + 1], f"K row {p}")
            assert_bitwise(ctx.kv_read(0, 1, p, 1), om.v_cache(0)[p:p + 1], f"V row {p}")


# (dim, heads, kv_heads), split counts: shapes with few KV-head groups take up
# to 512/groups splits (256/groups at hd 256); above 32 splits the merge runs
# as one workgroup per head of ceil(n/32) rows of threads, up to 1024 threads
# (512 splits at hd <= 64, 256 at hd 96/128, 128 at hd 256), beyond that
# 32 splits per round
MANY_SPLITS = [
    ((128, 4, 1), (33, 512)),        # hd 32, one KV head: 2 and 16 rows of threads
    ((128, 8, 2), (256,)),           # hd 16
    ((256, 8, 2), (200,)),           # hd 32
    ((288, 6, 6), (85,)),            # hd 48 MHA: the policy's cap
    ((576, 9, 3), (48, 65, 85)),     # hd 64 GQA 3 (SmolLM2)
    ((2048, 32, 8), (40,)),          # hd 64 GQA 4
    ((768, 8, 8), (40,)),            # hd 96: 128 threads per row
    ((1024, 8, 2), (128,)),          # hd 128 GQA 4
    ((1024, 4, 1), (128, 129, 256)), # hd 256: the wide merge's limit, then rounds
]


@pytest.mark.parametrize("dim,heads,kv_heads,target",
                         [s + (t,) for s, ts in MANY_SPLITS for t in ts])
def test_decode_many_splits_against_oracle(dim, heads, kv_heads, target):
    """Decode with append at a ragged length that gives `target` splits:
    output against the oracle, the appended K/V row bit for bit, and a
    second call giving the same bits."""
    with P.AttentionContext(dim, heads, kv_heads, 16, 1) as probe:
        run = []
        for n in range(1, 1 << 18):  # the first run of lengths with `target` splits
            ns_n, t_n = probe.decode_splits(n)
            if ns_n == target:
                run.append((n, t_n))
            elif run:
                break
    assert run, f"no length gives {target} splits"
    n, tile = run[len(run) // 2]
    if n % tile == 0 and len(run) > 1:  # ragged: the last tile not full
        n, tile = run[len(run) // 2 - 1]
    p = n - 1
    msl = p + 1
    cfg = orc.Cfg(dim, heads, kv_heads, msl, 1, 1e4)
    kvd = cfg.kv_dim
    om = orc.OracleModel(cfg)
    with P.AttentionContext(dim, heads, kv_heads, msl, 1) as ctx:
        ns, t = ctx.decode_splits(p + 1)
        log(f"dim {dim} heads {heads}/{kv_heads}: decode at {p}, {ns} splits of {t}-row tiles")
        assert (ns, t) == (target, tile)
        kr = gen([91, dim, target], (p, kvd))
        vr = gen([92, dim, target], (p, kvd))
        ctx.kv_write(0, 0, 0, kr)
        ctx.kv_write(0, 1, 0, vr)
        om.k_cache(0)[:p] = kr
        om.v_cache(0)[:p] = vr
        q1, k1, v1 = gen([93, p], dim), gen([94, p], kvd), gen([95, p], kvd)
        g = ctx.decode(0, p, q1, k1, v1)
        r = om.decode(0, p, q1, k1, v1)
        assert_close(g, r, what=f"decode at {p} ({ns} splits)")
        assert_bitwise(ctx.kv_read(0, 0, p, 1), om.k_cache(0)[p:p + 1], f"K row {p}")
        assert_bitwise(ctx.kv_read(0, 1, p, 1), om.v_cache(0)[p:p + 1], f"V row {p}")
        assert_bitwise(ctx.decode(0, p, q1, k1, v1), g, f"second decode at {p}")


def pick_gb(kv_mul):
    return 4 if kv_mul % 4 == 0 else 3 if kv_mul % 3 == 0 else 2 if kv_mul % 2 == 0 else 1


# the decode kernel's base tiling per head dim: lanes per position, positions
# per lane group and iteration, waves per workgroup, and the most tiles that
# still run as one split
DECODE_BASE = {16: (2, 2, 4, 3), 32: (4, 2, 4, 3), 48: (4, 2, 4, 2), 64: (8, 2, 4, 4),
               96: (8, 2, 4, 3), 128: (16, 1, 8, 4), 256: (32, 1, 8, 4)}


def decode_plan(seq_len, heads, kv_heads, hd, cus):
    """The decode split policy, restated: (n_splits, tile rows, tiling).  A
    tiling fills the CUs with up to 8 waves per CU, one tile per split.  One
    split up to the head dim's tile limit; then, where the base tiling takes
    two positions per lane group (hd <= 96), the short tiling (one position)
    while its splits stay within 32 and one workgroup per CU; for hd 64 and
    96 the wide tiling (8-wave workgroups, one position) once the base tiles
    reach 1.5 times its split count; else the base tiling."""
    lpg, tp, nw, mt = DECODE_BASE[hd]
    kv_mul = heads // kv_heads
    groups = kv_heads * (kv_mul // pick_gb(kv_mul))

    def plan(tp_, nw_):
        span = nw_ * (64 // lpg) * tp_
        wgs = 8 * cus // nw_
        want = 1 if groups >= wgs else wgs // groups
        tiles = -(-seq_len // span)
        return min(tiles, want, 1024), span, tiles, want

    ns_b, span_b, tiles_b, _ = plan(tp, nw)
    if tiles_b <= mt:
        return 1, span_b, "base"
    if tp == 2:
        ns_s, span_s, _, _ = plan(1, nw)
        if ns_s <= 32 and ns_s * groups <= cus:
            return ns_s, span_s, "short"
    if hd in (64, 96):
        ns_w, span_w, _, want_w = plan(1, 8)
        if 2 * tiles_b >= 3 * want_w:
            return ns_w, span_w, "wide"
    return ns_b, span_b, "base"


TILING_SHAPES = [
    (576, 9, 3),      # hd 64, SmolLM2-135M: GQA 3
    (2048, 32, 8),    # hd 64, the Llama-3.2-1B layout: GQA 4
    (1024, 16, 8),    # hd 64, GQA 2
    (1024, 16, 16),   # hd 64, MHA with 16 KV heads (short would take 272 workgroups)
    (2048, 32, 32),   # hd 64, MHA with 32 KV heads
    (256, 4, 4),      # hd 64, MHA with 4 KV heads (the reference's synthetic model)
    (3072, 32, 8),    # hd 96, GQA 4
    (768, 8, 8),      # hd 96, MHA
    (288, 6, 6),      # hd 48, Stories-15M
    (1536, 32, 8),    # hd 48, GQA 4
    (1024, 32, 8),    # hd 32, GQA 4
    (256, 16, 4),     # hd 16, GQA 4
    (4096, 32, 8),    # hd 128, Llama-3-8B: one tiling
    (1024, 4, 4),     # hd 256: one tiling
]


@pytest.mark.parametrize("dim,heads,kv_heads", TILING_SHAPES)
def test_decode_tilings_against_oracle(dim, heads, kv_heads):
    """The decode tiling and split count picked by length.  The policy at
    every length up to 300 rows past its last change of tiling against
    decode_plan;
    then decode with append at the first and last length of each run of one
    (tiling, split count) and inside each tiling, against the oracle, with the
    appended K/V rows bit for bit."""
    torch = pytest.importorskip("torch")
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    hd = dim // heads
    last = "wide" if hd in (64, 96) else "base"  # the regime long sequences end in
    runs = []  # [first length, last length, (ns, tile, tiling)]
    since = 0  # where the tiling last changed
    with P.AttentionContext(dim, heads, kv_heads, 16, 1) as probe:
        n = 1
        while True:
            want = decode_plan(n, heads, kv_heads, hd, cus)
            got = probe.decode_splits(n)
            assert got == want[:2], (n, got, want)
            if runs and runs[-1][2] == want:
                runs[-1][1] = n
            else:
                if not runs or runs[-1][2][2] != want[2] or (want[0] > 1) != (runs[-1][2][0] > 1):
                    since = n
                runs.append([n, n, want])
            if want[2] == last and want[0] > 1 and n - since > 300:
                break
            n += 1
    tilings = {r[2][2] for r in runs}
    picks = set()
    for first, end, _ in runs:
        picks |= {first, end}
    for t in tilings:
        r = max((r for r in runs if r[2][2] == t), key=lambda r: r[1] - r[0])
        mid = (r[0] + r[1]) // 2
        picks.add(mid if mid % r[2][1] else mid + 1 if mid < r[1] else mid - 1)
    # runs of one split count change every tile at short lengths: keep the
    # transitions between tilings and a sample of the rest
    keys = sorted(picks)
    trans = set()
    for a, b in zip(runs, runs[1:]):
        if a[2][2] != b[2][2]:
            trans |= {a[1], b[0]}
    sample = sorted(trans | set(keys[::max(1, len(keys) // 12)]) | {keys[-1]})
    msl = sample[-1]
    cfg = orc.Cfg(dim, heads, kv_heads, msl, 1, 1e4)
    kvd = cfg.kv_dim
    om = orc.OracleModel(cfg)
    log(f"hd {hd} {heads}/{kv_heads}: tilings {sorted(tilings)}, lengths {sample}")
    with P.AttentionContext(dim, heads, kv_heads, msl, 1) as ctx:
        top = msl - 1
        kr = gen([97, dim], (top, kvd))
        vr = gen([98, dim], (top, kvd))
        ctx.kv_write(0, 0, 0, kr)
        ctx.kv_write(0, 1, 0, vr)
        om.k_cache(0)[:top] = kr
        om.v_cache(0)[:top] = vr
        for n in sample:
            p = n - 1
            q1, k1, v1 = gen([99, p], dim), gen([100, p], kvd), gen([101, p], kvd)
            g = ctx.decode(0, p, q1, k1, v1)
            r = om.decode(0, p, q1, k1, v1)
            assert_close(g, r, what=f"decode at {p} ({decode_plan(n, heads, kv_heads, hd, cus)})")
            assert_bitwise(ctx.kv_read(0, 0, p, 1), om.k_cache(0)[p:p + 1], f"K row {p}")
            assert_bitwise(ctx.kv_read(0, 1, p, 1), om.v_cache(0)[p:p + 1], f"V row {p}")


def test_calibration_helpers_report_plausible_rates():
    r = P.calibrate_mfma_f32(iters=4000)
    log(f"fp32 MFMA {r['tflops']:.1f} TFLOP/s")
    assert 20.0 < r["tflops"] < 200.0
    gbs = P.calibrate_hbm_read(1 << 30, nontemporal=True)
    log(f"HBM read {gbs:.0f} GB/s")
    assert 500.0 < gbs < 10000.0
