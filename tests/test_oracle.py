"""Pins the CPU oracle (oracle/slm_oracle.c) before it is trusted as the checker.

The reference ships no golden vectors for this path (its tests are
differential), so each oracle function is pinned by what the mathematics
fixes or by the reference's own test relations and bounds:

  function                 pinned by
  -----------------------  ---------------------------------------------------
  orc_rope_tables          pos 0 gives cos 1 / sin 0 exactly; every entry
                           within 1 ulp of f64 cos/sin of the f32 angle; freq
                           within 2 ulp of f64 theta^-(2j/hd)
  orc_apply_rope_cached    equal bit for bit to apply_rope_in_place (the
                           reference's own test path, transformer.rs:1053);
                           pair norms kept; <R(a)q, R(b)k> depends on a-b only;
                           f64 rotation within 2 ulp-scale
  orc_jit_exp              e(0) == 1; relative error vs exp < 3e-6 over the
                           clamp range; clamp ends
  orc_softmax_jit          engine.rs:302-371 (n=256, < 1e-5 of exact) and
                           engine.rs:418-487 (lengths 1,2,3,5,7,15,33), on the
                           reference tests' own xorshift inputs; n=1 -> 1
  orc_softmax_scalar       same bounds; agrees with the JIT path < 1e-5
  orc_attention_jit        pos 0 returns V row 0 bit for bit; q = 0 gives the
                           mean of V; one-hot V rows recover the probabilities;
                           equal q in a GQA group gives equal heads; f64 brute
                           force < 2e-6; JIT vs scalar < 1e-5
  orc_kv_offset            an independent simulation of AlignedArena
                           alloc_slice in TransformerModel::new order
  orc_decode / prefill     prefill row b == decode at start+b bit for bit
                           (transformer.rs:1269-1358 relation); f64 brute
                           force over the oracle's own cache
"""
import ctypes
import math

import numpy as np
import pytest

from oracle import py_oracle as orc
from slm_testlib import WORKLOADS, gen, layer_inputs, xorshift_f32


def ulp32(x):
    return np.spacing(np.abs(np.float32(x))).astype(np.float64)


_libm = ctypes.CDLL("libm.so.6")
_libm.powf.restype = ctypes.c_float
_libm.powf.argtypes = [ctypes.c_float, ctypes.c_float]


def _libm_powf(x, y):
    return _libm.powf(x, y)


# --------------------------------------------------------------------------- RoPE
@pytest.mark.parametrize("hd,msl,theta", [(16, 8, 1e4), (32, 64, 1e4), (48, 256, 1e4),
                                          (64, 2048, 1e5), (128, 8192, 5e5)])
def test_rope_tables_closed_forms(hd, msl, theta):
    c, s = orc.rope_tables(hd, msl, theta)
    half = hd // 2
    assert c.shape == (msl, half)
    assert np.all(c[0] == 1.0) and np.all(s[0] == 0.0)
    # freq_j = 1 / theta^(2j/hd): f32 exponent, glibc powf (what Rust's
    # f32::powf calls; numpy's float32 power differs from it by 1 ulp at some
    # exponents), f32 division
    expo = (np.arange(half, dtype=np.float32) * np.float32(2)) / np.float32(hd)
    freq64 = 1.0 / np.power(np.float64(theta), expo.astype(np.float64))
    pos = np.arange(msl, dtype=np.float32)
    freq32 = np.array([np.float32(1.0) / np.float32(_libm_powf(theta, float(e))) for e in expo],
                      np.float32)
    assert np.all(np.abs(freq32 - freq64) <= 2 * ulp32(freq64))
    ang = (pos[:, None] * freq32[None, :]).astype(np.float32)  # f32 product
    rc = np.cos(ang.astype(np.float64))
    rs = np.sin(ang.astype(np.float64))
    assert np.all(np.abs(c - rc) <= ulp32(rc) + 1e-45)
    assert np.all(np.abs(s - rs) <= ulp32(rs) + 1e-45)


def test_rope_cached_equals_in_place_and_is_a_rotation():
    hd, msl = 64, 512
    c, s = orc.rope_tables(hd, msl)
    x = gen(1, 4 * hd)
    for pos in (0, 1, 7, 300, msl - 1):
        a = orc.apply_rope_cached(x, c[pos], s[pos], hd)
        b = orc.apply_rope_in_place(x, pos, hd)
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
        # pair norms preserved
        n0 = np.hypot(x[0::2].astype(np.float64), x[1::2].astype(np.float64))
        n1 = np.hypot(a[0::2].astype(np.float64), a[1::2].astype(np.float64))
        assert np.max(np.abs(n0 - n1)) < 4e-7
        # against an f64 rotation by the table angle
        cc = np.tile(c[pos].astype(np.float64), 4)
        ss = np.tile(s[pos].astype(np.float64), 4)
        x0, x1 = x[0::2].astype(np.float64), x[1::2].astype(np.float64)
        assert np.max(np.abs(a[0::2] - (x0 * cc - x1 * ss))) < 3e-7
        assert np.max(np.abs(a[1::2] - (x0 * ss + x1 * cc))) < 3e-7
    # interleaved pairs: a rotation by pos 1 must mix x[0] with x[1], not x[hd/2]
    e0 = np.zeros(hd, np.float32)
    e0[0] = 1.0
    r = orc.apply_rope_cached(e0, c[1], s[1], hd)
    assert r[1] != 0.0 and r[hd // 2] == 0.0


def test_rope_relative_position_property():
    hd = 64
    c, s = orc.rope_tables(hd, 64)
    q, k = gen(2, hd), gen(3, hd)
    dots = []
    for a, b in [(10, 3), (20, 13), (40, 33), (7, 0)]:
        qa = orc.apply_rope_cached(q, c[a], s[a], hd).astype(np.float64)
        kb = orc.apply_rope_cached(k, c[b], s[b], hd).astype(np.float64)
        dots.append(qa @ kb)
    assert np.ptp(dots) < 1e-5


# -------------------------------------------------------------------- exp/softmax
def test_jit_exp_closed_forms_and_accuracy():
    assert orc.jit_exp(np.float32([0.0]))[0] == 1.0
    x = np.linspace(-87.0, 88.0, 200001, dtype=np.float32)
    e = orc.jit_exp(x).astype(np.float64)
    ref = np.exp(x.astype(np.float64))
    rel = np.abs(e - ref) / ref
    # degree-5 Taylor on |r| <= ln2/2 truncates at r^6/720 = 2.4e-6, plus a
    # few f32 roundings; a dropped term or a dropped ln2_lo correction
    # (1.4e-6 * n, up to 1.8e-4) lands far above this bound
    assert rel.max() < 4e-6, rel.max()
    # clamping at -87.3 and 88.3
    lo, lo2, hi, hi2 = orc.jit_exp(np.float32([-87.3, -200.0, 88.3, 200.0]))
    assert lo > 0 and lo2 == lo
    assert np.isfinite(hi) and hi2 == hi
    assert abs(float(lo) / math.exp(-87.3) - 1) < 4e-6
    assert abs(float(hi) / math.exp(88.3) - 1) < 4e-6


def _exact_softmax_f32(x):
    # the reference tests' expectation: f32 libm exp, f32 sum (engine.rs:337-340)
    m = np.max(x)
    e = np.exp((x - m).astype(np.float32)).astype(np.float32)
    ssum = np.float32(0.0)
    for v in e:
        ssum = np.float32(ssum + v)
    return e / ssum


def test_softmax_jit_matches_reference_test_n256():
    # engine.rs:302-371: pseudo_random_f32(256, 0x7788_99AA) in [-2, 2)
    x = xorshift_f32(256, 0x778899AA, -2.0, 4.0)
    out = orc.softmax_jit(x)
    ref = _exact_softmax_f32(x)
    assert np.max(np.abs(out - ref)) < 1e-5


@pytest.mark.parametrize("n", [1, 2, 3, 5, 7, 15, 33])
def test_softmax_unaligned_lengths(n):
    # engine.rs:418-487: seeds 0x1111_2222 ^ len
    x = xorshift_f32(n, 0x11112222 ^ n, -2.0, 4.0)
    ref = _exact_softmax_f32(x)
    for fn in (orc.softmax_jit, orc.softmax_scalar):
        out = fn(x)
        assert out.shape == (n,)
        assert np.max(np.abs(out - ref)) < 1e-5


def test_softmax_closed_forms():
    assert orc.softmax_jit(np.float32([3.25]))[0] == 1.0
    assert orc.softmax_scalar(np.float32([3.25]))[0] == 1.0
    for n in (4, 7, 64, 1000):
        p = orc.softmax_jit(np.full(n, 0.3, np.float32))
        assert np.all(p == p[0]) and abs(float(p[0]) - 1.0 / n) < 1e-7 / n * 8
    x = gen(9, 1001) * 8
    pj, ps = orc.softmax_jit(x), orc.softmax_scalar(x)
    assert np.max(np.abs(pj - ps)) < 1e-5
    p64 = np.exp(x.astype(np.float64) - x.max())
    p64 /= p64.sum()
    assert np.max(np.abs(pj - p64)) < 1e-6


# ---------------------------------------------------------------------- attention
def _cache(w, seed, rows):
    cfg = w.cfg()
    kc = np.zeros((cfg.max_seq_len, cfg.kv_dim), np.float32)
    vc = np.zeros_like(kc)
    kc[:rows] = gen([seed, 1], (rows, cfg.kv_dim))
    vc[:rows] = gen([seed, 2], (rows, cfg.kv_dim))
    return cfg, kc, vc


@pytest.mark.parametrize("key", ["c0", "c1", "c2", "ref_mha", "ref_gqa"])
def test_attention_vs_f64_brute_force(key):
    w = WORKLOADS[key]
    cfg, kc, vc = _cache(w, 11, w.max_seq_len)
    for pos in sorted({0, 1, 5, min(63, w.max_seq_len - 1), w.max_seq_len - 1}):
        q = gen([12, pos], cfg.dim)
        out = orc.attention(q, kc, vc, cfg, pos)
        ref = orc.attention_f64(q, kc, vc, cfg, pos)
        assert np.max(np.abs(out - ref)) < 2e-6, (key, pos)
        out_s = orc.attention(q, kc, vc, cfg, pos, jit=False)
        assert np.max(np.abs(out - out_s)) < 1e-5


def test_attention_vs_numpy_sdpa():
    # library-routine check: a plain numpy f64 softmax(QK^T/sqrt(d))V per head
    w = WORKLOADS["c0"]
    cfg, kc, vc = _cache(w, 21, 40)
    pos = 39
    q = gen(22, cfg.dim)
    out = orc.attention(q, kc, vc, cfg, pos)
    hd = cfg.head_dim
    for h in range(cfg.num_heads):
        g = h // cfg.kv_mul
        K = kc[:pos + 1, g * hd:(g + 1) * hd].astype(np.float64)
        V = vc[:pos + 1, g * hd:(g + 1) * hd].astype(np.float64)
        sc = K @ q[h * hd:(h + 1) * hd].astype(np.float64) / math.sqrt(hd)
        p = np.exp(sc - sc.max())
        p /= p.sum()
        assert np.max(np.abs(out[h * hd:(h + 1) * hd] - p @ V)) < 2e-6


def test_attention_closed_forms():
    w = WORKLOADS["c0"]  # GQA: 8 heads over 2 KV heads
    cfg, kc, vc = _cache(w, 31, w.max_seq_len)
    hd = cfg.head_dim
    q = gen(32, cfg.dim)
    # pos 0: softmax of one score is exactly 1, so out_h is V row 0 bit for bit
    out = orc.attention(q, kc, vc, cfg, 0)
    for h in range(cfg.num_heads):
        g = h // cfg.kv_mul
        assert np.array_equal(out[h * hd:(h + 1) * hd].view(np.uint32),
                              vc[0, g * hd:(g + 1) * hd].view(np.uint32))
    # q = 0: uniform weights, out is the mean of V rows 0..pos
    pos = 37
    out = orc.attention(np.zeros(cfg.dim, np.float32), kc, vc, cfg, pos)
    for h in range(cfg.num_heads):
        g = h // cfg.kv_mul
        mean = vc[:pos + 1, g * hd:(g + 1) * hd].astype(np.float64).mean(0)
        assert np.max(np.abs(out[h * hd:(h + 1) * hd] - mean)) < 1e-6
    # heads of one GQA group with the same q give the same output, and heads
    # mapped to different KV heads do not (consecutive heads share, h / kv_mul)
    qs = np.tile(gen(33, hd), cfg.num_heads)
    out = orc.attention(qs, kc, vc, cfg, pos).reshape(cfg.num_heads, hd)
    for h in range(cfg.num_heads):
        assert np.array_equal(out[h], out[(h // cfg.kv_mul) * cfg.kv_mul])
    assert not np.array_equal(out[0], out[cfg.kv_mul])


def test_attention_one_hot_values_recover_probabilities():
    # V row t = e_t recovers p_t in out[t]
    cfg = orc.Cfg(64, 1, 1, 64)
    pos = 50
    kc = gen(41, (64, 64))
    vc = np.eye(64, dtype=np.float32)
    q = gen(42, 64)
    out = orc.attention(q, kc, vc, cfg, pos)
    sc = kc[:pos + 1].astype(np.float64) @ q.astype(np.float64) / 8.0
    p = np.exp(sc - sc.max())
    p /= p.sum()
    assert np.max(np.abs(out[:pos + 1] - p)) < 1e-7
    assert np.all(out[pos + 1:] == 0.0)


def test_kv_offset_matches_arena_bump_allocation():
    # AlignedArena::alloc_slice (arena.rs:96-113): offsets rounded up to 16
    # floats; TransformerModel::new allocates LayerWorkspace, BatchWorkspace,
    # then per layer K then V (transformer.rs:722-726).
    def arena_offsets(cfg, pre_len):
        cursor = pre_len
        offs = []
        for _ in range(cfg.num_layers):
            for _which in range(2):
                off = -(-cursor // 16) * 16
                offs.append(off)
                cursor = off + cfg.max_seq_len * cfg.kv_dim
        return offs

    for key in ("c0", "c2", "c3", "ref_gqa"):
        cfg = WORKLOADS[key].cfg()
        offs = arena_offsets(cfg, 12345)
        base = offs[0]
        for l in range(cfg.num_layers):
            for which in range(2):
                assert orc.kv_offset(cfg, l, which, 0) == offs[2 * l + which] - base
                assert orc.kv_offset(cfg, l, which, 5) == offs[2 * l + which] - base + 5 * cfg.kv_dim


def test_validate_mirrors_reference_asserts():
    ok = orc.Cfg(256, 4, 4, 512)
    assert orc.validate(ok) == 0
    for bad in (orc.Cfg(250, 5, 5, 8), orc.Cfg(256, 3, 3, 8), orc.Cfg(256, 8, 3, 8),
                orc.Cfg(96, 32, 32, 8), orc.Cfg(64, 4, 1, 8), orc.Cfg(64, 4, 4, 0)):
        assert orc.validate(bad) != 0, bad


# ----------------------------------------------------------------- decode/prefill
@pytest.mark.parametrize("key", ["c0", "ref_gqa", "c1"])
def test_prefill_row_equals_sequential_decode(key):
    # transformer.rs:1269-1358: batched prefill must agree with token-by-token
    # forward_token; in the oracle every row runs the same arithmetic, so bit
    # for bit, for outputs and for the cache.
    w = WORKLOADS[key]
    cfg = w.cfg()
    q, k, v = layer_inputs(w, 0)
    n = w.prefill
    a = orc.OracleModel(cfg)
    out_a = a.prefill(0, 0, q[:n], k[:n], v[:n])
    b = orc.OracleModel(cfg)
    out_b = np.stack([b.decode(0, p, q[p], k[p], v[p]) for p in range(n)])
    assert np.array_equal(out_a.view(np.uint32), out_b.view(np.uint32))
    assert np.array_equal(a.kv.view(np.uint32), b.kv.view(np.uint32))
    # continuing a prefill (start > 0) is the same as one longer prefill
    c = orc.OracleModel(cfg)
    c.prefill(0, 0, q[:n // 2], k[:n // 2], v[:n // 2])
    out_c = c.prefill(0, n // 2, q[n // 2:n], k[n // 2:n], v[n // 2:n])
    assert np.array_equal(out_c.view(np.uint32), out_a[n // 2:].view(np.uint32))


def test_decode_cache_rows_and_brute_force():
    w = WORKLOADS["c1"]
    cfg = w.cfg()
    m = orc.OracleModel(cfg)
    q, k, v = layer_inputs(w, 1)
    for p in range(6):
        out = m.decode(1, p, q[p], k[p], v[p])
        # V row is the input; K row is the rotated input; layer 0 untouched
        assert np.array_equal(m.v_cache(1)[p], v[p])
        assert np.array_equal(m.k_cache(1)[p], orc.apply_rope_cached(k[p], m.cos[p], m.sin[p], cfg.head_dim))
        qr = orc.apply_rope_in_place(q[p], p, cfg.head_dim)
        ref = orc.attention_f64(qr, m.k_cache(1), m.v_cache(1), cfg, p)
        assert np.max(np.abs(out - ref)) < 2e-6
    assert not m.k_cache(0).any() and not m.v_cache(0).any()
