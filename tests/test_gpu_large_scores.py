"""Large attention scores through the kernels' online softmax, on the GPU,
against the oracle and against closed forms.

Seeded N(0,1)*0.5 inputs give scores with a spread of ~0.25 nats, so over any
context the running maximum of the kernels' online softmax (log2 domain) is
set by a split's first tile and never again moves by the lazy-rescale
threshold (8 log2 units); split, wave and lane-group states never sit more
than a few units apart.  Real attention logits span tens of nats (attention
sinks, peaked heads).  The inputs here make every branch of the rescale run:

- needle: one key scoring 20+ nats above every other, planted late in one
  split's tile sequence (the running max jumps after many tiles: the alpha
  rescale of l and o, and in prefill the shift of the tile's scores and the
  reset of the accumulator offset);
- ramp: keys growing along q's direction, so a split's maximum rises by
  more than 8 log2 units on tile after tile;
- far apart: a 130-nat needle in one split and a 4-nat one in another, so
  the other splits' (and lane groups') weights underflow to 0 in the merges
  (more than 130 log2 units apart);
- early: the 130-nat needle in split 0's first tile (attended before the
  loop), every later score far below;
- appended: the new row itself is the needle (the owner's last step).

Each case checks the precondition it claims from f64 scores (rescales after
a split's first tile, maxima 130+ log2 units apart), then compares the GPU
with the oracle's causal_multi_head_attention_jit (transformer.rs:273-321)
at the 1e-4 / 1e-3 bar -- outputs are then O(|v|), so the relative bar binds
-- with the appended K/V rows bit for bit.  With zero background keys and
integer V rows the expected output also has a closed form: a needle of
score S over p other rows gives (sum_t V_t + (e^S - 1) V_needle) / (p + e^S),
checked at 2e-5 relative in decode (1e-4 for the ramp, whose scores reach
~190 nats) and 1e-4 in prefill, whose sums after the needle run longer (its
error there grows with their length: 3e-6 after 128 rows, 3e-5 after 1024,
the f32 rounding of 4-product MFMA accumulation steps; a wrong rescale factor
moves outputs by O(1)).
"""
import math
import sys

import numpy as np
import pytest

from oracle import py_oracle as orc
from slm_testlib import _note, assert_bitwise, assert_close, err_report, load_product

P = load_product()
pytestmark = pytest.mark.gpu

LOG2E = 1.0 / math.log(2.0)

# name: dim, heads, kv_heads, theta
SHAPES = {
    "llama3-8b": (4096, 32, 8, 5e5),   # hd 128: 16 lanes per position, two-level merge
    "hd64-gqa4": (2048, 32, 8, 5e5),   # hd 64: 8 lanes per position, third merge round
    "hd48-gqa4": (1536, 32, 8, 1e4),   # hd 48: 4 lanes per position, LDS slot merge
    "stories15m": (288, 6, 6, 1e4),    # hd 48 without GQA (one head per workgroup)
    "smollm2": (576, 9, 3, 5e5),       # hd 64, GQA 3 (prefill: three heads per workgroup)
    "hd96-gqa4": (3072, 32, 8, 1e4),   # hd 96: 8 lanes, four heads, third merge round
    "hd96-mha": (768, 8, 8, 1e4),      # hd 96, one head per workgroup: LDS slot merge
    "hd256-gqa4": (4096, 16, 4, 1e4),  # hd 256: 32 lanes per position, LDS slot merge
    "hd32-gqa4": (1024, 32, 8, 1e4),   # hd 32: 4 lanes per position
    "hd16-gqa4": (512, 32, 8, 1e4),    # hd 16: 2 lanes per position
    "hd128-mha": (4096, 32, 32, 5e5),  # hd 128 without GQA: one head per workgroup
}
# per-head sharpness: q_h = F[h % 4] * base_g (+ a little noise)
F = (1.0, 1.5, 0.8, 1.25)


def log(msg):
    print(msg, flush=True)
    sys.stdout.flush()


class Shape:
    def __init__(self, name, msl):
        self.name = name
        self.dim, self.heads, self.kv_heads, self.theta = SHAPES[name]
        self.hd = self.dim // self.heads
        self.kv_dim = self.hd * self.kv_heads
        self.kv_mul = self.heads // self.kv_heads
        self.msl = msl
        self.cfg = orc.Cfg(self.dim, self.heads, self.kv_heads, msl, 1, self.theta)

    def ctx(self):
        return P.AttentionContext(self.dim, self.heads, self.kv_heads, self.msl, 1, self.theta)


def rng(*seed):
    return np.random.default_rng(list(seed))


def make_q(s: Shape, seed):
    """q with the heads of a KV group along one base direction each:
    q_h = F[h % 4] * base_g + 0.05 * noise."""
    r = rng(seed, 1)
    base = r.standard_normal((s.kv_heads, s.hd)).astype(np.float32) * np.float32(0.5)
    q = np.empty((s.heads, s.hd), np.float32)
    for h in range(s.heads):
        q[h] = np.float32(F[h % 4]) * base[h // s.kv_mul] + np.float32(0.05) * \
            r.standard_normal(s.hd).astype(np.float32)
    return q.reshape(-1), base


def group_dirs(s: Shape, q_rot):
    """Unit direction of the rotated q of each group's first head, and the
    factor that turns a score in nats (for that head) into a key length."""
    qr = q_rot.reshape(s.heads, s.hd).astype(np.float64)
    dirs, per_nat = [], []
    for g in range(s.kv_heads):
        v = qr[g * s.kv_mul]
        nrm = float(np.linalg.norm(v))
        dirs.append(v / nrm)
        per_nat.append(math.sqrt(s.hd) / nrm)
    return np.array(dirs), np.array(per_nat)


def scores_log2(s: Shape, q_rot, k_rows):
    """f64 scores of every head against k_rows [n][kv_dim], log2 units."""
    qr = q_rot.reshape(s.kv_heads, s.kv_mul, s.hd).astype(np.float64)
    kr = k_rows.reshape(-1, s.kv_heads, s.hd).astype(np.float64)
    sc = np.einsum("gmd,ngd->ngm", qr, kr).reshape(-1, s.heads)
    return sc * (LOG2E / math.sqrt(s.hd))


def split_rescales(sc_head, ns, tile):
    """For one head's scores (log2) in position order: per split, how many
    tiles after its first raise its running max by more than 8, and every
    split's final max."""
    n = sc_head.shape[0]
    nt = (n + tile - 1) // tile
    pad = np.full(nt * tile, -np.inf)
    pad[:n] = sc_head
    tmax = pad.reshape(nt, tile).max(axis=1)
    counts, finals = [], []
    for sp in range(ns):
        seq = tmax[sp::ns]
        m = seq[0]
        c = 0
        for x in seq[1:]:
            if x > m + 8.0:
                c += 1
            m = max(m, x)
        counts.append(c)
        finals.append(m)
    return np.array(counts), np.array(finals)


def expected_softmax(s: Shape, q_rot, k_rows, v_rows):
    """f64 attention of one query over rows k_rows / v_rows [n][kv_dim]."""
    sc = scores_log2(s, q_rot, k_rows) / LOG2E  # nats, [n][heads]
    sc = sc - sc.max(axis=0, keepdims=True)
    w = np.exp(sc)
    w /= w.sum(axis=0, keepdims=True)
    vr = v_rows.reshape(-1, s.kv_heads, s.hd).astype(np.float64)
    out = np.empty((s.heads, s.hd))
    for h in range(s.heads):
        out[h] = w[:, h] @ vr[:, h // s.kv_mul]
    return out.reshape(-1)


def check_close_form(got, want, bar, what):
    got = np.asarray(got, np.float64)
    assert np.all(np.isfinite(got)), what
    rel = float((np.abs(got - want) / np.maximum(np.abs(want), 1.0)).max())
    _note(err_report(got, want))
    log(f"{what}: closed form max-rel {rel:.3e} (bar {bar:.0e})")
    assert rel <= bar, f"{what}: max-rel {rel:.3e} > {bar:.0e}"


# ---- decode ------------------------------------------------------------------

DECODE_CASES = [("llama3-8b", 32767), ("llama3-8b", 131072), ("hd64-gqa4", 32767),
                ("hd48-gqa4", 32767), ("stories15m", 49151), ("hd96-gqa4", 32767),
                ("hd96-mha", 32767), ("hd256-gqa4", 32767), ("hd32-gqa4", 32767),
                ("hd16-gqa4", 65535), ("hd128-mha", 32767)]
KINDS = ("needle", "ramp", "far", "early", "appended")


def late_row(ns, tile, n_rows, sp, back=2):
    """A row in the middle of split sp's back-th tile from its last."""
    tiles = n_rows // tile
    per = tiles // ns
    t = ((per - back) * ns + sp) * tile + tile // 3
    assert 0 <= t < n_rows
    return t


@pytest.mark.parametrize("name,p", DECODE_CASES)
def test_decode_large_scores_against_oracle(name, p):
    s = Shape(name, p + 1)
    r = rng(0x51, p)
    k_base = r.standard_normal((p, s.kv_dim), dtype=np.float32) * np.float32(0.5)
    v_rows = r.standard_normal((p, s.kv_dim), dtype=np.float32) * np.float32(0.5)
    q, base = make_q(s, p)
    k_new = r.standard_normal(s.kv_dim, dtype=np.float32) * np.float32(0.5)
    v_new = r.standard_normal(s.kv_dim, dtype=np.float32) * np.float32(0.5)
    om = orc.OracleModel(s.cfg)
    q_rot = om.rotated_q(q, p)
    dirs, per_nat = group_dirs(s, q_rot)
    om.v_cache(0)[:p] = v_rows
    with s.ctx() as ctx:
        ns, tile = ctx.decode_splits(p + 1)
        per = (p + 1) // tile // ns
        log(f"{name} decode at {p}: {ns} splits of {tile}-row tiles, {per}+ tiles per split")
        assert ns > 1 and per >= 4, "the case must walk several tiles per split"
        ctx.kv_write(0, 1, 0, v_rows)
        for kind in KINDS:
            k_rows = k_base.copy()
            kn = k_new.copy()
            kg = k_rows.reshape(p, s.kv_heads, s.hd)
            if kind == "needle":
                t = late_row(ns, tile, p, sp=min(5, ns - 1))
                kg[t] += (30.0 * per_nat[:, None] * dirs).astype(np.float32)
            elif kind == "ramp":
                # + 8 nats (head f = 1) per tile step of a split, over the
                # last R steps of every split
                rr = min(16, per - 1)
                t0 = p - rr * ns * tile
                step = 8.0 / (ns * tile)
                ramp = (np.arange(p - t0) * step)[:, None, None] * per_nat[None, :, None]
                kg[t0:] += (ramp * dirs[None]).astype(np.float32)
            elif kind == "far":
                ta = late_row(ns, tile, p, sp=min(3, ns - 1))
                tb = late_row(ns, tile, p, sp=min(7, ns - 1) if ns > 7 else ns - 2, back=3)
                kg[ta] += (130.0 * per_nat[:, None] * dirs).astype(np.float32)
                kg[tb] += (4.0 * per_nat[:, None] * dirs).astype(np.float32)
            elif kind == "early":
                kg[3] += (130.0 * per_nat[:, None] * dirs).astype(np.float32)
            elif kind == "appended":
                # un-rotated k along the un-rotated base: rotation keeps the dot
                for g in range(s.kv_heads):
                    b = base[g].astype(np.float64)
                    kn[g * s.hd:(g + 1) * s.hd] = (30.0 * math.sqrt(s.hd) / np.linalg.norm(b)
                                                   * b / np.linalg.norm(b)).astype(np.float32)
            # the precondition each kind claims, from f64 scores of head 0 of
            # every group (f = 1)
            sc = scores_log2(s, q_rot, k_rows)
            h0s = [g * s.kv_mul for g in range(s.kv_heads)]
            for h in h0s:
                counts, finals = split_rescales(sc[:, h], ns, tile)
                if kind == "ramp":
                    assert counts.min() >= max(1, min(16, per - 1) - 2), (h, counts)
                elif kind in ("needle", "far"):
                    assert counts.max() >= 1, (h, counts)
                if kind in ("far", "early"):
                    top = np.sort(finals)[::-1]
                    assert top[0] - top[1] > 130.0, (h, top[:3])
            log(f"{name} @{p} {kind}: max score {float(sc.max()) / LOG2E:.1f} nats")
            ctx.kv_write(0, 0, 0, k_rows)
            om.k_cache(0)[:p] = k_rows
            got = ctx.decode(0, p, q, kn, v_new)
            want = om.decode(0, p, q, kn, v_new)
            rep = err_report(got, want)
            log(f"{name} @{p} {kind}: max-abs {rep['max_abs']:.2e} max-rel {rep['max_rel']:.2e}")
            if kind == "appended":
                sp = scores_log2(s, q_rot, om.k_cache(0)[p:p + 1])[0]
                for h in h0s:
                    assert sp[h] - sc[:, h].max() > 20.0 * LOG2E, (h, sp[h], sc[:, h].max())
            assert_close(got, want, what=f"{name} decode @{p} {kind}")
            assert_bitwise(ctx.kv_read(0, 0, p, 1)[0], om.k_cache(0)[p], f"{kind}: K row {p}")
            assert_bitwise(ctx.kv_read(0, 1, p, 1)[0], om.v_cache(0)[p], f"{kind}: V row {p}")


CLOSED_DECODE = [("llama3-8b", 32767), ("hd64-gqa4", 32767), ("hd48-gqa4", 32767)]


@pytest.mark.parametrize("name,p", CLOSED_DECODE)
def test_decode_large_scores_closed_form(name, p):
    """Zero background keys, V integers 0..15: a needle of S in {8, 20, 100}
    nats (head f = 1; 11.5 log2 units already rescales) late in one split,
    and a ramp, against f64 closed forms."""
    s = Shape(name, p + 1)
    t = np.arange(p + 1)[:, None]
    d = np.arange(s.kv_dim)[None, :]
    v_all = ((t * 7 + d * 13 + (t // 32) * 5) % 16).astype(np.float32)
    q, _ = make_q(s, p + 7)
    with s.ctx() as ctx:
        ns, tile = ctx.decode_splits(p + 1)
        log(f"{name} closed-form decode at {p}: {ns} splits of {tile}-row tiles")
        ctx.kv_write(0, 1, 0, v_all[:p])
        cos, sin = ctx.rope_tables()
        q_rot = orc.apply_rope_cached(q, cos[p], sin[p], s.hd)
        dirs, per_nat = group_dirs(s, q_rot)
        zeros = np.zeros(s.kv_dim, np.float32)
        for kind, S in (("needle", 8.0), ("needle", 20.0), ("needle", 100.0), ("ramp", 0.0)):
            k_rows = np.zeros((p, s.kv_dim), np.float32)
            kg = k_rows.reshape(p, s.kv_heads, s.hd)
            if kind == "needle":
                tn = late_row(ns, tile, p, sp=min(5, ns - 1))
                kg[tn] = (S * per_nat[:, None] * dirs).astype(np.float32)
                lo, hi = tn, tn + 1
            else:
                per = (p + 1) // tile // ns
                rr = min(16, per - 1)
                t0 = p - rr * ns * tile
                step = 8.0 / (ns * tile)
                ramp = (np.arange(p - t0) * step)[:, None, None] * per_nat[None, :, None]
                kg[t0:] = (ramp * dirs[None]).astype(np.float32)
                lo, hi = t0, p
            ctx.kv_write(0, 0, lo, k_rows[lo:hi])
            out = ctx.decode(0, p, q, zeros, v_all[p])
            k_all = np.concatenate([k_rows, zeros[None]])
            want = expected_softmax(s, q_rot, k_all, v_all)
            bar = 2e-5 if kind == "needle" else 1e-4
            check_close_form(out, want, bar, f"{name} decode @{p} {kind} S={S:g}")
            ctx.kv_write(0, 0, lo, np.zeros((hi - lo, s.kv_dim), np.float32))


# ---- prefill -----------------------------------------------------------------

# (shape, start, n): the 4096-row Llama-3-8B-shape prefill takes the DMA-fed
# kernel on 256 CUs; the others the register-prefetch kernel: four heads per
# workgroup at hd 128, 256 and 32, one head and four query blocks for the hd
# 128 and hd 96 MHA shapes; the hd 64 (three heads), hd 48 and hd 16 shapes
# give under two workgroups per CU at these lengths and take the one-head
# kernel with the key tiles split over four waves; 480 Llama-3-8B-shape rows
# take the paired-block kernel (two heads, blocks i and n-1-i, two key
# splits), 256 rows of hd 128 MHA its one-head form (four key splits)
PREFILL_CASES = [("llama3-8b", 0, 4096), ("llama3-8b", 24, 1000), ("llama3-8b", 100, 480),
                 ("hd128-mha", 40, 256), ("smollm2", 0, 2048),
                 ("stories15m", 0, 512), ("hd128-mha", 0, 2048), ("hd256-gqa4", 24, 1000),
                 ("hd96-mha", 0, 1024), ("hd32-gqa4", 0, 1024), ("hd16-gqa4", 0, 512)]
A = (4.0, 4.5, 5.0, 3.5)  # per-head size of q's large component


def prefill_inputs(s: Shape, start, n, seed):
    """q rows whose dim hd-2 is a_h in every head (the slowest RoPE pair, which
    turns by under 0.02 rad over these lengths), background k/v rows."""
    rows = start + n
    r = rng(seed, rows)
    q = r.standard_normal((rows, s.heads, s.hd), dtype=np.float32) * np.float32(0.5)
    for h in range(s.heads):
        q[:, h, s.hd - 2] = np.float32(A[h % 4])
    k = r.standard_normal((rows, s.kv_heads, s.hd), dtype=np.float32) * np.float32(0.5)
    v = r.standard_normal((rows, s.kv_dim), dtype=np.float32) * np.float32(0.5)
    return q.reshape(rows, s.dim), k, v


def plant(s: Shape, k, kind, rows):
    """Large keys along dim hd-2 (a = 4 gives the named score in nats)."""
    c_per_nat = math.sqrt(s.hd) / 4.0
    if kind == "needle25":
        k[rows * 3 // 4, :, s.hd - 2] = np.float32(25.0 * c_per_nat)
    elif kind == "needle100":
        k[rows * 3 // 4, :, s.hd - 2] = np.float32(100.0 * c_per_nat)
    elif kind == "sawtooth":
        # +0.22 nats per row (a = 4), period 512: 7 nats (10 log2 units) per
        # 32-key tile, peaks of ~112 nats (140 for a = 5; at ~225 nats the
        # f32 rounding of the scores alone moves outputs by ~1e-4 in both
        # implementations)
        t = np.arange(rows)
        k[:, :, s.hd - 2] = ((t % 512) * 0.22 * c_per_nat)[:, None].astype(np.float32)
    elif kind == "late_far":
        # everything up to the needle far below it: 130 nats at 7/8
        k[rows * 7 // 8, :, s.hd - 2] = np.float32(130.0 * c_per_nat)


@pytest.mark.parametrize("name,start,n", PREFILL_CASES)
def test_prefill_large_scores_against_oracle(name, start, n):
    rows = start + n
    s = Shape(name, rows)
    with s.ctx() as ctx:
        for kind in ("needle25", "needle100", "sawtooth", "late_far"):
            q, k, v = prefill_inputs(s, start, n, 0x77)
            plant(s, k, kind, rows)
            k = k.reshape(rows, s.kv_dim)
            log(f"{name} prefill {start}+{n} {kind}")
            if start:
                ctx.prefill(0, 0, q[:start], k[:start], v[:start])
            got = ctx.prefill(0, start, q[start:], k[start:], v[start:])
            om = orc.OracleModel(s.cfg)
            om.append(0, 0, k, v)
            assert_bitwise(ctx.kv_read(0, 0, 0, rows), om.k_cache(0)[:rows], f"{kind}: K rows")
            assert_bitwise(ctx.kv_read(0, 1, 0, rows), om.v_cache(0)[:rows], f"{kind}: V rows")
            marks = {rows * 3 // 4, rows * 7 // 8, 511, 512, 1023, 1024, 2047}
            sample = sorted({start, start + 1, start + 31, start + 32, rows - 1, rows - 2,
                             rows - 33} | {m + d for m in marks for d in (-1, 0, 1, 31, 32)})
            worst = {"max_abs": 0.0, "max_rel": 0.0}
            for b in sample:
                if not start <= b < rows:
                    continue
                want = om.attend(0, q[b], b)
                rep = err_report(got[b - start], want)
                for key in worst:
                    worst[key] = max(worst[key], rep[key])
                assert_close(got[b - start], want, what=f"{name} prefill {kind} row {b}")
            log(f"{name} prefill {kind}: max-abs {worst['max_abs']:.2e} "
                f"max-rel {worst['max_rel']:.2e} over {len(sample)} rows")
            # the rescales the case claims: the max over keys <= row rises
            # by more than 8 log2 units after the first tile
            b = rows - 1
            sc = scores_log2(s, om.rotated_q(q[b], b), om.k_cache(0)[:rows])[:, 0]
            tiles = [sc[i:i + 32].max() for i in range(0, rows, 32)]
            m, rises = tiles[0], 0
            for x in tiles[1:]:
                rises += x > m + 8.0
                m = max(m, x)
            log(f"{name} prefill {kind}: row {b} max {max(tiles) / LOG2E:.1f} nats, "
                f"{rises} tiles raising the max by > 8 log2 units")
            assert rises >= 1


@pytest.mark.parametrize("name,start,n", PREFILL_CASES)
def test_prefill_needle_closed_form_every_row(name, start, n):
    """Zero keys but one needle (S in {8, 25, 100} nats for a = 4), V
    integers 0..15: every row against (C_p + (e^S - 1) V*) / (p + e^S),
    C_p the exact sum of V rows 0..p."""
    rows = start + n
    s = Shape(name, rows)
    t = np.arange(rows)[:, None]
    d = np.arange(s.kv_dim)[None, :]
    v = ((t * 7 + d * 13 + (t // 32) * 5) % 16).astype(np.float32)
    cums = np.cumsum(v.astype(np.int64), axis=0)
    q, _, _ = prefill_inputs(s, start, n, 0x78)
    tn = rows * 3 // 4
    c_per_nat = math.sqrt(s.hd) / 4.0
    with s.ctx() as ctx:
        cos, sin = ctx.rope_tables()
        # rotated q of the rows that see the needle, [rows - tn][heads][hd]
        qr = np.stack([orc.apply_rope_cached(q[b], cos[b], sin[b], s.hd)
                       for b in range(tn, rows)]).reshape(-1, s.heads, s.hd).astype(np.float64)
        b_all = np.arange(start, rows)
        cg = cums[start:].reshape(n, s.kv_heads, s.hd).astype(np.float64)
        vs = v[tn].reshape(s.kv_heads, s.hd).astype(np.float64)
        for S in (8.0, 25.0, 100.0):
            k = np.zeros((rows, s.kv_heads, s.hd), np.float32)
            k[tn, :, s.hd - 2] = np.float32(S * c_per_nat)
            k = k.reshape(rows, s.kv_dim)
            if start:
                ctx.prefill(0, 0, q[:start], k[:start], v[:start])
            got = ctx.prefill(0, start, q[start:], k[start:], v[start:])
            kn = ctx.kv_read(0, 0, tn, 1)[0].reshape(s.kv_heads, s.hd).astype(np.float64)
            # rows before the needle: the mean of V rows 0..b
            want = np.repeat(cg / (b_all + 1)[:, None, None], s.kv_mul, axis=1)
            # rows from it on: the needle's weight e^S against 1 for the others
            kh = np.repeat(kn, s.kv_mul, axis=0)  # the key segment each head reads
            e = np.exp(np.einsum("bhd,hd->bh", qr, kh) / math.sqrt(s.hd))
            ch = np.repeat(cg[tn - start:], s.kv_mul, axis=1)
            vh = np.repeat(vs, s.kv_mul, axis=0)
            bb = np.arange(tn, rows)[:, None, None].astype(np.float64)
            want[tn - start:] = (ch + (e[:, :, None] - 1.0) * vh[None]) / (bb + e[:, :, None])
            check_close_form(got, want.reshape(n, s.dim), 1e-4,
                             f"{name} prefill {start}+{n} needle S={S:g} (row {tn})")
