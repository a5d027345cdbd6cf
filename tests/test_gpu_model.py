"""GPU parity of the whole model (TransformerModel on device, include/slm_layer.h).

Bars: logits within the reference's layer-test bound (1e-4) of the oracle's
model on the reference's own prefill-test model (transformer.rs:1269-1358),
the same greedy tokens wherever the oracle's top two logits are further
apart than that bound, and the reference's relation that the first token of
generate (batched prefill) equals the last token of a token-by-token run.
On a larger shape the device is checked against itself: prefill logits
within the bound of token-by-token logits, generate equal to repeated
forward_token.  The embedding is checked against the oracle within 1e-4.
"""
import sys

import numpy as np
import pytest

from oracle import py_oracle as orc
from slm_testlib import gen, load_product
from test_oracle_layer import quantize_matrix, ref_model

P = load_product()
pytestmark = pytest.mark.gpu
torch = pytest.importorskip("torch")
EPS = 1e-5


def log(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def dev(a: np.ndarray):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


class DeviceModel:
    """The oracle's ModelWeights uploaded: Q4Matrix handles and norm vectors."""

    def __init__(self, cfg: orc.Cfg, w: orc.ModelWeights):
        dim, kvd = cfg.dim, cfg.kv_dim
        self.keep, self.mats = [], []

        def q4(blocks, rows, cols):
            m = P.Q4Matrix(blocks, rows, cols)
            self.mats.append(m)
            return m

        def vec(a):
            t = dev(a)
            self.keep.append(t)
            return t.data_ptr()

        layers = []
        for lw in w.layers:
            h = lw.hidden_dim
            layers.append(P.LayerWeights(
                vec(lw.rms_att), q4(lw.wq, dim, dim), q4(lw.wk, kvd, dim), q4(lw.wv, kvd, dim),
                q4(lw.wo, dim, dim), vec(lw.rms_ffn), q4(lw.w_gate, h, dim),
                q4(lw.w_up, h, dim), q4(lw.w_down, dim, h)))
        self.w = P.ModelWeights(q4(w.token_embd, w.vocab_size, dim), layers, vec(w.output_norm),
                                q4(w.lm_head, w.vocab_size, dim))
        self.vocab = w.vocab_size

    def close(self):
        for m in self.mats:
            m.close()


def clear_winner(logits, tol=1e-4):
    top = np.sort(logits)[-2:]
    return top[1] - top[0] > 2 * tol


def test_forward_token_and_prefill_against_oracle():
    cfg, w = ref_model()
    prompt = [1, 7, 19, 42]
    dm = DeviceModel(cfg, w)
    try:
        with P.AttentionContext(cfg.dim, cfg.num_heads, cfg.num_kv_heads, cfg.max_seq_len,
                                2, 1e4) as c:
            om = orc.OracleModel(cfg)
            logits = dev(np.full(dm.vocab, np.nan, np.float32))
            seq_next = None
            for pos, tok in enumerate(prompt):
                nxt = c.model_forward_token_dev(dm.w, EPS, tok, pos, logits.data_ptr())
                c.sync()
                got = logits.cpu().numpy()
                want, onext, _ = orc.model_forward(om, w, EPS, [tok], pos)
                err = np.abs(got - want).max()
                log(f"pos {pos}: next {nxt} (oracle {onext}), logits max abs {err:.3g}")
                assert err < 1e-4
                assert nxt == int(np.argmax(got))
                if clear_winner(want):
                    assert nxt == onext
                seq_next = nxt
        # batched prefill on a fresh cache: first generated token as the
        # token-by-token run's (transformer.rs:1351-1357)
        with P.AttentionContext(cfg.dim, cfg.num_heads, cfg.num_kv_heads, cfg.max_seq_len,
                                2, 1e4) as c:
            out = c.model_generate_dev(dm.w, EPS, prompt, 4)
            assert len(out) == 4 and out[0] == seq_next
            ref = orc.model_generate(orc.OracleModel(cfg), w, EPS, prompt, 4)
            log(f"generate {out} oracle {ref}")
            # the prompt's logits are compared above; the decode steps follow
            # the device's own tokens, so compare the oracle run only while
            # both have taken the same tokens
            for a, b in zip(out, ref):
                if a != b:
                    break
                assert 0 <= a < dm.vocab
    finally:
        dm.close()


def test_generate_stops_at_eos_and_max_seq_len():
    cfg, w = ref_model()
    dm = DeviceModel(cfg, w)
    try:
        with P.AttentionContext(cfg.dim, cfg.num_heads, cfg.num_kv_heads, cfg.max_seq_len,
                                2, 1e4) as c:
            full = c.model_generate_dev(dm.w, EPS, [5, 6], 40)
            # 14 decode positions after a 2-token prompt: 1 + 14 tokens
            assert len(full) == 1 + (cfg.max_seq_len - 2)
            eos = full[2]
            cut = c.model_generate_dev(dm.w, EPS, [5, 6], 40, eos=eos)
            assert cut == full[:full.index(eos) + 1]
            assert c.model_generate_dev(dm.w, EPS, [5, 6], 0) == []
            assert c.model_generate_dev(dm.w, EPS, [], 4) == []
    finally:
        dm.close()


def kv_snapshot(c, cfg, layers):
    return np.stack([c.kv_read(l, which, 0, cfg.max_seq_len)
                     for l in range(layers) for which in (0, 1)])


def sentinel_fill(c, cfg, layers):
    # rows no call has written keep these values, distinct per layer and side
    for l in range(layers):
        for which in (0, 1):
            rows = np.full((cfg.max_seq_len, cfg.kv_dim), -3.25 - l - 0.5 * which, np.float32)
            c.kv_write(l, which, 0, rows)


@pytest.mark.parametrize("stop", ["second", "middle", "last"])
def test_generate_eos_leaves_the_cache_as_the_reference(stop):
    """generate stops after forward_token produced EOS and never runs it on
    the EOS token (transformer.rs:874-889).  The device pipelines its decode
    steps, so one step has already run on the EOS token when the host sees
    it; the K/V rows that step wrote must be put back.  The whole cache after
    generate (every layer, K and V, every row, over a sentinel fill) must
    equal bit for bit the cache after prefill + forward_token of each
    returned token but the last, and the row after the returned sequence must
    keep the sentinel.  Tokens against the oracle's generate with the same
    EOS."""
    cfg, w = ref_model()
    layers = 2
    prompt = [5, 6]
    dm = DeviceModel(cfg, w)
    try:
        def ctx():
            return P.AttentionContext(cfg.dim, cfg.num_heads, cfg.num_kv_heads,
                                      cfg.max_seq_len, layers, 1e4)
        with ctx() as c:
            full = c.model_generate_dev(dm.w, EPS, prompt, 40)
        i = {"second": 1, "middle": len(full) // 2, "last": len(full) - 1}[stop]
        eos = full[i]
        want_tokens = full[:full.index(eos) + 1]
        log(f"full run {full}; EOS {eos} -> {want_tokens}")
        with ctx() as a:
            sentinel_fill(a, cfg, layers)
            before = kv_snapshot(a, cfg, layers)
            out = a.model_generate_dev(dm.w, EPS, prompt, 40, eos=eos)
            got = kv_snapshot(a, cfg, layers)
        assert out == want_tokens
        # the oracle on the same tokens: each step's argmax wherever its top
        # two logits are clearly apart, logits within the bound
        om = orc.OracleModel(cfg)
        feed = [(prompt, 0)] + [([out[j - 1]], len(prompt) + j - 1) for j in range(1, len(out))]
        for j, (toks, pos) in enumerate(feed):
            want, onext, _ = orc.model_forward(om, w, EPS, toks, pos)
            if clear_winner(want):
                assert onext == out[j], (j, onext, out[j])
        log(f"generate with EOS {out}: oracle argmax agrees")
        with ctx() as b:
            sentinel_fill(b, cfg, layers)
            nxt = b.model_prefill_dev(dm.w, EPS, prompt)
            assert nxt == out[0]
            for j in range(1, len(out)):
                nxt = b.model_forward_token_dev(dm.w, EPS, out[j - 1], len(prompt) + j - 1)
                assert nxt == out[j]
            b.sync()
            seq = kv_snapshot(b, cfg, layers)
        assert_kv_equal(got, seq, "generate with EOS against prefill + forward_token")
        last = len(prompt) + len(out) - 1  # the first row the reference leaves untouched
        assert_kv_equal(got[:, last:], before[:, last:], f"rows {last}.. keep their contents")
        assert not np.array_equal(got[:, last - 1], before[:, last - 1])
    finally:
        dm.close()


def assert_kv_equal(a, b, what):
    neq = a.view(np.uint32) != b.view(np.uint32)
    assert not neq.any(), f"{what}: {int(neq.sum())} of {neq.size} words differ"


def test_embedding_against_oracle():
    cfg, w = ref_model()
    dm = DeviceModel(cfg, w)
    tokens = [3, 9, 27, 81, 5, 125]
    try:
        with P.AttentionContext(cfg.dim, cfg.num_heads, cfg.num_kv_heads, cfg.max_seq_len,
                                2, 1e4) as c:
            out = dev(np.full(cfg.dim, np.nan, np.float32))
            c.model_embed_dev(dm.w, EPS, tokens, out.data_ptr())
            c.sync()
            got = out.cpu().numpy()
        want = orc.model_embed(orc.OracleModel(cfg), w, EPS, tokens)
        assert np.abs(got - want).max() < 1e-4
        assert abs(np.linalg.norm(got.astype(np.float64)) - 1.0) < 1e-5
    finally:
        dm.close()


def test_model_argument_checks():
    cfg, w = ref_model()
    dm = DeviceModel(cfg, w)
    try:
        with P.AttentionContext(cfg.dim, cfg.num_heads, cfg.num_kv_heads, cfg.max_seq_len,
                                2, 1e4) as c:
            with pytest.raises(P.SlmAttnError) as ei:
                c.model_forward_token_dev(dm.w, EPS, dm.vocab, 0)
            assert ei.value.code == P.ERR_TOKEN
            with pytest.raises(P.SlmAttnError) as ei:
                c.model_prefill_dev(dm.w, EPS, [1, -1, 2])
            assert ei.value.code == P.ERR_TOKEN
            with pytest.raises(P.SlmAttnError) as ei:
                c.model_forward_token_dev(dm.w, EPS, 1, cfg.max_seq_len)
            assert ei.value.code == P.ERR_POS
            one_layer = P.ModelWeights(dm.w.token_embd, dm.w.layers[:1], dm.w.output_norm,
                                       dm.w.lm_head)
            with pytest.raises(P.SlmAttnError) as ei:
                c.model_forward_token_dev(one_layer, EPS, 1, 0)
            assert ei.value.code == P.ERR_CONFIG
    finally:
        dm.close()


def test_larger_model_prefill_matches_token_by_token():
    # SmolLM2-135M's layer shape, 3 layers, vocab 2000: the batched path
    # (MFMA GEMM, prefill attention) against the decode path (GEMV, split-K
    # decode) on the same device
    dim, hidden, heads, kvh, msl, vocab, layers = 576, 1536, 9, 3, 48, 2000, 3
    cfg = orc.Cfg(dim, heads, kvh, msl, layers, 1e5)
    rng = np.random.default_rng(7)

    def mat(rows, cols):
        return orc.quantize_q4_0(rng.standard_normal((rows, cols), dtype=np.float32) *
                                 np.float32(0.08))

    lws = [orc.LayerWeights(
        rms_att=np.float32(1.0) + gen([61, l, 0], (dim,)) * np.float32(0.1),
        rms_ffn=np.float32(1.0) + gen([61, l, 1], (dim,)) * np.float32(0.1),
        wq=mat(dim, dim), wk=mat(cfg.kv_dim, dim), wv=mat(cfg.kv_dim, dim), wo=mat(dim, dim),
        w_gate=mat(hidden, dim), w_up=mat(hidden, dim), w_down=mat(dim, hidden),
        hidden_dim=hidden) for l in range(layers)]
    w = orc.ModelWeights(token_embd=mat(vocab, dim), layers=lws,
                         output_norm=np.float32(1.0) + gen(62, (dim,)) * np.float32(0.1),
                         lm_head=mat(vocab, dim), vocab_size=vocab)
    dm = DeviceModel(cfg, w)
    prompt = [int(t) for t in rng.integers(0, vocab, 23)]
    try:
        seq_logits = dev(np.zeros(vocab, np.float32))
        with P.AttentionContext(dim, heads, kvh, msl, layers, 1e5) as a:
            for pos, tok in enumerate(prompt):
                seq_next = a.model_forward_token_dev(dm.w, EPS, tok, pos, seq_logits.data_ptr())
            a.sync()
            seq = seq_logits.cpu().numpy()
        with P.AttentionContext(dim, heads, kvh, msl, layers, 1e5) as b:
            pre_logits = dev(np.zeros(vocab, np.float32))
            pre_next = b.model_prefill_dev(dm.w, EPS, prompt, 0, pre_logits.data_ptr())
            b.sync()
            pre = pre_logits.cpu().numpy()
        log(f"prefill next {pre_next} token-by-token next {seq_next}, "
            f"logits max abs {np.abs(pre - seq).max():.3g}")
        tol = 5e-3 * max(1.0, np.abs(seq).max())
        assert np.abs(pre - seq).max() < tol
        if clear_winner(seq, tol):
            assert pre_next == seq_next
        # generate == prefill + repeated forward_token on the device
        with P.AttentionContext(dim, heads, kvh, msl, layers, 1e5) as g, \
                P.AttentionContext(dim, heads, kvh, msl, layers, 1e5) as h:
            out = g.model_generate_dev(dm.w, EPS, prompt, 10)
            nxt = h.model_prefill_dev(dm.w, EPS, prompt, 0)
            manual = [nxt]
            for pos in range(len(prompt), len(prompt) + 9):
                nxt = h.model_forward_token_dev(dm.w, EPS, nxt, pos)
                manual.append(nxt)
            assert out == manual
    finally:
        dm.close()


def test_argmax_first_maximum_over_a_large_vocabulary():
    """sample_argmax (transformer.rs:654-666) over 70001 logits (4376 lm_head
    workgroup parts): the token is the first index of the maximum of the
    logits the device returns, also when the maximal lm_head row is copied to
    a higher index and to a lower one (exact ties); NaN logits never win,
    except a NaN at index 0, which gives token 0."""
    cfg, w = ref_model()
    vocab = 70001
    nbytes = cfg.dim // 32 * 18
    embd = quantize_matrix(vocab, cfg.dim, 0x0400)
    head = quantize_matrix(vocab, cfg.dim, 0x0500).reshape(vocab, nbytes)

    def run(lm_head):
        mw = orc.ModelWeights(embd, w.layers, w.output_norm, lm_head.reshape(-1), vocab)
        dm = DeviceModel(cfg, mw)
        try:
            with P.AttentionContext(cfg.dim, cfg.num_heads, cfg.num_kv_heads, cfg.max_seq_len,
                                    2, 1e4) as c:
                logits = dev(np.full(vocab, np.nan, np.float32))
                nxt = c.model_forward_token_dev(dm.w, EPS, 3, 0, logits.data_ptr())
                c.sync()
                return nxt, logits.cpu().numpy()
        finally:
            dm.close()

    nxt, lg = run(head)
    m = int(np.argmax(lg))
    log(f"vocab {vocab}: token {nxt}, max {lg[m]:.4f} at {m}")
    assert np.isfinite(lg).all() and nxt == m
    hi = vocab - 2 if m != vocab - 2 else vocab - 3
    dup = head.copy()
    dup[hi] = head[m]
    nxt, lg = run(dup)
    assert lg[hi] == lg[m] and nxt == m  # a tie goes to the lower index
    if m > 0:
        lo = m // 2
        dup[lo] = head[m]
        nxt, lg = run(dup)
        assert lg[lo] == lg[m] and nxt == lo
    # NaN logits (rows whose block scales are f16 NaN): skipped after index 0,
    # and a NaN at index 0 wins outright (the scan starts from logits[0])
    nan_rows = head.copy()
    nan_f16 = np.frombuffer(np.float16(np.nan).tobytes(), np.uint8)
    for r in (7, vocab - 1, m + 1 if m + 1 < vocab else 5):
        for b in range(cfg.dim // 32):
            nan_rows[r, 18 * b:18 * b + 2] = nan_f16
    nxt, lg = run(nan_rows)
    assert np.isnan(lg[7]) and nxt == m
    for b in range(cfg.dim // 32):
        nan_rows[0, 18 * b:18 * b + 2] = nan_f16
    nxt, lg = run(nan_rows)
    assert np.isnan(lg[0]) and nxt == 0
