"""Pins of the oracle's JIT norm / activation kernels and transformer block
(oracle/layer.c) -- CPU only.

What pins them:
  * closed forms and exact invariants (constant rows, zero rows, power-of-two
    scaling, silu at 0 and at large |v|, a one-hot L2 norm);
  * f64 evaluations of the same formulas within the f32 rounding budget;
  * the reference's own relations: its layer tests (transformer.rs:1000-1099
    MHA, 1102-1208 GQA) check the JIT block against a scalar restatement
    (scalar_rmsnorm, scalar GEMV, apply_rope_in_place, the scalar attention,
    libm exp in SwiGLU) within 1e-4 on xorshift inputs; the same inputs and
    the same bound are used here;
  * prefill == sequential decode (transformer.rs:1269-1358 checks the argmax;
    the restatement gives identical bits).
"""
import numpy as np
import pytest

from oracle import py_oracle as orc


def pseudo_random_f32(n: int, seed: int) -> np.ndarray:
    """The reference tests' generator (transformer.rs:962-975): xorshift32,
    (seed as f32) / (u32::MAX as f32), then (unit * 2 - 1) * 0.25 in f32."""
    out = np.empty(n, np.float32)
    s = seed & 0xFFFFFFFF
    umax = np.float32(4294967295.0)
    for i in range(n):
        s ^= (s << 13) & 0xFFFFFFFF
        s ^= s >> 17
        s ^= (s << 5) & 0xFFFFFFFF
        unit = np.float32(s) / umax
        out[i] = (unit * np.float32(2.0) - np.float32(1.0)) * np.float32(0.25)
    return out


def quantize_matrix(rows: int, cols: int, seed: int) -> np.ndarray:
    return orc.quantize_q4_0(pseudo_random_f32(rows * cols, seed))


def rng_rows(seed, rows, n, scale=1.0):
    return (np.random.default_rng(seed).standard_normal((rows, n)) * scale).astype(np.float32)


# ---- RMSNorm ----

def test_rmsnorm_constant_row_closed_form():
    n, eps = 4096, np.float32(1e-5)
    x = np.ones(n, np.float32)
    w = rng_rows(1, 1, n)[0]
    # sum of n ones is exact, 1/n and the mean are exact: rms = 1/sqrt(1 + eps)
    rms = np.float32(1.0) / np.sqrt(np.float32(1.0) + eps)
    assert orc.jit_rmsnorm_scale(x, float(eps)) == rms
    np.testing.assert_array_equal(orc.jit_rmsnorm(x, w, float(eps)), (x * rms) * w)


def test_rmsnorm_zero_row_is_zero_and_power_of_two_scaling_is_exact():
    n = 576
    w = rng_rows(2, 1, n)[0]
    assert not np.any(orc.jit_rmsnorm(np.zeros(n, np.float32), w, 1e-5))
    x = rng_rows(3, 1, n)[0]
    # eps = 0: scaling x by 4 scales every square by 16 exactly, so the sum,
    # mean and root scale exactly and the output bits do not change
    np.testing.assert_array_equal(orc.jit_rmsnorm(4 * x, w, 0.0), orc.jit_rmsnorm(x, w, 0.0))


@pytest.mark.parametrize("n", [32, 100, 576, 4096, 16384])
def test_rmsnorm_matches_f64_and_the_reference_scalar_form(n):
    x = rng_rows(4, 8, n, 3.0)
    w = rng_rows(5, 1, n)[0]
    for r in range(x.shape[0]):
        got = orc.jit_rmsnorm(x[r], w, 1e-5)
        xd = x[r].astype(np.float64)
        exact = xd / np.sqrt(np.mean(xd * xd) + 1e-5) * w
        tol = 4e-6 * np.abs(exact).max()
        assert np.abs(got - exact).max() <= tol
        # the reference's test-side scalar_rmsnorm: another rounding order
        assert np.abs(got - orc.scalar_rmsnorm(x[r], w, 1e-5)).max() <= tol


# ---- SiLU / SwiGLU / residual add ----

def test_silu_special_values():
    assert orc.jit_silu(np.float32([0.0]))[0] == 0.0
    # exp(-v) of a large v is clamped to exp(-87.3) ~ 1e-38: 1 + it rounds to 1
    big = np.float32([50.0, 100.0, 1e6])
    np.testing.assert_array_equal(orc.jit_silu(big), big)


def test_silu_and_swiglu_match_f64():
    g = np.concatenate([np.linspace(-100, 100, 40001, dtype=np.float32),
                        rng_rows(6, 1, 4096, 4.0)[0]])
    u = rng_rows(7, 1, g.size, 2.0)[0]
    s = orc.jit_silu(g)
    gd = g.astype(np.float64)
    exact = gd / (1.0 + np.exp(-gd))
    # the polynomial exp is within ~2e-7 relative and the divide adds half an
    # ulp; below v = -87.3 the exp's input clamp (lower.rs:23-26) leaves
    # silu(v) = v / e^88.3, a few 1e-37 where the exact value is smaller still
    assert (np.abs(s - exact) <= 4e-6 * np.abs(exact) + 1e-35).all()
    assert np.abs(s[g < -87.3]).max() < 1e-35
    sw = orc.jit_swiglu(g, u)
    np.testing.assert_array_equal(sw, s * u)
    assert (np.abs(sw - exact * u) <= 5e-6 * np.abs(exact * u) + 1e-34).all()


def test_residual_add_is_the_f32_sum():
    a, b = rng_rows(8, 1, 1000)[0], rng_rows(9, 1, 1000)[0]
    np.testing.assert_array_equal(orc.jit_residual_add(a, b), a + b)


# ---- L2 norm ----

def test_l2_norm_one_hot_and_unit_norm():
    x = np.zeros(64, np.float32)
    x[17] = 3.0
    y = orc.jit_l2_norm(x, 0.0)
    assert y[17] == np.float32(3.0) * (np.float32(1.0) / np.float32(3.0))
    assert np.count_nonzero(y) == 1
    for r, row in enumerate(rng_rows(10, 6, 576, 5.0)):
        y = orc.jit_l2_norm(row, 1e-12)
        assert abs(np.linalg.norm(y.astype(np.float64)) - 1.0) < 2e-6
        exact = row.astype(np.float64) / np.linalg.norm(row.astype(np.float64))
        assert np.abs(y - exact).max() < 2e-7


# ---- the block: the reference's own layer tests ----

def scalar_layer_step(cfg, hidden, eps, w, k_cache, v_cache, x, pos):
    """The scalar reference of transformer.rs:1044-1084 / 1153-1193 for one
    position: scalar_rmsnorm, scalar_gemv, apply_rope_in_place, the scalar
    attention, SwiGLU with libm exp, f32 residual adds."""
    dim, kvd = cfg.dim, cfg.kv_dim
    xb = orc.scalar_rmsnorm(x, w.rms_att, eps)
    q = orc.gemm_q4_0_f32(w.wq, xb, 1, dim, dim)[0]
    k = orc.gemm_q4_0_f32(w.wk, xb, 1, kvd, dim)[0]
    v = orc.gemm_q4_0_f32(w.wv, xb, 1, kvd, dim)[0]
    q = orc.apply_rope_in_place(q, pos, cfg.head_dim)
    k = orc.apply_rope_in_place(k, pos, cfg.head_dim)
    k_cache[pos] = k
    v_cache[pos] = v
    att = orc.attention(q, k_cache, v_cache, cfg, pos, jit=False)
    x_mid = x + orc.gemm_q4_0_f32(w.wo, att, 1, dim, dim)[0]
    ffn = orc.scalar_rmsnorm(x_mid, w.rms_ffn, eps)
    gate = orc.gemm_q4_0_f32(w.w_gate, ffn, 1, hidden, dim)[0]
    up = orc.gemm_q4_0_f32(w.w_up, ffn, 1, hidden, dim)[0]
    with np.errstate(over="ignore"):
        act = (gate / (np.float32(1.0) + np.exp(-gate))) * up
    return x_mid + orc.gemm_q4_0_f32(w.w_down, act.astype(np.float32), 1, dim, hidden)[0]


REF_LAYER_TESTS = [
    # dim, hidden, heads, kv_heads, seeds base (rms, w, ffn), init_x seed
    (64, 128, 4, 4, (0x1001, 0x2001, 0x3001), 0x9999),   # transformer.rs:1000-1099
    (128, 256, 8, 2, (0x1101, 0x2101, 0x3101), 0x8888),  # transformer.rs:1102-1208
]


def ref_weights(dim, hidden, kvd, seeds):
    s_rms, s_w, s_ffn = seeds
    return orc.LayerWeights(
        rms_att=pseudo_random_f32(dim, s_rms), rms_ffn=pseudo_random_f32(dim, s_rms + 1),
        wq=quantize_matrix(dim, dim, s_w), wk=quantize_matrix(kvd, dim, s_w + 1),
        wv=quantize_matrix(kvd, dim, s_w + 2), wo=quantize_matrix(dim, dim, s_w + 3),
        w_gate=quantize_matrix(hidden, dim, s_ffn), w_up=quantize_matrix(hidden, dim, s_ffn + 1),
        w_down=quantize_matrix(dim, hidden, s_ffn + 2), hidden_dim=hidden)


@pytest.mark.parametrize("dim,hidden,heads,kvh,seeds,xseed", REF_LAYER_TESTS)
def test_oracle_block_matches_scalar_reference_within_1e4(dim, hidden, heads, kvh, seeds, xseed):
    cfg = orc.Cfg(dim, heads, kvh, 8, 1, 10000.0)
    w = ref_weights(dim, hidden, cfg.kv_dim, seeds)
    om = orc.OracleModel(cfg)
    x = pseudo_random_f32(dim, xseed)
    ref_x = x.copy()
    kc = np.zeros((8, cfg.kv_dim), np.float32)
    vc = np.zeros((8, cfg.kv_dim), np.float32)
    for pos in range(4):
        x = om.layer_forward(0, pos, x, w, 1e-5)[0]
        ref_x = scalar_layer_step(cfg, hidden, np.float32(1e-5), w, kc, vc, ref_x, pos)
        assert np.abs(x - ref_x).max() < 1e-4, f"pos {pos}"


def test_oracle_prefill_equals_sequential_decode_bitwise():
    # transformer.rs:1269-1358 checks that a batched prefill and a sequence of
    # forward_token give the same next token; the restatement runs the same
    # operations per row either way, so the residual stream and cache match
    dim, hidden, heads, kvh = 64, 128, 4, 2
    cfg = orc.Cfg(dim, heads, kvh, 16, 2, 10000.0)
    w = ref_weights(dim, hidden, cfg.kv_dim, (0x1001, 0x2001, 0x3001))
    x0 = np.stack([pseudo_random_f32(dim, 0x100 + t) for t in range(4)])
    batch, seq = orc.OracleModel(cfg), orc.OracleModel(cfg)
    xb = x0.copy()
    for layer in range(2):
        xb = batch.layer_forward(layer, 0, xb, w, 1e-5)
    xs = x0.copy()
    for t in range(4):
        row = xs[t]
        for layer in range(2):
            row = seq.layer_forward(layer, t, row, w, 1e-5)[0]
        xs[t] = row
    np.testing.assert_array_equal(xb, xs)
    np.testing.assert_array_equal(batch.kv, seq.kv)


def ref_model():
    """The reference's prefill test model (transformer.rs:1269-1313): dim 64,
    4 heads over 2 KV heads, hidden 128, msl 16, vocab 128, 2 layers sharing
    one set of weights, output_norm of ones."""
    dim, hidden, vocab = 64, 128, 128
    cfg = orc.Cfg(dim, 4, 2, 16, 2, 10000.0)
    lw = ref_weights(dim, hidden, cfg.kv_dim, (0x1001, 0x2001, 0x3001))
    w = orc.ModelWeights(token_embd=quantize_matrix(vocab, dim, 0x0100), layers=[lw, lw],
                         output_norm=np.ones(dim, np.float32),
                         lm_head=quantize_matrix(vocab, dim, 0x0200), vocab_size=vocab)
    return cfg, w


def test_sample_argmax_first_maximum_and_nan():
    assert orc.sample_argmax(np.float32([1, 3, 3, 2])) == 1
    assert orc.sample_argmax(np.float32([np.nan, 5, 1])) == 0
    assert orc.sample_argmax(np.float32([1, np.nan, 5, 5])) == 2
    assert orc.sample_argmax(np.float32([-np.inf, -np.inf])) == 0


def test_oracle_model_prefill_first_token_matches_sequential_forward():
    # transformer.rs:1314-1357: generate's first token (batched prefill)
    # equals the last forward_token of a token-by-token run
    cfg, w = ref_model()
    prompt = [1, 7, 19, 42]
    seq = orc.OracleModel(cfg)
    for pos, tok in enumerate(prompt):
        _, seq_next, _ = orc.model_forward(seq, w, 1e-5, [tok], pos)
    out = orc.model_generate(orc.OracleModel(cfg), w, 1e-5, prompt, 4)
    assert len(out) == 4 and out[0] == seq_next
    assert all(0 <= t < 128 for t in out)


def test_oracle_model_embedding_is_unit_length():
    cfg, w = ref_model()
    e = orc.model_embed(orc.OracleModel(cfg), w, 1e-5, [3, 9, 27, 81, 5])
    assert abs(np.linalg.norm(e.astype(np.float64)) - 1.0) < 1e-5
