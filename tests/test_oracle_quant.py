"""Pins of the quantized-projection oracle (oracle/quant.c) without the reference
binary.  Each check is chosen so that a plausible slip fails it:

- f32 <-> f16: numpy's float16 (an independent round-to-nearest-even
  implementation) on ties, subnormals, overflow and random values, and every
  one of the 63488 finite f16 bit patterns back to f32.
- quantize_row_q8_0: closed forms (zero block, one-hot block -> +-127), the
  rounding of every element recomputed as half-away-from-zero from the f32
  product (a rint/round-half-even slip fails), the reference's round-trip
  bound (blocks.rs:172-188).
- quantize_row_q4_0: the reference's round-trip bound, zero block and
  all-negative block cases (blocks.rs:153-220), the extreme element landing
  exactly on nibble 0 or 15.
- vec_dot scalar and AVX2: with unit scales the result is the exact integer
  dot of the unpacked weights and activations (pins nibble order, the -8
  offset and the weight/activation index pairing); the reference's own
  SIMD-vs-scalar bound 1e-5 (kernels.rs:340-358, 481-503) and GEMV-vs-f32
  bounds (kernels.rs:360-409); an f64 bound on the scalar sum order.
"""
import numpy as np
import pytest

from oracle import py_oracle as orc


def xorshift_unit(n: int, seed: int) -> np.ndarray:
    """pseudo_random_f32 of kernels.rs:286-296 / blocks.rs:141-151 up to the
    final affine map: xorshift32 states as f32 over u32::MAX as f32."""
    s = seed & 0xFFFFFFFF
    states = []
    for _ in range(n):
        s ^= (s << 13) & 0xFFFFFFFF
        s ^= s >> 17
        s ^= (s << 5) & 0xFFFFFFFF
        states.append(s)
    return np.array(states, dtype=np.uint32).astype(np.float32) / np.float32(4294967295.0)


def prand(n: int, seed: int) -> np.ndarray:
    """unit * 2.0 - 1.0 in f32 (the reference helper's output)."""
    u = xorshift_unit(n, seed)
    return (u * np.float32(2.0)) - np.float32(1.0)


def unpack_q4(blocks: np.ndarray) -> np.ndarray:
    """Integer weights [nblocks*32] in [-8, 7] (weight i: low nibble of byte i
    for i < 16, high nibble of byte i - 16)."""
    qs = blocks[:, 2:].astype(np.int64)
    return np.concatenate([(qs & 0x0F) - 8, (qs >> 4) - 8], axis=1).ravel()


def unpack_q8(blocks: np.ndarray) -> np.ndarray:
    return blocks[:, 2:].view(np.int8).astype(np.int64).ravel()


def scales(blocks: np.ndarray) -> np.ndarray:
    return blocks[:, :2].copy().view(np.uint16).ravel()


# ---- f16 conversion ----

def test_f32_to_f16_matches_numpy_float16():
    rng = np.random.default_rng(11)
    vals = [0.0, -0.0, 1.0, -1.0, 65504.0, 65519.0, 65520.0, 1e9, -1e9, 6.1035156e-05,
            5.9604645e-08, 2.9802322e-08, 2.9802326e-08, 8.940697e-08, 1e-10]
    # exact ties between consecutive f16 values (normal and subnormal)
    h = np.arange(0x0001, 0x7BFF, 37, dtype=np.uint16)
    lo = h.view(np.float16).astype(np.float64)
    hi = (h + 1).view(np.float16).astype(np.float64)
    ties = ((lo + hi) / 2).astype(np.float32)
    x = np.concatenate([np.array(vals, np.float32), ties, -ties,
                        (rng.standard_normal(20000) * 10.0 ** rng.uniform(-9, 5, 20000))
                        .astype(np.float32)])
    ours = orc.f32_to_f16_bits(x)
    with np.errstate(over="ignore"):
        ref = x.astype(np.float16).view(np.uint16)
    bad = np.nonzero(ours != ref)[0]
    assert bad.size == 0, [(float(x[i]), hex(ours[i]), hex(ref[i])) for i in bad[:5]]


def test_f16_to_f32_exact_for_every_finite_pattern():
    bits = np.arange(0, 1 << 16, dtype=np.uint32).astype(np.uint16)
    finite = np.isfinite(bits.view(np.float16))
    bits = bits[finite]
    ours = orc.f16_bits_to_f32(bits)
    ref = bits.view(np.float16).astype(np.float32)
    assert np.array_equal(ours.view(np.uint32), ref.view(np.uint32))


# ---- Q8_0 ----

def test_q8_0_closed_forms():
    z = orc.quantize_q8_0(np.zeros(64, np.float32))
    assert not z.any()  # scale 0.0, all weights 0
    x = np.zeros(32, np.float32)
    x[5] = -3.25
    b = orc.quantize_q8_0(x)[0]
    q = b[2:].view(np.int8)
    assert q[5] == -127 and np.count_nonzero(q) == 1
    assert scales(b[None])[0] == np.float32(np.float32(3.25) / np.float32(127.0)).astype(
        np.float16).view(np.uint16)


def test_q8_0_rounds_half_away_from_zero_elementwise():
    rng = np.random.default_rng(3)
    x = (rng.standard_normal(32 * 200) * 3).astype(np.float32)
    blocks = orc.quantize_q8_0(x)
    xb = x.reshape(-1, 32)
    amax = np.abs(xb).max(axis=1).astype(np.float32)
    inv = (np.float32(127.0) / amax).astype(np.float32)
    prod = (xb * inv[:, None]).astype(np.float32).astype(np.float64)
    want = np.sign(prod) * np.floor(np.abs(prod) + 0.5)
    want = np.clip(want, -127, 127).astype(np.int64)
    assert np.array_equal(unpack_q8(blocks).reshape(-1, 32), want)
    # a product that is an exact .5 must go away from zero
    t = np.zeros(32, np.float32)
    t[0] = 127.0
    t[1] = 2.5
    t[2] = -2.5
    q = orc.quantize_q8_0(t)[0, 2:].view(np.int8)
    assert (q[0], q[1], q[2]) == (127, 3, -3)


def test_q8_0_reference_roundtrip_bound():
    # blocks.rs:172-188
    x = prand(256, 0x87654321)
    rec = orc.dequantize_q8_0(orc.quantize_q8_0(x))
    assert np.abs(x - rec).max() <= 0.005


# ---- Q4_0 ----

def test_q4_0_reference_roundtrip_and_edge_cases():
    # blocks.rs:153-170
    x = prand(256, 0x12345678)
    rec = orc.dequantize_q4_0(orc.quantize_q4_0(x))
    assert np.abs(x - rec).max() <= 0.0725
    # blocks.rs:190-220
    zb = orc.quantize_q4_0(np.zeros(64, np.float32))
    assert (scales(zb) == 0).all() and (orc.dequantize_q4_0(zb) == 0).all()
    neg = -(np.arange(32, dtype=np.float32) + 1) * np.float32(10.0)
    rec = orc.dequantize_q4_0(orc.quantize_q4_0(neg))
    assert np.abs(neg - rec).max() <= 20.5
    # the block minimum -320 = -8 * d with d = 40 exactly: nibble 0, exact
    assert rec[31] == -320.0 and unpack_q4(orc.quantize_q4_0(neg))[31] == -8


def test_q4_0_extremes_use_the_full_range():
    rng = np.random.default_rng(5)
    x = rng.standard_normal(32 * 100).astype(np.float32)
    w = unpack_q4(orc.quantize_q4_0(x)).reshape(-1, 32)
    xb = x.reshape(-1, 32)
    arg = np.abs(xb).argmax(axis=1)
    ext = w[np.arange(len(w)), arg]
    # the largest-magnitude element maps to -8 (if it decides the scale sign)
    assert ((ext == -8) | (ext == 7) | (ext == -7)).all()
    assert (w >= -8).all() and (w <= 7).all()


# ---- dot products ----

def unit_scale_blocks(rng, nblocks):
    """Q4_0 and Q8_0 blocks with f16 scale 1.0 and random payloads."""
    w = np.zeros((nblocks, 18), np.uint8)
    a = np.zeros((nblocks, 34), np.uint8)
    w[:, 0:2] = np.array([0x00, 0x3C], np.uint8)  # f16 1.0, little-endian
    a[:, 0:2] = np.array([0x00, 0x3C], np.uint8)
    w[:, 2:] = rng.integers(0, 256, (nblocks, 16), dtype=np.uint8)
    a[:, 2:] = rng.integers(-127, 128, (nblocks, 32), dtype=np.int8).view(np.uint8)
    return w, a


@pytest.mark.parametrize("avx2", [False, True])
def test_vec_dot_is_the_exact_integer_dot_at_unit_scales(avx2):
    rng = np.random.default_rng(9)
    for nb in (1, 3, 17, 128):
        w, a = unit_scale_blocks(rng, nb)
        exact = int(np.dot(unpack_q4(w), unpack_q8(a)))
        assert abs(exact) < 2 ** 24  # every partial sum is exact in f32
        assert orc.vec_dot_q4_0_q8_0(w, a, avx2=avx2) == float(exact)


def test_vec_dot_avx2_matches_scalar_within_reference_bound():
    # kernels.rs:340-358
    w = orc.quantize_q4_0(prand(1024, 0x11223344))
    a = orc.quantize_q8_0(prand(1024, 0x55667788))
    assert abs(orc.vec_dot_q4_0_q8_0(w, a) - orc.vec_dot_q4_0_q8_0(w, a, avx2=True)) < 1e-5
    # kernels.rs:481-503 (odd block counts)
    for nb in (1, 3, 7, 17):
        w = orc.quantize_q4_0(prand(nb * 32, 0x1000 + nb))
        a = orc.quantize_q8_0(prand(nb * 32, 0x2000 + nb))
        assert abs(orc.vec_dot_q4_0_q8_0(w, a) - orc.vec_dot_q4_0_q8_0(w, a, avx2=True)) < 1e-5


def test_vec_dot_scalar_reference_bounds_and_f64_order_bound():
    # kernels.rs:306-325: quantized dot within 1e-2 relative of the f32 dot
    w_f = prand(4096, 0xCAFEBABE) + np.float32(0.5)
    a_f = prand(4096, 0xDEADBEEF) + np.float32(0.5)
    w = orc.quantize_q4_0(w_f)
    a = orc.quantize_q8_0(a_f)
    q = orc.vec_dot_q4_0_q8_0(w, a)
    ref = np.float32(0.0)
    for i in range(4096):
        ref = np.float32(ref + np.float32(w_f[i] * a_f[i]))
    assert abs(ref - q) / abs(ref) < 1e-2
    # exact value of the same quantized data in f64: the sequential f32 sum of
    # 128 block terms stays within 128 half-ulps of the running magnitude
    isum = (unpack_q4(w) * unpack_q8(a)).reshape(-1, 32).sum(axis=1)
    d = (orc.f16_bits_to_f32(scales(w)).astype(np.float64)
         * orc.f16_bits_to_f32(scales(a)).astype(np.float64))
    exact = float((isum * d).sum())
    assert abs(q - exact) <= 128 * np.spacing(np.float32(abs(exact) * 2))


def test_gemv_reference_bounds():
    # kernels.rs:360-409 (rows 512 of the test, first 64 here), scalar and AVX2
    rows, cols = 64, 4096
    w_f = (prand(rows * cols, 0x99AABBCC) + np.float32(0.5)).reshape(rows, cols)
    x_f = prand(cols, 0xDDEEFF11) + np.float32(0.5)
    w = orc.quantize_q4_0(w_f)
    xq = orc.quantize_q8_0(x_f)
    s = orc.gemm_q4_0(w, xq, 1, rows, cols)[0]
    v = orc.gemm_q4_0(w, xq, 1, rows, cols, avx2=True)[0]
    assert (np.abs(s - v) / np.maximum(np.abs(s), 1.0)).max() < 1e-5
    ref = (w_f.astype(np.float64) @ x_f.astype(np.float64))
    rel = np.abs(ref - v) / np.abs(ref)
    assert rel.max() < 1.5e-2 and rel.mean() < 1e-2


def test_gemm_batch_layout():
    # output[b*rows + r] = vec_dot(W row r, x row b) (kernels.rs:386-393)
    rng = np.random.default_rng(2)
    batch, rows, cols = 3, 5, 96
    w = orc.quantize_q4_0(rng.standard_normal(rows * cols).astype(np.float32))
    xq = orc.quantize_q8_0(rng.standard_normal(batch * cols).astype(np.float32))
    out = orc.gemm_q4_0(w, xq, batch, rows, cols)
    nb = cols // 32
    for b in range(batch):
        for r in range(rows):
            assert out[b, r] == orc.vec_dot_q4_0_q8_0(w[r * nb:(r + 1) * nb],
                                                      xq[b * nb:(b + 1) * nb])
