"""Shared helpers for the tests: configs, seeded inputs, tolerance checks and
loading of the product package (whose directory name has a hyphen)."""
from __future__ import annotations

import importlib.util
import os
import sys
from dataclasses import dataclass
from pathlib import Path

import numpy as np

REPO = Path(__file__).resolve().parents[1]
if str(REPO) not in sys.path:
    sys.path.insert(0, str(REPO))

from oracle import py_oracle  # noqa: E402  (checker)

# Tolerance of the parity bar: max-abs 1e-4 and max-rel 1e-3, the relative
# error taken against max(|ref|, ATOL/RTOL) so that values near zero are held
# to the absolute bound.  KV-cache rows are compared bit for bit.
ATOL = 1e-4
RTOL = 1e-3


def load_product():
    """Imports static-lm_amd/ as module `static_lm_amd`."""
    name = "static_lm_amd"
    if name in sys.modules:
        return sys.modules[name]
    spec = importlib.util.spec_from_file_location(name, REPO / "static-lm_amd" / "__init__.py")
    mod = importlib.util.module_from_spec(spec)
    sys.modules[name] = mod
    spec.loader.exec_module(mod)
    return mod


@dataclass(frozen=True)
class Workload:
    name: str
    dim: int
    num_heads: int
    num_kv_heads: int
    max_seq_len: int
    num_layers: int
    theta: float
    prefill: int
    decode: int
    prefilled: int = 0  # rows written raw into the cache before the run
    seed: int = 0

    @property
    def head_dim(self):
        return self.dim // self.num_heads

    @property
    def kv_dim(self):
        return self.head_dim * self.num_kv_heads

    def cfg(self) -> py_oracle.Cfg:
        return py_oracle.Cfg(self.dim, self.num_heads, self.num_kv_heads, self.max_seq_len,
                             self.num_layers, self.theta)


WORKLOADS = {
    # the true built-in synthetic model of src/main.rs:266-274
    "c0": Workload("synthetic-main", 256, 8, 2, 64, 2, 1e4, 16, 8, seed=0x5EED0000),
    "c1": Workload("synthetic-256", 256, 4, 4, 512, 2, 1e4, 16, 8, seed=0x5EED0001),
    "c2": Workload("stories15m", 288, 6, 6, 256, 6, 1e4, 16, 64, seed=0x5EED0002),
    "c3": Workload("smollm2-135m", 576, 9, 3, 2048, 30, 1e5, 512, 256, seed=0x5EED0003),
    "c4": Workload("llama3-8b", 4096, 32, 8, 8192, 1, 5e5, 4096, 128, seed=0x5EED0004),
    "c5": Workload("llama3-8b-long", 4096, 32, 8, 131136, 1, 5e5, 0, 64, prefilled=131072,
                   seed=0x5EED0005),
    # shapes of the reference's own layer tests (transformer.rs:1000-1011, 1269-1278)
    "ref_mha": Workload("ref-mha", 64, 4, 4, 8, 1, 1e4, 2, 2, seed=0x5EED0010),
    "ref_gqa": Workload("ref-gqa", 64, 4, 2, 16, 2, 1e4, 4, 4, seed=0x5EED0011),
}


def gen(seed, shape) -> np.ndarray:
    """Seeded N(0,1)*0.5 f32."""
    rng = np.random.default_rng(seed)
    return rng.standard_normal(shape, dtype=np.float32) * np.float32(0.5)


def layer_inputs(w: Workload, layer: int):
    rows = w.prefill + w.decode
    q = gen([w.seed, layer, 0], (rows, w.dim))
    k = gen([w.seed, layer, 1], (rows, w.kv_dim))
    v = gen([w.seed, layer, 2], (rows, w.kv_dim))
    return q, k, v


def prefilled_rows(w: Workload, layer: int, which: int, pos0: int, n: int) -> np.ndarray:
    """Raw (already-final) cache rows for a pre-filled workload, by block of
    4096 positions so any sub-range can be regenerated on its own."""
    out = np.empty((n, w.kv_dim), np.float32)
    blk = 4096
    p = pos0
    while p < pos0 + n:
        b = p // blk
        rows = gen([w.seed, layer, 10 + which, b], (blk, w.kv_dim))
        lo = p - b * blk
        take = min(blk - lo, pos0 + n - p)
        out[p - pos0:p - pos0 + take] = rows[lo:lo + take]
        p += take
    return out


def err_stats(got, ref, atol=ATOL, rtol=RTOL):
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    diff = np.abs(got - ref)
    rel = diff / np.maximum(np.abs(ref), atol / rtol)
    return float(diff.max(initial=0.0)), float(rel.max(initial=0.0))


# |ref| above which the unfloored relative error is reported
UNFLOORED_MIN = 1e-2


def err_report(got, ref, atol=ATOL, rtol=RTOL) -> dict:
    """max-abs, the floored max-rel of the bar (against max(|ref|, 0.1)), and
    the unfloored max-rel over the elements with |ref| >= 1e-2, with the
    largest |ref| for scale."""
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    diff = np.abs(got - ref)
    big = np.abs(ref) >= UNFLOORED_MIN
    return {
        "max_abs": float(diff.max(initial=0.0)),
        "max_rel": float((diff / np.maximum(np.abs(ref), atol / rtol)).max(initial=0.0)),
        "max_rel_unfloored": float((diff[big] / np.abs(ref[big])).max(initial=0.0)),
        "max_ref": float(np.abs(ref).max(initial=0.0)),
    }


# Worst errors per test, printed in the pytest summary (tests/conftest.py).
WORST: dict = {}


def _note(rep: dict) -> None:
    test = os.environ.get("PYTEST_CURRENT_TEST", "?").split(" ")[0]
    w = WORST.setdefault(test, {"n": 0, "max_abs": 0.0, "max_rel": 0.0,
                                "max_rel_unfloored": 0.0, "max_ref": 0.0})
    w["n"] += 1
    for k in ("max_abs", "max_rel", "max_rel_unfloored", "max_ref"):
        w[k] = max(w[k], rep[k])


def assert_close(got, ref, atol=ATOL, rtol=RTOL, what=""):
    got = np.asarray(got)
    ref = np.asarray(ref)
    assert got.shape == ref.shape, (got.shape, ref.shape)
    assert np.all(np.isfinite(got)), f"{what}: non-finite values"
    rep = err_report(got, ref, atol, rtol)
    _note(rep)
    mabs, mrel = rep["max_abs"], rep["max_rel"]
    assert mabs <= atol and mrel <= rtol, (
        f"{what}: max-abs {mabs:.3e} max-rel {mrel:.3e} "
        f"(unfloored {rep['max_rel_unfloored']:.3e} over |ref| >= {UNFLOORED_MIN})")


def assert_bitwise(got, ref, what=""):
    got = np.ascontiguousarray(got, np.float32)
    ref = np.ascontiguousarray(ref, np.float32)
    assert got.shape == ref.shape, (got.shape, ref.shape)
    neq = got.view(np.uint32) != ref.view(np.uint32)
    assert not neq.any(), f"{what}: {int(neq.sum())} of {neq.size} words differ"


def xorshift_f32(n: int, seed: int, lo: float, span: float) -> np.ndarray:
    """The reference tests' pseudo_random_f32: xorshift32, unit = seed as f32 /
    u32::MAX as f32, value = unit*span + lo in f32 (engine.rs:214-224 uses
    span 4, lo -2)."""
    out = np.empty(n, np.float32)
    s = seed & 0xFFFFFFFF
    umax = np.float32(4294967295.0)
    for i in range(n):
        s ^= (s << 13) & 0xFFFFFFFF
        s ^= s >> 17
        s ^= (s << 5) & 0xFFFFFFFF
        unit = np.float32(np.float32(s) / umax)
        out[i] = np.float32(np.float32(unit * np.float32(span)) + np.float32(lo))
    return out


# Which prefill kernel a batch takes, restated from the dispatch rules for
# choosing test cases (the library answers the same question through
# slm_attn_prefill_kernel; tests/test_abi.py checks the two agree).
def takes_key_splits(dim, heads, kv_heads, start, n, cus=256):
    """Whether a prefill takes the one-head key-split kernel (prefill_plan.h):
    head_dim <= 64, fewer than two workgroups per CU in the
    head-group tiling, at least 8 key tiles in the heaviest block."""
    hd = dim // heads
    kv_mul = heads // kv_heads
    hw = 4 if kv_mul % 4 == 0 else 3 if kv_mul % 3 == 0 else 2 if kv_mul % 2 == 0 else 1
    qs = {4: 1, 3: 1, 2: 2, 1: 4}[hw]
    wgs = -(-n // (16 * qs)) * (heads // hw)
    return hd <= 64 and wgs < 2 * cus and (start + n + 31) // 32 >= 8


def paired_blocks(dim, heads, kv_heads, n, cus=256):
    """Which paired-block kernel an hd-128 prefill of n rows takes (blocks i
    and n_qb-1-i per workgroup), or None: for at least 256 rows whose
    head-group tiling gives at most one workgroup per CU, one head and four
    key splits ("h1k4") while pairs x heads fit the CUs, else two heads and
    two key splits ("h2k2") for an even kv_mul while pairs x heads/2 fit."""
    hd = dim // heads
    kv_mul = heads // kv_heads
    hw, qs = (4, 1) if kv_mul % 4 == 0 else (3, 1) if kv_mul % 3 == 0 else \
        (2, 2) if kv_mul % 2 == 0 else (1, 4)
    wgs = -(-n // (16 * qs)) * (heads // hw)
    pairs = (-(-n // 16) + 1) // 2
    if hd != 128 or n < 256 or wgs > cus:
        return None
    if pairs * heads <= cus:
        return "h1k4"
    if kv_mul % 2 == 0 and pairs * (heads // 2) <= cus:
        return "h2k2"
    return None


def paired_dma(dim, heads, kv_heads, n, cus=256):
    """hd-128 prefills of 512 rows or more with kv_mul a multiple of 4 that
    the short paired kernels leave take the DMA-fed kernel with paired blocks
    (blocks i and n_qb-1-i, four heads) when the four-head grid has more
    workgroups than CUs and the paired grid is at most the CU count or a
    whole multiple of it."""
    kv_mul = heads // kv_heads
    wgs = -(-n // 16) * (heads // 4)
    pwgs = (-(-n // 16) + 1) // 2 * (heads // 4)
    return (dim // heads == 128 and kv_mul % 4 == 0 and n >= 512
            and paired_blocks(dim, heads, kv_heads, n, cus) is None
            and wgs > cus and (pwgs <= cus or pwgs % cus == 0))


def paired_register(dim, heads, kv_heads, start, n, cus=256):
    """Prefills of hd 16-96 with kv_mul a multiple of 4 that the one-head
    key-split kernel leaves take the four-head register kernel with paired
    blocks when the four-head grid has more workgroups than CUs and the
    paired grid is at most one or two per CU."""
    hd, kv_mul = dim // heads, heads // kv_heads
    wgs = -(-n // 16) * (heads // 4)
    pwgs = (-(-n // 16) + 1) // 2 * (heads // 4)
    key_splits = hd <= 64 and wgs < 2 * cus and (start + n + 31) // 32 >= 8
    return (hd <= 96 and kv_mul % 4 == 0 and not key_splits and wgs > cus
            and (pwgs <= cus or pwgs == 2 * cus))


# Prefill kernels (slm_attn_prefill_kernel, static-lm_amd PREFILL_KERNELS) and
# a batch that takes each one on a 256-CU device.
SWEEP_TARGETED = [
    # dim, heads, kv_heads, start, n, kernel
    (2048, 32, 8, 0, 100, "four_heads"),          # hd 64 GQA 4, 56 workgroups
    (576, 9, 3, 0, 64, "three_heads"),            # the SmolLM2-135M shape, two key tiles
    (1536, 16, 8, 5, 200, "two_heads"),           # hd 96, kv_mul 2
    (768, 16, 16, 0, 40, "one_head"),             # hd 48 MHA
    (576, 9, 3, 0, 512, "key_split"),             # the SmolLM2-135M shape, 512 rows
    (3072, 32, 8, 0, 1024, "paired_four_heads"),  # hd 96 GQA 4, 256 paired workgroups
    (8192, 64, 16, 3, 2100, "dma"),               # hd 128, 1056 workgroups (not a multiple of 256)
    (4096, 32, 8, 0, 1024, "dma_paired"),         # the Llama-3-8B shape, 256 paired workgroups
    (4096, 32, 8, 0, 300, "paired_two_heads"),    # the Llama-3-8B shape, 10 pairs
    (4096, 32, 8, 0, 256, "paired_one_head"),     # the Llama-3-8B shape, 8 pairs
]


def sweep_random_cases(count=30, seed=20261202):
    """Seeded random shapes and batches: (dim, heads, kv_heads, start, n).
    Head dims the library compiles, kv_mul 1/2/3/4/8 with 1-8 KV heads (at
    most 64 query heads), configs the reference accepts (dim and kv_dim
    multiples of 32), starts 0-1499 half the time, n log-uniform in 1-2600."""
    rng = np.random.default_rng(seed)
    out = []
    while len(out) < count:
        hd = int(rng.choice((16, 32, 48, 64, 96, 128, 256)))
        kv_mul = int(rng.choice((1, 2, 3, 4, 8)))
        kvh = int(rng.choice((1, 2, 3, 4, 8)))
        heads = kvh * kv_mul
        if heads > 64 or (heads * hd) % 32 or (kvh * hd) % 32:
            continue
        start = int(rng.integers(0, 1500)) if rng.random() < 0.5 else 0
        n = max(1, int(np.exp(rng.uniform(0.0, np.log(2600.0)))))
        out.append((heads * hd, heads, kvh, start, n))
    return out
