"""C-ABI checks that need no GPU: the library loads, exports every function
include/*.h declares, and rejects bad arguments with the codes that mirror the
reference's asserts before touching a device."""
import ctypes
import subprocess

import pytest

from slm_testlib import (SWEEP_TARGETED, load_product, paired_blocks, paired_dma,
                         paired_register, sweep_random_cases, takes_key_splits)

P = load_product()


def test_library_exports_every_header_function():
    declared = P.header_functions()
    assert len(declared) >= 20
    lib = P.load_library()
    for name in declared:
        assert hasattr(lib, name), name
    assert set(declared) == set(P.SIGNATURES), "binding table out of step with the header"
    nm = subprocess.run(["nm", "-D", "--defined-only", str(P.LIB_PATH)], capture_output=True,
                        text=True, check=True).stdout
    exported = {ln.split()[-1] for ln in nm.splitlines() if " T " in ln}
    assert set(declared) <= exported


def test_measurement_probes_live_in_their_own_library():
    # the bench's probes are libslm_calib.so, not exported by the product
    declared = P.header_functions(P.CALIB_HEADER_PATH)
    assert set(declared) == set(P.CALIB_SIGNATURES)
    nm = subprocess.run(["nm", "-D", "--defined-only", str(P.LIB_PATH)], capture_output=True,
                        text=True, check=True).stdout
    assert not any("slm_calib" in ln for ln in nm.splitlines())
    cal = P.load_calib_library()
    for name in declared:
        assert hasattr(cal, name), name
    # argument checks before any HIP call
    assert cal.slm_calib_mfma_f32(0, 0, None, None) == P.ERR_ARG
    assert cal.slm_calib_hbm_read(0, 1 << 20, 1, None) == P.ERR_ARG


def test_version_and_null_handles():
    lib = P.load_library()
    assert b"gfx950" in lib.slm_attn_version()
    assert lib.slm_attn_sync(None) == P.ERR_ARG
    assert lib.slm_attn_decode(None, 0, 0, None, None, None, None) == P.ERR_ARG
    assert lib.slm_attn_prefill_dev(None, 0, 0, 1, None, None, None, None) == P.ERR_ARG
    assert lib.slm_kv_offset(None, 0, 0, 0) == ctypes.c_size_t(-1).value
    assert lib.slm_kv_device_ptr(None) is None
    lib.slm_attn_destroy(None)  # no-op
    g = ctypes.c_void_p(1)
    assert lib.slm_attn_capture_begin(None) == P.ERR_ARG
    assert lib.slm_attn_capture_end(None, ctypes.byref(g)) == P.ERR_ARG
    assert lib.slm_attn_graph_launch(None, None) == P.ERR_ARG
    lib.slm_attn_graph_destroy(None)  # no-op
    # quantized projections: argument checks before any device work
    out = P._P()
    assert lib.slm_q4_matrix_create(0, None, 4, 32, ctypes.byref(out)) == P.ERR_ARG
    blk = (ctypes.c_uint8 * 18)()
    assert lib.slm_q4_matrix_create(0, ctypes.addressof(blk), 1, 48, ctypes.byref(out)) == P.ERR_SHAPE
    assert lib.slm_q4_matrix_create(0, ctypes.addressof(blk), 0, 32, ctypes.byref(out)) == P.ERR_SHAPE
    assert lib.slm_quantize_q8_0_dev(None, None, 32, None) == P.ERR_ARG
    assert lib.slm_gemm_q4_0_dev(None, None, None, 1, None) == P.ERR_ARG
    assert lib.slm_attn_decode_xb_dev(None, 0, 0, None, None, None, None, None) == P.ERR_ARG
    assert lib.slm_attn_decode_xb_dev_noalloc(None, 0, 0, None, None, None, None, None) == P.ERR_ARG
    lib.slm_q4_matrix_destroy(None)  # no-op


@pytest.mark.parametrize("dim,heads,kv_heads,msl,layers,theta,why", [
    (250, 5, 5, 8, 1, 1e4, "dim must be a multiple of 32"),
    (256, 3, 3, 8, 1, 1e4, "dim must be divisible by num_heads"),
    (256, 8, 3, 8, 1, 1e4, "num_heads must be divisible by num_kv_heads"),
    (96, 32, 32, 8, 1, 1e4, "head_dim must be even"),
    (64, 4, 1, 8, 1, 1e4, "kv_dim must be a multiple of 32"),
    (64, 4, 4, 0, 1, 1e4, "max_seq_len and num_layers must be positive"),
    (64, 4, 4, 8, 0, 1e4, "max_seq_len and num_layers must be positive"),
    (64, 4, 4, 8, 1, 0.0, "rope_theta"),
    (64, 0, 0, 8, 1, 1e4, "num_heads and num_kv_heads must be positive"),
])
def test_create_rejects_configs_the_reference_asserts_on(dim, heads, kv_heads, msl, layers, theta,
                                                         why):
    with pytest.raises(P.SlmAttnError) as ei:
        P.AttentionContext(dim, heads, kv_heads, msl, layers, theta)
    assert ei.value.code == P.ERR_CONFIG
    assert why in ei.value.message


def test_create_rejects_uncompiled_head_dim():
    # head_dim 40 satisfies every reference assert (dim 320, 8 heads) but has
    # no compiled kernel
    with pytest.raises(P.SlmAttnError) as ei:
        P.AttentionContext(320, 8, 8, 16, 1)
    assert ei.value.code == P.ERR_UNSUPPORTED


def test_create_rejects_kv_dim_past_the_tile_offset_limit():
    # 65,600 KV heads of 16 dims: kv_dim 1,049,600 > 2^20, whose 32-row tile
    # offsets the prefill kernels could not hold in 32 bits; refused before
    # any device call
    with pytest.raises(P.SlmAttnError) as ei:
        P.AttentionContext(16 * 65600, 65600, 65600, 4, 1)
    assert ei.value.code == P.ERR_UNSUPPORTED
    assert "kv_dim" in ei.value.message


TILE_RANGE_PROBE = r"""
#include <stdio.h>
#include "tile_range.h"
int main(void) {
    static const int cases[][4] = {
        /* kv_len, kb, tile_rows, kv_dim */
        {1048600, 0, 32, 1024},     /* one layer's K slice past 4 GiB: the first tile */
        {1048600, 1048576, 32, 1024},  /* the tile at row 2^20: 24 rows left */
        {1048600, 1048576 + 8, 32, 1024},  /* 16 rows left */
        {262144, 0, 32, 4096},      /* hd-128 MHA, 262,144 rows: 4 GiB per slice */
        {2147483647, 0, 32, 1 << 20},  /* the largest kv_dim a context accepts */
        {100, 100, 32, 1024},       /* no rows left */
        {2147483647, 2147483647 - 5, 32, 1 << 20},  /* 5 rows left at the largest position */
    };
    for (unsigned i = 0; i < sizeof(cases) / sizeof(cases[0]); ++i)
        printf("%u\n", slm::tile_range_bytes(cases[i][0], cases[i][1], cases[i][2], cases[i][3]));
    printf("%d %d\n", (int)slm::tile_range_fits(32, slm::kMaxKvDim),
           (int)slm::tile_range_fits(1 << 11, 1 << 20));
    return 0;
}
"""


def test_prefill_tile_range_is_bounded_by_the_tile(tmp_path):
    """The prefill kernels' buffer-descriptor range (csrc/tile_range.h),
    compiled for the host: a layer slice past 4 GiB (1,048,600 rows of 1024
    floats) must still give whole 32-row tiles, where the 32-bit product
    (kv_len - kb) * kv_dim * 4 wrapped to 24 rows for the first tile."""
    src = tmp_path / "probe.cpp"
    src.write_text(TILE_RANGE_PROBE)
    exe = tmp_path / "probe"
    subprocess.run(["g++", "-std=c++17", "-O1", "-Wall", "-Werror",
                    f"-I{P.PKG_DIR / 'csrc'}", str(src), "-o", str(exe)], check=True)
    got = [int(x) for x in subprocess.run([str(exe)], capture_output=True, text=True,
                                          check=True).stdout.split()]
    row = 1024 * 4
    assert got[:7] == [32 * row, 24 * row, 16 * row, 32 * 4096 * 4, 32 * (1 << 20) * 4, 0,
                       5 * (1 << 20) * 4]
    # the kernels' 32-row tiles at the largest kv_dim a context accepts fit
    # 32 bits; 2048-row tiles at that kv_dim would not
    assert got[7:] == [1, 0]
    # what the old 32-bit product gave for the first case: the wrap the
    # clamp removes
    assert (1048600 * 1024 * 4) % (1 << 32) == 24 * row


PLAN_PROBE = r"""
#include <stdio.h>
#include "prefill_plan.h"
int main(void) {
    int hd, heads, kv_mul, cus, start, n;
    while (scanf("%d %d %d %d %d %d", &hd, &heads, &kv_mul, &cus, &start, &n) == 6)
        printf("%d\n", (int)slm::prefill_plan(hd, heads, kv_mul, cus, start, n));
    return 0;
}
"""


@pytest.fixture(scope="module")
def prefill_plan(tmp_path_factory):
    """csrc/prefill_plan.h compiled for the host: kernel names for a list of
    (head_dim, heads, kv_mul, cus, start, n)."""
    d = tmp_path_factory.mktemp("plan")
    src = d / "plan.cpp"
    src.write_text(PLAN_PROBE)
    exe = d / "plan"
    subprocess.run(["g++", "-std=c++17", "-O1", "-Wall", "-Werror",
                    f"-I{P.PKG_DIR / 'csrc'}", str(src), "-o", str(exe)], check=True)

    def plan(cases):
        inp = "".join(" ".join(str(x) for x in c) + "\n" for c in cases)
        out = subprocess.run([str(exe)], input=inp, capture_output=True, text=True,
                             check=True).stdout.split()
        assert len(out) == len(cases)
        return [P.PREFILL_KERNELS[int(x)] for x in out]
    return plan


def _plan_grid():
    ns = sorted(set(range(1, 41)) | set(range(41, 9000, 37)) |
                {m + d for m in (256, 512, 1024, 2048, 4096, 8192) for d in (-17, -1, 0, 1, 15)})
    for hd in (16, 32, 48, 64, 96, 128, 256):
        for kv_mul in (1, 2, 3, 4, 8):
            for kvh in (1, 2, 4, 8):
                for cus in (256, 32):
                    for start in (0, 7, 1000):
                        for n in ns:
                            yield hd, kvh * kv_mul, kv_mul, cus, start, n


def test_prefill_plan_picks_only_compiled_kernels(prefill_plan):
    # the launcher has each kernel for some head dims and head groupings only
    # (anything else returns hipErrorInvalidValue); the plan must never pick
    # one outside them
    def compiled(hd, kv_mul, k):
        return {"four_heads": kv_mul % 4 == 0, "three_heads": kv_mul % 3 == 0,
                "two_heads": kv_mul % 2 == 0, "one_head": True, "key_split": hd <= 64,
                "paired_four_heads": hd <= 96 and kv_mul % 4 == 0,
                "dma": hd == 128 and kv_mul % 4 == 0, "dma_paired": hd == 128 and kv_mul % 4 == 0,
                "paired_two_heads": hd == 128 and kv_mul % 2 == 0,
                "paired_one_head": hd == 128}[k]
    grid = list(_plan_grid())
    got = prefill_plan(grid)
    bad = [(c, k) for c, k in zip(grid, got) if not compiled(c[0], c[2], k)]
    assert not bad, bad[:5]
    assert set(got) == set(P.PREFILL_KERNELS)


def test_prefill_plan_agrees_with_the_restated_rules(prefill_plan):
    # two codings of the same dispatch rules: the header the library compiles
    # and the test library's restatement used to choose parity cases
    grid = list(_plan_grid())
    got = prefill_plan(grid)
    for (hd, heads, kv_mul, cus, start, n), k in zip(grid, got):
        dim, kvh = heads * hd, heads // kv_mul
        case = (hd, heads, kv_mul, cus, start, n, k)
        assert (k == "key_split") == takes_key_splits(dim, heads, kvh, start, n, cus), case
        pb = paired_blocks(dim, heads, kvh, n, cus)
        assert (k == "paired_one_head") == (pb == "h1k4"), case
        assert (k == "paired_two_heads") == (pb == "h2k2"), case
        assert (k == "dma_paired") == paired_dma(dim, heads, kvh, n, cus), case
        assert (k == "paired_four_heads") == paired_register(dim, heads, kvh, start, n, cus), case


def test_dispatch_sweep_reaches_every_prefill_kernel(prefill_plan):
    # the GPU sweep's targeted batches take the kernels they name on a 256-CU
    # device, and together reach every prefill kernel
    cases = [(dim // heads, heads, heads // kvh, 256, start, n)
             for dim, heads, kvh, start, n, _ in SWEEP_TARGETED]
    got = prefill_plan(cases)
    assert got == [c[5] for c in SWEEP_TARGETED]
    assert set(got) == set(P.PREFILL_KERNELS)
    rnd = sweep_random_cases()
    kinds = prefill_plan([(dim // heads, heads, heads // kvh, 256, start, n)
                          for dim, heads, kvh, start, n in rnd])
    assert len(set(kinds)) >= 5, kinds


def test_prefill_kernel_query_checks_its_arguments():
    lib = P.load_library()
    k = ctypes.c_int32(-1)
    assert lib.slm_attn_prefill_kernel(None, 0, 1, ctypes.byref(k)) == P.ERR_ARG
    assert k.value == -1


def test_header_numbers_the_prefill_kernels_like_the_binding():
    text = P.HEADER_PATH.read_text()
    for i, name in enumerate(P.PREFILL_KERNELS):
        assert f"SLM_PF_{name.upper()} = {i}," in text or f"SLM_PF_{name.upper()} = {i} " in text, name


def test_header_declares_error_codes_the_binding_uses():
    text = "".join(h.read_text() for h in (P.HEADER_PATH, P.QUANT_HEADER_PATH,
                                             P.LAYER_HEADER_PATH, P.GGUF_HEADER_PATH))
    for code, name in P.ERRORS.items():
        assert f"#define {name} ({code})" in text


class _RecordingLib:
    """Stands in for the library: records the calls a graph's lifetime makes."""

    def __init__(self):
        self.calls = []

    def slm_attn_sync(self, h):
        self.calls.append(("sync", h))
        return P.SLM_OK

    def slm_attn_graph_destroy(self, g):
        self.calls.append(("graph_destroy", g))

    def slm_attn_destroy(self, h):
        self.calls.append(("destroy", h))

    def slm_attn_last_error(self, h):
        return b""


def _fake_context(lib):
    ctx = P.AttentionContext.__new__(P.AttentionContext)
    ctx.lib = lib
    ctx._h = "ctx"
    ctx._graphs = P.weakref.WeakSet()
    return ctx


def test_graph_is_destroyed_after_a_sync_and_before_its_context():
    # slm_attn.h: destroy a graph only after its replays have finished, and
    # before its context
    lib = _RecordingLib()
    ctx = _fake_context(lib)
    g = P.AttentionGraph(ctx, "g1")
    ctx._graphs.add(g)
    g.close()
    g.close()  # no-op
    assert lib.calls == [("sync", "ctx"), ("graph_destroy", "g1")]
    # a live graph is closed by its context, ahead of the context itself
    lib.calls.clear()
    g2 = P.AttentionGraph(ctx, "g2")
    ctx._graphs.add(g2)
    ctx.close()
    assert lib.calls == [("sync", "ctx"), ("graph_destroy", "g2"), ("destroy", "ctx")]
    lib.calls.clear()
    g2.close()
    del g2
    assert lib.calls == []


def test_temporary_graph_keeps_its_context_alive():
    # a graph dropped without close() (e.g. ctx.graph_launch(ctx.capture_end()))
    # still syncs before destroying, because it holds its context
    import gc
    lib = _RecordingLib()
    ctx = _fake_context(lib)
    g = P.AttentionGraph(ctx, "g3")
    ctx._graphs.add(g)
    del ctx
    gc.collect()
    assert lib.calls == []  # the graph holds the context
    del g
    gc.collect()
    assert lib.calls[:2] == [("sync", "ctx"), ("graph_destroy", "g3")]
