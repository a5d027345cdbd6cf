#!/usr/bin/env python3
"""Benchmark of the static-lm attention hot path on one MI355X.

Headline (`value`): decode attention HBM throughput at 32k context on the
Llama-3-8B head shape (32 heads over 8 KV heads, head_dim 128, f32 KV).  One
step is one decode token through 8 layers whose KV caches (256 MiB each,
2 GiB together) are rotated so the 256 MB Infinity Cache cannot serve them:
per layer the KV append at position 32767, then attention over rows
0..32767.  Algorithmic bytes per layer-step:
    B(p) = 4 * (2*(p+1)*kv_dim + 2*dim + 4*kv_dim)
(K and V rows 0..p read once, shared by the 4 query heads of each KV head;
q in, out; k, v in; K, V row written).

Also reported: causal prefill of 4096 tokens (1 layer, same shape) in
TFLOP/s with F = 4*hd*H*sum_{p=1..4096} p, and 64 decode steps at 131072+
context (1 GiB KV, one layer).

Inputs are synthetic N(0,1)*0.5 f32 drawn on the GPU and resident in HBM
before timing.  The CPU baseline is the CPU oracle (the reference's
single-threaded attention arithmetic restated in C) timed on a bounded
sample on one host core.
"""
from __future__ import annotations

import argparse
import importlib.util
import json
import os
import platform
import sys
import time
from pathlib import Path

import numpy as np

REPO = Path(__file__).resolve().parent
METRIC = "decode attn HBM GB/s @32k ctx; prefill attn TFLOP/s @4k; % of MI355X roofline"
HBM_PEAK_GBS = 8000.0
FP32_MFMA_PEAK_TFLOPS = 157.3

DIM, HEADS, KV_HEADS = 4096, 32, 8
HD = DIM // HEADS
KV_DIM = HD * KV_HEADS
THETA = 500000.0


def load_product():
    name = "static_lm_amd"
    if name in sys.modules:
        return sys.modules[name]
    spec = importlib.util.spec_from_file_location(name, REPO / "static-lm_amd" / "__init__.py")
    mod = importlib.util.module_from_spec(spec)
    sys.modules[name] = mod
    spec.loader.exec_module(mod)
    return mod


def decode_bytes(pos: int) -> int:
    return 4 * (2 * (pos + 1) * KV_DIM + 2 * DIM + 4 * KV_DIM)


def prefill_flops(start: int, n: int) -> int:
    s = sum(range(start + 1, start + n + 1))
    return 4 * HD * HEADS * s


TRAFFIC_PROFILE = REPO / "profiles" / "decode_kernel_llama3-8b_ctx32k_ctx131k.md"


def _decode_profile_value(key: str) -> str | None:
    try:
        for ln in TRAFFIC_PROFILE.read_text().splitlines():
            if ln.startswith(key + "(decode_kernel @ pos 32767):"):
                return ln.split(":", 1)[1].strip()
    except OSError:
        pass
    return None


def measured_traffic() -> int | None:
    """HBM bytes per launch of the 32k decode kernel from the committed
    rocprofv3 FETCH_SIZE/WRITE_SIZE summary (scaled by the copy calibration),
    or None when the summary is absent."""
    v = _decode_profile_value("traffic_bytes_per_launch")
    return int(v) if v else None


def trace_mean_us() -> float | None:
    """Mean duration of the 32k decode launches in the committed rocprofv3
    kernel-trace summary, or None when it is absent."""
    v = _decode_profile_value("trace_mean_us")
    return float(v) if v else None


PREFILL_PROFILE = REPO / "profiles" / "prefill_mfma_kernel_llama3-8b_4096.md"


def prefill_profile() -> dict:
    """MFMA-busy fraction and LDS counters of the 4096-row prefill kernel from
    the committed rocprofv3 summary (empty when it is absent)."""
    out = {}
    try:
        for ln in PREFILL_PROFILE.read_text().splitlines():
            for key in ("mfma_busy_frac", "lds_bank_conflict_cycles", "lds_instructions",
                        "trace_median_ms"):
                if ln.startswith(key + "(prefill_mfma_kernel 4096):"):
                    v = ln.split(":", 1)[1].strip()
                    out[key] = float(v) if "." in v else int(v)
    except OSError:
        pass
    if out:
        out["counters_source"] = PREFILL_PROFILE.name
    return out


def host_cpu() -> str:
    try:
        for ln in open("/proc/cpuinfo"):
            if ln.startswith("model name"):
                return ln.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or "unknown"


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def fill_cache(torch, ctx, layers: int, msl: int, rows: int, seed: int) -> None:
    g = torch.Generator(device="cuda")
    g.manual_seed(seed)
    blk = 8192
    buf = torch.empty(blk * KV_DIM, device="cuda", dtype=torch.float32)
    for layer in range(layers):
        for which in (0, 1):
            for p0 in range(0, rows, blk):
                n = min(blk, rows - p0)
                torch.randn(blk * KV_DIM, generator=g, device="cuda", out=buf)
                buf.mul_(0.5)
                ctx.kv_write_dev(layer, which, p0, n, buf.data_ptr())
    ctx.sync()


def bench_decode_32k(torch, P, steps: int, warmup: int, ctx_len: int = 32768,
                     steady_warmup: int = 0, graph_reps: int = 0) -> dict:
    """Decode at position ctx_len - 1 through 8 layers of the Llama-3-8B head
    shape (KV caches of ctx_len rows each, rotated per step).  With
    steady_warmup > 0 the same steps are timed once more after that many
    further untimed steps (the clock's steady state).  With graph_reps > 0
    one step is also recorded as a HIP graph and replayed that many times
    back to back (the GPU's time per step without the host's per-call cost;
    every replay rewrites the same appended rows)."""
    layers = 8
    pos = ctx_len - 1
    ctx = P.AttentionContext(DIM, HEADS, KV_HEADS, ctx_len, layers, THETA)
    stream = torch.cuda.current_stream()
    assert stream.cuda_stream != 0, "run on a non-default stream"
    ctx.set_stream(stream.cuda_stream)
    fill_cache(torch, ctx, layers, ctx_len, ctx_len, 1234)
    q = torch.randn(layers, DIM, device="cuda") * 0.5
    k = torch.randn(layers, KV_DIM, device="cuda") * 0.5
    v = torch.randn(layers, KV_DIM, device="cuda") * 0.5
    out = torch.empty(layers, DIM, device="cuda")

    def step():
        for l in range(layers):
            ctx.decode_dev(l, pos, q[l].data_ptr(), k[l].data_ptr(), v[l].data_ptr(),
                           out[l].data_ptr())

    # The last (up to) two of the warm-up steps are queued after the
    # synchronize, right ahead of the timed ones: after a synchronize the GPU
    # idles and its clock takes a while to come back (timed steps that
    # started from an idle GPU read ~3% slower over 20 steps), while steps
    # that follow each other, as in serving, do not.  The number of untimed
    # steps before the timed ones stays `warmup`.
    queued = min(2, warmup)
    for _ in range(warmup - queued):
        step()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    for _ in range(queued):
        step()
    e0.record(stream)
    for _ in range(steps):
        step()
    e1.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms = e0.elapsed_time(e1)

    # second pass with per-launch events, for the dominant kernel's duration
    step()
    ctx.profile(True)
    for _ in range(steps):
        step()
    prof = ctx.profile_read()
    ctx.profile(False)
    n_split, split_ms = prof["decode"]
    n_comb, comb_ms = prof["combine"]
    avg_split_s = split_ms / max(n_split, 1) / 1e3
    kv_bytes = 2 * (pos + 1) * KV_DIM * 4
    achieved = kv_bytes / avg_split_s / 1e9
    step_bytes = layers * decode_bytes(pos)
    steady = None
    if steady_warmup > 0:
        # After a few warm-up steps the GPU clock is still ramping up: with
        # 50 of them these steps measured ~3% faster than with 5.  The
        # caller's warm-up stays the one `value` is measured with.
        for _ in range(steady_warmup):
            step()
        e0.record(stream)
        for _ in range(steps):
            step()
        e1.record(stream)
        torch.cuda.synchronize()
        ms_s = e0.elapsed_time(e1)
        # untimed steps before this window: the warm-up, the timed steps, the
        # profiled pass (one step and `steps` more) and steady_warmup
        steady = {"warmup_steps": warmup + steps + 1 + steps + steady_warmup,
                  "steady_warmup_steps": steady_warmup, "steps": steps,
                  "ms_per_step": round(ms_s / steps, 5),
                  "gbs": round(step_bytes * steps / (ms_s / 1e3) / 1e9, 2)}
    graph_us = None
    if graph_reps > 0:
        graph = None
        try:
            ctx.capture_begin()
            try:
                step()
            finally:  # the stream leaves capture mode whatever happened
                graph = ctx.capture_end()
            for _ in range(3):
                ctx.graph_launch(graph)
            e0.record(stream)
            for _ in range(graph_reps):
                ctx.graph_launch(graph)
            e1.record(stream)
            torch.cuda.synchronize()
            graph_us = e0.elapsed_time(e1) / graph_reps / layers * 1e3
        except P.SlmAttnError as exc:
            log(f"decode @{ctx_len}: graph replay not measured: {exc}")
        finally:
            if graph is not None:
                graph.close()
    ns, tile = ctx.decode_splits(pos + 1)
    finite = bool(torch.isfinite(out).all().item())
    # what the oracle needs to replay layer 0 of the timed configuration: its
    # cache rows before the step, q, k, v, and the GPU's output and appended row
    check = {"pos": pos, "k_rows": ctx.kv_read(0, 0, 0, pos), "v_rows": ctx.kv_read(0, 1, 0, pos),
             "q": q[0].cpu().numpy(), "k": k[0].cpu().numpy(), "v": v[0].cpu().numpy(),
             "out": out[0].cpu().numpy(), "k_row": ctx.kv_read(0, 0, pos, 1)[0],
             "v_row": ctx.kv_read(0, 1, pos, 1)[0]}
    ctx.close()
    return {
        "ms": ms, "wall_s": wall, "steps": steps, "layers": layers, "pos": pos,
        "step_bytes": step_bytes, "gbs": step_bytes * steps / (ms / 1e3) / 1e9,
        "profile": prof, "split_kernel_avg_us": avg_split_s * 1e6,
        "split_kernel_bytes": kv_bytes, "split_kernel_gbs": achieved,
        "splits": ns, "tile": tile, "finite": finite,
        "combine_avg_us": comb_ms / max(n_comb, 1) * 1e3,
        "steady": steady, "graph_us_per_layer_step": graph_us,
        "warmup_queued": queued,
        "_check": check,
    }


def bench_decode_short(torch, P, args) -> dict:
    """Decode steps back to back at 4096 and 600 cached rows (8 layers of the
    Llama-3-8B head shape): the latency-bound lengths of the C4 decode steps
    and of a model decode after a 512-token prompt.  Launched one call at a
    time from Python the host's cost per call is close to the GPU's per
    step, so the same step is also replayed as a HIP graph."""
    short = {}
    for n_ctx in (4096, 600):
        ds = bench_decode_32k(torch, P, max(20, args.steps), args.warmup, ctx_len=n_ctx,
                              graph_reps=100)
        us = ds["ms"] / ds["steps"] / ds["layers"] * 1e3
        gus = ds["graph_us_per_layer_step"]
        short[f"ctx{n_ctx}"] = {
            "us_per_layer_step": round(us, 3), "gbs": round(ds["gbs"], 1),
            "frac_hbm": round(ds["gbs"] / HBM_PEAK_GBS, 4), "splits": ds["splits"],
            "decode_kernel_us_stamped": round(ds["split_kernel_avg_us"], 3),
            "combine_kernel_us_stamped": round(ds["combine_avg_us"], 3),
            "us_per_layer_step_graph": round(gus, 3) if gus else None,
            "gbs_graph": (round(ds["step_bytes"] / ds["layers"] / (gus / 1e6) / 1e9, 1)
                          if gus else None),
        }
        log(f"decode @{n_ctx}: {us:.2f} us per layer-step, {ds['gbs']:.0f} GB/s"
            + (f"; replayed as a graph {gus:.2f} us" if gus else ""))
    return short


def bench_prefill_4k(torch, P, reps: int) -> dict:
    n, msl = 4096, 8192
    ctx = P.AttentionContext(DIM, HEADS, KV_HEADS, msl, 1, THETA)
    stream = torch.cuda.current_stream()
    assert stream.cuda_stream != 0, "run on a non-default stream"
    ctx.set_stream(stream.cuda_stream)
    q = torch.randn(n, DIM, device="cuda") * 0.5
    k = torch.randn(n, KV_DIM, device="cuda") * 0.5
    v = torch.randn(n, KV_DIM, device="cuda") * 0.5
    out = torch.empty(n, DIM, device="cuda")

    def run():
        ctx.prefill_dev(0, 0, n, q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr())

    run()
    torch.cuda.synchronize()
    # Warm-up calls are queued right before the timed ones, with no idle gap
    # in between: after an idle GPU the clock takes a few milliseconds to come
    # back up, which showed as 1.34 ms per call over 5 calls against 1.17 ms
    # in steady state.
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    for _ in range(3):
        run()
    e0.record(stream)
    for _ in range(reps):
        run()
    e1.record(stream)
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / reps
    for _ in range(3):
        run()
    ctx.profile(True)
    for _ in range(reps):
        run()
    prof = ctx.profile_read()
    ctx.profile(False)
    cnt, kms = prof["prefill"]
    flops = prefill_flops(0, n)
    kern_s = kms / max(cnt, 1) / 1e3
    ctx.close()
    return {"ms": ms, "reps": reps, "flops": flops, "tflops": flops / (ms / 1e3) / 1e12,
            "kernel_avg_ms": kern_s * 1e3, "kernel_tflops": flops / kern_s / 1e12,
            "profile": prof}


# Short causal prefills (start 0): name, dim, heads, KV heads, theta, rows.  The
# model prompt's length on the Llama-3-8B shape and the configurations' own
# short prefills on the SmolLM2-135M and Stories-15M shapes.
PREFILL_SHORT = [("llama3-8b", 4096, 32, 8, 5e5, 512), ("llama3-8b", 4096, 32, 8, 5e5, 1024),
                 ("llama3-8b", 4096, 32, 8, 5e5, 2048), ("smollm2-135m", 576, 9, 3, 1e5, 512),
                 ("stories15m", 288, 6, 6, 1e4, 256)]


def bench_prefill_short(torch, P, reps: int = 20) -> list:
    """Each short prefill of PREFILL_SHORT called back to back: per-call time
    (append + prefill kernels) and the prefill kernel's launch-stamped time,
    with its algorithmic TFLOP/s and fraction of the fp32 MFMA peak."""
    stream = torch.cuda.current_stream()
    out = []
    for name, dim, h, kvh, theta, n in PREFILL_SHORT:
        hd = dim // h
        kvd = hd * kvh
        ctx = P.AttentionContext(dim, h, kvh, n, 1, theta)
        ctx.set_stream(stream.cuda_stream)
        q = torch.randn(n, dim, device="cuda") * 0.5
        k = torch.randn(n, kvd, device="cuda") * 0.5
        v = torch.randn(n, kvd, device="cuda") * 0.5
        o = torch.empty(n, dim, device="cuda")

        def run():
            ctx.prefill_dev(0, 0, n, q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr())

        for _ in range(5):
            run()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        for _ in range(reps):
            run()
        e1.record(stream)
        torch.cuda.synchronize()
        call_us = e0.elapsed_time(e1) / reps * 1e3
        ctx.profile(True)
        for _ in range(reps):
            run()
        cnt, kms = ctx.profile_read()["prefill"]
        ctx.profile(False)
        ctx.close()
        kus = kms / max(cnt, 1) * 1e3
        flops = 4 * hd * h * (n * (n + 1) // 2)  # causal pairs, start 0
        out.append({"workload": f"{name} {h}/{kvh} heads hd{hd}, {n} rows", "rows": n,
                    "call_us": round(call_us, 2), "kernel_us_stamped": round(kus, 2),
                    "kernel_tflops": round(flops / (kus / 1e6) / 1e12, 2),
                    "kernel_frac_fp32_mfma": round(flops / (kus / 1e6) / 1e12
                                                   / FP32_MFMA_PEAK_TFLOPS, 4)})
        log(f"prefill {name} {n} rows: {call_us:.1f} us per call, kernel {kus:.1f} us "
            f"({out[-1]['kernel_tflops']:.1f} TFLOP/s)")
    return out


def random_q4_blocks(rng, rows: int, cols: int) -> np.ndarray:
    """Random BlockQ4_0 bytes (random nibbles, f16 scales in [1e-3, 1e-2]):
    projection timing does not depend on the values."""
    nblk = rows * (cols // 32)
    blk = rng.integers(0, 256, (nblk, 18), dtype=np.uint8)
    blk[:, :2] = rng.uniform(1e-3, 1e-2, nblk).astype(np.float16).view(np.uint8).reshape(-1, 2)
    return blk


def _ms_per_call(torch, stream, fn, reps: int) -> float:
    fn()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    for _ in range(2):  # queued right before the timed calls: no idle gap, clocks up
        fn()
    e0.record(stream)
    for _ in range(reps):
        fn()
    e1.record(stream)
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / reps


def _profiled(ctx, fn, reps: int) -> dict:
    ctx.profile(True)
    for _ in range(reps):
        fn()
    prof = ctx.profile_read()
    ctx.profile(False)
    return prof


def bench_block_xb(torch, P, steps: int) -> dict:
    """The attention half of the transformer block from the attention-RMSNorm
    output xb to the residual stream: fused Q/K/V GEMV (Q4_0 x Q8_0) + decode
    at position 32767 + Wo GEMV with the residual add, over 8 layers; the
    projections with residual alone at the Wo and w_down shapes; and the
    4096-row prefill block (Q8_0 quantize + Q/K/V MFMA GEMM + append +
    attention + Wo GEMM with the residual add)."""
    layers, ctx_len = 8, 32768
    pos = ctx_len - 1
    rng = np.random.default_rng(17)
    ctx = P.AttentionContext(DIM, HEADS, KV_HEADS, ctx_len, layers, THETA)
    stream = torch.cuda.current_stream()
    ctx.set_stream(stream.cuda_stream)
    fill_cache(torch, ctx, layers, ctx_len, ctx_len, 4321)
    mats = [(P.Q4Matrix(random_q4_blocks(rng, DIM, DIM), DIM, DIM),
             P.Q4Matrix(random_q4_blocks(rng, KV_DIM, DIM), KV_DIM, DIM),
             P.Q4Matrix(random_q4_blocks(rng, KV_DIM, DIM), KV_DIM, DIM),
             P.Q4Matrix(random_q4_blocks(rng, DIM, DIM), DIM, DIM)) for _ in range(layers)]
    xb = torch.randn(layers, DIM, device="cuda")
    x = torch.randn(layers, DIM, device="cuda")
    out = torch.empty(layers, DIM, device="cuda")

    def qkv_step():
        for l in range(layers):
            wq, wk, wv, _ = mats[l]
            ctx.decode_xb_dev(l, pos, xb[l].data_ptr(), wq, wk, wv, out[l].data_ptr())

    def block_step():
        for l in range(layers):
            wq, wk, wv, wo = mats[l]
            ctx.decode_wo_dev(l, pos, xb[l].data_ptr(), wq, wk, wv, wo, x[l].data_ptr(),
                              out[l].data_ptr())

    qkv_ms = _ms_per_call(torch, stream, qkv_step, steps)
    prof = _profiled(ctx, qkv_step, steps)
    n_g, g_ms = prof["gemm"]
    gemv_us = g_ms / max(n_g, 1) * 1e3
    block_ms = _ms_per_call(torch, stream, block_step, steps)
    bprof = _profiled(ctx, block_step, steps)
    wo_us = (bprof["gemm"][1] - g_ms) / max(bprof["gemm"][0] - n_g, 1) * 1e3
    w_bytes = (DIM + 2 * KV_DIM) * (DIM // 32) * 18
    wo_bytes = DIM * (DIM // 32) * 18
    decode = {
        "workload": "decode attention block from xb @32k, 8 layers: fused Q/K/V GEMV "
                    "(Llama-3-8B Wq/Wk/Wv, Q4_0) + decode attention + Wo GEMV with residual",
        "us_per_layer": block_ms / layers * 1e3,
        "us_per_layer_without_wo": qkv_ms / layers * 1e3,
        "gemv_us": gemv_us,
        "gemv_weight_bytes": w_bytes,
        "gemv_gbs": w_bytes / (gemv_us / 1e6) / 1e9,
        "gemv_frac_hbm": w_bytes / (gemv_us / 1e6) / 1e9 / HBM_PEAK_GBS,
        "wo_gemv_us": wo_us,
        "wo_gemv_gbs": wo_bytes / (wo_us / 1e6) / 1e9,
    }
    for m in mats:
        for w in m:
            w.close()

    # projection + residual alone: Wo (dim x dim) and w_down (dim x 14336),
    # 8 distinct matrices in turn so the weights stream from HBM
    hidden = 14336
    proj = {}
    for name, cols in (("wo", DIM), ("w_down", hidden)):
        ws = [P.Q4Matrix(random_q4_blocks(rng, DIM, cols), DIM, cols) for _ in range(layers)]
        xin = torch.randn(cols, device="cuda")
        res = torch.randn(DIM, device="cuda")

        def run_proj():
            for w in ws:
                ctx.gemm_q4_0_residual_dev(w, xin.data_ptr(), 1, res.data_ptr(), res.data_ptr())

        pp = _profiled(ctx, run_proj, steps)
        us = pp["gemm"][1] / max(pp["gemm"][0], 1) * 1e3
        nbytes = DIM * (cols // 32) * 18
        proj[name] = {"rows": DIM, "cols": cols, "us": us, "weight_bytes": nbytes,
                      "gbs": nbytes / (us / 1e6) / 1e9,
                      "frac_hbm": nbytes / (us / 1e6) / 1e9 / HBM_PEAK_GBS}
        for w in ws:
            w.close()
    decode["residual_gemv"] = proj
    ctx.close()

    n, msl = 4096, 8192
    ctx = P.AttentionContext(DIM, HEADS, KV_HEADS, msl, 1, THETA)
    ctx.set_stream(stream.cuda_stream)
    wq = P.Q4Matrix(random_q4_blocks(rng, DIM, DIM), DIM, DIM)
    wk = P.Q4Matrix(random_q4_blocks(rng, KV_DIM, DIM), KV_DIM, DIM)
    wv = P.Q4Matrix(random_q4_blocks(rng, KV_DIM, DIM), KV_DIM, DIM)
    wo = P.Q4Matrix(random_q4_blocks(rng, DIM, DIM), DIM, DIM)
    xs = torch.randn(n, DIM, device="cuda")
    xres = torch.randn(n, DIM, device="cuda")
    outs = torch.empty(n, DIM, device="cuda")

    def run_qkv():
        ctx.prefill_xb_dev(0, 0, n, xs.data_ptr(), wq, wk, wv, outs.data_ptr())

    def run_block():
        ctx.prefill_wo_dev(0, 0, n, xs.data_ptr(), wq, wk, wv, wo, xres.data_ptr(),
                           outs.data_ptr())

    reps = 3
    qkv_ms = _ms_per_call(torch, stream, run_qkv, reps)
    pprof = _profiled(ctx, run_qkv, reps)
    gemm_ms = pprof["gemm"][1] / max(pprof["gemm"][0], 1)
    quant_ms = pprof["quant"][1] / max(pprof["quant"][0], 1)
    block_ms = _ms_per_call(torch, stream, run_block, reps)
    bprof = _profiled(ctx, run_block, reps)
    wo_ms = (bprof["gemm"][1] - pprof["gemm"][1]) / max(bprof["gemm"][0] - pprof["gemm"][0], 1)
    macs = n * (DIM + 2 * KV_DIM) * DIM
    prefill = {
        "workload": "prefill attention block from xb, 4096 rows: Q8_0 quantize + Q/K/V MFMA "
                    "GEMM (Llama-3-8B, Q4_0) + append + causal attention + Q8_0 quantize + "
                    "Wo MFMA GEMM with residual",
        "ms": block_ms,
        "ms_without_wo": qkv_ms,
        "gemm_ms": gemm_ms,
        "quant_ms": quant_ms,
        "gemm_int8_tops": 2 * macs / (gemm_ms / 1e3) / 1e12,
        "wo_gemm_ms": wo_ms,
        "wo_gemm_int8_tops": 2 * n * DIM * DIM / (wo_ms / 1e3) / 1e12,
    }
    for w in (wq, wk, wv, wo):
        w.close()
    ctx.close()
    return {"decode_xb_32k": decode, "prefill_xb_4k": prefill}


HIDDEN = 14336  # Llama-3-8B feed-forward width


def layer_weight_bytes(hidden: int = HIDDEN) -> int:
    """Q4_0 bytes of one layer's seven projections (18 B per 32 weights)."""
    weights = 2 * DIM * DIM + 2 * KV_DIM * DIM + 3 * hidden * DIM
    return weights // 32 * 18


def make_layers(torch, P, rng, n: int, hidden: int = HIDDEN):
    """n layers of random Q4_0 weights, each uploaded to its own memory (one
    host copy per shape: timing does not depend on the values)."""
    shapes = {"wq": (DIM, DIM), "wk": (KV_DIM, DIM), "wv": (KV_DIM, DIM), "wo": (DIM, DIM),
              "w_gate": (hidden, DIM), "w_up": (hidden, DIM), "w_down": (DIM, hidden)}
    host = {name: random_q4_blocks(rng, r, c) for name, (r, c) in shapes.items()}
    norm = torch.ones(DIM, device="cuda")
    layers = []
    for _ in range(n):
        m = {name: P.Q4Matrix(host[name], r, c) for name, (r, c) in shapes.items()}
        layers.append(P.LayerWeights(norm.data_ptr(), m["wq"], m["wk"], m["wv"], m["wo"],
                                     norm.data_ptr(), m["w_gate"], m["w_up"], m["w_down"]))
    return layers, norm


def bench_layer(torch, P, steps: int) -> dict:
    """The whole transformer block (slm_layer_forward_dev), Llama-3-8B shape
    with Q4_0 weights: one decode token through 8 distinct layers at position
    32767 and at 4095 (weights + KV streamed from HBM), and a 4096-row
    prefill through one layer."""
    layers, ctx_len = 8, 32768
    rng = np.random.default_rng(23)
    stream = torch.cuda.current_stream()
    ctx = P.AttentionContext(DIM, HEADS, KV_HEADS, ctx_len, layers, THETA)
    ctx.set_stream(stream.cuda_stream)
    fill_cache(torch, ctx, layers, ctx_len, ctx_len, 77)
    lws, norm = make_layers(torch, P, rng, layers)
    x = torch.randn(DIM, device="cuda") * 0.5
    wb = layer_weight_bytes()
    out = {"workload": "transformer block, Llama-3-8B shape (dim 4096, 32/8 heads, hidden "
                       "14336), Q4_0 weights, 8 distinct layers", "weight_bytes_per_layer": wb}
    for pos in (ctx_len - 1, 4095):
        def step():
            for l in range(layers):
                ctx.layer_forward_dev(l, pos, 1, lws[l], 1e-5, x.data_ptr())

        ms = _ms_per_call(torch, stream, step, steps)
        prof = _profiled(ctx, step, max(2, steps // 2))
        per = {k: v[1] / max(v[0], 1) * 1e3 for k, v in prof.items() if v[0]}
        nbytes = wb + 2 * (pos + 1) * KV_DIM * 4
        us = ms / layers * 1e3
        out[f"decode_pos{pos}"] = {
            "us_per_layer": us, "bytes_per_layer": nbytes,
            "gbs": nbytes / (us * 1e-6) / 1e9, "frac_hbm": nbytes / (us * 1e-6) / 1e9 / HBM_PEAK_GBS,
            "kernel_us_mean": per,
        }
        log(f"layer decode @{pos}: {us:.1f} us/layer, {nbytes / (us * 1e-6) / 1e9:.0f} GB/s")
    ctx.close()

    n, msl = 4096, 4096
    ctx = P.AttentionContext(DIM, HEADS, KV_HEADS, msl, 1, THETA)
    ctx.set_stream(stream.cuda_stream)
    xs = torch.randn(n, DIM, device="cuda") * 0.5

    def run():
        ctx.layer_forward_dev(0, 0, n, lws[0], 1e-5, xs.data_ptr())

    ms = _ms_per_call(torch, stream, run, 3)
    prof = _profiled(ctx, run, 2)
    per = {k: v[1] / max(v[0], 1) for k, v in prof.items() if v[0]}
    weights = 2 * DIM * DIM + 2 * KV_DIM * DIM + 3 * HIDDEN * DIM
    out["prefill_4096"] = {
        "ms": ms, "tokens_per_s": n / (ms / 1e3),
        "int8_tops_projections": 2 * n * weights / (prof["gemm"][1] / 1e3) / 1e12,
        "kernel_ms_mean": per,
    }
    log(f"layer prefill 4096: {ms:.2f} ms, {n / (ms / 1e3):.0f} tokens/s")
    ctx.close()
    for lw in lws:
        lw.close()
    del norm
    return out


VOCAB = 128256  # Llama-3 vocabulary


def bench_model(torch, P, n_layers: int = 32, prompt_len: int = 512, gen: int = 64) -> dict:
    """The whole model on the device (slm_model_prefill_dev,
    slm_model_generate_dev): Llama-3-8B shape (32 layers, dim 4096, 32/8 heads,
    hidden 14336, vocabulary 128256) with random Q4_0 weights, a 512-token
    prompt, then greedy decode of 64 tokens (each token read back to the host,
    as the reference's generate returns it)."""
    rng = np.random.default_rng(29)
    msl = prompt_len + gen + 1
    stream = torch.cuda.current_stream()
    ctx = P.AttentionContext(DIM, HEADS, KV_HEADS, msl, n_layers, THETA)
    ctx.set_stream(stream.cuda_stream)
    lws, norm = make_layers(torch, P, rng, n_layers)
    emb_host = random_q4_blocks(rng, VOCAB, DIM)
    emb = P.Q4Matrix(emb_host, VOCAB, DIM)
    head = P.Q4Matrix(emb_host, VOCAB, DIM)  # an untied output matrix of its own
    mw = P.ModelWeights(emb, lws, norm.data_ptr(), head)
    prompt = rng.integers(0, VOCAB, prompt_len).astype(np.int32)
    ctx.model_generate_dev(mw, 1e-5, prompt[:32], 2)  # warm-up
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    ctx.model_prefill_dev(mw, 1e-5, prompt, 0)  # warm-up of the same shape, right before
    e0.record(stream)
    for _ in range(2):  # each call returns its token (one stream sync), as the API does
        ctx.model_prefill_dev(mw, 1e-5, prompt, 0)
    e1.record(stream)
    torch.cuda.synchronize()
    prefill_ms = e0.elapsed_time(e1) / 2
    walls = {}
    for n_out in (1, gen):
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        toks = ctx.model_generate_dev(mw, 1e-5, prompt, n_out)
        walls[n_out] = time.perf_counter() - t0
        assert len(toks) == n_out
    per_token = (walls[gen] - walls[1]) / (gen - 1)
    token_bytes = n_layers * layer_weight_bytes() + VOCAB * DIM // 32 * 18
    ctx.close()
    for lw in lws:
        lw.close()
    emb.close()
    head.close()
    del norm
    return {
        "workload": f"model forward on device, Llama-3-8B shape ({n_layers} layers, vocab {VOCAB}), "
                    f"random Q4_0 weights: {prompt_len}-token prompt, greedy decode of {gen} tokens",
        "prefill_ms": prefill_ms, "prefill_tokens_per_s": prompt_len / (prefill_ms / 1e3),
        "decode_ms_per_token": per_token * 1e3, "decode_tokens_per_s": 1.0 / per_token,
        "decode_weight_bytes_per_token": token_bytes,
        "decode_weight_gbs": token_bytes / per_token / 1e9,
    }


def bench_decode_131k(torch, P) -> dict:
    pre, steps = 131072, 64
    msl = pre + steps
    ctx = P.AttentionContext(DIM, HEADS, KV_HEADS, msl, 1, THETA)
    stream = torch.cuda.current_stream()
    assert stream.cuda_stream != 0, "run on a non-default stream"
    ctx.set_stream(stream.cuda_stream)
    fill_cache(torch, ctx, 1, msl, pre, 99)
    q = torch.randn(steps, DIM, device="cuda") * 0.5
    k = torch.randn(steps, KV_DIM, device="cuda") * 0.5
    v = torch.randn(steps, KV_DIM, device="cuda") * 0.5
    out = torch.empty(steps, DIM, device="cuda")

    def run():
        for s in range(steps):
            ctx.decode_dev(0, pre + s, q[s].data_ptr(), k[s].data_ptr(), v[s].data_ptr(),
                           out[s].data_ptr())

    run()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    run()  # queued right before the timed steps (same rows rewritten): no idle gap
    e0.record(stream)
    run()
    e1.record(stream)
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1)
    total = sum(decode_bytes(pre + s) for s in range(steps))
    ctx.close()
    return {"ms_total": ms, "steps": steps, "ms_per_step": ms / steps, "bytes": total,
            "gbs": total / (ms / 1e3) / 1e9}


# The five workload configurations: (name, dim, heads, kv_heads, layers, max_seq_len,
# theta, prefill rows, decode steps, pre-filled rows)
WORKLOADS = [
    ("c1 synthetic dim256 4/4 hd64 2L msl512", 256, 4, 4, 2, 512, 1e4, 16, 8, 0),
    ("c2 stories15m dim288 6/6 hd48 6L msl256", 288, 6, 6, 6, 256, 1e4, 16, 64, 0),
    ("c3 smollm2-135m dim576 9/3 hd64 30L msl2048", 576, 9, 3, 30, 2048, 1e5, 512, 256, 0),
    ("c4 llama3-8b dim4096 32/8 hd128 1L msl8192", 4096, 32, 8, 1, 8192, 5e5, 4096, 128, 0),
    ("c5 llama3-8b long 1L, 131072 pre-filled", 4096, 32, 8, 1, 131136, 5e5, 0, 64, 131072),
]


def workload_inputs(ci: int, dim: int, kvd: int, layers: int, rows: int):
    """Seeded N(0,1)*0.5 f32 q, k, v per layer: [layers][rows][dim | kv_dim]."""
    rng = np.random.default_rng(0x5EED0000 + ci)
    half = np.float32(0.5)
    q = rng.standard_normal((layers, rows, dim), dtype=np.float32) * half
    k = rng.standard_normal((layers, rows, kvd), dtype=np.float32) * half
    v = rng.standard_normal((layers, rows, kvd), dtype=np.float32) * half
    return q, k, v


def prefilled_cache(ci: int, rows: int, kvd: int):
    """Seeded raw K and V cache rows 0..rows-1 (layer 0) for a pre-filled workload."""
    rng = np.random.default_rng(0x5EED1000 + ci)
    half = np.float32(0.5)
    kc = rng.standard_normal((rows, kvd), dtype=np.float32) * half
    vc = rng.standard_normal((rows, kvd), dtype=np.float32) * half
    return kc, vc


def bench_workloads(torch, P) -> tuple[list, list]:
    """Each configuration end to end on device pointers: per layer one prefill
    of P rows then D decode steps.  Reports the host-bound wall time of a pass
    (one Python call per launch), the time of the same pass replayed as a HIP
    graph (one host call), and the kernels' own time (launch-stamped
    decode and merge events, events around the other launches), with the
    algorithmic rates and roofline fractions of the prefill and decode kernels.
    Also returns, per configuration, the inputs, outputs and appended cache
    rows of the last pass, for the oracle comparison of the CPU baseline leg."""
    out, checks = [], []
    stream = torch.cuda.current_stream()
    for ci, (name, dim, h, kvh, layers, msl, theta, npf, nd, pre) in enumerate(WORKLOADS, 1):
        hd = dim // h
        kvd = hd * kvh
        rows = npf + nd
        ctx = P.AttentionContext(dim, h, kvh, msl, layers, theta)
        ctx.set_stream(stream.cuda_stream)
        qh, kh, vh = workload_inputs(ci, dim, kvd, layers, rows)
        pre_k = pre_v = None
        if pre:
            pre_k, pre_v = prefilled_cache(ci, pre, kvd)
            ctx.kv_write(0, 0, 0, pre_k)
            ctx.kv_write(0, 1, 0, pre_v)
        q, k, v = (torch.from_numpy(a).cuda() for a in (qh, kh, vh))
        o = torch.empty(layers, rows, dim, device="cuda")

        def run_prefill(l):
            ctx.prefill_dev(l, pre, npf, q[l].data_ptr(), k[l].data_ptr(), v[l].data_ptr(),
                            o[l].data_ptr())

        def run_decode(l):
            for st in range(nd):
                r = npf + st
                ctx.decode_dev(l, pre + r, q[l, r].data_ptr(), k[l, r].data_ptr(),
                               v[l, r].data_ptr(), o[l, r].data_ptr())

        def run():
            for l in range(layers):
                if npf:
                    run_prefill(l)
                run_decode(l)

        def prefills():
            for l in range(layers):
                run_prefill(l)

        def decodes():
            for l in range(layers):
                run_decode(l)

        def graph_time(fn):
            """fn's launches recorded once as a HIP graph, replayed with one
            host call: their device time without the per-call host cost
            (None, with the reason logged, if recording fails)."""
            graph = None
            try:
                ctx.capture_begin()
                try:
                    fn()
                finally:  # the stream leaves capture mode whatever happened
                    graph = ctx.capture_end()
                ctx.graph_launch(graph)
                torch.cuda.synchronize()
                e0.record(stream)
                ctx.graph_launch(graph)
                e1.record(stream)
                torch.cuda.synchronize()
                return e0.elapsed_time(e1)
            except P.SlmAttnError as exc:
                log(f"{name}: graph replay not measured: {exc}")
                return None
            finally:
                if graph is not None:
                    graph.close()

        run()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        run()
        e1.record(stream)
        torch.cuda.synchronize()
        wall_ms = e0.elapsed_time(e1)
        # the whole pass, then its prefill launches and its decode launches
        # apart (the layers' caches are independent, so the two orders give
        # the same work), each as a replayed graph
        graph_ms = graph_time(run)
        graph_pf_ms = graph_time(prefills) if npf else None
        graph_dec_ms = graph_time(decodes)
        ctx.profile(True)
        run()
        prof = ctx.profile_read()
        ctx.profile(False)
        flops = layers * 4 * hd * h * sum(range(pre + 1, pre + npf + 1))
        dec_bytes = layers * sum(4 * (2 * (p + 1) * kvd + 2 * dim + 4 * kvd)
                                 for p in range(pre + npf, pre + npf + nd))
        kern = {kind: round(ms, 4) for kind, (cnt, ms) in prof.items() if cnt}
        # Rates from device time: the graph replays of the prefill launches
        # and of the decode launches.  Sums of launch-stamped events overstate
        # short kernels (an empty kernel stamps 3.9-4.0 us, and costs 2.4 us
        # back to back), so they are the fallback only.
        pf_ms = graph_pf_ms or (prof["prefill"][1] + prof["append"][1])
        dec_ms = graph_dec_ms or (prof["decode"][1] + prof["combine"][1])
        rec = {"workload": name, "wall_ms": round(wall_ms, 4),
               "graph_ms": round(graph_ms, 4) if graph_ms else None,
               "graph_prefill_ms": round(graph_pf_ms, 4) if graph_pf_ms else None,
               "graph_decode_ms": round(graph_dec_ms, 4) if graph_dec_ms else None,
               "rates_from": ("graph replays of the prefill and of the decode launches"
                              if (graph_dec_ms and (graph_pf_ms or not npf))
                              else "sums of launch-stamped kernel events"),
               "kernel_ms": round(sum(ms for _, ms in prof.values()), 4),
               "kernel_ms_by_kind": kern,
               "launches": int(sum(cnt for cnt, _ in prof.values())),
               "prefill_flops": flops, "decode_bytes": dec_bytes}
        if npf:
            rec["prefill_tflops"] = round(flops / (pf_ms / 1e3) / 1e12, 3)
            rec["prefill_frac_fp32_mfma"] = round(flops / (pf_ms / 1e3) / 1e12
                                                  / FP32_MFMA_PEAK_TFLOPS, 4)
        rec["decode_gbs"] = round(dec_bytes / (dec_ms / 1e3) / 1e9, 1)
        rec["decode_frac_hbm"] = round(dec_bytes / (dec_ms / 1e3) / 1e9 / HBM_PEAK_GBS, 4)
        rec["kernel_frac_of_wall"] = round(rec["kernel_ms"] / wall_ms, 3)
        rec["kernel_frac_of_graph"] = (round(rec["kernel_ms"] / graph_ms, 3) if graph_ms
                                       else None)
        out.append(rec)
        log(f"{name}: wall {wall_ms:.3f} ms per pass, graph replay "
            f"{f'{graph_ms:.3f} ms' if graph_ms else 'n/a'}, "
            f"kernels {rec['kernel_ms']:.3f} ms over {rec['launches']} launches")
        got = o.cpu().numpy()
        kv_rows = [(ctx.kv_read(l, 0, pre, rows), ctx.kv_read(l, 1, pre, rows))
                   for l in range(layers)]
        checks.append({"cfg": (dim, h, kvh, msl, layers, theta), "npf": npf, "nd": nd, "pre": pre,
                       "q": qh, "k": kh, "v": vh, "out": got, "kv": kv_rows,
                       "pre_k": pre_k, "pre_v": pre_v})
        ctx.close()
        del q, k, v, o
    return out, checks


def _errs(got, ref) -> dict:
    """max-abs; max-rel floored at |ref| = 0.1 (the parity bar's 1e-4 / 1e-3);
    unfloored max-rel over |ref| >= 1e-2."""
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    d = np.abs(got - ref)
    big = np.abs(ref) >= 1e-2
    return {"max_abs": float(d.max(initial=0.0)),
            "max_rel": float((d / np.maximum(np.abs(ref), 0.1)).max(initial=0.0)),
            "max_rel_unfloored": float((d[big] / np.abs(ref[big])).max(initial=0.0)),
            "n": int(d.size)}


def _merge_errs(a: dict | None, b: dict) -> dict:
    if a is None:
        return dict(b)
    return {k: (a[k] + b[k] if k == "n" else max(a[k], b[k])) for k in b}


def _bitwise(a, b) -> bool:
    a = np.ascontiguousarray(a, np.float32)
    b = np.ascontiguousarray(b, np.float32)
    return a.shape == b.shape and bool(np.array_equal(a.view(np.uint32), b.view(np.uint32)))


def cpu_configs(checks: list) -> list:
    """CPU baseline leg for the configurations: the oracle (the reference's
    single-threaded attention arithmetic restated in C, one host core) on the
    same inputs as the GPU run, timed, and used as the checker of the GPU
    outputs and appended cache rows.  C1-C4 run in full (C4: the 4096-row
    prefill and all 128 decode steps, ~20 s); C5 times its first four decode
    steps and its last (the others are appended to the oracle's cache
    untimed), and its full-run CPU time is extrapolated by bytes."""
    sys.path.insert(0, str(REPO))
    from oracle import py_oracle as orc

    res = []
    for ch in checks:
        dim, h, kvh, msl, layers, theta = ch["cfg"]
        cfg = orc.Cfg(dim, h, kvh, msl, layers, theta)
        hd, kvd = dim // h, dim // h * kvh
        npf, nd, pre = ch["npf"], ch["nd"], ch["pre"]
        q, k, v, got = ch["q"], ch["k"], ch["v"], ch["out"]
        om = orc.OracleModel(cfg)
        if pre:
            om.k_cache(0)[:pre] = ch["pre_k"]
            om.v_cache(0)[:pre] = ch["pre_v"]
        full = pre == 0  # C1-C4
        err, t_oracle = None, 0.0
        est_ms, sample = None, "full run"
        if full:
            for l in range(layers):
                if npf:
                    t0 = time.perf_counter()
                    r = om.prefill(l, pre, q[l, :npf], k[l, :npf], v[l, :npf])
                    t_oracle += time.perf_counter() - t0
                    err = _merge_errs(err, _errs(got[l, :npf], r))
                for st in range(nd):
                    p = pre + npf + st
                    t0 = time.perf_counter()
                    r = om.decode(l, p, q[l, npf + st], k[l, npf + st], v[l, npf + st])
                    t_oracle += time.perf_counter() - t0
                    err = _merge_errs(err, _errs(got[l, npf + st], r))
            est_ms = t_oracle * 1e3
        else:
            f_all = f_smp = b_all = b_smp = 0.0
            t_pf = t_dec = 0.0
            if npf:
                om.append(0, pre, k[0, :npf], v[0, :npf])
                rows = sorted(set(np.linspace(0, npf - 1, 24).astype(int).tolist()))
                for b in rows:
                    t0 = time.perf_counter()
                    r = om.attend(0, q[0, b], pre + b)
                    t_pf += time.perf_counter() - t0
                    f_smp += 4 * hd * h * (pre + b + 1)
                    err = _merge_errs(err, _errs(got[0, b], r))
                f_all = 4 * hd * h * sum(range(pre + 1, pre + npf + 1))
            steps = sorted({0, 1, nd // 2, nd - 1} if npf else {0, 1, 2, 3, nd - 1})
            for st in range(nd):
                p = pre + npf + st
                bp = 4 * (2 * (p + 1) * kvd + 2 * dim + 4 * kvd)
                b_all += bp
                if st in steps:
                    t0 = time.perf_counter()
                    r = om.decode(0, p, q[0, npf + st], k[0, npf + st], v[0, npf + st])
                    t_dec += time.perf_counter() - t0
                    b_smp += bp
                    err = _merge_errs(err, _errs(got[0, npf + st], r))
                else:
                    om.append(0, p, k[0, npf + st], v[0, npf + st])
            t_oracle = t_pf + t_dec
            est_ms = ((t_pf * f_all / f_smp if f_smp else 0.0) + t_dec * b_all / b_smp) * 1e3
            sample = ((f"prefill rows {rows[0]}..{rows[-1]} ({len(rows)} of {npf}) and " if npf
                       else "") + f"decode steps {steps} of {nd}, extrapolated by flops / bytes")
        kv_ok = all(_bitwise(ch["kv"][l][0], om.k_cache(l)[pre:pre + npf + nd]) and
                    _bitwise(ch["kv"][l][1], om.v_cache(l)[pre:pre + npf + nd])
                    for l in range(layers))
        res.append({"cpu_ms": round(est_ms, 3), "cpu_sample_s": round(t_oracle, 3),
                    "cpu_sample": sample, "cores": 1,
                    "parity": {**{k2: (round(v2, 10) if isinstance(v2, float) else v2)
                                  for k2, v2 in err.items()},
                               "kv_bitwise": kv_ok,
                               "pass": bool(kv_ok and err["max_abs"] <= 1e-4
                                            and err["max_rel"] <= 1e-3)}})
        del om
    return res


def cpu_baseline(budget_s: float, hc: dict) -> dict:
    """The oracle's decode (rope + append + JIT-softmax attention) of the
    headline workload -- one layer at position 32767 over the same cache rows,
    q, k and v as the GPU run's layer 0 -- on one host core, repeated until
    the time budget is spent; its output checks the GPU's (parity of the timed
    configuration).  Plus a sample of prefill rows of a 4096-token prefill."""
    sys.path.insert(0, str(REPO))
    from oracle import py_oracle as orc

    pos = hc["pos"]
    cfg = orc.Cfg(DIM, HEADS, KV_HEADS, pos + 1, 1, THETA)
    om = orc.OracleModel(cfg)
    om.k_cache(0)[:pos] = hc["k_rows"]
    om.v_cache(0)[:pos] = hc["v_rows"]
    calls = 0
    t0 = time.perf_counter()
    while True:
        r = om.decode(0, pos, hc["q"], hc["k"], hc["v"])
        calls += 1
        el = time.perf_counter() - t0
        if el >= budget_s * 0.75:
            break
    dec_gbs = decode_bytes(pos) * calls / el / 1e9
    parity = _errs(hc["out"], r)
    parity["kv_bitwise"] = (_bitwise(hc["k_row"], om.k_cache(0)[pos])
                            and _bitwise(hc["v_row"], om.v_cache(0)[pos]))
    parity["pass"] = bool(parity["kv_bitwise"] and parity["max_abs"] <= 1e-4
                          and parity["max_rel"] <= 1e-3)
    del om
    # prefill sample: the last rows of a 4096-token prefill, each attending
    # to 4090+ cached rows (the per-row loop of the reference)
    rng = np.random.default_rng(5)
    pcfg = orc.Cfg(DIM, HEADS, KV_HEADS, 4096, 1, THETA)
    pm = orc.OracleModel(pcfg)
    pm.k_cache(0)[:] = rng.standard_normal((4096, KV_DIM), dtype=np.float32) * 0.5
    pm.v_cache(0)[:] = rng.standard_normal((4096, KV_DIM), dtype=np.float32) * 0.5
    q = rng.standard_normal(DIM, dtype=np.float32) * 0.5
    rows = 0
    flops = 0
    t1 = time.perf_counter()
    while True:
        p = 4095 - rows
        pm.attend(0, q, p)
        flops += 4 * HD * HEADS * (p + 1)
        rows += 1
        el2 = time.perf_counter() - t1
        if el2 >= budget_s * 0.25:
            break
    return {
        "value": dec_gbs, "unit": "GB/s", "cores": 1, "kind": "port",
        "sample": f"{calls} oracle decode calls (rope+append+attention) at pos {pos} on layer 0 "
                  f"of the headline cache, {el:.1f} s on {host_cpu()} (nproc {os.cpu_count()})",
        "parity": parity,
        "prefill_tflops": flops / el2 / 1e12,
        "prefill_sample": f"last {rows} rows of a 4096-token prefill, {el2:.1f} s",
    }


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--cpu-seconds", type=float, default=10.0,
                    help="time budget of the CPU baseline sample (0 skips it)")
    ap.add_argument("--skip-extra", action="store_true",
                    help="only the headline decode @32k measurement")
    ap.add_argument("--prefill-only", action="store_true",
                    help="only the 4096-row prefill (a short program for counter passes); "
                         "prints its own JSON line, not the headline one")
    ap.add_argument("--xb-only", action="store_true",
                    help="only the attention block from xb (Q/K/V projections, attention, Wo + residual); "
                         "prints its own JSON line, not the headline one")
    ap.add_argument("--layer-only", action="store_true",
                    help="only the whole transformer block (decode and prefill); prints its "
                         "own JSON line, not the headline one")
    ap.add_argument("--model-only", action="store_true",
                    help="only the whole model (prefill and greedy decode, Llama-3-8B shape); "
                         "prints its own JSON line, not the headline one")
    ap.add_argument("--prefill-short-only", action="store_true",
                    help="only the short prefills (512-2048 rows, Llama-3-8B, SmolLM2-135M "
                         "and Stories-15M shapes)")
    ap.add_argument("--decode-only", action="store_true",
                    help="only the decode measurements (8 layers at 32767, 131072..131135, 8 layers "
                         "at 4095 and at 599; a short program for kernel traces); prints its own "
                         "JSON line, not the headline one")
    ap.add_argument("--configs-only", action="store_true",
                    help="only the five workload configurations, GPU side (a short program for "
                         "kernel traces); prints its own JSON line, not the headline one")
    ap.add_argument("--copy-calibration-mib", type=int, default=0,
                    help="first run one device-to-device copy of this many MiB: a plain "
                         "copy kernel of known size that scales rocprofv3 byte counters")
    args = ap.parse_args()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print("bench.py runs on exactly one GPU: this build has no multi-GPU path "
              "(sharding is design only); run it with --gpus 1", file=sys.stderr)
        return 2

    import torch

    P = load_product()
    P.load_library()
    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        return 1
    torch.manual_seed(0)
    log(f"device {torch.cuda.get_device_name(0)}")
    # A dedicated stream: the legacy default stream's handle is 0, which the
    # C ABI reads as "the context's own stream".  Every kernel of the library
    # and every timing event goes on this one stream.
    torch.cuda.set_stream(torch.cuda.Stream())

    if args.copy_calibration_mib > 0:
        n = args.copy_calibration_mib << 18  # floats
        src = torch.ones(n, device="cuda")
        dst = torch.empty(n, device="cuda")
        torch.cuda.synchronize()
        dst.copy_(src)
        torch.cuda.synchronize()
        log(f"copy calibration: {args.copy_calibration_mib} MiB read + "
            f"{args.copy_calibration_mib} MiB written")
        del src, dst

    if args.configs_only:
        wl, _ = bench_workloads(torch, P)
        print(json.dumps({"configs": wl}))
        return 0

    if args.layer_only:
        bl = bench_layer(torch, P, max(3, args.steps // 5))
        print(json.dumps(bl))
        return 0

    if args.model_only:
        bm = bench_model(torch, P)
        log(f"model: prefill {bm['prefill_tokens_per_s']:.0f} tokens/s, decode "
            f"{bm['decode_tokens_per_s']:.1f} tokens/s ({bm['decode_ms_per_token']:.2f} ms/token)")
        print(json.dumps(bm))
        return 0

    if args.xb_only:
        bx = bench_block_xb(torch, P, max(3, args.steps // 5))
        print(json.dumps(bx))
        return 0

    if args.prefill_only:
        pf = bench_prefill_4k(torch, P, reps=max(10, args.steps // 5))
        log(f"prefill 4096: {pf['ms']:.3f} ms, {pf['tflops']:.2f} TFLOP/s")
        print(json.dumps({"prefill_4k_tflops": pf["tflops"], "ms": pf["ms"],
                          "kernel_avg_ms": pf["kernel_avg_ms"]}))
        return 0

    if args.prefill_short_only:
        print(json.dumps({"prefill_short": bench_prefill_short(torch, P)}))
        return 0

    if args.decode_only:
        d = bench_decode_32k(torch, P, args.steps, args.warmup)
        dl = bench_decode_131k(torch, P)
        short = bench_decode_short(torch, P, args)
        print(json.dumps({"decode_32k_us_per_layer_step": d["ms"] / d["steps"] / d["layers"] * 1e3,
                          "decode_32k_gbs": d["gbs"],
                          "decode_32k_kernel_us_stamped": d["split_kernel_avg_us"],
                          "decode_32k_combine_us_stamped": d["combine_avg_us"],
                          "decode_131k_us_per_step": dl["ms_per_step"] * 1e3,
                          "decode_short": short}))
        return 0

    log("decode @32k")
    d = bench_decode_32k(torch, P, args.steps, args.warmup, steady_warmup=50)
    log(f"decode @32k: {d['gbs']:.1f} GB/s, split kernel {d['split_kernel_avg_us']:.1f} us "
        f"({d['split_kernel_gbs']:.1f} GB/s)")
    extra = {}
    if not args.skip_extra:
        log("prefill 4096")
        pf = bench_prefill_4k(torch, P, reps=max(10, args.steps // 5))
        log(f"prefill 4096: {pf['ms']:.3f} ms, {pf['tflops']:.2f} TFLOP/s")
        log("short prefills")
        pshort = bench_prefill_short(torch, P)
        log("decode @131k")
        dl = bench_decode_131k(torch, P)
        log("decode at short contexts")
        short = bench_decode_short(torch, P, args)
        log("all configurations")
        wl, wl_checks = bench_workloads(torch, P)
        log(f"decode @131k: {dl['ms_per_step']*1e3:.1f} us/step, {dl['gbs']:.1f} GB/s")
        log("attention block from xb")
        bx = bench_block_xb(torch, P, max(3, args.steps // 5))
        log(f"decode block from xb @32k: {bx['decode_xb_32k']['us_per_layer']:.1f} us/layer, "
            f"QKV GEMV {bx['decode_xb_32k']['gemv_us']:.2f} us "
            f"({bx['decode_xb_32k']['gemv_gbs']:.0f} GB/s); prefill block 4k "
            f"{bx['prefill_xb_4k']['ms']:.3f} ms (GEMM {bx['prefill_xb_4k']['gemm_ms']:.3f} ms)")
        log("transformer block")
        blk = bench_layer(torch, P, max(3, args.steps // 5))
        log("model")
        bm = bench_model(torch, P)
        log(f"model: prefill {bm['prefill_tokens_per_s']:.0f} tokens/s, decode "
            f"{bm['decode_tokens_per_s']:.1f} tokens/s ({bm['decode_ms_per_token']:.2f} ms/token)")
        log("measurement probes")
        cal_mfma = P.calibrate_mfma_f32(iters=20000)
        cal_nt = P.calibrate_hbm_read(4 << 30, nontemporal=True)
        cal_plain = P.calibrate_hbm_read(4 << 30, nontemporal=False)
        log(f"probes: fp32 MFMA {cal_mfma['tflops']:.1f} TFLOP/s, streaming read "
            f"{cal_nt:.0f} GB/s nontemporal, {cal_plain:.0f} GB/s plain")
        pf_prof = prefill_profile()
        extra = {
            "roofline_prefill": {
                "bound": "mfma",
                "kernel": "prefill_mfma_kernel<128,4,2,1,32,2,false,true,1,true> (causal "
                          "attention, fp32 v_mfma_f32_16x16x4f32, DMA-fed LDS tiles, paired "
                          "query blocks, 4096 rows)",
                "achieved": round(pf["kernel_tflops"], 2),
                "peak": FP32_MFMA_PEAK_TFLOPS,
                "unit": "TFLOP/s",
                "frac": round(pf["kernel_tflops"] / FP32_MFMA_PEAK_TFLOPS, 4),
                "avg_launch_ms": round(pf["kernel_avg_ms"], 4),
                "algorithmic_flops_per_launch": pf["flops"],
                **pf_prof,
            },
            "probes": {
                "mfma_f32_16x16x4_tflops": round(cal_mfma["tflops"], 2),
                "stream_read_nontemporal_gbs": round(cal_nt, 1),
                "stream_read_plain_gbs": round(cal_plain, 1),
                "note": "plain streaming-read and MFMA-chain probes on this device "
                        "(libslm_calib.so); not ceilings of the product kernels (the 131k "
                        "decode streams faster than the read probe); roofline peaks are the "
                        "published figures",
            },
            "prefill_4k": {
                "tflops": pf["tflops"], "ms": pf["ms"], "flops": pf["flops"],
                "frac_fp32_mfma": pf["tflops"] / FP32_MFMA_PEAK_TFLOPS,
                "kernel_avg_ms": pf["kernel_avg_ms"], "kernel_tflops": pf["kernel_tflops"],
                "workload": "causal prefill 4096 tokens, 1 layer, start 0",
            },
            "prefill_short": pshort,
            "decode_short": {
                "workload": "decode at position ctx-1 through 8 layers of the Llama-3-8B head "
                            "shape, steps back to back (decode + split merge per layer)",
                **short,
            },
            "decode_131k": {
                "gbs": dl["gbs"], "us_per_step": dl["ms_per_step"] * 1e3,
                "frac_hbm": dl["gbs"] / HBM_PEAK_GBS,
                "workload": "64 decode steps at positions 131072..131135, 1 layer, 1 GiB KV",
            },
            "configs": wl,
            **bx,
            "transformer_block": blk,
            "model": bm,
        }
    cpu = None
    if args.cpu_seconds > 0:
        log("cpu baseline")
        cpu = cpu_baseline(args.cpu_seconds, d["_check"])
        log(f"cpu baseline: {cpu['value']:.2f} GB/s; headline parity max-abs "
            f"{cpu['parity']['max_abs']:.2e}, KV bitwise {cpu['parity']['kv_bitwise']}")
        if not args.skip_extra:
            log("cpu baseline of the configurations (oracle on the same inputs)")
            for rec, c in zip(extra["configs"], cpu_configs(wl_checks)):
                rec.update(c)
                log(f"{rec['workload']}: cpu {c['cpu_ms']:.1f} ms ({c['cpu_sample']}), "
                    f"max-abs {c['parity']['max_abs']:.2e}, KV bitwise {c['parity']['kv_bitwise']}")

    ms_per_step = d["ms"] / d["steps"]
    tmu = trace_mean_us()
    res = {
        "metric": METRIC,
        "value": round(d["gbs"], 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        # of those untimed steps, how many were queued after the last
        # synchronize, right ahead of the timed ones (the rest ran before it)
        "warmup_queued": d["warmup_queued"],
        "ms_per_step": round(ms_per_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic",
        "config": {
            "workload": "decode attention @32k ctx, Llama-3-8B head shape (32 heads / 8 KV heads, "
                        "head_dim 128), 8 layers of f32 KV rotated per step",
            "dim": DIM, "num_heads": HEADS, "num_kv_heads": KV_HEADS, "head_dim": HD,
            "ctx": d["pos"] + 1, "layers": d["layers"], "rope_theta": THETA,
            "bytes_per_step": d["step_bytes"], "splits": d["splits"], "split_tile": d["tile"],
        },
        "roofline": {
            "bound": "hbm",
            "kernel": "decode_kernel<128,4,16,1,8> (append + interleaved split-K decode)",
            "achieved": round(d["split_kernel_gbs"], 2),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(d["split_kernel_gbs"] / HBM_PEAK_GBS, 4),
            "traffic": measured_traffic(),
            "traffic_source": "rocprofv3 FETCH_SIZE x2.0 + WRITE_SIZE x1.0 (copy-calibrated), "
                              + TRAFFIC_PROFILE.name,
            "avg_launch_us": round(d["split_kernel_avg_us"], 3),
            "combine_kernel_avg_us": round(d["combine_avg_us"], 3),
            "algorithmic_bytes_per_launch": d["split_kernel_bytes"],
            # the same kernel's mean over the committed kernel trace, and the
            # fraction it gives (the launch-stamped events above read ~1.5% lower)
            "trace_mean_us": tmu,
            "trace_frac": (round(d["split_kernel_bytes"] / (tmu * 1e-6) / 1e9 / HBM_PEAK_GBS, 4)
                           if tmu else None),
        },
        "cpu_baseline": cpu,
        "parity": cpu["parity"] if cpu else None,
        "frac_hbm_step": round(d["gbs"] / HBM_PEAK_GBS, 4),
        # the same steps timed again after 50 more untimed ones, once the GPU
        # clock has settled; `value` is the measurement with the warm-up asked for
        "steady_state": ({**d["steady"],
                          "frac_hbm": round(d["steady"]["gbs"] / HBM_PEAK_GBS, 4)}
                         if d.get("steady") else None),
        **extra,
    }
    print(json.dumps(res))
    return 0


if __name__ == "__main__":
    sys.exit(main())
