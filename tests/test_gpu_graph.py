"""HIP graphs of the device-pointer entry points (slm_attn_capture_begin /
slm_attn_capture_end / slm_attn_graph_launch).

A replay runs the recorded kernels with the recorded arguments, so its
outputs and appended K/V rows must equal the eager calls' bit for bit, and
the oracle's within the parity bar.  Each replay follows eager work on the
same stream (outputs cleared, the cache rows the sequence appends overwritten
with noise, an unrelated decode) and a synchronization, and every replay is
checked.  While capturing, calls that cannot be recorded are refused with
SLM_ERR_CAPTURE and record nothing.
"""
import sys

import numpy as np
import pytest

from oracle import py_oracle as orc
from slm_testlib import (WORKLOADS, assert_bitwise, assert_close, gen, layer_inputs,
                         load_product)

P = load_product()
pytestmark = pytest.mark.gpu
torch = pytest.importorskip("torch")


def log(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def make_ctx(w):
    return P.AttentionContext(w.dim, w.num_heads, w.num_kv_heads, w.max_seq_len, w.num_layers,
                              w.theta)


@pytest.mark.parametrize("key", ["c1", "c2"])
def test_graph_replays_match_eager_and_oracle(key):
    w = WORKLOADS[key]
    n, nd = w.prefill, w.decode
    rows = n + nd
    log(f"graph replay: workload {key} {w}, {w.num_layers} x (prefill {n} + {nd} decode steps)")
    stream = torch.cuda.Stream()
    inputs = [layer_inputs(w, l) for l in range(w.num_layers)]
    with make_ctx(w) as ctx, torch.cuda.stream(stream):
        ctx.set_stream(stream.cuda_stream)
        q, k, v = (torch.from_numpy(np.stack([x[i] for x in inputs])).cuda() for i in range(3))
        out = torch.zeros(w.num_layers, rows, w.dim, device="cuda")

        def run():
            for l in range(w.num_layers):
                ctx.prefill_dev(l, 0, n, q[l].data_ptr(), k[l].data_ptr(), v[l].data_ptr(),
                                out[l].data_ptr())
                for st in range(nd):
                    p = n + st
                    ctx.decode_dev(l, p, q[l, p].data_ptr(), k[l, p].data_ptr(),
                                   v[l, p].data_ptr(), out[l, p].data_ptr())

        run()
        ctx.sync()
        eager = out.cpu().numpy()
        eager_kv = [(ctx.kv_read(l, 0, 0, rows), ctx.kv_read(l, 1, 0, rows))
                    for l in range(w.num_layers)]

        om = orc.OracleModel(w.cfg())
        for l in range(w.num_layers):
            ql, kl, vl = inputs[l]
            ref = np.empty((rows, w.dim), np.float32)
            ref[:n] = om.prefill(l, 0, ql[:n], kl[:n], vl[:n])
            for st in range(nd):
                p = n + st
                ref[p] = om.decode(l, p, ql[p], kl[p], vl[p])
            assert_close(eager[l], ref, what=f"{key} eager layer {l}")
            assert_bitwise(eager_kv[l][0], om.k_cache(l)[:rows], f"{key} eager K layer {l}")
            assert_bitwise(eager_kv[l][1], om.v_cache(l)[:rows], f"{key} eager V layer {l}")

        out.zero_()
        ctx.capture_begin()
        run()
        graph = ctx.capture_end()
        ctx.sync()
        assert not out.any().item(), "a captured call ran instead of being recorded"
        noise_rng = np.random.default_rng(7)
        with graph:
            for rep in range(3):
                # eager work between replays, on the same stream
                out.fill_(float("nan"))
                for l in range(w.num_layers):
                    ctx.kv_write(l, 0, 0, noise_rng.standard_normal((rows, w.kv_dim),
                                                                   dtype=np.float32))
                    ctx.kv_write(l, 1, 0, noise_rng.standard_normal((rows, w.kv_dim),
                                                                   dtype=np.float32))
                extra = torch.from_numpy(gen([w.seed, 99, rep], (3, w.dim))).cuda()
                scratch_out = torch.empty(w.dim, device="cuda")
                ctx.decode_dev(0, rows + rep, extra[0].data_ptr(),
                               extra[1, :w.kv_dim].data_ptr(),
                               extra[2, :w.kv_dim].data_ptr(), scratch_out.data_ptr())
                ctx.sync()
                ctx.graph_launch(graph)
                ctx.sync()
                got = out.cpu().numpy()
                log(f"{key} replay {rep}: max |replay - eager| "
                    f"{float(np.nanmax(np.abs(got - eager))):.3g}")
                assert_bitwise(got, eager, f"{key} replay {rep} outputs")
                for l in range(w.num_layers):
                    assert_bitwise(ctx.kv_read(l, 0, 0, rows), eager_kv[l][0],
                                   f"{key} replay {rep} K layer {l}")
                    assert_bitwise(ctx.kv_read(l, 1, 0, rows), eager_kv[l][1],
                                   f"{key} replay {rep} V layer {l}")


def test_capture_refuses_unrecordable_calls():
    w = WORKLOADS["c1"]
    log(f"capture refusals: {w}")
    q, k, v = layer_inputs(w, 0)
    with make_ctx(w) as ctx:
        qd, kd, vd = (torch.from_numpy(a).cuda() for a in (q, k, v))
        out = torch.zeros(w.dim, device="cuda")
        torch.cuda.synchronize()

        def code(fn):
            with pytest.raises(P.SlmAttnError) as ei:
                fn()
            return ei.value.code

        assert code(ctx.capture_end) == P.ERR_CAPTURE  # none in progress
        ctx.profile(True)
        assert code(ctx.capture_begin) == P.ERR_CAPTURE  # timing on
        ctx.profile(False)

        ctx.capture_begin()
        assert code(ctx.capture_begin) == P.ERR_CAPTURE
        assert code(ctx.sync) == P.ERR_CAPTURE
        assert code(lambda: ctx.set_stream(None)) == P.ERR_CAPTURE
        assert code(lambda: ctx.profile(True)) == P.ERR_CAPTURE
        assert code(lambda: ctx.decode(0, 0, q[0], k[0], v[0])) == P.ERR_CAPTURE
        assert code(lambda: ctx.kv_read(0, 0, 0, 1)) == P.ERR_CAPTURE
        assert code(lambda: ctx.kv_write(0, 0, 0, k[:1])) == P.ERR_CAPTURE
        # a recordable call between the refusals, then the recording replays it
        ctx.decode_dev(0, 0, qd[0].data_ptr(), kd[0].data_ptr(), vd[0].data_ptr(),
                       out.data_ptr())
        with ctx.capture_end() as graph:
            torch.cuda.synchronize()
            assert not out.any().item()
            ctx.graph_launch(graph)
            ctx.sync()
        om = orc.OracleModel(w.cfg())
        assert_close(out.cpu().numpy(), om.decode(0, 0, q[0], k[0], v[0]),
                     what="decode replayed after refusals")
        # the context still runs eagerly
        assert_close(ctx.decode(0, 1, q[1], k[1], v[1]), om.decode(0, 1, q[1], k[1], v[1]),
                     what="eager decode after the capture")


def test_capture_refuses_workspace_growth_then_records_projection():
    """slm_attn_decode_xb_dev sizes its q | k | v workspace on its first call:
    inside a capture that growth is refused; after one eager call the same
    call records, and its replay equals the eager result bit for bit."""
    dim, heads, kvh, msl = 256, 4, 2, 64
    hd = dim // heads
    kvd = hd * kvh
    log(f"projection capture: dim {dim} heads {heads}/{kvh}")
    wq = orc.quantize_q4_0(gen([31, 1], (dim, dim)) * np.float32(0.1))
    wk = orc.quantize_q4_0(gen([31, 2], (kvd, dim)) * np.float32(0.1))
    wv = orc.quantize_q4_0(gen([31, 3], (kvd, dim)) * np.float32(0.1))
    xb = gen([31, 4], (4, dim))
    with P.AttentionContext(dim, heads, kvh, msl, 1, 1e4) as ctx, \
            P.Q4Matrix(wq, dim, dim) as mq, P.Q4Matrix(wk, kvd, dim) as mk, \
            P.Q4Matrix(wv, kvd, dim) as mv:
        x = torch.from_numpy(xb).cuda()
        out = torch.zeros(4, dim, device="cuda")
        torch.cuda.synchronize()
        ctx.capture_begin()
        with pytest.raises(P.SlmAttnError) as ei:
            ctx.decode_xb_dev(0, 0, x[0].data_ptr(), mq, mk, mv, out[0].data_ptr())
        assert ei.value.code == P.ERR_CAPTURE
        zeros = torch.zeros(kvd, device="cuda")  # something to record: row 10, never read
        ctx.kv_write_dev(0, 1, 10, 1, zeros.data_ptr())
        ctx.capture_end().close()
        for pos in range(3):  # eager: sizes the workspace
            ctx.decode_xb_dev(0, pos, x[pos].data_ptr(), mq, mk, mv, out[pos].data_ptr())
        ctx.sync()
        eager = out.cpu().numpy()
        eager_k = ctx.kv_read(0, 0, 0, 3)
        ctx.capture_begin()
        for pos in range(3):
            ctx.decode_xb_dev(0, pos, x[pos].data_ptr(), mq, mk, mv, out[pos].data_ptr())
        with ctx.capture_end() as graph:
            for rep in range(2):
                out.zero_()
                ctx.kv_write(0, 0, 0, np.zeros((3, kvd), np.float32))
                torch.cuda.synchronize()
                ctx.graph_launch(graph)
                ctx.sync()
                assert_bitwise(out.cpu().numpy(), eager, f"projection replay {rep}")
                assert_bitwise(ctx.kv_read(0, 0, 0, 3), eager_k, f"projection replay {rep} K")


def test_layer_decode_steps_in_a_graph():
    """Four one-token steps of the whole transformer block (RMSNorm + Q/K/V,
    decode attention with split merge, Wo + residual, RMSNorm + gate/up +
    SwiGLU, down + residual: slm_layer_forward_dev) recorded once and
    replayed: the residual rows and the appended K/V rows equal the eager
    steps' bit for bit on every replay."""
    from test_gpu_layer import Block

    dim, hidden, heads, kvh, msl, pre = 576, 1536, 9, 3, 640, 580
    kvd = dim // heads * kvh
    eps = 1e-5
    steps = 4
    log(f"layer decode graph: dim {dim} heads {heads}/{kvh} hidden {hidden} after {pre} rows")
    blk = Block(61, dim, kvd, hidden)
    try:
        with P.AttentionContext(dim, heads, kvh, msl, 1, 1e4) as ctx:
            assert ctx.decode_splits(pre + 1)[0] > 1  # the merge runs in the recording
            x = torch.from_numpy(gen([62, dim], (msl, dim))).cuda()
            ctx.layer_forward_dev(0, 0, pre, blk.dev, eps, x[:pre].data_ptr())
            ctx.sync()
            x_in = x[pre:pre + steps].clone()

            def run():
                for st in range(steps):
                    ctx.layer_forward_dev(0, pre + st, 1, blk.dev, eps, x[pre + st].data_ptr())

            run()
            ctx.sync()
            eager = x.cpu().numpy()
            eager_k = ctx.kv_read(0, 0, pre, steps)
            eager_v = ctx.kv_read(0, 1, pre, steps)
            x[pre:pre + steps].copy_(x_in)
            torch.cuda.synchronize()
            ctx.capture_begin()
            run()
            with ctx.capture_end() as graph:
                rng = np.random.default_rng(63)
                for rep in range(3):
                    x[pre:pre + steps].copy_(x_in)
                    ctx.kv_write(0, 0, pre, rng.standard_normal((steps, kvd), dtype=np.float32))
                    ctx.kv_write(0, 1, pre, rng.standard_normal((steps, kvd), dtype=np.float32))
                    torch.cuda.synchronize()
                    ctx.graph_launch(graph)
                    ctx.sync()
                    assert_bitwise(x.cpu().numpy(), eager, f"layer replay {rep} residual rows")
                    assert_bitwise(ctx.kv_read(0, 0, pre, steps), eager_k, f"layer replay {rep} K")
                    assert_bitwise(ctx.kv_read(0, 1, pre, steps), eager_v, f"layer replay {rep} V")
    finally:
        blk.close()
