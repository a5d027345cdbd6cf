"""Golden fixtures (tests/golden/*.npz, written by make_golden.py from the
oracle): the oracle must still reproduce them bit for bit (CPU), and the HIP
path must match them to the parity bar (GPU)."""
from pathlib import Path

import numpy as np
import pytest

from oracle import py_oracle as orc
from slm_testlib import assert_bitwise, assert_close, load_product

GOLDEN = Path(__file__).resolve().parent / "golden"
FILES = sorted(GOLDEN.glob("*.npz"))


def _load(path):
    d = np.load(path)  # plain arrays, allow_pickle stays False
    dim, h, kvh, msl, layers, npf, nd = (int(x) for x in d["config"])
    cfg = orc.Cfg(dim, h, kvh, msl, layers, float(d["theta"][0]))
    lays = sorted({int(k[1:k.index("_")]) for k in d.files if k.startswith("l")})
    return d, cfg, npf, nd, lays


def test_fixtures_present():
    assert {p.stem for p in FILES} >= {"ref_mha", "ref_gqa", "c0", "c1", "c2"}


@pytest.mark.parametrize("path", FILES, ids=[p.stem for p in FILES])
def test_oracle_reproduces_golden(path):
    d, cfg, npf, nd, lays = _load(path)
    om = orc.OracleModel(cfg)
    for l in lays:
        q, k, v = d[f"l{l}_q"], d[f"l{l}_k"], d[f"l{l}_v"]
        outs = [om.prefill(l, 0, q[:npf], k[:npf], v[:npf])]
        outs += [om.decode(l, p, q[p], k[p], v[p])[None] for p in range(npf, npf + nd)]
        assert_bitwise(np.concatenate(outs), d[f"l{l}_out"], f"{path.stem} layer {l} out")
        assert_bitwise(om.k_cache(l)[:npf + nd], d[f"l{l}_kcache"], f"{path.stem} K rows")


@pytest.mark.gpu
@pytest.mark.parametrize("path", FILES, ids=[p.stem for p in FILES])
def test_hip_path_matches_golden(path):
    P = load_product()
    d, cfg, npf, nd, lays = _load(path)
    print(f"golden {path.stem}", flush=True)
    with P.AttentionContext(cfg.dim, cfg.num_heads, cfg.num_kv_heads, cfg.max_seq_len,
                            cfg.num_layers, cfg.rope_theta) as ctx:
        for l in lays:
            q, k, v = d[f"l{l}_q"], d[f"l{l}_k"], d[f"l{l}_v"]
            outs = [ctx.prefill(l, 0, q[:npf], k[:npf], v[:npf])]
            outs += [ctx.decode(l, p, q[p], k[p], v[p])[None] for p in range(npf, npf + nd)]
            assert_close(np.concatenate(outs), d[f"l{l}_out"], what=f"{path.stem} layer {l}")
            assert_bitwise(ctx.kv_read(l, 0, 0, npf + nd), d[f"l{l}_kcache"], "K rows")
            assert_bitwise(ctx.kv_read(l, 1, 0, npf + nd), v, "V rows")
