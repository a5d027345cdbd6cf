"""Writes the golden fixtures under tests/golden/ from the CPU oracle.

The reference ships no golden vectors for this path, so these are the
oracle's own outputs (once the oracle is pinned by tests/test_oracle.py),
frozen so that later changes to the oracle or to the HIP path are caught
against fixed data.  Each fixture holds, per layer: the seeded inputs q, k, v
(prefill rows then decode rows), the attention outputs, and the K cache rows
after the run (V rows equal the v inputs).

    python tests/golden/make_golden.py
"""
from __future__ import annotations

import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parent))
sys.path.insert(0, str(HERE.parents[1]))

from oracle import py_oracle as orc  # noqa: E402
from slm_testlib import WORKLOADS, layer_inputs  # noqa: E402

# workload key -> layers to freeze
FIXTURES = {"ref_mha": (0,), "ref_gqa": (0, 1), "c0": (0, 1), "c1": (0, 1), "c2": (0,)}


def run(key: str, layers) -> dict:
    w = WORKLOADS[key]
    cfg = w.cfg()
    om = orc.OracleModel(cfg)
    data = {
        "config": np.array([w.dim, w.num_heads, w.num_kv_heads, w.max_seq_len, w.num_layers,
                            w.prefill, w.decode], np.int64),
        "theta": np.array([w.theta], np.float32),
    }
    for layer in layers:
        q, k, v = layer_inputs(w, layer)
        n = w.prefill
        outs = [om.prefill(layer, 0, q[:n], k[:n], v[:n])]
        for st in range(w.decode):
            p = n + st
            outs.append(om.decode(layer, p, q[p], k[p], v[p])[None])
        rows = n + w.decode
        data[f"l{layer}_q"] = q
        data[f"l{layer}_k"] = k
        data[f"l{layer}_v"] = v
        data[f"l{layer}_out"] = np.concatenate(outs)
        data[f"l{layer}_kcache"] = om.k_cache(layer)[:rows].copy()
    return data


def main() -> None:
    for key, layers in FIXTURES.items():
        path = HERE / f"{key}.npz"
        np.savez(path, **run(key, layers))
        print(f"wrote {path} ({path.stat().st_size} bytes)")


if __name__ == "__main__":
    main()
