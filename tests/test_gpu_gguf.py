"""A model read from a GGUF file and run on the device (slm_model_load_gguf,
then the slm_model_*_dev entry points), against the oracle's model on the
arrays the file was written from: the reference's prefill-test model,
with a separate and a tied lm_head, and with a rope.freq_base that the
context takes from the file."""
import sys

import numpy as np
import pytest

from gguf_writer import write_model
from oracle import py_oracle as orc
from slm_testlib import load_product
from test_oracle_layer import ref_model

P = load_product()
pytestmark = pytest.mark.gpu
torch = pytest.importorskip("torch")


def log(msg):
    print(msg, flush=True)
    sys.stdout.flush()


@pytest.mark.parametrize("tied,theta", [(False, None), (True, None), (False, 5e5)])
def test_gguf_model_on_device_matches_oracle(tmp_path, tied, theta):
    cfg, w = ref_model()
    if tied:
        w = orc.ModelWeights(w.token_embd, w.layers, w.output_norm, w.token_embd, w.vocab_size)
    if theta is not None:
        cfg = orc.Cfg(cfg.dim, cfg.num_heads, cfg.num_kv_heads, cfg.max_seq_len, cfg.num_layers,
                      theta)
    meta = dict(dim=cfg.dim, hidden_dim=128, num_heads=cfg.num_heads,
                num_kv_heads=cfg.num_kv_heads, max_seq_len=cfg.max_seq_len,
                num_layers=cfg.num_layers, rms_eps=1e-5)
    path = tmp_path / "model.gguf"
    write_model(path, meta, w, tied=tied, rope_theta=theta)
    prompt = [1, 7, 19, 42]
    with P.GgufFile(path) as f:
        c = f.model_config()
        assert c["rope_theta"] == np.float32(theta if theta is not None else 1e4)
        with P.GgufModel(f, c["num_layers"]) as m, \
                P.AttentionContext(c["dim"], c["num_heads"], c["num_kv_heads"], c["max_seq_len"],
                                   c["num_layers"], c["rope_theta"]) as ctx:
            assert m.vocab_size == w.vocab_size
            logits = torch.from_numpy(np.full(w.vocab_size, np.nan, np.float32)).cuda()
            nxt = ctx.model_prefill_dev(m, c["rms_eps"], prompt, 0, logits.data_ptr())
            ctx.sync()
            got = logits.cpu().numpy()
            want, onext, _ = orc.model_forward(orc.OracleModel(cfg), w, 1e-5, prompt, 0)
            err = np.abs(got - want).max()
            log(f"tied {tied} theta {theta}: next {nxt} (oracle {onext}), logits max abs {err:.3g}")
            assert err < 1e-4
            out = ctx.model_generate_dev(m, c["rms_eps"], prompt, 6)
            ref = orc.model_generate(orc.OracleModel(cfg), w, 1e-5, prompt, 6)
            log(f"  generate {out} oracle {ref}")
            assert out[0] == nxt
            assert out == ref
            emb = torch.from_numpy(np.zeros(cfg.dim, np.float32)).cuda()
            ctx.model_embed_dev(m, c["rms_eps"], prompt, emb.data_ptr())
            ctx.sync()
            e_want = orc.model_embed(orc.OracleModel(cfg), w, 1e-5, prompt)
            assert np.abs(emb.cpu().numpy() - e_want).max() < 1e-4


def test_gguf_model_missing_tensor_and_wrong_type(tmp_path):
    cfg, w = ref_model()
    meta = dict(dim=cfg.dim, hidden_dim=128, num_heads=cfg.num_heads,
                num_kv_heads=cfg.num_kv_heads, max_seq_len=cfg.max_seq_len,
                num_layers=cfg.num_layers, rms_eps=1e-5)
    path = tmp_path / "model.gguf"
    write_model(path, meta, w)
    with P.GgufFile(path) as f:
        with pytest.raises(P.SlmAttnError) as ei:   # asks for a third layer
            P.GgufModel(f, 3)
        assert ei.value.code == P.ERR_NOT_FOUND
