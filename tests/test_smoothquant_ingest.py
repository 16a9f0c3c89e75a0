"""SmoothQuant checkpoint ingestion (CPU): the converter's output format
(quantize/smooth_quant/layer.py:19-94, smooth_quant/qwen2.py, written by
tests/hf_tiny.py:make_smoothquant_checkpoint) read by the loader and by the
CPU oracle's W8A8 mode, with static activation quantisation where a
quant_scale is stored.

Pins of the static path, independent of the oracle's own formulas:
  * closed-form quantiser cases (half-to-even ties, clamping at both ends);
  * the quantised linear layer against the float product within the exact
    error bound of per-channel weight and per-tensor activation rounding:
    |y_q - y| <= sum_k (|w_k| s_a / 2 + |x_k| s_w / 2 + s_w s_a / 4), plus
    fp32 evaluation slack;
  * the whole int8 model tracks the float model it was converted from
    (prefill logits within 15 % relative L2; the same first token).
"""
import json
import os

import pytest
import torch

from oracle import ops as O
from tests.hf_tiny import corpus, make_checkpoint, make_smoothquant_checkpoint


@pytest.fixture(scope="module")
def ckpts(tmp_path_factory):
    from transformers import AutoTokenizer
    d = str(tmp_path_factory.mktemp("qwen2_tiny_float"))
    hf = make_checkpoint(d, seed=0)
    tok = AutoTokenizer.from_pretrained(d, local_files_only=True)
    sq = str(tmp_path_factory.mktemp("qwen2_tiny_sq"))
    sd = make_smoothquant_checkpoint(sq, hf, [tok(t)["input_ids"] for t in corpus(8, seed=3)])
    return d, sq, sd, tok


def test_static_quant_closed_form():
    s = torch.tensor(0.5, dtype=torch.float16)
    x = torch.tensor([[0.25, 0.75, -1.25, 100.0, -100.0, 63.0]], dtype=torch.float32)
    q, st = O.quantize_static(x, s)
    # x / s = 0.5 -> 0, 1.5 -> 2, -2.5 -> -2 (ties to even), 200 -> 127, -200 -> -128, 126
    assert q.tolist() == [[0, 2, -2, 127, -128, 126]]
    assert st.tolist() == [0.5]


def test_static_linear_within_rounding_bound():
    g = torch.Generator().manual_seed(5)
    M, N, K = 6, 40, 96
    w = (torch.randn(N, K, generator=g) * 0.05).to(torch.float16)
    x = torch.randn(M, K, generator=g).to(torch.float16)
    qw, sw = O.quantize_weight_per_channel_absmax(w)
    sa = (x.abs().max().float() / 127).to(torch.float16)  # calibrated on this input: no clamping
    qx, st = O.quantize_static(x, sa)
    yq = O.dequant_int32(O.int8_gemm_i32(qx, qw), st, sw).double()
    y = x.double() @ w.double().t()
    s_w = sw.double().view(1, N)
    s_a = float(sa)
    bound = (w.double().abs().sum(1).view(1, N) * s_a / 2 + x.double().abs().sum(1, keepdim=True)
             * s_w / 2 + K * s_w * s_a / 4)
    slack = 1e-5 * (yq.abs() + 1)
    assert bool(((yq - y).abs() <= bound + slack).all())
    # and the bound is not vacuous: the error uses a fair share of it
    assert float(((yq - y).abs() / bound).max()) > 0.05


def test_loader_reads_converter_output(ckpts):
    from lite_lang_amd.models.qwen2.weights import is_int8_checkpoint, load_state_dict
    _, sq, sd, _ = ckpts
    got = load_state_dict(sq)  # pytorch_model.bin through torch.load(weights_only=True)
    assert is_int8_checkpoint(got)
    assert set(got) == set(sd)
    for k, v in sd.items():
        assert got[k].dtype == v.dtype and torch.equal(got[k], v), k
    assert got["model.layers.1.mlp.down_proj.weight_scale"].shape == (256, 1)
    assert got["model.layers.1.self_attn.o_proj.quant_scale"].dim() == 0


def test_oracle_int8_checkpoint_tracks_float_model(ckpts):
    from lite_lang_amd.models.qwen2.weights import load_state_dict
    from oracle.qwen2 import Qwen2Cfg, Qwen2Oracle
    d, sq, sd, tok = ckpts
    oc = Qwen2Cfg(num_layers=2, hidden=256, heads=4, kv_heads=2, intermediate=688, vocab=1024)
    prompts = [tok(t)["input_ids"] for t in corpus(3, seed=7)]
    tf, lf = Qwen2Oracle(oc, load_state_dict(d), torch.float32, 4, 128, 512).generate(
        prompts, 1, return_logits=True)
    tq, lq = Qwen2Oracle(oc, sd, torch.float32, 4, 128, 512, quant="w8a8").generate(
        prompts, 1, return_logits=True)
    rel = float((lq - lf).norm() / lf.norm())
    assert rel < 0.15, rel
    assert tq[:, 0].tolist() == tf[:, 0].tolist()


def test_per_channel_quant_config_rejected(tmp_path):
    from lite_lang_amd.models.qwen2.weights import check_smoothquant_config
    check_smoothquant_config(str(tmp_path))  # no quant_config.json: accepted
    with open(os.path.join(tmp_path, "quant_config.json"), "w") as f:
        json.dump({"qkv": "per-channel", "out": "per-tensor", "fc1": "per-token",
                   "fc2": "per-tensor"}, f)
    with pytest.raises(ValueError, match="input_layernorm"):
        check_smoothquant_config(str(tmp_path))
