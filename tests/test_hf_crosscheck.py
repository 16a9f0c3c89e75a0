"""Cross-check against Hugging Face transformers (CPU), an implementation
independent of the reference, of the oracle and of this build.

A tiny Qwen2 checkpoint and a byte-level BPE tokenizer are written by
transformers/tokenizers themselves into a temporary directory (tests/hf_tiny.py,
offline, seeded). Checked here:
  * Qwen2Config.from_json and load_state_dict read that directory: dimensions
    and every tensor bit for bit;
  * the CPU oracle (fp32 storage, float64 compute) with the cos/sin table kept
    in fp32 and the final-norm eps set to HF's reproduces HF's greedy tokens on
    a ragged batch of three prompts, logits within 1e-3 (observed ~2e-5: fp32
    vs float64 arithmetic). This pins the oracle's whole forward -- embedding,
    RMSNorm, q/k/v biases, RoPE, GQA attention over the paged cache, SiLU MLP,
    tied lm_head, greedy argmax -- against transformers' Qwen2ForCausalLM;
  * the Tokenizer wrapper (litelang/scheduler/tokenizer/tokenizer.py:4-31):
    eos id, encode_single, left-padded batch encode, decode skipping eos.
"""
import os

import pytest
import torch

from tests.hf_tiny import EOS, corpus, hf_greedy, make_checkpoint


@pytest.fixture(scope="module")
def ckpt(tmp_path_factory):
    d = str(tmp_path_factory.mktemp("qwen2_tiny_hf"))
    return d, make_checkpoint(d, seed=0)


def _prompts(path, n=3):
    from transformers import AutoTokenizer
    tok = AutoTokenizer.from_pretrained(path, local_files_only=True)
    return [tok(t)["input_ids"] for t in corpus(n, seed=7)]


def test_config_and_loader_read_hf_checkpoint(ckpt):
    from lite_lang_amd.models.qwen2.weights import Qwen2Config, load_state_dict
    d, hf = ckpt
    cfg = Qwen2Config.from_json(os.path.join(d, "config.json"))
    assert (cfg.layer_nums, cfg.hidden_size, cfg.num_heads, cfg.num_key_value_heads,
            cfg.intermediate_size, cfg.vocab_size, cfg.tie_word_embeddings) == (
        2, 256, 4, 2, 688, 1024, True)
    assert cfg.head_dim == 64
    sd = load_state_dict(d)
    ref = hf.state_dict()
    for name, t in ref.items():
        if name == "lm_head.weight":  # tied: not stored in the checkpoint
            continue
        assert name in sd, name
        assert torch.equal(sd[name], t), name


def test_oracle_greedy_matches_hf(ckpt):
    from lite_lang_amd.models.qwen2.weights import load_state_dict
    from oracle.qwen2 import Qwen2Cfg, Qwen2Oracle
    d, hf = ckpt
    prompts = _prompts(d)
    assert sorted(len(p) for p in prompts) != [len(prompts[0])] * 3  # ragged
    ocfg = Qwen2Cfg(num_layers=2, hidden=256, heads=4, kv_heads=2, intermediate=688, vocab=1024,
                    eps=1e-6, final_eps=1e-6, table_dtype=torch.float32)
    orc = Qwen2Oracle(ocfg, load_state_dict(d), torch.float32, 4, 128, 512)
    n_new = 12
    toks, logits = orc.generate(prompts, n_new, return_logits=True)
    for b, p in enumerate(prompts):
        ref_ids, ref_logits = hf_greedy(hf, p, n_new)
        assert toks[b].tolist() == ref_ids.tolist(), f"prompt {b}"
        err = float((logits[b].double() - ref_logits.double()).abs().max())
        assert err <= 1e-3, f"prompt {b}: logits differ by {err}"


def test_tokenizer_wrapper(ckpt):
    from transformers import AutoTokenizer
    from lite_lang_amd.scheduler import Tokenizer
    d, _ = ckpt
    ref = AutoTokenizer.from_pretrained(d, local_files_only=True)
    tok = Tokenizer(d)
    assert tok.eos_token_id == EOS
    texts = corpus(2, seed=11)
    one = tok.encode_single(texts[0])
    assert one.shape[0] == 1 and one[0].tolist() == ref(texts[0])["input_ids"]
    ids, mask = tok.encode([texts[0], texts[1][:12]])
    n0, n1 = len(ref(texts[0])["input_ids"]), len(ref(texts[1][:12])["input_ids"])
    width = max(n0, n1)
    assert ids.shape == (2, width) and mask.shape == (2, width)
    short = 1 if n1 < n0 else 0
    pad = width - min(n0, n1)
    assert mask[short, :pad].sum() == 0 and mask[short, pad:].all()  # left padding
    assert ids[short, :pad].eq(EOS).all()                             # pad is eos
    out = tok.decode([one[0].tolist() + [EOS]])
    assert out == [texts[0]]  # byte-level round trip; eos skipped
