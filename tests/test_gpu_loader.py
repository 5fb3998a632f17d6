"""The offline checkpoint loader on the GPU paths, with an untied LM head.

A Qwen3-0.6B checkpoint directory is written the way HF lays one out (two
safetensors shards with HF's key names, ``config.json``), with an
``lm_head.weight`` that differs from the embedding.  ``load_weights(dir)``
(reference qwen_megakernel/model.py:21-94, without the hub download) must
build the weights dict from it, and both the decode megakernel and the batched
path must read the head from ``lm_head_weight``: a kernel that read the
embedding instead would be 0.3+ away from the oracle's logits.
"""

import json
import os

import pytest
import torch

from parity import (LAYERS28, Tally, check_kv_rows, check_rows, decoder, exact_oracle, history_envelopes, kernel_stream,
                    lazy_envelopes, oracle_steps, stream_rows)

pytestmark = pytest.mark.gpu

HF = {
    "input_layernorm": "input_layernorm.weight", "q_proj": "self_attn.q_proj.weight",
    "k_proj": "self_attn.k_proj.weight", "v_proj": "self_attn.v_proj.weight",
    "q_norm": "self_attn.q_norm.weight", "k_norm": "self_attn.k_norm.weight",
    "o_proj": "self_attn.o_proj.weight", "post_attention_layernorm": "post_attention_layernorm.weight",
    "gate_proj": "mlp.gate_proj.weight", "up_proj": "mlp.up_proj.weight", "down_proj": "mlp.down_proj.weight",
}


@pytest.fixture(scope="module")
def checkpoint(tmp_path_factory, shape):
    """Seeded weights with non-unit norms and an untied head, saved as a two-shard checkpoint."""
    from safetensors.torch import save_file

    from qwen_megakernel.shapes import LAYER_TENSOR_NAMES
    from qwen_megakernel.weights import make_weights

    w = make_weights(shape, seed=11, norm_std=0.1, max_seq_len=256)
    g = torch.Generator().manual_seed(12)
    head = (torch.randn(shape.vocab, shape.hidden, generator=g) * 0.02).to(torch.bfloat16)
    sd = {"model.embed_tokens.weight": w["embed_weight"], "model.norm.weight": w["final_norm_weight"],
          "lm_head.weight": head}
    for i in range(shape.num_layers):
        for j, name in enumerate(LAYER_TENSOR_NAMES):
            sd[f"model.layers.{i}.{HF[name]}"] = w["layer_weights"][11 * i + j]
    d = tmp_path_factory.mktemp("qwen3_ckpt")
    keys = sorted(sd)
    half = len(keys) // 2
    save_file({k: sd[k].contiguous() for k in keys[:half]}, str(d / "model-00001-of-00002.safetensors"))
    save_file({k: sd[k].contiguous() for k in keys[half:]}, str(d / "model-00002-of-00002.safetensors"))
    with open(d / "config.json", "w") as f:
        json.dump({"hidden_size": shape.hidden, "num_hidden_layers": shape.num_layers,
                   "tie_word_embeddings": False}, f)
    w["lm_head_weight"] = head
    return str(d), w


def test_loaded_checkpoint_untied_head_decode_and_batched(monkeypatch, shape, checkpoint):
    from oracle.qwen3_exact import ExactWeights
    from qwen_megakernel.model import BatchDecoder, load_weights
    from qwen_megakernel.weights import make_prompt

    monkeypatch.setenv("HF_HUB_OFFLINE", "1")
    path, w_ref = checkpoint
    w, tok = load_weights(path, verbose=False, max_seq_len=256)
    assert tok is None  # no tokenizer files in the directory
    assert w["lm_head_weight"] is not w["embed_weight"]
    assert torch.equal(w["lm_head_weight"].cpu(), w_ref["lm_head_weight"])
    for a, b in zip(w["layer_weights"], w_ref["layer_weights"]):
        assert torch.equal(a.cpu(), b)
    ew = ExactWeights(w_ref, shape)
    prompt = make_prompt(12, shape.vocab, seed=3)

    # the decode megakernel: 12 prompt steps, then 16 greedy steps, every row
    kd = decoder(w, max_seq_len=256)
    feed, toks, lgs = kernel_stream(kd, prompt, 16)
    orc = exact_oracle(ew, shape, 256)
    ref = oracle_steps(orc, kd._k_cache, kd._v_cache, 0, feed)
    envs = lazy_envelopes(w_ref, shape, 256, kd._k_cache, kd._v_cache, 0, feed, ref)
    print(check_rows(Tally("loaded checkpoint, decode kernel"), ref, toks, lgs, bar=LAYERS28, envs=envs))
    check_kv_rows("loaded checkpoint", orc, kd._k_cache, kd._v_cache, 0, len(feed))
    # the check has teeth: an oracle with the embedding as its head is far from the kernel
    wrong_head = exact_oracle(ew, shape, 256)
    wrong_head.lm_head64 = w_ref["embed_weight"].double()
    wrong = oracle_steps(wrong_head, kd._k_cache, kd._v_cache, 0, feed[:4])
    assert (wrong - lgs[:4]).abs().max().item() > 0.3

    # the batched path: every prefill row, then two batched steps of two sequences
    dec = decoder(w, max_seq_len=256)
    tok0, lg0 = dec.prefill(prompt, return_logits=True)
    t = Tally("loaded checkpoint, batched path")
    pre = oracle_steps(exact_oracle(ew, shape, 256), dec._k_cache, dec._v_cache, 0, prompt, emit=[len(prompt) - 1])
    envs = lazy_envelopes(w_ref, shape, 256, dec._k_cache, dec._v_cache, len(prompt) - 1, prompt[-1:], pre)
    check_rows(t, pre, [tok0], lg0[None].cpu(), bar=LAYERS28, envs=envs)
    bd = BatchDecoder(weights=w, batch_size=2, max_seq_len=256, verbose=False)
    prompts = [prompt, make_prompt(7, shape.vocab, seed=4)]
    first = bd.prefill_all(prompts)
    gen, lgs2 = [[first[0]], [first[1]]], [[], []]
    for _ in range(2):
        nxt, logits = bd.step_logits([g[-1] for g in gen])
        for b in range(2):
            gen[b].append(nxt[b])
            lgs2[b].append(logits[b].cpu())
    for b in range(2):
        rows = stream_rows(exact_oracle(ew, shape, 256), bd._k_cache[b], bd._v_cache[b], prompts[b], gen[b])
        envs = history_envelopes(w_ref, shape, 256, bd._k_cache[b], bd._v_cache[b], prompts[b], gen[b], rows)[1:]
        check_rows(t, rows[1:], gen[b][1:], torch.stack(lgs2[b]), bar=LAYERS28, envs=envs)
    print(t)
