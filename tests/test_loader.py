"""Offline checkpoint loader: HF-named safetensors -> the reference's weights dict (CPU)."""

import json
import os

import pytest
import torch

HERE = os.path.dirname(os.path.abspath(__file__))


def _tiny():
    from qwen_megakernel.shapes import Qwen3Shape

    cfg = json.load(open(os.path.join(HERE, "golden", "hf_tiny_keys.json")))
    c = cfg["config"]
    return Qwen3Shape("tiny", c["num_layers"], c["hidden"], c["intermediate"], 4, 2, 64, c["vocab"]), cfg["state_dict"]


def _state_from_hf_keys(keys, seed=0, tie=True):
    """A state dict with HF's own key names and shapes (fixture written by HF), distinct values per key."""
    g = torch.Generator().manual_seed(seed)
    sd = {k: torch.randn(*shp, generator=g).to(torch.bfloat16) for k, shp in keys.items()}
    if tie:
        sd["lm_head.weight"] = sd["model.embed_tokens.weight"].clone()
    return sd


def test_loader_consumes_hf_key_names_in_reference_order():
    from qwen_megakernel.shapes import LAYER_TENSOR_NAMES
    from qwen_megakernel.weights import load_weights_from_state_dict

    shape, keys = _tiny()
    sd = _state_from_hf_keys(keys)
    w = load_weights_from_state_dict(sd, shape, max_seq_len=32)
    hf = ["input_layernorm.weight", "self_attn.q_proj.weight", "self_attn.k_proj.weight",
          "self_attn.v_proj.weight", "self_attn.q_norm.weight", "self_attn.k_norm.weight",
          "self_attn.o_proj.weight", "post_attention_layernorm.weight", "mlp.gate_proj.weight",
          "mlp.up_proj.weight", "mlp.down_proj.weight"]
    assert len(LAYER_TENSOR_NAMES) == 11 and len(w["layer_weights"]) == 11 * shape.num_layers
    for i in range(shape.num_layers):
        for j, n in enumerate(hf):
            assert torch.equal(w["layer_weights"][11 * i + j], sd[f"model.layers.{i}.{n}"]), (i, n)
    assert torch.equal(w["embed_weight"], sd["model.embed_tokens.weight"])
    assert torch.equal(w["final_norm_weight"], sd["model.norm.weight"])
    assert w["lm_head_weight"] is w["embed_weight"]  # tied, as the reference (model.py:87)
    # every key HF's model has is consumed (nothing left over but the tied head)
    used = {f"model.layers.{i}.{n}" for i in range(shape.num_layers) for n in hf}
    used |= {"model.embed_tokens.weight", "model.norm.weight", "lm_head.weight"}
    assert used == set(keys)


def test_loader_untied_head_and_shape_errors():
    from qwen_megakernel.weights import load_weights_from_state_dict

    shape, keys = _tiny()
    sd = _state_from_hf_keys(keys, tie=False)
    w = load_weights_from_state_dict(sd, shape, max_seq_len=32)
    assert torch.equal(w["lm_head_weight"], sd["lm_head.weight"]) and w["lm_head_weight"] is not w["embed_weight"]
    bad = dict(sd)
    bad["model.layers.1.mlp.up_proj.weight"] = torch.zeros(3, 3, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="up_proj"):
        load_weights_from_state_dict(bad, shape, max_seq_len=32)
    missing = dict(sd)
    del missing["model.layers.0.self_attn.k_norm.weight"]
    with pytest.raises(KeyError, match="k_norm"):
        load_weights_from_state_dict(missing, shape, max_seq_len=32)


def test_safetensors_directory_roundtrip_gives_identical_oracle_logits(tmp_path):
    """Save seeded weights as an HF-named safetensors checkpoint, load them back through
    qwen_megakernel.load_weights, and decode with the oracle: logits are bit-identical."""
    from safetensors.torch import save_file

    from oracle.qwen3_ref import OracleDecoder
    from qwen_megakernel.model import load_weights
    from qwen_megakernel.weights import make_weights

    shape, keys = _tiny()
    w = make_weights(shape, seed=0, norm_std=0.1, max_seq_len=32)
    hf = ["input_layernorm.weight", "self_attn.q_proj.weight", "self_attn.k_proj.weight",
          "self_attn.v_proj.weight", "self_attn.q_norm.weight", "self_attn.k_norm.weight",
          "self_attn.o_proj.weight", "post_attention_layernorm.weight", "mlp.gate_proj.weight",
          "mlp.up_proj.weight", "mlp.down_proj.weight"]
    sd = {"model.embed_tokens.weight": w["embed_weight"], "model.norm.weight": w["final_norm_weight"]}
    for i in range(shape.num_layers):
        for j, n in enumerate(hf):
            sd[f"model.layers.{i}.{n}"] = w["layer_weights"][11 * i + j]
    assert set(sd) | {"lm_head.weight"} == set(keys)  # exactly HF's names
    # split over two files, as sharded checkpoints are
    names = sorted(sd)
    save_file({k: sd[k].contiguous() for k in names[: len(names) // 2]}, str(tmp_path / "model-00001-of-00002.safetensors"))
    save_file({k: sd[k].contiguous() for k in names[len(names) // 2:]}, str(tmp_path / "model-00002-of-00002.safetensors"))
    w2, tok = load_weights(str(tmp_path), verbose=False, max_seq_len=32, device="cpu", shape=shape)
    assert tok is None
    a = OracleDecoder(w, shape, max_seq_len=32)
    b = OracleDecoder(w2, shape, max_seq_len=32)
    for t in [3, 14, 159, 26, 535]:
        assert torch.equal(a.step_logits(t), b.step_logits(t))
