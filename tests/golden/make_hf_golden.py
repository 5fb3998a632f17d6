"""Write golden decode vectors from HuggingFace transformers' Qwen3 (CPU, bf16, eager).

The reference checks its kernel against HF Qwen3 (qwen_megakernel/bench.py:83-133);
HF is a third-party package (transformers 5.15.0 in this image), not part of the
reference.  This script builds ``Qwen3ForCausalLM`` from a local ``Qwen3Config``
(no network), loads the seeded synthetic weights of
``qwen_megakernel.weights.make_weights`` into it, and records, for a
token-at-a-time decode (the reference's ``Decoder.step`` pattern):

* ``hf_tiny.npz``         -- a 2-layer toy Qwen3 (hidden 256, 4/2 heads,
  head_dim 64, vocab 1000, random norm weights): full bf16 logits per step.
* ``hf_qwen3_0p6b.npz``   -- Qwen3-0.6B shape, seed-0 weights, 16-token seed-1
  prompt, 64 greedy steps: input/output tokens, top-2 gaps, top-16 logits and
  full-logit checksums per step, full logits of the first and last step, a
  weight fingerprint, and HF ``generate()`` tokens (batched prefill).
* ``hf_rope.npz``         -- HF rotary-embedding cos/sin rows for selected
  positions (head_dim 128, theta 1e6).
* ``hf_tiny_keys.json``   -- HF's state-dict names and shapes for the tiny
  config (``python tests/golden/make_hf_golden.py keys`` writes only this).
* ``qwen_megakernel/data/hf_greedy_qwen3_0p6b.json`` -- the prompt, HF's
  greedy tokens and top-2 gaps of ``hf_qwen3_0p6b.npz`` as JSON, for
  ``qwen_megakernel.bench.correctness_check`` (``python
  tests/golden/make_hf_golden.py package`` rewrites it from the npz alone).

Run:  python tests/golden/make_hf_golden.py   (about a minute on 8 cores)
"""

from __future__ import annotations

import os
import platform
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

from qwen_megakernel.shapes import QWEN3_0_6B, Qwen3Shape  # noqa: E402
from qwen_megakernel.weights import make_prompt, make_weights  # noqa: E402

TINY = Qwen3Shape("tiny", 2, 256, 512, 4, 2, 64, 1000)
HF_PARAM_NAMES = [
    "input_layernorm.weight", "self_attn.q_proj.weight", "self_attn.k_proj.weight",
    "self_attn.v_proj.weight", "self_attn.q_norm.weight", "self_attn.k_norm.weight",
    "self_attn.o_proj.weight", "post_attention_layernorm.weight", "mlp.gate_proj.weight",
    "mlp.up_proj.weight", "mlp.down_proj.weight",
]


def cpu_signature() -> str:
    flags = ""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("flags"):
                    fl = set(line.split(":")[1].split())
                    flags = ",".join(sorted(x for x in fl if x.startswith(("avx512", "amx", "avx2"))))
                    break
    except OSError:
        pass
    return f"torch={torch.__version__};machine={platform.machine()};{flags}"


def hf_model(shape: Qwen3Shape, w: dict, num_layers: int):
    from transformers import Qwen3Config, Qwen3ForCausalLM

    cfg = Qwen3Config(
        vocab_size=shape.vocab, hidden_size=shape.hidden, intermediate_size=shape.intermediate,
        num_hidden_layers=num_layers, num_attention_heads=shape.num_q_heads,
        num_key_value_heads=shape.num_kv_heads, head_dim=shape.head_dim,
        max_position_embeddings=40960, rms_norm_eps=shape.rms_eps,
        rope_parameters={"rope_type": "default", "rope_theta": shape.rope_theta},
        tie_word_embeddings=True, attention_bias=False, hidden_act="silu",
        attn_implementation="eager")
    # _from_config with a dtype mirrors from_pretrained(dtype=bf16): parameters
    # are bf16 while the rotary inv_freq buffer stays fp32.
    m = Qwen3ForCausalLM._from_config(cfg, dtype=torch.bfloat16).eval()
    assert m.model.rotary_emb.inv_freq.dtype == torch.float32
    sd = {"model.embed_tokens.weight": w["embed_weight"], "model.norm.weight": w["final_norm_weight"],
          "lm_head.weight": w["embed_weight"]}
    for i in range(num_layers):
        for j, n in enumerate(HF_PARAM_NAMES):
            sd[f"model.layers.{i}.{n}"] = w["layer_weights"][11 * i + j]
    res = m.load_state_dict(sd, strict=True)
    assert not res.missing_keys and not res.unexpected_keys
    return m


@torch.no_grad()
def hf_token_stream(m, prompt: list[int], steps: int):
    """Token-at-a-time greedy decode; returns inputs, outputs and per-step logits."""
    from transformers.cache_utils import DynamicCache

    cache = DynamicCache(config=m.config)
    feed = list(prompt)
    outs, logits = [], []
    total = len(prompt) - 1 + steps
    for p in range(total):
        o = m(input_ids=torch.tensor([[feed[p]]]), position_ids=torch.tensor([[p]]),
              past_key_values=cache, use_cache=True)
        lg = o.logits[0, -1].float()
        tok = int(torch.argmax(lg))
        outs.append(tok)
        logits.append(lg)
        if p + 1 >= len(feed) and p + 1 < total:
            feed.append(tok)
    return feed[:total], outs, torch.stack(logits)


def bf16_bits(t: torch.Tensor) -> np.ndarray:
    return t.to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)


def checksums(logits: torch.Tensor) -> np.ndarray:
    x = logits.double()
    idx = torch.arange(x.shape[-1], dtype=torch.float64)
    return torch.stack([x.sum(-1), (x * x).sum(-1), (x * idx).sum(-1) / x.shape[-1]], -1).numpy()


def weight_fingerprint(w: dict) -> np.ndarray:
    rows = [w["embed_weight"].double().sum(), w["embed_weight"][12345].double().sum()]
    for t in w["layer_weights"]:
        rows.append(t.double().sum())
    rows.append(w["final_norm_weight"].double().sum())
    return torch.stack(rows).numpy()


def write_state_dict_keys():
    """HF's own parameter names and shapes for the tiny config (pins the checkpoint loader's key walk)."""
    import json

    w = make_weights(TINY, seed=0, norm_std=0.1, max_seq_len=64)
    m = hf_model(TINY, w, TINY.num_layers)
    keys = {k: list(v.shape) for k, v in m.state_dict().items()}
    with open(os.path.join(HERE, "hf_tiny_keys.json"), "w") as f:
        json.dump({"config": {"num_layers": TINY.num_layers, "hidden": TINY.hidden,
                              "intermediate": TINY.intermediate, "vocab": TINY.vocab},
                   "state_dict": keys}, f, indent=0, sort_keys=True)


def main():
    torch.set_num_threads(max(1, len(os.sched_getaffinity(0))))
    sig = cpu_signature()
    write_state_dict_keys()

    # tiny config, full logits
    w = make_weights(TINY, seed=0, norm_std=0.1, max_seq_len=64)
    prompt = make_prompt(8, TINY.vocab, seed=1)
    m = hf_model(TINY, w, TINY.num_layers)
    inputs, outs, logits = hf_token_stream(m, prompt, 16)
    np.savez_compressed(os.path.join(HERE, "hf_tiny.npz"), inputs=np.array(inputs, np.int64),
                        tokens=np.array(outs, np.int64), logits_bf16=bf16_bits(logits),
                        prompt_len=len(prompt), cpu=sig)

    # Qwen3-0.6B shape, config-0 workload
    w = make_weights(QWEN3_0_6B, seed=0, max_seq_len=128)
    prompt = make_prompt(16, QWEN3_0_6B.vocab, seed=1)
    m = hf_model(QWEN3_0_6B, w, QWEN3_0_6B.num_layers)
    inputs, outs, logits = hf_token_stream(m, prompt, 64)
    top = torch.topk(logits, 16, dim=-1)
    gaps = (top.values[:, 0] - top.values[:, 1]).numpy()
    gen = m.generate(torch.tensor([prompt]), max_new_tokens=16, do_sample=False, use_cache=True,
                     pad_token_id=0)
    np.savez_compressed(
        os.path.join(HERE, "hf_qwen3_0p6b.npz"),
        prompt=np.array(prompt, np.int64), inputs=np.array(inputs, np.int64),
        tokens=np.array(outs, np.int64), gaps=gaps, top16_idx=top.indices.numpy().astype(np.int64),
        top16_bf16=bf16_bits(top.values), checksums=checksums(logits),
        logits_first_bf16=bf16_bits(logits[0]), logits_last_bf16=bf16_bits(logits[-1]),
        weight_fingerprint=weight_fingerprint(w),
        generate_tokens=gen[0, len(prompt):].numpy().astype(np.int64), cpu=sig)

    # RoPE rows from HF's rotary embedding
    from transformers import Qwen3Config
    from transformers.models.qwen3.modeling_qwen3 import Qwen3RotaryEmbedding
    cfg = Qwen3Config(head_dim=128, hidden_size=1024, num_attention_heads=16,
                      rope_parameters={"rope_type": "default", "rope_theta": 1e6},
                      max_position_embeddings=40960)
    rot = Qwen3RotaryEmbedding(cfg)
    positions = np.array([0, 1, 2, 3, 7, 100, 1023, 1024, 2047, 4095, 8191, 32767, 33023], np.int64)
    x = torch.zeros(1, 1, 128, dtype=torch.bfloat16)
    cos, sin = rot(x, torch.tensor(positions)[None])
    np.savez_compressed(os.path.join(HERE, "hf_rope.npz"), positions=positions,
                        cos_bf16=bf16_bits(cos[0]), sin_bf16=bf16_bits(sin[0]))
    print("golden fixtures written:", sig)


def write_package_tokens():
    """HF's greedy continuation of the config-0 prompt, from hf_qwen3_0p6b.npz, as package data."""
    import json

    d = np.load(os.path.join(HERE, "hf_qwen3_0p6b.npz"))
    n0 = len(d["prompt"]) - 1
    out = {
        "source": "HF transformers Qwen3ForCausalLM, bf16 eager, CPU; tests/golden/make_hf_golden.py",
        "weights": "qwen_megakernel.weights.make_weights(QWEN3_0_6B, seed=0): N(0, 0.02) bf16, norms 1, tied",
        "prompt": [int(t) for t in d["prompt"]],
        "greedy_tokens": [int(t) for t in d["tokens"][n0:]],
        "top2_gaps": [float(g) for g in d["gaps"][n0:]],
        "top_logits": [float(x) for x in
                       torch.from_numpy(d["top16_bf16"][n0:, 0].view(np.int16)).view(torch.bfloat16).float()],
        "generate_tokens": [int(t) for t in d["generate_tokens"]],
        "weight_fingerprint_head": [float(x) for x in d["weight_fingerprint"][:4]],
    }
    dst = os.path.join(os.path.dirname(os.path.dirname(HERE)), "qwen_megakernel", "data")
    os.makedirs(dst, exist_ok=True)
    with open(os.path.join(dst, "hf_greedy_qwen3_0p6b.json"), "w") as f:
        json.dump(out, f, indent=1)


if __name__ == "__main__" and sys.argv[1:] == ["keys"]:
    write_state_dict_keys()
elif __name__ == "__main__" and sys.argv[1:] == ["package"]:
    write_package_tokens()
elif __name__ == "__main__":
    main()
    write_package_tokens()
