"""Seeded synthetic weights and RoPE tables in the reference's weights-dict layout.

The reference's ``load_weights`` (qwen_megakernel/model.py:21-94) downloads
Qwen3-0.6B from the HuggingFace hub and returns::

    dict(embed_weight, layer_weights=[11 tensors per layer], final_norm_weight,
         lm_head_weight=embed_weight, cos_table, sin_table)

There is no network here, so :func:`make_weights` draws the same dict from a
seeded generator: ``torch.Generator('cpu').manual_seed(seed)`` and, in the
canonical order ``embed_tokens`` then, per layer, q, k, v, o, gate, up, down,
each ``randn(fp32) * std`` rounded to bf16.  Norm weights are 1 (or
``1 + N(0, norm_std)`` when ``norm_std > 0``, which the parity tests use so a
kernel that ignores a norm weight cannot pass).  :func:`load_weights_from_state_dict`
builds the same dict from a real checkpoint's state dict.
"""

from __future__ import annotations

import torch

from .shapes import QWEN3_0_6B, LAYER_TENSOR_NAMES, Qwen3Shape, layer_tensor_shapes

BF16 = torch.bfloat16


def rope_tables(max_seq_len: int, head_dim: int, theta: float):
    """cos/sin tables ``[max_seq_len, head_dim]`` in bf16.

    Layout of qwen_megakernel/model.py:53-60 (fp32 inv_freq, fp32 position
    products, duplicated halves, rounded to bf16), with the caller's theta.
    Row ``p`` equals what HF Qwen3's rotary embedding produces for position
    ``p`` (modeling_qwen3.py:121-137); tests/test_oracle.py checks that.
    """
    inv_freq = 1.0 / (theta ** (torch.arange(0, head_dim, 2, dtype=torch.int64).to(torch.float32) / head_dim))
    positions = torch.arange(max_seq_len, dtype=torch.float32)
    freqs = torch.outer(positions, inv_freq)
    emb = torch.cat((freqs, freqs), dim=-1)
    return emb.cos().to(BF16).contiguous(), emb.sin().to(BF16).contiguous()


def _draw(gen: torch.Generator, shape, std: float) -> torch.Tensor:
    return (torch.randn(shape, generator=gen, dtype=torch.float32) * std).to(BF16)


def make_weights(shape: Qwen3Shape = QWEN3_0_6B, seed: int = 0, std: float = 0.02,
                 norm_std: float = 0.0, max_seq_len: int = 2048,
                 num_layers: int | None = None, device: str | torch.device = "cpu"):
    """Seeded random weights in the reference's dict layout (CPU, then moved).

    ``num_layers`` < shape.num_layers draws only the first layers (same values
    as the full draw for those layers, since the order is canonical).
    """
    nl = shape.num_layers if num_layers is None else num_layers
    gen = torch.Generator("cpu").manual_seed(seed)
    shapes = layer_tensor_shapes(shape)
    embed = _draw(gen, (shape.vocab, shape.hidden), std)
    layers: list[torch.Tensor] = []
    for _ in range(nl):
        drawn = {}
        for name in ("q_proj", "k_proj", "v_proj", "o_proj", "gate_proj", "up_proj", "down_proj"):
            drawn[name] = _draw(gen, shapes[name], std)
        layers.append(drawn)
    # Norm weights come after all projections so that the projection draws do
    # not depend on norm_std.
    norm_gen = torch.Generator("cpu").manual_seed(seed + 7919)
    flat: list[torch.Tensor] = []
    for drawn in layers:
        for name in LAYER_TENSOR_NAMES:
            if name in drawn:
                flat.append(drawn[name])
            else:
                flat.append(_norm_weight(norm_gen, shapes[name], norm_std))
    final_norm = _norm_weight(norm_gen, (shape.hidden,), norm_std)
    cos, sin = rope_tables(max_seq_len, shape.head_dim, shape.rope_theta)
    w = dict(
        embed_weight=embed,
        layer_weights=flat,
        final_norm_weight=final_norm,
        lm_head_weight=embed,
        cos_table=cos,
        sin_table=sin,
    )
    return to_device(w, device)


def _norm_weight(gen: torch.Generator, shp, norm_std: float) -> torch.Tensor:
    if norm_std <= 0.0:
        return torch.ones(shp, dtype=BF16)
    return (1.0 + torch.randn(shp, generator=gen, dtype=torch.float32) * norm_std).to(BF16)


def to_device(weights: dict, device) -> dict:
    """Move a weights dict to ``device`` keeping the LM head tied to the embedding."""
    device = torch.device(device)
    if weights["embed_weight"].device == device:
        return weights
    embed = weights["embed_weight"].to(device).contiguous()
    tied = weights["lm_head_weight"] is weights["embed_weight"]
    out = dict(
        embed_weight=embed,
        layer_weights=[t.to(device).contiguous() for t in weights["layer_weights"]],
        final_norm_weight=weights["final_norm_weight"].to(device).contiguous(),
        lm_head_weight=embed if tied else weights["lm_head_weight"].to(device).contiguous(),
        cos_table=weights["cos_table"].to(device).contiguous(),
        sin_table=weights["sin_table"].to(device).contiguous(),
    )
    return out


def load_weights_from_state_dict(state: dict, shape: Qwen3Shape = QWEN3_0_6B,
                                 max_seq_len: int = 2048, device="cpu"):
    """Build the weights dict from a Qwen3 ``state_dict`` (HF key names).

    Mirrors the key walk of qwen_megakernel/model.py:63-90 without the hub
    download; the caller supplies the tensors (e.g. from a local safetensors
    file).  Every tensor is checked against ``shape``.  ``lm_head.weight`` is
    used when the checkpoint holds a separate one; otherwise (Qwen3-0.6B and
    -1.7B tie it) the LM head is the embedding, as in the reference
    (qwen_megakernel/model.py:87).
    """
    hf_names = {
        "input_layernorm": "input_layernorm.weight",
        "q_proj": "self_attn.q_proj.weight",
        "k_proj": "self_attn.k_proj.weight",
        "v_proj": "self_attn.v_proj.weight",
        "q_norm": "self_attn.q_norm.weight",
        "k_norm": "self_attn.k_norm.weight",
        "o_proj": "self_attn.o_proj.weight",
        "post_attention_layernorm": "post_attention_layernorm.weight",
        "gate_proj": "mlp.gate_proj.weight",
        "up_proj": "mlp.up_proj.weight",
        "down_proj": "mlp.down_proj.weight",
    }
    expect = layer_tensor_shapes(shape)

    def get(key, shp):
        if key not in state:
            raise KeyError(f"checkpoint has no {key}")
        t = state[key]
        if tuple(t.shape) != tuple(shp):
            raise ValueError(f"{key}: shape {tuple(t.shape)}, expected {tuple(shp)} for {shape.name}")
        return t.to(BF16).contiguous()

    flat = []
    for i in range(shape.num_layers):
        for name in LAYER_TENSOR_NAMES:
            flat.append(get(f"model.layers.{i}.{hf_names[name]}", expect[name]))
    embed = get("model.embed_tokens.weight", (shape.vocab, shape.hidden))
    lm_head = embed
    if "lm_head.weight" in state:
        head = get("lm_head.weight", (shape.vocab, shape.hidden))
        if not torch.equal(head, embed):
            lm_head = head
    cos, sin = rope_tables(max_seq_len, shape.head_dim, shape.rope_theta)
    w = dict(embed_weight=embed, layer_weights=flat,
             final_norm_weight=get("model.norm.weight", (shape.hidden,)),
             lm_head_weight=lm_head, cos_table=cos, sin_table=sin)
    return to_device(w, device)


def make_prompt(length: int, vocab: int, seed: int = 1) -> list[int]:
    """Random prompt token ids, ``randint(0, vocab)`` from ``manual_seed(seed)``."""
    gen = torch.Generator("cpu").manual_seed(seed)
    return torch.randint(0, vocab, (length,), generator=gen).tolist()


def make_kv_prefill(shape: Qwen3Shape, cache_len: int, seed: int = 2, max_seq_len: int | None = None):
    """Seeded N(0,1) bf16 K and V for ``cache_len`` positions, ``[L, NKV, S, D]``.

    Treated as post-RoPE cache contents (long-context workload).
    """
    s = cache_len if max_seq_len is None else max_seq_len
    gen = torch.Generator("cpu").manual_seed(seed)
    shp = (shape.num_layers, shape.num_kv_heads, cache_len, shape.head_dim)
    k = torch.zeros(shape.num_layers, shape.num_kv_heads, s, shape.head_dim, dtype=BF16)
    v = torch.zeros_like(k)
    k[:, :, :cache_len] = torch.randn(shp, generator=gen).to(BF16)
    v[:, :, :cache_len] = torch.randn(shp, generator=gen).to(BF16)
    return k, v
