"""Model shapes served by the decode kernel.

Qwen3-0.6B constants follow ``qwen_megakernel/model.py:8-16`` and
``csrc/kernel.cu:21-28`` of the reference; the 1.7B shape is the same
architecture family with hidden 2048 / MLP 6144.  RoPE theta is 1e6 (the
Qwen3 value), not the 10000 that ``qwen_megakernel/model.py:54-56`` uses.
"""

from __future__ import annotations

from dataclasses import dataclass


@dataclass(frozen=True)
class Qwen3Shape:
    name: str
    num_layers: int
    hidden: int
    intermediate: int
    num_q_heads: int
    num_kv_heads: int
    head_dim: int
    vocab: int
    rms_eps: float = 1e-6
    rope_theta: float = 1e6

    @property
    def q_size(self) -> int:
        return self.num_q_heads * self.head_dim

    @property
    def kv_size(self) -> int:
        return self.num_kv_heads * self.head_dim

    @property
    def attn_scale(self) -> float:
        # qwen_megakernel/model.py:137 -- 1/sqrt(head_dim)
        return self.head_dim ** -0.5

    def layer_weight_bytes(self) -> int:
        """bf16 bytes of one decoder layer (projections + four norm vectors)."""
        h, i, q, kv, d = self.hidden, self.intermediate, self.q_size, self.kv_size, self.head_dim
        proj = (q + 2 * kv) * h + h * q + 2 * i * h + h * i
        norms = 2 * h + 2 * d
        return 2 * (proj + norms)

    def weight_bytes_per_token(self) -> int:
        """Algorithmic weight bytes streamed per decode token (tied LM head)."""
        return (self.num_layers * self.layer_weight_bytes()
                + 2 * self.vocab * self.hidden   # LM head (= embedding table)
                + 2 * self.hidden                # embedding row
                + 2 * self.hidden)               # final norm

    def kv_bytes_per_position(self) -> int:
        """bf16 K+V bytes per cached position over all layers."""
        return self.num_layers * 2 * self.kv_size * 2

    def bytes_per_token(self, cache_len: int) -> int:
        """Weights + KV read over ``cache_len`` positions + KV written for one token."""
        return self.weight_bytes_per_token() + self.kv_bytes_per_position() * (cache_len + 1)


QWEN3_0_6B = Qwen3Shape("qwen3-0.6b", 28, 1024, 3072, 16, 8, 128, 151936)
QWEN3_1_7B = Qwen3Shape("qwen3-1.7b", 28, 2048, 6144, 16, 8, 128, 151936)

SHAPES = {s.name: s for s in (QWEN3_0_6B, QWEN3_1_7B)}

# Names of the 11 per-layer tensors, in the order of the packed pointer table
# (qwen_megakernel/model.py:66-79, csrc/torch_bindings.cpp:21-33).
LAYER_TENSOR_NAMES = (
    "input_layernorm",
    "q_proj",
    "k_proj",
    "v_proj",
    "q_norm",
    "k_norm",
    "o_proj",
    "post_attention_layernorm",
    "gate_proj",
    "up_proj",
    "down_proj",
)


def layer_tensor_shapes(shape: Qwen3Shape):
    h, i, q, kv, d = shape.hidden, shape.intermediate, shape.q_size, shape.kv_size, shape.head_dim
    return {
        "input_layernorm": (h,),
        "q_proj": (q, h),
        "k_proj": (kv, h),
        "v_proj": (kv, h),
        "q_norm": (d,),
        "k_norm": (d,),
        "o_proj": (h, q),
        "post_attention_layernorm": (h,),
        "gate_proj": (i, h),
        "up_proj": (i, h),
        "down_proj": (h, i),
    }
