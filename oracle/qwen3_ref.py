"""CPU oracle for the Qwen3 batch-1 bf16 decode step.

TEST INFRASTRUCTURE ONLY.  Only ``tests/``, ``__graft_entry__.smoke()`` and the
CPU-baseline leg of ``bench.py`` may import this module, and only as the
checker or the timed CPU baseline; the product path (the HIP kernel behind
``torch.ops.qwen_megakernel_C``) never calls it.

What it restates
----------------
The reference's correctness oracle and PyTorch baseline is HuggingFace
transformers' Qwen3 (reference qwen_megakernel/bench.py:19-55, 83-133 call
``AutoModelForCausalLM.from_pretrained("Qwen/Qwen3-0.6B")``).  That module is a
third-party dependency, unpinned in the reference (requirements.txt:2,
``transformers>=4.40.0``); the version installed here is 5.15.0.  This file
restates its bf16 eager decode semantics op for op, using the same torch CPU
operators and tensor ranks so that, on the same machine, results agree with
HF bit for bit (pinned by tests/test_oracle.py against fixtures written by
tests/golden/make_hf_golden.py):

* RMSNorm  -- modeling_qwen3.py:59-64: fp32 normalise, round to bf16, then
  ``weight * x`` in bf16.
* Linear   -- nn.Linear in bf16 (fp32 accumulation, one rounding).
* Q/K norm -- modeling_qwen3.py:252-253, per head over head_dim, before RoPE.
* RoPE     -- modeling_qwen3.py:140-169: ``x*cos + rotate_half(x)*sin`` in bf16
  with bf16 cos/sin tables; the tables are the reference's layout
  (qwen_megakernel/model.py:53-60) with theta = 1e6.
* Attention -- eager_attention_forward, modeling_qwen3.py:185-203: bf16
  ``q @ k^T`` then ``* head_dim**-0.5`` (scale as in
  qwen_megakernel/model.py:137), softmax in fp32, probabilities rounded to
  bf16, bf16 ``p @ v``; GQA by repeat_kv.
* Residual adds in bf16 (modeling_qwen3.py:316, 322); MLP
  ``down(silu(gate(x)) * up(x))`` in bf16 (:82); final norm (:423); tied LM
  head (:432, reference qwen_megakernel/model.py:87) producing bf16 logits.
* Greedy pick: ``argmax`` of the fp32 copy of the bf16 logits, first index on
  ties (HF generation/utils.py:2894, 2925).

State follows the reference's decode step (csrc/kernel.cu:1210, 1329): the K/V
of the new token are written at ``position`` of a ``[L, NKV, S, D]`` bf16
cache (qwen_megakernel/model.py:140-148) and attention covers positions
``0..position``.
"""

from __future__ import annotations

import math

import torch
import torch.nn.functional as F

BF16 = torch.bfloat16


def rms_norm(x: torch.Tensor, weight: torch.Tensor, eps: float) -> torch.Tensor:
    """HF Qwen3RMSNorm.forward (modeling_qwen3.py:59-64)."""
    h = x.to(torch.float32)
    var = h.pow(2).mean(-1, keepdim=True)
    h = h * torch.rsqrt(var + eps)
    return weight * h.to(x.dtype)


def rotate_half(x: torch.Tensor) -> torch.Tensor:
    """HF rotate_half (modeling_qwen3.py:140-144)."""
    half = x.shape[-1] // 2
    return torch.cat((-x[..., half:], x[..., :half]), dim=-1)


def apply_rope(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
    """``x*cos + rotate_half(x)*sin`` in x's dtype (modeling_qwen3.py:168)."""
    return (x * cos) + (rotate_half(x) * sin)


def attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, scale: float) -> torch.Tensor:
    """Eager GQA attention for one query.

    q: [1, NQ, 1, D]; k, v: [1, NKV, C, D] (bf16).  Returns [1, NQ, 1, D].
    modeling_qwen3.py:172-203 (repeat_kv + eager_attention_forward).
    """
    n_rep = q.shape[1] // k.shape[1]
    b, nkv, c, d = k.shape
    ks = k[:, :, None, :, :].expand(b, nkv, n_rep, c, d).reshape(b, nkv * n_rep, c, d)
    vs = v[:, :, None, :, :].expand(b, nkv, n_rep, c, d).reshape(b, nkv * n_rep, c, d)
    w = torch.matmul(q, ks.transpose(2, 3)) * scale
    w = F.softmax(w, dim=-1, dtype=torch.float32).to(q.dtype)
    return torch.matmul(w, vs)


class OracleDecoder:
    """Token-at-a-time Qwen3 decode on the CPU (HF eager bf16 semantics).

    ``weights`` is the reference's weights dict (qwen_megakernel/model.py:82-89):
    ``embed_weight, layer_weights (11 per layer), final_norm_weight,
    lm_head_weight, cos_table, sin_table``.
    """

    def __init__(self, weights: dict, shape, max_seq_len: int | None = None,
                 num_layers: int | None = None):
        self.shape = shape
        self.num_layers = shape.num_layers if num_layers is None else num_layers
        cpu = torch.device("cpu")
        self.embed = weights["embed_weight"].to(cpu)
        self.lm_head = weights["lm_head_weight"].to(cpu)
        self.final_norm = weights["final_norm_weight"].to(cpu)
        self.cos = weights["cos_table"].to(cpu)
        self.sin = weights["sin_table"].to(cpu)
        lw = [t.to(cpu) for t in weights["layer_weights"]]
        self.layers = [lw[11 * i: 11 * i + 11] for i in range(self.num_layers)]
        self.max_seq_len = self.cos.shape[0] if max_seq_len is None else max_seq_len
        if self.max_seq_len > self.cos.shape[0]:
            raise ValueError("max_seq_len exceeds the RoPE table length")
        s = shape
        self.k_cache = torch.zeros(self.num_layers, s.num_kv_heads, self.max_seq_len, s.head_dim, dtype=BF16)
        self.v_cache = torch.zeros_like(self.k_cache)
        self.position = 0
        self.scale = 1.0 / math.sqrt(s.head_dim)

    def reset(self):
        self.position = 0
        self.k_cache.zero_()
        self.v_cache.zero_()

    def load_kv(self, k: torch.Tensor, v: torch.Tensor, cache_len: int):
        """Inject cache contents for positions ``[0, cache_len)`` and continue at ``cache_len``."""
        self.k_cache[:, :, :cache_len] = k[: self.num_layers, :, :cache_len]
        self.v_cache[:, :, :cache_len] = v[: self.num_layers, :, :cache_len]
        self.position = cache_len

    @torch.no_grad()
    def hidden_after_layers(self, token_id: int) -> torch.Tensor:
        """Run the decoder layers for one token; returns bf16 hidden ``[1, 1, H]``."""
        s = self.shape
        p = self.position
        if not 0 <= p < self.max_seq_len:
            raise ValueError(f"position {p} outside [0, {self.max_seq_len})")
        c = p + 1
        cos = self.cos[p].view(1, 1, 1, s.head_dim)
        sin = self.sin[p].view(1, 1, 1, s.head_dim)
        x = self.embed[token_id].view(1, 1, s.hidden)
        for li, (w_in, wq, wk, wv, wqn, wkn, wo, w_post, wg, wu, wd) in enumerate(self.layers):
            residual = x
            h = rms_norm(x, w_in, s.rms_eps)
            q = rms_norm(F.linear(h, wq).view(1, 1, s.num_q_heads, s.head_dim), wqn, s.rms_eps).transpose(1, 2)
            k = rms_norm(F.linear(h, wk).view(1, 1, s.num_kv_heads, s.head_dim), wkn, s.rms_eps).transpose(1, 2)
            v = F.linear(h, wv).view(1, 1, s.num_kv_heads, s.head_dim).transpose(1, 2)
            q = apply_rope(q, cos, sin)
            k = apply_rope(k, cos, sin)
            self.k_cache[li, :, p] = k[0, :, 0]
            self.v_cache[li, :, p] = v[0, :, 0]
            kc = self.k_cache[li: li + 1, :, :c]
            vc = self.v_cache[li: li + 1, :, :c]
            a = attention(q, kc, vc, self.scale)
            a = a.transpose(1, 2).reshape(1, 1, s.q_size)
            x = residual + F.linear(a, wo)
            residual = x
            h = rms_norm(x, w_post, s.rms_eps)
            x = residual + F.linear(F.silu(F.linear(h, wg)) * F.linear(h, wu), wd)
        return x

    @torch.no_grad()
    def step_logits(self, token_id: int) -> torch.Tensor:
        """Decode one token at ``self.position``; returns fp32 copy of bf16 logits ``[V]``."""
        x = self.hidden_after_layers(token_id)
        x = rms_norm(x, self.final_norm, self.shape.rms_eps)
        logits = F.linear(x, self.lm_head)
        self.position += 1
        return logits.view(-1).float()

    def step(self, token_id: int) -> int:
        return int(torch.argmax(self.step_logits(token_id)))


def top2_gap(logits: torch.Tensor) -> float:
    """Difference between the largest and second-largest logit."""
    top = torch.topk(logits, 2).values
    return float(top[0] - top[1])


def greedy_stream(dec: OracleDecoder, prompt: list[int], steps: int, record_logits: bool = False):
    """Feed ``prompt`` one token at a time, then continue greedily.

    Mirrors the reference's ``Decoder.generate`` (qwen_megakernel/model.py:207-245):
    ``prompt[:-1]`` are stepped, then ``steps`` tokens are produced starting
    from ``prompt[-1]``.  Returns dict(inputs, tokens, gaps[, logits]) where
    ``tokens[i]`` is the argmax after feeding ``inputs[i]``; the generated
    stream is ``tokens[len(prompt)-1:]`` (``steps`` tokens).
    """
    out_tokens, gaps, logits_list = [], [], []
    feed = list(prompt)
    i = 0
    while True:
        lg = dec.step_logits(feed[i])
        tok = int(torch.argmax(lg))
        out_tokens.append(tok)
        gaps.append(top2_gap(lg))
        if record_logits:
            logits_list.append(lg)
        i += 1
        if i >= len(prompt) - 1 + steps:
            break
        if i >= len(feed):
            feed.append(tok)
    res = dict(tokens=out_tokens, gaps=gaps, inputs=feed[: len(prompt) - 1 + steps])
    if record_logits:
        res["logits"] = torch.stack(logits_list)
    return res
