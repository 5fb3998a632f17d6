"""Exact-arithmetic CPU oracle for the Qwen3 bf16 decode step.

TEST INFRASTRUCTURE ONLY.  Only ``tests/``, ``__graft_entry__.smoke()`` and the
CPU-baseline leg of ``bench.py`` may import this module, and only as the
checker; the product path never calls it.

What it restates
----------------
The same HF Qwen3 bf16 eager decode as :mod:`oracle.qwen3_ref` (the
reference's correctness oracle, qwen_megakernel/bench.py:83-133: HF
transformers' Qwen3, modeling_qwen3.py), with the same bf16 rounding points,
but with every computation between two rounding points done exactly: in
float64, where bf16 x bf16 products are exact and sums of a few thousand of
them carry 40+ bits more than the rounding needs, and rounded once, correctly
(to nearest, ties to even), to the dtype HF stores the result in.  HF itself
(and :mod:`oracle.qwen3_ref`) accumulates in fp32 in its BLAS's order and uses
an approximate exp inside softmax, so its logits move by a few bf16 ulps with
the host's CPU; this oracle's logits depend on nothing but the inputs.  It is
the centre the kernel's own fp32 accumulation is measured against.

Rounding points (HF modeling_qwen3.py, transformers 5.15.0):

* RMSNorm (:59-64): ``h = bf16(x * rsqrt(mean(x^2) + eps))``, then
  ``bf16(w * h)``; eps is the fp32 value of 1e-6 that HF adds.
* every Linear (q, k, v, o, gate, up, down, LM head; :82, :232-246, :495):
  ``bf16(exact dot)``.
* q/k head norm (:252-253): RMSNorm over head_dim.
* RoPE (:140-169): ``bf16(bf16(x*cos) + bf16(rotate_half(x)*sin))``.
* attention (:185-203): scores ``bf16(exact q.k)``, scaled
  ``bf16(s * scale)`` with the fp32 scale HF multiplies by, probabilities
  ``bf16(exact softmax)`` (HF: fp32 softmax, then bf16), output
  ``bf16(exact p.v)``.
* residual adds (:316, :322) ``bf16(a + b)``; MLP ``bf16(silu(g))``, then
  ``bf16(s * u)`` (:82).
* logits bf16, argmax first index on ties (HF generation/utils.py:2894).

State and layout follow the reference's decode step (csrc/kernel.cu:1210,
1329; qwen_megakernel/model.py:140-148): K/V of position ``p`` in a
``[L, NKV, S, D]`` bf16 cache, attention over ``0..p``.  :meth:`forward`
runs T tokens at consecutive positions at once (causal); because every
reduction is exact, each row is the same as a one-token step, so a whole
token stream is checked in one pass.  With ``given_cache`` it runs them over
another decoder's cache instead of its own: each row then sees exactly the
inputs that decoder's step saw (its earlier K/V rows), which is how a kernel's
steps are compared one by one without the two trajectories drifting apart.

Pinned by tests/test_oracle_exact.py: the single rounding against a brute
force over the two bf16 neighbours (midpoint cases included), exact dots
against ``math.fsum``, batched rows against one-token steps (bit for bit), the
closed forms of attention, the given-cache mode against the ordinary one on
the oracle's own cache (bit for bit) and on a perturbed one, HF's golden
logits (hf_tiny.npz in full, hf_qwen3_0p6b.npz top-16 values and tokens)
within a few bf16 ulps, and the fp32-accumulating oracle within the same
bound.
"""

from __future__ import annotations

import math

import torch

BF16 = torch.bfloat16
F64 = torch.float64


def round_bf16(x: torch.Tensor) -> torch.Tensor:
    """float64 -> bf16, one rounding to nearest, ties to even.

    torch converts float64 to bf16 through float32, which rounds twice: a
    value just above (below) a bf16 midpoint can land exactly on it in fp32
    and then round to even, the wrong way.  Such fp32 results are moved one
    fp32 ulp toward the true value first, so the second rounding goes the
    way a single rounding would.
    """
    x = x.to(F64).contiguous()
    f = x.to(torch.float32)
    u = f.view(torch.int32).view(-1)
    cand = ((u & 0xFFFF) == 0x8000).nonzero(as_tuple=True)[0]  # fp32 results on a bf16 midpoint (rare)
    if cand.numel():
        xs = x.view(-1)[cand]
        fs = f.view(-1)[cand].to(F64)
        fix = (fs != xs) & torch.isfinite(fs)
        # toward the true value: in the sign-magnitude bit pattern, +1 moves away from zero
        step = torch.where(xs.abs() > fs.abs(), 1, -1).to(torch.int32)
        u[cand] = torch.where(fix, u[cand] + step, u[cand])
    return f.to(BF16)


def exact_linear(x: torch.Tensor, w64: torch.Tensor) -> torch.Tensor:
    """``bf16(x @ w^T)`` with an exact dot: x bf16 ``[..., K]``, w64 float64 ``[N, K]``."""
    return round_bf16(x.to(F64) @ w64.t())


def rms_norm(x: torch.Tensor, weight: torch.Tensor, eps: float) -> torch.Tensor:
    """HF Qwen3RMSNorm with exact mean and rsqrt: ``bf16(w * bf16(x / sqrt(mean(x^2) + eps)))``."""
    x64 = x.to(F64)
    var = (x64 * x64).mean(-1, keepdim=True)
    eps32 = float(torch.tensor(eps, dtype=torch.float32))
    h = round_bf16(x64 / torch.sqrt(var + eps32))
    return weight * h  # bf16 x bf16, rounded once (the product is exact in fp32)


def rotate_half(x: torch.Tensor) -> torch.Tensor:
    half = x.shape[-1] // 2
    return torch.cat((-x[..., half:], x[..., :half]), dim=-1)


def apply_rope(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
    """bf16 ``x*cos + rotate_half(x)*sin``: each product and the sum rounded once (elementwise ops)."""
    return (x * cos) + (rotate_half(x) * sin)


class ExactWeights:
    """float64 copies (exact) of a weights dict's projection matrices, shareable by several oracles.

    ``weights`` is the reference's weights dict (qwen_megakernel/model.py:82-89): about 4.8 GB
    of float64 for Qwen3-0.6B, 14 GB for Qwen3-1.7B.
    """

    def __init__(self, weights: dict, shape, num_layers: int | None = None):
        cpu = torch.device("cpu")
        self.shape = shape
        self.num_layers = shape.num_layers if num_layers is None else num_layers
        self.embed = weights["embed_weight"].to(cpu)
        self.lm_head64 = weights["lm_head_weight"].to(cpu).to(F64)
        self.final_norm = weights["final_norm_weight"].to(cpu)
        self.cos = weights["cos_table"].to(cpu)
        self.sin = weights["sin_table"].to(cpu)
        lw = [t.to(cpu) for t in weights["layer_weights"]]
        self.layers = []
        for i in range(self.num_layers):
            w_in, wq, wk, wv, wqn, wkn, wo, w_post, wg, wu, wd = lw[11 * i: 11 * i + 11]
            self.layers.append(dict(w_in=w_in, wq=wq.to(F64), wk=wk.to(F64), wv=wv.to(F64), wqn=wqn, wkn=wkn,
                                    wo=wo.to(F64), w_post=w_post, wg=wg.to(F64), wu=wu.to(F64), wd=wd.to(F64)))


class ExactOracle:
    """Qwen3 decode on the CPU with exact arithmetic between HF's bf16 rounding points.

    ``weights``: the reference's weights dict or an :class:`ExactWeights` (shared
    between oracles).  ``cos``/``sin`` replace the dict's RoPE tables (longer
    contexts); ``num_layers`` runs only the first layers.
    """

    def __init__(self, weights, shape, max_seq_len: int | None = None, num_layers: int | None = None,
                 cos: torch.Tensor | None = None, sin: torch.Tensor | None = None):
        self.w = weights if isinstance(weights, ExactWeights) else ExactWeights(weights, shape, num_layers)
        self.shape = shape
        self.num_layers = self.w.num_layers if num_layers is None else num_layers
        if self.num_layers > self.w.num_layers:
            raise ValueError("more layers than the weights hold")
        s = shape
        self.embed = self.w.embed
        self.lm_head64 = self.w.lm_head64
        self.final_norm = self.w.final_norm
        self.cos = self.w.cos if cos is None else cos.cpu()
        self.sin = self.w.sin if sin is None else sin.cpu()
        self.layers = self.w.layers[: self.num_layers]
        self.max_seq_len = self.cos.shape[0] if max_seq_len is None else max_seq_len
        if self.max_seq_len > self.cos.shape[0]:
            raise ValueError("max_seq_len exceeds the RoPE table length")
        self.k_cache = torch.zeros(self.num_layers, s.num_kv_heads, self.max_seq_len, s.head_dim, dtype=BF16)
        self.v_cache = torch.zeros_like(self.k_cache)
        self.position = 0
        # HF multiplies the bf16 scores by head_dim**-0.5 as an fp32 scalar; its product with a
        # bf16 score is exact in float64
        self.scale = float(torch.tensor(1.0 / math.sqrt(s.head_dim), dtype=torch.float32))

    def reset(self):
        self.position = 0
        self.k_cache.zero_()
        self.v_cache.zero_()

    def load_kv(self, k: torch.Tensor, v: torch.Tensor, cache_len: int):
        """Inject cache contents for positions ``[0, cache_len)`` and continue at ``cache_len``."""
        self.k_cache[:, :, :cache_len] = k[: self.num_layers, :, :cache_len]
        self.v_cache[:, :, :cache_len] = v[: self.num_layers, :, :cache_len]
        self.position = cache_len

    def _attention(self, li: int, q: torch.Tensor, p0: int, t: int, own=None) -> torch.Tensor:
        """q: bf16 ``[NQ, T, D]`` at positions p0..p0+T-1; returns bf16 ``[T, NQ*D]``.

        ``own = (k, v)`` (bf16 ``[NKV, T, D]``): row i attends to the cache's rows
        for positions below p0+i and to ``own``'s row i at p0+i (the cache holds
        another decoder's rows there); otherwise the cache holds this oracle's rows.
        """
        s = self.shape
        rep = s.num_q_heads // s.num_kv_heads
        c = p0 + t
        k64 = self.k_cache[li, :, :c].to(F64)  # [NKV, C, D]
        v64 = self.v_cache[li, :, :c].to(F64)
        qg = q.to(F64).contiguous().view(s.num_kv_heads, rep * t, s.head_dim)  # heads 2g, 2g+1 share kv head g
        sc = round_bf16(qg @ k64.transpose(1, 2))  # [NKV, rep*T, C]
        rows = torch.arange(rep * t)
        diag = p0 + rows % t  # the position of row r = r // t * t + i is p0 + i
        if own is not None:
            k_own = own[0].to(F64).repeat(1, rep, 1)  # row r -> own row r % t
            sc[:, rows, diag] = round_bf16((qg * k_own).sum(-1))
        sc = round_bf16(sc.to(F64) * self.scale).to(F64)
        # causal: row i (position p0+i) sees positions 0..p0+i
        pos = torch.arange(c)
        mask = pos[None, :] > diag[:, None]
        sc = sc.masked_fill(mask[None], float("-inf"))
        m = sc.max(-1, keepdim=True).values
        e = torch.exp(sc - m)
        pr = round_bf16(e / e.sum(-1, keepdim=True)).to(F64)
        if own is None:
            out = round_bf16(pr @ v64)  # [NKV, rep*T, D]
        else:
            p_diag = pr[:, rows, diag].clone()
            pr[:, rows, diag] = 0.0
            out = round_bf16(pr @ v64 + p_diag[..., None] * own[1].to(F64).repeat(1, rep, 1))
        out = out.view(s.num_kv_heads, rep, t, s.head_dim).permute(2, 0, 1, 3)
        return out.reshape(t, s.num_q_heads * s.head_dim)

    @torch.no_grad()
    def hidden(self, tokens: list[int], given_cache: bool = False) -> torch.Tensor:
        """Run the decoder layers over ``tokens`` at positions position..position+T-1; bf16 ``[T, H]``.

        Appends their K/V to the cache and advances the position.  With
        ``given_cache`` the cache already holds another decoder's rows for these
        positions (and all before): row i then attends to those rows below its
        position and to its own K/V at its position, so every row is computed from
        exactly the inputs that decoder's step had; the cache is left as it is and
        this oracle's own K/V rows are kept in ``own_k`` / ``own_v``
        (``[L, NKV, T, D]``) for comparison with the given ones.
        """
        s = self.shape
        t = len(tokens)
        p0 = self.position
        if t < 1 or p0 + t > self.max_seq_len:
            raise ValueError(f"positions {p0}..{p0 + t - 1} outside [0, {self.max_seq_len})")
        cos = self.cos[p0:p0 + t].view(1, t, s.head_dim)
        sin = self.sin[p0:p0 + t].view(1, t, s.head_dim)
        x = self.embed[torch.tensor(tokens, dtype=torch.long)]  # [T, H] bf16
        eps = s.rms_eps
        if given_cache:
            self.own_k = torch.empty(self.num_layers, s.num_kv_heads, t, s.head_dim, dtype=BF16)
            self.own_v = torch.empty_like(self.own_k)
        for li, L in enumerate(self.layers):
            residual = x
            h = rms_norm(x, L["w_in"], eps)
            q = exact_linear(h, L["wq"]).view(t, s.num_q_heads, s.head_dim).transpose(0, 1)
            k = exact_linear(h, L["wk"]).view(t, s.num_kv_heads, s.head_dim).transpose(0, 1)
            v = exact_linear(h, L["wv"]).view(t, s.num_kv_heads, s.head_dim).transpose(0, 1)
            q = apply_rope(rms_norm(q, L["wqn"], eps), cos, sin)
            k = apply_rope(rms_norm(k, L["wkn"], eps), cos, sin)
            if given_cache:
                self.own_k[li], self.own_v[li] = k, v
                a = self._attention(li, q, p0, t, own=(k, v))
            else:
                self.k_cache[li, :, p0:p0 + t] = k
                self.v_cache[li, :, p0:p0 + t] = v
                a = self._attention(li, q, p0, t)
            x = residual + exact_linear(a, L["wo"])
            residual = x
            h = rms_norm(x, L["w_post"], eps)
            g = exact_linear(h, L["wg"]).to(F64)
            sg = round_bf16(g / (1.0 + torch.exp(-g)))
            x = residual + exact_linear(sg * exact_linear(h, L["wu"]), L["wd"])
        self.position = p0 + t
        return x

    @torch.no_grad()
    def logits(self, x: torch.Tensor, chunk: int = 64) -> torch.Tensor:
        """bf16 logits (as fp32) of final hidden rows ``x`` ``[T, H]``: final norm, exact LM head."""
        n = rms_norm(x, self.final_norm, self.shape.rms_eps)
        rows = [exact_linear(n[i:i + chunk], self.lm_head64).float() for i in range(0, n.shape[0], chunk)]
        return torch.cat(rows, 0)

    def forward(self, tokens: list[int], emit=None, given_cache: bool = False) -> torch.Tensor:
        """Logits ``[len(emit), V]`` (fp32 holding bf16 values) of the rows ``emit`` (default: all)
        after running ``tokens`` at consecutive positions from the current one (``given_cache``:
        see :meth:`hidden`)."""
        x = self.hidden(list(tokens), given_cache)
        if emit is not None:
            x = x[torch.as_tensor(emit, dtype=torch.long)]
        return self.logits(x)

    def step_logits(self, token_id: int) -> torch.Tensor:
        return self.forward([token_id])[0]


def top2(logits: torch.Tensor):
    """(argmax with first-index ties, top-2 gap, top value) of a logits row."""
    v, i = torch.topk(logits, 2)
    return int(torch.argmax(logits)), float(v[0] - v[1]), float(v[0])
