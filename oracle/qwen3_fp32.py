"""Host-independent fp32 restatement of the Qwen3 bf16 decode step (ctypes over qwen3_fp32.c).

TEST INFRASTRUCTURE ONLY.  Only ``tests/`` import this module, as a checker;
the product path never calls it.

It computes HF Qwen3's bf16 eager decode (the reference's correctness oracle,
reference qwen_megakernel/bench.py:83-133) the way an fp32 implementation
does -- fp32 sums between HF's bf16 rounding points -- with every sum taken by
one of four fixed orders (a pairwise tree, left to right, eight interleaved
partial sums, right to left) and exp evaluated in float64 (see the header
of ``qwen3_fp32.c``).  Its distances from :mod:`oracle.qwen3_exact` on given
inputs, over the four orders, are the size of error that fp32
implementations of the reference path carry on those inputs, independent of
the CPU it runs on.
The GPU tests use it to bound the kernel's error per step (tests/parity.py).

Same interface as :class:`oracle.qwen3_exact.ExactOracle` (``forward`` with
``given_cache``, ``k_cache`` / ``v_cache`` / ``position``, ``own_k`` /
``own_v``), so the helpers of tests/parity.py drive either.

Pinned by tests/test_oracle_fp32.py: each summation order against a
hand-built one, HF's golden logits (hf_tiny.npz, hf_qwen3_0p6b.npz) and the exact
oracle within fp32 noise, given-cache rows equal to ordinary rows on its own
cache, and planted mistakes that move it away from the exact oracle.
"""

from __future__ import annotations

import ctypes
import math
import os
import subprocess

import torch

_DIR = os.path.dirname(os.path.abspath(__file__))
LIB = os.path.join(_DIR, "libqwen3_fp32.so")
_lib = None

BF16 = torch.bfloat16


def build(force: bool = False) -> str:
    """Compile libqwen3_fp32.so with oracle/Makefile."""
    src = os.path.join(_DIR, "qwen3_fp32.c")
    if force or not os.path.exists(LIB) or os.path.getmtime(LIB) < os.path.getmtime(src):
        subprocess.run(["make", "-s", "-C", _DIR] + (["-B"] if force else []), check=True)
    return LIB


class _Model(ctypes.Structure):
    _fields_ = [
        ("num_layers", ctypes.c_int), ("hidden", ctypes.c_int), ("inter", ctypes.c_int), ("nq", ctypes.c_int),
        ("nkv", ctypes.c_int), ("hd", ctypes.c_int), ("vocab", ctypes.c_int), ("max_seq", ctypes.c_int),
        ("eps", ctypes.c_float), ("scale", ctypes.c_float),
        ("embed", ctypes.c_void_p), ("lm_head", ctypes.c_void_p), ("final_norm", ctypes.c_void_p),
        ("cos_t", ctypes.c_void_p), ("sin_t", ctypes.c_void_p), ("layers", ctypes.c_void_p),
        ("k_cache", ctypes.c_void_p), ("v_cache", ctypes.c_void_p),
    ]


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB):
            build()
        _lib = ctypes.CDLL(LIB)
        _lib.qf_forward.restype = ctypes.c_int
        _lib.qf_forward.argtypes = [ctypes.POINTER(_Model), ctypes.c_void_p, ctypes.c_int, ctypes.c_int,
                                    ctypes.c_int, ctypes.c_void_p, ctypes.c_int, ctypes.c_void_p,
                                    ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int]
        _lib.qf_tree_sum.restype = ctypes.c_float
        _lib.qf_tree_sum.argtypes = [ctypes.c_void_p, ctypes.c_int, ctypes.c_void_p, ctypes.c_int]
    return _lib


ORDERS = (0, 1, 2, 3)  # pairwise tree, left to right, eight interleaved sums, right to left


def tree_sum(x: torch.Tensor, order: int = 0) -> float:
    """The restatement's fp32 sum of ``x`` (1-D fp32) in summation order ``order``."""
    x = x.float().contiguous()
    p = 1 << max(0, (x.numel() - 1).bit_length())
    work = torch.empty(p, dtype=torch.float32)
    return float(lib().qf_tree_sum(x.data_ptr(), x.numel(), work.data_ptr(), order))


class Fp32Oracle:
    """Qwen3 decode on the CPU in fp32 with fixed-order sums.

    ``weights``: the reference's weights dict (qwen_megakernel/model.py:82-89), bf16 tensors on any
    device (kept as contiguous CPU copies).  ``cos``/``sin`` replace the dict's RoPE tables;
    ``num_layers`` runs only the first layers.
    """

    def __init__(self, weights: dict, shape, max_seq_len: int | None = None, num_layers: int | None = None,
                 cos: torch.Tensor | None = None, sin: torch.Tensor | None = None):
        cpu = torch.device("cpu")

        def c(t):
            return t.to(cpu).to(BF16).contiguous()

        self.shape = s = shape
        self.num_layers = s.num_layers if num_layers is None else num_layers
        self.embed = c(weights["embed_weight"])
        self.lm_head = c(weights["lm_head_weight"])
        self.final_norm = c(weights["final_norm_weight"])
        self.cos = c(weights["cos_table"] if cos is None else cos)
        self.sin = c(weights["sin_table"] if sin is None else sin)
        lw = weights["layer_weights"]
        if len(lw) < 11 * self.num_layers:
            raise ValueError("more layers than the weights hold")
        self.layer_w = [c(t) for t in lw[: 11 * self.num_layers]]
        self._ptrs = (ctypes.c_void_p * len(self.layer_w))(*[t.data_ptr() for t in self.layer_w])
        self.max_seq_len = self.cos.shape[0] if max_seq_len is None else max_seq_len
        if self.max_seq_len > self.cos.shape[0]:
            raise ValueError("max_seq_len exceeds the RoPE table length")
        self.k_cache = torch.zeros(self.num_layers, s.num_kv_heads, self.max_seq_len, s.head_dim, dtype=BF16)
        self.v_cache = torch.zeros_like(self.k_cache)
        self.position = 0
        self.scale = float(torch.tensor(1.0 / math.sqrt(s.head_dim), dtype=torch.float32))
        self.eps = float(torch.tensor(s.rms_eps, dtype=torch.float32))

    def _model(self) -> _Model:
        s = self.shape
        return _Model(self.num_layers, s.hidden, s.intermediate, s.num_q_heads, s.num_kv_heads, s.head_dim, s.vocab,
                      self.max_seq_len, self.eps, self.scale, self.embed.data_ptr(), self.lm_head.data_ptr(),
                      self.final_norm.data_ptr(), self.cos.data_ptr(), self.sin.data_ptr(),
                      ctypes.cast(self._ptrs, ctypes.c_void_p), self.k_cache.data_ptr(), self.v_cache.data_ptr())

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
    def forward(self, tokens, emit=None, given_cache: bool = False, order: int = 0) -> torch.Tensor:
        """Logits ``[len(emit), V]`` (fp32 holding bf16 values) of rows ``emit`` (default: all) after
        running ``tokens`` at consecutive positions from the current one.  ``given_cache``: the cache
        holds another decoder's rows for these positions and all before (as in
        :meth:`oracle.qwen3_exact.ExactOracle.hidden`); this oracle's own K/V rows are then kept in
        ``own_k`` / ``own_v`` and the cache is left as it is.  ``order``: the summation order of
        every sum (:data:`ORDERS`)."""
        s = self.shape
        toks = torch.tensor(list(tokens), dtype=torch.int32)
        t = toks.numel()
        p0 = self.position
        if t < 1 or p0 + t > self.max_seq_len:
            raise ValueError(f"positions {p0}..{p0 + t - 1} outside [0, {self.max_seq_len})")
        em = torch.arange(t, dtype=torch.int32) if emit is None else torch.as_tensor(emit, dtype=torch.int32)
        em = em.contiguous()
        logits = torch.empty(em.numel(), s.vocab, dtype=torch.float32)
        own_k = own_v = None
        if given_cache:
            own_k = torch.empty(self.num_layers, s.num_kv_heads, t, s.head_dim, dtype=BF16)
            own_v = torch.empty_like(own_k)
        m = self._model()
        rc = lib().qf_forward(ctypes.byref(m), toks.data_ptr(), t, p0, int(given_cache), em.data_ptr(), em.numel(),
                              logits.data_ptr(), own_k.data_ptr() if given_cache else None,
                              own_v.data_ptr() if given_cache else None, int(order))
        if rc != 0:
            raise ValueError("qf_forward rejected its arguments")
        if given_cache:
            self.own_k, self.own_v = own_k, own_v
        self.position = p0 + t
        return logits

    def step_logits(self, token_id: int) -> torch.Tensor:
        return self.forward([token_id])[0]
