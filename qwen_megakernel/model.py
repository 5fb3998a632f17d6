"""Weight loading and the high-level decode API for Qwen3-0.6B on MI355X.

Mirrors the reference's qwen_megakernel/model.py: the same constants, the same
weights dict, the same packed 11-pointer layer table, the same ``Decoder``
(``step``, ``reset``, ``position``, ``generate``) and module-level
``generate``, calling ``torch.ops.qwen_megakernel_C.decode`` /
``generate_nosync`` with the reference's argument lists.

Differences, all additive:

* ``load_weights`` has no network.  ``model_name`` may name a local directory
  holding a Qwen3 checkpoint (``*.safetensors`` + tokenizer files); anything
  else yields the seeded synthetic weights of :mod:`qwen_megakernel.weights`
  and no tokenizer.
* RoPE theta is 1e6 (Qwen3), not the reference's 10000 (model.py:54-56).
* ``max_seq_len`` is a parameter (the reference fixes 2048).
* ``Decoder`` also serves Qwen3-1.7B weights (hidden 2048, MLP 6144); the
  model is recognised from the embedding's width.
* ``Decoder.step`` raises on a device failure instead of returning a stale token;
  positions are range-checked.
* ``Decoder.step_logits`` returns the logits as well, ``Decoder.load_kv`` injects
  cache contents, and ``generate`` accepts token-id lists when there is no tokenizer.
* ``Decoder.prefill`` runs a whole prompt through the batched MFMA forward
  (``torch.ops.qwen_megakernel_C.forward_tokens``) in one pass; ``generate``
  uses it for the prompt instead of one decode step per prompt token
  (``use_prefill=False`` restores the reference's per-token feeding).
* ``BatchDecoder`` decodes several independent sequences together, one batched
  forward per step.
"""

from __future__ import annotations

import glob
import math
import os
import struct

import torch

from .shapes import QWEN3_0_6B, QWEN3_1_7B
from . import weights as _w

NUM_LAYERS = 28
NUM_KV_HEADS = 8
HEAD_DIM = 128
HIDDEN_SIZE = 1024
INTERMEDIATE_SIZE = 3072
Q_SIZE = 16 * HEAD_DIM  # 2048
KV_SIZE = 8 * HEAD_DIM  # 1024
MAX_SEQ_LEN = 2048
VOCAB_SIZE = 151936


def _ops():
    from .build import get_extension

    return get_extension()


def load_weights(model_name: str = "Qwen/Qwen3-0.6B", verbose: bool = True, *, max_seq_len: int = MAX_SEQ_LEN,
                 seed: int = 0, device: str = "cuda", shape=None):
    """Return ``(weights, tokenizer)`` in the reference's dict layout (model.py:21-94).

    A local directory with ``*.safetensors`` is loaded as a real checkpoint (its
    ``config.json`` ``hidden_size`` picks Qwen3-0.6B or -1.7B unless ``shape`` is
    given); otherwise the seeded synthetic weights of ``shape`` (default
    Qwen3-0.6B) are drawn and there is no tokenizer.
    """
    if os.path.isdir(model_name) and glob.glob(os.path.join(model_name, "*.safetensors")):
        from safetensors.torch import load_file

        state = {}
        for f in sorted(glob.glob(os.path.join(model_name, "*.safetensors"))):
            state.update(load_file(f))
        if shape is None:
            hidden = state["model.embed_tokens.weight"].shape[-1]
            cfg_path = os.path.join(model_name, "config.json")
            if os.path.exists(cfg_path):
                import json

                with open(cfg_path) as fh:
                    hidden = json.load(fh).get("hidden_size", hidden)
            shape = {QWEN3_0_6B.hidden: QWEN3_0_6B, QWEN3_1_7B.hidden: QWEN3_1_7B}.get(hidden)
            if shape is None:
                raise ValueError(f"{model_name}: hidden size {hidden} is neither Qwen3-0.6B nor Qwen3-1.7B")
        if verbose:
            print(f"Loading {model_name} (local safetensors, {shape.name})...")
        weights = _w.load_weights_from_state_dict(state, shape, max_seq_len=max_seq_len, device=device)
        tokenizer = None
        try:
            from transformers import AutoTokenizer

            tokenizer = AutoTokenizer.from_pretrained(model_name)
        except Exception:
            tokenizer = None
        return weights, tokenizer
    shape = QWEN3_0_6B if shape is None else shape
    if verbose:
        print(f"{model_name}: no local checkpoint; using seeded synthetic {shape.name} weights (seed {seed})")
    return _w.make_weights(shape, seed=seed, max_seq_len=max_seq_len, device=device), None


def _pack_layer_weights(layer_weights: list[torch.Tensor], num_layers: int = NUM_LAYERS) -> torch.Tensor:
    """Device blob of ``num_layers`` 11-pointer tables (model.py:97-108)."""
    n_ptrs = 11
    buf = bytearray(num_layers * n_ptrs * 8)
    for i in range(num_layers):
        for j in range(n_ptrs):
            struct.pack_into("Q", buf, (i * n_ptrs + j) * 8, layer_weights[i * n_ptrs + j].data_ptr())
    return torch.frombuffer(buf, dtype=torch.uint8).to(layer_weights[0].device)


def _as_i32(values, device) -> torch.Tensor:
    return torch.tensor([int(v) for v in values], dtype=torch.int32, device=device)


class _Forward:
    """Calls ``forward_tokens`` with one model's weights; caches workspaces by size."""

    def __init__(self, ops, weights: dict, num_layers: int):
        self._ops = ops
        self.embed = weights["embed_weight"]
        self.layers = list(weights["layer_weights"][: 11 * num_layers])
        self.final_norm = weights["final_norm_weight"]
        self.lm_head = weights["lm_head_weight"]
        self.cos = weights["cos_table"]
        self.sin = weights["sin_table"]
        self.num_layers = num_layers
        self.hidden = self.embed.shape[-1]
        self.scale = 1.0 / math.sqrt(HEAD_DIM)
        self._ws = torch.empty(0, dtype=torch.uint8, device=self.embed.device)

    def workspace(self, num_tokens: int, num_emit: int, max_context: int) -> torch.Tensor:
        need = int(self._ops.forward_workspace_bytes(self.hidden, num_tokens, num_emit, max_context))
        if self._ws.numel() < need:
            self._ws = torch.empty(need, dtype=torch.uint8, device=self.embed.device)
        return self._ws

    def decode(self, tokens, positions, out_tokens, logits, k_cache, v_cache, max_context: int):
        """One batched decode step (``decode_batch`` op): token b of sequence b at positions[b]."""
        need = int(self._ops.decode_batch_workspace_bytes(self.hidden, tokens.numel(), max_context))
        if self._ws.numel() < need:
            self._ws = torch.empty(need, dtype=torch.uint8, device=self.embed.device)
        self._ops.decode_batch(tokens, positions, out_tokens, logits, self.embed, self.layers, self.final_norm,
                               self.lm_head, self.cos, self.sin, k_cache, v_cache, self._ws, self.num_layers,
                               max_context, self.scale)

    def __call__(self, tokens, seq_ids, positions, emit_rows, out_tokens, logits, k_cache, v_cache,
                 max_context: int):
        ws = self.workspace(tokens.numel(), emit_rows.numel(), max_context)
        self._ops.forward_tokens(tokens, seq_ids, positions, emit_rows, out_tokens, logits, self.embed, self.layers,
                                 self.final_norm, self.lm_head, self.cos, self.sin, k_cache, v_cache, ws,
                                 self.num_layers, max_context, self.scale)


class Decoder:
    """Stateful decoder over torch.ops.qwen_megakernel_C (model.py:111-245)."""

    def __init__(self, weights=None, tokenizer=None, model_name: str = "Qwen/Qwen3-0.6B", verbose: bool = True,
                 max_seq_len: int = MAX_SEQ_LEN, num_layers: int = NUM_LAYERS, use_prefill: bool = True):
        self._ops = _ops()
        self.use_prefill = use_prefill
        if weights is None:
            weights, tokenizer = load_weights(model_name, verbose=verbose, max_seq_len=max_seq_len)
        weights = _w.to_device(weights, "cuda")
        if not 1 <= num_layers <= NUM_LAYERS or len(weights["layer_weights"]) < 11 * num_layers:
            raise ValueError(f"num_layers={num_layers} does not match the weights")
        if weights["cos_table"].shape[0] < max_seq_len:
            raise ValueError("RoPE tables are shorter than max_seq_len")
        hidden = weights["embed_weight"].shape[-1]
        shapes = {QWEN3_0_6B.hidden: QWEN3_0_6B, QWEN3_1_7B.hidden: QWEN3_1_7B}
        if hidden not in shapes:
            raise ValueError(f"embed_weight width {hidden}: expected 1024 (Qwen3-0.6B) or 2048 (Qwen3-1.7B)")
        self.shape = shapes[hidden]
        self.tokenizer = tokenizer
        self._position = 0
        self._num_layers = num_layers
        self._max_seq_len = max_seq_len
        self._weights = weights  # keeps the storage the packed pointers refer to alive
        self._embed_weight = weights["embed_weight"]
        self._final_norm_weight = weights["final_norm_weight"]
        self._lm_head_weight = weights["lm_head_weight"]
        self._cos_table = weights["cos_table"]
        self._sin_table = weights["sin_table"]
        self._layer_weights_packed = _pack_layer_weights(weights["layer_weights"], num_layers)
        self._attn_scale = 1.0 / math.sqrt(HEAD_DIM)
        dev = self._embed_weight.device
        self._k_cache = torch.zeros(num_layers, NUM_KV_HEADS, max_seq_len, HEAD_DIM, dtype=torch.bfloat16, device=dev)
        self._v_cache = torch.zeros_like(self._k_cache)
        f32 = dict(dtype=torch.float32, device=dev)
        bf16 = dict(dtype=torch.bfloat16, device=dev)
        h, inter = self.shape.hidden, self.shape.intermediate
        self._hidden = torch.empty(h, **bf16)
        self._act = torch.empty(h, **f32)
        self._res = torch.empty(h, **f32)
        self._q = torch.empty(Q_SIZE, **f32)
        self._k = torch.empty(KV_SIZE, **f32)
        self._v = torch.empty(KV_SIZE, **f32)
        self._attn_out = torch.empty(Q_SIZE, **f32)
        self._mlp_inter = torch.empty(inter, **f32)
        self._norm_out = torch.empty(h, **f32)
        self._bmax_vals = torch.empty(4096, **f32)
        self._bmax_idxs = torch.empty(4096, dtype=torch.int32, device=dev)
        self._out_token = torch.empty(1, dtype=torch.int32, device=dev)
        self._logits = torch.empty(VOCAB_SIZE, **f32)
        self._forward = _Forward(self._ops, weights, num_layers)

    # -- reference API --------------------------------------------------

    def _check_position(self, n: int = 1):
        if self._position + n > self._max_seq_len:
            raise ValueError(f"position {self._position} + {n} exceeds max_seq_len {self._max_seq_len}")

    def _scratch(self):
        return (self._embed_weight, self._layer_weights_packed, self._final_norm_weight, self._lm_head_weight,
                self._cos_table, self._sin_table, self._k_cache, self._v_cache, self._hidden, self._act,
                self._res, self._q, self._k, self._v, self._attn_out, self._mlp_inter, self._norm_out,
                self._bmax_vals, self._bmax_idxs)

    def _raise_device_error(self):
        err = int(self._ops.device_error())
        raise RuntimeError(f"decode failed on the device (error bits 0x{err:x}); call reset()")

    def step(self, token_id: int) -> int:
        """Decode one token. Returns the next token id."""
        self._check_position()
        self._ops.decode(self._out_token, int(token_id), *self._scratch(), self._num_layers, self._position,
                         self._max_seq_len, self._attn_scale)
        self._position += 1
        tok = int(self._out_token.item())
        if tok < 0:
            self._raise_device_error()
        return tok

    def reset(self):
        self._position = 0
        self._k_cache.zero_()
        self._v_cache.zero_()
        self._ops.reset()

    @property
    def position(self) -> int:
        return self._position

    def generate(self, prompt, max_tokens: int = 100, temperature: float = 0.0, top_k: int = 0, top_p: float = 1.0,
                 seed: int = 0):
        """Continuation of ``prompt`` (text with a tokenizer, or a list of ids): greedy, or sampled when
        ``temperature > 0`` (HF's temperature / top-k / top-p, one Gumbel-max draw per step on the GPU)."""
        self.reset()
        if isinstance(prompt, str):
            if self.tokenizer is None:
                raise ValueError("text prompts need a tokenizer; pass a list of token ids")
            ids = self.tokenizer.encode(prompt, add_special_tokens=True)
        else:
            ids = [int(t) for t in prompt]
        samp = dict(temperature=temperature, top_k=top_k, top_p=top_p, seed=seed)
        if not isinstance(prompt, str):
            return self.generate_ids(ids, max_tokens, **samp)
        eos = self.tokenizer.eos_token_id
        out = self.generate_ids(ids, max_tokens, eos_token_id=eos, **samp)
        if eos in out:
            out = out[: out.index(eos)]
        return self.tokenizer.decode(out, skip_special_tokens=True)

    # -- additions --------------------------------------------------------

    def generate_ids(self, ids: list[int], max_tokens: int, eos_token_id: int | None = None,
                     temperature: float = 0.0, top_k: int = 0, top_p: float = 1.0, seed: int = 0) -> list[int]:
        """Step ``ids[:-1]``, then ``max_tokens`` device-fed steps from ``ids[-1]``: greedy, or with
        ``temperature > 0`` sampled (the draw of the step at position p uses counter p).

        With ``eos_token_id`` the device stops after emitting it: the rest of the
        returned list is ``eos_token_id`` padding and the position advances only by
        the tokens actually generated.
        """
        if not ids:
            raise ValueError("empty prompt")
        if self.use_prefill and len(ids) > 1:
            self.prefill(ids[:-1])
        else:
            for tid in ids[:-1]:
                self.step(tid)
        self._check_position(max_tokens)
        if temperature > 0:
            eos = -1 if eos_token_id is None else int(eos_token_id)
            out = self._ops.generate_sample(int(ids[-1]), int(max_tokens), eos, float(temperature), int(top_k),
                                            float(top_p), int(seed), self._embed_weight,
                                            self._layer_weights_packed, self._final_norm_weight,
                                            self._lm_head_weight, self._cos_table, self._sin_table, self._k_cache,
                                            self._v_cache, self._hidden, self._norm_out, self._num_layers,
                                            self._position, self._max_seq_len, self._attn_scale).cpu().tolist()
            self._position += out.index(eos) + 1 if eos >= 0 and eos in out else max_tokens
            return out
        if eos_token_id is None:
            out = self._ops.generate_nosync(int(ids[-1]), int(max_tokens), *self._scratch(), self._num_layers,
                                            self._position, self._max_seq_len, self._attn_scale)
            self._position += max_tokens
            return out.cpu().tolist()
        out = self._ops.generate_eos(int(ids[-1]), int(max_tokens), int(eos_token_id), self._embed_weight,
                                     self._layer_weights_packed, self._final_norm_weight, self._lm_head_weight,
                                     self._cos_table, self._sin_table, self._k_cache, self._v_cache, self._hidden,
                                     self._norm_out, self._num_layers, self._position, self._max_seq_len,
                                     self._attn_scale).cpu().tolist()
        eos = int(eos_token_id)
        self._position += out.index(eos) + 1 if eos in out else max_tokens
        return out

    def step_logits(self, token_id: int):
        """Decode one token; returns ``(next_token, logits)`` with fp32 logits (bf16 values)."""
        self._check_position()
        self._ops.decode_logits(self._out_token, self._logits, int(token_id), self._embed_weight,
                                self._layer_weights_packed, self._final_norm_weight, self._lm_head_weight,
                                self._cos_table, self._sin_table, self._k_cache, self._v_cache, self._hidden,
                                self._norm_out, self._num_layers, self._position, self._max_seq_len,
                                self._attn_scale)
        self._position += 1
        tok = int(self._out_token.item())
        if tok < 0:
            self._raise_device_error()
        return tok, self._logits.clone()

    def prefill(self, ids, return_logits: bool = False):
        """Run ``ids`` at positions ``position .. position+len-1`` in one batched forward.

        Writes their K/V into the cache exactly as that many ``step`` calls
        would, and returns the greedy token after the last one (with its fp32
        logits when ``return_logits``).
        """
        ids = [int(t) for t in ids]
        if not ids:
            raise ValueError("empty prompt")
        if any(not 0 <= t < VOCAB_SIZE for t in ids):
            raise ValueError("token id outside the vocabulary")
        n = len(ids)
        self._check_position(n)
        dev = self._embed_weight.device
        start = self._position
        tokens = _as_i32(ids, dev)
        positions = torch.arange(start, start + n, dtype=torch.int32, device=dev)
        seqs = torch.zeros(n, dtype=torch.int32, device=dev)
        emit = _as_i32([n - 1], dev)
        out = torch.empty(1, dtype=torch.int32, device=dev)
        logits = torch.empty(1, VOCAB_SIZE, dtype=torch.float32, device=dev) if return_logits else None
        self._forward(tokens, seqs, positions, emit, out, logits, self._k_cache, self._v_cache, start + n)
        self._position += n
        tok = int(out.item())
        if tok < 0:
            raise RuntimeError("prefill produced no token (invalid input)")
        return (tok, logits[0].clone()) if return_logits else tok

    def load_kv(self, k: torch.Tensor, v: torch.Tensor, cache_len: int):
        """Inject cache contents for positions ``[0, cache_len)``; decoding continues at ``cache_len``."""
        if cache_len > self._max_seq_len:
            raise ValueError("cache_len exceeds max_seq_len")
        self._k_cache[:, :, :cache_len].copy_(k[: self._num_layers, :, :cache_len])
        self._v_cache[:, :, :cache_len].copy_(v[: self._num_layers, :, :cache_len])
        self._position = cache_len


class BatchDecoder:
    """Greedy (or sampled) decoding of ``batch_size`` independent sequences together.

    Each step is one batched decode step (``decode_batch``) over one token per
    sequence, so one read of the weights serves the whole batch; prompts are
    prefilled with ``forward_tokens``.  Sequence b
    keeps its own K/V cache (``[B, L, 8, S, 128]``) and position.  Not in the
    reference, which decodes one sequence.
    """

    def __init__(self, weights=None, batch_size: int = 4, tokenizer=None, model_name: str = "Qwen/Qwen3-0.6B",
                 verbose: bool = True, max_seq_len: int = MAX_SEQ_LEN, num_layers: int = NUM_LAYERS):
        self._ops = _ops()
        if weights is None:
            weights, tokenizer = load_weights(model_name, verbose=verbose, max_seq_len=max_seq_len)
        weights = _w.to_device(weights, "cuda")
        if not 1 <= num_layers <= NUM_LAYERS or len(weights["layer_weights"]) < 11 * num_layers:
            raise ValueError(f"num_layers={num_layers} does not match the weights")
        if weights["cos_table"].shape[0] < max_seq_len:
            raise ValueError("RoPE tables are shorter than max_seq_len")
        if not 1 <= batch_size <= 256:
            raise ValueError("batch_size must be in [1, 256]")
        self.tokenizer = tokenizer
        self.batch_size = batch_size
        self._weights = weights
        self._num_layers = num_layers
        self._max_seq_len = max_seq_len
        self._forward = _Forward(self._ops, weights, num_layers)
        dev = weights["embed_weight"].device
        self._dev = dev
        self._k_cache = torch.zeros(batch_size, num_layers, NUM_KV_HEADS, max_seq_len, HEAD_DIM,
                                    dtype=torch.bfloat16, device=dev)
        self._v_cache = torch.zeros_like(self._k_cache)
        self._positions = [0] * batch_size
        self._all = torch.arange(batch_size, dtype=torch.int32, device=dev)

    @property
    def positions(self) -> list[int]:
        return list(self._positions)

    def reset(self):
        self._positions = [0] * self.batch_size
        self._k_cache.zero_()
        self._v_cache.zero_()

    def _check(self, seq: int, n: int):
        if not 0 <= seq < self.batch_size:
            raise ValueError(f"sequence {seq} outside [0, {self.batch_size})")
        if self._positions[seq] + n > self._max_seq_len:
            raise ValueError(f"sequence {seq}: position {self._positions[seq]} + {n} exceeds max_seq_len")

    def load_kv(self, seq: int, k: torch.Tensor, v: torch.Tensor, cache_len: int):
        """Inject ``[L, 8, >=cache_len, 128]`` cache contents into sequence ``seq``; it continues at ``cache_len``."""
        self._check(seq, 0)
        if cache_len > self._max_seq_len:
            raise ValueError("cache_len exceeds max_seq_len")
        self._k_cache[seq, :, :, :cache_len].copy_(k[: self._num_layers, :, :cache_len])
        self._v_cache[seq, :, :, :cache_len].copy_(v[: self._num_layers, :, :cache_len])
        self._positions[seq] = cache_len

    def prefill(self, seq: int, ids, return_logits: bool = False):
        """Append ``ids`` to sequence ``seq`` in one forward; returns the next greedy token."""
        ids = [int(t) for t in ids]
        if not ids or any(not 0 <= t < VOCAB_SIZE for t in ids):
            raise ValueError("empty prompt or token id outside the vocabulary")
        n = len(ids)
        self._check(seq, n)
        start = self._positions[seq]
        tokens = _as_i32(ids, self._dev)
        positions = torch.arange(start, start + n, dtype=torch.int32, device=self._dev)
        seqs = torch.full((n,), seq, dtype=torch.int32, device=self._dev)
        out = torch.empty(1, dtype=torch.int32, device=self._dev)
        logits = torch.empty(1, VOCAB_SIZE, dtype=torch.float32, device=self._dev) if return_logits else None
        self._forward(tokens, seqs, positions, _as_i32([n - 1], self._dev), out, logits, self._k_cache,
                      self._v_cache, start + n)
        self._positions[seq] += n
        tok = int(out.item())
        if tok < 0:
            raise RuntimeError("prefill produced no token (invalid input)")
        return (tok, logits[0].clone()) if return_logits else tok

    def prefill_all(self, prompts, return_logits: bool = False):
        """Append ``prompts[b]`` to sequence b for every b in one forward (the prompts' tokens
        concatenated, each with its sequence and position); returns each sequence's next greedy
        token, and with ``return_logits`` also the fp32 logits ``[B, V]`` of its last prompt token.
        One pass reads the weights once for all the prompts, instead of once per sequence."""
        if len(prompts) != self.batch_size:
            raise ValueError(f"expected {self.batch_size} prompts")
        prompts = [[int(t) for t in ids] for ids in prompts]
        if any(not ids or any(not 0 <= t < VOCAB_SIZE for t in ids) for ids in prompts):
            raise ValueError("empty prompt or token id outside the vocabulary")
        for b, ids in enumerate(prompts):
            self._check(b, len(ids))
        toks, seqs, pos, emit = [], [], [], []
        for b, ids in enumerate(prompts):
            start = self._positions[b]
            toks += ids
            seqs += [b] * len(ids)
            pos += range(start, start + len(ids))
            emit.append(len(toks) - 1)
        max_context = max(self._positions[b] + len(ids) for b, ids in enumerate(prompts))
        out = torch.empty(self.batch_size, dtype=torch.int32, device=self._dev)
        logits = (torch.empty(self.batch_size, VOCAB_SIZE, dtype=torch.float32, device=self._dev)
                  if return_logits else None)
        self._forward(_as_i32(toks, self._dev), _as_i32(seqs, self._dev), _as_i32(pos, self._dev),
                      _as_i32(emit, self._dev), out, logits, self._k_cache, self._v_cache, max_context)
        for b, ids in enumerate(prompts):
            self._positions[b] += len(ids)
        res = out.cpu().tolist()
        if any(t < 0 for t in res):
            raise RuntimeError("prefill produced no token (invalid input)")
        return (res, logits) if return_logits else res

    def step_logits(self, tokens):
        """One token per sequence at its current position; returns (next tokens, fp32 logits [B, V])."""
        tokens = [int(t) for t in tokens]
        if len(tokens) != self.batch_size:
            raise ValueError(f"expected {self.batch_size} tokens")
        for b in range(self.batch_size):
            self._check(b, 1)
        out = torch.empty(self.batch_size, dtype=torch.int32, device=self._dev)
        logits = torch.empty(self.batch_size, VOCAB_SIZE, dtype=torch.float32, device=self._dev)
        self._forward.decode(_as_i32(tokens, self._dev), _as_i32(self._positions, self._dev), out, logits,
                             self._k_cache, self._v_cache, max(self._positions) + 1)
        self._positions = [p + 1 for p in self._positions]
        res = out.cpu().tolist()
        if any(t < 0 for t in res):
            raise RuntimeError("batched step produced no token (invalid input)")
        return res, logits

    def step(self, tokens) -> list[int]:
        return self.step_logits(tokens)[0]

    def _counters(self, positions: torch.Tensor) -> torch.Tensor:
        """Per-row random-number counters: position + (sequence << 32) (sequence 0: the position, as the
        single-sequence sampled loop uses)."""
        return positions.to(torch.int64) + (self._all.to(torch.int64) << 32)

    def decode_steps(self, tokens: torch.Tensor, steps: int, temperature: float = 0.0, top_k: int = 0,
                     top_p: float = 1.0, seed: int = 0) -> torch.Tensor:
        """``steps`` batched steps from device tokens (one per sequence, at the current positions),
        each step's outputs fed to the next on the device; no host synchronisation.  Greedy, or with
        ``temperature > 0`` sampled from each step's logits (``sample`` op).  Returns the device log
        ``[steps + 1, B]`` whose row 0 is ``tokens`` and row i the tokens after step i."""
        if tokens.numel() != self.batch_size:
            raise ValueError(f"expected {self.batch_size} tokens")
        for b in range(self.batch_size):
            self._check(b, steps)
        log = torch.empty(steps + 1, self.batch_size, dtype=torch.int32, device=self._dev)
        log[0] = tokens.to(device=self._dev, dtype=torch.int32)
        if steps:
            start = torch.tensor(self._positions, dtype=torch.int32, device=self._dev)
            pos_table = start[None, :] + torch.arange(steps, dtype=torch.int32, device=self._dev)[:, None]
            max_context = max(self._positions) + steps
            sampled = temperature > 0
            if sampled:
                logits = torch.empty(self.batch_size, VOCAB_SIZE, dtype=torch.float32, device=self._dev)
                greedy = torch.empty(self.batch_size, dtype=torch.int32, device=self._dev)
            for i in range(steps):
                if not sampled:
                    self._forward.decode(log[i], pos_table[i], log[i + 1], None, self._k_cache, self._v_cache,
                                         max_context)
                    continue
                self._forward.decode(log[i], pos_table[i], greedy, logits, self._k_cache, self._v_cache,
                                     max_context)
                self._ops.sample(logits, float(temperature), int(top_k), float(top_p), int(seed),
                                 self._counters(pos_table[i]), log[i + 1])
            self._positions = [p + steps for p in self._positions]
        return log

    def generate_ids(self, prompts, max_tokens: int, temperature: float = 0.0, top_k: int = 0, top_p: float = 1.0,
                     seed: int = 0) -> list[list[int]]:
        """Continuations (``max_tokens`` each) of one prompt per sequence, greedy or sampled.

        The prompts are prefilled together in one forward, then the batch is
        stepped with the tokens fed back on the device: no host synchronisation
        until the end.
        """
        if len(prompts) != self.batch_size:
            raise ValueError(f"expected {self.batch_size} prompts")
        if max_tokens < 1:
            return [[] for _ in prompts]
        self.reset()
        for b, ids in enumerate(prompts):
            self._check(b, len(ids) + max_tokens - 1)
        if temperature > 0:
            first_t = torch.empty(self.batch_size, dtype=torch.int32, device=self._dev)
            _, lg = self.prefill_all(prompts, return_logits=True)
            # counter of the draw after each prompt: its last position + (sequence << 32)
            last = torch.tensor([p - 1 for p in self._positions], dtype=torch.int32, device=self._dev)
            self._ops.sample(lg, float(temperature), int(top_k), float(top_p), int(seed), self._counters(last),
                             first_t)
        else:
            first_t = _as_i32(self.prefill_all(prompts), self._dev)
        log = self.decode_steps(first_t, max_tokens - 1, temperature, top_k, top_p, seed)
        out = log.t().cpu().tolist()
        if any(t < 0 for row in out for t in row):
            raise RuntimeError("batched generation produced an invalid token")
        return out


def generate(prompt, max_tokens: int = 100, verbose: bool = True):
    """One-shot convenience: load weights, generate, return text (or ids)."""
    return Decoder(verbose=verbose).generate(prompt, max_tokens)
