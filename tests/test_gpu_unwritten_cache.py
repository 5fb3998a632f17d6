"""GPU tests: cache rows that no token has written never reach the output.

The C ABI does not require zeroed K/V caches.  Every attention form reads
whole blocks of positions and gives the positions past the context a zero
weight; a NaN in such a row must still not reach the sum (0 * NaN is NaN).
Each test runs the same work twice on fresh caches, one zero-filled and one
NaN-filled, and requires bit-identical tokens and logits, all finite.
"""

import contextlib
from dataclasses import replace

import pytest
import torch

from parity import decoder, kernel_stream, with_rope

pytestmark = pytest.mark.gpu

NAN = float("nan")


def _poison(*caches, start=0):
    """Fill positions start.. (dimension -2) of each cache with NaN."""
    for c in caches:
        c[..., start:, :].fill_(NAN)


def _same(what, a, b):
    ta, la = a
    tb, lb = b
    assert ta == tb, f"{what}: tokens {ta} != {tb}"
    assert bool(torch.isfinite(la).all()), f"{what}: non-finite logits on the zeroed cache"
    assert torch.equal(la, lb), f"{what}: logits differ (max abs {(la - lb).abs().nan_to_num(1e9).max().item()})"


@pytest.mark.parametrize("c0", [0, 1500, 2100, 12300], ids=["from-0", "1500", "2100", "12300"])
def test_decode_ignores_unwritten_rows(shape, weights_gpu, prompt, c0):
    """Batch-1 decode, 4 layers: from position 0 (the short form), and after an injected cache of
    c0 positions (split over an XCD's workgroups at 1500, the long-context kernel at 2100, the deep
    form at 12300); every row from the context onwards is NaN on the second decoder."""
    from qwen_megakernel.weights import make_kv_prefill

    layers = 4
    max_seq = max(2048, c0 + 64)
    w = with_rope(weights_gpu, max_seq, "cuda") if max_seq > 2048 else weights_gpu
    kv = make_kv_prefill(replace(shape, num_layers=layers), c0, seed=2) if c0 else None
    runs = []
    for poison in (False, True):
        dec = decoder(w, num_layers=layers, max_seq_len=max_seq)
        if kv is not None:
            dec.load_kv(kv[0].cuda(), kv[1].cuda(), c0)
        if poison:
            _poison(dec._k_cache, dec._v_cache, start=c0)
        feed = prompt[:5] if c0 == 0 else [11, 22]
        _, toks, lgs = kernel_stream(dec, feed, 4)
        runs.append((toks, lgs))
    _same(f"decode from context {c0}", *runs)


@pytest.mark.parametrize("first,n", [(0, 100), (0, 333), (400, 150)], ids=["rows-100", "mfma-333", "mfma-chunks-150"])
def test_prefill_ignores_unwritten_rows(shape, weights_gpu, first, n):
    """The batched forward of n tokens after `first` prefilled ones (100 from position 0: the row
    attention; 333: the MFMA attention, whose last 64-position tile is ragged; 150 after 400: the
    MFMA attention with its keys in chunks), then a second prompt of 21 tokens and two decode
    steps, on a NaN-filled cache."""
    from qwen_megakernel.weights import make_prompt

    ids = make_prompt(n, shape.vocab, seed=31)
    more = make_prompt(21, shape.vocab, seed=32)
    runs = []
    for poison in (False, True):
        dec = decoder(weights_gpu, num_layers=4)
        if poison:
            _poison(dec._k_cache, dec._v_cache)
        if first:
            dec.prefill(make_prompt(first, shape.vocab, seed=30))
        t0, l0 = dec.prefill(ids, return_logits=True)
        t1, l1 = dec.prefill(more, return_logits=True)
        t2, l2 = dec.step_logits(t1)
        t3, l3 = dec.step_logits(t2)
        runs.append(([t0, t1, t2, t3], torch.stack([l0, l1, l2, l3]).cpu()))
    _same(f"prefill {first} + {n} + 21 + 2 steps", *runs)


@contextlib.contextmanager
def _persistent(on: bool):
    ops = torch.ops.qwen_megakernel_C
    was = ops.set_batch_persistent(on)
    try:
        yield
    finally:
        ops.set_batch_persistent(was)


@pytest.mark.parametrize("persistent", [True, False], ids=["persistent", "multi-launch"])
def test_batch_ignores_unwritten_rows(shape, weights_gpu, persistent):
    """Three sequences with ragged prompts (37, 70 and 333 tokens) prefilled together, then three
    batched steps on the persistent kernel or the multi-launch step; every cache row of every
    sequence past its context is NaN on the second run."""
    from qwen_megakernel.model import BatchDecoder
    from qwen_megakernel.weights import make_prompt

    prompts = [make_prompt(n, shape.vocab, seed=40 + i) for i, n in enumerate([37, 70, 333])]
    runs = []
    for poison in (False, True):
        bd = BatchDecoder(weights=weights_gpu, batch_size=3, max_seq_len=512, num_layers=4, verbose=False)
        if poison:
            _poison(bd._k_cache, bd._v_cache)
        toks, lg = bd.prefill_all(prompts, return_logits=True)
        out, lgs = list(toks), [lg.cpu()]
        with _persistent(persistent):
            for _ in range(3):
                toks, lg = bd.step_logits(toks)
                out += toks
                lgs.append(lg.cpu())
        runs.append((out, torch.cat(lgs)))
    _same(f"batch of 3, {'persistent' if persistent else 'multi-launch'}", *runs)
