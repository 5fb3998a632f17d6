"""GPU tests of the text path around the decode kernel: the stop token on the
device (generate_eos), HIP-graph replay of the device-fed loop, and tokenizer
injection.

Graph replays are compared with direct launches of the same kernel on the same
inputs: the tokens must be identical, on several replays in a row with eager
work (single steps, resets) in between.
"""

import pytest
import torch

from parity import decoder as _decoder

pytestmark = pytest.mark.gpu


def _ops():
    from qwen_megakernel.build import get_extension

    return get_extension()


def _stream(dec, prompt, n, graphs=True):
    _ops().set_graph_launch(graphs)
    try:
        return dec.generate(prompt, n)
    finally:
        _ops().set_graph_launch(True)


def test_graph_replay_matches_direct_launches(weights_gpu, prompt):
    """100 steps = 3 replays of the 32-step graph + 4 direct launches, three times over with eager
    steps and resets in between; always the tokens of 100 direct launches."""
    dec = _decoder(weights_gpu)
    ref = _stream(dec, prompt, 100, graphs=False)
    for rep in range(3):
        got = _stream(dec, prompt, 100, graphs=True)
        assert got == ref, f"replay round {rep}: first difference at {next(i for i in range(100) if got[i] != ref[i])}"
        assert dec.position == len(prompt) - 1 + 100
        dec.reset()
        dec.step(prompt[0])  # eager work between the graph replays
        dec.reset()


def test_graph_recorded_again_for_new_arguments(weights_gpu, prompt):
    """A second decoder (other caches) on the same stream gets its own recording, not the first's."""
    a = _decoder(weights_gpu)
    b = _decoder(weights_gpu)
    ra = _stream(a, prompt, 64)
    rb = _stream(b, prompt, 64)
    assert ra == rb
    # a's cache holds the stream; b's too: both advanced by their own launches
    assert torch.equal(a._k_cache[:, :, : len(prompt) + 63], b._k_cache[:, :, : len(prompt) + 63])


@pytest.mark.parametrize("graphs", [True, False], ids=["graph", "direct"])
def test_eos_stops_on_device(weights_gpu, prompt, graphs):
    """generate with a stop token: the stream up to and including it, then stop-token padding; the
    position advances by the generated tokens only, and decoding continues from there."""
    n = 70
    free = _stream(_decoder(weights_gpu), prompt, n, graphs=graphs)
    k = 40
    eos = free[k]
    k = free.index(eos)  # first occurrence
    dec = _decoder(weights_gpu)
    _ops().set_graph_launch(graphs)
    try:
        out = dec.generate_ids(list(prompt), n, eos_token_id=eos)
    finally:
        _ops().set_graph_launch(True)
    assert out[: k + 1] == free[: k + 1]
    assert out[k + 1:] == [eos] * (n - k - 1)
    start = len(prompt) - 1
    assert dec.position == start + k + 1
    # the stopped run left cache and position as k + 1 plain steps do: the next step agrees
    ref = _decoder(weights_gpu, use_prefill=True)
    ref.generate_ids(list(prompt), k + 1)
    assert ref.position == dec.position
    assert dec.step(eos) == ref.step(eos)
    assert int(_ops().device_error()) == 0


def test_eos_at_first_step(weights_gpu, prompt):
    free = _decoder(weights_gpu).generate(prompt, 4)
    dec = _decoder(weights_gpu)
    out = dec.generate_ids(list(prompt), 40, eos_token_id=free[0])
    assert out == [free[0]] * 40 and dec.position == len(prompt)


class _CharTokenizer:
    """A stand-in tokenizer (no files offline): one id per character, id 0 = EOS."""

    eos_token_id = 0

    def encode(self, text, add_special_tokens=True):
        return [1 + (ord(c) % 1000) for c in text]

    def decode(self, ids, skip_special_tokens=True):
        return "".join(chr(32 + (i % 90)) for i in ids if not (skip_special_tokens and i == 0))


def test_text_generate_with_injected_tokenizer(weights_gpu):
    """Decoder(tokenizer=...) encodes the prompt, stops at the tokenizer's EOS on the device and decodes
    the tokens before it (the reference's text generate, qwen_megakernel/model.py:207-245)."""
    tok = _CharTokenizer()
    dec = _decoder(weights_gpu)
    dec.tokenizer = tok
    text = dec.generate("Hello, MI355X", max_tokens=24)
    ids = _decoder(weights_gpu).generate(tok.encode("Hello, MI355X"), 24)
    assert isinstance(text, str)
    assert text == tok.decode(ids[: ids.index(0)] if 0 in ids else ids)
