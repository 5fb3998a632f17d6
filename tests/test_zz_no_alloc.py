"""The allocation-free decode entry point against the entry point it is a variant of.

qmk_decode_model_noalloc (include/qwen_megakernel.h) runs the same decode
kernel as qmk_decode_model with its device state and exchange words in a
file-scope device array instead of per-stream buffers.  Called through the C
ABI twice in a row -- a 28-layer step after a 16-token prompt, then a smaller
input (4 layers, a 3-token cache, a shorter max_seq_len) -- it must give the
existing entry point's token, logits and K/V cache rows bit for bit (the same
kernel on the same inputs), and the device's free memory must not change.
"""

import ctypes
import math

import pytest
import torch

from parity import decoder

pytestmark = pytest.mark.gpu


def _lib():
    from qwen_megakernel.build import load_c_library

    lib = load_c_library()
    lib.qmk_status_string.restype = ctypes.c_char_p
    return lib


def _call(fn, dec, tok, out, logits, num_layers, position, stream):
    vp = ctypes.c_void_p
    return fn(ctypes.c_int(0), ctypes.c_int(tok), vp(out.data_ptr()), vp(logits.data_ptr()),
              vp(dec._embed_weight.data_ptr()), vp(dec._layer_weights_packed.data_ptr()),
              vp(dec._final_norm_weight.data_ptr()), vp(dec._lm_head_weight.data_ptr()),
              vp(dec._cos_table.data_ptr()), vp(dec._sin_table.data_ptr()), vp(dec._k_cache.data_ptr()),
              vp(dec._v_cache.data_ptr()), vp(dec._hidden.data_ptr()), vp(dec._norm_out.data_ptr()),
              ctypes.c_int(num_layers), ctypes.c_int(position), ctypes.c_int(dec._max_seq_len),
              ctypes.c_float(1.0 / math.sqrt(128)), vp(stream.cuda_stream))


def test_noalloc_matches_decode_model_on_two_calls(weights_gpu, prompt):
    lib = _lib()
    assert lib.qmk_init() == 0, lib.qmk_status_string(lib.qmk_last_status())
    stream = torch.cuda.current_stream()
    cases = [(28, 2048, prompt, 9), (4, 64, prompt[:3], 77)]  # (layers, max_seq_len, cache tokens, input token)
    free_before = None
    for i, (layers, max_seq, ctx_ids, tok) in enumerate(cases):
        a = decoder(weights_gpu, num_layers=layers, max_seq_len=max_seq)
        b = decoder(weights_gpu, num_layers=layers, max_seq_len=max_seq)
        for d in (a, b):
            d.prefill(ctx_ids)
        torch.cuda.synchronize()
        pos = len(ctx_ids)
        outs = [torch.full((1,), -7, dtype=torch.int32, device="cuda") for _ in range(2)]
        lgs = [torch.zeros(151936, dtype=torch.float32, device="cuda") for _ in range(2)]
        assert _call(lib.qmk_decode_model, a, tok, outs[0], lgs[0], layers, pos, stream) == 0
        torch.cuda.synchronize()
        if i == 1:
            free_before = torch.cuda.mem_get_info()[0]
        st = _call(lib.qmk_decode_model_noalloc, b, tok, outs[1], lgs[1], layers, pos, stream)
        assert st == 0, lib.qmk_status_string(st)
        torch.cuda.synchronize()
        if i == 1:
            assert torch.cuda.mem_get_info()[0] == free_before, "the allocation-free call changed free memory"
        ta, tb = int(outs[0].item()), int(outs[1].item())
        assert ta >= 0 and ta == tb, (i, ta, tb)
        assert torch.equal(lgs[0], lgs[1]), f"call {i}: logits differ by {(lgs[0] - lgs[1]).abs().max().item()}"
        assert torch.equal(a._k_cache, b._k_cache) and torch.equal(a._v_cache, b._v_cache), f"call {i}: caches differ"


def test_noalloc_rejects_sizes_beyond_its_limits(weights_gpu):
    lib = _lib()
    assert lib.qmk_init() == 0
    dec = decoder(weights_gpu, max_seq_len=64)
    out = torch.empty(1, dtype=torch.int32, device="cuda")
    lg = torch.empty(151936, dtype=torch.float32, device="cuda")
    st = _call(lib.qmk_decode_model_noalloc, dec, 5, out, lg, 29, 0, torch.cuda.current_stream())
    assert st == 7 and b"limits" in lib.qmk_status_string(st)


def test_noalloc_failure_is_read_without_allocating_and_the_next_call_recovers(weights_gpu, prompt):
    """A call whose waits are bounded to one tick fails on the device: it leaves -1 in the output
    token and error bits in the scratch array, which qmk_noalloc_device_error reads without
    allocating.  The next call, with the default bound, starts clean and gives qmk_decode_model's
    token, logits and cache bit for bit."""
    lib = _lib()
    lib.qmk_noalloc_device_error.restype = ctypes.c_uint32
    lib.qmk_noalloc_device_error.argtypes = [ctypes.c_void_p]
    lib.qmk_noalloc_set_wait_limit.argtypes = [ctypes.c_uint32]
    assert lib.qmk_init() == 0
    stream = torch.cuda.current_stream()
    layers, max_seq, ctx_ids, tok = 4, 64, prompt[:3], 21
    a = decoder(weights_gpu, num_layers=layers, max_seq_len=max_seq)
    b = decoder(weights_gpu, num_layers=layers, max_seq_len=max_seq)
    for d in (a, b):
        d.prefill(ctx_ids)
    torch.cuda.synchronize()
    pos = len(ctx_ids)
    outs = [torch.full((1,), -7, dtype=torch.int32, device="cuda") for _ in range(2)]
    lgs = [torch.zeros(151936, dtype=torch.float32, device="cuda") for _ in range(2)]
    assert _call(lib.qmk_decode_model, a, tok, outs[0], lgs[0], layers, pos, stream) == 0
    torch.cuda.synchronize()
    free_before = torch.cuda.mem_get_info()[0]
    try:
        assert lib.qmk_noalloc_set_wait_limit(1) == 0
        assert _call(lib.qmk_decode_model_noalloc, b, tok, outs[1], lgs[1], layers, pos, stream) == 0
        err = lib.qmk_noalloc_device_error(ctypes.c_void_p(stream.cuda_stream))
        assert err not in (0, 0xFFFFFFFF), hex(err)
        assert int(outs[1].item()) == -1
    finally:
        assert lib.qmk_noalloc_set_wait_limit(0) == 0
    outs[1].fill_(-7)
    assert _call(lib.qmk_decode_model_noalloc, b, tok, outs[1], lgs[1], layers, pos, stream) == 0
    assert lib.qmk_noalloc_device_error(ctypes.c_void_p(stream.cuda_stream)) == 0
    assert torch.cuda.mem_get_info()[0] == free_before, "the allocation-free calls changed free memory"
    ta, tb = int(outs[0].item()), int(outs[1].item())
    assert ta >= 0 and ta == tb, (ta, tb)
    assert torch.equal(lgs[0], lgs[1]), f"logits differ by {(lgs[0] - lgs[1]).abs().max().item()}"
    assert torch.equal(a._k_cache, b._k_cache) and torch.equal(a._v_cache, b._v_cache), "caches differ"
