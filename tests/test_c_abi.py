"""CPU tests of the drop-in boundary (no GPU calls).

* libqwen_megakernel_amd.so loads and exports every function declared in
  include/qwen_megakernel.h.
* The C entry points validate their arguments on the host before touching the
  device. The reference validates nothing: csrc/torch_bindings.cpp has no
  TORCH_CHECK, and csrc/kernel.cu:344-356 indexes the tables and caches with the position it
  is given, never compared with max_seq_len.
* torch.ops.qwen_megakernel_C registers the reference's two schemas verbatim
  (reference csrc/torch_bindings.cpp:130-153).
"""

import ctypes
import math
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "qwen_megakernel.h")

REF_DECODE = ("decode(Tensor output_token, int input_token_id, Tensor embed_weight, Tensor layer_weights_packed, "
              "Tensor final_norm_weight, Tensor lm_head_weight, Tensor cos_table, Tensor sin_table, Tensor k_cache, "
              "Tensor v_cache, Tensor hidden_buffer, Tensor activations, Tensor residual, Tensor q, Tensor k, "
              "Tensor v, Tensor attn_out, Tensor mlp_intermediate, Tensor normalized, Tensor block_max_vals, "
              "Tensor block_max_idxs, int num_layers, int position, int max_seq_len, float attn_scale) -> ()")
REF_GENERATE = ("generate_nosync(int first_token_id, int num_steps, Tensor embed_weight, Tensor layer_weights_packed, "
                "Tensor final_norm_weight, Tensor lm_head_weight, Tensor cos_table, Tensor sin_table, "
                "Tensor k_cache, Tensor v_cache, Tensor hidden_buffer, Tensor activations, Tensor residual, "
                "Tensor q, Tensor k, Tensor v, Tensor attn_out, Tensor mlp_intermediate, Tensor normalized, "
                "Tensor block_max_vals, Tensor block_max_idxs, int num_layers, int start_position, "
                "int max_seq_len, float attn_scale) -> Tensor")


@pytest.fixture(scope="module")
def lib():
    from qwen_megakernel import build

    if not os.path.exists(build.LIB):
        build.build(force=False)
    return build.load_c_library()


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    names = re.findall(r"^\s*(?:const\s+)?[A-Za-z_][A-Za-z0-9_]*\s*\**\s*([A-Za-z_][A-Za-z0-9_]*)\s*\(", text, flags=re.M)
    return sorted(set(n for n in names if n not in ("if", "while", "return", "defined")))


def test_header_declares_reference_launchers():
    names = declared_functions()
    for n in ("launch_ldg_decode_direct", "launch_ldg_decode_persistent", "launch_ldg_generate_nosync"):
        assert n in names


def test_library_exports_every_declared_symbol(lib):
    missing = [n for n in declared_functions() if not hasattr(lib, n)]
    assert not missing, missing


QMK_OK, QMK_ERR_ARG, QMK_ERR_POSITION = 0, 1, 2
V = ctypes.c_void_p


def _decode_args(position=0, max_seq_len=16, null=False, num_layers=28, token=1, cache_len=None):
    p = V(0) if null else V(4096)
    args = [ctypes.c_int(token), V(4096)] + [p] * 19 + [ctypes.c_int(num_layers), ctypes.c_int(position)]
    if cache_len is not None:
        args.append(ctypes.c_int(cache_len))
    return args + [ctypes.c_int(max_seq_len), ctypes.c_float(0.088), V(0)]


def test_host_validation_rejects_bad_arguments_before_launch(lib):
    lib.qmk_status_string.restype = ctypes.c_char_p
    lib.launch_ldg_decode_direct(*_decode_args(null=True))
    assert lib.qmk_last_status() == QMK_ERR_ARG
    lib.launch_ldg_decode_direct(*_decode_args(position=16, max_seq_len=16))
    assert lib.qmk_last_status() == QMK_ERR_POSITION
    lib.launch_ldg_decode_direct(*_decode_args(position=-1))
    assert lib.qmk_last_status() == QMK_ERR_POSITION
    lib.launch_ldg_decode_direct(*_decode_args(num_layers=29))
    assert lib.qmk_last_status() == QMK_ERR_ARG
    lib.launch_ldg_decode_direct(*_decode_args(token=151936))
    assert lib.qmk_last_status() == QMK_ERR_ARG
    lib.launch_ldg_decode_direct(*_decode_args(max_seq_len=65537))  # 65536 is the largest
    assert lib.qmk_last_status() == QMK_ERR_ARG
    # persistent form: cache_len must be position + 1
    lib.launch_ldg_decode_persistent(*_decode_args(position=3, cache_len=7))
    assert lib.qmk_last_status() == QMK_ERR_ARG
    # a weight pointer that is not 16-byte aligned (the kernels read with 16-byte vector loads)
    args = _decode_args()
    args[2] = V(4096 + 2)  # embed
    lib.launch_ldg_decode_direct(*args)
    assert lib.qmk_last_status() == QMK_ERR_ARG
    assert b"position" in lib.qmk_status_string(QMK_ERR_POSITION)


def test_generate_validates_whole_range(lib):
    p = V(4096)
    base = [ctypes.c_int(5), ctypes.c_int(10)] + [p] * 19 + [V(4096), ctypes.c_int(28)]
    # 10 steps from position 8 need max_seq_len >= 18
    lib.launch_ldg_generate_nosync(*base, ctypes.c_int(8), ctypes.c_int(17), ctypes.c_float(0.088), V(0))
    assert lib.qmk_last_status() == QMK_ERR_POSITION
    # null output log
    args = [ctypes.c_int(5), ctypes.c_int(10)] + [p] * 19 + [V(0), ctypes.c_int(28), ctypes.c_int(0),
                                                             ctypes.c_int(64), ctypes.c_float(0.088), V(0)]
    lib.launch_ldg_generate_nosync(*args)
    assert lib.qmk_last_status() == QMK_ERR_ARG


def test_launch_geometry_fills_the_chip(lib):
    wg, th = ctypes.c_int(), ctypes.c_int()
    lib.qmk_launch_geometry(ctypes.byref(wg), ctypes.byref(th))
    assert wg.value == 256 and th.value % 64 == 0 and th.value <= 1024


def _norm_schema(s):
    return re.sub(r"\s+", " ", s.split("::", 1)[-1]).strip()


def test_torch_op_schemas_match_reference():
    from qwen_megakernel.build import get_extension

    ops = get_extension(build_if_missing=True)
    assert _norm_schema(str(ops.decode.default._schema)) == REF_DECODE
    assert _norm_schema(str(ops.generate_nosync.default._schema)) == REF_GENERATE


def test_package_exports_reference_names():
    import qwen_megakernel as q

    # the reference's three names, plus the batched decoder
    assert set(q.__all__) == {"load_weights", "Decoder", "generate", "BatchDecoder"}
    from qwen_megakernel import model

    assert (model.NUM_LAYERS, model.HIDDEN_SIZE, model.INTERMEDIATE_SIZE, model.VOCAB_SIZE) == (28, 1024, 3072, 151936)


def test_pack_layer_weights_layout():
    import struct

    import torch

    from qwen_megakernel.model import _pack_layer_weights

    ts = [torch.zeros(4) for _ in range(22)]
    blob = _pack_layer_weights(ts, num_layers=2)
    assert blob.dtype == torch.uint8 and blob.numel() == 2 * 11 * 8
    ptrs = struct.unpack("22Q", bytes(blob.tolist()))
    assert list(ptrs) == [t.data_ptr() for t in ts]


def test_algorithmic_bytes():
    """Bytes per token that the roofline divides by, summed tensor by tensor."""
    from qwen_megakernel.shapes import QWEN3_0_6B, layer_tensor_shapes

    s = QWEN3_0_6B
    layer = sum(2 * math.prod(shp) for shp in layer_tensor_shapes(s).values())
    assert layer == 31_461_888
    lm_head = 2 * s.vocab * s.hidden
    assert lm_head == 311_164_928
    assert s.weight_bytes_per_token() == 28 * layer + lm_head + 2 * s.hidden + 2 * s.hidden == 1_192_101_888
    assert s.kv_bytes_per_position() == 28 * 8 * 128 * 2 * 2 == 114_688
    assert s.bytes_per_token(1024) == 1_192_101_888 + 114_688 * 1025


class _LayerTable(ctypes.Structure):
    _fields_ = [(n, ctypes.c_void_p) for n in (
        "input_layernorm", "q_proj", "k_proj", "v_proj", "q_norm", "k_norm", "o_proj", "post_attn_layernorm",
        "gate_proj", "up_proj", "down_proj")]


def test_forward_workspace_bytes(lib):
    """Workspace grows with tokens and (for few tokens) with the context bound; invalid -> 0."""
    f = lib.qmk_forward_workspace_bytes
    f.restype = ctypes.c_size_t
    a = f(0, 4, 4, 512)
    b = f(0, 4, 4, 4096)
    c = f(1, 4, 4, 512)
    d = f(0, 128, 1, 128)
    assert 0 < a < b and a < c and d > 0
    assert f(0, 0, 1, 16) == 0 and f(0, 4, 0, 16) == 0 and f(0, 4, 257, 16) == 0 and f(2, 4, 4, 16) == 0
    # few tokens keep scores of max_context positions per (token, query head): 4 x 16 x 4096 fp32
    assert b - a >= 4 * 16 * (4096 - 512) * 4


def test_forward_tokens_host_validation(lib):
    """qmk_forward_tokens rejects bad arguments on the host, before any launch."""
    f = lib.qmk_forward_tokens
    f.restype = ctypes.c_int
    table = (_LayerTable * 2)()
    for t in table:
        for name, _ in _LayerTable._fields_:
            setattr(t, name, 4096)
    ws_bytes = lib.qmk_forward_workspace_bytes
    ws_bytes.restype = ctypes.c_size_t
    need = ws_bytes(0, 4, 4, 64)
    p = V(4096)

    def call(model=0, T=4, R=4, table_ptr=table, num_seqs=4, stride=2 * 8 * 64 * 128, layers=2, max_seq=64,
             max_ctx=64, ws=need, null_tokens=False, embed=p, k_cache=p):
        return f(ctypes.c_int(model), ctypes.c_int(T), V(0) if null_tokens else p, p, p, ctypes.c_int(R), p, p,
                 V(0), embed, table_ptr, p, p, p, p, k_cache, p, ctypes.c_int(num_seqs), ctypes.c_longlong(stride),
                 ctypes.c_int(layers), ctypes.c_int(max_seq), ctypes.c_int(max_ctx), ctypes.c_float(0.088), p,
                 ctypes.c_size_t(ws), V(0))

    assert call(model=3) == QMK_ERR_ARG
    assert call(null_tokens=True) == QMK_ERR_ARG
    assert call(max_ctx=65) == QMK_ERR_ARG            # context bound above the cache
    assert call(ws=need - 1) == QMK_ERR_ARG           # workspace too small
    assert call(stride=100) == QMK_ERR_ARG            # sequences would overlap
    assert call(R=257) == QMK_ERR_ARG
    assert call(layers=29) == QMK_ERR_ARG
    # the kernels read with 16-byte vector loads: every operand pointer 16-byte aligned, and the
    # per-sequence cache stride a multiple of 8 elements
    assert call(embed=V(4096 + 2)) == QMK_ERR_ARG
    assert call(k_cache=V(4096 + 8)) == QMK_ERR_ARG
    assert call(stride=2 * 8 * 64 * 128 + 4) == QMK_ERR_ARG
    table[0].q_norm = 4096 + 2
    assert call() == QMK_ERR_ARG
    table[0].q_norm = 4096
    table[1].o_proj = None
    assert call() == QMK_ERR_ARG                      # a null weight pointer in the host table


def test_generate_eos_validation(lib):
    """qmk_generate_eos rejects a negative stop token and out-of-range steps before any launch."""
    f = lib.qmk_generate_eos
    f.restype = ctypes.c_int
    p = V(4096)

    def call(eos=5, steps=10, start=0, max_seq=64):
        return f(ctypes.c_int(0), ctypes.c_int(1), ctypes.c_int(steps), ctypes.c_int(eos), p, p, p, p, p, p, p, p,
                 p, p, p, ctypes.c_int(28), ctypes.c_int(start), ctypes.c_int(max_seq), ctypes.c_float(0.088), V(0))

    assert call(eos=-1) == QMK_ERR_ARG
    assert call(eos=151936) == QMK_ERR_ARG
    assert call(start=60, steps=10) == QMK_ERR_POSITION


def test_reference_import_surface():
    """The reference's import names (qwen_megakernel/__init__.py:1-9, model.py, build.py, bench.py):
    importing the package registers torch.ops.qwen_megakernel_C, and the bench module has the
    reference's entry points and constants."""
    import torch

    import qwen_megakernel
    from qwen_megakernel import Decoder, generate, load_weights  # noqa: F401
    from qwen_megakernel.bench import (CHECK_TOKENS, PROMPT, RUNS, TOKENS, WARMUP, bench_megakernel,  # noqa: F401
                                       correctness_check, golden)
    from qwen_megakernel.build import get_extension
    from qwen_megakernel.model import Decoder as D2

    assert D2 is Decoder and qwen_megakernel.__all__[:3] == ["load_weights", "Decoder", "generate"]
    assert get_extension() is torch.ops.qwen_megakernel_C
    assert hasattr(torch.ops.qwen_megakernel_C, "decode") and hasattr(torch.ops.qwen_megakernel_C, "generate_nosync")
    assert (TOKENS, WARMUP, RUNS, PROMPT, CHECK_TOKENS) == (100, 3, 5, "Hello", 8)


def test_bench_golden_tokens_are_hf_fixture():
    """correctness_check's HF tokens are the HF fixture's (tests/golden/hf_qwen3_0p6b.npz)."""
    import numpy as np

    from qwen_megakernel.bench import golden
    from qwen_megakernel.shapes import QWEN3_0_6B
    from qwen_megakernel.weights import make_prompt

    g = golden()
    d = np.load(os.path.join(os.path.dirname(__file__), "golden", "hf_qwen3_0p6b.npz"))
    assert g["prompt"] == d["prompt"].tolist() == make_prompt(16, QWEN3_0_6B.vocab, seed=1)
    assert g["greedy_tokens"] == d["tokens"][15:].tolist()
    assert len(g["top_logits"]) == len(g["greedy_tokens"]) == 64
