"""GPU unit tests of the decode kernel's arithmetic building blocks.

Runs libqwen_megakernel_amd.so's qmk_selftest_blocks (one wave of the same
device functions the decode kernel uses) through the C ABI and checks:

* bf16 rounding equals torch's round-to-nearest-even on normals, exact ties,
  subnormals, +-0 and +-inf;
* the softmax exp is within 2 ulp of float64 exp and exactly 0 at -inf;
* the permlane row/half swaps and the four-row sum move lanes as documented.
"""

import ctypes

import pytest
import torch

pytestmark = pytest.mark.gpu


def _run(x):
    from qwen_megakernel.build import load_c_library

    lib = load_c_library()
    n = x.numel()
    out = torch.zeros(2 * n + 320, dtype=torch.float32, device="cuda")
    xs = x.cuda().contiguous()
    rc = lib.qmk_selftest_blocks(ctypes.c_void_p(xs.data_ptr()), ctypes.c_void_p(out.data_ptr()), ctypes.c_int(n),
                                 ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
    assert rc == 0
    torch.cuda.synchronize()
    return out.cpu()


def _inputs():
    g = torch.Generator().manual_seed(3)
    parts = [
        torch.randn(4096, generator=g) * 3,
        torch.randn(1024, generator=g) * 1e-3,
        torch.randn(512, generator=g) * 1e30,
        # exact bf16 ties: low 16 bits 0x8000, halfway between adjacent bf16 values
        ((torch.randint(0x0080, 0x7f00, (512,), generator=g, dtype=torch.int32) << 16) | 0x8000).view(torch.float32),
        ((torch.randint(0x8080, 0xff00, (512,), generator=g, dtype=torch.int64) << 16) | 0x8000).to(torch.int64)
        .bitwise_and(0xffffffff).to(torch.int32).view(torch.float32),
        torch.tensor([0.0, -0.0, float("inf"), float("-inf"), 1e-40, -1e-40, 1.17549435e-38, 3.4e38, -3.4e38]),
    ]
    x = torch.cat(parts)
    pad = (-x.numel()) % 64
    return torch.cat([x, torch.zeros(pad)])


def test_bf16_rounding_matches_torch():
    x = _inputs()
    out = _run(x)
    got = out[: x.numel()]
    exp = x.to(torch.bfloat16).float()
    assert torch.equal(got, exp), (got - exp).abs().max()


def test_softmax_exp_accuracy():
    g = torch.Generator().manual_seed(4)
    x = torch.cat([-torch.rand(8192, generator=g) * 60, torch.tensor([0.0, -1e-7, -87.0, -100.0, -float("inf")])])
    pad = (-x.numel()) % 64
    x = torch.cat([x, torch.zeros(pad)])
    out = _run(x)
    n = x.numel()
    got = out[n: 2 * n].double()
    ref = torch.exp(x.double())
    finite = ref > 1e-37  # above the fp32 subnormal range
    ulp = torch.abs(torch.nextafter(ref[finite].float(), torch.tensor(float("inf"))).double() - ref[finite])
    assert ((got[finite] - ref[finite]).abs() <= 2 * ulp).all()
    assert got[n - pad - 1] == 0.0  # exp(-inf)
    assert got[~finite].abs().max() < 1e-37


def test_lane_swaps_and_row_sum():
    x = torch.arange(64, dtype=torch.float32) * 3 + 1
    x = torch.cat([x, torch.zeros(64)])
    out = _run(x)
    base = 2 * x.numel()
    v = x[:64]
    rows = v.view(4, 16)
    rsum = (rows[0] + rows[1]) + (rows[2] + rows[3])
    assert torch.equal(out[base: base + 64], rsum.repeat(4))
    lane = torch.arange(64)
    row = lane // 16
    even_row = v[(row - row % 2) * 16 + lane % 16]
    odd_row = v[(row - row % 2 + 1) * 16 + lane % 16]
    assert torch.equal(out[base + 64: base + 128], even_row)
    assert torch.equal(out[base + 128: base + 192], odd_row)
    assert torch.equal(out[base + 192: base + 256], v[lane % 32])
    assert torch.equal(out[base + 256: base + 320], v[lane % 32 + 32])
