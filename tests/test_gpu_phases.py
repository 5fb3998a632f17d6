"""Per-phase microbenchmark kernels: outputs of the last weight copy against a torch fp32 reference."""

import pytest
import torch

pytestmark = pytest.mark.gpu


def _setup(pid, n=2, seed=3):
    from qwen_megakernel.build import get_extension
    from qwen_megakernel.phases import make_inputs, phases, run

    get_extension()
    ph = phases()[pid]
    w, act, norm = make_inputs(ph, n, seed=seed)
    out = run(ph, w, act, norm, n)
    torch.cuda.synchronize()
    last = w[(n - 1) * ph.weight_elems: n * ph.weight_elems]
    return ph, last, act, norm, out


def _bf16_close(got, ref, ulps=2):
    """|got - ref| within `ulps` bf16 ulps of |ref| (+ a tiny absolute floor)."""
    got, ref = got.float(), ref.float()
    tol = ulps * torch.clamp(ref.abs(), min=1e-3) * 2.0 ** -8
    bad = (got - ref).abs() > tol
    assert not bad.any(), f"{int(bad.sum())} mismatches, worst {((got - ref).abs() - tol).max().item()}"


def test_phase_qkv_rmsnorm():
    from oracle.qwen3_ref import rms_norm

    ph, w, act, norm, out = _setup(0)
    x = rms_norm(act.cpu().view(1, 1, -1), norm.cpu(), 1e-6).view(-1).cuda()
    ref = w.view(4096, 1024).float() @ x.float()
    _bf16_close(out, ref)


@pytest.mark.parametrize("pid,k,seg", [(1, 2048, 256), (3, 3072, 384)])
def test_phase_column_split_partials(pid, k, seg):
    ph, w, act, norm, out = _setup(pid)
    W = w.view(1024, k).float()
    ref = torch.stack([W[:, seg * x: seg * (x + 1)] @ act[seg * x: seg * (x + 1)].float() for x in range(8)])
    assert torch.allclose(out, ref, rtol=1e-4, atol=1e-4), (out - ref).abs().max().item()
    # the eight partials add up to the full product
    assert torch.allclose(out.sum(0), W @ act.float(), rtol=1e-4, atol=1e-3)


def test_phase_gate_up_silu_mul():
    ph, w, act, norm, out = _setup(2)
    W = w.view(2, 3072, 1024).float()
    g = (W[0] @ act.float()).to(torch.bfloat16).float()
    u = (W[1] @ act.float()).to(torch.bfloat16).float()
    ref = (torch.nn.functional.silu(g).to(torch.bfloat16).float() * u).to(torch.bfloat16)
    _bf16_close(out, ref, ulps=4)


def test_phase_lm_head_argmax():
    from qwen_megakernel.phases import argmax_from_keys

    ph, w, act, norm, out = _setup(4)
    logits = (w.view(151936, 1024).float() @ act.float()).to(torch.bfloat16).float()
    row = argmax_from_keys(out)
    top = logits.max().item()
    assert 0 <= row < 151936
    # the chosen row holds the maximum logit (to within one bf16 ulp of summation-order noise)
    assert logits[row].item() >= top - abs(top) * 2.0 ** -7, (row, logits[row].item(), top)
