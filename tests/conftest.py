import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built HIP library")
    config.addinivalue_line("markers", "slow: takes more than a few seconds on the CPU")


def pytest_collection_modifyitems(config, items):
    try:
        import torch
        have_gpu = torch.cuda.is_available()
    except Exception:  # pragma: no cover
        have_gpu = False
    if have_gpu:
        return
    skip = pytest.mark.skip(reason="no GPU in this environment")
    for item in items:
        if "gpu" in item.keywords:
            item.add_marker(skip)


# ------------------------------------------------------------------ shared GPU-test fixtures
# Session-scoped so that the Qwen3-0.6B weights (1.2 GB), their GPU copy and the
# exact oracle's float64 copy (4.8 GB) are built once per test run.

@pytest.fixture(scope="session")
def shape():
    from qwen_megakernel.shapes import QWEN3_0_6B

    return QWEN3_0_6B


@pytest.fixture(scope="session")
def weights_cpu(shape):
    import torch

    from qwen_megakernel.weights import make_weights

    torch.set_num_threads(min(16, len(os.sched_getaffinity(0))))
    return make_weights(shape, seed=0, max_seq_len=2048)


@pytest.fixture(scope="session")
def weights_gpu(weights_cpu):
    from qwen_megakernel.weights import to_device

    return to_device(weights_cpu, "cuda")


@pytest.fixture(scope="session")
def exact06(shape, weights_cpu):
    from oracle.qwen3_exact import ExactWeights

    return ExactWeights(weights_cpu, shape)


@pytest.fixture(scope="session")
def prompt(shape):
    from qwen_megakernel.weights import make_prompt

    return make_prompt(16, shape.vocab, seed=1)
