"""The C ABI's host code under AddressSanitizer (tests/asan/).

tests/asan/Makefile builds a copy of libqwen_megakernel_amd whose host code is
compiled with -fsanitize=address (device code unchanged) and a driver
(tests/asan/qmk_asan_driver.cpp) that calls every entry point: argument checks
that fail before any GPU work, and with a GPU every host path with real
launches (decode, the reference-named launchers, generate in its three forms,
the allocation-free entry point, the batched step on the persistent kernel
with its device layer-table cache and on the multi-launch path, an in-place
batched call, the batched forward, the row sampler, tracing, a second stream,
the bounded-wait failure and its reset).  ASan stops the driver with a report
on any invalid host memory access; the driver exits non-zero when a call's
status is not the expected one.  Leak checking is off: the library keeps its
per-device and per-stream state until the process ends, by design.
"""

import os
import subprocess

import pytest

ASAN_DIR = os.path.join(os.path.dirname(os.path.abspath(__file__)), "asan")
DRIVER = os.path.join(ASAN_DIR, "_build", "qmk_asan_driver")
ENV = dict(os.environ, ASAN_OPTIONS="detect_leaks=0:halt_on_error=1")


def _run(timeout):
    assert os.path.exists(DRIVER), "tests/asan/_build/qmk_asan_driver is not built (__graft_entry__.build())"
    res = subprocess.run([DRIVER], env=ENV, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True,
                         timeout=timeout)
    print(res.stdout[-4000:])
    assert "ERROR: AddressSanitizer" not in res.stdout, res.stdout[-4000:]
    assert res.returncode == 0, res.stdout[-4000:]
    return res.stdout


def test_asan_host_argument_checks():
    """Without a GPU in view (HIP_VISIBLE_DEVICES empty): every argument check runs under ASan."""
    if not os.path.exists(DRIVER):
        subprocess.run(["make", "-s", "-C", ASAN_DIR], check=True)
    env = dict(ENV, HIP_VISIBLE_DEVICES="", ROCR_VISIBLE_DEVICES="")
    res = subprocess.run([DRIVER], env=env, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True, timeout=120)
    assert "ERROR: AddressSanitizer" not in res.stdout, res.stdout[-4000:]
    assert res.returncode == 0 and "0 failed checks" in res.stdout, res.stdout[-4000:]


@pytest.mark.gpu
def test_asan_host_paths_on_the_gpu():
    out = _run(timeout=240)
    assert "GPU paths: 0 failed checks" in out
