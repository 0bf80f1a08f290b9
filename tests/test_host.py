"""Runs the C++ host tests (tests/host/host_tests.cpp).

cpu: plan vocabulary/validation, CapacityScheduler, MicrobatchScheduler,
     model and Qwen2 contract checks, f16 conversion and quantizers -- the
     cases of AIR's tests/scheduler_tests.cpp:77-348 and
     tests/core_tests.cpp:389-481.
gpu: HipPreparedModel residency and every projection of synthetic Q8_0,
     Q4_0 and Q4_K Qwen2 models against the CPU oracle.
"""
import os
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
BINARY = os.path.join(ROOT, "tests", "host", "host_tests")


def _run(mode, timeout):
    proc = subprocess.run([BINARY, mode], capture_output=True, text=True, timeout=timeout)
    print(proc.stdout[-4000:])
    assert proc.returncode == 0, proc.stderr[-4000:]
    assert f"host {mode} tests passed" in proc.stdout


def test_host_cpu():
    # The binary is cheap to (re)build with g++; the GPU box runs the prebuilt one.
    for d in ("air_amd/csrc", "air_amd/host", "tests/host"):
        subprocess.run(["make", "-s", "-C", os.path.join(ROOT, d)], check=True, capture_output=True)
    _run("cpu", 60)


@pytest.mark.gpu
def test_host_gpu():
    assert os.path.exists(BINARY), "tests/host/host_tests is not built"
    _run("gpu", 110)


@pytest.mark.gpu
def test_host_gpu_qwen2_7b_width():
    """configs[4]'s geometry (two layers at the full Qwen2-7B width) through
    prefill_batch at 512 rows on the MFMA tactic and graph-replayed decode at
    widths 4, 2 and 1, teacher-forced against the C oracle (logits and
    margin-certified top-1 per decision)."""
    assert os.path.exists(BINARY), "tests/host/host_tests is not built"
    _run("gpu7b", 280)


@pytest.mark.gpu
def test_host_gpu_qwen2_7b_decode_widths_64_32():
    """configs[4]'s decode widths at the Qwen2-7B width (two layers): 64
    sequences of 8-token prompts in one 512-row prefill_batch step, then
    graph-replayed decode at width 64 and width 32 and device greedy at
    width 32, teacher-forced against the C oracle (logits and
    margin-certified top-1 per decision), after an MFMA and an exact
    prefill."""
    assert os.path.exists(BINARY), "tests/host/host_tests is not built"
    _run("gpu7b-wide", 280)
