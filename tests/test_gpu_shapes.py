"""GPU parity at the benchmark configurations' real matrix shapes.

Every distinct matrix of BASELINE configs[1]-[3] runs through air_hip_linear
with the AUTOMATIC planner at the configuration's own decode widths, and is
compared with the CPU oracle (ReferenceTensorReader::matvec,
src/reference/tensor_reader.cpp:369-394, plus the f32 bias add of
reference_executor.cpp:315-323) to relative L2 1e-4 per activation row:

* configs[1], Qwen2-0.5B Q8_0 at M = 1: q 896x896 (+bias), k / v 128x896
  (+bias), the engine's fused q|k|v 1152x896, o 896x896, gate / up
  4864x896, the fused gate|up 9728x896, down 896x4864, lm_head 151936x896;
* configs[2], Qwen2-7B Q8_0 at M = 1, 8, 32: fused q|k|v 4608x3584 (+bias),
  k / v 512x3584, o 3584x3584, fused gate|up 37888x3584, down 3584x18944,
  lm_head 152064x3584;
* configs[3], the same 7B matrices in Q4_0 and Q4_K at M = 1, 16, 64.

Shapes are written N x K (rows x input width) as in the configurations.
Matrices with N <= 4864 are checked on every output row; larger ones on a
seeded sample of 2048 rows plus the first and the last 16-row tile.  Each
case prints the kernel variant the planner chose (air_hip_linear_plan).
Weights w ~ N(0, 0.02) are quantized on the device (quant.synthetic_weights_
device) and copied to the host for the oracle; activations x ~ N(0, 1).
"""
from __future__ import annotations

import os

import numpy as np
import pytest

import oracle
from air_amd import capi, quant
from tests import helpers

pytestmark = pytest.mark.gpu

TOL = 1e-4
SAMPLE_ROWS = 2048
FULL_ROWS_UP_TO = 4864

# (label, N, K, bias)
QWEN2_05B = [("q", 896, 896, True), ("k|v", 128, 896, True), ("q|k|v", 1152, 896, True), ("o", 896, 896, False),
             ("gate|up part", 4864, 896, False), ("gate|up", 9728, 896, False), ("down", 896, 4864, False),
             ("lm_head", 151936, 896, False)]
QWEN2_7B = [("q|k|v", 4608, 3584, True), ("k|v", 512, 3584, True), ("o", 3584, 3584, False),
            ("gate|up", 37888, 3584, False), ("down", 3584, 18944, False), ("lm_head", 152064, 3584, False)]

CASES = ([("configs[1]", capi.TYPE_Q8_0, label, n, k, bias, (1,)) for label, n, k, bias in QWEN2_05B] +
         [("configs[2]", capi.TYPE_Q8_0, label, n, k, bias, (1, 8, 32)) for label, n, k, bias in QWEN2_7B] +
         [("configs[3]", t, label, n, k, bias, (1, 16, 64))
          for t in (capi.TYPE_Q4_0, capi.TYPE_Q4_K) for label, n, k, bias in QWEN2_7B])


def _rows_checked(n: int, seed: int) -> np.ndarray:
    if n <= FULL_ROWS_UP_TO:
        return np.arange(n, dtype=np.uint64)
    rng = np.random.default_rng(seed)
    sample = rng.choice(n, size=SAMPLE_ROWS, replace=False)
    edges = np.concatenate([np.arange(16), np.arange(n - 16, n)])
    return np.unique(np.concatenate([sample, edges])).astype(np.uint64)


@pytest.fixture(scope="module", autouse=True)
def _oracle_threads():
    before = oracle.threads()
    oracle.set_threads(min(16, os.cpu_count() or 1))
    yield
    oracle.set_threads(before)


@pytest.mark.parametrize("config,type_id,label,n,k,with_bias,ms", CASES,
                         ids=[f"{c[0]}-{capi.TYPE_NAMES[c[1]]}-{c[2]}-{c[3]}x{c[4]}" for c in CASES])
def test_real_shape_matches_oracle(torch_cuda, hip_ctx, config, type_id, label, n, k, with_bias, ms):
    torch = torch_cuda
    dev = torch.device("cuda:0")
    seed = 90_000 + 131 * n + k + type_id
    canon_dev = quant.synthetic_weights_device(type_id, k, n, seed, dev)
    canon = canon_dev.cpu().numpy()
    mat = capi.Matrix(hip_ctx, type_id, k, n, canon_dev, canon_dev.numel(), on_device=True)
    del canon_dev
    bias = (np.random.default_rng(seed + 1).standard_normal(n).astype(np.float32) * 0.02) if with_bias else None
    bias_d = torch.from_numpy(bias).to(dev) if with_bias else None
    rows = _rows_checked(n, seed + 2)
    try:
        for m in ms:
            plan = mat.plan(m)
            print(f"{config} {capi.TYPE_NAMES[type_id]} {label} {n}x{k} M={m}: {plan}", flush=True)
            x = helpers.activations(m, k, seed=seed + 10 * m)
            y = torch.full((m, n), float("nan"), dtype=torch.float32, device=dev)
            mat.linear(torch.from_numpy(x).to(dev), y, m, bias=bias_d)
            torch.cuda.synchronize()
            got_all = y.cpu().numpy()
            assert np.isfinite(got_all).all(), (config, label, m, plan)
            got = got_all[:, rows.astype(np.int64)]
            want = oracle.linear_row_list(type_id, canon, k, n, x, rows, bias=bias)
            for r in range(m):
                err = helpers.rel_l2(got[r], want[r])
                assert err <= TOL, (config, capi.TYPE_NAMES[type_id], label, m, r, err, plan)
    finally:
        mat.release()


@pytest.mark.parametrize("type_id", [capi.TYPE_Q8_0, capi.TYPE_Q4_0, capi.TYPE_Q4_K])
@pytest.mark.parametrize("ms", [(1, 8, 32), (16, 64)])
def test_outlier_channels_keep_precision(torch_cuda, hip_ctx, type_id, ms):
    """Activations with a few channels 1e3-1e4 times their row-mates (the
    residual-stream outliers of real Qwen2 models).  The outliers dominate
    the output, so relative L2 against the whole output would hide a loss
    of the small channels; the error is also held against the small
    channels' own share of the output (the oracle on x with the outlier
    channels zeroed): 1e-3 of it, a bound set by the f32 rounding of
    outputs ~400x larger than that share.  A kernel whose power-of-two
    scales flushed the small channels would miss it by orders of
    magnitude."""
    torch = torch_cuda
    dev = torch.device("cuda:0")
    k, n = 3584, 4608
    seed = 4242 + type_id
    canon_dev = quant.synthetic_weights_device(type_id, k, n, seed, dev)
    canon = canon_dev.cpu().numpy()
    mat = capi.Matrix(hip_ctx, type_id, k, n, canon_dev, canon_dev.numel(), on_device=True)
    del canon_dev
    rows = np.arange(n, dtype=np.uint64)
    try:
        for m in ms:
            rng = np.random.default_rng(seed + m)
            x = rng.standard_normal((m, k), dtype=np.float32)
            channels = rng.choice(k, size=6, replace=False)
            x[:, channels] *= np.float32([1e3, -2e3, 5e3, 1e4, -8e3, 3e3])
            y = torch.empty((m, n), dtype=torch.float32, device=dev)
            mat.linear(torch.from_numpy(x).to(dev), y, m)
            torch.cuda.synchronize()
            got = y.cpu().numpy().astype(np.float64)
            want = oracle.linear_row_list(type_id, canon, k, n, x, rows).astype(np.float64)
            x_small = x.copy()
            x_small[:, channels] = 0.0
            small = oracle.linear_row_list(type_id, canon, k, n, x_small, rows).astype(np.float64)
            plan = mat.plan(m)
            print(f"outliers {capi.TYPE_NAMES[type_id]} M={m}: {plan}", flush=True)
            for r in range(m):
                err = np.linalg.norm(got[r] - want[r])
                assert err <= TOL * np.linalg.norm(want[r]), (m, r, plan)
                assert err <= 1e-3 * np.linalg.norm(small[r]), (m, r, err / np.linalg.norm(small[r]), plan)
    finally:
        mat.release()
