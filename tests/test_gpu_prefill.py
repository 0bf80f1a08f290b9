"""GPU parity of the prefill tactic (f16 MFMA GEMM) against the CPU oracle.

The prefill tactic rounds activations and dequantized weights to f16 and
accumulates in f32, so it is held to relative L2 1e-2 of the double
accumulating matvec (tensor_reader.cpp:369-394) plus the f32 bias add
(reference_executor.cpp:315-323); the observed error is about 3e-4, and the
tests also check that it stays below 2e-3 so a lost term cannot hide in the
tolerance.  Shapes cover ragged N (not whole 16-row tiles), K that is not a
whole 64/128/256-k tile, M that is not a whole activation tile, every
compiled launch shape and K splits.
"""
from __future__ import annotations

import numpy as np
import pytest

import oracle
from air_amd import capi, quant
from tests import helpers

pytestmark = pytest.mark.gpu

PREFILL_TOL = 1e-2      # gate for the MFMA path
PREFILL_EXPECT = 2e-3   # what f16 rounding of both operands leaves (~3e-4)


def _dev(torch, a):
    return torch.from_numpy(np.ascontiguousarray(a)).to("cuda:0")


def _run(torch, mat, x, n, m, bias=None, tactic=capi.LINEAR_PREFILL):
    y = torch.full((m, n), float("nan"), dtype=torch.float32, device="cuda:0")
    mat.linear(_dev(torch, x), y, m, bias=None if bias is None else _dev(torch, bias), tactic=tactic)
    torch.cuda.synchronize()
    return y.cpu().numpy()


CASES = [
    (capi.TYPE_Q8_0, 896, 4864, 65),     # config-0 shape
    (capi.TYPE_Q8_0, 96, 37, 100),       # ragged N, K = 1.5 tiles
    (capi.TYPE_Q8_0, 3584, 512, 257),    # M one past a 256-row multiple
    (capi.TYPE_Q4_0, 160, 45, 70),       # K = 1.25 tiles
    (capi.TYPE_Q4_0, 896, 640, 128),
    (capi.TYPE_Q4_K, 256, 19, 66),
    (capi.TYPE_Q4_K, 768, 200, 129),
]


@pytest.mark.parametrize("type_id,k,n,m", CASES)
@pytest.mark.parametrize("with_bias", [False, True])
def test_prefill_matches_oracle(torch_cuda, hip_ctx, type_id, k, n, m, with_bias):
    torch = torch_cuda
    canon = helpers.weights(type_id, k, n, seed=3 * k + n + type_id)
    mat = capi.Matrix(hip_ctx, type_id, k, n, canon, canon.nbytes, on_device=False)
    x = helpers.activations(m, k, seed=k + m)
    bias = np.random.default_rng(n).standard_normal(n).astype(np.float32) * 0.02 if with_bias else None
    want = oracle.linear(type_id, canon, k, n, x, bias=bias)
    got = _run(torch, mat, x, n, m, bias)
    assert np.isfinite(got).all()
    err = helpers.rel_l2(got, want)
    print(f"prefill type={type_id} k={k} n={n} m={m} bias={with_bias} rel_l2={err:.3e}")
    assert err <= PREFILL_TOL
    assert err <= PREFILL_EXPECT
    # every row on its own, so a dropped row cannot hide in the total
    for r in range(m):
        assert helpers.rel_l2(got[r], want[r]) <= PREFILL_TOL, r
    mat.release()


@pytest.mark.parametrize("type_id,k,n", [
    (capi.TYPE_Q8_0, 1024, 400), (capi.TYPE_Q4_0, 1024, 333), (capi.TYPE_Q4_K, 1280, 272)])
def test_prefill_launch_shapes_agree(torch_cuda, hip_ctx, type_id, k, n):
    """Every compiled tile shape and K split gives the oracle's answer; a
    fixed shape is bit-reproducible."""
    torch = torch_cuda
    m = 150
    canon = helpers.weights(type_id, k, n, seed=k * 5 + n)
    mat = capi.Matrix(hip_ctx, type_id, k, n, canon, canon.nbytes, on_device=False)
    x = helpers.activations(m, k, seed=77)
    bias = np.linspace(-1, 1, n, dtype=np.float32)
    want = oracle.linear(type_id, canon, k, n, x, bias=bias)
    try:
        for tm, tn, pf in ((4, 2, 2), (4, 4, 2), (8, 2, 2), (8, 4, 1), (8, 4, 2)):
                for splits in (1, 2, 3, 5):
                    hip_ctx.set_prefill_tuning(tm, tn, splits, pf)
                    got = _run(torch, mat, x, n, m, bias)
                    err = helpers.rel_l2(got, want)
                    assert err <= PREFILL_EXPECT, (tm, tn, pf, splits, err)
                    again = _run(torch, mat, x, n, m, bias)
                    assert helpers.same_bits(got, again), (tm, tn, pf, splits)
    finally:
        hip_ctx.set_prefill_tuning(0, 0, 0, 0)
    mat.release()


def test_prefill_scale_extremes(torch_cuda, hip_ctx):
    """Per-row activation scaling and the per-matrix weight exponent keep f16
    in range: huge and tiny activations, huge and tiny weights."""
    torch = torch_cuda
    k, n, m = 512, 96, 72
    x = helpers.activations(m, k, seed=5)
    x *= np.logspace(-8, 8, m, dtype=np.float32)[:, None]     # 1e-8 .. 1e8 per row
    for wscale in (1e-3, 1.0, 4e3):
        w = np.random.default_rng(9).standard_normal((n, k)).astype(np.float32) * 0.02 * wscale
        for type_id in (capi.TYPE_Q8_0, capi.TYPE_Q4_0, capi.TYPE_Q4_K):
            canon = quant.quantize(type_id, w).reshape(-1)
            mat = capi.Matrix(hip_ctx, type_id, k, n, canon, canon.nbytes, on_device=False)
            want = oracle.linear(type_id, canon, k, n, x)
            got = _run(torch, mat, x, n, m)
            assert np.isfinite(got).all(), (type_id, wscale)
            for r in range(m):
                assert helpers.rel_l2(got[r], want[r]) <= PREFILL_EXPECT, (type_id, wscale, r)
            mat.release()


def test_auto_routes_by_width(torch_cuda, hip_ctx):
    """AUTO takes the decode tactic up to 64 rows and the prefill GEMM above."""
    torch = torch_cuda
    k, n = 512, 128
    canon = helpers.weights(capi.TYPE_Q8_0, k, n, seed=2)
    mat = capi.Matrix(hip_ctx, capi.TYPE_Q8_0, k, n, canon, canon.nbytes, on_device=False)
    before = hip_ctx.stats()
    _run(torch, mat, helpers.activations(64, k, 1), n, 64, tactic=capi.LINEAR_AUTO)
    mid = hip_ctx.stats()
    _run(torch, mat, helpers.activations(65, k, 1), n, 65, tactic=capi.LINEAR_AUTO)
    after = hip_ctx.stats()
    assert mid["decode_linear_calls"] == before["decode_linear_calls"] + 1
    assert mid["prefill_linear_calls"] == before["prefill_linear_calls"]
    assert after["prefill_linear_calls"] == mid["prefill_linear_calls"] + 1
    assert after["prefill_rows"] == mid["prefill_rows"] + 65
    # prefill on a decode-sized width is allowed and correct
    x = helpers.activations(3, k, 4)
    got = _run(torch, mat, x, n, 3)
    assert helpers.rel_l2(got, oracle.linear(capi.TYPE_Q8_0, canon, k, n, x)) <= PREFILL_EXPECT
    mat.release()


def test_prefill_rejects_bad_arguments(torch_cuda, hip_ctx):
    torch = torch_cuda
    k, n = 64, 16
    canon = helpers.weights(capi.TYPE_Q8_0, k, n, seed=1)
    mat = capi.Matrix(hip_ctx, capi.TYPE_Q8_0, k, n, canon, canon.nbytes, on_device=False)
    x = torch.zeros((5000, k), dtype=torch.float32, device="cuda:0")
    y = torch.zeros((5000, n), dtype=torch.float32, device="cuda:0")
    with pytest.raises(capi.HipError) as e:
        mat.linear(x, y, 5000, tactic=capi.LINEAR_PREFILL)
    assert e.value.status_name == "unsupported"
    with pytest.raises(capi.HipError) as e:
        mat.linear(x, y, 0, tactic=capi.LINEAR_PREFILL)
    assert e.value.status_name == "invalid_argument"
    with pytest.raises(capi.HipError) as e:
        mat.linear_loaded(y, tactic=capi.LINEAR_PREFILL)
    assert e.value.status_name == "unsupported"
    with pytest.raises(capi.HipError) as e:
        hip_ctx.set_prefill_tuning(3, 0, 0, 0)
    assert e.value.status_name == "invalid_argument"
    mat.release()


# configs[4]'s prefill linears: the Qwen2-7B projections at M = 512 (a full
# prefill step of 512 prompt tokens), in Q8_0 and the two 4-bit formats.
REAL_SHAPES = [("q|k|v", 4608, 3584, True), ("o", 3584, 3584, False), ("gate|up", 37888, 3584, False),
               ("down", 3584, 18944, False)]


@pytest.fixture(scope="module")
def _oracle_threads():
    import os
    before = oracle.threads()
    oracle.set_threads(min(16, os.cpu_count() or 1))
    yield
    oracle.set_threads(before)


@pytest.mark.parametrize("type_id", [capi.TYPE_Q8_0, capi.TYPE_Q4_0, capi.TYPE_Q4_K],
                         ids=lambda t: capi.TYPE_NAMES[t])
@pytest.mark.parametrize("label,n,k,with_bias", REAL_SHAPES, ids=[s[0] for s in REAL_SHAPES])
def test_prefill_real_shapes_m512(torch_cuda, hip_ctx, _oracle_threads, type_id, label, n, k, with_bias):
    """Every 512-row activation block against the oracle on a seeded sample
    of 256 output rows plus the first and last 16-row tiles (rows checked
    one by one), on the planner's own launch shape."""
    torch = torch_cuda
    dev = torch.device("cuda:0")
    m = 512
    seed = 61_000 + n + k + type_id
    canon_dev = quant.synthetic_weights_device(type_id, k, n, seed, dev)
    canon = canon_dev.cpu().numpy()
    mat = capi.Matrix(hip_ctx, type_id, k, n, canon_dev, canon_dev.numel(), on_device=True)
    del canon_dev
    bias = np.random.default_rng(seed).standard_normal(n).astype(np.float32) * 0.02 if with_bias else None
    x = helpers.activations(m, k, seed=seed + 1)
    rows = np.unique(np.concatenate([np.random.default_rng(seed + 2).choice(n, size=256, replace=False),
                                     np.arange(16), np.arange(n - 16, n)])).astype(np.uint64)
    try:
        plan = mat.plan(m, tactic=capi.LINEAR_PREFILL)
        got = _run(torch, mat, x, n, m, bias)[:, rows.astype(np.int64)]
        want = oracle.linear_row_list(type_id, canon, k, n, x, rows, bias=bias)
        assert np.isfinite(got).all()
        err = helpers.rel_l2(got, want)
        print(f"prefill M=512 {capi.TYPE_NAMES[type_id]} {label} {n}x{k}: rel_l2={err:.3e} | {plan}", flush=True)
        assert err <= PREFILL_EXPECT
        for r in range(m):
            assert helpers.rel_l2(got[r], want[r]) <= PREFILL_TOL, r
    finally:
        mat.release()


HYB_TYPES = [capi.TYPE_Q8_0, capi.TYPE_Q4_0, capi.TYPE_Q4_K, capi.TYPE_F16, capi.TYPE_BF16, capi.TYPE_Q6_K]


@pytest.mark.parametrize("type_id", HYB_TYPES, ids=lambda t: capi.TYPE_NAMES[t])
@pytest.mark.parametrize("stages", [2, 3])
@pytest.mark.parametrize("k,n,m,tile", [(3584, 4608, 512, (4, 2, 2)), (4096, 700, 257, (8, 4, 8)),
                                         (768, 1000, 65, (8, 2, 1)), (1280, 37, 130, (8, 4, 3)),
                                         (512, 300, 100, (4, 2, 1))])
def test_prefill_hybrid_matches_register_path(torch_cuda, type_id, stages, k, n, m, tile):
    """The hybrid GEMM (activation fragments through an LDS ring, weight
    records straight into registers) runs the register kernel's arithmetic
    in the same order, so on the same tile and K split its outputs are
    bit-identical in every storage format; both are held to the oracle
    (ragged N, M not a whole activation tile, splits with a short last
    split, the 8x4 launch with its 4x2 remainder)."""
    from tests.test_gpu_dense import _weights as dense_weights
    torch = torch_cuda
    stream = torch.cuda.current_stream(torch.device("cuda:0")).cuda_stream
    ctx = capi.Context(0, stream)
    seed = k + 7 * n + type_id
    canon = (dense_weights(type_id, k, n, seed) if type_id in (capi.TYPE_F16, capi.TYPE_BF16, capi.TYPE_Q6_K)
             else helpers.weights(type_id, k, n, seed=seed))
    mat = capi.Matrix(ctx, type_id, k, n, canon, canon.nbytes, on_device=False)
    x = helpers.activations(m, k, seed=k + m + 1)
    bias = np.random.default_rng(n + 1).standard_normal(n).astype(np.float32) * 0.02
    try:
        tm, tn, splits = tile
        ctx.set_prefill_tuning(tm, tn, splits, 2)
        ctx.set_prefill_pipeline(1)
        ref = _run(torch, mat, x, n, m, bias)
        ctx.set_prefill_pipeline(0x10 + stages)
        plan = mat.plan(m, tactic=capi.LINEAR_PREFILL)
        assert plan.startswith("prefill_hyb_kernel"), plan
        got = _run(torch, mat, x, n, m, bias)
        again = _run(torch, mat, x, n, m, bias)
        print(f"hybrid {capi.TYPE_NAMES[type_id]} {stages} stages {n}x{k} M={m}: {plan}", flush=True)
        assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))
        assert np.array_equal(again.view(np.uint32), got.view(np.uint32))
        rows = np.unique(np.concatenate([np.arange(min(n, 16)), np.arange(max(0, n - 16), n),
                                         np.random.default_rng(k).choice(n, size=min(n, 128), replace=False)]))
        want = oracle.linear_row_list(type_id, canon, k, n, x, rows.astype(np.uint64), bias=bias)
        assert helpers.rel_l2(got[:, rows], want) <= PREFILL_EXPECT
    finally:
        mat.release()
        ctx.close()


@pytest.mark.parametrize("stages", [2, 3, 4])
@pytest.mark.parametrize("k,n,m,tile", [(3584, 4608, 512, (4, 2, 2)), (18944, 3584, 512, (8, 4, 8)),
                                         (896, 4864, 65, (8, 4, 1)), (512, 3584, 257, (4, 2, 1)),
                                         (96, 37, 100, (8, 4, 1)), (3584, 1000, 130, (4, 2, 3))])
def test_prefill_lds_pipeline_matches_register_path(torch_cuda, stages, k, n, m, tile):
    """The LDS-pipelined GEMM (operands streamed global -> LDS through a ring
    of `stages` steps) runs the register kernel's arithmetic in the same
    order, so on the same tile shape and K split its outputs are
    bit-identical; both are held to the oracle (Q8_0; ragged N, M and K
    splits that leave a short last split included)."""
    torch = torch_cuda
    stream = torch.cuda.current_stream(torch.device("cuda:0")).cuda_stream
    ctx = capi.Context(0, stream)
    canon = helpers.weights(capi.TYPE_Q8_0, k, n, seed=k + 7 * n)
    mat = capi.Matrix(ctx, capi.TYPE_Q8_0, k, n, canon, canon.nbytes, on_device=False)
    x = helpers.activations(m, k, seed=k + m + 1)
    bias = np.random.default_rng(n + 1).standard_normal(n).astype(np.float32) * 0.02
    try:
        tm, tn, splits = tile
        ctx.set_prefill_tuning(tm, tn, splits, 0)
        ctx.set_prefill_pipeline(1)
        ref = _run(torch, mat, x, n, m, bias)
        ctx.set_prefill_pipeline(stages)
        plan = mat.plan(m, tactic=capi.LINEAR_PREFILL)
        assert plan.startswith("prefill_lds_kernel"), plan
        got = _run(torch, mat, x, n, m, bias)
        again = _run(torch, mat, x, n, m, bias)
        print(f"lds pipeline {stages} stages {n}x{k} M={m}: {plan}", flush=True)
        assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))
        assert np.array_equal(again.view(np.uint32), got.view(np.uint32))
        rows = np.unique(np.concatenate([np.arange(min(n, 16)), np.arange(max(0, n - 16), n),
                                         np.random.default_rng(k).choice(n, size=min(n, 128), replace=False)]))
        want = oracle.linear_row_list(capi.TYPE_Q8_0, canon, k, n, x, rows.astype(np.uint64), bias=bias)
        assert helpers.rel_l2(got[:, rows], want) <= PREFILL_EXPECT
    finally:
        mat.release()
        ctx.close()


def test_prefill_remainder_launch_is_bit_identical(torch_cuda):
    """A grid of 8x4 tiles that would end in a mostly empty round of
    workgroups (here 532 on 512 slots) runs its whole rounds on the 8x4 tile
    and the remaining rows as a second launch on the 4x2 tile.  Without a K
    split every output is the same sequence of MFMAs whatever the register
    tile, so the result equals one 4x2 launch bit for bit (N = 33800 also
    leaves a ragged last row tile in the remainder); both are held to the
    oracle."""
    torch = torch_cuda
    stream = torch.cuda.current_stream(torch.device("cuda:0")).cuda_stream
    ctx = capi.Context(0, stream)
    k, n, m = 512, 33800, 512
    canon = helpers.weights(capi.TYPE_Q8_0, k, n, seed=33800)
    mat = capi.Matrix(ctx, capi.TYPE_Q8_0, k, n, canon, canon.nbytes, on_device=False)
    x = helpers.activations(m, k, seed=17)
    bias = np.random.default_rng(5).standard_normal(n).astype(np.float32) * 0.02
    try:
        ctx.set_prefill_tuning(8, 4, 1, 1)
        plan = mat.plan(m, tactic=capi.LINEAR_PREFILL)
        print(f"remainder split {n}x{k} M={m}: {plan}", flush=True)
        assert "remainder" in plan and "groups=128" in plan, plan
        got = _run(torch, mat, x, n, m, bias)
        ctx.set_prefill_tuning(4, 2, 1, 2)
        ctx.set_prefill_pipeline(1)
        ref = _run(torch, mat, x, n, m, bias)
        assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))
        rows = np.unique(np.concatenate([np.arange(16), np.arange(32768 - 16, 32768 + 16), np.arange(n - 24, n),
                                         np.random.default_rng(1).choice(n, size=256, replace=False)]))
        want = oracle.linear_row_list(capi.TYPE_Q8_0, canon, k, n, x, rows.astype(np.uint64), bias=bias)
        assert helpers.rel_l2(got[:, rows], want) <= PREFILL_EXPECT
    finally:
        mat.release()
        ctx.close()


@pytest.mark.parametrize("type_id", [capi.TYPE_Q8_0, capi.TYPE_Q4_K], ids=lambda t: capi.TYPE_NAMES[t])
def test_prefill_split_remainder(torch_cuda, type_id):
    """With a long K the 4x2 remainder launch splits K towards two
    workgroups per CU (here 72 workgroups x 7 splits of 8 steps, the most
    that keep 8 steps per split) and a column reduction sums
    its partials in split order into the remainder's columns only.  The
    8x4 launch's columns stay bit-identical to an unsplit 4x2 launch; the
    remainder's columns differ only in f32 summation order; both are held to
    the oracle, the boundary row tiles and the ragged last tile included."""
    torch = torch_cuda
    stream = torch.cuda.current_stream(torch.device("cuda:0")).cuda_stream
    ctx = capi.Context(0, stream)
    k, n, m = 3584, 33800, 512
    canon = helpers.weights(type_id, k, n, seed=33801 + type_id)
    mat = capi.Matrix(ctx, type_id, k, n, canon, canon.nbytes, on_device=False)
    x = helpers.activations(m, k, seed=19)
    bias = np.random.default_rng(6).standard_normal(n).astype(np.float32) * 0.02
    try:
        ctx.set_prefill_tuning(8, 4, 1, 1)
        plan = mat.plan(m, tactic=capi.LINEAR_PREFILL)
        print(f"split remainder {capi.TYPE_NAMES[type_id]} {n}x{k} M={m}: {plan}", flush=True)
        assert "remainder" in plan and plan.endswith("groups=9 splits=7"), plan
        got = _run(torch, mat, x, n, m, bias)
        again = _run(torch, mat, x, n, m, bias)
        assert np.array_equal(again.view(np.uint32), got.view(np.uint32))
        ctx.set_prefill_tuning(4, 2, 1, 2)
        ctx.set_prefill_pipeline(1)
        ref = _run(torch, mat, x, n, m, bias)
        assert np.array_equal(got[:, :32768].view(np.uint32), ref[:, :32768].view(np.uint32))
        assert helpers.rel_l2(got[:, 32768:], ref[:, 32768:]) <= 1e-6
        # An unsplit remainder (the override) is the 4x2 launch bit for bit.
        ctx.set_prefill_pipeline(0)
        ctx.set_prefill_tuning(8, 4, 1, 1)
        ctx.set_prefill_remainder_splits(1)
        assert mat.plan(m, tactic=capi.LINEAR_PREFILL).endswith("groups=9 splits=1")
        unsplit = _run(torch, mat, x, n, m, bias)
        assert np.array_equal(unsplit.view(np.uint32), ref.view(np.uint32))
        with pytest.raises(capi.HipError) as e:
            ctx.set_prefill_remainder_splits(65)
        assert e.value.status_name == "invalid_argument"
        rows = np.unique(np.concatenate([np.arange(32768 - 16, 32768 + 16), np.arange(n - 24, n),
                                         np.random.default_rng(2).choice(np.arange(32768, n), size=128,
                                                                         replace=False)]))
        want = oracle.linear_row_list(type_id, canon, k, n, x, rows.astype(np.uint64), bias=bias)
        assert helpers.rel_l2(got[:, rows], want) <= PREFILL_EXPECT
    finally:
        mat.release()
        ctx.close()


@pytest.mark.parametrize("k,f,m", [(3584, 18944, 512), (96, 600, 70), (992, 200, 65)])
def test_prefill_operand_from_norm_and_swiglu(torch_cuda, hip_ctx, k, f, m):
    """air_hip_rms_norm_prefill and air_hip_silu_mul_prefill leave the next
    prefill linear's f16 operand: that linear gives the bits of the plain
    norm / SwiGLU followed by the linear converting its input itself, with
    and without the residual add, at the 7B widths (k 3584, FFN 18944), at
    widths whose f16 rows are padded (96, 600 and 992 -> 256, 768 and 1024
    columns).  Another call in between cancels the operand (the linear
    converts again and still matches)."""
    torch = torch_cuda
    lib = capi.lib()
    h = hip_ctx.handle
    pf = capi.LINEAR_PREFILL
    canon_q = helpers.weights(capi.TYPE_Q8_0, k, 512, seed=k + 1)
    mat_q = capi.Matrix(hip_ctx, capi.TYPE_Q8_0, k, 512, canon_q, canon_q.nbytes, on_device=False)
    kf = (f + 31) // 32 * 32
    canon_d = helpers.weights(capi.TYPE_Q8_0, kf, 256, seed=f + 2) if kf == f else None
    mat_d = capi.Matrix(hip_ctx, capi.TYPE_Q8_0, f, 256, canon_d, canon_d.nbytes, on_device=False) if kf == f else None

    def bits(t):
        return t.cpu().numpy().view(np.uint32)

    try:
        w = _dev(torch, helpers.activations(1, k, seed=k + 3)[0])
        x0 = _dev(torch, helpers.activations(m, k, seed=m + 4) * 3.0)
        resid = _dev(torch, helpers.activations(m, k, seed=m + 5))
        for with_resid in (False, True):
            # reference: plain norm, then the linear converting its input
            xa = x0.clone()
            normed_ref = torch.empty((m, k), dtype=torch.float32, device="cuda:0")
            if with_resid:
                capi.check(lib.air_hip_add_rms_norm(h, xa.data_ptr(), resid.data_ptr(), w.data_ptr(),
                                                    normed_ref.data_ptr(), m, k, 1e-6))
            else:
                capi.check(lib.air_hip_rms_norm(h, xa.data_ptr(), w.data_ptr(), normed_ref.data_ptr(), m, k, 1e-6))
            y_ref = torch.empty((m, 512), dtype=torch.float32, device="cuda:0")
            mat_q.linear(normed_ref, y_ref, m, tactic=pf)
            # fused: the norm leaves the operand
            xb = x0.clone()
            normed = torch.full((m, k), float("nan"), dtype=torch.float32, device="cuda:0")
            capi.check(lib.air_hip_rms_norm_prefill(h, xb.data_ptr(), resid.data_ptr() if with_resid else None,
                                                    w.data_ptr(), normed.data_ptr(), m, k, 1e-6))
            y = torch.full((m, 512), float("nan"), dtype=torch.float32, device="cuda:0")
            mat_q.linear(normed, y, m, tactic=pf)
            torch.cuda.synchronize()
            assert np.array_equal(bits(normed), bits(normed_ref)), (k, m, with_resid)
            assert np.array_equal(bits(xb), bits(xa)), (k, m, with_resid)
            assert np.array_equal(bits(y), bits(y_ref)), (k, m, with_resid)
            # another call in between: the operand is not used, the result still matches
            capi.check(lib.air_hip_rms_norm_prefill(h, xb.data_ptr(), None, w.data_ptr(), normed.data_ptr(), m, k,
                                                    1e-6))
            normed.mul_(2.0)
            capi.check(lib.air_hip_rms_norm(h, normed.data_ptr(), w.data_ptr(), normed.data_ptr(), m, k, 1e-6))
            fresh = normed.clone()
            mat_q.linear(normed, y, m, tactic=pf)
            mat_q.linear(fresh, y_ref, m, tactic=pf)
            torch.cuda.synchronize()
            assert np.array_equal(bits(y), bits(y_ref)), (k, m, "cancelled")
        # SwiGLU
        gu = _dev(torch, helpers.activations(m, 2 * f, seed=f + 6) * 2.0)
        act_ref = torch.empty((m, f), dtype=torch.float32, device="cuda:0")
        capi.check(lib.air_hip_silu_mul(h, gu.data_ptr(), act_ref.data_ptr(), m, f))
        act = torch.full((m, f), float("nan"), dtype=torch.float32, device="cuda:0")
        capi.check(lib.air_hip_silu_mul_prefill(h, gu.data_ptr(), act.data_ptr(), m, f))
        torch.cuda.synchronize()
        assert np.array_equal(bits(act), bits(act_ref)), (f, m)
        if mat_d is not None:
            y_ref = torch.empty((m, 256), dtype=torch.float32, device="cuda:0")
            capi.check(lib.air_hip_silu_mul_prefill(h, gu.data_ptr(), act.data_ptr(), m, f))
            yd = torch.full((m, 256), float("nan"), dtype=torch.float32, device="cuda:0")
            mat_d.linear(act, yd, m, tactic=pf)
            mat_d.linear(act_ref, y_ref, m, tactic=pf)
            torch.cuda.synchronize()
            assert np.array_equal(bits(yd), bits(y_ref)), (f, m)
    finally:
        mat_q.release()
        if mat_d is not None:
            mat_d.release()


@pytest.mark.parametrize("k,n,m,splits", [(3584, 3584, 512, 0), (2048, 1024, 100, 4), (1024, 512, 65, 1)])
def test_prefill_residual_epilogues(torch_cuda, hip_ctx, k, n, m, splits):
    """air_hip_linear_epilogue on the prefill tactic: RESIDUAL and
    RESIDUAL_PREFILL give the bits of the prefill linear followed by
    air_hip_add_rms_norm, with the K split's reduction carrying them (auto
    and forced splits) and without a split; RESIDUAL_PREFILL also leaves the
    next prefill linear's operand (that linear matches the same linear on
    the separately normed rows)."""
    torch = torch_cuda
    lib = capi.lib()
    h = hip_ctx.handle
    pf = capi.LINEAR_PREFILL
    canon = helpers.weights(capi.TYPE_Q8_0, k, n, seed=k + n + 13)
    mat = capi.Matrix(hip_ctx, capi.TYPE_Q8_0, k, n, canon, canon.nbytes, on_device=False)
    canon2 = helpers.weights(capi.TYPE_Q8_0, n, 640, seed=n + 17)
    mat2 = capi.Matrix(hip_ctx, capi.TYPE_Q8_0, n, 640, canon2, canon2.nbytes, on_device=False)

    def bits(t):
        return t.cpu().numpy().view(np.uint32)

    try:
        hip_ctx.set_prefill_tuning(0, 0, splits, 0)
        x = _dev(torch, helpers.activations(m, k, seed=m + k) * 2.0)
        resid0 = _dev(torch, helpers.activations(m, n, seed=m + 7))
        bias = _dev(torch, helpers.activations(1, n, seed=k + 3)[0] * 0.1)
        w = _dev(torch, helpers.activations(1, n, seed=k + 2)[0])
        lin = torch.empty((m, n), dtype=torch.float32, device="cuda:0")
        capi.check(lib.air_hip_linear(h, mat.handle, x.data_ptr(), lin.data_ptr(), bias.data_ptr(), m, pf))
        resid_ref = resid0.clone()
        normed_ref = torch.empty((m, n), dtype=torch.float32, device="cuda:0")
        capi.check(lib.air_hip_add_rms_norm(h, resid_ref.data_ptr(), lin.data_ptr(), w.data_ptr(),
                                            normed_ref.data_ptr(), m, n, 1e-6))
        y2_ref = torch.empty((m, 640), dtype=torch.float32, device="cuda:0")
        capi.check(lib.air_hip_linear(h, mat2.handle, normed_ref.data_ptr(), y2_ref.data_ptr(), None, m, pf))
        for epi in (capi.EPILOGUE_RESIDUAL, capi.EPILOGUE_RESIDUAL_PREFILL):
            resid = resid0.clone()
            normed = torch.full((m, n), float("nan"), dtype=torch.float32, device="cuda:0")
            capi.check(lib.air_hip_linear_epilogue(h, mat.handle, x.data_ptr(), m, resid.data_ptr(), bias.data_ptr(),
                                                   epi, w.data_ptr(), normed.data_ptr(), 1e-6, pf))
            y2 = torch.full((m, 640), float("nan"), dtype=torch.float32, device="cuda:0")
            capi.check(lib.air_hip_linear(h, mat2.handle, normed.data_ptr(), y2.data_ptr(), None, m, pf))
            torch.cuda.synchronize()
            assert np.array_equal(bits(resid), bits(resid_ref)), (epi, k, n, m, splits)
            assert np.array_equal(bits(normed), bits(normed_ref)), (epi, k, n, m, splits)
            assert np.array_equal(bits(y2), bits(y2_ref)), (epi, k, n, m, splits)
        assert lib.air_hip_linear_epilogue(h, mat.handle, x.data_ptr(), m, resid0.data_ptr(), None,
                                           capi.EPILOGUE_RESIDUAL_PREFILL, None, None, 0.0, pf) == 1
    finally:
        hip_ctx.set_prefill_tuning(0, 0, 0, 0)
        mat.release()
        mat2.release()
