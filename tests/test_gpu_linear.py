"""GPU parity of the HIP engine against the CPU oracle, through the C ABI.

Dequantisation must be bit-exact (decode_all, tensor_reader.cpp:51-247);
linear outputs must be within relative L2 1e-4 of the double-accumulating
matvec (tensor_reader.cpp:369-394) on the decode tactic.
"""
from __future__ import annotations

import re

import numpy as np
import pytest

import oracle
from air_amd import capi, quant
from tests import helpers

pytestmark = pytest.mark.gpu

DECODE_TOL = 1e-4
FORMATS = [capi.TYPE_Q8_0, capi.TYPE_Q4_0, capi.TYPE_Q4_K]


def _dev(torch, a):
    return torch.from_numpy(np.ascontiguousarray(a)).to("cuda:0")


@pytest.mark.parametrize("type_id", FORMATS)
def test_dequantize_canonical_bit_exact(torch_cuda, hip_ctx, type_id):
    torch = torch_cuda
    be, bb = helpers.BLOCK[type_id]
    for seed, finite in [(1, True), (2, True), (3, False)]:
        raw = helpers.random_blocks(type_id, 257, seed, finite_scales=finite)
        elements = 257 * be
        want = oracle.decode(type_id, raw, elements)
        src = _dev(torch, raw)
        out = torch.empty(elements, dtype=torch.float32, device="cuda:0")
        hip_ctx.dequantize_canonical(type_id, src, raw.nbytes, elements, out)
        torch.cuda.synchronize()
        assert helpers.same_bits(out.cpu().numpy(), want), (type_id, seed)


@pytest.mark.parametrize("type_id,k,n", [
    (capi.TYPE_Q8_0, 96, 37), (capi.TYPE_Q8_0, 896, 64), (capi.TYPE_Q8_0, 32, 1),
    (capi.TYPE_Q4_0, 160, 45), (capi.TYPE_Q4_0, 896, 48),
    (capi.TYPE_Q4_K, 256, 19), (capi.TYPE_Q4_K, 768, 40),
])
def test_resident_tiles_decode_bit_exact(torch_cuda, hip_ctx, type_id, k, n):
    """The repacked planes decode to exactly the canonical values."""
    torch = torch_cuda
    be, bb = helpers.BLOCK[type_id]
    raw = helpers.random_blocks(type_id, n * (k // be), seed=k * 31 + n)
    want = oracle.decode(type_id, raw, n * k).reshape(n, k)
    for on_device in (False, True):
        src = _dev(torch, raw) if on_device else raw
        mat = capi.Matrix(hip_ctx, type_id, k, n, src, raw.nbytes, on_device=on_device)
        out = torch.empty((n, k), dtype=torch.float32, device="cuda:0")
        mat.dequantize(out)
        torch.cuda.synchronize()
        assert helpers.same_bits(out.cpu().numpy(), want)
        mat.release()


CASES = [
    # config 0 shape (Qwen2-0.5B FFN up-proj, Q8_0 4864 x 896)
    (capi.TYPE_Q8_0, 896, 4864, [1, 2, 7, 16, 33, 64, 100]),
    (capi.TYPE_Q8_0, 96, 37, [1, 5, 20]),
    (capi.TYPE_Q8_0, 32, 1, [1, 3]),
    (capi.TYPE_Q4_0, 896, 4864, [1, 16, 64]),
    (capi.TYPE_Q4_0, 160, 45, [1, 3, 17]),
    (capi.TYPE_Q4_K, 3584, 512, [1, 16, 64]),
    (capi.TYPE_Q4_K, 256, 19, [1, 4]),
    (capi.TYPE_Q4_K, 768, 40, [2, 31]),
]


@pytest.mark.parametrize("type_id,k,n,ms", CASES)
@pytest.mark.parametrize("with_bias", [False, True])
def test_linear_matches_oracle(torch_cuda, hip_ctx, type_id, k, n, ms, with_bias):
    torch = torch_cuda
    canon = helpers.weights(type_id, k, n, seed=k + 7 * n + type_id)
    mat = capi.Matrix(hip_ctx, type_id, k, n, canon, canon.nbytes, on_device=False)
    bias = (np.random.default_rng(5).standard_normal(n).astype(np.float32) * 0.02) if with_bias else None
    bias_d = _dev(torch, bias) if with_bias else None
    for m in ms:
        x = helpers.activations(m, k, seed=m * 1000 + k)
        want = oracle.linear(type_id, canon, k, n, x, bias=bias)
        y = torch.full((m, n), float("nan"), dtype=torch.float32, device="cuda:0")
        mat.linear(_dev(torch, x), y, m, bias=bias_d, tactic=capi.LINEAR_DECODE)
        torch.cuda.synchronize()
        got = y.cpu().numpy()
        assert np.isfinite(got).all(), (type_id, k, n, m)
        err = helpers.rel_l2(got, want)
        assert err <= DECODE_TOL, (type_id, k, n, m, err)
    mat.release()


def test_linear_scale_extremes(torch_cuda, hip_ctx):
    """Activations far from unit scale keep full relative precision
    (per-row power-of-two scaling of the split activations)."""
    torch = torch_cuda
    k, n = 896, 256
    canon = helpers.weights(capi.TYPE_Q8_0, k, n, seed=11)
    mat = capi.Matrix(hip_ctx, capi.TYPE_Q8_0, k, n, canon, canon.nbytes, on_device=False)
    base = helpers.activations(4, k, seed=3)
    x = base * np.array([[1e-6], [1.0], [3e3], [6e4]], dtype=np.float32)
    want = oracle.linear(capi.TYPE_Q8_0, canon, k, n, x)
    y = torch.empty((4, n), dtype=torch.float32, device="cuda:0")
    mat.linear(_dev(torch, x), y, 4)
    torch.cuda.synchronize()
    got = y.cpu().numpy()
    for i in range(4):
        assert helpers.rel_l2(got[i], want[i]) <= DECODE_TOL, i
    mat.release()


def test_linear_rejects_bad_arguments(torch_cuda, hip_ctx):
    torch = torch_cuda
    k, n = 64, 16
    canon = helpers.weights(capi.TYPE_Q8_0, k, n, seed=1)
    with pytest.raises(capi.HipError) as e:
        capi.Matrix(hip_ctx, capi.TYPE_Q8_0, k, n, canon, canon.nbytes - 1, on_device=False)
    assert e.value.status_name == "data_error"
    with pytest.raises(capi.HipError) as e:
        capi.Matrix(hip_ctx, capi.TYPE_Q8_0, 48, n, canon, canon.nbytes, on_device=False)
    assert e.value.status_name == "unsupported"
    mat = capi.Matrix(hip_ctx, capi.TYPE_Q8_0, k, n, canon, canon.nbytes, on_device=False)
    x = torch.zeros((1, k), device="cuda:0")
    y = torch.zeros((1, n), device="cuda:0")
    with pytest.raises(capi.HipError) as e:
        mat.linear(x, y, 0)
    assert e.value.status_name == "invalid_argument"
    with pytest.raises(capi.HipError) as e:
        mat.linear(x, y, 1, tactic=99)
    assert e.value.status_name == "invalid_argument"
    mat.release()


@pytest.mark.parametrize("type_id,k,n", [(capi.TYPE_Q8_0, 18944, 512), (capi.TYPE_Q4_0, 3584, 256),
                                         (capi.TYPE_Q4_K, 3584, 96)])
def test_linear_k_split_shapes_agree(torch_cuda, hip_ctx, type_id, k, n):
    """Every launch shape (row tiles per wave, waves per group, workgroups
    splitting K) gives the oracle's result, and repeated K-split launches
    re-arm their arrival counters (same bits on every repeat)."""
    torch = torch_cuda
    canon = helpers.weights(type_id, k, n, seed=k + n)
    mat = capi.Matrix(hip_ctx, type_id, k, n, canon, canon.nbytes, on_device=False)
    hip_ctx.set_decode_path(1)  # the fused / per-wave K-split kernels
    try:
        for m in (1, 3, 16, 40):
            x = helpers.activations(m, k, seed=m + 17)
            want = oracle.linear(type_id, canon, k, n, x)
            xd = _dev(torch, x)
            widest = (1, 4, 16) if type_id == capi.TYPE_Q4_K else (1, 16, 16)
            for rows, waves, splits in [(1, 1, 1), (1, 4, 8), (2, 2, 3), (4, 1, 2), widest]:
                hip_ctx.set_tuning(rows, waves, splits)
                outs = []
                for _ in range(3):
                    y = torch.full((m, n), float("nan"), dtype=torch.float32, device="cuda:0")
                    mat.linear(xd, y, m)
                    torch.cuda.synchronize()
                    outs.append(y.cpu().numpy())
                assert helpers.rel_l2(outs[0], want) <= DECODE_TOL, (m, rows, waves, splits)
                assert all(np.array_equal(o.view(np.uint32), outs[0].view(np.uint32)) for o in outs[1:])
    finally:
        hip_ctx.set_tuning(0, 0, 0)
        hip_ctx.set_decode_path(0)
        mat.release()


@pytest.mark.parametrize("type_id,k,n", [(capi.TYPE_Q8_0, 18944, 3584), (capi.TYPE_Q8_0, 4096, 1000),
                                         (capi.TYPE_Q4_0, 2048, 777), (capi.TYPE_Q4_K, 3584, 512),
                                         (capi.TYPE_Q8_0, 3584, 8192)])
def test_gemv_pair_split(torch_cuda, hip_ctx, type_id, k, n):
    """The one-row GEMV with two workgroups per row tile (their halves meet
    through one 64-bit slot per output row): the oracle's result with and
    without bias and at every wave count, the same bits on every repeat and
    after a launch on another shape (the slots return to zero), and the
    residual epilogue bit-exact against the linear plus the add."""
    torch = torch_cuda
    lib = capi.lib()
    canon = helpers.weights(type_id, k, n, seed=k + 3 * n + type_id)
    mat = capi.Matrix(hip_ctx, type_id, k, n, canon, canon.nbytes, on_device=False)
    small_canon = helpers.weights(capi.TYPE_Q8_0, 1024, 48, seed=5)
    small = capi.Matrix(hip_ctx, capi.TYPE_Q8_0, 1024, 48, small_canon, small_canon.nbytes, on_device=False)
    try:
        x = helpers.activations(1, k, seed=k + 29)
        xd = _dev(torch, x)
        bias = helpers.activations(1, n, seed=n + 31)[0] * 0.05
        bias_d = _dev(torch, bias)
        xs = _dev(torch, helpers.activations(1, 1024, seed=6))
        ys = torch.empty((1, 48), dtype=torch.float32, device="cuda:0")
        for b, bd in ((None, None), (bias, bias_d)):
            want = oracle.linear(type_id, canon, k, n, x, bias=b)
            for mode in (1, 2):
                hip_ctx.set_gemv_shape(mode)
                assert ("pair_split" in mat.plan(1)) == (mode == 2), mat.plan(1)
                for waves in (0, 1, 3, 8):
                    hip_ctx.set_tuning(0, waves, 0)
                    outs = []
                    for _ in range(3):
                        y = torch.full((1, n), float("nan"), dtype=torch.float32, device="cuda:0")
                        mat.linear(xd, y, 1, bias=bd)
                        small.linear(xs, ys, 1)
                        torch.cuda.synchronize()
                        outs.append(y.cpu().numpy())
                    assert helpers.rel_l2(outs[0], want) <= DECODE_TOL, (mode, waves, b is None)
                    assert all(np.array_equal(o.view(np.uint32), outs[0].view(np.uint32)) for o in outs[1:])
        # the residual epilogue on the paired launch
        hip_ctx.set_tuning(0, 0, 0)
        hip_ctx.set_gemv_shape(2)
        resid = _dev(torch, helpers.activations(1, n, seed=n + 37))
        lin = torch.empty((1, n), dtype=torch.float32, device="cuda:0")
        mat.linear(xd, lin, 1, bias=bias_d)
        want = (resid + lin).cpu().numpy()
        capi.check(lib.air_hip_decode_linear_fused(hip_ctx.handle, mat.handle, xd.data_ptr(), resid.data_ptr(),
                                                   bias_d.data_ptr(), None, 0.0, capi.EPILOGUE_RESIDUAL))
        torch.cuda.synchronize()
        assert np.array_equal(resid.cpu().numpy().view(np.uint32), want.view(np.uint32))
    finally:
        hip_ctx.set_tuning(0, 0, 0)
        hip_ctx.set_gemv_shape(0)
        small.release()
        mat.release()


def test_gemv_pair_split_limits(torch_cuda, hip_ctx):
    """Past 8192 output rows (the slot array) and on wide grids the GEMV
    keeps one workgroup per row tile; half-chunk work units stay Q8_0's (a
    4-bit chunk does not split); bad values are refused."""
    k, n = 1024, 8208
    canon = helpers.weights(capi.TYPE_Q8_0, k, n, seed=8)
    wide = capi.Matrix(hip_ctx, capi.TYPE_Q8_0, k, n, canon, canon.nbytes, on_device=False)
    canon4 = helpers.weights(capi.TYPE_Q4_0, k, 512, seed=9)
    q4 = capi.Matrix(hip_ctx, capi.TYPE_Q4_0, k, 512, canon4, canon4.nbytes, on_device=False)
    lib = capi.lib()
    try:
        hip_ctx.set_gemv_shape(2)
        assert "pair_split" not in wide.plan(1)
        hip_ctx.set_gemv_shape(0)
        assert "pair_split" not in wide.plan(1)
        hip_ctx.set_gemv_shape(1, 2, 0)
        assert "units_per_chunk=1" in q4.plan(1), q4.plan(1)
        assert "units_per_chunk=2" in wide.plan(1), wide.plan(1)
        assert lib.air_hip_context_set_gemv_shape(hip_ctx.handle, 3, 0, 0) == 1
        assert lib.air_hip_context_set_gemv_shape(hip_ctx.handle, 0, 3, 0) == 1
        assert lib.air_hip_context_set_gemv_shape(hip_ctx.handle, 0, 0, 3) == 1
    finally:
        hip_ctx.set_gemv_shape(0)
        q4.release()
        wide.release()


@pytest.mark.parametrize("type_id,k,n", [(capi.TYPE_Q8_0, 3584, 200), (capi.TYPE_Q4_0, 1152, 333),
                                         (capi.TYPE_Q4_K, 2304, 96), (capi.TYPE_Q8_0, 18944, 64)])
def test_skinny_shapes_agree(torch_cuda, hip_ctx, type_id, k, n):
    """The skinny decode kernel (M = 2..64): every activation-tile count,
    one and two weight tiles per wave, K splits of 1..5 workgroups; each
    matches the oracle to 1e-4 and repeats bit-identically."""
    torch = torch_cuda
    canon = helpers.weights(type_id, k, n, seed=k * 3 + n)
    mat = capi.Matrix(hip_ctx, type_id, k, n, canon, canon.nbytes, on_device=False)
    try:
        for m in (2, 16, 17, 33, 48, 64):
            x = helpers.activations(m, k, seed=m + 5)
            want = oracle.linear(type_id, canon, k, n, x)
            xd = _dev(torch, x)
            for tile_n, splits in [(1, 1), (2, 1), (1, 3), (2, 2), (1, 5), (0, 0)]:
                hip_ctx.set_decode_path(2, tile_n, splits)
                outs = []
                for _ in range(2):
                    y = torch.full((m, n), float("nan"), dtype=torch.float32, device="cuda:0")
                    mat.linear(xd, y, m)
                    torch.cuda.synchronize()
                    outs.append(y.cpu().numpy())
                err = helpers.rel_l2(outs[0], want)
                assert err <= DECODE_TOL, (m, tile_n, splits, err)
                for r in range(m):
                    assert helpers.rel_l2(outs[0][r], want[r]) <= DECODE_TOL, (m, tile_n, splits, r)
                assert np.array_equal(outs[1].view(np.uint32), outs[0].view(np.uint32)), (m, tile_n, splits)
    finally:
        hip_ctx.set_decode_path(0)
        mat.release()


@pytest.mark.parametrize("type_id,k,n", [(capi.TYPE_Q8_0, 3584, 200), (capi.TYPE_Q4_0, 1152, 333),
                                         (capi.TYPE_Q4_K, 2304, 96), (capi.TYPE_Q8_0, 18944, 64),
                                         (capi.TYPE_Q8_0, 96, 37), (capi.TYPE_Q4_K, 3584, 512)])
def test_wsplit_shapes_agree(torch_cuda, hip_ctx, type_id, k, n):
    """The wave-split decode kernel (M = 2..64, K split over the waves of a
    workgroup): every activation-tile count, one, two and four weight tiles
    per workgroup, one to eight waves, one and three steps of codes in
    flight, K split over one to three workgroups (mid-tile for the 128-k and
    256-k tiles), activations split in each wave and once into the
    workspace, a ragged last tile in N and a K that ends inside a 64-k step
    (96); each matches the oracle to 1e-4 per row and repeats
    bit-identically."""
    torch = torch_cuda
    canon = helpers.weights(type_id, k, n, seed=k * 5 + n)
    mat = capi.Matrix(hip_ctx, type_id, k, n, canon, canon.nbytes, on_device=False)
    shapes = [(1, 1, 2, 1, 2), (2, 3, 4, 1, 2), (4, 8, 2, 3, 2), (1, 4, 4, 3, 1), (2, 8, 2, 1, 1),
              (4, 2, 2, 2, 1), (0, 0, 0, 0, 0)]
    try:
        for m in (2, 9, 16, 17, 33, 48, 64):
            x = helpers.activations(m, k, seed=m + 23)
            want = oracle.linear(type_id, canon, k, n, x)
            xd = _dev(torch, x)
            for tile_n, waves, depth, splits, split_x in shapes:
                hip_ctx.set_wsplit(1, tile_n, waves, depth, splits, split_x)
                plan = mat.plan(m)
                assert "wsplit_kernel" in plan, plan
                outs = []
                for _ in range(2):
                    y = torch.full((m, n), float("nan"), dtype=torch.float32, device="cuda:0")
                    mat.linear(xd, y, m)
                    torch.cuda.synchronize()
                    outs.append(y.cpu().numpy())
                assert np.isfinite(outs[0]).all(), plan
                for r in range(m):
                    assert helpers.rel_l2(outs[0][r], want[r]) <= DECODE_TOL, (m, plan, r)
                assert np.array_equal(outs[1].view(np.uint32), outs[0].view(np.uint32)), (m, plan)
    finally:
        hip_ctx.set_wsplit(0)
        mat.release()


def test_wsplit_scale_extremes_and_bias(torch_cuda, hip_ctx):
    """Rows 1e-6 .. 6e4 apart in one activation tile keep their own relative
    precision (a power-of-two scale per row and step), with a fused bias and
    with the bias added by the split reduction; the automatic route takes
    the wave-split kernel at these widths."""
    torch = torch_cuda
    k, n = 3584, 512
    canon = helpers.weights(capi.TYPE_Q8_0, k, n, seed=29)
    mat = capi.Matrix(hip_ctx, capi.TYPE_Q8_0, k, n, canon, canon.nbytes, on_device=False)
    bias = np.random.default_rng(3).standard_normal(n).astype(np.float32) * 0.02
    try:
        base = helpers.activations(8, k, seed=8)
        x = base * np.array([[1e-6], [1.0], [3e3], [6e4], [2e-3], [1.0], [7.0], [1e2]], dtype=np.float32)
        want = oracle.linear(capi.TYPE_Q8_0, canon, k, n, x, bias=bias)
        assert "wsplit_kernel" in mat.plan(8), mat.plan(8)
        for splits in (0, 1, 3):
            hip_ctx.set_wsplit(0, 0, 0, 0, splits, 0)
            y = torch.empty((8, n), dtype=torch.float32, device="cuda:0")
            mat.linear(_dev(torch, x), y, 8, bias=_dev(torch, bias))
            torch.cuda.synchronize()
            got = y.cpu().numpy()
            for i in range(8):
                assert helpers.rel_l2(got[i], want[i]) <= DECODE_TOL, (splits, i)
    finally:
        hip_ctx.set_wsplit(0)
        mat.release()


@pytest.mark.parametrize("type_id,k,n", [(capi.TYPE_Q8_0, 3584, 8200), (capi.TYPE_Q8_0, 1024, 9000),
                                         (capi.TYPE_Q4_0, 3584, 8200), (capi.TYPE_Q4_K, 1024, 9000)])
def test_skinny_lds_pipeline_matches_registers(torch_cuda, hip_ctx, type_id, k, n):
    """The LDS-pipelined skinny kernel (on split activations: matrices of
    more than 512 row tiles, a ragged last tile here) gives the register
    pipeline's bits for 2..4 stages, one and two weight tiles per wave, with
    and without a K split (three splits start mid-tile for the 128-k and
    256-k tiles of Q4_0 and Q4_K), at every activation-tile count; the
    register pipeline matches the oracle to 1e-4."""
    torch = torch_cuda
    canon = helpers.weights(type_id, k, n, seed=k + 7 * n)
    mat = capi.Matrix(hip_ctx, type_id, k, n, canon, canon.nbytes, on_device=False)
    try:
        for m in (2, 16, 17, 32, 33, 64):
            x = helpers.activations(m, k, seed=m + 11)
            xd = _dev(torch, x)
            for tile_n, splits in [(1, 1), (2, 1), (2, 3), (1, 2)]:
                hip_ctx.set_decode_path(2, tile_n, splits)
                outs = {}
                for stages in (1, 2, 3, 4):
                    hip_ctx.set_decode_pipeline(stages)
                    plan = mat.plan(m)
                    assert ("skinny_lds_kernel" in plan) == (stages >= 2), (plan, stages)
                    y = torch.full((m, n), float("nan"), dtype=torch.float32, device="cuda:0")
                    mat.linear(xd, y, m)
                    torch.cuda.synchronize()
                    outs[stages] = y.cpu().numpy()
                for stages in (2, 3, 4):
                    assert np.array_equal(outs[stages].view(np.uint32), outs[1].view(np.uint32)), (
                        m, tile_n, splits, stages)
                if m in (17, 64) and (tile_n, splits) == (2, 3):
                    want = oracle.linear(type_id, canon, k, n, x)
                    assert helpers.rel_l2(outs[1], want) <= DECODE_TOL, m
    finally:
        hip_ctx.set_decode_pipeline(0)
        hip_ctx.set_decode_path(0)
        mat.release()


def test_graph_replay_after_workspace_growth(torch_cuda):
    """A HIP graph captured before the context grows its K-split partials
    replays on the buffer it captured (kept, not freed, until the context is
    destroyed) and still produces the oracle's result; the workspace
    generation records the growth.  A context of its own, so the partials
    start at the captured size."""
    torch = torch_cuda
    dev = torch.device("cuda:0")
    main = torch.cuda.current_stream(dev)
    type_id, k, n, m = capi.TYPE_Q8_0, 1024, 512, 8
    canon = helpers.weights(type_id, k, n, seed=77)
    x = helpers.activations(m, k, seed=78)
    want = oracle.linear(type_id, canon, k, n, x)
    ctx = capi.Context(0, main.cuda_stream)
    mat = capi.Matrix(ctx, type_id, k, n, canon, canon.nbytes, on_device=False)
    graph = None
    try:
        xd = _dev(torch, x)
        y = torch.zeros((m, n), dtype=torch.float32, device=dev)
        ctx.set_decode_path(2, 1, 2)              # skinny, K split over 2 workgroups
        mat.linear(xd, y, m)
        torch.cuda.synchronize()
        gen = ctx.stats()["workspace_generation"]
        capture = torch.cuda.Stream(dev)
        ctx.set_stream(capture.cuda_stream)
        graph = torch.cuda.CUDAGraph()
        try:
            with torch.cuda.graph(graph, stream=capture):
                mat.linear(xd, y, m)
        finally:
            ctx.set_stream(main.cuda_stream)
        assert ctx.stats()["workspace_generation"] == gen
        ctx.set_decode_path(2, 1, 8)              # four times the partials: the buffer grows
        y2 = torch.zeros((m, n), dtype=torch.float32, device=dev)
        mat.linear(xd, y2, m)
        torch.cuda.synchronize()
        assert ctx.stats()["workspace_generation"] > gen
        assert helpers.rel_l2(y2.cpu().numpy(), want) <= DECODE_TOL
        for _ in range(3):
            y.fill_(float("nan"))
            graph.replay()
            torch.cuda.synchronize()
            assert helpers.rel_l2(y.cpu().numpy(), want) <= DECODE_TOL
    finally:
        torch.cuda.synchronize()
        graph = None                              # before the context frees its kept buffers
        mat.release()
        ctx.close()


# (format, K, N, M, route override): the wave-split kernel (f32 rows and the
# row-scaled split, 2..8-way K splits), the skinny register and LDS kernels
# (2, 3 and 5-way splits), on 7B-like and ragged shapes.
CHAIN_CASES = [
    (capi.TYPE_Q8_0, 3584, 4608, 8, None),
    (capi.TYPE_Q8_0, 18944, 3584, 8, None),
    (capi.TYPE_Q8_0, 3584, 4608, 32, None),
    (capi.TYPE_Q8_0, 18944, 3584, 32, None),
    (capi.TYPE_Q8_0, 3584, 1000, 33, ("wsplit", 1, 4, 2, 3, 1)),
    (capi.TYPE_Q4_0, 2048, 777, 5, ("wsplit", 2, 4, 2, 4, 2)),
    (capi.TYPE_Q4_K, 2304, 512, 20, ("wsplit", 1, 8, 2, 2, 1)),
    (capi.TYPE_Q8_0, 3584, 1000, 40, ("skinny", 1, 3, 2)),
    (capi.TYPE_Q4_0, 1152, 333, 17, ("skinny", 2, 5, 1)),
    (capi.TYPE_Q4_K, 3584, 512, 64, ("skinny", 1, 2, 2)),
]


def _route(ctx, route):
    if route is None:
        return
    if route[0] == "wsplit":
        _, tn, waves, depth, splits, sx = route
        ctx.set_wsplit(1, tn, waves, depth, splits, sx)
    else:
        _, tn, splits, stages = route
        ctx.set_wsplit(2)
        ctx.set_decode_path(2, tn, splits)
        ctx.set_decode_pipeline(stages)


@pytest.mark.parametrize("type_id,k,n,m,route", CHAIN_CASES)
def test_split_chain_matches_reduction(torch_cuda, hip_ctx, type_id, k, n, m, route):
    """A K split over workgroups summed inside the kernel (each output's
    partials meet through 64-bit exchange slots in split order) gives the
    reduction launch's bits, with and without bias, on every repeat and after
    a launch on another shape (the slots return to zero); the oracle's result
    to 1e-4."""
    torch = torch_cuda
    canon = helpers.weights(type_id, k, n, seed=k + 5 * n + m)
    mat = capi.Matrix(hip_ctx, type_id, k, n, canon, canon.nbytes, on_device=False)
    other_canon = helpers.weights(capi.TYPE_Q8_0, 1024, 96, seed=4)
    other = capi.Matrix(hip_ctx, capi.TYPE_Q8_0, 1024, 96, other_canon, other_canon.nbytes, on_device=False)
    try:
        _route(hip_ctx, route)
        x = helpers.activations(m, k, seed=m + k)
        x[:, ::61] *= 40.0
        xd = _dev(torch, x)
        xo = _dev(torch, helpers.activations(m, 1024, seed=9))
        yo = torch.empty((m, 96), dtype=torch.float32, device="cuda:0")
        bias = helpers.activations(1, n, seed=n)[0] * 0.1
        bias_d = _dev(torch, bias)
        hip_ctx.set_split_chain(2)
        plan = mat.plan(m)
        print(f"chain {capi.TYPE_NAMES[type_id]} {n}x{k} M={m}: {plan}", flush=True)
        assert int(re.search(r"splits=(\d+)", plan).group(1)) > 1 and "in-kernel chain" in plan, plan
        for b, bd in ((None, None), (bias, bias_d)):
            hip_ctx.set_split_chain(1)
            ref = torch.full((m, n), float("nan"), dtype=torch.float32, device="cuda:0")
            mat.linear(xd, ref, m, bias=bd)
            torch.cuda.synchronize()
            want = ref.cpu().numpy()
            assert helpers.rel_l2(want, oracle.linear(type_id, canon, k, n, x, bias=b)) <= DECODE_TOL
            hip_ctx.set_split_chain(2)
            for _ in range(3):
                y = torch.full((m, n), float("nan"), dtype=torch.float32, device="cuda:0")
                mat.linear(xd, y, m, bias=bd)
                other.linear(xo, yo, m)
                torch.cuda.synchronize()
                assert np.array_equal(y.cpu().numpy().view(np.uint32), want.view(np.uint32)), (b is None)
    finally:
        hip_ctx.set_split_chain(0)
        hip_ctx.set_wsplit(0)
        hip_ctx.set_decode_path(0)
        hip_ctx.set_decode_pipeline(0)
        other.release()
        mat.release()


@pytest.mark.parametrize("type_id,k,n,m", [(capi.TYPE_Q8_0, 3584, 1000, 20), (capi.TYPE_Q8_0, 3584, 1000, 64),
                                           (capi.TYPE_Q4_0, 2048, 777, 32), (capi.TYPE_Q4_K, 2304, 520, 64),
                                           (capi.TYPE_Q8_0, 1024, 600, 45)])
def test_skinny_eight_waves_bit_identical(torch_cuda, hip_ctx, type_id, k, n, m):
    """The LDS skinny kernel with eight waves per workgroup (twice the weight
    rows sharing each step's activations) gives the four-wave kernel's bits
    at every split count, and the oracle's result; widths of one or three
    activation tiles keep four waves."""
    torch = torch_cuda
    canon = helpers.weights(type_id, k, n, seed=k + n + m)
    mat = capi.Matrix(hip_ctx, type_id, k, n, canon, canon.nbytes, on_device=False)
    try:
        x = helpers.activations(m, k, seed=m + 3)
        xd = _dev(torch, x)
        want = oracle.linear(type_id, canon, k, n, x)
        hip_ctx.set_wsplit(2)
        for splits in (1, 2, 4):
            hip_ctx.set_decode_path(2, 1, splits)
            outs = []
            for waves in (4, 8):
                hip_ctx.set_skinny_waves(waves)
                plan = mat.plan(m)
                assert ("waves=8" in plan) == (waves == 8 and -(-m // 16) in (2, 4)), plan
                y = torch.full((m, n), float("nan"), dtype=torch.float32, device="cuda:0")
                mat.linear(xd, y, m)
                torch.cuda.synchronize()
                outs.append(y.cpu().numpy())
            assert np.array_equal(outs[0].view(np.uint32), outs[1].view(np.uint32)), splits
            assert helpers.rel_l2(outs[1], want) <= DECODE_TOL, splits
    finally:
        hip_ctx.set_skinny_waves(0)
        hip_ctx.set_decode_path(0)
        hip_ctx.set_wsplit(0)
        mat.release()


def test_skinny_eight_waves_automatic(torch_cuda, hip_ctx):
    """Q8_0 gate|up-sized matrices at 17..32 rows take eight waves by
    themselves (one weight tile per wave, two K splits), with the bits of the
    four-wave kernel at the same tile and split counts."""
    torch = torch_cuda
    k, n, m = 3584, 37888, 32
    canon = quant.synthetic_weights_device(capi.TYPE_Q8_0, k, n, 9, torch.device("cuda:0"))
    mat = capi.Matrix(hip_ctx, capi.TYPE_Q8_0, k, n, canon, canon.numel(), on_device=True)
    del canon
    try:
        plan = mat.plan(m)
        assert "waves=8" in plan and "tile_n=1" in plan and "splits=2" in plan, plan
        assert "waves=8" not in mat.plan(40)
        xd = _dev(torch, helpers.activations(m, k, seed=8))
        outs = []
        for waves, tile_n, splits in ((0, 0, 0), (4, 1, 2)):
            hip_ctx.set_skinny_waves(waves)
            hip_ctx.set_decode_path(0, tile_n, splits)
            y = torch.full((m, n), float("nan"), dtype=torch.float32, device="cuda:0")
            mat.linear(xd, y, m)
            torch.cuda.synchronize()
            outs.append(y.cpu().numpy())
        assert np.isfinite(outs[0]).all()
        assert np.array_equal(outs[0].view(np.uint32), outs[1].view(np.uint32))
    finally:
        hip_ctx.set_skinny_waves(0)
        hip_ctx.set_decode_path(0)
        mat.release()


def test_skinny_wide_matrix_plans(torch_cuda, hip_ctx):
    """The automatic plans of wide (lm_head-sized) and gate|up-sized matrices
    between 17 and 64 rows: Q8_0 past 4096 row tiles at 49..64 rows takes
    eight waves (the four-wave kernel's bits), Q4_K past 4096 row tiles at
    17..32 rows two weight tiles per wave on the LDS pipeline, and Q4_0
    gate|up-sized matrices at 17..32 rows the register kernel with two
    tiles -- each within the decode tolerance of the oracle."""
    torch = torch_cuda
    big = capi.Matrix(hip_ctx, capi.TYPE_Q8_0, 1024, 65600,
                      *(lambda c: (c, c.nbytes))(helpers.weights(capi.TYPE_Q8_0, 1024, 65600, seed=71)),
                      on_device=False)
    try:
        m = 64
        plan = big.plan(m)
        assert "skinny_lds_kernel<q8_0>" in plan and "waves=8" in plan and "tile_n=1" in plan, plan
        splits = int(re.search(r"splits=(\d+)", plan).group(1))
        xd = _dev(torch, helpers.activations(m, 1024, seed=72))
        outs = []
        for waves, tile_n, k_splits in ((0, 0, 0), (4, 1, splits)):
            hip_ctx.set_skinny_waves(waves)
            hip_ctx.set_decode_path(0, tile_n, k_splits)
            y = torch.full((m, 65600), float("nan"), dtype=torch.float32, device="cuda:0")
            big.linear(xd, y, m)
            torch.cuda.synchronize()
            outs.append(y.cpu().numpy())
        assert np.isfinite(outs[0]).all()
        assert np.array_equal(outs[0].view(np.uint32), outs[1].view(np.uint32))
    finally:
        hip_ctx.set_skinny_waves(0)
        hip_ctx.set_decode_path(0)
        big.release()
    for type_id, k, n, m, kernel in ((capi.TYPE_Q4_K, 1024, 65600, 20, "skinny_lds_kernel<q4_k>"),
                                     (capi.TYPE_Q4_0, 512, 32016, 24, "skinny_kernel<q4_0>")):
        canon = helpers.weights(type_id, k, n, seed=n + m)
        mat = capi.Matrix(hip_ctx, type_id, k, n, canon, canon.nbytes, on_device=False)
        try:
            plan = mat.plan(m)
            assert kernel in plan and "tile_n=2" in plan, plan
            x = helpers.activations(m, k, seed=m + 5)
            y = torch.full((m, n), float("nan"), dtype=torch.float32, device="cuda:0")
            mat.linear(_dev(torch, x), y, m)
            torch.cuda.synchronize()
            assert helpers.rel_l2(y.cpu().numpy(), oracle.linear(type_id, canon, k, n, x)) <= DECODE_TOL, plan
        finally:
            mat.release()


def test_split_chain_under_graph_capture(torch_cuda):
    """A captured linear whose chain slots would have to grow during capture
    takes the reduction launch instead (same bits); once the slots exist, a
    captured chain replays correctly, the slots returning to zero between
    replays.  A context of its own, so no slots exist at first."""
    torch = torch_cuda
    dev = torch.device("cuda:0")
    main = torch.cuda.current_stream(dev)
    type_id, k, n, m = capi.TYPE_Q8_0, 3584, 4608, 8
    canon = helpers.weights(type_id, k, n, seed=91)
    x = helpers.activations(m, k, seed=92)
    ctx = capi.Context(0, main.cuda_stream)
    mat = capi.Matrix(ctx, type_id, k, n, canon, canon.nbytes, on_device=False)
    graphs = []
    try:
        assert "in-kernel chain" in mat.plan(m), mat.plan(m)
        xd = _dev(torch, x)
        ctx.set_split_chain(1)
        ref = torch.empty((m, n), dtype=torch.float32, device=dev)
        mat.linear(xd, ref, m)
        torch.cuda.synchronize()
        want = ref.cpu().numpy()
        ctx.set_split_chain(0)
        outs = []
        for _ in range(2):      # first capture: no slots yet; second: slots grown by the eager call between
            y = torch.full((m, n), float("nan"), dtype=torch.float32, device=dev)
            capture = torch.cuda.Stream(dev)
            ctx.set_stream(capture.cuda_stream)
            graph = torch.cuda.CUDAGraph()
            try:
                with torch.cuda.graph(graph, stream=capture):
                    mat.linear(xd, y, m)
            finally:
                ctx.set_stream(main.cuda_stream)
            graphs.append(graph)
            outs.append(y)
            eager = torch.full((m, n), float("nan"), dtype=torch.float32, device=dev)
            mat.linear(xd, eager, m)   # grows the slots outside capture
            torch.cuda.synchronize()
            assert np.array_equal(eager.cpu().numpy().view(np.uint32), want.view(np.uint32))
        for _ in range(3):
            for graph, y in zip(graphs, outs):
                y.fill_(float("nan"))
                graph.replay()
                torch.cuda.synchronize()
                assert np.array_equal(y.cpu().numpy().view(np.uint32), want.view(np.uint32))
    finally:
        torch.cuda.synchronize()
        graphs = None
        mat.release()
        ctx.close()


@pytest.mark.parametrize("type_id,k,f", [(capi.TYPE_Q8_0, 1056, 512), (capi.TYPE_Q8_0, 3584, 1184),
                                         (capi.TYPE_Q4_0, 1024, 256), (capi.TYPE_Q4_K, 2304, 512)])
def test_decode_linear_fused_matches_separate_kernels(torch_cuda, hip_ctx, type_id, k, f):
    """air_hip_decode_linear_fused against the separate kernels it replaces:
    RMSNorm then the linear (1e-6: the norm's sum runs in another order),
    the linear then a residual add (bit-exact: same launch plan), RMSNorm,
    the gate|up linear and SwiGLU (1e-6), and the gate|up linear and SwiGLU
    alone."""
    torch = torch_cuda
    lib = capi.lib()
    n = 2 * f
    canon = helpers.weights(type_id, k, n, seed=k + f)
    mat = capi.Matrix(hip_ctx, type_id, k, n, canon, canon.nbytes, on_device=False)
    try:
        x = _dev(torch, helpers.activations(1, k, seed=k + 1) * 3.0)
        w = _dev(torch, helpers.activations(1, k, seed=k + 2)[0])
        bias = _dev(torch, helpers.activations(1, n, seed=k + 3)[0] * 0.1)
        eps = 1e-6
        normed = torch.empty_like(x)
        ref = torch.empty((1, n), dtype=torch.float32, device="cuda:0")
        capi.check(lib.air_hip_rms_norm(hip_ctx.handle, x.data_ptr(), w.data_ptr(), normed.data_ptr(), 1, k, eps))
        mat.linear(normed, ref, 1, bias=bias)
        # RMSNorm + store
        got = torch.full((1, n), float("nan"), dtype=torch.float32, device="cuda:0")
        capi.check(lib.air_hip_decode_linear_fused(hip_ctx.handle, mat.handle, x.data_ptr(), got.data_ptr(),
                                                   bias.data_ptr(), w.data_ptr(), eps, capi.EPILOGUE_STORE))
        torch.cuda.synchronize()
        assert helpers.rel_l2(got.cpu().numpy(), ref.cpu().numpy()) <= 1e-6
        # residual add, bit-exact against linear + add
        resid = _dev(torch, helpers.activations(1, n, seed=k + 4))
        lin = torch.empty((1, n), dtype=torch.float32, device="cuda:0")
        mat.linear(x, lin, 1, bias=bias)
        want = (resid + lin).cpu().numpy()
        capi.check(lib.air_hip_decode_linear_fused(hip_ctx.handle, mat.handle, x.data_ptr(), resid.data_ptr(),
                                                   bias.data_ptr(), None, 0.0, capi.EPILOGUE_RESIDUAL))
        torch.cuda.synchronize()
        assert np.array_equal(resid.cpu().numpy().view(np.uint32), want.view(np.uint32))
        # RMSNorm + SwiGLU over the fused gate|up
        act_ref = torch.empty((1, f), dtype=torch.float32, device="cuda:0")
        capi.check(lib.air_hip_silu_mul(hip_ctx.handle, ref.data_ptr(), act_ref.data_ptr(), 1, f))
        act = torch.full((1, f), float("nan"), dtype=torch.float32, device="cuda:0")
        capi.check(lib.air_hip_decode_linear_fused(hip_ctx.handle, mat.handle, x.data_ptr(), act.data_ptr(),
                                                   bias.data_ptr(), w.data_ptr(), eps, capi.EPILOGUE_SWIGLU))
        torch.cuda.synchronize()
        assert helpers.rel_l2(act.cpu().numpy(), act_ref.cpu().numpy()) <= 1e-6
        # the gate|up linear and SwiGLU without the norm (1e-6: a workgroup
        # of twice the waves may split K over the waves differently; bit-exact
        # where the halves get the plain plan's wave count)
        # (the SwiGLU workgroup never pairs: the reference linear neither)
        hip_ctx.set_gemv_shape(1)
        mat.linear(x, lin, 1, bias=bias)
        hip_ctx.set_gemv_shape(0)
        act_ref = torch.empty((1, f), dtype=torch.float32, device="cuda:0")
        capi.check(lib.air_hip_silu_mul(hip_ctx.handle, lin.data_ptr(), act_ref.data_ptr(), 1, f))
        act = torch.full((1, f), float("nan"), dtype=torch.float32, device="cuda:0")
        capi.check(lib.air_hip_decode_linear_fused(hip_ctx.handle, mat.handle, x.data_ptr(), act.data_ptr(),
                                                   bias.data_ptr(), None, 0.0, capi.EPILOGUE_SWIGLU))
        torch.cuda.synchronize()
        assert helpers.rel_l2(act.cpu().numpy(), act_ref.cpu().numpy()) <= 1e-6
        if (type_id, k) == (capi.TYPE_Q8_0, 1056):
            assert np.array_equal(act.cpu().numpy().view(np.uint32), act_ref.cpu().numpy().view(np.uint32))
        # a combination that is not provided, and a bad epilogue
        assert lib.air_hip_decode_linear_fused(hip_ctx.handle, mat.handle, x.data_ptr(), resid.data_ptr(), None,
                                               w.data_ptr(), eps, capi.EPILOGUE_RESIDUAL) == 6
        assert lib.air_hip_decode_linear_fused(hip_ctx.handle, mat.handle, x.data_ptr(), resid.data_ptr(), None,
                                               None, 0.0, 7) == 1
        assert lib.air_hip_decode_linear_fused(hip_ctx.handle, mat.handle, x.data_ptr(), x.data_ptr(), None,
                                               None, 0.0, capi.EPILOGUE_STORE) == 1
    finally:
        hip_ctx.set_gemv_shape(0)
        mat.release()


@pytest.mark.parametrize("type_id,k,n", [(capi.TYPE_Q8_0, 1024, 1024), (capi.TYPE_Q4_0, 2048, 512),
                                         (capi.TYPE_Q4_K, 2304, 384), (capi.TYPE_Q8_0, 512, 666)])
def test_linear_epilogue_matches_separate_kernels(torch_cuda, hip_ctx, type_id, k, n):
    """air_hip_linear_epilogue against air_hip_linear followed by the kernel
    it replaces, bit-exact: SwiGLU (silu_mul), residual add + RMSNorm
    (add_rms_norm) and the add alone, at one row, widths served by the
    single-launch kernel, by the skinny kernel with and without a K split
    (the split reduction then carries the epilogue) and by the K-split kernel
    past 64 rows, and a width (n = 666)
    whose rows are too ragged for the reduction to carry it.  RESIDUAL_LOAD
    also leaves the norm's output split for the next linear on it: that
    linear (a wide one, which runs on split activations) must match the
    same linear over the separately normed rows, and a split must not be
    reused once another linear ran in between."""
    torch = torch_cuda
    lib = capi.lib()
    f = n // 2
    canon = helpers.weights(type_id, k, n, seed=k + n + 11)
    mat = capi.Matrix(hip_ctx, type_id, k, n, canon, canon.nbytes, on_device=False)
    n2 = 9216                                         # 576 row tiles: runs on split activations
    canon2 = helpers.weights(capi.TYPE_Q8_0, n, n2, seed=n + 5) if n % 32 == 0 else None
    mat2 = capi.Matrix(hip_ctx, capi.TYPE_Q8_0, n, n2, canon2, canon2.nbytes, on_device=False) if n % 32 == 0 else None
    dec = capi.LINEAR_DECODE
    h = hip_ctx.handle

    def bits(t):
        return t.cpu().numpy().view(np.uint32)

    try:
        bias = _dev(torch, helpers.activations(1, n, seed=k + 3)[0] * 0.1)
        w = _dev(torch, helpers.activations(1, n, seed=k + 2)[0])
        eps = 1e-6
        for m in (1, 8, 30, 64, 100):       # 100: the K-split kernel over loaded activations
            x = _dev(torch, helpers.activations(m, k, seed=m + k) * 2.0)
            resid0 = _dev(torch, helpers.activations(m, n, seed=m + 7))
            for path in [(0, 0, 0), (2, 1, 1), (2, 1, 3), (2, 2, 2)]:
                hip_ctx.set_decode_path(*path)
                case = (m, path)
                lin = torch.empty((m, n), dtype=torch.float32, device="cuda:0")
                capi.check(lib.air_hip_linear(h, mat.handle, x.data_ptr(), lin.data_ptr(), bias.data_ptr(), m, dec))
                # SwiGLU
                act_ref = torch.empty((m, f), dtype=torch.float32, device="cuda:0")
                capi.check(lib.air_hip_silu_mul(h, lin.data_ptr(), act_ref.data_ptr(), m, f))
                act = torch.full((m, f), float("nan"), dtype=torch.float32, device="cuda:0")
                capi.check(lib.air_hip_linear_epilogue(h, mat.handle, x.data_ptr(), m, act.data_ptr(),
                                                       bias.data_ptr(), capi.EPILOGUE_SWIGLU, None, None, 0.0, dec))
                # residual add + RMSNorm
                resid_ref = resid0.clone()
                normed_ref = torch.empty((m, n), dtype=torch.float32, device="cuda:0")
                capi.check(lib.air_hip_add_rms_norm(h, resid_ref.data_ptr(), lin.data_ptr(), w.data_ptr(),
                                                    normed_ref.data_ptr(), m, n, eps))
                resid = resid0.clone()
                normed = torch.full((m, n), float("nan"), dtype=torch.float32, device="cuda:0")
                capi.check(lib.air_hip_linear_epilogue(h, mat.handle, x.data_ptr(), m, resid.data_ptr(),
                                                       bias.data_ptr(), capi.EPILOGUE_RESIDUAL, w.data_ptr(),
                                                       normed.data_ptr(), eps, dec))
                # the add alone
                plain_ref = resid0.clone()
                capi.check(lib.air_hip_add(h, plain_ref.data_ptr(), lin.data_ptr(), m * n))
                plain = resid0.clone()
                capi.check(lib.air_hip_linear_epilogue(h, mat.handle, x.data_ptr(), m, plain.data_ptr(),
                                                       bias.data_ptr(), capi.EPILOGUE_RESIDUAL, None, None, 0.0,
                                                       dec))
                torch.cuda.synchronize()
                assert np.array_equal(bits(act), bits(act_ref)), case
                assert np.array_equal(bits(resid), bits(resid_ref)), case
                assert np.array_equal(bits(normed), bits(normed_ref)), case
                assert np.array_equal(bits(plain), bits(plain_ref)), case
                if mat2 is None:
                    assert lib.air_hip_linear_epilogue(h, mat.handle, x.data_ptr(), m, resid.data_ptr(), None,
                                                       capi.EPILOGUE_RESIDUAL_LOAD, w.data_ptr(), normed.data_ptr(),
                                                       eps, dec) == 1
                    continue
                # RESIDUAL_LOAD, then the next linear on the norm's output
                y2_ref = torch.empty((m, n2), dtype=torch.float32, device="cuda:0")
                capi.check(lib.air_hip_linear(h, mat2.handle, normed_ref.data_ptr(), y2_ref.data_ptr(), None, m, dec))
                resid = resid0.clone()
                normed = torch.full((m, n), float("nan"), dtype=torch.float32, device="cuda:0")
                capi.check(lib.air_hip_linear_epilogue(h, mat.handle, x.data_ptr(), m, resid.data_ptr(),
                                                       bias.data_ptr(), capi.EPILOGUE_RESIDUAL_LOAD, w.data_ptr(),
                                                       normed.data_ptr(), eps, dec))
                y2 = torch.full((m, n2), float("nan"), dtype=torch.float32, device="cuda:0")
                capi.check(lib.air_hip_linear(h, mat2.handle, normed.data_ptr(), y2.data_ptr(), None, m, dec))
                torch.cuda.synchronize()
                assert np.array_equal(bits(resid), bits(resid_ref)), case
                assert np.array_equal(bits(normed), bits(normed_ref)), case
                assert np.array_equal(bits(y2), bits(y2_ref)), case
                # another linear in between: the split is not reused for changed rows
                capi.check(lib.air_hip_linear_epilogue(h, mat.handle, x.data_ptr(), m, resid.data_ptr(),
                                                       bias.data_ptr(), capi.EPILOGUE_RESIDUAL_LOAD, w.data_ptr(),
                                                       normed.data_ptr(), eps, dec))
                capi.check(lib.air_hip_linear(h, mat.handle, x.data_ptr(), lin.data_ptr(), None, m, dec))
                normed.mul_(2.0)
                fresh = normed.clone()
                capi.check(lib.air_hip_linear(h, mat2.handle, normed.data_ptr(), y2.data_ptr(), None, m, dec))
                capi.check(lib.air_hip_linear(h, mat2.handle, fresh.data_ptr(), y2_ref.data_ptr(), None, m, dec))
                torch.cuda.synchronize()
                assert np.array_equal(bits(y2), bits(y2_ref)), case
                # another kernel of the context rewriting the norm's output in
                # between (here the RMSNorm with other weights): the split is
                # not reused either
                capi.check(lib.air_hip_linear_epilogue(h, mat.handle, x.data_ptr(), m, resid.data_ptr(),
                                                       bias.data_ptr(), capi.EPILOGUE_RESIDUAL_LOAD, w.data_ptr(),
                                                       normed.data_ptr(), eps, dec))
                w_other = w * 3.0
                capi.check(lib.air_hip_rms_norm(h, resid.data_ptr(), w_other.data_ptr(), normed.data_ptr(), m, n, eps))
                fresh = normed.clone()
                capi.check(lib.air_hip_linear(h, mat2.handle, normed.data_ptr(), y2.data_ptr(), None, m, dec))
                capi.check(lib.air_hip_linear(h, mat2.handle, fresh.data_ptr(), y2_ref.data_ptr(), None, m, dec))
                torch.cuda.synchronize()
                assert np.array_equal(bits(y2), bits(y2_ref)), case
        x = _dev(torch, helpers.activations(8, k, seed=1))
        out = torch.empty((8, n), dtype=torch.float32, device="cuda:0")
        assert lib.air_hip_linear_epilogue(h, mat.handle, x.data_ptr(), 8, out.data_ptr(), None,
                                           capi.EPILOGUE_STORE, None, None, 0.0, dec) == 1
        assert lib.air_hip_linear_epilogue(h, mat.handle, x.data_ptr(), 8, x.data_ptr(), None,
                                           capi.EPILOGUE_RESIDUAL, None, None, 0.0, dec) == 1
        assert lib.air_hip_linear_epilogue(h, mat.handle, x.data_ptr(), 8, out.data_ptr(), None,
                                           capi.EPILOGUE_SWIGLU, w.data_ptr(), out.data_ptr(), eps, dec) == 1
        assert lib.air_hip_linear_epilogue(h, mat.handle, x.data_ptr(), 8, out.data_ptr(), None,
                                           capi.EPILOGUE_RESIDUAL, w.data_ptr(), None, eps, dec) == 1
        assert lib.air_hip_linear_epilogue(h, mat.handle, x.data_ptr(), 0, out.data_ptr(), None,
                                           capi.EPILOGUE_RESIDUAL, None, None, 0.0, dec) == 1
    finally:
        hip_ctx.set_decode_path(0)
        mat.release()
        if mat2 is not None:
            mat2.release()


def test_argmax_flags_non_finite_rows(torch_cuda, hip_ctx):
    """air_hip_argmax: the first maximum of each row (lowest index among
    equal values, sampling.cpp:13-16), and -1 for a row holding NaN or
    +-inf anywhere -- the reference refuses such logits
    (cuda_backend.cu:613-624, 2368).  Both the vectorised and the scalar
    row paths; ties within one 4096-logit slice of the first pass and
    across slices."""
    torch = torch_cuda
    lib = capi.lib()
    for n in (152064, 1001):                          # float4 rows, and an odd width (scalar loop)
        rng = np.random.default_rng(n)
        rows = rng.standard_normal((9, n)).astype(np.float32)
        rows[1, 5] = np.nan
        rows[2, n - 1] = np.inf
        rows[3, n // 2] = -np.inf
        rows[4, :] = np.nan
        rows[5, [11, 700]] = 50.0                     # a tie: the lower index wins
        rows[6, 0] = 50.0
        far = [5000, 130000] if n > 130000 else [500, 900]
        rows[7, far] = 60.0                           # a tie across slices
        rows[8, n - 1] = 70.0                         # the maximum in the last (partial) slice
        x = _dev(torch, rows)
        out = torch.full((9,), 12345, dtype=torch.int32, device="cuda:0")
        capi.check(lib.air_hip_argmax(hip_ctx.handle, x.data_ptr(), 9, n, out.data_ptr()))
        torch.cuda.synchronize()
        got = out.cpu().numpy().tolist()
        assert got == [int(np.argmax(rows[0])), -1, -1, -1, -1, 11, 0, far[0], n - 1], (n, got)
