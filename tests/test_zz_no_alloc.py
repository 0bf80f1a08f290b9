"""air_hip_linear_noalloc: the decode linear that allocates nothing.

It runs the kernels and launch shapes of air_hip_linear, so its outputs must
be bit-identical to air_hip_linear's on the same context; its split
activations and K-split partials live in the library's per-GPU scratch
array.  Two calls in a row, the second with a smaller input, must both
match (the array keeps the previous call's contents).  The first call of
each case is also held to the oracle (ReferenceTensorReader::matvec,
src/reference/tensor_reader.cpp:369-394) at relative L2 1e-4 on sampled
rows.  The entry point must allocate nothing through the context (its
workspace generation stays put), work under HIP graph capture, and refuse
what exceeds its array.
"""
from __future__ import annotations

import numpy as np
import pytest

import oracle
from air_amd import capi, quant
from tests import helpers

pytestmark = pytest.mark.gpu

# (format, N, K, bias, (first M, second M)): the routes the planner takes at
# these shapes -- the skinny LDS pipeline over split activations (down at M =
# 64 with an 8-way K split, gate|up at M = 32 with two weight tiles per wave
# and a 2-way split, Q4_0 gate|up at M = 64), the wave-split kernel straight
# from f32 rows (down at M = 8 with a K split, q|k|v at M = 16 and 3, o at M
# = 4, Q4_0 gate|up at M = 2) and over the row-scaled split (gate|up at M =
# 16, Q4_K o at M = 17), Q4_K o at M = 64 on the LDS pipeline, and the M = 1
# GEMV (o; down with bias after down at M = 2) and its pair split (q|k|v at
# M = 1 after M = 2, its row slots in the second static array).
CASES = [
    (capi.TYPE_Q8_0, 3584, 18944, False, (64, 8)),
    (capi.TYPE_Q8_0, 37888, 3584, False, (32, 16)),
    (capi.TYPE_Q8_0, 4608, 3584, True, (16, 3)),
    (capi.TYPE_Q8_0, 3584, 3584, False, (4, 1)),
    (capi.TYPE_Q4_K, 3584, 3584, False, (64, 17)),
    (capi.TYPE_Q4_0, 37888, 3584, False, (64, 2)),
    (capi.TYPE_Q8_0, 3584, 18944, True, (2, 1)),
    (capi.TYPE_Q8_0, 4608, 3584, True, (2, 1)),
]


def _bits(t):
    return t.cpu().numpy().view(np.uint32)


@pytest.mark.parametrize("type_id,n,k,with_bias,ms", CASES,
                         ids=[f"{capi.TYPE_NAMES[c[0]]}-{c[1]}x{c[2]}-m{c[4][0]}-{c[4][1]}" for c in CASES])
def test_noalloc_matches_linear(torch_cuda, hip_ctx, type_id, n, k, with_bias, ms):
    torch = torch_cuda
    dev = torch.device("cuda:0")
    seed = 777 + n + k + type_id
    canon_dev = quant.synthetic_weights_device(type_id, k, n, seed, dev)
    canon = canon_dev.cpu().numpy()
    mat = capi.Matrix(hip_ctx, type_id, k, n, canon_dev, canon_dev.numel(), on_device=True)
    del canon_dev
    bias = (np.random.default_rng(seed).standard_normal(n).astype(np.float32) * 0.02) if with_bias else None
    bias_d = torch.from_numpy(bias).to(dev) if with_bias else None
    try:
        mmax = max(ms)
        x = torch.from_numpy(helpers.activations(mmax, k, seed=seed + 1)).to(dev)
        outs = []
        generation = hip_ctx.stats()["workspace_generation"]
        for m in ms:                       # two calls in a row, the second smaller
            print(f"noalloc {capi.TYPE_NAMES[type_id]} {n}x{k} M={m}: {mat.plan(m)}", flush=True)
            y = torch.full((m, n), float("nan"), dtype=torch.float32, device=dev)
            mat.linear_noalloc(x, y, m, bias=bias_d)
            outs.append(y)
        torch.cuda.synchronize()
        assert hip_ctx.stats()["workspace_generation"] == generation, "the no-allocation linear grew a buffer"
        for m, y in zip(ms, outs):
            ref = torch.full((m, n), float("nan"), dtype=torch.float32, device=dev)
            mat.linear(x, ref, m, bias=bias_d)
            torch.cuda.synchronize()
            assert np.array_equal(_bits(y), _bits(ref)), (m, mat.plan(m))
        rows = np.unique(np.concatenate([np.random.default_rng(seed).choice(n, size=min(n, 1024), replace=False),
                                         np.arange(n - 16, n)])).astype(np.uint64)
        m0 = ms[0]
        want = oracle.linear_row_list(type_id, canon, k, n, x[:m0].cpu().numpy(), rows, bias=bias)
        got = outs[0].cpu().numpy()[:, rows.astype(np.int64)]
        for r in range(m0):
            assert helpers.rel_l2(got[r], want[r]) <= 1e-4, (m0, r)
    finally:
        mat.release()


def test_noalloc_under_graph_capture(torch_cuda, hip_ctx):
    """Captured into a HIP graph and replayed with eager work in between:
    every replay equals the eager result."""
    torch = torch_cuda
    dev = torch.device("cuda:0")
    k, n, m = 18944, 3584, 32
    canon_dev = quant.synthetic_weights_device(capi.TYPE_Q8_0, k, n, 31, dev)
    mat = capi.Matrix(hip_ctx, capi.TYPE_Q8_0, k, n, canon_dev, canon_dev.numel(), on_device=True)
    del canon_dev
    stream = torch.cuda.current_stream(dev)
    try:
        x = torch.randn((m, k), device=dev)
        eager = torch.empty((m, n), device=dev)
        mat.linear(x, eager, m)
        torch.cuda.synchronize()
        y = torch.empty((m, n), device=dev)
        capture = torch.cuda.Stream(dev)
        hip_ctx.set_stream(capture.cuda_stream)
        graph = torch.cuda.CUDAGraph()
        try:
            with torch.cuda.graph(graph, stream=capture):
                mat.linear_noalloc(x, y, m)
        finally:
            hip_ctx.set_stream(stream.cuda_stream)
        other = torch.empty((8, n), device=dev)
        for i in range(3):
            y.fill_(float("nan"))
            graph.replay()
            torch.cuda.synchronize()
            assert np.array_equal(_bits(y), _bits(eager)), i
            mat.linear_noalloc(x[:8], other, 8)       # eager work on the same array between replays
            torch.cuda.synchronize()
        del graph
    finally:
        mat.release()


def test_noalloc_refuses_what_it_cannot_hold(torch_cuda, hip_ctx):
    torch = torch_cuda
    dev = torch.device("cuda:0")
    k, n = 3584, 37888
    canon_dev = quant.synthetic_weights_device(capi.TYPE_Q8_0, k, n, 5, dev)
    mat = capi.Matrix(hip_ctx, capi.TYPE_Q8_0, k, n, canon_dev, canon_dev.numel(), on_device=True)
    del canon_dev
    x = torch.randn((65, k), device=dev)
    y = torch.empty((65, n), device=dev)
    try:
        with pytest.raises(capi.HipError) as e:
            mat.linear_noalloc(x, y, 65)
        assert e.value.status_name == "unsupported"
        with pytest.raises(capi.HipError) as e:
            mat.linear_noalloc(x, y, 8, tactic=capi.LINEAR_PREFILL)
        assert e.value.status_name == "unsupported"
        with pytest.raises(capi.HipError) as e:
            mat.linear_noalloc(x, y, 0)
        assert e.value.status_name == "invalid_argument"
        hip_ctx.set_decode_path(2, 1, 64)           # 64 K splits x 64 rows of partials: 620 MB
        try:
            with pytest.raises(capi.HipError) as e:
                mat.linear_noalloc(x, y, 64)
            assert e.value.status_name == "unsupported" and "scratch" in str(e.value)
        finally:
            hip_ctx.set_decode_path(0)
    finally:
        mat.release()
