"""The encodings without a resident tile format: F32, F16, BF16 and Q6_K
(held as the file's rows -- Q6_K as super-block records -- on f32 FMA
kernels, and for F16, BF16 and Q6_K on the matrix cores at 2..64 rows and
through the f16 prefill GEMM above) and Q5_0 (rewritten exactly as Q8_0
blocks, then the Q8_0 kernels).  The reference decodes all
of them per element in decode_element (src/cuda/cuda_backend.cu:241-344);
a Qwen2.5 Q4_K_M file mixes Q6_K and Q5_0 tensors with Q4_K and Q8_0.

gpu: device decode of canonical bytes of all eight types bit-exact with the
     oracle (whose decode is pinned to the reference's golden vectors);
     resident decode, embedding rows and describe of the new types; linears
     at widths 1..100 under every tactic within 1e-5 (dense, f32 FMA) or
     the Q8_0 kernels' gates for Q5_0 (1e-4 decode, 1e-2 prefill GEMM)
     relative L2 of the oracle's double-accumulated rows; the epilogue entry points and the
     no-allocation linear give what the separate launches give, bit for
     bit; the fused GEMV and loaded activations refuse dense matrices.
"""
import ctypes

import numpy as np
import pytest

import oracle
from air_amd import capi
from tests import helpers

pytestmark = pytest.mark.gpu

# (elements, bytes) per canonical block, and the byte offsets of f16 scales
BLOCK = {capi.TYPE_F32: (1, 4), capi.TYPE_F16: (1, 2), capi.TYPE_BF16: (1, 2), capi.TYPE_Q4_0: (32, 18),
         capi.TYPE_Q5_0: (32, 22), capi.TYPE_Q8_0: (32, 34), capi.TYPE_Q4_K: (256, 144),
         capi.TYPE_Q6_K: (256, 210)}
SCALES = {capi.TYPE_Q4_0: (0,), capi.TYPE_Q5_0: (0,), capi.TYPE_Q8_0: (0,), capi.TYPE_Q4_K: (0, 2),
          capi.TYPE_Q6_K: (208,)}
DENSE = [capi.TYPE_F32, capi.TYPE_F16, capi.TYPE_BF16, capi.TYPE_Q6_K]
UNSUPPORTED = 6   # AIR_HIP_UNSUPPORTED


def _dev(torch, a):
    return torch.from_numpy(np.ascontiguousarray(a)).to("cuda:0")


def _random_bytes(type_id, blocks, seed, scale_bits=None):
    """Random canonical blocks; f16 scales drawn from scale_bits (a callable
    rng, size -> uint16) when given, else any bit pattern."""
    rng = np.random.default_rng(seed)
    _, bb = BLOCK[type_id]
    raw = rng.integers(0, 256, size=(blocks, bb), dtype=np.uint8)
    if scale_bits is not None:
        for off in SCALES.get(type_id, ()):
            raw[:, off:off + 2] = scale_bits(rng, blocks).astype(np.uint16).view(np.uint8).reshape(blocks, 2)
    return raw.reshape(-1)


def _weights(type_id, k, n, seed):
    """Canonical bytes of a {k, n} matrix with values of a sane magnitude."""
    rng = np.random.default_rng(seed)
    if type_id in (capi.TYPE_F32, capi.TYPE_F16, capi.TYPE_BF16):
        w = (rng.standard_normal((n, k)) * 0.05).astype(np.float32)
        if type_id == capi.TYPE_F32:
            return w.view(np.uint8).reshape(-1)
        if type_id == capi.TYPE_F16:
            return w.astype(np.float16).view(np.uint8).reshape(-1)
        return (w.view(np.uint32) >> 16).astype(np.uint16).view(np.uint8).reshape(-1)
    be, _ = BLOCK[type_id]
    scale = 2e-3 if type_id == capi.TYPE_Q5_0 else 1e-4

    def bits(r, size):
        return (r.uniform(0.5, 1.5, size) * scale * r.choice([-1, 1], size)).astype(np.float16).view(np.uint16)

    return _random_bytes(type_id, n * (k // be), seed, scale_bits=bits)


@pytest.mark.parametrize("type_id", sorted(BLOCK), ids=lambda t: capi.TYPE_NAMES[t])
def test_dequantize_canonical_all_types(torch_cuda, hip_ctx, type_id):
    """air_hip_dequantize_canonical of every type the reference decodes,
    bit for bit with the oracle: random bytes (any f16 / f32 / bf16 bit
    pattern, NaN and inf included, for the float types; finite and any
    scales for the block types)."""
    torch = torch_cuda
    be, _ = BLOCK[type_id]
    blocks = 257 if be > 1 else 4099
    cases = [(1, None), (2, lambda r, s: r.integers(0, 0x7C00, s) | (r.integers(0, 2, s) << 15))]
    for seed, scale_bits in cases:
        raw = _random_bytes(type_id, blocks, seed, scale_bits)
        elements = blocks * be
        want = oracle.decode(type_id, raw, elements)
        out = torch.empty(elements, dtype=torch.float32, device="cuda:0")
        hip_ctx.dequantize_canonical(type_id, _dev(torch, raw), raw.nbytes, elements, out)
        torch.cuda.synchronize()
        assert helpers.same_bits(out.cpu().numpy(), want), (type_id, seed)


NEW_CASES = [(capi.TYPE_F32, 96, 37), (capi.TYPE_F16, 512, 300), (capi.TYPE_BF16, 256, 129),
             (capi.TYPE_Q6_K, 512, 300), (capi.TYPE_Q6_K, 256, 5), (capi.TYPE_Q5_0, 896, 300),
             (capi.TYPE_Q5_0, 32, 3)]


@pytest.mark.parametrize("type_id,k,n", NEW_CASES, ids=[f"{capi.TYPE_NAMES[t]}-{n}x{k}" for t, k, n in NEW_CASES])
def test_new_types_match_oracle(torch_cuda, hip_ctx, type_id, k, n):
    torch = torch_cuda
    canon = _weights(type_id, k, n, seed=k * 7 + n + type_id)
    mat = capi.Matrix(hip_ctx, type_id, k, n, canon, canon.nbytes, on_device=False)
    try:
        desc = mat.describe()
        assert desc["type"] == type_id and desc["k"] == k and desc["n"] == n
        # Resident bytes: the file's own encoding (Q6_K: 210 bytes per
        # super-block, as records plus a plane of scales), never f32 rows.
        resident = {capi.TYPE_F32: 4 * k * n, capi.TYPE_F16: 2 * k * n, capi.TYPE_BF16: 2 * k * n,
                    capi.TYPE_Q6_K: k * n // 256 * 210}
        if type_id in resident:
            assert desc["resident_bytes"] == resident[type_id], (desc, resident[type_id])
        # resident decode and embedding rows, bit for bit
        want_w = oracle.decode(type_id, canon, k * n).reshape(n, k)
        got_w = torch.empty((n, k), dtype=torch.float32, device="cuda:0")
        mat.dequantize(got_w)
        rows = [n - 1, 0, -1, n, n // 2]
        rows_d = torch.tensor(rows, dtype=torch.int32, device="cuda:0")
        emb = torch.full((len(rows), k), 7.0, dtype=torch.float32, device="cuda:0")
        capi.check(capi.lib().air_hip_matrix_rows(hip_ctx.handle, mat.handle, rows_d.data_ptr(), len(rows),
                                                  emb.data_ptr()))
        torch.cuda.synchronize()
        assert helpers.same_bits(got_w.cpu().numpy(), want_w)
        e = emb.cpu().numpy()
        for i, r in enumerate(rows):
            if 0 <= r < n:
                assert helpers.same_bits(e[i], want_w[r]), (i, r)
            else:
                assert (e[i] == 7.0).all(), (i, r)
        # Q5_0 runs the Q8_0 kernels: split-f16 decode (1e-4); the prefill
        # GEMM (Q5_0 as Q8_0, and the F16 / BF16 / Q6_K rows) has single f16
        # operands (its 1e-2 gate); F32 rows stay on the f32 FMA GEMM.
        tol_decode = 1e-4 if type_id == capi.TYPE_Q5_0 else 1e-5
        tol_prefill = 1e-2
        bias = helpers.activations(1, n, seed=n)[0] * 0.1
        bias_d = _dev(torch, bias)
        for m in (1, 3, 16, 17, 64, 100):
            x = helpers.activations(m, k, seed=m + k)
            want = oracle.linear(type_id, canon, k, n, x, bias=bias)
            x_d = _dev(torch, x)
            for tactic in (capi.LINEAR_AUTO, capi.LINEAR_DECODE, capi.LINEAR_PREFILL):
                if tactic == capi.LINEAR_DECODE and m > 64:
                    continue
                plan = mat.plan(m, tactic)
                print(f"{capi.TYPE_NAMES[type_id]} {n}x{k} M={m} tactic={tactic}: {plan}", flush=True)
                assert ("dense" in plan) == (type_id in DENSE), plan
                y = torch.full((m, n), float("nan"), dtype=torch.float32, device="cuda:0")
                mat.linear(x_d, y, m, bias=bias_d, tactic=tactic)
                torch.cuda.synchronize()
                got = y.cpu().numpy()
                assert plan.startswith("prefill") == (type_id != capi.TYPE_F32 and (
                    tactic == capi.LINEAR_PREFILL or (tactic == capi.LINEAR_AUTO and m > 64))), plan
                tol = tol_prefill if plan.startswith("prefill") else tol_decode
                for r in range(m):
                    err = helpers.rel_l2(got[r], want[r])
                    assert err <= tol, (m, tactic, r, err, plan)
    finally:
        mat.release()


MFMA_CASES = [(capi.TYPE_F16, 96, 37), (capi.TYPE_F16, 3584, 300), (capi.TYPE_BF16, 1056, 129),
              (capi.TYPE_BF16, 256, 5), (capi.TYPE_Q6_K, 512, 300), (capi.TYPE_Q6_K, 768, 33)]


@pytest.mark.parametrize("type_id,k,n", MFMA_CASES, ids=[f"{capi.TYPE_NAMES[t]}-{n}x{k}" for t, k, n in MFMA_CASES])
def test_dense_mfma_shapes_match_oracle(torch_cuda, hip_ctx, type_id, k, n):
    """The matrix-core kernel of the dense encodings (F16 and BF16 weights as
    exact MFMA operands, Q6_K codes decoded to exact f16 integers with the
    sub-block scales in the f32 epilogue) at every activation-tile count and
    past one launch's rows (65, 100), for one, two and four weight tiles per
    workgroup, one to eight waves splitting K, one and three steps in flight,
    a ragged last row tile and a K ending inside a 64-k step (96, 1056):
    within 1e-5 of the oracle per row, repeats bit-identical."""
    torch = torch_cuda
    canon = _weights(type_id, k, n, seed=k * 11 + n + type_id)
    mat = capi.Matrix(hip_ctx, type_id, k, n, canon, canon.nbytes, on_device=False)
    bias = helpers.activations(1, n, seed=n + 1)[0] * 0.1
    bias_d = _dev(torch, bias)
    shapes = [(0, 0, 0), (1, 1, 2), (2, 3, 4), (4, 8, 2), (1, 8, 4)]
    try:
        for m in (1, 2, 16, 17, 32, 33, 64, 65, 100):
            x = helpers.activations(m, k, seed=m * 3 + k)
            want = oracle.linear(type_id, canon, k, n, x, bias=bias)
            x_d = _dev(torch, x)
            for tile_n, waves, depth in shapes:
                hip_ctx.set_dense_path(1, tile_n, waves, depth)
                plan = mat.plan(m)
                assert "dense_mfma_kernel" in plan, plan
                outs = []
                for _ in range(2):
                    y = torch.full((m, n), float("nan"), dtype=torch.float32, device="cuda:0")
                    mat.linear(x_d, y, m, bias=bias_d)
                    torch.cuda.synchronize()
                    outs.append(y.cpu().numpy())
                assert np.isfinite(outs[0]).all(), plan
                for r in range(m):
                    err = helpers.rel_l2(outs[0][r], want[r])
                    assert err <= 1e-5, (m, plan, r, err)
                assert np.array_equal(outs[1].view(np.uint32), outs[0].view(np.uint32)), (m, plan)
    finally:
        hip_ctx.set_dense_path(0)
        mat.release()


PREFILL_CASES = [(capi.TYPE_F16, 1056, 300), (capi.TYPE_BF16, 512, 200), (capi.TYPE_Q6_K, 768, 130)]


@pytest.mark.parametrize("type_id,k,n", PREFILL_CASES,
                         ids=[f"{capi.TYPE_NAMES[t]}-{n}x{k}" for t, k, n in PREFILL_CASES])
def test_dense_prefill_gemm_matches_oracle(torch_cuda, hip_ctx, type_id, k, n):
    """Prefill widths over dense storage run the f16 MFMA prefill GEMM on the
    rows themselves (F16 as they are, BF16 and Q6_K formed in f16 under the
    matrix's power-of-two weight exponent): within the prefill GEMM's 1e-2 of
    the oracle per row at 65..512 rows, every register tile and a K split,
    with a ragged last row tile and a K ending inside a 64-k step (1056);
    the FMA GEMM (dense path 2) stays within 1e-5."""
    torch = torch_cuda
    canon = _weights(type_id, k, n, seed=k + 13 * n + type_id)
    mat = capi.Matrix(hip_ctx, type_id, k, n, canon, canon.nbytes, on_device=False)
    bias = helpers.activations(1, n, seed=n + 2)[0] * 0.1
    bias_d = _dev(torch, bias)
    try:
        for m in (65, 200, 512):
            x = helpers.activations(m, k, seed=m + 7 * k)
            want = oracle.linear(type_id, canon, k, n, x, bias=bias)
            x_d = _dev(torch, x)
            for path, tiling in [(0, (0, 0, 0, 0)), (0, (4, 2, 0, 0)), (0, (8, 4, 3, 1)), (0, (8, 2, 0, 0)),
                                 (2, (0, 0, 0, 0))]:
                hip_ctx.set_dense_path(path)
                hip_ctx.set_prefill_tuning(*tiling)
                plan = mat.plan(m)
                assert plan.startswith("prefill_gemm_kernel") == (path == 0), plan
                y = torch.full((m, n), float("nan"), dtype=torch.float32, device="cuda:0")
                mat.linear(x_d, y, m, bias=bias_d)
                torch.cuda.synchronize()
                got = y.cpu().numpy()
                tol = 1e-2 if path == 0 else 1e-5
                for r in range(m):
                    err = helpers.rel_l2(got[r], want[r])
                    assert err <= tol, (m, plan, r, err)
    finally:
        hip_ctx.set_prefill_tuning(0, 0, 0, 0)
        hip_ctx.set_dense_path(0)
        mat.release()


@pytest.mark.parametrize("type_id", DENSE, ids=lambda t: capi.TYPE_NAMES[t])
def test_dense_entry_points_match_separate_launches(torch_cuda, hip_ctx, type_id):
    """On a dense matrix the epilogue entry points run the plain linear then
    the epilogue's own kernel: bit-identical to those calls made one by
    one; the no-allocation linear equals air_hip_linear; the fused GEMV and
    loaded activations refuse it."""
    torch = torch_cuda
    lib = capi.lib()
    h = hip_ctx.handle
    k, n = 256, 192
    f = n // 2
    canon = _weights(type_id, k, n, seed=31 + type_id)
    mat = capi.Matrix(hip_ctx, type_id, k, n, canon, canon.nbytes, on_device=False)

    def bits(t):
        return t.cpu().numpy().view(np.uint32)

    try:
        w = _dev(torch, helpers.activations(1, n, seed=5)[0])
        for m in (1, 8, 40, 100):
            x = _dev(torch, helpers.activations(m, k, seed=m) * 2.0)
            lin = torch.empty((m, n), dtype=torch.float32, device="cuda:0")
            capi.check(lib.air_hip_linear(h, mat.handle, x.data_ptr(), lin.data_ptr(), None, m, capi.LINEAR_AUTO))
            act_ref = torch.empty((m, f), dtype=torch.float32, device="cuda:0")
            capi.check(lib.air_hip_silu_mul(h, lin.data_ptr(), act_ref.data_ptr(), m, f))
            act = torch.empty((m, f), dtype=torch.float32, device="cuda:0")
            capi.check(lib.air_hip_linear_epilogue(h, mat.handle, x.data_ptr(), m, act.data_ptr(), None,
                                                   capi.EPILOGUE_SWIGLU, None, None, 0.0, capi.LINEAR_AUTO))
            resid0 = _dev(torch, helpers.activations(m, n, seed=m + 9))
            resid_ref = resid0.clone()
            normed_ref = torch.empty((m, n), dtype=torch.float32, device="cuda:0")
            capi.check(lib.air_hip_add_rms_norm(h, resid_ref.data_ptr(), lin.data_ptr(), w.data_ptr(),
                                                normed_ref.data_ptr(), m, n, ctypes.c_double(1e-6)))
            epis = [capi.EPILOGUE_RESIDUAL_LOAD, capi.EPILOGUE_RESIDUAL_PREFILL] if m > 1 else [capi.EPILOGUE_RESIDUAL]
            got = []
            for epi in epis:
                resid = resid0.clone()
                normed = torch.empty((m, n), dtype=torch.float32, device="cuda:0")
                capi.check(lib.air_hip_linear_epilogue(h, mat.handle, x.data_ptr(), m, resid.data_ptr(), None, epi,
                                                       w.data_ptr(), normed.data_ptr(), ctypes.c_double(1e-6),
                                                       capi.LINEAR_AUTO))
                got.append((epi, resid, normed))
            if m <= 64:
                y_na = torch.empty((m, n), dtype=torch.float32, device="cuda:0")
                mat.linear_noalloc(x, y_na, m)
            torch.cuda.synchronize()
            assert np.array_equal(bits(act), bits(act_ref)), m
            for epi, resid, normed in got:
                assert np.array_equal(bits(resid), bits(resid_ref)), (m, epi)
                assert np.array_equal(bits(normed), bits(normed_ref)), (m, epi)
            if m <= 64:
                assert np.array_equal(bits(y_na), bits(lin)), m
        x1 = _dev(torch, helpers.activations(1, k, seed=1))
        y1 = torch.empty((1, n), dtype=torch.float32, device="cuda:0")
        rc = lib.air_hip_decode_linear_fused(h, mat.handle, x1.data_ptr(), y1.data_ptr(), None, None,
                                             ctypes.c_double(0.0), capi.EPILOGUE_STORE)
        assert rc == UNSUPPORTED and b"quantized" in lib.air_hip_last_error()
        capi.check(lib.air_hip_activations_load(h, x1.data_ptr(), k, 1))
        rc = lib.air_hip_linear_loaded(h, mat.handle, y1.data_ptr(), None, capi.LINEAR_AUTO)
        assert rc == UNSUPPORTED and b"dense" in lib.air_hip_last_error()
    finally:
        mat.release()


def test_dense_rejects_ragged_width(torch_cuda, hip_ctx):
    """Dense matrices need k a multiple of 32 (the kernels' float4 K steps)."""
    canon = _weights(capi.TYPE_F16, 48, 4, seed=1)
    handle = ctypes.c_void_p()
    rc = capi.lib().air_hip_matrix_prepare(hip_ctx.handle, capi.TYPE_F16, 48, 4, canon.ctypes.data, canon.nbytes, 0,
                                           ctypes.byref(handle))
    assert rc == UNSUPPORTED and b"multiple of 32" in capi.lib().air_hip_last_error()
