"""Host-side checks that need no GPU: the synthetic-weight quantizers and the
C ABI library (loads, exports every declared entry point, argument
handling that happens before any device work)."""
from __future__ import annotations

import ctypes
import os
import re

import numpy as np
import pytest

import oracle
from air_amd import capi, quant

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


@pytest.mark.parametrize("type_id,k", [(8, 96), (2, 96), (12, 512)])
def test_quantizers_emit_valid_blocks(type_id, k):
    rng = np.random.default_rng(type_id)
    n = 9
    w = rng.standard_normal((n, k)).astype(np.float32) * np.float32(0.02)
    data = quant.quantize(type_id, w)
    be, bb = quant.BLOCK[type_id]
    assert data.shape == (n, (k // be) * bb)
    dq = oracle.decode(type_id, data, n * k).reshape(n, k)
    if type_id == 8:
        d = np.abs(w.reshape(n, -1, 32)).max(axis=2) / 127.0
        err = np.abs(dq - w).reshape(n, -1, 32).max(axis=2)
        # |w - d q| <= d/2 (+ the f16 rounding of d times |q| <= 127)
        assert np.all(err <= d * 0.5 + d * 127 * 2.0 ** -11 + 1e-9)
    rel = np.linalg.norm(dq - w) / np.linalg.norm(w)
    assert rel < {8: 0.01, 2: 0.12, 12: 0.12}[type_id]


def test_q4_k_scale_packing_round_trips():
    rng = np.random.default_rng(1)
    sc = rng.integers(0, 64, size=(50, 8), dtype=np.uint8)
    mn = rng.integers(0, 64, size=(50, 8), dtype=np.uint8)
    packed = quant.pack_q4_k_scales(sc, mn)
    for row in range(50):
        s = packed[row].astype(np.uint32)
        for j in range(8):  # unpack as src/reference/tensor_reader.cpp:153-165
            if j < 4:
                usc, umn = s[j] & 63, s[j + 4] & 63
            else:
                usc = (s[j + 4] & 0x0F) | ((s[j - 4] >> 6) << 4)
                umn = (s[j + 4] >> 4) | ((s[j] >> 6) << 4)
            assert (usc, umn) == (sc[row, j], mn[row, j])


def _declared_functions():
    with open(os.path.join(ROOT, "include", "air_hip.h")) as f:
        text = f.read()
    return sorted(set(re.findall(r"^\s*(?:int|uint64_t|const char\*)\s+(air_hip_\w+)\(", text, re.M)))


def test_library_exports_every_declared_entry_point():
    lib = capi.lib()
    declared = _declared_functions()
    assert len(declared) >= 20
    for name in declared:
        assert hasattr(lib, name), name
        assert name in capi.SIGNATURES, f"{name} lacks a Python signature"
    assert set(capi.SIGNATURES) == set(declared)


def test_library_basics_without_device_work():
    lib = capi.lib()
    assert lib.air_hip_abi_version() == 2
    assert lib.air_hip_status_string(0) == b"ok"
    assert lib.air_hip_status_string(6) == b"unsupported"
    assert lib.air_hip_status_string(99) == b"unknown"
    assert capi.canonical_bytes(capi.TYPE_Q8_0, 896, 4864) == 4_630_528
    assert capi.canonical_bytes(capi.TYPE_Q4_0, 3584, 18944) == 38_191_104
    assert capi.canonical_bytes(capi.TYPE_Q4_K, 3584, 18944) == 38_191_104
    assert capi.canonical_bytes(capi.TYPE_Q4_K, 896, 4864) == 0   # K not a multiple of 256
    assert capi.canonical_bytes(capi.TYPE_BF16, 64, 64) == 8192     # every type decode_element takes
    assert capi.canonical_bytes(capi.TYPE_Q6_K, 3584, 18944) == 55_695_360
    assert capi.canonical_bytes(capi.TYPE_Q5_0, 896, 4864) == 2_996_224
    assert capi.canonical_bytes(capi.TYPE_F16, 896, 896) == 1_605_632
    assert capi.canonical_bytes(capi.TYPE_F32, 32, 3) == 384
    assert capi.canonical_bytes(capi.TYPE_Q6_K, 896, 4864) == 0   # K not a multiple of 256
    assert capi.canonical_bytes(3, 64, 64) == 0                   # Q4_1 is not executed here
    with pytest.raises(capi.HipError) as e:
        capi.check(lib.air_hip_context_create(0, None, None))
    assert e.value.status_name == "invalid_argument"
    with pytest.raises(capi.HipError) as e:
        capi.check(lib.air_hip_linear(None, None, None, None, None, 1, 0))
    assert e.value.status_name == "invalid_argument"


def test_context_creation_reports_missing_device():
    try:
        import torch
        has_gpu = torch.cuda.is_available()
    except Exception:  # pragma: no cover
        has_gpu = False
    if has_gpu:
        pytest.skip("a GPU is visible")
    handle = ctypes.c_void_p()
    status = capi.lib().air_hip_context_create(0, None, ctypes.byref(handle))
    assert status == 6  # unsupported: no HIP device
    assert b"no HIP device" in capi.lib().air_hip_last_error()
