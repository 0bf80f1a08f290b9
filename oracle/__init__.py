"""CPU oracle for the quantized linear path -- TEST INFRASTRUCTURE ONLY.

Loads two checkers through ctypes:

* ``liboracle.so``  -- air_oracle.c, a plain-C restatement of AIR's reference
  block decoders and double-accumulating matvec
  (src/reference/tensor_reader.cpp:11-394);
* ``_ref/libairref.so`` -- AIR's own reference sources compiled where they lie
  (oracle/Makefile), present only where the reference checkout was available
  when the tree was built.

Only tests/, ``__graft_entry__.smoke()`` and the CPU-baseline leg of bench.py
may import this package, and only to check or time the reference algorithm;
the product (air_amd) never calls it.
"""
from __future__ import annotations

import ctypes
import os
from typing import Optional

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
ORACLE_PATH = os.path.join(_HERE, "liboracle.so")
REF_PATH = os.path.join(_HERE, "_ref", "libairref.so")

_P = ctypes.c_void_p
_U64 = ctypes.c_uint64

_oracle: Optional[ctypes.CDLL] = None
_ref: Optional[ctypes.CDLL] = None


def _load_oracle() -> ctypes.CDLL:
    global _oracle
    if _oracle is None:
        if not os.path.exists(ORACLE_PATH):
            raise RuntimeError(f"{ORACLE_PATH} missing: run `make -C oracle` or __graft_entry__.build()")
        lib = ctypes.CDLL(ORACLE_PATH)
        lib.oracle_f16_to_f32.restype = ctypes.c_float
        lib.oracle_f16_to_f32.argtypes = [ctypes.c_uint16]
        lib.oracle_decode.restype = ctypes.c_int
        lib.oracle_decode.argtypes = [ctypes.c_int, _P, _U64, _U64, _P]
        lib.oracle_linear_rows.restype = ctypes.c_int
        lib.oracle_linear_rows.argtypes = [ctypes.c_int, _P, _U64, _U64, _U64, ctypes.c_uint32, _P, _P, _P, _U64, _U64]
        lib.oracle_linear_row_list.restype = ctypes.c_int
        lib.oracle_linear_row_list.argtypes = [ctypes.c_int, _P, _U64, _U64, _U64, ctypes.c_uint32, _P, _P, _P, _U64,
                                               _P]
        lib.oracle_set_threads.restype = None
        lib.oracle_set_threads.argtypes = [ctypes.c_uint32]
        lib.oracle_threads.restype = ctypes.c_uint32
        lib.oracle_threads.argtypes = []
        _oracle = lib
    return _oracle


def ref_available() -> bool:
    return os.path.exists(REF_PATH)


def _load_ref() -> ctypes.CDLL:
    global _ref
    if _ref is None:
        if not ref_available():
            raise RuntimeError(f"{REF_PATH} missing: the reference build needs /root/reference at build time")
        lib = ctypes.CDLL(REF_PATH)
        lib.airref_decode.restype = ctypes.c_int
        lib.airref_decode.argtypes = [ctypes.c_int, _P, _U64, _U64, _P]
        lib.airref_matvec.restype = ctypes.c_int
        lib.airref_matvec.argtypes = [ctypes.c_int, _P, _U64, _U64, _U64, ctypes.c_uint32, _P, _P]
        lib.airref_model_create.restype = ctypes.c_int
        lib.airref_model_create.argtypes = [ctypes.c_int, _P, _U64, _U64, _U64, ctypes.POINTER(_P)]
        lib.airref_model_matvec.restype = ctypes.c_int
        lib.airref_model_matvec.argtypes = [_P, _P, _P]
        lib.airref_model_destroy.restype = None
        lib.airref_model_destroy.argtypes = [_P]
        _ref = lib
    return _ref


def _addr(a: np.ndarray) -> int:
    return int(a.ctypes.data)


def f16_to_f32(bits: int) -> float:
    return float(_load_oracle().oracle_f16_to_f32(bits))


def decode(type_id: int, data: np.ndarray, elements: int) -> np.ndarray:
    data = np.ascontiguousarray(data, dtype=np.uint8).reshape(-1)
    out = np.empty(elements, dtype=np.float32)
    rc = _load_oracle().oracle_decode(type_id, _addr(data), data.nbytes, elements, _addr(out))
    if rc != 0:
        raise ValueError(f"oracle_decode failed with status {rc}")
    return out


def linear(type_id: int, data: np.ndarray, k: int, n: int, x: np.ndarray,
           bias: Optional[np.ndarray] = None, rows: Optional[tuple] = None) -> np.ndarray:
    """y[m][r] = float(sum double(w[r,k]) * double(x[m,k])) (+ bias[r]).

    ``rows=(begin, end)`` restricts the output rows (the others stay 0)."""
    data = np.ascontiguousarray(data, dtype=np.uint8).reshape(-1)
    x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1, k)
    m = x.shape[0]
    y = np.zeros((m, n), dtype=np.float32)
    b = None if bias is None else np.ascontiguousarray(bias, dtype=np.float32)
    r0, r1 = rows if rows is not None else (0, n)
    rc = _load_oracle().oracle_linear_rows(type_id, _addr(data), data.nbytes, k, n, m, _addr(x),
                                           _addr(b) if b is not None else None, _addr(y), r0, r1)
    if rc != 0:
        raise ValueError(f"oracle_linear_rows failed with status {rc}")
    return y


def linear_row_list(type_id: int, data: np.ndarray, k: int, n: int, x: np.ndarray, rows,
                    bias: Optional[np.ndarray] = None) -> np.ndarray:
    """Output rows ``rows`` of the linear: y[m][j] = row rows[j] of input row m,
    each computed exactly as :func:`linear` computes it."""
    data = np.ascontiguousarray(data, dtype=np.uint8).reshape(-1)
    x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1, k)
    sel = np.ascontiguousarray(rows, dtype=np.uint64).reshape(-1)
    m = x.shape[0]
    y = np.zeros((m, sel.size), dtype=np.float32)
    b = None if bias is None else np.ascontiguousarray(bias, dtype=np.float32)
    rc = _load_oracle().oracle_linear_row_list(type_id, _addr(data), data.nbytes, k, n, m, _addr(x),
                                               _addr(b) if b is not None else None,
                                               _addr(sel) if sel.size else None, sel.size, _addr(y))
    if rc != 0:
        raise ValueError(f"oracle_linear_row_list failed with status {rc}")
    return y


def set_threads(threads: int) -> None:
    """Threads the oracle linears split their output rows over (results are
    bit-identical for every count)."""
    _load_oracle().oracle_set_threads(max(1, int(threads)))


def threads() -> int:
    return int(_load_oracle().oracle_threads())


def ref_decode(type_id: int, data: np.ndarray, elements: int) -> np.ndarray:
    data = np.ascontiguousarray(data, dtype=np.uint8).reshape(-1)
    out = np.empty(elements, dtype=np.float32)
    rc = _load_ref().airref_decode(type_id, _addr(data), data.nbytes, elements, _addr(out))
    if rc != 0:
        raise ValueError(f"airref_decode failed with status {rc}")
    return out


class RefMatrix:
    """One matrix held by AIR's reference ModelDefinition, for timing loops
    that should measure only ReferenceTensorReader::matvec."""

    def __init__(self, type_id: int, data: np.ndarray, k: int, n: int):
        self._data = np.ascontiguousarray(data, dtype=np.uint8).reshape(-1)
        self.k, self.n = k, n
        handle = _P()
        rc = _load_ref().airref_model_create(type_id, _addr(self._data), self._data.nbytes, k, n, ctypes.byref(handle))
        if rc != 0:
            raise ValueError(f"airref_model_create failed with status {rc}")
        self._handle = handle

    def matvec(self, x: np.ndarray) -> np.ndarray:
        x = np.ascontiguousarray(x, dtype=np.float32).reshape(self.k)
        y = np.empty(self.n, dtype=np.float32)
        rc = _load_ref().airref_model_matvec(self._handle, _addr(x), _addr(y))
        if rc != 0:
            raise ValueError(f"airref_model_matvec failed with status {rc}")
        return y

    def close(self) -> None:
        if self._handle:
            _load_ref().airref_model_destroy(self._handle)
            self._handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def ref_matvec(type_id: int, data: np.ndarray, k: int, n: int, x: np.ndarray) -> np.ndarray:
    data = np.ascontiguousarray(data, dtype=np.uint8).reshape(-1)
    x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1, k)
    y = np.empty((x.shape[0], n), dtype=np.float32)
    rc = _load_ref().airref_matvec(type_id, _addr(data), data.nbytes, k, n, x.shape[0], _addr(x), _addr(y))
    if rc != 0:
        raise ValueError(f"airref_matvec failed with status {rc}")
    return y


class RefGgufConfig(ctypes.Structure):
    _fields_ = [
        ("layers", ctypes.c_uint32), ("embedding", ctypes.c_uint32), ("ffn", ctypes.c_uint32),
        ("heads", ctypes.c_uint32), ("kv_heads", ctypes.c_uint32), ("rope_dims", ctypes.c_uint32),
        ("vocab", _U64), ("context", _U64), ("sliding_window", _U64),
        ("rope_base", ctypes.c_double), ("rms_eps", ctypes.c_double), ("eos", ctypes.c_int32),
        ("tensors", ctypes.c_uint32),
    ]


def ref_gguf_load(path: str, capacity: int = 4096):
    """AIR's own GgufFormat::load on a file: (status, config dict, [(offset, size, type)])."""
    lib = _load_ref()
    fn = lib.airref_gguf_load
    fn.restype = ctypes.c_int
    fn.argtypes = [ctypes.c_char_p, ctypes.POINTER(RefGgufConfig), _P, _P, _P, ctypes.c_uint32]
    cfg = RefGgufConfig()
    offsets = np.zeros(capacity, dtype=np.uint64)
    sizes = np.zeros(capacity, dtype=np.uint64)
    types = np.zeros(capacity, dtype=np.uint32)
    rc = fn(os.fsencode(path), ctypes.byref(cfg), _addr(offsets), _addr(sizes), _addr(types), capacity)
    if rc != 0:
        return rc, None, None
    n = min(cfg.tensors, capacity)
    table = [(int(offsets[i]), int(sizes[i]), int(types[i])) for i in range(n)]
    return 0, {name: getattr(cfg, name) for name, _ in RefGgufConfig._fields_}, table
