"""ctypes binding of libair_hip.so (the C ABI declared in include/air_hip.h).

This module is a thin Python view of the C boundary: every call goes through
the native library, and importing it fails loudly when the library has not
been built (there is no Python or CPU fallback for any compute entry point).
Pointers are plain integers; ``ptr()`` accepts ints, torch tensors
(``data_ptr()``) and numpy arrays (host memory, for matrix upload only).
"""
from __future__ import annotations

import ctypes
import os
from typing import Optional

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libair_hip.so")

AIR_HIP_OK = 0
STATUS_NAMES = {
    0: "ok",
    1: "invalid_argument",
    2: "invalid_state",
    3: "io_error",
    4: "cancelled",
    5: "data_error",
    6: "unsupported",
    7: "internal_error",
}

TYPE_F32 = 0
TYPE_F16 = 1
TYPE_Q4_0 = 2
TYPE_Q5_0 = 6
TYPE_Q8_0 = 8
TYPE_Q4_K = 12
TYPE_Q6_K = 14
TYPE_BF16 = 30
TYPE_NAMES = {TYPE_F32: "f32", TYPE_F16: "f16", TYPE_Q4_0: "q4_0", TYPE_Q5_0: "q5_0", TYPE_Q8_0: "q8_0",
              TYPE_Q4_K: "q4_k", TYPE_Q6_K: "q6_k", TYPE_BF16: "bf16"}

EPILOGUE_STORE = 0
EPILOGUE_RESIDUAL = 1
EPILOGUE_SWIGLU = 2
EPILOGUE_RESIDUAL_LOAD = 3
EPILOGUE_RESIDUAL_PREFILL = 4

LINEAR_AUTO = 0
LINEAR_DECODE = 1
LINEAR_PREFILL = 2
MAX_DECODE_ROWS = 64

# Every exported entry point of include/air_hip.h: name -> (restype, argtypes).
_P = ctypes.c_void_p
_U64 = ctypes.c_uint64
_U32 = ctypes.c_uint32
_I = ctypes.c_int


class MatrixDesc(ctypes.Structure):
    _fields_ = [
        ("type", ctypes.c_int32),
        ("device", ctypes.c_int32),
        ("k", ctypes.c_uint64),
        ("n", ctypes.c_uint64),
        ("canonical_bytes", ctypes.c_uint64),
        ("resident_bytes", ctypes.c_uint64),
    ]


class Stats(ctypes.Structure):
    _fields_ = [
        ("resident_matrix_bytes", ctypes.c_uint64),
        ("workspace_bytes", ctypes.c_uint64),
        ("host_to_device_bytes", ctypes.c_uint64),
        ("prepared_matrices", ctypes.c_uint64),
        ("decode_linear_calls", ctypes.c_uint64),
        ("prefill_linear_calls", ctypes.c_uint64),
        ("decode_rows", ctypes.c_uint64),
        ("prefill_rows", ctypes.c_uint64),
        ("workspace_generation", ctypes.c_uint64),
    ]


class KvLayout(ctypes.Structure):
    """air_hip_kv_layout: the paged fp32 KV pool."""
    _fields_ = [
        ("pool", ctypes.c_void_p),
        ("page_tokens", ctypes.c_uint32),
        ("kv_width", ctypes.c_uint32),
        ("layers", ctypes.c_uint32),
        ("max_pages", ctypes.c_uint32),
        ("pool_pages", ctypes.c_uint32),
        ("chunks", ctypes.c_void_p),       # device chunk table (null: one pool)
        ("chunk_shift", ctypes.c_uint32),
    ]


class AttentionTile(ctypes.Structure):
    """air_hip_attention_tile."""
    _fields_ = [("row", ctypes.c_uint32), ("rows", ctypes.c_uint32), ("head", ctypes.c_uint32),
                ("heads", ctypes.c_uint32)]


def attention_tiles(run_rows, q_heads: int, kv_heads: int):
    """Host tiles of the online attention for rows in runs of one sequence each."""
    runs = (ctypes.c_uint32 * max(len(run_rows), 1))(*run_rows)
    count = ctypes.c_uint32()
    check(lib().air_hip_attention_make_tiles(runs, len(run_rows), q_heads, kv_heads, None, 0, ctypes.byref(count)))
    tiles = (AttentionTile * max(count.value, 1))()
    check(lib().air_hip_attention_make_tiles(runs, len(run_rows), q_heads, kv_heads, tiles, count.value,
                                             ctypes.byref(count)))
    return [(t.row, t.rows, t.head, t.heads) for t in tiles[:count.value]]


SIGNATURES = {
    "air_hip_abi_version": (_I, []),
    "air_hip_status_string": (ctypes.c_char_p, [_I]),
    "air_hip_last_error": (ctypes.c_char_p, []),
    "air_hip_device_count": (_I, [ctypes.POINTER(_I)]),
    "air_hip_mem_info": (_I, [_I, ctypes.POINTER(_U64), ctypes.POINTER(_U64)]),
    "air_hip_stream_read": (_I, [_P, _P, _U64, _P, _U64]),
    "air_hip_context_create": (_I, [_I, _P, ctypes.POINTER(_P)]),
    "air_hip_context_destroy": (_I, [_P]),
    "air_hip_context_set_stream": (_I, [_P, _P]),
    "air_hip_context_reserve": (_I, [_P, _U64, _U32]),
    "air_hip_context_stats": (_I, [_P, ctypes.POINTER(Stats)]),
    "air_hip_context_set_tuning": (_I, [_P, _U32, _U32, _U32]),
    "air_hip_context_set_gemv_shape": (_I, [_P, _U32, _U32, _U32]),
    "air_hip_context_set_split_chain": (_I, [_P, _U32]),
    "air_hip_context_set_skinny_waves": (_I, [_P, _U32]),
    "air_hip_context_set_prefill_tuning": (_I, [_P, _U32, _U32, _U32, _U32]),
    "air_hip_context_set_decode_path": (_I, [_P, _U32, _U32, _U32]),
    "air_hip_context_set_wsplit": (_I, [_P, _U32, _U32, _U32, _U32, _U32, _U32]),
    "air_hip_context_set_dense_path": (_I, [_P, _U32, _U32, _U32, _U32]),
    "air_hip_context_set_prefill_pipeline": (_I, [_P, _U32]),
    "air_hip_context_set_prefill_remainder_splits": (_I, [_P, _U32]),
    "air_hip_context_set_decode_pipeline": (_I, [_P, _U32]),
    "air_hip_matrix_rows": (_I, [_P, _P, _P, _U32, _P]),
    "air_hip_rms_norm": (_I, [_P, _P, _P, _P, _U32, _U64, ctypes.c_double]),
    "air_hip_rope": (_I, [_P, _P, _U64, _U32, _P, _U32, _U32, _U32, _U32, _P, _U64]),
    "air_hip_kv_append": (_I, [_P, _P, _P, _U64, _U64, _U32, _P, _P, _U32]),
    "air_hip_decode_linear_fused": (_I, [_P, _P, _P, _P, _P, _P, ctypes.c_double, ctypes.c_int]),
    "air_hip_linear_epilogue": (_I, [_P, _P, _P, _U32, _P, _P, ctypes.c_int, _P, _P, ctypes.c_double, ctypes.c_int]),
    "air_hip_rope_kv_append": (_I, [_P, _P, _P, _U64, _U32, _P, _P, _U32, _U32, _U32, _U32, _U32, _P, _U64]),
    "air_hip_linear_rope_kv": (_I, [_P, _P, _P, _U32, _P, _P, _P, _P, _P, _U32, _U32, _U32, _U32, _U32, _P, _U64,
                                     ctypes.c_int]),
    "air_hip_attention": (_I, [_P, _P, _P, _U64, _U32, _P, _P, _U32, _U32, _U32, _U32, _U64, _P]),
    "air_hip_add_rms_norm": (_I, [_P, _P, _P, _P, _P, _U32, _U64, ctypes.c_double]),
    "air_hip_attention_make_tiles": (_I, [_P, _U32, _U32, _U32, _P, _U32, _P]),
    "air_hip_attention_online": (_I, [_P, _P, _P, _U64, _U32, _P, _P, _U32, _U32, _U32, _U32, _P, _U32, _U64, _P]),
    "air_hip_silu_mul": (_I, [_P, _P, _P, _U32, _U64]),
    "air_hip_silu_mul_prefill": (_I, [_P, _P, _P, _U32, _U64]),
    "air_hip_rms_norm_prefill": (_I, [_P, _P, _P, _P, _P, _U32, _U64, ctypes.c_double]),
    "air_hip_add": (_I, [_P, _P, _P, _U64]),
    "air_hip_argmax": (_I, [_P, _P, _U32, _U64, _P]),
    "air_hip_canonical_bytes": (_U64, [_I, _U64, _U64]),
    "air_hip_matrix_prepare": (_I, [_P, _I, _U64, _U64, _P, _U64, _I, ctypes.POINTER(_P)]),
    "air_hip_matrix_release": (_I, [_P]),
    "air_hip_matrix_describe": (_I, [_P, ctypes.POINTER(MatrixDesc)]),
    "air_hip_matrix_dequantize": (_I, [_P, _P, _P]),
    "air_hip_dequantize_canonical": (_I, [_P, _I, _P, _U64, _U64, _P]),
    "air_hip_activations_load": (_I, [_P, _P, _U64, _U32]),
    "air_hip_linear_loaded": (_I, [_P, _P, _P, _P, _I]),
    "air_hip_linear": (_I, [_P, _P, _P, _P, _P, _U32, _I]),
    "air_hip_linear_plan": (_I, [_P, _P, _U32, _I, ctypes.c_char_p, _U64]),
    "air_hip_linear_noalloc": (_I, [_P, _P, _P, _P, _P, _U32, _I]),
}


class HipError(RuntimeError):
    def __init__(self, status: int, message: str):
        self.status = status
        self.status_name = STATUS_NAMES.get(status, "unknown")
        super().__init__(f"{self.status_name}: {message}")


_lib: Optional[ctypes.CDLL] = None


def lib() -> ctypes.CDLL:
    """Loads the in-tree native library; raises if it was not built."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(
                f"{LIB_PATH} is missing: build it with __graft_entry__.build() "
                "(there is no fallback path)"
            )
        handle = ctypes.CDLL(LIB_PATH)
        for name, (restype, argtypes) in SIGNATURES.items():
            fn = getattr(handle, name)
            fn.restype = restype
            fn.argtypes = argtypes
        _lib = handle
    return _lib


def check(status: int) -> None:
    if status != AIR_HIP_OK:
        msg = lib().air_hip_last_error().decode("utf-8", "replace")
        raise HipError(status, msg)


def ptr(obj) -> int:
    """Address of a device/host buffer: int, torch tensor, or numpy array."""
    if obj is None:
        return 0
    if isinstance(obj, int):
        return obj
    if hasattr(obj, "data_ptr"):
        return int(obj.data_ptr())
    if hasattr(obj, "ctypes"):
        return int(obj.ctypes.data)
    raise TypeError(f"cannot take the address of {type(obj)!r}")


def canonical_bytes(type_id: int, k: int, n: int) -> int:
    return int(lib().air_hip_canonical_bytes(type_id, k, n))


def device_count() -> int:
    n = _I(0)
    check(lib().air_hip_device_count(ctypes.byref(n)))
    return n.value


def mem_info(device: int = 0):
    free, total = _U64(0), _U64(0)
    check(lib().air_hip_mem_info(device, ctypes.byref(free), ctypes.byref(total)))
    return free.value, total.value


class Context:
    """A device + stream + workspace (air_hip_context)."""

    def __init__(self, device: int = 0, stream: int = 0):
        handle = _P()
        check(lib().air_hip_context_create(device, stream or None, ctypes.byref(handle)))
        self.handle = handle
        self.device = device

    def set_stream(self, stream: int) -> None:
        check(lib().air_hip_context_set_stream(self.handle, stream or None))

    def reserve(self, max_k: int, max_m: int) -> None:
        check(lib().air_hip_context_reserve(self.handle, max_k, max_m))

    def set_tuning(self, rows_per_wave: int = 0, waves_per_group: int = 0, k_splits: int = 0) -> None:
        check(lib().air_hip_context_set_tuning(self.handle, rows_per_wave, waves_per_group, k_splits))

    def set_skinny_waves(self, waves: int = 0) -> None:
        """Waves per workgroup of the LDS skinny kernel: 0 / 4 automatic, 8."""
        check(lib().air_hip_context_set_skinny_waves(self.handle, waves))

    def set_split_chain(self, mode: int = 0) -> None:
        """K splits of the 2..64-row kernels: 0 automatic, 1 reduction launch,
        2 summed in the kernel."""
        check(lib().air_hip_context_set_split_chain(self.handle, mode))

    def set_gemv_shape(self, pair_mode: int = 0, units_per_chunk: int = 0, depth: int = 0) -> None:
        """One-row GEMV: pair split (0 automatic, 1 never, 2 wherever it
        applies), work units per chunk and chunk buffers per wave (0 automatic)."""
        check(lib().air_hip_context_set_gemv_shape(self.handle, pair_mode, units_per_chunk, depth))

    def set_decode_path(self, path: int = 0, tile_n: int = 0, k_splits: int = 0) -> None:
        check(lib().air_hip_context_set_decode_path(self.handle, path, tile_n, k_splits))

    def set_wsplit(self, mode: int = 0, tile_n: int = 0, waves: int = 0, depth: int = 0, k_splits: int = 0,
                   split_x: int = 0) -> None:
        """Wave-split decode kernel for 2..64 rows: mode 0 automatic, 1 always,
        2 never, plus launch-shape overrides (0 = automatic; split_x 1 = split
        into the workspace first, 2 = in each wave)."""
        check(lib().air_hip_context_set_wsplit(self.handle, mode, tile_n, waves, depth, k_splits, split_x))

    def set_dense_path(self, path: int = 0, tile_n: int = 0, waves: int = 0, depth: int = 0) -> None:
        """Dense matrices (F16 / BF16 / Q6_K): path 0 automatic, 1 the matrix-core
        kernel at every width, 2 the FMA kernels; shape overrides (0 = automatic)."""
        check(lib().air_hip_context_set_dense_path(self.handle, path, tile_n, waves, depth))

    def set_decode_pipeline(self, lds_stages: int = 0) -> None:
        """Decode (skinny) operand staging: 0 automatic, 1 registers, 2..4 LDS ring stages."""
        check(lib().air_hip_context_set_decode_pipeline(self.handle, lds_stages))

    def set_prefill_pipeline(self, lds_stages: int = 0) -> None:
        """Prefill operand staging: 0 automatic, 1 registers, 2..4 LDS ring stages."""
        check(lib().air_hip_context_set_prefill_pipeline(self.handle, lds_stages))

    def set_prefill_remainder_splits(self, splits: int = 0) -> None:
        """K split of the prefill remainder launch (0 automatic, 1 unsplit)."""
        check(lib().air_hip_context_set_prefill_remainder_splits(self.handle, splits))

    def set_prefill_tuning(self, tile_m: int = 0, tile_n: int = 0, k_splits: int = 0, prefetch: int = 0) -> None:
        check(lib().air_hip_context_set_prefill_tuning(self.handle, tile_m, tile_n, k_splits, prefetch))

    def stream_read(self, data, nbytes: int, sink, sink_words: int) -> None:
        """air_hip_stream_read: one read of `nbytes` device bytes, the XOR of
        each chunk's words stored in a word of the zeroed uint32 `sink`
        (`sink_words` long); the checksum is the XOR of the sink's words."""
        check(lib().air_hip_stream_read(self.handle, ptr(data), nbytes, ptr(sink), sink_words))

    def stats(self) -> dict:
        s = Stats()
        check(lib().air_hip_context_stats(self.handle, ctypes.byref(s)))
        return {name: getattr(s, name) for name, _ in Stats._fields_}

    def close(self) -> None:
        if self.handle:
            check(lib().air_hip_context_destroy(self.handle))
            self.handle = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def load_activations(self, x, k: int, m: int) -> None:
        """Stage 1 of a linear: split x [m][k] into this context's workspace."""
        check(lib().air_hip_activations_load(self.handle, ptr(x), k, m))

    def dequantize_canonical(self, type_id: int, canonical, nbytes: int, elements: int, out) -> None:
        check(lib().air_hip_dequantize_canonical(self.handle, type_id, ptr(canonical), nbytes, elements, ptr(out)))


class Matrix:
    """A resident quantized matrix with GGML dims {k, n} (air_hip_matrix)."""

    def __init__(self, ctx: Context, type_id: int, k: int, n: int, canonical, nbytes: int, on_device: bool):
        handle = _P()
        check(
            lib().air_hip_matrix_prepare(
                ctx.handle, type_id, k, n, ptr(canonical), nbytes, 1 if on_device else 0, ctypes.byref(handle)
            )
        )
        self.handle = handle
        self.ctx = ctx
        self.type_id, self.k, self.n = type_id, k, n

    def describe(self) -> dict:
        d = MatrixDesc()
        check(lib().air_hip_matrix_describe(self.handle, ctypes.byref(d)))
        return {name: getattr(d, name) for name, _ in MatrixDesc._fields_}

    def dequantize(self, out) -> None:
        check(lib().air_hip_matrix_dequantize(self.ctx.handle, self.handle, ptr(out)))

    def linear(self, x, y, m: int, bias=None, tactic: int = LINEAR_AUTO) -> None:
        check(lib().air_hip_linear(self.ctx.handle, self.handle, ptr(x), ptr(y), ptr(bias), m, tactic))

    def linear_noalloc(self, x, y, m: int, bias=None, tactic: int = LINEAR_AUTO) -> None:
        """air_hip_linear_noalloc: decode widths 1..64, no allocation."""
        check(lib().air_hip_linear_noalloc(self.ctx.handle, self.handle, ptr(x), ptr(y), ptr(bias), m, tactic))

    def plan(self, m: int, tactic: int = LINEAR_AUTO) -> str:
        """The kernels and launch shape a linear of m rows runs on."""
        buf = ctypes.create_string_buffer(256)
        check(lib().air_hip_linear_plan(self.ctx.handle, self.handle, m, tactic, buf, len(buf)))
        return buf.value.decode()

    def linear_loaded(self, y, bias=None, tactic: int = LINEAR_AUTO) -> None:
        """Stage 2 of a linear, over the context's loaded activations."""
        check(lib().air_hip_linear_loaded(self.ctx.handle, self.handle, ptr(y), ptr(bias), tactic))

    def release(self) -> None:
        if self.handle:
            check(lib().air_hip_matrix_release(self.handle))
            self.handle = None
