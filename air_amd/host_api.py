"""ctypes binding of libair_host.so (the C ABI declared in include/air_host.h).

The host library is the C++ executor: model definitions, the HIP prepared
model with its Qwen2 step engine and paged KV, and TokenService, the token-id
caller slice of AIR's InferenceService (src/runtime/serving.cpp:2401-2481).
Importing this module fails loudly when the library has not been built; no
part of it falls back to Python or CPU compute.
"""
from __future__ import annotations

import ctypes
import os
from typing import List, Optional, Sequence

from . import capi

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libair_host.so")

_P = ctypes.c_void_p
_PP = ctypes.POINTER(ctypes.c_void_p)
_U32 = ctypes.c_uint32
_U64 = ctypes.c_uint64
_I32 = ctypes.c_int32
_I = ctypes.c_int


class Qwen2Spec(ctypes.Structure):
    _fields_ = [
        ("layers", _U32), ("embedding", _U32), ("ffn", _U32), ("heads", _U32), ("kv_heads", _U32),
        ("vocab", _U64), ("context", _U64), ("weight_format", _U32), ("embedding_format", _U32),
        ("seed", _U64), ("sigma", ctypes.c_float), ("qkv_bias", _I32), ("output_bias", _I32),
        ("tied_output", _I32),
    ]


class ModelConfig(ctypes.Structure):
    _fields_ = [
        ("layers", _U32), ("embedding", _U32), ("ffn", _U32), ("heads", _U32), ("kv_heads", _U32),
        ("rope_dims", _U32), ("vocab", _U64), ("context", _U64), ("sliding_window", _U64),
        ("rope_base", ctypes.c_double), ("rms_eps", ctypes.c_double), ("eos", _I32), ("tensors", _U32),
    ]

    def as_dict(self) -> dict:
        return {name: getattr(self, name) for name, _ in self._fields_}


class TensorInfo(ctypes.Structure):
    _fields_ = [
        ("name", ctypes.c_char_p), ("type", _U32), ("rank", _U32), ("dims", _U64 * 8),
        ("offset", _U64), ("size", _U64),
    ]


class EngineConfig(ctypes.Structure):
    _fields_ = [
        ("device", _I32), ("page_tokens", _U32), ("kv_pool_pages", _U32), ("max_step_rows", _U32),
        ("prefill_tactic", _I32), ("prefill_quantum_tokens", _U32), ("token_budget_per_cycle", _U32),
        ("max_active_requests", _U32), ("attention_tactic", _I32), ("eager_decode", _I32),
        ("kv_chunk_pages", _U32),
    ]


class Capacity(ctypes.Structure):
    _fields_ = [("sequence_capacity_bytes", _U64), ("free_device_bytes", _U64), ("kv_pool_allocated_bytes", _U64),
                ("kv_pool_free_bytes", _U64)]


class CohortStats(ctypes.Structure):
    _fields_ = [
        ("wall_ms", ctypes.c_double), ("prefill_ms", ctypes.c_double), ("decode_ms", ctypes.c_double),
        ("cycles", _U64), ("prefill_calls", _U64), ("prefill_tokens", _U64), ("decode_calls", _U64),
        ("decode_rows", _U64), ("max_decode_width", _U32), ("max_prefill_sequences", _U32),
        ("generated_tokens", _U64), ("mean_ttft_ms", ctypes.c_double),
    ]

    def as_dict(self) -> dict:
        return {name: getattr(self, name) for name, _ in self._fields_}


# Every exported entry point of include/air_host.h: name -> (restype, argtypes).
SIGNATURES = {
    "air_host_abi_version": (_I, []),
    "air_host_last_error": (ctypes.c_char_p, []),
    "air_host_synthetic_qwen2": (_I, [ctypes.POINTER(Qwen2Spec), _PP]),
    "air_host_model_describe": (_I, [_P, ctypes.POINTER(_U64), ctypes.POINTER(_U64)]),
    "air_host_model_release": (_I, [_P]),
    "air_host_load_gguf": (_I, [ctypes.c_char_p, _PP]),
    "air_host_write_gguf": (_I, [_P, ctypes.c_char_p, _I32]),
    "air_host_model_get_config": (_I, [_P, ctypes.POINTER(ModelConfig)]),
    "air_host_model_tensor": (_I, [_P, _U32, ctypes.POINTER(TensorInfo)]),
    "air_host_engine_create": (_I, [_P, ctypes.POINTER(EngineConfig), _PP]),
    "air_host_engine_release": (_I, [_P]),
    "air_host_engine_capacity": (_I, [_P, ctypes.POINTER(Capacity)]),
    "air_host_engine_sequence_bytes": (_I, [_P, _U64, ctypes.POINTER(_U64)]),
    "air_host_generate_cohort": (_I, [_P, ctypes.POINTER(_I32), ctypes.POINTER(_U32), _U32, _U32, _I32,
                                      ctypes.POINTER(_I32), ctypes.POINTER(_U32), ctypes.POINTER(CohortStats)]),
}

ATTENTION_BASELINE = 0   # the reference executor's double-precision softmax
ATTENTION_ONLINE = 1     # tiled f32 online softmax

_lib: Optional[ctypes.CDLL] = None


def lib() -> ctypes.CDLL:
    """The loaded host library (libair_hip.so is loaded first, as its dependency)."""
    global _lib
    if _lib is None:
        capi.lib()
        if not os.path.exists(LIB_PATH):
            raise ImportError(f"{LIB_PATH} is not built; run __graft_entry__.build()")
        handle = ctypes.CDLL(LIB_PATH)
        for name, (restype, argtypes) in SIGNATURES.items():
            fn = getattr(handle, name)
            fn.restype = restype
            fn.argtypes = argtypes
        _lib = handle
    return _lib


def check(status: int) -> None:
    if status != capi.AIR_HIP_OK:
        message = lib().air_host_last_error().decode(errors="replace")
        raise capi.HipError(status, message)


class Model:
    """A model definition held by the host library."""

    def __init__(self, handle: int):
        self.handle = handle

    @classmethod
    def synthetic_qwen2(cls, layers: int, embedding: int, ffn: int, heads: int, kv_heads: int, vocab: int,
                        context: int = 4096, weight_format: int = capi.TYPE_Q8_0,
                        embedding_format: int = capi.TYPE_Q8_0, seed: int = 0xA17C0DE, sigma: float = 0.02,
                        qkv_bias: bool = True, output_bias: bool = False, tied_output: bool = False) -> "Model":
        spec = Qwen2Spec(layers, embedding, ffn, heads, kv_heads, vocab, context, weight_format,
                         embedding_format, seed, sigma, int(qkv_bias), int(output_bias), int(tied_output))
        out = ctypes.c_void_p()
        check(lib().air_host_synthetic_qwen2(ctypes.byref(spec), ctypes.byref(out)))
        return cls(out.value)

    @classmethod
    def load_gguf(cls, path: str) -> "Model":
        """A GGUF v3 file, memory-mapped (AIR's GgufFormat::load rules)."""
        out = ctypes.c_void_p()
        check(lib().air_host_load_gguf(os.fsencode(path), ctypes.byref(out)))
        return cls(out.value)

    def write_gguf(self, path: str, eos: int = -1) -> None:
        check(lib().air_host_write_gguf(self.handle, os.fsencode(path), eos))

    def config(self) -> dict:
        out = ModelConfig()
        check(lib().air_host_model_get_config(self.handle, ctypes.byref(out)))
        return out.as_dict()

    def tensors(self) -> list:
        """[(name, ggml type, dims, byte offset, byte size)] in table order."""
        out = []
        for i in range(self.config()["tensors"]):
            t = TensorInfo()
            check(lib().air_host_model_tensor(self.handle, i, ctypes.byref(t)))
            out.append((t.name.decode(), t.type, [t.dims[d] for d in range(t.rank)], t.offset, t.size))
        return out

    def describe(self):
        storage, tensors = _U64(), _U64()
        check(lib().air_host_model_describe(self.handle, ctypes.byref(storage), ctypes.byref(tensors)))
        return storage.value, tensors.value

    def close(self) -> None:
        if self.handle:
            lib().air_host_model_release(self.handle)
            self.handle = None

    def __del__(self):  # pragma: no cover - interpreter shutdown order
        try:
            self.close()
        except Exception:
            pass


class Engine:
    """A prepared model on one device plus its token service."""

    def __init__(self, model: Model, device: int = 0, page_tokens: int = 16, kv_pool_pages: int = 0,
                 max_step_rows: int = 512, prefill_tactic: int = capi.LINEAR_PREFILL,
                 prefill_quantum_tokens: int = 512, token_budget_per_cycle: int = 512,
                 max_active_requests: int = 64, attention: int = ATTENTION_ONLINE, eager_decode: bool = False,
                 kv_chunk_pages: int = 0):
        # kv_pool_pages 0: the KV pool grows in chunks of kv_chunk_pages pages
        # (0: about 256 MiB) and capacity is free device memory plus the pool.
        config = EngineConfig(device, page_tokens, kv_pool_pages, max_step_rows, prefill_tactic,
                              prefill_quantum_tokens, token_budget_per_cycle, max_active_requests, attention,
                              int(eager_decode), kv_chunk_pages)
        out = ctypes.c_void_p()
        check(lib().air_host_engine_create(model.handle, ctypes.byref(config), ctypes.byref(out)))
        self.handle = out.value

    def generate_cohort(self, prompts: Sequence[Sequence[int]], max_new_tokens: int,
                        stop_token: int = -1):
        """Greedy tokens of every prompt (list of lists) and the cohort's CohortStats."""
        n = len(prompts)
        flat = [int(t) for p in prompts for t in p]
        tokens = (_I32 * max(len(flat), 1))(*flat)
        lengths = (_U32 * max(n, 1))(*[len(p) for p in prompts])
        out = (_I32 * max(n * max_new_tokens, 1))()
        counts = (_U32 * max(n, 1))()
        stats = CohortStats()
        check(lib().air_host_generate_cohort(self.handle, tokens, lengths, n, max_new_tokens, stop_token, out,
                                             counts, ctypes.byref(stats)))
        result: List[List[int]] = []
        for i in range(n):
            result.append([out[i * max_new_tokens + t] for t in range(counts[i])])
        return result, stats

    def capacity(self) -> dict:
        """sequence_capacity_bytes, free_device_bytes, kv_pool_allocated_bytes, kv_pool_free_bytes."""
        c = Capacity()
        check(lib().air_host_engine_capacity(self.handle, ctypes.byref(c)))
        return {name: getattr(c, name) for name, _ in Capacity._fields_}

    def sequence_bytes(self, tokens: int) -> int:
        """Device bytes admission reserves for a request of `tokens` prompt + generated tokens."""
        out = _U64()
        check(lib().air_host_engine_sequence_bytes(self.handle, tokens, ctypes.byref(out)))
        return out.value

    def close(self) -> None:
        if self.handle:
            lib().air_host_engine_release(self.handle)
            self.handle = None

    def __del__(self):  # pragma: no cover
        try:
            self.close()
        except Exception:
            pass
