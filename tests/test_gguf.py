"""GGUF v3 reader, loader and writer (air_amd/host/src/gguf.cpp via include/air_host.h).

cpu: the cases of AIR's own GGUF tests (tests/core_tests.cpp:80-265: load and
     mapping, sliding-window metadata, version 2 refused, an unknown tensor
     encoding kept inspectable with its storage span, an out-of-vocabulary
     special token refused) on files built byte by byte here; the malformed
     headers AIR's reader refuses (gguf_reader.cpp:346-472) with the same
     error classes; every file also loaded by AIR's own GgufFormat::load
     (compiled into oracle/_ref) with the same outcome, config and tensor
     table; write -> load -> write reproduces the file byte for byte.
gpu: a synthetic model written to GGUF and loaded back generates the
     reference's golden greedy tokens through the token service.
"""
import os
import struct

import numpy as np
import pytest

import oracle
from air_amd import capi, host_api

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))

IO_ERROR, INVALID_ARGUMENT, DATA_ERROR, UNSUPPORTED = 3, 1, 5, 6


class GgufBytes:
    """Little-endian GGUF builder for test files (metadata, tensor infos, data)."""

    def __init__(self, version=3, alignment=32):
        self.version, self.alignment = version, alignment
        self.kv, self.infos, self.data = [], [], bytearray()

    @staticmethod
    def _str(s):
        b = s.encode()
        return struct.pack("<Q", len(b)) + b

    def string(self, k, v):
        self.kv.append(self._str(k) + struct.pack("<I", 8) + self._str(v))

    def u32(self, k, v):
        self.kv.append(self._str(k) + struct.pack("<II", 4, v))

    def f32(self, k, v):
        self.kv.append(self._str(k) + struct.pack("<If", 6, v))

    def i32(self, k, v):
        self.kv.append(self._str(k) + struct.pack("<Ii", 5, v))

    def boolean(self, k, v):
        self.kv.append(self._str(k) + struct.pack("<IB", 7, 1 if v else 0))

    def strings(self, k, vals):
        self.kv.append(self._str(k) + struct.pack("<IIQ", 9, 8, len(vals)) + b"".join(self._str(v) for v in vals))

    def raw_kv(self, blob):
        self.kv.append(blob)

    def tensor(self, name, dims, ggml_type, payload, offset=None):
        if offset is None:
            offset = len(self.data) + (-len(self.data)) % self.alignment
        if payload:
            end = offset + len(payload)
            if end > len(self.data):
                self.data.extend(b"\0" * (end - len(self.data)))
            self.data[offset:end] = payload
        self.infos.append(self._str(name) + struct.pack("<I", len(dims)) + b"".join(struct.pack("<Q", d) for d in dims)
                          + struct.pack("<IQ", ggml_type, offset))

    def build(self):
        head = b"GGUF" + struct.pack("<IQQ", self.version, len(self.infos), len(self.kv))
        body = head + b"".join(self.kv) + b"".join(self.infos)
        body += b"\0" * ((-len(body)) % self.alignment)
        return body + bytes(self.data)


def tiny_qwen2(version=3, tensor_type=0, bos=0, window=0):
    """The shape of AIR's core_tests.cpp write_test_gguf: one 4x2 f32 tensor."""
    g = GgufBytes(version)
    g.string("general.architecture", "qwen2")
    g.string("general.name", "AIR synthetic model")
    g.u32("general.alignment", 32)
    g.u32("qwen2.block_count", 1)
    g.u32("qwen2.context_length", 128)
    g.u32("qwen2.embedding_length", 4)
    g.u32("qwen2.feed_forward_length", 8)
    g.u32("qwen2.attention.head_count", 2)
    g.u32("qwen2.attention.head_count_kv", 1)
    if window:
        g.u32("qwen2.attention.sliding_window", window)
    g.u32("qwen2.rope.dimension_count", 2)
    g.f32("qwen2.rope.freq_base", 1000000.0)
    g.f32("qwen2.attention.layer_norm_rms_epsilon", 0.000001)
    g.string("tokenizer.ggml.model", "gpt2")
    g.string("tokenizer.ggml.pre", "gpt2")
    g.strings("tokenizer.ggml.tokens", ["a", "b"])
    g.strings("tokenizer.ggml.merges", [])
    g.u32("tokenizer.ggml.bos_token_id", bos)
    g.u32("tokenizer.ggml.eos_token_id", 1)
    g.boolean("tokenizer.ggml.add_bos_token", False)
    g.tensor("token_embd.weight", [4, 2], tensor_type, struct.pack("<8f", *range(8)))
    return g


def _write(tmp_path, name, blob):
    p = tmp_path / name
    p.write_bytes(blob)
    return str(p)


def _load_status(path):
    try:
        m = host_api.Model.load_gguf(path)
    except capi.HipError as e:
        return e.status, None
    return 0, m


def _agrees_with_reference(path, status, model):
    """AIR's own loader on the same file: same outcome, config and tensor table."""
    if not oracle.ref_available():
        return
    rc, cfg, table = oracle.ref_gguf_load(path)
    assert rc == status, (rc, status)
    if status != 0:
        return
    ours = model.config()
    for key in ("layers", "embedding", "ffn", "heads", "kv_heads", "rope_dims", "vocab", "context",
                "sliding_window", "rope_base", "rms_eps", "eos", "tensors"):
        assert ours[key] == cfg[key], key
    assert [(t[3], t[4], t[1]) for t in model.tensors()] == table


def test_load_and_mapping(tmp_path):
    path = _write(tmp_path, "tiny.gguf", tiny_qwen2().build())
    status, m = _load_status(path)
    assert status == 0
    cfg = m.config()
    assert (cfg["layers"], cfg["ffn"], cfg["vocab"], cfg["embedding"]) == (1, 8, 2, 4)
    assert cfg["eos"] == 1 and cfg["rope_base"] == 1000000.0
    name, ggml_type, dims, offset, size = m.tensors()[0]
    assert (name, ggml_type, dims, size) == ("token_embd.weight", 0, [4, 2], 32)
    storage, count = m.describe()
    assert storage == os.path.getsize(path) and count == 1     # the whole file is mapped
    raw = open(path, "rb").read()
    assert struct.unpack("<8f", raw[offset:offset + 32]) == tuple(float(i) for i in range(8))
    _agrees_with_reference(path, 0, m)


def test_sliding_window_is_kept(tmp_path):
    path = _write(tmp_path, "window.gguf", tiny_qwen2(window=64).build())
    status, m = _load_status(path)
    assert status == 0 and m.config()["sliding_window"] == 64
    _agrees_with_reference(path, 0, m)


def test_version_2_is_unsupported(tmp_path):
    path = _write(tmp_path, "v2.gguf", tiny_qwen2(version=2).build())
    assert _load_status(path)[0] == UNSUPPORTED
    _agrees_with_reference(path, UNSUPPORTED, None)


def test_unknown_encoding_keeps_its_span(tmp_path):
    path = _write(tmp_path, "t99.gguf", tiny_qwen2(tensor_type=99).build())
    status, m = _load_status(path)
    assert status == 0
    _, ggml_type, _, _, size = m.tensors()[0]
    assert ggml_type == 99 and size == 32                     # the span up to the end of the file
    _agrees_with_reference(path, 0, m)


def test_special_token_outside_vocabulary(tmp_path):
    path = _write(tmp_path, "bos99.gguf", tiny_qwen2(bos=99).build())
    assert _load_status(path)[0] == DATA_ERROR
    _agrees_with_reference(path, DATA_ERROR, None)


def _malformed():
    cases = {}
    g = tiny_qwen2()
    cases["not_gguf"] = (b"GGUX" + g.build()[4:], INVALID_ARGUMENT)
    cases["truncated"] = (g.build()[:40], DATA_ERROR)
    g = tiny_qwen2()
    g.u32("general.name", 5)                                         # duplicate key
    cases["duplicate_key"] = (g.build(), DATA_ERROR)
    g = tiny_qwen2()
    g.raw_kv(GgufBytes._str("x.bad") + struct.pack("<I", 13))        # value type 13
    cases["bad_value_type"] = (g.build(), DATA_ERROR)
    g = tiny_qwen2()
    g.raw_kv(GgufBytes._str("x.nested") + struct.pack("<IIQ", 9, 9, 1))
    cases["nested_array"] = (g.build(), DATA_ERROR)
    g = tiny_qwen2()
    g.kv = [kv for kv in g.kv if b"general.alignment" not in kv]
    g.u32("general.alignment", 48)
    cases["alignment_not_power_of_two"] = (g.build(), DATA_ERROR)
    g = tiny_qwen2()
    g.u32("split.count", 2)
    cases["split"] = (g.build(), UNSUPPORTED)
    g = tiny_qwen2()
    g.tensor("token_embd.weight", [4, 2], 0, b"\0" * 32)
    cases["duplicate_tensor"] = (g.build(), DATA_ERROR)
    g = tiny_qwen2()
    g.tensor("zero", [4, 0], 0, b"")
    cases["zero_dimension"] = (g.build(), DATA_ERROR)
    g = tiny_qwen2()
    g.tensor("big", [64, 4], 8, b"\0" * 20)                         # Q8_0 needs 272 bytes, 20 remain
    cases["overlap"] = (g.build(), DATA_ERROR)
    g = tiny_qwen2()
    g.kv = [kv for kv in g.kv if b"tokenizer.ggml.tokens" not in kv]
    cases["no_tokens"] = (g.build(), DATA_ERROR)
    g = tiny_qwen2()
    g.kv = [kv for kv in g.kv if b"qwen2.block_count" not in kv]
    cases["no_block_count"] = (g.build(), DATA_ERROR)
    g = tiny_qwen2()
    g.u32("qwen2.vocab_size", 3)
    cases["vocab_disagrees"] = (g.build(), DATA_ERROR)
    g = tiny_qwen2()
    g.tensor("far", [4], 0, b"", offset=1 << 20)                    # offset past the data blob
    cases["offset_past_end"] = (g.build(), DATA_ERROR)
    return cases


@pytest.mark.parametrize("case", sorted(_malformed()))
def test_malformed_files_are_refused(tmp_path, case):
    blob, expected = _malformed()[case]
    path = _write(tmp_path, case + ".gguf", blob)
    assert _load_status(path)[0] == expected
    _agrees_with_reference(path, expected, None)


def test_missing_file_is_io_error(tmp_path):
    assert _load_status(str(tmp_path / "absent.gguf"))[0] == IO_ERROR


@pytest.mark.parametrize("weight_format,tied,bias", [(8, False, True), (2, True, False), (12, False, False),
                                                    (14, False, False), (6, True, False), (1, False, True),
                                                    (30, False, False)])
def test_written_model_round_trips(tmp_path, weight_format, tied, bias):
    m = host_api.Model.synthetic_qwen2(2, 256, 512, 4, 2, 600, context=96, weight_format=weight_format,
                                       embedding_format=8, seed=77 + weight_format, qkv_bias=bias,
                                       output_bias=bias, tied_output=tied)
    first = str(tmp_path / "a.gguf")
    m.write_gguf(first, eos=5)
    loaded = host_api.Model.load_gguf(first)
    assert {k: v for k, v in loaded.config().items() if k != "eos"} == \
        {k: v for k, v in m.config().items() if k != "eos"}
    assert loaded.config()["eos"] == 5
    ours = m.tensors()
    back = loaded.tensors()
    assert [(t[0], t[1], t[2], t[4]) for t in ours] == [(t[0], t[1], t[2], t[4]) for t in back]
    assert all(t[3] % 32 == 0 for t in back)                            # aligned tensor data
    second = str(tmp_path / "b.gguf")
    loaded.write_gguf(second, eos=5)
    assert open(first, "rb").read() == open(second, "rb").read()
    _agrees_with_reference(first, 0, loaded)


@pytest.mark.parametrize("weight_format", [8, 12])
def test_truncated_and_corrupted_files(tmp_path, weight_format):
    """A written model cut short anywhere is refused (the header byte by
    byte, the tensor data in strides), and single-byte corruptions of the
    header either load or are refused with a status -- never a crash; the
    same files under AddressSanitizer and UBSan: `make -C tests/host
    sanitize`."""
    m = host_api.Model.synthetic_qwen2(1, 256, 512, 4, 2, 64, context=64, weight_format=weight_format,
                                       embedding_format=weight_format, seed=3)
    good = str(tmp_path / "good.gguf")
    m.write_gguf(good, eos=2)
    blob = open(good, "rb").read()
    bad = tmp_path / "bad.gguf"
    header = blob.find(b"token_embd.weight") + 256           # past the first tensor's record
    cuts = list(range(0, header)) + list(range(header, len(blob), 4099))
    for n in cuts:
        bad.write_bytes(blob[:n])
        status, model = _load_status(str(bad))
        assert status != 0 and model is None, n
    rng = np.random.default_rng(weight_format)
    outcomes = set()
    for _ in range(400):
        b = bytearray(blob)
        b[int(rng.integers(0, header))] = int(rng.integers(0, 256))
        bad.write_bytes(bytes(b))
        status, model = _load_status(str(bad))
        outcomes.add(status)
        if model is not None:
            model.close()
    assert 0 in outcomes and len(outcomes) > 1, outcomes


@pytest.mark.gpu
def test_gguf_model_generates_reference_tokens(torch_cuda, tmp_path):
    from test_service import _golden_cases, _golden_model
    for case in _golden_cases():
        path = str(tmp_path / (case["name"] + ".gguf"))
        _golden_model(case).write_gguf(path)
        model = host_api.Model.load_gguf(path)
        engine = host_api.Engine(model, prefill_tactic=capi.LINEAR_DECODE, page_tokens=16, kv_pool_pages=16)
        tokens, _ = engine.generate_cohort([s["prompt"] for s in case["sequences"]], 6)
        assert tokens == [s["generated"] for s in case["sequences"]], case["name"]
        engine.close()
        model.close()
