"""TokenService through the host C ABI (include/air_host.h).

cpu: libair_host.so loads and exports every entry point air_host.h declares,
     with a Python signature for each; argument errors come back as statuses.
gpu: cohorts of greedy requests on synthetic Qwen2 models reproduce the
     greedy tokens of AIR's ReferenceExecutor (tests/golden/qwen2_tiny.txt,
     written by tests/golden/make_qwen2_golden.cpp), through both prompt
     tactics; a cohort wider than the decode width (64) gives each request the
     tokens it gets alone; capacity and validation errors fail the cohort
     before any work.
"""
import ctypes
import os
import re

import pytest

from air_amd import capi, host_api

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
GOLDEN = os.path.join(ROOT, "tests", "golden", "qwen2_tiny.txt")


def _declared():
    with open(os.path.join(ROOT, "include", "air_host.h")) as f:
        text = f.read()
    return sorted(set(re.findall(r"^\s*(?:int|const char\*)\s+(air_host_\w+)\(", text, re.M)))


def test_host_library_exports_every_declared_entry_point():
    lib = host_api.lib()
    declared = _declared()
    assert len(declared) == 14
    for name in declared:
        assert hasattr(lib, name), name
    assert set(host_api.SIGNATURES) == set(declared)
    assert lib.air_host_abi_version() == 1


def test_host_argument_errors():
    lib = host_api.lib()
    out = ctypes.c_void_p()
    assert lib.air_host_synthetic_qwen2(None, ctypes.byref(out)) == 1
    assert b"must not be null" in lib.air_host_last_error()
    with pytest.raises(capi.HipError) as e:
        host_api.Model.synthetic_qwen2(layers=1, embedding=100, ffn=64, heads=0, kv_heads=0, vocab=10)
    assert e.value.status_name == "invalid_argument"


def test_synthetic_model_describes_itself():
    m = host_api.Model.synthetic_qwen2(layers=1, embedding=64, ffn=128, heads=2, kv_heads=1, vocab=96, context=32)
    storage, tensors = m.describe()
    # token_embd, output_norm, output, then 10 tensors per layer (+3 biases).
    assert tensors == 3 + 12
    assert storage > 64 * 96
    m.close()


def _golden_cases():
    cases, case = [], None
    with open(GOLDEN) as f:
        for line in f:
            parts = line.split()
            if not parts or parts[0].startswith("#"):
                continue
            tag = parts[0]
            if tag == "case":
                case = {"name": parts[1], "sequences": []}
                cases.append(case)
            elif tag == "config":
                case["config"] = [int(v) for v in parts[1:8]]
            elif tag == "weights":
                case["weights"] = [int(v) for v in parts[1:7]]
            elif tag == "sequence":
                case["sequences"].append({"prompt": [int(v) for v in parts[2:]]})
            elif tag == "generated":
                case["sequences"][-1]["generated"] = [int(v) for v in parts[2:]]
    return cases


def _golden_model(case):
    layers, e, ffn, heads, kv, vocab, ctx = case["config"]
    wf, ef, seed, qkv_bias, out_bias, tied = case["weights"]
    return host_api.Model.synthetic_qwen2(layers, e, ffn, heads, kv, vocab, ctx, wf, ef, seed, 0.02,
                                          bool(qkv_bias), bool(out_bias), bool(tied))


def test_golden_cases_parse():
    cases = _golden_cases()
    assert [c["name"] for c in cases] == ["q8_0", "q4_0_tied", "q4_k"]
    assert all(len(s["generated"]) == 6 for c in cases for s in c["sequences"])


@pytest.mark.gpu
@pytest.mark.parametrize("tactic", [capi.LINEAR_DECODE, capi.LINEAR_PREFILL])
@pytest.mark.parametrize("attention", [host_api.ATTENTION_BASELINE, host_api.ATTENTION_ONLINE])
def test_cohort_reproduces_reference_tokens(torch_cuda, tactic, attention):
    for case in _golden_cases():
        print("cohort", case["name"], "tactic", tactic, "attention", attention, flush=True)
        model = _golden_model(case)
        engine = host_api.Engine(model, prefill_tactic=tactic, page_tokens=4, kv_pool_pages=64,
                                 prefill_quantum_tokens=3, token_budget_per_cycle=5, attention=attention)
        prompts = [s["prompt"] for s in case["sequences"]]
        tokens, stats = engine.generate_cohort(prompts, 6)
        assert tokens == [s["generated"] for s in case["sequences"]], case["name"]
        assert stats.generated_tokens == 6 * len(prompts)
        assert stats.prefill_tokens == sum(len(p) for p in prompts)
        # Quantum 3 and budget 5: prompts arrive in several prefill calls.
        assert stats.prefill_calls >= 2
        engine.close()
        model.close()


@pytest.mark.gpu
def test_wide_cohort_matches_single_requests(torch_cuda):
    model = host_api.Model.synthetic_qwen2(layers=2, embedding=256, ffn=512, heads=4, kv_heads=2, vocab=512,
                                           context=96, seed=0x5EED)
    engine = host_api.Engine(model, prefill_tactic=capi.LINEAR_DECODE, page_tokens=16,
                             max_active_requests=80, token_budget_per_cycle=512, prefill_quantum_tokens=64)
    prompts = [[(7 * i + 3 * j) % 512 for j in range(1 + (i * 5) % 23)] for i in range(70)]
    print("wide cohort of 70", flush=True)
    tokens, stats = engine.generate_cohort(prompts, 8)
    assert stats.max_decode_width == 64          # the advertised width bounds each launch
    assert stats.decode_rows == 70 * 7
    alone = [engine.generate_cohort([p], 8)[0][0] for p in prompts[:6]]
    assert tokens[:6] == alone
    # A stop token ends a request early.
    stop = tokens[0][2]
    stopped, _ = engine.generate_cohort([prompts[0]], 8, stop_token=stop)
    assert stopped[0] == tokens[0][:tokens[0].index(stop) + 1]
    engine.close()
    model.close()


@pytest.mark.gpu
def test_cohort_validation_fails_before_work(torch_cuda):
    model = host_api.Model.synthetic_qwen2(layers=1, embedding=256, ffn=512, heads=4, kv_heads=2, vocab=512,
                                           context=32)
    engine = host_api.Engine(model, prefill_tactic=capi.LINEAR_DECODE, page_tokens=16, kv_pool_pages=4)
    with pytest.raises(capi.HipError) as e:
        engine.generate_cohort([[1, 2, 3], [5] * 30], 4)       # 30 + 4 > context 32
    assert "context length" in str(e.value)
    with pytest.raises(capi.HipError) as e:
        engine.generate_cohort([[1, 600]], 4)                  # token outside the vocabulary
    assert e.value.status_name == "invalid_argument"
    # Pool of 4 pages x 16 tokens: two 20+8-token requests need 2 pages each
    # and fit; the service runs them and the pool is whole afterwards.
    tokens, _ = engine.generate_cohort([[1] * 20, [2] * 20], 8)
    assert [len(t) for t in tokens] == [8, 8]
    tokens2, _ = engine.generate_cohort([[1] * 20, [2] * 20, [3] * 20], 8)
    assert tokens2[:2] == tokens                                # the third waits for pages, same results
    engine.close()
    model.close()


@pytest.mark.gpu
def test_capacity_is_free_plus_growing_pool_at_7b_width(torch_cuda):
    """By default the KV pool grows on demand in chunks (each its own
    allocation, named in a device chunk table), so sequence_capacity_bytes
    answers the device memory free plus the pool allocated, the reference's
    answer (src/runtime/backend.cpp:541-560), and admission sees the whole
    HBM.  With one-page chunks every page boundary a decode step crosses adds
    a chunk between graph replays; the greedy tokens must equal those of a
    fixed pool that never grows.  Qwen2-7B widths (hidden 3584, 28 / 4 heads
    of 128, FFN 18944), two layers."""
    model = host_api.Model.synthetic_qwen2(layers=2, embedding=3584, ffn=18944, heads=28, kv_heads=4, vocab=1024,
                                           context=4096)
    page_bytes = 2 * 2 * 16 * 512 * 4                  # layers x (K, V) x page tokens x kv width x f32
    prompts = [[(13 * i + 7 * j) % 1024 for j in range(14)] for i in range(3)]
    fixed = host_api.Engine(model, page_tokens=16, kv_pool_pages=64)
    expect, _ = fixed.generate_cohort(prompts, 40)
    fixed.close()

    engine = host_api.Engine(model, page_tokens=16, kv_chunk_pages=1)
    before = engine.capacity()
    assert before["kv_pool_allocated_bytes"] == 0
    assert before["sequence_capacity_bytes"] == before["free_device_bytes"]
    assert before["sequence_capacity_bytes"] > 64 * 2**30    # most of the HBM, not a pool sized up front
    tokens, stats = engine.generate_cohort(prompts, 40)
    assert tokens == expect, "graph replays after pool growth differ from a fixed pool"
    assert stats.max_decode_width == 3
    after = engine.capacity()
    # 54 tokens per sequence: 4 pages each, every one a chunk of its own.
    assert after["kv_pool_allocated_bytes"] == 12 * page_bytes
    assert after["kv_pool_free_bytes"] == after["kv_pool_allocated_bytes"]
    assert after["sequence_capacity_bytes"] == after["free_device_bytes"] + after["kv_pool_allocated_bytes"]
    print(f"7B-width growing pool: capacity {after['sequence_capacity_bytes']} B, "
          f"{after['kv_pool_allocated_bytes']} B allocated in 12 chunks", flush=True)
    engine.close()
    model.close()


@pytest.mark.gpu
def test_admission_holds_to_a_fixed_pool_at_7b_width(torch_cuda):
    """A pool of a fixed page count (kv_pool_pages) is one allocation made
    with the first sequence and never grows, so sequence_capacity_bytes
    answers that pool and admission reserves every request's forecast
    (PreparedModel::estimate_sequence_device_bytes) against it: a cohort
    larger than the pool runs at most capacity // forecast requests at once
    and finishes, with the pool whole afterwards.  Qwen2-7B widths, two
    layers."""
    model = host_api.Model.synthetic_qwen2(layers=2, embedding=3584, ffn=18944, heads=28, kv_heads=4, vocab=1024,
                                           context=4096)
    page_bytes = 2 * 2 * 16 * 512 * 4

    # A pool of 12 pages (192 tokens): 48-token requests (3 pages + the
    # page table) fit three at a time.
    engine = host_api.Engine(model, page_tokens=16, kv_pool_pages=12)
    capacity = engine.capacity()["sequence_capacity_bytes"]
    assert capacity == 12 * page_bytes
    forecast = engine.sequence_bytes(48)
    assert forecast == 3 * page_bytes + (4096 // 16) * 2 * 8
    fits = capacity // forecast
    assert fits == 3
    prompts = [[(11 * i + j) % 1024 for j in range(40)] for i in range(8)]
    print(f"7B-width admission: capacity {capacity} B, forecast {forecast} B, {fits} at a time", flush=True)
    tokens, stats = engine.generate_cohort(prompts, 8)
    assert [len(t) for t in tokens] == [8] * 8
    assert all(0 <= t < 1024 for seq in tokens for t in seq)
    assert stats.max_decode_width <= fits and stats.max_prefill_sequences <= fits
    end = engine.capacity()
    assert end["kv_pool_allocated_bytes"] == end["kv_pool_free_bytes"] == capacity
    engine.close()
    model.close()
