"""The two attention tactics over the paged fp32 KV pool.

cpu: tile construction of the online tactic (air_hip_attention_make_tiles).
gpu: at Qwen2-7B head geometry (28 q heads, 4 KV heads of 128) and at the
     0.5B-like geometry of the tiny models (head 64), one step mixing decode
     rows of many lengths with a 100-row prompt run: the online tactic equals
     the baseline (the reference executor's double softmax) within 1e-5
     relative, and both equal a float64 CPU attention computed from the same
     pool.  Split tiles (few rows, long keys) go through the merge pass;
     steps of more than 64 rows take the f32 MFMA kernel.
"""
import ctypes

import numpy as np
import pytest

from air_amd import capi
from tests import helpers


def test_tiles_for_decode_and_prefill_runs():
    # Two decode rows at 7B geometry: one tile per KV head with its 7 q heads.
    tiles = capi.attention_tiles([1, 1], 28, 4)
    assert tiles == [(r, 1, 7 * h, 7) for r in range(2) for h in range(4)]
    # A 37-row prompt run: 16-row tiles of one q head, the last rows first.
    tiles = capi.attention_tiles([37], 4, 2)
    assert tiles == [(r, min(16, 37 - r), h, 1) for r in (32, 16, 0) for h in range(4)]
    # Mixed: rows continue across runs.
    tiles = capi.attention_tiles([1, 20], 2, 2)
    assert tiles[:2] == [(0, 1, 0, 1), (0, 1, 1, 1)]
    assert tiles[2:] == [(17, 4, 0, 1), (17, 4, 1, 1), (1, 16, 0, 1), (1, 16, 1, 1)]
    with pytest.raises(capi.HipError):
        capi.attention_tiles([1], 6, 4)           # q heads not a multiple of KV heads
    with pytest.raises(capi.HipError):
        capi.attention_tiles([0], 4, 2)           # empty run


def _reference(pool, tables, positions, qkv, layer, q_heads, kv_heads, head, page_tokens, layers):
    """float64 attention of every row from the pool (CPU)."""
    kv_width = kv_heads * head
    m = len(positions)
    out = np.zeros((m, q_heads * head))
    pages = pool.reshape(-1, layers, 2, page_tokens, kv_width)
    for r in range(m):
        n = positions[r] + 1
        slots = [tables[r][t // page_tokens] for t in range(n)]
        k = np.stack([pages[slots[t], layer, 0, t % page_tokens] for t in range(n)]).astype(np.float64)
        v = np.stack([pages[slots[t], layer, 1, t % page_tokens] for t in range(n)]).astype(np.float64)
        for h in range(q_heads):
            g = h * kv_heads // q_heads
            q = qkv[r, h * head:(h + 1) * head].astype(np.float64)
            s = k[:, g * head:(g + 1) * head] @ q / np.sqrt(head)
            p = np.exp(s - s.max())
            out[r, h * head:(h + 1) * head] = (p / p.sum()) @ v[:, g * head:(g + 1) * head]
    return out


@pytest.mark.gpu
@pytest.mark.parametrize("q_heads,kv_heads,head,decode_lengths,prompt", [
    (28, 4, 128, [1, 17, 64, 65, 300, 700], (50, 100)),   # split tiles, merge pass
    (28, 4, 128, [3], (0, 60)),                           # one key chunk: no split
    (4, 2, 64, [1, 2, 63, 129], (0, 37)),
    (4, 2, 64, [1, 5, 300], (0, 90)),                     # over 64 rows: 64-key chunks on the matrix cores
])
def test_online_matches_baseline(torch_cuda, hip_ctx, q_heads, kv_heads, head, decode_lengths, prompt):
    torch = torch_cuda
    dev = torch.device("cuda:0")
    page_tokens, layers, layer = 16, 2, 1
    kv_width = kv_heads * head
    rng = np.random.default_rng(q_heads * 1000 + head)
    start, run = prompt
    lengths = decode_lengths + [start + run]
    max_tokens = max(lengths)
    max_pages = (max_tokens + page_tokens - 1) // page_tokens
    pool_pages = sum((n + page_tokens - 1) // page_tokens for n in lengths) + 3
    perm = rng.permutation(pool_pages)
    seq_tables, used = [], 0
    for n in lengths:
        need = (n + page_tokens - 1) // page_tokens
        seq_tables.append(list(perm[used:used + need]) + [-1] * (max_pages - need))
        used += need
    # Rows: one per decode sequence (its last token), then the prompt run.
    positions = [n - 1 for n in decode_lengths] + list(range(start, start + run))
    tables = seq_tables[:len(decode_lengths)] + [seq_tables[-1]] * run
    m = len(positions)
    print(f"attention q={q_heads} kv={kv_heads} head={head} rows={m} max_tokens={max_tokens}", flush=True)

    pool_h = rng.standard_normal(pool_pages * layers * 2 * page_tokens * kv_width).astype(np.float32)
    qkv_h = rng.standard_normal((m, q_heads * head + 2 * kv_width)).astype(np.float32)
    pool = torch.from_numpy(pool_h).to(dev)
    qkv = torch.from_numpy(qkv_h).to(dev)
    pos_d = torch.tensor(positions, dtype=torch.int32, device=dev)
    tab_d = torch.tensor(np.array(tables, dtype=np.int32), device=dev)
    kv = capi.KvLayout(pool.data_ptr(), page_tokens, kv_width, layers, max_pages, pool_pages)
    runs = [1] * len(decode_lengths) + [run]
    tiles_h = capi.attention_tiles(runs, q_heads, kv_heads)
    tiles_d = torch.tensor(np.array(tiles_h, dtype=np.uint32).view(np.int32), device=dev)
    out_base = torch.empty((m, q_heads * head), device=dev)
    out_online = torch.full((m, q_heads * head), float("nan"), device=dev)
    lib = capi.lib()
    stride = q_heads * head + 2 * kv_width
    capi.check(lib.air_hip_attention(hip_ctx.handle, ctypes.byref(kv), qkv.data_ptr(), stride, m, pos_d.data_ptr(),
                                     tab_d.data_ptr(), layer, q_heads, kv_heads, head, max_tokens,
                                     out_base.data_ptr()))
    capi.check(lib.air_hip_attention_online(hip_ctx.handle, ctypes.byref(kv), qkv.data_ptr(), stride, m,
                                            pos_d.data_ptr(), tab_d.data_ptr(), layer, q_heads, kv_heads, head,
                                            tiles_d.data_ptr(), len(tiles_h), max_tokens, out_online.data_ptr()))
    torch.cuda.synchronize()
    base = out_base.cpu().numpy().astype(np.float64)
    online = out_online.cpu().numpy().astype(np.float64)
    assert np.isfinite(online).all()
    ref = _reference(pool_h, tables, positions, qkv_h, layer, q_heads, kv_heads, head, page_tokens, layers)
    scale = np.abs(ref).max()
    assert np.abs(base - ref).max() <= 1e-6 * scale
    err = np.abs(online - ref).max() / scale
    assert err <= 1e-5, err
    # Per row relative L2 (each row's own softmax).
    rel = np.linalg.norm(online - base, axis=1) / np.linalg.norm(base, axis=1)
    assert rel.max() <= 1e-5, rel.max()


@pytest.mark.gpu
def test_online_rejects_bad_geometry(torch_cuda, hip_ctx):
    torch = torch_cuda
    dev = torch.device("cuda:0")
    pool = torch.zeros(4 * 2 * 2 * 16 * 96, device=dev)
    kv = capi.KvLayout(pool.data_ptr(), 16, 96, 2, 4, 4)
    qkv = torch.zeros((2, 3 * 96 + 2 * 96), device=dev)
    ints = torch.zeros(64, dtype=torch.int32, device=dev)
    out = torch.zeros((2, 3 * 96), device=dev)
    lib = capi.lib()
    status = lib.air_hip_attention_online(hip_ctx.handle, ctypes.byref(kv), qkv.data_ptr(), 5 * 96, 2,
                                          ints.data_ptr(), ints.data_ptr(), 0, 3, 1, 96, ints.data_ptr(), 1, 16,
                                          out.data_ptr())
    assert status == 6  # head width 96 is not compiled: unsupported
    assert b"64 and 128" in lib.air_hip_last_error()


@pytest.mark.gpu
@pytest.mark.parametrize("q_heads,kv_heads,head", [(28, 4, 128), (64, 2, 64), (4, 4, 64)])
def test_decode_rows_at_graph_max_tokens(torch_cuda, hip_ctx, q_heads, kv_heads, head):
    """Decode rows of distinct sequences (lengths 1 .. 2049) with max_tokens
    at the decode graphs' 4096 -- 64 key splits per tile, most of them past
    every row's keys, the merge taking only the live ones -- and at the
    step's own maximum: both within 1e-5 of the float64 attention.  Group
    sizes 7 (one tile per KV head), 32 (two tiles) and 1."""
    torch = torch_cuda
    dev = torch.device("cuda:0")
    page_tokens, layers, layer = 16, 2, 1
    kv_width = kv_heads * head
    lengths = [1, 5, 33, 700, 2049]
    max_pages = 4096 // page_tokens
    rng = np.random.default_rng(q_heads + head)
    pool_pages = sum((n + page_tokens - 1) // page_tokens for n in lengths) + 2
    perm = rng.permutation(pool_pages)
    tables, used = [], 0
    for n in lengths:
        need = (n + page_tokens - 1) // page_tokens
        tables.append(list(perm[used:used + need]) + [-1] * (max_pages - need))
        used += need
    positions = [n - 1 for n in lengths]
    m = len(positions)
    print(f"decode rows q={q_heads} kv={kv_heads} head={head} lengths={lengths}", flush=True)
    pool_h = rng.standard_normal(pool_pages * layers * 2 * page_tokens * kv_width).astype(np.float32)
    qkv_h = rng.standard_normal((m, q_heads * head + 2 * kv_width)).astype(np.float32)
    pool = torch.from_numpy(pool_h).to(dev)
    qkv = torch.from_numpy(qkv_h).to(dev)
    pos_d = torch.tensor(positions, dtype=torch.int32, device=dev)
    tab_d = torch.tensor(np.array(tables, dtype=np.int32), device=dev)
    kv = capi.KvLayout(pool.data_ptr(), page_tokens, kv_width, layers, max_pages, pool_pages)
    tiles_h = capi.attention_tiles([1] * m, q_heads, kv_heads)
    tiles_d = torch.tensor(np.array(tiles_h, dtype=np.uint32).view(np.int32), device=dev)
    stride = q_heads * head + 2 * kv_width
    lib = capi.lib()
    ref = _reference(pool_h, tables, positions, qkv_h, layer, q_heads, kv_heads, head, page_tokens, layers)
    for max_tokens in (4096, max(lengths)):
        out = torch.full((m, q_heads * head), float("nan"), device=dev)
        capi.check(lib.air_hip_attention_online(hip_ctx.handle, ctypes.byref(kv), qkv.data_ptr(), stride, m,
                                                pos_d.data_ptr(), tab_d.data_ptr(), layer, q_heads, kv_heads,
                                                head, tiles_d.data_ptr(), len(tiles_h), max_tokens, out.data_ptr()))
        torch.cuda.synchronize()
        got = out.cpu().numpy().astype(np.float64)
        err = np.abs(got - ref).max() / np.abs(ref).max()
        assert err <= 1e-5, (max_tokens, err)


@pytest.mark.gpu
@pytest.mark.parametrize("q_heads,kv_heads,head,rope_dims", [(28, 4, 128, 128), (4, 2, 64, 32)])
def test_rope_kv_append_matches_separate_calls(torch_cuda, hip_ctx, q_heads, kv_heads, head, rope_dims):
    """air_hip_rope_kv_append leaves q|k|v and the pool bit-identical to
    air_hip_rope then air_hip_kv_append: rotary and unrotated k dims, a row
    whose position lies past the RoPE table (stored unrotated), a row whose
    page-table entry is absent and a negative position (rotated / skipped
    alike)."""
    torch = torch_cuda
    dev = torch.device("cuda:0")
    page_tokens, layers, layer, max_pages = 16, 3, 2, 4
    kv_width = kv_heads * head
    stride = q_heads * head + 2 * kv_width + 8          # padded rows
    pool_pages = 12
    rng = np.random.default_rng(head + rope_dims)
    table_positions = 40
    positions = [0, 5, 17, 39, 45, 63, 3, -1]
    tables = [list(rng.permutation(pool_pages)[:max_pages]) for _ in positions]
    tables[6][0] = -1                                    # position 3: no page for it
    m = len(positions)
    half = rope_dims // 2
    ang = rng.uniform(0.0, 6.28, (table_positions, half))
    rope = np.stack([np.cos(ang), np.sin(ang)], axis=-1).astype(np.float32)
    qkv_h = rng.standard_normal((m, stride)).astype(np.float32)
    pool_h = rng.standard_normal(pool_pages * layers * 2 * page_tokens * kv_width).astype(np.float32)
    rope_d = torch.from_numpy(rope).to(dev)
    pos_d = torch.tensor(positions, dtype=torch.int32, device=dev)
    tab_d = torch.tensor(np.array(tables, dtype=np.int32), device=dev)
    lib = capi.lib()
    outs = []
    for fused in (False, True):
        qkv = torch.from_numpy(qkv_h).to(dev)
        pool = torch.from_numpy(pool_h).to(dev)
        kv = capi.KvLayout(pool.data_ptr(), page_tokens, kv_width, layers, max_pages, pool_pages)
        if fused:
            capi.check(lib.air_hip_rope_kv_append(hip_ctx.handle, ctypes.byref(kv), qkv.data_ptr(), stride, m,
                                                  pos_d.data_ptr(), tab_d.data_ptr(), layer, q_heads, kv_heads,
                                                  head, rope_dims, rope_d.data_ptr(), table_positions))
        else:
            capi.check(lib.air_hip_rope(hip_ctx.handle, qkv.data_ptr(), stride, m, pos_d.data_ptr(), q_heads,
                                        kv_heads, head, rope_dims, rope_d.data_ptr(), table_positions))
            capi.check(lib.air_hip_kv_append(hip_ctx.handle, ctypes.byref(kv), qkv.data_ptr(), stride,
                                             q_heads * head, m, pos_d.data_ptr(), tab_d.data_ptr(), layer))
        torch.cuda.synchronize()
        outs.append((qkv.cpu().numpy(), pool.cpu().numpy()))
    (q0, p0), (q1, p1) = outs
    assert not np.array_equal(q0, qkv_h)                 # something rotated
    assert not np.array_equal(p0, pool_h)                # something stored
    assert np.array_equal(q1.view(np.uint32), q0.view(np.uint32))
    assert np.array_equal(p1.view(np.uint32), p0.view(np.uint32))
    bad = lib.air_hip_rope_kv_append(hip_ctx.handle, ctypes.byref(kv), qkv.data_ptr(), stride, m, pos_d.data_ptr(),
                                     tab_d.data_ptr(), layer, q_heads, kv_heads + 1, head, rope_dims,
                                     rope_d.data_ptr(), table_positions)
    assert bad == 1 and b"KV width" in lib.air_hip_last_error()


@pytest.mark.gpu
@pytest.mark.parametrize("q_heads,kv_heads,head,rope_dims", [(28, 4, 128, 128), (4, 2, 64, 32)])
def test_linear_rope_kv_matches_separate_calls(torch_cuda, hip_ctx, q_heads, kv_heads, head, rope_dims):
    """air_hip_linear_rope_kv leaves q|k|v and the pool bit-identical to
    air_hip_linear then air_hip_rope_kv_append, on the routes where the
    linear's split reduction does the RoPE and the append (skinny kernel or
    prefill GEMM with a K split) and where it does not (no split, the
    single-launch kernel); rows as in the test above (past the table, no
    page, negative position)."""
    torch = torch_cuda
    dev = torch.device("cuda:0")
    page_tokens, layers, layer, max_pages, pool_pages = 16, 3, 1, 4, 12
    kv_width = kv_heads * head
    n, k = q_heads * head + 2 * kv_width, 1024
    rng = np.random.default_rng(head + rope_dims + 1)
    table_positions = 40
    positions = [0, 5, 17, 39, 45, 63, 3, -1]
    tables = [list(rng.permutation(pool_pages)[:max_pages]) for _ in positions]
    tables[6][0] = -1
    m = len(positions)
    half = rope_dims // 2
    ang = rng.uniform(0.0, 6.28, (table_positions, half))
    rope_d = torch.from_numpy(np.stack([np.cos(ang), np.sin(ang)], axis=-1).astype(np.float32)).to(dev)
    pool_h = rng.standard_normal(pool_pages * layers * 2 * page_tokens * kv_width).astype(np.float32)
    pos_d = torch.tensor(positions, dtype=torch.int32, device=dev)
    tab_d = torch.tensor(np.array(tables, dtype=np.int32), device=dev)
    canon = helpers.weights(capi.TYPE_Q8_0, k, n, seed=n + 3)
    mat = capi.Matrix(hip_ctx, capi.TYPE_Q8_0, k, n, canon, canon.nbytes, on_device=False)
    x = torch.from_numpy(helpers.activations(m, k, seed=n) * 2.0).to(dev)
    bias = torch.from_numpy(helpers.activations(1, n, seed=n + 1)[0] * 0.1).to(dev)
    lib = capi.lib()
    h = hip_ctx.handle
    try:
        # decode routes (skinny with and without a K split, the fused kernel),
        # then the prefill GEMM without and with a K split
        runs = [(capi.LINEAR_DECODE, p, 0) for p in [(0, 0, 0), (2, 1, 1), (2, 1, 3), (2, 2, 2)]]
        runs += [(capi.LINEAR_PREFILL, (0, 0, 0), s) for s in (1, 2)]
        for tactic, path, pf_splits in runs:
            hip_ctx.set_decode_path(*path)
            hip_ctx.set_prefill_tuning(0, 0, pf_splits, 0)
            outs = []
            for fused in (False, True):
                pool = torch.from_numpy(pool_h).to(dev)
                kv = capi.KvLayout(pool.data_ptr(), page_tokens, kv_width, layers, max_pages, pool_pages)
                qkv = torch.full((m, n), float("nan"), dtype=torch.float32, device=dev)
                if fused:
                    capi.check(lib.air_hip_linear_rope_kv(h, mat.handle, x.data_ptr(), m, qkv.data_ptr(),
                                                          bias.data_ptr(), ctypes.byref(kv), pos_d.data_ptr(),
                                                          tab_d.data_ptr(), layer, q_heads, kv_heads, head,
                                                          rope_dims, rope_d.data_ptr(), table_positions, tactic))
                else:
                    capi.check(lib.air_hip_linear(h, mat.handle, x.data_ptr(), qkv.data_ptr(), bias.data_ptr(), m,
                                                  tactic))
                    capi.check(lib.air_hip_rope_kv_append(h, ctypes.byref(kv), qkv.data_ptr(), n, m,
                                                          pos_d.data_ptr(), tab_d.data_ptr(), layer, q_heads,
                                                          kv_heads, head, rope_dims, rope_d.data_ptr(),
                                                          table_positions))
                torch.cuda.synchronize()
                outs.append((qkv.cpu().numpy(), pool.cpu().numpy()))
            (q0, p0), (q1, p1) = outs
            case = (tactic, path, pf_splits)
            assert not np.array_equal(p0, pool_h), case
            assert np.array_equal(q1.view(np.uint32), q0.view(np.uint32)), case
            assert np.array_equal(p1.view(np.uint32), p0.view(np.uint32)), case
        bad = lib.air_hip_linear_rope_kv(h, mat.handle, x.data_ptr(), m, qkv.data_ptr(), None, ctypes.byref(kv),
                                         pos_d.data_ptr(), tab_d.data_ptr(), layer, q_heads + 1, kv_heads, head,
                                         rope_dims, rope_d.data_ptr(), table_positions, capi.LINEAR_DECODE)
        assert bad == 1 and b"q|k|v" in lib.air_hip_last_error()
    finally:
        hip_ctx.set_decode_path(0)
        hip_ctx.set_prefill_tuning(0, 0, 0, 0)
        mat.release()
