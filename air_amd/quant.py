"""Deterministic GGUF quantizers for synthetic weights (numpy, host).

AIR ships no quantizer: it only decodes GGUF files (its fixture writers emit
random bytes, tests/make_quantized_qwen2_gguf.py:32-69).  The benchmark
configurations describe weights w ~ N(0, 0.02) quantized as

  Q8_0  blocks of 32, d = max|w| / 127 stored as f16, q = round(w / d)
  Q4_0  blocks of 32, d = (signed max-abs value) / -8 stored as f16,
        n = clamp(round(w / d) + 8, 0, 15); byte i = n[i] | n[i+16] << 4
  Q4_K  super-blocks of 256 = 8 sub-blocks of 32 with 6-bit scales and mins,
        f16 d and dmin, 4-bit n: w ~= (d*sc_j)*n - dmin*m_j

These functions produce valid canonical blocks from f32 weights; the engine's
parity is "same bytes in, same values out", so any valid blocks serve.
"""
from __future__ import annotations

import numpy as np

BLOCK = {2: (32, 18), 8: (32, 34), 12: (256, 144)}


def _round_half_away(v: np.ndarray) -> np.ndarray:
    return np.sign(v) * np.floor(np.abs(v) + 0.5)


def quantize_q8_0(w: np.ndarray) -> np.ndarray:
    """w: float32 [n, k] (k % 32 == 0) -> uint8 [n, k/32*34]."""
    n, k = w.shape
    b = w.reshape(n, k // 32, 32).astype(np.float32)
    amax = np.abs(b).max(axis=2)
    d = (amax / np.float32(127.0)).astype(np.float32)
    inv = np.where(d > 0, np.float32(1.0) / np.where(d > 0, d, 1), 0).astype(np.float32)
    q = np.clip(_round_half_away(b * inv[..., None]), -127, 127).astype(np.int8)
    out = np.empty((n, k // 32, 34), dtype=np.uint8)
    out[..., 0:2] = d.astype(np.float16).view(np.uint8).reshape(n, k // 32, 2)
    out[..., 2:] = q.view(np.uint8)
    return out.reshape(n, (k // 32) * 34)


def quantize_q4_0(w: np.ndarray) -> np.ndarray:
    """w: float32 [n, k] (k % 32 == 0) -> uint8 [n, k/32*18]."""
    n, k = w.shape
    b = w.reshape(n, k // 32, 32).astype(np.float32)
    idx = np.abs(b).argmax(axis=2)
    vmax = np.take_along_axis(b, idx[..., None], axis=2)[..., 0]
    d = (vmax / np.float32(-8.0)).astype(np.float32)
    inv = np.where(d != 0, np.float32(1.0) / np.where(d != 0, d, 1), 0).astype(np.float32)
    q = np.clip(np.floor(b * inv[..., None] + np.float32(8.5)), 0, 15).astype(np.uint8)
    out = np.empty((n, k // 32, 18), dtype=np.uint8)
    out[..., 0:2] = d.astype(np.float16).view(np.uint8).reshape(n, k // 32, 2)
    out[..., 2:] = q[..., :16] | (q[..., 16:] << 4)
    return out.reshape(n, (k // 32) * 18)


def pack_q4_k_scales(sc: np.ndarray, mn: np.ndarray) -> np.ndarray:
    """6-bit scales/mins [..., 8] -> the 12 packed bytes of a Q4_K block
    (inverse of the unpack in src/reference/tensor_reader.cpp:153-165)."""
    sc = sc.astype(np.uint8)
    mn = mn.astype(np.uint8)
    s = np.zeros(sc.shape[:-1] + (12,), dtype=np.uint8)
    s[..., 0:4] = (sc[..., 0:4] & 63) | ((sc[..., 4:8] >> 4) << 6)
    s[..., 4:8] = (mn[..., 0:4] & 63) | ((mn[..., 4:8] >> 4) << 6)
    s[..., 8:12] = (sc[..., 4:8] & 0x0F) | ((mn[..., 4:8] & 0x0F) << 4)
    return s


def quantize_q4_k(w: np.ndarray) -> np.ndarray:
    """w: float32 [n, k] (k % 256 == 0) -> uint8 [n, k/256*144]."""
    n, k = w.shape
    nb = k // 256
    b = w.reshape(n, nb, 8, 32).astype(np.float32)
    lo = np.minimum(b.min(axis=3), 0).astype(np.float32)          # sub-block min (<= 0)
    hi = b.max(axis=3).astype(np.float32)
    scale = ((hi - lo) / np.float32(15.0)).astype(np.float32)       # sub-block step
    d = (scale.max(axis=2) / np.float32(63.0)).astype(np.float16)   # super-block factors
    dmin = ((-lo).max(axis=2) / np.float32(63.0)).astype(np.float16)
    d32 = d.astype(np.float32)
    dmin32 = dmin.astype(np.float32)
    sc = np.clip(_round_half_away(np.where(d32[..., None] > 0, scale / np.where(d32[..., None] > 0, d32[..., None], 1), 0)), 0, 63)
    mn = np.clip(_round_half_away(np.where(dmin32[..., None] > 0, -lo / np.where(dmin32[..., None] > 0, dmin32[..., None], 1), 0)), 0, 63)
    step = (d32[..., None] * sc).astype(np.float32)
    offs = (dmin32[..., None] * mn).astype(np.float32)
    q = np.where(step[..., None] > 0, (b + offs[..., None]) / np.where(step[..., None] > 0, step[..., None], 1), 0)
    q = np.clip(_round_half_away(q), 0, 15).astype(np.uint8)       # [n, nb, 8, 32]
    out = np.zeros((n, nb, 144), dtype=np.uint8)
    out[..., 0:2] = d.view(np.uint8).reshape(n, nb, 2)
    out[..., 2:4] = dmin.view(np.uint8).reshape(n, nb, 2)
    out[..., 4:16] = pack_q4_k_scales(sc, mn)
    # 64-element group g: byte g*32+i = n[2g][i] | n[2g+1][i] << 4
    qs = q[:, :, 0::2, :] | (q[:, :, 1::2, :] << 4)               # [n, nb, 4, 32]
    out[..., 16:] = qs.reshape(n, nb, 128)
    return out.reshape(n, nb * 144)


QUANTIZERS = {8: quantize_q8_0, 2: quantize_q4_0, 12: quantize_q4_k}


def quantize(type_id: int, w: np.ndarray) -> np.ndarray:
    return QUANTIZERS[type_id](np.ascontiguousarray(w, dtype=np.float32))


def synthetic_weights(type_id: int, k: int, n: int, seed: int, sigma: float = 0.02) -> np.ndarray:
    """Canonical bytes [n, row_bytes] of w ~ N(0, sigma) quantized to type_id."""
    rng = np.random.default_rng(seed)
    w = rng.standard_normal((n, k), dtype=np.float32) * np.float32(sigma)
    return quantize(type_id, w)


# ---- device-side synthesis (torch) for benchmark-sized sweeps -------------
# The same quantization rules evaluated with torch on the GPU, so that
# multi-GB synthetic models are produced in seconds.  Used for benchmark
# inputs only; the parity tests use the host quantizers above.

def _torch_round_half_away(t):
    import torch

    return torch.sign(t) * torch.floor(torch.abs(t) + 0.5)


def synthetic_weights_device(type_id: int, k: int, n: int, seed: int, device, sigma: float = 0.02,
                             row_chunk: int = 8192):
    """Canonical bytes (torch uint8 [n, row_bytes] on `device`) of w ~ N(0, sigma)."""
    import torch

    gen = torch.Generator(device=device)
    gen.manual_seed(seed)
    be, bb = BLOCK[type_id]
    out = torch.empty((n, (k // be) * bb), dtype=torch.uint8, device=device)
    for r0 in range(0, n, row_chunk):
        r1 = min(n, r0 + row_chunk)
        w = torch.randn((r1 - r0, k), generator=gen, device=device, dtype=torch.float32) * sigma
        out[r0:r1] = _quantize_torch(type_id, w)
    return out


def _quantize_torch(type_id: int, w):
    import torch

    n, k = w.shape
    if type_id == 8:
        b = w.reshape(n, k // 32, 32)
        d = b.abs().amax(dim=2) / 127.0
        inv = torch.where(d > 0, 1.0 / torch.where(d > 0, d, torch.ones_like(d)), torch.zeros_like(d))
        q = torch.clamp(_torch_round_half_away(b * inv[..., None]), -127, 127).to(torch.int8)
        blk = torch.empty((n, k // 32, 34), dtype=torch.uint8, device=w.device)
        blk[..., 0:2] = d.to(torch.float16).view(torch.uint8).reshape(n, k // 32, 2)
        blk[..., 2:] = q.view(torch.uint8)
        return blk.reshape(n, -1)
    if type_id == 2:
        b = w.reshape(n, k // 32, 32)
        idx = b.abs().argmax(dim=2, keepdim=True)
        vmax = torch.gather(b, 2, idx)[..., 0]
        d = vmax / -8.0
        inv = torch.where(d != 0, 1.0 / torch.where(d != 0, d, torch.ones_like(d)), torch.zeros_like(d))
        q = torch.clamp(torch.floor(b * inv[..., None] + 8.5), 0, 15).to(torch.uint8)
        blk = torch.empty((n, k // 32, 18), dtype=torch.uint8, device=w.device)
        blk[..., 0:2] = d.to(torch.float16).view(torch.uint8).reshape(n, k // 32, 2)
        blk[..., 2:] = q[..., :16] | (q[..., 16:] << 4)
        return blk.reshape(n, -1)
    if type_id == 12:
        nb = k // 256
        b = w.reshape(n, nb, 8, 32)
        lo = torch.clamp(b.amin(dim=3), max=0.0)
        hi = b.amax(dim=3)
        scale = (hi - lo) / 15.0
        d = (scale.amax(dim=2) / 63.0).to(torch.float16)
        dmin = ((-lo).amax(dim=2) / 63.0).to(torch.float16)
        d32 = d.float()[..., None]
        dm32 = dmin.float()[..., None]
        one = torch.ones_like(d32)
        sc = torch.clamp(_torch_round_half_away(torch.where(d32 > 0, scale / torch.where(d32 > 0, d32, one), 0 * d32)), 0, 63)
        mn = torch.clamp(_torch_round_half_away(torch.where(dm32 > 0, -lo / torch.where(dm32 > 0, dm32, one), 0 * dm32)), 0, 63)
        step = (d32 * sc)[..., None]
        offs = (dm32 * mn)[..., None]
        q = torch.where(step > 0, (b + offs) / torch.where(step > 0, step, torch.ones_like(step)), torch.zeros_like(b))
        q = torch.clamp(_torch_round_half_away(q), 0, 15).to(torch.uint8)
        sc8 = sc.to(torch.uint8)
        mn8 = mn.to(torch.uint8)
        blk = torch.zeros((n, nb, 144), dtype=torch.uint8, device=w.device)
        blk[..., 0:2] = d.view(torch.uint8).reshape(n, nb, 2)
        blk[..., 2:4] = dmin.view(torch.uint8).reshape(n, nb, 2)
        blk[..., 4:8] = (sc8[..., 0:4] & 63) | ((sc8[..., 4:8] >> 4) << 6)
        blk[..., 8:12] = (mn8[..., 0:4] & 63) | ((mn8[..., 4:8] >> 4) << 6)
        blk[..., 12:16] = (sc8[..., 4:8] & 0x0F) | ((mn8[..., 4:8] & 0x0F) << 4)
        blk[..., 16:] = (q[:, :, 0::2, :] | (q[:, :, 1::2, :] << 4)).reshape(n, nb, 128)
        return blk.reshape(n, -1)
    raise ValueError(f"unsupported type {type_id}")
