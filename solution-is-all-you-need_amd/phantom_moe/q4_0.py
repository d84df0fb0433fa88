"""GGUF Q4_0 block format: host pack/unpack and the device repack.

Format (python/phantom/loader/gguf_loader.py:72 QUANT_SPECS[Q4_0] = (32, 18);
dequantisation at :362-381 and :588-596): a row of K weights is K/32 blocks of
18 bytes, an fp16 scale ``d`` (little endian) followed by 16 bytes ``qs``.
Element j of the block is ``((qs[j] & 0xF) - 8) * d`` and element j+16 is
``((qs[j] >> 4) - 8) * d``.  GGUF stores dims reversed (gguf_loader.py:171),
so a row-major ``[rows, K]`` matrix is ``rows`` consecutive rows of blocks.

``pack``/``unpack`` are exact host conversions between (q, d) and bytes used
to build inputs.  ``repack``/``unrepack`` run on the GPU and convert between
GGUF bytes and the MFMA-ordered layout the expert kernels read.
"""
from __future__ import annotations

import numpy as np
import torch

from . import _lib

BLOCK = 32
BLOCK_BYTES = 18


def pack(q: np.ndarray, d: np.ndarray) -> np.ndarray:
    """(q int in [-8, 7] of shape [..., K], d fp16 of shape [..., K/32]) -> uint8 [..., K/32, 18]."""
    q = np.asarray(q)
    d = np.asarray(d, dtype=np.float16)
    K = q.shape[-1]
    if K % BLOCK:
        raise ValueError("K must be a multiple of 32")
    if q.min(initial=0) < -8 or q.max(initial=0) > 7:
        raise ValueError("q must lie in [-8, 7]")
    lead = q.shape[:-1]
    nb = K // BLOCK
    if d.shape != lead + (nb,):
        raise ValueError(f"d must have shape {lead + (nb,)}, got {d.shape}")
    n = (q.reshape(*lead, nb, BLOCK) + 8).astype(np.uint8)
    out = np.empty(lead + (nb, BLOCK_BYTES), dtype=np.uint8)
    out[..., 0:2] = d.reshape(*lead, nb, 1).view(np.uint8)
    out[..., 2:] = n[..., :16] | (n[..., 16:] << 4)
    return out


def unpack(blocks: np.ndarray):
    """uint8 [..., nb, 18] -> (q int8 [..., nb*32], d fp16 [..., nb])."""
    b = np.asarray(blocks, dtype=np.uint8)
    if b.shape[-1] != BLOCK_BYTES:
        raise ValueError("last dim must be 18 bytes")
    d = np.ascontiguousarray(b[..., 0:2]).view(np.float16)[..., 0]
    qs = b[..., 2:]
    lo = (qs & 0x0F).astype(np.int8) - 8
    hi = (qs >> 4).astype(np.int8) - 8
    q = np.concatenate([lo, hi], axis=-1)
    return q.reshape(*b.shape[:-2], b.shape[-2] * BLOCK), d


def random_blocks(rng: np.random.Generator, shape, scale_sigma: float = 0.02) -> np.ndarray:
    """Q4_0 bytes for a [..., K] tensor: q uniform in [-8, 7], d = |N(0, sigma)| in fp16."""
    *lead, K = shape
    nb = K // BLOCK
    qs = np.frombuffer(rng.bytes(int(np.prod(lead, dtype=np.int64)) * nb * 16), dtype=np.uint8)
    d = (np.abs(rng.standard_normal(tuple(lead) + (nb,), dtype=np.float32)) * scale_sigma).astype(np.float16)
    out = np.empty(tuple(lead) + (nb, BLOCK_BYTES), dtype=np.uint8)
    out[..., 0:2] = d.reshape(*lead, nb, 1).view(np.uint8)
    out[..., 2:] = qs.reshape(*lead, nb, 16)
    return out


def nib_bytes(rows: int, K: int) -> int:
    n = _lib.load().phantom_q4_0_nib_bytes(rows, K)
    if n < 0:
        raise ValueError(f"repacked layout needs rows % 16 == 0 and K % 32 == 0 (rows={rows}, K={K})")
    return int(n)


def scale_count(rows: int, K: int) -> int:
    n = _lib.load().phantom_q4_0_scale_bytes(rows, K)
    if n < 0:
        raise ValueError(f"repacked layout needs rows % 16 == 0 and K % 32 == 0 (rows={rows}, K={K})")
    return int(n) // 2


def _dev_u8(t: torch.Tensor, what: str) -> torch.Tensor:
    if not isinstance(t, torch.Tensor) or t.device.type != "cuda":
        raise TypeError(f"{what} must be a CUDA (HIP) tensor")
    if t.dtype != torch.uint8:
        raise TypeError(f"{what} must be uint8, got {t.dtype}")
    return t.contiguous()


def repack(q4_0: torch.Tensor, rows: int, K: int, n_mats: int = 1):
    """GGUF Q4_0 bytes of ``n_mats`` stacked [rows, K] matrices (device uint8)
    -> (nib uint8 [n_mats * nib_bytes], scale int16-bits as torch.int16
    [n_mats * scale_count]) on the same device."""
    q = _dev_u8(q4_0, "q4_0")
    per = rows * (K // BLOCK) * BLOCK_BYTES
    if q.numel() != n_mats * per:
        raise ValueError(f"expected {n_mats * per} bytes for {n_mats} x [{rows}, {K}] Q4_0, got {q.numel()}")
    nb, ns = nib_bytes(rows, K), scale_count(rows, K)
    nib = torch.empty(n_mats * nb, dtype=torch.uint8, device=q.device)
    sc = torch.empty(n_mats * ns, dtype=torch.int16, device=q.device)
    lib = _lib.load()
    stream = _lib.stream_handle(q.device)
    # One launch per matrix keeps each call's indexing within one matrix.
    for i in range(n_mats):
        rc = lib.phantom_q4_0_repack(
            q.data_ptr() + i * per, rows, K, nib.data_ptr() + i * nb, sc.data_ptr() + i * ns * 2, stream
        )
        _lib.check(rc, "phantom_q4_0_repack")
    return nib, sc


def unrepack(nib: torch.Tensor, scale: torch.Tensor, rows: int, K: int, n_mats: int = 1) -> torch.Tensor:
    """Inverse of :func:`repack`: the original GGUF bytes (device uint8)."""
    nib = _dev_u8(nib, "nib")
    if scale.device != nib.device or scale.dtype != torch.int16:
        raise TypeError("scale must be an int16 tensor on the same device as nib")
    scale = scale.contiguous()
    per = rows * (K // BLOCK) * BLOCK_BYTES
    nb, ns = nib_bytes(rows, K), scale_count(rows, K)
    if nib.numel() != n_mats * nb or scale.numel() != n_mats * ns:
        raise ValueError("nib/scale sizes do not match the given shape")
    out = torch.empty(n_mats * per, dtype=torch.uint8, device=nib.device)
    lib = _lib.load()
    stream = _lib.stream_handle(nib.device)
    for i in range(n_mats):
        rc = lib.phantom_q4_0_unrepack(
            nib.data_ptr() + i * nb, scale.data_ptr() + i * ns * 2, rows, K, out.data_ptr() + i * per, stream
        )
        _lib.check(rc, "phantom_q4_0_unrepack")
    return out


def dequant_f32(q4_0: torch.Tensor, rows: int, K: int) -> torch.Tensor:
    """Device Q4_0 bytes -> fp32 [rows, K] (gguf_loader.py:369-378 values)."""
    q = _dev_u8(q4_0, "q4_0")
    if q.numel() != rows * (K // BLOCK) * BLOCK_BYTES or K % BLOCK:
        raise ValueError("size does not match [rows, K] Q4_0")
    out = torch.empty((rows, K), dtype=torch.float32, device=q.device)
    rc = _lib.load().phantom_q4_0_dequant_f32(q.data_ptr(), rows, K, out.data_ptr(), _lib.stream_handle(q.device))
    _lib.check(rc, "phantom_q4_0_dequant_f32")
    return out
