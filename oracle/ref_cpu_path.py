"""The reference's CPU MoE-layer path, restated for the CPU baseline.

TEST / BASELINE INFRASTRUCTURE ONLY: timed by bench.py's cpu_baseline leg;
never imported by the product package.

The reference has no SIMD MoE kernel; its CPU path is torch and numpy:
  router    tests/test_moe_routing.py:65-71: logits = x W^T (nn.Linear, fp32),
            torch.topk, softmax over the k selected logits (an nn.Linear bias
            is added to the logits when given).
  weights   python/phantom/loader/gguf_loader.py:363-380: numpy Q4_0
            dequantisation (fp16 scale -> fp32, low/high nibbles minus 8,
            times d) and a bf16 cast.  Weights stay packed in RAM and are
            expanded on every call, as the tiered runtime keeps cold experts
            quantised (docs/ARCHITECTURE.md:82).
  experts   SwiGLU h = silu(x W_g^T) * (x W_u^T), y = h W_d^T in torch CPU
            bf16 matmuls (the arithmetic of kernels/sparse_moe/
            sparse_matmul.cu:120-215 at the precision transformers runs).
  combine   y.index_add_(0, token_ids, w * y_e), as transformers' MoE blocks do.
"""
from __future__ import annotations

import numpy as np
import torch
import torch.nn.functional as F


def dequant_q4_0_bf16(raw: np.ndarray, rows: int, K: int) -> torch.Tensor:
    """numpy Q4_0 -> bf16 [rows, K] (gguf_loader.py:363-380)."""
    nb = rows * K // 32
    blk = np.ascontiguousarray(raw, dtype=np.uint8).reshape(nb, 18)
    d = blk[:, :2].copy().view(np.float16).astype(np.float32)
    qs = blk[:, 2:]
    low = (qs & 0x0F).astype(np.int8) - 8
    high = ((qs >> 4) & 0x0F).astype(np.int8) - 8
    w = np.empty((nb, 32), dtype=np.float32)
    w[:, 0:16] = low * d
    w[:, 16:32] = high * d
    return torch.from_numpy(w.reshape(rows, K)).to(torch.bfloat16)


class RefCPUMoE:
    """One MoE layer on the CPU in the reference's way.

    gate/up: uint8 [E, I, H/32, 18]; down: [E, H, I/32, 18] (GGUF Q4_0).
    predequant=True expands all experts once up front (the second variant)."""

    def __init__(self, router_w: np.ndarray, gate, up, down, H: int, I: int, top_k: int,
                 score: str = "softmax", router_bias=None, shared=None, predequant: bool = False):
        self.W = torch.from_numpy(np.ascontiguousarray(router_w, dtype=np.float32))
        self.b = None if router_bias is None else torch.from_numpy(np.asarray(router_bias, np.float32))
        self.gate, self.up, self.down = gate, up, down
        self.shared = shared
        self.H, self.I, self.k, self.score = H, I, top_k, score
        self.E = self.W.shape[0]
        self._cache = None
        if predequant:
            self._cache = [self._expert(e, force=True) for e in range(self.E)]

    def _expert(self, e: int, force: bool = False):
        if self._cache is not None and not force:
            return self._cache[e]
        H, I = self.H, self.I
        return (dequant_q4_0_bf16(self.gate[e], I, H), dequant_q4_0_bf16(self.up[e], I, H),
                dequant_q4_0_bf16(self.down[e], H, I))

    @staticmethod
    def _ffn(xe, wg, wu, wd):
        g = xe @ wg.T
        u = xe @ wu.T
        return (F.silu(g) * u) @ wd.T

    @torch.no_grad()
    def __call__(self, x_bf16: torch.Tensor) -> torch.Tensor:
        x = x_bf16.to(torch.bfloat16)
        logits = F.linear(x.float(), self.W, self.b)
        top_logits, top_idx = torch.topk(logits, self.k, dim=-1)
        if self.score == "softmax":
            w = F.softmax(top_logits, dim=-1)
        else:
            s = torch.sigmoid(top_logits)
            w = s / s.sum(-1, keepdim=True)
        y = torch.zeros(x.shape[0], self.H, dtype=torch.float32)
        for e in torch.unique(top_idx).tolist():
            tok, slot = torch.where(top_idx == e)
            wg, wu, wd = self._expert(e)
            ye = self._ffn(x[tok], wg, wu, wd).float()
            y.index_add_(0, tok, ye * w[tok, slot, None])
        if self.shared is not None:
            H, I = self.H, self.I
            sg, su, sd = self.shared
            y += self._ffn(x, dequant_q4_0_bf16(sg, I, H), dequant_q4_0_bf16(su, I, H),
                           dequant_q4_0_bf16(sd, H, I)).float()
        return y
