"""Runtime caller swap: run transformers' MoE blocks through moe_forward.

In the reference's `phantom run` path the MoE layers execute inside
transformers' blocks (python/phantom/phantom_cli.py:1393-1430).  These
helpers replace the forward of each Qwen3-MoE / Mixtral sparse block (the
transformers 5.x layout: ``block.gate.weight`` [E, H], ``block.experts.
gate_up_proj`` [E, 2I, H] with the gate rows first, ``block.experts.
down_proj`` [E, H, I]) by one call into libphantom_moe.so on Q4_0 weights:

  swap_from_gguf(model, reader)  the Q4_0 expert bytes of each layer come
                                 straight from the GGUF file the model was
                                 loaded from (phantom_moe.gguf)
  quantize_and_swap(model)       the block's float weights are quantised to
                                 Q4_0 here, and the module's own parameters
                                 are overwritten with the dequantised values,
                                 so the original forward and the swapped one
                                 use the same weights (for parity checks)

Both keep the block's contract: hidden states [B, S, H] in, the same shape
and dtype out.  Routing follows the block's router: softmax over the experts
then top-k renormalised, which is the library's softmax mode (equal to a
softmax over the k selected logits).  A Qwen3 block with
norm_topk_prob=False is refused.
"""
from __future__ import annotations

import types

import numpy as np
import torch

from . import q4_0
from .ops import MoEWeights, moe_forward


def quantize_q4_0(w: np.ndarray) -> np.ndarray:
    """float [..., K] -> GGUF Q4_0 bytes [..., K/32, 18].

    The rounding rule of llama.cpp's reference quantiser
    (quantize_row_q4_0_ref in ggml-quants.c): per 32-block, the element of
    largest magnitude m maps to -8, d = m / -8, q = min(15, int(x / d + 8.5)),
    d stored as fp16."""
    x = np.asarray(w, dtype=np.float32)
    K = x.shape[-1]
    if K % 32:
        raise ValueError("K must be a multiple of 32")
    b = x.reshape(x.shape[:-1] + (K // 32, 32))
    pos = np.abs(b).argmax(axis=-1)[..., None]
    m = np.take_along_axis(b, pos, axis=-1)[..., 0]
    d = m / np.float32(-8.0)
    with np.errstate(divide="ignore"):
        inv = np.where(d != 0, np.float32(1.0) / d, np.float32(0.0)).astype(np.float32)
    q = np.minimum(15, (b * inv[..., None] + np.float32(8.5)).astype(np.int32)).astype(np.int32) - 8
    q = np.clip(q, -8, 7).reshape(x.shape)
    return q4_0.pack(q, d.astype(np.float16))


def dequantize_q4_0(blocks: np.ndarray) -> np.ndarray:
    """GGUF Q4_0 bytes [..., nb, 18] -> float32 [..., nb*32], (q - 8) * d exactly."""
    q, d = q4_0.unpack(blocks)
    nb = d.shape[-1]
    return (q.reshape(q.shape[:-1] + (nb, 32)).astype(np.float32) * d[..., None].astype(np.float32)).reshape(q.shape)


def _is_moe_block(m) -> bool:
    return (hasattr(m, "gate") and hasattr(m.gate, "weight") and hasattr(m, "experts")
            and hasattr(m.experts, "gate_up_proj") and hasattr(m.experts, "down_proj"))


def moe_blocks(model):
    """(name, block) of every Qwen3-MoE / Mixtral-style sparse block."""
    return [(n, m) for n, m in model.named_modules() if _is_moe_block(m)]


def _phantom_forward(self, hidden_states: torch.Tensor) -> torch.Tensor:
    B, S, H = hidden_states.shape
    experts, router_w, router_bias, top_k, score = self._phantom_moe
    x = hidden_states.reshape(-1, H).to(torch.bfloat16)
    y = moe_forward(x, router_w, experts, top_k, score, router_bias)
    return y.to(hidden_states.dtype).reshape(B, S, H)


def swap_block(block, experts: MoEWeights, router_w: torch.Tensor, top_k: int, score: str = "softmax",
               router_bias: torch.Tensor | None = None) -> None:
    """Route `block.forward` through moe_forward with these weights."""
    block._phantom_moe = (experts, router_w.float().contiguous(), router_bias, int(top_k), score)
    block._phantom_original_forward = block.forward
    block.forward = types.MethodType(_phantom_forward, block)


def restore_block(block) -> None:
    if hasattr(block, "_phantom_original_forward"):
        block.forward = block._phantom_original_forward
        del block._phantom_original_forward, block._phantom_moe


def _top_k(block) -> int:
    g = block.gate
    if getattr(g, "norm_topk_prob", True) is False:
        raise NotImplementedError(f"{type(block).__name__}: norm_topk_prob=False (no renormalisation over the "
                                  f"top-k) is not a mode of the library")
    return int(g.top_k)


@torch.no_grad()
def quantize_and_swap(model) -> int:
    """Quantise every sparse block's experts to Q4_0, write the dequantised
    weights back into the block, and swap its forward.  Returns the number
    of blocks swapped."""
    n = 0
    for _, blk in moe_blocks(model):
        ex = blk.experts
        dev = ex.gate_up_proj.device
        E, I2, H = ex.gate_up_proj.shape
        I = I2 // 2
        gu = ex.gate_up_proj.detach().float().cpu().numpy()
        dn = ex.down_proj.detach().float().cpu().numpy()
        gate_q, up_q, down_q = quantize_q4_0(gu[:, :I]), quantize_q4_0(gu[:, I:]), quantize_q4_0(dn)
        deq = np.concatenate([dequantize_q4_0(gate_q), dequantize_q4_0(up_q)], axis=1)
        ex.gate_up_proj.copy_(torch.from_numpy(deq).to(ex.gate_up_proj.dtype))
        ex.down_proj.copy_(torch.from_numpy(dequantize_q4_0(down_q)).to(ex.down_proj.dtype))
        experts = MoEWeights.from_q4_0(torch.from_numpy(gate_q).to(dev), torch.from_numpy(up_q).to(dev),
                                       torch.from_numpy(down_q).to(dev), H, I, E)
        swap_block(blk, experts, blk.gate.weight.detach(), _top_k(blk))
        n += 1
    return n


@torch.no_grad()
def swap_from_gguf(model, reader, first_layer: int = 0) -> int:
    """Swap the k-th sparse block (in module order) to layer first_layer + k
    of the GGUF file, whose Q4_0 expert bytes are loaded without
    dequantisation (phantom_moe.gguf.load_moe_layer)."""
    from .gguf import load_moe_layer

    n = 0
    for k, (_, blk) in enumerate(moe_blocks(model)):
        dev = blk.gate.weight.device
        spec, experts, router_w, bias = load_moe_layer(reader, first_layer + k, dev)
        E, I2, H = blk.experts.gate_up_proj.shape
        if (spec.E, spec.I, spec.H) != (E, I2 // 2, H):
            raise ValueError(f"GGUF layer {first_layer + k} is E={spec.E}, I={spec.I}, H={spec.H}; the block is "
                             f"E={E}, I={I2 // 2}, H={H}")
        swap_block(blk, experts, router_w, _top_k(blk), spec.score, bias)
        n += 1
    return n
