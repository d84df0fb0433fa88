"""``PhantomTopKRouter``: the reference router module, computed by the HIP router.

Reference: tests/test_moe_routing.py:43-72.  Same constructor
``(hidden_dim, num_experts, top_k=2)``, same ``.gate`` parameter
(``nn.Linear(hidden_dim, num_experts, bias=False)``, weight [E, H]), same
forward contract: ``x [B, S, H] -> (top_weights [B, S, k] in x.dtype,
top_indices [B, S, k] int64)``, indices sorted by descending logit, weights
the softmax over the k selected logits.

Differences, by design:
  - logits are evaluated under a fixed-order fp64 contract, so selection is
    reproducible bit for bit and ties go to the lower expert index;
  - a NaN logit ranks below every number (-inf included), where torch.topk in
    the reference ranks NaN above every number;
  - the module is inference-only: the HIP router has no backward, so forward
    raises when autograd would need a gradient for ``gate.weight`` (wrap the
    call in ``torch.no_grad()`` or set ``gate.weight.requires_grad_(False)``);
  - the module runs only on the GPU; a CPU input raises.
"""
from __future__ import annotations

from typing import Tuple

import torch
import torch.nn as nn

from . import ops


class PhantomTopKRouter(nn.Module):
    """Top-k MoE router (softmax over the selected k logits)."""

    def __init__(self, hidden_dim: int, num_experts: int, top_k: int = 2):
        super().__init__()
        self.hidden_dim = hidden_dim
        self.num_experts = num_experts
        self.top_k = top_k
        self.gate = nn.Linear(hidden_dim, num_experts, bias=False)

    def forward(self, x: torch.Tensor) -> Tuple[torch.Tensor, torch.Tensor]:
        """
        Args:
            x: [batch_size, seq_len, hidden_dim] (any leading shape), bf16/fp16/fp32, on the GPU.
        Returns:
            top_weights: softmax over the selected logits, [..., top_k], x.dtype
            top_indices: selected experts, [..., top_k], int64, descending logit
        """
        if torch.is_grad_enabled() and (self.gate.weight.requires_grad or x.requires_grad):
            raise RuntimeError("PhantomTopKRouter has no backward: call it under torch.no_grad() "
                               "or set gate.weight.requires_grad_(False)")
        w, idx = ops.route(x, self.gate.weight, self.top_k, "softmax",
                           self.gate.bias if self.gate.bias is not None else None)
        return w.to(x.dtype), idx.to(torch.int64)
