"""torch front end of the legacy neuron-sparse FFN ABI (include/phantom_legacy.h).

The C symbols keep the reference's names and arguments
(kernels/sparse_moe/sparse_matmul.cu:240-255, gate_predict.cu:200-213 and
:253-258); these wrappers take torch tensors on the GPU, allocate the
outputs, and raise PhantomMoEError where the C call returns a negative
status (the reference exits the process instead).  There is no CPU path.
"""
from __future__ import annotations

import torch

from . import _lib


def _dev(t: torch.Tensor, what: str, dtype: torch.dtype) -> int:
    if not isinstance(t, torch.Tensor) or t.device.type != "cuda":
        raise _lib.PhantomMoEError(f"{what} must be a tensor on the GPU (there is no CPU path)")
    if t.dtype != dtype:
        raise _lib.PhantomMoEError(f"{what} must be {dtype}, got {t.dtype}")
    if not t.is_contiguous():
        raise _lib.PhantomMoEError(f"{what} must be contiguous")
    return t.data_ptr()


def _opt(t, what: str, dtype: torch.dtype):
    return None if t is None else _dev(t, what, dtype)


def _check(ret: float, what: str) -> float:
    if ret < 0:
        msg = _lib.load().phantom_moe_last_error().decode(errors="replace")
        raise _lib.PhantomMoEError(f"{what} failed (status {int(ret)}): {msg}")
    return ret


def predict_active_neurons(x: torch.Tensor, gate_weights: torch.Tensor, gate_bias: torch.Tensor | None,
                           threshold: float = 0.5, want_gate_output: bool = True):
    """x [B, D] fp16, gate_weights [D_ffn, D] fp16, gate_bias [D_ffn] fp16 or None.

    Returns (mask [B, D_ffn] uint8, indices [B, D_ffn] int32 whose first
    count[b] entries of row b are the active neurons in increasing order,
    count [B] int32, gate [B, D_ffn] fp32 or None, elapsed ms)."""
    B, D = x.shape
    D_ffn = gate_weights.shape[0]
    if gate_weights.shape != (D_ffn, D):
        raise _lib.PhantomMoEError(f"gate_weights must be [D_ffn, {D}], got {tuple(gate_weights.shape)}")
    dev = x.device
    mask = torch.empty((B, D_ffn), dtype=torch.uint8, device=dev)
    idx = torch.full((B, D_ffn), -1, dtype=torch.int32, device=dev)
    cnt = torch.empty((B,), dtype=torch.int32, device=dev)
    gate = torch.empty((B, D_ffn), dtype=torch.float32, device=dev) if want_gate_output else None
    ms = _lib.load().predict_active_neurons(
        _dev(x, "x", torch.float16), _dev(gate_weights, "gate_weights", torch.float16),
        _opt(gate_bias, "gate_bias", torch.float16), mask.data_ptr(), idx.data_ptr(), cnt.data_ptr(),
        None if gate is None else gate.data_ptr(), B, D, D_ffn, float(threshold), _lib.stream_handle(dev))
    _check(ms, "predict_active_neurons")
    return mask, idx, cnt, gate, ms


def sparse_mlp_forward(x: torch.Tensor, gate_weight: torch.Tensor, gate_bias: torch.Tensor | None,
                       up_weight: torch.Tensor, up_bias: torch.Tensor | None, down_weight: torch.Tensor,
                       active_indices: torch.Tensor | None, active_count: torch.Tensor | None,
                       sparsity_pct: float):
    """x [B, D] fp16; gate/up weights [D_ffn, D] fp16, biases [D_ffn] fp16 or
    None; down_weight [D, D_ffn] fp16; active_indices [B, D_ffn] int32 and
    active_count [B] int32 (unused when sparsity_pct < 30).

    Returns (y [B, D] fp16, elapsed ms)."""
    B, D = x.shape
    D_ffn = gate_weight.shape[0]
    for t, name, shape in ((gate_weight, "gate_weight", (D_ffn, D)), (up_weight, "up_weight", (D_ffn, D)),
                           (down_weight, "down_weight", (D, D_ffn))):
        if tuple(t.shape) != shape:
            raise _lib.PhantomMoEError(f"{name} must be {list(shape)}, got {list(t.shape)}")
    y = torch.empty((B, D), dtype=torch.float16, device=x.device)
    ms = _lib.load().sparse_mlp_forward(
        _dev(x, "x", torch.float16), _dev(gate_weight, "gate_weight", torch.float16),
        _opt(gate_bias, "gate_bias", torch.float16), _dev(up_weight, "up_weight", torch.float16),
        _opt(up_bias, "up_bias", torch.float16), _dev(down_weight, "down_weight", torch.float16),
        _opt(active_indices, "active_indices", torch.int32), _opt(active_count, "active_count", torch.int32),
        y.data_ptr(), B, D, D_ffn, float(sparsity_pct), _lib.stream_handle(x.device))
    _check(ms, "sparse_mlp_forward")
    return y, ms


def get_sparsity_stats(active_count: torch.Tensor, D_ffn: int) -> float:
    """Mean sparsity in percent of the counts (waits for the current stream)."""
    B = active_count.numel()
    ret = _lib.load().get_sparsity_stats(_dev(active_count, "active_count", torch.int32), B, int(D_ffn),
                                         _lib.stream_handle(active_count.device))
    if ret != ret:  # NaN: B == 0, as the reference's 0 / 0
        return ret
    return _check(ret, "get_sparsity_stats")


def calibrate_sparsity_gate(inputs: torch.Tensor, mlp_activations: torch.Tensor):
    """inputs [N, D] fp32, mlp_activations [N, D_ffn] fp32 (on the GPU).

    Returns (gate_w [D_ffn, D] fp32, gate_b [D_ffn] fp32, enabled, f1, sparsity_pct)."""
    import ctypes

    N, D = inputs.shape
    if mlp_activations.shape[0] != N:
        raise _lib.PhantomMoEError("inputs and mlp_activations must have the same number of rows")
    D_ffn = mlp_activations.shape[1]
    w = torch.empty((D_ffn, D), dtype=torch.float32, device=inputs.device)
    b = torch.empty((D_ffn,), dtype=torch.float32, device=inputs.device)
    en, f1, sp = ctypes.c_bool(False), ctypes.c_float(0.0), ctypes.c_float(0.0)
    rc = _lib.load().calibrate_sparsity_gate(
        _dev(inputs, "inputs", torch.float32), _dev(mlp_activations, "mlp_activations", torch.float32), N, D, D_ffn,
        w.data_ptr(), b.data_ptr(), ctypes.addressof(en), ctypes.addressof(f1), ctypes.addressof(sp),
        _lib.stream_handle(inputs.device))
    _lib.check(rc, "calibrate_sparsity_gate")
    return w, b, bool(en.value), float(f1.value), float(sp.value)
