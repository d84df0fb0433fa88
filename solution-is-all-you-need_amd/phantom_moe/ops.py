"""Python operator surface of the MI355X sparse-MoE layer.

``moe_forward`` is the whole layer (router -> permute -> Q4_0 SwiGLU experts
-> weighted combine); ``route`` and ``permute`` expose the first two stages.
All computation runs in libphantom_moe.so on the tensors' device and stream;
there is no CPU path.

Reference surface mirrored: ``PhantomTopKRouter`` semantics
(tests/test_moe_routing.py:43-72: logits = x W^T, top-k sorted descending,
softmax over the k) and the Q4_0 expert weights the GGUF loader reads
(python/phantom/loader/gguf_loader.py:362-381).  The combine follows the
index_add_ of w * FFN_e(x) that transformers' MoE blocks perform, which is
where the reference runs MoE layers (python/phantom/phantom_cli.py:1393-1430).
"""
from __future__ import annotations

import threading
from dataclasses import dataclass

import torch

from . import _lib, q4_0

SCORE_MODES = {"softmax": 0, "sigmoid": 1}

_ws_lock = threading.Lock()
_workspaces: dict = {}


def _score_mode(score) -> int:
    if isinstance(score, int) and score in (0, 1):
        return score
    if score not in SCORE_MODES:
        raise ValueError(f"score must be one of {sorted(SCORE_MODES)}, got {score!r}")
    return SCORE_MODES[score]


def _need_cuda(t: torch.Tensor, what: str) -> None:
    if not isinstance(t, torch.Tensor):
        raise TypeError(f"{what} must be a torch.Tensor")
    if t.device.type != "cuda":
        raise RuntimeError(f"{what} must live on the GPU (got {t.device}); this operator has no CPU path")


def workspace(device: torch.device, nbytes: int, stream: int | None = None) -> torch.Tensor:
    """Workspace of at least nbytes for (device, current stream).

    Cached per (device, stream) so calls on one stream reuse it in order;
    grows when a larger one is asked for.  Zero-filled when allocated (the
    library keeps the call counter of its single-launch path in it).
    ``stream``: the current stream's handle when the caller has it."""
    if stream is None:
        stream = _lib.stream_handle(device)
    key = (device.index, stream)
    with _ws_lock:
        ws = _workspaces.get(key)
        if ws is None or ws.numel() < nbytes:
            ws = torch.zeros(max(nbytes, 1 << 16), dtype=torch.uint8, device=device)
            _workspaces[key] = ws
        return ws


def _x_bf16(x: torch.Tensor) -> torch.Tensor:
    if x.dtype != torch.bfloat16:
        raise TypeError(f"moe_forward takes bf16 activations, got {x.dtype}")
    return x.contiguous()


@dataclass
class MoEWeights:
    """Repacked Q4_0 expert weights of one MoE layer, resident on one device.

    gate/up: E stacked [I, H]; down: E stacked [H, I]; optional shared expert.
    Build with :meth:`from_q4_0` from GGUF Q4_0 bytes."""

    H: int
    I: int
    E: int
    gate_nib: torch.Tensor
    gate_scale: torch.Tensor
    up_nib: torch.Tensor
    up_scale: torch.Tensor
    down_nib: torch.Tensor
    down_scale: torch.Tensor
    shared: tuple | None = None  # (gate_nib, gate_scale, up_nib, up_scale, down_nib, down_scale)

    @classmethod
    def from_q4_0(cls, gate: torch.Tensor, up: torch.Tensor, down: torch.Tensor, H: int, I: int, E: int,
                  shared: tuple | None = None) -> "MoEWeights":
        """gate/up: uint8 device tensors of E x [I, H] Q4_0; down: E x [H, I] Q4_0.
        shared: None or (gate, up, down) of one expert in the same layout."""
        gn, gs = q4_0.repack(gate.reshape(-1), I, H, E)
        un, us = q4_0.repack(up.reshape(-1), I, H, E)
        dn, ds = q4_0.repack(down.reshape(-1), H, I, E)
        sh = None
        if shared is not None:
            sgn, sgs = q4_0.repack(shared[0].reshape(-1), I, H, 1)
            sun, sus = q4_0.repack(shared[1].reshape(-1), I, H, 1)
            sdn, sds = q4_0.repack(shared[2].reshape(-1), H, I, 1)
            sh = (sgn, sgs, sun, sus, sdn, sds)
        return cls(H, I, E, gn, gs, un, us, dn, ds, sh)

    @property
    def device(self) -> torch.device:
        return self.gate_nib.device

    def nbytes(self) -> int:
        ts = [self.gate_nib, self.gate_scale, self.up_nib, self.up_scale, self.down_nib, self.down_scale]
        if self.shared:
            ts += list(self.shared)
        return sum(t.numel() * t.element_size() for t in ts)


def route(x: torch.Tensor, router_weight: torch.Tensor, top_k: int, score="softmax", router_bias=None):
    """Router only.  x [T, H] bf16 or fp32 (leading dims are flattened);
    router_weight [E, H] fp32.  Returns (topk_w fp32 [T, k], topk_idx int32 [T, k])."""
    _need_cuda(x, "x")
    lead = x.shape[:-1]
    H = x.shape[-1]
    x2 = x.reshape(-1, H)
    if x2.dtype == torch.float16:
        x2 = x2.float()  # exact widening
    if x2.dtype not in (torch.bfloat16, torch.float32):
        raise TypeError(f"x must be bf16, fp16 or fp32, got {x.dtype}")
    x2 = x2.contiguous()
    W = router_weight.detach().to(device=x.device, dtype=torch.float32).contiguous()
    E = W.shape[0]
    if W.shape != (E, H):
        raise ValueError(f"router_weight must be [E, {H}], got {tuple(W.shape)}")
    b = None
    if router_bias is not None:
        b = router_bias.detach().to(device=x.device, dtype=torch.float32).contiguous()
    T = x2.shape[0]
    idx = torch.empty((T, top_k), dtype=torch.int32, device=x.device)
    w = torch.empty((T, top_k), dtype=torch.float32, device=x.device)
    if T == 0:  # an empty batch routes to empty outputs
        return w.reshape(*lead, top_k), idx.reshape(*lead, top_k)
    lib = _lib.load()
    nbytes = lib.phantom_moe_workspace_bytes(T, H, 0, E, top_k, 0)
    ws = workspace(x.device, nbytes)
    rc = lib.phantom_moe_route(
        x2.data_ptr(), 0 if x2.dtype == torch.bfloat16 else 1, W.data_ptr(), None if b is None else b.data_ptr(),
        T, H, E, top_k, _score_mode(score), idx.data_ptr(), w.data_ptr(), ws.data_ptr(), ws.numel(),
        _lib.stream_handle(x.device),
    )
    _lib.check(rc, "phantom_moe_route")
    return w.reshape(*lead, top_k), idx.reshape(*lead, top_k)


def permute(topk_idx: torch.Tensor, num_experts: int):
    """Stable counting sort of (token, slot) pairs by expert.

    Returns (expert_offsets [E+1], sorted_slots [T*k], slot_pos [T*k]), int32."""
    _need_cuda(topk_idx, "topk_idx")
    idx = topk_idx.to(torch.int32).contiguous()
    k = idx.shape[-1]
    T = idx.numel() // k
    off = torch.empty(num_experts + 1, dtype=torch.int32, device=idx.device)
    ss = torch.empty(T * k, dtype=torch.int32, device=idx.device)
    sp = torch.empty(T * k, dtype=torch.int32, device=idx.device)
    if T == 0:  # no slots: every segment is empty
        return off.zero_(), ss, sp
    lib = _lib.load()
    nbytes = lib.phantom_moe_workspace_bytes(T, 32, 0, num_experts, k, 0)
    ws = workspace(idx.device, nbytes)
    rc = lib.phantom_moe_permute(idx.data_ptr(), T, k, num_experts, off.data_ptr(), ss.data_ptr(), sp.data_ptr(),
                                 ws.data_ptr(), ws.numel(), _lib.stream_handle(idx.device))
    _lib.check(rc, "phantom_moe_permute")
    return off, ss, sp


# phantom_moe_workspace_bytes per forward shape (T, H, I, E, k, shared)
_ws_bytes: dict = {}


def moe_forward(x: torch.Tensor, router_weight: torch.Tensor, experts: MoEWeights, top_k: int,
                score="softmax", router_bias=None, return_routing: bool = False, out: torch.Tensor | None = None):
    """The MoE layer: y[t] = sum_j w[t,j] FFN_{e[t,j]}(x[t]) (+ shared expert).

    x: [T, H] bf16 on the GPU (leading dims flattened); router_weight [E, H]
    fp32; experts: :class:`MoEWeights`.  Returns y fp32 of x's shape, and with
    return_routing=True also (topk_w fp32 [.., k], topk_idx int32 [.., k])."""
    _need_cuda(x, "x")
    H = experts.H
    if x.shape[-1] != H:
        raise ValueError(f"x has hidden size {x.shape[-1]}, experts expect {H}")
    lead = x.shape[:-1]
    x2 = _x_bf16(x.reshape(-1, H))
    T = x2.shape[0]
    E = experts.E
    W = router_weight
    if W.dtype != torch.float32 or W.device != x.device or not W.is_contiguous():
        W = W.detach().to(device=x.device, dtype=torch.float32).contiguous()
    if tuple(W.shape) != (E, H):
        raise ValueError(f"router_weight must be [{E}, {H}], got {tuple(W.shape)}")
    b = router_bias
    if b is not None and (b.dtype != torch.float32 or b.device != x.device or not b.is_contiguous()):
        b = b.detach().to(device=x.device, dtype=torch.float32).contiguous()
    if experts.device != x.device:
        raise ValueError(f"experts live on {experts.device}, x on {x.device}")
    y = out if out is not None else torch.empty((T, H), dtype=torch.float32, device=x.device)
    if y.dtype != torch.float32 or y.numel() != T * H or not y.is_contiguous():
        raise ValueError("out must be a contiguous fp32 tensor with T*H elements")
    idx = torch.empty((T, top_k), dtype=torch.int32, device=x.device)
    w = torch.empty((T, top_k), dtype=torch.float32, device=x.device)
    if T == 0:  # an empty batch: empty outputs, as torch's own operators give
        y = y.reshape(*lead, H)
        return (y, w.reshape(*lead, top_k), idx.reshape(*lead, top_k)) if return_routing else y
    lib = _lib.load()
    _lib.check_status()  # a failure an earlier call left
    has_sh = experts.shared is not None
    shape = (T, H, experts.I, E, top_k, int(has_sh))
    nbytes = _ws_bytes.get(shape)
    if nbytes is None:
        nbytes = _ws_bytes[shape] = lib.phantom_moe_workspace_bytes(*shape)
    stream = _lib.stream_handle(x.device)
    ws = workspace(x.device, nbytes, stream)
    sh = [t.data_ptr() for t in experts.shared] if has_sh else [None] * 6
    rc = lib.phantom_moe_forward(
        x2.data_ptr(), 0, T, H, experts.I, E, top_k, _score_mode(score), W.data_ptr(),
        None if b is None else b.data_ptr(),
        experts.gate_nib.data_ptr(), experts.gate_scale.data_ptr(), experts.up_nib.data_ptr(),
        experts.up_scale.data_ptr(), experts.down_nib.data_ptr(), experts.down_scale.data_ptr(),
        *sh, y.data_ptr(), idx.data_ptr(), w.data_ptr(), ws.data_ptr(), ws.numel(), stream,
    )
    _lib.check(rc, "phantom_moe_forward")
    _lib.after_call(x.device)
    y = y.reshape(*lead, H)
    if return_routing:
        return y, w.reshape(*lead, top_k), idx.reshape(*lead, top_k)
    return y


class PreparedForward:
    """A ``moe_forward`` call with every pointer bound once.

    For decode loops that call one layer repeatedly on fixed buffers: the
    caller writes tokens into ``self.x`` and calls the object, which issues
    the layer on the current stream of the device with one C call and no
    allocation.  Outputs land in ``self.y`` (fp32 [T, H]), ``self.topk_w`` and
    ``self.topk_idx``."""

    def __init__(self, experts: MoEWeights, router_weight: torch.Tensor, T: int, top_k: int, score="softmax",
                 router_bias=None, x: torch.Tensor | None = None):
        import ctypes

        dev = experts.device
        H, I, E = experts.H, experts.I, experts.E
        self.experts = experts
        self.router_weight = router_weight.detach().to(device=dev, dtype=torch.float32).contiguous()
        if tuple(self.router_weight.shape) != (E, H):
            raise ValueError(f"router_weight must be [{E}, {H}]")
        self.router_bias = None
        if router_bias is not None:
            self.router_bias = router_bias.detach().to(device=dev, dtype=torch.float32).contiguous()
        self.x = x if x is not None else torch.zeros((T, H), dtype=torch.bfloat16, device=dev)
        if self.x.dtype != torch.bfloat16 or tuple(self.x.shape) != (T, H) or not self.x.is_contiguous():
            raise ValueError("x must be a contiguous bf16 [T, H] tensor")
        self.y = torch.empty((T, H), dtype=torch.float32, device=dev)
        self.topk_idx = torch.empty((T, top_k), dtype=torch.int32, device=dev)
        self.topk_w = torch.empty((T, top_k), dtype=torch.float32, device=dev)
        lib = _lib.load()
        has_sh = experts.shared is not None
        nbytes = lib.phantom_moe_workspace_bytes(T, H, I, E, top_k, int(has_sh))
        self.workspace = torch.zeros(nbytes, dtype=torch.uint8, device=dev)
        sh = [t.data_ptr() for t in experts.shared] if has_sh else [None] * 6
        self._fn = lib.phantom_moe_forward
        self._args = [
            self.x.data_ptr(), 0, T, H, I, E, top_k, _score_mode(score), self.router_weight.data_ptr(),
            None if self.router_bias is None else self.router_bias.data_ptr(),
            experts.gate_nib.data_ptr(), experts.gate_scale.data_ptr(), experts.up_nib.data_ptr(),
            experts.up_scale.data_ptr(), experts.down_nib.data_ptr(), experts.down_scale.data_ptr(),
            *sh, self.y.data_ptr(), self.topk_idx.data_ptr(), self.topk_w.data_ptr(),
            self.workspace.data_ptr(), nbytes,
        ]
        self.device = dev
        self._ctypes = ctypes

    def __call__(self, stream: int | None = None) -> torch.Tensor:
        _lib.check_status()
        s = _lib.stream_handle(self.device) if stream is None else stream
        rc = self._fn(*self._args, s)
        if rc:
            _lib.check(rc, "phantom_moe_forward")
        _lib.after_call(self.device)
        return self.y
