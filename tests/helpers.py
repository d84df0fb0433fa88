"""Shared helpers of the parity tests (no product code depends on them)."""
from __future__ import annotations

import numpy as np

from oracle import oracle

# Output tolerance of the MoE layer against the fp64 oracle.
MAX_ABS = 1e-2
REL_L2 = 1e-3


def check_y(y_gpu, y_ref, what=""):
    """max |y - y_ref| <= 1e-2 and ||y - y_ref|| / ||y_ref|| <= 1e-3."""
    y = np.asarray(y_gpu, dtype=np.float64)
    r = np.asarray(y_ref, dtype=np.float64)
    assert y.shape == r.shape, (y.shape, r.shape)
    assert np.isfinite(y).all(), f"{what}: non-finite output"
    err = np.abs(y - r).max() if y.size else 0.0
    rel = np.linalg.norm(y - r) / max(np.linalg.norm(r), 1e-30)
    assert err <= MAX_ABS and rel <= REL_L2, f"{what}: max abs {err:.3e}, rel-L2 {rel:.3e}"
    return err, rel


def repacked_layout(q4: np.ndarray, rows: int, K: int):
    """Restates the repacked layout from its definition, for checking the
    device repack: (nib uint8 [rows*Kpad/2], scale uint16 [rows*Kpad/32])."""
    q4 = q4.reshape(rows, K // 32, 18)
    Kg = K // 32
    Kq = -(-K // 128)
    nib = np.empty((rows // 16, Kq, 64, 4, 4), dtype=np.uint8)
    sc = np.zeros((rows // 16, Kq, 16, 4), dtype=np.uint16)
    d = np.ascontiguousarray(q4[..., 0:2]).view(np.uint16)[..., 0]
    for lane in range(64):
        n, p = lane % 16, lane // 16
        for gi in range(4):
            g = np.arange(Kq) * 4 + gi
            valid = g < Kg
            gg = np.minimum(g, Kg - 1)
            rowsel = np.arange(rows // 16)[:, None] * 16 + n
            bytes4 = q4[rowsel, gg[None, :], 2 + 4 * p: 6 + 4 * p]  # [rt, Kq, 4]
            nib[:, :, lane, gi, :] = np.where(valid[None, :, None], bytes4, 0x88)
            if p == 0:
                sc[:, :, n, gi] = np.where(valid[None, :], d[rowsel, gg[None, :]], 0)
    return nib.reshape(-1), sc.reshape(-1)


def to_bf16_tensor(xb: np.ndarray, device):
    import torch

    return torch.from_numpy(np.ascontiguousarray(xb).view(np.int16)).view(torch.bfloat16).to(device)


def bf16_tensor_bits(x) -> np.ndarray:
    import torch

    return x.detach().contiguous().view(torch.int16).cpu().numpy().view(np.uint16)


def oracle_for_device_layer(dl, xb: np.ndarray, tokens=None):
    """Oracle result for a synth.DeviceLayer: route the tokens on the host,
    copy only the experts they use back from the device (the rest of the
    host expert arrays stay untouched zero pages), and run the oracle layer."""
    cfg = dl.cfg
    W = dl.router_w.cpu().numpy()
    b = None if dl.router_bias is None else dl.router_bias.cpu().numpy()
    xs = xb if tokens is None else xb[np.asarray(tokens)]
    idx, _ = oracle.route(xs, W, cfg.k, cfg.score_mode, b)
    used = np.unique(idx)
    g = np.zeros(tuple(dl.gate.shape), dtype=np.uint8)
    u = np.zeros(tuple(dl.up.shape), dtype=np.uint8)
    d = np.zeros(tuple(dl.down.shape), dtype=np.uint8)
    for e in used:
        g[e] = dl.gate[int(e)].cpu().numpy()
        u[e] = dl.up[int(e)].cpu().numpy()
        d[e] = dl.down[int(e)].cpu().numpy()
    shared = None if dl.shared is None else tuple(t.cpu().numpy() for t in dl.shared)
    return oracle.moe_forward(xs, W, g, u, d, cfg.k, cfg.score_mode, b, shared=shared)
