"""Seeded synthetic MoE layers of the benchmark shapes.

Distributions: activations N(0, 1) rounded to bf16; router weight fp32
N(0, 0.02) in nn.Linear layout [E, H]; expert weights Q4_0 with q uniform in
[-8, 7] (uniform random qs bytes) and scales |N(0, 0.02)| in fp16.  Seeds:
activations 42, router 7, expert weights of layer instance l 1000 + l, shared
expert 2000 + l, Zipf permutation 3.

Zipf-skewed routing (the 32-token Qwen3 decode case): a fixed bias
b_e = -s * ln(r_e) with r = 1 + a seeded permutation of 0..E-1 is added to the
router logits (as an nn.Linear bias), so a few experts take most tokens.
"""
from __future__ import annotations

from dataclasses import dataclass, field

import numpy as np

from . import q4_0


@dataclass(frozen=True)
class MoEConfig:
    name: str
    H: int
    I: int
    E: int
    k: int
    T: int
    score: str = "softmax"
    shared: bool = False
    zipf: float = 0.0
    notes: str = field(default="", compare=False)

    @property
    def score_mode(self) -> int:
        return 0 if self.score == "softmax" else 1

    def expert_bytes(self) -> int:
        """Q4_0 bytes of one expert (gate + up + down)."""
        return 3 * self.H * self.I // 32 * 18


CONFIGS = {
    c.name: c
    for c in [
        MoEConfig("qwen3_decode_t1", 2048, 768, 128, 8, 1),
        MoEConfig("qwen3_decode_t32_zipf", 2048, 768, 128, 8, 32, zipf=1.1),
        MoEConfig("mixtral_decode_t1", 4096, 14336, 8, 2, 1),
        MoEConfig("mixtral_decode_t16", 4096, 14336, 8, 2, 16),
        MoEConfig("qwen3_prefill_t4096", 2048, 768, 128, 8, 4096),
        MoEConfig("dsv3_decode_t1", 7168, 2048, 256, 8, 1, score="sigmoid", shared=True),
        MoEConfig("dsv3_decode_t8", 7168, 2048, 256, 8, 8, score="sigmoid", shared=True),
        MoEConfig("dsv3_decode_t64", 7168, 2048, 256, 8, 64, score="sigmoid", shared=True),
        MoEConfig("dsv3_prefill_t2048", 7168, 2048, 256, 8, 2048, score="sigmoid", shared=True),
    ]
}


def f32_to_bf16_bits(a: np.ndarray) -> np.ndarray:
    """Round-to-nearest-even fp32 -> bf16 bit patterns (uint16); finite inputs."""
    u = np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)
    r = (u + np.uint32(0x7FFF) + ((u >> np.uint32(16)) & np.uint32(1))) >> np.uint32(16)
    return r.astype(np.uint16)


def bf16_bits_to_f32(b: np.ndarray) -> np.ndarray:
    return (np.asarray(b, dtype=np.uint16).astype(np.uint32) << np.uint32(16)).view(np.float32)


def activations(T: int, H: int, seed: int = 42) -> np.ndarray:
    """x ~ N(0, 1) as bf16 bits [T, H] (uint16)."""
    rng = np.random.default_rng(seed)
    return f32_to_bf16_bits(rng.standard_normal((T, H), dtype=np.float32))


def router_weight(E: int, H: int, seed: int = 7) -> np.ndarray:
    rng = np.random.default_rng(seed)
    return (rng.standard_normal((E, H), dtype=np.float32) * np.float32(0.02)).astype(np.float32)


def zipf_bias(E: int, s: float, seed: int = 3) -> np.ndarray:
    """b_e = -s * ln(r_e), r = 1 + seeded permutation of 0..E-1 (fp32)."""
    r = 1 + np.random.default_rng(seed).permutation(E)
    return (-s * np.log(r.astype(np.float64))).astype(np.float32)


@dataclass
class HostLayer:
    """One MoE layer instance on the host (GGUF Q4_0 bytes)."""

    cfg: MoEConfig
    router_w: np.ndarray            # [E, H] fp32
    router_bias: np.ndarray | None  # [E] fp32
    gate: np.ndarray                # [E, I, H/32, 18] uint8
    up: np.ndarray                  # [E, I, H/32, 18]
    down: np.ndarray                # [E, H, I/32, 18]
    shared: tuple | None            # (gate [I,H/32,18], up, down [H,I/32,18]) or None


def host_layer(cfg: MoEConfig, layer: int = 0, router_seed: int = 7) -> HostLayer:
    rng = np.random.default_rng(1000 + layer)
    gate = q4_0.random_blocks(rng, (cfg.E, cfg.I, cfg.H))
    up = q4_0.random_blocks(rng, (cfg.E, cfg.I, cfg.H))
    down = q4_0.random_blocks(rng, (cfg.E, cfg.H, cfg.I))
    shared = None
    if cfg.shared:
        srng = np.random.default_rng(2000 + layer)
        shared = (
            q4_0.random_blocks(srng, (cfg.I, cfg.H)),
            q4_0.random_blocks(srng, (cfg.I, cfg.H)),
            q4_0.random_blocks(srng, (cfg.H, cfg.I)),
        )
    bias = zipf_bias(cfg.E, cfg.zipf) if cfg.zipf else None
    return HostLayer(cfg, router_weight(cfg.E, cfg.H, router_seed), bias, gate, up, down, shared)


def scaled(cfg: MoEConfig, **changes) -> MoEConfig:
    """A copy of cfg with some fields replaced (for reduced-size parity cases)."""
    d = dict(cfg.__dict__)
    d.update(changes)
    return MoEConfig(**d)


def device_q4_0(shape, gen, device, scale_sigma: float = 0.02):
    """Q4_0 bytes for a [..., K] tensor generated on ``device`` with the
    torch generator ``gen`` (same distributions as :func:`q4_0.random_blocks`).
    Returns uint8 [..., K/32, 18]."""
    import torch

    *lead, K = shape
    nb = K // 32
    qs = torch.randint(0, 256, (*lead, nb, 16), generator=gen, device=device, dtype=torch.uint8)
    d = (torch.randn((*lead, nb, 1), generator=gen, device=device, dtype=torch.float32).abs() * scale_sigma)
    d = d.to(torch.float16).view(torch.uint8)
    return torch.cat([d, qs], dim=-1).contiguous()


@dataclass
class DeviceLayer:
    """One MoE layer instance generated directly in device memory."""

    cfg: MoEConfig
    router_w: object       # torch fp32 [E, H]
    router_bias: object    # torch fp32 [E] or None
    gate: object           # torch uint8 [E, I, H/32, 18]
    up: object
    down: object           # [E, H, I/32, 18]
    shared: tuple | None


def device_layer(cfg: MoEConfig, device, layer: int = 0, router_seed: int = 7) -> DeviceLayer:
    """Like :func:`host_layer` but generated on the device (fast for the
    multi-GB shapes); the byte streams differ from the host generator's."""
    import torch

    g = torch.Generator(device=device)
    g.manual_seed(1000 + layer)
    gate = device_q4_0((cfg.E, cfg.I, cfg.H), g, device)
    up = device_q4_0((cfg.E, cfg.I, cfg.H), g, device)
    down = device_q4_0((cfg.E, cfg.H, cfg.I), g, device)
    shared = None
    if cfg.shared:
        sg = torch.Generator(device=device)
        sg.manual_seed(2000 + layer)
        shared = (device_q4_0((cfg.I, cfg.H), sg, device), device_q4_0((cfg.I, cfg.H), sg, device),
                  device_q4_0((cfg.H, cfg.I), sg, device))
    rg = torch.Generator(device=device)
    rg.manual_seed(router_seed + 10 * layer)
    W = torch.randn((cfg.E, cfg.H), generator=rg, device=device, dtype=torch.float32) * 0.02
    bias = torch.from_numpy(zipf_bias(cfg.E, cfg.zipf)).to(device) if cfg.zipf else None
    return DeviceLayer(cfg, W, bias, gate, up, down, shared)
