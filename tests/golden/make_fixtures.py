"""Writes the golden fixtures in this directory.

Nothing here runs the reference or the oracle.  Expected values come from:
  - the Q4_0 known-answer vector of the reference's own audit
    (tests/audit_suite.py:36-41: d = 1.5, qs = 0x88 * 16 -> 32 zeros) and
    hand-derived vectors from the block definition
    (python/phantom/loader/gguf_loader.py:369-378);
  - numpy float64 library routines (matmul, stable argsort, bincount,
    cumsum) and scipy's softmax / expit, on seeded inputs whose top-k logit
    gaps are far larger than any summation-order effect, so the expected
    selection does not depend on accumulation order;
  - the synthetic Zipf bias definition (b_e = -s ln r_e);
  - torch fp32 on the CPU for router_reference_module.npz: the reference
    router's forward, F.linear -> torch.topk -> softmax over the top-k logits
    (tests/test_moe_routing.py:65-71), written out here with torch's own
    operators (the reference module is not imported), on the benchmark
    layers' seeded activations and router weights.

Run:  python tests/golden/make_fixtures.py
"""
from __future__ import annotations

import json
import os

import sys

import numpy as np
from scipy.special import expit, softmax

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(HERE, "..", "..", "solution-is-all-you-need_amd"))


def f16_bits(v: float) -> int:
    return int(np.array([v], dtype=np.float16).view(np.uint16)[0])


def q4_0_vectors():
    vecs = []

    def add(name, d, qs, expected):
        vecs.append({"name": name, "d_f16_bits": f16_bits(d), "qs": list(qs), "expected": [float(v) for v in expected]})

    # The reference audit KAT: 0x88 bytes are nibble 8 in both halves -> q = 0.
    add("audit_0x88_d1.5", 1.5, [0x88] * 16, [0.0] * 32)
    # Nibble 0 -> q = -8; nibble 15 -> q = 7.
    add("all_0x00_d0.5", 0.5, [0x00] * 16, [-4.0] * 32)
    add("all_0xff_d0.25", 0.25, [0xFF] * 16, [1.75] * 32)
    # Low nibble -> elements 0..15, high nibble -> elements 16..31.
    add("0x10_d1", 1.0, [0x10] * 16, [-8.0] * 16 + [-7.0] * 16)
    add("0x01_d1", 1.0, [0x01] * 16, [-7.0] * 16 + [-8.0] * 16)
    # Byte j holds (j, 15 - j): element j = j - 8, element j + 16 = 7 - j.
    add("ramp_d2", 2.0, [(j) | ((15 - j) << 4) for j in range(16)],
        [2.0 * (j - 8) for j in range(16)] + [2.0 * (7 - j) for j in range(16)])
    # Negative scale flips signs.
    add("0x9a_d-1", -1.0, [0x9A] * 16, [-(0xA - 8)] * 16 + [-(0x9 - 8)] * 16)
    # Smallest fp16 subnormal scale: values are q * 2^-24 exactly.
    d = float(np.array([0x0001], dtype=np.uint16).view(np.float16)[0])
    add("subnormal_scale", d, [0x2F] * 16, [(0xF - 8) * d] * 16 + [(0x2 - 8) * d] * 16)
    return vecs


def bf16_round(a: np.ndarray) -> np.ndarray:
    u = a.astype(np.float32).view(np.uint32)
    r = (u + np.uint32(0x7FFF) + ((u >> np.uint32(16)) & np.uint32(1))) >> np.uint32(16)
    return r.astype(np.uint16)


def router_case(seed, T, H, E, k, score, zipf=0.0, x_bf16=True, dup_rows=None):
    rng = np.random.default_rng(seed)
    x32 = rng.standard_normal((T, H), dtype=np.float32)
    xb = bf16_round(x32)
    xv = (xb.astype(np.uint32) << 16).view(np.float32) if x_bf16 else x32
    W = (rng.standard_normal((E, H), dtype=np.float32) * np.float32(0.02)).astype(np.float32)
    if dup_rows:
        for a, b in dup_rows:
            W[b] = W[a]
    bias = None
    if zipf:
        r = 1 + np.random.default_rng(3).permutation(E)
        bias = (-zipf * np.log(r.astype(np.float64))).astype(np.float32)
    logits = xv.astype(np.float64) @ W.astype(np.float64).T
    if bias is not None:
        logits = logits + bias.astype(np.float64)
    order = np.argsort(-logits, axis=1, kind="stable")
    idx = order[:, :k]
    top = np.take_along_axis(logits, idx, axis=1)
    # The expected selection must not hinge on summation order: every gap
    # between consecutive ranks up to k (and k vs k+1) must be wide, except
    # exact ties created on purpose by duplicated rows.
    srt = np.take_along_axis(logits, order[:, : k + 1], axis=1)
    gaps = -np.diff(srt, axis=1)
    assert np.all((gaps > 1e-9) | (gaps == 0.0)), "near tie in fixture"
    if score == "softmax":
        w = softmax(top, axis=1)
    else:
        s = expit(top)
        w = s / s.sum(axis=1, keepdims=True)
    out = {
        "x": xb if x_bf16 else x32,
        "W": W,
        "idx": idx.astype(np.int32),
        "w": w.astype(np.float32),
        "k": np.int32(k),
        "score": np.int32(0 if score == "softmax" else 1),
    }
    if bias is not None:
        out["bias"] = bias
    return out


def permute_case(seed, T, k, E):
    rng = np.random.default_rng(seed)
    # Skewed draw so some experts are empty and some are crowded.
    p = 1.0 / np.arange(1, E + 1) ** 1.2
    p /= p.sum()
    idx = np.stack([rng.choice(E, size=k, replace=False, p=p) for _ in range(T)]).astype(np.int32)
    flat = idx.reshape(-1)
    counts = np.bincount(flat, minlength=E)
    offsets = np.concatenate([[0], np.cumsum(counts)]).astype(np.int32)
    sorted_slots = np.argsort(flat, kind="stable").astype(np.int32)
    slot_pos = np.empty_like(sorted_slots)
    slot_pos[sorted_slots] = np.arange(flat.size, dtype=np.int32)
    return {"idx": idx, "offsets": offsets, "sorted_slots": sorted_slots, "slot_pos": slot_pos, "E": np.int32(E)}


# Tokens of each benchmark layer that the reference-module fixture covers: all
# of them up to 64 tokens, the first 1024 of a prefill batch.
REFMOD_MAX_TOKENS = 1024


def reference_module_routing():
    """Per benchmark layer: the reference router's fp32 selection and weights.

    The reference module (tests/test_moe_routing.py:43-71) is nn.Linear(H, E,
    bias=False) -> torch.topk(logits, k) -> softmax(top logits), all fp32.  The
    Zipf-skewed layer adds its fixed bias as the Linear's bias.  x is the
    layer's bf16 activations widened to fp32 (the module needs x in the
    weight's dtype).  The sigmoid-scored layers keep the top-k indices only
    (the reference module has no sigmoid scoring; sigmoid is monotone, so the
    selection is the same top-k of the logits).

    A token is marked exempt when two of its k+1 largest fp64 logits are
    closer than twice the largest |fp32 - fp64| logit difference of that
    token: only there can fp32 and fp64 order the logits differently.
    """
    import torch
    import torch.nn.functional as F
    from phantom_moe import synth

    torch.set_num_threads(8)
    out = {}
    for name, cfg in synth.CONFIGS.items():
        n = min(cfg.T, REFMOD_MAX_TOKENS)
        xb = synth.activations(cfg.T, cfg.H)[:n]
        W = synth.router_weight(cfg.E, cfg.H)
        b = synth.zipf_bias(cfg.E, cfg.zipf) if cfg.zipf else None
        x = torch.from_numpy(synth.bf16_bits_to_f32(xb))
        with torch.no_grad():
            logits = F.linear(x, torch.from_numpy(W), None if b is None else torch.from_numpy(b))
            top, idx = torch.topk(logits, cfg.k, dim=-1)
            w = F.softmax(top, dim=-1)
        l64 = synth.bf16_bits_to_f32(xb).astype(np.float64) @ W.astype(np.float64).T
        if b is not None:
            l64 = l64 + b.astype(np.float64)
        err = np.abs(logits.numpy().astype(np.float64) - l64).max(axis=1)
        srt = -np.sort(-l64, axis=1)[:, : cfg.k + 1]
        gap = (-np.diff(srt, axis=1)).min(axis=1)
        out[f"{name}__idx"] = idx.numpy().astype(np.int16)
        if cfg.score == "softmax":
            out[f"{name}__w"] = w.numpy().astype(np.float32)
        out[f"{name}__exempt"] = (gap <= 2 * err)
        print(f"{name}: {n} tokens, {int(out[name + '__exempt'].sum())} exempt, "
              f"max fp32 logit error {err.max():.3g}, min gap {gap.min():.3g}")
    return out


def main():
    with open(os.path.join(HERE, "q4_0_kat.json"), "w") as f:
        json.dump({"source": "tests/audit_suite.py:36-41 and gguf_loader.py:369-378 (hand-derived)",
                   "vectors": q4_0_vectors()}, f, indent=1)
    np.savez_compressed(os.path.join(HERE, "router_ref_test_shape.npz"),
                        **router_case(11, 8, 256, 8, 2, "softmax"))
    np.savez_compressed(os.path.join(HERE, "router_ref_test_shape_f32.npz"),
                        **router_case(12, 8, 256, 8, 2, "softmax", x_bf16=False))
    np.savez_compressed(os.path.join(HERE, "router_e128_k8_t4.npz"),
                        **router_case(13, 4, 1024, 128, 8, "softmax"))
    np.savez_compressed(os.path.join(HERE, "router_zipf_t8.npz"),
                        **router_case(14, 8, 512, 128, 8, "softmax", zipf=1.1))
    np.savez_compressed(os.path.join(HERE, "router_sigmoid_t4.npz"),
                        **router_case(15, 4, 512, 64, 8, "sigmoid"))
    np.savez_compressed(os.path.join(HERE, "router_ties.npz"),
                        **router_case(16, 6, 256, 16, 4, "softmax", dup_rows=[(3, 9), (5, 6), (0, 15)]))
    np.savez_compressed(os.path.join(HERE, "permute_t64_k8_e32.npz"), **permute_case(21, 64, 8, 32))
    np.savez_compressed(os.path.join(HERE, "permute_t5_k2_e8.npz"), **permute_case(22, 5, 2, 8))
    r = 1 + np.random.default_rng(3).permutation(128)
    np.save(os.path.join(HERE, "zipf_bias_e128_s1.1.npy"), (-1.1 * np.log(r.astype(np.float64))).astype(np.float32))
    np.savez_compressed(os.path.join(HERE, "router_reference_module.npz"), **reference_module_routing())
    print("fixtures written to", HERE)


if __name__ == "__main__":
    main()
