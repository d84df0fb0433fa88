"""Pins the CPU oracle (oracle/moe_oracle.c) before it is trusted as the
parity reference of the HIP library.

Each oracle function is checked against something that does not retype its
formula: the reference's own known-answer vector and invariants, hand-derived
vectors from the format definition, numpy/scipy library routines, closed
forms, and constructed inputs whose result the numeric contract fixes by hand.
"""
import json
import os

import numpy as np
import pytest
from scipy.special import expit, softmax

from oracle import oracle
from phantom_moe import q4_0, synth

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


def load_npz(name):
    with np.load(os.path.join(GOLDEN, name), allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


# ---------------------------------------------------------------- Q4_0


def test_q4_0_known_answer_vectors():
    """tests/audit_suite.py:36-41 (0x88, d=1.5 -> zeros) and hand vectors."""
    with open(os.path.join(GOLDEN, "q4_0_kat.json")) as f:
        kat = json.load(f)
    assert any(v["name"].startswith("audit_0x88") for v in kat["vectors"])
    for v in kat["vectors"]:
        blk = np.array([v["d_f16_bits"] & 0xFF, v["d_f16_bits"] >> 8] + v["qs"], dtype=np.uint8)
        out = oracle.q4_0_dequant(blk, (32,))
        np.testing.assert_array_equal(out, np.array(v["expected"], dtype=np.float32), err_msg=v["name"])


def test_q4_0_pack_roundtrip_against_oracle_dequant():
    """pack() is written per element, the oracle per byte; they must agree."""
    rng = np.random.default_rng(0)
    q = rng.integers(-8, 8, size=(6, 96))
    d = (rng.standard_normal((6, 3)) * 0.05).astype(np.float16)
    blocks = q4_0.pack(q, d)
    assert blocks.shape == (6, 3, 18)
    want = (q.reshape(6, 3, 32) * d.astype(np.float32)[..., None]).reshape(6, 96).astype(np.float32)
    np.testing.assert_array_equal(oracle.q4_0_dequant(blocks, (6, 96)), want)
    q2, d2 = q4_0.unpack(blocks)
    np.testing.assert_array_equal(q2, q)
    np.testing.assert_array_equal(d2.view(np.uint16), d.view(np.uint16))


def test_q4_0_rejects_short_payload():
    with pytest.raises(ValueError):
        oracle.q4_0_dequant(np.zeros(17, dtype=np.uint8), (32,))
    with pytest.raises(ValueError):
        oracle.q4_0_dequant(np.zeros(36, dtype=np.uint8), (48,))


# ---------------------------------------------------------------- canonical dot


def _place(H, entries):
    x = np.zeros(H, dtype=np.float32)
    w = np.zeros(H, dtype=np.float32)
    for h, xv, wv in entries:
        x[h], w[h] = xv, wv
    return x, w


def test_canonical_dot_tree_order_by_hand():
    """Inputs where the contract's order is the only one giving the result.

    Partial l holds the h with (h % 256) // 4 == l; the tree pairs l with
    l ^ 32 first, then l ^ 16, ..., l ^ 1."""
    big = 2.0 ** 53
    # p0 = 2^53, p32 (h=128) = 1, p16 (h=64) = 1.  Tree: (p0+p32) + (p16+p48)
    # = 2^53 + 1 -> 2^53 (tie to even), then 2^53 + 1 -> 2^53.  Pairing p16
    # with p32 first would give 2^53 + 2.
    x, w = _place(256, [(0, 2.0 ** 27, 2.0 ** 26), (128, 1.0, 1.0), (64, 1.0, 1.0)])
    assert oracle.canonical_dot(x, w) == big
    # p0 = 2^53, p1 (h=4) = 1, p33 (h=132) = 1: level 32 gives p1+p33 = 2,
    # level 1 gives 2^53 + 2 exactly.  A sequential sum would lose both ones.
    x, w = _place(256, [(0, 2.0 ** 27, 2.0 ** 26), (4, 1.0, 1.0), (132, 1.0, 1.0)])
    assert oracle.canonical_dot(x, w) == big + 2.0
    # Within a partial the order is increasing h: h=0 (2^53), h=1 (1), h=2 (1)
    # -> (2^53 + 1) + 1 = 2^53; a pairwise sum of the two ones would keep 2.
    x, w = _place(256, [(0, 2.0 ** 27, 2.0 ** 26), (1, 1.0, 1.0), (2, 1.0, 1.0)])
    assert oracle.canonical_dot(x, w) == big
    # Chunks: h = 256 lands in partial 0 again, after h = 0..3.
    x, w = _place(512, [(0, 2.0 ** 27, 2.0 ** 26), (256, 1.0, 1.0), (64, 1.0, 1.0)])
    assert oracle.canonical_dot(x, w) == big


def test_canonical_dot_matches_exact_sum_closely():
    rng = np.random.default_rng(1)
    for H in (32, 256, 2048, 7168):
        x = rng.standard_normal(H).astype(np.float32)
        w = (rng.standard_normal(H) * 0.02).astype(np.float32)
        import math

        exact = math.fsum((x.astype(np.float64) * w.astype(np.float64)).tolist())
        got = oracle.canonical_dot(x, w)
        assert abs(got - exact) <= 1e-13 * max(1.0, np.abs(x.astype(np.float64) * w).sum())
    # Integer-valued products: every partial is exact, so the result is exact.
    x = rng.integers(-50, 50, 2048).astype(np.float32)
    w = rng.integers(-50, 50, 2048).astype(np.float32)
    assert oracle.canonical_dot(x, w) == float(np.dot(x.astype(np.int64), w.astype(np.int64)))


# ---------------------------------------------------------------- router


ROUTER_FIXTURES = [
    "router_ref_test_shape.npz",
    "router_ref_test_shape_f32.npz",
    "router_e128_k8_t4.npz",
    "router_zipf_t8.npz",
    "router_sigmoid_t4.npz",
    "router_ties.npz",
]


@pytest.mark.parametrize("name", ROUTER_FIXTURES)
def test_router_golden(name):
    f = load_npz(name)
    idx, w = oracle.route(f["x"], f["W"], int(f["k"]), int(f["score"]), f.get("bias"))
    np.testing.assert_array_equal(idx, f["idx"])
    np.testing.assert_allclose(w, f["w"], rtol=2e-7, atol=1e-8)


def test_router_ties_go_to_lower_index():
    f = load_npz("router_ties.npz")
    idx, _, lg = oracle.route(f["x"], f["W"], int(f["k"]), 0, return_logits=True)
    # the duplicated rows give bit-identical logits
    assert np.array_equal(lg[:, 3], lg[:, 9]) and np.array_equal(lg[:, 0], lg[:, 15])
    hit = 0
    for t in range(idx.shape[0]):
        row = list(idx[t])
        for a, b in [(3, 9), (5, 6), (0, 15)]:
            if a in row and b in row:
                assert row.index(a) < row.index(b)
                hit += 1
            elif b in row:
                raise AssertionError(f"token {t}: {b} selected without its lower-index twin {a}")
    assert hit > 0, "fixture has no tie inside the top-k"


def test_router_invariants_reference_shape():
    """tests/test_moe_routing.py:139-159: H=256, E=8, k=2, x [2, 4, 256]."""
    rng = np.random.default_rng(5)
    x = rng.standard_normal((8, 256)).astype(np.float32)
    W = (rng.standard_normal((8, 256)) * (1 / 16)).astype(np.float32)
    idx, w = oracle.route(x, W, 2, 0)
    assert idx.shape == (8, 2) and w.shape == (8, 2)
    np.testing.assert_allclose(w.sum(axis=1), 1.0, atol=1e-5)
    assert (idx >= 0).all() and (idx < 8).all()


def test_router_against_numpy_and_reference_torch_module():
    """Selection equals np.argsort over numpy logits, and agrees with the
    reference module's own torch fp32 computation on this seeded input."""
    import torch
    import torch.nn.functional as F

    rng = np.random.default_rng(9)
    T, H, E, k = 64, 2048, 128, 8
    xb = synth.f32_to_bf16_bits(rng.standard_normal((T, H), dtype=np.float32))
    xv = synth.bf16_bits_to_f32(xb)
    W = (rng.standard_normal((E, H), dtype=np.float32) * np.float32(0.02)).astype(np.float32)
    idx, w, lg = oracle.route(xb, W, k, 0, return_logits=True)
    ref = xv.astype(np.float64) @ W.astype(np.float64).T
    np.testing.assert_allclose(lg, ref, rtol=0, atol=1e-12)
    order = np.argsort(-lg, axis=1, kind="stable")[:, :k]
    np.testing.assert_array_equal(idx, order)
    np.testing.assert_allclose(w, softmax(np.take_along_axis(lg, idx, 1), axis=1), rtol=2e-7)
    # The reference forward (tests/test_moe_routing.py:65-71) in torch fp32.
    logits = torch.from_numpy(xv) @ torch.from_numpy(W).T
    tl, ti = torch.topk(logits, k, dim=-1)
    tw = F.softmax(tl, dim=-1)
    agree = (ti.numpy() == idx).all(axis=1)
    # Disagreement is only allowed where fp32 rounding can reorder logits.
    for t in np.nonzero(~agree)[0]:
        srt = np.sort(lg[t])[::-1][: k + 1]
        assert np.min(-np.diff(srt)) < 1e-4, f"token {t}: fp32 torch and the oracle differ away from a near tie"
    assert agree.mean() > 0.9
    ok = np.nonzero(agree)[0]
    np.testing.assert_allclose(tw.numpy()[ok], w[ok], rtol=1e-5, atol=1e-6)


@pytest.mark.parametrize("name", list(synth.CONFIGS))
def test_router_matches_reference_module_fixture(name):
    """The oracle's fp64 selection against the reference router module's fp32
    forward (F.linear -> topk -> softmax, tests/test_moe_routing.py:65-71)
    recorded in router_reference_module.npz for every benchmark layer: indices
    and their order are equal on every token the fixture does not mark as
    within fp32 rounding of a tie (it marks none of these seeded layers), and
    the softmax weights agree to fp32 rounding."""
    f = load_npz("router_reference_module.npz")
    cfg = synth.CONFIGS[name]
    ref_idx = f[f"{name}__idx"].astype(np.int64)
    exempt = f[f"{name}__exempt"]
    n = ref_idx.shape[0]
    assert n == min(cfg.T, 1024) and ref_idx.shape[1] == cfg.k
    xb = synth.activations(cfg.T, cfg.H)[:n]
    W = synth.router_weight(cfg.E, cfg.H)
    b = synth.zipf_bias(cfg.E, cfg.zipf) if cfg.zipf else None
    idx, w = oracle.route(xb, W, cfg.k, cfg.score_mode, b)
    ok = ~exempt
    np.testing.assert_array_equal(idx[ok], ref_idx[ok])
    assert (idx == ref_idx).all(axis=1).mean() == 1.0
    if cfg.score == "softmax":
        np.testing.assert_allclose(w[ok], f[f"{name}__w"][ok], rtol=1e-5, atol=1e-6)


def test_router_sigmoid_and_bias_closed_form():
    rng = np.random.default_rng(4)
    T, H, E, k = 5, 256, 32, 6
    x = rng.standard_normal((T, H)).astype(np.float32)
    W = (rng.standard_normal((E, H)) * 0.05).astype(np.float32)
    b = rng.standard_normal(E).astype(np.float32)
    idx, w, lg = oracle.route(x, W, k, 1, router_bias=b, return_logits=True)
    ref = x.astype(np.float64) @ W.astype(np.float64).T + b.astype(np.float64)
    np.testing.assert_allclose(lg, ref, atol=1e-12)
    np.testing.assert_array_equal(idx, np.argsort(-lg, axis=1, kind="stable")[:, :k])
    s = expit(np.take_along_axis(lg, idx, 1))
    np.testing.assert_allclose(w, s / s.sum(1, keepdims=True), rtol=2e-7)


def test_router_brute_force_tiny():
    """E=5, k=3: the selected set maximises the sum of logits over all
    3-subsets, and its order is descending."""
    import itertools

    rng = np.random.default_rng(8)
    x = rng.standard_normal((20, 32)).astype(np.float32)
    W = rng.standard_normal((5, 32)).astype(np.float32)
    idx, _, lg = oracle.route(x, W, 3, 0, return_logits=True)
    for t in range(20):
        best = max(itertools.combinations(range(5), 3), key=lambda c: sum(lg[t, list(c)]))
        assert set(idx[t]) == set(best)
        assert list(lg[t, idx[t]]) == sorted(lg[t, idx[t]], reverse=True)


def test_router_rejects_bad_k():
    with pytest.raises(ValueError):
        oracle.route(np.zeros((1, 32), np.float32), np.zeros((4, 32), np.float32), 5)


# ---------------------------------------------------------------- permute


@pytest.mark.parametrize("name", ["permute_t64_k8_e32.npz", "permute_t5_k2_e8.npz"])
def test_permute_golden(name):
    f = load_npz(name)
    off, ss, sp = oracle.permute(f["idx"], int(f["E"]))
    np.testing.assert_array_equal(off, f["offsets"])
    np.testing.assert_array_equal(ss, f["sorted_slots"])
    np.testing.assert_array_equal(sp, f["slot_pos"])


def test_permute_properties():
    rng = np.random.default_rng(3)
    idx = rng.integers(0, 16, size=(40, 4)).astype(np.int32)
    off, ss, sp = oracle.permute(idx, 16)
    flat = idx.reshape(-1)
    assert off[0] == 0 and off[-1] == flat.size and (np.diff(off) >= 0).all()
    np.testing.assert_array_equal(sp[ss], np.arange(flat.size))
    for e in range(16):
        seg = ss[off[e]:off[e + 1]]
        assert (flat[seg] == e).all() and (np.diff(seg) > 0).all()
    with pytest.raises(ValueError):
        oracle.permute(np.array([[0, 16]], np.int32), 16)


# ---------------------------------------------------------------- expert FFN / layer


def _numpy_expert(x, g, u, d, H, I):
    wg = oracle.q4_0_dequant(g, (I, H)).astype(np.float64)
    wu = oracle.q4_0_dequant(u, (I, H)).astype(np.float64)
    wd = oracle.q4_0_dequant(d, (H, I)).astype(np.float64)
    gx = wg @ x.astype(np.float64)
    ux = wu @ x.astype(np.float64)
    return wd @ (gx / (1.0 + np.exp(-gx)) * ux)


def test_expert_ffn_against_numpy():
    rng = np.random.default_rng(6)
    H, I = 128, 64
    g = q4_0.random_blocks(rng, (I, H))
    u = q4_0.random_blocks(rng, (I, H))
    d = q4_0.random_blocks(rng, (H, I))
    x = rng.standard_normal(H).astype(np.float32)
    np.testing.assert_allclose(oracle.expert_ffn(x, g, u, d, H, I), _numpy_expert(x, g, u, d, H, I), rtol=1e-10, atol=1e-12)


def test_expert_ffn_zero_weights_closed_form():
    H, I = 64, 32
    z = np.full((I, H // 32, 18), 0x88, dtype=np.uint8)
    z[..., 0:2] = np.array([1.0], np.float16).view(np.uint8)
    zd = np.full((H, I // 32, 18), 0x88, dtype=np.uint8)
    x = np.ones(H, np.float32)
    assert not oracle.expert_ffn(x, z, z, zd, H, I).any()


def test_layer_against_numpy_composition():
    cfg = synth.MoEConfig("t", H=128, I=64, E=8, k=3, T=6)
    L = synth.host_layer(cfg)
    xb = synth.activations(cfg.T, cfg.H)
    xv = synth.bf16_bits_to_f32(xb)
    y, idx, w = oracle.moe_forward(xb, L.router_w, L.gate, L.up, L.down, cfg.k)
    lg = xv.astype(np.float64) @ L.router_w.astype(np.float64).T
    np.testing.assert_array_equal(idx, np.argsort(-lg, axis=1, kind="stable")[:, : cfg.k])
    for t in range(cfg.T):
        acc = np.zeros(cfg.H)
        for j in range(cfg.k):
            e = idx[t, j]
            acc += np.float64(w[t, j]) * _numpy_expert(xv[t], L.gate[e], L.up[e], L.down[e], cfg.H, cfg.I)
        np.testing.assert_allclose(y[t], acc, rtol=1e-6, atol=1e-6)


def test_layer_identical_experts_reduce_to_one_expert():
    """With every expert equal, y = FFN(x) since the weights sum to one."""
    cfg = synth.MoEConfig("t", H=64, I=32, E=6, k=4, T=3)
    L = synth.host_layer(cfg)
    g = np.repeat(L.gate[:1], cfg.E, 0)
    u = np.repeat(L.up[:1], cfg.E, 0)
    d = np.repeat(L.down[:1], cfg.E, 0)
    xb = synth.activations(cfg.T, cfg.H)
    y, _, _ = oracle.moe_forward(xb, L.router_w, g, u, d, cfg.k)
    for t in range(cfg.T):
        single = oracle.expert_ffn(synth.bf16_bits_to_f32(xb[t]), g[0], u[0], d[0], cfg.H, cfg.I)
        np.testing.assert_allclose(y[t], single, rtol=1e-6, atol=1e-6)


def test_layer_shared_expert_adds_its_ffn():
    cfg = synth.MoEConfig("t", H=64, I=32, E=8, k=2, T=4, score="sigmoid", shared=True)
    L = synth.host_layer(cfg)
    xb = synth.activations(cfg.T, cfg.H)
    y0, idx0, _ = oracle.moe_forward(xb, L.router_w, L.gate, L.up, L.down, cfg.k, 1)
    y1, idx1, _ = oracle.moe_forward(xb, L.router_w, L.gate, L.up, L.down, cfg.k, 1, shared=L.shared)
    np.testing.assert_array_equal(idx0, idx1)
    for t in range(cfg.T):
        sh = oracle.expert_ffn(synth.bf16_bits_to_f32(xb[t]), *L.shared, cfg.H, cfg.I)
        np.testing.assert_allclose(y1[t].astype(np.float64) - y0[t], sh, rtol=1e-5, atol=1e-5)


def test_layer_token_subset_is_a_restriction():
    cfg = synth.MoEConfig("t", H=64, I=32, E=8, k=2, T=10)
    L = synth.host_layer(cfg)
    xb = synth.activations(cfg.T, cfg.H)
    y, idx, w = oracle.moe_forward(xb, L.router_w, L.gate, L.up, L.down, cfg.k)
    sub = np.array([7, 2, 9])
    ys, idxs, ws = oracle.moe_forward(xb, L.router_w, L.gate, L.up, L.down, cfg.k, tokens=sub)
    np.testing.assert_array_equal(ys, y[sub])
    np.testing.assert_array_equal(idxs, idx[sub])


def test_reference_cpu_path_port_agrees_with_oracle():
    """oracle/ref_cpu_path.py (the timed CPU baseline) computes the same layer
    up to its bf16 weight/matmul rounding."""
    import torch

    from oracle.ref_cpu_path import RefCPUMoE

    cfg = synth.MoEConfig("t", H=256, I=128, E=16, k=4, T=12, zipf=1.1)
    L = synth.host_layer(cfg)
    xb = synth.activations(cfg.T, cfg.H)
    y, idx, _ = oracle.moe_forward(xb, L.router_w, L.gate, L.up, L.down, cfg.k, 0, L.router_bias)
    for pre in (False, True):
        ref = RefCPUMoE(L.router_w, L.gate, L.up, L.down, cfg.H, cfg.I, cfg.k, "softmax", L.router_bias,
                        predequant=pre)
        yc = ref(torch.from_numpy(xb.view(np.int16)).view(torch.bfloat16)).numpy()
        rel = np.linalg.norm(yc - y) / np.linalg.norm(y)
        assert rel < 2e-2, rel
