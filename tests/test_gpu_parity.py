"""Parity of the HIP library against the CPU oracle, through the C ABI.

Routing indices, their order and the permutation must be bit-exact; layer
outputs must satisfy max |y - y_ref| <= 1e-2 and rel-L2 <= 1e-3 against the
fp64 oracle (helpers.check_y).  Full-size shapes are checked on token subsets
(tokens are independent, so a subset is an exact restriction of the layer)
and through size-independent properties.
"""
import os

import numpy as np
import pytest

torch = pytest.importorskip("torch")

import phantom_moe  # noqa: E402
from helpers import (bf16_tensor_bits, check_y, oracle_for_device_layer, repacked_layout,  # noqa: E402
                     to_bf16_tensor)
from oracle import oracle  # noqa: E402
from phantom_moe import _lib, q4_0, synth  # noqa: E402

pytestmark = pytest.mark.gpu
GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


@pytest.fixture(scope="module")
def dev():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return torch.device("cuda:0")


def load_npz(name):
    with np.load(os.path.join(GOLDEN, name), allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


def dev_weights(L, dev):
    sh = None
    if L.shared is not None:
        sh = tuple(torch.from_numpy(a).to(dev) for a in L.shared)
    return phantom_moe.MoEWeights.from_q4_0(
        torch.from_numpy(L.gate).to(dev), torch.from_numpy(L.up).to(dev), torch.from_numpy(L.down).to(dev),
        L.cfg.H, L.cfg.I, L.cfg.E, shared=sh)


# ------------------------------------------------------------------ Q4_0


@pytest.mark.parametrize("rows,K", [(16, 32), (16, 128), (32, 96), (48, 256), (64, 2048), (2048, 768)])
def test_repack_layout_and_roundtrip(dev, rows, K):
    rng = np.random.default_rng(rows * 7 + K)
    q4 = q4_0.random_blocks(rng, (rows, K))
    t = torch.from_numpy(q4.reshape(-1)).to(dev)
    nib, sc = q4_0.repack(t, rows, K)
    want_nib, want_sc = repacked_layout(q4, rows, K)
    np.testing.assert_array_equal(nib.cpu().numpy(), want_nib)
    np.testing.assert_array_equal(sc.cpu().numpy().view(np.uint16), want_sc)
    back = q4_0.unrepack(nib, sc, rows, K)
    np.testing.assert_array_equal(back.cpu().numpy(), q4.reshape(-1))


def test_dequant_matches_oracle_and_kat(dev):
    import json

    with open(os.path.join(GOLDEN, "q4_0_kat.json")) as f:
        kat = json.load(f)["vectors"]
    blocks = np.array([[v["d_f16_bits"] & 0xFF, v["d_f16_bits"] >> 8] + v["qs"] for v in kat], dtype=np.uint8)
    out = q4_0.dequant_f32(torch.from_numpy(blocks.reshape(-1)).to(dev), len(kat), 32).cpu().numpy()
    np.testing.assert_array_equal(out, np.array([v["expected"] for v in kat], dtype=np.float32))
    rng = np.random.default_rng(2)
    q4 = q4_0.random_blocks(rng, (40, 320))
    out = q4_0.dequant_f32(torch.from_numpy(q4.reshape(-1)).to(dev), 40, 320).cpu().numpy()
    np.testing.assert_array_equal(out, oracle.q4_0_dequant(q4, (40, 320)))


# ------------------------------------------------------------------ router


@pytest.mark.parametrize("name", ["router_ref_test_shape.npz", "router_ref_test_shape_f32.npz",
                                  "router_e128_k8_t4.npz", "router_zipf_t8.npz", "router_sigmoid_t4.npz",
                                  "router_ties.npz"])
def test_route_golden(dev, name):
    f = load_npz(name)
    if f["x"].dtype == np.uint16:
        x = to_bf16_tensor(f["x"], dev)
    else:
        x = torch.from_numpy(f["x"]).to(dev)
    b = torch.from_numpy(f["bias"]).to(dev) if "bias" in f else None
    w, idx = phantom_moe.route(x, torch.from_numpy(f["W"]).to(dev), int(f["k"]), int(f["score"]), b)
    np.testing.assert_array_equal(idx.cpu().numpy(), f["idx"])
    np.testing.assert_allclose(w.cpu().numpy(), f["w"], rtol=1e-6, atol=1e-7)


@pytest.mark.parametrize("T,H,E,k,score,xdt", [
    (1, 2048, 128, 8, 0, "bf16"), (3, 96, 8, 2, 0, "bf16"), (5, 4096, 8, 2, 0, "f32"),
    (17, 512, 64, 6, 1, "bf16"), (64, 7168, 256, 8, 1, "bf16"), (65, 2048, 128, 8, 0, "bf16"),
    (300, 1024, 512, 32, 0, "f32"), (40, 256, 1, 1, 0, "bf16"), (33, 320, 3, 3, 1, "f32"),
    # four-token logits waves (33-64 tokens): ragged H, E not a multiple of 8
    (48, 416, 20, 4, 1, "bf16"), (64, 1056, 40, 8, 0, "f32"),
])
def test_route_random_vs_oracle(dev, T, H, E, k, score, xdt):
    rng = np.random.default_rng(T * 131 + H + E)
    xf = rng.standard_normal((T, H), dtype=np.float32)
    xb = synth.f32_to_bf16_bits(xf)
    W = (rng.standard_normal((E, H), dtype=np.float32) * np.float32(0.02)).astype(np.float32)
    x = to_bf16_tensor(xb, dev) if xdt == "bf16" else torch.from_numpy(xf).to(dev)
    w, idx = phantom_moe.route(x, torch.from_numpy(W).to(dev), k, score)
    ridx, rw = oracle.route(xb if xdt == "bf16" else xf, W, k, score)
    np.testing.assert_array_equal(idx.cpu().numpy(), ridx)
    np.testing.assert_allclose(w.cpu().numpy(), rw, rtol=1e-6, atol=1e-7)


@pytest.mark.parametrize("E,k,T", [(7, 7, 9), (32, 32, 9), (64, 4, 9), (128, 8, 9), (200, 32, 9), (256, 16, 9),
                                   (128, 8, 40), (256, 16, 64)])
def test_route_special_values(dev, E, k, T):
    """NaN, +-inf, +-0 and exactly tied logits: NaN ranks below every number,
    -0 ties +0, ties go to the lower expert index (the oracle's ranks_before)."""
    rng = np.random.default_rng(1000 + E)
    H = 64
    xb = synth.f32_to_bf16_bits(rng.standard_normal((T, H), dtype=np.float32))
    W = (rng.standard_normal((E, H), dtype=np.float32) * np.float32(0.02)).astype(np.float32)
    W[1::5] = 0.0  # logit exactly +0 (plus bias)
    n3 = len(W[3::7])
    W[3::7] = W[2::7][:n3]  # duplicated rows: exact ties at distinct indices
    bias = np.zeros(E, np.float32)
    bias[::11] = np.nan
    if E >= 200:
        bias[4::13] = np.inf  # +inf in the top-k: softmax weights are NaN, selection still exact
    bias[6::13] = -np.inf
    bias[8::17] = -0.0
    x = to_bf16_tensor(xb, dev)
    w, idx = phantom_moe.route(x, torch.from_numpy(W).to(dev), k, 0, torch.from_numpy(bias).to(dev))
    ridx, rw = oracle.route(xb, W, k, 0, bias)
    np.testing.assert_array_equal(idx.cpu().numpy(), ridx)
    np.testing.assert_allclose(w.cpu().numpy(), rw, rtol=1e-6, atol=1e-7, equal_nan=True)


@pytest.mark.parametrize("name", list(synth.CONFIGS))
def test_route_full_size_configs(dev, name):
    cfg = synth.CONFIGS[name]
    xb = synth.activations(cfg.T, cfg.H)
    W = synth.router_weight(cfg.E, cfg.H)
    b = synth.zipf_bias(cfg.E, cfg.zipf) if cfg.zipf else None
    w, idx = phantom_moe.route(to_bf16_tensor(xb, dev), torch.from_numpy(W).to(dev), cfg.k, cfg.score,
                               None if b is None else torch.from_numpy(b).to(dev))
    # every token of the batch (the prefill batches run the two-pass router)
    ridx, rw = oracle.route(xb, W, cfg.k, cfg.score_mode, b)
    np.testing.assert_array_equal(idx.cpu().numpy(), ridx)
    np.testing.assert_allclose(w.cpu().numpy(), rw, rtol=1e-6, atol=1e-7)
    np.testing.assert_allclose(w.sum(-1).cpu().numpy(), 1.0, atol=1e-5)


@pytest.mark.parametrize("name", list(synth.CONFIGS))
def test_route_matches_reference_module_fixture(dev, name):
    """The HIP router on a whole benchmark batch against the reference router
    module's fp32 forward (tests/test_moe_routing.py:65-71) recorded in
    router_reference_module.npz for its first tokens (all up to 64, 1024 of a
    prefill batch): equal indices in equal order on every token not marked as
    within fp32 rounding of a tie, softmax weights to fp32 rounding."""
    f = load_npz("router_reference_module.npz")
    cfg = synth.CONFIGS[name]
    ref_idx = f[f"{name}__idx"].astype(np.int64)
    ok = ~f[f"{name}__exempt"]
    n = ref_idx.shape[0]
    xb = synth.activations(cfg.T, cfg.H)
    W = synth.router_weight(cfg.E, cfg.H)
    b = synth.zipf_bias(cfg.E, cfg.zipf) if cfg.zipf else None
    w, idx = phantom_moe.route(to_bf16_tensor(xb, dev), torch.from_numpy(W).to(dev), cfg.k, cfg.score,
                               None if b is None else torch.from_numpy(b).to(dev))
    idx = idx.cpu().numpy()[:n]
    np.testing.assert_array_equal(idx[ok], ref_idx[ok])
    if cfg.score == "softmax":
        np.testing.assert_allclose(w.cpu().numpy()[:n][ok], f[f"{name}__w"][ok], rtol=1e-5, atol=1e-6)


def test_router_module_reference_contract(dev):
    """tests/test_moe_routing.py:139-159 on the drop-in module."""
    torch.manual_seed(0)
    router = phantom_moe.PhantomTopKRouter(256, 8, 2).to(dev)
    with pytest.raises(RuntimeError, match="no backward"):
        router(torch.randn(2, 4, 256, device=dev))
    router.gate.weight.requires_grad_(False)
    for dt in (torch.float32, torch.bfloat16):
        x = torch.randn(2, 4, 256, device=dev).to(dt)
        weights, indices = router(x)
        assert weights.shape == (2, 4, 2) and indices.shape == (2, 4, 2)
        assert weights.dtype == dt and indices.dtype == torch.int64
        assert torch.allclose(weights.float().sum(-1), torch.ones(2, 4, device=dev), atol=1e-2 if dt == torch.bfloat16 else 1e-5)
        assert (indices >= 0).all() and (indices < 8).all()
        W = router.gate.weight.detach().cpu().numpy()
        xin = bf16_tensor_bits(x.reshape(8, 256)) if dt == torch.bfloat16 else x.reshape(8, 256).cpu().numpy()
        ridx, _ = oracle.route(xin, W, 2, 0)
        np.testing.assert_array_equal(indices.reshape(8, 2).cpu().numpy(), ridx)


# ------------------------------------------------------------------ permute


@pytest.mark.parametrize("name", ["permute_t64_k8_e32.npz", "permute_t5_k2_e8.npz"])
def test_permute_golden(dev, name):
    f = load_npz(name)
    off, ss, sp = phantom_moe.permute(torch.from_numpy(f["idx"]).to(dev), int(f["E"]))
    np.testing.assert_array_equal(off.cpu().numpy(), f["offsets"])
    np.testing.assert_array_equal(ss.cpu().numpy(), f["sorted_slots"])
    np.testing.assert_array_equal(sp.cpu().numpy(), f["slot_pos"])


@pytest.mark.parametrize("T,k,E,mode", [(1, 8, 128, "rand"), (32, 8, 128, "rand"), (4096, 8, 128, "rand"),
                                        (2048, 8, 256, "rand"), (100, 4, 16, "one"), (77, 3, 512, "rand"),
                                        (1, 1, 1, "one"), (9000, 2, 8, "rand"),
                                        # E x blocks above the fused scan's table: separate scan launch
                                        (4096, 8, 512, "rand")])
def test_permute_vs_numpy(dev, T, k, E, mode):
    rng = np.random.default_rng(T + k + E)
    if mode == "one":
        idx = np.tile(np.arange(k, dtype=np.int32), (T, 1))
    else:
        idx = np.stack([rng.choice(E, k, replace=False) for _ in range(T)]).astype(np.int32)
    off, ss, sp = phantom_moe.permute(torch.from_numpy(idx).to(dev), E)
    roff, rss, rsp = oracle.permute(idx, E)
    np.testing.assert_array_equal(off.cpu().numpy(), roff)
    np.testing.assert_array_equal(ss.cpu().numpy(), rss)
    np.testing.assert_array_equal(sp.cpu().numpy(), rsp)
    np.testing.assert_array_equal(rss, np.argsort(idx.reshape(-1), kind="stable"))


def test_empty_batch(dev):
    """No tokens: empty outputs of the right shapes (leading dims kept), as
    torch's own operators give, and an all-zero offset table."""
    cfg = synth.MoEConfig("empty", 256, 128, 16, 4, 1)
    L = synth.host_layer(cfg)
    ex = dev_weights(L, dev)
    W = torch.from_numpy(L.router_w).to(dev)
    x = torch.empty((2, 0, cfg.H), dtype=torch.bfloat16, device=dev)
    y, w, idx = phantom_moe.moe_forward(x, W, ex, cfg.k, return_routing=True)
    assert y.shape == (2, 0, cfg.H) and y.dtype == torch.float32
    assert w.shape == (2, 0, cfg.k) and idx.shape == (2, 0, cfg.k)
    rw, ridx = phantom_moe.route(x, W, cfg.k)
    assert rw.shape == (2, 0, cfg.k) and ridx.shape == (2, 0, cfg.k)
    off, ss, sp = phantom_moe.permute(torch.empty((0, cfg.k), dtype=torch.int32, device=dev), cfg.E)
    assert off.shape == (cfg.E + 1,) and not off.any() and ss.numel() == 0 and sp.numel() == 0


# ------------------------------------------------------------------ layer


SMALL_CASES = [
    synth.MoEConfig("tiny", 256, 128, 16, 4, 8),
    synth.MoEConfig("one_token", 512, 256, 32, 8, 1),
    synth.MoEConfig("pad_k", 96, 96, 8, 2, 5),
    synth.MoEConfig("many_per_expert", 256, 64, 4, 2, 70),
    synth.MoEConfig("sigmoid_shared", 512, 128, 32, 4, 12, score="sigmoid", shared=True),
    synth.MoEConfig("zipf", 1024, 256, 128, 8, 32, zipf=1.1),
    synth.MoEConfig("k1", 128, 32, 4, 1, 3),
    # 8800 slots: the many-workgroup permute, feeding the token-tile table and
    # the shared expert (decode regime: 17 positions per expert on average)
    synth.MoEConfig("many_slots_tiles", 256, 256, 512, 8, 1100, shared=True),
    # 16800 slots over 512 experts: 17 count blocks x 512 experts exceed the
    # fused scan's table, so the scan runs as its own launch
    synth.MoEConfig("many_slots_unfused", 256, 256, 512, 8, 2100, shared=True),
    # GEMM regime (T*k >= 64 * min(E, T*k)): fp16 operands, 128-position tiles
    synth.MoEConfig("gemm_e4", 256, 128, 4, 2, 200),
    synth.MoEConfig("gemm_multi_block", 256, 256, 2, 2, 300),
    synth.MoEConfig("gemm_ragged_k_and_rows", 416, 96, 3, 1, 257),
    synth.MoEConfig("gemm_sigmoid_shared", 512, 256, 8, 2, 300, score="sigmoid", shared=True),
    # about 130 positions per expert: a full 128-position block plus a short
    # tail block (its 16-position tiles past the segment skipped)
    synth.MoEConfig("gemm_tail", 256, 128, 2, 1, 262),
]


@pytest.mark.parametrize("cfg", SMALL_CASES, ids=lambda c: c.name)
def test_moe_forward_small_vs_oracle(dev, cfg):
    L = synth.host_layer(cfg)
    xb = synth.activations(cfg.T, cfg.H, seed=hash(cfg.name) % 1000)
    ex = dev_weights(L, dev)
    b = None if L.router_bias is None else torch.from_numpy(L.router_bias).to(dev)
    y, w, idx = phantom_moe.moe_forward(to_bf16_tensor(xb, dev), torch.from_numpy(L.router_w).to(dev), ex, cfg.k,
                                        cfg.score, b, return_routing=True)
    ry, ridx, rw = oracle.moe_forward(xb, L.router_w, L.gate, L.up, L.down, cfg.k, cfg.score_mode,
                                      L.router_bias, shared=L.shared)
    np.testing.assert_array_equal(idx.cpu().numpy(), ridx)
    np.testing.assert_allclose(w.cpu().numpy(), rw, rtol=1e-6, atol=1e-7)
    check_y(y.cpu().numpy(), ry, cfg.name)


FULL = ["qwen3_decode_t1", "qwen3_decode_t32_zipf", "mixtral_decode_t1", "mixtral_decode_t16",
        "qwen3_prefill_t4096", "dsv3_decode_t1", "dsv3_decode_t8", "dsv3_decode_t64", "dsv3_prefill_t2048"]


def covering_tokens(idx: np.ndarray, E: int, block: int = 64) -> np.ndarray:
    """Tokens whose outputs together touch every work item of the expert
    GEMMs: every (expert, block-position block) of the stable per-expert
    segments (the gate/up items are 128-position blocks or their 64-position
    halves, the down items 64-position blocks, each over all rows), chosen
    greedily (each token covers its k slots' blocks).  Segment position of
    slot s = t*k + j: its rank among the slots of expert idx[t, j] in slot
    order."""
    T, k = idx.shape
    flat = idx.reshape(-1).astype(np.int64)
    order = np.argsort(flat, kind="stable")
    counts = np.bincount(flat, minlength=E)
    starts = np.concatenate([[0], np.cumsum(counts)[:-1]])
    pos = np.empty_like(order)
    pos[order] = np.arange(flat.size) - starts[flat[order]]
    nblk = -(-counts // block)
    base = np.concatenate([[0], np.cumsum(nblk)[:-1]])
    item = (base[flat] + pos // block).reshape(T, k)
    covered = np.zeros(int(nblk.sum()), dtype=bool)
    chosen = []
    while not covered.all():
        gain = (~covered[item]).sum(axis=1)
        t = int(np.argmax(gain))
        chosen.append(t)
        covered[item[t]] = True
    return np.sort(np.asarray(chosen, dtype=np.int64))


@pytest.mark.parametrize("name", FULL)
def test_moe_forward_full_size_vs_oracle(dev, name):
    """Full-size layers: routing of every token equal to the oracle's; outputs
    of every token for decode batches, and for prefill batches of a token set
    that covers every GEMM work item (covering_tokens)."""
    cfg = synth.CONFIGS[name]
    print(f"[case] {name}", flush=True)
    dl = synth.device_layer(cfg, dev)
    ex = phantom_moe.MoEWeights.from_q4_0(dl.gate, dl.up, dl.down, cfg.H, cfg.I, cfg.E, shared=dl.shared)
    xb = synth.activations(cfg.T, cfg.H)
    y, w, idx = phantom_moe.moe_forward(to_bf16_tensor(xb, dev), dl.router_w, ex, cfg.k, cfg.score,
                                        dl.router_bias, return_routing=True)
    torch.cuda.synchronize()
    if cfg.T <= 64:
        sub = np.arange(cfg.T)
    else:
        b = None if dl.router_bias is None else dl.router_bias.cpu().numpy()
        all_idx, all_w = oracle.route(xb, dl.router_w.cpu().numpy(), cfg.k, cfg.score_mode, b)
        np.testing.assert_array_equal(idx.cpu().numpy(), all_idx)
        np.testing.assert_allclose(w.cpu().numpy(), all_w, rtol=1e-6, atol=1e-7)
        sub = covering_tokens(all_idx, cfg.E)
        print(f"[case] {name}: routing of all {cfg.T} tokens equal; outputs of {sub.size} covering tokens",
              flush=True)
    ry, ridx, rw = oracle_for_device_layer(dl, xb, sub)
    np.testing.assert_array_equal(idx.cpu().numpy()[sub], ridx)
    np.testing.assert_allclose(w.cpu().numpy()[sub], rw, rtol=1e-6, atol=1e-7)
    err, rel = check_y(y.cpu().numpy()[sub], ry, name)
    print(f"[case] {name}: max_abs={err:.2e} rel_l2={rel:.2e}", flush=True)


def test_layer_properties(dev):
    """Determinism, token-permutation equivariance, and exact linearity in the
    down-projection scales (doubling every fp16 scale doubles y bit for bit)."""
    cfg = synth.MoEConfig("props", 1024, 256, 64, 8, 40)
    L = synth.host_layer(cfg)
    xb = synth.activations(cfg.T, cfg.H, seed=5)
    ex = dev_weights(L, dev)
    W = torch.from_numpy(L.router_w).to(dev)
    x = to_bf16_tensor(xb, dev)
    y1, w1, i1 = phantom_moe.moe_forward(x, W, ex, cfg.k, return_routing=True)
    y2, w2, i2 = phantom_moe.moe_forward(x, W, ex, cfg.k, return_routing=True)
    assert torch.equal(y1, y2) and torch.equal(i1, i2) and torch.equal(w1, w2)
    perm = np.random.default_rng(0).permutation(cfg.T)
    yp, wp, ip = phantom_moe.moe_forward(to_bf16_tensor(xb[perm], dev), W, ex, cfg.k, return_routing=True)
    assert torch.equal(ip, i1[torch.from_numpy(perm).to(dev)])
    assert torch.equal(yp, y1[torch.from_numpy(perm).to(dev)])
    down2 = L.down.copy()
    d = np.ascontiguousarray(down2[..., 0:2]).view(np.float16)
    down2[..., 0:2] = (d * np.float16(2)).view(np.uint8)
    ex2 = phantom_moe.MoEWeights.from_q4_0(torch.from_numpy(L.gate).to(dev), torch.from_numpy(L.up).to(dev),
                                           torch.from_numpy(down2).to(dev), cfg.H, cfg.I, cfg.E)
    y3 = phantom_moe.moe_forward(x, W, ex2, cfg.k)
    assert torch.equal(y3, 2 * y1)


def test_profiled_forward_is_identical(dev):
    """Stage timing changes no output bit and brackets every stage."""
    import ctypes

    from phantom_moe import _lib

    cfg = synth.CONFIGS["qwen3_decode_t32_zipf"]
    dl = synth.device_layer(cfg, dev)
    ex = phantom_moe.MoEWeights.from_q4_0(dl.gate, dl.up, dl.down, cfg.H, cfg.I, cfg.E)
    x = to_bf16_tensor(synth.activations(cfg.T, cfg.H), dev)
    y0 = phantom_moe.moe_forward(x, dl.router_w, ex, cfg.k, cfg.score, dl.router_bias)
    hip = ctypes.CDLL("libamdhip64.so.7")
    hip.hipEventCreateWithFlags.argtypes = [ctypes.POINTER(ctypes.c_void_p), ctypes.c_uint]
    hip.hipEventElapsedTime.argtypes = [ctypes.POINTER(ctypes.c_float), ctypes.c_void_p, ctypes.c_void_p]
    hip.hipEventDestroy.argtypes = [ctypes.c_void_p]
    n = 5
    evs = []
    for _ in range(n):
        e = ctypes.c_void_p()
        assert hip.hipEventCreateWithFlags(ctypes.byref(e), 0) == 0
        evs.append(e.value)
    arr = (ctypes.c_void_p * n)(*evs)
    lib = _lib.load()
    try:
        assert lib.phantom_moe_set_profile_events(arr, n) == 0
        y1 = phantom_moe.moe_forward(x, dl.router_w, ex, cfg.k, cfg.score, dl.router_bias)
    finally:
        assert lib.phantom_moe_set_profile_events(None, 0) == 0
    torch.cuda.synchronize()
    assert torch.equal(y0, y1)
    ms = ctypes.c_float()
    for i in range(n - 1):
        assert hip.hipEventElapsedTime(ctypes.byref(ms), evs[i], evs[i + 1]) == 0 and ms.value > 0, i
    for e in evs:
        hip.hipEventDestroy(ctypes.c_void_p(e))


TILE_CASES = [
    synth.MoEConfig("tile_sigmoid_shared", 512, 512, 64, 8, 40, score="sigmoid", shared=True),
    synth.MoEConfig("tile_ragged_h", 416, 512, 64, 8, 60),
    synth.MoEConfig("tile_ragged_i", 512, 480, 64, 8, 40),
    synth.MoEConfig("tile_zipf", 1024, 768, 128, 8, 32, zipf=1.1),
]


@pytest.mark.parametrize("cfg", TILE_CASES, ids=lambda c: c.name)
def test_expert_kernels_agree(dev, cfg):
    """Each decode expert stage has two kernels: the token-tile kernel (the
    operand of a 16-position tile copied into LDS once, one wave per row tile)
    where the row tiles of all token tiles give at least four waves per CU
    (eight for down), else the K-split kernel.  These shapes are in the
    token-tile regime of both stages; the K-split pair is forced with the
    option PHANTOM_MOE_OPT_DECODE_KSPLIT.  Both pairs must meet the layer
    tolerance against the oracle, shared expert and ragged last quads of H and
    of I included, with identical routing."""
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    n_slots = cfg.T * cfg.k
    max_tiles = -(-n_slots // 16) + min(n_slots, cfg.E) + (-(-cfg.T // 16) if cfg.shared else 0)
    assert max_tiles * (cfg.I // 16) >= 4 * cus, "shape not in the gate/up token-tile regime"
    assert max_tiles * (cfg.H // 16) >= 8 * cus, "shape not in the down token-tile regime"
    L = synth.host_layer(cfg)
    xb = synth.activations(cfg.T, cfg.H, seed=7)
    ex = dev_weights(L, dev)
    b = None if L.router_bias is None else torch.from_numpy(L.router_bias).to(dev)
    W = torch.from_numpy(L.router_w).to(dev)
    x = to_bf16_tensor(xb, dev)
    ry, ridx, _ = oracle.moe_forward(xb, L.router_w, L.gate, L.up, L.down, cfg.k, cfg.score_mode,
                                     L.router_bias, shared=L.shared)
    lib = phantom_moe._lib.load()
    names = lib.phantom_moe_expert_kernels(cfg.T, cfg.H, cfg.I, cfg.E, cfg.k, int(cfg.shared)).decode()
    assert names == "gate_up=gate_up_tile_kernel;down=down_tile_kernel"
    y_tile, _, idx_tile = phantom_moe.moe_forward(x, W, ex, cfg.k, cfg.score, b, return_routing=True)
    old = _lib.set_option(_lib.OPT_DECODE_KSPLIT, 1)
    try:
        names = lib.phantom_moe_expert_kernels(cfg.T, cfg.H, cfg.I, cfg.E, cfg.k, int(cfg.shared)).decode()
        assert names == "gate_up=gate_up_kernel;down=down_kernel"
        y_cls, _, idx_cls = phantom_moe.moe_forward(x, W, ex, cfg.k, cfg.score, b, return_routing=True)
    finally:
        _lib.set_option(_lib.OPT_DECODE_KSPLIT, old)
    np.testing.assert_array_equal(idx_tile.cpu().numpy(), ridx)
    np.testing.assert_array_equal(idx_cls.cpu().numpy(), ridx)
    check_y(y_tile.cpu().numpy(), ry, cfg.name + " token-tile")
    check_y(y_cls.cpu().numpy(), ry, cfg.name + " K-split")


