"""The one-token streaming single launch (csrc/decode_stream.hip) against the
oracle and against the staged launches, through the C ABI.

It takes one-token layers whose experts are too large for the staging
single launch (Mixtral-8x7B- and DeepSeek-V3-shaped); the option
PHANTOM_MOE_OPT_DECODE_STREAM = 2 forces it onto any one-token shape, which
the small cases here use.  Routing indices and order must be bit-exact,
outputs within the layer tolerance of the fp64 oracle, repeated calls
identical bit for bit.
"""
import numpy as np
import pytest

torch = pytest.importorskip("torch")

import phantom_moe  # noqa: E402
from helpers import check_y, oracle_for_device_layer, to_bf16_tensor  # noqa: E402
from oracle import oracle  # noqa: E402
from phantom_moe import _lib, synth  # noqa: E402

pytestmark = pytest.mark.gpu

STREAM = "gate_up=moe_decode_stream_kernel;down=moe_decode_stream_kernel"


@pytest.fixture(scope="module")
def dev():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return torch.device("cuda:0")


@pytest.fixture
def option():
    saved = []

    def set_(opt, value):
        saved.append((opt, _lib.set_option(opt, value)))

    yield set_
    for opt, value in reversed(saved):
        _lib.set_option(opt, value)


def kernels(cfg):
    return _lib.load().phantom_moe_expert_kernels(cfg.T, cfg.H, cfg.I, cfg.E, cfg.k, int(cfg.shared)).decode()


def dev_weights(L, dev):
    sh = None
    if L.shared is not None:
        sh = tuple(torch.from_numpy(a).to(dev) for a in L.shared)
    return phantom_moe.MoEWeights.from_q4_0(
        torch.from_numpy(L.gate).to(dev), torch.from_numpy(L.up).to(dev), torch.from_numpy(L.down).to(dev),
        L.cfg.H, L.cfg.I, L.cfg.E, shared=sh)


def run(prep, stream=None):
    prep(stream)
    return prep.y.clone(), prep.topk_w.clone(), prep.topk_idx.clone()


CASES = [
    synth.MoEConfig("s_basic", 512, 256, 32, 8, 1),
    synth.MoEConfig("s_sigmoid_shared", 512, 384, 32, 4, 1, score="sigmoid", shared=True),
    synth.MoEConfig("s_ragged_h", 416, 256, 16, 4, 1),
    synth.MoEConfig("s_ragged_i", 256, 160, 16, 2, 1),
    synth.MoEConfig("s_k1", 256, 128, 8, 1, 1),
    synth.MoEConfig("s_e512_k32", 256, 64, 512, 32, 1),
    synth.MoEConfig("s_wide_i", 256, 4096, 8, 2, 1),
    # I of 65 (66) quads: a slot's down work is cut into 8 slices of I, whose
    # parts the combine sums; the second also ends I in a ragged quad
    synth.MoEConfig("s_kx8", 256, 8320, 4, 2, 1),
    synth.MoEConfig("s_kx8_ragged_shared", 288, 8352, 4, 2, 1, score="sigmoid", shared=True),
]


@pytest.mark.parametrize("cfg", CASES, ids=lambda c: c.name)
def test_stream_vs_oracle_and_staged(dev, cfg, option):
    option(_lib.OPT_DECODE_STREAM, 2)
    assert kernels(cfg) == STREAM, kernels(cfg)
    L = synth.host_layer(cfg)
    xb = synth.activations(cfg.T, cfg.H, seed=len(cfg.name) * 17)
    ex = dev_weights(L, dev)
    b = None if L.router_bias is None else torch.from_numpy(L.router_bias).to(dev)
    W = torch.from_numpy(L.router_w).to(dev)
    prep = phantom_moe.PreparedForward(ex, W, cfg.T, cfg.k, cfg.score, b, x=to_bf16_tensor(xb, dev))
    ry, ridx, rw = oracle.moe_forward(xb, L.router_w, L.gate, L.up, L.down, cfg.k, cfg.score_mode,
                                      L.router_bias, shared=L.shared)
    outs = [run(prep) for _ in range(3)]
    torch.cuda.synchronize()
    assert _lib.workspace_status(prep.workspace) == 0
    y, w, idx = outs[0]
    np.testing.assert_array_equal(idx.cpu().numpy(), ridx)
    np.testing.assert_allclose(w.cpu().numpy(), rw, rtol=1e-6, atol=1e-7)
    check_y(y.cpu().numpy(), ry, cfg.name + " stream")
    for i, (yi, wi, ii) in enumerate(outs[1:], 2):
        assert torch.equal(yi, y) and torch.equal(wi, w) and torch.equal(ii, idx), f"call {i} differs"
    # the staged launches route identically
    option(_lib.OPT_DECODE_FUSED, 0)
    assert kernels(cfg) != STREAM
    ys, ws_, iss = run(prep)
    assert torch.equal(iss, idx) and torch.equal(ws_, w)
    check_y(ys.cpu().numpy(), ry, cfg.name + " staged")


@pytest.mark.parametrize("name", ["mixtral_decode_t1", "dsv3_decode_t1"])
def test_stream_full_size(dev, name):
    """The one-token Mixtral-8x7B- and DeepSeek-V3-shaped layers take the
    streaming single launch by default and match the oracle."""
    cfg = synth.CONFIGS[name]
    assert kernels(cfg) == STREAM, kernels(cfg)
    dl = synth.device_layer(cfg, dev)
    ex = phantom_moe.MoEWeights.from_q4_0(dl.gate, dl.up, dl.down, cfg.H, cfg.I, cfg.E, shared=dl.shared)
    for seed in (42, 43):
        xb = synth.activations(cfg.T, cfg.H, seed=seed)
        prep = phantom_moe.PreparedForward(ex, dl.router_w, cfg.T, cfg.k, cfg.score, dl.router_bias,
                                           x=to_bf16_tensor(xb, dev))
        y, w, idx = run(prep)
        y2, w2, idx2 = run(prep)
        torch.cuda.synchronize()
        assert _lib.workspace_status(prep.workspace) == 0
        assert torch.equal(y2, y) and torch.equal(w2, w) and torch.equal(idx2, idx)
        ry, ridx, rw = oracle_for_device_layer(dl, xb)
        np.testing.assert_array_equal(idx.cpu().numpy(), ridx)
        np.testing.assert_allclose(w.cpu().numpy(), rw, rtol=1e-6, atol=1e-7)
        err, rel = check_y(y.cpu().numpy(), ry, f"{name} seed {seed}")
        print(f"[case] {name} stream seed {seed}: max_abs={err:.2e} rel_l2={rel:.2e}", flush=True)


def small_prep(dev, option, seed=9, shared=True):
    option(_lib.OPT_DECODE_STREAM, 2)
    cfg = synth.MoEConfig("s_fail", 256, 192, 16, 4, 1, score="sigmoid" if shared else "softmax", shared=shared)
    assert kernels(cfg) == STREAM
    L = synth.host_layer(cfg)
    ex = dev_weights(L, dev)
    b = None if L.router_bias is None else torch.from_numpy(L.router_bias).to(dev)
    W = torch.from_numpy(L.router_w).to(dev)
    x = to_bf16_tensor(synth.activations(1, cfg.H, seed=seed), dev)
    return cfg, phantom_moe.PreparedForward(ex, W, 1, cfg.k, cfg.score, b, x=x)


def test_stream_graph_replays(dev, option):
    """Captured calls draw fresh tags on every replay: each replay, with
    eager calls between replays, equals the eager result bit for bit."""
    cfg, prep = small_prep(dev, option)
    xs = [to_bf16_tensor(synth.activations(1, cfg.H, seed=s), dev) for s in (1, 2, 3)]
    eager = []
    for x in xs:
        prep.x.copy_(x)
        eager.append(run(prep)[0])
    s = torch.cuda.Stream()
    g = torch.cuda.CUDAGraph()
    outs = [torch.empty_like(eager[0]) for _ in xs]
    torch.cuda.synchronize()
    with torch.cuda.graph(g, stream=s):
        for x, o in zip(xs, outs):
            prep.x.copy_(x)
            prep(_lib.stream_handle(dev))
            o.copy_(prep.y)
    for rep in range(4):
        g.replay()
        torch.cuda.synchronize()
        for i, (o, e) in enumerate(zip(outs, eager)):
            assert torch.equal(o, e), f"replay {rep}, call {i} differs"
        prep.x.copy_(xs[rep % 3])
        assert torch.equal(run(prep)[0], eager[rep % 3])
        torch.cuda.synchronize()
    assert _lib.workspace_status(prep.workspace) == 0


@pytest.mark.parametrize("fault", [1, 2])
def test_stream_wait_failure_is_reported(dev, option, fault):
    """A wait that gives up (forced from the host with a short bound: the
    waiters expect a tag nobody writes) ends normally, raises
    FusedWaitError, sets the workspace status and leaves NaN in y (and in
    the routing outputs when the logit wait gave up); the next call is
    correct again."""
    cfg, prep = small_prep(dev, option, seed=21)
    y_ok, w_ok, i_ok = run(prep)
    option(_lib.OPT_FUSED_WAIT_POLLS, 64)
    option(_lib.OPT_FUSED_FAULT, fault)
    with pytest.raises(phantom_moe.FusedWaitError):
        prep()
        torch.cuda.synchronize()
        phantom_moe.check_status()
    torch.cuda.synchronize()
    try:
        phantom_moe.check_status()
    except phantom_moe.FusedWaitError:
        pass
    y, w, idx = prep.y.clone(), prep.topk_w.clone(), prep.topk_idx.clone()
    st = _lib.workspace_status(prep.workspace)
    assert st & fault, f"status {st:#x} lacks bit {fault:#x}"
    assert torch.isnan(y).all()
    if fault == 1:
        assert (idx == -1).all() and torch.isnan(w).all()
    else:
        assert torch.equal(idx, i_ok) and torch.equal(w, w_ok)
    _lib.set_option(_lib.OPT_FUSED_FAULT, 0)
    y2, _, _ = run(prep)
    torch.cuda.synchronize()
    assert _lib.workspace_status(prep.workspace) == 0
    assert torch.equal(y2, y_ok)


def test_stream_late_start_takes_its_launch_tag(dev, option):
    """A workgroup that reads the generation counter one ahead (as one that
    starts after workgroup 0 gave up waiting for it would) still takes its
    launch's tag: outputs unchanged, no status, two calls in a row."""
    cfg, prep = small_prep(dev, option, seed=31)
    y_ok, w_ok, i_ok = run(prep)
    option(_lib.OPT_FUSED_WAIT_POLLS, 4096)
    option(_lib.OPT_FUSED_FAULT, 4)
    for call in range(2):
        y, w, idx = run(prep)
        torch.cuda.synchronize()
        phantom_moe.check_status()
        assert _lib.workspace_status(prep.workspace) == 0, f"call {call}"
        assert torch.equal(y, y_ok) and torch.equal(w, w_ok) and torch.equal(idx, i_ok), f"call {call}"
