"""The single-launch decode layer (csrc/decode_fused.hip) against the oracle
and against the staged launches, through the C ABI.

Routing indices and their order must be bit-exact; outputs within the layer
tolerance of the fp64 oracle (helpers.check_y).  The outputs must also be
identical bit for bit across repeated calls (each call's hand-off tags come
from the workspace call counter; a stale tag accepted would change the
output).
"""
import numpy as np
import pytest

torch = pytest.importorskip("torch")

import phantom_moe  # noqa: E402
from helpers import check_y, oracle_for_device_layer, to_bf16_tensor  # noqa: E402
from oracle import oracle  # noqa: E402
from phantom_moe import _lib, synth  # noqa: E402

pytestmark = pytest.mark.gpu

FUSED = "gate_up=moe_decode_fused_kernel;down=moe_decode_fused_kernel"
X8 = "gate_up=moe_decode_x8_kernel;down=moe_decode_x8_kernel"


@pytest.fixture(scope="module")
def dev():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return torch.device("cuda:0")


@pytest.fixture
def option():
    """Set library options for one test and restore them afterwards."""
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


def faulty_call(prep):
    """One call whose wait is forced to give up: the pinned status word makes
    it raise FusedWaitError, from the call itself or from the check after
    the stream has finished; the outputs are read afterwards."""
    with pytest.raises(phantom_moe.FusedWaitError):
        prep()
        torch.cuda.synchronize()
        phantom_moe.check_status()
    torch.cuda.synchronize()
    try:  # workgroups that gave up after the check above stored the bit again
        phantom_moe.check_status()
    except phantom_moe.FusedWaitError:
        pass
    return prep.y.clone(), prep.topk_w.clone(), prep.topk_idx.clone()


CASES = [
    synth.MoEConfig("f_t1", 512, 256, 32, 8, 1),
    synth.MoEConfig("f_t1_e16_k4", 256, 128, 16, 4, 1),
    synth.MoEConfig("f_t2", 256, 128, 16, 4, 2),
    synth.MoEConfig("f_t4_sigmoid_shared", 512, 128, 32, 4, 4, score="sigmoid", shared=True),
    synth.MoEConfig("f_t8", 256, 128, 16, 4, 8),
    synth.MoEConfig("f_ragged", 96, 96, 8, 2, 3),
    synth.MoEConfig("f_ragged_i", 384, 160, 24, 3, 2),
    synth.MoEConfig("f_k1", 128, 32, 4, 1, 3),
    synth.MoEConfig("f_zipf", 1024, 256, 128, 8, 1, zipf=1.1),
    synth.MoEConfig("f_e512", 256, 64, 512, 32, 1),
    synth.MoEConfig("f_e1", 128, 64, 1, 1, 2),
    synth.MoEConfig("f_e64_k64", 128, 64, 64, 32, 2),
]


@pytest.mark.parametrize("cfg", CASES, ids=lambda c: c.name)
def test_fused_vs_oracle_and_staged(dev, cfg, option):
    assert kernels(cfg) == FUSED, f"{cfg.name} is not in the single-launch regime"
    L = synth.host_layer(cfg)
    xb = synth.activations(cfg.T, cfg.H, seed=len(cfg.name) * 13)
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
    check_y(y.cpu().numpy(), ry, cfg.name + " fused")
    for i, (yi, wi, ii) in enumerate(outs[1:], 2):
        assert torch.equal(yi, y) and torch.equal(wi, w) and torch.equal(ii, idx), f"call {i} differs"
    # the staged launches give the same routing and meet the same tolerance
    option(_lib.OPT_DECODE_FUSED, 0)
    assert kernels(cfg) != FUSED
    ys, ws_, iss = run(prep)
    np.testing.assert_array_equal(iss.cpu().numpy(), ridx)
    assert torch.equal(ws_, w)
    check_y(ys.cpu().numpy(), ry, cfg.name + " staged")


@pytest.mark.parametrize("x8", [1, 0], ids=["per_xcd", "generic"])
def test_fused_full_size_qwen3_t1(dev, option, x8):
    """The batch-1 Qwen3-30B-A3B-shaped layer (H 2048, I 768, E 128, top-8)
    takes the single-launch path and matches the oracle: per XCD (expert
    slot j on XCD j) on an 8-XCD, 256-CU part, else in the generic kernel.
    Repeated calls are identical bit for bit."""
    cfg = synth.CONFIGS["qwen3_decode_t1"]
    option(_lib.OPT_DECODE_X8, x8)
    name = kernels(cfg)
    if x8 and name != X8:
        pytest.skip(f"the per-XCD kernel needs 8 XCDs of 32 CUs ({name})")
    assert name == (X8 if x8 else FUSED)
    dl = synth.device_layer(cfg, dev)
    ex = phantom_moe.MoEWeights.from_q4_0(dl.gate, dl.up, dl.down, cfg.H, cfg.I, cfg.E)
    for seed in (42, 43, 44):
        xb = synth.activations(cfg.T, cfg.H, seed=seed)
        prep = phantom_moe.PreparedForward(ex, dl.router_w, cfg.T, cfg.k, cfg.score, dl.router_bias,
                                           x=to_bf16_tensor(xb, dev))
        y, w, idx = run(prep)
        y2, w2, idx2 = run(prep)
        assert _lib.workspace_status(prep.workspace) == 0
        assert torch.equal(y2, y) and torch.equal(w2, w) and torch.equal(idx2, idx)
        ry, ridx, rw = oracle_for_device_layer(dl, xb)
        np.testing.assert_array_equal(idx.cpu().numpy(), ridx)
        np.testing.assert_allclose(w.cpu().numpy(), rw, rtol=1e-6, atol=1e-7)
        err, rel = check_y(y.cpu().numpy(), ry, f"qwen3_decode_t1 seed {seed}")
        print(f"[case] qwen3_decode_t1 {'per-XCD' if x8 else 'generic'} seed {seed}: "
              f"max_abs={err:.2e} rel_l2={rel:.2e}", flush=True)


def x8_prep(dev, seed=7, xb=None):
    """A batch-1 Qwen3-shaped layer on the per-XCD kernel (skips the test
    where the device does not take it)."""
    cfg = synth.CONFIGS["qwen3_decode_t1"]
    if kernels(cfg) != X8:
        pytest.skip(f"the per-XCD kernel needs 8 XCDs of 32 CUs ({kernels(cfg)})")
    dl = synth.device_layer(cfg, dev, layer=1)
    ex = phantom_moe.MoEWeights.from_q4_0(dl.gate, dl.up, dl.down, cfg.H, cfg.I, cfg.E)
    if xb is None:
        xb = synth.activations(cfg.T, cfg.H, seed=seed)
    prep = phantom_moe.PreparedForward(ex, dl.router_w, cfg.T, cfg.k, cfg.score, dl.router_bias,
                                       x=to_bf16_tensor(xb, dev))
    return cfg, dl, prep, xb


def test_x8_graph_replays(dev):
    """Captured per-XCD calls draw fresh tags on every replay: each replay,
    with eager calls between replays, equals the eager result bit for bit."""
    cfg, dl, prep, _ = x8_prep(dev)
    xs = [to_bf16_tensor(synth.activations(1, cfg.H, seed=s), dev) for s in (11, 12, 13)]
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
def test_x8_wait_failure_is_reported(dev, option, fault):
    """A per-XCD wait that gives up (forced from the host with a short bound:
    the waiters expect a tag nobody writes) ends normally, sets the status
    and leaves NaN in y (and in the routing outputs when the logit wait gave
    up); the next call is correct again."""
    cfg, dl, prep, xb = x8_prep(dev, seed=21)
    y_ok, w_ok, i_ok = run(prep)
    option(_lib.OPT_FUSED_WAIT_POLLS, 64)
    option(_lib.OPT_FUSED_FAULT, fault)
    y, w, idx = faulty_call(prep)
    st = _lib.workspace_status(prep.workspace)
    assert st & fault, f"status {st:#x} lacks bit {fault:#x}"
    assert torch.isnan(y).all()
    if fault == 1:
        assert (idx == -1).all() and torch.isnan(w).all()
    else:
        assert torch.equal(idx, i_ok) and torch.equal(w, w_ok)
    _lib.set_option(_lib.OPT_FUSED_FAULT, 0)
    y2, _, _ = run(prep)
    assert _lib.workspace_status(prep.workspace) == 0
    assert torch.equal(y2, y_ok)


@pytest.mark.parametrize("special", ["nan", "inf", "zero"])
def test_x8_nonfinite_and_zero_activations(dev, special):
    """NaN, +-inf or an all-zero x: no fault, routing as the oracle's
    contract gives it (NaN logits rank below every number; all-zero logits
    tie, so experts 0..7 in index order), identical to the generic kernel."""
    cfg = synth.CONFIGS["qwen3_decode_t1"]
    xb = synth.activations(cfg.T, cfg.H, seed=5)
    if special == "nan":
        xb[0, 100] = 0x7FC0
    elif special == "inf":
        xb[0, 7] = 0x7F80
        xb[0, 900] = 0xFF80
    else:
        xb[:] = 0
    _, dl, prep, _ = x8_prep(dev, xb=xb)
    y, w, idx = run(prep)
    torch.cuda.synchronize()
    assert _lib.workspace_status(prep.workspace) == 0
    bias = None if dl.router_bias is None else dl.router_bias.cpu().numpy()
    ridx, _ = oracle.route(xb, dl.router_w.cpu().numpy(), cfg.k, 0, bias)
    np.testing.assert_array_equal(idx.cpu().numpy(), ridx)
    old = _lib.set_option(_lib.OPT_DECODE_X8, 0)
    try:
        assert kernels(cfg) == FUSED
        yg, wg, ig = run(prep)
    finally:
        _lib.set_option(_lib.OPT_DECODE_X8, old)
    assert torch.equal(ig, idx)
    assert torch.equal(wg.isnan(), w.isnan()) and torch.equal(wg.nan_to_num(), w.nan_to_num())
    assert torch.equal(yg.isnan(), y.isnan())
    if special == "zero":
        assert (idx.cpu().numpy() == np.arange(cfg.k)).all()
        assert torch.equal(y, torch.zeros_like(y))


def test_fused_graph_replays(dev):
    """Replays of a captured single-launch layer (three dependent calls) each
    draw fresh hand-off tags from the workspace counter: every replay, with
    eager calls on the same workspace between replays, equals the eager
    result bit for bit."""
    cfg = synth.MoEConfig("g_t1", 512, 256, 32, 8, 1)
    L = synth.host_layer(cfg)
    ex = dev_weights(L, dev)
    W = torch.from_numpy(L.router_w).to(dev)
    xs = [to_bf16_tensor(synth.activations(1, cfg.H, seed=s), dev) for s in (1, 2, 3)]
    prep = phantom_moe.PreparedForward(ex, W, 1, cfg.k, x=xs[0].clone())
    assert kernels(cfg) == FUSED
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
def test_fused_wait_failure_is_reported(dev, option, fault):
    """A wait that gives up (forced from the host: the waiters expect a tag
    nobody writes, with a short bound) ends normally, sets the workspace
    status and leaves NaN in the outputs it could not compute; the next call
    is correct again."""
    cfg = synth.MoEConfig("fail_t1", 256, 128, 16, 4, 1)
    L = synth.host_layer(cfg)
    ex = dev_weights(L, dev)
    W = torch.from_numpy(L.router_w).to(dev)
    xb = synth.activations(1, cfg.H, seed=9)
    prep = phantom_moe.PreparedForward(ex, W, 1, cfg.k, x=to_bf16_tensor(xb, dev))
    assert kernels(cfg) == FUSED
    y_ok, w_ok, i_ok = run(prep)
    option(_lib.OPT_FUSED_WAIT_POLLS, 64)
    option(_lib.OPT_FUSED_FAULT, fault)
    y, w, idx = faulty_call(prep)
    st = _lib.workspace_status(prep.workspace)
    assert st & fault, f"status {st:#x} lacks bit {fault:#x}"
    assert torch.isnan(y).all()
    if fault == 1:
        assert (idx == -1).all() and torch.isnan(w).all()
    else:
        assert torch.equal(idx, i_ok) and torch.equal(w, w_ok)
    _lib.set_option(_lib.OPT_FUSED_FAULT, 0)
    y2, _, _ = run(prep)
    assert _lib.workspace_status(prep.workspace) == 0
    assert torch.equal(y2, y_ok)


def test_fused_nonfinite_activations(dev):
    """NaN and +-inf in x: no fault, routing as the oracle's contract gives it
    (NaN logits rank below every number, ties to the lower index), the other
    tokens unaffected; the staged launches route identically."""
    cfg = synth.MoEConfig("nan_t4", 256, 128, 16, 4, 4)
    L = synth.host_layer(cfg)
    ex = dev_weights(L, dev)
    W = torch.from_numpy(L.router_w).to(dev)
    xb = synth.activations(cfg.T, cfg.H, seed=3)
    xb[1, 17] = 0x7FC0  # NaN
    xb[2, 5] = 0x7F80   # +inf
    xb[2, 6] = 0xFF80   # -inf
    prep = phantom_moe.PreparedForward(ex, W, cfg.T, cfg.k, x=to_bf16_tensor(xb, dev))
    assert kernels(cfg) == FUSED
    y, w, idx = run(prep)
    torch.cuda.synchronize()
    assert _lib.workspace_status(prep.workspace) == 0
    ridx, _ = oracle.route(xb, L.router_w, cfg.k, 0)
    np.testing.assert_array_equal(idx.cpu().numpy(), ridx)
    ok = [0, 3]
    ry, _, _ = oracle.moe_forward(xb[ok], L.router_w, L.gate, L.up, L.down, cfg.k)
    check_y(y.cpu().numpy()[ok], ry, "finite tokens")
    old = _lib.set_option(_lib.OPT_DECODE_FUSED, 0)
    try:
        ys, ws_, iss = run(prep)
    finally:
        _lib.set_option(_lib.OPT_DECODE_FUSED, old)
    assert torch.equal(iss, idx)


def small_fused_layer(dev, seed=9):
    cfg = synth.MoEConfig("fail_t1", 256, 128, 16, 4, 1)
    L = synth.host_layer(cfg)
    ex = dev_weights(L, dev)
    W = torch.from_numpy(L.router_w).to(dev)
    x = to_bf16_tensor(synth.activations(1, cfg.H, seed=seed), dev)
    assert kernels(cfg) == FUSED
    return cfg, ex, W, x


@pytest.mark.parametrize("sync_check", [False, True], ids=["next_call", "sync_check"])
def test_wait_failure_raises_from_moe_forward(dev, option, sync_check):
    """A forced wait failure reaches the caller of moe_forward as
    FusedWaitError, not as silent NaN: under sync check from the failing
    call itself, otherwise from the next call (the kernel stores the bit
    into the pinned host word; no synchronisation on the normal path).  The
    call after that is correct again."""
    cfg, ex, W, x = small_fused_layer(dev)
    y_ok = phantom_moe.moe_forward(x, W, ex, cfg.k).clone()
    torch.cuda.synchronize()
    phantom_moe.check_status()
    option(_lib.OPT_FUSED_WAIT_POLLS, 64)
    option(_lib.OPT_FUSED_FAULT, 2)
    old = phantom_moe.set_sync_check(sync_check)
    try:
        if sync_check:
            with pytest.raises(phantom_moe.FusedWaitError, match="gate/up"):
                phantom_moe.moe_forward(x, W, ex, cfg.k)
        else:
            y_bad = phantom_moe.moe_forward(x, W, ex, cfg.k)
            torch.cuda.synchronize()
            assert torch.isnan(y_bad).all()
            _lib.set_option(_lib.OPT_FUSED_FAULT, 0)
            with pytest.raises(phantom_moe.FusedWaitError, match="gate/up"):
                phantom_moe.moe_forward(x, W, ex, cfg.k)
    finally:
        phantom_moe.set_sync_check(old)
    _lib.set_option(_lib.OPT_FUSED_FAULT, 0)
    torch.cuda.synchronize()
    phantom_moe.check_status()  # the raise cleared the word
    y2 = phantom_moe.moe_forward(x, W, ex, cfg.k)
    torch.cuda.synchronize()
    phantom_moe.check_status()
    assert torch.equal(y2, y_ok)


@pytest.mark.parametrize("x8", [1, 0], ids=["per_xcd", "generic"])
def test_late_start_takes_its_launch_tag(dev, option, x8):
    """A workgroup that starts after workgroup 0 gave up waiting for it reads
    the generation counter one ahead of its launch.  Forced from the host
    (the last workgroup adds one to the counter it reads), it must still take
    its own launch's tag from its presence word: outputs equal to a normal
    call's, bit for bit, on two calls in a row, with no status set.  Taking
    the counter + 1 instead would publish its h units under a tag nobody in
    its launch waits for (NaN outputs and status bits)."""
    if x8:
        cfg, dl, prep, xb = x8_prep(dev, seed=31)
    else:
        option(_lib.OPT_DECODE_X8, 0)
        cfg, ex, W, x = small_fused_layer(dev, seed=31)
        prep = phantom_moe.PreparedForward(ex, W, 1, cfg.k, x=x)
    y_ok, w_ok, i_ok = run(prep)  # every presence word now holds this call's tag
    option(_lib.OPT_FUSED_WAIT_POLLS, 4096)
    option(_lib.OPT_FUSED_FAULT, 4)
    for call in range(2):
        y, w, idx = run(prep)
        torch.cuda.synchronize()
        phantom_moe.check_status()
        assert _lib.workspace_status(prep.workspace) == 0, f"call {call}"
        assert torch.equal(y, y_ok) and torch.equal(w, w_ok) and torch.equal(idx, i_ok), f"call {call}"
    _lib.set_option(_lib.OPT_FUSED_FAULT, 0)
    y, _, _ = run(prep)
    torch.cuda.synchronize()
    assert _lib.workspace_status(prep.workspace) == 0
    assert torch.equal(y, y_ok)
