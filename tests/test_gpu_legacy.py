"""Parity of the legacy neuron-sparse FFN ABI (include/phantom_legacy.h) on
the GPU against the CPU oracle (oracle/legacy_oracle.c), through the
reference's own C symbols.

The GPU follows the oracle's order-0 summation bit for bit, so gates, masks,
active lists, counts and fp16 outputs are compared for equality.  The one
operation the two sides do not share is the float64 exp inside the sigmoid
(device library vs C library): it can move an fp32 result by one ulp, so
fp16 outputs may differ by one fp16 ulp in rare elements; the tests allow at
most 0.1% such elements and nothing larger.  Against the reference kernels'
own sequential loops (oracle order 1) the outputs must meet the layer
tolerance: max abs <= 1e-2 and rel-L2 <= 1e-3.
"""
import math

import numpy as np
import pytest

torch = pytest.importorskip("torch")

from phantom_moe import legacy  # noqa: E402
from oracle import oracle as O  # noqa: E402

pytestmark = pytest.mark.gpu
F16 = np.float16


@pytest.fixture(scope="module")
def dev():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return torch.device("cuda:0")


def T(a, dev):
    return None if a is None else torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def _case(seed, B, D, Dffn, density, scale_g=None):
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((B, D)).astype(F16)
    s = 1.0 / math.sqrt(max(D, 1)) if scale_g is None else scale_g
    wg = (rng.standard_normal((Dffn, D)) * s).astype(F16)
    wu = (rng.standard_normal((Dffn, D)) * s).astype(F16)
    wd = (rng.standard_normal((D, Dffn)) / math.sqrt(Dffn)).astype(F16)
    bg = (rng.standard_normal(Dffn) * 0.1).astype(F16)
    bu = (rng.standard_normal(Dffn) * 0.1).astype(F16)
    idx = np.full((B, Dffn), -1, np.int32)
    cnt = np.zeros(B, np.int32)
    for b in range(B):
        on = np.flatnonzero(rng.random(Dffn) < density).astype(np.int32)
        idx[b, : on.size] = on
        cnt[b] = on.size
    return x, wg, bg, wu, bu, wd, idx, cnt


def assert_f16_close_bits(got, want, what):
    """Equal fp16 bit patterns, except at most 0.1% of elements one ulp apart."""
    g = np.asarray(got).view(np.uint16).astype(np.int32)
    w = np.asarray(want).view(np.uint16).astype(np.int32)
    # ordered integer view of fp16 so adjacent values differ by 1
    og = np.where(g & 0x8000, 0x8000 - (g & 0x7FFF), 0x8000 + g)
    ow = np.where(w & 0x8000, 0x8000 - (w & 0x7FFF), 0x8000 + w)
    d = np.abs(og - ow)
    assert d.max() <= 1, f"{what}: {int((d > 1).sum())} elements more than one ulp apart"
    assert (d > 0).mean() <= 1e-3, f"{what}: {int((d > 0).sum())} of {d.size} elements differ"


def check_layer_tolerance(got_bits, ref_bits):
    y = np.asarray(got_bits).view(F16).astype(np.float64)
    r = np.asarray(ref_bits).view(F16).astype(np.float64)
    assert np.abs(y - r).max() <= 1e-2
    assert np.linalg.norm(y - r) <= 1e-3 * max(np.linalg.norm(r), 1e-30)


# ------------------------------------------------------------ predictor


@pytest.mark.parametrize("B,D,Dffn", [(1, 4096, 1024), (3, 200, 300), (8, 512, 777), (11, 64, 100),
                                      (2, 0, 64), (5, 1031, 2049)])
def test_predict_matches_oracle(dev, B, D, Dffn):
    rng = np.random.default_rng(B * 1000 + D + Dffn)
    x = rng.standard_normal((B, D)).astype(F16)
    w = (rng.standard_normal((Dffn, D)) * 0.05).astype(F16)
    b = (rng.standard_normal(Dffn) * 0.5).astype(F16)
    thr = 0.5
    mask, idx, cnt, gate, ms = legacy.predict_active_neurons(T(x, dev), T(w, dev), T(b, dev), thr)
    g0, m0, i0, c0 = O.lg_predict(x, w, b, thr, order=0)
    assert ms >= 0.0
    gate = gate.cpu().numpy()
    np.testing.assert_array_equal(gate, g0)
    np.testing.assert_array_equal(mask.cpu().numpy(), m0)
    np.testing.assert_array_equal(cnt.cpu().numpy(), c0)
    idx = idx.cpu().numpy()
    for bi in range(B):
        np.testing.assert_array_equal(idx[bi, : c0[bi]], i0[bi, : c0[bi]])
        assert (idx[bi, c0[bi]:] == -1).all()  # entries past the count are not written
    # against the reference's sequential loop: the two fp32 summation orders
    # differ by a few ulps of |w . x| (about 1e-5 here at D = 4096), and the
    # sigmoid's slope is at most 1/4
    g1 = O.lg_predict(x, w, b, thr, order=1)[0]
    np.testing.assert_allclose(gate, g1, rtol=0, atol=1e-5)


def test_predict_without_bias_or_gate_output(dev):
    x, w, *_ = _case(21, 4, 256, 512, 0.5, scale_g=0.1)
    mask, idx, cnt, gate, _ = legacy.predict_active_neurons(T(x, dev), T(w, dev), None, 0.55,
                                                            want_gate_output=False)
    assert gate is None
    _, m0, i0, c0 = O.lg_predict(x, w, None, 0.55)
    np.testing.assert_array_equal(mask.cpu().numpy(), m0)
    np.testing.assert_array_equal(cnt.cpu().numpy(), c0)
    got = idx.cpu().numpy()
    for bi in range(4):
        np.testing.assert_array_equal(got[bi, : c0[bi]], i0[bi, : c0[bi]])
    s = legacy.get_sparsity_stats(cnt, 512)
    assert np.float32(s) == O.lg_sparsity(c0, 512)


# ------------------------------------------------------------ sparse MLP


@pytest.mark.parametrize(
    "B,D,Dffn,density,pct",
    [
        (1, 4096, 1024, 0.5, 50.0),    # sparse branch, vector loads
        (3, 256, 384, 0.5, 50.0),
        (3, 256, 384, 0.8, 10.0),      # dense branch: biases and lists ignored
        (9, 512, 640, 0.7, 20.0),      # dense, two batch tiles
        (2, 200, 300, 0.4, 60.0),      # D not a multiple of 8: element loads
        (1, 64, 1024, 0.6, 90.0),      # coverage 256 < count: later positions stay zero
        (4, 1024, 2048, 0.3, 70.0),
    ],
)
def test_sparse_mlp_matches_oracle(dev, B, D, Dffn, density, pct):
    x, wg, bg, wu, bu, wd, idx, cnt = _case(B * 31 + D + Dffn, B, D, Dffn, density)
    y, ms = legacy.sparse_mlp_forward(T(x, dev), T(wg, dev), T(bg, dev), T(wu, dev), T(bu, dev), T(wd, dev),
                                      T(idx, dev), T(cnt, dev), pct)
    assert ms >= 0.0
    got = y.cpu().numpy().view(np.uint16)
    want = O.lg_sparse_mlp(x, wg, bg, wu, bu, wd, idx, cnt, pct, order=0)
    assert_f16_close_bits(got, want, f"y B={B} D={D} Dffn={Dffn} pct={pct}")
    check_layer_tolerance(got, O.lg_sparse_mlp(x, wg, bg, wu, bu, wd, idx, cnt, pct, order=1))


def test_sparse_mlp_duplicates_invalid_and_counts(dev):
    x, wg, bg, wu, bu, wd, _, _ = _case(41, 2, 128, 256, 0.0)
    idx = np.zeros((2, 256), np.int32)
    idx[0, :6] = [3, 9, 200, 9, -5, 256]   # a duplicate and two out-of-range entries
    idx[1, :3] = [1, 2, 3]
    for cnt in (np.array([6, 3], np.int32), np.array([-2, 999], np.int32)):
        y, _ = legacy.sparse_mlp_forward(T(x, dev), T(wg, dev), T(bg, dev), T(wu, dev), T(bu, dev), T(wd, dev),
                                         T(idx, dev), T(cnt, dev), 50.0)
        want = O.lg_sparse_mlp(x, wg, bg, wu, bu, wd, idx, cnt, 50.0)
        assert_f16_close_bits(y.cpu().numpy(), want, f"counts {cnt.tolist()}")


def test_predict_then_sparse_mlp_pipeline(dev):
    """The reference's intended use: the predictor's lists drive the FFN, and
    get_sparsity_stats picks the branch."""
    rng = np.random.default_rng(51)
    B, D, Dffn = 2, 1024, 1536
    x = rng.standard_normal((B, D)).astype(F16)
    wp = (rng.standard_normal((Dffn, D)) * 0.04).astype(F16)
    bp = (rng.standard_normal(Dffn) * 0.3).astype(F16)
    _, wg, bg, wu, bu, wd, _, _ = _case(52, B, D, Dffn, 0.0)
    tx = T(x, dev)
    _, idx, cnt, _, _ = legacy.predict_active_neurons(tx, T(wp, dev), T(bp, dev), 0.6)
    pct = legacy.get_sparsity_stats(cnt, Dffn)
    _, _, i0, c0 = O.lg_predict(x, wp, bp, 0.6)
    assert np.float32(pct) == O.lg_sparsity(c0, Dffn)
    y, _ = legacy.sparse_mlp_forward(tx, T(wg, dev), T(bg, dev), T(wu, dev), T(bu, dev), T(wd, dev), idx, cnt, pct)
    i0 = np.where(i0 < 0, 0, i0)  # entries past the count are never read
    want = O.lg_sparse_mlp(x, wg, bg, wu, bu, wd, i0, c0, pct)
    assert_f16_close_bits(y.cpu().numpy(), want, "pipeline")


def test_activation_buffer_grows_and_is_reused(dev):
    for B, Dffn in ((1, 256), (4, 4096), (2, 512)):
        x, wg, bg, wu, bu, wd, idx, cnt = _case(60 + B, B, 128, Dffn, 0.5)
        y, _ = legacy.sparse_mlp_forward(T(x, dev), T(wg, dev), T(bg, dev), T(wu, dev), T(bu, dev), T(wd, dev),
                                         T(idx, dev), T(cnt, dev), 50.0)
        assert_f16_close_bits(y.cpu().numpy(), O.lg_sparse_mlp(x, wg, bg, wu, bu, wd, idx, cnt, 50.0),
                              f"B={B} Dffn={Dffn}")


@pytest.mark.filterwarnings("ignore:The CUDA Graph is empty")  # the refused capture records nothing
def test_captured_graph_survives_buffer_growth(dev):
    """A graph that captured sparse_mlp_forward keeps its activation buffer:
    eager calls use a buffer of their own, and an eager call at a larger size
    allocates a larger capture buffer without freeing the one the graph holds.
    A capture at a size no eager call has reserved is refused."""
    x, wg, bg, wu, bu, wd, idx, cnt = _case(80, 2, 128, 512, 0.5)
    args = [T(a, dev) for a in (x, wg, bg, wu, bu, wd, idx, cnt)]
    want = O.lg_sparse_mlp(x, wg, bg, wu, bu, wd, idx, cnt, 50.0)
    legacy.sparse_mlp_forward(*args, 50.0)  # reserves both buffers at this size
    side = torch.cuda.Stream(dev)
    side.wait_stream(torch.cuda.current_stream(dev))
    g = torch.cuda.CUDAGraph()
    with torch.cuda.stream(side), torch.cuda.graph(g, stream=side):
        y_cap, ms = legacy.sparse_mlp_forward(*args, 50.0)
    assert ms == 0.0
    torch.cuda.current_stream(dev).wait_stream(side)
    g.replay()
    torch.cuda.synchronize(dev)
    assert_f16_close_bits(y_cap.cpu().numpy(), want, "first replay")
    # eager calls in between, the second one larger than anything before
    y_small, _ = legacy.sparse_mlp_forward(*args, 50.0)
    assert_f16_close_bits(y_small.cpu().numpy(), want, "eager")
    xl, wgl, bgl, wul, bul, wdl, idxl, cntl = _case(81, 8, 128, 8192, 0.5)
    y_big, _ = legacy.sparse_mlp_forward(*[T(a, dev) for a in (xl, wgl, bgl, wul, bul, wdl, idxl, cntl)], 50.0)
    assert_f16_close_bits(y_big.cpu().numpy(), O.lg_sparse_mlp(xl, wgl, bgl, wul, bul, wdl, idxl, cntl, 50.0),
                          "eager after growth")
    y_cap.zero_()
    g.replay()
    torch.cuda.synchronize(dev)
    assert_f16_close_bits(y_cap.cpu().numpy(), want, "replay after growth")
    # refused: no buffer of this size was reserved outside capture
    xh, wgh, bgh, wuh, buh, wdh, idxh, cnth = _case(82, 16, 64, 16384, 0.5)
    huge = [T(a, dev) for a in (xh, wgh, bgh, wuh, buh, wdh, idxh, cnth)]
    torch.cuda.synchronize(dev)
    g2 = torch.cuda.CUDAGraph()
    err = None
    with torch.cuda.stream(side), torch.cuda.graph(g2, stream=side):
        try:
            legacy.sparse_mlp_forward(*huge, 50.0)
        except RuntimeError as e:
            err = str(e)
    assert err is not None and "under stream capture" in err
    del g2
    g.replay()
    torch.cuda.synchronize(dev)
    assert_f16_close_bits(y_cap.cpu().numpy(), want, "replay after a refused capture")


def test_errors_raise_not_exit(dev):
    x, wg, bg, wu, bu, wd, idx, cnt = _case(70, 1, 64, 128, 0.5)
    with pytest.raises(RuntimeError, match="no list position"):
        legacy.sparse_mlp_forward(T(x, dev), T(wg, dev), T(bg, dev), T(wu, dev), T(bu, dev), T(wd, dev),
                                  T(idx, dev), T(cnt, dev), 500.0)
    with pytest.raises(RuntimeError, match="float16"):
        legacy.sparse_mlp_forward(T(x, dev).float(), T(wg, dev), None, T(wu, dev), None, T(wd, dev),
                                  None, None, 0.0)


# ------------------------------------------------------------ gate calibration


@pytest.mark.parametrize("N,D,Dffn", [(37, 200, 96), (8, 512, 1000), (1, 64, 33), (64, 1031, 130)])
def test_calibrate_matches_oracle(dev, N, D, Dffn):
    rng = np.random.default_rng(N * 7 + D + Dffn)
    x = rng.standard_normal((N, D)).astype(np.float32)
    W = (rng.standard_normal((Dffn, D)) / np.sqrt(D)).astype(np.float32)
    act = np.maximum(x @ W.T, 0).astype(np.float32) * rng.random((N, Dffn)).astype(np.float32)
    w, b, en, f1, sp = legacy.calibrate_sparsity_gate(T(x, dev), T(act, dev))
    w0, b0, m0, p0, en0, f10, sp0 = O.lg_calibrate(x, act, 0)
    assert np.float32(sp) == sp0
    # same order, same fused operations: bit-exact unless an fp64 exp of the
    # device library and of the C library round apart in one sigmoid
    np.testing.assert_allclose(w.cpu().numpy(), w0, rtol=1e-6, atol=1e-12)
    np.testing.assert_allclose(b.cpu().numpy(), b0, rtol=1e-6, atol=1e-12)
    assert abs(f1 - float(f10)) <= 1e-6 and en == en0
    # against the reference's loops: weights agree to fp32 rounding
    w1, b1, _, _, en1, f11, _ = O.lg_calibrate(x, act, 1)
    np.testing.assert_allclose(w.cpu().numpy(), w1, rtol=1e-4, atol=1e-7)
    assert abs(f1 - float(f11)) <= 1e-2


def test_calibrate_errors(dev):
    x = torch.zeros((4, 8), dtype=torch.float32, device=dev)
    with pytest.raises(RuntimeError, match="same number of rows"):
        legacy.calibrate_sparsity_gate(x, torch.zeros((3, 8), dtype=torch.float32, device=dev))
    with pytest.raises(RuntimeError, match="float32"):
        legacy.calibrate_sparsity_gate(x.half(), torch.zeros((4, 8), dtype=torch.float32, device=dev))
