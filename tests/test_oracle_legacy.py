"""Pins of the legacy neuron-sparse FFN oracle (oracle/legacy_oracle.c) on the
CPU, each against something other than the oracle's own formula: numpy's
sequential float32 accumulation and float16 conversion, exact integer sums,
hand-built inputs whose result only the contracted summation order gives,
and float64 compositions of the reference kernels' steps."""
import math

import numpy as np
import pytest

from oracle import oracle as O

F16 = np.float16


def h(a):
    return np.asarray(a, dtype=F16)


# --- fp32 -> fp16 conversion -------------------------------------------------

def test_f2h_matches_numpy_rne():
    rng = np.random.default_rng(3)
    vals = np.concatenate([
        rng.standard_normal(20000).astype(np.float32) * np.float32(100.0),
        rng.standard_normal(5000).astype(np.float32) * np.float32(1e-5),   # fp16 subnormals
        np.array([0.0, -0.0, 65504.0, 65519.99, 65520.0, -65520.0, 1e9, -1e9, np.inf, -np.inf,
                  2.0 ** -24, 2.0 ** -25, 3 * 2.0 ** -26, 2.0 ** -14 - 2.0 ** -26, 1.0 + 2.0 ** -11,
                  1.0 + 3 * 2.0 ** -11], dtype=np.float32),
    ])
    with np.errstate(over="ignore"):
        want = vals.astype(F16).view(np.uint16)
    got = np.array([O.lg_f2h(v) for v in vals], dtype=np.uint16)
    np.testing.assert_array_equal(got, want)


# --- dot products ---------------------------------------------------------------

def test_sequential_order_is_numpy_float32_accumulate():
    rng = np.random.default_rng(5)
    for D in (1, 7, 64, 513, 2000):
        w = rng.standard_normal(D).astype(F16)
        x = rng.standard_normal(D).astype(F16)
        prods = w.astype(np.float32) * x.astype(np.float32)  # exact in fp32
        want = np.add.accumulate(prods, dtype=np.float32)[-1]
        assert O.lg_dot(w, x, order=1) == want


def test_contract_order_exact_on_integers():
    rng = np.random.default_rng(6)
    for D in (8, 512, 1500, 4096):
        w = rng.integers(-8, 8, D).astype(F16)
        x = rng.integers(-8, 8, D).astype(F16)
        exact = int(np.dot(w.astype(np.int64), x.astype(np.int64)))
        assert O.lg_dot(w, x, 0) == exact
        assert O.lg_dot(w, x, 1) == exact


def _spikes(D, entries):
    """w, x with the product v at element d for each (d, v), v = a*b, fp16 a, b."""
    w = np.zeros(D, F16)
    x = np.zeros(D, F16)
    for d, (a, b) in entries.items():
        w[d], x[d] = a, b
    return w, x


def test_contract_order_lane_boundaries_and_tree():
    big = (4096.0, 4096.0)      # 2^24
    nbig = (-4096.0, 4096.0)    # -2^24
    one = (1.0, 1.0)
    D = 1024
    # d = 0..7 share partial 0: 2^24 + 1 rounds back to 2^24, then cancels
    assert O.lg_dot(*_spikes(D, {0: big, 7: one, 8: nbig}), 0) == 0.0
    # d = 8 starts partial 1: -2^24 + 1 is exact, so the 1 survives
    assert O.lg_dot(*_spikes(D, {0: big, 8: one, 9: nbig}), 0) == 1.0
    # d = 512 wraps to partial 0 again
    assert O.lg_dot(*_spikes(D, {0: big, 512: one, 8: nbig}), 0) == 0.0
    # tree: partial 32 (d = 256) joins partial 0 at s = 32, before partial 1
    # does (s = 1), so the 1 is absorbed into 2^24
    assert O.lg_dot(*_spikes(D, {0: big, 256: one, 8: nbig}), 0) == 0.0
    # partial 33 (d = 264) joins partial 1 at s = 32: -2^24 + 1 is exact, and
    # adding 2^24 at s = 1 leaves 1
    assert O.lg_dot(*_spikes(D, {0: big, 264: one, 8: nbig}), 0) == 1.0
    # partial 63 (d = 511) travels 63 -> 31 -> 15 -> 7 -> 3 -> 1 -> 0: it meets
    # partial 1 (s = 2) before partial 0, so it survives as well
    assert O.lg_dot(*_spikes(D, {0: big, 511: one, 8: nbig}), 0) == 1.0
    # the sequential order keeps the 1 whenever it comes after the cancellation
    assert O.lg_dot(*_spikes(D, {0: big, 8: nbig, 512: one}), 1) == 1.0
    assert O.lg_dot(*_spikes(D, {0: big, 7: one, 8: nbig}), 1) == 0.0


def test_contract_order_close_to_exact_sum():
    rng = np.random.default_rng(8)
    for D in (100, 4096, 7000):
        w = rng.standard_normal(D).astype(F16)
        x = rng.standard_normal(D).astype(F16)
        p = w.astype(np.float64) * x.astype(np.float64)
        exact = math.fsum(p)
        bound = 80 * 2.0 ** -24 * np.abs(p).sum()  # (D/64 + 6) roundings at most along any path
        assert abs(float(O.lg_dot(w, x, 0)) - exact) <= bound
        assert abs(float(O.lg_dot(w, x, 1)) - exact) <= D * 2.0 ** -24 * np.abs(p).sum()


# --- predictor -------------------------------------------------------------------

def _rand_layer(rng, B, D, Dffn, scale=0.05):
    x = rng.standard_normal((B, D)).astype(F16)
    w = (rng.standard_normal((Dffn, D)) * scale).astype(F16)
    b = (rng.standard_normal(Dffn) * 0.5).astype(F16)
    return x, w, b


def test_predict_gate_mask_and_compaction():
    rng = np.random.default_rng(9)
    x, w, b = _rand_layer(rng, 3, 200, 300)
    gate, mask, idx, cnt = O.lg_predict(x, w, b, 0.5)
    for bi in range(3):
        for n in range(0, 300, 37):
            a = np.float32(O.lg_dot(w[n], x[bi], 0) + np.float32(b[n]))
            assert gate[bi, n] == np.float32(1.0 / (1.0 + math.exp(-float(a))))
        on = np.flatnonzero(gate[bi] >= np.float32(0.5))
        np.testing.assert_array_equal(mask[bi], (gate[bi] >= np.float32(0.5)).astype(np.uint8))
        assert cnt[bi] == on.size
        np.testing.assert_array_equal(idx[bi, : on.size], on)
        assert (idx[bi, on.size:] == -1).all()  # untouched past the count
    # no bias: gate = sigmoid(dot); threshold 0 marks everything, > 1 nothing
    g0, m0, _, c0 = O.lg_predict(x, w, None, 0.0)
    assert (c0 == 300).all() and (m0 == 1).all()
    _, _, _, c1 = O.lg_predict(x, w, None, 1.5)
    assert (c1 == 0).all()


def test_predict_orders_agree_closely():
    rng = np.random.default_rng(10)
    x, w, b = _rand_layer(rng, 2, 1024, 256)
    g0 = O.lg_predict(x, w, b, 0.5, order=0)[0]
    g1 = O.lg_predict(x, w, b, 0.5, order=1)[0]
    np.testing.assert_allclose(g0, g1, rtol=0, atol=1e-6)


# --- sparse MLP ------------------------------------------------------------------

def _ffn_ref_f64(x, wg, bg, wu, bu, wd, lists, cover, dense):
    """float64 composition of the reference kernels' steps with their fp16
    stores (sparse_matmul.cu:56-100, :120-167, :187-215)."""
    B, D = x.shape
    Dffn = wg.shape[0]
    y = np.zeros((B, D), np.float64)
    for bi in range(B):
        act = np.zeros(Dffn, np.float64)
        lst = list(range(Dffn)) if dense else list(lists[bi])
        for i, n in enumerate(lst):
            if (not dense and i >= cover) or not (0 <= n < Dffn):
                continue
            g = float(np.dot(wg[n].astype(np.float64), x[bi].astype(np.float64)))
            u = float(np.dot(wu[n].astype(np.float64), x[bi].astype(np.float64)))
            if not dense:
                g += float(bg[n]) if bg is not None else 0.0
                u += float(bu[n]) if bu is not None else 0.0
            g, u = float(F16(g)), float(F16(u))
            act[n] = float(F16(g / (1.0 + math.exp(-g)) * u))
        for n in lst:
            if 0 <= n < Dffn:
                y[bi] += act[n] * wd[:, n].astype(np.float64)
    return y


def _mlp_case(rng, B, D, Dffn, density):
    x = rng.standard_normal((B, D)).astype(F16)
    wg = (rng.standard_normal((Dffn, D)) / math.sqrt(D)).astype(F16)
    wu = (rng.standard_normal((Dffn, D)) / math.sqrt(D)).astype(F16)
    wd = (rng.standard_normal((D, Dffn)) / math.sqrt(Dffn)).astype(F16)
    bg = (rng.standard_normal(Dffn) * 0.1).astype(F16)
    bu = (rng.standard_normal(Dffn) * 0.1).astype(F16)
    idx = np.full((B, Dffn), -1, np.int32)
    cnt = np.zeros(B, np.int32)
    for bi in range(B):
        on = np.flatnonzero(rng.random(Dffn) < density)
        idx[bi, : on.size] = on
        cnt[bi] = on.size
    return x, wg, bg, wu, bu, wd, idx, cnt


def _y(yb):
    return yb.view(F16).astype(np.float64)


@pytest.mark.parametrize("pct", [10.0, 50.0])
def test_sparse_mlp_matches_f64_composition(pct):
    rng = np.random.default_rng(11)
    B, D, Dffn = 3, 256, 384
    x, wg, bg, wu, bu, wd, idx, cnt = _mlp_case(rng, B, D, Dffn, 0.5)
    dense = pct < 30
    lists = [idx[bi, : cnt[bi]] for bi in range(B)]
    ref = _ffn_ref_f64(x, wg, bg, wu, bu, wd, lists, 10 ** 9, dense)
    for order in (0, 1):
        y = _y(O.lg_sparse_mlp(x, wg, bg, wu, bu, wd, idx, cnt, pct, order))
        err = np.abs(y - ref)
        # fp16 output rounding plus fp32 sums and an occasional one-ulp act flip
        assert err.max() <= 2e-3 + 2 ** -10 * np.abs(ref).max(), (order, err.max())
        assert np.linalg.norm(y - ref) <= 1e-3 * np.linalg.norm(ref)


def test_dense_branch_ignores_biases_and_lists():
    rng = np.random.default_rng(12)
    x, wg, bg, wu, bu, wd, idx, cnt = _mlp_case(rng, 2, 128, 256, 0.3)
    y1 = O.lg_sparse_mlp(x, wg, bg, wu, bu, wd, idx, cnt, 29.9)
    y2 = O.lg_sparse_mlp(x, wg, None, wu, None, wd, None, None, 0.0)
    np.testing.assert_array_equal(y1, y2)
    # at 30% the sparse branch runs, with the biases
    y3 = O.lg_sparse_mlp(x, wg, bg, wu, bu, wd, idx, cnt, 30.0)
    assert not np.array_equal(y1, y3)


def test_sparse_branch_grid_coverage():
    """sparse_matmul.cu:320-333: at 90% sparsity and D_ffn = 1024 the grid
    covers ceil((int(0.1 * 1024) + 32) / 256) * 256 = 256 list positions;
    later positions keep their zero activation, so listing more neurons than
    that changes nothing."""
    rng = np.random.default_rng(13)
    B, D, Dffn = 1, 64, 1024
    x, wg, bg, wu, bu, wd, _, _ = _mlp_case(rng, B, D, Dffn, 0.0)
    order = rng.permutation(Dffn).astype(np.int32)
    idx = order[None, :].copy()
    y300 = O.lg_sparse_mlp(x, wg, bg, wu, bu, wd, idx, np.array([300], np.int32), 90.0)
    y256 = O.lg_sparse_mlp(x, wg, bg, wu, bu, wd, idx, np.array([256], np.int32), 90.0)
    np.testing.assert_array_equal(y300, y256)
    y255 = O.lg_sparse_mlp(x, wg, bg, wu, bu, wd, idx, np.array([255], np.int32), 90.0)
    assert not np.array_equal(y255, y256)
    ref = _ffn_ref_f64(x, wg, bg, wu, bu, wd, [order[:300]], 256, False)
    np.testing.assert_allclose(_y(y300), ref, atol=2e-3, rtol=2e-3)
    with pytest.raises(ValueError):
        O.lg_sparse_mlp(x, wg, bg, wu, bu, wd, idx, np.array([300], np.int32), 1000.0)


def test_sparse_branch_duplicates_invalid_and_counts():
    rng = np.random.default_rng(14)
    B, D, Dffn = 1, 64, 256
    x, wg, bg, wu, bu, wd, _, _ = _mlp_case(rng, B, D, Dffn, 0.0)
    base = np.array([[3, 9, 200] + [0] * (Dffn - 3)], np.int32)
    y = O.lg_sparse_mlp(x, wg, bg, wu, bu, wd, base, np.array([3], np.int32), 50.0)
    # a duplicate entry adds its term twice to the down projection
    dup = base.copy()
    dup[0, 3] = 9
    y_dup = O.lg_sparse_mlp(x, wg, bg, wu, bu, wd, dup, np.array([4], np.int32), 50.0)
    ref_dup = _ffn_ref_f64(x, wg, bg, wu, bu, wd, [[3, 9, 200, 9]], 10 ** 9, False)
    np.testing.assert_allclose(_y(y_dup), ref_dup, atol=2e-3, rtol=2e-3)
    assert not np.array_equal(y, y_dup)
    # out-of-range indices are skipped
    bad = base.copy()
    bad[0, 3], bad[0, 4] = -5, Dffn
    np.testing.assert_array_equal(O.lg_sparse_mlp(x, wg, bg, wu, bu, wd, bad, np.array([5], np.int32), 50.0), y)
    # negative count: nothing active, y = 0; count above D_ffn is clamped
    z = O.lg_sparse_mlp(x, wg, bg, wu, bu, wd, base, np.array([-3], np.int32), 50.0)
    assert (z.view(F16) == 0).all()


def test_sparsity_stats_closed_form():
    c = np.array([100, 250, 0, 1024], np.int32)
    want = np.float32((np.float32(1.0) - np.float32(c.sum()) / np.float32(4) / np.float32(1024)) * np.float32(100))
    assert O.lg_sparsity(c, 1024) == want
    assert O.lg_sparsity(np.array([512], np.int32), 1024) == np.float32(50.0)


# --- gate calibration ------------------------------------------------------------

def test_calibration_mask_rule():
    """gate_calibrate.cu:54-85: active iff |a| >= 0.01 * max(row max |a|, 1e-10);
    NaN is never active (fmaxf ignores it in the max)."""
    act = np.array([[0.5, -0.004, 0.006, np.nan, 0.0, -0.005],
                    [0.0, 0.0, 0.0, 0.0, 0.0, 0.0]], np.float32)
    x = np.zeros((2, 8), np.float32)
    _, _, masks, _, _, _, sp = O.lg_calibrate(x, act, 0, epochs=0)
    np.testing.assert_array_equal(masks, [[1, 0, 1, 0, 0, 1], [0, 0, 0, 0, 0, 0]])
    assert sp == np.float32((1.0 - 3 / 12) * 100)


def test_calibration_first_step_closed_form():
    """From zero weights every prediction is sigmoid(0) = 1/2, so one step is
    w = -lr * mean_s((1/2 - y_s) x_s), b = -lr * mean_s(1/2 - y_s)."""
    rng = np.random.default_rng(20)
    x = rng.standard_normal((13, 40)).astype(np.float32)
    act = rng.standard_normal((13, 24)).astype(np.float32)
    w, b, masks, _, _, _, _ = O.lg_calibrate(x, act, 0, epochs=1)
    e = 0.5 - masks.astype(np.float64)
    w_ref = -1e-3 * (e.T @ x.astype(np.float64)) / 13
    b_ref = -1e-3 * e.mean(0)
    np.testing.assert_allclose(w, w_ref, rtol=1e-5, atol=1e-9)
    np.testing.assert_allclose(b, b_ref, rtol=1e-5, atol=1e-9)


def test_calibration_f1_and_orders():
    rng = np.random.default_rng(21)
    x = rng.standard_normal((30, 64)).astype(np.float32)
    W = (rng.standard_normal((48, 64)) * 0.3).astype(np.float32)
    act = np.maximum(x @ W.T, 0).astype(np.float32)
    w0, b0, m0, p0, en0, f10, sp0 = O.lg_calibrate(x, act, 0)
    pr, ac = p0 >= np.float32(0.5), m0 > 0
    tp, fp, fn = int((pr & ac).sum()), int((pr & ~ac).sum()), int((~pr & ac).sum())
    prec, rec = np.float32(tp) / np.float32(tp + fp), np.float32(tp) / np.float32(tp + fn)
    assert f10 == np.float32(np.float32(2.0) * prec * rec / (prec + rec))
    assert en0 == (f10 >= np.float32(0.70))
    w1, b1, m1, _, en1, f11, sp1 = O.lg_calibrate(x, act, 1)
    np.testing.assert_array_equal(m0, m1)
    assert sp0 == sp1
    np.testing.assert_allclose(w0, w1, rtol=1e-4, atol=1e-7)
    assert abs(f10 - f11) <= 1e-2
