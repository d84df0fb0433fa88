"""The many-token router (two passes: approximate logits on the matrix cores
with an error bound, then the fixed-order fp64 logits of the candidate
experts) against the oracle's exact routing.

From 128 bf16 tokens on (E >= 16) phantom_moe_route takes this path.  Its
result must equal the one-pass contract bit for bit: the same experts in the
same order and the same weights.  The cases force what the bound must get
right: logits so close that the approximate pass cannot order them (every
expert a candidate, candidates taken 16 at a time), exact ties between
duplicated rows (the lower index wins), a clear top k beside a cluster of
near ties, and non-finite inputs (a token with NaN or inf falls back to the
full exact row)."""
import numpy as np
import pytest

torch = pytest.importorskip("torch")

import phantom_moe  # noqa: E402
from helpers import to_bf16_tensor  # noqa: E402
from oracle import oracle  # noqa: E402
from phantom_moe import synth  # noqa: E402

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def dev():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return torch.device("cuda:0")


def check(dev, xb, W, k, score=0, bias=None):
    x = to_bf16_tensor(xb, dev)
    b = None if bias is None else torch.from_numpy(bias).to(dev)
    w, idx = phantom_moe.route(x, torch.from_numpy(W).to(dev), k, score, b)
    ridx, rw = oracle.route(xb, W, k, score, bias)
    np.testing.assert_array_equal(idx.cpu().numpy(), ridx)
    np.testing.assert_allclose(w.cpu().numpy(), rw, rtol=1e-6, atol=1e-7, equal_nan=True)
    return ridx


def base_inputs(T, H, E, seed):
    rng = np.random.default_rng(seed)
    xb = synth.f32_to_bf16_bits(rng.standard_normal((T, H), dtype=np.float32))
    W = (rng.standard_normal((E, H), dtype=np.float32) * np.float32(0.02)).astype(np.float32)
    return rng, xb, W


@pytest.mark.parametrize("kind", ["cluster", "mixed", "duplicates", "one_ulp"])
def test_near_ties(dev, kind):
    T, H, E, k = 256, 512, 64, 8
    rng, xb, W = base_inputs(T, H, E, seed=hash(kind) % 1000)
    base = W[0].copy()
    if kind == "cluster":
        # every logit within about 1e-6 of the others: all 64 are candidates
        W[:] = base * (1.0 + np.float32(1e-6) * rng.standard_normal((E, H), dtype=np.float32))
    elif kind == "mixed":
        # a cluster of 32 near-identical experts among 32 ordinary ones
        W[:32] = base * (1.0 + np.float32(1e-6) * rng.standard_normal((32, H), dtype=np.float32))
    elif kind == "duplicates":
        # exact ties: rows duplicated at distinct indices
        W[1::4] = W[0::4]
    else:
        # rows one ulp apart in a single element
        W[:] = base
        for e in range(E):
            W[e, e % H] = np.nextafter(base[e % H], np.float32(np.inf) if e % 2 else np.float32(-np.inf))
    ridx = check(dev, xb, W.astype(np.float32), k)
    assert ridx.shape == (T, k)


@pytest.mark.parametrize("T,H,E,k,score", [
    (128, 416, 16, 4, 0),      # the smallest two-pass batch; H not a multiple of 256
    (333, 2048, 128, 8, 0),    # ragged token blocks
    (200, 7168, 256, 8, 1),    # DeepSeek-V3 router shape, sigmoid scores
    (160, 256, 512, 32, 0),    # the widest rows (8 logits per lane), top-32
    (129, 1024, 100, 6, 1),    # E not a multiple of 16
])
def test_shapes_with_bias(dev, T, H, E, k, score):
    rng, xb, W = base_inputs(T, H, E, seed=T + H + E)
    bias = (rng.standard_normal(E).astype(np.float32) * np.float32(0.05)).astype(np.float32)
    check(dev, xb, W, k, score, bias)


def test_non_finite_inputs(dev):
    """NaN and +-inf in some tokens and in the bias: those rows take the full
    exact path and rank exactly as the contract says; other tokens are
    unaffected."""
    T, H, E, k = 192, 256, 64, 8
    rng, xb, W = base_inputs(T, H, E, seed=77)
    xb[3, 10] = 0x7FC0   # NaN
    xb[50, 0] = 0x7F80   # +inf
    xb[51, 7] = 0xFF80   # -inf
    xb[52, 0] = 0x7F80
    xb[52, 1] = 0xFF80   # inf - inf
    check(dev, xb, W, k)
    bias = np.zeros(E, np.float32)
    bias[5] = np.nan
    bias[9] = -np.inf
    bias[12] = np.inf
    check(dev, xb, W, k, 0, bias)


def test_wide_logit_range(dev):
    """Logits from tiny to large magnitudes (scaled rows and tokens): the
    bound scales with |x| |w|, so the selection stays exact."""
    T, H, E, k = 256, 512, 128, 8
    rng, xb, W = base_inputs(T, H, E, seed=5)
    W *= (10.0 ** rng.uniform(-6, 3, size=(E, 1))).astype(np.float32)
    xf = synth.bf16_bits_to_f32(xb) * (10.0 ** rng.uniform(-4, 4, size=(T, 1))).astype(np.float32)
    check(dev, synth.f32_to_bf16_bits(xf.astype(np.float32)), W.astype(np.float32), k)


@pytest.mark.parametrize("H,E,k", [(512, 128, 8), (2048, 128, 8), (7168, 256, 8)])
def test_tiny_rows_underflow(dev, H, E, k):
    """Tokens and expert rows scaled by 2^-80 (every square underflows fp32)
    and by 2^-66..2^-72 (squares in or near the subnormal range): their fp32
    norms lose everything or most bits, and the bound still has to cover the
    bf16 rounding of the approximate logits, so routing stays the oracle's."""
    T = 256
    rng, xb, W = base_inputs(T, H, E, seed=H + E + 3)
    xf = synth.bf16_bits_to_f32(xb).astype(np.float64)
    scale_t = np.ones((T, 1))
    scale_t[::4] = 2.0 ** -80
    scale_t[1::8] = 2.0 ** -70
    scale_t[3::16] = 2.0 ** -66
    xf = (xf * scale_t).astype(np.float32)
    scale_e = np.ones((E, 1))
    scale_e[::3] = 2.0 ** -80
    scale_e[1::10] = 2.0 ** -72
    W = (W.astype(np.float64) * scale_e).astype(np.float32)
    check(dev, synth.f32_to_bf16_bits(xf), W, k)


def _bf16_rne(v):
    """float64 array -> the nearest bf16 values (ties to even), as float64."""
    b = v.astype(np.float32).view(np.uint32).astype(np.uint64)
    b = (b + 0x7FFF + ((b >> 16) & 1)) >> 16 << 16
    return b.astype(np.uint32).view(np.float32).astype(np.float64)


def test_systematic_bf16_ties(dev):
    """Router weights placed on bf16 rounding ties, with the signs of x
    lined up so that every rounding pushes the approximate logit of expert 3
    (the exact top 1) down and that of expert 5 (0.06 below it) up, by
    2^-8 |w| an element: one bf16 copy of w is then off by about 1 in each
    logit, more than 2^-9 |x| |w| covers, and expert 3 would fall out of the
    candidates.  The hi + lo split of w leaves about 2^-12, so routing stays
    the oracle's (checked here on the CPU for the one-copy case too)."""
    T, H, E = 128, 288, 16
    rng = np.random.default_rng(11)
    x = np.ones(H)
    x[128:256] = -1.0
    W = rng.standard_normal((E, H)) * 0.02
    tie, above = 1.0 + 2.0 ** -8, 1.0 + 2.0 ** -8 + 2.0 ** -20
    W[3, :128], W[3, 128:256], W[3, 256:] = tie, above, 0.5
    W[5, :128], W[5, 128:256], W[5, 256:] = above, tie, 0.5 - 2.0 ** -9
    W = W.astype(np.float32)
    w64 = W.astype(np.float64)
    exact = w64 @ x
    one_copy = _bf16_rne(w64) @ x
    assert exact[3] > exact[5] and one_copy[5] - one_copy[3] > 1.9
    b = (2.0 ** -9 + H * 2.0 ** -22) * np.linalg.norm(x) * np.linalg.norm(w64, axis=1)
    assert one_copy[5] - b[5] > one_copy[3] + b[3], "the construction defeats a 2^-9 bound"
    scales = 2.0 ** rng.integers(-3, 4, size=(T, 1))
    xb = synth.f32_to_bf16_bits((x[None, :] * scales).astype(np.float32))
    for k in (1, 2):
        ridx = check(dev, xb, W, k)
        assert (ridx[:, 0] == 3).all()
