"""phantom_moe_forward_static -- the layer entry point that allocates nothing
(its scratch is a static device array of the library) -- against
phantom_moe_forward with a caller workspace, through the C ABI.

Both run the same kernels, and the layer is deterministic, so routing, routing
weights and outputs must agree bit for bit.  Each case makes two static calls
in a row on the shared scratch, the second with a smaller input (the first
leaves its contents behind), and a third at a size beyond the scratch must be
refused without touching the outputs."""
import numpy as np
import pytest

torch = pytest.importorskip("torch")

import phantom_moe  # noqa: E402
from phantom_moe import _lib, synth  # noqa: E402

pytestmark = pytest.mark.gpu

STATIC_SCRATCH_BYTES = 16 << 20
EWORKSPACE = -2


@pytest.fixture(scope="module")
def dev():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return torch.device("cuda:0")


def prepared(ex, dl, cfg, T, dev, seed):
    xb = synth.activations(T, cfg.H, seed=seed)
    x = torch.from_numpy(xb.view(np.int16)).view(torch.bfloat16).to(dev)
    return phantom_moe.PreparedForward(ex, dl.router_w, T, cfg.k, cfg.score, dl.router_bias, x=x)


def call_static(prep, stream):
    """The same call as ``prep`` with the workspace pointer and size left out
    (the last two of its bound arguments)."""
    lib = _lib.load()
    y = torch.full_like(prep.y, float("nan"))
    idx = torch.full_like(prep.topk_idx, -1)
    w = torch.full_like(prep.topk_w, float("nan"))
    args = list(prep._args[:-2])
    args[-3], args[-2], args[-1] = y.data_ptr(), idx.data_ptr(), w.data_ptr()
    rc = lib.phantom_moe_forward_static(*args, stream)
    return rc, y, idx, w


@pytest.mark.parametrize("cfg,sizes", [
    (synth.CONFIGS["qwen3_decode_t1"], (32, 1, 256)),  # staged launches, then the single launch
    (synth.MoEConfig("na_sigmoid_shared", 512, 128, 32, 4, 1, score="sigmoid", shared=True), (8, 3, 4096)),
], ids=["qwen3", "sigmoid_shared"])
def test_static_scratch_matches_workspace(dev, cfg, sizes):
    dl = synth.device_layer(cfg, dev)
    ex = phantom_moe.MoEWeights.from_q4_0(dl.gate, dl.up, dl.down, cfg.H, cfg.I, cfg.E, shared=dl.shared)
    lib = _lib.load()
    stream = _lib.stream_handle(dev)
    big, small, too_big = sizes
    assert lib.phantom_moe_workspace_bytes(too_big, cfg.H, cfg.I, cfg.E, cfg.k, int(cfg.shared)) > STATIC_SCRATCH_BYTES
    for i, T in enumerate((big, small)):
        assert lib.phantom_moe_workspace_bytes(T, cfg.H, cfg.I, cfg.E, cfg.k, int(cfg.shared)) <= STATIC_SCRATCH_BYTES
        prep = prepared(ex, dl, cfg, T, dev, seed=50 + i)
        print(f"[case] {cfg.name} T={T} ({lib.phantom_moe_expert_kernels(T, cfg.H, cfg.I, cfg.E, cfg.k, int(cfg.shared)).decode()})",
              flush=True)
        rc, y, idx, w = call_static(prep, stream)
        assert rc == 0, _lib.load().phantom_moe_last_error().decode()
        prep()
        torch.cuda.synchronize()
        assert _lib.workspace_status(prep.workspace) == 0
        assert torch.equal(idx, prep.topk_idx), f"T={T}: routing differs"
        assert torch.equal(w, prep.topk_w), f"T={T}: routing weights differ"
        assert torch.equal(y, prep.y), f"T={T}: layer output differs"
        assert torch.isfinite(y).all()

    prep = prepared(ex, dl, cfg, too_big, dev, seed=99)
    rc, y, idx, w = call_static(prep, stream)
    torch.cuda.synchronize()
    assert rc == EWORKSPACE
    assert "static scratch" in _lib.load().phantom_moe_last_error().decode()
    assert torch.isnan(y).all() and (idx == -1).all()
