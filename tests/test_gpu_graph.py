"""A layer forward captured in a HIP graph replays to the eager result.

Every launch of phantom_moe_forward is a kernel on the caller's stream (no
allocation, no memset node, no host synchronisation), so the call can be
captured.  The graph is replayed several times, with eager work and a
clobbered output between replays, and every replay must reproduce the eager
outputs bit for bit (the layer is deterministic)."""
import numpy as np
import pytest

torch = pytest.importorskip("torch")

import phantom_moe  # noqa: E402
from phantom_moe import synth  # noqa: E402

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def dev():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return torch.device("cuda:0")


def prepared(cfg, dev, layer):
    dl = synth.device_layer(cfg, dev, layer=layer)
    ex = phantom_moe.MoEWeights.from_q4_0(dl.gate, dl.up, dl.down, cfg.H, cfg.I, cfg.E, shared=dl.shared)
    xb = synth.activations(cfg.T, cfg.H, seed=100 + layer)
    x = torch.from_numpy(xb.view(np.int16)).view(torch.bfloat16).to(dev)
    return phantom_moe.PreparedForward(ex, dl.router_w, cfg.T, cfg.k, cfg.score, dl.router_bias, x=x)


@pytest.mark.parametrize("cfg", [
    synth.CONFIGS["qwen3_decode_t32_zipf"],                                           # grouped GEMV regime
    synth.scaled(synth.CONFIGS["dsv3_decode_t8"], H=1024, I=256, E=32, name="dsv3_small"),  # shared expert
    synth.scaled(synth.CONFIGS["qwen3_prefill_t4096"], E=16, k=4, T=512, name="prefill_small"),  # MFMA GEMM regime
], ids=lambda c: c.name)
def test_graph_replay_matches_eager(dev, cfg):
    layers = [prepared(cfg, dev, l) for l in range(2)]
    eager = []
    for p in layers:
        p()
        eager.append((p.y.clone(), p.topk_idx.clone(), p.topk_w.clone()))
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for p in layers:
            p()
    for rep in range(3):
        for p in layers:
            p.y.fill_(float("nan"))
            p.topk_idx.fill_(-1)
        layers[0]()  # eager work between replays
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        for p, (y, idx, w) in zip(layers, eager):
            assert torch.equal(p.topk_idx, idx), f"replay {rep}: routing differs"
            assert torch.equal(p.topk_w, w), f"replay {rep}: routing weights differ"
            assert torch.equal(p.y, y), f"replay {rep}: layer output differs"
