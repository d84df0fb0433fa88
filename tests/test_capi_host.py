"""Host-side checks of libphantom_moe.so that need no GPU: it loads, exports
every entry point include/phantom_moe.h declares, reports sizes, and rejects
invalid arguments with a status code (never an exit) before touching the
device."""
import ctypes
import os
import re

import numpy as np
import pytest

from phantom_moe import _lib, q4_0, synth

HEADER = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "include", "phantom_moe.h")
EINVAL, EWORKSPACE, ELAUNCH, EUNSUPPORTED = -1, -2, -3, -4
FAKE = 0x10000  # never dereferenced: every call below fails validation first


LEGACY_HEADER = os.path.join(os.path.dirname(HEADER), "phantom_legacy.h")


def declared_symbols():
    text = open(HEADER).read()
    names = re.findall(r"PHANTOM_MOE_API\s+[\w\s\*]+?\b(phantom_\w+)\s*\(", text)
    legacy = re.findall(r"PHANTOM_LEGACY_API\s+[\w\s\*]+?\b(\w+)\s*\(", open(LEGACY_HEADER).read())
    return names + legacy


def test_library_exports_every_declared_symbol():
    lib = _lib.load()
    names = declared_symbols()
    assert len(names) >= 14
    assert {"sparse_mlp_forward", "predict_active_neurons", "get_sparsity_stats"} <= set(names)
    for n in names:
        assert hasattr(lib, n), f"{n} declared in include/ but not exported"
        assert n in _lib.SIGNATURES, f"{n} has no ctypes signature"
    assert set(_lib.SIGNATURES) == set(names)


def test_legacy_validation_returns_status_not_exit():
    """The reference exits on these (kernels/common/cuda_utils.h:31-52); the
    library returns the negative status as a float before any HIP call."""
    lib = _lib.load()
    F = FAKE
    smf = lib.sparse_mlp_forward
    assert smf(F, F, None, F, None, F, F, F, F, 0, 64, 128, 50.0, None) == EINVAL  # B = 0
    assert smf(F, F, None, F, None, F, F, F, F, 1, -1, 128, 50.0, None) == EINVAL  # D < 0
    assert smf(None, F, None, F, None, F, F, F, F, 1, 64, 128, 50.0, None) == EINVAL
    assert smf(F, F, None, F, None, F, None, F, F, 1, 64, 128, 50.0, None) == EINVAL  # sparse needs lists
    # 1000% sparsity: the reference grid would be empty (launch failure there)
    assert smf(F, F, None, F, None, F, F, F, F, 1, 64, 128, 1000.0, None) == EINVAL
    assert smf(F, F, None, F, None, F, F, F, F, 1, 64, 128, float("nan"), None) == EINVAL
    pan = lib.predict_active_neurons
    assert pan(F, F, None, F, F, F, None, 0, 64, 128, 0.5, None) == EINVAL
    assert pan(F, F, None, None, F, F, None, 1, 64, 128, 0.5, None) == EINVAL
    assert pan(F, F, None, F, F, F, None, 1, 64, 0, 0.5, None) == EINVAL
    gss = lib.get_sparsity_stats
    assert gss(F, -1, 128, None) == EINVAL
    assert gss(None, 2, 128, None) == EINVAL
    assert np.isnan(gss(None, 0, 128, None))  # 0 / 0, as the reference
    msg = lib.phantom_moe_last_error().decode()
    assert msg == "" or "get_sparsity_stats" in msg
    cal = lib.calibrate_sparsity_gate
    assert cal(F, F, 0, 8, 8, F, F, F, F, F, None) == EINVAL
    assert cal(F, None, 4, 8, 8, F, F, F, F, F, None) == EINVAL
    assert "calibrate_sparsity_gate" in lib.phantom_moe_last_error().decode()


def test_version_and_sizes():
    lib = _lib.load()
    assert b"gfx950" in lib.phantom_moe_version()
    assert q4_0.nib_bytes(768, 2048) == 768 * 2048 // 2
    assert q4_0.scale_count(768, 2048) == 768 * 2048 // 32
    # K padded to a multiple of 128
    assert q4_0.nib_bytes(16, 96) == 16 * 128 // 2
    with pytest.raises(ValueError):
        q4_0.nib_bytes(15, 64)
    with pytest.raises(ValueError):
        q4_0.nib_bytes(16, 40)
    a = lib.phantom_moe_workspace_bytes(32, 2048, 768, 128, 8, 0)
    b = lib.phantom_moe_workspace_bytes(64, 2048, 768, 128, 8, 0)
    c = lib.phantom_moe_workspace_bytes(32, 2048, 768, 128, 8, 1)
    assert 0 < a < b and a < c
    assert lib.phantom_moe_workspace_bytes(0, 2048, 768, 128, 8, 0) == 0
    # one-token layers reserve the streaming single launch's hand-off regions
    # (logit slots 128 B apart, h units, expert-output units) on top of the
    # staged plan's; a two-token layer does not
    one = lib.phantom_moe_workspace_bytes(1, 4096, 14336, 8, 2, 0)
    two = lib.phantom_moe_workspace_bytes(2, 4096, 14336, 8, 2, 0)
    assert one > 16 * 3 * (14336 // 2) + 16 * 3 * (4096 // 2) + 128 * 8
    assert two > 0


def test_decode_stream_option():
    """PHANTOM_MOE_OPT_DECODE_STREAM takes 0 (off), 1 (default: where no
    staging single launch fits) or 2 (every one-token shape); anything else
    is rejected and leaves the value unchanged."""
    lib = _lib.load()
    old = _lib.set_option(_lib.OPT_DECODE_STREAM, 2)
    try:
        v = ctypes.c_int()
        assert lib.phantom_moe_get_option(_lib.OPT_DECODE_STREAM, ctypes.byref(v)) == 0 and v.value == 2
        assert lib.phantom_moe_set_option(_lib.OPT_DECODE_STREAM, 3) == EINVAL
        assert "DECODE_STREAM" in lib.phantom_moe_last_error().decode()
        assert lib.phantom_moe_set_option(_lib.OPT_DECODE_STREAM, -1) == EINVAL
        assert lib.phantom_moe_get_option(_lib.OPT_DECODE_STREAM, ctypes.byref(v)) == 0 and v.value == 2
    finally:
        _lib.set_option(_lib.OPT_DECODE_STREAM, old)


def _route(**kw):
    args = dict(x=FAKE, x_dtype=0, W=FAKE, b=None, T=4, H=256, E=8, k=2, score=0, idx=FAKE, w=FAKE, ws=None,
                wsb=0, stream=None)
    args.update(kw)
    lib = _lib.load()
    return lib.phantom_moe_route(args["x"], args["x_dtype"], args["W"], args["b"], args["T"], args["H"], args["E"],
                                 args["k"], args["score"], args["idx"], args["w"], args["ws"], args["wsb"],
                                 args["stream"])


@pytest.mark.parametrize(
    "kw,code",
    [
        (dict(x=None), EINVAL),
        (dict(W=None), EINVAL),
        (dict(x_dtype=2), EINVAL),
        (dict(T=0), EINVAL),
        (dict(H=100), EINVAL),
        (dict(H=0), EINVAL),
        (dict(k=9), EINVAL),
        (dict(k=0), EINVAL),
        (dict(E=0), EINVAL),
        (dict(E=1000, k=2), EUNSUPPORTED),
        (dict(E=64, k=40), EUNSUPPORTED),
        (dict(score=3), EINVAL),
        (dict(idx=None), EINVAL),
        (dict(ws=None), EWORKSPACE),
        (dict(ws=FAKE, wsb=16), EWORKSPACE),
    ],
)
def test_route_validation(kw, code):
    assert _route(**kw) == code
    assert _lib.load().phantom_moe_last_error()


def _forward(**kw):
    a = dict(x=FAKE, xd=0, T=4, H=256, I=128, E=8, k=2, score=0, W=FAKE, b=None, w6=[FAKE] * 6, sh=[None] * 6,
             y=FAKE, idx=FAKE, tw=FAKE, ws=None, wsb=0)
    a.update(kw)
    lib = _lib.load()
    return lib.phantom_moe_forward(a["x"], a["xd"], a["T"], a["H"], a["I"], a["E"], a["k"], a["score"], a["W"],
                                   a["b"], *a["w6"], *a["sh"], a["y"], a["idx"], a["tw"], a["ws"], a["wsb"], None)


@pytest.mark.parametrize(
    "kw,code",
    [
        (dict(xd=1), EUNSUPPORTED),
        (dict(I=48), EINVAL),
        (dict(I=0), EINVAL),
        (dict(w6=[FAKE] * 5 + [None]), EINVAL),
        (dict(sh=[FAKE] + [None] * 5), EINVAL),
        (dict(y=None), EINVAL),
        (dict(ws=None), EWORKSPACE),
        (dict(T=-1), EINVAL),
        # decode regime (under 64 positions per expert) with one segment's
        # down operand above 2 GiB
        (dict(T=32000, I=16896, E=512, k=1), EUNSUPPORTED),
    ],
)
def test_forward_validation(kw, code):
    assert _forward(**kw) == code


def test_repack_and_permute_validation():
    lib = _lib.load()
    assert lib.phantom_q4_0_repack(FAKE, 15, 64, FAKE, FAKE, None) == EINVAL
    assert lib.phantom_q4_0_repack(FAKE, 16, 40, FAKE, FAKE, None) == EINVAL
    assert lib.phantom_q4_0_repack(None, 16, 64, FAKE, FAKE, None) == EINVAL
    assert lib.phantom_q4_0_repack(FAKE, 16, 64, FAKE + 4, FAKE, None) == EINVAL  # misaligned nib
    assert lib.phantom_q4_0_repack(None, 0, 64, None, None, None) == 0  # empty is a no-op
    assert lib.phantom_q4_0_unrepack(FAKE, FAKE, 16, 33, FAKE, None) == EINVAL
    assert lib.phantom_q4_0_dequant_f32(FAKE, 4, 31, FAKE, None) == EINVAL
    assert lib.phantom_moe_permute(None, 4, 2, 8, FAKE, FAKE, FAKE, None, 0, None) == EINVAL
    assert lib.phantom_moe_permute(FAKE, 4, 9, 8, FAKE, FAKE, FAKE, None, 0, None) == EINVAL
    assert lib.phantom_moe_permute(FAKE, 4, 2, 8, FAKE, FAKE, FAKE, None, 0, None) == EWORKSPACE
    assert lib.phantom_moe_permute(FAKE, 4, 2, 600, FAKE, FAKE, FAKE, None, 0, None) == EUNSUPPORTED


def test_python_surface_rejects_cpu_tensors():
    import torch

    import phantom_moe

    r = phantom_moe.PhantomTopKRouter(256, 8, 2)
    with pytest.raises(RuntimeError, match="no CPU path"), torch.no_grad():
        r(torch.randn(2, 4, 256))
    # inference only: no silent detach of the gate weight
    with pytest.raises(RuntimeError, match="no backward"):
        r(torch.randn(2, 4, 256))
    with pytest.raises(TypeError):
        q4_0.repack(torch.zeros(18, dtype=torch.uint8), 16, 32)


def test_synth_configs_and_determinism():
    c = synth.CONFIGS["qwen3_decode_t32_zipf"]
    assert (c.H, c.I, c.E, c.k, c.T) == (2048, 768, 128, 8, 32)
    assert c.expert_bytes() == 2654208
    assert synth.CONFIGS["dsv3_decode_t1"].shared and synth.CONFIGS["dsv3_decode_t1"].score_mode == 1
    small = synth.scaled(c, H=64, I=32, E=8, k=2, T=4)
    a = synth.host_layer(small)
    b = synth.host_layer(small)
    assert np.array_equal(a.gate, b.gate) and np.array_equal(a.router_w, b.router_w)
    bias = synth.zipf_bias(128, 1.1)
    golden = np.load(os.path.join(os.path.dirname(__file__), "golden", "zipf_bias_e128_s1.1.npy"))
    np.testing.assert_array_equal(bias, golden)
    x = synth.activations(3, 64)
    assert x.dtype == np.uint16
    # bf16 rounding is round-to-nearest-even
    np.testing.assert_array_equal(synth.f32_to_bf16_bits(np.array([1.0 + 2.0 ** -8], np.float32)),
                                  np.array([0x3F80], np.uint16))
    np.testing.assert_array_equal(synth.f32_to_bf16_bits(np.array([1.0 + 3 * 2.0 ** -8], np.float32)),
                                  np.array([0x3F82], np.uint16))


def test_profile_events_validation():
    """The timing hook takes the documented number of non-null events or NULL."""
    lib = _lib.load()
    hdr = open(os.path.join(os.path.dirname(__file__), "..", "include", "phantom_moe.h")).read()
    n = int(re.search(r"#define PHANTOM_MOE_PROFILE_EVENTS (\d+)", hdr).group(1))
    assert lib.phantom_moe_set_profile_events(None, 0) == 0
    short = (ctypes.c_void_p * n)(*([FAKE] * n))
    assert lib.phantom_moe_set_profile_events(short, n - 1) == EINVAL
    holes = (ctypes.c_void_p * n)(*([FAKE] * (n - 1) + [None]))
    assert lib.phantom_moe_set_profile_events(holes, n) == EINVAL
    assert lib.phantom_moe_set_profile_events(None, 0) == 0
