"""numpy front end of the CPU oracle (moe_oracle.c).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg, never by the product package.  Every function
here calls the C restatement in ``oracle/_build/libmoe_oracle.so``; the
reference file:line each one follows is given in moe_oracle.c.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
# PHANTOM_ORACLE_LIB selects another build of the same sources (the sanitized
# one of `make -C oracle asan`).
_LIB_PATH = os.environ.get("PHANTOM_ORACLE_LIB") or os.path.join(_HERE, "_build", "libmoe_oracle.so")
_lib = None

_f32p = np.ctypeslib.ndpointer(dtype=np.float32, flags="C_CONTIGUOUS")
_f64p = np.ctypeslib.ndpointer(dtype=np.float64, flags="C_CONTIGUOUS")
_i32p = np.ctypeslib.ndpointer(dtype=np.int32, flags="C_CONTIGUOUS")
_u8p = np.ctypeslib.ndpointer(dtype=np.uint8, flags="C_CONTIGUOUS")
_u16p = np.ctypeslib.ndpointer(dtype=np.uint16, flags="C_CONTIGUOUS")
_vp = ctypes.c_void_p
_i64 = ctypes.c_int64
_int = ctypes.c_int


def build() -> str:
    """Compile the oracle with its Makefile (gcc)."""
    subprocess.run(["make", "-s", "-C", _HERE], check=True)
    return _LIB_PATH


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        L = ctypes.CDLL(_LIB_PATH)
        L.oracle_q4_0_dequant.argtypes = [_u8p, _i64, _f32p]
        L.oracle_q4_0_dequant.restype = None
        L.oracle_canonical_dot.argtypes = [_f32p, _f32p, _i64]
        L.oracle_canonical_dot.restype = ctypes.c_double
        L.oracle_route.argtypes = [_f32p, _f32p, _vp, _i64, _i64, _int, _int, _int, _i32p, _f32p, _vp]
        L.oracle_route.restype = _int
        L.oracle_permute.argtypes = [_i32p, _i64, _int, _i32p, _i32p, _i32p]
        L.oracle_permute.restype = _int
        L.oracle_expert_ffn.argtypes = [_f32p, _u8p, _u8p, _u8p, _i64, _i64, _f64p]
        L.oracle_expert_ffn.restype = _int
        L.oracle_moe_forward.argtypes = [
            _f32p, _i64, _i64, _i64, _int, _int, _int, _f32p, _vp,
            _u8p, _u8p, _u8p, _vp, _vp, _vp, _f32p, _i32p, _f32p,
        ]
        L.oracle_moe_forward.restype = _int
        L.oracle_half_to_float.argtypes = [ctypes.c_uint16]
        L.oracle_half_to_float.restype = ctypes.c_float
        L.oracle_bf16_to_float.argtypes = [_u16p, _i64, _f32p]
        L.oracle_bf16_to_float.restype = None
        # legacy_oracle.c
        L.oracle_lg_dot.argtypes = [_u16p, _u16p, _i64, _int]
        L.oracle_lg_dot.restype = ctypes.c_float
        L.oracle_lg_f2h.argtypes = [ctypes.c_float]
        L.oracle_lg_f2h.restype = ctypes.c_uint16
        L.oracle_lg_predict.argtypes = [_u16p, _u16p, _vp, _i64, _i64, _i64, ctypes.c_float, _int,
                                        _f32p, _u8p, _i32p, _i32p]
        L.oracle_lg_predict.restype = None
        L.oracle_lg_sparse_mlp.argtypes = [_u16p, _u16p, _vp, _u16p, _vp, _u16p, _vp, _vp,
                                           _i64, _i64, _i64, ctypes.c_float, _int, _u16p]
        L.oracle_lg_sparse_mlp.restype = _int
        L.oracle_lg_sparsity.argtypes = [_i32p, _i64, _i64]
        L.oracle_lg_sparsity.restype = ctypes.c_float
        L.oracle_lg_calibrate.argtypes = [_f32p, _f32p, _i64, _i64, _i64, _int, _int, _f32p, _f32p, _u8p, _f32p,
                                          _vp, _vp, _vp]
        L.oracle_lg_calibrate.restype = None
        _lib = L
    return _lib


def _ptr(a):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


def as_f32(x) -> np.ndarray:
    """Widen x to fp32 exactly.  Accepts fp32 arrays or raw bf16 bits (uint16)."""
    x = np.ascontiguousarray(x)
    if x.dtype == np.uint16:
        out = np.empty(x.shape, dtype=np.float32)
        lib().oracle_bf16_to_float(x.reshape(-1), x.size, out.reshape(-1))
        return out
    if x.dtype != np.float32:
        raise TypeError(f"oracle expects fp32 values or bf16 bits, got {x.dtype}")
    return x


def q4_0_dequant(blocks: np.ndarray, shape) -> np.ndarray:
    """Q4_0 bytes -> fp32 values of ``shape`` (gguf_loader.py:362-381)."""
    blocks = np.ascontiguousarray(blocks, dtype=np.uint8).reshape(-1)
    n = int(np.prod(shape))
    if n % 32 or blocks.size < n // 32 * 18:
        raise ValueError("Q4_0 payload too short or element count not a multiple of 32")
    out = np.empty(n, dtype=np.float32)
    lib().oracle_q4_0_dequant(blocks, n // 32, out)
    return out.reshape(shape)


def canonical_dot(x: np.ndarray, w: np.ndarray) -> float:
    x = as_f32(x).reshape(-1)
    w = np.ascontiguousarray(w, dtype=np.float32).reshape(-1)
    assert x.size == w.size
    return float(lib().oracle_canonical_dot(x, w, x.size))


def route(x, router_w, top_k: int, score_mode: int = 0, router_bias=None, return_logits=False):
    """Router of tests/test_moe_routing.py:56-72 under the fixed-order contract.

    Returns (idx [T,k] int32, w [T,k] fp32[, logits [T,E] fp64])."""
    x = as_f32(x)
    T, H = x.shape
    W = np.ascontiguousarray(router_w, dtype=np.float32)
    E = W.shape[0]
    assert W.shape == (E, H)
    b = None if router_bias is None else np.ascontiguousarray(router_bias, dtype=np.float32)
    idx = np.empty((T, top_k), dtype=np.int32)
    w = np.empty((T, top_k), dtype=np.float32)
    lg = np.empty((T, E), dtype=np.float64) if return_logits else None
    rc = lib().oracle_route(x, W, _ptr(b), T, H, E, top_k, score_mode, idx, w, _ptr(lg))
    if rc:
        raise ValueError(f"oracle_route rejected the arguments (rc={rc})")
    return (idx, w, lg) if return_logits else (idx, w)


def permute(idx: np.ndarray, num_experts: int):
    """Stable counting sort of slots by expert.

    Returns (offsets [E+1], sorted_slots [n], slot_pos [n]) as int32."""
    flat = np.ascontiguousarray(idx, dtype=np.int32).reshape(-1)
    n = flat.size
    off = np.empty(num_experts + 1, dtype=np.int32)
    ss = np.empty(n, dtype=np.int32)
    sp = np.empty(n, dtype=np.int32)
    rc = lib().oracle_permute(flat, n, num_experts, off, ss, sp)
    if rc:
        raise ValueError("expert index out of range")
    return off, ss, sp


def expert_ffn(x, gate_q4, up_q4, down_q4, H: int, I: int) -> np.ndarray:
    """One SwiGLU expert on Q4_0 bytes, fp64 result [H]."""
    x = as_f32(x).reshape(-1)
    y = np.empty(H, dtype=np.float64)
    rc = lib().oracle_expert_ffn(
        x,
        np.ascontiguousarray(gate_q4, dtype=np.uint8).reshape(-1),
        np.ascontiguousarray(up_q4, dtype=np.uint8).reshape(-1),
        np.ascontiguousarray(down_q4, dtype=np.uint8).reshape(-1),
        H,
        I,
        y,
    )
    if rc:
        raise ValueError("oracle_expert_ffn: H and I must be multiples of 32")
    return y


def moe_forward(x, router_w, gate_q4, up_q4, down_q4, top_k: int, score_mode: int = 0,
                router_bias=None, shared=None, tokens=None):
    """Whole MoE layer in fp64 arithmetic, fp32 result.

    gate_q4/up_q4: uint8 [E, I, H/32, 18] (or flat); down_q4: [E, H, I/32, 18].
    shared: None or (gate_q4, up_q4, down_q4) of one expert.
    tokens: optional index array selecting a subset of rows of x (tokens are
    independent, so a subset is an exact restriction of the layer).
    Returns (y [n,H] fp32, idx [n,k] int32, w [n,k] fp32)."""
    x = as_f32(x)
    if tokens is not None:
        x = np.ascontiguousarray(x[np.asarray(tokens)])
    n, H = x.shape
    W = np.ascontiguousarray(router_w, dtype=np.float32)
    E = W.shape[0]
    g = np.ascontiguousarray(gate_q4, dtype=np.uint8).reshape(-1)
    u = np.ascontiguousarray(up_q4, dtype=np.uint8).reshape(-1)
    d = np.ascontiguousarray(down_q4, dtype=np.uint8).reshape(-1)
    I = g.size // (E * (H // 32) * 18)
    assert g.size == E * I * (H // 32) * 18, "gate_q4 size does not match [E, I, H/32, 18]"
    b = None if router_bias is None else np.ascontiguousarray(router_bias, dtype=np.float32)
    sh = [None, None, None]
    if shared is not None:
        sh = [np.ascontiguousarray(a, dtype=np.uint8).reshape(-1) for a in shared]
    y = np.empty((n, H), dtype=np.float32)
    idx = np.empty((n, top_k), dtype=np.int32)
    w = np.empty((n, top_k), dtype=np.float32)
    rc = lib().oracle_moe_forward(
        x, n, H, I, E, top_k, score_mode, W, _ptr(b), g, u, d,
        _ptr(sh[0]), _ptr(sh[1]), _ptr(sh[2]), y, idx, w,
    )
    if rc:
        raise ValueError(f"oracle_moe_forward rejected the arguments (rc={rc})")
    return y, idx, w


# ---------------------------------------------------------------------------
# legacy neuron-sparse FFN ABI (legacy_oracle.c).  fp16 arrays are passed as
# numpy float16 or as their uint16 bit patterns; order 0 is this build's fixed
# summation order, order 1 the reference kernels' sequential loops.


def _h16(a) -> np.ndarray:
    a = np.asarray(a)
    if a.dtype == np.float16:
        a = a.view(np.uint16)
    return np.ascontiguousarray(a, dtype=np.uint16)


def lg_dot(w, x, order: int = 0) -> np.float32:
    w, x = _h16(w).reshape(-1), _h16(x).reshape(-1)
    assert w.size == x.size
    return np.float32(lib().oracle_lg_dot(w, x, w.size, order))


def lg_f2h(f: float) -> np.uint16:
    """fp32 -> fp16 bits, round to nearest even (the oracle's own conversion)."""
    return np.uint16(lib().oracle_lg_f2h(float(np.float32(f))))


def lg_predict(x, w, bias, threshold: float, order: int = 0):
    """predict_active_neurons: returns (gate [B,Dffn] f32, mask [B,Dffn] u8,
    indices [B,Dffn] i32 (first count[b] valid, rest -1), count [B] i32)."""
    x, w = _h16(x), _h16(w)
    B, D = x.shape
    D_ffn = w.shape[0]
    b = None if bias is None else _h16(bias).reshape(-1)
    gate = np.empty((B, D_ffn), np.float32)
    mask = np.empty((B, D_ffn), np.uint8)
    idx = np.full((B, D_ffn), -1, np.int32)
    cnt = np.empty(B, np.int32)
    lib().oracle_lg_predict(x, w, _ptr(b), B, D, D_ffn, float(np.float32(threshold)), order, gate, mask, idx, cnt)
    return gate, mask, idx, cnt


def lg_sparse_mlp(x, wg, bg, wu, bu, wd, idx, count, sparsity_pct: float, order: int = 0) -> np.ndarray:
    """sparse_mlp_forward: returns y [B, D] as fp16 bits (uint16)."""
    x, wg, wu, wd = _h16(x), _h16(wg), _h16(wu), _h16(wd)
    B, D = x.shape
    D_ffn = wg.shape[0]
    bg = None if bg is None else _h16(bg).reshape(-1)
    bu = None if bu is None else _h16(bu).reshape(-1)
    idx = None if idx is None else np.ascontiguousarray(idx, dtype=np.int32)
    count = None if count is None else np.ascontiguousarray(count, dtype=np.int32)
    y = np.empty((B, D), np.uint16)
    rc = lib().oracle_lg_sparse_mlp(x, wg, _ptr(bg), wu, _ptr(bu), wd, _ptr(idx), _ptr(count),
                                    B, D, D_ffn, float(np.float32(sparsity_pct)), order, y)
    if rc:
        raise ValueError("oracle_lg_sparse_mlp: sparsity_pct leaves no list position to compute")
    return y


def lg_sparsity(count, D_ffn: int) -> np.float32:
    c = np.ascontiguousarray(count, dtype=np.int32).reshape(-1)
    return np.float32(lib().oracle_lg_sparsity(c, c.size, D_ffn))


def lg_calibrate(x, act, order: int = 0, epochs: int = 50):
    """calibrate_sparsity_gate: returns (w [D_ffn, D], b [D_ffn], masks, final
    predictions [N, D_ffn], enabled, f1, sparsity_pct)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    act = np.ascontiguousarray(act, dtype=np.float32)
    N, D = x.shape
    D_ffn = act.shape[1]
    w = np.empty((D_ffn, D), np.float32)
    b = np.empty(D_ffn, np.float32)
    masks = np.empty((N, D_ffn), np.uint8)
    pred = np.empty((N, D_ffn), np.float32)
    en, f1, sp = ctypes.c_int(0), ctypes.c_float(0), ctypes.c_float(0)
    lib().oracle_lg_calibrate(x, act, N, D, D_ffn, order, epochs, w, b, masks, pred, ctypes.byref(en),
                              ctypes.byref(f1), ctypes.byref(sp))
    return w, b, masks, pred, bool(en.value), np.float32(f1.value), np.float32(sp.value)
