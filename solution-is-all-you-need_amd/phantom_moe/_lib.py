"""ctypes binding of libphantom_moe.so (declared in include/phantom_moe.h).

The library is built in-tree by ``phantom_moe._build.build()`` into
``phantom_moe/lib/libphantom_moe.so``.  There is no fallback: if the library
is missing, every operator raises.

torch is imported before the library is loaded.  torch ships its own HIP
runtime (soname libamdhip64.so.7); loading torch first makes the dynamic
linker bind our library's libamdhip64.so.7 dependency to that same runtime,
so device pointers and streams from torch are valid in our calls.  The loader
checks /proc/self/maps afterwards and refuses to run with two HIP runtimes.
"""
from __future__ import annotations

import ctypes
import os
import threading

import torch  # noqa: F401  (must precede the CDLL, see module docstring)

LIB_DIR = os.path.join(os.path.dirname(os.path.abspath(__file__)), "lib")
# PHANTOM_MOE_LIB selects another build of the same sources (the host-sanitized
# lib/asan/libphantom_moe.so of ``python -m phantom_moe._build --sanitize``).
LIB_PATH = os.environ.get("PHANTOM_MOE_LIB") or os.path.join(LIB_DIR, "libphantom_moe.so")

# Function name -> (restype, argtypes).  Mirrors include/phantom_moe.h and
# include/phantom_legacy.h.
_vp = ctypes.c_void_p
_i64 = ctypes.c_int64
_int = ctypes.c_int
_sz = ctypes.c_size_t
_f32 = ctypes.c_float
SIGNATURES = {
    "phantom_moe_last_error": (ctypes.c_char_p, []),
    "phantom_moe_version": (ctypes.c_char_p, []),
    "phantom_moe_set_profile_events": (_int, [_vp, _int]),
    "phantom_moe_expert_kernels": (ctypes.c_char_p, [_i64, _i64, _i64, _int, _int, _int]),
    "phantom_q4_0_nib_bytes": (_i64, [_i64, _i64]),
    "phantom_q4_0_scale_bytes": (_i64, [_i64, _i64]),
    "phantom_q4_0_repack": (_int, [_vp, _i64, _i64, _vp, _vp, _vp]),
    "phantom_q4_0_unrepack": (_int, [_vp, _vp, _i64, _i64, _vp, _vp]),
    "phantom_q4_0_dequant_f32": (_int, [_vp, _i64, _i64, _vp, _vp]),
    "phantom_moe_workspace_bytes": (_sz, [_i64, _i64, _i64, _int, _int, _int]),
    "phantom_moe_workspace_status": (_int, [_vp, _sz, _vp, _vp]),
    "phantom_moe_status_word": (ctypes.POINTER(ctypes.c_uint32), []),
    "phantom_moe_set_option": (_int, [_int, _int]),
    "phantom_moe_get_option": (_int, [_int, _vp]),
    "phantom_moe_route": (_int, [_vp, _int, _vp, _vp, _i64, _i64, _int, _int, _int, _vp, _vp, _vp, _sz, _vp]),
    "phantom_moe_permute": (_int, [_vp, _i64, _int, _int, _vp, _vp, _vp, _vp, _sz, _vp]),
    "phantom_moe_forward": (
        _int,
        [_vp, _int, _i64, _i64, _i64, _int, _int, _int, _vp, _vp]
        + [_vp] * 6
        + [_vp] * 6
        + [_vp, _vp, _vp, _vp, _sz, _vp],
    ),
    "phantom_moe_forward_static": (
        _int,
        [_vp, _int, _i64, _i64, _i64, _int, _int, _int, _vp, _vp] + [_vp] * 6 + [_vp] * 6 + [_vp, _vp, _vp, _vp],
    ),
    # include/phantom_legacy.h: the reference's own symbol names and order
    "sparse_mlp_forward": (_f32, [_vp] * 9 + [_int, _int, _int, _f32, _vp]),
    "predict_active_neurons": (_f32, [_vp] * 7 + [_int, _int, _int, _f32, _vp]),
    "get_sparsity_stats": (_f32, [_vp, _int, _int, _vp]),
    "calibrate_sparsity_gate": (_int, [_vp, _vp, _int, _int, _int, _vp, _vp, _vp, _vp, _vp, _vp]),
}

_lock = threading.Lock()
_lib = None
_status_word = None  # ctypes view of the pinned host word (phantom_moe_status_word)
_sync_check = os.environ.get("PHANTOM_MOE_SYNC_CHECK", "0") == "1"


OPT_DECODE_FUSED = 1  # PHANTOM_MOE_OPT_DECODE_FUSED
OPT_DECODE_KSPLIT = 2  # PHANTOM_MOE_OPT_DECODE_KSPLIT
OPT_FUSED_WAIT_POLLS = 3  # PHANTOM_MOE_OPT_FUSED_WAIT_POLLS
OPT_FUSED_FAULT = 4  # PHANTOM_MOE_OPT_FUSED_FAULT
OPT_DECODE_X8 = 5  # PHANTOM_MOE_OPT_DECODE_X8
OPT_DECODE_STREAM = 6  # PHANTOM_MOE_OPT_DECODE_STREAM


class PhantomMoEError(RuntimeError):
    """A libphantom_moe.so entry point returned a non-zero status."""


def _hip_runtimes_mapped() -> set:
    paths = set()
    try:
        with open("/proc/self/maps") as f:
            for line in f:
                parts = line.split()
                if len(parts) >= 6 and os.path.basename(parts[5]).startswith("libamdhip64.so"):
                    paths.add(os.path.realpath(parts[5]))
    except OSError:
        pass
    return paths


def load(path: str = LIB_PATH):
    """Load (once) and return the ctypes handle with typed signatures."""
    global _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not os.path.exists(path):
            raise PhantomMoEError(
                f"{path} is missing: build the HIP library first (python -c 'import __graft_entry__ as g; g.build()')"
            )
        lib = ctypes.CDLL(path)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        runtimes = _hip_runtimes_mapped()
        if len(runtimes) > 1:
            raise PhantomMoEError(f"two HIP runtimes are mapped in this process: {sorted(runtimes)}")
        global _status_word
        if torch.cuda.is_available():
            ptr = lib.phantom_moe_status_word()
            if not ptr:
                raise PhantomMoEError("phantom_moe_status_word failed: "
                                      + lib.phantom_moe_last_error().decode(errors="replace"))
            _status_word = ptr.contents
        _lib = lib
        return lib


def check(rc: int, what: str) -> None:
    if rc != 0:
        msg = load().phantom_moe_last_error().decode(errors="replace")
        raise PhantomMoEError(f"{what} failed (status {rc}): {msg}")


# torch's raw current-stream getter returns the handle as an int without
# building a Stream object (0.04 against 1.8 us a call); the public API is
# the fallback.
_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def stream_handle(device: torch.device | None = None) -> int:
    """hipStream_t of torch's current stream on ``device`` (as an int)."""
    if _raw_stream is not None:
        index = device.index if device is not None else None
        return _raw_stream(torch.cuda.current_device() if index is None else index)
    return torch.cuda.current_stream(device).cuda_stream


def set_option(option: int, value: int) -> int:
    """Set a library option (include/phantom_moe.h); returns the previous value."""
    lib = load()
    old = ctypes.c_int()
    check(lib.phantom_moe_get_option(option, ctypes.byref(old)), "phantom_moe_get_option")
    check(lib.phantom_moe_set_option(option, value), "phantom_moe_set_option")
    return old.value


_STATUS_BITS = ((1, "the router logits"), (2, "the gate/up results or the down partials"),
                (4, "every workgroup to start"))


class FusedWaitError(PhantomMoEError):
    """A single-launch decode call gave up one of its bounded waits: the
    outputs it could not compute are NaN.  Its workgroups were not all
    resident at once (another stream or process held CUs)."""


def check_status() -> None:
    """Raise FusedWaitError if a single-launch decode call of this process
    (eager or a graph replay) gave up a wait since the last check.  Reads the
    pinned host word the kernels set on failure: no synchronisation, so a
    failure shows once its call has finished on the GPU."""
    w = _status_word
    if w is None:
        return
    v = w.value
    if v == 0:
        return
    w.value = 0
    what = ", ".join(name for bit, name in _STATUS_BITS if v & bit) or f"status {v:#x}"
    raise FusedWaitError(
        f"single-launch decode: a bounded wait gave up (waiting for {what}); the outputs that call could not "
        "compute are NaN.  Its workgroups must all be resident at once: do not share the GPU with other work "
        "while it runs, or set PHANTOM_MOE_DECODE=staged for the staged launches.")


def set_sync_check(on: bool) -> bool:
    """With sync check on, every layer call waits for its stream and checks
    the status word before it returns (for debugging; off by default, or
    PHANTOM_MOE_SYNC_CHECK=1).  Returns the previous setting."""
    global _sync_check
    old = _sync_check
    _sync_check = bool(on)
    return old


def after_call(device) -> None:
    """Status check after a layer call: immediate under sync check, else
    whatever earlier calls have left."""
    if _sync_check:
        torch.cuda.current_stream(device).synchronize()
    check_status()


def workspace_status(ws: torch.Tensor) -> int:
    """Status bits the single-launch decode path left in workspace ``ws``
    (0 = every call completed normally); waits for the stream and clears them."""
    lib = load()
    st = ctypes.c_uint32()
    check(lib.phantom_moe_workspace_status(ws.data_ptr(), ws.numel() * ws.element_size(), ctypes.byref(st),
                                           stream_handle(ws.device)), "phantom_moe_workspace_status")
    return st.value
