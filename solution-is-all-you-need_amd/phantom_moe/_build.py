"""In-tree build of libphantom_moe.so for gfx950 with hipcc.

Every call compiles (no up-to-date check), so the library always matches the
sources.  The output goes to ``phantom_moe/lib/``, which travels with the
repository tree; nothing is installed into site-packages.
"""
from __future__ import annotations

import os
import subprocess
import tempfile

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG_DIR)
CSRC = os.path.join(ROOT, "csrc")
INCLUDE = os.path.join(os.path.dirname(ROOT), "include")
SOURCES = ["q4_repack.hip", "router.hip", "expert_ffn.hip", "expert_gemm.hip", "decode_fused.hip",
           "decode_stream.hip", "legacy_ffn.hip", "gate_calibrate.hip", "capi.hip"]
ARCH = "gfx950"

HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-shared",
    "-fvisibility=hidden",
    # No packed fp32 VALU instructions anywhere in device code.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # Atomics stay plain instructions: the wave-aggregating rewrite waits for
    # an atomic's result right after issuing it, which would put the job
    # ticket of the fused expert kernel on its critical path.
    "-mllvm", "-amdgpu-atomic-optimizer-strategy=None",
    "-Wall",
    # a variable read in its own initializer is undefined behaviour that the
    # optimizer exploits (it can delete whole phases of a kernel): an error
    "-Werror=uninitialized",
]


# Host-side AddressSanitizer + UndefinedBehaviorSanitizer for a CPU-only test
# build (lib/asan/libphantom_moe.so): the C-ABI validation, planning and error
# paths run instrumented; device code is compiled as usual.  Each flag applies
# to the host pass only.
SANITIZE_FLAGS = [
    "-Xarch_host", "-fsanitize=address",
    "-Xarch_host", "-fsanitize=undefined",
    "-Xarch_host", "-fno-sanitize-recover=undefined",
    "-Xarch_host", "-fno-omit-frame-pointer",
    "-Xarch_host", "-g",
]
SANITIZE_LINK_FLAGS = ["-shared-libsan"]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", "hipcc"):
        if cand and (os.path.sep not in cand or os.path.exists(cand)):
            return cand
    return "hipcc"


def _compile(src: str, obj: str, extra: tuple = ()) -> None:
    flags = [f for f in HIPCC_FLAGS if f != "-shared"] + list(extra)
    cmd = [hipcc(), *flags, f"-I{INCLUDE}", f"-I{CSRC}", "-c", os.path.join(CSRC, src), "-o", obj]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed ({res.returncode}):\n{' '.join(cmd)}\n{res.stderr}")


def build(verbose: bool = False, sanitize: bool = False) -> str:
    """Compile all HIP sources (one hipcc per source, in parallel) and link
    them into lib/libphantom_moe.so (with ``sanitize``: the host-sanitized
    lib/asan/libphantom_moe.so); returns its path."""
    from concurrent.futures import ThreadPoolExecutor

    out_dir = os.path.join(PKG_DIR, "lib", "asan") if sanitize else os.path.join(PKG_DIR, "lib")
    extra = tuple(SANITIZE_FLAGS) if sanitize else ()
    os.makedirs(out_dir, exist_ok=True)
    out = os.path.join(out_dir, "libphantom_moe.so")
    fd, tmp = tempfile.mkstemp(prefix="libphantom_moe.", suffix=".so.tmp", dir=out_dir)
    os.close(fd)
    with tempfile.TemporaryDirectory(prefix="phantom_moe_build.") as objdir:
        objs = [os.path.join(objdir, os.path.splitext(s)[0] + ".o") for s in SOURCES]
        jobs = max(1, min(len(SOURCES), len(os.sched_getaffinity(0)), 8))
        try:
            with ThreadPoolExecutor(max_workers=jobs) as pool:
                list(pool.map(_compile, SOURCES, objs, [extra] * len(SOURCES)))
            cmd = [hipcc(), *HIPCC_FLAGS, *extra, *(SANITIZE_LINK_FLAGS if sanitize else []), *objs, "-o", tmp]
            res = subprocess.run(cmd, capture_output=True, text=True)
            if res.returncode != 0:
                raise RuntimeError(f"hipcc link failed ({res.returncode}):\n{' '.join(cmd)}\n{res.stderr}")
            if verbose and res.stderr:
                print(res.stderr)
            os.replace(tmp, out)
        finally:
            if os.path.exists(tmp):
                os.unlink(tmp)
    return out


if __name__ == "__main__":
    import sys

    print(build(verbose=True, sanitize="--sanitize" in sys.argv[1:]))
