"""GGUF ingestion for the MoE layer: header and tensor catalog, then the Q4_0
expert stacks of a layer copied as raw bytes to the GPU and repacked there.

Follows the reference's reader (python/phantom/loader/gguf_loader.py:133-209
header and catalog, :211-249 metadata values, :306-315 raw tensor bytes) for
the file format, and replaces the step after it: the reference dequantises
every tensor to bf16 on the host (:362-381) and, when its GPU path fails,
silently substitutes zeros (:319-325).  Here the Q4_0 bytes go to HBM
untouched and phantom_q4_0_repack lays them out for the kernels (lossless),
and every malformed input raises.

Expert tensors use llama.cpp's GGUF names: blk.{L}.ffn_gate_inp.weight
(router [E, H]), blk.{L}.ffn_{gate,up,down}_exps.weight (stacked experts,
GGUF dims [H, I, E] / [I, H, E], i.e. row-major [E, I, H] / [E, H, I]),
blk.{L}.ffn_{gate,up,down}_shexp.weight (one shared expert) and
blk.{L}.exp_probs_b.bias (router selection bias).
"""
from __future__ import annotations

import mmap
import os
import struct
from dataclasses import dataclass
from enum import IntEnum
from typing import Any, Dict, Optional, Tuple

import numpy as np

GGUF_MAGIC = 0x46554747  # "GGUF", little-endian


class GGMLType(IntEnum):
    """Tensor element types (the reference's GGUFQuantType numbering)."""
    F32 = 0
    F16 = 1
    Q4_0 = 2
    Q4_1 = 3
    Q5_0 = 6
    Q5_1 = 7
    Q8_0 = 8
    Q8_1 = 9
    Q2_K = 10
    Q3_K = 11
    Q4_K = 12
    Q5_K = 13
    Q6_K = 14
    Q8_K = 15
    I8 = 24
    I16 = 25
    I32 = 26
    I64 = 27
    F64 = 28
    BF16 = 30


# (elements per block, bytes per block)
BLOCK = {
    GGMLType.F32: (1, 4), GGMLType.F16: (1, 2), GGMLType.BF16: (1, 2), GGMLType.F64: (1, 8),
    GGMLType.I8: (1, 1), GGMLType.I16: (1, 2), GGMLType.I32: (1, 4), GGMLType.I64: (1, 8),
    GGMLType.Q4_0: (32, 18), GGMLType.Q4_1: (32, 20), GGMLType.Q5_0: (32, 22), GGMLType.Q5_1: (32, 24),
    GGMLType.Q8_0: (32, 34), GGMLType.Q8_1: (32, 40), GGMLType.Q4_K: (256, 144), GGMLType.Q5_K: (256, 176),
    GGMLType.Q6_K: (256, 210),
}

# metadata value types (the reference's _read_value codes 0..12)
_SCALAR = {0: "<B", 1: "<b", 2: "<H", 3: "<h", 4: "<I", 5: "<i", 6: "<f", 7: "<B", 10: "<Q", 11: "<q", 12: "<d"}
_STRING, _ARRAY = 8, 9


class GGUFError(ValueError):
    """A GGUF file or tensor is malformed or not what the MoE path needs."""


@dataclass
class TensorInfo:
    name: str
    n_dims: int
    shape: Tuple[int, ...]  # row-major (GGUF dims reversed)
    ggml_type: int          # raw type id (a GGMLType when known)
    offset: int             # relative to the data section
    size_bytes: Optional[int]  # None for types without a known block size


class GGUFReader:
    """Memory-mapped GGUF file: ``metadata``, ``tensors`` and raw tensor bytes.

    The header and catalog are read as gguf_loader.py:133-209 reads them
    (magic, version, counts, key/value metadata, tensor infos with dims
    reversed to row-major, data section aligned to general.alignment,
    default 32), with bounds checks on every read."""

    def __init__(self, path: str):
        self.path = os.fspath(path)
        self._f = open(self.path, "rb")
        try:
            self._mm = mmap.mmap(self._f.fileno(), 0, access=mmap.ACCESS_READ)
        except ValueError as e:  # empty file
            self._f.close()
            raise GGUFError(f"{self.path}: cannot map ({e})") from None
        try:
            self._parse()
        except Exception:
            self.close()
            raise

    def close(self):
        mm, f = getattr(self, "_mm", None), getattr(self, "_f", None)
        if mm is not None:
            mm.close()
            self._mm = None
        if f is not None:
            f.close()
            self._f = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    # -- parsing ---------------------------------------------------------
    def _take(self, fmt: str):
        n = struct.calcsize(fmt)
        if self._cur + n > len(self._mm):
            raise GGUFError(f"{self.path}: truncated at byte {self._cur} (need {n} more)")
        v = struct.unpack_from(fmt, self._mm, self._cur)
        self._cur += n
        return v if len(v) > 1 else v[0]

    def _string(self) -> str:
        n = self._take("<Q")
        if self._cur + n > len(self._mm):
            raise GGUFError(f"{self.path}: string of {n} bytes runs past the end")
        s = bytes(self._mm[self._cur:self._cur + n]).decode("utf-8", errors="replace")
        self._cur += n
        return s

    def _value(self, vtype: int, depth: int = 0) -> Any:
        if vtype in _SCALAR:
            v = self._take(_SCALAR[vtype])
            return v != 0 if vtype == 7 else v
        if vtype == _STRING:
            return self._string()
        if vtype == _ARRAY:
            if depth > 8:
                raise GGUFError(f"{self.path}: arrays nested too deep")
            et = self._take("<I")
            n = self._take("<Q")
            if et in _SCALAR and et != 7:
                size = struct.calcsize(_SCALAR[et]) * n
                if self._cur + size > len(self._mm):
                    raise GGUFError(f"{self.path}: array of {n} values runs past the end")
                out = list(struct.unpack_from(f"<{n}{_SCALAR[et][1]}", self._mm, self._cur))
                self._cur += size
                return out
            return [self._value(et, depth + 1) for _ in range(n)]
        raise GGUFError(f"{self.path}: unsupported metadata value type {vtype}")

    def _parse(self):
        self._cur = 0
        magic, self.version = self._take("<II")
        if magic != GGUF_MAGIC:
            raise GGUFError(f"{self.path}: bad magic 0x{magic:08X} (expected 0x{GGUF_MAGIC:08X})")
        if self.version < 2:
            raise GGUFError(f"{self.path}: GGUF version {self.version} has 32-bit counts; versions 2 and 3 are read")
        n_tensors, n_kv = self._take("<QQ")
        self.metadata: Dict[str, Any] = {}
        for _ in range(n_kv):
            key = self._string()
            self.metadata[key] = self._value(self._take("<I"))
        self.tensors: Dict[str, TensorInfo] = {}
        for _ in range(n_tensors):
            name = self._string()
            n_dims = self._take("<I")
            if n_dims > 8:
                raise GGUFError(f"{self.path}: tensor {name!r} has {n_dims} dims")
            dims = [self._take("<Q") for _ in range(n_dims)]
            gtype = self._take("<I")
            offset = self._take("<Q")
            shape = tuple(reversed(dims))
            n_el = int(np.prod(shape, dtype=np.int64)) if shape else 1
            size = None
            if gtype in BLOCK:
                bs, bb = BLOCK[GGMLType(gtype)]
                size = (n_el + bs - 1) // bs * bb
            self.tensors[name] = TensorInfo(name, n_dims, shape, gtype, offset, size)
        align = int(self.metadata.get("general.alignment", 32))
        if align <= 0 or align & (align - 1):
            raise GGUFError(f"{self.path}: general.alignment {align} is not a power of two")
        self.alignment = align
        self.data_offset = (self._cur + align - 1) // align * align
        for t in self.tensors.values():
            if t.size_bytes is not None and self.data_offset + t.offset + t.size_bytes > len(self._mm):
                raise GGUFError(f"{self.path}: tensor {t.name!r} runs past the end of the file")

    # -- tensor bytes ---------------------------------------------------------
    def raw(self, name: str) -> memoryview:
        """The tensor's bytes in the file (zero-copy view of the mapping)."""
        t = self.tensors.get(name)
        if t is None:
            raise GGUFError(f"{self.path}: no tensor {name!r}")
        if t.size_bytes is None:
            raise GGUFError(f"{self.path}: tensor {name!r} has element type {t.ggml_type} of unknown size")
        a = self.data_offset + t.offset
        return memoryview(self._mm)[a:a + t.size_bytes]

    def array(self, name: str) -> np.ndarray:
        """A float tensor (F32/F16/BF16) as a float32 array of its row-major shape."""
        t = self.tensors[name] if name in self.tensors else None
        buf = self.raw(name)
        if t.ggml_type == GGMLType.F32:
            a = np.frombuffer(buf, dtype="<f4")
        elif t.ggml_type == GGMLType.F16:
            a = np.frombuffer(buf, dtype="<f2").astype(np.float32)
        elif t.ggml_type == GGMLType.BF16:
            a = (np.frombuffer(buf, dtype="<u2").astype(np.uint32) << 16).view(np.float32)
        else:
            raise GGUFError(f"{self.path}: tensor {name!r} is type {t.ggml_type}, not a float type")
        return np.array(a, dtype=np.float32).reshape(t.shape)


@dataclass
class MoELayerSpec:
    """What a layer's tensors and the file's metadata say about its MoE block."""
    layer: int
    H: int
    I: int
    E: int
    top_k: int
    score: str        # "softmax" or "sigmoid"
    shared: bool
    has_router_bias: bool


def moe_layer_spec(r: GGUFReader, layer: int) -> MoELayerSpec:
    p = f"blk.{layer}."
    names = {k: p + v for k, v in (("gate", "ffn_gate_exps.weight"), ("up", "ffn_up_exps.weight"),
                                    ("down", "ffn_down_exps.weight"), ("router", "ffn_gate_inp.weight"))}
    for k, n in names.items():
        if n not in r.tensors:
            raise GGUFError(f"{r.path}: layer {layer} has no {n}")
    g, u, d, w = (r.tensors[names[k]] for k in ("gate", "up", "down", "router"))
    if len(g.shape) != 3 or g.shape != u.shape:
        raise GGUFError(f"{r.path}: {g.name} / {u.name} must both be [E, I, H], got {g.shape} / {u.shape}")
    E, I, H = g.shape
    if d.shape != (E, H, I):
        raise GGUFError(f"{r.path}: {d.name} must be [E, H, I] = {(E, H, I)}, got {d.shape}")
    if w.shape != (E, H):
        raise GGUFError(f"{r.path}: {w.name} must be [E, H] = {(E, H)}, got {w.shape}")
    for t in (g, u, d):
        if t.ggml_type != GGMLType.Q4_0:
            raise GGUFError(f"{r.path}: {t.name} is element type {t.ggml_type}; the MoE path takes Q4_0 (2)")
    arch = r.metadata.get("general.architecture", "")
    kv = r.metadata
    top_k = int(kv.get(f"{arch}.expert_used_count", 0))
    if not 1 <= top_k <= E:
        raise GGUFError(f"{r.path}: {arch}.expert_used_count = {top_k} is not in [1, {E}]")
    n_exp = kv.get(f"{arch}.expert_count")
    if n_exp is not None and int(n_exp) != E:
        raise GGUFError(f"{r.path}: {arch}.expert_count = {n_exp} but the expert stacks hold {E}")
    # llama.cpp's expert_gating_func: 1 softmax, 2 sigmoid (absent: softmax)
    gating = int(kv.get(f"{arch}.expert_gating_func", 1))
    if gating not in (1, 2):
        raise GGUFError(f"{r.path}: {arch}.expert_gating_func = {gating} is not softmax (1) or sigmoid (2)")
    sh = [p + f"ffn_{k}_shexp.weight" for k in ("gate", "up", "down")]
    n_sh = sum(n in r.tensors for n in sh)
    if n_sh not in (0, 3):
        raise GGUFError(f"{r.path}: layer {layer} has {n_sh} of the 3 shared-expert tensors")
    if n_sh == 3:
        sg, su, sd = (r.tensors[n] for n in sh)
        if sg.shape != (I, H) or su.shape != (I, H) or sd.shape != (H, I):
            raise GGUFError(f"{r.path}: shared expert shapes {sg.shape}, {su.shape}, {sd.shape} do not match "
                            f"[I, H] = {(I, H)} and [H, I]")
        for t in (sg, su, sd):
            if t.ggml_type != GGMLType.Q4_0:
                raise GGUFError(f"{r.path}: {t.name} is element type {t.ggml_type}; the MoE path takes Q4_0 (2)")
    return MoELayerSpec(layer, H, I, E, top_k, "sigmoid" if gating == 2 else "softmax", n_sh == 3,
                        p + "exp_probs_b.bias" in r.tensors)


def load_moe_layer(r: GGUFReader, layer: int, device):
    """Layer `layer`'s MoE block on `device`: returns (spec, MoEWeights,
    router_weight [E, H] fp32, router_bias [E] fp32 or None).

    Each Q4_0 stack is copied to HBM as the file holds it and repacked there;
    nothing is dequantised, and a missing or mistyped tensor raises instead of
    loading zeros."""
    import torch

    from .ops import MoEWeights

    spec = moe_layer_spec(r, layer)
    p = f"blk.{layer}."

    def dev_bytes(name):
        buf = np.frombuffer(r.raw(name), dtype=np.uint8)
        return torch.from_numpy(buf.copy()).to(device)

    gate, up, down = (dev_bytes(p + f"ffn_{k}_exps.weight") for k in ("gate", "up", "down"))
    shared = None
    if spec.shared:
        shared = tuple(dev_bytes(p + f"ffn_{k}_shexp.weight") for k in ("gate", "up", "down"))
    experts = MoEWeights.from_q4_0(gate, up, down, spec.H, spec.I, spec.E, shared=shared)
    del gate, up, down, shared
    router_w = torch.from_numpy(r.array(p + "ffn_gate_inp.weight")).to(device)
    bias = None
    if spec.has_router_bias:
        b = r.array(p + "exp_probs_b.bias").reshape(-1)
        if b.shape != (spec.E,):
            raise GGUFError(f"{r.path}: {p}exp_probs_b.bias has {b.size} values, expected {spec.E}")
        bias = torch.from_numpy(b).to(device)
    return spec, experts, router_w, bias
