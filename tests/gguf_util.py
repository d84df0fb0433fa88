"""A small GGUF v3 writer for test files (there is no GGUF model offline).

Writes the layout gguf_loader.py:133-209 reads: magic "GGUF", version,
tensor and key/value counts (u64), key/value pairs (u64-length strings, u32
value type, value), tensor infos (name, u32 n_dims, u64 dims innermost first,
u32 type, u64 offset into the data section), padding to the alignment, then
the tensor data, each tensor starting at an aligned offset.
"""
from __future__ import annotations

import struct

import numpy as np

SCALAR = {0: "<B", 1: "<b", 2: "<H", 3: "<h", 4: "<I", 5: "<i", 6: "<f", 7: "<B", 10: "<Q", 11: "<q", 12: "<d"}


def _str(s: str) -> bytes:
    b = s.encode()
    return struct.pack("<Q", len(b)) + b


def _val(vtype: int, v) -> bytes:
    if vtype in SCALAR:
        return struct.pack(SCALAR[vtype], int(v) if vtype == 7 else v)
    if vtype == 8:
        return _str(v)
    if vtype == 9:
        et, items = v
        return struct.pack("<IQ", et, len(items)) + b"".join(_val(et, x) for x in items)
    raise ValueError(vtype)


def write_gguf(path, kv, tensors, alignment=32, version=3):
    """kv: list of (key, vtype, value) -- arrays as (9, (elem_type, [values]));
    tensors: list of (name, ggml_type, row-major shape, raw bytes)."""
    head = struct.pack("<IIQQ", 0x46554747, version, len(tensors), len(kv))
    head += b"".join(_str(k) + struct.pack("<I", t) + _val(t, v) for k, t, v in kv)
    offs, off = [], 0
    for _, _, _, data in tensors:
        offs.append(off)
        off = (off + len(data) + alignment - 1) // alignment * alignment
    for (name, gt, shape, _), o in zip(tensors, offs):
        dims = list(reversed(shape))
        head += _str(name) + struct.pack("<I", len(dims)) + struct.pack(f"<{len(dims)}Q", *dims)
        head += struct.pack("<IQ", gt, o)
    pad = (-len(head)) % alignment
    with open(path, "wb") as f:
        f.write(head + b"\0" * pad)
        for (_, _, _, data), o in zip(tensors, offs):
            f.write(bytes(data))
            f.write(b"\0" * ((-len(data)) % alignment))


def moe_layer_file(path, layer_arrays, arch="qwen3moe", top_k=8, gating=None, layer=0, extra_kv=()):
    """A one-layer MoE GGUF from synth-style arrays: router_w [E, H] f32,
    gate/up [E, I, H/32, 18] and down [E, H, I/32, 18] Q4_0 bytes, optional
    shared (gate, up, down) and router bias [E] f32."""
    router_w, gate, up, down, shared, bias = layer_arrays
    E, H = router_w.shape
    I = gate.shape[1]
    kv = [("general.architecture", 8, arch), (f"{arch}.expert_count", 4, E), (f"{arch}.expert_used_count", 4, top_k),
          (f"{arch}.embedding_length", 4, H), (f"{arch}.expert_feed_forward_length", 4, I)]
    if gating is not None:
        kv.append((f"{arch}.expert_gating_func", 4, gating))
    kv += list(extra_kv)
    p = f"blk.{layer}."
    t = [(p + "ffn_gate_inp.weight", 0, (E, H), np.ascontiguousarray(router_w, np.float32).tobytes()),
         (p + "ffn_gate_exps.weight", 2, (E, I, H), np.ascontiguousarray(gate).tobytes()),
         (p + "ffn_up_exps.weight", 2, (E, I, H), np.ascontiguousarray(up).tobytes()),
         (p + "ffn_down_exps.weight", 2, (E, H, I), np.ascontiguousarray(down).tobytes())]
    if shared is not None:
        sg, su, sd = shared
        t += [(p + "ffn_gate_shexp.weight", 2, (I, H), np.ascontiguousarray(sg).tobytes()),
              (p + "ffn_up_shexp.weight", 2, (I, H), np.ascontiguousarray(su).tobytes()),
              (p + "ffn_down_shexp.weight", 2, (H, I), np.ascontiguousarray(sd).tobytes())]
    if bias is not None:
        t.append((p + "exp_probs_b.bias", 0, (E,), np.ascontiguousarray(bias, np.float32).tobytes()))
    write_gguf(path, kv, t)
