"""GGUF ingestion (phantom_moe.gguf): the header and catalog parse against
hand-assembled bytes in the read order of gguf_loader.py:133-249, error
handling, MoE layer validation, and (GPU) a layer loaded from a GGUF file
matching the oracle on the same bytes."""
import struct

import numpy as np
import pytest

from gguf_util import moe_layer_file, write_gguf
from phantom_moe import gguf, synth


def _s(x: str) -> bytes:
    b = x.encode()
    return struct.pack("<Q", len(b)) + b


def test_parse_hand_assembled_header(tmp_path):
    """Every metadata value type 0..12, nested arrays, dims reversed to
    row-major, sizes from the block table, a 64-byte data alignment."""
    kv = b""
    kv += _s("u8") + struct.pack("<IB", 0, 200)
    kv += _s("i8") + struct.pack("<Ib", 1, -5)
    kv += _s("u16") + struct.pack("<IH", 2, 65000)
    kv += _s("i16") + struct.pack("<Ih", 3, -300)
    kv += _s("u32") + struct.pack("<II", 4, 4000000000)
    kv += _s("i32") + struct.pack("<Ii", 5, -7)
    kv += _s("f32") + struct.pack("<If", 6, 0.25)
    kv += _s("bool") + struct.pack("<IB", 7, 1)
    kv += _s("str") + struct.pack("<I", 8) + _s("qwen3moe")
    kv += _s("arr") + struct.pack("<IIQ", 9, 5, 3) + struct.pack("<3i", 1, -2, 3)
    kv += _s("strs") + struct.pack("<IIQ", 9, 8, 2) + _s("a") + _s("bc")
    kv += _s("nested") + struct.pack("<IIQ", 9, 9, 2) + struct.pack("<IQ", 4, 1) + struct.pack("<I", 9) \
        + struct.pack("<IQ", 7, 2) + struct.pack("<2B", 0, 1)
    kv += _s("u64") + struct.pack("<IQ", 10, 2 ** 40)
    kv += _s("i64") + struct.pack("<Iq", 11, -(2 ** 40))
    kv += _s("f64") + struct.pack("<Id", 12, -1.5)
    kv += _s("general.alignment") + struct.pack("<II", 4, 64)
    n_kv = 16
    ti = _s("blk.0.ffn_gate_exps.weight") + struct.pack("<I3QIQ", 3, 64, 16, 4, 2, 0)  # dims [H, I, E]
    ti += _s("tok") + struct.pack("<I2QIQ", 2, 8, 3, 0, 64 * 1024)                    # f32 [3, 8]
    ti += _s("odd") + struct.pack("<I1QIQ", 1, 10, 99, 64 * 1024 + 128)                # unknown type
    head = struct.pack("<IIQQ", 0x46554747, 3, 3, n_kv) + kv + ti
    data_off = (len(head) + 63) // 64 * 64
    body = bytearray(64 * 1024 + 256)
    q = np.arange(4 * 16 * 2 * 18, dtype=np.uint32).astype(np.uint8)  # 4*16 rows x 2 blocks
    body[: q.size] = q.tobytes()
    body[64 * 1024: 64 * 1024 + 96] = np.arange(24, dtype=np.float32).tobytes()
    p = tmp_path / "h.gguf"
    p.write_bytes(head + b"\0" * (data_off - len(head)) + bytes(body))

    with gguf.GGUFReader(p) as r:
        m = r.metadata
        assert r.version == 3
        assert (m["u8"], m["i8"], m["u16"], m["i16"], m["u32"], m["i32"]) == (200, -5, 65000, -300, 4000000000, -7)
        assert m["f32"] == 0.25 and m["bool"] is True and m["str"] == "qwen3moe"
        assert m["arr"] == [1, -2, 3] and m["strs"] == ["a", "bc"] and m["nested"] == [[9], [False, True]]
        assert m["u64"] == 2 ** 40 and m["i64"] == -(2 ** 40) and m["f64"] == -1.5
        assert r.alignment == 64 and r.data_offset == data_off
        t = r.tensors["blk.0.ffn_gate_exps.weight"]
        assert t.shape == (4, 16, 64) and t.ggml_type == gguf.GGMLType.Q4_0 and t.offset == 0
        assert t.size_bytes == 4 * 16 * 64 // 32 * 18
        np.testing.assert_array_equal(np.frombuffer(r.raw(t.name), np.uint8), q)
        np.testing.assert_array_equal(r.array("tok"), np.arange(24, dtype=np.float32).reshape(3, 8))
        assert r.tensors["odd"].size_bytes is None
        with pytest.raises(gguf.GGUFError, match="unknown size"):
            r.raw("odd")


def test_writer_roundtrip_and_default_alignment(tmp_path):
    rng = np.random.default_rng(0)
    a = rng.standard_normal((5, 7)).astype(np.float16)
    b = rng.integers(0, 256, 3 * 18, dtype=np.uint8)
    p = tmp_path / "w.gguf"
    write_gguf(p, [("general.architecture", 8, "x"), ("v", 9, (6, [1.0, 2.5]))],
               [("a", 1, (5, 7), a.tobytes()), ("b", 2, (96,), b.tobytes())])
    with gguf.GGUFReader(p) as r:
        assert r.alignment == 32 and r.data_offset % 32 == 0
        assert r.metadata["v"] == [1.0, 2.5]
        np.testing.assert_array_equal(r.array("a"), a.astype(np.float32))
        assert r.tensors["b"].offset % 32 == 0
        np.testing.assert_array_equal(np.frombuffer(r.raw("b"), np.uint8), b)


def test_malformed_files_raise(tmp_path):
    good = tmp_path / "g.gguf"
    write_gguf(good, [("k", 4, 1)], [("t", 0, (4,), np.zeros(4, np.float32).tobytes())])
    raw = good.read_bytes()
    cases = {
        "magic": b"GGUX" + raw[4:],
        "version": raw[:4] + struct.pack("<I", 1) + raw[8:],
        "truncated": raw[:30],
        "past_end": raw[:-20],  # the 16 data bytes are followed by 16 of padding
        "empty": b"",
    }
    for name, data in cases.items():
        p = tmp_path / f"{name}.gguf"
        p.write_bytes(data)
        with pytest.raises(gguf.GGUFError):
            gguf.GGUFReader(p)
    bad_type = tmp_path / "vt.gguf"
    bad_type.write_bytes(struct.pack("<IIQQ", 0x46554747, 3, 0, 1) + _s("k") + struct.pack("<I", 13) + b"\0" * 16)
    with pytest.raises(gguf.GGUFError, match="value type 13"):
        gguf.GGUFReader(bad_type)
    bad_align = tmp_path / "al.gguf"
    write_gguf(bad_align, [("general.alignment", 4, 48)], [], alignment=16)
    with pytest.raises(gguf.GGUFError, match="power of two"):
        gguf.GGUFReader(bad_align)


def _small_layer(shared=False, zipf=0.0, score="softmax"):
    cfg = synth.MoEConfig("g", 256, 128, 8, 2, 4, score=score, shared=shared, zipf=zipf)
    L = synth.host_layer(cfg)
    return cfg, L, (L.router_w, L.gate, L.up, L.down, L.shared, L.router_bias)


def test_moe_layer_spec_and_validation(tmp_path):
    cfg, L, arrays = _small_layer(shared=True, zipf=1.1)
    p = tmp_path / "m.gguf"
    moe_layer_file(p, arrays, arch="deepseek2", top_k=2, gating=2, layer=3)
    with gguf.GGUFReader(p) as r:
        s = gguf.moe_layer_spec(r, 3)
        assert (s.H, s.I, s.E, s.top_k, s.score, s.shared, s.has_router_bias) == (256, 128, 8, 2, "sigmoid", True, True)
        with pytest.raises(gguf.GGUFError, match="no blk.0"):
            gguf.moe_layer_spec(r, 0)
    # experts stored as F16 instead of Q4_0: refused, not zero-filled
    p2 = tmp_path / "f16.gguf"
    E, H, I = 8, 256, 128
    write_gguf(p2, [("general.architecture", 8, "qwen3moe"), ("qwen3moe.expert_used_count", 4, 2)], [
        ("blk.0.ffn_gate_inp.weight", 0, (E, H), np.zeros((E, H), np.float32).tobytes()),
        ("blk.0.ffn_gate_exps.weight", 1, (E, I, H), np.zeros(E * I * H, np.float16).tobytes()),
        ("blk.0.ffn_up_exps.weight", 2, (E, I, H), L.up.tobytes()),
        ("blk.0.ffn_down_exps.weight", 2, (E, H, I), L.down.tobytes())])
    with gguf.GGUFReader(p2) as r:
        with pytest.raises(gguf.GGUFError, match="takes Q4_0"):
            gguf.moe_layer_spec(r, 0)
    # top-k outside [1, E], and a partial shared expert
    p3 = tmp_path / "k.gguf"
    moe_layer_file(p3, arrays[:4] + (None, None), top_k=9)
    with gguf.GGUFReader(p3) as r:
        with pytest.raises(gguf.GGUFError, match="expert_used_count"):
            gguf.moe_layer_spec(r, 0)
    p4 = tmp_path / "sh.gguf"
    write_gguf(p4, [("general.architecture", 8, "qwen3moe"), ("qwen3moe.expert_used_count", 4, 2)], [
        ("blk.0.ffn_gate_inp.weight", 0, (E, H), L.router_w.tobytes()),
        ("blk.0.ffn_gate_exps.weight", 2, (E, I, H), L.gate.tobytes()),
        ("blk.0.ffn_up_exps.weight", 2, (E, I, H), L.up.tobytes()),
        ("blk.0.ffn_down_exps.weight", 2, (E, H, I), L.down.tobytes()),
        ("blk.0.ffn_gate_shexp.weight", 2, (I, H), L.shared[0].tobytes())])
    with gguf.GGUFReader(p4) as r:
        with pytest.raises(gguf.GGUFError, match="1 of the 3 shared"):
            gguf.moe_layer_spec(r, 0)


@pytest.mark.gpu
@pytest.mark.parametrize("shared,zipf,score", [(False, 0.0, "softmax"), (True, 1.1, "sigmoid")])
def test_gpu_layer_from_gguf_matches_oracle(tmp_path, shared, zipf, score):
    torch = pytest.importorskip("torch")
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    import phantom_moe
    from helpers import check_y
    from oracle import oracle
    from phantom_moe import q4_0

    dev = torch.device("cuda:0")
    cfg, L, arrays = _small_layer(shared, zipf, score)
    p = tmp_path / "layer.gguf"
    moe_layer_file(p, arrays, arch="deepseek2" if shared else "qwen3moe", top_k=cfg.k,
                   gating=2 if score == "sigmoid" else None)
    with gguf.GGUFReader(p) as r:
        spec, experts, rw, rb = gguf.load_moe_layer(r, 0, dev)
    assert spec.score == score and spec.shared == shared and (rb is not None) == bool(zipf)
    # the repacked stacks hold exactly the file's bytes
    back = q4_0.unrepack(experts.gate_nib, experts.gate_scale, cfg.I, cfg.H, n_mats=cfg.E)
    np.testing.assert_array_equal(back.cpu().numpy(), L.gate.reshape(-1))
    xb = synth.activations(16, cfg.H, seed=5)
    x = torch.from_numpy(xb.view(np.int16)).view(torch.bfloat16).to(dev)
    y = phantom_moe.moe_forward(x, rw, experts, spec.top_k, spec.score, rb)
    y_ref, idx_ref, _ = oracle.moe_forward(xb, L.router_w, L.gate, L.up, L.down, cfg.k, cfg.score_mode,
                                           router_bias=L.router_bias, shared=L.shared)
    check_y(y.cpu().numpy(), y_ref, "gguf layer")
