"""The runtime caller swap (phantom_moe.hf): transformers' Qwen3-MoE and
Mixtral sparse blocks routed through moe_forward, checked against the
blocks' own forward on the same (Q4_0-dequantised) weights.

Per block: the swapped forward on hidden states x must match the original
block's forward on x rounded to bf16 (the library takes bf16 activations)
within the layer tolerance (helpers.check_y).  Whole model: the logits of
the swapped model agree with the original model's to rel-L2 <= 2e-2, the
difference being the bf16 rounding of each block's input, and the greedy
next token agrees everywhere."""
import numpy as np
import pytest

torch = pytest.importorskip("torch")
transformers = pytest.importorskip("transformers")

from gguf_util import write_gguf  # noqa: E402
from helpers import check_y  # noqa: E402
from phantom_moe import gguf, hf  # noqa: E402

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def dev():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return torch.device("cuda:0")


def tiny_model(family, dev, seed=0):
    torch.manual_seed(seed)
    if family == "qwen3moe":
        cfg = transformers.Qwen3MoeConfig(
            vocab_size=128, hidden_size=256, intermediate_size=512, moe_intermediate_size=128, num_experts=8,
            num_experts_per_tok=2, norm_topk_prob=True, num_hidden_layers=2, num_attention_heads=4,
            num_key_value_heads=2, head_dim=64, max_position_embeddings=64)
        m = transformers.Qwen3MoeForCausalLM(cfg)
    else:
        cfg = transformers.MixtralConfig(
            vocab_size=128, hidden_size=256, intermediate_size=128, num_local_experts=4, num_experts_per_tok=2,
            num_hidden_layers=2, num_attention_heads=4, num_key_value_heads=2, max_position_embeddings=64)
        m = transformers.MixtralForCausalLM(cfg)
    return m.float().eval().to(dev)


def capture_block_inputs(model):
    got, hooks = {}, []
    for name, blk in hf.moe_blocks(model):
        hooks.append(blk.register_forward_pre_hook(lambda mod, args, name=name: got.__setitem__(name, args[0].detach().clone())))
    return got, hooks


def compare(model, ids):
    """Run swapped, capture block inputs, restore, compare per block and logits."""
    inputs, hooks = capture_block_inputs(model)
    with torch.no_grad():
        logits_ph = model(ids).logits.float()
    for h in hooks:
        h.remove()
    blocks = hf.moe_blocks(model)
    with torch.no_grad():
        for name, blk in blocks:
            x = inputs[name]
            y_ph = blk(x)                                   # swapped
            hf.restore_block(blk)
            y_hf = blk(x.to(torch.bfloat16).float())        # original, same bf16 input
            check_y(y_ph.cpu().numpy().reshape(-1, x.shape[-1]), y_hf.cpu().numpy().reshape(-1, x.shape[-1]), name)
        logits_hf = model(ids).logits.float()
    rel = (torch.linalg.norm(logits_ph - logits_hf) / torch.linalg.norm(logits_hf)).item()
    assert rel <= 2e-2, rel
    assert torch.equal(logits_ph.argmax(-1), logits_hf.argmax(-1))


@pytest.mark.parametrize("family", ["qwen3moe", "mixtral"])
def test_quantize_and_swap_matches_transformers(dev, family):
    model = tiny_model(family, dev)
    assert hf.quantize_and_swap(model) == 2
    ids = torch.randint(0, 128, (2, 12), generator=torch.Generator().manual_seed(1)).to(dev)
    compare(model, ids)


def test_swap_from_gguf(dev, tmp_path):
    """Expert bytes taken from a GGUF file, as the `phantom run` path would."""
    model = tiny_model("qwen3moe", dev, seed=3)
    tensors = []
    with torch.no_grad():
        for L, (_, blk) in enumerate(hf.moe_blocks(model)):
            ex = blk.experts
            E, I2, H = ex.gate_up_proj.shape
            I = I2 // 2
            gu = ex.gate_up_proj.float().cpu().numpy()
            g, u, d = hf.quantize_q4_0(gu[:, :I]), hf.quantize_q4_0(gu[:, I:]), hf.quantize_q4_0(ex.down_proj.float().cpu().numpy())
            ex.gate_up_proj.copy_(torch.from_numpy(np.concatenate([hf.dequantize_q4_0(g), hf.dequantize_q4_0(u)], 1)))
            ex.down_proj.copy_(torch.from_numpy(hf.dequantize_q4_0(d)))
            p = f"blk.{L}."
            tensors += [(p + "ffn_gate_inp.weight", 0, (E, H), blk.gate.weight.float().cpu().numpy().tobytes()),
                        (p + "ffn_gate_exps.weight", 2, (E, I, H), g.tobytes()),
                        (p + "ffn_up_exps.weight", 2, (E, I, H), u.tobytes()),
                        (p + "ffn_down_exps.weight", 2, (E, H, I), d.tobytes())]
    path = tmp_path / "tiny.gguf"
    write_gguf(path, [("general.architecture", 8, "qwen3moe"), ("qwen3moe.expert_count", 4, 8),
                      ("qwen3moe.expert_used_count", 4, 2)], tensors)
    with gguf.GGUFReader(path) as r:
        assert hf.swap_from_gguf(model, r) == 2
    ids = torch.randint(0, 128, (1, 16), generator=torch.Generator().manual_seed(2)).to(dev)
    compare(model, ids)
