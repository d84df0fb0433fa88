"""phantom_moe -- MI355X (gfx950) sparse-MoE layer for PHANTOM.

Python surface over libphantom_moe.so (C ABI in include/phantom_moe.h):

  PhantomTopKRouter   drop-in for the reference router module
                      (tests/test_moe_routing.py:43-72)
  moe_forward         router -> permute -> Q4_0 SwiGLU experts -> combine
  check_status        raise if a single-launch decode call (eager or a
                      graph replay) gave up a wait (FusedWaitError)
  route, permute      the first two stages on their own
  MoEWeights          repacked Q4_0 expert weights resident in HBM
  q4_0                GGUF Q4_0 pack / unpack / device repack
  legacy              the reference's neuron-sparse fp16 FFN ABI
                      (sparse_mlp_forward, predict_active_neurons,
                      get_sparsity_stats; include/phantom_legacy.h)
  gguf                GGUF reader; a layer's Q4_0 experts straight to HBM
  hf                  transformers MoE blocks routed through moe_forward
                      (imported on demand: ``from phantom_moe import hf``)
"""
from . import gguf, legacy, q4_0, synth
from ._lib import FusedWaitError, PhantomMoEError, check_status, set_sync_check
from .ops import MoEWeights, PreparedForward, moe_forward, permute, route
from .router import PhantomTopKRouter

__all__ = [
    "PhantomTopKRouter",
    "MoEWeights",
    "PreparedForward",
    "moe_forward",
    "route",
    "permute",
    "q4_0",
    "legacy",
    "gguf",
    "synth",
    "PhantomMoEError",
    "FusedWaitError",
    "check_status",
    "set_sync_check",
]
