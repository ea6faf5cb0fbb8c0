"""Host-side mirror of the reference's ``ane`` engine package over the HIP C-ABI.

``ane.Open(Options)`` / ``Engine.Step`` / ``Engine.EvalLogits`` / ``Flush`` /
``SetLR`` / ``State`` / ``LoadState`` / ``Close`` keep the names, argument
meaning and error behaviour of ane/engine.go; everything computes on the GPU
through libane_hip.so (no CPU fallback: a missing library raises).
"""
from .config import (Config, stories110m, tiny, decode_gqa, tiny_decode, is_ve_layer, param_layout, param_count,  # noqa: F401
                     views, init_params, make_tokens, VE_GATE_CHANNELS)
from .engine import Options, Open, Engine, EngineError  # noqa: F401
from .decode import Decoder  # noqa: F401
