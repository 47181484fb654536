"""MI355X-native (gfx950) implementation of the uTTT per-layer hot path.

The shared fast-weight chunk update, its frozen readout, the elastic pull and
sliding-window attention (prefill and ring-buffer decode) run as hand-written HIP
kernels in ``libuttt_amd.so``.  ``kernels`` is the torch-tensor front end of that
library; ``layer`` and ``model`` mirror the reference's module API
(``model/uttt_layer.py`` / ``model/uttt_model.py``) on top of it.
"""
from .layer import (  # noqa: F401
    FastWeightState,
    RMSNorm,
    RotaryEmbedding,
    SharedFastWeightPool,
    SlidingWindowAttention,
    apply_rope,
    fused_chunk_ttt_step,
    fused_slow_projections,
    swiglu_fast_forward,
    uTTTBlock,
    uTTTLayer,
)
from .model import uTTTConfig, uTTTModel, uTTTModelOutput  # noqa: F401

__all__ = [
    "FastWeightState", "RMSNorm", "RotaryEmbedding", "SharedFastWeightPool", "SlidingWindowAttention",
    "apply_rope", "fused_chunk_ttt_step", "fused_slow_projections", "swiglu_fast_forward", "uTTTBlock",
    "uTTTLayer", "uTTTConfig", "uTTTModel", "uTTTModelOutput",
]
