"""MI355X-native (gfx950) implementation of the uTTT per-layer hot path.

The shared fast-weight chunk update, its frozen readout and sliding-window
attention (prefill and ring-buffer decode) run as hand-written HIP kernels in
``libuttt_amd.so``; ``kernels`` is the torch-tensor front end of that library.
"""
from . import kernels  # noqa: F401
