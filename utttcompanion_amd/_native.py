"""ctypes binding of libuttt_amd.so (the C ABI declared in include/uttt_amd.h).

The library is loaded lazily on first use and there is no fallback: a missing or
stale library raises ``RuntimeError`` naming the build command.
"""
from __future__ import annotations

import ctypes as C
import os
import threading

from .build import HEADER_PATH, LIB_PATH


def _header_abi_version(path: str = HEADER_PATH) -> int:
    """UTTT_ABI_VERSION as include/uttt_amd.h defines it (the library is built from that header)."""
    import re
    with open(path, "r", encoding="utf-8") as fh:
        m = re.search(r"^#define UTTT_ABI_VERSION (\d+)$", fh.read(), re.M)
    if m is None:
        raise RuntimeError(f"{path} defines no UTTT_ABI_VERSION")
    return int(m.group(1))


ABI_VERSION = _header_abi_version()
MAX_CHAIN = 64
MAX_UPDATE_TOKENS = 512  # UTTT_MAX_UPDATE_TOKENS: longest chunk one uttt_chunk_update writes
DTYPE_F32 = 0
DTYPE_BF16 = 1
UPDATE_PHASES = 5

_P = C.c_void_p
_I64 = C.c_int64
_I32 = C.c_int32
_F = C.c_float


class ChunkUpdateArgs(C.Structure):
    _fields_ = [
        ("batch", _I64), ("tokens", _I64), ("d_model", _I64), ("d_ff", _I64),
        ("act_dtype", _I32), ("normalize_by_dim", _I32),
        ("momentum_beta", _F), ("max_inner_grad_norm", _F), ("eps", _F),
        ("q", _P), ("q_row_stride", _I64),
        ("k", _P), ("k_row_stride", _I64),
        ("v", _P), ("v_row_stride", _I64),
        ("eta", _P), ("eta_row_stride", _I64),
        ("alpha", _P), ("alpha_row_stride", _I64),
        ("token_mask", _P), ("mask_row_stride", _I64),
        ("w_up", _P), ("w_gate", _P), ("w_down", _P),
        ("s_up", _P), ("s_gate", _P), ("s_down", _P),
        ("r_up", _P), ("r_gate", _P), ("r_down", _P), ("r_row_stride", _I64),
        ("ln_weight", _P), ("ln_bias", _P),
        ("w_up_out", _P), ("w_gate_out", _P), ("w_down_out", _P),
        ("s_up_out", _P), ("s_gate_out", _P), ("s_down_out", _P),
        ("out", _P), ("out_row_stride", _I64),
        ("surprise", _P), ("row_loss", _P), ("min_row_surprise", _F),
    ]


class LayerUpdateArgs(C.Structure):
    _fields_ = [
        ("batch", _I64), ("tokens", _I64), ("d_model", _I64), ("d_ff", _I64), ("chunk_size", _I64),
        ("normalize_by_dim", _I32),
        ("momentum_beta", _F), ("max_inner_grad_norm", _F), ("eps", _F),
        ("q", _P), ("k", _P), ("v", _P),
        ("eta", _P), ("alpha", _P), ("token_mask", _P),
        ("w_up", _P), ("w_gate", _P), ("w_down", _P),
        ("s_up", _P), ("s_gate", _P), ("s_down", _P),
        ("ln_weight", _P), ("ln_bias", _P),
        ("w_up_out", _P), ("w_gate_out", _P), ("w_down_out", _P),
        ("s_up_out", _P), ("s_gate_out", _P), ("s_down_out", _P),
        ("out", _P),
        ("surprise", _P),
        ("error_word", _P), ("force_timeout", _I32),
    ]


class LinearArgs(C.Structure):
    _fields_ = [
        ("m", _I64), ("n", _I64), ("k", _I64), ("act_dtype", _I32),
        ("x", _P), ("x_row_stride", _I64),
        ("w", _P), ("w_row_stride", _I64),
        ("residual", _P), ("residual_row_stride", _I64),
        ("out", _P), ("out_row_stride", _I64),
        ("workspace", _P), ("workspace_bytes", C.c_size_t),
    ]


class ChunkChainArgs(C.Structure):
    _fields_ = [
        ("batch", _I64), ("layers", _I64), ("tokens", _I64), ("d_model", _I64), ("d_ff", _I64),
        ("act_dtype", _I32), ("normalize_by_dim", _I32),
        ("momentum_beta", _F), ("max_inner_grad_norm", _F), ("eps", _F), ("min_row_surprise", _F),
        ("k", _P * 64), ("v", _P * 64), ("kv_row_stride", _I64),
        ("eta", _P * 64), ("alpha", _P * 64), ("ea_row_stride", _I64),
        ("token_mask", _P), ("mask_row_stride", _I64),
        ("w_up", _P), ("w_gate", _P), ("w_down", _P),
        ("s_up", _P), ("s_gate", _P), ("s_down", _P),
        ("ln_weight", _P), ("ln_bias", _P),
        ("w_up_copy", _P), ("w_gate_copy", _P), ("w_down_copy", _P),
        ("s_up_copy", _P), ("s_gate_copy", _P), ("s_down_copy", _P),
        ("surprise", _P), ("row_loss", _P),
        ("w_products_given", _I32),
    ]


class ProjEpilogueArgs(C.Structure):
    _fields_ = [
        ("rows", _I64), ("d_model", _I64), ("act_dtype", _I32),
        ("eps", _F), ("inner_lr", _F), ("weight_decay", _F),
        ("y", _P), ("y_row_stride", _I64),
        ("q_weight", _P), ("k_weight", _P),
        ("q", _P), ("k", _P), ("v", _P), ("out_row_stride", _I64),
        ("eta", _P), ("alpha", _P),
        ("x", _P), ("x_row_stride", _I64), ("x_eps", _F),
        ("eta_alpha_bias", _P),
    ]


class SkinnyLinearArgs(C.Structure):
    _fields_ = [
        ("m", _I64), ("n", _I64), ("k", _I64), ("act_dtype", _I32), ("x_eps", _F),
        ("x", _P), ("x_row_stride", _I64),
        ("w", _P), ("w_row_stride", _I64),
        ("residual", _P), ("residual_row_stride", _I64),
        ("out", _P), ("out_row_stride", _I64),
    ]


class GreedyArgs(C.Structure):
    _fields_ = [
        ("rows", _I64), ("vocab", _I64), ("dtype", _I32), ("n_banned", _I32),
        ("banned", _I32 * 8), ("active_limit", _I64),
        ("logits", _P), ("row_stride", _I64),
        ("out", _P), ("advance", _P),
    ]


class ReadoutArgs(C.Structure):
    _fields_ = [
        ("batch", _I64), ("tokens", _I64), ("d_model", _I64), ("d_ff", _I64),
        ("act_dtype", _I32), ("w_dtype", _I32), ("eps", _F),
        ("x", _P), ("x_row_stride", _I64),
        ("w_up", _P), ("w_gate", _P), ("w_down", _P), ("w_row_stride", _I64),
        ("ln_weight", _P), ("ln_bias", _P),
        ("out", _P), ("out_row_stride", _I64),
        ("keys", _P), ("keys_row_stride", _I64),
        ("key_up_out", _P), ("key_gate_out", _P),
        ("x_norm_weight", _P), ("x_norm_eps", _F),
        ("row_counters", _P),
        ("sweep_reverse", _I32),
    ]


class RopeAppendArgs(C.Structure):
    _fields_ = [
        ("batch", _I64), ("tokens", _I64), ("n_heads", _I64), ("n_kv_heads", _I64), ("head_dim", _I64),
        ("act_dtype", _I32),
        ("start_pos", _I64), ("table_len", _I64),
        ("cos_table", _P), ("sin_table", _P),
        ("q", _P), ("q_stride_b", _I64), ("q_stride_t", _I64), ("q_stride_h", _I64),
        ("k", _P), ("k_stride_b", _I64), ("k_stride_t", _I64), ("k_stride_h", _I64),
        ("v", _P), ("v_stride_b", _I64), ("v_stride_t", _I64), ("v_stride_h", _I64),
        ("k_cache", _P), ("v_cache", _P), ("kv_stride_b", _I64), ("kv_stride_h", _I64), ("kv_stride_t", _I64),
        ("kv_offset", _I64),
        ("x", _P), ("x_stride_b", _I64), ("x_stride_t", _I64), ("x_dim", _I64), ("x_eps", _F),
    ]


class SwaPrefillArgs(C.Structure):
    _fields_ = [
        ("batch", _I64), ("n_heads", _I64), ("n_kv_heads", _I64), ("q_len", _I64), ("kv_len", _I64),
        ("head_dim", _I64), ("q_offset", _I64), ("window", _I64),
        ("act_dtype", _I32), ("scale", _F),
        ("q", _P), ("q_stride_b", _I64), ("q_stride_h", _I64), ("q_stride_t", _I64),
        ("k", _P), ("k_stride_b", _I64), ("k_stride_h", _I64), ("k_stride_t", _I64),
        ("v", _P), ("v_stride_b", _I64), ("v_stride_h", _I64), ("v_stride_t", _I64),
        ("out", _P), ("o_stride_b", _I64), ("o_stride_h", _I64), ("o_stride_t", _I64),
        ("workspace", _P), ("workspace_bytes", C.c_size_t),
    ]


class SwaDecodeArgs(C.Structure):
    _fields_ = [
        ("n_req", _I64), ("n_heads", _I64), ("n_kv_heads", _I64), ("head_dim", _I64), ("window", _I64),
        ("act_dtype", _I32), ("scale", _F),
        ("positions", _P),
        ("cos_table", _P), ("sin_table", _P), ("table_len", _I64),
        ("q", _P), ("q_stride_n", _I64),
        ("k_new", _P), ("v_new", _P), ("kv_new_stride_n", _I64),
        ("k_ring", _P), ("v_ring", _P), ("ring_stride_n", _I64),
        ("out", _P), ("o_stride_n", _I64),
        ("workspace", _P), ("workspace_bytes", C.c_size_t),
    ]


class ElasticPullArgs(C.Structure):
    _fields_ = [
        ("batch", _I64), ("d_model", _I64), ("d_ff", _I64),
        ("anchor_lambda", _F), ("max_drift_ratio", _F),
        ("w_up", _P), ("w_gate", _P), ("w_down", _P),
        ("w0_up", _P), ("w0_gate", _P), ("w0_down", _P),
        ("out_up", _P), ("out_gate", _P), ("out_down", _P),
    ]


# exported symbol -> (restype, argtypes)
class PrefillLayerCalls(C.Structure):
    _fields_ = [
        ("qkv", LinearArgs), ("rope", RopeAppendArgs), ("attn", SwaPrefillArgs), ("attn_out", LinearArgs),
        ("proj", LinearArgs), ("epilogue", ProjEpilogueArgs), ("readout", ReadoutArgs),
        ("readout_workspace", _P), ("readout_workspace_bytes", C.c_size_t), ("uttt_out", LinearArgs),
    ]


class PrefillChunkArgs(C.Structure):
    _fields_ = [
        ("n_layers", _I32), ("layers", C.POINTER(PrefillLayerCalls)), ("chain", C.POINTER(ChunkChainArgs)),
        ("chain_workspace", _P), ("chain_workspace_bytes", C.c_size_t),
        ("start_pos", _I64), ("kv_offset", _I64),
        ("token_mask", _P), ("mask_row_stride", _I64), ("surprise", _P), ("defer_join", _I32),
        ("events", C.POINTER(_P)), ("n_events", _I32), ("wait_event", _P),
    ]


SIGNATURES = {
    "uttt_last_error": (C.c_char_p, []),
    "uttt_abi_version": (C.c_int, []),
    "uttt_chunk_update_workspace": (C.c_size_t, [_I64, _I64, _I64, _I32]),
    "uttt_chunk_update_workspace_tokens": (C.c_size_t, [_I64, _I64, _I64, _I64, _I32]),
    "uttt_chunk_update": (C.c_int, [C.POINTER(ChunkUpdateArgs), _P, C.c_size_t, _P]),
    "uttt_chunk_update_phase": (C.c_int, [C.POINTER(ChunkUpdateArgs), _P, C.c_size_t, _I32, _P]),
    "uttt_chunk_update_noalloc": (C.c_int, [C.POINTER(ChunkUpdateArgs), _P]),
    "uttt_layer_update_resident_supported": (C.c_int, [_I64, _I64, _I64]),
    "uttt_layer_update_resident_workspace": (C.c_size_t, [_I64, _I64]),
    "uttt_layer_update_resident_flag_offset": (C.c_size_t, [_I64, _I64]),
    "uttt_layer_update_resident": (C.c_int, [C.POINTER(LayerUpdateArgs), _P, C.c_size_t, _P]),
    "uttt_linear": (C.c_int, [C.POINTER(LinearArgs), _P]),
    "uttt_linear_workspace": (C.c_size_t, [_I64, _I64, _I64]),
    "uttt_prefill_chunk": (C.c_int, [C.POINTER(PrefillChunkArgs), _P, _P]),
    "uttt_events_create": (C.c_int, [_I32, C.POINTER(_P)]),
    "uttt_events_destroy": (C.c_int, [_I32, C.POINTER(_P)]),
    "uttt_stream_wait_event": (C.c_int, [_P, _P]),
    "uttt_chunk_chain_workspace": (C.c_size_t, [_I64, _I64, _I64, _I64, _I32]),
    "uttt_chunk_chain": (C.c_int, [C.POINTER(ChunkChainArgs), _P, C.c_size_t, _P]),
    "uttt_chunk_chain_stage": (C.c_int, [C.POINTER(ChunkChainArgs), _P, C.c_size_t, _I32, _P]),
    "uttt_chunk_chain_stage_part": (C.c_int, [C.POINTER(ChunkChainArgs), _P, C.c_size_t, _I32, _I32, _P]),
    "uttt_chunk_chain_stage_launch": (C.c_int, [C.POINTER(ChunkChainArgs), _P, C.c_size_t, _I32, _I32, _I32, _I32,
                                                C.POINTER(C.c_char_p), _I32, C.POINTER(_I32), _P]),
    "uttt_chunk_chain_w_products": (C.c_int, [_I64, _I64, _I64, _I64, _I32, _I32, C.POINTER(C.c_size_t),
                                              C.POINTER(C.c_size_t)]),
    "uttt_proj_epilogue": (C.c_int, [C.POINTER(ProjEpilogueArgs), _P]),
    "uttt_readout_workspace": (C.c_size_t, [_I64, _I64, _I64, _I64, _I32]),
    "uttt_swiglu_readout": (C.c_int, [C.POINTER(ReadoutArgs), _P, C.c_size_t, _P]),
    "uttt_rope_kv_append": (C.c_int, [C.POINTER(RopeAppendArgs), _P]),
    "uttt_swa_prefill_workspace": (C.c_size_t, [_I64, _I64, _I64, _I64, _I64, _I64]),
    "uttt_swa_prefill": (C.c_int, [C.POINTER(SwaPrefillArgs), _P]),
    "uttt_swa_decode_workspace": (C.c_size_t, [_I64, _I64, _I64, _I64, _I64]),
    "uttt_swa_decode": (C.c_int, [C.POINTER(SwaDecodeArgs), _P]),
    "uttt_elastic_pull_workspace": (C.c_size_t, [_I64]),
    "uttt_elastic_pull": (C.c_int, [C.POINTER(ElasticPullArgs), _P, C.c_size_t, _P]),
    "uttt_fast_weight_drift": (C.c_int, [_I64, _I64, _I64, _P, _P, _P, _P, _P, _P, _P, _P, C.c_size_t, _P]),
    "uttt_skinny_linear": (C.c_int, [C.POINTER(SkinnyLinearArgs), _P]),
    "uttt_greedy_select": (C.c_int, [C.POINTER(GreedyArgs), _P]),
}

_lib = None
_lock = threading.Lock()


def load_library(path: str = LIB_PATH) -> C.CDLL:
    """Load (once) and type the HIP library; raise if it is absent or of another ABI."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not os.path.exists(path):
            raise RuntimeError(
                f"{path} is missing: the uTTT HIP kernels are not built "
                "(run `python -m utttcompanion_amd.build`); there is no fallback path")
        lib = C.CDLL(path)
        for name, (res, argt) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = argt
        version = lib.uttt_abi_version()
        if version != ABI_VERSION:
            raise RuntimeError(f"{path} has ABI version {version}, expected {ABI_VERSION}: rebuild it")
        _lib = lib
        return lib


def check(status: int, what: str) -> None:
    if status != 0:
        msg = load_library().uttt_last_error().decode(errors="replace")
        raise RuntimeError(f"{what} failed (status {status}): {msg}")
