"""Torch-tensor front end of the HIP kernels in libuttt_amd.so.

Each function validates shapes, dtypes and devices the way the reference modules
do (``ValueError``), hands raw device pointers, strides and the current HIP
stream to the C ABI, and raises ``RuntimeError`` when the library reports an
error.  Nothing here computes on the host: CPU tensors are rejected.  The HIP
path is forward-only, so inputs that require grad under grad mode are rejected
as well (the reference's update is differentiable; meta-training stays on the
reference's PyTorch path).
"""
from __future__ import annotations

import ctypes as C
import math
from typing import Optional, Sequence, Tuple

import torch

from . import _native as N

Tensor = torch.Tensor
_ACT = {torch.float32: N.DTYPE_F32, torch.bfloat16: N.DTYPE_BF16}


def _act_code(dtype: torch.dtype) -> int:
    try:
        return _ACT[dtype]
    except KeyError:
        raise ValueError(f"the uTTT HIP kernels take float32 or bfloat16 activations, got {dtype}") from None


def _require_device(device: torch.device, *tensors: Optional[Tensor]) -> None:
    if device.type != "cuda":
        raise ValueError("the uTTT HIP kernels need GPU (ROCm) tensors; there is no CPU path")
    for t in tensors:
        if t is not None and t.device != device:
            raise ValueError(f"all tensors must be on {device}, found one on {t.device}")


def _forward_only(*tensors: Optional[Tensor]) -> None:
    if torch.is_grad_enabled() and any(t is not None and t.requires_grad for t in tensors):
        raise ValueError("the HIP fast-weight path is forward-only: run it under torch.no_grad() "
                         "or pass tensors that do not require grad")


def _p(t: Optional[Tensor]) -> Optional[int]:
    return None if t is None else t.data_ptr()


def _stream(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def _rows(x: Tensor) -> Tensor:
    """(B, T, D) with feature stride 1, token stride D and a 16-byte aligned base and row
    stride (the kernels read activations with 16-byte vector loads)."""
    vec = 16 // x.element_size()
    if (x.stride(2) != 1 or (x.shape[1] > 1 and x.stride(1) != x.shape[2])
            or x.data_ptr() % 16 or (x.shape[0] > 1 and x.stride(0) % vec)):
        x = x.contiguous()
    return x


def _row_vector(x: Tensor, act: torch.dtype) -> Tensor:
    """(B, T) or (B, T, 1) per-token scalars with token stride 1, in ``act``."""
    if x.dim() == 3:
        x = x[..., 0]
    if x.dtype != act:
        x = x.to(act)
    if x.shape[1] > 1 and x.stride(1) != 1:
        x = x.contiguous()
    return x


def _per_token(x: Tensor, bsz: int, tokens: int, name: str) -> Tensor:
    """eta / alpha as one value per (row, token): (B, C) or (B, C, 1) pass through; anything the
    reference broadcasts against (B, C, 1) (model/uttt_layer.py:371-378, :501-511: a per-row
    (B, 1, 1), a shared (1, 1, 1), a (B, 1) ...) is expanded into a new (B, C) tensor, since the
    kernels read C entries per row; other shapes raise ``ValueError``."""
    if tuple(x.shape) in ((bsz, tokens), (bsz, tokens, 1)):
        return x
    try:
        if x.dim() > 3 or (x.dim() == 3 and x.shape[-1] != 1):
            raise RuntimeError
        y = x if x.dim() < 3 else x[..., 0]
        return torch.broadcast_to(y, (bsz, tokens)).contiguous()
    except RuntimeError:
        raise ValueError(f"{name} must broadcast to ({bsz}, {tokens}, 1), got {tuple(x.shape)}") from None


def _state(t: Tensor, name: str) -> Tensor:
    if t.dtype == torch.float64:
        raise ValueError(f"{name}: float64 fast-weight state is not supported by the HIP path")
    if t.dtype != torch.float32:
        t = t.float()  # exact widening of a bf16/fp16 state to the fp32 master
    t = t.contiguous()
    return t if t.data_ptr() % 16 == 0 else t.clone()


def _read_weight(t: Tensor, bsz: int, name: str, keep_bf16: bool = False) -> Tuple[Tensor, int]:
    """A read-only weight of shape (B|1, r, c): returns (tensor, row stride in elements).
    fp32 is the default; ``keep_bf16`` passes bf16 read copies through unchanged."""
    if t.dtype == torch.float64:
        raise ValueError(f"{name}: float64 weights are not supported by the HIP path")
    if t.dtype != torch.float32 and not (keep_bf16 and t.dtype == torch.bfloat16):
        t = t.float()
    shared = t.shape[0] == 1 or t.stride(0) == 0
    if shared:
        base = t[:1]
        if not base.is_contiguous() or base.data_ptr() % 16:
            base = base.contiguous() if not base.is_contiguous() else base.clone()
        return base, 0
    if t.shape[0] != bsz:
        raise ValueError(f"{name}: batch {t.shape[0]} does not match {bsz}")
    t = t.contiguous()
    return (t if t.data_ptr() % 16 == 0 else t.clone()), t.shape[1] * t.shape[2]


# ---------------------------------------------------------------------------
# fast-weight chunk update (reference fused_chunk_ttt_step, model/uttt_layer.py:414-534)
# ---------------------------------------------------------------------------

# Longest chunk the layer chain (uttt_chunk_chain) takes: its Gram blocks and token slabs are one
# 64-token tile per layer.  Longer write chunks run one uttt_chunk_update per layer.
MAX_CHAIN_CHUNK = 64


class PreparedUpdate:
    """A validated ``uttt_chunk_update`` call: the argument block, the tensors it points to
    and the result tuple.  ``launch()`` enqueues the whole update on the current stream;
    ``launch(phase)`` enqueues one of its ``N.UPDATE_PHASES`` stream-ordered phases."""

    def __init__(self, args, keep, workspace, result, device):
        self.args, self._keep, self.workspace, self.result, self.device = args, keep, workspace, result, device

    def launch(self, phase: Optional[int] = None) -> Tuple[Tensor, ...]:
        lib = N.load_library()
        with torch.cuda.device(self.device):
            if phase is None:
                rc = lib.uttt_chunk_update(C.byref(self.args), _p(self.workspace), self.workspace.numel(),
                                           _stream(self.device))
            else:
                rc = lib.uttt_chunk_update_phase(C.byref(self.args), _p(self.workspace), self.workspace.numel(),
                                                 int(phase), _stream(self.device))
        N.check(rc, "uttt_chunk_update")
        return self.result

    def launch_noalloc(self) -> Tuple[Tensor, ...]:
        """Enqueue the whole update through ``uttt_chunk_update_noalloc`` (the library's
        device-resident scratch instead of ``workspace``; calls on one GPU must not overlap)."""
        lib = N.load_library()
        with torch.cuda.device(self.device):
            rc = lib.uttt_chunk_update_noalloc(C.byref(self.args), _stream(self.device))
        N.check(rc, "uttt_chunk_update_noalloc")
        return self.result


def prepare_chunk_update(q: Tensor, k: Tensor, v: Tensor, eta: Tensor, alpha: Tensor,
                         w_up: Tensor, w_gate: Tensor, w_down: Tensor,
                         s_up: Tensor, s_gate: Tensor, s_down: Tensor,
                         ln_weight: Tensor, ln_bias: Tensor, token_mask: Optional[Tensor],
                         momentum_beta: float, max_inner_grad_norm: float, normalize_by_dim: bool, eps: float,
                         read_w_up: Optional[Tensor] = None, read_w_gate: Optional[Tensor] = None,
                         read_w_down: Optional[Tensor] = None,
                         out_state: Optional[Sequence[Tensor]] = None,
                         out: Optional[Tensor] = None,
                         surprise: Optional[Tensor] = None,
                         workspace: Optional[Tensor] = None,
                         row_loss: Optional[Tensor] = None,
                         min_row_surprise: float = 0.0) -> PreparedUpdate:
    """Validate and marshal one chunk update (see ``chunk_update``) without launching it."""
    if q.dim() != 3 or q.shape != k.shape or q.shape != v.shape:
        raise ValueError(f"q/k/v must share one (B, C, D) shape, got {tuple(q.shape)}, {tuple(k.shape)}, {tuple(v.shape)}")
    bsz, tokens, dim = q.shape
    if not 1 <= tokens <= N.MAX_UPDATE_TOKENS:
        raise ValueError(f"a chunk update holds 1..{N.MAX_UPDATE_TOKENS} tokens on the HIP path, got {tokens}")
    if q.dtype != k.dtype or q.dtype != v.dtype:
        raise ValueError("q, k and v must share one dtype")
    act = q.dtype
    code = _act_code(act)
    dev = q.device
    ff = w_up.shape[-1]
    if w_up.shape != (bsz, dim, ff) or w_gate.shape != (bsz, dim, ff) or w_down.shape != (bsz, ff, dim):
        raise ValueError(f"state shapes {tuple(w_up.shape)}, {tuple(w_gate.shape)}, {tuple(w_down.shape)} "
                         f"do not match B={bsz}, D={dim}, F={ff}")
    for s, w in ((s_up, w_up), (s_gate, w_gate), (s_down, w_down)):
        if s.shape != w.shape:
            raise ValueError("momentum buffers must match the weight shapes")
    if dim % 64 or ff % 64 or dim > 4096:
        raise ValueError(f"d_model and d_ff must be multiples of 64 (d_model <= 4096); got {dim}, {ff}")
    eta = _per_token(eta, bsz, tokens, "eta")
    alpha = _per_token(alpha, bsz, tokens, "alpha")
    _require_device(dev, k, v, eta, alpha, w_up, w_gate, w_down, s_up, s_gate, s_down, ln_weight, ln_bias,
                    token_mask, read_w_up, read_w_gate, read_w_down)
    _forward_only(q, k, v, eta, alpha, w_up, w_gate, w_down, s_up, s_gate, s_down, ln_weight, ln_bias)

    q, k, v = _rows(q), _rows(k), _rows(v)
    eta, alpha = _row_vector(eta, act), _row_vector(alpha, act)
    mask = None
    if token_mask is not None:
        if token_mask.shape != (bsz, tokens):
            raise ValueError(f"token_mask must be (B, C) = ({bsz}, {tokens})")
        mask = token_mask.to(torch.float32)
        if tokens > 1 and mask.stride(1) != 1:
            mask = mask.contiguous()
    ws = [_state(t, n) for t, n in ((w_up, "w_up"), (w_gate, "w_gate"), (w_down, "w_down"),
                                     (s_up, "s_up"), (s_gate, "s_gate"), (s_down, "s_down"))]
    if read_w_up is None and read_w_gate is None and read_w_down is None:
        rw, r_stride = ws[:3], dim * ff
    else:
        if read_w_up is None or read_w_gate is None or read_w_down is None:
            raise ValueError("read weights must be given all three or none")
        parts = [_read_weight(t, bsz, n) for t, n in ((read_w_up, "read_w_up"), (read_w_gate, "read_w_gate"),
                                                        (read_w_down, "read_w_down"))]
        if len({p[1] for p in parts}) != 1:
            raise ValueError("read weights must all be shared (batch 1) or all per-row")
        rw, r_stride = [p[0] for p in parts], parts[0][1]
    ln_w = ln_weight.to(torch.float32).contiguous()
    ln_b = ln_bias.to(torch.float32).contiguous()
    if ln_w.numel() != dim or ln_b.numel() != dim:
        raise ValueError("ln_weight / ln_bias must have d_model elements")

    if out_state is None:
        outs = [torch.empty_like(t) for t in ws]
    else:
        outs = list(out_state)
        if len(outs) != 6 or any(o.dtype != torch.float32 or not o.is_contiguous() or o.shape != t.shape
                                 for o, t in zip(outs, ws)):
            raise ValueError("out_state must be six contiguous fp32 tensors shaped like the state")
    if out is None:
        out = torch.empty((bsz, tokens, dim), dtype=act, device=dev)
    elif out.shape != (bsz, tokens, dim) or out.dtype != act or out.stride(2) != 1 or (tokens > 1 and out.stride(1) != dim):
        raise ValueError("out must be (B, C, D) in the activation dtype with token stride D")
    if surprise is None:
        surprise = torch.empty((), dtype=torch.float32, device=dev)

    lib = N.load_library()
    nbytes = lib.uttt_chunk_update_workspace_tokens(bsz, tokens, dim, ff, code)
    if workspace is None or workspace.numel() < nbytes or workspace.device != dev:
        workspace = torch.empty(max(nbytes, 1), dtype=torch.uint8, device=dev)
    a = N.ChunkUpdateArgs()
    a.batch, a.tokens, a.d_model, a.d_ff = bsz, tokens, dim, ff
    a.act_dtype, a.normalize_by_dim = code, int(bool(normalize_by_dim))
    a.momentum_beta, a.max_inner_grad_norm, a.eps = float(momentum_beta), float(max_inner_grad_norm or 0.0), float(eps)
    a.q, a.q_row_stride = _p(q), q.stride(0)
    a.k, a.k_row_stride = _p(k), k.stride(0)
    a.v, a.v_row_stride = _p(v), v.stride(0)
    a.eta, a.eta_row_stride = _p(eta), eta.stride(0)
    a.alpha, a.alpha_row_stride = _p(alpha), alpha.stride(0)
    a.token_mask, a.mask_row_stride = _p(mask), (mask.stride(0) if mask is not None else 0)
    a.w_up, a.w_gate, a.w_down, a.s_up, a.s_gate, a.s_down = (_p(t) for t in ws)
    a.r_up, a.r_gate, a.r_down = (_p(t) for t in rw)
    a.r_row_stride = r_stride
    a.ln_weight, a.ln_bias = _p(ln_w), _p(ln_b)
    a.w_up_out, a.w_gate_out, a.w_down_out, a.s_up_out, a.s_gate_out, a.s_down_out = (_p(t) for t in outs)
    a.out, a.out_row_stride = _p(out), out.stride(0)
    a.surprise = _p(surprise)
    if row_loss is not None:
        if row_loss.shape != (bsz, 2) or row_loss.dtype != torch.float32 or not row_loss.is_contiguous():
            raise ValueError("row_loss must be a contiguous fp32 (B, 2) tensor")
        a.row_loss = _p(row_loss)
    a.min_row_surprise = float(min_row_surprise or 0.0)
    keep = (q, k, v, eta, alpha, mask, ws, rw, ln_w, ln_b, row_loss)
    return PreparedUpdate(a, keep, workspace, (out, *outs, surprise), dev)


def chunk_update(q: Tensor, k: Tensor, v: Tensor, eta: Tensor, alpha: Tensor,
                 w_up: Tensor, w_gate: Tensor, w_down: Tensor,
                 s_up: Tensor, s_gate: Tensor, s_down: Tensor,
                 ln_weight: Tensor, ln_bias: Tensor, token_mask: Optional[Tensor],
                 momentum_beta: float, max_inner_grad_norm: float, normalize_by_dim: bool, eps: float,
                 read_w_up: Optional[Tensor] = None, read_w_gate: Optional[Tensor] = None,
                 read_w_down: Optional[Tensor] = None,
                 out_state: Optional[Sequence[Tensor]] = None,
                 out: Optional[Tensor] = None,
                 surprise: Optional[Tensor] = None,
                 workspace: Optional[Tensor] = None) -> Tuple[Tensor, ...]:
    """One chunk of the shared fast-weight update on the GPU.

    Returns ``(readout, W_up', W_gate', W_down', S_up', S_gate', S_down', surprise)``
    like the reference.  ``out_state`` (six fp32 tensors) receives the new state
    and may be the input state itself for an in-place update; by default new
    tensors are allocated.  ``surprise`` is a 0-d fp32 device tensor (no sync).
    ``workspace`` (uint8, at least ``uttt_chunk_update_workspace_tokens`` bytes) is reused
    when given; calls that share one workspace must be ordered on one stream.  A chunk
    may hold up to ``N.MAX_UPDATE_TOKENS`` (512) tokens: one write for the whole chunk, as
    the reference's chunk loop does with its configs' 128- and 512-token chunks.
    """
    return prepare_chunk_update(q, k, v, eta, alpha, w_up, w_gate, w_down, s_up, s_gate, s_down, ln_weight,
                                ln_bias, token_mask, momentum_beta, max_inner_grad_norm, normalize_by_dim, eps,
                                read_w_up, read_w_gate, read_w_down, out_state, out, surprise,
                                workspace).launch()


# ---------------------------------------------------------------------------
# every chunk of one standalone layer in one launch (uTTTLayer.forward's chunk loop,
# model/uttt_layer.py:1451-1478)
# ---------------------------------------------------------------------------

_RESIDENT_DIMS = (128, 256, 512)


class _ResidentErrors:
    """Per device: a sticky device word that every resident launch sets on a barrier timeout, and a
    pinned host mirror refreshed by an asynchronous copy after each launch (no allocation per call;
    the mirror lags the device word by at most the calls still in flight)."""

    def __init__(self, device: torch.device):
        self.word = torch.zeros(1, dtype=torch.int32, device=device)
        self.mirror = torch.zeros(1, dtype=torch.int32, pin_memory=True)
        self.event = torch.cuda.Event()
        self.recorded = False


_resident_errors = {}


def _errors_for(device: torch.device) -> _ResidentErrors:
    key = device.index if device.index is not None else torch.cuda.current_device()
    if key not in _resident_errors:
        _resident_errors[key] = _ResidentErrors(torch.device("cuda", key))
    return _resident_errors[key]


def resident_update_eligible(q: Tensor, w_up: Tensor, chunk_size: int) -> bool:
    """True when ``layer_update_resident`` takes these operands: one fp32 row on the GPU,
    d_model 128 / 256 / 512, d_ff a multiple of 64 with d_ff / 8 workgroups fitting the CUs,
    chunks of at most 64 tokens."""
    if q.device.type != "cuda" or q.dtype != torch.float32 or q.dim() != 3 or q.shape[0] != 1:
        return False
    dim, ff = q.shape[2], w_up.shape[-1]
    if dim not in _RESIDENT_DIMS or ff % 64 or not 1 <= chunk_size <= 64 or q.shape[1] < 1:
        return False
    with torch.cuda.device(q.device):
        return bool(N.load_library().uttt_layer_update_resident_supported(1, dim, ff))


def check_resident_flags(wait: bool = False) -> None:
    """Raise if a finished ``layer_update_resident`` launch reports a device-wide barrier that
    waited past its bound (that call's results are then invalid: it wrote NaN into its state,
    surprise and readout).  ``wait`` blocks until every launch so far has been accounted for.
    A report is raised once: the device word and its mirror are cleared first, so later calls
    are not blamed for it."""
    for dev, errs in _resident_errors.items():
        if wait:
            errs.mirror.copy_(errs.word.cpu())
        elif not (errs.recorded and errs.event.query()):
            continue
        if int(errs.mirror[0]) != 0:
            with torch.cuda.device(dev):
                errs.word.zero_()
                torch.cuda.current_stream().synchronize()
            errs.mirror.zero_()
            raise RuntimeError(f"uttt_layer_update_resident on cuda:{dev}: a device-wide barrier timed out (the "
                               "workgroups were not all resident); that call's results are invalid (NaN)")


def layer_update_resident(q: Tensor, k: Tensor, v: Tensor, eta: Tensor, alpha: Tensor,
                          w_up: Tensor, w_gate: Tensor, w_down: Tensor,
                          s_up: Tensor, s_gate: Tensor, s_down: Tensor,
                          ln_weight: Tensor, ln_bias: Tensor, token_mask: Optional[Tensor],
                          momentum_beta: float, max_inner_grad_norm: float, normalize_by_dim: bool, eps: float,
                          chunk_size: int = 64, out_state: Optional[Sequence[Tensor]] = None,
                          workspace: Optional[Tensor] = None, force_timeout: bool = False) -> Tuple[Tensor, ...]:
    """All chunks of one layer's forward for one fp32 row (``uttt_layer_update_resident``):
    chunk c reads the state left by chunk c - 1, its readout goes through its own pre-update
    state.  ``q/k/v`` (1, T, D); ``eta/alpha`` (1, T) or (1, T, 1); ``token_mask`` (1, T) or
    None; state (1, D, F) / (1, F, D).  Returns ``(readout (1, T, D), W_up', W_gate', W_down',
    S_up', S_gate', S_down', surprise (n_chunks,))``; ``out_state`` may be the input state
    for an in-place update.  A device-wide barrier that times out makes every result NaN and is
    reported by ``check_resident_flags`` (also at the start of a later call);
    ``force_timeout`` (a test hook) runs the call as if its first barrier had timed out."""
    if q.dim() != 3 or q.shape != k.shape or q.shape != v.shape:
        raise ValueError(f"q/k/v must share one (1, T, D) shape, got {tuple(q.shape)}, {tuple(k.shape)}, "
                         f"{tuple(v.shape)}")
    bsz, tokens, dim = q.shape
    ff = w_up.shape[-1]
    if not resident_update_eligible(q, w_up, chunk_size) or k.dtype != q.dtype or v.dtype != q.dtype:
        raise ValueError(f"the resident layer update takes one fp32 row with d_model in {_RESIDENT_DIMS}, d_ff a "
                         f"multiple of 64 within the CU count and chunks of 1..64 tokens; got {tuple(q.shape)} "
                         f"{q.dtype}, d_ff {ff}, chunk {chunk_size}")
    if w_up.shape != (1, dim, ff) or w_gate.shape != (1, dim, ff) or w_down.shape != (1, ff, dim):
        raise ValueError(f"state shapes {tuple(w_up.shape)}, {tuple(w_gate.shape)}, {tuple(w_down.shape)} "
                         f"do not match B=1, D={dim}, F={ff}")
    for s, w in ((s_up, w_up), (s_gate, w_gate), (s_down, w_down)):
        if s.shape != w.shape:
            raise ValueError("momentum buffers must match the weight shapes")
    eta = _per_token(eta, bsz, tokens, "eta")
    alpha = _per_token(alpha, bsz, tokens, "alpha")
    dev = q.device
    _require_device(dev, k, v, eta, alpha, w_up, w_gate, w_down, s_up, s_gate, s_down, ln_weight, ln_bias,
                    token_mask)
    _forward_only(q, k, v, eta, alpha, w_up, w_gate, w_down, s_up, s_gate, s_down, ln_weight, ln_bias)
    q, k, v = (t.contiguous() for t in (q, k, v))
    q, k, v = (t if t.data_ptr() % 16 == 0 else t.clone() for t in (q, k, v))
    eta = _row_vector(eta, torch.float32).contiguous()
    alpha = _row_vector(alpha, torch.float32).contiguous()
    mask = None
    if token_mask is not None:
        if token_mask.shape != (bsz, tokens):
            raise ValueError(f"token_mask must be (1, T) = (1, {tokens})")
        mask = token_mask.to(torch.float32).contiguous()
    ws = [_state(t, n) for t, n in ((w_up, "w_up"), (w_gate, "w_gate"), (w_down, "w_down"),
                                     (s_up, "s_up"), (s_gate, "s_gate"), (s_down, "s_down"))]
    ln_w = ln_weight.to(torch.float32).contiguous()
    ln_b = ln_bias.to(torch.float32).contiguous()
    if ln_w.numel() != dim or ln_b.numel() != dim:
        raise ValueError("ln_weight / ln_bias must have d_model elements")
    if out_state is None:
        outs = [torch.empty_like(t) for t in ws]
    else:
        outs = list(out_state)
        if len(outs) != 6 or any(o.dtype != torch.float32 or not o.is_contiguous() or o.shape != t.shape
                                 for o, t in zip(outs, ws)):
            raise ValueError("out_state must be six contiguous fp32 tensors shaped like the state")
    n_chunks = (tokens + chunk_size - 1) // chunk_size
    out = torch.empty((1, tokens, dim), dtype=torch.float32, device=dev)
    surprise = torch.empty((n_chunks,), dtype=torch.float32, device=dev)
    lib = N.load_library()
    nbytes = lib.uttt_layer_update_resident_workspace(dim, ff)
    if workspace is None or workspace.numel() < nbytes or workspace.device != dev:
        workspace = torch.empty(nbytes, dtype=torch.uint8, device=dev)
    a = N.LayerUpdateArgs()
    a.batch, a.tokens, a.d_model, a.d_ff, a.chunk_size = 1, tokens, dim, ff, int(chunk_size)
    a.normalize_by_dim = int(bool(normalize_by_dim))
    a.momentum_beta, a.max_inner_grad_norm, a.eps = float(momentum_beta), float(max_inner_grad_norm or 0.0), float(eps)
    a.q, a.k, a.v = _p(q), _p(k), _p(v)
    a.eta, a.alpha, a.token_mask = _p(eta), _p(alpha), _p(mask)
    a.w_up, a.w_gate, a.w_down, a.s_up, a.s_gate, a.s_down = (_p(t) for t in ws)
    a.ln_weight, a.ln_bias = _p(ln_w), _p(ln_b)
    a.w_up_out, a.w_gate_out, a.w_down_out, a.s_up_out, a.s_gate_out, a.s_down_out = (_p(t) for t in outs)
    a.out, a.surprise = _p(out), _p(surprise)
    errs = _errors_for(dev)
    a.error_word = _p(errs.word)
    a.force_timeout = int(bool(force_timeout))
    with torch.cuda.device(dev):
        capturing = torch.cuda.is_current_stream_capturing()
        if not capturing:  # (event queries are not allowed under graph capture)
            check_resident_flags()
        rc = lib.uttt_layer_update_resident(C.byref(a), _p(workspace), workspace.numel(), _stream(dev))
        N.check(rc, "uttt_layer_update_resident")
        if not capturing:
            errs.mirror.copy_(errs.word, non_blocking=True)
            errs.event.record()
            errs.recorded = True
    return (out, *outs, surprise)


# ---------------------------------------------------------------------------
# one chunk, all layers (the chunk-first shared schedule, model/uttt_model.py:453-608)
# ---------------------------------------------------------------------------

class PreparedChain:
    """A validated ``uttt_chunk_chain`` call; ``launch()`` enqueues it on the current stream."""

    def __init__(self, args, keep, workspace, result, device, n_layers):
        self.args, self._keep, self.workspace, self.result, self.device = args, keep, workspace, result, device
        self.n_layers = n_layers

    _launch_names: dict = {}

    def stage_launches(self, stage: int, part: int = 0) -> Tuple[str, ...]:
        """Kernel names of the launches stage ``stage`` (part ``part``) makes, in enqueue order
        (they depend only on the chain's shape and options, so they are kept per shape)."""
        a = self.args
        key = (a.batch, a.layers, a.tokens, a.d_model, a.d_ff, a.act_dtype, bool(a.w_up_copy), a.w_products_given,
               bool(a.token_mask), int(stage), int(part))
        hit = PreparedChain._launch_names.get(key)
        if hit is not None:
            return hit
        lib = N.load_library()
        names = (C.c_char_p * 64)()
        count = C.c_int32(0)
        with torch.cuda.device(self.device):
            N.check(lib.uttt_chunk_chain_stage_launch(C.byref(a), _p(self.workspace), self.workspace.numel(),
                                                      int(stage), int(part), 0, 0, names, 64, C.byref(count), None),
                    "uttt_chunk_chain_stage_launch")
        out = tuple(names[i].decode() for i in range(min(count.value, 64)))
        PreparedChain._launch_names[key] = out
        return out

    def launch(self, stage: Optional[int] = None, part: int = 0,
               timer: Optional["KernelTimer"] = None) -> Tuple[Tensor, Optional[Tensor]]:
        """Enqueue the whole chain, or one of its ``layers + 1`` stream-ordered stages, or one
        part of a stage (1: its snapshot products and key Gram rows, 2: the rest).  With a
        ``timer``, a stage is enqueued launch by launch, with events around the kernels the timer
        follows (same kernels, same order)."""
        lib = N.load_library()
        if timer is not None and stage is not None:
            stream = torch.cuda.current_stream(self.device)
            names = self.stage_launches(stage, part)

            def enqueue(lo: int, hi: int) -> None:
                if hi > lo:
                    with torch.cuda.device(self.device):
                        N.check(lib.uttt_chunk_chain_stage_launch(C.byref(self.args), _p(self.workspace),
                                                                  self.workspace.numel(), int(stage), int(part), lo, hi,
                                                                  None, 0, None, _stream(self.device)),
                                "uttt_chunk_chain_stage_launch")
            done = 0  # launches between followed kernels go out as one range
            for i, name in enumerate(names):
                if name in timer.kernels:
                    enqueue(done, i)
                    pair = timer.begin(name, stream)
                    enqueue(i, i + 1)
                    timer.end(pair, stream)
                    done = i + 1
            enqueue(done, len(names))
            return self.result
        with torch.cuda.device(self.device):
            if stage is None:
                rc = lib.uttt_chunk_chain(C.byref(self.args), _p(self.workspace), self.workspace.numel(),
                                          _stream(self.device))
            elif part:
                rc = lib.uttt_chunk_chain_stage_part(C.byref(self.args), _p(self.workspace),
                                                     self.workspace.numel(), int(stage), int(part),
                                                     _stream(self.device))
            else:
                rc = lib.uttt_chunk_chain_stage(C.byref(self.args), _p(self.workspace), self.workspace.numel(),
                                                int(stage), _stream(self.device))
        N.check(rc, "uttt_chunk_chain")
        return self.result


class KernelTimer:
    """HIP events around chosen kernels of the layer chain, recorded on the stream each kernel
    is enqueued on: ``kernels`` names the kernels to follow (``ChunkChainRun.stage_launches``
    names).  ``summary()`` (after a synchronize) gives, per followed kernel, the number of
    launches and their mean duration in ms."""

    def __init__(self, kernels: Sequence[str]):
        self.kernels = set(kernels)
        self.pairs = {k: [] for k in self.kernels}

    def begin(self, name: str, stream) -> Optional[Tuple[str, "torch.cuda.Event"]]:
        if name not in self.kernels:
            return None
        start = torch.cuda.Event(enable_timing=True)
        start.record(stream)
        return name, start

    def end(self, pair, stream) -> None:
        if pair is None:
            return
        stop = torch.cuda.Event(enable_timing=True)
        stop.record(stream)
        self.pairs[pair[0]].append((pair[1], stop))

    def reset(self) -> None:
        self.pairs = {k: [] for k in self.kernels}

    def summary(self) -> dict:
        out = {}
        for name, pairs in self.pairs.items():
            if pairs:
                ms = [a.elapsed_time(b) for a, b in pairs]
                out[name] = {"launches": len(ms), "mean_ms": sum(ms) / len(ms)}
        return out


def _inplace_state(t: Tensor, name: str) -> Tensor:
    if t.dtype != torch.float32 or not t.is_contiguous() or t.data_ptr() % 16:
        raise ValueError(f"{name}: the layer chain updates the state in place and needs contiguous, "
                         f"16-byte aligned fp32 tensors")
    return t


class ChunkChainRun(PreparedChain):
    """One chunk's layer chain fed layer by layer (``uttt_chunk_chain_stage``).

    ``add_layer(k, v, eta, alpha)`` records layer l's inputs and enqueues stage l on the
    current stream; it reads only layers <= l, so it can run while the caller computes the
    next layers.  ``finish()`` enqueues the last stage (the state write), which must follow
    every reader of the chunk-start state and its copies.  Arguments as ``prepare_chunk_chain``
    with the layer count and chunk length given up front.

    With ``w_products_given`` (bf16 copies only) the caller forms layer l's products
    k_l W_up and k_l W_gate with the chunk-start copies itself, into ``w_product_outputs(l)``
    (``swiglu_readout(..., keys=k_l, key_outputs=...)`` shares the readout's weight reads),
    before stage l's second part (``launch(l, part=2)``) runs."""

    def __init__(self, n_layers: int, tokens: int, state: Sequence[Tensor], ln_weight: Tensor, ln_bias: Tensor,
                 token_mask: Optional[Tensor], momentum_beta: float, max_inner_grad_norm: float,
                 normalize_by_dim: bool, eps: float, act_dtype: torch.dtype,
                 copies: Optional[Sequence[Tensor]] = None, surprise: Optional[Tensor] = None,
                 row_loss: Optional[Tensor] = None, min_row_surprise: float = 0.0,
                 workspace: Optional[Tensor] = None, w_products_given: bool = False) -> None:
        if not 1 <= n_layers <= N.MAX_CHAIN:
            raise ValueError(f"need 1..{N.MAX_CHAIN} layers")
        if w_products_given and copies is None:
            raise ValueError("w_products_given needs the bf16 state copies")
        if not 1 <= tokens <= 64:
            raise ValueError(f"a chunk holds 1..64 tokens on the HIP path, got {tokens}")
        code = _act_code(act_dtype)
        w_up, w_gate, w_down, s_up, s_gate, s_down = (_inplace_state(t, n) for t, n in zip(
            state, ("w_up", "w_gate", "w_down", "s_up", "s_gate", "s_down")))
        bsz, dim, ff = w_up.shape
        dev = w_up.device
        if w_gate.shape != (bsz, dim, ff) or w_down.shape != (bsz, ff, dim) \
                or s_up.shape != w_up.shape or s_gate.shape != w_gate.shape or s_down.shape != w_down.shape:
            raise ValueError(f"state shapes do not match B={bsz}, D={dim}, F={ff}")
        if dim % 64 or ff % 64 or dim > 4096:
            raise ValueError(f"d_model and d_ff must be multiples of 64 (d_model <= 4096); got {dim}, {ff}")
        _require_device(dev, *state, ln_weight, ln_bias, token_mask)
        _forward_only(*state)
        mask = None
        keep = []
        if token_mask is not None:
            if token_mask.shape != (bsz, tokens):
                raise ValueError(f"token_mask must be (B, C) = ({bsz}, {tokens})")
            mask = token_mask.to(torch.float32)
            if tokens > 1 and mask.stride(1) != 1:
                mask = mask.contiguous()
            keep.append(mask)
        ln_w = ln_weight.to(torch.float32).contiguous()
        ln_b = ln_bias.to(torch.float32).contiguous()
        if ln_w.numel() != dim or ln_b.numel() != dim:
            raise ValueError("ln_weight / ln_bias must have d_model elements")
        if copies is not None:
            if act_dtype != torch.bfloat16:
                raise ValueError("bf16 state copies go with bf16 activations only")
            if len(copies) != 6 or any(c.dtype != torch.bfloat16 or not c.is_contiguous() or c.shape != w.shape
                                       or c.device != dev or c.data_ptr() % 16
                                       for c, w in zip(copies, (w_up, w_gate, w_down, s_up, s_gate, s_down))):
                raise ValueError("copies must be six contiguous, aligned bf16 tensors shaped like the state")
        if surprise is None:
            surprise = torch.empty(n_layers, dtype=torch.float32, device=dev)
        elif surprise.shape != (n_layers,) or surprise.dtype != torch.float32 or not surprise.is_contiguous():
            raise ValueError("surprise must be a contiguous fp32 (layers,) tensor")
        if row_loss is not None and (row_loss.shape != (n_layers, bsz, 2) or row_loss.dtype != torch.float32
                                     or not row_loss.is_contiguous()):
            raise ValueError("row_loss must be a contiguous fp32 (layers, B, 2) tensor")
        if not math.isfinite(min_row_surprise) or min_row_surprise < 0:
            raise ValueError("min_row_surprise must be finite and >= 0")
        nbytes = N.load_library().uttt_chunk_chain_workspace(bsz, n_layers, dim, ff, code)
        if nbytes == 0:
            raise ValueError("unsupported layer chain dimensions")
        if workspace is None or workspace.numel() < nbytes or workspace.device != dev:
            workspace = torch.empty(nbytes, dtype=torch.uint8, device=dev)
        a = N.ChunkChainArgs()
        a.batch, a.layers, a.tokens, a.d_model, a.d_ff = bsz, n_layers, tokens, dim, ff
        a.act_dtype, a.normalize_by_dim = code, int(bool(normalize_by_dim))
        a.momentum_beta, a.max_inner_grad_norm, a.eps = (float(momentum_beta), float(max_inner_grad_norm or 0.0),
                                                         float(eps))
        a.min_row_surprise = float(min_row_surprise)
        a.token_mask, a.mask_row_stride = _p(mask), (mask.stride(0) if mask is not None else 0)
        a.w_up, a.w_gate, a.w_down, a.s_up, a.s_gate, a.s_down = (_p(t) for t in
                                                                  (w_up, w_gate, w_down, s_up, s_gate, s_down))
        a.ln_weight, a.ln_bias = _p(ln_w), _p(ln_b)
        if copies is not None:
            (a.w_up_copy, a.w_gate_copy, a.w_down_copy,
             a.s_up_copy, a.s_gate_copy, a.s_down_copy) = (_p(c) for c in copies)
        a.surprise, a.row_loss = _p(surprise), _p(row_loss)
        a.w_products_given = int(bool(w_products_given))
        keep += [ln_w, ln_b, state, copies]
        super().__init__(a, keep, workspace, (surprise, row_loss), dev, n_layers)
        self._act, self._shape, self._ff, self._code = act_dtype, (bsz, tokens, dim), ff, code
        self.layers_added = 0

    def w_product_outputs(self, layer: int) -> Tuple[Tensor, Tensor]:
        """Workspace views (B, 64, d_ff) that take layer ``layer``'s k W_up and k W_gate."""
        bsz, _, dim = self._shape
        up, gate = C.c_size_t(0), C.c_size_t(0)
        N.check(N.load_library().uttt_chunk_chain_w_products(bsz, self.n_layers, dim, self._ff, self._code,
                                                               int(layer), C.byref(up), C.byref(gate)),
                "uttt_chunk_chain_w_products")
        n = bsz * 64 * self._ff * torch.empty((), dtype=self._act).element_size()

        def view(off: int) -> Tensor:
            return self.workspace[off:off + n].view(self._act).view(bsz, 64, self._ff)
        return view(up.value), view(gate.value)

    def set_layer(self, k: Tensor, v: Tensor, eta: Tensor, alpha: Tensor) -> int:
        """Record the next layer's inputs without launching; returns its index."""
        l = self.layers_added
        if l >= self.n_layers:
            raise ValueError("all layers of the chain were already given")
        bsz, tokens, dim = self._shape
        act = self._act
        if k.shape != (bsz, tokens, dim) or v.shape != k.shape or k.dtype != act or v.dtype != act:
            raise ValueError(f"layer {l}: k/v must be ({bsz}, {tokens}, {dim}) {act}")
        eta = _per_token(eta, bsz, tokens, f"layer {l}: eta")
        alpha = _per_token(alpha, bsz, tokens, f"layer {l}: alpha")
        _require_device(self.device, k, v, eta, alpha)
        _forward_only(k, v, eta, alpha)
        k, v = _rows(k), _rows(v)
        e, al = _row_vector(eta, act), _row_vector(alpha, act)
        a = self.args
        if l == 0:
            a.kv_row_stride, a.ea_row_stride = k.stride(0), e.stride(0)
        if bsz > 1 and (k.stride(0) != a.kv_row_stride or v.stride(0) != a.kv_row_stride):
            k, v = k.contiguous(), v.contiguous()
            if k.stride(0) != a.kv_row_stride:
                raise ValueError("all layers' k/v must share one row stride")
        if bsz > 1 and (e.stride(0) != a.ea_row_stride or al.stride(0) != a.ea_row_stride):
            e, al = e.contiguous(), al.contiguous()
            if e.stride(0) != a.ea_row_stride:
                raise ValueError("all layers' eta/alpha must share one row stride")
        a.k[l], a.v[l], a.eta[l], a.alpha[l] = _p(k), _p(v), _p(e), _p(al)
        self._keep += [k, v, e, al]
        self.layers_added = l + 1
        return l

    def add_layer(self, k: Tensor, v: Tensor, eta: Tensor, alpha: Tensor) -> None:
        """Record layer l's inputs and enqueue stage l on the current stream."""
        self.launch(self.set_layer(k, v, eta, alpha))

    def finish(self) -> Tuple[Tensor, Optional[Tensor]]:
        """Enqueue the state write (after every layer was added)."""
        if self.layers_added != self.n_layers:
            raise ValueError(f"{self.layers_added} of {self.n_layers} layers were given")
        return self.launch(self.n_layers)


def prepare_chunk_chain(ks: Sequence[Tensor], vs: Sequence[Tensor], etas: Sequence[Tensor],
                        alphas: Sequence[Tensor], state: Sequence[Tensor], ln_weight: Tensor, ln_bias: Tensor,
                        token_mask: Optional[Tensor], momentum_beta: float, max_inner_grad_norm: float,
                        normalize_by_dim: bool, eps: float, copies: Optional[Sequence[Tensor]] = None,
                        surprise: Optional[Tensor] = None, row_loss: Optional[Tensor] = None,
                        min_row_surprise: float = 0.0, workspace: Optional[Tensor] = None) -> PreparedChain:
    """Validate and marshal the L chained layer updates of one chunk (``uttt_chunk_chain``).

    ``ks[l]``/``vs[l]`` (B, C, D), ``etas[l]``/``alphas[l]`` (B, C) or (B, C, 1) are layer l's
    update inputs; ``state`` = (w_up, w_gate, w_down, s_up, s_gate, s_down), fp32, updated in
    place; ``copies`` optional bf16 tensors shaped like the six state tensors (bf16 activations
    only): on entry the chunk-start state rounded to bf16, which the kernels then read instead
    of the fp32 masters; on exit the final state rounded to bf16."""
    n_layers = len(ks)
    if not 1 <= n_layers <= N.MAX_CHAIN or not (len(vs) == len(etas) == len(alphas) == n_layers):
        raise ValueError(f"need 1..{N.MAX_CHAIN} layers with k, v, eta and alpha each")
    if ks[0].dim() != 3:
        raise ValueError("k must be (B, C, D)")
    run = ChunkChainRun(n_layers, ks[0].shape[1], state, ln_weight, ln_bias, token_mask, momentum_beta,
                        max_inner_grad_norm, normalize_by_dim, eps, ks[0].dtype, copies=copies, surprise=surprise,
                        row_loss=row_loss, min_row_surprise=min_row_surprise, workspace=workspace)
    for l in range(n_layers):
        run.set_layer(ks[l], vs[l], etas[l], alphas[l])
    return run


def chunk_chain(*args, **kwargs) -> Tuple[Tensor, Optional[Tensor]]:
    """Run ``prepare_chunk_chain(...)`` and launch it; returns (per-layer surprise, row_loss)."""
    return prepare_chunk_chain(*args, **kwargs).launch()


# ---------------------------------------------------------------------------
# frozen readout (reference swiglu_fast_forward, model/uttt_layer.py:211-247)
# ---------------------------------------------------------------------------

def proj_epilogue(y: Tensor, dim: int, q_weight: Tensor, k_weight: Tensor, eps: float, inner_lr: float,
                  weight_decay: float, x: Optional[Tensor] = None, x_eps: float = 0.0,
                  eta_alpha_bias: Optional[Tensor] = None, outs: Optional[Tuple[Tensor, Tensor]] = None,
                  build_only: bool = False):
    """q, k, v, eta, alpha from the packed slow-projection product y (..., 3 D + 2)
    (``uttt_proj_epilogue``; the RMSNorm / sigmoid part of reference fused_slow_projections,
    model/uttt_layer.py:1193-1231).  Returns q, k, v (..., D) and eta, alpha (..., 1).
    With ``x`` (..., D), the un-normalised rows y was projected from by a weight with the input
    RMSNorm weight folded in and no bias, y's rows are scaled by 1 / sqrt(mean(x^2) + x_eps)
    and ``eta_alpha_bias`` (2,) is added to its last two entries first.  ``outs`` = (qkv, ea),
    contiguous (3, rows, D) and (2, rows) tensors in y's dtype, receive the results;
    ``build_only`` returns (``uttt_proj_epilogue_args``, the tensors it points at) without
    launching."""
    if y.shape[-1] != 3 * dim + 2:
        raise ValueError(f"y must end in 3 * d_model + 2 = {3 * dim + 2} features, got {y.shape[-1]}")
    code = _act_code(y.dtype)
    dev = y.device
    _require_device(dev, q_weight, k_weight)
    _forward_only(y)
    lead = y.shape[:-1]
    y2 = y.reshape(-1, y.shape[-1])
    if y2.stride(1) != 1:
        y2 = y2.contiguous()
    rows = y2.shape[0]
    if outs is None:
        qkv = torch.empty((3, rows, dim), dtype=y.dtype, device=dev)
        ea = torch.empty((2, rows), dtype=y.dtype, device=dev)
    else:
        qkv, ea = outs
        if qkv.shape != (3, rows, dim) or ea.shape != (2, rows) or not qkv.is_contiguous() \
                or not ea.is_contiguous() or qkv.dtype != y.dtype or ea.dtype != y.dtype:
            raise ValueError(f"outs must be contiguous (3, {rows}, {dim}) and (2, {rows}) tensors in y's dtype")
        _require_device(dev, qkv, ea)
    qw = q_weight.detach().to(y.dtype).contiguous()  # the reference casts the weights to x's dtype
    kw = k_weight.detach().to(y.dtype).contiguous()
    a = N.ProjEpilogueArgs()
    a.rows, a.d_model, a.act_dtype = rows, dim, code
    a.eps, a.inner_lr, a.weight_decay = float(eps), float(inner_lr), float(weight_decay)
    a.y, a.y_row_stride = _p(y2), y2.stride(0)
    a.q_weight, a.k_weight = _p(qw), _p(kw)
    a.q, a.k, a.v, a.out_row_stride = _p(qkv[0]), _p(qkv[1]), _p(qkv[2]), dim
    a.eta, a.alpha = _p(ea[0]), _p(ea[1])
    keep = None
    if x is not None:
        x2 = x.reshape(-1, x.shape[-1])
        if x2.shape != (rows, dim) or x.dtype != y.dtype or x2.stride(1) != 1:
            raise ValueError("x must hold one d_model-wide row per row of y, in y's dtype")
        if not x_eps > 0.0 or eta_alpha_bias is None or eta_alpha_bias.numel() != 2:
            raise ValueError("a folded norm needs eps > 0 and the two eta / alpha biases")
        keep = eta_alpha_bias.detach().to(y.dtype).contiguous()
        _require_device(dev, x, keep)
        a.x, a.x_row_stride, a.x_eps, a.eta_alpha_bias = _p(x2), x2.stride(0), float(x_eps), _p(keep)
    if build_only:
        return a, (y2, qw, kw, keep, qkv, ea)
    lib = N.load_library()
    with torch.cuda.device(dev):
        N.check(lib.uttt_proj_epilogue(C.byref(a), _stream(dev)), "uttt_proj_epilogue")
    del keep
    return (qkv[0].view(*lead, dim), qkv[1].view(*lead, dim), qkv[2].view(*lead, dim),
            ea[0].view(*lead, 1), ea[1].view(*lead, 1))


def skinny_linear(x: Tensor, weight: Tensor, out: Optional[Tensor] = None,
                  residual: Optional[Tensor] = None, x_eps: float = 0.0) -> Tensor:
    """out = x weight^T (+ residual) for at most 64 bf16 rows (``uttt_skinny_linear``): the
    decode step's projections and LM head (reference engine/inference.py:263-276, the
    ``h + linear(x)`` residuals of model/uttt_layer.py:1528-1555).  x (m, k) and weight (n, k)
    with unit column stride; ``residual`` (m, n) may be ``out`` itself (an in-place update).
    ``x_eps`` > 0 RMS-normalises x's rows first (pass the weight with the norm weight
    multiplied into its columns)."""
    if x.dim() != 2 or weight.dim() != 2 or x.shape[1] != weight.shape[1]:
        raise ValueError(f"x (m, k) and weight (n, k) must agree on k, got {tuple(x.shape)} and {tuple(weight.shape)}")
    if x.dtype != torch.bfloat16 or weight.dtype != torch.bfloat16:
        raise ValueError("skinny_linear takes bf16 x and weight")
    dev = x.device
    _require_device(dev, weight, out, residual)
    _forward_only(x)
    m, k = x.shape
    n = weight.shape[0]
    if x.stride(1) != 1 or weight.stride(1) != 1:
        raise ValueError("x and weight need unit column stride")
    if out is None:
        out = torch.empty((m, n), dtype=x.dtype, device=dev)
    for name, t in (("out", out), ("residual", residual)):
        if t is not None and (t.shape != (m, n) or t.dtype != x.dtype or t.stride(1) != 1):
            raise ValueError(f"{name} must be ({m}, {n}) bf16 with unit column stride")
    a = N.SkinnyLinearArgs()
    if not x_eps >= 0.0:
        raise ValueError("x_eps must be >= 0")
    a.m, a.n, a.k, a.act_dtype, a.x_eps = m, n, k, N.DTYPE_BF16, float(x_eps)
    a.x, a.x_row_stride = _p(x), x.stride(0)
    a.w, a.w_row_stride = _p(weight), weight.stride(0)
    if residual is not None:
        a.residual, a.residual_row_stride = _p(residual), residual.stride(0)
    a.out, a.out_row_stride = _p(out), out.stride(0)
    lib = N.load_library()
    with torch.cuda.device(dev):
        N.check(lib.uttt_skinny_linear(C.byref(a), _stream(dev)), "uttt_skinny_linear")
    return out


_LINEAR_WS: dict = {}


def _linear_workspace(dev: torch.device, nbytes: int) -> Tensor:
    """The device's zero-filled ``uttt_linear`` workspace, grown to at least ``nbytes`` (every
    call leaves it zero-filled, so one buffer serves every call made in stream order)."""
    key = dev.index if dev.index is not None else torch.cuda.current_device()
    ws = _LINEAR_WS.get(key)
    if ws is None or ws.numel() < nbytes:
        ws = torch.zeros(max(nbytes, 1 << 20), dtype=torch.uint8, device=dev)
        _LINEAR_WS[key] = ws
    return ws


def linear(x: Tensor, weight: Tensor, out: Optional[Tensor] = None, residual: Optional[Tensor] = None,
           workspace: Optional[Tensor] = None, build_only: bool = False):
    """out = x weight^T (+ residual) for many bf16 rows (``uttt_linear``): the chunk-first forward
    pass's slow-weight projections (reference model/uttt_layer.py:1058-1081 the packed QKV
    projection, :1193-1231 the packed uTTT projections, :1528-1555 the ``h + linear(x)``
    residuals).  x (m, k) and weight (n, k) with unit column stride, 16-byte aligned, row strides
    multiples of 8 elements, k a multiple of 64; ``residual`` (m, n) may be ``out`` itself.
    ``workspace`` (uint8, zero-filled) defaults to one buffer per device shared by every call:
    calls on concurrent streams must each pass their own.  ``build_only`` returns the validated
    ``uttt_linear_args`` without launching (``out`` and, when the shape needs one, ``workspace``
    must then be given)."""
    if x.dim() != 2 or weight.dim() != 2 or x.shape[1] != weight.shape[1]:
        raise ValueError(f"x (m, k) and weight (n, k) must agree on k, got {tuple(x.shape)} and {tuple(weight.shape)}")
    if x.dtype != torch.bfloat16 or weight.dtype != torch.bfloat16:
        raise ValueError("linear takes bf16 x and weight")
    dev = x.device
    _require_device(dev, weight, out, residual)
    _forward_only(x)
    m, k = x.shape
    n = weight.shape[0]
    if x.stride(1) != 1 or weight.stride(1) != 1:
        raise ValueError("x and weight need unit column stride")
    if out is None:
        out = torch.empty((m, n), dtype=x.dtype, device=dev)
    for name, t in (("out", out), ("residual", residual)):
        if t is not None and (t.shape != (m, n) or t.dtype != x.dtype or t.stride(1) != 1):
            raise ValueError(f"{name} must be ({m}, {n}) bf16 with unit column stride")
    a = N.LinearArgs()
    a.m, a.n, a.k, a.act_dtype = m, n, k, N.DTYPE_BF16
    a.x, a.x_row_stride = _p(x), x.stride(0)
    a.w, a.w_row_stride = _p(weight), weight.stride(0)
    if residual is not None:
        a.residual, a.residual_row_stride = _p(residual), residual.stride(0)
    a.out, a.out_row_stride = _p(out), out.stride(0)
    lib = N.load_library()
    with torch.cuda.device(dev):
        need = lib.uttt_linear_workspace(m, n, k)
        if need:
            if workspace is None:
                if build_only:
                    raise ValueError(f"this shape needs a workspace of {need} bytes")
                workspace = _linear_workspace(dev, need)
            _require_device(dev, workspace)
            if workspace.numel() * workspace.element_size() < need:
                raise ValueError(f"the workspace holds fewer than the {need} bytes this shape needs")
            a.workspace, a.workspace_bytes = _p(workspace), workspace.numel() * workspace.element_size()
        if build_only:
            return a
        N.check(lib.uttt_linear(C.byref(a), _stream(dev)), "uttt_linear")
    return out


def linear_fits(x: Tensor, weight: Tensor) -> bool:
    """Whether ``linear`` takes these operands: bf16, k % 64 == 0, unit column stride, aligned
    bases and row strides."""
    return (x.dim() == 2 and weight.dim() == 2 and x.dtype == torch.bfloat16 and weight.dtype == torch.bfloat16
            and x.shape[1] == weight.shape[1] and x.shape[1] % 64 == 0 and x.shape[0] >= 1
            and x.stride(1) == 1 and weight.stride(1) == 1 and x.stride(0) % 8 == 0 and weight.stride(0) % 8 == 0
            and x.data_ptr() % 16 == 0 and weight.data_ptr() % 16 == 0)


def greedy_select(logits: Tensor, banned: Sequence[int] = (), active_limit: Optional[int] = None,
                  out: Optional[Tensor] = None, advance: Optional[Tensor] = None) -> Tensor:
    """Greedy next tokens (rows,) int64 from logits (rows, vocab) bf16 / fp32
    (``uttt_greedy_select``): argmax after setting the ``banned`` ids and the ids at or past
    ``active_limit`` to -inf (the temperature-0 branch of reference sample_next_token,
    model/uttt_model.py:1203-1221), one launch.  ``advance`` (rows,) int64, when given, is
    incremented by one in the same launch (a decode step's position counters)."""
    if logits.dim() != 2 or logits.stride(1) != 1:
        raise ValueError("logits must be (rows, vocab) with unit column stride")
    if len(banned) > 8:
        raise ValueError("at most 8 excluded ids")
    dev = logits.device
    _require_device(dev, out)
    code = _act_code(logits.dtype)
    rows, vocab = logits.shape
    if out is None:
        out = torch.empty(rows, dtype=torch.int64, device=dev)
    elif out.dtype != torch.int64 or out.numel() != rows or not out.is_contiguous():
        raise ValueError(f"out must be {rows} contiguous int64 entries")
    a = N.GreedyArgs()
    a.rows, a.vocab, a.dtype, a.n_banned = rows, vocab, code, len(banned)
    for i, t in enumerate(banned):
        a.banned[i] = int(t)
    a.active_limit = -1 if active_limit is None else int(active_limit)
    a.logits, a.row_stride, a.out = _p(logits), logits.stride(0), _p(out)
    if advance is not None:
        if advance.dtype != torch.int64 or advance.numel() != rows or not advance.is_contiguous():
            raise ValueError(f"advance must be {rows} contiguous int64 entries")
        _require_device(dev, advance)
        a.advance = _p(advance)
    lib = N.load_library()
    with torch.cuda.device(dev):
        N.check(lib.uttt_greedy_select(C.byref(a), _stream(dev)), "uttt_greedy_select")
    return out


def readout_workspace(x: Tensor, w_up: Tensor) -> Tensor:
    """A workspace for ``swiglu_readout`` of x (B, T, D) through weights shaped like ``w_up``,
    reusable by every later call with the same or smaller shapes."""
    bsz, tokens, dim = x.shape
    nbytes = N.load_library().uttt_readout_workspace(bsz, tokens, dim, w_up.shape[-1], _act_code(x.dtype))
    return torch.empty(max(nbytes, 1), dtype=torch.uint8, device=x.device)


def swiglu_readout(x: Tensor, w_up: Tensor, w_gate: Tensor, w_down: Tensor, ln_weight: Tensor,
                   ln_bias: Tensor, eps: float = 1e-5, out: Optional[Tensor] = None,
                   workspace: Optional[Tensor] = None, keys: Optional[Tensor] = None,
                   key_outputs: Optional[Tuple[Tensor, Tensor]] = None,
                   x_norm: Optional[Tuple[Tensor, float]] = None,
                   row_counters: Optional[Tensor] = None, sweep_reverse: bool = False,
                   build_only: bool = False):
    """f_W(x) = x + LN((SiLU(x W_gate) * x W_up) W_down) with per-row (or shared) W.

    W is read as fp32 masters, or -- when x and all three weights are bf16 -- as bf16 read
    copies (the reference casts W to the activation dtype for these matmuls, so a bf16
    copy yields the same operands at half the bytes).  With ``keys`` (B, T <= 64, D) bf16 the
    same weight reads also give keys W_up and keys W_gate, written to ``key_outputs``
    ((B, 64, d_ff) each, rows past T zero): the layer chain's products with the chunk-start
    copies (``ChunkChainRun.w_product_outputs``).

    One bf16 token per row only: ``x_norm`` = (weight, eps) reads out RMSNorm(x) with that
    weight instead of x (the decode step's q_norm), and ``row_counters`` (B,) int32, zero before
    the first call and left zero by every call, makes the readout a single launch (the
    LayerNorm runs in each row's last weight block); calls sharing counters must not overlap.
    ``sweep_reverse`` walks the weight rows in descending order (one-token rows only): successive
    calls over the same copies that alternate it start on what the infinity cache still holds
    from the previous call.  ``build_only`` returns (``uttt_readout_args``, workspace, the tensors they point at) without
    launching."""
    if x.dim() != 3:
        raise ValueError(f"x must be (B, T, D), got {tuple(x.shape)}")
    bsz, tokens, dim = x.shape
    code = _act_code(x.dtype)
    ff = w_up.shape[-1]
    if w_up.shape[-2:] != (dim, ff) or w_gate.shape[-2:] != (dim, ff) or w_down.shape[-2:] != (ff, dim):
        raise ValueError("fast weights do not match x's d_model")
    if dim % 64 or ff % 64 or dim > 4096:
        raise ValueError(f"d_model and d_ff must be multiples of 64 (d_model <= 4096); got {dim}, {ff}")
    dev = x.device
    _require_device(dev, w_up, w_gate, w_down, ln_weight, ln_bias)
    _forward_only(x, w_up, w_gate, w_down, ln_weight, ln_bias)
    x = _rows(x)
    bf16_copies = x.dtype == torch.bfloat16 and all(t.dtype == torch.bfloat16 for t in (w_up, w_gate, w_down))
    parts = [_read_weight(t, bsz, n, bf16_copies) for t, n in ((w_up, "w_up"), (w_gate, "w_gate"),
                                                               (w_down, "w_down"))]
    if len({p[1] for p in parts}) != 1:
        raise ValueError("fast weights must all be shared (batch 1) or all per-row")
    ln_w = ln_weight.to(torch.float32).contiguous()
    ln_b = ln_bias.to(torch.float32).contiguous()
    if out is None:
        out = torch.empty((bsz, tokens, dim), dtype=x.dtype, device=dev)
    lib = N.load_library()
    nbytes = lib.uttt_readout_workspace(bsz, tokens, dim, ff, code)
    if workspace is None or workspace.numel() < nbytes or workspace.device != dev:
        workspace = torch.empty(max(nbytes, 1), dtype=torch.uint8, device=dev)
    a = N.ReadoutArgs()
    a.batch, a.tokens, a.d_model, a.d_ff, a.act_dtype, a.eps = bsz, tokens, dim, ff, code, float(eps)
    a.w_dtype = N.DTYPE_BF16 if bf16_copies else N.DTYPE_F32
    a.x, a.x_row_stride = _p(x), x.stride(0)
    a.w_up, a.w_gate, a.w_down = (_p(p[0]) for p in parts)
    a.w_row_stride = parts[0][1]
    a.ln_weight, a.ln_bias = _p(ln_w), _p(ln_b)
    a.out, a.out_row_stride = _p(out), out.stride(0)
    if keys is not None:
        if not bf16_copies or tokens > 64:
            raise ValueError("key products need bf16 activations and weights and at most 64 tokens")
        if keys.shape != (bsz, tokens, dim) or keys.dtype != x.dtype:
            raise ValueError(f"keys must be ({bsz}, {tokens}, {dim}) {x.dtype}")
        _require_device(dev, keys)
        _forward_only(keys)
        keys = _rows(keys)
        if key_outputs is None or len(key_outputs) != 2 or any(
                t.shape != (bsz, 64, ff) or t.dtype != x.dtype or not t.is_contiguous() or t.device != dev
                for t in key_outputs):
            raise ValueError(f"key_outputs must be two contiguous ({bsz}, 64, {ff}) {x.dtype} tensors")
        a.keys, a.keys_row_stride = _p(keys), keys.stride(0)
        a.key_up_out, a.key_gate_out = _p(key_outputs[0]), _p(key_outputs[1])
    keep = None
    if x_norm is not None:
        keep = x_norm[0].detach().to(x.dtype).contiguous()
        if keep.shape != (dim,):
            raise ValueError(f"the x norm weight must be ({dim},)")
        _require_device(dev, keep)
        a.x_norm_weight, a.x_norm_eps = _p(keep), float(x_norm[1])
    if row_counters is not None:
        if row_counters.dtype != torch.int32 or row_counters.numel() < bsz or not row_counters.is_contiguous():
            raise ValueError(f"row_counters must be a contiguous int32 tensor of >= {bsz} entries")
        _require_device(dev, row_counters)
        a.row_counters = _p(row_counters)
    a.sweep_reverse = int(bool(sweep_reverse))
    if build_only:
        return a, workspace, (x, parts, ln_w, ln_b, out, keys, keep)
    with torch.cuda.device(dev):
        N.check(lib.uttt_swiglu_readout(C.byref(a), _p(workspace), workspace.numel(), _stream(dev)),
                "uttt_swiglu_readout")
    del keep
    return out


# ---------------------------------------------------------------------------
# RoPE + KV append (reference apply_rope + cache concat, model/uttt_layer.py:935-958, 1079-1102)
# ---------------------------------------------------------------------------

def rope_kv_append(q: Tensor, k: Tensor, v: Tensor, cos: Tensor, sin: Tensor, start_pos: int,
                   k_cache: Tensor, v_cache: Tensor, kv_offset: int, x: Optional[Tensor] = None,
                   x_eps: float = 0.0, build_only: bool = False):
    """Rotate ``q`` (B, T, H, hd) in place; write rotated ``k`` and ``v`` (B, T, Hkv, hd) into
    ``k_cache``/``v_cache`` (B, Hkv, L, hd) at time ``kv_offset + t``.  RoPE position of
    token t is ``start_pos + t``; cos/sin are fp32 (positions, hd) tables.  With ``x`` (B, T, D),
    the un-normalised input of a projection whose RMSNorm weight was folded into the weight,
    token t's q / k / v are first scaled by 1 / sqrt(mean(x_t^2) + x_eps).  ``build_only``
    returns the validated ``uttt_rope_append_args`` without launching."""
    bsz, tokens, heads, hd = q.shape
    hkv = k.shape[2]
    if k.shape != (bsz, tokens, hkv, hd) or v.shape != k.shape:
        raise ValueError("k/v must be (B, T, Hkv, hd) matching q")
    if k_cache.shape[0] != bsz or k_cache.shape[1] != hkv or k_cache.shape[3] != hd or v_cache.shape != k_cache.shape:
        raise ValueError("kv caches must be (B, Hkv, L, hd)")
    if kv_offset < 0 or kv_offset + tokens > k_cache.shape[2]:
        raise ValueError("kv_offset + tokens exceeds the cache length")
    if start_pos < 0:
        raise ValueError("RoPE start_pos must be nonnegative")
    if start_pos + tokens > cos.shape[0]:
        raise ValueError("positions exceed the RoPE table")
    if any(t.dtype != q.dtype for t in (k, v, k_cache, v_cache)):
        raise ValueError("q/k/v and the caches must share one dtype")
    if cos.dtype != torch.float32 or sin.dtype != torch.float32 or not cos.is_contiguous() or not sin.is_contiguous():
        raise ValueError("RoPE tables must be contiguous fp32")
    for t in (q, k, v, k_cache, v_cache):
        if t.stride(-1) != 1:
            raise ValueError("the head dimension must be contiguous")
    dev = q.device
    _require_device(dev, k, v, cos, sin, k_cache, v_cache)
    a = N.RopeAppendArgs()
    a.batch, a.tokens, a.n_heads, a.n_kv_heads, a.head_dim = bsz, tokens, heads, hkv, hd
    a.act_dtype = _act_code(q.dtype)
    a.start_pos, a.table_len = int(start_pos), cos.shape[0]
    a.cos_table, a.sin_table = _p(cos), _p(sin)
    a.q, a.q_stride_b, a.q_stride_t, a.q_stride_h = _p(q), q.stride(0), q.stride(1), q.stride(2)
    a.k, a.k_stride_b, a.k_stride_t, a.k_stride_h = _p(k), k.stride(0), k.stride(1), k.stride(2)
    a.v, a.v_stride_b, a.v_stride_t, a.v_stride_h = _p(v), v.stride(0), v.stride(1), v.stride(2)
    a.k_cache, a.v_cache = _p(k_cache), _p(v_cache)
    if k_cache.stride() != v_cache.stride():
        raise ValueError("k_cache and v_cache must share strides")
    a.kv_stride_b, a.kv_stride_h, a.kv_stride_t = k_cache.stride(0), k_cache.stride(1), k_cache.stride(2)
    a.kv_offset = int(kv_offset)
    if x is not None:
        if x.dim() != 3 or x.shape[:2] != (bsz, tokens) or x.dtype != q.dtype or x.stride(-1) != 1:
            raise ValueError("x must be (B, T, D) in q's dtype with a contiguous last dimension")
        if not x_eps > 0.0:
            raise ValueError("a folded norm needs eps > 0")
        _require_device(dev, x)
        a.x, a.x_stride_b, a.x_stride_t, a.x_dim, a.x_eps = _p(x), x.stride(0), x.stride(1), x.shape[2], float(x_eps)
    if build_only:
        return a
    lib = N.load_library()
    with torch.cuda.device(dev):
        N.check(lib.uttt_rope_kv_append(C.byref(a), _stream(dev)), "uttt_rope_kv_append")


# ---------------------------------------------------------------------------
# sliding-window attention (reference SDPA / FlexAttention dispatch, model/uttt_layer.py:1119-1165)
# ---------------------------------------------------------------------------

_ATTN_WS: dict = {}


def _attention_workspace(dev: torch.device, nbytes: int) -> Tensor:
    """The device's ``uttt_swa_prefill`` workspace (split partials, rewritten by every call),
    grown to at least ``nbytes``: one buffer serves every call made in stream order."""
    key = dev.index if dev.index is not None else torch.cuda.current_device()
    ws = _ATTN_WS.get(key)
    if ws is None or ws.numel() < nbytes:
        ws = torch.empty(max(nbytes, 1 << 20), dtype=torch.uint8, device=dev)
        _ATTN_WS[key] = ws
    return ws


def swa_prefill(q: Tensor, k: Tensor, v: Tensor, window: int, q_offset: int,
                out: Optional[Tensor] = None, kv_len: Optional[int] = None,
                workspace: Optional[Tensor] = None, build_only: bool = False):
    """q (B, H, Tq, hd), k/v (B, Hkv, Tkv, hd) (any strides with hd contiguous).  Query i sits
    at key index q_offset + i and sees key j iff 0 <= q_offset + i - j < window.  ``out``
    (B, H, Tq, hd) may be a strided view, e.g. of a (B, Tq, H, hd) buffer.  Without a
    ``workspace`` the call uses one zero-filled buffer per device, shared by every call: calls on
    concurrent streams must each pass their own.  ``build_only``
    returns the validated ``uttt_swa_prefill_args`` without launching (the operands must then
    be usable as they are, and ``out`` and ``workspace`` given)."""
    bsz, heads, tq, hd = q.shape
    hkv, tkv = k.shape[1], k.shape[2] if kv_len is None else kv_len
    if k.shape[0] != bsz or k.shape[3] != hd or v.shape != k.shape or heads % hkv:
        raise ValueError("k/v must be (B, Hkv, Tkv, hd) with n_heads a multiple of n_kv_heads")
    if hd not in (64, 128):
        raise ValueError(f"head_dim must be 64 or 128 on the HIP path, got {hd}")
    if q_offset < 0 or q_offset + tq > tkv or tkv > k.shape[2]:
        raise ValueError("queries must index keys inside the kv range")
    if window < 1:
        raise ValueError("window must be >= 1")
    if k.dtype != q.dtype or v.dtype != q.dtype:
        raise ValueError("q/k/v must share one dtype")
    vec = 16 // q.element_size()
    fixed = []
    for t in (q, k, v):
        if t.stride(-1) != 1:
            raise ValueError("the head dimension must be contiguous")
        if t.data_ptr() % 16 or any(st % vec for st in t.stride()[:3]):
            if build_only:
                raise ValueError("q/k/v need 16-byte aligned rows for a prepared call")
            t = t.contiguous()  # the kernel reads 16-byte vectors
        fixed.append(t)
    q, k, v = fixed
    dev = q.device
    _require_device(dev, k, v)
    _forward_only(q, k, v)
    if out is None:
        out = torch.empty((bsz, tq, heads, hd), dtype=q.dtype, device=dev).transpose(1, 2)
    elif out.shape != q.shape or out.dtype != q.dtype or out.stride(-1) != 1:
        raise ValueError("out must match q's shape and dtype with hd contiguous")
    a = N.SwaPrefillArgs()
    a.batch, a.n_heads, a.n_kv_heads, a.q_len, a.kv_len, a.head_dim = bsz, heads, hkv, tq, tkv, hd
    a.q_offset, a.window, a.act_dtype, a.scale = int(q_offset), int(window), _act_code(q.dtype), 1.0 / math.sqrt(hd)
    a.q, a.q_stride_b, a.q_stride_h, a.q_stride_t = _p(q), q.stride(0), q.stride(1), q.stride(2)
    a.k, a.k_stride_b, a.k_stride_h, a.k_stride_t = _p(k), k.stride(0), k.stride(1), k.stride(2)
    a.v, a.v_stride_b, a.v_stride_h, a.v_stride_t = _p(v), v.stride(0), v.stride(1), v.stride(2)
    a.out, a.o_stride_b, a.o_stride_h, a.o_stride_t = _p(out), out.stride(0), out.stride(1), out.stride(2)
    lib = N.load_library()
    nbytes = lib.uttt_swa_prefill_workspace(bsz, heads, tq, tkv, hd, window)
    if workspace is None:
        workspace = _attention_workspace(dev, nbytes)
    elif workspace.numel() < nbytes or workspace.device != dev:
        raise ValueError(f"the attention workspace must hold {nbytes} bytes on {dev}")
    a.workspace, a.workspace_bytes = _p(workspace), workspace.numel()
    if build_only:
        return a
    with torch.cuda.device(dev):
        N.check(lib.uttt_swa_prefill(C.byref(a), _stream(dev)), "uttt_swa_prefill")
    return out


def swa_decode(q: Tensor, k_new: Tensor, v_new: Tensor, k_ring: Tensor, v_ring: Tensor, positions: Tensor,
               cos: Optional[Tensor] = None, sin: Optional[Tensor] = None, out: Optional[Tensor] = None,
               workspace: Optional[Tensor] = None) -> Tensor:
    """One decode step for N requests.  q (N, H, hd), k_new/v_new (N, Hkv, hd) (un-rotated when
    tables are given), rings (N, Hkv, W, hd), positions (N,) int64 on the device."""
    n, heads, hd = q.shape
    hkv, window = k_ring.shape[1], k_ring.shape[2]
    if k_new.shape != (n, hkv, hd) or v_new.shape != k_new.shape:
        raise ValueError("k_new / v_new must be (N, Hkv, hd)")
    if k_ring.shape != (n, hkv, window, hd) or v_ring.shape != k_ring.shape:
        raise ValueError("rings must be (N, Hkv, W, hd)")
    if positions.shape != (n,) or positions.dtype != torch.int64:
        raise ValueError("positions must be an int64 (N,) device tensor")
    if hd not in (64, 128) or heads % hkv or heads // hkv > 8:
        raise ValueError("head_dim must be 64/128 and n_heads / n_kv_heads <= 8")
    if any(t.dtype != q.dtype for t in (k_new, v_new, k_ring, v_ring)):
        raise ValueError("q, new k/v and rings must share one dtype")
    for t, shape_tail in ((q, (heads, hd)), (k_new, (hkv, hd)), (v_new, (hkv, hd)), (k_ring, (hkv, window, hd))):
        if not t[0].is_contiguous():
            raise ValueError("per-request slices of q, k_new, v_new and the rings must be contiguous")
    if k_new.stride(0) != v_new.stride(0) or k_ring.stride(0) != v_ring.stride(0):
        raise ValueError("k and v tensors must share their request stride")
    dev = q.device
    _require_device(dev, k_new, v_new, k_ring, v_ring, positions, cos, sin)
    if (cos is None) != (sin is None):
        raise ValueError("cos and sin must both be given or both omitted")
    if out is None:
        out = torch.empty_like(q)
    a = N.SwaDecodeArgs()
    a.n_req, a.n_heads, a.n_kv_heads, a.head_dim, a.window = n, heads, hkv, hd, window
    a.act_dtype, a.scale = _act_code(q.dtype), 1.0 / math.sqrt(hd)
    a.positions = _p(positions)
    a.cos_table, a.sin_table = _p(cos), _p(sin)
    a.table_len = 0 if cos is None else cos.shape[0]
    a.q, a.q_stride_n = _p(q), q.stride(0)
    a.k_new, a.v_new, a.kv_new_stride_n = _p(k_new), _p(v_new), k_new.stride(0)
    a.k_ring, a.v_ring, a.ring_stride_n = _p(k_ring), _p(v_ring), k_ring.stride(0)
    a.out, a.o_stride_n = _p(out), out.stride(0)
    lib = N.load_library()
    nbytes = lib.uttt_swa_decode_workspace(n, heads, hkv, hd, window)
    if workspace is None or workspace.numel() < nbytes or workspace.device != dev:
        workspace = torch.empty(max(nbytes, 1), dtype=torch.uint8, device=dev)
    a.workspace, a.workspace_bytes = _p(workspace), workspace.numel()
    with torch.cuda.device(dev):
        N.check(lib.uttt_swa_decode(C.byref(a), _stream(dev)), "uttt_swa_decode")
    return out


# ---------------------------------------------------------------------------
# elastic pull and drift (reference SharedFastWeightPool.apply_elastic_pull / compute_drift,
# model/uttt_layer.py:773-874)
# ---------------------------------------------------------------------------

def _pull_operands(w: Sequence[Tensor], w0: Sequence[Tensor]):
    if len(w) != 3 or len(w0) != 3:
        raise ValueError("expected (W_up, W_gate, W_down) and three base matrices")
    bsz, dim, ff = w[0].shape
    if w[1].shape != (bsz, dim, ff) or w[2].shape != (bsz, ff, dim):
        raise ValueError("fast weights must be (B, D, F), (B, D, F), (B, F, D)")
    if w0[0].shape != (dim, ff) or w0[1].shape != (dim, ff) or w0[2].shape != (ff, dim):
        raise ValueError("base weights must be (D, F), (D, F), (F, D)")
    dev = w[0].device
    _require_device(dev, *w, *w0)
    ws = [_state(t, "w") for t in w]
    bases = [t.detach().to(torch.float32).contiguous() for t in w0]
    return bsz, dim, ff, dev, ws, bases


def elastic_pull(w: Sequence[Tensor], w0: Sequence[Tensor], anchor_lambda: float,
                 max_drift_ratio: Optional[float] = None, out: Optional[Sequence[Tensor]] = None):
    """(1 - lambda) W + lambda W_0 with the optional per-row drift ceiling; new fp32 tensors
    unless ``out`` (which may be ``w`` itself) is given."""
    bsz, dim, ff, dev, ws, bases = _pull_operands(w, w0)
    outs = [torch.empty_like(t) for t in ws] if out is None else list(out)
    lib = N.load_library()
    workspace = torch.empty(lib.uttt_elastic_pull_workspace(bsz), dtype=torch.uint8, device=dev)
    a = N.ElasticPullArgs()
    a.batch, a.d_model, a.d_ff = bsz, dim, ff
    a.anchor_lambda = float(anchor_lambda)
    a.max_drift_ratio = float(max_drift_ratio) if max_drift_ratio is not None and max_drift_ratio > 0 else 0.0
    a.w_up, a.w_gate, a.w_down = (_p(t) for t in ws)
    a.w0_up, a.w0_gate, a.w0_down = (_p(t) for t in bases)
    a.out_up, a.out_gate, a.out_down = (_p(t) for t in outs)
    with torch.cuda.device(dev):
        N.check(lib.uttt_elastic_pull(C.byref(a), _p(workspace), workspace.numel(), _stream(dev)),
                "uttt_elastic_pull")
    return tuple(outs)


def drift_sums(w: Sequence[Tensor], w0: Sequence[Tensor]) -> Tensor:
    """Device fp32 (6,): sum over rows of |W_m - W0_m|^2 per matrix, then |W0_m|^2 per matrix."""
    bsz, dim, ff, dev, ws, bases = _pull_operands(w, w0)
    lib = N.load_library()
    workspace = torch.empty(lib.uttt_elastic_pull_workspace(bsz), dtype=torch.uint8, device=dev)
    out = torch.empty(6, dtype=torch.float32, device=dev)
    with torch.cuda.device(dev):
        N.check(lib.uttt_fast_weight_drift(bsz, dim, ff, *(_p(t) for t in ws), *(_p(t) for t in bases), _p(out),
                                           _p(workspace), workspace.numel(), _stream(dev)),
                "uttt_fast_weight_drift")
    return out
