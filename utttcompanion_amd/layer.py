"""Drop-in counterparts of the reference's ``model/uttt_layer.py`` modules on the HIP path.

Class names, constructor arguments, parameter names/shapes (so ``state_dict`` keys
match the reference checkpoints), initial draws and call signatures follow the
reference.  The arithmetic of the hot path runs in ``libuttt_amd.so``:

* ``fused_chunk_ttt_step`` / ``SharedFastWeightPool.chunk_step`` -> ``uttt_chunk_update``
* ``swiglu_fast_forward`` / ``forward_readout``               -> ``uttt_swiglu_readout``
* ``SlidingWindowAttention.forward``                            -> ``uttt_rope_kv_append`` + ``uttt_swa_prefill``
* ``apply_elastic_pull`` / ``compute_drift``                    -> ``uttt_elastic_pull`` / ``uttt_fast_weight_drift``

Dense slow-weight projections (``F.linear``) and RMSNorm stay on PyTorch-ROCm
(hipBLASLt GEMMs on the GPU).  Everything is forward-only; CPU tensors are rejected.
"""
from __future__ import annotations

import math
from dataclasses import dataclass, field
from typing import Dict, List, Optional, Sequence, Tuple

import torch
import torch.nn as nn
import torch.nn.functional as F

from . import kernels as K

Tensor = torch.Tensor
_STATE_NAMES = ("w_up", "w_gate", "w_down", "s_up", "s_gate", "s_down")

# Longest chunk one fast-weight write takes (uttt_chunk_update, UTTT_MAX_UPDATE_TOKENS): the
# reference's shipped configs use 128 and 512.  Chunks of up to 64 tokens also run the fused layer
# chain and the resident loop.  Frozen reads (update_fast_weights=False, decoding) do not chunk
# and take any chunk_size.
MAX_WRITE_CHUNK = 512


def require_write_chunk(chunk_size: int) -> None:
    """Refuse a fast-weight write with chunks the kernels do not take, before any work (one write
    per chunk, as the reference's chunk loop does; a longer chunk is never split into several
    writes)."""
    if not 1 <= int(chunk_size) <= MAX_WRITE_CHUNK:
        raise ValueError(f"chunk_size={chunk_size}: fast-weight writes on the HIP path take chunks of 1.."
                         f"{MAX_WRITE_CHUNK} tokens; frozen reads (update_fast_weights=False, decoding) take "
                         f"any chunk_size")


# ==============================================================================
# Fast-weight state (reference model/uttt_layer.py:59-205)
# ==============================================================================

@dataclass
class FastWeightState:
    """Per-row fast weights W = {W_up, W_gate, W_down} and momentum S (fp32 masters).

    Shapes: w_up, w_gate, s_up, s_gate (B, D, F); w_down, s_down (B, F, D);
    ln_weight, ln_bias (D,).
    """
    w_up: Tensor
    w_gate: Tensor
    w_down: Tensor
    s_up: Tensor
    s_gate: Tensor
    s_down: Tensor
    ln_weight: Tensor
    ln_bias: Tensor
    step: int = 0
    last_surprise_loss: float = 0.0
    surprise_history: List[float] = field(default_factory=list)
    _shared_readonly: bool = field(default=False, repr=False)
    # versioned activation-dtype read copies (SharedFastWeightPool.inference_read_weights and
    # the fused inference readout); disposable, never part of a persona payload
    _packed_up_gate: Optional[Tensor] = field(default=None, repr=False)
    _read_w_down: Optional[Tensor] = field(default=None, repr=False)
    _packed_key: Optional[tuple] = field(default=None, repr=False)
    _read_copies: Optional[Tuple[Tensor, Tensor, Tensor]] = field(default=None, repr=False)
    _read_key: Optional[tuple] = field(default=None, repr=False)

    def tensors(self) -> Tuple[Tensor, ...]:
        return tuple(getattr(self, n) for n in _STATE_NAMES)

    def clone(self, detach: bool = False) -> "FastWeightState":
        cp = (lambda t: t.detach().clone()) if detach else (lambda t: t.clone())
        return FastWeightState(*(cp(t) for t in self.tensors()), cp(self.ln_weight), cp(self.ln_bias),
                               int(self.step), float(self.last_surprise_loss), list(self.surprise_history[-100:]))

    def detach(self) -> "FastWeightState":
        return self.clone(detach=True)

    def to(self, device=None, dtype=None, non_blocking: bool = True) -> "FastWeightState":
        kw = {"non_blocking": non_blocking}
        if device is not None:
            kw["device"] = device
        if dtype is not None:
            kw["dtype"] = dtype
        return FastWeightState(*(t.to(**kw) for t in self.tensors()), self.ln_weight.to(**kw),
                               self.ln_bias.to(**kw), self.step, self.last_surprise_loss,
                               list(self.surprise_history))

    def ensure_batch_size(self, batch_size: int) -> "FastWeightState":
        """Broadcast a batch-1 state to ``batch_size`` rows (reference :142-163)."""
        cur = self.w_up.shape[0]
        if cur == batch_size:
            return self
        if cur == 1 and batch_size > 1:
            return FastWeightState(*(t.expand(batch_size, -1, -1).contiguous() for t in self.tensors()),
                                   self.ln_weight, self.ln_bias, self.step, self.last_surprise_loss,
                                   list(self.surprise_history))
        raise ValueError(f"Cannot broadcast FastWeightState from batch_size={cur} to {batch_size}")

    def to_state_dict(self) -> Dict[str, object]:
        """Persona payload with the reference's keys (reference :165-179)."""
        out = {n: getattr(self, n).detach().cpu() for n in _STATE_NAMES}
        out.update(ln_weight=self.ln_weight.detach().cpu(), ln_bias=self.ln_bias.detach().cpu(),
                   step=self.step, last_surprise_loss=self.last_surprise_loss,
                   surprise_history=list(self.surprise_history[-100:]))
        return out

    @classmethod
    def from_state_dict(cls, state_dict: Dict[str, object], device=None, dtype=None) -> "FastWeightState":
        state = cls(*(state_dict[n] for n in _STATE_NAMES), state_dict["ln_weight"], state_dict["ln_bias"],
                    int(state_dict.get("step", 0)), float(state_dict.get("last_surprise_loss", 0.0)),
                    list(state_dict.get("surprise_history", [])))
        if device is not None or dtype is not None:
            state = state.to(device=device, dtype=dtype)
        return state


# ==============================================================================
# Operators (reference :211-534)
# ==============================================================================

def swiglu_fast_forward(x: Tensor, w_up: Tensor, w_gate: Tensor, w_down: Tensor, ln_weight: Tensor,
                        ln_bias: Tensor, eps: float = 1e-5) -> Tensor:
    """f_W(x) = x + LN((SiLU(x W_gate) * (x W_up)) W_down) on the GPU (reference :211-247)."""
    return K.swiglu_readout(x, w_up, w_gate, w_down, ln_weight, ln_bias, eps)


def fused_chunk_ttt_step(q_chunk: Tensor, k_chunk: Tensor, v_chunk: Tensor, eta_chunk: Tensor,
                         alpha_chunk: Tensor, w_up: Tensor, w_gate: Tensor, w_down: Tensor,
                         s_up: Tensor, s_gate: Tensor, s_down: Tensor, ln_weight: Tensor, ln_bias: Tensor,
                         token_mask: Optional[Tensor], momentum_beta: float, max_inner_grad_norm: float,
                         normalize_by_dim: bool, eps: float, read_w_up: Optional[Tensor] = None,
                         read_w_gate: Optional[Tensor] = None,
                         read_w_down: Optional[Tensor] = None) -> Tuple[Tensor, ...]:
    """Gradient + clip + momentum + decay + masked select + causal readout for one chunk
    (reference :414-534).  Returns the reference's 8-tuple; new state tensors are fp32."""
    return K.chunk_update(q_chunk, k_chunk, v_chunk, eta_chunk, alpha_chunk, w_up, w_gate, w_down,
                          s_up, s_gate, s_down, ln_weight, ln_bias, token_mask, momentum_beta,
                          max_inner_grad_norm, normalize_by_dim, eps, read_w_up, read_w_gate, read_w_down)


# ==============================================================================
# Shared fast-weight pool (reference :541-874)
# ==============================================================================

class SharedFastWeightPool(nn.Module):
    """Meta-initialised W_0 plus the chunk-wise update / readout entry points."""

    def __init__(self, d_model: int, d_ff: int, momentum_beta: float = 0.90, max_inner_grad_norm: float = 1.0,
                 normalize_loss_by_dim: bool = False, rms_norm_eps: float = 1e-5) -> None:
        super().__init__()
        # set by uTTTModel.prepare_for_inference: frozen readouts read versioned
        # activation-dtype copies of W instead of the fp32 masters (reference :677-689)
        self.fused_inference_readout = False
        self.d_model = d_model
        self.d_ff = d_ff
        self.momentum_beta = momentum_beta
        self.max_inner_grad_norm = max_inner_grad_norm
        self.normalize_loss_by_dim = normalize_loss_by_dim
        self.eps = rms_norm_eps
        std_in = 1.0 / math.sqrt(d_model)
        std_out = 1.0 / math.sqrt(d_ff)
        self.w_up_init = nn.Parameter(torch.randn(d_model, d_ff) * std_in)
        self.w_gate_init = nn.Parameter(torch.randn(d_model, d_ff) * std_in)
        self.w_down_init = nn.Parameter(torch.randn(d_ff, d_model) * (0.1 * std_out))
        self.ln_weight = nn.Parameter(torch.ones(d_model))
        self.ln_bias = nn.Parameter(torch.zeros(d_model))

    def base_weights(self) -> Tuple[Tensor, Tensor, Tensor]:
        return self.w_up_init, self.w_gate_init, self.w_down_init

    def init_state(self, batch_size: int = 1, device=None, dtype=None, detach: bool = False) -> FastWeightState:
        """W_0 expanded to ``batch_size`` rows with S = 0 (reference :582-632)."""
        dev = device if device is not None else self.w_up_init.device
        dt = dtype if dtype is not None else self.w_up_init.dtype
        ws = [t.detach().to(device=dev, dtype=dt).unsqueeze(0).expand(batch_size, -1, -1).clone()
              for t in self.base_weights()]
        return FastWeightState(ws[0], ws[1], ws[2], *(torch.zeros_like(w) for w in ws),
                               self.ln_weight.detach().to(device=dev, dtype=dt).clone(),
                               self.ln_bias.detach().to(device=dev, dtype=dt).clone())

    def readonly_state(self, batch_size=1, device=None, dtype=None, detach=False) -> FastWeightState:
        """Stride-0 views of W_0 for frozen reads (reference :634-646)."""
        def view(t):
            return t.detach().to(device=device, dtype=dtype)
        up, gate, down = (view(t).unsqueeze(0).expand(batch_size, -1, -1) for t in self.base_weights())
        zero = up.new_zeros(())
        return FastWeightState(up, gate, down, zero.expand_as(up), zero.expand_as(gate), zero.expand_as(down),
                               view(self.ln_weight), view(self.ln_bias), _shared_readonly=True)

    @staticmethod
    def _read_key(state: FastWeightState, dtype: torch.dtype, device) -> tuple:
        weights = (state.w_up, state.w_gate, state.w_down)
        if torch.is_grad_enabled() or any(t.is_inference() for t in weights):
            raise ValueError("Inference read caches require no-grad, version-tracked weights")
        return (dtype, torch.device(device), tuple((id(t), t.data_ptr(), t._version, t.device, t.dtype,
                                                    tuple(t.shape)) for t in weights))

    def inference_read_weights(self, state: FastWeightState, dtype: torch.dtype,
                               device) -> Tuple[Tensor, Tensor]:
        """Versioned read copies in the reference's packed layout (reference :648-668):
        ``(cat(W_up, W_gate) (B, D, 2F), W_down (B, F, D))`` in ``dtype`` on ``device``, rebuilt
        when any master's storage, version, dtype or shape changes.  Read-only for the caller;
        needs no-grad mode and version-tracked (non-inference) tensors, like the reference."""
        key = self._read_key(state, dtype, device)
        if state._packed_up_gate is None or state._read_w_down is None or state._packed_key != key:
            state._packed_up_gate = torch.cat((state.w_up.to(device=device, dtype=dtype),
                                               state.w_gate.to(device=device, dtype=dtype)), dim=-1)
            state._read_w_down = state.w_down.to(device=device, dtype=dtype)
            state._packed_key = key
        return state._packed_up_gate, state._read_w_down

    def inference_read_copies(self, state: FastWeightState, dtype: torch.dtype,
                              device) -> Tuple[Tensor, Tensor, Tensor]:
        """The same versioned copies in the layout ``uttt_swiglu_readout`` reads:
        ``(W_up (B, D, F), W_gate (B, D, F), W_down (B, F, D))``, contiguous, in ``dtype``."""
        key = self._read_key(state, dtype, device)
        if state._read_copies is None or state._read_key != key:
            state._read_copies = tuple(t.to(device=device, dtype=dtype).contiguous()
                                       for t in (state.w_up, state.w_gate, state.w_down))
            state._read_key = key
        return state._read_copies

    def forward_readout(self, x: Tensor, state: FastWeightState) -> Tensor:
        """Frozen readout f_W(x) (reference :670-695); shared W_0 views are read once per launch.
        With ``fused_inference_readout`` (eval, no grad, 16-bit activations) the readout reads
        the state's versioned activation-dtype copies: the same operands (the reference casts W
        to x's dtype for these products) at half the bytes of the fp32 masters."""
        state = state.ensure_batch_size(x.shape[0])
        weights = (state.w_up, state.w_gate, state.w_down)
        if (self.fused_inference_readout and not self.training and not torch.is_grad_enabled()
                and x.dtype != torch.float32 and not state._shared_readonly
                and not any(t.is_inference() for t in weights)):
            weights = self.inference_read_copies(state, x.dtype, x.device)
        return K.swiglu_readout(x, *weights, state.ln_weight, state.ln_bias, self.eps)

    def chunk_step(self, state: FastWeightState, q_chunk: Tensor, k_chunk: Tensor, v_chunk: Tensor,
                   eta_chunk: Tensor, alpha_chunk: Tensor, token_mask: Optional[Tensor] = None,
                   update_fast_weights: bool = True, read_state: Optional[FastWeightState] = None,
                   out_state: Optional[Sequence[Tensor]] = None) -> Tuple[Tensor, FastWeightState, Tensor]:
        """One chunk: readout through ``read_state`` (default: the incoming cursor) and the
        write W_t -> W_{t+1} (reference :697-771).  ``out_state`` optionally names the six
        fp32 buffers receiving the new state (they may be the cursor's own tensors)."""
        bsz = q_chunk.shape[0]
        state = state.ensure_batch_size(bsz)
        read = state if read_state is None else read_state.ensure_batch_size(bsz)
        if not update_fast_weights:
            out = self.forward_readout(q_chunk, read)
            return out, state, q_chunk.new_zeros((), dtype=torch.float32)
        res = K.chunk_update(
            q_chunk, k_chunk, v_chunk, eta_chunk, alpha_chunk, *state.tensors(), state.ln_weight, state.ln_bias,
            token_mask, self.momentum_beta, float(self.max_inner_grad_norm or 0.0), self.normalize_loss_by_dim,
            self.eps, *((None, None, None) if read_state is None else (read.w_up, read.w_gate, read.w_down)),
            out_state=out_state)
        new_state = FastWeightState(*res[1:7], state.ln_weight, state.ln_bias, state.step + 1,
                                    state.last_surprise_loss, state.surprise_history)
        return res[0], new_state, res[7]

    def chunk_loop(self, state: FastWeightState, q: Tensor, k: Tensor, v: Tensor, eta: Tensor, alpha: Tensor,
                   token_mask: Optional[Tensor], chunk_size: int) -> Optional[Tuple[Tensor, FastWeightState, Tensor]]:
        """Every ``chunk_step`` of one layer's forward (write, readout through each chunk's own
        pre-update state) in one launch, when ``K.layer_update_resident`` takes the operands
        (one fp32 row; see ``K.resident_update_eligible``); None otherwise.  Returns the
        readout, the state after the last chunk and the mean chunk surprise, as the chunk loop
        of the reference's uTTTLayer.forward does (reference :1451-1478)."""
        state = state.ensure_batch_size(q.shape[0])
        if not K.resident_update_eligible(q, state.w_up, chunk_size):
            return None
        res = K.layer_update_resident(q, k, v, eta, alpha, *state.tensors(), state.ln_weight, state.ln_bias,
                                      token_mask, self.momentum_beta, float(self.max_inner_grad_norm or 0.0),
                                      self.normalize_loss_by_dim, self.eps, chunk_size)
        n_chunks = res[7].shape[0]
        new_state = FastWeightState(*res[1:7], state.ln_weight, state.ln_bias, state.step + n_chunks,
                                    state.last_surprise_loss, state.surprise_history)
        return res[0], new_state, res[7].sum() / n_chunks

    @torch.no_grad()
    def apply_elastic_pull(self, state: FastWeightState, anchor_lambda: float = 0.02,
                           max_drift_ratio: Optional[float] = None) -> FastWeightState:
        """W <- (1 - lambda) W + lambda W_0 with an optional per-row drift ceiling (reference :773-832)."""
        if anchor_lambda <= 0.0 and max_drift_ratio is None:
            return state
        w = K.elastic_pull((state.w_up, state.w_gate, state.w_down), self.base_weights(), anchor_lambda,
                           max_drift_ratio)
        return FastWeightState(*w, state.s_up, state.s_gate, state.s_down, state.ln_weight, state.ln_bias,
                               state.step, state.last_surprise_loss, list(state.surprise_history))

    @torch.no_grad()
    def compute_drift(self, state: FastWeightState) -> Dict[str, float]:
        """Frobenius drift of W from W_0 (reference :834-874); one device-to-host copy."""
        sums = K.drift_sums((state.w_up, state.w_gate, state.w_down), self.base_weights()).tolist()
        d_up, d_gate, d_down, b_up, b_gate, b_down = (math.sqrt(max(x, 0.0)) for x in sums)
        total = math.sqrt(d_up ** 2 + d_gate ** 2 + d_down ** 2)
        base = math.sqrt(b_up ** 2 + b_gate ** 2 + b_down ** 2) + 1e-8
        return {"drift_frobenius": total, "base_frobenius": base, "drift_pct": total / base * 100.0,
                "w_up_drift": d_up, "w_gate_drift": d_gate, "w_down_drift": d_down,
                "w_up_drift_pct": d_up / (b_up + 1e-8) * 100.0,
                "w_gate_drift_pct": d_gate / (b_gate + 1e-8) * 100.0,
                "w_down_drift_pct": d_down / (b_down + 1e-8) * 100.0,
                "step": state.step, "last_surprise_loss": state.last_surprise_loss}


# ==============================================================================
# Norm, RoPE, sliding-window attention (reference :881-1168)
# ==============================================================================

class RMSNorm(nn.Module):
    """Root-mean-square norm via ``F.rms_norm`` (reference :881-896)."""

    def __init__(self, dim: int, eps: float = 1e-5) -> None:
        super().__init__()
        self.eps = eps
        self.weight = nn.Parameter(torch.ones(dim))

    def forward(self, x: Tensor) -> Tensor:
        return F.rms_norm(x, (self.weight.shape[0],), self.weight.to(x.dtype), self.eps)


class RotaryEmbedding(nn.Module):
    """fp32 cos/sin tables, extended on demand keeping existing rows (reference :899-943)."""

    def __init__(self, head_dim: int, max_seq_len: int = 4096, theta: float = 10000.0) -> None:
        super().__init__()
        self.head_dim = head_dim
        self.theta = float(theta)
        self.cos_cached: Optional[Tensor] = None
        self.sin_cached: Optional[Tensor] = None
        self._build_cache(max_seq_len, torch.device("cpu"))

    def _build_cache(self, seq_len: int, device: torch.device) -> None:
        old_len = 0 if self.cos_cached is None else self.cos_cached.shape[0]
        if self.cos_cached is not None and self.cos_cached.device != device:
            self.cos_cached = self.cos_cached.to(device)
            self.sin_cached = self.sin_cached.to(device)
        if seq_len <= old_len:
            return
        inv_freq = 1.0 / (self.theta ** (torch.arange(0, self.head_dim, 2, device=device, dtype=torch.float32)
                                         / self.head_dim))
        t = torch.arange(old_len, seq_len, device=device, dtype=torch.float32)
        freqs = torch.outer(t, inv_freq)
        emb = torch.cat((freqs, freqs), dim=-1)
        cos, sin = emb.cos(), emb.sin()
        if self.cos_cached is not None:
            cos = torch.cat((self.cos_cached, cos), dim=0)
            sin = torch.cat((self.sin_cached, sin), dim=0)
        self.cos_cached, self.sin_cached = cos.contiguous(), sin.contiguous()

    def tables(self, length: int, device: torch.device) -> Tuple[Tensor, Tensor]:
        """fp32 (>= length, head_dim) tables on ``device``."""
        if self.cos_cached.device != device or self.cos_cached.shape[0] < length:
            self._build_cache(max(length + 512, self.cos_cached.shape[0]), device)
        return self.cos_cached, self.sin_cached

    def forward(self, x: Tensor, start_pos: int = 0) -> Tuple[Tensor, Tensor]:
        if start_pos < 0:
            raise ValueError("RoPE start_pos must be nonnegative")
        seq = x.shape[2]
        cos, sin = self.tables(start_pos + seq, x.device)
        return (cos[start_pos:start_pos + seq].to(x.dtype)[None, None],
                sin[start_pos:start_pos + seq].to(x.dtype)[None, None])


def apply_rope(q: Tensor, k: Tensor, cos: Tensor, sin: Tensor) -> Tuple[Tensor, Tensor]:
    """Reference-compatible functional RoPE on (B, H, T, hd) tensors (reference :946-958).

    The attention path does not call this: it rotates inside ``uttt_rope_kv_append``.
    """
    def rot(x):
        half = x.shape[-1] // 2
        return torch.cat((-x[..., half:], x[..., :half]), dim=-1)
    return q * cos + rot(q) * sin, k * cos + rot(k) * sin


class SlidingWindowAttention(nn.Module):
    """Local sliding-window GQA with RoPE and a bounded KV cache (reference :961-1168)."""

    def __init__(self, d_model: int, n_heads: int, n_kv_heads: int, window_size: int = 512,
                 max_seq_len: int = 4096, rope_theta: float = 10000.0, dropout: float = 0.0) -> None:
        super().__init__()
        if d_model % n_heads or n_heads % n_kv_heads:
            raise ValueError("d_model must divide by n_heads and n_heads by n_kv_heads")
        self.d_model = d_model
        self.n_heads = n_heads
        self.n_kv_heads = n_kv_heads
        self.n_rep = n_heads // n_kv_heads
        self.head_dim = d_model // n_heads
        self.window_size = window_size
        self.dropout = dropout
        self.wq = nn.Linear(d_model, n_heads * self.head_dim, bias=False)
        self.wk = nn.Linear(d_model, n_kv_heads * self.head_dim, bias=False)
        self.wv = nn.Linear(d_model, n_kv_heads * self.head_dim, bias=False)
        self.wo = nn.Linear(n_heads * self.head_dim, d_model, bias=False)
        self.rope = RotaryEmbedding(self.head_dim, max_seq_len=max_seq_len, theta=rope_theta)
        # [wq; wk; wv] as one weight, outside the checkpoint keys (reference :1000-1001)
        self.register_buffer("_packed_qkv", None, persistent=False)
        self._packed_qkv_key = None

    def _projection_key(self):
        """Identity of the three projection weights; None for inference tensors (no version)."""
        ws = (self.wq.weight, self.wk.weight, self.wv.weight)
        if any(t.is_inference() for t in ws):
            return None
        return tuple((id(t), t.data_ptr(), t._version, t.device, t.dtype) for t in ws)

    @torch.no_grad()
    def prepare_for_inference(self) -> None:
        """Build (or refresh) ``_packed_qkv`` (reference :1008-1018)."""
        key = self._projection_key()
        if key is None:
            self._packed_qkv = None
            self._packed_qkv_key = None
            return
        if self._packed_qkv is None or key != self._packed_qkv_key:
            self._packed_qkv = torch.cat([t.detach() for t in (self.wq.weight, self.wk.weight, self.wv.weight)],
                                         dim=0)
            self._packed_qkv_key = key

    def train(self, mode: bool = True):
        if mode:  # reference :1020-1024: packs are dropped when training resumes
            self._packed_qkv = None
            self._packed_qkv_key = None
        return super().train(mode)

    def packed_qkv(self) -> Tensor:
        """[wq; wk; wv] as one (H + 2 Hkv) hd x D weight (``_packed_qkv``), rebuilt when any
        weight changes."""
        key = self._projection_key()
        if key is None:
            return torch.cat([t.detach() for t in (self.wq.weight, self.wk.weight, self.wv.weight)], dim=0)
        if self._packed_qkv is None or self._packed_qkv_key != key:
            self.prepare_for_inference()
        return self._packed_qkv

    def packed_qkv_folded(self, norm: "RMSNorm") -> Tensor:
        """The packed QKV weight with an input RMSNorm's weight folded into its columns
        (W diag(g), formed in fp32 and rounded once), rebuilt when any of them changes."""
        w = self.packed_qkv()
        key = (self._packed_qkv_key, norm.weight.data_ptr(), norm.weight._version, norm.weight.dtype)
        if getattr(self, "_fold_key", None) != key:
            self._fold = (w.float() * norm.weight.detach().float()[None, :]).to(w.dtype)
            self._fold_key = key
        return self._fold

    def project(self, x: Tensor, start_pos: int, k_buf: Tensor, v_buf: Tensor, kv_offset: int,
                norm: Optional["RMSNorm"] = None) -> Tensor:
        """QKV projection + RoPE; writes rotated k / v into the KV buffers at ``kv_offset`` and
        returns rotated q as a (B, T, H, hd) view.  With ``norm``, ``x`` is the un-normalised
        input of that RMSNorm: its weight is folded into the projection weight and the per-token
        1 / rms scale is applied inside the RoPE kernel, so the norm needs no launch of its own."""
        bsz, seq, _ = x.shape
        hd, h, hkv = self.head_dim, self.n_heads, self.n_kv_heads
        w = self.packed_qkv() if norm is None else self.packed_qkv_folded(norm)
        qkv = F.linear(x, w.to(x.dtype)).view(bsz, seq, h + 2 * hkv, hd)
        q, k, v = qkv[:, :, :h], qkv[:, :, h:h + hkv], qkv[:, :, h + hkv:]
        cos, sin = self.rope.tables(start_pos + seq, x.device)
        K.rope_kv_append(q, k, v, cos, sin, start_pos, k_buf, v_buf, kv_offset,
                         x=None if norm is None else x, x_eps=0.0 if norm is None else norm.eps)
        return q

    def forward(self, x: Tensor, kv_cache: Optional[Tuple[Tensor, Tensor]] = None,
                start_pos: int = 0) -> Tuple[Tensor, Tuple[Tensor, Tensor]]:
        """Attention over the window; returns (out, cache of the last <= window rotated k/v)."""
        if self.training and torch.is_grad_enabled():
            raise ValueError("the HIP attention path is inference-only")
        bsz, seq, _ = x.shape
        hd, hkv, win = self.head_dim, self.n_kv_heads, self.window_size
        hist = 0
        if kv_cache is not None:
            hist = min(kv_cache[0].shape[2], win - 1)
        k_buf = torch.empty((bsz, hkv, hist + seq, hd), dtype=x.dtype, device=x.device)
        v_buf = torch.empty_like(k_buf)
        if hist:
            k_buf[:, :, :hist].copy_(kv_cache[0][:, :, -hist:])
            v_buf[:, :, :hist].copy_(kv_cache[1][:, :, -hist:])
        q = self.project(x, start_pos, k_buf, v_buf, hist)
        attn = torch.empty((bsz, seq, self.n_heads, hd), dtype=x.dtype, device=x.device)
        K.swa_prefill(q.transpose(1, 2), k_buf, v_buf, win, hist, out=attn.transpose(1, 2))
        kv_len = hist + seq
        if kv_len > win:
            cache = (k_buf[:, :, -win:].contiguous(), v_buf[:, :, -win:].contiguous())
        else:
            cache = (k_buf, v_buf)
        return self.wo(attn.view(bsz, seq, self.d_model)), cache


# ==============================================================================
# Slow projections, uTTTLayer, uTTTBlock (reference :1175-1555)
# ==============================================================================

def fused_fast_q_proj(x: Tensor, wq_w: Tensor, q_norm_w: Tensor, eps: float) -> Tensor:
    """Query-only projection + RMSNorm for frozen reads (reference :1175-1190)."""
    q = F.linear(x, wq_w)
    return F.rms_norm(q, (x.shape[-1],), q_norm_w.to(q.dtype), eps)


def linear_residual(h: Tensor, x: Tensor, weight: Tensor) -> Tensor:
    """h += x W^T in place, as one GEMM that accumulates into the residual (the reference's
    ``h + linear(x)``, model/uttt_layer.py:1528-1555, without a separate add kernel or copy).
    ``h`` must be contiguous and owned by the caller."""
    if not h.is_contiguous():
        raise ValueError("the residual stream must be contiguous to be updated in place")
    h.view(-1, h.shape[-1]).addmm_(x.reshape(-1, x.shape[-1]), weight.to(x.dtype).t())
    return h


def fused_slow_projections(x: Tensor, wq_w: Tensor, wk_w: Tensor, wv_w: Tensor, q_norm_w: Tensor,
                           k_norm_w: Tensor, w_eta_w: Tensor, w_eta_b: Tensor, w_alpha_w: Tensor,
                           w_alpha_b: Tensor, base_inner_lr: float, base_weight_decay: float,
                           eps: float) -> Tuple[Tensor, ...]:
    """q, k (RMSNorm with weight), v (RMSNorm), eta, alpha (reference :1193-1231)."""
    dim = x.shape[-1]
    q = F.rms_norm(F.linear(x, wq_w), (dim,), q_norm_w.to(x.dtype), eps)
    k = F.rms_norm(F.linear(x, wk_w), (dim,), k_norm_w.to(x.dtype), eps)
    v = F.rms_norm(F.linear(x, wv_w), (dim,), None, eps)
    eta = base_inner_lr * torch.sigmoid(F.linear(x, w_eta_w, w_eta_b))
    alpha = base_weight_decay * torch.sigmoid(F.linear(x, w_alpha_w, w_alpha_b))
    return q, k, v, eta, alpha


class uTTTLayer(nn.Module):
    """Slow projections + chunk-wise shared fast-weight read/write (reference :1234-1479)."""

    def __init__(self, d_model: int, chunk_size: int = 64, base_inner_lr: float = 0.015,
                 base_weight_decay: float = 0.005, rms_norm_eps: float = 1e-5,
                 chunk_checkpoint_segments: int = 0) -> None:
        super().__init__()
        self.d_model = d_model
        self.chunk_size = chunk_size
        self.base_inner_lr = base_inner_lr
        self.base_weight_decay = base_weight_decay
        self.chunk_checkpoint_segments = chunk_checkpoint_segments
        self.w_q = nn.Linear(d_model, d_model, bias=False)
        self.w_k = nn.Linear(d_model, d_model, bias=False)
        self.w_v = nn.Linear(d_model, d_model, bias=False)
        self.w_o = nn.Linear(d_model, d_model, bias=False)
        self.w_eta = nn.Linear(d_model, 1, bias=True)
        self.w_alpha = nn.Linear(d_model, 1, bias=True)
        nn.init.zeros_(self.w_eta.weight)
        nn.init.constant_(self.w_eta.bias, 0.0)
        nn.init.zeros_(self.w_alpha.weight)
        nn.init.constant_(self.w_alpha.bias, -1.386)
        self.q_norm = RMSNorm(d_model, eps=rms_norm_eps)
        self.k_norm = RMSNorm(d_model, eps=rms_norm_eps)
        self._pack: Optional[Tensor] = None
        self._pack_key = None

    def packed_projection(self) -> Tuple[Tensor, Tensor]:
        """([W_q; W_k; W_v; W_eta; W_alpha], [0; 0; 0; b_eta; b_alpha]) for one GEMM."""
        ws = (self.w_q.weight, self.w_k.weight, self.w_v.weight, self.w_eta.weight, self.w_alpha.weight,
              self.w_eta.bias, self.w_alpha.bias)
        key = tuple((t.data_ptr(), t._version, t.dtype, t.device) for t in ws)
        if self._pack is None or self._pack_key != key:
            w = torch.cat([t.detach() for t in ws[:5]], dim=0)
            b = torch.zeros(w.shape[0], dtype=w.dtype, device=w.device)
            b[-2] = ws[5].detach()[0]
            b[-1] = ws[6].detach()[0]
            self._pack = (w, b)
            self._pack_key = key
        return self._pack

    def packed_projection_folded(self, norm: "RMSNorm") -> Tuple[Tensor, Tensor]:
        """(packed weight with an input RMSNorm's weight folded into its columns, the eta / alpha
        biases), rebuilt when any of them changes."""
        w, b = self.packed_projection()
        key = (self._pack_key, norm.weight.data_ptr(), norm.weight._version, norm.weight.dtype)
        if getattr(self, "_fold_key", None) != key:
            self._fold = ((w.float() * norm.weight.detach().float()[None, :]).to(w.dtype), b[-2:].contiguous())
            self._fold_key = key
        return self._fold

    def projections(self, x: Tensor, norm: Optional["RMSNorm"] = None) -> Tuple[Tensor, ...]:
        """q, k, v, eta, alpha from one packed GEMM (same values as fused_slow_projections).
        With ``norm``, ``x`` is the un-normalised input of that RMSNorm, folded into the GEMM
        weight and the epilogue (per-row 1 / rms scale, then the eta / alpha biases)."""
        if norm is None:
            w, b = self.packed_projection()
            y = F.linear(x, w.to(x.dtype), b.to(x.dtype))
            return K.proj_epilogue(y, self.d_model, self.q_norm.weight, self.k_norm.weight, self.q_norm.eps,
                                   self.base_inner_lr, self.base_weight_decay)
        w, eab = self.packed_projection_folded(norm)
        y = F.linear(x, w.to(x.dtype))
        return K.proj_epilogue(y, self.d_model, self.q_norm.weight, self.k_norm.weight, self.q_norm.eps,
                               self.base_inner_lr, self.base_weight_decay, x=x, x_eps=norm.eps,
                               eta_alpha_bias=eab.to(x.dtype))

    def forward(self, x: Tensor, fast_pool: SharedFastWeightPool, fast_state: FastWeightState,
                attention_mask: Optional[Tensor] = None, update_fast_weights: bool = True,
                read_state: Optional[FastWeightState] = None) -> Tuple[Tensor, FastWeightState, Tensor]:
        bsz, seq, _ = x.shape
        if not update_fast_weights:
            q = fused_fast_q_proj(x, self.w_q.weight, self.q_norm.weight, self.q_norm.eps)
            readout = fast_pool.forward_readout(q, fast_state.ensure_batch_size(bsz))
            return self.w_o(readout), fast_state, x.new_zeros((), dtype=torch.float32)
        require_write_chunk(self.chunk_size)
        q, k, v, eta, alpha = self.projections(x)
        cur = fast_state.ensure_batch_size(bsz)
        if read_state is None:
            fused = fast_pool.chunk_loop(cur, q, k, v, eta, alpha, attention_mask, self.chunk_size)
            if fused is not None:
                return self.w_o(fused[0]), fused[1], fused[2]
        outs, losses = [], []
        n_chunks = (seq + self.chunk_size - 1) // self.chunk_size
        own = None  # buffers this call owns after the first write: later chunks update in place
        for c in range(n_chunks):
            sl = slice(c * self.chunk_size, min(seq, (c + 1) * self.chunk_size))
            mask = attention_mask[:, sl] if attention_mask is not None else None
            out_c, cur, loss_c = fast_pool.chunk_step(cur, q[:, sl], k[:, sl], v[:, sl], eta[:, sl], alpha[:, sl],
                                                      mask, True, read_state, out_state=own)
            own = cur.tensors()
            outs.append(out_c)
            losses.append(loss_c)
        out = torch.cat(outs, dim=1)
        return self.w_o(out), cur, torch.stack(losses).sum() / n_chunks


class uTTTBlock(nn.Module):
    """Pre-norm sliding-window attention + pre-norm uTTT layer (reference :1482-1555)."""

    def __init__(self, layer_idx: int, d_model: int, n_heads: int, n_kv_heads: int, window_size: int = 512,
                 chunk_size: int = 64, base_inner_lr: float = 0.015, base_weight_decay: float = 0.005,
                 max_seq_len: int = 4096, rope_theta: float = 10000.0, rms_norm_eps: float = 1e-5,
                 dropout: float = 0.0) -> None:
        super().__init__()
        self.layer_idx = layer_idx
        self.attn_norm = RMSNorm(d_model, eps=rms_norm_eps)
        self.attn = SlidingWindowAttention(d_model, n_heads, n_kv_heads, window_size, max_seq_len, rope_theta,
                                           dropout)
        self.uttt_norm = RMSNorm(d_model, eps=rms_norm_eps)
        self.uttt = uTTTLayer(d_model, chunk_size, base_inner_lr, base_weight_decay, rms_norm_eps)

    def forward(self, x: Tensor, fast_pool: SharedFastWeightPool, fast_state: FastWeightState,
                attention_mask: Optional[Tensor] = None, kv_cache: Optional[Tuple[Tensor, Tensor]] = None,
                start_pos: int = 0, update_fast_weights: bool = True,
                read_state: Optional[FastWeightState] = None):
        attn_out, new_cache = self.attn(self.attn_norm(x), kv_cache=kv_cache, start_pos=start_pos)
        h = x + attn_out
        u, state, surprise = self.uttt(self.uttt_norm(h), fast_pool=fast_pool, fast_state=fast_state,
                                       attention_mask=attention_mask, update_fast_weights=update_fast_weights,
                                       read_state=read_state)
        return h + u, state, surprise, new_cache
