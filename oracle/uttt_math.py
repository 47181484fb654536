"""CPU restatement of the reference uTTT hot-path arithmetic -- TEST INFRASTRUCTURE ONLY.

Every function here follows one piece of the reference
(``/root/reference/model/uttt_layer.py`` = ``L``, ``model/uttt_model.py`` = ``M``,
``engine/inference.py`` = ``I``, ``engine/personalizer.py`` = ``P``) and cites the
lines it restates.  The functions are dtype-generic in the same way the
reference is: fp64 inputs compute in fp64 (used by the autograd audits),
fp32 inputs compute in fp32 (the parity reference for the fp32 HIP path) and
bf16 inputs reproduce the reference's bf16 rounding points (the context for the
bf16 HIP path, which is judged against the fp32 result).

Weights are passed explicitly (plain tensors), so nothing here depends on
the reference's module construction or parameter draw order.

Pinning (what fixes each function's values independently of this file):

* ``swiglu_fast_forward`` -- scalar per-token loop in tests + golden vectors.
* ``analytical_swiglu_chunk_grad`` -- ``torch.autograd.grad`` of the restated
  loss in fp64 (the reference's own method) + golden vectors.
* ``fused_chunk_ttt_step`` -- an autograd-based independent step, the
  reference's closed forms (momentum derivative 0.99+0.7, (1-a)^10 decay,
  exact 1e-5 increment) + golden vectors.
* ``apply_elastic_pull`` / ``compute_drift`` -- closed forms in tests.
* ``rope_tables`` / ``apply_rope`` -- complex-rotation closed form and the
  relative-position invariant.
* ``sliding_window_attention`` -- scalar per-query loop, window=1 and
  window>=T special cases.
* ``ring_decode_attention`` -- equality with full-prefix attention.
* ``OracleModel`` (chunk-first schedule) -- the reference's schedule
  invariants + golden vectors written by ``tests/golden/make_golden.py``.
"""

from __future__ import annotations

import math
from dataclasses import dataclass, field
from typing import Dict, List, Optional, Sequence, Tuple

import torch
import torch.nn.functional as F

Tensor = torch.Tensor


def _math_dtype(dtype: torch.dtype) -> torch.dtype:
    """fp64 stays fp64, everything else computes in fp32 (L:335, L:448)."""
    return torch.float64 if dtype == torch.float64 else torch.float32


# ---------------------------------------------------------------------------
# Fast-weight memory: readout, analytical chunk gradient, fused step
# ---------------------------------------------------------------------------

def swiglu_fast_forward(x: Tensor, w_up: Tensor, w_gate: Tensor, w_down: Tensor,
                        ln_weight: Tensor, ln_bias: Tensor, eps: float = 1e-5) -> Tensor:
    """f_W(x) = x + LN((SiLU(x W_gate) * (x W_up)) W_down).  Follows L:211-247.

    Matmuls run in the activation dtype with W cast to it; LayerNorm parameters
    are cast to the activation dtype as well (L:239-246).
    """
    act = x.dtype
    up = torch.bmm(x, w_up.to(act))
    gate = torch.bmm(x, w_gate.to(act))
    projected = torch.bmm(F.silu(gate) * up, w_down.to(act))
    normed = F.layer_norm(projected, (projected.shape[-1],), ln_weight.to(act), ln_bias.to(act), eps)
    return x + normed


def analytical_swiglu_chunk_grad(k: Tensor, v: Tensor, eta: Tensor, w_up: Tensor, w_gate: Tensor,
                                 w_down: Tensor, ln_weight: Tensor, ln_bias: Tensor,
                                 token_mask: Optional[Tensor] = None, normalize_by_dim: bool = False,
                                 eps: float = 1e-5) -> Tuple[Tensor, Tensor, Tensor, Tensor]:
    """Closed-form gradient of the eta-weighted chunk reconstruction loss.  Follows L:279-411.

    Rounding points (all no-ops in fp32/fp64): u, g, h, z come out of
    activation-dtype matmuls (L:343-354); LN statistics, the loss and the LN
    backward are fp32 (L:357-389); delta_z is rounded to the activation dtype
    (L:389); the SwiGLU backward is fp32 and rounded (L:398-403); the three
    gradient matmuls produce activation-dtype results (L:393-409).
    """
    act = k.dtype
    cdt = _math_dtype(act)
    _, chunk_len, dim = k.shape
    r_up, r_gate, r_down = w_up.to(act), w_gate.to(act), w_down.to(act)

    up = torch.bmm(k, r_up)
    gate = torch.bmm(k, r_gate)
    hidden = F.silu(gate) * up
    z = torch.bmm(hidden, r_down).to(cdt)

    mean = z.mean(dim=-1, keepdim=True)
    centered = z - mean
    rstd = torch.rsqrt(centered.square().mean(dim=-1, keepdim=True) + eps)
    z_hat = centered * rstd
    gamma = ln_weight.to(cdt).view(1, 1, dim)
    beta = ln_bias.to(cdt).view(1, 1, dim)
    err = (k.to(cdt) + (z_hat * gamma + beta)) - v.to(cdt)

    inv_scale = (1.0 / float(dim)) if normalize_by_dim else 1.0
    token_loss = 0.5 * err.square().sum(dim=-1) * inv_scale
    if token_mask is None:
        surprise = token_loss.mean()
        weight = eta.to(cdt) * (1.0 / float(chunk_len))
    else:
        m = token_mask.to(cdt)
        per_row = m.sum(dim=-1, keepdim=True).clamp_min(1.0)
        surprise = (token_loss * m).sum() / m.sum().clamp_min(1.0)
        weight = (eta.to(cdt) * m.unsqueeze(-1)) / per_row.unsqueeze(-1)

    dz_hat = (weight * inv_scale) * err * gamma
    delta_z = rstd * (dz_hat - dz_hat.mean(dim=-1, keepdim=True)
                      - z_hat * (dz_hat * z_hat).mean(dim=-1, keepdim=True))
    delta_z = delta_z.to(act)

    grad_down = torch.bmm(hidden.transpose(1, 2), delta_z)
    delta_h = torch.bmm(delta_z, r_down.transpose(1, 2)).to(cdt)
    gate_c, up_c = gate.to(cdt), up.to(cdt)
    sig = torch.sigmoid(gate_c)
    delta_up = (delta_h * (gate_c * sig)).to(act)
    delta_gate = (delta_h * up_c * (sig * (1.0 + gate_c * (1.0 - sig)))).to(act)
    k_t = k.transpose(1, 2)
    return torch.bmm(k_t, delta_up), torch.bmm(k_t, delta_gate), grad_down, surprise


def fused_chunk_ttt_step(q: Tensor, k: Tensor, v: Tensor, eta: Tensor, alpha: Tensor,
                         w_up: Tensor, w_gate: Tensor, w_down: Tensor,
                         s_up: Tensor, s_gate: Tensor, s_down: Tensor,
                         ln_weight: Tensor, ln_bias: Tensor, token_mask: Optional[Tensor],
                         momentum_beta: float, max_inner_grad_norm: float, normalize_by_dim: bool,
                         eps: float, read_w_up: Optional[Tensor] = None,
                         read_w_gate: Optional[Tensor] = None,
                         read_w_down: Optional[Tensor] = None,
                         min_row_surprise: float = 0.0) -> Tuple[Tensor, ...]:
    """One chunk: gradient -> per-row Frobenius clip -> momentum -> decay -> masked
    select -> readout through the read weights.  Follows L:414-534.

    Returns (readout, W_up', W_gate', W_down', S_up', S_gate', S_down', surprise)
    with W/S in the master dtype (fp32, or fp64 for fp64 state).

    ``min_row_surprise`` > 0 is the per-chunk surprise gate of BASELINE config 5, which
    the reference does not have (its gate is per turn, P:524-551): a row whose masked mean
    token loss in this chunk is below the threshold keeps W and S, like an all-padding row.
    """
    bsz = q.shape[0]
    g_up, g_gate, g_down, surprise = analytical_swiglu_chunk_grad(
        k, v, eta, w_up, w_gate, w_down, ln_weight, ln_bias, token_mask=token_mask,
        normalize_by_dim=normalize_by_dim, eps=eps)
    mdt = torch.float64 if w_up.dtype == torch.float64 else torch.float32

    if max_inner_grad_norm > 0.0:
        gu, gg = g_up.to(mdt), g_gate.to(mdt)
        gd = g_down.to(mdt).reshape(bsz, w_up.shape[1], w_up.shape[2])
        norm_sq = (gu.square() + gg.square() + gd.square()).sum(dim=-1).sum(dim=-1)
        clip = (max_inner_grad_norm * torch.rsqrt(norm_sq + 1e-8)).clamp(max=1.0).view(bsz, 1, 1)
        steps = (g_up.to(mdt) * clip, g_gate.to(mdt) * clip, g_down.to(mdt) * clip)
    else:
        steps = (g_up, g_gate, g_down)

    new_s = tuple(momentum_beta * s.to(mdt) - st.to(mdt)
                  for s, st in zip((s_up, s_gate, s_down), steps))
    if token_mask is None:
        alpha_bar = alpha.to(mdt).mean(dim=1, keepdim=True)
    else:
        m = token_mask.unsqueeze(-1).to(mdt)
        alpha_bar = (alpha.to(mdt) * m).sum(dim=1, keepdim=True) / m.sum(dim=1, keepdim=True).clamp_min(1)
    decay = 1.0 - alpha_bar
    new_w = tuple(decay * w.to(mdt) + s for w, s in zip((w_up, w_gate, w_down), new_s))

    active = None
    if token_mask is not None:
        active = token_mask.any(dim=1).view(bsz, 1, 1)
    if min_row_surprise and min_row_surprise > 0.0:
        row_mean = row_surprise(k, v, w_up, w_gate, w_down, ln_weight, ln_bias, token_mask, normalize_by_dim, eps)
        keep = (row_mean >= min_row_surprise).view(bsz, 1, 1)
        active = keep if active is None else (active & keep)
    if active is not None:
        new_w = tuple(torch.where(active, n, o) for n, o in zip(new_w, (w_up, w_gate, w_down)))
        new_s = tuple(torch.where(active, n, o) for n, o in zip(new_s, (s_up, s_gate, s_down)))

    out = swiglu_fast_forward(
        q,
        w_up if read_w_up is None else read_w_up,
        w_gate if read_w_gate is None else read_w_gate,
        w_down if read_w_down is None else read_w_down,
        ln_weight, ln_bias, eps)
    return (out,) + new_w + new_s + (surprise,)


def row_surprise(k: Tensor, v: Tensor, w_up: Tensor, w_gate: Tensor, w_down: Tensor, ln_weight: Tensor,
                 ln_bias: Tensor, token_mask: Optional[Tensor], normalize_by_dim: bool, eps: float) -> Tensor:
    """Per-row masked mean token loss of a chunk (the batch-global surprise of L:369-380
    restricted to one row): sum_t l_t m_t / max(1, sum_t m_t), or the row mean unmasked."""
    act = k.dtype
    cdt = _math_dtype(act)
    dim = k.shape[-1]
    pred = swiglu_fast_forward(k, w_up, w_gate, w_down, ln_weight, ln_bias, eps).to(cdt)
    loss = 0.5 * (pred - v.to(cdt)).square().sum(-1) * ((1.0 / dim) if normalize_by_dim else 1.0)
    if token_mask is None:
        return loss.mean(dim=1)
    m = token_mask.to(cdt)
    return (loss * m).sum(dim=1) / m.sum(dim=1).clamp_min(1.0)


def apply_elastic_pull(w: Sequence[Tensor], w0: Sequence[Tensor], anchor_lambda: float,
                       max_drift_ratio: Optional[float] = None) -> Tuple[Tensor, Tensor, Tensor]:
    """W <- (1-lambda) W + lambda W_0, then an optional per-row drift ceiling.  Follows L:773-832.

    ``w`` = (W_up, W_gate, W_down) batched (B, ., .); ``w0`` = the unbatched base weights.
    """
    if anchor_lambda <= 0.0 and max_drift_ratio is None:
        return tuple(w)
    dt = w[0].dtype
    base = tuple(t.detach().to(dtype=dt).unsqueeze(0) for t in w0)
    pulled = tuple((1.0 - anchor_lambda) * cur + anchor_lambda * b for cur, b in zip(w, base))
    if max_drift_ratio is not None and max_drift_ratio > 0.0:
        base_norm = torch.sqrt(sum(b.float().pow(2).sum() for b in base) + 1e-8)
        diffs = tuple(p - b for p, b in zip(pulled, base))
        drift = torch.sqrt(sum(d.float().pow(2).sum(dim=(1, 2), keepdim=True) for d in diffs) + 1e-8)
        scale = torch.clamp(max_drift_ratio * base_norm / drift, max=1.0).to(dt)
        pulled = tuple(b + d * scale for b, d in zip(base, diffs))
    return pulled


def compute_drift(w: Sequence[Tensor], w0: Sequence[Tensor]) -> Dict[str, float]:
    """Frobenius drift of W from W_0 (over the whole batch).  Follows L:834-874."""
    d = [float((cur.float() - b.float().unsqueeze(0)).norm(p="fro")) for cur, b in zip(w, w0)]
    b = [float(t.float().norm(p="fro")) for t in w0]
    total = math.sqrt(sum(x * x for x in d))
    base = math.sqrt(sum(x * x for x in b)) + 1e-8
    return {"drift_frobenius": total, "base_frobenius": base, "drift_pct": total / base * 100.0,
            "w_up_drift": d[0], "w_gate_drift": d[1], "w_down_drift": d[2],
            "w_up_drift_pct": d[0] / (b[0] + 1e-8) * 100.0,
            "w_gate_drift_pct": d[1] / (b[1] + 1e-8) * 100.0,
            "w_down_drift_pct": d[2] / (b[2] + 1e-8) * 100.0}


# ---------------------------------------------------------------------------
# Norms, RoPE, sliding-window attention
# ---------------------------------------------------------------------------

def rms_norm(x: Tensor, weight: Optional[Tensor], eps: float) -> Tensor:
    """RMSNorm through ``F.rms_norm`` with the weight cast to x.dtype.  Follows L:889-891, L:1218-1220."""
    return F.rms_norm(x, (x.shape[-1],), None if weight is None else weight.to(x.dtype), eps)


def rope_tables(head_dim: int, length: int, theta: float = 10000.0) -> Tuple[Tensor, Tensor]:
    """fp32 cos/sin tables (length, head_dim), emb = [f, f] with f_i = p * theta^(-2i/hd).

    Follows L:906-933 (the prefix-preserving extension computes the same
    per-position values, so one build of the full length is equivalent).
    """
    inv_freq = 1.0 / (theta ** (torch.arange(0, head_dim, 2, dtype=torch.float32) / head_dim))
    pos = torch.arange(length, dtype=torch.float32)
    freqs = torch.outer(pos, inv_freq)
    emb = torch.cat((freqs, freqs), dim=-1)
    return emb.cos(), emb.sin()


def apply_rope(x: Tensor, cos: Tensor, sin: Tensor) -> Tensor:
    """x*cos + rotate_half(x)*sin with tables cast to x.dtype.  Follows L:940-958.

    ``x`` is (B, H, T, hd); ``cos``/``sin`` are (T, hd) rows for x's positions.
    """
    c = cos.to(x.dtype)
    s = sin.to(x.dtype)
    half = x.shape[-1] // 2
    rotated = torch.cat((-x[..., half:], x[..., :half]), dim=-1)
    return (x * c) + (rotated * s)


def sliding_window_attention(q: Tensor, k: Tensor, v: Tensor, window: int, q_offset: int) -> Tensor:
    """GQA softmax attention where query i (absolute slot q_offset+i) sees key j iff
    0 <= (q_offset + i) - j < window.  Follows L:1028-1037 and L:1119-1165.

    q (B, H, Tq, hd); k, v (B, Hkv, Tkv, hd); head h reads kv head h // (H/Hkv).
    Scores, softmax and the value sum are computed in fp32 (fp64 for fp64
    inputs) and the result is cast to q.dtype.
    """
    bsz, heads, tq, hd = q.shape
    rep = heads // k.shape[1]
    cdt = _math_dtype(q.dtype)
    kk = k.to(cdt).repeat_interleave(rep, dim=1)
    vv = v.to(cdt).repeat_interleave(rep, dim=1)
    qi = torch.arange(tq, device=q.device).view(-1, 1) + q_offset
    kj = torch.arange(k.shape[2], device=q.device).view(1, -1)
    visible = (qi >= kj) & ((qi - kj) < window)
    scores = torch.matmul(q.to(cdt), kk.transpose(-1, -2)) * (1.0 / math.sqrt(hd))
    scores = scores.masked_fill(~visible, float("-inf"))
    return torch.matmul(torch.softmax(scores, dim=-1), vv).to(q.dtype)


def ring_decode_attention(q: Tensor, k_new: Tensor, v_new: Tensor, k_ring: Tensor, v_ring: Tensor,
                          positions: Sequence[int], window: int) -> Tensor:
    """One decode step over a ring-buffer SWA cache, per request.  Follows I:212-259.

    q (N, H, hd), k_new/v_new (N, Hkv, hd), rings (N, Hkv, window, hd) updated in
    place: slot = pos mod window; valid slots are those < min(pos+1, window).
    Returns (N, H, hd).
    """
    n, heads, hd = q.shape
    rep = heads // k_new.shape[1]
    cdt = _math_dtype(q.dtype)
    out = torch.empty_like(q)
    for r in range(n):
        pos = int(positions[r])
        slot = pos % window
        k_ring[r, :, slot] = k_new[r]
        v_ring[r, :, slot] = v_new[r]
        valid = min(pos + 1, window)
        kk = k_ring[r, :, :valid].to(cdt).repeat_interleave(rep, dim=0)
        vv = v_ring[r, :, :valid].to(cdt).repeat_interleave(rep, dim=0)
        scores = torch.einsum("hd,hkd->hk", q[r].to(cdt), kk) * (1.0 / math.sqrt(hd))
        out[r] = torch.einsum("hk,hkd->hd", torch.softmax(scores, dim=-1), vv).to(q.dtype)
    return out


# ---------------------------------------------------------------------------
# Layer / block / model composition with explicit weights
# ---------------------------------------------------------------------------

@dataclass
class OracleState:
    """Fast-weight state (L:59-91): W/S batched, LN params, step counter."""
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

    NAMES = ("w_up", "w_gate", "w_down", "s_up", "s_gate", "s_down")

    def clone(self) -> "OracleState":
        return OracleState(*(getattr(self, n).clone() for n in self.NAMES),
                           self.ln_weight.clone(), self.ln_bias.clone(), self.step,
                           self.last_surprise_loss, list(self.surprise_history))

    def ensure_batch_size(self, bsz: int) -> "OracleState":
        """Broadcast a batch-1 state to ``bsz`` rows (L:142-163)."""
        cur = self.w_up.shape[0]
        if cur == bsz:
            return self
        if cur != 1:
            raise ValueError(f"Cannot broadcast FastWeightState from batch_size={cur} to {bsz}")
        return OracleState(*(getattr(self, n).expand(bsz, -1, -1).contiguous() for n in self.NAMES),
                           self.ln_weight, self.ln_bias, self.step, self.last_surprise_loss,
                           list(self.surprise_history))


def init_state(pool: Dict[str, Tensor], batch: int, dtype: torch.dtype = torch.float32) -> OracleState:
    """W_0 expanded to ``batch`` rows, S = 0.  Follows L:582-632."""
    ws = [pool[name].to(dtype).unsqueeze(0).expand(batch, -1, -1).clone()
          for name in ("w_up_init", "w_gate_init", "w_down_init")]
    return OracleState(ws[0], ws[1], ws[2], *(torch.zeros_like(w) for w in ws),
                       pool["ln_weight"].to(dtype).clone(), pool["ln_bias"].to(dtype).clone())


@dataclass
class OracleConfig:
    """The subset of uTTTConfig (M:44-80) the hot path reads."""
    d_model: int
    n_layers: int
    n_heads: int
    n_kv_heads: int
    d_ff_fast: int
    sliding_window_size: int
    vocab_size: int = 32000
    rope_theta: float = 10000.0
    rms_norm_eps: float = 1e-5
    chunk_size: int = 64
    base_inner_lr: float = 0.015
    base_weight_decay: float = 0.005
    momentum_beta: float = 0.9
    max_inner_grad_norm: float = 1.0
    normalize_loss_by_dim: bool = True
    # not a reference option: the per-chunk surprise gate of BASELINE config 5 (0 = off)
    min_chunk_surprise: float = 0.0

    @property
    def head_dim(self) -> int:
        return self.d_model // self.n_heads


def slow_projections(x: Tensor, lw: Dict[str, Tensor], cfg: OracleConfig) -> Tuple[Tensor, ...]:
    """q, k (RMSNorm with weight), v (RMSNorm, no weight), eta, alpha.  Follows L:1193-1231."""
    eps = cfg.rms_norm_eps
    q = rms_norm(F.linear(x, lw["uttt.w_q.weight"]), lw["uttt.q_norm.weight"], eps)
    k = rms_norm(F.linear(x, lw["uttt.w_k.weight"]), lw["uttt.k_norm.weight"], eps)
    v = rms_norm(F.linear(x, lw["uttt.w_v.weight"]), None, eps)
    eta = cfg.base_inner_lr * torch.sigmoid(F.linear(x, lw["uttt.w_eta.weight"], lw["uttt.w_eta.bias"]))
    alpha = cfg.base_weight_decay * torch.sigmoid(
        F.linear(x, lw["uttt.w_alpha.weight"], lw["uttt.w_alpha.bias"]))
    return q, k, v, eta, alpha


def swa_forward(x: Tensor, lw: Dict[str, Tensor], cfg: OracleConfig, cos: Tensor, sin: Tensor,
                kv_cache: Optional[Tuple[Tensor, Tensor]] = None,
                start_pos: int = 0) -> Tuple[Tensor, Tuple[Tensor, Tensor]]:
    """SlidingWindowAttention.forward in eval/no-grad mode.  Follows L:1058-1168.

    The cache handed in is trimmed to window-1 entries before the append, the
    kv used for attention is at most window-1+T long, and the returned cache is
    the last ``window`` entries (L:1082-1114).
    """
    bsz, seq, _ = x.shape
    h, hkv, hd, win = cfg.n_heads, cfg.n_kv_heads, cfg.head_dim, cfg.sliding_window_size
    q = F.linear(x, lw["attn.wq.weight"]).view(bsz, seq, h, hd).transpose(1, 2)
    k = F.linear(x, lw["attn.wk.weight"]).view(bsz, seq, hkv, hd).transpose(1, 2)
    v = F.linear(x, lw["attn.wv.weight"]).view(bsz, seq, hkv, hd).transpose(1, 2)
    q = apply_rope(q, cos[start_pos:start_pos + seq], sin[start_pos:start_pos + seq])
    k = apply_rope(k, cos[start_pos:start_pos + seq], sin[start_pos:start_pos + seq])
    if kv_cache is not None:
        k_prev, v_prev = kv_cache
        history = win - 1
        k_prev, v_prev = k_prev[:, :, max(0, k_prev.shape[2] - history):], v_prev[:, :, max(0, v_prev.shape[2] - history):]
        if history == 0:
            k_prev, v_prev = k_prev[:, :, :0], v_prev[:, :, :0]
        k = torch.cat([k_prev, k], dim=2)
        v = torch.cat([v_prev, v], dim=2)
        needed = win - 1 + seq
        k, v = k[:, :, -needed:], v[:, :, -needed:]
    new_cache = (k[:, :, -win:].contiguous(), v[:, :, -win:].contiguous())
    attn = sliding_window_attention(q, k, v, win, k.shape[2] - seq)
    out = attn.transpose(1, 2).reshape(bsz, seq, h * hd)
    return F.linear(out, lw["attn.wo.weight"]), new_cache


def uttt_layer_forward(x: Tensor, lw: Dict[str, Tensor], cfg: OracleConfig, state: OracleState,
                       attention_mask: Optional[Tensor] = None, update_fast_weights: bool = True,
                       read_state: Optional[OracleState] = None) -> Tuple[Tensor, OracleState, Tensor]:
    """uTTTLayer.forward (eval, no segment checkpointing).  Follows L:1278-1479 and the
    chunk_step wrapper L:697-771 (each chunk reads ``read_state`` when given, else
    its own pre-update cursor)."""
    bsz, seq, _ = x.shape
    if not update_fast_weights:
        q = rms_norm(F.linear(x, lw["uttt.w_q.weight"]), lw["uttt.q_norm.weight"], cfg.rms_norm_eps)
        rs = state.ensure_batch_size(bsz)
        readout = swiglu_fast_forward(q, rs.w_up, rs.w_gate, rs.w_down, rs.ln_weight, rs.ln_bias,
                                      cfg.rms_norm_eps)
        return F.linear(readout, lw["uttt.w_o.weight"]), state, x.new_zeros((), dtype=torch.float32)
    q, k, v, eta, alpha = slow_projections(x, lw, cfg)
    cur = state.ensure_batch_size(bsz)
    read = None if read_state is None else read_state.ensure_batch_size(bsz)
    outs, losses = [], []
    c = cfg.chunk_size
    n_chunks = (seq + c - 1) // c
    for i in range(n_chunks):
        sl = slice(i * c, min(seq, (i + 1) * c))
        r = cur if read is None else read
        res = fused_chunk_ttt_step(
            q[:, sl], k[:, sl], v[:, sl], eta[:, sl], alpha[:, sl],
            cur.w_up, cur.w_gate, cur.w_down, cur.s_up, cur.s_gate, cur.s_down,
            cur.ln_weight, cur.ln_bias,
            None if attention_mask is None else attention_mask[:, sl],
            cfg.momentum_beta, float(cfg.max_inner_grad_norm or 0.0), cfg.normalize_loss_by_dim,
            cfg.rms_norm_eps, r.w_up, r.w_gate, r.w_down, cfg.min_chunk_surprise)
        outs.append(res[0])
        losses.append(res[7])
        cur = OracleState(*res[1:7], cur.ln_weight, cur.ln_bias, cur.step + 1,
                          cur.last_surprise_loss, cur.surprise_history)
    out = torch.cat(outs, dim=1)
    return F.linear(out, lw["uttt.w_o.weight"]), cur, torch.stack(losses).sum() / n_chunks


def block_forward(x: Tensor, lw: Dict[str, Tensor], cfg: OracleConfig, cos: Tensor, sin: Tensor,
                  state: OracleState, attention_mask: Optional[Tensor] = None,
                  kv_cache: Optional[Tuple[Tensor, Tensor]] = None, start_pos: int = 0,
                  update_fast_weights: bool = True, read_state: Optional[OracleState] = None):
    """x + SWA(RMSNorm x); h + uTTT(RMSNorm h).  Follows L:1528-1555."""
    eps = cfg.rms_norm_eps
    attn, cache = swa_forward(rms_norm(x, lw["attn_norm.weight"], eps), lw, cfg, cos, sin, kv_cache, start_pos)
    h = x + attn
    u, st, surprise = uttt_layer_forward(rms_norm(h, lw["uttt_norm.weight"], eps), lw, cfg, state,
                                         attention_mask, update_fast_weights, read_state)
    return h + u, st, surprise, cache


class OracleModel:
    """uTTTModel forward with the chunk-first shared schedule.  Follows M:453-608, M:714-960.

    ``weights`` uses the reference's state_dict key names (``tok_embeddings.weight``,
    ``layers.{i}.attn.wq.weight``, ``fast_weight_pool.w_up_init`` ...).
    """

    def __init__(self, cfg: OracleConfig, weights: Dict[str, Tensor], dtype: torch.dtype = torch.float32):
        self.cfg = cfg
        self.dtype = dtype
        self.w = {k: (v.to(dtype) if not k.startswith("fast_weight_pool.") else v.float())
                  for k, v in weights.items()}
        self.layers = [{k[len(f"layers.{i}."):]: v for k, v in self.w.items()
                        if k.startswith(f"layers.{i}.")} for i in range(cfg.n_layers)]
        self.pool = {k[len("fast_weight_pool."):]: v for k, v in self.w.items()
                     if k.startswith("fast_weight_pool.")}
        self.cos, self.sin = rope_tables(cfg.head_dim, 1 << 14, cfg.rope_theta)

    def init_state(self, batch: int = 1) -> OracleState:
        return init_state(self.pool, batch, torch.float32)

    def logits(self, h: Tensor) -> Tensor:
        head = self.w.get("lm_head.weight", self.w["tok_embeddings.weight"])
        return F.linear(rms_norm(h, self.w["norm.weight"], self.cfg.rms_norm_eps), head)

    def forward(self, input_ids: Tensor, state: Optional[OracleState] = None,
                attention_mask: Optional[Tensor] = None, kv_caches=None, start_pos: int = 0,
                update_fast_weights: bool = True, logits_to_keep: int = 0):
        """Returns (logits or None, state, per-layer surprise tensor, kv caches)."""
        cfg = self.cfg
        bsz, seq = input_ids.shape
        h = F.embedding(input_ids, self.w["tok_embeddings.weight"])
        state = self.init_state(bsz) if state is None else state.ensure_batch_size(bsz)
        n_layers = cfg.n_layers
        caches = list(kv_caches) if kv_caches is not None else [None] * n_layers
        if update_fast_weights:
            tensors = state
            pieces, losses, counts = [], [], []
            step = state.step
            for off in range(0, seq, cfg.chunk_size):
                end = min(off + cfg.chunk_size, seq)
                mask = None if attention_mask is None else attention_mask[:, off:end]
                read = OracleState(*(getattr(tensors, n) for n in OracleState.NAMES),
                                   tensors.ln_weight, tensors.ln_bias, step)
                cursor = read
                hid = h[:, off:end]
                chunk_losses = []
                for li in range(n_layers):
                    hid, cursor, surprise, cache = block_forward(
                        hid, self.layers[li], cfg, self.cos, self.sin, cursor, mask, caches[li],
                        start_pos + off, True, read)
                    caches[li] = tuple(t[:, :, -cfg.sliding_window_size:] for t in cache)
                    chunk_losses.append(surprise)
                tensors = cursor
                pieces.append(hid)
                losses.append(torch.stack(chunk_losses))
                counts.append(mask.sum().to(torch.float32) if mask is not None
                              else torch.tensor(float(bsz * (end - off))))
                step += n_layers
            cnt = torch.stack(counts)
            per_layer = (torch.stack(losses) * cnt[:, None]).sum(dim=0) / cnt.sum().clamp_min(1)
            h = torch.cat(pieces, dim=1)
            new_state = OracleState(*(getattr(tensors, n) for n in OracleState.NAMES),
                                    tensors.ln_weight, tensors.ln_bias, step,
                                    state.last_surprise_loss, list(state.surprise_history))
            floats = [float(x) for x in per_layer.tolist()]
            new_state.last_surprise_loss = sum(floats) / max(len(floats), 1)
            new_state.surprise_history = (list(new_state.surprise_history) + floats)[-100:]
        else:
            new_state = state
            per = []
            for li in range(n_layers):
                h, _, s, cache = block_forward(h, self.layers[li], cfg, self.cos, self.sin, state,
                                               attention_mask, caches[li], start_pos, False, None)
                caches[li] = cache
                per.append(s)
            per_layer = torch.stack(per)
        if logits_to_keep < 0:
            logits = None
        elif logits_to_keep > 0 and seq > logits_to_keep:
            logits = self.logits(h[:, -logits_to_keep:])
        else:
            logits = self.logits(h)
        return logits, new_state, per_layer, caches

    def test_time_update(self, ids: Tensor, state: OracleState,
                         attention_mask: Optional[Tensor] = None):
        """Clone, update over the interaction, report mean surprise.  Follows M:1237-1271."""
        _, cand, per_layer, _ = self.forward(ids, state.clone(), attention_mask, None, 0, True, -1)
        return cand, float(cand.last_surprise_loss), [float(x) for x in per_layer.tolist()]

    def greedy_generate(self, ids: Tensor, state: OracleState, max_new_tokens: int,
                        active_vocab_limit: Optional[int] = None) -> List[int]:
        """Frozen-state greedy decode of one prompt.  Follows M:966-1179 with temperature 0 and
        the logit masking of M:1181-1235 (PAD/BOS/UNK = ids 0/1/3 and ids >= the active
        vocabulary limit are excluded; a USER/ASSISTANT id (4/5) ends the reply unyielded)."""
        logits, _, _, caches = self.forward(ids, state, None, None, 0, False, 1)
        pos = ids.shape[1]
        out: List[int] = []
        limit = self.cfg.vocab_size if active_vocab_limit is None else active_vocab_limit
        while len(out) < max_new_tokens:
            work = logits[:, -1, :].float().clone()
            work[:, [0, 1, 3]] = float("-inf")
            if limit < work.shape[-1]:
                work[:, limit:] = float("-inf")
            tok = int(work.argmax(dim=-1))
            if tok in (4, 5):
                break
            out.append(tok)
            if len(out) >= max_new_tokens:
                break
            logits, _, _, caches = self.forward(torch.tensor([[tok]]), state, None, caches, pos, False, 0)
            pos += 1
        return out


def personalizer_gate(surprise: float, threshold: float) -> bool:
    """Turn-level gate: refuse non-finite/negative, write iff surprise > threshold.  Follows P:524-526."""
    if not math.isfinite(surprise) or surprise < 0:
        raise ValueError("Test-time update returned a non-finite or negative surprise loss")
    return bool(surprise > threshold)
