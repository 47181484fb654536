"""Batched frozen-state decoding over ring-buffer SWA caches.

The reference decodes one request at a time, either eagerly (``uTTTModel.stream_generate``,
``model/uttt_model.py:966-1179``) or through ``CUDAGraphDecoder`` (``engine/inference.py:71-302``),
whose captured step writes the new key/value into ring slot ``pos mod window``, masks the slots
that are not yet valid and reads each layer's fast weights through activation-dtype copies.

``BatchedDecoder`` runs N independent requests in one step: every request keeps its own fp32
fast-weight master state (read through per-request activation-dtype copies), its own position
and its own ring slots.  One step is, per layer: RMSNorm -> packed QKV GEMM -> ``uttt_swa_decode``
(RoPE at each request's position, ring write, window attention) -> output GEMM -> RMSNorm ->
query projection -> per-request fast-weight readout (``uttt_swiglu_readout`` over the stacked
copies) -> output GEMM; then the final norm, the LM head and greedy selection, all on the
device, so ``capture()`` can record the whole step into one HIP graph.
"""
from __future__ import annotations

from typing import List, Optional, Sequence

import torch
import torch.nn.functional as F

from . import kernels as K
from .layer import FastWeightState, linear_residual
from .model import BOS_ID, PAD_ID, UNK_ID, uTTTModel

Tensor = torch.Tensor


class BatchedDecoder:
    """N requests, one token each per step, frozen fast weights (decode never writes them)."""

    def __init__(self, model: uTTTModel, states: Sequence[FastWeightState], max_positions: int = 8192):
        if model.training:
            raise ValueError("call model.eval() before decoding")
        if not states:
            raise ValueError("need at least one request state")
        self.model = model
        self.n = len(states)
        dev = model.tok_embeddings.weight.device
        if dev.type != "cuda":
            raise ValueError("BatchedDecoder needs the model on the GPU")
        self.device = dev
        self.dtype = model.tok_embeddings.weight.dtype
        for st in states:
            if st.w_up.shape[0] != 1:
                raise ValueError("each request state must hold one row (batch 1)")
        ln_w, ln_b = states[0].ln_weight, states[0].ln_bias
        for st in states[1:]:
            if not (torch.equal(st.ln_weight, ln_w) and torch.equal(st.ln_bias, ln_b)):
                raise ValueError("batched decoding needs one shared LayerNorm pair for all requests")
        self.ln_weight = ln_w.detach().float().contiguous()
        self.ln_bias = ln_b.detach().float().contiguous()
        # per-request read copies in the activation dtype (reference inference_read_weights,
        # model/uttt_layer.py:648-668): same operands the reference's bf16 matmuls see
        with torch.no_grad():
            self.w_up = torch.cat([st.w_up.detach() for st in states]).to(self.dtype).contiguous()
            self.w_gate = torch.cat([st.w_gate.detach() for st in states]).to(self.dtype).contiguous()
            self.w_down = torch.cat([st.w_down.detach() for st in states]).to(self.dtype).contiguous()
        attn = model.layers[0].attn
        self.window, self.hkv, self.hd, self.heads = attn.window_size, attn.n_kv_heads, attn.head_dim, attn.n_heads
        self.rings = [(torch.zeros((self.n, self.hkv, self.window, self.hd), dtype=self.dtype, device=dev),
                       torch.zeros((self.n, self.hkv, self.window, self.hd), dtype=self.dtype, device=dev))
                      for _ in model.layers]
        self.cos, self.sin = attn.rope.tables(max_positions, dev)
        self.positions = torch.zeros(self.n, dtype=torch.int64, device=dev)
        self.host_positions = [0] * self.n
        self.tokens = torch.zeros(self.n, dtype=torch.int64, device=dev)
        self.logits: Optional[Tensor] = None
        self.next_tokens: Optional[Tensor] = None
        self._graph = None
        self._ws_attn = torch.zeros(1, dtype=torch.uint8, device=dev)
        self._ws_read = torch.zeros(1, dtype=torch.uint8, device=dev)
        self._states = list(states)
        self._key = self._state_key(states)
        self._folds = {}
        d_model = model.config.d_model
        self._fused_readout = self.dtype == torch.bfloat16 and d_model <= 2048 and all(
            (blk.uttt.q_norm.eps or 0.0) > 0.0 for blk in model.layers)
        self._counters = torch.zeros(self.n, dtype=torch.int32, device=dev)  # left zero by every readout

    # ------------------------------------------------------------------ prefill
    @torch.no_grad()
    def prefill(self, prompts: Sequence[Tensor]) -> Tensor:
        """Frozen prefill of each request's prompt (its own state), then load the last
        ``window`` keys/values into the ring slots.  Returns the next-token logits (N, V)."""
        if len(prompts) != self.n:
            raise ValueError(f"expected {self.n} prompts, got {len(prompts)}")
        out_logits = []
        for i, (ids, st) in enumerate(zip(prompts, self._states)):
            ids = ids.to(self.device).view(1, -1)
            if ids.shape[1] == 0:
                raise ValueError("prompts must be non-empty")
            out = self.model(ids, fast_state=st, update_fast_weights=False, logits_to_keep=1)
            self._load_request(i, out.kv_caches, ids.shape[1])
            out_logits.append(out.logits[:, -1, :])
        self.positions.copy_(torch.tensor(self.host_positions, dtype=torch.int64))
        return torch.cat(out_logits, dim=0)

    def _load_request(self, i: int, kv_caches, length: int) -> None:
        """Request i's ring slots from a frozen prefill's per-layer caches (the last <= window
        rotated keys / values of ``length`` tokens): token p goes to slot p mod window."""
        if len(kv_caches) != len(self.rings):
            raise ValueError(f"expected {len(self.rings)} layer caches, got {len(kv_caches)}")
        for (kr, vr), (k, v) in zip(self.rings, kv_caches):
            cached = k.shape[2]
            if (k.shape != (1, self.hkv, cached, self.hd) or v.shape != k.shape or cached > min(length, self.window)
                    or cached < min(length, self.window - 1)):
                raise ValueError("a cache must be (1, n_kv_heads, min(length, window) or window - 1, head_dim)")
            slots = torch.arange(length - cached, length, device=self.device) % self.window
            kr[i].index_copy_(1, slots, k[0].to(device=self.device, dtype=kr.dtype))
            vr[i].index_copy_(1, slots, v[0].to(device=self.device, dtype=vr.dtype))
        self.host_positions[i] = int(length)

    @torch.no_grad()
    def reset(self, kv_caches_per_request: Sequence, lengths: Sequence[int]) -> None:
        """Start again from other prompts' frozen-prefill caches (same requests and states):
        the rings, positions and buffers keep their addresses, so a captured step stays valid."""
        if len(kv_caches_per_request) != self.n or len(lengths) != self.n:
            raise ValueError(f"expected caches and lengths for {self.n} requests")
        for kr, vr in self.rings:
            kr.zero_()
            vr.zero_()
        for i, (caches, length) in enumerate(zip(kv_caches_per_request, lengths)):
            if length < 1:
                raise ValueError("a request needs at least one prompt token")
            self._load_request(i, caches, int(length))
        self.positions.copy_(torch.tensor(self.host_positions, dtype=torch.int64))

    @torch.no_grad()
    def export_kv_caches(self, i: int = 0) -> List:
        """Request i's per-layer caches in the eager layout (the last min(position, window)
        rotated keys / values in token order), e.g. to continue a decode eagerly."""
        pos = self.host_positions[i]
        kept = min(pos, self.window)
        slots = torch.arange(pos - kept, pos, device=self.device) % self.window
        return [(kr[i:i + 1].index_select(2, slots), vr[i:i + 1].index_select(2, slots)) for kr, vr in self.rings]

    def matches(self, model: uTTTModel, states: Sequence[FastWeightState]) -> bool:
        """Whether this decoder's read copies and LayerNorm pair still stand for ``states`` of
        ``model`` (same tensors, unchanged versions), so it can be ``reset`` and reused."""
        return model is self.model and len(states) == self.n and self._state_key(states) == self._key

    @staticmethod
    def _state_key(states: Sequence[FastWeightState]) -> tuple:
        return tuple((t.data_ptr(), t._version, t.dtype) for st in states
                     for t in (st.w_up, st.w_gate, st.w_down, st.ln_weight, st.ln_bias))

    # ------------------------------------------------------------------ one step
    def _folded(self, weight: Tensor, norm) -> Tensor:
        """W diag(g) for an RMSNorm ``norm`` applied to W's input (formed in fp32, rounded
        once), rebuilt when either changes."""
        key = (weight.data_ptr(), weight._version, norm.weight.data_ptr(), norm.weight._version)
        hit = self._folds.get(id(weight))
        if hit is None or hit[0] != key:
            fold = (weight.detach().float() * norm.weight.detach().float()[None, :]).to(weight.dtype).contiguous()
            hit = (key, fold)
            self._folds[id(weight)] = hit
        return hit[1]

    def _linear(self, x: Tensor, weight: Tensor, residual: Optional[Tensor] = None, norm=None) -> Tensor:
        """norm(x) W^T (+ residual, updated in place): ``uttt_skinny_linear`` for bf16 steps of
        at most 64 requests (the RMSNorm folded in), the norm and the library GEMM otherwise."""
        skinny = (x.dtype == torch.bfloat16 and weight.dtype == torch.bfloat16 and x.shape[0] <= 64
                  and weight.shape[0] % 32 == 0 and x.shape[1] % 64 == 0 and x.stride(1) == 1
                  and weight.is_contiguous() and (norm is None or (norm.eps or 0.0) > 0.0))
        if skinny:
            if norm is None:
                return K.skinny_linear(x, weight, out=residual, residual=residual)
            return K.skinny_linear(x, self._folded(weight, norm), out=residual, residual=residual,
                                   x_eps=norm.eps)
        if norm is not None:
            x = norm(x)
        if residual is not None:
            return linear_residual(residual, x, weight)
        return F.linear(x, weight)

    def _step_body(self) -> None:
        m = self.model
        n = self.n
        h = F.embedding(self.tokens, m.tok_embeddings.weight)  # (N, D)
        for li, block in enumerate(m.layers):
            attn = block.attn
            qkv = self._linear(h, attn.packed_qkv().to(h.dtype), norm=block.attn_norm)  # (N, (H + 2 Hkv) hd)
            hq = self.heads * self.hd
            hk = self.hkv * self.hd
            q = qkv[:, :hq].view(n, self.heads, self.hd)
            k = qkv[:, hq:hq + hk].view(n, self.hkv, self.hd)
            v = qkv[:, hq + hk:].view(n, self.hkv, self.hd)
            kr, vr = self.rings[li]
            att = K.swa_decode(q, k, v, kr, vr, self.positions, self.cos, self.sin, workspace=self._ws_attn)
            h = self._linear(att.reshape(n, -1), attn.wo.weight, residual=h)
            y = self._linear(h, block.uttt.w_q.weight, norm=block.uttt_norm)
            qn = block.uttt.q_norm
            # every layer reads the same per-request copies: odd layers walk them backwards, so
            # each readout starts on the lines the previous one left in the infinity cache
            rev = li % 2 == 1
            if self._fused_readout:  # q_norm, readout, LayerNorm and residual in one launch
                r = K.swiglu_readout(y.view(n, 1, -1), self.w_up, self.w_gate, self.w_down, self.ln_weight,
                                     self.ln_bias, m.fast_weight_pool.eps, workspace=self._ws_read,
                                     x_norm=(qn.weight, qn.eps), row_counters=self._counters, sweep_reverse=rev)
            else:
                uq = F.rms_norm(y, (h.shape[-1],), qn.weight.to(h.dtype), qn.eps)
                r = K.swiglu_readout(uq.view(n, 1, -1), self.w_up, self.w_gate, self.w_down, self.ln_weight,
                                     self.ln_bias, m.fast_weight_pool.eps, workspace=self._ws_read,
                                     sweep_reverse=rev)
            h = self._linear(r.view(n, -1), block.uttt.w_o.weight, residual=h)
        logits = self._linear(h, m.lm_head.weight, norm=m.norm)
        self.logits = logits
        # temperature-0 selection: PAD / BOS / UNK and ids past the active vocabulary excluded
        limit = m.active_vocab_limit if m.active_vocab_limit < logits.shape[-1] else None
        # written straight into the next step's input (stepping with `next_tokens` copies
        # nothing), and the positions advance in the same launch
        self.next_tokens = K.greedy_select(logits, (PAD_ID, BOS_ID, UNK_ID), limit, out=self.tokens,
                                           advance=self.positions)

    def _warm_workspaces(self) -> None:
        from . import _native as N
        nbytes = N.load_library().uttt_swa_decode_workspace(self.n, self.heads, self.hkv, self.hd, self.window)
        self._ws_attn = torch.empty(max(nbytes, 1), dtype=torch.uint8, device=self.device)
        d = self.model.config.d_model
        ff = self.model.config.d_ff_fast
        code = N.DTYPE_BF16 if self.dtype == torch.bfloat16 else N.DTYPE_F32
        self._ws_read = torch.zeros(max(N.load_library().uttt_readout_workspace(self.n, 1, d, ff, code), 1),
                                    dtype=torch.uint8, device=self.device)

    @torch.no_grad()
    def capture(self) -> None:
        """Record one step into a HIP graph (after ``prefill``); ``step`` then replays it."""
        self._warm_workspaces()
        saved = (self.positions.clone(), [(k.clone(), v.clone()) for k, v in self.rings])
        self._step_body()  # warm-up outside the graph (packs, tables, allocator)
        torch.cuda.synchronize()
        self.positions.copy_(saved[0])
        for (k, v), (k0, v0) in zip(self.rings, saved[1]):
            k.copy_(k0)
            v.copy_(v0)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            self._step_body()
        torch.cuda.synchronize()
        # capture ran no kernels; positions and rings are as before
        self._graph = graph

    @torch.no_grad()
    def step(self, tokens: Tensor) -> Tensor:
        """Append one token per request; returns the logits (N, V) for the next position."""
        if tokens.shape != (self.n,):
            raise ValueError(f"tokens must be ({self.n},)")
        limit = self.cos.shape[0]
        if max(self.host_positions) >= limit:
            raise ValueError("a request reached the end of the RoPE table")
        if tokens.data_ptr() != self.tokens.data_ptr():
            self.tokens.copy_(tokens)
        if self._graph is not None:
            self._graph.replay()
        else:
            if self._ws_attn.numel() == 1:
                self._warm_workspaces()
            self._step_body()
        self.host_positions = [p + 1 for p in self.host_positions]
        return self.logits

    @torch.no_grad()
    def generate_greedy(self, first_logits: Tensor, steps: int) -> Tensor:
        """Greedy tokens (N, steps) continuing from ``first_logits`` (no EOS stop)."""
        m = self.model
        work = first_logits.float().clone()
        work[:, [PAD_ID, BOS_ID, UNK_ID]] = float("-inf")
        if m.active_vocab_limit < work.shape[-1]:
            work[:, m.active_vocab_limit:] = float("-inf")
        tok = work.argmax(dim=-1)
        out = [tok]
        for _ in range(steps - 1):
            self.step(tok)
            tok = self.next_tokens  # already the next step's input
            out.append(tok.clone())
        return torch.stack(out, dim=1)
