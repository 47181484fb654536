"""Drop-in counterpart of the reference's ``model/uttt_model.py`` (uTTTConfig / uTTTModel).

Parameter names and shapes match the reference, so its base checkpoints load with
``load_dual_base_state`` / ``load_state_dict``.  The forward pass with fast-weight
writes runs the reference's chunk-first shared schedule (every layer of a chunk
reads the chunk-start snapshot; writes chain one cursor through the layers;
reference ``uttt_model.py:453-608``) on the HIP kernels, with

* per chunk, every layer's attention, projections and readout first (the readouts read
  the chunk-start state, through bf16 copies on the bf16 path), then one layer-chain
  launch (``uttt_chunk_chain``) that applies all L chained updates to one fp32 state set
  in place (a copy of the caller's state, whose tensors are never written);
* one linear KV buffer per layer for the whole call (rotated keys appended by the
  RoPE kernel, the window enforced by the attention kernel);
* per-(chunk, layer) surprise kept on the device; the only host sync is the
  reference's end-of-forward surprise read, which ``prefill_with_writes`` skips so
  the whole prefill can be recorded into a HIP graph.
"""
from __future__ import annotations

import math
from dataclasses import asdict, dataclass, field
from pathlib import Path
from typing import Any, Dict, Iterator, List, Optional, Tuple

import torch
import torch.nn as nn
import torch.nn.functional as F

from . import _native as N
from . import kernels as K
from .prefill_plan import PrefillPlan, plan_supported
from .layer import FastWeightState, RMSNorm, SharedFastWeightPool, linear_residual, require_write_chunk, uTTTBlock

Tensor = torch.Tensor
_NAMES = ("w_up", "w_gate", "w_down", "s_up", "s_gate", "s_down")

# Special token ids of the reference's SimpleUTF8Tokenizer (uttt_model.py:140-151)
PAD_ID, BOS_ID, EOS_ID, UNK_ID, USER_ID, ASSISTANT_ID = 0, 1, 2, 3, 4, 5
ACTIVE_VOCAB_LIMIT = 21478


@dataclass
class uTTTConfig:
    """Model and inner-loop configuration (reference uttt_model.py:44-111)."""
    name: str = "uTTT-151M-Base"
    vocab_size: int = 32000
    d_model: int = 1024
    n_layers: int = 16
    n_heads: int = 16
    n_kv_heads: int = 4
    d_ff_fast: int = 2816
    sliding_window_size: int = 512
    max_seq_len: int = 4096
    rope_theta: float = 10000.0
    rms_norm_eps: float = 1e-5
    dropout: float = 0.0
    chunk_size: int = 64
    base_inner_lr: float = 0.015
    base_weight_decay: float = 0.005
    momentum_beta: float = 0.90
    max_inner_grad_norm: float = 1.0
    normalize_loss_by_dim: bool = True
    surprise_threshold: float = 0.25
    elastic_anchor_lambda: float = 0.02
    max_weight_drift_ratio: float = 0.35
    gradient_checkpointing: bool = True
    gradient_checkpointing_every: int = 1
    meta_checkpoint_layers: int = 0
    meta_checkpoint_time_chunks: bool = True
    meta_checkpoint_reentrant: bool = False
    tie_word_embeddings: bool = True
    write_schedule: str = "sequential"
    dspark_speculative_k: int = 0
    dspark_conf_threshold: float = 0.82
    tokenizer_json: Optional[str] = None
    repetition_penalty: float = 1.0

    def to_dict(self) -> Dict[str, Any]:
        return asdict(self)

    @classmethod
    def from_dict(cls, data: Dict[str, Any]) -> "uTTTConfig":
        merged: Dict[str, Any] = {}
        if "model" in data or "uttt" in data:
            merged.update(data.get("model", {}))
            merged.update(data.get("uttt", {}))
            for name in ("gradient_checkpointing", "gradient_checkpointing_every", "meta_checkpoint_layers",
                         "meta_checkpoint_time_chunks", "meta_checkpoint_reentrant"):
                if name in data.get("training", {}):
                    merged[name] = data["training"][name]
        else:
            merged.update(data)
        valid = {f for f in cls.__dataclass_fields__}
        return cls(**{k: v for k, v in merged.items() if k in valid})

    @classmethod
    def from_yaml(cls, path: str | Path) -> "uTTTConfig":
        import yaml
        with open(path, "r", encoding="utf-8") as fh:
            return cls.from_dict(yaml.safe_load(fh))


@dataclass
class uTTTModelOutput:
    """Structured forward output (reference uttt_model.py:114-124)."""
    logits: Tensor
    fast_state: Optional[FastWeightState]
    loss: Optional[Tensor] = None
    ce_loss: Optional[Tensor] = None
    surprise_loss: Optional[Tensor] = None
    layer_surprise_losses: List[float] = field(default_factory=list)
    kv_caches: Optional[List[Tuple[Tensor, Tensor]]] = None


class uTTTModel(nn.Module):
    """Embeddings, L x (SWA + uTTT) blocks, final norm and tied LM head around one shared
    fast-weight pool (reference uttt_model.py:261-1271), inference on the HIP path."""

    INNER_LOOP_PROTOCOL = "chunk_shared_fp32_exact_v2"

    def __init__(self, config: uTTTConfig) -> None:
        super().__init__()
        self.config = config
        self.active_vocab_limit = ACTIVE_VOCAB_LIMIT if config.vocab_size >= 24000 else config.vocab_size
        self.tok_embeddings = nn.Embedding(config.vocab_size, config.d_model)
        self.fast_weight_pool = SharedFastWeightPool(config.d_model, config.d_ff_fast, config.momentum_beta,
                                                     config.max_inner_grad_norm, config.normalize_loss_by_dim,
                                                     config.rms_norm_eps)
        self.layers = nn.ModuleList([
            uTTTBlock(i, config.d_model, config.n_heads, config.n_kv_heads, config.sliding_window_size,
                      config.chunk_size, config.base_inner_lr, config.base_weight_decay, config.max_seq_len,
                      config.rope_theta, config.rms_norm_eps, config.dropout)
            for i in range(config.n_layers)])
        self.norm = RMSNorm(config.d_model, eps=config.rms_norm_eps)
        self.lm_head = nn.Linear(config.d_model, config.vocab_size, bias=False)
        self._init_slow_weights()
        if config.tie_word_embeddings:
            self.lm_head.weight = self.tok_embeddings.weight

    def _init_slow_weights(self) -> None:
        """N(0, 0.02) for slow Linear / Embedding weights except the eta / alpha routers
        (reference uttt_model.py:340-352)."""
        for name, module in self.named_modules():
            if "fast_weight_pool" in name:
                continue
            if isinstance(module, nn.Linear) and not name.endswith(("w_eta", "w_alpha")):
                nn.init.normal_(module.weight, mean=0.0, std=0.02)
                if module.bias is not None:
                    nn.init.zeros_(module.bias)
            elif isinstance(module, nn.Embedding):
                nn.init.normal_(module.weight, mean=0.0, std=0.02)

    # ------------------------------------------------------------------ checkpoints
    def get_slow_parameters(self) -> List[nn.Parameter]:
        fast = {id(p) for p in self.fast_weight_pool.parameters()}
        return [p for p in self.parameters() if id(p) not in fast]

    def get_meta_fast_parameters(self) -> List[nn.Parameter]:
        return list(self.fast_weight_pool.parameters())

    def slow_state_dict(self) -> Dict[str, Tensor]:
        return {k: v.detach().to("cpu", copy=True) for k, v in self.state_dict().items()
                if not k.startswith("fast_weight_pool.")}

    def init_fast_state_dict(self) -> Dict[str, Tensor]:
        return {k: v.detach().to("cpu", copy=True) for k, v in self.fast_weight_pool.state_dict().items()}

    def load_dual_base_state(self, slow_weights: Dict[str, Tensor], init_fast_weights: Dict[str, Tensor],
                             strict: bool = True) -> None:
        """Load a reference base checkpoint's two tracks (reference uttt_model.py:383-394)."""
        merged = dict(slow_weights)
        for k, v in init_fast_weights.items():
            merged[k if k.startswith("fast_weight_pool.") else f"fast_weight_pool.{k}"] = v
        self.load_state_dict(merged, strict=strict)

    def freeze_slow_weights(self) -> None:
        for p in self.parameters():
            p.requires_grad_(False)

    def prepare_for_inference(self, enabled: bool = True) -> None:
        """Build (or drop) the disposable inference packs without changing checkpoint keys
        (reference uttt_model.py:401-422): each attention's ``_packed_qkv`` and the pool's
        ``fused_inference_readout`` switch (frozen readouts through versioned activation-dtype
        copies of W).  A change drops the cached decode graph."""
        if type(enabled) is not bool:
            raise ValueError("Inference projection packing must be boolean")
        if self.training:
            raise ValueError("Call eval() before preparing inference projections")
        changed = bool(getattr(self.fast_weight_pool, "fused_inference_readout", False)) != enabled
        for block in self.layers:
            previous = block.attn._packed_qkv
            if enabled:
                block.attn.prepare_for_inference()
            else:
                block.attn._packed_qkv = None
                block.attn._packed_qkv_key = None
            changed = changed or previous is not block.attn._packed_qkv
        self.fast_weight_pool.fused_inference_readout = enabled
        if changed:
            self._cuda_graph_decoder = None

    def init_fast_state(self, batch_size: int = 1, device=None, dtype=None, detach: bool = False) -> FastWeightState:
        return self.fast_weight_pool.init_state(batch_size=batch_size, device=device, dtype=dtype, detach=detach)

    def num_parameters(self) -> Dict[str, int]:
        slow = sum(p.numel() for p in self.get_slow_parameters())
        fast = sum(p.numel() for p in self.get_meta_fast_parameters())
        return {"slow_weights": slow, "fast_weight_pool": fast, "total": slow + fast}

    # ------------------------------------------------------------------ chunk-first schedule
    def _compute_dtype(self) -> torch.dtype:
        return self.tok_embeddings.weight.dtype

    def prefill_with_writes(self, input_ids: Tensor, state: FastWeightState,
                            attention_mask: Optional[Tensor] = None,
                            kv_caches: Optional[List[Tuple[Tensor, Tensor]]] = None, start_pos: int = 0,
                            kernel_timer: Optional["K.KernelTimer"] = None, executor: bool = True):
        """Chunk-first forward with fast-weight writes, without any host synchronisation: every
        chunk of ``prefill_steps`` enqueued back to back; returns what it returns."""
        steps = self.prefill_steps(input_ids, state, attention_mask, kv_caches, start_pos, kernel_timer, executor)
        while True:
            try:
                next(steps)
            except StopIteration as done:
                return done.value

    def prefill_steps(self, input_ids: Tensor, state: FastWeightState, attention_mask: Optional[Tensor] = None,
                      kv_caches: Optional[List[Tuple[Tensor, Tensor]]] = None, start_pos: int = 0,
                      kernel_timer: Optional["K.KernelTimer"] = None, executor: bool = True):
        """Generator form of ``prefill_with_writes``: yields each chunk's index once the chunk is
        enqueued (on the stream current at the first step, which every later step must keep
        current) and returns the result.  Two prefills on different streams may interleave
        their steps: a prefill's state is its own (the chunk executor's events belong to its
        plans), and if the generator is abandoned after a chunk whose state write was deferred,
        the main stream still waits for that write.

        Chunk-first forward with fast-weight writes, without any host synchronisation.
        ``kernel_timer`` (measurement only) records events around the chain kernels it follows.
        With bf16 activations each chunk goes to the GPU in one call (``uttt_prefill_chunk``,
        ``PrefillPlan``); ``executor=False`` (or a ``kernel_timer``) enqueues it launch by launch
        from here instead, with the slow-weight products on torch.

        Per chunk: every layer's attention, projections and fast-weight readout run first
        (all readouts read the chunk-start state, reference uttt_model.py:519-608), then one
        ``uttt_chunk_chain`` launch applies the layers' chained updates to the state in place.
        Returns (hidden (B, T, D), final state tensors (6,), per-layer surprise (L,) fp32
        device tensor, per-layer KV caches (last <= window rotated keys/values)).
        """
        cfg = self.config
        if cfg.write_schedule != "sequential":
            raise ValueError("Only the causal sequential write schedule is implemented; aggregated writes must "
                             "not be silently treated as sequential")
        require_write_chunk(cfg.chunk_size)
        bsz, seq = input_ids.shape
        dev = input_ids.device
        h = F.embedding(input_ids, self.tok_embeddings.weight)
        n_layers, c = len(self.layers), cfg.chunk_size
        n_chunks = (seq + c - 1) // c
        attn0 = self.layers[0].attn
        hd, hkv, win = attn0.head_dim, attn0.n_kv_heads, attn0.window_size

        hist = 0
        if kv_caches is not None:
            hist = min(kv_caches[0][0].shape[2], win - 1)
        k_bufs, v_bufs = [], []
        for li in range(n_layers):
            kb = torch.empty((bsz, hkv, hist + seq, hd), dtype=h.dtype, device=dev)
            vb = torch.empty_like(kb)
            if hist:
                kb[:, :, :hist].copy_(kv_caches[li][0][:, :, -hist:])
                vb[:, :, :hist].copy_(kv_caches[li][1][:, :, -hist:])
            k_bufs.append(kb)
            v_bufs.append(vb)

        # one fp32 state set, updated in place chunk by chunk (the caller's tensors are not written)
        cur = tuple(t.detach().to(device=dev, dtype=torch.float32).clone(memory_format=torch.contiguous_format)
                    for t in state.tensors())
        ln_w, ln_b = state.ln_weight, state.ln_bias
        surprises = torch.zeros((n_chunks, n_layers), dtype=torch.float32, device=dev)
        counts = torch.full((n_chunks,), float(bsz * c), dtype=torch.float32, device=dev)
        if seq % c:
            counts[-1:].fill_(float(bsz * (seq % c)))
        if c > K.MAX_CHAIN_CHUNK:  # longer write chunks: one update per layer (no layer chain)
            return (yield from self._prefill_per_layer_updates(h, cur, ln_w, ln_b, attention_mask, k_bufs, v_bufs,
                                                                hist, start_pos, surprises, counts))
        # bf16 copies of the state on the bf16 path (the reference casts W to the activation
        # dtype for these matmuls): the readouts and the chain read them; each chain refreshes them
        copies = [t.to(torch.bfloat16) for t in cur] if h.dtype == torch.bfloat16 else None
        read = copies[:3] if copies is not None else cur[:3]
        pool = self.fast_weight_pool
        clip = float(pool.max_inner_grad_norm or 0.0)
        pieces = []
        # the layer chain runs on a second stream, one layer behind the forward pass: stage l
        # needs only layers <= l, and the forward of later layers needs nothing from it (every
        # readout reads the chunk-start state); the state write joins after the last readout
        main = torch.cuda.current_stream(dev)
        side = self._chain_stream(dev)
        if executor and kernel_timer is None and plan_supported(self, h, copies):
            mask_f = None
            if attention_mask is not None:
                mask_f = attention_mask.to(device=dev, dtype=torch.float32).contiguous()
                counts = F.pad(mask_f, (0, n_chunks * c - seq)).view(bsz, n_chunks, c).sum(dim=(0, 2))
            plans: Dict[int, PrefillPlan] = {}
            ws_chain = None
            capturing = torch.cuda.is_current_stream_capturing()
            pending = None  # the state-write event of a chunk whose join was deferred
            try:
                for ci in range(n_chunks):
                    off = ci * c
                    tokens = min(seq, off + c) - off
                    plan = plans.get(tokens)
                    if plan is None:
                        run = K.ChunkChainRun(n_layers, tokens, cur, ln_w, ln_b, None, pool.momentum_beta, clip,
                                              pool.normalize_loss_by_dim, pool.eps, h.dtype, copies=copies,
                                              surprise=surprises[ci], workspace=ws_chain, w_products_given=True)
                        ws_chain = run.workspace
                        plan = PrefillPlan(self, bsz, tokens, dev, k_bufs, v_bufs, hist + seq, start_pos + seq,
                                           read, ln_w, ln_b, pool.eps, run)
                        plans[tokens] = plan
                    # each chunk's state write overlaps the next chunk's layer-0 projections and
                    # attention; not in a HIP graph, whose executor runs the chunks' cross joins
                    # slower (config 2: 88 ms against 64.7 ms per prefill with every call joined)
                    pending = plan.run(h, off, start_pos + off, hist + off, mask_f, surprises[ci], main, side,
                                       defer_join=ci + 1 < n_chunks and not capturing, wait_event=pending)
                    yield ci
            finally:
                if pending is not None:  # stopped after a deferred chunk: the main stream still joins it
                    N.check(N.load_library().uttt_stream_wait_event(main.cuda_stream, pending),
                            "uttt_stream_wait_event")
            per_layer = (surprises * counts[:, None]).sum(dim=0) / counts.sum().clamp_min(1.0)
            caches = [(kb[:, :, -win:].contiguous(), vb[:, :, -win:].contiguous()) if kb.shape[2] > win
                      else (kb, vb) for kb, vb in zip(k_bufs, v_bufs)]
            return h, cur, per_layer, caches
        ws_chain = ws_read = None
        # bf16: each layer's readout also forms the chain's products of that layer's keys with
        # W_up / W_gate (one read of those weights for both), and the chain stage runs in two
        # parts: the S products and key Gram rows as soon as the keys exist, the rest after the
        # readout
        shared = copies is not None
        for ci in range(n_chunks):
            off = ci * c
            end = min(seq, off + c)
            mask = attention_mask[:, off:end] if attention_mask is not None else None
            if mask is not None:
                counts[ci].copy_(mask.to(torch.float32).sum())
            hid = h[:, off:end].contiguous()  # this chunk's residual stream, updated in place
            run = K.ChunkChainRun(n_layers, end - off, cur, ln_w, ln_b, mask, pool.momentum_beta, clip,
                                  pool.normalize_loss_by_dim, pool.eps, h.dtype, copies=copies,
                                  surprise=surprises[ci], workspace=ws_chain, w_products_given=shared)
            ws_chain = run.workspace
            for li, block in enumerate(self.layers):
                attn = block.attn
                q = attn.project(hid, start_pos + off, k_bufs[li], v_bufs[li], hist + off, norm=block.attn_norm)
                att = torch.empty((bsz, end - off, attn.n_heads, hd), dtype=h.dtype, device=dev)
                K.swa_prefill(q.transpose(1, 2), k_bufs[li], v_bufs[li], win, hist + off,
                              out=att.transpose(1, 2), kv_len=hist + end)
                hid = linear_residual(hid, att.view(bsz, end - off, -1), attn.wo.weight)
                uq, uk, uv, eta, alpha = block.uttt.projections(hid, norm=block.uttt_norm)
                ready = torch.cuda.Event()
                ready.record(main)
                if ws_read is None:
                    ws_read = K.readout_workspace(uq, read[0])
                r = K.swiglu_readout(uq, *read, ln_w, ln_b, pool.eps, workspace=ws_read,
                                     keys=uk if shared else None,
                                     key_outputs=run.w_product_outputs(li) if shared else None)
                if shared:
                    read_done = torch.cuda.Event()
                    read_done.record(main)
                hid = linear_residual(hid, r, block.uttt.w_o.weight)
                # the chain stage is enqueued after the readout it overlaps, so that a captured
                # graph's executor keeps the forward pass on one in-order queue of its own
                side.wait_event(ready)
                with torch.cuda.stream(side):
                    layer = run.set_layer(uk, uv, eta, alpha)
                    if shared:
                        run.launch(layer, part=1, timer=kernel_timer)
                        side.wait_event(read_done)
                        run.launch(layer, part=2, timer=kernel_timer)
                    else:
                        run.launch(layer, timer=kernel_timer)
            side.wait_stream(main)
            with torch.cuda.stream(side):
                if run.layers_added != run.n_layers:
                    raise ValueError(f"{run.layers_added} of {run.n_layers} layers were given")
                run.launch(run.n_layers, timer=kernel_timer)
            main.wait_stream(side)
            pieces.append(hid)
            yield ci
        per_layer = (surprises * counts[:, None]).sum(dim=0) / counts.sum().clamp_min(1.0)
        caches = [(kb[:, :, -win:].contiguous(), vb[:, :, -win:].contiguous()) if kb.shape[2] > win else (kb, vb)
                  for kb, vb in zip(k_bufs, v_bufs)]
        return torch.cat(pieces, dim=1), cur, per_layer, caches

    def _prefill_per_layer_updates(self, h: Tensor, cur: Tuple[Tensor, ...], ln_w: Tensor, ln_b: Tensor,
                                   attention_mask: Optional[Tensor], k_bufs: List[Tensor], v_bufs: List[Tensor],
                                   hist: int, start_pos: int, surprises: Tensor, counts: Tensor):
        """The chunk-first schedule for write chunks longer than the layer chain takes (the
        reference's configs write 128- and 512-token chunks): per chunk, layer by layer, the
        block's attention and projections, then one ``uttt_chunk_update`` that writes the layer's
        update into the cursor state and reads its readout through the chunk-start state
        (reference uttt_model.py:519-608 with ``fused_chunk_ttt_step``'s ``read_w_*``,
        uttt_layer.py:414-534).  The state lives in two buffer sets that swap roles per chunk:
        layer 0 writes the chunk-start set into the other one, later layers update that one in
        place, and the chunk-start set is read by every layer's readout.  Each update streams the
        fp32 state; the layer chain's single state write per chunk does not apply here.  A
        generator like ``prefill_steps``; returns the same tuple."""
        cfg = self.config
        bsz, seq, _ = h.shape
        c, n_layers = cfg.chunk_size, len(self.layers)
        n_chunks = (seq + c - 1) // c
        attn0 = self.layers[0].attn
        hd, win = attn0.head_dim, attn0.window_size
        pool = self.fast_weight_pool
        clip = float(pool.max_inner_grad_norm or 0.0)
        sets = [tuple(cur), tuple(torch.empty_like(t) for t in cur)]
        start_set = 0
        ws = None
        pieces = []
        for ci in range(n_chunks):
            off = ci * c
            end = min(seq, off + c)
            mask = attention_mask[:, off:end] if attention_mask is not None else None
            if mask is not None:
                mask = mask.to(torch.float32)
                counts[ci].copy_(mask.sum())
            snap, cursor = sets[start_set], sets[start_set ^ 1]
            hid = h[:, off:end].contiguous()
            for li, block in enumerate(self.layers):
                attn = block.attn
                q = attn.project(hid, start_pos + off, k_bufs[li], v_bufs[li], hist + off, norm=block.attn_norm)
                att = torch.empty((bsz, end - off, attn.n_heads, hd), dtype=h.dtype, device=h.device)
                K.swa_prefill(q.transpose(1, 2), k_bufs[li], v_bufs[li], win, hist + off, out=att.transpose(1, 2),
                              kv_len=hist + end)
                hid = linear_residual(hid, att.view(bsz, end - off, -1), attn.wo.weight)
                uq, uk, uv, eta, alpha = block.uttt.projections(hid, norm=block.uttt_norm)
                src = snap if li == 0 else cursor  # layer 0 writes the chunk-start state out of place
                prep = K.prepare_chunk_update(uq, uk, uv, eta, alpha, *src, ln_w, ln_b, mask, pool.momentum_beta,
                                              clip, pool.normalize_loss_by_dim, pool.eps, read_w_up=snap[0],
                                              read_w_gate=snap[1], read_w_down=snap[2], out_state=cursor,
                                              surprise=surprises[ci, li], workspace=ws)
                ws = prep.workspace
                r = prep.launch()[0]
                hid = linear_residual(hid, r, block.uttt.w_o.weight)
            start_set ^= 1
            pieces.append(hid)
            yield ci
        per_layer = (surprises * counts[:, None]).sum(dim=0) / counts.sum().clamp_min(1.0)
        caches = [(kb[:, :, -win:].contiguous(), vb[:, :, -win:].contiguous()) if kb.shape[2] > win else (kb, vb)
                  for kb, vb in zip(k_bufs, v_bufs)]
        return torch.cat(pieces, dim=1), sets[start_set], per_layer, caches

    def _chain_stream(self, device: torch.device) -> "torch.cuda.Stream":
        """The second stream the layer chain runs on (default priority, created once per device)."""
        streams = self.__dict__.setdefault("_chain_streams", {})
        key = torch.device(device).index or 0
        if key not in streams:
            streams[key] = torch.cuda.Stream(device=device)
        return streams[key]

    # ------------------------------------------------------------------ forward
    def _logits(self, h: Tensor) -> Tensor:
        return F.linear(self.norm(h), self.lm_head.weight)

    def forward(self, input_ids: Tensor, fast_state: Optional[FastWeightState] = None,
                labels: Optional[Tensor] = None, attention_mask: Optional[Tensor] = None,
                kv_caches: Optional[List[Tuple[Tensor, Tensor]]] = None, start_pos: int = 0,
                update_fast_weights: bool = True, surprise_aux_weight: float = 0.10, logits_to_keep: int = 0,
                return_fast_state: bool = True, **unsupported: Any) -> uTTTModelOutput:
        """Inference forward with the reference's arguments (uttt_model.py:714-960).

        Training-only options (meta-gradients through the writes, CE token index
        selection) are not part of the HIP path and are rejected.
        """
        if unsupported:
            raise ValueError(f"options not supported on the HIP inference path: {sorted(unsupported)}")
        if self.training and torch.is_grad_enabled():
            raise ValueError("uTTTModel on the HIP path is inference-only; call eval() / torch.no_grad()")
        bsz, seq = input_ids.shape
        if seq == 0 or self.config.chunk_size < 1:
            raise ValueError("input sequence and chunk_size must be non-empty/positive")
        dev = input_ids.device
        dt = self._compute_dtype()
        if fast_state is None:
            if not update_fast_weights and not return_fast_state:
                fast_state = self.fast_weight_pool.readonly_state(bsz, device=dev, dtype=dt, detach=True)
            else:
                state_dtype = torch.float32 if update_fast_weights else dt
                fast_state = self.init_fast_state(bsz, device=dev, dtype=state_dtype, detach=True)
        else:
            fast_state = fast_state.ensure_batch_size(bsz)

        with torch.no_grad():
            if update_fast_weights:
                h, tensors, per_layer, new_caches = self.prefill_with_writes(
                    input_ids, fast_state, attention_mask, kv_caches, start_pos)
                n_chunks = (seq + self.config.chunk_size - 1) // self.config.chunk_size
                cur = FastWeightState(*tensors, fast_state.ln_weight, fast_state.ln_bias,
                                      fast_state.step + n_chunks * len(self.layers),
                                      fast_state.last_surprise_loss, list(fast_state.surprise_history))
                floats = [float(x) for x in per_layer.tolist()]  # the reference's end-of-forward sync
                cur.last_surprise_loss = sum(floats) / max(len(floats), 1)
                cur.surprise_history = (list(cur.surprise_history) + floats)[-100:]
                layer_tensors = per_layer
            else:
                h = self.tok_embeddings(input_ids)
                cur = fast_state
                new_caches = []
                for li, block in enumerate(self.layers):
                    cache = kv_caches[li] if kv_caches is not None else None
                    h, cur, _, cache = block(h, self.fast_weight_pool, cur, attention_mask, cache, start_pos, False)
                    new_caches.append(cache)
                layer_tensors = torch.zeros(len(self.layers), dtype=torch.float32, device=dev)
                floats = [0.0] * len(self.layers)
            mean_surprise = layer_tensors.mean()

            ce_loss = total = None
            if labels is not None:
                logits = self._logits(h)
                shift = torch.full_like(labels, -100)
                shift[:, :-1] = labels[:, 1:]
                ce_loss = F.cross_entropy(logits.reshape(-1, logits.shape[-1]).float(), shift.reshape(-1),
                                          ignore_index=-100, reduction="sum") / (shift != -100).sum().clamp_min(1)
                total = ce_loss if surprise_aux_weight == 0.0 else ce_loss + surprise_aux_weight * mean_surprise
            elif logits_to_keep < 0:
                logits = torch.empty((bsz, 0, self.config.vocab_size), device=dev, dtype=h.dtype)
            elif 0 < logits_to_keep < seq:
                logits = self._logits(h[:, -logits_to_keep:])
            else:
                logits = self._logits(h)
        return uTTTModelOutput(logits=logits, fast_state=cur if return_fast_state else None, loss=total,
                               ce_loss=ce_loss, surprise_loss=mean_surprise, layer_surprise_losses=floats,
                               kv_caches=new_caches)

    # ------------------------------------------------------------------ interaction API
    @torch.no_grad()
    def test_time_update(self, interaction_ids: Tensor, fast_state: FastWeightState,
                         attention_mask: Optional[Tensor] = None) -> Tuple[FastWeightState, float, List[float]]:
        """Writes over [prompt + reply] on a copy of the state (reference uttt_model.py:1237-1271)."""
        was = self.training
        self.eval()
        try:
            out = self.forward(interaction_ids, fast_state=fast_state, attention_mask=attention_mask,
                               update_fast_weights=True, logits_to_keep=-1)
            cand = out.fast_state
            return cand, float(cand.last_surprise_loss), out.layer_surprise_losses
        finally:
            if was:
                self.train()

    def test_time_update_batched(self, interactions, fast_states, attention_masks=None,
                                 min_chunk_surprise: float = 0.0):
        """``test_time_update`` for N ragged requests in one chunk loop; one
        (candidate, surprise, per-layer surprise) tuple per request (see ``evolve``)."""
        from .evolve import ragged_test_time_update
        return ragged_test_time_update(self, interactions, fast_states, attention_masks, min_chunk_surprise)

    @staticmethod
    def _sample_next_token(logits: Tensor, temperature: float = 0.7, top_p: float = 0.9,
                           recent_tokens: Optional[List[int]] = None, repetition_penalty: float = 1.18,
                           active_vocab_limit: Optional[int] = None,
                           generator: Optional[torch.Generator] = None) -> Tensor:
        """Top-p sampling with repetition penalty and vocabulary masking (reference uttt_model.py:1181-1235)."""
        if not math.isfinite(temperature) or temperature < 0:
            raise ValueError("temperature must be finite and nonnegative")
        if not math.isfinite(top_p) or not 0 < top_p <= 1:
            raise ValueError("top_p must be finite and in (0, 1]")
        if not math.isfinite(repetition_penalty):
            raise ValueError("repetition_penalty must be finite")
        if logits.ndim != 2 or logits.shape[-1] <= UNK_ID:
            raise ValueError("Sampling logits must have batch and vocabulary dimensions")
        if active_vocab_limit is not None and active_vocab_limit <= EOS_ID:
            raise ValueError("Active vocabulary must include EOS")
        work = logits.to(dtype=torch.float32, copy=True)
        work[:, PAD_ID] = -torch.inf
        work[:, BOS_ID] = -torch.inf
        work[:, UNK_ID] = -torch.inf
        if active_vocab_limit is not None and active_vocab_limit < work.shape[-1]:
            work[:, active_vocab_limit:] = -torch.inf
        if recent_tokens and repetition_penalty > 1.0:
            idx = torch.tensor(list(set(recent_tokens[-48:])), dtype=torch.long, device=work.device)
            score = work[:, idx]
            work[:, idx] = torch.where(score < 0, score * repetition_penalty, score / repetition_penalty)
        if temperature <= 1e-5:
            return torch.argmax(work, dim=-1)
        probs = F.softmax(work / temperature, dim=-1)
        if 0.0 < top_p < 1.0:
            sp, si = torch.sort(probs, descending=True, dim=-1)
            cum = torch.cumsum(sp, dim=-1)
            sp[cum - sp > top_p] = 0.0
            sp = sp / sp.sum(dim=-1, keepdim=True).clamp_min(1e-8)
            return si.gather(-1, torch.multinomial(sp, 1, generator=generator)).squeeze(-1)
        return torch.multinomial(probs, 1, generator=generator).squeeze(-1)

    def _graph_decoder_for(self, fast_state: FastWeightState, caches, pos: int):
        """A one-request ``BatchedDecoder`` holding the prompt's caches, with its step captured in
        a HIP graph; reused while the model and the state's W are unchanged (the reference keeps
        its ``CUDAGraphDecoder`` the same way, uttt_model.py:1138-1152).  None (eager decoding)
        where the decode kernels do not take the model or state."""
        from .decoder import BatchedDecoder
        dev = self.tok_embeddings.weight.device
        if (dev.type != "cuda" or torch.is_inference_mode_enabled() or pos < 1
                or fast_state.w_up.shape[0] != 1 or fast_state._shared_readonly):
            return None
        cached = getattr(self, "_cuda_graph_decoder", None)
        try:
            if cached is not None and cached.matches(self, [fast_state]):
                cached.reset([caches], [pos])
                return cached
            self._cuda_graph_decoder = None  # release the previous state's graph first
            dec = BatchedDecoder(self, [fast_state])
            dec.reset([caches], [pos])
            dec.capture()
            self._cuda_graph_decoder = dec
            return dec
        except (RuntimeError, ValueError) as error:
            import warnings
            self._cuda_graph_decoder = None
            warnings.warn(f"HIP graph decode unavailable; using standard decode ({error})")
            return None

    @torch.no_grad()
    def stream_generate(self, input_ids: Tensor, fast_state: FastWeightState, max_new_tokens: int = 128,
                        temperature: float = 0.7, top_p: float = 0.9, eos_token_id: Optional[int] = EOS_ID,
                        speculative_draft_k: Optional[int] = None, dspark_conf_threshold: Optional[float] = None,
                        use_cuda_graph: bool = False,
                        generator: Optional[torch.Generator] = None) -> Iterator[int]:
        """Frozen-state streaming generation for one prompt (reference uttt_model.py:966-1179).

        ``use_cuda_graph`` decodes through a one-request ring-buffer ``BatchedDecoder`` whose
        step is replayed from a HIP graph (falling back to eager steps where it does not apply,
        or, with the exact KV history, when a step is refused).  The experimental
        self-speculative branch is not part of this path: a positive draft length is refused."""
        if max_new_tokens < 0:
            raise ValueError("max_new_tokens must be nonnegative")
        if max_new_tokens == 0:
            return
        if input_ids.ndim != 2 or input_ids.shape[0] != 1 or input_ids.shape[1] == 0:
            raise ValueError("Streaming generation requires one non-empty prompt")
        draft_k = (speculative_draft_k if speculative_draft_k is not None
                   else int(getattr(self.config, "dspark_speculative_k", 0)))
        if draft_k > 0:
            raise ValueError("self-speculative decoding is not part of the HIP path; use speculative_draft_k=0")
        was = self.training
        self.eval()
        try:
            out = self.forward(input_ids, fast_state=fast_state, update_fast_weights=False, logits_to_keep=1)
            caches, logits = out.kv_caches, out.logits[:, -1, :]
            pos, recent = input_ids.shape[1], []
            graph, tried = None, False
            while len(recent) < max_new_tokens:
                tok = self._sample_next_token(logits, temperature, top_p, recent, self.config.repetition_penalty,
                                              self.active_vocab_limit, generator)
                tid = int(tok.item())
                if tid in (USER_ID, ASSISTANT_ID):
                    break
                recent.append(tid)
                yield tid
                if (eos_token_id is not None and tid == eos_token_id) or len(recent) >= max_new_tokens:
                    break
                if use_cuda_graph and not tried:  # after the first token, as the reference does
                    tried = True
                    graph = self._graph_decoder_for(fast_state, caches, pos)
                if graph is not None:
                    try:
                        logits = graph.step(tok.view(1).to(graph.device))
                        pos += 1
                        continue
                    except ValueError:  # e.g. the RoPE table's end: continue eagerly from the ring
                        caches = graph.export_kv_caches(0)
                        graph = None
                        self._cuda_graph_decoder = None
                step = self.forward(tok.view(1, 1), fast_state=fast_state, kv_caches=caches, start_pos=pos,
                                    update_fast_weights=False)
                caches, logits = step.kv_caches, step.logits[:, -1, :]
                pos += 1
        finally:
            if was:
                self.train()
