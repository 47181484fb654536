"""Ragged per-request fast-weight updates for many requests in one pass (interact_and_evolve).

The reference updates one request at a time: ``uTTTPersonalizer.stream_interact_and_evolve``
(``engine/personalizer.py:480-551``) right-pads the turn to a multiple of 64 with a mask,
runs ``uTTTModel.test_time_update`` on a clone of that user's state (``model/uttt_model.py:
1237-1271``), and only if the turn's surprise passes the gate (``surprise > tau``,
``personalizer.py:524-526``) keeps the update after an elastic pull toward W_0
(``uttt_layer.py:773-832``).

``ragged_test_time_update`` runs N such updates together.  Requests are ordered by chunk
count, longest first, so the requests still running at chunk ``c`` are a leading block of
rows: every kernel of chunk ``c`` (attention, projections, readouts and the layer chain that
applies the chunk's L updates) runs over just those rows, and a request costs its own chunks
and nothing more.  A request's state rows are its own (the kernels index the state per row),
and its rows keep their final state once its last chunk is written.  Each request's result equals its
batch-1 ``test_time_update`` on the same padded turn: the chunk-first schedule, the token
masking, the per-layer surprise weighting (``uttt_model.py:598-607``) and the step count are
all per row.

``evolve_batched`` adds the reference's turn-level gate and elastic pull per request, and
optionally the per-chunk surprise gate (a chunk whose masked mean token loss is below a
threshold leaves that row's W and S unchanged), which the reference does not have.
"""
from __future__ import annotations

import math
from dataclasses import dataclass
from typing import List, Optional, Sequence, Tuple

import torch
import torch.nn.functional as F

from . import kernels as K
from .layer import FastWeightState, linear_residual, require_write_chunk
from .model import PAD_ID, uTTTModel

Tensor = torch.Tensor


@dataclass
class EvolveResult:
    """One request's outcome: the state to keep, the turn surprise, the per-layer surprise,
    whether the turn-level gate fired, and the candidate (pre-gate, pre-pull) state."""
    state: FastWeightState
    surprise: float
    layer_surprises: List[float]
    gate_triggered: bool
    candidate: FastWeightState


def _as_row(t: Tensor, name: str) -> Tensor:
    if t.dim() == 2:
        if t.shape[0] != 1:
            raise ValueError(f"{name} must be one request: shape (T,) or (1, T)")
        t = t[0]
    if t.dim() != 1 or t.shape[0] == 0:
        raise ValueError(f"{name} must be a non-empty (T,) or (1, T) tensor")
    return t


@torch.no_grad()
def ragged_test_time_update(model: uTTTModel, interactions: Sequence[Tensor],
                            fast_states: Sequence[FastWeightState],
                            attention_masks: Optional[Sequence[Optional[Tensor]]] = None,
                            min_chunk_surprise: float = 0.0) -> List[Tuple[FastWeightState, float, List[float]]]:
    """``test_time_update`` for N requests of different lengths in one chunk loop.

    ``interactions[i]`` holds request i's token ids ((T_i,) or (1, T_i)), ``fast_states[i]``
    its batch-1 state and ``attention_masks[i]`` (optional, same length) its token mask.
    Returns, per request and in the given order, what ``model.test_time_update`` returns:
    (candidate state, mean surprise over layers, per-layer surprise).  The candidate states'
    tensors are rows of shared batch tensors; the caller's states are never written.
    ``min_chunk_surprise`` > 0 switches on the per-chunk gate (not in the reference).
    """
    cfg = model.config
    if cfg.write_schedule != "sequential":
        raise ValueError("Only the causal sequential write schedule is implemented")
    require_write_chunk(cfg.chunk_size)
    if model.training and torch.is_grad_enabled():
        raise ValueError("the HIP update path is inference-only; call eval() / torch.no_grad()")
    n = len(interactions)
    if n == 0 or len(fast_states) != n:
        raise ValueError("need one state per interaction and at least one interaction")
    if attention_masks is not None and len(attention_masks) != n:
        raise ValueError("need one (possibly None) attention mask per interaction")
    if not math.isfinite(min_chunk_surprise) or min_chunk_surprise < 0.0:
        raise ValueError("min_chunk_surprise must be finite and >= 0")
    dev = model.tok_embeddings.weight.device
    if dev.type != "cuda":
        raise ValueError("the model must be on the GPU")
    c = cfg.chunk_size
    ids_rows = [_as_row(t, "interaction") for t in interactions]
    lengths = [int(t.shape[0]) for t in ids_rows]
    chunks = [(t + c - 1) // c for t in lengths]
    ln_w, ln_b = fast_states[0].ln_weight, fast_states[0].ln_bias
    for st in fast_states:
        if st.w_up.shape[0] != 1:
            raise ValueError("each request state must hold one row (batch 1)")
        if not (torch.equal(st.ln_weight, ln_w) and torch.equal(st.ln_bias, ln_b)):
            raise ValueError("all requests must share one LayerNorm pair (states of one pool)")

    # longest first: the requests still running at any chunk are a leading block of rows
    order = sorted(range(n), key=lambda i: -chunks[i])
    n_chunks = chunks[order[0]]
    seq = n_chunks * c
    ids = torch.full((n, seq), PAD_ID, dtype=torch.long)
    mask = torch.zeros((n, seq), dtype=torch.float32)
    for row, i in enumerate(order):
        ids[row, :lengths[i]] = ids_rows[i].to("cpu", torch.long)
        if attention_masks is not None and attention_masks[i] is not None:
            m = _as_row(attention_masks[i], "attention mask")
            if m.shape[0] != lengths[i]:
                raise ValueError("an attention mask must have its interaction's length")
            mask[row, :lengths[i]] = m.to("cpu", torch.float32)
        else:
            mask[row, :lengths[i]] = 1.0
    ids = ids.to(dev, non_blocking=True)
    mask = mask.to(dev, non_blocking=True)
    active = [sum(1 for i in order if chunks[i] > ci) for ci in range(n_chunks)]

    h = F.embedding(ids, model.tok_embeddings.weight)
    dt = h.dtype
    n_layers = len(model.layers)
    attn0 = model.layers[0].attn
    hd, hkv, win = attn0.head_dim, attn0.n_kv_heads, attn0.window_size
    k_bufs = [torch.empty((n, hkv, seq, hd), dtype=dt, device=dev) for _ in range(n_layers)]
    v_bufs = [torch.empty_like(kb) for kb in k_bufs]

    # the requests' states, stacked in order; each chunk's chain updates the leading rows in
    # place, so a finished request's rows keep its final state
    cur = tuple(torch.cat([getattr(fast_states[i], name).detach().to(dev, torch.float32) for i in order])
                .contiguous() for name in ("w_up", "w_gate", "w_down", "s_up", "s_gate", "s_down"))
    ln_w = ln_w.to(dev)
    ln_b = ln_b.to(dev)
    copies = [t.to(torch.bfloat16) for t in cur] if dt == torch.bfloat16 else None
    read = copies[:3] if copies is not None else cur[:3]
    row_loss = torch.zeros((n_layers, n, 2), dtype=torch.float32, device=dev)
    surprise = torch.empty((n_chunks, n_layers), dtype=torch.float32, device=dev)
    pool = model.fast_weight_pool
    clip = float(pool.max_inner_grad_norm or 0.0)
    ws_chain = ws_read = None
    main = torch.cuda.current_stream(dev)
    side = model._chain_stream(dev)  # the layer chain runs one layer behind the forward pass
    # bf16: each layer's readout also forms the chain's products of that layer's keys with W_up /
    # W_gate (one read of those weights for both), and the chain stage runs in two parts, as in
    # the model's prefill with writes
    shared = copies is not None
    long_chunks = c > K.MAX_CHAIN_CHUNK
    if long_chunks:  # one update per layer; two state sets that swap roles per chunk
        sets = [cur, tuple(torch.empty_like(t) for t in cur)]
        ws_update = None
    for ci in range(n_chunks):
        rows, off = active[ci], ci * c
        end = off + c
        cur_mask = mask[:rows, off:end]
        hid = h[:rows, off:end].contiguous()  # this chunk's residual stream, updated in place
        rd = [t[:rows] for t in read]
        chunk_rl = torch.empty((n_layers, rows, 2), dtype=torch.float32, device=dev)
        if long_chunks:
            # chunks longer than the layer chain takes (the reference's configs write 128 and 512):
            # per layer, the update into the cursor set with the readout through the chunk-start
            # set (layer 0 writes the chunk-start set into the other one)
            snap = [t[:rows] for t in sets[ci % 2]]
            cursor = [t[:rows] for t in sets[(ci + 1) % 2]]
            for li, block in enumerate(model.layers):
                attn = block.attn
                kb, vb = k_bufs[li][:rows], v_bufs[li][:rows]
                q = attn.project(hid, off, kb, vb, off, norm=block.attn_norm)
                att = torch.empty((rows, c, attn.n_heads, hd), dtype=dt, device=dev)
                K.swa_prefill(q.transpose(1, 2), kb, vb, win, off, out=att.transpose(1, 2), kv_len=end)
                hid = linear_residual(hid, att.view(rows, c, -1), attn.wo.weight)
                uq, uk, uv, eta, alpha = block.uttt.projections(hid, norm=block.uttt_norm)
                prep = K.prepare_chunk_update(uq, uk, uv, eta, alpha, *(snap if li == 0 else cursor), ln_w, ln_b,
                                              cur_mask, pool.momentum_beta, clip, pool.normalize_loss_by_dim,
                                              pool.eps, read_w_up=snap[0], read_w_gate=snap[1], read_w_down=snap[2],
                                              out_state=cursor, surprise=surprise[ci, li], workspace=ws_update,
                                              row_loss=chunk_rl[li], min_row_surprise=min_chunk_surprise)
                ws_update = prep.workspace
                hid = linear_residual(hid, prep.launch()[0], block.uttt.w_o.weight)
            row_loss[:, :rows] += chunk_rl
            continue
        run = K.ChunkChainRun(n_layers, c, [t[:rows] for t in cur], ln_w, ln_b, cur_mask, pool.momentum_beta, clip,
                              pool.normalize_loss_by_dim, pool.eps, dt,
                              copies=None if copies is None else [t[:rows] for t in copies],
                              surprise=surprise[ci], row_loss=chunk_rl, min_row_surprise=min_chunk_surprise,
                              workspace=ws_chain, w_products_given=shared)
        ws_chain = run.workspace
        for li, block in enumerate(model.layers):
            attn = block.attn
            kb, vb = k_bufs[li][:rows], v_bufs[li][:rows]
            q = attn.project(hid, off, kb, vb, off, norm=block.attn_norm)
            att = torch.empty((rows, c, attn.n_heads, hd), dtype=dt, device=dev)
            K.swa_prefill(q.transpose(1, 2), kb, vb, win, off, out=att.transpose(1, 2), kv_len=end)
            hid = linear_residual(hid, att.view(rows, c, -1), attn.wo.weight)
            uq, uk, uv, eta, alpha = block.uttt.projections(hid, norm=block.uttt_norm)
            ready = torch.cuda.Event()
            ready.record(main)
            if ws_read is None:
                ws_read = K.readout_workspace(uq, rd[0])
            r = K.swiglu_readout(uq, *rd, ln_w, ln_b, pool.eps, workspace=ws_read, keys=uk if shared else None,
                                 key_outputs=run.w_product_outputs(li) if shared else None)
            if shared:
                read_done = torch.cuda.Event()
                read_done.record(main)
            hid = linear_residual(hid, r, block.uttt.w_o.weight)
            side.wait_event(ready)  # enqueued after the readout it overlaps
            with torch.cuda.stream(side):
                if shared:
                    layer = run.set_layer(uk, uv, eta, alpha)
                    run.launch(layer, part=1)
                    side.wait_event(read_done)
                    run.launch(layer, part=2)
                else:
                    run.add_layer(uk, uv, eta, alpha)
        side.wait_stream(main)
        with torch.cuda.stream(side):
            run.finish()
        main.wait_stream(side)
        row_loss[:, :rows] += chunk_rl

    final = cur
    if long_chunks:  # a request's final state is in the set its last chunk wrote
        for row, i in enumerate(order):
            if chunks[i] % 2:
                for dst, src in zip(sets[0], sets[1]):
                    dst[row].copy_(src[row])
    per_layer = (row_loss[..., 0] / row_loss[..., 1].clamp_min(1.0)).t()  # (N, L)
    floats = per_layer.tolist()  # the reference's end-of-forward read, once for all requests

    results: List[Optional[Tuple[FastWeightState, float, List[float]]]] = [None] * n
    for row, i in enumerate(order):
        st = fast_states[i]
        layers = [float(x) for x in floats[row]]
        mean = sum(layers) / max(len(layers), 1)
        cand = FastWeightState(*(t[row:row + 1] for t in final), st.ln_weight, st.ln_bias,
                               st.step + chunks[i] * n_layers, mean,
                               (list(st.surprise_history) + layers)[-100:])
        results[i] = (cand, mean, layers)
    return results  # type: ignore[return-value]


@torch.no_grad()
def evolve_batched(model: uTTTModel, interactions: Sequence[Tensor], fast_states: Sequence[FastWeightState],
                   attention_masks: Optional[Sequence[Optional[Tensor]]] = None,
                   surprise_threshold: float = 0.5, anchor_lambda: float = 0.02,
                   max_drift_ratio: Optional[float] = 0.35,
                   min_chunk_surprise: float = 0.0) -> List[EvolveResult]:
    """Update, gate and pull N requests (``personalizer.py:480-551`` per request).

    A request whose turn surprise exceeds ``surprise_threshold`` keeps its candidate state
    after ``apply_elastic_pull(anchor_lambda, max_drift_ratio)``; the others keep their
    state.  A non-finite or negative surprise raises ``ValueError`` (``personalizer.py:524``)
    before any request is changed.
    """
    updates = ragged_test_time_update(model, interactions, fast_states, attention_masks, min_chunk_surprise)
    for _, s, _ in updates:
        if not math.isfinite(s) or s < 0:
            raise ValueError("Test-time update returned a non-finite or negative surprise loss; "
                             "no persona was changed")
    gated = [i for i, (_, s, _) in enumerate(updates) if s > surprise_threshold]
    pulled = {}
    if gated:
        # one batched pull over the gated requests' rows
        rows = [updates[i][0] for i in gated]
        w = [torch.cat([getattr(st, name) for st in rows]) for name in ("w_up", "w_gate", "w_down")]
        joined = FastWeightState(*w, *(torch.cat([getattr(st, name) for st in rows])
                                       for name in ("s_up", "s_gate", "s_down")),
                                 rows[0].ln_weight, rows[0].ln_bias)
        stab = model.fast_weight_pool.apply_elastic_pull(joined, anchor_lambda, max_drift_ratio)
        for j, i in enumerate(gated):
            cand = updates[i][0]
            pulled[i] = FastWeightState(stab.w_up[j:j + 1], stab.w_gate[j:j + 1], stab.w_down[j:j + 1],
                                        cand.s_up, cand.s_gate, cand.s_down, cand.ln_weight, cand.ln_bias,
                                        cand.step, cand.last_surprise_loss, list(cand.surprise_history))
    out = []
    for i, (cand, s, layers) in enumerate(updates):
        out.append(EvolveResult(pulled.get(i, fast_states[i]), s, layers, i in pulled, cand))
    return out
