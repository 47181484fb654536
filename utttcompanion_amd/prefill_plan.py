"""Host side of the one-call chunk executor (``uttt_prefill_chunk``) for the chunk-first prefill
with fast-weight writes (reference model/uttt_model.py:453-608).

A ``PrefillPlan`` marshals, once per prefill and chunk length, every per-layer call of a chunk
(the argument structs of the entry points the per-call path launches one by one) against
buffers the plan owns: the chunk's residual rows, the QKV and projection products, the
attention output, each layer's q / k / v / eta / alpha (the layer chain reads every layer's k,
v, eta and alpha until the chunk's state write), the readout rows and the workspaces.  Per
chunk the host then copies the chunk's rows in, makes one library call that enqueues the whole
chunk on the two streams, and copies the rows out: the per-layer kernels are the same, only
the slow-weight products run on ``uttt_linear`` instead of the library GEMM, and the host no
longer spends a binding call per launch.
"""
from __future__ import annotations

import ctypes as C
from typing import List, Optional, Sequence

import torch
from torch import Tensor

from . import _native as N
from . import kernels as K


def plan_supported(model, h: Tensor, copies) -> bool:
    """Whether ``uttt_prefill_chunk`` runs this prefill: bf16 activations with the state's bf16
    copies (the shared-weight-read schedule) and slow-weight products whose k is a multiple of
    64."""
    if h.dtype != torch.bfloat16 or copies is None or h.device.type != "cuda":
        return False
    attn = model.layers[0].attn
    return (model.config.d_model % 64 == 0 and (attn.n_heads * attn.head_dim) % 64 == 0
            and len(model.layers) <= N.MAX_CHAIN)


class PrefillPlan:
    """Every layer's calls of one chunk of ``tokens`` tokens, marshalled once.

    ``chain`` is the chunk's ``ChunkChainRun`` built with this plan's layer inputs (its mask and
    surprise row are set per chunk by the executor); ``k_bufs`` / ``v_bufs`` are the prefill's
    per-layer KV buffers, ``kv_capacity`` their length, ``rope_len`` the RoPE table length needed
    (the last position + 1)."""

    def __init__(self, model, bsz: int, tokens: int, dev: torch.device, k_bufs: Sequence[Tensor],
                 v_bufs: Sequence[Tensor], kv_capacity: int, rope_len: int, read: Sequence[Tensor],
                 ln_w: Tensor, ln_b: Tensor, eps: float, chain: "K.ChunkChainRun") -> None:
        cfg = model.config
        layers = model.layers
        n_layers = len(layers)
        attn0 = layers[0].attn
        dim, hd, heads, hkv, win = cfg.d_model, attn0.head_dim, attn0.n_heads, attn0.n_kv_heads, attn0.window_size
        act = torch.bfloat16
        rows = bsz * tokens
        self.tokens, self.n_layers, self.chain = tokens, n_layers, chain
        self.kv_capacity, self.rope_len = kv_capacity, rope_len
        # buffers shared by the layers (each consumed inside its layer on the main stream)
        self.hid = torch.empty((bsz, tokens, dim), dtype=act, device=dev)
        self.qkv = torch.empty((bsz, tokens, heads + 2 * hkv, hd), dtype=act, device=dev)
        self.att = torch.empty((bsz, tokens, heads, hd), dtype=act, device=dev)
        # the projection rows padded to whole 16-byte vectors (the epilogue's vector path)
        self.y = torch.empty((rows, (3 * dim + 2 + 7) // 8 * 8), dtype=act, device=dev)[:, :3 * dim + 2]
        self.r = torch.empty((bsz, tokens, dim), dtype=act, device=dev)
        # per layer: q, k, v and eta, alpha (the chain reads layers <= l until the state write);
        # layer 0 has a second set, used by every other chunk: a chunk's layer-0 epilogue may
        # run while the previous chunk's state write still reads layer 0's keys
        new_out = lambda: (torch.empty((3, rows, dim), dtype=act, device=dev),
                           torch.empty((2, rows), dtype=act, device=dev))
        self.proj_out = [new_out() for _ in range(n_layers)]
        self.proj_out0_alt = new_out()
        lib = N.load_library()
        n_qkv = (heads + 2 * hkv) * hd
        need = max(lib.uttt_linear_workspace(rows, n, k) for n, k in
                   ((n_qkv, dim), (dim, heads * hd), (3 * dim + 2, dim), (dim, dim)))
        self.linear_ws = torch.zeros(max(need, 256), dtype=torch.uint8, device=dev)
        # the attention's split count (and partials) depends on the keys in range: size the
        # workspace for every KV length a chunk of this plan can see
        nbytes = max(lib.uttt_swa_prefill_workspace(bsz, heads, tokens, kv, hd, win)
                     for kv in range(tokens, kv_capacity + 1))
        self.attn_ws = torch.empty(max(nbytes, 16), dtype=torch.uint8, device=dev)
        self.read_ws = K.readout_workspace(self.hid, read[0])
        hid2 = self.hid.view(rows, dim)
        q = self.qkv[:, :, :heads]
        k = self.qkv[:, :, heads:heads + hkv]
        v = self.qkv[:, :, heads + hkv:]
        keep: List = []
        calls = (N.PrefillLayerCalls * n_layers)()
        for li, block in enumerate(layers):
            attn, uttt = block.attn, block.uttt
            c = calls[li]
            w_qkv = attn.packed_qkv_folded(block.attn_norm).to(act)
            c.qkv = K.linear(hid2, w_qkv, out=self.qkv.view(rows, n_qkv), workspace=self.linear_ws, build_only=True)
            cos, sin = attn.rope.tables(rope_len, dev)
            c.rope = K.rope_kv_append(q, k, v, cos, sin, 0, k_bufs[li], v_bufs[li], 0, x=self.hid,
                                      x_eps=block.attn_norm.eps, build_only=True)
            c.attn = K.swa_prefill(q.transpose(1, 2), k_bufs[li], v_bufs[li], win, 0, out=self.att.transpose(1, 2),
                                   kv_len=tokens, workspace=self.attn_ws, build_only=True)
            w_o_attn = attn.wo.weight.detach().to(act)
            c.attn_out = K.linear(self.att.view(rows, heads * hd), w_o_attn, out=hid2, residual=hid2,
                                  workspace=self.linear_ws, build_only=True)
            w_proj, eab = uttt.packed_projection_folded(block.uttt_norm)
            w_proj = w_proj.to(act)
            c.proj = K.linear(hid2, w_proj, out=self.y, workspace=self.linear_ws, build_only=True)
            eab = eab.to(act)

            def epilogue_readout(cc, outs):
                # the epilogue into ``outs`` and the readout of its q / k rows; returns k, v, eta, alpha
                cc.epilogue, kept = K.proj_epilogue(self.y, dim, uttt.q_norm.weight, uttt.k_norm.weight,
                                                    uttt.q_norm.eps, uttt.base_inner_lr, uttt.base_weight_decay,
                                                    x=self.hid, x_eps=block.uttt_norm.eps, eta_alpha_bias=eab,
                                                    outs=outs, build_only=True)
                qkv3, ea = outs
                uq, uk, uv = (t.view(bsz, tokens, dim) for t in qkv3)
                eta, alpha = (t.view(bsz, tokens, 1) for t in ea)
                cc.readout, ws, kept_r = K.swiglu_readout(uq, *read, ln_w, ln_b, eps, out=self.r,
                                                          workspace=self.read_ws, keys=uk,
                                                          key_outputs=chain.w_product_outputs(li), build_only=True)
                cc.readout_workspace, cc.readout_workspace_bytes = ws.data_ptr(), ws.numel()
                keep.extend([kept, kept_r])
                return uk, uv, eta, alpha

            layer_inputs = epilogue_readout(c, self.proj_out[li])
            w_o = uttt.w_o.weight.detach().to(act)
            c.uttt_out = K.linear(self.r.view(rows, dim), w_o, out=hid2, residual=hid2, workspace=self.linear_ws,
                                  build_only=True)
            chain.set_layer(*layer_inputs)
            if li == 0:
                # the same layer-0 calls and chain inputs over the second buffer set
                calls_alt = (N.PrefillLayerCalls * n_layers)()
                calls_alt[0] = N.PrefillLayerCalls.from_buffer_copy(c)
                layer0_alt = epilogue_readout(calls_alt[0], self.proj_out0_alt)
            keep += [w_qkv, cos, sin, w_o_attn, w_proj, w_o]
        for li in range(1, n_layers):
            calls_alt[li] = calls[li]
        if chain.args.k[0] != self.proj_out[0][0][1].data_ptr():
            raise RuntimeError("the chain's layer-0 keys are not the epilogue's output rows")
        chain_alt = N.ChunkChainArgs.from_buffer_copy(chain.args)
        k0, v0, eta0, alpha0 = layer0_alt
        chain_alt.k[0], chain_alt.v[0] = k0.data_ptr(), v0.data_ptr()
        chain_alt.eta[0], chain_alt.alpha[0] = eta0.data_ptr(), alpha0.data_ptr()
        self.calls, self._keep = (calls, calls_alt), keep
        self._chain_args = (chain.args, chain_alt)
        # the events that order the two streams belong to the plan (no state in the library): two
        # per layer, the forward's end and the state write, created on this device, destroyed
        # with the plan
        self._lib = lib
        self._n_events = 2 * n_layers + 2
        self._events = (C.c_void_p * self._n_events)()
        with torch.cuda.device(dev):
            N.check(lib.uttt_events_create(self._n_events, self._events), "uttt_events_create")
        self.args = []
        for cl, ch in zip(self.calls, self._chain_args):
            args = N.PrefillChunkArgs()
            args.n_layers = n_layers
            args.layers = C.cast(cl, C.POINTER(N.PrefillLayerCalls))
            args.chain = C.pointer(ch)
            args.chain_workspace, args.chain_workspace_bytes = chain.workspace.data_ptr(), chain.workspace.numel()
            args.events, args.n_events = C.cast(self._events, C.POINTER(C.c_void_p)), self._n_events
            self.args.append(args)
        self._next = 0  # which buffer set the next chunk uses

    @property
    def state_write_event(self) -> int:
        """Handle of the event the state write of this plan's calls records (what a deferred
        call hands to the next one)."""
        return int(self._events[self._n_events - 1])

    def __del__(self) -> None:
        events = getattr(self, "_events", None)
        if events is not None and getattr(self, "_lib", None) is not None:
            # an event whose recorded work is still running is released when that work ends
            self._lib.uttt_events_destroy(self._n_events, events)
            self._events = None

    def run(self, h: Tensor, off: int, start_pos: int, kv_offset: int, mask: Optional[Tensor],
            surprise: Tensor, main: "torch.cuda.Stream", side: "torch.cuda.Stream", defer_join: bool = False,
            wait_event: Optional[int] = None) -> Optional[int]:
        """One chunk: rows ``off .. off + tokens`` of ``h`` (B, T, D) are updated in place through
        every layer, and the chain writes the state; ``mask`` is the fp32 (B, T) token mask (or
        None) and ``surprise`` this chunk's (layers,) row.  ``defer_join``: ``main`` does not wait
        for the state write; the call returns the state write's event handle, which the caller
        passes as ``wait_event`` to its next call (of this plan or another plan of the same
        prefill), whose ``main`` waits for it before its layer-0 readout (consecutive chunks of a
        plan alternate layer 0's buffers for that).  The last chunk of a prefill passes False.
        Neither is allowed under graph capture (``ValueError``)."""
        if (defer_join or wait_event is not None) and torch.cuda.is_current_stream_capturing():
            raise ValueError("a deferred join cannot be part of a graph capture: every captured chunk joins its "
                             "own state write")
        end = off + self.tokens
        # the executor sets these per chunk where the wrappers checked them per call
        if not (0 <= kv_offset and kv_offset + self.tokens <= self.kv_capacity and 0 <= start_pos
                and start_pos + self.tokens <= self.rope_len and 0 <= off and end <= h.shape[1]):
            raise ValueError("chunk outside the planned KV buffers or RoPE tables")
        if mask is not None and (mask.dtype != torch.float32 or mask.shape != h.shape[:2] or mask.stride(1) != 1):
            raise ValueError("mask must be the fp32 (B, T) token mask")
        if surprise.shape != (self.n_layers,) or surprise.dtype != torch.float32 or not surprise.is_contiguous():
            raise ValueError("surprise must be a contiguous fp32 (layers,) tensor")
        self.hid.copy_(h[:, off:end])
        a = self.args[self._next]
        self._next ^= 1
        a.start_pos, a.kv_offset, a.defer_join = int(start_pos), int(kv_offset), int(bool(defer_join))
        a.wait_event = wait_event
        if mask is not None:
            a.token_mask, a.mask_row_stride = mask.data_ptr() + off * mask.element_size(), mask.stride(0)
        else:
            a.token_mask, a.mask_row_stride = None, 0
        a.surprise = surprise.data_ptr()
        lib = N.load_library()
        N.check(lib.uttt_prefill_chunk(C.byref(a), main.cuda_stream, side.cuda_stream), "uttt_prefill_chunk")
        h[:, off:end].copy_(self.hid)
        return self.state_write_event if defer_join else None
