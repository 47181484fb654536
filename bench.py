#!/usr/bin/env python3
"""Benchmark of the uTTT hot path on one MI355X; prints one JSON line on stdout.

Workload: the ~151M-label uTTT model (12 layers, d_model 768,
12 x 64 heads, 4 kv heads, window 512, shared SwiGLU fast weights F = 2048, chunk 64,
vocab 32000), bf16 activations with fp32 fast-weight masters, random-init weights, token
ids uniform over the vocabulary, batch 8 x 2048.  One step = one full prefill with the
per-chunk fast-weight writes of every layer (the chunk-first schedule), recorded once
into a HIP graph and replayed.  ``value`` = tokens / s over the timed steps.

Per chunk the prefill runs every layer's attention, projections and readout, then one layer
chain (``uttt_chunk_chain``) that applies the chunk's 12 chained fast-weight updates.

Also reported:
* ``roofline``: the chain's state write (``k_chain_apply_lds`` after the last layer's small
  recurrence step; the largest single kernel of the prefill), timed live with HIP events
  between the chain's stream-ordered stages at the
  config-2 chunk shape (8 rows, 12 layers, C 64, D 768, F 2048), against 48 D F bytes per
  row (W and S read and written once per chunk), with the HBM traffic rocprofv3 measured;
* ``chain``: the whole chain per chunk and its stages;
* ``update``: the single-chunk update (``uttt_chunk_update``, the per-layer drop-in for
  ``fused_chunk_ttt_step``) phase by phase, with its own dominant kernel's roofline;
* ``config3_prefill``, ``config5_evolve``: the 1.58B-label model's prefill and the ragged
  per-request updates of 16 requests;
* ``decode``: the ring-buffer SWA decode kernel at the config-4 shape (32 requests,
  4 kv heads x 64, window 512, bf16) against its K/V bytes;
* ``cpu_baseline``: the CPU oracle (tests-only restatement) on a bounded sample of the
  same workload, on this host's cores.
"""
from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time

METRIC = "chunk-TTT layer prefill tok/s + SWA decode tok/s; % of MFMA/HBM roofline"
PEAK_HBM_GBS = 8000.0
PEAK_BF16_TFLOPS = 2500.0

C2 = dict(vocab_size=32000, d_model=768, n_layers=12, n_heads=12, n_kv_heads=4, d_ff_fast=2048,
          sliding_window_size=512, chunk_size=64, max_seq_len=4096)
C2_BATCH, C2_SEQ = 8, 2048
C3 = dict(vocab_size=32000, d_model=2048, n_layers=24, n_heads=16, n_kv_heads=4, d_ff_fast=5504,
          sliding_window_size=1024, chunk_size=64, max_seq_len=4096)
C3_BATCH, C3_SEQ = 4, 4096
C5_REQUESTS, C5_LENGTHS = 16, (128, 4096)
PHASES = ("k_up_gate", "k_down_partial", "k_ln_grad+k_ln_readout", "k_backward", "k_apply")


def measured_traffic(kernel: str):
    """HBM bytes per launch of ``kernel`` at the config-2 update shape, from the committed
    rocprofv3 FETCH_SIZE / WRITE_SIZE summary (scaled by a copy kernel of known size), or
    None when no summary for that kernel is present."""
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles", f"{kernel}_c2_traffic.md")
    try:
        with open(path) as fh:
            for line in fh:
                if line.startswith("traffic_bytes_per_launch:"):
                    return int(line.split(":", 1)[1].strip())
    except OSError:
        return None
    return None


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def parse_args():
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=5)
    ap.add_argument("--warmup", type=int, default=2)
    ap.add_argument("--phase-iters", type=int, default=20)
    ap.add_argument("--no-cpu-baseline", action="store_true", help="skip the CPU oracle timing")
    ap.add_argument("--sections", default="prefill,update,chain,decode,cpu,c3,evolve",
                    help="comma list of prefill, update, chain, decode, cpu, c3, evolve, copyref "
                         "(profiling runs pick a subset)")
    ap.add_argument("--c3-steps", type=int, default=2, help="timed config-3 prefills / config-5 updates")
    ap.add_argument("--cpu-tokens", type=int, default=2048, help="tokens per row of the CPU baseline sample")
    ap.add_argument("--cpu-rows", type=int, default=4, help="rows of the CPU baseline sample")
    ap.add_argument("--decode-steps", type=int, default=256)
    return ap.parse_args()


def build_model():
    import torch
    from utttcompanion_amd import uTTTConfig, uTTTModel
    torch.manual_seed(0)
    model = uTTTModel(uTTTConfig(**C2)).eval()
    model = model.to("cuda").to(torch.bfloat16)
    model.fast_weight_pool.float()
    return model


def bench_prefill(model, steps: int, warmup: int):
    import torch
    g = torch.Generator().manual_seed(1)
    ids = torch.randint(0, C2["vocab_size"], (C2_BATCH, C2_SEQ), generator=g).to("cuda")
    state = model.init_fast_state(C2_BATCH, device="cuda", dtype=torch.float32, detach=True)
    with torch.no_grad():
        log("eager warmup prefill")
        model.prefill_with_writes(ids, state)
        torch.cuda.synchronize()
        log("capturing the prefill into a HIP graph")
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            out = model.prefill_with_writes(ids, state)
        torch.cuda.synchronize()
        for _ in range(warmup):
            graph.replay()
        torch.cuda.synchronize()
        log(f"timing {steps} replays")
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        start.record()
        for _ in range(steps):
            graph.replay()
        end.record()
        torch.cuda.synchronize()
        ms = start.elapsed_time(end) / steps
    finite = bool(torch.isfinite(out[0]).all().item()) and bool(torch.isfinite(out[2]).all().item())
    return ms, finite


def bench_update_phases(iters: int):
    """HIP-event timing of each update phase at the config-2 shape (read snapshot distinct
    from the cursor, as for layers 1..L-1 of a chunk; state updated in place)."""
    import torch
    from utttcompanion_amd import kernels as K
    from utttcompanion_amd import _native as N
    B, C, D, F = C2_BATCH, C2["chunk_size"], C2["d_model"], C2["d_ff_fast"]
    g = torch.Generator(device="cuda").manual_seed(2)
    act = lambda *s: torch.randn(*s, device="cuda", generator=g).to(torch.bfloat16)
    q, k, v = act(B, C, D), act(B, C, D), act(B, C, D)
    eta = torch.full((B, C, 1), 0.005, device="cuda").to(torch.bfloat16)
    alpha = torch.full((B, C, 1), 0.001, device="cuda").to(torch.bfloat16)
    w = [torch.randn(B, D, F, device="cuda", generator=g) * 0.03, torch.randn(B, D, F, device="cuda", generator=g) * 0.03,
         torch.randn(B, F, D, device="cuda", generator=g) * 0.003]
    s = [torch.zeros_like(t) for t in w]
    r = [t.clone() for t in w]
    ln_w, ln_b = torch.ones(D, device="cuda"), torch.zeros(D, device="cuda")
    with torch.no_grad():
        prep = K.prepare_chunk_update(q, k, v, eta, alpha, *w, *s, ln_w, ln_b, None, 0.9, 1.0, True, 1e-5,
                                      *r, out_state=w + s)
        for _ in range(3):
            prep.launch()
        torch.cuda.synchronize()
        n = N.UPDATE_PHASES
        events = [[torch.cuda.Event(enable_timing=True) for _ in range(n + 1)] for _ in range(iters)]
        for it in range(iters):
            events[it][0].record()
            for p in range(n):
                prep.launch(p)
                events[it][p + 1].record()
        torch.cuda.synchronize()
    per = [sum(events[it][p].elapsed_time(events[it][p + 1]) for it in range(iters)) / iters for p in range(n)]
    return per, dict(B=B, C=C, D=D, F=F)


def bench_chain(iters: int, B: int = None, L: int = None, D: int = None, F: int = None):
    """HIP-event timing of one chunk's layer chain (``uttt_chunk_chain``) at the config-2
    shape (8 rows, 12 layers, C 64, D 768, F 2048), bf16 activations, fp32 state in place."""
    import torch
    from utttcompanion_amd import kernels as K
    B = B or C2_BATCH
    L = L or C2["n_layers"]
    D = D or C2["d_model"]
    F = F or C2["d_ff_fast"]
    C = C2["chunk_size"]
    g = torch.Generator(device="cuda").manual_seed(9)
    act = lambda *s: (torch.randn(*s, device="cuda", generator=g)).to(torch.bfloat16)
    ks = [act(B, C, D) for _ in range(L)]
    vs = [act(B, C, D) for _ in range(L)]
    etas = [torch.full((B, C), 0.005, device="cuda").to(torch.bfloat16) for _ in range(L)]
    alphas = [torch.full((B, C), 0.001, device="cuda").to(torch.bfloat16) for _ in range(L)]
    state = [torch.randn(B, D, F, device="cuda", generator=g) * 0.03, torch.randn(B, D, F, device="cuda", generator=g) * 0.03,
             torch.randn(B, F, D, device="cuda", generator=g) * 0.003]
    state += [torch.zeros_like(t) for t in state]
    copies = [t.to(torch.bfloat16) for t in state]
    ln_w, ln_b = torch.ones(D, device="cuda"), torch.zeros(D, device="cuda")
    with torch.no_grad():
        prep = K.prepare_chunk_chain(ks, vs, etas, alphas, state, ln_w, ln_b, None, 0.9, 1.0, True, 1e-5,
                                     copies=copies)
        for _ in range(2):
            prep.launch()
        torch.cuda.synchronize()
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record()
        for _ in range(iters):
            prep.launch()
        end.record()
        torch.cuda.synchronize()
        # the same chain stage by stage, with events between the stages (stream order kept)
        ev = [[torch.cuda.Event(enable_timing=True) for _ in range(L + 2)] for _ in range(iters)]
        for it in range(iters):
            ev[it][0].record()
            for stg in range(L + 1):
                prep.launch(stg)
                ev[it][stg + 1].record()
        torch.cuda.synchronize()
    stage_ms = [sum(ev[it][k].elapsed_time(ev[it][k + 1]) for it in range(iters)) / iters for k in range(L + 1)]
    return start.elapsed_time(end) / iters, stage_ms, dict(B=B, L=L, C=C, D=D, F=F)


def phase_work(p: int, B: int, C: int, D: int, F: int):
    """Algorithmic (bytes, flops) of one launch of phase p (two read paths: K through the
    cursor, Q through a distinct snapshot).  Bytes count the fp32 state each phase must
    stream once; activations (<= 64 tokens per row) are second order and left out."""
    DF = D * F
    if p == 0:
        return 16 * DF * B, 8 * C * DF * B
    if p == 1:
        return 8 * DF * B, 4 * C * DF * B
    if p == 2:
        return 0, 0
    if p == 3:
        return 4 * DF * B, 8 * C * DF * B
    return 48 * DF * B, 6 * C * DF * B


def bench_decode(iters: int):
    """The ring-buffer decode kernel at the config-4 shape: one decode step's 12 layer calls
    (each layer its own rings) recorded in a HIP graph, replayed ``iters`` times."""
    import torch
    from utttcompanion_amd import kernels as K
    N_REQ, H, HKV, HD, W, LAYERS = 32, 12, 4, 64, 512, 12
    g = torch.Generator(device="cuda").manual_seed(3)
    q = torch.randn(N_REQ, H, HD, device="cuda", generator=g).to(torch.bfloat16)
    kn = torch.randn(N_REQ, HKV, HD, device="cuda", generator=g).to(torch.bfloat16)
    vn = torch.randn_like(kn)
    rings = [(torch.randn(N_REQ, HKV, W, HD, device="cuda", generator=g).to(torch.bfloat16),
              torch.randn(N_REQ, HKV, W, HD, device="cuda", generator=g).to(torch.bfloat16)) for _ in range(LAYERS)]
    pos = torch.randint(W, 4 * W, (N_REQ,), device="cuda", generator=g)
    out = torch.empty_like(q)
    ws = torch.empty(1 << 20, dtype=torch.uint8, device="cuda")
    with torch.no_grad():
        for kr, vr in rings:
            K.swa_decode(q, kn, vn, kr, vr, pos, out=out, workspace=ws)
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            for kr, vr in rings:
                K.swa_decode(q, kn, vn, kr, vr, pos, out=out, workspace=ws)
        graph.replay()
        torch.cuda.synchronize()
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record()
        for _ in range(iters):
            graph.replay()
        end.record()
        torch.cuda.synchronize()
    ms = start.elapsed_time(end) / (iters * LAYERS)
    kv_bytes = 2 * N_REQ * HKV * W * HD * 2 + 2 * N_REQ * HKV * HD * 2 + 2 * N_REQ * H * HD * 2
    return ms, kv_bytes, dict(requests=N_REQ, heads=H, kv_heads=HKV, head_dim=HD, window=W)


def bench_decode_readout(iters: int):
    """The decode step's dominant kernel at the config-4 shape: the one-launch fast-weight
    readout (q_norm, GEMV through the 32 requests' bf16 copies, LayerNorm in each request's last
    block) of one token per request, 12 calls (one per layer, each its own copies) recorded in
    a HIP graph and replayed ``iters`` times.  Returns (us per call, algorithmic bytes per call)."""
    import torch
    from utttcompanion_amd import kernels as K
    N_REQ, D, F, LAYERS = 32, C2["d_model"], C2["d_ff_fast"], C2["n_layers"]
    g = torch.Generator(device="cuda").manual_seed(4)
    xs = [torch.randn(N_REQ, 1, D, device="cuda", generator=g).to(torch.bfloat16) for _ in range(LAYERS)]
    ws = [[(0.02 * torch.randn(N_REQ, D, F, device="cuda", generator=g)).to(torch.bfloat16),
           (0.02 * torch.randn(N_REQ, D, F, device="cuda", generator=g)).to(torch.bfloat16),
           (0.02 * torch.randn(N_REQ, F, D, device="cuda", generator=g)).to(torch.bfloat16)] for _ in range(LAYERS)]
    ln_w, ln_b = torch.ones(D, device="cuda"), torch.zeros(D, device="cuda")
    qn = torch.ones(D, device="cuda", dtype=torch.bfloat16)
    counters = torch.zeros(N_REQ, dtype=torch.int32, device="cuda")
    ws_read = K.readout_workspace(xs[0], ws[0][0])
    outs = [torch.empty_like(x) for x in xs]

    def run():
        for i in range(LAYERS):
            K.swiglu_readout(xs[i], *ws[i], ln_w, ln_b, 1e-5, out=outs[i], workspace=ws_read,
                             x_norm=(qn, 1e-5), row_counters=counters)

    with torch.no_grad():
        run()
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            run()
        graph.replay()
        torch.cuda.synchronize()
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record()
        for _ in range(iters):
            graph.replay()
        end.record()
        torch.cuda.synchronize()
    us = start.elapsed_time(end) * 1e3 / (iters * LAYERS)
    return us, 3 * D * F * 2 * N_REQ


def bench_decode_step(model, steps: int):
    """Config 4: 32 requests on the config-2 model, each with its own fp32 fast weights
    (W_up/W_gate/W_down ~ N(0, 0.02) drawn from a generator seeded with the request id,
    S = 0), ragged prompts with lengths uniform in [64, 2048], frozen prefill into ring
    caches (window 512, bf16 K/V), then ``steps`` greedy steps of one token per request
    replayed from one HIP graph (no EOS stop).  Returns (decode tok/s, ms per step, info)."""
    import torch
    from utttcompanion_amd.decoder import BatchedDecoder
    from utttcompanion_amd.layer import FastWeightState
    N_REQ = 32
    D, F = C2["d_model"], C2["d_ff_fast"]
    ln_w = model.fast_weight_pool.ln_weight.detach().float()
    ln_b = model.fast_weight_pool.ln_bias.detach().float()
    states = []
    for rid in range(N_REQ):
        g = torch.Generator().manual_seed(rid)
        w = [torch.randn(1, D, F, generator=g) * 0.02, torch.randn(1, D, F, generator=g) * 0.02,
             torch.randn(1, F, D, generator=g) * 0.02]
        w = [t.to("cuda") for t in w]
        states.append(FastWeightState(*w, *(torch.zeros_like(t) for t in w), ln_w, ln_b))
    g = torch.Generator().manual_seed(5)
    lengths = torch.randint(64, 2049, (N_REQ,), generator=g).tolist()
    prompts = [torch.randint(0, C2["vocab_size"], (n,), generator=g) for n in lengths]
    with torch.no_grad():
        dec = BatchedDecoder(model, states)
        log("decode: frozen prefill of 32 ragged prompts")
        first = dec.prefill(prompts)
        dec.capture()
        tok = first.float().argmax(-1)
        for _ in range(3):
            dec.step(tok)
            tok = dec.next_tokens.clone()
        torch.cuda.synchronize()
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record()
        for _ in range(steps):
            dec.step(tok)
            tok = dec.next_tokens
        end.record()
        torch.cuda.synchronize()
    ms = start.elapsed_time(end) / steps
    readout_bytes = 3 * D * F * 2 * N_REQ * C2["n_layers"]  # bf16 read copies, once per step
    return N_REQ / (ms * 1e-3), ms, {"requests": N_REQ, "steps": steps, "prompt_lengths": [min(lengths), max(lengths)],
                                      "readout_bytes_per_step": readout_bytes,
                                      "readout_hbm_gbs": round(readout_bytes / (ms * 1e-3) / 1e9, 1)}


def build_c3_model():
    """The config-3 model (1.58B-label: 24 layers, d 2048, 16 x 128 heads, 4 kv heads, window
    1024, F 5504), initialised directly on the GPU, bf16 with fp32 fast-weight masters."""
    import torch
    from utttcompanion_amd import uTTTConfig, uTTTModel
    torch.manual_seed(0)
    with torch.device("cuda"):
        model = uTTTModel(uTTTConfig(**C3)).eval()
    model = model.to(torch.bfloat16)
    model.fast_weight_pool.float()
    return model


def bench_c3_prefill(model, steps: int):
    """Config 3: batch 4 x 4096 uniform token ids, full prefill with the per-chunk writes
    (64 chunks x 24 layers), launched eagerly (each chunk-layer's update moves ~2 GB of
    state, so launch overhead is hidden).  Returns (tok/s, ms per prefill)."""
    import torch
    g = torch.Generator().manual_seed(6)
    ids = torch.randint(0, C3["vocab_size"], (C3_BATCH, C3_SEQ), generator=g).to("cuda")
    state = model.init_fast_state(C3_BATCH, device="cuda", dtype=torch.float32, detach=True)
    with torch.no_grad():
        log("config 3: warm-up prefill")
        model.prefill_with_writes(ids, state)
        torch.cuda.synchronize()
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record()
        for i in range(steps):
            out = model.prefill_with_writes(ids, state)
            log(f"config 3: prefill {i + 1}/{steps} launched")
        end.record()
        torch.cuda.synchronize()
        finite = bool(torch.isfinite(out[2]).all().item())
    ms = start.elapsed_time(end) / steps
    return C3_BATCH * C3_SEQ / (ms * 1e-3), ms, finite


def bench_evolve(model, steps: int):
    """Config 5: 16 requests with [prompt + reply] lengths uniform in [128, 4096] on the
    config-3 model, each with its own fp32 state (W ~ N(0, 0.02) from a generator seeded with
    the request id, S = 0); one step = ``evolve_batched``: the ragged chunk-wise updates of all
    requests in one chunk loop (per-chunk surprise gate 0.5), the turn gate (surprise > 0.5) and
    the elastic pull (lambda 1e-3, drift ceiling 0.35) of the gated requests.  Returns
    (valid tok/s, ms per step, info)."""
    import torch
    from utttcompanion_amd.evolve import evolve_batched
    from utttcompanion_amd.layer import FastWeightState
    D, F = C3["d_model"], C3["d_ff_fast"]
    ln_w = model.fast_weight_pool.ln_weight.detach().float()
    ln_b = model.fast_weight_pool.ln_bias.detach().float()
    states = []
    for rid in range(C5_REQUESTS):
        g = torch.Generator(device="cuda").manual_seed(rid)
        w = [torch.randn(1, D, F, device="cuda", generator=g) * 0.02,
             torch.randn(1, D, F, device="cuda", generator=g) * 0.02,
             torch.randn(1, F, D, device="cuda", generator=g) * 0.02]
        states.append(FastWeightState(*w, *(torch.zeros_like(t) for t in w), ln_w, ln_b))
    g = torch.Generator().manual_seed(8)
    lengths = torch.randint(C5_LENGTHS[0], C5_LENGTHS[1] + 1, (C5_REQUESTS,), generator=g).tolist()
    turns = [torch.randint(6, C3["vocab_size"], (n,), generator=g).to("cuda") for n in lengths]
    kw = dict(surprise_threshold=0.5, anchor_lambda=1e-3, max_drift_ratio=0.35, min_chunk_surprise=0.5)
    with torch.no_grad():
        log("config 5: warm-up ragged update")
        res = evolve_batched(model, turns, states, **kw)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for i in range(steps):
            res = evolve_batched(model, turns, states, **kw)
            log(f"config 5: step {i + 1}/{steps} done")
        torch.cuda.synchronize()
        ms = (time.perf_counter() - t0) * 1e3 / steps
    tokens = sum(lengths)
    chunks = sum((n + 63) // 64 for n in lengths)
    info = {"requests": C5_REQUESTS, "lengths": [min(lengths), max(lengths)], "valid_tokens": tokens,
            "row_chunks": chunks, "turn_gate_fired": sum(int(r.gate_triggered) for r in res),
            "mean_surprise": round(sum(r.surprise for r in res) / len(res), 4),
            "min_state_bytes_per_step": 48 * D * F * chunks}  # W, S read + written once per row-chunk
    info["state_hbm_gbs"] = round(info["min_state_bytes_per_step"] / (ms * 1e-3) / 1e9, 1)
    return tokens / (ms * 1e-3), ms, info


def bench_copy_reference(iters: int = 5, nbytes: int = 1 << 30):
    """A plain device copy of known size (torch copy_), the scale for rocprofv3's
    FETCH_SIZE / WRITE_SIZE counters in the traffic figure."""
    import torch
    src = torch.empty(nbytes, dtype=torch.uint8, device="cuda").fill_(1)
    dst = torch.empty_like(src)
    for _ in range(iters):
        dst.copy_(src)
    torch.cuda.synchronize()
    return nbytes


def cpu_baseline(model, tokens: int, rows: int):
    """The CPU oracle (PyTorch-CPU fp32 restatement) on ``rows`` x ``tokens`` of config 2 with writes."""
    import torch
    from oracle import uttt_math as om
    threads = min(16, os.cpu_count() or 1)
    torch.set_num_threads(threads)
    weights = {k: v.detach().float().cpu() for k, v in model.state_dict().items()}
    ocfg = om.OracleConfig(**{k: C2[k] for k in ("d_model", "n_layers", "n_heads", "n_kv_heads", "d_ff_fast",
                                                 "sliding_window_size", "vocab_size", "chunk_size")},
                           base_inner_lr=model.config.base_inner_lr,
                           base_weight_decay=model.config.base_weight_decay)
    oracle = om.OracleModel(ocfg, weights)
    ids = torch.randint(0, C2["vocab_size"], (rows, tokens), generator=torch.Generator().manual_seed(4))
    t0 = time.perf_counter()
    oracle.forward(ids, None, None, update_fast_weights=True, logits_to_keep=-1)
    dt = time.perf_counter() - t0
    return {"value": round(rows * tokens / dt, 2), "unit": "tok/s", "cores": threads, "kind": "port",
            "sample": f"oracle.OracleModel fp32 on the host CPU: {rows} rows x {tokens} tokens "
                      f"({tokens // C2['chunk_size']} chunks) x 12 layers of config 2 with writes "
                      f"(half the config-2 batch); {dt:.1f} s"}


def main() -> int:
    args = parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only: every workload here fits one MI355X and the build has no "
              f"multi-GPU path (requested --gpus {args.gpus}); run with --gpus 1", file=sys.stderr)
        return 2
    import torch
    if not torch.cuda.is_available():
        print("bench.py needs an MI355X (no GPU visible)", file=sys.stderr)
        return 1
    sections = set(args.sections.split(","))
    if "copyref" in sections:
        log(f"copy reference: {bench_copy_reference()} bytes x 5")
    model = build_model()
    tokens = C2_BATCH * C2_SEQ
    ms, finite = float("nan"), False
    if "prefill" in sections:
        ms, finite = bench_prefill(model, args.steps, args.warmup)
        log(f"prefill {ms:.2f} ms/step -> {tokens / ms * 1e3:.0f} tok/s (finite={finite})")
    roofline = update = decode = None
    if "update" in sections:
        per, shape = bench_update_phases(args.phase_iters)
        total_ms = sum(per)
        B, C, D, F = shape["B"], shape["C"], shape["D"], shape["F"]
        dom = max(range(len(per)), key=lambda p: per[p])
        dbytes, dflops = phase_work(dom, B, C, D, F)
        d_gbs = dbytes / (per[dom] * 1e-3) / 1e9
        d_tfl = dflops / (per[dom] * 1e-3) / 1e12
        hbm_bound = dbytes > 0 and dflops / dbytes < PEAK_BF16_TFLOPS * 1e12 / (PEAK_HBM_GBS * 1e9)
        upd_roof = ({"bound": "hbm", "achieved": round(d_gbs, 1), "peak": PEAK_HBM_GBS, "unit": "GB/s",
                     "frac": round(d_gbs / PEAK_HBM_GBS, 4)} if hbm_bound else
                    {"bound": "mfma", "achieved": round(d_tfl, 2), "peak": PEAK_BF16_TFLOPS, "unit": "TFLOP/s",
                     "frac": round(d_tfl / PEAK_BF16_TFLOPS, 4)})
        upd_roof.update(kernel=PHASES[dom], traffic=measured_traffic(PHASES[dom]),
                        per_launch={"algorithmic_bytes": dbytes, "algorithmic_flops": dflops,
                                    "avg_ms": round(per[dom], 4), "shape": shape})
        roofline = upd_roof
        upd_bytes, upd_flops = 48 * D * F * B, 20 * C * D * F * B
        update = {"ms": round(total_ms, 4), "phase_ms": dict(zip(PHASES, [round(x, 4) for x in per])),
                  "hbm_frac_min_state_bytes": round(upd_bytes / (total_ms * 1e-3) / 1e9 / PEAK_HBM_GBS, 4),
                  "mfma_frac": round(upd_flops / (total_ms * 1e-3) / 1e12 / PEAK_BF16_TFLOPS, 4),
                  "roofline": upd_roof}
        log(f"update phases (ms): {update['phase_ms']}")

    if "decode" in sections:
        dec_ms, dec_bytes, dec_shape = bench_decode(20)
        dec_gbs = dec_bytes / (dec_ms * 1e-3) / 1e9
        decode = {"kernel": "k_swa_decode", "us_per_layer_step": round(dec_ms * 1e3, 2),
                  "achieved_gbs": round(dec_gbs, 1), "hbm_frac": round(dec_gbs / PEAK_HBM_GBS, 4), "shape": dec_shape}
        log(f"decode kernel {dec_ms * 1e3:.1f} us -> {dec_gbs:.0f} GB/s")
        rd_us, rd_bytes = bench_decode_readout(20)
        rd_gbs = rd_bytes / (rd_us * 1e-6) / 1e9
        decode["readout"] = {"kernel": "k_readout_gemv", "us_per_layer_step": round(rd_us, 2),
                             "algorithmic_bytes": rd_bytes, "achieved_gbs": round(rd_gbs, 1),
                             "hbm_frac": round(rd_gbs / PEAK_HBM_GBS, 4),
                             "unit_bytes": "3 D F bf16 per request (W_up, W_gate, W_down copies read once)"}
        log(f"decode readout {rd_us:.1f} us -> {rd_gbs:.0f} GB/s")
        tps, step_ms, info = bench_decode_step(model, args.decode_steps)
        decode.update(decode_tok_s=round(tps, 1), ms_per_decode_step=round(step_ms, 4), workload=info)
        log(f"decode step {step_ms:.3f} ms -> {tps:.0f} tok/s")

    cpu = None
    if not args.no_cpu_baseline and "cpu" in sections:
        log("timing the CPU oracle baseline")
        cpu = cpu_baseline(model, args.cpu_tokens, args.cpu_rows)
        log(f"cpu baseline {cpu['value']} tok/s on {cpu['cores']} threads")

    chain = None
    if "chain" in sections:
        ch_ms, stage_ms, ch_shape = bench_chain(args.phase_iters)
        Bc, Lc, Cc, Dc, Fc = ch_shape["B"], ch_shape["L"], ch_shape["C"], ch_shape["D"], ch_shape["F"]
        state_bytes = 48 * Dc * Fc * Bc  # W and S read and written once per chunk
        chain = {"ms": round(ch_ms, 4), "shape": ch_shape,
                 "stage_ms": {"layers_mean": round(sum(stage_ms[:-1]) / Lc, 4),
                              "state_write": round(stage_ms[-1], 4)},
                 "hbm_frac_min_state_bytes": round(state_bytes / (ch_ms * 1e-3) / 1e9 / PEAK_HBM_GBS, 4),
                 "mfma_frac_update_flops": round(20 * Cc * Dc * Fc * Lc * Bc / (ch_ms * 1e-3) / 1e12
                                                 / PEAK_BF16_TFLOPS, 4)}
        apply_ms = stage_ms[-1]
        a_gbs = state_bytes / (apply_ms * 1e-3) / 1e9
        roofline = {"bound": "hbm", "achieved": round(a_gbs, 1), "peak": PEAK_HBM_GBS, "unit": "GB/s",
                    "frac": round(a_gbs / PEAK_HBM_GBS, 4), "kernel": "k_chain_apply_lds",
                    "traffic": measured_traffic("k_chain_apply"),
                    "per_launch": {"algorithmic_bytes": state_bytes, "avg_ms": round(apply_ms, 4),
                                   "unit_bytes": "48 D F per row per chunk (W and S read and written once)",
                                   "shape": ch_shape}}
        log(f"layer chain {ch_ms:.3f} ms per chunk; stages (ms) {chain['stage_ms']}")

    big = {}
    if sections & {"c3", "evolve"}:
        del model
        torch.cuda.empty_cache()
        log("building the config-3 model on the GPU")
        model3 = build_c3_model()
        if "c3" in sections:
            tps, c3_ms, fin = bench_c3_prefill(model3, args.c3_steps)
            big["config3_prefill"] = {"tok_s": round(tps, 1), "ms_per_prefill": round(c3_ms, 2), "finite": fin,
                                      "batch": C3_BATCH, "seq_len": C3_SEQ, "layers": C3["n_layers"],
                                      "d_model": C3["d_model"], "d_ff_fast": C3["d_ff_fast"]}
            log(f"config 3 prefill {c3_ms:.1f} ms -> {tps:.0f} tok/s")
        if "evolve" in sections:
            tps, ev_ms, info = bench_evolve(model3, args.c3_steps)
            big["config5_evolve"] = {"tok_s": round(tps, 1), "ms_per_step": round(ev_ms, 2), **info}
            log(f"config 5 ragged update {ev_ms:.1f} ms -> {tps:.0f} tok/s")
        del model3
        torch.cuda.empty_cache()

    line = {"metric": METRIC, "value": round(tokens / ms * 1e3, 1), "unit": "tok/s", "n_gpus": 1,
            "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms, 3), "higher_is_better": True,
            "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
            "data": "synthetic: uniform token ids, random-init weights (reference init), fp32 fast-weight masters",
            "config": {"workload": "config2_prefill_with_fast_weight_writes", "global_batch": C2_BATCH,
                       "seq_len": C2_SEQ, "layers": C2["n_layers"], "d_model": C2["d_model"],
                       "d_ff_fast": C2["d_ff_fast"], "window": C2["sliding_window_size"], "chunk": C2["chunk_size"],
                       "parallelism": "none (1 GPU)", "hip_graph": True, "finite": finite},
            "roofline": roofline, "update": update, "chain": chain, "decode": decode, **big, "cpu_baseline": cpu}
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
