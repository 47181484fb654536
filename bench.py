#!/usr/bin/env python3
"""Benchmark of the uTTT hot path on one MI355X; prints one JSON line on stdout.

Headline workload (the largest single-GPU configuration): the
1.58B-label uTTT model (24 layers, d_model 2048, 16 x 128 heads, 4 kv heads, window 1024, shared
SwiGLU fast weights F = 5504, chunk 64, vocab 32000), bf16 activations with fp32 fast-weight
masters, random-init weights (reference initialisation), token ids uniform over the vocabulary,
batch 4 x 4096.  One step = one full prefill with the per-chunk fast-weight writes of every layer
(64 chunks x 24 chained layer updates, the chunk-first schedule).  ``value`` = tokens / s over
the timed steps, inputs resident in HBM.

Per chunk the prefill runs every layer's attention, projections and readout on one stream and
the layer chain (``uttt_chunk_chain`` stages) that applies the chunk's chained fast-weight
updates on a second stream, one layer behind.

Also reported:
* ``roofline``: the whole config-3 prefill's algorithmic flops over its timed duration against
  the bf16 MFMA peak (the north star's axis for the update + prefill), its state-byte fractions
  of the HBM peak, and the HBM traffic per prefill rocprofv3 measured when a summary is committed
  under profiles/; beside it, ``dominant_kernel``: the chain kernel with the largest total time in
  a calibration prefill (every chain launch bracketed by HIP events on the chain's stream),
  against its algorithmic bytes per launch (it streams bf16 copies of the state: HBM-bound), in
  the prefill and timed alone;
* ``prefill``: the whole prefill's algorithmic work against the bf16 MFMA peak and its minimum
  state bytes against the HBM peak, and the timed chain kernels;
* ``config1_block``: BASELINE config 1 (one fp32 uTTT block, B 1 x T 1024, 16 chunk updates)
  against the fp32 MFMA peak;
* ``config2_prefill``: the 151M-label model's prefill with writes (8 x 2048), one HIP graph;
* ``update``, ``chain``: the single-chunk update and one chunk's layer chain at the config-2 shape;
* ``decode``: config 4 (32 requests of the config-2 model, ring-buffer SWA decode, one HIP graph
  per step) and its attention and readout kernels against HBM;
* ``config5_evolve``: the ragged per-request updates of 16 requests on the config-3 model;
* ``cpu_baseline`` (config 3) and ``cpu_baselines`` (configs 1 and 4): the CPU oracle (the tests'
  restatement) on bounded samples of the same workloads, on the cores this process may use.
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
PEAK_FP32_TFLOPS = 157.3
C1 = dict(d_model=512, n_heads=8, n_kv_heads=4, window=256, d_ff=1024, chunk=64, seq=1024, inner_lr=0.01,
          weight_decay=0.005)

C2 = dict(vocab_size=32000, d_model=768, n_layers=12, n_heads=12, n_kv_heads=4, d_ff_fast=2048,
          sliding_window_size=512, chunk_size=64, max_seq_len=4096)
C2_BATCH, C2_SEQ = 8, 2048
C3 = dict(vocab_size=32000, d_model=2048, n_layers=24, n_heads=16, n_kv_heads=4, d_ff_fast=5504,
          sliding_window_size=1024, chunk_size=64, max_seq_len=4096)
C3_BATCH, C3_SEQ = 4, 4096
C5_REQUESTS, C5_LENGTHS = 16, (128, 4096)
PHASES = ("k_up_gate", "k_down_partial", "k_ln_grad+k_ln_readout", "k_backward", "k_apply")


def measured_traffic(kernel: str, config: str = "c2"):
    """HBM bytes per launch of ``kernel`` at a config's shape, from the committed rocprofv3
    FETCH_SIZE / WRITE_SIZE summary (scaled by a copy kernel of known size), or None when no
    summary for that kernel is present.  Looks for a ``traffic_bytes_per_launch <kernel>:`` line
    in ``profiles/prefill_<config>_traffic.md`` (the state write's launch of ``k_chain_apply_lds``
    runs ``k_chain_apply_wide`` at config 3), then a ``traffic_bytes_per_launch:`` line in
    ``profiles/<kernel>_<config>_traffic.md``."""
    here = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles")
    names = [kernel] + (["k_chain_apply_wide"] if kernel == "k_chain_apply_lds" else [])
    candidates = [(os.path.join(here, f"prefill_{config}_traffic.md"), f"traffic_bytes_per_launch {n}:") for n in names]
    candidates.append((os.path.join(here, f"{kernel}_{config}_traffic.md"), "traffic_bytes_per_launch:"))
    for path, prefix in candidates:
        try:
            with open(path) as fh:
                for line in fh:
                    if line.startswith(prefix):
                        return int(line.split(":", 1)[1].strip())
        except OSError:
            continue
    return None


def measured_prefill_traffic(config: str = "c3"):
    """HBM bytes per prefill from the committed rocprofv3 summary
    ``profiles/prefill_<config>_traffic.md`` (its ``traffic_bytes_per_prefill:`` line), or None."""
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles", f"prefill_{config}_traffic.md")
    try:
        with open(path) as fh:
            for line in fh:
                if line.startswith("traffic_bytes_per_prefill:"):
                    return int(line.split(":", 1)[1].strip())
    except OSError:
        pass
    return None


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def parse_args():
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=3, help="timed config-3 prefills (the headline)")
    ap.add_argument("--warmup", type=int, default=1)
    ap.add_argument("--phase-iters", type=int, default=20)
    ap.add_argument("--no-cpu-baseline", action="store_true", help="skip the CPU oracle timings")
    ap.add_argument("--sections", default="c3,c1,prefill,update,chain,decode,evolve,cpu",
                    help="comma list of c3 (the headline), c1, prefill (config 2), update, chain, decode, "
                         "evolve, cpu, copyref, c3kern, c3once (profiling runs pick a subset)")
    ap.add_argument("--c2-steps", type=int, default=5, help="timed config-2 prefills")
    ap.add_argument("--evolve-steps", type=int, default=2, help="timed config-5 updates")
    ap.add_argument("--cpu-tokens", type=int, default=256, help="tokens of the config-3 CPU baseline sample")
    ap.add_argument("--cpu-decode-steps", type=int, default=4, help="decode steps per request, config-4 CPU sample")
    ap.add_argument("--decode-steps", type=int, default=256)
    ap.add_argument("--kernel", default="k_chain_back_lds", help="chain kernel timed by the c3kern section")
    return ap.parse_args()


def build_model():
    import torch
    from utttcompanion_amd import uTTTConfig, uTTTModel
    torch.manual_seed(0)
    model = uTTTModel(uTTTConfig(**C2)).eval()
    model = model.to("cuda").to(torch.bfloat16)
    model.fast_weight_pool.float()
    return model


def bench_c2_prefill(model, steps: int, warmup: int):
    """Config 2: batch 8 x 2048, full prefill with writes, recorded once into a HIP graph and
    replayed.  Returns (ms per prefill, finite)."""
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


# per-launch algorithmic bytes of the chain kernels that stream the state (bf16 copies), in units of
# D F B bytes: the S_up / S_gate products, the W_down / S_down reads of the down and back passes,
# and the state write (W and S read and written once per row-chunk, fp32)
CHAIN_STATE_BYTES = {"k_chain_keys_lds": 4, "k_chain_pq_lds": 4, "k_chain_down_lds": 4, "k_chain_back_lds": 4,
                     "k_chain_apply_lds": 48}
CHAIN_STATE_WHAT = {
    "k_chain_keys_lds": "4 D F per row (bf16 S_up and S_gate copies read once, with the key Gram row in the same "
                        "launch; the W products come from the readouts)",
    "k_chain_pq_lds": "4 D F per row (bf16 S_up and S_gate copies read once; the W products come from the readouts)",
    "k_chain_down_lds": "4 D F per row (bf16 W_down and S_down copies read once)",
    "k_chain_back_lds": "4 D F per row (bf16 W_down and S_down copies read once)",
    "k_chain_apply_lds": "48 D F per row (fp32 W and S read and written once)",
}
CHAIN_KERNELS = ("k_chain_keys_lds", "k_chain_pq_lds", "k_chain_gram_lds", "k_chain_up_lds", "k_chain_down_lds",
                 "k_ln_grad",
                 "k_chain_back_lds", "k_chain_coef", "k_chain_apply_lds", "k_chain_init")


def prefill_flops(cfg: dict, batch: int, seq: int) -> dict:
    """Algorithmic flops of one prefill with writes: the update + readout
    (20 D F per token and layer), the window attention (4 hd H per visible query-key pair) and
    the slow projections (2 [D (2 D + 2 Hkv hd) + 4 D^2 + 2 D] per token and layer)."""
    D, F, L, H, Hkv = cfg["d_model"], cfg["d_ff_fast"], cfg["n_layers"], cfg["n_heads"], cfg["n_kv_heads"]
    hd, W = D // H, cfg["sliding_window_size"]
    pairs = W * (W + 1) // 2 + (seq - W) * W if seq >= W else seq * (seq + 1) // 2
    upd = 20 * D * F * seq * L * batch
    swa = 4 * hd * H * pairs * L * batch
    proj = 2 * (D * (2 * D + 2 * Hkv * hd) + 4 * D * D + 2 * D) * seq * L * batch
    return {"update_readout": upd, "swa": swa, "projections": proj, "total": upd + swa + proj}


def prefill_bytes(cfg: dict, batch: int, seq: int) -> dict:
    """HBM bytes of one prefill with writes: the minimum (the fp32 state read and written once per
    row-chunk, 48 D F) and this design's streamed floor: per row, layer and chunk the
    bf16 copies of W_up, W_gate, W_down (readout), S_up, S_gate (products), W_down and S_down twice
    (down and back passes), 18 D F; per row and chunk the state write, 60 D F (48 + bf16 copies)."""
    D, F, L, C = cfg["d_model"], cfg["d_ff_fast"], cfg["n_layers"], cfg["chunk_size"]
    chunks = (seq + C - 1) // C
    return {"min_state": 48 * D * F * batch * chunks, "design": (18 * L + 60) * D * F * batch * chunks}


def bench_c3_prefill(model, steps: int, warmup: int):
    """Config 3: batch 4 x 4096 uniform token ids, full prefill with the per-chunk writes
    (64 chunks x 24 layers), launched eagerly (launch overhead is hidden behind the GPU), timed
    without instrumentation.  Then one calibration prefill brackets every chain kernel launch with
    HIP events (``KernelTimer``; the chain's stages then go out launch by launch, so it runs
    slower): the streaming kernel with the largest total there is the dominant one.  Returns
    (tok/s, ms per prefill, finite, dominant kernel, calibration table, ms of the calibration)."""
    import torch
    from utttcompanion_amd.kernels import KernelTimer
    g = torch.Generator().manual_seed(6)
    ids = torch.randint(0, C3["vocab_size"], (C3_BATCH, C3_SEQ), generator=g).to("cuda")
    state = model.init_fast_state(C3_BATCH, device="cuda", dtype=torch.float32, detach=True)
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    with torch.no_grad():
        for i in range(max(warmup, 1)):
            log(f"config 3: warm-up prefill {i + 1}")
            model.prefill_with_writes(ids, state)
        torch.cuda.synchronize()
        start.record()
        for i in range(steps):
            out = model.prefill_with_writes(ids, state)
            log(f"config 3: timed prefill {i + 1}/{steps} launched")
        end.record()
        torch.cuda.synchronize()
        ms = start.elapsed_time(end) / steps
        finite = bool(torch.isfinite(out[0]).all().item()) and bool(torch.isfinite(out[2]).all().item())
        calib = KernelTimer(CHAIN_KERNELS)
        start.record()
        model.prefill_with_writes(ids, state, kernel_timer=calib)
        end.record()
        torch.cuda.synchronize()
    table = calib.summary()
    streamed = [k for k in table if k in CHAIN_STATE_BYTES]
    dom = max(streamed, key=lambda k: table[k]["launches"] * table[k]["mean_ms"])
    log(f"config 3: calibration prefill {start.elapsed_time(end):.1f} ms; dominant streaming chain kernel {dom}")
    return C3_BATCH * C3_SEQ / (ms * 1e-3), ms, finite, dom, table, start.elapsed_time(end)


def bench_chain_kernel(kernel: str, replays: int = 5, B: int = None, L: int = None, D: int = None, F: int = None):
    """One chain kernel in isolation at the config-3 chunk shape (4 rows, 24 layers, C 64, D 2048,
    F 5504, bf16 activations and state copies, W products given as in the prefill): a chain is run
    stage by stage on random layer inputs (so the workspace holds every layer's activations), then
    the kernel's launches for all layers (or the state write's one launch) are captured in a HIP
    graph and the graph is replayed; HIP events bracket the replays on the capture stream.  Returns
    (mean us per launch, launches per replay)."""
    import torch
    from utttcompanion_amd import kernels as K
    B, L = B or C3_BATCH, L or C3["n_layers"]
    D, F = D or C3["d_model"], F or C3["d_ff_fast"]
    C = 64
    g = torch.Generator(device="cuda").manual_seed(10)
    act = lambda *s: torch.randn(*s, device="cuda", generator=g).to(torch.bfloat16)
    state = [torch.randn(B, D, F, device="cuda", generator=g) * 0.02, torch.randn(B, D, F, device="cuda", generator=g) * 0.02,
             torch.randn(B, F, D, device="cuda", generator=g) * 0.02]
    state += [torch.zeros_like(t) for t in state]
    copies = [t.to(torch.bfloat16) for t in state]
    ln_w, ln_b = torch.ones(D, device="cuda"), torch.zeros(D, device="cuda")
    stream = torch.cuda.Stream()
    with torch.no_grad(), torch.cuda.stream(stream):
        run = K.ChunkChainRun(L, C, state, ln_w, ln_b, None, 0.9, 1.0, True, 1e-5, torch.bfloat16, copies=copies,
                              w_products_given=True)
        for l in range(L):
            up, gate = run.w_product_outputs(l)
            up.copy_(act(B, 64, F))
            gate.copy_(act(B, 64, F))
            run.set_layer(act(B, C, D), act(B, C, D), torch.full((B, C), 0.005, device="cuda").to(torch.bfloat16),
                          torch.full((B, C), 0.001, device="cuda").to(torch.bfloat16))
            run.launch(l)
        run.launch(L)
        stages = [L] if kernel == "k_chain_apply_lds" else list(range(L))
        idx = [run.stage_launches(st).index(kernel) for st in stages]

        def once():
            for st, i in zip(stages, idx):
                _enqueue_chain_launch(run, st, i)
        once()
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=stream):
            once()
        graph.replay()
        torch.cuda.synchronize()
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record(stream)
        for _ in range(replays):
            graph.replay()
        end.record(stream)
        torch.cuda.synchronize()
    return start.elapsed_time(end) * 1e3 / (replays * len(stages)), len(stages)


def _enqueue_chain_launch(run, stage: int, launch: int) -> None:
    """Enqueue launch ``launch`` of ``stage`` of a chain run on the current stream."""
    import ctypes as C
    import torch
    from utttcompanion_amd import _native as N
    lib = N.load_library()
    N.check(lib.uttt_chunk_chain_stage_launch(C.byref(run.args), run.workspace.data_ptr(), run.workspace.numel(),
                                              stage, 0, launch, launch + 1, None, 0, None,
                                              torch.cuda.current_stream().cuda_stream), "uttt_chunk_chain_stage_launch")


def chain_kernel_table(summary: dict, steps: int, B: int, D: int, F: int) -> dict:
    """Per followed chain kernel: launches per prefill, mean us, total ms per prefill and, for the
    kernels that stream the state, algorithmic bytes per launch and GB/s."""
    out = {}
    for name, t in sorted(summary.items(), key=lambda kv: -kv[1]["launches"] * kv[1]["mean_ms"]):
        row = {"launches_per_prefill": t["launches"] // steps, "mean_us": round(t["mean_ms"] * 1e3, 2),
               "ms_per_prefill": round(t["launches"] * t["mean_ms"] / steps, 2)}
        if name in CHAIN_STATE_BYTES:
            nbytes = CHAIN_STATE_BYTES[name] * D * F * B
            row["algorithmic_bytes"] = nbytes
            row["gbs"] = round(nbytes / (t["mean_ms"] * 1e-3) / 1e9, 1)
        out[name] = row
    return out


def bench_c1_block(iters: int):
    """Config 1: one uTTT block in fp32 (d_model 512, 8 x 64 heads, 4 kv heads, window 256,
    F 1024, chunk 64, inner lr 0.01, weight decay 0.005, random weights N(0, 0.02) as the
    reference initialises them, eta/alpha routers at their reference init), input (1, 1024, 512)
    ~ N(0, 1): the block forward with 16 chunk updates (the persistent resident update).  Timed
    eagerly (back-to-back forwards) and as replays of one captured HIP graph of the forward (no
    per-kernel launch cost).  Returns (tok/s, ms per forward, finite, graph ms per forward,
    graph replays equal to eager)."""
    import torch
    from utttcompanion_amd import SharedFastWeightPool, uTTTBlock
    from utttcompanion_amd import kernels as K
    torch.manual_seed(0)
    c = C1
    block = uTTTBlock(0, c["d_model"], c["n_heads"], c["n_kv_heads"], window_size=c["window"], chunk_size=c["chunk"],
                      base_inner_lr=c["inner_lr"], base_weight_decay=c["weight_decay"], max_seq_len=2048).eval()
    with torch.no_grad():
        for name, p in block.named_parameters():
            if p.dim() == 2 and "w_eta" not in name and "w_alpha" not in name:
                p.normal_(0, 0.02)
    pool = SharedFastWeightPool(c["d_model"], c["d_ff"], normalize_loss_by_dim=True)
    with torch.no_grad():
        for p in (pool.w_up_init, pool.w_gate_init, pool.w_down_init):
            p.normal_(0, 0.02)
    block, pool = block.to("cuda"), pool.to("cuda")
    x = torch.randn(1, c["seq"], c["d_model"], generator=torch.Generator().manual_seed(1)).to("cuda")
    state = pool.init_state(1, device="cuda", dtype=torch.float32, detach=True)
    with torch.no_grad():
        for _ in range(3):
            out = block(x, pool, state)
        torch.cuda.synchronize()
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record()
        for _ in range(iters):
            out = block(x, pool, state)
        end.record()
        torch.cuda.synchronize()
        ms = start.elapsed_time(end) / iters
        eager = out[0].clone()
        graph = torch.cuda.CUDAGraph()
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            block(x, pool, state)  # allocations of the capture's shapes are made once, outside it
        torch.cuda.current_stream().wait_stream(side)
        with torch.cuda.graph(graph):
            gout = block(x, pool, state)
        graph.replay()
        torch.cuda.synchronize()
        same = bool(torch.equal(gout[0], eager))
        start.record()
        for _ in range(iters):
            graph.replay()
        end.record()
        torch.cuda.synchronize()
        gms = start.elapsed_time(end) / iters
        same = same and bool(torch.equal(gout[0], eager))
        K.check_resident_flags(wait=True)
    return c["seq"] / (ms * 1e-3), ms, bool(torch.isfinite(out[0]).all().item()), gms, same


def c1_flops() -> int:
    """Algorithmic flops of the config-1 block forward: update + readout, window attention and
    the slow projections; 15.0 GFLOP."""
    c = C1
    cfg = dict(d_model=c["d_model"], d_ff_fast=c["d_ff"], n_layers=1, n_heads=c["n_heads"],
               n_kv_heads=c["n_kv_heads"], sliding_window_size=c["window"])
    return prefill_flops(cfg, 1, c["seq"])["total"]


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
    # the design's streamed bytes per row-chunk, as for config 3: every layer's bf16 state copies
    # (18 D F) and the state write (60 D F)
    info["design_bytes_per_step"] = (18 * C3["n_layers"] + 60) * D * F * chunks
    info["design_hbm_frac"] = round(info["design_bytes_per_step"] / (ms * 1e-3) / 1e9 / PEAK_HBM_GBS, 4)
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


def cpu_threads() -> int:
    """The cores this process may run on (its CPU affinity), all used by the CPU baselines."""
    try:
        return len(os.sched_getaffinity(0))
    except AttributeError:
        return os.cpu_count() or 1


def _oracle_for(model, cfg: dict):
    from oracle import uttt_math as om
    weights = {k: v.detach().float().cpu() for k, v in model.state_dict().items()}
    ocfg = om.OracleConfig(**{k: cfg[k] for k in ("d_model", "n_layers", "n_heads", "n_kv_heads", "d_ff_fast",
                                                  "sliding_window_size", "vocab_size", "chunk_size")},
                           base_inner_lr=model.config.base_inner_lr, base_weight_decay=model.config.base_weight_decay)
    return om.OracleModel(ocfg, weights)


def cpu_baseline_c3(model, tokens: int) -> dict:
    """The CPU oracle (PyTorch-CPU fp32 restatement) on one row x ``tokens`` of config 3 with
    writes, all 24 layers; tok/s scales per token to the full workload (every chunk does the
    same work per token)."""
    import torch
    threads = cpu_threads()
    torch.set_num_threads(threads)
    oracle = _oracle_for(model, C3)
    ids = torch.randint(0, C3["vocab_size"], (1, tokens), generator=torch.Generator().manual_seed(4))
    t0 = time.perf_counter()
    oracle.forward(ids, None, None, update_fast_weights=True, logits_to_keep=-1)
    dt = time.perf_counter() - t0
    return {"value": round(tokens / dt, 2), "unit": "tok/s", "cores": threads, "host_cpus": os.cpu_count(),
            "kind": "port",
            "sample": f"oracle.OracleModel fp32 on the host CPU: 1 row x {tokens} tokens ({tokens // 64} chunks) "
                      f"x 24 layers of config 3 with writes; {dt:.1f} s (the full workload is 4 rows x 4096 tokens, "
                      f"the same work per token)"}


def cpu_baseline_c1() -> dict:
    """The CPU oracle's config-1 block (fp32, 1 x 1024 tokens, 16 chunk updates), timed in full."""
    import torch
    from oracle import uttt_math as om
    threads = cpu_threads()
    torch.set_num_threads(threads)
    c = C1
    g = torch.Generator().manual_seed(2)
    D, F = c["d_model"], c["d_ff"]
    hkv, hd = c["n_kv_heads"], D // c["n_heads"]
    lw = {"attn_norm.weight": torch.ones(D), "uttt_norm.weight": torch.ones(D),
          "attn.wq.weight": 0.02 * torch.randn(D, D, generator=g), "attn.wk.weight": 0.02 * torch.randn(hkv * hd, D, generator=g),
          "attn.wv.weight": 0.02 * torch.randn(hkv * hd, D, generator=g), "attn.wo.weight": 0.02 * torch.randn(D, D, generator=g),
          "uttt.w_q.weight": 0.02 * torch.randn(D, D, generator=g), "uttt.w_k.weight": 0.02 * torch.randn(D, D, generator=g),
          "uttt.w_v.weight": 0.02 * torch.randn(D, D, generator=g), "uttt.w_o.weight": 0.02 * torch.randn(D, D, generator=g),
          "uttt.w_eta.weight": torch.zeros(1, D), "uttt.w_eta.bias": torch.zeros(1),
          "uttt.w_alpha.weight": torch.zeros(1, D), "uttt.w_alpha.bias": torch.full((1,), -1.386),
          "uttt.q_norm.weight": torch.ones(D), "uttt.k_norm.weight": torch.ones(D)}
    pool = {"w_up_init": 0.02 * torch.randn(D, F, generator=g), "w_gate_init": 0.02 * torch.randn(D, F, generator=g),
            "w_down_init": 0.02 * torch.randn(F, D, generator=g), "ln_weight": torch.ones(D), "ln_bias": torch.zeros(D)}
    cfg = om.OracleConfig(d_model=D, n_layers=1, n_heads=c["n_heads"], n_kv_heads=hkv, d_ff_fast=F,
                          sliding_window_size=c["window"], chunk_size=c["chunk"], base_inner_lr=c["inner_lr"],
                          base_weight_decay=c["weight_decay"])
    cos, sin = om.rope_tables(hd, 2048)
    x = torch.randn(1, c["seq"], D, generator=g)
    om.block_forward(x[:, :128], lw, cfg, cos, sin, om.init_state(pool, 1))  # warm the CPU kernels
    t0 = time.perf_counter()
    om.block_forward(x, lw, cfg, cos, sin, om.init_state(pool, 1))
    dt = time.perf_counter() - t0
    return {"value": round(c["seq"] / dt, 2), "unit": "tok/s", "cores": threads, "kind": "port",
            "sample": f"oracle.block_forward fp32 on the host CPU: the whole config-1 block (1 x 1024 tokens, "
                      f"16 chunk updates); {dt:.2f} s"}


def cpu_baseline_c4(model, steps: int) -> dict:
    """Config 4 on the CPU oracle: for each of the 32 requests (its own fp32 fast weights drawn as
    the GPU decode draws them), batch-1 frozen decode steps after a 64-token prompt; only the steps
    are timed.  Reports aggregate tok/s and the per-token latency."""
    import torch
    from oracle import uttt_math as om
    threads = cpu_threads()
    torch.set_num_threads(threads)
    oracle = _oracle_for(model, C2)
    D, F = C2["d_model"], C2["d_ff_fast"]
    ln = (oracle.pool["ln_weight"], oracle.pool["ln_bias"])
    total, tokens = 0.0, 0
    for rid in range(32):
        g = torch.Generator().manual_seed(rid)
        w = [torch.randn(1, D, F, generator=g) * 0.02, torch.randn(1, D, F, generator=g) * 0.02,
             torch.randn(1, F, D, generator=g) * 0.02]
        st = om.OracleState(*w, *(torch.zeros_like(t) for t in w), *ln)
        ids = torch.randint(6, C2["vocab_size"], (1, 64), generator=g)
        logits, _, _, caches = oracle.forward(ids, st, None, None, 0, False, 1)
        tok = int(logits[0, -1].argmax())
        t0 = time.perf_counter()
        for i in range(steps):
            logits, _, _, caches = oracle.forward(torch.tensor([[tok]]), st, None, caches, 64 + i, False, 0)
            tok = int(logits[0, -1].argmax())
        total += time.perf_counter() - t0
        tokens += steps
    return {"value": round(tokens / total, 2), "unit": "tok/s", "cores": threads, "kind": "port",
            "ms_per_token": round(total / tokens * 1e3, 2),
            "sample": f"oracle.OracleModel fp32 on the host CPU: 32 requests x {steps} batch-1 frozen decode steps "
                      f"of the config-2 model after 64-token prompts (steps timed, prompts not); {total:.1f} s"}


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
    run_cpu = "cpu" in sections and not args.no_cpu_baseline
    if "copyref" in sections:
        log(f"copy reference: {bench_copy_reference()} bytes x 5")

    # ---------------- headline: config 3 prefill with writes
    line_value, c3_ms, finite, roofline, prefill, cpu, big = float("nan"), float("nan"), False, None, None, None, {}
    if sections & {"c3", "c3kern", "c3once", "evolve"}:
        log("building the config-3 model on the GPU")
        model3 = build_c3_model()
        if "c3once" in sections:  # profiling runs: prefills only (no calibration, no isolated kernel)
            g = torch.Generator().manual_seed(6)
            ids = torch.randint(0, C3["vocab_size"], (C3_BATCH, C3_SEQ), generator=g).to("cuda")
            state = model3.init_fast_state(C3_BATCH, device="cuda", dtype=torch.float32, detach=True)
            with torch.no_grad():
                for i in range(args.steps):
                    model3.prefill_with_writes(ids, state)
                    torch.cuda.synchronize()
                    log(f"config 3: prefill {i + 1}/{args.steps} done")
        if "c3kern" in sections:  # profiling runs: the isolated kernel timing alone
            us, per_replay = bench_chain_kernel(args.kernel)
            log(f"{args.kernel} at the config-3 chunk shape: {us:.2f} us per launch ({per_replay} per replay)")
        if "c3" in sections:
            line_value, c3_ms, finite, dom, calib, calib_ms = bench_c3_prefill(model3, args.steps, args.warmup)
            log(f"config 3 prefill {c3_ms:.1f} ms -> {line_value:.0f} tok/s")
            D, F = C3["d_model"], C3["d_ff_fast"]
            table = chain_kernel_table(calib, 1, C3_BATCH, D, F)
            us, per_replay = bench_chain_kernel(dom)
            flops = prefill_flops(C3, C3_BATCH, C3_SEQ)
            nbytes = prefill_bytes(C3, C3_BATCH, C3_SEQ)
            sec = c3_ms * 1e-3
            prefill = {"ms": round(c3_ms, 2), "calibration_prefill_ms": round(calib_ms, 2),
                       "algorithmic_tflop": round(flops["total"] / 1e12, 2),
                       "tflop_parts": {k: round(v / 1e12, 3) for k, v in flops.items() if k != "total"},
                       "mfma_frac": round(flops["total"] / sec / 1e12 / PEAK_BF16_TFLOPS, 4),
                       "hbm_frac_min_state_bytes": round(nbytes["min_state"] / sec / 1e9 / PEAK_HBM_GBS, 4),
                       "hbm_frac_design_bytes": round(nbytes["design"] / sec / 1e9 / PEAK_HBM_GBS, 4),
                       "bytes": nbytes,
                       "chain_kernels_calibration": table,
                       "chain_kernels_note": "one calibration prefill with every chain launch bracketed by events "
                                             "(stages enqueued launch by launch, so slower than the timed prefills)"}
            nbytes_dom = CHAIN_STATE_BYTES[dom] * D * F * C3_BATCH
            gbs = nbytes_dom / (us * 1e-6) / 1e9
            in_us = table[dom]["mean_us"]
            in_gbs = nbytes_dom / (in_us * 1e-6) / 1e9
            tfs = flops["total"] / sec / 1e12
            prefill_traffic = measured_prefill_traffic("c3")
            # the headline's roofline is the whole prefill's: its algorithmic flops against the
            # bf16 MFMA peak (the north star's axis; the state-byte fractions beside it); the
            # dominant streaming kernel is reported separately, in the prefill and alone
            roofline = {"bound": "mfma", "achieved": round(tfs, 2), "peak": PEAK_BF16_TFLOPS, "unit": "TFLOP/s",
                        "frac": round(tfs / PEAK_BF16_TFLOPS, 4), "traffic": prefill_traffic,
                        "scope": "one whole config-3 prefill with writes: algorithmic flops (update + readout "
                                 "20 D F per token and layer, window attention, slow projections) over the timed "
                                 "prefill's time; traffic = HBM bytes per prefill (rocprofv3 FETCH_SIZE + WRITE_SIZE "
                                 "over the library's kernels of one prefill) or null",
                        "hbm_frac_min_state_bytes": prefill["hbm_frac_min_state_bytes"],
                        "hbm_frac_design_bytes": prefill["hbm_frac_design_bytes"],
                        "hbm_frac_measured_traffic": (round(prefill_traffic / sec / 1e9 / PEAK_HBM_GBS, 4)
                                                      if prefill_traffic else None),
                        "dominant_kernel": {
                            "kernel": dom, "unit_bytes": CHAIN_STATE_WHAT[dom], "algorithmic_bytes": nbytes_dom,
                            "shape": {"B": C3_BATCH, "D": D, "F": F, "L": C3["n_layers"]},
                            "in_prefill": {"avg_us": in_us, "gbs": round(in_gbs, 1),
                                           "hbm_frac": round(in_gbs / PEAK_HBM_GBS, 4),
                                           "timing": "calibration prefill, HIP events around each launch"},
                            "isolated": {"avg_us": round(us, 2), "gbs": round(gbs, 1),
                                         "hbm_frac": round(gbs / PEAK_HBM_GBS, 4),
                                         "timing": f"{per_replay} launches (one per layer) at the config-3 chunk "
                                                   f"shape in a HIP graph, replayed 5 times, HIP events around the "
                                                   f"replays"},
                            "traffic": measured_traffic(dom, "c3")}}
            log(f"config 3: {tfs:.1f} TFLOP/s of algorithmic work ({tfs / PEAK_BF16_TFLOPS:.3f} of bf16 peak); "
                f"dominant streaming chain kernel {dom}: {in_us:.1f} us in the prefill, {us:.1f} us alone -> "
                f"{gbs:.0f} GB/s")
            if run_cpu:
                log("timing the CPU oracle on a config-3 sample")
                cpu = cpu_baseline_c3(model3, args.cpu_tokens)
                log(f"cpu baseline {cpu['value']} tok/s on {cpu['cores']} threads")
        if "evolve" in sections:
            tps, ev_ms, info = bench_evolve(model3, args.evolve_steps)
            big["config5_evolve"] = {"tok_s": round(tps, 1), "ms_per_step": round(ev_ms, 2), **info}
            log(f"config 5 ragged update {ev_ms:.1f} ms -> {tps:.0f} tok/s")
        del model3
        torch.cuda.empty_cache()

    cpu_more = {}
    if "c1" in sections:
        tps, c1_ms, c1_fin, c1_gms, c1_same = bench_c1_block(20)
        fl = c1_flops()
        tfl = fl / (c1_ms * 1e-3) / 1e12
        gtfl = fl / (c1_gms * 1e-3) / 1e12
        big["config1_block"] = {"tok_s": round(tps, 1), "ms_per_forward": round(c1_ms, 4), "finite": c1_fin,
                                "graph_tok_s": round(C1["seq"] / (c1_gms * 1e-3), 1),
                                "graph_ms_per_forward": round(c1_gms, 4), "graph_equals_eager": c1_same,
                                "algorithmic_gflop": round(fl / 1e9, 2), "achieved_tflops": round(tfl, 2),
                                "fp32_mfma_frac": round(tfl / PEAK_FP32_TFLOPS, 4),
                                "graph_fp32_mfma_frac": round(gtfl / PEAK_FP32_TFLOPS, 4),
                                "shape": "B1 T1024 D512 8x64 heads (4 kv) W256 F1024 C64, fp32, 16 chunk updates"}
        log(f"config 1 block {c1_ms:.3f} ms eager, {c1_gms:.3f} ms graph -> {tps:.0f} / "
            f"{C1['seq'] / (c1_gms * 1e-3):.0f} tok/s ({tfl:.1f} / {gtfl:.1f} TFLOP/s fp32)")
        if run_cpu:
            cpu_more["config1"] = cpu_baseline_c1()
            log(f"cpu config 1: {cpu_more['config1']['value']} tok/s")

    model = None
    if sections & {"prefill", "decode"} or (run_cpu and "decode" in sections):
        model = build_model()
    if "prefill" in sections:
        ms, fin = bench_c2_prefill(model, args.c2_steps, 2)
        tokens = C2_BATCH * C2_SEQ
        flops = prefill_flops(C2, C2_BATCH, C2_SEQ)
        big["config2_prefill"] = {"tok_s": round(tokens / ms * 1e3, 1), "ms_per_prefill": round(ms, 3), "finite": fin,
                                  "hip_graph": True,
                                  "mfma_frac": round(flops["total"] / (ms * 1e-3) / 1e12 / PEAK_BF16_TFLOPS, 4)}
        log(f"config 2 prefill {ms:.2f} ms -> {tokens / ms * 1e3:.0f} tok/s")

    update = chain = decode = None
    if "update" in sections:
        per, shape = bench_update_phases(args.phase_iters)
        total_ms = sum(per)
        B, C, D, F = shape["B"], shape["C"], shape["D"], shape["F"]
        dom = max(range(len(per)), key=lambda p: per[p])
        dbytes, dflops = phase_work(dom, B, C, D, F)
        d_gbs = dbytes / (per[dom] * 1e-3) / 1e9
        upd_bytes, upd_flops = 48 * D * F * B, 20 * C * D * F * B
        update = {"ms": round(total_ms, 4), "phase_ms": dict(zip(PHASES, [round(x, 4) for x in per])), "shape": shape,
                  "hbm_frac_min_state_bytes": round(upd_bytes / (total_ms * 1e-3) / 1e9 / PEAK_HBM_GBS, 4),
                  "mfma_frac": round(upd_flops / (total_ms * 1e-3) / 1e12 / PEAK_BF16_TFLOPS, 4),
                  "dominant": {"kernel": PHASES[dom], "gbs": round(d_gbs, 1), "hbm_frac": round(d_gbs / PEAK_HBM_GBS, 4),
                               "traffic": measured_traffic(PHASES[dom])}}
        log(f"update phases (ms): {update['phase_ms']}")

    if "chain" in sections:
        ch_ms, stage_ms, ch_shape = bench_chain(args.phase_iters)
        Bc, Lc, Cc, Dc, Fc = ch_shape["B"], ch_shape["L"], ch_shape["C"], ch_shape["D"], ch_shape["F"]
        state_bytes = 48 * Dc * Fc * Bc  # W and S read and written once per chunk
        apply_ms = stage_ms[-1]
        chain = {"ms": round(ch_ms, 4), "shape": ch_shape,
                 "stage_ms": {"layers_mean": round(sum(stage_ms[:-1]) / Lc, 4), "state_write": round(apply_ms, 4)},
                 "hbm_frac_min_state_bytes": round(state_bytes / (ch_ms * 1e-3) / 1e9 / PEAK_HBM_GBS, 4),
                 "mfma_frac_update_flops": round(20 * Cc * Dc * Fc * Lc * Bc / (ch_ms * 1e-3) / 1e12
                                                 / PEAK_BF16_TFLOPS, 4),
                 "state_write_hbm_frac": round(state_bytes / (apply_ms * 1e-3) / 1e9 / PEAK_HBM_GBS, 4),
                 "state_write_traffic": measured_traffic("k_chain_apply")}
        log(f"layer chain {ch_ms:.3f} ms per chunk; stages (ms) {chain['stage_ms']}")

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
        if run_cpu:
            cpu_more["config4"] = cpu_baseline_c4(model, args.cpu_decode_steps)
            log(f"cpu config 4: {cpu_more['config4']['value']} tok/s")

    line = {"metric": METRIC, "value": round(line_value, 1), "unit": "tok/s", "n_gpus": 1,
            "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(c3_ms, 2), "higher_is_better": True,
            "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
            "data": "synthetic: uniform token ids, random-init weights (reference init), fp32 fast-weight masters",
            "config": {"workload": "config3_prefill_with_fast_weight_writes", "global_batch": C3_BATCH,
                       "seq_len": C3_SEQ, "layers": C3["n_layers"], "d_model": C3["d_model"],
                       "d_ff_fast": C3["d_ff_fast"], "heads": C3["n_heads"], "kv_heads": C3["n_kv_heads"],
                       "window": C3["sliding_window_size"], "chunk": C3["chunk_size"],
                       "parallelism": "none (1 GPU)", "hip_graph": False, "finite": finite},
            "roofline": roofline, "prefill": prefill, **big, "update": update, "chain": chain, "decode": decode,
            "cpu_baseline": cpu, "cpu_baselines": cpu_more or None}
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
