"""GPU parity at the dimensions of BASELINE configs 2-5 (the other GPU tests use small shapes).

* Config 3 / 5 dimensions (d_model 2048, d_ff 5504, 16 heads x 128, window 1024): the single
  update (fp32 and bf16), the readout, the window-skipping attention, and the layer chain with
  the grouped snapshot products -- at 2 rows the state read of a product launch,
  8 * D * F * B bytes = 180 MB, is past the 128 MiB single-layer limit, so layers 0-3 share one
  ``k_chain_pq`` launch (fp32 masters fed stage by stage, and bf16 copies without the readouts'
  W products).  A two-layer model of these dimensions runs ``evolve_batched`` on ragged
  requests against the oracle's per-request ``test_time_update`` + gate + pull.
* Config 2 / 4 model (12 layers, d_model 768, 12 heads x 64, 4 kv heads, window 512, d_ff 2048,
  vocab 32000, reference initialisation): prefill with writes against the oracle (fp32 and
  bf16), and the batched ring decoder's bf16 logits against the fp32 oracle.

Tolerances (north star): fp32 <= 1e-5 relative (max|err| / max|ref|); bf16 updated fp32 fast
weights <= 2e-2 max-abs against the fp32 oracle and against the reference's own bf16 arithmetic
(the oracle run in bf16, rounding where the reference rounds: "oracle16").  bf16 logits: <= 2e-2
max-abs against both, except where the reference's bf16 arithmetic is itself further than that
from a second run of the same arithmetic.  Through the 12 layers of the config-2 model the
oracle16 logits on the host CPU and the same oracle16 run by torch on the GPU (identical rounding
points; only the libraries' accumulation order differs) are 0.065 apart (largest logit 2.9; a
bf16 ulp there is 0.016), and either is 0.07 from fp32: no bf16 implementation that is not
bit-identical to one of them can be within 2e-2 of it.  There the bound is 1.5 x oracle16's own
error + 1e-3 against fp32 (the rule the small-model bf16 tests use), and against oracle16 1.5 x the
larger of that error and the measured spread, + 1e-3 (two bf16 implementations each about that far
from fp32 are up to about that far from each other).  Every case prints its measured distances.
"""
import math

import pytest
import torch

from oracle import uttt_math as om
from test_gpu_chain import NAMES, make_layers, oracle_chain, rel_err
from test_gpu_kernels import BF16_ABS, F32_REL, check_bf16_activation, make_chunk, max_abs, to_dev

pytestmark = pytest.mark.gpu
DEV = "cuda"
D3, F3 = 2048, 5504


def _report(name, err, bound):
    print(f"  {name}: {err:.3e} (bound {bound:.1e})", flush=True)
    assert err <= bound, f"{name}: {err:.3e} > {bound:.1e}"


def _bf16_logit_bound(reference_bf16_err):
    """2e-2, or 1.5x the reference's own bf16 error (+1e-3) where that is larger."""
    return max(BF16_ABS, 1.5 * reference_bf16_err + 1e-3)


# ---------------------------------------------------------------------------------------------
# config-3 / config-5 dimensions, kernel level
# ---------------------------------------------------------------------------------------------

def test_chunk_update_fp32_config3_dims():
    from utttcompanion_amd import kernels as K
    print("fp32 chunk update, B 1, D 2048, F 5504", flush=True)
    q, k, v, eta, alpha, w, s, ln_w, ln_b = make_chunk(1, 64, D3, F3, seed=303, scale_w=0.02)
    ref = om.fused_chunk_ttt_step(q, k, v, eta, alpha, *w, *s, ln_w, ln_b, None, 0.9, 1.0, True, 1e-5)
    with torch.no_grad():
        got = K.chunk_update(*to_dev(q, k, v, eta, alpha, *w, *s, ln_w, ln_b), None, 0.9, 1.0, True, 1e-5)
    torch.cuda.synchronize()
    for name, a, e in zip(("readout", *NAMES, "surprise"), got, ref):
        _report(name, rel_err(a, e), F32_REL)


def test_chunk_update_bf16_config3_dims():
    from utttcompanion_amd import kernels as K
    print("bf16 chunk update, B 2, D 2048, F 5504", flush=True)
    q, k, v, eta, alpha, w, s, ln_w, ln_b = make_chunk(2, 64, D3, F3, seed=305, scale_w=0.02)
    q16, k16, v16, e16, a16 = (t.bfloat16() for t in (q, k, v, eta, alpha))
    ref = om.fused_chunk_ttt_step(q16.float(), k16.float(), v16.float(), e16.float(), a16.float(), *w, *s,
                                  ln_w, ln_b, None, 0.9, 1.0, True, 1e-5)
    ref16 = om.fused_chunk_ttt_step(q16, k16, v16, e16, a16, *w, *s, ln_w, ln_b, None, 0.9, 1.0, True, 1e-5)
    with torch.no_grad():
        got = K.chunk_update(*to_dev(q16, k16, v16, e16, a16, *w, *s, ln_w, ln_b), None, 0.9, 1.0, True, 1e-5)
    torch.cuda.synchronize()
    check_bf16_activation("readout", got[0], ref[0], ref16[0])
    for name, a, e in zip(NAMES, got[1:7], ref[1:7]):
        _report(name, max_abs(a, e), BF16_ABS)
    _report("surprise", abs(got[7].item() - ref[7].item()) / max(1.0, abs(ref[7].item())), 2e-2)


@pytest.mark.parametrize("tokens", [64, 1])
def test_readout_config3_dims(tokens):
    """The frozen readout at d_model 2048, d_ff 5504: fp32 masters (fp32 and bf16 activations)
    and bf16 read copies."""
    from utttcompanion_amd import kernels as K
    print(f"readout D 2048 F 5504, {tokens} tokens", flush=True)
    b = 3
    g = torch.Generator().manual_seed(311 + tokens)
    x = torch.randn(b, tokens, D3, generator=g)
    w = (torch.randn(b, D3, F3, generator=g) * 0.02, torch.randn(b, D3, F3, generator=g) * 0.02,
         torch.randn(b, F3, D3, generator=g) * 0.02)
    ln_w, ln_b = 1 + 0.1 * torch.randn(D3, generator=g), 0.1 * torch.randn(D3, generator=g)
    dw = to_dev(*w, ln_w, ln_b)
    with torch.no_grad():
        f32 = K.swiglu_readout(x.to(DEV), *dw, eps=1e-5)
        x16 = x.bfloat16()
        from_masters = K.swiglu_readout(x16.to(DEV), *dw, eps=1e-5)
        from_copies = K.swiglu_readout(x16.to(DEV), *(t.bfloat16() for t in dw[:3]), *dw[3:], eps=1e-5)
    torch.cuda.synchronize()
    _report("fp32 readout", rel_err(f32, om.swiglu_fast_forward(x, *w, ln_w, ln_b, 1e-5)), F32_REL)
    ref = om.swiglu_fast_forward(x16.float(), *(t.bfloat16().float() for t in w), ln_w, ln_b, 1e-5)
    ref16 = om.swiglu_fast_forward(x16, *w, ln_w, ln_b, 1e-5)
    # the two reads take the same bf16 operands; with several tokens they run in different
    # kernels (fp32 tiles rounded in registers, bf16 tiles loaded straight into LDS), whose MFMA
    # accumulation orders differ, so both are held to the bf16 bound rather than to each other
    check_bf16_activation("bf16 readout from fp32 masters", from_masters, ref, ref16)
    check_bf16_activation("bf16 readout from bf16 copies", from_copies, ref, ref16)
    if tokens == 1:  # one token: both take the same GEMV, so they agree bit for bit
        assert torch.equal(from_masters, from_copies)


@pytest.mark.parametrize("case", [
    dict(b=1, tq=64, tkv=1152),   # one chunk after 1088 keys: the first key tiles are outside the window
    dict(b=2, tq=300, tkv=1400),  # several query tiles, windows clipped on both sides
])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_swa_prefill_config3_window(case, dtype):
    """head_dim 128, 16 query heads on 4 kv heads, window 1024, more keys than the window: the
    kernel visits only in-window key tiles and splits the key range over workgroups."""
    from utttcompanion_amd import kernels as K
    print(f"swa prefill hd 128 window 1024 {case} {dtype}", flush=True)
    g = torch.Generator().manual_seed(313 + case["tq"])
    b, tq, tkv, h, hkv, hd, win = case["b"], case["tq"], case["tkv"], 16, 4, 128, 1024
    q = torch.randn(b, tq, h, hd, generator=g).to(dtype).transpose(1, 2)
    k = torch.randn(b, hkv, tkv, hd, generator=g).to(dtype)
    v = torch.randn(b, hkv, tkv, hd, generator=g).to(dtype)
    off = tkv - tq
    ref = om.sliding_window_attention(q.float(), k.float(), v.float(), win, off)
    with torch.no_grad():
        got = K.swa_prefill(*to_dev(q, k, v), win, off)
    torch.cuda.synchronize()
    if dtype == torch.float32:
        _report("attention", rel_err(got, ref), F32_REL)
    else:
        _report("attention", max_abs(got, ref), BF16_ABS)
    # a key just outside every query's window must not matter
    k2 = k.clone()
    k2[:, :, : max(0, off - win + 1)] = 1e4
    with torch.no_grad():
        got2 = K.swa_prefill(*to_dev(q, k2, v), win, off)
    torch.cuda.synchronize()
    assert torch.equal(got, got2)


def test_chain_grouped_products_fp32_stage_by_stage_config3_dims():
    """fp32 masters, 5 layers, 2 rows at D 2048 / F 5504: layers 0-3 form their snapshot
    products in one grouped launch (stage 3), layer 4 alone; fed layer by layer through
    ``ChunkChainRun.add_layer`` as the prefill does."""
    from utttcompanion_amd import kernels as K
    print("fp32 chain, 5 layers, B 2, D 2048, F 5504 (grouped snapshot products)", flush=True)
    assert 8 * D3 * F3 * 2 > 128 * (1 << 20)
    layers, w, s, ln_w, ln_b = make_layers(5, 2, 64, D3, F3, seed=321, w_scale=0.02)
    ref, ref_s = oracle_chain(layers, w, s, ln_w, ln_b, None, 0.9, 1.0, True)
    state = [t.clone().to(DEV) for t in w + s]
    with torch.no_grad():
        run = K.ChunkChainRun(5, 64, state, ln_w.to(DEV), ln_b.to(DEV), None, 0.9, 1.0, True, 1e-5, torch.float32)
        for k, v, eta, alpha in layers:
            run.add_layer(k.to(DEV), v.to(DEV), eta.to(DEV), alpha.to(DEV))
        surprise, _ = run.finish()
    torch.cuda.synchronize()
    for name, a, e in zip(NAMES, state, ref):
        _report(name, rel_err(a, e), F32_REL)
    _report("surprise", rel_err(surprise, ref_s), F32_REL)


def test_chain_grouped_products_bf16_copies_config3_dims():
    """bf16 activations and bf16 state copies without the readouts' W products: the grouped
    ``k_chain_pq`` forms all four products from the copies.  The copies hold the final state
    rounded to bf16 afterwards."""
    from utttcompanion_amd import kernels as K
    print("bf16 chain with copies, 5 layers, B 2, D 2048, F 5504 (grouped snapshot products)", flush=True)
    layers, w, s, ln_w, ln_b = make_layers(5, 2, 64, D3, F3, seed=323, w_scale=0.02)
    layers = [tuple(x.bfloat16().float() for x in layer) for layer in layers]
    ref, ref_s = oracle_chain(layers, w, s, ln_w, ln_b, None, 0.9, 1.0, True)
    state = [t.clone().to(DEV) for t in w + s]
    cps = [t.to(torch.bfloat16) for t in state]
    with torch.no_grad():
        surprise, _ = K.chunk_chain([x[0].to(DEV, torch.bfloat16) for x in layers],
                                    [x[1].to(DEV, torch.bfloat16) for x in layers],
                                    [x[2].to(DEV, torch.bfloat16) for x in layers],
                                    [x[3].to(DEV, torch.bfloat16) for x in layers], state, ln_w.to(DEV),
                                    ln_b.to(DEV), None, 0.9, 1.0, True, 1e-5, copies=cps)
    torch.cuda.synchronize()
    for name, a, e in zip(NAMES, state, ref):
        _report(name, max_abs(a, e), BF16_ABS)
    _report("surprise", (surprise.cpu() - ref_s).abs().max().item() / max(1.0, ref_s.abs().max().item()), 2e-2)
    for cp, st in zip(cps, state):
        assert torch.equal(cp, st.to(torch.bfloat16))


# ---------------------------------------------------------------------------------------------
# config-5 dimensions, model level: ragged evolve on a two-layer D 2048 / F 5504 model
# ---------------------------------------------------------------------------------------------

C5_MODEL = dict(vocab_size=256, d_model=D3, n_layers=2, n_heads=16, n_kv_heads=4, d_ff_fast=F3, chunk_size=64,
                sliding_window_size=1024, max_seq_len=4096)
ORACLE_KEYS = ("d_model", "n_layers", "n_heads", "n_kv_heads", "d_ff_fast", "sliding_window_size", "vocab_size",
               "chunk_size")


def _reference_init_model(cfg_kw, seed, dtype):
    """A model with the reference initialisation (its own draws) and the matching oracle; slow
    weights rounded to ``dtype`` for both, the fast-weight pool (W_0, LayerNorm) fp32 for both
    (the model's pool is reloaded after the cast, which would otherwise have rounded it)."""
    from utttcompanion_amd import uTTTConfig, uTTTModel
    torch.manual_seed(seed)
    model = uTTTModel(uTTTConfig(**cfg_kw)).eval()
    weights = {k: v.detach().clone() for k, v in model.state_dict().items()}
    if dtype != torch.float32:
        weights = {k: (v if k.startswith("fast_weight_pool.") else v.to(dtype).float()) for k, v in weights.items()}
    model = model.to(DEV)
    if dtype != torch.float32:
        model.to(dtype)
        model.fast_weight_pool.float()
        pre = "fast_weight_pool."
        model.fast_weight_pool.load_state_dict({k[len(pre):]: v for k, v in weights.items() if k.startswith(pre)})
    ocfg = om.OracleConfig(**{k: cfg_kw[k] for k in ORACLE_KEYS})
    return model, om.OracleModel(ocfg, weights), weights


def _oracle_on(oracle, dev):
    """The oracle's weights moved to ``dev`` (the same restated arithmetic, run by torch there)."""
    oracle.w = {k: v.to(dev) for k, v in oracle.w.items()}
    oracle.layers = [{k: v.to(dev) for k, v in lw.items()} for lw in oracle.layers]
    oracle.pool = {k: v.to(dev) for k, v in oracle.pool.items()}
    oracle.cos, oracle.sin = oracle.cos.to(dev), oracle.sin.to(dev)
    return oracle


def _state_on(st, dev):
    return om.OracleState(*(getattr(st, n).to(dev) for n in om.OracleState.NAMES), st.ln_weight.to(dev),
                          st.ln_bias.to(dev), st.step)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_evolve_batched_config5_dims(dtype):
    """Three ragged requests (150, 64, 97 tokens; the first one padded by its caller) on a
    two-layer model of the config-5 dimensions: per request, the oracle's batch-1
    ``test_time_update``, the turn gate and the elastic pull (lambda 1e-3, drift ceiling
    0.35)."""
    from utttcompanion_amd import FastWeightState
    from utttcompanion_amd.evolve import evolve_batched
    print(f"evolve_batched, 2 layers, D 2048, F 5504, {dtype}", flush=True)
    model, oracle, weights = _reference_init_model(C5_MODEL, 51, dtype)
    g = torch.Generator().manual_seed(52)
    lengths = [150, 64, 97]
    ids = [torch.randint(6, 256, (n,), generator=g) for n in lengths]
    masks = [torch.ones(n) for n in lengths]
    masks[0][-9:] = 0
    ostates, states = [], []
    for i in range(len(lengths)):
        st = oracle.init_state(1)
        for name in ("w_up", "w_gate", "w_down"):
            t = getattr(st, name)
            t.add_(0.005 * torch.randn(t.shape, generator=g))
        ostates.append(st)
        states.append(FastWeightState(*(getattr(st, n).clone().to(DEV) for n in NAMES), st.ln_weight.to(DEV),
                                      st.ln_bias.to(DEV), 0, 0.0, []))
    per = [oracle.test_time_update(ids[i].view(1, -1), ostates[i], masks[i].view(1, -1)) for i in range(3)]
    surprises = sorted(p[1] for p in per)
    threshold = (surprises[0] + surprises[1]) / 2  # two of three requests pass
    res = evolve_batched(model, [t.to(DEV) for t in ids], states, [m.to(DEV) for m in masks],
                         surprise_threshold=threshold, anchor_lambda=1e-3, max_drift_ratio=0.35)
    torch.cuda.synchronize()
    w0 = tuple(oracle.pool[n] for n in ("w_up_init", "w_gate_init", "w_down_init"))
    fired = 0
    for i, r in enumerate(res):
        ocand, osurprise, olayers = per[i]
        f32 = dtype == torch.float32
        _report(f"request {i} surprise", abs(r.surprise - osurprise) / max(1.0, abs(osurprise)),
                F32_REL if f32 else 2e-2)
        for n in NAMES:
            a, e = getattr(r.candidate, n), getattr(ocand, n)
            _report(f"request {i} {n}", rel_err(a, e) if f32 else max_abs(a, e), F32_REL if f32 else BF16_ABS)
        assert r.candidate.step == ocand.step
        gate = om.personalizer_gate(osurprise, threshold)
        assert r.gate_triggered == gate, i
        if gate:
            fired += 1
            expect = om.apply_elastic_pull((ocand.w_up, ocand.w_gate, ocand.w_down), w0, 1e-3, 0.35)
            for n, a, e in zip(NAMES[:3], (r.state.w_up, r.state.w_gate, r.state.w_down), expect):
                _report(f"request {i} pulled {n}", rel_err(a, e) if f32 else max_abs(a, e),
                        F32_REL if f32 else BF16_ABS)
        else:
            assert r.state is states[i]
    assert fired == 2


# ---------------------------------------------------------------------------------------------
# config-2 / config-4 model (12 layers, d_model 768, vocab 32000)
# ---------------------------------------------------------------------------------------------

C2_MODEL = dict(vocab_size=32000, d_model=768, n_layers=12, n_heads=12, n_kv_heads=4, d_ff_fast=2048, chunk_size=64,
                sliding_window_size=512, max_seq_len=4096)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_config2_model_prefill_with_writes(dtype):
    """The 12-layer config-2 model, 2 rows x 192 tokens (3 chunks x 12 layers of chained
    writes; the second row right-padded by 11 masked tokens), reference initialisation."""
    print(f"config-2 model prefill with writes, 2 x 192 tokens, {dtype}", flush=True)
    model, oracle, weights = _reference_init_model(C2_MODEL, 61, dtype)
    g = torch.Generator().manual_seed(62)
    ids = torch.randint(6, 32000, (2, 192), generator=g)
    mask = torch.ones(2, 192)
    mask[1, -11:] = 0
    out = model(ids.to(DEV), attention_mask=mask.to(DEV), update_fast_weights=True)
    logits, state, per_layer, _ = oracle.forward(ids, None, mask, update_fast_weights=True)
    if dtype == torch.float32:
        _report("logits", rel_err(out.logits, logits), F32_REL)
        for n in NAMES:
            _report(n, rel_err(getattr(out.fast_state, n), getattr(state, n)), F32_REL)
        _report("layer surprise", rel_err(torch.tensor(out.layer_surprise_losses), per_layer), F32_REL)
    else:
        oracle16 = om.OracleModel(oracle.cfg, weights, dtype=torch.bfloat16)
        logits16, state16, _, _ = oracle16.forward(ids, None, mask, update_fast_weights=True)
        o16gpu = _oracle_on(om.OracleModel(oracle.cfg, weights, dtype=torch.bfloat16), DEV)
        with torch.no_grad():
            logits16g, state16g, _, _ = o16gpu.forward(ids.to(DEV), None, mask.to(DEV), update_fast_weights=True)
        theirs = max_abs(logits16, logits)
        spread = max_abs(logits16g, logits16)
        print(f"  reference bf16 logits vs fp32: {theirs:.3e}; reference bf16 on the GPU vs on the CPU: "
              f"{spread:.3e}", flush=True)
        _report("logits vs fp32", max_abs(out.logits, logits), _bf16_logit_bound(theirs))
        _report("logits vs reference bf16", max_abs(out.logits, logits16), _bf16_logit_bound(max(spread, theirs)))
        for n in NAMES:
            _report(f"{n} vs fp32", max_abs(getattr(out.fast_state, n), getattr(state, n)), BF16_ABS)
            _report(f"{n} vs reference bf16", max_abs(getattr(out.fast_state, n), getattr(state16, n)), BF16_ABS)
            print(f"    (reference bf16 on two devices: {max_abs(getattr(state16g, n), getattr(state16, n)):.3e})")
    assert out.fast_state.step == state.step == 3 * 12


def test_config4_batched_decoder_bf16_logits_against_fp32_oracle():
    """The config-4 decode path: the 12-layer config-2 model in bf16, 4 requests with their own
    fp32 fast-weight states (N(0, 0.02), seeded by request id) and ragged prompts (one longer
    than the 512 window), one HIP graph per step.  Each step's logits against the fp32
    oracle's frozen forward of the same tokens, within the bf16 logit bound (the reference's own
    bf16 error measured on the same steps)."""
    from utttcompanion_amd import FastWeightState
    from utttcompanion_amd.decoder import BatchedDecoder
    print("config-4 batched decoder, bf16 logits against the fp32 oracle", flush=True)
    model, oracle, weights = _reference_init_model(C2_MODEL, 71, torch.bfloat16)
    oracle16 = om.OracleModel(oracle.cfg, weights, dtype=torch.bfloat16)
    o16gpu = _oracle_on(om.OracleModel(oracle.cfg, weights, dtype=torch.bfloat16), DEV)
    lengths = [70, 33, 600, 5]
    states, ostates, prompts = [], [], []
    for rid, n in enumerate(lengths):
        g = torch.Generator().manual_seed(rid)
        ws = [0.02 * torch.randn(1, 768, 2048, generator=g), 0.02 * torch.randn(1, 768, 2048, generator=g),
              0.02 * torch.randn(1, 2048, 768, generator=g)]
        zeros = [torch.zeros_like(t) for t in ws]
        ln = (oracle.pool["ln_weight"], oracle.pool["ln_bias"])
        ostates.append(om.OracleState(*ws, *zeros, *ln))
        states.append(FastWeightState(*(t.to(DEV) for t in ws + zeros), ln[0].to(DEV), ln[1].to(DEV)))
        prompts.append(torch.randint(6, 32000, (n,), generator=g))
    dec = BatchedDecoder(model, states)
    first = dec.prefill(prompts).float()
    caches, caches16, caches16g = [], [], []
    gstates = [_state_on(st, DEV) for st in ostates]
    ours = ours16 = theirs = spread = 0.0

    def record(got_row, lg, lg16, lg16g):
        nonlocal ours, ours16, theirs, spread
        ours, ours16 = max(ours, max_abs(got_row, lg)), max(ours16, max_abs(got_row, lg16))
        theirs, spread = max(theirs, max_abs(lg16, lg)), max(spread, max_abs(lg16g, lg16))

    with torch.no_grad():
        for i, ids in enumerate(prompts):
            lg, _, _, cache = oracle.forward(ids.view(1, -1), ostates[i], None, None, 0, False, 1)
            lg16, _, _, cache16 = oracle16.forward(ids.view(1, -1), ostates[i], None, None, 0, False, 1)
            lg16g, _, _, cache16g = o16gpu.forward(ids.view(1, -1).to(DEV), gstates[i], None, None, 0, False, 1)
            caches.append(cache)
            caches16.append(cache16)
            caches16g.append(cache16g)
            record(first[i], lg[0, -1], lg16[0, -1], lg16g[0, -1])
        print(f"  prefill logits: ours {ours:.3e} (vs reference bf16 {ours16:.3e}), reference bf16 {theirs:.3e}",
              flush=True)
        dec.capture()
        tok = first.argmax(-1)
        for step in range(8):
            got = dec.step(tok).float()
            torch.cuda.synchronize()
            for i, ids in enumerate(prompts):
                t = tok[i].view(1, 1).cpu()
                pos = len(ids) + step
                lg, _, _, caches[i] = oracle.forward(t, ostates[i], None, caches[i], pos, False, 0)
                lg16, _, _, caches16[i] = oracle16.forward(t, ostates[i], None, caches16[i], pos, False, 0)
                lg16g, _, _, caches16g[i] = o16gpu.forward(t.to(DEV), gstates[i], None, caches16g[i], pos, False, 0)
                record(got[i], lg[0, -1], lg16[0, -1], lg16g[0, -1])
            tok = dec.next_tokens.clone()
    print(f"  reference bf16 logits vs fp32 (prefill + 8 steps x 4 requests): {theirs:.3e}; reference bf16 on the "
          f"GPU vs on the CPU: {spread:.3e}", flush=True)
    _report("logits vs fp32, worst of prefill + 8 steps x 4 requests", ours, _bf16_logit_bound(theirs))
    _report("logits vs reference bf16, worst of prefill + 8 steps x 4 requests", ours16, _bf16_logit_bound(max(spread, theirs)))


EXEC_MODEL = dict(vocab_size=512, d_model=D3, n_layers=2, n_heads=16, n_kv_heads=4, d_ff_fast=2048, chunk_size=64,
                  sliding_window_size=1024, max_seq_len=2048)


def test_prefill_chunk_executor_config3_attention_shape_against_oracle():
    """The headline path, ``uttt_prefill_chunk`` (bf16), at the config-3 layer shape: d_model
    2048, 16 heads x 128 (4 kv heads), window 1024; two layers, 2 rows x 1152 tokens (18 chunks:
    the window fills after 16 and then slides; row 1's last 29 tokens masked), reference
    initialisation.  Logits and updated fast weights against the fp32 oracle and the
    reference's bf16 arithmetic (oracle16), with the bounds of the config-2 test."""
    from utttcompanion_amd.prefill_plan import PrefillPlan
    print("executor at the config-3 layer shape, 2 layers, 2 x 1152 tokens", flush=True)
    model, oracle, weights = _reference_init_model(EXEC_MODEL, 81, torch.bfloat16)
    g = torch.Generator().manual_seed(82)
    ids = torch.randint(6, 512, (2, 1152), generator=g)
    mask = torch.ones(2, 1152)
    mask[1, -29:] = 0
    runs = []
    orig_run = PrefillPlan.run
    PrefillPlan.run = lambda self, *a, **k: (runs.append(1), orig_run(self, *a, **k))[1]
    try:
        with torch.no_grad():
            out = model(ids.to(DEV), attention_mask=mask.to(DEV), update_fast_weights=True)
        torch.cuda.synchronize()
    finally:
        PrefillPlan.run = orig_run
    assert len(runs) == 18, "the executor ran every chunk"
    logits, state, per_layer, _ = oracle.forward(ids, None, mask, update_fast_weights=True)
    oracle16 = om.OracleModel(oracle.cfg, weights, dtype=torch.bfloat16)
    logits16, state16, _, _ = oracle16.forward(ids, None, mask, update_fast_weights=True)
    o16gpu = _oracle_on(om.OracleModel(oracle.cfg, weights, dtype=torch.bfloat16), DEV)
    with torch.no_grad():
        logits16g, _, _, _ = o16gpu.forward(ids.to(DEV), None, mask.to(DEV), update_fast_weights=True)
    theirs, spread = max_abs(logits16, logits), max_abs(logits16g, logits16)
    print(f"  reference bf16 logits vs fp32: {theirs:.3e}; reference bf16 on the GPU vs on the CPU: {spread:.3e} "
          f"(largest logit {logits.abs().max().item():.2f})", flush=True)
    _report("logits vs fp32", max_abs(out.logits, logits), _bf16_logit_bound(theirs))
    _report("logits vs reference bf16", max_abs(out.logits, logits16), _bf16_logit_bound(max(spread, theirs)))
    for n in NAMES:
        _report(f"{n} vs fp32", max_abs(getattr(out.fast_state, n), getattr(state, n)), BF16_ABS)
        _report(f"{n} vs reference bf16", max_abs(getattr(out.fast_state, n), getattr(state16, n)), BF16_ABS)
    _report("layer surprise", rel_err(torch.tensor(out.layer_surprise_losses), per_layer), 1e-2)
    assert out.fast_state.step == state.step == 18 * 2

