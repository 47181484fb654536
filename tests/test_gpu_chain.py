"""GPU parity of the layer chain (``uttt_chunk_chain``) with L sequential updates.

The chain computes one chunk's updates of all L layers at once: layer l's update is
applied to the state left by layers 0..l-1.  The expected state is the oracle's
``fused_chunk_ttt_step`` applied L times in sequence (reference model/uttt_layer.py:414-534
inside the chunk-first schedule of model/uttt_model.py:453-608).  Tolerances as for the
single update: fp32 <= 1e-5 relative (max|err| / max|ref|) for W, S and the per-layer
surprise; bf16 activations <= 2e-2 max-abs for the fp32 state against the fp32 oracle.
"""
import math

import pytest
import torch

from oracle import uttt_math as om

pytestmark = pytest.mark.gpu
DEV = "cuda"
NAMES = ("w_up", "w_gate", "w_down", "s_up", "s_gate", "s_down")


def rel_err(actual, expected):
    actual = actual.detach().double().cpu()
    expected = expected.detach().double().cpu()
    return (actual - expected).abs().max().item() / max(expected.abs().max().item(), 1e-30)


def make_layers(n_layers, b, c, d, f, seed, w_scale=None):
    g = torch.Generator().manual_seed(seed)
    sw = w_scale if w_scale is not None else 1.0 / math.sqrt(d)
    layers = []
    for _ in range(n_layers):
        k, v = torch.randn(b, c, d, generator=g), torch.randn(b, c, d, generator=g)
        eta = 0.02 * torch.sigmoid(torch.randn(b, c, 1, generator=g))
        alpha = 0.01 * torch.sigmoid(torch.randn(b, c, 1, generator=g) - 1.386)
        layers.append((k, v, eta, alpha))
    w = (torch.randn(b, d, f, generator=g) * sw, torch.randn(b, d, f, generator=g) * sw,
         torch.randn(b, f, d, generator=g) * 0.3 / math.sqrt(f))
    s = tuple(torch.randn(t.shape, generator=g) * 1e-3 for t in w)
    ln_w = 1.0 + 0.1 * torch.randn(d, generator=g)
    ln_b = 0.05 * torch.randn(d, generator=g)
    return layers, w, s, ln_w, ln_b


def oracle_chain(layers, w, s, ln_w, ln_b, mask, beta, clip, norm, gate=0.0):
    surprises = []
    for k, v, eta, alpha in layers:
        res = om.fused_chunk_ttt_step(k, k, v, eta, alpha, *w, *s, ln_w, ln_b, mask, beta, clip, norm, 1e-5,
                                      min_row_surprise=gate)
        w, s = res[1:4], res[4:7]
        surprises.append(res[7])
    return w + s, torch.stack(surprises)


def run_chain(layers, w, s, ln_w, ln_b, mask, beta, clip, norm, dtype, gate=0.0, copies=False, row_loss=False):
    from utttcompanion_amd import kernels as K
    b, c, d = layers[0][0].shape
    state = [t.clone().to(DEV) for t in w + s]
    ks = [x[0].to(DEV, dtype) for x in layers]
    vs = [x[1].to(DEV, dtype) for x in layers]
    etas = [x[2].to(DEV, dtype) for x in layers]
    alphas = [x[3].to(DEV, dtype) for x in layers]
    cps = [t.to(torch.bfloat16) for t in state] if copies else None  # chunk-start state in bf16
    rl = torch.full((len(layers), b, 2), float("nan"), device=DEV) if row_loss else None
    with torch.no_grad():
        surprise, _ = K.chunk_chain(ks, vs, etas, alphas, state, ln_w.to(DEV), ln_b.to(DEV),
                                    None if mask is None else mask.to(DEV), beta, clip, norm, 1e-5, copies=cps,
                                    row_loss=rl, min_row_surprise=gate)
    torch.cuda.synchronize()
    return state, surprise, cps, rl


CASES = [
    dict(L=3, b=2, c=64, d=128, f=192, mask=False, clip=1.0, norm=True, beta=0.9),
    dict(L=5, b=3, c=40, d=64, f=128, mask=True, clip=1e-3, norm=True, beta=0.9),    # tail chunk, clip active
    dict(L=12, b=1, c=64, d=256, f=512, mask=False, clip=1.0, norm=False, beta=0.95),  # 12 layers, 1 row
    dict(L=2, b=4, c=17, d=192, f=320, mask=True, clip=0.0, norm=True, beta=0.0),     # no clip, no momentum
]


@pytest.mark.parametrize("case", CASES)
def test_chain_fp32_matches_sequential_oracle(case):
    print(f"chain case {case}", flush=True)
    layers, w, s, ln_w, ln_b = make_layers(case["L"], case["b"], case["c"], case["d"], case["f"], seed=3 + case["L"])
    mask = None
    if case["mask"]:
        mask = torch.ones(case["b"], case["c"])
        mask[0, case["c"] // 2:] = 0
        if case["b"] > 2:
            mask[2] = 0  # a row with no valid token keeps W and S through every layer
    ref, ref_s = oracle_chain(layers, w, s, ln_w, ln_b, mask, case["beta"], case["clip"], case["norm"])
    got, got_s, _, _ = run_chain(layers, w, s, ln_w, ln_b, mask, case["beta"], case["clip"], case["norm"],
                                 torch.float32)
    for name, a, e in zip(NAMES, got, ref):
        err = rel_err(a, e)
        assert err <= 1e-5, f"{name}: rel err {err:.3e}"
    assert rel_err(got_s, ref_s) <= 1e-5
    if case["mask"] and case["b"] > 2:
        for a, o in zip(got, w + s):
            assert torch.equal(a[2].cpu(), o[2]), "a row without tokens changed"


@pytest.mark.parametrize("copies", [False, True])
def test_chain_bf16_within_tolerance(copies):
    """bf16 activations, reading the fp32 masters or their bf16 copies (which then hold the
    final state, rounded)."""
    layers, w, s, ln_w, ln_b = make_layers(6, 2, 64, 256, 512, seed=41, w_scale=0.02)
    ref, ref_s = oracle_chain(layers, w, s, ln_w, ln_b, None, 0.9, 1.0, True)
    got, got_s, cps, _ = run_chain(layers, w, s, ln_w, ln_b, None, 0.9, 1.0, True, torch.bfloat16, copies=copies)
    for name, a, e in zip(NAMES, got, ref):
        err = (a.cpu() - e).abs().max().item()
        assert err <= 2e-2, f"{name}: max abs err {err:.3e}"
    assert (got_s.cpu() - ref_s).abs().max().item() <= 2e-2 * max(1.0, ref_s.abs().max().item())
    if copies:
        for cp, st in zip(cps, got):
            assert torch.equal(cp, st.to(torch.bfloat16))


def test_chain_equals_per_layer_hip_updates_bf16():
    """The chain and L calls of the single-layer HIP update take the same bf16 operands."""
    from utttcompanion_amd import kernels as K
    layers, w, s, ln_w, ln_b = make_layers(4, 3, 64, 128, 256, seed=7, w_scale=0.05)
    got, got_s, _, _ = run_chain(layers, w, s, ln_w, ln_b, None, 0.9, 1.0, True, torch.bfloat16)
    state = [t.clone().to(DEV) for t in w + s]
    surprises = []
    with torch.no_grad():
        for k, v, eta, alpha in layers:
            kb = k.to(DEV, torch.bfloat16)
            res = K.chunk_update(kb, kb, v.to(DEV, torch.bfloat16), eta.to(DEV, torch.bfloat16),
                                 alpha.to(DEV, torch.bfloat16), *state, ln_w.to(DEV), ln_b.to(DEV), None, 0.9, 1.0,
                                 True, 1e-5)
            state = list(res[1:7])
            surprises.append(res[7])
    for name, a, e in zip(NAMES, got, state):
        scale = e.abs().max().item()
        err = (a - e).abs().max().item()
        assert err <= 5e-3 * scale + 1e-6, f"{name}: {err:.3e} vs scale {scale:.3e}"
    assert rel_err(got_s, torch.stack(surprises)) <= 1e-2


def test_chain_equals_per_layer_hip_updates_at_config2_shape():
    """The full config-2 chunk (8 rows, 12 layers, C 64, D 768, F 2048, bf16 activations,
    reference init N(0, 0.02)): the chain against 12 calls of the single-layer HIP update,
    which takes the same bf16 operands.  Bound: 1e-3 of each tensor's largest entry (measured:
    at most 1.5e-4, in the momentum S_up)."""
    from utttcompanion_amd import kernels as K
    print("chain at the config-2 chunk shape", flush=True)
    layers, w, s, ln_w, ln_b = make_layers(12, 8, 64, 768, 2048, seed=12, w_scale=0.02)
    got, got_s, _, _ = run_chain(layers, w, s, ln_w, ln_b, None, 0.9, 1.0, True, torch.bfloat16)
    state = [t.clone().to(DEV) for t in w + s]
    surprises = []
    with torch.no_grad():
        for k, v, eta, alpha in layers:
            kb = k.to(DEV, torch.bfloat16)
            res = K.chunk_update(kb, kb, v.to(DEV, torch.bfloat16), eta.to(DEV, torch.bfloat16),
                                 alpha.to(DEV, torch.bfloat16), *state, ln_w.to(DEV), ln_b.to(DEV), None, 0.9, 1.0,
                                 True, 1e-5)
            state = list(res[1:7])
            surprises.append(res[7])
    torch.cuda.synchronize()
    for name, a, e in zip(NAMES, got, state):
        scale = e.abs().max().item()
        err = (a - e).abs().max().item()
        print(f"{name}: max err {err:.3e} scale {scale:.3e}", flush=True)
        assert torch.isfinite(a).all()
        assert err <= 1e-3 * scale + 1e-7, f"{name}: {err:.3e} vs scale {scale:.3e}"
    assert rel_err(got_s, torch.stack(surprises)) <= 1e-2


@pytest.mark.parametrize("masked", [False, True])
def test_chain_row_loss_and_gate_match_oracle(masked):
    layers, w, s, ln_w, ln_b = make_layers(3, 4, 64, 128, 192, seed=13)
    for i, x in enumerate(layers):  # rows with losses far apart, so a threshold separates them
        layers[i] = (x[0], x[1] * torch.tensor([0.3, 1.0, 3.0, 10.0]).view(4, 1, 1), x[2], x[3])
    mask = None
    if masked:
        mask = torch.ones(4, 64)
        mask[1, 40:] = 0
        mask[3, ::3] = 0
    means = [om.row_surprise(x[0], x[1], *w, ln_w, ln_b, mask, True, 1e-5) for x in layers[:1]]
    thr = float(means[0][1] + means[0][2]) / 2
    ref, ref_s = oracle_chain(layers, w, s, ln_w, ln_b, mask, 0.9, 1.0, True, gate=thr)
    got, got_s, _, rl = run_chain(layers, w, s, ln_w, ln_b, mask, 0.9, 1.0, True, torch.float32, gate=thr,
                                  row_loss=True)
    for name, a, e in zip(NAMES, got, ref):
        assert rel_err(a, e) <= 1e-5, name
    assert rel_err(got_s, ref_s) <= 1e-5
    counts = mask.sum(1) if masked else torch.full((4,), 64.0)
    assert torch.equal(rl[0, :, 1].cpu(), counts)
    assert rel_err(rl[0, :, 0].cpu() / counts, means[0]) <= 1e-5


def test_chain_rejects_bad_input():
    from utttcompanion_amd import kernels as K
    layers, w, s, ln_w, ln_b = make_layers(2, 1, 8, 64, 64, seed=1)
    state = [t.to(DEV) for t in w + s]
    ks = [x[0].to(DEV) for x in layers]
    with pytest.raises(ValueError):
        K.chunk_chain(ks, ks[:1], ks, ks, state, ln_w.to(DEV), ln_b.to(DEV), None, 0.9, 1.0, True, 1e-5)
    with pytest.raises(ValueError):  # in-place state must be fp32
        K.chunk_chain(ks, ks, [x[2].to(DEV) for x in layers], [x[3].to(DEV) for x in layers],
                      [t.double() for t in state], ln_w.to(DEV), ln_b.to(DEV), None, 0.9, 1.0, True, 1e-5)


def _chain_run(layers, w, s, ln_w, ln_b, shared):
    """Chunk-start state (fp32 + bf16 copies) and a stage-by-stage ChunkChainRun over it."""
    from utttcompanion_amd import kernels as K
    state = [t.clone().to(DEV) for t in w + s]
    cps = [t.to(torch.bfloat16) for t in state]
    b, c, _ = layers[0][0].shape
    run = K.ChunkChainRun(len(layers), c, state, ln_w.to(DEV), ln_b.to(DEV), None, 0.9, 1.0, True, 1e-5,
                          torch.bfloat16, copies=cps, w_products_given=shared)
    return run, state, cps


def _layer_inputs(layer):
    return tuple(x.to(DEV, torch.bfloat16) for x in layer)


@pytest.mark.parametrize("c, d", [(64, 256), (40, 192)])
def test_readout_key_products_equal_chain_products(c, d):
    """The readout's key block forms k W_up and k W_gate bit for bit as the chain's own
    snapshot products (same operands, same MFMA order), and leaves the readout unchanged."""
    from utttcompanion_amd import kernels as K
    print(f"key products c={c} d={d}", flush=True)
    layers, w, s, ln_w, ln_b = make_layers(1, 3, c, d, 384, seed=91, w_scale=0.05)
    run, state, cps = _chain_run(layers, w, s, ln_w, ln_b, shared=False)
    k, v, eta, alpha = _layer_inputs(layers[0])
    g = torch.Generator().manual_seed(5)
    q = torch.randn(3, c, d, generator=g).to(DEV, torch.bfloat16)
    out_up = torch.full((3, 64, 384), float("nan"), dtype=torch.bfloat16, device=DEV)
    out_gate = torch.full_like(out_up, float("nan"))
    with torch.no_grad():
        layer = run.set_layer(k, v, eta, alpha)
        run.launch(layer, part=1)  # all four snapshot products of layer 0
        plain = K.swiglu_readout(q, *cps[:3], ln_w.to(DEV), ln_b.to(DEV), 1e-5)
        with_keys = K.swiglu_readout(q, *cps[:3], ln_w.to(DEV), ln_b.to(DEV), 1e-5, keys=k,
                                     key_outputs=(out_up, out_gate))
    torch.cuda.synchronize()
    ref_up, ref_gate = run.w_product_outputs(0)
    assert torch.equal(with_keys, plain)
    assert torch.equal(out_up, ref_up)
    assert torch.equal(out_gate, ref_gate)
    assert torch.all(out_up[:, c:] == 0) and torch.all(out_gate[:, c:] == 0)
    expect = (k.float() @ cps[0].float())  # loose check of the products themselves
    assert (out_up[:, :c].float() - expect).abs().max().item() <= 2e-2 * expect.abs().max().item()


def test_chain_with_shared_products_equals_plain_chain():
    """Stage parts with the W products from the readouts give the same chunk, bit for bit, as
    the whole stages forming every product themselves."""
    from utttcompanion_amd import kernels as K
    layers, w, s, ln_w, ln_b = make_layers(4, 3, 64, 256, 384, seed=23, w_scale=0.05)
    g = torch.Generator().manual_seed(8)
    qs = [torch.randn(3, 64, 256, generator=g).to(DEV, torch.bfloat16) for _ in layers]
    run_a, state_a, cps_a = _chain_run(layers, w, s, ln_w, ln_b, shared=False)
    run_b, state_b, cps_b = _chain_run(layers, w, s, ln_w, ln_b, shared=True)
    with torch.no_grad():
        for layer in layers:
            run_a.add_layer(*_layer_inputs(layer))
        surprise_a, _ = run_a.finish()
        for l, layer in enumerate(layers):
            k, v, eta, alpha = _layer_inputs(layer)
            run_b.set_layer(k, v, eta, alpha)
            run_b.launch(l, part=1)
            K.swiglu_readout(qs[l], *cps_b[:3], ln_w.to(DEV), ln_b.to(DEV), 1e-5, keys=k,
                             key_outputs=run_b.w_product_outputs(l))
            run_b.launch(l, part=2)
        surprise_b, _ = run_b.finish()
    torch.cuda.synchronize()
    for name, a, b_ in zip(NAMES, state_a, state_b):
        assert torch.equal(a, b_), name
    for a, b_ in zip(cps_a, cps_b):
        assert torch.equal(a, b_)
    assert torch.equal(surprise_a, surprise_b)


BF16_TAIL_CASES = [
    dict(L=5, b=3, c=40, d=192, f=320, mask=True, copies=True),   # tail chunk, masked rows, bf16 copies
    dict(L=3, b=2, c=17, d=128, f=192, mask=False, copies=True),  # short chunk
    dict(L=4, b=9, c=64, d=64, f=128, mask=True, copies=False),   # more rows than XCDs, fp32 masters
    dict(L=6, b=3, c=40, d=1024, f=1536, mask=True, copies=True),  # Gram features split over 2 and 3 slices
    dict(L=4, b=9, c=64, d=256, f=2048, mask=True, copies=True),   # 288 back-pass tiles: d range split in two
]


@pytest.mark.parametrize("case", BF16_TAIL_CASES)
def test_chain_bf16_tail_chunks_within_tolerance(case):
    """bf16 chains over partial chunks (rows past C are zero in every operand) and masked rows,
    against the fp32 oracle's sequential steps."""
    print(f"bf16 tail case {case}", flush=True)
    layers, w, s, ln_w, ln_b = make_layers(case["L"], case["b"], case["c"], case["d"], case["f"], seed=61 + case["c"],
                                           w_scale=0.03)
    mask = None
    if case["mask"]:
        mask = torch.ones(case["b"], case["c"])
        mask[0, case["c"] // 2:] = 0
        mask[case["b"] - 1] = 0  # a row with no valid token keeps W and S through every layer
    ref, ref_s = oracle_chain(layers, w, s, ln_w, ln_b, mask, 0.9, 1.0, True)
    got, got_s, _, _ = run_chain(layers, w, s, ln_w, ln_b, mask, 0.9, 1.0, True, torch.bfloat16,
                                 copies=case["copies"])
    for name, a, e in zip(NAMES, got, ref):
        err = (a.cpu() - e).abs().max().item()
        assert err <= 2e-2, f"{name}: max abs err {err:.3e}"
    assert (got_s.cpu() - ref_s).abs().max().item() <= 2e-2 * max(1.0, ref_s.abs().max().item())
    if case["mask"]:
        for a, o in zip(got, w + s):
            assert torch.equal(a[case["b"] - 1].cpu(), o[case["b"] - 1]), "a row without tokens changed"


def test_single_launches_with_timer_equal_whole_stages():
    """``uttt_chunk_chain_stage_launch``: a stage enqueued launch by launch (with events around
    the followed kernels) equals the stage enqueued at once, bit for bit; the names follow the
    launch sequence and every followed launch is timed."""
    from utttcompanion_amd import kernels as K
    layers, w, s, ln_w, ln_b = make_layers(4, 3, 64, 256, 384, seed=29, w_scale=0.05)
    run_a, state_a, cps_a = _chain_run(layers, w, s, ln_w, ln_b, shared=False)
    run_b, state_b, cps_b = _chain_run(layers, w, s, ln_w, ln_b, shared=False)
    timer = K.KernelTimer(("k_chain_back_lds", "k_chain_apply_lds", "k_chain_gram_lds", "k_chain_keys_lds"))
    with torch.no_grad():
        for layer in layers:
            run_a.add_layer(*_layer_inputs(layer))
        sa, _ = run_a.finish()
        for l, layer in enumerate(layers):
            run_b.set_layer(*_layer_inputs(layer))
            names = run_b.stage_launches(l)
            assert names[-1] == "k_chain_back_lds" and "k_chain_up_lds" in names
            run_b.launch(l, timer=timer)
        assert run_b.stage_launches(4) == ("k_chain_coef", "k_chain_apply_lds")
        sb, _ = run_b.launch(4, timer=timer)
    torch.cuda.synchronize()
    for name, a, b_ in zip(NAMES, state_a, state_b):
        assert torch.equal(a, b_), name
    assert torch.equal(sa, sb)
    summary = timer.summary()
    assert summary["k_chain_back_lds"]["launches"] == 4 and summary["k_chain_apply_lds"]["launches"] == 1
    # per layer: the snapshot products with the key Gram row in one launch, then the H and dZ Grams
    assert summary["k_chain_keys_lds"]["launches"] == 4 and summary["k_chain_gram_lds"]["launches"] == 8
    assert all(v["mean_ms"] > 0 for v in summary.values())
    with pytest.raises(RuntimeError, match="out of range"):
        from utttcompanion_amd import _native as N
        import ctypes as C
        N.check(N.load_library().uttt_chunk_chain_stage_launch(C.byref(run_b.args), run_b.workspace.data_ptr(),
                                                                 run_b.workspace.numel(), 4, 0, 1, 3, None, 0, None,
                                                                 None), "stage launch")


DEEP_CASES = [
    dict(b=2, d=1024, f=1536, mask=False),  # one snapshot-product launch per layer
    dict(b=2, d=2048, f=5504, mask=True),   # config-3 dims: 180 MB per product launch, grouped layers
]


@pytest.mark.parametrize("case", DEEP_CASES, ids=[f"d{c['d']}-f{c['f']}" for c in DEEP_CASES])
def test_chain_bf16_24_layers_against_both_oracles(case):
    """The depth of configs 3 and 5: a 24-layer bf16 chain reading bf16 copies of the chunk-start
    state (the prefill's form), against 24 sequential oracle steps in fp32 (host CPU) and in the
    reference's bf16 arithmetic (oracle16: bf16 keys, values, eta, alpha and bf16 matmuls with the
    fp32 masters; run by torch on the GPU).  Bound: 2e-2 max-abs for the fp32 state against
    either, the surprise within 2e-2 of each (relative above 1)."""
    b, d, f = case["b"], case["d"], case["f"]
    print(f"24-layer bf16 chain, B {b}, D {d}, F {f}", flush=True)
    layers, w, s, ln_w, ln_b = make_layers(24, b, 64, d, f, seed=240 + d, w_scale=0.02)
    mask = None
    if case["mask"]:
        mask = torch.ones(b, 64)
        mask[1, 40:] = 0
    ref, ref_s = oracle_chain(layers, w, s, ln_w, ln_b, mask, 0.9, 1.0, True)
    l16 = [tuple(x.to(DEV, torch.bfloat16) for x in layer) for layer in layers]
    with torch.no_grad():
        ref16, ref16_s = oracle_chain(l16, tuple(t.to(DEV) for t in w), tuple(t.to(DEV) for t in s), ln_w.to(DEV),
                                      ln_b.to(DEV), None if mask is None else mask.to(DEV), 0.9, 1.0, True)
    got, got_s, cps, _ = run_chain(layers, w, s, ln_w, ln_b, mask, 0.9, 1.0, True, torch.bfloat16, copies=True)
    for name, a, e, e16 in zip(NAMES, got, ref, ref16):
        assert torch.isfinite(a).all(), name
        err, err16 = (a.cpu() - e).abs().max().item(), (a - e16).abs().max().item()
        print(f"  {name}: vs fp32 {err:.3e}, vs reference bf16 {err16:.3e}", flush=True)
        assert err <= 2e-2 and err16 <= 2e-2, name
    for ref_sur in (ref_s, ref16_s.float().cpu()):
        assert (got_s.cpu() - ref_sur).abs().max().item() <= 2e-2 * max(1.0, ref_sur.abs().max().item())
    for cp, st in zip(cps, got):
        assert torch.equal(cp, st.to(torch.bfloat16))
