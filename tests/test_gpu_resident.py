"""GPU parity of ``uttt_layer_update_resident`` (every chunk of one standalone layer's forward in
one persistent launch) against the CPU oracle's chunk loop: ``fused_chunk_ttt_step`` applied
chunk after chunk, each chunk reading the state the previous one left and reading out through
its own pre-update state, as uTTTLayer.forward does (reference model/uttt_layer.py:1451-1478).

Tolerance (north star): fp32 <= 1e-5 relative error, max|gpu - oracle| / max|oracle| per tensor.
"""
import math

import pytest
import torch

from oracle import uttt_math as om

pytestmark = pytest.mark.gpu
DEV = "cuda"
F32_REL = 1e-5
NAMES = ("w_up", "w_gate", "w_down", "s_up", "s_gate", "s_down")


def rel_err(actual, expected):
    actual = actual.detach().double().cpu()
    expected = expected.detach().double().cpu()
    return (actual - expected).abs().max().item() / max(expected.abs().max().item(), 1e-30)


def make_inputs(T, d, f, seed, eta_scale):
    g = torch.Generator().manual_seed(seed)
    q, k, v = (torch.randn(1, T, d, generator=g) for _ in range(3))
    eta = eta_scale * 0.01 * torch.sigmoid(torch.randn(1, T, 1, generator=g))
    alpha = 0.005 * torch.sigmoid(torch.randn(1, T, 1, generator=g) - 1.386)
    sw = 1.0 / math.sqrt(d)
    w = (torch.randn(1, d, f, generator=g) * sw, torch.randn(1, d, f, generator=g) * sw,
         torch.randn(1, f, d, generator=g) * 0.1 / math.sqrt(f))
    s = tuple(torch.randn(t.shape, generator=g) * 1e-3 for t in w)
    ln_w = 1.0 + 0.1 * torch.randn(d, generator=g)
    ln_b = 0.05 * torch.randn(d, generator=g)
    return q, k, v, eta, alpha, w, s, ln_w, ln_b


def make_mask(kind, T, cs, seed):
    if kind is None:
        return None
    g = torch.Generator().manual_seed(seed)
    mask = torch.ones(1, T)
    if kind == "tail":
        mask[0, T - 23:] = 0
    elif kind == "holes":
        mask[0, cs:2 * cs] = 0  # one chunk with no valid token keeps W and S
        mask[0, (torch.rand(T, generator=g) < 0.2)] = 0
    return mask


def oracle_loop(q, k, v, eta, alpha, w, s, ln_w, ln_b, mask, cs, clip, norm):
    T = q.shape[1]
    outs, surprises = [], []
    for c0 in range(0, T, cs):
        sl = slice(c0, min(T, c0 + cs))
        r = om.fused_chunk_ttt_step(q[:, sl], k[:, sl], v[:, sl], eta[:, sl], alpha[:, sl], *w, *s, ln_w, ln_b,
                                    None if mask is None else mask[:, sl], 0.9, clip, norm, 1e-5)
        outs.append(r[0])
        w, s = r[1:4], r[4:7]
        surprises.append(r[7])
    return torch.cat(outs, 1), w + s, torch.stack(surprises)


CASES = [
    dict(T=1024, d=512, f=1024, cs=64, mask=None, clip=1.0, norm=True, eta=1.0),    # config-1 layer
    dict(T=1000, d=512, f=1024, cs=64, mask="tail", clip=1.0, norm=True, eta=30.0),  # ragged tail, strong writes
    dict(T=150, d=256, f=192, cs=32, mask="holes", clip=0.0, norm=False, eta=10.0),  # 24 workgroups, empty chunk
    dict(T=2100, d=256, f=256, cs=64, mask="tail", clip=1.0, norm=True, eta=3.0),   # three launches of <= 16 chunks
    dict(T=37, d=128, f=64, cs=16, mask=None, clip=1e-4, norm=True, eta=1.0),        # clip active, 8 workgroups
]


@pytest.mark.parametrize("case", CASES, ids=[f"T{c['T']}-d{c['d']}-f{c['f']}-cs{c['cs']}" for c in CASES])
def test_resident_layer_update_matches_oracle_chunk_loop(case):
    from utttcompanion_amd import kernels as K
    T, d, f, cs = case["T"], case["d"], case["f"], case["cs"]
    print(f"resident case {case}", flush=True)
    q, k, v, eta, alpha, w, s, ln_w, ln_b = make_inputs(T, d, f, seed=T + d, eta_scale=case["eta"])
    mask = make_mask(case["mask"], T, cs, seed=3)
    ref_out, ref_state, ref_sur = oracle_loop(q, k, v, eta, alpha, w, s, ln_w, ln_b, mask, cs, case["clip"],
                                              case["norm"])
    dev = [t.to(DEV) for t in (q, k, v, eta, alpha, *w, *s, ln_w, ln_b)]
    dmask = None if mask is None else mask.to(DEV)
    with torch.no_grad():
        got = K.layer_update_resident(*dev, dmask, 0.9, case["clip"], case["norm"], 1e-5, chunk_size=cs)
    torch.cuda.synchronize()
    K.check_resident_flags(wait=True)
    assert rel_err(got[0], ref_out) <= F32_REL, "readout"
    for name, a, e in zip(NAMES, got[1:7], ref_state):
        assert rel_err(a, e) <= F32_REL, name
    assert rel_err(got[7], ref_sur) <= F32_REL, "surprise"
    if case["mask"] == "holes":  # the empty chunk's surprise is 0
        assert got[7][1].item() == 0.0


def test_resident_update_in_place_equals_fresh_outputs_and_repeats():
    from utttcompanion_amd import kernels as K
    q, k, v, eta, alpha, w, s, ln_w, ln_b = make_inputs(300, 256, 512, seed=9, eta_scale=5.0)
    dev = [t.to(DEV) for t in (q, k, v, eta, alpha, *w, *s, ln_w, ln_b)]
    with torch.no_grad():
        fresh = K.layer_update_resident(*dev, None, 0.9, 1.0, True, 1e-5)
        again = K.layer_update_resident(*dev, None, 0.9, 1.0, True, 1e-5)
        state = [t.clone() for t in dev[5:11]]
        inplace = K.layer_update_resident(*dev[:5], *state, *dev[11:13], None, 0.9, 1.0, True, 1e-5,
                                          out_state=state)
    torch.cuda.synchronize()
    K.check_resident_flags(wait=True)
    for a, b, c in zip(fresh, again, inplace):
        assert torch.equal(a, b) and torch.equal(a, c)
    assert inplace[1].data_ptr() == state[0].data_ptr()


def test_resident_barrier_timeout_is_loud_and_reported_once():
    """The timeout path, forced from the host (``force_timeout``: the flag is raised before the
    first launch, so no barrier waits and every kernel runs to its end): every result of that
    call is NaN (state, surprise, readout, over all three launches of a 33-chunk call), the
    report is raised once (the sticky device word is cleared with it), and the next call is
    clean and matches the oracle."""
    from utttcompanion_amd import kernels as K
    q, k, v, eta, alpha, w, s, ln_w, ln_b = make_inputs(2100, 256, 256, seed=21, eta_scale=3.0)
    dev = [t.to(DEV) for t in (q, k, v, eta, alpha, *w, *s, ln_w, ln_b)]
    K.check_resident_flags(wait=True)  # nothing pending from earlier tests
    with torch.no_grad():
        bad = K.layer_update_resident(*dev, None, 0.9, 1.0, True, 1e-5, force_timeout=True)
    torch.cuda.synchronize()
    for name, t in zip(("readout",) + NAMES + ("surprise",), bad):
        assert torch.isnan(t).all(), name
    with pytest.raises(RuntimeError, match="barrier timed out"):
        K.check_resident_flags(wait=True)
    K.check_resident_flags(wait=True)  # reported once
    ref_out, ref_state, ref_sur = oracle_loop(q[:, :200], k[:, :200], v[:, :200], eta[:, :200], alpha[:, :200], w,
                                              s, ln_w, ln_b, None, 64, 1.0, True)
    with torch.no_grad():
        good = K.layer_update_resident(*(t[:, :200] for t in dev[:5]), *dev[5:], None, 0.9, 1.0, True, 1e-5)
    torch.cuda.synchronize()
    K.check_resident_flags(wait=True)
    assert rel_err(good[0], ref_out) <= F32_REL
    for name, a, e in zip(NAMES, good[1:7], ref_state):
        assert rel_err(a, e) <= F32_REL, name
    assert rel_err(good[7], ref_sur) <= F32_REL


def test_layer_forward_takes_the_resident_path_for_one_fp32_row(monkeypatch):
    """uTTTLayer.forward with one fp32 row runs the resident launch (counted) and matches the
    oracle's layer forward; two rows take the per-chunk path and match it too."""
    from utttcompanion_amd import SharedFastWeightPool, kernels as K, uTTTLayer
    calls = []
    real = K.layer_update_resident

    def counted(*args, **kwargs):
        calls.append(1)
        return real(*args, **kwargs)

    monkeypatch.setattr(K, "layer_update_resident", counted)
    torch.manual_seed(0)
    d, f = 256, 512
    layer = uTTTLayer(d, chunk_size=32, base_inner_lr=0.05, base_weight_decay=0.01).eval()
    g = torch.Generator().manual_seed(4)
    lw = {}
    for name, t in layer.state_dict().items():
        if name.endswith("norm.weight"):
            lw[name] = 1.0 + 0.1 * torch.randn(t.shape, generator=g)
        elif name.endswith("w_alpha.bias"):
            lw[name] = torch.full(t.shape, -1.386)
        elif name.endswith("bias"):
            lw[name] = torch.zeros(t.shape)
        else:
            lw[name] = 0.05 * torch.randn(t.shape, generator=g)
    layer.load_state_dict(lw)
    pool = SharedFastWeightPool(d, f, normalize_loss_by_dim=True)
    layer, pool = layer.to(DEV), pool.to(DEV)
    cfg = om.OracleConfig(d_model=d, n_layers=1, n_heads=4, n_kv_heads=2, d_ff_fast=f, sliding_window_size=64,
                          chunk_size=32, base_inner_lr=0.05, base_weight_decay=0.01)
    pool_w = {n: p.detach().cpu() for n, p in pool.named_parameters()}
    for rows in (1, 2):
        x = torch.randn(rows, 200, d, generator=g)
        mask = torch.ones(rows, 200)
        mask[0, 150:] = 0
        ostate = om.init_state(pool_w, rows)
        oout, ost, osur = om.uttt_layer_forward(x, {"uttt." + n: t for n, t in lw.items()}, cfg, ostate, mask)
        state = pool.init_state(rows, device=DEV, dtype=torch.float32, detach=True)
        n0 = len(calls)
        with torch.no_grad():
            out, st, sur = layer(x.to(DEV), pool, state, attention_mask=mask.to(DEV))
        torch.cuda.synchronize()
        assert len(calls) - n0 == (1 if rows == 1 else 0)
        assert rel_err(out, oout) <= F32_REL
        for n in NAMES:
            assert rel_err(getattr(st, n), getattr(ost, n)) <= F32_REL, n
        assert rel_err(sur, osur) <= F32_REL
        assert st.step == (200 + 31) // 32
    K.check_resident_flags(wait=True)


def test_resident_update_refuses_unsupported_operands():
    from utttcompanion_amd import kernels as K
    q, k, v, eta, alpha, w, s, ln_w, ln_b = make_inputs(64, 512, 1024, seed=1, eta_scale=1.0)
    dev = [t.to(DEV) for t in (q, k, v, eta, alpha, *w, *s, ln_w, ln_b)]
    assert K.resident_update_eligible(dev[0], dev[5], 64)
    assert not K.resident_update_eligible(dev[0].bfloat16(), dev[5], 64)
    assert not K.resident_update_eligible(dev[0], dev[5], 128)
    assert not K.resident_update_eligible(dev[0].expand(2, -1, -1), dev[5], 64)
    with pytest.raises(ValueError, match="one fp32 row"):
        K.layer_update_resident(*dev, None, 0.9, 1.0, True, 1e-5, chunk_size=65)
