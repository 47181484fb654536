"""The two surprise gates at their exact boundaries (CPU).

* The turn-level gate of ``interact_and_evolve`` (reference engine/personalizer.py:524-526):
  a non-finite or negative surprise is refused with ``ValueError`` and nothing is changed; the
  persona is written iff ``surprise > threshold`` (strict).  The reference's own test of the
  refusal patches ``test_time_update`` to return NaN (tests/test_lifecycle_audit.py:177-190);
  ``test_evolve_batched_*`` below patch this library's ragged update the same way, so the gate
  and the pull selection of ``evolve_batched`` run without a GPU.
* The per-chunk gate of config 5 (a chunk whose masked mean token loss is below the threshold
  leaves the row's W and S unchanged; "skip the chunk if loss < threshold"): a row exactly at
  the threshold is updated.

Each boundary is probed at the threshold itself and one float step either side, so a ``>=``
for ``>`` slip (or the reverse), a dropped sign check or a dropped finiteness check fails.
"""
import math

import numpy as np
import pytest
import torch

from oracle import uttt_math as om


def _up(x: float) -> float:
    return float(np.nextafter(x, np.inf))


def _down(x: float) -> float:
    return float(np.nextafter(x, -np.inf))


# ---------------------------------------------------------------------------------------------
# oracle: turn-level gate (personalizer.py:524-526)
# ---------------------------------------------------------------------------------------------

@pytest.mark.parametrize("tau", [0.5, 0.25, 0.0, 3.0])
def test_oracle_turn_gate_is_strict(tau):
    assert om.personalizer_gate(tau, tau) is False
    assert om.personalizer_gate(_up(tau), tau) is True
    if tau > 0:
        assert om.personalizer_gate(_down(tau), tau) is False
    assert om.personalizer_gate(tau + 10.0, tau) is True


@pytest.mark.parametrize("bad", [float("nan"), float("inf"), -float("inf"), -1e-30, -0.5])
def test_oracle_turn_gate_refuses_non_finite_and_negative(bad):
    with pytest.raises(ValueError, match="non-finite or negative"):
        om.personalizer_gate(bad, 0.5)


def test_oracle_turn_gate_accepts_zero():
    assert om.personalizer_gate(0.0, 0.5) is False
    assert om.personalizer_gate(-0.0, 0.5) is False  # -0.0 < 0 is False in IEEE arithmetic


# ---------------------------------------------------------------------------------------------
# oracle: per-chunk gate (min_row_surprise of fused_chunk_ttt_step)
# ---------------------------------------------------------------------------------------------

def _chunk(seed=5, b=3, c=16, d=32, f=48):
    g = torch.Generator().manual_seed(seed)
    q, k, v = (torch.randn(b, c, d, generator=g) for _ in range(3))
    v = v * torch.tensor([0.5, 1.0, 2.0])[:b].view(b, 1, 1)
    eta = torch.full((b, c, 1), 0.02)
    alpha = torch.full((b, c, 1), 0.003)
    w = (torch.randn(b, d, f, generator=g) / d ** 0.5, torch.randn(b, d, f, generator=g) / d ** 0.5,
         torch.randn(b, f, d, generator=g) * 0.05)
    s = tuple(0.01 * torch.randn(t.shape, generator=g) for t in w)
    return q, k, v, eta, alpha, w, s, torch.ones(d), torch.zeros(d)


@pytest.mark.parametrize("masked", [False, True])
def test_oracle_chunk_gate_keeps_a_row_exactly_at_the_threshold(masked):
    q, k, v, eta, alpha, w, s, ln_w, ln_b = _chunk()
    b, c = q.shape[:2]
    mask = None
    if masked:
        mask = torch.ones(b, c)
        mask[0, 5:] = 0
        mask[2, ::2] = 0
    rows = om.row_surprise(k, v, *w, ln_w, ln_b, mask, True, 1e-5)
    plain = om.fused_chunk_ttt_step(q, k, v, eta, alpha, *w, *s, ln_w, ln_b, mask, 0.9, 1.0, True, 1e-5)
    for r in range(b):
        thr = float(rows[r])
        assert thr > 0
        at = om.fused_chunk_ttt_step(q, k, v, eta, alpha, *w, *s, ln_w, ln_b, mask, 0.9, 1.0, True, 1e-5,
                                     min_row_surprise=thr)
        above = om.fused_chunk_ttt_step(q, k, v, eta, alpha, *w, *s, ln_w, ln_b, mask, 0.9, 1.0, True, 1e-5,
                                        min_row_surprise=_up(thr))
        for i in range(b):
            # a row is written iff its loss is >= the threshold: at the threshold it is written
            for got, upd, old in zip(at[1:7], plain[1:7], w + s):
                want = upd[i] if rows[i] >= thr else old[i]
                assert torch.equal(got[i], want), (r, i)
            for got, upd, old in zip(above[1:7], plain[1:7], w + s):
                want = upd[i] if rows[i] >= _up(thr) else old[i]
                assert torch.equal(got[i], want), (r, i)
        # the readout and the batch-global surprise do not depend on the gate
        assert torch.equal(at[0], plain[0]) and torch.equal(at[7], plain[7])


def test_oracle_row_surprise_is_the_masked_mean_token_loss():
    """Row loss against a per-token scalar loop (the gate's input)."""
    q, k, v, eta, alpha, w, s, ln_w, ln_b = _chunk(seed=9)
    b, c, d = k.shape
    mask = torch.ones(b, c)
    mask[1, 3:9] = 0
    got = om.row_surprise(k.double(), v.double(), *(t.double() for t in w), ln_w.double(), ln_b.double(), mask,
                          True, 1e-5)
    for i in range(b):
        tot, n = 0.0, 0.0
        for t in range(c):
            x = k[i, t].double()
            hdn = torch.nn.functional.silu(x @ w[1][i].double()) * (x @ w[0][i].double())
            z = hdn @ w[2][i].double()
            zn = (z - z.mean()) / torch.sqrt(z.var(unbiased=False) + 1e-5)
            e = x + zn - v[i, t].double()
            tot += float(mask[i, t]) * 0.5 * float(e.square().sum()) / d
            n += float(mask[i, t])
        assert abs(float(got[i]) - tot / max(n, 1.0)) <= 1e-12 * max(1.0, abs(tot))


# ---------------------------------------------------------------------------------------------
# evolve_batched: the turn gate and the pull selection, with the update patched out
# ---------------------------------------------------------------------------------------------

def _tiny_model():
    from utttcompanion_amd import uTTTConfig, uTTTModel
    torch.manual_seed(0)
    cfg = uTTTConfig(vocab_size=64, d_model=64, n_layers=1, n_heads=1, n_kv_heads=1, d_ff_fast=64, chunk_size=16,
                     sliding_window_size=16)
    return uTTTModel(cfg).eval()


def _patched(monkeypatch, model, surprises):
    """evolve_batched over len(surprises) requests whose updates return ``surprises``; returns
    (states, candidates, the list of states the pull was called with)."""
    from utttcompanion_amd import evolve
    states = [model.init_fast_state(1) for _ in surprises]
    cands = [st.clone() for st in states]
    for i, c in enumerate(cands):
        c.w_up.add_(float(i + 1))  # tell the candidates apart from the states
        c.step = states[i].step + 1

    def fake_update(m, interactions, fast_states, attention_masks=None, min_chunk_surprise=0.0):
        assert m is model and len(interactions) == len(surprises)
        return [(cands[i], s, [s]) for i, s in enumerate(surprises)]

    pulled = []

    def fake_pull(state, anchor_lambda=0.02, max_drift_ratio=None):
        pulled.append((state, anchor_lambda, max_drift_ratio))
        return state

    monkeypatch.setattr(evolve, "ragged_test_time_update", fake_update)
    monkeypatch.setattr(model.fast_weight_pool, "apply_elastic_pull", fake_pull)
    return states, cands, pulled


@pytest.mark.parametrize("bad", [float("nan"), float("inf"), -1e-6])
def test_evolve_batched_refuses_bad_surprise_and_changes_nothing(monkeypatch, bad):
    from utttcompanion_amd.evolve import evolve_batched
    model = _tiny_model()
    states, _, pulled = _patched(monkeypatch, model, [0.9, bad, 0.7])
    before = [st.w_up.clone() for st in states]
    ids = [torch.tensor([7, 8, 9]) for _ in states]
    with pytest.raises(ValueError, match="non-finite or negative"):
        evolve_batched(model, ids, states, surprise_threshold=0.5)
    assert pulled == []  # nothing was pulled (or written) before the refusal
    for st, w in zip(states, before):
        assert torch.equal(st.w_up, w)


def test_evolve_batched_gate_is_strict_at_the_threshold(monkeypatch):
    from utttcompanion_amd.evolve import evolve_batched
    model = _tiny_model()
    tau = 0.5
    surprises = [tau, _up(tau), _down(tau), 0.0, 4.0]
    states, cands, pulled = _patched(monkeypatch, model, surprises)
    ids = [torch.tensor([7, 8, 9]) for _ in states]
    res = evolve_batched(model, ids, states, surprise_threshold=tau, anchor_lambda=0.125, max_drift_ratio=0.25)
    assert [r.gate_triggered for r in res] == [om.personalizer_gate(s, tau) for s in surprises] \
        == [False, True, False, False, True]
    assert len(pulled) == 1  # one batched pull over the gated rows only
    joined, lam, ratio = pulled[0]
    assert (lam, ratio) == (0.125, 0.25)
    assert joined.w_up.shape[0] == 2
    assert torch.equal(joined.w_up[0], cands[1].w_up[0]) and torch.equal(joined.w_up[1], cands[4].w_up[0])
    for i, r in enumerate(res):
        assert r.surprise == surprises[i] and r.candidate is cands[i]
        if r.gate_triggered:
            assert torch.equal(r.state.w_up, cands[i].w_up) and r.state.step == cands[i].step
        else:
            assert r.state is states[i]  # gated off: the persona is unchanged


def test_evolve_batched_no_pull_when_nothing_passes(monkeypatch):
    from utttcompanion_amd.evolve import evolve_batched
    model = _tiny_model()
    states, _, pulled = _patched(monkeypatch, model, [0.1, 0.5])
    res = evolve_batched(model, [torch.tensor([7]), torch.tensor([8])], states, surprise_threshold=0.5)
    assert pulled == [] and not any(r.gate_triggered for r in res)
    assert all(r.state is st for r, st in zip(res, states))
    assert math.isfinite(res[0].surprise)
