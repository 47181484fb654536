"""Ragged per-request updates (utttcompanion_amd.evolve) against the per-request path.

The reference updates one request at a time (batch 1, turn right-padded to a chunk
multiple with a mask).  Each request of a ragged batch must give what its own batch-1
update gives: the oracle's ``test_time_update`` (fp32, <= 1e-5 relative for W, S and the
surprise values; exact step count) and this library's batch-1 ``uTTTModel.test_time_update``.
The per-chunk surprise gate (not in the reference) is checked against the oracle's
restatement of it, at thresholds kept away from every chunk's row loss so rounding cannot
flip a decision.
"""
import math

import pytest
import torch

from oracle import uttt_math as om
from test_gpu_model import DEV, NAMES, SMALL, build, rel_err

pytestmark = pytest.mark.gpu

LENGTHS = [7, 16, 33, 50, 21, 48]  # chunk size 16: 1, 1, 3, 4, 2, 3 chunks


def requests(model, oracle, seed=3, vocab=256):
    g = torch.Generator().manual_seed(seed)
    ids, masks, states, ostates = [], [], [], []
    for i, n in enumerate(LENGTHS):
        ids.append(torch.randint(6, vocab, (n,), generator=g))
        m = torch.ones(n)
        if i == 2:
            m[-5:] = 0  # caller-side right padding, as the personalizer sends it
        if i == 3:
            m[16:32] = 0  # a whole chunk without valid tokens: no write, no surprise weight
        masks.append(m)
        st = oracle.init_state(1)
        for name in ("w_up", "w_gate", "w_down"):
            t = getattr(st, name)
            t.add_(0.02 * torch.randn(t.shape, generator=g))
        st.s_up.add_(1e-3 * torch.randn(st.s_up.shape, generator=g))
        st.step = 3 * i
        ostates.append(st)
        states.append(to_state(st))
    return ids, masks, states, ostates


def to_state(ost):
    from utttcompanion_amd import FastWeightState
    return FastWeightState(*(getattr(ost, n).clone().to(DEV) for n in NAMES), ost.ln_weight.to(DEV),
                           ost.ln_bias.to(DEV), ost.step, 0.0, [])


def test_ragged_update_rows_match_oracle_and_batch1():
    from utttcompanion_amd.evolve import ragged_test_time_update
    model, oracle = build()
    ids, masks, states, ostates = requests(model, oracle)
    print("ragged update, lengths", LENGTHS, flush=True)
    got = ragged_test_time_update(model, [t.to(DEV) for t in ids], states, [m.to(DEV) for m in masks])
    torch.cuda.synchronize()
    for i, (cand, surprise, layers) in enumerate(got):
        ocand, osurprise, olayers = oracle.test_time_update(ids[i].view(1, -1), ostates[i], masks[i].view(1, -1))
        for n in NAMES:
            assert rel_err(getattr(cand, n), getattr(ocand, n)) <= 1e-5, (i, n)
        assert abs(surprise - osurprise) <= 1e-5 * max(1.0, abs(osurprise)), i
        assert rel_err(torch.tensor(layers), torch.tensor(olayers)) <= 1e-5, i
        assert cand.step == ocand.step, i
        one, s1, l1 = model.test_time_update(ids[i].view(1, -1).to(DEV), states[i], masks[i].view(1, -1).to(DEV))
        for n in NAMES:
            assert rel_err(getattr(cand, n), getattr(one, n)) <= 1e-5, (i, n)
        assert abs(surprise - s1) <= 1e-5 * max(1.0, abs(s1))
    for st, ost in zip(states, ostates):  # the caller's states are untouched
        for n in NAMES:
            assert torch.equal(getattr(st, n).cpu(), getattr(ost, n)), n


def test_ragged_update_without_masks_equals_padded_turns():
    """Unmasked turns of any length equal the personalizer's padded + masked form."""
    from utttcompanion_amd.evolve import ragged_test_time_update
    model, oracle = build()
    ids, _, states, ostates = requests(model, oracle, seed=9)
    got = ragged_test_time_update(model, [t.to(DEV) for t in ids], states)
    c = SMALL["chunk_size"]
    for i, (cand, surprise, _) in enumerate(got):
        n = ids[i].shape[0]
        padded = ((n + c - 1) // c) * c
        pid = torch.zeros(1, padded, dtype=torch.long)
        pid[0, :n] = ids[i]
        pm = torch.zeros(1, padded)
        pm[0, :n] = 1
        ocand, osurprise, _ = oracle.test_time_update(pid, ostates[i], pm)
        for name in NAMES:
            assert rel_err(getattr(cand, name), getattr(ocand, name)) <= 1e-5, (i, name)
        assert abs(surprise - osurprise) <= 1e-5 * max(1.0, abs(osurprise))


def _chunk_row_means(oracle, ids, masks, ostates, threshold):
    """Every (chunk, layer) row surprise the oracle's gated run meets, by wrapping its step."""
    seen = []
    real = om.fused_chunk_ttt_step

    def spy(q, k, v, eta, alpha, w_up, w_gate, w_down, s_up, s_gate, s_down, ln_w, ln_b, mask, *rest):
        seen.append(om.row_surprise(k, v, w_up, w_gate, w_down, ln_w, ln_b, mask, True, 1e-5).flatten())
        return real(q, k, v, eta, alpha, w_up, w_gate, w_down, s_up, s_gate, s_down, ln_w, ln_b, mask, *rest)

    om.fused_chunk_ttt_step = spy
    try:
        oracle.cfg.min_chunk_surprise = threshold
        outs = [oracle.test_time_update(ids[i].view(1, -1), ostates[i], masks[i].view(1, -1))
                for i in range(len(ids))]
    finally:
        om.fused_chunk_ttt_step = real
        oracle.cfg.min_chunk_surprise = 0.0
    return outs, torch.cat(seen)


def test_per_chunk_surprise_gate_matches_oracle():
    from utttcompanion_amd.evolve import ragged_test_time_update
    model, oracle = build()
    ids, masks, states, ostates = requests(model, oracle, seed=5)
    _, means = _chunk_row_means(oracle, ids, masks, ostates, 0.0)
    vals = torch.sort(means[means > 0]).values
    gaps = vals[1:] - vals[:-1]
    j = int(torch.argmax(gaps[len(gaps) // 4: 3 * len(gaps) // 4])) + len(gaps) // 4
    threshold = float((vals[j] + vals[j + 1]) / 2)
    outs, seen = _chunk_row_means(oracle, ids, masks, ostates, threshold)
    margin = (seen[seen > 0] - threshold).abs().min().item()
    assert margin > 1e-4 * threshold, "threshold too close to a chunk's row loss"
    assert bool(((seen > 0) & (seen < threshold)).any())
    got = ragged_test_time_update(model, [t.to(DEV) for t in ids], states, [m.to(DEV) for m in masks],
                                  min_chunk_surprise=threshold)
    changed = 0
    for i, (cand, surprise, layers) in enumerate(got):
        ocand, osurprise, olayers = outs[i]
        for n in NAMES:
            assert rel_err(getattr(cand, n), getattr(ocand, n)) <= 1e-5, (i, n)
        assert abs(surprise - osurprise) <= 1e-5 * max(1.0, abs(osurprise)), i
        changed += int(not torch.equal(ocand.w_up, ostates[i].w_up))
    assert 0 < changed  # the gate skipped some chunks, not all
    # a threshold above every loss leaves every state as it was (step still advances)
    got = ragged_test_time_update(model, [t.to(DEV) for t in ids], states, [m.to(DEV) for m in masks],
                                  min_chunk_surprise=1e30)
    for i, (cand, _, _) in enumerate(got):
        for n in NAMES:
            assert torch.equal(getattr(cand, n).cpu(), getattr(ostates[i], n)), (i, n)
        assert cand.step == ostates[i].step + math.ceil(LENGTHS[i] / 16) * SMALL["n_layers"]


def test_evolve_batched_gate_and_pull_match_per_request():
    from utttcompanion_amd.evolve import evolve_batched
    model, oracle = build()
    ids, masks, states, ostates = requests(model, oracle, seed=7)
    per = [oracle.test_time_update(ids[i].view(1, -1), ostates[i], masks[i].view(1, -1)) for i in range(len(ids))]
    s = sorted(p[1] for p in per)
    gaps = [b - a for a, b in zip(s, s[1:])]
    j = max(range(len(gaps)), key=gaps.__getitem__)
    threshold = (s[j] + s[j + 1]) / 2
    res = evolve_batched(model, [t.to(DEV) for t in ids], states, [m.to(DEV) for m in masks],
                         surprise_threshold=threshold, anchor_lambda=0.02, max_drift_ratio=1e-3)
    w0 = tuple(oracle.pool[n] for n in ("w_up_init", "w_gate_init", "w_down_init"))
    fired = 0
    for i, r in enumerate(res):
        ocand, osurprise, _ = per[i]
        gate = om.personalizer_gate(osurprise, threshold)
        assert r.gate_triggered == gate, i
        if gate:
            fired += 1
            expect = om.apply_elastic_pull((ocand.w_up, ocand.w_gate, ocand.w_down), w0, 0.02, 1e-3)
            for a, e in zip((r.state.w_up, r.state.w_gate, r.state.w_down), expect):
                assert rel_err(a, e) <= 1e-5, i
            for n in ("s_up", "s_gate", "s_down"):
                assert rel_err(getattr(r.state, n), getattr(ocand, n)) <= 1e-5, (i, n)
        else:
            assert r.state is states[i]
    assert 0 < fired < len(res)


def test_ragged_update_bf16_rows_match_batch1():
    """bf16 activations: each row equals its batch-1 update (same kernels, same rounding
    points; only the batch the GEMMs see differs), within the bf16 weight bound."""
    from utttcompanion_amd.evolve import ragged_test_time_update
    model, oracle = build(dtype=torch.bfloat16)
    ids, masks, states, _ = requests(model, oracle, seed=11)
    got = ragged_test_time_update(model, [t.to(DEV) for t in ids], states, [m.to(DEV) for m in masks])
    for i, (cand, surprise, _) in enumerate(got):
        one, s1, _ = model.test_time_update(ids[i].view(1, -1).to(DEV), states[i], masks[i].view(1, -1).to(DEV))
        for n in NAMES:
            err = (getattr(cand, n) - getattr(one, n)).abs().max().item()
            assert err <= 2e-2, (i, n, err)
        assert abs(surprise - s1) <= 2e-2 * max(1.0, abs(s1))


def test_ragged_update_rejects_bad_input():
    from utttcompanion_amd.evolve import ragged_test_time_update
    model, oracle = build()
    ids, masks, states, _ = requests(model, oracle)
    with pytest.raises(ValueError):
        ragged_test_time_update(model, [t.to(DEV) for t in ids], states[:-1])
    with pytest.raises(ValueError):
        ragged_test_time_update(model, [ids[0].to(DEV)], [states[0]], [masks[1].to(DEV)])
    with pytest.raises(ValueError):
        ragged_test_time_update(model, [ids[0].to(DEV)], [states[0]], min_chunk_surprise=-1.0)
    with pytest.raises(ValueError):
        ragged_test_time_update(model, [torch.zeros(0, dtype=torch.long, device=DEV)], [states[0]])


@pytest.mark.parametrize("masked", [False, True])
def test_chunk_update_row_loss_and_gate_match_oracle(masked):
    """Kernel level: the per-row [sum of masked token losses, valid tokens] output and the
    per-chunk gate of ``uttt_chunk_update`` against the oracle's step and row surprise."""
    from test_gpu_kernels import make_chunk, to_dev
    from utttcompanion_amd import kernels as K
    b, c, d, f = 4, 64, 128, 192
    q, k, v, eta, alpha, w, s, ln_w, ln_b = make_chunk(b, c, d, f, seed=31)
    v = v * torch.tensor([0.3, 1.0, 3.0, 10.0]).view(b, 1, 1)  # row losses far apart
    mask = None
    if masked:
        mask = torch.ones(b, c)
        mask[1, 40:] = 0
        mask[3, ::3] = 0
    rows = om.row_surprise(k, v, *w, ln_w, ln_b, mask, True, 1e-5)
    assert all(rows[i] < rows[i + 1] for i in range(b - 1))
    thr = float(rows[1] + rows[2]) / 2
    ref = om.fused_chunk_ttt_step(q, k, v, eta, alpha, *w, *s, ln_w, ln_b, mask, 0.9, 1.0, True, 1e-5,
                                  min_row_surprise=thr)
    dev_in = to_dev(q, k, v, eta, alpha, *w, *s, ln_w, ln_b, mask)
    row_loss = torch.full((b, 2), float("nan"), device=DEV)
    with torch.no_grad():
        prep = K.prepare_chunk_update(*dev_in[:13], dev_in[13], 0.9, 1.0, True, 1e-5,
                                      row_loss=row_loss, min_row_surprise=thr)
        got = prep.launch()
    torch.cuda.synchronize()
    for name, a, e in zip(("readout", *NAMES, "surprise"), got, ref):
        assert rel_err(a, e) <= 1e-5, name
    for i in (0, 1):  # under the gate: W and S unchanged
        for a, o in zip(got[1:7], w + s):
            assert torch.equal(a[i].cpu(), o[i])
    counts = mask.sum(1) if masked else torch.full((b,), float(c))
    assert torch.equal(row_loss[:, 1].cpu(), counts)
    assert rel_err(row_loss[:, 0].cpu() / counts, rows) <= 1e-5


def _kernel_row_means(row_loss):
    """The per-chunk gate's input as the kernels form it: sum / max(count, 1) in fp32."""
    rl = row_loss.detach().float().cpu()
    return rl[..., 0] / torch.clamp(rl[..., 1], min=1.0)


@pytest.mark.parametrize("masked", [False, True])
def test_chunk_update_gate_is_inclusive_at_the_threshold(masked):
    """``uttt_chunk_update``: a row whose chunk loss equals the threshold exactly is written
    (the gate skips a chunk only when its loss is below the threshold); one float step above
    its loss it keeps W and S.  The threshold is the kernel's own row mean, read from its
    ``row_loss`` output, so the comparison is exact."""
    import numpy as np
    from test_gpu_kernels import make_chunk, to_dev
    from utttcompanion_amd import kernels as K
    b, c, d, f = 4, 64, 128, 192
    q, k, v, eta, alpha, w, s, ln_w, ln_b = make_chunk(b, c, d, f, seed=37)
    v = v * torch.tensor([0.3, 1.0, 3.0, 10.0]).view(b, 1, 1)
    mask = None
    if masked:
        mask = torch.ones(b, c)
        mask[2, 30:] = 0
    dev_in = to_dev(q, k, v, eta, alpha, *w, *s, ln_w, ln_b, mask)

    def run(thr):
        rl = torch.full((b, 2), float("nan"), device=DEV)
        with torch.no_grad():
            out = K.prepare_chunk_update(*dev_in[:13], dev_in[13], 0.9, 1.0, True, 1e-5, row_loss=rl,
                                         min_row_surprise=thr).launch()
        torch.cuda.synchronize()
        return out, rl

    plain, rl = run(0.0)
    means = _kernel_row_means(rl)
    for r in (1, 2):
        thr = float(means[r])
        for t in (thr, float(np.nextafter(np.float32(thr), np.float32(np.inf)))):
            got, _ = run(t)
            for i in range(b):
                written = bool(means[i] >= np.float32(t))
                if i == r:
                    assert written == (t == thr)
                for a, p, o in zip(got[1:7], plain[1:7], w + s):
                    if written:
                        assert torch.equal(a[i], p[i]), (r, t, i)
                    else:
                        assert torch.equal(a[i].cpu(), o[i]), (r, t, i)


def test_chain_gate_is_inclusive_at_the_threshold():
    """``uttt_chunk_chain`` (one layer, so the gate reads the chunk-start state): the same
    boundary as the single update, at the chain's own row mean."""
    import numpy as np
    from test_gpu_chain import make_layers
    from utttcompanion_amd import kernels as K
    layers, w, s, ln_w, ln_b = make_layers(1, 4, 64, 128, 192, seed=39)
    layers = [(x[0], x[1] * torch.tensor([0.3, 1.0, 3.0, 10.0]).view(4, 1, 1), x[2], x[3]) for x in layers]
    k, v, eta, alpha = (t.to(DEV) for t in layers[0])

    def run(thr):
        state = [t.clone().to(DEV) for t in w + s]
        rl = torch.full((1, 4, 2), float("nan"), device=DEV)
        with torch.no_grad():
            K.chunk_chain([k], [v], [eta], [alpha], state, ln_w.to(DEV), ln_b.to(DEV), None, 0.9, 1.0, True, 1e-5,
                          row_loss=rl, min_row_surprise=thr)
        torch.cuda.synchronize()
        return state, rl

    plain, rl = run(0.0)
    means = _kernel_row_means(rl[0])
    thr = float(means[2])
    for t in (thr, float(np.nextafter(np.float32(thr), np.float32(np.inf)))):
        got, _ = run(t)
        for i in range(4):
            written = bool(means[i] >= np.float32(t))
            if i == 2:
                assert written == (t == thr)
            for a, p, o in zip(got, plain, w + s):
                if written:
                    assert torch.equal(a[i], p[i]), (t, i)
                else:
                    assert torch.equal(a[i].cpu(), o[i]), (t, i)


def test_evolve_batched_turn_gate_at_a_real_surprise():
    """The turn gate with real HIP surprises: the threshold is one request's surprise
    exactly, so that request is not written (strict ``>``, personalizer.py:525) while the
    requests above it are, each after the real elastic pull."""
    from utttcompanion_amd import evolve
    model, oracle = build()
    ids, masks, states, _ = requests(model, oracle, seed=13)
    dids, dmasks = [t.to(DEV) for t in ids], [m.to(DEV) for m in masks]
    updates = evolve.ragged_test_time_update(model, dids, states, dmasks)
    surprises = [u[1] for u in updates]
    order = sorted(range(len(surprises)), key=surprises.__getitem__)
    j = order[len(order) // 2]
    threshold = surprises[j]
    real = evolve.ragged_test_time_update
    evolve.ragged_test_time_update = lambda *a, **kw: updates
    try:
        res = evolve.evolve_batched(model, dids, states, dmasks, surprise_threshold=threshold, anchor_lambda=0.05,
                                    max_drift_ratio=None)
    finally:
        evolve.ragged_test_time_update = real
    pool = model.fast_weight_pool
    for i, r in enumerate(res):
        assert r.gate_triggered == (surprises[i] > threshold), i
        if r.gate_triggered:
            want = pool.apply_elastic_pull(updates[i][0], 0.05, None)
            for n in ("w_up", "w_gate", "w_down"):
                assert torch.equal(getattr(r.state, n), getattr(want, n)), (i, n)
        else:
            assert r.state is states[i]
    assert not res[j].gate_triggered and any(r.gate_triggered for r in res)
