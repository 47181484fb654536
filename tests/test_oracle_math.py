"""Pins of the CPU oracle against autograd, brute force and the reference's closed forms.

These mirror the reference's own numerical audits (``tests/test_meta_math_audit.py``,
``tests/test_uttt_pipeline.py:43-83``, ``tests/test_reliability.py:192-207``) but run
against the oracle restatement.  Each check is independent of the formula it pins.
"""
import math

import pytest
import torch
import torch.nn.functional as F

from oracle import uttt_math as om


def _weights(b, d, f, dtype=torch.float64, scale=0.3, grad=False):
    shapes = ((b, d, f), (b, d, f), (b, f, d))
    ws = tuple(torch.randn(*s, dtype=dtype) * scale for s in shapes)
    return tuple(w.requires_grad_() for w in ws) if grad else ws


def _autograd_step(q, k, v, eta, alpha, weights, momentum, ln_w, ln_b, mask, beta, max_norm, eps):
    """Independent fused step: gradients from torch.autograd of the eta-weighted loss."""
    pred = om.swiglu_fast_forward(k, *weights, ln_w, ln_b, eps)
    losses = 0.5 * (pred - v).square().sum(-1) / k.shape[-1]
    if mask is None:
        weighted = (losses * eta.squeeze(-1)).sum() / k.shape[1]
        alpha_bar = alpha.mean(1, keepdim=True)
    else:
        counts = mask.sum(-1, keepdim=True).clamp_min(1)
        weighted = (losses * eta.squeeze(-1) * mask / counts).sum()
        alpha_bar = (alpha * mask.unsqueeze(-1)).sum(1, keepdim=True) / counts.unsqueeze(-1)
    grads = torch.autograd.grad(weighted, weights, create_graph=True)
    if max_norm > 0:
        sq = sum(g.square().sum((1, 2)) for g in grads)
        scale = (max_norm * torch.rsqrt(sq + 1e-8)).clamp(max=1).view(-1, 1, 1)
        grads = tuple(g * scale for g in grads)
    new_s = tuple(beta * s - g for s, g in zip(momentum, grads))
    new_w = tuple((1 - alpha_bar) * w + s for w, s in zip(weights, new_s))
    if mask is not None:
        act = mask.any(-1).view(-1, 1, 1)
        new_w = tuple(torch.where(act, n, o) for n, o in zip(new_w, weights))
        new_s = tuple(torch.where(act, n, o) for n, o in zip(new_s, momentum))
    return new_w, new_s


@pytest.fixture(autouse=True)
def _seed():
    torch.manual_seed(193)


@pytest.mark.parametrize("masked", [False, True])
@pytest.mark.parametrize("normalize", [False, True])
def test_analytical_gradient_matches_autograd_fp64(masked, normalize):
    b, c, d, f = 2, 5, 6, 7
    k, v = torch.randn(b, c, d, dtype=torch.float64), torch.randn(b, c, d, dtype=torch.float64)
    eta = torch.rand(b, c, 1, dtype=torch.float64) * 0.08
    ws = _weights(b, d, f, grad=True)
    ln_w, ln_b = torch.randn(d, dtype=torch.float64), torch.randn(d, dtype=torch.float64)
    mask = torch.tensor([[1, 1, 0, 1, 0], [0, 1, 0, 0, 0]], dtype=torch.float64) if masked else None
    got = om.analytical_swiglu_chunk_grad(k, v, eta, *ws, ln_w, ln_b, token_mask=mask,
                                          normalize_by_dim=normalize, eps=1e-4)
    pred = om.swiglu_fast_forward(k, *ws, ln_w, ln_b, 1e-4)
    losses = 0.5 * (pred - v).square().sum(-1) / (d if normalize else 1)
    if mask is None:
        loss, surprise = (losses * eta.squeeze(-1)).sum() / c, losses.mean()
    else:
        loss = (losses * eta.squeeze(-1) * mask / mask.sum(-1, keepdim=True).clamp_min(1)).sum()
        surprise = (losses * mask).sum() / mask.sum()
    expected = torch.autograd.grad(loss, ws)
    for g, e in zip(got[:3], expected):
        torch.testing.assert_close(g, e, atol=1e-11, rtol=1e-9)
    torch.testing.assert_close(got[3], surprise, atol=1e-12, rtol=1e-10)


def test_analytical_gradient_fp32_matches_autograd():
    """fp32 tolerance of the reference's pipeline test (test_uttt_pipeline.py:43-83)."""
    b, c, d, f = 2, 16, 32, 64
    k, v = torch.randn(b, c, d), torch.randn(b, c, d)
    eta = torch.rand(b, c, 1) * 0.05
    ws = _weights(b, d, f, dtype=torch.float32, scale=0.1, grad=True)
    ln_w, ln_b = torch.ones(d), torch.zeros(d)
    got = om.analytical_swiglu_chunk_grad(k, v, eta, *ws, ln_w, ln_b)
    pred = om.swiglu_fast_forward(k, *ws, ln_w, ln_b)
    losses = 0.5 * (pred - v).pow(2).sum(-1)
    expected = torch.autograd.grad(((eta.squeeze(-1) / c) * losses).sum(), ws)
    for g, e in zip(got[:3], expected):
        torch.testing.assert_close(g, e, atol=1e-5, rtol=1e-4)
    torch.testing.assert_close(got[3], losses.mean(), atol=1e-5, rtol=1e-5)


@pytest.mark.parametrize("max_norm", [0.0, 0.01, 1.0])
@pytest.mark.parametrize("masked", [False, True])
def test_fused_step_matches_autograd_step_over_two_chunks(max_norm, masked):
    b, c, d, f = 2, 4, 5, 6
    ws = _weights(b, d, f)
    ms = tuple(torch.randn_like(w) * 0.01 for w in ws)
    ln_w = torch.randn(d, dtype=torch.float64) * 0.8
    ln_b = torch.randn(d, dtype=torch.float64) * 0.1
    mask = torch.tensor([[1, 1, 0, 1], [0, 0, 0, 0]], dtype=torch.float64) if masked else None
    got_w, got_s = ws, ms
    exp_w, exp_s = tuple(w.clone().requires_grad_() for w in ws), ms
    for _ in range(2):
        q, k, v = (torch.randn(b, c, d, dtype=torch.float64) for _ in range(3))
        eta = torch.rand(b, c, 1, dtype=torch.float64) * 0.05
        alpha = torch.rand(b, c, 1, dtype=torch.float64) * 0.02
        pre_w = got_w
        res = om.fused_chunk_ttt_step(q, k, v, eta, alpha, *got_w, *got_s, ln_w, ln_b, mask,
                                      0.7, max_norm, True, 1e-4)
        exp_w, exp_s = _autograd_step(q, k, v, eta, alpha, exp_w, exp_s, ln_w, ln_b, mask, 0.7, max_norm, 1e-4)
        got_w, got_s = res[1:4], res[4:7]
        # the readout goes through the pre-update weights (reference: uttt_layer.py:525-533)
        torch.testing.assert_close(res[0], om.swiglu_fast_forward(q, *pre_w, ln_w, ln_b, 1e-4),
                                   atol=1e-11, rtol=1e-9)
        for g, e in zip(got_w + got_s, exp_w + exp_s):
            torch.testing.assert_close(g, e.detach(), atol=1e-11, rtol=1e-9)
        exp_w = tuple(w.detach().requires_grad_() for w in exp_w)
        exp_s = tuple(s.detach() for s in exp_s)
    if masked:  # row 1 never had a valid token: W and S are bit-identical to the start
        for g, o in zip(got_w + got_s, ws + ms):
            assert torch.equal(g[1], o[1])


def test_momentum_derivative_closed_form():
    """d W_2 / d S_1 = (1 - alpha) + beta = 0.99 + 0.7 (test_meta_math_audit.py:141-159)."""
    dim, hidden = 3, 4
    zero = torch.zeros(1, 2, dim, dtype=torch.float64)
    ws = tuple(torch.ones(*s, dtype=torch.float64) for s in ((1, dim, hidden), (1, dim, hidden), (1, hidden, dim)))
    ms = tuple(torch.zeros_like(w).requires_grad_() for w in ws)
    eta = torch.zeros(1, 2, 1, dtype=torch.float64)
    alpha = torch.full_like(eta, 0.01)
    first = None
    for i in range(2):
        res = om.fused_chunk_ttt_step(zero, zero, zero, eta, alpha, *ws, *ms,
                                      torch.ones(dim, dtype=torch.float64), torch.zeros(dim, dtype=torch.float64),
                                      None, 0.7, 0.0, True, 1e-4)
        ws, ms = res[1:4], res[4:7]
        if i == 0:
            first = ms[0]
    grad, = torch.autograd.grad(ws[0].sum(), first)
    torch.testing.assert_close(grad, torch.full_like(grad, 0.99 + 0.7), atol=1e-12, rtol=1e-12)


def test_bf16_inputs_accumulate_decay_and_small_momentum_in_fp32_master():
    """(1 - alpha)^10 and an exact 1e-5 increment (test_meta_math_audit.py:161-189)."""
    dim, hidden = 3, 4
    tok = torch.zeros(1, 2, dim, dtype=torch.bfloat16)
    init = tuple(torch.ones(*s, dtype=torch.bfloat16) for s in ((1, dim, hidden), (1, dim, hidden), (1, hidden, dim)))
    zero_m = tuple(torch.zeros_like(w) for w in init)
    eta = torch.zeros(1, 2, 1, dtype=torch.bfloat16)
    alpha = torch.full_like(eta, 0.001)
    ln_w, ln_b = torch.ones(dim, dtype=torch.bfloat16), torch.zeros(dim, dtype=torch.bfloat16)
    ws, ms = init, zero_m
    for _ in range(10):
        res = om.fused_chunk_ttt_step(tok, tok, tok, eta, alpha, *ws, *ms, ln_w, ln_b, None, 0.0, 0.0, True, 1e-4)
        ws, ms = res[1:4], res[4:7]
        assert all(t.dtype == torch.float32 for t in ws + ms)
    expected = (1 - alpha.float().mean()).pow(10)
    for w in ws:
        torch.testing.assert_close(w, expected.expand_as(w), atol=2e-7, rtol=1e-7)
    small = tuple(torch.full_like(w, 1e-5) for w in init)
    res = om.fused_chunk_ttt_step(tok, tok, tok, eta, torch.zeros_like(alpha), *init, *small,
                                  ln_w, ln_b, None, 1.0, 0.0, True, 1e-4)
    torch.testing.assert_close(res[1], init[0].float() + small[0].float(), atol=0, rtol=0)


def test_read_weights_change_only_the_readout():
    b, c, d, f = 1, 3, 4, 5
    ws = _weights(b, d, f)
    zero = tuple(torch.zeros_like(w) for w in ws)
    read = (ws[0] + torch.randn_like(ws[0]) * 0.1, ws[1], ws[2])
    q, k, v = (torch.randn(b, c, d, dtype=torch.float64) for _ in range(3))
    eta = torch.full((b, c, 1), 0.03, dtype=torch.float64)
    alpha = torch.full_like(eta, 0.01)
    ln = (torch.ones(d, dtype=torch.float64), torch.zeros(d, dtype=torch.float64))
    a = om.fused_chunk_ttt_step(q, k, v, eta, alpha, *ws, *zero, *ln, None, 0.9, 1.0, True, 1e-5, *read)
    o = om.fused_chunk_ttt_step(q, k, v, eta, alpha, *ws, *zero, *ln, None, 0.9, 1.0, True, 1e-5)
    torch.testing.assert_close(a[0], om.swiglu_fast_forward(q, *read, *ln, 1e-5), atol=1e-12, rtol=1e-10)
    assert not torch.allclose(a[0], o[0])
    for x, y in zip(a[1:], o[1:]):
        assert torch.equal(x, y)


def test_padding_does_not_decay_or_apply_momentum():
    """Padded tail tokens and fully masked rows are no-ops (test_reliability.py:192-207)."""
    d, f = 16, 32
    ws = _weights(2, d, f, dtype=torch.float32, scale=0.2)
    ms = (torch.full_like(ws[0], 0.1), torch.full_like(ws[1], 0.2), torch.full_like(ws[2], 0.3))
    q, k, v = (torch.randn(2, 4, d) for _ in range(3))
    eta, alpha = torch.rand(2, 4, 1) * 0.01, torch.rand(2, 4, 1) * 0.01
    mask = torch.tensor([[1, 1, 0, 0], [0, 0, 0, 0]], dtype=torch.float32)
    ln = (torch.ones(d), torch.zeros(d))
    pad = om.fused_chunk_ttt_step(q, k, v, eta, alpha, *ws, *ms, *ln, mask, 0.9, 1.0, False, 1e-5)
    cut = om.fused_chunk_ttt_step(q[:, :2], k[:, :2], v[:, :2], eta[:, :2], alpha[:, :2], *ws, *ms, *ln,
                                  mask[:, :2], 0.9, 1.0, False, 1e-5)
    for x, y, o in zip(pad[1:7], cut[1:7], ws + ms):
        torch.testing.assert_close(x[0], y[0])
        assert torch.equal(x[1], o[1])


def test_swiglu_readout_matches_scalar_loop():
    b, t, d, f = 2, 3, 4, 5
    x = torch.randn(b, t, d, dtype=torch.float64)
    wu, wg, wd = _weights(b, d, f)
    g, beta = torch.randn(d, dtype=torch.float64), torch.randn(d, dtype=torch.float64)
    got = om.swiglu_fast_forward(x, wu, wg, wd, g, beta, 1e-5)
    for r in range(b):
        for i in range(t):
            h = [0.0] * f
            for j in range(f):
                u = sum(float(x[r, i, a]) * float(wu[r, a, j]) for a in range(d))
                gg = sum(float(x[r, i, a]) * float(wg[r, a, j]) for a in range(d))
                h[j] = gg / (1.0 + math.exp(-gg)) * u
            z = [sum(h[j] * float(wd[r, j, a]) for j in range(f)) for a in range(d)]
            mu = sum(z) / d
            var = sum((zz - mu) ** 2 for zz in z) / d
            for a in range(d):
                want = float(x[r, i, a]) + (z[a] - mu) / math.sqrt(var + 1e-5) * float(g[a]) + float(beta[a])
                assert abs(float(got[r, i, a]) - want) < 1e-12


def test_sliding_window_attention_matches_scalar_loop():
    b, h, hkv, tq, tkv, hd, win = 1, 4, 2, 5, 9, 3, 3
    q = torch.randn(b, h, tq, hd, dtype=torch.float64)
    k = torch.randn(b, hkv, tkv, hd, dtype=torch.float64)
    v = torch.randn(b, hkv, tkv, hd, dtype=torch.float64)
    off = tkv - tq
    got = om.sliding_window_attention(q, k, v, win, off)
    for hh in range(h):
        kv = hh // (h // hkv)
        for i in range(tq):
            p = off + i
            keys = [j for j in range(tkv) if 0 <= p - j < win]
            s = [sum(float(q[0, hh, i, e]) * float(k[0, kv, j, e]) for e in range(hd)) / math.sqrt(hd) for j in keys]
            m = max(s)
            w = [math.exp(x - m) for x in s]
            tot = sum(w)
            for e in range(hd):
                want = sum(wi * float(v[0, kv, j, e]) for wi, j in zip(w, keys)) / tot
                assert abs(float(got[0, hh, i, e]) - want) < 1e-12


def test_attention_special_cases_window_one_and_full_causal():
    q = torch.randn(2, 4, 7, 8)
    k = torch.randn(2, 2, 7, 8)
    v = torch.randn(2, 2, 7, 8)
    self_only = om.sliding_window_attention(q, k, v, 1, 0)
    torch.testing.assert_close(self_only, v.repeat_interleave(2, dim=1))
    causal = om.sliding_window_attention(q, k, v, 64, 0)
    ref = F.scaled_dot_product_attention(q, k.repeat_interleave(2, 1), v.repeat_interleave(2, 1), is_causal=True)
    torch.testing.assert_close(causal, ref, atol=1e-6, rtol=1e-5)


def test_rope_is_a_rotation_with_relative_phase():
    hd = 8
    cos, sin = om.rope_tables(hd, 64)
    x = torch.randn(1, 1, 64, hd, dtype=torch.float64)
    rot = om.apply_rope(x, cos.double(), sin.double())
    # complex form: (x1 + i x2) * exp(i p theta_j) with theta_j = 10000^(-2j/hd)
    p = torch.arange(64, dtype=torch.float64).view(-1, 1)
    theta = 10000.0 ** (-torch.arange(0, hd, 2, dtype=torch.float64) / hd)
    z = torch.complex(x[0, 0, :, :hd // 2], x[0, 0, :, hd // 2:]) * torch.exp(1j * p * theta)
    torch.testing.assert_close(rot[0, 0, :, :hd // 2], z.real, atol=1e-5, rtol=1e-5)
    torch.testing.assert_close(rot[0, 0, :, hd // 2:], z.imag, atol=1e-5, rtol=1e-5)
    # q(p) . k(p') depends only on p - p'
    qv, kv = torch.randn(hd, dtype=torch.float64), torch.randn(hd, dtype=torch.float64)
    rq = om.apply_rope(qv.expand(1, 1, 64, hd), cos.double(), sin.double())[0, 0]
    rk = om.apply_rope(kv.expand(1, 1, 64, hd), cos.double(), sin.double())[0, 0]
    torch.testing.assert_close(rq[10] @ rk[7], rq[40] @ rk[37], atol=1e-5, rtol=1e-5)


def test_ring_decode_equals_full_prefix_attention():
    n, h, hkv, hd, win = 3, 4, 2, 8, 5
    steps = 13
    ks = torch.randn(n, hkv, steps, hd)
    vs = torch.randn(n, hkv, steps, hd)
    qs = torch.randn(n, h, steps, hd)
    k_ring = torch.zeros(n, hkv, win, hd)
    v_ring = torch.zeros(n, hkv, win, hd)
    starts = [0, 2, 4]
    for s in range(steps - max(starts)):
        pos = [st + s for st in starts]
        if s == 0:
            for r, p in enumerate(pos):  # pre-load earlier history into the ring
                for j in range(max(0, p - win + 1), p):
                    k_ring[r, :, j % win] = ks[r, :, j]
                    v_ring[r, :, j % win] = vs[r, :, j]
        q = torch.stack([qs[r, :, p] for r, p in enumerate(pos)])
        kn = torch.stack([ks[r, :, p] for r, p in enumerate(pos)])
        vn = torch.stack([vs[r, :, p] for r, p in enumerate(pos)])
        got = om.ring_decode_attention(q, kn, vn, k_ring, v_ring, pos, win)
        for r, p in enumerate(pos):
            want = om.sliding_window_attention(qs[r:r + 1, :, p:p + 1], ks[r:r + 1, :, :p + 1],
                                               vs[r:r + 1, :, :p + 1], win, p)
            torch.testing.assert_close(got[r], want[0, :, 0], atol=1e-6, rtol=1e-5)


def test_elastic_pull_closed_forms():
    w0 = tuple(torch.randn(*s) for s in ((4, 6), (4, 6), (6, 4)))
    w = tuple(b.unsqueeze(0).repeat(2, 1, 1) + torch.randn(2, *b.shape) for b in w0)
    full = om.apply_elastic_pull(w, w0, 1.0)
    for x, b in zip(full, w0):
        torch.testing.assert_close(x, b.unsqueeze(0).expand_as(x))
    assert om.apply_elastic_pull(w, w0, 0.0) is not None
    same = om.apply_elastic_pull(w, w0, 0.0, None)
    for x, y in zip(same, w):
        assert x is y
    ratio = 0.05
    capped = om.apply_elastic_pull(w, w0, 0.1, ratio)
    base = math.sqrt(sum(float(b.square().sum()) for b in w0))
    for r in range(2):
        drift = math.sqrt(sum(float((x[r] - b).square().sum()) for x, b in zip(capped, w0)))
        assert drift <= ratio * base * (1 + 1e-5)
    d = om.compute_drift(capped, w0)
    assert abs(d["base_frobenius"] - base) < 1e-4


def test_row_surprise_is_each_rows_batch1_surprise():
    """Per-row chunk surprise = the batch-global surprise (L:369-380) of that row alone,
    and = the masked mean of 0.5 |f_W(k) - v|^2 / d written as a per-token loop."""
    b, c, d, f = 3, 6, 8, 12
    k, v = torch.randn(b, c, d, dtype=torch.float64), torch.randn(b, c, d, dtype=torch.float64)
    ws = _weights(b, d, f)
    ln_w, ln_b = torch.randn(d, dtype=torch.float64), torch.randn(d, dtype=torch.float64)
    mask = torch.tensor([[1, 1, 1, 1, 1, 1], [1, 0, 1, 0, 0, 0], [0, 0, 0, 0, 0, 0]], dtype=torch.float64)
    eta = torch.full((b, c, 1), 0.01, dtype=torch.float64)
    rows = om.row_surprise(k, v, *ws, ln_w, ln_b, mask, True, 1e-5)
    for r in range(b):
        one = om.analytical_swiglu_chunk_grad(k[r:r + 1], v[r:r + 1], eta[r:r + 1], *(w[r:r + 1] for w in ws),
                                              ln_w, ln_b, mask[r:r + 1], True, 1e-5)[3]
        assert abs(float(rows[r]) - float(one)) < 1e-12
        pred = om.swiglu_fast_forward(k[r:r + 1], *(w[r:r + 1] for w in ws), ln_w, ln_b, 1e-5)[0]
        num = sum(0.5 * float((pred[t] - v[r, t]).square().sum()) / d * float(mask[r, t]) for t in range(c))
        assert abs(float(rows[r]) - num / max(1.0, float(mask[r].sum()))) < 1e-12
    assert float(rows[2]) == 0.0


def test_chunk_gate_keeps_rows_whose_surprise_is_below_threshold():
    """Rows under the per-chunk gate keep W and S bit for bit; rows over it take the
    ungated step; a zero threshold is the ungated step."""
    d, f = 16, 24
    ws = _weights(3, d, f, dtype=torch.float32, scale=0.2)
    ms = tuple(torch.randn_like(w) * 1e-3 for w in ws)
    q, k = torch.randn(3, 5, d), torch.randn(3, 5, d)
    v = torch.randn(3, 5, d) * torch.tensor([0.1, 1.0, 10.0]).view(3, 1, 1)  # row losses far apart
    eta, alpha = torch.rand(3, 5, 1) * 0.01, torch.rand(3, 5, 1) * 0.01
    ln = (torch.ones(d), torch.zeros(d))
    rows = om.row_surprise(k, v, *ws, *ln, None, True, 1e-5)
    assert rows[0] < rows[1] < rows[2]
    plain = om.fused_chunk_ttt_step(q, k, v, eta, alpha, *ws, *ms, *ln, None, 0.9, 1.0, True, 1e-5)
    zero = om.fused_chunk_ttt_step(q, k, v, eta, alpha, *ws, *ms, *ln, None, 0.9, 1.0, True, 1e-5,
                                   min_row_surprise=0.0)
    for x, y in zip(plain, zero):
        assert torch.equal(x, y)
    thr = float(rows[1] + rows[2]) / 2
    gated = om.fused_chunk_ttt_step(q, k, v, eta, alpha, *ws, *ms, *ln, None, 0.9, 1.0, True, 1e-5,
                                    min_row_surprise=thr)
    for x, p, o in zip(gated[1:7], plain[1:7], ws + ms):
        assert torch.equal(x[0], o[0]) and torch.equal(x[1], o[1])
        assert torch.equal(x[2], p[2])
    torch.testing.assert_close(gated[0], plain[0])  # the readout is the same either way
