"""GPU parity of the HIP kernels against the CPU oracle (same seeded inputs).

Tolerances (north star): fp32 paths <= 1e-5 relative error, measured as
max|gpu - oracle| / max|oracle| per tensor; updated fp32 fast weights from bf16
activations <= 2e-2 max-abs against the fp32 oracle.  bf16 *activations* (readouts)
are stored with an 8-bit mantissa, so one unit in the last place at |x| in [4, 8) is
already 0.031: they must satisfy |gpu - fp32| <= 2e-2 + 2^-7 |fp32| elementwise AND be
no less accurate than the reference's own bf16 arithmetic (the oracle run on bf16
inputs, which rounds u, g, h, z to bf16 as the reference does):
max|gpu - fp32| <= 1.5 max|ref_bf16 - fp32| + 1e-3.  RoPE is bit-exact (the kernel
reproduces the reference's operation order and rounding).
"""
import math

import pytest
import torch

from oracle import uttt_math as om

pytestmark = pytest.mark.gpu
DEV = "cuda"
F32_REL = 1e-5
BF16_ABS = 2e-2


def rel_err(actual, expected):
    actual = actual.detach().double().cpu()
    expected = expected.detach().double().cpu()
    scale = expected.abs().max().item()
    return (actual - expected).abs().max().item() / max(scale, 1e-30)


def max_abs(actual, expected):
    return (actual.detach().double().cpu() - expected.detach().double().cpu()).abs().max().item()


def check_bf16_activation(name, got, fp32_ref, bf16_ref):
    got, fp32_ref, bf16_ref = (t.detach().double().cpu() for t in (got, fp32_ref, bf16_ref))
    diff = (got - fp32_ref).abs()
    bound = 2e-2 + 2.0 ** -7 * fp32_ref.abs()
    worst = (diff - bound).max().item()
    assert worst <= 0, f"{name}: exceeds 2e-2 + 2^-7|x| by {worst:.3e}"
    ours, theirs = diff.max().item(), (bf16_ref - fp32_ref).abs().max().item()
    assert ours <= 1.5 * theirs + 1e-3, f"{name}: max err {ours:.3e} vs reference-bf16 {theirs:.3e}"


def kernels():
    from utttcompanion_amd import kernels as K
    return K


def make_chunk(b, c, d, f, seed, scale_w=None):
    g = torch.Generator().manual_seed(seed)
    sw = scale_w if scale_w is not None else 1.0 / math.sqrt(d)
    q, k, v = (torch.randn(b, c, d, generator=g) for _ in range(3))
    eta = 0.01 * torch.sigmoid(torch.randn(b, c, 1, generator=g))
    alpha = 0.005 * torch.sigmoid(torch.randn(b, c, 1, generator=g) - 1.386)
    w = (torch.randn(b, d, f, generator=g) * sw, torch.randn(b, d, f, generator=g) * sw,
         torch.randn(b, f, d, generator=g) * 0.1 / math.sqrt(f))
    s = tuple(torch.randn(t.shape, generator=g) * 1e-3 for t in w)
    ln_w = 1.0 + 0.1 * torch.randn(d, generator=g)
    ln_b = 0.05 * torch.randn(d, generator=g)
    return q, k, v, eta, alpha, w, s, ln_w, ln_b


def to_dev(*ts):
    return [t.to(DEV) if t is not None else None for t in ts]


@pytest.mark.parametrize("case", [
    dict(b=1, c=64, d=512, f=1024, mask=False, read=False, clip=1.0, norm=True),   # config-1 chunk shape
    dict(b=2, c=40, d=128, f=256, mask=True, read=True, clip=1.0, norm=True),     # tail chunk, mask, snapshot
    dict(b=3, c=64, d=192, f=320, mask=True, read=False, clip=0.0, norm=False),   # no clip, 1/1 scale
    dict(b=2, c=64, d=64, f=128, mask=False, read=True, clip=1e-4, norm=True),    # clip active
])
def test_chunk_update_fp32_matches_oracle(case):
    K = kernels()
    b, c, d, f = case["b"], case["c"], case["d"], case["f"]
    print(f"case {case}", flush=True)
    q, k, v, eta, alpha, w, s, ln_w, ln_b = make_chunk(b, c, d, f, seed=11 + b + c)
    mask = None
    if case["mask"]:
        mask = torch.ones(b, c)
        mask[0, c // 2:] = 0
        if b > 2:
            mask[2] = 0  # a row with no valid token keeps W and S
    read = None
    if case["read"]:
        read = tuple(t + 0.01 * torch.randn_like(t) for t in w)
    ref = om.fused_chunk_ttt_step(q, k, v, eta, alpha, *w, *s, ln_w, ln_b, mask, 0.9, case["clip"], case["norm"],
                                  1e-5, *(read if read else (None, None, None)))
    dev_in = to_dev(q, k, v, eta, alpha, *w, *s, ln_w, ln_b, mask)
    dev_read = to_dev(*read) if read else (None, None, None)
    with torch.no_grad():
        got = K.chunk_update(*dev_in[:13], dev_in[13], 0.9, case["clip"], case["norm"], 1e-5, *dev_read)
    torch.cuda.synchronize()
    names = ("readout", "w_up", "w_gate", "w_down", "s_up", "s_gate", "s_down", "surprise")
    for name, a, e in zip(names, got, ref):
        err = rel_err(a, e)
        assert err <= F32_REL, f"{name}: rel err {err:.3e}"
    if case["mask"] and b > 2:
        for a, o in zip(got[1:7], w + s):
            assert torch.equal(a[2].cpu(), o[2]), "inactive row changed"


def test_chunk_update_fp32_sixteen_chunks_config1():
    """Config 1: B=1, T=1024 as 16 sequential chunks; each chunk reads its pre-update W."""
    K = kernels()
    b, d, f, T = 1, 512, 1024, 1024
    q, k, v, eta, alpha, w, s, ln_w, ln_b = make_chunk(b, T, d, f, seed=5, scale_w=0.02)
    s = tuple(torch.zeros_like(t) for t in w)
    ref_w, ref_s, ref_outs = w, s, []
    dev = to_dev(q, k, v, eta, alpha, ln_w, ln_b)
    cur = to_dev(*w, *s)
    outs, surprises = [], []
    with torch.no_grad():
        for i in range(T // 64):
            sl = slice(64 * i, 64 * (i + 1))
            r = om.fused_chunk_ttt_step(q[:, sl], k[:, sl], v[:, sl], eta[:, sl], alpha[:, sl], *ref_w, *ref_s,
                                        ln_w, ln_b, None, 0.9, 1.0, True, 1e-5)
            ref_outs.append(r[0])
            ref_w, ref_s = r[1:4], r[4:7]
            g = K.chunk_update(dev[0][:, sl], dev[1][:, sl], dev[2][:, sl], dev[3][:, sl], dev[4][:, sl], *cur,
                               dev[5], dev[6], None, 0.9, 1.0, True, 1e-5)
            outs.append(g[0])
            surprises.append(g[7])
            cur = list(g[1:7])
    torch.cuda.synchronize()
    assert rel_err(torch.cat(outs, 1), torch.cat(ref_outs, 1)) <= F32_REL
    for a, e in zip(cur, ref_w + ref_s):
        assert rel_err(a, e) <= F32_REL


def test_chunk_update_in_place_equals_out_of_place():
    K = kernels()
    q, k, v, eta, alpha, w, s, ln_w, ln_b = make_chunk(2, 64, 128, 192, seed=3)
    dev = to_dev(q, k, v, eta, alpha, *w, *s, ln_w, ln_b)
    with torch.no_grad():
        fresh = K.chunk_update(*dev[:13], None, 0.9, 1.0, True, 1e-5)
        state = [t.clone() for t in dev[5:11]]
        inplace = K.chunk_update(*dev[:5], *state, *dev[11:13], None, 0.9, 1.0, True, 1e-5, out_state=state)
    torch.cuda.synchronize()
    for a, e in zip(inplace[:7], fresh[:7]):
        assert torch.equal(a, e)
    assert inplace[1].data_ptr() == state[0].data_ptr()


@pytest.mark.parametrize("b,c,d,f", [(1, 64, 512, 1024), (2, 64, 768, 2048), (2, 37, 256, 512)])
def test_chunk_update_bf16_within_tolerance_of_fp32_oracle(b, c, d, f):
    K = kernels()
    print(f"bf16 chunk b={b} c={c} d={d} f={f}", flush=True)
    q, k, v, eta, alpha, w, s, ln_w, ln_b = make_chunk(b, c, d, f, seed=17 + d)
    q16, k16, v16, e16, a16 = (t.bfloat16() for t in (q, k, v, eta, alpha))
    ref = om.fused_chunk_ttt_step(q16.float(), k16.float(), v16.float(), e16.float(), a16.float(), *w, *s,
                                  ln_w, ln_b, None, 0.9, 1.0, True, 1e-5)
    ref16 = om.fused_chunk_ttt_step(q16, k16, v16, e16, a16, *w, *s, ln_w, ln_b, None, 0.9, 1.0, True, 1e-5)
    with torch.no_grad():
        got = K.chunk_update(*to_dev(q16, k16, v16, e16, a16, *w, *s, ln_w, ln_b), None, 0.9, 1.0, True, 1e-5)
    torch.cuda.synchronize()
    assert got[0].dtype == torch.bfloat16 and got[1].dtype == torch.float32
    check_bf16_activation("readout", got[0], ref[0], ref16[0])
    for name, a, e in zip(("w_up", "w_gate", "w_down", "s_up", "s_gate", "s_down"), got[1:7], ref[1:7]):
        err = max_abs(a, e)
        assert err <= BF16_ABS, f"{name}: max abs {err:.3e}"
    assert abs(got[7].item() - ref[7].item()) <= 2e-2 * max(1.0, abs(ref[7].item()))


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("shared", [False, True])
def test_swiglu_readout_matches_oracle(dtype, shared):
    K = kernels()
    b, t, d, f = 3, 150, 256, 512
    g = torch.Generator().manual_seed(23)
    x = torch.randn(b, t, d, generator=g).to(dtype)
    wb = 1 if shared else b
    w = (torch.randn(wb, d, f, generator=g) / 16, torch.randn(wb, d, f, generator=g) / 16,
         torch.randn(wb, f, d, generator=g) / 64)
    ln_w, ln_b = 1 + 0.1 * torch.randn(d, generator=g), 0.1 * torch.randn(d, generator=g)
    ref = om.swiglu_fast_forward(x.float(), *(t_.expand(b, -1, -1) for t_ in w), ln_w, ln_b, 1e-5)
    with torch.no_grad():
        got = K.swiglu_readout(*to_dev(x, *(t_.expand(b, -1, -1) for t_ in w), ln_w, ln_b), eps=1e-5)
    torch.cuda.synchronize()
    if dtype == torch.float32:
        assert rel_err(got, ref) <= F32_REL
    else:
        ref16 = om.swiglu_fast_forward(x, *(t_.expand(b, -1, -1) for t_ in w), ln_w, ln_b, 1e-5)
        check_bf16_activation("readout", got, ref, ref16)


def test_swiglu_readout_with_bf16_weight_copies():
    """bf16 read copies of W give the operands the fp32 path rounds to (same readout)."""
    K = kernels()
    b, t, d, f = 4, 1, 768, 2048
    g = torch.Generator().manual_seed(27)
    x = torch.randn(b, t, d, generator=g).bfloat16()
    w = (torch.randn(b, d, f, generator=g) * 0.03, torch.randn(b, d, f, generator=g) * 0.03,
         torch.randn(b, f, d, generator=g) * 0.02)
    ln_w, ln_b = 1 + 0.1 * torch.randn(d, generator=g), 0.1 * torch.randn(d, generator=g)
    with torch.no_grad():
        from_f32 = K.swiglu_readout(*to_dev(x, *w, ln_w, ln_b))
        from_bf16 = K.swiglu_readout(*to_dev(x, *(t_.bfloat16() for t_ in w), ln_w, ln_b))
    torch.cuda.synchronize()
    assert torch.equal(from_f32, from_bf16)
    ref = om.swiglu_fast_forward(x.float(), *(t_.bfloat16().float() for t_ in w), ln_w, ln_b, 1e-5)
    ref16 = om.swiglu_fast_forward(x, *w, ln_w, ln_b, 1e-5)
    check_bf16_activation("readout", from_bf16, ref, ref16)


@pytest.mark.parametrize("b,d,f", [(32, 768, 2048), (5, 512, 1024), (3, 1536, 640), (3, 576, 640)])
def test_decode_readout_with_query_norm_in_one_launch(b, d, f):
    """One token per row: the readout of RMSNorm(y) (q_norm folded into the readout's x staging)
    equals the readout of torch's normalised rows to the bf16 readout bound, and the one-launch
    form (row counters: LayerNorm in each row's last weight block) equals the two-launch form
    bit for bit on two calls in a row; the counters are zero again after each call.  The
    descending weight walk (``sweep_reverse``) meets the same bound, in both forms, and repeats
    bit for bit (576 x 640 leaves partial row batches in both weight loops)."""
    import torch.nn.functional as F
    K = kernels()
    g = torch.Generator().manual_seed(b + d + f)
    eps = 1e-5
    w = [(torch.randn(b, d, f, generator=g) * 0.03).bfloat16(), (torch.randn(b, d, f, generator=g) * 0.03).bfloat16(),
         (torch.randn(b, f, d, generator=g) * 0.02).bfloat16()]
    ln_w, ln_b = 1 + 0.1 * torch.randn(d, generator=g), 0.1 * torch.randn(d, generator=g)
    qw = (1 + 0.1 * torch.randn(d, generator=g)).bfloat16()
    dw = to_dev(*w, ln_w, ln_b, qw)
    counters = torch.zeros(b, dtype=torch.int32, device=DEV)
    for call in range(2):
        y = (2.0 * torch.randn(b, 1, d, generator=g)).bfloat16()
        yd = y.to(DEV)
        with torch.no_grad():
            two = K.swiglu_readout(yd, *dw[:5], eps=1e-5, x_norm=(dw[5], eps))
            one = K.swiglu_readout(yd, *dw[:5], eps=1e-5, x_norm=(dw[5], eps), row_counters=counters)
            plain = K.swiglu_readout(F.rms_norm(yd, (d,), dw[5], eps), *dw[:5], eps=1e-5)
            rev_one = K.swiglu_readout(yd, *dw[:5], eps=1e-5, x_norm=(dw[5], eps), row_counters=counters,
                                       sweep_reverse=True)
            rev_two = K.swiglu_readout(yd, *dw[:5], eps=1e-5, x_norm=(dw[5], eps), sweep_reverse=True)
            rev_again = K.swiglu_readout(yd, *dw[:5], eps=1e-5, x_norm=(dw[5], eps), row_counters=counters,
                                         sweep_reverse=True)
        torch.cuda.synchronize()
        assert torch.equal(one, two), call
        assert torch.equal(rev_one, rev_two) and torch.equal(rev_one, rev_again), call
        assert counters.abs().sum().item() == 0
        yf = y.float()
        xn = (yf * torch.rsqrt(yf.pow(2).mean(-1, keepdim=True) + eps) * qw.float()).bfloat16()
        ref = om.swiglu_fast_forward(xn.float(), *(t_.float() for t_ in w), ln_w, ln_b, 1e-5)
        ref16 = om.swiglu_fast_forward(xn, *w, ln_w, ln_b, 1e-5)
        check_bf16_activation("fused readout", one, ref, ref16)
        check_bf16_activation("plain readout", plain, ref, ref16)
        check_bf16_activation("reversed readout", rev_one, ref, ref16)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_rope_append_is_bit_exact(dtype):
    K = kernels()
    b, t, h, hkv, hd = 2, 7, 4, 2, 64
    g = torch.Generator().manual_seed(29)
    q = torch.randn(b, t, h, hd, generator=g).to(dtype)
    k = torch.randn(b, t, hkv, hd, generator=g).to(dtype)
    v = torch.randn(b, t, hkv, hd, generator=g).to(dtype)
    cos, sin = om.rope_tables(hd, 64)
    start = 9
    ref_q = om.apply_rope(q.transpose(1, 2), cos[start:start + t], sin[start:start + t])
    ref_k = om.apply_rope(k.transpose(1, 2), cos[start:start + t], sin[start:start + t])
    dq, dk, dv, dcos, dsin = to_dev(q.clone(), k, v, cos, sin)
    kc = torch.zeros(b, hkv, 20, hd, dtype=dtype, device=DEV)
    vc = torch.zeros_like(kc)
    K.rope_kv_append(dq, dk, dv, dcos, dsin, start, kc, vc, 5)
    torch.cuda.synchronize()
    assert torch.equal(dq.transpose(1, 2).cpu(), ref_q)
    assert torch.equal(kc[:, :, 5:5 + t].cpu(), ref_k)
    assert torch.equal(vc[:, :, 5:5 + t].cpu(), v.transpose(1, 2))
    assert kc[:, :, :5].abs().sum().item() == 0 and kc[:, :, 5 + t:].abs().sum().item() == 0


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_rope_append_folded_norm(dtype):
    """With the projection input x given, q / k / v of token t are scaled by
    1 / sqrt(mean(x_t^2) + eps) before RoPE (the input RMSNorm folded into the projection):
    against the oracle's RoPE of the scaled values, fp32 <= 1e-5 relative, bf16 within two bf16
    roundings (2^-7) of the largest magnitude."""
    K = kernels()
    b, t, h, hkv, hd, d = 2, 5, 4, 2, 64, 96
    g = torch.Generator().manual_seed(31)
    q = torch.randn(b, t, h, hd, generator=g).to(dtype)
    k = torch.randn(b, t, hkv, hd, generator=g).to(dtype)
    v = torch.randn(b, t, hkv, hd, generator=g).to(dtype)
    x = (torch.randn(b, t, d, generator=g) * torch.tensor([0.3, 3.0]).view(2, 1, 1)).to(dtype)
    cos, sin = om.rope_tables(hd, 64)
    start = 3
    rstd = 1.0 / torch.sqrt(x.float().pow(2).mean(-1) + 1e-5)  # (b, t)
    qs, ks, vs = (z.float() * rstd[:, :, None, None] for z in (q, k, v))
    ref_q = om.apply_rope(qs.transpose(1, 2), cos[start:start + t], sin[start:start + t])
    ref_k = om.apply_rope(ks.transpose(1, 2), cos[start:start + t], sin[start:start + t])
    dq, dk, dv, dcos, dsin, dx = to_dev(q.clone(), k, v, cos, sin, x)
    kc = torch.zeros(b, hkv, 12, hd, dtype=dtype, device=DEV)
    vc = torch.zeros_like(kc)
    K.rope_kv_append(dq, dk, dv, dcos, dsin, start, kc, vc, 2, x=dx, x_eps=1e-5)
    torch.cuda.synchronize()
    tol = 1e-5 if dtype == torch.float32 else 2.0 ** -7
    for got, ref in ((dq.transpose(1, 2).cpu(), ref_q), (kc[:, :, 2:2 + t].cpu(), ref_k),
                     (vc[:, :, 2:2 + t].cpu(), vs.transpose(1, 2))):
        err = (got.float() - ref.float()).abs().max().item() / ref.float().abs().max().item()
        assert err <= tol, f"rel err {err:.3e}"
    assert kc[:, :, :2].abs().sum().item() == 0 and kc[:, :, 2 + t:].abs().sum().item() == 0
    with pytest.raises(ValueError):
        K.rope_kv_append(dq, dk, dv, dcos, dsin, start, kc, vc, 2, x=dx, x_eps=0.0)


@pytest.mark.parametrize("case", [
    dict(b=2, h=12, hkv=4, tq=300, tkv=300, hd=64, win=128),     # multi-tile window, ragged tail
    dict(b=1, h=4, hkv=4, tq=64, tkv=575, hd=64, win=512),       # chunk step over a cache (C2 shape)
    dict(b=1, h=16, hkv=4, tq=130, tkv=400, hd=128, win=1024),   # hd 128, window > kv (causal)
    dict(b=2, h=4, hkv=1, tq=70, tkv=70, hd=64, win=1),          # window 1: self only
    dict(b=4, h=8, hkv=4, tq=1024, tkv=1024, hd=64, win=256),    # config-1 attention: no key split
])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_swa_prefill_matches_oracle(case, dtype):
    K = kernels()
    print(f"swa prefill {case} {dtype}", flush=True)
    g = torch.Generator().manual_seed(31)
    b, h, hkv, tq, tkv, hd, win = (case[k] for k in ("b", "h", "hkv", "tq", "tkv", "hd", "win"))
    q = torch.randn(b, tq, h, hd, generator=g).to(dtype).transpose(1, 2)
    k = torch.randn(b, hkv, tkv, hd, generator=g).to(dtype)
    v = torch.randn(b, hkv, tkv, hd, generator=g).to(dtype)
    off = tkv - tq
    ref = om.sliding_window_attention(q.float(), k.float(), v.float(), win, off)
    with torch.no_grad():
        got = K.swa_prefill(*to_dev(q, k, v), win, off)
    torch.cuda.synchronize()
    if dtype == torch.float32:
        assert rel_err(got, ref) <= F32_REL
    else:
        assert max_abs(got, ref) <= BF16_ABS


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_swa_prefill_ignores_stale_workspace_contents(dtype):
    """Splits with no visible key leave their partial rows unwritten; partial rows full of
    NaN (reused memory) must not leak into the output.  Single-query steps exercise it."""
    K = kernels()
    g = torch.Generator().manual_seed(41)
    for tkv, win in ((21, 24), (70, 8), (300, 128)):
        q = torch.randn(1, 1, 2, 64, generator=g).to(dtype).transpose(1, 2)
        k = torch.randn(1, 1, tkv, 64, generator=g).to(dtype)
        v = torch.randn(1, 1, tkv, 64, generator=g).to(dtype)
        ref = om.sliding_window_attention(q.float(), k.float(), v.float(), win, tkv - 1)
        ws = torch.full((1 << 22,), float("nan"), device=DEV).view(torch.uint8)
        with torch.no_grad():
            got = K.swa_prefill(*to_dev(q, k, v), win, tkv - 1, workspace=ws)
        torch.cuda.synchronize()
        assert torch.isfinite(got).all(), (tkv, win)
        tol = F32_REL if dtype == torch.float32 else BF16_ABS
        err = rel_err(got, ref) if dtype == torch.float32 else max_abs(got, ref)
        assert err <= tol, (tkv, win, err)


def test_swa_prefill_one_workspace_serves_every_shape():
    """Calls of different shapes, one after another, sharing one workspace (as the default
    per-device workspace and the chunk executor's are shared; the split count, and with it the
    partials' layout, changes with the keys in range): each matches its own fresh-workspace
    result exactly."""
    K = kernels()
    g = torch.Generator().manual_seed(43)
    ws = torch.zeros(1 << 24, dtype=torch.uint8, device=DEV)
    for b, h, hkv, tq, tkv, hd, win in ((2, 12, 4, 300, 300, 64, 128), (1, 4, 4, 64, 575, 64, 512),
                                        (1, 16, 4, 130, 400, 128, 1024), (4, 16, 4, 64, 1088, 128, 1024),
                                        (1, 4, 4, 64, 575, 64, 512)):
        q = torch.randn(b, tq, h, hd, generator=g).bfloat16().transpose(1, 2)
        k = torch.randn(b, hkv, tkv, hd, generator=g).bfloat16()
        v = torch.randn(b, hkv, tkv, hd, generator=g).bfloat16()
        with torch.no_grad():
            shared = K.swa_prefill(*to_dev(q, k, v), win, tkv - tq, workspace=ws)
            fresh = K.swa_prefill(*to_dev(q, k, v), win, tkv - tq,
                                  workspace=torch.zeros(1 << 24, dtype=torch.uint8, device=DEV))
        torch.cuda.synchronize()
        assert torch.equal(shared, fresh), (b, h, tq, tkv)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("hd", [64, 128])
def test_swa_decode_ring_matches_full_prefix(dtype, hd):
    """Ragged positions, several window wraps; RoPE applied inside the kernel."""
    K = kernels()
    n, h, hkv, win, steps = 5, 12, 4, 16, 40
    g = torch.Generator().manual_seed(37)
    starts = [0, 3, 15, 16, 33]
    total = max(starts) + steps
    qs = torch.randn(n, total, h, hd, generator=g).to(dtype)
    ks = torch.randn(n, total, hkv, hd, generator=g).to(dtype)
    vs = torch.randn(n, total, hkv, hd, generator=g).to(dtype)
    cos, sin = om.rope_tables(hd, 256)
    rq = om.apply_rope(qs.transpose(1, 2), cos[:total], sin[:total])  # (n, h, total, hd)
    rk = om.apply_rope(ks.transpose(1, 2), cos[:total], sin[:total])
    rv = vs.transpose(1, 2)
    k_ring = torch.zeros(n, hkv, win, hd, dtype=dtype)
    v_ring = torch.zeros_like(k_ring)
    for r, p0 in enumerate(starts):  # history before the first step, already rotated
        for j in range(max(0, p0 - win), p0):
            k_ring[r, :, j % win] = rk[r, :, j]
            v_ring[r, :, j % win] = rv[r, :, j]
    dk_ring, dv_ring, dcos, dsin = to_dev(k_ring, v_ring, cos, sin)
    with torch.no_grad():
        for step in range(steps):
            pos = [p0 + step for p0 in starts]
            q = torch.stack([qs[r, p] for r, p in enumerate(pos)])
            kn = torch.stack([ks[r, p] for r, p in enumerate(pos)])
            vn = torch.stack([vs[r, p] for r, p in enumerate(pos)])
            positions = torch.tensor(pos, dtype=torch.int64, device=DEV)
            got = K.swa_decode(*to_dev(q, kn, vn), dk_ring, dv_ring, positions, dcos, dsin)
            for r, p in enumerate(pos):
                want = om.sliding_window_attention(rq[r:r + 1, :, p:p + 1].float(), rk[r:r + 1, :, :p + 1].float(),
                                                   rv[r:r + 1, :, :p + 1].float(), win, p)[0, :, 0]
                a = got[r].float().cpu()
                if dtype == torch.float32:
                    assert rel_err(a, want) <= F32_REL, f"step {step} req {r}"
                else:
                    assert max_abs(a, want) <= BF16_ABS, f"step {step} req {r}"
    torch.cuda.synchronize()


@pytest.mark.parametrize("win,hkv", [(512, 4), (300, 4), (512, 3)])
def test_swa_decode_wide_windows_bf16(win, hkv):
    """bf16 head_dim 64 at the decode shapes: windows up to 512 with at most 4 query heads per kv
    head run as one workgroup per (request, kv head); 5 query heads per kv head take the split
    form.  Positions before, at and well past the first wrap; one step each."""
    K = kernels()
    hd = 64
    h = 12 if hkv != 3 else 15
    pos = [0, 37, win - 1, win, 3 * win + 5]
    n = len(pos)
    g = torch.Generator().manual_seed(win + hkv)
    total = max(pos) + 1
    qs = torch.randn(n, total, h, hd, generator=g).bfloat16()
    ks = torch.randn(n, total, hkv, hd, generator=g).bfloat16()
    vs = torch.randn(n, total, hkv, hd, generator=g).bfloat16()
    cos, sin = om.rope_tables(hd, total)
    rq = om.apply_rope(qs.transpose(1, 2), cos, sin)
    rk = om.apply_rope(ks.transpose(1, 2), cos, sin)
    rv = vs.transpose(1, 2)
    k_ring = torch.randn(n, hkv, win, hd, generator=g).bfloat16()  # stale slots must not be read
    v_ring = torch.randn(n, hkv, win, hd, generator=g).bfloat16()
    for r, p in enumerate(pos):
        for j in range(max(0, p - win + 1), p):
            k_ring[r, :, j % win] = rk[r, :, j]
            v_ring[r, :, j % win] = rv[r, :, j]
    q = torch.stack([qs[r, p] for r, p in enumerate(pos)])
    kn = torch.stack([ks[r, p] for r, p in enumerate(pos)])
    vn = torch.stack([vs[r, p] for r, p in enumerate(pos)])
    dk, dv = to_dev(k_ring, v_ring)
    with torch.no_grad():
        got = K.swa_decode(*to_dev(q, kn, vn), dk, dv, torch.tensor(pos, dtype=torch.int64, device=DEV),
                           *to_dev(cos, sin))
    torch.cuda.synchronize()
    for r, p in enumerate(pos):
        want = om.sliding_window_attention(rq[r:r + 1, :, p:p + 1].float(), rk[r:r + 1, :, :p + 1].float(),
                                           rv[r:r + 1, :, :p + 1].float(), win, p)[0, :, 0]
        assert max_abs(got[r].float().cpu(), want) <= BF16_ABS, f"request {r} at {p}"
        assert torch.equal(dk[r, :, p % win].cpu(), rk[r, :, p]), "the new key goes to slot pos mod window"


def test_swa_decode_nan_slots_and_bad_position_bf16():
    """Ring slots that are not yet valid hold NaN (the kernel reads whole pieces before it knows
    the position, so their value rows must not reach the output), and a position past the RoPE
    table gives a NaN output with that request's ring untouched while the others decode."""
    K = kernels()
    hd, h, hkv, win = 64, 12, 4, 512
    pos = [0, 5, 130, 300]
    n = len(pos)
    total = 512
    g = torch.Generator().manual_seed(11)
    qs = torch.randn(n, total, h, hd, generator=g).bfloat16()
    ks = torch.randn(n, total, hkv, hd, generator=g).bfloat16()
    vs = torch.randn(n, total, hkv, hd, generator=g).bfloat16()
    cos, sin = om.rope_tables(hd, total)
    rq = om.apply_rope(qs.transpose(1, 2), cos, sin)
    rk = om.apply_rope(ks.transpose(1, 2), cos, sin)
    rv = vs.transpose(1, 2)
    k_ring = torch.full((n, hkv, win, hd), float("nan")).bfloat16()
    v_ring = torch.full((n, hkv, win, hd), float("nan")).bfloat16()
    for r, p in enumerate(pos):
        for j in range(p):
            k_ring[r, :, j] = rk[r, :, j]
            v_ring[r, :, j] = rv[r, :, j]
    q = torch.stack([qs[r, p] for r, p in enumerate(pos)])
    kn = torch.stack([ks[r, p] for r, p in enumerate(pos)])
    vn = torch.stack([vs[r, p] for r, p in enumerate(pos)])
    bad = 2
    run_pos = list(pos)
    run_pos[bad] = total  # one past the table
    dk, dv = to_dev(k_ring, v_ring)
    with torch.no_grad():
        got = K.swa_decode(*to_dev(q, kn, vn), dk, dv, torch.tensor(run_pos, dtype=torch.int64, device=DEV),
                           *to_dev(cos, sin))
    torch.cuda.synchronize()
    for r, p in enumerate(pos):
        if r == bad:
            assert torch.isnan(got[r].float()).all(), "a position past the RoPE table must give NaN"
            assert torch.equal(dk[r].cpu().nan_to_num(7.0), k_ring[r].nan_to_num(7.0)), "ring must stay untouched"
            assert torch.equal(dv[r].cpu().nan_to_num(7.0), v_ring[r].nan_to_num(7.0)), "ring must stay untouched"
            continue
        want = om.sliding_window_attention(rq[r:r + 1, :, p:p + 1].float(), rk[r:r + 1, :, :p + 1].float(),
                                           rv[r:r + 1, :, :p + 1].float(), win, p)[0, :, 0]
        out = got[r].float().cpu()
        assert torch.isfinite(out).all(), f"request {r} at {p}: a stale NaN slot reached the output"
        assert max_abs(out, want) <= BF16_ABS, f"request {r} at {p}"


def padded(t):
    """t (..., n) as a view of a buffer whose rows are padded to a whole number of 16-byte
    vectors: the form the one-wave-per-row epilogue (16-byte accesses) takes."""
    vec = 16 // t.element_size()
    n = t.shape[-1]
    buf = torch.full((*t.shape[:-1], (n + vec - 1) // vec * vec), float("nan"), dtype=t.dtype, device=t.device)
    buf[..., :n] = t
    return buf[..., :n]


@pytest.mark.parametrize("layout", ["packed", "padded"])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_proj_epilogue_matches_oracle(dtype, layout):
    """q/k/v RMSNorm and eta/alpha sigmoid of the packed projection (reference
    fused_slow_projections, model/uttt_layer.py:1193-1231) against the oracle's ops in fp32:
    fp32 <= 1e-6 relative; bf16 within one bf16 rounding of the fp32 result (2^-8 relative).
    ``padded`` rows (16-byte multiples, NaN past the row) take the one-wave-per-row kernel."""
    K = kernels()
    g = torch.Generator().manual_seed(17)
    rows, d = 37, 192
    y = torch.randn(2, rows, 3 * d + 2, generator=g) * 3.0
    qw, kw = 1.0 + 0.2 * torch.randn(d, generator=g), 1.0 + 0.2 * torch.randn(d, generator=g)
    y_in = y.to(dtype)
    yf = y_in.float()
    ref = (om.rms_norm(yf[..., :d], qw.to(dtype).float(), 1e-5), om.rms_norm(yf[..., d:2 * d], kw.to(dtype).float(), 1e-5),
           om.rms_norm(yf[..., 2 * d:3 * d], None, 1e-5), 0.01 * torch.sigmoid(yf[..., 3 * d:3 * d + 1]),
           0.005 * torch.sigmoid(yf[..., 3 * d + 1:]))
    with torch.no_grad():
        y_dev = y_in.to(DEV)
        if layout == "padded":
            y_dev = padded(y_dev)
        got = K.proj_epilogue(y_dev, d, qw.to(DEV, dtype), kw.to(DEV, dtype), 1e-5, 0.01, 0.005)
    for name, a, e in zip(("q", "k", "v", "eta", "alpha"), got, ref):
        assert a.shape == e.shape and a.dtype == dtype, name
        err = ((a.float().cpu() - e).abs() / e.abs().clamp_min(1e-6)).max().item()
        assert err <= (1e-6 if dtype == torch.float32 else 2.0 ** -8), f"{name}: rel err {err:.3e}"


@pytest.mark.parametrize("layout", ["packed", "padded"])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_proj_epilogue_folded_norm(dtype, layout):
    """With the GEMM input x given, y's rows are scaled by 1 / sqrt(mean(x^2) + eps) and the eta /
    alpha biases added before the q/k/v RMSNorm and the sigmoids: against the same steps in fp32
    from the same (rounded) y, fp32 <= 1e-5 relative, bf16 within 2^-7 relative."""
    K = kernels()
    g = torch.Generator().manual_seed(23)
    rows, d = 29, 128
    x = (torch.randn(rows, d, generator=g) * 2.0).to(dtype)
    y = (torch.randn(rows, 3 * d + 2, generator=g) * 3.0).to(dtype)
    qw, kw = 1.0 + 0.2 * torch.randn(d, generator=g), 1.0 + 0.2 * torch.randn(d, generator=g)
    bias = torch.tensor([0.3, -1.386]).to(dtype)
    rstd = 1.0 / torch.sqrt(x.float().pow(2).mean(-1, keepdim=True) + 1e-5)
    yf = y.float() * rstd
    yf[:, 3 * d] += bias[0].float()
    yf[:, 3 * d + 1] += bias[1].float()
    ref = (om.rms_norm(yf[:, :d], qw.to(dtype).float(), 1e-5), om.rms_norm(yf[:, d:2 * d], kw.to(dtype).float(), 1e-5),
           om.rms_norm(yf[:, 2 * d:3 * d], None, 1e-5), 0.01 * torch.sigmoid(yf[:, 3 * d:3 * d + 1]),
           0.005 * torch.sigmoid(yf[:, 3 * d + 1:]))
    with torch.no_grad():
        y_dev = y.to(DEV) if layout == "packed" else padded(y.to(DEV))
        got = K.proj_epilogue(y_dev, d, qw.to(DEV, dtype), kw.to(DEV, dtype), 1e-5, 0.01, 0.005,
                              x=x.to(DEV), x_eps=1e-5, eta_alpha_bias=bias.to(DEV))
    tol = 1e-5 if dtype == torch.float32 else 2.0 ** -7
    for name, a, e in zip(("q", "k", "v", "eta", "alpha"), got, ref):
        err = ((a.float().cpu() - e).abs() / e.abs().clamp_min(1e-6)).max().item()
        assert err <= tol, f"{name}: rel err {err:.3e}"


# ---------------------------------------------------------------------------
# skinny slow-weight products of the decode step (out = x W^T (+ residual), bf16 in / out,
# fp32 accumulation): against the fp32 product of the same bf16 operands.  Bound: half a
# bf16 unit of the result (2^-9 relative) doubled for the residual's own rounding, plus a
# small absolute floor for results near zero.
# ---------------------------------------------------------------------------
SKINNY_CASES = [  # (m, n, k): decode q/k/v and LM head, two row blocks, a 4-step tail wave, k = F
    (32, 2304, 768), (1, 32, 64), (40, 768, 768), (64, 32000, 768), (5, 96, 832), (8, 256, 2048)]


def check_skinny(got, ref):
    got, ref = got.double().cpu(), ref.double().cpu()
    bound = 2.0 ** -8 * ref.abs() + 1e-4
    bad = (got - ref).abs() > bound
    assert not bad.any(), f"{int(bad.sum())} entries off, max err {(got - ref).abs().max().item():.3g}"


@pytest.mark.parametrize("m,n,k", SKINNY_CASES)
def test_skinny_linear_matches_fp32_product(m, n, k):
    from utttcompanion_amd import kernels as K
    g = torch.Generator().manual_seed(m * 7 + n + k)
    x = torch.randn(m, k, generator=g).to(torch.bfloat16)
    w = (torch.randn(n, k, generator=g) / math.sqrt(k)).to(torch.bfloat16)
    ref = x.float() @ w.float().t()
    got = K.skinny_linear(x.to(DEV), w.to(DEV))
    torch.cuda.synchronize()
    check_skinny(got, ref)


def test_skinny_linear_residual_in_place_and_strided_rows():
    from utttcompanion_amd import kernels as K
    g = torch.Generator().manual_seed(11)
    m, n, k = 24, 768, 768
    wide = torch.randn(m, 3 * k, generator=g).to(torch.bfloat16)  # x is a column slice of it
    w = (torch.randn(n, k, generator=g) / math.sqrt(k)).to(torch.bfloat16)
    h = torch.randn(m, n, generator=g).to(torch.bfloat16)
    ref = h.float() + wide[:, k:2 * k].float() @ w.float().t()
    hd = h.to(DEV)
    xd = wide.to(DEV)[:, k:2 * k]
    assert xd.stride(0) == 3 * k
    out = K.skinny_linear(xd, w.to(DEV), out=hd, residual=hd)
    torch.cuda.synchronize()
    assert out.data_ptr() == hd.data_ptr()
    check_skinny(hd, ref)
    # a separate output leaves the residual untouched
    h2 = h.to(DEV)
    out2 = K.skinny_linear(xd, w.to(DEV), residual=h2)
    torch.cuda.synchronize()
    assert torch.equal(h2.cpu(), h)
    assert torch.equal(out2.cpu(), hd.cpu())


@pytest.mark.parametrize("m,n,k,with_residual", [(32, 1280, 768, False), (40, 768, 768, True), (3, 64, 2048, False)])
def test_skinny_linear_folded_rms_norm(m, n, k, with_residual):
    """x_eps > 0: rows of x RMS-normalised over k, the norm weight already in W's columns."""
    from utttcompanion_amd import kernels as K
    g = torch.Generator().manual_seed(m + 3 * n + k)
    eps = 1e-5
    x = (3.0 * torch.randn(m, k, generator=g)).to(torch.bfloat16)
    gain = 1.0 + 0.1 * torch.randn(k, generator=g)
    w = (torch.randn(n, k, generator=g) / math.sqrt(k))
    wf = (w * gain[None, :]).to(torch.bfloat16)
    xf = x.float()
    ref = (xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + eps)) @ wf.float().t()
    h = torch.randn(m, n, generator=g).to(torch.bfloat16)
    if with_residual:
        ref = ref + h.float()
        hd = h.to(DEV)
        K.skinny_linear(x.to(DEV), wf.to(DEV), out=hd, residual=hd, x_eps=eps)
        got = hd
    else:
        got = K.skinny_linear(x.to(DEV), wf.to(DEV), x_eps=eps)
    torch.cuda.synchronize()
    check_skinny(got, ref)


@pytest.mark.parametrize("dtype,rows,vocab,limit", [(torch.bfloat16, 32, 32000, 30000), (torch.float32, 5, 1003, None),
                                                   (torch.bfloat16, 3, 256, 200)])
def test_greedy_select_matches_masked_argmax(dtype, rows, vocab, limit):
    """Against the reference's own steps (float copy, -inf at the excluded ids and past the
    active limit, torch.argmax), including ties, NaN and fully masked rows."""
    K = kernels()
    g = torch.Generator().manual_seed(rows + vocab)
    x = torch.randn(rows, vocab, generator=g).to(dtype)
    x[0, 1] = 1e4  # an excluded id holding the largest value
    x[1 % rows, 7] = x[1 % rows, 9] = 50.0  # a tie: the lower id wins
    if rows > 2:
        x[2, 5] = float("nan")  # NaN counts as the largest value
    if limit is not None and rows > 3:
        x[3, limit + 1:] = 100.0  # past the active vocabulary
    banned = (0, 1, 2)
    ref = x.float().clone()
    ref[:, list(banned)] = float("-inf")
    if limit is not None:
        ref[:, limit:] = float("-inf")
    want = ref.argmax(dim=-1)
    pos = torch.arange(rows, dtype=torch.int64, device=DEV) * 7
    got = K.greedy_select(x.to(DEV), banned, limit, advance=pos)
    torch.cuda.synchronize()
    assert torch.equal(got.cpu(), want)
    assert torch.equal(pos.cpu(), torch.arange(rows, dtype=torch.int64) * 7 + 1)  # advanced once
    allmasked = torch.full((2, vocab), float("-inf")).to(dtype)
    got2 = K.greedy_select(allmasked.to(DEV), banned, limit)
    torch.cuda.synchronize()
    assert got2.tolist() == [0, 0]


def test_chunk_update_broadcast_eta_alpha_match_oracle():
    """Per-row eta / alpha of shape (B, 1, 1), and one shared (1, 1, 1) value, broadcast over the
    chunk as the reference does (model/uttt_layer.py:371-378, :501-511): the same result as the
    oracle given the same broadcast tensors."""
    K = kernels()
    q, k, v, _, _, w, s, ln_w, ln_b = make_chunk(3, 40, 128, 256, seed=31)
    mask = torch.ones(3, 40)
    mask[1, 30:] = 0
    for eta, alpha in ((torch.tensor([0.01, 0.02, 0.005]).view(3, 1, 1), torch.full((1, 1, 1), 0.003)),
                       (torch.full((1, 1, 1), 0.02), torch.tensor([0.001, 0.004, 0.002]).view(3, 1, 1))):
        ref = om.fused_chunk_ttt_step(q, k, v, eta, alpha, *w, *s, ln_w, ln_b, mask, 0.9, 1.0, True, 1e-5)
        with torch.no_grad():
            got = K.chunk_update(*to_dev(q, k, v, eta, alpha, *w, *s, ln_w, ln_b), mask.to(DEV), 0.9, 1.0, True, 1e-5)
        torch.cuda.synchronize()
        for name, a, e in zip(("readout", "w_up", "w_gate", "w_down", "s_up", "s_gate", "s_down", "surprise"), got,
                              ref):
            assert rel_err(a, e) <= F32_REL, name
