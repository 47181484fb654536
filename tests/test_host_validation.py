"""Host-side argument checks of the decode-step entry points (no GPU needed: every case is
rejected before any device call).  The wrappers raise ValueError like the reference's own
shape checks; the C ABI returns a status with a message."""
import ctypes as C

import pytest
import torch

from utttcompanion_amd import _native as N
from utttcompanion_amd import kernels as K


def test_skinny_linear_rejects_bad_operands():
    x = torch.zeros(4, 64, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="agree on k"):
        K.skinny_linear(x, torch.zeros(32, 128, dtype=torch.bfloat16))
    with pytest.raises(ValueError, match="bf16"):
        K.skinny_linear(x.float(), torch.zeros(32, 64))
    with pytest.raises(ValueError, match="no CPU path"):
        K.skinny_linear(x, torch.zeros(32, 64, dtype=torch.bfloat16))


def test_greedy_select_rejects_bad_arguments():
    logits = torch.zeros(2, 100)
    with pytest.raises(ValueError, match="at most 8"):
        K.greedy_select(logits, banned=tuple(range(9)))
    with pytest.raises(ValueError, match="rows, vocab"):
        K.greedy_select(torch.zeros(100))
    with pytest.raises(ValueError, match="no CPU path"):
        K.greedy_select(logits, banned=(0, 1, 2))


@pytest.fixture(scope="module")
def lib():
    return N.load_library()


def _fake(n):  # aligned, never dereferenced: every call below fails its checks first
    return C.c_void_p(0x100000 + 0x1000 * n)


def test_c_abi_rejects_decode_options_outside_one_token_rows(lib):
    a = N.ReadoutArgs()
    a.batch, a.tokens, a.d_model, a.d_ff = 2, 2, 256, 512
    a.act_dtype, a.w_dtype, a.eps = N.DTYPE_BF16, N.DTYPE_BF16, 1e-5
    a.x, a.w_up, a.w_gate, a.w_down = _fake(1), _fake(2), _fake(3), _fake(4)
    a.ln_weight, a.ln_bias, a.out = _fake(5), _fake(6), _fake(7)
    a.x_row_stride, a.out_row_stride = 2 * 256, 2 * 256
    a.x_norm_weight, a.x_norm_eps = _fake(8), 1e-5
    rc = lib.uttt_swiglu_readout(C.byref(a), _fake(9), 1 << 40, None)
    assert rc != 0
    assert b"one bf16 token per row" in lib.uttt_last_error()
    a.tokens = 1
    a.x_norm_eps = 0.0
    assert lib.uttt_swiglu_readout(C.byref(a), _fake(9), 1 << 40, None) != 0
    assert b"x_norm_eps" in lib.uttt_last_error()


def test_c_abi_rejects_bad_greedy_and_skinny_calls(lib):
    g = N.GreedyArgs()
    g.rows, g.vocab, g.dtype, g.n_banned = 2, 100, N.DTYPE_BF16, 1
    g.banned[0] = -3
    g.logits, g.row_stride, g.out = _fake(1), 100, _fake(2)
    assert lib.uttt_greedy_select(C.byref(g), None) != 0
    assert b"excluded ids must be >= 0" in lib.uttt_last_error()
    s = N.SkinnyLinearArgs()
    s.m, s.n, s.k, s.act_dtype, s.x_eps = 4, 64, 64, N.DTYPE_BF16, -1.0
    assert lib.uttt_skinny_linear(C.byref(s), None) != 0
    assert b"x_eps" in lib.uttt_last_error()


@pytest.mark.parametrize("shape", [(2, 15), (2, 16, 2), (3, 16, 1), (2, 2, 16, 1)])
def test_chunk_update_refuses_eta_and_alpha_that_do_not_broadcast(shape):
    """One eta / alpha per (row, token), or a shape the reference broadcasts against (B, C, 1);
    anything else is refused before any launch (the check runs ahead of the device check, so on
    the CPU)."""
    b, c, d, f = 2, 16, 64, 64
    q = torch.zeros(b, c, d)
    w = (torch.zeros(b, d, f), torch.zeros(b, d, f), torch.zeros(b, f, d))
    good = torch.zeros(b, c, 1)
    for eta, alpha in ((torch.zeros(shape), good), (good, torch.zeros(shape))):
        with pytest.raises(ValueError, match=r"must broadcast to \(2, 16, 1\)"):
            K.prepare_chunk_update(q, q, q, eta, alpha, *w, *w, torch.ones(d), torch.zeros(d), None, 0.9, 1.0,
                                   True, 1e-5)
    for ok in ((b, c), (b, c, 1), (b, 1, 1), (b, 1), (1, c, 1), (1, 1, 1)):  # get as far as the device check
        with pytest.raises(ValueError, match="no CPU path"):
            K.prepare_chunk_update(q, q, q, torch.zeros(ok), torch.zeros(ok), *w, *w, torch.ones(d),
                                   torch.zeros(d), None, 0.9, 1.0, True, 1e-5)


def test_noalloc_update_refuses_shapes_past_its_scratch(lib):
    """``uttt_chunk_update_noalloc`` checks the shape's workspace against its fixed scratch before
    any device call: config 5's 16 rows at D 2048 / F 5504 need about 106 MiB."""
    a = N.ChunkUpdateArgs()
    a.batch, a.tokens, a.d_model, a.d_ff, a.act_dtype = 16, 64, 2048, 5504, N.DTYPE_BF16
    need = lib.uttt_chunk_update_workspace(16, 2048, 5504, N.DTYPE_BF16)
    assert need > (64 << 20)
    assert lib.uttt_chunk_update_noalloc(C.byref(a), None) == 1  # UTTT_ERR_INVALID
    msg = lib.uttt_last_error()
    assert b"device-resident scratch" in msg and str(need).encode() in msg
    assert lib.uttt_chunk_update_noalloc(None, None) == 1


def test_prefill_plan_refuses_a_deferred_join_under_capture(monkeypatch):
    """``PrefillPlan.run`` refuses ``defer_join`` and ``wait_event`` while the current stream is
    capturing, before it touches a buffer or the library (the plan itself is never consulted)."""
    from utttcompanion_amd.prefill_plan import PrefillPlan
    monkeypatch.setattr(torch.cuda, "is_current_stream_capturing", lambda: True)
    for kw in (dict(defer_join=True), dict(wait_event=12345)):
        with pytest.raises(ValueError, match="graph capture"):
            PrefillPlan.run(object(), None, 0, 0, 0, None, None, None, None, **kw)


def test_per_token_scalars_broadcast_like_the_reference():
    """eta / alpha that broadcast against (B, C, 1) are expanded to one value per (row, token);
    shapes that do not broadcast are refused before any device work."""
    per = K._per_token(torch.tensor([0.1, 0.2]).view(2, 1, 1), 2, 5, "eta")
    assert per.shape == (2, 5) and per.is_contiguous() and torch.equal(per[1], torch.full((5,), 0.2))
    assert K._per_token(torch.tensor(0.3), 2, 5, "eta").shape == (2, 5)
    same = torch.zeros(2, 5, 1)
    assert K._per_token(same, 2, 5, "eta") is same
    for bad in (torch.zeros(3, 5), torch.zeros(2, 4, 1), torch.zeros(2, 5, 2), torch.zeros(1, 2, 5, 1)):
        with pytest.raises(ValueError, match="broadcast"):
            K._per_token(bad, 2, 5, "eta")
