"""Fast-weight writes with the chunk sizes the reference's own configs use (128 and 512 tokens:
configs/5090_config.yaml:31, configs/5090_pretrain_20261029.yaml:28), one write per chunk as the
reference's chunk loop does (model/uttt_layer.py:1451-1478, model/uttt_model.py:453-608).

The update kernels work in 64-token blocks: a longer chunk runs them per block, and its clip norm
sums every gradient tile over all of the chunk's blocks before squaring.  Checked against the
oracle at the kernel level (``uttt_chunk_update``: 128, a ragged 200 and 512 tokens, masks, an
active clip, the per-row gate and row losses), in the model's chunk-first prefill (chunk 128 with a
ragged tail chunk), in a standalone layer (chunk 512) and in the ragged per-request update
(chunk 128).  Tolerances as everywhere: fp32 <= 1e-5 relative (max|err| / max|ref|); bf16 fast
weights <= 2e-2 max-abs against the fp32 oracle and against the reference's own bf16 arithmetic
(the oracle run in bf16), bf16 logits <= 2e-2 max-abs or, where the reference's own bf16 error is
larger, 1.5x it + 1e-3.
"""
import math

import pytest
import torch

from oracle import uttt_math as om
from test_gpu_kernels import check_bf16_activation, make_chunk, max_abs, to_dev
from test_gpu_model import DEV, NAMES, build, ids_and_mask, rel_err

pytestmark = pytest.mark.gpu

CASES = [
    dict(C=128, b=3, d=256, f=512, mask=False, clip=1.0),
    dict(C=200, b=2, d=128, f=320, mask=True, clip=1e-3),   # a ragged last block, clip active
    dict(C=512, b=2, d=256, f=384, mask=True, clip=1.0),
]


def _mask(b, c, seed):
    g = torch.Generator().manual_seed(seed)
    m = torch.ones(b, c)
    m[0, c - 37:] = 0
    m[1, (torch.rand(c, generator=g) < 0.2)] = 0
    return m


@pytest.mark.parametrize("case", CASES, ids=[f"C{c['C']}" for c in CASES])
def test_chunk_update_long_chunks_fp32_match_oracle(case):
    from utttcompanion_amd import kernels as K
    C, b, d, f = case["C"], case["b"], case["d"], case["f"]
    print(f"long-chunk update {case}", flush=True)
    q, k, v, eta, alpha, w, s, ln_w, ln_b = make_chunk(b, C, d, f, seed=C + d)
    mask = _mask(b, C, 5) if case["mask"] else None
    ref = om.fused_chunk_ttt_step(q, k, v, eta, alpha, *w, *s, ln_w, ln_b, mask, 0.9, case["clip"], True, 1e-5)
    with torch.no_grad():
        got = K.chunk_update(*to_dev(q, k, v, eta, alpha, *w, *s, ln_w, ln_b), None if mask is None else mask.to(DEV),
                             0.9, case["clip"], True, 1e-5)
    torch.cuda.synchronize()
    for name, a, e in zip(("readout", *NAMES, "surprise"), got, ref):
        err = rel_err(a, e)
        print(f"  {name}: {err:.3e}", flush=True)
        assert err <= 1e-5, name


def test_chunk_update_512_bf16_against_both_oracles():
    from utttcompanion_amd import kernels as K
    q, k, v, eta, alpha, w, s, ln_w, ln_b = make_chunk(2, 512, 256, 512, seed=77, scale_w=0.05)
    mask = _mask(2, 512, 6)
    qb, kb, vb, eb, ab = (t.bfloat16() for t in (q, k, v, eta, alpha))
    ref = om.fused_chunk_ttt_step(*(t.float() for t in (qb, kb, vb, eb, ab)), *w, *s, ln_w, ln_b, mask, 0.9, 1.0,
                                  True, 1e-5)
    ref16 = om.fused_chunk_ttt_step(qb, kb, vb, eb, ab, *w, *s, ln_w, ln_b, mask, 0.9, 1.0, True, 1e-5)
    with torch.no_grad():
        got = K.chunk_update(*to_dev(qb, kb, vb, eb, ab, *w, *s, ln_w, ln_b), mask.to(DEV), 0.9, 1.0, True, 1e-5)
    torch.cuda.synchronize()
    check_bf16_activation("readout", got[0], ref[0], ref16[0])
    for name, a, e, e16 in zip(NAMES, got[1:7], ref[1:7], ref16[1:7]):
        assert max_abs(a, e) <= 2e-2 and max_abs(a, e16) <= 2e-2, name
    assert abs(got[7].item() - ref[7].item()) <= 2e-2 * max(1.0, abs(ref[7].item()))


def test_chunk_update_128_row_loss_and_gate_match_oracle():
    """Per-row losses over the whole 128-token chunk and the per-row gate (a row whose chunk
    surprise is below the threshold keeps W and S bit for bit)."""
    from utttcompanion_amd import kernels as K
    q, k, v, eta, alpha, w, s, ln_w, ln_b = make_chunk(4, 128, 128, 192, seed=13)
    v = v * torch.tensor([0.3, 1.0, 3.0, 10.0]).view(4, 1, 1)  # row losses far apart
    mask = torch.ones(4, 128)
    mask[1, 90:] = 0
    mask[3, ::3] = 0
    means = om.row_surprise(k, v, *w, ln_w, ln_b, mask, True, 1e-5)
    thr = float(means[1] + means[2]) / 2
    ref = om.fused_chunk_ttt_step(q, k, v, eta, alpha, *w, *s, ln_w, ln_b, mask, 0.9, 1.0, True, 1e-5,
                                  min_row_surprise=thr)
    rl = torch.full((4, 2), float("nan"), device=DEV)
    with torch.no_grad():
        prep = K.prepare_chunk_update(*to_dev(q, k, v, eta, alpha, *w, *s, ln_w, ln_b), mask.to(DEV), 0.9, 1.0, True,
                                      1e-5, row_loss=rl, min_row_surprise=thr)
        got = prep.launch()
    torch.cuda.synchronize()
    for name, a, e in zip(("readout", *NAMES, "surprise"), got, ref):
        assert rel_err(a, e) <= 1e-5, name
    for row in (0, 1):  # gated off: W and S unchanged
        for a, o in zip(got[1:7], w + s):
            assert torch.equal(a[row].cpu(), o[row])
    assert torch.equal(rl[:, 1].cpu(), mask.sum(1))
    assert rel_err(rl[:, 0].cpu() / mask.sum(1), means) <= 1e-5


LONG = dict(vocab_size=256, d_model=128, n_layers=3, n_heads=2, n_kv_heads=1, d_ff_fast=192, chunk_size=128,
            sliding_window_size=96, max_seq_len=1024, base_inner_lr=0.05, base_weight_decay=0.01)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_model_prefill_with_128_token_chunks_matches_oracle(dtype):
    """A 3-layer model writing 128-token chunks: 2 x 300 tokens (two full chunks and a ragged tail
    of 44; row 1's last 11 tokens masked), the chunk-first schedule with one update per layer."""
    print(f"model prefill, chunk 128, {dtype}", flush=True)
    model, oracle = build(LONG, dtype=dtype)
    ids, mask = ids_and_mask(2, 300, 256, seed=17)
    with torch.no_grad():
        out = model(ids.to(DEV), attention_mask=mask.to(DEV), update_fast_weights=True)
    torch.cuda.synchronize()
    logits, state, per_layer, _ = oracle.forward(ids, None, mask, update_fast_weights=True)
    assert out.fast_state.step == state.step == 3 * 3
    if dtype == torch.float32:
        assert rel_err(out.logits, logits) <= 1e-5
        for n in NAMES:
            assert rel_err(getattr(out.fast_state, n), getattr(state, n)) <= 1e-5, n
        assert rel_err(torch.tensor(out.layer_surprise_losses), per_layer) <= 1e-5
        return
    oracle16 = om.OracleModel(oracle.cfg, oracle.w, dtype=torch.bfloat16)
    logits16, state16, _, _ = oracle16.forward(ids, None, mask, update_fast_weights=True)
    ours, theirs = max_abs(out.logits, logits), max_abs(logits16, logits)
    print(f"  logits vs fp32 {ours:.3e}, reference bf16 vs fp32 {theirs:.3e}", flush=True)
    assert ours <= max(2e-2, 1.5 * theirs + 1e-3)
    for n in NAMES:
        assert max_abs(getattr(out.fast_state, n), getattr(state, n)) <= 2e-2, n
        assert max_abs(getattr(out.fast_state, n), getattr(state16, n)) <= 2e-2, n


def test_standalone_layer_with_512_token_chunks_matches_oracle():
    """``uTTTLayer.forward`` with chunk_size 512 on 2 rows x 700 tokens (a full chunk and a tail of
    188), each chunk reading its own pre-update state, against the oracle's layer forward."""
    from utttcompanion_amd import uTTTConfig, uTTTModel
    from test_gpu_model import draw
    cfg_kw = dict(LONG, chunk_size=512, n_layers=1)
    torch.manual_seed(0)
    model = uTTTModel(uTTTConfig(**cfg_kw)).eval()
    sd = draw(model.state_dict(), 21)
    sd["lm_head.weight"] = sd["tok_embeddings.weight"]
    model.load_state_dict(sd)
    model = model.to(DEV)
    layer = model.layers[0].uttt
    lw = {k[len("layers.0."):]: v for k, v in sd.items() if k.startswith("layers.0.")}
    ocfg = om.OracleConfig(d_model=128, n_layers=1, n_heads=2, n_kv_heads=1, d_ff_fast=192, sliding_window_size=96,
                           chunk_size=512, base_inner_lr=0.05, base_weight_decay=0.01)
    oracle = om.OracleModel(ocfg, {k: v for k, v in sd.items() if k != "lm_head.weight"})
    g = torch.Generator().manual_seed(12)
    x = torch.randn(2, 700, 128, generator=g)
    mask = torch.ones(2, 700)
    mask[1, 650:] = 0
    ostate = oracle.init_state(2)
    state = model.fast_weight_pool.init_state(2, device=DEV, dtype=torch.float32, detach=True)
    with torch.no_grad():
        out, st, sur = layer(x.to(DEV), model.fast_weight_pool, state, attention_mask=mask.to(DEV))
    torch.cuda.synchronize()
    oout, ost, osur = om.uttt_layer_forward(x, lw, ocfg, ostate, mask)
    assert rel_err(out, oout) <= 1e-5
    for n in NAMES:
        assert rel_err(getattr(st, n), getattr(ost, n)) <= 1e-5, n
    assert rel_err(sur, osur) <= 1e-5
    assert st.step == 2


def test_ragged_update_with_128_token_chunks_matches_oracle():
    """Ragged per-request updates (lengths 50, 300, 129, 256) with 128-token chunks: every request
    equals its own batch-1 oracle ``test_time_update`` (fp32, 1e-5), the finished requests'
    states taken from whichever state set their last chunk wrote."""
    from utttcompanion_amd.evolve import ragged_test_time_update
    from test_gpu_evolve import to_state
    model, oracle = build(LONG)
    g = torch.Generator().manual_seed(4)
    lengths = [50, 300, 129, 256]
    ids = [torch.randint(6, 256, (n,), generator=g) for n in lengths]
    masks = [torch.ones(n) for n in lengths]
    masks[1][-20:] = 0
    ostates = []
    for i in range(len(lengths)):
        st = oracle.init_state(1)
        for name in ("w_up", "w_gate", "w_down"):
            getattr(st, name).add_(0.02 * torch.randn(getattr(st, name).shape, generator=g))
        ostates.append(st)
    states = [to_state(st) for st in ostates]
    got = ragged_test_time_update(model, [t.to(DEV) for t in ids], states, [m.to(DEV) for m in masks])
    torch.cuda.synchronize()
    for i, (cand, surprise, layers) in enumerate(got):
        ocand, osurprise, olayers = oracle.test_time_update(ids[i].view(1, -1), ostates[i], masks[i].view(1, -1))
        for n in NAMES:
            assert rel_err(getattr(cand, n), getattr(ocand, n)) <= 1e-5, (i, n)
        assert abs(surprise - osurprise) <= 1e-5 * max(1.0, abs(osurprise)), i
        assert rel_err(torch.tensor(layers), torch.tensor(olayers)) <= 1e-5, i
        assert cand.step == ocand.step == math.ceil(lengths[i] / 128) * 3, i
