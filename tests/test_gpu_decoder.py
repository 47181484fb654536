"""Batched ring-buffer decoding (utttcompanion_amd.decoder) against the per-request eager path.

Each request has its own fast-weight state and a ragged prompt (some longer than the window,
so the ring wraps).  Greedy tokens must equal the reference-style batch-1 ``stream_generate``
(temperature 0) for every request; logits of a graph-replayed step must equal the eager step.
"""
import pytest
import torch

pytestmark = pytest.mark.gpu
DEV = "cuda"

CFG = dict(vocab_size=256, d_model=128, n_layers=3, n_heads=2, n_kv_heads=1, d_ff_fast=192, chunk_size=16,
           sliding_window_size=24, max_seq_len=512)


def make(dtype=torch.float32, seed=0, slow_std=0.08, cfg=None):
    """``slow_std`` 0.08 (larger than the reference's 0.02 init) makes greedy tokens vary in
    the token-equality test; the bf16 logits test uses the reference init."""
    from utttcompanion_amd import uTTTConfig, uTTTModel
    torch.manual_seed(seed)
    model = uTTTModel(uTTTConfig(**(cfg or CFG))).eval()
    with torch.no_grad():
        for name, p in model.named_parameters():
            if p.dim() == 2 and "fast_weight_pool" not in name and "w_eta" not in name and "w_alpha" not in name:
                p.normal_(0, slow_std)
    model = model.to(DEV)
    if dtype != torch.float32:
        model.to(dtype)
        model.fast_weight_pool.float()
    g = torch.Generator().manual_seed(seed + 1)
    states = []
    for i in range(4):
        st = model.init_fast_state(1, device=DEV, dtype=torch.float32, detach=True)
        for name in ("w_up", "w_gate", "w_down"):
            t = getattr(st, name)
            t.add_(0.05 * torch.randn(t.shape, generator=g).to(DEV))
        states.append(st)
    lengths = [5, 17, 30, 40]
    prompts = [torch.randint(6, (cfg or CFG)["vocab_size"], (n,), generator=g) for n in lengths]
    return model, states, prompts


def test_batched_greedy_tokens_equal_per_request_stream_generate():
    from utttcompanion_amd.decoder import BatchedDecoder
    model, states, prompts = make()
    dec = BatchedDecoder(model, states)
    first = dec.prefill(prompts)
    tokens = dec.generate_greedy(first, 24).cpu()
    for i, (st, ids) in enumerate(zip(states, prompts)):
        want = list(model.stream_generate(ids.view(1, -1).to(DEV), st, max_new_tokens=24, temperature=0.0,
                                          eos_token_id=None))
        assert tokens[i, :len(want)].tolist() == want, f"request {i}"


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_graph_step_equals_eager_step(dtype):
    from utttcompanion_amd.decoder import BatchedDecoder
    model, states, prompts = make(dtype)
    eager = BatchedDecoder(model, states)
    graph = BatchedDecoder(model, states)
    f1, f2 = eager.prefill(prompts), graph.prefill(prompts)
    assert torch.equal(f1, f2)
    graph.capture()
    tok = f1.float().argmax(-1)
    for step in range(30):  # crosses several ring wraps for the short prompts
        a = eager.step(tok).clone()
        b = graph.step(tok).clone()
        torch.cuda.synchronize()
        assert torch.equal(a, b), step
        tok = eager.next_tokens.clone()


# head_dim 128 (split attention form), d_model 1024, d_ff 640 (128-column readout blocks)
CFG_WIDE = dict(vocab_size=512, d_model=1024, n_layers=2, n_heads=8, n_kv_heads=2, d_ff_fast=640, chunk_size=16,
                sliding_window_size=24, max_seq_len=512)


@pytest.mark.parametrize("cfg,atol", [(None, 0.015), (CFG_WIDE, 0.035)], ids=["c2-like", "wide"])
def test_decoder_logits_match_eager_frozen_forward_bf16(cfg, atol):
    """bf16 model: batched step logits vs the eager frozen single-request forward, at the
    reference's own bound for ring decode vs eager bf16 logits (atol 0.015, rtol 0.025,
    reference tests/test_inference_cuda_graph.py:54-90): the batched GEMMs and the ring
    change bf16 reduction orders, so the two need not be bitwise equal.  The wide model's
    logits reach |2.5|, where one bf16 unit is 2^-6: there the absolute bound is two such units
    plus a little (a step through the library GEMMs and separate norms differs from the eager
    forward by the same 0.02-0.025)."""
    from utttcompanion_amd.decoder import BatchedDecoder
    model, states, prompts = make(torch.bfloat16, seed=3, slow_std=0.02, cfg=cfg)
    dec = BatchedDecoder(model, states)
    first = dec.prefill(prompts)
    tok = first.float().argmax(-1)
    caches = []
    for st, ids in zip(states, prompts):
        out = model(ids.view(1, -1).to(DEV), fast_state=st, update_fast_weights=False, logits_to_keep=1)
        caches.append(out.kv_caches)
    for step in range(6):
        got = dec.step(tok).float()
        for i, (st, ids) in enumerate(zip(states, prompts)):
            pos = len(ids) + step
            out = model(tok[i].view(1, 1), fast_state=st, kv_caches=caches[i], start_pos=pos,
                        update_fast_weights=False)
            caches[i] = out.kv_caches
            torch.testing.assert_close(got[i], out.logits[0, -1].float(), atol=atol, rtol=0.025,
                                       msg=f"step {step} request {i}")
        tok = dec.next_tokens.clone()


def test_stream_generate_graph_route_equals_eager_tokens():
    """``use_cuda_graph=True`` (one-request ring decoder replayed from a HIP graph) yields the
    eager tokens; a second call with the same state reuses the captured decoder, and a write
    to the state's W makes the next call build a new one."""
    model, states, prompts = make()
    kw = dict(max_new_tokens=20, temperature=0.0, eos_token_id=None)
    for st, ids in zip(states[2:], prompts[2:]):  # prompts of 30 and 40 tokens: past the 24 window
        p = ids.view(1, -1).to(DEV)
        eager = list(model.stream_generate(p, st, **kw))
        graph = list(model.stream_generate(p, st, use_cuda_graph=True, **kw))
        assert graph == eager
        dec = model._cuda_graph_decoder
        assert dec is not None and dec._graph is not None
        assert list(model.stream_generate(p, st, use_cuda_graph=True, **kw)) == eager
        assert model._cuda_graph_decoder is dec
    st, p = states[3], prompts[3].view(1, -1).to(DEV)
    with torch.no_grad():
        st.w_up.add_(0.05)
    eager = list(model.stream_generate(p, st, **kw))
    assert list(model.stream_generate(p, st, use_cuda_graph=True, **kw)) == eager
    assert model._cuda_graph_decoder is not dec


def test_fused_inference_readout_reads_versioned_copies():
    """``prepare_for_inference()``: frozen readouts of a bf16 model read the state's versioned
    bf16 copies -- bit for bit the readout of explicit bf16 copies -- and a write to the master
    refreshes them."""
    from utttcompanion_amd import kernels as K
    model, states, _ = make(torch.bfloat16, seed=5, slow_std=0.02)
    model.prepare_for_inference()
    pool, st = model.fast_weight_pool, states[0]
    x = torch.randn(1, 7, CFG["d_model"], device=DEV).bfloat16()
    with torch.no_grad():
        got = pool.forward_readout(x, st)
        want = K.swiglu_readout(x, *(t.bfloat16() for t in (st.w_up, st.w_gate, st.w_down)), st.ln_weight,
                                st.ln_bias, pool.eps)
        assert torch.equal(got, want)
        copies = st._read_copies
        pool.forward_readout(x, st)
        assert st._read_copies is copies
        st.w_down.mul_(1.5)
        got2 = pool.forward_readout(x, st)
        want2 = K.swiglu_readout(x, *(t.bfloat16() for t in (st.w_up, st.w_gate, st.w_down)), st.ln_weight,
                                 st.ln_bias, pool.eps)
    torch.cuda.synchronize()
    assert st._read_copies is not copies and torch.equal(got2, want2)
    model.prepare_for_inference(False)
