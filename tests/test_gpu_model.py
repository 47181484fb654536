"""GPU parity of the drop-in modules (utttcompanion_amd.layer / .model) against the CPU oracle.

The oracle's compositions are pinned to the reference by tests/golden (see
test_oracle_golden.py); here the HIP path runs the same seeded weights and inputs at
kernel-supported sizes (d_model and d_ff multiples of 64, head_dim 64/128).
Tolerances (north star): fp32 <= 1e-5 relative (max|err| / max|ref|) for fast-weight
state, surprise, logits and activations; bf16 <= 2e-2 max-abs for logits and updated fast
weights.
"""
import math

import pytest
import torch

from oracle import uttt_math as om

pytestmark = pytest.mark.gpu
DEV = "cuda"
NAMES = ("w_up", "w_gate", "w_down", "s_up", "s_gate", "s_down")


def rel_err(a, e):
    a, e = a.detach().double().cpu(), e.detach().double().cpu()
    return (a - e).abs().max().item() / max(e.abs().max().item(), 1e-30)


def max_abs(a, e):
    return (a.detach().double().cpu() - e.detach().double().cpu()).abs().max().item()


def draw(sd, seed):
    g = torch.Generator().manual_seed(seed)
    out = {}
    for name, t in sd.items():
        if name == "lm_head.weight":
            continue
        shape = tuple(t.shape)
        if name.endswith(("norm.weight", "ln_weight")):
            v = 1.0 + 0.1 * torch.randn(shape, generator=g)
        elif name.endswith("ln_bias"):
            v = 0.05 * torch.randn(shape, generator=g)
        elif name.endswith(("w_up_init", "w_gate_init")):
            v = torch.randn(shape, generator=g) / shape[0] ** 0.5
        elif name.endswith("w_down_init"):
            v = 0.3 * torch.randn(shape, generator=g) / shape[0] ** 0.5
        elif name.endswith(("w_eta.weight", "w_alpha.weight")):
            v = 0.05 * torch.randn(shape, generator=g)
        elif name.endswith("w_eta.bias"):
            v = torch.zeros(shape)
        elif name.endswith("w_alpha.bias"):
            v = torch.full(shape, -1.386)
        elif name == "tok_embeddings.weight":
            v = torch.randn(shape, generator=g)
        else:
            v = 0.05 * torch.randn(shape, generator=g)
        out[name] = v.float()
    return out


SMALL = dict(vocab_size=256, d_model=128, n_layers=3, n_heads=2, n_kv_heads=1, d_ff_fast=192, chunk_size=16,
             sliding_window_size=24, max_seq_len=512, base_inner_lr=0.05, base_weight_decay=0.01)


def build(cfg_kw=SMALL, seed=5, dtype=torch.float32):
    from utttcompanion_amd import uTTTConfig, uTTTModel
    cfg = uTTTConfig(**cfg_kw)
    torch.manual_seed(0)
    model = uTTTModel(cfg).eval()
    weights = draw(model.state_dict(), seed)
    sd = dict(weights)
    sd["lm_head.weight"] = sd["tok_embeddings.weight"]
    if dtype != torch.float32:  # round slow weights as the bf16 model will hold them
        weights = {k: (v if k.startswith("fast_weight_pool.") else v.to(dtype).float()) for k, v in weights.items()}
    model.load_state_dict(sd)
    model = model.to(DEV)
    if dtype != torch.float32:
        model.to(dtype)
        model.fast_weight_pool.float()  # fp32 masters: reload the pool the cast has rounded
        pre = "fast_weight_pool."
        model.fast_weight_pool.load_state_dict({k[len(pre):]: v for k, v in sd.items() if k.startswith(pre)})
    ocfg = om.OracleConfig(**{k: cfg_kw[k] for k in ("d_model", "n_layers", "n_heads", "n_kv_heads", "d_ff_fast",
                                                     "sliding_window_size", "vocab_size", "chunk_size",
                                                     "base_inner_lr", "base_weight_decay")})
    return model, om.OracleModel(ocfg, weights)


def ids_and_mask(bsz, seq, vocab, seed=7):
    g = torch.Generator().manual_seed(seed)
    ids = torch.randint(6, vocab, (bsz, seq), generator=g)
    mask = torch.ones(bsz, seq)
    if bsz > 1:
        mask[1, seq - 11:] = 0
    return ids, mask


def test_model_forward_with_writes_fp32_matches_oracle():
    model, oracle = build()
    ids, mask = ids_and_mask(2, 56, 256)
    out = model(ids.to(DEV), attention_mask=mask.to(DEV), update_fast_weights=True)
    logits, state, per_layer, caches = oracle.forward(ids, None, mask, update_fast_weights=True)
    assert rel_err(out.logits, logits) <= 1e-5
    for n in NAMES:
        assert rel_err(getattr(out.fast_state, n), getattr(state, n)) <= 1e-5, n
    assert rel_err(torch.tensor(out.layer_surprise_losses), per_layer) <= 1e-5
    assert out.fast_state.step == state.step
    for (k, v), (ok, ov) in zip(out.kv_caches, caches):
        assert rel_err(k, ok) <= 1e-5 and rel_err(v, ov) <= 1e-5


def test_model_forward_with_writes_bf16_within_tolerance():
    """bf16 slow weights / activations with fp32 fast-weight masters, reference initialisation
    (N(0, 0.02) slow weights, pool W_0 draws): logits and updated fast weights within 2e-2
    max-abs of the fp32 oracle, and no further from it than the reference's own bf16
    arithmetic (the oracle run in bf16) plus 50%."""
    from utttcompanion_amd import uTTTConfig, uTTTModel
    cfg_kw = dict(SMALL, d_ff_fast=256)
    torch.manual_seed(3)
    model = uTTTModel(uTTTConfig(**cfg_kw)).eval()
    weights = {k: v.detach().clone() for k, v in model.state_dict().items()}
    rounded = {k: (v if k.startswith("fast_weight_pool.") else v.bfloat16().float()) for k, v in weights.items()}
    model = model.to(DEV).to(torch.bfloat16)
    model.fast_weight_pool.float()  # fp32 masters: reload the pool the cast has rounded
    pre = "fast_weight_pool."
    model.fast_weight_pool.load_state_dict({k[len(pre):]: v for k, v in weights.items() if k.startswith(pre)})
    ocfg = om.OracleConfig(**{k: cfg_kw[k] for k in ("d_model", "n_layers", "n_heads", "n_kv_heads", "d_ff_fast",
                                                     "sliding_window_size", "vocab_size", "chunk_size",
                                                     "base_inner_lr", "base_weight_decay")})
    oracle = om.OracleModel(ocfg, rounded)
    oracle16 = om.OracleModel(ocfg, rounded, dtype=torch.bfloat16)
    ids, mask = ids_and_mask(2, 64, 256, seed=9)
    out = model(ids.to(DEV), attention_mask=mask.to(DEV), update_fast_weights=True)
    logits, state, _, _ = oracle.forward(ids, None, mask, update_fast_weights=True)
    logits16, state16, _, _ = oracle16.forward(ids, None, mask, update_fast_weights=True)
    assert out.logits.dtype == torch.bfloat16 and out.fast_state.w_up.dtype == torch.float32
    ours, theirs = max_abs(out.logits, logits), max_abs(logits16, logits)
    assert ours <= 2e-2, f"logits max abs {ours:.3e} (reference bf16: {theirs:.3e})"
    assert ours <= 1.5 * theirs + 1e-3, f"logits max abs {ours:.3e} vs reference bf16 {theirs:.3e}"
    for n in NAMES[:3]:
        assert max_abs(getattr(out.fast_state, n), getattr(state, n)) <= 2e-2, n


def test_caller_state_is_not_modified_and_split_prefill_matches():
    model, _ = build()
    ids, _ = ids_and_mask(1, 48, 256, seed=3)
    d_ids = ids.to(DEV)
    state = model.init_fast_state(1, device=DEV, dtype=torch.float32, detach=True)
    before = [t.clone() for t in state.tensors()]
    full = model(d_ids, fast_state=state)
    for a, b in zip(state.tensors(), before):
        assert torch.equal(a, b)
    first = model(d_ids[:, :32], fast_state=state)
    second = model(d_ids[:, 32:], fast_state=first.fast_state, kv_caches=first.kv_caches, start_pos=32)
    both = torch.cat([first.logits, second.logits], 1)
    assert rel_err(both, full.logits) <= 1e-5
    for n in NAMES:
        assert rel_err(getattr(second.fast_state, n), getattr(full.fast_state, n)) <= 1e-5


def test_no_future_leakage_with_writes_on_gpu():
    model, _ = build()
    ids, _ = ids_and_mask(2, 48, 256, seed=4)
    changed = ids.clone()
    changed[:, 20:] = (changed[:, 20:] + 37) % 250 + 6
    a = model(ids.to(DEV)).logits
    b = model(changed.to(DEV)).logits
    assert torch.equal(a[:, :20], b[:, :20])


def test_trailing_padding_leaves_writes_and_logits_unchanged():
    """Padding invariance (reference tests/test_shared_schedule_audit.py:95-127): a row padded at
    the end with masked tokens takes the same writes, and gives the same logits on its valid
    tokens, as the unpadded row: masked tokens carry no loss, and a chunk without a valid token
    neither decays the state nor applies momentum.  40 valid tokens (two full chunks of 16 and a
    partial one) padded to 64: the partial chunk completed with 8 masked tokens, then a fully
    masked chunk."""
    model, _ = build()
    ids, _ = ids_and_mask(1, 40, 256, seed=31)
    padded = torch.cat([ids, torch.full((1, 24), 7)], 1)
    mask = torch.cat([torch.ones(1, 40), torch.zeros(1, 24)], 1)
    plain = model(ids.to(DEV), update_fast_weights=True)
    pad = model(padded.to(DEV), attention_mask=mask.to(DEV), update_fast_weights=True)
    assert rel_err(pad.logits[:, :40], plain.logits) <= 1e-5
    for n in NAMES:
        assert rel_err(getattr(pad.fast_state, n), getattr(plain.fast_state, n)) <= 1e-5, n


def test_writes_reach_only_later_chunks():
    """Chunk-first schedule (reference tests/test_shared_schedule_audit.py:40-60): a chunk's
    writes reach later chunks only.  With writes, the first chunk's logits equal those of a
    forward without writes (every layer of it reads the initial state); later chunks differ."""
    model, _ = build()
    ids, _ = ids_and_mask(1, 48, 256, seed=33)
    written = model(ids.to(DEV), update_fast_weights=True).logits
    frozen = model(ids.to(DEV), update_fast_weights=False).logits
    assert rel_err(written[:, :16], frozen[:, :16]) <= 1e-5
    assert max_abs(written[:, 16:32], frozen[:, 16:32]) > 1e-3


def test_test_time_update_pull_and_drift_match_oracle():
    model, oracle = build()
    ids, mask = ids_and_mask(2, 40, 256, seed=12)
    base = model.init_fast_state(1, device=DEV, dtype=torch.float32, detach=True)
    cand, surprise, layers = model.test_time_update(ids[1:2].to(DEV), base, attention_mask=mask[1:2].to(DEV))
    ocand, osurprise, olayers = oracle.test_time_update(ids[1:2], oracle.init_state(1), mask[1:2])
    for n in NAMES:
        assert rel_err(getattr(cand, n), getattr(ocand, n)) <= 1e-5, n
    assert abs(surprise - osurprise) <= 1e-5 * max(1.0, abs(osurprise))
    assert rel_err(torch.tensor(layers), torch.tensor(olayers)) <= 1e-5
    w0 = tuple(oracle.pool[n] for n in ("w_up_init", "w_gate_init", "w_down_init"))
    for ratio in (0.35, 1e-4, None):
        pulled = model.fast_weight_pool.apply_elastic_pull(cand, 0.02, ratio)
        opulled = om.apply_elastic_pull((ocand.w_up, ocand.w_gate, ocand.w_down), w0, 0.02, ratio)
        for a, e in zip((pulled.w_up, pulled.w_gate, pulled.w_down), opulled):
            assert rel_err(a, e) <= 1e-5, ratio
    drift = model.fast_weight_pool.compute_drift(pulled)
    odrift = om.compute_drift(opulled, w0)
    for key in ("drift_frobenius", "base_frobenius", "w_up_drift", "w_down_drift_pct"):
        assert abs(drift[key] - odrift[key]) <= 1e-4 * max(1.0, abs(odrift[key])), key


def test_greedy_stream_generate_matches_oracle_tokens():
    model, oracle = build()
    ids, _ = ids_and_mask(1, 30, 256, seed=21)
    state = model.init_fast_state(1, device=DEV, dtype=torch.float32, detach=True)
    tokens = list(model.stream_generate(ids.to(DEV), state, max_new_tokens=16, temperature=0.0, eos_token_id=None))
    want = oracle.greedy_generate(ids, oracle.init_state(1), 16)
    assert tokens == want


def test_incremental_decode_equals_full_prefix():
    """reference tests/test_inference_edge_audit.py:48-62 on the HIP path."""
    model, _ = build()
    ids, _ = ids_and_mask(1, 40, 256, seed=22)
    d_ids = ids.to(DEV)
    state = model.init_fast_state(1, device=DEV, dtype=torch.float32, detach=True)
    caches = None
    for length in range(20, 41):
        full = model(d_ids[:, :length], fast_state=state, update_fast_weights=False, logits_to_keep=1)
        if caches is None:
            step = full
        else:
            step = model(d_ids[:, length - 1:length], fast_state=state, kv_caches=caches, start_pos=length - 1,
                         update_fast_weights=False, logits_to_keep=1)
        caches = step.kv_caches
        assert rel_err(step.logits, full.logits) <= 1e-5, length


def test_cached_block_and_standalone_layer_match_oracle():
    from utttcompanion_amd import uTTTBlock
    torch.manual_seed(0)
    block = uTTTBlock(0, 128, 2, 1, window_size=24, chunk_size=16, base_inner_lr=0.05, base_weight_decay=0.01).eval()
    lw = draw(block.state_dict(), 99)
    block.load_state_dict(lw)
    block = block.to(DEV)
    model, oracle = build()
    pool = model.fast_weight_pool
    cfg = om.OracleConfig(d_model=128, n_layers=1, n_heads=2, n_kv_heads=1, d_ff_fast=192, sliding_window_size=24,
                          chunk_size=16, base_inner_lr=0.05, base_weight_decay=0.01)
    g = torch.Generator().manual_seed(11)
    x, x_prev = torch.randn(2, 40, 128, generator=g), torch.randn(2, 20, 128, generator=g)
    mask = torch.ones(2, 40)
    mask[0, 33:] = 0
    ostate = oracle.init_state(2)
    for n in ("s_up", "s_gate", "s_down"):
        setattr(ostate, n, 0.01 * torch.randn(getattr(ostate, n).shape, generator=g))
    state = pool.init_state(2, device=DEV, dtype=torch.float32, detach=True)
    for n in ("s_up", "s_gate", "s_down"):
        setattr(state, n, getattr(ostate, n).to(DEV))
    with torch.no_grad():
        out, st, sur = block.uttt(x.to(DEV), pool, state.clone(), attention_mask=mask.to(DEV))
    oout, ost, osur = om.uttt_layer_forward(x, lw, cfg, ostate.clone(), mask)
    assert rel_err(out, oout) <= 1e-5
    for n in NAMES:
        assert rel_err(getattr(st, n), getattr(ost, n)) <= 1e-5, n
    assert rel_err(sur, osur) <= 1e-5
    cos, sin = om.rope_tables(64, 512)
    with torch.no_grad():
        _, _, _, cache = block(x_prev.to(DEV), pool, state.clone(), update_fast_weights=False)
        bout, bst, bsur, bcache = block(x.to(DEV), pool, state.clone(), mask.to(DEV), cache, 20)
    _, _, _, ocache = om.block_forward(x_prev, lw, cfg, cos, sin, ostate.clone(), update_fast_weights=False)
    obout, obst, obsur, obcache = om.block_forward(x, lw, cfg, cos, sin, ostate.clone(), mask, ocache, 20)
    assert rel_err(bout, obout) <= 1e-5
    for n in NAMES:
        assert rel_err(getattr(bst, n), getattr(obst, n)) <= 1e-5, n
    assert rel_err(bcache[0], obcache[0]) <= 1e-5 and rel_err(bcache[1], obcache[1]) <= 1e-5


def test_config1_block_fp32_matches_oracle():
    """Config 1: one uTTT block, fp32, B1 T1024 D512 8x64 heads, window 256, F1024, C64, 16 chunks."""
    from utttcompanion_amd import SharedFastWeightPool, uTTTBlock
    torch.manual_seed(0)
    block = uTTTBlock(0, 512, 8, 4, window_size=256, chunk_size=64, base_inner_lr=0.01,
                      base_weight_decay=0.005, max_seq_len=2048).eval()
    pool = SharedFastWeightPool(512, 1024, normalize_loss_by_dim=True)
    g = torch.Generator().manual_seed(1)
    lw = {}
    for k, t in block.state_dict().items():
        if k.endswith("norm.weight"):
            lw[k] = torch.ones(t.shape)
        elif k.endswith(("w_eta.weight", "w_alpha.weight")):
            lw[k] = torch.zeros(t.shape)
        elif k.endswith("w_eta.bias"):
            lw[k] = torch.zeros(t.shape)
        elif k.endswith("w_alpha.bias"):
            lw[k] = torch.full(t.shape, -1.386)
        else:
            lw[k] = 0.02 * torch.randn(t.shape, generator=g)
    block.load_state_dict(lw)
    w0 = [0.02 * torch.randn(512, 1024, generator=g), 0.02 * torch.randn(512, 1024, generator=g),
          0.02 * torch.randn(1024, 512, generator=g)]
    with torch.no_grad():
        pool.w_up_init.copy_(w0[0]); pool.w_gate_init.copy_(w0[1]); pool.w_down_init.copy_(w0[2])
    block, pool = block.to(DEV), pool.to(DEV)
    x = torch.randn(1, 1024, 512, generator=g)
    cfg = om.OracleConfig(d_model=512, n_layers=1, n_heads=8, n_kv_heads=4, d_ff_fast=1024, sliding_window_size=256,
                          chunk_size=64, base_inner_lr=0.01, base_weight_decay=0.005)
    ostate = om.init_state({"w_up_init": w0[0], "w_gate_init": w0[1], "w_down_init": w0[2],
                            "ln_weight": torch.ones(512), "ln_bias": torch.zeros(512)}, 1)
    cos, sin = om.rope_tables(64, 2048)
    oout, ost, osur, _ = om.block_forward(x, lw, cfg, cos, sin, ostate)
    state = pool.init_state(1, device=DEV, dtype=torch.float32, detach=True)
    with torch.no_grad():
        out, st, sur, _ = block(x.to(DEV), pool, state)
    assert rel_err(out, oout) <= 1e-5
    for n in NAMES:
        assert rel_err(getattr(st, n), getattr(ost, n)) <= 1e-5, n
    assert rel_err(sur, osur) <= 1e-5


def test_prefill_with_kernel_timer_equals_plain_prefill():
    """The measurement hook (events around chain kernels, stages enqueued launch by launch) leaves
    the prefill's results unchanged, bit for bit (fp32 and bf16)."""
    from utttcompanion_amd.kernels import KernelTimer
    for dtype in (torch.float32, torch.bfloat16):
        model, _ = build(dtype=dtype)
        ids, mask = ids_and_mask(2, 80, 256, seed=31)
        d_ids, d_mask = ids.to(DEV), mask.to(DEV)
        state = model.init_fast_state(2, device=DEV, dtype=torch.float32, detach=True)
        timer = KernelTimer(("k_chain_back_lds", "k_chain_back", "k_chain_apply_lds", "k_chain_apply"))
        with torch.no_grad():  # the timer enqueues launch by launch: compare with that path
            a = model.prefill_with_writes(d_ids, state, d_mask, executor=False)
            b = model.prefill_with_writes(d_ids, state, d_mask, kernel_timer=timer)
        torch.cuda.synchronize()
        assert torch.equal(a[0], b[0]) and torch.equal(a[2], b[2])
        for x, y in zip(a[1], b[1]):
            assert torch.equal(x, y)
        summary = timer.summary()
        back = "k_chain_back_lds" if dtype == torch.bfloat16 else "k_chain_back"
        assert summary[back]["launches"] == 5 * SMALL["n_layers"]  # 5 chunks of 16 tokens


def test_prefill_graph_replays_match_eager():
    """The whole prefill with writes recorded in one HIP graph; several replays with eager
    work and syncs between them must each equal the eager result."""
    model, _ = build()
    ids, _ = ids_and_mask(2, 64, 256, seed=30)
    d_ids = ids.to(DEV)
    state = model.init_fast_state(2, device=DEV, dtype=torch.float32, detach=True)
    with torch.no_grad():
        h, tensors, per_layer, _ = model.prefill_with_writes(d_ids, state)
        eager = (h.clone(), [t.clone() for t in tensors], per_layer.clone())
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            gout = model.prefill_with_writes(d_ids, state)
        for rep in range(3):
            graph.replay()
            torch.cuda.synchronize()
            assert torch.equal(gout[0], eager[0]), rep
            for a, e in zip(gout[1], eager[1]):
                assert torch.equal(a, e), rep
            assert torch.equal(gout[2], eager[2]), rep
            model(d_ids[:, :16], fast_state=state)  # unrelated eager work between replays
            torch.cuda.synchronize()


def test_prefill_chunk_executor_matches_per_call_path():
    """bf16: one ``uttt_prefill_chunk`` call per chunk (slow-weight products on ``uttt_linear``)
    against the launch-by-launch path (the same kernels, products on torch), with a token mask,
    a ragged last chunk (two plans), and a second prefill continuing from the first's KV caches
    (history offsets and positions).  The two differ only in the products' accumulation order
    (one bf16 rounding of each product either way, carried through the layers): hidden rows and
    KV caches within 2e-2 relative (max|diff| / max|ref|; a few bf16 ulps of the largest
    values), fast-weight state within 2e-2 max-abs (the bf16 bar), surprise within 1e-2
    relative."""
    model, _ = build(dtype=torch.bfloat16)
    ids, mask = ids_and_mask(2, 72, 256, seed=41)  # 4 chunks of 16 + one of 8
    ids2, mask2 = ids_and_mask(2, 40, 256, seed=42)
    d_ids, d_mask, d_ids2, d_mask2 = ids.to(DEV), mask.to(DEV), ids2.to(DEV), mask2.to(DEV)
    state = model.init_fast_state(2, device=DEV, dtype=torch.float32, detach=True)
    outs = []
    with torch.no_grad():
        for executor in (True, False):
            a = model.prefill_with_writes(d_ids, state, d_mask, executor=executor)
            nxt = model.init_fast_state(2, device=DEV, dtype=torch.float32, detach=True)
            for t, n in zip(a[1], NAMES):
                getattr(nxt, n).copy_(t)
            b = model.prefill_with_writes(d_ids2, nxt, d_mask2, kv_caches=a[3], start_pos=72, executor=executor)
            outs.append((a, b))
    torch.cuda.synchronize()
    (ea, eb), (pa, pb) = outs
    for x, y in ((ea, pa), (eb, pb)):
        assert x[0].dtype == torch.bfloat16 and torch.isfinite(x[0].float()).all()
        assert rel_err(x[0], y[0]) <= 2e-2
        for n, t, u in zip(NAMES, x[1], y[1]):
            assert max_abs(t, u) <= 2e-2, n
        assert rel_err(x[2], y[2]) <= 1e-2
        for (k1, v1), (k2, v2) in zip(x[3], y[3]):
            assert k1.shape == k2.shape and rel_err(k1, k2) <= 2e-2 and rel_err(v1, v2) <= 2e-2


def test_prefill_chunk_executor_graph_replays_match_eager():
    """The executor path (bf16) recorded in one HIP graph: its native events join the chain
    stream into the capture; replays with eager work between them equal the eager result."""
    model, _ = build(dtype=torch.bfloat16)
    ids, mask = ids_and_mask(2, 48, 256, seed=43)
    d_ids, d_mask = ids.to(DEV), mask.to(DEV)
    state = model.init_fast_state(2, device=DEV, dtype=torch.float32, detach=True)
    with torch.no_grad():
        h, tensors, per_layer, _ = model.prefill_with_writes(d_ids, state, d_mask)
        eager = (h.clone(), [t.clone() for t in tensors], per_layer.clone())
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            gout = model.prefill_with_writes(d_ids, state, d_mask)
        for rep in range(3):
            graph.replay()
            torch.cuda.synchronize()
            assert torch.equal(gout[0], eager[0]), rep
            for a, e in zip(gout[1], eager[1]):
                assert torch.equal(a, e), rep
            assert torch.equal(gout[2], eager[2]), rep
            model.prefill_with_writes(d_ids[:, :16], state)  # unrelated eager work between replays
            torch.cuda.synchronize()


def test_prefill_chunk_executor_long_window_matches_per_call_path():
    """bf16, 16 heads x 4 rows with a 1024-token window over 17 chunks of 64: the attention's key
    split changes with the keys in range (and not monotonically), so the executor's one attention
    workspace serves calls of several split layouts; the executor stays within the bf16 bar of
    the launch-by-launch path (hidden rows 2e-2 relative, fast weights 2e-2 max-abs)."""
    from utttcompanion_amd import uTTTConfig, uTTTModel
    cfg = uTTTConfig(vocab_size=512, d_model=1024, n_layers=2, n_heads=16, n_kv_heads=4, d_ff_fast=256,
                     chunk_size=64, sliding_window_size=1024, max_seq_len=2048)
    torch.manual_seed(7)
    model = uTTTModel(cfg).eval().to(DEV).to(torch.bfloat16)
    model.fast_weight_pool.float()
    g = torch.Generator().manual_seed(44)
    ids = torch.randint(6, 512, (4, 1088), generator=g).to(DEV)
    state = model.init_fast_state(4, device=DEV, dtype=torch.float32, detach=True)
    with torch.no_grad():
        a = model.prefill_with_writes(ids, state)
        b = model.prefill_with_writes(ids, state, executor=False)
    torch.cuda.synchronize()
    assert torch.isfinite(a[0].float()).all()
    assert rel_err(a[0], b[0]) <= 2e-2
    for n, t, u in zip(NAMES, a[1], b[1]):
        assert max_abs(t, u) <= 2e-2, n
    assert rel_err(a[2], b[2]) <= 1e-2


def test_prefill_chunk_executor_interleaved_prefills_match_separate_runs():
    """Two bf16 prefills with deferred joins on stream pairs of their own (two models, so two
    chain streams), their chunk calls interleaved one by one: each equals the same prefill run
    alone, bit for bit.  The executor keeps no state between calls (each plan owns its events and
    hands its deferred state write to its own next call), so neither prefill waits on, or skips,
    the other's state write."""
    ma, _ = build(dtype=torch.bfloat16)
    mb, _ = build(dtype=torch.bfloat16, seed=9)
    ids_a, mask_a = ids_and_mask(2, 72, 256, seed=45)  # 4 chunks of 16 + a tail of 8: two plans
    ids_b, _ = ids_and_mask(2, 56, 256, seed=46)
    ids_a, mask_a, ids_b = ids_a.to(DEV), mask_a.to(DEV), ids_b.to(DEV)
    sa = ma.init_fast_state(2, device=DEV, dtype=torch.float32, detach=True)
    sb = mb.init_fast_state(2, device=DEV, dtype=torch.float32, detach=True)
    with torch.no_grad():
        alone = {"a": ma.prefill_with_writes(ids_a, sa, mask_a), "b": mb.prefill_with_writes(ids_b, sb)}
        torch.cuda.synchronize()
        s1, s2 = torch.cuda.Stream(), torch.cuda.Stream()
        live = {"a": (ma.prefill_steps(ids_a, sa, mask_a), s1), "b": (mb.prefill_steps(ids_b, sb), s2)}
        together, steps = {}, 0
        while live:
            for name in list(live):
                gen, st = live[name]
                with torch.cuda.stream(st):
                    try:
                        next(gen)
                        steps += 1
                    except StopIteration as done:
                        together[name] = done.value
                        del live[name]
        torch.cuda.synchronize()
    assert steps == 5 + 4
    for name in ("a", "b"):
        x, y = together[name], alone[name]
        assert torch.equal(x[0], y[0]), name
        for n, t, u in zip(NAMES, x[1], y[1]):
            assert torch.equal(t, u), (name, n)
        assert torch.equal(x[2], y[2]), name


def test_prefill_chunk_refuses_a_deferred_join_under_capture():
    """``uttt_prefill_chunk`` with ``defer_join`` or a ``wait_event`` on a capturing stream is
    refused before it enqueues anything (a deferred join would leave the chain stream unjoined
    at the end of the capture, and the event to wait for was recorded outside it); the capture
    then goes on and replays normally."""
    import ctypes as C
    from utttcompanion_amd import _native as N
    lib = N.load_library()
    ev = (C.c_void_p * 4)()
    N.check(lib.uttt_events_create(4, ev), "uttt_events_create")
    ch = N.ChunkChainArgs()
    ch.layers = 1
    calls = (N.PrefillLayerCalls * 1)()
    a = N.PrefillChunkArgs()
    a.n_layers, a.layers, a.chain = 1, C.cast(calls, C.POINTER(N.PrefillLayerCalls)), C.pointer(ch)
    a.events, a.n_events = C.cast(ev, C.POINTER(C.c_void_p)), 4
    side = torch.cuda.Stream()
    x = torch.zeros(4, device=DEV)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        a.defer_join = 1
        rc1 = lib.uttt_prefill_chunk(C.byref(a), torch.cuda.current_stream().cuda_stream, side.cuda_stream)
        err1 = lib.uttt_last_error()
        a.defer_join, a.wait_event = 0, ev[3]
        rc2 = lib.uttt_prefill_chunk(C.byref(a), torch.cuda.current_stream().cuda_stream, side.cuda_stream)
        err2 = lib.uttt_last_error()
        x.add_(1.0)
    assert rc1 == 1 and b"graph capture" in err1
    assert rc2 == 1 and b"graph capture" in err2
    graph.replay()
    graph.replay()
    torch.cuda.synchronize()
    assert torch.equal(x.cpu(), torch.full((4,), 2.0))
    N.check(lib.uttt_events_destroy(4, ev), "uttt_events_destroy")
