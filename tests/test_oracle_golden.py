"""The oracle reproduces the reference's golden vectors (tests/golden/*.npz) and schedule invariants.

The fixtures were written by ``tests/golden/make_golden.py`` from the reference's
``uTTTLayer``/``uTTTBlock``/``uTTTModel`` on seeded inputs; they pin the
compositions (chunk-first schedule, surprise aggregation, caches, decode) that
no closed form fixes.  The invariants below follow the reference's
``tests/test_shared_schedule_audit.py`` and ``tests/test_uttt_pipeline.py:192-230``.
"""
import json
import os

import numpy as np
import pytest
import torch

from oracle import uttt_math as om

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")
NAMES = ("w_up", "w_gate", "w_down", "s_up", "s_gate", "s_down")


def _load(name):
    with np.load(os.path.join(GOLDEN, name), allow_pickle=False) as data:
        return {k: data[k] for k in data.files}


def _meta():
    with open(os.path.join(GOLDEN, "golden.json")) as fh:
        return json.load(fh)


def _tiny_model():
    meta = _meta()
    t = meta["tiny_config"]
    cfg = om.OracleConfig(d_model=t["d_model"], n_layers=t["n_layers"], n_heads=t["n_heads"],
                          n_kv_heads=t["n_kv_heads"], d_ff_fast=t["d_ff_fast"],
                          sliding_window_size=t["sliding_window_size"], vocab_size=t["vocab_size"],
                          chunk_size=t["chunk_size"], base_inner_lr=t["base_inner_lr"],
                          base_weight_decay=t["base_weight_decay"], momentum_beta=t["momentum_beta"],
                          max_inner_grad_norm=t["max_inner_grad_norm"],
                          normalize_loss_by_dim=t["normalize_loss_by_dim"], rms_norm_eps=t["rms_norm_eps"])
    data = _load("model_tiny.npz")
    weights = {k[2:]: torch.from_numpy(v) for k, v in data.items() if k.startswith("w/")}
    return om.OracleModel(cfg, weights), data


def _close(actual, expected, atol=2e-5, rtol=2e-4):
    torch.testing.assert_close(torch.as_tensor(actual).float(), torch.from_numpy(np.asarray(expected)).float(),
                               atol=atol, rtol=rtol)


def _row(state, i):
    return om.OracleState(*(getattr(state, n)[i:i + 1].clone() for n in NAMES),
                          state.ln_weight, state.ln_bias, state.step)


def test_model_update_matches_reference_golden():
    model, g = _tiny_model()
    ids = torch.from_numpy(g["in/ids"])
    mask = torch.from_numpy(g["in/mask"])
    logits, state, per_layer, caches = model.forward(ids, None, mask, update_fast_weights=True)
    _close(logits, g["out/update_logits"])
    for n in NAMES:
        _close(getattr(state, n), g[f"out/update_state/{n}"], atol=1e-6, rtol=1e-5)
    _close(per_layer, g["out/update_layer_surprise"], atol=1e-6, rtol=1e-6)
    assert state.step == int(g["out/update_step"])
    for i, (k, v) in enumerate(caches):
        _close(k, g[f"out/update_kv{i}_k"])
        _close(v, g[f"out/update_kv{i}_v"])


def test_frozen_forward_and_greedy_decode_match_reference_golden():
    model, g = _tiny_model()
    ids = torch.from_numpy(g["in/ids"])
    mask = torch.from_numpy(g["in/mask"])
    _, state, _, _ = model.forward(ids, None, mask, update_fast_weights=True)
    frozen, _, _, _ = model.forward(ids[:1, :30], _row(state, 1), None, update_fast_weights=False)
    _close(frozen, g["out/frozen_logits"])
    tokens = model.greedy_generate(ids[:1, :30], _row(state, 1), 12)
    assert tokens == g["out/greedy_tokens"].tolist()


def test_test_time_update_pull_and_drift_match_reference_golden():
    model, g = _tiny_model()
    ids = torch.from_numpy(g["in/ids"])
    mask = torch.from_numpy(g["in/mask"])
    cand, surprise, layers = model.test_time_update(ids[1:2], model.init_state(1), mask[1:2])
    for n in NAMES:
        _close(getattr(cand, n), g[f"out/ttu_state/{n}"], atol=1e-6, rtol=1e-5)
    assert abs(surprise - float(g["out/ttu_surprise"])) < 1e-6
    _close(layers, g["out/ttu_layer_surprise"], atol=1e-6, rtol=1e-6)
    w0 = tuple(model.pool[n] for n in ("w_up_init", "w_gate_init", "w_down_init"))
    for key, ratio in (("pull_state", 0.35), ("pull_tight_state", 1e-4)):
        pulled = om.apply_elastic_pull((cand.w_up, cand.w_gate, cand.w_down), w0, 0.02, ratio)
        for n, t in zip(NAMES[:3], pulled):
            _close(t, g[f"out/{key}/{n}"], atol=1e-6, rtol=1e-5)
    pulled = om.apply_elastic_pull((cand.w_up, cand.w_gate, cand.w_down), w0, 0.02, 0.35)
    drift = om.compute_drift(pulled, w0)
    _close([drift[k] for k in _meta()["files"]["model_tiny.npz"]["drift_keys"]], g["out/drift"],
           atol=1e-5, rtol=1e-5)


def test_standalone_layer_and_cached_block_match_reference_golden():
    model, _ = _tiny_model()
    meta = _meta()["files"]["block_tiny.npz"]["layer_config"]
    b = _load("block_tiny.npz")
    lw = {k[2:]: torch.from_numpy(v) for k, v in b.items() if k.startswith("w/")}
    cfg = om.OracleConfig(d_model=meta["d_model"], n_layers=1, n_heads=meta["n_heads"],
                          n_kv_heads=meta["n_kv_heads"], d_ff_fast=64,
                          sliding_window_size=meta["window_size"], chunk_size=meta["chunk_size"],
                          base_inner_lr=meta["base_inner_lr"], base_weight_decay=meta["base_weight_decay"],
                          normalize_loss_by_dim=model.cfg.normalize_loss_by_dim,
                          momentum_beta=model.cfg.momentum_beta,
                          max_inner_grad_norm=model.cfg.max_inner_grad_norm)
    state = model.init_state(2)
    for n in ("s_up", "s_gate", "s_down"):
        setattr(state, n, torch.from_numpy(b[f"in/state/{n}"]).clone())
    x, x_prev, mask = (torch.from_numpy(b[k]) for k in ("in/x", "in/x_prev", "in/mask"))
    out, st, sur = om.uttt_layer_forward(x, lw, cfg, state.clone(), mask)
    _close(out, b["out/layer_out"])
    for n in NAMES:
        _close(getattr(st, n), b[f"out/layer_state/{n}"], atol=1e-6, rtol=1e-5)
    _close(sur, b["out/layer_surprise"], atol=1e-6, rtol=1e-6)
    cos, sin = om.rope_tables(cfg.head_dim, 256)
    _, _, _, cache = om.block_forward(x_prev, lw, cfg, cos, sin, state.clone(), update_fast_weights=False)
    bout, bst, bsur, bcache = om.block_forward(x, lw, cfg, cos, sin, state.clone(), mask, cache, 20)
    _close(bout, b["out/block_out"])
    for n in NAMES:
        _close(getattr(bst, n), b[f"out/block_state/{n}"], atol=1e-6, rtol=1e-5)
    _close(bsur, b["out/block_surprise"], atol=1e-6, rtol=1e-6)
    _close(bcache[0], b["out/block_cache_k"])
    _close(bcache[1], b["out/block_cache_v"])


# ---------------------------------------------------------------------------
# schedule invariants (reference tests/test_shared_schedule_audit.py)
# ---------------------------------------------------------------------------

def test_no_future_leakage_with_writes():
    model, g = _tiny_model()
    ids = torch.from_numpy(g["in/ids"])[:, :40]
    changed = ids.clone()
    changed[:, 20:] = (changed[:, 20:] + 37) % 128
    a, _, _, _ = model.forward(ids, None, None, update_fast_weights=True)
    b, _, _, _ = model.forward(changed, None, None, update_fast_weights=True)
    torch.testing.assert_close(a[:, :20], b[:, :20], atol=0, rtol=0)


def test_trailing_padding_chunks_keep_state_and_surprise():
    model, g = _tiny_model()
    ids = torch.from_numpy(g["in/ids"])[:, :24]
    mask = torch.ones(2, 24)
    mask[0, 19:] = 0
    padded = torch.cat([ids, torch.zeros(2, 16, dtype=ids.dtype)], dim=1)
    pmask = torch.cat([mask, torch.zeros(2, 16)], dim=1)
    _, st_a, sur_a, _ = model.forward(ids, None, mask, update_fast_weights=True)
    _, st_b, sur_b, _ = model.forward(padded, None, pmask, update_fast_weights=True)
    for n in NAMES:
        torch.testing.assert_close(getattr(st_a, n), getattr(st_b, n), atol=0, rtol=0)
    torch.testing.assert_close(sur_a, sur_b)


def test_split_prefill_with_caches_equals_single_pass():
    """Two forwards with carried KV caches and state == one forward (chunk-aligned split)."""
    model, g = _tiny_model()
    ids = torch.from_numpy(g["in/ids"])[:, :48]
    full, st_full, _, _ = model.forward(ids, None, None, update_fast_weights=True)
    first, st1, _, caches = model.forward(ids[:, :32], None, None, update_fast_weights=True)
    second, st2, _, _ = model.forward(ids[:, 32:], st1, None, caches, 32, True)
    torch.testing.assert_close(torch.cat([first, second], 1), full, atol=1e-5, rtol=1e-5)
    for n in NAMES:
        torch.testing.assert_close(getattr(st2, n), getattr(st_full, n), atol=1e-6, rtol=1e-5)


def test_deep_write_changes_only_next_chunk_reads():
    """A write by the last layer of chunk 0 is invisible to chunk 0 and visible to chunk 1."""
    model, g = _tiny_model()
    ids = torch.from_numpy(g["in/ids"])[:1, :32]
    base_logits, _, _, _ = model.forward(ids, None, None, update_fast_weights=True)
    w = model.layers[1]["uttt.w_v.weight"]
    model.layers[1]["uttt.w_v.weight"] = w + 0.05 * torch.randn_like(w)
    new_logits, _, _, _ = model.forward(ids, None, None, update_fast_weights=True)
    model.layers[1]["uttt.w_v.weight"] = w
    torch.testing.assert_close(new_logits[:, :16], base_logits[:, :16], atol=0, rtol=0)
    assert float((new_logits[:, 16:] - base_logits[:, 16:]).abs().max()) > 1e-7
