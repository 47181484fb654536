"""Write golden vectors for the compositions of the uTTT hot path.

Run once, in the build container, with the reference checkout mounted at
``/root/reference`` (``python tests/golden/make_golden.py``).  It imports the
reference's ``model.uttt_layer`` / ``model.uttt_model`` and records, for small
seeded inputs, the outputs that no closed form pins:

* ``uTTTLayer.forward`` standalone (each chunk reads its own pre-update W);
* ``uTTTBlock.forward`` with an incoming KV cache and start position;
* ``uTTTModel.forward(update_fast_weights=True)`` -- the chunk-first shared
  schedule with right padding, per-layer surprise aggregation and step count;
* ``uTTTModel.forward(update_fast_weights=False)`` and greedy ``stream_generate``;
* ``uTTTModel.test_time_update`` followed by ``apply_elastic_pull`` and
  ``compute_drift`` (the personalizer's step 2-3 arithmetic);
* (``formats``) the two on-disk payloads a deployment loads: a base checkpoint laid out as
  ``train_5090.py:918-930`` writes it (``slow_weights`` / ``init_fast_weights`` from the
  reference model's ``state_dict``) and a persona file laid out as
  ``engine/checkpoint_manager.py:547-557`` writes it (``fast_state`` from the reference's
  ``FastWeightState.to_state_dict``), with the reference's logits on them.

Weights are drawn here from a seeded generator and loaded into the reference
modules, so the fixtures hold every input explicitly: nothing depends on the
reference's parameter initialisation order.  Outputs are stored in ``.npz``
files (read with ``numpy.load(allow_pickle=False)``) beside a JSON description.
The GPU box never runs this script; the fixtures travel instead.
"""

from __future__ import annotations

import json
import os
import sys
from pathlib import Path

import numpy as np
import torch

HERE = Path(__file__).resolve().parent
REFERENCE = Path(os.environ.get("UTTT_REFERENCE", "/root/reference"))

TINY = dict(vocab_size=128, d_model=32, n_layers=2, n_heads=2, n_kv_heads=1, d_ff_fast=64,
            chunk_size=16, sliding_window_size=24, max_seq_len=256, base_inner_lr=0.05,
            base_weight_decay=0.01, momentum_beta=0.9, max_inner_grad_norm=1.0,
            normalize_loss_by_dim=True, gradient_checkpointing=False, rms_norm_eps=1e-5)


def draw_weights(model: torch.nn.Module, seed: int) -> dict:
    """Seeded weights for every parameter of ``model`` (by state_dict key)."""
    gen = torch.Generator().manual_seed(seed)
    out = {}
    for name, tensor in model.state_dict().items():
        if name == "lm_head.weight":
            continue  # tied to tok_embeddings.weight
        shape = tuple(tensor.shape)
        if name.endswith(("norm.weight", "ln_weight")):
            value = 1.0 + 0.1 * torch.randn(shape, generator=gen)
        elif name.endswith("ln_bias"):
            value = 0.05 * torch.randn(shape, generator=gen)
        elif name.endswith(("w_up_init", "w_gate_init")):
            value = torch.randn(shape, generator=gen) / shape[0] ** 0.5
        elif name.endswith("w_down_init"):
            value = 0.3 * torch.randn(shape, generator=gen) / shape[0] ** 0.5
        elif name.endswith(("w_eta.weight", "w_alpha.weight")):
            value = 0.2 * torch.randn(shape, generator=gen)
        elif name.endswith("w_eta.bias"):
            value = torch.zeros(shape)
        elif name.endswith("w_alpha.bias"):
            value = torch.full(shape, -1.386)
        elif name == "tok_embeddings.weight":
            value = torch.randn(shape, generator=gen)
        else:
            value = 0.08 * torch.randn(shape, generator=gen)
        out[name] = value.float()
    return out


def load_into(model, weights):
    sd = dict(weights)
    sd["lm_head.weight"] = sd["tok_embeddings.weight"]
    model.load_state_dict(sd, strict=True)


def state_arrays(prefix: str, state) -> dict:
    return {f"{prefix}/{n}": getattr(state, n).detach().float().numpy()
            for n in ("w_up", "w_gate", "w_down", "s_up", "s_gate", "s_down")}


# the format fixtures also run on the GPU: d_model and d_ff multiples of 64, head_dim 64
FORMAT_TINY = dict(TINY, d_model=128, n_layers=1, n_heads=2, n_kv_heads=1, d_ff_fast=64)


def write_formats() -> dict:
    """base_tiny.pt, persona_tiny.pt and formats_tiny.npz (see the module docstring)."""
    sys.path.insert(0, str(REFERENCE))
    from model.uttt_model import uTTTConfig, uTTTModel  # noqa: E402

    torch.set_num_threads(1)
    cfg = uTTTConfig(**FORMAT_TINY)
    model = uTTTModel(cfg).eval()
    load_into(model, draw_weights(model, 20261202))
    state = model.state_dict()
    prefix = "fast_weight_pool."
    base = {
        "checkpoint_type": "uTTT_Base_Checkpoint", "version": "1.0.0", "step": 1234,
        "timestamp": "2026-12-02T00:00:00Z", "config": cfg.to_dict(),
        "slow_weights": {k: v.detach().clone() for k, v in state.items() if not k.startswith(prefix)},
        "init_fast_weights": {k[len(prefix):]: v.detach().clone() for k, v in state.items() if k.startswith(prefix)},
        "metrics": {"loss": 1.5},
    }
    torch.save(base, HERE / "base_tiny.pt")
    gen = torch.Generator().manual_seed(17)
    turn = torch.randint(6, TINY["vocab_size"], (1, 40), generator=gen)
    ids = torch.randint(6, TINY["vocab_size"], (1, 33), generator=gen)
    with torch.no_grad():
        persona_state, _, _ = model.test_time_update(turn, model.init_fast_state(detach=True))
        persona = {
            "checkpoint_type": "uTTT_User_Persona_State", "version": "1.0.0", "user_id": "alice",
            "base_signature": "tiny", "base_fingerprint": "tiny", "timestamp": "2026-12-02T00:00:00Z",
            "fast_state": persona_state.to_state_dict(),
            "drift_metrics": model.fast_weight_pool.compute_drift(persona_state),
            "metadata": {"user_id": "alice", "turns": 1},
        }
        torch.save(persona, HERE / "persona_tiny.pt")
        frozen = model(ids, fast_state=persona_state, update_fast_weights=False)
        written = model(ids, fast_state=persona_state, update_fast_weights=True)
    arrays = {"in/turn": turn.numpy(), "in/ids": ids.numpy(),
              "out/frozen_logits": frozen.logits.float().numpy(),
              "out/update_logits": written.logits.float().numpy()}
    arrays.update(state_arrays("out/persona_state", persona_state))
    arrays.update(state_arrays("out/update_state", written.fast_state))
    arrays["out/update_step"] = np.array(written.fast_state.step)
    np.savez_compressed(HERE / "formats_tiny.npz", **arrays)
    return {
        "base_tiny.pt": {"what": "base checkpoint payload (train_5090.py:918-930 layout), weights seed 20261202; "
                                 "load with torch.load(weights_only=True)", "config": FORMAT_TINY},
        "persona_tiny.pt": {"what": "persona payload (checkpoint_manager.py:547-557 layout): fast_state = "
                                    "FastWeightState.to_state_dict() after test_time_update of in/turn"},
        "formats_tiny.npz": {"what": "reference frozen forward and forward with writes of in/ids (1 x 33) "
                                     "from the persona state, and the persona state itself"},
    }


def main() -> None:
    if sys.argv[1:] == ["formats"]:  # only the on-disk payloads, merged into golden.json
        meta = json.loads((HERE / "golden.json").read_text())
        meta["files"].update(write_formats())
        (HERE / "golden.json").write_text(json.dumps(meta, indent=1) + "\n")
        print("wrote the on-disk format fixtures")
        return
    sys.path.insert(0, str(REFERENCE))
    from model.uttt_layer import uTTTBlock, uTTTLayer  # noqa: E402
    from model.uttt_model import uTTTConfig, uTTTModel  # noqa: E402

    torch.set_num_threads(1)
    meta = {"tiny_config": TINY, "files": {}}

    # ---- model: chunk-first schedule with writes, padding, frozen decode ----
    cfg = uTTTConfig(**TINY)
    model = uTTTModel(cfg).eval()
    weights = draw_weights(model, 20261201)
    load_into(model, weights)
    gen = torch.Generator().manual_seed(7)
    ids = torch.randint(6, TINY["vocab_size"], (2, 56), generator=gen)
    mask = torch.ones(2, 56)
    mask[1, 45:] = 0.0
    arrays = {f"w/{k}": v.numpy() for k, v in weights.items()}
    arrays["in/ids"] = ids.numpy()
    arrays["in/mask"] = mask.numpy()
    with torch.no_grad():
        out = model(ids, attention_mask=mask, update_fast_weights=True)
        arrays["out/update_logits"] = out.logits.float().numpy()
        arrays.update(state_arrays("out/update_state", out.fast_state))
        arrays["out/update_layer_surprise"] = np.array(out.layer_surprise_losses, dtype=np.float64)
        arrays["out/update_step"] = np.array(out.fast_state.step)
        arrays["out/update_surprise"] = np.array(float(out.surprise_loss))
        for i, (k, v) in enumerate(out.kv_caches):
            arrays[f"out/update_kv{i}_k"] = k.float().numpy()
            arrays[f"out/update_kv{i}_v"] = v.float().numpy()

        # frozen readout through the updated state + greedy decode
        frozen = model(ids[:1, :30], fast_state=_row(out.fast_state, 1), update_fast_weights=False)
        arrays["out/frozen_logits"] = frozen.logits.float().numpy()
        tokens = list(model.stream_generate(ids[:1, :30], _row(out.fast_state, 1), max_new_tokens=12,
                                            temperature=0.0, eos_token_id=None))
        arrays["out/greedy_tokens"] = np.array(tokens, dtype=np.int64)

        # test_time_update + elastic pull + drift (personalizer steps 2-3)
        base = model.init_fast_state(detach=True)
        cand, surprise, layers = model.test_time_update(ids[1:2], base, attention_mask=mask[1:2])
        arrays.update(state_arrays("out/ttu_state", cand))
        arrays["out/ttu_surprise"] = np.array(surprise, dtype=np.float64)
        arrays["out/ttu_layer_surprise"] = np.array(layers, dtype=np.float64)
        pulled = model.fast_weight_pool.apply_elastic_pull(cand, anchor_lambda=0.02, max_drift_ratio=0.35)
        arrays.update(state_arrays("out/pull_state", pulled))
        tight = model.fast_weight_pool.apply_elastic_pull(cand, anchor_lambda=0.02, max_drift_ratio=1e-4)
        arrays.update(state_arrays("out/pull_tight_state", tight))
        drift = model.fast_weight_pool.compute_drift(pulled)
        arrays["out/drift"] = np.array([drift[k] for k in DRIFT_KEYS], dtype=np.float64)
    np.savez_compressed(HERE / "model_tiny.npz", **arrays)
    meta["files"]["model_tiny.npz"] = {
        "what": "uTTTModel forward with writes (B=2, T=56, row 1 padded from 45), frozen forward, "
                "greedy stream_generate (12 tokens), test_time_update, elastic pull (0.35 and 1e-4 "
                "drift ceilings, lambda 0.02), compute_drift",
        "drift_keys": DRIFT_KEYS, "seed_weights": 20261201, "seed_ids": 7}

    # ---- standalone layer and block with an incoming cache ----
    layer_cfg = dict(d_model=32, n_heads=2, n_kv_heads=1, window_size=24, chunk_size=16,
                     base_inner_lr=0.05, base_weight_decay=0.01, max_seq_len=256)
    torch.manual_seed(0)
    block = uTTTBlock(layer_idx=0, **layer_cfg).eval()
    bweights = {k: v for k, v in draw_weights(block, 99).items()}
    block.load_state_dict(bweights, strict=True)
    pool = model.fast_weight_pool
    gen = torch.Generator().manual_seed(11)
    x = torch.randn(2, 40, 32, generator=gen)
    x_prev = torch.randn(2, 20, 32, generator=gen)
    bmask = torch.ones(2, 40)
    bmask[0, 33:] = 0.0
    state = pool.init_state(batch_size=2, detach=True)
    for name in ("s_up", "s_gate", "s_down"):
        getattr(state, name).copy_(0.01 * torch.randn(getattr(state, name).shape, generator=gen))
    barr = {f"w/{k}": v.numpy() for k, v in bweights.items()}
    barr.update({"in/x": x.numpy(), "in/x_prev": x_prev.numpy(), "in/mask": bmask.numpy()})
    barr.update({f"in/state/{n}": getattr(state, n).numpy()
                 for n in ("s_up", "s_gate", "s_down")})
    with torch.no_grad():
        lout, lstate, lsur = block.uttt(x, pool, state.clone(detach=True), attention_mask=bmask)
        barr["out/layer_out"] = lout.numpy()
        barr.update(state_arrays("out/layer_state", lstate))
        barr["out/layer_surprise"] = np.array(float(lsur))
        _, _, _, cache = block(x_prev, pool, state.clone(detach=True), update_fast_weights=False)
        bout, bstate, bsur, bcache = block(x, pool, state.clone(detach=True), attention_mask=bmask,
                                           kv_cache=cache, start_pos=20)
        barr["out/block_out"] = bout.numpy()
        barr.update(state_arrays("out/block_state", bstate))
        barr["out/block_surprise"] = np.array(float(bsur))
        barr["out/block_cache_k"] = bcache[0].numpy()
        barr["out/block_cache_v"] = bcache[1].numpy()
    np.savez_compressed(HERE / "block_tiny.npz", **barr)
    meta["files"]["block_tiny.npz"] = {
        "what": "uTTTLayer.forward standalone (B=2, T=40, row 0 padded from 33; pool from model_tiny) "
                "and uTTTBlock.forward with a 20-token frozen-prefill cache at start_pos 20",
        "layer_config": layer_cfg, "seed_weights": 99, "seed_inputs": 11}

    meta["files"].update(write_formats())
    import platform
    meta["generated_with"] = {"torch": torch.__version__, "python": platform.python_version()}
    (HERE / "golden.json").write_text(json.dumps(meta, indent=1) + "\n")
    print("wrote", sorted(meta["files"]))


DRIFT_KEYS = ["drift_frobenius", "base_frobenius", "drift_pct", "w_up_drift", "w_gate_drift",
              "w_down_drift", "w_up_drift_pct", "w_gate_drift_pct", "w_down_drift_pct"]


def _row(state, index):
    """Batch row ``index`` of a state as a detached batch-1 state."""
    from model.uttt_layer import FastWeightState
    return FastWeightState(**{n: getattr(state, n)[index:index + 1].detach().clone()
                              for n in ("w_up", "w_gate", "w_down", "s_up", "s_gate", "s_down")},
                           ln_weight=state.ln_weight.detach().clone(),
                           ln_bias=state.ln_bias.detach().clone(), step=state.step)


if __name__ == "__main__":
    main()
