"""The on-disk payloads a deployment loads into this path.

``tests/golden/base_tiny.pt`` is a base checkpoint laid out as the reference's trainer writes
it (train_5090.py:918-930: ``config``, ``slow_weights``, ``init_fast_weights`` ...) and
``tests/golden/persona_tiny.pt`` a persona file laid out as its checkpoint manager writes it
(engine/checkpoint_manager.py:547-557: ``fast_state`` = ``FastWeightState.to_state_dict()``),
both written from the reference's own modules by ``tests/golden/make_golden.py``.  They load
with the weights-only loader (nothing in them executes) into ``uTTTConfig.from_dict`` +
``uTTTModel.load_dual_base_state`` (reference uttt_model.py:383-394) and
``FastWeightState.from_state_dict`` (reference uttt_layer.py:181-204).  On the GPU the loaded
model reproduces the reference's logits and write from that persona (fp32, <= 1e-5 relative).
"""
from pathlib import Path

import numpy as np
import pytest
import torch

from utttcompanion_amd import FastWeightState, uTTTConfig, uTTTModel

GOLDEN = Path(__file__).resolve().parent / "golden"
NAMES = ("w_up", "w_gate", "w_down", "s_up", "s_gate", "s_down")


def _load(name):
    return torch.load(GOLDEN / name, map_location="cpu", weights_only=True)


def load_base():
    payload = _load("base_tiny.pt")
    model = uTTTModel(uTTTConfig.from_dict(payload["config"])).eval()
    model.load_dual_base_state(payload["slow_weights"], payload["init_fast_weights"])
    return model, payload


def load_persona():
    payload = _load("persona_tiny.pt")
    return FastWeightState.from_state_dict(payload["fast_state"]), payload


def test_base_checkpoint_loads_every_weight():
    model, payload = load_base()
    assert payload["checkpoint_type"] == "uTTT_Base_Checkpoint"
    sd = model.state_dict()
    for k, v in payload["slow_weights"].items():
        assert torch.equal(sd[k], v), k
    for k, v in payload["init_fast_weights"].items():
        assert torch.equal(sd["fast_weight_pool." + k], v), k
    assert len(payload["slow_weights"]) + len(payload["init_fast_weights"]) == len(sd)
    cfg = payload["config"]
    assert (model.config.d_model, model.config.n_layers, model.config.chunk_size) == \
        (cfg["d_model"], cfg["n_layers"], cfg["chunk_size"])
    assert model.lm_head.weight is model.tok_embeddings.weight  # tied, as the reference keeps it


def test_persona_state_loads_and_round_trips():
    st, payload = load_persona()
    assert payload["checkpoint_type"] == "uTTT_User_Persona_State"
    ref = np.load(GOLDEN / "formats_tiny.npz")
    for n in NAMES:
        assert torch.equal(getattr(st, n), torch.from_numpy(ref[f"out/persona_state/{n}"])), n
        assert getattr(st, n).dtype == torch.float32
    fs = payload["fast_state"]
    assert st.step == fs["step"] > 0 and st.last_surprise_loss == fs["last_surprise_loss"]
    assert st.surprise_history == list(fs["surprise_history"])
    mine = st.to_state_dict()
    assert set(mine) == set(fs)
    for k, v in fs.items():
        assert torch.equal(mine[k], v) if isinstance(v, torch.Tensor) else mine[k] == v, k


def test_state_dict_payload_survives_the_weights_only_loader(tmp_path):
    st, _ = load_persona()
    torch.save({"fast_state": st.to_state_dict()}, tmp_path / "p.pt")
    back = FastWeightState.from_state_dict(torch.load(tmp_path / "p.pt", weights_only=True)["fast_state"])
    for n in NAMES + ("ln_weight", "ln_bias"):
        assert torch.equal(getattr(back, n), getattr(st, n))
    assert back.step == st.step


@pytest.mark.gpu
def test_loaded_model_reproduces_reference_logits_on_the_persona():
    dev = "cuda"
    model, _ = load_base()
    model = model.to(dev)
    st, _ = load_persona()
    st = st.to(device=dev)
    ref = np.load(GOLDEN / "formats_tiny.npz")
    ids = torch.from_numpy(ref["in/ids"]).to(dev)

    def rel(a, e):
        a, e = a.detach().double().cpu(), torch.from_numpy(e).double()
        return (a - e).abs().max().item() / max(e.abs().max().item(), 1e-30)

    frozen = model(ids, fast_state=st, update_fast_weights=False)
    assert rel(frozen.logits, ref["out/frozen_logits"]) <= 1e-5
    written = model(ids, fast_state=st, update_fast_weights=True)
    assert rel(written.logits, ref["out/update_logits"]) <= 1e-5
    for n in NAMES:
        assert rel(getattr(written.fast_state, n), ref[f"out/update_state/{n}"]) <= 1e-5, n
    assert written.fast_state.step == int(ref["out/update_step"])
