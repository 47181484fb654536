"""Host-side behaviour of the drop-in module API (CPU): the inference read caches and packs the
reference's serving code uses, and argument refusals that happen before any device work.

* ``SharedFastWeightPool.inference_read_weights`` (reference model/uttt_layer.py:648-668):
  the packed (B, D, 2F) copy equals the concatenated casts, is reused while the masters are
  unchanged and rebuilt after an in-place write (version bump); grad mode and inference
  tensors are refused.
* ``SlidingWindowAttention.prepare_for_inference`` / ``_packed_qkv`` (:1002-1024) and
  ``uTTTModel.prepare_for_inference`` (reference uttt_model.py:401-422).
* Writes take chunks of up to 512 tokens (the reference's shipped configs use chunk_size 128 /
  512); longer ones are refused at the write entry points (construction and frozen reads stay
  valid).
"""
import pytest
import torch

from utttcompanion_amd import FastWeightState, SharedFastWeightPool, SlidingWindowAttention, uTTTConfig, uTTTModel

TINY = dict(vocab_size=64, d_model=64, n_layers=2, n_heads=2, n_kv_heads=1, d_ff_fast=128, chunk_size=16,
            sliding_window_size=16)


def _state(b=2, d=64, f=128, seed=0):
    g = torch.Generator().manual_seed(seed)
    w = [torch.randn(b, d, f, generator=g), torch.randn(b, d, f, generator=g), torch.randn(b, f, d, generator=g)]
    return FastWeightState(*w, *(torch.zeros_like(t) for t in w), torch.ones(d), torch.zeros(d))


def test_inference_read_weights_packs_casts_and_reuses():
    pool = SharedFastWeightPool(64, 128)
    st = _state()
    with torch.no_grad():
        packed, down = pool.inference_read_weights(st, torch.bfloat16, "cpu")
        assert packed.shape == (2, 64, 256) and down.shape == (2, 128, 64)
        assert packed.dtype == down.dtype == torch.bfloat16
        assert torch.equal(packed, torch.cat((st.w_up.bfloat16(), st.w_gate.bfloat16()), dim=-1))
        assert torch.equal(down, st.w_down.bfloat16())
        again = pool.inference_read_weights(st, torch.bfloat16, "cpu")
        assert again[0] is packed and again[1] is down  # unchanged masters: the same copies
        st.w_gate.add_(1.0)  # an in-place write bumps the version: the copies are rebuilt
        fresh, _ = pool.inference_read_weights(st, torch.bfloat16, "cpu")
        assert fresh is not packed
        assert torch.equal(fresh[..., 128:], st.w_gate.bfloat16())
        other, _ = pool.inference_read_weights(st, torch.float16, "cpu")  # another dtype: rebuilt
        assert other.dtype == torch.float16


def test_inference_read_copies_follow_the_same_versions():
    pool = SharedFastWeightPool(64, 128)
    st = _state(seed=1)
    with torch.no_grad():
        up, gate, down = pool.inference_read_copies(st, torch.bfloat16, "cpu")
        assert all(t.is_contiguous() and t.dtype == torch.bfloat16 for t in (up, gate, down))
        assert torch.equal(gate, st.w_gate.bfloat16())
        assert pool.inference_read_copies(st, torch.bfloat16, "cpu")[0] is up
        st.w_up.mul_(2.0)
        assert torch.equal(pool.inference_read_copies(st, torch.bfloat16, "cpu")[0], st.w_up.bfloat16())


def test_inference_read_weights_refuses_grad_mode_and_inference_tensors():
    pool = SharedFastWeightPool(64, 128)
    st = _state()
    with torch.enable_grad(), pytest.raises(ValueError, match="no-grad"):
        pool.inference_read_weights(st, torch.bfloat16, "cpu")
    with torch.inference_mode():
        inf = _state()
    with torch.no_grad(), pytest.raises(ValueError, match="version-tracked"):
        pool.inference_read_weights(inf, torch.bfloat16, "cpu")
    assert st.to_state_dict().keys() == {"w_up", "w_gate", "w_down", "s_up", "s_gate", "s_down", "ln_weight",
                                         "ln_bias", "step", "last_surprise_loss", "surprise_history"}


def test_attention_packed_qkv_lifecycle():
    attn = SlidingWindowAttention(64, 4, 2, window_size=16).eval()
    assert attn._packed_qkv is None
    attn.prepare_for_inference()
    packed = attn._packed_qkv
    assert torch.equal(packed, torch.cat((attn.wq.weight, attn.wk.weight, attn.wv.weight), dim=0))
    assert attn.packed_qkv() is packed
    assert "_packed_qkv" not in attn.state_dict()  # not a checkpoint key
    with torch.no_grad():
        attn.wk.weight.add_(1.0)
    rebuilt = attn.packed_qkv()
    assert rebuilt is not packed and torch.equal(rebuilt[64:96], attn.wk.weight)
    attn.train()
    assert attn._packed_qkv is None and attn._packed_qkv_key is None


def test_model_prepare_for_inference():
    model = uTTTModel(uTTTConfig(**TINY))
    with pytest.raises(ValueError, match="eval"):
        model.prepare_for_inference()
    model.eval()
    with pytest.raises(ValueError, match="boolean"):
        model.prepare_for_inference(1)
    model._cuda_graph_decoder = object()
    model.prepare_for_inference(True)
    assert model.fast_weight_pool.fused_inference_readout is True
    assert all(b.attn._packed_qkv is not None for b in model.layers)
    assert model._cuda_graph_decoder is None  # the packs changed: the decode graph is dropped
    marker = model._cuda_graph_decoder = object()
    model.prepare_for_inference(True)  # nothing changed: the graph is kept
    assert model._cuda_graph_decoder is marker
    model.prepare_for_inference(False)
    assert model.fast_weight_pool.fused_inference_readout is False
    assert all(b.attn._packed_qkv is None for b in model.layers)
    assert model._cuda_graph_decoder is None
    assert set(model.state_dict()) == set(uTTTModel(uTTTConfig(**TINY)).state_dict())


def test_write_chunk_limit_takes_the_reference_configs():
    from utttcompanion_amd.layer import MAX_WRITE_CHUNK, require_write_chunk
    assert MAX_WRITE_CHUNK == 512
    for chunk in (1, 64, 128, 512):  # 128 / 512: configs/5090_config.yaml:31, 5090_pretrain_20261029.yaml:28
        require_write_chunk(chunk)
    for chunk in (0, 513, 1024):
        with pytest.raises(ValueError, match=f"chunk_size={chunk}"):
            require_write_chunk(chunk)


@pytest.mark.parametrize("chunk", [513, 1024])
def test_writes_with_longer_chunks_are_refused_before_any_work(chunk):
    from utttcompanion_amd.evolve import ragged_test_time_update
    model = uTTTModel(uTTTConfig(**dict(TINY, chunk_size=chunk))).eval()  # constructs: frozen reads are valid
    ids = torch.randint(6, 64, (1, 40))
    with pytest.raises(ValueError, match=f"chunk_size={chunk}"):
        model(ids, update_fast_weights=True)
    with pytest.raises(ValueError, match=f"chunk_size={chunk}"):
        model.test_time_update(ids, model.init_fast_state(1))
    with pytest.raises(ValueError, match=f"chunk_size={chunk}"):
        ragged_test_time_update(model, [ids[0]], [model.init_fast_state(1)])
    block = model.layers[0]
    with pytest.raises(ValueError, match=f"chunk_size={chunk}"):
        block.uttt(torch.zeros(1, 40, 64), model.fast_weight_pool, model.init_fast_state(1))


def test_stream_generate_refuses_speculative_drafts():
    model = uTTTModel(uTTTConfig(**TINY)).eval()
    gen = model.stream_generate(torch.tensor([[7, 8]]), model.init_fast_state(1), speculative_draft_k=2)
    with pytest.raises(ValueError, match="self-speculative"):
        next(gen)
