"""``uttt_chunk_update_noalloc`` (no workspace argument, no allocation) against
``uttt_chunk_update`` with a caller workspace.

The no-alloc entry point works in the library's device-resident scratch array, which keeps the
previous call's contents.  Two calls in a row, the second with a smaller input (fewer rows, a
tail chunk, a mask), must each give exactly what the workspace entry point gives; that entry
point's workspace is filled with NaN first, so neither path can lean on cleared memory.  fp32 and
bf16 activations; shapes past the scratch size are refused before any launch.
"""
import pytest
import torch

from test_gpu_kernels import make_chunk, to_dev

pytestmark = pytest.mark.gpu
DEV = "cuda"
NAMES = ("readout", "w_up", "w_gate", "w_down", "s_up", "s_gate", "s_down", "surprise")


def _prepare(b, c, d, f, dtype, seed, masked, workspace=None):
    from utttcompanion_amd import kernels as K
    q, k, v, eta, alpha, w, s, ln_w, ln_b = make_chunk(b, c, d, f, seed=seed)
    mask = None
    if masked:
        mask = torch.ones(b, c)
        mask[0, c // 2:] = 0
    acts = [t.to(dtype) for t in (q, k, v, eta, alpha)]
    dev = to_dev(*acts, *w, *s, ln_w, ln_b, mask)
    return K.prepare_chunk_update(*dev[:13], dev[13], 0.9, 1.0, True, 1e-5, workspace=workspace)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_noalloc_update_equals_workspace_update_on_two_calls(dtype):
    from utttcompanion_amd import _native as N
    lib = N.load_library()
    code = N.DTYPE_BF16 if dtype == torch.bfloat16 else N.DTYPE_F32
    cases = [dict(b=4, c=64, d=512, f=1024, masked=False, seed=1),  # config-1 width, four rows
             dict(b=2, c=40, d=256, f=512, masked=True, seed=2)]    # smaller: tail chunk and mask
    for case in cases:
        b, c, d, f = case["b"], case["c"], case["d"], case["f"]
        print(f"no-alloc update {dtype} {case}", flush=True)
        nbytes = lib.uttt_chunk_update_workspace(b, d, f, code)
        ws = torch.full((nbytes // 4 + 1,), float("nan"), device=DEV).view(torch.uint8)
        with torch.no_grad():
            ref = _prepare(b, c, d, f, dtype, case["seed"], case["masked"], workspace=ws).launch()
            got = _prepare(b, c, d, f, dtype, case["seed"], case["masked"]).launch_noalloc()
        torch.cuda.synchronize()
        for name, a, e in zip(NAMES, got, ref):
            assert torch.isfinite(e).all(), name
            assert torch.equal(a, e), (case, name)


def test_noalloc_update_refuses_shapes_past_the_scratch():
    from utttcompanion_amd import _native as N
    lib = N.load_library()
    b, d, f = 16, 2048, 5504  # config 5: about 106 MiB of workspace
    assert lib.uttt_chunk_update_workspace(b, d, f, N.DTYPE_BF16) > (64 << 20)
    prep = _prepare(1, 8, 64, 64, torch.bfloat16, 3, False)
    prep.args.batch, prep.args.d_model, prep.args.d_ff = b, d, f  # refused before any pointer is read
    with pytest.raises(RuntimeError, match="device-resident scratch"):
        prep.launch_noalloc()
