"""GPU parity of ``uttt_linear`` (out = x W^T (+ residual), bf16 operands, fp32 accumulation)
against a float32 product of the same bf16 operands rounded once to bf16.

Tolerance (north star, bf16 <= 2e-2 max-abs): per element |gpu - ref| <= 2^-8 |ref| + 1e-3 (one
bf16 rounding of an fp32 sum whose order differs from the reference's).
"""
import pytest
import torch

pytestmark = pytest.mark.gpu
DEV = "cuda"


def ref_linear(x, w, residual=None):
    y = x.float() @ w.float().t()
    if residual is not None:
        y = y + residual.float()
    return y


def check(got, ref):
    err = (got.float() - ref).abs()
    bound = ref.abs() * 2.0 ** -8 + 1e-3
    assert bool((err <= bound).all()), f"max err {err.max().item():.3e}"
    assert err.max().item() <= 2e-2


# (m, n, k): config-3 chunk shapes (256 rows of d_model 2048: packed uTTT projections 3 D + 2,
# packed QKV, the output / residual projections), config-2 (512 rows of 768), ragged m and n
SHAPES = [(256, 6146, 2048), (256, 3072, 2048), (256, 2048, 2048), (512, 2306, 768), (512, 768, 768),
          (100, 70, 128), (1, 33, 64), (200, 130, 192), (4096, 256, 512)]


@pytest.mark.parametrize("shape", SHAPES, ids=[f"m{m}-n{n}-k{k}" for m, n, k in SHAPES])
@pytest.mark.parametrize("with_residual", [False, True], ids=["plain", "residual"])
def test_linear_matches_fp32_product(shape, with_residual):
    from utttcompanion_amd import kernels as K
    m, n, k = shape
    print(f"linear m {m} n {n} k {k} residual {with_residual}", flush=True)
    g = torch.Generator().manual_seed(m + n + k)
    x = torch.randn(m, k, generator=g).bfloat16().to(DEV)
    w = (torch.randn(n, k, generator=g) / k ** 0.5).bfloat16().to(DEV)
    r = torch.randn(m, n, generator=g).bfloat16().to(DEV) if with_residual else None
    got = K.linear(x, w, residual=r)
    torch.cuda.synchronize()
    check(got, ref_linear(x, w, r))


def test_linear_strided_operands_and_in_place_residual():
    """x and W as column slices of wider tensors (row strides > k), out a column slice of a wider
    buffer, the residual the output itself (h += x W^T)."""
    from utttcompanion_amd import kernels as K
    g = torch.Generator().manual_seed(5)
    xb = torch.randn(300, 1088, generator=g).bfloat16().to(DEV)
    wb = (torch.randn(500, 1032, generator=g) / 32).bfloat16().to(DEV)
    x, w = xb[:, 64:1024], wb[:, 8:968]
    hb = torch.randn(300, 520, generator=g).bfloat16().to(DEV)
    h = hb[:, 8:508]
    before = h.clone()
    spare = hb[:, :8].clone(), hb[:, 508:].clone()
    K.linear(x, w, out=h, residual=h)
    torch.cuda.synchronize()
    check(h, ref_linear(x, w, before))
    assert torch.equal(hb[:, :8], spare[0]) and torch.equal(hb[:, 508:], spare[1])


def test_linear_refuses_unsupported_operands():
    from utttcompanion_amd import kernels as K
    x = torch.randn(8, 96, device=DEV).bfloat16()
    w = torch.randn(16, 96, device=DEV).bfloat16()
    assert not K.linear_fits(x, w)
    with pytest.raises(RuntimeError, match="multiple of 64"):
        K.linear(x, w)
    with pytest.raises(ValueError, match="bf16"):
        K.linear(x.float(), w.float())
