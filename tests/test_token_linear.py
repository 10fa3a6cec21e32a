"""TokenLinearFn: the block's training projections (nn.Linear, block.py:65-81, with out_proj's residual add,
block.py:229) with the weight gradient dW = dY^T X split over token slabs on the GPU (each slab's product in
fp32, the slabs summed in a fixed order by cdssm_slab_sum) and the bias gradient by cdssm_col_sum.

CPU (fp64; one product for dW there): output, dx, dW, db and the residual's gradient against autograd
through F.linear + add.  GPU: bf16 and fp32 at the block's shapes (T = B L = 16384; out_proj 1024 x 1024,
readout_proj 1024 x 256, gate_proj 336 x 1024 with bias: 8 slabs; in_proj 3328 x 1024 with bias: 2 slabs)
against fp64 autograd on the same rounded inputs: fp32 <= 1e-5, bf16 <= 1e-2 normwise (the bf16 rounding of
each output), and bit-identical repeats.
"""

import pytest
import torch

from _gpu_util import DEV, log, rel


def run_fn(x, w, b, r, g):
    from cdssm_hip.lm import TokenLinearFn
    x, w = x.clone().requires_grad_(True), w.clone().requires_grad_(True)
    b = b.clone().requires_grad_(True) if b is not None else None
    r = r.clone().requires_grad_(True) if r is not None else None
    y = TokenLinearFn.apply(x, w, b, r)
    y.backward(g)
    return y, x.grad, w.grad, (b.grad if b is not None else None), (r.grad if r is not None else None)


def run_ref(x, w, b, r, g):
    x, w = x.double().requires_grad_(True), w.double().requires_grad_(True)
    b = b.double().requires_grad_(True) if b is not None else None
    r = r.double().requires_grad_(True) if r is not None else None
    y = torch.nn.functional.linear(x, w, b)
    if r is not None:
        y = y + r
    y.backward(g.double())
    return y, x.grad, w.grad, (b.grad if b is not None else None), (r.grad if r is not None else None)


def draw(B, L, O, I, bias, residual, dtype, device, seed=0):
    gen = torch.Generator().manual_seed(seed)
    t = lambda *s: torch.randn(*s, generator=gen).to(dtype).to(device)  # noqa: E731
    return (t(B, L, I), 0.05 * t(O, I), t(O) if bias else None, t(B, L, O) if residual else None, t(B, L, O))


@pytest.mark.parametrize("B,L,O,I,bias,residual", [(8, 2048, 64, 32, True, False), (8, 2048, 48, 40, False, True),
                                                    (2, 75, 7, 5, True, False)])
def test_token_linear_matches_linear_fp64_cpu(B, L, O, I, bias, residual):
    from cdssm_hip.lm import _wgrad_slabs
    x, w, b, r, g = draw(B, L, O, I, bias, residual, torch.float64, "cpu")
    got, want = run_fn(x, w, b, r, g), run_ref(x, w, b, r, g)
    log(f"[token linear cpu] T{B * L} {O}x{I}: slabs {_wgrad_slabs(B * L, O, I)}")
    for n, a, e in zip(("y", "dx", "dW", "db", "dres"), got, want):
        assert (a is None) == (e is None), n
        if a is not None:
            assert rel(a, e) <= 1e-12, n


@pytest.mark.parametrize("O,bias", [(3104, True), (3104, False), (3328, True), (1040, True)])
def test_padded_linear_matches_linear_fp64_cpu(O, bias):
    """padded_linear: the product with the output features rounded up to a multiple of 256 (zero weight rows,
    O >= 2048) and sliced back equals F.linear; the result is a column slice (row stride O_pad)."""
    from cdssm_hip.lm import _padded_features, padded_linear
    gen = torch.Generator().manual_seed(2)
    x = torch.randn(70, 96, generator=gen, dtype=torch.float64)
    w = torch.randn(O, 96, generator=gen, dtype=torch.float64)
    b = torch.randn(O, generator=gen, dtype=torch.float64) if bias else None
    y = padded_linear(x, w, b)
    assert y.shape == (70, O) and y.stride(0) == _padded_features(O)
    assert _padded_features(3104) == 3328 and _padded_features(3328) == 3328 and _padded_features(1040) == 1040
    assert torch.equal(y, torch.nn.functional.linear(x, w, b))


@pytest.mark.gpu
@pytest.mark.parametrize("name,O,I,bias,residual,dtype", [
    ("out_proj_bf16", 1024, 1024, False, True, torch.bfloat16),
    ("readout_proj_bf16", 1024, 256, False, False, torch.bfloat16),
    ("gate_proj_bf16", 336, 1024, True, False, torch.bfloat16),
    ("in_proj_bf16", 3328, 1024, True, False, torch.bfloat16),
    ("in_proj_state2_padded_bf16", 3104, 1024, True, False, torch.bfloat16),
    ("out_proj_fp32", 1024, 1024, False, True, torch.float32),
    ("odd_tokens_single_product_bf16", 1024, 1024, True, False, torch.bfloat16),
])
def test_token_linear_gpu_matches_fp64(name, O, I, bias, residual, dtype):
    from cdssm_hip.lm import _wgrad_slabs
    B, L = (8, 2048) if not name.startswith("odd") else (3, 2731)  # 8193 tokens: one product, no slabs
    want_slabs = 1 if name.startswith("odd") else (8 if O * I <= 1 << 20 else 2)
    assert _wgrad_slabs(B * L, O, I) == want_slabs
    log(f"[token linear gpu] {name}: T{B * L} {O}x{I} slabs {want_slabs}")
    x, w, b, r, g = draw(B, L, O, I, bias, residual, dtype, DEV, seed=1)
    got = run_fn(x, w, b, r, g)
    again = run_fn(x, w, b, r, g)
    torch.cuda.synchronize()
    want = run_ref(*[t.cpu() if t is not None else None for t in (x, w, b, r, g)])
    tol = 1e-5 if dtype == torch.float32 else 1e-2
    errs = {}
    for n, a, a2, e in zip(("y", "dx", "dW", "db", "dres"), got, again, want):
        assert (a is None) == (e is None), n
        if a is None:
            continue
        assert a.dtype == dtype, n
        assert torch.equal(a, a2), n
        errs[n] = rel(a, e)
    log("   " + "  ".join(f"{n} {e:.1e}" for n, e in errs.items()))
    bad = {n: e for n, e in errs.items() if not e <= tol}
    assert not bad, f"beyond {tol}: {bad}"


@pytest.mark.gpu
@pytest.mark.parametrize("name,T,C,ld,off,dtype", [
    ("gate_bias_bf16", 16384, 336, 336, 0, torch.bfloat16),
    ("in_proj_bias_bf16", 16384, 3328, 3328, 0, torch.bfloat16),
    ("column_slice_bf16", 3000, 1024, 3104, 1024, torch.bfloat16),
    ("ragged_fp32", 1000, 44, 52, 8, torch.float32),
    ("fallback_bf16", 500, 30, 30, 0, torch.bfloat16),
])
def test_column_sum_matches_fp64(name, T, C, ld, off, dtype):
    """column_sum (cdssm_col_sum: fixed-order slab sums in fp32, one rounding; torch's sum where the kernel
    does not serve the layout) against the fp64 sum: one rounding of the result (bf16 <= 2^-8, fp32 <= 1e-6
    of the largest column sum), bit-identical on a repeat."""
    from cdssm_hip.lm import column_sum
    log(f"[column sum] {name}: T{T} C{C} ld{ld}")
    gen = torch.Generator().manual_seed(3)
    full = (torch.randn(T, ld, generator=gen) + 0.2).to(dtype).to(DEV)
    x = full[:, off:off + C]
    a, b = column_sum(x), column_sum(x)
    torch.cuda.synchronize()
    assert a.dtype == dtype and a.shape == (C,)
    assert torch.equal(a, b)
    err = rel(a, x.double().sum(0))
    log(f"   rel err {err:.1e}")
    assert err <= (2.0 ** -8 if dtype == torch.bfloat16 else 1e-6)


def test_token_linear_rejects_bias_with_residual():
    from cdssm_hip.lm import TokenLinearFn
    x, w = torch.randn(2, 3, 4, dtype=torch.float64), torch.randn(5, 4, dtype=torch.float64)
    with pytest.raises(ValueError):
        TokenLinearFn.apply(x, w, torch.zeros(5, dtype=torch.float64), torch.zeros(2, 3, 5, dtype=torch.float64))
