"""GPU parity of the block's fused elementwise / normalisation kernels
(cdssm_rms_norm_fwd, cdssm_normalize_kq_qk_fwd, cdssm_shortcut_readout_fwd,
cdssm_group_norm_gate_fwd, cdssm_conv1d_silu_fwd_strided) against the CPU
oracle's restatements in fp64 on the same (dtype-rounded) inputs.

Tolerances (normwise max|x-ref|/max|ref|): fp32 1e-5 (fp32 statistics and
hardware rsqrt / exp); bf16 1e-2 (the outputs are rounded to bf16 at the
reference's rounding points, each a relative 2^-9, a few in a row for the
gated GroupNorm output).
"""

import pytest
import torch
import torch.nn.functional as F

from _gpu_util import DEV, log, rel
from oracle import cdssm_lm_oracle as lo
from oracle import cdssm_oracle as o

pytestmark = pytest.mark.gpu


def _tol(dtype):
    return 1e-5 if dtype == torch.float32 else 1e-2


@pytest.mark.parametrize("dtype,rows,C", [(torch.float32, 33, 128), (torch.bfloat16, 100, 1024),
                                          (torch.bfloat16, 7, 20), (torch.float32, 5, 3)])
def test_rms_norm(dtype, rows, C):
    from cdssm_hip.lm import rms_norm
    log(f"[rms_norm] {dtype} rows {rows} C {C}")
    g = torch.Generator().manual_seed(1)
    x = (torch.randn(rows, C, generator=g) * 3 + 0.5).to(dtype)
    w = (1 + 0.1 * torch.randn(C, generator=g)).to(dtype)
    eps = 6.103515625e-05
    y = rms_norm(x.to(DEV), w.to(DEV), eps).cpu()
    yr = lo.rms_norm(x.double(), w.double(), eps)
    e = rel(y, yr)
    log(f"   rel err {e:.2e}")
    assert y.dtype == dtype and e <= _tol(dtype)


@pytest.mark.parametrize("dtype,B,L,H,D,pad", [(torch.bfloat16, 2, 50, 16, 64, 96), (torch.float32, 1, 9, 3, 64, 0),
                                               (torch.bfloat16, 1, 4, 2, 128, 8), (torch.float32, 2, 5, 2, 128, 4),
                                               (torch.bfloat16, 1, 1, 1, 32, 0), (torch.bfloat16, 5, 1, 4, 64, 32)])
def test_normalize_kq_qk(dtype, B, L, H, D, pad):
    """K read as a column slice of a wider (B, L, pad + H*D + 8) tensor, as from the block's in_proj."""
    from cdssm_hip.lm import normalize_kq_qk
    log(f"[normalize_kq_qk] {dtype} B{B} L{L} H{H} D{D} K column offset {pad}")
    g = torch.Generator().manual_seed(2)
    wide = torch.randn(B, L, pad + H * D + 8, generator=g).to(dtype)
    q = torch.randn(B, L, H, D, generator=g).to(dtype)
    wd = wide.to(DEV)
    Kv = wd[..., pad:pad + H * D].reshape(B, L, H, D)
    assert not Kv.is_contiguous() or pad == 0
    Ko, Qo, qk = normalize_kq_qk(Kv, q.to(DEV))
    Kr, Qr = o.normalize_kq(wide[..., pad:pad + H * D].reshape(B, L, H, D).double(), q.double())
    ek, eq = rel(Ko.cpu(), Kr), rel(Qo.cpu(), Qr)
    # qk from the kernel's own (rounded) outputs, in fp64
    eqk = rel(qk.cpu(), (Ko.cpu().double() * Qo.cpu().double()).sum(-1))
    log(f"   rel err K {ek:.2e} Q {eq:.2e} qk {eqk:.2e}")
    assert ek <= _tol(dtype) and eq <= _tol(dtype) and eqk <= 1e-5


@pytest.mark.parametrize("dtype,qk_dtype", [(torch.float32, torch.float32), (torch.bfloat16, torch.float32),
                                            (torch.float32, torch.float64)])
def test_shortcut_readout(dtype, qk_dtype):
    """qk in fp64 too: the wrapper hands the kernel fp32 whatever floating dtype it gets."""
    from cdssm_hip.lm import shortcut_readout_
    B, L, H = 2, 33, 4
    log(f"[shortcut_readout] {dtype} qk {qk_dtype} B{B} L{L} H{H}")
    g = torch.Generator().manual_seed(3)
    ret = torch.randn(B, L, H, 2, generator=g, dtype=torch.float32).to(dtype)
    qk = torch.rand(B, L, H, generator=g, dtype=torch.float32).to(qk_dtype) * 2 - 1
    V = torch.randn(B, L, H, 2, generator=g, dtype=torch.float32).to(dtype)
    vp = torch.rand(B, L, H, 1, generator=g, dtype=torch.float32).to(dtype)
    sel = torch.rand(B, L, H, generator=g, dtype=torch.float32).to(dtype)
    scale = torch.tensor([0.7], dtype=torch.float32)
    out = shortcut_readout_(ret.to(DEV), qk.to(DEV), V.to(DEV), vp.to(DEV), sel.to(DEV), scale.to(DEV)).cpu()
    # the reference's form: Y += s (q.k) V_gated k^T, read by q and gated by sel_C (block.py:202-211), with q.k
    # standing for both the shortcut's factor and the readout's k.q
    ref = ret.double() + (0.7 * qk.double() ** 2 * sel.double())[..., None] * V.double() * vp.double()
    e = rel(out, ref)
    log(f"   rel err {e:.2e}")
    if not e <= _tol(dtype):
        bad = (out.double() - ref).abs() > 1e-3
        log(f"   bad {int(bad.sum())} of {bad.numel()}; first {bad.nonzero()[:4].tolist()}; "
            f"out {out[bad][:4].tolist()} ref {ref[bad][:4].tolist()}")
    assert e <= _tol(dtype)


@pytest.mark.parametrize("dtype,B,L,H,N,D", [(torch.bfloat16, 2, 37, 3, 16, 64), (torch.float32, 1, 50, 2, 16, 128),
                                             (torch.bfloat16, 1, 9, 4, 4, 48), (torch.float32, 2, 5, 1, 32, 12)])
def test_state_readout(dtype, B, L, H, N, D):
    """StateReadoutFn (cdssm_state_readout_fwd / _bwd) against fp64 autograd of einsum('blhsd,blhd->blhs', Y, Q)
    (block.py:208) on the same rounded inputs: fp32 1e-5, bf16 4e-3 (one rounding of each output)."""
    from cdssm_hip.lm import StateReadoutFn
    log(f"[state_readout] {dtype} B{B} L{L} H{H} N{N} D{D}")
    g = torch.Generator().manual_seed(5)
    Y = torch.randn(B, L, H, N, D, generator=g).to(dtype)
    Q = torch.randn(B, L, H, D, generator=g).to(dtype)
    dr = torch.randn(B, L, H, N, generator=g).to(dtype)
    Yr, Qr = Y.double().requires_grad_(True), Q.double().requires_grad_(True)
    rr = torch.einsum('blhsd,blhd->blhs', Yr, Qr)
    rr.backward(dr.double())
    Yg, Qg = Y.to(DEV).requires_grad_(True), Q.to(DEV).requires_grad_(True)
    r = StateReadoutFn.apply(Yg, Qg)
    r.backward(dr.to(DEV))
    tol = 1e-5 if dtype == torch.float32 else 4e-3
    errs = dict(r=rel(r.cpu(), rr), dY=rel(Yg.grad.cpu(), Yr.grad), dQ=rel(Qg.grad.cpu(), Qr.grad))
    log("   " + "  ".join(f"{k} {v:.1e}" for k, v in errs.items()))
    assert all(v <= tol for v in errs.values()), errs


@pytest.mark.parametrize("dtype,B,L,C,G,zpad", [(torch.bfloat16, 2, 300, 1024, 32, 64), (torch.float32, 1, 77, 128, 32, 0),
                                                 (torch.bfloat16, 1, 40, 128, 32, 8), (torch.bfloat16, 2, 513, 96, 3, 3),
                                                 (torch.float32, 3, 1, 64, 4, 4)])
def test_group_norm_gate(dtype, B, L, C, G, zpad):
    from cdssm_hip.lm import group_norm_gate
    log(f"[group_norm_gate] {dtype} B{B} L{L} C{C} G{G} z column offset {zpad}")
    g = torch.Generator().manual_seed(4)
    y = (torch.randn(B, L, C, generator=g) * 2 + 3).to(dtype)  # a mean far from zero
    zw = torch.randn(B, L, zpad + C + 5, generator=g).to(dtype)
    xc = torch.randn(B, L, C, generator=g).to(dtype)
    gamma = 1 + 0.2 * torch.randn(C, generator=g)
    beta = 0.1 * torch.randn(C, generator=g)
    Dp = (0.3 * torch.randn(C, generator=g)).to(dtype)
    eps = 1e-5
    zd = zw.to(DEV)[..., zpad:zpad + C]
    out = group_norm_gate(y.to(DEV), G, gamma.to(DEV), beta.to(DEV), eps, zd, xc.to(DEV), Dp.to(DEV)).cpu()
    z = zw[..., zpad:zpad + C].double()
    gn = F.group_norm(y.double().transpose(1, 2), G, gamma.double(), beta.double(), eps).transpose(1, 2)
    ref = gn * (z * torch.sigmoid(z)) + Dp.double() * xc.double()  # block.py:216-225
    e = rel(out, ref)
    log(f"   rel err {e:.2e}")
    assert out.dtype == dtype and e <= (1e-5 if dtype == torch.float32 else 2e-2)


@pytest.mark.parametrize("dtype,B,L,C,K,pad", [(torch.bfloat16, 2, 130, 1024, 4, 1024), (torch.float32, 1, 20, 12, 3, 5)])
def test_conv1d_silu_strided(dtype, B, L, C, K, pad):
    """conv input read in place as a column slice (the block's x_gate)."""
    from cdssm_hip.lm import conv1d_silu
    log(f"[conv1d_silu strided] {dtype} B{B} L{L} C{C} K{K} column offset {pad}")
    g = torch.Generator().manual_seed(5)
    wide = torch.randn(B, L, pad + C + 16, generator=g).to(dtype)
    w = (torch.randn(C, 1, K, generator=g) / K ** 0.5).to(dtype)
    b = torch.randn(C, generator=g).to(dtype)
    y = conv1d_silu(wide.to(DEV)[..., pad:pad + C], w.to(DEV), b.to(DEV)).cpu()
    yr = lo.conv1d_silu(wide[..., pad:pad + C].double(), w.double(), b.double())
    e = rel(y, yr)
    log(f"   rel err {e:.2e}")
    assert e <= (1e-6 if dtype == torch.float32 else 1e-2)


@pytest.mark.parametrize("dtype,B,L,C,K,pad", [(torch.float32, 2, 37, 24, 4, 0), (torch.float32, 1, 50, 16, 3, 5),
                                               (torch.bfloat16, 2, 300, 256, 4, 64), (torch.float32, 1, 3, 8, 8, 0),
                                               (torch.bfloat16, 1, 70, 64, 4, 3)])
def test_conv1d_silu_backward(dtype, B, L, C, K, pad):
    """Conv1dSiLU backward (cdssm_conv1d_silu_bwd) against autograd through the oracle's fp64 conv on the same
    rounded inputs; x read as a column slice when pad > 0."""
    from cdssm_hip.lm import Conv1dSiLU
    log(f"[conv1d_silu bwd] {dtype} B{B} L{L} C{C} K{K} column offset {pad}")
    g = torch.Generator().manual_seed(6)
    f32 = dict(generator=g, dtype=torch.float32)
    wide = torch.randn(B, L, pad + C + 8, **f32).to(dtype)
    w = (torch.randn(C, 1, K, **f32) / K ** 0.5).to(dtype)
    b = torch.randn(C, **f32).to(dtype)
    gy = torch.randn(B, L, C, **f32).to(dtype)
    conv = Conv1dSiLU(C, kernel_size=K).to(dtype).to(DEV)
    with torch.no_grad():
        conv.weight.copy_(w)
        conv.bias.copy_(b)
    xd = wide.to(DEV)[..., pad:pad + C].detach().requires_grad_(True)
    conv(xd).backward(gy.to(DEV))
    xr = wide[..., pad:pad + C].double().requires_grad_(True)
    wr, br = w.double().requires_grad_(True), b.double().requires_grad_(True)
    lo.conv1d_silu(xr, wr, br).backward(gy.double())
    ex, ew, eb = rel(xd.grad, xr.grad), rel(conv.weight.grad, wr.grad), rel(conv.bias.grad, br.grad)
    log(f"   rel err grad_x {ex:.2e} grad_w {ew:.2e} grad_b {eb:.2e}")
    tol = 1e-5 if dtype == torch.float32 else 1e-2
    assert ex <= tol and ew <= tol and eb <= tol
    assert conv.weight.grad.dtype == dtype and xd.grad.dtype == dtype


@pytest.mark.parametrize("N", [2, 16])
def test_lm_training_gradients_match_oracle(N):
    """Training through the model (block.py:140-229 with gradients): every parameter's gradient of
    sum(logits * g) against the fp64 oracle LM with the reference's own backward rules for the dynamics
    and the exact correction (grad_mode="reference"), fp32, 2 layers with the value residual, the
    shortcut and the D-skip active.  1e-3 normwise per parameter."""
    from cdssm_hip.lm import CDSSMConfig, CDSSMLMHeadModel
    log(f"[lm training grads] fp32 d_model 64 d_inner 128 layers 2 N{N}")
    torch.manual_seed(0)
    cfg = CDSSMConfig(d_model=64, n_layers=2, context_length=256, vocab_size=50, state_dim=N, d_inner=128)
    m = CDSSMLMHeadModel(cfg)
    with torch.no_grad():
        for blk in m.blocks:
            blk.v_residual_gate.normal_(std=1.0)
            blk.shortcut_scale.fill_(0.3)
            blk.D.normal_(std=0.1)
    m = m.float().to(DEV).train()
    gen = torch.Generator().manual_seed(3)
    ids = torch.randint(0, cfg.vocab_size, (2, 100), generator=gen)
    gl = torch.randn(2, 100, cfg.vocab_size, generator=gen)
    p = {k: v.detach().double().cpu().clone().requires_grad_(True) for k, v in m.state_dict().items()}
    logits = m(ids.to(DEV))
    (logits * gl.to(DEV)).sum().backward()
    torch.cuda.synchronize()
    ref = lo.lm_forward(p, ids, cfg, grad_mode="reference")
    (ref * gl.double()).sum().backward()
    e_out = rel(logits.detach(), ref.detach())
    worst, errs = 0.0, {}
    for name, prm in m.named_parameters():
        want = p[name].grad
        if name == "embedding.weight":  # tied with lm_head.weight (model.py:29-30)
            want = want + p["lm_head.weight"].grad if p["lm_head.weight"].grad is not None else want
        if prm.grad is None and want is None:
            continue  # unused, as in the reference (layer 0's v_residual_gate: no v_first yet)
        assert prm.grad is not None and want is not None, name
        errs[name] = rel(prm.grad, want)
        worst = max(worst, errs[name])
    log(f"   logits {e_out:.1e}; worst parameter gradient {worst:.1e} "
        f"({max(errs, key=errs.get)})")
    assert e_out <= 1e-3
    bad = {n: e for n, e in errs.items() if not e <= 1e-3}
    assert not bad, bad


@pytest.mark.parametrize("dtype,K", [(torch.bfloat16, 4), (torch.float32, 4), (torch.bfloat16, 3)])
def test_conv1d_silu_backward_vector_and_scalar_paths_agree_bitwise(dtype, K):
    """cdssm_conv1d_silu_bwd takes 16-byte channel vectors where x, grad_out and grad_x rows are 16-byte
    aligned and one channel per thread otherwise; both add every sum in the same order, so the same inputs
    give the same bits (x read at an aligned and at a misaligned column offset)."""
    from cdssm_hip.lm import conv1d_silu_bwd
    B, L, C = 2, 531, 512
    log(f"[conv1d_silu bwd paths] {dtype} K{K}")
    g = torch.Generator().manual_seed(8)
    f32 = dict(generator=g, dtype=torch.float32)
    x = torch.randn(B, L, C, **f32).to(dtype)
    w = (torch.randn(C, 1, K, **f32) / K ** 0.5).to(dtype).to(DEV)
    b = torch.randn(C, **f32).to(dtype).to(DEV)
    gy = torch.randn(B, L, C, **f32).to(dtype).to(DEV)
    wide = torch.zeros(B, L, C + 16, dtype=dtype)
    wide[..., 8:8 + C] = x        # 16-byte aligned rows (bf16: 16 bytes in; fp32: 32 bytes)
    odd = torch.zeros(B, L, C + 16, dtype=dtype)
    odd[..., 1:1 + C] = x         # misaligned: one channel per thread
    ga = conv1d_silu_bwd(wide.to(DEV)[..., 8:8 + C], w, b, gy)
    gb = conv1d_silu_bwd(odd.to(DEV)[..., 1:1 + C], w, b, gy)
    torch.cuda.synchronize()
    for a, c in zip(ga, gb):
        assert torch.equal(a, c)
