"""GPU parity of the block's training ops on the HIP kernels with their backwards.

The GroupNorm + gate epilogue (GroupNormGateFn:
cdssm_group_norm_gate_fwd / cdssm_group_norm_gate_bwd) against autograd through the reference's op sequence
(block.py:215-225): out = group_norm(y.float(), G, gamma.float(), beta.float(), eps).to(dtype) * silu(z)
+ D * x_conv, in fp64 on the CPU from the same (rounded) inputs.  z is a column slice of a wider tensor
(a token stride, as the block's in_proj output gives it).  Tolerances: fp32 <= 1e-4, bf16 <= 2e-2 normwise
for the output and every gradient (y, z, x_conv, gamma, beta, D).

The K/Q normalisation with the current-token q.k (NormalizeKQQkFn: cdssm_normalize_kq_qk_fwd / _bwd) against
fp64 autograd of NormalizeKQFn's rule (normalize_kq.cu:75-79) and q.k (block.py:191-192, 202), K a strided
column slice as in the block: fp32 <= 1e-4, bf16 <= 2e-2.

RMSNorm (RMSNormFn: cdssm_rms_norm_fwd / _bwd) against fp64 autograd of the reference expression
(modules.py:49-53): fp32 <= 1e-4, bf16 <= 2e-2 for the output, dx and the weight's gradient.
"""

import pytest
import torch

from _gpu_util import DEV, log, rel

pytestmark = pytest.mark.gpu


def reference(y, z, x, gamma, beta, D, G, eps):
    B, L, C = y.shape
    a = torch.nn.functional.group_norm(y.transpose(1, 2), G, gamma, beta, eps).transpose(1, 2)
    return a * torch.nn.functional.silu(z) + D * x


def draw(B, L, C, dtype, seed, wide=3104):
    g = torch.Generator().manual_seed(seed)
    y = (torch.randn(B, L, C, generator=g) * 1.5 + 0.3).to(dtype)
    proj = torch.randn(B, L, wide, generator=g).to(dtype)
    x = torch.randn(B, L, C, generator=g).to(dtype)
    gamma = (1.0 + 0.2 * torch.randn(C, generator=g)).to(dtype)
    beta = (0.1 * torch.randn(C, generator=g)).to(dtype)
    D = torch.randn(C, generator=g).to(dtype)
    dout = torch.randn(B, L, C, generator=g).to(dtype)
    return y, proj, x, gamma, beta, D, dout


CASES = [
    ("fp32_B2_L300_C1024_G32", 2, 300, 1024, 32, torch.float32),
    ("fp32_B1_L1024_C512_G16", 1, 1024, 512, 16, torch.float32),
    ("bf16_B2_L700_C1024_G32", 2, 700, 1024, 32, torch.bfloat16),
    ("bf16_C4_shape_B8_L2048_C1024_G32", 8, 2048, 1024, 32, torch.bfloat16),
]


@pytest.mark.parametrize("name,B,L,C,G,dtype", CASES, ids=[c[0] for c in CASES])
def test_group_norm_gate_forward_and_backward(name, B, L, C, G, dtype):
    from cdssm_hip.lm import GroupNormGateFn
    log(f"[group norm gate] {name}")
    eps = 1e-5
    y, proj, x, gamma, beta, D, dout = draw(B, L, C, dtype, seed=1)
    # reference in fp64 on the CPU from the rounded inputs
    ref = {n: t.double().clone().requires_grad_(True) for n, t in
           dict(y=y, z=proj[..., :C], x=x, gamma=gamma, beta=beta, D=D).items()}
    out_r = reference(ref["y"], ref["z"], ref["x"], ref["gamma"], ref["beta"], ref["D"], G, eps)
    out_r.backward(dout.double())
    # HIP on the GPU: z a column slice (token stride 3104) of the projection output
    got = {n: t.to(DEV).clone().requires_grad_(True) for n, t in
           dict(y=y, proj=proj, x=x, gamma=gamma, beta=beta, D=D).items()}
    z = got["proj"][..., :C]
    assert GroupNormGateFn.usable(got["y"], z, got["x"], G, (got["gamma"], got["beta"], got["D"]))
    out = GroupNormGateFn.apply(got["y"], z, got["x"], got["gamma"], got["beta"], got["D"], G, eps)
    out.backward(dout.to(DEV))
    torch.cuda.synchronize()
    errs = {"out": rel(out, out_r), "y": rel(got["y"].grad, ref["y"].grad),
            "z": rel(got["proj"].grad[..., :C], ref["z"].grad), "x": rel(got["x"].grad, ref["x"].grad),
            "gamma": rel(got["gamma"].grad, ref["gamma"].grad), "beta": rel(got["beta"].grad, ref["beta"].grad),
            "D": rel(got["D"].grad, ref["D"].grad)}
    assert float(got["proj"].grad[..., C:].abs().max()) == 0.0
    log("   " + "  ".join(f"{n} {e:.1e}" for n, e in errs.items()))
    tol = 1e-4 if dtype == torch.float32 else 2e-2
    bad = {n: e for n, e in errs.items() if not e <= tol}
    assert not bad, f"beyond {tol}: {bad}"


def test_group_norm_gate_backward_is_deterministic_and_matches_torch_bf16_ops():
    """Two backward calls give bit-identical gradients (fixed-order sums); and in bf16 the HIP gradients
    agree with torch's own autograd of the same op sequence on the GPU to a few bf16 roundings."""
    from cdssm_hip.lm import GroupNormGateFn
    B, L, C, G, eps = 2, 512, 1024, 32, 1e-5
    y, proj, x, gamma, beta, D, dout = draw(B, L, C, torch.bfloat16, seed=2)
    args = [t.to(DEV) for t in (y, proj[..., :C].contiguous(), x, gamma, beta, D)]
    grads = []
    for _ in range(2):
        leaves = [t.clone().requires_grad_(True) for t in args]
        out = GroupNormGateFn.apply(*leaves, G, eps)
        out.backward(dout.to(DEV))
        grads.append([t.grad for t in leaves])
    torch.cuda.synchronize()
    for a, b in zip(*grads):
        assert torch.equal(a, b)
    leaves = [t.clone().float().requires_grad_(True) for t in args]
    yy, zz, xx, gg, bb, dd = leaves
    # torch's op sequence with the bf16 rounding points of a bf16 model (block.py:216-225)
    a = torch.nn.functional.group_norm(yy.transpose(1, 2), G, gg, bb, eps).transpose(1, 2).bfloat16()
    o = a * torch.nn.functional.silu(zz.bfloat16()) + dd.bfloat16() * xx.bfloat16()
    o.backward(dout.to(DEV))
    errs = [rel(g1, g2.grad) for g1, g2 in zip(grads[0], leaves)]
    log("   vs torch bf16 ops: " + "  ".join(f"{e:.1e}" for e in errs))
    assert max(errs) <= 2e-2


KQ_CASES = [("fp32_D64", torch.float32, 64), ("fp32_D128", torch.float32, 128), ("bf16_D64", torch.bfloat16, 64),
            ("bf16_D128", torch.bfloat16, 128)]


@pytest.mark.parametrize("name,dtype,D", KQ_CASES, ids=[c[0] for c in KQ_CASES])
def test_normalize_kq_qk_forward_and_backward(name, dtype, D):
    from cdssm_hip.lm import NormalizeKQQkFn
    B, L, H = 2, 300, 16
    g = torch.Generator().manual_seed(3)
    wide = torch.randn(B, L, 3 * H * D + 48, generator=g).to(dtype)   # K a column slice of it
    Q = torch.randn(B, L, H, D, generator=g).to(dtype)
    gK = torch.randn(B, L, H, D, generator=g).to(dtype)
    gQ = torch.randn(B, L, H, D, generator=g).to(dtype)
    gqk = torch.randn(B, L, H, generator=g)
    off = H * D
    # reference: fp64 on the CPU
    wr = wide.double().requires_grad_(True)
    qr = Q.double().requires_grad_(True)
    Kr = wr[..., off:off + H * D].reshape(B, L, H, D)
    Kn = Kr * torch.rsqrt((Kr * Kr).sum(-1, keepdim=True) + 1e-6)
    Qn = qr * torch.rsqrt((qr * qr).sum(-1, keepdim=True) + 1e-6)
    qk = (Kn * Qn).sum(-1)
    torch.autograd.backward([Kn, Qn, qk], [gK.double(), gQ.double(), gqk.double()])
    wg = wide.to(DEV).requires_grad_(True)
    qg = Q.to(DEV).requires_grad_(True)
    Kg = wg[..., off:off + H * D].reshape(B, L, H, D)
    Ko, Qo, qko = NormalizeKQQkFn.apply(Kg, qg)
    torch.autograd.backward([Ko, Qo, qko], [gK.to(DEV), gQ.to(DEV), gqk.to(DEV)])
    torch.cuda.synchronize()
    errs = {"K^": rel(Ko, Kn), "Q^": rel(Qo, Qn), "qk": rel(qko, qk), "dK": rel(wg.grad, wr.grad),
            "dQ": rel(qg.grad, qr.grad)}
    log(f"[normalize kq qk] {name}: " + "  ".join(f"{n} {e:.1e}" for n, e in errs.items()))
    tol = 1e-4 if dtype == torch.float32 else 2e-2
    bad = {n: e for n, e in errs.items() if not e <= tol}
    assert not bad, f"beyond {tol}: {bad}"


RMS_CASES = [("fp32_C1024", torch.float32, 1024), ("fp32_C512", torch.float32, 512),
             ("bf16_C1024", torch.bfloat16, 1024), ("bf16_C2048", torch.bfloat16, 2048)]


@pytest.mark.parametrize("name,dtype,C", RMS_CASES, ids=[c[0] for c in RMS_CASES])
def test_rms_norm_forward_and_backward(name, dtype, C):
    from cdssm_hip.lm import RMSNormFn
    B, L, eps = 2, 301, 1e-5
    g = torch.Generator().manual_seed(4)
    x = (torch.randn(B, L, C, generator=g) * 2.0 + 0.5).to(dtype)
    w = (1.0 + 0.3 * torch.randn(C, generator=g)).to(dtype)
    dout = torch.randn(B, L, C, generator=g).to(dtype)
    xr, wr = x.double().requires_grad_(True), w.double().requires_grad_(True)
    yr = xr * torch.rsqrt(xr.pow(2).mean(-1, keepdim=True) + eps) * wr
    yr.backward(dout.double())
    assert RMSNormFn.usable(x.to(DEV))
    grads = []
    for _ in range(2):
        xg, wg = x.to(DEV).requires_grad_(True), w.to(DEV).requires_grad_(True)
        y = RMSNormFn.apply(xg, wg, eps)
        y.backward(dout.to(DEV))
        grads.append((xg.grad, wg.grad))
    torch.cuda.synchronize()
    assert torch.equal(grads[0][0], grads[1][0]) and torch.equal(grads[0][1], grads[1][1])
    errs = {"y": rel(y, yr), "dx": rel(grads[0][0], xr.grad), "dw": rel(grads[0][1], wr.grad)}
    log(f"[rms norm] {name}: " + "  ".join(f"{n} {e:.1e}" for n, e in errs.items()))
    tol = 1e-4 if dtype == torch.float32 else 2e-2
    bad = {n: e for n, e in errs.items() if not e <= tol}
    assert not bad, f"beyond {tol}: {bad}"
