"""GPU parity of the gate-level dynamics in the branches random gates never reach.

DynamicsFusedFn (dynamics_fused.cu:35-387) has three branches that N(0, 1) gates
with log_dt_scale near 0 do not enter: the adaptive-dt cap with a material blend
(forward :88-93; backward :350-359), the VP clamp (vp = sqrt(1e-6); forward
:113-118, the reference's clamp gradient :247-259) and vp = 1.  The rows below
force each of them per head (H = 8):

  head 0      VP clamp, flat: alpha ~ softplus(-30) ~ 1e-13 and r = sigmoid(-5): E is
              1 - O(1e-6) (the 1e-6 in the Cayley denominator), 1 - E^(c r) < 1e-6
  head 1      VP clamp, damped: alpha ~ softplus(N(0, 0.5)), E ~ 0.1-0.9, and
              r = sigmoid(-20 +- 0.3) ~ 2e-9, so c r |ln E| < 1e-6 for any E >= 1e-8
  head 2      vp = 1: alpha ~ 1, omega ~ 0, dt ~ 1.4 (tau alpha ~ 0.7, E ~ 0.03)
              and r ~ 1, so E^(c r) is below fp32's resolution at 1
  head 3      N(0, 0.8^2) gates (the existing test's draw)
  heads 4-7   the cap: alpha_0 ~ 0.05, |omega_0| within 0.035 of omega_thresh,
              log_dt_scale ~ 3 (dt_raw ~ 2.7 > dt_max ~ 1.8), blend in (0.1, 0.9)

The test counts the branches from the oracle on the same (dtype-rounded) rows
and requires >= 20% of token-heads capped with the blend in (0.05, 0.95), so the
coverage cannot silently drop.  Outputs and gradients are compared with the
fp64 oracle (its backward restates the reference's analytic rule, pinned to
autograd with the cap active in tests/test_oracle_pins.py); the cap heads'
gradients are also compared on their own slice, so the blend terms are not
hidden under the other heads' gradients.  The same rows go through
cdssm_dynamics_fused_fwd_at (the decode path's dynamics, gate_math.hpp shared
with the fused decode-token kernel), bit-identical to the full-sequence kernel.

The clamp gradient itself (d vp -> -0.5/vp d E^(c r), which exact differentiation
of the clamped forward would make zero) is checked with only the vp cotangent
nonzero, on head 1.  On head 0 it depends on 1 - E ~ 1e-6, an fp32 cancellation
the reference's kernel has as well (the oracle itself evaluated in fp32 is 30%
off its fp64 value there), so head 0 enters only the mixed test above; on head 1
E is moderate and the rule is well conditioned.

Tolerances (normwise max|x-ref|/max|ref|): fp32 1e-4, bf16 2e-2.
"""

import math

import pytest
import torch

from _gpu_util import DEV, log, rel
from oracle import cdssm_oracle as o

pytestmark = pytest.mark.gpu
TOL = {torch.float32: 1e-4, torch.bfloat16: 2e-2}
H = 8
REGIME = ("clamp_flat", "clamp", "vp1", "random", "cap", "cap", "cap", "cap")
CONSTS = dict(gating_c=math.log(2048), omega_thresh=math.sqrt(2 ** -7), adt_delta=16 * 2 ** -7,
              adt_smoothness=math.sqrt(2 ** -7) / 5, adt_eps=1.0)


def regime_rows(B, L, N, seed):
    """gate_raw (B, L, (N+5) H), log_dt_scale (H), rope freqs (H), all float64."""
    gen = torch.Generator().manual_seed(seed)
    Nh = N // 2
    freqs = 1.0 / (2048.0 ** (torch.arange(H, dtype=torch.float64) / H))
    g = torch.randn(B, L, N + 5, H, generator=gen, dtype=torch.float64) * 0.8
    lds = torch.randn(H, generator=gen, dtype=torch.float64) * 0.5
    pos = torch.arange(L, dtype=torch.float64)[None, :]

    def noise(*shape, s=1.0):
        return torch.randn(*shape, generator=gen, dtype=torch.float64) * s

    for h, kind in enumerate(REGIME):
        if kind == "clamp_flat":
            lds[h] = 0.4
            g[:, :, :Nh, h] = -30.0
            g[:, :, N + 4, h] = -5.0 + noise(B, L, s=0.3)
        elif kind == "clamp":
            g[:, :, :Nh, h] = noise(B, L, Nh, s=0.5)
            g[:, :, N + 4, h] = -20.0 + noise(B, L, s=0.3)
        elif kind == "vp1":
            g[:, :, :Nh, h] = 0.54 + noise(B, L, Nh, s=0.1)
            g[:, :, Nh:N, h] = noise(B, L, Nh, s=0.2) - (pos * freqs[h])[..., None]
            g[:, :, N + 2, h] = 0.6 + noise(B, L, s=0.1)
            g[:, :, N + 4, h] = 5.0 + noise(B, L, s=0.3)
        elif kind == "cap":
            lds[h] = 3.0 + 0.2 * float(noise(1))
            g[:, :, 0, h] = -3.0 + noise(B, L, s=0.3)
            sign = torch.where(torch.rand(B, L, generator=gen, dtype=torch.float64) < 0.5, -1.0, 1.0)
            target = CONSTS["omega_thresh"] + (torch.rand(B, L, generator=gen, dtype=torch.float64) * 2 - 1) * 0.035
            g[:, :, Nh, h] = sign * target - pos * freqs[h]
    return g.reshape(B, L, (N + 5) * H), lds, freqs


def _coverage(gate64, lds, freqs, N):
    reg = o.dynamics_regimes(gate64, lds, freqs, n_heads=H, state_dim=N, **CONSTS)
    cov = {k: float(v.double().mean()) for k, v in reg.items()}
    log("   coverage: " + " ".join(f"{k} {v:.1%}" for k, v in cov.items()))
    assert cov["blend_mid"] >= 0.20, "too few token-heads in the cap with a material blend"
    assert cov["vp_clamped"] >= 0.2 and cov["vp_one"] >= 0.1
    return reg


def _run(gate, lds, freqs, N, gs):
    from cdssm_hip.ops import DynamicsFusedFn
    gd = gate.to(DEV).requires_grad_(True)
    ld = lds.float().to(DEV).requires_grad_(True)
    outs = DynamicsFusedFn.apply(gd, ld, freqs.float().to(DEV), CONSTS["gating_c"], CONSTS["omega_thresh"],
                                 CONSTS["adt_delta"], CONSTS["adt_smoothness"], CONSTS["adt_eps"], H, N)
    torch.autograd.backward(list(outs), [x.to(DEV) for x in gs])
    torch.cuda.synchronize()
    return [x.detach() for x in outs], gd.grad, ld.grad


@pytest.mark.parametrize("dtype,N,L", [(torch.float32, 2, 300), (torch.float32, 16, 130), (torch.bfloat16, 2, 300),
                                       (torch.bfloat16, 16, 70)])
def test_dynamics_branches_match_oracle(dtype, N, L):
    B = 2
    log(f"[dynamics branches] {dtype} N{N} B{B} L{L} H{H}")
    gate64, lds, freqs = regime_rows(B, L, N, seed=31)
    gate = gate64.to(dtype)
    gate_r = gate.double()  # the oracle runs on the rounded rows
    lds32 = lds.float().double()
    freqs32 = freqs.float().double()
    _coverage(gate_r, lds32, freqs32, N)
    outs_ref = o.dynamics_fused_fwd(gate_r, lds32, freqs32, n_heads=H, state_dim=N, **CONSTS)
    gen = torch.Generator().manual_seed(32)
    gs = [torch.randn(*t.shape, generator=gen).to(dtype) for t in outs_ref]
    gg_ref, gl_ref = o.dynamics_fused_bwd_ref(*[x.double() for x in gs], gate_r, lds32, freqs32, n_heads=H,
                                              state_dim=N, **CONSTS)
    outs, gg, gl = _run(gate, lds, freqs, N, gs)
    errs = {n: rel(x, y) for n, x, y in zip(("A_bar", "vp", "beta", "sel_C"), outs, outs_ref)}
    errs["grad_gate_raw"] = rel(gg, gg_ref)
    errs["grad_log_dt_scale"] = rel(gl, gl_ref)
    cap = torch.tensor([k == "cap" for k in REGIME])
    gg_cap = gg.reshape(B, L, N + 5, H)[..., cap]
    errs["grad_gate_raw[cap heads]"] = rel(gg_cap, gg_ref.reshape(B, L, N + 5, H)[..., cap])
    errs["grad_log_dt_scale[cap heads]"] = rel(gl[cap.to(DEV)], gl_ref[cap])
    log("   " + " ".join(f"{k} {v:.1e}" for k, v in errs.items()))
    assert max(errs.values()) <= TOL[dtype], errs
    # the decode path's dynamics (same device code) on the same rows, at the same positions
    from cdssm_hip.lm import dynamics_at
    args = (lds.float().to(DEV), freqs.float().to(DEV), CONSTS["gating_c"], CONSTS["omega_thresh"],
            CONSTS["adt_delta"], CONSTS["adt_smoothness"], CONSTS["adt_eps"], H, N)
    gd = gate.to(DEV)
    for t in (0, 1, L // 2, L - 1):
        one = dynamics_at(gd[:, t:t + 1], *args, t)
        for a, b in zip(one, outs):
            assert torch.equal(a[:, 0], b[:, t]), f"dynamics_at differs at position {t}"


def test_vp_clamp_gradient_matches_oracle():
    """Only the vp cotangent nonzero, rows of the damped clamp head (fp32): every gradient entry is the
    reference's clamp rule (d vp -> -0.5/vp d E^(c r)), which exact differentiation of the clamped forward
    would make zero.  1e-3 normwise: with E moderate the rule has no cancellation (the oracle evaluated in fp32
    is within 1e-6 of fp64 here)."""
    N, B, L = 2, 2, 200
    log(f"[vp clamp gradient] fp32 N{N} B{B} L{L}")
    gate64, lds, freqs = regime_rows(B, L, N, seed=33)
    gate = gate64.float()
    gate_r, lds32, freqs32 = gate.double(), lds.float().double(), freqs.float().double()
    reg = o.dynamics_regimes(gate_r, lds32, freqs32, n_heads=H, state_dim=N, **CONSTS)
    clamp = torch.tensor([k == "clamp" for k in REGIME])
    assert bool(reg["vp_clamped"][:, :, clamp].all())
    outs_ref = o.dynamics_fused_fwd(gate_r, lds32, freqs32, n_heads=H, state_dim=N, **CONSTS)
    gen = torch.Generator().manual_seed(34)
    gs = [torch.zeros(t.shape) for t in outs_ref]
    gvp = torch.randn(*outs_ref[1].shape, generator=gen)
    gvp[:, :, ~clamp] = 0.0
    gs[1] = gvp
    gg_ref, gl_ref = o.dynamics_fused_bwd_ref(*[x.double() for x in gs], gate_r, lds32, freqs32, n_heads=H,
                                              state_dim=N, **CONSTS)
    _, gg, gl = _run(gate, lds, freqs, N, gs)
    got = gg.reshape(B, L, N + 5, H)[..., clamp]
    want = gg_ref.reshape(B, L, N + 5, H)[..., clamp]
    e, el = rel(got, want), rel(gl[clamp.to(DEV)], gl_ref[clamp])
    log(f"   damped clamp head: grad_gate_raw {e:.1e} (max |ref| {float(want.abs().max()):.1e}), "
        f"grad_log_dt_scale {el:.1e}")
    assert float(want.abs().max()) > 1e-6
    assert e <= 1e-3 and el <= 1e-3
    # outside the clamp heads nothing flows (their vp cotangent is zero)
    assert float(gg.reshape(B, L, N + 5, H)[..., ~clamp].abs().max()) == 0.0
