"""GPU parity of the fused scan on gate-level inputs (cdssm_fused_scan_fwd_abar, and the training pair
cdssm_fused_scan_fwd_abar_train / cdssm_fused_scan_bwd_abar).

The model's block feeds the scan with DynamicsFusedFn's A_bar and vp_scale
(block.py:177-211) rather than scan-level (dt, r, alpha, omega).  Here A_bar
and vp are given as inputs (from the oracle's Cayley/gating formula, rounded
once to the input dtype), and the fused scan must equal the oracle's
SSDChunkwiseScan(A_bar, K, V * vp, beta) (ssd.py:39-111) with the sel_C-gated
readout (block.py:208-211), computed in fp64 on the same rounded values.
Tolerances: fp32 <= 1e-4; bf16 y <= 2e-2, final-state norms <= 1e-3.
"""

import pytest
import torch

from _gpu_util import DEV, ScanConfig, cotangents, draw_inputs, log, rel, state_norm_rel, to_dev
from oracle import cdssm_oracle as o

pytestmark = pytest.mark.gpu

CASES = [
    ("fp32_C0", ScanConfig("C0", B=1, H=4, L=512, D=64, dtype="fp32"), None),
    ("fp32_ragged_h0", ScanConfig("t", B=2, H=5, L=300, D=64, dtype="fp32", h0_std=0.1), None),
    ("fp32_D128_chunk20", ScanConfig("t", B=1, H=3, L=230, D=128, dtype="fp32", h0_std=0.1), 20),
    ("bf16_D64", ScanConfig("t", B=2, H=16, L=640, D=64), None),
    ("bf16_D128_fast_omega", ScanConfig("t", B=1, H=9, L=333, D=128, omega_std=3.0, h0_std=0.1), None),
    ("bf16_C1_shape", ScanConfig("C1", B=8, H=16, L=4096, D=64), None),
    # config 4's gate-level scan: 128 one-pass workgroups at 8 heads per wave, so it runs 4 per wave
    ("bf16_C4_shape", ScanConfig("C4", B=8, H=16, L=2048, D=64), None),
]


@pytest.mark.parametrize("name,cfg,chunk", CASES, ids=[c[0] for c in CASES])
def test_fused_abar_matches_oracle(name, cfg, chunk):
    from cdssm_hip.scan import chunkwise_delta_scan_abar
    log(f"[fused abar] {name}: B{cfg.B} H{cfg.H} L{cfg.L} D{cfg.D} {cfg.dtype} chunk={chunk or cfg.D}")
    x = draw_inputs(cfg, seed=0)
    dtype = x["q"].dtype
    A, vp = o.scan_dynamics(x["alpha"].double(), x["omega"].double(), x["dt"].double(), x["r"].double(), x["c"])
    A, vp = A.to(dtype), vp.to(dtype)  # the gate-level op returns them in the input dtype
    g = to_dev(x)
    y, hf = chunkwise_delta_scan_abar(g["q"], g["k"], g["v"], g["beta"], g["sel_C"], A.to(DEV), vp.to(DEV),
                                      h0=g.get("h0"), chunk_size=chunk)
    torch.cuda.synchronize()
    y, hf = y.cpu(), hf.cpu()
    # oracle on (a few sequences of) the same rounded inputs
    bsel = [0, cfg.B - 1] if cfg.B > 2 else list(range(cfg.B))
    hsel = [0, cfg.H - 1] if cfg.H > 4 else list(range(cfg.H))
    sl = lambda t: t.double()[bsel][:, :, hsel]  # noqa: E731
    Q = chunk or cfg.D
    Vg = sl(x["v"]) * sl(vp).repeat_interleave(2, dim=-1)
    h0 = x["h0"].double()[bsel][:, hsel] if x.get("h0") is not None else None
    Y, hr = o.ssd_chunkwise_scan(sl(A), sl(x["k"]), Vg, sl(x["beta"]), Q, 2, h0=h0, return_final=True)
    yr = o.readout(Y, sl(x["q"]), sl(x["sel_C"]))
    ys, hs = y[bsel][:, :, hsel], hf[bsel][:, hsel]
    ey, eh, en = rel(ys, yr), rel(hs, hr), state_norm_rel(hs, hr)
    log(f"   rel err y {ey:.2e}  h_final {eh:.2e}  state-norm {en:.2e}")
    if cfg.dtype == "fp32":
        assert ey <= 1e-4 and eh <= 1e-4
    else:
        assert ey <= 2e-2 and en <= 1e-3


def test_fused_abar_equals_scan_level_forward_fp32():
    """fp32: with A_bar and vp computed by the oracle's formula, the gate-level entry
    reproduces the scan-level entry (which computes them in the kernel) to rounding."""
    from cdssm_hip import chunkwise_delta_scan
    from cdssm_hip.scan import chunkwise_delta_scan_abar
    cfg = ScanConfig("t", B=1, H=8, L=256, D=64, dtype="fp32", h0_std=0.1)
    x = draw_inputs(cfg, seed=1)
    A, vp = o.scan_dynamics(x["alpha"].double(), x["omega"].double(), x["dt"].double(), x["r"].double(), x["c"])
    g = to_dev(x)
    y1, h1 = chunkwise_delta_scan_abar(g["q"], g["k"], g["v"], g["beta"], g["sel_C"], A.float().to(DEV),
                                       vp.float().to(DEV), h0=g["h0"])
    y2, h2 = chunkwise_delta_scan(g["q"], g["k"], g["v"], g["beta"], g["sel_C"], g["dt"], g["r"], g["alpha"],
                                  g["omega"], g["c"], h0=g["h0"])
    e1, e2 = rel(y1, y2), rel(h1, h2)
    log(f"   abar vs scan-level: y {e1:.2e}  h_final {e2:.2e}")
    assert e1 <= 1e-4 and e2 <= 1e-4


GRAD_CASES = [
    ("fp32_h0_ragged", ScanConfig("t", B=2, H=5, L=300, D=64, dtype="fp32", h0_std=0.1), None),
    ("fp32_D128_chunk20", ScanConfig("t", B=1, H=3, L=230, D=128, dtype="fp32", h0_std=0.1), 20),
    ("fp32_one_round_multi_segment", ScanConfig("t", B=1, H=8, L=1500, D=64, dtype="fp32", h0_std=0.1), None),
    ("bf16_D64", ScanConfig("t", B=2, H=16, L=640, D=64), None),
    ("bf16_D128_h0", ScanConfig("t", B=1, H=9, L=333, D=128, omega_std=3.0, h0_std=0.1), None),
]


@pytest.mark.parametrize("name,cfg,chunk", GRAD_CASES, ids=[c[0] for c in GRAD_CASES])
def test_fused_abar_gradients_match_oracle(name, cfg, chunk):
    """ChunkwiseDeltaScanAbarFn (cdssm_fused_scan_fwd_abar_train + cdssm_fused_scan_bwd_abar) against fp64
    autograd through the oracle's SSDChunkwiseScan with the reference's correction backward
    (exact_correction.cu:213-382) and the readout: gradients of q, k, v, beta, sel_C, A_bar, vp and h0 for
    cotangents on y and h_final.  fp32 <= 1e-4, bf16 <= 2e-2 normwise per tensor."""
    from cdssm_hip import ChunkwiseDeltaScanAbarFn
    log(f"[fused abar grads] {name}: B{cfg.B} H{cfg.H} L{cfg.L} D{cfg.D} {cfg.dtype} chunk={chunk or cfg.D}")
    x = draw_inputs(cfg, seed=0)
    dtype = x["q"].dtype
    A, vp = o.scan_dynamics(x["alpha"].double(), x["omega"].double(), x["dt"].double(), x["r"].double(), x["c"])
    x["A_bar"], x["vp"] = A.to(dtype), vp.to(dtype)
    gy, gh = cotangents(cfg)
    names = ["q", "k", "v", "beta", "sel_C", "A_bar", "vp"]
    Q = chunk or cfg.D
    ref = {n: x[n].double().clone().requires_grad_(True) for n in names}
    h0r = x["h0"].double().clone().requires_grad_(True) if x.get("h0") is not None else None
    Vg = ref["v"] * ref["vp"].repeat_interleave(2, dim=-1)
    Y, hr = o.ssd_chunkwise_scan(ref["A_bar"], ref["k"], Vg, ref["beta"], Q, 2, h0=h0r, return_final=True,
                                 correction_fn=o.correction_with_reference_grad)
    yr = o.readout(Y, ref["q"], ref["sel_C"])
    torch.autograd.backward([yr, hr], [gy.to(dtype).double(), gh.double()])
    got = {n: x[n].to(DEV).clone().requires_grad_(True) for n in names}
    h0g = x["h0"].to(DEV).clone().requires_grad_(True) if x.get("h0") is not None else None
    y, hf = ChunkwiseDeltaScanAbarFn.apply(*[got[n] for n in names], h0g, chunk)
    torch.autograd.backward([y, hf], [gy.to(DEV, dtype), gh.to(DEV)])
    torch.cuda.synchronize()
    errs = {"y": rel(y, yr)}
    errs.update({n: rel(got[n].grad, ref[n].grad) for n in names})
    if h0g is not None:
        errs["h0"] = rel(h0g.grad, h0r.grad)
    log("   " + "  ".join(f"{n} {e:.1e}" for n, e in errs.items()))
    tol = 1e-4 if cfg.dtype == "fp32" else 2e-2
    bad = {n: e for n, e in errs.items() if not e <= tol}
    assert not bad, f"beyond {tol}: {bad}"
