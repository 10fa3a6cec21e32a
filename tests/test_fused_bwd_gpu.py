"""GPU parity of the fused backward (cdssm_fused_scan_bwd) against the oracle.

The reference gradient is torch autograd through the fp64 oracle with the
reference's correction-pass backward attached (oracle fused_scan,
grad_mode="reference"), on the same inputs and the same cotangents.
Tolerances per gradient tensor, normwise max|g-ref|/max|ref|:
fp32 inputs <= 1e-4, bf16 inputs <= 2e-2.
"""

import contextlib
import math

import pytest
import torch

from _gpu_util import DEV, GRAD_NAMES as NAMES, ScanConfig, cotangents, draw_inputs, log, oracle_grads, rel, select, to_dev

pytestmark = pytest.mark.gpu


def hip_grads(x, gy, gh, chunk_size=None):
    from cdssm_hip import chunkwise_delta_scan_train
    g = to_dev(x)
    leaves = {n: g[n].clone().requires_grad_(True) for n in NAMES}
    h0 = g.get("h0")
    if h0 is not None:
        h0 = h0.clone().requires_grad_(True)
    y, hf = chunkwise_delta_scan_train(*[leaves[n] for n in NAMES], g["c"], h0=h0, chunk_size=chunk_size)
    torch.autograd.backward([y, hf], [gy.to(DEV, y.dtype), gh.to(DEV)])
    torch.cuda.synchronize()
    out = {n: leaves[n].grad.cpu() for n in NAMES}
    if h0 is not None:
        out["h0"] = h0.grad.cpu()
    return out


CASES = [
    ("C0_fp32", ScanConfig("C0", B=1, H=4, L=512, D=64, dtype="fp32"), None),
    ("fp32_h0_ragged", ScanConfig("t", B=2, H=3, L=300, D=64, dtype="fp32", h0_std=0.1), None),
    ("fp32_D128_h0", ScanConfig("t", B=1, H=2, L=333, D=128, dtype="fp32", h0_std=0.1), None),
    ("fp32_chunk32", ScanConfig("t", B=1, H=2, L=200, D=64, dtype="fp32", h0_std=0.1), 32),
    # chunk % 8 in 1..4: the main pass's token loop runs past round_up(chunk, 4)
    ("fp32_chunk20", ScanConfig("t", B=1, H=5, L=230, D=64, dtype="fp32", h0_std=0.1), 20),
    ("bf16_D128_chunk100", ScanConfig("t", B=1, H=3, L=300, D=128, h0_std=0.1), 100),
    ("bf16_D64", ScanConfig("t", B=2, H=4, L=640, D=64), None),
    ("bf16_D128", ScanConfig("t", B=1, H=3, L=512, D=128, h0_std=0.1), None),
]


@contextlib.contextmanager
def forward_path(path):
    from cdssm_hip import set_forward_path
    prev = set_forward_path(path)
    try:
        yield
    finally:
        set_forward_path(prev)


@pytest.mark.parametrize("path", ["four_launch", "one_pass"])
@pytest.mark.parametrize("name,cfg,chunk", CASES, ids=[c[0] for c in CASES])
def test_fused_bwd_matches_oracle(name, cfg, chunk, path):
    """Backward from the training forward's workspace, as written by either forward path."""
    log(f"[fused bwd] {name} (forward {path}): B{cfg.B} H{cfg.H} L{cfg.L} D{cfg.D} {cfg.dtype} "
        f"chunk={chunk or cfg.D}")
    x = draw_inputs(cfg, seed=0)
    gy, gh = cotangents(cfg)
    ref = oracle_grads(x, gy, gh, chunk)
    with forward_path(path):
        got = hip_grads(x, gy, gh, chunk)
    tol = 1e-4 if cfg.dtype == "fp32" else 2e-2
    errs = {n: rel(got[n], ref[n]) for n in ref}
    log("   " + "  ".join(f"{n} {e:.1e}" for n, e in errs.items()))
    bad = {n: e for n, e in errs.items() if not e <= tol}
    assert not bad, f"gradients beyond {tol}: {bad}"


@pytest.mark.parametrize("dtype,D", [("bf16", 64), ("fp32", 128)])
def test_fused_bwd_vanishing_transitions_match_oracle(dtype, D):
    """A few tokens of head 1 with a vanishing transition: alpha = 2, omega = 0,
    dt = 1 and r = 1 give tau * alpha = 1, so E sits at its 1e-8 floor and
    |a_t|^2 = 1e-8^(c r) is below the fp32 range.  The main pass's rescaled
    frames need every segment's rotation products within 2^-120 .. 2^120, so
    the waves holding those tokens take the unscaled step and the rest the
    rescaled one, in the same call; both must match the oracle."""
    cfg = ScanConfig("t", B=2, H=4, L=640, D=D, dtype=dtype)
    log(f"[fused bwd vanishing a] B2 H4 L640 D{D} {dtype}")
    x = draw_inputs(cfg, seed=5)
    x["alpha"][1] = 2.0
    x["omega"][1] = 0.0
    dt, r = x["dt"].clone(), x["r"].clone()
    for b, t in ((0, 70), (0, 71), (0, 400), (1, 200)):
        dt[b, t, 1] = 1.0
        r[b, t, 1] = 1.0
    x["dt"], x["r"] = dt, r
    gy, gh = cotangents(cfg)
    ref = oracle_grads(x, gy, gh)
    got = hip_grads(x, gy, gh)
    tol = 1e-4 if dtype == "fp32" else 2e-2
    errs = {n: rel(got[n], ref[n]) for n in ref}
    log("   " + "  ".join(f"{n} {e:.1e}" for n, e in errs.items()))
    bad = {n: e for n, e in errs.items() if not e <= tol}
    assert not bad, f"gradients beyond {tol}: {bad}"


def test_fused_bwd_full_c2_sequences_match_oracle():
    """C2 shape (B4 H24 L8192 D128, bf16) on the GPU; selected sequences re-derived by the oracle.

    Per-(b, h) gradients of per-token inputs depend only on that sequence and are
    compared on the full-shape run.  The per-head alpha/omega gradients sum over
    batch rows, so they are compared on a second HIP run over the one selected
    batch row (all 24 heads), whose sums then cover exactly the oracle's row.
    """
    cfg = ScanConfig("C2", B=4, H=24, L=8192, D=128)
    log("[fused bwd full] C2 B4 H24 L8192 D128 bf16")
    x = draw_inputs(cfg, seed=0)
    gy, gh = cotangents(cfg)
    got = hip_grads(x, gy, gh)
    for n in NAMES:
        assert torch.isfinite(got[n].float()).all(), n
    b, heads = [2], [0, 23]
    bt, ht = torch.tensor(b), torch.tensor(heads)
    xs = select(x, b, heads)
    gys = gy.index_select(0, bt).index_select(2, ht)
    ghs = gh.index_select(0, bt).index_select(1, ht)
    ref = oracle_grads(xs, gys, ghs)
    errs = {}
    for n in ("q", "k", "v", "beta", "sel_C", "dt", "r"):
        gsel = got[n].index_select(0, bt).index_select(2, ht)
        errs[n] = rel(gsel, ref[n])
    log("   one-row run for the per-head sums (B1 H24 L8192)")
    row = hip_grads(select(x, b), gy.index_select(0, bt), gh.index_select(0, bt))
    for n in ("alpha", "omega"):
        errs[n] = rel(row[n].index_select(0, ht), ref[n])
    log("   " + "  ".join(f"{n} {e:.1e}" for n, e in errs.items()))
    assert all(e <= 2e-2 for e in errs.values()), errs


def test_one_launch_bwd_carry_past_the_anchor_matches_oracle():
    """B1 H8 L38400 D64 bf16 with h0: 600 chunks, 150 look-back segments, so the
    one-launch correction adjoint + reverse carry folds from published anchor
    states (one every 63 segments, counted from the right).  Both kernels are
    forced onto their one-launch paths (the call raises if it cannot take them);
    the oracle re-derives two heads, every gradient including alpha/omega (B = 1)."""
    cfg = ScanConfig("t", B=1, H=8, L=38400, D=64, h0_std=0.1)
    log("[fused bwd anchor] B1 H8 L38400 D64 bf16 h0, one-launch forward and carry")
    x = draw_inputs(cfg, seed=3)
    gy, gh = cotangents(cfg, seed=11)
    with forward_path("one_pass"):
        got = hip_grads(x, gy, gh)
    from cdssm_hip import lookback_status
    assert lookback_status() == 0, "a look-back wait timed out"
    heads = [1, 6]
    ht = torch.tensor(heads)
    ref = oracle_grads(select(x, None, heads), gy.index_select(2, ht), gh.index_select(1, ht))
    errs = {}
    for n in NAMES:
        g = got[n].index_select(0, ht) if n in ("alpha", "omega") else got[n].index_select(2, ht)
        errs[n] = rel(g, ref[n])
    errs["h0"] = rel(got["h0"].index_select(1, ht), ref["h0"])
    log("   " + "  ".join(f"{n} {e:.1e}" for n, e in errs.items()))
    assert all(e <= 2e-2 for e in errs.values()), errs


def test_fused_bwd_c3_shape_sequences_match_oracle():
    """C3 shape (B1 H32 L65536 D64 bf16, fast-rotating heads, h0 ~ N(0, 0.1)) forward +
    backward on the GPU; the oracle re-derives one head's gradients (B = 1, so the
    head's alpha/omega gradients too)."""
    cfg = ScanConfig("C3", B=1, H=32, L=65536, D=64, omega_std=3.0, h0_std=0.1)
    log("[fused bwd C3] B1 H32 L65536 D64 bf16 h0")
    x = draw_inputs(cfg, seed=0)
    gy, gh = cotangents(cfg)
    got = hip_grads(x, gy, gh)
    for n in NAMES:
        assert torch.isfinite(got[n].float()).all(), n
    heads = [9]
    ht = torch.tensor(heads)
    ref = oracle_grads(select(x, None, heads), gy.index_select(2, ht), gh.index_select(1, ht))
    errs = {}
    for n in NAMES:
        g = got[n].index_select(0, ht) if n in ("alpha", "omega") else got[n].index_select(2, ht)
        errs[n] = rel(g, ref[n])
    errs["h0"] = rel(got["h0"].index_select(1, ht), ref["h0"])
    log("   " + "  ".join(f"{n} {e:.1e}" for n, e in errs.items()))
    assert all(e <= 2e-2 for e in errs.values()), errs


def test_one_pass_training_forward_writes_the_four_launch_records():
    """The training forward's workspace (entering state of every chunk, chunk
    rotations, per-token records, g_t, z checkpoints, correction state at chunk
    ends) is the backward's input: the one-pass
    kernel must leave the same values there as the four-launch scan (fp32,
    several look-back segments, ragged last chunk, h0)."""
    from cdssm_hip.scan import chunkwise_delta_scan_fwd
    cfg = ScanConfig("t", B=2, H=5, L=64 * 4 * 5 + 37, D=64, dtype="fp32", h0_std=0.1)
    log("[fused fwd train] one-pass vs four-launch workspace: B2 H5 L1317 D64 fp32")
    g = to_dev(draw_inputs(cfg, seed=8))
    a = [g[n] for n in ("q", "k", "v", "beta", "sel_C", "dt", "r")]
    outs = {}
    for path in ("one_pass", "four_launch"):
        with forward_path(path):
            y, hf, ws = chunkwise_delta_scan_fwd(*a, g["alpha"], g["omega"], g["c"], h0=g["h0"], train=True)
            torch.cuda.synchronize()
        outs[path] = (y.cpu(), hf.cpu(), ws.view(-1, 2).cpu())
    B, L, H, D, Q = cfg.B, cfg.L, cfg.H, cfg.D, cfg.D
    NC = -(-L // Q)
    S = -(-NC // 16)
    n_states, n_gam = B * NC * H * D, B * NC * H
    carry = n_states + n_gam + B * H * S * (D + 1)
    off_saved = carry + (carry & 1)
    NSEG, NCK = -(-NC // 4), -(-Q // 8) * 8 // 8
    NGRP = -(-NSEG // 8)  # group maps of the two-level look-back fold
    # look-back area, control block, group maps
    off_zck = off_saved + 5 * B * L * H + B * NSEG * H * (2 * D + 2) + 8 + B * NGRP * H * (D + 1)
    n_zck = B * NC * H * NCK * D
    regions = {"states": (0, n_states), "gam": (n_states, n_states + n_gam),
               "saved": (off_saved, off_saved + 4 * B * L * H),
               "gsaved": (off_saved + 4 * B * L * H, off_saved + 5 * B * L * H),
               "z checkpoints": (off_zck, off_zck + n_zck),
               "c^ at chunk ends": (off_zck + n_zck, off_zck + n_zck + B * NC * H * D)}
    (y1, h1, w1), (y4, h4, w4) = outs["one_pass"], outs["four_launch"]
    assert rel(y1, y4) <= 1e-5 and rel(h1, h4) <= 1e-5
    # checkpoint slots past a ragged last chunk's token loop are not written
    nt_last = L - (NC - 1) * Q
    ck_used = torch.ones(B, NC, H, NCK, D, 2, dtype=torch.bool)
    ck_used[:, NC - 1, :, -(-nt_last // 8) * 8 // 8:] = False
    for name, (lo, hi) in regions.items():
        a1, a4 = w1[lo:hi], w4[lo:hi]
        if name == "z checkpoints":
            a1, a4 = a1.reshape(ck_used.shape)[ck_used], a4.reshape(ck_used.shape)[ck_used]
        e = rel(a1, a4)
        log(f"   {name}: rel diff {e:.1e}")
        assert e <= 1e-5, name
