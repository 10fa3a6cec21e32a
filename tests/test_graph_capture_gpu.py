"""The one-launch passes under HIP graph capture.

The one-pass forward and the backward's one-launch correction adjoint + carry
exchange chunk summaries between workgroups through flags tagged with a
per-call epoch.  The epoch is drawn on the device: by a one-thread kernel
launched before the pass, or, for the calls PreparedForward / PreparedBackward
make after their first (captured here), by the previous call's last workgroup,
so a captured graph gets a fresh epoch on every replay either way.  These
tests capture the passes once, then rewrite the bound inputs in
place with new seeds between replays and check every replay against the fp64
oracle (and against an eager call on the same inputs).  Tolerances as the
other parity tests: fp32 <= 1e-4; bf16 y <= 2e-2, state norms <= 1e-3.
"""

import contextlib

import pytest
import torch

from _gpu_util import (DEV, GRAD_NAMES, ScanConfig, cotangents, draw_inputs, log, oracle_fwd, oracle_grads, rel,
                       select, state_norm_rel, to_dev)

pytestmark = pytest.mark.gpu

TOKEN_INPUTS = ("q", "k", "v", "beta", "sel_C", "dt", "r", "alpha", "omega")


@contextlib.contextmanager
def forward_path(path):
    from cdssm_hip import set_forward_path
    prev = set_forward_path(path)
    try:
        yield
    finally:
        set_forward_path(prev)


def _rewrite(static: dict, x: dict) -> None:
    """Copy a drawn input set into the tensors a captured graph reads."""
    for n in TOKEN_INPUTS:
        static[n].copy_(x[n].to(DEV))
    if static.get("h0") is not None:
        static["h0"].copy_(x["h0"].to(DEV))


def test_captured_one_pass_forward_replays_match_oracle_c1():
    """C1 (B8 H16 L4096 D64 bf16), one-pass forward captured once; three replays on
    three input sets written in place; selected sequences checked against the oracle."""
    from cdssm_hip import lookback_status
    from cdssm_hip.scan import PreparedForward
    cfg = ScanConfig("C1", B=8, H=16, L=4096, D=64)
    log("[graph fwd] C1 B8 H16 L4096 D64 bf16, one-pass forward captured")
    static = to_dev(draw_inputs(cfg, seed=0))
    with forward_path("one_pass"):
        pf = PreparedForward(*[static[n] for n in TOKEN_INPUTS], static["c"])
        pf()  # eager call first: fills the launcher's occupancy cache outside capture
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            pf()
    torch.cuda.synchronize()
    assert lookback_status() == 0
    first = None
    for seed in (1, 2, 3):
        x = draw_inputs(cfg, seed=seed)
        _rewrite(static, x)
        graph.replay()
        torch.cuda.synchronize()
        y, hf = pf.y.cpu().clone(), pf.h_final.cpu().clone()
        if first is None:
            first = (y, hf)
        b, heads = [seed % cfg.B, 7], [seed % cfg.H, 15]
        yr, hr = oracle_fwd(select(x, b, heads))
        bt, ht = torch.tensor(b), torch.tensor(heads)
        ys = y.index_select(0, bt).index_select(2, ht)
        hs = hf.index_select(0, bt).index_select(1, ht)
        ey, en = rel(ys, yr), state_norm_rel(hs, hr)
        log(f"   replay seed {seed}: rel err y {ey:.2e}  state-norm {en:.2e}")
        assert ey <= 2e-2 and en <= 1e-3, (seed, ey, en)
        # the same inputs through an eager call: identical bits (fixed fold order)
        with forward_path("one_pass"):
            pf()
        torch.cuda.synchronize()
        assert torch.equal(pf.y.cpu(), y) and torch.equal(pf.h_final.cpu(), hf), f"eager != replay (seed {seed})"
    # back to the first input set: the replay reproduces the first replay's bits
    _rewrite(static, draw_inputs(cfg, seed=1))
    graph.replay()
    torch.cuda.synchronize()
    assert torch.equal(pf.y.cpu(), first[0]) and torch.equal(pf.h_final.cpu(), first[1])
    assert lookback_status() == 0, "a look-back wait timed out"


@pytest.mark.parametrize("dtype", ["fp32", "bf16"])
def test_captured_training_forward_and_backward_replays_match_oracle(dtype):
    """PreparedForward(train=True) + PreparedBackward captured in one graph, both on
    their one-launch paths (B2 H5 L1317 D64 with h0: 21 chunks, 6 look-back segments
    per sequence); inputs and cotangents rewritten between replays; every gradient
    checked against the oracle's reference-mode gradients on every replay."""
    from cdssm_hip import lookback_status
    from cdssm_hip.scan import PreparedBackward, PreparedForward
    cfg = ScanConfig("t", B=2, H=5, L=64 * 4 * 5 + 37, D=64, dtype=dtype, h0_std=0.1)
    log(f"[graph fwd+bwd] B2 H5 L1317 D64 {dtype} h0, one-launch forward and carry captured")
    static = to_dev(draw_inputs(cfg, seed=0))
    gy0, gh0 = cotangents(cfg, seed=0)
    dy = gy0.to(DEV, static["q"].dtype).contiguous()
    dhf = gh0.to(DEV).contiguous()
    with forward_path("one_pass"):
        pf = PreparedForward(*[static[n] for n in TOKEN_INPUTS], static["c"], h0=static["h0"], train=True)
        pb = PreparedBackward(pf, dy, dhf)
        pf()
        pb()
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            pf()
            pb()
    torch.cuda.synchronize()
    tol = 1e-4 if dtype == "fp32" else 2e-2
    for seed in (4, 5, 6):
        x = draw_inputs(cfg, seed=seed)
        gy, gh = cotangents(cfg, seed=seed + 100)
        _rewrite(static, x)
        pb.dy.copy_(gy.to(DEV, pb.dy.dtype))
        pb.dh_final.copy_(gh.to(DEV))
        graph.replay()
        torch.cuda.synchronize()
        got = dict(zip(GRAD_NAMES, [g.cpu() for g in pb.grads] + [pb.dalpha.cpu(), pb.domega.cpu()]))
        got["h0"] = pb.dh0.cpu()
        ref = oracle_grads(x, gy, gh)
        yr, hr = oracle_fwd(x)
        errs = {n: rel(got[n], ref[n]) for n in ref}
        errs["y"] = rel(pf.y.cpu(), yr)
        # final state: elementwise for fp32, norms for bf16 inputs (the stated bars)
        hf_err = rel(pf.h_final.cpu(), hr) if dtype == "fp32" else state_norm_rel(pf.h_final.cpu(), hr)
        log(f"   replay seed {seed}: " + "  ".join(f"{n} {e:.1e}" for n, e in errs.items()) +
            f"  h_final {hf_err:.1e}")
        assert all(e <= tol for e in errs.values()), (seed, errs)
        assert hf_err <= (1e-4 if dtype == "fp32" else 1e-3), (seed, hf_err)
    assert lookback_status() == 0, "a look-back wait timed out"
