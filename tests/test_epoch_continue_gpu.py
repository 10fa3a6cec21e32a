"""Calls that reuse the look-back epoch left in their workspace (*_continue).

The one-launch passes tag their look-back flags with a per-call epoch.  The
plain entry points draw it with a one-thread kernel before the pass; the
*_continue entry points, which PreparedForward / PreparedBackward use after
their first call, run on the epoch that the previous call's last workgroup
left in the workspace.  If that hand-over failed, a later call would read the
previous call's flags as ready and fold stale chunk maps: its outputs would
differ from a fresh call's.  These tests run many consecutive prepared calls
with inputs rewritten in place and require each to be bit-identical to a
plain call (own workspace, epoch kernel) on the same inputs; the kernels and
their fixed fold order are the same, so any difference is a stale fold.
Shapes: a one-round one-pass forward, a persistent (multi-round) one-pass
forward, and the training forward with the backward's one-launch carry.
"""

import contextlib

import pytest
import torch

from _gpu_util import DEV, ScanConfig, cotangents, draw_inputs, log, to_dev

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
    for n in TOKEN_INPUTS:
        static[n].copy_(x[n].to(DEV))
    if static.get("h0") is not None:
        static["h0"].copy_(x["h0"].to(DEV))


def _fresh_forward(static: dict):
    from cdssm_hip.scan import chunkwise_delta_scan
    y, hf = chunkwise_delta_scan(*[static[n] for n in TOKEN_INPUTS], static["c"], h0=static.get("h0"))
    torch.cuda.synchronize()
    return y.cpu(), hf.cpu()


@pytest.mark.parametrize("name,B,H,L", [("one round", 2, 16, 4096), ("persistent", 1, 32, 65536)])
def test_continuing_forward_calls_equal_fresh_calls(name, B, H, L):
    """PreparedForward: the first call draws the epoch, the next seven reuse the
    previous call's; inputs cycle through four seeds (each seen twice)."""
    from cdssm_hip import lookback_status
    from cdssm_hip.scan import PreparedForward
    cfg = ScanConfig("c", B=B, H=H, L=L, D=64, h0_std=0.1)
    log(f"[continue fwd] {name}: B{B} H{H} L{L} D64 bf16 h0, eight prepared calls")
    static = to_dev(draw_inputs(cfg, seed=0))
    with forward_path("one_pass"):
        pf = PreparedForward(*[static[n] for n in TOKEN_INPUTS], static["c"], h0=static["h0"])
        for i, seed in enumerate((11, 12, 13, 14, 11, 12, 13, 14)):
            _rewrite(static, draw_inputs(cfg, seed=seed))
            pf()
            torch.cuda.synchronize()
            y, hf = pf.y.cpu(), pf.h_final.cpu()
            yr, hr = _fresh_forward(static)
            same = torch.equal(y, yr) and torch.equal(hf, hr)
            log(f"   call {i} seed {seed}: {'bit-identical' if same else 'DIFFERENT'} to a fresh call")
            assert same, (name, i, seed, float((y.float() - yr.float()).abs().max()))
    assert lookback_status() == 0, "a look-back wait timed out"


def test_continuing_training_forward_and_backward_equal_fresh_calls():
    """PreparedForward(train=True) + PreparedBackward (one-launch forward and carry,
    B2 H5 L1317 D64 with h0): five steps with new inputs and cotangents, each
    step's gradients bit-identical to the plain backward entry on the same
    inputs."""
    from cdssm_hip import lookback_status
    from cdssm_hip.scan import PreparedBackward, PreparedForward, chunkwise_delta_scan_bwd
    cfg = ScanConfig("t", B=2, H=5, L=64 * 4 * 5 + 37, D=64, h0_std=0.1)
    log("[continue fwd+bwd] B2 H5 L1317 D64 bf16 h0, five prepared steps")
    static = to_dev(draw_inputs(cfg, seed=0))
    gy0, gh0 = cotangents(cfg, seed=0)
    dy = gy0.to(DEV, static["q"].dtype).contiguous()
    dhf = gh0.to(DEV).contiguous()
    with forward_path("one_pass"):
        pf = PreparedForward(*[static[n] for n in TOKEN_INPUTS], static["c"], h0=static["h0"], train=True)
        pb = PreparedBackward(pf, dy, dhf)
        for step, seed in enumerate((21, 22, 23, 21, 22)):
            _rewrite(static, draw_inputs(cfg, seed=seed))
            gy, gh = cotangents(cfg, seed=seed + 100)
            pb.dy.copy_(gy.to(DEV, pb.dy.dtype))
            pb.dh_final.copy_(gh.to(DEV))
            pf()
            pb()
            torch.cuda.synchronize()
            got = [g.cpu() for g in pb.grads] + [pb.dalpha.cpu(), pb.domega.cpu(), pb.dh0.cpu()]
            yr, hr = _fresh_forward(static)
            ref = chunkwise_delta_scan_bwd(pb.dy, pb.dh_final, *[static[n] for n in TOKEN_INPUTS], static["c"],
                                           pf.workspace, True, pf.shape[-1])
            torch.cuda.synchronize()
            same_fwd = torch.equal(pf.y.cpu(), yr) and torch.equal(pf.h_final.cpu(), hr)
            same_bwd = all(torch.equal(a, b.cpu()) for a, b in zip(got, ref))
            log(f"   step {step} seed {seed}: forward {'bit-identical' if same_fwd else 'DIFFERENT'}, "
                f"backward {'bit-identical' if same_bwd else 'DIFFERENT'}")
            assert same_fwd and same_bwd, (step, seed)
    assert lookback_status() == 0, "a look-back wait timed out"


def test_first_call_under_capture_keeps_the_epoch_kernel():
    """A PreparedForward whose first call is captured holds no executed call, so the
    graph keeps the plain entry (epoch kernel in the graph); replays on rewritten
    inputs and the eager calls after them equal fresh calls."""
    from cdssm_hip import lookback_status
    from cdssm_hip.scan import PreparedForward
    cfg = ScanConfig("g", B=2, H=16, L=4096, D=64)
    log("[continue capture] B2 H16 L4096 D64 bf16, first call captured")
    static = to_dev(draw_inputs(cfg, seed=0))
    with forward_path("one_pass"):
        _fresh_forward(static)  # fills the launcher's occupancy cache outside capture
        pf = PreparedForward(*[static[n] for n in TOKEN_INPUTS], static["c"])
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            pf()
        assert not pf._continue, "a captured call must not count as executed"
        torch.cuda.synchronize()
        for seed in (31, 32, 31):
            _rewrite(static, draw_inputs(cfg, seed=seed))
            graph.replay()
            torch.cuda.synchronize()
            y, hf = pf.y.cpu().clone(), pf.h_final.cpu().clone()
            yr, hr = _fresh_forward(static)
            assert torch.equal(y, yr) and torch.equal(hf, hr), f"replay seed {seed}"
            pf()  # eager: the plain entry first, then continuing calls
            torch.cuda.synchronize()
            assert torch.equal(pf.y.cpu(), yr) and torch.equal(pf.h_final.cpu(), hr), f"eager seed {seed}"
            log(f"   seed {seed}: replay and eager call bit-identical to a fresh call")
    assert lookback_status() == 0, "a look-back wait timed out"
