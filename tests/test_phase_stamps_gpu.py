"""The instrumentation entry cdssm_fused_scan_fwd_stamped.

It runs the inference forward's one-pass kernel with a caller buffer in which
lane 0 of every wave records the real-time counter at eight points of its
segment.  The stamps are reads of a clock and stores into that buffer only:
the call's outputs must be bit-identical to a plain call's, every wave of the
grid must leave one record, and the eight points of a record are in program
order, so they never decrease.
"""

import contextlib

import pytest
import torch

from _gpu_util import DEV, ScanConfig, draw_inputs, log, to_dev

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


def _prepared(cfg, seed=0):
    from cdssm_hip.scan import PreparedForward
    x = to_dev(draw_inputs(cfg, seed=seed))
    return PreparedForward(*[x[n] for n in TOKEN_INPUTS], x["c"], h0=x.get("h0"))


@pytest.mark.parametrize("name,B,H,L", [("one round", 2, 16, 4096), ("persistent", 1, 32, 65536)])
def test_stamped_call_equals_plain_call_and_records_every_wave(name, B, H, L):
    """bf16 D64: 8 heads per wave (4 where the 8-head grid has fewer workgroups than the GPU has
    CUs), so H/8 (H/4) head groups; segments of 4 chunks of 64 tokens; 4 waves per segment item."""
    cfg = ScanConfig("s", B=B, H=H, L=L, D=64, h0_std=0.1)
    log(f"[phase stamps] {name}: B{B} H{H} L{L} D64 bf16 h0")
    with forward_path("one_pass"):
        pf = _prepared(cfg)
        pf()
        torch.cuda.synchronize()
        y, hf = pf.y.cpu().clone(), pf.h_final.cpu().clone()
        st = pf.phase_stamps()
        torch.cuda.synchronize()
    assert torch.equal(pf.y.cpu(), y) and torch.equal(pf.h_final.cpu(), hf), "stamped call changed the outputs"
    items = (L // 64 // 4) * B * (H // 8)
    if items < torch.cuda.get_device_properties(0).multi_processor_count and H > 4:
        items *= 2  # 4 heads per wave
    assert st.shape == (items * 4, 8), (st.shape, items)
    steps = st[:, 1:] - st[:, :-1]
    assert bool((steps >= 0).all()), "a wave's stamps go backwards"
    span_us = float(st[:, 7].max() - st[:, 0].min()) * 0.01
    log(f"   {st.shape[0]} wave records, points in order; kernel span {span_us:.1f} us")
    assert 0 < span_us < 1e6


def test_stamped_call_rejects_a_short_buffer_and_the_four_launch_forward():
    from cdssm_hip import _lib
    cfg = ScanConfig("s", B=1, H=16, L=1024, D=64)
    log("[phase stamps] rejections: B1 H16 L1024 D64 bf16")
    with forward_path("one_pass"):
        pf = _prepared(cfg)
        buf = torch.zeros(8, dtype=torch.int64, device=DEV)  # 32 records of 8 words are needed
        st = pf._lib.cdssm_fused_scan_fwd_stamped(*pf._args, _lib.ptr(buf), buf.numel(), _lib.stream_of(DEV))
        assert st == -1 and "stamp words needed" in _lib.last_error()
        torch.cuda.synchronize()
        assert int(buf.abs().sum()) == 0, "a refused call wrote stamps"
    with forward_path("four_launch"):
        pf = _prepared(cfg)
        with pytest.raises(RuntimeError, match="four-launch"):
            pf.phase_stamps()


@pytest.mark.parametrize("name,B,H,L,D", [("C1-like D64", 2, 16, 2048, 64), ("D128", 1, 8, 1024, 128)])
def test_stamped_backward_equals_plain_backward_and_records_every_wave(name, B, H, L, D):
    """cdssm_fused_scan_bwd_stamped: the gradients of a stamped backward are bit-identical to a plain
    backward's of the same forward; every wave of the one-launch correction adjoint + carry (segments of
    4 chunks, 4 waves each) and every main-pass wave (one per chunk and head group) leaves a record
    whose points never decrease."""
    from cdssm_hip.scan import PreparedBackward, PreparedForward
    cfg = ScanConfig("s", B=B, H=H, L=L, D=D, h0_std=0.1)
    log(f"[bwd phase stamps] {name}: B{B} H{H} L{L} D{D} bf16 h0")
    x = to_dev(draw_inputs(cfg, seed=2))
    gen = torch.Generator().manual_seed(3)
    dy = torch.randn(B, L, H, 2, generator=gen).to(DEV)
    dhf = torch.randn(B, H, 2, D, generator=gen).to(DEV)
    with forward_path("one_pass"):
        fwd = PreparedForward(*[x[n] for n in TOKEN_INPUTS], x["c"], h0=x.get("h0"), train=True)
        bwd = PreparedBackward(fwd, dy, dhf)
        fwd()
        grads = [t.cpu().clone() for t in bwd()] + [bwd.dh0.cpu().clone()]
        corr, main = bwd.phase_stamps()
        torch.cuda.synchronize()
    again = [t.cpu() for t in bwd.grads] + [bwd.dh0.cpu()]
    assert all(torch.equal(a, b) for a, b in zip(grads, again)), "stamped backward changed the gradients"
    nc = L // 64 if D == 64 else L // 128
    assert corr.shape[0] > 0 and corr.shape[0] % 4 == 0 and main.shape[0] > 0
    assert bool(((corr[:, 1:] - corr[:, :-1]) >= 0).all()), "a correction-pass wave's stamps go backwards"
    assert bool(((main[:, 1:] - main[:, :-1]) >= 0).all()), "a main-pass wave's stamps go backwards"
    # one main-pass wave per (b, chunk, head group): head groups divide H
    assert (B * nc * H) % main.shape[0] == 0, (main.shape, B, nc, H)
    log(f"   {corr.shape[0]} correction-pass and {main.shape[0]} main-pass wave records, points in order")
