"""The no-allocation forward entry point (cdssm_fused_scan_fwd_noalloc) against the
workspace forward (cdssm_fused_scan_fwd), both called through the C-ABI.

The two run the same kernels with the same fixed fold order, so the results
must be bit-identical (the bar for the same arithmetic on the same inputs).
Two no-alloc calls in a row, the second with a smaller input, check that the
static scratch left by one call does not leak into the next (look-back flags
of the first call must not count in the second).
"""

import ctypes

import pytest
import torch

from _gpu_util import DEV, ScanConfig, draw_inputs, log, to_dev

pytestmark = pytest.mark.gpu

TOKEN = ("q", "k", "v", "beta", "sel_C", "dt", "r")


def _call(lib, fn_name, g, cfg, y, hf, ws=None):
    from cdssm_hip import _lib
    args = [_lib.DTYPE_CODE[g["q"].dtype]] + [_lib.ptr(g[n]) for n in TOKEN]
    args += [_lib.ptr(g["alpha"]), _lib.ptr(g["omega"]), float(g["c"]), _lib.ptr(g.get("h0")), _lib.ptr(y),
             _lib.ptr(hf)]
    if ws is not None:
        args.append(_lib.ptr(ws))
    args += [cfg.B, cfg.L, cfg.H, cfg.D, cfg.N, cfg.D, _lib.stream_of(DEV)]
    st = getattr(lib, fn_name)(*args)
    _lib.check(st, fn_name)


def _both(cfg, seed):
    from cdssm_hip import _lib
    lib = _lib.load()
    g = to_dev(draw_inputs(cfg, seed=seed))
    dtype = g["q"].dtype
    out = {}
    for name in ("cdssm_fused_scan_fwd", "cdssm_fused_scan_fwd_noalloc"):
        y = torch.full((cfg.B, cfg.L, cfg.H, cfg.N), float("nan"), dtype=dtype, device=DEV)
        hf = torch.full((cfg.B, cfg.H, cfg.N, cfg.D), float("nan"), dtype=torch.float32, device=DEV)
        ws = None
        if name == "cdssm_fused_scan_fwd":
            nbytes = lib.cdssm_fused_scan_workspace_bytes(cfg.B, cfg.L, cfg.H, cfg.D, cfg.N, cfg.D)
            ws = torch.empty(nbytes // 4, dtype=torch.float32, device=DEV)
        _call(lib, name, g, cfg, y, hf, ws)
        torch.cuda.synchronize()
        out[name] = (y.cpu(), hf.cpu())
    return out


@pytest.mark.parametrize("path", ["auto", "four_launch"])
def test_noalloc_forward_matches_workspace_forward_on_two_calls(path):
    from cdssm_hip import lookback_status, set_forward_path
    prev = set_forward_path(path)
    try:
        for cfg, seed in ((ScanConfig("C1", B=8, H=16, L=4096, D=64), 0),
                          (ScanConfig("t", B=1, H=5, L=700, D=64, dtype="fp32", h0_std=0.1), 1)):
            log(f"[no-alloc fwd] {path}: B{cfg.B} H{cfg.H} L{cfg.L} D{cfg.D} {cfg.dtype}")
            out = _both(cfg, seed)
            (y0, h0), (y1, h1) = out["cdssm_fused_scan_fwd"], out["cdssm_fused_scan_fwd_noalloc"]
            assert torch.isfinite(y1.float()).all() and torch.isfinite(h1).all()
            assert torch.equal(y0, y1) and torch.equal(h0, h1), "no-alloc result differs from the workspace call"
    finally:
        set_forward_path(prev)
    assert lookback_status() == 0, "a look-back wait timed out"
