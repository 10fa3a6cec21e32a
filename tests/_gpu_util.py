"""Helpers shared by the GPU parity tests (imported by tests only)."""

from __future__ import annotations

import sys

import torch

from cdssm_hip.workloads import ScanConfig, draw_inputs  # noqa: F401
from oracle import cdssm_oracle as o

DEV = torch.device("cuda:0") if torch.cuda.is_available() else None
TOKEN_KEYS = ("q", "k", "v", "beta", "sel_C", "dt", "r")


def log(msg: str) -> None:
    print(msg, flush=True)
    sys.stdout.flush()


def to_dev(x: dict) -> dict:
    return {n: (t.to(DEV) if isinstance(t, torch.Tensor) else t) for n, t in x.items()}


def rel(a: torch.Tensor, b: torch.Tensor) -> float:
    """Normwise relative error max|a-b| / max|b| (fp64, on the CPU)."""
    a = a.detach().double().cpu()
    b = b.detach().double().cpu()
    den = float(b.abs().max())
    return float((a - b).abs().max()) / (den if den > 0 else 1.0)


def state_norm_rel(a: torch.Tensor, b: torch.Tensor) -> float:
    """max over (b, h) of | ||a|| - ||b|| | / ||b||, norms over the (N, D) state."""
    a = a.detach().double().cpu().flatten(2)
    b = b.detach().double().cpu().flatten(2)
    na, nb = a.norm(dim=-1), b.norm(dim=-1)
    return float(((na - nb).abs() / nb.clamp_min(1e-30)).max())


def select(x: dict, batches=None, heads=None) -> dict:
    """Slice a drawn input set to some batch rows / heads (CPU tensors)."""
    out = dict(x)
    bi = None if batches is None else torch.as_tensor(list(batches))
    hi = None if heads is None else torch.as_tensor(list(heads))
    for n in TOKEN_KEYS:
        t = x[n]
        if bi is not None:
            t = t.index_select(0, bi)
        if hi is not None:
            t = t.index_select(2, hi)
        out[n] = t
    for n in ("alpha", "omega"):
        out[n] = x[n] if hi is None else x[n].index_select(0, hi)
    if x.get("h0") is not None:
        t = x["h0"]
        if bi is not None:
            t = t.index_select(0, bi)
        if hi is not None:
            t = t.index_select(1, hi)
        out["h0"] = t
    return out


def oracle_fwd(x: dict, chunk_size=None):
    """fp64 oracle fused forward (R-mode) on the CPU inputs in ``x``.

    The scan is independent per (b, h), so a ``select``-ed slice gives exactly
    the oracle's answer for those sequences.
    """
    d = {n: (t.double() if isinstance(t, torch.Tensor) else t) for n, t in x.items()}
    return o.fused_scan(d["q"], d["k"], d["v"], d["beta"], d["sel_C"], d["dt"], d["r"], d["alpha"],
                        d["omega"], d["c"], h0=d.get("h0"), chunk_size=chunk_size)


GRAD_NAMES = ("q", "k", "v", "beta", "sel_C", "dt", "r", "alpha", "omega")


def oracle_grads(x: dict, gy: torch.Tensor, gh: torch.Tensor, chunk_size=None) -> dict:
    """Reference-mode gradients of sum(y * gy) + sum(h_final * gh) from the fp64 oracle
    (autograd through the restatement, with the reference's correction-pass backward)."""
    d = {n: (x[n].double().clone().requires_grad_(True)) for n in GRAD_NAMES}
    h0 = x.get("h0")
    h0d = h0.double().clone().requires_grad_(True) if h0 is not None else None
    y, hf = o.fused_scan(*[d[n] for n in GRAD_NAMES], x["c"], h0=h0d, chunk_size=chunk_size,
                         grad_mode="reference")
    loss = (y * gy.double()).sum() + (hf * gh.double()).sum()
    wrt = [d[n] for n in GRAD_NAMES] + ([h0d] if h0d is not None else [])
    gs = torch.autograd.grad(loss, wrt)
    out = dict(zip(GRAD_NAMES, gs[:9]))
    if h0d is not None:
        out["h0"] = gs[9]
    return out


def cotangents(cfg, seed: int = 7):
    """Seeded (dy, dh_final) for a config; dy rounded to bf16 for bf16 configs."""
    gen = torch.Generator().manual_seed(seed)
    gy = torch.randn(cfg.B, cfg.L, cfg.H, cfg.N, generator=gen)
    gh = torch.randn(cfg.B, cfg.H, cfg.N, cfg.D, generator=gen)
    if cfg.dtype == "bf16":
        gy = gy.bfloat16().float()
    return gy, gh
