"""Synthetic scan workloads: the five BASELINE configurations and their input draws.

Inputs follow the configuration text: q, k ~ N(0,1) then L2-normalised over D
with the reference formula x * rsqrt(sum x^2 + 1e-6) (normalize_kq.cu:75-79);
v ~ N(0,1); beta = sigmoid(N(0,1)) * sigmoid(N(0,1)); sel_C = sigmoid(N(0,1));
r = sigmoid(N(0,1)); per head alpha = softplus(N(-1,1)), omega = pi * N(0,s_omega);
dt = softplus(N(0,1)) / (alpha + |omega| + 1e-6) + softplus(N(-2,1));
c = ln(L); h0 = 0, or N(0, 0.1) (0.1 read as the standard deviation).

Draw order is fixed (the order of the fields in ``draw_inputs``) and all draws
come from one ``torch.Generator`` seeded with ``seed``.  bf16 workloads round
the drawn per-token tensors to bf16 once; alpha, omega, h0 stay fp32 (they
are per-head parameters / the carried state).
"""

from __future__ import annotations

import math
from dataclasses import dataclass, replace
from typing import Dict, Optional

import torch


@dataclass(frozen=True)
class ScanConfig:
    name: str
    B: int
    H: int
    L: int
    D: int
    N: int = 2
    dtype: str = "bf16"          # per-token input dtype: "bf16" or "fp32"
    omega_std: float = 1.0       # omega = pi * N(0, omega_std)
    h0_std: float = 0.0          # 0 => zero initial state
    backward: bool = False       # fwd+bwd workload

    @property
    def Q(self) -> int:
        return self.D

    @property
    def NC(self) -> int:
        return math.ceil(self.L / self.Q)

    @property
    def c(self) -> float:
        return math.log(self.L)

    @property
    def torch_dtype(self) -> torch.dtype:
        return torch.bfloat16 if self.dtype == "bf16" else torch.float32

    def scaled(self, **kw) -> "ScanConfig":
        return replace(self, **kw)


CONFIGS: Dict[str, ScanConfig] = {
    "C0": ScanConfig("C0", B=1, H=4, L=512, D=64, dtype="fp32"),
    "C1": ScanConfig("C1", B=8, H=16, L=4096, D=64),
    "C2": ScanConfig("C2", B=4, H=24, L=8192, D=128, backward=True),
    "C3": ScanConfig("C3", B=1, H=32, L=65536, D=64, omega_std=3.0, h0_std=0.1),
    # the scan inside one config-4 block (B8 L2048, 16 heads x 64), scan-level inputs: for the kernel's phase
    # stamps at that shape (the block itself calls the gate-level form, the same kernel structure)
    "C4scan": ScanConfig("C4scan", B=8, H=16, L=2048, D=64),
}


def _normalize(x: torch.Tensor) -> torch.Tensor:
    return x * torch.rsqrt((x * x).sum(-1, keepdim=True) + 1e-6)


def draw_inputs(cfg: ScanConfig, seed: int = 0, device: str = "cpu",
                gen_device: str = "cpu") -> Dict[str, torch.Tensor]:
    """Draw one seeded input set for ``cfg``.

    Returns q, k, v, beta, sel_C, dt, r (per token; cfg dtype), alpha, omega
    (H,) fp32, h0 (B,H,N,D) fp32 or None, and the scalar c.
    ``gen_device`` selects the generator (cpu draws are the reproducible ones
    used by fixtures; large bench shapes may draw on the GPU).
    """
    B, H, L, D, N = cfg.B, cfg.H, cfg.L, cfg.D, cfg.N
    g = torch.Generator(device=gen_device)
    g.manual_seed(seed)
    f32 = dict(dtype=torch.float32, device=gen_device, generator=g)

    def normal(*shape, mean=0.0, std=1.0):
        return torch.randn(*shape, **f32) * std + mean

    q = _normalize(normal(B, L, H, D))
    k = _normalize(normal(B, L, H, D))
    v = normal(B, L, H, N)
    beta = torch.sigmoid(normal(B, L, H)) * torch.sigmoid(normal(B, L, H))
    sel_C = torch.sigmoid(normal(B, L, H))
    r = torch.sigmoid(normal(B, L, H))
    dt_a = normal(B, L, H)
    dt_b = normal(B, L, H, mean=-2.0)
    alpha = torch.nn.functional.softplus(normal(H, mean=-1.0))
    omega = math.pi * normal(H, std=cfg.omega_std)
    dt = torch.nn.functional.softplus(dt_a) / (alpha + omega.abs() + 1e-6) \
        + torch.nn.functional.softplus(dt_b)
    h0 = normal(B, H, N, D, std=cfg.h0_std) if cfg.h0_std > 0 else None

    td = cfg.torch_dtype
    out = dict(q=q.to(td), k=k.to(td), v=v.to(td), beta=beta.to(td), sel_C=sel_C.to(td),
               dt=dt.to(td), r=r.to(td), alpha=alpha, omega=omega, h0=h0)
    out = {n: (t.to(device) if t is not None else None) for n, t in out.items()}
    out["c"] = cfg.c
    return out


def scan_bytes(cfg: ScanConfig, backward: Optional[bool] = None, h0: Optional[bool] = None) -> Dict[str, int]:
    """Algorithmic HBM bytes of the fused scan.

    fwd = B*H*L*(2D + 2N + 4)*s + B*H*N*D*4*(1 + [h0 != 0]):
      read q, k (D each), v (N), beta, sel_C, dt, r; write y (N); write the fp32
      final state (+ read h0).
    bwd = B*H*L*(4D + 3N + 8)*s: re-read the 2D+N+4 inputs and dy (N), write
      dq, dk, dv, dbeta, dsel_C, ddt, dr.  Per-head dalpha / domega are negligible.
    """
    s = 2 if cfg.dtype == "bf16" else 4
    has_h0 = (cfg.h0_std > 0) if h0 is None else h0
    bwd = cfg.backward if backward is None else backward
    BHL = cfg.B * cfg.H * cfg.L
    D, N = cfg.D, cfg.N
    fwd = BHL * (2 * D + 2 * N + 4) * s + cfg.B * cfg.H * N * D * 4 * (1 + int(has_h0))
    out = {"fwd": fwd}
    if bwd:
        out["bwd"] = BHL * (4 * D + 3 * N + 8) * s
    return out
