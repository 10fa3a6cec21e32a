"""CPU oracle of the reference CD-SSM language-model forward (the scan's caller).

TEST INFRASTRUCTURE ONLY, like ``oracle/cdssm_oracle.py``: used by ``tests/``
as the checker; nothing in the product path imports it.

Restates, in PyTorch on the CPU (run in float64 by the tests):
  * conv1d_silu      conv1d_silu.cu:25-90 (CUDAConv1dSiLUOp.forward, ops.py:13-21)
  * rms_norm         modules.py:38-53
  * block_forward    block.py:140-229, composed from the pinned scan-path pieces
                     of cdssm_oracle (dynamics_fused_fwd, normalize_kq,
                     ssd_chunkwise_scan, readout)
  * lm_forward       model.py:38-51 (embedding, blocks, final RMSNorm, tied head)
  * group_norm_running_sums  the decode step's GroupNorm state (statistics of
                     block.py:216-223 over the positions so far)
Parameters come as a ``state_dict`` with the reference's names.

Pins (tests/test_oracle_lm.py): conv1d_silu against torch.nn.functional.conv1d
(causal padding, groups = C) followed by F.silu, i.e. a library routine with
the tap order fixed by the reference's comment (conv1d_silu.cu:74-80);
rms_norm against its closed form; block_forward by invariants (a zero
out_proj makes the block the identity; batch rows are independent) and by
closed-form special cases of its wiring: a zero readout_proj leaves
residual + out_proj(GroupNorm bias * silu(z) + D * x_conv) built from library
routines (pins the in_proj split order, the gate and the D-skip), the
value-residual lerp's direction at sigmoid(gate) = 0 and 1, and the shortcut
read out as sel_C s (q.k)^2 V_gated; group_norm_running_sums against
the groups' mean and variance (torch) and by appending a token.  Note: the model is not causal in
the reference: its GroupNorm (block.py:216-223) takes statistics over the
group's channels and all L positions, which this restatement reproduces.
"""

from __future__ import annotations

from typing import Optional

import torch
import torch.nn.functional as F

from . import cdssm_oracle as o

Tensor = torch.Tensor


def conv1d_silu(x: Tensor, weight: Tensor, bias: Tensor) -> Tensor:
    """y[b, t, c] = silu(bias[c] + sum_j w[c, j] x[b, t - (K-1) + j, c]), x = 0 before t = 0
    (conv1d_silu.cu:74-86); x (B, L, C), weight (C, 1, K) or (C, K), bias (C)."""
    B, L, C = x.shape
    w = weight.reshape(C, -1)
    K = w.shape[1]
    xp = torch.cat([x.new_zeros(B, K - 1, C), x], dim=1)
    u = bias.reshape(1, 1, C).expand(B, L, C).clone()
    for j in range(K):
        u = u + w[:, j] * xp[:, j:j + L]
    return u * torch.sigmoid(u)


def rms_norm(x: Tensor, weight: Tensor, eps: float) -> Tensor:
    """x * rsqrt(mean(x^2) + eps) * weight (modules.py:49-53)."""
    return x * torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + eps) * weight


def _linear(x: Tensor, w: Tensor, b: Optional[Tensor] = None) -> Tensor:
    y = x @ w.transpose(0, 1)
    return y if b is None else y + b


def block_gate_rows(p: dict, pre: str, x: Tensor, cfg) -> tuple:
    """The block's in_proj output, conv output and gate rows (block.py:160-181): (proj, x_conv, gate_raw)."""
    Di = cfg.d_inner
    g = lambda n: p[pre + n]  # noqa: E731
    proj = _linear(rms_norm(x, g("norm.weight"), cfg.eps_norm), g("in_proj.weight"), g("in_proj.bias"))
    x_gate = proj[..., Di:2 * Di]                                       # block.py:162-166 split order
    x_conv = conv1d_silu(x_gate, g("conv.weight"), g("conv.bias"))      # block.py:177
    gates = _linear(x_conv, g("gate_proj.weight"), g("gate_proj.bias"))
    return proj, x_conv, gates


def block_forward(p: dict, pre: str, x: Tensor, v_first: Optional[Tensor], cfg, grad_mode: str = "exact") -> tuple:
    """One CDSSMBlock.forward (block.py:140-229) with the block's parameters p[pre + name].

    grad_mode "reference" attaches the reference's own backward rules where they are not the exact
    derivative of the forward: DynamicsFusedFn.backward (dynamics_fused.cu:145-387) and
    ExactCorrectionFn.backward (exact_correction.cu:169-383); "exact" differentiates the forward."""
    N, H, D, Di = cfg.state_dim, cfg.n_heads, cfg.head_dim, cfg.d_inner
    B, L, _ = x.shape
    g = lambda n: p[pre + n]  # noqa: E731
    residual = x
    proj, x_conv, gates = block_gate_rows(p, pre, x, cfg)
    z, _, K, V = proj.split([Di, Di, Di, H * N], dim=-1)                # block.py:162-166
    K = K.reshape(B, L, H, D)
    V = V.reshape(B, L, H, N)
    if v_first is None:                                                 # block.py:169-174
        v_first = V.detach()                                            # layer 0's values, no gradient path
    else:
        V = torch.lerp(v_first, V, torch.sigmoid(g("v_residual_gate"))[None, None, :, None])
    rope = 1.0 / (cfg.rope_base ** (torch.arange(0, H, dtype=x.dtype) / H))   # block.py:59-62
    dyn = o.dynamics_with_reference_grad if grad_mode == "reference" else o.dynamics_fused_fwd
    A_bar, vp, beta, sel_C = dyn(gates, g("log_dt_scale"), rope, cfg.gating_c, cfg.bf16_omega_thresh,
                                 cfg.bf16_delta, cfg.bf16_smoothness, cfg.eps_adaptive_dt, H, N)   # block.py:184-188
    Q = _linear(x_conv, g("Q_proj.weight")).reshape(B, L, H, D)
    K, Q = o.normalize_kq(K, Q)                                         # block.py:191-192
    V_gated = V * vp.repeat_interleave(2, dim=-1)                       # block.py:194-195
    corr = o.correction_with_reference_grad if grad_mode == "reference" else None
    Y = o.ssd_chunkwise_scan(A_bar, K, V_gated, beta, cfg.chunk_size, N, correction_fn=corr)   # block.py:198
    retrieved = o.readout(Y, Q, sel_C, K=K, V_gated=V_gated,
                          shortcut_scale=g("shortcut_scale").reshape(()))  # block.py:202-211
    y = _linear(retrieved.reshape(B, L, H * N), g("readout_proj.weight"))
    y = F.group_norm(y.transpose(1, 2), cfg.ssm_norm_groups, g("ssm_norm.weight"), g("ssm_norm.bias"),
                     1e-5).transpose(1, 2)                              # block.py:216-223 (nn.GroupNorm eps)
    y = y * F.silu(z) + g("D") * x_conv
    return residual + _linear(y, g("out_proj.weight")), v_first


def group_norm_running_sums(y: Tensor, num_groups: int) -> Tensor:
    """The GroupNorm decode state after positions 0 .. L-1 of y (B, L, C): per (b, group) the shift (the
    group's first element), sum (x - shift), sum (x - shift)^2 and the count, (B, G, 4) -- the statistics
    of block.py:216-223 over every position so far, in the layout the decode step keeps.  Computed in
    float64 (the caller casts)."""
    B, L, C = y.shape
    G = int(num_groups)
    yg = y.reshape(B, L, G, C // G).double()
    k0 = yg[:, 0, :, 0]
    d = yg - k0[:, None, :, None]
    n = torch.full_like(k0, float(L * (C // G)))
    return torch.stack([k0, d.sum((1, 3)), (d * d).sum((1, 3)), n], dim=-1)


def lm_forward(p: dict, input_ids: Tensor, cfg, grad_mode: str = "exact") -> Tensor:
    """CDSSMLMHeadModel.forward (model.py:38-51): logits (B, L, vocab); grad_mode as block_forward."""
    x = p["embedding.weight"][input_ids]
    v_first = None
    for i in range(cfg.n_layers):
        x, v_first = block_forward(p, f"blocks.{i}.", x, v_first, cfg, grad_mode)
    x = rms_norm(x, p["final_norm.weight"], 2.0 ** -14)   # RMSNorm default eps (modules.py:46)
    return x @ p["embedding.weight"].transpose(0, 1)       # tied head (model.py:29-30)
