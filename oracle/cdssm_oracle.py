"""CPU oracle: a restatement of the reference CD-SSM scan path in PyTorch (CPU).

TEST INFRASTRUCTURE ONLY.  Nothing in the product path may import this module:
only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` use it, and only as the checker / the timed CPU baseline.

Every function restates one piece of the reference implementation
(indrajeetadityaroy9/Cayley-Delta-State-Space-Model) and cites the file:line it
follows.  Functions run in the dtype of their inputs; parity tests feed float64.

Layout conventions are the reference's:
  * the N state rows are N/2 complex pairs, interleaved (re, im);
  * A_bar stores conj(mu) * scale and multiplies a state row pair as a complex
    scalar (intra_chunk_scan.cu:151-162, cayley_math.cuh:20-24);
  * tensors are (B, L, H, ...) token-major.

Pinning status of each function is recorded in tests/test_oracle_*.py; the
one function whose reference behaviour is an execution artefact of an NVIDIA
GPU (fp32 rounding of --use_fast_math intrinsics, setup.py:44) is matched to
its mathematical definition, not to those artefacts.
"""

from __future__ import annotations

import math
from typing import Optional, Tuple

import torch
import torch.nn.functional as F

Tensor = torch.Tensor

EPS_DEFAULT = 1e-6          # common.cuh:142
E_CLAMP = 1e-8              # dynamics_fused.cu:114
SOFTPLUS_THRESHOLD = 20.0   # common.cuh:88-91


# --------------------------------------------------------------------------
# Elementwise helpers (common.cuh:71-96)
# --------------------------------------------------------------------------

def softplus(x: Tensor) -> Tensor:
    """softplus with the reference's threshold: x for x > 20 (common.cuh:88-91)."""
    return F.softplus(x, beta=1.0, threshold=SOFTPLUS_THRESHOLD)


def sigmoid(x: Tensor) -> Tensor:
    """1 / (1 + exp(-x)) (common.cuh:82-84)."""
    return torch.sigmoid(x)


# --------------------------------------------------------------------------
# Complex-pair arithmetic on the interleaved (re, im) layout
# --------------------------------------------------------------------------

def cmul_rows(a: Tensor, h: Tensor) -> Tensor:
    """Multiply state rows by complex scalars, pairwise.

    a: (..., N) interleaved pairs; h: (..., N, D).  Row pair j of h is
    multiplied by a[2j] + i a[2j+1] (intra_chunk_scan.cu:155-162).
    """
    ar = a[..., 0::2].unsqueeze(-1)
    ai = a[..., 1::2].unsqueeze(-1)
    hr = h[..., 0::2, :]
    hi = h[..., 1::2, :]
    out = torch.stack([ar * hr - ai * hi, ar * hi + ai * hr], dim=-2)
    return out.flatten(-3, -2)


def cmul_vec(a: Tensor, b: Tensor) -> Tensor:
    """Pairwise complex product of two interleaved vectors (intra_chunk_scan.cu:179-186)."""
    ar, ai = a[..., 0::2], a[..., 1::2]
    br, bi = b[..., 0::2], b[..., 1::2]
    return torch.stack([ar * br - ai * bi, ar * bi + ai * br], dim=-1).flatten(-2)


def identity_pairs(shape, like: Tensor) -> Tensor:
    """Interleaved complex ones of shape (..., N) (intra_chunk_scan.cu:93-98)."""
    out = torch.zeros(shape, dtype=like.dtype, device=like.device)
    out[..., 0::2] = 1.0
    return out


# --------------------------------------------------------------------------
# Cayley discretisation and gating (cayley_math.cuh:51-99, dynamics_fused.cu:109-131)
# --------------------------------------------------------------------------

def cayley_conj_mu(alpha: Tensor, omega: Tensor, dt: Tensor, eps: float = EPS_DEFAULT):
    """conj(mu), mu = (1 + tau*lam)/(1 - tau*lam), lam = -alpha + i*omega, tau = dt/2.

    Follows cayley_math.cuh:51-85: alpha clamped at 0, |D|^2 + eps denominator.
    Returns (re, im) of the stored value (im already negated).
    """
    alpha = torch.clamp(alpha, min=0.0)
    tau = dt * 0.5
    ta = tau * alpha
    tw = tau * omega
    denom = (1.0 + ta) * (1.0 + ta) + tw * tw + eps
    mu_re = (1.0 - ta * ta - tw * tw) / denom
    mu_im = (2.0 * tw) / denom
    return mu_re, -mu_im


def cayley_eig_sq(alpha: Tensor, omega: Tensor, dt: Tensor, eps: float = EPS_DEFAULT) -> Tensor:
    """|A_bar|^2 = ((1-ta)^2 + tw^2) / ((1+ta)^2 + tw^2 + eps) (cayley_math.cuh:89-99)."""
    alpha = torch.clamp(alpha, min=0.0)
    tau = dt * 0.5
    ta = tau * alpha
    tw = tau * omega
    numer = (1.0 - ta) * (1.0 - ta) + tw * tw
    denom = (1.0 + ta) * (1.0 + ta) + tw * tw
    return numer / (denom + eps)


def gated_transition(alpha: Tensor, omega: Tensor, dt: Tensor, r: Tensor, c: float):
    """One eigenvalue pair: stored A_bar (re, im) and the VP injection scale.

    dynamics_fused.cu:109-131:
      E = max(eig_sq, 1e-8); scale = E^((c r - 1)/2); A = conj(mu) * scale;
      vp = min(sqrt(max(1 - E^(c r), 1e-6)), 1).
    """
    re, im = cayley_conj_mu(alpha, omega, dt)
    E = torch.clamp(cayley_eig_sq(alpha, omega, dt), min=E_CLAMP)
    cr = c * r
    scale = torch.pow(E, (cr - 1.0) * 0.5)
    vp = torch.clamp(torch.sqrt(torch.clamp(1.0 - torch.pow(E, cr), min=EPS_DEFAULT)), max=1.0)
    return re * scale, im * scale, vp


def scan_dynamics(alpha: Tensor, omega: Tensor, dt: Tensor, r: Tensor, c: float):
    """Scan-level dynamics used by the scan configs: per-head alpha/omega, per-token dt, r.

    alpha, omega: (H,) or (H, N/2); dt, r: (B, L, H).
    Returns A_bar (B, L, H, N) interleaved and vp (B, L, H, N/2).
    The per-pair formula is gated_transition (dynamics_fused.cu:109-131); the
    gate parsing and adaptive dt of the gate-level op are bypassed (dt, r given).
    """
    if alpha.dim() == 1:
        alpha = alpha[:, None]
        omega = omega[:, None]
    al = alpha[None, None]              # (1,1,H,Nh)
    om = omega[None, None]
    dtb = dt[..., None]                 # (B,L,H,1)
    rb = r[..., None]
    re, im, vp = gated_transition(al, om, dtb, rb, c)
    A = torch.stack([re, im], dim=-1).flatten(-2)   # (B,L,H,N)
    return A, vp


# --------------------------------------------------------------------------
# Gate-level fused dynamics (dynamics_fused.cu:35-140, ops.py:39-66)
# --------------------------------------------------------------------------

def _split_gates(gate_raw: Tensor, n_heads: int, state_dim: int):
    B, L, GH = gate_raw.shape
    H, N = n_heads, state_dim
    Nh = N // 2
    G = N + 5
    assert GH == G * H, "gate_raw last dim must be (N+5)*H"
    g = gate_raw.reshape(B, L, G, H)
    return dict(
        alpha_raw=g[:, :, :Nh],            # (B,L,Nh,H)
        omega_raw=g[:, :, Nh:N],
        sel_B=g[:, :, N + 0], sel_C=g[:, :, N + 1], sel_dt=g[:, :, N + 2],
        beta=g[:, :, N + 3], r=g[:, :, N + 4],
    )


def adaptive_dt_parts(alpha0: Tensor, omega0: Tensor, log_dt_scale: Tensor, sel_dt_raw: Tensor,
                      omega_thresh: float, adt_delta: float, adt_smoothness: float, adt_eps: float) -> dict:
    """The adaptive timestep's pieces (dynamics_fused.cu:85-94): dt_raw, dt_max, blend, capped
    (dt_raw > dt_max, the branch :350-352 differentiates) and dt."""
    dt_scale = softplus(log_dt_scale)
    om_abs = omega0.abs()
    char_freq = alpha0 + om_abs + adt_eps
    dt_raw = dt_scale / char_freq
    dt_max = (2.0 - adt_delta) / (alpha0 + adt_eps)
    blend = sigmoid((omega_thresh - om_abs) / adt_smoothness)
    dt_capped = torch.minimum(dt_raw, dt_max)
    dt = blend * dt_capped + (1.0 - blend) * dt_raw + softplus(sel_dt_raw)
    return dict(dt_raw=dt_raw, dt_max=dt_max, blend=blend, capped=dt_raw > dt_max, dt=dt)


def adaptive_dt(alpha0: Tensor, omega0: Tensor, log_dt_scale: Tensor, sel_dt_raw: Tensor,
                omega_thresh: float, adt_delta: float, adt_smoothness: float, adt_eps: float) -> Tensor:
    """dt = blend*min(dt_raw, dt_max) + (1-blend)*dt_raw + softplus(sel_dt) (dynamics_fused.cu:85-94)."""
    return adaptive_dt_parts(alpha0, omega0, log_dt_scale, sel_dt_raw, omega_thresh, adt_delta,
                             adt_smoothness, adt_eps)["dt"]


def dynamics_regimes(gate_raw: Tensor, log_dt_scale: Tensor, rope_freqs: Tensor, gating_c: float,
                     omega_thresh: float, adt_delta: float, adt_smoothness: float, adt_eps: float,
                     n_heads: int, state_dim: int) -> dict:
    """Which branches of DynamicsFusedFn each (b, l, h) takes, from this module's own forward: boolean
    (B, L, H) masks ``capped`` (the adaptive-dt cap, dt_raw > dt_max), ``blend_mid`` (capped with the
    blend in (0.05, 0.95), where the blend's derivative :355-359 is material) and, per pair (B, L, H, N/2),
    ``vp_clamped`` (vp at its floor sqrt(1e-6), the clamp :113-118 / :247-259) and ``vp_one`` (vp within
    2^-25 of 1, i.e. 1 in fp32, where the reference's backward drops the vp cotangent, :247)."""
    B, L, _ = gate_raw.shape
    g = _split_gates(gate_raw, n_heads, state_dim)
    pos = torch.arange(L, dtype=gate_raw.dtype)[None, :, None]
    alpha0 = softplus(g["alpha_raw"][:, :, 0])
    omega0 = g["omega_raw"][:, :, 0] + pos * rope_freqs.to(gate_raw.dtype)[None, None, :]
    parts = adaptive_dt_parts(alpha0, omega0, log_dt_scale.to(gate_raw.dtype)[None, None, :], g["sel_dt"],
                              omega_thresh, adt_delta, adt_smoothness, adt_eps)
    _, vp, _, _ = dynamics_fused_fwd(gate_raw, log_dt_scale, rope_freqs, gating_c, omega_thresh, adt_delta,
                                     adt_smoothness, adt_eps, n_heads, state_dim)
    mid = (parts["blend"] > 0.05) & (parts["blend"] < 0.95)
    return dict(capped=parts["capped"], blend_mid=parts["capped"] & mid,
                vp_clamped=(vp - math.sqrt(EPS_DEFAULT)).abs() < 1e-12, vp_one=vp >= 1.0 - 2.0 ** -25)


def dynamics_fused_fwd(gate_raw: Tensor, log_dt_scale: Tensor, rope_freqs: Tensor,
                       gating_c: float, omega_thresh: float, adt_delta: float,
                       adt_smoothness: float, adt_eps: float, n_heads: int, state_dim: int):
    """Restates dynamics_fused.cu:50-139 (DynamicsFusedFn.forward, ops.py:39-66).

    Returns A_bar (B,L,H,N), vp_scale (B,L,H,N/2), beta (B,L,H), sel_C (B,L,H).
    """
    B, L, _ = gate_raw.shape
    H, N = n_heads, state_dim
    g = _split_gates(gate_raw, H, N)
    pos = torch.arange(L, dtype=gate_raw.dtype, device=gate_raw.device)[None, :, None]
    freq = rope_freqs.to(gate_raw.dtype)[None, None, :]
    r = sigmoid(g["r"])
    alpha0 = softplus(g["alpha_raw"][:, :, 0])
    omega0 = g["omega_raw"][:, :, 0] + pos * freq
    dt = adaptive_dt(alpha0, omega0, log_dt_scale.to(gate_raw.dtype)[None, None, :], g["sel_dt"],
                     omega_thresh, adt_delta, adt_smoothness, adt_eps)          # (B,L,H)
    alpha = softplus(g["alpha_raw"])                                              # (B,L,Nh,H)
    omega = g["omega_raw"] + pos[..., None] * freq[:, :, None, :]            # (B,L,Nh,H)
    re, im, vp = gated_transition(alpha, omega, dt[:, :, None, :], r[:, :, None, :], gating_c)
    A = torch.stack([re, im], dim=-1)              # (B,L,Nh,H,2)
    A = A.permute(0, 1, 3, 2, 4).reshape(B, L, H, N)
    vp = vp.permute(0, 1, 3, 2).contiguous()       # (B,L,H,Nh)
    beta = sigmoid(g["beta"]) * sigmoid(g["sel_B"])
    sel_C = sigmoid(g["sel_C"])
    return A, vp, beta, sel_C


def dynamics_fused_bwd_ref(grad_A: Tensor, grad_vp: Tensor, grad_beta: Tensor, grad_sel_C: Tensor,
                           gate_raw: Tensor, log_dt_scale: Tensor, rope_freqs: Tensor,
                           gating_c: float, omega_thresh: float, adt_delta: float,
                           adt_smoothness: float, adt_eps: float, n_heads: int, state_dim: int):
    """Hand restatement of the reference's analytic backward (dynamics_fused.cu:166-386).

    It agrees with autograd of dynamics_fused_fwd except where the reference's
    formula deliberately differs:
      * the VP clamp: the reference passes g_vp * (-0.5 / vp) whenever
        1e-6 < vp < 1 with vp = sqrt(max(1 - E^cr, 1e-6)) (:247-259), i.e. also
        inside the clamp where the forward is flat;
      * sign(0) = +1 for |omega0| (:361);
      * the Cayley derivative uses the eps-free |D|^2 in one term (:318-321).
    Returns grad_gate_raw (B, L, (N+5)H) and grad_log_dt_scale (H,).
    """
    dtype = gate_raw.dtype
    B, L, _ = gate_raw.shape
    H, N = n_heads, state_dim
    Nh = N // 2
    g = _split_gates(gate_raw, H, N)
    pos = torch.arange(L, dtype=dtype)[None, :, None]
    freq = rope_freqs.to(dtype)[None, None, :]
    log_scale = log_dt_scale.to(dtype)[None, None, :]
    c = gating_c

    r_gate = sigmoid(g["r"])
    alpha0_raw = g["alpha_raw"][:, :, 0]
    alpha0 = softplus(alpha0_raw)
    omega0 = g["omega_raw"][:, :, 0] + pos * freq
    dt_scale = softplus(log_scale)
    om_abs = omega0.abs()
    char_freq = alpha0 + om_abs + adt_eps
    dt_raw = dt_scale / char_freq
    dt_max = (2.0 - adt_delta) / (alpha0 + adt_eps)
    blend = sigmoid((omega_thresh - om_abs) / adt_smoothness)
    dt_capped = torch.minimum(dt_raw, dt_max)
    is_capped = dt_raw > dt_max
    dt = blend * dt_capped + (1.0 - blend) * dt_raw + softplus(g["sel_dt"])

    # scalar gates (:214-220)
    sb, ss, sc = sigmoid(g["beta"]), sigmoid(g["sel_B"]), sigmoid(g["sel_C"])
    g_sel_C_raw = grad_sel_C * sc * (1 - sc)
    g_beta_raw = grad_beta * ss * sb * (1 - sb)
    g_sel_B_raw = grad_beta * sb * ss * (1 - ss)

    # per-pair (:229-343)
    alpha_raw = g["alpha_raw"]                                   # (B,L,Nh,H)
    alpha = softplus(alpha_raw)
    omega = g["omega_raw"] + pos[..., None] * freq[:, :, None, :]
    dtj = dt[:, :, None, :]
    rj = r_gate[:, :, None, :]
    mre, mim = cayley_conj_mu(alpha, omega, dtj)                # stored cm.re, cm.im
    eig_sq = cayley_eig_sq(alpha, omega, dtj)
    E = torch.clamp(eig_sq, min=E_CLAMP)
    exponent = (c * rj - 1.0) / 2.0
    scale = torch.pow(E, exponent)
    cr = c * rj
    eff = torch.pow(E, cr)
    vp = torch.sqrt(torch.clamp(1.0 - eff, min=EPS_DEFAULT))

    gA = grad_A.reshape(B, L, H, Nh, 2).permute(0, 1, 3, 2, 4)  # (B,L,Nh,H,2)
    gA_re, gA_im = gA[..., 0], gA[..., 1]
    g_vp = grad_vp.permute(0, 1, 3, 2)                          # (B,L,Nh,H)

    active = (vp > EPS_DEFAULT) & (vp < 1.0)
    d_eff = torch.where(active, g_vp * (-0.5 / vp), torch.zeros_like(vp))
    unclamped = E > E_CLAMP
    d_eig = torch.where(unclamped, d_eff * cr * torch.pow(E, cr - 1.0), torch.zeros_like(E))
    d_r = d_eff * c * torch.log(E) * eff
    d_scale = gA_re * mre + gA_im * mim
    d_eig = d_eig + torch.where(unclamped, d_scale * exponent * torch.pow(E, exponent - 1.0),
                                torch.zeros_like(E))
    d_r = d_r + d_scale * (c / 2.0) * torch.log(E) * scale
    gA_re = gA_re * scale
    gA_im = gA_im * scale

    tau = dtj * 0.5
    alpha_c = torch.clamp(alpha, min=0.0)
    ta = tau * alpha_c
    tw = tau * omega
    opa, oma = 1.0 + ta, 1.0 - ta
    det = opa * opa + tw * tw
    inv_det = 1.0 / (det + EPS_DEFAULT)
    d_numer = d_eig * inv_det
    d_denom = -d_eig * eig_sq * inv_det
    d_ta = d_numer * (-2.0 * oma) + d_denom * 2.0 * opa
    d_tw = d_numer * 2.0 * tw + d_denom * 2.0 * tw
    g_mu_re = gA_re
    g_mu_im = -gA_im
    num_re = 1.0 - ta * ta - tw * tw
    da_re_dta = (-2.0 * ta * det - num_re * 2.0 * opa) * inv_det * inv_det
    da_re_dtw = (-2.0 * tw * det - num_re * 2.0 * tw) * inv_det * inv_det
    da_im_dta = -2.0 * tw * 2.0 * opa * inv_det * inv_det
    da_im_dtw = (2.0 * det - 2.0 * tw * 2.0 * tw) * inv_det * inv_det
    d_ta = d_ta + g_mu_re * da_re_dta + g_mu_im * da_im_dta
    d_tw = d_tw + g_mu_re * da_re_dtw + g_mu_im * da_im_dtw
    g_alpha = torch.where(alpha >= 0.0, d_ta * tau, torch.zeros_like(d_ta))
    g_omega = d_tw * tau
    g_dt = (d_ta * alpha_c * 0.5 + d_tw * omega * 0.5).sum(2)   # (B,L,H)
    g_rg = d_r.sum(2)
    g_alpha_raw = g_alpha * sigmoid(alpha_raw)
    g_omega_raw = g_omega.clone()

    # adaptive dt (:345-374)
    g_sel_dt_raw = g_dt * sigmoid(g["sel_dt"])
    capf = is_capped.to(dtype)
    g_dt_raw_adt = g_dt * (1.0 - capf * blend)
    g_dt_max_adt = g_dt * capf * blend
    g_blend = g_dt * (dt_capped - dt_raw)
    dblend = -blend * (1.0 - blend) / adt_smoothness
    g_dt_scale = g_dt_raw_adt / char_freq
    g_char = g_dt_raw_adt * (-dt_scale / (char_freq * char_freq))
    g_alpha_max = g_dt_max_adt * (-(2.0 - adt_delta) / ((alpha0 + adt_eps) ** 2))
    g_om_abs = g_char + g_blend * dblend
    sign = torch.where(omega0 >= 0.0, torch.ones_like(omega0), -torch.ones_like(omega0))
    g_alpha_raw[:, :, 0] = g_alpha_raw[:, :, 0] + (g_char + g_alpha_max) * sigmoid(alpha0_raw)
    g_omega_raw[:, :, 0] = g_omega_raw[:, :, 0] + g_om_abs * sign
    g_log_scale = (g_dt_scale * sigmoid(log_scale)).sum(dim=(0, 1))
    g_r_raw = g_rg * r_gate * (1.0 - r_gate)

    G = N + 5
    out = torch.zeros(B, L, G, H, dtype=dtype)
    out[:, :, :Nh] = g_alpha_raw
    out[:, :, Nh:N] = g_omega_raw
    out[:, :, N + 0] = g_sel_B_raw
    out[:, :, N + 1] = g_sel_C_raw
    out[:, :, N + 2] = g_sel_dt_raw
    out[:, :, N + 3] = g_beta_raw
    out[:, :, N + 4] = g_r_raw
    return out.reshape(B, L, G * H), g_log_scale


# --------------------------------------------------------------------------
# K/Q normalisation (normalize_kq.cu:75-79, :143-163)
# --------------------------------------------------------------------------

def normalize_kq(K: Tensor, Q: Tensor, eps: float = EPS_DEFAULT):
    """x * rsqrt(sum(x^2) + 1e-6) over the last dim, any D (intended formula of
    normalize_kq.cu:75-79; the reference kernel is only correct for D = 64)."""
    kn = K * torch.rsqrt((K * K).sum(-1, keepdim=True) + eps)
    qn = Q * torch.rsqrt((Q * Q).sum(-1, keepdim=True) + eps)
    return kn, qn


def normalize_kq_bwd(gK: Tensor, gQ: Tensor, K: Tensor, Q: Tensor, eps: float = EPS_DEFAULT):
    """g_in = (g - x_hat * <g, x_hat>) * rsqrt(sum x^2 + eps) (normalize_kq.cu:143-163)."""
    def one(g, x):
        inv = torch.rsqrt((x * x).sum(-1, keepdim=True) + eps)
        xh = x * inv
        return (g - xh * (g * xh).sum(-1, keepdim=True)) * inv
    return one(gK, K), one(gQ, Q)


# --------------------------------------------------------------------------
# The three scan passes (R-mode: the reference ops.py algorithm)
# --------------------------------------------------------------------------

def _erase(h: Tensor, k: Tensor, b: Tensor) -> Tensor:
    """h - beta * (h k) k^T per state row (intra_chunk_scan.cu:117-149)."""
    kTh = (h * k.unsqueeze(-2)).sum(-1, keepdim=True)
    return h - b[..., None, None] * kTh * k.unsqueeze(-2)


def intra_chunk_scan(A_flat: Tensor, K_flat: Tensor, V_flat: Tensor, beta_flat: Tensor,
                     state_dim: int):
    """Zero-init delta-rule scan inside each chunk (intra_chunk_scan.cu:86-195).

    Step t: erase -> complex rotate by A[t] -> inject beta v k^T; local_h[t] is
    stored AFTER the step; cum_A[t] = A[t] * cum_A[t-1].
    A (BNC,C,H,N), K (BNC,C,H,D), V (BNC,C,H,N), beta (BNC,C,H)
      -> local_h (BNC,C,H,N,D), cum_A (BNC,C,H,N).
    """
    BNC, C, H, D = K_flat.shape
    N = state_dim
    h = torch.zeros(BNC, H, N, D, dtype=K_flat.dtype)
    cA = identity_pairs((BNC, H, N), K_flat)
    lh, ca = [], []
    for t in range(C):
        a, k, v, b = A_flat[:, t], K_flat[:, t], V_flat[:, t], beta_flat[:, t]
        h = cmul_rows(a, _erase(h, k, b)) + b[..., None, None] * v.unsqueeze(-1) * k.unsqueeze(-2)
        cA = cmul_vec(a, cA)
        lh.append(h)
        ca.append(cA)
    return torch.stack(lh, 1), torch.stack(ca, 1)


def inter_chunk_scan(total_A: Tensor, final_local_h: Tensor, state_dim: int,
                     h0: Optional[Tensor] = None):
    """Serial carry over chunk summaries (inter_chunk_scan.cu:49-84).

    chunk_states[k] = s_k stored BEFORE the update; s_{k+1} = total_A[k] * s_k + flh[k]
    (rotation-only carry).  s_0 = 0 in the reference; h0 (B,H,N,D) is the
    initial-state extension.  Returns (chunk_states (B,NC,H,N,D), s_NC).
    """
    B, NC, H, N, D = final_local_h.shape
    s = torch.zeros(B, H, N, D, dtype=final_local_h.dtype) if h0 is None else h0
    states = []
    for k in range(NC):
        states.append(s)
        s = cmul_rows(total_A[:, k], s) + final_local_h[:, k]
    return torch.stack(states, 1), s


def exact_correction(A_chunk: Tensor, K_chunk: Tensor, beta_chunk: Tensor,
                     chunk_states: Tensor, state_dim: int) -> Tensor:
    """Push each chunk's entering state through erase+rotate, no injection.

    corrections[t] = state BEFORE step t (exact_correction.cu:83-150).
    A (B,NC,C,H,N), K (B,NC,C,H,D), beta (B,NC,C,H), chunk_states (B,NC,H,N,D)
      -> corrections (B,NC,C,H,N,D).
    """
    C = K_chunk.shape[2]
    h = chunk_states
    out = []
    for t in range(C):
        out.append(h)
        h = cmul_rows(A_chunk[:, :, t], _erase(h, K_chunk[:, :, t], beta_chunk[:, :, t]))
    return torch.stack(out, 2)


def ssd_chunkwise_scan(A_bar: Tensor, K: Tensor, V: Tensor, beta: Tensor, chunk_size: int,
                       state_dim: int, h0: Optional[Tensor] = None, return_final: bool = False,
                       correction_fn=None):
    """SSDChunkwiseScan.forward (ssd.py:39-111): pad, chunk, intra, summaries,
    inter, correction, Y = local_h + correction, unpad.

    Extension (not in the reference): h0 seeds chunk_states[0]; with
    return_final the R-mode carry after the last real token is also returned
    (equal to s_NC when L is a multiple of the chunk size).
    correction_fn replaces exact_correction (used to attach a custom backward).
    """
    B, L, H, D = K.shape
    N = state_dim
    Q = chunk_size
    NC = math.ceil(L / Q)
    pad = NC * Q - L
    if pad > 0:                                   # ssd.py:58-67 (zero padding, A=0)
        A_bar = F.pad(A_bar, (0, 0, 0, 0, 0, pad))
        K = F.pad(K, (0, 0, 0, 0, 0, pad))
        V = F.pad(V, (0, 0, 0, 0, 0, pad))
        beta = F.pad(beta, (0, 0, 0, pad))
    A_chunk = A_bar.reshape(B, NC, Q, H, N)
    K_chunk = K.reshape(B, NC, Q, H, D)
    V_chunk = V.reshape(B, NC, Q, H, N)
    b_chunk = beta.reshape(B, NC, Q, H)
    local_h, cum_A = intra_chunk_scan(A_chunk.reshape(B * NC, Q, H, N), K_chunk.reshape(B * NC, Q, H, D),
                                      V_chunk.reshape(B * NC, Q, H, N), b_chunk.reshape(B * NC, Q, H), N)
    local_h = local_h.reshape(B, NC, Q, H, N, D)
    cum_A = cum_A.reshape(B, NC, Q, H, N)
    total_A = cum_A[:, :, -1]                                  # ssd.py:90
    flh = local_h[:, :, -1]                                    # ssd.py:91
    chunk_states, s_final = inter_chunk_scan(total_A, flh, N, h0)
    corr_fn = exact_correction if correction_fn is None else correction_fn
    corr = corr_fn(A_chunk, K_chunk, b_chunk, chunk_states, N)
    Y = (local_h + corr).reshape(B, NC * Q, H, N, D)           # ssd.py:102-105
    if pad > 0:
        Y = Y[:, :L]
    if not return_final:
        return Y
    if pad > 0:
        last = Q - 1 - pad                                     # last real token of the last chunk
        s_final = cmul_rows(cum_A[:, -1, last], chunk_states[:, -1]) + local_h[:, -1, last]
    return Y, s_final


def exact_recurrence(A_bar: Tensor, K: Tensor, V: Tensor, beta: Tensor, state_dim: int,
                     h0: Optional[Tensor] = None):
    """E-mode: the exact sequential delta-rule recurrence over the whole sequence
    (not the reference's algorithm; used to pin where R-mode departs from it)."""
    B, L, H, D = K.shape
    h = torch.zeros(B, H, state_dim, D, dtype=K.dtype) if h0 is None else h0
    ys = []
    for t in range(L):
        h = cmul_rows(A_bar[:, t], _erase(h, K[:, t], beta[:, t])) \
            + beta[:, t][..., None, None] * V[:, t].unsqueeze(-1) * K[:, t].unsqueeze(-2)
        ys.append(h)
    return torch.stack(ys, 1), h


def readout(Y: Tensor, Qn: Tensor, sel_C: Tensor, K: Optional[Tensor] = None,
            V_gated: Optional[Tensor] = None, shortcut_scale: float = 0.0) -> Tensor:
    """Shortcut + readout + sel_C gate (block.py:202-211): y = sel_C * (Y q).  shortcut_scale may be a
    tensor (the block's parameter, so that it receives a gradient)."""
    if isinstance(shortcut_scale, torch.Tensor) or shortcut_scale != 0.0:
        qk = (Qn * K).sum(-1)
        Y = Y + shortcut_scale * qk[..., None, None] * V_gated.unsqueeze(-1) * K.unsqueeze(-2)
    return torch.einsum('blhsd,blhd->blhs', Y, Qn) * sel_C.unsqueeze(-1)


# --------------------------------------------------------------------------
# Hand restatements of the reference's scan backward kernels
# --------------------------------------------------------------------------

def intra_chunk_scan_bwd_ref(grad_local_h, grad_cum_A, A_flat, K_flat, V_flat, beta_flat, state_dim):
    """Reverse scan of intra_chunk_scan.cu:261-552 with fp64 recomputed states.

    Returns grad_A, grad_K, grad_V, grad_beta.  The reference kernel is the exact
    gradient of its forward; tests check this restatement against autograd.
    """
    BNC, C, H, D = K_flat.shape
    local_h, cum_A = intra_chunk_scan(A_flat, K_flat, V_flat, beta_flat, state_dim)
    dh = torch.zeros_like(local_h[:, 0])
    dcA = torch.zeros_like(cum_A[:, 0])
    gA, gK, gV, gB = (torch.zeros_like(A_flat), torch.zeros_like(K_flat),
                      torch.zeros_like(V_flat), torch.zeros_like(beta_flat))
    for t in range(C - 1, -1, -1):
        dh = dh + grad_local_h[:, t]
        a, k, v, b = A_flat[:, t], K_flat[:, t], V_flat[:, t], beta_flat[:, t]
        hp = local_h[:, t - 1] if t > 0 else torch.zeros_like(dh)
        kTh = (hp * k.unsqueeze(-2)).sum(-1)                          # (BNC,H,N)
        hm = hp - b[..., None, None] * kTh.unsqueeze(-1) * k.unsqueeze(-2)
        gV[:, t] = b[..., None] * (dh * k.unsqueeze(-2)).sum(-1)
        gk_inj = b[..., None] * (v.unsqueeze(-1) * dh).sum(-2)
        gb_inj = (v.unsqueeze(-1) * k.unsqueeze(-2) * dh).sum((-1, -2))
        a_conj = a.clone()
        a_conj[..., 1::2] = -a_conj[..., 1::2]
        dhm = cmul_rows(a_conj, dh)
        hm_conj = hm.clone()
        hm_conj[..., 1::2, :] = -hm_conj[..., 1::2, :]
        gA_state = _pair_sum_mul(dh, hm_conj)
        dcA = dcA + grad_cum_A[:, t]
        prev = cum_A[:, t - 1] if t > 0 else identity_pairs(dcA.shape, dcA)
        prev_conj = prev.clone()
        prev_conj[..., 1::2] = -prev_conj[..., 1::2]
        gA[:, t] = gA_state + cmul_vec(dcA, prev_conj)
        dcA = cmul_vec(a_conj, dcA)
        zeta = (dhm * k.unsqueeze(-2)).sum(-1)                         # (BNC,H,N)
        gk_er = -b[..., None] * (kTh.unsqueeze(-1) * dhm + hp * zeta.unsqueeze(-1)).sum(-2)
        gb_er = -(kTh * zeta).sum(-1)
        gK[:, t] = gk_inj + gk_er
        gB[:, t] = gb_inj + gb_er
        dh = dhm - b[..., None, None] * zeta.unsqueeze(-1) * k.unsqueeze(-2)
    return gA, gK, gV, gB


def _pair_sum_mul(g: Tensor, x: Tensor) -> Tensor:
    """sum_d g_pair * x_pair (complex product per row pair, summed over D)."""
    gr, gi = g[..., 0::2, :], g[..., 1::2, :]
    xr, xi = x[..., 0::2, :], x[..., 1::2, :]
    re = (gr * xr - gi * xi).sum(-1)
    im = (gr * xi + gi * xr).sum(-1)
    return torch.stack([re, im], -1).flatten(-2)


def inter_chunk_scan_bwd_ref(grad_chunk_states, total_A, chunk_states, state_dim,
                             grad_final: Optional[Tensor] = None):
    """Reverse scan of inter_chunk_scan.cu:117-195.  grad_final is the extension's
    gradient w.r.t. s_NC (zero in the reference).  Returns grad_total_A,
    grad_final_local_h and (extension) the gradient w.r.t. s_0."""
    B, NC, H, N, D = chunk_states.shape
    ds = torch.zeros_like(chunk_states[:, 0]) if grad_final is None else grad_final.clone()
    g_tA = torch.zeros_like(total_A)
    g_flh = torch.zeros_like(chunk_states)
    for k in range(NC - 1, -1, -1):
        a = total_A[:, k]
        sk = chunk_states[:, k]
        g_flh[:, k] = ds
        s_conj = sk.clone()
        s_conj[..., 1::2, :] = -s_conj[..., 1::2, :]
        g_tA[:, k] = _pair_sum_mul(ds, s_conj)
        a_conj = a.clone()
        a_conj[..., 1::2] = -a_conj[..., 1::2]
        ds = cmul_rows(a_conj, ds) + grad_chunk_states[:, k]
    return g_tA, g_flh, ds


def exact_correction_bwd_ref(grad_corr, A_chunk, K_chunk, beta_chunk, chunk_states, state_dim):
    """Reverse scan of exact_correction.cu:213-382, restated with its ordering.

    The reference adds grad_corrections[t] to the running state gradient BEFORE
    back-propagating through step t (:219-223), although its forward stores
    corrections[t] before step t (:90-94).  The result is the gradient of
    sum_t <grad_corr[t], c_{t+1}> (state AFTER step t), not of the forward's
    sum_t <grad_corr[t], c_t>.  This restatement keeps that ordering; tests
    pin it against autograd of the shifted functional.
    Returns grad_A, grad_K, grad_beta, grad_states.
    """
    corr = exact_correction(A_chunk, K_chunk, beta_chunk, chunk_states, state_dim)
    C = K_chunk.shape[2]
    dh = torch.zeros_like(chunk_states)
    gA, gK, gB = torch.zeros_like(A_chunk), torch.zeros_like(K_chunk), torch.zeros_like(beta_chunk)
    for t in range(C - 1, -1, -1):
        dh = dh + grad_corr[:, :, t]
        a, k, b = A_chunk[:, :, t], K_chunk[:, :, t], beta_chunk[:, :, t]
        hb = corr[:, :, t]
        kTh = (hb * k.unsqueeze(-2)).sum(-1)
        hm = hb - b[..., None, None] * kTh.unsqueeze(-1) * k.unsqueeze(-2)
        a_conj = a.clone()
        a_conj[..., 1::2] = -a_conj[..., 1::2]
        dhm = cmul_rows(a_conj, dh)
        hm_conj = hm.clone()
        hm_conj[..., 1::2, :] = -hm_conj[..., 1::2, :]
        gA[:, :, t] = _pair_sum_mul(dh, hm_conj)
        zeta = (dhm * k.unsqueeze(-2)).sum(-1)
        gK[:, :, t] = -b[..., None] * (kTh.unsqueeze(-1) * dhm + hb * zeta.unsqueeze(-1)).sum(-2)
        gB[:, :, t] = -(kTh * zeta).sum(-1)
        dh = dhm - b[..., None, None] * zeta.unsqueeze(-1) * k.unsqueeze(-2)
    return gA, gK, gB, dh


class _CorrectionRefGrad(torch.autograd.Function):
    """exact_correction whose backward is the reference's (exact_correction_bwd_ref)."""

    @staticmethod
    def forward(ctx, A_chunk, K_chunk, beta_chunk, chunk_states, state_dim):
        ctx.save_for_backward(A_chunk, K_chunk, beta_chunk, chunk_states)
        ctx.state_dim = state_dim
        return exact_correction(A_chunk, K_chunk, beta_chunk, chunk_states, state_dim)

    @staticmethod
    def backward(ctx, g):
        A_chunk, K_chunk, beta_chunk, chunk_states = ctx.saved_tensors
        with torch.no_grad():
            gA, gK, gB, gS = exact_correction_bwd_ref(g, A_chunk, K_chunk, beta_chunk,
                                                      chunk_states, ctx.state_dim)
        return gA, gK, gB, gS, None


def correction_with_reference_grad(A_chunk, K_chunk, beta_chunk, chunk_states, state_dim):
    return _CorrectionRefGrad.apply(A_chunk, K_chunk, beta_chunk, chunk_states, state_dim)


class _DynamicsRefGrad(torch.autograd.Function):
    """dynamics_fused_fwd whose backward is the reference's analytic rule (dynamics_fused_bwd_ref);
    gradients for gate_raw and log_dt_scale, None for the rest (ops.py:68-81)."""

    @staticmethod
    def forward(ctx, gate_raw, log_dt_scale, rope_freqs, gating_c, omega_thresh, adt_delta, adt_smoothness,
                adt_eps, n_heads, state_dim):
        ctx.save_for_backward(gate_raw, log_dt_scale, rope_freqs)
        ctx.args = (gating_c, omega_thresh, adt_delta, adt_smoothness, adt_eps, n_heads, state_dim)
        return dynamics_fused_fwd(gate_raw, log_dt_scale, rope_freqs, *ctx.args)

    @staticmethod
    def backward(ctx, gA, gvp, gbeta, gsel):
        gate_raw, log_dt_scale, rope_freqs = ctx.saved_tensors
        with torch.no_grad():
            g_raw, g_lds = dynamics_fused_bwd_ref(gA, gvp, gbeta, gsel, gate_raw, log_dt_scale, rope_freqs,
                                                  *ctx.args)
        return g_raw, g_lds.to(log_dt_scale.dtype), None, None, None, None, None, None, None, None


def dynamics_with_reference_grad(gate_raw, log_dt_scale, rope_freqs, gating_c, omega_thresh, adt_delta,
                                 adt_smoothness, adt_eps, n_heads, state_dim):
    return _DynamicsRefGrad.apply(gate_raw, log_dt_scale, rope_freqs, gating_c, omega_thresh, adt_delta,
                                  adt_smoothness, adt_eps, n_heads, state_dim)


# --------------------------------------------------------------------------
# The fused scan (the metric op): dynamics + VP + R-mode scan + readout
# --------------------------------------------------------------------------

def fused_scan(q: Tensor, k: Tensor, v: Tensor, beta: Tensor, sel_C: Tensor, dt: Tensor,
               r: Tensor, alpha: Tensor, omega: Tensor, c: float, h0: Optional[Tensor] = None,
               chunk_size: Optional[int] = None, mode: str = "R", grad_mode: str = "reference",
               normalize: bool = False):
    """y = sel_C * (Y q) with Y from the reference ops.py scan (block.py:181-211 minus
    the gate parsing): A_bar, vp from scan_dynamics; V_gated = v * vp
    (block.py:194-195); Y = SSDChunkwiseScan(A_bar, k, V_gated, beta) (ssd.py:39-111).

    q, k: (B,L,H,D); v: (B,L,H,N); beta, sel_C, dt, r: (B,L,H); alpha, omega: (H,)
    or (H,N/2); c scalar; h0 (B,H,N,D) or None.
    mode "R" = reference algorithm, "E" = exact recurrence.
    grad_mode "reference" attaches the reference's correction backward,
    "exact" uses autograd of the forward.
    Returns y (B,L,H,N) and the final state (B,H,N,D).
    """
    B, L, H, D = k.shape
    N = v.shape[-1]
    if normalize:
        k, q = normalize_kq(k, q)
    A, vp = scan_dynamics(alpha, omega, dt, r, c)
    Vg = v * vp.repeat_interleave(2, dim=-1)
    if mode == "R":
        corr_fn = correction_with_reference_grad if grad_mode == "reference" else None
        Y, s_final = ssd_chunkwise_scan(A, k, Vg, beta, chunk_size or D, N, h0=h0,
                                        return_final=True, correction_fn=corr_fn)
    elif mode == "E":
        Y, s_final = exact_recurrence(A, k, Vg, beta, N, h0)
    else:
        raise ValueError(f"mode must be 'R' or 'E', got {mode!r}")
    return readout(Y, q, sel_C), s_final
