"""Pins the CPU oracle (oracle/cdssm_oracle.py) before anything is compared to it.

The reference ships no tests, fixtures or golden vectors (its tree has no
tests/ and no assert outside one config check), so every check here comes from
mathematics the reference's own comments and code fix: textbook 2x2 Cayley
matrices, brute-force loops over explicit real matrices, closed-form
recurrences, known-answer cases, and autograd.  Each check is chosen so that a
plausible slip (a conjugate dropped, a sign flipped, the store-before /
store-after step swapped, a transposed operand) fails it.
"""

import math

import numpy as np
import pytest
import torch

from oracle import cdssm_oracle as o

DT = torch.float64


@pytest.fixture(autouse=True)
def _fp64_default():
    """fp64 as torch's default dtype for this module's tests only, restored after each (a module-level
    setting would leak into every other test module of the session)."""
    prev = torch.get_default_dtype()
    torch.set_default_dtype(torch.float64)
    yield
    torch.set_default_dtype(prev)


def rng(seed=0):
    g = torch.Generator().manual_seed(seed)
    return g


def randn(g, *shape):
    return torch.randn(*shape, generator=g, dtype=DT)


def unit(x):
    return x / x.norm(dim=-1, keepdim=True)


# --------------------------------------------------------------------------
# Cayley discretisation: textbook (I - tau A)^-1 (I + tau A)
# --------------------------------------------------------------------------

def test_cayley_matches_textbook_2x2_and_rotation_direction():
    g = rng(1)
    for _ in range(50):
        alpha = float(torch.rand(1, generator=g) * 3)
        omega = float(randn(g, 1) * 4)
        dt = float(torch.rand(1, generator=g) * 2 + 1e-3)
        tau = dt / 2
        A2 = np.array([[-alpha, omega], [-omega, -alpha]])
        Abar = np.linalg.solve(np.eye(2) - tau * A2, np.eye(2) + tau * A2)
        re, im = o.cayley_conj_mu(torch.tensor(alpha), torch.tensor(omega), torch.tensor(dt), eps=0.0)
        # the stored value acts on (h_re, h_im) as the complex product (re + i im) h
        M = np.array([[float(re), -float(im)], [float(im), float(re)]])
        np.testing.assert_allclose(M, Abar, atol=1e-12)
        # ... and cmul_rows applies exactly that matrix to a state row pair
        h = randn(g, 2, 3)
        a = torch.tensor([float(re), float(im)])
        np.testing.assert_allclose(o.cmul_rows(a, h).numpy(), Abar @ h.numpy(), atol=1e-12)
        # |A_bar|^2 = det(A_bar) = eig_sq
        E = o.cayley_eig_sq(torch.tensor(alpha), torch.tensor(omega), torch.tensor(dt), eps=0.0)
        assert abs(float(E) - np.linalg.det(Abar)) < 1e-12
        assert float(E) <= 1.0 + 1e-15          # A-stability for alpha >= 0


def test_cayley_clamps_negative_alpha_and_eps_is_small():
    a = torch.tensor([-0.5, 0.0])
    re1, im1 = o.cayley_conj_mu(a, torch.tensor([0.3, 0.3]), torch.tensor([0.7, 0.7]))
    assert torch.allclose(re1[0], re1[1]) and torch.allclose(im1[0], im1[1])
    re2, _ = o.cayley_conj_mu(torch.tensor(0.2), torch.tensor(0.1), torch.tensor(0.5), eps=0.0)
    re3, _ = o.cayley_conj_mu(torch.tensor(0.2), torch.tensor(0.1), torch.tensor(0.5))
    assert 0 < float(re2 - re3) < 2e-6


def test_gating_magnitude_and_vp_identity():
    g = rng(2)
    alpha = torch.rand(500, generator=g) * 3
    omega = randn(g, 500) * 3
    dt = torch.rand(500, generator=g) * 2 + 0.01
    r = torch.rand(500, generator=g)
    c = math.log(4096)
    re, im, vp = o.gated_transition(alpha, omega, dt, r, c)
    E = torch.clamp(o.cayley_eig_sq(alpha, omega, dt), min=1e-8)
    mag2 = re * re + im * im
    # |A_eff|^2 = |mu|^2 E^(cr-1) with |mu|^2 = E * |D|^2/(|D|^2+eps): ~ E^(cr)
    assert torch.allclose(mag2, E ** (c * r), rtol=1e-5, atol=0)
    inside = (1 - E ** (c * r)) > 1e-6
    assert inside.sum() > 400
    assert torch.allclose((vp * vp + E ** (c * r))[inside], torch.ones(int(inside.sum())), atol=1e-12)
    # clamp region: vp = sqrt(1e-6)
    _, _, vpc = o.gated_transition(torch.tensor(1e-9), torch.tensor(0.0), torch.tensor(1e-3),
                                   torch.tensor(1e-3), c)
    assert abs(float(vpc) - 1e-3) < 1e-12


# --------------------------------------------------------------------------
# Adaptive dt and gate-level dynamics
# --------------------------------------------------------------------------

def test_adaptive_dt_cap_form():
    g = rng(3)
    a0 = torch.rand(400, generator=g) * 2
    w0 = randn(g, 400) * 0.2
    lds = randn(g, 400) * 2
    sdt = randn(g, 400)
    thr, delta, sm, eps = math.sqrt(2 ** -7), 16 * 2 ** -7, math.sqrt(2 ** -7) / 5, 1.0
    dt = o.adaptive_dt(a0, w0, lds, sdt, thr, delta, sm, eps)
    # independent form: dt_raw - blend * relu(dt_raw - dt_max) + softplus(sel_dt)
    dt_raw = torch.log1p(torch.exp(lds)) / (a0 + w0.abs() + eps)
    dt_max = (2 - delta) / (a0 + eps)
    blend = 1 / (1 + torch.exp(-(thr - w0.abs()) / sm))
    alt = dt_raw - blend * torch.relu(dt_raw - dt_max) + torch.log1p(torch.exp(sdt))
    assert torch.allclose(dt, alt, atol=1e-12)
    assert bool((dt > 0).all())


def _gate_inputs(g, B, L, H, N):
    gate = randn(g, B, L, (N + 5) * H) * 0.8
    lds = randn(g, H) * 0.5
    freqs = 1.0 / (float(L) ** (torch.arange(H, dtype=DT) / H))
    return gate, lds, freqs


CONSTS = dict(gating_c=math.log(64), omega_thresh=math.sqrt(2 ** -7), adt_delta=16 * 2 ** -7,
              adt_smoothness=math.sqrt(2 ** -7) / 5, adt_eps=1.0)


def test_dynamics_layout_matches_scan_level_formula():
    g = rng(4)
    B, L, H, N = 2, 9, 3, 4
    gate, lds, freqs = _gate_inputs(g, B, L, H, N)
    A, vp, beta, selc = o.dynamics_fused_fwd(gate, lds, freqs, n_heads=H, state_dim=N, **CONSTS)
    gg = gate.reshape(B, L, N + 5, H)
    for b in range(B):
        for l in range(L):
            for h in range(H):
                a0 = math.log1p(math.exp(gg[b, l, 0, h]))
                w0 = float(gg[b, l, N // 2, h]) + l * float(freqs[h])
                dt = float(o.adaptive_dt(torch.tensor(a0), torch.tensor(w0), lds[h], gg[b, l, N + 2, h],
                                         CONSTS["omega_thresh"], CONSTS["adt_delta"],
                                         CONSTS["adt_smoothness"], CONSTS["adt_eps"]))
                r = 1 / (1 + math.exp(-float(gg[b, l, N + 4, h])))
                for j in range(N // 2):
                    aj = math.log1p(math.exp(gg[b, l, j, h]))
                    wj = float(gg[b, l, N // 2 + j, h]) + l * float(freqs[h])
                    re, im, v = o.gated_transition(torch.tensor(aj), torch.tensor(wj), torch.tensor(dt),
                                                   torch.tensor(r), CONSTS["gating_c"])
                    assert abs(float(A[b, l, h, 2 * j]) - float(re)) < 1e-12
                    assert abs(float(A[b, l, h, 2 * j + 1]) - float(im)) < 1e-12
                    assert abs(float(vp[b, l, h, j]) - float(v)) < 1e-12
                sb = 1 / (1 + math.exp(-float(gg[b, l, N + 3, h]))) / (1 + math.exp(-float(gg[b, l, N, h])))
                assert abs(float(beta[b, l, h]) - sb) < 1e-12
                assert abs(float(selc[b, l, h]) - 1 / (1 + math.exp(-float(gg[b, l, N + 1, h])))) < 1e-12


def test_dynamics_bwd_restatement_matches_autograd_off_clamps():
    g = rng(5)
    B, L, H, N = 2, 16, 3, 4
    gate, lds, freqs = _gate_inputs(g, B, L, H, N)
    gate.requires_grad_(True)
    lds.requires_grad_(True)
    outs = o.dynamics_fused_fwd(gate, lds, freqs, n_heads=H, state_dim=N, **CONSTS)
    grads = [randn(g, *t.shape) for t in outs]
    loss = sum((t * w).sum() for t, w in zip(outs, grads))
    ga, gl = torch.autograd.grad(loss, [gate, lds])
    gh, glh = o.dynamics_fused_bwd_ref(*grads, gate.detach(), lds.detach(), freqs,
                                       n_heads=H, state_dim=N, **CONSTS)
    # inputs are far from the VP clamp and from omega0 = 0
    _, vp, _, _ = outs
    assert float(vp.detach().min()) > 2e-3
    # the reference differentiates mu with the eps-free |D|^2 in one term
    # (dynamics_fused.cu:318-321): O(1e-6) departures from exact autograd
    assert float((gh - ga).abs().max()) < 5e-6
    assert float((glh - gl).abs().max()) < 5e-6
    assert float(ga.abs().max()) > 0.1


def _capped_gate_inputs(g, B, L, H, N):
    """Gate rows in the adaptive-dt cap with a material blend: alpha_0 ~ softplus(-3) ~ 0.05,
    |omega_0| within 0.035 of omega_thresh (0.088; either sign), log_dt_scale ~ 3, so
    dt_raw = softplus(3)/(alpha_0 + |omega_0| + 1) ~ 2.7 > dt_max = 1.875/(alpha_0 + 1) ~ 1.8 and
    blend = sigmoid((thr - |omega_0|)/smooth) spans (0.1, 0.9).  Other gates: N(0, 0.5)."""
    freqs = 1.0 / (float(L) ** (torch.arange(H, dtype=DT) / H))
    gate = randn(g, B, L, N + 5, H) * 0.5
    pos = torch.arange(L, dtype=DT)[None, :, None]
    gate[:, :, 0] = -3.0 + 0.3 * randn(g, B, L, H)
    sign = torch.where(torch.rand(B, L, H, generator=g, dtype=DT) < 0.5, -1.0, 1.0)
    target = CONSTS["omega_thresh"] + (torch.rand(B, L, H, generator=g, dtype=DT) * 2 - 1) * 0.035
    gate[:, :, N // 2] = sign * target - pos * freqs
    lds = 3.0 + 0.2 * randn(g, H)
    return gate.reshape(B, L, (N + 5) * H), lds, freqs


@pytest.mark.parametrize("N", [2, 4])
def test_dynamics_bwd_restatement_matches_autograd_with_the_cap_active(N):
    """The cap branch of the restated backward (dynamics_fused.cu:345-374: the capped/uncapped split of
    g_dt, d blend / d|omega_0|, the dt_max term of alpha_0) against autograd of the forward, on rows where
    every token-head is capped with the blend in (0.05, 0.95) and no VP clamp is near.  The reference's
    cap terms are the exact derivative, so the only departure is the eps-free |D|^2 term (O(1e-6)).  A
    swapped sign of the blend's derivative changes the omega_0 gradients by O(1) here."""
    g = rng(21)
    B, L, H = 2, 24, 3
    gate, lds, freqs = _capped_gate_inputs(g, B, L, H, N)
    reg = o.dynamics_regimes(gate, lds, freqs, n_heads=H, state_dim=N, **CONSTS)
    assert bool(reg["blend_mid"].all()), "every token-head must be capped with a material blend"
    assert not bool(reg["vp_clamped"].any()) and not bool(reg["vp_one"].any())
    gate.requires_grad_(True)
    lds.requires_grad_(True)
    outs = o.dynamics_fused_fwd(gate, lds, freqs, n_heads=H, state_dim=N, **CONSTS)
    grads = [randn(g, *t.shape) for t in outs]
    loss = sum((t * w).sum() for t, w in zip(outs, grads))
    ga, gl = torch.autograd.grad(loss, [gate, lds])
    gh, glh = o.dynamics_fused_bwd_ref(*grads, gate.detach(), lds.detach(), freqs,
                                       n_heads=H, state_dim=N, **CONSTS)
    assert float((gh - ga).abs().max()) <= 1e-5 * float(ga.abs().max())
    assert float((glh - gl).abs().max()) <= 1e-5 * float(gl.abs().max())
    # the omega_0 column carries the blend's derivative: it is large here
    w0 = ga.reshape(B, L, N + 5, H)[:, :, N // 2]
    assert float(w0.abs().max()) > 1.0


def test_dynamics_bwd_restatement_keeps_vp_clamp_gradient():
    """Inside the VP clamp the reference still passes -0.5/vp * g_vp (dynamics_fused.cu:256-259)."""
    H, N, L = 1, 2, 1
    gate = torch.zeros(1, L, (N + 5) * H)
    gate[0, 0, 0] = -30.0            # alpha -> ~0
    gate[0, 0, 1] = 0.0              # omega = 0 (position 0)
    gate[0, 0, N + 2] = -30.0        # sel_dt -> 0
    gate[0, 0, N + 4] = -10.0        # r -> small
    lds = torch.tensor([-30.0])      # dt_scale -> 0
    A, vp, _, _ = o.dynamics_fused_fwd(gate, lds, torch.zeros(1), n_heads=H, state_dim=N, **CONSTS)
    assert abs(float(vp) - 1e-3) < 1e-12
    gz = torch.zeros(1, L, H, N)
    gvp = torch.ones(1, L, H, 1)
    gh, _ = o.dynamics_fused_bwd_ref(gz, gvp, torch.zeros(1, L, H), torch.zeros(1, L, H), gate, lds,
                                     torch.zeros(1), n_heads=H, state_dim=N, **CONSTS)
    # the r-gate gradient is -0.5/vp * c * log(E) * E^cr * r(1-r): nonzero although vp is flat
    assert abs(float(gh[0, 0, N + 4])) > 0


# --------------------------------------------------------------------------
# Normalisation
# --------------------------------------------------------------------------

def test_normalize_matches_library_up_to_eps_and_bwd_matches_autograd():
    g = rng(6)
    K = randn(g, 2, 5, 3, 128)
    Qm = randn(g, 2, 5, 3, 128)
    kn, qn = o.normalize_kq(K, Qm)
    nrm = K.norm(dim=-1, keepdim=True)
    ref = torch.nn.functional.normalize(K, dim=-1) * nrm / torch.sqrt(nrm * nrm + 1e-6)
    assert torch.allclose(kn, ref, atol=1e-14)
    assert torch.allclose((kn * kn).sum(-1), (K * K).sum(-1) / ((K * K).sum(-1) + 1e-6), atol=1e-14)
    K.requires_grad_(True)
    Qm.requires_grad_(True)
    kn, qn = o.normalize_kq(K, Qm)
    gk, gq = randn(g, *K.shape), randn(g, *K.shape)
    ak, aq = torch.autograd.grad((kn * gk).sum() + (qn * gq).sum(), [K, Qm])
    hk, hq = o.normalize_kq_bwd(gk, gq, K.detach(), Qm.detach())
    assert torch.allclose(hk, ak, atol=1e-12) and torch.allclose(hq, aq, atol=1e-12)


# --------------------------------------------------------------------------
# Scan passes vs brute force over explicit real matrices
# --------------------------------------------------------------------------

def _blockdiag_rot(a):
    """Real N x N matrix acting on the rows of the state for interleaved pairs a (N,)."""
    N = a.shape[0]
    R = np.zeros((N, N))
    for j in range(N // 2):
        re, im = a[2 * j], a[2 * j + 1]
        R[2 * j:2 * j + 2, 2 * j:2 * j + 2] = [[re, -im], [im, re]]
    return R


def _brute_intra(A, K, V, beta):
    A, K, V, beta = (x.numpy() for x in (A, K, V, beta))
    BNC, C, H, D = K.shape
    N = A.shape[-1]
    lh = np.zeros((BNC, C, H, N, D))
    ca = np.zeros((BNC, C, H, N))
    for n in range(BNC):
        for h in range(H):
            S = np.zeros((N, D))
            P = np.eye(N)
            for t in range(C):
                k = K[n, t, h]
                R = _blockdiag_rot(A[n, t, h])
                S = R @ (S @ (np.eye(D) - beta[n, t, h] * np.outer(k, k))) \
                    + beta[n, t, h] * np.outer(V[n, t, h], k)
                P = R @ P
                lh[n, t, h] = S
                ca[n, t, h, 0::2] = P[0::2, 0::2].diagonal()
                ca[n, t, h, 1::2] = P[1::2, 0::2].diagonal()
    return lh, ca


def _rand_scan_inputs(g, BNC, C, H, D, N, amax=1.0):
    ang = torch.rand(BNC, C, H, N // 2, generator=g) * 2 * math.pi
    mag = torch.rand(BNC, C, H, N // 2, generator=g) * amax
    A = torch.stack([mag * torch.cos(ang), mag * torch.sin(ang)], -1).flatten(-2)
    K = unit(randn(g, BNC, C, H, D))
    V = randn(g, BNC, C, H, N)
    beta = torch.rand(BNC, C, H, generator=g)
    return A, K, V, beta


def test_intra_matches_brute_force_matrices():
    g = rng(7)
    A, K, V, beta = _rand_scan_inputs(g, 3, 7, 2, 5, 4)
    lh, ca = o.intra_chunk_scan(A, K, V, beta, 4)
    blh, bca = _brute_intra(A, K, V, beta)
    np.testing.assert_allclose(lh.numpy(), blh, atol=1e-12)
    np.testing.assert_allclose(ca.numpy(), bca, atol=1e-12)


def test_intra_known_answers():
    g = rng(8)
    A, K, V, beta = _rand_scan_inputs(g, 2, 6, 2, 6, 2)
    lh, _ = o.intra_chunk_scan(A, K, V, torch.zeros_like(beta), 2)
    assert float(lh.abs().max()) == 0.0                       # beta = 0 => no memory
    # a = 1, beta = 1, k = e_j: column j overwritten by v, other columns unchanged
    C, D = 6, 6
    A1 = torch.zeros(1, C, 1, 2)
    A1[..., 0] = 1.0
    K1 = torch.zeros(1, C, 1, D)
    idx = [0, 3, 0, 5, 2, 3]
    for t, j in enumerate(idx):
        K1[0, t, 0, j] = 1.0
    V1 = randn(g, 1, C, 1, 2)
    lh, _ = o.intra_chunk_scan(A1, K1, V1, torch.ones(1, C, 1), 2)
    last = {}
    for t, j in enumerate(idx):
        last[j] = V1[0, t, 0]
        for col in range(D):
            want = last.get(col, torch.zeros(2))
            assert torch.allclose(lh[0, t, 0, :, col], want, atol=1e-14)
    # orthonormal keys, a = 1, beta = 1: exact retrieval z_t k_s = v_s for s <= t
    Qmat, _ = torch.linalg.qr(randn(g, D, D))
    K2 = Qmat.T[None, :, None, :]
    V2 = randn(g, 1, D, 1, 2)
    A2 = torch.zeros(1, D, 1, 2)
    A2[..., 0] = 1.0
    lh2, _ = o.intra_chunk_scan(A2, K2, V2, torch.ones(1, D, 1), 2)
    ret = torch.einsum('snd,sd->sn', lh2[0, D - 1, 0].expand(D, 2, D), K2[0, :, 0])
    assert torch.allclose(ret, V2[0, :, 0], atol=1e-12)


def test_cum_A_is_complex_cumprod_and_inter_is_closed_form():
    g = rng(9)
    A, K, V, beta = _rand_scan_inputs(g, 2, 9, 3, 4, 4)
    _, ca = o.intra_chunk_scan(A, K, V, beta, 4)
    Ac = A[..., 0::2] + 1j * A[..., 1::2]
    np.testing.assert_allclose((ca[..., 0::2] + 1j * ca[..., 1::2]).numpy(),
                               np.cumprod(Ac.numpy(), axis=1), atol=1e-12)
    # inter: s_k = sum_{j<k} prod_{i=j+1}^{k-1} A_i F_j  + prod_{i<k} A_i h0
    B, NC, H, N, D = 2, 6, 3, 4, 5
    tA = _rand_scan_inputs(g, B, NC, H, D, N)[0]
    flh = randn(g, B, NC, H, N, D)
    h0 = randn(g, B, H, N, D)
    cs, sfin = o.inter_chunk_scan(tA, flh, N, h0)
    tc = (tA[..., 0::2] + 1j * tA[..., 1::2]).numpy()            # (B,NC,H,N/2)
    Fc = (flh[..., 0::2, :] + 1j * flh[..., 1::2, :]).numpy()     # (B,NC,H,N/2,D)
    hc = (h0[..., 0::2, :] + 1j * h0[..., 1::2, :]).numpy()
    for kk in range(NC + 1):
        want = np.prod(tc[:, :kk], axis=1)[..., None] * hc
        for j in range(kk):
            want = want + np.prod(tc[:, j + 1:kk], axis=1)[..., None] * Fc[:, j]
        got = cs[:, kk] if kk < NC else sfin
        np.testing.assert_allclose((got[..., 0::2, :] + 1j * got[..., 1::2, :]).numpy(), want, atol=1e-12)


def test_correction_known_answers_and_linearity():
    g = rng(10)
    B, NC, C, H, D, N = 2, 3, 5, 2, 4, 2
    A, K, _, beta = _rand_scan_inputs(g, B * NC, C, H, D, N)
    A, K, beta = A.reshape(B, NC, C, H, N), K.reshape(B, NC, C, H, D), beta.reshape(B, NC, C, H)
    s1, s2 = randn(g, B, NC, H, N, D), randn(g, B, NC, H, N, D)
    c1 = o.exact_correction(A, K, beta, s1, N)
    c2 = o.exact_correction(A, K, beta, s2, N)
    c12 = o.exact_correction(A, K, beta, 2.0 * s1 - 3.0 * s2, N)
    assert torch.allclose(c12, 2.0 * c1 - 3.0 * c2, atol=1e-12)
    assert torch.allclose(c1[:, :, 0], s1)                               # stored before step 0
    # beta = 0: c_t = gamma_{t-1} s (rotation only, lagging one step)
    c0 = o.exact_correction(A, K, torch.zeros_like(beta), s1, N)
    Ac = (A[..., 0::2] + 1j * A[..., 1::2]).numpy()
    sc = (s1[..., 0::2, :] + 1j * s1[..., 1::2, :]).numpy()
    for t in range(C):
        gam = np.prod(Ac[:, :, :t], axis=2)
        want = gam[..., None] * sc
        got = c0[:, :, t]
        np.testing.assert_allclose((got[..., 0::2, :] + 1j * got[..., 1::2, :]).numpy(), want, atol=1e-12)


def _brute_correction(A, K, beta, S0):
    """Explicit real matrices: corrections[t] = state before step t, each step
    S <- R_t (S (I - beta_t k_t k_t^T)) with R_t the block-diagonal rotation of the
    interleaved pairs (exact_correction.cu:83-150).  A (B,NC,C,H,N), S0 (B,NC,H,N,D)."""
    A, K, beta, S0 = (x.numpy() for x in (A, K, beta, S0))
    B, NC, C, H, D = K.shape
    N = A.shape[-1]
    out = np.zeros((B, NC, C, H, N, D))
    for b in range(B):
        for n in range(NC):
            for h in range(H):
                S = S0[b, n, h].copy()
                for t in range(C):
                    out[b, n, t, h] = S
                    k = K[b, n, t, h]
                    S = _blockdiag_rot(A[b, n, t, h]) @ (S @ (np.eye(D) - beta[b, n, t, h] * np.outer(k, k)))
    return out


def test_correction_matches_brute_force_matrices_with_erasures():
    """beta != 0, N = 4 (two pairs), several chunks: every stored correction state
    against products of explicit (N x N) rotation and (D x D) projection matrices --
    a k / beta index slip or a store-after would fail."""
    g = rng(21)
    B, NC, C, H, D, N = 2, 3, 6, 2, 5, 4
    A, K, _, beta = _rand_scan_inputs(g, B * NC, C, H, D, N)
    A, K, beta = A.reshape(B, NC, C, H, N), K.reshape(B, NC, C, H, D), beta.reshape(B, NC, C, H)
    S0 = randn(g, B, NC, H, N, D)
    got = o.exact_correction(A, K, beta, S0, N)
    np.testing.assert_allclose(got.numpy(), _brute_correction(A, K, beta, S0), atol=1e-12)


def test_single_chunk_R_runs_one_step_behind_E_with_state_and_writes():
    """One chunk, h0 != 0, beta != 0: by linearity E's state is z_t (the local scan from
    zero) plus h0 pushed through steps 0..t, while R's correction pushes h0 through steps
    0..t-1 only (F2), so  Y^R_{t+1} - z_{t+1} = Y^E_t - z_t  for every t."""
    g = rng(22)
    B, L, H, D, N = 2, 10, 3, 6, 4
    A, K, V, beta = _full_inputs(g, B, L, H, D, N)
    h0 = randn(g, B, H, N, D)
    YR = o.ssd_chunkwise_scan(A, K, V, beta, L, N, h0=h0)
    YE, _ = o.exact_recurrence(A, K, V, beta, N, h0)
    z, _ = o.exact_recurrence(A, K, V, beta, N)           # the local scan from zero (one chunk)
    assert torch.allclose(YR[:, 0] - z[:, 0], h0, atol=1e-12)
    for t in range(L - 1):
        assert torch.allclose(YR[:, t + 1] - z[:, t + 1], YE[:, t] - z[:, t], atol=1e-12), t


def _eig_sq_np(alpha, omega, dt):
    """((1-ta)^2 + tw^2) / ((1+ta)^2 + tw^2 + 1e-6), ta = dt/2 max(alpha,0), tw = dt/2 omega (plain numpy)."""
    ta, tw = 0.5 * dt * max(alpha, 0.0), 0.5 * dt * omega
    return ((1 - ta) ** 2 + tw ** 2) / ((1 + ta) ** 2 + tw ** 2 + 1e-6)


def test_dynamics_bwd_vp_clamp_gradient_by_value():
    """Inside the VP clamp (1 - E^(c r) < 1e-6, so vp = sqrt(1e-6)) the forward is flat, but the
    reference passes g_vp * (-0.5 / vp) into d|eig_eff| anyway (dynamics_fused.cu:247-259).  That is
    the derivative of the smooth surrogate sqrt(1 - E^(c r) + delta) with the constant delta that puts
    it at 1e-6 here.  The surrogate is built in plain numpy from the closed forms (softplus, sigmoid,
    Cayley |eig|^2, the adaptive dt with its cap) and differentiated by central differences in every
    gate it depends on; the restated reference backward must give the same values."""
    H, N, c = 1, 2, math.log(2048.0)
    # alpha ~ 1e-13 (E ~ 1 - 1e-6 / D), r ~ 0.0067 (c r ~ 0.05): 1 - E^(c r) ~ 4e-8 < 1e-6
    raw = {"alpha": -30.0, "omega": 0.7, "sel_B": 0.1, "sel_C": 0.2, "sel_dt": -0.5, "beta": 0.3, "r": -5.0}
    log_dt_scale, rope, omega_thresh, delta, smooth, eps_adt = 0.4, 0.0, 0.0883883, 0.125, 0.0176777, 1.0

    def sp(x):
        return x if x > 20 else math.log1p(math.exp(x))

    def sg(x):
        return 1.0 / (1.0 + math.exp(-x))

    def dt_of(rw, lds):
        a0, w0 = sp(rw["alpha"]), rw["omega"]
        dt_raw = sp(lds) / (a0 + abs(w0) + eps_adt)
        dt_max = (2.0 - delta) / (a0 + eps_adt)
        bl = sg((omega_thresh - abs(w0)) / smooth)
        return bl * min(dt_raw, dt_max) + (1 - bl) * dt_raw + sp(rw["sel_dt"])

    def parts(rw, lds):
        E = max(_eig_sq_np(sp(rw["alpha"]), rw["omega"], dt_of(rw, lds)), 1e-8)
        return 1.0 - E ** (c * sg(rw["r"]))

    base = parts(raw, log_dt_scale)
    assert 0 < base < 1e-6                                   # inside the clamp
    shift = 1e-6 - base

    def surrogate(rw, lds):
        return math.sqrt(parts(rw, lds) + shift)

    gate_raw = torch.tensor([[[raw["alpha"], raw["omega"], raw["sel_B"], raw["sel_C"], raw["sel_dt"],
                               raw["beta"], raw["r"]]]], dtype=DT)
    A, vp, _, _ = o.dynamics_fused_fwd(gate_raw, torch.tensor([log_dt_scale]), torch.tensor([rope]), c,
                                       omega_thresh, delta, smooth, eps_adt, H, N)
    assert abs(float(vp) - 1e-3) < 1e-15                     # the clamp value sqrt(1e-6)
    g_raw, g_lds = o.dynamics_fused_bwd_ref(torch.zeros_like(A), torch.ones_like(vp), torch.zeros(1, 1, 1),
                                            torch.zeros(1, 1, 1), gate_raw, torch.tensor([log_dt_scale]),
                                            torch.tensor([rope]), c, omega_thresh, delta, smooth, eps_adt, H, N)
    order = ["alpha", "omega", "sel_B", "sel_C", "sel_dt", "beta", "r"]
    h = 1e-6
    for i, name in enumerate(order):
        up, dn = dict(raw), dict(raw)
        up[name] += h
        dn[name] -= h
        fd = (surrogate(up, log_dt_scale) - surrogate(dn, log_dt_scale)) / (2 * h)
        got = float(g_raw[0, 0, i])
        assert abs(got - fd) <= 1e-6 * max(1.0, abs(fd)), (name, got, fd)
    fd = (surrogate(raw, log_dt_scale + h) - surrogate(raw, log_dt_scale - h)) / (2 * h)
    assert abs(float(g_lds[0]) - fd) <= 1e-6 * max(1.0, abs(fd)), (float(g_lds[0]), fd)
    # the clamped forward itself is flat here: its differences are exactly 0, the rule's gradient is not
    def clamped(rw):
        return math.sqrt(max(parts(rw, log_dt_scale), 1e-6))
    up, dn = dict(raw), dict(raw)
    up["omega"] += h
    dn["omega"] -= h
    assert clamped(up) == clamped(dn)
    assert float(g_raw.abs().max()) > 1e-5


# --------------------------------------------------------------------------
# Full R-mode scan: relation to the exact recurrence, causality, linearity
# --------------------------------------------------------------------------

def _full_inputs(g, B, L, H, D, N):
    A, K, V, beta = _rand_scan_inputs(g, B, L, H, D, N)
    return A, K, V, beta


def test_R_equals_E_for_single_chunk_zero_state():
    g = rng(11)
    A, K, V, beta = _full_inputs(g, 2, 16, 3, 8, 4)
    YR = o.ssd_chunkwise_scan(A, K, V, beta, 16, 4)
    YE, _ = o.exact_recurrence(A, K, V, beta, 4)
    assert torch.allclose(YR, YE, atol=1e-12)
    YR4 = o.ssd_chunkwise_scan(A, K, V, beta, 4, 4)
    assert not torch.allclose(YR4, YE, atol=1e-3)          # R depends on the chunk size


def test_R_lags_E_by_one_step_without_writes():
    """beta = 0: E gives prod_{u<=t} a_u h0, R gives prod_{u<t} a_u h0 (F2)."""
    g = rng(12)
    B, L, H, D, N, Q = 1, 12, 2, 3, 2, 4
    A, K, V, _ = _full_inputs(g, B, L, H, D, N)
    beta = torch.zeros(B, L, H)
    h0 = randn(g, B, H, N, D)
    YR = o.ssd_chunkwise_scan(A, K, V, beta, Q, N, h0=h0)
    YE, _ = o.exact_recurrence(A, K, V, beta, N, h0)
    Ac = (A[..., 0::2] + 1j * A[..., 1::2]).numpy()
    hc = (h0[..., 0::2, :] + 1j * h0[..., 1::2, :]).numpy()
    for t in range(L):
        gE = np.prod(Ac[:, :t + 1], axis=1)[..., None] * hc
        gR = np.prod(Ac[:, :t], axis=1)[..., None] * hc
        yR, yE = YR[:, t], YE[:, t]
        np.testing.assert_allclose((yE[..., 0::2, :] + 1j * yE[..., 1::2, :]).numpy(), gE, atol=1e-12)
        np.testing.assert_allclose((yR[..., 0::2, :] + 1j * yR[..., 1::2, :]).numpy(), gR, atol=1e-12)


def test_R_scan_causal_padding_and_linearity():
    g = rng(13)
    B, H, D, N, Q = 2, 2, 6, 2, 8
    A, K, V, beta = _full_inputs(g, B, 32, H, D, N)
    Y32 = o.ssd_chunkwise_scan(A, K, V, beta, Q, N)
    Y27 = o.ssd_chunkwise_scan(A[:, :27], K[:, :27], V[:, :27], beta[:, :27], Q, N)
    assert torch.allclose(Y32[:, :27], Y27, atol=1e-12)     # causal; zero padding is inert
    V2 = randn(g, *V.shape)
    h1, h2 = randn(g, B, H, N, D), randn(g, B, H, N, D)
    Ya = o.ssd_chunkwise_scan(A, K, V, beta, Q, N, h0=h1)
    Yb = o.ssd_chunkwise_scan(A, K, V2, beta, Q, N, h0=h2)
    Yab = o.ssd_chunkwise_scan(A, K, V + V2, beta, Q, N, h0=h1 + h2)
    assert torch.allclose(Yab, Ya + Yb, atol=1e-12)


def test_final_state_continues_the_scan():
    """s_final of a prefix is chunk_states[k] of the longer sequence (decode continuity)."""
    g = rng(14)
    B, H, D, N, Q = 1, 3, 4, 2, 4
    A, K, V, beta = _full_inputs(g, B, 20, H, D, N)
    h0 = randn(g, B, H, N, D)
    _, s8 = o.ssd_chunkwise_scan(A[:, :8], K[:, :8], V[:, :8], beta[:, :8], Q, N, h0=h0, return_final=True)
    Yfull = o.ssd_chunkwise_scan(A, K, V, beta, Q, N, h0=h0)
    Ytail = o.ssd_chunkwise_scan(A[:, 8:], K[:, 8:], V[:, 8:], beta[:, 8:], Q, N, h0=s8)
    assert torch.allclose(Yfull[:, 8:], Ytail, atol=1e-12)
    # padded tail: s_final after 10 tokens seeds the scan of the next tokens at a chunk boundary
    _, s10 = o.ssd_chunkwise_scan(A[:, :10], K[:, :10], V[:, :10], beta[:, :10], Q, N, h0=h0,
                                  return_final=True)
    Y10 = o.ssd_chunkwise_scan(A[:, :10], K[:, :10], V[:, :10], beta[:, :10], 10, N, h0=None)
    # with Q = L (one chunk, zero state) the R carry is the local state after the last token
    _, s10b = o.ssd_chunkwise_scan(A[:, :10], K[:, :10], V[:, :10], beta[:, :10], 10, N, return_final=True)
    assert torch.allclose(s10b, Y10[:, -1], atol=1e-12)
    assert s10.shape == h0.shape


# --------------------------------------------------------------------------
# Gradients
# --------------------------------------------------------------------------

def test_intra_and_inter_bwd_restatements_match_autograd():
    g = rng(15)
    A, K, V, beta = _rand_scan_inputs(g, 3, 6, 2, 5, 4)
    for t in (A, K, V, beta):
        t.requires_grad_(True)
    lh, ca = o.intra_chunk_scan(A, K, V, beta, 4)
    glh, gca = randn(g, *lh.shape), randn(g, *ca.shape)
    auto = torch.autograd.grad((lh * glh).sum() + (ca * gca).sum(), [A, K, V, beta])
    hand = o.intra_chunk_scan_bwd_ref(glh, gca, A.detach(), K.detach(), V.detach(), beta.detach(), 4)
    for x, y in zip(hand, auto):
        assert torch.allclose(x, y, atol=1e-11)
    B, NC, H, N, D = 2, 5, 3, 4, 6
    tA = _rand_scan_inputs(g, B, NC, H, D, N)[0].requires_grad_(True)
    flh = randn(g, B, NC, H, N, D).requires_grad_(True)
    h0 = randn(g, B, H, N, D).requires_grad_(True)
    cs, sf = o.inter_chunk_scan(tA, flh, N, h0)
    gcs, gsf = randn(g, *cs.shape), randn(g, *sf.shape)
    auto = torch.autograd.grad((cs * gcs).sum() + (sf * gsf).sum(), [tA, flh, h0])
    hand = o.inter_chunk_scan_bwd_ref(gcs, tA.detach(), cs.detach(), N, grad_final=gsf)
    for x, y in zip(hand, auto):
        assert torch.allclose(x, y, atol=1e-11)


def test_correction_bwd_restatement_is_the_shifted_gradient():
    """The reference's correction backward equals the gradient of sum <g_t, c_{t+1}>,
    and differs from the gradient of its own forward sum <g_t, c_t>."""
    g = rng(16)
    B, NC, C, H, D, N = 2, 2, 5, 2, 4, 4
    A, K, _, beta = _rand_scan_inputs(g, B * NC, C, H, D, N)
    A = A.reshape(B, NC, C, H, N).requires_grad_(True)
    K = K.reshape(B, NC, C, H, D).requires_grad_(True)
    beta = beta.reshape(B, NC, C, H).requires_grad_(True)
    s = randn(g, B, NC, H, N, D).requires_grad_(True)
    gc = randn(g, B, NC, C, H, N, D)
    hand = o.exact_correction_bwd_ref(gc, A.detach(), K.detach(), beta.detach(), s.detach(), N)
    # states after each step: c_{t+1}
    h = s
    after = []
    for t in range(C):
        h = o.cmul_rows(A[:, :, t], o._erase(h, K[:, :, t], beta[:, :, t]))
        after.append(h)
    after = torch.stack(after, 2)
    shifted = torch.autograd.grad((after * gc).sum(), [A, K, beta, s])
    for x, y in zip(hand, shifted):
        assert torch.allclose(x, y, atol=1e-11)
    true = torch.autograd.grad((o.exact_correction(A, K, beta, s, N) * gc).sum(), [A, K, beta, s])
    assert not torch.allclose(hand[3], true[3], atol=1e-3)
    assert not torch.allclose(hand[0], true[0], atol=1e-3)


def test_gradcheck_fused_scan_both_grad_modes():
    g = rng(17)
    B, L, H, D, N, Q = 1, 8, 2, 3, 2, 4
    q = unit(randn(g, B, L, H, D)).requires_grad_(True)
    k = unit(randn(g, B, L, H, D)).requires_grad_(True)
    v = randn(g, B, L, H, N).requires_grad_(True)
    beta = (torch.rand(B, L, H, generator=g) * 0.9 + 0.05).requires_grad_(True)
    selc = torch.rand(B, L, H, generator=g).requires_grad_(True)
    dt = (torch.rand(B, L, H, generator=g) + 0.1).requires_grad_(True)
    r = (torch.rand(B, L, H, generator=g) * 0.8 + 0.1).requires_grad_(True)
    alpha = (torch.rand(H, generator=g) + 0.1).requires_grad_(True)
    omega = randn(g, H).requires_grad_(True)
    h0 = randn(g, B, H, N, D).requires_grad_(True)
    args = (q, k, v, beta, selc, dt, r, alpha, omega)

    def f(*a):
        y, s = o.fused_scan(*a, c=math.log(L), h0=h0, chunk_size=Q, grad_mode="exact")
        return y, s
    assert torch.autograd.gradcheck(f, args, eps=1e-6, atol=1e-6)
    # reference grad mode differs from the exact gradient (correction pass), same forward
    yr, sr = o.fused_scan(*args, c=math.log(L), h0=h0, chunk_size=Q, grad_mode="reference")
    ye, se = o.fused_scan(*args, c=math.log(L), h0=h0, chunk_size=Q, grad_mode="exact")
    assert torch.equal(yr, ye) and torch.equal(sr, se)
    w = randn(g, *yr.shape)
    gr = torch.autograd.grad((yr * w).sum(), [k, h0])
    ge = torch.autograd.grad((ye * w).sum(), [k, h0])
    assert not torch.allclose(gr[1], ge[1], atol=1e-4)
