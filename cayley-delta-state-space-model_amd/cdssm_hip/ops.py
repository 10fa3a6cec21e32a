"""Drop-in autograd Functions with the reference ``cdssm/ops.py`` signatures.

Each class keeps the reference's ``forward``/``backward`` argument order,
return arity, shapes and save-for-backward policy (ops.py:31-195), and runs
one C-ABI entry point of ``libcdssm_hip.so`` per pass.  Tensor inputs may be
bfloat16 (the reference's only dtype) or float32; outputs take the input
dtype.  Non-tensor arguments get ``None`` gradients, as in the reference.
``CUDAConv1dSiLUOp`` (ops.py:13-28) is not part of this library.

There is no CPU path: every op requires CUDA (ROCm) tensors and raises
otherwise, as the reference launchers do (intra_chunk_scan.cu:568-571).
"""

from __future__ import annotations

from typing import Tuple

import torch
from torch import Tensor
from torch.autograd import Function

from . import _lib


def _prep(op: str, *tensors: Tensor):
    """Contiguous copies, one shared dtype (bf16/fp32), one CUDA device."""
    dev = tensors[0].device
    if dev.type != "cuda":
        raise RuntimeError(f"{op}: inputs must be CUDA tensors (GPU only)")
    dtype = tensors[0].dtype
    if dtype not in _lib.DTYPE_CODE:
        raise TypeError(f"{op}: dtype must be bfloat16 or float32, got {dtype}")
    out = []
    for t in tensors:
        if t.device != dev:
            raise RuntimeError(f"{op}: all tensors must be on {dev}")
        if t.dtype != dtype:
            raise TypeError(f"{op}: all tensors must share dtype {dtype}, got {t.dtype}")
        out.append(t.contiguous())
    return out, _lib.DTYPE_CODE[dtype], dev


def _check_n(op: str, state_dim: int) -> int:
    n = int(state_dim)
    if n <= 0 or n % 2 or n > 32:
        raise ValueError(f"{op}: state_dim must be even and in [2, 32], got {state_dim}")
    return n


def _stream(dev):
    return _lib.stream_of(dev)


# ---------------------------------------------------------------------------
# DynamicsFusedFn (ops.py:31-81)
# ---------------------------------------------------------------------------

class DynamicsFusedFn(Function):
    """gate_raw (B, L, (N+5)H) -> A_bar (B,L,H,N), vp_scale (B,L,H,N/2), beta (B,L,H), sel_C (B,L,H)."""

    @staticmethod
    def forward(ctx, gate_raw, log_dt_scale, rope_freqs, gating_c, omega_thresh, adt_delta,
                adt_smoothness, adt_eps, n_heads, state_dim):
        op = "DynamicsFusedFn"
        (g,), code, dev = _prep(op, gate_raw)
        H, N = int(n_heads), _check_n(op, state_dim)
        B, L, GH = g.shape
        if GH != (N + 5) * H:
            raise ValueError(f"{op}: gate_raw last dim must be (state_dim + 5) * n_heads = {(N + 5) * H}, got {GH}")
        lds = log_dt_scale.float().contiguous()
        rf = rope_freqs.float().contiguous()
        if lds.shape != (H,) or rf.shape != (H,):
            raise ValueError(f"{op}: log_dt_scale and rope_freqs must have shape ({H},)")
        A = torch.empty(B, L, H, N, dtype=g.dtype, device=dev)
        vp = torch.empty(B, L, H, N // 2, dtype=g.dtype, device=dev)
        beta = torch.empty(B, L, H, dtype=g.dtype, device=dev)
        selc = torch.empty(B, L, H, dtype=g.dtype, device=dev)
        lib = _lib.load()
        st = lib.cdssm_dynamics_fused_fwd(code, _lib.ptr(g), _lib.ptr(lds), _lib.ptr(rf), float(gating_c),
                                          float(omega_thresh), float(adt_delta), float(adt_smoothness),
                                          float(adt_eps), _lib.ptr(A), _lib.ptr(vp), _lib.ptr(beta),
                                          _lib.ptr(selc), B, L, H, N, _stream(dev))
        _lib.check(st, "cdssm_dynamics_fused_fwd")
        ctx.save_for_backward(g, lds, rf)
        ctx.consts = (float(gating_c), float(omega_thresh), float(adt_delta), float(adt_smoothness),
                      float(adt_eps), H, N)
        return A, vp, beta, selc

    @staticmethod
    def backward(ctx, grad_A_bar, grad_vp_scale, grad_beta, grad_sel_C):
        g, lds, rf = ctx.saved_tensors
        c, thr, delta, smooth, eps, H, N = ctx.consts
        B, L, _ = g.shape
        grads, code, dev = _prep("DynamicsFusedFn.backward", *[x.to(g.dtype) for x in
                                                               (grad_A_bar, grad_vp_scale, grad_beta, grad_sel_C)])
        ggate = torch.empty_like(g)
        glds = torch.empty(H, dtype=torch.float32, device=dev)
        lib = _lib.load()
        ws = torch.empty(lib.cdssm_dynamics_fused_bwd_workspace_bytes(B, L, H) // 4, dtype=torch.float32,
                         device=dev)
        st = lib.cdssm_dynamics_fused_bwd(code, *[_lib.ptr(x) for x in grads], _lib.ptr(g), _lib.ptr(lds),
                                          _lib.ptr(rf), c, thr, delta, smooth, eps, _lib.ptr(ggate),
                                          _lib.ptr(glds), _lib.ptr(ws), B, L, H, N, _stream(dev))
        _lib.check(st, "cdssm_dynamics_fused_bwd")
        return ggate, glds, None, None, None, None, None, None, None, None


# ---------------------------------------------------------------------------
# NormalizeKQFn (ops.py:84-97)
# ---------------------------------------------------------------------------

class NormalizeKQFn(Function):
    """L2 normalisation x * rsqrt(sum x^2 + 1e-6) of K and Q over the last dim."""

    @staticmethod
    def forward(ctx, K: Tensor, Q: Tensor) -> Tuple[Tensor, Tensor]:
        (k, q), code, dev = _prep("NormalizeKQFn", K, Q)
        if k.shape != q.shape:
            raise ValueError(f"NormalizeKQFn: K and Q shapes differ: {tuple(k.shape)} vs {tuple(q.shape)}")
        D = k.shape[-1]
        rows = k.numel() // D
        ko, qo = torch.empty_like(k), torch.empty_like(q)
        st = _lib.load().cdssm_normalize_kq_fwd(code, _lib.ptr(k), _lib.ptr(q), _lib.ptr(ko), _lib.ptr(qo),
                                                rows, D, _stream(dev))
        _lib.check(st, "cdssm_normalize_kq_fwd")
        ctx.save_for_backward(k, q)
        return ko, qo

    @staticmethod
    def backward(ctx, grad_K_out: Tensor, grad_Q_out: Tensor):
        k, q = ctx.saved_tensors
        (gk, gq), code, dev = _prep("NormalizeKQFn.backward", grad_K_out.to(k.dtype), grad_Q_out.to(k.dtype))
        D = k.shape[-1]
        rows = k.numel() // D
        ok, oq = torch.empty_like(k), torch.empty_like(q)
        st = _lib.load().cdssm_normalize_kq_bwd(code, _lib.ptr(gk), _lib.ptr(gq), _lib.ptr(k), _lib.ptr(q),
                                                _lib.ptr(ok), _lib.ptr(oq), rows, D, _stream(dev))
        _lib.check(st, "cdssm_normalize_kq_bwd")
        return ok, oq


# ---------------------------------------------------------------------------
# IntraChunkScanFn (ops.py:100-135)
# ---------------------------------------------------------------------------

class IntraChunkScanFn(Function):
    """(A (BNC,C,H,N), K (BNC,C,H,D), V (BNC,C,H,N), beta (BNC,C,H), N) -> (local_h, cum_A)."""

    @staticmethod
    def forward(ctx, A_flat, K_flat, V_flat, beta_flat, state_dim):
        op = "IntraChunkScanFn"
        N = _check_n(op, state_dim)
        (A, K, V, b), code, dev = _prep(op, A_flat, K_flat, V_flat, beta_flat)
        BNC, C, H, D = K.shape
        if A.shape != (BNC, C, H, N) or V.shape != (BNC, C, H, N) or b.shape != (BNC, C, H):
            raise ValueError(f"{op}: shape mismatch A {tuple(A.shape)} K {tuple(K.shape)} "
                             f"V {tuple(V.shape)} beta {tuple(b.shape)} for state_dim {N}")
        local_h = torch.empty(BNC, C, H, N, D, dtype=K.dtype, device=dev)
        cum_A = torch.empty(BNC, C, H, N, dtype=K.dtype, device=dev)
        st = _lib.load().cdssm_intra_chunk_scan_fwd(code, _lib.ptr(A), _lib.ptr(K), _lib.ptr(V), _lib.ptr(b),
                                                    _lib.ptr(local_h), _lib.ptr(cum_A), BNC, C, H, D, N,
                                                    _stream(dev))
        _lib.check(st, "cdssm_intra_chunk_scan_fwd")
        ctx.save_for_backward(A, K, V, b, local_h, cum_A)
        ctx.state_dim = N
        return local_h, cum_A

    @staticmethod
    def backward(ctx, grad_local_h, grad_cum_A):
        A, K, V, b, local_h, cum_A = ctx.saved_tensors
        N = ctx.state_dim
        BNC, C, H, D = K.shape
        if grad_local_h is None:
            grad_local_h = torch.zeros_like(local_h)
        if grad_cum_A is None:
            grad_cum_A = torch.zeros_like(cum_A)
        (glh, gca), code, dev = _prep("IntraChunkScanFn.backward", grad_local_h.to(K.dtype),
                                      grad_cum_A.to(K.dtype))
        gA, gK, gV, gB = (torch.empty_like(A), torch.empty_like(K), torch.empty_like(V), torch.empty_like(b))
        st = _lib.load().cdssm_intra_chunk_scan_bwd(code, _lib.ptr(glh), _lib.ptr(gca), _lib.ptr(A), _lib.ptr(K),
                                                    _lib.ptr(V), _lib.ptr(b), _lib.ptr(local_h), _lib.ptr(cum_A),
                                                    _lib.ptr(gA), _lib.ptr(gK), _lib.ptr(gV), _lib.ptr(gB),
                                                    BNC, C, H, D, N, _stream(dev))
        _lib.check(st, "cdssm_intra_chunk_scan_bwd")
        return gA, gK, gV, gB, None


# ---------------------------------------------------------------------------
# InterChunkScanFn (ops.py:138-163)
# ---------------------------------------------------------------------------

class InterChunkScanFn(Function):
    """(total_A (B,NC,H,N), final_local_h (B,NC,H,N,D), N) -> chunk_states (B,NC,H,N,D)."""

    @staticmethod
    def forward(ctx, total_A, final_local_h, state_dim):
        op = "InterChunkScanFn"
        N = _check_n(op, state_dim)
        (tA, flh), code, dev = _prep(op, total_A, final_local_h)
        B, NC, H, N2, D = flh.shape
        if N2 != N or tA.shape != (B, NC, H, N):
            raise ValueError(f"{op}: shape mismatch total_A {tuple(tA.shape)} final_local_h {tuple(flh.shape)}")
        cs = torch.empty_like(flh)
        st = _lib.load().cdssm_inter_chunk_scan_fwd(code, _lib.ptr(tA), _lib.ptr(flh), _lib.ptr(cs), B, NC, H, D, N,
                                                    _stream(dev))
        _lib.check(st, "cdssm_inter_chunk_scan_fwd")
        ctx.save_for_backward(tA, cs)
        ctx.state_dim = N
        return cs

    @staticmethod
    def backward(ctx, grad_chunk_states):
        tA, cs = ctx.saved_tensors
        N = ctx.state_dim
        B, NC, H, _, D = cs.shape
        (g,), code, dev = _prep("InterChunkScanFn.backward", grad_chunk_states.to(cs.dtype))
        gtA, gflh = torch.empty_like(tA), torch.empty_like(cs)
        st = _lib.load().cdssm_inter_chunk_scan_bwd(code, _lib.ptr(g), _lib.ptr(tA), _lib.ptr(cs), _lib.ptr(gtA),
                                                    _lib.ptr(gflh), B, NC, H, D, N, _stream(dev))
        _lib.check(st, "cdssm_inter_chunk_scan_bwd")
        return gtA, gflh, None


# ---------------------------------------------------------------------------
# ExactCorrectionFn (ops.py:166-195)
# ---------------------------------------------------------------------------

class ExactCorrectionFn(Function):
    """(A (B,NC,C,H,N), K (B,NC,C,H,D), beta (B,NC,C,H), chunk_states (B,NC,H,N,D), N) -> corrections."""

    @staticmethod
    def forward(ctx, A_chunk, K_chunk, beta_chunk, chunk_states, state_dim):
        op = "ExactCorrectionFn"
        N = _check_n(op, state_dim)
        (A, K, b, cs), code, dev = _prep(op, A_chunk, K_chunk, beta_chunk, chunk_states)
        B, NC, C, H, D = K.shape
        if A.shape != (B, NC, C, H, N) or b.shape != (B, NC, C, H) or cs.shape != (B, NC, H, N, D):
            raise ValueError(f"{op}: shape mismatch A {tuple(A.shape)} K {tuple(K.shape)} beta {tuple(b.shape)} "
                             f"chunk_states {tuple(cs.shape)}")
        corr = torch.empty(B, NC, C, H, N, D, dtype=K.dtype, device=dev)
        st = _lib.load().cdssm_exact_correction_fwd(code, _lib.ptr(A), _lib.ptr(K), _lib.ptr(b), _lib.ptr(cs),
                                                    _lib.ptr(corr), B, NC, C, H, D, N, _stream(dev))
        _lib.check(st, "cdssm_exact_correction_fwd")
        ctx.save_for_backward(A, K, b, cs, corr)
        ctx.state_dim = N
        return corr

    @staticmethod
    def backward(ctx, grad_corrections):
        A, K, b, cs, corr = ctx.saved_tensors
        N = ctx.state_dim
        B, NC, C, H, D = K.shape
        (g,), code, dev = _prep("ExactCorrectionFn.backward", grad_corrections.to(K.dtype))
        gA, gK, gB, gS = torch.empty_like(A), torch.empty_like(K), torch.empty_like(b), torch.empty_like(cs)
        st = _lib.load().cdssm_exact_correction_bwd(code, _lib.ptr(g), _lib.ptr(A), _lib.ptr(K), _lib.ptr(b),
                                                    _lib.ptr(cs), _lib.ptr(corr), _lib.ptr(gA), _lib.ptr(gK),
                                                    _lib.ptr(gB), _lib.ptr(gS), B, NC, C, H, D, N, _stream(dev))
        _lib.check(st, "cdssm_exact_correction_bwd")
        return gA, gK, gB, gS, None
