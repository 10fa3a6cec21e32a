"""Recurrent decode of the fused scan, host side.

The reference generates one token at a time by re-running the whole forward
over the growing sequence (predict.py:53-67).  ``decode_step`` instead
advances a per-(b, h) R-mode state by one token on the GPU
(``cdssm_decode_step``) and returns the same output the chunked scan
(ssd.py:39-111, readout block.py:208-211) gives at that position, chunk
boundaries included.  ``prefill`` runs the fused forward over the longest
chunk-aligned prefix and decode steps over the rest, and returns the state
to continue from.
"""

from __future__ import annotations

from typing import Optional, Tuple

import torch

from . import _lib
from .scan import chunkwise_delta_scan, chunkwise_delta_scan_abar

Tensor = torch.Tensor


class DecodeState:
    """R-mode state of B sequences x H heads (fp32, on the GPU).

    ``state`` (B, H, 3, 2, D): local state z, decay-free correction c^ and the
    carry s entering the current chunk; ``gam`` (B, H, 2): rotation product of
    the chunk so far; ``pos`` (B, H) int32: position in the chunk.
    """

    def __init__(self, state: Tensor, gam: Tensor, pos: Tensor, chunk_size: int):
        self.state, self.gam, self.pos, self.chunk_size = state, gam, pos, int(chunk_size)

    @property
    def shape(self) -> Tuple[int, int, int]:
        B, H, _, _, D = self.state.shape
        return B, H, D

    @classmethod
    def at_boundary(cls, h: Optional[Tensor], B: int, H: int, D: int, chunk_size: int,
                    device: torch.device) -> "DecodeState":
        """State at a chunk boundary with carry h (B, H, 2, D) fp32 (None: zero state)."""
        if h is not None:
            if h.dtype != torch.float32 or tuple(h.shape) != (B, H, 2, D) or h.device != device:
                raise ValueError(f"h must be float32 ({B}, {H}, 2, {D}) on {device}")
            h = h.contiguous()
        if not 1 <= int(chunk_size) <= 128:
            raise ValueError(f"chunk_size must be in [1, 128], got {chunk_size}")
        state = torch.empty(B, H, 3, 2, D, dtype=torch.float32, device=device)
        gam = torch.empty(B, H, 2, dtype=torch.float32, device=device)
        pos = torch.empty(B, H, dtype=torch.int32, device=device)
        st = _lib.load().cdssm_decode_init(_lib.ptr(h), _lib.ptr(state), _lib.ptr(gam), _lib.ptr(pos), B, H, D, 2,
                                           _lib.stream_of(device))
        _lib.check(st, "cdssm_decode_init")
        return cls(state, gam, pos, chunk_size)


def _token(x: Tensor, B: int, H: int, tail: Tuple[int, ...], name: str) -> Tensor:
    # accept (B, H, ...) or the (B, 1, H, ...) slice of a sequence tensor
    if x.dim() == 3 + len(tail) and x.shape[1] == 1:
        x = x.reshape((B, H) + tail)
    if tuple(x.shape) != (B, H) + tail:
        raise ValueError(f"{name} has shape {tuple(x.shape)}, expected {(B, H) + tail} or {(B, 1, H) + tail}")
    return x.contiguous()


def decode_step(st: DecodeState, q: Tensor, k: Tensor, v: Tensor, beta: Tensor, sel_C: Tensor, dt: Tensor,
                r: Tensor, alpha: Tensor, omega: Tensor, c: float,
                return_carry: bool = False):
    """One token for every (b, h): y (B, H, 2) [, carry after it (B, H, 2, D) fp32]."""
    B, H, D = st.shape
    dev = st.state.device
    if q.device != dev:
        raise RuntimeError(f"inputs are on {q.device}, the state on {dev}")
    dtype = q.dtype
    if dtype not in _lib.DTYPE_CODE:
        raise TypeError(f"inputs must be float32 or bfloat16, got {dtype}")
    toks = dict(q=_token(q, B, H, (D,), "q"), k=_token(k, B, H, (D,), "k"), v=_token(v, B, H, (2,), "v"),
                beta=_token(beta, B, H, (), "beta"), sel_C=_token(sel_C, B, H, (), "sel_C"),
                dt=_token(dt, B, H, (), "dt"), r=_token(r, B, H, (), "r"))
    for n, t in toks.items():
        if t.dtype != dtype or t.device != dev:
            raise TypeError(f"{n} is {t.dtype} on {t.device}, expected {dtype} on {dev}")
    for n, t in (("alpha", alpha), ("omega", omega)):
        if t.dtype != torch.float32 or tuple(t.shape) != (H,) or t.device != dev:
            raise ValueError(f"{n} must be float32 of shape ({H},) on {dev}")
    y = torch.empty(B, H, 2, dtype=dtype, device=dev)
    h = torch.empty(B, H, 2, D, dtype=torch.float32, device=dev) if return_carry else None
    status = _lib.load().cdssm_decode_step(
        _lib.DTYPE_CODE[dtype], *[_lib.ptr(toks[n]) for n in ("q", "k", "v", "beta", "sel_C", "dt", "r")],
        _lib.ptr(alpha.contiguous()), _lib.ptr(omega.contiguous()), float(c), _lib.ptr(st.state), _lib.ptr(st.gam),
        _lib.ptr(st.pos), _lib.ptr(y), _lib.ptr(h), B, H, D, 2, st.chunk_size, _lib.stream_of(dev))
    _lib.check(status, "cdssm_decode_step")
    return (y, h) if return_carry else y


def prefill(q: Tensor, k: Tensor, v: Tensor, beta: Tensor, sel_C: Tensor, dt: Tensor, r: Tensor,
            alpha: Tensor, omega: Tensor, c: float, h0: Optional[Tensor] = None,
            chunk_size: Optional[int] = None) -> Tuple[Tensor, DecodeState]:
    """y (B, L, H, 2) of the prompt and the decode state after its last token.

    The longest prefix of whole chunks goes through the fused scan; the
    remaining L mod Q tokens through decode steps.
    """
    B, L, H, D = q.shape
    Q = D if chunk_size is None else int(chunk_size)
    L0 = (L // Q) * Q
    ys = []
    if L0 > 0:
        pre = [x[:, :L0] for x in (q, k, v, beta, sel_C, dt, r)]
        y0, h = chunkwise_delta_scan(*pre, alpha, omega, c, h0=h0, chunk_size=Q)
        ys.append(y0)
        st = DecodeState.at_boundary(h, B, H, D, Q, q.device)
    else:
        st = DecodeState.at_boundary(h0, B, H, D, Q, q.device)
    for t in range(L0, L):
        tok = [x[:, t] for x in (q, k, v, beta, sel_C, dt, r)]
        ys.append(decode_step(st, *tok, alpha, omega, c).unsqueeze(1))
    y = torch.cat(ys, dim=1) if len(ys) > 1 else ys[0]
    return y, st


def decode_step_abar(st: DecodeState, q: Tensor, k: Tensor, v: Tensor, beta: Tensor, sel_C: Tensor, A_bar: Tensor,
                     vp: Tensor, return_carry: bool = False):
    """``decode_step`` on the gate-level inputs: A_bar (B, H, 2) and vp (B, H) (or (B, H, 1), or the
    (B, 1, H, ...) slices) of the token in place of (dt, r, alpha, omega, c); the form the model's scan
    takes (``chunkwise_delta_scan_abar``)."""
    B, H, D = st.shape
    dev = st.state.device
    if q.device != dev:
        raise RuntimeError(f"inputs are on {q.device}, the state on {dev}")
    dtype = q.dtype
    if dtype not in _lib.DTYPE_CODE:
        raise TypeError(f"inputs must be float32 or bfloat16, got {dtype}")
    vp = vp.reshape(B, H) if vp.numel() == B * H else vp
    toks = dict(q=_token(q, B, H, (D,), "q"), k=_token(k, B, H, (D,), "k"), v=_token(v, B, H, (2,), "v"),
                beta=_token(beta, B, H, (), "beta"), sel_C=_token(sel_C, B, H, (), "sel_C"),
                A_bar=_token(A_bar, B, H, (2,), "A_bar"), vp=_token(vp, B, H, (), "vp"))
    for n, t in toks.items():
        if t.dtype != dtype or t.device != dev:
            raise TypeError(f"{n} is {t.dtype} on {t.device}, expected {dtype} on {dev}")
    y = torch.empty(B, H, 2, dtype=dtype, device=dev)
    h = torch.empty(B, H, 2, D, dtype=torch.float32, device=dev) if return_carry else None
    status = _lib.load().cdssm_decode_step_abar(
        _lib.DTYPE_CODE[dtype], *[_lib.ptr(toks[n]) for n in ("q", "k", "v", "beta", "sel_C", "A_bar", "vp")],
        _lib.ptr(st.state), _lib.ptr(st.gam), _lib.ptr(st.pos), _lib.ptr(y), _lib.ptr(h), B, H, D, 2,
        st.chunk_size, _lib.stream_of(dev))
    _lib.check(status, "cdssm_decode_step_abar")
    return (y, h) if return_carry else y


def prefill_abar(q: Tensor, k: Tensor, v: Tensor, beta: Tensor, sel_C: Tensor, A_bar: Tensor, vp: Tensor,
                 chunk_size: Optional[int] = None) -> Tuple[Tensor, DecodeState]:
    """``prefill`` on the gate-level inputs: y (B, L, H, 2) of the prompt and the decode state after it
    (the chunk-aligned prefix through ``chunkwise_delta_scan_abar``, the rest through decode steps)."""
    B, L, H, D = q.shape
    Q = D if chunk_size is None else int(chunk_size)
    L0 = (L // Q) * Q
    ys = []
    if L0 > 0:
        pre = [x[:, :L0] for x in (q, k, v, beta, sel_C, A_bar, vp)]
        y0, h = chunkwise_delta_scan_abar(*pre, chunk_size=Q)
        ys.append(y0)
        st = DecodeState.at_boundary(h, B, H, D, Q, q.device)
    else:
        st = DecodeState.at_boundary(None, B, H, D, Q, q.device)
    for t in range(L0, L):
        tok = [x[:, t] for x in (q, k, v, beta, sel_C, A_bar, vp)]
        ys.append(decode_step_abar(st, *tok).unsqueeze(1))
    y = torch.cat(ys, dim=1) if len(ys) > 1 else ys[0]
    return y, st
