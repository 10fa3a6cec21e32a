"""Fused chunkwise delta-rule scan (the metric op), host side.

``chunkwise_delta_scan`` runs the scan-level CD-SSM path in one C-ABI call
(``cdssm_fused_scan_fwd``): Cayley/gated dynamics from (dt, r, alpha, omega),
VP-scaled values, the reference's three-pass R-mode scan (intra-chunk,
inter-chunk carry, exact correction; ssd.py:39-111) and the sel_C-gated
readout (block.py:208-211).  It validates on the host, allocates the outputs
and the workspace with torch, and launches on torch's current stream.
"""

from __future__ import annotations

import ctypes

from typing import Optional, Tuple

import torch

from . import _lib

Tensor = torch.Tensor

PER_TOKEN = ("q", "k", "v", "beta", "sel_C", "dt", "r")


def _validate(q, k, v, beta, sel_C, dt, r, alpha, omega, h0, chunk_size, rows: bool = False):
    """Shapes, dtypes and devices of a fused-scan call; ``rows`` admits the gate-level form's even
    state_dim N up to 32 (N / 2 complex state rows per head), else N = 2."""
    named = dict(q=q, k=k, v=v, beta=beta, sel_C=sel_C, dt=dt, r=r, alpha=alpha, omega=omega)
    for n, t in named.items():
        if not isinstance(t, torch.Tensor):
            raise TypeError(f"{n} must be a tensor")
    dev = q.device
    if dev.type != "cuda":
        raise RuntimeError("chunkwise_delta_scan runs on the GPU only: inputs must be on a cuda device")
    for n, t in named.items():
        if t.device != dev:
            raise RuntimeError(f"{n} is on {t.device}, expected {dev}")
    if q.dim() != 4:
        raise ValueError(f"q must be (B, L, H, D), got {tuple(q.shape)}")
    B, L, H, D = q.shape
    N = v.shape[-1] if v.dim() == 4 else -1
    shapes = dict(q=(B, L, H, D), k=(B, L, H, D), v=(B, L, H, N), beta=(B, L, H), sel_C=(B, L, H),
                  dt=(B, L, H), r=(B, L, H))
    for n, shp in shapes.items():
        if tuple(named[n].shape) != shp:
            raise ValueError(f"{n} has shape {tuple(named[n].shape)}, expected {shp}")
    dtype = q.dtype
    if dtype not in _lib.DTYPE_CODE:
        raise TypeError(f"inputs must be float32 or bfloat16, got {dtype}")
    for n in PER_TOKEN:
        if named[n].dtype != dtype:
            raise TypeError(f"{n} has dtype {named[n].dtype}, expected {dtype} (same as q)")
    for n in ("alpha", "omega"):
        t = named[n]
        if t.dtype != torch.float32 or tuple(t.shape) != (H,):
            raise ValueError(f"{n} must be float32 of shape ({H},), got {t.dtype} {tuple(t.shape)}")
    if rows and not (2 <= N <= 32 and N % 2 == 0):
        raise ValueError(f"state_dim N must be even, 2 <= N <= 32, got N = {N}")
    if not rows and N != 2:
        raise ValueError(f"the fused scan supports N = 2 (one complex pair per head), got N = {N}")
    if D not in (64, 128):
        raise ValueError(f"head_dim D must be 64 or 128, got {D}")
    Q = D if chunk_size is None else int(chunk_size)
    if not 1 <= Q <= 128:
        raise ValueError(f"chunk_size must be in [1, 128], got {Q}")
    if h0 is not None:
        if h0.dtype != torch.float32 or tuple(h0.shape) != (B, H, N, D) or h0.device != dev:
            raise ValueError(f"h0 must be float32 ({B}, {H}, {N}, {D}) on {dev}")
    return B, L, H, D, N, Q, dtype


def chunkwise_delta_scan_fwd(q: Tensor, k: Tensor, v: Tensor, beta: Tensor, sel_C: Tensor, dt: Tensor,
                             r: Tensor, alpha: Tensor, omega: Tensor, c: float,
                             h0: Optional[Tensor] = None, chunk_size: Optional[int] = None,
                             train: bool = False) -> Tuple[Tensor, Tensor, Tensor]:
    """Forward only.  Returns (y (B,L,H,2), h_final (B,H,2,D) fp32, carry).

    ``carry`` is the workspace: the complex fp32 state entering every chunk,
    shape (B, NC, H, D, 2), the per-chunk rotation products and, with
    ``train=True`` (cdssm_fused_scan_fwd_train), the per-token dot products the
    backward consumes.
    """
    B, L, H, D, N, Q, dtype = _validate(q, k, v, beta, sel_C, dt, r, alpha, omega, h0, chunk_size)
    lib = _lib.load()
    ins = [t.contiguous() for t in (q, k, v, beta, sel_C, dt, r, alpha, omega)]
    h0c = h0.contiguous() if h0 is not None else None
    dev = q.device
    y = torch.empty(B, L, H, N, dtype=dtype, device=dev)
    h_final = torch.empty(B, H, N, D, dtype=torch.float32, device=dev)
    nbytes = lib.cdssm_fused_scan_workspace_bytes(B, L, H, D, N, Q)
    if nbytes <= 0:
        raise RuntimeError(f"cdssm_fused_scan_workspace_bytes rejected the shape ({nbytes})")
    ws = torch.empty(nbytes // 4, dtype=torch.float32, device=dev)
    fn = lib.cdssm_fused_scan_fwd_train if train else lib.cdssm_fused_scan_fwd
    st = fn(_lib.DTYPE_CODE[dtype], *[_lib.ptr(t) for t in ins[:7]], _lib.ptr(ins[7]), _lib.ptr(ins[8]),
            float(c), _lib.ptr(h0c), _lib.ptr(y), _lib.ptr(h_final), _lib.ptr(ws), B, L, H, D, N, Q,
            _lib.stream_of(dev))
    _lib.check(st, "cdssm_fused_scan_fwd_train" if train else "cdssm_fused_scan_fwd")
    return y, h_final, ws


def _abar_validate(q, k, v, beta, sel_C, A_bar, vp, h0, chunk_size):
    if not isinstance(A_bar, torch.Tensor) or not isinstance(vp, torch.Tensor):
        raise TypeError("A_bar and vp must be tensors")
    B, L, H, D = q.shape
    N = v.shape[-1] if v.dim() == 4 else 2
    if tuple(A_bar.shape) != (B, L, H, N) or tuple(vp.shape) != (B, L, H, max(N // 2, 1)):
        raise ValueError(f"A_bar must be ({B}, {L}, {H}, {N}) and vp ({B}, {L}, {H}, {max(N // 2, 1)}), got "
                         f"{tuple(A_bar.shape)} and {tuple(vp.shape)}")
    if A_bar.dtype != q.dtype or vp.dtype != q.dtype or A_bar.device != q.device or vp.device != q.device:
        raise TypeError("A_bar and vp must have q's dtype and device")
    # shape/dtype checks of the other inputs (A_bar and vp stand in for dt and r there)
    ones = torch.empty(H, dtype=torch.float32, device=q.device)
    return _validate(q, k, v, beta, sel_C, beta, beta, ones, ones, h0, chunk_size, rows=True)


def chunkwise_delta_scan_abar_fwd(q: Tensor, k: Tensor, v: Tensor, beta: Tensor, sel_C: Tensor, A_bar: Tensor,
                                  vp: Tensor, h0: Optional[Tensor] = None, chunk_size: Optional[int] = None,
                                  train: bool = False) -> Tuple[Tensor, Tensor, Tensor]:
    """The fused scan on gate-level inputs: (y, h_final, workspace).  ``train=True``
    (cdssm_fused_scan_fwd_abar_train) keeps in the workspace what
    ``chunkwise_delta_scan_abar_bwd`` reads."""
    B, L, H, D, N, Q, dtype = _abar_validate(q, k, v, beta, sel_C, A_bar, vp, h0, chunk_size)
    lib = _lib.load()
    ins = [t.contiguous() for t in (q, k, v, beta, sel_C, A_bar, vp)]
    h0c = h0.contiguous() if h0 is not None else None
    y = torch.empty(B, L, H, N, dtype=dtype, device=q.device)
    h_final = torch.empty(B, H, N, D, dtype=torch.float32, device=q.device)
    nbytes = lib.cdssm_fused_scan_workspace_bytes(B, L, H, D, N, Q)
    if nbytes <= 0:
        raise RuntimeError(f"cdssm_fused_scan_workspace_bytes rejected the shape ({nbytes})")
    ws = torch.empty(nbytes // 4, dtype=torch.float32, device=q.device)
    name = "cdssm_fused_scan_fwd_abar_train" if train else "cdssm_fused_scan_fwd_abar"
    st = getattr(lib, name)(_lib.DTYPE_CODE[dtype], *[_lib.ptr(t) for t in ins], _lib.ptr(h0c), _lib.ptr(y),
                            _lib.ptr(h_final), _lib.ptr(ws), B, L, H, D, N, Q, _lib.stream_of(q.device))
    _lib.check(st, name)
    return y, h_final, ws


def chunkwise_delta_scan_abar(q: Tensor, k: Tensor, v: Tensor, beta: Tensor, sel_C: Tensor, A_bar: Tensor,
                              vp: Tensor, h0: Optional[Tensor] = None,
                              chunk_size: Optional[int] = None) -> Tuple[Tensor, Tensor]:
    """The fused scan on gate-level inputs (cdssm_fused_scan_fwd_abar), inference.

    ``A_bar`` (B,L,H,N) and ``vp`` (B,L,H,N/2) are DynamicsFusedFn's outputs (N even, 2 to 32); the
    result is ``sel_C * einsum('blhsd,blhd->blhs', SSDChunkwiseScan(Q, N)(A_bar, k,
    v * vp.repeat_interleave(2, -1), beta), q)`` (B,L,H,N) (block.py:194-211 without the shortcut) and the
    final R-mode state (B,H,N,D) fp32.  For N > 2 the head's N / 2 complex state rows, which share k, q,
    beta and sel_C, run as virtual heads of the sequential scan.  ``ChunkwiseDeltaScanAbarFn`` is the
    differentiable form.
    """
    y, h_final, _ = chunkwise_delta_scan_abar_fwd(q, k, v, beta, sel_C, A_bar, vp, h0, chunk_size)
    return y, h_final


def chunked_scan_abar(q: Tensor, k: Tensor, v: Tensor, beta: Tensor, sel_C: Tensor, A_bar: Tensor, vp: Tensor,
                      h0: Optional[Tensor] = None, chunk_size: Optional[int] = None,
                      shortcut_scale: Optional[Tensor] = None) -> Tuple[Tensor, Tensor]:
    """The gate-level readout form for state_dim N = 16 in the chunked (UT) form on the matrix cores
    (cdssm_chunked_scan_fwd_abar), inference, bf16: ``(y, h_final)`` with
    ``y = sel_C * einsum('blhsd,blhd->blhs', SSDChunkwiseScan(Q, 16)(A_bar, k, v * vp.repeat_interleave(2, -1),
    beta), q)`` (B,L,H,16) (block.py:194-211 without the shortcut) and the final R-mode state (B,H,16,D) fp32,
    without forming Y.  ``A_bar`` (B,L,H,16) and ``vp`` (B,L,H,8) are DynamicsFusedFn's outputs; q, k (B,L,H,D)
    with D in {64, 128}; chunk_size (default D) a multiple of 16 up to 256.  With ``shortcut_scale`` (a
    one-element fp32 tensor on the device) y also carries the current-token shortcut
    ``sel_C * shortcut_scale * (q.k)^2 * v * vp`` (block.py:202-208): the block's retrieved vector."""
    named = dict(q=q, k=k, v=v, beta=beta, sel_C=sel_C, A_bar=A_bar, vp=vp)
    for n, t in named.items():
        if not isinstance(t, torch.Tensor):
            raise TypeError(f"{n} must be a tensor")
    dev = q.device
    if dev.type != "cuda":
        raise RuntimeError("chunked_scan_abar runs on the GPU only: inputs must be on a cuda device")
    if q.dim() != 4:
        raise ValueError(f"q must be (B, L, H, D), got {tuple(q.shape)}")
    B, L, H, D = q.shape
    N = v.shape[-1] if v.dim() == 4 else -1
    shapes = dict(q=(B, L, H, D), k=(B, L, H, D), v=(B, L, H, N), beta=(B, L, H), sel_C=(B, L, H),
                  A_bar=(B, L, H, N), vp=(B, L, H, N // 2))
    for n, shp in shapes.items():
        t = named[n]
        if tuple(t.shape) != shp:
            raise ValueError(f"{n} has shape {tuple(t.shape)}, expected {shp}")
        if t.dtype != torch.bfloat16 or t.device != dev:
            raise TypeError(f"{n} must be bfloat16 on {dev} (the chunked form takes bf16), got {t.dtype} {t.device}")
    Q = D if chunk_size is None else int(chunk_size)
    lib = _lib.load()
    nbytes = lib.cdssm_chunked_scan_workspace_bytes(B, L, H, D, N, Q)
    if nbytes <= 0:
        raise ValueError(f"the chunked form needs N = 16, D in (64, 128) and chunk_size a multiple of 16 in "
                         f"[16, 256] (N={N} D={D} chunk_size={Q})")
    if h0 is not None and (h0.dtype != torch.float32 or tuple(h0.shape) != (B, H, N, D) or h0.device != dev):
        raise ValueError(f"h0 must be float32 ({B}, {H}, {N}, {D}) on {dev}")
    ins = [t.contiguous() for t in (q, k, v, beta, sel_C, A_bar, vp)]
    h0c = h0.contiguous() if h0 is not None else None
    sc = None
    if shortcut_scale is not None:
        sc = shortcut_scale.detach().reshape(1).to(device=dev, dtype=torch.float32).contiguous()
    y = torch.empty(B, L, H, N, dtype=q.dtype, device=dev)
    h_final = torch.empty(B, H, N, D, dtype=torch.float32, device=dev)
    ws = torch.empty(nbytes // 4, dtype=torch.float32, device=dev)
    st = lib.cdssm_chunked_scan_fwd_abar(_lib.DTYPE_CODE[q.dtype], *[_lib.ptr(t) for t in ins], _lib.ptr(h0c),
                                         _lib.ptr(sc), _lib.ptr(y), _lib.ptr(h_final), _lib.ptr(ws), B, L, H, D, N, Q,
                                         _lib.stream_of(dev))
    _lib.check(st, "cdssm_chunked_scan_fwd_abar")
    return y, h_final


def chunkwise_delta_scan_abar_bwd(dy: Tensor, dh_final: Optional[Tensor], q, k, v, beta, sel_C, A_bar, vp,
                                  fwd_ws: Tensor, has_h0: bool, chunk_size: int):
    """Backward of ``chunkwise_delta_scan_abar_fwd(..., train=True)`` (cdssm_fused_scan_bwd_abar):
    (dq, dk, dv, dbeta, dsel_C, dA_bar, dvp, dh0), dh0 None without an initial state."""
    B, L, H, D = q.shape
    N = v.shape[-1]
    Q = int(chunk_size)
    lib = _lib.load()
    dev = q.device
    dy = dy.to(q.dtype).contiguous()
    dhf = None if dh_final is None else dh_final.float().contiguous()
    outs = [torch.empty_like(t) for t in (q, k, v, beta, sel_C, A_bar, vp)]
    dh0 = torch.empty(B, H, N, D, dtype=torch.float32, device=dev) if has_h0 else None
    nbytes = lib.cdssm_fused_scan_bwd_workspace_bytes(B, L, H, D, N, Q)
    if nbytes <= 0:
        raise RuntimeError(f"cdssm_fused_scan_bwd_workspace_bytes rejected the shape ({nbytes})")
    ws = torch.empty(nbytes // 4, dtype=torch.float32, device=dev)
    st = lib.cdssm_fused_scan_bwd_abar(_lib.DTYPE_CODE[q.dtype], *[_lib.ptr(t) for t in (q, k, v, beta, sel_C, A_bar, vp)],
                                       _lib.ptr(dy), _lib.ptr(dhf), _lib.ptr(fwd_ws), *[_lib.ptr(t) for t in outs],
                                       _lib.ptr(dh0), _lib.ptr(ws), B, L, H, D, N, Q, _lib.stream_of(dev))
    _lib.check(st, "cdssm_fused_scan_bwd_abar")
    return (*outs, dh0)


class ChunkwiseDeltaScanAbarFn(torch.autograd.Function):
    """Autograd Function of the fused scan on gate-level inputs: (q, k, v, beta, sel_C, A_bar, vp, h0,
    chunk_size) -> (y, h_final), y = sel_C (Y . q) of SSDChunkwiseScan(A_bar, k, v * vp, beta)
    (block.py:194-211 without the shortcut), for any even state_dim N up to 32 (vp (B,L,H,N/2) per
    complex state row).  The training step through the block (trainer.py:235-247) without the
    (B,L,H,N,D) Y: the forward keeps only the training records in its workspace, the backward rebuilds
    chunk states from them and returns the reference's gradients (exact for the readout, the local and
    carry branches; the correction branch's shifted rule); with N > 2 the gradients of the per-head
    k, q, beta and sel_C are summed over the head's state rows in a fixed order."""

    @staticmethod
    def forward(ctx, q, k, v, beta, sel_C, A_bar, vp, h0=None, chunk_size=None):
        _, _, _, _, _, Q, _ = _abar_validate(q, k, v, beta, sel_C, A_bar, vp, h0, chunk_size)
        ins = [t.contiguous() for t in (q, k, v, beta, sel_C, A_bar, vp)]
        y, h_final, ws = chunkwise_delta_scan_abar_fwd(*ins, h0, Q, train=True)
        ctx.save_for_backward(*ins, ws)
        ctx.Q = Q
        ctx.has_h0 = h0 is not None
        return y, h_final

    @staticmethod
    def backward(ctx, dy, dh_final):
        *ins, ws = ctx.saved_tensors
        if dy is None:
            dy = torch.zeros_like(ins[2])
        dq, dk, dv, dbeta, dsel, dA, dvp, dh0 = chunkwise_delta_scan_abar_bwd(dy, dh_final, *ins, ws, ctx.has_h0,
                                                                              ctx.Q)
        return dq, dk, dv, dbeta, dsel, dA, dvp, dh0, None


FORWARD_PATHS = {"auto": 0, "four_launch": 1, "one_pass": 2, "four_launch_mfma": 3}

# Bumped by every set_forward_path call.  A prepared call continues on the
# look-back epoch its previous call left only while the path setting is the one
# that call ran under: a call made under another setting may have taken the
# multi-launch passes, which never write the workspace's control block.
_path_generation = [0]


def set_forward_path(path: str) -> str:
    """Select how the inference forward is launched; returns the previous setting.

    "auto" (default) takes the one-pass forward where one round of resident
    workgroups holds every segment of 4 chunks (and, for inference, where the
    persistent one-pass fills whole rounds), else the four-launch scan;
    "four_launch" always takes the multi-launch passes; "one_pass" requires
    the one-launch passes (calls they cannot serve raise); "four_launch_mfma"
    takes the multi-launch passes with the correction as the chunked MFMA
    pass (bf16 inference forward, chunk a multiple of 16 up to 128; other calls
    raise).  Process-wide; the same choice applies to the backward's correction
    adjoint + reverse carry.
    """
    if path not in FORWARD_PATHS:
        raise ValueError(f"path must be one of {sorted(FORWARD_PATHS)}, got {path!r}")
    prev = _lib.load().cdssm_fused_scan_fwd_set_path(FORWARD_PATHS[path])
    if prev < 0:
        _lib.check(prev, "cdssm_fused_scan_fwd_set_path")
    _path_generation[0] += 1
    return {v: n for n, v in FORWARD_PATHS.items()}[prev]


LOOKBACK_BITS = {1: "forward one-pass", 2: "backward correction adjoint + carry"}


def lookback_status(clear: bool = True) -> int:
    """Sticky look-back status of the current device (cdssm_lookback_status).

    0 means no look-back wait of a one-launch pass has timed out since the last
    clear; bit 0 (1) marks the forward, bit 1 (2) the backward.  A timed-out
    wait writes NaN states, so the affected outputs are NaN as well.
    Synchronises with the device; do not call it while capturing a graph.
    """
    out = ctypes.c_int(0)
    st = _lib.load().cdssm_lookback_status(1 if clear else 0, ctypes.byref(out))
    _lib.check(st, "cdssm_lookback_status")
    return int(out.value)


def check_lookback(clear: bool = True) -> None:
    """Raise RuntimeError if a look-back wait of a one-launch pass has timed out."""
    bits = lookback_status(clear)
    if bits:
        which = ", ".join(n for b, n in LOOKBACK_BITS.items() if bits & b)
        raise RuntimeError(f"look-back wait timed out in the {which} (status {bits}): the workgroups of a "
                           f"one-launch pass were not all resident at once; the affected outputs are NaN")


def chunkwise_delta_scan(q, k, v, beta, sel_C, dt, r, alpha, omega, c, h0=None, chunk_size=None):
    """y (B,L,H,2) and the final R-mode state (B,H,2,D) of the fused scan."""
    y, h_final, _ = chunkwise_delta_scan_fwd(q, k, v, beta, sel_C, dt, r, alpha, omega, c, h0, chunk_size)
    return y, h_final


class PreparedForward:
    """A forward scan with inputs, outputs and workspace bound once.

    Calling it re-launches the scan's kernels on torch's current stream with no
    validation, allocation or tensor creation on the host: the launch path for
    serving loops, graph capture and timing.  The bound tensors must stay alive
    and keep their shapes.  The first call draws the one-launch pass's look-back
    epoch with a kernel of its own (cdssm_fused_scan_fwd); later calls reuse
    the epoch the previous call left in the workspace it owns
    (cdssm_fused_scan_fwd_continue): one launch per call.
    """

    def __init__(self, q, k, v, beta, sel_C, dt, r, alpha, omega, c, h0=None, chunk_size=None,
                 train: bool = False):
        B, L, H, D, N, Q, dtype = _validate(q, k, v, beta, sel_C, dt, r, alpha, omega, h0, chunk_size)
        self.train = bool(train)
        for n, t in dict(q=q, k=k, v=v, beta=beta, sel_C=sel_C, dt=dt, r=r, alpha=alpha, omega=omega).items():
            if not t.is_contiguous():
                raise ValueError(f"{n} must be contiguous for a prepared scan")
        if h0 is not None and not h0.is_contiguous():
            raise ValueError("h0 must be contiguous for a prepared scan")
        self._lib = _lib.load()
        dev = q.device
        self.inputs = (q, k, v, beta, sel_C, dt, r, alpha, omega, h0)
        self.y = torch.empty(B, L, H, N, dtype=dtype, device=dev)
        self.h_final = torch.empty(B, H, N, D, dtype=torch.float32, device=dev)
        nbytes = self._lib.cdssm_fused_scan_workspace_bytes(B, L, H, D, N, Q)
        self.workspace = torch.empty(nbytes // 4, dtype=torch.float32, device=dev)
        self.shape = (B, L, H, D, N, Q)
        self.device = dev
        self._args = (_lib.DTYPE_CODE[dtype], *[_lib.ptr(t) for t in self.inputs[:9]], float(c),
                      _lib.ptr(h0), _lib.ptr(self.y), _lib.ptr(self.h_final), _lib.ptr(self.workspace),
                      B, L, H, D, N, Q)
        self._continue = False  # the workspace holds a previous forward call's look-back area
        self._gen = -1  # the path setting that call ran under

    def __call__(self):
        lib = self._lib
        gen = _path_generation[0]
        cont = self._continue and self._gen == gen
        if cont:
            fn = lib.cdssm_fused_scan_fwd_train_continue if self.train else lib.cdssm_fused_scan_fwd_continue
        else:
            fn = lib.cdssm_fused_scan_fwd_train if self.train else lib.cdssm_fused_scan_fwd
        st = fn(*self._args, _lib.stream_of(self.device))
        if st != 0:
            _lib.check(st, "cdssm_fused_scan_fwd")
        # a captured call does not run now: the workspace holds no call until one executes
        self._continue = cont or not torch.cuda.is_current_stream_capturing()
        self._gen = gen
        return self.y, self.h_final

    PHASES = ("summary", "carry_fold", "carry_replay", "main")
    STAMP_POINTS = ("entry", "staged", "local", "published", "waited", "folded", "corrected", "end")

    def phase_stamps(self) -> Tensor:
        """One inference forward (cdssm_fused_scan_fwd_stamped, instrumentation) recording,
        per wave of the one-pass kernel, the 100 MHz real-time counter at the points
        STAMP_POINTS of its segment.  Returns an int64 (waves, 8) CPU tensor in ticks
        (rows of unwritten records dropped); raises if the shape takes the four-launch
        forward."""
        B, L, H, D, N, Q = self.shape
        nseg = -(-(-(-L // Q)) // 4)
        n_items = nseg * B * H  # an upper bound on segment items (head groups <= H)
        buf = torch.zeros(n_items * 4 * 8, dtype=torch.int64, device=self.device)
        st = self._lib.cdssm_fused_scan_fwd_stamped(*self._args, _lib.ptr(buf), buf.numel(),
                                                    _lib.stream_of(self.device))
        if st != 0:
            _lib.check(st, "cdssm_fused_scan_fwd_stamped")
        out = buf.view(-1, 8).cpu()
        return out[out[:, 0] != 0]

    def profile(self, iters: int) -> dict:
        """Average milliseconds of each kernel launch over `iters` calls, from HIP
        events recorded on the launch stream between the launches.  A call that
        takes the one-pass kernel reports it as "main" and 0 for the others."""
        out = (ctypes.c_float * len(self.PHASES))()
        st = self._lib.cdssm_fused_scan_fwd_profile(*self._args, _lib.stream_of(self.device), int(self.train),
                                                    int(iters), out)
        if st != 0:
            _lib.check(st, "cdssm_fused_scan_fwd_profile")
        return dict(zip(self.PHASES, list(out)))


def chunkwise_delta_scan_bwd(dy: Tensor, dh_final: Optional[Tensor], q, k, v, beta, sel_C, dt, r,
                             alpha, omega, c, carry: Tensor, has_h0: bool, chunk_size: int):
    """Backward of the fused scan (cdssm_fused_scan_bwd), reference-mode gradients.

    Returns (dq, dk, dv, dbeta, dsel_C, ddt, dr, dalpha, domega, dh0); dh0 is
    None when the forward had no initial state.
    """
    B, L, H, D = q.shape
    N = v.shape[-1]
    Q = int(chunk_size)
    lib = _lib.load()
    dev = q.device
    dtype = q.dtype
    dy = dy.to(dtype).contiguous()
    dhf = None if dh_final is None else dh_final.float().contiguous()
    outs = [torch.empty_like(t) for t in (q, k, v, beta, sel_C, dt, r)]
    dalpha = torch.empty(H, dtype=torch.float32, device=dev)
    domega = torch.empty(H, dtype=torch.float32, device=dev)
    dh0 = torch.empty(B, H, N, D, dtype=torch.float32, device=dev) if has_h0 else None
    nbytes = lib.cdssm_fused_scan_bwd_workspace_bytes(B, L, H, D, N, Q)
    if nbytes <= 0:
        raise RuntimeError(f"cdssm_fused_scan_bwd_workspace_bytes rejected the shape ({nbytes})")
    ws = torch.empty(nbytes // 4, dtype=torch.float32, device=dev)
    st = lib.cdssm_fused_scan_bwd(_lib.DTYPE_CODE[dtype], *[_lib.ptr(t) for t in (q, k, v, beta, sel_C, dt, r)],
                                  _lib.ptr(alpha), _lib.ptr(omega), float(c), _lib.ptr(dy), _lib.ptr(dhf),
                                  _lib.ptr(carry), *[_lib.ptr(t) for t in outs], _lib.ptr(dalpha),
                                  _lib.ptr(domega), _lib.ptr(dh0), _lib.ptr(ws), B, L, H, D, N, Q,
                                  _lib.stream_of(dev))
    _lib.check(st, "cdssm_fused_scan_bwd")
    return (*outs, dalpha, domega, dh0)


class ChunkwiseDeltaScanFn(torch.autograd.Function):
    """Autograd Function of the fused scan: (q, k, v, beta, sel_C, dt, r, alpha,
    omega, c, h0, chunk_size) -> (y, h_final).

    Saves the inputs and the per-chunk entering states (no per-step state);
    the backward recomputes chunk-local states and returns the gradients that
    the reference ops.py path yields (exact for the readout, the intra-chunk
    and inter-chunk passes; the reference's shifted gradient for the exact
    correction pass, exact_correction.cu:213-382).
    """

    @staticmethod
    def forward(ctx, q, k, v, beta, sel_C, dt, r, alpha, omega, c, h0=None, chunk_size=None):
        B, L, H, D, N, Q, _ = _validate(q, k, v, beta, sel_C, dt, r, alpha, omega, h0, chunk_size)
        ins = [t.contiguous() for t in (q, k, v, beta, sel_C, dt, r, alpha, omega)]
        y, h_final, ws = chunkwise_delta_scan_fwd(*ins, c, h0, Q, train=True)
        ctx.save_for_backward(*ins, ws)
        ctx.c = float(c)
        ctx.Q = Q
        ctx.has_h0 = h0 is not None
        return y, h_final

    @staticmethod
    def backward(ctx, dy, dh_final):
        *ins, ws = ctx.saved_tensors
        g = chunkwise_delta_scan_bwd(dy, dh_final, *ins, ctx.c, ws, ctx.has_h0, ctx.Q)
        dq, dk, dv, dbeta, dsel, ddt, dr, dalpha, domega, dh0 = g
        return dq, dk, dv, dbeta, dsel, ddt, dr, dalpha, domega, None, dh0, None


def chunkwise_delta_scan_train(q, k, v, beta, sel_C, dt, r, alpha, omega, c, h0=None, chunk_size=None):
    """Differentiable fused scan: (y, h_final) with gradients for every tensor input."""
    return ChunkwiseDeltaScanFn.apply(q, k, v, beta, sel_C, dt, r, alpha, omega, c, h0, chunk_size)


def _validate_ssd(A_bar, K, V, beta, chunk_size):
    named = dict(A_bar=A_bar, K=K, V=V, beta=beta)
    for n, t in named.items():
        if not isinstance(t, torch.Tensor):
            raise TypeError(f"{n} must be a tensor")
    dev = K.device
    if dev.type != "cuda":
        raise RuntimeError("the fused SSD scan runs on the GPU only: inputs must be on a cuda device")
    if K.dim() != 4:
        raise ValueError(f"K must be (B, L, H, D), got {tuple(K.shape)}")
    B, L, H, D = K.shape
    N = V.shape[-1] if V.dim() == 4 else -1
    shapes = dict(A_bar=(B, L, H, N), V=(B, L, H, N), beta=(B, L, H))
    for n, shp in shapes.items():
        if tuple(named[n].shape) != shp:
            raise ValueError(f"{n} has shape {tuple(named[n].shape)}, expected {shp}")
    dtype = K.dtype
    if dtype not in _lib.DTYPE_CODE:
        raise TypeError(f"inputs must be float32 or bfloat16, got {dtype}")
    for n, t in named.items():
        if t.dtype != dtype or t.device != dev:
            raise TypeError(f"{n} is {t.dtype} on {t.device}, expected {dtype} on {dev} (as K)")
    if N < 2 or N > 32 or N % 2:
        raise ValueError(f"the fused SSD scan supports even state_dim 2 <= N <= 32, got N = {N}")
    if D not in (64, 128):
        raise ValueError(f"head_dim D must be 64 or 128, got {D}")
    Q = int(chunk_size)
    if not 1 <= Q <= 128:
        raise ValueError(f"chunk_size must be in [1, 128], got {Q}")
    return B, L, H, D, N, Q, dtype


def ssd_scan_fwd(A_bar: Tensor, K: Tensor, V: Tensor, beta: Tensor, chunk_size: int,
                 train: bool = False) -> Tuple[Tensor, Tensor, Tensor]:
    """The SSDChunkwiseScan interface on the fused kernels (cdssm_ssd_scan_fwd).

    A_bar (B,L,H,N), K (B,L,H,D), V (B,L,H,N) (already VP-scaled), beta (B,L,H), one dtype, N even
    (N / 2 complex state rows per head, each scanned as a virtual head that shares the head's k and
    beta).  Returns (Y (B,L,H,N,D) of that dtype = local state + correction per token
    (ssd.py:39-111), h_final (B,H,N,D) fp32, the workspace); ``train=True`` keeps in the workspace
    what ``ssd_scan_bwd`` reads.
    """
    B, L, H, D, N, Q, dtype = _validate_ssd(A_bar, K, V, beta, chunk_size)
    lib = _lib.load()
    ins = [t.contiguous() for t in (A_bar, K, V, beta)]
    dev = K.device
    Y = torch.empty(B, L, H, N, D, dtype=dtype, device=dev)
    h_final = torch.empty(B, H, N, D, dtype=torch.float32, device=dev)
    nbytes = lib.cdssm_ssd_scan_workspace_bytes(B, L, H, D, N, Q)
    if nbytes <= 0:
        raise RuntimeError(f"cdssm_ssd_scan_workspace_bytes rejected the shape ({nbytes})")
    ws = torch.empty(nbytes // 4, dtype=torch.float32, device=dev)
    st = lib.cdssm_ssd_scan_fwd(_lib.DTYPE_CODE[dtype], *[_lib.ptr(t) for t in ins], _lib.ptr(Y), _lib.ptr(h_final),
                                _lib.ptr(ws), B, L, H, D, N, Q, 1 if train else 0, _lib.stream_of(dev))
    _lib.check(st, "cdssm_ssd_scan_fwd")
    return Y, h_final, ws


def ssd_scan_bwd(dY: Tensor, A_bar: Tensor, K: Tensor, V: Tensor, beta: Tensor, fwd_ws: Tensor,
                 chunk_size: int) -> Tuple[Tensor, Tensor, Tensor, Tensor]:
    """Backward of ``ssd_scan_fwd(..., train=True)`` (cdssm_ssd_scan_bwd): (dA_bar, dK, dV, dbeta)
    with the reference's rules (exact local and carry branches, the correction branch's shifted
    gradient, exact_correction.cu:213-382)."""
    B, L, H, D = K.shape
    N = V.shape[-1]
    Q = int(chunk_size)
    lib = _lib.load()
    dev = K.device
    dY = dY.to(K.dtype).contiguous()
    if tuple(dY.shape) != (B, L, H, N, D):
        raise ValueError(f"dY must be ({B}, {L}, {H}, {N}, {D}), got {tuple(dY.shape)}")
    outs = [torch.empty_like(t) for t in (A_bar, K, V, beta)]
    nbytes = lib.cdssm_ssd_scan_bwd_workspace_bytes(B, L, H, D, N, Q)
    if nbytes <= 0:
        raise RuntimeError(f"cdssm_ssd_scan_bwd_workspace_bytes rejected the shape ({nbytes})")
    ws = torch.empty(nbytes // 4, dtype=torch.float32, device=dev)
    st = lib.cdssm_ssd_scan_bwd(_lib.DTYPE_CODE[K.dtype], *[_lib.ptr(t) for t in (A_bar, K, V, beta)], _lib.ptr(dY),
                                _lib.ptr(fwd_ws), *[_lib.ptr(t) for t in outs], _lib.ptr(ws), B, L, H, D, N, Q,
                                _lib.stream_of(dev))
    _lib.check(st, "cdssm_ssd_scan_bwd")
    return tuple(outs)


class SSDScanFn(torch.autograd.Function):
    """Autograd Function of the fused SSD scan: (A_bar, K, V, beta, chunk_size) -> Y (B,L,H,N,D).

    The same result and gradients as SSDChunkwiseScan over IntraChunkScanFn, InterChunkScanFn and
    ExactCorrectionFn (ssd.py:39-111, ops.py:100-195), from one forward and one backward call.
    Saves the inputs and the training forward's workspace (per-token records, the local state every
    8 tokens, the state entering and the correction leaving every chunk), no per-token states.
    """

    @staticmethod
    def forward(ctx, A_bar, K, V, beta, chunk_size):
        _validate_ssd(A_bar, K, V, beta, chunk_size)
        ins = [t.contiguous() for t in (A_bar, K, V, beta)]
        train = any(t.requires_grad for t in (A_bar, K, V, beta))
        Y, _, ws = ssd_scan_fwd(*ins, chunk_size, train=train)
        if train:
            ctx.save_for_backward(*ins, ws)
        ctx.Q = int(chunk_size)
        return Y

    @staticmethod
    def backward(ctx, dY):
        A_bar, K, V, beta, ws = ctx.saved_tensors
        dA, dK, dV, dbeta = ssd_scan_bwd(dY, A_bar, K, V, beta, ws, ctx.Q)
        return dA, dK, dV, dbeta, None


class PreparedBackward:
    """The fused backward bound to a PreparedForward's inputs and workspace.

    Gradient buffers and the backward workspace are allocated once; each call
    re-launches the backward kernels for the bound cotangents on torch's
    current stream.  Call the forward first: the backward reads the entering
    states the forward left in its workspace.  As PreparedForward, calls after
    the first reuse the look-back epoch the previous call left in the backward
    workspace (cdssm_fused_scan_bwd_continue).
    """

    def __init__(self, fwd: PreparedForward, dy: Tensor, dh_final: Optional[Tensor] = None, c: float = None):
        if not fwd.train:
            raise ValueError("PreparedBackward needs a PreparedForward(..., train=True): the backward reads the "
                             "per-token records the training forward keeps")
        q, k, v, beta, sel_C, dt, r, alpha, omega, h0 = fwd.inputs
        B, L, H, D, N, Q = fwd.shape
        self._lib = fwd._lib
        dev = fwd.device
        self.dy = dy.to(q.dtype).contiguous()
        self.dh_final = None if dh_final is None else dh_final.float().contiguous()
        self.grads = [torch.empty_like(t) for t in (q, k, v, beta, sel_C, dt, r)]
        self.dalpha = torch.empty(H, dtype=torch.float32, device=dev)
        self.domega = torch.empty(H, dtype=torch.float32, device=dev)
        self.dh0 = torch.empty(B, H, N, D, dtype=torch.float32, device=dev) if h0 is not None else None
        nbytes = self._lib.cdssm_fused_scan_bwd_workspace_bytes(B, L, H, D, N, Q)
        self.workspace = torch.empty(nbytes // 4, dtype=torch.float32, device=dev)
        self.device = dev
        cval = fwd._args[10] if c is None else float(c)
        self._args = (_lib.DTYPE_CODE[q.dtype], *[_lib.ptr(t) for t in (q, k, v, beta, sel_C, dt, r)],
                      _lib.ptr(alpha), _lib.ptr(omega), cval, _lib.ptr(self.dy), _lib.ptr(self.dh_final),
                      _lib.ptr(fwd.workspace), *[_lib.ptr(t) for t in self.grads], _lib.ptr(self.dalpha),
                      _lib.ptr(self.domega), _lib.ptr(self.dh0), _lib.ptr(self.workspace), B, L, H, D, N, Q)
        self._continue = False
        self._gen = -1
        self.shape = fwd.shape

    def __call__(self):
        gen = _path_generation[0]
        cont = self._continue and self._gen == gen
        fn = self._lib.cdssm_fused_scan_bwd_continue if cont else self._lib.cdssm_fused_scan_bwd
        st = fn(*self._args, _lib.stream_of(self.device))
        if st != 0:
            _lib.check(st, "cdssm_fused_scan_bwd")
        self._continue = cont or not torch.cuda.is_current_stream_capturing()
        self._gen = gen
        return self.grads

    PHASES = ("corr_adjoint", "rcarry_fold", "rcarry_replay", "main", "heads")
    CORR_STAMP_POINTS = ("entry", "staged", "lambda", "published", "waited", "folded", "left_end", "end")
    MAIN_STAMP_POINTS = ("entry", "staged", "reverse", "end")

    def phase_stamps(self) -> Tuple[Tensor, Tensor]:
        """One backward (cdssm_fused_scan_bwd_stamped, instrumentation) recording the 100 MHz real-time
        counter per wave at CORR_STAMP_POINTS of the one-launch correction adjoint + carry and at
        MAIN_STAMP_POINTS of the main pass.  Returns two int64 CPU tensors in ticks, (waves, 8) and
        (waves, 4), rows of unwritten records dropped; raises if the shape runs the three-launch
        correction adjoint."""
        B, L, H, D, N, Q = self.shape
        nc = -(-L // Q)
        nseg = -(-nc // 4)
        m = nseg * B * H * 32
        buf = torch.zeros(m + B * nc * H * 4, dtype=torch.int64, device=self.device)
        st = self._lib.cdssm_fused_scan_bwd_stamped(*self._args, _lib.ptr(buf), buf.numel(),
                                                    _lib.stream_of(self.device))
        if st != 0:
            _lib.check(st, "cdssm_fused_scan_bwd_stamped")
        out = buf.cpu()
        corr, main = out[:m].view(-1, 8), out[m:].view(-1, 4)
        return corr[corr[:, 0] != 0], main[main[:, 0] != 0]

    def profile(self, iters: int) -> dict:
        """Average milliseconds of each backward kernel launch over `iters` calls."""
        out = (ctypes.c_float * len(self.PHASES))()
        st = self._lib.cdssm_fused_scan_bwd_profile(*self._args, _lib.stream_of(self.device), int(iters), out)
        if st != 0:
            _lib.check(st, "cdssm_fused_scan_bwd_profile")
        return dict(zip(self.PHASES, list(out)))
