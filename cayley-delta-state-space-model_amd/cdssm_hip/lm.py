"""CD-SSM language model forward on the MI355X kernels (the scan's caller).

Mirrors the reference model (model.py:12-51, block.py:14-229, modules.py:14-53,
init.py:13-126, config/model.py:38-178) with the same module and parameter
names, so a reference ``state_dict`` loads unchanged.  Per block:
RMSNorm (HIP) -> in_proj -> value residual -> conv1d+SiLU on the in_proj
column slice (HIP) -> gate_proj -> DynamicsFusedFn (HIP) -> K/Q normalisation
with q.k (HIP) -> fused scan with the sel_C readout on the gate-level A_bar /
vp (HIP, ``cdssm_fused_scan_fwd_abar``) -> current-token shortcut (HIP) ->
readout_proj -> fp32 GroupNorm, * silu(z), + D x (HIP) -> out_proj with the
residual in the GEMM epilogue.  Dense projections and the embedding are
PyTorch (hipBLASLt GEMMs).  With gradients enabled (training) the block takes a
differentiable path instead: conv1d+SiLU, DynamicsFusedFn, NormalizeKQFn and
the fused scan (HIP, with the reference's backward rules: the gate-level
readout form ChunkwiseDeltaScanAbarFn, which never forms the (B,L,H,N,D) Y; for
state_dim N > 2 the head's N/2 complex state rows run as virtual heads sharing
k, q, beta and sel_C) and torch for the rest.  With state_dim 16 (the
reference's default) in bf16 the inference forward runs the scan, readout and
shortcut in the chunked (UT) form on the matrix cores
(``cdssm_chunked_scan_fwd_abar``); other state_dim take the readout form too.
With ``readout_scan`` off the block materialises Y through SSDChunkwiseScan
(the reference's op sequence).

Generation: ``CDSSMLMHeadModel.prefill`` runs the forward over a prompt and keeps
per-layer decode state (conv window, the scan's R-mode state, GroupNorm running
sums, position); ``decode_step`` then advances one token per row without
re-forwarding (the reference re-forwards, predict.py:53-67).
"""

from __future__ import annotations

import math
from dataclasses import dataclass, field
from typing import List, Optional

import torch
import torch.nn as nn

from . import _lib
from .ops import DynamicsFusedFn, NormalizeKQFn
from .decode import DecodeState, decode_step_abar, prefill_abar
from .scan import (ChunkwiseDeltaScanAbarFn, _abar_validate, chunked_scan_abar, chunkwise_delta_scan_abar,
                   chunkwise_delta_scan_abar_bwd, chunkwise_delta_scan_abar_fwd)
from .ssd import SSDChunkwiseScan

Tensor = torch.Tensor

_BF16_EPS = 2.0 ** -7  # torch.finfo(torch.bfloat16).eps


@dataclass
class CDSSMConfig:
    """The reference's config surface and derived constants (config/model.py:38-178).

    ``d_inner`` defaults to the reference's 2 * d_model (config/model.py:57);
    pass it explicitly for other widths (the config-4 workload states
    16 heads x 64 = 1024 = d_model).
    """

    d_model: int = 768
    n_layers: int = 12
    context_length: int = 8192
    vocab_size: int = 50257
    state_dim: int = 16
    d_inner: Optional[int] = None
    head_dim: int = 64
    n_heads: int = field(init=False)
    chunk_size: int = field(init=False)
    ssm_norm_groups: int = field(init=False)
    conv_kernel_size: int = field(init=False)
    rope_base: float = field(init=False)
    gating_c: float = field(init=False)
    spectral_band_fraction: float = field(init=False)
    eps_norm: float = field(init=False)
    eps_log_argument: float = field(init=False)
    eps_adaptive_dt: float = field(init=False)
    init_biases: dict = field(init=False)
    bf16_omega_thresh: float = field(init=False)
    bf16_delta: float = field(init=False)
    bf16_smoothness: float = field(init=False)

    def __post_init__(self):
        if self.state_dim % 2:
            raise ValueError("state_dim must be even (complex pairs)")
        if self.d_inner is None:
            self.d_inner = 2 * self.d_model
        if self.d_inner % self.head_dim:
            raise ValueError("d_inner must be a multiple of head_dim")
        self.n_heads = self.d_inner // self.head_dim
        self.chunk_size = self.head_dim
        self.ssm_norm_groups = 32
        self.conv_kernel_size = max(2, self.head_dim // 16)
        self.rope_base = float(self.context_length)
        self.gating_c = math.log(self.context_length)
        self.spectral_band_fraction = 2.0 / (self.n_layers + 1)
        self.eps_norm = _BF16_EPS ** 2
        self.eps_log_argument = _BF16_EPS ** 2
        self.eps_adaptive_dt = 1.0
        ln2 = math.log(2.0)
        self.init_biases = {"sel_B_bias": ln2, "sel_C_bias": ln2, "r_gate_bias": ln2,
                            "beta_bias": 0.0, "sel_dt_bias": 0.0}
        self.bf16_omega_thresh = math.sqrt(_BF16_EPS)
        self.bf16_delta = 16.0 * _BF16_EPS
        self.bf16_smoothness = self.bf16_omega_thresh / 5.0


def layer_stds(d_model: int, d_inner: int, n_layers: int) -> dict:
    """T-Fixup depth-scaled init stds (init.py:13-41)."""
    depth = 1.0 / math.sqrt(2 * n_layers)
    return {
        "embedding": math.sqrt(1.0 / d_model),
        "in_proj": math.sqrt(2.0 / (d_model + d_inner)) * depth,
        "dynamics_proj": math.sqrt(2.0 / (2 * d_inner)) * depth / math.sqrt(n_layers),
        "out_proj": math.sqrt(2.0 / (d_model + d_inner)) * depth,
    }


def spectral_biases(cfg: CDSSMConfig, layer_idx: int):
    """Per-pair alpha / omega gate biases of a layer (init.py:44-126): log-spaced
    timescales in a band that slides from short to long with depth; alpha = 1/tau
    through an inverse softplus, omega log-spaced between the band's frequencies."""
    H, nh = cfg.n_heads, cfg.state_dim // 2
    lo, hi = 0.0, math.log(float(cfg.context_length))
    width = cfg.spectral_band_fraction * (hi - lo)
    start = lo + layer_idx / max(cfg.n_layers - 1, 1) * (hi - lo - width)
    step = width / max(nh, 1)
    alphas, omegas = [], []
    for j in range(nh):
        j0 = start + j * step / nh
        j1 = j0 + width
        tau = torch.exp(torch.linspace(j0, j1, H))
        a = 1.0 / tau
        alphas.append(torch.log(torch.exp(a) - 1 + cfg.eps_log_argument))
        f_lo = max(1.0 / math.exp(j1), cfg.eps_log_argument)
        f_hi = min(0.5, 1.0 / math.exp(j0))
        omegas.append(torch.exp(torch.linspace(math.log(f_lo), math.log(f_hi), H)))
    return alphas, omegas


class _Conv1dSiLUFn(torch.autograd.Function):
    """CUDAConv1dSiLUOp (ops.py:13-28): forward cdssm_conv1d_silu_fwd_strided, backward cdssm_conv1d_silu_bwd
    (grad_x in x's dtype; grad_weight / grad_bias summed in fp32 and cast to the parameters' dtype, as the
    reference's launcher does)."""

    @staticmethod
    def forward(ctx, x: Tensor, weight: Tensor, bias: Tensor) -> Tensor:
        ctx.save_for_backward(x, weight, bias)
        return conv1d_silu(x, weight, bias)

    @staticmethod
    def backward(ctx, grad_out):
        x, weight, bias = ctx.saved_tensors
        gx, gw, gb = conv1d_silu_bwd(x, weight, bias, grad_out)
        return gx, gw.to(weight.dtype).view_as(weight), gb.to(bias.dtype)


def _check_gpu(op: str, *ts: Tensor) -> torch.dtype:
    dt = ts[0].dtype
    for t in ts:
        if t.device.type != "cuda":
            raise RuntimeError(f"{op} runs on the GPU only")
        if t.dtype != dt:
            raise TypeError(f"{op}: all tensors must share one dtype, got {dt} and {t.dtype}")
    if dt not in _lib.DTYPE_CODE:
        raise TypeError(f"{op}: dtype must be float32 or bfloat16, got {dt}")
    return dt


def _token_stride(x: Tensor, dense: int) -> Optional[int]:
    """Stride (elements) between consecutive tokens b * L + l of a (B, L, ...) view, or None when the B*L
    tokens are not uniformly strided; ``dense`` (the elements of one token) when there is one token."""
    B, L = x.shape[0], x.shape[1]
    if L > 1 and B > 1:
        return x.stride(1) if x.stride(0) == L * x.stride(1) else None
    if L > 1:
        return x.stride(1)
    return x.stride(0) if B > 1 else dense


def _token_view(x: Tensor, width: int) -> int:
    """Token stride (elements) of a (B, L, width) view whose rows are dense; raises otherwise."""
    ts = _token_stride(x, width)
    if x.stride(-1) != 1 or ts is None:
        raise ValueError("expected a (B, L, C) view with dense channels and a uniform token stride")
    return ts


def conv1d_silu(x: Tensor, weight: Tensor, bias: Tensor) -> Tensor:
    """silu(causal depthwise conv1d(x) + bias); x (B, L, C) (dense channels, any token stride, e.g. a
    column slice of a projection output), weight (C, 1, K) or (C, K), bias (C)."""
    _check_gpu("conv1d_silu", x)
    B, L, C = x.shape
    K = weight.shape[-1]
    if weight.numel() != C * K or tuple(bias.shape) != (C,):
        raise ValueError(f"weight must be ({C}, 1, K) and bias ({C},), got {tuple(weight.shape)}, {tuple(bias.shape)}")
    try:
        xs = _token_view(x, C)
    except ValueError:
        x = x.contiguous()
        xs = C
    wc = weight.to(x.dtype).contiguous()
    bc = bias.to(x.dtype).contiguous()
    y = torch.empty((B, L, C), dtype=x.dtype, device=x.device)
    st = _lib.load().cdssm_conv1d_silu_fwd_strided(_lib.DTYPE_CODE[x.dtype], _lib.ptr(x), xs, _lib.ptr(wc),
                                                  _lib.ptr(bc), _lib.ptr(y), B, L, C, K, _lib.stream_of(x.device))
    _lib.check(st, "cdssm_conv1d_silu_fwd_strided")
    return y


def conv1d_silu_bwd(x: Tensor, weight: Tensor, bias: Tensor, grad_out: Tensor) -> tuple:
    """Gradients of conv1d_silu: grad_x (B, L, C) in x's dtype, grad_weight (C, K) and grad_bias (C) fp32
    (conv1d_silu.cu:95-276; deterministic sums)."""
    _check_gpu("conv1d_silu_bwd", x)
    B, L, C = x.shape
    K = weight.shape[-1]
    try:
        xs = _token_view(x, C)
    except ValueError:
        x = x.contiguous()
        xs = C
    go = grad_out.to(x.dtype).contiguous()
    wc = weight.detach().to(x.dtype).contiguous()
    bc = bias.detach().to(x.dtype).contiguous()
    gx = torch.empty((B, L, C), dtype=x.dtype, device=x.device)
    gw = torch.empty((C, K), dtype=torch.float32, device=x.device)
    gb = torch.empty((C,), dtype=torch.float32, device=x.device)
    lib = _lib.load()
    nb = lib.cdssm_conv1d_silu_bwd_workspace_bytes(B, L, C, K)
    if nb < 0:
        raise ValueError(f"conv1d_silu_bwd: invalid shape B={B} L={L} C={C} K={K}")
    ws = torch.empty(max(1, nb // 4), dtype=torch.float32, device=x.device)
    st = lib.cdssm_conv1d_silu_bwd(_lib.DTYPE_CODE[x.dtype], _lib.ptr(x), xs, _lib.ptr(wc), _lib.ptr(bc),
                                   _lib.ptr(go), _lib.ptr(gx), _lib.ptr(gw), _lib.ptr(gb), _lib.ptr(ws), B, L, C, K,
                                   _lib.stream_of(x.device))
    _lib.check(st, "cdssm_conv1d_silu_bwd")
    return gx, gw, gb


def rms_norm(x: Tensor, weight: Tensor, eps: float) -> Tensor:
    """(x * rsqrt(mean(x^2) + eps)).to(x.dtype) * weight over the last dim (modules.py:49-53)."""
    w = weight.to(x.dtype).contiguous()
    _check_gpu("rms_norm", x, w)
    xc = x.contiguous()
    C = x.shape[-1]
    y = torch.empty_like(xc)
    st = _lib.load().cdssm_rms_norm_fwd(_lib.DTYPE_CODE[x.dtype], _lib.ptr(xc), _lib.ptr(w), _lib.ptr(y),
                                       xc.numel() // C, C, float(eps), _lib.stream_of(x.device))
    _lib.check(st, "cdssm_rms_norm_fwd")
    return y


class RMSNormFn(torch.autograd.Function):
    """RMSNorm with gradients on the HIP kernels (modules.py:49-53 under autograd): forward
    ``cdssm_rms_norm_fwd``, backward ``cdssm_rms_norm_bwd`` (dx and the weight's gradient, with the
    reference expression's rounding points; the weight's column sums in a fixed order), in place of
    torch's cast, power, mean, rsqrt and products and their backwards.  ``usable`` says whether a call
    qualifies (C a multiple of 64 16-byte vectors, at most 4 of them per lane)."""

    @staticmethod
    def usable(x: Tensor) -> bool:
        if not (x.is_cuda and x.dtype in _lib.DTYPE_CODE):
            return False
        v = 64 * (16 // x.element_size())
        return x.shape[-1] % v == 0 and x.shape[-1] // v <= 4

    @staticmethod
    def forward(ctx, x, weight, eps):
        xc = x.contiguous()
        w = weight.detach().to(x.dtype).contiguous()
        y = rms_norm(xc, w, eps)
        ctx.save_for_backward(xc, w)
        ctx.meta = (float(eps), weight.dtype)
        return y

    @staticmethod
    def backward(ctx, dout):
        xc, w = ctx.saved_tensors
        eps, wdt = ctx.meta
        C = xc.shape[-1]
        rows = xc.numel() // C
        dout = dout.to(xc.dtype).contiguous()
        lib = _lib.load()
        ws = torch.empty(max(1, lib.cdssm_rms_norm_bwd_workspace_bytes(rows, C) // 4), dtype=torch.float32,
                         device=xc.device)
        dx, dw = torch.empty_like(xc), torch.empty_like(w)
        st = lib.cdssm_rms_norm_bwd(_lib.DTYPE_CODE[xc.dtype], _lib.ptr(xc), _lib.ptr(w), _lib.ptr(dout), _lib.ptr(dx),
                                    _lib.ptr(dw), _lib.ptr(ws), rows, C, eps, _lib.stream_of(xc.device))
        _lib.check(st, "cdssm_rms_norm_bwd")
        return dx, dw.to(wdt), None


def _skinny_ok(x: Tensor, weight: Tensor) -> bool:
    """Whether cdssm_skinny_gemm serves x (M, K) @ weight (N, K)^T: bf16, M <= 64, K % 128 == 0,
    16-byte aligned rows."""
    return (x.dim() == 2 and x.dtype == torch.bfloat16 and weight.dtype == torch.bfloat16 and x.is_cuda
            and 1 <= x.shape[0] <= 64 and x.shape[1] % 128 == 0 and weight.shape[1] == x.shape[1]
            and x.stride(1) == 1 and weight.stride(1) == 1 and x.stride(0) % 8 == 0 and weight.stride(0) % 8 == 0
            and x.data_ptr() % 16 == 0 and weight.data_ptr() % 16 == 0)


def skinny_linear(x: Tensor, weight: Tensor, bias: Optional[Tensor] = None, residual: Optional[Tensor] = None,
                  norm_weight: Optional[Tensor] = None, eps: float = 0.0) -> Tensor:
    """Decode-size linear layer on the skinny GEMM kernel (cdssm_skinny_gemm): x (M, K) bf16, M <= 64,
    -> (M, N) = x' @ weight^T (+ bias) (+ residual), where x' = rms_norm(x, norm_weight, eps) when a
    norm weight is given (the RMSNorm folded into the product: x * norm_weight rounded to bf16 enters
    the matrix cores, the row scale rsqrt(mean(x^2) + eps) is applied to the fp32 result).  Shapes the
    kernel does not serve raise (callers check ``_skinny_ok``)."""
    if not _skinny_ok(x, weight):
        raise ValueError("skinny_linear: needs bf16 x (M <= 64, K % 128 == 0) and weight with aligned rows")
    M, K = x.shape
    N = weight.shape[0]
    b = None if bias is None else bias.to(torch.bfloat16).contiguous()
    r = None if residual is None else residual.to(torch.bfloat16)
    if r is not None and (r.shape != (M, N) or r.stride(1) != 1):
        raise ValueError("skinny_linear: residual must be (M, N) with unit column stride")
    g = None if norm_weight is None else norm_weight.to(torch.bfloat16).contiguous()
    y = torch.empty(M, N, dtype=torch.bfloat16, device=x.device)
    st = _lib.load().cdssm_skinny_gemm(1, _lib.ptr(x), x.stride(0), _lib.ptr(weight), weight.stride(0), _lib.ptr(b),
                                       _lib.ptr(r), r.stride(0) if r is not None else 0, _lib.ptr(g), float(eps),
                                       _lib.ptr(y), N, M, N, K, _lib.stream_of(x.device))
    _lib.check(st, "cdssm_skinny_gemm")
    return y


def _wgrad_slabs(T: int, O: int, I: int) -> int:
    """Token slabs of a weight gradient dW = dY^T X over T tokens (O x I output).  One GEMM with an O x I
    output of at most 1024 x 1024 and T = 16384 leaves most CUs idle (hipBLASLt: 64 x 64 tiles, no split
    over the reduction; 0.1-0.3 PFLOP/s on MI355X); 8 slabs as one batched product with fp32 partials ran
    2-3x faster there (out_proj / Q_proj 100-111 -> 39 us, readout_proj 91 -> 23, gate_proj 98 -> 29 us
    before the slab sum); in_proj's 3328 x 1024 takes 2 slabs (185 -> 141 us before the sum)."""
    if T < 8192 or T % 8:
        return 1
    return 8 if O * I <= (1 << 20) else 2


def _padded_features(O: int) -> int:
    """Output features a wide projection's forward GEMM is computed with: O rounded up to a multiple of 256
    where O >= 2048 is not one.  hipBLASLt's kernel for (16384 x 1024) @ (1024 x O) on MI355X takes 159 us at
    O = 3104 (in_proj at state_dim 2: 3 d_inner + 2 H) and 103 us at O = 3328 (0.65 against 1.09 PFLOP/s);
    the extra features are zero rows of the weight, sliced off the output."""
    return O if O < 2048 or O % 256 == 0 else (O + 255) // 256 * 256


def padded_linear(x2: Tensor, weight: Tensor, bias: Optional[Tensor], padded: Optional[tuple] = None) -> Tensor:
    """x2 (T, I) @ weight^T (+ bias) -> (T, O), computed with the output features padded as
    ``_padded_features`` says (the result a column slice of the padded product, row stride O_pad).
    ``padded``: the (weight, bias) already padded, else they are padded here."""
    O = weight.shape[0]
    Op = _padded_features(O)
    if Op == O:
        return torch.addmm(bias, x2, weight.t()) if bias is not None else torch.mm(x2, weight.t())
    if padded is None:
        w = torch.cat([weight, weight.new_zeros(Op - O, weight.shape[1])])
        b = None if bias is None else torch.cat([bias, bias.new_zeros(Op - O)])
    else:
        w, b = padded
    y = torch.addmm(b, x2, w.t()) if b is not None else torch.mm(x2, w.t())
    return y[:, :O]


def _weight_grad(gy: Tensor, x: Tensor, dtype: torch.dtype) -> Tensor:
    """dW = gy^T x in ``dtype`` for gy (T, O) and x (T, I), accumulated in fp32 as one GEMM does: split over
    token slabs, a batched product of the slabs with fp32 outputs and their fixed-order sum rounded once
    (cdssm_slab_sum) where the HIP kernel serves the dtype; otherwise one product."""
    T, O = gy.shape
    I = x.shape[1]
    S = _wgrad_slabs(T, O, I)
    if S == 1 or not gy.is_cuda or dtype not in _lib.DTYPE_CODE:
        return torch.mm(gy.t(), x).to(dtype)
    a = gy.as_strided((S, T // S, O), (T // S * gy.stride(0), gy.stride(0), gy.stride(1))).transpose(1, 2)
    b = x.as_strided((S, T // S, I), (T // S * x.stride(0), x.stride(0), x.stride(1)))
    half = gy.dtype in (torch.bfloat16, torch.float16)
    part = (torch.bmm(a, b, out_dtype=torch.float32) if half else torch.bmm(a, b)).contiguous()
    out = torch.empty(O, I, dtype=dtype, device=gy.device)
    st = _lib.load().cdssm_slab_sum(_lib.DTYPE_CODE[dtype], _lib.ptr(part), S, O * I, _lib.ptr(out),
                                    _lib.stream_of(gy.device))
    _lib.check(st, "cdssm_slab_sum")
    return out


def column_sum(x: Tensor) -> Tensor:
    """x (T, C) -> sum over T (C,) in x's dtype: fp32 accumulation in a fixed order, one rounding
    (cdssm_col_sum) where the HIP kernel serves the layout (CUDA bf16 / fp32, unit column stride, C and the
    row stride multiples of the 16-byte vector, 16-byte aligned); otherwise ``x.sum(0)``.  torch's reduction
    over the token dimension is slow on MI355X for these shapes (gate_proj's 16384 x 336 bias gradient: 19 us,
    in_proj's 16384 x 3328: 37 us; the two HIP launches: 13 and 24 us)."""
    T_, C = x.shape
    nv = 16 // x.element_size()
    if not (x.is_cuda and x.dtype in (torch.bfloat16, torch.float32) and x.stride(1) == 1 and C % nv == 0
            and x.stride(0) % nv == 0 and x.stride(0) >= C and x.data_ptr() % 16 == 0 and 0 < T_ < (1 << 22)):
        return x.sum(0)
    lib = _lib.load()
    ws = torch.empty(lib.cdssm_col_sum_workspace_bytes(T_, C) // 4, dtype=torch.float32, device=x.device)
    out = torch.empty(C, dtype=x.dtype, device=x.device)
    st = lib.cdssm_col_sum(_lib.DTYPE_CODE[x.dtype], _lib.ptr(x), x.stride(0), T_, C, _lib.ptr(out), _lib.ptr(ws),
                           _lib.stream_of(x.device))
    _lib.check(st, "cdssm_col_sum")
    return out


class TokenLinearFn(torch.autograd.Function):
    """x @ weight^T (+ bias) (+ residual) over (..., in) token rows -- nn.Linear plus the block's residual
    add (block.py:229) -- whose weight gradient is split over token slabs (``_weight_grad``) and whose bias
    gradient is ``column_sum``; wide outputs are computed with padded features (``padded_linear``).  The
    residual enters the GEMM's epilogue (one rounding of the sum, as the inference forward's out_proj); its
    gradient is the output's.  A bias and a residual are not taken together."""

    @staticmethod
    def forward(ctx, x, weight, bias, residual):
        if bias is not None and residual is not None:
            raise ValueError("TokenLinearFn: a bias and a residual are not taken together")
        O = weight.shape[0]
        x2 = x.reshape(-1, x.shape[-1])
        if residual is not None:
            y = torch.addmm(residual.reshape(-1, O), x2, weight.t())
        else:
            y = padded_linear(x2, weight, bias)
        ctx.save_for_backward(x2, weight)
        ctx.xshape, ctx.has_bias = x.shape, bias is not None
        ctx.bias_dtype = None if bias is None else bias.dtype
        return y.view(*x.shape[:-1], O)

    @staticmethod
    def backward(ctx, gy):
        x2, w = ctx.saved_tensors
        g2 = gy.reshape(-1, w.shape[0])
        dx = dw = db = None
        if ctx.needs_input_grad[0]:
            dx = torch.mm(g2, w).view(ctx.xshape)
        if ctx.needs_input_grad[1]:
            dw = _weight_grad(g2, x2, w.dtype)
        if ctx.has_bias and ctx.needs_input_grad[2]:
            db = column_sum(g2).to(ctx.bias_dtype)
        return dx, dw, db, (gy if ctx.needs_input_grad[3] else None)


def module_linear(lin: nn.Linear, x: Tensor, residual: Optional[Tensor] = None) -> Tensor:
    """``lin(x)`` (+ ``residual``): the module and torch's add."""
    y = lin(x)
    return y if residual is None else residual + y


def token_linear(lin: nn.Linear, x: Tensor, residual: Optional[Tensor] = None) -> Tensor:
    """``lin(x)`` (+ ``residual``) through TokenLinearFn where it applies (a CUDA x of the weight's dtype, no
    autocast; a residual only for a layer without bias), else ``module_linear``."""
    if (x.is_cuda and x.dtype == lin.weight.dtype and not torch.is_autocast_enabled()
            and (residual is None or (lin.bias is None and residual.dtype == x.dtype))):
        return TokenLinearFn.apply(x, lin.weight, lin.bias, residual)
    return module_linear(lin, x, residual)


def _kq_rows(K: Tensor, Q: Tensor) -> tuple:
    """K, Q (B, L, H, D) as the fused normalisation reads them: in place where each token's (H, D) block is
    dense and 16-byte aligned with a uniform token stride, else dense copies; (K, Q, token strides)."""
    B, L, H, D = K.shape
    if tuple(Q.shape) != (B, L, H, D):
        raise ValueError(f"K and Q shapes differ: {tuple(K.shape)} vs {tuple(Q.shape)}")
    strides, dense = [], []
    for t in (K, Q):
        ts = _token_stride(t, H * D)
        if (t.stride(3) != 1 or t.stride(2) != D or ts is None or t.data_ptr() % 16
                or (ts * t.element_size()) % 16):
            t, ts = t.contiguous(), H * D
        strides.append(ts)
        dense.append(t)
    return dense[0], dense[1], strides


def normalize_kq_qk(K: Tensor, Q: Tensor) -> tuple:
    """K^, Q^ = x * rsqrt(sum_d x^2 + 1e-6) per (token, head) and qk = K^.Q^ (fp32), in one pass.

    K, Q (B, L, H, D) with dense (H, D) blocks per token and any token stride (K may be a column slice
    of the in_proj output); returns dense K^, Q^ and qk (B, L, H) fp32 (normalize_kq.cu:75-79,
    block.py:191-192, 202)."""
    dt = _check_gpu("normalize_kq_qk", K, Q)
    B, L, H, D = K.shape
    K, Q, strides = _kq_rows(K, Q)
    Ko = torch.empty((B, L, H, D), dtype=dt, device=K.device)
    Qo = torch.empty_like(Ko)
    qk = torch.empty((B, L, H), dtype=torch.float32, device=K.device)
    st = _lib.load().cdssm_normalize_kq_qk_fwd(_lib.DTYPE_CODE[dt], _lib.ptr(K), strides[0], _lib.ptr(Q), strides[1],
                                              _lib.ptr(Ko), _lib.ptr(Qo), _lib.ptr(qk), B * L, H, D,
                                              _lib.stream_of(K.device))
    _lib.check(st, "cdssm_normalize_kq_qk_fwd")
    return Ko, Qo, qk


class NormalizeKQQkFn(torch.autograd.Function):
    """NormalizeKQFn (ops.py:84-97, normalize_kq.cu's rule) with the current-token q.k (block.py:191-192,
    202) in one kernel each way: (K, Q) -> (K^, Q^, qk) with qk = K^.Q^ fp32 (B, L, H), forward
    ``cdssm_normalize_kq_qk_fwd`` and backward ``cdssm_normalize_kq_qk_bwd``, which folds qk's gradient
    (dK^ += dqk Q^, dQ^ += dqk K^) into the normalisation's backward.  For training through the block, in
    place of NormalizeKQFn followed by torch's product and sum."""

    @staticmethod
    def forward(ctx, K, Q):
        B, L, H, D = K.shape
        Kr, Qr, strides = _kq_rows(K, Q)
        Ko, Qo, qk = normalize_kq_qk(Kr, Qr)
        ctx.save_for_backward(Kr, Qr)
        ctx.strides = strides
        return Ko, Qo, qk

    @staticmethod
    def backward(ctx, dKo, dQo, dqk):
        Kr, Qr = ctx.saved_tensors
        B, L, H, D = Kr.shape
        dt = Kr.dtype
        dKo = torch.zeros((B, L, H, D), dtype=dt, device=Kr.device) if dKo is None else dKo.to(dt).contiguous()
        dQo = torch.zeros((B, L, H, D), dtype=dt, device=Kr.device) if dQo is None else dQo.to(dt).contiguous()
        dqk = (torch.zeros((B, L, H), dtype=torch.float32, device=Kr.device) if dqk is None
               else dqk.to(torch.float32).contiguous())
        dK, dQ = torch.empty_like(dKo), torch.empty_like(dQo)
        st = _lib.load().cdssm_normalize_kq_qk_bwd(_lib.DTYPE_CODE[dt], _lib.ptr(Kr), ctx.strides[0], _lib.ptr(Qr),
                                                  ctx.strides[1], _lib.ptr(dKo), _lib.ptr(dQo), _lib.ptr(dqk),
                                                  _lib.ptr(dK), _lib.ptr(dQ), B * L, H, D, _lib.stream_of(Kr.device))
        _lib.check(st, "cdssm_normalize_kq_qk_bwd")
        return dK, dQ


class StateReadoutFn(torch.autograd.Function):
    """The block's readout of per-token states for state_dim N > 2 (block.py:208): (Y (B,L,H,N,D), Q
    (B,L,H,D)) -> einsum('blhsd,blhd->blhs', Y, Q) with fp32 accumulation, rounded once to the input dtype
    (cdssm_state_readout_fwd); backward dY = dr Q, dQ = sum_s dr_s Y_s (cdssm_state_readout_bwd)."""

    @staticmethod
    def forward(ctx, Y, Q):
        dt = _check_gpu("state_readout", Y, Q)
        B, L, H, N, D = Y.shape
        if tuple(Q.shape) != (B, L, H, D):
            raise ValueError(f"Q must be {(B, L, H, D)}, got {tuple(Q.shape)}")
        Yc, Qc = Y.contiguous(), Q.contiguous()
        r = torch.empty(B, L, H, N, dtype=dt, device=Y.device)
        st = _lib.load().cdssm_state_readout_fwd(_lib.DTYPE_CODE[dt], _lib.ptr(Yc), _lib.ptr(Qc), _lib.ptr(r),
                                                 B * L * H, N, D, _lib.stream_of(Y.device))
        _lib.check(st, "cdssm_state_readout_fwd")
        ctx.save_for_backward(Yc, Qc)
        return r

    @staticmethod
    def backward(ctx, dr):
        Y, Q = ctx.saved_tensors
        B, L, H, N, D = Y.shape
        drc = dr.to(Y.dtype).contiguous()
        dY, dQ = torch.empty_like(Y), torch.empty_like(Q)
        st = _lib.load().cdssm_state_readout_bwd(_lib.DTYPE_CODE[Y.dtype], _lib.ptr(Y), _lib.ptr(Q), _lib.ptr(drc),
                                                 _lib.ptr(dY), _lib.ptr(dQ), B * L * H, N, D,
                                                 _lib.stream_of(Y.device))
        _lib.check(st, "cdssm_state_readout_bwd")
        return dY, dQ


def shortcut_readout_(retrieved: Tensor, qk: Tensor, V: Tensor, vp: Tensor, sel_C: Tensor, scale: Tensor) -> Tensor:
    """In place: retrieved += sel_C * scale * qk^2 * vp * V (the shortcut of block.py:202-205 through the
    readout of block.py:208-211).  retrieved, V (B, L, H, 2); vp (B, L, H, 1); sel_C (B, L, H); qk fp32."""
    dt = _check_gpu("shortcut_readout", retrieved, V, vp, sel_C)
    if qk.device != retrieved.device or not qk.is_floating_point():
        raise TypeError(f"qk must be a floating tensor on {retrieved.device}, got {qk.dtype} on {qk.device}")
    qk = qk.to(torch.float32)  # the kernel reads fp32 q.k
    for n, t in dict(retrieved=retrieved, V=V, vp=vp, sel_C=sel_C, qk=qk).items():
        if not t.is_contiguous():
            raise ValueError(f"{n} must be contiguous")
    n = sel_C.numel()
    if retrieved.numel() != 2 * n or V.numel() != 2 * n or vp.numel() != n or qk.numel() != n:
        raise ValueError("retrieved, V (n, 2), vp, sel_C, qk (n) with n = B*L*H")
    sc = scale.detach().reshape(1).to(device=retrieved.device, dtype=torch.float32).contiguous()
    st = _lib.load().cdssm_shortcut_readout_fwd(_lib.DTYPE_CODE[dt], _lib.ptr(retrieved), _lib.ptr(qk), _lib.ptr(V),
                                               _lib.ptr(vp), _lib.ptr(sel_C), _lib.ptr(sc), n,
                                               _lib.stream_of(retrieved.device))
    _lib.check(st, "cdssm_shortcut_readout_fwd")
    return retrieved


def shortcut_readout_rows_(y: Tensor, qk: Tensor, V: Tensor, vp: Tensor, sel_C: Tensor, scale: Tensor) -> Tensor:
    """In place: y += sel_C * scale * qk^2 * vp.repeat_interleave(2, -1) * V, in fp32 with one rounding
    (block.py:194-211's shortcut through the readout, N/2 complex state rows per head;
    cdssm_shortcut_readout_rows_fwd).  y, V (B, L, H, N) dense; vp (B, L, H, N/2); sel_C (B, L, H); qk fp32."""
    dt = _check_gpu("shortcut_readout_rows", y, V, vp, sel_C)
    B, L, H, N = y.shape
    if tuple(V.shape) != (B, L, H, N) or tuple(vp.shape) != (B, L, H, N // 2) or tuple(sel_C.shape) != (B, L, H):
        raise ValueError("y, V (B, L, H, N), vp (B, L, H, N/2), sel_C (B, L, H)")
    if not y.is_contiguous():
        raise ValueError("y must be contiguous")
    qk32 = qk.to(torch.float32).contiguous()
    sc = scale.detach().reshape(1).to(device=y.device, dtype=torch.float32).contiguous()
    Vc, vpc, sc_ = V.contiguous(), vp.contiguous(), sel_C.contiguous()
    st = _lib.load().cdssm_shortcut_readout_rows_fwd(_lib.DTYPE_CODE[dt], _lib.ptr(y), _lib.ptr(qk32), _lib.ptr(Vc),
                                                     _lib.ptr(vpc), _lib.ptr(sc_), _lib.ptr(sc), B * L * H, N,
                                                     _lib.stream_of(y.device))
    _lib.check(st, "cdssm_shortcut_readout_rows_fwd")
    return y


class ScanShortcutFn(torch.autograd.Function):
    """The block's retrieved vector for training, one autograd node: the readout-form scan
    (ChunkwiseDeltaScanAbarFn's kernels: sel_C (Y.q) of SSDChunkwiseScan(A_bar, K, V vp, beta), never forming
    Y) plus the current-token shortcut sel_C scale (q.k)^2 V vp (block.py:194-211), any even state_dim up to
    32.  (q, k, v, beta, sel_C, A_bar, vp, qk, scale, chunk_size) -> retrieved (B,L,H,N); qk (B,L,H) fp32, scale
    the one-element shortcut_scale.  The shortcut is added in fp32 with one rounding
    (cdssm_shortcut_readout_rows_fwd); its backward adds its gradients to the scan's in place and returns
    dL/d(q.k) in fp32 and dL/dscale from fixed-order partial sums (cdssm_shortcut_readout_rows_bwd)."""

    @staticmethod
    def forward(ctx, q, k, v, beta, sel_C, A_bar, vp, qk, scale, chunk_size):
        B, L, H, D, N, Q, dtype = _abar_validate(q, k, v, beta, sel_C, A_bar, vp, None, chunk_size)
        if qk.shape != (B, L, H):
            raise ValueError(f"qk must be ({B}, {L}, {H}), got {tuple(qk.shape)}")
        ins = [t.contiguous() for t in (q, k, v, beta, sel_C, A_bar, vp)]
        qk32 = qk.detach().to(torch.float32).contiguous()
        sc = scale.detach().reshape(1).to(device=q.device, dtype=torch.float32).contiguous()
        y, _, ws = chunkwise_delta_scan_abar_fwd(*ins, None, Q, train=True)
        st = _lib.load().cdssm_shortcut_readout_rows_fwd(_lib.DTYPE_CODE[dtype], _lib.ptr(y), _lib.ptr(qk32),
                                                         _lib.ptr(ins[2]), _lib.ptr(ins[6]), _lib.ptr(ins[4]),
                                                         _lib.ptr(sc), B * L * H, N, _lib.stream_of(q.device))
        _lib.check(st, "cdssm_shortcut_readout_rows_fwd")
        ctx.save_for_backward(*ins, qk32, sc, ws)
        ctx.Q, ctx.qk_dtype, ctx.scale_dtype, ctx.scale_shape = Q, qk.dtype, scale.dtype, scale.shape
        return y

    @staticmethod
    def backward(ctx, dy):
        *ins, qk32, sc, ws = ctx.saved_tensors
        dy = dy.to(ins[0].dtype).contiguous()
        dq, dk, dv, dbeta, dsel, dA, dvp, _ = chunkwise_delta_scan_abar_bwd(dy, None, *ins, ws, False, ctx.Q)
        B, L, H, N = dv.shape
        lib = _lib.load()
        n = B * L * H
        dqk = torch.empty(B, L, H, dtype=torch.float32, device=dy.device)
        part = torch.empty(lib.cdssm_shortcut_readout_rows_partials(n, N), dtype=torch.float32, device=dy.device)
        st = lib.cdssm_shortcut_readout_rows_bwd(_lib.DTYPE_CODE[dy.dtype], _lib.ptr(dy), _lib.ptr(qk32),
                                                 _lib.ptr(ins[2]), _lib.ptr(ins[6]), _lib.ptr(ins[4]), _lib.ptr(sc),
                                                 _lib.ptr(dv), _lib.ptr(dvp), _lib.ptr(dsel), _lib.ptr(dqk),
                                                 _lib.ptr(part), n, N, _lib.stream_of(dy.device))
        _lib.check(st, "cdssm_shortcut_readout_rows_bwd")
        dscale = part.sum().reshape(ctx.scale_shape).to(ctx.scale_dtype)
        return dq, dk, dv, dbeta, dsel, dA, dvp, dqk.to(ctx.qk_dtype), dscale, None


def group_norm_gate(y: Tensor, num_groups: int, gamma: Tensor, beta: Tensor, eps: float, z: Tensor,
                    x_conv: Tensor, D: Tensor, return_sums: bool = False):
    """GroupNorm over (channels of a group, all L) in fp32, cast to y's dtype, * silu(z) + D * x_conv
    (block.py:215-225).  y, x_conv (B, L, C) dense; z (B, L, C) with any token stride.  With
    ``return_sums`` also the running statistics a decode step continues from, (B, G, 4) fp32 = (shift,
    sum (x - shift), sum (x - shift)^2, count) with the shift the group's first element, taken from the
    kernel's own partial sums."""
    Dp = D.to(y.dtype).contiguous()
    dt = _check_gpu("group_norm_gate", y, z, x_conv, Dp)
    B, L, C = y.shape
    if tuple(z.shape) != (B, L, C) or tuple(x_conv.shape) != (B, L, C):
        raise ValueError("y, z and x_conv must all be (B, L, C)")
    yc, xc = y.contiguous(), x_conv.contiguous()
    try:
        zs = _token_view(z, C)
    except ValueError:  # not one uniform token stride (e.g. a slice along L of a column slice): a dense copy
        z = z.contiguous()
        zs = C
    # the affine parameters are read in their own dtype (bf16 or fp32) and widened exactly in the kernel
    pdt = gamma.dtype if gamma.dtype in _lib.DTYPE_CODE else torch.float32
    g = gamma.detach().to(device=y.device, dtype=pdt).contiguous()
    b = beta.detach().to(device=y.device, dtype=pdt).contiguous()
    lib = _lib.load()
    nb = lib.cdssm_group_norm_workspace_bytes(B, num_groups, L)
    if nb < 0:
        raise ValueError(f"invalid group norm shape B={B} G={num_groups} L={L}")
    ws = torch.empty(max(1, nb // 4), dtype=torch.float32, device=y.device)
    out = torch.empty_like(yc)
    st = lib.cdssm_group_norm_gate_fwd(_lib.DTYPE_CODE[dt], _lib.DTYPE_CODE[pdt], _lib.ptr(yc), _lib.ptr(g),
                                       _lib.ptr(b), _lib.ptr(z), zs,
                                       _lib.ptr(xc), _lib.ptr(Dp), _lib.ptr(out), _lib.ptr(ws), B, L, C, num_groups,
                                       float(eps), _lib.stream_of(y.device))
    _lib.check(st, "cdssm_group_norm_gate_fwd")
    if not return_sums:
        return out
    # the partial sums (B, G, S) of (x - shift, (x - shift)^2), shift = the group's first element
    G = int(num_groups)
    S = (nb // 8 - B * G) // (B * G)
    part = ws[:B * G * S * 2].view(B, G, S, 2).sum(2)
    k0 = yc[:, 0].reshape(B, G, C // G)[..., 0].float()
    n = torch.full_like(k0, float(L * (C // G)))
    return out, torch.stack([k0, part[..., 0], part[..., 1], n], dim=-1).contiguous()


class GroupNormGateFn(torch.autograd.Function):
    """The block's epilogue after readout_proj with gradients (block.py:215-225 under autograd):
    out = GroupNorm_G(y) (fp32, rounded to y's dtype) * silu(z) + D * x_conv on the HIP kernels, forward
    ``cdssm_group_norm_gate_fwd`` and backward ``cdssm_group_norm_gate_bwd`` (dy, dz, dx_conv for the
    D x_conv term, dgamma, dbeta, dD with the reference's rounding points and the GroupNorm backward in
    fp32), in place of torch's cast, group_norm, silu, products and sum and their backwards.  y, x_conv
    (B, L, C) dense, z (B, L, C) with one token stride, all 16-byte aligned; ``usable`` says whether a call
    qualifies."""

    @staticmethod
    def usable(y: Tensor, z: Tensor, x_conv: Tensor, num_groups: int, params) -> bool:
        if not (y.is_cuda and y.dtype in _lib.DTYPE_CODE and z.dtype == y.dtype and x_conv.dtype == y.dtype):
            return False
        B, L, C = y.shape
        nv = 16 // y.element_size()
        if C % num_groups or (C // num_groups) % nv or (64 * nv) % (C // num_groups):
            return False
        try:
            zs = _token_view(z, C)
        except ValueError:
            return False
        if not (y.is_contiguous() and x_conv.is_contiguous()) or (zs * y.element_size()) % 16:
            return False
        return all(t.data_ptr() % 16 == 0 for t in (y, z, x_conv, *params))

    @staticmethod
    def forward(ctx, y, z, x_conv, gamma, beta, D, num_groups, eps):
        B, L, C = y.shape
        G = int(num_groups)
        zs = _token_view(z, C)
        pdt = gamma.dtype if gamma.dtype in _lib.DTYPE_CODE else torch.float32
        g = gamma.detach().to(dtype=pdt).contiguous()
        b = beta.detach().to(dtype=pdt).contiguous()
        Dp = D.detach().to(y.dtype).contiguous()
        lib = _lib.load()
        ws = torch.empty(max(1, lib.cdssm_group_norm_workspace_bytes(B, G, L) // 4), dtype=torch.float32,
                         device=y.device)
        out = torch.empty_like(y)
        st = lib.cdssm_group_norm_gate_fwd(_lib.DTYPE_CODE[y.dtype], _lib.DTYPE_CODE[pdt], _lib.ptr(y), _lib.ptr(g),
                                           _lib.ptr(b), _lib.ptr(z), zs, _lib.ptr(x_conv), _lib.ptr(Dp),
                                           _lib.ptr(out), _lib.ptr(ws), B, L, C, G, float(eps),
                                           _lib.stream_of(y.device))
        _lib.check(st, "cdssm_group_norm_gate_fwd")
        ctx.save_for_backward(y, z, x_conv, g, b, Dp, ws)
        ctx.meta = (G, zs, pdt, gamma.dtype, beta.dtype, D.dtype, tuple(D.shape))
        return out

    @staticmethod
    def backward(ctx, dout):
        y, z, x_conv, g, b, Dp, ws = ctx.saved_tensors
        G, zs, pdt, gdt, bdt, ddt, dshape = ctx.meta
        B, L, C = y.shape
        dout = dout.to(y.dtype).contiguous()
        lib = _lib.load()
        wsb = torch.empty(max(1, lib.cdssm_group_norm_gate_bwd_workspace_bytes(B, G, L, C) // 4),
                          dtype=torch.float32, device=y.device)
        dy, dz, dx = torch.empty_like(y), torch.empty_like(y), torch.empty_like(y)
        dg, db = torch.empty_like(g), torch.empty_like(b)
        dD = torch.empty_like(Dp)
        st = lib.cdssm_group_norm_gate_bwd(_lib.DTYPE_CODE[y.dtype], _lib.DTYPE_CODE[pdt], _lib.ptr(y), _lib.ptr(g),
                                           _lib.ptr(b), _lib.ptr(z), zs, _lib.ptr(x_conv), _lib.ptr(Dp),
                                           _lib.ptr(ws), _lib.ptr(dout), _lib.ptr(dy), _lib.ptr(dz), _lib.ptr(dx),
                                           _lib.ptr(dg), _lib.ptr(db), _lib.ptr(dD), _lib.ptr(wsb), B, L, C, G,
                                           _lib.stream_of(y.device))
        _lib.check(st, "cdssm_group_norm_gate_bwd")
        return (dy, dz, dx, dg.to(gdt), db.to(bdt), dD.to(ddt).reshape(dshape), None, None)


class Conv1dSiLU(nn.Module):
    """Depthwise causal conv1d + SiLU (modules.py:14-35); weight (C, 1, K), bias (C)."""

    def __init__(self, d_inner: int, kernel_size: int = 4):
        super().__init__()
        self.d_inner = d_inner
        self.kernel_size = kernel_size
        self.weight = nn.Parameter(torch.empty(d_inner, 1, kernel_size))
        self.bias = nn.Parameter(torch.zeros(d_inner))
        with torch.no_grad():
            nn.init.normal_(self.weight, std=1.0 / math.sqrt(kernel_size))

    def forward(self, x: Tensor) -> Tensor:
        return _Conv1dSiLUFn.apply(x, self.weight, self.bias)


def dynamics_at(gate_raw: Tensor, log_dt_scale: Tensor, rope_freqs: Tensor, gating_c: float, omega_thresh: float,
                adt_delta: float, adt_smoothness: float, adt_eps: float, n_heads: int, state_dim: int,
                l0: int = 0, l0_dev: Optional[Tensor] = None) -> tuple:
    """DynamicsFusedFn's forward (dynamics_fused.cu:35-140) for gate rows at sequence positions l0 .. l0+L-1:
    the RoPE term omega + l * rope_freqs (block.py:59-62) takes the absolute position.  ``l0_dev`` (one
    int64 on the device) adds a position the kernel reads at run time (a graph-captured decode step).
    Forward only."""
    g = gate_raw.contiguous()
    _check_gpu("dynamics_at", g)
    H, N = int(n_heads), int(state_dim)
    B, L, GH = g.shape
    if GH != (N + 5) * H:
        raise ValueError(f"gate_raw last dim must be (state_dim + 5) * n_heads = {(N + 5) * H}, got {GH}")
    lds = log_dt_scale.detach().float().contiguous()
    rf = rope_freqs.detach().float().contiguous()
    A = torch.empty(B, L, H, N, dtype=g.dtype, device=g.device)
    vp = torch.empty(B, L, H, N // 2, dtype=g.dtype, device=g.device)
    beta = torch.empty(B, L, H, dtype=g.dtype, device=g.device)
    selc = torch.empty(B, L, H, dtype=g.dtype, device=g.device)
    st = _lib.load().cdssm_dynamics_fused_fwd_at(
        _lib.DTYPE_CODE[g.dtype], _lib.ptr(g), _lib.ptr(lds), _lib.ptr(rf), float(gating_c), float(omega_thresh),
        float(adt_delta), float(adt_smoothness), float(adt_eps), _lib.ptr(A), _lib.ptr(vp), _lib.ptr(beta),
        _lib.ptr(selc), B, L, H, N, int(l0), _lib.ptr(l0_dev), _lib.stream_of(g.device))
    _lib.check(st, "cdssm_dynamics_fused_fwd_at")
    return A, vp, beta, selc


def conv1d_silu_step(x: Tensor, window: Tensor, weight: Tensor, bias: Tensor) -> Tensor:
    """One decode token of conv1d+SiLU: x (B, C) (dense channels, any row stride); window (B, K-1, C), the
    last K-1 inputs of each row (oldest first), updated in place.  Returns y (B, C), the full
    convolution's output at the new position."""
    _check_gpu("conv1d_silu_step", x)
    B, C = x.shape
    K = weight.shape[-1]
    if x.stride(1) != 1:
        x = x.contiguous()
    if tuple(window.shape) != (B, K - 1, C) or window.dtype != x.dtype or not window.is_contiguous():
        raise ValueError(f"window must be a contiguous ({B}, {K - 1}, {C}) {x.dtype} tensor")
    wc = weight.to(x.dtype).contiguous()
    bc = bias.to(x.dtype).contiguous()
    y = torch.empty((B, C), dtype=x.dtype, device=x.device)
    st = _lib.load().cdssm_conv1d_silu_step(_lib.DTYPE_CODE[x.dtype], _lib.ptr(x), x.stride(0) if B > 1 else C,
                                           _lib.ptr(window), _lib.ptr(wc), _lib.ptr(bc), _lib.ptr(y), B, C, K,
                                           _lib.stream_of(x.device))
    _lib.check(st, "cdssm_conv1d_silu_step")
    return y


def group_norm_gate_step(y: Tensor, gsum: Tensor, gamma: Tensor, beta: Tensor, eps: float, z: Tensor,
                         x_conv: Tensor, D: Tensor, position: Optional[Tensor] = None,
                         readout_weight: Optional[Tensor] = None) -> Tensor:
    """One decode token of the GroupNorm epilogue (block.py:215-225) with running statistics ``gsum``
    (B, G, 4) fp32 = (shift, sum (x - shift), sum (x - shift)^2, count) per (b, group) over every position
    so far (as ``group_norm_gate(..., return_sums=True)`` returns them), updated in place; y, x_conv (B, C);
    z (B, C) with any row stride.  ``position`` (one int64 on the device) is incremented by the call.
    With ``readout_weight`` (C, K), ``y`` is the retrieved readout (B, K) and the readout projection
    y @ readout_weight^T (block.py:213) runs inside the kernel (cdssm_readout_group_norm_gate_step)."""
    Dp = D.to(y.dtype).contiguous()
    yc, xc = y.contiguous(), x_conv.contiguous()
    dt = _check_gpu("group_norm_gate_step", yc, z, xc, Dp)
    B, C = xc.shape
    G = gsum.shape[1]
    if tuple(gsum.shape) != (B, G, 4) or gsum.dtype != torch.float32 or not gsum.is_contiguous():
        raise ValueError(f"gsum must be a contiguous float32 ({B}, G, 4) tensor")
    if z.stride(1) != 1:
        z = z.contiguous()
    pdt = gamma.dtype if gamma.dtype in _lib.DTYPE_CODE else torch.float32
    g = gamma.detach().to(device=y.device, dtype=pdt).contiguous()
    b = beta.detach().to(device=y.device, dtype=pdt).contiguous()
    out = torch.empty_like(xc)
    if readout_weight is not None:
        wr = readout_weight.detach().to(dt).contiguous()
        if tuple(wr.shape) != (C, yc.shape[1]) or yc.shape[0] != B:
            raise ValueError(f"readout_weight must be ({C}, {yc.shape[1]}) and y ({B}, {yc.shape[1]}), got "
                             f"{tuple(wr.shape)} and {tuple(yc.shape)}")
        st = _lib.load().cdssm_readout_group_norm_gate_step(
            _lib.DTYPE_CODE[dt], _lib.DTYPE_CODE[pdt], _lib.ptr(yc), _lib.ptr(wr), yc.shape[1], _lib.ptr(gsum),
            _lib.ptr(g), _lib.ptr(b), _lib.ptr(z), z.stride(0) if B > 1 else C, _lib.ptr(xc), _lib.ptr(Dp),
            _lib.ptr(out), B, C, G, float(eps), _lib.ptr(position), _lib.stream_of(y.device))
        _lib.check(st, "cdssm_readout_group_norm_gate_step")
        return out
    st = _lib.load().cdssm_group_norm_gate_step(_lib.DTYPE_CODE[dt], _lib.DTYPE_CODE[pdt], _lib.ptr(yc),
                                               _lib.ptr(gsum), _lib.ptr(g), _lib.ptr(b), _lib.ptr(z),
                                               z.stride(0) if B > 1 else C, _lib.ptr(xc), _lib.ptr(Dp),
                                               _lib.ptr(out), B, C, G, float(eps), _lib.ptr(position),
                                               _lib.stream_of(y.device))
    _lib.check(st, "cdssm_group_norm_gate_step")
    return out


class RMSNorm(nn.Module):
    """x * rsqrt(mean(x^2) + eps) in fp32, cast back, times weight (modules.py:38-53)."""

    # training on the HIP forward and backward (RMSNormFn); False: the reference's torch expression
    fused_backward: bool = True

    def __init__(self, d_model: int, eps: float = _BF16_EPS ** 2):
        super().__init__()
        self.eps = eps
        self.weight = nn.Parameter(torch.ones(d_model))

    def forward(self, x: Tensor) -> Tensor:
        if torch.is_grad_enabled() and (x.requires_grad or self.weight.requires_grad):
            if self.fused_backward and RMSNormFn.usable(x):
                return RMSNormFn.apply(x, self.weight, self.eps)
            # training: the reference's expression (modules.py:49-53), differentiable through torch
            x32 = x.float()
            return (x32 * torch.rsqrt(x32.pow(2).mean(-1, keepdim=True) + self.eps)).to(x.dtype) * self.weight
        return rms_norm(x, self.weight, self.eps)


class CDSSMBlock(nn.Module):
    """One CD-SSM block (block.py:14-229), forward on the HIP kernels."""

    # decode steps take the one-launch token kernel (cdssm_decode_block_token) where its alignment holds;
    # False: the separate per-token kernels (the same values)
    fused_step: bool = True
    # ... and, with it, the readout + GroupNorm + gate epilogue in the same launch (cdssm_decode_block_tail);
    # False: the epilogue in a launch of its own
    fused_tail: bool = True
    # training (and inference where the chunked form does not apply) takes the readout-form scan
    # (ChunkwiseDeltaScanAbarFn, no Y); False: SSDChunkwiseScan's Y read out in torch (the reference's op
    # sequence; the same gradients)
    readout_scan: bool = True
    # inference with state_dim 16 in bf16 takes the chunked MFMA form (cdssm_chunked_scan_fwd_abar, no Y);
    # False: SSDChunkwiseScan's Y read out in fp32 torch (the reference's op sequence)
    chunked_scan: bool = True
    # training runs the GroupNorm + gate epilogue on the HIP kernels with their backward (GroupNormGateFn);
    # False: torch's group_norm and elementwise ops (the reference's op sequence)
    fused_epilogue: bool = True
    # training with the readout-form scan adds the current-token shortcut in the scan's autograd node
    # (ScanShortcutFn, HIP forward and backward); False: torch's elementwise ops for the shortcut
    fused_shortcut: bool = True
    # training runs the five projections (out_proj with the residual add) through TokenLinearFn (weight
    # gradients split over token slabs where that is faster, bias gradients by cdssm_col_sum); False:
    # nn.Linear and torch's add
    token_linear: bool = True

    def __init__(self, config: CDSSMConfig, layer_idx: int = 0):
        super().__init__()
        self.config = config
        N, H, Di = config.state_dim, config.n_heads, config.d_inner
        G = N + 5
        self.in_proj = nn.Linear(config.d_model, 3 * Di + H * N, bias=True)
        self.conv = Conv1dSiLU(Di, kernel_size=config.conv_kernel_size)
        self.gate_proj = nn.Linear(Di, H * G, bias=True)
        self.log_dt_scale = nn.Parameter(torch.zeros(H))
        freqs = 1.0 / (config.rope_base ** (torch.arange(0, H, dtype=torch.float32) / H))
        self.register_buffer("rope_freqs", freqs, persistent=False)
        self.Q_proj = nn.Linear(Di, Di, bias=False)
        self.readout_proj = nn.Linear(H * N, Di, bias=False)
        self.out_proj = nn.Linear(Di, config.d_model, bias=False)
        self.norm = RMSNorm(config.d_model, eps=config.eps_norm)
        self.ssm_norm = nn.GroupNorm(config.ssm_norm_groups, Di)
        self.D = nn.Parameter(torch.zeros(Di))
        self.v_residual_gate = nn.Parameter(torch.zeros(H))
        self.shortcut_scale = nn.Parameter(torch.zeros(1))
        self._f32_cache: dict = {}
        self._init_weights(layer_idx)

    def _fp32(self, name: str) -> Tensor:
        """A contiguous fp32 copy of parameter / buffer ``name`` (the reference's ``.float()`` casts), kept
        while the tensor's storage and version are unchanged, so a forward launches no cast kernels."""
        t = getattr(self, name)
        key = (t.data_ptr(), t._version, t.dtype, t.device)
        hit = self._f32_cache.get(name)
        if hit is None or hit[0] != key:
            hit = (key, t.detach().float().contiguous())
            self._f32_cache[name] = hit
        return hit[1]

    def _param_as(self, name: str, t: Tensor, dtype: torch.dtype) -> Tensor:
        """A contiguous copy of parameter ``t`` in ``dtype`` (``t`` itself where it already is one), kept while
        the parameter's storage and version are unchanged, so a decode step launches no cast kernels."""
        if t.dtype == dtype and t.is_contiguous():
            return t.detach()
        key = (t.data_ptr(), t._version, dtype, t.device)
        hit = self._f32_cache.get(("as", name))
        if hit is None or hit[0] != key:
            hit = (key, t.detach().to(dtype).contiguous())
            self._f32_cache[("as", name)] = hit
        return hit[1]

    def _value_gate(self, dtype: torch.dtype) -> Tensor:
        """sigmoid(v_residual_gate) as (1, 1, H, 1) in ``dtype`` (block.py:169-174), kept while the parameter's
        storage and version are unchanged, so an inference forward launches no kernel for it."""
        g = self.v_residual_gate
        key = (g.data_ptr(), g._version, dtype, g.device)
        hit = self._f32_cache.get("vgate")
        if hit is None or hit[0] != key:
            hit = (key, torch.sigmoid(g.detach())[None, None, :, None].to(dtype))
            self._f32_cache["vgate"] = hit
        return hit[1]

    def _padded_in_proj(self) -> Optional[tuple]:
        """in_proj's weight and bias with zero rows up to ``_padded_features`` (None where no padding
        applies), kept while the parameters' storage and versions are unchanged."""
        w, b = self.in_proj.weight, self.in_proj.bias
        O = w.shape[0]
        Op = _padded_features(O)
        if Op == O:
            return None
        key = tuple((t.data_ptr(), t._version, t.dtype, t.device) for t in (w, b))
        hit = self._f32_cache.get("in_proj_pad")
        if hit is None or hit[0] != key:
            wp = torch.cat([w.detach(), w.new_zeros(Op - O, w.shape[1])]).contiguous()
            bp = torch.cat([b.detach(), b.new_zeros(Op - O)]).contiguous()
            hit = (key, (wp, bp))
            self._f32_cache["in_proj_pad"] = hit
        return hit[1]

    def _stacked_gate_q(self) -> tuple:
        """[gate_proj.weight; Q_proj.weight] and [gate_proj.bias; 0]: the decode step's two projections of
        x_conv (block.py:180, 190) as one GEMM (one launch fewer per layer; at the forward's B*L rows the
        two GEMMs are faster apart), kept while the parameters' storage and versions are unchanged."""
        gw, gb, qw = self.gate_proj.weight, self.gate_proj.bias, self.Q_proj.weight
        key = tuple((t.data_ptr(), t._version, t.dtype, t.device) for t in (gw, gb, qw))
        hit = self._f32_cache.get("gate_q")
        if hit is None or hit[0] != key:
            w = torch.cat([gw.detach(), qw.detach().to(gw.dtype)], dim=0).contiguous()
            b = torch.cat([gb.detach(), torch.zeros(qw.shape[0], dtype=gb.dtype, device=gb.device)]).contiguous()
            hit = (key, (w, b))
            self._f32_cache["gate_q"] = hit
        return hit[1]

    @torch.no_grad()
    def _init_weights(self, layer_idx: int) -> None:
        """Variance-preserving init (block.py:90-138) and spectral init (init.py:44-126)."""
        cfg = self.config
        N, H, Di = cfg.state_dim, cfg.n_heads, cfg.d_inner
        std = layer_stds(cfg.d_model, Di, cfg.n_layers)
        nn.init.normal_(self.in_proj.weight, std=std["in_proj"])
        nn.init.zeros_(self.in_proj.bias)
        v0 = 3 * Di
        self.in_proj.weight[v0:v0 + H * N].normal_(std=std["in_proj"] / math.sqrt(cfg.head_dim))
        nn.init.normal_(self.gate_proj.weight[:N * H], std=std["dynamics_proj"])
        nn.init.normal_(self.gate_proj.weight[N * H:], std=1.0 / math.sqrt(Di))
        b = self.gate_proj.bias
        b.zero_()
        ib = cfg.init_biases
        for seg, key in enumerate(("sel_B_bias", "sel_C_bias", "sel_dt_bias", "beta_bias", "r_gate_bias")):
            b[(N + seg) * H:(N + seg + 1) * H] = ib[key]
        alphas, omegas = spectral_biases(cfg, layer_idx)
        nh = N // 2
        for j in range(nh):
            b[j * H:(j + 1) * H] = alphas[j]
            b[(nh + j) * H:(nh + j + 1) * H] = omegas[j]
        nn.init.eye_(self.Q_proj.weight)
        nn.init.normal_(self.readout_proj.weight, std=1.0 / math.sqrt(H * N))
        nn.init.normal_(self.out_proj.weight, std=std["out_proj"])
        nn.init.zeros_(self.D)

    def forward(self, x: Tensor, v_first: Optional[Tensor] = None, cache: Optional[dict] = None,
                inplace_residual: bool = False):
        """x (B, L, d_model) -> (x + block(x), v_first).  With ``cache`` (a dict), also fills it with the
        state a decode step continues from: the conv window, the scan's decode state, the GroupNorm's
        running sums and the position.  ``inplace_residual`` (inference, a dense x the caller no longer
        needs): the output is accumulated into x itself by the out_proj GEMM, with no copy of x."""
        cfg = self.config
        N, H, D, Di = cfg.state_dim, cfg.n_heads, cfg.head_dim, cfg.d_inner
        if N != 2 and cache is not None:
            raise NotImplementedError("decode caches need state_dim = 2 (the decode kernels' state layout)")
        if torch.is_grad_enabled() and (x.requires_grad or any(p.requires_grad for p in self.parameters())):
            # training: the fused block kernels carry no autograd graph, so take the differentiable path
            if cache is not None:
                raise RuntimeError("decode caches are filled under torch.no_grad() / torch.inference_mode()")
            return self._forward_autograd(x, v_first)
        B, L, _ = x.shape
        residual = x
        # (B, L, 3 Di + H N), a column slice of the product with the features padded where that is faster;
        # z, x_gate and K are read in place
        xn = self.norm(x)
        proj = padded_linear(xn.reshape(B * L, -1), self.in_proj.weight, self.in_proj.bias,
                             self._padded_in_proj()).view(B, L, -1)
        z, x_gate, K, V = proj.split([Di, Di, Di, H * N], dim=-1)
        K = K.reshape(B, L, H, D)
        V = V.reshape(B, L, H, N)
        if v_first is None:
            v_first = V.detach()
        else:
            V = torch.lerp(v_first, V, self._value_gate(V.dtype))
        x_conv = self.conv(x_gate)
        if cache is not None:
            Kc = self.conv.kernel_size - 1
            win = x_gate.new_zeros(B, Kc, Di)
            nk = min(Kc, L)
            if nk > 0:
                win[:, Kc - nk:] = x_gate[:, L - nk:]
            cache["conv"] = win
            # the position of the next token, and an arrival count the fused decode tail uses to advance it
            cache["l"] = torch.tensor([L, 0], dtype=torch.int64, device=x.device)
            # the step's parameter-derived constants, formed once (the weights are fixed while decoding)
            cache["lds"] = self.log_dt_scale.detach().float().contiguous()
            cache["rope"] = self.rope_freqs.detach().float().contiguous()
            cache["scale"] = self.shortcut_scale.detach().float().reshape(1).contiguous()
            cache["vgate"] = torch.sigmoid(self.v_residual_gate.detach().float())[None, :, None].to(x.dtype)
            cache["vgate_h"] = cache["vgate"].reshape(-1).contiguous()
            # gate_proj and Q_proj share their input: one GEMM per step over the stacked weights
            cache["w_gq"], cache["b_gq"] = self._stacked_gate_q()
        gates = self.gate_proj(x_conv)
        A_bar, vp, beta, sel_C = DynamicsFusedFn.apply(
            gates.contiguous(), self._fp32("log_dt_scale"), self._fp32("rope_freqs"), cfg.gating_c,
            cfg.bf16_omega_thresh, cfg.bf16_delta, cfg.bf16_smoothness, cfg.eps_adaptive_dt, H, N)
        Q = self.Q_proj(x_conv).reshape(B, L, H, D)
        K, Q, qk = normalize_kq_qk(K, Q)
        V = V.contiguous()
        if self.chunked_scan and N == 16 and x.dtype == torch.bfloat16 and D in (64, 128) \
                and cfg.chunk_size % 16 == 0 and 16 <= cfg.chunk_size <= 256:
            # the reference's default state_dim: the chunked (UT) form on the matrix cores returns the
            # retrieved vector sel_C (Y.q + shortcut) (block.py:194-211) without forming Y
            retrieved, _ = chunked_scan_abar(Q, K, V, beta, sel_C, A_bar, vp, chunk_size=cfg.chunk_size,
                                             shortcut_scale=self._fp32("shortcut_scale"))
        elif N != 2 and self.readout_scan and D in (64, 128) and 1 <= cfg.chunk_size <= 128:
            # N/2 complex state rows per head: the fused scan with its readout, each row a virtual head
            # sharing k, q, beta and sel_C (block.py:194-211 with ssd.py:39-111), without forming Y; the
            # shortcut s (q.k)^2 V_gated (block.py:202-205) through the readout in fp32
            retrieved, _ = chunkwise_delta_scan_abar(Q, K, V, beta, sel_C, A_bar, vp, chunk_size=cfg.chunk_size)
            shortcut_readout_rows_(retrieved, qk, V, vp, sel_C, self._fp32("shortcut_scale"))
        elif N != 2:
            # N/2 complex pairs per head (the reference default is 16): Y from SSDChunkwiseScan (its
            # fused kernels, each pair a virtual head sharing k; block.py:194-211 with ssd.py:39-111);
            # the readout and the shortcut in fp32, then rounded to the model dtype
            V_gated = V * vp.repeat_interleave(2, dim=-1)                                 # block.py:194-195
            Y = SSDChunkwiseScan(cfg.chunk_size, N)(A_bar, K, V_gated, beta)              # block.py:198
            ret = (Y.float() * Q.float().unsqueeze(-2)).sum(-1)                           # block.py:208
            ret = ret + self._fp32("shortcut_scale") * (qk * qk).unsqueeze(-1) * V_gated.float()  # :202-205
            retrieved = (ret * sel_C.float().unsqueeze(-1)).to(x.dtype)                   # block.py:211
        elif cache is None:
            retrieved, _ = chunkwise_delta_scan_abar(Q, K, V, beta, sel_C, A_bar, vp, chunk_size=cfg.chunk_size)
        else:
            retrieved, cache["scan"] = prefill_abar(Q, K, V, beta, sel_C, A_bar, vp, chunk_size=cfg.chunk_size)
        if N == 2:
            # current-token shortcut (block.py:202-205) through the readout: sel_C s (q.k)^2 V vp
            shortcut_readout_(retrieved, qk, V, vp, sel_C, self._fp32("shortcut_scale"))
        y = self.readout_proj(retrieved.reshape(B, L, H * N))
        y = group_norm_gate(y, self.ssm_norm.num_groups, self.ssm_norm.weight, self.ssm_norm.bias,
                            self.ssm_norm.eps, z, x_conv, self.D, return_sums=cache is not None)
        if cache is not None:
            y, cache["gsum"] = y
        # out_proj with the residual added in the GEMM epilogue (in place: no copy of the residual first)
        if inplace_residual and residual.is_contiguous():
            out = residual.view(B * L, -1).addmm_(y.reshape(B * L, Di), self.out_proj.weight.t())
        else:
            out = torch.addmm(residual.reshape(B * L, -1), y.reshape(B * L, Di), self.out_proj.weight.t())
        return out.reshape(residual.shape), v_first

    def _forward_autograd(self, x: Tensor, v_first: Optional[Tensor]):
        """The block with gradients (block.py:140-229, for training): the HIP ops that have a backward --
        conv1d+SiLU (CUDAConv1dSiLUOp), DynamicsFusedFn, NormalizeKQFn and the fused scan, whose backwards
        are the reference's, and the GroupNorm + gate epilogue (GroupNormGateFn) -- and torch for the
        projections, the RMSNorm and the shortcut.  The scan is ChunkwiseDeltaScanAbarFn, which returns the readout sel_C (Y.q) itself
        and never forms Y (state_dim N > 2: N/2 state rows per head as virtual heads); with
        ``readout_scan`` off, SSDChunkwiseScan's Y is read out here by StateReadoutFn (the HIP readout
        and its backward).  The
        shortcut enters as s (q.k)^2 V_gated (the reference adds s (q.k) V_gated k^T to Y and reads it with
        q: the same value), with elementwise products in the compute dtype."""
        cfg = self.config
        N, H, D, Di = cfg.state_dim, cfg.n_heads, cfg.head_dim, cfg.d_inner
        B, L, _ = x.shape
        residual = x
        lin = token_linear if self.token_linear else module_linear
        proj = lin(self.in_proj, self.norm(x))
        z, x_gate, K, V = proj.split([Di, Di, Di, H * N], dim=-1)                     # block.py:162-166
        K = K.reshape(B, L, H, D)
        V = V.reshape(B, L, H, N)
        if v_first is None:                                                           # block.py:169-174
            v_first = V.detach()
        else:
            V = torch.lerp(v_first, V, torch.sigmoid(self.v_residual_gate)[None, None, :, None].to(V.dtype))
        x_conv = self.conv(x_gate)                                                    # block.py:177
        gates = lin(self.gate_proj, x_conv)
        A_bar, vp, beta, sel_C = DynamicsFusedFn.apply(
            gates, self.log_dt_scale.float(), self.rope_freqs, cfg.gating_c, cfg.bf16_omega_thresh,
            cfg.bf16_delta, cfg.bf16_smoothness, cfg.eps_adaptive_dt, H, N)           # block.py:184-188
        Q = lin(self.Q_proj, x_conv).reshape(B, L, H, D)
        if self.fused_epilogue and D // (16 // K.element_size()) in (4, 8, 16, 32) and D % (16 // K.element_size()) == 0:
            # block.py:191-192 and the q.k of :202 in one kernel each way
            K, Q, qk = NormalizeKQQkFn.apply(K, Q)                                    # qk in fp32
        else:
            K, Q = NormalizeKQFn.apply(K, Q)                                          # block.py:191-192
            qk = (Q * K).sum(-1)                                                      # block.py:202
        readout = self.readout_scan and D in (64, 128) and 1 <= cfg.chunk_size <= 128
        if readout and self.fused_shortcut:
            # the fused scan with its readout, sel_C (Y.q) (block.py:198, 208-211), without forming the
            # (B,L,H,N,D) Y (its backward rebuilds chunk states from the forward's records; N > 2: the
            # head's N/2 complex state rows run as virtual heads sharing k, q, beta and sel_C), and the
            # current-token shortcut sel_C s (q.k)^2 V vp (block.py:194-195, 202-205) in the same node
            retrieved = ScanShortcutFn.apply(Q, K, V, beta, sel_C, A_bar, vp, qk, self.shortcut_scale,
                                             cfg.chunk_size)
        else:
            qk = qk.to(V.dtype)
            V_gated = V * vp.repeat_interleave(2, dim=-1)                             # block.py:194-195
            shortcut = self.shortcut_scale * (qk * qk).unsqueeze(-1) * V_gated        # block.py:204-208
            if readout:
                y_scan, _ = ChunkwiseDeltaScanAbarFn.apply(Q, K, V, beta, sel_C, A_bar, vp, None, cfg.chunk_size)
                retrieved = y_scan + shortcut * sel_C.unsqueeze(-1)
            else:
                Y = SSDChunkwiseScan(cfg.chunk_size, N)(A_bar, K, V_gated, beta)      # block.py:198
                retrieved = (StateReadoutFn.apply(Y, Q) + shortcut) * sel_C.unsqueeze(-1)  # block.py:208-211
        y = lin(self.readout_proj, retrieved.reshape(B, L, H * N))
        G, gn = self.ssm_norm.num_groups, self.ssm_norm
        if self.fused_epilogue and GroupNormGateFn.usable(y, z, x_conv, G, (gn.weight, gn.bias, self.D)):
            # block.py:216-225 on the HIP kernels, forward and backward
            y = GroupNormGateFn.apply(y, z, x_conv, gn.weight, gn.bias, self.D, G, gn.eps)
        else:
            y = torch.nn.functional.group_norm(y.float().transpose(1, 2), G, gn.weight.float(), gn.bias.float(),
                                               gn.eps).to(y.dtype).transpose(1, 2)  # block.py:216-223
            y = y * torch.nn.functional.silu(z) + self.D * x_conv
        return lin(self.out_proj, y.to(self.out_proj.weight.dtype), residual=residual), v_first

    def step(self, x: Tensor, v_first: Optional[Tensor], cache: dict):
        """One decode token: x (B, d_model) at position cache["l"] -> (x + block(x), v_first (B, H, N)),
        advancing ``cache`` (filled by ``forward(..., cache=...)`` over the prompt).  Every piece of state,
        the position included, lives on the device, so the step can be captured in a HIP graph.  The scan, conv and
        dynamics reproduce the forward over prompt + token at that token; the GroupNorm takes running
        statistics over every position so far, which is the forward's for a one-layer model (the
        reference's GroupNorm spans all L positions, so in deeper models appending a token also changes
        earlier positions' activations, which a recurrent step does not revisit)."""
        cfg = self.config
        N, H, D, Di = cfg.state_dim, cfg.n_heads, cfg.head_dim, cfg.d_inner
        B = x.shape[0]
        if _skinny_ok(x, self.in_proj.weight):  # RMSNorm + in_proj in one skinny product
            proj = skinny_linear(x, self.in_proj.weight, self.in_proj.bias, norm_weight=self.norm.weight,
                                 eps=self.norm.eps)
        else:
            proj = self.in_proj(rms_norm(x, self.norm.weight, self.norm.eps))  # (B, 3 Di + H N)
        z, x_gate, K, V = proj.split([Di, Di, Di, H * N], dim=-1)
        K = K.reshape(B, 1, H, D)
        V = V.reshape(B, H, N)
        x_conv = conv1d_silu_step(x_gate, cache["conv"], self.conv.weight, self.conv.bias)
        GH = (N + 5) * H
        if _skinny_ok(x_conv, cache["w_gq"]):
            gq = skinny_linear(x_conv, cache["w_gq"], cache["b_gq"])  # (B, GH + Di): gates | Q
        else:
            gq = torch.addmm(cache["b_gq"], x_conv, cache["w_gq"].t())
        es = x.element_size()
        rows_ok = ((gq.data_ptr() + GH * es) % 16 == 0 and (gq.stride(0) * es) % 16 == 0
                   and (proj.data_ptr() + 2 * Di * es) % 16 == 0 and (proj.stride(0) * es) % 16 == 0
                   and proj.stride(1) == 1 and gq.stride(1) == 1)
        if (self.fused_step and self.fused_tail and D in (64, 128) and rows_ok and cache["l"].numel() == 2
                and x_conv.is_contiguous() and z.stride(1) == 1):
            # the token step and the readout + GroupNorm + gate epilogue in one launch (cdssm_decode_block_tail)
            st = cache["scan"]
            v_used = torch.empty(B, H, N, dtype=x.dtype, device=x.device)
            y = torch.empty(B, Di, dtype=x.dtype, device=x.device)
            vf = None if v_first is None else v_first.contiguous()
            gn = self.ssm_norm
            pdt = gn.weight.dtype if gn.weight.dtype in _lib.DTYPE_CODE else torch.float32
            gam_w = self._param_as("ssm_norm.weight", gn.weight, pdt)
            bet_w = self._param_as("ssm_norm.bias", gn.bias, pdt)
            Dp = self._param_as("D", self.D, x.dtype)
            wr = self._param_as("readout_proj.weight", self.readout_proj.weight, x.dtype)
            status = _lib.load().cdssm_decode_block_tail(
                _lib.DTYPE_CODE[x.dtype], _lib.DTYPE_CODE[pdt], _lib.ptr(gq), gq.stride(0), _lib.ptr(proj),
                proj.stride(0), 2 * Di, 3 * Di, _lib.ptr(vf), _lib.ptr(cache["vgate_h"]) if vf is not None else None,
                _lib.ptr(cache["lds"]), _lib.ptr(cache["rope"]), float(cfg.gating_c), float(cfg.bf16_omega_thresh),
                float(cfg.bf16_delta), float(cfg.bf16_smoothness), float(cfg.eps_adaptive_dt), _lib.ptr(cache["l"]),
                _lib.ptr(cache["scale"]), _lib.ptr(st.state), _lib.ptr(st.gam), _lib.ptr(st.pos), _lib.ptr(v_used),
                _lib.ptr(wr), _lib.ptr(cache["gsum"]), _lib.ptr(gam_w), _lib.ptr(bet_w), _lib.ptr(z), z.stride(0),
                _lib.ptr(x_conv), _lib.ptr(Dp), _lib.ptr(y), B, H, D, N, st.chunk_size, Di, gn.num_groups,
                float(gn.eps), _lib.stream_of(x.device))
            _lib.check(status, "cdssm_decode_block_tail")
            if v_first is None:
                v_first = v_used
            if _skinny_ok(y, self.out_proj.weight) and x.dtype == torch.bfloat16:
                return skinny_linear(y, self.out_proj.weight, residual=x), v_first
            return torch.addmm(x, y, self.out_proj.weight.t()), v_first
        if self.fused_step and D in (64, 128) and rows_ok:
            # the token's dynamics, K/Q norm, value residual, scan step and shortcut in one launch
            st = cache["scan"]
            retrieved = torch.empty(B, H, N, dtype=x.dtype, device=x.device)
            v_used = torch.empty(B, H, N, dtype=x.dtype, device=x.device)
            vf = None if v_first is None else v_first.contiguous()
            status = _lib.load().cdssm_decode_block_token(
                _lib.DTYPE_CODE[x.dtype], _lib.ptr(gq), gq.stride(0), _lib.ptr(proj), proj.stride(0), 2 * Di,
                3 * Di, _lib.ptr(vf), _lib.ptr(cache["vgate_h"]) if vf is not None else None, _lib.ptr(cache["lds"]),
                _lib.ptr(cache["rope"]), float(cfg.gating_c), float(cfg.bf16_omega_thresh), float(cfg.bf16_delta),
                float(cfg.bf16_smoothness), float(cfg.eps_adaptive_dt), _lib.ptr(cache["l"]), _lib.ptr(cache["scale"]),
                _lib.ptr(st.state), _lib.ptr(st.gam), _lib.ptr(st.pos), _lib.ptr(retrieved), _lib.ptr(v_used), B, H,
                D, N, st.chunk_size, _lib.stream_of(x.device))
            _lib.check(status, "cdssm_decode_block_token")
            if v_first is None:
                v_first = v_used
            return self._step_tail(x, retrieved, z, x_conv, cache), v_first
        if v_first is None:
            v_first = V.detach()
        else:
            V = torch.lerp(v_first, V, cache["vgate"])
        A_bar, vp, beta, sel_C = dynamics_at(gq[:, :GH].reshape(B, 1, GH), cache["lds"], cache["rope"], cfg.gating_c,
                                             cfg.bf16_omega_thresh, cfg.bf16_delta, cfg.bf16_smoothness,
                                             cfg.eps_adaptive_dt, H, N, 0, cache["l"])
        Q = gq[:, GH:].reshape(B, 1, H, D)  # read in place (a column slice)
        K, Q, qk = normalize_kq_qk(K, Q)
        V = V.contiguous()
        retrieved = decode_step_abar(cache["scan"], Q, K, V, beta, sel_C, A_bar, vp)  # (B, H, 2)
        shortcut_readout_(retrieved, qk, V, vp, sel_C, cache["scale"])
        return self._step_tail(x, retrieved, z, x_conv, cache), v_first

    def _step_tail(self, x: Tensor, retrieved: Tensor, z: Tensor, x_conv: Tensor, cache: dict) -> Tensor:
        """readout_proj + the GroupNorm step (one kernel), out_proj + residual; advances the position."""
        B = x.shape[0]
        # readout_proj inside the GroupNorm step kernel; the kernel also advances the position
        y = group_norm_gate_step(retrieved.reshape(B, -1), cache["gsum"], self.ssm_norm.weight, self.ssm_norm.bias,
                                 self.ssm_norm.eps, z, x_conv, self.D, position=cache["l"],
                                 readout_weight=self.readout_proj.weight)
        if _skinny_ok(y, self.out_proj.weight) and x.dtype == torch.bfloat16:
            return skinny_linear(y, self.out_proj.weight, residual=x)
        return torch.addmm(x, y, self.out_proj.weight.t())


class CDSSMLMHeadModel(nn.Module):
    """Embedding -> blocks -> RMSNorm -> tied LM head (model.py:12-51)."""

    def __init__(self, config: CDSSMConfig):
        super().__init__()
        self.config = config
        self.embedding = nn.Embedding(config.vocab_size, config.d_model)
        self.blocks = nn.ModuleList(CDSSMBlock(config, layer_idx=i) for i in range(config.n_layers))
        self.final_norm = RMSNorm(config.d_model)
        self.lm_head = nn.Linear(config.d_model, config.vocab_size, bias=False)
        self.lm_head.weight = self.embedding.weight
        with torch.no_grad():
            nn.init.normal_(self.embedding.weight,
                            std=layer_stds(config.d_model, config.d_inner, config.n_layers)["embedding"])

    def forward(self, input_ids: Tensor) -> Tensor:
        x = self.embedding(input_ids)
        v_first = None
        for blk in self.blocks:
            # the hidden state is this loop's own tensor: each block accumulates into it in place
            x, v_first = blk(x, v_first=v_first, inplace_residual=True)
        return self.lm_head(self.final_norm(x))

    def prefill(self, input_ids: Tensor) -> tuple:
        """Forward over the prompt (B, L): the last position's logits (B, vocab) and the per-layer decode
        caches that ``decode_step`` continues from (generation without re-forwarding; the reference
        re-forwards, predict.py:53-67)."""
        x = self.embedding(input_ids)
        v_first = None
        caches: List[dict] = []
        for blk in self.blocks:
            c: dict = {}
            x, v_first = blk(x, v_first=v_first, cache=c, inplace_residual=True)
            caches.append(c)
        return self.lm_head(self.final_norm(x[:, -1])), caches

    def decode_step(self, token_ids: Tensor, caches: List[dict]) -> Tensor:
        """One new token per row, token_ids (B,): logits (B, vocab); advances ``caches`` (see
        ``CDSSMBlock.step`` for what the step reproduces exactly)."""
        x = self.embedding(token_ids)
        v_first = None
        for blk, c in zip(self.blocks, caches):
            x, v_first = blk.step(x, v_first, c)
        # the tied head (N = vocab) stays on the library GEMM: the skinny kernel re-reads the 64-row
        # activation for every 16 of the 32000 columns (46 us against 18 us, measured on MI355X)
        return self.lm_head(self.final_norm(x))

    def decode_graph(self, caches: List[dict], warmup: int = 2) -> "DecodeGraph":
        """``decode_step`` captured once in a HIP graph over ``caches`` (see ``DecodeGraph``)."""
        return DecodeGraph(self, caches, warmup)


def _clone_cache(c: dict) -> dict:
    out = {}
    for k, v in c.items():
        if torch.is_tensor(v):
            out[k] = v.clone()
        elif isinstance(v, DecodeState):
            out[k] = DecodeState(v.state.clone(), v.gam.clone(), v.pos.clone(), v.chunk_size)
        else:
            out[k] = v
    return out


class DecodeGraph:
    """A model's decode step captured in one HIP graph: each call copies the B new token ids into the
    graph's input, replays every layer's launches at once (no per-kernel host launch cost) and returns
    the graph's logits buffer (B, vocab), overwritten by the next call.  The graph advances the same
    ``caches`` as ``decode_step`` would; the warm-up steps before the capture run on copies of them."""

    def __init__(self, model: "CDSSMLMHeadModel", caches: List[dict], warmup: int = 2):
        dev = caches[0]["conv"].device
        B = caches[0]["conv"].shape[0]
        self.ids = torch.zeros(B, dtype=torch.long, device=dev)
        side = torch.cuda.Stream(device=dev)
        side.wait_stream(torch.cuda.current_stream(dev))
        with torch.cuda.stream(side), torch.no_grad():
            scratch = [_clone_cache(c) for c in caches]
            for _ in range(warmup):
                model.decode_step(self.ids, scratch)
        torch.cuda.current_stream(dev).wait_stream(side)
        torch.cuda.synchronize(dev)
        del scratch
        self.graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(self.graph), torch.no_grad():
            self.logits = model.decode_step(self.ids, caches)

    def __call__(self, token_ids: Tensor) -> Tensor:
        self.ids.copy_(token_ids)
        self.graph.replay()
        return self.logits
