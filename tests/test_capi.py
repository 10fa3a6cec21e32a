"""The C-ABI library on the CPU host: it loads, exports every symbol the header
declares, and its host-side argument checks reject bad calls before any GPU
work (these calls launch nothing, so they run without a GPU)."""

import os
import re

import pytest

from cdssm_hip import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADERS = [os.path.join(ROOT, "include", f) for f in os.listdir(os.path.join(ROOT, "include"))
           if f.endswith(".h")]


def declared_functions():
    names = set()
    for h in HEADERS:
        text = open(h).read()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        for m in re.finditer(r"\b(cdssm_[a-z0-9_]+)\s*\(", text):
            names.add(m.group(1))
    return sorted(names)


def test_header_declares_entry_points():
    names = declared_functions()
    assert "cdssm_fused_scan_fwd" in names and "cdssm_last_error" in names


def test_library_loads_and_exports_every_declared_symbol():
    lib = _lib.load()
    for name in declared_functions():
        assert hasattr(lib, name), f"{name} declared in include/ but not exported"
    assert lib.cdssm_abi_version() >= 1


def test_binding_signatures_cover_the_header():
    assert set(declared_functions()) <= set(_lib.SIGNATURES), \
        "every declared entry point needs a ctypes signature"


def _fused_call(lib, **over):
    args = dict(dtype=1, q=16, k=16, v=16, beta=16, sel_c=16, dt=16, r=16, alpha=16, omega=16, c=1.0,
                h0=None, y=16, h_final=16, ws=16, B=1, L=64, H=2, D=64, N=2, chunk=64, stream=None)
    args.update(over)
    return lib.cdssm_fused_scan_fwd(*args.values())


@pytest.mark.parametrize("bad,msg", [
    (dict(dtype=7), "dtype"),
    (dict(N=4), "state_dim"),
    (dict(D=96), "head_dim"),
    (dict(chunk=0), "chunk"),
    (dict(chunk=256), "chunk"),
    (dict(B=0), "positive"),
    (dict(q=None), "null"),
    (dict(k=8), "aligned"),
    (dict(y=18), "(re, im) pair"),
    (dict(dtype=0, y=20), "(re, im) pair"),
    (dict(H=1 << 19, D=128), "32-bit row offsets"),
])
def test_fused_fwd_rejects_invalid_arguments_without_launching(bad, msg):
    lib = _lib.load()
    st = _fused_call(lib, **bad)
    assert st == -1
    assert msg in _lib.last_error()


@pytest.mark.parametrize("stamps,n", [(None, 64), (16, 0), (16, -1)])
def test_stamped_fwd_rejects_a_missing_stamp_buffer_without_launching(stamps, n):
    """The instrumentation entry refuses a null or empty stamp buffer before its
    other checks (a short buffer is refused by the launcher, which first queries
    the device: covered by the gpu test)."""
    lib = _lib.load()
    args = dict(dtype=1, q=16, k=16, v=16, beta=16, sel_c=16, dt=16, r=16, alpha=16, omega=16, c=1.0,
                h0=None, y=16, h_final=16, ws=16, B=1, L=64, H=2, D=64, N=2, chunk=64)
    st = lib.cdssm_fused_scan_fwd_stamped(*args.values(), stamps, n, None)
    msg = "stamp buffer"
    assert st == -1
    assert msg in _lib.last_error()


@pytest.mark.parametrize("over,msg", [
    (dict(dtype=0), "bf16 only"),
    (dict(X=None), "must not be null"),
    (dict(M=65), "M <= 64"),
    (dict(K=200, ldx=200, ldw=200), "multiple of 128"),
    (dict(ldx=1000), "16-byte aligned"),
    (dict(W=24), "16-byte aligned"),
])
def test_skinny_gemm_rejects_invalid_arguments_without_launching(over, msg):
    lib = _lib.load()
    args = dict(dtype=1, X=16, ldx=1024, W=16, ldw=1024, bias=None, R=None, ldr=0, wnorm=None, eps=0.0, Y=16,
                ldy=1024, M=64, N=1024, K=1024, stream=None)
    args.update(over)
    assert lib.cdssm_skinny_gemm(*args.values()) == -1
    assert msg in _lib.last_error()


@pytest.mark.parametrize("over,msg", [
    (dict(N=5), "even N <= 64"),
    (dict(N=66), "even N <= 64"),
    (dict(n=0), "n > 0"),
    (dict(y=18), "aligned to a (re, im) pair"),
    (dict(qk=None), "null pointer"),
])
def test_shortcut_rows_fwd_rejects_invalid_arguments_without_launching(over, msg):
    lib = _lib.load()
    args = dict(dtype=1, y=16, qk=16, V=16, vp=16, sel=16, scale=16, n=1024, N=16, stream=None)
    args.update(over)
    assert lib.cdssm_shortcut_readout_rows_fwd(*args.values()) == -1
    assert msg in _lib.last_error()


def test_shortcut_rows_bwd_rejects_a_misaligned_gradient_and_sizes_its_partials():
    lib = _lib.load()
    args = [1, 16, 16, 16, 16, 16, 16, 18, 16, 16, 16, 16, 1024, 16, None]
    assert lib.cdssm_shortcut_readout_rows_bwd(*args) == -1
    assert "dV must be aligned" in _lib.last_error()
    # one partial per 256-lane workgroup: a lane per complex pair where N/2 is a power of two, else per row
    assert lib.cdssm_shortcut_readout_rows_partials(1024, 16) == 1024 * 8 // 256
    assert lib.cdssm_shortcut_readout_rows_partials(1000, 2) == 4
    assert lib.cdssm_shortcut_readout_rows_partials(1024, 6) == 4
    assert lib.cdssm_shortcut_readout_rows_partials(0, 16) == -1


@pytest.mark.parametrize("over,msg", [
    (dict(C=30, ld=30), "multiple of 8"),
    (dict(ld=300), "row stride >= C"),
    (dict(x=24), "16-byte aligned"),
    (dict(ws=None), "non-null"),
    (dict(rows=0), "rows > 0"),
])
def test_col_sum_rejects_invalid_arguments_without_launching(over, msg):
    lib = _lib.load()
    args = dict(dtype=1, x=16, ld=336, rows=1024, C=336, out=16, ws=16, stream=None)
    args.update(over)
    assert lib.cdssm_col_sum(*args.values()) == -1
    assert msg in _lib.last_error()
    assert lib.cdssm_col_sum_workspace_bytes(16384, 336) == 256 * 336 * 4


def test_slab_sum_rejects_invalid_arguments_without_launching():
    lib = _lib.load()
    assert lib.cdssm_slab_sum(1, 16, 0, 1024, 16, None) == -1 and "0 < S" in _lib.last_error()
    assert lib.cdssm_slab_sum(1, 16, 8, 0, 16, None) == -1 and "n > 0" in _lib.last_error()
    assert lib.cdssm_slab_sum(1, None, 8, 1024, 16, None) == -1 and "null pointer" in _lib.last_error()
    assert lib.cdssm_slab_sum(7, 16, 8, 1024, 16, None) == -1


def test_fused_bwd_rejects_rows_beyond_32_bit_offsets_without_launching():
    lib = _lib.load()
    ptrs = [16] * 9
    st = lib.cdssm_fused_scan_bwd(1, *ptrs, 1.0, 16, None, 16, *([16] * 9), None, 16,
                                  1, 64, 1 << 19, 128, 2, 64, None)
    assert st == -1
    assert "32-bit row offsets" in _lib.last_error()


def _ssd_fwd_call(lib, **over):
    args = dict(dtype=1, a_bar=16, k=16, v=16, beta=16, Y=16, h_final=16, ws=16, B=1, L=64, H=2, D=64, N=2,
                chunk=64, train=0, stream=None)
    args.update(over)
    return lib.cdssm_ssd_scan_fwd(*args.values())


def _ssd_bwd_call(lib, **over):
    args = dict(dtype=1, a_bar=16, k=16, v=16, beta=16, dY=16, fwd_ws=16, dA=16, dK=16, dV=16, dbeta=16, ws=16,
                B=1, L=64, H=2, D=64, N=2, chunk=64, stream=None)
    args.update(over)
    return lib.cdssm_ssd_scan_bwd(*args.values())


@pytest.mark.parametrize("bad,msg", [
    (dict(dtype=5), "dtype"),
    (dict(N=3), "state_dim N must be even"),
    (dict(N=34), "state_dim N must be even"),
    (dict(D=48), "head_dim"),
    (dict(chunk=129), "chunk"),
    (dict(k=None), "null"),
    (dict(Y=None), "null"),
    (dict(k=8), "aligned"),
    (dict(Y=24), "Y must be 16-byte aligned"),
    (dict(H=1 << 18, D=128), "32-bit row offsets"),
])
def test_ssd_fwd_rejects_invalid_arguments_without_launching(bad, msg):
    lib = _lib.load()
    assert _ssd_fwd_call(lib, **bad) == -1
    assert msg in _lib.last_error()


@pytest.mark.parametrize("bad,msg", [
    (dict(N=5), "state_dim N must be even"),
    (dict(D=96), "head_dim"),
    (dict(dY=None), "null"),
    (dict(fwd_ws=None), "null"),
    (dict(dY=8), "16-byte aligned"),
    (dict(dK=40), "16-byte aligned"),
    (dict(dA=2), "(re, im) pair"),
])
def test_ssd_bwd_rejects_invalid_arguments_without_launching(bad, msg):
    lib = _lib.load()
    assert _ssd_bwd_call(lib, **bad) == -1
    assert msg in _lib.last_error()


def test_ssd_workspaces_are_the_fused_scans_with_virtual_heads():
    """N / 2 state rows per head scan as that many virtual heads: the forward workspace is the fused
    scan's with H N / 2 heads; the backward's adds, for N > 2, fp32 dk partials (P rows per head: R = N / 2,
    or R / 4 where a D-64 backward wave of 4 virtual heads sums its rows first) and dbeta partials per
    state row after a 16-byte aligned layout."""
    lib = _lib.load()
    B, L, H, D, Q = 2, 1000, 3, 64, 64
    for N in (2, 4, 16):
        Hv = H * N // 2
        assert lib.cdssm_ssd_scan_workspace_bytes(B, L, H, D, N, Q) == \
            lib.cdssm_fused_scan_workspace_bytes(B, L, Hv, D, 2, Q)
        base = lib.cdssm_fused_scan_bwd_workspace_bytes(B, L, Hv, D, 2, Q)
        R = N // 2
        P = R // 4 if R % 4 == 0 else R
        want = base if N == 2 else (-(-base // 16) * 16 + B * L * H * (P * D + R) * 4)
        assert lib.cdssm_ssd_scan_bwd_workspace_bytes(B, L, H, D, N, Q) == want
    assert lib.cdssm_ssd_scan_workspace_bytes(B, L, H, D, 3, Q) == -1
    assert lib.cdssm_ssd_scan_bwd_workspace_bytes(B, L, H, D, 34, Q) == -1


def test_gate_level_workspaces_with_state_rows():
    """The gate-level form at even N > 2 scans N / 2 state rows per head as virtual heads: the forward
    workspace is the fused scan's with H N / 2 heads; the backward's adds fp32 dk and dq partials (B, L,
    H P, D) (P = N / 2, or N / 8 where a D-64 backward wave of 4 virtual heads sums its rows first) and
    dbeta, dsel (B, L, H N/2) partials after a 16-byte aligned layout."""
    lib = _lib.load()
    B, L, H, D, Q = 2, 1000, 3, 64, 64
    for N in (4, 6, 16, 32):
        Hv = H * N // 2
        assert lib.cdssm_fused_scan_workspace_bytes(B, L, H, D, N, Q) == \
            lib.cdssm_fused_scan_workspace_bytes(B, L, Hv, D, 2, Q)
        base = lib.cdssm_fused_scan_bwd_workspace_bytes(B, L, Hv, D, 2, Q)
        R = N // 2
        P = R // 4 if R % 4 == 0 else R
        want = -(-base // 16) * 16 + 2 * B * L * H * (P * D + R) * 4
        assert lib.cdssm_fused_scan_bwd_workspace_bytes(B, L, H, D, N, Q) == want
    for N in (3, 34, 0):
        assert lib.cdssm_fused_scan_workspace_bytes(B, L, H, D, N, Q) == -1
        assert lib.cdssm_fused_scan_bwd_workspace_bytes(B, L, H, D, N, Q) == -1


def test_scan_level_entries_still_reject_state_rows():
    """Only the gate-level and SSD entries take N > 2; the scan-level forward rejects it before any
    device work (fake pointers are never touched)."""
    lib = _lib.load()
    p = 16
    st = lib.cdssm_fused_scan_fwd(1, *([p] * 7), p, p, 1.0, None, p, p, p, 1, 64, 2, 64, 4, 64, None)
    assert st != 0 and "state_dim N = 2" in _lib.last_error()


def test_lookback_status_rejects_a_null_status_pointer_without_touching_the_gpu():
    lib = _lib.load()
    assert lib.cdssm_lookback_status(1, None) == -1
    assert "status must not be NULL" in _lib.last_error()


def test_one_launch_areas_have_a_control_block_for_the_device_epoch():
    """The workspaces end their look-back areas with the 64-byte control block the
    epoch kernel writes (8 float2 words more than the flags and maps need)."""
    lib = _lib.load()
    B, L, H, D, Q = 2, 1000, 3, 64, 64
    NC = -(-L // Q)
    S = -(-NC // 16)
    NSEG = -(-NC // 4)
    NCK = -(-Q // 8) * 8 // 8
    carry = B * NC * H * D + B * NC * H + B * H * S * (D + 1)
    NGRP = -(-NSEG // 8)  # groups of 8 segments of the two-level fold
    fwd = (carry + (carry & 1) + 5 * B * L * H + B * NSEG * H * (2 * D + 2) + 8 + B * NGRP * H * (D + 1)
           + B * NC * H * NCK * D + B * NC * H * D + B * L * H)
    assert lib.cdssm_fused_scan_workspace_bytes(B, L, H, D, 2, Q) == 8 * fwd
    bwd = 2 * B * NC * H * D + B * H * S + B * H * S * D + B * NC * H + B * NSEG * H * (2 * D + 2) + 8
    assert lib.cdssm_fused_scan_bwd_workspace_bytes(B, L, H, D, 2, Q) == 8 * bwd


def _decode_call(lib, **over):
    args = dict(dtype=1, q=16, k=16, v=16, beta=16, sel_c=16, dt=16, r=16, alpha=16, omega=16, c=1.0,
                state=16, gam=16, pos=16, y=16, h_out=None, B=2, H=3, D=64, N=2, chunk=64, stream=None)
    args.update(over)
    return lib.cdssm_decode_step(*args.values())


@pytest.mark.parametrize("bad,msg", [
    (dict(dtype=3), "dtype"),
    (dict(N=4), "N = 2"),
    (dict(D=32), "D in"),
    (dict(chunk=0), "chunk"),
    (dict(B=0), "B, H > 0"),
    (dict(state=None), "null"),
])
def test_decode_step_rejects_invalid_arguments_without_launching(bad, msg):
    lib = _lib.load()
    assert _decode_call(lib, **bad) == -1
    assert msg in _lib.last_error()


def test_decode_init_rejects_invalid_arguments_without_launching():
    lib = _lib.load()
    assert lib.cdssm_decode_init(None, 16, 16, 16, 1, 2, 96, 2, None) == -1
    assert "D in" in _lib.last_error()
    assert lib.cdssm_decode_init(None, None, 16, 16, 1, 2, 64, 2, None) == -1
    assert "null" in _lib.last_error()


def test_workspace_size_formula():
    lib = _lib.load()
    B, L, H, D, N, Q = 8, 4096, 16, 64, 2, 64

    def expect(L):
        NC = -(-L // Q)
        S = -(-NC // 16)          # carry segments of 16 chunks
        carry = B * NC * H * D + B * NC * H + B * H * S * (D + 1)   # float2 counts
        pad = carry & 1               # the training records start 16-byte aligned
        saved = 4 * B * L * H         # (p, pc), (c.q, Y.q) per token-head: 2 float4
        gsaved = B * L * H            # g_t per token-head: float2
        NSEG = -(-NC // 4)            # one-pass look-back segments of 4 chunks
        NGRP = -(-NSEG // 8)          # groups of 8 segments (the two-level look-back fold)
        # maps, leaving states, rotations, flags, control block; group maps and their rotations
        onepass = B * NSEG * H * (2 * D + 2) + 8 + B * NGRP * H * (D + 1)
        NCK = -(-Q // 8) * 8 // 8     # z checkpoints per chunk (every 8 tokens of the 8-rounded loop)
        zck = B * NC * H * NCK * D
        cend = B * NC * H * D         # correction state after each chunk
        ycorr = B * L * H             # the chunked MFMA correction's readout
        return (carry + pad + saved + gsaved + onepass + zck + cend + ycorr) * 8
    assert lib.cdssm_fused_scan_workspace_bytes(B, L, H, D, N, Q) == expect(L)
    assert lib.cdssm_fused_scan_workspace_bytes(B, 100, H, D, N, Q) == expect(100)
    assert lib.cdssm_fused_scan_workspace_bytes(0, L, H, D, N, Q) == -1


def test_product_path_has_no_cpu_fallback():
    """The scan raises on CPU tensors instead of computing anything on the host."""
    import torch
    from cdssm_hip import chunkwise_delta_scan
    x = torch.zeros(1, 64, 2, 64)
    s = torch.zeros(1, 64, 2)
    with pytest.raises(RuntimeError, match="GPU only"):
        chunkwise_delta_scan(x, x, torch.zeros(1, 64, 2, 2), s, s, s, s, torch.zeros(2), torch.zeros(2), 1.0)


# The block / decode entry points: invalid arguments return -1 with a message and launch nothing
# (fake, 16-byte-aligned addresses: validation happens before any device access).
_BLOCK_CALLS = {
    "cdssm_rms_norm_fwd": dict(dtype=1, x=16, w=16, y=16, rows=4, C=64, eps=1e-5, stream=None),
    "cdssm_normalize_kq_qk_fwd": dict(dtype=1, K=16, ks=1024, Q=16, qs=1024, Ko=16, Qo=16, qk=16, BL=4, H=16,
                                      D=64, stream=None),
    "cdssm_shortcut_readout_fwd": dict(dtype=1, ret=16, qk=16, V=16, vp=16, sel=16, scale=16, n=8, stream=None),
    "cdssm_group_norm_gate_fwd": dict(dtype=1, pdt=1, y=16, g=16, b=16, z=16, zs=64, xc=16, D=16, out=16, ws=16,
                                      B=1, L=8, C=64, G=4, eps=1e-5, stream=None),
    "cdssm_group_norm_gate_step": dict(dtype=1, pdt=1, y=16, gsum=16, g=16, b=16, z=16, zs=64, xc=16, D=16,
                                       out=16, B=2, C=64, G=4, eps=1e-5, position=None, stream=None),
    "cdssm_conv1d_silu_step": dict(dtype=1, x=16, xs=64, win=16, w=16, b=16, y=16, B=2, C=64, K=4, stream=None),
    "cdssm_conv1d_silu_bwd": dict(dtype=1, x=16, xs=64, w=16, b=16, go=16, gx=16, gw=16, gb=16, ws=16, B=1, L=8,
                                  C=64, K=4, stream=None),
    "cdssm_decode_step_abar": dict(dtype=1, q=16, k=16, v=16, beta=16, sel=16, a=16, vp=16, state=16, gam=16,
                                   pos=16, y=16, h=None, B=2, H=3, D=64, N=2, chunk=64, stream=None),
    "cdssm_dynamics_fused_fwd_at": dict(dtype=1, gate=16, lds=16, rope=16, c=1.0, thr=1.0, delta=0.1, smooth=1.0,
                                        eps=1.0, A=16, vp=16, beta=16, sel=16, B=1, L=1, H=4, N=2, l0=5,
                                        l0_dev=None, stream=None),
}


@pytest.mark.parametrize("fn,bad,msg", [
    ("cdssm_rms_norm_fwd", dict(dtype=5), "dtype"),
    ("cdssm_rms_norm_fwd", dict(rows=0), "rows > 0"),
    ("cdssm_rms_norm_fwd", dict(w=None), "null"),
    ("cdssm_normalize_kq_qk_fwd", dict(D=48), "need D in"),
    ("cdssm_normalize_kq_qk_fwd", dict(ks=512), "token strides"),
    ("cdssm_normalize_kq_qk_fwd", dict(K=8), "aligned"),
    ("cdssm_shortcut_readout_fwd", dict(n=0), "n > 0"),
    ("cdssm_shortcut_readout_fwd", dict(scale=None), "null"),
    ("cdssm_group_norm_gate_fwd", dict(G=5), "divisible by G"),
    ("cdssm_group_norm_gate_fwd", dict(pdt=3), "param_dtype"),
    ("cdssm_group_norm_gate_fwd", dict(ws=None), "null"),
    ("cdssm_group_norm_gate_step", dict(zs=32), "row stride"),
    ("cdssm_conv1d_silu_step", dict(K=9), "kernel_size"),
    ("cdssm_conv1d_silu_step", dict(win=None), "null"),
    ("cdssm_conv1d_silu_bwd", dict(xs=32), "token stride"),
    ("cdssm_conv1d_silu_bwd", dict(ws=None), "null"),
    ("cdssm_decode_step_abar", dict(D=32), "D in"),
    ("cdssm_decode_step_abar", dict(a=None), "null"),
    ("cdssm_dynamics_fused_fwd_at", dict(l0=-1), "position offset"),
])
def test_block_entry_points_reject_invalid_arguments_without_launching(fn, bad, msg):
    lib = _lib.load()
    args = dict(_BLOCK_CALLS[fn])
    args.update(bad)
    assert getattr(lib, fn)(*args.values()) == -1
    assert msg in _lib.last_error()


def test_noalloc_rejects_shapes_beyond_its_scratch_without_launching():
    # the size check comes before any device query, so fake pointers never reach a kernel
    lib = _lib.load()
    st = lib.cdssm_fused_scan_fwd_noalloc(1, *([16] * 9), 1.0, None, 16, 16, 64, 65536, 32, 64, 2, 64, None)
    assert st == -1 and "static scratch" in _lib.last_error()
