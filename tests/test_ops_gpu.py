"""GPU parity of the drop-in ops (cdssm_hip.ops, cdssm_hip.ssd) against the oracle.

Every op is compared with its fp64 restatement in oracle/cdssm_oracle.py on
the same inputs (rounded to the op's dtype first).  Tolerances, normwise
max|x-ref|/max|ref| per tensor: fp32 1e-4, bf16 2e-2.
"""

import math

import pytest
import torch

from _gpu_util import DEV, log, rel
from oracle import cdssm_oracle as o

pytestmark = pytest.mark.gpu
TOL = {torch.float32: 1e-4, torch.bfloat16: 2e-2}


def rand_scan(gen, lead, C, H, D, N, amax=1.0):
    ang = torch.rand(*lead, C, H, N // 2, generator=gen) * 2 * math.pi
    mag = torch.rand(*lead, C, H, N // 2, generator=gen) * amax
    A = torch.stack([mag * torch.cos(ang), mag * torch.sin(ang)], -1).flatten(-2)
    K = torch.randn(*lead, C, H, D, generator=gen)
    K = K / K.norm(dim=-1, keepdim=True)
    V = torch.randn(*lead, C, H, N, generator=gen)
    beta = torch.rand(*lead, C, H, generator=gen)
    return A, K, V, beta


def rounded(dtype, *ts):
    return [t.to(dtype) for t in ts]


def dev(*ts, req=False):
    return [t.to(DEV).requires_grad_(req) if req else t.to(DEV) for t in ts]


CASES = [
    (torch.float32, 2, 64, 64), (torch.float32, 16, 48, 16), (torch.float32, 4, 128, 32),
    (torch.bfloat16, 2, 64, 64), (torch.bfloat16, 16, 128, 32),
]
IDS = [f"{str(d).split('.')[-1]}-N{n}-D{dd}-C{c}" for d, n, dd, c in CASES]


@pytest.mark.parametrize("dtype,N,D,C", CASES, ids=IDS)
def test_intra_chunk_scan_fwd_bwd(dtype, N, D, C):
    from cdssm_hip.ops import IntraChunkScanFn
    log(f"[intra] {dtype} N{N} D{D} C{C}")
    gen = torch.Generator().manual_seed(1)
    BNC, H = 6, 3
    A, K, V, beta = rounded(dtype, *rand_scan(gen, (BNC,), C, H, D, N))
    glh = torch.randn(BNC, C, H, N, D, generator=gen).to(dtype)
    gca = torch.randn(BNC, C, H, N, generator=gen).to(dtype)
    d64 = [t.double() for t in (A, K, V, beta)]
    lh_ref, ca_ref = o.intra_chunk_scan(*d64, N)
    gref = o.intra_chunk_scan_bwd_ref(glh.double(), gca.double(), *d64, N)
    a, k, v, b = dev(A, K, V, beta, req=True)
    lh, ca = IntraChunkScanFn.apply(a, k, v, b, N)
    torch.autograd.backward([lh, ca], [glh.to(DEV), gca.to(DEV)])
    torch.cuda.synchronize()
    errs = [rel(lh, lh_ref), rel(ca, ca_ref)] + [rel(x.grad, y) for x, y in zip((a, k, v, b), gref)]
    log("   " + " ".join(f"{e:.1e}" for e in errs))
    assert max(errs) <= TOL[dtype]
    assert lh.dtype == dtype and ca.dtype == dtype


@pytest.mark.parametrize("dtype,N,D", [(torch.float32, 2, 64), (torch.float32, 8, 100), (torch.bfloat16, 16, 128)])
def test_inter_chunk_scan_fwd_bwd(dtype, N, D):
    from cdssm_hip.ops import InterChunkScanFn
    log(f"[inter] {dtype} N{N} D{D}")
    gen = torch.Generator().manual_seed(2)
    B, NC, H = 2, 37, 3
    tA = rand_scan(gen, (B,), NC, H, D, N)[0].to(dtype)
    flh = torch.randn(B, NC, H, N, D, generator=gen).to(dtype)
    gcs = torch.randn(B, NC, H, N, D, generator=gen).to(dtype)
    cs_ref, _ = o.inter_chunk_scan(tA.double(), flh.double(), N)
    g_tA, g_flh, _ = o.inter_chunk_scan_bwd_ref(gcs.double(), tA.double(), cs_ref, N)
    a, f = dev(tA, flh, req=True)
    cs = InterChunkScanFn.apply(a, f, N)
    cs.backward(gcs.to(DEV))
    torch.cuda.synchronize()
    errs = [rel(cs, cs_ref), rel(a.grad, g_tA), rel(f.grad, g_flh)]
    log("   " + " ".join(f"{e:.1e}" for e in errs))
    assert max(errs) <= TOL[dtype]


@pytest.mark.parametrize("dtype,N,D,C", CASES, ids=IDS)
def test_exact_correction_fwd_bwd(dtype, N, D, C):
    from cdssm_hip.ops import ExactCorrectionFn
    log(f"[correction] {dtype} N{N} D{D} C{C}")
    gen = torch.Generator().manual_seed(3)
    B, NC, H = 2, 3, 3
    A, K, _, beta = rounded(dtype, *rand_scan(gen, (B, NC), C, H, D, N))
    cs = torch.randn(B, NC, H, N, D, generator=gen).to(dtype)
    gc = torch.randn(B, NC, C, H, N, D, generator=gen).to(dtype)
    d64 = [t.double() for t in (A, K, beta, cs)]
    corr_ref = o.exact_correction(*d64, N)
    gref = o.exact_correction_bwd_ref(gc.double(), *d64, N)
    a, k, b, s = dev(A, K, beta, cs, req=True)
    corr = ExactCorrectionFn.apply(a, k, b, s, N)
    corr.backward(gc.to(DEV))
    torch.cuda.synchronize()
    errs = [rel(corr, corr_ref)] + [rel(x.grad, y) for x, y in zip((a, k, b, s), gref)]
    log("   " + " ".join(f"{e:.1e}" for e in errs))
    assert max(errs) <= TOL[dtype]


@pytest.mark.parametrize("fused", [False, None], ids=["per_pass", "auto"])
@pytest.mark.parametrize("dtype,L,N,D,Q", [(torch.float32, 200, 2, 64, 64), (torch.float32, 130, 16, 64, 32),
                                           (torch.bfloat16, 256, 2, 128, 128)])
def test_ssd_chunkwise_scan_module_matches_reference_algorithm(dtype, L, N, D, Q, fused):
    """SSDChunkwiseScan forward (Y) and its autograd gradients vs the oracle's
    ssd.py restatement with the reference's correction backward attached; the
    per-pass ops (fused=False) and the module's own choice (the fused kernels
    for N = 2)."""
    from cdssm_hip.ssd import SSDChunkwiseScan
    log(f"[SSDChunkwiseScan] {dtype} L{L} N{N} D{D} Q{Q} fused={fused}")
    gen = torch.Generator().manual_seed(4)
    B, H = 2, 3
    A, K, V, beta = rounded(dtype, *rand_scan(gen, (B,), L, H, D, N, amax=0.99))
    gY = torch.randn(B, L, H, N, D, generator=gen).to(dtype)
    leaves = [t.double().requires_grad_(True) for t in (A, K, V, beta)]
    Y_ref = o.ssd_chunkwise_scan(*leaves, Q, N, correction_fn=o.correction_with_reference_grad)
    g_ref = torch.autograd.grad((Y_ref * gY.double()).sum(), leaves)
    a, k, v, b = dev(A, K, V, beta, req=True)
    Y = SSDChunkwiseScan(Q, N, fused=fused)(a, k, v, b)
    Y.backward(gY.to(DEV))
    torch.cuda.synchronize()
    errs = [rel(Y, Y_ref)] + [rel(x.grad, y) for x, y in zip((a, k, v, b), g_ref)]
    log("   " + " ".join(f"{e:.1e}" for e in errs))
    assert Y.shape == (B, L, H, N, D)
    assert max(errs) <= TOL[dtype]


CONSTS = dict(gating_c=math.log(2048), omega_thresh=math.sqrt(2 ** -7), adt_delta=16 * 2 ** -7,
              adt_smoothness=math.sqrt(2 ** -7) / 5, adt_eps=1.0)


@pytest.mark.parametrize("dtype,N", [(torch.float32, 2), (torch.float32, 16), (torch.bfloat16, 16)])
def test_dynamics_fused_fwd_bwd(dtype, N):
    from cdssm_hip.ops import DynamicsFusedFn
    log(f"[dynamics] {dtype} N{N}")
    gen = torch.Generator().manual_seed(5)
    B, L, H = 2, 300, 4
    gate = (torch.randn(B, L, (N + 5) * H, generator=gen) * 0.8).to(dtype)
    lds = torch.randn(H, generator=gen) * 0.5
    freqs = 1.0 / (2048.0 ** (torch.arange(H, dtype=torch.float32) / H))
    outs_ref = o.dynamics_fused_fwd(gate.double(), lds.double(), freqs.double(), n_heads=H, state_dim=N, **CONSTS)
    gs = [torch.randn(*t.shape, generator=gen).to(dtype) for t in outs_ref]
    gg_ref, gl_ref = o.dynamics_fused_bwd_ref(*[g.double() for g in gs], gate.double(), lds.double(),
                                              freqs.double(), n_heads=H, state_dim=N, **CONSTS)
    gd = gate.to(DEV).requires_grad_(True)
    ld = lds.to(DEV).requires_grad_(True)
    outs = DynamicsFusedFn.apply(gd, ld, freqs.to(DEV), CONSTS["gating_c"], CONSTS["omega_thresh"],
                                 CONSTS["adt_delta"], CONSTS["adt_smoothness"], CONSTS["adt_eps"], H, N)
    torch.autograd.backward(list(outs), [g.to(DEV) for g in gs])
    torch.cuda.synchronize()
    errs = [rel(x, y) for x, y in zip(outs, outs_ref)] + [rel(gd.grad, gg_ref), rel(ld.grad, gl_ref)]
    log("   " + " ".join(f"{e:.1e}" for e in errs))
    assert max(errs) <= TOL[dtype]


@pytest.mark.parametrize("dtype,D", [(torch.float32, 64), (torch.float32, 128), (torch.float32, 48),
                                     (torch.bfloat16, 64), (torch.bfloat16, 128)])
def test_normalize_kq_fwd_bwd_any_head_dim(dtype, D):
    from cdssm_hip.ops import NormalizeKQFn
    log(f"[normalize] {dtype} D{D}")
    gen = torch.Generator().manual_seed(6)
    K = torch.randn(3, 77, 5, D, generator=gen).to(dtype)
    Q = (torch.randn(3, 77, 5, D, generator=gen) * 3).to(dtype)
    gk = torch.randn(K.shape, generator=gen).to(dtype)
    gq = torch.randn(K.shape, generator=gen).to(dtype)
    kn_ref, qn_ref = o.normalize_kq(K.double(), Q.double())
    gk_ref, gq_ref = o.normalize_kq_bwd(gk.double(), gq.double(), K.double(), Q.double())
    k, q = dev(K, Q, req=True)
    kn, qn = NormalizeKQFn.apply(k, q)
    torch.autograd.backward([kn, qn], [gk.to(DEV), gq.to(DEV)])
    torch.cuda.synchronize()
    errs = [rel(kn, kn_ref), rel(qn, qn_ref), rel(k.grad, gk_ref), rel(q.grad, gq_ref)]
    log("   " + " ".join(f"{e:.1e}" for e in errs))
    assert max(errs) <= TOL[dtype]


def test_ops_reject_cpu_tensors_and_bad_state_dim():
    from cdssm_hip.ops import InterChunkScanFn, IntraChunkScanFn
    x = torch.zeros(1, 4, 2, 2)
    with pytest.raises(RuntimeError, match="GPU only"):
        InterChunkScanFn.apply(x, torch.zeros(1, 4, 2, 2, 8), 2)
    k = torch.zeros(2, 4, 1, 8, device=DEV)
    with pytest.raises(ValueError, match="state_dim"):
        IntraChunkScanFn.apply(torch.zeros(2, 4, 1, 3, device=DEV), k, torch.zeros(2, 4, 1, 3, device=DEV),
                               torch.zeros(2, 4, 1, device=DEV), 3)
