"""GPU parity of the fused SSDChunkwiseScan (cdssm_ssd_scan_fwd / cdssm_ssd_scan_bwd).

The reference is the oracle's fp64 restatement of ssd.py:39-111 with the
reference's correction backward attached (exact_correction.cu:213-382), on the
same inputs rounded to the tested dtype and the same cotangent dY.  Tolerances,
normwise max|x-ref|/max|ref| per tensor: fp32 1e-4, bf16 2e-2.
"""

import contextlib
import math

import pytest
import torch

from _gpu_util import DEV, log, rel
from oracle import cdssm_oracle as o

pytestmark = pytest.mark.gpu
TOL = {torch.float32: 1e-4, torch.bfloat16: 2e-2}


def rand_ssd(gen, B, L, H, D, amax=1.0, amin=0.0, N=2):
    """A_bar (N / 2 complex pairs per head) of magnitude in [amin, amax) and uniform phase, unit-norm
    keys, N(0,1) values, beta in [0, 1)."""
    ang = torch.rand(B, L, H, N // 2, generator=gen) * 2 * math.pi
    mag = amin + torch.rand(B, L, H, N // 2, generator=gen) * (amax - amin)
    A = torch.stack([mag * torch.cos(ang), mag * torch.sin(ang)], -1).flatten(-2)
    K = torch.randn(B, L, H, D, generator=gen)
    K = K / K.norm(dim=-1, keepdim=True)
    V = torch.randn(B, L, H, N, generator=gen)
    beta = torch.rand(B, L, H, generator=gen)
    return A, K, V, beta


@contextlib.contextmanager
def forward_path(path):
    from cdssm_hip import set_forward_path
    prev = set_forward_path(path)
    try:
        yield
    finally:
        set_forward_path(prev)


def fused_grads(A, K, V, beta, gY, Q):
    from cdssm_hip import SSDScanFn
    leaves = [t.to(DEV).requires_grad_(True) for t in (A, K, V, beta)]
    Y = SSDScanFn.apply(*leaves, Q)
    Y.backward(gY.to(DEV, Y.dtype))
    torch.cuda.synchronize()
    return Y.detach().cpu(), [x.grad.cpu() for x in leaves]


def oracle_grads(A, K, V, beta, gY, Q):
    leaves = [t.double().requires_grad_(True) for t in (A, K, V, beta)]
    Y = o.ssd_chunkwise_scan(*leaves, Q, V.shape[-1], correction_fn=o.correction_with_reference_grad)
    g = torch.autograd.grad((Y * gY.double()).sum(), leaves)
    return Y.detach(), list(g)


CASES = [
    # name, dtype, B, L, H, D, Q, amax
    ("fp32_D64", torch.float32, 2, 256, 4, 64, 64, 0.99),
    ("fp32_ragged_H5", torch.float32, 2, 300, 5, 64, 64, 0.99),
    ("fp32_D128_chunk48", torch.float32, 1, 333, 3, 128, 48, 0.99),
    ("fp32_small_a", torch.float32, 1, 256, 4, 64, 64, 0.05),
    ("bf16_D64", torch.bfloat16, 2, 512, 16, 64, 64, 0.99),
    ("bf16_D128_ragged", torch.bfloat16, 1, 700, 6, 128, 128, 0.99),
    ("bf16_chunk20", torch.bfloat16, 1, 200, 3, 64, 20, 0.99),
]


@pytest.mark.parametrize("path", ["four_launch", "one_pass"])
@pytest.mark.parametrize("name,dtype,B,L,H,D,Q,amax", CASES, ids=[c[0] for c in CASES])
def test_fused_ssd_matches_oracle(name, dtype, B, L, H, D, Q, amax, path):
    """Y and dA_bar, dK, dV, dbeta on both forward paths (the backward's carry takes its three-launch
    form with four_launch, its one-launch form with one_pass)."""
    log(f"[fused SSD] {name} B{B} L{L} H{H} D{D} Q{Q} path {path}")
    gen = torch.Generator().manual_seed(11)
    A, K, V, beta = [t.to(dtype) for t in rand_ssd(gen, B, L, H, D, amax=amax)]
    gY = torch.randn(B, L, H, 2, D, generator=gen).to(dtype)
    Y_ref, g_ref = oracle_grads(A, K, V, beta, gY, Q)
    with forward_path(path):
        Y, g = fused_grads(A, K, V, beta, gY, Q)
    from cdssm_hip import lookback_status
    assert lookback_status() == 0, "a look-back wait timed out"
    errs = {"Y": rel(Y, Y_ref)}
    errs.update({n: rel(x, y) for n, x, y in zip(("dA", "dK", "dV", "dbeta"), g, g_ref)})
    log("   " + "  ".join(f"{n} {e:.1e}" for n, e in errs.items()))
    assert Y.shape == (B, L, H, 2, D) and Y.dtype == dtype
    assert all(e <= TOL[dtype] for e in errs.values()), errs


def test_fused_ssd_c1_shape_matches_oracle_and_per_pass():
    """The C1 shape (B8 H16 L4096 D64 bf16): the fused module against the oracle on one batch row and
    two heads, and against the per-pass ops on everything (the per-pass ops round local_h,
    chunk_states and corrections to bf16 between passes, as the reference does, so the two agree to
    bf16 accuracy)."""
    from cdssm_hip.ssd import SSDChunkwiseScan
    log("[fused SSD C1] B8 H16 L4096 D64 bf16")
    gen = torch.Generator().manual_seed(2)
    B, L, H, D, Q = 8, 4096, 16, 64, 64
    A, K, V, beta = [t.to(torch.bfloat16) for t in rand_ssd(gen, B, L, H, D, amax=0.99, amin=0.5)]
    gY = torch.randn(B, L, H, 2, D, generator=gen).to(torch.bfloat16)
    Y, g = fused_grads(A, K, V, beta, gY, Q)
    b, heads = 5, torch.tensor([3, 12])
    sel = lambda t: t[b:b + 1].index_select(2, heads)  # noqa: E731
    Y_ref, g_ref = oracle_grads(*[sel(t) for t in (A, K, V, beta)], sel(gY), Q)
    errs = {"Y": rel(sel(Y), Y_ref)}
    errs.update({n: rel(sel(x), y) for n, x, y in zip(("dA", "dK", "dV", "dbeta"), g, g_ref)})
    log("   oracle: " + "  ".join(f"{n} {e:.1e}" for n, e in errs.items()))
    assert all(e <= 2e-2 for e in errs.values()), errs
    leaves = [t.to(DEV).requires_grad_(True) for t in (A, K, V, beta)]
    Yp = SSDChunkwiseScan(Q, 2, fused=False)(*leaves)
    Yp.backward(gY.to(DEV))
    torch.cuda.synchronize()
    perr = {"Y": rel(Y, Yp)}
    perr.update({n: rel(x, y.grad) for n, x, y in zip(("dA", "dK", "dV", "dbeta"), g, leaves)})
    log("   per-pass: " + "  ".join(f"{n} {e:.1e}" for n, e in perr.items()))
    assert all(e <= 2e-2 for e in perr.values()), perr


def test_fused_ssd_one_launch_past_the_anchor_matches_oracle():
    """B1 H4 L19200 D64 bf16 forced onto the one-launch paths: 300 chunks = 75 segments, so the
    forward and the backward carry both fold from published anchor states (every 63 segments)."""
    log("[fused SSD anchor] B1 H4 L19200 D64 bf16 one_pass")
    gen = torch.Generator().manual_seed(5)
    B, L, H, D, Q = 1, 19200, 4, 64, 64
    A, K, V, beta = [t.to(torch.bfloat16) for t in rand_ssd(gen, B, L, H, D, amax=0.999, amin=0.9)]
    gY = torch.randn(B, L, H, 2, D, generator=gen).to(torch.bfloat16)
    with forward_path("one_pass"):
        Y, g = fused_grads(A, K, V, beta, gY, Q)
    from cdssm_hip import lookback_status
    assert lookback_status() == 0, "a look-back wait timed out"
    heads = torch.tensor([0, 3])
    sel = lambda t: t.index_select(2, heads)  # noqa: E731
    Y_ref, g_ref = oracle_grads(*[sel(t) for t in (A, K, V, beta)], sel(gY), Q)
    errs = {"Y": rel(sel(Y), Y_ref)}
    errs.update({n: rel(sel(x), y) for n, x, y in zip(("dA", "dK", "dV", "dbeta"), g, g_ref)})
    log("   " + "  ".join(f"{n} {e:.1e}" for n, e in errs.items()))
    assert all(e <= 2e-2 for e in errs.values()), errs


ROW_CASES = [
    # name, dtype, N, B, L, H, D, Q
    ("fp32_N4_D64", torch.float32, 4, 2, 300, 3, 64, 64),
    # 6 rows per head: not a multiple of the backward's 4 heads per wave (its dK partials stay per row)
    ("fp32_N12_D64", torch.float32, 12, 1, 200, 2, 64, 64),
    ("fp32_N16_D64", torch.float32, 16, 1, 256, 2, 64, 64),
    ("fp32_N16_D128_chunk48", torch.float32, 16, 1, 200, 3, 128, 48),
    ("bf16_N16_D64", torch.bfloat16, 16, 2, 512, 4, 64, 64),
    ("bf16_N8_D128_ragged", torch.bfloat16, 8, 1, 333, 5, 128, 128),
    ("bf16_N32_D64", torch.bfloat16, 32, 1, 256, 2, 64, 64),
]


@pytest.mark.parametrize("path", ["four_launch", "one_pass"])
@pytest.mark.parametrize("name,dtype,N,B,L,H,D,Q", ROW_CASES, ids=[c[0] for c in ROW_CASES])
def test_fused_ssd_state_rows_match_oracle(name, dtype, N, B, L, H, D, Q, path):
    """state_dim N > 2 (the reference default is 16): the N / 2 complex rows of each head run as
    virtual heads sharing the head's k and beta; Y and every gradient against the oracle's
    ssd_chunkwise_scan at that N (dK and dbeta sum the rows' contributions)."""
    log(f"[fused SSD rows] {name} N{N} B{B} L{L} H{H} D{D} Q{Q} path {path}")
    gen = torch.Generator().manual_seed(21)
    A, K, V, beta = [t.to(dtype) for t in rand_ssd(gen, B, L, H, D, amax=0.99, N=N)]
    gY = torch.randn(B, L, H, N, D, generator=gen).to(dtype)
    Y_ref, g_ref = oracle_grads(A, K, V, beta, gY, Q)
    with forward_path(path):
        Y, g = fused_grads(A, K, V, beta, gY, Q)
    from cdssm_hip import lookback_status
    assert lookback_status() == 0, "a look-back wait timed out"
    errs = {"Y": rel(Y, Y_ref)}
    errs.update({n: rel(x, y) for n, x, y in zip(("dA", "dK", "dV", "dbeta"), g, g_ref)})
    log("   " + "  ".join(f"{n} {e:.1e}" for n, e in errs.items()))
    assert Y.shape == (B, L, H, N, D)
    assert all(e <= TOL[dtype] for e in errs.values()), errs


@pytest.mark.parametrize("N,L", [(2, 256), (2, 300), (16, 200)])
def test_fused_ssd_final_state_matches_oracle(N, L):
    """h_final (B,H,N,D) fp32 of cdssm_ssd_scan_fwd: the R-mode carry after the last token, against the
    oracle's return_final (equal to the state after the last chunk when L is a multiple of the chunk)."""
    from cdssm_hip.scan import ssd_scan_fwd
    gen = torch.Generator().manual_seed(31)
    B, H, D, Q = 2, 3, 64, 64
    A, K, V, beta = rand_ssd(gen, B, L, H, D, amax=0.99, N=N)
    with torch.no_grad():
        _, hf, _ = ssd_scan_fwd(*[t.to(DEV) for t in (A, K, V, beta)], Q)
    torch.cuda.synchronize()
    _, h_ref = o.ssd_chunkwise_scan(*[t.double() for t in (A, K, V, beta)], Q, N, return_final=True)
    e = rel(hf, h_ref)
    log(f"[fused SSD h_final] N{N} L{L}: rel err {e:.1e}")
    assert hf.shape == (B, H, N, D) and e <= 1e-4


def test_fused_ssd_inference_call_keeps_no_records_and_matches_training_forward():
    """Without gradients the forward runs without the training records; Y is the same (bit-identical)
    as the training forward's."""
    from cdssm_hip import SSDScanFn
    gen = torch.Generator().manual_seed(9)
    A, K, V, beta = [t.to(torch.bfloat16).to(DEV) for t in rand_ssd(gen, 2, 640, 8, 64, amax=0.99)]
    with torch.no_grad():
        Y0 = SSDScanFn.apply(A, K, V, beta, 64)
    leaves = [t.clone().requires_grad_(True) for t in (A, K, V, beta)]
    Y1 = SSDScanFn.apply(*leaves, 64)
    torch.cuda.synchronize()
    assert torch.equal(Y0, Y1.detach())


def test_fused_ssd_rejects_what_it_cannot_serve():
    from cdssm_hip.ssd import SSDChunkwiseScan
    gen = torch.Generator().manual_seed(1)
    A, K, V, beta = [t.to(DEV) for t in rand_ssd(gen, 1, 64, 2, 48)]
    with pytest.raises(ValueError, match="head_dim"):
        SSDChunkwiseScan(64, 2, fused=True)(A, K, V, beta)
    # the module's own choice falls back to the per-pass ops for such a shape
    Y = SSDChunkwiseScan(64, 2)(A, K, V, beta)
    assert Y.shape == (1, 64, 2, 2, 48)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_captured_ssd_forward_and_backward_replays_match_oracle(dtype):
    """The SSD form's training forward and backward captured in one HIP graph, both on their
    one-launch paths (B2 H5 L1317 D64: 21 chunks, 6 look-back segments per sequence); inputs and dY
    rewritten in place between replays; every replay checked against the oracle and, bit for bit,
    against an eager call on the same inputs."""
    from cdssm_hip import lookback_status
    from cdssm_hip.scan import ssd_scan_bwd, ssd_scan_fwd
    B, L, H, D, Q = 2, 64 * 4 * 5 + 37, 5, 64, 64
    log(f"[graph SSD fwd+bwd] B{B} L{L} H{H} D{D} {dtype}, one-launch paths captured")

    def draw(seed):
        gen = torch.Generator().manual_seed(seed)
        A, K, V, beta = rand_ssd(gen, B, L, H, D, amax=0.99)
        gY = torch.randn(B, L, H, 2, D, generator=gen)
        return [t.to(dtype) for t in (A, K, V, beta, gY)]

    static = [t.to(DEV) for t in draw(0)]

    def step():
        Y, _, ws = ssd_scan_fwd(*static[:4], Q, train=True)
        return Y, ssd_scan_bwd(static[4], *static[:4], ws, Q)

    with forward_path("one_pass"):
        step()  # eager call first: fills the launchers' occupancy caches outside capture
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            Yc, gc = step()
    torch.cuda.synchronize()
    tol = TOL[dtype]
    for seed in (4, 5, 6):
        x = draw(seed)
        for dst, src in zip(static, x):
            dst.copy_(src.to(DEV))
        graph.replay()
        torch.cuda.synchronize()
        Y, g = Yc.cpu().clone(), [t.cpu().clone() for t in gc]
        Y_ref, g_ref = oracle_grads(*x[:4], x[4], Q)
        errs = {"Y": rel(Y, Y_ref)}
        errs.update({n: rel(a, b) for n, a, b in zip(("dA", "dK", "dV", "dbeta"), g, g_ref)})
        log(f"   replay seed {seed}: " + "  ".join(f"{n} {e:.1e}" for n, e in errs.items()))
        assert all(e <= tol for e in errs.values()), (seed, errs)
        with forward_path("one_pass"):
            Ye, ge = step()
        torch.cuda.synchronize()
        assert torch.equal(Ye.cpu(), Y) and all(torch.equal(a.cpu(), b) for a, b in zip(ge, g)), \
            f"eager != replay (seed {seed})"
    assert lookback_status() == 0, "a look-back wait timed out"
