"""GPU parity of the chunked (UT) N = 16 readout form on the matrix cores (cdssm_chunked_scan_fwd_abar).

The block at the reference's default state_dim 16 runs SSDChunkwiseScan(A_bar, K, V * vp, beta)
(ssd.py:39-111) and reads it out as sel_C (Y . q) (block.py:194-211).  Here A_bar (B,L,H,16),
v (B,L,H,16) and vp (B,L,H,8) are drawn directly, rounded once to bf16, and the HIP result is compared
with the oracle's ssd_chunkwise_scan + readout in fp64 on the same rounded values.  Heads with strong
decay (|a| <= 0.02, so a 16-token product falls below 2^-48) run the kernel's true-units blocks; the
others its rescaled blocks; a token with a = 0 exactly is included.  Tolerances (bf16 inputs, fp32
state): y <= 2e-2 normwise, final-state norms <= 1e-3.  Cases with a shortcut scale also check the
current-token shortcut folded into y (block.py:202-208).
"""

import math

import pytest
import torch

from _gpu_util import DEV, log, rel, state_norm_rel
from oracle import cdssm_oracle as o

pytestmark = pytest.mark.gpu


def draw(B, L, H, D, N=16, seed=0, strong_heads=(), h0_std=0.0):
    g = torch.Generator().manual_seed(seed)
    R = N // 2
    ang = torch.rand(B, L, H, R, generator=g) * 2 * math.pi
    mag = 0.5 + 0.49 * torch.rand(B, L, H, R, generator=g)
    for h in strong_heads:
        mag[:, :, h] = 0.02 * torch.rand(B, L, R, generator=g)
    if strong_heads:
        mag[0, min(L - 1, 5), strong_heads[0], 0] = 0.0     # a = 0 exactly
    A = torch.stack([mag * torch.cos(ang), mag * torch.sin(ang)], -1).flatten(-2)
    k = torch.randn(B, L, H, D, generator=g)
    q = torch.randn(B, L, H, D, generator=g)
    x = dict(A_bar=A, k=k / k.norm(dim=-1, keepdim=True), q=q / q.norm(dim=-1, keepdim=True),
             v=torch.randn(B, L, H, N, generator=g), vp=torch.rand(B, L, H, R, generator=g),
             beta=torch.sigmoid(torch.randn(B, L, H, generator=g)),
             sel_C=torch.sigmoid(torch.randn(B, L, H, generator=g)))
    x = {n: t.to(torch.bfloat16) for n, t in x.items()}
    x["h0"] = h0_std * torch.randn(B, H, N, D, generator=g) if h0_std else None
    return x


def oracle_of(x, chunk, bsel, hsel, shortcut=0.0):
    sl = lambda t: t.double()[bsel][:, :, hsel]  # noqa: E731
    N = x["v"].shape[-1]
    Vg = sl(x["v"]) * sl(x["vp"]).repeat_interleave(2, dim=-1)
    h0 = x["h0"].double()[bsel][:, hsel] if x["h0"] is not None else None
    Y, hr = o.ssd_chunkwise_scan(sl(x["A_bar"]), sl(x["k"]), Vg, sl(x["beta"]), chunk, N, h0=h0, return_final=True)
    return o.readout(Y, sl(x["q"]), sl(x["sel_C"]), K=sl(x["k"]), V_gated=Vg, shortcut_scale=shortcut), hr


CASES = [
    # name, B, L, H, D, chunk, strong-decay heads, h0 std, shortcut scale
    ("D64_chunk64_ragged_h0", 2, 300, 4, 64, 64, (), 0.1, None),
    ("D64_strong_decay_heads", 1, 256, 4, 64, 64, (1, 3), 0.0, None),
    ("D64_chunk16_shortcut", 1, 100, 2, 64, 16, (1,), 0.1, 0.7),
    ("D64_chunk48_items_not_multiple_of_4", 1, 130, 3, 64, 48, (), 0.0, None),
    ("D128_chunk64_shortcut", 1, 200, 3, 128, 64, (2,), 0.1, -1.3),
    ("D128_chunk128", 2, 300, 2, 128, 128, (), 0.0, None),
    ("D64_chunk256", 1, 600, 2, 64, 256, (0,), 0.0, None),
    ("C4_shape_B8_L2048_H16_shortcut", 8, 2048, 16, 64, 64, (5,), 0.0, 0.5),
]


@pytest.mark.parametrize("name,B,L,H,D,chunk,strong,h0_std,scut", CASES, ids=[c[0] for c in CASES])
def test_chunked_scan_matches_oracle(name, B, L, H, D, chunk, strong, h0_std, scut):
    from cdssm_hip import chunked_scan_abar
    log(f"[chunked N16] {name}: B{B} L{L} H{H} D{D} chunk={chunk} strong={strong} shortcut={scut}")
    x = draw(B, L, H, D, seed=3, strong_heads=strong, h0_std=h0_std)
    g = {n: (t.to(DEV) if t is not None else None) for n, t in x.items()}
    sc = torch.tensor([scut], device=DEV) if scut is not None else None
    y, hf = chunked_scan_abar(g["q"], g["k"], g["v"], g["beta"], g["sel_C"], g["A_bar"], g["vp"], h0=g["h0"],
                              chunk_size=chunk, shortcut_scale=sc)
    torch.cuda.synchronize()
    y, hf = y.cpu(), hf.cpu()
    assert torch.isfinite(y.float()).all() and torch.isfinite(hf).all()
    bsel = [0, B - 1] if B > 2 else list(range(B))
    hsel = sorted({0, H - 1, *strong}) if H > 4 else list(range(H))
    yr, hr = oracle_of(x, chunk, bsel, hsel, shortcut=scut or 0.0)
    ys, hs = y[bsel][:, :, hsel], hf[bsel][:, hsel]
    ey, eh, en = rel(ys, yr), rel(hs, hr), state_norm_rel(hs, hr)
    log(f"   rel err y {ey:.2e}  h_final {eh:.2e}  state-norm {en:.2e}")
    assert ey <= 2e-2 and en <= 1e-3


def test_chunked_scan_is_deterministic_and_matches_the_ssd_form():
    """Two calls give bit-identical outputs; and the readout of the fused SSD form's Y (cdssm_ssd_scan_fwd,
    the drop-in SSDChunkwiseScan) on the same inputs agrees to the bf16 rounding of that Y."""
    from cdssm_hip import chunked_scan_abar
    from cdssm_hip.ssd import SSDChunkwiseScan
    B, L, H, D = 2, 512, 8, 64
    x = draw(B, L, H, D, seed=5, strong_heads=(2,))
    g = {n: (t.to(DEV) if t is not None else None) for n, t in x.items()}
    args = [g[n] for n in ("q", "k", "v", "beta", "sel_C", "A_bar", "vp")]
    y1, h1 = chunked_scan_abar(*args)
    y2, h2 = chunked_scan_abar(*args)
    torch.cuda.synchronize()
    assert torch.equal(y1, y2) and torch.equal(h1, h2)
    Vg = (g["v"].float() * g["vp"].float().repeat_interleave(2, dim=-1)).to(torch.bfloat16)
    with torch.no_grad():
        Y = SSDChunkwiseScan(D, 16)(g["A_bar"], g["k"], Vg, g["beta"])
    ys = (Y.float() * g["q"].float().unsqueeze(-2)).sum(-1) * g["sel_C"].float().unsqueeze(-1)
    e = rel(y1.float().cpu(), ys.cpu())
    log(f"   chunked vs SSD form + readout: {e:.2e}")
    assert e <= 2e-2


def test_chunked_scan_rejects_unsupported_inputs():
    from cdssm_hip import chunked_scan_abar
    x = draw(1, 64, 2, 64)
    g = {n: (t.to(DEV) if t is not None else None) for n, t in x.items()}
    args = [g[n] for n in ("q", "k", "v", "beta", "sel_C", "A_bar", "vp")]
    with pytest.raises(ValueError):
        chunked_scan_abar(*args, chunk_size=40)   # not a multiple of 16
    with pytest.raises(TypeError):
        chunked_scan_abar(*[t.float() for t in args])   # fp32 inputs
