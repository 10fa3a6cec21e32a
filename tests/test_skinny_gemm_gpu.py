"""cdssm_skinny_gemm (decode-size linear layers) against a float32 reference.

The reference is the unfused computation the decode step would otherwise run:
the model's RMSNorm (x * rsqrt(mean(x^2) + eps), rounded to bf16, times the
norm weight, rounded again), then the product in float32 from the bf16
operands, plus bias and residual.  The kernel rounds x * w_norm (not the
normalised x) to bf16 and applies the row scale to the float32 result, so the
two differ by bf16 rounding of the operands: tolerance 1e-2 normwise on the
bf16 output (max |y - ref| / max |ref|), 5e-3 without the norm (the output's
rounding to bf16, up to half a unit in the last place = 2^-8 relative, and the
summation order).
"""

import pytest
import torch

from _gpu_util import DEV, log, rel

pytestmark = pytest.mark.gpu


def _reference(x, w, bias=None, residual=None, norm_weight=None, eps=0.0):
    x32 = x.float()
    if norm_weight is not None:
        xn = (x32 * torch.rsqrt(x32.pow(2).mean(-1, keepdim=True) + eps)).to(torch.bfloat16)
        x32 = (xn * norm_weight.to(torch.bfloat16)).float()
    y = x32 @ w.float().t()
    if bias is not None:
        y = y + bias.float()
    if residual is not None:
        y = y + residual.float()
    return y


@pytest.mark.parametrize("name,M,K,N,use_bias,use_res,use_norm", [
    ("in_proj + RMSNorm", 64, 1024, 3104, True, False, True),
    ("gate/Q stacked", 64, 1024, 1136, True, False, False),
    ("out_proj + residual", 64, 1024, 1024, False, True, False),
    ("tied head + RMSNorm", 64, 1024, 32000, False, False, True),
    ("ragged rows and columns", 7, 256, 45, True, True, True),
    ("K 2048 (d_inner of the reference config)", 64, 2048, 1024, False, True, False),
    ("K 384: four waves", 33, 384, 100, True, False, True),
    ("one row", 1, 128, 16, False, False, False),
])
def test_skinny_gemm_matches_fp32_reference(name, M, K, N, use_bias, use_res, use_norm):
    from cdssm_hip.lm import skinny_linear
    g = torch.Generator().manual_seed(M * 7 + N)
    x = (torch.randn(M, K, generator=g) * 2.0).to(torch.bfloat16)
    w = (torch.randn(N, K, generator=g) / K ** 0.5).to(torch.bfloat16)
    bias = (torch.randn(N, generator=g) * 0.1).to(torch.bfloat16) if use_bias else None
    res = torch.randn(M, N, generator=g).to(torch.bfloat16) if use_res else None
    nw = (1.0 + 0.1 * torch.randn(K, generator=g)).to(torch.bfloat16) if use_norm else None
    eps = 1e-5
    log(f"[skinny gemm] {name}: M{M} K{K} N{N}")
    y = skinny_linear(x.to(DEV), w.to(DEV), None if bias is None else bias.to(DEV),
                      None if res is None else res.to(DEV), None if nw is None else nw.to(DEV), eps)
    torch.cuda.synchronize()
    ref = _reference(x, w, bias, res, nw, eps)
    e = rel(y.float().cpu(), ref)
    log(f"   rel err {e:.2e}")
    assert e <= (1e-2 if use_norm else 5e-3), (name, e)


def test_skinny_gemm_strided_rows_and_graph_replay():
    """x a column slice of a wider buffer (row stride > K); the call captured in a HIP
    graph and replayed on rewritten inputs gives the eager result each time."""
    from cdssm_hip.lm import skinny_linear
    M, K, N = 64, 1024, 1136
    g = torch.Generator().manual_seed(3)
    buf = torch.randn(M, K + 128, generator=g).to(torch.bfloat16).to(DEV)
    x = buf[:, 128:]
    w = (torch.randn(N, K, generator=g) / K ** 0.5).to(torch.bfloat16).to(DEV)
    b = torch.randn(N, generator=g).to(torch.bfloat16).to(DEV)
    y_eager = skinny_linear(x, w, b)
    torch.cuda.synchronize()
    assert rel(y_eager.float().cpu(), _reference(x.cpu(), w.cpu(), b.cpu())) <= 5e-3
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        y_g = skinny_linear(x, w, b)
    for seed in (4, 5, 4):
        buf.copy_(torch.randn(M, K + 128, generator=torch.Generator().manual_seed(seed)).to(torch.bfloat16))
        graph.replay()
        torch.cuda.synchronize()
        ref = skinny_linear(x, w, b)
        torch.cuda.synchronize()
        assert torch.equal(y_g.cpu(), ref.cpu()), seed
    log("[skinny gemm] strided rows, graph replays equal eager calls")
