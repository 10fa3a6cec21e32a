"""Pins of the LM oracle (oracle/cdssm_lm_oracle.py), CPU only.

conv1d_silu is checked against torch.nn.functional.conv1d (causal padding,
groups = channels) + silu -- a library routine, so a reversed tap order or a
wrong causal offset fails; rms_norm against its closed form; block_forward and
lm_forward by invariants (a zero out_proj makes a block the identity; batch
rows are independent; the GroupNorm statistics span the sequence, as in the
reference) and by closed-form special cases of the block's wiring (zero
readout_proj, the value-residual lerp at its two ends, the shortcut's readout).
"""

import torch
import torch.nn.functional as F

from oracle import cdssm_lm_oracle as lo


def test_conv1d_silu_is_the_causal_depthwise_conv_of_the_library():
    g = torch.Generator().manual_seed(0)
    for K in (1, 2, 4, 7):
        x = torch.randn(2, 37, 6, generator=g, dtype=torch.float64)
        w = torch.randn(6, 1, K, generator=g, dtype=torch.float64)
        b = torch.randn(6, generator=g, dtype=torch.float64)
        ref = F.conv1d(x.transpose(1, 2), w, b, padding=K - 1, groups=6)[..., :37].transpose(1, 2)
        assert torch.allclose(lo.conv1d_silu(x, w, b), F.silu(ref), atol=1e-12, rtol=1e-12)


def test_rms_norm_closed_form():
    x = torch.tensor([[3.0, 4.0]], dtype=torch.float64)
    w = torch.tensor([2.0, 0.5], dtype=torch.float64)
    out = lo.rms_norm(x, w, 0.0)
    assert torch.allclose(out, torch.tensor([[6.0 / 12.5 ** 0.5, 2.0 / 12.5 ** 0.5]], dtype=torch.float64))


def _small_model(seed=0):
    from cdssm_hip.lm import CDSSMConfig, CDSSMLMHeadModel
    torch.manual_seed(seed)
    cfg = CDSSMConfig(d_model=64, n_layers=2, context_length=128, vocab_size=97, state_dim=2, d_inner=128)
    m = CDSSMLMHeadModel(cfg)
    p = {k: v.detach().double() for k, v in m.state_dict().items()}
    return cfg, p


def test_block_with_zero_out_proj_is_the_identity():
    cfg, p = _small_model()
    p["blocks.0.out_proj.weight"].zero_()
    x = torch.randn(1, 70, cfg.d_model, dtype=torch.float64)
    y, _ = lo.block_forward(p, "blocks.0.", x, None, cfg)
    assert torch.equal(y, x)


def test_lm_forward_rows_are_independent_and_groupnorm_spans_the_sequence():
    """Batch rows never mix.  Positions do: the reference normalises each group over
    (channels of the group) x (all L positions) (F.group_norm on (B, d_inner, L),
    block.py:216-223), so earlier outputs change when a later token changes -- the
    restatement must reproduce that, not a causal norm."""
    cfg, p = _small_model(1)
    ids = torch.randint(0, cfg.vocab_size, (2, 90))
    a = lo.lm_forward(p, ids, cfg)
    ids2 = ids.clone()
    ids2[1, 50:] = (ids2[1, 50:] + 1) % cfg.vocab_size
    b = lo.lm_forward(p, ids2, cfg)
    assert torch.equal(a[0], b[0])
    assert not torch.allclose(a[1, :50], b[1, :50])


def test_group_norm_running_sums_give_the_group_statistics():
    """The decode state's (shift, S1, S2, n) reproduce each group's mean and biased variance over all
    positions (torch's var on the (L, C/G) block), and appending a token's sums equals the sums of the
    longer sequence."""
    g = torch.Generator().manual_seed(9)
    y = torch.randn(2, 37, 24, generator=g, dtype=torch.float64) * 3 + 5
    s = lo.group_norm_running_sums(y, 4)
    blk = y.reshape(2, 37, 4, 6)
    mean = s[..., 0] + s[..., 1] / s[..., 3]
    var = s[..., 2] / s[..., 3] - (s[..., 1] / s[..., 3]) ** 2
    assert torch.allclose(mean, blk.mean((1, 3)), rtol=0, atol=1e-12)
    assert torch.allclose(var, blk.var((1, 3), unbiased=False), rtol=0, atol=1e-10)
    s36 = lo.group_norm_running_sums(y[:, :36], 4)
    d = y[:, 36].reshape(2, 4, 6) - s36[..., 0:1]
    step = torch.stack([s36[..., 0], s36[..., 1] + d.sum(-1), s36[..., 2] + (d * d).sum(-1), s36[..., 3] + 6], -1)
    assert torch.allclose(step, s, rtol=1e-12, atol=1e-10)


def test_block_with_zero_readout_is_the_closed_form_gate_path():
    """readout_proj = 0 makes the GroupNorm input zero, so GroupNorm returns its bias and the block is
    residual + out_proj(bias * silu(z) + D * x_conv), with z and x_gate the first two d_inner-wide
    slices of in_proj(RMSNorm(x)) (block.py:162-166) and x_conv = silu(causal depthwise conv(x_gate)).
    Built here from library routines (F.linear, F.conv1d, F.silu) -- a swapped split order, a missing
    D-skip or a gate on the wrong slice fails."""
    cfg, p = _small_model(2)
    pre = "blocks.1."
    g = torch.Generator().manual_seed(3)
    p[pre + "readout_proj.weight"].zero_()
    p[pre + "ssm_norm.bias"].copy_(torch.randn(cfg.d_inner, generator=g, dtype=torch.float64))
    p[pre + "D"].copy_(torch.randn(cfg.d_inner, generator=g, dtype=torch.float64))
    x = torch.randn(2, 40, cfg.d_model, generator=g, dtype=torch.float64)
    v_first = torch.randn(2, 40, cfg.n_heads, cfg.state_dim, generator=g, dtype=torch.float64)
    got, _ = lo.block_forward(p, pre, x, v_first, cfg)
    xn = x * torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + cfg.eps_norm) * p[pre + "norm.weight"]
    proj = F.linear(xn, p[pre + "in_proj.weight"], p[pre + "in_proj.bias"])
    Di = cfg.d_inner
    z, x_gate = proj[..., :Di], proj[..., Di:2 * Di]
    K = p[pre + "conv.weight"].shape[-1]
    xc = F.silu(F.conv1d(x_gate.transpose(1, 2), p[pre + "conv.weight"], p[pre + "conv.bias"], padding=K - 1,
                         groups=Di)[..., :40].transpose(1, 2))
    y = p[pre + "ssm_norm.bias"] * F.silu(z) + p[pre + "D"] * xc
    want = x + F.linear(y, p[pre + "out_proj.weight"])
    assert torch.allclose(got, want, rtol=1e-10, atol=1e-10)


def test_value_residual_lerp_direction():
    """V = lerp(v_first, V_own, sigmoid(gate)) (block.py:169-174): with sigmoid(gate) = 0 exactly the block
    ignores its own V slice of in_proj (the last H*N rows) and uses v_first; with sigmoid(gate) = 1 it
    ignores v_first.  Reversing the lerp flips both."""
    cfg, p = _small_model(4)
    pre = "blocks.1."
    g = torch.Generator().manual_seed(5)
    HN = cfg.n_heads * cfg.state_dim
    x = torch.randn(1, 33, cfg.d_model, generator=g, dtype=torch.float64)
    v1 = torch.randn(1, 33, cfg.n_heads, cfg.state_dim, generator=g, dtype=torch.float64)
    v2 = torch.randn(1, 33, cfg.n_heads, cfg.state_dim, generator=g, dtype=torch.float64)
    p2 = dict(p)
    p2[pre + "in_proj.weight"] = p[pre + "in_proj.weight"].clone()
    p2[pre + "in_proj.weight"][-HN:] = torch.randn(HN, cfg.d_model, generator=g, dtype=torch.float64)
    p[pre + "v_residual_gate"].fill_(-1e4)       # sigmoid -> 0.0 exactly in fp64
    p2[pre + "v_residual_gate"] = p[pre + "v_residual_gate"]
    a, _ = lo.block_forward(p, pre, x, v1, cfg)
    b, _ = lo.block_forward(p2, pre, x, v1, cfg)
    assert torch.equal(a, b)                     # own V unused
    c, _ = lo.block_forward(p, pre, x, v2, cfg)
    assert not torch.allclose(a, c)              # v_first used
    p[pre + "v_residual_gate"].fill_(1e4)        # sigmoid -> 1.0
    a, _ = lo.block_forward(p, pre, x, v1, cfg)
    c, _ = lo.block_forward(p, pre, x, v2, cfg)
    assert torch.equal(a, c)                     # v_first unused


def test_shortcut_through_the_readout_is_sel_c_times_qk_squared_v():
    """The reference adds s (q.k) V_gated k^T to the (B,L,H,N,D) state and reads it with q (block.py:202-211);
    read out, that term is sel_C s (q.k)^2 V_gated -- the closed form the fused kernels use."""
    from oracle import cdssm_oracle as o
    g = torch.Generator().manual_seed(6)
    B, L, H, N, D = 2, 5, 3, 4, 8
    Y = torch.randn(B, L, H, N, D, generator=g, dtype=torch.float64)
    q = torch.randn(B, L, H, D, generator=g, dtype=torch.float64)
    k = torch.randn(B, L, H, D, generator=g, dtype=torch.float64)
    v = torch.randn(B, L, H, N, generator=g, dtype=torch.float64)
    sel = torch.rand(B, L, H, generator=g, dtype=torch.float64)
    got = o.readout(Y, q, sel, K=k, V_gated=v, shortcut_scale=0.37)
    qk = (q * k).sum(-1)
    want = sel[..., None] * ((Y * q[..., None, :]).sum(-1) + 0.37 * (qk * qk)[..., None] * v)
    assert torch.allclose(got, want, rtol=1e-12, atol=1e-12)
