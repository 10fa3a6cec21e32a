"""GPU parity of generation without re-forwarding (CDSSMLMHeadModel.prefill /
decode_step) and of its per-token kernels, against the forward over the prompt
plus the new tokens (the reference's way to generate, predict.py:53-67):

  * cdssm_conv1d_silu_step  == the full conv at each position (same tap order)
  * cdssm_dynamics_fused_fwd_at at position t == the full-sequence dynamics' row t
  * cdssm_decode_step_abar (after prefill_abar) == chunkwise_delta_scan_abar over
    the whole sequence, across chunk boundaries and from ragged prompt lengths
  * cdssm_group_norm_gate_step with the prompt's running sums == the GroupNorm
    epilogue over prompt + token, at the token
  * a one-layer model's decode-step logits == its forward's logits at the new
    position.  With more layers the reference's GroupNorm (statistics over all L
    positions, block.py:216-223) makes every earlier position of layers >= 2
    change when a token is appended; a recurrent step cannot revisit them, so
    there the test only reports the difference.

Tolerances (normwise): fp32 1e-5 for the exact-order kernels, 1e-4 for the scan
and the model (different summation orders), bf16 2e-2.
"""

import pytest
import torch

from _gpu_util import DEV, log, rel

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("dtype,B,L,C,K", [(torch.float32, 2, 40, 24, 4), (torch.bfloat16, 3, 9, 1024, 4),
                                           (torch.float32, 1, 5, 8, 1), (torch.float32, 2, 3, 16, 8)])
def test_conv_step_matches_full_conv(dtype, B, L, C, K):
    from cdssm_hip.lm import conv1d_silu, conv1d_silu_step
    log(f"[conv step] {dtype} B{B} L{L} C{C} K{K}")
    g = torch.Generator().manual_seed(11)
    x = torch.randn(B, L, C + 6, generator=g, dtype=torch.float32).to(dtype).to(DEV)[..., 3:3 + C]
    w = (torch.randn(C, 1, K, generator=g, dtype=torch.float32) / K ** 0.5).to(dtype).to(DEV)
    b = torch.randn(C, generator=g, dtype=torch.float32).to(dtype).to(DEV)
    full = conv1d_silu(x, w, b)
    win = torch.zeros(B, K - 1, C, dtype=dtype, device=DEV)
    ys = torch.stack([conv1d_silu_step(x[:, t], win, w, b) for t in range(L)], dim=1)
    e = rel(ys, full)
    log(f"   rel err {e:.2e}")
    assert e <= (1e-6 if dtype == torch.float32 else 1e-2)


def _cfg(dtype, d_model=128, n_layers=1, d_inner=128, L_ctx=512, vocab=97):
    from cdssm_hip.lm import CDSSMConfig, CDSSMLMHeadModel
    torch.manual_seed(0)
    cfg = CDSSMConfig(d_model=d_model, n_layers=n_layers, context_length=L_ctx, vocab_size=vocab, state_dim=2,
                      d_inner=d_inner)
    m = CDSSMLMHeadModel(cfg)
    with torch.no_grad():  # exercise the value-residual, shortcut and skip paths (zero at init)
        for blk in m.blocks:
            blk.v_residual_gate.normal_(std=1.0)
            blk.shortcut_scale.fill_(0.3)
            blk.D.normal_(std=0.1)
    return cfg, m.to(dtype).to(DEV).eval()


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_dynamics_at_position(dtype):
    from cdssm_hip.lm import dynamics_at
    from cdssm_hip.ops import DynamicsFusedFn
    cfg, m = _cfg(dtype)
    blk = m.blocks[0]
    H, N = cfg.n_heads, cfg.state_dim
    log(f"[dynamics at position] {dtype} H{H}")
    g = torch.Generator().manual_seed(12)
    gates = torch.randn(2, 70, (N + 5) * H, generator=g, dtype=torch.float32).to(dtype).to(DEV)
    args = (blk.log_dt_scale.float(), blk.rope_freqs, cfg.gating_c, cfg.bf16_omega_thresh, cfg.bf16_delta,
            cfg.bf16_smoothness, cfg.eps_adaptive_dt, H, N)
    full = DynamicsFusedFn.apply(gates, *args)
    for t in (0, 1, 63, 69):
        one = dynamics_at(gates[:, t:t + 1], *args, t)
        for a, b in zip(one, full):
            assert torch.equal(a[:, 0], b[:, t])


@pytest.mark.parametrize("dtype,B,H,L0,T", [(torch.float32, 2, 3, 64, 70), (torch.float32, 1, 2, 37, 30),
                                             (torch.bfloat16, 2, 4, 128, 3), (torch.float32, 1, 1, 0, 5)])
def test_decode_abar_matches_scan(dtype, B, H, L0, T):
    """prefill_abar over L0 tokens, then T decode steps == the chunked scan over L0 + T tokens."""
    from cdssm_hip.decode import decode_step_abar, prefill_abar
    from cdssm_hip.scan import chunkwise_delta_scan_abar
    D, L = 64, L0 + T
    log(f"[decode abar] {dtype} B{B} H{H} prompt {L0} steps {T}")
    g = torch.Generator().manual_seed(13)
    f32 = dict(generator=g, dtype=torch.float32)
    q = torch.nn.functional.normalize(torch.randn(B, L, H, D, **f32), dim=-1)
    k = torch.nn.functional.normalize(torch.randn(B, L, H, D, **f32), dim=-1)
    v = torch.randn(B, L, H, 2, **f32)
    beta = torch.sigmoid(torch.randn(B, L, H, **f32))
    sel = torch.sigmoid(torch.randn(B, L, H, **f32))
    ang = torch.randn(B, L, H, **f32)
    mag = 0.6 + 0.4 * torch.rand(B, L, H, **f32)
    A = torch.stack([mag * torch.cos(ang), mag * torch.sin(ang)], dim=-1)
    vp = torch.sqrt(1 - mag ** 2).unsqueeze(-1)
    ins = [x.to(dtype).to(DEV) for x in (q, k, v, beta, sel, A, vp)]
    y_full, _ = chunkwise_delta_scan_abar(*ins)
    if L0 > 0:
        y0, st = prefill_abar(*[x[:, :L0] for x in ins])
        assert rel(y0, y_full[:, :L0]) <= (1e-4 if dtype == torch.float32 else 2e-2)
    else:
        from cdssm_hip.decode import DecodeState
        st = DecodeState.at_boundary(None, B, H, D, D, DEV)
    ys = torch.stack([decode_step_abar(st, *[x[:, t] for x in ins]) for t in range(L0, L)], dim=1)
    e = rel(ys, y_full[:, L0:])
    log(f"   rel err {e:.2e}")
    assert e <= (1e-4 if dtype == torch.float32 else 2e-2)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_group_norm_step_matches_forward(dtype):
    from cdssm_hip.lm import group_norm_gate, group_norm_gate_step
    from oracle.cdssm_lm_oracle import group_norm_running_sums
    B, L, C, G = 2, 90, 128, 32
    log(f"[group norm step] {dtype} B{B} L{L} C{C} G{G}")
    g = torch.Generator().manual_seed(14)
    f32 = dict(generator=g, dtype=torch.float32)
    y = (torch.randn(B, L + 2, C, **f32) * 2 + 1).to(dtype).to(DEV)
    z = torch.randn(B, L + 2, C + 8, **f32).to(dtype).to(DEV)[..., 8:]
    xc = torch.randn(B, L + 2, C, **f32).to(dtype).to(DEV)
    gamma = (1 + 0.2 * torch.randn(C, **f32)).to(DEV)
    beta = (0.1 * torch.randn(C, **f32)).to(DEV)
    Dp = (0.3 * torch.randn(C, **f32)).to(dtype).to(DEV)
    gs = group_norm_running_sums(y[:, :L], G).float().contiguous()
    # the prefill's sums from the fused kernel's partials agree with the fp64 restatement
    _, gk = group_norm_gate(y[:, :L], G, gamma, beta, 1e-5, z[:, :L], xc[:, :L].contiguous(), Dp, return_sums=True)
    log(f"   kernel sums vs fp64 sums {rel(gk, gs):.2e}")
    assert rel(gk, gs) <= 1e-5
    for t in (L, L + 1):
        out = group_norm_gate_step(y[:, t], gs, gamma, beta, 1e-5, z[:, t], xc[:, t], Dp)
        ref = group_norm_gate(y[:, :t + 1], G, gamma, beta, 1e-5, z[:, :t + 1], xc[:, :t + 1].contiguous(), Dp)[:, t]
        e = rel(out, ref)
        log(f"   token {t}: rel err {e:.2e}")
        assert e <= (1e-5 if dtype == torch.float32 else 2e-2)


@pytest.mark.parametrize("dtype,B,K,C,G", [(torch.float32, 3, 32, 128, 32), (torch.bfloat16, 64, 32, 1024, 32),
                                        (torch.bfloat16, 2, 48, 96, 3)])
def test_readout_group_norm_step_matches_separate(dtype, B, K, C, G):
    """cdssm_readout_group_norm_gate_step (the readout projection in the GroupNorm step kernel) against the
    projection as one fp32-accumulated product rounded to the dtype (as a GEMM's output) followed by
    cdssm_group_norm_gate_step; both the outputs and the updated running sums."""
    from cdssm_hip.lm import group_norm_gate_step
    log(f"[readout + group norm step] {dtype} B{B} K{K} C{C} G{G}")
    g = torch.Generator().manual_seed(15)
    f32 = dict(generator=g, dtype=torch.float32)
    r = torch.randn(B, K, **f32).to(dtype).to(DEV)
    W = (torch.randn(C, K, **f32) / K ** 0.5).to(dtype).to(DEV)
    z = torch.randn(B, C + 8, **f32).to(dtype).to(DEV)[:, 8:]
    xc = torch.randn(B, C, **f32).to(dtype).to(DEV)
    gamma = (1 + 0.2 * torch.randn(C, **f32)).to(DEV)
    beta = (0.1 * torch.randn(C, **f32)).to(DEV)
    Dp = (0.3 * torch.randn(C, **f32)).to(dtype).to(DEV)
    gs0 = torch.cat([torch.randn(B, G, 1, **f32), torch.randn(B, G, 1, **f32) * 3,
                     torch.rand(B, G, 1, **f32) * 50 + 20, torch.full((B, G, 1), 40.0)], -1).to(DEV)
    gs_a, gs_b = gs0.clone(), gs0.clone()
    y = (r.float() @ W.float().t()).to(dtype)
    ref = group_norm_gate_step(y, gs_a, gamma, beta, 1e-5, z, xc, Dp)
    out = group_norm_gate_step(r, gs_b, gamma, beta, 1e-5, z, xc, Dp, readout_weight=W)
    e, es = rel(out, ref), rel(gs_b, gs_a)
    log(f"   rel err out {e:.2e} running sums {es:.2e}")
    assert out.shape == (B, C) and e <= (1e-5 if dtype == torch.float32 else 2e-2)
    assert es <= (1e-5 if dtype == torch.float32 else 1e-3)


@pytest.mark.parametrize("dtype,n_layers,L0,T,d_inner", [
    (torch.float32, 1, 64, 3, 128), (torch.float32, 1, 45, 2, 128), (torch.bfloat16, 1, 128, 2, 128),
    (torch.float32, 3, 64, 2, 128), (torch.float32, 1, 70, 3, 512), (torch.bfloat16, 1, 64, 2, 512),
    (torch.bfloat16, 2, 40, 3, 512)])
def test_model_decode_matches_reforward(dtype, n_layers, L0, T, d_inner):
    """d_inner 128 (2 heads) takes the separate per-token kernels (the stacked gate / Q columns are not 16-byte
    aligned); d_inner 512 (8 heads) the one-launch token kernel."""
    cfg, m = _cfg(dtype, n_layers=n_layers, d_inner=d_inner)
    B = 2
    log(f"[model decode] {dtype} layers {n_layers} prompt {L0} steps {T}")
    g = torch.Generator().manual_seed(15)
    ids = torch.randint(0, cfg.vocab_size, (B, L0 + T), generator=g).to(DEV)
    with torch.no_grad():
        last, caches = m.prefill(ids[:, :L0])
        e0 = rel(last, m(ids[:, :L0])[:, -1])
        log(f"   prefill last logits vs forward: {e0:.2e}")
        assert e0 <= (1e-5 if dtype == torch.float32 else 1e-2)
        for t in range(L0, L0 + T):
            step = m.decode_step(ids[:, t], caches)
            ref = m(ids[:, :t + 1])[:, -1]
            e = rel(step, ref)
            log(f"   token {t}: decode vs re-forward logits {e:.2e}")
            assert torch.isfinite(step).all()
            if n_layers == 1:
                assert e <= (1e-4 if dtype == torch.float32 else 2e-2)
            else:
                # deeper: the re-forward also revises earlier positions above layer 1 (the reference's
                # GroupNorm spans all positions); the step keeps running statistics -- bounded, not equal
                assert e <= (2e-3 if dtype == torch.float32 else 3e-2)


@pytest.mark.parametrize("dtype,n_layers", [(torch.float32, 2), (torch.bfloat16, 2)])
def test_decode_graph_matches_eager(dtype, n_layers):
    """The graph-captured decode step against eager steps from an identical prefill: every replay, with
    the eager steps (and their synchronisation) between replays."""
    cfg, m = _cfg(dtype, n_layers=n_layers)
    B, L0, T = 3, 70, 4
    log(f"[decode graph] {dtype} layers {n_layers} prompt {L0} replays {T}")
    g = torch.Generator().manual_seed(16)
    ids = torch.randint(0, cfg.vocab_size, (B, L0 + T), generator=g).to(DEV)
    with torch.no_grad():
        _, c_eager = m.prefill(ids[:, :L0])
        _, c_graph = m.prefill(ids[:, :L0])
        dg = m.decode_graph(c_graph)
        for t in range(L0, L0 + T):
            want = m.decode_step(ids[:, t], c_eager).clone()
            torch.cuda.synchronize()
            got = dg(ids[:, t]).clone()
            torch.cuda.synchronize()
            e = rel(got, want)
            log(f"   token {t}: graph vs eager {e:.2e}")
            assert e <= 1e-6
        # the graph advanced the same state as the eager steps
        assert torch.equal(c_graph[0]["l"], c_eager[0]["l"])
        assert rel(c_graph[-1]["scan"].state, c_eager[-1]["scan"].state) <= 1e-6


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_fused_token_kernel_matches_separate_kernels(dtype):
    """cdssm_decode_block_token against the separate per-token kernels on the same caches: equal logits and
    scan state up to fp32 rounding (the fused kernel rounds where the separate kernels store; the compiler may
    contract a multiply-add differently), 1e-5 fp32 / 2e-2 bf16 normwise."""
    from cdssm_hip.lm import CDSSMBlock, _clone_cache
    cfg, m = _cfg(dtype, n_layers=2, d_inner=512)
    B, L0, T = 3, 66, 3
    log(f"[fused token kernel] {dtype} prompt {L0} steps {T}")
    g = torch.Generator().manual_seed(17)
    ids = torch.randint(0, cfg.vocab_size, (B, L0 + T), generator=g).to(DEV)
    with torch.no_grad():
        _, ca = m.prefill(ids[:, :L0])
        cb = [_clone_cache(c) for c in ca]
        try:
            for t in range(L0, L0 + T):
                CDSSMBlock.fused_step = True
                la = m.decode_step(ids[:, t], ca)
                CDSSMBlock.fused_step = False
                lb = m.decode_step(ids[:, t], cb)
                e = rel(la, lb)
                log(f"   token {t}: fused vs separate {e:.2e}")
                assert e <= (1e-5 if dtype == torch.float32 else 2e-2)
        finally:
            CDSSMBlock.fused_step = True
        assert rel(ca[-1]["scan"].state, cb[-1]["scan"].state) <= (1e-5 if dtype == torch.float32 else 2e-2)


@pytest.mark.parametrize("dtype,d_inner", [(torch.float32, 512), (torch.bfloat16, 1024)])
def test_fused_tail_matches_token_kernel_and_separate_epilogue(dtype, d_inner):
    """cdssm_decode_block_tail (token step + readout + GroupNorm step in one launch, one workgroup per batch
    row) against cdssm_decode_block_token followed by cdssm_readout_group_norm_gate_step on the same caches:
    the same arithmetic in the same order, so bit-identical logits, scan state, GroupNorm sums and position
    (whose arrival count is back to zero after every step)."""
    from cdssm_hip.lm import CDSSMBlock, _clone_cache
    cfg, m = _cfg(dtype, n_layers=2, d_inner=d_inner)
    B, L0, T = 5, 70, 3
    log(f"[fused decode tail] {dtype} d_inner {d_inner} prompt {L0} steps {T}")
    g = torch.Generator().manual_seed(19)
    ids = torch.randint(0, cfg.vocab_size, (B, L0 + T), generator=g).to(DEV)
    with torch.no_grad():
        _, ca = m.prefill(ids[:, :L0])
        cb = [_clone_cache(c) for c in ca]
        try:
            for t in range(L0, L0 + T):
                CDSSMBlock.fused_tail = True
                la = m.decode_step(ids[:, t], ca)
                CDSSMBlock.fused_tail = False
                lb = m.decode_step(ids[:, t], cb)
                torch.cuda.synchronize()
                log(f"   token {t}: fused tail vs separate {rel(la, lb):.2e}")
                assert torch.equal(la, lb)
        finally:
            CDSSMBlock.fused_tail = True
        for c1, c2 in zip(ca, cb):
            assert torch.equal(c1["l"], c2["l"]) and int(c1["l"][1]) == 0 and int(c1["l"][0]) == L0 + T
            assert torch.equal(c1["gsum"], c2["gsum"])
            assert torch.equal(c1["scan"].state, c2["scan"].state)


def test_config4_decode_24_layers_batch_64():
    """Config 4's decode: 24 layers, d_model 1024, 16 heads x 64, vocab 32000, bf16, B = 64 from a
    2048-token prefill.  Each step is finite; the graph-captured step equals the eager step on every
    replay (with eager work and synchronisation between replays); and layer 0's step output equals the
    re-forward of layer 0 over prompt + tokens at the new token (its input, the embedding, is not
    revised by a re-forward), 2e-2 bf16."""
    from cdssm_hip.lm import CDSSMConfig, CDSSMLMHeadModel, _clone_cache
    torch.manual_seed(0)
    cfg = CDSSMConfig(d_model=1024, n_layers=24, context_length=2048, vocab_size=32000, state_dim=2, d_inner=1024)
    m = CDSSMLMHeadModel(cfg)
    with torch.no_grad():
        for blk in m.blocks:
            blk.v_residual_gate.normal_(std=1.0)
            blk.shortcut_scale.fill_(0.3)
            blk.D.normal_(std=0.1)
    m = m.to(torch.bfloat16).to(DEV).eval()
    B, L0, T = 64, 2048, 3
    log(f"[config-4 decode] 24 layers B{B} prefill {L0} steps {T} bf16")
    g = torch.Generator().manual_seed(18)
    ids = torch.randint(0, cfg.vocab_size, (B, L0 + T), generator=g).to(DEV)
    with torch.no_grad():
        _, caches = m.prefill(ids[:, :L0])
        c_eager = [_clone_cache(c) for c in caches]
        c_layer0 = _clone_cache(caches[0])
        dg = m.decode_graph(caches)
        for t in range(L0, L0 + T):
            want = m.decode_step(ids[:, t], c_eager).clone()
            torch.cuda.synchronize()
            got = dg(ids[:, t]).clone()
            torch.cuda.synchronize()
            assert torch.isfinite(want).all() and torch.isfinite(got).all()
            eg = rel(got, want)
            x0, _ = m.blocks[0].step(m.embedding(ids[:, t]), None, c_layer0)
            ref0, _ = m.blocks[0](m.embedding(ids[:, :t + 1]))
            e0 = rel(x0, ref0[:, -1])
            log(f"   token {t}: graph vs eager {eg:.2e}  layer-0 step vs re-forward {e0:.2e}")
            assert eg <= 1e-6
            assert e0 <= 2e-2
