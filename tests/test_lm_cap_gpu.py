"""The model path with the adaptive-dt cap engaged (dynamics_fused.cu:88-93, :350-359).

With the block's init (log_dt_scale = 0, block.py:53) the cap can never engage:
dt_raw = softplus(0) / (alpha_0 + |omega_0| + 1) < 0.7 is always below
dt_max = 1.875 / (alpha_0 + 1) for alpha_0 < 1.7.  These models raise
log_dt_scale to 3 and steer the gate projection's alpha_0 / omega_0 rows
(bias -3 and 0.06, weights scaled down), with context_length 65536 so the RoPE
term l * 65536^(-h/H) of the upper heads stays inside the blend's window: about
a third of the token-heads of every layer are capped with the blend in
(0.05, 0.95), counted from the oracle (block_gate_rows, dynamics_regimes) on
the model's own weights.  Through them:

  * the forward (gate-level dynamics kernel, fused gate-level scan) against the
    fp64 oracle LM: 1e-3 fp32, 2e-2 bf16;
  * a one-layer decode step (d_inner 512: the one-launch decode-token kernel,
    whose dynamics are gate_math.hpp) against the re-forward at the new token:
    1e-4 fp32, 2e-2 bf16;
  * training (DynamicsFusedFn's backward with the cap's terms) against the
    oracle with the reference's backward rules: every parameter gradient 1e-3.
"""

import pytest
import torch

from _gpu_util import DEV, log, rel
from oracle import cdssm_lm_oracle as lo
from oracle import cdssm_oracle as o

pytestmark = pytest.mark.gpu


def _cap_model(n_layers, dtype=None):
    from cdssm_hip.lm import CDSSMConfig, CDSSMLMHeadModel
    torch.manual_seed(0)
    cfg = CDSSMConfig(d_model=128, n_layers=n_layers, context_length=65536, vocab_size=97, state_dim=2,
                      d_inner=512)
    m = CDSSMLMHeadModel(cfg)
    H, Nh = cfg.n_heads, cfg.state_dim // 2
    with torch.no_grad():
        for blk in m.blocks:
            blk.v_residual_gate.normal_(std=1.0)
            blk.shortcut_scale.fill_(0.3)
            blk.D.normal_(std=0.1)
            blk.log_dt_scale.fill_(3.0)
            W, b = blk.gate_proj.weight, blk.gate_proj.bias
            W[0:H] *= 0.1                       # alpha_0 rows: softplus(-3) ~ 0.05
            b[0:H] = -3.0
            W[Nh * H:(Nh + 1) * H] *= 0.02      # omega_0 rows: near omega_thresh
            b[Nh * H:(Nh + 1) * H] = 0.06
    if dtype is not None:
        m = m.to(dtype)
    p = {k: v.detach().double().cpu() for k, v in m.state_dict().items()}
    return cfg, m.to(DEV), p


def _cap_coverage(cfg, m, p, ids):
    """Per layer, the fraction of token-heads capped with a material blend (oracle, fp64, exact model)."""
    x = p["embedding.weight"][ids]
    v_first = None
    out = []
    for i in range(cfg.n_layers):
        pre = f"blocks.{i}."
        _, _, gates = lo.block_gate_rows(p, pre, x, cfg)
        reg = o.dynamics_regimes(gates, p[pre + "log_dt_scale"], m.blocks[i].rope_freqs.double().cpu(),
                                 cfg.gating_c, cfg.bf16_omega_thresh, cfg.bf16_delta, cfg.bf16_smoothness,
                                 cfg.eps_adaptive_dt, cfg.n_heads, cfg.state_dim)
        out.append(float(reg["blend_mid"].double().mean()))
        x, v_first = lo.block_forward(p, pre, x, v_first, cfg)
    log("   capped with a material blend, per layer: " + " ".join(f"{c:.1%}" for c in out))
    assert min(out) >= 0.2, "the cap must engage on >= 20% of every layer's token-heads"


@pytest.mark.parametrize("dtype,tol", [(torch.float32, 1e-3), (torch.bfloat16, 2e-2)])
def test_lm_forward_with_the_cap_matches_oracle(dtype, tol):
    log(f"[lm fwd, cap engaged] {dtype} 2 layers d_inner 512 B2 L200")
    cfg, m, p = _cap_model(2, dtype)
    ids = torch.randint(0, cfg.vocab_size, (2, 200), generator=torch.Generator().manual_seed(1))
    _cap_coverage(cfg, m, p, ids)
    with torch.no_grad():
        logits = m.eval()(ids.to(DEV)).float().cpu()
    e = rel(logits, lo.lm_forward(p, ids, cfg))
    log(f"   rel err logits {e:.2e}")
    assert torch.isfinite(logits).all() and e <= tol


@pytest.mark.parametrize("dtype,tol", [(torch.float32, 1e-4), (torch.bfloat16, 2e-2)])
def test_decode_token_kernel_with_the_cap_matches_reforward(dtype, tol):
    from cdssm_hip.lm import CDSSMBlock
    assert CDSSMBlock.fused_step
    cfg, m, p = _cap_model(1, dtype)
    m = m.eval()
    B, L0, T = 2, 64, 3
    log(f"[decode, cap engaged] {dtype} 1 layer d_inner 512 prompt {L0} steps {T}")
    ids = torch.randint(0, cfg.vocab_size, (B, L0 + T), generator=torch.Generator().manual_seed(2))
    _cap_coverage(cfg, m, p, ids)
    ids = ids.to(DEV)
    with torch.no_grad():
        _, caches = m.prefill(ids[:, :L0])
        for t in range(L0, L0 + T):
            step = m.decode_step(ids[:, t], caches)
            ref = m(ids[:, :t + 1])[:, -1]
            e = rel(step, ref)
            log(f"   token {t}: decode vs re-forward logits {e:.2e}")
            assert torch.isfinite(step).all() and e <= tol


def test_lm_training_gradients_with_the_cap_match_oracle():
    log("[lm training grads, cap engaged] fp32 2 layers d_inner 512 B2 L100")
    cfg, m, p = _cap_model(2)
    m = m.float().train()
    gen = torch.Generator().manual_seed(3)
    ids = torch.randint(0, cfg.vocab_size, (2, 100), generator=gen)
    gl = torch.randn(2, 100, cfg.vocab_size, generator=gen)
    _cap_coverage(cfg, m, p, ids)
    p = {k: v.clone().requires_grad_(True) for k, v in p.items()}
    logits = m(ids.to(DEV))
    (logits * gl.to(DEV)).sum().backward()
    torch.cuda.synchronize()
    ref = lo.lm_forward(p, ids, cfg, grad_mode="reference")
    (ref * gl.double()).sum().backward()
    e_out = rel(logits.detach(), ref.detach())
    errs = {}
    for name, prm in m.named_parameters():
        want = p[name].grad
        if name == "embedding.weight" and p["lm_head.weight"].grad is not None:
            want = want + p["lm_head.weight"].grad  # tied (model.py:29-30)
        if prm.grad is None and want is None:
            continue
        assert prm.grad is not None and want is not None, name
        errs[name] = rel(prm.grad, want)
    worst = max(errs, key=errs.get)
    log(f"   logits {e_out:.1e}; worst parameter gradient {errs[worst]:.1e} ({worst}); "
        f"log_dt_scale {max(v for k, v in errs.items() if k.endswith('log_dt_scale')):.1e}")
    assert e_out <= 1e-3
    bad = {n: e for n, e in errs.items() if not e <= 1e-3}
    assert not bad, bad
