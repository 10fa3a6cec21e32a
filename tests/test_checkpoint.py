"""Reference checkpoints load into cdssm_hip.lm, and run on the GPU as predict.py does.

The key list below is written out from the reference's modules -- block.py:41-82
(in_proj, conv, gate_proj, log_dt_scale, Q_proj, readout_proj, out_proj, norm,
ssm_norm, D, v_residual_gate, shortcut_scale; rope_freqs is a non-persistent
buffer, block.py:62), modules.py:23-24 / :48 (Conv1dSiLU weight and bias, RMSNorm
weight) and model.py:22-29 (embedding, blocks, final_norm, the tied lm_head) --
with the shapes their constructors give for the reference config, so a renamed
or reshaped parameter in this build fails the strict load.  The checkpoint is
written the way trainer.py:201-215 writes it, with torch.compile's `_orig_mod.`
prefix (predict.py:23) and asdict(config) including the derived fields.

The one GPU test (marked gpu) follows predict.py:10-30 to the end: a checkpoint of
the reference config (d_inner = 2 d_model, the default state_dim 16) loaded onto the
GPU in bf16 (predict.py:27) and run, its logits against the fp64 oracle LM on the
loaded (bf16-rounded) weights, 2e-2 normwise.
"""

import math

import pytest
import torch

from cdssm_hip.checkpoint import COMPUTED_FIELDS, config_from_dict, load_reference_checkpoint


def reference_config_dict(d_model, n_layers, context_length, vocab_size, state_dim):
    """asdict(CDSSMConfig(...)) of the reference (config/model.py:60-110, :119-178)."""
    d_inner = 2 * d_model
    eps = (2.0 ** -7) ** 2
    return dict(d_model=d_model, n_layers=n_layers, context_length=context_length, vocab_size=vocab_size,
                state_dim=state_dim, d_inner=d_inner, n_heads=d_inner // 64, head_dim=64, ssm_norm_groups=32,
                chunk_size=64, conv_kernel_size=4, rope_base=float(context_length),
                gating_c=math.log(context_length), spectral_band_fraction=2.0 / (n_layers + 1), eps_norm=eps,
                eps_log_argument=eps, eps_adaptive_dt=1.0,
                init_biases={"sel_B_bias": math.log(2), "sel_C_bias": math.log(2), "r_gate_bias": math.log(2),
                             "beta_bias": 0.0, "sel_dt_bias": 0.0},
                bf16_omega_thresh=math.sqrt(2.0 ** -7), bf16_delta=16 * 2.0 ** -7,
                bf16_smoothness=math.sqrt(2.0 ** -7) / 5)


def reference_state_dict_shapes(d_model, n_layers, vocab_size, state_dim):
    d_inner = 2 * d_model
    H, N = d_inner // 64, state_dim
    shapes = {"embedding.weight": (vocab_size, d_model)}
    for i in range(n_layers):
        p = f"blocks.{i}."
        shapes.update({
            p + "in_proj.weight": (3 * d_inner + H * N, d_model), p + "in_proj.bias": (3 * d_inner + H * N,),
            p + "conv.weight": (d_inner, 1, 4), p + "conv.bias": (d_inner,),
            p + "gate_proj.weight": (H * (N + 5), d_inner), p + "gate_proj.bias": (H * (N + 5),),
            p + "log_dt_scale": (H,),
            p + "Q_proj.weight": (d_inner, d_inner),
            p + "readout_proj.weight": (d_inner, H * N),
            p + "out_proj.weight": (d_model, d_inner),
            p + "norm.weight": (d_model,),
            p + "ssm_norm.weight": (d_inner,), p + "ssm_norm.bias": (d_inner,),
            p + "D": (d_inner,), p + "v_residual_gate": (H,), p + "shortcut_scale": (1,),
        })
    shapes["final_norm.weight"] = (d_model,)
    shapes["lm_head.weight"] = (vocab_size, d_model)
    return shapes


def _write_checkpoint(path, cfg_dict, shapes, prefix="_orig_mod.", seed=0):
    g = torch.Generator().manual_seed(seed)
    sd = {prefix + k: torch.randn(*s, generator=g) for k, s in shapes.items()}
    sd[prefix + "lm_head.weight"] = sd[prefix + "embedding.weight"]  # tied (model.py:29-30)
    torch.save({"model_state_dict": sd, "config": cfg_dict, "step": 10, "tokens_seen": 1234, "seed": 0,
                "timestamp": "2026-01-01T00:00:00", "optimizer_state_dict": {"state": {}, "param_groups": []},
                "metrics": {"best_val_ppl": 12.5, "epoch": 0}}, path)
    return {k[len(prefix):]: v for k, v in sd.items()}


@pytest.mark.parametrize("state_dim", [16, 2])
def test_reference_checkpoint_loads_strictly(tmp_path, state_dim):
    """The reference default (state_dim 16) and the scan configs' state_dim 2."""
    cfg_dict = reference_config_dict(64, 2, 256, 101, state_dim)
    shapes = reference_state_dict_shapes(64, 2, 101, state_dim)
    path = tmp_path / "ref_best.pt"
    sd = _write_checkpoint(path, cfg_dict, shapes)
    model, ckpt = load_reference_checkpoint(str(path))
    assert ckpt["step"] == 10 and ckpt["metrics"]["best_val_ppl"] == 12.5
    cfg = model.config
    assert (cfg.d_model, cfg.n_layers, cfg.context_length, cfg.vocab_size, cfg.state_dim) == (64, 2, 256, 101,
                                                                                             state_dim)
    assert cfg.d_inner == 128 and cfg.n_heads == 2  # derived as the reference does, not read
    got = model.state_dict()
    assert set(got) == set(shapes)
    for k, v in sd.items():
        assert torch.equal(got[k], v), k
    assert model.lm_head.weight.data_ptr() == model.embedding.weight.data_ptr()


def test_key_list_matches_this_builds_model_exactly():
    from cdssm_hip.lm import CDSSMConfig, CDSSMLMHeadModel
    m = CDSSMLMHeadModel(CDSSMConfig(d_model=64, n_layers=3, context_length=128, vocab_size=50, state_dim=16))
    want = reference_state_dict_shapes(64, 3, 50, 16)
    assert {k: tuple(v.shape) for k, v in m.state_dict().items()} == want


def test_computed_fields_are_never_taken_from_the_checkpoint():
    d = reference_config_dict(64, 2, 256, 101, 16)
    d.update(d_inner=999, n_heads=7, gating_c=-1.0, chunk_size=3)  # nonsense in derived fields
    cfg = config_from_dict(d)
    assert cfg.d_inner == 128 and cfg.n_heads == 2 and cfg.chunk_size == 64
    assert abs(cfg.gating_c - math.log(256)) < 1e-12
    assert {"d_inner", "n_heads", "head_dim", "gating_c", "init_biases"} <= COMPUTED_FIELDS
    with pytest.raises(KeyError):
        config_from_dict({"d_model": 64})


def test_a_strict_load_rejects_a_missing_or_renamed_key(tmp_path):
    cfg_dict = reference_config_dict(64, 1, 128, 40, 2)
    shapes = reference_state_dict_shapes(64, 1, 40, 2)
    shapes["blocks.0.renamed.weight"] = shapes.pop("blocks.0.Q_proj.weight")
    path = tmp_path / "bad.pt"
    _write_checkpoint(path, cfg_dict, shapes)
    with pytest.raises(RuntimeError, match="Q_proj"):
        load_reference_checkpoint(str(path))


@pytest.mark.gpu
def test_reference_checkpoint_runs_on_the_gpu_in_bf16_like_predict(tmp_path):
    from _gpu_util import DEV, log, rel
    from cdssm_hip.lm import CDSSMConfig, CDSSMLMHeadModel
    from oracle import cdssm_lm_oracle as lo
    torch.manual_seed(0)
    cfg = CDSSMConfig(d_model=128, n_layers=2, context_length=512, vocab_size=97, state_dim=16)
    assert cfg.d_inner == 256 and cfg.n_heads == 4  # the reference's derivation (config/model.py:57)
    m = CDSSMLMHeadModel(cfg)
    with torch.no_grad():  # trained-looking weights: the value residual, shortcut and skip are live
        for blk in m.blocks:
            blk.v_residual_gate.normal_(std=1.0)
            blk.shortcut_scale.fill_(0.3)
            blk.D.normal_(std=0.1)
            blk.log_dt_scale.normal_(std=0.5)
    sd = {"_orig_mod." + k: v for k, v in m.state_dict().items()}
    path = tmp_path / "ref_best.pt"
    torch.save({"model_state_dict": sd, "config": reference_config_dict(128, 2, 512, 97, 16), "step": 3,
                "tokens_seen": 99, "seed": 0, "timestamp": "2026-01-01T00:00:00",
                "optimizer_state_dict": {"state": {}, "param_groups": []}, "metrics": {}}, path)
    log("[checkpoint on the GPU] reference config d_model 128 d_inner 256 N16, bf16 like predict.py:27")
    model, _ = load_reference_checkpoint(str(path), device=DEV, dtype=torch.bfloat16)
    assert model.config.d_inner == 256 and model.config.state_dim == 16
    assert next(model.parameters()).dtype == torch.bfloat16 and next(model.parameters()).is_cuda
    p = {k: v.detach().double().cpu() for k, v in model.state_dict().items()}
    ids = torch.randint(0, cfg.vocab_size, (2, 150), generator=torch.Generator().manual_seed(4))
    with torch.no_grad():
        logits = model(ids.to(DEV)).float().cpu()
    e = rel(logits, lo.lm_forward(p, ids, model.config))
    log(f"   rel err logits {e:.2e}")
    assert torch.isfinite(logits).all() and e <= 2e-2
