"""Loading checkpoints written by the reference trainer.

The reference saves ``{"model_state_dict", "config": asdict(config), "step", "tokens_seen", "seed",
"timestamp", "optimizer_state_dict", "metrics"}`` (trainer.py:201-215).  Its loader
(predict.py:10-30) rebuilds the config from the checkpoint's dict minus the fields
``CDSSMConfig.__post_init__`` derives (``COMPUTED_FIELDS``, config/model.py:22-33), strips
``torch.compile``'s ``_orig_mod.`` key prefix (predict.py:23) and loads the weights with
``strict=True``.  This module does the same for ``cdssm_hip.lm.CDSSMLMHeadModel``, whose module and
parameter names are the reference's, with a loader that executes nothing from the file
(``torch.load(..., weights_only=True)``; the reference passes ``weights_only=False``).
"""

from __future__ import annotations

from typing import Optional, Tuple

import torch

from .lm import CDSSMConfig, CDSSMLMHeadModel

# Fields CDSSMConfig.__post_init__ derives (config/model.py:22-33): never taken from a checkpoint.
COMPUTED_FIELDS = frozenset({
    "d_inner", "n_heads", "head_dim", "chunk_size", "conv_kernel_size", "ssm_norm_groups", "rope_base",
    "gating_c", "spectral_band_fraction", "eps_norm", "eps_log_argument", "eps_adaptive_dt", "init_biases",
    "bf16_omega_thresh", "bf16_delta", "bf16_smoothness",
})

# The reference's user-specified config surface (config/model.py:121-128).
USER_FIELDS = ("d_model", "n_layers", "context_length", "vocab_size", "state_dim")


def config_from_dict(cfg_dict: dict) -> CDSSMConfig:
    """The model config of a checkpoint's ``config`` dict, as predict.py:14-19 rebuilds it: every
    dataclass field that is not derived.  For the reference's dataclass those are the five user fields;
    d_inner therefore comes out as the reference's 2 * d_model (config/model.py:57)."""
    kwargs = {k: v for k, v in cfg_dict.items() if k in USER_FIELDS and k not in COMPUTED_FIELDS}
    missing = [k for k in USER_FIELDS if k not in kwargs]
    if missing:
        raise KeyError(f"checkpoint config lacks {missing}")
    return CDSSMConfig(**kwargs)


def clean_state_dict(state_dict: dict) -> dict:
    """Drop torch.compile's ``_orig_mod.`` prefix from every key (predict.py:23)."""
    return {k.replace("_orig_mod.", ""): v for k, v in state_dict.items()}


def load_reference_checkpoint(path: str, device: Optional[torch.device] = None,
                              dtype: Optional[torch.dtype] = None) -> Tuple[CDSSMLMHeadModel, dict]:
    """Build the model a reference checkpoint describes and load its weights (strict).

    Returns (model in eval mode, the checkpoint dict).  ``device`` / ``dtype`` move the model (the
    reference's loader moves it to the GPU in bf16, predict.py:27).  The file is read with
    ``torch.load(weights_only=True)``: tensors and plain containers only.
    """
    ckpt = torch.load(path, map_location="cpu", weights_only=True)
    if not isinstance(ckpt, dict) or "model_state_dict" not in ckpt or "config" not in ckpt:
        raise ValueError(f"{path}: not a reference checkpoint (needs 'model_state_dict' and 'config')")
    model = CDSSMLMHeadModel(config_from_dict(ckpt["config"]))
    model.load_state_dict(clean_state_dict(ckpt["model_state_dict"]), strict=True)
    if device is not None or dtype is not None:
        model = model.to(device=device, dtype=dtype)
    return model.eval(), ckpt
