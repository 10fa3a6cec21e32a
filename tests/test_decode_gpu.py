"""GPU parity of the recurrent decode step (cdssm_decode_init / cdssm_decode_step).

A prompt goes through ``prefill`` (fused scan over whole chunks, decode steps for
the ragged rest), then tokens are generated one at a time with ``decode_step``.
Every output must equal the chunked R-mode scan over the whole sequence, which
the fp64 oracle computes in one pass (ssd.py:39-111 restated): the decode
path crosses chunk boundaries (carry s' = g s + z, restart of the local and
correction states), so a wrong boundary rule or an off-by-one in the
correction read fails here.  Tolerances as for the fused scan: fp32 <= 1e-4,
bf16 y <= 2e-2 and final-state norms <= 1e-3 (normwise, against the oracle
fed the same bf16-rounded inputs).
"""

import pytest
import torch

from _gpu_util import DEV, TOKEN_KEYS, ScanConfig, draw_inputs, log, oracle_fwd, rel, select, state_norm_rel, to_dev

pytestmark = pytest.mark.gpu


def run_decode(x, L_prompt, chunk=None):
    """prefill(L_prompt), then decode steps to the end; y (B, L, H, 2) and the final carry."""
    from cdssm_hip import decode_step, prefill
    g = to_dev(x)
    L = g["q"].shape[1]
    prompt = {n: g[n][:, :L_prompt] for n in TOKEN_KEYS}
    y0, st = prefill(*[prompt[n] for n in TOKEN_KEYS], g["alpha"], g["omega"], g["c"], h0=g.get("h0"),
                     chunk_size=chunk)
    ys, h = [y0], None
    for t in range(L_prompt, L):
        y, h = decode_step(st, *[g[n][:, t] for n in TOKEN_KEYS], g["alpha"], g["omega"], g["c"],
                           return_carry=True)
        ys.append(y.unsqueeze(1))
    torch.cuda.synchronize()
    return torch.cat(ys, dim=1).cpu(), (h.cpu() if h is not None else None)


CASES = [
    # name, cfg, prompt length, chunk
    ("fp32_boundary_prompt", ScanConfig("t", B=2, H=5, L=200, D=64, dtype="fp32"), 128, None),
    ("fp32_ragged_prompt_h0", ScanConfig("t", B=2, H=3, L=190, D=64, dtype="fp32", h0_std=0.1), 70, None),
    ("fp32_short_prompt", ScanConfig("t", B=1, H=4, L=100, D=64, dtype="fp32", h0_std=0.1), 5, None),
    ("fp32_D128", ScanConfig("t", B=1, H=3, L=300, D=128, dtype="fp32", h0_std=0.1), 131, None),
    ("fp32_chunk20", ScanConfig("t", B=1, H=5, L=130, D=64, dtype="fp32", h0_std=0.1), 47, 20),
    ("bf16_D64", ScanConfig("t", B=2, H=16, L=260, D=64), 130, None),
    ("bf16_D128_fast_omega", ScanConfig("t", B=1, H=9, L=300, D=128, omega_std=3.0, h0_std=0.1), 200, None),
]


@pytest.mark.parametrize("name,cfg,L_prompt,chunk", CASES, ids=[c[0] for c in CASES])
def test_decode_matches_oracle(name, cfg, L_prompt, chunk):
    log(f"[decode] {name}: B{cfg.B} H{cfg.H} L{cfg.L} (prompt {L_prompt}) D{cfg.D} {cfg.dtype} chunk={chunk or cfg.D}")
    x = draw_inputs(cfg, seed=0)
    y, h = run_decode(x, L_prompt, chunk)
    yr, hr = oracle_fwd(x, chunk_size=chunk)
    ey, eg, eh, en = rel(y, yr), rel(y[:, L_prompt:], yr[:, L_prompt:]), rel(h, hr), state_norm_rel(h, hr)
    log(f"   rel err y {ey:.2e} (generated {eg:.2e})  carry {eh:.2e}  state-norm {en:.2e}")
    if cfg.dtype == "fp32":
        assert ey <= 1e-4 and eh <= 1e-4
    else:
        assert ey <= 2e-2 and en <= 1e-3


def test_decode_from_2048_token_prompt_at_batch_64():
    """SURVEY config-4 decode shape, one layer: B64 H16 D64 bf16, 2048-token prompt (a
    chunk boundary), then 70 generated tokens (across the next boundary).  The oracle
    re-computes four (b, h) sequences in full."""
    cfg = ScanConfig("dec", B=64, H=16, L=2048 + 70, D=64)
    log(f"[decode C4 shape] B{cfg.B} H{cfg.H} prompt 2048 + 70 steps D{cfg.D} bf16")
    x = draw_inputs(cfg, seed=0)
    y, h = run_decode(x, 2048)
    for b, hh in ((0, 0), (17, 5), (40, 11), (63, 15)):
        xs = select(x, [b], [hh])
        yr, hr = oracle_fwd(xs)
        ey = rel(y[b:b + 1, :, hh:hh + 1], yr)
        eg = rel(y[b:b + 1, 2048:, hh:hh + 1], yr[:, 2048:])
        en = state_norm_rel(h[b:b + 1, hh:hh + 1], hr)
        log(f"   (b={b}, h={hh}) rel err y {ey:.2e} generated {eg:.2e} state-norm {en:.2e}")
        assert ey <= 2e-2 and eg <= 2e-2 and en <= 1e-3


def test_decode_continues_exactly_where_the_fused_scan_stops():
    """fp32: the carry the decode step reports after each token equals the fused scan's
    h_final for the sequence ending there, at and between chunk boundaries."""
    from cdssm_hip import chunkwise_delta_scan
    cfg = ScanConfig("t", B=1, H=4, L=140, D=64, dtype="fp32", h0_std=0.1)
    x = draw_inputs(cfg, seed=3)
    g = to_dev(x)
    from cdssm_hip import decode_step, prefill
    y0, st = prefill(*[g[n][:, :60] for n in TOKEN_KEYS], g["alpha"], g["omega"], g["c"], h0=g["h0"])
    for t in range(60, 140):
        _, h = decode_step(st, *[g[n][:, t] for n in TOKEN_KEYS], g["alpha"], g["omega"], g["c"],
                           return_carry=True)
        if t + 1 in (64, 65, 100, 128, 140):
            _, hf = chunkwise_delta_scan(*[g[n][:, :t + 1] for n in TOKEN_KEYS], g["alpha"], g["omega"], g["c"],
                                         h0=g["h0"])
            e = rel(h, hf)
            log(f"   after {t + 1} tokens: carry vs fused h_final {e:.2e}")
            assert e <= 1e-5
