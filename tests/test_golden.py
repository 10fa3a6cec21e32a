"""Golden fixtures (tests/golden/*.npz, written by tests/golden/make_golden.py).

CPU: the inputs re-drawn from the recorded seed match the recorded checksum,
and the fp64 oracle still reproduces the frozen outputs (a regression pin on
the oracle and the draw).  GPU: the HIP fused forward and backward reproduce
the frozen answers within the fp32 bar (1e-4 normwise).
"""

import os

import numpy as np
import pytest
import torch

from cdssm_hip.workloads import draw_inputs

HERE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
import sys  # noqa: E402
sys.path.insert(0, HERE)
from make_golden import FIXTURES, NAMES, checksum, compute, cotangents  # noqa: E402


def load(name):
    with np.load(os.path.join(HERE, name + ".npz"), allow_pickle=False) as f:
        return {k: f[k] for k in f.files}


def rel(a, b):
    a, b = np.asarray(a, dtype=np.float64), np.asarray(b, dtype=np.float64)
    return float(np.abs(a - b).max() / max(np.abs(b).max(), 1e-300))


@pytest.mark.parametrize("name", sorted(FIXTURES))
def test_oracle_reproduces_golden(name):
    cfg, seed, grads = FIXTURES[name]
    g = load(name)
    x = draw_inputs(cfg, seed=int(g["seed"]))
    np.testing.assert_allclose(checksum(x), g["checksum"], rtol=0, atol=1e-9)
    now = compute(cfg, seed, grads)
    for k in g:
        if k in ("seed", "checksum"):
            continue
        assert rel(now[k], g[k]) <= 1e-12, k


@pytest.mark.gpu
@pytest.mark.parametrize("name", sorted(FIXTURES))
def test_hip_matches_golden(name):
    from cdssm_hip import chunkwise_delta_scan_train
    cfg, seed, grads = FIXTURES[name]
    g = load(name)
    x = draw_inputs(cfg, seed=seed)
    dev = torch.device("cuda:0")
    leaves = {n: x[n].to(dev).requires_grad_(grads) for n in NAMES}
    h0 = None if x["h0"] is None else x["h0"].to(dev).requires_grad_(grads)
    y, hf = chunkwise_delta_scan_train(*[leaves[n] for n in NAMES], x["c"], h0=h0)
    assert rel(y.detach().cpu(), g["y"]) <= 1e-4
    assert rel(hf.detach().cpu(), g["h_final"]) <= 1e-4
    if grads:
        gy, gh = cotangents(cfg, seed)
        torch.autograd.backward([y, hf], [gy.float().to(dev), gh.float().to(dev)])
        for n in NAMES:
            assert rel(leaves[n].grad.cpu(), g["grad_" + n]) <= 1e-4, n
        assert rel(h0.grad.cpu(), g["grad_h0"]) <= 1e-4
