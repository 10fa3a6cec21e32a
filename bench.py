"""Benchmark of the fused CD-SSM chunkwise delta-rule scan on one MI355X.

Default workload (the metric's headline shape): forward
scan, B=8 H=16 L=4096 D=Q=64 N=2, bf16 q/k/v/gates, fp32 state, synthetic
inputs drawn as the configuration text specifies (seed 0), zero initial state.
One step = one forward scan over the batch: at C1 one launch of the one-pass
kernel (chunk scans, look-back carry and correction in one kernel); shapes it
cannot take run as four launches (chunk summaries, carry fold, carry replay,
main pass).

Prints ONE JSON line with the metric, the roofline of the dominant kernel (the
one-pass kernel, or the four-launch scan's main pass; either reads every
algorithmic byte: q, k, v, beta, sel_C, dt, r, and writes y) against HBM, and a
CPU baseline: the fp32 CPU restatement of the reference algorithm
(oracle/cdssm_oracle.py) timed on this host's cores on a bounded sample.
Kernel durations come from HIP events recorded on the launch stream around the
launches (cdssm_fused_scan_fwd_profile).  `traffic` is the HBM bytes per launch
of that kernel measured by rocprofv3 counters and recorded in profiles/ (the
file named below), or null when that file is absent.
"""

from __future__ import annotations

import argparse
import json
import math
import os
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
PKG_DIR = os.path.join(ROOT, "cayley-delta-state-space-model_amd")
for _p in (ROOT, PKG_DIR):
    if _p not in sys.path:
        sys.path.insert(0, _p)

HBM_PEAK_GBS = 8000.0  # MI355X HBM3E, vendor peak
TRAFFIC_FILES = {
    "fused_fwd_onepass_kernel": os.path.join(ROOT, "profiles", "fused_fwd_onepass_C1_hbm_traffic.txt"),
    "fused_fwd_main_kernel": os.path.join(ROOT, "profiles", "fused_fwd_main_C1_hbm_traffic.txt"),
}


def recorded_traffic(path, key="traffic_bytes_per_launch"):
    """A number recorded in a committed counter summary (a `key: N` line), or None."""
    try:
        with open(path) as f:
            for line in f:
                if line.startswith(key + ":"):
                    return float(line.split(":", 1)[1])
    except OSError:
        return None
    return None


FWD_BWD_TRAFFIC = os.path.join(ROOT, "profiles", "fused_fwd_bwd_C1_C2_hbm_traffic.txt")
MFMA_PROFILE = os.path.join(ROOT, "profiles", "fused_fwd_onepass_C1_sq_counters.md")
MFMA_VARIANT_PROFILE = os.path.join(ROOT, "profiles", "mfma_correction_vs_sequential_C1_C2.md")
CHUNKED_PROFILE = os.path.join(ROOT, "profiles", "chunked_scan_n16_C4_counters.md")


def mfma_util(kernel):
    """MFMA utilisation of the forward kernel the bench times, from committed SQ counters (rocprofv3 cannot
    run inside this process): MFMA FLOPs / kernel time / 2.5 PFLOP/s dense bf16, with the path named.  The
    chunked MFMA correction (not the default) is quoted beside it."""
    return {"path": kernel + " (sequential correction: no MFMA instructions)"
            if kernel == "fused_fwd_onepass_kernel" else kernel,
            "value": recorded_traffic(MFMA_PROFILE, "mfma_util"),
            "mfma_insts_per_wave": recorded_traffic(MFMA_PROFILE, "mfma_insts_per_wave"),
            "source": os.path.relpath(MFMA_PROFILE, ROOT),
            "chunked_mfma_correction": {"path": "four_launch_mfma (fused_fwd_corr_sweep_kernel, not default)",
                                        "value": recorded_traffic(MFMA_VARIANT_PROFILE, "mfma_util_C1"),
                                        "source": os.path.relpath(MFMA_VARIANT_PROFILE, ROOT)},
            "state_dim16_block_scan": {"path": "cdssm_chunked_scan_fwd_abar (chunked_sweep_kernel, the block's "
                                               "default at state_dim 16 bf16)",
                                       "value_local_pass": recorded_traffic(CHUNKED_PROFILE, "mfma_util_local"),
                                       "value_correction_pass": recorded_traffic(CHUNKED_PROFILE, "mfma_util_corr"),
                                       "source": os.path.relpath(CHUNKED_PROFILE, ROOT)}}


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--config", default="C1", choices=["C1", "C2", "C3", "C4scan"],
                    help="forward workload (C1 is the metric's; C2, C3 and C4scan, the config-4 block's scan shape, for profiling)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-sample-batches", type=int, default=1)
    ap.add_argument("--no-fwd-bwd", action="store_true")
    ap.add_argument("--no-extras", action="store_true",
                    help="skip the decode and config-4 LM timings (profiling runs)")
    ap.add_argument("--forward-path", default="auto", choices=["auto", "four_launch", "one_pass", "four_launch_mfma"],
                    help="how the forward is launched (default: the library's own choice)")
    ap.add_argument("--only-dropin", action="store_true",
                    help="only time the drop-in SSDChunkwiseScan at C1 (fused and per-pass) and print its JSON")
    ap.add_argument("--only-chunked", action="store_true",
                    help="only time the chunked state_dim-16 scan (and the Y route beside it) and print its JSON")
    ap.add_argument("--phase-stamps", type=int, default=0,
                    help="only run this many stamped one-pass forwards of --config (after --warmup plain "
                         "calls) and print the per-wave phase durations of the one-pass kernel as JSON")
    ap.add_argument("--copy-probe-mib", type=int, default=0,
                    help="only run a device copy of this many MiB (read + write), 10 times, and exit: "
                         "the reference kernel for scaling HBM byte counters")
    return ap.parse_args()


def copy_probe(mib):
    import torch
    n = mib * (1 << 20) // 4
    a = torch.ones(n, dtype=torch.float32, device="cuda:0")
    b = torch.empty_like(a)
    for _ in range(10):
        b.copy_(a)
    torch.cuda.synchronize()
    print(json.dumps({"copy_probe_bytes_read_per_call": n * 4, "bytes_written_per_call": n * 4, "calls": 10}))


def _stamp_rows(cfg_name, calls, warmup):
    """Per-wave phase durations (waves x 7, microseconds) of `calls` stamped one-pass
    forwards of the configuration, the waves' entry offsets from the first, and each
    call's kernel span.  The stamped entry records the 100 MHz real-time counter at
    eight points of each wave's segment (PreparedForward.STAMP_POINTS)."""
    import torch
    from cdssm_hip.scan import PreparedForward
    from cdssm_hip.workloads import CONFIGS, draw_inputs

    cfg = CONFIGS[cfg_name]
    dev = torch.device("cuda:0")
    x = draw_inputs(cfg, seed=0)
    g = {n: (t.to(dev) if isinstance(t, torch.Tensor) else t) for n, t in x.items()}
    run = PreparedForward(g["q"], g["k"], g["v"], g["beta"], g["sel_C"], g["dt"], g["r"], g["alpha"],
                          g["omega"], g["c"], h0=g["h0"])
    for _ in range(warmup):
        run()
    torch.cuda.synchronize()
    us = 0.01  # microseconds per tick
    rows, spans, starts = [], [], []
    for _ in range(calls):
        st = run.phase_stamps().double()
        t0 = st[:, 0].min()
        spans.append(float(st[:, 7].max() - t0) * us)
        starts.append((st[:, 0] - t0) * us)
        rows.append((st[:, 1:] - st[:, :-1]) * us)
    del run, g
    torch.cuda.synchronize()
    return torch.cat(rows), torch.cat(starts), spans


def _pct(t):
    import torch
    return [round(float(v), 2) for v in torch.quantile(t, torch.tensor([0.1, 0.5, 0.9], dtype=torch.float64))]


def phase_stamps(cfg_name, calls, warmup):
    """Per-wave phase durations of the one-pass forward kernel: percentiles over every
    wave of `calls` stamped calls, in microseconds."""
    from cdssm_hip.scan import PreparedForward
    d, start, spans = _stamp_rows(cfg_name, calls, warmup)
    pts = PreparedForward.STAMP_POINTS
    phases = {f"{pts[i]}->{pts[i + 1]}": _pct(d[:, i]) for i in range(len(pts) - 1)}
    phases["entry offset"] = _pct(start)
    phases["wave total"] = _pct(d.sum(dim=1))
    return {"phase_stamps": {"config": cfg_name, "calls": calls, "waves_per_call": int(d.shape[0] // calls),
                             "unit": "us (p10, p50, p90 over waves)", "phases": phases,
                             "kernel_span_us_median": round(statistics.median(spans), 2)}}


def interchunk_share(cfg_name="C3", calls=3, warmup=3):
    """The inter-chunk part of the default (one-pass) forward's time, from live phase stamps: per wave,
    (segment map composed and published + look-back wait + carry fold) / the wave's whole segment.  This
    is the work the reference does in its serial inter-chunk pass (inter_chunk_scan.cu:52-84)."""
    d, _, spans = _stamp_rows(cfg_name, calls, warmup)
    inter = d[:, 2] + d[:, 3] + d[:, 4]   # local->published, published->waited, waited->folded
    total = d.sum(dim=1)
    med = [float(d[:, i].median()) for i in (2, 3, 4)]
    return {"config": cfg_name, "path": "one-pass forward (persistent at C3)", "calls": calls,
            "waves": int(d.shape[0]),
            "share": sum(med) / float(total.median()),
            "share_per_wave_p10_p50_p90": _pct(inter / total),
            "median_us": {"compose_publish": round(med[0], 2), "lookback_wait": round(med[1], 2),
                          "fold": round(med[2], 2), "wave_total": round(float(total.median()), 2)},
            "kernel_span_us_median": round(statistics.median(spans), 2),
            "target": "< 0.15",
            "basis": "share = (median compose+publish + median wait + median fold) / median wave total, "
                     "from the stamped entry (cdssm_fused_scan_fwd_stamped) on this run"}


def time_fwd_bwd(cfg_name, steps, warmup):
    """Forward + backward scan steps on one configuration (bf16, seeded draws,
    cotangents dy ~ N(0,1) and dh_final ~ N(0,1)).  Returns tokens/s, ms/step,
    the HBM roofline fraction of the algorithmic fwd+bwd bytes, and the
    per-pass split."""
    import torch
    from cdssm_hip.scan import PreparedBackward, PreparedForward
    from cdssm_hip.workloads import CONFIGS, draw_inputs, scan_bytes

    cfg = CONFIGS[cfg_name]
    dev = torch.device("cuda:0")
    x = draw_inputs(cfg, seed=0)
    g = {n: (t.to(dev) if isinstance(t, torch.Tensor) else t) for n, t in x.items()}
    gen = torch.Generator().manual_seed(7)
    dy = torch.randn(cfg.B, cfg.L, cfg.H, cfg.N, generator=gen).to(dev)
    dhf = torch.randn(cfg.B, cfg.H, cfg.N, cfg.D, generator=gen).to(dev)
    fwd = PreparedForward(g["q"], g["k"], g["v"], g["beta"], g["sel_C"], g["dt"], g["r"], g["alpha"],
                          g["omega"], g["c"], h0=g["h0"], train=True)
    bwd = PreparedBackward(fwd, dy, dhf)
    fwd()
    stream = torch.cuda.current_stream(dev)
    for _ in range(warmup):
        fwd()
        bwd()
    torch.cuda.synchronize()

    def timed(fn):
        # `steps` back-to-back calls between two events on the launch stream
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        e0.record(stream)
        for _ in range(steps):
            fn()
        e1.record(stream)
        torch.cuda.synchronize()
        return e0.elapsed_time(e1)

    def step():
        fwd()
        bwd()
    ms = timed(step) / steps
    tf = timed(fwd)
    fwd()  # the backward reads this forward's workspace
    tb = timed(bwd)
    by = scan_bytes(cfg, backward=True)
    alg = by["fwd"] + by["bwd"]
    stored = training_record_bytes(cfg)
    fwd()
    phases = {"fwd_" + k: v for k, v in fwd.profile(steps).items()}
    phases.update({"bwd_" + k: v for k, v in bwd.profile(steps).items()})
    fwd()
    stamps = bwd_phase_summary(bwd, 3)
    return {"workload": f"{cfg.name} fwd+bwd B{cfg.B} H{cfg.H} L{cfg.L} D{cfg.D} bf16",
            "bwd_phase_stamps": stamps,
            "tokens_per_s": cfg.B * cfg.L / (ms * 1e-3), "ms_per_step": ms,
            "fwd_ms": tf / steps, "bwd_ms": tb / steps,
            "hbm_frac": alg / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS,
            "alg_bytes": alg,
            "stored_record_bytes": stored,
            "hbm_frac_with_records": (alg + 2 * stored) / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS,
            "bytes_note": ("alg_bytes: the inputs read and outputs written by forward and backward (272 B / 812 B "
                           "per token-head at D 64 bf16); stored_record_bytes: what the training forward writes "
                           "for the backward (per-token records, z every 8 tokens, chunk entering states, c^ at "
                           "chunk ends), counted twice (written, read back) in hbm_frac_with_records"),
            "phase_ms": phases,
            "traffic_bytes": recorded_traffic(FWD_BWD_TRAFFIC, f"traffic_bytes_per_step_{cfg.name}"),
            "traffic_over_alg": (lambda t: None if t is None else t / alg)(
                recorded_traffic(FWD_BWD_TRAFFIC, f"traffic_bytes_per_step_{cfg.name}")),
            "traffic_source": os.path.relpath(FWD_BWD_TRAFFIC, ROOT)}


def bwd_phase_summary(bwd, calls):
    """Per-wave phase durations of the backward kernels from `calls` stamped backwards
    (cdssm_fused_scan_bwd_stamped, PreparedBackward.phase_stamps): 10th/50th/90th
    percentiles in microseconds, per phase of the one-launch correction adjoint + carry
    and of the main pass, and each kernel's span (first entry to last end, median over
    the calls).  None when the shape runs the three-launch correction adjoint."""
    import torch
    us = 0.01  # microseconds per tick of the 100 MHz counter
    corr, main, spans_c, spans_m = [], [], [], []
    try:
        for _ in range(calls):
            c, m = bwd.phase_stamps()
            c, m = c.double(), m.double()
            corr.append((c[:, 1:] - c[:, :-1]) * us)
            main.append((m[:, 1:] - m[:, :-1]) * us)
            spans_c.append(float(c[:, 7].max() - c[:, 0].min()) * us)
            spans_m.append(float(m[:, 3].max() - m[:, 0].min()) * us)
    except RuntimeError:
        return None
    corr, main = torch.cat(corr), torch.cat(main)
    cp = bwd.CORR_STAMP_POINTS
    mp = bwd.MAIN_STAMP_POINTS
    return {"corr_adjoint_carry": {f"{cp[i]}->{cp[i + 1]}": _pct(corr[:, i]) for i in range(7)},
            "corr_adjoint_carry_wave_total": _pct(corr.sum(1)),
            "corr_adjoint_carry_span_us": sorted(spans_c)[len(spans_c) // 2],
            "main": {f"{mp[i]}->{mp[i + 1]}": _pct(main[:, i]) for i in range(3)},
            "main_wave_total": _pct(main.sum(1)),
            "main_span_us": sorted(spans_m)[len(spans_m) // 2],
            "basis": "cdssm_fused_scan_bwd_stamped: per wave, percentiles 10/50/90 of each phase in us"}


def training_record_bytes(cfg):
    """Bytes the training forward stores for the backward (and the backward reads back): per token-head
    two float4 records and the float2 g_t (40 B); per chunk-head the state every 8 tokens (bf16 complex
    pairs for bf16 inputs: 4 B per element), the entering state and c^ at the chunk end (fp32 complex),
    and G_k."""
    NC = -(-cfg.L // cfg.D)
    NCK = -(-cfg.D // 8) * 8 // 8
    pair = 4 if cfg.dtype == "bf16" else 8
    per_chunk_head = NCK * cfg.D * pair + 2 * cfg.D * 8 + 8
    return cfg.B * cfg.H * (cfg.L * 40 + NC * per_chunk_head)


def time_dropin(cfg_name, steps=10, warmup=2):
    """The drop-in path unchanged reference callers get (ssd.py:83-100 through the reference's own op
    classes): SSDChunkwiseScan(chunk, 2) materialising Y (B,L,H,N,D) bf16 as the reference does, in its
    two executions -- the fused kernels (the module's choice for N = 2: cdssm_ssd_scan_fwd / _bwd) and
    the per-pass ops (intra-chunk scan, inter-chunk carry, exact correction, Y = local_h + correction,
    fused=False).  Forward alone and forward + backward (autograd with dY ~ N(0,1)).  Algorithmic bytes
    of this interface: the forward reads A_bar, K, V, beta and writes Y, B*H*L*((D + 2N + 1) + N*D)*2;
    the backward reads dY and the inputs and writes their gradients, B*H*L*(N*D + 2*(D + 2N + 1))*2."""
    import torch
    from cdssm_hip.ssd import SSDChunkwiseScan
    from cdssm_hip.workloads import CONFIGS, draw_inputs

    cfg = CONFIGS[cfg_name]
    dev = torch.device("cuda:0")
    x = draw_inputs(cfg, seed=0)
    # the workload's A_bar and VP scale from (dt, r, alpha, omega, c): conj(mu) E^((c r - 1)/2) and
    # sqrt(max(1 - E^(c r), 1e-6)) of the Cayley map (dynamics_fused.cu:109-131), in torch on the GPU
    dt, r = x["dt"].to(dev).float(), x["r"].to(dev).float()
    ta = 0.5 * dt * x["alpha"].to(dev).clamp_min(0.0)
    tw = 0.5 * dt * x["omega"].to(dev)
    den = (1 + ta) ** 2 + tw ** 2 + 1e-6
    E = (((1 - ta) ** 2 + tw ** 2) / den).clamp_min(1e-8)
    cr = x["c"] * r
    scale = E ** ((cr - 1) * 0.5)
    A = torch.stack([(1 - ta ** 2 - tw ** 2) / den * scale, -(2 * tw) / den * scale], -1).to(torch.bfloat16)
    vp = (1 - E ** cr).clamp_min(1e-6).sqrt().clamp_max(1.0)
    V = (x["v"].to(dev).float() * vp[..., None]).to(torch.bfloat16)
    K = x["k"].to(dev)
    beta = x["beta"].to(dev)
    stream = torch.cuda.current_stream(dev)
    gY = torch.randn(cfg.B, cfg.L, cfg.H, 2, cfg.D, generator=torch.Generator().manual_seed(3)).to(
        torch.bfloat16).to(dev)
    BHL, D, N = cfg.B * cfg.H * cfg.L, cfg.D, 2
    by_f = BHL * ((D + 2 * N + 1) + N * D) * 2
    by_b = BHL * (N * D + 2 * (D + 2 * N + 1)) * 2

    def timed(fn):
        for _ in range(warmup):
            fn()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        for _ in range(steps):
            fn()
        e1.record(stream)
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / steps

    def leg(fused):
        scan = SSDChunkwiseScan(cfg.D, 2, fused=fused)
        with torch.no_grad():
            ms_f = timed(lambda: scan(A, K, V, beta))
        leaves = [t.detach().clone().requires_grad_(True) for t in (A, K, V, beta)]

        def fb():
            for t in leaves:
                t.grad = None  # each step's gradients, not a running sum
            Y = scan(*leaves)
            Y.backward(gY)

        ms_fb = timed(fb)
        return {"fwd_ms": ms_f, "fwd_tokens_per_s": cfg.B * cfg.L / (ms_f * 1e-3),
                "fwd_hbm_frac": by_f / (ms_f * 1e-3) / 1e9 / HBM_PEAK_GBS,
                "fwd_bwd_ms": ms_fb, "fwd_bwd_tokens_per_s": cfg.B * cfg.L / (ms_fb * 1e-3),
                "fwd_bwd_hbm_frac": (by_f + by_b) / (ms_fb * 1e-3) / 1e9 / HBM_PEAK_GBS}

    def graphed(fn):
        """GPU time per call without the host's per-call work: the call captured once in a HIP graph
        (torch.cuda.graph) and replayed back to back."""
        side = torch.cuda.Stream(dev)
        side.wait_stream(stream)
        with torch.cuda.stream(side):
            for _ in range(warmup):
                fn()
        stream.wait_stream(side)
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            fn()
        return timed(graph.replay)

    from cdssm_hip.scan import ssd_scan_bwd, ssd_scan_fwd
    out = {"workload": f"drop-in SSDChunkwiseScan, {cfg.name} B{cfg.B} H{cfg.H} L{cfg.L} D{D} bf16",
           "alg_bytes_fwd": by_f, "alg_bytes_bwd": by_b}
    out["fused"] = leg(None)
    g_f = graphed(lambda: ssd_scan_fwd(A, K, V, beta, cfg.D))
    g_fb = graphed(lambda: ssd_scan_bwd(gY, A, K, V, beta, ssd_scan_fwd(A, K, V, beta, cfg.D, train=True)[2], cfg.D))
    out["fused"].update({"graph_fwd_ms": g_f, "graph_fwd_hbm_frac": by_f / (g_f * 1e-3) / 1e9 / HBM_PEAK_GBS,
                         "graph_fwd_bwd_ms": g_fb,
                         "graph_fwd_bwd_hbm_frac": (by_f + by_b) / (g_fb * 1e-3) / 1e9 / HBM_PEAK_GBS})
    out["per_pass"] = leg(False)
    out["note"] = ("fused: cdssm_ssd_scan_fwd / cdssm_ssd_scan_bwd (its training forward also writes the backward's "
                   "records into the workspace); per_pass: the reference's op sequence over the per-pass kernels; "
                   "*_ms: back-to-back module calls (host work per call included); graph_*: the same kernels "
                   "replayed from a captured graph (GPU time)")
    return out


def time_dropin_rows(B=4, L=2048, H=16, D=64, N=16, steps=5, warmup=2):
    """The drop-in SSDChunkwiseScan at the reference's default state_dim (N = 16: 8 complex state rows per
    head), fused kernels (each row a virtual head sharing k) against the per-pass ops, bf16, synthetic
    inputs (|A_bar| in [0.5, 0.99), unit-norm keys).  Bytes of the interface: forward reads A_bar, K, V,
    beta and writes Y (N D per token-head); backward reads dY and the inputs and writes their gradients."""
    import torch
    from cdssm_hip.ssd import SSDChunkwiseScan

    dev = torch.device("cuda:0")
    g = torch.Generator().manual_seed(0)
    ang = torch.rand(B, L, H, N // 2, generator=g) * 2 * math.pi
    mag = 0.5 + 0.49 * torch.rand(B, L, H, N // 2, generator=g)
    A = torch.stack([mag * torch.cos(ang), mag * torch.sin(ang)], -1).flatten(-2).to(torch.bfloat16).to(dev)
    K = torch.randn(B, L, H, D, generator=g)
    K = (K / K.norm(dim=-1, keepdim=True)).to(torch.bfloat16).to(dev)
    V = torch.randn(B, L, H, N, generator=g).to(torch.bfloat16).to(dev)
    beta = torch.rand(B, L, H, generator=g).to(torch.bfloat16).to(dev)
    gY = torch.randn(B, L, H, N, D, generator=g).to(torch.bfloat16).to(dev)
    stream = torch.cuda.current_stream(dev)
    BHL = B * H * L
    by_f = BHL * ((D + 2 * N + 1) + N * D) * 2
    by_b = BHL * (N * D + 2 * (D + 2 * N + 1)) * 2

    def timed(fn):
        for _ in range(warmup):
            fn()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        for _ in range(steps):
            fn()
        e1.record(stream)
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / steps

    out = {"workload": f"drop-in SSDChunkwiseScan B{B} L{L} H{H} D{D} N{N} bf16", "alg_bytes_fwd": by_f,
           "alg_bytes_bwd": by_b}
    for name, fused in (("fused", None), ("per_pass", False)):
        m = SSDChunkwiseScan(D, N, fused=fused)
        with torch.no_grad():
            ms_f = timed(lambda: m(A, K, V, beta))
        leaves = [t.detach().clone().requires_grad_(True) for t in (A, K, V, beta)]

        def fb():
            for t in leaves:
                t.grad = None  # each step's gradients, not a running sum
            Y = m(*leaves)
            Y.backward(gY)

        ms_fb = timed(fb)
        out[name] = {"fwd_ms": ms_f, "fwd_hbm_frac": by_f / (ms_f * 1e-3) / 1e9 / HBM_PEAK_GBS,
                     "fwd_bwd_ms": ms_fb,
                     "fwd_bwd_hbm_frac": (by_f + by_b) / (ms_fb * 1e-3) / 1e9 / HBM_PEAK_GBS}
    return out


def time_chunked_rows(B=8, L=2048, H=16, D=64, N=16, steps=20, warmup=3):
    """The block's scan at the reference's default state_dim 16 (8 complex rows per head), inference,
    bf16, config 4's shape: the chunked (UT) form on the matrix cores (cdssm_chunked_scan_fwd_abar: the
    readout y = sel_C (Y.q) without Y) against this build's other route for N > 2, the fused SSD form
    writing Y (B,L,H,16,D) and the readout in torch (what block.py:198-211 computes).  Synthetic inputs
    (|A_bar| in [0.5, 0.99), unit-norm k and q).  Bytes of the interface: q, k, v, A_bar, vp, beta, sel_C
    read, y written."""
    import torch
    from cdssm_hip import chunked_scan_abar
    from cdssm_hip.ssd import SSDChunkwiseScan

    dev = torch.device("cuda:0")
    g = torch.Generator().manual_seed(0)
    R = N // 2
    ang = torch.rand(B, L, H, R, generator=g) * 2 * math.pi
    mag = 0.5 + 0.49 * torch.rand(B, L, H, R, generator=g)
    bf = lambda t: t.to(torch.bfloat16).to(dev)  # noqa: E731
    A = bf(torch.stack([mag * torch.cos(ang), mag * torch.sin(ang)], -1).flatten(-2))
    k = torch.randn(B, L, H, D, generator=g)
    q = torch.randn(B, L, H, D, generator=g)
    k, q = bf(k / k.norm(dim=-1, keepdim=True)), bf(q / q.norm(dim=-1, keepdim=True))
    v, vp = bf(torch.randn(B, L, H, N, generator=g)), bf(torch.rand(B, L, H, R, generator=g))
    beta, sel = bf(torch.rand(B, L, H, generator=g)), bf(torch.rand(B, L, H, generator=g))
    stream = torch.cuda.current_stream(dev)
    alg = B * L * H * (2 * D + 2 * N + R + 2 + N) * 2

    def timed(fn):
        for _ in range(warmup):
            fn()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        for _ in range(steps):
            fn()
        e1.record(stream)
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / steps

    m = SSDChunkwiseScan(D, N)

    def via_y():
        Vg = v * vp.repeat_interleave(2, dim=-1)
        Y = m(A, k, Vg, beta)
        return (Y.float() * q.float().unsqueeze(-2)).sum(-1) * sel.float().unsqueeze(-1)

    with torch.no_grad():
        ms_c = timed(lambda: chunked_scan_abar(q, k, v, beta, sel, A, vp))
        ms_y = timed(via_y)
    return {"workload": f"block scan, state_dim {N}, B{B} L{L} H{H} D{D} bf16 inference", "alg_bytes": alg,
            "chunked_ms": ms_c, "chunked_tokens_per_s": B * L / (ms_c * 1e-3),
            "chunked_hbm_frac": alg / (ms_c * 1e-3) / 1e9 / HBM_PEAK_GBS,
            "ssd_form_plus_readout_ms": ms_y,
            "mfma_util": {"local_pass": recorded_traffic(CHUNKED_PROFILE, "mfma_util_local"),
                          "correction_pass": recorded_traffic(CHUNKED_PROFILE, "mfma_util_corr"),
                          "source": os.path.relpath(CHUNKED_PROFILE, ROOT)},
            "note": "chunked: cdssm_chunked_scan_fwd_abar (local pass, carry, correction pass; MFMA); "
                    "ssd_form_plus_readout: SSDChunkwiseScan's fused kernels write Y, torch reads it out"}


def time_decode(steps, warmup, B=64, H=16, D=64, prompt=2048):
    """Recurrent decode at the config-4 decode shape, one layer: B64 H16 D64 bf16
    from a 2048-token prompt (fused scan over the prompt, then decode steps).
    `steps` back-to-back cdssm_decode_step calls between two events on the launch
    stream; the token inputs are those of position `prompt` (synthetic)."""
    import ctypes
    import torch
    from cdssm_hip import _lib
    from cdssm_hip.decode import DecodeState
    from cdssm_hip.scan import chunkwise_delta_scan
    from cdssm_hip.workloads import ScanConfig, draw_inputs

    cfg = ScanConfig("decode", B=B, H=H, L=prompt + 1, D=D)
    dev = torch.device("cuda:0")
    x = draw_inputs(cfg, seed=0)
    g = {n: (t.to(dev) if isinstance(t, torch.Tensor) else t) for n, t in x.items()}
    keys = ("q", "k", "v", "beta", "sel_C", "dt", "r")
    stream = torch.cuda.current_stream(dev)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    pre = [g[n][:, :prompt].contiguous() for n in keys]
    _, h = chunkwise_delta_scan(*pre, g["alpha"], g["omega"], g["c"])
    e0.record(stream)
    _, h = chunkwise_delta_scan(*pre, g["alpha"], g["omega"], g["c"])  # warm: the prompt's fused scan
    e1.record(stream)
    torch.cuda.synchronize()
    prefill_ms = e0.elapsed_time(e1)
    del pre
    st = DecodeState.at_boundary(h, B, H, D, D, dev)
    tok = [g[n][:, prompt].contiguous() for n in keys]
    y = torch.empty(B, H, 2, dtype=torch.bfloat16, device=dev)
    lib = _lib.load()
    fn = lib.cdssm_decode_step
    args = [1] + [_lib.ptr(t) for t in tok] + [_lib.ptr(g["alpha"]), _lib.ptr(g["omega"]), ctypes.c_float(g["c"]),
                                                _lib.ptr(st.state), _lib.ptr(st.gam), _lib.ptr(st.pos), _lib.ptr(y),
                                                None, B, H, D, 2, D, _lib.stream_of(dev)]
    for _ in range(warmup):
        _lib.check(fn(*args), "cdssm_decode_step")
    torch.cuda.synchronize()
    e0.record(stream)
    for _ in range(steps):
        fn(*args)
    e1.record(stream)
    torch.cuda.synchronize()
    us = e0.elapsed_time(e1) * 1e3 / steps
    # per (b, h): z and c^ read and written (4 D fp32 each way), q and k (2 D bf16),
    # v, beta, sel_C, dt, r (6 bf16), y (2 bf16); the carry s at chunk ends only (1/Q)
    Q = D
    per_bh = 16 * D + 16 * D + 4 * D + 12 + 4 + 16 * D / Q
    alg = B * H * per_bh
    return {"workload": f"decode B{B} H{H} D{D} bf16, one layer, from a {prompt}-token prompt",
            "us_per_step": us, "tokens_per_s": B / (us * 1e-6), "alg_bytes_per_step": alg,
            "achieved_GBs": alg / (us * 1e-6) / 1e9, "hbm_frac": alg / (us * 1e-6) / 1e9 / HBM_PEAK_GBS,
            "prefill_ms": prefill_ms, "prefill_note": "fused scan over the prompt (one call, warm)",
            "note": "steps launched back to back from Python through ctypes; per-step time includes the launch"}


def time_lm_decode(steps=20, warmup=3, B=64, prompt=2048):
    """Config-4 model decode: the 24-layer LM (as time_lm_forward) prefilled with a 2048-token prompt at
    batch 64, then one new token per row per step (no re-forward): CDSSMLMHeadModel.decode_step eagerly,
    then the same step captured in a HIP graph (DecodeGraph).  Time per step (HIP events around `steps`
    back-to-back steps); ms_per_step is the graph's."""
    import torch
    from cdssm_hip.lm import CDSSMConfig, CDSSMLMHeadModel

    dev = torch.device("cuda:0")
    torch.manual_seed(0)
    cfg = CDSSMConfig(d_model=1024, n_layers=24, context_length=2048, vocab_size=32000, state_dim=2, d_inner=1024)
    m = CDSSMLMHeadModel(cfg).to(torch.bfloat16).to(dev).eval()
    g = torch.Generator().manual_seed(2)
    ids = torch.randint(0, cfg.vocab_size, (B, prompt), generator=g).to(dev)
    new = torch.randint(0, cfg.vocab_size, (warmup + steps, B), generator=g).to(dev)
    stream = torch.cuda.current_stream(dev)
    with torch.no_grad():
        m.prefill(ids)  # warm (the first forward of a process also pays library and kernel loading)
        torch.cuda.synchronize()
        p0, p1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        p0.record(stream)
        _, caches = m.prefill(ids)
        p1.record(stream)
        for i in range(warmup):
            m.decode_step(new[i], caches)
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        for i in range(steps):
            m.decode_step(new[warmup + i], caches)
        e1.record(stream)
        torch.cuda.synchronize()
        # the same step captured in one HIP graph (continues from the eager steps' state)
        dg = m.decode_graph(caches)
        for i in range(warmup):
            dg(new[i])
        torch.cuda.synchronize()
        g0, g1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        g0.record(stream)
        for i in range(steps):
            dg(new[warmup + i])
        g1.record(stream)
        torch.cuda.synchronize()
    ms_eager = e0.elapsed_time(e1) / steps
    ms = g0.elapsed_time(g1) / steps
    wbytes = sum(p.numel() * p.element_size() for p in m.parameters())
    return {"workload": f"config 4: LM decode step B{B} from a {prompt}-token prefill, 24 layers, bf16",
            "ms_per_step": ms, "tokens_per_s": B / (ms * 1e-3), "eager_ms_per_step": ms_eager,
            "prefill_ms": p0.elapsed_time(p1), "weight_bytes": wbytes, "weight_read_GBs": wbytes / (ms * 1e-3) / 1e9,
            "note": "one HIP graph per step (DecodeGraph); per layer 5 launches: RMSNorm + in_proj (skinny GEMM), "
                    "conv step, stacked gate/Q projection (skinny GEMM), one tail kernel (dynamics, K/Q norm, value "
                    "residual, scan step, shortcut, then readout_proj and the GroupNorm step of the batch row: "
                    "cdssm_decode_block_tail), out_proj with the residual (skinny GEMM); then the final RMSNorm and "
                    "the tied head (library GEMM)"}


def time_lm_forward(steps=5, warmup=2, state_dim=2):
    """Config-4 LM forward: B8 L2048, d_model 1024, 24 layers, 16 heads x 64 (d_inner = 1024,
    as the config states), state_dim 2 (or the reference's default 16), vocab 32000, bf16, random init
    (the reference's init scheme), uniform random tokens.  Tokens/s of the whole forward (logits
    included)."""
    import torch
    from cdssm_hip.lm import CDSSMConfig, CDSSMLMHeadModel

    dev = torch.device("cuda:0")
    torch.manual_seed(0)
    cfg = CDSSMConfig(d_model=1024, n_layers=24, context_length=2048, vocab_size=32000, state_dim=state_dim,
                      d_inner=1024)
    m = CDSSMLMHeadModel(cfg).to(torch.bfloat16).to(dev).eval()
    B, L = 8, 2048
    ids = torch.randint(0, cfg.vocab_size, (B, L), generator=torch.Generator().manual_seed(1)).to(dev)
    stream = torch.cuda.current_stream(dev)
    with torch.no_grad():
        for _ in range(warmup):
            m(ids)
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        for _ in range(steps):
            m(ids)
        e1.record(stream)
        torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / steps
    n_params = sum(p.numel() for p in m.parameters())
    flops = 2.0 * n_params * B * L  # dense GEMM work; the scan adds O(L D) per head
    return {"workload": f"config 4: LM forward B8 L2048 d_model 1024 24 layers 16x64 heads N={state_dim} vocab "
                        "32000 bf16",
            "ms_per_step": ms, "tokens_per_s": B * L / (ms * 1e-3), "params": n_params,
            "gemm_tflops": flops / (ms * 1e-3) / 1e12,
            "note": "GEMMs through torch (hipBLASLt); RMSNorm, conv1d+SiLU, dynamics, K/Q norm + q.k, scan, shortcut, "
                    "GroupNorm + gate on the HIP kernels"}


def time_lm_forward_state16(steps=3, warmup=1):
    """time_lm_forward at the reference's default state_dim 16 with each route of the block's scan: the
    chunked MFMA form (its default there), the sequential readout form over 8 state rows per head as
    virtual heads, and SSDChunkwiseScan's Y read out in torch (the reference's op sequence)."""
    from cdssm_hip.lm import CDSSMBlock
    prev = CDSSMBlock.chunked_scan, CDSSMBlock.readout_scan
    res = {}
    try:
        for name, chunked, readout in (("chunked", True, True), ("rows", False, True), ("via_y", False, False)):
            CDSSMBlock.chunked_scan, CDSSMBlock.readout_scan = chunked, readout
            res[name] = time_lm_forward(steps, warmup, state_dim=16)
    finally:
        CDSSMBlock.chunked_scan, CDSSMBlock.readout_scan = prev
    return {"workload": res["chunked"]["workload"], "chunked_ms_per_step": res["chunked"]["ms_per_step"],
            "chunked_tokens_per_s": res["chunked"]["tokens_per_s"], "rows_ms_per_step": res["rows"]["ms_per_step"],
            "via_y_ms_per_step": res["via_y"]["ms_per_step"],
            "note": "chunked: each block's scan, readout and shortcut in one cdssm_chunked_scan_fwd_abar call; "
                    "rows: cdssm_fused_scan_fwd_abar with the 8 state rows of a head as virtual heads; "
                    "via_y: SSDChunkwiseScan's fused kernels write Y and torch reads it out"}


def time_block_train(steps=10, warmup=3, B=8, L=2048, state_dims=(2, 16), routes=("readout_scan", "ssd_y_readout")):
    """One training step through one CDSSMBlock at config 4's shape (d_model 1024, 16 heads x 64,
    d_inner 1024, bf16; B8 L2048): forward and backward of sum(out * g), the way the reference trains
    (block.py:140-229 under autograd, trainer.py:235-247; gradients cleared each step as
    zero_grad(set_to_none=True) does).  state_dim 2 and 16 (the reference's default), each with the
    readout-form scan (no (B,L,H,N,D) Y; at N = 16 the 8 complex state rows of a head run as virtual heads)
    and with SSDChunkwiseScan's Y read out by the HIP readout (the reference's op sequence); ``state_dims`` and
    ``routes`` select a subset (for a profile of one of them)."""
    import torch
    from cdssm_hip.lm import CDSSMBlock, CDSSMConfig

    dev = torch.device("cuda:0")
    gen = torch.Generator().manual_seed(1)
    x = torch.randn(B, L, 1024, generator=gen).to(torch.bfloat16).to(dev).requires_grad_(True)
    g = torch.randn(B, L, 1024, generator=gen).to(torch.bfloat16).to(dev)
    stream = torch.cuda.current_stream(dev)

    def measure(blk):
        def step():
            x.grad = None
            for p in blk.parameters():
                p.grad = None
            out, _ = blk(x)
            out.backward(g)

        for _ in range(warmup):
            step()
        torch.cuda.synchronize()
        torch.cuda.reset_peak_memory_stats(dev)
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        for _ in range(steps):
            step()
        e1.record(stream)
        torch.cuda.synchronize()
        ms = e0.elapsed_time(e1) / steps
        return {"ms_per_step": ms, "tokens_per_s": B * L / (ms * 1e-3),
                "peak_mem_GB": torch.cuda.max_memory_allocated(dev) / 1e9}

    res = {}
    prev = CDSSMBlock.readout_scan
    try:
        for N in state_dims:
            torch.manual_seed(0)
            cfg = CDSSMConfig(d_model=1024, n_layers=24, context_length=2048, vocab_size=32000, state_dim=N,
                              d_inner=1024)
            blk = CDSSMBlock(cfg, 0).to(torch.bfloat16).to(dev).train()
            pre = "" if N == 2 else "state16_"
            for name, flag in (("readout_scan", True), ("ssd_y_readout", False)):
                if name not in routes:
                    continue
                CDSSMBlock.readout_scan = flag
                res[pre + name] = measure(blk)
            del blk
    finally:
        CDSSMBlock.readout_scan = prev
    return {"workload": "one CDSSMBlock training step (forward + backward), config 4 shape B8 L2048 d_model 1024 "
                        "16x64 heads bf16", **res,
            "note": "readout_scan: ChunkwiseDeltaScanAbarFn (cdssm_fused_scan_fwd_abar_train / "
                    "cdssm_fused_scan_bwd_abar; N=16: 8 state rows per head as virtual heads); ssd_y_readout: "
                    "SSDChunkwiseScan's (B,L,H,N,D) Y read out by StateReadoutFn (cdssm_state_readout_fwd/_bwd)"}


def host_cores():
    """Cores this process may run on (the GPU box gives a job a share of the host)."""
    try:
        return len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        return os.cpu_count() or 1


def cpu_baseline(cfg, x, batches, min_seconds=10.0, threads=None, heads=None, backward=False):
    """Time the fp32 oracle (CPU restatement of ops.py's R-mode scan) on `batches` batch rows and
    `heads` heads (all if None) of the workload at full length, repeated until about `min_seconds` of
    CPU work (at least 3 timed repetitions).  `backward`: forward + backward by autograd through the
    restatement (loss sum(y * g), g ~ N(0,1)).  Tokens/s are scaled to the whole workload's tokens per
    sample second: (sampled token-heads / all token-heads) of the workload's B*L tokens."""
    import torch
    from oracle import cdssm_oracle as o

    n = threads or host_cores()
    torch.set_num_threads(n)
    hs = list(range(cfg.H)) if heads is None else list(heads)
    hi = torch.tensor(hs)
    sl = {k: x[k][:batches].index_select(2, hi).float() for k in ("q", "k", "v", "beta", "sel_C", "dt", "r")}
    sl["alpha"], sl["omega"] = x["alpha"].index_select(0, hi).float(), x["omega"].index_select(0, hi).float()
    h0 = None if x["h0"] is None else x["h0"][:batches].index_select(1, hi).float()
    names = ("q", "k", "v", "beta", "sel_C", "dt", "r", "alpha", "omega")
    gy = torch.randn(batches, cfg.L, len(hs), cfg.N, generator=torch.Generator().manual_seed(4))

    def once():
        t0 = time.perf_counter()
        if backward:
            leaves = [sl[m].clone().requires_grad_(True) for m in names]
            y, _ = o.fused_scan(*leaves, x["c"], h0=h0, grad_mode="reference")
            (y * gy).sum().backward()
        else:
            with torch.no_grad():
                o.fused_scan(*[sl[m] for m in names], x["c"], h0=h0)
        return time.perf_counter() - t0

    once()  # warm-up
    times = []
    while len(times) < 3 or sum(times) < min_seconds:
        times.append(once())
    med = statistics.median(times)
    frac = batches * len(hs) / (cfg.B * cfg.H)
    tokens = cfg.B * cfg.L * frac
    what = "forward + backward (autograd)" if backward else "forward"
    return {"value": tokens / med, "unit": "tokens/s", "cores": n, "kind": "port",
            "workload": f"{cfg.name} {what}",
            "sample": (f"oracle fp32 R-mode fused scan {what} (torch CPU, {n} threads) on {batches} of "
                       f"{cfg.B} batch rows x {len(hs)} of {cfg.H} heads x L={cfg.L}; median of {len(times)} "
                       f"repetitions after 1 warm-up ({sum(times):.1f} s timed); {med:.3f} s per sample; "
                       f"tokens/s = the sample's share ({frac:.4f}) of B*L tokens per second")}


def main():
    args = parse()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(json.dumps({"error": "this build runs on one GPU only; --gpus must be 1",
                          "n_gpus": args.gpus}))
        sys.exit(2)

    if args.copy_probe_mib:
        copy_probe(args.copy_probe_mib)
        return
    if args.phase_stamps:
        print(json.dumps(phase_stamps(args.config, args.phase_stamps, args.warmup)), flush=True)
        return
    if args.only_chunked:
        print(json.dumps({"chunked_scan_n16": time_chunked_rows(steps=args.steps, warmup=args.warmup),
                          "lm_forward_state16": time_lm_forward_state16()}), flush=True)
        return
    if args.only_dropin:
        print(json.dumps({"dropin_ssd_scan": time_dropin("C1", steps=args.steps, warmup=args.warmup),
                          "dropin_ssd_scan_n16": time_dropin_rows()}), flush=True)
        return

    import torch
    from cdssm_hip.scan import PreparedForward, set_forward_path
    from cdssm_hip.workloads import CONFIGS, draw_inputs, scan_bytes

    set_forward_path(args.forward_path)

    cfg = CONFIGS[args.config]
    dev = torch.device("cuda:0")
    x = draw_inputs(cfg, seed=0)
    g = {n: (t.to(dev) if isinstance(t, torch.Tensor) else t) for n, t in x.items()}
    run = PreparedForward(g["q"], g["k"], g["v"], g["beta"], g["sel_C"], g["dt"], g["r"], g["alpha"],
                          g["omega"], g["c"], h0=g["h0"])

    for _ in range(args.warmup):
        run()
    torch.cuda.synchronize()

    # timed region: exactly `steps` back-to-back forward scans
    stream = torch.cuda.current_stream(dev)
    ev0 = torch.cuda.Event(enable_timing=True)
    ev1 = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    ev0.record(stream)
    for _ in range(args.steps):
        run()
    ev1.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    gpu_ms = ev0.elapsed_time(ev1)
    ms_per_step = gpu_ms / args.steps

    # per-launch durations (events around each call on the launch stream)
    evs = [torch.cuda.Event(enable_timing=True) for _ in range(2 * 50)]
    for i in range(50):
        evs[2 * i].record(stream)
        run()
        evs[2 * i + 1].record(stream)
    torch.cuda.synchronize()
    per_call = sorted(evs[2 * i].elapsed_time(evs[2 * i + 1]) for i in range(50))
    call_ms = statistics.median(per_call)

    # cold: the last-level cache (256 MB MALL) and the L2s refilled with other data before each call.  The
    # refill reads 1 GiB (a max over it): a write would leave dirty lines whose write-back then competes
    # with the timed call's reads, which would understate the cold rate.
    flush = torch.zeros(1 << 28, dtype=torch.float32, device=dev)  # 1 GiB, written once here
    torch.cuda.synchronize()
    cold = []
    for i in range(10):
        flush.max()
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        run()
        e1.record(stream)
        torch.cuda.synchronize()
        cold.append(e0.elapsed_time(e1))
    cold_ms = statistics.median(cold)
    del flush

    # per-kernel durations, HIP events between the launches on the launch stream
    phases = run.profile(args.steps)
    main_ms = phases["main"]
    one_pass = all(phases[k] == 0.0 for k in ("summary", "carry_fold", "carry_replay"))
    kernel = "fused_fwd_onepass_kernel" if one_pass else "fused_fwd_main_kernel"
    traffic_file = TRAFFIC_FILES[kernel]

    tokens = cfg.B * cfg.L
    alg = scan_bytes(cfg)["fwd"]
    # the kernel's time: its event-timed mean launch, never more than the back-to-back step time
    kern_ms = min(main_ms, ms_per_step)
    achieved = alg / (kern_ms * 1e-3) / 1e9
    traffic = recorded_traffic(traffic_file) if args.config == "C1" else None
    out = {
        "metric": f"scan tokens/sec (fwd), B{cfg.B} H{cfg.H} L{cfg.L} D{cfg.D} bf16",
        "value": tokens / (ms_per_step * 1e-3),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms_per_step,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (BASELINE config draws, seed 0)",
        "config": {"workload": f"{cfg.name} forward scan", "B": cfg.B, "H": cfg.H, "L": cfg.L,
                   "D": cfg.D, "Q": cfg.D, "N": cfg.N, "inputs": "bf16", "state": "fp32",
                   "h0": cfg.h0_std > 0, "global_batch": cfg.B, "seq_len": cfg.L},
        "roofline": {"bound": "hbm", "achieved": achieved, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": achieved / HBM_PEAK_GBS, "traffic": traffic,
                     "kernel": kernel,
                     "headline": "warm: back-to-back calls, inputs resident in HBM (142.7 MB of them also fit "
                                 "the 256 MB last-level cache between calls)",
                     "cold_frac": alg / (cold_ms * 1e-3) / 1e9 / HBM_PEAK_GBS,
                     "cold_basis": "one call after a 1 GiB read refilled the last-level cache, median of 10",
                     "basis": (f"algorithmic {alg / 1e6:.2f} MB per launch (272 B per token-head: q, k, v, "
                               f"beta, sel_C, dt, r read, y written) / {kernel} launch {kern_ms * 1e3:.2f} us "
                               f"(HIP events on the launch stream, mean of {args.steps} launches, capped by the "
                               f"back-to-back step time {ms_per_step * 1e3:.2f} us)"),
                     "traffic_source": (os.path.relpath(traffic_file, ROOT) if traffic is not None else None)},
        "whole_call": {"ms": call_ms, "achieved_GBs": alg / (call_ms * 1e-3) / 1e9,
                       "frac": alg / (call_ms * 1e-3) / 1e9 / HBM_PEAK_GBS,
                       "note": ("one launch" if one_pass else "all four launches") +
                               " of one scan call, median of 50 event-timed calls"},
        "phase_ms": phases,
        "cold_ms_per_call": cold_ms,
        "cold_frac": alg / (cold_ms * 1e-3) / 1e9 / HBM_PEAK_GBS,
        "wall_s_timed": wall,
    }
    out["mfma_util"] = mfma_util(kernel)
    if not args.no_extras:
        out["c3_interchunk"] = interchunk_share()
    if not args.no_fwd_bwd:
        out["fwd_bwd"] = [time_fwd_bwd(n, 20, 3) for n in ("C1", "C2")]
        if not args.no_extras:
            out["decode"] = time_decode(200, 20)
            out["lm_forward"] = time_lm_forward()
            out["block_train"] = time_block_train()
            out["lm_decode"] = time_lm_decode()
    if not args.no_extras:
        out["dropin_ssd_scan"] = time_dropin("C1")
        out["dropin_ssd_scan_n16"] = time_dropin_rows()
        out["chunked_scan_n16"] = time_chunked_rows()
        if not args.no_fwd_bwd:
            out["lm_forward_state16"] = time_lm_forward_state16()
    if not args.no_cpu_baseline:
        out["cpu_baseline"] = cpu_baseline(cfg, x, args.cpu_sample_batches)
        if not args.no_extras:
            from cdssm_hip.workloads import CONFIGS as _C
            extra = [cpu_baseline(cfg, x, args.cpu_sample_batches, threads=1, heads=range(4))]
            x3 = draw_inputs(_C["C3"], seed=0)
            extra.append(cpu_baseline(_C["C3"], x3, 1, heads=range(4)))
            x2 = draw_inputs(_C["C2"], seed=0)
            extra.append(cpu_baseline(_C["C2"], x2, 1, heads=range(2), backward=True))
            out["cpu_baseline_more"] = extra
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
