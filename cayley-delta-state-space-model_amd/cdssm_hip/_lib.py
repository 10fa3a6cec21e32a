"""ctypes binding of ``libcdssm_hip.so``, the C-ABI of the HIP kernels.

The library is built in-tree (``__graft_entry__.build()``) next to this file.
There is no fallback: if the library is missing or fails to load, every op
raises ``RuntimeError`` naming the path it looked for.  Entry points take raw
device pointers, int64 sizes, fp32 scalars and a ``hipStream_t``; they return
0 on success and a negative status otherwise, with the message available from
``cdssm_last_error()``.
"""

from __future__ import annotations

import ctypes
import os
import threading
from typing import Optional

import torch

LIB_NAME = "libcdssm_hip.so"
# CDSSM_HIP_LIB names another build of the same library (e.g. a variant
# compiled with different launch parameters); default: the in-tree build.
LIB_PATH = os.environ.get("CDSSM_HIP_LIB") or os.path.join(os.path.dirname(os.path.abspath(__file__)), LIB_NAME)

_P = ctypes.c_void_p
_I64 = ctypes.c_int64
_I32 = ctypes.c_int
_F32 = ctypes.c_float

# name -> (restype, argtypes).  Mirrors include/cdssm_hip.h.
SIGNATURES = {
    "cdssm_abi_version": (_I32, []),
    "cdssm_fused_scan_fwd_set_path": (_I32, [_I32]),
    "cdssm_lookback_status": (_I32, [_I32, _P]),
    "cdssm_last_error": (ctypes.c_char_p, []),
    "cdssm_fused_scan_workspace_bytes": (_I64, [_I64, _I64, _I64, _I64, _I64, _I64]),
    "cdssm_fused_scan_fwd": (_I32, [_I32, _P, _P, _P, _P, _P, _P, _P, _P, _P, _F32, _P,
                                    _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _I64, _P]),
    "cdssm_fused_scan_fwd_noalloc": (_I32, [_I32] + [_P] * 9 + [_F32] + [_P] * 3 + [_I64] * 6 + [_P]),
    "cdssm_fused_scan_bwd_workspace_bytes": (_I64, [_I64, _I64, _I64, _I64, _I64, _I64]),
    "cdssm_fused_scan_bwd": (_I32, [_I32, _P, _P, _P, _P, _P, _P, _P, _P, _P, _F32, _P, _P, _P,
                                    _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P,
                                    _I64, _I64, _I64, _I64, _I64, _I64, _P]),
    "cdssm_fused_scan_bwd_stamped": (_I32, [_I32, _P, _P, _P, _P, _P, _P, _P, _P, _P, _F32, _P, _P, _P,
                                            _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P,
                                            _I64, _I64, _I64, _I64, _I64, _I64, _P, _I64, _P]),
    "cdssm_fused_scan_fwd_train": (_I32, [_I32, _P, _P, _P, _P, _P, _P, _P, _P, _P, _F32, _P,
                                          _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _I64, _P]),
    "cdssm_skinny_gemm": (_I32, [_I32, _P, _I64, _P, _I64, _P, _P, _I64, _P, _F32, _P, _I64, _I64, _I64, _I64, _P]),
    "cdssm_fused_scan_fwd_stamped": (_I32, [_I32] + [_P] * 9 + [_F32] + [_P] * 4 + [_I64] * 6 + [_P, _I64, _P]),
    "cdssm_fused_scan_fwd_continue": (_I32, [_I32] + [_P] * 9 + [_F32] + [_P] * 4 + [_I64] * 6 + [_P]),
    "cdssm_fused_scan_fwd_train_continue": (_I32, [_I32] + [_P] * 9 + [_F32] + [_P] * 4 + [_I64] * 6 + [_P]),
    "cdssm_fused_scan_bwd_continue": (_I32, [_I32] + [_P] * 9 + [_F32] + [_P] * 14 + [_I64] * 6 + [_P]),
    "cdssm_fused_scan_fwd_profile": (_I32, [_I32, _P, _P, _P, _P, _P, _P, _P, _P, _P, _F32, _P,
                                            _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _I64, _P, _I32, _I32,
                                            _P]),
    "cdssm_fused_scan_bwd_profile": (_I32, [_I32, _P, _P, _P, _P, _P, _P, _P, _P, _P, _F32, _P, _P, _P,
                                            _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P,
                                            _I64, _I64, _I64, _I64, _I64, _I64, _P, _I32, _P]),
    "cdssm_fused_scan_fwd_abar": (_I32, [_I32] + [_P] * 11 + [_I64] * 6 + [_P]),
    "cdssm_fused_scan_fwd_abar_train": (_I32, [_I32] + [_P] * 11 + [_I64] * 6 + [_P]),
    "cdssm_fused_scan_bwd_abar": (_I32, [_I32] + [_P] * 19 + [_I64] * 6 + [_P]),
    "cdssm_ssd_scan_workspace_bytes": (_I64, [_I64] * 6),
    "cdssm_chunked_scan_workspace_bytes": (_I64, [_I64] * 6),
    "cdssm_chunked_scan_fwd_abar": (_I32, [_I32] + [_P] * 12 + [_I64] * 6 + [_P]),
    "cdssm_ssd_scan_bwd_workspace_bytes": (_I64, [_I64] * 6),
    "cdssm_ssd_scan_fwd": (_I32, [_I32] + [_P] * 7 + [_I64] * 6 + [_I32, _P]),
    "cdssm_ssd_scan_bwd": (_I32, [_I32] + [_P] * 11 + [_I64] * 6 + [_P]),
    "cdssm_conv1d_silu_fwd": (_I32, [_I32] + [_P] * 4 + [_I64] * 4 + [_P]),
    "cdssm_conv1d_silu_fwd_strided": (_I32, [_I32, _P, _I64] + [_P] * 3 + [_I64] * 4 + [_P]),
    "cdssm_conv1d_silu_bwd_workspace_bytes": (_I64, [_I64] * 4),
    "cdssm_conv1d_silu_bwd": (_I32, [_I32, _P, _I64] + [_P] * 7 + [_I64] * 4 + [_P]),
    "cdssm_rms_norm_fwd": (_I32, [_I32, _P, _P, _P, _I64, _I64, _F32, _P]),
    "cdssm_normalize_kq_qk_fwd": (_I32, [_I32, _P, _I64, _P, _I64, _P, _P, _P, _I64, _I64, _I64, _P]),
    "cdssm_shortcut_readout_fwd": (_I32, [_I32] + [_P] * 6 + [_I64, _P]),
    "cdssm_shortcut_readout_rows_partials": (_I64, [_I64, _I64]),
    "cdssm_col_sum_workspace_bytes": (_I64, [_I64, _I64]),
    "cdssm_slab_sum": (_I32, [_I32, _P, _I64, _I64, _P, _P]),
    "cdssm_col_sum": (_I32, [_I32, _P, _I64, _I64, _I64, _P, _P, _P]),
    "cdssm_shortcut_readout_rows_fwd": (_I32, [_I32] + [_P] * 6 + [_I64, _I64, _P]),
    "cdssm_shortcut_readout_rows_bwd": (_I32, [_I32] + [_P] * 11 + [_I64, _I64, _P]),
    "cdssm_state_readout_fwd": (_I32, [_I32] + [_P] * 3 + [_I64] * 3 + [_P]),
    "cdssm_state_readout_bwd": (_I32, [_I32] + [_P] * 5 + [_I64] * 3 + [_P]),
    "cdssm_group_norm_workspace_bytes": (_I64, [_I64, _I64, _I64]),
    "cdssm_rms_norm_bwd_workspace_bytes": (_I64, [_I64, _I64]),
    "cdssm_rms_norm_bwd": (_I32, [_I32, _P, _P, _P, _P, _P, _P, _I64, _I64, _F32, _P]),
    "cdssm_normalize_kq_qk_bwd": (_I32, [_I32, _P, _I64, _P, _I64, _P, _P, _P, _P, _P, _I64, _I64, _I64, _P]),
    "cdssm_group_norm_gate_bwd_workspace_bytes": (_I64, [_I64, _I64, _I64, _I64]),
    "cdssm_group_norm_gate_bwd": (_I32, [_I32, _I32, _P, _P, _P, _P, _I64, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P,
                                         _P, _I64, _I64, _I64, _I64, _P]),
    "cdssm_group_norm_gate_fwd": (_I32, [_I32, _I32, _P, _P, _P, _P, _I64, _P, _P, _P, _P, _I64, _I64, _I64, _I64,
                                         _F32, _P]),
    "cdssm_decode_init": (_I32, [_P, _P, _P, _P, _I64, _I64, _I64, _I64, _P]),
    "cdssm_decode_step": (_I32, [_I32] + [_P] * 9 + [_F32] + [_P] * 5 + [_I64] * 5 + [_P]),
    "cdssm_decode_step_abar": (_I32, [_I32] + [_P] * 12 + [_I64] * 5 + [_P]),
    "cdssm_decode_block_tail": (_I32, [_I32, _I32, _P, _I64, _P, _I64, _I64, _I64, _P, _P, _P, _P, _F32, _F32, _F32,
                                        _F32, _F32, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _I64, _P, _P, _P,
                                        _I64, _I64, _I64, _I64, _I64, _I64, _I64, _F32, _P]),
    "cdssm_decode_block_token": (_I32, [_I32, _P, _I64, _P, _I64, _I64, _I64, _P, _P, _P, _P] + [_F32] * 5 +
                                 [_P] * 7 + [_I64] * 5 + [_P]),
    "cdssm_dynamics_fused_fwd_at": (_I32, [_I32, _P, _P, _P] + [_F32] * 5 + [_P] * 4 + [_I64] * 5 + [_P, _P]),
    "cdssm_conv1d_silu_step": (_I32, [_I32, _P, _I64, _P, _P, _P, _P, _I64, _I64, _I64, _P]),
    "cdssm_group_norm_gate_step": (_I32, [_I32, _I32, _P, _P, _P, _P, _P, _I64, _P, _P, _P, _I64, _I64, _I64, _F32,
                                          _P, _P]),
    "cdssm_readout_group_norm_gate_step": (_I32, [_I32, _I32, _P, _P, _I64, _P, _P, _P, _P, _I64, _P, _P, _P, _I64,
                                                  _I64, _I64, _F32, _P, _P]),
    "cdssm_intra_chunk_scan_fwd": (_I32, [_I32] + [_P] * 6 + [_I64] * 5 + [_P]),
    "cdssm_intra_chunk_scan_bwd": (_I32, [_I32] + [_P] * 12 + [_I64] * 5 + [_P]),
    "cdssm_inter_chunk_scan_fwd": (_I32, [_I32] + [_P] * 3 + [_I64] * 5 + [_P]),
    "cdssm_inter_chunk_scan_bwd": (_I32, [_I32] + [_P] * 5 + [_I64] * 5 + [_P]),
    "cdssm_exact_correction_fwd": (_I32, [_I32] + [_P] * 5 + [_I64] * 6 + [_P]),
    "cdssm_exact_correction_bwd": (_I32, [_I32] + [_P] * 10 + [_I64] * 6 + [_P]),
    "cdssm_dynamics_fused_fwd": (_I32, [_I32, _P, _P, _P] + [_F32] * 5 + [_P] * 4 + [_I64] * 4 + [_P]),
    "cdssm_dynamics_fused_bwd_workspace_bytes": (_I64, [_I64] * 3),
    "cdssm_dynamics_fused_bwd": (_I32, [_I32] + [_P] * 7 + [_F32] * 5 + [_P] * 3 + [_I64] * 4 + [_P]),
    "cdssm_normalize_kq_fwd": (_I32, [_I32] + [_P] * 4 + [_I64] * 2 + [_P]),
    "cdssm_normalize_kq_bwd": (_I32, [_I32] + [_P] * 6 + [_I64] * 2 + [_P]),
}

_lock = threading.Lock()
_lib: Optional[ctypes.CDLL] = None
_load_error: Optional[str] = None


def load() -> ctypes.CDLL:
    """Load the HIP library once; raise RuntimeError if it is absent or broken."""
    global _lib, _load_error
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not os.path.exists(LIB_PATH):
            _load_error = (f"{LIB_PATH} not found: build it with "
                           f"`python -c 'import __graft_entry__ as g; g.build()'` from the repo root")
            raise RuntimeError(_load_error)
        lib = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        _lib = lib
        return lib


def last_error() -> str:
    msg = load().cdssm_last_error()
    return msg.decode() if msg else ""


def check(status: int, op: str) -> None:
    if status != 0:
        raise RuntimeError(f"{op} failed (status {status}): {last_error()}")


def ptr(t: Optional[torch.Tensor]) -> Optional[int]:
    return None if t is None else t.data_ptr()


_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def stream_of(device: torch.device) -> int:
    """The current HIP stream of ``device`` as an integer handle (torch's raw-stream query where this build
    has it: 0.05 us against 1.9 us for current_stream(device).cuda_stream on the MI355X boxes' hosts, and a
    training step makes some thirty of these calls)."""
    if _raw_stream is not None:
        idx = device.index if device.index is not None else torch.cuda.current_device()
        return _raw_stream(idx)
    return torch.cuda.current_stream(device).cuda_stream


DTYPE_CODE = {torch.float32: 0, torch.bfloat16: 1}
