"""MI355X-native (gfx950 HIP) CD-SSM chunkwise delta-rule scan.

Host side of the HIP library ``libcdssm_hip.so``: the fused scan op and the
reference-compatible autograd Functions.  Importing this package does not
touch the GPU; the library is loaded on first use and its absence is an error.
"""

from .scan import (ChunkwiseDeltaScanAbarFn, ChunkwiseDeltaScanFn, SSDScanFn, check_lookback,  # noqa: F401
                   chunked_scan_abar, chunkwise_delta_scan, chunkwise_delta_scan_abar, chunkwise_delta_scan_bwd,
                   chunkwise_delta_scan_fwd, chunkwise_delta_scan_train, lookback_status, set_forward_path,
                   ssd_scan_bwd, ssd_scan_fwd)

from .ops import (DynamicsFusedFn, ExactCorrectionFn, InterChunkScanFn,  # noqa: F401
                  IntraChunkScanFn, NormalizeKQFn)
from .ssd import SSDChunkwiseScan  # noqa: F401
from .decode import DecodeState, decode_step, prefill  # noqa: F401

__all__ = ["DynamicsFusedFn", "NormalizeKQFn", "IntraChunkScanFn", "InterChunkScanFn", "ExactCorrectionFn",
           "SSDChunkwiseScan", "SSDScanFn", "ssd_scan_fwd", "ssd_scan_bwd", "ChunkwiseDeltaScanFn", "ChunkwiseDeltaScanAbarFn", "chunkwise_delta_scan",
           "chunkwise_delta_scan_abar", "chunked_scan_abar", "chunkwise_delta_scan_fwd",
           "chunkwise_delta_scan_bwd", "chunkwise_delta_scan_train", "set_forward_path", "lookback_status",
           "check_lookback", "DecodeState",
           "decode_step", "prefill"]
