"""``SSDChunkwiseScan``: the reference module (ssd.py:31-111) over the HIP ops.

Same constructor, forward signature and result as the reference.  Two
executions of the same algorithm:

* fused (even state_dim up to 32, head_dim 64 or 128, chunk <= 128, one float
  dtype on the GPU): ``scan.SSDScanFn``, one forward call (cdssm_ssd_scan_fwd)
  that writes Y once, and one backward call (cdssm_ssd_scan_bwd) with the
  reference's gradient rules; each of a head's N / 2 complex state rows is
  scanned as a virtual head sharing the head's k and beta; intermediate states
  stay fp32 (the reference rounds local_h, chunk_states and corrections to the
  input dtype between passes);
* per-pass (any other shape): pad the sequence to whole chunks with zeros
  (A_bar = 0 on padded steps), run the intra-chunk scan, take the chunk
  summaries (total_A = cum_A[:, :, -1], final_local_h = local_h[:, :, -1]), run
  the inter-chunk scan and the exact correction, return Y = local_h +
  correction cut back to length L -- the reference's own sequence of ops.
"""

from __future__ import annotations

import math
from typing import Optional

import torch
import torch.nn as nn
import torch.nn.functional as F
from torch import Tensor

from .ops import ExactCorrectionFn, InterChunkScanFn, IntraChunkScanFn
from .scan import SSDScanFn


class SSDChunkwiseScan(nn.Module):
    """Chunkwise scan with complex-diagonal Cayley dynamics and delta-rule updates."""

    def __init__(self, chunk_size: int, state_dim: int, fused: Optional[bool] = None):
        """``fused``: None takes the fused kernels where they apply, True requires them, False runs
        the per-pass ops."""
        super().__init__()
        self.chunk_size = chunk_size
        self.state_dim = state_dim
        self.fused = fused

    def fused_applies(self, A_bar: Tensor, K: Tensor, V: Tensor, beta: Tensor) -> bool:
        """Whether the fused kernels serve these inputs."""
        return (2 <= self.state_dim <= 32 and self.state_dim % 2 == 0 and K.dim() == 4 and K.is_cuda
                and V.shape[-1] == self.state_dim and K.shape[-1] in (64, 128)
                and 1 <= self.chunk_size <= 128 and K.dtype in (torch.float32, torch.bfloat16)
                and all(t.dtype == K.dtype and t.device == K.device for t in (A_bar, V, beta)))

    def forward(self, A_bar: Tensor, K: Tensor, V: Tensor, beta: Tensor) -> Tensor:
        """A_bar (B,L,H,N), K (B,L,H,D), V (B,L,H,N), beta (B,L,H) -> Y (B,L,H,N,D)."""
        if self.fused is not False:
            if self.fused_applies(A_bar, K, V, beta):
                return SSDScanFn.apply(A_bar, K, V, beta, self.chunk_size)
            if self.fused:
                raise ValueError("the fused SSD scan needs an even state_dim <= 32, head_dim 64 or 128, "
                                 "chunk_size <= 128 and float32 or bfloat16 inputs of one dtype on the GPU")
        B, L, H, D = K.shape
        N = self.state_dim
        C = self.chunk_size
        n_chunks = math.ceil(L / C)
        pad = n_chunks * C - L
        if pad > 0:
            A_bar = F.pad(A_bar, (0, 0, 0, 0, 0, pad))
            K = F.pad(K, (0, 0, 0, 0, 0, pad))
            V = F.pad(V, (0, 0, 0, 0, 0, pad))
            beta = F.pad(beta, (0, 0, 0, pad))
        A_chunk = A_bar.reshape(B, n_chunks, C, H, N)
        K_chunk = K.reshape(B, n_chunks, C, H, D)
        V_chunk = V.reshape(B, n_chunks, C, H, N)
        beta_chunk = beta.reshape(B, n_chunks, C, H)

        local_h, cum_A = IntraChunkScanFn.apply(A_chunk.reshape(B * n_chunks, C, H, N),
                                                K_chunk.reshape(B * n_chunks, C, H, D),
                                                V_chunk.reshape(B * n_chunks, C, H, N),
                                                beta_chunk.reshape(B * n_chunks, C, H), N)
        local_h = local_h.view(B, n_chunks, C, H, N, D)
        cum_A = cum_A.view(B, n_chunks, C, H, N)
        chunk_states = InterChunkScanFn.apply(cum_A[:, :, -1], local_h[:, :, -1], N)
        correction = ExactCorrectionFn.apply(A_chunk, K_chunk, beta_chunk, chunk_states, N)
        Y = (local_h + correction).reshape(B, -1, H, N, D)
        if pad > 0:
            Y = Y[:, :L]
        return Y
