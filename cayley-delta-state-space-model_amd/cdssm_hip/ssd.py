"""``SSDChunkwiseScan``: the reference module (ssd.py:31-111) over the HIP ops.

Same constructor, forward signature and result as the reference: pad the
sequence to whole chunks with zeros (A_bar = 0 on padded steps), run the
intra-chunk scan, take the chunk summaries (total_A = cum_A[:, :, -1],
final_local_h = local_h[:, :, -1]), run the inter-chunk scan and the exact
correction, return Y = local_h + correction cut back to length L.
"""

from __future__ import annotations

import math

import torch.nn as nn
import torch.nn.functional as F
from torch import Tensor

from .ops import ExactCorrectionFn, InterChunkScanFn, IntraChunkScanFn


class SSDChunkwiseScan(nn.Module):
    """Chunkwise scan with complex-diagonal Cayley dynamics and delta-rule updates."""

    def __init__(self, chunk_size: int, state_dim: int):
        super().__init__()
        self.chunk_size = chunk_size
        self.state_dim = state_dim

    def forward(self, A_bar: Tensor, K: Tensor, V: Tensor, beta: Tensor) -> Tensor:
        """A_bar (B,L,H,N), K (B,L,H,D), V (B,L,H,N), beta (B,L,H) -> Y (B,L,H,N,D)."""
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
