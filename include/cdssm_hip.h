/*
 * cdssm_hip.h -- C-ABI of the MI355X (gfx950) CD-SSM scan library.
 *
 * Every entry point takes raw device pointers to contiguous tensors, int64
 * sizes, fp32 scalars and the hipStream_t to launch on; it allocates nothing,
 * keeps no pointer past the call, launches asynchronously on that stream and
 * returns 0 on success, a negative status on invalid arguments (-1) or a HIP
 * launch error (-2).  cdssm_last_error() describes the last failure on the
 * calling thread.
 *
 * dtype codes: 0 = fp32, 1 = bf16 (raw 16-bit patterns).
 * Layouts are the reference's (token-major, complex pairs interleaved re/im).
 */
#ifndef CDSSM_HIP_H
#define CDSSM_HIP_H

#include <stdint.h>
#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Version of this ABI (bumped on incompatible change). */
int cdssm_abi_version(void);

/* Message describing the last non-zero status returned on this thread. */
const char* cdssm_last_error(void);

/*
 * Fused chunkwise delta-rule scan, forward (R-mode: the reference ops.py
 * algorithm).  Replaces, in one call, the scan-level path
 *   DynamicsFusedFn (Cayley + gating + VP, dynamics_fused.cu:109-131)
 *   -> V * vp (block.py:194-195)
 *   -> SSDChunkwiseScan.forward (ssd.py:39-111):
 *        IntraChunkScanFn   (ops.py:107-121, intra_chunk_scan.cu:560-609)
 *        InterChunkScanFn   (ops.py:146-155, inter_chunk_scan.cu:201-234)
 *        ExactCorrectionFn  (ops.py:173-186, exact_correction.cu:390-438)
 *        Y = local_h + correction (ssd.py:102)
 *   -> readout y = sel_C * (Y . q) (block.py:208-211).
 * Shapes: q, k (B,L,H,D); v (B,L,H,N); beta, sel_c, dt, r (B,L,H), all of
 * `dtype`; alpha, omega (H,) fp32; h0 (B,H,N,D) fp32 or NULL (zero state);
 * outputs y (B,L,H,N) of `dtype`, h_final (B,H,N,D) fp32 (the R-mode carry
 * after the last token; an extension -- the reference has no state output).
 * workspace: cdssm_fused_scan_workspace_bytes() bytes; on return it holds the
 * state entering every chunk, (B, L/chunk, H, D) complex fp32, which the
 * backward consumes.  Supported: N = 2, D in {64, 128}, 1 <= chunk <= 128.
 */
int64_t cdssm_fused_scan_workspace_bytes(int64_t B, int64_t L, int64_t H, int64_t D, int64_t N,
                                         int64_t chunk);
int cdssm_fused_scan_fwd(int dtype, const void* q, const void* k, const void* v, const void* beta,
                         const void* sel_c, const void* dt, const void* r, const float* alpha,
                         const float* omega, float c, const float* h0, void* y, float* h_final,
                         float* workspace, int64_t B, int64_t L, int64_t H, int64_t D, int64_t N,
                         int64_t chunk, hipStream_t stream);

/*
 * Fused scan, backward.  Gradients are those the reference ops.py autograd
 * path produces for the same forward: exact for the readout (block.py:208-211),
 * for IntraChunkScanFn.backward (ops.py:123-135, intra_chunk_scan.cu:611-674)
 * and for InterChunkScanFn.backward (ops.py:158-163, inter_chunk_scan.cu:236-275);
 * for ExactCorrectionFn.backward (ops.py:189-195, exact_correction.cu:440-498)
 * the reference's own rule, which treats grad_corrections[t] as the gradient
 * of the state after step t; and the exact chain rule of the scan-level
 * Cayley/gating formula for dt, r, alpha, omega.
 * Inputs: the forward's inputs, dy (B,L,H,N) of `dtype`, dh_final (B,H,N,D)
 * fp32 or NULL, and fwd_workspace as filled by cdssm_fused_scan_fwd.
 * Outputs: dq, dk, dv, dbeta, dsel_c, ddt, dr (shapes/dtype of the inputs),
 * dalpha, domega (H,) fp32, dh0 (B,H,N,D) fp32 or NULL.
 * workspace: cdssm_fused_scan_bwd_workspace_bytes() bytes.
 */
int64_t cdssm_fused_scan_bwd_workspace_bytes(int64_t B, int64_t L, int64_t H, int64_t D, int64_t N,
                                             int64_t chunk);
int cdssm_fused_scan_bwd(int dtype, const void* q, const void* k, const void* v, const void* beta,
                         const void* sel_c, const void* dt, const void* r, const float* alpha,
                         const float* omega, float c, const void* dy, const float* dh_final,
                         const float* fwd_workspace, void* dq, void* dk, void* dv, void* dbeta,
                         void* dsel_c, void* ddt, void* dr, float* dalpha, float* domega, float* dh0,
                         float* workspace, int64_t B, int64_t L, int64_t H, int64_t D, int64_t N,
                         int64_t chunk, hipStream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* CDSSM_HIP_H */
