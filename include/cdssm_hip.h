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
 * workspace: cdssm_fused_scan_workspace_bytes() bytes of device memory, any
 * contents (scratch for this call; the backward takes the workspace of
 * cdssm_fused_scan_fwd_train instead; the size function also takes the
 * gate-level form's even N <= 32).  Supported: N = 2, D in {64, 128},
 * 1 <= chunk <= 128; q, k 16-byte aligned, y aligned to one (re, im) pair
 * (4 bytes bf16, 8 fp32).  Where every segment of 4 chunks fits in one round of
 * resident workgroups (or, for this inference forward, the segments fill
 * whole rounds of a persistent grid), the scan runs as one launch (chunk maps
 * composed by a look-back between workgroups); otherwise as four (chunk
 * summaries, carry fold, carry replay, main pass).
 */
int64_t cdssm_fused_scan_workspace_bytes(int64_t B, int64_t L, int64_t H, int64_t D, int64_t N,
                                         int64_t chunk);
int cdssm_fused_scan_fwd(int dtype, const void* q, const void* k, const void* v, const void* beta,
                         const void* sel_c, const void* dt, const void* r, const float* alpha,
                         const float* omega, float c, const float* h0, void* y, float* h_final,
                         float* workspace, int64_t B, int64_t L, int64_t H, int64_t D, int64_t N,
                         int64_t chunk, hipStream_t stream);

/*
 * The inference forward above with no workspace argument and no allocation.
 * No counterpart in the reference: for callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc).  Its scratch (the look-back area and carry arrays) is a
 * static 32 MiB device array inside the library, one per GPU, held until the
 * process ends; shapes needing more return -1 with a message naming the size
 * (C1 needs 6.7 MB, C3 26.6 MB).  Every call on a GPU shares that GPU's array:
 * calls that overlap on one GPU (concurrent streams) race and must not be
 * issued.  Nothing in the array needs clearing between calls.  Results are
 * bit-identical to cdssm_fused_scan_fwd on the same inputs.  Arguments and
 * limits otherwise as cdssm_fused_scan_fwd.
 */
int cdssm_fused_scan_fwd_noalloc(int dtype, const void* q, const void* k, const void* v, const void* beta,
                                 const void* sel_c, const void* dt, const void* r, const float* alpha,
                                 const float* omega, float c, const float* h0, void* y, float* h_final,
                                 int64_t B, int64_t L, int64_t H, int64_t D, int64_t N, int64_t chunk,
                                 hipStream_t stream);

/*
 * The fused forward on gate-level inputs, for the model's block
 * (block.py:177-211): instead of the scan-level dt, r, alpha, omega, c it takes
 * the transition a_bar (B,L,H,N) and VP scale vp (B,L,H,N/2), both of `dtype`,
 * as DynamicsFusedFn produces them (ops.py:39-66, dynamics_fused.cu:35-140),
 * and computes SSDChunkwiseScan(A_bar, K, V * vp, beta) (ssd.py:39-111) with the
 * readout y = sel_C (Y . q) (block.py:194-211, shortcut excluded).  N even,
 * 2 <= N <= 32: the N / 2 complex state rows of a head share its k, q, beta and
 * sel_c and are scanned as virtual heads (v, a_bar, y (B,L,H,N), vp (B,L,H,N/2),
 * h0 / h_final (B,H,N,D) in the reference's layouts).  Other arguments,
 * workspace (cdssm_fused_scan_workspace_bytes with this N) and limits as
 * cdssm_fused_scan_fwd.  Inference only.
 */
int cdssm_fused_scan_fwd_abar(int dtype, const void* q, const void* k, const void* v, const void* beta,
                              const void* sel_c, const void* a_bar, const void* vp, const float* h0, void* y,
                              float* h_final, float* workspace, int64_t B, int64_t L, int64_t H, int64_t D,
                              int64_t N, int64_t chunk, hipStream_t stream);

/*
 * Training path of the gate-level form: the scan the block's training step
 * runs (block.py:181-211 under autograd, trainer.py:235-247) without writing
 * the (B,L,H,2,D) Y that SSDChunkwiseScan returns (ssd.py:39-111; the reference
 * stores it, and its passes' states, for its backward, ops.py:119,153,184).
 * cdssm_fused_scan_fwd_abar_train: the forward above that also stores in the
 * workspace what the backward reads (the records of cdssm_fused_scan_fwd_train).
 * cdssm_fused_scan_bwd_abar: given dy (B,L,H,N), dh_final (B,H,N,D) fp32 or
 * NULL and that workspace, writes dq, dk (B,L,H,D), dv (B,L,H,N), dbeta,
 * dsel_c (B,L,H), da_bar (B,L,H,N), dvp (B,L,H,N/2) of `dtype` and dh0
 * (B,H,N,D) fp32 or NULL: the gradients ops.py's autograd yields through
 * SSDChunkwiseScan and the readout (exact for the readout, the local and carry
 * branches; the correction branch's shifted rule, exact_correction.cu:213-382),
 * with d A_bar and d vp in place of the scan-level dynamics chain of
 * cdssm_fused_scan_bwd.  N even, 2 <= N <= 32 as in the forward; for N > 2
 * the gradients of the shared dq, dk, dbeta, dsel_c are summed over the head's
 * state rows in a fixed order (bit-reproducible).  workspace:
 * cdssm_fused_scan_bwd_workspace_bytes() with this N (for N > 2 it holds the
 * fp32 per-row partials of those sums).
 */
int cdssm_fused_scan_fwd_abar_train(int dtype, const void* q, const void* k, const void* v, const void* beta,
                                    const void* sel_c, const void* a_bar, const void* vp, const float* h0, void* y,
                                    float* h_final, float* workspace, int64_t B, int64_t L, int64_t H, int64_t D,
                                    int64_t N, int64_t chunk, hipStream_t stream);
int cdssm_fused_scan_bwd_abar(int dtype, const void* q, const void* k, const void* v, const void* beta,
                              const void* sel_c, const void* a_bar, const void* vp, const void* dy,
                              const float* dh_final, const float* fwd_workspace, void* dq, void* dk, void* dv,
                              void* dbeta, void* dsel_c, void* da_bar, void* dvp, float* dh0, float* workspace,
                              int64_t B, int64_t L, int64_t H, int64_t D, int64_t N, int64_t chunk,
                              hipStream_t stream);

/*
 * Gate-level readout form for state_dim N = 16 (the reference's default,
 * config/model.py:128) in the chunked (UT) form on the matrix cores, inference:
 * replaces SSDChunkwiseScan.forward (ssd.py:39-111: IntraChunkScanFn,
 * InterChunkScanFn, ExactCorrectionFn, Y = local_h + correction) followed by
 * the block's readout y = sel_C * (Y . q) (block.py:194-211) without forming
 * Y (B,L,H,16,D).  bf16 only (dtype 1): q, k (B,L,H,D) 16-byte aligned, v
 * (B,L,H,16) and a_bar (B,L,H,16) 8-byte aligned, vp (B,L,H,8) 4-byte aligned,
 * beta, sel_c (B,L,H); h0 (B,H,16,D) fp32 or NULL; shortcut_scale: one fp32 on
 * the device, or NULL -- when given, y also carries the current-token shortcut
 * sel_C * scale * (q.k)^2 * vp v (block.py:202-208), as the block's retrieved
 * vector; outputs y (B,L,H,16) bf16 (8-byte aligned) and h_final (B,H,16,D)
 * fp32 or NULL.  D in {64, 128}; chunk a multiple of 16 in [16, 256].  workspace:
 * cdssm_chunked_scan_workspace_bytes() bytes, 16-byte aligned (-1: the shape
 * is not supported).  Three launches: the local pass, the carry, the
 * correction pass.
 */
int64_t cdssm_chunked_scan_workspace_bytes(int64_t B, int64_t L, int64_t H, int64_t D, int64_t N, int64_t chunk);
int cdssm_chunked_scan_fwd_abar(int dtype, const void* q, const void* k, const void* v, const void* beta,
                                const void* sel_c, const void* a_bar, const void* vp, const float* h0,
                                const float* shortcut_scale, void* y, float* h_final, float* workspace, int64_t B,
                                int64_t L, int64_t H, int64_t D, int64_t N, int64_t chunk, hipStream_t stream);

/*
 * Training forward (no counterpart in the reference; the reference keeps its
 * passes' full outputs for backward instead): the forward above, which also
 * stores in the workspace what the backward reads: per (token, head) the dot
 * products of the chunk recurrences (p_t = z_{t-1}.k_t, c^_t.k_t,
 * c^_{t+1}.q_t, Y_t.q_t; 32 bytes) and g_t, the local state every 8 tokens and
 * the correction state after every chunk, so that the backward rebuilds the
 * chunk states without reductions or a forward recompute.  Same arguments and
 * workspace size as cdssm_fused_scan_fwd.
 */
int cdssm_fused_scan_fwd_train(int dtype, const void* q, const void* k, const void* v, const void* beta,
                               const void* sel_c, const void* dt, const void* r, const float* alpha,
                               const float* omega, float c, const float* h0, void* y, float* h_final,
                               float* workspace, int64_t B, int64_t L, int64_t H, int64_t D, int64_t N,
                               int64_t chunk, hipStream_t stream);

/*
 * cdssm_fused_scan_fwd and cdssm_fused_scan_fwd_train for a workspace whose
 * previous use was a call of one of these four forward entries with the same
 * shape, completed or ordered earlier on the same stream, with the workspace
 * untouched since.  No counterpart in the reference: for callers that keep a
 * workspace across calls (serving loops, training steps, captured graphs).
 * Every one-launch pass draws a look-back epoch, a tag that tells this call's
 * flags from earlier calls' in the never-cleared workspace; the entries above
 * launch a one-thread kernel for it, while these reuse the one that the
 * previous call's last workgroup left in the workspace (one launch per call
 * instead of two).  Results are bit-identical to the entries above.  Calling
 * them on a workspace that has not held such a call, or whose contents were
 * changed since, may read stale look-back flags as ready.
 */
int cdssm_fused_scan_fwd_continue(int dtype, const void* q, const void* k, const void* v, const void* beta,
                                  const void* sel_c, const void* dt, const void* r, const float* alpha,
                                  const float* omega, float c, const float* h0, void* y, float* h_final,
                                  float* workspace, int64_t B, int64_t L, int64_t H, int64_t D, int64_t N,
                                  int64_t chunk, hipStream_t stream);
int cdssm_fused_scan_fwd_train_continue(int dtype, const void* q, const void* k, const void* v, const void* beta,
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
 * fp32 or NULL, and fwd_workspace as filled by cdssm_fused_scan_fwd_train.
 * Outputs: dq, dk, dv, dbeta, dsel_c, ddt, dr (shapes/dtype of the inputs),
 * dalpha, domega (H,) fp32, dh0 (B,H,N,D) fp32 or NULL.
 * workspace: cdssm_fused_scan_bwd_workspace_bytes() bytes.
 */
int64_t cdssm_fused_scan_bwd_workspace_bytes(int64_t B, int64_t L, int64_t H, int64_t D, int64_t N,
                                             int64_t chunk);

/*
 * Instrumentation (no reference counterpart): cdssm_fused_scan_bwd, recording
 * the 100 MHz real-time counter (s_memrealtime) per wave at 8 points of the
 * one-launch correction adjoint + carry (entry, staged, lambda pass done,
 * segment map published, look-back wait done, carry folded, left-end state
 * published, end; word (workgroup * 4 + wave) * 8 + point) and at 4 points of
 * the main pass (entry, staged, reverse pass done, end; word M + workgroup * 4
 * + point, M = NSEG * B * H * 32, NSEG = ceil(ceil(L / chunk) / 4)).  stamps:
 * device memory of stamps_len 8-byte words, at least M + B * ceil(L / chunk) *
 * H * 4; the caller clears it to tell unwritten records.  Returns -1 (nothing
 * launched) if the buffer is too small or the shape runs the three-launch
 * correction adjoint.  Results are bit-identical to cdssm_fused_scan_bwd.
 */
int cdssm_fused_scan_bwd_stamped(int dtype, const void* q, const void* k, const void* v, const void* beta,
                                 const void* sel_c, const void* dt, const void* r, const float* alpha,
                                 const float* omega, float c, const void* dy, const float* dh_final,
                                 const float* fwd_workspace, void* dq, void* dk, void* dv, void* dbeta,
                                 void* dsel_c, void* ddt, void* dr, float* dalpha, float* domega, float* dh0,
                                 float* workspace, int64_t B, int64_t L, int64_t H, int64_t D, int64_t N,
                                 int64_t chunk, unsigned long long* stamps, int64_t stamps_len, hipStream_t stream);
int cdssm_fused_scan_bwd(int dtype, const void* q, const void* k, const void* v, const void* beta,
                         const void* sel_c, const void* dt, const void* r, const float* alpha,
                         const float* omega, float c, const void* dy, const float* dh_final,
                         const float* fwd_workspace, void* dq, void* dk, void* dv, void* dbeta,
                         void* dsel_c, void* ddt, void* dr, float* dalpha, float* domega, float* dh0,
                         float* workspace, int64_t B, int64_t L, int64_t H, int64_t D, int64_t N,
                         int64_t chunk, hipStream_t stream);

/*
 * cdssm_fused_scan_bwd for a workspace whose previous use was a call of this
 * entry or cdssm_fused_scan_bwd with the same shape, completed or ordered
 * earlier on the same stream, with the workspace untouched since: the
 * one-launch correction adjoint + carry reuses the look-back epoch the
 * previous call left (as cdssm_fused_scan_fwd_continue; no counterpart in the
 * reference).  Results are bit-identical to cdssm_fused_scan_bwd.
 */
int cdssm_fused_scan_bwd_continue(int dtype, const void* q, const void* k, const void* v, const void* beta,
                                  const void* sel_c, const void* dt, const void* r, const float* alpha,
                                  const float* omega, float c, const void* dy, const float* dh_final,
                                  const float* fwd_workspace, void* dq, void* dk, void* dv, void* dbeta,
                                  void* dsel_c, void* ddt, void* dr, float* dalpha, float* domega, float* dh0,
                                  float* workspace, int64_t B, int64_t L, int64_t H, int64_t D, int64_t N,
                                  int64_t chunk, hipStream_t stream);

/*
 * SSDChunkwiseScan on the fused kernels, forward: replaces SSDChunkwiseScan.forward
 * (ssd.py:39-111), i.e. IntraChunkScanFn (ops.py:108-121, intra_chunk_scan.cu:560-609),
 * InterChunkScanFn (ops.py:146-155, inter_chunk_scan.cu:201-234), ExactCorrectionFn
 * (ops.py:173-186, exact_correction.cu:390-438) and Y = local_h + corrections, for even
 * state_dim 2 <= N <= 32.  Inputs of `dtype`: a_bar (B,L,H,N), k (B,L,H,D), v (B,L,H,N)
 * (already VP-scaled, as block.py:194-195 passes it), beta (B,L,H).  Output Y (B,L,H,N,D) of
 * `dtype` (16-byte aligned) and h_final (B,H,N,D) fp32, the carry after the last token (the
 * scan starts from zero, as the reference's).  Each head's N / 2 complex state rows are scanned
 * as virtual heads sharing the head's k rows and beta (the rows' recurrences are independent);
 * intermediate states stay fp32.  train != 0 also writes what cdssm_ssd_scan_bwd reads into the
 * workspace (cdssm_ssd_scan_workspace_bytes() bytes).  Limits otherwise as cdssm_fused_scan_fwd,
 * with H N / 2 heads.
 */
int64_t cdssm_ssd_scan_workspace_bytes(int64_t B, int64_t L, int64_t H, int64_t D, int64_t N, int64_t chunk);
int cdssm_ssd_scan_fwd(int dtype, const void* a_bar, const void* k, const void* v, const void* beta, void* Y,
                       float* h_final, float* workspace, int64_t B, int64_t L, int64_t H, int64_t D, int64_t N,
                       int64_t chunk, int train, hipStream_t stream);

/*
 * SSDChunkwiseScan on the fused kernels, backward: replaces the autograd backward of
 * SSDChunkwiseScan through IntraChunkScanFn.backward (ops.py:123-135), InterChunkScanFn.backward
 * (ops.py:157-163) and ExactCorrectionFn.backward (ops.py:188-195, the reference's shifted rule),
 * as cdssm_fused_scan_bwd does for the readout form.  Inputs: the forward's inputs, dY
 * (B,L,H,N,D) of `dtype` and fwd_workspace as filled by cdssm_ssd_scan_fwd with train != 0.
 * Outputs of `dtype`: dA (B,L,H,N), dK (B,L,H,D), dV (B,L,H,N), dbeta (B,L,H); for N > 2, dK
 * and dbeta sum the state rows' fp32 contributions in a fixed order.  k, dY and dK 16-byte
 * aligned.  workspace: cdssm_ssd_scan_bwd_workspace_bytes() bytes.
 */
int64_t cdssm_ssd_scan_bwd_workspace_bytes(int64_t B, int64_t L, int64_t H, int64_t D, int64_t N,
                                           int64_t chunk);
int cdssm_ssd_scan_bwd(int dtype, const void* a_bar, const void* k, const void* v, const void* beta,
                       const void* dY, const float* fwd_workspace, void* dA, void* dK, void* dV, void* dbeta,
                       float* workspace, int64_t B, int64_t L, int64_t H, int64_t D, int64_t N, int64_t chunk,
                       hipStream_t stream);

/*
 * Instrumentation (no counterpart in the reference; for benchmarks and
 * profilers): run the fused forward / backward `iters` times on `stream` with
 * HIP events recorded between its kernel launches, synchronise, and return in
 * phase_ms the average milliseconds of each launch:
 *   forward  phase_ms[4]: chunk summaries, carry fold, carry replay, main pass;
 *   backward phase_ms[5]: correction adjoint, reverse-carry fold, reverse-carry
 *            replay, main pass, per-head reduction.
 * `train` != 0 profiles cdssm_fused_scan_fwd_train.  Arguments otherwise as
 * cdssm_fused_scan_fwd / cdssm_fused_scan_bwd.
 */
int cdssm_fused_scan_fwd_profile(int dtype, const void* q, const void* k, const void* v, const void* beta,
                                 const void* sel_c, const void* dt, const void* r, const float* alpha,
                                 const float* omega, float c, const float* h0, void* y, float* h_final,
                                 float* workspace, int64_t B, int64_t L, int64_t H, int64_t D, int64_t N,
                                 int64_t chunk, hipStream_t stream, int train, int iters, float* phase_ms);
int cdssm_fused_scan_bwd_profile(int dtype, const void* q, const void* k, const void* v, const void* beta,
                                 const void* sel_c, const void* dt, const void* r, const float* alpha,
                                 const float* omega, float c, const void* dy, const float* dh_final,
                                 const float* fwd_workspace, void* dq, void* dk, void* dv, void* dbeta,
                                 void* dsel_c, void* ddt, void* dr, float* dalpha, float* domega,
                                 float* dh0, float* workspace, int64_t B, int64_t L, int64_t H, int64_t D,
                                 int64_t N, int64_t chunk, hipStream_t stream, int iters, float* phase_ms);

/*
 * Instrumentation (no counterpart in the reference): cdssm_fused_scan_fwd
 * (with its epoch kernel), recording for every wave of the one-pass kernel the
 * 100 MHz real-time counter (s_memrealtime) at 8 points of its segment: entry,
 * staging done, local pass done, segment map published, look-back wait done,
 * carry folded, correction pass done, segment end.  stamps: device memory of
 * stamps_len 8-byte words; word ((item * 4 + wave) * 8 + point) for wave
 * 0..3 of the workgroup of item = segment * B * n_hg + b * n_hg + head group
 * (n_hg = ceil(H / 8) head groups for bf16 D = 64, the same layout for the
 * other instances with their heads per wave); the caller clears the buffer to
 * tell unwritten records.
 * Returns -1 (nothing launched) if the buffer holds fewer than
 * items * 32 words or the shape takes the four-launch forward.  Results are
 * bit-identical to cdssm_fused_scan_fwd.
 */
int cdssm_fused_scan_fwd_stamped(int dtype, const void* q, const void* k, const void* v, const void* beta,
                                 const void* sel_c, const void* dt, const void* r, const float* alpha,
                                 const float* omega, float c, const float* h0, void* y, float* h_final,
                                 float* workspace, int64_t B, int64_t L, int64_t H, int64_t D, int64_t N,
                                 int64_t chunk, unsigned long long* stamps, int64_t stamps_len,
                                 hipStream_t stream);

/*
 * Launch-path selection (no counterpart in the reference; for tests and
 * benchmarks): 0 = automatic (default), 1 = always the multi-launch passes,
 * 2 = one launch required (calls it cannot serve return -1), 3 = the
 * multi-launch forward with the correction as the chunked MFMA pass (Gram
 * tiles K K^T, Q K^T and the projections K s, Q s on v_mfma_f32_16x16x32_bf16,
 * then a per-token triangular solve; bf16 inference forward with a workspace,
 * chunk a multiple of 16 up to 128; other calls return -1).  Applies to the
 * forward (one-pass scan vs four launches) and to the backward's correction
 * adjoint + reverse carry (one launch vs three).  Process-wide; returns the
 * previous mode, or -1 for an invalid mode.  A one-launch forward is reported
 * as the main pass in cdssm_fused_scan_fwd_profile, a one-launch correction
 * adjoint + carry as its first phase (0 for the fold and replay phases) in
 * cdssm_fused_scan_bwd_profile.
 */
int cdssm_fused_scan_fwd_set_path(int mode);

/*
 * Look-back health (no counterpart in the reference, whose inter-chunk pass is
 * a separate serial launch, inter_chunk_scan.cu:201-234).  The one-launch
 * forward and the backward's one-launch correction adjoint + carry pass chunk
 * summaries between workgroups through flags; a wait for a flag is bounded
 * (50 ms) and, if it gives up, the affected states are written as NaN and a
 * sticky bit is set on the device: bit 0 (1) for the forward, bit 1 (2) for
 * the backward.  This call stores the bits of the current device in *status
 * (0: no wait has timed out) and, if clear != 0, resets them.  It synchronises
 * with the device (device-to-host copies), so it must not be called while the
 * stream is being captured into a graph.
 *
 * The one-launch passes draw their flag epoch on the device: a one-thread
 * kernel launched on the same stream just before the pass writes a fresh
 * epoch from a per-device counter into the workspace, so the workspace needs
 * no clearing between calls and a captured graph stays correct on every replay.
 */
int cdssm_lookback_status(int clear, int* status);

/*
 * Recurrent decode: one new token per (b, h) with the R-mode state carried
 * between calls.  No reference counterpart: the reference generates by
 * re-running the whole forward for every new token (predict.py:53-67, through
 * SSDChunkwiseScan.forward, ssd.py:39-111); the step gives the same outputs as
 * that chunked scan over the longer sequence (same chunk boundaries).
 * State (fp32, caller-owned, contiguous): state (B,H,3,N,D) = local state z,
 * decay-free correction c^ and the carry s entering the current chunk;
 * gam (B,H,N) = rotation product of the chunk so far; pos (B,H) int32 =
 * position in the chunk.
 * cdssm_decode_init: the state at a chunk boundary with carry h (B,H,N,D) fp32
 * (the fused forward's h_final after a multiple of `chunk` tokens), or the
 * zero state for h = NULL.
 * cdssm_decode_step: token tensors q, k (B,H,D), v (B,H,N), beta, sel_c, dt,
 * r (B,H) of `dtype` (a (B,1,H,.) slice of the scan inputs), alpha, omega (H,)
 * fp32; writes y (B,H,N) of `dtype`, advances the state, and, if h_out is not
 * NULL, writes the R-mode carry after the token to h_out (B,H,N,D) fp32 (what
 * the fused forward returns as h_final for a sequence ending there).
 * Supported: N = 2, D in {64, 128}, 1 <= chunk <= 128.
 */
int cdssm_decode_init(const float* h, float* state, float* gam, int* pos, int64_t B, int64_t H, int64_t D,
                      int64_t N, hipStream_t stream);
int cdssm_decode_step(int dtype, const void* q, const void* k, const void* v, const void* beta, const void* sel_c,
                      const void* dt, const void* r, const float* alpha, const float* omega, float c,
                      float* state, float* gam, int* pos, void* y, float* h_out, int64_t B, int64_t H, int64_t D,
                      int64_t N, int64_t chunk, hipStream_t stream);

/*
 * The reference's three scan passes as separate ops, same tensor contracts
 * (all tensors `dtype`, contiguous; N even, N <= 32; D <= 128).
 *
 * Replaces intra_chunk_scan_fwd_cuda (intra_chunk_scan.cu:560-609; bound at
 * binding.cpp:143, called by IntraChunkScanFn.forward, ops.py:107-121):
 *   A (BNC,C,H,N), K (BNC,C,H,D), V (BNC,C,H,N), beta (BNC,C,H)
 *   -> local_h (BNC,C,H,N,D) (state after each step), cum_A (BNC,C,H,N).
 */
int cdssm_intra_chunk_scan_fwd(int dtype, const void* A, const void* K, const void* V, const void* beta,
                               void* local_h, void* cum_A, int64_t BNC, int64_t C, int64_t H, int64_t D,
                               int64_t N, hipStream_t stream);
/* Replaces intra_chunk_scan_bwd_cuda (intra_chunk_scan.cu:611-674; IntraChunkScanFn.backward,
 * ops.py:123-135).  grad_beta is written in `dtype` (ops.py:134 casts it). */
int cdssm_intra_chunk_scan_bwd(int dtype, const void* grad_local_h, const void* grad_cum_A, const void* A,
                               const void* K, const void* V, const void* beta, const void* local_h,
                               const void* cum_A, void* grad_A, void* grad_K, void* grad_V, void* grad_beta,
                               int64_t BNC, int64_t C, int64_t H, int64_t D, int64_t N, hipStream_t stream);
/* Replaces inter_chunk_scan_fwd_cuda (inter_chunk_scan.cu:201-234; InterChunkScanFn.forward,
 * ops.py:146-155): total_A (B,NC,H,N), final_local_h (B,NC,H,N,D) -> chunk_states (B,NC,H,N,D). */
int cdssm_inter_chunk_scan_fwd(int dtype, const void* total_A, const void* final_local_h,
                               void* chunk_states, int64_t B, int64_t NC, int64_t H, int64_t D, int64_t N,
                               hipStream_t stream);
/* Replaces inter_chunk_scan_bwd_cuda (inter_chunk_scan.cu:236-275; InterChunkScanFn.backward,
 * ops.py:158-163). */
int cdssm_inter_chunk_scan_bwd(int dtype, const void* grad_chunk_states, const void* total_A,
                               const void* chunk_states, void* grad_total_A, void* grad_final_local_h,
                               int64_t B, int64_t NC, int64_t H, int64_t D, int64_t N, hipStream_t stream);
/* Replaces exact_correction_fwd_cuda (exact_correction.cu:390-438; ExactCorrectionFn.forward,
 * ops.py:173-186): A (B,NC,C,H,N), K (B,NC,C,H,D), beta (B,NC,C,H), chunk_states (B,NC,H,N,D)
 * -> corrections (B,NC,C,H,N,D) (state before each step). */
int cdssm_exact_correction_fwd(int dtype, const void* A_chunk, const void* K_chunk, const void* beta_chunk,
                               const void* chunk_states, void* corrections, int64_t B, int64_t NC,
                               int64_t C, int64_t H, int64_t D, int64_t N, hipStream_t stream);
/* Replaces exact_correction_bwd_cuda (exact_correction.cu:440-498; ExactCorrectionFn.backward,
 * ops.py:189-195), with the reference's rule (grad_corrections[t] applied to the state after
 * step t).  chunk_states is accepted for signature parity; corrections holds every pre-step state. */
int cdssm_exact_correction_bwd(int dtype, const void* grad_corrections, const void* A_chunk,
                               const void* K_chunk, const void* beta_chunk, const void* chunk_states,
                               const void* corrections, void* grad_A, void* grad_K, void* grad_beta,
                               void* grad_states, int64_t B, int64_t NC, int64_t C, int64_t H, int64_t D,
                               int64_t N, hipStream_t stream);

/*
 * Replaces dynamics_fused_fwd_cuda (dynamics_fused.cu:392-440; DynamicsFusedFn.forward,
 * ops.py:39-66): gate_raw (B,L,(N+5)H) `dtype`; log_dt_scale, rope_freqs (H,) fp32
 * -> A_bar (B,L,H,N), vp_scale (B,L,H,N/2), beta (B,L,H), sel_c (B,L,H), all `dtype`.
 */
int cdssm_dynamics_fused_fwd(int dtype, const void* gate_raw, const float* log_dt_scale,
                             const float* rope_freqs, float gating_c, float omega_thresh, float adt_delta,
                             float adt_smoothness, float adt_eps, void* A_bar, void* vp_scale, void* beta,
                             void* sel_c, int64_t B, int64_t L, int64_t H, int64_t N, hipStream_t stream);
/* Replaces dynamics_fused_bwd_cuda (dynamics_fused.cu:442-499; DynamicsFusedFn.backward,
 * ops.py:68-81) with the reference's analytic rule; grad_log_dt_scale (H,) fp32 is a
 * deterministic per-head sum.  workspace: cdssm_dynamics_fused_bwd_workspace_bytes() bytes. */
int64_t cdssm_dynamics_fused_bwd_workspace_bytes(int64_t B, int64_t L, int64_t H);
int cdssm_dynamics_fused_bwd(int dtype, const void* grad_A_bar, const void* grad_vp_scale,
                             const void* grad_beta, const void* grad_sel_c, const void* gate_raw,
                             const float* log_dt_scale, const float* rope_freqs, float gating_c,
                             float omega_thresh, float adt_delta, float adt_smoothness, float adt_eps,
                             void* grad_gate_raw, float* grad_log_dt_scale, float* workspace, int64_t B,
                             int64_t L, int64_t H, int64_t N, hipStream_t stream);

/*
 * Replaces conv1d_silu_fwd_cuda (conv1d_silu.cu:25-90 and its launcher :223-274;
 * bound at binding.cpp:134, called by CUDAConv1dSiLUOp.forward, ops.py:13-21, for
 * Conv1dSiLU, modules.py:14-35): causal depthwise conv + SiLU,
 *   y[b,t,c] = silu(bias[c] + sum_{j<K} w[c,j] x[b, t-(K-1)+j, c]), x = 0 before t = 0.
 * x, y (B,L,C); weight (C,1,K); bias (C); all `dtype` (the reference: bf16,
 * K = 4 only).  Supported: 1 <= K <= 8, B * ceil(L/8) * C < 2^31.  Backward:
 * cdssm_conv1d_silu_bwd.
 */
int cdssm_conv1d_silu_fwd(int dtype, const void* x, const void* weight, const void* bias, void* y, int64_t B,
                          int64_t L, int64_t C, int64_t K, hipStream_t stream);

/* Bytes of the fp32 workspace cdssm_conv1d_silu_bwd needs (-1 if invalid).  No reference counterpart: the
 * reference's launcher allocates its gradient buffers itself (conv1d_silu.cu:301-312); this library never
 * allocates. */
int64_t cdssm_conv1d_silu_bwd_workspace_bytes(int64_t B, int64_t L, int64_t C, int64_t K);

/*
 * Replaces conv1d_silu_bwd_cuda (conv1d_silu.cu:95-276, bound at
 * binding.cpp, called by CUDAConv1dSiLUOp.backward, ops.py:22-28):
 *   gu = grad_out * silu'(u) with u the recomputed conv output,
 *   grad_x[t] = sum_j w[c,j] gu[t+(K-1)-j]        (`dtype`, (B,L,C) dense),
 *   grad_weight[c,j] = sum_{b,t} gu x[t-(K-1)+j]   (fp32 (C,K)),
 *   grad_bias[c] = sum_{b,t} gu                   (fp32 (C)),
 * as the reference (which returns the fp32 sums cast to the parameters'
 * dtype).  x read through a token stride (elements); grad_out (B,L,C) dense.
 * The weight and bias sums are formed from per-(b, 16-token block) partials
 * added in a fixed order (the reference uses float atomics): deterministic.
 * workspace: cdssm_conv1d_silu_bwd_workspace_bytes.  1 <= K <= 8.
 */
int cdssm_conv1d_silu_bwd(int dtype, const void* x, int64_t x_token_stride, const void* weight, const void* bias,
                          const void* grad_out, void* grad_x, float* grad_weight, float* grad_bias, float* workspace,
                          int64_t B, int64_t L, int64_t C, int64_t K, hipStream_t stream);

/*
 * cdssm_conv1d_silu_fwd with x read through a token stride (elements between
 * consecutive tokens, >= C): the block's conv input x_gate is a column slice
 * of the in_proj output (block.py:162-166, 177), which this reads in place
 * instead of copying it.  The reference's launcher calls .contiguous() on
 * the slice (conv1d_silu.cu:223-274).
 */
int cdssm_conv1d_silu_fwd_strided(int dtype, const void* x, int64_t x_token_stride, const void* weight,
                                  const void* bias, void* y, int64_t B, int64_t L, int64_t C, int64_t K,
                                  hipStream_t stream);

/*
 * Replaces RMSNorm.forward (modules.py:49-53):
 *   y = (x * rsqrt(mean(x^2) + eps)).to(dtype) * weight,
 * statistics in fp32; x, y (rows, C) dense, weight (C), all `dtype`.
 */
int cdssm_rms_norm_fwd(int dtype, const void* x, const void* weight, void* y, int64_t rows, int64_t C, float eps,
                       hipStream_t stream);

/*
 * Backward of cdssm_rms_norm_fwd, for training (modules.py:49-53 under
 * autograd): given dout (rows, C) and the forward's x and weight (`dtype`),
 * writes dx (rows, C) and dw (C), with the reference expression's rounding
 * points (xn = (x r).to(dtype), out = xn w): dxn = dout w, dw = sum over rows
 * of dout xn (fixed order), dx = dxn r - x r^3 (sum dxn x) / C in fp32,
 * r = rsqrt(mean(x^2) + eps).  C a multiple of 64 16-byte vectors, at most 4
 * per lane (bf16: 512 .. 2048; fp32: 256 .. 1024); 16-byte aligned.
 * Workspace: cdssm_rms_norm_bwd_workspace_bytes (the per-block partial rows
 * of dw).  Replaces the backward of torch's expression.
 */
int64_t cdssm_rms_norm_bwd_workspace_bytes(int64_t rows, int64_t C);
int cdssm_rms_norm_bwd(int dtype, const void* x, const void* w, const void* dout, void* dx, void* dw, float* workspace,
                       int64_t rows, int64_t C, float eps, hipStream_t stream);

/*
 * Replaces the block's two NormalizeKQFn.forward calls (block.py:191-192 ->
 * normalize_kq.cu:75-79, x * rsqrt(sum x^2 + 1e-6) per (token, head)) and the
 * shortcut's q.k (block.py:202, einsum 'blhd,blhd->blh') in one pass.  K and Q
 * rows (H*D elements per token) are read through token strides (elements;
 * K may be the in_proj output's column slice); K_out, Q_out (B*L, H, D) dense
 * in `dtype`; qk (B*L, H) fp32 from the rounded K_out, Q_out.  D = 32, 64,
 * 128 or 256 (bf16) / 16, 32, 64 or 128 (fp32).
 */
int cdssm_normalize_kq_qk_fwd(int dtype, const void* K, int64_t k_token_stride, const void* Q,
                              int64_t q_token_stride, void* K_out, void* Q_out, float* qk, int64_t BL, int64_t H,
                              int64_t D, hipStream_t stream);

/*
 * Backward of cdssm_normalize_kq_qk_fwd, for training through the block: given
 * the gradients dK_out, dQ_out (B*L, H, D) dense of `dtype` and dqk (B*L, H)
 * fp32 of its outputs, and its inputs K, Q (token strides as in the forward),
 * writes dK, dQ (B*L, H, D) dense: per row g = dK_out + dqk Q^ (Q^ rounded as
 * the forward rounds it), dK = (g - K^ <g, K^>) rsqrt(sum k^2 + 1e-6), the
 * normalisation's rule of normalize_kq.cu (NormalizeKQFn, ops.py:84-97); dQ
 * likewise.  Replaces NormalizeKQFn's backward together with the backward of
 * torch's q.k product and sum (block.py:202).  Limits as the forward.
 */
int cdssm_normalize_kq_qk_bwd(int dtype, const void* K, int64_t k_token_stride, const void* Q, int64_t q_token_stride,
                              const void* dK_out, const void* dQ_out, const float* dqk, void* dK, void* dQ, int64_t BL,
                              int64_t H, int64_t D, hipStream_t stream);

/*
 * The block's readout of per-token states for state_dim N > 2, where
 * SSDChunkwiseScan returns Y (block.py:208: einsum('blhsd,blhd->blhs', Y, Q)):
 * cdssm_state_readout_fwd writes r (n, N) = Y (n, N, D) . q (n, D) with fp32
 * accumulation; cdssm_state_readout_bwd, given dr (n, N), writes dY = dr q
 * (n, N, D) and dq = sum over N of dr Y (n, D).  All of `dtype`; n = B*L*H; D a
 * multiple of 8 (bf16) or 4 (fp32); Y, q, dY, dq 16-byte aligned.
 */
int cdssm_state_readout_fwd(int dtype, const void* Y, const void* q, void* r, int64_t n, int64_t N, int64_t D,
                            hipStream_t stream);
int cdssm_state_readout_bwd(int dtype, const void* Y, const void* q, const void* dr, void* dY, void* dq, int64_t n,
                            int64_t N, int64_t D, hipStream_t stream);

/*
 * The current-token shortcut (block.py:202-205) carried through the readout
 * (block.py:208-211): shortcut_scale (q.k) V_gated k^T read by q and gated
 * by sel_C adds sel_C * scale * (q.k)^2 * vp * V to the retrieved pair, in
 * place:  retrieved (n, 2), V (n, 2), vp, sel_c (n) in `dtype`; qk (n) fp32;
 * scale: one fp32 on the device.  n = B*L*H.
 */
int cdssm_shortcut_readout_fwd(int dtype, void* retrieved, const float* qk, const void* V, const void* vp,
                               const void* sel_c, const float* scale, int64_t n, hipStream_t stream);

/*
 * The same shortcut with N/2 complex state rows per (token, head) (block.py:194-211 at any even
 * state_dim N <= 64, the rows sharing q.k and sel_C), forward and backward, for the training step:
 *   forward, in place:  y[i, j] += scale (q.k)_i^2 sel_C[i] vp[i, j/2] V[i, j],  one rounding;
 *   backward (dy = dL/dy): adds the shortcut's gradients to the scan's, in place, in fp32 with one
 *   rounding each -- dV[i, j] += c_i vp[i, j/2] dy[i, j], dvp[i, p] += c_i (dy V)[i, 2p] + c_i (dy V)[i, 2p+1],
 *   dsel_c[i] += scale (q.k)_i^2 u_i with c_i = scale (q.k)_i^2 sel_C[i] and u_i = sum_j dy vp V;
 *   writes dqk[i] = 2 scale (q.k)_i sel_C[i] u_i (fp32) and, per workgroup, the partial sum of
 *   (q.k)^2 sel_C u over its rows to dscale_partials (cdssm_shortcut_readout_rows_partials(n, N) floats;
 *   their sum, in any fixed order, is dL/dscale).
 * y, dy, V, dV (n, N); vp, dvp (n, N/2); sel_c, dsel_c (n) in `dtype`, dense, y and dV aligned to a
 * (re, im) pair; qk, dqk (n) fp32; scale one fp32 on the device.  n = B*L*H.  The reference forms V_gated = V vp, scale (q.k)^2 V_gated and
 * (Y.q + shortcut) sel_C with torch ops (block.py:194-211) and autograd's rules for them; no launcher.
 */
int64_t cdssm_shortcut_readout_rows_partials(int64_t n, int64_t N);

/*
 * Column sums out[c] = sum_r x[r, c] of a (rows, C) matrix read through a row stride ld (elements), fp32
 * accumulation in a fixed order (slabs of 64 rows, then the slabs in order), rounded once to `dtype`:
 * the bias gradient of a linear layer (the sum of dL/dy over tokens), which autograd forms for the
 * reference's nn.Linear projections (block.py:65-81; no launcher).  C and ld multiples of the 16-byte
 * vector (8 bf16, 4 fp32), x 16-byte aligned; workspace of cdssm_col_sum_workspace_bytes(rows, C).
 */
int64_t cdssm_col_sum_workspace_bytes(int64_t rows, int64_t C);

/*
 * out[i] = sum_s part[s n + i] over S fp32 slabs of n elements, in slab order, rounded once to `dtype`:
 * the token-slab partials of a weight gradient dW = dY^T X (autograd's rule for the reference's
 * nn.Linear projections, block.py:65-81; no launcher) joined into the weight's dtype.
 */
int cdssm_slab_sum(int dtype, const float* part, int64_t S, int64_t n, void* out, hipStream_t stream);
int cdssm_col_sum(int dtype, const void* x, int64_t ld, int64_t rows, int64_t C, void* out, float* workspace,
                  hipStream_t stream);
int cdssm_shortcut_readout_rows_fwd(int dtype, void* y, const float* qk, const void* V, const void* vp,
                                    const void* sel_c, const float* scale, int64_t n, int64_t N, hipStream_t stream);
int cdssm_shortcut_readout_rows_bwd(int dtype, const void* dy, const float* qk, const void* V, const void* vp,
                                    const void* sel_c, const float* scale, void* dV, void* dvp, void* dsel_c,
                                    float* dqk, float* dscale_partials, int64_t n, int64_t N, hipStream_t stream);

/* Bytes of the fp32 workspace cdssm_group_norm_gate_fwd needs (-1 if invalid).  No reference counterpart:
 * torch's group_norm allocates its statistics (block.py:216-223); this library never allocates. */
int64_t cdssm_group_norm_workspace_bytes(int64_t B, int64_t G, int64_t L);

/*
 * Replaces the block's epilogue after readout_proj (block.py:215-225):
 *   a = GroupNorm_G(y)  (statistics per (b, group) over the group's C/G
 *       channels and all L positions, fp32, biased variance, eps; affine
 *       gamma, beta in fp32), rounded to `dtype`;
 *   out = a * silu(z) + D * x_conv, each product and the sum rounded to `dtype`
 * as the reference's torch ops round them.  y, x_conv, out (B, L, C) dense;
 * z read through a token stride (the in_proj output's column slice);
 * gamma, beta (C) of `param_dtype` (0 fp32, 1 bf16; read exactly, as the
 * reference's .float()); D (C) `dtype`; C divisible by G.  Three launches
 * (partial sums, per-group statistics, apply); workspace of
 * cdssm_group_norm_workspace_bytes.
 */
int cdssm_group_norm_gate_fwd(int dtype, int param_dtype, const void* y, const void* gamma, const void* beta,
                              const void* z, int64_t z_token_stride, const void* x_conv, const void* D, void* out,
                              float* workspace, int64_t B, int64_t L, int64_t C, int64_t G, float eps,
                              hipStream_t stream);

/*
 * Backward of cdssm_group_norm_gate_fwd, for training through the block
 * (block.py:215-225 under autograd; replaces the backward of torch's
 * group_norm, silu, the products and the sum): given dout (B, L, C) and the
 * forward's workspace (its per-group statistics), writes dy, dz, dx_conv
 * (B, L, C) dense of `dtype` (dx_conv: the D x_conv term's part only),
 * dgamma, dbeta (C) of `param_dtype` and dD (C) of `dtype`, with the rounding
 * points of the reference's ops (each torch op's bf16 output) and the
 * GroupNorm backward in fp32; every sum in a fixed order (bit-reproducible).
 * The group width C / G must be a multiple of 16 / element bytes dividing
 * 64 times that; every tensor 16-byte aligned.  Three launches (partial sums
 * per batch row and token slice, totals, elementwise); workspace of
 * cdssm_group_norm_gate_bwd_workspace_bytes.  No reference counterpart beyond
 * the torch ops it replaces.
 */
int64_t cdssm_group_norm_gate_bwd_workspace_bytes(int64_t B, int64_t G, int64_t L, int64_t C);
int cdssm_group_norm_gate_bwd(int dtype, int param_dtype, const void* y, const void* gamma, const void* beta,
                              const void* z, int64_t z_token_stride, const void* x_conv, const void* D,
                              const float* fwd_workspace, const void* dout, void* dy, void* dz, void* dx_conv,
                              void* dgamma, void* dbeta, void* dD, float* workspace, int64_t B, int64_t L, int64_t C,
                              int64_t G, hipStream_t stream);

/*
 * Replaces normalize_kq_fwd_cuda / normalize_kq_bwd_cuda (normalize_kq.cu:168-244;
 * NormalizeKQFn, ops.py:84-97): rows of length D (any D <= 256; the reference kernel is
 * correct only for D = 64), x_hat = x rsqrt(sum x^2 + 1e-6).
 */
int cdssm_normalize_kq_fwd(int dtype, const void* K, const void* Q, void* K_out, void* Q_out, int64_t rows,
                           int64_t D, hipStream_t stream);
int cdssm_normalize_kq_bwd(int dtype, const void* grad_K_out, const void* grad_Q_out, const void* K,
                           const void* Q, void* grad_K, void* grad_Q, int64_t rows, int64_t D,
                           hipStream_t stream);

/*
 * cdssm_decode_step on the gate-level inputs (the model's DynamicsFusedFn
 * outputs, block.py:184-198): a_bar (B, H, 2) = A_bar and vp (B, H) = vp_scale
 * of the token in place of (dt, r, alpha, omega, c); otherwise as
 * cdssm_decode_step.  No reference counterpart (predict.py:53-67 re-forwards);
 * the scan it continues is cdssm_fused_scan_fwd_abar's.
 */
int cdssm_decode_step_abar(int dtype, const void* q, const void* k, const void* v, const void* beta,
                           const void* sel_c, const void* a_bar, const void* vp, float* state, float* gam, int* pos,
                           void* y, float* h_out, int64_t B, int64_t H, int64_t D, int64_t N, int64_t chunk,
                           hipStream_t stream);

/*
 * cdssm_dynamics_fused_fwd for gate rows at sequence positions l0 .. l0+L-1
 * (the RoPE term omega + l * rope_freqs[h] of block.py:59-62, 184-188, uses
 * the absolute position): one decode token is L = 1 at l0 = its position.
 * The offset is l0 plus, when l0_dev is non-null, the int64 it points to on
 * the device (read by the kernel: a decode step captured in a HIP graph keeps
 * its position there).
 */
int cdssm_dynamics_fused_fwd_at(int dtype, const void* gate_raw, const float* log_dt_scale, const float* rope_freqs,
                                float gating_c, float omega_thresh, float adt_delta, float adt_smoothness,
                                float adt_eps, void* A_bar, void* vp_scale, void* beta, void* sel_c, int64_t B,
                                int64_t L, int64_t H, int64_t N, int64_t l0, const int64_t* l0_dev,
                                hipStream_t stream);

/*
 * One decode token of the conv1d+SiLU (conv1d_silu.cu:25-90 at the newest
 * position): x (B, C) with a row stride (elements), window (B, K-1, C) the
 * last K-1 inputs of each row, oldest first (zeros before the sequence
 * start), updated in place; y (B, C).  Equals the full convolution's output at
 * that position.  No reference counterpart (the reference re-forwards).
 */
int cdssm_conv1d_silu_step(int dtype, const void* x, int64_t x_batch_stride, void* window, const void* weight,
                           const void* bias, void* y, int64_t B, int64_t C, int64_t K, hipStream_t stream);

/*
 * One decode token of the block's GroupNorm epilogue (block.py:215-225) with
 * running statistics: gsum (B, G, 4) fp32 = (shift, sum (x - shift),
 * sum (x - shift)^2, count) over every position so far, updated in place with
 * the token's y (B, C); then out = rnd(rnd(GN(y)) * rnd(silu(z))) + rnd(D x_conv)
 * as cdssm_group_norm_gate_fwd.  For the token this equals the GroupNorm of a
 * forward over the prefix plus the token (the reference's statistics span all
 * positions).  z with a row stride.  position (nullable): an int64 on the
 * device incremented once by the call (the layer's decode position, read by
 * the step's earlier kernels).  No reference counterpart.
 */
int cdssm_group_norm_gate_step(int dtype, int param_dtype, const void* y, float* gsum, const void* gamma,
                               const void* beta, const void* z, int64_t z_batch_stride, const void* x_conv,
                               const void* D, void* out, int64_t B, int64_t C, int64_t G, float eps,
                               int64_t* position, hipStream_t stream);

/*
 * cdssm_group_norm_gate_step with the block's readout projection
 * (block.py:213, readout_proj: nn.Linear(H N, C, bias=False)) folded in: y of
 * each row is computed in the kernel as rnd(retrieved (B, K) . W (C, K)^T),
 * rounded to the dtype as the projection's output is, and never written.
 * retrieved and readout_weight dense, in the activation dtype; K <= 4096,
 * C + 2 G + K <= 16384.  No reference counterpart (one decode launch fewer).
 */
int cdssm_readout_group_norm_gate_step(int dtype, int param_dtype, const void* retrieved, const void* readout_weight,
                                       int64_t K, float* gsum, const void* gamma, const void* beta, const void* z,
                                       int64_t z_batch_stride, const void* x_conv, const void* Dp, void* out,
                                       int64_t B, int64_t C, int64_t G, float eps, int64_t* position,
                                       hipStream_t stream);

/*
 * Decode-size linear layer: Y (M x N, row stride ldy) = X (M x K, row stride
 * ldx) W^T (W: N x K, row stride ldw) + bias (N, or NULL) + R (M x N, row
 * stride ldr, or NULL).  With wnorm (K, or NULL) the rows of X are
 * RMS-normalised first as the model's RMSNorm does (modules.py:49-53; eps):
 * X * wnorm enters the product rounded to bf16 and the row scale
 * rsqrt(mean(X^2) + eps) is applied to the fp32 result.  bf16 only (dtype 1),
 * M in 1..64, K a multiple of 128, X / W / wnorm rows 16-byte aligned.
 * Replaces, in the decode step, torch's GEMMs behind nn.Linear for in_proj
 * (with the block's RMSNorm; block.py:155-156), the stacked gate/Q projection
 * (gate_proj, Q_proj) and out_proj (with the residual).  No reference
 * counterpart as a function: the reference decodes by re-forwarding
 * (predict.py:53-67).
 */
int cdssm_skinny_gemm(int dtype, const void* X, int64_t ldx, const void* W, int64_t ldw, const void* bias,
                      const void* R, int64_t ldr, const void* wnorm, float eps, void* Y, int64_t ldy, int64_t M,
                      int64_t N, int64_t K, hipStream_t stream);

/*
 * One decode token of the model block's scan path in one launch, per (b, h):
 * the gate-level dynamics at the device-held position (as
 * cdssm_dynamics_fused_fwd_at), K/Q normalisation and q.k (as
 * cdssm_normalize_kq_qk_fwd), the value residual V = lerp(v_first, V, vgate)
 * (block.py:169-174; v_first null for layer 0), the gate-level scan decode
 * step (as cdssm_decode_step_abar) and the current-token shortcut (as
 * cdssm_shortcut_readout_fwd), each intermediate rounded where those kernels
 * store it.  gq (B, 7H + H*D) rows: [gate row | Q] (the stacked gate_proj /
 * Q_proj GEMM output), row stride gq_stride; proj (B, P) the in_proj output
 * with K at column k_off and V at v_off, row stride proj_stride; Q and K rows
 * 16-byte aligned.  vgate (H) = sigmoid(v_residual_gate) in `dtype`;
 * log_dt_scale, rope_freqs (H) fp32; position: int64 on the device;
 * shortcut_scale: one fp32 on the device.  Outputs retrieved (B, H, 2) and
 * v_out (B, H, 2) (the V used; layer 0's is v_first of the later layers).
 * N = 2, D in {64, 128}.  No reference counterpart (the reference re-forwards).
 */
int cdssm_decode_block_token(int dtype, const void* gq, int64_t gq_stride, const void* proj, int64_t proj_stride,
                             int64_t k_off, int64_t v_off, const void* v_first, const void* vgate,
                             const float* log_dt_scale, const float* rope_freqs, float gating_c, float omega_thresh,
                             float adt_delta, float adt_smoothness, float adt_eps, const int64_t* position,
                             const float* shortcut_scale, float* state, float* gam, int* pos, void* retrieved,
                             void* v_out, int64_t B, int64_t H, int64_t D, int64_t N, int64_t chunk,
                             hipStream_t stream);

/*
 * cdssm_decode_block_token and the readout + GroupNorm + gate step after it
 * (cdssm_readout_group_norm_gate_step) in one launch, for the model's decode
 * step (block.py:169-225 between the gate / Q projection and out_proj): one
 * workgroup per batch row whose waves run the token step of its heads into
 * LDS, then the row's readout projection (readout_weight (C, 2 H)) and
 * GroupNorm step with running sums gsum (B, G, 4), writing out (B, C).  The
 * outputs equal the two separate calls'.  position points at two int64s: the
 * layer's decode position and an arrival count, zero on entry (and left zero):
 * every workgroup arrives after reading the position and the last advances it,
 * as cdssm_readout_group_norm_gate_step does.  Arguments, shapes and limits as
 * the two calls (v_out as cdssm_decode_block_token's); at most 16 head groups
 * (H <= 128 in bf16 at D = 64), 2 H + 2 G + C <= 16384.  No reference
 * counterpart: the reference re-forwards the sequence per token.
 */
int cdssm_decode_block_tail(int dtype, int param_dtype, const void* gq, int64_t gq_stride, const void* proj,
                            int64_t proj_stride, int64_t k_off, int64_t v_off, const void* v_first, const void* vgate,
                            const float* log_dt_scale, const float* rope_freqs, float gating_c, float omega_thresh,
                            float adt_delta, float adt_smoothness, float adt_eps, int64_t* position,
                            const float* shortcut_scale, float* state, float* gam, int* pos, void* v_out,
                            const void* readout_weight, float* gsum, const void* gamma, const void* beta,
                            const void* z, int64_t z_batch_stride, const void* x_conv, const void* D_skip, void* out,
                            int64_t B, int64_t H, int64_t D, int64_t N, int64_t chunk, int64_t C, int64_t G,
                            float eps, hipStream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* CDSSM_HIP_H */
