// Fused forward of the CD-SSM chunkwise delta-rule scan, R-mode semantics.
//
// What is computed (per batch b, head h; complex notation, N = 2 so each
// head's state is one complex D-vector; reference algorithm: ssd.py:39-111 with
// intra_chunk_scan.cu:86-195, inter_chunk_scan.cu:49-84,
// exact_correction.cu:83-150, block.py:194-211):
//   per token:  a_t, vp_t from (dt_t, r_t, alpha_h, omega_h, c)   [Cayley + gating]
//               w_t = beta_t * vp_t * v_t                          [VP-scaled value]
//   chunk k, local index t, zero-initialised local state z:
//               z_t = a_t * (z_{t-1} - beta_t (z_{t-1}.k_t) k_t) + w_t k_t
//   carry:      s_0 = h0 (0 if absent), s_{k+1} = G_k * s_k + z_{Q-1},
//               G_k = prod_t a_t   (rotation-only carry, inter_chunk_scan.cu:73-83)
//   correction: c_0 = s_k, c_{t+1} = a_t * (c_t - beta_t (c_t.k_t) k_t),
//               read BEFORE step t (exact_correction.cu:89-94)
//   output:     y_t = sel_C_t * ((z_t + c_t) . q_t)
//   final:      s_NC (the R-mode carry after the last real token).
//
// The correction is carried in a decay-free frame: c_t = g_{t-1} * c^_t with
// g_{t-1} = prod_{u<t} a_u and c^_{t+1} = c^_t - beta_t (c^_t.k_t) k_t, because
// the complex scalar a_t commutes with the real projection I - beta k k^T.
// That removes the per-element rotation from the correction update.
//
// Four launches, all on the caller's stream:
//   1. summary:  one pass over k, v, beta, dt, r per chunk -> (F_k = z_{Q-1}, G_k)
//   2. fold:     per (b, h, segment of kSegLen chunks, d): compose the segment's
//                carry maps -> (A_seg = prod G, X_seg = segment carry from 0)
//   3. replay:   per (b, h, segment, d): state entering the segment from the
//                earlier segments' (A, X), then replay the segment, writing the
//                state entering every chunk over F_k, and the final state
//   4. main:     per chunk: z and c^ recurrences with the readout; writes y.
//
// Work layout of passes 1 and 4: one wave64 holds HPW = 64/LPH heads of one
// (b, chunk); each head is owned by LPH consecutive lanes, each lane holding
// DPL = D/LPH consecutive state elements, so every q/k row slice is one 8- or
// 16-byte load and a head's row is one contiguous segment.  Dot products
// reduce over the LPH lanes with DPP.  The per-token scalars (a, w, beta,
// sel_C) are computed once per token-head into LDS, one lane per token.
// Row loads are unconditional (addresses clamped into the tile) and issued
// kPrefetch tokens ahead, so the loop carries no branch and the memory waits
// count only the oldest load.  Tokens past the end of a ragged last chunk are
// inert steps (a = 1, w = 0, beta = 0).
#include <atomic>
#include <mutex>

#include "chunk_sweep.hpp"
#include "common.hpp"

namespace cdssm {

constexpr int kPrefetch = 8;

// Device-side state of this unit's one-pass forward, one copy per GPU:
// the count of one-pass calls (the source of their look-back epochs) and the
// sticky status word (kTimeoutFwd once a look-back wait gave up).
__device__ unsigned long long g_fwd_calls;
__device__ unsigned int g_fwd_status;

// One thread: draw the next forward epoch into the control block and clear
// the count of finished workgroups.
__global__ __launch_bounds__(64) void fwd_epoch_kernel(unsigned long long* ctl) {
  if (threadIdx.x == 0) {
    const unsigned long long n =
        __hip_atomic_fetch_add(&g_fwd_calls, 1ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) + 1ull;
    __hip_atomic_store(ctl + 1, 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __hip_atomic_store(ctl, epoch_word(1u, n), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
}

// Lanes per head of the bf16 D = 64 forward (8: one 16-byte row slice per
// lane; 16 or 32: more waves per SIMD at smaller slices).
#ifndef CDSSM_FWD_LPH_BF16_D64
#define CDSSM_FWD_LPH_BF16_D64 8
#endif
#ifndef CDSSM_FWD_LPHS_BF16_D64
#define CDSSM_FWD_LPHS_BF16_D64 8
#endif
#ifndef CDSSM_FWD_LPHS_BF16_D128
#define CDSSM_FWD_LPHS_BF16_D128 16
#endif

template <typename T, int D, int LPH>
struct FusedCfg {
  static constexpr int DPL = D / LPH;
  static constexpr int HPW = kWave / LPH;
  static_assert(HPW * LPH == kWave, "lane groups tile the wave");
};

// Per-token scalars of the tile in LDS, slot p = t*HPW + j (token t, head j):
//   A[p] = (e_re, e_im, beta, sel_C)   the step's write coefficient: w/f_t, or w
//                                       at a frame reset
//   B[p] = (f_re, f_im, gp_re, gp_im)  the local frame f_t and g_{t-1}
//   M[p] = (m_re, m_im)                 1, or f_{t-1} a_t at a frame reset
struct TileScalars {
  float4* A;
  float4* B;
  float2* M;
};

// Tokens where some head of the wave resets its frame.  The staging lanes own
// (head, block of TPB tokens) of a 64-token slab; after staging, every lane
// holds in v0 (slab 0) / v1 (slab 1) the OR over the wave's heads of its
// block's TPB flags (bit i: token block * TPB + i), so lane b holds block b's.
template <int TPB>
struct ResetMask {
  static_assert(TPB >= 1 && TPB <= 8 && 8 % TPB == 0, "blocks tile an 8-token group");
  uint32_t v0, v1;
  // Bits of the 8 tokens tb .. tb + 7 (tb a multiple of 8), bit i for token
  // tb + i, as a scalar: 8 / TPB lane reads, once per token group.
  __device__ __forceinline__ uint32_t group8(int tb) const {
    const int src = int(tb < 64 ? v0 : v1);
    const int b0 = (tb & 63) / TPB;
    uint32_t g = 0;
#pragma unroll
    for (int u = 0; u < 8 / TPB; ++u) g |= uint32_t(__builtin_amdgcn_readlane(src, b0 + u)) << (u * TPB);
    return g;
  }
};

// The local state is kept in a rescaled frame, z_t = f_t zh_t (f complex, per
// head).  A step z_t = a (z_{t-1} - beta (z_{t-1}.k) k) + w k becomes
//   zh_t = zh_{t-1} + (w/f_t - beta ph) k,   f_t = f_{t-1} a_t,   ph = zh_{t-1}.k
// (two FMAs per element), or, at a frame reset, the direct step
//   zh_t = m zh_{t-1} + (w - m beta ph) k,   m = f_{t-1} a_t,   f_t = 1.
// Resets are placed where log2 |g_t|^2 (g_t = prod_{u<=t} a_u) crosses a
// multiple of -kBand, and at every token with |a_t|^2 < 2^-kBandStep; the
// decay between two resets then stays above 2^-kBand, so |f|^2 > 2^-kBand and
// 1/f is finite.  The positions depend only on the a_t, so they are found
// here, in parallel over tokens (prefix sums), and the loops branch on a
// wave-uniform mask instead of testing |f| every step.
constexpr float kBand = 120.0f;
constexpr float kBandStep = 60.0f;

// Stage the tile's per-token scalars.  Work layout: lane = (head j, block of
// TPB = HPW consecutive tokens of a 64-token slab), NB = 64/HPW blocks per
// head.  Each lane first issues all of its loads (addresses clamped into the
// tile), computes its tokens' dynamics, runs the three prefix scans (log2|g|^2
// for the reset bands, the segmented frame product f, the plain product g)
// sequentially over its own tokens, and joins them across the head's NB
// lanes with log2(NB) shuffle steps.  `pre` (the caller's row prefetch) is
// issued right after the first slab's loads.  Slots past the last token and heads
// >= H hold inert steps (a = 1, w = 0, beta = 0).  Summary pass (MAIN false):
// writes G_k = g over the chunk to gam and the last frame f to B[j]; with
// cend (MAIN true) the same pair goes to cend[j].
struct NoPrefetch {
  __device__ void operator()() const {}
};

// Wide staging loads (WIDE: the scan-level bf16 form, 8 heads per wave, H a
// multiple of 8 and chunks of at most 64 tokens): lane t loads token t's
// 16-byte rows of the wave's 8 heads (beta, sel_C, dt, r; v as two rows of 4
// (re, im) pairs) -- six loads instead of 7 * 8 two-byte ones -- and writes
// them to LDS, from where the staging lanes read their (head, token block)
// values.  Token t's rows sit at 16-byte unit t + t / 8 of each array (a
// 16-byte pad after every 8 tokens), so the reads of one instruction fall in
// 32 distinct banks.
constexpr int kWideUnits = kWave + kWave / 8;  // 16-byte units of one array

template <typename T, int HPW, bool MAIN, typename Pre = NoPrefetch, bool WIDE = false>
__device__ __forceinline__ ResetMask<HPW> stage_scalars(const ChunkTile& tc, int H, int ntr,
                                                   const typename T::raw* __restrict__ v,
                                                   const typename T::raw* __restrict__ beta,
                                                   const typename T::raw* __restrict__ sel_c,
                                                   const typename T::raw* __restrict__ dt,
                                                   const typename T::raw* __restrict__ r,
                                                   const float* __restrict__ alpha,
                                                   const float* __restrict__ omega, float c,
                                                   const TileScalars& s, float2* __restrict__ gam,
                                                   int64_t gam_base, float2* __restrict__ gsv = nullptr,
                                                   float4* __restrict__ cend = nullptr, Pre pre = Pre{}, int R = 1) {
  constexpr int NB = kWave / HPW;
  constexpr int TPB = HPW;
  static_assert(NB * TPB == kWave, "blocks tile the slab");
  const int lane = int(threadIdx.x) % kWave;  // lane in the wave (the one-pass workgroup has several)
  const int j = lane / NB;
  const int blk = lane % NB;
  const int hj = tc.hbase + j;
  const bool hok = hj < H;
  const int hl = hok ? hj : H - 1;
  constexpr bool kAbar = GivenA<T>::value;  // a_t and vp_t given (dt -> a (B,L,H,2), r -> vp)
  constexpr bool kSsd = IsSsdY<T>::value;   // SSD form: vp = 1 (values already scaled), no sel_C
  const float al = kAbar ? 0.0f : alpha[hl], om = kAbar ? 0.0f : omega[hl];
  const int glast = j * NB + NB - 1;  // the head's last lane

  ResetMask<HPW> rm{0u, 0u};
  float cL = 0.0f, cfr = 1.0f, cfi = 0.0f, cgr = 1.0f, cgi = 0.0f;  // carries from earlier slabs
  for (int tl = 0; tl < ntr; tl += kWave) {
    const int t0 = tl + blk * TPB;
    float bb[TPB], dd[TPB], rr[TPB], v0[TPB], v1[TPB], sc[TPB], vq[TPB];
    if constexpr (WIDE) {
      static_assert(MAIN && HPW == 8 && T::bytes == 2 && !kAbar, "wide staging: scan-level bf16, 8 heads");
      // lane = token (clamped into the chunk): 16-byte rows of the wave's 8 heads
      const int64_t e0 = (tc.row0 + min(lane, tc.nt - 1)) * H + tc.hbase;
      const uint4 lb = *reinterpret_cast<const uint4*>(beta + e0);
      const uint4 ls = *reinterpret_cast<const uint4*>(sel_c + e0);
      const uint4 ld = *reinterpret_cast<const uint4*>(dt + e0);
      const uint4 lr = *reinterpret_cast<const uint4*>(r + e0);
      const uint4 lv0 = *reinterpret_cast<const uint4*>(v + 2 * e0);
      const uint4 lv1 = *reinterpret_cast<const uint4*>(v + 2 * e0 + 8);
      // the caller's row loads go out before these rows are waited for
      pre();
      __builtin_amdgcn_sched_barrier(0);
      // exchange through LDS: the wave's B slots, which are written only after these reads
      uint4* xw = reinterpret_cast<uint4*>(s.B);
      const int u = lane + lane / 8;
      xw[0 * kWideUnits + u] = lb;
      xw[1 * kWideUnits + u] = ls;
      xw[2 * kWideUnits + u] = ld;
      xw[3 * kWideUnits + u] = lr;
      xw[4 * kWideUnits + u] = lv0;
      xw[5 * kWideUnits + u] = lv1;
      const uint16_t* xh = reinterpret_cast<const uint16_t*>(s.B);
      const uint32_t* xv = reinterpret_cast<const uint32_t*>(s.B);
#pragma unroll
      for (int i = 0; i < TPB; ++i) {
        const int ut = t0 + i + blk;  // 16-byte unit of token t0 + i (t0 = 8 blk)
        bb[i] = bf16_to_f32(xh[(0 * kWideUnits + ut) * 8 + j]);
        sc[i] = bf16_to_f32(xh[(1 * kWideUnits + ut) * 8 + j]);
        dd[i] = bf16_to_f32(xh[(2 * kWideUnits + ut) * 8 + j]);
        rr[i] = bf16_to_f32(xh[(3 * kWideUnits + ut) * 8 + j]);
        const uint32_t pv = xv[((4 + j / 4) * kWideUnits + ut) * 4 + j % 4];
        v0[i] = bf16_lo(pv);
        v1[i] = bf16_hi(pv);
        vq[i] = 0.0f;
      }
    } else {
    // R state rows per head (the given-transition forms): beta and sel_C per real
    // head, which the head's R virtual heads share; R = 1 otherwise
    const int Hk = H / R, hk = hl / R;
#pragma unroll
    for (int i = 0; i < TPB; ++i) {
      const int t = min(t0 + i, tc.nt - 1);
      const int64_t e = (tc.row0 + t) * H + hl;
      const int64_t ek = (tc.row0 + t) * Hk + hk;
      bb[i] = T::load(beta + ek);
      if constexpr (kAbar) {
        dd[i] = T::load(dt + 2 * e);  // a_t re, im
        rr[i] = T::load(dt + 2 * e + 1);
        vq[i] = kSsd ? 1.0f : T::load(r + e);  // vp_t
      } else {
        dd[i] = T::load(dt + e);
        rr[i] = T::load(r + e);
        vq[i] = 0.0f;
      }
      v0[i] = T::load(v + 2 * e);
      v1[i] = T::load(v + 2 * e + 1);
      sc[i] = MAIN && !kSsd ? T::load(sel_c + ek) : 0.0f;
    }
    // the caller's row prefetch goes after these small loads, so waiting for
    // them does not wait for the rows
    if (tl == 0) pre();
    }
    // dynamics and local (in-block) prefixes; computed for every slot (the
    // clamped loads hold valid numbers) and replaced by an inert step where
    // the slot is not a real token, so the tokens interleave without branches
    float ar[TPB], ai[TPB], wr[TPB], wi[TPB], Ls[TPB], Gr[TPB], Gi[TPB];
    bool forced[TPB];
    float lsum = 0.0f, gpr = 1.0f, gpi = 0.0f;
#pragma unroll
    for (int i = 0; i < TPB; ++i) {
      const bool real = hok && t0 + i < tc.nt;
      const Transition tr = kAbar ? Transition{dd[i], rr[i], vq[i]} : cayley_gated(dd[i], rr[i], al, om, c);
      const float f = bb[i] * tr.vp;
      ar[i] = real ? tr.ar : 1.0f;
      ai[i] = real ? tr.ai : 0.0f;
      wr[i] = real ? f * v0[i] : 0.0f;
      wi[i] = real ? f * v1[i] : 0.0f;
      bb[i] = real ? bb[i] : 0.0f;
      sc[i] = real ? sc[i] : 0.0f;
      const float m2 = ar[i] * ar[i] + ai[i] * ai[i];
      forced[i] = !(m2 >= 0x1p-60f);  // also NaN
      lsum += forced[i] ? -kBandStep : __builtin_amdgcn_logf(m2);
      Ls[i] = lsum;
      cmul_acc(gpr, gpi, ar[i], ai[i]);
      Gr[i] = gpr;
      Gi[i] = gpi;
    }
    // exclusive prefix over the head's blocks: sum of log2|a|^2, product of a
    float xL = lsum, xgr = gpr, xgi = gpi;
    for_shifts<NB>([&](auto offc) {
      constexpr int off = decltype(offc)::value;
      const float yL = seg_shift_up<NB, off>(xL), ygr = seg_shift_up<NB, off>(xgr),
                  ygi = seg_shift_up<NB, off>(xgi);
      if (blk >= off) {
        xL += yL;
        cmul_acc(xgr, xgi, ygr, ygi);
      }
    });
    float eL = seg_shift_up<NB, 1>(xL), egr = seg_shift_up<NB, 1>(xgr), egi = seg_shift_up<NB, 1>(xgi);
    if (blk == 0) {
      eL = 0.0f;
      egr = 1.0f;
      egi = 0.0f;
    }
    eL += cL;
    cmul_acc(egr, egi, cgr, cgi);  // g entering the block
    // reset positions and the in-block segmented frame product
    bool reset[TPB];
    float Fr[TPB], Fi[TPB];
    bool anyr = false;
    {
      float bprev = floorf(eL * (-1.0f / kBand));
      float fr = 1.0f, fi = 0.0f;
#pragma unroll
      for (int i = 0; i < TPB; ++i) {
        const float band = floorf((eL + Ls[i]) * (-1.0f / kBand));
        reset[i] = forced[i] || band != bprev;
        bprev = band;
        const float nr = fr * ar[i] - fi * ai[i];
        const float ni = fr * ai[i] + fi * ar[i];
        fr = reset[i] ? 1.0f : nr;
        fi = reset[i] ? 0.0f : ni;
        anyr = anyr || reset[i];
        Fr[i] = fr;
        Fi[i] = fi;
      }
    }
    // frame entering the block: segmented exclusive scan over blocks, seeded
    // with the carry (which acts as a reset element)
    float xfr = Fr[TPB - 1], xfi = Fi[TPB - 1];
    int xfl = anyr;
    for_shifts<NB>([&](auto offc) {
      constexpr int off = decltype(offc)::value;
      const float yr = seg_shift_up<NB, off>(xfr), yi = seg_shift_up<NB, off>(xfi);
      const int yf = seg_shift_up<NB, off>(xfl);
      if (blk >= off && !xfl) {
        cmul_acc(xfr, xfi, yr, yi);
        xfl = yf;
      }
    });
    float efr = seg_shift_up<NB, 1>(xfr), efi = seg_shift_up<NB, 1>(xfi);
    int efl = seg_shift_up<NB, 1>(xfl);
    if (blk == 0) {
      efr = 1.0f;
      efi = 0.0f;
      efl = 0;
    }
    if (!efl) cmul_acc(efr, efi, cfr, cfi);
    // per token outputs (every slot of the slab: LDS holds whole slabs)
    float fpr = efr, fpi = efi;  // f_{t-1}
    float lfr = efr, lfi = efi;  // f_t
    bool seen = false;           // a reset at or before this token in the block
#pragma unroll
    for (int i = 0; i < TPB; ++i) {
      seen = seen || reset[i];
      lfr = seen ? Fr[i] : Fr[i] * efr - Fi[i] * efi;
      lfi = seen ? Fi[i] : Fr[i] * efi + Fi[i] * efr;
      const int t = t0 + i;
      const int p = t * HPW + j;
      const float inv = __builtin_amdgcn_rcpf(lfr * lfr + lfi * lfi);
      const float er = reset[i] ? wr[i] : (wr[i] * lfr + wi[i] * lfi) * inv;
      const float ei = reset[i] ? wi[i] : (wi[i] * lfr - wr[i] * lfi) * inv;
      s.A[p] = make_float4(er, ei, bb[i], sc[i]);
      if (MAIN) {
        // g_{t-1} = g entering the block times the in-block product before t
        float gr = egr, gi = egi;
        if (i > 0) cmul_acc(gr, gi, Gr[i - 1], Gi[i - 1]);
        s.B[p] = make_float4(lfr, lfi, gr, gi);
        if (gsv && hok && t < tc.nt) {
          // training forward: keep g_t for the backward's correction adjoint
          cmul_acc(gr, gi, ar[i], ai[i]);
          gsv[(tc.row0 + t) * H + hj] = make_float2(gr, gi);
        }
      }
      const float mr = fpr * ar[i] - fpi * ai[i], mi = fpr * ai[i] + fpi * ar[i];
      s.M[p] = reset[i] ? make_float2(mr, mi) : make_float2(1.0f, 0.0f);
      fpr = lfr;
      fpi = lfi;
    }
    // this lane's block flags, then OR over the heads (lanes NB apart)
    uint32_t r8 = 0;
#pragma unroll
    for (int i = 0; i < TPB; ++i) r8 |= reset[i] ? (1u << i) : 0u;
#pragma unroll
    for (int sh = NB; sh < kWave; sh <<= 1) r8 |= uint32_t(__shfl_xor(int(r8), sh, kWave));
    if (tl == 0)
      rm.v0 = r8;
    else
      rm.v1 = r8;
    // carries to the next slab, from the head's last lane
    float gtr = egr, gti = egi;
    cmul_acc(gtr, gti, gpr, gpi);
    cL = __shfl(eL + lsum, glast, kWave);
    cfr = __shfl(lfr, glast, kWave);
    cfi = __shfl(lfi, glast, kWave);
    cgr = __shfl(gtr, glast, kWave);
    cgi = __shfl(gti, glast, kWave);
  }
  if (!MAIN && blk == 0) {
    // G_k = g over the whole (padded) chunk and the frame after its last step
    // (inert steps have a = 1)
    if (hok) gam[gam_base + j] = make_float2(cgr, cgi);
    s.B[j] = make_float4(cfr, cfi, 0.0f, 0.0f);
  }
  // one-pass forward: (G_k, frame after the last step) per head of the tile
  if (MAIN && cend && blk == 0) cend[j] = make_float4(cgr, cgi, cfr, cfi);
  return rm;
}

// zh *= m (complex, in place)
template <int DPL>
__device__ __forceinline__ void zscale(float (&zr)[DPL], float (&zi)[DPL], float2 m) {
#pragma unroll
  for (int j = 0; j < DPL; ++j) {
    const float xr = m.x * zr[j] - m.y * zi[j];
    zi[j] = m.x * zi[j] + m.y * zr[j];
    zr[j] = xr;
  }
}

// One local step for a lane's DPL elements (see the frame rule above).  At a
// token where some head of the wave resets, zh is first scaled in place by m
// (m = 1 for the other heads), then every head takes the common update
// zh += e k; returns e, which replays the step without the dot product.
template <int DPL>
__device__ __forceinline__ float2 local_step(float (&zr)[DPL], float (&zi)[DPL], const float (&kk)[DPL],
                                             bool reset_any, float2 m, float er0, float ei0,
                                             float bb, float pr, float pi) {
  float bpr = bb * pr, bpi = bb * pi;
  if (reset_any) {
    zscale<DPL>(zr, zi, m);
    const float nr = m.x * bpr - m.y * bpi;
    bpi = m.x * bpi + m.y * bpr;
    bpr = nr;
  }
  const float er = er0 - bpr, ei = ei0 - bpi;
#pragma unroll
  for (int j = 0; j < DPL; ++j) {
    zr[j] = fmaf(er, kk[j], zr[j]);
    zi[j] = fmaf(ei, kk[j], zi[j]);
  }
  return make_float2(er, ei);
}

// ---------------------------------------------------------------------------
// Pass 1: chunk summaries F_k = z_{Q-1} (local state from zero) and G_k.
// ---------------------------------------------------------------------------
template <typename T, int D, int LPH>
__global__ __launch_bounds__(kWave) void fused_fwd_summary_kernel(
    const typename T::raw* __restrict__ k, const typename T::raw* __restrict__ v,
    const typename T::raw* __restrict__ beta, const typename T::raw* __restrict__ dt,
    const typename T::raw* __restrict__ r, const float* __restrict__ alpha,
    const float* __restrict__ omega, float c, float2* __restrict__ summ, float2* __restrict__ gam,
    int L, int H, int Q, int NC, int n_hg, int R = 1) {
  using Cfg = FusedCfg<T, D, LPH>;
  constexpr int DPL = Cfg::DPL, HPW = Cfg::HPW, PF = kPrefetch;
  // the given-transition forms: R virtual heads (state rows) share each k row
  constexpr bool RW = GivenA<T>::value;
  extern __shared__ float4 smem4[];
  const ChunkTile tc = decode_tile(L, Q, NC, n_hg, HPW);
  const int lane = threadIdx.x;
  const int hh = lane / LPH;
  const int sub = lane % LPH;
  const int h = tc.hbase + hh;
  const bool hok = h < H;
  const int ntr = round_up(tc.nt, PF);
  const int slots = round_up(Q, kWave) * HPW;
  const int64_t ch0 = (int64_t(tc.b) * NC + tc.chunk) * H + tc.hbase;

  const RowStream ks = RW ? tile_stream_rows<T>(k, tc, L, H, R, D, hh, sub * DPL)
                          : tile_stream<T>(k, tc, L, H, D, hh, sub * DPL);
  const int rowb = (RW ? H / R : H) * D * T::bytes;  // token stride of k in bytes
  const int tlast = tc.nt - 1;
  const int slim = tlast * rowb;
  RowVec<T, DPL> kb[PF];
  TileScalars s{smem4, smem4 + slots, reinterpret_cast<float2*>(smem4 + slots + HPW)};
  const auto rm = stage_scalars<T, HPW, false>(tc, H, ntr, v, beta, nullptr, dt, r, alpha, omega, c, s,
                                                    gam, ch0, nullptr, nullptr, [&] {
#pragma unroll
                                                      for (int i = 0; i < PF; ++i)
                                                        kb[i].load(ks, min(i * rowb, slim));
                                                    }, R);
#pragma unroll
  for (int i = 0; i < PF; ++i) kb[i].pin();
  __syncthreads();

  float zr[DPL], zi[DPL];
#pragma unroll
  for (int j = 0; j < DPL; ++j) zr[j] = zi[j] = 0.0f;

  for (int tb = 0; tb < ntr; tb += PF) {
    float4 sa[PF];
    float2 sm[PF];
#pragma unroll
    for (int i = 0; i < PF; ++i) {
      sa[i] = s.A[(tb + i) * HPW + hh];
      sm[i] = s.M[(tb + i) * HPW + hh];
    }
    const int nb = (tb + PF) * rowb;
    const uint32_t rg = rm.group8(tb);
#pragma unroll
    for (int i = 0; i < PF; ++i) {
      float kk[DPL];
      kb[i].unpack_then_reload(kk);
      kb[i].load(ks, min(nb + i * rowb, slim));
      float pr0 = 0.0f, pi0 = 0.0f, pr1 = 0.0f, pi1 = 0.0f;
#pragma unroll
      for (int j = 0; j < DPL; j += 2) {
        pr0 = fmaf(zr[j], kk[j], pr0);
        pi0 = fmaf(zi[j], kk[j], pi0);
        pr1 = fmaf(zr[j + 1], kk[j + 1], pr1);
        pi1 = fmaf(zi[j + 1], kk[j + 1], pi1);
      }
      const float pr = group_sum<LPH>(pr0 + pr1);
      const float pi = group_sum<LPH>(pi0 + pi1);
      local_step<DPL>(zr, zi, kk, (rg >> i) & 1u, sm[i], sa[i].x, sa[i].y, sa[i].z, pr, pi);
    }
  }

  if (hok) {
    const float4 fe = s.B[hh];
    float2* sp = summ + (ch0 + hh) * D + sub * DPL;
#pragma unroll
    for (int j = 0; j < DPL; ++j) sp[j] = make_float2(fe.x * zr[j] - fe.y * zi[j], fe.x * zi[j] + fe.y * zr[j]);
  }
}

// ---------------------------------------------------------------------------
// Passes 2-3: inter-chunk carry, s_{k+1} = G_k s_k + F_k (elementwise complex),
// split into segments of kSegLen chunks.  Loads are issued in groups of 8
// with clamped indices so the serial chain waits on memory once per group.
// ---------------------------------------------------------------------------
__device__ __forceinline__ float2 cmul(float2 a, float2 b) {
  return make_float2(a.x * b.x - a.y * b.y, a.x * b.y + a.y * b.x);
}
__device__ __forceinline__ float2 cfma(float2 a, float2 b, float2 c) {
  return make_float2(fmaf(a.x, b.x, fmaf(-a.y, b.y, c.x)), fmaf(a.x, b.y, fmaf(a.y, b.x, c.y)));
}

struct CarryIdx {
  int b, h, seg, d, c0, c1;
  int64_t base;  // chunk ch of (b, h) is element base + ch * H
};

__device__ __forceinline__ CarryIdx carry_index(int64_t tid, int NC, int H, int D, int S) {
  CarryIdx x;
  x.d = int(tid % D);
  int64_t rest = tid / D;
  x.seg = int(rest % S);
  rest /= S;
  x.h = int(rest % H);
  x.b = int(rest / H);
  x.c0 = min(NC, x.seg * kSegLen);
  x.c1 = min(NC, x.c0 + kSegLen);
  x.base = int64_t(x.b) * NC * H + x.h;
  return x;
}

__global__ __launch_bounds__(256) void fused_fwd_fold_kernel(const float2* __restrict__ summ,
                                                            const float2* __restrict__ gam,
                                                            float2* __restrict__ segA,
                                                            float2* __restrict__ segX, int B, int NC,
                                                            int H, int D, int S) {
  const int64_t tid = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  if (tid >= int64_t(B) * H * S * D) return;
  const CarryIdx x = carry_index(tid, NC, H, D, S);
  float2 A = make_float2(1.0f, 0.0f), X = make_float2(0.0f, 0.0f);
  const int last = max(x.c1 - 1, 0);
  for (int cb = x.c0; cb < x.c1; cb += 8) {
    float2 G[8], F[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int64_t e = x.base + int64_t(min(cb + i, last)) * H;
      G[i] = gam[e];
      F[i] = summ[e * D + x.d];
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      if (cb + i < x.c1) {
        X = cfma(G[i], X, F[i]);
        A = cmul(G[i], A);
      }
    }
  }
  const int64_t sidx = (int64_t(x.b) * H + x.h) * S + x.seg;
  segX[sidx * D + x.d] = X;
  if (x.d == 0) segA[sidx] = A;
}

__global__ __launch_bounds__(256) void fused_fwd_replay_kernel(float2* __restrict__ summ,
                                                              const float2* __restrict__ gam,
                                                              const float2* __restrict__ segA,
                                                              const float2* __restrict__ segX,
                                                              const float* __restrict__ h0,
                                                              float* __restrict__ h_final, int B,
                                                              int NC, int H, int D, int S) {
  const int64_t tid = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  if (tid >= int64_t(B) * H * S * D) return;
  const CarryIdx x = carry_index(tid, NC, H, D, S);
  const int64_t sbase = (int64_t(x.b) * H + x.h) * S;
  const int64_t hb = (int64_t(x.b) * H + x.h) * 2 * D;
  float2 s = make_float2(0.0f, 0.0f);
  if (h0 != nullptr) s = make_float2(h0[hb + x.d], h0[hb + D + x.d]);
  // state entering the segment
  for (int jb = 0; jb < x.seg; jb += 8) {
    float2 A[8], X[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int64_t j = sbase + min(jb + i, x.seg - 1);
      A[i] = segA[j];
      X[i] = segX[j * D + x.d];
    }
#pragma unroll
    for (int i = 0; i < 8; ++i)
      if (jb + i < x.seg) s = cfma(A[i], s, X[i]);
  }
  // replay the segment, writing the state entering each chunk over F
  const int last = max(x.c1 - 1, 0);
  for (int cb = x.c0; cb < x.c1; cb += 8) {
    float2 G[8], F[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int64_t e = x.base + int64_t(min(cb + i, last)) * H;
      G[i] = gam[e];
      F[i] = summ[e * D + x.d];
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      if (cb + i < x.c1) {
        summ[(x.base + int64_t(cb + i) * H) * D + x.d] = s;
        s = cfma(G[i], s, F[i]);
      }
    }
  }
  if (x.c0 < x.c1 && x.c1 == NC) {
    h_final[hb + x.d] = s.x;
    h_final[hb + D + x.d] = s.y;
  }
}

// ---------------------------------------------------------------------------
// Pass 4: per chunk, local state z (rescaled frame) and decay-free correction
// c^ from s_k; output y_t = sel_C_t (f_t (zh_t . q_t) + g_{t-1} (c^_t . q_t)).
// SAVE (training forward): also keeps, per (token, head), the dot products the
// backward needs, saved[2 e] = (p_t, pc_t), saved[2 e + 1] = (c^_{t+1}.q_t,
// Y_t.q_t), with p_t = z_{t-1}.k_t in true units and pc_t = c^_t.k_t, so the
// backward recomputes the chunk states without any reduction, gsaved[e] =
// g_t (the in-chunk decay product the correction adjoint needs), the z
// checkpoints z_{t-1} at t % kZck == 0 and c^ after the chunk's last step.
// ---------------------------------------------------------------------------
// CORR false: the local part only, y_t = sel_C_t f_t (zh_t . q_t) + ycorr_t, with
// the correction readout ycorr (B, L, H) complex fp32 computed beforehand by the
// chunked correction (fused_fwd_corr_sweep_kernel).
template <typename T, int D, int LPH, bool SAVE, bool CORR = true>
__global__ __launch_bounds__(kWave) void fused_fwd_main_kernel(
    const typename T::raw* __restrict__ q, const typename T::raw* __restrict__ k,
    const typename T::raw* __restrict__ v, const typename T::raw* __restrict__ beta,
    const typename T::raw* __restrict__ sel_c, const typename T::raw* __restrict__ dt,
    const typename T::raw* __restrict__ r, const float* __restrict__ alpha,
    const float* __restrict__ omega, float c, const float2* __restrict__ states,
    typename T::raw* __restrict__ y, float4* __restrict__ saved, float2* __restrict__ gsaved,
    float2* __restrict__ zck, float2* __restrict__ cend, int L, int H, int Q, int NC, int NCK, int n_hg,
    const float2* __restrict__ ycorr = nullptr, int R = 1) {
  static_assert(CORR || !SAVE, "the training forward keeps the sequential correction");
  constexpr bool YM = IsSsdY<T>::value;  // SSD form: write Y (B,L,H,2,D), no q, no readout
  static_assert(CORR || !YM, "the SSD form keeps the sequential correction");
  using Cfg = FusedCfg<T, D, LPH>;
  constexpr int DPL = Cfg::DPL, HPW = Cfg::HPW, PF = kPrefetch;
  static_assert(PF == kTokRound && PF % kZck == 0, "z checkpoints fall at fixed positions of a prefetch group");
  extern __shared__ float4 smem4[];
  const ChunkTile tc = decode_tile(L, Q, NC, n_hg, HPW);
  const int lane = threadIdx.x;
  const int hh = lane / LPH;
  const int sub = lane % LPH;
  const int h = tc.hbase + hh;
  const bool hok = h < H;
  const int ntr = round_up(tc.nt, PF);
  const int slots = round_up(Q, kWave) * HPW;

  // the given-transition forms: R virtual heads (state rows) share each k (and q) row
  constexpr bool RW = GivenA<T>::value;
  const RowStream ks = RW ? tile_stream_rows<T>(k, tc, L, H, R, D, hh, sub * DPL)
                          : tile_stream<T>(k, tc, L, H, D, hh, sub * DPL);
  const RowStream qs = YM   ? RowStream{}
                       : RW ? tile_stream_rows<T>(q, tc, L, H, R, D, hh, sub * DPL)
                            : tile_stream<T>(q, tc, L, H, D, hh, sub * DPL);
  // SSD form: this lane's slices of its head's Y re and im rows (D apart)
  const RowStream yre = YM ? tile_stream<T>(y, tc, L, H, 2 * D, hh, sub * DPL) : RowStream{};
  const RowStream yim = YM ? tile_stream<T>(y, tc, L, H, 2 * D, hh, D + sub * DPL) : RowStream{};
  const int rowy = 2 * H * D * T::bytes;  // token stride of Y in bytes
  const int rowb = (RW ? H / R : H) * D * T::bytes;  // token stride of k (and q) in bytes
  const int tlast = tc.nt - 1;
  const int slim = tlast * rowb;
  RowVec<T, DPL> kb[PF], qb[PF];
  float zr[DPL], zi[DPL], cr[DPL], ci[DPL];
  {
    const int hl = hok ? h : H - 1;
    const float2* sp = states + ((int64_t(tc.b) * NC + tc.chunk) * H + hl) * D + sub * DPL;
#pragma unroll
    for (int j = 0; j < DPL; ++j) {
      const float2 sv = sp[j];
      zr[j] = zi[j] = 0.0f;
      cr[j] = hok ? sv.x : 0.0f;
      ci[j] = hok ? sv.y : 0.0f;
    }
  }

  TileScalars s{smem4, smem4 + slots, reinterpret_cast<float2*>(smem4 + 2 * slots)};
  float2* s_y = s.M + slots;
  const auto rm = stage_scalars<T, HPW, true>(tc, H, ntr, v, beta, sel_c, dt, r, alpha, omega, c, s,
                                                   nullptr, 0, SAVE ? gsaved : nullptr, nullptr, [&] {
#pragma unroll
                                                     for (int i = 0; i < PF; ++i) {
                                                       kb[i].load(ks, min(i * rowb, slim));
                                                       if constexpr (!YM) qb[i].load(qs, min(i * rowb, slim));
                                                     }
                                                   }, R);
#pragma unroll
  for (int i = 0; i < PF; ++i) {
    kb[i].pin();
    if constexpr (!YM) qb[i].pin();
  }
  __syncthreads();

  float fpr = 1.0f, fpi = 0.0f;  // frame f_{t-1}
  float4* svp = SAVE ? saved + 2 * ((tc.row0 * H) + (hok ? h : H - 1)) : nullptr;
  const int64_t tile_h = (int64_t(tc.b) * NC + tc.chunk) * H + (hok ? h : H - 1);  // (b, chunk, h)
  const int64_t zc0 = tile_h * NCK * D + sub * DPL;  // this lane's z checkpoint row, slot 0

  for (int tb = 0; tb < ntr; tb += PF) {
    float4 sa[PF], sb[PF];
    float2 sm[PF];
#pragma unroll
    for (int i = 0; i < PF; ++i) {
      sa[i] = s.A[(tb + i) * HPW + hh];
      sb[i] = s.B[(tb + i) * HPW + hh];
      sm[i] = s.M[(tb + i) * HPW + hh];
    }
    float yr[PF], yi[PF];
    const int nb = (tb + PF) * rowb;
    const uint32_t rg = rm.group8(tb);
#pragma unroll
    for (int i = 0; i < PF; ++i) {
      const int t = tb + i;
      if (SAVE && i % kZck == 0 && hok) {
        // z_{t-1} = f_{t-1} zh_{t-1}
        float xr[DPL], xi[DPL];
#pragma unroll
        for (int j = 0; j < DPL; ++j) {
          xr[j] = fpr * zr[j] - fpi * zi[j];
          xi[j] = fpr * zi[j] + fpi * zr[j];
        }
        store_zck<T, DPL>(zck, zc0 + (t / kZck) * D, xr, xi);
      }
      float kk[DPL], qq[DPL];
      kb[i].unpack_then_reload(kk);
      if constexpr (!YM) qb[i].unpack_then_reload(qq);
      kb[i].load(ks, min(nb + i * rowb, slim));
      if constexpr (!YM) qb[i].load(qs, min(nb + i * rowb, slim));

      float pzr = 0.0f, pzi = 0.0f, pcr = 0.0f, pci = 0.0f, qcr = 0.0f, qci = 0.0f;
#pragma unroll
      for (int j = 0; j < DPL; ++j) {
        pzr = fmaf(zr[j], kk[j], pzr);
        pzi = fmaf(zi[j], kk[j], pzi);
        if (CORR) {
          pcr = fmaf(cr[j], kk[j], pcr);
          pci = fmaf(ci[j], kk[j], pci);
          if constexpr (!YM) {
            qcr = fmaf(cr[j], qq[j], qcr);
            qci = fmaf(ci[j], qq[j], qci);
          }
        }
      }
      pzr = group_sum<LPH>(pzr);
      pzi = group_sum<LPH>(pzi);
      if (CORR) {
        pcr = group_sum<LPH>(pcr);
        pci = group_sum<LPH>(pci);
      }

      const float bb = sa[i].z;
      local_step<DPL>(zr, zi, kk, (rg >> i) & 1u, sm[i], sa[i].x, sa[i].y, bb, pzr, pzi);
      const float ecr = bb * pcr, eci = bb * pci;
      if constexpr (YM) {
        // Y_t = f_t zh_t + g_{t-1} c^_t (the correction before this token's step)
        const float4 fb = sb[i];
        float ya[DPL], yb[DPL];
#pragma unroll
        for (int j = 0; j < DPL; ++j) {
          ya[j] = fmaf(fb.x, zr[j], fmaf(-fb.y, zi[j], fmaf(fb.z, cr[j], -fb.w * ci[j])));
          yb[j] = fmaf(fb.x, zi[j], fmaf(fb.y, zr[j], fmaf(fb.z, ci[j], fb.w * cr[j])));
          cr[j] = fmaf(-ecr, kk[j], cr[j]);
          ci[j] = fmaf(-eci, kk[j], ci[j]);
        }
        if (hok && t < tc.nt) {
          store_row<T, DPL>(yre, t * rowy, ya);
          store_row<T, DPL>(yim, t * rowy, yb);
        }
        if (SAVE) {
          if (sub == 0 && hok && t < tc.nt)
            svp[2 * int64_t(t) * H] = make_float4(fpr * pzr - fpi * pzi, fpr * pzi + fpi * pzr, pcr, pci);
          fpr = fb.x;
          fpi = fb.y;
        }
        continue;
      }
      float qzr = 0.0f, qzi = 0.0f, cnr = 0.0f, cni = 0.0f;
#pragma unroll
      for (int j = 0; j < DPL; ++j) {
        qzr = fmaf(zr[j], qq[j], qzr);
        qzi = fmaf(zi[j], qq[j], qzi);
        if (CORR) {
          cr[j] = fmaf(-ecr, kk[j], cr[j]);
          ci[j] = fmaf(-eci, kk[j], ci[j]);
        }
        if (SAVE) {
          cnr = fmaf(cr[j], qq[j], cnr);  // c^_{t+1}.q
          cni = fmaf(ci[j], qq[j], cni);
        }
      }
      // readout partial: f_t (zh_t.q) + g_{t-1} (c^_t.q)
      const float4 fb = sb[i];
      float Rr = fb.x * qzr - fb.y * qzi;
      float Ri = fb.x * qzi + fb.y * qzr;
      if (CORR) {
        Rr += fb.z * qcr - fb.w * qci;
        Ri += fb.z * qci + fb.w * qcr;
      }
      Rr = group_sum<LPH>(Rr);
      Ri = group_sum<LPH>(Ri);
      yr[i] = sa[i].w * Rr;
      yi[i] = sa[i].w * Ri;
      if (SAVE) {
        const float cqr = group_sum<LPH>(cnr), cqi = group_sum<LPH>(cni);
        if (sub == 0 && hok && t < tc.nt) {
          // p_t = f_{t-1} (zh_{t-1}.k_t)
          svp[2 * int64_t(t) * H] = make_float4(fpr * pzr - fpi * pzi, fpr * pzi + fpi * pzr, pcr, pci);
          svp[2 * int64_t(t) * H + 1] = make_float4(cqr, cqi, Rr, Ri);
        }
        fpr = fb.x;
        fpi = fb.y;
      }
    }
    if (!YM && sub == 0) {
#pragma unroll
      for (int i = 0; i < PF; ++i) s_y[(tb + i) * HPW + hh] = make_float2(yr[i], yi[i]);
    }
  }
  if (SAVE && hok) {
#pragma unroll
    for (int j = 0; j < DPL; ++j) cend[tile_h * D + sub * DPL + j] = make_float2(cr[j], ci[j]);
  }
  if constexpr (YM) return;  // Y went out token by token
  __syncthreads();

  // coalesced write of y (B, L, H, 2) for the tile
  const int n = tc.nt * HPW;
  for (int p = lane; p < n; p += kWave) {
    const int t = p / HPW;
    const int hj = tc.hbase + (p - t * HPW);
    if (hj < H) {
      const int64_t e = ((tc.row0 + t) * H + hj) * 2;
      float2 yv = s_y[p];
      if (!CORR) {
        const float2 yc = ycorr[e / 2];
        yv.x += yc.x;
        yv.y += yc.y;
      }
      store_pair<T>(y + e, yv.x, yv.y);
    }
  }
}

// ---------------------------------------------------------------------------
// Chunked correction on MFMA (bf16 inputs, chunk = 16 NB tokens): one wave per
// (b, chunk, 4 heads) computes the correction readout sel_C_t g_{t-1}
// (c^_t . q_t) of every token from the chunk's entering state (see
// chunk_sweep.hpp) into ycorr (B, L, H) complex fp32; the main pass with
// CORR = false adds it to the local readout.
// ---------------------------------------------------------------------------
template <int D, int NB>
__global__ __launch_bounds__(kWave) void fused_fwd_corr_sweep_kernel(
    const uint16_t* __restrict__ q, const uint16_t* __restrict__ k, const uint16_t* __restrict__ beta,
    const uint16_t* __restrict__ sel_c, const uint16_t* __restrict__ dt, const uint16_t* __restrict__ r,
    const float* __restrict__ alpha, const float* __restrict__ omega, float c, const float2* __restrict__ states,
    float2* __restrict__ ycorr, int L, int H, int NC, int n_hg) {
  constexpr int Q = 16 * NB;
  __shared__ float lds[sweep_lds_floats<NB>()];
  const ChunkTile tc = decode_tile(L, Q, NC, n_hg, kSweepHeads);
  const int lane = threadIdx.x;
  const int i = lane % 16;
  const int h = tc.hbase + lane / 16;
  const bool hok = h < H;
  const float al = alpha[hok ? h : H - 1], om = omega[hok ? h : H - 1];
  float car = 1.0f, cai = 0.0f;  // rotation product of the chunk's earlier blocks

  // the lane's token of block b: beta, sel_C and g_{t-1} from the scan-level dynamics
  auto tok = [&](int b, float& bt, float& sel, float& gr, float& gi) {
    const int t = 16 * b + i;
    const bool ok = hok && t < tc.nt;
    const int64_t e = (tc.row0 + min(t, tc.nt - 1)) * H + (hok ? h : H - 1);
    float ar = 1.0f, ai = 0.0f;
    bt = 0.0f;
    sel = 0.0f;
    if (ok) {
      const Transition tn = cayley_gated(bf16_to_f32(dt[e]), bf16_to_f32(r[e]), al, om, c);
      ar = tn.ar;
      ai = tn.ai;
      bt = bf16_to_f32(beta[e]);
      sel = bf16_to_f32(sel_c[e]);
    }
    row_cumprod(ar, ai);  // product of a over the block up to t
    gr = row_shr<1>(ar, 1.0f);
    gi = row_shr<1>(ai, 0.0f);
    cmul_acc(gr, gi, car, cai);
    cmul_acc(car, cai, row_bcast<15>(ar), row_bcast<15>(ai));
  };
  auto emit = [&](int b, float yr, float yi) {
    const int t = 16 * b + i;
    if (hok && t < tc.nt) ycorr[(tc.row0 + t) * H + h] = make_float2(yr, yi);
  };
  const float2* sp = states + (int64_t(tc.b) * NC + tc.chunk) * H * D;
  corr_sweep<D, NB>(k, q, tc.row0, tc.nt, H, tc.hbase, sp, lds, tok, emit);
}

// ---------------------------------------------------------------------------
// One-pass forward (inference): the four passes above in one launch.
// A workgroup of kOnePassW waves takes kOnePassW consecutive chunks (a
// segment) of one (b, head group); wave w owns chunk seg * kOnePassW + w.
//   1. each wave stages its chunk's scalars and runs the local recurrence
//      (rescaled frame) over the k rows, keeping each step's update
//      coefficient in LDS; its chunk map is (G_k, F_k = z_{Q-1});
//   2. the segment's chunk maps are composed through LDS into the segment
//      map, which is published.  Every kFwdGroup-th segment (a group end)
//      then composes and publishes its group's map from the maps of the
//      group's segments.  The state entering a segment is the composition,
//      oldest first, of the maps of the whole groups since its anchor
//      (segment kFwdAnchor * floor((seg - 1) / kFwdAnchor)) and then of its
//      own group's earlier segments, applied to the anchor state (h0, or the
//      published state leaving the segment before the anchor): a fixed order,
//      so the results do not depend on timing, and at most
//      kFwdAnchor / kFwdGroup + kFwdGroup - 1 maps read per segment (the fold
//      reads published maps from the device-coherent level; one level over
//      62 maps made that read the bound at 1024 chunks).  Anchor ends publish
//      their leaving state for the next kFwdAnchor segments;
//   3. each wave derives the state entering its chunk and runs the decay-free
//      correction, replaying the local state from the stored coefficients,
//      with the full readout f_t (zh_t.q_t) + g_{t-1} (c^_t.q_t) reduced once;
//      y is written coalesced.  q is read once, k twice.
// SAVE (training forward) also writes what the backward reads: the state
// entering every chunk and G_k (the four-launch layout), the per-token records
// (p_t, pc_t), (c^_{t+1}.q_t, Y_t.q_t) and g_t, as the main pass does.
// Flags hold epoch << 3 | bits (kFlagMap, kFlagLeave, kFlagGroup) with a
// per-call epoch read from the look-back area's control block, where
// fwd_epoch_kernel (launched just before, on the same stream) writes it from a
// device-side counter; so the workspace needs no clearing between calls and a
// captured HIP graph draws a new epoch on every replay.  Published
// data and flags are written and read with agent-scope atomics (stores written
// through to the device-coherent level, loads served from it), so no cache
// maintenance is needed: a writer waits until its data stores are acknowledged
// before the flag is stored, and a reader issues its data loads only after it
// has seen the flag (agent-scope release / acquire fences would write back or
// invalidate the whole L2 instead, microseconds per publish and the k, q rows
// the correction pass re-reads).  A workgroup waits only on segments of lower
// index; the launcher sizes the grid to the workgroups resident at once (one
// per segment, or fewer that take the segments in order), and a bounded wait
// turns a missing flag into NaN output instead of a hang, and sets the
// kTimeoutFwd bit of the sticky status word g_fwd_status.
// ---------------------------------------------------------------------------
// Look-back flag bits of the one-pass forward (below the epoch, flag = epoch << 3 | bits).
constexpr unsigned long long kFlagMap = 1ull;    // segment map published
constexpr unsigned long long kFlagLeave = 2ull;  // state leaving the segment published (anchor ends)
constexpr unsigned long long kFlagGroup = 4ull;  // group map published (group ends)

// Wave-wide wait: lane i watches the flag of segment js (>= 0; -1: nothing)
// of the head group's flags f0 (stride H per segment) until it carries this
// call's epoch and the bits `need`.  True once every lane's flag does; false
// when the wait bound passes first.  Wave-uniform.
__device__ __forceinline__ bool watch_flags(const unsigned long long* f0, int H, unsigned long long epoch, int js,
                                            unsigned long long need) {
  const uint64_t t_start = __builtin_amdgcn_s_memrealtime();
  for (;;) {
    bool ready = true;
    if (js >= 0) {
      const unsigned long long fv = __hip_atomic_load(const_cast<unsigned long long*>(f0 + int64_t(js) * H),
                                                      __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      ready = (fv >> 3) == epoch && (fv & need) == need;
    }
    if (__builtin_amdgcn_ballot_w64(!ready) == 0ull) return true;
    if (__builtin_amdgcn_s_memrealtime() - t_start > kSpinTicks) return false;
    __builtin_amdgcn_s_sleep(2);
  }
}

template <typename T>
struct OnePassArgs {
  const typename T::raw *q, *k, *v, *beta, *sel_c, *dt, *r;
  const float *alpha, *omega;
  float c;
  const float* h0;
  typename T::raw* y;
  float* h_final;
  OnePassBufs ob;
  float2* states;  // SAVE: state entering every chunk (B, NC, H, D)
  float2* gam;     // SAVE: G_k (B, NC, H)
  float4* saved;   // SAVE: per-token records (B, L, H, 2)
  float2* gsaved;  // SAVE: g_t (B, L, H)
  float2* zck;     // SAVE: z_{t-1} at t % kZck == 0 (B, NC, H, NCK, D)
  float2* cend;    // SAVE: c^ after the chunk's last step (B, NC, H, D)
  int L, H, Q, NC, NSEG, NCK, n_hg, n_chain, n_items;
  int R;           // SSD form: state rows per head (virtual heads sharing a k row); 1 otherwise
  // instrumentation (cdssm_fused_scan_fwd_stamped), else null: per (item, wave) the
  // 100 MHz real-time counter at kStampPoints points of the segment
  unsigned long long* stamps;
};

// One segment (work item): item = seg * n_chain + chain.
// Phase stamps of cdssm_fused_scan_fwd_stamped: segment entry, staging done,
// local pass done, segment map published, look-back wait done, carry folded,
// correction pass done, segment end.
constexpr int kStampPoints = 8;

// epoch: this call's, read once by the workgroup at entry; arrive: this is the
// workgroup's first segment, after whose first flag it counts itself for the
// next call's epoch (arrive_and_draw_next_epoch).
template <typename T, int D, int LPH, bool SAVE, bool WIDE>
__device__ __forceinline__ void onepass_segment(const OnePassArgs<T>& a, int item, unsigned long long epoch,
                                                bool arrive) {
  // phase stamps, read and stored only when a.stamps is set (a uniform branch)
  unsigned long long ts[kStampPoints] = {};
  const bool stamping = a.stamps != nullptr;
  auto stamp = [&](int i) {
    if (stamping) ts[i] = __builtin_amdgcn_s_memrealtime();
  };
  stamp(0);
  const typename T::raw* __restrict__ q = a.q;
  const typename T::raw* __restrict__ k = a.k;
  const typename T::raw* __restrict__ v = a.v;
  const typename T::raw* __restrict__ beta = a.beta;
  const typename T::raw* __restrict__ sel_c = a.sel_c;
  const typename T::raw* __restrict__ dt = a.dt;
  const typename T::raw* __restrict__ r = a.r;
  const float* __restrict__ alpha = a.alpha;
  const float* __restrict__ omega = a.omega;
  const float c = a.c;
  const float* __restrict__ h0 = a.h0;
  typename T::raw* __restrict__ y = a.y;
  float* __restrict__ h_final = a.h_final;
  const OnePassBufs& ob = a.ob;
  float2* __restrict__ states = a.states;
  float2* __restrict__ gam = a.gam;
  float4* __restrict__ saved = a.saved;
  float2* __restrict__ gsaved = a.gsaved;
  float2* __restrict__ zck = a.zck;
  float2* __restrict__ cend = a.cend;
  const int L = a.L, H = a.H, Q = a.Q, NC = a.NC, NSEG = a.NSEG, n_hg = a.n_hg;
  using Cfg = FusedCfg<T, D, LPH>;
  constexpr bool YM = IsSsdY<T>::value;  // SSD form: write Y (B,L,H,2,D), no q, no readout
  constexpr int DPL = Cfg::DPL, HPW = Cfg::HPW, PF = kPrefetch, W = kOnePassW;
  constexpr int SEGN = HPW * D;  // complex elements of a head group's state
  constexpr int EPT = DPL / W;   // of which each thread of the workgroup composes EPT
  static_assert(EPT * W == DPL && EPT * kWave * W == SEGN, "segment state tiles the workgroup");
  static_assert(PF == kTokRound && PF % kZck == 0, "z checkpoints fall at fixed positions of a prefetch group");
  extern __shared__ float4 smem4[];

  // wave index made wave-uniform, so the tile's fields live in scalar registers
  const int wv = __builtin_amdgcn_readfirstlane(int(threadIdx.x) / kWave);
  const int lane = int(threadIdx.x) % kWave;
  const int chain = item % a.n_chain;
  const int seg = item / a.n_chain;
  const int bi = chain / n_hg;
  const int hbase = (chain % n_hg) * HPW;
  const int n_live = min(W, NC - seg * W);  // chunks in this segment
  const bool live = wv < n_live;

  ChunkTile tc;
  tc.b = bi;
  tc.chunk = min(seg * W + wv, NC - 1);
  tc.hbase = hbase;
  tc.t0 = tc.chunk * Q;
  tc.nt = min(Q, L - tc.t0);
  tc.row0 = int64_t(bi) * L + tc.t0;

  const int hh = lane / LPH;
  const int sub = lane % LPH;
  const int h = hbase + hh;
  const bool hok = h < H;
  const int ntr = round_up(tc.nt, PF);
  const int slots = round_up(Q, kWave) * HPW;

  // LDS: per wave the A, B (float4) and M, Y (float2) token slots; then the
  // segment's chunk maps (F per wave, (G, last frame) per wave and head), the
  // state entering the segment and the look-back result
  float4* wbase = smem4 + size_t(wv) * 3 * slots;
  TileScalars s{wbase, wbase + slots, reinterpret_cast<float2*>(wbase + 2 * slots)};
  float2* s_y = s.M + slots;
  float2* Fx = reinterpret_cast<float2*>(smem4 + size_t(W) * 3 * slots);
  float4* GF = reinterpret_cast<float4*>(Fx + W * SEGN);
  float2* Sx = reinterpret_cast<float2*>(GF + W * HPW);
  int* ctrl = reinterpret_cast<int*>(Sx + SEGN);

  // the given-transition forms: R virtual heads (state rows) share each k (and q) row
  constexpr bool RW = GivenA<T>::value;
  const RowStream ks = RW ? tile_stream_rows<T>(k, tc, L, H, a.R, D, hh, sub * DPL)
                          : tile_stream<T>(k, tc, L, H, D, hh, sub * DPL);
  const RowStream qs = YM   ? RowStream{}
                       : RW ? tile_stream_rows<T>(q, tc, L, H, a.R, D, hh, sub * DPL)
                            : tile_stream<T>(q, tc, L, H, D, hh, sub * DPL);
  // SSD form: this lane's slices of its head's Y re and im rows (D apart)
  const RowStream yre = YM ? tile_stream<T>(y, tc, L, H, 2 * D, hh, sub * DPL) : RowStream{};
  const RowStream yim = YM ? tile_stream<T>(y, tc, L, H, 2 * D, hh, D + sub * DPL) : RowStream{};
  const int rowy = 2 * H * D * T::bytes;  // token stride of Y in bytes
  const int rowb = (RW ? H / a.R : H) * D * T::bytes;  // token stride of k (and q) in bytes
  const int tlast = tc.nt - 1;
  const int slim = tlast * rowb;
  RowVec<T, DPL> kb[PF], qb[PF];
  float zr[DPL], zi[DPL];
#pragma unroll
  for (int j = 0; j < DPL; ++j) zr[j] = zi[j] = 0.0f;
  ResetMask<HPW> rm{0u, 0u};

  if (live) {
    const auto pre = [&] {
#pragma unroll
      for (int i = 0; i < PF; ++i) kb[i].load(ks, min(i * rowb, slim));
    };
    rm = stage_scalars<T, HPW, true, decltype(pre), WIDE>(tc, H, ntr, v, beta, sel_c, dt, r, alpha, omega, c, s,
                                                          nullptr, 0, SAVE ? gsaved : nullptr, GF + wv * HPW, pre,
                                                          a.R);
#pragma unroll
    for (int i = 0; i < PF; ++i) kb[i].pin();
  }
  stamp(1);
  __syncthreads();

  const int64_t tile_h = (int64_t(bi) * NC + tc.chunk) * H + (hok ? h : H - 1);  // (b, chunk, h)
  float4* svp = SAVE ? saved + 2 * ((tc.row0 * H) + (hok ? h : H - 1)) : nullptr;
  const int64_t zc0 = tile_h * a.NCK * D + sub * DPL;  // this lane's z checkpoint row, slot 0

  // 1. local recurrence (k rows only); each step's update coefficient e_t is
  // kept in LDS, so the correction pass replays zh without dot products.  In
  // the last PF steps the k prefetch wraps to the first tokens; the q ring is
  // loaded after the loop (the carry hand-off hides its latency), which keeps
  // it out of the load burst at the start of the kernel.
  if (live) {
    if (SAVE && sub == 0 && hok) gam[tile_h] = make_float2(GF[wv * HPW + hh].x, GF[wv * HPW + hh].y);
    float fpr = 1.0f, fpi = 0.0f;  // frame f_{t-1} (SAVE)
    for (int tb = 0; tb < ntr; tb += PF) {
      float4 sa[PF], sb[PF];
      float2 sm[PF];
#pragma unroll
      for (int i = 0; i < PF; ++i) {
        sa[i] = s.A[(tb + i) * HPW + hh];
        sb[i] = s.B[(tb + i) * HPW + hh];
        sm[i] = s.M[(tb + i) * HPW + hh];
      }
      float2 ec[PF];
      // prefetch targets of this group: tokens tb + PF .., or the first tokens
      const int nb = (tb + PF < ntr ? tb + PF : 0) * rowb;
      const uint32_t rg = rm.group8(tb);
#pragma unroll
      for (int i = 0; i < PF; ++i) {
        const int t = tb + i;
        if (SAVE && i % kZck == 0 && hok) {
          // z_{t-1} = f_{t-1} zh_{t-1}
          float xr[DPL], xi[DPL];
#pragma unroll
          for (int j = 0; j < DPL; ++j) {
            xr[j] = fpr * zr[j] - fpi * zi[j];
            xi[j] = fpr * zi[j] + fpi * zr[j];
          }
          store_zck<T, DPL>(zck, zc0 + (t / kZck) * D, xr, xi);
        }
        float kk[DPL];
        kb[i].unpack_then_reload(kk);
        kb[i].load(ks, min(nb + i * rowb, slim));
        float pr0 = 0.0f, pi0 = 0.0f, pr1 = 0.0f, pi1 = 0.0f;
#pragma unroll
        for (int j = 0; j < DPL; j += 2) {
          pr0 = fmaf(zr[j], kk[j], pr0);
          pi0 = fmaf(zi[j], kk[j], pi0);
          pr1 = fmaf(zr[j + 1], kk[j + 1], pr1);
          pi1 = fmaf(zi[j + 1], kk[j + 1], pi1);
        }
        const float pr = group_sum<LPH>(pr0 + pr1);
        const float pi = group_sum<LPH>(pi0 + pi1);
        ec[i] = local_step<DPL>(zr, zi, kk, (rg >> i) & 1u, sm[i], sa[i].x, sa[i].y, sa[i].z, pr, pi);
        if (SAVE) {
          const float4 fb = sb[i];
          // p_t = f_{t-1} (zh_{t-1}.k_t), the first half of the token's first record
          if (sub == 0 && hok && t < tc.nt)
            reinterpret_cast<float2*>(svp + 2 * int64_t(t) * H)[0] =
                make_float2(fpr * pr - fpi * pi, fpr * pi + fpi * pr);
          fpr = fb.x;
          fpi = fb.y;
        }
      }
      if (sub == 0) {
#pragma unroll
        for (int i = 0; i < PF; ++i) s_y[(tb + i) * HPW + hh] = ec[i];
      }
    }
    if constexpr (!YM) {
#pragma unroll
      for (int i = 0; i < PF; ++i) qb[i].load(qs, min(i * rowb, slim));
    }
#pragma unroll
    for (int i = 0; i < PF; ++i) kb[i].pin();
    // chunk map F = f_end zh (zero for heads >= H: their steps are inert)
    const float4 ge = GF[wv * HPW + hh];
#pragma unroll
    for (int j = 0; j < DPL; ++j)
      Fx[wv * SEGN + hh * D + sub * DPL + j] =
          make_float2(ge.z * zr[j] - ge.w * zi[j], ge.z * zi[j] + ge.w * zr[j]);
  }
  __syncthreads();

  stamp(2);
  // 2. segment map over the live chunks; thread x composes elements
  // e = x * EPT + i of the head group's state (head e / D, element e % D)
  const int e0 = int(threadIdx.x) * EPT;
  const int ej = e0 / D;
  const int ed = e0 % D;
  const int eh = hbase + ej;
  const bool ehok = eh < H;
  float2 segF[EPT];
  float2 segG = make_float2(1.0f, 0.0f);
#pragma unroll
  for (int i = 0; i < EPT; ++i) segF[i] = make_float2(0.0f, 0.0f);
  for (int u = 0; u < n_live; ++u) {
    const float4 g = GF[u * HPW + ej];
    const float2 gu = make_float2(g.x, g.y);
#pragma unroll
    for (int i = 0; i < EPT; ++i) {
      const float2 f = Fx[u * SEGN + e0 + i];
      segF[i] = make_float2(gu.x * segF[i].x - gu.y * segF[i].y + f.x, gu.x * segF[i].y + gu.y * segF[i].x + f.y);
    }
    segG = make_float2(gu.x * segG.x - gu.y * segG.y, gu.x * segG.y + gu.y * segG.x);
  }
  const int64_t sb0 = (int64_t(bi) * NSEG + seg) * H;  // (b, seg, head 0)
  unsigned long long* flag = ob.flag + sb0 + hbase;

  // publish the segment map (every segment: later ones fold it in).  Flag
  // words are epoch << 3 | bits: kFlagMap the segment map, kFlagLeave the
  // state leaving the segment (anchor ends), kFlagGroup its group's map
  // (group ends); thread 0 stores the word with every bit published so far.
  // A group end whose group map some later segment reads flags its own map
  // together with the group map (one store acknowledgement, one flag): it
  // waits only on lower segments' maps, which never wait on it.
  if (ehok) {
#pragma unroll
    for (int i = 0; i < EPT; ++i) st_agent(ob.seg_f + (sb0 + eh) * D + ed + i, segF[i]);
    if (ed == 0) st_agent(ob.seg_g + sb0 + eh, segG);
  }
  const bool gend = seg % kFwdGroup == kFwdGroup - 1 && fwd_group_read(seg / kFwdGroup, NSEG);
  unsigned long long bits = kFlagMap;
  if (!gend) {
    wait_stores_acked();
    __syncthreads();
    if (threadIdx.x == 0) {
      __hip_atomic_store(flag, (epoch << 3) | bits, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      if (arrive) arrive_and_draw_next_epoch(ob.ctl, &g_fwd_calls, 1u);
    }
  }

  stamp(3);
  const unsigned long long* f0 = ob.flag + (int64_t(bi) * NSEG) * H + hbase;  // (b, segment 0, head group)
  const int64_t lb = int64_t(bi) * NSEG * H + eh;                            // (b, segment 0, head eh)
  const int ngrp_all = fwd_groups(NSEG);
  // a group end (the last segment of a group some later segment folds)
  // composes its group's map, oldest first: the maps its group's other
  // segments published, then its own
  if (gend) {
    const int s0 = seg - (kFwdGroup - 1);
    if (wv == 0) {
      const bool got = watch_flags(f0, H, epoch, lane < kFwdGroup - 1 ? s0 + lane : -1, kFlagMap);
      if (lane == 0) {
        ctrl[0] = got;
        if (!got) __hip_atomic_fetch_or(&g_fwd_status, kTimeoutFwd, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
    }
    __syncthreads();
    const int okg = ctrl[0];
    if (ehok) {
      float2 G[kFwdGroup - 1], F[kFwdGroup - 1][EPT];
#pragma unroll
      for (int u = 0; u < kFwdGroup - 1; ++u) {
        G[u] = ld_agent(ob.seg_g + lb + int64_t(s0 + u) * H);
#pragma unroll
        for (int i = 0; i < EPT; ++i) F[u][i] = ld_agent(ob.seg_f + (lb + int64_t(s0 + u) * H) * D + ed + i);
      }
      float2 Gg = make_float2(1.0f, 0.0f), Fg[EPT];
#pragma unroll
      for (int i = 0; i < EPT; ++i) Fg[i] = make_float2(0.0f, 0.0f);
#pragma unroll
      for (int u = 0; u < kFwdGroup; ++u) {
        const float2 gu = u < kFwdGroup - 1 ? G[u] : segG;
#pragma unroll
        for (int i = 0; i < EPT; ++i) {
          const float2 f = u < kFwdGroup - 1 ? F[u][i] : segF[i];
          Fg[i] = make_float2(gu.x * Fg[i].x - gu.y * Fg[i].y + f.x, gu.x * Fg[i].y + gu.y * Fg[i].x + f.y);
        }
        Gg = make_float2(gu.x * Gg.x - gu.y * Gg.y, gu.x * Gg.y + gu.y * Gg.x);
      }
      if (!okg) {
#pragma unroll
        for (int i = 0; i < EPT; ++i) Fg[i] = make_float2(__builtin_nanf(""), __builtin_nanf(""));
      }
      const int64_t gb = (int64_t(bi) * ngrp_all + seg / kFwdGroup) * H + eh;
#pragma unroll
      for (int i = 0; i < EPT; ++i) st_agent(ob.grp_f + gb * D + ed + i, Fg[i]);
      if (ed == 0) st_agent(ob.grp_g + gb, Gg);
    }
    wait_stores_acked();  // the segment map and the group map
    __syncthreads();
    bits |= kFlagGroup;
    if (threadIdx.x == 0) {
      __hip_atomic_store(flag, (epoch << 3) | bits, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      if (arrive) arrive_and_draw_next_epoch(ob.ctl, &g_fwd_calls, 1u);
    }
  }

  // state entering the segment, in a fixed order (so results do not depend on
  // timing): from the anchor a = kFwdAnchor * floor((seg - 1) / kFwdAnchor)
  // -- h0 for a = 0, else the published state leaving segment a - 1 -- fold
  // the maps of the segments a .. seg - 1 where there are at most kFwdDirect
  // of them, else the maps of the whole groups in [a, seg) and then those of
  // the segments of seg's own group before it; oldest first.  Wave 0 waits
  // until they are published (lanes 0 .. ngrp-1: group maps; then the segment
  // maps; lane 63: the anchor state).
  const int anc = seg == 0 ? 0 : kFwdAnchor * ((seg - 1) / kFwdAnchor);
  const bool direct = seg - anc <= kFwdDirect;
  const int g0 = anc / kFwdGroup, g1 = direct ? g0 : seg / kFwdGroup;
  const int ngrp = g1 - g0;                  // <= kFwdAnchor / kFwdGroup
  const int sg0 = g1 * kFwdGroup;            // first segment folded one by one
  const int nmap = seg - sg0;                // <= kFwdDirect
  int ok = 1;
  if (seg > 0) {
    if (wv == 0) {
      int js = -1;
      unsigned long long need = 0ull;
      if (lane < ngrp) {
        js = (g0 + lane) * kFwdGroup + kFwdGroup - 1;
        need = kFlagGroup;
      } else if (lane < ngrp + nmap) {
        js = sg0 + lane - ngrp;
        need = kFlagMap;
      } else if (lane == kWave - 1 && anc > 0) {
        js = anc - 1;
        need = kFlagLeave;
      }
      const bool got = watch_flags(f0, H, epoch, js, need);
      if (lane == 0) {
        ctrl[0] = got;
        if (!got) __hip_atomic_fetch_or(&g_fwd_status, kTimeoutFwd, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
    }
    __syncthreads();
    ok = ctrl[0];
  }
  stamp(4);
  float2 Sin[EPT];
#pragma unroll
  for (int i = 0; i < EPT; ++i) Sin[i] = make_float2(0.0f, 0.0f);
  if (ehok) {
    if (anc == 0) {
      if (h0) {
        const int64_t hb = (int64_t(bi) * H + eh) * 2 * D;
#pragma unroll
        for (int i = 0; i < EPT; ++i) Sin[i] = make_float2(h0[hb + ed + i], h0[hb + D + ed + i]);
      }
    } else {
#pragma unroll
      for (int i = 0; i < EPT; ++i) Sin[i] = ld_agent(ob.seg_s + (lb + int64_t(anc - 1) * H) * D + ed + i);
    }
    // at most max(kFwdDirect, kFwdAnchor / kFwdGroup + kFwdGroup - 1) maps, all requested at once
    constexpr int kMaps = kFwdDirect > kFwdAnchor / kFwdGroup + kFwdGroup - 1 ? kFwdDirect
                                                                            : kFwdAnchor / kFwdGroup + kFwdGroup - 1;
    float2 G[kMaps], F[kMaps][EPT];
#pragma unroll
    for (int u = 0; u < kMaps; ++u) {
      if (u < ngrp) {
        const int64_t gb = (int64_t(bi) * ngrp_all + g0 + u) * H + eh;
        G[u] = ld_agent(ob.grp_g + gb);
#pragma unroll
        for (int i = 0; i < EPT; ++i) F[u][i] = ld_agent(ob.grp_f + gb * D + ed + i);
      } else if (u < ngrp + nmap) {
        const int64_t sb = lb + int64_t(sg0 + u - ngrp) * H;
        G[u] = ld_agent(ob.seg_g + sb);
#pragma unroll
        for (int i = 0; i < EPT; ++i) F[u][i] = ld_agent(ob.seg_f + sb * D + ed + i);
      }
    }
#pragma unroll
    for (int u = 0; u < kMaps; ++u) {
      if (u < ngrp + nmap) {
#pragma unroll
        for (int i = 0; i < EPT; ++i)
          Sin[i] = make_float2(G[u].x * Sin[i].x - G[u].y * Sin[i].y + F[u][i].x,
                               G[u].x * Sin[i].y + G[u].y * Sin[i].x + F[u][i].y);
      }
    }
    if (!ok) {
#pragma unroll
      for (int i = 0; i < EPT; ++i) Sin[i] = make_float2(__builtin_nanf(""), __builtin_nanf(""));
    }
  }
  // the state leaving the segment: h_final for the last segment; published
  // for the segments that start from it (anchor ends, (seg + 1) % kFwdAnchor == 0)
  const bool anchor_end = seg + 1 < NSEG && (seg + 1) % kFwdAnchor == 0;
#pragma unroll
  for (int i = 0; i < EPT; ++i) Sx[e0 + i] = Sin[i];
  if (ehok && (anchor_end || seg + 1 == NSEG)) {
#pragma unroll
    for (int i = 0; i < EPT; ++i) {
      const float2 so = make_float2(segG.x * Sin[i].x - segG.y * Sin[i].y + segF[i].x,
                                    segG.x * Sin[i].y + segG.y * Sin[i].x + segF[i].y);
      if (anchor_end) {
        st_agent(ob.seg_s + (sb0 + eh) * D + ed + i, so);
      } else {
        const int64_t hb = (int64_t(bi) * H + eh) * 2 * D;
        h_final[hb + ed + i] = so.x;
        h_final[hb + D + ed + i] = so.y;
      }
    }
  }
  if (anchor_end) wait_stores_acked();
  __syncthreads();
  if (anchor_end && threadIdx.x == 0)
    __hip_atomic_store(flag, (epoch << 3) | bits | kFlagLeave, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);

  stamp(5);
  // 3. state entering this wave's chunk, then the correction with the readout
  if (live) {
    float cr[DPL], ci[DPL];
#pragma unroll
    for (int j = 0; j < DPL; ++j) {
      const float2 sv = Sx[hh * D + sub * DPL + j];
      cr[j] = sv.x;
      ci[j] = sv.y;
    }
    for (int u = 0; u < wv; ++u) {
      const float4 g = GF[u * HPW + hh];
#pragma unroll
      for (int j = 0; j < DPL; ++j) {
        const float2 f = Fx[u * SEGN + hh * D + sub * DPL + j];
        const float nr = g.x * cr[j] - g.y * ci[j] + f.x;
        ci[j] = g.x * ci[j] + g.y * cr[j] + f.y;
        cr[j] = nr;
      }
    }
    if (!hok) {
#pragma unroll
      for (int j = 0; j < DPL; ++j) cr[j] = ci[j] = 0.0f;
    } else if (SAVE) {
#pragma unroll
      for (int j = 0; j < DPL; ++j) states[tile_h * D + sub * DPL + j] = make_float2(cr[j], ci[j]);
    }

    // the local state is replayed from its update coefficients
#pragma unroll
    for (int j = 0; j < DPL; ++j) zr[j] = zi[j] = 0.0f;
    if constexpr (!YM) {
#pragma unroll
      for (int i = 0; i < PF; ++i) qb[i].pin();  // loaded after the local pass
    }
    for (int tb = 0; tb < ntr; tb += PF) {
      float4 sa[PF], sb[PF];
      float2 se[PF], sm[PF];
#pragma unroll
      for (int i = 0; i < PF; ++i) {
        sa[i] = s.A[(tb + i) * HPW + hh];
        sb[i] = s.B[(tb + i) * HPW + hh];
        se[i] = s_y[(tb + i) * HPW + hh];
        sm[i] = s.M[(tb + i) * HPW + hh];
      }
      float yr[PF], yi[PF];
      const int nb = (tb + PF) * rowb;
      const uint32_t rg = rm.group8(tb);
#pragma unroll
      for (int i = 0; i < PF; ++i) {
        const int t = tb + i;
        float kk[DPL], qq[DPL];
        kb[i].unpack_then_reload(kk);
        if constexpr (!YM) qb[i].unpack_then_reload(qq);
        kb[i].load(ks, min(nb + i * rowb, slim));
        if constexpr (!YM) qb[i].load(qs, min(nb + i * rowb, slim));
        // zh_t = (m_t zh_{t-1} at a frame reset) + e_t k_t
        if ((rg >> i) & 1u) zscale<DPL>(zr, zi, sm[i]);
        if constexpr (YM) {
          float pcr = 0.0f, pci = 0.0f;
#pragma unroll
          for (int j = 0; j < DPL; ++j) {
            zr[j] = fmaf(se[i].x, kk[j], zr[j]);
            zi[j] = fmaf(se[i].y, kk[j], zi[j]);
            pcr = fmaf(cr[j], kk[j], pcr);
            pci = fmaf(ci[j], kk[j], pci);
          }
          pcr = group_sum<LPH>(pcr);
          pci = group_sum<LPH>(pci);
          const float bb = sa[i].z;
          const float ecr = bb * pcr, eci = bb * pci;
          // Y_t = f_t zh_t + g_{t-1} c^_t (the correction before this token's step)
          const float4 fb = sb[i];
          float ya[DPL], yb[DPL];
#pragma unroll
          for (int j = 0; j < DPL; ++j) {
            ya[j] = fmaf(fb.x, zr[j], fmaf(-fb.y, zi[j], fmaf(fb.z, cr[j], -fb.w * ci[j])));
            yb[j] = fmaf(fb.x, zi[j], fmaf(fb.y, zr[j], fmaf(fb.z, ci[j], fb.w * cr[j])));
            cr[j] = fmaf(-ecr, kk[j], cr[j]);
            ci[j] = fmaf(-eci, kk[j], ci[j]);
          }
          if (hok && t < tc.nt) {
            store_row<T, DPL>(yre, t * rowy, ya);
            store_row<T, DPL>(yim, t * rowy, yb);
            if (SAVE && sub == 0) reinterpret_cast<float2*>(svp + 2 * int64_t(t) * H)[1] = make_float2(pcr, pci);
          }
          continue;
        }
        float pcr = 0.0f, pci = 0.0f, zqr = 0.0f, zqi = 0.0f, qcr = 0.0f, qci = 0.0f;
#pragma unroll
        for (int j = 0; j < DPL; ++j) {
          zr[j] = fmaf(se[i].x, kk[j], zr[j]);
          zi[j] = fmaf(se[i].y, kk[j], zi[j]);
          pcr = fmaf(cr[j], kk[j], pcr);
          pci = fmaf(ci[j], kk[j], pci);
          zqr = fmaf(zr[j], qq[j], zqr);
          zqi = fmaf(zi[j], qq[j], zqi);
          qcr = fmaf(cr[j], qq[j], qcr);
          qci = fmaf(ci[j], qq[j], qci);
        }
        pcr = group_sum<LPH>(pcr);
        pci = group_sum<LPH>(pci);
        const float bb = sa[i].z;
        const float ecr = bb * pcr, eci = bb * pci;
        float cnr = 0.0f, cni = 0.0f;
#pragma unroll
        for (int j = 0; j < DPL; ++j) {
          cr[j] = fmaf(-ecr, kk[j], cr[j]);
          ci[j] = fmaf(-eci, kk[j], ci[j]);
          if (SAVE) {
            cnr = fmaf(cr[j], qq[j], cnr);  // c^_{t+1}.q
            cni = fmaf(ci[j], qq[j], cni);
          }
        }
        // y_t = sel_C (f_t (zh_t.q_t) + g_{t-1} (c^_t.q_t)), reduced once
        const float4 fb = sb[i];
        const float Rr = group_sum<LPH>((fb.x * zqr - fb.y * zqi) + (fb.z * qcr - fb.w * qci));
        const float Ri = group_sum<LPH>((fb.x * zqi + fb.y * zqr) + (fb.z * qci + fb.w * qcr));
        yr[i] = sa[i].w * Rr;
        yi[i] = sa[i].w * Ri;
        if (SAVE) {
          const float cqr = group_sum<LPH>(cnr), cqi = group_sum<LPH>(cni);
          if (sub == 0 && hok && t < tc.nt) {
            float4* rec = svp + 2 * int64_t(t) * H;
            reinterpret_cast<float2*>(rec)[1] = make_float2(pcr, pci);
            rec[1] = make_float4(cqr, cqi, Rr, Ri);
          }
        }
      }
      if (!YM && sub == 0) {
#pragma unroll
        for (int i = 0; i < PF; ++i) s_y[(tb + i) * HPW + hh] = make_float2(yr[i], yi[i]);
      }
    }
    if (SAVE && hok) {
#pragma unroll
      for (int j = 0; j < DPL; ++j) cend[tile_h * D + sub * DPL + j] = make_float2(cr[j], ci[j]);
    }
  }
  __syncthreads();

  stamp(6);
  // coalesced write of y (B, L, H, 2) for the wave's tile
  if (!YM && live) {
    const int n = tc.nt * HPW;
    for (int p = lane; p < n; p += kWave) {
      const int t = p / HPW;
      const int hj = hbase + (p - t * HPW);
      if (hj < H) {
        const int64_t e = ((tc.row0 + t) * H + hj) * 2;
        const float2 yv = s_y[p];
        store_pair<T>(y + e, yv.x, yv.y);
      }
    }
  }
  if (stamping && lane == 0) {
    ts[7] = __builtin_amdgcn_s_memrealtime();
    unsigned long long* o = a.stamps + (int64_t(item) * kOnePassW + wv) * kStampPoints;
#pragma unroll
    for (int i = 0; i < kStampPoints; ++i) o[i] = ts[i];
  }
}

// PERSIST false: one workgroup per segment (grid = segments, all resident).
// PERSIST true: the grid is resident at once and takes the segments in order,
// so the lowest unfinished segment is always running and waits only on
// finished ones.
// WIDE: the wide staging loads (the caller checks H % 8 == 0 and chunk <= 64).
template <typename T, int D, int LPH, bool SAVE, bool PERSIST, bool WIDE = false>
__global__ __launch_bounds__(kWave * kOnePassW) void fused_fwd_onepass_kernel(OnePassArgs<T> a) {
  // read once: the call's last workgroup to have read it stores the next call's
  const unsigned long long epoch = load_epoch(a.ob.ctl);
  if (!PERSIST) {
    onepass_segment<T, D, LPH, SAVE, WIDE>(a, int(blockIdx.x), epoch, true);
    return;
  }
  for (int item = int(blockIdx.x); item < a.n_items; item += int(gridDim.x)) {
    onepass_segment<T, D, LPH, SAVE, WIDE>(a, item, epoch, item == int(blockIdx.x));
    __syncthreads();  // LDS is reused by the next segment
  }
}

}  // namespace cdssm

// ---------------------------------------------------------------------------
// C-ABI
// ---------------------------------------------------------------------------
namespace {

using namespace cdssm;


template <int D, int LPH>
size_t onepass_lds(int Q) {
  constexpr int HPW = kWave / LPH;
  const size_t slots = size_t(round_up(Q, kWave)) * HPW;
  return size_t(kOnePassW) * 3 * slots * sizeof(float4) + size_t(kOnePassW) * HPW * D * sizeof(float2) +
         size_t(kOnePassW) * HPW * sizeof(float4) + size_t(HPW) * D * sizeof(float2) + 16;
}

// Workgroups of the one-pass kernel resident at once (its grid: a workgroup
// may wait on any earlier segment); 0 if it cannot run.
template <typename T, int D, int LPH, bool SAVE, bool PERSIST, bool WIDE = false>
int onepass_capacity(size_t lds) {
  return cdssm_host::resident_capacity(
      reinterpret_cast<const void*>(&fused_fwd_onepass_kernel<T, D, LPH, SAVE, PERSIST, WIDE>), kWave * kOnePassW,
      lds);
}

// Where a forward call keeps its scratch: the carry arrays of the four-launch
// scan, the one-pass look-back area and, for the training forward, what the
// backward reads.  The caller's workspace holds all of them (full layout); the
// inference-only layout (no training records) packs the look-back area and
// the carry arrays alone.
struct FwdRegions {
  float2 *summ, *gam, *segA, *segX;
  float4* saved;
  float2 *gsaved, *zck, *cend, *onepass, *ycorr;
};

FwdRegions full_regions(float* ws, const FwdLayout& w) {
  FwdRegions g;
  g.summ = reinterpret_cast<float2*>(ws);
  g.gam = g.summ + w.n_summ;
  g.segA = g.gam + w.n_gam;
  g.segX = g.segA + w.n_segA;
  g.saved = reinterpret_cast<float4*>(g.segX + w.n_segX + w.n_pad);
  g.gsaved = reinterpret_cast<float2*>(ws) + w.gsaved_offset();
  g.onepass = reinterpret_cast<float2*>(ws) + w.onepass_offset();
  g.zck = reinterpret_cast<float2*>(ws) + w.zck_offset();
  g.cend = reinterpret_cast<float2*>(ws) + w.cend_offset();
  g.ycorr = reinterpret_cast<float2*>(ws) + w.ycorr_offset();
  return g;
}

int64_t infer_float2s(const FwdLayout& w) { return w.n_op + w.n_summ + w.n_gam + w.n_segA + w.n_segX; }

FwdRegions infer_regions(float2* base, const FwdLayout& w) {
  FwdRegions g;
  g.onepass = base;
  g.summ = base + w.n_op;
  g.gam = g.summ + w.n_summ;
  g.segA = g.gam + w.n_gam;
  g.segX = g.segA + w.n_segA;
  g.saved = nullptr;
  g.gsaved = g.zck = g.cend = g.ycorr = nullptr;
  return g;
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// The bf16 D = 64 forward runs 8 heads per wave (8 lanes per head).  Where the
// one-pass grid that gives (segments x batch x head groups) has fewer
// workgroups than the device has CUs, CUs sit idle for the whole call; 4 heads
// per wave (16 lanes per head) doubles the workgroups (measured on MI355X at
// config 4's B8 L2048 H16: 128 -> 256 workgroups).
bool fill_with_4_heads_per_wave(int64_t B, int64_t L, int64_t H, int64_t chunk) {
  const int64_t nc = (L + chunk - 1) / chunk, nseg = (nc + kOnePassW - 1) / kOnePassW;
  const int64_t items = nseg * B * ((H + 7) / 8);
  return H > 4 && items < cdssm_host::device_cus();
}

// Phase-stamp buffer of the running cdssm_fused_scan_fwd_stamped call on this
// host thread (instrumentation only): device memory of `len` 8-byte words.
struct StampRequest {
  unsigned long long* buf = nullptr;
  int64_t len = 0;
};
thread_local StampRequest t_stamps;

template <typename T, int D, int LPH, int LPHS>
int launch_fused_fwd(const void* q, const void* k, const void* v, const void* beta, const void* sel_c,
                     const void* dt, const void* r, const float* alpha, const float* omega, float c,
                     const float* h0, void* y, float* h_final, const FwdRegions& reg, int B, int L, int H,
                     int Q, hipStream_t stream, hipEvent_t* ev, bool save, int* path, bool cont, int R = 1) {
  using raw = typename T::raw;
  constexpr int HPW = kWave / LPH, HPWS = kWave / LPHS;
  constexpr bool kSv = true;  // the training instances (every input form has a training forward)
  const FwdLayout w = fwd_layout(B, L, H, D, Q);
  const int NC = w.NC, S = w.S;
  const int n_hg = (H + HPW - 1) / HPW, n_hgs = (H + HPWS - 1) / HPWS;
  const int64_t tiles = int64_t(B) * NC * n_hg, tiles_s = int64_t(B) * NC * n_hgs;
  const int64_t carry_threads = int64_t(B) * H * S * D;
  if (tiles_s > 0x7fffffff || carry_threads / 256 > 0x7fffffff) {
    cdssm_host::set_error("cdssm_fused_scan_fwd: grid too large (%lld tiles)", (long long)tiles);
    return CDSSM_EINVAL;
  }
  float2* summ = reg.summ;
  float2* gam = reg.gam;
  float2* segA = reg.segA;
  float2* segX = reg.segX;
  float4* saved = reg.saved;
  float2* gsaved = reg.gsaved;
  float2* zck = reg.zck;
  float2* cend = reg.cend;
  const int slots = round_up(Q, kWave) * HPW, slots_s = round_up(Q, kWave) * HPWS;

  // the SSD form has no chunked-correction variant: it takes the automatic choice there
  const int mode = IsSsdY<T>::value && cdssm_host::scan_path() == cdssm_host::kPathSweep ? cdssm_host::kPathAuto
                                                                                          : cdssm_host::scan_path();
  const bool sweep = mode == cdssm_host::kPathSweep;
  if (sweep) {
    if (!std::is_same<T, BF16>::value || save || Q % 16 != 0 || Q > 128 || !reg.ycorr) {
      cdssm_host::set_error("cdssm_fused_scan_fwd: the chunked MFMA correction serves the bf16 inference forward "
                            "with a workspace and chunk a multiple of 16 up to 128 (chunk %d)", Q);
      return CDSSM_EINVAL;
    }
  } else if (mode != cdssm_host::kPathFour) {
    const int64_t items = int64_t(w.NSEG) * B * n_hg;
    const size_t lds = onepass_lds<D, LPH>(Q);
    // one round of resident workgroups takes every segment: one-pass.  More
    // segments than that: the persistent one-pass only for inference with
    // full rounds (measured on MI355X: faster than four launches at C3,
    // slower at C2's 1.5 rounds and for the training forward's records)
    // wide staging loads (bf16 scan-level form, 8 heads per wave); the persistent
    // training forward (taken only when the one-pass path is forced) keeps the narrow ones
    constexpr bool kWideOk = std::is_same<T, BF16>::value && kWave / LPH == 8;
    // the wide loads are 16-byte vector loads of beta, sel_C, dt, r and v rows:
    // every one of those arrays must start on a 16-byte boundary
    const bool wide = kWideOk && H % 8 == 0 && Q <= kWave && cdssm_host::wide_staging() && aligned16(beta) &&
                      aligned16(sel_c) && aligned16(dt) && aligned16(r) && aligned16(v);
    const int cap1 = save   ? (wide ? onepass_capacity<T, D, LPH, kSv, false, kWideOk>(lds)
                                    : onepass_capacity<T, D, LPH, kSv, false>(lds))
                     : wide ? onepass_capacity<T, D, LPH, false, false, kWideOk>(lds)
                            : onepass_capacity<T, D, LPH, false, false>(lds);
    const int capp = save   ? onepass_capacity<T, D, LPH, kSv, true>(lds)
                     : wide ? onepass_capacity<T, D, LPH, false, true, kWideOk>(lds)
                            : onepass_capacity<T, D, LPH, false, true>(lds);
    const bool single = cap1 > 0 && items <= cap1;
    const bool forced = mode == cdssm_host::kPathOne;
    const int64_t rounds = capp > 0 ? (items + capp - 1) / capp : 0;
    const bool persist = !single && capp > 0 && items <= 0x7fffffff &&
                         (forced || (!save && items * 10 >= rounds * capp * 9));
    if (single || persist) {
      // a persistent workgroup joins the epoch count on its first item, so the
      // grid never exceeds the items (every workgroup gets at least one)
      const int grid = single ? int(items) : int(std::min<int64_t>(capp, items));
      float2* base = reg.onepass;
      const int64_t nsd = int64_t(B) * w.NSEG * H * D, nsh = int64_t(B) * w.NSEG * H;
      OnePassArgs<T> a;
      a.q = (const raw*)q;
      a.k = (const raw*)k;
      a.v = (const raw*)v;
      a.beta = (const raw*)beta;
      a.sel_c = (const raw*)sel_c;
      a.dt = (const raw*)dt;
      a.r = (const raw*)r;
      a.alpha = alpha;
      a.omega = omega;
      a.c = c;
      a.h0 = h0;
      a.y = (raw*)y;
      a.h_final = h_final;
      unsigned long long* flags = reinterpret_cast<unsigned long long*>(base + 2 * nsd + nsh);
      a.ob = OnePassBufs{base, base + nsd, base + 2 * nsd, flags, flags + nsh};
      a.ob.grp_f = reinterpret_cast<float2*>(flags + nsh + kCtlWords);
      a.ob.grp_g = a.ob.grp_f + int64_t(B) * fwd_groups(w.NSEG) * H * D;
      a.states = save ? summ : nullptr;
      a.gam = save ? gam : nullptr;
      a.saved = save ? saved : nullptr;
      a.gsaved = save ? gsaved : nullptr;
      a.zck = save ? zck : nullptr;
      a.cend = save ? cend : nullptr;
      a.L = L;
      a.H = H;
      a.Q = Q;
      a.NC = NC;
      a.NSEG = w.NSEG;
      a.NCK = w.NCK;
      a.n_hg = n_hg;
      a.n_chain = B * n_hg;
      a.n_items = int(items);
      a.R = R;
      a.stamps = nullptr;
      if (t_stamps.buf) {
        if (t_stamps.len < items * kOnePassW * kStampPoints) {
          cdssm_host::set_error("cdssm_fused_scan_fwd_stamped: %lld stamp words needed (%lld given)",
                                (long long)(items * kOnePassW * kStampPoints), (long long)t_stamps.len);
          return CDSSM_EINVAL;
        }
        a.stamps = t_stamps.buf;
      }
      if (path) *path = cdssm_host::kPathOne;
      // a continuing call runs on the epoch the previous call's last workgroup left
      if (!cont) {
        hipLaunchKernelGGL(fwd_epoch_kernel, dim3(1), dim3(64), 0, stream, a.ob.ctl);
        const int est = cdssm_host::check_launch("cdssm_fused_scan_fwd/epoch");
        if (est) return est;
      }
      if (ev)
        for (int i = 0; i < 4; ++i) (void)hipEventRecord(ev[i], stream);
      const dim3 gd = dim3(unsigned(grid)), bd = dim3(kWave * kOnePassW);
      if (save && single && wide)
        hipLaunchKernelGGL((fused_fwd_onepass_kernel<T, D, LPH, kSv, false, kWideOk>), gd, bd, lds, stream, a);
      else if (save && single)
        hipLaunchKernelGGL((fused_fwd_onepass_kernel<T, D, LPH, kSv, false>), gd, bd, lds, stream, a);
      else if (save)
        hipLaunchKernelGGL((fused_fwd_onepass_kernel<T, D, LPH, kSv, true>), gd, bd, lds, stream, a);
      else if (single && wide)
        hipLaunchKernelGGL((fused_fwd_onepass_kernel<T, D, LPH, false, false, kWideOk>), gd, bd, lds, stream, a);
      else if (wide)
        hipLaunchKernelGGL((fused_fwd_onepass_kernel<T, D, LPH, false, true, kWideOk>), gd, bd, lds, stream, a);
      else if (single)
        hipLaunchKernelGGL((fused_fwd_onepass_kernel<T, D, LPH, false, false>), gd, bd, lds, stream, a);
      else
        hipLaunchKernelGGL((fused_fwd_onepass_kernel<T, D, LPH, false, true>), gd, bd, lds, stream, a);
      const int st = cdssm_host::check_launch("cdssm_fused_scan_fwd/onepass");
      if (ev) (void)hipEventRecord(ev[4], stream);
      return st;
    }
    if (forced) {
      cdssm_host::set_error("cdssm_fused_scan_fwd: one-pass path required but not possible for this shape "
                            "(%zu bytes of LDS per workgroup)", lds);
      return CDSSM_EINVAL;
    }
  }

  if (t_stamps.buf) {
    cdssm_host::set_error("cdssm_fused_scan_fwd_stamped: the shape runs the four-launch forward, which has no phase stamps");
    return CDSSM_EINVAL;
  }
  if (path) *path = cdssm_host::kPathFour;
  if (ev) (void)hipEventRecord(ev[0], stream);
  hipLaunchKernelGGL((fused_fwd_summary_kernel<T, D, LPHS>), dim3(unsigned(tiles_s)), dim3(kWave),
                     size_t(slots_s) * (sizeof(float4) + sizeof(float2)) + HPWS * sizeof(float4), stream,
                     (const raw*)k, (const raw*)v, (const raw*)beta, (const raw*)dt, (const raw*)r, alpha,
                     omega, c, summ, gam, L, H, Q, NC, n_hgs, R);
  int st = cdssm_host::check_launch("cdssm_fused_scan_fwd/summary");
  if (st) return st;

  if (ev) (void)hipEventRecord(ev[1], stream);
  const unsigned cblocks = unsigned((carry_threads + 255) / 256);
  hipLaunchKernelGGL(fused_fwd_fold_kernel, dim3(cblocks), dim3(256), 0, stream, (const float2*)summ,
                     (const float2*)gam, segA, segX, B, NC, H, D, S);
  st = cdssm_host::check_launch("cdssm_fused_scan_fwd/fold");
  if (st) return st;
  if (ev) (void)hipEventRecord(ev[2], stream);
  hipLaunchKernelGGL(fused_fwd_replay_kernel, dim3(cblocks), dim3(256), 0, stream, summ,
                     (const float2*)gam, (const float2*)segA, (const float2*)segX, h0, h_final, B, NC,
                     H, D, S);
  st = cdssm_host::check_launch("cdssm_fused_scan_fwd/replay");
  if (st) return st;
  if (ev) (void)hipEventRecord(ev[3], stream);

  const size_t lds_main = size_t(slots) * (2 * sizeof(float4) + 2 * sizeof(float2));
  if constexpr (std::is_same<T, BF16>::value) {
    if (sweep) {
      const int n_hgw = (H + kSweepHeads - 1) / kSweepHeads;
      const unsigned waves = unsigned(int64_t(B) * NC * n_hgw);
      const uint16_t *q16 = (const uint16_t*)q, *k16 = (const uint16_t*)k;
      const uint16_t *b16 = (const uint16_t*)beta, *s16 = (const uint16_t*)sel_c;
      const uint16_t *d16 = (const uint16_t*)dt, *r16 = (const uint16_t*)r;
      const float2* st2 = (const float2*)summ;
#define CDSSM_SWEEP(NBV)                                                                                           \
  hipLaunchKernelGGL((fused_fwd_corr_sweep_kernel<D, NBV>), dim3(waves), dim3(kWave), 0, stream, q16, k16, b16, s16, \
                     d16, r16, alpha, omega, c, st2, reg.ycorr, L, H, NC, n_hgw)
      switch (Q / 16) {
        case 1: CDSSM_SWEEP(1); break;
        case 2: CDSSM_SWEEP(2); break;
        case 3: CDSSM_SWEEP(3); break;
        case 4: CDSSM_SWEEP(4); break;
        case 5: CDSSM_SWEEP(5); break;
        case 6: CDSSM_SWEEP(6); break;
        case 7: CDSSM_SWEEP(7); break;
        default: CDSSM_SWEEP(8); break;
      }
#undef CDSSM_SWEEP
      st = cdssm_host::check_launch("cdssm_fused_scan_fwd/corr_sweep");
      if (st) return st;
      hipLaunchKernelGGL((fused_fwd_main_kernel<T, D, LPH, false, false>), dim3(unsigned(tiles)), dim3(kWave),
                         lds_main, stream, (const raw*)q, (const raw*)k, (const raw*)v, (const raw*)beta,
                         (const raw*)sel_c, (const raw*)dt, (const raw*)r, alpha, omega, c, (const float2*)summ,
                         (raw*)y, nullptr, nullptr, nullptr, nullptr, L, H, Q, NC, w.NCK, n_hg,
                         (const float2*)reg.ycorr);
      st = cdssm_host::check_launch("cdssm_fused_scan_fwd/main_local");
      if (ev) (void)hipEventRecord(ev[4], stream);
      return st;
    }
  }
  if (save)
    hipLaunchKernelGGL((fused_fwd_main_kernel<T, D, LPH, kSv>), dim3(unsigned(tiles)), dim3(kWave), lds_main,
                       stream, (const raw*)q, (const raw*)k, (const raw*)v, (const raw*)beta, (const raw*)sel_c,
                       (const raw*)dt, (const raw*)r, alpha, omega, c, (const float2*)summ, (raw*)y, saved,
                       gsaved, zck, cend, L, H, Q, NC, w.NCK, n_hg, nullptr, R);
  else
    hipLaunchKernelGGL((fused_fwd_main_kernel<T, D, LPH, false>), dim3(unsigned(tiles)), dim3(kWave), lds_main,
                       stream, (const raw*)q, (const raw*)k, (const raw*)v, (const raw*)beta, (const raw*)sel_c,
                       (const raw*)dt, (const raw*)r, alpha, omega, c, (const float2*)summ, (raw*)y, nullptr,
                       nullptr, nullptr, nullptr, L, H, Q, NC, w.NCK, n_hg, nullptr, R);
  st = cdssm_host::check_launch("cdssm_fused_scan_fwd/main");
  if (ev) (void)hipEventRecord(ev[4], stream);
  return st;
}

}  // namespace

// ---------------------------------------------------------------------------
// Static scratch of cdssm_fused_scan_fwd_noalloc: the inference forward's
// look-back area and carry arrays, for callers that cannot allocate device
// memory.  One copy per GPU, held until the process ends; every no-alloc call
// on a GPU uses that GPU's copy, so such calls must not overlap on one GPU.
// Nothing in it needs clearing between calls: the carry arrays are written
// before they are read in each call, and the look-back flags only count when
// they carry the running call's epoch (fresh per call, written by the epoch
// kernel into the area's control block).
// ---------------------------------------------------------------------------
constexpr size_t kScratchBytes = size_t(32) << 20;  // 32 MiB
static __device__ __align__(256) unsigned char scratch[kScratchBytes];

namespace {
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
float2* g_scratch_ptr[kMaxDevices];  // device address of `scratch` on each GPU, 0 until looked up

int scratch_regions(const FwdLayout& w, FwdRegions* reg) {
  const int64_t need = infer_float2s(w) * int64_t(sizeof(float2));
  if (need > int64_t(kScratchBytes)) {
    cdssm_host::set_error("cdssm_fused_scan_fwd_noalloc: this shape needs %lld bytes of scratch, more than the "
                          "%zu bytes of the library's static scratch; use cdssm_fused_scan_fwd with a workspace",
                          (long long)need, kScratchBytes);
    return CDSSM_EINVAL;
  }
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) {
    (void)hipGetLastError();
    cdssm_host::set_error("cdssm_fused_scan_fwd_noalloc: no usable current device (%d)", dev);
    return CDSSM_EHIP;
  }
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    // the array's address on this device (the host-side name is only a stand-in)
    void* ptr = nullptr;
    const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !ptr) {
      (void)hipGetLastError();
      cdssm_host::set_error("cdssm_fused_scan_fwd_noalloc: hipGetSymbolAddress(scratch) failed on device %d: %s",
                            dev, hipGetErrorString(e));
      return CDSSM_EHIP;
    }
    g_scratch_ptr[dev] = static_cast<float2*>(ptr);
  }
  *reg = infer_regions(g_scratch_ptr[dev], w);
  return CDSSM_OK;
}
}  // namespace

int cdssm_host::fwd_lookback_status(bool clear, unsigned* out) {
  unsigned v = 0;
  if (hipMemcpyFromSymbol(&v, HIP_SYMBOL(cdssm::g_fwd_status), sizeof(v), 0, hipMemcpyDeviceToHost) != hipSuccess) {
    cdssm_host::set_error("cdssm_lookback_status: reading the forward status word failed: %s",
                          hipGetErrorString(hipGetLastError()));
    return CDSSM_EHIP;
  }
  if (clear && v) {
    const unsigned zero = 0;
    if (hipMemcpyToSymbol(HIP_SYMBOL(cdssm::g_fwd_status), &zero, sizeof(zero), 0, hipMemcpyHostToDevice) !=
        hipSuccess) {
      cdssm_host::set_error("cdssm_lookback_status: clearing the forward status word failed: %s",
                            hipGetErrorString(hipGetLastError()));
      return CDSSM_EHIP;
    }
  }
  *out = v;
  return CDSSM_OK;
}

extern "C" int64_t cdssm_fused_scan_workspace_bytes(int64_t B, int64_t L, int64_t H, int64_t D,
                                                    int64_t N, int64_t chunk) {
  if (B <= 0 || L <= 0 || H <= 0 || D <= 0 || chunk <= 0 || N < 2 || N > 32 || N % 2 != 0) return -1;
  // N > 2 (the gate-level form): the N / 2 state rows of a head are scanned as virtual heads
  return fwd_layout(B, L, H * (N / 2), D, chunk).total() * int64_t(sizeof(float2));
}

// The SSD form's forward workspace: its N / 2 state rows per head are scanned as
// virtual heads, so the layout is the fused scan's with H N / 2 heads.
extern "C" int64_t cdssm_ssd_scan_workspace_bytes(int64_t B, int64_t L, int64_t H, int64_t D, int64_t N,
                                                  int64_t chunk) {
  if (N < 2 || N > 32 || N % 2 != 0) return -1;
  return cdssm_fused_scan_workspace_bytes(B, L, H * (N / 2), D, 2, chunk);
}

namespace {
// Scratch of a forward call: the caller's workspace (full layout), or, with
// workspace NULL, the library's static per-device scratch (inference only).
int scratch_regions(const FwdLayout& w, FwdRegions* reg);

int fused_fwd_entry(int dtype, const void* q, const void* k, const void* v, const void* beta,
                    const void* sel_c, const void* dt, const void* r, const float* alpha,
                    const float* omega, float c, const float* h0, void* y, float* h_final,
                    float* workspace, int64_t B, int64_t L, int64_t H, int64_t D, int64_t N,
                    int64_t chunk, hipStream_t stream, hipEvent_t* ev, bool save, int* path = nullptr,
                    bool abar = false, bool no_alloc = false, bool ssd = false, bool cont = false) {
  const char* op = ssd ? "cdssm_ssd_scan_fwd"
                       : (no_alloc ? "cdssm_fused_scan_fwd_noalloc"
                                   : (abar ? "cdssm_fused_scan_fwd_abar" : "cdssm_fused_scan_fwd"));
  if (dtype != 0 && dtype != 1) {
    cdssm_host::set_error("%s: dtype must be 0 (fp32) or 1 (bf16), got %d", op, dtype);
    return CDSSM_EINVAL;
  }
  if (B <= 0 || L <= 0 || H <= 0) {
    cdssm_host::set_error("%s: B, L, H must be positive (B=%lld L=%lld H=%lld)", op, (long long)B,
                          (long long)L, (long long)H);
    return CDSSM_EINVAL;
  }
  // SSD and gate-level forms: the N / 2 complex state rows of a head run as R
  // virtual heads sharing the head's k, beta (and q, sel_C); each has its own
  // a_t, values (and vp_t, readout pair), in the (B,L,H,N) layouts as given
  int64_t R = 1;
  if ((ssd || abar) && N > 2 && N % 2 == 0 && N <= 32) {
    R = N / 2;
    H *= R;
    N = 2;
  }
  if (N != 2) {
    cdssm_host::set_error(ssd || abar ? "%s: state_dim N must be even, 2 <= N <= 32, got %lld"
                                      : "%s: the fused scan supports state_dim N = 2, got %lld", op, (long long)N);
    return CDSSM_EINVAL;
  }
  if (D != 64 && D != 128) {
    cdssm_host::set_error("%s: head_dim D must be 64 or 128, got %lld", op, (long long)D);
    return CDSSM_EINVAL;
  }
  if (chunk < 1 || chunk > 128) {
    cdssm_host::set_error("%s: chunk size must be in [1, 128], got %lld", op, (long long)chunk);
    return CDSSM_EINVAL;
  }
  if (B * H > 0x7fffffffLL || L > 0x7fffffffLL || B * L * H * D > (int64_t(1) << 46)) {
    cdssm_host::set_error("%s: problem too large", op);
    return CDSSM_EINVAL;
  }
  // q/k rows (Y rows: 2 D per head) of a chunk tile are addressed by 32-bit byte offsets
  if ((chunk + 16) * H * D * 4 * (ssd ? 2 : 1) > 0x7fffffffLL) {
    cdssm_host::set_error("%s: H * D too large for 32-bit row offsets (H=%lld D=%lld)", op, (long long)H,
                          (long long)D);
    return CDSSM_EINVAL;
  }
  if ((!ssd && (!q || !sel_c || !r || (!abar && (!alpha || !omega)))) || !k || !v || !beta || !dt || !y ||
      !h_final || (!workspace && !no_alloc)) {
    cdssm_host::set_error("%s: null pointer argument", op);
    return CDSSM_EINVAL;
  }
  if ((!ssd && !aligned16(q)) || !aligned16(k)) {
    cdssm_host::set_error("%s: q and k must be 16-byte aligned", op);
    return CDSSM_EINVAL;
  }
  if (ssd && !aligned16(y)) {
    cdssm_host::set_error("%s: Y must be 16-byte aligned", op);
    return CDSSM_EINVAL;
  }
  if (reinterpret_cast<uintptr_t>(y) % (dtype == 1 ? 4 : 8) != 0) {
    cdssm_host::set_error("%s: y must be aligned to its (re, im) pair (%d bytes)", op, dtype == 1 ? 4 : 8);
    return CDSSM_EINVAL;
  }
  const FwdLayout lay = fwd_layout(B, L, H, D, chunk);
  FwdRegions reg;
  if (no_alloc) {
    const int st = scratch_regions(lay, &reg);
    if (st) return st;
  } else {
    reg = full_regions(workspace, lay);
  }
  const int b = int(B), l = int(L), hh = int(H), qc = int(chunk);
#define CDSSM_FWD_ARGS q, k, v, beta, sel_c, dt, r, alpha, omega, c, h0, y, h_final, reg, b, l, hh, qc, stream, \
                       ev, save, path, cont
  if (ssd) {
    const int rr = int(R);
    if (dtype == 1) {
      if (D == 64)
        return launch_fused_fwd<SsdY<BF16>, 64, CDSSM_FWD_LPH_BF16_D64, CDSSM_FWD_LPHS_BF16_D64>(CDSSM_FWD_ARGS, rr);
      return launch_fused_fwd<SsdY<BF16>, 128, 16, CDSSM_FWD_LPHS_BF16_D128>(CDSSM_FWD_ARGS, rr);
    }
    if (D == 64) return launch_fused_fwd<SsdY<F32>, 64, 16, 16>(CDSSM_FWD_ARGS, rr);
    return launch_fused_fwd<SsdY<F32>, 128, 32, 32>(CDSSM_FWD_ARGS, rr);
  }
  if (abar) {
    const int rr = int(R);
    if (dtype == 1) {
      if (D == 64 && fill_with_4_heads_per_wave(B, L, H, chunk))
        return launch_fused_fwd<ABar<BF16>, 64, 16, CDSSM_FWD_LPHS_BF16_D64>(CDSSM_FWD_ARGS, rr);
      if (D == 64)
        return launch_fused_fwd<ABar<BF16>, 64, CDSSM_FWD_LPH_BF16_D64, CDSSM_FWD_LPHS_BF16_D64>(CDSSM_FWD_ARGS,
                                                                                               rr);
      return launch_fused_fwd<ABar<BF16>, 128, 16, CDSSM_FWD_LPHS_BF16_D128>(CDSSM_FWD_ARGS, rr);
    }
    if (D == 64) return launch_fused_fwd<ABar<F32>, 64, 16, 16>(CDSSM_FWD_ARGS, rr);
    return launch_fused_fwd<ABar<F32>, 128, 32, 32>(CDSSM_FWD_ARGS, rr);
  }
  if (dtype == 1) {
    // the training forward takes the same layout as the inference forward of the
    // shape (its workspace does not depend on it), so the two stay bit-identical
    if (D == 64 && fill_with_4_heads_per_wave(B, L, H, chunk))
      return launch_fused_fwd<BF16, 64, 16, CDSSM_FWD_LPHS_BF16_D64>(CDSSM_FWD_ARGS);
    if (D == 64)
      return launch_fused_fwd<BF16, 64, CDSSM_FWD_LPH_BF16_D64, CDSSM_FWD_LPHS_BF16_D64>(CDSSM_FWD_ARGS);
    return launch_fused_fwd<BF16, 128, 16, CDSSM_FWD_LPHS_BF16_D128>(CDSSM_FWD_ARGS);
  }
  if (D == 64) return launch_fused_fwd<F32, 64, 16, 16>(CDSSM_FWD_ARGS);
  return launch_fused_fwd<F32, 128, 32, 32>(CDSSM_FWD_ARGS);
#undef CDSSM_FWD_ARGS
}
}  // namespace

extern "C" int cdssm_fused_scan_fwd(int dtype, const void* q, const void* k, const void* v,
                                    const void* beta, const void* sel_c, const void* dt,
                                    const void* r, const float* alpha, const float* omega, float c,
                                    const float* h0, void* y, float* h_final, float* workspace,
                                    int64_t B, int64_t L, int64_t H, int64_t D, int64_t N,
                                    int64_t chunk, hipStream_t stream) {
  return fused_fwd_entry(dtype, q, k, v, beta, sel_c, dt, r, alpha, omega, c, h0, y, h_final, workspace,
                         B, L, H, D, N, chunk, stream, nullptr, false);
}

// cdssm_fused_scan_fwd for a workspace whose previous use was a forward call
// (this entry, cdssm_fused_scan_fwd, or their training forms) of the same
// shape, completed or ordered before this one on the stream, with the
// workspace untouched since: the one-pass kernel reuses the look-back epoch
// that call's last workgroup left in the workspace instead of a separate
// launch drawing one.
extern "C" int cdssm_fused_scan_fwd_continue(int dtype, const void* q, const void* k, const void* v,
                                             const void* beta, const void* sel_c, const void* dt,
                                             const void* r, const float* alpha, const float* omega, float c,
                                             const float* h0, void* y, float* h_final, float* workspace,
                                             int64_t B, int64_t L, int64_t H, int64_t D, int64_t N,
                                             int64_t chunk, hipStream_t stream) {
  return fused_fwd_entry(dtype, q, k, v, beta, sel_c, dt, r, alpha, omega, c, h0, y, h_final, workspace,
                         B, L, H, D, N, chunk, stream, nullptr, false, nullptr, false, false, false, true);
}

// The inference forward with the library's static scratch in place of a
// workspace: no allocation, no workspace argument (see `scratch` above).
extern "C" int cdssm_fused_scan_fwd_noalloc(int dtype, const void* q, const void* k, const void* v,
                                            const void* beta, const void* sel_c, const void* dt,
                                            const void* r, const float* alpha, const float* omega, float c,
                                            const float* h0, void* y, float* h_final, int64_t B, int64_t L,
                                            int64_t H, int64_t D, int64_t N, int64_t chunk,
                                            hipStream_t stream) {
  return fused_fwd_entry(dtype, q, k, v, beta, sel_c, dt, r, alpha, omega, c, h0, y, h_final, nullptr, B, L, H,
                         D, N, chunk, stream, nullptr, false, nullptr, false, true);
}

// The fused forward on gate-level inputs: a_t (B,L,H,2) and vp_t (B,L,H,1) of
// `dtype` (DynamicsFusedFn's A_bar and vp_scale) in place of dt, r, alpha,
// omega and c.
extern "C" int cdssm_fused_scan_fwd_abar(int dtype, const void* q, const void* k, const void* v,
                                         const void* beta, const void* sel_c, const void* a_bar,
                                         const void* vp, const float* h0, void* y, float* h_final,
                                         float* workspace, int64_t B, int64_t L, int64_t H, int64_t D,
                                         int64_t N, int64_t chunk, hipStream_t stream) {
  return fused_fwd_entry(dtype, q, k, v, beta, sel_c, a_bar, vp, nullptr, nullptr, 0.0f, h0, y, h_final, workspace,
                         B, L, H, D, N, chunk, stream, nullptr, false, nullptr, true);
}

// Training forward of the gate-level form: cdssm_fused_scan_fwd_abar that also
// stores in the workspace what cdssm_fused_scan_bwd_abar reads (the records of
// cdssm_fused_scan_fwd_train).
extern "C" int cdssm_fused_scan_fwd_abar_train(int dtype, const void* q, const void* k, const void* v,
                                               const void* beta, const void* sel_c, const void* a_bar,
                                               const void* vp, const float* h0, void* y, float* h_final,
                                               float* workspace, int64_t B, int64_t L, int64_t H, int64_t D,
                                               int64_t N, int64_t chunk, hipStream_t stream) {
  return fused_fwd_entry(dtype, q, k, v, beta, sel_c, a_bar, vp, nullptr, nullptr, 0.0f, h0, y, h_final, workspace,
                         B, L, H, D, N, chunk, stream, nullptr, true, nullptr, true);
}

// The SSDChunkwiseScan interface (ssd.py:39-111) on the fused kernels: A_bar
// (B,L,H,2), K (B,L,H,D), V (B,L,H,2), already VP-scaled, and beta (B,L,H) of
// `dtype` -> Y (B,L,H,2,D) of `dtype`, the R-mode local state + correction of
// every token; h_final (B,H,2,D) fp32 receives the carry after the last token
// (the sequence starts from a zero state).  train != 0 also writes, into the
// workspace, what cdssm_ssd_scan_bwd reads.
extern "C" int cdssm_ssd_scan_fwd(int dtype, const void* a_bar, const void* k, const void* v, const void* beta,
                                  void* Y, float* h_final, float* workspace, int64_t B, int64_t L, int64_t H,
                                  int64_t D, int64_t N, int64_t chunk, int train, hipStream_t stream) {
  return fused_fwd_entry(dtype, nullptr, k, v, beta, nullptr, a_bar, nullptr, nullptr, nullptr, 0.0f, nullptr, Y,
                         h_final, workspace, B, L, H, D, N, chunk, stream, nullptr, train != 0, nullptr, false, false,
                         true);
}

extern "C" int cdssm_fused_scan_fwd_train(int dtype, const void* q, const void* k, const void* v,
                                          const void* beta, const void* sel_c, const void* dt,
                                          const void* r, const float* alpha, const float* omega, float c,
                                          const float* h0, void* y, float* h_final, float* workspace,
                                          int64_t B, int64_t L, int64_t H, int64_t D, int64_t N,
                                          int64_t chunk, hipStream_t stream) {
  return fused_fwd_entry(dtype, q, k, v, beta, sel_c, dt, r, alpha, omega, c, h0, y, h_final, workspace,
                         B, L, H, D, N, chunk, stream, nullptr, true);
}

// cdssm_fused_scan_fwd_train on the same terms as cdssm_fused_scan_fwd_continue.
extern "C" int cdssm_fused_scan_fwd_train_continue(int dtype, const void* q, const void* k, const void* v,
                                                   const void* beta, const void* sel_c, const void* dt,
                                                   const void* r, const float* alpha, const float* omega,
                                                   float c, const float* h0, void* y, float* h_final,
                                                   float* workspace, int64_t B, int64_t L, int64_t H, int64_t D,
                                                   int64_t N, int64_t chunk, hipStream_t stream) {
  return fused_fwd_entry(dtype, q, k, v, beta, sel_c, dt, r, alpha, omega, c, h0, y, h_final, workspace,
                         B, L, H, D, N, chunk, stream, nullptr, true, nullptr, false, false, false, true);
}

// Instrumentation (no reference counterpart): cdssm_fused_scan_fwd, recording
// for every wave of the one-pass kernel the 100 MHz real-time counter at
// kStampPoints points of its segment into `stamps` (device memory, stamps_len
// 8-byte words, word ((segment item * 4 + wave) * 8 + point)); -1 if the
// buffer is too small or the shape takes the four-launch forward.
extern "C" int cdssm_fused_scan_fwd_stamped(int dtype, const void* q, const void* k, const void* v,
                                            const void* beta, const void* sel_c, const void* dt, const void* r,
                                            const float* alpha, const float* omega, float c, const float* h0,
                                            void* y, float* h_final, float* workspace, int64_t B, int64_t L,
                                            int64_t H, int64_t D, int64_t N, int64_t chunk,
                                            unsigned long long* stamps, int64_t stamps_len, hipStream_t stream) {
  if (!stamps || stamps_len <= 0) {
    cdssm_host::set_error("cdssm_fused_scan_fwd_stamped: a stamp buffer is required");
    return CDSSM_EINVAL;
  }
  t_stamps = StampRequest{stamps, stamps_len};
  const int st = fused_fwd_entry(dtype, q, k, v, beta, sel_c, dt, r, alpha, omega, c, h0, y, h_final, workspace,
                                 B, L, H, D, N, chunk, stream, nullptr, false);
  t_stamps = StampRequest{};
  return st;
}

extern "C" int cdssm_fused_scan_fwd_profile(int dtype, const void* q, const void* k, const void* v,
                                            const void* beta, const void* sel_c, const void* dt,
                                            const void* r, const float* alpha, const float* omega,
                                            float c, const float* h0, void* y, float* h_final,
                                            float* workspace, int64_t B, int64_t L, int64_t H,
                                            int64_t D, int64_t N, int64_t chunk, hipStream_t stream,
                                            int train, int iters, float* phase_ms) {
  if (iters < 1 || !phase_ms) {
    cdssm_host::set_error("cdssm_fused_scan_fwd_profile: iters >= 1 and phase_ms required");
    return CDSSM_EINVAL;
  }
  hipEvent_t ev[5];
  for (int i = 0; i < 5; ++i)
    if (hipEventCreate(&ev[i]) != hipSuccess) {
      for (int j = 0; j < i; ++j) (void)hipEventDestroy(ev[j]);
      cdssm_host::set_error("cdssm_fused_scan_fwd_profile: hipEventCreate failed");
      return CDSSM_EHIP;
    }
  for (int p = 0; p < 4; ++p) phase_ms[p] = 0.0f;
  int st = CDSSM_OK;
  for (int it = 0; it < iters && st == CDSSM_OK; ++it) {
    int path = cdssm_host::kPathFour;
    st = fused_fwd_entry(dtype, q, k, v, beta, sel_c, dt, r, alpha, omega, c, h0, y, h_final, workspace, B,
                         L, H, D, N, chunk, stream, ev, train != 0, &path);
    if (st != CDSSM_OK) break;
    if (hipEventSynchronize(ev[4]) != hipSuccess) {
      cdssm_host::set_error("cdssm_fused_scan_fwd_profile: hipEventSynchronize failed");
      st = CDSSM_EHIP;
      break;
    }
    // a one-pass call is one launch: reported as the main pass, 0 for the others
    for (int p = path == cdssm_host::kPathOne ? 3 : 0; p < 4; ++p) {
      float ms = 0.0f;
      (void)hipEventElapsedTime(&ms, ev[p], ev[p + 1]);
      phase_ms[p] += ms / float(iters);
    }
  }
  for (int i = 0; i < 5; ++i) (void)hipEventDestroy(ev[i]);
  return st;
}

