// Fused backward of the CD-SSM chunkwise delta-rule scan (R-mode), with the
// reference ops.py gradient semantics.
//
// Forward (per (b, h), chunk k, local step t; see fused_scan_fwd.hip):
//   z_t = a_t (z_{t-1} - beta_t p_t k_t) + w_t k_t,  p_t = z_{t-1}.k_t,  z_{-1} = 0
//   c^_{t+1} = c^_t - beta_t pc_t k_t,  pc_t = c^_t.k_t,  c^_0 = s_k
//   Y_t = z_t + g_{t-1} c^_t,  y_t = sel_t (Y_t . q_t),  g_t = prod_{u<=t} a_u
//   s_{k+1} = G_k s_k + z_{n-1},  G_k = g_{n-1}
//
// Gradient semantics (what ops.py's autograd produces, ops.py:100-195):
//   * readout, intra-chunk and inter-chunk branches: exact reverse mode
//     (intra_chunk_scan.cu:215-553, inter_chunk_scan.cu:89-196);
//   * correction branch: exact_correction.cu:213-382 adds grad_corrections[t]
//     to the running adjoint BEFORE stepping back through step t, i.e. it is the
//     exact gradient of sum_t <G_t, c_{t+1}> (the state AFTER step t), where
//     G_t = dL/dY_t = sel_t dy_t q_t.  In the decay-free frame this is the loss
//     sum_t <G_t, g_t c^_{t+1}>; its adjoint lambda of c^ runs backward as
//     lambda_{t+1} += conj(g_t) G_t,  lambda_t = P_t lambda_{t+1}, and the
//     rotation products receive delta g_t = sum_d G_t[d] conj(c^_{t+1}[d]).
//   * scan-level dynamics (a_t, vp_t from dt, r, alpha, omega): exact chain
//     rule of the forward formula, clamps included.
//
// Launches (all on the caller's stream):
//   B1 corr:    per chunk, reverse lambda pass only -> lambda_0 = d s_k (corr)
//   B2 rfold/rreplay: reverse carry over chunks,
//               d s_k = conj(G_k) d s_{k+1} + lambda_0^(k),  d s_NC = d h_final,
//               storing d s_{k+1} per chunk and d h0 = d s_0
//   B3 main:    per chunk: segment-wise reverse of both branches from the
//               training forward's z checkpoints and records, emitting dq,
//               dk, dv, dbeta, dsel_C, ddt, dr and per-chunk d alpha / d omega
//   B4 heads:   deterministic sum of the per-chunk d alpha / d omega.
//
// Work layout of B1 and B3: one wave64 per (b, chunk, group of HPW heads);
// each head is owned by LPH = D/4 consecutive lanes, each lane holding 4
// consecutive state elements (HPW = 4 for D = 64, 2 for D = 128); dot
// products reduce over the head's lanes with DPP and row swaps.  Per-token
// scalars are staged in LDS, one slot per (token, head), by lanes that each
// own a block of tokens of one head.
#include "common.hpp"

namespace cdssm {

constexpr int kBwdSeg = 16;   // chunks per reverse-carry segment
// lanes per head and state elements per lane (LPH * DPL = D)
#ifndef CDSSM_BWD_LPH_D128
#define CDSSM_BWD_LPH_D128 32
#endif
template <int D>
struct BwdCfg {
  static constexpr int LPH = D == 64 ? 16 : CDSSM_BWD_LPH_D128;
  static constexpr int HPW = kWave / LPH;
  static constexpr int DPL = D / LPH;
};
// the correction-adjoint pass is light on registers and latency-bound: at
// D = 128, 32 lanes per head (two heads per wave, twice the waves) measured
// 4% faster on MI355X than 16 at C2; D = 64 keeps 16 (the one-launch
// reverse carry needs HPW * D >= 256)
#ifndef CDSSM_BWD_CORR_LPH
#define CDSSM_BWD_CORR_LPH 16
#endif
#ifndef CDSSM_BWD_CORR_LPH_D128
#define CDSSM_BWD_CORR_LPH_D128 32
#endif
template <int D>
struct BwdCorrCfg {
  static constexpr int LPH = D == 128 ? CDSSM_BWD_CORR_LPH_D128 : CDSSM_BWD_CORR_LPH;
  static constexpr int HPW = kWave / LPH;
  static constexpr int DPL = D / LPH;
};
constexpr int kBwdCK = 8;     // z checkpoint interval (the training forward writes them)
constexpr int kBwdPF = 8;     // row prefetch depth (main pass)
#ifndef CDSSM_BWD_CORR_PF
#define CDSSM_BWD_CORR_PF 8
#endif
constexpr int kBwdCorrPF = CDSSM_BWD_CORR_PF;  // row prefetch depth (correction-adjoint pass)

// Per-token scalars of a backward tile in LDS, slot p = t*HPW + j:
//   S0 = (a_re, a_im, e_re, e_im)       transition and the coefficient of k_t in
//                                       z_t = a_t z_{t-1} + e_t k_t: e = w - beta a p,
//                                       w = beta vp v, p = z_{t-1}.k_t (recorded)
//   S1 = (beta, f_re, f_im, 0)          f = sel_C dy
//   S2 = (h_re, h_im, gp_re, gp_im)     h = conj(g_t) f, gp = g_{t-1}
// SSD form (a_t read from A_bar, vp = 1, the adjoint input a whole row dY_t):
// f = 0 and S2 = (g_t, g_{t-1}).
struct BwdScalars {
  float4 *S0, *S1, *S2;
};

// Rescaled frames of the main pass (readout form).  In a segment of CK tokens
// from tb, with the segment's own rotation products G_i = prod_{u=tb}^{tb+i-1}
// a_u (G_0 = 1), token t = tb + i:
//   z~_i  = z_{t-1} / G_i:         z~_{i+1} = z~_i + (e_t / G_{i+1}) k_t
//   mu^_t = conj(G_{i+1}) mu_t:    mu^ += (conj(G_{i+1}) f_t) q_t, then
//                                  mu^ -= beta (mu^.k) k_t
// (mu_t the adjoint of z_t), so neither recurrence multiplies by a_t per state
// element.  The products the step needs keep their form with per-token
// coefficients: Re(mu conj(e)) = Re(mu^ conj(e / G_{i+1})), the z_{t-1} term of
// dk is Re(z~_i conj(beta mu^.k)), Re(z_t conj(f)) = Re(z~_{i+1} conj(conj(G_{i+1})
// f)); what leaves the step is mu^.k = conj(G_{i+1}) (mu.k) and
// mu^ conj(z~_i) = conj(a_t) mu conj(z_{t-1}), converted back per token after
// the pass.  mu^ enters a segment as conj(G_CK) mu and leaves it as mu_{tb-1}
// (G_0 = 1).  The frames stay within 2^-60 .. 2^60 of the true scale when every
// |G_i|^2 lies in [2^-120, 2^120]; a wave with any segment outside that runs
// the unscaled step instead.
// Slots (RS staging): S0 = (e / G_{i+1}, conj(G_{i+1}) f), S1 = (beta, pc, Re
// G_CK for even t or Im G_CK for odd t), S2 = (h, conj(g_{t-1}) f), P = (p, a),
// G = (delta g, g_{t-1}); d sel_C is stored by the staging itself.
constexpr float kRsLo = 0x1p-120f, kRsHi = 0x1p120f;

// Stage the per-token scalars of a tile, every slot of the slabs covering
// [0, ntr).  Lane = (head j, block of TPB tokens); each lane loads and computes
// its own tokens, runs g = prod a sequentially over them and joins the blocks
// of its head with log2(NB) shuffle steps.  Slots past the last token and
// heads >= H hold inert steps (a = 1, w = 0, beta = 0, f = 0).  With RS each
// slab takes the rescaled-frame layout described above while every segment of
// the wave's heads so far is in range (a wave vote per slab, before its slots
// are written), else the unscaled layout; the return value is kStageRs when
// every slab is rescaled, kStagePlain when none is, and kStageMixed when a
// later slab fell back after an earlier one was written rescaled (the caller
// then stages again without RS).  Without RS it is kStagePlain.
constexpr int kStagePlain = 0, kStageMixed = 1, kStageRs = 2;
template <typename T, int HPW, bool WITH_W, bool RS = false>
__device__ __forceinline__ int stage_bwd(const ChunkTile& tc, int H, int ntr,
                                          const typename T::raw* __restrict__ v,
                                          const typename T::raw* __restrict__ beta,
                                          const typename T::raw* __restrict__ sel_c,
                                          const typename T::raw* __restrict__ dt,
                                          const typename T::raw* __restrict__ r,
                                          const typename T::raw* __restrict__ dy, float al, float om,
                                          float c, const BwdScalars& s,
                                          const float4* __restrict__ saved = nullptr,
                                          float4* __restrict__ sP = nullptr, float4* __restrict__ sG = nullptr,
                                          int R = 1, typename T::raw* __restrict__ dsel = nullptr,
                                          float* __restrict__ dsp = nullptr) {
  constexpr int NB = kWave / HPW, TPB = HPW;
  const int lane = int(threadIdx.x) % kWave;  // lane in the wave (one-launch workgroups have several)
  const int j = lane / NB;
  const int blk = lane % NB;
  const int hj = tc.hbase + j;
  const bool hok = hj < H;
  const int hl = hok ? hj : H - 1;
  constexpr bool YM = IsSsdY<T>::value;
  constexpr bool GA = GivenA<T>::value;  // a_t read from A_bar (dt's place); ABar: vp from r's place
  constexpr bool kAbar = IsABar<T>::value;
  static_assert(!RS || (WITH_W && !YM), "rescaled frames: the readout form's main pass");
  static_assert(kBwdCK % TPB == 0, "a segment is a whole number of blocks");
  constexpr int SB = kBwdCK / TPB;  // blocks per segment
  bool rsok = RS, wrote_rs = false;
  float cgr = 1.0f, cgi = 0.0f;  // g carried in from earlier slabs
  // a slab's inputs and the training forward's records (p, pc), (c^_{t+1}.q, Y.q);
  // the next slab's are requested before this one is worked on
  struct SlabIn {
    float bb[TPB], dd[TPB], rr[TPB], vq[TPB], v0[TPB], v1[TPB], sc[TPB], g0[TPB], g1[TPB];
    float4 rp[TPB], rq[TPB];
  };
  // R state rows per head (the given-transition forms): beta and sel_C per real
  // head, which its R virtual heads share
  const int Hk = H / R, hk = hl / R;
  const auto load_slab = [&](SlabIn& in, int tl) {
#pragma unroll
    for (int i = 0; i < TPB; ++i) {
      const int t = min(tl + blk * TPB + i, tc.nt - 1);
      const int64_t e = (tc.row0 + t) * H + hl;
      const int64_t ek = (tc.row0 + t) * Hk + hk;
      in.bb[i] = T::load(beta + ek);
      in.dd[i] = T::load(dt + (GA ? 2 * e : e));  // SSD and ABar forms: a_t (re, im) from A_bar
      in.rr[i] = T::load(GA ? dt + 2 * e + 1 : r + e);
      in.vq[i] = kAbar ? T::load(r + e) : 1.0f;   // ABar form: vp_t
      in.v0[i] = WITH_W ? T::load(v + 2 * e) : 0.0f;
      in.v1[i] = WITH_W ? T::load(v + 2 * e + 1) : 0.0f;
      in.sc[i] = YM ? 0.0f : T::load(sel_c + ek);
      in.g0[i] = YM ? 0.0f : T::load(dy + 2 * e);
      in.g1[i] = YM ? 0.0f : T::load(dy + 2 * e + 1);
      if constexpr (WITH_W) {
        in.rp[i] = saved[2 * e];
        in.rq[i] = YM ? make_float4(0.0f, 0.0f, 0.0f, 0.0f) : saved[2 * e + 1];
      }
    }
  };
  SlabIn nx;
  load_slab(nx, 0);
  for (int tl = 0; tl < ntr; tl += kWave) {
    const int t0 = tl + blk * TPB;
    const SlabIn in = nx;
    if (tl + kWave < ntr) load_slab(nx, tl + kWave);
    float bb[TPB], dd[TPB], rr[TPB], vq[TPB], v0[TPB], v1[TPB], sc[TPB], g0[TPB], g1[TPB];
    float4 rp[TPB], rq[TPB];
#pragma unroll
    for (int i = 0; i < TPB; ++i) {
      bb[i] = in.bb[i];
      dd[i] = in.dd[i];
      rr[i] = in.rr[i];
      vq[i] = in.vq[i];
      v0[i] = in.v0[i];
      v1[i] = in.v1[i];
      sc[i] = in.sc[i];
      g0[i] = in.g0[i];
      g1[i] = in.g1[i];
      rp[i] = in.rp[i];
      rq[i] = in.rq[i];
    }
    float ar[TPB], ai[TPB], Gr[TPB], Gi[TPB];
    float gpr = 1.0f, gpi = 0.0f;
#pragma unroll
    for (int i = 0; i < TPB; ++i) {
      const bool real = hok && t0 + i < tc.nt;
      if constexpr (RS) {
        // d sel_C = dy . (Y.q) needs nothing from the reverse pass: stored here (R > 1:
        // the state row's part, summed over the head's rows by the row-sum kernel)
        if (real) {
          const int64_t e = (tc.row0 + t0 + i) * H + hl;
          const float ds = g0[i] * rq[i].z + g1[i] * rq[i].w;
          if (R > 1)
            dsp[e] = ds;
          else
            T::store(dsel + e, ds);
        }
      }
      const Transition tr = GA ? Transition{dd[i], rr[i], vq[i]} : cayley_gated(dd[i], rr[i], al, om, c);
      ar[i] = real ? tr.ar : 1.0f;
      ai[i] = real ? tr.ai : 0.0f;
      const float f = bb[i] * tr.vp;
      v0[i] = real ? f * v0[i] : 0.0f;  // w
      v1[i] = real ? f * v1[i] : 0.0f;
      bb[i] = real ? bb[i] : 0.0f;
      g0[i] = real ? sc[i] * g0[i] : 0.0f;  // f = sel dy
      g1[i] = real ? sc[i] * g1[i] : 0.0f;
      cmul_acc(gpr, gpi, ar[i], ai[i]);
      Gr[i] = gpr;
      Gi[i] = gpi;
    }
    // g entering the block: exclusive product over the head's earlier blocks
    float xgr = gpr, xgi = gpi;
    for_shifts<NB>([&](auto offc) {
      constexpr int off = decltype(offc)::value;
      const float ygr = seg_shift_up<NB, off>(xgr), ygi = seg_shift_up<NB, off>(xgi);
      if (blk >= off) cmul_acc(xgr, xgi, ygr, ygi);
    });
    float egr = seg_shift_up<NB, 1>(xgr), egi = seg_shift_up<NB, 1>(xgi);
    if (blk == 0) {
      egr = 1.0f;
      egi = 0.0f;
    }
    cmul_acc(egr, egi, cgr, cgi);
    // RS: the segment's product entering this block (sgr, sgi) and over the
    // whole segment (Sr, Si), by a scan over the SB blocks of the segment
    float sgr = 1.0f, sgi = 0.0f, Sr = 1.0f, Si = 0.0f;
    if constexpr (RS) {
      float ir = gpr, ii = gpi;
      for_shifts<SB>([&](auto offc) {
        constexpr int off = decltype(offc)::value;
        const float yr = seg_shift_up<SB, off>(ir), yi = seg_shift_up<SB, off>(ii);
        if (blk % SB >= off) cmul_acc(ir, ii, yr, yi);
      });
      if constexpr (SB > 1) {
        sgr = seg_shift_up<SB, 1>(ir);
        sgi = seg_shift_up<SB, 1>(ii);
        if (blk % SB == 0) {
          sgr = 1.0f;
          sgi = 0.0f;
        }
      }
      const int last = lane - blk % SB + SB - 1;
      Sr = __shfl(ir, last, kWave);
      Si = __shfl(ii, last, kWave);
      // every |G_{i+1}|^2 of the slab within the frames' range, on every lane
      bool ok = true;
#pragma unroll
      for (int i = 0; i < TPB; ++i) {
        float zr = sgr, zi = sgi;
        cmul_acc(zr, zi, Gr[i], Gi[i]);
        const float n2 = zr * zr + zi * zi;
        ok = ok && n2 >= kRsLo && n2 <= kRsHi;
      }
      rsok = rsok && __all(ok);
      wrote_rs = wrote_rs || rsok;
    }
#pragma unroll
    for (int i = 0; i < TPB; ++i) {
      const int p = (t0 + i) * HPW + j;
      float gr = egr, gi = egi;  // g_t
      cmul_acc(gr, gi, Gr[i], Gi[i]);
      float pr = egr, pi = egi;  // g_{t-1}
      if (i > 0) cmul_acc(pr, pi, Gr[i - 1], Gi[i - 1]);
      if (RS && rsok) {
        // G_{i+1} of the token's segment, e = w - beta a p, and the rescaled coefficients
        float zr = sgr, zi = sgi;
        cmul_acc(zr, zi, Gr[i], Gi[i]);
        const float inv = __builtin_amdgcn_rcpf(zr * zr + zi * zi);
        const bool real = hok && t0 + i < tc.nt;
        const float4 pp = real ? rp[i] : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        const float4 qq = real ? rq[i] : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        const float bpr = bb[i] * pp.x, bpi = bb[i] * pp.y;
        const float er = v0[i] - (ar[i] * bpr - ai[i] * bpi), ei = v1[i] - (ar[i] * bpi + ai[i] * bpr);
        const float ezr = (er * zr + ei * zi) * inv, ezi = (ei * zr - er * zi) * inv;  // e / G
        const float fmr = zr * g0[i] + zi * g1[i], fmi = zr * g1[i] - zi * g0[i];      // conj(G) f
        s.S0[p] = make_float4(ezr, ezi, fmr, fmi);
        s.S1[p] = make_float4(bb[i], pp.z, pp.w, ((t0 + i) & 1) ? Si : Sr);
        s.S2[p] = make_float4(gr * g0[i] + gi * g1[i], gr * g1[i] - gi * g0[i], pr * g0[i] + pi * g1[i],
                              pr * g1[i] - pi * g0[i]);
        sP[p] = make_float4(pp.x, pp.y, ar[i], ai[i]);
        sG[p] = make_float4(g0[i] * qq.x + g1[i] * qq.y, g1[i] * qq.x - g0[i] * qq.y, pr, pi);
        continue;
      }
      s.S1[p] = make_float4(bb[i], g0[i], g1[i], 0.0f);
      if constexpr (YM)  // g_t weights the row dY_t: zero past the last token (the rows are clamped there)
        s.S2[p] = hok && t0 + i < tc.nt ? make_float4(gr, gi, pr, pi) : make_float4(0.0f, 0.0f, pr, pi);
      else
        s.S2[p] = make_float4(gr * g0[i] + gi * g1[i], gr * g1[i] - gi * g0[i], pr, pi);
      if constexpr (WITH_W) {
        // past the last token: p = pc = 0 (inert), delta g = 0, Y.q = 0
        const bool real = hok && t0 + i < tc.nt;
        const float4 pp = real ? rp[i] : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        const float4 qq = real ? rq[i] : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        // e = w - beta a p, the coefficient of k_t in z_t = a z_{t-1} + e k_t
        const float bpr = bb[i] * pp.x, bpi = bb[i] * pp.y;
        s.S0[p] = make_float4(ar[i], ai[i], v0[i] - (ar[i] * bpr - ai[i] * bpi), v1[i] - (ar[i] * bpi + ai[i] * bpr));
        sP[p] = pp;
        // delta g_t = f conj(c^_{t+1}.q), f = sel dy
        sG[p] = make_float4(g0[i] * qq.x + g1[i] * qq.y, g1[i] * qq.x - g0[i] * qq.y, qq.z, qq.w);
      }
    }
    float gtr = egr, gti = egi;
    cmul_acc(gtr, gti, gpr, gpi);
    cgr = __shfl(gtr, j * NB + NB - 1, kWave);
    cgi = __shfl(gti, j * NB + NB - 1, kWave);
  }
  return rsok ? kStageRs : wrote_rs ? kStageMixed : kStagePlain;
}

// Per-token scalars of the correction-adjoint pass: S1 = (beta, 0, 0, 0),
// S2 = (h, 0, 0) with h = conj(g_t) sel_C dy, g_t read from the training
// forward's records (SSD form: S2 = (g_t, 0, 0), the adjoint's input being a
// whole row dY_t).  Slots past the last token and heads >= H are inert.
template <typename T, int HPW>
__device__ __forceinline__ void stage_corr(const ChunkTile& tc, int H, int ntr,
                                           const typename T::raw* __restrict__ beta,
                                           const typename T::raw* __restrict__ sel_c,
                                           const typename T::raw* __restrict__ dy,
                                           const float2* __restrict__ gsaved, const BwdScalars& s, int R = 1) {
  constexpr int NB = kWave / HPW, TPB = HPW;
  const int lane = int(threadIdx.x) % kWave;  // lane in the wave (one-launch workgroups have several)
  const int j = lane / NB;
  const int blk = lane % NB;
  const int hj = tc.hbase + j;
  const bool hok = hj < H;
  const int hl = hok ? hj : H - 1;
  constexpr bool YM = IsSsdY<T>::value;
  const int Hk = H / R, hk = hl / R;  // beta and sel_C per real head (R state rows share them)
  for (int tl = 0; tl < ntr; tl += kWave) {
    const int t0 = tl + blk * TPB;
    float bb[TPB], sc[TPB], g0[TPB], g1[TPB];
    float2 gg[TPB];
#pragma unroll
    for (int i = 0; i < TPB; ++i) {
      const int t = min(t0 + i, tc.nt - 1);
      const int64_t e = (tc.row0 + t) * H + hl;
      const int64_t ek = (tc.row0 + t) * Hk + hk;
      bb[i] = T::load(beta + ek);
      sc[i] = YM ? 1.0f : T::load(sel_c + ek);
      g0[i] = YM ? 0.0f : T::load(dy + 2 * e);
      g1[i] = YM ? 0.0f : T::load(dy + 2 * e + 1);
      gg[i] = gsaved[e];
    }
#pragma unroll
    for (int i = 0; i < TPB; ++i) {
      const bool real = hok && t0 + i < tc.nt;
      const float fr = real ? sc[i] * g0[i] : 0.0f, fi = real ? sc[i] * g1[i] : 0.0f;
      const int p = (t0 + i) * HPW + j;
      s.S1[p] = make_float4(real ? bb[i] : 0.0f, 0.0f, 0.0f, 0.0f);
      if constexpr (YM)
        s.S2[p] = real ? make_float4(gg[i].x, gg[i].y, 0.0f, 0.0f) : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
      else
        s.S2[p] = make_float4(gg[i].x * fr + gg[i].y * fi, gg[i].x * fi - gg[i].y * fr, 0.0f, 0.0f);
    }
  }
}

// ---------------------------------------------------------------------------
// B1: correction-branch adjoint of the entering state, per chunk.
//   lambda = 0; for t = n-1..0: lambda += conj(g_t) sel_t dy_t q_t;
//   lambda <- lambda - beta_t (lambda.k_t) k_t.   Result: lambda_0 = d s_k.
// ---------------------------------------------------------------------------
template <typename T, int D>
__global__ __launch_bounds__(kWave) void fused_bwd_corr_kernel(
    const typename T::raw* __restrict__ q, const typename T::raw* __restrict__ k,
    const typename T::raw* __restrict__ beta, const typename T::raw* __restrict__ sel_c,
    const typename T::raw* __restrict__ dy, const float2* __restrict__ gsaved, float2* __restrict__ lam0,
    int L, int H, int Q, int NC, int n_hg, int R = 1) {
  constexpr int LPH = BwdCorrCfg<D>::LPH, HPW = BwdCorrCfg<D>::HPW, DPL = BwdCorrCfg<D>::DPL, PF = kBwdCorrPF;
  constexpr bool YM = IsSsdY<T>::value;  // SSD form: q points at dY (B,L,H,2,D)
  extern __shared__ float4 smem4[];
  const ChunkTile tc = decode_tile(L, Q, NC, n_hg, HPW);
  const int lane = threadIdx.x;
  const int hh = lane / LPH, sub = lane % LPH;
  const int h = tc.hbase + hh;
  const bool hok = h < H;
  const int hl = hok ? h : H - 1;
  const int slots = round_up(Q, kWave) * HPW;
  const int ntr = round_up(tc.nt, PF);

  // the given-transition forms: R virtual heads (state rows) share each k (and q) row
  constexpr bool RW = GivenA<T>::value;
  const RowStream ks = RW ? tile_stream_rows<T>(k, tc, L, H, R, D, hh, sub * DPL)
                          : tile_stream<T>(k, tc, L, H, D, hh, sub * DPL);
  // readout form: q rows; SSD form: this lane's slices of the dY re (qs) and im (gs) rows
  const RowStream qs = YM   ? tile_stream<T>(q, tc, L, H, 2 * D, hh, sub * DPL)
                       : RW ? tile_stream_rows<T>(q, tc, L, H, R, D, hh, sub * DPL)
                            : tile_stream<T>(q, tc, L, H, D, hh, sub * DPL);
  const RowStream gs = YM ? tile_stream<T>(q, tc, L, H, 2 * D, hh, D + sub * DPL) : RowStream{};
  const int rowb = (RW ? H / R : H) * D * T::bytes;  // token stride of k (and q) in bytes
  const int rowq = YM ? 2 * H * D * T::bytes : rowb;  // of q, or of dY
  const int tlast = tc.nt - 1;
  const int slim = tlast * rowb, slimq = tlast * rowq;
  // reverse ring: slot i holds token ntr-1-(tb+i)
  RowVec<T, DPL> kb[PF], qb[PF], gb[YM ? PF : 1];
#pragma unroll
  for (int i = 0; i < PF; ++i) {
    kb[i].load(ks, min((ntr - 1 - i) * rowb, slim));
    qb[i].load(qs, min((ntr - 1 - i) * rowq, slimq));
    if constexpr (YM) gb[i].load(gs, min((ntr - 1 - i) * rowq, slimq));
  }
  BwdScalars s{nullptr, smem4, smem4 + slots};
  stage_corr<T, HPW>(tc, H, ntr, beta, sel_c, dy, gsaved, s, R);
#pragma unroll
  for (int i = 0; i < PF; ++i) {
    kb[i].pin();
    qb[i].pin();
    if constexpr (YM) gb[i].pin();
  }
  __syncthreads();

  float lr[DPL], li[DPL];
#pragma unroll
  for (int jj = 0; jj < DPL; ++jj) lr[jj] = li[jj] = 0.0f;
  for (int tb = 0; tb < ntr; tb += PF) {
    float4 s1[PF], s2[PF];
#pragma unroll
    for (int i = 0; i < PF; ++i) {
      const int p = (ntr - 1 - (tb + i)) * HPW + hh;
      s1[i] = s.S1[p];
      s2[i] = s.S2[p];
    }
    const int nb = (ntr - 1 - tb - PF) * rowb;  // row offset of the reload for slot 0
    const int nbq = (ntr - 1 - tb - PF) * rowq;
#pragma unroll
    for (int i = 0; i < PF; ++i) {
      float kk[DPL], qq[DPL], gi[DPL];
      kb[i].unpack_then_reload(kk);
      qb[i].unpack_then_reload(qq);
      if constexpr (YM) gb[i].unpack_then_reload(gi);
      kb[i].load(ks, max(min(nb - i * rowb, slim), 0));
      qb[i].load(qs, max(min(nbq - i * rowq, slimq), 0));
      if constexpr (YM) gb[i].load(gs, max(min(nbq - i * rowq, slimq), 0));
      __builtin_amdgcn_sched_barrier(0);  // issue the reloads here, not sunk below later tokens
      // padded steps have h = 0 and beta = 0
      float sr = 0.0f, si = 0.0f;
#pragma unroll
      for (int jj = 0; jj < DPL; ++jj) {
        if constexpr (YM) {
          // lambda += conj(g_t) dY_t
          lr[jj] = fmaf(s2[i].x, qq[jj], fmaf(s2[i].y, gi[jj], lr[jj]));
          li[jj] = fmaf(s2[i].x, gi[jj], fmaf(-s2[i].y, qq[jj], li[jj]));
        } else {
          lr[jj] = fmaf(s2[i].x, qq[jj], lr[jj]);
          li[jj] = fmaf(s2[i].y, qq[jj], li[jj]);
        }
        sr = fmaf(lr[jj], kk[jj], sr);
        si = fmaf(li[jj], kk[jj], si);
      }
      sr = group_sum<LPH>(sr);
      si = group_sum<LPH>(si);
      const float br = s1[i].x * sr, bi = s1[i].x * si;
#pragma unroll
      for (int jj = 0; jj < DPL; ++jj) {
        lr[jj] = fmaf(-br, kk[jj], lr[jj]);
        li[jj] = fmaf(-bi, kk[jj], li[jj]);
      }
    }
  }
  if (hok) {
    float2* lp = lam0 + ((int64_t(tc.b) * NC + tc.chunk) * H + h) * D + sub * DPL;
#pragma unroll
    for (int jj = 0; jj < DPL; ++jj) lp[jj] = make_float2(lr[jj], li[jj]);
  }
}

// ---------------------------------------------------------------------------
// B2: reverse carry, d s_k = conj(G_k) d s_{k+1} + lam0_k, in segments.
// ---------------------------------------------------------------------------
__device__ __forceinline__ float2 cfma_conj(float2 a, float2 b, float2 c) {
  // conj(a) * b + c
  return make_float2(fmaf(a.x, b.x, fmaf(a.y, b.y, c.x)), fmaf(a.x, b.y, fmaf(-a.y, b.x, c.y)));
}
__device__ __forceinline__ float2 cmul_conj(float2 a, float2 b) {
  return make_float2(a.x * b.x + a.y * b.y, a.x * b.y - a.y * b.x);
}

struct RCarry {
  int b, h, seg, d, c0, c1;
  int64_t base;
};
__device__ __forceinline__ RCarry rcarry_index(int64_t tid, int NC, int H, int D, int S) {
  RCarry x;
  x.d = int(tid % D);
  int64_t rest = tid / D;
  x.seg = int(rest % S);
  rest /= S;
  x.h = int(rest % H);
  x.b = int(rest / H);
  x.c0 = min(NC, x.seg * kBwdSeg);
  x.c1 = min(NC, x.c0 + kBwdSeg);
  x.base = int64_t(x.b) * NC * H + x.h;
  return x;
}

__global__ __launch_bounds__(256) void fused_bwd_rfold_kernel(const float2* __restrict__ lam0,
                                                             const float2* __restrict__ gam,
                                                             float2* __restrict__ segA,
                                                             float2* __restrict__ segX, int B, int NC,
                                                             int H, int D, int S) {
  const int64_t tid = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  if (tid >= int64_t(B) * H * S * D) return;
  const RCarry x = rcarry_index(tid, NC, H, D, S);
  // map: ds_{c0} = A ds_{c1} + X; all loads of the segment issued first
  float2 G[kBwdSeg], Lm[kBwdSeg];
#pragma unroll
  for (int i = 0; i < kBwdSeg; ++i) {
    const int64_t e = x.base + int64_t(min(x.c0 + i, x.c1 - 1)) * H;
    G[i] = gam[e];
    Lm[i] = lam0[e * D + x.d];
  }
  float2 A = make_float2(1.0f, 0.0f), X = make_float2(0.0f, 0.0f);
#pragma unroll
  for (int i = kBwdSeg - 1; i >= 0; --i) {
    if (x.c0 + i < x.c1) {
      X = cfma_conj(G[i], X, Lm[i]);
      A = cmul_conj(G[i], A);
    }
  }
  const int64_t sidx = (int64_t(x.b) * H + x.h) * S + x.seg;
  segX[sidx * D + x.d] = X;
  if (x.d == 0) segA[sidx] = A;
}

__global__ __launch_bounds__(256) void fused_bwd_rreplay_kernel(
    const float2* __restrict__ lam0, const float2* __restrict__ gam, const float2* __restrict__ segA,
    const float2* __restrict__ segX, const float* __restrict__ dh_final, float2* __restrict__ dsn,
    float* __restrict__ dh0, int B, int NC, int H, int D, int S) {
  const int64_t tid = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  if (tid >= int64_t(B) * H * S * D) return;
  const RCarry x = rcarry_index(tid, NC, H, D, S);
  const int64_t sbase = (int64_t(x.b) * H + x.h) * S;
  const int64_t hb = (int64_t(x.b) * H + x.h) * 2 * D;
  float2 ds = make_float2(0.0f, 0.0f);
  if (dh_final != nullptr) ds = make_float2(dh_final[hb + x.d], dh_final[hb + D + x.d]);
  // the segment's own loads first, then the later segments' maps (in groups of 8)
  float2 G[kBwdSeg], Lm[kBwdSeg];
#pragma unroll
  for (int i = 0; i < kBwdSeg; ++i) {
    const int64_t e = x.base + int64_t(min(x.c0 + i, max(x.c1 - 1, 0))) * H;
    G[i] = gam[e];
    Lm[i] = lam0[e * D + x.d];
  }
  for (int jb = S - 1; jb > x.seg; jb -= 8) {
    float2 A[8], X[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int64_t j = sbase + max(jb - i, x.seg + 1);
      A[i] = segA[j];
      X[i] = segX[j * D + x.d];
    }
#pragma unroll
    for (int i = 0; i < 8; ++i)
      if (jb - i > x.seg)
        ds = make_float2(A[i].x * ds.x - A[i].y * ds.y + X[i].x, A[i].x * ds.y + A[i].y * ds.x + X[i].y);
  }
#pragma unroll
  for (int i = kBwdSeg - 1; i >= 0; --i) {
    if (x.c0 + i < x.c1) {
      dsn[(x.base + int64_t(x.c0 + i) * H) * D + x.d] = ds;
      ds = cfma_conj(G[i], ds, Lm[i]);
    }
  }
  if (x.seg == 0 && dh0 != nullptr) {
    dh0[hb + x.d] = ds.x;
    dh0[hb + D + x.d] = ds.y;
  }
}


// ---------------------------------------------------------------------------
// B1 + B2 in one launch (when one round of resident workgroups holds every
// segment).  A workgroup of kOnePassW waves takes kOnePassW consecutive chunks
// (a segment) of one (b, head group), segments taken from the last: wave w
// runs B1 for chunk kOnePassW * seg + w; the segment's reverse map
// d s_{k0} = A d s_{k0+n} + X (A = prod conj(G_k), X from the chunks' lambda_0)
// is composed through LDS and published; the carry adjoint at the segment's
// right end is the composition, in a fixed order, of the maps of the segments
// since its anchor (kAnchor segments, counted from the right) applied to the
// anchor state (d h_final, or the published left-end state of the segment
// right of the anchor); each wave then writes d s_{k+1} of its chunk, and the
// first segment writes d h0.  Flags and ordering as in the one-pass forward;
// the epoch comes from bwd_epoch_kernel, launched just before on the same
// stream, and a wait that gives up sets kTimeoutBwd in g_bwd_status.
// ---------------------------------------------------------------------------

// Device-side state of this unit's one-launch carry, one copy per GPU: the
// count of calls (the source of their epochs, tagged apart from the forward's)
// and the sticky status word.
__device__ unsigned long long g_bwd_calls;
__device__ unsigned int g_bwd_status;

__global__ __launch_bounds__(64) void bwd_epoch_kernel(unsigned long long* ctl) {
  if (threadIdx.x == 0) {
    const unsigned long long n =
        __hip_atomic_fetch_add(&g_bwd_calls, 1ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) + 1ull;
    __hip_atomic_store(ctl + 1, 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __hip_atomic_store(ctl, epoch_word(2u, n), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
}
// Phase stamps of cdssm_fused_scan_bwd_stamped (instrumentation only): the 100
// MHz real-time counter per wave at kBwdCorrStamps points of the one-launch
// correction adjoint + carry and kBwdMainStamps points of the main pass.
constexpr int kBwdCorrStamps = 8, kBwdMainStamps = 4;

template <typename T>
struct CorrCarryArgs {
  const typename T::raw *q, *k, *beta, *sel_c, *dy;
  const float2* gsaved;   // the training forward's g_t (B, L, H)
  const float2* gam;      // the training forward's G_k (B, NC, H)
  const float* dh_final;  // (B, H, 2, D) or null
  float2* dsn;            // out: d s_{k+1} per chunk (B, NC, H, D)
  float* dh0;             // out: (B, H, 2, D) or null
  OnePassBufs ob;         // X in seg_f, A in seg_g, left-end states in seg_s; epoch in ctl[0]
  int L, H, Q, NC, NSEG, n_hg, n_chain;
  int R;                  // SSD form: state rows per head (virtual heads sharing a k row); 1 otherwise
  unsigned long long* stamps;  // instrumentation: kBwdCorrStamps words per wave, or null
};

template <typename T, int D>
__global__ __launch_bounds__(kWave * kOnePassW) void fused_bwd_corrcarry_kernel(CorrCarryArgs<T> a) {
  constexpr int LPH = BwdCorrCfg<D>::LPH, HPW = BwdCorrCfg<D>::HPW, DPL = BwdCorrCfg<D>::DPL, PF = kBwdCorrPF;
  constexpr int W = kOnePassW;
  constexpr int SEGN = HPW * D;             // complex elements of a head group's state
  constexpr int EPT = SEGN / (kWave * W);   // composed by each thread of the workgroup
  static_assert(EPT >= 1 && EPT * kWave * W == SEGN && D % EPT == 0, "segment state tiles the workgroup");
  extern __shared__ float4 smem4[];
  const int L = a.L, H = a.H, Q = a.Q, NC = a.NC, NSEG = a.NSEG;
  const unsigned long long epoch = load_epoch(a.ob.ctl);

  const int wv = __builtin_amdgcn_readfirstlane(int(threadIdx.x) / kWave);
  const int lane = int(threadIdx.x) % kWave;
  // phase stamps, read and stored only when a.stamps is set (a uniform branch): entry, staged, lambda pass
  // done, segment map published, look-back wait done, carry folded, left-end state published, end
  const bool stamping = a.stamps != nullptr;
  unsigned long long ts[kBwdCorrStamps];
  auto stamp = [&](int i) {
    if (stamping) ts[i] = __builtin_amdgcn_s_memrealtime();
  };
  stamp(0);
  const int chain = int(blockIdx.x) % a.n_chain;
  const int rs = int(blockIdx.x) / a.n_chain;  // segments counted from the right
  const int seg = NSEG - 1 - rs;
  const int bi = chain / a.n_hg;
  const int hbase = (chain % a.n_hg) * HPW;
  const int n_live = min(W, NC - seg * W);
  const bool live = wv < n_live;

  ChunkTile tc;
  tc.b = bi;
  tc.chunk = min(seg * W + wv, NC - 1);
  tc.hbase = hbase;
  tc.t0 = tc.chunk * Q;
  tc.nt = min(Q, L - tc.t0);
  tc.row0 = int64_t(bi) * L + tc.t0;
  const int hh = lane / LPH, sub = lane % LPH;
  const int h = hbase + hh;
  const bool hok = h < H;
  const int hl = hok ? h : H - 1;
  const int slots = round_up(Q, kWave) * HPW;
  const int ntr = round_up(tc.nt, PF);

  // LDS: per wave S1, S2 (float4 token slots), which after the wave's lambda
  // pass hold its lambda_0 (SEGN float2 <= 2 * slots float4); G per (wave,
  // head); the carry adjoint at the segment's right end
  BwdScalars s{nullptr, smem4 + size_t(wv) * 2 * slots, smem4 + size_t(wv) * 2 * slots + slots};
  auto Lw = [&](int u) { return reinterpret_cast<float2*>(smem4 + size_t(u) * 2 * slots); };
  float2* Gx = reinterpret_cast<float2*>(smem4 + size_t(W) * 2 * slots);
  float2* Sx = Gx + W * HPW;
  int* ctrl = reinterpret_cast<int*>(Sx + SEGN);

  // ---- B1 for this wave's chunk: lambda backward through the chunk ----
  float lr[DPL], li[DPL];
#pragma unroll
  for (int jj = 0; jj < DPL; ++jj) lr[jj] = li[jj] = 0.0f;
  constexpr bool YM = IsSsdY<T>::value;  // SSD form: q points at dY (B,L,H,2,D)
  // the given-transition forms: R virtual heads (state rows) share each k (and q) row
  constexpr bool RW = GivenA<T>::value;
  const RowStream ks = RW ? tile_stream_rows<T>(a.k, tc, L, H, a.R, D, hh, sub * DPL)
                          : tile_stream<T>(a.k, tc, L, H, D, hh, sub * DPL);
  // readout form: q rows; SSD form: this lane's slices of the dY re (qs) and im (gs) rows
  const RowStream qs = YM   ? tile_stream<T>(a.q, tc, L, H, 2 * D, hh, sub * DPL)
                       : RW ? tile_stream_rows<T>(a.q, tc, L, H, a.R, D, hh, sub * DPL)
                            : tile_stream<T>(a.q, tc, L, H, D, hh, sub * DPL);
  const RowStream gs = YM ? tile_stream<T>(a.q, tc, L, H, 2 * D, hh, D + sub * DPL) : RowStream{};
  const int rowb = (RW ? H / a.R : H) * D * T::bytes;  // token stride of k (and q) in bytes
  const int rowq = YM ? 2 * H * D * T::bytes : rowb;   // of q, or of dY
  const int tlast = tc.nt - 1;
  const int slim = tlast * rowb, slimq = tlast * rowq;
  RowVec<T, DPL> kb[PF], qb[PF], gb[YM ? PF : 1];
  if (live) {
#pragma unroll
    for (int i = 0; i < PF; ++i) {
      kb[i].load(ks, min((ntr - 1 - i) * rowb, slim));
      qb[i].load(qs, min((ntr - 1 - i) * rowq, slimq));
      if constexpr (YM) gb[i].load(gs, min((ntr - 1 - i) * rowq, slimq));
    }
    stage_corr<T, HPW>(tc, H, ntr, a.beta, a.sel_c, a.dy, a.gsaved, s, a.R);
#pragma unroll
    for (int i = 0; i < PF; ++i) {
      kb[i].pin();
      qb[i].pin();
      if constexpr (YM) gb[i].pin();
    }
  }
  __syncthreads();  // every wave reaches every barrier of this kernel
  stamp(1);
  if (live) {
    for (int tb = 0; tb < ntr; tb += PF) {
      float4 s1[PF], s2[PF];
#pragma unroll
      for (int i = 0; i < PF; ++i) {
        const int p = (ntr - 1 - (tb + i)) * HPW + hh;
        s1[i] = s.S1[p];
        s2[i] = s.S2[p];
      }
      const int nb = (ntr - 1 - tb - PF) * rowb;  // row offset of the reload for slot 0
      const int nbq = (ntr - 1 - tb - PF) * rowq;
#pragma unroll
      for (int i = 0; i < PF; ++i) {
        float kk[DPL], qq[DPL], gi[DPL];
        kb[i].unpack_then_reload(kk);
        qb[i].unpack_then_reload(qq);
        if constexpr (YM) gb[i].unpack_then_reload(gi);
        kb[i].load(ks, max(min(nb - i * rowb, slim), 0));
        qb[i].load(qs, max(min(nbq - i * rowq, slimq), 0));
        if constexpr (YM) gb[i].load(gs, max(min(nbq - i * rowq, slimq), 0));
        __builtin_amdgcn_sched_barrier(0);
        float sr = 0.0f, si = 0.0f;
#pragma unroll
        for (int jj = 0; jj < DPL; ++jj) {
          if constexpr (YM) {
            // lambda += conj(g_t) dY_t
            lr[jj] = fmaf(s2[i].x, qq[jj], fmaf(s2[i].y, gi[jj], lr[jj]));
            li[jj] = fmaf(s2[i].x, gi[jj], fmaf(-s2[i].y, qq[jj], li[jj]));
          } else {
            lr[jj] = fmaf(s2[i].x, qq[jj], lr[jj]);
            li[jj] = fmaf(s2[i].y, qq[jj], li[jj]);
          }
          sr = fmaf(lr[jj], kk[jj], sr);
          si = fmaf(li[jj], kk[jj], si);
        }
        sr = group_sum<LPH>(sr);
        si = group_sum<LPH>(si);
        const float br = s1[i].x * sr, bi2 = s1[i].x * si;
#pragma unroll
        for (int jj = 0; jj < DPL; ++jj) {
          lr[jj] = fmaf(-br, kk[jj], lr[jj]);
          li[jj] = fmaf(-bi2, kk[jj], li[jj]);
        }
      }
    }
#pragma unroll
    for (int i = 0; i < PF; ++i) {
      kb[i].pin();
      qb[i].pin();
      if constexpr (YM) gb[i].pin();
    }
    // lambda_0 and G_k of the chunk (heads >= H: zero map)
#pragma unroll
    for (int jj = 0; jj < DPL; ++jj)
      Lw(wv)[hh * D + sub * DPL + jj] = hok ? make_float2(lr[jj], li[jj]) : make_float2(0.0f, 0.0f);
    if (sub == 0)
      Gx[wv * HPW + hh] = hok ? a.gam[(int64_t(bi) * NC + tc.chunk) * H + h] : make_float2(1.0f, 0.0f);
  }
  stamp(2);
  __syncthreads();

  // ---- the segment's reverse map over its live chunks ----
  const int e0 = int(threadIdx.x) * EPT;
  const int ej = e0 / D, ed = e0 % D;
  const int eh = hbase + ej;
  const bool ehok = eh < H;
  float2 X[EPT];
  float2 A = make_float2(1.0f, 0.0f);
#pragma unroll
  for (int i = 0; i < EPT; ++i) X[i] = make_float2(0.0f, 0.0f);
  for (int u = n_live - 1; u >= 0; --u) {
    const float2 g = Gx[u * HPW + ej];
#pragma unroll
    for (int i = 0; i < EPT; ++i) {
      const float2 l = Lw(u)[e0 + i];
      X[i] = make_float2(g.x * X[i].x + g.y * X[i].y + l.x, g.x * X[i].y - g.y * X[i].x + l.y);
    }
    A = make_float2(g.x * A.x + g.y * A.y, g.x * A.y - g.y * A.x);
  }
  const OnePassBufs& ob = a.ob;
  const int64_t sb0 = (int64_t(bi) * NSEG + seg) * H;  // (b, seg, head 0)
  unsigned long long* flag = ob.flag + sb0 + hbase;
  if (ehok) {
#pragma unroll
    for (int i = 0; i < EPT; ++i) st_agent(ob.seg_f + (sb0 + eh) * D + ed + i, X[i]);
    if (ed == 0) st_agent(ob.seg_g + sb0 + eh, A);
  }
  wait_stores_acked();
  __syncthreads();
  if (threadIdx.x == 0) {
    __hip_atomic_store(flag, (epoch << 2) | 1ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    // every workgroup of the grid holds this call's epoch once all have published
    arrive_and_draw_next_epoch(ob.ctl, &g_bwd_calls, 2u);
  }

  stamp(3);
  // ---- carry adjoint at the segment's right end, from its anchor ----
  const int anc = rs == 0 ? 0 : kAnchor * ((rs - 1) / kAnchor);  // counted from the right
  const int nmap = rs - anc;
  int ok = 1;
  if (rs > 0) {
    if (wv == 0) {
      const unsigned long long* f0 = ob.flag + (int64_t(bi) * NSEG) * H + hbase;
      int got = 0;
      const uint64_t t_start = __builtin_amdgcn_s_memrealtime();
      for (;;) {
        int st = 3;
        // lane i: map of the segment anc + i from the right; lane 63: the anchor state
        const int jr = lane < nmap ? anc + lane : (lane == kWave - 1 && anc > 0 ? anc - 1 : -1);
        if (jr >= 0) {
          const unsigned long long fv =
              __hip_atomic_load(const_cast<unsigned long long*>(f0 + int64_t(NSEG - 1 - jr) * H), __ATOMIC_RELAXED,
                                __HIP_MEMORY_SCOPE_AGENT);
          st = (fv >> 2) == epoch ? int(fv & 3ull) : 0;
        }
        const bool ready = lane < nmap ? st >= 1 : (lane == kWave - 1 && anc > 0 ? st == 2 : true);
        if (__builtin_amdgcn_ballot_w64(!ready) == 0ull) {
          got = 1;
          break;
        }
        if (__builtin_amdgcn_s_memrealtime() - t_start > kSpinTicks) break;
        __builtin_amdgcn_s_sleep(2);
      }
      if (lane == 0) {
        ctrl[0] = got;
        if (!got) __hip_atomic_fetch_or(&g_bwd_status, kTimeoutBwd, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
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
    const int64_t lb = int64_t(bi) * NSEG * H + eh;  // (b, segment 0, head eh)
    if (anc == 0) {
      if (a.dh_final) {
        const int64_t hb = (int64_t(bi) * H + eh) * 2 * D;
#pragma unroll
        for (int i = 0; i < EPT; ++i) Sin[i] = make_float2(a.dh_final[hb + ed + i], a.dh_final[hb + D + ed + i]);
      }
    } else {
#pragma unroll
      for (int i = 0; i < EPT; ++i)
        Sin[i] = ld_agent(ob.seg_s + (lb + int64_t(NSEG - anc) * H) * D + ed + i);
    }
    for (int jb = 0; jb < nmap; jb += kLookbackBatch) {
      float2 G[kLookbackBatch], F[kLookbackBatch][EPT];
#pragma unroll
      for (int u = 0; u < kLookbackBatch; ++u) {
        const int js = NSEG - 1 - (anc + min(jb + u, nmap - 1));
        G[u] = ld_agent(ob.seg_g + lb + int64_t(js) * H);
#pragma unroll
        for (int i = 0; i < EPT; ++i) F[u][i] = ld_agent(ob.seg_f + (lb + int64_t(js) * H) * D + ed + i);
      }
#pragma unroll
      for (int u = 0; u < kLookbackBatch; ++u) {
        if (jb + u < nmap) {
#pragma unroll
          for (int i = 0; i < EPT; ++i)
            Sin[i] = make_float2(G[u].x * Sin[i].x - G[u].y * Sin[i].y + F[u][i].x,
                                 G[u].x * Sin[i].y + G[u].y * Sin[i].x + F[u][i].y);
        }
      }
    }
    if (!ok) {
#pragma unroll
      for (int i = 0; i < EPT; ++i) Sin[i] = make_float2(__builtin_nanf(""), __builtin_nanf(""));
    }
  }
  stamp(5);
  // the segment's left-end state: published for the segments that start from
  // it, and d h0 for the first segment
  const bool anchor_end = rs + 1 < NSEG && (rs + 1) % kAnchor == 0;
#pragma unroll
  for (int i = 0; i < EPT; ++i) Sx[e0 + i] = Sin[i];
  if (ehok && (anchor_end || (seg == 0 && a.dh0))) {
#pragma unroll
    for (int i = 0; i < EPT; ++i) {
      const float2 so = make_float2(A.x * Sin[i].x - A.y * Sin[i].y + X[i].x, A.x * Sin[i].y + A.y * Sin[i].x + X[i].y);
      if (anchor_end) {
        st_agent(ob.seg_s + (sb0 + eh) * D + ed + i, so);
      } else {
        const int64_t hb = (int64_t(bi) * H + eh) * 2 * D;
        a.dh0[hb + ed + i] = so.x;
        a.dh0[hb + D + ed + i] = so.y;
      }
    }
  }
  if (anchor_end) wait_stores_acked();
  __syncthreads();
  if (anchor_end && threadIdx.x == 0)
    __hip_atomic_store(flag, (epoch << 2) | 2ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);

  stamp(6);
  // ---- d s_{k+1} of this wave's chunk: the maps of the later chunks of the
  // segment applied to the right-end state ----
  if (live && hok) {
    float2 acc[DPL];
#pragma unroll
    for (int jj = 0; jj < DPL; ++jj) acc[jj] = Sx[hh * D + sub * DPL + jj];
    for (int u = n_live - 1; u > wv; --u) {
      const float2 g = Gx[u * HPW + hh];
#pragma unroll
      for (int jj = 0; jj < DPL; ++jj) {
        const float2 l = Lw(u)[hh * D + sub * DPL + jj];
        acc[jj] = make_float2(g.x * acc[jj].x + g.y * acc[jj].y + l.x, g.x * acc[jj].y - g.y * acc[jj].x + l.y);
      }
    }
    float2* dp = a.dsn + ((int64_t(bi) * NC + tc.chunk) * H + h) * D + sub * DPL;
#pragma unroll
    for (int jj = 0; jj < DPL; ++jj) dp[jj] = acc[jj];
  }
  stamp(7);
  if (stamping && lane == 0) {
    unsigned long long* o = a.stamps + (int64_t(blockIdx.x) * W + wv) * kBwdCorrStamps;
#pragma unroll
    for (int i = 0; i < kBwdCorrStamps; ++i) o[i] = ts[i];
  }
}

// ---------------------------------------------------------------------------
// Scan-level dynamics backward for one token: (d ar, d ai, d vp) ->
// (d dt, d r, d alpha, d omega), exact derivative of cayley_gated().
// ---------------------------------------------------------------------------
struct DynGrad {
  float ddt, dr, dalpha, domega;
};

__device__ __forceinline__ DynGrad cayley_gated_bwd(float dt, float r, float alpha, float omega, float c,
                                                    float gar, float gai, float gvp) {
  const float tau = 0.5f * dt;
  const float ap = fmaxf(alpha, 0.0f);
  const float ta = tau * ap;
  const float tw = tau * omega;
  const float tw2 = tw * tw;
  const float opa = 1.0f + ta, oma = 1.0f - ta;
  const float den = opa * opa + tw2 + 1e-6f;
  const float inv = 1.0f / den;
  const float nre = 1.0f - ta * ta - tw2;
  const float mur = nre * inv;
  const float mui = (2.0f * tw) * inv;
  const float num = oma * oma + tw2;
  const float E0 = num * inv;
  const float E = fmaxf(E0, 1e-8f);
  const float cr = c * r;
  const float lE2 = __builtin_amdgcn_logf(E);
  const float lE = lE2 * 0.69314718055994531f;  // natural log
  const float scale = __builtin_amdgcn_exp2f(0.5f * (cr - 1.0f) * lE2);
  const float eff = __builtin_amdgcn_exp2f(cr * lE2);
  const float u = 1.0f - eff;
  const float vpu = sqrtf(fmaxf(u, 1e-6f));

  // ar = mur*scale, ai = -mui*scale
  const float dscale = gar * mur - gai * mui;
  const float dmur = gar * scale;
  const float dmui = -gai * scale;
  // vp = min(sqrt(max(u, 1e-6)), 1)
  float du = 0.0f;
  if (u >= 1e-6f && vpu <= 1.0f) du = gvp * 0.5f / vpu;
  const float deff = -du;
  const float Einv = 1.0f / E;
  float dE = dscale * 0.5f * (cr - 1.0f) * scale * Einv + deff * cr * eff * Einv;
  const float dcr = dscale * 0.5f * lE * scale + deff * lE * eff;
  const float dE0 = E0 >= 1e-8f ? dE : 0.0f;
  const float dnum = dE0 * inv;
  const float dinv = dE0 * num + dmur * nre + dmui * 2.0f * tw;
  const float dden = -dinv * inv * inv;
  const float dta = dnum * (-2.0f * oma) + dden * 2.0f * opa + dmur * (-2.0f * ta * inv);
  const float dtw = dnum * 2.0f * tw + dden * 2.0f * tw + dmur * (-2.0f * tw * inv) + dmui * 2.0f * inv;
  const float dtau = dta * ap + dtw * omega;
  DynGrad g;
  g.ddt = 0.5f * dtau;
  g.dr = c * dcr;
  g.dalpha = alpha >= 0.0f ? dta * tau : 0.0f;
  g.domega = dtw * tau;
  return g;
}

// ---------------------------------------------------------------------------
// B3: per-chunk backward of both branches, from the training forward's
//   workspace: z_{t-1} every kBwdCK tokens, c^ after the chunk's last step,
//   and per token p_t = z_{t-1}.k_t, pc_t = c^_t.k_t, c^_{t+1}.q_t, Y_t.q_t
//   (staged in LDS with the correction's delta g_t);
//   reverse pass, kBwdCK tokens at a time: z of the segment is recomputed
//     from its checkpoint with the staged e_t (no reductions); c^_t is rebuilt
//     backward, exactly, as c^_t = c^_{t+1} + beta_t pc_t k_t; the local adjoint
//     mu and the correction adjoint lambda step back and dk, dq are emitted.
//     Readout form: z and mu run in the segment's rescaled frames (no
//     multiply by a_t per state element), unless a segment's rotation
//     products leave the frames' range (then the wave takes the unscaled step);
//   epilogue, lanes owning blocks of tokens: the token's scalar gradients
//     (d a_t with the backward recurrence psi of the rotation products, the
//     erase part of d beta), the dynamics chain rule, dv, dbeta, dsel, ddt, dr,
//     and the chunk's d alpha / d omega per head.
// LDS (float4 per (token, head) slot): S0, S1, S2 (staged scalars), P = (p,
// pc), G = (delta g, Y.q); the reverse step of token t leaves S0 = (a,
// mu.z_{t-1}) and S1 = (mu.k, lambda.k) for the epilogue (SSD form: G =
// (delta g, 0, 0), delta g formed in the step).
// ---------------------------------------------------------------------------
// A token's dk (and dq) rows: per virtual head into dk / dq, or, with R > 1
// state rows per head, as fp32 partials (dkp / dqp) that the row-sum kernel adds
// up; where the wave's heads are rows of one real head they are summed over the
// wave first and stored by head 0's lanes.
template <typename T, int LPH, int DPL, bool WITH_Q>
__device__ __forceinline__ void store_dk_dq(bool rows, bool rows_pre, bool hok, int hh, float (&dkv)[DPL],
                                            float (&dqv)[DPL], const RowStream& dks, const RowStream& dkps,
                                            const RowStream& dqs, const RowStream& dqps, int off, int offp) {
  if (rows_pre) {
#pragma unroll
    for (int jj = 0; jj < DPL; ++jj) dkv[jj] = cross_head_sum<LPH>(dkv[jj]);
    if constexpr (WITH_Q) {
#pragma unroll
      for (int jj = 0; jj < DPL; ++jj) dqv[jj] = cross_head_sum<LPH>(dqv[jj]);
    }
    if (hh == 0) {
      store_row<F32, DPL>(dkps, offp, dkv);
      if constexpr (WITH_Q) store_row<F32, DPL>(dqps, offp, dqv);
    }
  } else if (hok) {
    if (rows) {
      store_row<F32, DPL>(dkps, offp, dkv);
      if constexpr (WITH_Q) store_row<F32, DPL>(dqps, offp, dqv);
    } else {
      store_row<T, DPL>(dks, off, dkv);
      if constexpr (WITH_Q) store_row<T, DPL>(dqs, off, dqv);
    }
  }
}

template <typename T, int D>
__global__ __launch_bounds__(kWave) __attribute__((amdgpu_waves_per_eu(T::bytes == 2 ? 2 : 1, 2))) void fused_bwd_main_kernel(
    const typename T::raw* __restrict__ q, const typename T::raw* __restrict__ k,
    const typename T::raw* __restrict__ v, const typename T::raw* __restrict__ beta,
    const typename T::raw* __restrict__ sel_c, const typename T::raw* __restrict__ dt,
    const typename T::raw* __restrict__ r, const float* __restrict__ alpha,
    const float* __restrict__ omega, float c, const typename T::raw* __restrict__ dy,
    const float2* __restrict__ states, const float4* __restrict__ saved, const float2* __restrict__ dsn,
    const float2* __restrict__ zck, const float2* __restrict__ cend, typename T::raw* __restrict__ dq,
    typename T::raw* __restrict__ dk,
    typename T::raw* __restrict__ dv,
    typename T::raw* __restrict__ dbeta, typename T::raw* __restrict__ dsel,
    typename T::raw* __restrict__ ddt, typename T::raw* __restrict__ dr, float2* __restrict__ dhead_parts,
    int L, int H, int Q, int NC, int NCK, int n_hg, int R = 1, float* __restrict__ dkp = nullptr,
    float* __restrict__ dbp = nullptr, float* __restrict__ dqp = nullptr, float* __restrict__ dsp = nullptr,
    unsigned long long* __restrict__ stamps = nullptr) {
  constexpr int LPH = BwdCfg<D>::LPH, HPW = BwdCfg<D>::HPW, DPL = BwdCfg<D>::DPL, PF = kBwdPF, CK = kBwdCK;
  static_assert(CK == kZck && PF == kTokRound, "the training forward's z checkpoints: every CK tokens");
  extern __shared__ float4 smem4[];
  // Two waves per SIMD, never three: the attribute above holds the 2-byte
  // kernels (rescaled and unscaled step in one kernel) to the 256-register
  // budget of two waves, spilling a few values that live across the reverse
  // pass; the reservation below keeps a lighter build from letting three waves
  // onto some SIMDs while others hold one (one-wave workgroups are placed per
  // SIMD as slots free up), which measured 287 against 248 us at C2 (D = 128,
  // 1.5 rounds of waves) on MI355X.
  asm volatile("" ::: "v255");
  // phase stamps (instrumentation, when stamps is set): entry, staged, reverse pass done, end
  const bool stamping = stamps != nullptr;
  unsigned long long ts[kBwdMainStamps];
  auto stamp = [&](int i) {
    if (stamping) ts[i] = __builtin_amdgcn_s_memrealtime();
  };
  stamp(0);
  const ChunkTile tc = decode_tile(L, Q, NC, n_hg, HPW);
  const int lane = threadIdx.x;
  const int hh = lane / LPH, sub = lane % LPH;
  const int h = tc.hbase + hh;
  const bool hok = h < H;
  const int hl = hok ? h : H - 1;
  const int slots = round_up(Q, kWave) * HPW;
  const int ntr = round_up(tc.nt, PF);
  constexpr bool YM = IsSsdY<T>::value;  // SSD form: q points at dY (B,L,H,2,D); dq not formed
  constexpr bool kAbar = IsABar<T>::value;  // gate-level a_t and vp given: no per-head dynamics parameters
  const float al = YM || kAbar ? 0.0f : alpha[hl], om = YM || kAbar ? 0.0f : omega[hl];

  // The given-transition forms (SSD, gate-level): R virtual heads (state rows) share each k row (and q,
  // beta, sel_C); with R > 1 their fp32 dk (and dq) rows go to dkp (dqp) and a row-sum kernel forms dk
  // (dq).  Where a wave's HPW heads are rows of one real head (R % HPW == 0) the wave sums them first and
  // writes one row per wave, dkp (B, L, H / HPW, D); otherwise one per virtual head, dkp (B, L, H, D)
  constexpr bool RW = GivenA<T>::value;
  const bool rows = RW && R > 1;
  const bool rows_pre = rows && R % HPW == 0;
  const RowStream ks = RW ? tile_stream_rows<T>(k, tc, L, H, R, D, hh, sub * DPL)
                          : tile_stream<T>(k, tc, L, H, D, hh, sub * DPL);
  // readout form: q rows; SSD form: this lane's slices of the dY re (qs) and im (gs) rows
  const RowStream qs = YM   ? tile_stream<T>(q, tc, L, H, 2 * D, hh, sub * DPL)
                       : RW ? tile_stream_rows<T>(q, tc, L, H, R, D, hh, sub * DPL)
                            : tile_stream<T>(q, tc, L, H, D, hh, sub * DPL);
  const RowStream gs = YM ? tile_stream<T>(q, tc, L, H, 2 * D, hh, D + sub * DPL) : RowStream{};
  const RowStream dks = rows ? RowStream{} : tile_stream<T>(dk, tc, L, H, D, hh, sub * DPL);
  ChunkTile tcp = tc;  // the wave's partial row: head hbase / HPW of H / HPW
  tcp.hbase = tc.hbase / HPW;
  const RowStream dkps = !rows      ? RowStream{}
                         : rows_pre ? tile_stream<F32>(dkp, tcp, L, H / HPW, D, 0, sub * DPL)
                                    : tile_stream<F32>(dkp, tc, L, H, D, hh, sub * DPL);
  const RowStream dqs = YM || rows ? RowStream{} : tile_stream<T>(dq, tc, L, H, D, hh, sub * DPL);
  const RowStream dqps = YM || !rows ? RowStream{}
                         : rows_pre  ? tile_stream<F32>(dqp, tcp, L, H / HPW, D, 0, sub * DPL)
                                     : tile_stream<F32>(dqp, tc, L, H, D, hh, sub * DPL);
  const int rowb = (RW ? H / R : H) * D * T::bytes;  // token stride of k (and q, dq, dk) in bytes
  const int rowq = YM ? 2 * H * D * T::bytes : rowb;  // of q, or of dY
  const int rowp = (rows_pre ? H / HPW : H) * D * 4;   // of dkp (and dqp)
  const int tlast = tc.nt - 1;
  const int slim = tlast * rowb, slimq = tlast * rowq;
  const int64_t chh = (int64_t(tc.b) * NC + tc.chunk) * H + hl;  // (b, chunk, head) index
  // the training forward's z checkpoints of this (chunk, head): z_{t-1} at t = CK * seg
  const int64_t ck0 = chh * NCK * D + sub * DPL;

  // c^ after the chunk's last step (the reverse pass rebuilds it backward)
  float cr[DPL], ci[DPL];
  const float2* sp = states + chh * D + sub * DPL;
  {
    const float2* ce = cend + chh * D + sub * DPL;
#pragma unroll
    for (int jj = 0; jj < DPL; ++jj) {
      const float2 cv = ce[jj];
      cr[jj] = hok ? cv.x : 0.0f;
      ci[jj] = hok ? cv.y : 0.0f;
    }
  }
  BwdScalars s{smem4, smem4 + slots, smem4 + 2 * slots};
  float4* sP = smem4 + 3 * slots;
  float4* sG = smem4 + 4 * slots;
  // readout form: rescaled frames unless a segment's rotation product leaves their range
  int staged = kStagePlain;
  if constexpr (!YM)
    staged = stage_bwd<T, HPW, true, true>(tc, H, ntr, v, beta, sel_c, dt, r, dy, al, om, c, s, saved, sP, sG, R,
                                           dsel, dsp);
  else
    stage_bwd<T, HPW, true>(tc, H, ntr, v, beta, sel_c, dt, r, dy, al, om, c, s, saved, sP, sG, R);
  if (staged == kStageMixed) stage_bwd<T, HPW, true>(tc, H, ntr, v, beta, sel_c, dt, r, dy, al, om, c, s, saved, sP, sG, R);
  const bool rs = staged == kStageRs;
  __syncthreads();
  stamp(1);

  // ---- reverse pass ----
  float mr[DPL], mi[DPL], lr[DPL], li[DPL];
  float dGr = 0.0f, dGi = 0.0f;
  {
    const float2* dp = dsn + chh * D + sub * DPL;
#pragma unroll
    for (int jj = 0; jj < DPL; ++jj) {
      const float2 ds = dp[jj];
      const float2 s0 = sp[jj];
      mr[jj] = ds.x;
      mi[jj] = ds.y;
      lr[jj] = li[jj] = 0.0f;
      dGr = fmaf(ds.x, s0.x, fmaf(ds.y, s0.y, dGr));
      dGi = fmaf(ds.y, s0.x, fmaf(-ds.x, s0.y, dGi));
    }
    dGr = group_sum<LPH>(dGr);
    dGi = group_sum<LPH>(dGi);
  }
  // Segments run last to first; the next segment's k / q rows and z checkpoint
  // are loaded while the current one is processed (two buffers, alternating).
  struct SegBuf {
    RowVec<T, DPL> k[CK], q[CK], g[YM ? CK : 1];
    float2 z0[DPL];
  };
  auto load_seg = [&](SegBuf& R, int seg) {
    const int tb = seg * CK;
#pragma unroll
    for (int i = 0; i < CK; ++i) {
      R.k[i].load(ks, min((tb + i) * rowb, slim));
      R.q[i].load(qs, min((tb + i) * rowq, slimq));
      if constexpr (YM) R.g[i].load(gs, min((tb + i) * rowq, slimq));
    }
    load_zck<T, DPL>(zck, ck0 + int64_t(seg) * D, R.z0);
  };
  auto run_seg = [&](const SegBuf& R, int seg) {
    const int tb = seg * CK;
    // z_{tb-1+i} for i = 0..CK, recomputed with the staged e_t (no reductions);
    // the unpacked k rows are kept for the reverse steps
    float zbr[CK + 1][DPL], zbi[CK + 1][DPL], kr[CK][DPL];
#pragma unroll
    for (int jj = 0; jj < DPL; ++jj) {
      zbr[0][jj] = R.z0[jj].x;
      zbi[0][jj] = R.z0[jj].y;
    }
#pragma unroll
    for (int i = 0; i < CK; ++i) {
      // slots past the last token are inert: a = 1, e = 0
      const float4 s0 = s.S0[(tb + i) * HPW + hh];
      R.k[i].unpack(kr[i]);
#pragma unroll
      for (int jj = 0; jj < DPL; ++jj) {
        zbr[i + 1][jj] = fmaf(s0.x, zbr[i][jj], fmaf(-s0.y, zbi[i][jj], s0.z * kr[i][jj]));
        zbi[i + 1][jj] = fmaf(s0.x, zbi[i][jj], fmaf(s0.y, zbr[i][jj], s0.w * kr[i][jj]));
      }
    }
#pragma unroll
    for (int i = CK - 1; i >= 0; --i) {
      const int t = tb + i;
      if (t < tc.nt) {
        const int p = t * HPW + hh;
        const float4 s0 = s.S0[p], s1 = s.S1[p], s2 = s.S2[p], pv = sP[p];
        const float ar = s0.x, ai = s0.y, er = s0.z, ei = s0.w, bb = s1.x;
        const float pcr = pv.z, pci = pv.w;
        const float* kk = kr[i];
        float qq[DPL], gq[DPL];
        R.q[i].unpack(qq);
        if constexpr (YM) R.g[i].unpack(gq);
        constexpr int NRED = YM ? 8 : 6;
        float red[NRED];
#pragma unroll
        for (int x = 0; x < NRED; ++x) red[x] = 0.0f;
        float dqv[DPL];
        // dq = Re(conj(f) Y_t), Y_t = z_t + g_{t-1} c^_t, f = (s1.y, -s1.z), g_{t-1} = (s2.z, s2.w):
        // the c^ part's weight conj(f) g_{t-1} is formed once per token
        const float wcr = s2.z * s1.y + s2.w * s1.z, wci = s2.z * s1.z - s2.w * s1.y;
        const float bpcr = bb * pcr, bpci = bb * pci;
#pragma unroll
        for (int jj = 0; jj < DPL; ++jj) {
          if constexpr (YM) {
            // delta g_t = sum_d dY_t[d] conj(c^_{t+1}[d]), c^_{t+1} before the rebuild below
            red[6] = fmaf(qq[jj], cr[jj], fmaf(gq[jj], ci[jj], red[6]));
            red[7] = fmaf(gq[jj], cr[jj], fmaf(-qq[jj], ci[jj], red[7]));
          }
          // c^_t = c^_{t+1} + beta pc k
          cr[jj] = fmaf(bpcr, kk[jj], cr[jj]);
          ci[jj] = fmaf(bpci, kk[jj], ci[jj]);
          if constexpr (YM) {
            // mu += dY_t; lambda += conj(g_t) dY_t
            mr[jj] += qq[jj];
            mi[jj] += gq[jj];
            lr[jj] = fmaf(s2.x, qq[jj], fmaf(s2.y, gq[jj], lr[jj]));
            li[jj] = fmaf(s2.x, gq[jj], fmaf(-s2.y, qq[jj], li[jj]));
          } else {
            dqv[jj] = fmaf(zbr[i + 1][jj], s1.y, fmaf(zbi[i + 1][jj], s1.z, fmaf(cr[jj], wcr, ci[jj] * wci)));
            mr[jj] = fmaf(s1.y, qq[jj], mr[jj]);
            mi[jj] = fmaf(s1.z, qq[jj], mi[jj]);
            lr[jj] = fmaf(s2.x, qq[jj], lr[jj]);
            li[jj] = fmaf(s2.y, qq[jj], li[jj]);
          }
          red[0] = fmaf(mr[jj], kk[jj], red[0]);
          red[1] = fmaf(mi[jj], kk[jj], red[1]);
          red[2] = fmaf(mr[jj], zbr[i][jj], fmaf(mi[jj], zbi[i][jj], red[2]));
          red[3] = fmaf(mi[jj], zbr[i][jj], fmaf(-mr[jj], zbi[i][jj], red[3]));
          red[4] = fmaf(lr[jj], kk[jj], red[4]);
          red[5] = fmaf(li[jj], kk[jj], red[5]);
        }
#pragma unroll
        for (int x = 0; x < NRED; ++x) red[x] = group_sum<LPH>(red[x]);
        // dw = mu.k, mk = conj(a) dw, sl = lambda.k
        const float dwr = red[0], dwi = red[1], slr = red[4], sli = red[5];
        const float mkr = ar * dwr + ai * dwi, mki = ar * dwi - ai * dwr;
        // dk = mu.e - beta (z_{t-1}.mk + c^_t.(lambda.k) + lambda.pc), e = w - beta a p:
        // the mu.w and conj(a) mu . p terms combine into mu.e
        const float bmkr = bb * mkr, bmki = bb * mki, bslr = bb * slr, bsli = bb * sli;
        float dkv[DPL];
#pragma unroll
        for (int jj = 0; jj < DPL; ++jj) {
          float acc = mr[jj] * er;
          acc = fmaf(mi[jj], ei, acc);
          acc = fmaf(-zbr[i][jj], bmkr, acc);
          acc = fmaf(-zbi[i][jj], bmki, acc);
          acc = fmaf(-cr[jj], bslr, acc);
          acc = fmaf(-ci[jj], bsli, acc);
          acc = fmaf(-lr[jj], bpcr, acc);
          dkv[jj] = fmaf(-li[jj], bpci, acc);
          const float m_r = ar * mr[jj] + ai * mi[jj], m_i = ar * mi[jj] - ai * mr[jj];
          mr[jj] = fmaf(-bmkr, kk[jj], m_r);
          mi[jj] = fmaf(-bmki, kk[jj], m_i);
          lr[jj] = fmaf(-bslr, kk[jj], lr[jj]);
          li[jj] = fmaf(-bsli, kk[jj], li[jj]);
        }
        if constexpr (YM)
          store_dk_dq<T, LPH, DPL, false>(rows, rows_pre, hok, hh, dkv, dkv, dks, dkps, dqs, dqps, t * rowb,
                                          t * rowp);
        else
          store_dk_dq<T, LPH, DPL, true>(rows, rows_pre, hok, hh, dkv, dqv, dks, dkps, dqs, dqps, t * rowb,
                                         t * rowp);
        // the token's scalar gradients are formed in the epilogue (one lane per
        // token, not LPH): keep mu.z_{t-1}, dw and sl in the slots this step
        // has read (a stays for the epilogue's psi recurrence)
        if (sub == 0) {
          s.S0[p] = make_float4(ar, ai, red[2], red[3]);
          s.S1[p] = make_float4(dwr, dwi, slr, sli);
          if constexpr (YM) sG[p] = make_float4(red[6], red[7], 0.0f, 0.0f);  // delta g_t
        }
      }
    }
  };
  // The same step in the rescaled frames (readout form; slots in the RS layout).
  // It leaves S0 = (mu^ conj(z~_i), mu^.k) and S1 = (lambda.k, pc); the
  // epilogue converts them back to the true scale.
  auto run_seg_rs = [&](const SegBuf& R, int seg) {
    const int tb = seg * CK;
    // z~_i for i = 0..CK: z~_{i+1} = z~_i + (e/G_{i+1}) k (no reductions); the k rows stay unpacked
    float zbr[CK + 1][DPL], zbi[CK + 1][DPL], kr[CK][DPL];
#pragma unroll
    for (int jj = 0; jj < DPL; ++jj) {
      zbr[0][jj] = R.z0[jj].x;
      zbi[0][jj] = R.z0[jj].y;
    }
#pragma unroll
    for (int i = 0; i < CK; ++i) {
      const float4 s0 = s.S0[(tb + i) * HPW + hh];
      R.k[i].unpack(kr[i]);
#pragma unroll
      for (int jj = 0; jj < DPL; ++jj) {
        zbr[i + 1][jj] = fmaf(s0.x, kr[i][jj], zbr[i][jj]);
        zbi[i + 1][jj] = fmaf(s0.y, kr[i][jj], zbi[i][jj]);
      }
    }
    // mu into this segment's frame: mu^ = conj(G_CK) mu (G_CK: Re in the slot of
    // an even token, Im in the slot of an odd one)
    {
      const float Gr = s.S1[(tb + CK - 2) * HPW + hh].w, Gi = s.S1[(tb + CK - 1) * HPW + hh].w;
#pragma unroll
      for (int jj = 0; jj < DPL; ++jj) {
        const float nr = fmaf(Gr, mr[jj], Gi * mi[jj]);
        mi[jj] = fmaf(Gr, mi[jj], -Gi * mr[jj]);
        mr[jj] = nr;
      }
    }
#pragma unroll
    for (int i = CK - 1; i >= 0; --i) {
      const int t = tb + i;
      if (t < tc.nt) {
        const int p = t * HPW + hh;
        const float4 s0 = s.S0[p], s1 = s.S1[p], s2 = s.S2[p];
        const float ezr = s0.x, ezi = s0.y, fmr = s0.z, fmi = s0.w, bb = s1.x;
        const float pcr = s1.y, pci = s1.z;
        const float* kk = kr[i];
        float qq[DPL];
        R.q[i].unpack(qq);
        float red[6];
#pragma unroll
        for (int x = 0; x < 6; ++x) red[x] = 0.0f;
        float dqv[DPL];
        const float bpcr = bb * pcr, bpci = bb * pci;
#pragma unroll
        for (int jj = 0; jj < DPL; ++jj) {
          // c^_t = c^_{t+1} + beta pc k
          cr[jj] = fmaf(bpcr, kk[jj], cr[jj]);
          ci[jj] = fmaf(bpci, kk[jj], ci[jj]);
          // dq = Re(z_t conj(f)) + Re(c^_t conj(conj(g_{t-1}) f))
          dqv[jj] = fmaf(zbr[i + 1][jj], fmr, fmaf(zbi[i + 1][jj], fmi, fmaf(cr[jj], s2.z, ci[jj] * s2.w)));
          mr[jj] = fmaf(fmr, qq[jj], mr[jj]);
          mi[jj] = fmaf(fmi, qq[jj], mi[jj]);
          lr[jj] = fmaf(s2.x, qq[jj], lr[jj]);
          li[jj] = fmaf(s2.y, qq[jj], li[jj]);
          red[0] = fmaf(mr[jj], kk[jj], red[0]);
          red[1] = fmaf(mi[jj], kk[jj], red[1]);
          red[2] = fmaf(mr[jj], zbr[i][jj], fmaf(mi[jj], zbi[i][jj], red[2]));
          red[3] = fmaf(mi[jj], zbr[i][jj], fmaf(-mr[jj], zbi[i][jj], red[3]));
          red[4] = fmaf(lr[jj], kk[jj], red[4]);
          red[5] = fmaf(li[jj], kk[jj], red[5]);
        }
#pragma unroll
        for (int x = 0; x < 6; ++x) red[x] = group_sum<LPH>(red[x]);
        // mu^.k, lambda.k
        const float bdwr = bb * red[0], bdwi = bb * red[1], bslr = bb * red[4], bsli = bb * red[5];
        float dkv[DPL];
#pragma unroll
        for (int jj = 0; jj < DPL; ++jj) {
          float acc = mr[jj] * ezr;
          acc = fmaf(mi[jj], ezi, acc);
          acc = fmaf(-zbr[i][jj], bdwr, acc);
          acc = fmaf(-zbi[i][jj], bdwi, acc);
          acc = fmaf(-cr[jj], bslr, acc);
          acc = fmaf(-ci[jj], bsli, acc);
          acc = fmaf(-lr[jj], bpcr, acc);
          dkv[jj] = fmaf(-li[jj], bpci, acc);
          mr[jj] = fmaf(-bdwr, kk[jj], mr[jj]);
          mi[jj] = fmaf(-bdwi, kk[jj], mi[jj]);
          lr[jj] = fmaf(-bslr, kk[jj], lr[jj]);
          li[jj] = fmaf(-bsli, kk[jj], li[jj]);
        }
        store_dk_dq<T, LPH, DPL, true>(rows, rows_pre, hok, hh, dkv, dqv, dks, dkps, dqs, dqps, t * rowb, t * rowp);
        if (sub == 0) {
          s.S0[p] = make_float4(red[2], red[3], red[0], red[1]);
          s.S1[p] = make_float4(red[4], red[5], pcr, pci);
        }
      }
    }
  };
  auto drive = [&](auto run) {
    SegBuf bufA, bufB;
    int seg = ntr / CK - 1;
    load_seg(bufA, seg);
    while (true) {
      load_seg(bufB, max(seg - 1, 0));  // unconditional: a clamped reload past segment 0 is harmless
      __builtin_amdgcn_sched_barrier(0);
      run(bufA, seg);
      if (--seg < 0) break;
      load_seg(bufA, max(seg - 1, 0));
      __builtin_amdgcn_sched_barrier(0);
      run(bufB, seg);
      if (--seg < 0) break;
    }
  };
  if constexpr (!YM)
    drive([&](const SegBuf& R, int seg) {
      if (rs)
        run_seg_rs(R, seg);
      else
        run_seg(R, seg);
    });
  else
    drive(run_seg);
  __syncthreads();
  stamp(2);
  // ---- per-token scalar gradients and dynamics backward: lane = (head j, block of TPB tokens) ----
  // Slots now hold S0 = (a, mu.z_{t-1}), S1 = (dw, sl), S2 = (h, g_{t-1}), P = (p, pc),
  // G = (delta g, Y.q); after the rescaled step S0 = (mu^ conj(z~_i), mu^.k),
  // S1 = (sl, pc), P = (p, a), G = (delta g, g_{t-1}), and per token, with G_i and
  // G_{i+1} of its segment, mu.k = (mu^.k) / conj(G_{i+1}) and mu conj(z_{t-1}) =
  // (mu^ conj(z~_i)) conj(G_i) / conj(G_{i+1}).  psi_t, the adjoint of the rotation product g_t, runs
  // backward: psi_t = delta g_t + conj(a_{t+1}) psi_{t+1} (+ dG at the chunk's last
  // token), psi_nt = 0; each lane composes its block, a segmented suffix scan over
  // the head's NB blocks joins them, and slabs of kWave tokens run last to first.
  {
    constexpr int NB = kWave / HPW, TPB = HPW;
    static_assert(NB == LPH, "the epilogue's head of a lane is its reverse-pass head");
    const int j = lane / NB, blk = lane % NB;
    const int hj = tc.hbase + j;
    const bool jok = hj < H;
    const int hjl = jok ? hj : H - 1;
    const float alj = al, omj = om;  // head j is the reverse pass's head hh
    const int tend = round_up(ntr, kWave);  // staged slots: [0, tend)
    constexpr int SB = CK / TPB;            // blocks per segment
    // a_t of a slot in either layout
    const auto a_of = [&](int p) {
      if (rs) {
        const float4 v4 = sP[p];
        return make_float2(v4.z, v4.w);
      }
      const float4 v4 = s.S0[p];
      return make_float2(v4.x, v4.y);
    };
    float dal = 0.0f, dom = 0.0f;
    float pinr = 0.0f, pini = 0.0f;  // psi at the first token right of the slab
    for (int tl = tend - kWave; tl >= 0; tl -= kWave) {
      const int t0 = tl + blk * TPB;
      // the slab's per-token inputs, requested before the psi pass so that its
      // latency covers theirs (rows past the last token clamped, unused)
      float lbb[TPB], lv0[TPB], lv1[TPB], ldt[TPB], lrr[TPB], lg0[TPB], lg1[TPB];
#pragma unroll
      for (int i = 0; i < TPB; ++i) {
        const int tt = min(t0 + i, tc.nt - 1);
        const int64_t ee = (tc.row0 + tt) * H + hjl;
        // beta per real head (the R virtual heads of its state rows share it)
        lbb[i] = T::load(beta + (tc.row0 + tt) * (H / R) + hjl / R);
        lv0[i] = T::load(v + 2 * ee);
        lv1[i] = T::load(v + 2 * ee + 1);
        ldt[i] = lrr[i] = lg0[i] = lg1[i] = 0.0f;
        if constexpr (!YM) {
          if constexpr (!kAbar) ldt[i] = T::load(dt + ee);
          lrr[i] = T::load(r + ee);  // ABar form: vp_t
          if (!rs) {
            lg0[i] = T::load(dy + 2 * ee);
            lg1[i] = T::load(dy + 2 * ee + 1);
          }
        }
      }
      // the block with zero input: psi_t = X_t + A_t psi_{t0+TPB}
      float xr[TPB], xi[TPB], Ar[TPB], Ai[TPB];
      float2 aa[TPB];  // a_t of the block's tokens
      {
        float2 an = t0 + TPB < tend ? a_of((t0 + TPB) * HPW + j) : make_float2(1.0f, 0.0f);
        float cxr = 0.0f, cxi = 0.0f, car = 1.0f, cai = 0.0f;
#pragma unroll
        for (int i = TPB - 1; i >= 0; --i) {
          const int t = t0 + i;
          const int p = t * HPW + j;
          const float4 gv = sG[p];
          float dgr = gv.x, dgi = gv.y;
          if (t == tc.nt - 1) {
            dgr += dGr;
            dgi += dGi;
          }
          // (X, A) <- (dg + conj(an) X, conj(an) A)
          const float nxr = dgr + an.x * cxr + an.y * cxi, nxi = dgi + an.x * cxi - an.y * cxr;
          const float nar = an.x * car + an.y * cai, nai = an.x * cai - an.y * car;
          cxr = nxr;
          cxi = nxi;
          car = nar;
          cai = nai;
          xr[i] = cxr;
          xi[i] = cxi;
          Ar[i] = car;
          Ai[i] = cai;
          an = a_of(p);
          aa[i] = an;
        }
      }
      // rescaled step: the factors back to the true scale, 1 / conj(G_{i+1}) and
      // conj(G_i) / conj(G_{i+1}), from the segment's products over the block's
      // tokens and a scan over the SB blocks of the segment
      float cfr[TPB], cfi[TPB], gar[TPB], gai[TPB];
      if (rs) {
        float Pr[TPB], Pi[TPB], br = 1.0f, bi = 0.0f;
#pragma unroll
        for (int i = 0; i < TPB; ++i) {
          cmul_acc(br, bi, aa[i].x, aa[i].y);
          Pr[i] = br;
          Pi[i] = bi;
        }
        float ir = br, ii = bi;
        for_shifts<SB>([&](auto offc) {
          constexpr int off = decltype(offc)::value;
          const float yr = seg_shift_up<SB, off>(ir), yi = seg_shift_up<SB, off>(ii);
          if (blk % SB >= off) cmul_acc(ir, ii, yr, yi);
        });
        float sgr = 1.0f, sgi = 0.0f;
        if constexpr (SB > 1) {
          sgr = seg_shift_up<SB, 1>(ir);
          sgi = seg_shift_up<SB, 1>(ii);
          if (blk % SB == 0) {
            sgr = 1.0f;
            sgi = 0.0f;
          }
        }
#pragma unroll
        for (int i = 0; i < TPB; ++i) {
          float g0r = sgr, g0i = sgi, g1r = sgr, g1i = sgi;  // G_i, G_{i+1}
          if (i > 0) cmul_acc(g0r, g0i, Pr[i - 1], Pi[i - 1]);
          cmul_acc(g1r, g1i, Pr[i], Pi[i]);
          const float inv = __builtin_amdgcn_rcpf(g1r * g1r + g1i * g1i);
          cfr[i] = g1r * inv;
          cfi[i] = g1i * inv;
          gar[i] = g0r * cfr[i] + g0i * cfi[i];
          gai[i] = g0r * cfi[i] - g0i * cfr[i];
        }
      }
      // suffix scan over the head's blocks: (SX, SA) maps psi right of block
      // blk + span - 1 to psi at the block's first token
      float sxr = xr[0], sxi = xi[0], sar = Ar[0], sai = Ai[0];
      for_shifts<NB>([&](auto offc) {
        constexpr int off = decltype(offc)::value;
        const float yxr = seg_shift_down<NB, off>(sxr), yxi = seg_shift_down<NB, off>(sxi);
        const float yar = seg_shift_down<NB, off>(sar), yai = seg_shift_down<NB, off>(sai);
        if (blk + off < NB) {
          // (SX, SA) o (YX, YA): SX + SA YX, SA YA
          const float nxr = sxr + (sar * yxr - sai * yxi), nxi = sxi + (sar * yxi + sai * yxr);
          const float nar = sar * yar - sai * yai, nai = sar * yai + sai * yar;
          sxr = nxr;
          sxi = nxi;
          sar = nar;
          sai = nai;
        }
      });
      // psi right of this block: the next block's inclusive map applied to the slab's input
      float rxr = seg_shift_down<NB, 1>(sxr), rxi = seg_shift_down<NB, 1>(sxi);
      float rar = seg_shift_down<NB, 1>(sar), rai = seg_shift_down<NB, 1>(sai);
      if (blk == NB - 1) {
        rxr = rxi = 0.0f;
        rar = 1.0f;
        rai = 0.0f;
      }
      const float per = rxr + (rar * pinr - rai * pini), pei = rxi + (rar * pini + rai * pinr);
      // psi at the slab's first token, for the slab to the left (block 0 of the head)
      const float hxr = sxr + (sar * pinr - sai * pini), hxi = sxi + (sar * pini + sai * pinr);
      pinr = __shfl(hxr, j * NB, kWave);
      pini = __shfl(hxi, j * NB, kWave);
#pragma unroll
      for (int i = 0; i < TPB; ++i) {
        const int t = t0 + i;
        if (t < tc.nt && jok) {
          const int64_t e = (tc.row0 + t) * H + hj;
          const int p = t * HPW + j;
          const float4 s0 = s.S0[p], s1 = s.S1[p], s2 = s.S2[p], pv = sP[p], gv = sG[p];
          const float psr = xr[i] + (Ar[i] * per - Ai[i] * pei), psi = xi[i] + (Ar[i] * pei + Ai[i] * per);
          float ar = s0.x, ai = s0.y, mzr = s0.z, mzi = s0.w, dwr = s1.x, dwi = s1.y, slr = s1.z, sli = s1.w;
          float pcr = pv.z, pci = pv.w, gpr = s2.z, gpi = s2.w;
          if (rs) {
            ar = aa[i].x;
            ai = aa[i].y;
            mzr = s0.x * gar[i] - s0.y * gai[i];
            mzi = s0.x * gai[i] + s0.y * gar[i];
            dwr = s0.z * cfr[i] - s0.w * cfi[i];
            dwi = s0.z * cfi[i] + s0.w * cfr[i];
            slr = s1.x;
            sli = s1.y;
            pcr = s1.z;
            pci = s1.w;
            gpr = gv.z;
            gpi = gv.w;
          }
          const float pr = pv.x, pi = pv.y;
          const float bb = lbb[i];
          // d a_t = mu.z_{t-1} - beta (mu.k) conj(p) + psi_t conj(g_{t-1})
          const float dar = mzr - bb * (pr * dwr + pi * dwi) + (gpr * psr + gpi * psi);
          const float dai = mzi - bb * (pr * dwi - pi * dwr) + (gpr * psi - gpi * psr);
          // d beta (erase part) = -(p . conj(a) dw) - (pc . sl)
          const float mkr = ar * dwr + ai * dwi, mki = ar * dwi - ai * dwr;
          const float dbe = -(pr * mkr + pi * mki) - (pcr * slr + pci * sli);
          const float v0 = lv0[i], v1 = lv1[i];
          if constexpr (YM) {
            // SSD form: d A_bar_t = d a_t (into ddt's place, (re, im) pairs), dV = beta dw,
            // dbeta = erase part + dw . V (w = beta V)
            store_pair<T>(ddt + 2 * e, dar, dai);
            T::store(dv + 2 * e, bb * dwr);
            T::store(dv + 2 * e + 1, bb * dwi);
            const float db = dbe + (dwr * v0 + dwi * v1);
            if (R > 1)
              dbp[e] = db;  // summed over the head's rows by the row-sum kernel
            else
              T::store(dbeta + e, db);
            continue;
          }
          const float g0 = lg0[i], g1 = lg1[i];
          if constexpr (kAbar) {
            // gate-level form (w = beta vp v): d A_bar_t = d a_t ((re, im) pairs in ddt's place),
            // d vp_t = beta (dw . v) in dr's place, dv = beta vp dw, dbeta = erase part + vp (dw . v)
            const float vpv = lrr[i];
            const float dwv = dwr * v0 + dwi * v1;
            store_pair<T>(ddt + 2 * e, dar, dai);
            T::store(dr + e, bb * dwv);
            T::store(dv + 2 * e, bb * vpv * dwr);
            T::store(dv + 2 * e + 1, bb * vpv * dwi);
            // R > 1: the state row's parts of dbeta and dsel, summed over the head's rows by the row-sum kernel
            if (R > 1) {
              dbp[e] = dbe + vpv * dwv;
              if (!rs) dsp[e] = g0 * gv.z + g1 * gv.w;
            } else {
              T::store(dbeta + e, dbe + vpv * dwv);
              if (!rs) T::store(dsel + e, g0 * gv.z + g1 * gv.w);  // (rescaled: stored by the staging)
            }
            continue;
          }
          const float dtv = ldt[i], rrv = lrr[i];
          const Transition tr = cayley_gated(dtv, rrv, alj, omj, c);
          const float dwv = dwr * v0 + dwi * v1;
          const DynGrad g = cayley_gated_bwd(dtv, rrv, alj, omj, c, dar, dai, bb * dwv);
          T::store(dv + 2 * e, bb * tr.vp * dwr);
          T::store(dv + 2 * e + 1, bb * tr.vp * dwi);
          T::store(dbeta + e, dbe + tr.vp * dwv);
          if (!rs) T::store(dsel + e, g0 * gv.z + g1 * gv.w);  // (rescaled: stored by the staging)
          T::store(ddt + e, g.ddt);
          T::store(dr + e, g.dr);
          dal += g.dalpha;
          dom += g.domega;
        }
      }
    }
    if constexpr (!YM && !kAbar) {
      dal = group_sum<NB>(dal);
      dom = group_sum<NB>(dom);
      if (blk == 0 && jok) dhead_parts[(int64_t(tc.b) * NC + tc.chunk) * H + hj] = make_float2(dal, dom);
    }
  }
  stamp(3);
  if (stamping && threadIdx.x == 0) {
#pragma unroll
    for (int i = 0; i < kBwdMainStamps; ++i) stamps[int64_t(blockIdx.x) * kBwdMainStamps + i] = ts[i];
  }
}

// ---------------------------------------------------------------------------
// B4: d alpha[h], d omega[h] = sum over (b, chunk) of the per-chunk parts.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void fused_bwd_heads_kernel(const float2* __restrict__ parts,
                                                             float* __restrict__ dalpha,
                                                             float* __restrict__ domega, int BNC, int H) {
  __shared__ float sa[256], so[256];
  const int h = blockIdx.x;
  float a = 0.0f, o = 0.0f;
  for (int i = threadIdx.x; i < BNC; i += 256) {
    const float2 p = parts[int64_t(i) * H + h];
    a += p.x;
    o += p.y;
  }
  sa[threadIdx.x] = a;
  so[threadIdx.x] = o;
  __syncthreads();
  for (int s = 128; s > 0; s >>= 1) {
    if (int(threadIdx.x) < s) {
      sa[threadIdx.x] += sa[threadIdx.x + s];
      so[threadIdx.x] += so[threadIdx.x + s];
    }
    __syncthreads();
  }
  if (threadIdx.x == 0) {
    dalpha[h] = sa[0];
    domega[h] = so[0];
  }
}

// ---------------------------------------------------------------------------
// R > 1 state rows per head (the SSD and gate-level forms): dk and dbeta (the
// gate-level form: also dq and dsel) of each head are the sums of the fp32
// partials the main pass wrote, dk[n, h, :] = sum_j dkp[n, h P + j, :] over the
// head's P partial rows (P = R, or R / HPW where the main pass already summed
// each wave's HPW rows), dbeta[n, h] = sum_j dbp[n, h R + j] (n = token), dq
// and dsel alike from dqp and dsp, in a fixed order.  One thread per 4
// consecutive elements of dk (D % 4 == 0); the first of a row's threads also
// sums dbeta (and dsel).
// ---------------------------------------------------------------------------
template <typename T>
__global__ __launch_bounds__(256) void rows_sum_kernel(const float* __restrict__ dkp,
                                                       const float* __restrict__ dbp,
                                                       const float* __restrict__ dqp,
                                                       const float* __restrict__ dsp,
                                                       typename T::raw* __restrict__ dk,
                                                       typename T::raw* __restrict__ dbeta,
                                                       typename T::raw* __restrict__ dq,
                                                       typename T::raw* __restrict__ dsel, int64_t n_rows,
                                                       int R, int P, int D) {
  const int64_t i = int64_t(blockIdx.x) * 256 + threadIdx.x;  // (token, head, 8 elements)
  const int qd = D / 8;
  if (i >= n_rows * qd) return;
  const int64_t row = i / qd;  // token * Hk + head
  const int d0 = int(i - row * qd) * 8;
  const auto sum8 = [&](const float* x, typename T::raw* o) {
    float a[8] = {};
    for (int j = 0; j < P; ++j) {
      const float4* src = reinterpret_cast<const float4*>(x + (row * P + j) * D + d0);
      const float4 v0 = src[0], v1 = src[1];
      a[0] += v0.x;
      a[1] += v0.y;
      a[2] += v0.z;
      a[3] += v0.w;
      a[4] += v1.x;
      a[5] += v1.y;
      a[6] += v1.z;
      a[7] += v1.w;
    }
    store_row<T, 8>(o + row * D + d0, a);
  };
  sum8(dkp, dk);
  if (dqp) sum8(dqp, dq);
  if (d0 == 0) {
    // the rows' partials of dbeta (and dsel) in order, four at a time where R allows
    const auto sum_r = [&](const float* x) {
      float b = 0.0f;
      if (R % 4 == 0) {
        const float4* src = reinterpret_cast<const float4*>(x + row * R);
        for (int j = 0; j < R / 4; ++j) {
          const float4 v = src[j];
          b = (((b + v.x) + v.y) + v.z) + v.w;
        }
      } else {
        for (int j = 0; j < R; ++j) b += x[row * R + j];
      }
      return b;
    };
    T::store(dbeta + row, sum_r(dbp));
    if (dsp) T::store(dsel + row, sum_r(dsp));
  }
}

}  // namespace cdssm

// ---------------------------------------------------------------------------
// C-ABI
// ---------------------------------------------------------------------------
namespace {
using namespace cdssm;

struct BwdLayout {
  int NC, S, NSEG;
  int64_t n_lam, n_dsn, n_segA, n_segX, n_parts, n_cc;  // float2 counts
  int64_t total() const { return n_lam + n_dsn + n_segA + n_segX + n_parts + n_cc; }
};

BwdLayout bwd_layout(int64_t B, int64_t L, int64_t H, int64_t D, int64_t chunk) {
  BwdLayout w;
  w.NC = int((L + chunk - 1) / chunk);
  w.S = (w.NC + kBwdSeg - 1) / kBwdSeg;
  w.n_lam = B * w.NC * H * D;
  w.n_dsn = B * w.NC * H * D;
  w.n_segA = B * H * w.S;
  w.n_segX = B * H * w.S * D;
  w.n_parts = B * w.NC * H;
  // one-launch correction adjoint + reverse carry: look-back area per (b,
  // segment of kOnePassW chunks, h): map X (D), left-end state (D), A, flag
  w.NSEG = (w.NC + kOnePassW - 1) / kOnePassW;
  w.n_cc = B * w.NSEG * H * (2 * D + 2) + kCtlWords;
  return w;
}

// R > 1 state rows per head, after the layout above, 16-byte aligned: the fp32
// partials dkp (B, L, Hk P, D) and dbp (B, L, Hk R) of the SSD form; dkp, dqp
// (B, L, Hk P, D), dbp and dsp (B, L, Hk R) of the gate-level form (Hk real
// heads; P partial rows per head: R, or R / HPW where the main pass sums each
// wave's HPW rows first).
int64_t rows_partials_offset_floats(const BwdLayout& w) { return 2 * ((w.total() + 1) / 2) * 2; }
int64_t rows_partials_per_head(int64_t D, int64_t R) {
  const int64_t hpw = D == 64 ? BwdCfg<64>::HPW : BwdCfg<128>::HPW;
  return R % hpw == 0 ? R / hpw : R;
}
// one form's dk (or dq) and dbeta (or dsel) partials
int64_t rows_partials_floats(int64_t B, int64_t L, int64_t Hk, int64_t R, int64_t D) {
  return B * L * Hk * (rows_partials_per_head(D, R) * D + R);
}

// Phase-stamp buffer of the running cdssm_fused_scan_bwd_stamped call on this
// host thread (instrumentation only): device memory of `len` 8-byte words.
struct BwdStampRequest {
  unsigned long long* buf = nullptr;
  int64_t len = 0;
};
thread_local BwdStampRequest t_bstamps;

template <typename T, int D>
int launch_fused_bwd(const void* q, const void* k, const void* v, const void* beta, const void* sel_c,
                     const void* dt, const void* r, const float* alpha, const float* omega, float c,
                     const void* dy, const float* dh_final, const float* fwd_ws, void* dq, void* dk,
                     void* dv, void* dbeta, void* dsel, void* ddt, void* dr, float* dalpha,
                     float* domega, float* dh0, float* ws, int B, int L, int H, int Q,
                     hipStream_t stream, hipEvent_t* ev, int* carry_fused, bool cont, int R = 1) {
  using raw = typename T::raw;
  const BwdLayout w = bwd_layout(B, L, H, D, Q);
  const int NC = w.NC, S = w.S;
  constexpr int HPW = BwdCfg<D>::HPW, HPWC = BwdCorrCfg<D>::HPW;
  const int n_hg = (H + HPW - 1) / HPW, n_hgc = (H + HPWC - 1) / HPWC;
  const int64_t tiles = int64_t(B) * NC * n_hg, tiles_c = int64_t(B) * NC * n_hgc;
  const int64_t carry_threads = int64_t(B) * H * S * D;
  if (tiles > 0x7fffffff || tiles_c > 0x7fffffff || carry_threads / 256 > 0x7fffffff) {
    cdssm_host::set_error("cdssm_fused_scan_bwd: grid too large");
    return CDSSM_EINVAL;
  }
  const float2* states = reinterpret_cast<const float2*>(fwd_ws);
  const float2* gam = states + int64_t(B) * NC * H * D;
  const FwdLayout fw = fwd_layout(B, L, H, D, Q);
  const float4* saved = reinterpret_cast<const float4*>(states + fw.saved_offset());
  const float2* gsaved = states + fw.gsaved_offset();
  float2* lam0 = reinterpret_cast<float2*>(ws);
  float2* dsn = lam0 + w.n_lam;
  float2* segA = dsn + w.n_dsn;
  float2* segX = segA + w.n_segA;
  float2* parts = segX + w.n_segX;
  const float2* zck = states + fw.zck_offset();
  const float2* cend = states + fw.cend_offset();
  const int slots = round_up(Q, kWave) * HPW, slots_c = round_up(Q, kWave) * HPWC;

  // correction adjoint + reverse carry: one launch when one round of resident
  // workgroups holds every segment, else three (B1, fold, replay)
  int st = CDSSM_OK;
  bool fused = false;
  int64_t corr_words = 0;  // stamp words of the one-launch carry (instrumentation)
  if (cdssm_host::scan_path() != cdssm_host::kPathFour) {
    constexpr int SEGN = HPWC * D;
    const int64_t items = int64_t(w.NSEG) * B * n_hgc;
    static_assert(SEGN * sizeof(float2) <= 2 * kWave * HPWC * sizeof(float4), "lambda_0 fits a wave's slots");
    const size_t lds = size_t(kOnePassW) * 2 * slots_c * sizeof(float4) + size_t(kOnePassW) * HPWC * sizeof(float2) +
                       size_t(SEGN) * sizeof(float2) + 16;
    const int cap = cdssm_host::resident_capacity(reinterpret_cast<const void*>(&fused_bwd_corrcarry_kernel<T, D>),
                                                  kWave * kOnePassW, lds);
    if (cap > 0 && items <= cap) {
      float2* base = parts + w.n_parts;
      const int64_t nsd = int64_t(B) * w.NSEG * H * D, nsh = int64_t(B) * w.NSEG * H;
      CorrCarryArgs<T> a;
      a.q = (const raw*)q;
      a.k = (const raw*)k;
      a.beta = (const raw*)beta;
      a.sel_c = (const raw*)sel_c;
      a.dy = (const raw*)dy;
      a.gsaved = gsaved;
      a.gam = gam;
      a.dh_final = dh_final;
      a.dsn = dsn;
      a.dh0 = dh0;
      unsigned long long* flags = reinterpret_cast<unsigned long long*>(base + 2 * nsd + nsh);
      a.ob = OnePassBufs{base, base + nsd, base + 2 * nsd, flags, flags + nsh};
      a.L = L;
      a.H = H;
      a.Q = Q;
      a.NC = NC;
      a.NSEG = w.NSEG;
      a.n_hg = n_hgc;
      a.n_chain = B * n_hgc;
      a.R = R;
      a.stamps = nullptr;
      if (t_bstamps.buf) {
        // the main pass's words follow a region sized for one workgroup per (segment, batch, head), a bound
        // the caller can form without the pass's heads per wave
        corr_words = int64_t(w.NSEG) * B * H * kOnePassW * kBwdCorrStamps;
        const int64_t need = corr_words + int64_t(tiles) * kBwdMainStamps;
        if (t_bstamps.len < need) {
          cdssm_host::set_error("cdssm_fused_scan_bwd_stamped: %lld stamp words needed (%lld given)",
                                (long long)need, (long long)t_bstamps.len);
          return CDSSM_EINVAL;
        }
        a.stamps = t_bstamps.buf;
      }
      // a continuing call runs on the epoch the previous call's last workgroup left
      if (!cont) {
        hipLaunchKernelGGL(bwd_epoch_kernel, dim3(1), dim3(64), 0, stream, a.ob.ctl);
        st = cdssm_host::check_launch("cdssm_fused_scan_bwd/epoch");
        if (st) return st;
      }
      if (ev) (void)hipEventRecord(ev[0], stream);
      hipLaunchKernelGGL((fused_bwd_corrcarry_kernel<T, D>), dim3(unsigned(items)), dim3(kWave * kOnePassW), lds,
                         stream, a);
      st = cdssm_host::check_launch("cdssm_fused_scan_bwd/corrcarry");
      if (st) return st;
      if (ev)
        for (int i = 1; i < 4; ++i) (void)hipEventRecord(ev[i], stream);
      fused = true;
    } else if (cdssm_host::scan_path() == cdssm_host::kPathOne) {
      cdssm_host::set_error("cdssm_fused_scan_bwd: one-launch carry required but %lld segments exceed the %d "
                            "resident workgroups", (long long)items, cap);
      return CDSSM_EINVAL;
    }
  }
  if (carry_fused) *carry_fused = fused;
  if (!fused && t_bstamps.buf) {
    cdssm_host::set_error("cdssm_fused_scan_bwd_stamped: the shape runs the three-launch correction adjoint, "
                          "which has no phase stamps");
    return CDSSM_EINVAL;
  }
  if (!fused) {
    if (ev) (void)hipEventRecord(ev[0], stream);
    hipLaunchKernelGGL((fused_bwd_corr_kernel<T, D>), dim3(unsigned(tiles_c)), dim3(kWave),
                       size_t(slots_c) * 2 * sizeof(float4), stream, (const raw*)q, (const raw*)k,
                       (const raw*)beta, (const raw*)sel_c, (const raw*)dy, gsaved, lam0, L, H, Q, NC, n_hgc, R);
    st = cdssm_host::check_launch("cdssm_fused_scan_bwd/corr");
    if (st) return st;
    if (ev) (void)hipEventRecord(ev[1], stream);
    const unsigned cblocks = unsigned((carry_threads + 255) / 256);
    hipLaunchKernelGGL(fused_bwd_rfold_kernel, dim3(cblocks), dim3(256), 0, stream, (const float2*)lam0,
                       gam, segA, segX, B, NC, H, D, S);
    st = cdssm_host::check_launch("cdssm_fused_scan_bwd/rfold");
    if (st) return st;
    if (ev) (void)hipEventRecord(ev[2], stream);
    hipLaunchKernelGGL(fused_bwd_rreplay_kernel, dim3(cblocks), dim3(256), 0, stream, (const float2*)lam0,
                       gam, (const float2*)segA, (const float2*)segX, dh_final, dsn, dh0, B, NC, H, D, S);
    st = cdssm_host::check_launch("cdssm_fused_scan_bwd/rreplay");
    if (st) return st;
    if (ev) (void)hipEventRecord(ev[3], stream);
  }
  constexpr bool kAbar = IsABar<T>::value;
  const int64_t nrow = int64_t(B) * L * H;                                  // (token, virtual head) pairs
  const int64_t nprow = int64_t(B) * L * (H / R) * rows_partials_per_head(D, R);  // (token, partial row)
  float* dkp = R > 1 ? ws + rows_partials_offset_floats(w) : nullptr;
  float* dqp = R > 1 && kAbar ? dkp + nprow * D : nullptr;
  float* dbp = R > 1 ? dkp + nprow * D * (kAbar ? 2 : 1) : nullptr;
  float* dsp = R > 1 && kAbar ? dbp + nrow : nullptr;
  hipLaunchKernelGGL((fused_bwd_main_kernel<T, D>), dim3(unsigned(tiles)), dim3(kWave),
                     size_t(slots) * 5 * sizeof(float4), stream, (const raw*)q, (const raw*)k, (const raw*)v,
                     (const raw*)beta, (const raw*)sel_c, (const raw*)dt, (const raw*)r, alpha, omega, c,
                     (const raw*)dy, states, saved, (const float2*)dsn, zck, cend, (raw*)dq, (raw*)dk, (raw*)dv,
                     (raw*)dbeta, (raw*)dsel, (raw*)ddt, (raw*)dr, parts, L, H, Q, NC, fw.NCK, n_hg, R, dkp, dbp,
                     dqp, dsp, t_bstamps.buf ? t_bstamps.buf + corr_words : nullptr);
  st = cdssm_host::check_launch("cdssm_fused_scan_bwd/main");
  if (st) return st;
  if (ev) (void)hipEventRecord(ev[4], stream);
  if constexpr (GivenA<T>::value) {  // SSD and gate-level forms: no per-head dynamics parameters
    if (R > 1) {
      const int64_t n_rows = int64_t(B) * L * (H / R);
      const int64_t threads = n_rows * (D / 8);
      hipLaunchKernelGGL(rows_sum_kernel<T>, dim3(unsigned((threads + 255) / 256)), dim3(256), 0, stream,
                         (const float*)dkp, (const float*)dbp, (const float*)dqp, (const float*)dsp, (raw*)dk,
                         (raw*)dbeta, (raw*)dq, (raw*)dsel, n_rows, R, int(rows_partials_per_head(D, R)), D);
      st = cdssm_host::check_launch(kAbar ? "cdssm_fused_scan_bwd_abar/rows_sum" : "cdssm_ssd_scan_bwd/rows_sum");
    }
    if (ev) (void)hipEventRecord(ev[5], stream);
    return st;
  }
  hipLaunchKernelGGL(fused_bwd_heads_kernel, dim3(unsigned(H)), dim3(256), 0, stream,
                     (const float2*)parts, dalpha, domega, B * NC, H);
  st = cdssm_host::check_launch("cdssm_fused_scan_bwd/heads");
  if (ev) (void)hipEventRecord(ev[5], stream);
  return st;
}

}  // namespace

int cdssm_host::bwd_lookback_status(bool clear, unsigned* out) {
  unsigned v = 0;
  if (hipMemcpyFromSymbol(&v, HIP_SYMBOL(cdssm::g_bwd_status), sizeof(v), 0, hipMemcpyDeviceToHost) != hipSuccess) {
    cdssm_host::set_error("cdssm_lookback_status: reading the backward status word failed: %s",
                          hipGetErrorString(hipGetLastError()));
    return CDSSM_EHIP;
  }
  if (clear && v) {
    const unsigned zero = 0;
    if (hipMemcpyToSymbol(HIP_SYMBOL(cdssm::g_bwd_status), &zero, sizeof(zero), 0, hipMemcpyHostToDevice) !=
        hipSuccess) {
      cdssm_host::set_error("cdssm_lookback_status: clearing the backward status word failed: %s",
                            hipGetErrorString(hipGetLastError()));
      return CDSSM_EHIP;
    }
  }
  *out = v;
  return CDSSM_OK;
}

extern "C" int64_t cdssm_fused_scan_bwd_workspace_bytes(int64_t B, int64_t L, int64_t H, int64_t D,
                                                        int64_t N, int64_t chunk) {
  if (B <= 0 || L <= 0 || H <= 0 || D <= 0 || chunk <= 0 || N < 2 || N > 32 || N % 2 != 0) return -1;
  if (N == 2) return bwd_layout(B, L, H, D, chunk).total() * int64_t(sizeof(float2));
  // the gate-level form's N / 2 state rows per head as virtual heads, plus the
  // fp32 dk, dq, dbeta and dsel partials of the state rows
  const int64_t Hv = H * (N / 2);
  const BwdLayout w = bwd_layout(B, L, Hv, D, chunk);
  return (rows_partials_offset_floats(w) + 2 * rows_partials_floats(B, L, H, N / 2, D)) * int64_t(sizeof(float));
}

// The SSD form's backward workspace: the fused scan's with H N / 2 (virtual)
// heads, plus, for N > 2, the fp32 dk and dbeta partials of the state rows.
extern "C" int64_t cdssm_ssd_scan_bwd_workspace_bytes(int64_t B, int64_t L, int64_t H, int64_t D, int64_t N,
                                                      int64_t chunk) {
  if (B <= 0 || L <= 0 || H <= 0 || D <= 0 || chunk <= 0 || N < 2 || N > 32 || N % 2 != 0) return -1;
  const int64_t Hv = H * (N / 2);
  const BwdLayout w = bwd_layout(B, L, Hv, D, chunk);
  if (N == 2) return w.total() * int64_t(sizeof(float2));
  return (rows_partials_offset_floats(w) + rows_partials_floats(B, L, H, N / 2, D)) * int64_t(sizeof(float));
}

namespace {
int fused_bwd_entry(int dtype, const void* q, const void* k, const void* v, const void* beta,
                    const void* sel_c, const void* dt, const void* r, const float* alpha,
                    const float* omega, float c, const void* dy, const float* dh_final,
                    const float* fwd_workspace, void* dq, void* dk, void* dv, void* dbeta, void* dsel,
                    void* ddt, void* dr, float* dalpha, float* domega, float* dh0, float* workspace,
                    int64_t B, int64_t L, int64_t H, int64_t D, int64_t N, int64_t chunk,
                    hipStream_t stream, hipEvent_t* ev, int* carry_fused = nullptr, bool ssd = false,
                    bool cont = false, bool abar = false) {
  const char* op = ssd ? "cdssm_ssd_scan_bwd" : (abar ? "cdssm_fused_scan_bwd_abar" : "cdssm_fused_scan_bwd");
  if (dtype != 0 && dtype != 1) {
    cdssm_host::set_error("%s: dtype must be 0 (fp32) or 1 (bf16), got %d", op, dtype);
    return CDSSM_EINVAL;
  }
  if (B <= 0 || L <= 0 || H <= 0) {
    cdssm_host::set_error("%s: B, L, H must be positive", op);
    return CDSSM_EINVAL;
  }
  // SSD and gate-level forms: the N / 2 complex state rows of a head run as R
  // virtual heads sharing the head's k, beta (and q, sel_C)
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
  // q/k/dq/dk rows (dY rows: 2 D per head) of a chunk tile are addressed by 32-bit byte offsets
  if ((chunk + 16) * H * D * 4 * (ssd ? 2 : 1) > 0x7fffffffLL) {
    cdssm_host::set_error("%s: H * D too large for 32-bit row offsets (H=%lld D=%lld)", op, (long long)H,
                          (long long)D);
    return CDSSM_EINVAL;
  }
  if (ssd ? (!q || !k || !v || !beta || !dt || !fwd_workspace || !dk || !dv || !dbeta || !ddt || !workspace)
          : (!q || !k || !v || !beta || !sel_c || !dt || !r || (!abar && (!alpha || !omega)) || !dy ||
             !fwd_workspace || !dq || !dk || !dv || !dbeta || !dsel || !ddt || !dr ||
             (!abar && (!dalpha || !domega)) || !workspace)) {
    cdssm_host::set_error("%s: null pointer argument", op);
    return CDSSM_EINVAL;
  }
  const int b = int(B), l = int(L), hh = int(H), qc = int(chunk);
  if (abar) {
    // a_bar / dA_bar hold (re, im) pairs
    if (reinterpret_cast<uintptr_t>(dt) % (dtype == 1 ? 4 : 8) != 0 ||
        reinterpret_cast<uintptr_t>(ddt) % (dtype == 1 ? 4 : 8) != 0) {
      cdssm_host::set_error("%s: A_bar and dA_bar must be aligned to their (re, im) pairs", op);
      return CDSSM_EINVAL;
    }
    // q, k rows are read, and with state rows dq, dk written, as 16-byte vectors
    const auto a16 = [](const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; };
    if (!a16(q) || !a16(k) || !a16(dq) || !a16(dk)) {
      cdssm_host::set_error("%s: q, k, dq and dk must be 16-byte aligned", op);
      return CDSSM_EINVAL;
    }
    const int rr = int(R);
#define CDSSM_ABAR_BWD(TT, DD)                                                                                   \
  launch_fused_bwd<TT, DD>(q, k, v, beta, sel_c, dt, r, nullptr, nullptr, 0.0f, dy, dh_final, fwd_workspace, dq,  \
                           dk, dv, dbeta, dsel, ddt, dr, nullptr, nullptr, dh0, workspace, b, l, hh, qc, stream, \
                           ev, carry_fused, cont, rr)
    if (dtype == 1) return D == 64 ? CDSSM_ABAR_BWD(ABar<BF16>, 64) : CDSSM_ABAR_BWD(ABar<BF16>, 128);
    return D == 64 ? CDSSM_ABAR_BWD(ABar<F32>, 64) : CDSSM_ABAR_BWD(ABar<F32>, 128);
#undef CDSSM_ABAR_BWD
  }
  if (ssd) {
    const auto a16 = [](const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; };
    if (!a16(q) || !a16(k) || !a16(dk) || reinterpret_cast<uintptr_t>(ddt) % (dtype == 1 ? 4 : 8) != 0) {
      cdssm_host::set_error("%s: K, dY and dK must be 16-byte aligned, dA_bar aligned to its (re, im) pair", op);
      return CDSSM_EINVAL;
    }
    const int rr = int(R);
#define CDSSM_SSD_BWD(TT, DD)                                                                                     \
  launch_fused_bwd<TT, DD>(q, k, v, beta, nullptr, dt, nullptr, nullptr, nullptr, 0.0f, nullptr, nullptr,        \
                           fwd_workspace, nullptr, dk, dv, dbeta, nullptr, ddt, nullptr, nullptr, nullptr, nullptr, \
                           workspace, b, l, hh, qc, stream, ev, carry_fused, cont, rr)
    if (dtype == 1) return D == 64 ? CDSSM_SSD_BWD(SsdY<BF16>, 64) : CDSSM_SSD_BWD(SsdY<BF16>, 128);
    return D == 64 ? CDSSM_SSD_BWD(SsdY<F32>, 64) : CDSSM_SSD_BWD(SsdY<F32>, 128);
#undef CDSSM_SSD_BWD
  }
  if (dtype == 1) {
    if (D == 64)
      return launch_fused_bwd<BF16, 64>(q, k, v, beta, sel_c, dt, r, alpha, omega, c, dy, dh_final,
                                        fwd_workspace, dq, dk, dv, dbeta, dsel, ddt, dr, dalpha, domega,
                                        dh0, workspace, b, l, hh, qc, stream, ev, carry_fused, cont);
    return launch_fused_bwd<BF16, 128>(q, k, v, beta, sel_c, dt, r, alpha, omega, c, dy, dh_final,
                                       fwd_workspace, dq, dk, dv, dbeta, dsel, ddt, dr, dalpha, domega,
                                       dh0, workspace, b, l, hh, qc, stream, ev, carry_fused, cont);
  }
  if (D == 64)
    return launch_fused_bwd<F32, 64>(q, k, v, beta, sel_c, dt, r, alpha, omega, c, dy, dh_final,
                                     fwd_workspace, dq, dk, dv, dbeta, dsel, ddt, dr, dalpha, domega, dh0,
                                     workspace, b, l, hh, qc, stream, ev, carry_fused, cont);
  return launch_fused_bwd<F32, 128>(q, k, v, beta, sel_c, dt, r, alpha, omega, c, dy, dh_final,
                                    fwd_workspace, dq, dk, dv, dbeta, dsel, ddt, dr, dalpha, domega, dh0,
                                    workspace, b, l, hh, qc, stream, ev, carry_fused, cont);
}
}  // namespace

extern "C" int cdssm_fused_scan_bwd(int dtype, const void* q, const void* k, const void* v,
                                    const void* beta, const void* sel_c, const void* dt,
                                    const void* r, const float* alpha, const float* omega, float c,
                                    const void* dy, const float* dh_final, const float* fwd_workspace,
                                    void* dq, void* dk, void* dv, void* dbeta, void* dsel, void* ddt,
                                    void* dr, float* dalpha, float* domega, float* dh0, float* workspace,
                                    int64_t B, int64_t L, int64_t H, int64_t D, int64_t N,
                                    int64_t chunk, hipStream_t stream) {
  return fused_bwd_entry(dtype, q, k, v, beta, sel_c, dt, r, alpha, omega, c, dy, dh_final, fwd_workspace,
                         dq, dk, dv, dbeta, dsel, ddt, dr, dalpha, domega, dh0, workspace, B, L, H, D, N,
                         chunk, stream, nullptr);
}

// Instrumentation (no reference counterpart): cdssm_fused_scan_bwd, recording
// the 100 MHz real-time counter per wave at kBwdCorrStamps points of the
// one-launch correction adjoint + carry (words ((workgroup * 4 + wave) * 8 +
// point)) and kBwdMainStamps points of the main pass (words M + workgroup * 4 +
// point, M = NSEG B H * 32 with NSEG = ceil(ceil(L / chunk) / 4)); -1 if the
// buffer is too small or the shape runs the three-launch correction adjoint.
extern "C" int cdssm_fused_scan_bwd_stamped(int dtype, const void* q, const void* k, const void* v,
                                            const void* beta, const void* sel_c, const void* dt,
                                            const void* r, const float* alpha, const float* omega, float c,
                                            const void* dy, const float* dh_final, const float* fwd_workspace,
                                            void* dq, void* dk, void* dv, void* dbeta, void* dsel, void* ddt,
                                            void* dr, float* dalpha, float* domega, float* dh0, float* workspace,
                                            int64_t B, int64_t L, int64_t H, int64_t D, int64_t N, int64_t chunk,
                                            unsigned long long* stamps, int64_t stamps_len, hipStream_t stream) {
  if (!stamps || stamps_len <= 0) {
    cdssm_host::set_error("cdssm_fused_scan_bwd_stamped: a stamp buffer is required");
    return CDSSM_EINVAL;
  }
  t_bstamps = BwdStampRequest{stamps, stamps_len};
  const int st = fused_bwd_entry(dtype, q, k, v, beta, sel_c, dt, r, alpha, omega, c, dy, dh_final, fwd_workspace,
                                 dq, dk, dv, dbeta, dsel, ddt, dr, dalpha, domega, dh0, workspace, B, L, H, D, N,
                                 chunk, stream, nullptr);
  t_bstamps = BwdStampRequest{};
  return st;
}

// cdssm_fused_scan_bwd for a workspace whose previous use was a backward call
// (this entry or cdssm_fused_scan_bwd) of the same shape, completed or
// ordered before this one on the stream, with the workspace untouched since:
// the one-launch correction adjoint + carry reuses the look-back epoch that
// call's last workgroup left in the workspace instead of a separate launch
// drawing one.
extern "C" int cdssm_fused_scan_bwd_continue(int dtype, const void* q, const void* k, const void* v,
                                             const void* beta, const void* sel_c, const void* dt,
                                             const void* r, const float* alpha, const float* omega, float c,
                                             const void* dy, const float* dh_final, const float* fwd_workspace,
                                             void* dq, void* dk, void* dv, void* dbeta, void* dsel, void* ddt,
                                             void* dr, float* dalpha, float* domega, float* dh0, float* workspace,
                                             int64_t B, int64_t L, int64_t H, int64_t D, int64_t N,
                                             int64_t chunk, hipStream_t stream) {
  return fused_bwd_entry(dtype, q, k, v, beta, sel_c, dt, r, alpha, omega, c, dy, dh_final, fwd_workspace,
                         dq, dk, dv, dbeta, dsel, ddt, dr, dalpha, domega, dh0, workspace, B, L, H, D, N,
                         chunk, stream, nullptr, nullptr, false, true);
}

// Backward of the gate-level (A_bar, vp) forward, cdssm_fused_scan_fwd_abar_train:
// the readout form's gradients with dA_bar (B,L,H,2) and dvp (B,L,H) in place
// of the scan-level dynamics chain (no per-head dalpha / domega).  Same rules
// as cdssm_fused_scan_bwd (the correction branch's shifted rule).
extern "C" int cdssm_fused_scan_bwd_abar(int dtype, const void* q, const void* k, const void* v, const void* beta,
                                         const void* sel_c, const void* a_bar, const void* vp, const void* dy,
                                         const float* dh_final, const float* fwd_workspace, void* dq, void* dk,
                                         void* dv, void* dbeta, void* dsel, void* da_bar, void* dvp, float* dh0,
                                         float* workspace, int64_t B, int64_t L, int64_t H, int64_t D, int64_t N,
                                         int64_t chunk, hipStream_t stream) {
  return fused_bwd_entry(dtype, q, k, v, beta, sel_c, a_bar, vp, nullptr, nullptr, 0.0f, dy, dh_final,
                         fwd_workspace, dq, dk, dv, dbeta, dsel, da_bar, dvp, nullptr, nullptr, dh0, workspace, B, L,
                         H, D, N, chunk, stream, nullptr, nullptr, false, false, true);
}

// Backward of cdssm_ssd_scan_fwd (the SSDChunkwiseScan interface), with the
// reference's gradient rules (exact for the local and carry branches, the
// correction branch's shifted rule): given dY (B,L,H,2,D) of `dtype` and the
// workspace of a cdssm_ssd_scan_fwd call with train != 0 on the same inputs,
// writes dA_bar (B,L,H,2), dK (B,L,H,D), dV (B,L,H,2) and dbeta (B,L,H), all of
// `dtype`.  workspace: cdssm_fused_scan_bwd_workspace_bytes().
extern "C" int cdssm_ssd_scan_bwd(int dtype, const void* a_bar, const void* k, const void* v, const void* beta,
                                  const void* dY, const float* fwd_workspace, void* dA, void* dK, void* dV,
                                  void* dbeta, float* workspace, int64_t B, int64_t L, int64_t H, int64_t D,
                                  int64_t N, int64_t chunk, hipStream_t stream) {
  return fused_bwd_entry(dtype, dY, k, v, beta, nullptr, a_bar, nullptr, nullptr, nullptr, 0.0f, nullptr, nullptr,
                         fwd_workspace, nullptr, dK, dV, dbeta, nullptr, dA, nullptr, nullptr, nullptr, nullptr,
                         workspace, B, L, H, D, N, chunk, stream, nullptr, nullptr, true);
}

extern "C" int cdssm_fused_scan_bwd_profile(int dtype, const void* q, const void* k, const void* v,
                                            const void* beta, const void* sel_c, const void* dt,
                                            const void* r, const float* alpha, const float* omega,
                                            float c, const void* dy, const float* dh_final,
                                            const float* fwd_workspace, void* dq, void* dk, void* dv,
                                            void* dbeta, void* dsel, void* ddt, void* dr, float* dalpha,
                                            float* domega, float* dh0, float* workspace, int64_t B,
                                            int64_t L, int64_t H, int64_t D, int64_t N, int64_t chunk,
                                            hipStream_t stream, int iters, float* phase_ms) {
  if (iters < 1 || !phase_ms) {
    cdssm_host::set_error("cdssm_fused_scan_bwd_profile: iters >= 1 and phase_ms required");
    return CDSSM_EINVAL;
  }
  hipEvent_t ev[6];
  for (int i = 0; i < 6; ++i)
    if (hipEventCreate(&ev[i]) != hipSuccess) {
      for (int j = 0; j < i; ++j) (void)hipEventDestroy(ev[j]);
      cdssm_host::set_error("cdssm_fused_scan_bwd_profile: hipEventCreate failed");
      return CDSSM_EHIP;
    }
  for (int p = 0; p < 5; ++p) phase_ms[p] = 0.0f;
  int st = CDSSM_OK;
  for (int it = 0; it < iters; ++it) {
    int fusedc = 0;
    st = fused_bwd_entry(dtype, q, k, v, beta, sel_c, dt, r, alpha, omega, c, dy, dh_final, fwd_workspace,
                         dq, dk, dv, dbeta, dsel, ddt, dr, dalpha, domega, dh0, workspace, B, L, H, D, N,
                         chunk, stream, ev, &fusedc);
    if (st != CDSSM_OK) break;
    if (hipEventSynchronize(ev[5]) != hipSuccess) {
      cdssm_host::set_error("cdssm_fused_scan_bwd_profile: hipEventSynchronize failed");
      st = CDSSM_EHIP;
      break;
    }
    for (int p = 0; p < 5; ++p) {
      // a one-launch correction adjoint + carry is reported as the first phase
      if (fusedc && (p == 1 || p == 2)) continue;
      float ms = 0.0f;
      (void)hipEventElapsedTime(&ms, ev[p], ev[p + 1]);
      phase_ms[p] += ms / float(iters);
    }
  }
  for (int i = 0; i < 6; ++i) (void)hipEventDestroy(ev[i]);
  return st;
}
