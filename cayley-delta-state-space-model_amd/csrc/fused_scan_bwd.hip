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
//   B3 main:    per chunk: forward recompute with checkpoints,
//               then segment-wise reverse of both branches (checkpoint
//               interval 16 / DPL steps), emitting dq, dk,
//               dv, dbeta, dsel_C, ddt, dr and per-chunk d alpha / d omega
//   B4 heads:   deterministic sum of the per-chunk d alpha / d omega.
//
// Work layout of B1 and B3: one wave64 per (b, chunk, h); lane owns
// DPL = D/64 state elements; per-token scalars live one token per lane
// (two slots for 128-token chunks) and are broadcast with readlane.
#include "common.hpp"

namespace cdssm {

constexpr int kBwdSeg = 16;

__device__ __forceinline__ float rl(float x, int lane) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), lane));
}
// Value of token t from a two-slot lane-per-token register pair.
__device__ __forceinline__ float tok(const float (&s)[2], int t) {
  return t < 64 ? rl(s[0], t) : rl(s[1], t - 64);
}
__device__ __forceinline__ void set_tok(float (&s)[2], int t, float v) {
  const int lane = threadIdx.x;
  if (t < 64) {
    if (lane == t) s[0] = v;
  } else {
    if (lane == t - 64) s[1] = v;
  }
}

// Full-wave sum, broadcast to every lane.
__device__ __forceinline__ float wsum(float x) { return group_sum<64>(x); }

struct BwdTile {
  int b, chunk, h, t0, nt;
  int64_t row0, tile;
};

__device__ __forceinline__ BwdTile bwd_tile(int L, int Q, int NC, int H) {
  BwdTile c;
  const int g = blockIdx.x;
  c.tile = g;  // (b*NC + chunk)*H + h
  c.h = g % H;
  const int bc = g / H;
  c.chunk = bc % NC;
  c.b = bc / NC;
  c.t0 = c.chunk * Q;
  c.nt = min(Q, L - c.t0);
  c.row0 = int64_t(c.b) * L + c.t0;
  return c;
}

// Exclusive/inclusive complex prefix product over the tokens held one per
// lane in two slots.  Returns inclusive g_t and exclusive g_{t-1} (g_{-1}=1).
__device__ __forceinline__ void prefix_prod(const float (&ar)[2], const float (&ai)[2], float (&gr)[2],
                                            float (&gi)[2], float (&gpr)[2], float (&gpi)[2]) {
  const int lane = threadIdx.x;
#pragma unroll
  for (int s = 0; s < 2; ++s) {
    float xr = ar[s], xi = ai[s];
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
      const float yr = __shfl_up(xr, off, 64);
      const float yi = __shfl_up(xi, off, 64);
      if (lane >= off) {
        const float nr = xr * yr - xi * yi;
        xi = xr * yi + xi * yr;
        xr = nr;
      }
    }
    gr[s] = xr;
    gi[s] = xi;
  }
  // slot 1 continues after slot 0's total
  const float tr = rl(gr[0], 63), ti = rl(gi[0], 63);
  {
    const float nr = gr[1] * tr - gi[1] * ti;
    gi[1] = gr[1] * ti + gi[1] * tr;
    gr[1] = nr;
  }
#pragma unroll
  for (int s = 0; s < 2; ++s) {
    float er = __shfl_up(gr[s], 1, 64), ei = __shfl_up(gi[s], 1, 64);
    if (lane == 0) {
      er = s == 0 ? 1.0f : tr;
      ei = s == 0 ? 0.0f : ti;
    }
    gpr[s] = er;
    gpi[s] = ei;
  }
}

// Per-token inputs of a chunk tile, one token per lane (two slots).
template <typename T>
struct TokenInputs {
  float ar[2], ai[2], vp[2], vr[2], vi[2], b[2], sel[2], dyr[2], dyi[2], dt[2], r[2];

  __device__ __forceinline__ void load(const BwdTile& tc, int H, const typename T::raw* v,
                                       const typename T::raw* beta, const typename T::raw* sel_c,
                                       const typename T::raw* dtp, const typename T::raw* rp,
                                       const typename T::raw* dy, float alpha, float omega, float c) {
    const int lane = threadIdx.x;
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      const int t = lane + 64 * s;
      const int tcl = min(t, tc.nt - 1);
      const int64_t e = (tc.row0 + tcl) * H + tc.h;
      const float bb = T::load(beta + e), d = T::load(dtp + e), rr = T::load(rp + e);
      const float v0 = T::load(v + 2 * e), v1 = T::load(v + 2 * e + 1);
      const float sc = T::load(sel_c + e);
      const float g0 = T::load(dy + 2 * e), g1 = T::load(dy + 2 * e + 1);
      const bool real = t < tc.nt;
      const Transition tr = cayley_gated(d, rr, alpha, omega, c);
      ar[s] = real ? tr.ar : 1.0f;
      ai[s] = real ? tr.ai : 0.0f;
      vp[s] = real ? tr.vp : 0.0f;
      vr[s] = real ? v0 : 0.0f;
      vi[s] = real ? v1 : 0.0f;
      b[s] = real ? bb : 0.0f;
      sel[s] = real ? sc : 0.0f;
      dyr[s] = real ? g0 : 0.0f;
      dyi[s] = real ? g1 : 0.0f;
      dt[s] = d;
      r[s] = rr;
    }
  }
};

// Load lane's DPL elements of row t (clamped into the tile).
template <typename T, int DPL>
__device__ __forceinline__ void load_row(const typename T::raw* base, int64_t stride, int t, int tlast,
                                         float (&o)[DPL]) {
  const typename T::raw* p = base + int64_t(min(t, tlast)) * stride;
#pragma unroll
  for (int j = 0; j < DPL; ++j) o[j] = T::load(p + j);
}

// ---------------------------------------------------------------------------
// B1: correction-branch adjoint of the entering state, per chunk.
// ---------------------------------------------------------------------------
template <typename T, int D>
__global__ __launch_bounds__(kWave) void fused_bwd_corr_kernel(
    const typename T::raw* __restrict__ q, const typename T::raw* __restrict__ k,
    const typename T::raw* __restrict__ v, const typename T::raw* __restrict__ beta,
    const typename T::raw* __restrict__ sel_c, const typename T::raw* __restrict__ dt,
    const typename T::raw* __restrict__ r, const float* __restrict__ alpha,
    const float* __restrict__ omega, float c, const typename T::raw* __restrict__ dy,
    float2* __restrict__ lam0, int L, int H, int Q, int NC) {
  constexpr int DPL = D / kWave;
  const BwdTile tc = bwd_tile(L, Q, NC, H);
  const int lane = threadIdx.x;
  TokenInputs<T> in;
  in.load(tc, H, v, beta, sel_c, dt, r, dy, alpha[tc.h], omega[tc.h], c);
  float gr[2], gi[2], gpr[2], gpi[2];
  prefix_prod(in.ar, in.ai, gr, gi, gpr, gpi);
  // h_t = conj(g_t) * sel_t * dy_t
  float hr[2], hi[2];
#pragma unroll
  for (int s = 0; s < 2; ++s) {
    const float fr = in.sel[s] * in.dyr[s], fi = in.sel[s] * in.dyi[s];
    hr[s] = gr[s] * fr + gi[s] * fi;
    hi[s] = gr[s] * fi - gi[s] * fr;
  }

  const int64_t stride = int64_t(H) * D;
  const int64_t off = (tc.row0 * H + tc.h) * D + lane * DPL;
  const typename T::raw* kp = k + off;
  const typename T::raw* qp = q + off;
  const int tlast = tc.nt - 1;
  float lr[DPL], li[DPL];
#pragma unroll
  for (int j = 0; j < DPL; ++j) lr[j] = li[j] = 0.0f;

  for (int t = tc.nt - 1; t >= 0; --t) {
    float kk[DPL], qq[DPL];
    load_row<T, DPL>(kp, stride, t, tlast, kk);
    load_row<T, DPL>(qp, stride, t, tlast, qq);
    const float h_r = tok(hr, t), h_i = tok(hi, t), bb = tok(in.b, t);
    float sr = 0.0f, si = 0.0f;
#pragma unroll
    for (int j = 0; j < DPL; ++j) {
      lr[j] = fmaf(h_r, qq[j], lr[j]);
      li[j] = fmaf(h_i, qq[j], li[j]);
      sr = fmaf(lr[j], kk[j], sr);
      si = fmaf(li[j], kk[j], si);
    }
    sr = wsum(sr);
    si = wsum(si);
#pragma unroll
    for (int j = 0; j < DPL; ++j) {
      lr[j] = fmaf(-bb * sr, kk[j], lr[j]);
      li[j] = fmaf(-bb * si, kk[j], li[j]);
    }
  }
  float2* o = lam0 + tc.tile * D + lane * DPL;
#pragma unroll
  for (int j = 0; j < DPL; ++j) o[j] = make_float2(lr[j], li[j]);
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
  // map: ds_{c0} = A ds_{c1} + X
  float2 A = make_float2(1.0f, 0.0f), X = make_float2(0.0f, 0.0f);
  for (int ch = x.c1 - 1; ch >= x.c0; --ch) {
    const int64_t e = x.base + int64_t(ch) * H;
    const float2 G = gam[e];
    X = cfma_conj(G, X, lam0[e * D + x.d]);
    A = cmul_conj(G, A);
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
  for (int j = S - 1; j > x.seg; --j) {
    const float2 A = segA[sbase + j];
    const float2 X = segX[(sbase + j) * D + x.d];
    ds = make_float2(A.x * ds.x - A.y * ds.y + X.x, A.x * ds.y + A.y * ds.x + X.y);
  }
  for (int ch = x.c1 - 1; ch >= x.c0; --ch) {
    const int64_t e = x.base + int64_t(ch) * H;
    dsn[e * D + x.d] = ds;
    ds = cfma_conj(gam[e], ds, lam0[e * D + x.d]);
  }
  if (x.seg == 0 && dh0 != nullptr) {
    dh0[hb + x.d] = ds.x;
    dh0[hb + D + x.d] = ds.y;
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
// B3: per-chunk backward of both branches with checkpointed recompute.
// ---------------------------------------------------------------------------
template <typename T, int D>
__global__ __launch_bounds__(kWave) void fused_bwd_main_kernel(
    const typename T::raw* __restrict__ q, const typename T::raw* __restrict__ k,
    const typename T::raw* __restrict__ v, const typename T::raw* __restrict__ beta,
    const typename T::raw* __restrict__ sel_c, const typename T::raw* __restrict__ dt,
    const typename T::raw* __restrict__ r, const float* __restrict__ alpha,
    const float* __restrict__ omega, float c, const typename T::raw* __restrict__ dy,
    const float2* __restrict__ states, const float2* __restrict__ dsn, typename T::raw* __restrict__ dq,
    typename T::raw* __restrict__ dk, typename T::raw* __restrict__ dv,
    typename T::raw* __restrict__ dbeta, typename T::raw* __restrict__ dsel,
    typename T::raw* __restrict__ ddt, typename T::raw* __restrict__ dr,
    float2* __restrict__ dhead_parts, int L, int H, int Q, int NC) {
  constexpr int DPL = D / kWave;
  constexpr int kCk = 16 / DPL;  // checkpoint interval of the recompute
  extern __shared__ float4 ck[];  // [Q/kCk][64*DPL] checkpoints (zr, zi, cr, ci)
  const BwdTile tc = bwd_tile(L, Q, NC, H);
  const int lane = threadIdx.x;
  const float al = alpha[tc.h], om = omega[tc.h];
  TokenInputs<T> in;
  in.load(tc, H, v, beta, sel_c, dt, r, dy, al, om, c);
  float gr[2], gi[2], gpr[2], gpi[2];
  prefix_prod(in.ar, in.ai, gr, gi, gpr, gpi);
  float wr[2], wi[2];
#pragma unroll
  for (int s = 0; s < 2; ++s) {
    const float f = in.b[s] * in.vp[s];
    wr[s] = f * in.vr[s];
    wi[s] = f * in.vi[s];
  }

  const int64_t stride = int64_t(H) * D;
  const int64_t off = (tc.row0 * H + tc.h) * D + lane * DPL;
  const typename T::raw* kp = k + off;
  const typename T::raw* qp = q + off;
  const int tlast = tc.nt - 1;
  const int ntr = (tc.nt + kCk - 1) / kCk * kCk;

  // ---- forward recompute with checkpoints; per-token dots kept per lane ----
  float zr[DPL], zi[DPL], cr[DPL], ci[DPL];
  const float2* sp = states + tc.tile * D + lane * DPL;
#pragma unroll
  for (int j = 0; j < DPL; ++j) {
    zr[j] = zi[j] = 0.0f;
    cr[j] = sp[j].x;
    ci[j] = sp[j].y;
  }
  float p_r[2] = {0, 0}, p_i[2] = {0, 0}, pc_r[2] = {0, 0}, pc_i[2] = {0, 0};
  float zq_r[2] = {0, 0}, zq_i[2] = {0, 0}, cq_r[2] = {0, 0}, cq_i[2] = {0, 0}, kq[2] = {0, 0};
  for (int t = 0; t < ntr; ++t) {
    if (t % kCk == 0) {
#pragma unroll
      for (int j = 0; j < DPL; ++j) ck[(t / kCk) * (64 * DPL) + lane * DPL + j] = make_float4(zr[j], zi[j], cr[j], ci[j]);
    }
    float kk[DPL], qq[DPL];
    load_row<T, DPL>(kp, stride, t, tlast, kk);
    load_row<T, DPL>(qp, stride, t, tlast, qq);
    const bool real = t < tc.nt;
    float s0 = 0, s1 = 0, s2 = 0, s3 = 0, s4 = 0, s5 = 0, s6 = 0, s7 = 0, s8 = 0;
#pragma unroll
    for (int j = 0; j < DPL; ++j) {
      s0 = fmaf(zr[j], kk[j], s0);
      s1 = fmaf(zi[j], kk[j], s1);
      s2 = fmaf(cr[j], kk[j], s2);
      s3 = fmaf(ci[j], kk[j], s3);
      s4 = fmaf(zr[j], qq[j], s4);
      s5 = fmaf(zi[j], qq[j], s5);
      s6 = fmaf(cr[j], qq[j], s6);
      s7 = fmaf(ci[j], qq[j], s7);
      s8 = fmaf(kk[j], qq[j], s8);
    }
    s0 = wsum(s0); s1 = wsum(s1); s2 = wsum(s2); s3 = wsum(s3);
    s4 = wsum(s4); s5 = wsum(s5); s6 = wsum(s6); s7 = wsum(s7); s8 = wsum(s8);
    const float ar = tok(in.ar, t), ai = tok(in.ai, t), bb = tok(in.b, t);
    const float w_r = tok(wr, t), w_i = tok(wi, t);
    const float bpr = bb * s0, bpi = bb * s1;
    const float er = w_r - (ar * bpr - ai * bpi);
    const float ei = w_i - (ar * bpi + ai * bpr);
    // z_t . q = a (z_{t-1}.q) + e (k.q)
    const float zqr = ar * s4 - ai * s5 + er * s8;
    const float zqi = ar * s5 + ai * s4 + ei * s8;
    set_tok(p_r, t, real ? s0 : 0.0f);
    set_tok(p_i, t, real ? s1 : 0.0f);
    set_tok(pc_r, t, real ? s2 : 0.0f);
    set_tok(pc_i, t, real ? s3 : 0.0f);
    set_tok(zq_r, t, zqr);
    set_tok(zq_i, t, zqi);
    set_tok(cq_r, t, s6);
    set_tok(cq_i, t, s7);
    set_tok(kq, t, s8);
    const float ecr = bb * s2, eci = bb * s3;
#pragma unroll
    for (int j = 0; j < DPL; ++j) {
      const float nr = fmaf(ar, zr[j], fmaf(-ai, zi[j], er * kk[j]));
      const float ni = fmaf(ar, zi[j], fmaf(ai, zr[j], ei * kk[j]));
      zr[j] = nr;
      zi[j] = ni;
      cr[j] = fmaf(-ecr, kk[j], cr[j]);
      ci[j] = fmaf(-eci, kk[j], ci[j]);
    }
  }

  // ---- reverse ----
  // local adjoint mu starts at d s_{k+1}; delta G = sum_d ds_{k+1} conj(s_k)
  float mr[DPL], mi[DPL], lr[DPL], li[DPL];
  const float2* dp = dsn + tc.tile * D + lane * DPL;
  float dGr = 0.0f, dGi = 0.0f;
#pragma unroll
  for (int j = 0; j < DPL; ++j) {
    const float2 ds = dp[j];
    const float2 s0 = sp[j];
    mr[j] = ds.x;
    mi[j] = ds.y;
    lr[j] = li[j] = 0.0f;
    dGr = fmaf(ds.x, s0.x, fmaf(ds.y, s0.y, dGr));
    dGi = fmaf(ds.y, s0.x, fmaf(-ds.x, s0.y, dGi));
  }
  dGr = wsum(dGr);
  dGi = wsum(dGi);

  // per-token gradient scalars (lane = token)
  float da_r[2] = {0, 0}, da_i[2] = {0, 0}, dw_r[2] = {0, 0}, dw_i[2] = {0, 0}, db_e[2] = {0, 0},
        dsl[2] = {0, 0};
  float psr = 0.0f, psi = 0.0f;    // psi_{t+1}
  float anr = 1.0f, ani = 0.0f;    // a_{t+1}
  const int64_t doff = off;
  for (int seg = ntr / kCk - 1; seg >= 0; --seg) {
    const int tb = seg * kCk;
    // recompute the segment's states: zb[i] = z_{tb+i-1}, cb[i] = c^_{tb+i}
    float zbr[kCk + 1][DPL], zbi[kCk + 1][DPL], cbr[kCk][DPL], cbi[kCk][DPL];
    float kseg[kCk][DPL], qseg[kCk][DPL];
#pragma unroll
    for (int j = 0; j < DPL; ++j) {
      const float4 cv = ck[seg * (64 * DPL) + lane * DPL + j];
      zbr[0][j] = cv.x;
      zbi[0][j] = cv.y;
      cbr[0][j] = cv.z;
      cbi[0][j] = cv.w;
    }
#pragma unroll
    for (int i = 0; i < kCk; ++i) {
      load_row<T, DPL>(kp, stride, tb + i, tlast, kseg[i]);
      load_row<T, DPL>(qp, stride, tb + i, tlast, qseg[i]);
    }
#pragma unroll
    for (int i = 0; i < kCk; ++i) {
      const int t = tb + i;
      const float ar = tok(in.ar, t), ai = tok(in.ai, t), bb = tok(in.b, t);
      const float w_r = tok(wr, t), w_i = tok(wi, t);
      const float pr = tok(p_r, t), pi = tok(p_i, t), pcr = tok(pc_r, t), pci = tok(pc_i, t);
      const float bpr = bb * pr, bpi = bb * pi;
      const float er = w_r - (ar * bpr - ai * bpi);
      const float ei = w_i - (ar * bpi + ai * bpr);
#pragma unroll
      for (int j = 0; j < DPL; ++j) {
        zbr[i + 1][j] = fmaf(ar, zbr[i][j], fmaf(-ai, zbi[i][j], er * kseg[i][j]));
        zbi[i + 1][j] = fmaf(ar, zbi[i][j], fmaf(ai, zbr[i][j], ei * kseg[i][j]));
        if (i + 1 < kCk) {
          cbr[i + 1][j] = fmaf(-bb * pcr, kseg[i][j], cbr[i][j]);
          cbi[i + 1][j] = fmaf(-bb * pci, kseg[i][j], cbi[i][j]);
        }
      }
    }
#pragma unroll
    for (int i = kCk - 1; i >= 0; --i) {
      const int t = tb + i;
      const bool real = t < tc.nt;
      const float ar = tok(in.ar, t), ai = tok(in.ai, t), bb = tok(in.b, t);
      const float w_r = tok(wr, t), w_i = tok(wi, t);
      const float pr = tok(p_r, t), pi = tok(p_i, t), pcr = tok(pc_r, t), pci = tok(pc_i, t);
      const float sel = tok(in.sel, t), dyr = tok(in.dyr, t), dyi = tok(in.dyi, t);
      const float g_r = tok(gr, t), g_i = tok(gi, t), gp_r = tok(gpr, t), gp_i = tok(gpi, t);
      const float fr = sel * dyr, fi = sel * dyi;
      // conj(g_t) f
      const float hr = g_r * fr + g_i * fi, hi = g_r * fi - g_i * fr;
      float sk0 = 0, sk1 = 0, sz0 = 0, sz1 = 0, sl0 = 0, sl1 = 0;
      float dqv[DPL];
#pragma unroll
      for (int j = 0; j < DPL; ++j) {
        const float qv = qseg[i][j], kv = kseg[i][j];
        // Y_t = z_t + g_{t-1} c^_t
        const float Yr = zbr[i + 1][j] + gp_r * cbr[i][j] - gp_i * cbi[i][j];
        const float Yi = zbi[i + 1][j] + gp_r * cbi[i][j] + gp_i * cbr[i][j];
        dqv[j] = sel * (Yr * dyr + Yi * dyi);
        mr[j] = fmaf(fr, qv, mr[j]);
        mi[j] = fmaf(fi, qv, mi[j]);
        lr[j] = fmaf(hr, qv, lr[j]);
        li[j] = fmaf(hi, qv, li[j]);
        sk0 = fmaf(mr[j], kv, sk0);
        sk1 = fmaf(mi[j], kv, sk1);
        sz0 = fmaf(mr[j], zbr[i][j], fmaf(mi[j], zbi[i][j], sz0));
        sz1 = fmaf(mi[j], zbr[i][j], fmaf(-mr[j], zbi[i][j], sz1));
        sl0 = fmaf(lr[j], kv, sl0);
        sl1 = fmaf(li[j], kv, sl1);
      }
      sk0 = wsum(sk0); sk1 = wsum(sk1); sz0 = wsum(sz0); sz1 = wsum(sz1); sl0 = wsum(sl0); sl1 = wsum(sl1);
      // dw = mu.k; mk = conj(a) dw
      const float dwr = sk0, dwi = sk1;
      const float mkr = ar * dwr + ai * dwi, mki = ar * dwi - ai * dwr;
      // da (local) = mu.conj(z_{t-1}) - beta conj(p) dw
      float dar = sz0 - bb * (pr * dwr + pi * dwi);
      float dai = sz1 - bb * (pr * dwi - pi * dwr);
      const float dbe = -(pr * mkr + pi * mki) - (pcr * sl0 + pci * sl1);
      // delta g_t from the correction branch: f conj(c^_{t+1}.q)
      const float cnr = tok(cq_r, t) - bb * pcr * tok(kq, t);
      const float cni = tok(cq_i, t) - bb * pci * tok(kq, t);
      float dgr = fr * cnr + fi * cni, dgi = fi * cnr - fr * cni;
      if (t == tc.nt - 1) {
        dgr += dGr;
        dgi += dGi;
      }
      // psi_t = dg_t + conj(a_{t+1}) psi_{t+1}
      const float npr = dgr + anr * psr + ani * psi;
      const float npi = dgi + anr * psi - ani * psr;
      psr = npr;
      psi = npi;
      anr = ar;
      ani = ai;
      // da += conj(g_{t-1}) psi_t
      dar += gp_r * psr + gp_i * psi;
      dai += gp_r * psi - gp_i * psr;
      // dsel_t = dy . (Y . q)
      const float yqr = tok(zq_r, t) + gp_r * tok(cq_r, t) - gp_i * tok(cq_i, t);
      const float yqi = tok(zq_i, t) + gp_r * tok(cq_i, t) + gp_i * tok(cq_r, t);
      const float dsv = dyr * yqr + dyi * yqi;
      float dkv[DPL];
#pragma unroll
      for (int j = 0; j < DPL; ++j) {
        const float kv = kseg[i][j];
        // m = conj(a) mu
        const float m_r = ar * mr[j] + ai * mi[j], m_i = ar * mi[j] - ai * mr[j];
        dkv[j] = mr[j] * w_r + mi[j] * w_i
                 - bb * (zbr[i][j] * mkr + zbi[i][j] * mki + m_r * pr + m_i * pi)
                 - bb * (cbr[i][j] * sl0 + cbi[i][j] * sl1 + lr[j] * pcr + li[j] * pci);
        // mu <- P_t m ; lambda <- P_t lambda
        mr[j] = fmaf(-bb * mkr, kv, m_r);
        mi[j] = fmaf(-bb * mki, kv, m_i);
        lr[j] = fmaf(-bb * sl0, kv, lr[j]);
        li[j] = fmaf(-bb * sl1, kv, li[j]);
      }
      if (real) {
        const int64_t o = doff + int64_t(t) * stride;
#pragma unroll
        for (int j = 0; j < DPL; ++j) {
          T::store(dq + o + j, dqv[j]);
          T::store(dk + o + j, dkv[j]);
        }
      }
      set_tok(da_r, t, dar);
      set_tok(da_i, t, dai);
      set_tok(dw_r, t, dwr);
      set_tok(dw_i, t, dwi);
      set_tok(db_e, t, dbe);
      set_tok(dsl, t, dsv);
    }
  }

  // ---- per-token dynamics backward (lane = token) ----
  float dal = 0.0f, dom = 0.0f;
#pragma unroll
  for (int s = 0; s < 2; ++s) {
    const int t = lane + 64 * s;
    if (t < tc.nt) {
      const float bb = in.b[s], vp = in.vp[s], vr = in.vr[s], vi = in.vi[s];
      const float dwv = dw_r[s] * vr + dw_i[s] * vi;
      const float dbeta_t = db_e[s] + vp * dwv;
      const float dvp = bb * dwv;
      const DynGrad g = cayley_gated_bwd(in.dt[s], in.r[s], al, om, c, da_r[s], da_i[s], dvp);
      const int64_t e = (tc.row0 + t) * H + tc.h;
      T::store(dv + 2 * e, bb * vp * dw_r[s]);
      T::store(dv + 2 * e + 1, bb * vp * dw_i[s]);
      T::store(dbeta + e, dbeta_t);
      T::store(dsel + e, dsl[s]);
      T::store(ddt + e, g.ddt);
      T::store(dr + e, g.dr);
      dal += g.dalpha;
      dom += g.domega;
    }
  }
  dal = wsum(dal);
  dom = wsum(dom);
  if (lane == 0) dhead_parts[tc.tile] = make_float2(dal, dom);
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

}  // namespace cdssm

// ---------------------------------------------------------------------------
// C-ABI
// ---------------------------------------------------------------------------
namespace {
using namespace cdssm;

struct BwdLayout {
  int NC, S;
  int64_t n_lam, n_dsn, n_segA, n_segX, n_parts;  // float2 counts
  int64_t total() const { return n_lam + n_dsn + n_segA + n_segX + n_parts; }
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
  return w;
}

template <typename T, int D>
int launch_fused_bwd(const void* q, const void* k, const void* v, const void* beta, const void* sel_c,
                     const void* dt, const void* r, const float* alpha, const float* omega, float c,
                     const void* dy, const float* dh_final, const float* fwd_ws, void* dq, void* dk,
                     void* dv, void* dbeta, void* dsel, void* ddt, void* dr, float* dalpha,
                     float* domega, float* dh0, float* ws, int B, int L, int H, int Q,
                     hipStream_t stream) {
  using raw = typename T::raw;
  const BwdLayout w = bwd_layout(B, L, H, D, Q);
  const int NC = w.NC, S = w.S;
  const int64_t tiles = int64_t(B) * NC * H;
  const int64_t carry_threads = int64_t(B) * H * S * D;
  if (tiles > 0x7fffffff || carry_threads / 256 > 0x7fffffff) {
    cdssm_host::set_error("cdssm_fused_scan_bwd: grid too large");
    return CDSSM_EINVAL;
  }
  const float2* states = reinterpret_cast<const float2*>(fwd_ws);
  const float2* gam = states + int64_t(B) * NC * H * D;
  float2* lam0 = reinterpret_cast<float2*>(ws);
  float2* dsn = lam0 + w.n_lam;
  float2* segA = dsn + w.n_dsn;
  float2* segX = segA + w.n_segA;
  float2* parts = segX + w.n_segX;

  hipLaunchKernelGGL((fused_bwd_corr_kernel<T, D>), dim3(unsigned(tiles)), dim3(kWave), 0, stream,
                     (const raw*)q, (const raw*)k, (const raw*)v, (const raw*)beta, (const raw*)sel_c,
                     (const raw*)dt, (const raw*)r, alpha, omega, c, (const raw*)dy, lam0, L, H, Q, NC);
  int st = cdssm_host::check_launch("cdssm_fused_scan_bwd/corr");
  if (st) return st;
  const unsigned cblocks = unsigned((carry_threads + 255) / 256);
  hipLaunchKernelGGL(fused_bwd_rfold_kernel, dim3(cblocks), dim3(256), 0, stream, (const float2*)lam0,
                     gam, segA, segX, B, NC, H, D, S);
  st = cdssm_host::check_launch("cdssm_fused_scan_bwd/rfold");
  if (st) return st;
  hipLaunchKernelGGL(fused_bwd_rreplay_kernel, dim3(cblocks), dim3(256), 0, stream, (const float2*)lam0,
                     gam, (const float2*)segA, (const float2*)segX, dh_final, dsn, dh0, B, NC, H, D, S);
  st = cdssm_host::check_launch("cdssm_fused_scan_bwd/rreplay");
  if (st) return st;
  constexpr int kCk = 16 / (D / kWave);
  const size_t ck_bytes = size_t((Q + kCk - 1) / kCk) * 64 * (D / kWave) * sizeof(float4);
  hipLaunchKernelGGL((fused_bwd_main_kernel<T, D>), dim3(unsigned(tiles)), dim3(kWave), ck_bytes, stream,
                     (const raw*)q, (const raw*)k, (const raw*)v, (const raw*)beta, (const raw*)sel_c,
                     (const raw*)dt, (const raw*)r, alpha, omega, c, (const raw*)dy, states,
                     (const float2*)dsn, (raw*)dq, (raw*)dk, (raw*)dv, (raw*)dbeta, (raw*)dsel, (raw*)ddt,
                     (raw*)dr, parts, L, H, Q, NC);
  st = cdssm_host::check_launch("cdssm_fused_scan_bwd/main");
  if (st) return st;
  hipLaunchKernelGGL(fused_bwd_heads_kernel, dim3(unsigned(H)), dim3(256), 0, stream,
                     (const float2*)parts, dalpha, domega, B * NC, H);
  return cdssm_host::check_launch("cdssm_fused_scan_bwd/heads");
}

}  // namespace

extern "C" int64_t cdssm_fused_scan_bwd_workspace_bytes(int64_t B, int64_t L, int64_t H, int64_t D,
                                                        int64_t N, int64_t chunk) {
  if (B <= 0 || L <= 0 || H <= 0 || D <= 0 || N != 2 || chunk <= 0) return -1;
  return bwd_layout(B, L, H, D, chunk).total() * int64_t(sizeof(float2));
}

extern "C" int cdssm_fused_scan_bwd(int dtype, const void* q, const void* k, const void* v,
                                    const void* beta, const void* sel_c, const void* dt,
                                    const void* r, const float* alpha, const float* omega, float c,
                                    const void* dy, const float* dh_final, const float* fwd_workspace,
                                    void* dq, void* dk, void* dv, void* dbeta, void* dsel, void* ddt,
                                    void* dr, float* dalpha, float* domega, float* dh0, float* workspace,
                                    int64_t B, int64_t L, int64_t H, int64_t D, int64_t N,
                                    int64_t chunk, hipStream_t stream) {
  const char* op = "cdssm_fused_scan_bwd";
  if (dtype != 0 && dtype != 1) {
    cdssm_host::set_error("%s: dtype must be 0 (fp32) or 1 (bf16), got %d", op, dtype);
    return CDSSM_EINVAL;
  }
  if (B <= 0 || L <= 0 || H <= 0) {
    cdssm_host::set_error("%s: B, L, H must be positive", op);
    return CDSSM_EINVAL;
  }
  if (N != 2) {
    cdssm_host::set_error("%s: the fused scan supports state_dim N = 2, got %lld", op, (long long)N);
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
  if (!q || !k || !v || !beta || !sel_c || !dt || !r || !alpha || !omega || !dy || !fwd_workspace ||
      !dq || !dk || !dv || !dbeta || !dsel || !ddt || !dr || !dalpha || !domega || !workspace) {
    cdssm_host::set_error("%s: null pointer argument", op);
    return CDSSM_EINVAL;
  }
  const int b = int(B), l = int(L), hh = int(H), qc = int(chunk);
  if (dtype == 1) {
    if (D == 64)
      return launch_fused_bwd<BF16, 64>(q, k, v, beta, sel_c, dt, r, alpha, omega, c, dy, dh_final,
                                        fwd_workspace, dq, dk, dv, dbeta, dsel, ddt, dr, dalpha, domega,
                                        dh0, workspace, b, l, hh, qc, stream);
    return launch_fused_bwd<BF16, 128>(q, k, v, beta, sel_c, dt, r, alpha, omega, c, dy, dh_final,
                                       fwd_workspace, dq, dk, dv, dbeta, dsel, ddt, dr, dalpha, domega,
                                       dh0, workspace, b, l, hh, qc, stream);
  }
  if (D == 64)
    return launch_fused_bwd<F32, 64>(q, k, v, beta, sel_c, dt, r, alpha, omega, c, dy, dh_final,
                                     fwd_workspace, dq, dk, dv, dbeta, dsel, ddt, dr, dalpha, domega, dh0,
                                     workspace, b, l, hh, qc, stream);
  return launch_fused_bwd<F32, 128>(q, k, v, beta, sel_c, dt, r, alpha, omega, c, dy, dh_final,
                                    fwd_workspace, dq, dk, dv, dbeta, dsel, ddt, dr, dalpha, domega, dh0,
                                    workspace, b, l, hh, qc, stream);
}
