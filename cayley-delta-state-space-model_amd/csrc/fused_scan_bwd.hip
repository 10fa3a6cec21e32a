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
//   B3 main:    per chunk: forward recompute (z checkpoints every 16 steps),
//               then segment-wise reverse of both branches, emitting dq, dk,
//               dv, dbeta, dsel_C, ddt, dr and per-chunk d alpha / d omega
//   B4 heads:   deterministic sum of the per-chunk d alpha / d omega.
//
// Work layout of B1 and B3: one wave64 per (b, chunk, h); lane owns
// DPL = D/64 state elements; per-token scalars are computed one token per
// lane (two slots for 128-token chunks) and read back from LDS.
#include "common.hpp"

namespace cdssm {

constexpr int kBwdSeg = 16;

__device__ __forceinline__ float rl(float x, int lane) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), lane));
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

// A lane's DPL contiguous state columns d = lane*DPL + j of one row.
template <typename T, int DPL>
struct Cols {
  float x[DPL];
  __device__ __forceinline__ void load(const typename T::raw* p) {
#pragma unroll
    for (int j = 0; j < DPL; ++j) x[j] = T::load(p + j);
  }
  // Opaque copy that keeps prefetched values in their registers (see RowVec::pin).
  __device__ __forceinline__ void pin() {
#pragma unroll
    for (int j = 0; j < DPL; ++j) asm volatile("" : "+v"(x[j]));
  }
};

// Sum of NV <= 8 values over the 64 lanes of a one-wave block, returned to
// every lane.  Transposes through LDS: lane l writes its NV partials, then
// lane l adds 8 lanes' partials of value l%8, and three swizzle/permute
// stages combine the 8 blocks.  scratch: 8*65 floats.
template <int NV>
__device__ __forceinline__ void wave_reduce(float (&v)[NV], float* scratch) {
  static_assert(NV >= 1 && NV <= 8, "up to 8 values");
  const int lane = threadIdx.x;
#pragma unroll
  for (int i = 0; i < NV; ++i) scratch[i * 65 + lane] = v[i];
  asm volatile("" ::: "memory");
  const int vi = lane & 7, blk = lane >> 3;
  float s = 0.0f;
  if (vi < NV) {
    const float* row = scratch + vi * 65 + blk * 8;
#pragma unroll
    for (int i = 0; i < 8; ++i) s += row[i];
  }
  s += __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(s), 0x201F));  // lane ^ 8
  s += __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(s), 0x401F));  // lane ^ 16
  s += __shfl_xor(s, 32, 64);
  asm volatile("" ::: "memory");
#pragma unroll
  for (int i = 0; i < NV; ++i) v[i] = rl(s, i);
}

// ---------------------------------------------------------------------------
// B1: correction-branch adjoint of the entering state, per chunk.
//   lambda = 0; for t = n-1..0: lambda += conj(g_t) sel_t dy_t q_t;
//   lambda <- lambda - beta_t (lambda.k_t) k_t.   Result: lambda_0 = d s_k.
// ---------------------------------------------------------------------------
template <typename T, int D>
__global__ __launch_bounds__(kWave) void fused_bwd_corr_kernel(
    const typename T::raw* __restrict__ q, const typename T::raw* __restrict__ k,
    const typename T::raw* __restrict__ v, const typename T::raw* __restrict__ beta,
    const typename T::raw* __restrict__ sel_c, const typename T::raw* __restrict__ dt,
    const typename T::raw* __restrict__ r, const float* __restrict__ alpha,
    const float* __restrict__ omega, float c, const typename T::raw* __restrict__ dy,
    float2* __restrict__ lam0, int L, int H, int Q, int NC) {
  constexpr int DPL = D / kWave, PF = 8;
  __shared__ float4 sh[128];  // (h_re, h_im, beta, 0) per token
  const BwdTile tc = bwd_tile(L, Q, NC, H);
  const int lane = threadIdx.x;
  {
    TokenInputs<T> in;
    in.load(tc, H, v, beta, sel_c, dt, r, dy, alpha[tc.h], omega[tc.h], c);
    float gr[2], gi[2], gpr[2], gpi[2];
    prefix_prod(in.ar, in.ai, gr, gi, gpr, gpi);
#pragma unroll
    for (int s2 = 0; s2 < 2; ++s2) {
      const int t = lane + 64 * s2;
      if (t < Q) {
        const float fr = in.sel[s2] * in.dyr[s2], fi = in.sel[s2] * in.dyi[s2];
        sh[t] = make_float4(gr[s2] * fr + gi[s2] * fi, gr[s2] * fi - gi[s2] * fr, in.b[s2], 0.0f);
      }
    }
  }
  __syncthreads();

  const int64_t stride = int64_t(H) * D;
  const int64_t off = (tc.row0 * H + tc.h) * D + lane * DPL;
  const typename T::raw* kp = k + off;
  const typename T::raw* qp = q + off;
  const int tlast = tc.nt - 1;
  float lr[DPL], li[DPL];
#pragma unroll
  for (int j = 0; j < DPL; ++j) lr[j] = li[j] = 0.0f;
  // reverse order, rows prefetched PF tokens ahead
  Cols<T, DPL> kb[PF], qb[PF];
#pragma unroll
  for (int i = 0; i < PF; ++i) {
    const int t = max(tlast - i, 0);
    kb[i].load(kp + t * stride);
    qb[i].load(qp + t * stride);
  }
#pragma unroll
  for (int i = 0; i < PF; ++i) {
    kb[i].pin();
    qb[i].pin();
  }
  const int nr = (tc.nt + PF - 1) / PF * PF;
  for (int ib = 0; ib < nr; ib += PF) {
#pragma unroll
    for (int i = 0; i < PF; ++i) {
      const int t = tlast - (ib + i);  // may go negative: inert (h = 0, beta = 0)
      float kk[DPL], qq[DPL];
#pragma unroll
      for (int j = 0; j < DPL; ++j) {
        kk[j] = kb[i].x[j];
        qq[j] = qb[i].x[j];
      }
      const int tn = max(t - PF, 0);
      kb[i].load(kp + tn * stride);
      qb[i].load(qp + tn * stride);
      const float4 hv = t >= 0 ? sh[t] : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
      float sr = 0.0f, si = 0.0f;
#pragma unroll
      for (int j = 0; j < DPL; ++j) {
        lr[j] = fmaf(hv.x, qq[j], lr[j]);
        li[j] = fmaf(hv.y, qq[j], li[j]);
        sr = fmaf(lr[j], kk[j], sr);
        si = fmaf(li[j], kk[j], si);
      }
      sr = wsum(sr);
      si = wsum(si);
#pragma unroll
      for (int j = 0; j < DPL; ++j) {
        lr[j] = fmaf(-hv.z * sr, kk[j], lr[j]);
        li[j] = fmaf(-hv.z * si, kk[j], li[j]);
      }
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
// B3: per-chunk backward of both branches.
//   forward pass: z and c^ from (0, s_k); per token keeps p_t = z_{t-1}.k_t,
//     pc_t = c^_t.k_t, Y_t.q_t and the correction's delta g_t in LDS, emits dq,
//     and stores z every CK tokens;
//   reverse pass, CK tokens at a time: z of the segment is recomputed from its
//     checkpoint with the stored p_t (no reductions); c^_t is rebuilt backward,
//     exactly, as c^_t = c^_{t+1} + beta_t pc_t k_t; the local adjoint mu and
//     the correction adjoint lambda step back and dk is emitted;
//   epilogue, one token per lane: dynamics chain rule, dv, dbeta, dsel, ddt,
//     dr, and the chunk's d alpha / d omega partial.
// LDS (float4 per token unless noted): S0 (a, w), S1 (beta, f = sel dy),
// S2 (h = conj(g_t) f, g_{t-1}), P (p, pc), G (delta g, Y.q), R (da, dw),
// RB (dbeta from the erasures, float), z checkpoints, reduction scratch.
// ---------------------------------------------------------------------------
template <int D>
struct BwdSmem {
  static constexpr int DPL = D / kWave;
  static constexpr int CK = 16;
  static constexpr int QMAX = 128;
  float4 S0[QMAX], S1[QMAX], S2[QMAX], P[QMAX], G[QMAX], R[QMAX];
  float RB[QMAX];
  float2 ck[QMAX / CK][kWave * DPL];
  float red[8 * 65];
};

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
  using SM = BwdSmem<D>;
  constexpr int DPL = SM::DPL, CK = SM::CK, PF = 8;
  __shared__ SM sm;
  const BwdTile tc = bwd_tile(L, Q, NC, H);
  const int lane = threadIdx.x;
  const float al = alpha[tc.h], om = omega[tc.h];

  // ---- per-token scalars (lane = token, two slots) ----
  TokenInputs<T> in;
  in.load(tc, H, v, beta, sel_c, dt, r, dy, al, om, c);
  {
    float gr[2], gi[2], gpr[2], gpi[2];
    prefix_prod(in.ar, in.ai, gr, gi, gpr, gpi);
#pragma unroll
    for (int s2 = 0; s2 < 2; ++s2) {
      const int t = lane + 64 * s2;
      if (t < Q) {
        const float f = in.b[s2] * in.vp[s2];
        const float fr = in.sel[s2] * in.dyr[s2], fi = in.sel[s2] * in.dyi[s2];
        sm.S0[t] = make_float4(in.ar[s2], in.ai[s2], f * in.vr[s2], f * in.vi[s2]);
        sm.S1[t] = make_float4(in.b[s2], fr, fi, 0.0f);
        sm.S2[t] = make_float4(gr[s2] * fr + gi[s2] * fi, gr[s2] * fi - gi[s2] * fr, gpr[s2], gpi[s2]);
      }
    }
  }
  __syncthreads();

  const int64_t stride = int64_t(H) * D;
  const int64_t off = (tc.row0 * H + tc.h) * D + lane * DPL;
  const typename T::raw* kp = k + off;
  const typename T::raw* qp = q + off;
  const int tlast = tc.nt - 1;
  const int ntr = (tc.nt + CK - 1) / CK * CK;

  // ---- forward pass ----
  float zr[DPL], zi[DPL], cr[DPL], ci[DPL];
  const float2* sp = states + tc.tile * D + lane * DPL;
#pragma unroll
  for (int j = 0; j < DPL; ++j) {
    zr[j] = zi[j] = 0.0f;
    cr[j] = sp[j].x;
    ci[j] = sp[j].y;
  }
  {
    Cols<T, DPL> kb[PF], qb[PF];
#pragma unroll
    for (int i = 0; i < PF; ++i) {
      kb[i].load(kp + min(i, tlast) * stride);
      qb[i].load(qp + min(i, tlast) * stride);
    }
#pragma unroll
    for (int i = 0; i < PF; ++i) {
      kb[i].pin();
      qb[i].pin();
    }
    for (int tb = 0; tb < ntr; tb += PF) {
#pragma unroll
      for (int i = 0; i < PF; ++i) {
        const int t = tb + i;
        float kk[DPL], qq[DPL];
#pragma unroll
        for (int j = 0; j < DPL; ++j) {
          kk[j] = kb[i].x[j];
          qq[j] = qb[i].x[j];
        }
        kb[i].load(kp + min(t + PF, tlast) * stride);
        qb[i].load(qp + min(t + PF, tlast) * stride);
        if (t % CK == 0) {
#pragma unroll
          for (int j = 0; j < DPL; ++j) sm.ck[t / CK][lane * DPL + j] = make_float2(zr[j], zi[j]);
        }
        if (t < tc.nt) {
          const float4 s0 = sm.S0[t], s1 = sm.S1[t], s2 = sm.S2[t];
          float red[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
          for (int j = 0; j < DPL; ++j) {
            red[0] = fmaf(zr[j], kk[j], red[0]);
            red[1] = fmaf(zi[j], kk[j], red[1]);
            red[2] = fmaf(cr[j], kk[j], red[2]);
            red[3] = fmaf(ci[j], kk[j], red[3]);
          }
          wave_reduce<4>(red, sm.red);
          const float pr = red[0], pi = red[1], pcr = red[2], pci = red[3];
          const float ar = s0.x, ai = s0.y, bb = s1.x;
          const float bpr = bb * pr, bpi = bb * pi;
          const float er = s0.z - (ar * bpr - ai * bpi);
          const float ei = s0.w - (ar * bpi + ai * bpr);
          const float ecr = bb * pcr, eci = bb * pci;
          float o4[4] = {0.0f, 0.0f, 0.0f, 0.0f};
          float dqv[DPL];
#pragma unroll
          for (int j = 0; j < DPL; ++j) {
            const float nr = fmaf(ar, zr[j], fmaf(-ai, zi[j], er * kk[j]));
            const float ni = fmaf(ar, zi[j], fmaf(ai, zr[j], ei * kk[j]));
            // Y_t = z_t + g_{t-1} c^_t
            const float Yr = nr + s2.z * cr[j] - s2.w * ci[j];
            const float Yi = ni + s2.z * ci[j] + s2.w * cr[j];
            dqv[j] = Yr * s1.y + Yi * s1.z;
            o4[0] = fmaf(Yr, qq[j], o4[0]);
            o4[1] = fmaf(Yi, qq[j], o4[1]);
            zr[j] = nr;
            zi[j] = ni;
            cr[j] = fmaf(-ecr, kk[j], cr[j]);
            ci[j] = fmaf(-eci, kk[j], ci[j]);
            o4[2] = fmaf(cr[j], qq[j], o4[2]);
            o4[3] = fmaf(ci[j], qq[j], o4[3]);
          }
          const int64_t o = off + int64_t(t) * stride;
#pragma unroll
          for (int j = 0; j < DPL; ++j) T::store(dq + o + j, dqv[j]);
          wave_reduce<4>(o4, sm.red);
          if (lane == 0) {
            // delta g_t = f conj(c^_{t+1}.q)
            sm.P[t] = make_float4(pr, pi, pcr, pci);
            sm.G[t] = make_float4(s1.y * o4[2] + s1.z * o4[3], s1.z * o4[2] - s1.y * o4[3], o4[0], o4[1]);
          }
        }
      }
    }
  }
  __syncthreads();

  // ---- reverse pass ----
  float mr[DPL], mi[DPL], lr[DPL], li[DPL];
  float dG[2] = {0.0f, 0.0f};
  {
    const float2* dp = dsn + tc.tile * D + lane * DPL;
#pragma unroll
    for (int j = 0; j < DPL; ++j) {
      const float2 ds = dp[j];
      const float2 s0 = sp[j];
      mr[j] = ds.x;
      mi[j] = ds.y;
      lr[j] = li[j] = 0.0f;
      dG[0] = fmaf(ds.x, s0.x, fmaf(ds.y, s0.y, dG[0]));
      dG[1] = fmaf(ds.y, s0.x, fmaf(-ds.x, s0.y, dG[1]));
    }
    wave_reduce<2>(dG, sm.red);
  }
  float psr = 0.0f, psi = 0.0f;  // psi_{t+1}
  float anr = 1.0f, ani = 0.0f;  // a_{t+1}
  for (int seg = ntr / CK - 1; seg >= 0; --seg) {
    const int tb = seg * CK;
    Cols<T, DPL> ks[CK], qs[CK];
#pragma unroll
    for (int i = 0; i < CK; ++i) {
      ks[i].load(kp + min(tb + i, tlast) * stride);
      qs[i].load(qp + min(tb + i, tlast) * stride);
    }
    // z_{tb-1+i} for i = 0..CK (recomputed with the stored p_t)
    float zbr[CK + 1][DPL], zbi[CK + 1][DPL];
#pragma unroll
    for (int j = 0; j < DPL; ++j) {
      const float2 z0 = sm.ck[seg][lane * DPL + j];
      zbr[0][j] = z0.x;
      zbi[0][j] = z0.y;
    }
#pragma unroll
    for (int i = 0; i < CK; ++i) {
      const int t = tb + i;
      // steps past the chunk's last token are inert (their LDS slots may be unset)
      const bool real = t < tc.nt;
      const float4 s0 = sm.S0[t];
      const float4 pv = sm.P[t];
      const float bb = sm.S1[t].x;
      const float ar = real ? s0.x : 1.0f, ai = real ? s0.y : 0.0f;
      const float wr = real ? s0.z : 0.0f, wi = real ? s0.w : 0.0f;
      const float bpr = real ? bb * pv.x : 0.0f, bpi = real ? bb * pv.y : 0.0f;
      const float er = wr - (ar * bpr - ai * bpi);
      const float ei = wi - (ar * bpi + ai * bpr);
#pragma unroll
      for (int j = 0; j < DPL; ++j) {
        zbr[i + 1][j] = fmaf(ar, zbr[i][j], fmaf(-ai, zbi[i][j], er * ks[i].x[j]));
        zbi[i + 1][j] = fmaf(ar, zbi[i][j], fmaf(ai, zbr[i][j], ei * ks[i].x[j]));
      }
    }
#pragma unroll
    for (int i = CK - 1; i >= 0; --i) {
      const int t = tb + i;
      if (t < tc.nt) {
        const float4 s0 = sm.S0[t], s1 = sm.S1[t], s2 = sm.S2[t], pv = sm.P[t], gv = sm.G[t];
        const float ar = s0.x, ai = s0.y, wr = s0.z, wi = s0.w, bb = s1.x;
        const float pr = pv.x, pi = pv.y, pcr = pv.z, pci = pv.w;
        float red[6] = {0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int j = 0; j < DPL; ++j) {
          const float kv = ks[i].x[j], qv = qs[i].x[j];
          // c^_t = c^_{t+1} + beta pc k
          cr[j] = fmaf(bb * pcr, kv, cr[j]);
          ci[j] = fmaf(bb * pci, kv, ci[j]);
          mr[j] = fmaf(s1.y, qv, mr[j]);
          mi[j] = fmaf(s1.z, qv, mi[j]);
          lr[j] = fmaf(s2.x, qv, lr[j]);
          li[j] = fmaf(s2.y, qv, li[j]);
          red[0] = fmaf(mr[j], kv, red[0]);
          red[1] = fmaf(mi[j], kv, red[1]);
          red[2] = fmaf(mr[j], zbr[i][j], fmaf(mi[j], zbi[i][j], red[2]));
          red[3] = fmaf(mi[j], zbr[i][j], fmaf(-mr[j], zbi[i][j], red[3]));
          red[4] = fmaf(lr[j], kv, red[4]);
          red[5] = fmaf(li[j], kv, red[5]);
        }
        wave_reduce<6>(red, sm.red);
        const float dwr = red[0], dwi = red[1], slr = red[4], sli = red[5];
        const float mkr = ar * dwr + ai * dwi, mki = ar * dwi - ai * dwr;
        float dar = red[2] - bb * (pr * dwr + pi * dwi);
        float dai = red[3] - bb * (pr * dwi - pi * dwr);
        const float dbe = -(pr * mkr + pi * mki) - (pcr * slr + pci * sli);
        float dgr = gv.x, dgi = gv.y;
        if (t == tc.nt - 1) {
          dgr += dG[0];
          dgi += dG[1];
        }
        const float npr = dgr + anr * psr + ani * psi;
        const float npi = dgi + anr * psi - ani * psr;
        psr = npr;
        psi = npi;
        anr = ar;
        ani = ai;
        dar += s2.z * psr + s2.w * psi;
        dai += s2.z * psi - s2.w * psr;
        float dkv[DPL];
#pragma unroll
        for (int j = 0; j < DPL; ++j) {
          const float kv = ks[i].x[j];
          const float m_r = ar * mr[j] + ai * mi[j], m_i = ar * mi[j] - ai * mr[j];
          dkv[j] = mr[j] * wr + mi[j] * wi -
                   bb * (zbr[i][j] * mkr + zbi[i][j] * mki + m_r * pr + m_i * pi) -
                   bb * (cr[j] * slr + ci[j] * sli + lr[j] * pcr + li[j] * pci);
          mr[j] = fmaf(-bb * mkr, kv, m_r);
          mi[j] = fmaf(-bb * mki, kv, m_i);
          lr[j] = fmaf(-bb * slr, kv, lr[j]);
          li[j] = fmaf(-bb * sli, kv, li[j]);
        }
        const int64_t o = off + int64_t(t) * stride;
#pragma unroll
        for (int j = 0; j < DPL; ++j) T::store(dk + o + j, dkv[j]);
        if (lane == 0) {
          sm.R[t] = make_float4(dar, dai, dwr, dwi);
          sm.RB[t] = dbe;
        }
      }
    }
  }
  __syncthreads();

  // ---- per-token dynamics backward (lane = token) ----
  float dal = 0.0f, dom = 0.0f;
#pragma unroll
  for (int s2 = 0; s2 < 2; ++s2) {
    const int t = lane + 64 * s2;
    if (t < tc.nt) {
      const float4 rv = sm.R[t];
      const float4 gv = sm.G[t];
      const float bb = in.b[s2], vp = in.vp[s2], vr = in.vr[s2], vi = in.vi[s2];
      const float dwv = rv.z * vr + rv.w * vi;
      const float dbeta_t = sm.RB[t] + vp * dwv;
      const float dvp = bb * dwv;
      const DynGrad g = cayley_gated_bwd(in.dt[s2], in.r[s2], al, om, c, rv.x, rv.y, dvp);
      const int64_t e = (tc.row0 + t) * H + tc.h;
      T::store(dv + 2 * e, bb * vp * rv.z);
      T::store(dv + 2 * e + 1, bb * vp * rv.w);
      T::store(dbeta + e, dbeta_t);
      T::store(dsel + e, in.dyr[s2] * gv.z + in.dyi[s2] * gv.w);
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
  hipLaunchKernelGGL((fused_bwd_main_kernel<T, D>), dim3(unsigned(tiles)), dim3(kWave), 0, stream,
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
