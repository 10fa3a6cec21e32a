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
// Three launches, all on the caller's stream:
//   1. summary:  one pass over k, v, beta, dt, r per chunk -> (F_k = z_{Q-1}, G_k)
//   2. carry:    per (b, h, d) scan of s_{k+1} = G_k s_k + F_k over chunks, in
//                three phases (segment fold, segment prefix, segment replay) so
//                the serial depth is ~2 NC/S + S instead of NC;
//   3. main:     per chunk: z and c^ recurrences with the readout; writes y.
//
// Work layout of passes 1 and 3: one wave64 holds HPW = 64/LPH heads of one
// (b, chunk); each head is owned by LPH consecutive lanes, each lane holding
// DPL = D/LPH consecutive state elements, so every q/k row is read with one
// 16-byte load per lane and a head's 64..256-byte row is one contiguous
// segment.  Dot products reduce over the LPH lanes with DPP.  The per-token
// scalars (a, w, beta, sel_C) are computed once per token-head into LDS.
#include "common.hpp"

namespace cdssm {

template <typename T, int D, int LPH>
struct FusedCfg {
  static constexpr int DPL = D / LPH;
  static constexpr int HPW = kWave / LPH;
  static_assert(DPL == Vec16<T>::n, "one 16-byte vector per lane per row");
  static_assert(HPW * LPH == kWave, "lane groups tile the wave");
};

constexpr int kPrefetch = 4;

// Decode blockIdx.x -> (b, chunk, head group).
struct ChunkTile {
  int b, chunk, hbase, t0, nt;
  int64_t row0;
};

__device__ __forceinline__ ChunkTile decode_tile(int L, int Q, int NC, int n_hg, int HPW) {
  ChunkTile c;
  int g = blockIdx.x;
  const int hg = g % n_hg;
  g /= n_hg;
  c.chunk = g % NC;
  c.b = g / NC;
  c.hbase = hg * HPW;
  c.t0 = c.chunk * Q;
  c.nt = min(Q, L - c.t0);
  c.row0 = int64_t(c.b) * L + c.t0;
  return c;
}

// Stage per-token scalars of the tile into LDS.  Slot p = t*HPW + j.
// Heads beyond H get an inert step (a = 1, w = 0, beta = 0).
template <typename T, bool WITH_SELC>
__device__ __forceinline__ void stage_scalars(const ChunkTile& tc, int H, int HPW,
                                              const typename T::raw* __restrict__ v,
                                              const typename T::raw* __restrict__ beta,
                                              const typename T::raw* __restrict__ sel_c,
                                              const typename T::raw* __restrict__ dt,
                                              const typename T::raw* __restrict__ r,
                                              const float* __restrict__ alpha,
                                              const float* __restrict__ omega, float c,
                                              float* s_ar, float* s_ai, float* s_wr, float* s_wi,
                                              float* s_b, float* s_sc) {
  const int n = tc.nt * HPW;
  for (int p = threadIdx.x; p < n; p += kWave) {
    const int t = p / HPW;
    const int hj = tc.hbase + (p - t * HPW);
    float ar = 1.0f, ai = 0.0f, wr = 0.0f, wi = 0.0f, bb = 0.0f, sc = 0.0f;
    if (hj < H) {
      const int64_t e = (tc.row0 + t) * H + hj;
      bb = T::load(beta + e);
      const Transition tr = cayley_gated(T::load(dt + e), T::load(r + e), alpha[hj], omega[hj], c);
      ar = tr.ar;
      ai = tr.ai;
      const float s = bb * tr.vp;
      wr = s * T::load(v + 2 * e);
      wi = s * T::load(v + 2 * e + 1);
      if constexpr (WITH_SELC) sc = T::load(sel_c + e);
    }
    s_ar[p] = ar;
    s_ai[p] = ai;
    s_wr[p] = wr;
    s_wi[p] = wi;
    s_b[p] = bb;
    if constexpr (WITH_SELC) s_sc[p] = sc;
  }
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
    int L, int H, int Q, int NC, int n_hg) {
  using Cfg = FusedCfg<T, D, LPH>;
  constexpr int DPL = Cfg::DPL, HPW = Cfg::HPW;
  extern __shared__ float smem[];
  const ChunkTile tc = decode_tile(L, Q, NC, n_hg, HPW);
  const int lane = threadIdx.x;
  const int hh = lane / LPH;
  const int sub = lane % LPH;
  const int h = tc.hbase + hh;
  const bool hok = h < H;

  float* s_ar = smem;
  float* s_ai = s_ar + Q * HPW;
  float* s_wr = s_ai + Q * HPW;
  float* s_wi = s_wr + Q * HPW;
  float* s_b = s_wi + Q * HPW;
  stage_scalars<T, false>(tc, H, HPW, v, beta, nullptr, dt, r, alpha, omega, c, s_ar, s_ai, s_wr,
                          s_wi, s_b, nullptr);
  __syncthreads();

  float zr[DPL], zi[DPL];
#pragma unroll
  for (int j = 0; j < DPL; ++j) zr[j] = zi[j] = 0.0f;
  float gr = 1.0f, gi = 0.0f;

  const int64_t stride = int64_t(H) * D;
  const typename T::raw* kp = k + (tc.row0 * H + (hok ? h : 0)) * D + sub * DPL;
  const uint4 zero4 = make_uint4(0, 0, 0, 0);
  uint4 kb[kPrefetch];
#pragma unroll
  for (int i = 0; i < kPrefetch; ++i) kb[i] = (hok && i < tc.nt) ? ld16(kp + i * stride) : zero4;

  for (int tb = 0; tb < tc.nt; tb += kPrefetch) {
#pragma unroll
    for (int i = 0; i < kPrefetch; ++i) {
      const int t = tb + i;
      if (t < tc.nt) {
        float kk[DPL];
        Vec16<T>::unpack(kb[i], kk);
        kb[i] = (hok && t + kPrefetch < tc.nt) ? ld16(kp + (t + kPrefetch) * stride) : zero4;
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
        const int s = t * HPW + hh;
        const float ar = s_ar[s], ai = s_ai[s], wr = s_wr[s], wi = s_wi[s], bb = s_b[s];
        const float bpr = bb * pr, bpi = bb * pi;
        // z <- a (z - beta p k) + w k = a z + (w - a beta p) k
        const float cr = wr - (ar * bpr - ai * bpi);
        const float ci = wi - (ar * bpi + ai * bpr);
#pragma unroll
        for (int j = 0; j < DPL; ++j) {
          const float nr = fmaf(ar, zr[j], fmaf(-ai, zi[j], cr * kk[j]));
          const float ni = fmaf(ar, zi[j], fmaf(ai, zr[j], ci * kk[j]));
          zr[j] = nr;
          zi[j] = ni;
        }
        const float ngr = ar * gr - ai * gi;
        gi = ar * gi + ai * gr;
        gr = ngr;
      }
    }
  }

  if (hok) {
    const int64_t ch = (int64_t(tc.b) * NC + tc.chunk) * H + h;
    float2* sp = summ + ch * D + sub * DPL;
#pragma unroll
    for (int j = 0; j < DPL; ++j) sp[j] = make_float2(zr[j], zi[j]);
    if (sub == 0) gam[ch] = make_float2(gr, gi);
  }
}

// ---------------------------------------------------------------------------
// Pass 2: inter-chunk carry, s_{k+1} = G_k s_k + F_k (elementwise complex).
// One block per (b, h) with D * S threads; thread (seg, d) owns chunks
// [seg*len, (seg+1)*len).  Overwrites F_k with the entering state s_k and
// writes the final state s_NC as (B, H, 2, D) fp32 (row 0 = re, row 1 = im).
// ---------------------------------------------------------------------------
__device__ __forceinline__ float2 cmul(float2 a, float2 b) {
  return make_float2(a.x * b.x - a.y * b.y, a.x * b.y + a.y * b.x);
}
__device__ __forceinline__ float2 cfma(float2 a, float2 b, float2 c) {
  return make_float2(fmaf(a.x, b.x, fmaf(-a.y, b.y, c.x)), fmaf(a.x, b.y, fmaf(a.y, b.x, c.y)));
}

__global__ __launch_bounds__(1024) void fused_fwd_carry_kernel(float2* __restrict__ summ,
                                                               const float2* __restrict__ gam,
                                                               const float* __restrict__ h0,
                                                               float* __restrict__ h_final, int NC,
                                                               int H, int D, int S) {
  extern __shared__ float2 csm[];  // [S] segment transitions, then [S][D] segment folds
  float2* s_A = csm;
  float2* s_X = csm + S;
  const int b = blockIdx.x / H;
  const int h = blockIdx.x % H;
  const int d = threadIdx.x % D;
  const int seg = threadIdx.x / D;
  const int len = (NC + S - 1) / S;
  const int c0 = min(NC, seg * len);
  const int c1 = min(NC, c0 + len);
  const int64_t base = (int64_t(b) * NC) * H + h;  // chunk ch -> base + ch*H

  // phase 1: fold the segment from zero
  float2 A = make_float2(1.0f, 0.0f), X = make_float2(0.0f, 0.0f);
  for (int ch = c0; ch < c1; ++ch) {
    const int64_t e = base + int64_t(ch) * H;
    const float2 G = gam[e];
    X = cfma(G, X, summ[e * D + d]);
    A = cmul(G, A);
  }
  s_X[seg * D + d] = X;
  if (d == 0) s_A[seg] = A;
  __syncthreads();

  // phase 2: state entering the segment
  float2 s = make_float2(0.0f, 0.0f);
  if (h0 != nullptr) {
    const int64_t hb = (int64_t(b) * H + h) * 2 * D;
    s = make_float2(h0[hb + d], h0[hb + D + d]);
  }
  for (int j = 0; j < seg; ++j) s = cfma(s_A[j], s, s_X[j * D + d]);

  // phase 3: replay, writing entering states
  for (int ch = c0; ch < c1; ++ch) {
    const int64_t e = base + int64_t(ch) * H;
    const float2 G = gam[e];
    const float2 F = summ[e * D + d];
    summ[e * D + d] = s;
    s = cfma(G, s, F);
  }
  if (c0 < c1 && c1 == NC) {
    const int64_t hb = (int64_t(b) * H + h) * 2 * D;
    h_final[hb + d] = s.x;
    h_final[hb + D + d] = s.y;
  }
}

// ---------------------------------------------------------------------------
// Pass 3: per chunk, local state z and decay-free correction c^ from s_k,
// output y_t = sel_C_t ((z_t + g_{t-1} c^_t) . q_t).
// ---------------------------------------------------------------------------
template <typename T, int D, int LPH>
__global__ __launch_bounds__(kWave) void fused_fwd_main_kernel(
    const typename T::raw* __restrict__ q, const typename T::raw* __restrict__ k,
    const typename T::raw* __restrict__ v, const typename T::raw* __restrict__ beta,
    const typename T::raw* __restrict__ sel_c, const typename T::raw* __restrict__ dt,
    const typename T::raw* __restrict__ r, const float* __restrict__ alpha,
    const float* __restrict__ omega, float c, const float2* __restrict__ states,
    typename T::raw* __restrict__ y, int L, int H, int Q, int NC, int n_hg) {
  using Cfg = FusedCfg<T, D, LPH>;
  constexpr int DPL = Cfg::DPL, HPW = Cfg::HPW;
  extern __shared__ float smem[];
  const ChunkTile tc = decode_tile(L, Q, NC, n_hg, HPW);
  const int lane = threadIdx.x;
  const int hh = lane / LPH;
  const int sub = lane % LPH;
  const int h = tc.hbase + hh;
  const bool hok = h < H;

  float* s_ar = smem;
  float* s_ai = s_ar + Q * HPW;
  float* s_wr = s_ai + Q * HPW;
  float* s_wi = s_wr + Q * HPW;
  float* s_b = s_wi + Q * HPW;
  float* s_sc = s_b + Q * HPW;
  float* s_yr = s_sc + Q * HPW;
  float* s_yi = s_yr + Q * HPW;
  stage_scalars<T, true>(tc, H, HPW, v, beta, sel_c, dt, r, alpha, omega, c, s_ar, s_ai, s_wr, s_wi,
                         s_b, s_sc);

  float zr[DPL], zi[DPL], cr[DPL], ci[DPL];
#pragma unroll
  for (int j = 0; j < DPL; ++j) zr[j] = zi[j] = cr[j] = ci[j] = 0.0f;
  if (hok) {
    const float2* sp = states + ((int64_t(tc.b) * NC + tc.chunk) * H + h) * D + sub * DPL;
#pragma unroll
    for (int j = 0; j < DPL; ++j) {
      const float2 sv = sp[j];
      cr[j] = sv.x;
      ci[j] = sv.y;
    }
  }
  __syncthreads();
  float gr = 1.0f, gi = 0.0f;  // g_{t-1}

  const int64_t stride = int64_t(H) * D;
  const int64_t off = (tc.row0 * H + (hok ? h : 0)) * D + sub * DPL;
  const typename T::raw* kp = k + off;
  const typename T::raw* qp = q + off;
  const uint4 zero4 = make_uint4(0, 0, 0, 0);
  uint4 kb[kPrefetch], qb[kPrefetch];
#pragma unroll
  for (int i = 0; i < kPrefetch; ++i) {
    const bool ld = hok && i < tc.nt;
    kb[i] = ld ? ld16(kp + i * stride) : zero4;
    qb[i] = ld ? ld16(qp + i * stride) : zero4;
  }

  for (int tb = 0; tb < tc.nt; tb += kPrefetch) {
#pragma unroll
    for (int i = 0; i < kPrefetch; ++i) {
      const int t = tb + i;
      if (t < tc.nt) {
        float kk[DPL], qq[DPL];
        Vec16<T>::unpack(kb[i], kk);
        Vec16<T>::unpack(qb[i], qq);
        const bool ld = hok && t + kPrefetch < tc.nt;
        kb[i] = ld ? ld16(kp + (t + kPrefetch) * stride) : zero4;
        qb[i] = ld ? ld16(qp + (t + kPrefetch) * stride) : zero4;

        float pzr = 0.0f, pzi = 0.0f, pcr = 0.0f, pci = 0.0f, qcr = 0.0f, qci = 0.0f;
#pragma unroll
        for (int j = 0; j < DPL; ++j) {
          pzr = fmaf(zr[j], kk[j], pzr);
          pzi = fmaf(zi[j], kk[j], pzi);
          pcr = fmaf(cr[j], kk[j], pcr);
          pci = fmaf(ci[j], kk[j], pci);
          qcr = fmaf(cr[j], qq[j], qcr);
          qci = fmaf(ci[j], qq[j], qci);
        }
        pzr = group_sum<LPH>(pzr);
        pzi = group_sum<LPH>(pzi);
        pcr = group_sum<LPH>(pcr);
        pci = group_sum<LPH>(pci);

        const int s = t * HPW + hh;
        const float ar = s_ar[s], ai = s_ai[s], wr = s_wr[s], wi = s_wi[s], bb = s_b[s];
        const float bpr = bb * pzr, bpi = bb * pzi;
        const float er = wr - (ar * bpr - ai * bpi);
        const float ei = wi - (ar * bpi + ai * bpr);
        const float ecr = bb * pcr, eci = bb * pci;
        float qzr = 0.0f, qzi = 0.0f;
#pragma unroll
        for (int j = 0; j < DPL; ++j) {
          const float nr = fmaf(ar, zr[j], fmaf(-ai, zi[j], er * kk[j]));
          const float ni = fmaf(ar, zi[j], fmaf(ai, zr[j], ei * kk[j]));
          zr[j] = nr;
          zi[j] = ni;
          qzr = fmaf(nr, qq[j], qzr);
          qzi = fmaf(ni, qq[j], qzi);
          cr[j] = fmaf(-ecr, kk[j], cr[j]);
          ci[j] = fmaf(-eci, kk[j], ci[j]);
        }
        // readout partial: z_t.q + g_{t-1} (c^_t.q)
        float Rr = qzr + (gr * qcr - gi * qci);
        float Ri = qzi + (gr * qci + gi * qcr);
        Rr = group_sum<LPH>(Rr);
        Ri = group_sum<LPH>(Ri);
        if (sub == 0) {
          const float sc = s_sc[s];
          s_yr[s] = sc * Rr;
          s_yi[s] = sc * Ri;
        }
        const float ngr = ar * gr - ai * gi;
        gi = ar * gi + ai * gr;
        gr = ngr;
      }
    }
  }
  __syncthreads();

  // coalesced write of y (B, L, H, 2) for the tile
  const int n = tc.nt * HPW;
  for (int p = lane; p < n; p += kWave) {
    const int t = p / HPW;
    const int hj = tc.hbase + (p - t * HPW);
    if (hj < H) {
      const int64_t e = ((tc.row0 + t) * H + hj) * 2;
      T::store(y + e, s_yr[p]);
      T::store(y + e + 1, s_yi[p]);
    }
  }
}

}  // namespace cdssm

// ---------------------------------------------------------------------------
// C-ABI
// ---------------------------------------------------------------------------
namespace {

using namespace cdssm;

int carry_segments(int NC, int D) {
  int S = 1024 / D;
  while (S > 1 && S * 2 > NC) S >>= 1;  // no more segments than chunks (roughly)
  return S;
}

template <typename T, int D, int LPH>
int launch_fused_fwd(const void* q, const void* k, const void* v, const void* beta, const void* sel_c,
                     const void* dt, const void* r, const float* alpha, const float* omega, float c,
                     const float* h0, void* y, float* h_final, float* ws, int B, int L, int H, int Q,
                     hipStream_t stream) {
  using raw = typename T::raw;
  constexpr int HPW = kWave / LPH;
  const int NC = (L + Q - 1) / Q;
  const int n_hg = (H + HPW - 1) / HPW;
  const int64_t tiles = int64_t(B) * NC * n_hg;
  if (tiles > 0x7fffffff) {
    cdssm_host::set_error("cdssm_fused_scan_fwd: too many chunk tiles (%lld)", (long long)tiles);
    return CDSSM_EINVAL;
  }
  float2* summ = reinterpret_cast<float2*>(ws);
  float2* gam = summ + int64_t(B) * NC * H * D;

  const size_t sm1 = size_t(5) * Q * HPW * sizeof(float);
  hipLaunchKernelGGL((fused_fwd_summary_kernel<T, D, LPH>), dim3(unsigned(tiles)), dim3(kWave), sm1,
                     stream, (const raw*)k, (const raw*)v, (const raw*)beta, (const raw*)dt,
                     (const raw*)r, alpha, omega, c, summ, gam, L, H, Q, NC, n_hg);
  int st = cdssm_host::check_launch("cdssm_fused_scan_fwd/summary");
  if (st) return st;

  const int S = carry_segments(NC, D);
  const size_t sm2 = size_t(S) * (D + 1) * sizeof(float2);
  hipLaunchKernelGGL(fused_fwd_carry_kernel, dim3(unsigned(B * H)), dim3(unsigned(S * D)), sm2, stream,
                     summ, (const float2*)gam, h0, h_final, NC, H, D, S);
  st = cdssm_host::check_launch("cdssm_fused_scan_fwd/carry");
  if (st) return st;

  const size_t sm3 = size_t(8) * Q * HPW * sizeof(float);
  hipLaunchKernelGGL((fused_fwd_main_kernel<T, D, LPH>), dim3(unsigned(tiles)), dim3(kWave), sm3, stream,
                     (const raw*)q, (const raw*)k, (const raw*)v, (const raw*)beta, (const raw*)sel_c,
                     (const raw*)dt, (const raw*)r, alpha, omega, c, (const float2*)summ, (raw*)y, L, H,
                     Q, NC, n_hg);
  return cdssm_host::check_launch("cdssm_fused_scan_fwd/main");
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

}  // namespace

extern "C" int64_t cdssm_fused_scan_workspace_bytes(int64_t B, int64_t L, int64_t H, int64_t D,
                                                    int64_t N, int64_t chunk) {
  if (B <= 0 || L <= 0 || H <= 0 || D <= 0 || N <= 0 || chunk <= 0) return -1;
  const int64_t NC = (L + chunk - 1) / chunk;
  return (B * NC * H * D * (N / 2) + B * NC * H * (N / 2)) * int64_t(sizeof(float2));
}

extern "C" int cdssm_fused_scan_fwd(int dtype, const void* q, const void* k, const void* v,
                                    const void* beta, const void* sel_c, const void* dt,
                                    const void* r, const float* alpha, const float* omega, float c,
                                    const float* h0, void* y, float* h_final, float* workspace,
                                    int64_t B, int64_t L, int64_t H, int64_t D, int64_t N,
                                    int64_t chunk, hipStream_t stream) {
  const char* op = "cdssm_fused_scan_fwd";
  if (dtype != 0 && dtype != 1) {
    cdssm_host::set_error("%s: dtype must be 0 (fp32) or 1 (bf16), got %d", op, dtype);
    return CDSSM_EINVAL;
  }
  if (B <= 0 || L <= 0 || H <= 0) {
    cdssm_host::set_error("%s: B, L, H must be positive (B=%lld L=%lld H=%lld)", op, (long long)B,
                          (long long)L, (long long)H);
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
  if (!q || !k || !v || !beta || !sel_c || !dt || !r || !alpha || !omega || !y || !h_final ||
      !workspace) {
    cdssm_host::set_error("%s: null pointer argument", op);
    return CDSSM_EINVAL;
  }
  if (!aligned16(q) || !aligned16(k)) {
    cdssm_host::set_error("%s: q and k must be 16-byte aligned", op);
    return CDSSM_EINVAL;
  }
  const int b = int(B), l = int(L), hh = int(H), qc = int(chunk);
  if (dtype == 1) {
    if (D == 64)
      return launch_fused_fwd<BF16, 64, 8>(q, k, v, beta, sel_c, dt, r, alpha, omega, c, h0, y, h_final,
                                           workspace, b, l, hh, qc, stream);
    return launch_fused_fwd<BF16, 128, 16>(q, k, v, beta, sel_c, dt, r, alpha, omega, c, h0, y, h_final,
                                           workspace, b, l, hh, qc, stream);
  }
  if (D == 64)
    return launch_fused_fwd<F32, 64, 16>(q, k, v, beta, sel_c, dt, r, alpha, omega, c, h0, y, h_final,
                                         workspace, b, l, hh, qc, stream);
  return launch_fused_fwd<F32, 128, 32>(q, k, v, beta, sel_c, dt, r, alpha, omega, c, h0, y, h_final,
                                        workspace, b, l, hh, qc, stream);
}
