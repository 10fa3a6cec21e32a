// The reference's three scan passes as separate ops, with its tensor
// contracts, for callers that use IntraChunkScanFn / InterChunkScanFn /
// ExactCorrectionFn directly (ops.py:100-195, ssd.py:83-100).
//
//   intra   (BNC,C,H,N) A, (BNC,C,H,D) K, (BNC,C,H,N) V, (BNC,C,H) beta
//           -> local_h (BNC,C,H,N,D) [state AFTER step t], cum_A (BNC,C,H,N)
//           z_t = A_t (z_{t-1} - beta_t (z_{t-1}.k_t) k_t) + beta_t v_t k_t, z_{-1} = 0
//           (intra_chunk_scan.cu:86-195)
//   inter   (B,NC,H,N) total_A, (B,NC,H,N,D) final_local_h -> chunk_states (B,NC,H,N,D)
//           s_0 = 0, chunk_states[k] = s_k, s_{k+1} = total_A[k] s_k + flh[k]
//           (inter_chunk_scan.cu:49-84)
//   corr    (B,NC,C,H,N) A, (B,NC,C,H,D) K, (B,NC,C,H) beta, (B,NC,H,N,D) states
//           -> corrections (B,NC,C,H,N,D) [state BEFORE step t],
//           c_0 = states[k], c_{t+1} = A_t (c_t - beta_t (c_t.k_t) k_t)
//           (exact_correction.cu:83-150)
// and their backward rules (intra_chunk_scan.cu:215-553,
// inter_chunk_scan.cu:89-196, exact_correction.cu:169-383; the correction rule
// adds grad_corrections[t] before stepping back through step t, as the
// reference does).  The backward passes read the saved forward outputs
// (local_h, cum_A, chunk_states, corrections), as the reference's do.
//
// State rows come in N/2 complex pairs (re, im interleaved) multiplied by the
// stored complex A.  Layout: one wave64 per (unit, head); lane owns state
// columns d = lane + 64 j (j < DPL, D <= 64 * DPL); every dot product is a
// wave-wide DPP/swizzle reduction.  Element type T (bf16 or fp32) for every
// tensor, fp32 arithmetic.  N <= NM (template), even.
#include <type_traits>

#include "common.hpp"

namespace cdssm {
namespace passes {

__device__ __forceinline__ float wsum(float x) { return group_sum<64>(x); }

template <typename T, int DPL>
__device__ __forceinline__ void load_cols(const typename T::raw* p, int D, float (&o)[DPL]) {
  const int lane = threadIdx.x;
#pragma unroll
  for (int j = 0; j < DPL; ++j) {
    const int d = lane + 64 * j;
    o[j] = d < D ? T::load(p + d) : 0.0f;
  }
}
template <typename T, int DPL>
__device__ __forceinline__ void store_cols(typename T::raw* p, int D, const float (&v)[DPL]) {
  const int lane = threadIdx.x;
#pragma unroll
  for (int j = 0; j < DPL; ++j) {
    const int d = lane + 64 * j;
    if (d < D) T::store(p + d, v[j]);
  }
}
template <int DPL>
__device__ __forceinline__ float dot(const float (&a)[DPL], const float (&b)[DPL]) {
  float s = 0.0f;
#pragma unroll
  for (int j = 0; j < DPL; ++j) s = fmaf(a[j], b[j], s);
  return s;
}

// ---------------------------------------------------------------------------
// intra-chunk forward
// ---------------------------------------------------------------------------
template <typename T, int DPL, int NM>
__global__ __launch_bounds__(kWave) void intra_fwd_kernel(
    const typename T::raw* __restrict__ A, const typename T::raw* __restrict__ K,
    const typename T::raw* __restrict__ V, const typename T::raw* __restrict__ beta,
    typename T::raw* __restrict__ local_h, typename T::raw* __restrict__ cum_A, int C, int H, int D,
    int N) {
  const int unit = blockIdx.x / H, h = blockIdx.x % H;
  float hs[NM][DPL];
  float ca[NM];
#pragma unroll
  for (int s = 0; s < NM; ++s) {
#pragma unroll
    for (int j = 0; j < DPL; ++j) hs[s][j] = 0.0f;
    ca[s] = (s % 2 == 0) ? 1.0f : 0.0f;
  }
  for (int t = 0; t < C; ++t) {
    const int64_t row = (int64_t(unit) * C + t) * H + h;
    float kk[DPL];
    load_cols<T, DPL>(K + row * D, D, kk);
    const float bb = T::load(beta + row);
    float a[NM], v[NM], kth[NM];
#pragma unroll
    for (int s = 0; s < NM; ++s) {
      a[s] = s < N ? T::load(A + row * N + s) : 0.0f;
      v[s] = s < N ? T::load(V + row * N + s) : 0.0f;
      kth[s] = s < N ? wsum(dot(hs[s], kk)) : 0.0f;
    }
#pragma unroll
    for (int p = 0; p < NM / 2; ++p) {
      if (2 * p < N) {
        const float ar = a[2 * p], ai = a[2 * p + 1];
#pragma unroll
        for (int j = 0; j < DPL; ++j) {
          const float er = hs[2 * p][j] - bb * kth[2 * p] * kk[j];
          const float ei = hs[2 * p + 1][j] - bb * kth[2 * p + 1] * kk[j];
          hs[2 * p][j] = ar * er - ai * ei + bb * v[2 * p] * kk[j];
          hs[2 * p + 1][j] = ar * ei + ai * er + bb * v[2 * p + 1] * kk[j];
        }
        const float cr = ca[2 * p], ci = ca[2 * p + 1];
        ca[2 * p] = ar * cr - ai * ci;
        ca[2 * p + 1] = ar * ci + ai * cr;
      }
    }
#pragma unroll
    for (int s = 0; s < NM; ++s) {
      if (s < N) {
        store_cols<T, DPL>(local_h + (row * N + s) * D, D, hs[s]);
        if (threadIdx.x == 0) T::store(cum_A + row * N + s, ca[s]);
      }
    }
  }
}

// ---------------------------------------------------------------------------
// intra-chunk backward (exact reverse mode; previous state read from local_h)
// ---------------------------------------------------------------------------
template <typename T, int DPL, int NM>
__global__ __launch_bounds__(kWave) void intra_bwd_kernel(
    const typename T::raw* __restrict__ g_lh, const typename T::raw* __restrict__ g_ca,
    const typename T::raw* __restrict__ A, const typename T::raw* __restrict__ K,
    const typename T::raw* __restrict__ V, const typename T::raw* __restrict__ beta,
    const typename T::raw* __restrict__ local_h, const typename T::raw* __restrict__ cum_A,
    typename T::raw* __restrict__ gA, typename T::raw* __restrict__ gK, typename T::raw* __restrict__ gV,
    typename T::raw* __restrict__ gB, int C, int H, int D, int N) {
  const int unit = blockIdx.x / H, h = blockIdx.x % H;
  float dh[NM][DPL];
  float dca[NM];
#pragma unroll
  for (int s = 0; s < NM; ++s) {
#pragma unroll
    for (int j = 0; j < DPL; ++j) dh[s][j] = 0.0f;
    dca[s] = 0.0f;
  }
  for (int t = C - 1; t >= 0; --t) {
    const int64_t row = (int64_t(unit) * C + t) * H + h;
    const int64_t prow = row - H;  // step t-1 of the same chunk and head
    float kk[DPL];
    load_cols<T, DPL>(K + row * D, D, kk);
    const float bb = T::load(beta + row);
    float a[NM], v[NM], kth[NM], dks[NM], prev[NM];
    float hp[NM][DPL];
#pragma unroll
    for (int s = 0; s < NM; ++s) {
      if (s < N) {
        float g[DPL];
        load_cols<T, DPL>(g_lh + (row * N + s) * D, D, g);
#pragma unroll
        for (int j = 0; j < DPL; ++j) dh[s][j] += g[j];
        if (t > 0) {
          load_cols<T, DPL>(local_h + (prow * N + s) * D, D, hp[s]);
          prev[s] = T::load(cum_A + prow * N + s);
        } else {
#pragma unroll
          for (int j = 0; j < DPL; ++j) hp[s][j] = 0.0f;
          prev[s] = (s % 2 == 0) ? 1.0f : 0.0f;
        }
        a[s] = T::load(A + row * N + s);
        v[s] = T::load(V + row * N + s);
        dca[s] += T::load(g_ca + row * N + s);
        kth[s] = wsum(dot(hp[s], kk));
        dks[s] = wsum(dot(dh[s], kk));
      } else {
        a[s] = v[s] = kth[s] = dks[s] = prev[s] = 0.0f;
#pragma unroll
        for (int j = 0; j < DPL; ++j) hp[s][j] = 0.0f;
      }
    }
    float gk[DPL];
#pragma unroll
    for (int j = 0; j < DPL; ++j) gk[j] = 0.0f;
    float gb = 0.0f;
#pragma unroll
    for (int p = 0; p < NM / 2; ++p) {
      if (2 * p < N) {
        const int s0 = 2 * p, s1 = 2 * p + 1;
        const float ar = a[s0], ai = a[s1];
        // injection terms
        if (threadIdx.x == 0) {
          T::store(gV + row * N + s0, bb * dks[s0]);
          T::store(gV + row * N + s1, bb * dks[s1]);
        }
        gb += v[s0] * dks[s0] + v[s1] * dks[s1];
        // rotation: grad of stored A from the state path, sum_d dh conj(hm)
        float gre = 0.0f, gim = 0.0f;
#pragma unroll
        for (int j = 0; j < DPL; ++j) {
          const float hmr = hp[s0][j] - bb * kth[s0] * kk[j];
          const float hmi = hp[s1][j] - bb * kth[s1] * kk[j];
          gre = fmaf(dh[s0][j], hmr, fmaf(dh[s1][j], hmi, gre));
          gim = fmaf(dh[s1][j], hmr, fmaf(-dh[s0][j], hmi, gim));
        }
        gre = wsum(gre);
        gim = wsum(gim);
        // cum_A path: grad += dcA conj(cum_A[t-1]); dcA <- conj(A_t) dcA
        const float dcr = dca[s0], dci = dca[s1];
        gre += dcr * prev[s0] + dci * prev[s1];
        gim += dci * prev[s0] - dcr * prev[s1];
        dca[s0] = ar * dcr + ai * dci;
        dca[s1] = ar * dci - ai * dcr;
        if (threadIdx.x == 0) {
          T::store(gA + row * N + s0, gre);
          T::store(gA + row * N + s1, gim);
        }
        // back through the rotation: dhm = conj(A) dh, zeta = dhm . k
        const float zr = ar * dks[s0] + ai * dks[s1];
        const float zi = ar * dks[s1] - ai * dks[s0];
        gb -= kth[s0] * zr + kth[s1] * zi;
#pragma unroll
        for (int j = 0; j < DPL; ++j) {
          const float mr = ar * dh[s0][j] + ai * dh[s1][j];
          const float mi = ar * dh[s1][j] - ai * dh[s0][j];
          gk[j] += bb * (v[s0] * dh[s0][j] + v[s1] * dh[s1][j]);
          gk[j] -= bb * (kth[s0] * mr + kth[s1] * mi + hp[s0][j] * zr + hp[s1][j] * zi);
          dh[s0][j] = mr - bb * zr * kk[j];
          dh[s1][j] = mi - bb * zi * kk[j];
        }
      }
    }
    store_cols<T, DPL>(gK + row * D, D, gk);
    if (threadIdx.x == 0) T::store(gB + row, gb);
  }
}

// ---------------------------------------------------------------------------
// inter-chunk forward / backward
// ---------------------------------------------------------------------------
template <typename T, int DPL, int NM>
__global__ __launch_bounds__(kWave) void inter_fwd_kernel(const typename T::raw* __restrict__ tA,
                                                         const typename T::raw* __restrict__ flh,
                                                         typename T::raw* __restrict__ cs, int NC,
                                                         int H, int D, int N) {
  const int b = blockIdx.x / H, h = blockIdx.x % H;
  float st[NM][DPL];
#pragma unroll
  for (int s = 0; s < NM; ++s)
#pragma unroll
    for (int j = 0; j < DPL; ++j) st[s][j] = 0.0f;
  for (int k = 0; k < NC; ++k) {
    const int64_t row = (int64_t(b) * NC + k) * H + h;
#pragma unroll
    for (int p = 0; p < NM / 2; ++p) {
      if (2 * p < N) {
        const int s0 = 2 * p, s1 = 2 * p + 1;
        store_cols<T, DPL>(cs + (row * N + s0) * D, D, st[s0]);
        store_cols<T, DPL>(cs + (row * N + s1) * D, D, st[s1]);
        const float ar = T::load(tA + row * N + s0), ai = T::load(tA + row * N + s1);
        float f0[DPL], f1[DPL];
        load_cols<T, DPL>(flh + (row * N + s0) * D, D, f0);
        load_cols<T, DPL>(flh + (row * N + s1) * D, D, f1);
#pragma unroll
        for (int j = 0; j < DPL; ++j) {
          const float r = st[s0][j], i = st[s1][j];
          st[s0][j] = ar * r - ai * i + f0[j];
          st[s1][j] = ar * i + ai * r + f1[j];
        }
      }
    }
  }
}

template <typename T, int DPL, int NM>
__global__ __launch_bounds__(kWave) void inter_bwd_kernel(const typename T::raw* __restrict__ g_cs,
                                                         const typename T::raw* __restrict__ tA,
                                                         const typename T::raw* __restrict__ cs,
                                                         typename T::raw* __restrict__ g_tA,
                                                         typename T::raw* __restrict__ g_flh, int NC,
                                                         int H, int D, int N) {
  const int b = blockIdx.x / H, h = blockIdx.x % H;
  float ds[NM][DPL];
#pragma unroll
  for (int s = 0; s < NM; ++s)
#pragma unroll
    for (int j = 0; j < DPL; ++j) ds[s][j] = 0.0f;
  for (int k = NC - 1; k >= 0; --k) {
    const int64_t row = (int64_t(b) * NC + k) * H + h;
#pragma unroll
    for (int p = 0; p < NM / 2; ++p) {
      if (2 * p < N) {
        const int s0 = 2 * p, s1 = 2 * p + 1;
        store_cols<T, DPL>(g_flh + (row * N + s0) * D, D, ds[s0]);
        store_cols<T, DPL>(g_flh + (row * N + s1) * D, D, ds[s1]);
        float sr[DPL], si[DPL], gr[DPL], gi[DPL];
        load_cols<T, DPL>(cs + (row * N + s0) * D, D, sr);
        load_cols<T, DPL>(cs + (row * N + s1) * D, D, si);
        load_cols<T, DPL>(g_cs + (row * N + s0) * D, D, gr);
        load_cols<T, DPL>(g_cs + (row * N + s1) * D, D, gi);
        float gre = 0.0f, gim = 0.0f;
#pragma unroll
        for (int j = 0; j < DPL; ++j) {
          gre = fmaf(ds[s0][j], sr[j], fmaf(ds[s1][j], si[j], gre));
          gim = fmaf(ds[s1][j], sr[j], fmaf(-ds[s0][j], si[j], gim));
        }
        gre = wsum(gre);
        gim = wsum(gim);
        if (threadIdx.x == 0) {
          T::store(g_tA + row * N + s0, gre);
          T::store(g_tA + row * N + s1, gim);
        }
        const float ar = T::load(tA + row * N + s0), ai = T::load(tA + row * N + s1);
#pragma unroll
        for (int j = 0; j < DPL; ++j) {
          const float r = ds[s0][j], i = ds[s1][j];
          ds[s0][j] = ar * r + ai * i + gr[j];
          ds[s1][j] = ar * i - ai * r + gi[j];
        }
      }
    }
  }
}

// ---------------------------------------------------------------------------
// exact correction forward / backward
// ---------------------------------------------------------------------------
template <typename T, int DPL, int NM>
__global__ __launch_bounds__(kWave) void corr_fwd_kernel(const typename T::raw* __restrict__ A,
                                                        const typename T::raw* __restrict__ K,
                                                        const typename T::raw* __restrict__ beta,
                                                        const typename T::raw* __restrict__ states,
                                                        typename T::raw* __restrict__ corr, int C, int H,
                                                        int D, int N) {
  const int unit = blockIdx.x / H, h = blockIdx.x % H;  // unit = b*NC + nc
  float c[NM][DPL];
  const int64_t srow = int64_t(unit) * H + h;
#pragma unroll
  for (int s = 0; s < NM; ++s) {
    if (s < N) {
      load_cols<T, DPL>(states + (srow * N + s) * D, D, c[s]);
    } else {
#pragma unroll
      for (int j = 0; j < DPL; ++j) c[s][j] = 0.0f;
    }
  }
  for (int t = 0; t < C; ++t) {
    const int64_t row = (int64_t(unit) * C + t) * H + h;
    float kk[DPL];
    load_cols<T, DPL>(K + row * D, D, kk);
    const float bb = T::load(beta + row);
    float kth[NM];
#pragma unroll
    for (int s = 0; s < NM; ++s) {
      if (s < N) {
        store_cols<T, DPL>(corr + (row * N + s) * D, D, c[s]);
        kth[s] = wsum(dot(c[s], kk));
      } else {
        kth[s] = 0.0f;
      }
    }
#pragma unroll
    for (int p = 0; p < NM / 2; ++p) {
      if (2 * p < N) {
        const int s0 = 2 * p, s1 = 2 * p + 1;
        const float ar = T::load(A + row * N + s0), ai = T::load(A + row * N + s1);
#pragma unroll
        for (int j = 0; j < DPL; ++j) {
          const float er = c[s0][j] - bb * kth[s0] * kk[j];
          const float ei = c[s1][j] - bb * kth[s1] * kk[j];
          c[s0][j] = ar * er - ai * ei;
          c[s1][j] = ar * ei + ai * er;
        }
      }
    }
  }
}

template <typename T, int DPL, int NM>
__global__ __launch_bounds__(kWave) void corr_bwd_kernel(
    const typename T::raw* __restrict__ g_corr, const typename T::raw* __restrict__ A,
    const typename T::raw* __restrict__ K, const typename T::raw* __restrict__ beta,
    const typename T::raw* __restrict__ corr, typename T::raw* __restrict__ gA,
    typename T::raw* __restrict__ gK, typename T::raw* __restrict__ gB,
    typename T::raw* __restrict__ g_states, int C, int H, int D, int N) {
  const int unit = blockIdx.x / H, h = blockIdx.x % H;
  float dh[NM][DPL];
#pragma unroll
  for (int s = 0; s < NM; ++s)
#pragma unroll
    for (int j = 0; j < DPL; ++j) dh[s][j] = 0.0f;
  for (int t = C - 1; t >= 0; --t) {
    const int64_t row = (int64_t(unit) * C + t) * H + h;
    float kk[DPL];
    load_cols<T, DPL>(K + row * D, D, kk);
    const float bb = T::load(beta + row);
    float hb[NM][DPL], kth[NM], dks[NM];
#pragma unroll
    for (int s = 0; s < NM; ++s) {
      if (s < N) {
        float g[DPL];
        load_cols<T, DPL>(g_corr + (row * N + s) * D, D, g);
#pragma unroll
        for (int j = 0; j < DPL; ++j) dh[s][j] += g[j];
        load_cols<T, DPL>(corr + (row * N + s) * D, D, hb[s]);
        kth[s] = wsum(dot(hb[s], kk));
        dks[s] = wsum(dot(dh[s], kk));
      } else {
        kth[s] = dks[s] = 0.0f;
#pragma unroll
        for (int j = 0; j < DPL; ++j) hb[s][j] = 0.0f;
      }
    }
    float gk[DPL];
#pragma unroll
    for (int j = 0; j < DPL; ++j) gk[j] = 0.0f;
    float gb = 0.0f;
#pragma unroll
    for (int p = 0; p < NM / 2; ++p) {
      if (2 * p < N) {
        const int s0 = 2 * p, s1 = 2 * p + 1;
        const float ar = T::load(A + row * N + s0), ai = T::load(A + row * N + s1);
        float gre = 0.0f, gim = 0.0f;
#pragma unroll
        for (int j = 0; j < DPL; ++j) {
          const float hmr = hb[s0][j] - bb * kth[s0] * kk[j];
          const float hmi = hb[s1][j] - bb * kth[s1] * kk[j];
          gre = fmaf(dh[s0][j], hmr, fmaf(dh[s1][j], hmi, gre));
          gim = fmaf(dh[s1][j], hmr, fmaf(-dh[s0][j], hmi, gim));
        }
        gre = wsum(gre);
        gim = wsum(gim);
        if (threadIdx.x == 0) {
          T::store(gA + row * N + s0, gre);
          T::store(gA + row * N + s1, gim);
        }
        const float zr = ar * dks[s0] + ai * dks[s1];
        const float zi = ar * dks[s1] - ai * dks[s0];
        gb -= kth[s0] * zr + kth[s1] * zi;
#pragma unroll
        for (int j = 0; j < DPL; ++j) {
          const float mr = ar * dh[s0][j] + ai * dh[s1][j];
          const float mi = ar * dh[s1][j] - ai * dh[s0][j];
          gk[j] -= bb * (kth[s0] * mr + kth[s1] * mi + hb[s0][j] * zr + hb[s1][j] * zi);
          dh[s0][j] = mr - bb * zr * kk[j];
          dh[s1][j] = mi - bb * zi * kk[j];
        }
      }
    }
    store_cols<T, DPL>(gK + row * D, D, gk);
    if (threadIdx.x == 0) T::store(gB + row, gb);
  }
  const int64_t srow = int64_t(unit) * H + h;
#pragma unroll
  for (int s = 0; s < NM; ++s)
    if (s < N) store_cols<T, DPL>(g_states + (srow * N + s) * D, D, dh[s]);
}

}  // namespace passes
}  // namespace cdssm

// ---------------------------------------------------------------------------
// C-ABI
// ---------------------------------------------------------------------------
namespace {
using namespace cdssm;
using namespace cdssm::passes;

int check_common(const char* op, int dtype, int64_t units, int64_t H, int64_t D, int64_t N,
                 int64_t steps) {
  if (dtype != 0 && dtype != 1) {
    cdssm_host::set_error("%s: dtype must be 0 (fp32) or 1 (bf16), got %d", op, dtype);
    return CDSSM_EINVAL;
  }
  if (units <= 0 || H <= 0 || D <= 0 || steps <= 0) {
    cdssm_host::set_error("%s: sizes must be positive", op);
    return CDSSM_EINVAL;
  }
  if (D > 128) {
    cdssm_host::set_error("%s: head_dim must be <= 128, got %lld", op, (long long)D);
    return CDSSM_EINVAL;
  }
  if (N <= 0 || N > 32 || N % 2 != 0) {
    cdssm_host::set_error("%s: state_dim must be even and in [2, 32], got %lld", op, (long long)N);
    return CDSSM_EINVAL;
  }
  if (units * H > 0x7fffffffLL || units * steps * H * N * D > (int64_t(1) << 46)) {
    cdssm_host::set_error("%s: problem too large", op);
    return CDSSM_EINVAL;
  }
  return CDSSM_OK;
}

// Dispatch on (dtype, DPL, NM) and launch KERNEL<T, DPL, NM> with ARGS.
#define CDSSM_PASS_DISPATCH(KERNEL, GRID, ...)                                                     \
  do {                                                                                           \
    const int dpl_ = D <= 64 ? 1 : 2;                                                            \
    const int nm_ = N <= 2 ? 2 : (N <= 8 ? 8 : (N <= 16 ? 16 : 32));                             \
    auto go = [&](auto tag_t, auto tag_d, auto tag_n) {                                           \
      using TT = decltype(tag_t);                                                                \
      constexpr int DD = decltype(tag_d)::value;                                                 \
      constexpr int NN = decltype(tag_n)::value;                                                 \
      hipLaunchKernelGGL((KERNEL<TT, DD, NN>), dim3(unsigned(GRID)), dim3(kWave), 0, stream,     \
                         __VA_ARGS__);                                                           \
    };                                                                                           \
    auto by_n = [&](auto tag_t, auto tag_d) {                                                    \
      switch (nm_) {                                                                             \
        case 2: go(tag_t, tag_d, std::integral_constant<int, 2>{}); break;                      \
        case 8: go(tag_t, tag_d, std::integral_constant<int, 8>{}); break;                      \
        case 16: go(tag_t, tag_d, std::integral_constant<int, 16>{}); break;                    \
        default: go(tag_t, tag_d, std::integral_constant<int, 32>{}); break;                    \
      }                                                                                          \
    };                                                                                           \
    auto by_d = [&](auto tag_t) {                                                                \
      if (dpl_ == 1) by_n(tag_t, std::integral_constant<int, 1>{});                              \
      else by_n(tag_t, std::integral_constant<int, 2>{});                                        \
    };                                                                                           \
    if (dtype == 1) by_d(BF16{}); else by_d(F32{});                                              \
  } while (0)

}  // namespace

extern "C" int cdssm_intra_chunk_scan_fwd(int dtype, const void* A, const void* K, const void* V,
                                          const void* beta, void* local_h, void* cum_A, int64_t BNC,
                                          int64_t C, int64_t H, int64_t D, int64_t N,
                                          hipStream_t stream) {
  const char* op = "cdssm_intra_chunk_scan_fwd";
  int st = check_common(op, dtype, BNC, H, D, N, C);
  if (st) return st;
  if (!A || !K || !V || !beta || !local_h || !cum_A) {
    cdssm_host::set_error("%s: null pointer argument", op);
    return CDSSM_EINVAL;
  }
  const int c = int(C), h = int(H), d = int(D), n = int(N);
  CDSSM_PASS_DISPATCH(intra_fwd_kernel, BNC * H, (const typename TT::raw*)A, (const typename TT::raw*)K,
                      (const typename TT::raw*)V, (const typename TT::raw*)beta,
                      (typename TT::raw*)local_h, (typename TT::raw*)cum_A, c, h, d, n);
  return cdssm_host::check_launch(op);
}

extern "C" int cdssm_intra_chunk_scan_bwd(int dtype, const void* grad_local_h, const void* grad_cum_A,
                                          const void* A, const void* K, const void* V,
                                          const void* beta, const void* local_h, const void* cum_A,
                                          void* grad_A, void* grad_K, void* grad_V, void* grad_beta,
                                          int64_t BNC, int64_t C, int64_t H, int64_t D, int64_t N,
                                          hipStream_t stream) {
  const char* op = "cdssm_intra_chunk_scan_bwd";
  int st = check_common(op, dtype, BNC, H, D, N, C);
  if (st) return st;
  if (!grad_local_h || !grad_cum_A || !A || !K || !V || !beta || !local_h || !cum_A || !grad_A ||
      !grad_K || !grad_V || !grad_beta) {
    cdssm_host::set_error("%s: null pointer argument", op);
    return CDSSM_EINVAL;
  }
  const int c = int(C), h = int(H), d = int(D), n = int(N);
  CDSSM_PASS_DISPATCH(intra_bwd_kernel, BNC * H, (const typename TT::raw*)grad_local_h,
                      (const typename TT::raw*)grad_cum_A, (const typename TT::raw*)A,
                      (const typename TT::raw*)K, (const typename TT::raw*)V,
                      (const typename TT::raw*)beta, (const typename TT::raw*)local_h,
                      (const typename TT::raw*)cum_A, (typename TT::raw*)grad_A,
                      (typename TT::raw*)grad_K, (typename TT::raw*)grad_V,
                      (typename TT::raw*)grad_beta, c, h, d, n);
  return cdssm_host::check_launch(op);
}

extern "C" int cdssm_inter_chunk_scan_fwd(int dtype, const void* total_A, const void* final_local_h,
                                          void* chunk_states, int64_t B, int64_t NC, int64_t H,
                                          int64_t D, int64_t N, hipStream_t stream) {
  const char* op = "cdssm_inter_chunk_scan_fwd";
  int st = check_common(op, dtype, B, H, D, N, NC);
  if (st) return st;
  if (!total_A || !final_local_h || !chunk_states) {
    cdssm_host::set_error("%s: null pointer argument", op);
    return CDSSM_EINVAL;
  }
  const int nc = int(NC), h = int(H), d = int(D), n = int(N);
  CDSSM_PASS_DISPATCH(inter_fwd_kernel, B * H, (const typename TT::raw*)total_A,
                      (const typename TT::raw*)final_local_h, (typename TT::raw*)chunk_states, nc, h,
                      d, n);
  return cdssm_host::check_launch(op);
}

extern "C" int cdssm_inter_chunk_scan_bwd(int dtype, const void* grad_chunk_states,
                                          const void* total_A, const void* chunk_states,
                                          void* grad_total_A, void* grad_final_local_h, int64_t B,
                                          int64_t NC, int64_t H, int64_t D, int64_t N,
                                          hipStream_t stream) {
  const char* op = "cdssm_inter_chunk_scan_bwd";
  int st = check_common(op, dtype, B, H, D, N, NC);
  if (st) return st;
  if (!grad_chunk_states || !total_A || !chunk_states || !grad_total_A || !grad_final_local_h) {
    cdssm_host::set_error("%s: null pointer argument", op);
    return CDSSM_EINVAL;
  }
  const int nc = int(NC), h = int(H), d = int(D), n = int(N);
  CDSSM_PASS_DISPATCH(inter_bwd_kernel, B * H, (const typename TT::raw*)grad_chunk_states,
                      (const typename TT::raw*)total_A, (const typename TT::raw*)chunk_states,
                      (typename TT::raw*)grad_total_A, (typename TT::raw*)grad_final_local_h, nc, h,
                      d, n);
  return cdssm_host::check_launch(op);
}

extern "C" int cdssm_exact_correction_fwd(int dtype, const void* A_chunk, const void* K_chunk,
                                          const void* beta_chunk, const void* chunk_states,
                                          void* corrections, int64_t B, int64_t NC, int64_t C,
                                          int64_t H, int64_t D, int64_t N, hipStream_t stream) {
  const char* op = "cdssm_exact_correction_fwd";
  int st = check_common(op, dtype, B * NC, H, D, N, C);
  if (st) return st;
  if (!A_chunk || !K_chunk || !beta_chunk || !chunk_states || !corrections) {
    cdssm_host::set_error("%s: null pointer argument", op);
    return CDSSM_EINVAL;
  }
  const int c = int(C), h = int(H), d = int(D), n = int(N);
  CDSSM_PASS_DISPATCH(corr_fwd_kernel, B * NC * H, (const typename TT::raw*)A_chunk,
                      (const typename TT::raw*)K_chunk, (const typename TT::raw*)beta_chunk,
                      (const typename TT::raw*)chunk_states, (typename TT::raw*)corrections, c, h, d,
                      n);
  return cdssm_host::check_launch(op);
}

extern "C" int cdssm_exact_correction_bwd(int dtype, const void* grad_corrections, const void* A_chunk,
                                          const void* K_chunk, const void* beta_chunk,
                                          const void* chunk_states, const void* corrections,
                                          void* grad_A, void* grad_K, void* grad_beta,
                                          void* grad_states, int64_t B, int64_t NC, int64_t C,
                                          int64_t H, int64_t D, int64_t N, hipStream_t stream) {
  const char* op = "cdssm_exact_correction_bwd";
  int st = check_common(op, dtype, B * NC, H, D, N, C);
  if (st) return st;
  if (!grad_corrections || !A_chunk || !K_chunk || !beta_chunk || !corrections || !grad_A ||
      !grad_K || !grad_beta || !grad_states) {
    cdssm_host::set_error("%s: null pointer argument", op);
    return CDSSM_EINVAL;
  }
  (void)chunk_states;  // the saved corrections already hold every pre-step state
  const int c = int(C), h = int(H), d = int(D), n = int(N);
  CDSSM_PASS_DISPATCH(corr_bwd_kernel, B * NC * H, (const typename TT::raw*)grad_corrections,
                      (const typename TT::raw*)A_chunk, (const typename TT::raw*)K_chunk,
                      (const typename TT::raw*)beta_chunk, (const typename TT::raw*)corrections,
                      (typename TT::raw*)grad_A, (typename TT::raw*)grad_K, (typename TT::raw*)grad_beta,
                      (typename TT::raw*)grad_states, c, h, d, n);
  return cdssm_host::check_launch(op);
}
