// Fused elementwise and normalisation kernels of the CD-SSM block around the
// scan (the scan's callers in block.py:140-229 and model.py:38-51), each one
// pass over HBM with 16-byte vector loads:
//   * RMSNorm               (x * rsqrt(mean(x^2) + eps)).to(dtype) * weight   modules.py:49-53
//   * K/Q normalisation     x * rsqrt(sum x^2 + 1e-6) of K (a strided view of
//                           the block's in_proj output) and Q, plus q.k per
//                           (token, head) for the current-token shortcut      normalize_kq.cu:75-79,
//                                                                             block.py:191-192, 202
//   * shortcut readout      retrieved += sel_C s (q.k)^2 V vp                 block.py:202-211
//   * GroupNorm statistics  mean and rstd per (batch row, group) over the
//                           group's channels and all L positions              block.py:215-223
//   * GroupNorm + gate      ((y - mean) rstd gamma + beta).to(dtype) * silu(z)
//                           + D x_conv                                        block.py:216-225
// Roundings to the model dtype happen where the reference's torch ops round
// (each op's output), so a bf16 model keeps the reference's rounding points.
#include "lm_common.hpp"

namespace cdssm {
namespace lm {

// Column sum of a (R, W) fp32 matrix for a 256-thread block of 16 columns x
// 16 thread rows (tx = threadIdx % 16 the column, ty the row group): every
// thread adds rows ty, ty + 16, ...; the 16 row groups are joined in a fixed
// order.  Returns the total to the ty == 0 threads.
__device__ __forceinline__ float col_sum16(const float* __restrict__ part, int R, int W, int col) {
  __shared__ float red[16][16];
  const int tx = int(threadIdx.x) % 16, ty = int(threadIdx.x) / 16;
  float a = 0.0f;
  if (col < W)
    for (int r = ty; r < R; r += 16) a += part[int64_t(r) * W + col];
  red[ty][tx] = a;
  __syncthreads();
  float t = 0.0f;
  if (ty == 0)
    for (int u = 0; u < 16; ++u) t += red[u][tx];
  return t;
}

// NV elements in registers: one 16-byte access (NV = 16 / element bytes, 8
// bf16 or 4 fp32) or a single element (NV = 1).
template <typename T, int NV = 16 / T::bytes>
struct Vec16 {
  static constexpr int N = NV;
  static_assert(NV == 1 || NV * T::bytes == 16, "one element or 16 bytes");
  float v[N];
  __device__ __forceinline__ void load(const typename T::raw* p) {
    if constexpr (NV == 1) {
      v[0] = T::load(p);
      return;
    }
    const uint4 u = *reinterpret_cast<const uint4*>(p);
    const uint32_t w[4] = {u.x, u.y, u.z, u.w};
    if constexpr (T::bytes == 2) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        v[2 * i] = bf16_lo(w[i]);
        v[2 * i + 1] = bf16_hi(w[i]);
      }
    } else {
#pragma unroll
      for (int i = 0; i < 4; ++i) v[i] = __uint_as_float(w[i]);
    }
  }
  __device__ __forceinline__ void store(typename T::raw* p) const {
    if constexpr (NV == 1) {
      T::store(p, v[0]);
      return;
    }
    uint32_t w[4];
    if constexpr (T::bytes == 2) {
#pragma unroll
      for (int i = 0; i < 4; ++i) w[i] = pack_bf16x2(v[2 * i], v[2 * i + 1]);
    } else {
#pragma unroll
      for (int i = 0; i < 4; ++i) w[i] = __float_as_uint(v[i]);
    }
    *reinterpret_cast<uint4*>(p) = make_uint4(w[0], w[1], w[2], w[3]);
  }
};

// ---------------------------------------------------------------------------
// RMSNorm: one wave per row of C elements, N elements per access.
// ---------------------------------------------------------------------------
template <typename T, int N>
__global__ __launch_bounds__(256) void rms_norm_kernel(const typename T::raw* __restrict__ x,
                                                       const typename T::raw* __restrict__ w,
                                                       typename T::raw* __restrict__ y, int64_t rows, int C,
                                                       float eps) {
  const int64_t row = int64_t(blockIdx.x) * 4 + threadIdx.x / kWave;
  const int lane = threadIdx.x % kWave;
  if (row >= rows) return;  // whole waves: the reduction below stays inside one wave
  const typename T::raw* xr = x + row * C;
  float s = 0.0f;
  for (int c = lane * N; c < C; c += kWave * N) {
    Vec16<T, N> a;
    a.load(xr + c);
#pragma unroll
    for (int i = 0; i < N; ++i) s = fmaf(a.v[i], a.v[i], s);
  }
  s = group_sum<kWave>(s);
  const float r = rsqrtf(s / float(C) + eps);
  for (int c = lane * N; c < C; c += kWave * N) {
    Vec16<T, N> a, g;
    a.load(xr + c);
    g.load(w + c);
#pragma unroll
    for (int i = 0; i < N; ++i) a.v[i] = rnd<T>(a.v[i] * r) * g.v[i];
    a.store(y + row * C + c);
  }
}

// Backward of rms_norm_kernel (training; modules.py:49-53 under autograd), with
// the forward's rounding points: xn = rnd(x r), r = rsqrt(mean(x^2) + eps),
// out = rnd(xn w).  Given dout: dxn = rnd(dout w); dw = sum over rows of
// rnd(dout xn); dx = rnd(dxn r - x r^3 (sum_j dxn_j x_j) / C).  A block of 4
// waves takes kRmsRows rows (a wave every 4th), each lane KV 16-byte vectors
// of channels (C = KV * 64 * vector width); the block's dw partial row is
// written for rms_col_sum_kernel.
constexpr int kRmsRows = 32;

template <typename T, int KV>
__global__ __launch_bounds__(256) void rms_norm_bwd_kernel(const typename T::raw* __restrict__ x,
                                                           const typename T::raw* __restrict__ w,
                                                           const typename T::raw* __restrict__ dout,
                                                           typename T::raw* __restrict__ dx,
                                                           float* __restrict__ wpart, int64_t rows, float eps) {
  constexpr int N = Vec16<T>::N, C = KV * kWave * N;
  __shared__ float red[4][kWave][KV * N];
  const int lane = int(threadIdx.x) % kWave, wv = int(threadIdx.x) / kWave;
  Vec16<T> wk[KV];
#pragma unroll
  for (int k = 0; k < KV; ++k) wk[k].load(w + (k * kWave + lane) * N);
  float acc[KV][N];
#pragma unroll
  for (int k = 0; k < KV; ++k)
#pragma unroll
    for (int i = 0; i < N; ++i) acc[k][i] = 0.0f;
  const int64_t r0 = int64_t(blockIdx.x) * kRmsRows;
  for (int rr = wv; rr < kRmsRows; rr += 4) {
    const int64_t row = r0 + rr;
    if (row >= rows) break;  // uniform over the wave
    Vec16<T> xv[KV], gv[KV];
    float s2 = 0.0f;
#pragma unroll
    for (int k = 0; k < KV; ++k) {
      xv[k].load(x + row * C + (k * kWave + lane) * N);
      gv[k].load(dout + row * C + (k * kWave + lane) * N);
#pragma unroll
      for (int i = 0; i < N; ++i) s2 = fmaf(xv[k].v[i], xv[k].v[i], s2);
    }
    s2 = group_sum<kWave>(s2);
    const float r = rsqrtf(s2 / float(C) + eps);
    float sd = 0.0f;
#pragma unroll
    for (int k = 0; k < KV; ++k)
#pragma unroll
      for (int i = 0; i < N; ++i) {
        const float xn = rnd<T>(xv[k].v[i] * r);
        acc[k][i] += rnd<T>(gv[k].v[i] * xn);
        const float dxn = rnd<T>(gv[k].v[i] * wk[k].v[i]);
        gv[k].v[i] = dxn;
        sd = fmaf(dxn, xv[k].v[i], sd);
      }
    sd = group_sum<kWave>(sd);
    const float c3 = r * r * r * sd / float(C);
#pragma unroll
    for (int k = 0; k < KV; ++k) {
#pragma unroll
      for (int i = 0; i < N; ++i) gv[k].v[i] = gv[k].v[i] * r - xv[k].v[i] * c3;
      gv[k].store(dx + row * C + (k * kWave + lane) * N);
    }
  }
#pragma unroll
  for (int k = 0; k < KV; ++k)
#pragma unroll
    for (int i = 0; i < N; ++i) red[wv][lane][k * N + i] = acc[k][i];
  __syncthreads();
  for (int e = int(threadIdx.x); e < C; e += 256) {
    const int ln = (e / N) % kWave, k = e / (N * kWave), i = e % N;
    const float v = ((red[0][ln][k * N + i] + red[1][ln][k * N + i]) + red[2][ln][k * N + i]) + red[3][ln][k * N + i];
    wpart[int64_t(blockIdx.x) * C + e] = v;
  }
}

// out[c] = sum over the partial rows of part (R, C), in a fixed order (16
// columns per block).
template <typename T>
__global__ __launch_bounds__(256) void rms_col_sum_kernel(const float* __restrict__ part, int R, int C,
                                                          typename T::raw* __restrict__ out) {
  const int c = int(blockIdx.x) * 16 + int(threadIdx.x) % 16;
  const float v = col_sum16(part, R, C, c);
  if (int(threadIdx.x) < 16 && c < C) T::store(out + c, v);
}

// ---------------------------------------------------------------------------
// Column sums of a (rows, C) matrix read through a row stride (a linear layer's
// bias gradient: the sum of dL/dy over tokens).  Stage one: a workgroup of 4
// waves takes kColSlab rows of a 64-vector column tile (one 16-byte vector per
// lane), the waves interleaving rows; the 4 waves' sums are joined in order
// into part[slab][c].  Stage two: rms_col_sum_kernel adds the slabs in order.
// ---------------------------------------------------------------------------
constexpr int kColSlab = 64;

template <typename T>
__global__ __launch_bounds__(256) void col_part_kernel(const typename T::raw* __restrict__ x, int64_t ld,
                                                       int64_t rows, int C, float* __restrict__ part) {
  constexpr int N = Vec16<T>::N;
  __shared__ float red[4][kWave * N];
  const int lane = int(threadIdx.x) % kWave, wv = int(threadIdx.x) / kWave;
  const int c0 = (int(blockIdx.x) * kWave + lane) * N;
  const int64_t r0 = int64_t(blockIdx.y) * kColSlab;
  float acc[N];
#pragma unroll
  for (int i = 0; i < N; ++i) acc[i] = 0.0f;
  if (c0 < C) {
    for (int rr = wv; rr < kColSlab && r0 + rr < rows; rr += 4) {
      Vec16<T> v;
      v.load(x + (r0 + rr) * ld + c0);
#pragma unroll
      for (int i = 0; i < N; ++i) acc[i] += v.v[i];
    }
  }
#pragma unroll
  for (int i = 0; i < N; ++i) red[wv][lane * N + i] = acc[i];
  __syncthreads();
  // threads 0..255 write the tile's kWave * N columns (N * 64 <= 512 = 2 per thread for bf16)
  for (int j = int(threadIdx.x); j < kWave * N; j += 256) {
    const int c = int(blockIdx.x) * kWave * N + j;
    if (c < C) part[int64_t(blockIdx.y) * C + c] = ((red[0][j] + red[1][j]) + red[2][j]) + red[3][j];
  }
}

// ---------------------------------------------------------------------------
// Sum of S fp32 slabs of n elements, out[i] = sum_s part[s n + i] in slab
// order, rounded once (the token-slab partials of a weight gradient).  Four
// consecutive elements per thread where n % 4 == 0, else one.
// ---------------------------------------------------------------------------
template <typename T, int V>
__global__ __launch_bounds__(256) void slab_sum_kernel(const float* __restrict__ part, int S, int64_t n,
                                                       typename T::raw* __restrict__ out) {
  const int64_t i = (int64_t(blockIdx.x) * 256 + threadIdx.x) * V;
  if (i >= n) return;
  float a[V] = {};
  for (int s = 0; s < S; ++s) {
    if constexpr (V == 4) {
      const float4 v = *reinterpret_cast<const float4*>(part + int64_t(s) * n + i);
      a[0] += v.x;
      a[1] += v.y;
      a[2] += v.z;
      a[3] += v.w;
    } else {
      a[0] += part[int64_t(s) * n + i];
    }
  }
  if constexpr (V == 4) {
    store_row<T, 4>(out + i, a);
  } else {
    T::store(out + i, a[0]);
  }
}

// ---------------------------------------------------------------------------
// K/Q normalisation and q.k: LPR lanes per (token, head) row of D elements,
// one 16-byte vector each (D = LPR * vector width).  K and Q rows are read
// through a token stride (elements), so K may be a column slice of a wider
// projection output; K^, Q^ (B, L, H, D) and qk (B, L, H) fp32 are dense.
// ---------------------------------------------------------------------------
template <typename T, int LPR>
__global__ __launch_bounds__(256) void normalize_qk_kernel(const typename T::raw* __restrict__ k, int64_t k_ts,
                                                           const typename T::raw* __restrict__ q, int64_t q_ts,
                                                           typename T::raw* __restrict__ ko,
                                                           typename T::raw* __restrict__ qo, float* __restrict__ qk,
                                                           int64_t rows, int H) {
  constexpr int N = Vec16<T>::N, D = LPR * N;
  const int r = int((int64_t(blockIdx.x) * blockDim.x + threadIdx.x) / LPR);  // rows < 2^31 (host check)
  const int sub = threadIdx.x % LPR;
  const bool ok = r < rows;
  const int rr = ok ? r : int(rows) - 1;  // clamped row: every lane takes part in the reductions
  const int tok = rr / H;
  const int h = rr - tok * H;
  Vec16<T> a, b;
  a.load(k + int64_t(tok) * k_ts + h * D + sub * N);
  b.load(q + int64_t(tok) * q_ts + h * D + sub * N);
  float sk = 0.0f, sq = 0.0f;
#pragma unroll
  for (int i = 0; i < N; ++i) {
    sk = fmaf(a.v[i], a.v[i], sk);
    sq = fmaf(b.v[i], b.v[i], sq);
  }
  sk = group_sum<LPR>(sk);
  sq = group_sum<LPR>(sq);
  const float ik = rsqrtf(sk + 1e-6f), iq = rsqrtf(sq + 1e-6f);
  float d = 0.0f;
#pragma unroll
  for (int i = 0; i < N; ++i) {
    a.v[i] = rnd<T>(a.v[i] * ik);
    b.v[i] = rnd<T>(b.v[i] * iq);
    d = fmaf(a.v[i], b.v[i], d);
  }
  d = group_sum<LPR>(d);
  if (!ok) return;
  a.store(ko + int64_t(r) * D + sub * N);
  b.store(qo + int64_t(r) * D + sub * N);
  if (sub == 0) qk[r] = d;
}

// Backward of normalize_qk_kernel (training): given the gradients of K^, Q^
// (dense) and of qk (fp32), per row gk = dK^ + dqk Q^, gq = dQ^ + dqk K^ in
// fp32 and the normalisation's backward dK = (gk - K^ <gk, K^>) rsqrt(sum k^2
// + 1e-6) (normalize_kq.cu's rule, as NormalizeKQFn), likewise dQ; K^, Q^ are
// rebuilt from K, Q as the forward rounds them.  dK, dQ dense.
template <typename T, int LPR>
__global__ __launch_bounds__(256) void normalize_qk_bwd_kernel(const typename T::raw* __restrict__ k, int64_t k_ts,
                                                               const typename T::raw* __restrict__ q, int64_t q_ts,
                                                               const typename T::raw* __restrict__ dko,
                                                               const typename T::raw* __restrict__ dqo,
                                                               const float* __restrict__ dqk,
                                                               typename T::raw* __restrict__ dk,
                                                               typename T::raw* __restrict__ dq, int64_t rows,
                                                               int H) {
  constexpr int N = Vec16<T>::N, D = LPR * N;
  const int r = int((int64_t(blockIdx.x) * blockDim.x + threadIdx.x) / LPR);  // rows < 2^31 (host check)
  const int sub = threadIdx.x % LPR;
  const bool ok = r < rows;
  const int rr = ok ? r : int(rows) - 1;  // clamped row: every lane takes part in the reductions
  const int tok = rr / H;
  const int h = rr - tok * H;
  Vec16<T> a, b, ga, gb;
  a.load(k + int64_t(tok) * k_ts + h * D + sub * N);
  b.load(q + int64_t(tok) * q_ts + h * D + sub * N);
  ga.load(dko + int64_t(rr) * D + sub * N);
  gb.load(dqo + int64_t(rr) * D + sub * N);
  const float g = dqk[rr];
  float sk = 0.0f, sq = 0.0f;
#pragma unroll
  for (int i = 0; i < N; ++i) {
    sk = fmaf(a.v[i], a.v[i], sk);
    sq = fmaf(b.v[i], b.v[i], sq);
  }
  sk = group_sum<LPR>(sk);
  sq = group_sum<LPR>(sq);
  const float ik = rsqrtf(sk + 1e-6f), iq = rsqrtf(sq + 1e-6f);
  float kh[N], qh[N], pk = 0.0f, pq = 0.0f;
#pragma unroll
  for (int i = 0; i < N; ++i) {
    kh[i] = rnd<T>(a.v[i] * ik);
    qh[i] = rnd<T>(b.v[i] * iq);
    ga.v[i] = fmaf(g, qh[i], ga.v[i]);
    gb.v[i] = fmaf(g, kh[i], gb.v[i]);
    // the projections onto the unrounded directions x * inv, as the normalisation's backward takes them
    pk = fmaf(ga.v[i], a.v[i] * ik, pk);
    pq = fmaf(gb.v[i], b.v[i] * iq, pq);
  }
  pk = group_sum<LPR>(pk);
  pq = group_sum<LPR>(pq);
  if (!ok) return;
#pragma unroll
  for (int i = 0; i < N; ++i) {
    ga.v[i] = (ga.v[i] - a.v[i] * ik * pk) * ik;
    gb.v[i] = (gb.v[i] - b.v[i] * iq * pq) * iq;
  }
  ga.store(dk + int64_t(r) * D + sub * N);
  gb.store(dq + int64_t(r) * D + sub * N);
}

// ---------------------------------------------------------------------------
// Current-token shortcut through the readout, per (token, head):
//   retrieved[j] += scale * (q.k)^2 * sel_C * vp * V[j],  j = re, im.
// ---------------------------------------------------------------------------
template <typename T>
__global__ __launch_bounds__(256) void shortcut_kernel(typename T::raw* __restrict__ ret,
                                                       const float* __restrict__ qk,
                                                       const typename T::raw* __restrict__ v,
                                                       const typename T::raw* __restrict__ vp,
                                                       const typename T::raw* __restrict__ sel,
                                                       const float* __restrict__ scale, int64_t n) {
  const int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const float x = qk[i];
  const float c = scale[0] * x * x * T::load(sel + i) * T::load(vp + i);
  T::store(ret + 2 * i, T::load(ret + 2 * i) + c * T::load(v + 2 * i));
  T::store(ret + 2 * i + 1, T::load(ret + 2 * i + 1) + c * T::load(v + 2 * i + 1));
}

// ---------------------------------------------------------------------------
// The same shortcut over R = N/2 complex state rows per (token, head), with its
// backward (the training step).  Per row i, c = scale (q.k)^2 sel_C:
//   forward   y[j] += c vp[j/2] V[j]                       (j < N, one rounding)
//   backward  (g = dL/dy; dV, dvp, dsel_C hold the scan's gradients and take
//             the shortcut's added in fp32, one rounding each)
//             dV[j] += c vp[j/2] g[j]
//             dvp[p] += c (g[2p] V[2p] + g[2p+1] V[2p+1])
//             u = sum_j g[j] vp[j/2] V[j];  dsel_C += scale (q.k)^2 u
//             dqk = 2 scale (q.k) sel_C u  (fp32, written)
//             dscale: each workgroup's sum of (q.k)^2 sel_C u over its rows, in a
//             fixed tree order, to part[blockIdx.x] (the caller adds the partials).
// Where R is a power of two (N = 2, 4, 8, 16, 32, 64) a lane takes one complex
// pair (consecutive lanes read consecutive pairs) and a row's R lanes, which
// sit in one wave, add u with a fixed butterfly; otherwise a thread takes a row.
// ---------------------------------------------------------------------------
constexpr int kShortcutThreads = 256;

template <typename T>
__global__ __launch_bounds__(kShortcutThreads) void shortcut_pairs_fwd_kernel(
    typename T::raw* __restrict__ y, const float* __restrict__ qk, const typename T::raw* __restrict__ v,
    const typename T::raw* __restrict__ vp, const typename T::raw* __restrict__ sel,
    const float* __restrict__ scale, int64_t n_pairs, int log2R) {
  const int64_t j = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  if (j >= n_pairs) return;
  const int64_t i = j >> log2R;
  const float x = qk[i];
  const float w = scale[0] * x * x * T::load(sel + i) * T::load(vp + j);
  store_pair<T>(y + 2 * j, T::load(y + 2 * j) + w * T::load(v + 2 * j),
                T::load(y + 2 * j + 1) + w * T::load(v + 2 * j + 1));
}

template <typename T>
__global__ __launch_bounds__(kShortcutThreads) void shortcut_pairs_bwd_kernel(
    const typename T::raw* __restrict__ g, const float* __restrict__ qk, const typename T::raw* __restrict__ v,
    const typename T::raw* __restrict__ vp, const typename T::raw* __restrict__ sel,
    const float* __restrict__ scale, typename T::raw* __restrict__ dv, typename T::raw* __restrict__ dvp,
    typename T::raw* __restrict__ dsel, float* __restrict__ dqk, float* __restrict__ part, int64_t n_pairs,
    int log2R) {
  __shared__ float red[kShortcutThreads];
  const int64_t j = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  const bool live = j < n_pairs;
  const int64_t i = j >> log2R;
  float x = 0.f, s = 0.f, t = 0.f;
  const float sc = scale[0];
  if (live) {
    x = qk[i];
    s = T::load(sel + i);
    const float c = sc * x * x * s;
    const float a = T::load(vp + j);
    const float g0 = T::load(g + 2 * j), g1 = T::load(g + 2 * j + 1);
    const float gv = g0 * T::load(v + 2 * j) + g1 * T::load(v + 2 * j + 1);
    store_pair<T>(dv + 2 * j, T::load(dv + 2 * j) + c * a * g0, T::load(dv + 2 * j + 1) + c * a * g1);
    T::store(dvp + j, T::load(dvp + j) + c * gv);
    t = a * gv;
  }
  // u over the row's R consecutive lanes (a row never straddles a wave: 64 % R == 0)
  for (int m = 1; m < (1 << log2R); m <<= 1) t += __shfl_xor(t, m, kWave);
  float mine = 0.f;
  if (live && (j & ((int64_t(1) << log2R) - 1)) == 0) {
    T::store(dsel + i, T::load(dsel + i) + sc * x * x * t);
    dqk[i] = 2.f * sc * x * s * t;
    mine = x * x * s * t;
  }
  red[threadIdx.x] = mine;
  __syncthreads();
  for (int w = kShortcutThreads / 2; w > 0; w >>= 1) {
    if (int(threadIdx.x) < w) red[threadIdx.x] += red[threadIdx.x + w];
    __syncthreads();
  }
  if (threadIdx.x == 0) part[blockIdx.x] = red[0];
}

template <typename T>
__global__ __launch_bounds__(kShortcutThreads) void shortcut_rows_fwd_kernel(
    typename T::raw* __restrict__ y, const float* __restrict__ qk, const typename T::raw* __restrict__ v,
    const typename T::raw* __restrict__ vp, const typename T::raw* __restrict__ sel,
    const float* __restrict__ scale, int64_t n, int R) {
  const int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const float x = qk[i];
  const float c = scale[0] * x * x * T::load(sel + i);
  const int64_t o = i * 2 * R;
  for (int p = 0; p < R; ++p) {
    const float w = c * T::load(vp + i * R + p);
    T::store(y + o + 2 * p, T::load(y + o + 2 * p) + w * T::load(v + o + 2 * p));
    T::store(y + o + 2 * p + 1, T::load(y + o + 2 * p + 1) + w * T::load(v + o + 2 * p + 1));
  }
}

template <typename T>
__global__ __launch_bounds__(kShortcutThreads) void shortcut_rows_bwd_kernel(
    const typename T::raw* __restrict__ g, const float* __restrict__ qk, const typename T::raw* __restrict__ v,
    const typename T::raw* __restrict__ vp, const typename T::raw* __restrict__ sel,
    const float* __restrict__ scale, typename T::raw* __restrict__ dv, typename T::raw* __restrict__ dvp,
    typename T::raw* __restrict__ dsel, float* __restrict__ dqk, float* __restrict__ part, int64_t n, int R) {
  __shared__ float red[kShortcutThreads];
  const int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  float mine = 0.f;
  if (i < n) {
    const float x = qk[i], sc = scale[0], s = T::load(sel + i);
    const float c = sc * x * x * s;
    const int64_t o = i * 2 * R;
    float u = 0.f;
    for (int p = 0; p < R; ++p) {
      const float a = T::load(vp + i * R + p);
      const float g0 = T::load(g + o + 2 * p), g1 = T::load(g + o + 2 * p + 1);
      const float gv = g0 * T::load(v + o + 2 * p) + g1 * T::load(v + o + 2 * p + 1);
      T::store(dv + o + 2 * p, T::load(dv + o + 2 * p) + c * a * g0);
      T::store(dv + o + 2 * p + 1, T::load(dv + o + 2 * p + 1) + c * a * g1);
      T::store(dvp + i * R + p, T::load(dvp + i * R + p) + c * gv);
      u += a * gv;
    }
    T::store(dsel + i, T::load(dsel + i) + sc * x * x * u);
    dqk[i] = 2.f * sc * x * s * u;
    mine = x * x * s * u;
  }
  red[threadIdx.x] = mine;
  __syncthreads();
  for (int w = kShortcutThreads / 2; w > 0; w >>= 1) {
    if (int(threadIdx.x) < w) red[threadIdx.x] += red[threadIdx.x + w];
    __syncthreads();
  }
  if (threadIdx.x == 0) part[blockIdx.x] = red[0];
}

// ---------------------------------------------------------------------------
// GroupNorm statistics over (L positions x Cg channels) per (b, g), Cg = C/G.
// Sums of (x - K) and (x - K)^2 with a shift K = y[b, 0, g Cg] (the first
// element of the group), which keeps the variance free of cancellation when
// the mean is far from zero.  Partial sums per (b, g, split) in a fixed order,
// then one thread per (b, g) adds the splits in order: deterministic.
// ---------------------------------------------------------------------------
constexpr int kGnThreads = 256;

template <typename T, int N>
__global__ __launch_bounds__(kGnThreads) void gn_partial_kernel(const typename T::raw* __restrict__ y,
                                                                float2* __restrict__ part, int L, int C, int G,
                                                                int S) {
  __shared__ float2 red[kGnThreads / kWave];
  const int sp = blockIdx.x % S;
  const int bg = blockIdx.x / S;
  const int g = bg % G, b = bg / G;
  const int Cg = C / G, vpt = Cg / N;  // vectors per token of the group
  const int ls = (L + S - 1) / S;
  const int t0 = sp * ls, t1 = min(L, t0 + ls);
  const typename T::raw* base = y + int64_t(b) * L * C + int64_t(g) * Cg;
  const float K = T::load(base);
  float s1 = 0.0f, s2 = 0.0f;
  const int nv = max(0, t1 - t0) * vpt;
  for (int i = threadIdx.x; i < nv; i += kGnThreads) {
    const int t = t0 + i / vpt;
    const int c = (i % vpt) * N;
    Vec16<T, N> a;
    a.load(base + int64_t(t) * C + c);
#pragma unroll
    for (int j = 0; j < N; ++j) {
      const float d = a.v[j] - K;
      s1 += d;
      s2 = fmaf(d, d, s2);
    }
  }
  s1 = group_sum<kWave>(s1);
  s2 = group_sum<kWave>(s2);
  const int wv = threadIdx.x / kWave;
  if (threadIdx.x % kWave == 0) red[wv] = make_float2(s1, s2);
  __syncthreads();
  if (threadIdx.x == 0) {
    float2 acc = red[0];
#pragma unroll
    for (int u = 1; u < kGnThreads / kWave; ++u) {
      acc.x += red[u].x;
      acc.y += red[u].y;
    }
    part[blockIdx.x] = acc;
  }
}

template <typename T>
__global__ __launch_bounds__(256) void gn_finalize_kernel(const typename T::raw* __restrict__ y,
                                                          const float2* __restrict__ part,
                                                          float2* __restrict__ stats, int BG, int L, int C, int G,
                                                          int S, float eps) {
  const int bg = int(blockIdx.x) * blockDim.x + threadIdx.x;
  if (bg >= BG) return;
  const int g = bg % G, b = bg / G;
  const int Cg = C / G;
  const float K = T::load(y + int64_t(b) * L * C + int64_t(g) * Cg);
  float s1 = 0.0f, s2 = 0.0f;
  for (int sp = 0; sp < S; ++sp) {
    s1 += part[int64_t(bg) * S + sp].x;
    s2 += part[int64_t(bg) * S + sp].y;
  }
  const float n = float(L) * float(Cg);
  const float m = s1 / n;
  const float var = fmaxf(s2 / n - m * m, 0.0f);
  stats[bg] = make_float2(K + m, rsqrtf(var + eps));
}

// ---------------------------------------------------------------------------
// GroupNorm apply + gate + skip, one 16-byte vector of channels per thread:
//   a = rnd(((y - mean) rstd) gamma + beta);  s = rnd(silu(z));
//   out = rnd(rnd(a s) + rnd(D x_conv))
// z is read through a token stride (a column slice of the projection output).
// ---------------------------------------------------------------------------
template <typename T, typename P, int N>
__global__ __launch_bounds__(256) void gn_gate_kernel(const typename T::raw* __restrict__ y,
                                                      const float2* __restrict__ stats,
                                                      const typename P::raw* __restrict__ gamma,
                                                      const typename P::raw* __restrict__ beta,
                                                      const typename T::raw* __restrict__ z, int64_t z_ts,
                                                      const typename T::raw* __restrict__ xc,
                                                      const typename T::raw* __restrict__ Dp,
                                                      typename T::raw* __restrict__ out, int BL, int L, int C, int G) {
  // block: 4 tokens x 64 channel vectors; grid (tokens / 4, vectors per row / 64)
  const int tok = int(blockIdx.x) * 4 + int(threadIdx.x) / kWave;
  const int c = (int(blockIdx.y) * kWave + int(threadIdx.x) % kWave) * N;
  if (tok >= BL || c >= C) return;
  const int b = tok / L;
  const float2 st = stats[b * G + c / (C / G)];
  Vec16<T, N> a, zz, xv, dv;
  a.load(y + int64_t(tok) * C + c);
  zz.load(z + int64_t(tok) * z_ts + c);
  xv.load(xc + int64_t(tok) * C + c);
  dv.load(Dp + c);
  // the affine parameters in 16-byte pieces of their own type (or one at a time)
  constexpr int M = 16 / P::bytes <= N ? 16 / P::bytes : 1;
  float ga[N], be[N];
#pragma unroll
  for (int h = 0; h < N; h += M) {
    Vec16<P, M> g, bb;
    g.load(gamma + c + h);
    bb.load(beta + c + h);
#pragma unroll
    for (int j = 0; j < M; ++j) {
      ga[h + j] = g.v[j];
      be[h + j] = bb.v[j];
    }
  }
  float gn[N], s[N], p[N], d[N];
#pragma unroll
  for (int j = 0; j < N; ++j) {
    gn[j] = fmaf((a.v[j] - st.x) * st.y, ga[j], be[j]);
    s[j] = silu_fast(zz.v[j]);
    d[j] = dv.v[j] * xv.v[j];
  }
  if constexpr (N == 1) {
    gn[0] = rnd<T>(gn[0]);
    s[0] = rnd<T>(s[0]);
    d[0] = rnd<T>(d[0]);
    p[0] = rnd<T>(gn[0] * s[0]);
    a.v[0] = rnd<T>(p[0] + d[0]);
  } else {
#pragma unroll
    for (int j = 0; j < N; j += 2) {
      rnd2<T>(gn[j], gn[j + 1]);
      rnd2<T>(s[j], s[j + 1]);
      rnd2<T>(d[j], d[j + 1]);
      p[j] = gn[j] * s[j];
      p[j + 1] = gn[j + 1] * s[j + 1];
      rnd2<T>(p[j], p[j + 1]);
      a.v[j] = p[j] + d[j];
      a.v[j + 1] = p[j + 1] + d[j + 1];
    }
  }
  a.store(out + int64_t(tok) * C + c);  // the store rounds the sum
}

// GroupNorm + gate for one decode token per batch row (gn_row_step): one
// workgroup per row.
template <typename T, typename P>
__global__ __launch_bounds__(256) void gn_gate_step_kernel(const typename T::raw* __restrict__ y,
                                                           const typename T::raw* __restrict__ ret,
                                                           const typename T::raw* __restrict__ wr, int kr,
                                                           float4* __restrict__ gsum,
                                                           const typename P::raw* __restrict__ gamma,
                                                           const typename P::raw* __restrict__ beta,
                                                           const typename T::raw* __restrict__ z, int64_t z_bs,
                                                           const typename T::raw* __restrict__ xc,
                                                           const typename T::raw* __restrict__ Dp,
                                                           typename T::raw* __restrict__ out, int C, int G,
                                                           float eps, int64_t* __restrict__ position) {
  // (mean, rstd) per group; with ret, the row's y (C values) and retrieved row (kr values) after them
  extern __shared__ float2 gst[];
  float* ys = reinterpret_cast<float*>(gst + G);
  float* rs = ys + C;
  // the layer's decode position advances with its last per-token kernel
  if (position && blockIdx.x == 0 && threadIdx.x == 0) position[0] += 1;
  const int b = blockIdx.x;
  if (ret) {
    const typename T::raw* rr = ret + int64_t(b) * kr;
    for (int j = threadIdx.x; j < kr; j += blockDim.x) rs[j] = T::load(rr + j);
    __syncthreads();
  }
  gn_row_step<T, P>(b, y, ret ? rs : nullptr, wr, kr, gsum, gamma, beta, z, z_bs, xc, Dp, out, C, G, eps, gst, ys);
}

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// The block's readout of the per-token states (block.py:208, torch.einsum('blhsd,blhd->blhs', Y, Q)) for
// state_dim N > 2, where the scan returns Y (B,L,H,N,D): r[n] = Y[n] . q, fp32 accumulation, rounded
// once to the element type.  One thread per (token-head, state row), 16-byte loads.
template <typename T>
__global__ __launch_bounds__(256) void state_readout_fwd_kernel(const typename T::raw* __restrict__ Y,
                                                                const typename T::raw* __restrict__ q,
                                                                typename T::raw* __restrict__ r, int64_t rows, int N,
                                                                int D) {
  constexpr int V = Vec16<T>::N;
  const int64_t idx = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  if (idx >= rows) return;
  const typename T::raw* y = Y + idx * D;
  const typename T::raw* qq = q + (idx / N) * D;
  float acc = 0.0f;
  for (int c = 0; c < D; c += V) {
    Vec16<T> a, b;
    a.load(y + c);
    b.load(qq + c);
#pragma unroll
    for (int e = 0; e < V; ++e) acc = fmaf(a.v[e], b.v[e], acc);
  }
  T::store(r + idx, acc);
}

// Its backward: dY[n] = dr[n] q (each product rounded once), dq = sum_n dr[n] Y[n] (fp32 accumulation in row
// order).  One thread per (token-head, 16-byte slice of D).
template <typename T>
__global__ __launch_bounds__(256) void state_readout_bwd_kernel(const typename T::raw* __restrict__ Y,
                                                                const typename T::raw* __restrict__ q,
                                                                const typename T::raw* __restrict__ dr,
                                                                typename T::raw* __restrict__ dY,
                                                                typename T::raw* __restrict__ dq, int64_t n, int N,
                                                                int D) {
  constexpr int V = Vec16<T>::N;
  const int S = D / V;
  const int64_t idx = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  if (idx >= n * S) return;
  const int64_t th = idx / S;
  const int off = int(idx - th * S) * V;
  Vec16<T> qv, acc;
  qv.load(q + th * D + off);
#pragma unroll
  for (int e = 0; e < V; ++e) acc.v[e] = 0.0f;
  for (int s = 0; s < N; ++s) {
    const float g = T::load(dr + th * N + s);
    const int64_t row = (th * N + s) * D + off;
    Vec16<T> yv, o;
    yv.load(Y + row);
#pragma unroll
    for (int e = 0; e < V; ++e) {
      o.v[e] = g * qv.v[e];
      acc.v[e] = fmaf(g, yv.v[e], acc.v[e]);
    }
    o.store(dY + row);
  }
  acc.store(dq + th * D + off);
}

// ---------------------------------------------------------------------------
// Backward of the GroupNorm + gate + skip epilogue (block.py:215-225 under
// autograd) with the forward's rounding points: xh = (y - mean) rstd,
// gn = rnd(xh gamma + beta), s = rnd(silu(z)), out = rnd(rnd(gn s) + rnd(D x)).
// Given dout: dgn = rnd(dout s) (from here the GroupNorm backward in fp32),
//   dgamma = sum over (b, l) of dgn xh, dbeta = sum dgn, dD = sum rnd(dout x),
//   dy = rnd(rstd (dgn gamma - A - xh Bm)) with A, Bm the means of dgn gamma
//        and dgn gamma xh over the (b, group) the element normalises with,
//   dz = rnd(rnd(dout gn) sigmoid(z) (1 + z (1 - sigmoid(z)))),
//   dx = rnd(dout D).
// Three launches: per (b, slice of tokens) the partial sums (gnb_reduce), their
// totals in a fixed order (gnb_finalize), the elementwise gradients
// (gnb_apply).  One 16-byte vector of channels per thread; a channel vector
// lies in one group and a block's 64 vectors hold whole groups (the entry
// checks both).
// ---------------------------------------------------------------------------
template <typename P, int N>
__device__ __forceinline__ void load_affine(const typename P::raw* gamma, const typename P::raw* beta, int c,
                                            float (&ga)[N], float (&be)[N]) {
  constexpr int M = 16 / P::bytes <= N ? 16 / P::bytes : 1;
#pragma unroll
  for (int h = 0; h < N; h += M) {
    Vec16<P, M> g, bb;
    g.load(gamma + c + h);
    bb.load(beta + c + h);
#pragma unroll
    for (int j = 0; j < M; ++j) {
      ga[h + j] = g.v[j];
      be[h + j] = bb.v[j];
    }
  }
}

template <typename T, typename P>
__global__ __launch_bounds__(256) void gnb_reduce_kernel(const typename T::raw* __restrict__ y,
                                                         const float2* __restrict__ stats,
                                                         const typename P::raw* __restrict__ gamma,
                                                         const typename P::raw* __restrict__ beta,
                                                         const typename T::raw* __restrict__ z, int64_t z_ts,
                                                         const typename T::raw* __restrict__ xc,
                                                         const typename T::raw* __restrict__ dout,
                                                         float* __restrict__ chan_part, float2* __restrict__ grp_part,
                                                         int L, int C, int G, int S) {
  constexpr int N = 16 / T::bytes;
  __shared__ float red[4][kWave][3 * N];
  __shared__ float2 gred[4][kWave];
  const int tx = int(threadIdx.x) % kWave, ty = int(threadIdx.x) / kWave;
  const int bs = blockIdx.x, b = bs / S, sp = bs % S;
  const int ls = (L + S - 1) / S;
  const int t0 = sp * ls, t1 = min(L, t0 + ls);
  const int Cg = C / G, vpg = Cg / N;  // channel vectors per group
  const int c = (int(blockIdx.y) * kWave + tx) * N;
  const bool act = c < C;
  const int cc = act ? c : 0;
  const int g = cc / Cg;
  const float2 st = stats[b * G + g];
  float ga[N], be[N];
  load_affine<P, N>(gamma, beta, cc, ga, be);
  float ag[N], ab[N], ad[N];
#pragma unroll
  for (int j = 0; j < N; ++j) ag[j] = ab[j] = ad[j] = 0.0f;
  float sa = 0.0f, sb = 0.0f;
  if (act) {
    for (int t = t0 + ty; t < t1; t += 4) {
      const int64_t tok = int64_t(b) * L + t;
      Vec16<T> yv, zv, xv, dv;
      yv.load(y + tok * C + c);
      zv.load(z + tok * z_ts + c);
      xv.load(xc + tok * C + c);
      dv.load(dout + tok * C + c);
#pragma unroll
      for (int j = 0; j < N; ++j) {
        const float xh = (yv.v[j] - st.x) * st.y;
        const float sv = rnd<T>(silu_fast(zv.v[j]));
        const float dg = rnd<T>(dv.v[j] * sv);
        ag[j] = fmaf(dg, xh, ag[j]);
        ab[j] += dg;
        ad[j] += rnd<T>(dv.v[j] * xv.v[j]);
        const float dgg = dg * ga[j];
        sa += dgg;
        sb = fmaf(dgg, xh, sb);
      }
    }
  }
#pragma unroll
  for (int j = 0; j < N; ++j) {
    red[ty][tx][j] = ag[j];
    red[ty][tx][N + j] = ab[j];
    red[ty][tx][2 * N + j] = ad[j];
  }
  gred[ty][tx] = make_float2(sa, sb);
  __syncthreads();
  if (ty == 0 && act) {
#pragma unroll
    for (int k = 0; k < 3; ++k) {
#pragma unroll
      for (int j = 0; j < N; ++j) {
        const float v = ((red[0][tx][k * N + j] + red[1][tx][k * N + j]) + red[2][tx][k * N + j]) +
                        red[3][tx][k * N + j];
        chan_part[(int64_t(bs) * 3 + k) * C + c + j] = v;
      }
    }
    if (tx % vpg == 0) {
      float2 acc = make_float2(0.0f, 0.0f);
      for (int u = 0; u < vpg; ++u)
        for (int r = 0; r < 4; ++r) {
          acc.x += gred[r][tx + u].x;
          acc.y += gred[r][tx + u].y;
        }
      grp_part[(int64_t(b) * G + g) * S + sp] = acc;
    }
  }
}

// Blocks [0, ceil(3 C / 16)): column sums of the (BS, 3 C) partials (dgamma,
// dbeta, dD side by side); the blocks after: one (b, group) per thread.
template <typename T, typename P>
__global__ __launch_bounds__(256) void gnb_finalize_kernel(const float* __restrict__ chan_part,
                                                           const float2* __restrict__ grp_part,
                                                           typename P::raw* __restrict__ dgamma,
                                                           typename P::raw* __restrict__ dbeta,
                                                           typename T::raw* __restrict__ dD,
                                                           float2* __restrict__ gmeans, int BS, int C, int BG,
                                                           int S, float inv_n) {
  const int ncb = (3 * C + 15) / 16;
  if (int(blockIdx.x) < ncb) {
    const int col = int(blockIdx.x) * 16 + int(threadIdx.x) % 16;
    const float v = col_sum16(chan_part, BS, 3 * C, col);
    if (int(threadIdx.x) < 16 && col < 3 * C) {
      const int k = col / C, c = col - k * C;
      if (k == 0)
        P::store(dgamma + c, v);
      else if (k == 1)
        P::store(dbeta + c, v);
      else
        T::store(dD + c, v);
    }
    return;
  }
  const int i = (int(blockIdx.x) - ncb) * 256 + int(threadIdx.x);
  if (i < BG) {
    float2 acc = make_float2(0.0f, 0.0f);
    for (int s = 0; s < S; ++s) {
      acc.x += grp_part[int64_t(i) * S + s].x;
      acc.y += grp_part[int64_t(i) * S + s].y;
    }
    gmeans[i] = make_float2(acc.x * inv_n, acc.y * inv_n);
  }
}

template <typename T, typename P>
__global__ __launch_bounds__(256) void gnb_apply_kernel(const typename T::raw* __restrict__ y,
                                                        const float2* __restrict__ stats,
                                                        const float2* __restrict__ gmeans,
                                                        const typename P::raw* __restrict__ gamma,
                                                        const typename P::raw* __restrict__ beta,
                                                        const typename T::raw* __restrict__ z, int64_t z_ts,
                                                        const typename T::raw* __restrict__ Dp,
                                                        const typename T::raw* __restrict__ dout,
                                                        typename T::raw* __restrict__ dy,
                                                        typename T::raw* __restrict__ dz,
                                                        typename T::raw* __restrict__ dx, int BL, int L, int C,
                                                        int G) {
  constexpr int N = 16 / T::bytes;
  // block: 4 tokens x 64 channel vectors; grid (tokens / 4, vectors per row / 64)
  const int tok = int(blockIdx.x) * 4 + int(threadIdx.x) / kWave;
  const int c = (int(blockIdx.y) * kWave + int(threadIdx.x) % kWave) * N;
  if (tok >= BL || c >= C) return;
  const int bg = (tok / L) * G + c / (C / G);
  const float2 st = stats[bg], gm = gmeans[bg];
  float ga[N], be[N];
  load_affine<P, N>(gamma, beta, c, ga, be);
  Vec16<T> yv, zv, dv, Dv, oy, oz, ox;
  yv.load(y + int64_t(tok) * C + c);
  zv.load(z + int64_t(tok) * z_ts + c);
  dv.load(dout + int64_t(tok) * C + c);
  Dv.load(Dp + c);
#pragma unroll
  for (int j = 0; j < N; ++j) {
    const float xh = (yv.v[j] - st.x) * st.y;
    const float gn = rnd<T>(fmaf(xh, ga[j], be[j]));
    const float zj = zv.v[j];
    const float sg = __builtin_amdgcn_rcpf(1.0f + __expf(-zj));
    const float sv = rnd<T>(zj * sg);
    const float dg = rnd<T>(dv.v[j] * sv);
    oy.v[j] = st.y * (dg * ga[j] - gm.x - xh * gm.y);
    oz.v[j] = rnd<T>(dv.v[j] * gn) * sg * (1.0f + zj * (1.0f - sg));
    ox.v[j] = dv.v[j] * Dv.v[j];
  }
  oy.store(dy + int64_t(tok) * C + c);
  oz.store(dz + int64_t(tok) * C + c);
  ox.store(dx + int64_t(tok) * C + c);
}

template <typename F>
int by_dtype(int dtype, const char* op, F&& f) {
  if (dtype == 1) return f(BF16{});
  if (dtype == 0) return f(F32{});
  cdssm_host::set_error("%s: dtype must be 0 (fp32) or 1 (bf16), got %d", op, dtype);
  return CDSSM_EINVAL;
}

}  // namespace lm
}  // namespace cdssm

using namespace cdssm;
using namespace cdssm::lm;

extern "C" int cdssm_rms_norm_fwd(int dtype, const void* x, const void* weight, void* y, int64_t rows, int64_t C,
                                  float eps, hipStream_t stream) {
  const char* op = "cdssm_rms_norm_fwd";
  return by_dtype(dtype, op, [&](auto t) -> int {
    using T = decltype(t);
    if (rows <= 0 || C <= 0 || C > (1 << 24) || rows > (int64_t(1) << 31)) {
      cdssm_host::set_error("%s: need rows > 0 and 0 < C <= 2^24 (rows=%lld C=%lld)", op, (long long)rows,
                            (long long)C);
      return CDSSM_EINVAL;
    }
    if (!x || !weight || !y) {
      cdssm_host::set_error("%s: null pointer argument", op);
      return CDSSM_EINVAL;
    }
    using raw = typename T::raw;
    constexpr int NV = 16 / T::bytes;
    const bool vec = C % NV == 0 && aligned16(x) && aligned16(weight) && aligned16(y);
    auto go = [&](auto nc) {
      constexpr int N = decltype(nc)::value;
      hipLaunchKernelGGL((rms_norm_kernel<T, N>), dim3(unsigned((rows + 3) / 4)), dim3(256), 0, stream,
                         static_cast<const raw*>(x), static_cast<const raw*>(weight), static_cast<raw*>(y), rows,
                         int(C), eps);
    };
    if (vec)
      go(std::integral_constant<int, NV>{});
    else
      go(std::integral_constant<int, 1>{});
    return cdssm_host::check_launch(op);
  });
}

extern "C" int cdssm_normalize_kq_qk_fwd(int dtype, const void* K, int64_t k_token_stride, const void* Q,
                                         int64_t q_token_stride, void* K_out, void* Q_out, float* qk, int64_t BL,
                                         int64_t H, int64_t D, hipStream_t stream) {
  const char* op = "cdssm_normalize_kq_qk_fwd";
  return by_dtype(dtype, op, [&](auto t) -> int {
    using T = decltype(t);
    using raw = typename T::raw;
    constexpr int N = Vec16<T>::N;
    const int64_t lpr = D / N;
    if (BL <= 0 || H <= 0 || D % N != 0 || !(lpr == 4 || lpr == 8 || lpr == 16 || lpr == 32) ||
        k_token_stride < H * D || q_token_stride < H * D || BL * H >= (int64_t(1) << 31)) {
      cdssm_host::set_error("%s: need D in {%d, %d, %d, %d} and token strides >= H*D (BL=%lld H=%lld D=%lld)", op,
                            4 * N, 8 * N, 16 * N, 32 * N, (long long)BL, (long long)H, (long long)D);
      return CDSSM_EINVAL;
    }
    if (!K || !Q || !K_out || !Q_out || !qk || !aligned16(K) || !aligned16(Q) || !aligned16(K_out) ||
        !aligned16(Q_out) || (k_token_stride * T::bytes) % 16 != 0 || (q_token_stride * T::bytes) % 16 != 0) {
      cdssm_host::set_error("%s: pointers must be non-null and 16-byte aligned, token strides whole 16 bytes", op);
      return CDSSM_EINVAL;
    }
    const int64_t rows = BL * H;
    const unsigned grid = unsigned((rows * lpr + 255) / 256);
    auto go = [&](auto lc) {
      constexpr int LPR = decltype(lc)::value;
      hipLaunchKernelGGL((normalize_qk_kernel<T, LPR>), dim3(grid), dim3(256), 0, stream,
                         static_cast<const raw*>(K), k_token_stride, static_cast<const raw*>(Q), q_token_stride,
                         static_cast<raw*>(K_out), static_cast<raw*>(Q_out), qk, rows, int(H));
    };
    if (lpr == 4) go(std::integral_constant<int, 4>{});
    else if (lpr == 8) go(std::integral_constant<int, 8>{});
    else if (lpr == 16) go(std::integral_constant<int, 16>{});
    else go(std::integral_constant<int, 32>{});
    return cdssm_host::check_launch(op);
  });
}

extern "C" int64_t cdssm_rms_norm_bwd_workspace_bytes(int64_t rows, int64_t C) {
  if (rows <= 0 || C <= 0) return -1;
  return (rows + kRmsRows - 1) / kRmsRows * C * int64_t(sizeof(float));
}

extern "C" int cdssm_rms_norm_bwd(int dtype, const void* x, const void* w, const void* dout, void* dx, void* dw,
                                  float* workspace, int64_t rows, int64_t C, float eps, hipStream_t stream) {
  const char* op = "cdssm_rms_norm_bwd";
  return by_dtype(dtype, op, [&](auto t) -> int {
    using T = decltype(t);
    using raw = typename T::raw;
    constexpr int N = Vec16<T>::N;
    const int64_t kv = C / (int64_t(kWave) * N);
    if (rows <= 0 || rows >= (int64_t(1) << 31) || C % (int64_t(kWave) * N) != 0 || kv < 1 || kv > 4) {
      cdssm_host::set_error("%s: need C a multiple of %d up to %d (rows=%lld C=%lld)", op, kWave * N, 4 * kWave * N,
                            (long long)rows, (long long)C);
      return CDSSM_EINVAL;
    }
    if (!x || !w || !dout || !dx || !dw || !workspace || !aligned16(x) || !aligned16(w) || !aligned16(dout) ||
        !aligned16(dx)) {
      cdssm_host::set_error("%s: pointers must be non-null and 16-byte aligned", op);
      return CDSSM_EINVAL;
    }
    const int nb = int((rows + kRmsRows - 1) / kRmsRows);
    auto go = [&](auto kc) {
      constexpr int KV = decltype(kc)::value;
      hipLaunchKernelGGL((rms_norm_bwd_kernel<T, KV>), dim3(unsigned(nb)), dim3(256), 0, stream,
                         static_cast<const raw*>(x), static_cast<const raw*>(w), static_cast<const raw*>(dout),
                         static_cast<raw*>(dx), workspace, rows, eps);
    };
    if (kv == 1) go(std::integral_constant<int, 1>{});
    else if (kv == 2) go(std::integral_constant<int, 2>{});
    else if (kv == 3) go(std::integral_constant<int, 3>{});
    else go(std::integral_constant<int, 4>{});
    hipLaunchKernelGGL(rms_col_sum_kernel<T>, dim3(unsigned((C + 15) / 16)), dim3(256), 0, stream,
                       static_cast<const float*>(workspace), nb, int(C), static_cast<raw*>(dw));
    return cdssm_host::check_launch(op);
  });
}

extern "C" int cdssm_normalize_kq_qk_bwd(int dtype, const void* K, int64_t k_token_stride, const void* Q,
                                         int64_t q_token_stride, const void* dK_out, const void* dQ_out,
                                         const float* dqk, void* dK, void* dQ, int64_t BL, int64_t H, int64_t D,
                                         hipStream_t stream) {
  const char* op = "cdssm_normalize_kq_qk_bwd";
  return by_dtype(dtype, op, [&](auto t) -> int {
    using T = decltype(t);
    using raw = typename T::raw;
    constexpr int N = Vec16<T>::N;
    const int64_t lpr = D / N;
    if (BL <= 0 || H <= 0 || D % N != 0 || !(lpr == 4 || lpr == 8 || lpr == 16 || lpr == 32) ||
        k_token_stride < H * D || q_token_stride < H * D || BL * H >= (int64_t(1) << 31)) {
      cdssm_host::set_error("%s: need D in {%d, %d, %d, %d} and token strides >= H*D (BL=%lld H=%lld D=%lld)", op,
                            4 * N, 8 * N, 16 * N, 32 * N, (long long)BL, (long long)H, (long long)D);
      return CDSSM_EINVAL;
    }
    if (!K || !Q || !dK_out || !dQ_out || !dqk || !dK || !dQ || !aligned16(K) || !aligned16(Q) ||
        !aligned16(dK_out) || !aligned16(dQ_out) || !aligned16(dK) || !aligned16(dQ) ||
        (k_token_stride * T::bytes) % 16 != 0 || (q_token_stride * T::bytes) % 16 != 0) {
      cdssm_host::set_error("%s: pointers must be non-null and 16-byte aligned, token strides whole 16 bytes", op);
      return CDSSM_EINVAL;
    }
    const int64_t rows = BL * H;
    const unsigned grid = unsigned((rows * lpr + 255) / 256);
    auto go = [&](auto lc) {
      constexpr int LPR = decltype(lc)::value;
      hipLaunchKernelGGL((normalize_qk_bwd_kernel<T, LPR>), dim3(grid), dim3(256), 0, stream,
                         static_cast<const raw*>(K), k_token_stride, static_cast<const raw*>(Q), q_token_stride,
                         static_cast<const raw*>(dK_out), static_cast<const raw*>(dQ_out), dqk, static_cast<raw*>(dK),
                         static_cast<raw*>(dQ), rows, int(H));
    };
    if (lpr == 4) go(std::integral_constant<int, 4>{});
    else if (lpr == 8) go(std::integral_constant<int, 8>{});
    else if (lpr == 16) go(std::integral_constant<int, 16>{});
    else go(std::integral_constant<int, 32>{});
    return cdssm_host::check_launch(op);
  });
}

extern "C" int64_t cdssm_col_sum_workspace_bytes(int64_t rows, int64_t C) {
  if (rows <= 0 || C <= 0) return -1;
  return ((rows + kColSlab - 1) / kColSlab) * C * int64_t(sizeof(float));
}

extern "C" int cdssm_col_sum(int dtype, const void* x, int64_t ld, int64_t rows, int64_t C, void* out,
                             float* workspace, hipStream_t stream) {
  const char* op = "cdssm_col_sum";
  return by_dtype(dtype, op, [&](auto t) -> int {
    using T = decltype(t);
    using raw = typename T::raw;
    constexpr int N = Vec16<T>::N;
    if (rows <= 0 || C <= 0 || C % N != 0 || ld < C || ld % N != 0 || rows >= (int64_t(1) << 31) ||
        C >= (int64_t(1) << 24)) {
      cdssm_host::set_error("%s: need rows > 0, C a positive multiple of %d and a row stride >= C, a multiple of "
                            "%d (rows=%lld C=%lld ld=%lld)", op, N, N, (long long)rows, (long long)C, (long long)ld);
      return CDSSM_EINVAL;
    }
    if (!x || !out || !workspace || (reinterpret_cast<uintptr_t>(x) & 15u) != 0) {
      cdssm_host::set_error("%s: x, out and workspace must be non-null, x 16-byte aligned", op);
      return CDSSM_EINVAL;
    }
    const int slabs = int((rows + kColSlab - 1) / kColSlab);
    if (slabs > 65535) {
      cdssm_host::set_error("%s: at most %d rows", op, 65535 * kColSlab);
      return CDSSM_EINVAL;
    }
    hipLaunchKernelGGL(col_part_kernel<T>, dim3(unsigned((C + kWave * N - 1) / (kWave * N)), unsigned(slabs)),
                       dim3(256), 0, stream, static_cast<const raw*>(x), ld, rows, int(C), workspace);
    int st = cdssm_host::check_launch(op);
    if (st) return st;
    hipLaunchKernelGGL(rms_col_sum_kernel<T>, dim3(unsigned((C + 15) / 16)), dim3(256), 0, stream,
                       static_cast<const float*>(workspace), slabs, int(C), static_cast<raw*>(out));
    return cdssm_host::check_launch(op);
  });
}

extern "C" int cdssm_slab_sum(int dtype, const float* part, int64_t S, int64_t n, void* out, hipStream_t stream) {
  const char* op = "cdssm_slab_sum";
  return by_dtype(dtype, op, [&](auto t) -> int {
    using T = decltype(t);
    using raw = typename T::raw;
    if (S <= 0 || S > 4096 || n <= 0 || n >= (int64_t(1) << 40)) {
      cdssm_host::set_error("%s: need 0 < S <= 4096 and n > 0 (S=%lld n=%lld)", op, (long long)S, (long long)n);
      return CDSSM_EINVAL;
    }
    if (!part || !out) {
      cdssm_host::set_error("%s: null pointer argument", op);
      return CDSSM_EINVAL;
    }
    const bool vec = n % 4 == 0 && (reinterpret_cast<uintptr_t>(part) & 15u) == 0 &&
                     (reinterpret_cast<uintptr_t>(out) & uintptr_t(4 * T::bytes - 1)) == 0;
    if (vec)
      hipLaunchKernelGGL((slab_sum_kernel<T, 4>), dim3(unsigned((n / 4 + 255) / 256)), dim3(256), 0, stream, part,
                         int(S), n, static_cast<raw*>(out));
    else
      hipLaunchKernelGGL((slab_sum_kernel<T, 1>), dim3(unsigned((n + 255) / 256)), dim3(256), 0, stream, part,
                         int(S), n, static_cast<raw*>(out));
    return cdssm_host::check_launch(op);
  });
}

extern "C" int cdssm_shortcut_readout_fwd(int dtype, void* retrieved, const float* qk, const void* V,
                                          const void* vp, const void* sel_c, const float* scale, int64_t n,
                                          hipStream_t stream) {
  const char* op = "cdssm_shortcut_readout_fwd";
  return by_dtype(dtype, op, [&](auto t) -> int {
    using T = decltype(t);
    using raw = typename T::raw;
    if (n <= 0 || n > (int64_t(1) << 38)) {
      cdssm_host::set_error("%s: need n > 0 (n=%lld)", op, (long long)n);
      return CDSSM_EINVAL;
    }
    if (!retrieved || !qk || !V || !vp || !sel_c || !scale) {
      cdssm_host::set_error("%s: null pointer argument", op);
      return CDSSM_EINVAL;
    }
    hipLaunchKernelGGL(shortcut_kernel<T>, dim3(unsigned((n + 255) / 256)), dim3(256), 0, stream,
                       static_cast<raw*>(retrieved), qk, static_cast<const raw*>(V), static_cast<const raw*>(vp),
                       static_cast<const raw*>(sel_c), scale, n);
    return cdssm_host::check_launch(op);
  });
}

namespace {
int shortcut_rows_check(const char* op, int64_t n, int64_t N) {
  if (n <= 0 || N <= 0 || N % 2 != 0 || N > 64 || n * N > (int64_t(1) << 38)) {
    cdssm_host::set_error("%s: need n > 0 and an even N <= 64 (n=%lld N=%lld)", op, (long long)n, (long long)N);
    return CDSSM_EINVAL;
  }
  return CDSSM_OK;
}

// log2(N/2) where N/2 is a power of two (the lane-per-pair kernels), else -1
int shortcut_log2_rows(int64_t N) {
  const int64_t R = N / 2;
  return (R & (R - 1)) == 0 ? __builtin_ctzll(uint64_t(R)) : -1;
}

// workgroups of a launch: one lane per pair, or per row
int64_t shortcut_groups(int64_t n, int64_t N) {
  const int64_t units = shortcut_log2_rows(N) >= 0 ? n * (N / 2) : n;
  return (units + kShortcutThreads - 1) / kShortcutThreads;
}

// the pair stores need each (re, im) pair aligned to its size
bool pair_aligned(const void* p, int bytes) { return (reinterpret_cast<uintptr_t>(p) % (2 * bytes)) == 0; }
}  // namespace

extern "C" int64_t cdssm_shortcut_readout_rows_partials(int64_t n, int64_t N) {
  return n > 0 && N > 0 && N % 2 == 0 ? shortcut_groups(n, N) : -1;
}

extern "C" int cdssm_shortcut_readout_rows_fwd(int dtype, void* y, const float* qk, const void* V, const void* vp,
                                               const void* sel_c, const float* scale, int64_t n, int64_t N,
                                               hipStream_t stream) {
  const char* op = "cdssm_shortcut_readout_rows_fwd";
  return by_dtype(dtype, op, [&](auto t) -> int {
    using T = decltype(t);
    using raw = typename T::raw;
    if (shortcut_rows_check(op, n, N) != CDSSM_OK) return CDSSM_EINVAL;
    if (!y || !qk || !V || !vp || !sel_c || !scale) {
      cdssm_host::set_error("%s: null pointer argument", op);
      return CDSSM_EINVAL;
    }
    if (!pair_aligned(y, T::bytes)) {
      cdssm_host::set_error("%s: y must be aligned to a (re, im) pair (%d bytes)", op, 2 * T::bytes);
      return CDSSM_EINVAL;
    }
    const int lr = shortcut_log2_rows(N);
    if (lr >= 0)
      hipLaunchKernelGGL(shortcut_pairs_fwd_kernel<T>, dim3(unsigned(shortcut_groups(n, N))), dim3(kShortcutThreads),
                         0, stream, static_cast<raw*>(y), qk, static_cast<const raw*>(V), static_cast<const raw*>(vp),
                         static_cast<const raw*>(sel_c), scale, n * (N / 2), lr);
    else
      hipLaunchKernelGGL(shortcut_rows_fwd_kernel<T>, dim3(unsigned(shortcut_groups(n, N))), dim3(kShortcutThreads),
                         0, stream, static_cast<raw*>(y), qk, static_cast<const raw*>(V), static_cast<const raw*>(vp),
                         static_cast<const raw*>(sel_c), scale, n, int(N / 2));
    return cdssm_host::check_launch(op);
  });
}

extern "C" int cdssm_shortcut_readout_rows_bwd(int dtype, const void* dy, const float* qk, const void* V,
                                               const void* vp, const void* sel_c, const float* scale, void* dV,
                                               void* dvp, void* dsel_c, float* dqk, float* dscale_partials,
                                               int64_t n, int64_t N, hipStream_t stream) {
  const char* op = "cdssm_shortcut_readout_rows_bwd";
  return by_dtype(dtype, op, [&](auto t) -> int {
    using T = decltype(t);
    using raw = typename T::raw;
    if (shortcut_rows_check(op, n, N) != CDSSM_OK) return CDSSM_EINVAL;
    if (!dy || !qk || !V || !vp || !sel_c || !scale || !dV || !dvp || !dsel_c || !dqk || !dscale_partials) {
      cdssm_host::set_error("%s: null pointer argument", op);
      return CDSSM_EINVAL;
    }
    if (!pair_aligned(dV, T::bytes)) {
      cdssm_host::set_error("%s: dV must be aligned to a (re, im) pair (%d bytes)", op, 2 * T::bytes);
      return CDSSM_EINVAL;
    }
    const int lr = shortcut_log2_rows(N);
    if (lr >= 0)
      hipLaunchKernelGGL(shortcut_pairs_bwd_kernel<T>, dim3(unsigned(shortcut_groups(n, N))), dim3(kShortcutThreads),
                         0, stream, static_cast<const raw*>(dy), qk, static_cast<const raw*>(V),
                         static_cast<const raw*>(vp), static_cast<const raw*>(sel_c), scale, static_cast<raw*>(dV),
                         static_cast<raw*>(dvp), static_cast<raw*>(dsel_c), dqk, dscale_partials, n * (N / 2), lr);
    else
      hipLaunchKernelGGL(shortcut_rows_bwd_kernel<T>, dim3(unsigned(shortcut_groups(n, N))), dim3(kShortcutThreads),
                         0, stream, static_cast<const raw*>(dy), qk, static_cast<const raw*>(V),
                         static_cast<const raw*>(vp), static_cast<const raw*>(sel_c), scale, static_cast<raw*>(dV),
                         static_cast<raw*>(dvp), static_cast<raw*>(dsel_c), dqk, dscale_partials, n, int(N / 2));
    return cdssm_host::check_launch(op);
  });
}

extern "C" int cdssm_state_readout_fwd(int dtype, const void* Y, const void* q, void* r, int64_t n, int64_t N,
                                       int64_t D, hipStream_t stream) {
  const char* op = "cdssm_state_readout_fwd";
  return by_dtype(dtype, op, [&](auto t) -> int {
    using T = decltype(t);
    using raw = typename T::raw;
    constexpr int V = Vec16<T>::N;
    if (n <= 0 || N <= 0 || D <= 0 || D % V != 0 || n * N > (int64_t(1) << 38)) {
      cdssm_host::set_error("%s: need n, N > 0 and D a positive multiple of %d (n=%lld N=%lld D=%lld)", op, V,
                            (long long)n, (long long)N, (long long)D);
      return CDSSM_EINVAL;
    }
    if (!Y || !q || !r) {
      cdssm_host::set_error("%s: null pointer argument", op);
      return CDSSM_EINVAL;
    }
    if ((reinterpret_cast<uintptr_t>(Y) | reinterpret_cast<uintptr_t>(q)) & 15) {
      cdssm_host::set_error("%s: Y and q must be 16-byte aligned", op);
      return CDSSM_EINVAL;
    }
    const int64_t rows = n * N;
    hipLaunchKernelGGL(state_readout_fwd_kernel<T>, dim3(unsigned((rows + 255) / 256)), dim3(256), 0, stream,
                       static_cast<const raw*>(Y), static_cast<const raw*>(q), static_cast<raw*>(r), rows, int(N),
                       int(D));
    return cdssm_host::check_launch(op);
  });
}

extern "C" int cdssm_state_readout_bwd(int dtype, const void* Y, const void* q, const void* dr, void* dY, void* dq,
                                       int64_t n, int64_t N, int64_t D, hipStream_t stream) {
  const char* op = "cdssm_state_readout_bwd";
  return by_dtype(dtype, op, [&](auto t) -> int {
    using T = decltype(t);
    using raw = typename T::raw;
    constexpr int V = Vec16<T>::N;
    if (n <= 0 || N <= 0 || D <= 0 || D % V != 0 || n * N > (int64_t(1) << 38)) {
      cdssm_host::set_error("%s: need n, N > 0 and D a positive multiple of %d (n=%lld N=%lld D=%lld)", op, V,
                            (long long)n, (long long)N, (long long)D);
      return CDSSM_EINVAL;
    }
    if (!Y || !q || !dr || !dY || !dq) {
      cdssm_host::set_error("%s: null pointer argument", op);
      return CDSSM_EINVAL;
    }
    if ((reinterpret_cast<uintptr_t>(Y) | reinterpret_cast<uintptr_t>(q) | reinterpret_cast<uintptr_t>(dY) |
         reinterpret_cast<uintptr_t>(dq)) & 15) {
      cdssm_host::set_error("%s: Y, q, dY and dq must be 16-byte aligned", op);
      return CDSSM_EINVAL;
    }
    const int64_t threads = n * (D / V);
    hipLaunchKernelGGL(state_readout_bwd_kernel<T>, dim3(unsigned((threads + 255) / 256)), dim3(256), 0, stream,
                       static_cast<const raw*>(Y), static_cast<const raw*>(q), static_cast<const raw*>(dr),
                       static_cast<raw*>(dY), static_cast<raw*>(dq), n, int(N), int(D));
    return cdssm_host::check_launch(op);
  });
}

// Slices of the token axis per batch row in the GroupNorm passes.
static int gn_slices(int64_t L) { return int(std::min<int64_t>(16, std::max<int64_t>(1, L / 256))); }

extern "C" int64_t cdssm_group_norm_workspace_bytes(int64_t B, int64_t G, int64_t L) {
  if (B <= 0 || G <= 0 || L <= 0) return -1;
  const int64_t S = gn_slices(L);
  return (B * G * S + B * G) * int64_t(sizeof(float2));
}

extern "C" int cdssm_group_norm_gate_fwd(int dtype, int param_dtype, const void* y, const void* gamma, const void* beta,
                                         const void* z, int64_t z_token_stride, const void* x_conv, const void* Dp,
                                         void* out, float* workspace, int64_t B, int64_t L, int64_t C, int64_t G,
                                         float eps, hipStream_t stream) {
  const char* op = "cdssm_group_norm_gate_fwd";
  return by_dtype(dtype, op, [&](auto t) -> int {
    using T = decltype(t);
    using raw = typename T::raw;
    if (param_dtype != 0 && param_dtype != 1) {
      cdssm_host::set_error("%s: param_dtype must be 0 (fp32) or 1 (bf16), got %d", op, param_dtype);
      return CDSSM_EINVAL;
    }
    if (B <= 0 || L <= 0 || C <= 0 || G <= 0 || C % G != 0 || z_token_stride < C || B * L >= (int64_t(1) << 31) ||
        C >= (int64_t(1) << 24) || B * G * C > 0x7fffffffLL) {
      cdssm_host::set_error("%s: need C divisible by G and a z token stride >= C (B=%lld L=%lld C=%lld G=%lld)",
                            op, (long long)B, (long long)L, (long long)C, (long long)G);
      return CDSSM_EINVAL;
    }
    if (!y || !gamma || !beta || !z || !x_conv || !Dp || !out || !workspace) {
      cdssm_host::set_error("%s: null pointer argument", op);
      return CDSSM_EINVAL;
    }
    // 16-byte vectors where every access stays aligned, else one element per access
    constexpr int NV = 16 / T::bytes;
    const bool vec = (C / G) % NV == 0 && aligned16(y) && aligned16(z) && aligned16(x_conv) && aligned16(Dp) &&
                     aligned16(out) && aligned16(gamma) && aligned16(beta) && (z_token_stride * T::bytes) % 16 == 0;
    const int S = gn_slices(L);
    const int BG = int(B * G);
    float2* part = reinterpret_cast<float2*>(workspace);
    float2* stats = part + int64_t(BG) * S;
    auto go = [&](auto nc, auto pt) {
      constexpr int N = decltype(nc)::value;
      using P = decltype(pt);
      using praw = typename P::raw;
      hipLaunchKernelGGL((gn_partial_kernel<T, N>), dim3(unsigned(BG * S)), dim3(kGnThreads), 0, stream,
                         static_cast<const raw*>(y), part, int(L), int(C), int(G), S);
      hipLaunchKernelGGL(gn_finalize_kernel<T>, dim3(unsigned((BG + 255) / 256)), dim3(256), 0, stream,
                         static_cast<const raw*>(y), part, stats, BG, int(L), int(C), int(G), S, eps);
      const int vpr = int(C) / N;
      const dim3 grid(unsigned((B * L + 3) / 4), unsigned((vpr + kWave - 1) / kWave));
      hipLaunchKernelGGL((gn_gate_kernel<T, P, N>), grid, dim3(256), 0, stream, static_cast<const raw*>(y), stats,
                         static_cast<const praw*>(gamma), static_cast<const praw*>(beta), static_cast<const raw*>(z),
                         z_token_stride, static_cast<const raw*>(x_conv), static_cast<const raw*>(Dp),
                         static_cast<raw*>(out), int(B * L), int(L), int(C), int(G));
    };
    if (vec && param_dtype == 1)
      go(std::integral_constant<int, NV>{}, BF16{});
    else if (vec)
      go(std::integral_constant<int, NV>{}, F32{});
    else if (param_dtype == 1)
      go(std::integral_constant<int, 1>{}, BF16{});
    else
      go(std::integral_constant<int, 1>{}, F32{});
    return cdssm_host::check_launch(op);
  });
}

// Token slices per batch row of the backward's partial sums: 32 tokens each
// (8 per thread), so that a config-4 call (B8 L2048, C 1024) has 1024 blocks.
static int gnb_slices(int64_t L) { return int(std::min<int64_t>(512, std::max<int64_t>(1, (L + 31) / 32))); }

extern "C" int64_t cdssm_group_norm_gate_bwd_workspace_bytes(int64_t B, int64_t G, int64_t L, int64_t C) {
  if (B <= 0 || G <= 0 || L <= 0 || C <= 0) return -1;
  const int64_t S = gnb_slices(L);
  // per-channel partials (B S, 3, C), per-group partials (B G S) and means (B G)
  return B * S * 3 * C * int64_t(sizeof(float)) + (B * G * S + B * G) * int64_t(sizeof(float2));
}

extern "C" int cdssm_group_norm_gate_bwd(int dtype, int param_dtype, const void* y, const void* gamma,
                                         const void* beta, const void* z, int64_t z_token_stride, const void* x_conv,
                                         const void* Dp, const float* fwd_workspace, const void* dout, void* dy,
                                         void* dz, void* dx_conv, void* dgamma, void* dbeta, void* dD,
                                         float* workspace, int64_t B, int64_t L, int64_t C, int64_t G,
                                         hipStream_t stream) {
  const char* op = "cdssm_group_norm_gate_bwd";
  return by_dtype(dtype, op, [&](auto t) -> int {
    using T = decltype(t);
    using raw = typename T::raw;
    constexpr int NV = 16 / T::bytes;
    if (param_dtype != 0 && param_dtype != 1) {
      cdssm_host::set_error("%s: param_dtype must be 0 (fp32) or 1 (bf16), got %d", op, param_dtype);
      return CDSSM_EINVAL;
    }
    if (B <= 0 || L <= 0 || C <= 0 || G <= 0 || C % G != 0 || z_token_stride < C || B * L >= (int64_t(1) << 31) ||
        C >= (int64_t(1) << 24) || B * G * C > 0x7fffffffLL) {
      cdssm_host::set_error("%s: need C divisible by G and a z token stride >= C (B=%lld L=%lld C=%lld G=%lld)",
                            op, (long long)B, (long long)L, (long long)C, (long long)G);
      return CDSSM_EINVAL;
    }
    // a channel vector in one group, whole groups in a block's 64 vectors
    const int64_t Cg = C / G;
    if (Cg % NV != 0 || (int64_t(kWave) * NV) % Cg != 0) {
      cdssm_host::set_error("%s: the group width C / G = %lld must be a multiple of %d dividing %d", op,
                            (long long)Cg, NV, kWave * NV);
      return CDSSM_EINVAL;
    }
    if (!y || !gamma || !beta || !z || !x_conv || !Dp || !fwd_workspace || !dout || !dy || !dz || !dx_conv ||
        !dgamma || !dbeta || !dD || !workspace) {
      cdssm_host::set_error("%s: null pointer argument", op);
      return CDSSM_EINVAL;
    }
    if (!aligned16(y) || !aligned16(z) || !aligned16(x_conv) || !aligned16(Dp) || !aligned16(dout) ||
        !aligned16(dy) || !aligned16(dz) || !aligned16(dx_conv) || !aligned16(gamma) || !aligned16(beta) ||
        (z_token_stride * T::bytes) % 16 != 0) {
      cdssm_host::set_error("%s: tensors must be 16-byte aligned (and z's token stride a multiple of 16 bytes)", op);
      return CDSSM_EINVAL;
    }
    const int S = gnb_slices(L);
    const int BG = int(B * G), BS = int(B) * S;
    // the forward's statistics (mean, rstd) follow its partial sums
    const float2* stats = reinterpret_cast<const float2*>(fwd_workspace) + int64_t(BG) * gn_slices(L);
    float* chan = workspace;
    float2* gpart = reinterpret_cast<float2*>(chan + int64_t(BS) * 3 * C);
    float2* gm = gpart + int64_t(BG) * S;
    auto go = [&](auto pt) {
      using P = decltype(pt);
      using praw = typename P::raw;
      const int vpr = int(C) / NV;
      hipLaunchKernelGGL((gnb_reduce_kernel<T, P>), dim3(unsigned(BS), unsigned((vpr + kWave - 1) / kWave)),
                         dim3(256), 0, stream, static_cast<const raw*>(y), stats, static_cast<const praw*>(gamma),
                         static_cast<const praw*>(beta), static_cast<const raw*>(z), z_token_stride,
                         static_cast<const raw*>(x_conv), static_cast<const raw*>(dout), chan, gpart, int(L), int(C),
                         int(G), S);
      const unsigned fblocks = unsigned((3 * C + 15) / 16 + (BG + 255) / 256);
      hipLaunchKernelGGL((gnb_finalize_kernel<T, P>), dim3(fblocks), dim3(256), 0, stream, chan,
                         gpart, static_cast<praw*>(dgamma), static_cast<praw*>(dbeta), static_cast<raw*>(dD), gm, BS,
                         int(C), BG, S, 1.0f / (float(L) * float(Cg)));
      const dim3 grid(unsigned((B * L + 3) / 4), unsigned((vpr + kWave - 1) / kWave));
      hipLaunchKernelGGL((gnb_apply_kernel<T, P>), grid, dim3(256), 0, stream, static_cast<const raw*>(y), stats, gm,
                         static_cast<const praw*>(gamma), static_cast<const praw*>(beta), static_cast<const raw*>(z),
                         z_token_stride, static_cast<const raw*>(Dp), static_cast<const raw*>(dout),
                         static_cast<raw*>(dy), static_cast<raw*>(dz), static_cast<raw*>(dx_conv), int(B * L), int(L),
                         int(C), int(G));
    };
    if (param_dtype == 1)
      go(BF16{});
    else
      go(F32{});
    return cdssm_host::check_launch(op);
  });
}

static int gn_step(const char* op, int dtype, int param_dtype, const void* y, const void* ret, const void* wr,
                   int64_t kr, float* gsum, const void* gamma, const void* beta, const void* z, int64_t z_batch_stride,
                   const void* x_conv, const void* Dp, void* out, int64_t B, int64_t C, int64_t G, float eps,
                   int64_t* position, hipStream_t stream) {
  return by_dtype(dtype, op, [&](auto t) -> int {
    using T = decltype(t);
    using raw = typename T::raw;
    if (param_dtype != 0 && param_dtype != 1) {
      cdssm_host::set_error("%s: param_dtype must be 0 (fp32) or 1 (bf16), got %d", op, param_dtype);
      return CDSSM_EINVAL;
    }
    if (B <= 0 || C <= 0 || G <= 0 || C % G != 0 || G > 8192 || B > 0x7fffffffLL || C >= (int64_t(1) << 24) ||
        z_batch_stride < C) {
      cdssm_host::set_error("%s: need C divisible by G <= 8192 and a z row stride >= C (B=%lld C=%lld G=%lld)", op,
                            (long long)B, (long long)C, (long long)G);
      return CDSSM_EINVAL;
    }
    if (ret && (kr <= 0 || kr > 4096 || (2 * G + C + kr) * int64_t(sizeof(float)) > 65536)) {
      cdssm_host::set_error("%s: need 0 < readout width K <= 4096 and C + 2 G + K <= 16384 (K=%lld C=%lld G=%lld)", op,
                            (long long)kr, (long long)C, (long long)G);
      return CDSSM_EINVAL;
    }
    if (!(y || (ret && wr)) || !gsum || !gamma || !beta || !z || !x_conv || !Dp || !out) {
      cdssm_host::set_error("%s: null pointer argument", op);
      return CDSSM_EINVAL;
    }
    auto go = [&](auto pt) {
      using P = decltype(pt);
      using praw = typename P::raw;
      const size_t lds = size_t(G) * sizeof(float2) + (ret ? size_t(C + kr) * sizeof(float) : 0);
      hipLaunchKernelGGL((gn_gate_step_kernel<T, P>), dim3(unsigned(B)), dim3(256), lds, stream,
                         static_cast<const raw*>(y), static_cast<const raw*>(ret), static_cast<const raw*>(wr),
                         int(kr), reinterpret_cast<float4*>(gsum),
                         static_cast<const praw*>(gamma), static_cast<const praw*>(beta), static_cast<const raw*>(z),
                         z_batch_stride, static_cast<const raw*>(x_conv), static_cast<const raw*>(Dp),
                         static_cast<raw*>(out), int(C), int(G), eps, position);
    };
    if (param_dtype == 1)
      go(BF16{});
    else
      go(F32{});
    return cdssm_host::check_launch(op);
  });
}

extern "C" int cdssm_group_norm_gate_step(int dtype, int param_dtype, const void* y, float* gsum, const void* gamma,
                                          const void* beta, const void* z, int64_t z_batch_stride, const void* x_conv,
                                          const void* Dp, void* out, int64_t B, int64_t C, int64_t G, float eps,
                                          int64_t* position, hipStream_t stream) {
  return gn_step("cdssm_group_norm_gate_step", dtype, param_dtype, y, nullptr, nullptr, 0, gsum, gamma, beta, z,
                 z_batch_stride, x_conv, Dp, out, B, C, G, eps, position, stream);
}

extern "C" int cdssm_readout_group_norm_gate_step(int dtype, int param_dtype, const void* retrieved,
                                                  const void* readout_weight, int64_t K, float* gsum,
                                                  const void* gamma, const void* beta, const void* z,
                                                  int64_t z_batch_stride, const void* x_conv, const void* Dp,
                                                  void* out, int64_t B, int64_t C, int64_t G, float eps,
                                                  int64_t* position, hipStream_t stream) {
  const char* op = "cdssm_readout_group_norm_gate_step";
  if (!retrieved || !readout_weight) {
    cdssm_host::set_error("%s: null pointer argument", op);
    return CDSSM_EINVAL;
  }
  return gn_step(op, dtype, param_dtype, nullptr, retrieved, readout_weight, K, gsum, gamma, beta, z, z_batch_stride,
                 x_conv, Dp, out, B, C, G, eps, position, stream);
}
