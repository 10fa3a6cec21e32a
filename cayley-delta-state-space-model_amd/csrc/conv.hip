// Causal depthwise conv1d + SiLU on the block's gate pathway
// (conv1d_silu.cu:25-90, CUDAConv1dSiLUOp.forward ops.py:13-21, Conv1dSiLU
// modules.py:14-35):
//   y[b, t, c] = silu(bias[c] + sum_{j<K} w[c, j] x[b, t - (K-1) + j, c]),
//   x[b, s, c] = 0 for s < 0,  silu(u) = u sigmoid(u).
// Layouts as the reference: x, y (B, L, C) token-major, weight (C, 1, K) ->
// (C, K), bias (C); all of one dtype.
//
// Work layout: a thread owns VEC consecutive channels (one 16-byte load per
// token) over TB consecutive tokens, sliding a K-token window in registers,
// so each input element is read once per token block (plus K-1 halo rows).
// Consecutive threads take consecutive channel vectors of the same token:
// every load and store of a wave is one contiguous segment.
#include "common.hpp"

namespace cdssm {

#ifndef CDSSM_CONV_TB
#define CDSSM_CONV_TB 8
#endif
constexpr int kConvTB = CDSSM_CONV_TB;  // tokens per thread

// silu(u) = u sigmoid(u), with the hardware reciprocal (about 1 ulp)
__device__ __forceinline__ float silu_f(float u) { return u * __builtin_amdgcn_rcpf(1.0f + __expf(-u)); }

template <typename T, int VEC>
struct ChanVec {
  static constexpr int W = VEC * T::bytes / 4;
  uint32_t u[W > 0 ? W : 1];
  __device__ __forceinline__ void load(const typename T::raw* p) {
    if constexpr (T::bytes * VEC == 16) {
      const uint4 v = *reinterpret_cast<const uint4*>(p);
      u[0] = v.x; u[1] = v.y; u[2] = v.z; u[3] = v.w;
    } else {
      static_assert(VEC == 1, "scalar or 16-byte channel vectors");
    }
  }
};

template <typename T, int VEC>
__device__ __forceinline__ void load_vec(const typename T::raw* p, float (&o)[VEC]) {
  if constexpr (VEC == 1) {
    o[0] = T::load(p);
  } else {
    ChanVec<T, VEC> cv;
    cv.load(p);
    if constexpr (T::bytes == 2) {
#pragma unroll
      for (int i = 0; i < VEC / 2; ++i) {
        o[2 * i] = bf16_lo(cv.u[i]);
        o[2 * i + 1] = bf16_hi(cv.u[i]);
      }
    } else {
#pragma unroll
      for (int i = 0; i < VEC; ++i) o[i] = __uint_as_float(cv.u[i]);
    }
  }
}

template <typename T, int VEC>
__device__ __forceinline__ void store_vec(typename T::raw* p, const float (&x)[VEC]) {
  if constexpr (VEC == 1) {
    T::store(p, x[0]);
  } else if constexpr (T::bytes == 2) {
    uint32_t u[VEC / 2];
#pragma unroll
    for (int i = 0; i < VEC / 2; ++i) u[i] = pack_bf16x2(x[2 * i], x[2 * i + 1]);
    *reinterpret_cast<uint4*>(p) = make_uint4(u[0], u[1], u[2], u[3]);
  } else {
    *reinterpret_cast<float4*>(p) = make_float4(x[0], x[1], x[2], x[3]);
  }
}

template <typename T, int VEC, int K>
__global__ __launch_bounds__(256) void conv1d_silu_fwd_kernel(const typename T::raw* __restrict__ x,
                                                              const typename T::raw* __restrict__ w,
                                                              const typename T::raw* __restrict__ bias,
                                                              typename T::raw* __restrict__ y, int L, int C,
                                                              int64_t x_ts, int ntb, int n_threads) {
  const int gid = int(blockIdx.x) * int(blockDim.x) + int(threadIdx.x);  // n_threads < 2^31 (host check)
  if (gid >= n_threads) return;
  const int ncv = C / VEC;
  const int rest = gid / ncv;
  const int cv = gid - rest * ncv;
  const int b = rest / ntb;
  const int tb = rest - b * ntb;
  const int c0 = cv * VEC;

  float wt[K][VEC], bs[VEC];
#pragma unroll
  for (int i = 0; i < VEC; ++i) {
    bs[i] = T::load(bias + c0 + i);
#pragma unroll
    for (int j = 0; j < K; ++j) wt[j][i] = T::load(w + int64_t(c0 + i) * K + j);
  }
  const int t0 = tb * kConvTB;
  const typename T::raw* xb = x + int64_t(b) * L * x_ts + c0;
  typename T::raw* yb = y + int64_t(b) * L * C + c0;
  // window: win[j] holds x[t - (K-1) + j]
  float win[K][VEC];
#pragma unroll
  for (int j = 0; j < K - 1; ++j) {
    const int s = t0 - (K - 1) + j;
    if (s >= 0) {
      load_vec<T, VEC>(xb + int64_t(s) * x_ts, win[j + 1]);
    } else {
#pragma unroll
      for (int i = 0; i < VEC; ++i) win[j + 1][i] = 0.0f;
    }
  }
  const int t1 = min(t0 + kConvTB, L);
  for (int t = t0; t < t1; ++t) {
#pragma unroll
    for (int j = 0; j < K - 1; ++j)
#pragma unroll
      for (int i = 0; i < VEC; ++i) win[j][i] = win[j + 1][i];
    load_vec<T, VEC>(xb + int64_t(t) * x_ts, win[K - 1]);
    float o[VEC];
#pragma unroll
    for (int i = 0; i < VEC; ++i) {
      float u = bs[i];
#pragma unroll
      for (int j = 0; j < K; ++j) u = fmaf(wt[j][i], win[j][i], u);
      o[i] = silu_f(u);
    }
    store_vec<T, VEC>(yb + int64_t(t) * C, o);
  }
}

// One decode step of the conv: window (B, K-1, C) holds the last K-1 inputs
// of each row (oldest first, zeros before the sequence start); the new input x
// (B, C) completes the K taps in the order of the full convolution (so the
// output equals the full conv's at that position), then the window shifts.
template <typename T>
__global__ __launch_bounds__(256) void conv1d_silu_step_kernel(const typename T::raw* __restrict__ x, int64_t x_bs,
                                                               typename T::raw* __restrict__ win,
                                                               const typename T::raw* __restrict__ w,
                                                               const typename T::raw* __restrict__ bias,
                                                               typename T::raw* __restrict__ y, int B, int C, int K) {
  const int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= int64_t(B) * C) return;
  const int b = int(i / C), ch = int(i - int64_t(b) * C);
  typename T::raw* wr = win + int64_t(b) * (K - 1) * C + ch;
  const float xn = T::load(x + int64_t(b) * x_bs + ch);
  float u = T::load(bias + ch);
  for (int j = 0; j < K - 1; ++j) u = fmaf(T::load(w + int64_t(ch) * K + j), T::load(wr + int64_t(j) * C), u);
  u = fmaf(T::load(w + int64_t(ch) * K + K - 1), xn, u);
  T::store(y + i, silu_f(u));
  for (int j = 0; j + 1 < K - 1; ++j) wr[int64_t(j) * C] = wr[int64_t(j + 1) * C];
  if (K > 1) T::store(wr + int64_t(K - 2) * C, xn);
}

// ---------------------------------------------------------------------------
// Backward (conv1d_silu.cu:95-276, CUDAConv1dSiLUOp.backward ops.py:22-28):
//   u[t] = bias + sum_j w[j] x[t-(K-1)+j],  gu[t] = gy[t] silu'(u[t]),
//   silu'(u) = s (1 + u (1 - s)), s = sigmoid(u)
//   gx[t] = sum_j w[j] gu[t+(K-1)-j]       (gu = 0 past the end)
//   gw[j] = sum_{b,t} gu[t] x[t-(K-1)+j],  gb = sum_{b,t} gu[t]
// A thread owns one channel over kConvBwdTB tokens: it recomputes u over its
// tokens plus the K-1 after them (x from K-1 before to K-1 after), writes gx,
// and its partial weight / bias sums go to a workspace row per (b, token
// block); a second kernel adds the rows in order per (channel, tap).  No
// atomics: the gradients do not depend on timing.
// ---------------------------------------------------------------------------
constexpr int kConvBwdTB = 16;

template <typename T, int K>
__global__ __launch_bounds__(256) void conv1d_silu_bwd_kernel(const typename T::raw* __restrict__ x, int64_t x_ts,
                                                              const typename T::raw* __restrict__ w,
                                                              const typename T::raw* __restrict__ bias,
                                                              const typename T::raw* __restrict__ gy,
                                                              typename T::raw* __restrict__ gx,
                                                              float* __restrict__ part, int L, int C, int ntb,
                                                              int n_threads) {
  constexpr int TB = kConvBwdTB, NX = TB + 2 * (K - 1), NU = TB + K - 1;
  const int gid = int(blockIdx.x) * int(blockDim.x) + int(threadIdx.x);  // n_threads < 2^31 (host check)
  if (gid >= n_threads) return;
  const int rest = gid / C;
  const int c = gid - rest * C;
  const int b = rest / ntb;
  const int tb = rest - b * ntb;
  const int t0 = tb * TB;
  float wt[K];
#pragma unroll
  for (int j = 0; j < K; ++j) wt[j] = T::load(w + int64_t(c) * K + j);
  const float bs = T::load(bias + c);
  const typename T::raw* xb = x + int64_t(b) * L * x_ts + c;
  const typename T::raw* gyb = gy + int64_t(b) * L * C + c;
  // xs[i] = x[t0 - (K-1) + i], zero outside [0, L)
  float xs[NX];
#pragma unroll
  for (int i = 0; i < NX; ++i) {
    const int s = t0 - (K - 1) + i;
    xs[i] = (s >= 0 && s < L) ? T::load(xb + int64_t(s) * x_ts) : 0.0f;
  }
  // gu[i] at token t0 + i (zero at and past L)
  float gu[NU];
#pragma unroll
  for (int i = 0; i < NU; ++i) {
    const int t = t0 + i;
    float u = bs;
#pragma unroll
    for (int j = 0; j < K; ++j) u = fmaf(wt[j], xs[i + j], u);
    const float sg = 1.0f / (1.0f + __expf(-u));
    gu[i] = t < L ? T::load(gyb + int64_t(t) * C) * (sg * (1.0f + u * (1.0f - sg))) : 0.0f;
  }
  float gw[K], gb = 0.0f;
#pragma unroll
  for (int j = 0; j < K; ++j) gw[j] = 0.0f;
#pragma unroll
  for (int i = 0; i < TB; ++i) {
    const int t = t0 + i;
    if (t < L) {
      float a = 0.0f;
#pragma unroll
      for (int j = 0; j < K; ++j) a = fmaf(wt[j], gu[i + K - 1 - j], a);
      T::store(gx + (int64_t(b) * L + t) * C + c, a);
#pragma unroll
      for (int j = 0; j < K; ++j) gw[j] = fmaf(gu[i], xs[i + j], gw[j]);
      gb += gu[i];
    }
  }
  float* pr = part + int64_t(b * ntb + tb) * (K + 1) * C + c;
#pragma unroll
  for (int j = 0; j < K; ++j) pr[int64_t(j) * C] = gw[j];
  pr[int64_t(K) * C] = gb;
}

// The same backward with VEC adjacent channels per thread (16-byte rows of x,
// grad_out and grad_x; the caller checks C % VEC == 0, 16-byte aligned rows):
// the thread walks its kConvBwdTB tokens plus the K-1 after them once, keeping
// the last K inputs and the last K values of gu in registers; gu at token t is
// formed when x[t] arrives, the weight / bias partials take it at once (owned
// tokens), and gx[t-(K-1)] is complete when gu[t] is.  Every sum runs in the
// order of the kernel above, so both give the same bits.
template <typename T, int K, int VEC>
__global__ __launch_bounds__(256) void conv1d_silu_bwd_vec_kernel(const typename T::raw* __restrict__ x, int64_t x_ts,
                                                                  const typename T::raw* __restrict__ w,
                                                                  const typename T::raw* __restrict__ bias,
                                                                  const typename T::raw* __restrict__ gy,
                                                                  typename T::raw* __restrict__ gx,
                                                                  float* __restrict__ part, int L, int C, int ntb,
                                                                  int n_threads) {
  constexpr int TB = kConvBwdTB;
  const int gid = int(blockIdx.x) * int(blockDim.x) + int(threadIdx.x);  // n_threads < 2^31 (host check)
  if (gid >= n_threads) return;
  const int ncv = C / VEC;
  const int rest = gid / ncv;
  const int c = (gid - rest * ncv) * VEC;
  const int b = rest / ntb;
  const int tb = rest - b * ntb;
  const int t0 = tb * TB;
  float wt[K][VEC], bs[VEC];
#pragma unroll
  for (int v = 0; v < VEC; ++v) {
    bs[v] = T::load(bias + c + v);
#pragma unroll
    for (int j = 0; j < K; ++j) wt[j][v] = T::load(w + int64_t(c + v) * K + j);
  }
  const typename T::raw* xb = x + int64_t(b) * L * x_ts + c;
  const typename T::raw* gyb = gy + int64_t(b) * L * C + c;
  typename T::raw* gxb = gx + int64_t(b) * L * C + c;
  // xw[j] = x[t - (K-1) + j] (zero outside [0, L)), gw_[j] = gu[t - (K-1) + j] at step t
  float xw[K][VEC], gw_[K][VEC];
#pragma unroll
  for (int j = 0; j < K; ++j)
#pragma unroll
    for (int v = 0; v < VEC; ++v) {
      xw[j][v] = 0.0f;
      gw_[j][v] = 0.0f;
    }
#pragma unroll
  for (int j = 1; j < K; ++j) {
    const int s = t0 - K + j;  // x[t0 - (K-1) + (j - 1)]
    if (s >= 0 && s < L) load_vec<T, VEC>(xb + int64_t(s) * x_ts, xw[j]);
  }
  float gwt[K][VEC], gbs[VEC];
#pragma unroll
  for (int v = 0; v < VEC; ++v) {
    gbs[v] = 0.0f;
#pragma unroll
    for (int j = 0; j < K; ++j) gwt[j][v] = 0.0f;
  }
#pragma unroll
  for (int i = 0; i < TB + K - 1; ++i) {
    const int t = t0 + i;
    // shift the windows and bring in x[t] and grad_out[t]
#pragma unroll
    for (int j = 0; j < K - 1; ++j)
#pragma unroll
      for (int v = 0; v < VEC; ++v) {
        xw[j][v] = xw[j + 1][v];
        gw_[j][v] = gw_[j + 1][v];
      }
    float g[VEC];
    if (t < L) {
      load_vec<T, VEC>(xb + int64_t(t) * x_ts, xw[K - 1]);
      load_vec<T, VEC>(gyb + int64_t(t) * C, g);
    } else {
#pragma unroll
      for (int v = 0; v < VEC; ++v) {
        xw[K - 1][v] = 0.0f;
        g[v] = 0.0f;
      }
    }
#pragma unroll
    for (int v = 0; v < VEC; ++v) {
      float u = bs[v];
#pragma unroll
      for (int j = 0; j < K; ++j) u = fmaf(wt[j][v], xw[j][v], u);
      const float sg = 1.0f / (1.0f + __expf(-u));
      gw_[K - 1][v] = t < L ? g[v] * (sg * (1.0f + u * (1.0f - sg))) : 0.0f;
    }
    if (i < TB && t < L) {  // an owned token: the weight and bias partials
#pragma unroll
      for (int v = 0; v < VEC; ++v) {
#pragma unroll
        for (int j = 0; j < K; ++j) gwt[j][v] = fmaf(gw_[K - 1][v], xw[j][v], gwt[j][v]);
        gbs[v] += gw_[K - 1][v];
      }
    }
    const int so = t - (K - 1);  // gx[so] = sum_j w[j] gu[so + (K-1) - j] = sum_j w[j] gu[t - j]
    if (i >= K - 1 && so < L) {
      float a[VEC];
#pragma unroll
      for (int v = 0; v < VEC; ++v) {
        a[v] = 0.0f;
#pragma unroll
        for (int j = 0; j < K; ++j) a[v] = fmaf(wt[j][v], gw_[K - 1 - j][v], a[v]);
      }
      store_vec<T, VEC>(gxb + int64_t(so) * C, a);
    }
  }
  float* pr = part + int64_t(b * ntb + tb) * (K + 1) * C + c;
#pragma unroll
  for (int j = 0; j < K; ++j)
#pragma unroll
    for (int v = 0; v < VEC; ++v) pr[int64_t(j) * C + v] = gwt[j][v];
#pragma unroll
  for (int v = 0; v < VEC; ++v) pr[int64_t(K) * C + v] = gbs[v];
}

// grad_weight (C, K) and grad_bias (C), fp32: the partial rows added in order.
// Sum of the partial rows: a workgroup of kRedWaves waves owns 64 adjacent
// columns (j, c) of the (rows, K + 1, C) partials (one column per lane, so each
// row's 64 values are one 256-byte load); wave w adds rows w, w + kRedWaves, ...
// with four independent accumulators, and the waves' sums are added through LDS
// in wave order, so the result does not depend on timing.
constexpr int kRedWaves = 16;

__global__ __launch_bounds__(64 * kRedWaves) void conv1d_silu_bwd_reduce_kernel(const float* __restrict__ part,
                                                                                float* __restrict__ gw,
                                                                                float* __restrict__ gb, int rows,
                                                                                int C, int K) {
  __shared__ float acc_s[kRedWaves][64];
  const int lane = int(threadIdx.x) % 64, wv = int(threadIdx.x) / 64;
  const int ncol = (K + 1) * C;
  const int col = int(blockIdx.x) * 64 + lane;  // (tap j, channel c) = j * C + c; j = K: bias
  const bool ok = col < ncol;
  const int cc = ok ? col : ncol - 1;
  float a0 = 0.0f, a1 = 0.0f, a2 = 0.0f, a3 = 0.0f;
  int r = wv;
  for (; r + 3 * kRedWaves < rows; r += 4 * kRedWaves) {
    a0 += part[int64_t(r) * ncol + cc];
    a1 += part[int64_t(r + kRedWaves) * ncol + cc];
    a2 += part[int64_t(r + 2 * kRedWaves) * ncol + cc];
    a3 += part[int64_t(r + 3 * kRedWaves) * ncol + cc];
  }
  for (; r < rows; r += kRedWaves) a0 += part[int64_t(r) * ncol + cc];
  acc_s[wv][lane] = (a0 + a1) + (a2 + a3);
  __syncthreads();
  if (wv == 0 && ok) {
    float a = 0.0f;
#pragma unroll
    for (int w = 0; w < kRedWaves; ++w) a += acc_s[w][lane];
    const int j = col / C, c = col - j * C;
    if (j < K)
      gw[int64_t(c) * K + j] = a;
    else
      gb[c] = a;
  }
}

template <typename T, int K>
int launch_conv_bwd(const void* x, int64_t x_ts, const void* w, const void* bias, const void* gy, void* gx,
                    float* gw, float* gb, float* ws, int64_t B, int64_t L, int64_t C, hipStream_t stream) {
  using raw = typename T::raw;
  constexpr int VEC = 16 / T::bytes;
  const int ntb = int((L + kConvBwdTB - 1) / kConvBwdTB);
  const auto a16 = [](const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; };
  const bool vec = C % VEC == 0 && (x_ts * T::bytes) % 16 == 0 && a16(x) && a16(gy) && a16(gx);
  if (vec) {
    const int n = int(B * ntb * (C / VEC));
    hipLaunchKernelGGL((conv1d_silu_bwd_vec_kernel<T, K, VEC>), dim3(unsigned((n + 255) / 256)), dim3(256), 0,
                       stream, static_cast<const raw*>(x), x_ts, static_cast<const raw*>(w),
                       static_cast<const raw*>(bias), static_cast<const raw*>(gy), static_cast<raw*>(gx), ws, int(L),
                       int(C), ntb, n);
  } else {
    const int n = int(B * ntb * C);
    hipLaunchKernelGGL((conv1d_silu_bwd_kernel<T, K>), dim3(unsigned((n + 255) / 256)), dim3(256), 0, stream,
                       static_cast<const raw*>(x), x_ts, static_cast<const raw*>(w), static_cast<const raw*>(bias),
                       static_cast<const raw*>(gy), static_cast<raw*>(gx), ws, int(L), int(C), ntb, n);
  }
  const int nr = int((K + 1) * C);
  hipLaunchKernelGGL(conv1d_silu_bwd_reduce_kernel, dim3(unsigned((nr + 63) / 64)), dim3(64 * kRedWaves), 0, stream,
                     ws, gw, gb, int(B * ntb), int(C), K);
  return cdssm_host::check_launch("cdssm_conv1d_silu_bwd");
}

template <typename T>
int dispatch_bwd(int64_t K, const void* x, int64_t x_ts, const void* w, const void* bias, const void* gy, void* gx,
                 float* gw, float* gb, float* ws, int64_t B, int64_t L, int64_t C, hipStream_t stream) {
  switch (K) {
    case 1: return launch_conv_bwd<T, 1>(x, x_ts, w, bias, gy, gx, gw, gb, ws, B, L, C, stream);
    case 2: return launch_conv_bwd<T, 2>(x, x_ts, w, bias, gy, gx, gw, gb, ws, B, L, C, stream);
    case 3: return launch_conv_bwd<T, 3>(x, x_ts, w, bias, gy, gx, gw, gb, ws, B, L, C, stream);
    case 4: return launch_conv_bwd<T, 4>(x, x_ts, w, bias, gy, gx, gw, gb, ws, B, L, C, stream);
    case 5: return launch_conv_bwd<T, 5>(x, x_ts, w, bias, gy, gx, gw, gb, ws, B, L, C, stream);
    case 6: return launch_conv_bwd<T, 6>(x, x_ts, w, bias, gy, gx, gw, gb, ws, B, L, C, stream);
    case 7: return launch_conv_bwd<T, 7>(x, x_ts, w, bias, gy, gx, gw, gb, ws, B, L, C, stream);
    default: return launch_conv_bwd<T, 8>(x, x_ts, w, bias, gy, gx, gw, gb, ws, B, L, C, stream);
  }
}

template <typename T, int VEC, int K>
int launch_conv(const void* x, int64_t x_ts, const void* w, const void* bias, void* y, int64_t B, int64_t L,
                int64_t C, hipStream_t stream) {
  using raw = typename T::raw;
  const int ntb = int((L + kConvTB - 1) / kConvTB);
  const int64_t n = B * ntb * (C / VEC);
  hipLaunchKernelGGL((conv1d_silu_fwd_kernel<T, VEC, K>), dim3(unsigned((n + 255) / 256)), dim3(256), 0, stream,
                     static_cast<const raw*>(x), static_cast<const raw*>(w), static_cast<const raw*>(bias),
                     static_cast<raw*>(y), int(L), int(C), x_ts, ntb, int(n));
  return cdssm_host::check_launch("cdssm_conv1d_silu_fwd");
}

template <typename T, int VEC>
int dispatch_k(const void* x, int64_t x_ts, const void* w, const void* bias, void* y, int64_t B, int64_t L,
               int64_t C, int64_t K, hipStream_t stream) {
  switch (K) {
    case 1: return launch_conv<T, VEC, 1>(x, x_ts, w, bias, y, B, L, C, stream);
    case 2: return launch_conv<T, VEC, 2>(x, x_ts, w, bias, y, B, L, C, stream);
    case 3: return launch_conv<T, VEC, 3>(x, x_ts, w, bias, y, B, L, C, stream);
    case 4: return launch_conv<T, VEC, 4>(x, x_ts, w, bias, y, B, L, C, stream);
    case 5: return launch_conv<T, VEC, 5>(x, x_ts, w, bias, y, B, L, C, stream);
    case 6: return launch_conv<T, VEC, 6>(x, x_ts, w, bias, y, B, L, C, stream);
    case 7: return launch_conv<T, VEC, 7>(x, x_ts, w, bias, y, B, L, C, stream);
    default: return launch_conv<T, VEC, 8>(x, x_ts, w, bias, y, B, L, C, stream);
  }
}

}  // namespace cdssm

using namespace cdssm;

extern "C" int cdssm_conv1d_silu_fwd_strided(int dtype, const void* x, int64_t x_token_stride, const void* weight,
                                             const void* bias, void* y, int64_t B, int64_t L, int64_t C, int64_t K,
                                             hipStream_t stream) {
  const char* op = "cdssm_conv1d_silu_fwd";
  if (dtype != 0 && dtype != 1) {
    cdssm_host::set_error("%s: dtype must be 0 (fp32) or 1 (bf16), got %d", op, dtype);
    return CDSSM_EINVAL;
  }
  if (B <= 0 || L <= 0 || C <= 0 || K < 1 || K > 8 || L > 0x7fffffffLL || C > 0x7fffffffLL ||
      B * ((L + kConvTB - 1) / kConvTB) * C >= (int64_t(1) << 31)) {
    cdssm_host::set_error("%s: need B, L, C > 0, B * ceil(L/8) * C < 2^31 and 1 <= kernel_size <= 8 "
                          "(B=%lld L=%lld C=%lld K=%lld)", op,
                          (long long)B, (long long)L, (long long)C, (long long)K);
    return CDSSM_EINVAL;
  }
  if (!x || !weight || !bias || !y) {
    cdssm_host::set_error("%s: null pointer argument", op);
    return CDSSM_EINVAL;
  }
  if (x_token_stride < C) {
    cdssm_host::set_error("%s: x token stride %lld below C = %lld", op, (long long)x_token_stride, (long long)C);
    return CDSSM_EINVAL;
  }
  const int64_t eb = dtype == 1 ? 2 : 4;
  const bool vec = (reinterpret_cast<uintptr_t>(x) % 16 == 0) && (reinterpret_cast<uintptr_t>(y) % 16 == 0) &&
                   (x_token_stride * eb) % 16 == 0;
  if (dtype == 1) {
    if (vec && C % 8 == 0) return dispatch_k<BF16, 8>(x, x_token_stride, weight, bias, y, B, L, C, K, stream);
    return dispatch_k<BF16, 1>(x, x_token_stride, weight, bias, y, B, L, C, K, stream);
  }
  if (vec && C % 4 == 0) return dispatch_k<F32, 4>(x, x_token_stride, weight, bias, y, B, L, C, K, stream);
  return dispatch_k<F32, 1>(x, x_token_stride, weight, bias, y, B, L, C, K, stream);
}

extern "C" int cdssm_conv1d_silu_fwd(int dtype, const void* x, const void* weight, const void* bias, void* y,
                                     int64_t B, int64_t L, int64_t C, int64_t K, hipStream_t stream) {
  return cdssm_conv1d_silu_fwd_strided(dtype, x, C, weight, bias, y, B, L, C, K, stream);
}

extern "C" int cdssm_conv1d_silu_step(int dtype, const void* x, int64_t x_batch_stride, void* window,
                                      const void* weight, const void* bias, void* y, int64_t B, int64_t C, int64_t K,
                                      hipStream_t stream) {
  const char* op = "cdssm_conv1d_silu_step";
  if (dtype != 0 && dtype != 1) {
    cdssm_host::set_error("%s: dtype must be 0 (fp32) or 1 (bf16), got %d", op, dtype);
    return CDSSM_EINVAL;
  }
  if (B <= 0 || C <= 0 || K < 1 || K > 8 || B * C >= (int64_t(1) << 31) || x_batch_stride < C) {
    cdssm_host::set_error("%s: need B, C > 0, B*C < 2^31, 1 <= kernel_size <= 8, x row stride >= C "
                          "(B=%lld C=%lld K=%lld)", op, (long long)B, (long long)C, (long long)K);
    return CDSSM_EINVAL;
  }
  if (!x || (K > 1 && !window) || !weight || !bias || !y) {
    cdssm_host::set_error("%s: null pointer argument", op);
    return CDSSM_EINVAL;
  }
  const unsigned grid = unsigned((B * C + 255) / 256);
  if (dtype == 1)
    hipLaunchKernelGGL(conv1d_silu_step_kernel<BF16>, dim3(grid), dim3(256), 0, stream,
                       static_cast<const uint16_t*>(x), x_batch_stride, static_cast<uint16_t*>(window),
                       static_cast<const uint16_t*>(weight), static_cast<const uint16_t*>(bias),
                       static_cast<uint16_t*>(y), int(B), int(C), int(K));
  else
    hipLaunchKernelGGL(conv1d_silu_step_kernel<F32>, dim3(grid), dim3(256), 0, stream, static_cast<const float*>(x),
                       x_batch_stride, static_cast<float*>(window), static_cast<const float*>(weight),
                       static_cast<const float*>(bias), static_cast<float*>(y), int(B), int(C), int(K));
  return cdssm_host::check_launch(op);
}

extern "C" int64_t cdssm_conv1d_silu_bwd_workspace_bytes(int64_t B, int64_t L, int64_t C, int64_t K) {
  if (B <= 0 || L <= 0 || C <= 0 || K < 1 || K > 8) return -1;
  return B * ((L + kConvBwdTB - 1) / kConvBwdTB) * (K + 1) * C * int64_t(sizeof(float));
}

extern "C" int cdssm_conv1d_silu_bwd(int dtype, const void* x, int64_t x_token_stride, const void* weight,
                                     const void* bias, const void* grad_out, void* grad_x, float* grad_weight,
                                     float* grad_bias, float* workspace, int64_t B, int64_t L, int64_t C, int64_t K,
                                     hipStream_t stream) {
  const char* op = "cdssm_conv1d_silu_bwd";
  if (dtype != 0 && dtype != 1) {
    cdssm_host::set_error("%s: dtype must be 0 (fp32) or 1 (bf16), got %d", op, dtype);
    return CDSSM_EINVAL;
  }
  if (B <= 0 || L <= 0 || C <= 0 || K < 1 || K > 8 || x_token_stride < C ||
      B * ((L + kConvBwdTB - 1) / kConvBwdTB) * C >= (int64_t(1) << 31) || B * L >= (int64_t(1) << 31)) {
    cdssm_host::set_error("%s: need B, L, C > 0, B * ceil(L/16) * C < 2^31, 1 <= kernel_size <= 8, "
                          "x token stride >= C (B=%lld L=%lld C=%lld K=%lld)",
                          op, (long long)B, (long long)L, (long long)C, (long long)K);
    return CDSSM_EINVAL;
  }
  if (!x || !weight || !bias || !grad_out || !grad_x || !grad_weight || !grad_bias || !workspace) {
    cdssm_host::set_error("%s: null pointer argument", op);
    return CDSSM_EINVAL;
  }
  if (dtype == 1)
    return dispatch_bwd<BF16>(K, x, x_token_stride, weight, bias, grad_out, grad_x, grad_weight, grad_bias, workspace,
                              B, L, C, stream);
  return dispatch_bwd<F32>(K, x, x_token_stride, weight, bias, grad_out, grad_x, grad_weight, grad_bias, workspace,
                           B, L, C, stream);
}
