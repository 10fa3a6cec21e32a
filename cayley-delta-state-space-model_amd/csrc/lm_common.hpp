// Device helpers shared by the block's fused elementwise kernels (lm_fused.hip)
// and the decode step's fused tail (decode.hip).
#pragma once

#include "common.hpp"

namespace cdssm {
namespace lm {

// Round to the element type (identity for fp32).
template <typename T>
__device__ __forceinline__ float rnd(float x) {
  if constexpr (T::bytes == 2)
    return bf16_to_f32(f32_to_bf16(x));
  else
    return x;
}

// Round a pair to the element type with one packed conversion (identity for fp32).
template <typename T>
__device__ __forceinline__ void rnd2(float& a, float& b) {
  if constexpr (T::bytes == 2) {
    const uint32_t p = pack_bf16x2(a, b);
    a = bf16_lo(p);
    b = bf16_hi(p);
  }
}

// silu(u) = u sigmoid(u) with the hardware reciprocal (about 1 ulp)
__device__ __forceinline__ float silu_fast(float u) { return u * __builtin_amdgcn_rcpf(1.0f + __expf(-u)); }

// ---------------------------------------------------------------------------
// GroupNorm + gate for one decode token of batch row b, with running
// statistics: gsum (B, G, 4) fp32 = (shift K, sum (x - K), sum (x - K)^2,
// count) over every position so far (block.py:215-225).  The row's y is read
// from `y`, or, with `rs` (the row's kr retrieved values in LDS, rounded to the
// element type), formed by the readout projection y_c = rnd(sum_j rs_j W[c][j])
// (block.py:213).  The new token's group sums are added in a fixed order (one
// thread per group), the statistics formed from the totals, and the token
// normalised, gated and skipped as gn_gate_kernel does: with the prefix's sums
// this equals the GroupNorm of a forward over the prefix plus the token, for
// that token.  Every thread of the workgroup takes part (barriers inside);
// gst (G float2) and ys (C floats) are the caller's LDS.
// ---------------------------------------------------------------------------
template <typename T, typename P>
__device__ __forceinline__ void gn_row_step(int b, const typename T::raw* __restrict__ y, const float* rs,
                                            const typename T::raw* __restrict__ wr, int kr,
                                            float4* __restrict__ gsum, const typename P::raw* __restrict__ gamma,
                                            const typename P::raw* __restrict__ beta,
                                            const typename T::raw* __restrict__ z, int64_t z_bs,
                                            const typename T::raw* __restrict__ xc,
                                            const typename T::raw* __restrict__ Dp, typename T::raw* __restrict__ out,
                                            int C, int G, float eps, float2* gst, float* ys) {
  using raw = typename T::raw;
  const int Cg = C / G;
  const raw* yr = y ? y + int64_t(b) * C : nullptr;
  if (rs) {
    constexpr int E = 16 / int(sizeof(raw));  // elements per 16-byte load
    // W rows as 16-byte loads when every row starts on a 16-byte boundary
    const bool vec = kr % E == 0 && (reinterpret_cast<uintptr_t>(wr) & 15u) == 0;
    for (int c = threadIdx.x; c < C; c += blockDim.x) {
      const raw* wc = wr + int64_t(c) * kr;
      float a = 0.0f;
      if (vec) {
        for (int j = 0; j < kr; j += E) {
          const uint4 v = *reinterpret_cast<const uint4*>(wc + j);
          const raw* e = reinterpret_cast<const raw*>(&v);
#pragma unroll
          for (int u = 0; u < E; ++u) a = fmaf(rs[j + u], T::load(e + u), a);
        }
      } else {
        for (int j = 0; j < kr; ++j) a = fmaf(rs[j], T::load(wc + j), a);
      }
      ys[c] = rnd<T>(a);
    }
    __syncthreads();
  }
  auto yv = [&](int c) -> float { return rs ? ys[c] : T::load(yr + c); };
  for (int g = threadIdx.x; g < G; g += blockDim.x) {
    float4 a = gsum[int64_t(b) * G + g];
    float s1 = 0.0f, s2 = 0.0f;
    for (int c = 0; c < Cg; ++c) {
      const float d = yv(g * Cg + c) - a.x;
      s1 += d;
      s2 = fmaf(d, d, s2);
    }
    a.y += s1;
    a.z += s2;
    a.w += float(Cg);
    gsum[int64_t(b) * G + g] = a;
    const float m = a.y / a.w;
    gst[g] = make_float2(a.x + m, rsqrtf(fmaxf(a.z / a.w - m * m, 0.0f) + eps));
  }
  __syncthreads();
  // the token normalised, gated and skipped: 8 channels per thread with 16-byte accesses where the bf16 rows
  // allow (every pointer, and z's row stride, on 16 bytes), else one channel per thread
  const raw* zr = z + int64_t(b) * z_bs;
  const raw* xr = xc + int64_t(b) * C;
  raw* orow = out + int64_t(b) * C;
  const auto a16 = [](const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; };
  if constexpr (T::bytes == 2 && P::bytes == 2) {
    if (C % 8 == 0 && Cg % 8 == 0 && a16(zr) && a16(xr) && a16(orow) && a16(Dp) && a16(gamma) && a16(beta)) {
      for (int c0 = 8 * int(threadIdx.x); c0 < C; c0 += 8 * int(blockDim.x)) {
        const float2 st = gst[c0 / Cg];
        const uint4 zv = *reinterpret_cast<const uint4*>(zr + c0), xv = *reinterpret_cast<const uint4*>(xr + c0);
        const uint4 dv = *reinterpret_cast<const uint4*>(Dp + c0);
        const uint4 gv = *reinterpret_cast<const uint4*>(gamma + c0), bv = *reinterpret_cast<const uint4*>(beta + c0);
        const uint32_t zw[4] = {zv.x, zv.y, zv.z, zv.w}, xw[4] = {xv.x, xv.y, xv.z, xv.w};
        const uint32_t dw[4] = {dv.x, dv.y, dv.z, dv.w}, gw[4] = {gv.x, gv.y, gv.z, gv.w};
        const uint32_t bw[4] = {bv.x, bv.y, bv.z, bv.w};
        uint32_t o[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          float r2[2];
#pragma unroll
          for (int h = 0; h < 2; ++h) {
            const int c = c0 + 2 * i + h;
            const float zz = h ? bf16_hi(zw[i]) : bf16_lo(zw[i]);
            const float xx = h ? bf16_hi(xw[i]) : bf16_lo(xw[i]);
            const float dd = h ? bf16_hi(dw[i]) : bf16_lo(dw[i]);
            const float ga = h ? bf16_hi(gw[i]) : bf16_lo(gw[i]);
            const float be = h ? bf16_hi(bw[i]) : bf16_lo(bw[i]);
            const float gn = rnd<T>(fmaf((yv(c) - st.x) * st.y, ga, be));
            const float sv = rnd<T>(silu_fast(zz));
            r2[h] = rnd<T>(gn * sv) + rnd<T>(dd * xx);
          }
          o[i] = pack_bf16x2(r2[0], r2[1]);
        }
        *reinterpret_cast<uint4*>(orow + c0) = make_uint4(o[0], o[1], o[2], o[3]);
      }
      return;
    }
  }
  for (int c = threadIdx.x; c < C; c += blockDim.x) {
    const float2 st = gst[c / Cg];
    const float gn = rnd<T>(fmaf((yv(c) - st.x) * st.y, P::load(gamma + c), P::load(beta + c)));
    const float s = rnd<T>(silu_fast(T::load(zr + c)));
    const float p = rnd<T>(gn * s);
    const float d = rnd<T>(T::load(Dp + c) * T::load(xr + c));
    T::store(orow + c, p + d);
  }
}

}  // namespace lm
}  // namespace cdssm
