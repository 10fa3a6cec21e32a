// Skinny GEMM for decode batches: Y (M x N) = X (M x K) W^T (+ bias) (+ R),
// M <= 64, bf16 operands, fp32 accumulation, bf16 out.  With a norm weight
// the rows of X are RMS-normalised first (the model's RMSNorm ahead of
// in_proj and of the LM head, modules.py:49-53):
//   Y = rs ⊙ ((X ⊙ w_norm) W^T),  rs[m] = rsqrt(mean_k X[m,k]^2 + eps),
// with X ⊙ w_norm rounded to bf16 on the way into the matrix cores and rs
// applied to the fp32 result.
//
// These products (decode: in_proj 1024 -> 3104, the stacked gate/Q
// projection 1024 -> 1136 and out_proj 1024 -> 1024 at M = 64) read a weight
// once and a 128 KB activation many times; the library GEMMs tile them for
// large M.  (At N = 32000, the tied head, the activation's re-reads dominate:
// 46 us here against 18 us for the library GEMM.)  Here a workgroup owns 16
// output columns and all M <= 64 rows: its waves split K (8 waves when K is a
// multiple of 256, so that at K = 1024 each wave issues all of its loads in
// one batch; 4 otherwise), each running v_mfma_f32_16x16x32_bf16 on operands
// loaded straight from global memory in the instruction's layout (a 16-byte
// load per lane per fragment: rows of X, rows of W), and the waves' partial
// tiles are summed in a fixed order through LDS.
// So W streams from HBM once with 16-byte loads, X is served by the L2, and a
// call launches ceil(N / 16) workgroups.
//
// Fragment layouts of v_mfma_f32_16x16x32_bf16 (checked on MI355X):
//   A (16 x 32): lane l holds row l % 16, k = 8 (l / 16) .. + 8
//   B (32 x 16): lane l holds column l % 16, k = 8 (l / 16) .. + 8
//   C (16 x 16): lane l holds column l % 16, rows 4 (l / 16) .. + 4
#include <hip/hip_runtime.h>

#include "common.hpp"

namespace cdssm {
namespace sg {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

constexpr int kCols = 16;   // output columns per workgroup
constexpr int kMaxRows = 64;
constexpr int kUnroll = 4;  // k-steps (of 32) whose loads are issued together

__device__ __forceinline__ uint4 ld16(const uint16_t* p) { return *reinterpret_cast<const uint4*>(p); }

// a 16-byte fragment times 8 bf16 weights, rounded back to bf16
__device__ __forceinline__ uint4 scale_frag(uint4 a, uint4 w) {
  uint4 o;
  o.x = pack_bf16x2(bf16_lo(a.x) * bf16_lo(w.x), bf16_hi(a.x) * bf16_hi(w.x));
  o.y = pack_bf16x2(bf16_lo(a.y) * bf16_lo(w.y), bf16_hi(a.y) * bf16_hi(w.y));
  o.z = pack_bf16x2(bf16_lo(a.z) * bf16_lo(w.z), bf16_hi(a.z) * bf16_hi(w.z));
  o.w = pack_bf16x2(bf16_lo(a.w) * bf16_lo(w.w), bf16_hi(a.w) * bf16_hi(w.w));
  return o;
}

__device__ __forceinline__ float sumsq_frag(uint4 a, float s) {
  const uint32_t u[4] = {a.x, a.y, a.z, a.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    s = fmaf(bf16_lo(u[i]), bf16_lo(u[i]), s);
    s = fmaf(bf16_hi(u[i]), bf16_hi(u[i]), s);
  }
  return s;
}

template <bool NORM, int kWaves>
__global__ __launch_bounds__(kWave * kWaves) void skinny_gemm_kernel(
    const uint16_t* __restrict__ X, int64_t ldx, const uint16_t* __restrict__ W, int64_t ldw,
    const uint16_t* __restrict__ bias, const uint16_t* __restrict__ R, int64_t ldr,
    const uint16_t* __restrict__ wnorm, float eps, uint16_t* __restrict__ Y, int64_t ldy, int M, int N, int K) {
  __shared__ f32x4_t part[kWaves][kMaxRows / 16][kWave];  // 4 KB per wave: its partial tiles
  __shared__ float ssq[kWaves][kMaxRows];                  // each wave's partial row sums of squares
  const int wave = int(threadIdx.x) / kWave;
  const int lane = int(threadIdx.x) % kWave;
  const int col = lane % 16, kq = lane / 16;
  const int n0 = int(blockIdx.x) * kCols;
  const int n = min(n0 + col, N - 1);  // loads clamped into the matrix; stores masked
  const int kw = K / kWaves;
  const int kb = wave * kw;
  const uint16_t* wrow = W + int64_t(n) * ldw + kb + 8 * kq;
  const uint16_t* xrow[kMaxRows / 16];
#pragma unroll
  for (int mt = 0; mt < kMaxRows / 16; ++mt) xrow[mt] = X + int64_t(min(mt * 16 + col, M - 1)) * ldx + kb + 8 * kq;
  const uint16_t* nrow = NORM ? wnorm + kb + 8 * kq : nullptr;

  f32x4_t acc[kMaxRows / 16];
  float sq[kMaxRows / 16];
#pragma unroll
  for (int mt = 0; mt < kMaxRows / 16; ++mt) {
    acc[mt] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
    sq[mt] = 0.0f;
  }
  // U k-steps of 32 from k: every load first, then the products
  const auto steps = [&](int k, auto uc) {
    constexpr int U = decltype(uc)::value;
    uint4 b[U], a[U][kMaxRows / 16], g[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      b[u] = ld16(wrow + k + 32 * u);
#pragma unroll
      for (int mt = 0; mt < kMaxRows / 16; ++mt) a[u][mt] = ld16(xrow[mt] + k + 32 * u);
      if constexpr (NORM) g[u] = ld16(nrow + k + 32 * u);
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const bf16x8_t bv = __builtin_bit_cast(bf16x8_t, b[u]);
#pragma unroll
      for (int mt = 0; mt < kMaxRows / 16; ++mt) {
        uint4 av = a[u][mt];
        if constexpr (NORM) {
          sq[mt] = sumsq_frag(av, sq[mt]);
          av = scale_frag(av, g[u]);
        }
        acc[mt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, av), bv, acc[mt], 0, 0, 0);
      }
    }
  };
  // the wave's quarter of K (a multiple of 32): groups of kUnroll steps, then single steps
  int k = 0;
  for (; k + 32 * kUnroll <= kw; k += 32 * kUnroll) steps(k, std::integral_constant<int, kUnroll>{});
  for (; k < kw; k += 32) steps(k, std::integral_constant<int, 1>{});
#pragma unroll
  for (int mt = 0; mt < kMaxRows / 16; ++mt) part[wave][mt][lane] = acc[mt];
  if constexpr (NORM) {
    // the lanes of a row (col) over kq: lanes col, col + 16, col + 32, col + 48
#pragma unroll
    for (int mt = 0; mt < kMaxRows / 16; ++mt) {
      float s = sq[mt];
      s += __shfl_xor(s, 16, kWave);
      s += __shfl_xor(s, 32, kWave);
      if (kq == 0) ssq[wave][mt * 16 + col] = s;
    }
  }
  __syncthreads();

  // wave w < 4 finishes row tile w: the partials in wave order, then the epilogue
  if (wave >= kMaxRows / 16) return;
  const int mt = wave;
  f32x4_t c = part[0][mt][lane];
#pragma unroll
  for (int w = 1; w < kWaves; ++w) {
    const f32x4_t p = part[w][mt][lane];
    c[0] += p[0];
    c[1] += p[1];
    c[2] += p[2];
    c[3] += p[3];
  }
  const int nn = n0 + col;
  if (nn >= N) return;
  const float bv = bias ? bf16_to_f32(bias[nn]) : 0.0f;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int m = mt * 16 + 4 * kq + i;
    if (m < M) {
      float y = c[i];
      if constexpr (NORM) {
        float s = 0.0f;
#pragma unroll
        for (int w = 0; w < kWaves; ++w) s += ssq[w][m];
        s /= float(K);
        y *= __builtin_amdgcn_rsqf(s + eps);
      }
      y += bv;
      if (R) y += bf16_to_f32(R[int64_t(m) * ldr + nn]);
      Y[int64_t(m) * ldy + nn] = f32_to_bf16(y);
    }
  }
}

}  // namespace sg
}  // namespace cdssm

using namespace cdssm;

// Y (M x N, row stride ldy) = X (M x K, row stride ldx) W^T (W: N x K, row
// stride ldw) + bias (N, or null) + R (M x N, row stride ldr, or null); with
// wnorm (K, or null) the rows of X are RMS-normalised first (eps), as
// described above.  bf16 only (dtype 1); M in 1..64, K a multiple of 128,
// rows 16-byte aligned.  No counterpart in the reference (its decode
// re-forwards the whole sequence through torch's GEMMs).
extern "C" int cdssm_skinny_gemm(int dtype, const void* X, int64_t ldx, const void* W, int64_t ldw,
                                 const void* bias, const void* R, int64_t ldr, const void* wnorm, float eps,
                                 void* Y, int64_t ldy, int64_t M, int64_t N, int64_t K, hipStream_t stream) {
  if (dtype != 1) {
    cdssm_host::set_error("cdssm_skinny_gemm: bf16 only (dtype 1), got %d", dtype);
    return CDSSM_EINVAL;
  }
  if (!X || !W || !Y) {
    cdssm_host::set_error("cdssm_skinny_gemm: X, W and Y must not be null");
    return CDSSM_EINVAL;
  }
  if (M < 1 || M > sg::kMaxRows || N < 1 || K < 128 || K % 128 != 0 || N > 0x7fffffffLL / sg::kCols) {
    cdssm_host::set_error("cdssm_skinny_gemm: needs 1 <= M <= 64, K a positive multiple of 128, N >= 1 "
                          "(M %lld, N %lld, K %lld)", (long long)M, (long long)N, (long long)K);
    return CDSSM_EINVAL;
  }
  if (ldx < K || ldw < K || ldy < N || (R && ldr < N) || ldx % 8 || ldw % 8 ||
      (reinterpret_cast<uintptr_t>(X) | reinterpret_cast<uintptr_t>(W) |
       reinterpret_cast<uintptr_t>(wnorm)) % 16) {
    cdssm_host::set_error("cdssm_skinny_gemm: rows of X and W (and wnorm) must be 16-byte aligned and the "
                          "leading dimensions cover the rows");
    return CDSSM_EINVAL;
  }
  const bool eight = K % 256 == 0;  // 8 waves of K / 8 (a multiple of 32) each
  const dim3 grid(unsigned((N + sg::kCols - 1) / sg::kCols)), block(kWave * (eight ? 8 : 4));
  const auto* x = static_cast<const uint16_t*>(X);
  const auto* w = static_cast<const uint16_t*>(W);
  const auto* b = static_cast<const uint16_t*>(bias);
  const auto* r = static_cast<const uint16_t*>(R);
  const auto* g = static_cast<const uint16_t*>(wnorm);
  auto* y = static_cast<uint16_t*>(Y);
  if (wnorm && eight)
    hipLaunchKernelGGL((sg::skinny_gemm_kernel<true, 8>), grid, block, 0, stream, x, ldx, w, ldw, b, r, ldr, g, eps,
                       y, ldy, int(M), int(N), int(K));
  else if (wnorm)
    hipLaunchKernelGGL((sg::skinny_gemm_kernel<true, 4>), grid, block, 0, stream, x, ldx, w, ldw, b, r, ldr, g, eps,
                       y, ldy, int(M), int(N), int(K));
  else if (eight)
    hipLaunchKernelGGL((sg::skinny_gemm_kernel<false, 8>), grid, block, 0, stream, x, ldx, w, ldw, b, r, ldr, g,
                       eps, y, ldy, int(M), int(N), int(K));
  else
    hipLaunchKernelGGL((sg::skinny_gemm_kernel<false, 4>), grid, block, 0, stream, x, ldx, w, ldw, b, r, ldr, g,
                       eps, y, ldy, int(M), int(N), int(K));
  return cdssm_host::check_launch("cdssm_skinny_gemm");
}
