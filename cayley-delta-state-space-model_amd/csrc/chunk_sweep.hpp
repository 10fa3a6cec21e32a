// Chunked (UT-transform) form of the correction pass on the gfx950 matrix
// cores, for bf16 inputs.
//
// For one chunk and head, with the state s entering the chunk (complex
// D-vector), the decay-free correction state c^_t = s - sum_{j<t} x_j k_j
// (exact_correction.cu:83-150 in the decay-free frame) has the coefficients
//   x_j = beta_j (c^_j . k_j) = beta_j ((K s)_j - sum_{i<j} G_ji x_i),  G = K K^T,
// and the readout
//   c^_t . q_t = (Q s)_t - sum_{j<t} P_tj x_j,                          P = Q K^T.
// So the correction needs, per chunk-head, the two Gram tiles G and P and the
// projections K s, Q s -- dense contractions over D that run on MFMA with
// operands read straight from HBM in the instruction's layout (bf16 K, Q
// products are exact in the fp32 accumulator) -- and then a unit-lower-
// triangular solve for x that is scalar per token, with no reduction over D.
//
// Work layout: one wave holds 4 heads of one chunk, processed in blocks of 16
// tokens; lane (g, i) = (lane / 16, lane % 16) owns token 16 b + i of head
// hbase + g of block b.  Every MFMA is v_mfma_f32_16x16x32_bf16:
//   A (16 x 32): lane l holds row l % 16, k = 8 (l / 16) .. + 8
//   B (32 x 16): lane l holds column l % 16, k = 8 (l / 16) .. + 8
//   C (16 x 16): lane l holds column l % 16, rows 4 (l / 16) .. + 4
// (checked on MI355X).  A 16-row slice of K in the A layout and in the B
// layout is the same 16-byte load per lane, so one fragment serves both.
//  * K s, Q s: A = the 4 heads' s split into bf16 hi/lo parts, rows 4 g + {re
//    hi, im hi, re lo, im lo} (head g's rows only, zero elsewhere), B = K / Q
//    fragments of head g, accumulated over the 4 heads: C lands with lane
//    (g, i) holding head g's four parts for token i -- no data movement.
//  * Gram tiles G_b,c, P_b,c (16 x 16, token block b against block c):
//    C = K_c K_b^T per head, so lane (g, i) holds columns 4 g .. 4 g + 3 of
//    row 16 b + i; the 4 heads' tiles are transposed through 4 KB of LDS so
//    that lane (g, i) holds the whole row of its own head.
//  * Solve: in block b, x of token 16 b + j is broadcast to the 16 lanes of
//    its head with DPP row_newbcast:j, and every lane adds G_ij x_j and
//    P_ij x_j; earlier blocks contribute the same way, without a serial
//    dependence.  16 serial steps per block, 4 heads at once.
#pragma once

#include "common.hpp"

namespace cdssm {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

constexpr int kSweepHeads = 4;  // heads per wave
constexpr int kSweepBlock = 16;  // tokens per block
constexpr int kSweepRow = 20;    // LDS row stride (floats) of the tile transpose: conflict-free reads

// 8 bf16 from a 16-byte aligned address.
__device__ __forceinline__ bf16x8_t load_frag(const uint16_t* p) {
  return __builtin_bit_cast(bf16x8_t, *reinterpret_cast<const uint4*>(p));
}

__device__ __forceinline__ f32x4_t mfma16(bf16x8_t a, bf16x8_t b, f32x4_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

// x of lane J of the lane's 16-lane row (DPP row_newbcast).
template <int J>
__device__ __forceinline__ float row_bcast(float x) {
  return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x), 0x150 + J, 0xF, 0xF, true));
}

// row_bcast<j> for a j that is a constant after loop unrolling (the switch folds away).
__device__ __forceinline__ float row_bcast_dyn(float x, int j) {
  switch (j) {
    case 0: return row_bcast<0>(x);
    case 1: return row_bcast<1>(x);
    case 2: return row_bcast<2>(x);
    case 3: return row_bcast<3>(x);
    case 4: return row_bcast<4>(x);
    case 5: return row_bcast<5>(x);
    case 6: return row_bcast<6>(x);
    case 7: return row_bcast<7>(x);
    case 8: return row_bcast<8>(x);
    case 9: return row_bcast<9>(x);
    case 10: return row_bcast<10>(x);
    case 11: return row_bcast<11>(x);
    case 12: return row_bcast<12>(x);
    case 13: return row_bcast<13>(x);
    case 14: return row_bcast<14>(x);
    default: return row_bcast<15>(x);
  }
}

// x from lane i - N of the row; lanes i < N get `fill` (DPP row_shr).
template <int N>
__device__ __forceinline__ float row_shr(float x, float fill) {
  return __int_as_float(__builtin_amdgcn_update_dpp(__float_as_int(fill), __float_as_int(x), 0x110 + N, 0xF, 0xF,
                                                    false));
}

// Inclusive complex product scan over the 16 lanes of each row.
__device__ __forceinline__ void row_cumprod(float& xr, float& xi) {
  for_shifts<16>([&](auto s) {
    constexpr int N = decltype(s)::value;
    const float yr = row_shr<N>(xr, 1.0f), yi = row_shr<N>(xi, 0.0f);
    cmul_acc(xr, xi, yr, yi);
  });
}

// Round-to-nearest bf16 of x and of its remainder: x ~= hi + lo to ~2^-17.
__device__ __forceinline__ void split_bf16(float x, float& hi, float& lo) {
  hi = __builtin_bit_cast(float, uint32_t(f32_to_bf16(x)) << 16);
  lo = x - hi;
}

// LDS of one wave's sweep (floats): the tile transpose, then x of every token
// of the chunk for each of the 4 heads (complex).
template <int NB>
constexpr int sweep_lds_floats() {
  return kSweepHeads * 16 * kSweepRow + kSweepHeads * 16 * NB * 2;
}

// The correction readout of 4 heads x NB blocks of 16 tokens of one chunk.
//  k, q:  (B, L, H, D) bf16; row0 = b L + first token of the chunk, nt = tokens in the chunk
//  s:     the chunk's entering states, head h at s + h D (complex fp32)
//  lds:   sweep_lds_floats<NB>() floats of wave-private LDS
//  tok(b, &beta, &sel, &gr, &gi): the lane's token of block b: beta, the sel_C gate and
//         g_{t-1} (zero beta and sel for tokens past the chunk end or heads past H)
//  emit(b, yr, yi): its correction readout sel_t g_{t-1} (c^_t . q_t)
template <int D, int NB, typename Tok, typename Emit>
__device__ __forceinline__ void corr_sweep(const uint16_t* __restrict__ k, const uint16_t* __restrict__ q,
                                           int64_t row0, int nt, int H, int hbase, const float2* __restrict__ s,
                                           float* lds, Tok&& tok, Emit&& emit) {
  constexpr int KS = D / 32;  // k-steps of 32 over the head dimension
  const int lane = threadIdx.x % kWave;
  const int g = lane / 16, i = lane % 16;
  const int fk = (lane / 16) * 8;  // fragment k offset; the fragment row / column is i
  float* tr = lds;                                  // tile transpose
  float2* xs = reinterpret_cast<float2*>(lds + kSweepHeads * 16 * kSweepRow);  // x per (head, token)

  // A operand of K s and Q s: row m = lane % 16 is part (m % 4) of head m / 4:
  // (re hi, im hi, re lo, im lo); the MFMA of head h uses it only in head h's rows
  const int hs = i / 4, part = i % 4;
  bf16x8_t sv[KS];
  {
    const bool ok = hbase + hs < H;
    const float2* sp = s + int64_t(ok ? hbase + hs : 0) * D;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks)
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float2 x = ok ? sp[ks * 32 + fk + e] : make_float2(0.0f, 0.0f);
        float hi, lo;
        split_bf16((part & 1) ? x.y : x.x, hi, lo);
        sv[ks][e] = __builtin_bit_cast(__bf16, f32_to_bf16((part & 2) ? lo : hi));
      }
  }
  const bf16x8_t zero8 = {};

  // fragment of token tok (clamped into the chunk) of head hbase + h
  auto frag = [&](const uint16_t* x, int t, int h, int ks) {
    const int tt = min(t, nt - 1);
    const int hh = min(hbase + h, H - 1);
    return load_frag(x + ((row0 + tt) * H + hh) * D + ks * 32 + fk);
  };
  // Gram tiles of block b (rows, B operands kb / qb) against block c (A operands kc), 4 heads,
  // transposed so that lane (g, i) holds its head's row i: grow = G[16b + i][16c + 0..15], prow = P[..]
  auto gram_rows = [&](const bf16x8_t (&kc)[kSweepHeads][KS], const bf16x8_t (&kb)[kSweepHeads][KS],
                       const bf16x8_t (&qb)[kSweepHeads][KS], float (&grow)[16], float (&prow)[16]) {
    f32x4_t gt[kSweepHeads], pt[kSweepHeads];
#pragma unroll
    for (int h = 0; h < kSweepHeads; ++h) {
      gt[h] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
      pt[h] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        gt[h] = mfma16(kc[h][ks], kb[h][ks], gt[h]);
        pt[h] = mfma16(kc[h][ks], qb[h][ks], pt[h]);
      }
    }
#pragma unroll
    for (int m = 0; m < 2; ++m) {
      const f32x4_t* src = m == 0 ? gt : pt;
#pragma unroll
      for (int h = 0; h < kSweepHeads; ++h)
        *reinterpret_cast<float4*>(tr + (h * 16 + i) * kSweepRow + 4 * g) =
            make_float4(src[h][0], src[h][1], src[h][2], src[h][3]);
      __builtin_amdgcn_wave_barrier();
      float* dst = m == 0 ? grow : prow;
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const float4 v = *reinterpret_cast<const float4*>(tr + (g * 16 + i) * kSweepRow + 4 * u);
        dst[4 * u + 0] = v.x;
        dst[4 * u + 1] = v.y;
        dst[4 * u + 2] = v.z;
        dst[4 * u + 3] = v.w;
      }
      __builtin_amdgcn_wave_barrier();
    }
  };

#pragma unroll 1
  for (int b = 0; b < NB; ++b) {
    bf16x8_t kb[kSweepHeads][KS], qb[kSweepHeads][KS];
#pragma unroll
    for (int h = 0; h < kSweepHeads; ++h)
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        kb[h][ks] = frag(k, 16 * b + i, h, ks);
        qb[h][ks] = frag(q, 16 * b + i, h, ks);
      }
    // K s and Q s: lane (g, i) gets head g's four parts for token 16 b + i
    f32x4_t cks = {0.0f, 0.0f, 0.0f, 0.0f}, cqs = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int h = 0; h < kSweepHeads; ++h)
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        const bf16x8_t a = hs == h ? sv[ks] : zero8;
        cks = mfma16(a, kb[h][ks], cks);
        cqs = mfma16(a, qb[h][ks], cqs);
      }
    const float ksr = cks[0] + cks[2], ksi = cks[1] + cks[3];
    const float qsr = cqs[0] + cqs[2], qsi = cqs[1] + cqs[3];
    float bt, sel, gr, gi;
    tok(b, bt, sel, gr, gi);

    float ar = 0.0f, ai = 0.0f, rr = 0.0f, ri = 0.0f;  // sum_j G_tj x_j, sum_j P_tj x_j
    float grow[16], prow[16];
    // earlier blocks: x known, no serial dependence
#pragma unroll 1
    for (int c = 0; c < b; ++c) {
      bf16x8_t kc[kSweepHeads][KS];
#pragma unroll
      for (int h = 0; h < kSweepHeads; ++h)
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) kc[h][ks] = frag(k, 16 * c + i, h, ks);
      gram_rows(kc, kb, qb, grow, prow);
      const float2* xc = xs + (g * NB + c) * 16;
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        const float2 x = xc[j];  // the same address across the head's 16 lanes: an LDS broadcast
        ar = fmaf(grow[j], x.x, ar);
        ai = fmaf(grow[j], x.y, ai);
        rr = fmaf(prow[j], x.x, rr);
        ri = fmaf(prow[j], x.y, ri);
      }
    }
    // this block: strictly lower part, 16 serial steps
    gram_rows(kb, kb, qb, grow, prow);
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      grow[j] = j < i ? grow[j] : 0.0f;
      prow[j] = j < i ? prow[j] : 0.0f;
    }
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      const float cr = bt * (ksr - ar), ci = bt * (ksi - ai);
      const float bxr = row_bcast_dyn(cr, j), bxi = row_bcast_dyn(ci, j);
      ar = fmaf(grow[j], bxr, ar);
      ai = fmaf(grow[j], bxi, ai);
      rr = fmaf(prow[j], bxr, rr);
      ri = fmaf(prow[j], bxi, ri);
    }
    xs[(g * NB + b) * 16 + i] = make_float2(bt * (ksr - ar), bt * (ksi - ai));
    __builtin_amdgcn_wave_barrier();
    // y_corr = sel g_{t-1} (Q s - sum_{j<t} P_tj x_j)
    const float cqr = qsr - rr, cqi = qsi - ri;
    emit(b, sel * (gr * cqr - gi * cqi), sel * (gr * cqi + gi * cqr));
  }
}

}  // namespace cdssm
