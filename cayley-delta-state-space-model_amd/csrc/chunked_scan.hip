// Chunked (UT-transform) scan on the gfx950 matrix cores for state_dim N = 16,
// the reference's default (config/model.py:128), gate-level readout form:
//   y = sel_C (Y . q),  Y = SSDChunkwiseScan(A_bar, K, V vp, beta)
// (ssd.py:39-111 with block.py:194-211; the current-token shortcut of
// block.py:202-205 optionally folded in), without forming Y (B,L,H,N,D).
// bf16 inputs, fp32 states.
//
// A head's N/2 = 8 complex state rows share k, q and beta; only their
// transitions a_t and values differ.  So a block of 16 tokens of the chunk
// scan is a dense problem over the head's 16 real state columns.  With H the
// state entering the block (D x 16), per row and token t of the block
//   g_t = prod_{u<=t} a_u (within the block),  e_t the row's update coefficient
//   (z_t = a_t z_{t-1} + e_t k_t, intra_chunk_scan.cu:146-167 restated),
//   e_t / g_t = w_t / g_t - beta_t (k_t.H) - beta_t sum_{s<t} (k_t.k_s) e_s / g_s
//   z_t . q_t = g_t ((q_t.H) + sum_{s<=t} (q_t.k_s) e_s / g_s)
//   H'        = g_15 (H + sum_s (e_s / g_s) k_s)
// The contractions over D -- the Gram tiles K K^T and K Q^T (16 x 16), K H and
// Q H (16 tokens x 16 columns) and the state update K^T E (D x 16) -- run on
// v_mfma_f32_16x16x32_bf16 (k, q are exact in bf16; H and E are split into bf16
// hi + lo parts, ~2^-17 relative).  The triangular solve for e is 16 serial
// steps of DPP broadcasts over the block's 16 tokens, 8 rows at once.  Where
// some row's |g_t| falls below 2^-48 in a block, the wave runs that block in
// true units instead: the same steps with the products prod_{s<u<=t} a_u
// carried forward, which never divides.
//
// R-mode (the reference's three passes): per chunk the local state from zero
// gives the readout z_t.q_t and the chunk's end state (IntraChunkScanFn,
// intra_chunk_scan.cu:100-195); the carry s_{k+1} = (prod_t a_t) s_k + z_end
// (InterChunkScanFn, inter_chunk_scan.cu:52-84); the correction from s_k,
// c_{t+1} = a_t (c_t - beta_t (c_t.k_t) k_t) read before token t
// (ExactCorrectionFn, exact_correction.cu:89-150) is the same block recurrence
// with w = 0 and the readout one token behind.  Three launches:
//   local  per (b, chunk, h): y_loc (fp32 workspace), the chunk's z_end and prod a
//   carry  per (b, h, row, d): the entering state of every chunk, and h_final
//   corr   per (b, chunk, h): y = sel_C (y_loc + c_t . q_t)
//
// Work layout: one wave per (b, chunk, h); lane (g, j) = (lane / 16, lane % 16)
// owns token j of the current block and state rows 2g, 2g+1 (columns 4g .. 4g+3:
// re, im, re, im), which is where the MFMA result tiles put them.
#include "chunk_sweep.hpp"

namespace cdssm {

namespace {

constexpr int kCsRows = 8;    // complex state rows per head (N = 16)
constexpr int kCsCols = 16;   // real state columns
constexpr int kCsWaves = 4;   // waves per workgroup, one (b, chunk, h) each
constexpr float kCsTiny = 0x1p-96f;  // |g|^2 below this: the block runs in true units

// LDS of one wave (floats): the two Gram tile transposes, state transpose, K^T of the block (bf16), E (bf16 hi | lo)
template <int D>
constexpr int cs_lds_floats() {
  return 2 * 16 * kSweepRow + 16 * (D + 4) + D * 8 + 256;
}

struct CsArgs {
  const uint16_t *q, *k, *v, *beta, *sel, *a, *vp;
  const float* scut;  // shortcut scale (one fp32 on the device) or null
  float* yloc;  // (B, L, H, 16) local readout
  float* st;    // (B, NC, H, 16, D): the chunk's z_end, then (carry) its entering state
  float2* ap;   // (B, NC, H, 8): the chunk's product of a
  uint16_t* y;  // (B, L, H, 16)
  int L, H, Q, NC;
  int64_t items;  // B NC H
};

// Lanes of the wave hand data to each other through LDS: every store issued so far completes, and no
// memory access moves across this point (the stores and loads use different types, so the compiler
// would otherwise be free to reorder them).
__device__ __forceinline__ void wave_lds_sync() {
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
  __builtin_amdgcn_wave_barrier();
}

// Two floats as bf16 hi + lo parts, packed in pairs: hi is x truncated to bf16 (its upper 16 bits, taken
// with one v_perm), lo = bf16(x - hi) rounded to nearest; hi + lo = x within 2^-16 |x|.
__device__ __forceinline__ void split_pair(float x0, float x1, uint32_t& hi, uint32_t& lo) {
  const uint32_t u0 = __float_as_uint(x0), u1 = __float_as_uint(x1);
  hi = __builtin_amdgcn_perm(u1, u0, 0x07060302u);
  lo = pack_bf16x2(x0 - __uint_as_float(u0 & 0xffff0000u), x1 - __uint_as_float(u1 & 0xffff0000u));
}

// One block's inputs of a lane (token j of the block): the k and q fragments and the token's scalars,
// loaded a block ahead of their use.
template <int KS>
struct CsBlockIn {
  bf16x8_t kf[KS], qf[KS];
  uint2 araw, vraw;
  uint32_t praw;
  uint16_t braw, sraw;
  bool ok;
};

// x from lane i + N of the lane's 16-lane row; lanes past the row get `fill` (DPP row_shl)
template <int N>
__device__ __forceinline__ float row_shl(float x, float fill) {
  return __int_as_float(__builtin_amdgcn_update_dpp(__float_as_int(fill), __float_as_int(x), 0x100 + N, 0xF, 0xF,
                                                    false));
}

template <int D, bool CORR>
__global__ __launch_bounds__(kWave* kCsWaves) void chunked_sweep_kernel(CsArgs p) {
  extern __shared__ float cs_lds[];
  constexpr int KS = D / 32;  // k-steps of the contractions over D
  constexpr int NT = D / 16;  // 16-column tiles of the state
  const int wave = threadIdx.x / kWave;
  const int64_t item = int64_t(blockIdx.x) * kCsWaves + wave;
  if (item >= p.items) return;  // the whole wave; only wave-level barriers below
  const int lane = threadIdx.x % kWave, g = lane / 16, j = lane % 16;
  const int h = int(item % p.H);
  const int64_t bc = item / p.H;
  const int c = int(bc % p.NC);
  const int64_t b = bc / p.NC;
  const int nt = min(p.Q, p.L - c * p.Q);  // tokens of this chunk
  const int64_t row0 = b * p.L + int64_t(c) * p.Q;

  float* tr = cs_lds + wave * cs_lds_floats<D>();
  float* tp = tr + 16 * kSweepRow;  // the second Gram tile's transpose
  float* hs = tp + 16 * kSweepRow;
  uint16_t* kt = reinterpret_cast<uint16_t*>(hs + 16 * (D + 4));
  uint16_t* et = kt + D * 16;

  // the state in the MFMA result layout: hc[m][r] = column 4g + r, d = 16 m + j
  float hc[NT][4];
  float* stp = p.st + item * kCsCols * D;
#pragma unroll
  for (int m = 0; m < NT; ++m)
#pragma unroll
    for (int r = 0; r < 4; ++r) hc[m][r] = CORR ? stp[(4 * g + r) * D + 16 * m + j] : 0.0f;
  float par[2] = {1.0f, 1.0f}, pai[2] = {0.0f, 0.0f};  // product of a over the chunk (local)
  const bf16x8_t zero8 = {};

  // the inputs of block ib (token j of the block; tokens past the chunk read as inert: a = 1, k = q = 0, beta = 0)
  auto load_block = [&](int ib, CsBlockIn<KS>& in) {
    const int tl = 16 * ib + j;
    in.ok = tl < nt;
    const int64_t tk = (row0 + min(tl, nt - 1)) * p.H + h;  // (b, t, h), clamped into the chunk
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      in.kf[ks] = in.ok ? load_frag(p.k + tk * D + 32 * ks + 8 * g) : zero8;
      in.qf[ks] = in.ok ? load_frag(p.q + tk * D + 32 * ks + 8 * g) : zero8;
    }
    in.araw = in.ok ? *reinterpret_cast<const uint2*>(p.a + tk * 16 + 4 * g) : make_uint2(0x3f80u, 0x3f80u);
    in.braw = in.ok ? p.beta[tk] : uint16_t(0);
    if constexpr (CORR) {
      in.sraw = in.ok ? p.sel[tk] : uint16_t(0);
    } else {
      in.vraw = in.ok ? *reinterpret_cast<const uint2*>(p.v + tk * 16 + 4 * g) : make_uint2(0u, 0u);
      in.praw = in.ok ? *reinterpret_cast<const uint32_t*>(p.vp + tk * 8 + 2 * g) : 0u;
    }
  };
  CsBlockIn<KS> nxt;
  load_block(0, nxt);

#pragma unroll 1
  for (int ib = 0; ib * 16 < p.Q; ++ib) {
    const CsBlockIn<KS> cur = nxt;
    if ((ib + 1) * 16 < p.Q) load_block(ib + 1, nxt);
    const int tl = 16 * ib + j;
    const bool ok = cur.ok;
    const int64_t tk = (row0 + min(tl, nt - 1)) * p.H + h;
    const bf16x8_t* kf = cur.kf;
    const bf16x8_t* qf = cur.qf;
    // the lane's token: a of rows 2g, 2g+1, beta, and w = beta vp v (local) or sel_C (corr)
    float ar[2], ai[2], wr[2] = {0.0f, 0.0f}, wi[2] = {0.0f, 0.0f};
    float vr[2] = {0.0f, 0.0f}, vi[2] = {0.0f, 0.0f};  // vp v (the shortcut's value)
    ar[0] = bf16_lo(cur.araw.x);
    ai[0] = bf16_hi(cur.araw.x);
    ar[1] = bf16_lo(cur.araw.y);
    ai[1] = bf16_hi(cur.araw.y);
    const float bt = bf16_to_f32(cur.braw);
    float sel = 0.0f;
    {
      if constexpr (CORR) {
        sel = bf16_to_f32(cur.sraw);
      } else {
        const uint2 vraw = cur.vraw;
        const uint32_t praw = cur.praw;
        const float p0 = bf16_lo(praw), p1 = bf16_hi(praw);
        vr[0] = p0 * bf16_lo(vraw.x);
        vi[0] = p0 * bf16_hi(vraw.x);
        vr[1] = p1 * bf16_lo(vraw.y);
        vi[1] = p1 * bf16_hi(vraw.y);
#pragma unroll
        for (int u = 0; u < 2; ++u) {
          wr[u] = bt * vr[u];
          wi[u] = bt * vi[u];
        }
      }
    }

    // Gram rows: lane (g, j) gets row j of G = K K^T and of P = Q K^T (P[t][s] = q_t . k_s)
    float grow[16], prow[16];
    float qk = 0.0f;  // q_t . k_t
    {
      f32x4_t gt = {0.0f, 0.0f, 0.0f, 0.0f}, pt = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        gt = mfma16(kf[ks], kf[ks], gt);
        pt = mfma16(kf[ks], qf[ks], pt);
      }
      // masked by the writing lane, which holds columns s = 4g + r of row j: G for the solve (s < t),
      // P for the readout (s <= t after the token, local; s < t before it, correction)
      float gm[4], pm[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int sc = 4 * g + r;
        gm[r] = sc < j ? gt[r] : 0.0f;
        pm[r] = (CORR ? sc < j : sc <= j) ? pt[r] : 0.0f;
      }
      *reinterpret_cast<float4*>(tr + j * kSweepRow + 4 * g) = make_float4(gm[0], gm[1], gm[2], gm[3]);
      *reinterpret_cast<float4*>(tp + j * kSweepRow + 4 * g) = make_float4(pm[0], pm[1], pm[2], pm[3]);
      wave_lds_sync();
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const float4 x = *reinterpret_cast<const float4*>(tr + j * kSweepRow + 4 * u);
        const float4 y = *reinterpret_cast<const float4*>(tp + j * kSweepRow + 4 * u);
        grow[4 * u + 0] = x.x;
        grow[4 * u + 1] = x.y;
        grow[4 * u + 2] = x.z;
        grow[4 * u + 3] = x.w;
        prow[4 * u + 0] = y.x;
        prow[4 * u + 1] = y.y;
        prow[4 * u + 2] = y.z;
        prow[4 * u + 3] = y.w;
      }
      if constexpr (!CORR) qk = tp[j * kSweepRow + j];  // the local readout keeps the diagonal
      wave_lds_sync();
    }

    // K H and Q H: lane (g, j) gets k_j . H and q_j . H for columns 4g .. 4g+3
    f32x4_t ckh = {0.0f, 0.0f, 0.0f, 0.0f}, cqh = {0.0f, 0.0f, 0.0f, 0.0f};
    {
#pragma unroll
      for (int m = 0; m < NT; ++m)
#pragma unroll
        for (int r = 0; r < 4; ++r) hs[(4 * g + r) * (D + 4) + 16 * m + j] = hc[m][r];
      wave_lds_sync();
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        const float* src = hs + j * (D + 4) + 32 * ks + 8 * g;
        const float4 x0 = *reinterpret_cast<const float4*>(src), x1 = *reinterpret_cast<const float4*>(src + 4);
        uint4 uh, ul;
        split_pair(x0.x, x0.y, uh.x, ul.x);
        split_pair(x0.z, x0.w, uh.y, ul.y);
        split_pair(x1.x, x1.y, uh.z, ul.z);
        split_pair(x1.z, x1.w, uh.w, ul.w);
        const bf16x8_t hhi = __builtin_bit_cast(bf16x8_t, uh), hlo = __builtin_bit_cast(bf16x8_t, ul);
        ckh = mfma16(hhi, kf[ks], ckh);
        ckh = mfma16(hlo, kf[ks], ckh);
        cqh = mfma16(hhi, qf[ks], cqh);
        cqh = mfma16(hlo, qf[ks], cqh);
      }
      wave_lds_sync();
    }

    // g_t per row, and whether every row of the wave keeps |g_t|^2 >= kCsTiny in this block
    float gr[2], gi[2];
    bool small = false;
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      gr[u] = ar[u];
      gi[u] = ai[u];
      row_cumprod(gr[u], gi[u]);
      small = small || !(gr[u] * gr[u] + gi[u] * gi[u] >= kCsTiny);
    }
    const bool exact = __ballot(small) != 0;

    float ro[4];   // readout of rows 2g, 2g+1 (re, im)
    float ec[4];   // E of the state update, columns 4g .. 4g+3 of token j
    float g15r[2], g15i[2];
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const float khr = ckh[2 * u], khi = ckh[2 * u + 1], qhr = cqh[2 * u], qhi = cqh[2 * u + 1];
      g15r[u] = row_bcast<15>(gr[u]);
      g15i[u] = row_bcast<15>(gi[u]);
      // g_{t-1} (1 at the block's first token), the factor of the correction's readout
      const float gpr = row_shr<1>(gr[u], 1.0f), gpi = row_shr<1>(gi[u], 0.0f);
      const float fr = CORR ? gpr : gr[u], fi = CORR ? gpi : gi[u];
      float Ar = 0.0f, Ai = 0.0f, Rr = 0.0f, Ri = 0.0f;
      if (!exact) {
        // rescaled frame: r_t = w_t / g_t - beta_t (k_t . H), e^_t = r_t - beta_t sum_{s<t} G_ts e^_s
        const float m2 = gr[u] * gr[u] + gi[u] * gi[u];
        const float rm = __builtin_amdgcn_rcpf(m2);
        const float ir = gr[u] * rm, ii = -gi[u] * rm;
        const float rr = wr[u] * ir - wi[u] * ii - bt * khr, ri = wr[u] * ii + wi[u] * ir - bt * khi;
#pragma unroll
        for (int s = 0; s < 16; ++s) {
          const float er = row_bcast_dyn(rr - bt * Ar, s), ei = row_bcast_dyn(ri - bt * Ai, s);
          Ar = fmaf(grow[s], er, Ar);
          Ai = fmaf(grow[s], ei, Ai);
          Rr = fmaf(prow[s], er, Rr);
          Ri = fmaf(prow[s], ei, Ri);
        }
        ec[2 * u] = rr - bt * Ar;
        ec[2 * u + 1] = ri - bt * Ai;
        const float xr = qhr + Rr, xi = qhi + Ri;
        ro[2 * u] = fr * xr - fi * xi;
        ro[2 * u + 1] = fr * xi + fi * xr;
      } else {
        // true units: e_t = w_t - beta_t (g_t (k_t . H) + a_t A_t),
        // A_t = sum_{s<t} prod_{s<u<t} a_u G_ts e_s carried forward by a_s each step
        const float br = wr[u] - bt * (gr[u] * khr - gi[u] * khi), bi = wi[u] - bt * (gr[u] * khi + gi[u] * khr);
        float efr = 0.0f, efi = 0.0f;
#pragma unroll
        for (int s = 0; s < 16; ++s) {
          const float cr = br - bt * (ar[u] * Ar - ai[u] * Ai), ci = bi - bt * (ar[u] * Ai + ai[u] * Ar);
          efr = s == j ? cr : efr;
          efi = s == j ? ci : efi;
          const float er = row_bcast_dyn(cr, s), ei = row_bcast_dyn(ci, s);
          const float asr = row_bcast_dyn(ar[u], s), asi = row_bcast_dyn(ai[u], s);
          const float nAr = asr * Ar - asi * Ai + grow[s] * er, nAi = asr * Ai + asi * Ar + grow[s] * ei;
          Ar = nAr;
          Ai = nAi;
          const bool upd = CORR ? s < j : s <= j;
          const float nRr = asr * Rr - asi * Ri + prow[s] * er, nRi = asr * Ri + asi * Rr + prow[s] * ei;
          Rr = upd ? nRr : Rr;
          Ri = upd ? nRi : Ri;
        }
        // E_s = prod_{s<u<=15} a_u e_s (an exclusive suffix product over the row)
        float sr = ar[u], si = ai[u];
        for_shifts<16>([&](auto sh) {
          constexpr int N = decltype(sh)::value;
          const float yr = row_shl<N>(sr, 1.0f), yi = row_shl<N>(si, 0.0f);
          cmul_acc(sr, si, yr, yi);
        });
        const float xr = row_shl<1>(sr, 1.0f), xi = row_shl<1>(si, 0.0f);
        ec[2 * u] = xr * efr - xi * efi;
        ec[2 * u + 1] = xr * efi + xi * efr;
        ro[2 * u] = fr * qhr - fi * qhi + Rr;
        ro[2 * u + 1] = fr * qhi + fi * qhr + Ri;
      }
    }

    // outputs of the block's tokens
    if (ok) {
      float* yl = p.yloc + tk * 16 + 4 * g;
      if constexpr (CORR) {
        const float4 l = *reinterpret_cast<const float4*>(yl);
        uint2 o;
        o.x = pack_bf16x2(sel * (l.x + ro[0]), sel * (l.y + ro[1]));
        o.y = pack_bf16x2(sel * (l.z + ro[2]), sel * (l.w + ro[3]));
        *reinterpret_cast<uint2*>(p.y + tk * 16 + 4 * g) = o;
      } else {
        if (p.scut) {
          // the current-token shortcut through the readout (block.py:202-208): scale (q.k)^2 vp v
          const float sq = *p.scut * qk * qk;
#pragma unroll
          for (int u = 0; u < 2; ++u) {
            ro[2 * u] = fmaf(sq, vr[u], ro[2 * u]);
            ro[2 * u + 1] = fmaf(sq, vi[u], ro[2 * u + 1]);
          }
        }
        *reinterpret_cast<float4*>(yl) = make_float4(ro[0], ro[1], ro[2], ro[3]);
      }
    }

    // state update: H' = g_15 H + K^T E (true units) or g_15 (H + K^T E^) (rescaled)
    auto scale_state = [&]() {
#pragma unroll
      for (int m = 0; m < NT; ++m)
#pragma unroll
        for (int u = 0; u < 2; ++u) cmul_acc(hc[m][2 * u], hc[m][2 * u + 1], g15r[u], g15i[u]);
    };
    if (exact) scale_state();
#pragma unroll
    for (int r = 0; r < 4; r += 2) {
      uint32_t hi, lo;
      split_pair(ec[r], ec[r + 1], hi, lo);
      et[(4 * g + r) * 32 + j] = uint16_t(hi & 0xffffu);
      et[(4 * g + r + 1) * 32 + j] = uint16_t(hi >> 16);
      et[(4 * g + r) * 32 + 16 + j] = uint16_t(lo & 0xffffu);
      et[(4 * g + r + 1) * 32 + 16 + j] = uint16_t(lo >> 16);
    }
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      const uint4 kv = __builtin_bit_cast(uint4, kf[ks]);
      const uint32_t w4[4] = {kv.x, kv.y, kv.z, kv.w};
#pragma unroll
      for (int e = 0; e < 8; ++e)
        kt[(32 * ks + 8 * g + e) * 16 + j] = uint16_t((e & 1) ? w4[e / 2] >> 16 : w4[e / 2] & 0xffffu);
    }
    wave_lds_sync();
    // A: row c = j, k = (hi s 0-7 | hi s 8-15 | lo s 0-7 | lo s 8-15)[g]; B: column d, k = tokens (s 0-7 | 8-15)[g & 1]
    const bf16x8_t ea = load_frag(et + j * 32 + 8 * g);
#pragma unroll
    for (int m = 0; m < NT; ++m) {
      const bf16x8_t kb = load_frag(kt + (16 * m + j) * 16 + 8 * (g & 1));
      f32x4_t acc = {hc[m][0], hc[m][1], hc[m][2], hc[m][3]};
      acc = mfma16(ea, kb, acc);
      hc[m][0] = acc[0];
      hc[m][1] = acc[1];
      hc[m][2] = acc[2];
      hc[m][3] = acc[3];
    }
    wave_lds_sync();
    if (!exact) scale_state();
    if constexpr (!CORR) {
#pragma unroll
      for (int u = 0; u < 2; ++u) cmul_acc(par[u], pai[u], g15r[u], g15i[u]);
    }
  }

  if constexpr (!CORR) {
#pragma unroll
    for (int m = 0; m < NT; ++m)
#pragma unroll
      for (int r = 0; r < 4; ++r) stp[(4 * g + r) * D + 16 * m + j] = hc[m][r];
    if (j == 0) {
      p.ap[item * kCsRows + 2 * g] = make_float2(par[0], pai[0]);
      p.ap[item * kCsRows + 2 * g + 1] = make_float2(par[1], pai[1]);
    }
  }
}

// The carry over chunks, one thread per (b, h, row, d): s_0 = h0, s_{k+1} = (prod a)_k s_k + z_end_k;
// st[k] (z_end_k) is replaced by s_k, the state entering chunk k, and h_final = s_NC.
__global__ __launch_bounds__(256) void chunked_carry_kernel(float* __restrict__ st, const float2* __restrict__ ap,
                                                            const float* __restrict__ h0, float* __restrict__ h_final,
                                                            int64_t lines, int H, int NC, int D) {
  const int64_t idx = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  if (idx >= lines) return;
  const int d = int(idx % D);
  const int n = int((idx / D) % kCsRows);
  const int64_t bh = idx / (int64_t(D) * kCsRows);
  const int h = int(bh % H);
  const int64_t b = bh / H;
  const int64_t hrow = (bh * kCsCols + 2 * n) * D + d;
  float sr = h0 ? h0[hrow] : 0.0f, si = h0 ? h0[hrow + D] : 0.0f;
  constexpr int U = 16;  // chunks whose loads are in flight at once (they do not depend on the carry)
#pragma unroll 1
  for (int c0 = 0; c0 < NC; c0 += U) {
    float zr[U], zi[U];
    float2 a[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int c = min(c0 + u, NC - 1);
      const int64_t item = (b * NC + c) * H + h;
      const float* zp = st + (item * kCsCols + 2 * n) * D + d;
      zr[u] = zp[0];
      zi[u] = zp[D];
      a[u] = ap[item * kCsRows + n];
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      if (c0 + u < NC) {
        const int64_t item = (b * NC + c0 + u) * H + h;
        float* zp = st + (item * kCsCols + 2 * n) * D + d;
        zp[0] = sr;
        zp[D] = si;
        const float nr = a[u].x * sr - a[u].y * si + zr[u];
        si = a[u].x * si + a[u].y * sr + zi[u];
        sr = nr;
      }
    }
  }
  if (h_final) {
    h_final[hrow] = sr;
    h_final[hrow + D] = si;
  }
}

struct CsLayout {
  int64_t NC, yloc, st, ap, floats;
};

CsLayout cs_layout(int64_t B, int64_t L, int64_t H, int64_t D, int64_t chunk) {
  CsLayout w;
  w.NC = (L + chunk - 1) / chunk;
  w.yloc = 0;
  w.st = w.yloc + B * L * H * kCsCols;
  w.ap = w.st + B * w.NC * H * kCsCols * D;
  w.floats = w.ap + B * w.NC * H * kCsRows * 2;
  return w;
}

bool cs_aligned(const void* p, uintptr_t n) { return (reinterpret_cast<uintptr_t>(p) & (n - 1)) == 0; }

template <int D>
int chunked_launch(const CsArgs& a, hipStream_t stream) {
  const unsigned grid = unsigned((a.items + kCsWaves - 1) / kCsWaves);
  const size_t lds = size_t(kCsWaves) * cs_lds_floats<D>() * sizeof(float);
  hipLaunchKernelGGL((chunked_sweep_kernel<D, false>), dim3(grid), dim3(kWave * kCsWaves), lds, stream, a);
  int st = cdssm_host::check_launch("cdssm_chunked_scan_fwd_abar/local");
  if (st) return st;
  return 0;
}

template <int D>
int chunked_launch_corr(const CsArgs& a, hipStream_t stream) {
  const unsigned grid = unsigned((a.items + kCsWaves - 1) / kCsWaves);
  const size_t lds = size_t(kCsWaves) * cs_lds_floats<D>() * sizeof(float);
  hipLaunchKernelGGL((chunked_sweep_kernel<D, true>), dim3(grid), dim3(kWave * kCsWaves), lds, stream, a);
  return cdssm_host::check_launch("cdssm_chunked_scan_fwd_abar/corr");
}

}  // namespace

}  // namespace cdssm

using namespace cdssm;

extern "C" int64_t cdssm_chunked_scan_workspace_bytes(int64_t B, int64_t L, int64_t H, int64_t D, int64_t N,
                                                      int64_t chunk) {
  if (B <= 0 || L <= 0 || H <= 0 || N != 16 || (D != 64 && D != 128) || chunk < 16 || chunk % 16 != 0 ||
      chunk > 256)
    return -1;
  return cs_layout(B, L, H, D, chunk).floats * int64_t(sizeof(float));
}

extern "C" int cdssm_chunked_scan_fwd_abar(int dtype, const void* q, const void* k, const void* v, const void* beta,
                                           const void* sel_c, const void* a_bar, const void* vp, const float* h0,
                                           const float* shortcut_scale, void* y, float* h_final, float* workspace,
                                           int64_t B, int64_t L,
                                           int64_t H, int64_t D, int64_t N, int64_t chunk, hipStream_t stream) {
  const char* op = "cdssm_chunked_scan_fwd_abar";
  if (dtype != 1) {
    cdssm_host::set_error("%s: the chunked MFMA form takes bf16 inputs (dtype 1), got %d", op, dtype);
    return CDSSM_EINVAL;
  }
  if (cdssm_chunked_scan_workspace_bytes(B, L, H, D, N, chunk) < 0) {
    cdssm_host::set_error("%s: need B, L, H > 0, N = 16, D in {64, 128}, chunk a multiple of 16 in [16, 256] "
                          "(B=%lld L=%lld H=%lld D=%lld N=%lld chunk=%lld)",
                          op, (long long)B, (long long)L, (long long)H, (long long)D, (long long)N,
                          (long long)chunk);
    return CDSSM_EINVAL;
  }
  const CsLayout w = cs_layout(B, L, H, D, chunk);
  const int64_t items = B * w.NC * H;
  if (items > (int64_t(1) << 32) || B * L > 0x7fffffffLL || B * H * kCsRows * D > 0x7fffffffLL * 256LL) {
    cdssm_host::set_error("%s: shape too large (B=%lld L=%lld H=%lld)", op, (long long)B, (long long)L,
                          (long long)H);
    return CDSSM_EINVAL;
  }
  if (!q || !k || !v || !beta || !sel_c || !a_bar || !vp || !y || !workspace) {
    cdssm_host::set_error("%s: null pointer argument", op);
    return CDSSM_EINVAL;
  }
  if (!cs_aligned(q, 16) || !cs_aligned(k, 16) || !cs_aligned(a_bar, 8) || !cs_aligned(v, 8) ||
      !cs_aligned(vp, 4) || !cs_aligned(y, 8) || !cs_aligned(workspace, 16)) {
    cdssm_host::set_error("%s: q, k and the workspace must be 16-byte aligned, a_bar, v and y 8-byte, vp 4-byte",
                          op);
    return CDSSM_EINVAL;
  }
  CsArgs a;
  a.q = static_cast<const uint16_t*>(q);
  a.k = static_cast<const uint16_t*>(k);
  a.v = static_cast<const uint16_t*>(v);
  a.beta = static_cast<const uint16_t*>(beta);
  a.sel = static_cast<const uint16_t*>(sel_c);
  a.a = static_cast<const uint16_t*>(a_bar);
  a.vp = static_cast<const uint16_t*>(vp);
  a.scut = shortcut_scale;
  a.yloc = workspace + w.yloc;
  a.st = workspace + w.st;
  a.ap = reinterpret_cast<float2*>(workspace + w.ap);
  a.y = static_cast<uint16_t*>(y);
  a.L = int(L);
  a.H = int(H);
  a.Q = int(chunk);
  a.NC = int(w.NC);
  a.items = items;
  int st = D == 64 ? chunked_launch<64>(a, stream) : chunked_launch<128>(a, stream);
  if (st) return st;
  const int64_t lines = B * H * kCsRows * D;
  hipLaunchKernelGGL(chunked_carry_kernel, dim3(unsigned((lines + 255) / 256)), dim3(256), 0, stream, a.st, a.ap,
                     h0, h_final, lines, int(H), int(w.NC), int(D));
  st = cdssm_host::check_launch("cdssm_chunked_scan_fwd_abar/carry");
  if (st) return st;
  return D == 64 ? chunked_launch_corr<64>(a, stream) : chunked_launch_corr<128>(a, stream);
}
