// Recurrent decode step of the CD-SSM scan: one new token per (b, h), with the
// R-mode state carried between calls, so that generating after a prefill
// needs no re-forward of the sequence.
//
// The reference generates by re-running the whole forward for every new
// token (predict.py:53-67); its outputs are those of the chunked R-mode scan
// (ssd.py:39-111).  The decode step reproduces that scan one token at a time
// (same chunk boundaries, chunk size Q):
//   state entering token t, local index j = t mod Q of chunk k:
//     z     local state of chunk k after token t-1 (z = 0 at j = 0)
//     c^    decay-free correction state, c^_j (c^_0 = s_k)
//     s     s_k, the carry entering chunk k
//     g     g_{j-1} = prod_{u<j} a_u within the chunk (g = 1 at j = 0)
//   step:   z' = a (z - beta (z.k) k) + w k              (intra_chunk_scan.cu:146-167)
//           y  = sel_C ((z' + g c^) . q)                 (ssd.py:102, block.py:208-211;
//                                                         c_j = g_{j-1} c^_j, exact_correction.cu:89-94)
//           c^' = c^ - beta (c^.k) k,  g' = g a
//   chunk end (j = Q - 1): s' = g' s + z' (inter_chunk_scan.cu:73-83); then
//           z = 0, c^ = s', s = s', g = 1.
// g' s + z' is also the R-mode carry after the token (the fused scan's
// h_final for a sequence ending there).
//
// Input forms: T = BF16 / F32 takes the scan-level (dt, r, alpha, omega, c);
// ABar<T> takes the gate-level transition a_t (B, H, 2) in dt's place and the
// VP scale vp_t (B, H) in r's (alpha, omega unused), as the fused scan's
// ABar form (the model's DynamicsFusedFn outputs).
//
// State layout (fp32, caller-owned): state (B, H, 3, 2, D) = rows z_re, z_im,
// c^_re, c^_im, s_re, s_im; gam (B, H, 2) = g; pos (B, H) int32 = j.
// Work layout: one wave per (b, group of HPW heads), LPH lanes per head, each
// lane DPL consecutive state elements (as the fused scan's main pass).
#include "gate_math.hpp"
#include "lm_common.hpp"

namespace cdssm {

template <typename T, int D, int LPH>
__global__ __launch_bounds__(kWave) void decode_step_kernel(
    const typename T::raw* __restrict__ q, const typename T::raw* __restrict__ k,
    const typename T::raw* __restrict__ v, const typename T::raw* __restrict__ beta,
    const typename T::raw* __restrict__ sel_c, const typename T::raw* __restrict__ dt,
    const typename T::raw* __restrict__ r, const float* __restrict__ alpha, const float* __restrict__ omega,
    float c, float* __restrict__ state, float2* __restrict__ gam, int* __restrict__ pos,
    typename T::raw* __restrict__ y, float* __restrict__ h_out, int H, int Q, int n_hg) {
  constexpr int DPL = D / LPH, HPW = kWave / LPH;
  static_assert(DPL % 4 == 0, "state slices are whole float4s");
  const int bi = int(blockIdx.x) / n_hg;
  const int hbase = (int(blockIdx.x) % n_hg) * HPW;
  const int lane = int(threadIdx.x);
  const int hh = lane / LPH, sub = lane % LPH;
  const int h = hbase + hh;
  const bool hok = h < H;
  const int hl = hok ? h : H - 1;
  const int64_t bh = int64_t(bi) * H + hl;  // (b, h); the token is (b, 0, h)

  // per-token scalars and dynamics (every lane of the head computes them)
  const float bb = T::load(beta + bh), sc = T::load(sel_c + bh);
  Transition tr;
  if constexpr (IsABar<T>::value)
    tr = Transition{T::load(dt + 2 * bh), T::load(dt + 2 * bh + 1), T::load(r + bh)};
  else
    tr = cayley_gated(T::load(dt + bh), T::load(r + bh), alpha[hl], omega[hl], c);
  const float wr = bb * tr.vp * T::load(v + 2 * bh), wi = bb * tr.vp * T::load(v + 2 * bh + 1);

  float kk[DPL], qq[DPL];
  {
    RowVec<T, DPL> kv, qv;
    kv.load(k + bh * D + sub * DPL);
    qv.load(q + bh * D + sub * DPL);
    kv.unpack(kk);
    qv.unpack(qq);
  }
  float* st = state + bh * 6 * D + sub * DPL;
  float zr[DPL], zi[DPL], cr[DPL], ci[DPL];
#pragma unroll
  for (int j = 0; j < DPL; j += 4) {
    const float4 a0 = *reinterpret_cast<const float4*>(st + j);
    const float4 a1 = *reinterpret_cast<const float4*>(st + D + j);
    const float4 a2 = *reinterpret_cast<const float4*>(st + 2 * D + j);
    const float4 a3 = *reinterpret_cast<const float4*>(st + 3 * D + j);
    zr[j] = a0.x; zr[j + 1] = a0.y; zr[j + 2] = a0.z; zr[j + 3] = a0.w;
    zi[j] = a1.x; zi[j + 1] = a1.y; zi[j + 2] = a1.z; zi[j + 3] = a1.w;
    cr[j] = a2.x; cr[j + 1] = a2.y; cr[j + 2] = a2.z; cr[j + 3] = a2.w;
    ci[j] = a3.x; ci[j + 1] = a3.y; ci[j + 2] = a3.z; ci[j + 3] = a3.w;
  }
  const float2 g = gam[bh];
  const int jpos = pos[bh];

  // z.k, c^.k, c^.q (c^ before its step: the correction is read before token t)
  float pzr = 0.0f, pzi = 0.0f, pcr = 0.0f, pci = 0.0f, cqr = 0.0f, cqi = 0.0f;
#pragma unroll
  for (int j = 0; j < DPL; ++j) {
    pzr = fmaf(zr[j], kk[j], pzr);
    pzi = fmaf(zi[j], kk[j], pzi);
    pcr = fmaf(cr[j], kk[j], pcr);
    pci = fmaf(ci[j], kk[j], pci);
    cqr = fmaf(cr[j], qq[j], cqr);
    cqi = fmaf(ci[j], qq[j], cqi);
  }
  pzr = group_sum<LPH>(pzr);
  pzi = group_sum<LPH>(pzi);
  pcr = group_sum<LPH>(pcr);
  pci = group_sum<LPH>(pci);
  cqr = group_sum<LPH>(cqr);
  cqi = group_sum<LPH>(cqi);

  // z' = a (z - beta (z.k) k) + w k ; c^' = c^ - beta (c^.k) k ; z'.q
  float zqr = 0.0f, zqi = 0.0f;
#pragma unroll
  for (int j = 0; j < DPL; ++j) {
    const float ur = fmaf(-bb * pzr, kk[j], zr[j]);
    const float ui = fmaf(-bb * pzi, kk[j], zi[j]);
    zr[j] = fmaf(tr.ar, ur, fmaf(-tr.ai, ui, wr * kk[j]));
    zi[j] = fmaf(tr.ar, ui, fmaf(tr.ai, ur, wi * kk[j]));
    cr[j] = fmaf(-bb * pcr, kk[j], cr[j]);
    ci[j] = fmaf(-bb * pci, kk[j], ci[j]);
    zqr = fmaf(zr[j], qq[j], zqr);
    zqi = fmaf(zi[j], qq[j], zqi);
  }
  zqr = group_sum<LPH>(zqr);
  zqi = group_sum<LPH>(zqi);
  const float yr = sc * (zqr + (g.x * cqr - g.y * cqi));
  const float yi = sc * (zqi + (g.x * cqi + g.y * cqr));
  const float2 gn = make_float2(g.x * tr.ar - g.y * tr.ai, g.x * tr.ai + g.y * tr.ar);

  if (!hok) return;  // nothing below reduces across lanes
  if (sub == 0) {
    T::store(y + 2 * bh, yr);
    T::store(y + 2 * bh + 1, yi);
  }
  // carry after the token: g' s + z' (also the next chunk's start at a chunk end)
  const bool chunk_end = jpos + 1 >= Q;
  if (chunk_end || h_out) {
    float sr[DPL], si[DPL];
#pragma unroll
    for (int j = 0; j < DPL; j += 4) {
      const float4 a4 = *reinterpret_cast<const float4*>(st + 4 * D + j);
      const float4 a5 = *reinterpret_cast<const float4*>(st + 5 * D + j);
      sr[j] = a4.x; sr[j + 1] = a4.y; sr[j + 2] = a4.z; sr[j + 3] = a4.w;
      si[j] = a5.x; si[j + 1] = a5.y; si[j + 2] = a5.z; si[j + 3] = a5.w;
    }
#pragma unroll
    for (int j = 0; j < DPL; ++j) {
      const float nr = fmaf(gn.x, sr[j], fmaf(-gn.y, si[j], zr[j]));
      si[j] = fmaf(gn.x, si[j], fmaf(gn.y, sr[j], zi[j]));
      sr[j] = nr;
    }
    if (h_out) {
      float* ho = h_out + bh * 2 * D + sub * DPL;
#pragma unroll
      for (int j = 0; j < DPL; j += 4) {
        *reinterpret_cast<float4*>(ho + j) = make_float4(sr[j], sr[j + 1], sr[j + 2], sr[j + 3]);
        *reinterpret_cast<float4*>(ho + D + j) = make_float4(si[j], si[j + 1], si[j + 2], si[j + 3]);
      }
    }
    if (chunk_end) {
      // next chunk: z = 0, c^ = s = s', g = 1
#pragma unroll
      for (int j = 0; j < DPL; ++j) {
        zr[j] = zi[j] = 0.0f;
        cr[j] = sr[j];
        ci[j] = si[j];
      }
#pragma unroll
      for (int j = 0; j < DPL; j += 4) {
        *reinterpret_cast<float4*>(st + 4 * D + j) = make_float4(sr[j], sr[j + 1], sr[j + 2], sr[j + 3]);
        *reinterpret_cast<float4*>(st + 5 * D + j) = make_float4(si[j], si[j + 1], si[j + 2], si[j + 3]);
      }
    }
  }
#pragma unroll
  for (int j = 0; j < DPL; j += 4) {
    *reinterpret_cast<float4*>(st + j) = make_float4(zr[j], zr[j + 1], zr[j + 2], zr[j + 3]);
    *reinterpret_cast<float4*>(st + D + j) = make_float4(zi[j], zi[j + 1], zi[j + 2], zi[j + 3]);
    *reinterpret_cast<float4*>(st + 2 * D + j) = make_float4(cr[j], cr[j + 1], cr[j + 2], cr[j + 3]);
    *reinterpret_cast<float4*>(st + 3 * D + j) = make_float4(ci[j], ci[j + 1], ci[j + 2], ci[j + 3]);
  }
  if (sub == 0) {
    gam[bh] = chunk_end ? make_float2(1.0f, 0.0f) : gn;
    pos[bh] = chunk_end ? 0 : jpos + 1;
  }
}

// ---------------------------------------------------------------------------
// One decode token of the model block's scan path in one launch (the step
// forms of block.py:169-211 between the projections): per (b, h)
//   dynamics  A_bar, vp, beta, sel_C from the gate row at the device-held
//             position (gate_math.hpp, as cdssm_dynamics_fused_fwd_at)
//   K, Q      x * rsqrt(sum x^2 + 1e-6) and q.k (as cdssm_normalize_kq_qk_fwd)
//   V         the in_proj V, or lerp(v_first, V, sigmoid(v_residual_gate))
//   scan      the decode step on (A_bar, vp) (as cdssm_decode_step_abar)
//   shortcut  retrieved += scale (q.k)^2 sel_C vp V (as cdssm_shortcut_readout_fwd)
// with every intermediate rounded to the element type where the separate
// kernels store it, so the outputs equal theirs.  Inputs are read in place:
// gq (B, GH + H D) = [gate row | Q] (the stacked gate_proj / Q_proj GEMM) and
// proj (B, P) with K at column k_off and V at column v_off (the in_proj
// output).  Outputs: retrieved (B, H, 2) and V (B, H, 2) (layer 0's V is
// v_first of the later layers).  Work layout as decode_step_kernel.
// ---------------------------------------------------------------------------
struct DecodeTokenArgs {
  int64_t gq_stride, proj_stride;
  int k_off, v_off;
  const float* lds;        // (H) fp32 log_dt_scale
  const float* rope;       // (H) fp32
  gates::GateConsts kc;
  const int64_t* l_dev;    // the token's position
  const float* scale;      // shortcut_scale, one fp32
  int H, Q, n_hg;
};

template <typename T>
__device__ __forceinline__ float round_to(float x) {
  if constexpr (T::bytes == 2)
    return bf16_to_f32(f32_to_bf16(x));
  else
    return x;
}

// The token step of one wave: batch row bi, heads hbase .. hbase + HPW - 1,
// lane the lane in the wave.  The retrieved pair of each head goes to ret
// (B, H, 2) or, with rs, to rs[2 h], rs[2 h + 1] (LDS; rounded as ret stores it).
template <typename T, int D, int LPH>
__device__ __forceinline__ void decode_token_wave(
    int bi, int hbase, int lane, const typename T::raw* __restrict__ gq, const typename T::raw* __restrict__ proj,
    const typename T::raw* __restrict__ v_first, const typename T::raw* __restrict__ vgate,
    float* __restrict__ state, float2* __restrict__ gam, int* __restrict__ pos, typename T::raw* __restrict__ ret,
    float* rs, typename T::raw* __restrict__ v_out, const DecodeTokenArgs& a) {
  constexpr int DPL = D / LPH, N = 2;
  static_assert(DPL % 4 == 0, "state slices are whole float4s");
  const int H = a.H;
  const int hh = lane / LPH, sub = lane % LPH;
  const int h = hbase + hh;
  const bool hok = h < H;
  const int hl = hok ? h : H - 1;
  const int64_t bh = int64_t(bi) * H + hl;
  const typename T::raw* grow = gq + int64_t(bi) * a.gq_stride;
  const typename T::raw* prow = proj + int64_t(bi) * a.proj_stride;

  // dynamics at the token's position, rounded as DynamicsFusedFn stores them
  const float pp = float(*a.l_dev) * a.rope[hl];
  const gates::GateToken gt = gates::gate_token<T>(grow + hl, H, N, a.lds[hl], pp, a.kc);
  const Transition tr0 = gates::gate_pair<T>(grow + hl, H, N, 0, pp, gt, a.kc);
  const Transition tr{round_to<T>(tr0.ar), round_to<T>(tr0.ai), round_to<T>(tr0.vp)};
  const float bb = round_to<T>(gt.beta), sc = round_to<T>(gt.selc);

  // V (B, H, 2): the in_proj's, or the value-residual lerp with layer 0's
  float v0 = T::load(prow + a.v_off + 2 * hl), v1 = T::load(prow + a.v_off + 2 * hl + 1);
  if (v_first) {
    // torch.lerp(start, end, w): start + w (end - start) for w < 0.5, else end - (end - start)(1 - w)
    const float w = T::load(vgate + hl);
    const float s0 = T::load(v_first + 2 * bh), s1 = T::load(v_first + 2 * bh + 1);
    v0 = round_to<T>(w < 0.5f ? fmaf(w, v0 - s0, s0) : v0 - (v0 - s0) * (1.0f - w));
    v1 = round_to<T>(w < 0.5f ? fmaf(w, v1 - s1, s1) : v1 - (v1 - s1) * (1.0f - w));
  }
  const float wr = bb * tr.vp * v0, wi = bb * tr.vp * v1;

  // K, Q normalised (the same lane split and summation order as normalize_qk_kernel)
  float kk[DPL], qq[DPL];
  {
    RowVec<T, DPL> kv, qv;
    kv.load(prow + a.k_off + hl * D + sub * DPL);
    qv.load(grow + (N + 5) * H + hl * D + sub * DPL);
    kv.unpack(kk);
    qv.unpack(qq);
  }
  float sk = 0.0f, sq = 0.0f;
#pragma unroll
  for (int j = 0; j < DPL; ++j) {
    sk = fmaf(kk[j], kk[j], sk);
    sq = fmaf(qq[j], qq[j], sq);
  }
  sk = group_sum<LPH>(sk);
  sq = group_sum<LPH>(sq);
  const float ik = rsqrtf(sk + 1e-6f), iq = rsqrtf(sq + 1e-6f);
  float qkd = 0.0f;
#pragma unroll
  for (int j = 0; j < DPL; ++j) {
    kk[j] = round_to<T>(kk[j] * ik);
    qq[j] = round_to<T>(qq[j] * iq);
    qkd = fmaf(kk[j], qq[j], qkd);
  }
  qkd = group_sum<LPH>(qkd);

  // the scan's decode step (decode_step_kernel's arithmetic)
  float* st = state + bh * 6 * D + sub * DPL;
  float zr[DPL], zi[DPL], cr[DPL], ci[DPL];
#pragma unroll
  for (int j = 0; j < DPL; j += 4) {
    const float4 a0 = *reinterpret_cast<const float4*>(st + j);
    const float4 a1 = *reinterpret_cast<const float4*>(st + D + j);
    const float4 a2 = *reinterpret_cast<const float4*>(st + 2 * D + j);
    const float4 a3 = *reinterpret_cast<const float4*>(st + 3 * D + j);
    zr[j] = a0.x; zr[j + 1] = a0.y; zr[j + 2] = a0.z; zr[j + 3] = a0.w;
    zi[j] = a1.x; zi[j + 1] = a1.y; zi[j + 2] = a1.z; zi[j + 3] = a1.w;
    cr[j] = a2.x; cr[j + 1] = a2.y; cr[j + 2] = a2.z; cr[j + 3] = a2.w;
    ci[j] = a3.x; ci[j + 1] = a3.y; ci[j + 2] = a3.z; ci[j + 3] = a3.w;
  }
  const float2 g = gam[bh];
  const int jpos = pos[bh];
  float pzr = 0.0f, pzi = 0.0f, pcr = 0.0f, pci = 0.0f, cqr = 0.0f, cqi = 0.0f;
#pragma unroll
  for (int j = 0; j < DPL; ++j) {
    pzr = fmaf(zr[j], kk[j], pzr);
    pzi = fmaf(zi[j], kk[j], pzi);
    pcr = fmaf(cr[j], kk[j], pcr);
    pci = fmaf(ci[j], kk[j], pci);
    cqr = fmaf(cr[j], qq[j], cqr);
    cqi = fmaf(ci[j], qq[j], cqi);
  }
  pzr = group_sum<LPH>(pzr);
  pzi = group_sum<LPH>(pzi);
  pcr = group_sum<LPH>(pcr);
  pci = group_sum<LPH>(pci);
  cqr = group_sum<LPH>(cqr);
  cqi = group_sum<LPH>(cqi);
  float zqr = 0.0f, zqi = 0.0f;
#pragma unroll
  for (int j = 0; j < DPL; ++j) {
    const float ur = fmaf(-bb * pzr, kk[j], zr[j]);
    const float ui = fmaf(-bb * pzi, kk[j], zi[j]);
    zr[j] = fmaf(tr.ar, ur, fmaf(-tr.ai, ui, wr * kk[j]));
    zi[j] = fmaf(tr.ar, ui, fmaf(tr.ai, ur, wi * kk[j]));
    cr[j] = fmaf(-bb * pcr, kk[j], cr[j]);
    ci[j] = fmaf(-bb * pci, kk[j], ci[j]);
    zqr = fmaf(zr[j], qq[j], zqr);
    zqi = fmaf(zi[j], qq[j], zqi);
  }
  zqr = group_sum<LPH>(zqr);
  zqi = group_sum<LPH>(zqi);
  const float yr = round_to<T>(sc * (zqr + (g.x * cqr - g.y * cqi)));
  const float yi = round_to<T>(sc * (zqi + (g.x * cqi + g.y * cqr)));
  const float2 gn = make_float2(g.x * tr.ar - g.y * tr.ai, g.x * tr.ai + g.y * tr.ar);

  if (!hok) return;  // nothing below reduces across lanes
  if (sub == 0) {
    // the shortcut through the readout (shortcut_kernel's arithmetic)
    const float c = a.scale[0] * qkd * qkd * sc * tr.vp;
    if (rs) {
      rs[2 * hl] = round_to<T>(yr + c * v0);
      rs[2 * hl + 1] = round_to<T>(yi + c * v1);
    } else {
      T::store(ret + 2 * bh, yr + c * v0);
      T::store(ret + 2 * bh + 1, yi + c * v1);
    }
    T::store(v_out + 2 * bh, v0);
    T::store(v_out + 2 * bh + 1, v1);
  }
  const bool chunk_end = jpos + 1 >= a.Q;
  if (chunk_end) {
    float sr[DPL], si[DPL];
#pragma unroll
    for (int j = 0; j < DPL; j += 4) {
      const float4 a4 = *reinterpret_cast<const float4*>(st + 4 * D + j);
      const float4 a5 = *reinterpret_cast<const float4*>(st + 5 * D + j);
      sr[j] = a4.x; sr[j + 1] = a4.y; sr[j + 2] = a4.z; sr[j + 3] = a4.w;
      si[j] = a5.x; si[j + 1] = a5.y; si[j + 2] = a5.z; si[j + 3] = a5.w;
    }
#pragma unroll
    for (int j = 0; j < DPL; ++j) {
      const float nr = fmaf(gn.x, sr[j], fmaf(-gn.y, si[j], zr[j]));
      si[j] = fmaf(gn.x, si[j], fmaf(gn.y, sr[j], zi[j]));
      sr[j] = nr;
      zr[j] = zi[j] = 0.0f;
      cr[j] = sr[j];
      ci[j] = si[j];
    }
#pragma unroll
    for (int j = 0; j < DPL; j += 4) {
      *reinterpret_cast<float4*>(st + 4 * D + j) = make_float4(sr[j], sr[j + 1], sr[j + 2], sr[j + 3]);
      *reinterpret_cast<float4*>(st + 5 * D + j) = make_float4(si[j], si[j + 1], si[j + 2], si[j + 3]);
    }
  }
#pragma unroll
  for (int j = 0; j < DPL; j += 4) {
    *reinterpret_cast<float4*>(st + j) = make_float4(zr[j], zr[j + 1], zr[j + 2], zr[j + 3]);
    *reinterpret_cast<float4*>(st + D + j) = make_float4(zi[j], zi[j + 1], zi[j + 2], zi[j + 3]);
    *reinterpret_cast<float4*>(st + 2 * D + j) = make_float4(cr[j], cr[j + 1], cr[j + 2], cr[j + 3]);
    *reinterpret_cast<float4*>(st + 3 * D + j) = make_float4(ci[j], ci[j + 1], ci[j + 2], ci[j + 3]);
  }
  if (sub == 0) {
    gam[bh] = chunk_end ? make_float2(1.0f, 0.0f) : gn;
    pos[bh] = chunk_end ? 0 : jpos + 1;
  }
}

template <typename T, int D, int LPH>
__global__ __launch_bounds__(kWave) void decode_token_kernel(
    const typename T::raw* __restrict__ gq, const typename T::raw* __restrict__ proj,
    const typename T::raw* __restrict__ v_first, const typename T::raw* __restrict__ vgate,
    float* __restrict__ state, float2* __restrict__ gam, int* __restrict__ pos, typename T::raw* __restrict__ ret,
    typename T::raw* __restrict__ v_out, DecodeTokenArgs a) {
  constexpr int HPW = kWave / LPH;
  decode_token_wave<T, D, LPH>(int(blockIdx.x) / a.n_hg, (int(blockIdx.x) % a.n_hg) * HPW, int(threadIdx.x), gq,
                               proj, v_first, vgate, state, gam, pos, ret, nullptr, v_out, a);
}

// The block's decode tail in one launch (block.py:169-225 after the gate / Q
// projection): one workgroup per batch row, a wave per group of HPW heads
// running decode_token_wave into LDS, then the row's readout projection and
// GroupNorm + gate step (lm::gn_row_step).  position[0] is the layer's decode
// position and position[1] an arrival count: every workgroup arrives once it
// has read the position, and the last to arrive advances it and clears the
// count (so the next launch, and a replayed graph, find it zero).
struct DecodeTailArgs {
  const void* wr;  // readout_proj weight (C, 2 H)
  float4* gsum;    // (B, G, 4) running GroupNorm sums
  const void *gamma, *beta, *z, *xc, *Dp;
  void* out;       // (B, C)
  int64_t z_bs;
  int C, G;
  float eps;
  unsigned long long* arrive;  // position + 1
};

template <typename T, int D, int LPH, typename P>
__global__ __launch_bounds__(1024) void decode_tail_kernel(
    const typename T::raw* __restrict__ gq, const typename T::raw* __restrict__ proj,
    const typename T::raw* __restrict__ v_first, const typename T::raw* __restrict__ vgate,
    float* __restrict__ state, float2* __restrict__ gam, int* __restrict__ pos, typename T::raw* __restrict__ v_out,
    DecodeTokenArgs a, DecodeTailArgs t) {
  using raw = typename T::raw;
  constexpr int HPW = kWave / LPH;
  extern __shared__ float tail_lds[];
  const int kr = 2 * a.H;
  float* rs = tail_lds;                                                  // the row's retrieved values (kr)
  float2* gst = reinterpret_cast<float2*>(tail_lds + ((kr + 1) & ~1));  // (mean, rstd) per group
  float* ys = reinterpret_cast<float*>(gst + t.G);                       // the row's y (C)
  const int bi = int(blockIdx.x);
  const int wv = int(threadIdx.x) / kWave;
  // the first n_hg waves run the token step; the whole workgroup (at least 8 waves) the epilogue
  if (wv < a.n_hg)
    decode_token_wave<T, D, LPH>(bi, wv * HPW, int(threadIdx.x) % kWave, gq, proj, v_first, vgate, state, gam, pos,
                                 nullptr, rs, v_out, a);
  __syncthreads();  // every wave has read the position and written its heads' retrieved values
  if (threadIdx.x == 0) {
    const unsigned long long n = __hip_atomic_fetch_add(t.arrive, 1ull, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT);
    if (n + 1 == gridDim.x) {
      __hip_atomic_store(t.arrive, 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      int64_t* position = const_cast<int64_t*>(a.l_dev);
      position[0] += 1;
    }
  }
  lm::gn_row_step<T, P>(bi, nullptr, rs, static_cast<const raw*>(t.wr), kr, t.gsum,
                        static_cast<const typename P::raw*>(t.gamma), static_cast<const typename P::raw*>(t.beta),
                        static_cast<const raw*>(t.z), t.z_bs, static_cast<const raw*>(t.xc),
                        static_cast<const raw*>(t.Dp), static_cast<raw*>(t.out), t.C, t.G, t.eps, gst, ys);
}

// state = (0, h, h) per (b, h) (h = 0 if null), g = 1, j = 0: the decode state
// at a chunk boundary with carry h (the fused scan's h_final there).
__global__ __launch_bounds__(256) void decode_init_kernel(const float* __restrict__ h, float* __restrict__ state,
                                                          float2* __restrict__ gam, int* __restrict__ pos,
                                                          int64_t BH, int D) {
  const int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;  // (b, h, element of 2D)
  if (i >= BH * 2 * D) return;
  const int64_t bh = i / (2 * D);
  const int e = int(i % (2 * D));  // row re (e < D) or im, element e % D
  const float hv = h ? h[i] : 0.0f;
  float* st = state + bh * 6 * D;
  st[e] = 0.0f;          // z
  st[2 * D + e] = hv;    // c^
  st[4 * D + e] = hv;    // s
  if (e == 0) {
    gam[bh] = make_float2(1.0f, 0.0f);
    pos[bh] = 0;
  }
}

template <typename T, int D, int LPH>
int launch_decode(const void* q, const void* k, const void* v, const void* beta, const void* sel_c,
                  const void* dt, const void* r, const float* alpha, const float* omega, float c, float* state,
                  float* gam, int* pos, void* y, float* h_out, int B, int H, int Q, hipStream_t stream) {
  using raw = typename T::raw;
  constexpr int HPW = kWave / LPH;
  const int n_hg = (H + HPW - 1) / HPW;
  hipLaunchKernelGGL((decode_step_kernel<T, D, LPH>), dim3(unsigned(int64_t(B) * n_hg)), dim3(kWave), 0, stream,
                     static_cast<const raw*>(q), static_cast<const raw*>(k), static_cast<const raw*>(v),
                     static_cast<const raw*>(beta), static_cast<const raw*>(sel_c), static_cast<const raw*>(dt),
                     static_cast<const raw*>(r), alpha, omega, c, state, reinterpret_cast<float2*>(gam), pos,
                     static_cast<raw*>(y), h_out, H, Q, n_hg);
  return cdssm_host::check_launch("cdssm_decode_step");
}

}  // namespace cdssm

using namespace cdssm;

extern "C" int cdssm_decode_init(const float* h, float* state, float* gam, int* pos, int64_t B, int64_t H,
                                 int64_t D, int64_t N, hipStream_t stream) {
  const char* op = "cdssm_decode_init";
  if (B <= 0 || H <= 0 || B * H > 0x7fffffffLL || N != 2 || (D != 64 && D != 128)) {
    cdssm_host::set_error("%s: need B, H > 0, N = 2, D in {64, 128} (B=%lld H=%lld D=%lld N=%lld)", op,
                          (long long)B, (long long)H, (long long)D, (long long)N);
    return CDSSM_EINVAL;
  }
  if (!state || !gam || !pos) {
    cdssm_host::set_error("%s: null pointer argument", op);
    return CDSSM_EINVAL;
  }
  const int64_t n = B * H * 2 * D;
  hipLaunchKernelGGL(decode_init_kernel, dim3(unsigned((n + 255) / 256)), dim3(256), 0, stream, h, state,
                     reinterpret_cast<float2*>(gam), pos, B * H, int(D));
  return cdssm_host::check_launch(op);
}

namespace {

template <bool ABAR>
int decode_entry(const char* op, int dtype, const void* q, const void* k, const void* v, const void* beta,
                 const void* sel_c, const void* dt, const void* r, const float* alpha, const float* omega, float c,
                 float* state, float* gam, int* pos, void* y, float* h_out, int64_t B, int64_t H, int64_t D,
                 int64_t N, int64_t chunk, hipStream_t stream) {
  if (dtype != 0 && dtype != 1) {
    cdssm_host::set_error("%s: dtype must be 0 (fp32) or 1 (bf16), got %d", op, dtype);
    return CDSSM_EINVAL;
  }
  if (B <= 0 || H <= 0 || B * H > 0x7fffffffLL || N != 2 || (D != 64 && D != 128) || chunk < 1 ||
      chunk > 128) {
    cdssm_host::set_error("%s: need B, H > 0, N = 2, D in {64, 128}, 1 <= chunk <= 128 "
                          "(B=%lld H=%lld D=%lld N=%lld chunk=%lld)",
                          op, (long long)B, (long long)H, (long long)D, (long long)N, (long long)chunk);
    return CDSSM_EINVAL;
  }
  if (!q || !k || !v || !beta || !sel_c || !dt || !r || (!ABAR && (!alpha || !omega)) || !state || !gam || !pos ||
      !y) {
    cdssm_host::set_error("%s: null pointer argument", op);
    return CDSSM_EINVAL;
  }
  const int b = int(B), hh = int(H), qc = int(chunk);
  using TB = std::conditional_t<ABAR, ABar<BF16>, BF16>;
  using TF = std::conditional_t<ABAR, ABar<F32>, F32>;
  if (dtype == 1) {
    if (D == 64)
      return launch_decode<TB, 64, 8>(q, k, v, beta, sel_c, dt, r, alpha, omega, c, state, gam, pos, y, h_out, b, hh,
                                      qc, stream);
    return launch_decode<TB, 128, 16>(q, k, v, beta, sel_c, dt, r, alpha, omega, c, state, gam, pos, y, h_out, b, hh,
                                      qc, stream);
  }
  if (D == 64)
    return launch_decode<TF, 64, 16>(q, k, v, beta, sel_c, dt, r, alpha, omega, c, state, gam, pos, y, h_out, b, hh,
                                     qc, stream);
  return launch_decode<TF, 128, 32>(q, k, v, beta, sel_c, dt, r, alpha, omega, c, state, gam, pos, y, h_out, b, hh,
                                    qc, stream);
}

}  // namespace

extern "C" int cdssm_decode_step(int dtype, const void* q, const void* k, const void* v, const void* beta,
                                 const void* sel_c, const void* dt, const void* r, const float* alpha,
                                 const float* omega, float c, float* state, float* gam, int* pos, void* y,
                                 float* h_out, int64_t B, int64_t H, int64_t D, int64_t N, int64_t chunk,
                                 hipStream_t stream) {
  return decode_entry<false>("cdssm_decode_step", dtype, q, k, v, beta, sel_c, dt, r, alpha, omega, c, state, gam,
                             pos, y, h_out, B, H, D, N, chunk, stream);
}

extern "C" int cdssm_decode_step_abar(int dtype, const void* q, const void* k, const void* v, const void* beta,
                                      const void* sel_c, const void* a_bar, const void* vp, float* state, float* gam,
                                      int* pos, void* y, float* h_out, int64_t B, int64_t H, int64_t D, int64_t N,
                                      int64_t chunk, hipStream_t stream) {
  return decode_entry<true>("cdssm_decode_step_abar", dtype, q, k, v, beta, sel_c, a_bar, vp, nullptr, nullptr,
                            0.0f, state, gam, pos, y, h_out, B, H, D, N, chunk, stream);
}

extern "C" int cdssm_decode_block_token(int dtype, const void* gq, int64_t gq_stride, const void* proj,
                                        int64_t proj_stride, int64_t k_off, int64_t v_off, const void* v_first,
                                        const void* vgate, const float* log_dt_scale, const float* rope_freqs,
                                        float gating_c, float omega_thresh, float adt_delta, float adt_smoothness,
                                        float adt_eps, const int64_t* position, const float* shortcut_scale,
                                        float* state, float* gam, int* pos, void* retrieved, void* v_out, int64_t B,
                                        int64_t H, int64_t D, int64_t N, int64_t chunk, hipStream_t stream) {
  const char* op = "cdssm_decode_block_token";
  if (dtype != 0 && dtype != 1) {
    cdssm_host::set_error("%s: dtype must be 0 (fp32) or 1 (bf16), got %d", op, dtype);
    return CDSSM_EINVAL;
  }
  if (B <= 0 || H <= 0 || B * H > 0x7fffffffLL || N != 2 || (D != 64 && D != 128) || chunk < 1 || chunk > 128 ||
      gq_stride < 7 * H + H * D || k_off < 0 || v_off < 0 || proj_stride < k_off + H * D ||
      proj_stride < v_off + 2 * H || proj_stride > (int64_t(1) << 40) || gq_stride > (int64_t(1) << 40)) {
    cdssm_host::set_error("%s: need B, H > 0, N = 2, D in {64, 128}, 1 <= chunk <= 128 and the gate / Q and "
                          "K / V columns inside their rows (B=%lld H=%lld D=%lld N=%lld chunk=%lld)",
                          op, (long long)B, (long long)H, (long long)D, (long long)N, (long long)chunk);
    return CDSSM_EINVAL;
  }
  if (!gq || !proj || (v_first && !vgate) || !log_dt_scale || !rope_freqs || !position || !shortcut_scale ||
      !state || !gam || !pos || !retrieved || !v_out) {
    cdssm_host::set_error("%s: null pointer argument", op);
    return CDSSM_EINVAL;
  }
  if (!(adt_smoothness != 0.0f)) {
    cdssm_host::set_error("%s: adt_smoothness must be nonzero", op);
    return CDSSM_EINVAL;
  }
  const int64_t eb = dtype == 1 ? 2 : 4;
  const int64_t qcol = 7 * H;  // Q's first column in gq
  if ((reinterpret_cast<uintptr_t>(gq) + qcol * eb) % 16 || (gq_stride * eb) % 16 ||
      (reinterpret_cast<uintptr_t>(proj) + k_off * eb) % 16 || (proj_stride * eb) % 16) {
    cdssm_host::set_error("%s: the Q and K rows must start 16-byte aligned", op);
    return CDSSM_EINVAL;
  }
  DecodeTokenArgs a;
  a.gq_stride = gq_stride;
  a.proj_stride = proj_stride;
  a.k_off = int(k_off);
  a.v_off = int(v_off);
  a.lds = log_dt_scale;
  a.rope = rope_freqs;
  a.kc = gates::GateConsts{gating_c, omega_thresh, adt_delta, adt_smoothness, adt_eps};
  a.l_dev = position;
  a.scale = shortcut_scale;
  a.H = int(H);
  a.Q = int(chunk);
  auto go = [&](auto tt, auto dc, auto lc) {
    using T = decltype(tt);
    using raw = typename T::raw;
    constexpr int DD = decltype(dc)::value, LP = decltype(lc)::value, HPW = kWave / LP;
    a.n_hg = int((H + HPW - 1) / HPW);
    hipLaunchKernelGGL((decode_token_kernel<T, DD, LP>), dim3(unsigned(B * a.n_hg)), dim3(kWave), 0, stream,
                       static_cast<const raw*>(gq), static_cast<const raw*>(proj), static_cast<const raw*>(v_first),
                       static_cast<const raw*>(vgate), state, reinterpret_cast<float2*>(gam), pos,
                       static_cast<raw*>(retrieved), static_cast<raw*>(v_out), a);
  };
  using I = std::integral_constant<int, 64>;
  using J = std::integral_constant<int, 128>;
  if (dtype == 1) {
    if (D == 64)
      go(BF16{}, I{}, std::integral_constant<int, 8>{});
    else
      go(BF16{}, J{}, std::integral_constant<int, 16>{});
  } else {
    if (D == 64)
      go(F32{}, I{}, std::integral_constant<int, 16>{});
    else
      go(F32{}, J{}, std::integral_constant<int, 32>{});
  }
  return cdssm_host::check_launch(op);
}

extern "C" int cdssm_decode_block_tail(int dtype, int param_dtype, const void* gq, int64_t gq_stride,
                                       const void* proj, int64_t proj_stride, int64_t k_off, int64_t v_off,
                                       const void* v_first, const void* vgate, const float* log_dt_scale,
                                       const float* rope_freqs, float gating_c, float omega_thresh, float adt_delta,
                                       float adt_smoothness, float adt_eps, int64_t* position,
                                       const float* shortcut_scale, float* state, float* gam, int* pos, void* v_out,
                                       const void* readout_weight, float* gsum, const void* gamma, const void* beta,
                                       const void* z, int64_t z_batch_stride, const void* x_conv, const void* Dp,
                                       void* out, int64_t B, int64_t H, int64_t D, int64_t N, int64_t chunk,
                                       int64_t C, int64_t G, float eps, hipStream_t stream) {
  const char* op = "cdssm_decode_block_tail";
  if (dtype != 0 && dtype != 1) {
    cdssm_host::set_error("%s: dtype must be 0 (fp32) or 1 (bf16), got %d", op, dtype);
    return CDSSM_EINVAL;
  }
  if (param_dtype != 0 && param_dtype != 1) {
    cdssm_host::set_error("%s: param_dtype must be 0 (fp32) or 1 (bf16), got %d", op, param_dtype);
    return CDSSM_EINVAL;
  }
  if (B <= 0 || H <= 0 || B > 0x7fffffffLL || N != 2 || (D != 64 && D != 128) || chunk < 1 || chunk > 128 ||
      gq_stride < 7 * H + H * D || k_off < 0 || v_off < 0 || proj_stride < k_off + H * D ||
      proj_stride < v_off + 2 * H || proj_stride > (int64_t(1) << 40) || gq_stride > (int64_t(1) << 40)) {
    cdssm_host::set_error("%s: need B, H > 0, N = 2, D in {64, 128}, 1 <= chunk <= 128 and the gate / Q and "
                          "K / V columns inside their rows (B=%lld H=%lld D=%lld N=%lld chunk=%lld)",
                          op, (long long)B, (long long)H, (long long)D, (long long)N, (long long)chunk);
    return CDSSM_EINVAL;
  }
  const int64_t lph = D == 64 ? (dtype == 1 ? 8 : 16) : (dtype == 1 ? 16 : 32);
  const int64_t waves = (H + kWave / lph - 1) / (kWave / lph);
  if (waves > 16 || C <= 0 || G <= 0 || C % G != 0 || G > 8192 || C >= (int64_t(1) << 24) || z_batch_stride < C ||
      ((2 * H + 1) / 2 * 2 + 2 * G + C) * int64_t(sizeof(float)) > 65536) {
    cdssm_host::set_error("%s: need at most 16 head groups, C divisible by G <= 8192, a z row stride >= C and "
                          "2 H + 2 G + C <= 16384 (H=%lld C=%lld G=%lld)", op, (long long)H, (long long)C,
                          (long long)G);
    return CDSSM_EINVAL;
  }
  if (!gq || !proj || (v_first && !vgate) || !log_dt_scale || !rope_freqs || !position || !shortcut_scale ||
      !state || !gam || !pos || !v_out || !readout_weight || !gsum || !gamma || !beta || !z || !x_conv || !Dp ||
      !out) {
    cdssm_host::set_error("%s: null pointer argument", op);
    return CDSSM_EINVAL;
  }
  if (!(adt_smoothness != 0.0f)) {
    cdssm_host::set_error("%s: adt_smoothness must be nonzero", op);
    return CDSSM_EINVAL;
  }
  const int64_t eb = dtype == 1 ? 2 : 4;
  const int64_t qcol = 7 * H;  // Q's first column in gq
  if ((reinterpret_cast<uintptr_t>(gq) + qcol * eb) % 16 || (gq_stride * eb) % 16 ||
      (reinterpret_cast<uintptr_t>(proj) + k_off * eb) % 16 || (proj_stride * eb) % 16 ||
      reinterpret_cast<uintptr_t>(position) % 8) {
    cdssm_host::set_error("%s: the Q and K rows must start 16-byte aligned", op);
    return CDSSM_EINVAL;
  }
  DecodeTokenArgs a;
  a.gq_stride = gq_stride;
  a.proj_stride = proj_stride;
  a.k_off = int(k_off);
  a.v_off = int(v_off);
  a.lds = log_dt_scale;
  a.rope = rope_freqs;
  a.kc = gates::GateConsts{gating_c, omega_thresh, adt_delta, adt_smoothness, adt_eps};
  a.l_dev = position;
  a.scale = shortcut_scale;
  a.H = int(H);
  a.Q = int(chunk);
  DecodeTailArgs t;
  t.wr = readout_weight;
  t.gsum = reinterpret_cast<float4*>(gsum);
  t.gamma = gamma;
  t.beta = beta;
  t.z = z;
  t.xc = x_conv;
  t.Dp = Dp;
  t.out = out;
  t.z_bs = z_batch_stride;
  t.C = int(C);
  t.G = int(G);
  t.eps = eps;
  t.arrive = reinterpret_cast<unsigned long long*>(position + 1);
  const size_t lds = size_t((2 * H + 1) / 2 * 2 + 2 * G + C) * sizeof(float);
  auto go = [&](auto tt, auto pt, auto dc, auto lc) {
    using T = decltype(tt);
    using P = decltype(pt);
    using raw = typename T::raw;
    constexpr int DD = decltype(dc)::value, LP = decltype(lc)::value, HPW = kWave / LP;
    a.n_hg = int((H + HPW - 1) / HPW);
    const unsigned threads = unsigned(kWave * std::max(a.n_hg, 8));
    hipLaunchKernelGGL((decode_tail_kernel<T, DD, LP, P>), dim3(unsigned(B)), dim3(threads), lds,
                       stream, static_cast<const raw*>(gq), static_cast<const raw*>(proj),
                       static_cast<const raw*>(v_first), static_cast<const raw*>(vgate), state,
                       reinterpret_cast<float2*>(gam), pos, static_cast<raw*>(v_out), a, t);
  };
  using I = std::integral_constant<int, 64>;
  using J = std::integral_constant<int, 128>;
  using L8 = std::integral_constant<int, 8>;
  using L16 = std::integral_constant<int, 16>;
  using L32 = std::integral_constant<int, 32>;
  if (dtype == 1) {
    if (D == 64)
      param_dtype == 1 ? go(BF16{}, BF16{}, I{}, L8{}) : go(BF16{}, F32{}, I{}, L8{});
    else
      param_dtype == 1 ? go(BF16{}, BF16{}, J{}, L16{}) : go(BF16{}, F32{}, J{}, L16{});
  } else {
    if (D == 64)
      param_dtype == 1 ? go(F32{}, BF16{}, I{}, L16{}) : go(F32{}, F32{}, I{}, L16{});
    else
      param_dtype == 1 ? go(F32{}, BF16{}, J{}, L32{}) : go(F32{}, F32{}, J{}, L32{});
  }
  return cdssm_host::check_launch(op);
}
