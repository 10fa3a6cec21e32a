// Per-token gate-level dynamics (dynamics_fused.cu:35-140, cayley_math.cuh:51-99,
// common.cuh:82-91), shared by the dynamics kernel (gates.hip) and the fused
// decode-token kernel (decode.hip) so both compute bit-identical values.
//   alpha_j = softplus(alpha_raw_j); omega_j = omega_raw_j + pos (pos = l * rope_freq[h])
//   dt = blend*min(dt_raw, dt_max) + (1-blend)*dt_raw + softplus(sel_dt)
//     dt_raw = softplus(log_dt_scale[h]) / (alpha_0 + |omega_0| + adt_eps)
//     dt_max = (2 - adt_delta) / (alpha_0 + adt_eps), blend = sigmoid((thr - |omega_0|)/smooth)
//   beta = sigmoid(beta_raw) sigmoid(sel_B), sel_C = sigmoid(sel_C_raw)
// Gate row layout per (b, l): [alpha_0..alpha_{N/2-1}, omega_0.., sel_B, sel_C,
// sel_dt, beta, r] x H, element (segment s, head h) at s * H + h.
#pragma once
#include "common.hpp"

namespace cdssm {
namespace gates {

__device__ __forceinline__ float softplus(float x) { return x > 20.0f ? x : log1pf(__expf(x)); }
__device__ __forceinline__ float sigmoid(float x) { return 1.0f / (1.0f + __expf(-x)); }

struct GateConsts {
  float gating_c, omega_thresh, adt_delta, adt_smooth, adt_eps;
};

// The token's shared quantities: dt, sigmoid(r), beta, sel_C.
struct GateToken {
  float dt, rg, beta, selc;
};

// row points at head h's element of segment 0 (gate + bl * G * H + h).
template <typename T>
__device__ __forceinline__ GateToken gate_token(const typename T::raw* row, int H, int N, float lds_h, float pos,
                                                const GateConsts& k) {
  const int Nh = N / 2;
  const float selB = T::load(row + int64_t(N) * H), selC = T::load(row + int64_t(N + 1) * H);
  const float seldt = T::load(row + int64_t(N + 2) * H), braw = T::load(row + int64_t(N + 3) * H);
  const float rraw = T::load(row + int64_t(N + 4) * H);
  const float a0 = softplus(T::load(row));
  const float w0 = T::load(row + int64_t(Nh) * H) + pos;
  const float dts = softplus(lds_h);
  const float wabs = fabsf(w0);
  const float dt_raw = dts / (a0 + wabs + k.adt_eps);
  const float dt_max = (2.0f - k.adt_delta) / (a0 + k.adt_eps);
  const float blend = sigmoid((k.omega_thresh - wabs) / k.adt_smooth);
  GateToken o;
  o.dt = blend * fminf(dt_raw, dt_max) + (1.0f - blend) * dt_raw + softplus(seldt);
  o.rg = sigmoid(rraw);
  o.beta = sigmoid(braw) * sigmoid(selB);
  o.selc = sigmoid(selC);
  return o;
}

// Transition (A_bar pair j, vp_j) of the token; r enters only through c*r.
template <typename T>
__device__ __forceinline__ Transition gate_pair(const typename T::raw* row, int H, int N, int j, float pos,
                                                const GateToken& g, const GateConsts& k) {
  const int Nh = N / 2;
  const float aj = softplus(T::load(row + int64_t(j) * H));
  const float wj = T::load(row + int64_t(Nh + j) * H) + pos;
  return cayley_gated(g.dt, g.rg, aj, wj, k.gating_c);
}

}  // namespace gates
}  // namespace cdssm
