// Gate-level dynamics and K/Q normalisation ops around the scan.
//
// dynamics fwd (DynamicsFusedFn.forward, ops.py:39-66; dynamics_fused.cu:50-139,
// cayley_math.cuh:51-99), one thread per (b, l, h):
//   gate row (b, l): segments [alpha_0..alpha_{N/2-1}, omega_0..omega_{N/2-1},
//   sel_B, sel_C, sel_dt, beta, r] each H wide.
//   alpha_j = softplus(alpha_raw_j); omega_j = omega_raw_j + l * rope_freq[h]
//   dt = blend*min(dt_raw, dt_max) + (1-blend)*dt_raw + softplus(sel_dt)
//     dt_raw = softplus(log_dt_scale[h]) / (alpha_0 + |omega_0| + adt_eps)
//     dt_max = (2 - adt_delta) / (alpha_0 + adt_eps)
//     blend  = sigmoid((omega_thresh - |omega_0|) / adt_smoothness)
//   per pair: Cayley + gating + VP (cayley_gated() in common.hpp, c = gating_c,
//   r = sigmoid(r_raw)); beta = sigmoid(beta_raw) sigmoid(sel_B);
//   sel_C = sigmoid(sel_C_raw).
// dynamics bwd (DynamicsFusedFn.backward, ops.py:68-81; dynamics_fused.cu:166-386):
//   the reference's analytic rule, including its two departures from the exact
//   derivative of the forward: inside the VP clamp it still passes
//   -0.5/vp * grad_vp (dynamics_fused.cu:247-259), and its Cayley derivative
//   uses the eps-free |D|^2 in one factor (:318-321).  grad_log_dt_scale is a
//   deterministic per-head sum (per-token terms, then a fixed-order reduce).
// normalize fwd/bwd (NormalizeKQFn, ops.py:84-97; normalize_kq.cu:75-79,
//   :143-163): x_hat = x rsqrt(sum x^2 + 1e-6); g_in = (g - x_hat <g, x_hat>) rsqrt(...).
//   Any head_dim D <= 256 (the reference kernel is correct only for D = 64).
#include "gate_math.hpp"

namespace cdssm {
namespace gates {

struct GateIdx {
  int64_t bl;   // b*L + l
  int l, h;
};

__device__ __forceinline__ bool gate_idx(int64_t tid, int L, int H, int64_t total, GateIdx& g) {
  if (tid >= total) return false;
  g.h = int(tid % H);
  g.bl = tid / H;
  g.l = int(g.bl % L);
  return true;
}

template <typename T>
__global__ __launch_bounds__(256) void dynamics_fwd_kernel(
    const typename T::raw* __restrict__ gate, const float* __restrict__ log_dt_scale,
    const float* __restrict__ rope, typename T::raw* __restrict__ A_out, typename T::raw* __restrict__ vp_out,
    typename T::raw* __restrict__ beta_out, typename T::raw* __restrict__ selc_out, float gating_c,
    float omega_thresh, float adt_delta, float adt_smooth, float adt_eps, int L, int H, int N,
    int64_t total, int64_t l0, const int64_t* __restrict__ l0_dev) {
  GateIdx g;
  if (!gate_idx(int64_t(blockIdx.x) * blockDim.x + threadIdx.x, L, H, total, g)) return;
  const int Nh = N / 2, G = N + 5;
  const typename T::raw* row = gate + g.bl * int64_t(G) * H + g.h;
  const float freq = rope[g.h];
  const float pos = float(g.l + l0 + (l0_dev ? *l0_dev : 0)) * freq;  // sequence position
  const GateConsts kc{gating_c, omega_thresh, adt_delta, adt_smooth, adt_eps};
  const GateToken gt = gate_token<T>(row, H, N, log_dt_scale[g.h], pos, kc);
  const int64_t o = g.bl * H + g.h;
  for (int j = 0; j < Nh; ++j) {
    const Transition tr = gate_pair<T>(row, H, N, j, pos, gt, kc);
    T::store(A_out + o * N + 2 * j, tr.ar);
    T::store(A_out + o * N + 2 * j + 1, tr.ai);
    T::store(vp_out + o * Nh + j, tr.vp);
  }
  T::store(beta_out + o, gt.beta);
  T::store(selc_out + o, gt.selc);
}

template <typename T>
__global__ __launch_bounds__(256) void dynamics_bwd_kernel(
    const typename T::raw* __restrict__ gA, const typename T::raw* __restrict__ gvp,
    const typename T::raw* __restrict__ gbeta, const typename T::raw* __restrict__ gselc,
    const typename T::raw* __restrict__ gate, const float* __restrict__ log_dt_scale,
    const float* __restrict__ rope, typename T::raw* __restrict__ ggate, float* __restrict__ glog_terms,
    float c, float omega_thresh, float adt_delta, float adt_smooth, float adt_eps, int L, int H, int N,
    int64_t total) {
  GateIdx g;
  if (!gate_idx(int64_t(blockIdx.x) * blockDim.x + threadIdx.x, L, H, total, g)) return;
  const int Nh = N / 2, G = N + 5;
  const int64_t roff = g.bl * int64_t(G) * H + g.h;
  const typename T::raw* row = gate + roff;
  typename T::raw* grow = ggate + roff;
  const int64_t o = g.bl * H + g.h;
  const float freq = rope[g.h];
  const float pos = float(g.l) * freq;
  const float log_scale = log_dt_scale[g.h];

  const float selB = T::load(row + int64_t(N) * H), selC = T::load(row + int64_t(N + 1) * H);
  const float seldt = T::load(row + int64_t(N + 2) * H), braw = T::load(row + int64_t(N + 3) * H);
  const float rraw = T::load(row + int64_t(N + 4) * H);
  const float rg = sigmoid(rraw);
  const float a0raw = T::load(row);
  const float a0 = softplus(a0raw);
  const float w0 = T::load(row + int64_t(Nh) * H) + pos;
  const float dts = softplus(log_scale);
  const float wabs = fabsf(w0);
  const float chr = a0 + wabs + adt_eps;
  const float dt_raw = dts / chr;
  const float dt_max = (2.0f - adt_delta) / (a0 + adt_eps);
  const float blend = sigmoid((omega_thresh - wabs) / adt_smooth);
  const float dt_capped = fminf(dt_raw, dt_max);
  const bool capped = dt_raw > dt_max;
  const float dt = blend * dt_capped + (1.0f - blend) * dt_raw + softplus(seldt);

  // scalar gates
  const float sb = sigmoid(braw), ss = sigmoid(selB), sc = sigmoid(selC);
  const float g_b = T::load(gbeta + o), g_sc = T::load(gselc + o);
  T::store(grow + int64_t(N + 1) * H, g_sc * sc * (1.0f - sc));
  T::store(grow + int64_t(N + 3) * H, g_b * ss * sb * (1.0f - sb));
  T::store(grow + int64_t(N) * H, g_b * sb * ss * (1.0f - ss));

  const float cr = c * rg;
  const float expo = 0.5f * (cr - 1.0f);
  float g_dt = 0.0f, g_r = 0.0f, ga0 = 0.0f, gw0 = 0.0f;
  for (int j = 0; j < Nh; ++j) {
    const float araw = T::load(row + int64_t(j) * H);
    const float alpha = softplus(araw);
    const float omega = T::load(row + int64_t(Nh + j) * H) + pos;
    const float tau = 0.5f * dt;
    const float ac = fmaxf(alpha, 0.0f);
    const float ta = tau * ac, tw = tau * omega;
    const float opa = 1.0f + ta, oma = 1.0f - ta;
    const float det = opa * opa + tw * tw;
    const float inv = 1.0f / (det + 1e-6f);
    const float num_re = 1.0f - ta * ta - tw * tw;
    const float mre = num_re * inv, mim = -(2.0f * tw) * inv;   // stored conj(mu)
    const float eig = (oma * oma + tw * tw) * inv;
    const float E = fmaxf(eig, 1e-8f);
    const float lE2 = __builtin_amdgcn_logf(E);
    const float lE = lE2 * 0.69314718055994531f;
    const float scale = __builtin_amdgcn_exp2f(expo * lE2);
    const float eff = __builtin_amdgcn_exp2f(cr * lE2);
    const float vp = sqrtf(fmaxf(1.0f - eff, 1e-6f));
    float gar = T::load(gA + o * N + 2 * j), gai = T::load(gA + o * N + 2 * j + 1);
    const float gv = T::load(gvp + o * Nh + j);
    const bool active = vp > 1e-6f && vp < 1.0f;
    const float d_eff = active ? gv * (-0.5f / vp) : 0.0f;
    const bool unclamped = E > 1e-8f;
    float d_eig = unclamped ? d_eff * cr * (eff / E) : 0.0f;
    float d_r = d_eff * c * lE * eff;
    const float d_scale = gar * mre + gai * mim;
    if (unclamped) d_eig += d_scale * expo * (scale / E);
    d_r += d_scale * (0.5f * c) * lE * scale;
    gar *= scale;
    gai *= scale;
    const float d_numer = d_eig * inv;
    const float d_denom = -d_eig * eig * inv;
    float d_ta = d_numer * (-2.0f * oma) + d_denom * 2.0f * opa;
    float d_tw = d_numer * 2.0f * tw + d_denom * 2.0f * tw;
    const float gmr = gar, gmi = -gai;
    const float inv2 = inv * inv;
    d_ta += gmr * ((-2.0f * ta * det - num_re * 2.0f * opa) * inv2) + gmi * (-2.0f * tw * 2.0f * opa * inv2);
    d_tw += gmr * ((-2.0f * tw * det - num_re * 2.0f * tw) * inv2) +
            gmi * ((2.0f * det - 4.0f * tw * tw) * inv2);
    const float g_alpha = alpha >= 0.0f ? d_ta * tau : 0.0f;
    const float g_omega = d_tw * tau;
    g_dt += d_ta * ac * 0.5f + d_tw * omega * 0.5f;
    g_r += d_r;
    float ga_raw = g_alpha * sigmoid(araw);
    float gw_raw = g_omega;
    if (j == 0) {  // pair 0 also feeds the adaptive dt; stored after the loop
      ga0 = ga_raw;
      gw0 = gw_raw;
    } else {
      T::store(grow + int64_t(j) * H, ga_raw);
      T::store(grow + int64_t(Nh + j) * H, gw_raw);
    }
  }
  // adaptive dt
  const float g_seldt = g_dt * sigmoid(seldt);
  const float capf = capped ? 1.0f : 0.0f;
  const float g_raw_adt = g_dt * (1.0f - capf * blend);
  const float g_max_adt = g_dt * capf * blend;
  const float g_blend = g_dt * (dt_capped - dt_raw);
  const float dblend = -blend * (1.0f - blend) / adt_smooth;
  const float g_dts = g_raw_adt / chr;
  const float g_chr = g_raw_adt * (-dts / (chr * chr));
  const float g_amax = g_max_adt * (-(2.0f - adt_delta) / ((a0 + adt_eps) * (a0 + adt_eps)));
  const float g_wabs = g_chr + g_blend * dblend;
  const float sgn = w0 >= 0.0f ? 1.0f : -1.0f;
  T::store(grow, ga0 + (g_chr + g_amax) * sigmoid(a0raw));
  T::store(grow + int64_t(Nh) * H, gw0 + g_wabs * sgn);
  T::store(grow + int64_t(N + 2) * H, g_seldt);
  T::store(grow + int64_t(N + 4) * H, g_r * rg * (1.0f - rg));
  glog_terms[o] = g_dts * sigmoid(log_scale);
}

// Fixed-order per-head sum of the per-token grad_log_dt_scale terms (BL, H):
// the workgroup (h, slab) adds its slab of kHeadSlabs consecutive row ranges
// (threads strided, then a fixed tree) into part[slab][h]; a second launch
// adds the slabs in order per head.  H x kHeadSlabs workgroups keep the loads
// in flight across the device (one workgroup per head left 240 CUs idle).
constexpr int kHeadSlabs = 64;

__global__ __launch_bounds__(256) void head_part_kernel(const float* __restrict__ terms,
                                                        float* __restrict__ part, int64_t BL, int H) {
  __shared__ float sm[256];
  const int h = blockIdx.x, sl = blockIdx.y;
  const int64_t r0 = BL * sl / kHeadSlabs, r1 = BL * (sl + 1) / kHeadSlabs;
  float a = 0.0f;
  for (int64_t i = r0 + threadIdx.x; i < r1; i += 256) a += terms[i * H + h];
  sm[threadIdx.x] = a;
  __syncthreads();
  for (int s = 128; s > 0; s >>= 1) {
    if (int(threadIdx.x) < s) sm[threadIdx.x] += sm[threadIdx.x + s];
    __syncthreads();
  }
  if (threadIdx.x == 0) part[int64_t(sl) * H + h] = sm[0];
}

__global__ __launch_bounds__(256) void head_sum_kernel(const float* __restrict__ part, float* __restrict__ out,
                                                       int H) {
  const int h = int(blockIdx.x) * 256 + int(threadIdx.x);
  if (h >= H) return;
  float a = 0.0f;
  for (int sl = 0; sl < kHeadSlabs; ++sl) a += part[int64_t(sl) * H + h];
  out[h] = a;
}

// ---------------------------------------------------------------------------
// K/Q normalisation: 16 lanes per row, 4 rows per wave.
// ---------------------------------------------------------------------------
constexpr int kNormLanes = 16;

template <typename T>
__global__ __launch_bounds__(256) void normalize_fwd_kernel(const typename T::raw* __restrict__ x,
                                                            typename T::raw* __restrict__ y, int64_t rows,
                                                            int D) {
  const int64_t row = (int64_t(blockIdx.x) * blockDim.x + threadIdx.x) / kNormLanes;
  const int sub = threadIdx.x % kNormLanes;
  const bool ok = row < rows;
  const typename T::raw* p = x + (ok ? row : 0) * D;
  float s = 0.0f;
  for (int d = sub; d < D; d += kNormLanes) {
    const float v = T::load(p + d);
    s = fmaf(v, v, s);
  }
  s = group_sum<kNormLanes>(s);
  const float inv = rsqrtf(s + 1e-6f);
  if (!ok) return;
  for (int d = sub; d < D; d += kNormLanes) T::store(y + row * D + d, T::load(p + d) * inv);
}

template <typename T>
__global__ __launch_bounds__(256) void normalize_bwd_kernel(const typename T::raw* __restrict__ g,
                                                            const typename T::raw* __restrict__ x,
                                                            typename T::raw* __restrict__ gx,
                                                            int64_t rows, int D) {
  const int64_t row = (int64_t(blockIdx.x) * blockDim.x + threadIdx.x) / kNormLanes;
  const int sub = threadIdx.x % kNormLanes;
  const bool ok = row < rows;
  const int64_t base = (ok ? row : 0) * D;
  float s = 0.0f, gxd = 0.0f;
  for (int d = sub; d < D; d += kNormLanes) {
    const float v = T::load(x + base + d);
    s = fmaf(v, v, s);
    gxd = fmaf(T::load(g + base + d), v, gxd);
  }
  s = group_sum<kNormLanes>(s);
  gxd = group_sum<kNormLanes>(gxd);
  const float inv = rsqrtf(s + 1e-6f);
  const float proj = gxd * inv;  // <g, x_hat>
  if (!ok) return;
  for (int d = sub; d < D; d += kNormLanes) {
    const float xh = T::load(x + base + d) * inv;
    T::store(gx + base + d, (T::load(g + base + d) - xh * proj) * inv);
  }
}

}  // namespace gates
}  // namespace cdssm

// ---------------------------------------------------------------------------
// C-ABI
// ---------------------------------------------------------------------------
namespace {
using namespace cdssm;
using namespace cdssm::gates;

int check_dtype(const char* op, int dtype) {
  if (dtype != 0 && dtype != 1) {
    cdssm_host::set_error("%s: dtype must be 0 (fp32) or 1 (bf16), got %d", op, dtype);
    return CDSSM_EINVAL;
  }
  return CDSSM_OK;
}

int check_gate_shape(const char* op, int64_t B, int64_t L, int64_t H, int64_t N) {
  if (B <= 0 || L <= 0 || H <= 0) {
    cdssm_host::set_error("%s: B, L, H must be positive", op);
    return CDSSM_EINVAL;
  }
  if (N <= 0 || N % 2 != 0 || N > 32) {
    cdssm_host::set_error("%s: state_dim must be even and in [2, 32], got %lld", op, (long long)N);
    return CDSSM_EINVAL;
  }
  if (B * L * H * (N + 5) > (int64_t(1) << 40) || L > (int64_t(1) << 24)) {
    cdssm_host::set_error("%s: problem too large", op);
    return CDSSM_EINVAL;
  }
  return CDSSM_OK;
}

}  // namespace

extern "C" int cdssm_dynamics_fused_fwd_at(int dtype, const void* gate_raw, const float* log_dt_scale,
                                           const float* rope_freqs, float gating_c, float omega_thresh,
                                           float adt_delta, float adt_smoothness, float adt_eps, void* A_bar,
                                           void* vp_scale, void* beta, void* sel_c, int64_t B, int64_t L, int64_t H,
                                           int64_t N, int64_t l0, const int64_t* l0_dev, hipStream_t stream) {
  const char* op = "cdssm_dynamics_fused_fwd";
  if (l0 < 0 || l0 > (int64_t(1) << 40)) {
    cdssm_host::set_error("%s: position offset %lld out of range", op, (long long)l0);
    return CDSSM_EINVAL;
  }
  int st = check_dtype(op, dtype);
  if (!st) st = check_gate_shape(op, B, L, H, N);
  if (st) return st;
  if (!gate_raw || !log_dt_scale || !rope_freqs || !A_bar || !vp_scale || !beta || !sel_c) {
    cdssm_host::set_error("%s: null pointer argument", op);
    return CDSSM_EINVAL;
  }
  if (!(adt_smoothness != 0.0f)) {
    cdssm_host::set_error("%s: adt_smoothness must be nonzero", op);
    return CDSSM_EINVAL;
  }
  const int64_t total = B * L * H;
  const unsigned blocks = unsigned((total + 255) / 256);
  if (dtype == 1)
    hipLaunchKernelGGL(dynamics_fwd_kernel<BF16>, dim3(blocks), dim3(256), 0, stream, (const uint16_t*)gate_raw,
                       log_dt_scale, rope_freqs, (uint16_t*)A_bar, (uint16_t*)vp_scale, (uint16_t*)beta,
                       (uint16_t*)sel_c, gating_c, omega_thresh, adt_delta, adt_smoothness, adt_eps, int(L),
                       int(H), int(N), total, l0, l0_dev);
  else
    hipLaunchKernelGGL(dynamics_fwd_kernel<F32>, dim3(blocks), dim3(256), 0, stream, (const float*)gate_raw,
                       log_dt_scale, rope_freqs, (float*)A_bar, (float*)vp_scale, (float*)beta, (float*)sel_c,
                       gating_c, omega_thresh, adt_delta, adt_smoothness, adt_eps, int(L), int(H), int(N),
                       total, l0, l0_dev);
  return cdssm_host::check_launch(op);
}

extern "C" int cdssm_dynamics_fused_fwd(int dtype, const void* gate_raw, const float* log_dt_scale,
                                        const float* rope_freqs, float gating_c, float omega_thresh,
                                        float adt_delta, float adt_smoothness, float adt_eps,
                                        void* A_bar, void* vp_scale, void* beta, void* sel_c, int64_t B,
                                        int64_t L, int64_t H, int64_t N, hipStream_t stream) {
  return cdssm_dynamics_fused_fwd_at(dtype, gate_raw, log_dt_scale, rope_freqs, gating_c, omega_thresh, adt_delta,
                                     adt_smoothness, adt_eps, A_bar, vp_scale, beta, sel_c, B, L, H, N, 0, nullptr,
                                     stream);
}

extern "C" int64_t cdssm_dynamics_fused_bwd_workspace_bytes(int64_t B, int64_t L, int64_t H) {
  if (B <= 0 || L <= 0 || H <= 0) return -1;
  return (B * L + kHeadSlabs) * H * int64_t(sizeof(float));  // the per-token terms, then the slab sums
}

extern "C" int cdssm_dynamics_fused_bwd(int dtype, const void* grad_A_bar, const void* grad_vp_scale,
                                        const void* grad_beta, const void* grad_sel_c,
                                        const void* gate_raw, const float* log_dt_scale,
                                        const float* rope_freqs, float gating_c, float omega_thresh,
                                        float adt_delta, float adt_smoothness, float adt_eps,
                                        void* grad_gate_raw, float* grad_log_dt_scale, float* workspace,
                                        int64_t B, int64_t L, int64_t H, int64_t N, hipStream_t stream) {
  const char* op = "cdssm_dynamics_fused_bwd";
  int st = check_dtype(op, dtype);
  if (!st) st = check_gate_shape(op, B, L, H, N);
  if (st) return st;
  if (!grad_A_bar || !grad_vp_scale || !grad_beta || !grad_sel_c || !gate_raw || !log_dt_scale ||
      !rope_freqs || !grad_gate_raw || !grad_log_dt_scale || !workspace) {
    cdssm_host::set_error("%s: null pointer argument", op);
    return CDSSM_EINVAL;
  }
  if (!(adt_smoothness != 0.0f)) {
    cdssm_host::set_error("%s: adt_smoothness must be nonzero", op);
    return CDSSM_EINVAL;
  }
  const int64_t total = B * L * H;
  const unsigned blocks = unsigned((total + 255) / 256);
  if (dtype == 1)
    hipLaunchKernelGGL(dynamics_bwd_kernel<BF16>, dim3(blocks), dim3(256), 0, stream,
                       (const uint16_t*)grad_A_bar, (const uint16_t*)grad_vp_scale, (const uint16_t*)grad_beta,
                       (const uint16_t*)grad_sel_c, (const uint16_t*)gate_raw, log_dt_scale, rope_freqs,
                       (uint16_t*)grad_gate_raw, workspace, gating_c, omega_thresh, adt_delta, adt_smoothness,
                       adt_eps, int(L), int(H), int(N), total);
  else
    hipLaunchKernelGGL(dynamics_bwd_kernel<F32>, dim3(blocks), dim3(256), 0, stream, (const float*)grad_A_bar,
                       (const float*)grad_vp_scale, (const float*)grad_beta, (const float*)grad_sel_c,
                       (const float*)gate_raw, log_dt_scale, rope_freqs, (float*)grad_gate_raw, workspace,
                       gating_c, omega_thresh, adt_delta, adt_smoothness, adt_eps, int(L), int(H), int(N),
                       total);
  st = cdssm_host::check_launch(op);
  if (st) return st;
  float* part = workspace + B * L * H;
  hipLaunchKernelGGL(head_part_kernel, dim3(unsigned(H), unsigned(kHeadSlabs)), dim3(256), 0, stream,
                     (const float*)workspace, part, B * L, int(H));
  st = cdssm_host::check_launch(op);
  if (st) return st;
  hipLaunchKernelGGL(head_sum_kernel, dim3(unsigned((H + 255) / 256)), dim3(256), 0, stream, (const float*)part,
                     grad_log_dt_scale, int(H));
  return cdssm_host::check_launch(op);
}

extern "C" int cdssm_normalize_kq_fwd(int dtype, const void* K, const void* Q, void* K_out, void* Q_out,
                                      int64_t rows, int64_t D, hipStream_t stream) {
  const char* op = "cdssm_normalize_kq_fwd";
  int st = check_dtype(op, dtype);
  if (st) return st;
  if (rows <= 0 || D <= 0 || D > 256 || rows > (int64_t(1) << 36)) {
    cdssm_host::set_error("%s: need rows > 0 and 0 < D <= 256 (rows=%lld D=%lld)", op, (long long)rows,
                          (long long)D);
    return CDSSM_EINVAL;
  }
  if (!K || !Q || !K_out || !Q_out) {
    cdssm_host::set_error("%s: null pointer argument", op);
    return CDSSM_EINVAL;
  }
  const unsigned blocks = unsigned((rows * kNormLanes + 255) / 256);
  if (dtype == 1) {
    hipLaunchKernelGGL(normalize_fwd_kernel<BF16>, dim3(blocks), dim3(256), 0, stream, (const uint16_t*)K,
                       (uint16_t*)K_out, rows, int(D));
    hipLaunchKernelGGL(normalize_fwd_kernel<BF16>, dim3(blocks), dim3(256), 0, stream, (const uint16_t*)Q,
                       (uint16_t*)Q_out, rows, int(D));
  } else {
    hipLaunchKernelGGL(normalize_fwd_kernel<F32>, dim3(blocks), dim3(256), 0, stream, (const float*)K,
                       (float*)K_out, rows, int(D));
    hipLaunchKernelGGL(normalize_fwd_kernel<F32>, dim3(blocks), dim3(256), 0, stream, (const float*)Q,
                       (float*)Q_out, rows, int(D));
  }
  return cdssm_host::check_launch(op);
}

extern "C" int cdssm_normalize_kq_bwd(int dtype, const void* grad_K_out, const void* grad_Q_out,
                                      const void* K, const void* Q, void* grad_K, void* grad_Q, int64_t rows,
                                      int64_t D, hipStream_t stream) {
  const char* op = "cdssm_normalize_kq_bwd";
  int st = check_dtype(op, dtype);
  if (st) return st;
  if (rows <= 0 || D <= 0 || D > 256 || rows > (int64_t(1) << 36)) {
    cdssm_host::set_error("%s: need rows > 0 and 0 < D <= 256 (rows=%lld D=%lld)", op, (long long)rows,
                          (long long)D);
    return CDSSM_EINVAL;
  }
  if (!grad_K_out || !grad_Q_out || !K || !Q || !grad_K || !grad_Q) {
    cdssm_host::set_error("%s: null pointer argument", op);
    return CDSSM_EINVAL;
  }
  const unsigned blocks = unsigned((rows * kNormLanes + 255) / 256);
  if (dtype == 1) {
    hipLaunchKernelGGL(normalize_bwd_kernel<BF16>, dim3(blocks), dim3(256), 0, stream,
                       (const uint16_t*)grad_K_out, (const uint16_t*)K, (uint16_t*)grad_K, rows, int(D));
    hipLaunchKernelGGL(normalize_bwd_kernel<BF16>, dim3(blocks), dim3(256), 0, stream,
                       (const uint16_t*)grad_Q_out, (const uint16_t*)Q, (uint16_t*)grad_Q, rows, int(D));
  } else {
    hipLaunchKernelGGL(normalize_bwd_kernel<F32>, dim3(blocks), dim3(256), 0, stream, (const float*)grad_K_out,
                       (const float*)K, (float*)grad_K, rows, int(D));
    hipLaunchKernelGGL(normalize_bwd_kernel<F32>, dim3(blocks), dim3(256), 0, stream, (const float*)grad_Q_out,
                       (const float*)Q, (float*)grad_Q, rows, int(D));
  }
  return cdssm_host::check_launch(op);
}
