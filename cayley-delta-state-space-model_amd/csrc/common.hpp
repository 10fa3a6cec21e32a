// Shared device helpers for the CD-SSM scan kernels (gfx950, wave64).
//
// Conventions used by every kernel in this library:
//   * tensors are contiguous, token-major (B, L, H, ...), as in the reference's
//     ops.py contracts;
//   * bf16 values travel as raw 16-bit patterns (uint16_t) and are widened to
//     fp32 by a shift; every state and every accumulation is fp32;
//   * a complex pair (re, im) is stored interleaved, and the stored transition
//     A_bar = conj(mu) * scale multiplies a state row pair as a complex scalar
//     (reference: intra_chunk_scan.cu:151-162, cayley_math.cuh:20-24).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

namespace cdssm {

constexpr int kWave = 64;

// ---------------------------------------------------------------------------
// bf16 <-> fp32
// ---------------------------------------------------------------------------

__device__ __forceinline__ float bf16_lo(uint32_t packed) { return __uint_as_float(packed << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t packed) { return __uint_as_float(packed & 0xffff0000u); }
__device__ __forceinline__ float bf16_to_f32(uint16_t x) { return __uint_as_float(uint32_t(x) << 16); }

// Round-to-nearest-even narrowing; NaN stays NaN.
__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return uint16_t((u >> 16) | 0x40u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return uint16_t(u >> 16);
}

// A copy of x in a new register (an explicit v_mov the compiler cannot fold
// away): lets a prefetch ring slot be reloaded while its old value is in use.
__device__ __forceinline__ float fresh(float x) {
  float r;
  asm volatile("v_mov_b32 %0, %1" : "=v"(r) : "v"(x));
  return r;
}

// Two fp32 -> packed bf16 pair (lo = a), round-to-nearest-even in one
// v_cvt_pk_bf16_f32.
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t pack_bf16x2(float a, float b) {
  const f32x2_t x = {a, b};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(x, bf16x2_t));
}

// Element type tags: loads of one element and stores of one element.
struct BF16 {
  using raw = uint16_t;
  static constexpr int bytes = 2;
  __device__ __forceinline__ static float load(const raw* p) { return bf16_to_f32(*p); }
  __device__ __forceinline__ static void store(raw* p, float v) { *p = f32_to_bf16(v); }
};
struct F32 {
  using raw = float;
  static constexpr int bytes = 4;
  __device__ __forceinline__ static float load(const raw* p) { return *p; }
  __device__ __forceinline__ static void store(raw* p, float v) { *p = v; }
};

// An (re, im) pair in one store (the pair's address aligned to its size).
template <typename T>
__device__ __forceinline__ void store_pair(typename T::raw* p, float re, float im) {
  if constexpr (T::bytes == 2)
    *reinterpret_cast<uint32_t*>(p) = pack_bf16x2(re, im);
  else
    *reinterpret_cast<float2*>(p) = make_float2(re, im);
}

// Input form of the fused forward: ABar<T> (elements of type T) takes the
// per-token transition a_t (B,L,H,2) and VP scale (B,L,H,1) as computed by the
// gate-level dynamics (in place of dt and r), instead of the scan-level
// (dt, r, alpha, omega, c) from which the kernels compute them.
template <typename Base>
struct ABar : Base {};
template <typename T>
struct IsABar {
  static constexpr bool value = false;
};
template <typename Base>
struct IsABar<ABar<Base>> {
  static constexpr bool value = true;
};

// Form SsdY<T>: the SSDChunkwiseScan interface (ssd.py:39-111).  The transition
// a_t comes as A_bar (B,L,H,2) in dt's place, the values are already VP-scaled
// (vp = 1, r unused), there is no q or sel_C, and the scan's
// Y_t = local state + correction, (B,L,H,2,D) with the (re, im) rows of each
// head D apart, is written in place of the readout.
template <typename Base>
struct SsdY : Base {};
template <typename T>
struct IsSsdY {
  static constexpr bool value = false;
};
template <typename Base>
struct IsSsdY<SsdY<Base>> {
  static constexpr bool value = true;
};
// a_t read from the input (A_bar) rather than computed from (dt, r, alpha, omega, c)
template <typename T>
struct GivenA {
  static constexpr bool value = IsABar<T>::value || IsSsdY<T>::value;
};

// A wave's (chunk, head group) tile of a (B, L, H, D) tensor as a buffer
// resource: the base (wave-uniform, scalar registers) is the tile's first row
// at its first head, each lane adds its constant byte offset (head, slice),
// and a token is selected by a scalar byte offset, so a row load costs one
// scalar add instead of a 64-bit address computation.  num_records covers
// the tensor's bytes from the base (clamped to 32 bits); every access the
// kernels make is in range by construction.
struct RowStream {
  __amdgpu_buffer_rsrc_t rs;
  int voff;
};

__device__ __forceinline__ RowStream make_row_stream(const void* base, int64_t bytes_from_base, int lane_off_bytes) {
  const uint64_t n = bytes_from_base > 0 ? uint64_t(bytes_from_base) : 0ull;
  const int nrec = int(uint32_t(n > 0xffffffffull ? 0xffffffffull : n));
  return RowStream{__builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), short(0), nrec, 0x00020000),
                   lane_off_bytes};
}

// A lane's slice of one row: DPL consecutive elements, loaded with a single
// 4-, 8- or 16-byte load into W = DPL * bytes / 4 dwords and widened on use.
template <typename T, int DPL>
struct RowVec {
  static constexpr int W = DPL * T::bytes / 4;
  static_assert(W == 1 || W == 2 || W == 4 || W == 8, "a lane slice is 4, 8, 16 or 32 bytes");
  uint32_t u[W];

  // The slice at scalar byte offset soff of a row stream.
  __device__ __forceinline__ void load(const RowStream& s, int soff) {
    if constexpr (W == 8) {
      const auto v0 = __builtin_amdgcn_raw_buffer_load_b128(s.rs, s.voff, soff, 0);
      const auto v1 = __builtin_amdgcn_raw_buffer_load_b128(s.rs, s.voff + 16, soff, 0);
      u[0] = v0[0]; u[1] = v0[1]; u[2] = v0[2]; u[3] = v0[3];
      u[4] = v1[0]; u[5] = v1[1]; u[6] = v1[2]; u[7] = v1[3];
    } else if constexpr (W == 4) {
      const auto v = __builtin_amdgcn_raw_buffer_load_b128(s.rs, s.voff, soff, 0);
      u[0] = v[0]; u[1] = v[1]; u[2] = v[2]; u[3] = v[3];
    } else if constexpr (W == 2) {
      const auto v = __builtin_amdgcn_raw_buffer_load_b64(s.rs, s.voff, soff, 0);
      u[0] = v[0]; u[1] = v[1];
    } else {
      u[0] = __builtin_amdgcn_raw_buffer_load_b32(s.rs, s.voff, soff, 0);
    }
  }

  __device__ __forceinline__ void load(const typename T::raw* p) {
    if constexpr (W == 8) {
      const uint4 v0 = reinterpret_cast<const uint4*>(p)[0];
      const uint4 v1 = reinterpret_cast<const uint4*>(p)[1];
      u[0] = v0.x; u[1] = v0.y; u[2] = v0.z; u[3] = v0.w;
      u[4] = v1.x; u[5] = v1.y; u[6] = v1.z; u[7] = v1.w;
    } else if constexpr (W == 4) {
      const uint4 v = *reinterpret_cast<const uint4*>(p);
      u[0] = v.x; u[1] = v.y; u[2] = v.z; u[3] = v.w;
    } else if constexpr (W == 2) {
      const uint2 v = *reinterpret_cast<const uint2*>(p);
      u[0] = v.x; u[1] = v.y;
    } else {
      u[0] = *reinterpret_cast<const uint32_t*>(p);
    }
  }
  // Opaque copy: keeps the compiler from merging a prefetch ring's initial
  // loads with the in-loop loads into one load at the loop head (which would
  // undo the software pipelining).  Waits for this slice's load.
  __device__ __forceinline__ void pin() {
#pragma unroll
    for (int i = 0; i < W; ++i) asm volatile("" : "+v"(u[i]));
  }
  // Unpack, then order the caller's next load of this slice after the unpack:
  // without the barrier the scheduler may hoist that load above the unpack,
  // the old and new slice overlap, and the register allocator copies the ring
  // at the loop latch, which waits for every outstanding load.
  __device__ __forceinline__ void unpack_then_reload(float (&o)[DPL]) const {
    unpack(o);
#pragma unroll
    for (int i = 0; i < DPL; ++i) asm volatile("" ::"v"(o[i]) : "memory");
  }
  __device__ __forceinline__ void unpack(float (&o)[DPL]) const {
    if constexpr (T::bytes == 2) {
#pragma unroll
      for (int i = 0; i < W; ++i) {
        o[2 * i] = bf16_lo(u[i]);
        o[2 * i + 1] = bf16_hi(u[i]);
      }
    } else {
#pragma unroll
      for (int i = 0; i < W; ++i) o[i] = __uint_as_float(u[i]);
    }
  }
};

// ---------------------------------------------------------------------------
// Lane-group all-reduce (sum) over G consecutive lanes, G in {1,2,4,...,64}.
// DPP quad permutes and row mirrors stay inside a 16-lane row; the 32- and
// 64-lane stages use the gfx950 row / half-wave swaps.  All stages are VALU
// (no LDS round trip).  Every lane of the group ends with the group sum.
// ---------------------------------------------------------------------------

// Full-row permutes only (every source lane valid), so bound_ctrl never
// zeroes a lane; with it set the compiler folds the move into the add
// (v_add_f32_dpp).
template <int CTRL>
__device__ __forceinline__ float dpp(float x) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), CTRL, 0xF, 0xF, true));
}

// x from lane (lane - OFF) of the same NB-lane segment: a DPP row shift when
// the segments fit the 16-lane DPP rows (a few cycles), else a lane shuffle
// (an LDS-crossbar permute).  Lanes whose offset in the segment is below OFF
// get an unspecified value; callers mask them.
template <int NB, int OFF, typename V>
__device__ __forceinline__ V seg_shift_up(V x) {
  static_assert(sizeof(V) == 4 && OFF >= 1 && OFF < NB, "32-bit values, shift inside the segment");
  if constexpr (NB <= 16) {
    const int u = __builtin_bit_cast(int, x);
    return __builtin_bit_cast(V, __builtin_amdgcn_update_dpp(u, u, 0x110 + OFF, 0xF, 0xF, false));
  } else {
    return __shfl_up(x, OFF, NB);
  }
}

// x from lane (lane + OFF) of the same NB-lane segment (the mirror of
// seg_shift_up); lanes whose offset in the segment is NB - OFF or more get an
// unspecified value; callers mask them.
template <int NB, int OFF, typename V>
__device__ __forceinline__ V seg_shift_down(V x) {
  static_assert(sizeof(V) == 4 && OFF >= 1 && OFF < NB, "32-bit values, shift inside the segment");
  if constexpr (NB <= 16) {
    const int u = __builtin_bit_cast(int, x);
    return __builtin_bit_cast(V, __builtin_amdgcn_update_dpp(u, u, 0x100 + OFF, 0xF, 0xF, false));
  } else {
    return __shfl_down(x, OFF, NB);
  }
}

// f(std::integral_constant<int, s>) for s = 1, 2, 4, ... < NB (the steps of a
// segmented Hillis-Steele scan over NB lanes)
template <int NB, typename F>
__device__ __forceinline__ void for_shifts(F&& f) {
  if constexpr (NB > 1) f(std::integral_constant<int, 1>{});
  if constexpr (NB > 2) f(std::integral_constant<int, 2>{});
  if constexpr (NB > 4) f(std::integral_constant<int, 4>{});
  if constexpr (NB > 8) f(std::integral_constant<int, 8>{});
  if constexpr (NB > 16) f(std::integral_constant<int, 16>{});
  if constexpr (NB > 32) f(std::integral_constant<int, 32>{});
}

template <int G>
__device__ __forceinline__ float group_sum(float x) {
  static_assert(G == 1 || G == 2 || G == 4 || G == 8 || G == 16 || G == 32 || G == 64, "group size");
  if constexpr (G >= 2) x += dpp<0xB1>(x);     // quad_perm [1,0,3,2]: lane ^ 1
  if constexpr (G >= 4) x += dpp<0x4E>(x);     // quad_perm [2,3,0,1]: lane ^ 2
  if constexpr (G >= 8) x += dpp<0x141>(x);    // row_half_mirror: other quad of the 8
  if constexpr (G >= 16) x += dpp<0x140>(x);   // row_mirror: other half of the row
  if constexpr (G >= 32) {
    // v_permlane16_swap: each row meets its neighbour row (lane ^ 16)
    const auto sw = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    x = __uint_as_float(sw[0]) + __uint_as_float(sw[1]);
  }
  if constexpr (G >= 64) {
    // v_permlane32_swap: the two halves of the wave meet (lane ^ 32)
    const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    x = __uint_as_float(sw[0]) + __uint_as_float(sw[1]);
  }
  return x;
}

// Sum over the wave's heads of a value its lanes hold per head, for heads of
// LPH lanes (lane = head * LPH + slice): every lane gets the sum over the lanes
// of its slice in all heads.  Row swaps only (heads are whole rows of 16 lanes
// or more), in a fixed order.
template <int LPH>
__device__ __forceinline__ float cross_head_sum(float x) {
  static_assert(LPH == 16 || LPH == 32 || LPH == 64, "heads of whole 16-lane rows");
  if constexpr (LPH <= 16) {
    const auto sw = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    x = __uint_as_float(sw[0]) + __uint_as_float(sw[1]);
  }
  if constexpr (LPH <= 32) {
    const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    x = __uint_as_float(sw[0]) + __uint_as_float(sw[1]);
  }
  return x;
}

// ---------------------------------------------------------------------------
// Tiles of the fused scan: one wave per (b, chunk, group of HPW heads).
// ---------------------------------------------------------------------------
__host__ __device__ constexpr int round_up(int x, int m) { return (x + m - 1) / m * m; }

// Decode blockIdx.x -> (b, chunk, head group).
struct ChunkTile {
  int b, chunk, hbase, t0, nt;
  int64_t row0;
};

// Row streams of a (B, L, H, D) tensor for the lane's head of a chunk tile:
// base at (row0, hbase), lane offset (head of the lane, or H - 1 past the
// last head; element slice), token stride H * D elements; the range is the
// rest of the tile's batch row.
template <typename T>
__device__ __forceinline__ RowStream tile_stream(const typename T::raw* x, const ChunkTile& tc, int L, int H,
                                                 int D, int hh, int sub_off) {
  const int64_t base = (tc.row0 * H + tc.hbase) * D;
  const int hl = tc.hbase + hh < H ? hh : H - 1 - tc.hbase;
  return make_row_stream(x + base, (int64_t(L - tc.t0) * H - tc.hbase) * D * T::bytes,
                         (hl * D + sub_off) * T::bytes);
}

// Store a lane's DPL consecutive elements (bf16 pairs packed into dwords).
template <typename T, int DPL>
__device__ __forceinline__ void store_row(typename T::raw* p, const float (&x)[DPL]) {
  if constexpr (T::bytes == 2) {
    uint32_t u[DPL / 2];
#pragma unroll
    for (int i = 0; i < DPL / 2; ++i) u[i] = pack_bf16x2(x[2 * i], x[2 * i + 1]);
    if constexpr (DPL == 8) {
      *reinterpret_cast<uint4*>(p) = make_uint4(u[0], u[1], u[2], u[3]);
    } else if constexpr (DPL == 4) {
      *reinterpret_cast<uint2*>(p) = make_uint2(u[0], u[1]);
    } else {
#pragma unroll
      for (int i = 0; i < DPL / 2; ++i) reinterpret_cast<uint32_t*>(p)[i] = u[i];
    }
  } else {
    if constexpr (DPL % 4 == 0) {
#pragma unroll
      for (int i = 0; i < DPL / 4; ++i)
        reinterpret_cast<float4*>(p)[i] = make_float4(x[4 * i], x[4 * i + 1], x[4 * i + 2], x[4 * i + 3]);
    } else {
#pragma unroll
      for (int i = 0; i < DPL; ++i) p[i] = x[i];
    }
  }
}

// The same slice stored through a row stream at scalar byte offset soff.
template <typename T, int DPL>
__device__ __forceinline__ void store_row(const RowStream& s, int soff, const float (&x)[DPL]) {
  using u32x4 = __attribute__((ext_vector_type(4))) unsigned int;
  using u32x2 = __attribute__((ext_vector_type(2))) unsigned int;
  if constexpr (T::bytes == 2) {
    uint32_t u[DPL / 2];
#pragma unroll
    for (int i = 0; i < DPL / 2; ++i) u[i] = pack_bf16x2(x[2 * i], x[2 * i + 1]);
    if constexpr (DPL == 8) {
      __builtin_amdgcn_raw_buffer_store_b128(u32x4{u[0], u[1], u[2], u[3]}, s.rs, s.voff, soff, 0);
    } else if constexpr (DPL == 4) {
      __builtin_amdgcn_raw_buffer_store_b64(u32x2{u[0], u[1]}, s.rs, s.voff, soff, 0);
    } else {
#pragma unroll
      for (int i = 0; i < DPL / 2; ++i) __builtin_amdgcn_raw_buffer_store_b32(u[i], s.rs, s.voff + 4 * i, soff, 0);
    }
  } else {
    static_assert(DPL % 4 == 0, "fp32 slices are whole 16-byte vectors");
#pragma unroll
    for (int i = 0; i < DPL / 4; ++i)
      __builtin_amdgcn_raw_buffer_store_b128(
          u32x4{__float_as_uint(x[4 * i]), __float_as_uint(x[4 * i + 1]), __float_as_uint(x[4 * i + 2]),
                __float_as_uint(x[4 * i + 3])},
          s.rs, s.voff + 16 * i, soff, 0);
  }
}

// The tile stream of a per-head tensor (B, L, H / R, D) read by virtual heads:
// with state_dim N = 2 R each head's R complex state rows are scanned as R
// consecutive virtual heads (H counts them) that share the head's k rows.
template <typename T>
__device__ __forceinline__ RowStream tile_stream_rows(const typename T::raw* x, const ChunkTile& tc, int L, int H, int R,
                                                      int D, int hh, int sub_off) {
  const int Hk = H / R;
  const int hv = min(tc.hbase + hh, H - 1);  // this lane's virtual head, clamped into the tensor
  return make_row_stream(x + tc.row0 * Hk * D, int64_t(L - tc.t0) * Hk * D * T::bytes,
                         ((hv / R) * D + sub_off) * T::bytes);
}

__device__ __forceinline__ ChunkTile decode_tile(int L, int Q, int NC, int n_hg, int HPW) {
  ChunkTile c;
  int g = blockIdx.x;
  const int hg = g % n_hg;
  g /= n_hg;
  c.chunk = g % NC;
  c.b = g / NC;
  c.hbase = hg * HPW;
  c.t0 = c.chunk * Q;
  c.nt = min(Q, L - c.t0);
  c.row0 = int64_t(c.b) * L + c.t0;
  return c;
}


// x *= y (complex)
__device__ __forceinline__ void cmul_acc(float& xr, float& xi, float yr, float yi) {
  const float nr = xr * yr - xi * yi;
  xi = xr * yi + xi * yr;
  xr = nr;
}

// ---------------------------------------------------------------------------
// Forward workspace layout shared by the forward and the backward (float2
// units): entering states (B, NC, H, D), chunk rotations (B, NC, H), carry
// segment maps (B, H, S) and (B, H, S, D), a pad to 16 bytes, the training
// forward's per-token records (B, L, H, 2) float4 and (B, L, H) float2, then
// the one-pass forward's look-back area over segments of kOnePassW chunks:
// segment maps (B, NSEG, H, D), leaving states (B, NSEG, H, D), segment
// rotations (B, NSEG, H) and flags (B, NSEG, H) (8-byte words); then, written
// by the training forward for the backward, the local state z_{t-1} at every
// kZck-th token t of each chunk (B, NC, H, NCK, D) and the decay-free
// correction state after each chunk's last step (B, NC, H, D).
// ---------------------------------------------------------------------------
// Complex rows of the z checkpoints, element idx = ((b, chunk, h) * NCK +
// slot) * D + d: fp32 pairs for fp32 inputs; for bf16 inputs bf16 pairs, (re,
// im) in one dword, in the first half of the region -- the precision the
// reference keeps its saved local states in (intra_chunk_scan.cu:588-589).
template <typename T, int N>
__device__ __forceinline__ void store_zck(float2* base, int64_t idx, const float (&re)[N], const float (&im)[N]) {
  if constexpr (T::bytes == 2) {
    uint32_t* p = reinterpret_cast<uint32_t*>(base) + idx;
    if constexpr (N % 4 == 0) {
#pragma unroll
      for (int j = 0; j < N; j += 4)
        *reinterpret_cast<uint4*>(p + j) = make_uint4(pack_bf16x2(re[j], im[j]), pack_bf16x2(re[j + 1], im[j + 1]),
                                                      pack_bf16x2(re[j + 2], im[j + 2]),
                                                      pack_bf16x2(re[j + 3], im[j + 3]));
    } else {
#pragma unroll
      for (int j = 0; j < N; ++j) p[j] = pack_bf16x2(re[j], im[j]);
    }
  } else {
#pragma unroll
    for (int j = 0; j < N; ++j) base[idx + j] = make_float2(re[j], im[j]);
  }
}
template <typename T, int N>
__device__ __forceinline__ void load_zck(const float2* base, int64_t idx, float2 (&out)[N]) {
  if constexpr (T::bytes == 2) {
    const uint32_t* p = reinterpret_cast<const uint32_t*>(base) + idx;
#pragma unroll
    for (int j = 0; j < N; ++j) {
      const uint32_t u = p[j];
      out[j] = make_float2(__uint_as_float(u << 16), __uint_as_float(u & 0xffff0000u));
    }
  } else {
#pragma unroll
    for (int j = 0; j < N; ++j) out[j] = base[idx + j];
  }
}

constexpr int kSegLen = 16;   // chunks per forward carry segment
constexpr int kOnePassW = 4;  // chunks (waves) per workgroup of the one-pass forward
constexpr int kCtlWords = 8;  // 8-byte words of a look-back area's control block
constexpr int kZck = 8;       // token interval of the z checkpoints
constexpr int kTokRound = 8;  // token loops run to round_up(tokens, kTokRound)

struct FwdLayout {
  int NC, S, NSEG, NCK;
  int64_t n_summ, n_gam, n_segA, n_segX, n_pad, n_saved, n_gsaved, n_op, n_zck, n_cend, n_ycorr;
  int64_t total() const {
    return n_summ + n_gam + n_segA + n_segX + n_pad + n_saved + n_gsaved + n_op + n_zck + n_cend + n_ycorr;
  }
  int64_t ycorr_offset() const { return cend_offset() + n_cend; }
  int64_t saved_offset() const { return n_summ + n_gam + n_segA + n_segX + n_pad; }
  int64_t gsaved_offset() const { return saved_offset() + n_saved; }
  int64_t onepass_offset() const { return gsaved_offset() + n_gsaved; }
  int64_t zck_offset() const { return onepass_offset() + n_op; }
  int64_t cend_offset() const { return zck_offset() + n_zck; }
};

// The one-pass forward's look-back folds two levels: every kFwdGroup-th
// segment publishes the composed map of its group of kFwdGroup segments, and
// the state entering a segment is folded from its anchor (every kFwdAnchor
// segments, a multiple of kFwdGroup) over the maps of the whole groups since
// the anchor, then over the maps of its own group's earlier segments.
// A segment at most kFwdDirect segments past its anchor folds the segment
// maps directly (no wait on a group map); group ends compose their group's
// map only where a later segment reads it.
constexpr int kFwdGroup = 8;
constexpr int kFwdAnchor = 64;
constexpr int kFwdDirect = 2 * kFwdGroup - 1;
static_assert(kFwdAnchor % kFwdGroup == 0, "anchors start groups");
__host__ __device__ constexpr int fwd_groups(int nseg) { return (nseg + kFwdGroup - 1) / kFwdGroup; }
// Whether some segment folds the map of group g (segments kFwdGroup g ..
// kFwdGroup g + kFwdGroup - 1): one past the group, more than kFwdDirect
// past its anchor, in the same anchor window, before NSEG.
__host__ __device__ constexpr bool fwd_group_read(int g, int nseg) {
  return (g * kFwdGroup + kFwdGroup > (g * kFwdGroup / kFwdAnchor) * kFwdAnchor + kFwdDirect + 1
              ? g * kFwdGroup + kFwdGroup
              : (g * kFwdGroup / kFwdAnchor) * kFwdAnchor + kFwdDirect + 1) <= nseg - 1;
}

inline FwdLayout fwd_layout(int64_t B, int64_t L, int64_t H, int64_t D, int64_t chunk) {
  FwdLayout w;
  w.NC = int((L + chunk - 1) / chunk);
  w.S = (w.NC + kSegLen - 1) / kSegLen;
  w.n_summ = B * w.NC * H * D;
  w.n_gam = B * w.NC * H;
  w.n_segA = B * H * w.S;
  w.n_segX = B * H * w.S * D;
  w.n_pad = (w.n_summ + w.n_gam + w.n_segA + w.n_segX) & 1;
  w.n_saved = 4 * B * L * H;
  w.n_gsaved = B * L * H;
  w.NSEG = (w.NC + kOnePassW - 1) / kOnePassW;
  // maps, leaving states, rotations, flags, the control block, then the group maps of the two-level fold
  w.n_op = B * w.NSEG * H * (2 * D + 2) + kCtlWords + B * int64_t(fwd_groups(w.NSEG)) * H * (D + 1);
  // checkpoints at t = 0, kZck, ... < round_up(chunk, kTokRound)
  w.NCK = int((chunk + kTokRound - 1) / kTokRound * kTokRound / kZck);
  w.n_zck = B * w.NC * H * int64_t(w.NCK) * D;
  w.n_cend = B * w.NC * H * D;
  w.n_ycorr = B * L * H;  // the chunked correction's readout (four-launch path with the MFMA correction)
  return w;
}

// ---------------------------------------------------------------------------
// Scan-level Cayley dynamics for one eigenvalue pair (reference:
// dynamics_fused.cu:109-131, cayley_math.cuh:51-99):
//   tau = dt/2, ta = tau*max(alpha,0), tw = tau*omega,
//   mu  = ((1 - ta^2 - tw^2) + i 2 tw) / ((1+ta)^2 + tw^2 + 1e-6),
//   E   = max(((1-ta)^2 + tw^2) / ((1+ta)^2 + tw^2 + 1e-6), 1e-8),
//   A   = conj(mu) * E^((c r - 1)/2),
//   vp  = min(sqrt(max(1 - E^(c r), 1e-6)), 1).
// Powers use the hardware base-2 log/exp (v_log_f32 / v_exp_f32); E >= 1e-8
// keeps the log argument normal.
// ---------------------------------------------------------------------------

struct Transition {
  float ar, ai, vp;
};

__device__ __forceinline__ Transition cayley_gated(float dt, float r, float alpha, float omega, float c) {
  const float tau = 0.5f * dt;
  const float ta = tau * fmaxf(alpha, 0.0f);
  const float tw = tau * omega;
  const float tw2 = tw * tw;
  const float opa = 1.0f + ta;
  const float oma = 1.0f - ta;
  const float den = opa * opa + tw2 + 1e-6f;
  const float inv = __builtin_amdgcn_rcpf(den);  // den >= 1
  const float mur = (1.0f - ta * ta - tw2) * inv;
  const float mui = (2.0f * tw) * inv;
  const float E = fmaxf((oma * oma + tw2) * inv, 1e-8f);
  const float cr = c * r;
  const float lE = __builtin_amdgcn_logf(E);
  const float scale = __builtin_amdgcn_exp2f(0.5f * (cr - 1.0f) * lE);
  const float eff = __builtin_amdgcn_exp2f(cr * lE);
  Transition o;
  o.ar = mur * scale;
  o.ai = -mui * scale;
  o.vp = fminf(__builtin_amdgcn_sqrtf(fmaxf(1.0f - eff, 1e-6f)), 1.0f);
  return o;
}

// ---------------------------------------------------------------------------
// Segment look-back between the workgroups of a one-launch pass.
// ---------------------------------------------------------------------------
constexpr int kLookbackBatch = 8;
constexpr int kAnchor = 63;  // segments folded from one anchor state (<= 63: one watch window)
constexpr uint64_t kSpinTicks = 5000000;  // look-back wait bound: 50 ms of the 100 MHz real-time counter

// Look-back area of a one-launch pass: per (b, segment, head) a map (D
// complex + one complex scalar), a state (D complex) and an 8-byte flag, then
// a control block of kCtlWords 8-byte words whose first word is the call's
// epoch and second a count of workgroups.  The area is never cleared: a flag
// counts only when its upper bits equal the epoch of the running call, which
// a one-thread kernel launched just before the pass draws from a device-side
// counter and writes into the control block, or, for the *_continue calls,
// the previous call left there (arrive_and_draw_next_epoch).  Drawing it on
// the device keeps a captured HIP graph correct: every replay gets a new
// epoch.
struct OnePassBufs {
  float2* seg_f;             // (B, NSEG, H, D) segment map F: state at the segment's end from zero
  float2* seg_s;             // (B, NSEG, H, D) state leaving the segment
  float2* seg_g;             // (B, NSEG, H)    segment rotation product
  unsigned long long* flag;  // (B, NSEG, H); entry hbase serves the head group
  unsigned long long* ctl;   // kCtlWords words; ctl[0] = epoch of the running call
  // forward only (two-level fold): (B, NGRP, H, D) group map F and (B, NGRP, H) its rotation product
  float2* grp_f = nullptr;
  float2* grp_g = nullptr;
};

// Epoch words: the pass's tag in bits 58..59 (so epochs of different passes
// never match each other's flags, should their areas share memory over time)
// and the count of calls so far in bits 0..57.  A flag word is epoch << 2 | state.
__device__ __forceinline__ unsigned long long epoch_word(unsigned tag, unsigned long long n) {
  return (static_cast<unsigned long long>(tag) << 58) | (n & ((1ull << 58) - 1ull));
}
__device__ __forceinline__ unsigned long long load_epoch(const unsigned long long* ctl) {
  return __hip_atomic_load(const_cast<unsigned long long*>(ctl), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// The epoch of the next call on the same look-back area is drawn by the last
// workgroup of a one-launch pass to have read this call's.  Each workgroup
// reads ctl[0] once, at entry, and after it has published its first flag
// (which used that epoch) one thread counts the workgroup in ctl[1]; the one
// whose count completes a multiple of the grid size resets the count and
// stores a new epoch, drawn from the pass's call counter, into ctl[0].  Every
// workgroup of the call holds its epoch by then, so the store can come
// mid-pass, off the kernel's tail.  Counting modulo the grid size elects
// exactly one workgroup whatever ctl[1] held before.  A caller whose previous
// use of the workspace was a call of the same pass and shape can then skip the
// epoch kernel (the *_continue entry points); a captured graph of such calls
// leaves a new epoch after every replay.
__device__ __forceinline__ void arrive_and_draw_next_epoch(unsigned long long* ctl, unsigned long long* calls,
                                                           unsigned tag) {
  const unsigned long long g = gridDim.x;
  const unsigned long long old = __hip_atomic_fetch_add(ctl + 1, 1ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  if ((old + 1ull) % g == 0ull) {
    const unsigned long long n = __hip_atomic_fetch_add(calls, 1ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) + 1ull;
    __hip_atomic_store(ctl + 1, 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __hip_atomic_store(ctl, epoch_word(tag, n), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
}
// Bits of the sticky look-back status word (cdssm_lookback_status).
constexpr unsigned kTimeoutFwd = 1u;  // a one-pass forward wait timed out (NaN states were written)
constexpr unsigned kTimeoutBwd = 2u;  // a one-launch backward carry wait timed out

// Wait until this wave's earlier stores are acknowledged; also a compiler
// barrier, so no memory access moves across it.
__device__ __forceinline__ void wait_stores_acked() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

__device__ __forceinline__ void st_agent(float2* p, float2 v) {
  __hip_atomic_store(reinterpret_cast<unsigned long long*>(p), __builtin_bit_cast(unsigned long long, v),
                     __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float2 ld_agent(const float2* p) {
  const unsigned long long x = __hip_atomic_load(
      reinterpret_cast<unsigned long long*>(const_cast<float2*>(p)), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  return __builtin_bit_cast(float2, x);
}

}  // namespace cdssm

// ---------------------------------------------------------------------------
// Host-side status plumbing shared by the C-ABI entry points.
// ---------------------------------------------------------------------------

namespace cdssm_host {
void set_error(const char* fmt, ...);
int check_launch(const char* op);
// Sticky look-back timeout words of the forward and backward units (bits
// kTimeoutFwd / kTimeoutBwd) on the current device; `clear` resets them.
// Synchronous (device-to-host copies).
int fwd_lookback_status(bool clear, unsigned* out);
int bwd_lookback_status(bool clear, unsigned* out);
// Workgroups of kernel `fn` (block threads, lds bytes of dynamic LDS) resident
// on the current device at once; 0 if it cannot run.  Cached.
int resident_capacity(const void* fn, int block, size_t lds);
// Compute units of the current device (0 if it cannot be read).  Cached.
int device_cus();
// Launch-path selection of the fused scan (forward and backward carry):
// automatic, always the multi-launch passes, or one launch required.
// kPathSweep: the four launches with the correction as the chunked MFMA pass
// (bf16 inference forward, chunk a multiple of 16 up to 128; for measurement).
enum { kPathAuto = 0, kPathFour = 1, kPathOne = 2, kPathSweep = 3 };
int scan_path();
// Wide staging loads in the one-pass inference forward (off with CDSSM_NARROW_STAGING set; for measurement).
bool wide_staging();
}  // namespace cdssm_host

// Status codes returned by every entry point.
#define CDSSM_OK 0
#define CDSSM_EINVAL (-1)
#define CDSSM_EHIP (-2)
