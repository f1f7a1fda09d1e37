// Shared device helpers and C-ABI error plumbing for the MI355X (gfx950) MoE
// kernels. Everything here is written for CDNA4: 64-lane wavefronts, the OCP
// e4m3 conversion instructions of gfx950 and its fp8 MFMA.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/mlops_mi355x.h"

#define MI355X_WAVE 64

typedef int v8i __attribute__((ext_vector_type(8)));
typedef float v4f __attribute__((ext_vector_type(4)));

// ---------------------------------------------------------------- errors
// Host-side: a thread-local message for the last failing entry point.
void mi355x_set_error(const char* fmt, ...);

#define MI355X_REQUIRE(cond, ...)                 \
  do {                                            \
    if (!(cond)) {                                \
      mi355x_set_error(__VA_ARGS__);              \
      return MI355X_EINVAL;                       \
    }                                             \
  } while (0)

#define MI355X_LAUNCH_CHECK()                                              \
  do {                                                                     \
    hipError_t _e = hipGetLastError();                                     \
    if (_e != hipSuccess) {                                                \
      mi355x_set_error("kernel launch failed: %s", hipGetErrorString(_e)); \
      return MI355X_ELAUNCH;                                               \
    }                                                                      \
  } while (0)

// ---------------------------------------------------------------- numbers
static constexpr float kE4M3Max = 448.0f;
// The row quantizer's descale is amax times the fp32-rounded reciprocal of
// 448 (a multiply, not a division); the weight-block quantizer divides.
static constexpr float kInv448 = 1.0f / 448.0f;
static constexpr float kMinScale = 1e-12f;

__device__ __forceinline__ float bf16_to_f32(uint16_t v) {
  return __uint_as_float(((uint32_t)v) << 16);
}

// fp32 -> bf16 with gfx950's v_cvt_pk_bf16_f32: round to nearest even, what
// torch's .to(bfloat16) does for every non-NaN value (NaNs stay NaN).
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));

__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  const f32x2_t v = {lo, hi};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2_t));
}

// Streaming 16-byte store (non-temporal): for GEMM outputs, which are far
// larger than L2 and are not re-read by the kernel writing them; keeps them
// from evicting the operand panels other workgroups are about to read.
typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));
__device__ __forceinline__ void store_stream(void* p, uint4 v) {
  __builtin_nontemporal_store((u32x4_t){v.x, v.y, v.z, v.w}, (u32x4_t*)p);
}

// Streaming 16-byte load (non-temporal): for inputs read exactly once, so
// they do not displace cached data (combine / token sum: 5.2 -> 6.2 TB/s).
__device__ __forceinline__ uint4 load_stream(const void* p) {
  const u32x4_t v = __builtin_nontemporal_load((const u32x4_t*)p);
  return make_uint4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ void store_stream8(void* p, uint2 v) {
  typedef unsigned int u32x2_t __attribute__((ext_vector_type(2)));
  __builtin_nontemporal_store((u32x2_t){v.x, v.y}, (u32x2_t*)p);
}

__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
  return (uint16_t)(pack_bf16x2(f, 0.0f) & 0xffffu);
}

// OCP e4m3 (float8_e4m3fn) encode of two values with gfx950's converter:
// round-to-nearest-even, matching torch's cast for finite inputs in range.
// Returns the two bytes in the low 16 bits (lo first).
__device__ __forceinline__ uint32_t f32x2_to_e4m3(float lo, float hi) {
  return (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(lo, hi, __float_as_int(lo), false) & 0xffffu;
}

// Four values divided by a power-of-two descale and encoded e4m3 by gfx950's
// scaled converter (v_cvt_scalef32_pk_fp8_f32: e4m3(x / scale), RNE). For a
// power-of-two scale the quotient is exact, so this equals multiplying by
// 1 / scale and converting (checked bit for bit on MI355X over 4M pairs,
// e4m3 subnormals included). It does not saturate: callers guarantee
// |x / scale| <= 448, which holds for bf16 x and scale = pow2_ceil(amax / 448).
typedef short v2i16_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t f32x4_to_e4m3_pow2(float a, float b, float c, float d,
                                                      float scale) {
  // The first conversion writes the low half and the second the high half,
  // so the destination's prior contents never matter: it starts as a's bits
  // (a register the first conversion can take over, where a zero would need
  // a move).
  v2i16_t w = __builtin_amdgcn_cvt_scalef32_pk_fp8_f32(
      __builtin_bit_cast(v2i16_t, a), a, b, scale, false);
  w = __builtin_amdgcn_cvt_scalef32_pk_fp8_f32(w, c, d, scale, true);
  return __builtin_bit_cast(uint32_t, w);
}

__device__ __forceinline__ uint32_t f32x4_to_e4m3(float a, float b, float c, float d) {
  int w = __builtin_amdgcn_cvt_pk_fp8_f32(a, b, __float_as_int(a), false);  // see above
  w = __builtin_amdgcn_cvt_pk_fp8_f32(c, d, w, true);
  return (uint32_t)w;
}

__device__ __forceinline__ float e4m3_to_f32(uint32_t byte) {
  return __builtin_amdgcn_cvt_f32_fp8((int)byte, 0);
}

// Quantize one value given its descale: IEEE division, clip to +-448.
// Smallest power of two >= x (x positive, normal): the descale of an operand
// the MFMA scales in hardware (E8M0 = the fp32 biased exponent byte).
__device__ __forceinline__ float pow2_ceil(float x) {
  uint32_t b = __float_as_uint(x);
  if (b & 0x7fffffu) b = (b & 0x7f800000u) + 0x800000u;
  return __uint_as_float(b);
}

__device__ __forceinline__ float quant_div(float x, float scale) {
  float q = x / scale;
  return fminf(fmaxf(q, -kE4M3Max), kE4M3Max);
}

// x / scale, correctly rounded like the division above, for many x sharing
// one scale: with inv = RN(1 / scale) (one IEEE division per scale),
// q0 = RN(x inv), the residual e = x - scale q0 is exact (FMA) and
// RN(q0 + e inv) = RN(x / scale) (Markstein) for quotients that neither
// overflow nor underflow, which covers every quotient that reaches a nonzero
// e4m3 value.
// No clip to +-448: every caller's scale is max(amax * RN(1/448), 1e-12) or
// max(amax / 448, 1e-12) over a group holding x, so |x / scale| <=
// 448 (1 + 2^-22) < 464, which round-to-nearest e4m3 takes to 448 (the clip
// of the division form above would not change it), and a NaN or infinite x
// stays NaN, as the reference's clamp-then-cast leaves it.
__device__ __forceinline__ float quant_div_inv(float x, float scale, float inv) {
  const float q0 = x * inv;
  const float e = fmaf(-scale, q0, x);
  return fmaf(e, inv, q0);
}

// SwiGLU clamp (limit <= 0: none): gate from above, up on both sides.
__device__ __forceinline__ void clamp_gate_up(float& g, float& u, float limit) {
  if (limit > 0.0f) {
    g = fminf(g, limit);
    u = fminf(fmaxf(u, -limit), limit);
  }
}
// sigmoid / silu with the hardware exp and reciprocal (v_exp_f32, v_rcp_f32,
// 1 ulp) instead of an IEEE division: these run per element in the SwiGLU
// passes, which are ALU-bound on them.
__device__ __forceinline__ float sigmoid_f(float g) {
  return __builtin_amdgcn_rcpf(1.0f + __expf(-g));
}
__device__ __forceinline__ float silu_f(float g) { return g * sigmoid_f(g); }

// Eight bf16 values from one 16-byte load (or from its bits), as fp32.
__device__ __forceinline__ void load_bf16x8(const uint16_t* p, float* v) {
  uint4 r = *(const uint4*)p;
  uint32_t w4[4] = {r.x, r.y, r.z, r.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    v[2 * i] = bf16_to_f32(w4[i] & 0xffff);
    v[2 * i + 1] = bf16_to_f32(w4[i] >> 16);
  }
}

__device__ __forceinline__ void unpack_bf16x8(uint4 r, float* v) {
  const uint32_t w4[4] = {r.x, r.y, r.z, r.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    v[2 * i] = bf16_to_f32(w4[i] & 0xffff);
    v[2 * i + 1] = bf16_to_f32(w4[i] >> 16);
  }
}

__device__ __forceinline__ uint2 quant8(const float* v, float s, float inv) {
  uint32_t lo = f32x4_to_e4m3(quant_div_inv(v[0], s, inv), quant_div_inv(v[1], s, inv),
                              quant_div_inv(v[2], s, inv), quant_div_inv(v[3], s, inv));
  uint32_t hi = f32x4_to_e4m3(quant_div_inv(v[4], s, inv), quant_div_inv(v[5], s, inv),
                              quant_div_inv(v[6], s, inv), quant_div_inv(v[7], s, inv));
  return make_uint2(lo, hi);
}
__device__ __forceinline__ uint2 quant8(const float* v, float s) { return quant8(v, s, 1.0f / s); }

// ---------------------------------------------------------------- waves
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  return v;
}
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}
// Exclusive prefix over experts of their padded 128-row block counts,
// ceil(rows_e / 128), into ptile[0..experts] (ptile[experts] = total), for a
// block of THREADS threads: a 64-lane scan per wave plus one pass over the
// wave totals per THREADS experts. wsum: THREADS / 64 ints of scratch.
template <int THREADS>
__device__ inline void padded_block_prefix(const int32_t* __restrict__ offsets, int experts,
                                           int* ptile, int* wsum) {
  constexpr int kWaves = THREADS / 64;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  int carry = 0;
  for (int base = 0; base < experts; base += THREADS) {
    const int e = base + tid;
    const int v = e < experts ? (offsets[e + 1] - offsets[e] + 127) >> 7 : 0;
    int x = v;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      const int y = __shfl_up(x, o, 64);
      if (lane >= o) x += y;
    }
    if (lane == 63) wsum[wave] = x;
    __syncthreads();
    int before = 0, total = 0;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) {
      const int t = wsum[w];
      before += w < wave ? t : 0;
      total += t;
    }
    if (e < experts) ptile[e] = carry + before + x - v;
    carry += total;
    __syncthreads();
  }
  if (tid == 0) ptile[experts] = carry;
  __syncthreads();
}

// Reductions over aligned groups of W lanes (W a power of two <= 64), the
// result in every lane of the group. Within a DPP row (16 lanes) they are
// DPP moves: quad swaps [1,0,3,2] and [2,3,0,1], then the half-row mirror
// (lane i <-> 7 - i) and the row mirror (i <-> 15 - i), each pairing two
// partial results that cover disjoint lanes; every lane adds the same two
// values, so all lanes of the group hold the same sum. Wider groups finish
// with lane shuffles. A source lane that is not active returns the lane's
// own value for max and 0 for sums.
template <int kCtrl>
__device__ __forceinline__ float dpp_max_step(float v) {
  const int b = __float_as_int(v);
  return fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(b, b, kCtrl, 0xF, 0xF, false)));
}
template <int kCtrl>
__device__ __forceinline__ float dpp_sum_step(float v) {
  return v + __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), kCtrl, 0xF, 0xF,
                                                        true));
}
template <int W>
__device__ __forceinline__ float group_max(float v) {
  static_assert(W >= 2 && W <= 64 && (W & (W - 1)) == 0, "group width");
  v = dpp_max_step<0xB1>(v);
  if constexpr (W >= 4) v = dpp_max_step<0x4E>(v);
  if constexpr (W >= 8) v = dpp_max_step<0x141>(v);
  if constexpr (W >= 16) v = dpp_max_step<0x140>(v);
#pragma unroll
  for (int o = 16; o < W; o <<= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  return v;
}
template <int W>
__device__ __forceinline__ float group_sum(float v) {
  static_assert(W >= 2 && W <= 64 && (W & (W - 1)) == 0, "group width");
  v = dpp_sum_step<0xB1>(v);
  if constexpr (W >= 4) v = dpp_sum_step<0x4E>(v);
  if constexpr (W >= 8) v = dpp_sum_step<0x141>(v);
  if constexpr (W >= 16) v = dpp_sum_step<0x140>(v);
#pragma unroll
  for (int o = 16; o < W; o <<= 1) v += __shfl_xor(v, o, 64);
  return v;
}

// Maximum of non-negative, non-NaN floats (the block amax values of the
// quantizers, each a running fmaxf from 0) over aligned groups of W lanes.
// Such floats order like their bit patterns as unsigned integers, so each
// DPP step fuses into one v_max_u32 (an fmaxf step needs a copy and a
// canonicalizing max besides); a source lane that is not active reads as 0,
// the identity. W = 64 combines the four rows' results as scalars.
template <int kCtrl>
__device__ __forceinline__ uint32_t dpp_umax_step(uint32_t v) {
  return max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, kCtrl, 0xF, 0xF, true));
}
template <int W>
__device__ __forceinline__ float group_amax(float x) {
  static_assert(W >= 2 && W <= 64 && (W & (W - 1)) == 0, "group width");
  uint32_t v = __float_as_uint(x);
  v = dpp_umax_step<0xB1>(v);
  if constexpr (W >= 4) v = dpp_umax_step<0x4E>(v);
  if constexpr (W >= 8) v = dpp_umax_step<0x141>(v);
  if constexpr (W >= 16) v = dpp_umax_step<0x140>(v);
  if constexpr (W == 32) v = max(v, (uint32_t)__shfl_xor((int)v, 16, 64));
  if constexpr (W == 64) {
    const uint32_t r0 = __builtin_amdgcn_readlane((int)v, 0), r1 = __builtin_amdgcn_readlane((int)v, 16);
    const uint32_t r2 = __builtin_amdgcn_readlane((int)v, 32), r3 = __builtin_amdgcn_readlane((int)v, 48);
    v = max(max(r0, r1), max(r2, r3));
  }
  return __uint_as_float(v);
}

__device__ __forceinline__ int lane_id() { return threadIdx.x & 63; }

__device__ __forceinline__ uint64_t lanes_below() {
  int l = lane_id();
  return l == 0 ? 0ull : (~0ull >> (64 - l));
}

// Blocks are assigned to the 8 XCDs round-robin; this renumbering gives each
// XCD a contiguous run of logical tiles so neighbours share its L2.
__device__ __forceinline__ int xcd_swizzle(int bid, int nblocks) {
  const int xcds = 8;
  if (nblocks % xcds) return bid;
  int per = nblocks / xcds;
  return (bid % xcds) * per + bid / xcds;
}
