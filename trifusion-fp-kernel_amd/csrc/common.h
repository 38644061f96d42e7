// Device helpers shared by the gfx950 kernels: dtype-generic loads/stores,
// round-to-nearest-even conversions, wave64 reductions and scans, and the
// fast transcendentals used by the recurrence.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "trifusion_amd.h"

namespace tf {

constexpr float kLog2e = 1.44269504089f;  // rounded log2(e) the recurrence scales adt by
constexpr float kPi = 3.141592653589793f;
constexpr float kTwoPi = 6.283185307179586f;
constexpr float kInvTwoPi = 0.15915494309189535f;

__device__ __forceinline__ float bf16_to_f32(uint16_t b) {
  return __uint_as_float(static_cast<uint32_t>(b) << 16);
}

// fp32 -> bf16 bits, round to nearest even (gfx950 v_cvt_pk_bf16_f32).
__device__ __forceinline__ uint16_t f32_to_bf16(float x) {
  return __builtin_bit_cast(uint16_t, static_cast<__bf16>(x));
}

__device__ __forceinline__ float round_bf16(float x) { return bf16_to_f32(f32_to_bf16(x)); }

__device__ __forceinline__ float round_f16(float x) {
  return static_cast<float>(static_cast<_Float16>(x));
}

// Round an fp32 value to `dtype` and back (identity for fp32).
__device__ __forceinline__ float round_to(float x, int dtype) {
  if (dtype == TF_BFLOAT16) return round_bf16(x);
  if (dtype == TF_FLOAT16) return round_f16(x);
  return x;
}

__device__ __forceinline__ float load_f32(const void* p, int dtype, int64_t i) {
  if (dtype == TF_BFLOAT16) return bf16_to_f32(static_cast<const uint16_t*>(p)[i]);
  if (dtype == TF_FLOAT16) return static_cast<float>(static_cast<const _Float16*>(p)[i]);
  return static_cast<const float*>(p)[i];
}

__device__ __forceinline__ void store_f32(void* p, int dtype, int64_t i, float x) {
  if (dtype == TF_BFLOAT16) {
    static_cast<uint16_t*>(p)[i] = f32_to_bf16(x);
  } else if (dtype == TF_FLOAT16) {
    static_cast<_Float16*>(p)[i] = static_cast<_Float16>(x);
  } else {
    static_cast<float*>(p)[i] = x;
  }
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

__device__ __forceinline__ float sigmoidf(float x) { return 1.0f / (1.0f + __expf(-x)); }

// Mamba-3 discretisation controls of one step from the raw in-projection
// columns (src/trifusion_l4/kernels/primitives.py:209-214): the step
// dt = softplus(ddt + bias), linear above 20, and the signed decay
// adt = min(-(relu(a) + 1/(1 - min(a, 0))), -floor) * dt. Shared by the
// controls kernel and the recurrence's raw-controls prologue, so both give
// the same bits.
__device__ __forceinline__ float softplus_le20(float v);

__device__ __forceinline__ float control_step(float ddt, float bias) {
  const float v = ddt + bias;
  return v > 20.f ? v : softplus_le20(v);
}

__device__ __forceinline__ float control_decay(float a, float step, float floor_) {
  return fminf(-(fmaxf(a, 0.f) + __builtin_amdgcn_rcpf(1.f - fminf(a, 0.f))), -floor_) * step;
}

// softplus(v) = log(1 + e^v) for v <= 20 from the hardware exp2, log2 and
// reciprocal (each within about 1 ulp), a few ulp in all:
//   e^v = 2^h (1 + l ln 2) with h + l = v log2(e): h = v L1 rounded, l its
//   rounding error (one fma) plus v L2, where L1 + L2 = log2(e) to 2^-48;
//   log(1 + x) = x log(u) / (u - 1) with u = 1 + x rounded, and x itself when
//   u == 1 (W. Kahan's identity: D. Goldberg, "What every computer scientist
//   should know about floating-point arithmetic", ACM Computing Surveys 23(1),
//   1991, Theorem 4).
// Below -104, e^v is under half the least fp32 subnormal, so the result is 0
// (also at v = -inf, where the split of v log2(e) would form -inf + inf).
__device__ __forceinline__ float softplus_le20(float v) {
  constexpr float kL1 = 1.4426950216293335f;     // log2(e) rounded to float
  constexpr float kL2 = 1.925963033500011e-08f;  // log2(e) - kL1
  constexpr float kLn2 = 0.6931471824645996f;
  const float h = v * kL1;
  const float l = __builtin_fmaf(v, kL1, -h) + v * kL2;
  const float e0 = __builtin_amdgcn_exp2f(h);
  const float x = __builtin_fmaf(e0, l * kLn2, e0);
  const float u = 1.f + x;
  const float r = (__builtin_amdgcn_logf(u) * kLn2) * (x * __builtin_amdgcn_rcpf(u - 1.f));
  return v < -104.f ? 0.f : (u == 1.f ? x : r);
}

// x - 2pi*floor(x/2pi), the reduction the reference applies to phases.
__device__ __forceinline__ float mod_two_pi(float x) {
  return x - kTwoPi * floorf(x / kTwoPi);
}

constexpr double kPiD = 3.141592653589793;
constexpr double kTwoPiD = 6.283185307179586;

__device__ __forceinline__ double mod_two_pi_d(double x) {
  return x - kTwoPiD * floor(x / kTwoPiD);
}

// Wave64 sum via xor shuffles (every lane receives the total).
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}

// Inclusive prefix sum across the 64 lanes of a wave (Hillis-Steele).
__device__ __forceinline__ float wave_inclusive_scan(float v) {
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    float o = __shfl_up(v, off, 64);
    if (lane >= off) v += o;
  }
  return v;
}

// Typed element wrappers for the bandwidth kernels.
struct bf16_t {
  uint16_t bits;
};
using f16_t = _Float16;

__device__ __forceinline__ float to_f32(float x) { return x; }
__device__ __forceinline__ float to_f32(bf16_t x) { return bf16_to_f32(x.bits); }
__device__ __forceinline__ float to_f32(f16_t x) { return static_cast<float>(x); }

template <typename T>
__device__ __forceinline__ T from_f32(float x);
template <>
__device__ __forceinline__ float from_f32<float>(float x) { return x; }
template <>
__device__ __forceinline__ bf16_t from_f32<bf16_t>(float x) { return bf16_t{f32_to_bf16(x)}; }
template <>
__device__ __forceinline__ f16_t from_f32<f16_t>(float x) { return static_cast<f16_t>(x); }

// Calls BODY with `T` bound to the element type of dtype code `code`.
#define TF_DISPATCH(code, T, ...)                       \
  switch (code) {                                       \
    case TF_FLOAT32: {                                  \
      using T = float;                                  \
      __VA_ARGS__;                                      \
    } break;                                            \
    case TF_BFLOAT16: {                                 \
      using T = ::tf::bf16_t;                           \
      __VA_ARGS__;                                      \
    } break;                                            \
    case TF_FLOAT16: {                                  \
      using T = ::tf::f16_t;                            \
      __VA_ARGS__;                                      \
    } break;                                            \
    default:                                            \
      return TF_ERR_DTYPE;                              \
  }

inline bool dtype_ok(int d) { return d == TF_FLOAT32 || d == TF_BFLOAT16 || d == TF_FLOAT16; }

inline int dtype_size(int d) { return d == TF_FLOAT32 ? 4 : 2; }

inline int launch_status() {
  return hipGetLastError() == hipSuccess ? TF_OK : TF_ERR_LAUNCH;
}

}  // namespace tf
