// Bandwidth kernels of the TriFusion block and front end around the fused
// recurrence: masked depthwise convolution, 4:1 masked pooling, rotary Q/K/V
// packing, the front end's channel RMSNorm and frequency bands, linear
// interpolation back to the frame grid, the evidence-gated RMSNorm and the
// sigmoid-gated concatenation. Each is one HBM pass with fp32 arithmetic; where
// the reference computes with fused multiply-add disabled, products and sums
// here are rounded on their own too.
#include "common.h"

#pragma clang fp contract(off)

namespace tf {
namespace {

constexpr int kWaves = 4;  // waves per 256-thread block

__device__ __forceinline__ int dev_len(const int64_t* lengths, int b, int T) {
  const int64_t l = lengths[b];
  return l < 0 ? 0 : (l > T ? T : static_cast<int>(l));
}

__device__ __forceinline__ float sigmoid_acc(float x) { return 1.0f / (1.0f + expf(-x)); }

// y[b, t, c] = t < L ? sum_k x[b, t + k - K/2, c] w[c, k] + bias[c] : 0, sources
// outside [0, T) read as 0 (primitives.py:_dw_forward). One block per (b, t)
// row, threads over channels.
template <typename T>
__global__ __launch_bounds__(256) void depthwise_masked_kernel(const T* __restrict__ x, const T* __restrict__ w,
                                                               const T* __restrict__ bias,
                                                               const int64_t* __restrict__ lengths,
                                                               T* __restrict__ y, int Tn, int D, int K) {
  const int64_t row = blockIdx.x;
  const int b = static_cast<int>(row / Tn);
  const int t = static_cast<int>(row - static_cast<int64_t>(b) * Tn);
  const bool valid = t < dev_len(lengths, b, Tn);
  for (int c = threadIdx.x; c < D; c += blockDim.x) {
    float acc = 0.f;
    if (valid) {
      for (int k = 0; k < K; ++k) {
        const int src = t + k - K / 2;
        const float xv = (src >= 0 && src < Tn) ? to_f32(x[(static_cast<int64_t>(b) * Tn + src) * D + c]) : 0.f;
        acc += xv * to_f32(w[static_cast<int64_t>(c) * K + k]);
      }
      acc += to_f32(bias[c]);
    }
    y[row * D + c] = from_f32<T>(valid ? acc : 0.f);
  }
}

// y[b, j, c] = sum_{k < 4, 4j + k < L} x[b, 4j + k, c] / max(min(L - 4j, 4), 1)
// (primitives.py:_pool4 forward). One block per (b, j) row.
template <typename T>
__global__ __launch_bounds__(256) void pool4_kernel(const T* __restrict__ x, const int64_t* __restrict__ lengths,
                                                    T* __restrict__ y, int Tn, int LT, int D) {
  const int64_t row = blockIdx.x;
  const int b = static_cast<int>(row / LT);
  const int j = static_cast<int>(row - static_cast<int64_t>(b) * LT);
  const int L = dev_len(lengths, b, Tn);
  const int count = max(min(L - 4 * j, 4), 1);
  for (int c = threadIdx.x; c < D; c += blockDim.x) {
    float acc = 0.f;
    for (int k = 0; k < 4; ++k) {
      const int src = 4 * j + k;
      acc += src < L ? to_f32(x[(static_cast<int64_t>(b) * Tn + src) * D + c]) : 0.f;
    }
    y[row * D + c] = from_f32<T>(acc / static_cast<float>(count));
  }
}

// x [B, T, 3 H D] -> y [3, B, H, T, D]; q and k rotated by interleaved pairs,
// (a, z) -> (a cos - z sin, a sin + z cos), cos/sin [T, D/2] fp32; v copied
// (primitives.py:_rotary_qkv forward). One thread per output pair.
template <typename T>
__global__ __launch_bounds__(256) void rotary_qkv_kernel(const T* __restrict__ x, const float* __restrict__ cs,
                                                         const float* __restrict__ sn, T* __restrict__ y, int B,
                                                         int Tn, int H, int D, int64_t pairs) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= pairs) return;
  const int hd = D / 2;
  const int c = static_cast<int>(i % hd);
  const int64_t r1 = i / hd;
  const int t = static_cast<int>(r1 % Tn);
  const int64_t r2 = r1 / Tn;
  const int h = static_cast<int>(r2 % H);
  const int64_t r3 = r2 / H;
  const int b = static_cast<int>(r3 % B);
  const int qkv = static_cast<int>(r3 / B);
  const int64_t src = ((static_cast<int64_t>(b) * Tn + t) * (3 * H) + qkv * H + h) * D + 2 * c;
  const float a = to_f32(x[src]), z = to_f32(x[src + 1]);
  float u = a, v = z;
  if (qkv < 2) {
    const float co = cs[static_cast<int64_t>(t) * hd + c], si = sn[static_cast<int64_t>(t) * hd + c];
    u = a * co - z * si;
    v = a * si + z * co;
  }
  y[2 * i] = from_f32<T>(u);
  y[2 * i + 1] = from_f32<T>(v);
}

// Channel RMSNorm of the front end's [B, C, T, F] maps (any strides), written
// as [B, T, F, C]: rows t >= L are 0; y = round(x r w) and, with silu, y * sigmoid(y)
// (primitives.py:_front_norm). One wave per (b, t, f) row, C <= 256.
template <typename T>
__global__ __launch_bounds__(256) void front_norm_kernel(const T* __restrict__ x, const float* __restrict__ w,
                                                         const int64_t* __restrict__ lengths, T* __restrict__ y,
                                                         int Tn, int F, int C, int64_t rows, int64_t sb,
                                                         int64_t sc, int64_t st, int64_t sf, float eps, int silu) {
  const int lane = threadIdx.x & 63;
  const int64_t row = static_cast<int64_t>(blockIdx.x) * kWaves + (threadIdx.x >> 6);
  if (row >= rows) return;
  const int f = static_cast<int>(row % F);
  const int64_t bt = row / F;
  const int t = static_cast<int>(bt % Tn);
  const int b = static_cast<int>(bt / Tn);
  const bool valid = t < dev_len(lengths, b, Tn);
  const T* src = x + b * sb + t * st + f * sf;
  float v[4];
  float ss = 0.f;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int c = lane + 64 * j;
    v[j] = (valid && c < C) ? to_f32(src[c * sc]) : 0.f;
    ss += v[j] * v[j];
  }
  ss = wave_sum(ss);
  const float r = rsqrtf(ss / static_cast<float>(C) + eps);
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int c = lane + 64 * j;
    if (c < C) {
      float o = to_f32(from_f32<T>(v[j] * r * w[c]));
      if (silu) o = o * sigmoid_acc(o);
      y[row * C + c] = from_f32<T>(o);
    }
  }
}

// 8 consecutive elements of a row as fp32 (16- or 32-byte aligned loads and stores).
template <typename T>
__device__ __forceinline__ void load8v(const T* p, float (&v)[8]) {
  if constexpr (sizeof(T) == 4) {
    const float4 a = reinterpret_cast<const float4*>(p)[0];
    const float4 b = reinterpret_cast<const float4*>(p)[1];
    v[0] = a.x, v[1] = a.y, v[2] = a.z, v[3] = a.w, v[4] = b.x, v[5] = b.y, v[6] = b.z, v[7] = b.w;
  } else {
    const uint4 u = *reinterpret_cast<const uint4*>(p);
    const uint32_t wd[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      v[2 * e] = to_f32(__builtin_bit_cast(T, static_cast<uint16_t>(wd[e] & 0xffffu)));
      v[2 * e + 1] = to_f32(__builtin_bit_cast(T, static_cast<uint16_t>(wd[e] >> 16)));
    }
  }
}

template <typename T>
__device__ __forceinline__ void store8v(T* p, const float (&v)[8]) {
  if constexpr (sizeof(T) == 4) {
    reinterpret_cast<float4*>(p)[0] = make_float4(v[0], v[1], v[2], v[3]);
    reinterpret_cast<float4*>(p)[1] = make_float4(v[4], v[5], v[6], v[7]);
  } else {
    uint32_t wd[4];
#pragma unroll
    for (int e = 0; e < 4; ++e)
      wd[e] = static_cast<uint32_t>(__builtin_bit_cast(uint16_t, from_f32<T>(v[2 * e]))) |
              (static_cast<uint32_t>(__builtin_bit_cast(uint16_t, from_f32<T>(v[2 * e + 1]))) << 16);
    *reinterpret_cast<uint4*>(p) = make_uint4(wd[0], wd[1], wd[2], wd[3]);
  }
}

// y[b, t, c] = t < L ? a + (z - a) alpha : 0, a = low[b, left[b, t], c],
// z = low[b, right[b, t], c] (kernels/native.py:_interpolate). One block per row.
template <typename T>
__global__ __launch_bounds__(256) void interpolate_kernel(const T* __restrict__ low,
                                                          const int64_t* __restrict__ left,
                                                          const int64_t* __restrict__ right,
                                                          const float* __restrict__ alpha,
                                                          const int64_t* __restrict__ lengths, T* __restrict__ y,
                                                          int Tn, int LT, int D) {
  const int64_t row = blockIdx.x;
  const int b = static_cast<int>(row / Tn);
  const int t = static_cast<int>(row - static_cast<int64_t>(b) * Tn);
  const bool valid = t < dev_len(lengths, b, Tn);
  int64_t l = valid ? left[row] : 0, r = valid ? right[row] : 0;
  l = l < 0 ? 0 : (l >= LT ? LT - 1 : l);
  r = r < 0 ? 0 : (r >= LT ? LT - 1 : r);
  const float al = valid ? alpha[row] : 0.f;
  const T* pa = low + (static_cast<int64_t>(b) * LT + l) * D;
  const T* pz = low + (static_cast<int64_t>(b) * LT + r) * D;
  for (int c = threadIdx.x; c < D; c += blockDim.x) {
    float o = 0.f;
    if (valid) {
      const float a = to_f32(pa[c]), z = to_f32(pz[c]);
      o = a + (z - a) * al;
    }
    y[row * D + c] = from_f32<T>(o);
  }
}

// interpolate_kernel through 8-element vectors (D % 8 == 0, 16-byte aligned
// rows), 128 threads per row. The row's neighbour indices and weight are read
// whatever the row's length, so the data loads wait for one round trip only.
template <typename T>
__global__ __launch_bounds__(128) void interpolate_vec_kernel(const T* __restrict__ low,
                                                              const int64_t* __restrict__ left,
                                                              const int64_t* __restrict__ right,
                                                              const float* __restrict__ alpha,
                                                              const int64_t* __restrict__ lengths, T* __restrict__ y,
                                                              int Tn, int LT, int D) {
  const int64_t row = blockIdx.x;
  const int b = static_cast<int>(row / Tn);
  const int t = static_cast<int>(row - static_cast<int64_t>(b) * Tn);
  const int64_t l0 = left[row], r0 = right[row];
  const float al0 = alpha[row];
  const bool valid = t < dev_len(lengths, b, Tn);
  const int64_t l = valid ? (l0 < 0 ? 0 : (l0 >= LT ? LT - 1 : l0)) : 0;
  const int64_t r = valid ? (r0 < 0 ? 0 : (r0 >= LT ? LT - 1 : r0)) : 0;
  const float al = valid ? al0 : 0.f;
  const T* pa = low + (static_cast<int64_t>(b) * LT + l) * D;
  const T* pz = low + (static_cast<int64_t>(b) * LT + r) * D;
  for (int c = 8 * static_cast<int>(threadIdx.x); c < D; c += 8 * static_cast<int>(blockDim.x)) {
    float a[8], z[8], o[8];
    load8v(pa + c, a);
    load8v(pz + c, z);
#pragma unroll
    for (int e = 0; e < 8; ++e) o[e] = valid ? a[e] + (z[e] - a[e]) * al : 0.f;
    store8v(y + row * D + c, o);
  }
}

// interpolate then RMSNorm of each row in one pass: one wave per row, lane
// holding elements 8 (lane + 64 j) .. +7, j < PER8, the layout and summation
// order of the RMSNorm kernel (row_norm_vec_kernel), so the result is the one
// the two launches give. The interpolated value is rounded to T as the
// interpolation's output is; rows past the length are 0 before the norm.
template <typename T, int PER8>
__global__ __launch_bounds__(256) void interp_norm_kernel(const T* __restrict__ low,
                                                          const int64_t* __restrict__ left,
                                                          const int64_t* __restrict__ right,
                                                          const float* __restrict__ alpha,
                                                          const int64_t* __restrict__ lengths,
                                                          const float* __restrict__ w, T* __restrict__ y,
                                                          int64_t rows, int Tn, int LT, int D, float eps) {
  const int lane = threadIdx.x & 63;
  const int64_t row = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;
  const int b = static_cast<int>(row / Tn);
  const int t = static_cast<int>(row - static_cast<int64_t>(b) * Tn);
  const int64_t l0 = left[row], r0 = right[row];
  const float al0 = alpha[row];
  const bool valid = t < dev_len(lengths, b, Tn);
  const int64_t l = valid ? (l0 < 0 ? 0 : (l0 >= LT ? LT - 1 : l0)) : 0;
  const int64_t r = valid ? (r0 < 0 ? 0 : (r0 >= LT ? LT - 1 : r0)) : 0;
  const float al = valid ? al0 : 0.f;
  const T* pa = low + (static_cast<int64_t>(b) * LT + l) * D;
  const T* pz = low + (static_cast<int64_t>(b) * LT + r) * D;
  float v[PER8][8];
#pragma unroll
  for (int j = 0; j < PER8; ++j) {
    const int i0 = 8 * (lane + 64 * j);
    if (i0 < D) {
      float a[8], z[8];
      load8v(pa + i0, a);
      load8v(pz + i0, z);
#pragma unroll
      for (int e = 0; e < 8; ++e) v[j][e] = to_f32(from_f32<T>(valid ? a[e] + (z[e] - a[e]) * al : 0.f));
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) v[j][e] = 0.f;
    }
  }
  // The sum of squares as the RMSNorm kernel's compiled code forms it (its
  // source adds v * v in element order, contracted): the first two terms as
  // fma(v0, v0, v1 v1), then one fused multiply-add per element in order.
  float ss = __builtin_fmaf(v[0][0], v[0][0], v[0][1] * v[0][1]);
#pragma unroll
  for (int j = 0; j < PER8; ++j) {
#pragma unroll
    for (int e = j == 0 ? 2 : 0; e < 8; ++e) ss = __builtin_fmaf(v[j][e], v[j][e], ss);
  }
  ss = wave_sum(ss);
  const float rn = rsqrtf(ss / static_cast<float>(D) + eps);
#pragma unroll
  for (int j = 0; j < PER8; ++j) {
    const int i0 = 8 * (lane + 64 * j);
    if (i0 < D) {
      float wv[8], o[8];
      load8v(w + i0, wv);
#pragma unroll
      for (int e = 0; e < 8; ++e) o[e] = v[j][e] * rn * wv[e];
      store8v(y + row * D + i0, o);
    }
  }
}

// [B, C, T, F] (any strides) -> [B, T, 8, C]: band i averages frequencies
// floor(i F / 8) .. ceil((i + 1) F / 8) - 1 (kernels/native.py:_bands). One
// thread per output element.
template <typename T>
__global__ __launch_bounds__(256) void bands_kernel(const T* __restrict__ x, T* __restrict__ y, int Tn, int F, int C,
                                                    int64_t total, int64_t sb, int64_t sc, int64_t st, int64_t sf) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= total) return;
  const int c = static_cast<int>(i % C);
  const int band = static_cast<int>((i / C) % 8);
  const int64_t bt = i / (static_cast<int64_t>(C) * 8);
  const int t = static_cast<int>(bt % Tn);
  const int b = static_cast<int>(bt / Tn);
  const int start = band * F / 8;
  const int end = ((band + 1) * F + 7) / 8;
  const T* src = x + b * sb + c * sc + t * st;
  float acc = 0.f;
  for (int f = start; f < end; ++f) acc += to_f32(src[f * sf]);
  y[i] = from_f32<T>(acc / static_cast<float>(end - start));
}

// s = mask[row] ? x + a * (2 sigmoid(g)) : 0 (fp32), y = s rsqrt(mean(s^2) + eps) w
// in fp32 (kernels/native.py:_norm MODE 1 via evidence_norm). One wave per row;
// the second pass recomputes s from the (now cached) row.
template <typename TA, typename TY>
__global__ __launch_bounds__(256) void evidence_norm_kernel(const float* __restrict__ x, const TA* __restrict__ a,
                                                            const TA* __restrict__ g, int64_t ag_stride,
                                                            const uint8_t* __restrict__ mask,
                                                            const float* __restrict__ w, TY* __restrict__ y,
                                                            int64_t rows, int D, float eps) {
  const int lane = threadIdx.x & 63;
  const int64_t row = static_cast<int64_t>(blockIdx.x) * kWaves + (threadIdx.x >> 6);
  if (row >= rows) return;
  const bool valid = mask == nullptr || mask[row] != 0;
  auto value = [&](int c) {
    const int64_t o = row * D + c, oa = row * ag_stride + c;
    return valid ? x[o] + to_f32(a[oa]) * (2.f * sigmoid_acc(to_f32(g[oa]))) : 0.f;
  };
  float ss = 0.f;
  for (int c = lane; c < D; c += 64) {
    const float s = value(c);
    ss += s * s;
  }
  ss = wave_sum(ss);
  const float r = rsqrtf(ss / static_cast<float>(D) + eps);
  for (int c = lane; c < D; c += 64) y[row * D + c] = from_f32<TY>(value(c) * r * w[c]);
}

// evidence_norm_kernel through 8-element vectors: one wave per row, lane holds
// elements 8 (lane + 64 i) .. +7, i < PER8.
template <typename TA, typename TY, int PER8>
__global__ __launch_bounds__(256) void evidence_norm_vec_kernel(const float* __restrict__ x,
                                                                const TA* __restrict__ a, const TA* __restrict__ g,
                                                                int64_t ag_stride, const uint8_t* __restrict__ mask,
                                                                const float* __restrict__ w, TY* __restrict__ y,
                                                                int64_t rows, int D, float eps) {
  const int lane = threadIdx.x & 63;
  const int64_t row = static_cast<int64_t>(blockIdx.x) * kWaves + (threadIdx.x >> 6);
  if (row >= rows) return;
  const bool valid = mask == nullptr || mask[row] != 0;
  float v[PER8][8];
  float ss = 0.f;
#pragma unroll
  for (int i = 0; i < PER8; ++i) {
    const int i0 = 8 * (lane + 64 * i);
#pragma unroll
    for (int e = 0; e < 8; ++e) v[i][e] = 0.f;
    if (i0 < D && valid) {
      float xv[8], av[8], gv[8];
      load8v(x + row * D + i0, xv);
      load8v(a + row * ag_stride + i0, av);
      load8v(g + row * ag_stride + i0, gv);
#pragma unroll
      for (int e = 0; e < 8; ++e) v[i][e] = xv[e] + av[e] * (2.f * sigmoid_acc(gv[e]));
    }
#pragma unroll
    for (int e = 0; e < 8; ++e) ss += v[i][e] * v[i][e];
  }
  ss = wave_sum(ss);
  const float r = rsqrtf(ss / static_cast<float>(D) + eps);
#pragma unroll
  for (int i = 0; i < PER8; ++i) {
    const int i0 = 8 * (lane + 64 * i);
    if (i0 < D) {
      float wv[8], o[8];
      load8v(w + i0, wv);
#pragma unroll
      for (int e = 0; e < 8; ++e) o[e] = v[i][e] * r * wv[e];
      store8v(y + row * D + i0, o);
    }
  }
}

// y[row, k d + j] = x[row, k d + j] * 2 sigmoid(gate[row, k]), k < 3
// (primitives.py:_gate forward through gated_concat).
template <typename T>
__global__ __launch_bounds__(256) void gated_concat_kernel(const T* __restrict__ x, const T* __restrict__ gate,
                                                           T* __restrict__ y, int d, int64_t total) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= total) return;
  const int64_t gi = i / d;  // row * 3 + branch
  const float s = sigmoid_acc(to_f32(gate[gi]));
  y[i] = from_f32<T>(to_f32(x[i]) * (2.f * s));
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

uint32_t nblocks(int64_t n, int per) { return static_cast<uint32_t>((n + per - 1) / per); }

}  // namespace
}  // namespace tf

#define TF_ROW_GRID(rows) dim3(static_cast<uint32_t>(rows))

extern "C" int tf_depthwise_masked(const void* x, const void* w, const void* bias, int32_t dtype,
                                   const int64_t* lengths, void* y, int64_t batch, int64_t time, int64_t d,
                                   int64_t k, void* stream) {
  if (!x || !w || !bias || !lengths || !y) return TF_ERR_NULL;
  if (batch < 0 || time < 0 || d < 1 || k < 1 || k > 63 || batch * time > 0x7fffffff) return TF_ERR_SHAPE;
  if (batch * time == 0) return TF_OK;
  hipStream_t s = static_cast<hipStream_t>(stream);
  TF_DISPATCH(dtype, T,
              hipLaunchKernelGGL(tf::depthwise_masked_kernel<T>, TF_ROW_GRID(batch * time), dim3(256), 0, s,
                                 static_cast<const T*>(x), static_cast<const T*>(w), static_cast<const T*>(bias),
                                 lengths, static_cast<T*>(y), static_cast<int>(time), static_cast<int>(d),
                                 static_cast<int>(k));
              return tf::launch_status());
  return TF_ERR_DTYPE;
}

extern "C" int tf_pool4(const void* x, int32_t dtype, const int64_t* lengths, void* y, int64_t batch, int64_t time,
                        int64_t d, void* stream) {
  if (!x || !lengths || !y) return TF_ERR_NULL;
  if (batch < 0 || time < 0 || d < 1 || batch * time > 0x7fffffff) return TF_ERR_SHAPE;
  const int64_t lt = (time + 3) / 4;
  if (batch * lt == 0) return TF_OK;
  hipStream_t s = static_cast<hipStream_t>(stream);
  TF_DISPATCH(dtype, T,
              hipLaunchKernelGGL(tf::pool4_kernel<T>, TF_ROW_GRID(batch * lt), dim3(256), 0, s,
                                 static_cast<const T*>(x), lengths, static_cast<T*>(y), static_cast<int>(time),
                                 static_cast<int>(lt), static_cast<int>(d));
              return tf::launch_status());
  return TF_ERR_DTYPE;
}

extern "C" int tf_rotary_qkv(const void* x, int32_t dtype, const float* cos_t, const float* sin_t, void* y,
                             int64_t batch, int64_t time, int64_t heads, int64_t head_dim, void* stream) {
  if (!x || !cos_t || !sin_t || !y) return TF_ERR_NULL;
  if (batch < 0 || time < 0 || heads < 1 || head_dim < 2 || head_dim % 2) return TF_ERR_SHAPE;
  const int64_t pairs = 3 * batch * heads * time * (head_dim / 2);
  if (pairs == 0) return TF_OK;
  if (pairs > (int64_t(1) << 40)) return TF_ERR_SHAPE;
  hipStream_t s = static_cast<hipStream_t>(stream);
  TF_DISPATCH(dtype, T,
              hipLaunchKernelGGL(tf::rotary_qkv_kernel<T>, dim3(tf::nblocks(pairs, 256)), dim3(256), 0, s,
                                 static_cast<const T*>(x), cos_t, sin_t, static_cast<T*>(y),
                                 static_cast<int>(batch), static_cast<int>(time), static_cast<int>(heads),
                                 static_cast<int>(head_dim), pairs);
              return tf::launch_status());
  return TF_ERR_DTYPE;
}

extern "C" int tf_front_norm(const void* x, int32_t dtype, const int64_t* strides, const float* w,
                             const int64_t* lengths, void* y, int64_t batch, int64_t chans, int64_t time,
                             int64_t freq, float eps, int32_t silu, void* stream) {
  if (!x || !strides || !w || !lengths || !y) return TF_ERR_NULL;
  if (batch < 0 || chans < 1 || chans > 256 || time < 0 || freq < 1) return TF_ERR_SHAPE;
  const int64_t rows = batch * time * freq;
  if (rows == 0) return TF_OK;
  hipStream_t s = static_cast<hipStream_t>(stream);
  TF_DISPATCH(dtype, T,
              hipLaunchKernelGGL(tf::front_norm_kernel<T>, dim3(tf::nblocks(rows, tf::kWaves)), dim3(256), 0, s,
                                 static_cast<const T*>(x), w, lengths, static_cast<T*>(y), static_cast<int>(time),
                                 static_cast<int>(freq), static_cast<int>(chans), rows, strides[0], strides[1],
                                 strides[2], strides[3], eps, silu);
              return tf::launch_status());
  return TF_ERR_DTYPE;
}

extern "C" int tf_interpolate(const void* low, int32_t dtype, const int64_t* left, const int64_t* right,
                              const float* alpha, const int64_t* lengths, void* y, int64_t batch, int64_t time,
                              int64_t low_time, int64_t d, void* stream) {
  if (!low || !left || !right || !alpha || !lengths || !y) return TF_ERR_NULL;
  if (batch < 0 || time < 0 || low_time < 1 || d < 1 || batch * time > 0x7fffffff) return TF_ERR_SHAPE;
  if (batch * time == 0) return TF_OK;
  hipStream_t s = static_cast<hipStream_t>(stream);
  // 16-byte rows (d % 8 == 0 for every dtype) from 16-byte aligned bases
  const bool vec = d % 8 == 0 && (reinterpret_cast<uintptr_t>(low) & 15) == 0 && (reinterpret_cast<uintptr_t>(y) & 15) == 0;
  if (vec)
    TF_DISPATCH(dtype, T,
                hipLaunchKernelGGL(tf::interpolate_vec_kernel<T>, TF_ROW_GRID(batch * time), dim3(128), 0, s,
                                   static_cast<const T*>(low), left, right, alpha, lengths, static_cast<T*>(y),
                                   static_cast<int>(time), static_cast<int>(low_time), static_cast<int>(d));
                return tf::launch_status());
  TF_DISPATCH(dtype, T,
              hipLaunchKernelGGL(tf::interpolate_kernel<T>, TF_ROW_GRID(batch * time), dim3(256), 0, s,
                                 static_cast<const T*>(low), left, right, alpha, lengths, static_cast<T*>(y),
                                 static_cast<int>(time), static_cast<int>(low_time), static_cast<int>(d));
              return tf::launch_status());
  return TF_ERR_DTYPE;
}

extern "C" int tf_interpolate_rmsnorm(const void* low, int32_t dtype, const int64_t* left, const int64_t* right,
                                      const float* alpha, const int64_t* lengths, const float* w, float eps, void* y,
                                      int64_t batch, int64_t time, int64_t low_time, int64_t d, void* stream) {
  if (!low || !left || !right || !alpha || !lengths || !w || !y) return TF_ERR_NULL;
  if (batch < 0 || time < 0 || low_time < 1 || d < 8 || d % 8 || d > 4096 || batch * time > 0x7fffffff)
    return TF_ERR_SHAPE;
  if ((reinterpret_cast<uintptr_t>(low) & 15) || (reinterpret_cast<uintptr_t>(y) & 15) ||
      (reinterpret_cast<uintptr_t>(w) & 15))
    return TF_ERR_STRIDE;
  const int64_t rows = batch * time;
  if (rows == 0) return TF_OK;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const dim3 grid(static_cast<uint32_t>((rows + 3) / 4)), block(256);
  int per8 = 1;
  while (per8 * 512 < d) per8 <<= 1;
#define TF_IN(P)                                                                                                 \
  if (per8 == P) {                                                                                               \
    TF_DISPATCH(dtype, T,                                                                                        \
                hipLaunchKernelGGL((tf::interp_norm_kernel<T, P>), grid, block, 0, s, static_cast<const T*>(low), \
                                   left, right, alpha, lengths, w, static_cast<T*>(y), rows, static_cast<int>(time), \
                                   static_cast<int>(low_time), static_cast<int>(d), eps);                        \
                return tf::launch_status());                                                                     \
    return TF_ERR_DTYPE;                                                                                         \
  }
  TF_IN(1) TF_IN(2) TF_IN(4) TF_IN(8)
#undef TF_IN
  return TF_ERR_SHAPE;
}

extern "C" int tf_bands(const void* x, int32_t dtype, const int64_t* strides, void* y, int64_t batch, int64_t chans,
                        int64_t time, int64_t freq, void* stream) {
  if (!x || !strides || !y) return TF_ERR_NULL;
  if (batch < 0 || chans < 1 || time < 0 || freq < 8) return TF_ERR_SHAPE;
  const int64_t total = batch * time * 8 * chans;
  if (total == 0) return TF_OK;
  hipStream_t s = static_cast<hipStream_t>(stream);
  TF_DISPATCH(dtype, T,
              hipLaunchKernelGGL(tf::bands_kernel<T>, dim3(tf::nblocks(total, 256)), dim3(256), 0, s,
                                 static_cast<const T*>(x), static_cast<T*>(y), static_cast<int>(time),
                                 static_cast<int>(freq), static_cast<int>(chans), total, strides[0], strides[1],
                                 strides[2], strides[3]);
              return tf::launch_status());
  return TF_ERR_DTYPE;
}

extern "C" int tf_evidence_norm(const float* x, const void* a, const void* g, int32_t ag_dtype, int64_t ag_stride,
                                const uint8_t* mask, const float* w, void* y, int32_t y_dtype, int64_t rows, int64_t d,
                                float eps, void* stream) {
  if (!x || !a || !g || !w || !y) return TF_ERR_NULL;
  if (rows < 0 || d < 1 || ag_stride < d) return TF_ERR_SHAPE;
  if (y_dtype != TF_FLOAT32 && y_dtype != TF_BFLOAT16) return TF_ERR_DTYPE;
  if (rows == 0) return TF_OK;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const dim3 grid(tf::nblocks(rows, tf::kWaves));
  const bool vec = d % 8 == 0 && ag_stride % 8 == 0 && d <= 2048 && tf::aligned16(x) && tf::aligned16(a) &&
                   tf::aligned16(g) && tf::aligned16(w) && tf::aligned16(y);
  if (vec) {
    const int per8 = d <= 512 ? 1 : (d <= 1024 ? 2 : 4);
#define TF_EVN(TAV, TYV, P)                                                                                   \
  hipLaunchKernelGGL((tf::evidence_norm_vec_kernel<TAV, TYV, P>), grid, dim3(256), 0, s, x,                   \
                     static_cast<const TAV*>(a), static_cast<const TAV*>(g), ag_stride, mask, w,              \
                     static_cast<TYV*>(y),                                                                      \
                     rows, static_cast<int>(d), eps)
#define TF_EVN_P(TAV, TYV)          \
  if (per8 == 1) TF_EVN(TAV, TYV, 1); \
  else if (per8 == 2) TF_EVN(TAV, TYV, 2); \
  else TF_EVN(TAV, TYV, 4);
    TF_DISPATCH(ag_dtype, TA,
                if (y_dtype == TF_FLOAT32) { TF_EVN_P(TA, float) } else { TF_EVN_P(TA, tf::bf16_t) } return
                tf::launch_status());
#undef TF_EVN_P
#undef TF_EVN
    return TF_ERR_DTYPE;
  }
  TF_DISPATCH(ag_dtype, TA,
              if (y_dtype == TF_FLOAT32) {
                hipLaunchKernelGGL((tf::evidence_norm_kernel<TA, float>), grid, dim3(256), 0, s, x,
                                   static_cast<const TA*>(a), static_cast<const TA*>(g), ag_stride, mask, w,
                                   static_cast<float*>(y), rows, static_cast<int>(d), eps);
              } else {
                hipLaunchKernelGGL((tf::evidence_norm_kernel<TA, tf::bf16_t>), grid, dim3(256), 0, s, x,
                                   static_cast<const TA*>(a), static_cast<const TA*>(g), ag_stride, mask, w,
                                   static_cast<tf::bf16_t*>(y), rows, static_cast<int>(d), eps);
              } return tf::launch_status());
  return TF_ERR_DTYPE;
}

extern "C" int tf_gated_concat(const void* x, const void* gate, int32_t dtype, void* y, int64_t rows, int64_t d,
                               void* stream) {
  if (!x || !gate || !y) return TF_ERR_NULL;
  if (rows < 0 || d < 1) return TF_ERR_SHAPE;
  const int64_t total = rows * 3 * d;
  if (total == 0) return TF_OK;
  hipStream_t s = static_cast<hipStream_t>(stream);
  TF_DISPATCH(dtype, T,
              hipLaunchKernelGGL(tf::gated_concat_kernel<T>, dim3(tf::nblocks(total, 256)), dim3(256), 0, s,
                                 static_cast<const T*>(x), static_cast<const T*>(gate), static_cast<T*>(y),
                                 static_cast<int>(d), total);
              return tf::launch_status());
  return TF_ERR_DTYPE;
}
