// Single-pass bandwidth kernels around the recurrence: RMSNorm (optionally
// fused with the residual add that precedes it), SwiGLU, row masking, masked
// add, the Mamba-3 controls and masked mean-pooling. Reductions are wave64
// shuffles; every kernel reads each input element once and writes each output
// element once.
#include "common.h"

namespace tf {
namespace {

constexpr int kRowsPerBlock = 4;  // one wave64 per row

// One wave per row; lane holds elements lane + 64*j, j < PER (64*PER >= d).
template <typename TX, typename TB, typename TS, typename TY, int PER, bool ADD>
__global__ __launch_bounds__(256) void row_norm_kernel(const TX* __restrict__ x, int64_t x_stride,
                                                       const TB* __restrict__ bsrc,
                                                       const uint8_t* __restrict__ mask,
                                                       const float* __restrict__ w, TS* __restrict__ s,
                                                       TY* __restrict__ y, int64_t rows, int d, float eps) {
  const int lane = threadIdx.x & 63;
  const int64_t row = static_cast<int64_t>(blockIdx.x) * kRowsPerBlock + (threadIdx.x >> 6);
  if (row >= rows) return;
  const bool keep = !ADD || mask == nullptr || mask[row] != 0;
  float v[PER];
  float ss = 0.f;
#pragma unroll
  for (int j = 0; j < PER; ++j) {
    const int i = lane + 64 * j;
    float val = 0.f;
    if (i < d) {
      val = to_f32(x[row * x_stride + i]);
      if constexpr (ADD) {
        val = keep ? val + to_f32(bsrc[row * d + i]) : 0.f;
        const TS stored = from_f32<TS>(val);
        s[row * d + i] = stored;
        val = to_f32(stored);
      }
    }
    v[j] = val;
    ss += val * val;
  }
  ss = wave_sum(ss);
  const float r = rsqrtf(ss / static_cast<float>(d) + eps);
#pragma unroll
  for (int j = 0; j < PER; ++j) {
    const int i = lane + 64 * j;
    if (i < d) y[row * d + i] = from_f32<TY>(v[j] * r * w[i]);
  }
}

template <typename TX, typename TB, typename TS, typename TY, bool ADD>
int launch_row_norm(const void* x, int64_t x_stride, const void* bsrc, const uint8_t* mask,
                    const float* w, void* s, void* y, int64_t rows, int d, float eps,
                    hipStream_t stream) {
  int per = 1;
  while (per * 64 < d) per <<= 1;
  const dim3 grid(static_cast<uint32_t>((rows + kRowsPerBlock - 1) / kRowsPerBlock));
  const dim3 block(64 * kRowsPerBlock);
  const TX* xp = static_cast<const TX*>(x);
  const TB* bp = static_cast<const TB*>(bsrc);
  TS* sp = static_cast<TS*>(s);
  TY* yp = static_cast<TY*>(y);
#define TF_NORM_CASE(P)                                                                          \
  case P:                                                                                         \
    hipLaunchKernelGGL((row_norm_kernel<TX, TB, TS, TY, P, ADD>), grid, block, 0, stream, xp,    \
                       x_stride, bp, mask, w, sp, yp, rows, d, eps);                              \
    break;
  switch (per) {
    TF_NORM_CASE(1)
    TF_NORM_CASE(2)
    TF_NORM_CASE(4)
    TF_NORM_CASE(8)
    TF_NORM_CASE(16)
    TF_NORM_CASE(32)
    TF_NORM_CASE(64)
    default:
      return TF_ERR_SHAPE;
  }
#undef TF_NORM_CASE
  return launch_status();
}

// SwiGLU over [rows, 2d] -> [rows, d]; one block per row.
template <typename T>
__global__ __launch_bounds__(256) void swiglu_kernel(const T* __restrict__ x, T* __restrict__ y,
                                                     int64_t d) {
  const int64_t row = blockIdx.x;
  const T* xr = x + row * 2 * d;
  T* yr = y + row * d;
  for (int64_t j = threadIdx.x; j < d; j += blockDim.x) {
    const float g = to_f32(xr[j]);
    const float u = to_f32(xr[d + j]);
    yr[j] = from_f32<T>(g * sigmoidf(g) * u);
  }
}

template <typename T>
__global__ __launch_bounds__(256) void mask_rows_kernel(const T* __restrict__ x, T* __restrict__ y,
                                                        const uint8_t* __restrict__ mask, int64_t d) {
  const int64_t row = blockIdx.x;
  const bool keep = mask[row] != 0;
  for (int64_t j = threadIdx.x; j < d; j += blockDim.x)
    y[row * d + j] = keep ? x[row * d + j] : from_f32<T>(0.f);
}

template <typename TA, typename TB, typename TY>
__global__ __launch_bounds__(256) void add_kernel(const TA* __restrict__ a, const TB* __restrict__ b,
                                                  const uint8_t* __restrict__ mask, TY* __restrict__ y,
                                                  int64_t d) {
  const int64_t row = blockIdx.x;
  const bool keep = mask == nullptr || mask[row] != 0;
  for (int64_t j = threadIdx.x; j < d; j += blockDim.x) {
    const int64_t i = row * d + j;
    y[i] = from_f32<TY>(keep ? to_f32(a[i]) + to_f32(b[i]) : 0.f);
  }
}

// Output index i runs over [B, H, T] with t fastest (coalesced fp32 writes).
template <typename T>
__global__ __launch_bounds__(256) void controls_kernel(const T* __restrict__ a, const T* __restrict__ ddt,
                                                       int64_t sb, int64_t st,
                                                       const float* __restrict__ bias,
                                                       float* __restrict__ adt, float* __restrict__ dt,
                                                       int64_t time, int64_t heads, int64_t total,
                                                       float floor_) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= total) return;
  const int64_t t = i % time;
  const int64_t bh = i / time;
  const int64_t h = bh % heads;
  const int64_t b = bh / heads;
  const int64_t src = b * sb + t * st + h;
  const float av = to_f32(a[src]);
  const float v = to_f32(ddt[src]) + bias[h];
  const float control = fminf(-(fmaxf(av, 0.f) + 1.f / (1.f - fminf(av, 0.f))), -floor_);
  const float step = v > 20.f ? v : log1pf(expf(v));
  dt[i] = step;
  adt[i] = control * step;
}

// Block = 4 waves over (batch b, 64 columns); wave w sums frames t = w (mod 4).
template <typename T>
__global__ __launch_bounds__(256) void masked_mean_kernel(const T* __restrict__ x,
                                                          const int64_t* __restrict__ lengths,
                                                          float* __restrict__ y, int64_t time,
                                                          int64_t d) {
  __shared__ float part[4][64];
  const int lane = threadIdx.x & 63;
  const int w = threadIdx.x >> 6;
  const int64_t b = blockIdx.y;
  const int64_t col = static_cast<int64_t>(blockIdx.x) * 64 + lane;
  const int64_t len = lengths[b];
  const int64_t L = len < 0 ? 0 : (len > time ? time : len);
  float acc = 0.f;
  if (col < d)
    for (int64_t t = w; t < L; t += 4) acc += to_f32(x[(b * time + t) * d + col]);
  part[w][lane] = acc;
  __syncthreads();
  if (w == 0 && col < d)
    y[b * d + col] = (part[0][lane] + part[1][lane] + part[2][lane] + part[3][lane]) /
                     static_cast<float>(len);
}

__global__ __launch_bounds__(256) void time_mask_kernel(const int64_t* __restrict__ lengths,
                                                        uint8_t* __restrict__ mask, int64_t time,
                                                        int64_t total) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= total) return;
  mask[i] = (i % time) < lengths[i / time] ? 1 : 0;
}

uint32_t blocks_for(int64_t n, int per_block) {
  return static_cast<uint32_t>((n + per_block - 1) / per_block);
}

}  // namespace
}  // namespace tf

using tf::bf16_t;

extern "C" int tf_rmsnorm(const void* x, int32_t x_dtype, int64_t x_row_stride, const float* w,
                          void* y, int32_t y_dtype, int64_t rows, int64_t d, float eps,
                          void* stream) {
  if (!x || !w || !y) return TF_ERR_NULL;
  if (rows < 0 || d < 1 || d > 4096) return TF_ERR_SHAPE;
  if (x_row_stride == 0) x_row_stride = d;
  if (x_row_stride < d) return TF_ERR_STRIDE;
  if (rows == 0) return TF_OK;
  hipStream_t s = static_cast<hipStream_t>(stream);
  TF_DISPATCH(x_dtype, TX,
              TF_DISPATCH(y_dtype, TY,
                          return (tf::launch_row_norm<TX, float, float, TY, false>(
                              x, x_row_stride, nullptr, nullptr, w, nullptr, y, rows,
                              static_cast<int>(d), eps, s))));
  return TF_ERR_DTYPE;
}

extern "C" int tf_add_rmsnorm(const void* a, int32_t a_dtype, const void* b, int32_t b_dtype,
                              const uint8_t* mask, const float* w, void* s, int32_t s_dtype,
                              void* y, int32_t y_dtype, int64_t rows, int64_t d, float eps,
                              void* stream) {
  if (!a || !b || !w || !s || !y) return TF_ERR_NULL;
  if (rows < 0 || d < 1 || d > 4096) return TF_ERR_SHAPE;
  if (a_dtype != TF_FLOAT32 || s_dtype != TF_FLOAT32) return TF_ERR_DTYPE;
  if (rows == 0) return TF_OK;
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int di = static_cast<int>(d);
  if (b_dtype == TF_FLOAT32 && y_dtype == TF_FLOAT32)
    return tf::launch_row_norm<float, float, float, float, true>(a, d, b, mask, w, s, y, rows, di, eps, st);
  if (b_dtype == TF_FLOAT32 && y_dtype == TF_BFLOAT16)
    return tf::launch_row_norm<float, float, float, bf16_t, true>(a, d, b, mask, w, s, y, rows, di, eps, st);
  if (b_dtype == TF_BFLOAT16 && y_dtype == TF_FLOAT32)
    return tf::launch_row_norm<float, bf16_t, float, float, true>(a, d, b, mask, w, s, y, rows, di, eps, st);
  if (b_dtype == TF_BFLOAT16 && y_dtype == TF_BFLOAT16)
    return tf::launch_row_norm<float, bf16_t, float, bf16_t, true>(a, d, b, mask, w, s, y, rows, di, eps, st);
  return TF_ERR_DTYPE;
}

extern "C" int tf_swiglu(const void* x, void* y, int32_t dtype, int64_t rows, int64_t d,
                         void* stream) {
  if (!x || !y) return TF_ERR_NULL;
  if (rows < 0 || d < 1 || rows > 0x7fffffff) return TF_ERR_SHAPE;
  if (rows == 0) return TF_OK;
  hipStream_t s = static_cast<hipStream_t>(stream);
  TF_DISPATCH(dtype, T,
              hipLaunchKernelGGL(tf::swiglu_kernel<T>, dim3(static_cast<uint32_t>(rows)), dim3(256), 0,
                                 s, static_cast<const T*>(x), static_cast<T*>(y), d);
              return tf::launch_status());
  return TF_ERR_DTYPE;
}

extern "C" int tf_mask_rows(const void* x, void* y, int32_t dtype, const uint8_t* mask, int64_t rows,
                            int64_t d, void* stream) {
  if (!x || !y || !mask) return TF_ERR_NULL;
  if (rows < 0 || d < 1 || rows > 0x7fffffff) return TF_ERR_SHAPE;
  if (rows == 0) return TF_OK;
  hipStream_t s = static_cast<hipStream_t>(stream);
  TF_DISPATCH(dtype, T,
              hipLaunchKernelGGL(tf::mask_rows_kernel<T>, dim3(static_cast<uint32_t>(rows)), dim3(256), 0,
                                 s, static_cast<const T*>(x), static_cast<T*>(y), mask, d);
              return tf::launch_status());
  return TF_ERR_DTYPE;
}

extern "C" int tf_add(const void* a, int32_t a_dtype, const void* b, int32_t b_dtype,
                      const uint8_t* mask, void* y, int32_t y_dtype, int64_t rows, int64_t d,
                      void* stream) {
  if (!a || !b || !y) return TF_ERR_NULL;
  if (rows < 0 || d < 1 || rows > 0x7fffffff) return TF_ERR_SHAPE;
  if (rows == 0) return TF_OK;
  hipStream_t s = static_cast<hipStream_t>(stream);
  TF_DISPATCH(
      a_dtype, TA,
      TF_DISPATCH(b_dtype, TB,
                  TF_DISPATCH(y_dtype, TY,
                              hipLaunchKernelGGL((tf::add_kernel<TA, TB, TY>),
                                                 dim3(static_cast<uint32_t>(rows)), dim3(256), 0, s,
                                                 static_cast<const TA*>(a), static_cast<const TB*>(b),
                                                 mask, static_cast<TY*>(y), d);
                              return tf::launch_status())));
  return TF_ERR_DTYPE;
}

extern "C" int tf_mamba_controls(const void* a, const void* ddt, int32_t dtype, int64_t sb, int64_t st,
                                 const float* bias, float* adt, float* dt, int64_t batch, int64_t time,
                                 int64_t heads, float floor_, void* stream) {
  if (!a || !ddt || !bias || !adt || !dt) return TF_ERR_NULL;
  if (batch < 0 || time < 0 || heads < 1) return TF_ERR_SHAPE;
  const int64_t total = batch * heads * time;
  if (total == 0) return TF_OK;
  hipStream_t s = static_cast<hipStream_t>(stream);
  TF_DISPATCH(dtype, T,
              hipLaunchKernelGGL(tf::controls_kernel<T>, dim3(tf::blocks_for(total, 256)), dim3(256), 0,
                                 s, static_cast<const T*>(a), static_cast<const T*>(ddt), sb, st, bias,
                                 adt, dt, time, heads, total, floor_);
              return tf::launch_status());
  return TF_ERR_DTYPE;
}

extern "C" int tf_masked_mean(const void* x, int32_t dtype, const int64_t* lengths, float* y,
                              int64_t batch, int64_t time, int64_t d, void* stream) {
  if (!x || !lengths || !y) return TF_ERR_NULL;
  if (batch < 0 || time < 0 || d < 1 || batch > 65535) return TF_ERR_SHAPE;
  if (batch == 0) return TF_OK;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const dim3 grid(tf::blocks_for(d, 64), static_cast<uint32_t>(batch));
  TF_DISPATCH(dtype, T,
              hipLaunchKernelGGL(tf::masked_mean_kernel<T>, grid, dim3(256), 0, s, static_cast<const T*>(x),
                                 lengths, y, time, d);
              return tf::launch_status());
  return TF_ERR_DTYPE;
}

extern "C" int tf_time_mask(const int64_t* lengths, uint8_t* mask, int64_t batch, int64_t time,
                            void* stream) {
  if (!lengths || !mask) return TF_ERR_NULL;
  if (batch < 0 || time < 0) return TF_ERR_SHAPE;
  const int64_t total = batch * time;
  if (total == 0) return TF_OK;
  hipLaunchKernelGGL(tf::time_mask_kernel, dim3(tf::blocks_for(total, 256)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), lengths, mask, time, total);
  return tf::launch_status();
}
