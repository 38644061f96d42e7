// Single-pass bandwidth kernels around the recurrence: RMSNorm (optionally
// fused with the residual add that precedes it, or with the mean of the two
// directions of a bidirectional block), SwiGLU, row masking, masked add, the
// Mamba-3 controls, masked mean-pooling and valid-prefix reversal. Reductions are wave64
// shuffles; every kernel reads each input element once and writes each output
// element once.
#include "common.h"

namespace tf {
namespace {

constexpr int kRowsPerBlock = 4;  // one wave64 per row

// What the row norms normalise: x itself; the masked sum s = (x + b) * mask,
// stored as it is normalised; the mean of two directions (x + b) / 2; or the
// masked row s = x * mask, stored as it is normalised.
enum NormOp { kNormPlain = 0, kNormAdd = 1, kNormMean = 2, kNormMask = 3 };

// Eight consecutive elements through 16-byte accesses (two for fp32): a wave
// moves 1-2 KB per load instruction instead of 128-256 B, which is what keeps
// enough bytes in flight to approach the HBM roofline.
template <typename T>
__device__ __forceinline__ void load8(const T* p, float (&v)[8]) {
  if constexpr (sizeof(T) == 4) {
    const float4 a = reinterpret_cast<const float4*>(p)[0];
    const float4 b = reinterpret_cast<const float4*>(p)[1];
    v[0] = a.x, v[1] = a.y, v[2] = a.z, v[3] = a.w;
    v[4] = b.x, v[5] = b.y, v[6] = b.z, v[7] = b.w;
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
__device__ __forceinline__ void store8(T* p, const float (&v)[8]) {
  if constexpr (sizeof(T) == 4) {
    reinterpret_cast<float4*>(p)[0] = make_float4(v[0], v[1], v[2], v[3]);
    reinterpret_cast<float4*>(p)[1] = make_float4(v[4], v[5], v[6], v[7]);
  } else {
    uint32_t wd[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const uint32_t lo = __builtin_bit_cast(uint16_t, from_f32<T>(v[2 * e]));
      const uint32_t hi = __builtin_bit_cast(uint16_t, from_f32<T>(v[2 * e + 1]));
      wd[e] = lo | (hi << 16);
    }
    *reinterpret_cast<uint4*>(p) = make_uint4(wd[0], wd[1], wd[2], wd[3]);
  }
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

// RMSNorm rows through 8-element vectors: one wave per row, lane holds
// elements 8*(lane + 64*j) .. +7, j < PER8 (512*PER8 >= d, d % 8 == 0).
template <typename TX, typename TB, typename TS, typename TY, int PER8, int OP>
__global__ __launch_bounds__(256) void row_norm_vec_kernel(const TX* __restrict__ x, int64_t x_stride,
                                                           const TB* __restrict__ bsrc,
                                                           const uint8_t* __restrict__ mask,
                                                           const float* __restrict__ w, TS* __restrict__ s,
                                                           TY* __restrict__ y, int64_t rows, int d, float eps) {
  const int lane = threadIdx.x & 63;
  const int64_t row = static_cast<int64_t>(blockIdx.x) * kRowsPerBlock + (threadIdx.x >> 6);
  if (row >= rows) return;
  const bool keep = (OP != kNormAdd && OP != kNormMask) || mask == nullptr || mask[row] != 0;
  float v[PER8][8];
  float ss = 0.f;
#pragma unroll
  for (int j = 0; j < PER8; ++j) {
    const int i0 = 8 * (lane + 64 * j);
    if (i0 < d) {
      load8(x + row * x_stride + i0, v[j]);
      if constexpr (OP == kNormAdd || OP == kNormMean) {
        float bv[8];
        load8(bsrc + row * d + i0, bv);
        if constexpr (OP == kNormAdd) {
#pragma unroll
          for (int e = 0; e < 8; ++e) v[j][e] = keep ? to_f32(from_f32<TS>(v[j][e] + bv[e])) : 0.f;
          store8(s + row * d + i0, v[j]);
        } else {
#pragma unroll
          for (int e = 0; e < 8; ++e) v[j][e] = (v[j][e] + bv[e]) * 0.5f;
        }
      }
      if constexpr (OP == kNormMask) {
#pragma unroll
        for (int e = 0; e < 8; ++e) v[j][e] = keep ? to_f32(from_f32<TS>(v[j][e])) : 0.f;
        store8(s + row * d + i0, v[j]);
      }
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) v[j][e] = 0.f;
    }
#pragma unroll
    for (int e = 0; e < 8; ++e) ss += v[j][e] * v[j][e];
  }
  ss = wave_sum(ss);
  const float r = rsqrtf(ss / static_cast<float>(d) + eps);
#pragma unroll
  for (int j = 0; j < PER8; ++j) {
    const int i0 = 8 * (lane + 64 * j);
    if (i0 < d) {
      float wv[8], o[8];
      load8(w + i0, wv);
#pragma unroll
      for (int e = 0; e < 8; ++e) o[e] = v[j][e] * r * wv[e];
      store8(y + row * d + i0, o);
    }
  }
}

// One wave per row; lane holds elements lane + 64*j, j < PER (64*PER >= d).
template <typename TX, typename TB, typename TS, typename TY, int PER, int OP>
__global__ __launch_bounds__(256) void row_norm_kernel(const TX* __restrict__ x, int64_t x_stride,
                                                       const TB* __restrict__ bsrc,
                                                       const uint8_t* __restrict__ mask,
                                                       const float* __restrict__ w, TS* __restrict__ s,
                                                       TY* __restrict__ y, int64_t rows, int d, float eps) {
  const int lane = threadIdx.x & 63;
  const int64_t row = static_cast<int64_t>(blockIdx.x) * kRowsPerBlock + (threadIdx.x >> 6);
  if (row >= rows) return;
  const bool keep = (OP != kNormAdd && OP != kNormMask) || mask == nullptr || mask[row] != 0;
  float v[PER];
  float ss = 0.f;
#pragma unroll
  for (int j = 0; j < PER; ++j) {
    const int i = lane + 64 * j;
    float val = 0.f;
    if (i < d) {
      val = to_f32(x[row * x_stride + i]);
      if constexpr (OP == kNormAdd) {
        val = keep ? val + to_f32(bsrc[row * d + i]) : 0.f;
        const TS stored = from_f32<TS>(val);
        s[row * d + i] = stored;
        val = to_f32(stored);
      } else if constexpr (OP == kNormMean) {
        val = (val + to_f32(bsrc[row * d + i])) * 0.5f;
      } else if constexpr (OP == kNormMask) {
        const TS stored = from_f32<TS>(keep ? val : 0.f);
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

template <typename TX, typename TB, typename TS, typename TY, int OP>
int launch_row_norm(const void* x, int64_t x_stride, const void* bsrc, const uint8_t* mask,
                    const float* w, void* s, void* y, int64_t rows, int d, float eps,
                    hipStream_t stream) {
  // 8-element vectors pay off once a row fills at least half a wave of them
  const bool vec = d >= 256 && d % 8 == 0 && x_stride % 8 == 0 && aligned16(x) && aligned16(w) &&
                   aligned16(y) && (OP == kNormPlain || OP == kNormMask || aligned16(bsrc)) &&
                   ((OP != kNormAdd && OP != kNormMask) || aligned16(s));
  if (vec) {
    int per8 = 1;
    while (per8 * 512 < d) per8 <<= 1;
    const dim3 grid(static_cast<uint32_t>((rows + kRowsPerBlock - 1) / kRowsPerBlock));
    const dim3 block(64 * kRowsPerBlock);
    const TX* xp = static_cast<const TX*>(x);
    const TB* bp = static_cast<const TB*>(bsrc);
    TS* sp = static_cast<TS*>(s);
    TY* yp = static_cast<TY*>(y);
#define TF_NORM_VEC_CASE(P)                                                                       \
  case P:                                                                                          \
    hipLaunchKernelGGL((row_norm_vec_kernel<TX, TB, TS, TY, P, OP>), grid, block, 0, stream, xp,  \
                       x_stride, bp, mask, w, sp, yp, rows, d, eps);                               \
    return launch_status();
    switch (per8) {
      TF_NORM_VEC_CASE(1)
      TF_NORM_VEC_CASE(2)
      TF_NORM_VEC_CASE(4)
      TF_NORM_VEC_CASE(8)
      default:
        break;
    }
#undef TF_NORM_VEC_CASE
  }
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
    hipLaunchKernelGGL((row_norm_kernel<TX, TB, TS, TY, P, OP>), grid, block, 0, stream, xp,     \
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

// SwiGLU over [rows, 2d] -> [rows, d]; one block per row (element loads: the
// encoder's d = 1365 leaves rows at every 2-byte alignment).
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

// SwiGLU with d % 8 == 0 and aligned rows: 8 outputs per thread, grid-stride
// (vector counts fit int32: the launcher checks).
template <typename T>
__global__ __launch_bounds__(256) void swiglu_vec_kernel(const T* __restrict__ x, T* __restrict__ y, int d8,
                                                         int n8) {
  for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < n8; i += gridDim.x * blockDim.x) {
    const int row = i / d8, c = i - row * d8;
    const int64_t g0 = (static_cast<int64_t>(row) * 2 * d8 + c) * 8;
    float g[8], u[8], o[8];
    load8(x + g0, g);
    load8(x + g0 + static_cast<int64_t>(d8) * 8, u);
#pragma unroll
    for (int e = 0; e < 8; ++e) o[e] = g[e] * sigmoidf(g[e]) * u[e];
    store8(y + static_cast<int64_t>(i) * 8, o);
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

// Row mask through 8-element vectors (d % 8 == 0, aligned): grid-stride over
// vector indices that fit int32 (the launcher checks), 32-bit row division.
template <typename T>
__global__ __launch_bounds__(256) void mask_rows_vec_kernel(const T* __restrict__ x, T* __restrict__ y,
                                                            const uint8_t* __restrict__ mask, int d8, int n8) {
  for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < n8; i += gridDim.x * blockDim.x) {
    const int64_t e0 = static_cast<int64_t>(i) * 8;
    float v[8];
    load8(x + e0, v);
    if (mask[i / d8] == 0) {
#pragma unroll
      for (int e = 0; e < 8; ++e) v[e] = 0.f;
    }
    store8(y + e0, v);
  }
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

template <typename TA, typename TB, typename TY>
__global__ __launch_bounds__(256) void add_vec_kernel(const TA* __restrict__ a, const TB* __restrict__ b,
                                                      const uint8_t* __restrict__ mask, TY* __restrict__ y,
                                                      int d8, int n8) {
  for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < n8; i += gridDim.x * blockDim.x) {
    const int64_t e0 = static_cast<int64_t>(i) * 8;
    float av[8], bv[8];
    load8(a + e0, av);
    load8(b + e0, bv);
    const bool keep = mask == nullptr || mask[i / d8] != 0;
#pragma unroll
    for (int e = 0; e < 8; ++e) av[e] = keep ? av[e] + bv[e] : 0.f;
    store8(y + e0, av);
  }
}

// Grid of a grid-stride vector kernel: enough 256-thread blocks to cover n8
// vectors, capped so large tensors loop instead of launching millions of blocks.
uint32_t vec_blocks(int64_t n8) {
  const int64_t blocks = (n8 + 255) / 256;
  return static_cast<uint32_t>(blocks < 16384 ? blocks : 16384);
}

// Vector path preconditions shared by the flat kernels: whole 8-element
// vectors per row, 16-byte aligned pointers, vector indices within int32.
bool flat_vec_ok(int64_t rows, int64_t d, std::initializer_list<const void*> ptrs) {
  if (d % 8 != 0 || rows * (d / 8) > 0x7fffffff - 65536) return false;
  for (const void* p : ptrs)
    if (!aligned16(p)) return false;
  return true;
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
  const float step = control_step(to_f32(ddt[src]), bias[h]);
  dt[i] = step;
  adt[i] = control_decay(to_f32(a[src]), step, floor_);
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

// Masked mean over 128-byte column slices. Workgroup (slice, b, split) sums
// frames [split*span, (split+1)*span) of clip b, clipped to its valid prefix,
// for the V*8 columns of the slice (V = 16 / sizeof(T) per lane): lane l of
// wave w loads 16 bytes at column V*(l % 8) of frame 8*w + l / 8 + 64*j, eight
// frames in flight per lane, and a lane issues no load past the span's end.
// Lanes l and l^8 meet by a DPP row rotation, then l and l^16 by a swizzle;
// lanes 0-7 and 32-39 of the 8 waves write 16 partial rows to LDS, which one
// thread per column adds in row order, so the sum's order is fixed by
// (span, split count) alone. One split: y = sum / lengths[b]; more: the sum
// goes to partial[split, b, :] and masked_mean_finish_kernel adds the splits in
// order.
template <typename T>
__global__ __launch_bounds__(512) void masked_mean_slice_kernel(const T* __restrict__ x,
                                                                const int64_t* __restrict__ lengths,
                                                                float* __restrict__ y, float* __restrict__ partial,
                                                                int64_t time, int64_t d, int64_t span) {
  constexpr int V = 16 / sizeof(T);
  constexpr int kWaves = 8;
  constexpr int kStep = 8 * kWaves;  // frames per pass of the workgroup
  __shared__ float part[2 * kWaves][8][V];
  const int lane = threadIdx.x & 63;
  const int w = threadIdx.x >> 6;
  const int64_t b = blockIdx.y;
  const int split = blockIdx.z;
  const int64_t col = static_cast<int64_t>(blockIdx.x) * 8 * V + V * (lane & 7);
  const int64_t len = lengths[b];
  const int64_t L = len < 0 ? 0 : (len > time ? time : len);
  const int64_t t0 = split * span;
  const int64_t t1 = t0 + span < L ? t0 + span : L;
  float acc[V];
#pragma unroll
  for (int e = 0; e < V; ++e) acc[e] = 0.f;
  if (col < d) {
    const T* base = x + b * time * d + col;
    for (int64_t t = t0 + 8 * w + (lane >> 3); t < t1; t += 8 * kStep) {
      float v[8][V];
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        // frames past t1 add zero and issue no load
        const int64_t tu = t + u * kStep;
        const T* src = base + tu * d;
        if (tu >= t1) {
#pragma unroll
          for (int e = 0; e < V; ++e) v[u][e] = 0.f;
        } else if constexpr (sizeof(T) == 4) {
          const float4 f = *reinterpret_cast<const float4*>(src);
          v[u][0] = f.x, v[u][1] = f.y, v[u][2] = f.z, v[u][3] = f.w;
        } else {
          const uint4 q = *reinterpret_cast<const uint4*>(src);
          const uint32_t wd[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            v[u][2 * e] = to_f32(__builtin_bit_cast(T, static_cast<uint16_t>(wd[e] & 0xffffu)));
            v[u][2 * e + 1] = to_f32(__builtin_bit_cast(T, static_cast<uint16_t>(wd[e] >> 16)));
          }
        }
      }
#pragma unroll
      for (int u = 0; u < 8; ++u)
#pragma unroll
        for (int e = 0; e < V; ++e) acc[e] += v[u][e];
    }
  }
  constexpr int kRowRor8 = 0x128;     // DPP row_ror:8: lane l reads lane l^8 of its row of 16
  constexpr int kSwizzleXor16 = 0x401f;  // ds_swizzle bit mode, xor mask 16: lane l reads lane l^16
#pragma unroll
  for (int e = 0; e < V; ++e) {
    const int a = __builtin_bit_cast(int, acc[e]);
    acc[e] += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, a, kRowRor8, 0xf, 0xf, false));
    acc[e] += __builtin_bit_cast(float, __builtin_amdgcn_ds_swizzle(__builtin_bit_cast(int, acc[e]), kSwizzleXor16));
  }
  if ((lane & 24) == 0)
#pragma unroll
    for (int e = 0; e < V; ++e) part[2 * w + (lane >> 5)][lane & 7][e] = acc[e];
  __syncthreads();
  const int c = threadIdx.x;  // column of the slice this thread finishes
  if (c >= 8 * V) return;
  const int64_t out_col = static_cast<int64_t>(blockIdx.x) * 8 * V + c;
  if (out_col >= d) return;
  float sum = 0.f;
#pragma unroll
  for (int i = 0; i < 2 * kWaves; ++i) sum += part[i][c / V][c % V];
  if (gridDim.z == 1)
    y[b * d + out_col] = sum / static_cast<float>(len);
  else
    partial[(static_cast<int64_t>(split) * gridDim.y + b) * d + out_col] = sum;
}

// y[b, c] = (partial[0, b, c] + ... + partial[splits-1, b, c]) / lengths[b].
__global__ __launch_bounds__(256) void masked_mean_finish_kernel(const float* __restrict__ partial,
                                                                 const int64_t* __restrict__ lengths,
                                                                 float* __restrict__ y, int64_t batch, int64_t d,
                                                                 int splits) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= batch * d) return;
  float sum = 0.f;
  for (int s = 0; s < splits; ++s) sum += partial[s * batch * d + i];
  y[i] = sum / static_cast<float>(lengths[i / d]);
}

// Time splits of the slice kernel: enough workgroups to give each CU one
// (256), each split at least 64 frames, at most 16 splits.
struct MeanPlan {
  int64_t slices = 0;
  int splits = 1;
  int64_t span = 0;
};

MeanPlan mean_plan(int64_t batch, int64_t time, int64_t d, int64_t elem_bytes) {
  MeanPlan m;
  const int64_t cols = 128 / elem_bytes;
  m.slices = (d + cols - 1) / cols;
  const int64_t groups = m.slices * batch;
  int64_t splits = groups > 0 ? (256 + groups - 1) / groups : 1;
  const int64_t by_time = time / 64;
  if (splits > by_time) splits = by_time;
  if (splits > 16) splits = 16;
  m.splits = splits < 1 ? 1 : static_cast<int>(splits);
  m.span = (time + m.splits - 1) / m.splits;
  if (m.span < 1) m.span = 1;
  return m;
}

__global__ __launch_bounds__(256) void time_mask_kernel(const int64_t* __restrict__ lengths,
                                                        uint8_t* __restrict__ mask, int64_t time,
                                                        int64_t total) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= total) return;
  mask[i] = (i % time) < lengths[i / time] ? 1 : 0;
}

// Two RMSNorms per row, one wave per (row, group): group g of row r is the d
// elements at x + r * x_stride + g * d, normalised with weight w_g into
// y[(2 r + g) * d ...]. The B and C projections of the Mamba-3 block sit side
// by side in the in-projection output, so both norms take one launch.
template <typename TX, typename TY>
__global__ __launch_bounds__(256) void pair_norm_kernel(const TX* __restrict__ x, int64_t x_stride,
                                                        const float* __restrict__ w0, const float* __restrict__ w1,
                                                        TY* __restrict__ y, int64_t rows, int d, float eps) {
  const int lane = threadIdx.x & 63;
  const int64_t vrow = static_cast<int64_t>(blockIdx.x) * kRowsPerBlock + (threadIdx.x >> 6);
  if (vrow >= 2 * rows) return;
  const int64_t row = vrow >> 1;
  const int g = static_cast<int>(vrow & 1);
  const TX* src = x + row * x_stride + g * d;
  const float* w = g ? w1 : w0;
  float ss = 0.f;
  for (int i = lane; i < d; i += 64) {
    const float v = to_f32(src[i]);
    ss += v * v;
  }
  ss = wave_sum(ss);
  const float r = rsqrtf(ss / static_cast<float>(d) + eps);
  for (int i = lane; i < d; i += 64) y[vrow * d + i] = from_f32<TY>(to_f32(src[i]) * r * w[i]);
}

// The same through 8-element vectors for power-of-two d in [8, 256]: lane l of
// a wave takes elements 8*(l % (2d/8)) .. +7 of row 256/d * wave + l / (2d/8),
// so a wave moves 256/d whole rows (both groups) per 16-byte access instead of
// one group per 2-byte access; the d/8 lanes of a group reduce by xor shuffles.
template <typename TX, typename TY>
__global__ __launch_bounds__(256) void pair_norm_vec_kernel(const TX* __restrict__ x, int64_t x_stride,
                                                            const float* __restrict__ w0,
                                                            const float* __restrict__ w1, TY* __restrict__ y,
                                                            int64_t rows, int d, float eps) {
  const int lane = threadIdx.x & 63;
  const int per_row = d / 4;  // lanes per row: 2d / 8
  const int64_t row = (static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6)) * (64 / per_row) + lane / per_row;
  const int c = 8 * (lane % per_row);  // column within [group 0 | group 1]
  const int g = c >= d;
  float v[8];
  float ss = 0.f;
  if (row < rows) {
    load8(x + row * x_stride + c, v);
#pragma unroll
    for (int e = 0; e < 8; ++e) ss += v[e] * v[e];
  }
  for (int off = 1; off < d / 8; off <<= 1) ss += __shfl_xor(ss, off);
  if (row >= rows) return;
  const float r = rsqrtf(ss / static_cast<float>(d) + eps);
  float wv[8], o[8];
  load8((g ? w1 : w0) + (c - g * d), wv);
#pragma unroll
  for (int e = 0; e < 8; ++e) o[e] = v[e] * r * wv[e];
  store8(y + row * 2 * d + c, o);
}

// Valid-prefix reversal, one wave per (b, t) row moving U-sized units:
// y[b, t] = x[b, L-1-t] for t < L, else 0 (primitives.py:40-47).
template <typename U>
__global__ __launch_bounds__(256) void reverse_valid_kernel(const U* __restrict__ x, U* __restrict__ y,
                                                            const int64_t* __restrict__ lengths, int time,
                                                            int units, int rows) {
  const int lane = threadIdx.x & 63;
  const int row = static_cast<int>(blockIdx.x) * kRowsPerBlock + static_cast<int>(threadIdx.x >> 6);
  if (row >= rows) return;
  const int b = row / time;
  const int t = row - b * time;
  const int64_t l = lengths[b];
  const int L = l < 0 ? 0 : (l > time ? time : static_cast<int>(l));
  U* dst = y + static_cast<int64_t>(row) * units;
  if (t < L) {
    const U* src = x + (static_cast<int64_t>(b) * time + (L - 1 - t)) * units;
    for (int c = lane; c < units; c += 64) dst[c] = src[c];
  } else {
    for (int c = lane; c < units; c += 64) dst[c] = U{};
  }
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
                          return (tf::launch_row_norm<TX, float, float, TY, tf::kNormPlain>(
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
    return tf::launch_row_norm<float, float, float, float, tf::kNormAdd>(a, d, b, mask, w, s, y, rows, di, eps, st);
  if (b_dtype == TF_FLOAT32 && y_dtype == TF_BFLOAT16)
    return tf::launch_row_norm<float, float, float, bf16_t, tf::kNormAdd>(a, d, b, mask, w, s, y, rows, di, eps, st);
  if (b_dtype == TF_BFLOAT16 && y_dtype == TF_FLOAT32)
    return tf::launch_row_norm<float, bf16_t, float, float, tf::kNormAdd>(a, d, b, mask, w, s, y, rows, di, eps, st);
  if (b_dtype == TF_BFLOAT16 && y_dtype == TF_BFLOAT16)
    return tf::launch_row_norm<float, bf16_t, float, bf16_t, tf::kNormAdd>(a, d, b, mask, w, s, y, rows, di, eps, st);
  return TF_ERR_DTYPE;
}

extern "C" int tf_swiglu(const void* x, void* y, int32_t dtype, int64_t rows, int64_t d,
                         void* stream) {
  if (!x || !y) return TF_ERR_NULL;
  if (rows < 0 || d < 1 || rows > 0x7fffffff) return TF_ERR_SHAPE;
  if (rows == 0) return TF_OK;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const bool vec = tf::flat_vec_ok(rows, d, {x, y});  // whole output vectors; input rows follow
  const int64_t n8 = rows * d / 8;
  TF_DISPATCH(dtype, T,
              if (vec) {
                hipLaunchKernelGGL(tf::swiglu_vec_kernel<T>, dim3(tf::vec_blocks(n8)), dim3(256), 0, s,
                                   static_cast<const T*>(x), static_cast<T*>(y), static_cast<int>(d / 8),
                                   static_cast<int>(n8));
              } else {
                hipLaunchKernelGGL(tf::swiglu_kernel<T>, dim3(static_cast<uint32_t>(rows)), dim3(256), 0, s,
                                   static_cast<const T*>(x), static_cast<T*>(y), d);
              } return tf::launch_status());
  return TF_ERR_DTYPE;
}

extern "C" int tf_mask_rows(const void* x, void* y, int32_t dtype, const uint8_t* mask, int64_t rows,
                            int64_t d, void* stream) {
  if (!x || !y || !mask) return TF_ERR_NULL;
  if (rows < 0 || d < 1 || rows > 0x7fffffff) return TF_ERR_SHAPE;
  if (rows == 0) return TF_OK;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const bool vec = tf::flat_vec_ok(rows, d, {x, y});
  const int64_t n8 = rows * d / 8;
  TF_DISPATCH(dtype, T,
              if (vec) {
                hipLaunchKernelGGL(tf::mask_rows_vec_kernel<T>, dim3(tf::vec_blocks(n8)), dim3(256), 0, s,
                                   static_cast<const T*>(x), static_cast<T*>(y), mask, static_cast<int>(d / 8),
                                   static_cast<int>(n8));
              } else {
                hipLaunchKernelGGL(tf::mask_rows_kernel<T>, dim3(static_cast<uint32_t>(rows)), dim3(256), 0, s,
                                   static_cast<const T*>(x), static_cast<T*>(y), mask, d);
              } return tf::launch_status());
  return TF_ERR_DTYPE;
}

extern "C" int tf_add(const void* a, int32_t a_dtype, const void* b, int32_t b_dtype,
                      const uint8_t* mask, void* y, int32_t y_dtype, int64_t rows, int64_t d,
                      void* stream) {
  if (!a || !b || !y) return TF_ERR_NULL;
  if (rows < 0 || d < 1 || rows > 0x7fffffff) return TF_ERR_SHAPE;
  if (rows == 0) return TF_OK;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const bool vec = tf::flat_vec_ok(rows, d, {a, b, y});
  const int64_t n8 = rows * d / 8;
  TF_DISPATCH(
      a_dtype, TA,
      TF_DISPATCH(b_dtype, TB,
                  TF_DISPATCH(y_dtype, TY,
                              if (vec) {
                                hipLaunchKernelGGL((tf::add_vec_kernel<TA, TB, TY>), dim3(tf::vec_blocks(n8)),
                                                   dim3(256), 0, s, static_cast<const TA*>(a),
                                                   static_cast<const TB*>(b), mask, static_cast<TY*>(y),
                                                   static_cast<int>(d / 8), static_cast<int>(n8));
                              } else {
                                hipLaunchKernelGGL((tf::add_kernel<TA, TB, TY>), dim3(static_cast<uint32_t>(rows)),
                                                   dim3(256), 0, s, static_cast<const TA*>(a),
                                                   static_cast<const TB*>(b), mask, static_cast<TY*>(y), d);
                              } return tf::launch_status())));
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

namespace {

bool mean_slices_ok(const void* x, int32_t dtype, int64_t d) {
  return tf::dtype_ok(dtype) && d % (16 / tf::dtype_size(dtype)) == 0 && tf::aligned16(x);
}

}  // namespace

extern "C" int64_t tf_masked_mean_workspace_size(int32_t dtype, int64_t batch, int64_t time, int64_t d) {
  if (!tf::dtype_ok(dtype) || batch < 0 || time < 0 || d < 1) return -TF_ERR_SHAPE;
  const tf::MeanPlan m = tf::mean_plan(batch, time, d, tf::dtype_size(dtype));
  return m.splits > 1 ? static_cast<int64_t>(m.splits) * batch * d * 4 : 0;
}

extern "C" int tf_masked_mean(const void* x, int32_t dtype, const int64_t* lengths, float* y, int64_t batch,
                              int64_t time, int64_t d, void* workspace, int64_t workspace_bytes, void* stream) {
  if (!x || !lengths || !y) return TF_ERR_NULL;
  if (batch < 0 || time < 0 || d < 1 || batch > 65535) return TF_ERR_SHAPE;
  if (batch == 0) return TF_OK;
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (mean_slices_ok(x, dtype, d)) {
    tf::MeanPlan m = tf::mean_plan(batch, time, d, tf::dtype_size(dtype));
    const int64_t need = static_cast<int64_t>(m.splits) * batch * d * 4;
    if (m.splits > 1 && (workspace == nullptr || workspace_bytes < need ||
                         (reinterpret_cast<uintptr_t>(workspace) & 3) != 0)) {
      m.splits = 1;  // no room for the partial sums: one workgroup per slice over all frames
      m.span = time > 0 ? time : 1;
    }
    if (m.slices > 0x7fffffff) return TF_ERR_SHAPE;
    const dim3 grid(static_cast<uint32_t>(m.slices), static_cast<uint32_t>(batch), static_cast<uint32_t>(m.splits));
    float* partial = static_cast<float*>(workspace);
    TF_DISPATCH(dtype, T,
                hipLaunchKernelGGL(tf::masked_mean_slice_kernel<T>, grid, dim3(512), 0, s,
                                   static_cast<const T*>(x), lengths, y, partial, time, d, m.span);
                if (m.splits > 1) hipLaunchKernelGGL(tf::masked_mean_finish_kernel,
                                                     dim3(tf::blocks_for(batch * d, 256)), dim3(256), 0, s,
                                                     partial, lengths, y, batch, d, m.splits);
                return tf::launch_status());
    return TF_ERR_DTYPE;
  }
  TF_DISPATCH(dtype, T,
              const dim3 grid(tf::blocks_for(d, 64), static_cast<uint32_t>(batch));
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

extern "C" int tf_reverse_valid(const void* x, void* y, int32_t dtype, const int64_t* lengths, int64_t batch,
                                int64_t time, int64_t d, void* stream) {
  if (!x || !y || !lengths) return TF_ERR_NULL;
  if (!tf::dtype_ok(dtype)) return TF_ERR_DTYPE;
  if (batch < 0 || time < 0 || d < 1 || batch * time > 0x7fffffff - 64) return TF_ERR_SHAPE;
  const int rows = static_cast<int>(batch * time);
  if (rows == 0) return TF_OK;
  const int64_t bytes = d * tf::dtype_size(dtype);  // bytes per row
  hipStream_t s = static_cast<hipStream_t>(stream);
  const dim3 grid(tf::blocks_for(rows, tf::kRowsPerBlock)), block(64 * tf::kRowsPerBlock);
  const int t = static_cast<int>(time);
  if (bytes % 16 == 0 && tf::aligned16(x) && tf::aligned16(y)) {
    hipLaunchKernelGGL(tf::reverse_valid_kernel<uint4>, grid, block, 0, s, static_cast<const uint4*>(x),
                       static_cast<uint4*>(y), lengths, t, static_cast<int>(bytes / 16), rows);
  } else if (bytes % 4 == 0 && reinterpret_cast<uintptr_t>(x) % 4 == 0 && reinterpret_cast<uintptr_t>(y) % 4 == 0) {
    hipLaunchKernelGGL(tf::reverse_valid_kernel<uint32_t>, grid, block, 0, s, static_cast<const uint32_t*>(x),
                       static_cast<uint32_t*>(y), lengths, t, static_cast<int>(bytes / 4), rows);
  } else {
    hipLaunchKernelGGL(tf::reverse_valid_kernel<uint16_t>, grid, block, 0, s, static_cast<const uint16_t*>(x),
                       static_cast<uint16_t*>(y), lengths, t, static_cast<int>(bytes / 2), rows);
  }
  return tf::launch_status();
}

extern "C" int tf_mean_rmsnorm(const void* a, int32_t a_dtype, const void* b, int32_t b_dtype, const float* w,
                               float* y, int64_t rows, int64_t d, float eps, void* stream) {
  if (!a || !b || !w || !y) return TF_ERR_NULL;
  if (rows < 0 || d < 1 || d > 4096) return TF_ERR_SHAPE;
  if (rows == 0) return TF_OK;
  hipStream_t s = static_cast<hipStream_t>(stream);
  TF_DISPATCH(a_dtype, TA,
              TF_DISPATCH(b_dtype, TB,
                          return (tf::launch_row_norm<TA, TB, float, float, tf::kNormMean>(
                              a, d, b, nullptr, w, nullptr, y, rows, static_cast<int>(d), eps, s))));
  return TF_ERR_DTYPE;
}

extern "C" int tf_mask_rmsnorm(const void* x, int32_t x_dtype, const uint8_t* mask, const float* w, float* s,
                               void* y, int32_t y_dtype, int64_t rows, int64_t d, float eps, void* stream) {
  if (!x || !w || !s || !y) return TF_ERR_NULL;
  if (rows < 0 || d < 1 || d > 4096) return TF_ERR_SHAPE;
  if (rows == 0) return TF_OK;
  hipStream_t st = static_cast<hipStream_t>(stream);
  TF_DISPATCH(x_dtype, TX,
              TF_DISPATCH(y_dtype, TY,
                          return (tf::launch_row_norm<TX, float, float, TY, tf::kNormMask>(
                              x, d, nullptr, mask, w, s, y, rows, static_cast<int>(d), eps, st))));
  return TF_ERR_DTYPE;
}

extern "C" int tf_rmsnorm_pair(const void* x, int32_t x_dtype, int64_t x_row_stride, const float* w0,
                               const float* w1, void* y, int32_t y_dtype, int64_t rows, int64_t d, float eps,
                               void* stream) {
  if (!x || !w0 || !w1 || !y) return TF_ERR_NULL;
  if (rows < 0 || d < 1 || d > 4096) return TF_ERR_SHAPE;
  if (x_row_stride == 0) x_row_stride = 2 * d;
  if (x_row_stride < 2 * d) return TF_ERR_STRIDE;
  if (rows == 0) return TF_OK;
  hipStream_t st = static_cast<hipStream_t>(stream);
  const bool pow2 = d >= 8 && d <= 256 && (d & (d - 1)) == 0;
  if (pow2 && x_row_stride % 8 == 0 && tf::aligned16(x) && tf::aligned16(y) && tf::aligned16(w0) &&
      tf::aligned16(w1)) {
    const int64_t rows_per_block = 4 * (256 / d);
    const dim3 vgrid(tf::blocks_for(rows, static_cast<int>(rows_per_block))), vblock(256);
    TF_DISPATCH(x_dtype, TX,
                TF_DISPATCH(y_dtype, TY,
                            hipLaunchKernelGGL((tf::pair_norm_vec_kernel<TX, TY>), vgrid, vblock, 0, st,
                                               static_cast<const TX*>(x), x_row_stride, w0, w1,
                                               static_cast<TY*>(y), rows, static_cast<int>(d), eps);
                            return tf::launch_status()));
    return TF_ERR_DTYPE;
  }
  const dim3 grid(tf::blocks_for(2 * rows, tf::kRowsPerBlock)), block(64 * tf::kRowsPerBlock);
  TF_DISPATCH(x_dtype, TX,
              TF_DISPATCH(y_dtype, TY,
                          hipLaunchKernelGGL((tf::pair_norm_kernel<TX, TY>), grid, block, 0, st,
                                             static_cast<const TX*>(x), x_row_stride, w0, w1,
                                             static_cast<TY*>(y), rows, static_cast<int>(d), eps);
                          return tf::launch_status()));
  return TF_ERR_DTYPE;
}
