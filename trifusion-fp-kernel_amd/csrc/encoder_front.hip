// Front and head of the benchmark encoder (4 s mono x 16 clips through a
// strided Conv1d stem, Mamba-3 blocks and a linear head): the stem's channel
// mix and framing, the valid-frame lengths and row mask, and the head's small
// linear layer. Each replaces a handful of tiny torch launches (mask, multiply,
// sum, divide, pad, cast; floor-divide, clamp, compare; cast, GEMM, cast) with
// one kernel, which is what a graph replay of the forward pays for.
#include "common.h"

namespace tf {
namespace {

// framed[b, t, k] = bf16(mono[b, t*stride + k - pad]) for k < K, 0 for
// K <= k < width; mono[b, n] = sum_{c < min(ch, C)} audio[b, c, n] / ch for
// 0 <= n < N, else 0 (zero padding). One 64-thread block per frame row; each
// thread writes 8 consecutive columns, reading them as two float4 when the
// 8 samples are inside the clip and 16-byte aligned.
__global__ __launch_bounds__(64) void frame_audio_kernel(const float* __restrict__ audio,
                                                         const int64_t* __restrict__ channels,
                                                         uint16_t* __restrict__ framed, int C, int N, int T, int K,
                                                         int width, int stride, int pad) {
  const int64_t row = blockIdx.x;  // b * T + t
  const int b = static_cast<int>(row / T);
  const int t = static_cast<int>(row - static_cast<int64_t>(b) * T);
  const int64_t chl = channels[b];
  const int nch = chl < C ? static_cast<int>(chl < 0 ? 0 : chl) : C;
  const float denom = static_cast<float>(chl);
  const float* src = audio + static_cast<int64_t>(b) * C * N;
  uint16_t* dst = framed + row * width;
  for (int k0 = 8 * static_cast<int>(threadIdx.x); k0 < width; k0 += 8 * 64) {
    const int n0 = t * stride + k0 - pad;
    float v[8];
    const bool whole = k0 + 8 <= K && n0 >= 0 && n0 + 8 <= N && ((reinterpret_cast<uintptr_t>(src + n0) & 15) == 0) &&
                       (N % 4 == 0);
    if (whole) {
      float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
      for (int c = 0; c < nch; ++c) {
        const float4* q = reinterpret_cast<const float4*>(src + static_cast<int64_t>(c) * N + n0);
        const float4 a = q[0], bq = q[1];
        acc[0] += a.x, acc[1] += a.y, acc[2] += a.z, acc[3] += a.w;
        acc[4] += bq.x, acc[5] += bq.y, acc[6] += bq.z, acc[7] += bq.w;
      }
#pragma unroll
      for (int e = 0; e < 8; ++e) v[e] = acc[e] / denom;
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int k = k0 + e, n = n0 + e;
        float x = 0.f;
        if (k < K && n >= 0 && n < N) {
          float acc = 0.f;
          for (int c = 0; c < nch; ++c) acc += src[static_cast<int64_t>(c) * N + n];
          x = acc / denom;
        }
        v[e] = x;
      }
    }
    uint32_t wd[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const uint32_t lo = k0 + 2 * q < K ? f32_to_bf16(v[2 * q]) : 0u;
      const uint32_t hi = k0 + 2 * q + 1 < K ? f32_to_bf16(v[2 * q + 1]) : 0u;
      wd[q] = lo | (hi << 16);
    }
    *reinterpret_cast<uint4*>(dst + k0) = make_uint4(wd[0], wd[1], wd[2], wd[3]);
  }
}

// The same framing for a block of F consecutive frames per workgroup when the
// stride is a multiple of 8 samples: the block's audio span (F-1)*stride + K
// samples is read once, coalesced, mixed to mono and rounded to bf16 into LDS
// (zero outside [0, N)); frame t0 + r, columns k0..k0+7, is then the 16 bytes
// at LDS sample r*stride + k0 (16-byte aligned), written as one 16-byte store,
// consecutive threads covering consecutive output bytes. VEC: the span is read
// as float4 (N, pad and the audio base 16-byte aligned, so each 4-sample group
// lies wholly inside or wholly outside the clip). 512 threads: one pass of
// span loads and one of output stores for the stem's 8-frame blocks.
template <bool VEC>
__global__ __launch_bounds__(512) void frame_block_kernel(const float* __restrict__ audio,
                                                          const int64_t* __restrict__ channels,
                                                          uint16_t* __restrict__ framed, int C, int N, int T, int K,
                                                          int width, int stride, int pad, int F) {
  extern __shared__ uint16_t span_bf16[];
  const int b = blockIdx.y;
  const int t0 = static_cast<int>(blockIdx.x) * F;
  const int nf = T - t0 < F ? T - t0 : F;
  const int64_t chl = channels[b];
  const int nch = chl < C ? static_cast<int>(chl < 0 ? 0 : chl) : C;
  const float denom = static_cast<float>(chl);
  const float* src = audio + static_cast<int64_t>(b) * C * N;
  const int n0 = t0 * stride - pad;
  const int span = (nf - 1) * stride + K;
  if constexpr (VEC) {
    for (int g = threadIdx.x; 4 * g < span; g += 512) {
      const int n = n0 + 4 * g;
      float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
      const bool inside = n >= 0 && n < N;
      if (inside)
        for (int c = 0; c < nch; ++c) {
          const float4 a = *reinterpret_cast<const float4*>(src + static_cast<int64_t>(c) * N + n);
          acc.x += a.x, acc.y += a.y, acc.z += a.z, acc.w += a.w;
        }
      const uint32_t lo = inside ? f32_to_bf16(acc.x / denom) | (uint32_t(f32_to_bf16(acc.y / denom)) << 16) : 0u;
      const uint32_t hi = inside ? f32_to_bf16(acc.z / denom) | (uint32_t(f32_to_bf16(acc.w / denom)) << 16) : 0u;
      *reinterpret_cast<uint2*>(span_bf16 + 4 * g) = make_uint2(lo, hi);
    }
  } else {
    for (int i = threadIdx.x; i < span; i += 512) {
      const int n = n0 + i;
      uint16_t v = 0;
      if (n >= 0 && n < N) {
        float acc = 0.f;
        for (int c = 0; c < nch; ++c) acc += src[static_cast<int64_t>(c) * N + n];
        v = f32_to_bf16(acc / denom);
      }
      span_bf16[i] = v;
    }
  }
  __syncthreads();
  const int per_row = width / 8;
  uint16_t* dst = framed + (static_cast<int64_t>(b) * T + t0) * width;
  for (int q = threadIdx.x; q < nf * per_row; q += 512) {
    const int r = q / per_row;
    const int k0 = 8 * (q - r * per_row);
    const uint16_t* row = span_bf16 + r * stride;
    uint4 out;
    if (k0 + 8 <= K) {
      out = *reinterpret_cast<const uint4*>(row + k0);
    } else {
      uint32_t wd[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const uint32_t lo = k0 + 2 * e < K ? row[k0 + 2 * e] : 0u;
        const uint32_t hi = k0 + 2 * e + 1 < K ? row[k0 + 2 * e + 1] : 0u;
        wd[e] = lo | (hi << 16);
      }
      out = make_uint4(wd[0], wd[1], wd[2], wd[3]);
    }
    *reinterpret_cast<uint4*>(dst + static_cast<int64_t>(q) * 8) = out;
  }
}

// frames[b] = clamp(floor(lengths[b] / stride), 1, T); mask[b, t] = t < frames[b].
__global__ __launch_bounds__(256) void frames_mask_kernel(const int64_t* __restrict__ lengths,
                                                          int64_t* __restrict__ frames,
                                                          uint8_t* __restrict__ mask, int64_t stride, int T,
                                                          int64_t total) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= total) return;
  const int64_t b = i / T;
  const int t = static_cast<int>(i - b * T);
  const int64_t l = lengths[b];
  int64_t q = l / stride;
  if ((l % stride != 0) && ((l < 0) != (stride < 0))) --q;  // floor division
  const int64_t f = q < 1 ? 1 : (q > T ? T : q);
  mask[i] = t < f ? 1 : 0;
  if (t == 0) frames[b] = f;
}

// y[b, o] = round_bf16(sum_k round_bf16(x[b, k]) * round_bf16(w[o, k]) +
// round_bf16(bias[o])) as fp32, one wave per (b, o): the bf16 linear layer of
// an autocast forward (operands cast to bf16, fp32 accumulation, bf16 result).
template <typename TW>
__global__ __launch_bounds__(256) void small_linear_kernel(const float* __restrict__ x, const TW* __restrict__ w,
                                                           const TW* __restrict__ bias, float* __restrict__ y,
                                                           int B, int O, int D) {
  const int lane = threadIdx.x & 63;
  const int item = static_cast<int>(blockIdx.x) * 4 + static_cast<int>(threadIdx.x >> 6);
  if (item >= B * O) return;
  const int b = item / O;
  const int o = item - b * O;
  float acc = 0.f;
  for (int k = lane; k < D; k += 64)
    acc += round_bf16(x[static_cast<int64_t>(b) * D + k]) * round_bf16(to_f32(w[static_cast<int64_t>(o) * D + k]));
  acc = wave_sum(acc);
  if (lane == 0) y[item] = round_bf16(acc + (bias != nullptr ? round_bf16(to_f32(bias[o])) : 0.f));
}

uint32_t grid_for(int64_t n, int per_block, int64_t cap) {
  const int64_t g = (n + per_block - 1) / per_block;
  return static_cast<uint32_t>(g < cap ? g : cap);
}

}  // namespace
}  // namespace tf

extern "C" int tf_frame_audio(const float* audio, const int64_t* channels, void* framed, int64_t batch,
                              int64_t chans, int64_t samples, int64_t frames, int64_t kernel, int64_t width,
                              int64_t stride, int64_t pad, void* stream) {
  if (!audio || !channels || !framed) return TF_ERR_NULL;
  if (batch < 0 || chans < 1 || samples < 0 || frames < 0 || kernel < 1 || stride < 1 || pad < 0)
    return TF_ERR_SHAPE;
  if (width < kernel || width % 8 != 0 || frames != (samples + 2 * pad - kernel) / stride + 1) return TF_ERR_SHAPE;
  if (batch * frames * width > (int64_t(1) << 40) || chans * samples > 0x7fffffff || frames * stride > 0x7fffffff)
    return TF_ERR_SHAPE;
  if ((reinterpret_cast<uintptr_t>(framed) & 15) != 0) return TF_ERR_STRIDE;
  const int64_t rows = batch * frames;
  if (rows == 0) return TF_OK;
  if (rows > 0x7fffffff) return TF_ERR_SHAPE;
  hipStream_t s = static_cast<hipStream_t>(stream);
  // frames per workgroup of the staged form, and its LDS span (samples, padded to 4)
  constexpr int64_t kBlockFrames = 8;
  const int64_t nf = frames < kBlockFrames ? frames : kBlockFrames;
  const int64_t span = ((nf - 1) * stride + kernel + 3) / 4 * 4;
  if (stride % 8 == 0 && span * 2 <= 64 * 1024 && batch <= 65535) {
    const bool vec = samples % 4 == 0 && pad % 4 == 0 && (reinterpret_cast<uintptr_t>(audio) & 15) == 0;
    const dim3 grid(static_cast<uint32_t>((frames + nf - 1) / nf), static_cast<uint32_t>(batch));
    const size_t lds = static_cast<size_t>(span) * 2;
    auto kernel_fn = vec ? tf::frame_block_kernel<true> : tf::frame_block_kernel<false>;
    hipLaunchKernelGGL(kernel_fn, grid, dim3(512), lds, s, audio, channels, static_cast<uint16_t*>(framed),
                       static_cast<int>(chans), static_cast<int>(samples), static_cast<int>(frames),
                       static_cast<int>(kernel), static_cast<int>(width), static_cast<int>(stride),
                       static_cast<int>(pad), static_cast<int>(nf));
    return tf::launch_status();
  }
  hipLaunchKernelGGL(tf::frame_audio_kernel, dim3(static_cast<uint32_t>(rows)), dim3(64), 0, s, audio, channels, static_cast<uint16_t*>(framed),
                     static_cast<int>(chans), static_cast<int>(samples), static_cast<int>(frames),
                     static_cast<int>(kernel), static_cast<int>(width), static_cast<int>(stride),
                     static_cast<int>(pad));
  return tf::launch_status();
}

extern "C" int tf_frames_mask(const int64_t* lengths, int64_t stride, int64_t* frames, uint8_t* mask,
                              int64_t batch, int64_t time, void* stream) {
  if (!lengths || !frames || !mask) return TF_ERR_NULL;
  if (batch < 0 || time < 1 || time > 0x7fffffff || stride == 0) return TF_ERR_SHAPE;
  const int64_t total = batch * time;
  if (total == 0) return TF_OK;
  hipLaunchKernelGGL(tf::frames_mask_kernel, dim3(tf::grid_for(total, 256, int64_t(1) << 31)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), lengths, frames, mask, stride, static_cast<int>(time),
                     total);
  return tf::launch_status();
}

extern "C" int tf_small_linear(const float* x, const void* w, const void* bias, int32_t w_dtype, float* y,
                               int64_t batch, int64_t out_features, int64_t in_features, void* stream) {
  if (!x || !w || !y) return TF_ERR_NULL;
  if (batch < 0 || out_features < 1 || in_features < 1 || batch * out_features > 0x7fffffff ||
      in_features > 0x7fffffff)
    return TF_ERR_SHAPE;
  const int64_t items = batch * out_features;
  if (items == 0) return TF_OK;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const dim3 grid(tf::grid_for(items, 4, int64_t(1) << 31)), block(256);
  TF_DISPATCH(w_dtype, TW,
              hipLaunchKernelGGL(tf::small_linear_kernel<TW>, grid, block, 0, s, x, static_cast<const TW*>(w),
                                 static_cast<const TW*>(bias), y, static_cast<int>(batch),
                                 static_cast<int>(out_features), static_cast<int>(in_features));
              return tf::launch_status());
  return TF_ERR_DTYPE;
}
