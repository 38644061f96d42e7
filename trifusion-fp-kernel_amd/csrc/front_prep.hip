// Small per-forward preparations of the TriFusion front end and frame grids
// (front.py:46-90, masking.py:14-57), each a single launch in place of a run of
// elementwise torch ops:
//   mask_audio     waveform with samples past each clip's length and channels past
//                  its channel count cleared (fp32);
//   log_power      log(1e-6 + sum_c |STFT|^2 / channels) with frames past the
//                  clip's frame count cleared, written [B, frames, bins];
//   front_lengths  frame counts (n // hop + 1) and the counts after each CNN stage;
//   grids          frame mask, pooled lengths and mask, and the left/right pooled
//                  neighbours and weight of every frame.
// Arithmetic follows the torch expressions op by op (no fused multiply-add).
#include "common.h"

#pragma clang fp contract(off)

namespace tf {
namespace {

__global__ __launch_bounds__(256) void mask_audio_kernel(const float* __restrict__ x, const int64_t* __restrict__ lengths,
                                                         const int64_t* __restrict__ channels, float* __restrict__ y,
                                                         int C, int64_t N, int64_t total) {
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < total;
       i += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    const int64_t n = i % N;
    const int64_t bc = i / N;
    const int c = static_cast<int>(bc % C);
    const int64_t b = bc / C;
    y[i] = (n < lengths[b] && c < channels[b]) ? x[i] : 0.f;
  }
}

// spec: complex64 as interleaved floats, element (bc, k, f) at 2 (bc s0 + k s1 + f s2).
__global__ __launch_bounds__(256) void log_power_kernel(const float* __restrict__ spec, int64_t s0, int64_t s1,
                                                        int64_t s2, const int64_t* __restrict__ channels,
                                                        const int64_t* __restrict__ sample_lengths,
                                                        float* __restrict__ y, int C, int K, int F, int hop,
                                                        int64_t total) {
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < total;
       i += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    const int k = static_cast<int>(i % K);
    const int64_t r = i / K;
    const int f = static_cast<int>(r % F);
    const int64_t b = r / F;
    const int64_t frames = sample_lengths[b] / hop + 1;
    float out = 0.f;
    if (f < frames) {
      float p = 0.f;
      for (int c = 0; c < C; ++c) {
        const float* e = spec + 2 * ((b * C + c) * s0 + k * s1 + f * s2);
        const float re = e[0], im = e[1];
        const float pc = re * re + im * im;
        p = c == 0 ? pc : p + pc;
      }
      out = logf(1e-6f + p / static_cast<float>(channels[b]));
    }
    y[i] = out;
  }
}

__global__ void front_lengths_kernel(const int64_t* __restrict__ n, int64_t* __restrict__ out, int B, int hop,
                                     int s0, int s1, int s2) {
  const int b = blockIdx.x * blockDim.x + threadIdx.x;
  if (b >= B) return;
  const int64_t l0 = n[b] / hop + 1;
  const int64_t l1 = (l0 + s0 - 1) / s0;
  const int64_t l2 = (l1 + s1 - 1) / s1;
  const int64_t l3 = (l2 + s2 - 1) / s2;
  out[b] = l0;
  out[B + b] = l1;
  out[2 * B + b] = l2;
  out[3 * B + b] = l3;
}

__global__ __launch_bounds__(256) void grids_kernel(const int64_t* __restrict__ lengths, uint8_t* __restrict__ mask,
                                                    int64_t* __restrict__ low_lengths, uint8_t* __restrict__ low_mask,
                                                    int64_t* __restrict__ left, int64_t* __restrict__ right,
                                                    float* __restrict__ alpha, int B, int T, int LT) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  const int64_t frames = static_cast<int64_t>(B) * T;
  if (i < frames) {
    const int64_t b = i / T;
    const int t = static_cast<int>(i - b * T);
    const int64_t L = lengths[b];
    const int64_t low = (L + 3) / 4;
    mask[i] = t < L ? 1 : 0;
    int64_t l = 0, rr = 0;
    float a = 0.f;
    if (L > 0) {
      float pos = (static_cast<float>(t) + 0.5f) * static_cast<float>(low) / static_cast<float>(L) - 0.5f;
      pos = fmaxf(pos, 0.f);
      pos = fminf(pos, static_cast<float>(low - 1));
      l = static_cast<int64_t>(pos);
      rr = min(l + 1, low - 1);
      a = pos - static_cast<float>(l);
    }
    left[i] = l;
    right[i] = rr;
    alpha[i] = a;
  } else if (i < frames + static_cast<int64_t>(B) * LT) {
    const int64_t k = i - frames;
    const int64_t b = k / LT;
    const int j = static_cast<int>(k - b * LT);
    low_mask[k] = j < (lengths[b] + 3) / 4 ? 1 : 0;
    if (j == 0) low_lengths[b] = (lengths[b] + 3) / 4;
  }
}

uint32_t grid_for(int64_t total) {
  const int64_t blocks = (total + 255) / 256;
  return static_cast<uint32_t>(blocks < 65536 ? blocks : 65536);
}

}  // namespace
}  // namespace tf

extern "C" int tf_mask_audio(const float* audio, const int64_t* lengths, const int64_t* channels, float* y,
                             int64_t batch, int64_t chans, int64_t samples, void* stream) {
  if (!audio || !lengths || !channels || !y) return TF_ERR_NULL;
  if (batch < 0 || chans < 1 || samples < 0) return TF_ERR_SHAPE;
  const int64_t total = batch * chans * samples;
  if (total == 0) return TF_OK;
  hipLaunchKernelGGL(tf::mask_audio_kernel, dim3(tf::grid_for(total)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), audio, lengths, channels, y, static_cast<int>(chans), samples,
                     total);
  return tf::launch_status();
}

extern "C" int tf_log_power(const void* spec, const int64_t* strides, const int64_t* channels,
                            const int64_t* sample_lengths, float* y, int64_t batch, int64_t chans, int64_t bins,
                            int64_t frames, int64_t hop, void* stream) {
  if (!spec || !strides || !channels || !sample_lengths || !y) return TF_ERR_NULL;
  if (batch < 0 || chans < 1 || bins < 1 || frames < 0 || hop < 1 || strides[0] < 0 || strides[1] < 0 ||
      strides[2] < 0)
    return TF_ERR_SHAPE;
  const int64_t total = batch * frames * bins;
  if (total == 0) return TF_OK;
  hipLaunchKernelGGL(tf::log_power_kernel, dim3(tf::grid_for(total)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), static_cast<const float*>(spec), strides[0], strides[1],
                     strides[2], channels, sample_lengths, y, static_cast<int>(chans), static_cast<int>(bins),
                     static_cast<int>(frames), static_cast<int>(hop), total);
  return tf::launch_status();
}

extern "C" int tf_front_lengths(const int64_t* sample_lengths, int64_t* out, int64_t batch, int64_t hop,
                                const int64_t* strides, void* stream) {
  if (!sample_lengths || !out || !strides) return TF_ERR_NULL;
  if (batch < 0 || hop < 1 || strides[0] < 1 || strides[1] < 1 || strides[2] < 1) return TF_ERR_SHAPE;
  if (batch == 0) return TF_OK;
  hipLaunchKernelGGL(tf::front_lengths_kernel, dim3(static_cast<uint32_t>((batch + 255) / 256)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), sample_lengths, out, static_cast<int>(batch),
                     static_cast<int>(hop), static_cast<int>(strides[0]), static_cast<int>(strides[1]),
                     static_cast<int>(strides[2]));
  return tf::launch_status();
}

extern "C" int tf_grids(const int64_t* lengths, void* mask, int64_t* low_lengths, void* low_mask, int64_t* left,
                        int64_t* right, float* alpha, int64_t batch, int64_t time, void* stream) {
  if (!lengths || !mask || !low_lengths || !low_mask || !left || !right || !alpha) return TF_ERR_NULL;
  if (batch < 0 || time < 0 || batch * time > 0x7fffffff) return TF_ERR_SHAPE;
  const int64_t lt = (time + 3) / 4;
  const int64_t total = batch * time + batch * lt;
  if (total == 0) return TF_OK;
  hipLaunchKernelGGL(tf::grids_kernel, dim3(static_cast<uint32_t>((total + 255) / 256)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), lengths, static_cast<uint8_t*>(mask), low_lengths,
                     static_cast<uint8_t*>(low_mask), left, right, alpha, static_cast<int>(batch),
                     static_cast<int>(time), static_cast<int>(lt));
  return tf::launch_status();
}
