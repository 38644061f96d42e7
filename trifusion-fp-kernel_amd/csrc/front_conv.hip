// The TriFusion front end's CNN stage (front.py:8-43) as two fused kernels per
// stage on channels-last bf16 maps [B, T, F, C]:
//   conv1: y = silu(norm1(mask(conv3x3_{stride (s, 2), pad 1}(x))))
//   conv2: y = mask(silu(norm2(mask(conv3x3_{pad 1}(h))) + mask(skip1x1_{stride (s, 2)}(x))))
// where norm is the channel RMSNorm of kernels/buffers.py:58-80 and mask clears
// time steps t >= L. Values are rounded to bf16 wherever the autocast forward
// holds a bf16 tensor: each convolution output, the norm output, the residual
// sum and the SiLU output.
//
// The 3x3 convolutions with cin >= 16 are implicit GEMMs on MFMA 32x32x16 (bf16
// operands, fp32 accumulation). A 256-thread block owns 128 * MT output pixels
// (32 * MT per wave) and all cout channels. The weights of one filter tap,
// [cout][cin], are staged in LDS (double-buffered across taps) and shared by the
// four waves; the pixel operand is read straight from HBM, 8 channels (16 bytes)
// per lane, and reused across taps through the caches. Operands are arranged so
// that the accumulator's lane index is the pixel and its 16 values are output
// channels: the channel RMS then needs one cross-lane add. Every output value is
// one lane's fixed-order sum, so results do not depend on the launch.
//
// The first stage's conv1 has a single input channel (the log power
// spectrogram, fp32) and runs as plain FMAs, one thread per pixel.
#include "common.h"

#pragma clang fp contract(off)

namespace tf {
namespace {

typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8;
typedef __attribute__((ext_vector_type(16))) float f32x16;
typedef __attribute__((ext_vector_type(4))) uint32_t u32x4;
typedef __attribute__((ext_vector_type(2))) uint32_t u32x2;

constexpr int kThreads = 256;

// MFMA 32x32x16 with both operands as rows: D[i][j] += sum_k X[i][k] Y[j][k].
// Lane (c, h) = (l & 31, l >> 5) holds X[c][8h .. 8h+7] and Y[c][8h .. 8h+7];
// D[i][j] sits in lane j + 32 ((i / 4) % 2), element (i / 8) * 4 + i % 4.
__device__ __forceinline__ f32x16 mfma(const u32x4& x, const u32x4& y, const f32x16& acc) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, x), __builtin_bit_cast(bf16x8, y),
                                                 acc, 0, 0, 0);
}

// Output channel (within a 32-channel tile) of accumulator element e in lane half h.
__device__ __forceinline__ int dchan(int e, int h) { return 8 * (e >> 2) + 4 * h + (e & 3); }

__device__ __forceinline__ int clamp_len(const int64_t* lengths, int b, int T) {
  const int64_t l = lengths[b];
  return l < 0 ? 0 : (l > T ? T : static_cast<int>(l));
}

// SiLU as the front norm computes it, y * (1 / (1 + e^-y)).
__device__ __forceinline__ float silu_norm(float y) { return y * (1.0f / (1.0f + expf(-y))); }
// SiLU as torch computes it for a bf16 tensor, x / (1 + e^-x) in fp32.
__device__ __forceinline__ float silu_torch(float x) { return x / (1.0f + expf(-x)); }

__device__ __forceinline__ uint32_t pack2(float lo, float hi) {
  return static_cast<uint32_t>(f32_to_bf16(lo)) | (static_cast<uint32_t>(f32_to_bf16(hi)) << 16);
}

struct StageArgs {
  const uint16_t* x;       // conv input [B, Ti, Fi, CIN] bf16
  const uint16_t* w;       // conv weight [9][cout][CIN] bf16, tap-major
  const float* nw;         // norm weight [cout]
  const void* xs;          // skip input: fp32 [B, Ts, Fs] (CS == 1) or bf16 [B, Ts, Fs, CS]
  const uint16_t* ws;      // skip weight [cout][CS] bf16
  const int64_t* lengths;  // valid output time steps per batch row
  uint16_t* y;             // output [B, To, Fo, cout] bf16
  int Ti, Fi, To, Fo;      // conv input and output grids
  int st, sf;              // conv strides (time, frequency); padding 1
  int Ts, Fs, kst, ksf;    // skip input grid and strides; padding 0
  int64_t M;               // B * To * Fo output pixels
  float eps;
};

// SKIP: 0 = conv1 epilogue (norm, SiLU); 1 = conv2 with a single-channel fp32
// skip input; 2 = conv2 with a CS-channel bf16 skip input.
template <int CIN, int NT, int MT, int SKIP, int CS>
__global__ __launch_bounds__(kThreads) void stage_conv_kernel(StageArgs A) {
  constexpr int COUT = 32 * NT;
  constexpr int KS = CIN / 16;              // MFMA k-steps per tap
  constexpr int ROW = CIN + 8;              // LDS row stride (elements), 16 bytes of padding
  constexpr int WBUF = COUT * ROW;          // one tap's weights in LDS
  constexpr int WCH = COUT * CIN / 8;       // 16-byte chunks per tap
  constexpr int WPT = (WCH + kThreads - 1) / kThreads;
  static_assert(CIN % 16 == 0 && (SKIP != 2 || CS % 16 == 0), "channel counts must be multiples of 16");
  __shared__ __align__(16) uint16_t wl[2 * WBUF];

  const int tid = threadIdx.x;
  const int lane = tid & 63, c32 = lane & 31, hh = lane >> 5;
  const int wave = tid >> 6;
  const int64_t m0 = static_cast<int64_t>(blockIdx.x) * (128 * MT) + wave * (32 * MT);

  // Pixel of each M tile held by this lane: batch row, output (t, f), validity.
  int pb[MT], pt[MT], pf[MT];
  bool pin[MT], pvalid[MT];
  bool any = false;
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    const int64_t m = m0 + 32 * mt + c32;
    pin[mt] = m < A.M;
    const int64_t mm = pin[mt] ? m : 0;
    pf[mt] = static_cast<int>(mm % A.Fo);
    const int64_t r = mm / A.Fo;
    pt[mt] = static_cast<int>(r % A.To);
    pb[mt] = static_cast<int>(r / A.To);
    pvalid[mt] = pin[mt] && pt[mt] < clamp_len(A.lengths, pb[mt], A.To);
    any = any || pvalid[mt];
  }
  // Block-uniform: a block whose pixels are all padding only writes zeros.
  const bool work = __syncthreads_or(any);

  f32x16 acc[MT][NT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int n = 0; n < NT; ++n)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[mt][n][e] = 0.f;

  if (work) {
    u32x4 wst[WPT];
    auto load_w = [&](int tap) {
      const u32x4* src = reinterpret_cast<const u32x4*>(A.w + static_cast<int64_t>(tap) * COUT * CIN);
#pragma unroll
      for (int i = 0; i < WPT; ++i) {
        const int c = tid + i * kThreads;
        if (c < WCH) wst[i] = src[c];
      }
    };
    auto store_w = [&](int buf) {
#pragma unroll
      for (int i = 0; i < WPT; ++i) {
        const int c = tid + i * kThreads;
        if (c < WCH) {
          const int row = c / (CIN / 8), col = c % (CIN / 8);
          *reinterpret_cast<u32x4*>(wl + buf * WBUF + row * ROW + col * 8) = wst[i];
        }
      }
    };
    load_w(0);
    store_w(0);
    __syncthreads();
#pragma unroll 1
    for (int tap = 0; tap < 9; ++tap) {
      if (tap < 8) load_w(tap + 1);
      const int dy = tap / 3, dx = tap % 3;
      u32x4 xa[MT][KS];
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        const int ti = pt[mt] * A.st + dy - 1, fi = pf[mt] * A.sf + dx - 1;
        const bool ok = pvalid[mt] && ti >= 0 && ti < A.Ti && fi >= 0 && fi < A.Fi;
        const u32x4* src = reinterpret_cast<const u32x4*>(
            A.x + ((static_cast<int64_t>(pb[mt]) * A.Ti + (ok ? ti : 0)) * A.Fi + (ok ? fi : 0)) * CIN + 8 * hh);
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
          if (ok) {
            xa[mt][ks] = src[2 * ks];
          } else {
            xa[mt][ks] = u32x4{0u, 0u, 0u, 0u};
          }
        }
      }
      const uint16_t* wt = wl + (tap & 1) * WBUF + c32 * ROW + 8 * hh;
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
#pragma unroll
        for (int n = 0; n < NT; ++n) {
          const u32x4 wv = *reinterpret_cast<const u32x4*>(wt + n * 32 * ROW + 16 * ks);
#pragma unroll
          for (int mt = 0; mt < MT; ++mt) acc[mt][n] = mfma(wv, xa[mt][ks], acc[mt][n]);
        }
      }
      if (tap < 8) store_w((tap + 1) & 1);
      __syncthreads();
    }
  }

#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    // conv output rounded to bf16, cleared past the length; channel sum of squares
    float ss = 0.f;
#pragma unroll
    for (int n = 0; n < NT; ++n)
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const float c = pvalid[mt] ? round_bf16(acc[mt][n][e]) : 0.f;
        acc[mt][n][e] = c;
        ss += c * c;
      }
    ss += __shfl_xor(ss, 32, 64);
    const float r = rsqrtf(ss / static_cast<float>(COUT) + A.eps);

    f32x16 sk[NT];
    if constexpr (SKIP == 2) {
#pragma unroll
      for (int n = 0; n < NT; ++n)
#pragma unroll
        for (int e = 0; e < 16; ++e) sk[n][e] = 0.f;
      // MFMA runs with every lane active; padding pixels contribute zeros
      const u32x4* src = reinterpret_cast<const u32x4*>(
          static_cast<const uint16_t*>(A.xs) +
          ((static_cast<int64_t>(pb[mt]) * A.Ts + static_cast<int64_t>(pt[mt]) * A.kst) * A.Fs +
           static_cast<int64_t>(pf[mt]) * A.ksf) * CS + 8 * hh);
      const u32x4* wsrc = reinterpret_cast<const u32x4*>(A.ws + c32 * CS + 8 * hh);
#pragma unroll
      for (int ks = 0; ks < CS / 16; ++ks) {
        u32x4 xv = u32x4{0u, 0u, 0u, 0u};
        if (pvalid[mt]) xv = src[2 * ks];
#pragma unroll
        for (int n = 0; n < NT; ++n) sk[n] = mfma(wsrc[n * 32 * CS / 8 + 2 * ks], xv, sk[n]);
      }
    }
    float xs1 = 0.f;
    if constexpr (SKIP == 1) {
      if (pvalid[mt]) {
        const float* src = static_cast<const float*>(A.xs);
        xs1 = round_bf16(src[(static_cast<int64_t>(pb[mt]) * A.Ts + static_cast<int64_t>(pt[mt]) * A.kst) * A.Fs +
                             static_cast<int64_t>(pf[mt]) * A.ksf]);
      }
    }

    uint16_t* dst = A.y + (m0 + 32 * mt + c32) * COUT;
#pragma unroll
    for (int n = 0; n < NT && pin[mt]; ++n) {
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        float o[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const int e = 4 * g + q;
          const int ch = n * 32 + dchan(e, hh);
          const float y = round_bf16(acc[mt][n][e] * r * A.nw[ch]);
          if constexpr (SKIP == 0) {
            o[q] = silu_norm(y);
          } else {
            float s = 0.f;
            if constexpr (SKIP == 1) s = round_bf16(xs1 * bf16_to_f32(A.ws[ch]));
            if constexpr (SKIP == 2) s = pvalid[mt] ? round_bf16(sk[n][e]) : 0.f;
            const float a = round_bf16(y + s);
            o[q] = pvalid[mt] ? silu_torch(a) : 0.f;
          }
        }
        *reinterpret_cast<u32x2*>(dst + n * 32 + 8 * g + 4 * hh) = u32x2{pack2(o[0], o[1]), pack2(o[2], o[3])};
      }
    }
  }
}

// First stage conv1: one input channel (fp32 log power, rounded to bf16 as the
// autocast convolution does), 32 output channels, stride (st, 2), padding 1,
// then the norm and SiLU. One thread per output pixel.
__global__ __launch_bounds__(kThreads) void stage_conv1_c1_kernel(const float* __restrict__ x,
                                                                   const uint16_t* __restrict__ w,
                                                                   const float* __restrict__ nw,
                                                                   const int64_t* __restrict__ lengths,
                                                                   uint16_t* __restrict__ y, int Ti, int Fi,
                                                                   int To, int Fo, int st, int64_t M, float eps) {
  constexpr int C = 32;
  __shared__ float ws[9 * C];
  for (int i = threadIdx.x; i < 9 * C; i += kThreads) ws[i] = bf16_to_f32(w[i]);
  __syncthreads();
  const int64_t m = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
  if (m >= M) return;
  const int f = static_cast<int>(m % Fo);
  const int64_t r = m / Fo;
  const int t = static_cast<int>(r % To);
  const int b = static_cast<int>(r / To);
  u32x4* dst = reinterpret_cast<u32x4*>(y + m * C);
  if (t >= clamp_len(lengths, b, To)) {
#pragma unroll
    for (int i = 0; i < C / 8; ++i) dst[i] = u32x4{0u, 0u, 0u, 0u};
    return;
  }
  float xv[9];
#pragma unroll
  for (int tap = 0; tap < 9; ++tap) {
    const int ti = t * st + tap / 3 - 1, fi = 2 * f + tap % 3 - 1;
    xv[tap] = (ti >= 0 && ti < Ti && fi >= 0 && fi < Fi)
                  ? round_bf16(x[(static_cast<int64_t>(b) * Ti + ti) * Fi + fi])
                  : 0.f;
  }
  float c[C];
  float ss = 0.f;
#pragma unroll
  for (int ch = 0; ch < C; ++ch) {
    float a = 0.f;
#pragma unroll
    for (int tap = 0; tap < 9; ++tap) a = __builtin_fmaf(xv[tap], ws[tap * C + ch], a);
    c[ch] = round_bf16(a);
    ss += c[ch] * c[ch];
  }
  const float rr = rsqrtf(ss / static_cast<float>(C) + eps);
#pragma unroll
  for (int i = 0; i < C / 8; ++i) {
    uint32_t p[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int ch = 8 * i + 2 * q;
      p[q] = pack2(silu_norm(round_bf16(c[ch] * rr * nw[ch])), silu_norm(round_bf16(c[ch + 1] * rr * nw[ch + 1])));
    }
    dst[i] = u32x4{p[0], p[1], p[2], p[3]};
  }
}

template <int CIN, int NT, int MT, int SKIP, int CS>
int launch_stage(const StageArgs& a, hipStream_t s) {
  const int64_t blocks = (a.M + 128 * MT - 1) / (128 * MT);
  hipLaunchKernelGGL((stage_conv_kernel<CIN, NT, MT, SKIP, CS>), dim3(static_cast<uint32_t>(blocks)),
                     dim3(kThreads), 0, s, a);
  return launch_status();
}

// Pixels per wave: two 32-pixel tiles while the accumulators stay small.
template <int CIN, int NT, int SKIP, int CS>
int launch_tiles(const StageArgs& a, hipStream_t s) {
  if constexpr (NT <= 2) {
    return launch_stage<CIN, NT, 2, SKIP, CS>(a, s);
  } else {
    return launch_stage<CIN, NT, 1, SKIP, CS>(a, s);
  }
}

int out_grid(int64_t in, int64_t stride) { return static_cast<int>((in - 1) / stride + 1); }

}  // namespace
}  // namespace tf

extern "C" int tf_front_conv1(const void* x, int32_t x_dtype, const void* w, const float* norm_w,
                              const int64_t* lengths, void* y, int64_t batch, int64_t time_in, int64_t freq_in,
                              int64_t cin, int64_t cout, int64_t stride, float eps, void* stream) {
  if (!x || !w || !norm_w || !lengths || !y) return TF_ERR_NULL;
  if (batch < 0 || time_in < 1 || freq_in < 1 || stride < 1 || batch * time_in * freq_in > 0x7fffffffLL)
    return TF_ERR_SHAPE;
  const bool c1 = x_dtype == TF_FLOAT32 && cin == 1 && cout == 32;
  const bool mf = x_dtype == TF_BFLOAT16 && (cin == 32 || cin == 64) && (cout == 32 || cout == 64 || cout == 128);
  if (x_dtype != TF_FLOAT32 && x_dtype != TF_BFLOAT16) return TF_ERR_DTYPE;
  if (!c1 && !mf) return TF_ERR_SHAPE;
  const int To = tf::out_grid(time_in, stride), Fo = tf::out_grid(freq_in, 2);
  const int64_t M = batch * To * Fo;
  if (M == 0) return TF_OK;
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (c1) {
    hipLaunchKernelGGL(tf::stage_conv1_c1_kernel, dim3(static_cast<uint32_t>((M + tf::kThreads - 1) / tf::kThreads)),
                       dim3(tf::kThreads), 0, s, static_cast<const float*>(x), static_cast<const uint16_t*>(w), norm_w,
                       lengths, static_cast<uint16_t*>(y), static_cast<int>(time_in), static_cast<int>(freq_in), To,
                       Fo, static_cast<int>(stride), M, eps);
    return tf::launch_status();
  }
  tf::StageArgs a{};
  a.x = static_cast<const uint16_t*>(x);
  a.w = static_cast<const uint16_t*>(w);
  a.nw = norm_w;
  a.lengths = lengths;
  a.y = static_cast<uint16_t*>(y);
  a.Ti = static_cast<int>(time_in);
  a.Fi = static_cast<int>(freq_in);
  a.To = To;
  a.Fo = Fo;
  a.st = static_cast<int>(stride);
  a.sf = 2;
  a.M = M;
  a.eps = eps;
#define TF_CONV1(CI, NTV) \
  if (cin == CI && cout == 32 * NTV) return tf::launch_tiles<CI, NTV, 0, 16>(a, s);
  TF_CONV1(32, 1) TF_CONV1(32, 2) TF_CONV1(32, 4) TF_CONV1(64, 1) TF_CONV1(64, 2) TF_CONV1(64, 4)
#undef TF_CONV1
  return TF_ERR_SHAPE;
}

extern "C" int tf_front_conv2(const void* h, const void* w, const float* norm_w, const void* x, int32_t x_dtype,
                              const void* w_skip, const int64_t* lengths, void* y, int64_t batch, int64_t time_in,
                              int64_t freq_in, int64_t cin, int64_t cout, int64_t stride, float eps, void* stream) {
  if (!h || !w || !norm_w || !x || !w_skip || !lengths || !y) return TF_ERR_NULL;
  if (batch < 0 || time_in < 1 || freq_in < 1 || stride < 1 || batch * time_in * freq_in > 0x7fffffffLL)
    return TF_ERR_SHAPE;
  if (x_dtype != TF_FLOAT32 && x_dtype != TF_BFLOAT16) return TF_ERR_DTYPE;
  if (x_dtype == TF_FLOAT32 ? cin != 1 : (cin != 32 && cin != 64)) return TF_ERR_SHAPE;
  if (cout != 32 && cout != 64 && cout != 128) return TF_ERR_SHAPE;
  const int To = tf::out_grid(time_in, stride), Fo = tf::out_grid(freq_in, 2);
  const int64_t M = batch * To * Fo;
  if (M == 0) return TF_OK;
  hipStream_t s = static_cast<hipStream_t>(stream);
  tf::StageArgs a{};
  a.x = static_cast<const uint16_t*>(h);
  a.w = static_cast<const uint16_t*>(w);
  a.nw = norm_w;
  a.xs = x;
  a.ws = static_cast<const uint16_t*>(w_skip);
  a.lengths = lengths;
  a.y = static_cast<uint16_t*>(y);
  a.Ti = To;
  a.Fi = Fo;
  a.To = To;
  a.Fo = Fo;
  a.st = 1;
  a.sf = 1;
  a.Ts = static_cast<int>(time_in);
  a.Fs = static_cast<int>(freq_in);
  a.kst = static_cast<int>(stride);
  a.ksf = 2;
  a.M = M;
  a.eps = eps;
#define TF_CONV2(CO, NTV)                                                    \
  if (cout == CO) {                                                          \
    if (cin == 1) return tf::launch_tiles<CO, NTV, 1, 16>(a, s);             \
    if (cin == 32) return tf::launch_tiles<CO, NTV, 2, 32>(a, s);            \
    return tf::launch_tiles<CO, NTV, 2, 64>(a, s);                           \
  }
  TF_CONV2(32, 1) TF_CONV2(64, 2) TF_CONV2(128, 4)
#undef TF_CONV2
  return TF_ERR_SHAPE;
}
