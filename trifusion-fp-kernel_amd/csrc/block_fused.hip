// Fused kernels of the TriFusion block (model.py:140-200) under bf16 autocast.
// Each replaces a run of the reference's elementwise ops, casts and small
// launches around the block's GEMMs with one HBM pass, keeping the values the
// autocast forward produces:
//   block_pre      mask_buffer(x) -> pre RMSNorm -> bf16 copy for local.up, and
//                  the 4:1 pooled grid (fp32 pooling of the fp32 norm) as bf16
//                  for the attention's qkv projection (model.py:144-160,
//                  masking.py:59-67);
//   glu_depthwise  F.glu -> masked depthwise conv (model.py:73);
//   norm_silu      RMSNorm of a bf16 row -> SiLU (model.py:74);
//   attention      rotary q/k (bf16) -> masked fp32 softmax attention ->
//                  [B, T, H D] bf16 (model.py:84-104, attention.py:8-18);
//   merge_gate     mean of the two Mamba directions -> RMSNorm (fp32), and the
//                  3-way gate linear of cat(cn, mn, an) (model.py:180-186);
//   merge_conv     gated concatenation (fp32) -> masked depthwise conv (bf16)
//                  -> residual add rounded to bf16 (model.py:187-196).
// Arithmetic per element follows the unfused kernels the block otherwise runs
// (the row norms of elementwise.hip, the depthwise, pooling, rotary and gate
// kernels of trifusion_block.hip), so outputs match those paths bit for bit
// except the gate dot product and the attention, whose sums run in another
// order than the library GEMM and softmax.
#include "common.h"

namespace tf {
namespace {

// Eight bf16 values (16 bytes) as floats (exact).
__device__ __forceinline__ void unpack8(const uint4& u, float (&v)[8]) {
  const uint32_t wd[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    v[2 * e] = __uint_as_float(wd[e] << 16);
    v[2 * e + 1] = __uint_as_float(wd[e] & 0xffff0000u);
  }
}

template <typename T>
__device__ __forceinline__ void ld8(const T* p, float (&v)[8]) {
  if constexpr (sizeof(T) == 4) {
    const float4 a = reinterpret_cast<const float4*>(p)[0];
    const float4 b = reinterpret_cast<const float4*>(p)[1];
    v[0] = a.x, v[1] = a.y, v[2] = a.z, v[3] = a.w;
    v[4] = b.x, v[5] = b.y, v[6] = b.z, v[7] = b.w;
  } else {
    unpack8(*reinterpret_cast<const uint4*>(p), v);
  }
}

__device__ __forceinline__ void st8_f32(float* p, const float (&v)[8]) {
  reinterpret_cast<float4*>(p)[0] = make_float4(v[0], v[1], v[2], v[3]);
  reinterpret_cast<float4*>(p)[1] = make_float4(v[4], v[5], v[6], v[7]);
}

__device__ __forceinline__ void st8_bf16(uint16_t* p, const float (&v)[8]) {
  uint32_t wd[4];
#pragma unroll
  for (int e = 0; e < 4; ++e)
    wd[e] = static_cast<uint32_t>(f32_to_bf16(v[2 * e])) | (static_cast<uint32_t>(f32_to_bf16(v[2 * e + 1])) << 16);
  *reinterpret_cast<uint4*>(p) = make_uint4(wd[0], wd[1], wd[2], wd[3]);
}

__device__ __forceinline__ int clamp_len(const int64_t* lengths, int b, int T) {
  const int64_t l = lengths[b];
  return l < 0 ? 0 : (l > T ? T : static_cast<int>(l));
}

// 1 / (1 + e^-x), as the block kernels compute the gate sigmoid.
__device__ __forceinline__ float sigmoid_acc(float x) { return 1.0f / (1.0f + expf(-x)); }

// fp32 ops with fused multiply-add disabled (the block kernels' convention).
__device__ __forceinline__ float mul_nc(float a, float b) {
#pragma clang fp contract(off)
  return a * b;
}
__device__ __forceinline__ float add_nc(float a, float b) {
#pragma clang fp contract(off)
  return a + b;
}

// ---- mask + pre RMSNorm + 4:1 pool ---------------------------------------------
// Block (j, b): its four waves take rows t = 4j + k. Each row is masked
// (t >= L -> 0, written to xm), normalised like the fp32 row norm (wave per row,
// lane holds elements 8 (lane + 64 i) .. +7) and written as bf16; the fp32 norm
// rows meet in LDS for the pooled row: sum over valid rows in order, / count.
template <int PER8, bool ADD>
__global__ __launch_bounds__(256) void block_pre_kernel(const float* __restrict__ x,
                                                        const uint16_t* __restrict__ addend,
                                                        const int64_t* __restrict__ lengths,
                                                        const float* __restrict__ w, float* __restrict__ xm,
                                                        uint16_t* __restrict__ h16, uint16_t* __restrict__ p16,
                                                        int T, int LT, int d, float eps) {
  // fp32 norm rows as float4 [4 rows][2 halves][d / 8]: half e of 8-element group
  // c8 holds elements 8 c8 + 4 e .. + 3, so consecutive lanes touch consecutive
  // 16-byte slots (conflict-free LDS access)
  extern __shared__ float4 hs4[];
  const int lane = threadIdx.x & 63, k = threadIdx.x >> 6;
  const int j = blockIdx.x, b = blockIdx.y;
  const int t = 4 * j + k;
  const int L = clamp_len(lengths, b, T);
  if (t < T) {
    const int64_t row = static_cast<int64_t>(b) * T + t;
    const bool keep = t < L;
    float v[PER8][8];
    float ss = 0.f;
#pragma unroll
    for (int i = 0; i < PER8; ++i) {
      const int i0 = 8 * (lane + 64 * i);
      if (i0 < d) {
        ld8(x + row * d + i0, v[i]);
        if constexpr (ADD) {
          // the previous block's closing residual add (masked add kernel: a + b in fp32)
          float av[8];
          ld8(addend + row * d + i0, av);
#pragma unroll
          for (int e = 0; e < 8; ++e) v[i][e] = v[i][e] + av[e];
        }
#pragma unroll
        for (int e = 0; e < 8; ++e) v[i][e] = keep ? v[i][e] : 0.f;
        st8_f32(xm + row * d + i0, v[i]);
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) v[i][e] = 0.f;
      }
#pragma unroll
      for (int e = 0; e < 8; ++e) ss += v[i][e] * v[i][e];
    }
    ss = wave_sum(ss);
    const float r = rsqrtf(ss / static_cast<float>(d) + eps);
#pragma unroll
    for (int i = 0; i < PER8; ++i) {
      const int i0 = 8 * (lane + 64 * i);
      if (i0 < d) {
        float wv[8], o[8];
        ld8(w + i0, wv);
#pragma unroll
        for (int e = 0; e < 8; ++e) o[e] = v[i][e] * r * wv[e];
        st8_bf16(h16 + row * d + i0, o);
        const int c8 = lane + 64 * i;
        hs4[(2 * k) * (d / 8) + c8] = make_float4(o[0], o[1], o[2], o[3]);
        hs4[(2 * k + 1) * (d / 8) + c8] = make_float4(o[4], o[5], o[6], o[7]);
      }
    }
  }
  __syncthreads();
  const int count = max(min(L - 4 * j, 4), 1);
  const int64_t prow = static_cast<int64_t>(b) * LT + j;
  for (int c8 = threadIdx.x; c8 < d / 8; c8 += blockDim.x) {
    float hv[4][8];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const float4 lo = hs4[(2 * q) * (d / 8) + c8], hi = hs4[(2 * q + 1) * (d / 8) + c8];
      const float e8[8] = {lo.x, lo.y, lo.z, lo.w, hi.x, hi.y, hi.z, hi.w};
#pragma unroll
      for (int e = 0; e < 8; ++e) hv[q][e] = 4 * j + q < L ? e8[e] : 0.f;
    }
    float o[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      float acc = 0.f;
#pragma unroll
      for (int q = 0; q < 4; ++q) acc = add_nc(acc, hv[q][e]);
      o[e] = acc / static_cast<float>(count);
    }
    st8_bf16(p16 + prow * d + 8 * c8, o);
  }
}

// ---- RMSNorm of a bf16 row, then SiLU ------------------------------------------
template <int PER8>
__global__ __launch_bounds__(256) void norm_silu_kernel(const uint16_t* __restrict__ x, const float* __restrict__ w,
                                                        uint16_t* __restrict__ y, int64_t rows, int d, float eps) {
  const int lane = threadIdx.x & 63;
  const int64_t row = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;
  float v[PER8][8];
  float ss = 0.f;
#pragma unroll
  for (int i = 0; i < PER8; ++i) {
    const int i0 = 8 * (lane + 64 * i);
    if (i0 < d) {
      ld8(x + row * d + i0, v[i]);
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) v[i][e] = 0.f;
    }
#pragma unroll
    for (int e = 0; e < 8; ++e) ss += v[i][e] * v[i][e];
  }
  ss = wave_sum(ss);
  const float r = rsqrtf(ss / static_cast<float>(d) + eps);
#pragma unroll
  for (int i = 0; i < PER8; ++i) {
    const int i0 = 8 * (lane + 64 * i);
    if (i0 < d) {
      float wv[8], o[8];
      ld8(w + i0, wv);
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float n = round_bf16(v[i][e] * r * wv[e]);
        o[e] = n / (1.0f + expf(-n));
      }
      st8_bf16(y + row * d + i0, o);
    }
  }
}

// Depthwise taps of 8 consecutive channels ([channel][K] bf16, 16-byte aligned:
// 8 K elements are K 16-byte vectors) and their biases (one 16-byte vector).
template <int K>
__device__ __forceinline__ void load_taps(const uint16_t* w, const uint16_t* bias, float (&wk)[8][K], float (&bb)[8]) {
  float flat[8 * K];
#pragma unroll
  for (int v = 0; v < K; ++v) {
    float part[8];
    ld8(w + 8 * v, part);
#pragma unroll
    for (int e = 0; e < 8; ++e) flat[8 * v + e] = part[e];
  }
#pragma unroll
  for (int e = 0; e < 8; ++e)
#pragma unroll
    for (int q = 0; q < K; ++q) wk[e][q] = flat[e * K + q];
  ld8(bias, bb);
}

// ---- GLU + masked depthwise conv ----------------------------------------------
// One workgroup per (512 channels, TW time steps, batch row), lane = 8 channels.
// Its four waves form the GLU rows t0 - K/2 .. t0 + TW - 1 + K/2 once (row r by
// wave r % 4, a * 1 / (1 + e^-b) rounded to bf16, kept as bf16 in LDS), then
// each wave convolves TW / 4 consecutive time steps from LDS. Sources outside
// [0, T) are 0, outputs at t >= L are 0.
template <int K, int TW>
__global__ __launch_bounds__(256) void glu_depthwise_kernel(const uint16_t* __restrict__ up,
                                                            const uint16_t* __restrict__ w,
                                                            const uint16_t* __restrict__ bias,
                                                            const int64_t* __restrict__ lengths,
                                                            uint16_t* __restrict__ y, int T, int d) {
  constexpr int R = TW + K - 1;  // GLU rows of the tile
  constexpr int TO = TW / 4;     // outputs per wave
  static_assert(TW % 4 == 0, "four waves share the tile's time steps");
  __shared__ uint4 glu[R][64];   // [row][lane]: 8 bf16 channels per 16 bytes
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int t0 = blockIdx.y * TW, b = blockIdx.z;
  const int L = clamp_len(lengths, b, T);
  const int c8 = blockIdx.x * 64 + lane;
  const bool on = c8 < d / 8;
  const int c = 8 * c8;
  // The wave's GLU rows r = wave + 4 i: every load is issued before the first
  // is used, from a clamped row and channel (values outside the tile, [0, T) or
  // the channels dropped), so no load waits behind the one before.
  constexpr int NR = (R + 3) / 4;
  uint4 ra[NR], rg[NR];
#pragma unroll
  for (int i = 0; i < NR; ++i) {
    const int t = min(max(t0 - K / 2 + wave + 4 * i, 0), T - 1);
    const uint16_t* src = up + (static_cast<int64_t>(b) * T + t) * 2 * d + (on ? c : 0);
    ra[i] = *reinterpret_cast<const uint4*>(src);
    rg[i] = *reinterpret_cast<const uint4*>(src + d);
  }
#pragma unroll
  for (int i = 0; i < NR; ++i) {
    const int r = wave + 4 * i;
    if (r < R) {
      const int t = t0 - K / 2 + r;
      float o[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
      if (on && t >= 0 && t < T) {
        float a[8], g[8];
        unpack8(ra[i], a);
        unpack8(rg[i], g);
#pragma unroll
        for (int e = 0; e < 8; ++e) o[e] = a[e] * (1.0f / (1.0f + expf(-g[e])));
      }
      uint32_t wd[4];
#pragma unroll
      for (int e = 0; e < 4; ++e)
        wd[e] = static_cast<uint32_t>(f32_to_bf16(o[2 * e])) | (static_cast<uint32_t>(f32_to_bf16(o[2 * e + 1])) << 16);
      glu[r][lane] = make_uint4(wd[0], wd[1], wd[2], wd[3]);
    }
  }
  __syncthreads();
  if (!on) return;
  float wk[8][K], bb[8];
  load_taps<K>(w + static_cast<int64_t>(c) * K, bias + c, wk, bb);
  float win[TO + K - 1][8];
#pragma unroll
  for (int r = 0; r < TO + K - 1; ++r) {
    const uint4 q = glu[wave * TO + r][lane];
    const uint32_t wd[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      win[r][2 * e] = __uint_as_float(wd[e] << 16);
      win[r][2 * e + 1] = __uint_as_float(wd[e] & 0xffff0000u);
    }
  }
#pragma unroll
  for (int i = 0; i < TO; ++i) {
    const int t = t0 + wave * TO + i;
    if (t < T) {
      float o[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        float acc = 0.f;
        if (t < L) {
#pragma unroll
          for (int q = 0; q < K; ++q) acc = add_nc(acc, mul_nc(win[i + q][e], wk[e][q]));
          acc = add_nc(acc, bb[e]);
        }
        o[e] = acc;
      }
      st8_bf16(y + (static_cast<int64_t>(b) * T + t) * d + c, o);
    }
  }
}

// ---- GLU + masked depthwise conv, then RMSNorm + SiLU of each output row -------
// glu_depthwise_kernel followed by norm_silu_kernel in one launch: one
// workgroup per (TW time steps, batch row) owns whole rows (d <= 512 PER8). The
// GLU rows of the tile go to LDS (bf16) as glu_depthwise forms them; wave w
// convolves output rows t0 + TO w .. + TO - 1 for every channel (lane = channel
// groups 8 (lane + 64 j)), rounds them to bf16 as glu_depthwise's output is, and
// normalises each row as norm_silu does (same per-lane order of the sum of
// squares), so the values are those of the two launches.
template <int K, int TW, int PER8>
__global__ __launch_bounds__(256) void glu_norm_silu_kernel(const uint16_t* __restrict__ up,
                                                            const uint16_t* __restrict__ w,
                                                            const uint16_t* __restrict__ bias,
                                                            const int64_t* __restrict__ lengths,
                                                            const float* __restrict__ nw, uint16_t* __restrict__ y,
                                                            int T, int d, float eps) {
  constexpr int R = TW + K - 1;
  constexpr int TO = TW / 4;
  static_assert(TW % 4 == 0, "four waves share the tile's time steps");
  extern __shared__ uint4 glu_s[];  // [R][d / 8]
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int t0 = blockIdx.x * TW, b = blockIdx.y;
  const int L = clamp_len(lengths, b, T);
  const int d8 = d / 8;
  // All of the thread's GLU-row loads are issued before the first is used, at
  // most NL of each half (d <= 512 PER8): a slot past the tile or a row outside
  // [0, T) reads a clamped, valid address and its values are dropped. Loads
  // consumed inside a runtime-bounded loop would each wait for the one before.
  constexpr int NL = (R * 64 * PER8 + 255) / 256;
  uint4 ra[NL], rg[NL];
#pragma unroll
  for (int i = 0; i < NL; ++i) {
    const int idx = static_cast<int>(threadIdx.x) + 256 * i;
    const int r = idx / d8, c8 = idx < R * d8 ? idx - r * d8 : 0;
    const int t = min(max(t0 - K / 2 + r, 0), T - 1);
    const uint16_t* src = up + (static_cast<int64_t>(b) * T + t) * 2 * d + 8 * c8;
    ra[i] = *reinterpret_cast<const uint4*>(src);
    rg[i] = *reinterpret_cast<const uint4*>(src + d);
  }
#pragma unroll
  for (int i = 0; i < NL; ++i) {
    const int idx = static_cast<int>(threadIdx.x) + 256 * i;
    if (idx < R * d8) {
      const int r = idx / d8, c8 = idx - r * d8;
      const int t = t0 - K / 2 + r;
      float o[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
      if (t >= 0 && t < T) {
        float a[8], g[8];
        unpack8(ra[i], a);
        unpack8(rg[i], g);
#pragma unroll
        for (int e = 0; e < 8; ++e) o[e] = a[e] * (1.0f / (1.0f + expf(-g[e])));
      }
      uint32_t wd[4];
#pragma unroll
      for (int e = 0; e < 4; ++e)
        wd[e] = static_cast<uint32_t>(f32_to_bf16(o[2 * e])) | (static_cast<uint32_t>(f32_to_bf16(o[2 * e + 1])) << 16);
      glu_s[r * d8 + c8] = make_uint4(wd[0], wd[1], wd[2], wd[3]);
    }
  }
  __syncthreads();
  float cv[TO][PER8][8];
#pragma unroll
  for (int j = 0; j < PER8; ++j) {
    const int c8 = lane + 64 * j;
    if (c8 < d8) {
      float wk[8][K], bb[8];
      load_taps<K>(w + static_cast<int64_t>(8 * c8) * K, bias + 8 * c8, wk, bb);
      float win[TO + K - 1][8];
#pragma unroll
      for (int r = 0; r < TO + K - 1; ++r) {
        const uint4 q = glu_s[(wave * TO + r) * d8 + c8];
        const uint32_t wd[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          win[r][2 * e] = __uint_as_float(wd[e] << 16);
          win[r][2 * e + 1] = __uint_as_float(wd[e] & 0xffff0000u);
        }
      }
#pragma unroll
      for (int i = 0; i < TO; ++i) {
        const int t = t0 + wave * TO + i;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          float acc = 0.f;
          if (t < L) {
#pragma unroll
            for (int q = 0; q < K; ++q) acc = add_nc(acc, mul_nc(win[i + q][e], wk[e][q]));
            acc = add_nc(acc, bb[e]);
          }
          cv[i][j][e] = round_bf16(acc);
        }
      }
    } else {
#pragma unroll
      for (int i = 0; i < TO; ++i)
#pragma unroll
        for (int e = 0; e < 8; ++e) cv[i][j][e] = 0.f;
    }
  }
#pragma unroll
  for (int i = 0; i < TO; ++i) {
    const int t = t0 + wave * TO + i;
    if (t < T) {  // wave-uniform
      float ss = 0.f;
#pragma unroll
      for (int j = 0; j < PER8; ++j) {
#pragma unroll
        for (int e = 0; e < 8; ++e) ss += cv[i][j][e] * cv[i][j][e];
      }
      ss = wave_sum(ss);
      const float r = rsqrtf(ss / static_cast<float>(d) + eps);
#pragma unroll
      for (int j = 0; j < PER8; ++j) {
        const int c8 = lane + 64 * j;
        if (c8 < d8) {
          float wv[8], o[8];
          ld8(nw + 8 * c8, wv);
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            const float n = round_bf16(cv[i][j][e] * r * wv[e]);
            o[e] = n / (1.0f + expf(-n));
          }
          st8_bf16(y + (static_cast<int64_t>(b) * T + t) * d + 8 * c8, o);
        }
      }
    }
  }
}

// ---- rotary + masked attention on the pooled grid -------------------------------
// One wave per (tile of 16 queries, head, batch row). Each query belongs to four
// lanes, each holding a quarter of its head dims; together they walk the valid
// keys j < low_length with one online softmax, G keys at a time (independent
// dot products). Keys (rotated and rounded to bf16 like the rotary kernel's
// output) and values of 64 positions at a time sit in LDS as bf16.

// Rotation of the 8 dims 8 c8 .. 8 c8 + 7 of a row (pairs 4 c8 .. 4 c8 + 3):
// x1 cos - x2 sin and x1 sin + x2 cos with separate multiplies and adds, rounded
// to bf16, as the reference's rotary forms them. cs4, sn4: the pairs' cos and
// sin (16-byte aligned).
__device__ __forceinline__ void rotate8(const uint16_t* src, const float* cs4, const float* sn4, float (&o)[8]) {
#pragma clang fp contract(off)
  float v[8];
  ld8(src, v);
  const float4 c = *reinterpret_cast<const float4*>(cs4), n = *reinterpret_cast<const float4*>(sn4);
  const float co[4] = {c.x, c.y, c.z, c.w}, si[4] = {n.x, n.y, n.z, n.w};
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const float a = v[2 * e], z = v[2 * e + 1];
    o[2 * e] = round_bf16(a * co[e] - z * si[e]);
    o[2 * e + 1] = round_bf16(a * si[e] + z * co[e]);
  }
}

constexpr int kAttSplit = 4;                  // lanes per query
constexpr int kAttQueries = 64 / kAttSplit;   // queries per wave
constexpr int kAttGroup = 4;                  // keys scored together

// Lane (qi, part) = (lane % 16, lane / 16) holds dims [part D/4, (part+1) D/4) of
// query qi's rotated q and of its output; a score is the sum of the four lanes'
// partial dots (two xor shuffles), so all four keep the same softmax state.
template <int D>
__global__ __launch_bounds__(64) void attention_kernel(const uint16_t* __restrict__ qkv, const float* __restrict__ cs,
                                                       const float* __restrict__ sn,
                                                       const int64_t* __restrict__ low_lengths,
                                                       uint16_t* __restrict__ y, int LT, int H, float scale) {
  constexpr int RS = D + 8;  // LDS row stride (bf16 elements; rows stay 16-byte aligned)
  constexpr int DP = D / kAttSplit;  // dims per lane
  // the rotated keys and the values are bf16 numbers, so bf16 storage is exact
  __shared__ __align__(16) uint16_t ks[64 * RS];
  __shared__ __align__(16) uint16_t vs[64 * RS];
  const int lane = threadIdx.x;
  const int qi = lane % kAttQueries, part = lane / kAttQueries;
  const int t = blockIdx.x * kAttQueries + qi, h = blockIdx.y, b = blockIdx.z;
  const int LL = clamp_len(low_lengths, b, LT);
  const int64_t width = static_cast<int64_t>(3) * H * D;
  constexpr int G8 = D / 8;  // 8-dim groups per row
  // the lane's own dims of its query, rotated (groups part DP / 8 ..)
  float q[DP];
  {
    const int tq = t < LT ? t : 0;
    const uint16_t* qrow = qkv + (static_cast<int64_t>(b) * LT + tq) * width + static_cast<int64_t>(h) * D;
#pragma unroll
    for (int gi = 0; gi < DP / 8; ++gi) {
      const int c8 = part * (DP / 8) + gi;
      float o[8];
      rotate8(qrow + 8 * c8, cs + static_cast<int64_t>(tq) * (D / 2) + 4 * c8,
              sn + static_cast<int64_t>(tq) * (D / 2) + 4 * c8, o);
#pragma unroll
      for (int e = 0; e < 8; ++e) q[8 * gi + e] = o[e];
    }
  }
  float acc[DP];
#pragma unroll
  for (int i = 0; i < DP; ++i) acc[i] = 0.f;
  float m = -INFINITY, l = 0.f;
  for (int j0 = 0; j0 < LL; j0 += 64) {
    const int nk = min(64, LL - j0);
    // stage the tile's keys (rotated) and values: task (row r, group c8) per
    // lane, G8 lanes per row, so a load instruction reads whole 128-byte rows.
    // Rows past the tile's keys repeat its last key (never read by the scores).
#pragma unroll
    for (int it = 0; it < G8; ++it) {
      const int idx = lane + 64 * it, r = idx / G8, c8 = idx % G8;
      const int j = j0 + min(r, nk - 1);
      const uint16_t* row = qkv + (static_cast<int64_t>(b) * LT + j) * width + static_cast<int64_t>(h) * D;
      float o[8];
      rotate8(row + static_cast<int64_t>(H) * D + 8 * c8, cs + static_cast<int64_t>(j) * (D / 2) + 4 * c8,
              sn + static_cast<int64_t>(j) * (D / 2) + 4 * c8, o);
      st8_bf16(ks + r * RS + 8 * c8, o);
      *reinterpret_cast<uint4*>(vs + r * RS + 8 * c8) =
          *reinterpret_cast<const uint4*>(row + static_cast<int64_t>(2) * H * D + 8 * c8);
    }
    __syncthreads();
    const uint16_t* kp = ks + part * DP;
    const uint16_t* vp = vs + part * DP;
    for (int jb = 0; jb < nk; jb += kAttGroup) {
      float sc[kAttGroup];
#pragma unroll
      for (int g = 0; g < kAttGroup; ++g) {
        const int jj = jb + g < nk ? jb + g : 0;
        float part_dot = 0.f;
#pragma unroll
        for (int i = 0; i < DP; i += 8) {
          float kv[8];
          ld8(kp + jj * RS + i, kv);
#pragma unroll
          for (int e = 0; e < 8; e += 2) part_dot += q[i + e] * kv[e] + q[i + e + 1] * kv[e + 1];
        }
        sc[g] = part_dot;
      }
#pragma unroll
      for (int g = 0; g < kAttGroup; ++g) {
        sc[g] += __shfl_xor(sc[g], kAttQueries, 64);
        sc[g] += __shfl_xor(sc[g], 2 * kAttQueries, 64);
      }
      float mx = m;
#pragma unroll
      for (int g = 0; g < kAttGroup; ++g) {
        sc[g] = jb + g < nk ? sc[g] * scale : -INFINITY;
        mx = fmaxf(mx, sc[g]);
      }
      const float corr = expf(m - mx);
      float pr[kAttGroup];
      float psum = 0.f;
#pragma unroll
      for (int g = 0; g < kAttGroup; ++g) {
        pr[g] = expf(sc[g] - mx);
        psum += pr[g];
      }
      l = l * corr + psum;
#pragma unroll
      for (int i = 0; i < DP; ++i) acc[i] *= corr;
#pragma unroll
      for (int g = 0; g < kAttGroup; ++g) {
        const int jj = jb + g < nk ? jb + g : 0;
#pragma unroll
        for (int i = 0; i < DP; i += 8) {
          float vv[8];
          ld8(vp + jj * RS + i, vv);
#pragma unroll
          for (int e = 0; e < 8; ++e) acc[i + e] += pr[g] * vv[e];
        }
      }
      m = mx;
    }
    __syncthreads();
  }
  if (t < LT) {
    const float inv = l > 0.f ? 1.0f / l : 0.f;
    uint16_t* dst = y + (static_cast<int64_t>(b) * LT + t) * H * D + static_cast<int64_t>(h) * D + part * DP;
#pragma unroll
    for (int i = 0; i < DP; i += 8) {
      float o[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) o[e] = acc[i + e] * inv;
      st8_bf16(dst + i, o);
    }
  }
}

// ---- mean of the two directions -> RMSNorm, and the 3-way gate ------------------
// One wave per row: mn = rms((mf + mb) / 2) w as the mean row norm computes it
// (fp32 out), then g_j = bf16(sum_c bf16(s_c) W[j, c] + bias_j) over
// s = cat(cn, mn, an), the gate linear under autocast.
template <int PER8>
__global__ __launch_bounds__(256) void merge_gate_kernel(const uint16_t* __restrict__ cn,
                                                         const uint16_t* __restrict__ mf,
                                                         const uint16_t* __restrict__ mb,
                                                         const uint16_t* __restrict__ an,
                                                         const float* __restrict__ w, const uint16_t* __restrict__ gw,
                                                         const uint16_t* __restrict__ gb, float* __restrict__ mn,
                                                         uint16_t* __restrict__ g, int64_t rows, int d, float eps) {
  const int lane = threadIdx.x & 63;
  const int64_t row = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;
  float v[PER8][8];
  // the row's cn and an pieces and the norm weights, requested with mf and mb
  // so that the gate's dot products do not wait for a second round trip
  float sc[PER8][8], sa[PER8][8], wv[PER8][8];
  float ss = 0.f;
#pragma unroll
  for (int i = 0; i < PER8; ++i) {
    const int i0 = 8 * (lane + 64 * i);
    if (i0 < d) {
      float bv[8];
      ld8(mf + row * d + i0, v[i]);
      ld8(mb + row * d + i0, bv);
      ld8(cn + row * d + i0, sc[i]);
      ld8(an + row * d + i0, sa[i]);
      ld8(w + i0, wv[i]);
#pragma unroll
      for (int e = 0; e < 8; ++e) v[i][e] = (v[i][e] + bv[e]) * 0.5f;
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) v[i][e] = 0.f;
    }
#pragma unroll
    for (int e = 0; e < 8; ++e) ss += v[i][e] * v[i][e];
  }
  ss = wave_sum(ss);
  const float r = rsqrtf(ss / static_cast<float>(d) + eps);
  float dot[3] = {0.f, 0.f, 0.f};
  const int64_t d3 = 3 * static_cast<int64_t>(d);
#pragma unroll
  for (int i = 0; i < PER8; ++i) {
    const int i0 = 8 * (lane + 64 * i);
    if (i0 < d) {
      float o[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) o[e] = v[i][e] * r * wv[i][e];
      st8_f32(mn + row * d + i0, o);
#pragma unroll
      for (int jj = 0; jj < 3; ++jj) {
        float w0[8], w1[8], w2[8];
        ld8(gw + jj * d3 + i0, w0);
        ld8(gw + jj * d3 + d + i0, w1);
        ld8(gw + jj * d3 + 2 * d + i0, w2);
#pragma unroll
        for (int e = 0; e < 8; ++e) dot[jj] += sc[i][e] * w0[e] + round_bf16(o[e]) * w1[e] + sa[i][e] * w2[e];
      }
    }
  }
#pragma unroll
  for (int jj = 0; jj < 3; ++jj) dot[jj] = wave_sum(dot[jj]);
  if (lane < 3) {
    const float val = lane == 0 ? dot[0] : (lane == 1 ? dot[1] : dot[2]);
    g[row * 3 + lane] = f32_to_bf16(val + bf16_to_f32(gb[lane]));
  }
}

// ---- gated concatenation -> masked depthwise conv -> residual add ---------------
// One wave per (512 channels of one third of the 3 d channels -- cn, mn or an --,
// TT time steps, batch row); each lane 8 channels. v = s * (2 sigmoid(g)) in fp32, the conv reads bf16(v); the output is
// bf16(v + bf16(conv)) with conv = 0 at t >= L.
template <int K, int TT, typename TS>
__device__ __forceinline__ void merge_conv_third(const TS* __restrict__ src, const uint16_t* __restrict__ g,
                                                 const uint16_t* __restrict__ w, const uint16_t* __restrict__ bias,
                                                 uint16_t* __restrict__ y, int third, int c8, int t0, int b, int T,
                                                 int L, int d) {
  if (c8 < d / 8) {
    const int c = 8 * c8, gc = third * d + c;
    float vb[TT + K - 1][8], vc[TT][8];
#pragma unroll
    for (int r = 0; r < TT + K - 1; ++r) {
      const int t = t0 - K / 2 + r;
      if (t >= 0 && t < T) {
        const int64_t row = static_cast<int64_t>(b) * T + t;
        float s[8];
        ld8(src + row * d + c, s);
        const float gate = mul_nc(2.f, sigmoid_acc(bf16_to_f32(g[row * 3 + third])));
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const float v = mul_nc(s[e], gate);
          vb[r][e] = round_bf16(v);
          if (r >= K / 2 && r < K / 2 + TT) vc[r - K / 2][e] = v;
        }
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          vb[r][e] = 0.f;
          if (r >= K / 2 && r < K / 2 + TT) vc[r - K / 2][e] = 0.f;
        }
      }
    }
    float wk[8][K], bb[8];
    load_taps<K>(w + static_cast<int64_t>(gc) * K, bias + gc, wk, bb);
#pragma unroll
    for (int i = 0; i < TT; ++i) {
      const int t = t0 + i;
      if (t < T) {
        float o[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          float acc = 0.f;
          if (t < L) {
#pragma unroll
            for (int q = 0; q < K; ++q) acc = add_nc(acc, mul_nc(vb[i + q][e], wk[e][q]));
            acc = round_bf16(add_nc(acc, bb[e]));
          }
          o[e] = vc[i][e] + acc;
        }
        st8_bf16(y + (static_cast<int64_t>(b) * T + t) * 3 * d + gc, o);
      }
    }
  }
}

template <int K, int TT>
__global__ __launch_bounds__(64) void merge_conv_kernel(const uint16_t* __restrict__ cn, const float* __restrict__ mn,
                                                        const uint16_t* __restrict__ an,
                                                        const uint16_t* __restrict__ g,
                                                        const uint16_t* __restrict__ w,
                                                        const uint16_t* __restrict__ bias,
                                                        const int64_t* __restrict__ lengths, uint16_t* __restrict__ y,
                                                        int T, int d, int chunks) {
  const int third = blockIdx.x / chunks, c8 = (blockIdx.x % chunks) * 64 + threadIdx.x;
  const int t0 = blockIdx.y * TT, b = blockIdx.z;
  const int L = clamp_len(lengths, b, T);
  if (third == 1) {
    merge_conv_third<K, TT, float>(mn, g, w, bias, y, third, c8, t0, b, T, L, d);
  } else {
    merge_conv_third<K, TT, uint16_t>(third == 0 ? cn : an, g, w, bias, y, third, c8, t0, b, T, L, d);
  }
}

bool a16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

int per8_of(int64_t d) {
  int per8 = 1;
  while (per8 * 512 < d) per8 <<= 1;
  return per8;
}

constexpr int kTT = 4;     // time steps per depthwise tile (merge_conv)
constexpr int kGluTW = 8;  // time steps per GLU + depthwise workgroup
constexpr int kGnsTW = 4;  // time steps per GLU + depthwise + norm + SiLU workgroup

}  // namespace
}  // namespace tf

namespace tf {
namespace {
int launch_block_pre(const float* x, const uint16_t* addend, const int64_t* lengths, const float* w, float eps,
                     float* xm, void* h, void* p, int64_t batch, int64_t time, int64_t d, hipStream_t s);
}  // namespace
}  // namespace tf

extern "C" int tf_block_pre(const float* x, const int64_t* lengths, const float* w, float eps, float* xm, void* h,
                            void* p, int64_t batch, int64_t time, int64_t d, void* stream) {
  return tf::launch_block_pre(x, nullptr, lengths, w, eps, xm, h, p, batch, time, d,
                              static_cast<hipStream_t>(stream));
}

extern "C" int tf_block_pre_add(const float* x, const void* addend, const int64_t* lengths, const float* w,
                                float eps, float* xm, void* h, void* p, int64_t batch, int64_t time, int64_t d,
                                void* stream) {
  if (!addend) return TF_ERR_NULL;
  if (!tf::a16(addend)) return TF_ERR_SHAPE;
  return tf::launch_block_pre(x, static_cast<const uint16_t*>(addend), lengths, w, eps, xm, h, p, batch, time, d,
                              static_cast<hipStream_t>(stream));
}

namespace tf {
namespace {
int launch_block_pre(const float* x, const uint16_t* addend, const int64_t* lengths, const float* w, float eps,
                     float* xm, void* h, void* p, int64_t batch, int64_t time, int64_t d, hipStream_t s) {
  if (!x || !lengths || !w || !xm || !h || !p) return TF_ERR_NULL;
  if (batch < 0 || time < 0 || d < 8 || d % 8 || d > 4096 || batch > 65535 || batch * time > 0x7fffffff)
    return TF_ERR_SHAPE;
  if (!a16(x) || !a16(w) || !a16(xm) || !a16(h) || !a16(p)) return TF_ERR_SHAPE;
  const int64_t lt = (time + 3) / 4;
  if (batch * lt == 0) return TF_OK;
  const dim3 grid(static_cast<uint32_t>(lt), static_cast<uint32_t>(batch));
  const size_t lds = 4 * static_cast<size_t>(d) * sizeof(float);
  const int per8 = per8_of(d);
#define TF_PRE(P)                                                                                                \
  case P:                                                                                                         \
    if (addend)                                                                                                   \
      hipLaunchKernelGGL((block_pre_kernel<P, true>), grid, dim3(256), lds, s, x, addend, lengths, w, xm,        \
                         static_cast<uint16_t*>(h), static_cast<uint16_t*>(p), static_cast<int>(time),            \
                         static_cast<int>(lt), static_cast<int>(d), eps);                                         \
    else                                                                                                          \
      hipLaunchKernelGGL((block_pre_kernel<P, false>), grid, dim3(256), lds, s, x, addend, lengths, w, xm,       \
                         static_cast<uint16_t*>(h), static_cast<uint16_t*>(p), static_cast<int>(time),            \
                         static_cast<int>(lt), static_cast<int>(d), eps);                                         \
    return launch_status();
  switch (per8) {
    TF_PRE(1) TF_PRE(2) TF_PRE(4) TF_PRE(8)
    default:
      return TF_ERR_SHAPE;
  }
#undef TF_PRE
}
}  // namespace
}  // namespace tf

extern "C" int tf_norm_silu(const void* x, const float* w, void* y, int64_t rows, int64_t d, float eps,
                            void* stream) {
  if (!x || !w || !y) return TF_ERR_NULL;
  if (rows < 0 || d < 8 || d % 8 || d > 4096) return TF_ERR_SHAPE;
  if (!tf::a16(x) || !tf::a16(w) || !tf::a16(y)) return TF_ERR_SHAPE;
  if (rows == 0) return TF_OK;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const dim3 grid(static_cast<uint32_t>((rows + 3) / 4));
#define TF_NS(P)                                                                                            \
  case P:                                                                                                    \
    hipLaunchKernelGGL(tf::norm_silu_kernel<P>, grid, dim3(256), 0, s, static_cast<const uint16_t*>(x), w,   \
                       static_cast<uint16_t*>(y), rows, static_cast<int>(d), eps);                           \
    return tf::launch_status();
  switch (tf::per8_of(d)) {
    TF_NS(1) TF_NS(2) TF_NS(4) TF_NS(8)
    default:
      return TF_ERR_SHAPE;
  }
#undef TF_NS
}

extern "C" int tf_glu_depthwise_norm_silu(const void* up, const void* w, const void* bias, const int64_t* lengths,
                                          const float* norm_w, float eps, void* y, int64_t batch, int64_t time,
                                          int64_t d, int64_t k, void* stream) {
  if (!up || !w || !bias || !lengths || !norm_w || !y) return TF_ERR_NULL;
  if (batch < 0 || time < 0 || d < 8 || d % 8 || d > 1024 || batch > 65535 || batch * time > 0x7fffffff ||
      (time + tf::kGnsTW - 1) / tf::kGnsTW > 65535)
    return TF_ERR_SHAPE;
  if (!tf::a16(up) || !tf::a16(y) || !tf::a16(w) || !tf::a16(bias) || !tf::a16(norm_w)) return TF_ERR_SHAPE;
  if (batch * time == 0) return TF_OK;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const dim3 grid(static_cast<uint32_t>((time + tf::kGnsTW - 1) / tf::kGnsTW), static_cast<uint32_t>(batch));
  const size_t lds = static_cast<size_t>(tf::kGnsTW + k - 1) * (d / 8) * 16;
#define TF_GNS(KV, P)                                                                                            \
  if (k == KV && (d <= 512 * P) && (P == 1 || d > 512 * (P / 2))) {                                              \
    hipLaunchKernelGGL((tf::glu_norm_silu_kernel<KV, tf::kGnsTW, P>), grid, dim3(256), lds, s,                 \
                       static_cast<const uint16_t*>(up), static_cast<const uint16_t*>(w),                        \
                       static_cast<const uint16_t*>(bias), lengths, norm_w, static_cast<uint16_t*>(y),          \
                       static_cast<int>(time), static_cast<int>(d), eps);                                        \
    return tf::launch_status();                                                                                  \
  }
  TF_GNS(3, 1) TF_GNS(3, 2) TF_GNS(7, 1) TF_GNS(7, 2)
#undef TF_GNS
  return TF_ERR_SHAPE;
}

extern "C" int tf_glu_depthwise(const void* up, const void* w, const void* bias, const int64_t* lengths, void* y,
                                int64_t batch, int64_t time, int64_t d, int64_t k, void* stream) {
  if (!up || !w || !bias || !lengths || !y) return TF_ERR_NULL;
  if (batch < 0 || time < 0 || d < 8 || d % 8 || batch > 65535 || batch * time > 0x7fffffff ||
      (time + tf::kGluTW - 1) / tf::kGluTW > 65535)
    return TF_ERR_SHAPE;
  if (!tf::a16(up) || !tf::a16(y) || !tf::a16(w) || !tf::a16(bias)) return TF_ERR_SHAPE;
  if (batch * time == 0) return TF_OK;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const dim3 grid(static_cast<uint32_t>((d / 8 + 63) / 64),
                  static_cast<uint32_t>((time + tf::kGluTW - 1) / tf::kGluTW), static_cast<uint32_t>(batch));
#define TF_GLU(KV)                                                                                               \
  if (k == KV) {                                                                                                  \
    hipLaunchKernelGGL((tf::glu_depthwise_kernel<KV, tf::kGluTW>), grid, dim3(256), 0, s,                        \
                       static_cast<const uint16_t*>(up), static_cast<const uint16_t*>(w),                        \
                       static_cast<const uint16_t*>(bias), lengths, static_cast<uint16_t*>(y),                   \
                       static_cast<int>(time), static_cast<int>(d));                                             \
    return tf::launch_status();                                                                                  \
  }
  TF_GLU(3) TF_GLU(7)
#undef TF_GLU
  return TF_ERR_SHAPE;
}

extern "C" int tf_pooled_attention(const void* qkv, const float* cos_t, const float* sin_t,
                                   const int64_t* low_lengths, void* y, int64_t batch, int64_t low_time,
                                   int64_t heads, int64_t head_dim, void* stream) {
  if (!qkv || !cos_t || !sin_t || !low_lengths || !y) return TF_ERR_NULL;
  if (batch < 0 || low_time < 0 || heads < 1 || heads > 65535 || batch > 65535 || batch * low_time > 0x7fffffff)
    return TF_ERR_SHAPE;
  // the tables are read 4 pairs (16 bytes) at a time
  if (!tf::a16(qkv) || !tf::a16(y) || !tf::a16(cos_t) || !tf::a16(sin_t)) return TF_ERR_SHAPE;
  if (batch * low_time == 0) return TF_OK;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const dim3 grid(static_cast<uint32_t>((low_time + tf::kAttQueries - 1) / tf::kAttQueries),
                  static_cast<uint32_t>(heads), static_cast<uint32_t>(batch));
  const float scale = 1.0f / sqrtf(static_cast<float>(head_dim));
#define TF_ATT(DV)                                                                                                \
  if (head_dim == DV) {                                                                                            \
    hipLaunchKernelGGL(tf::attention_kernel<DV>, grid, dim3(64), 0, s, static_cast<const uint16_t*>(qkv), cos_t,   \
                       sin_t, low_lengths, static_cast<uint16_t*>(y), static_cast<int>(low_time),                  \
                       static_cast<int>(heads), scale);                                                            \
    return tf::launch_status();                                                                                    \
  }
  TF_ATT(32) TF_ATT(64)
#undef TF_ATT
  return TF_ERR_SHAPE;
}

extern "C" int tf_merge_gate(const void* cn, const void* mf, const void* mb, const void* an, const float* norm_w,
                             float eps, const void* gate_w, const void* gate_b, float* mn, void* g, int64_t rows,
                             int64_t d, void* stream) {
  if (!cn || !mf || !mb || !an || !norm_w || !gate_w || !gate_b || !mn || !g) return TF_ERR_NULL;
  if (rows < 0 || d < 8 || d % 8 || d > 4096) return TF_ERR_SHAPE;
  for (const void* p : {cn, mf, mb, an, static_cast<const void*>(norm_w), gate_w, static_cast<const void*>(mn)})
    if (!tf::a16(p)) return TF_ERR_SHAPE;
  if (rows == 0) return TF_OK;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const dim3 grid(static_cast<uint32_t>((rows + 3) / 4));
#define TF_MG(P)                                                                                                  \
  case P:                                                                                                          \
    hipLaunchKernelGGL(tf::merge_gate_kernel<P>, grid, dim3(256), 0, s, static_cast<const uint16_t*>(cn),          \
                       static_cast<const uint16_t*>(mf), static_cast<const uint16_t*>(mb),                         \
                       static_cast<const uint16_t*>(an), norm_w, static_cast<const uint16_t*>(gate_w),             \
                       static_cast<const uint16_t*>(gate_b), mn, static_cast<uint16_t*>(g), rows,                  \
                       static_cast<int>(d), eps);                                                                  \
    return tf::launch_status();
  switch (tf::per8_of(d)) {
    TF_MG(1) TF_MG(2) TF_MG(4) TF_MG(8)
    default:
      return TF_ERR_SHAPE;
  }
#undef TF_MG
}

extern "C" int tf_merge_conv(const void* cn, const float* mn, const void* an, const void* g, const void* w,
                             const void* bias, const int64_t* lengths, void* y, int64_t batch, int64_t time,
                             int64_t d, int64_t k, void* stream) {
  if (!cn || !mn || !an || !g || !w || !bias || !lengths || !y) return TF_ERR_NULL;
  if (batch < 0 || time < 0 || d < 8 || d % 8 || batch > 65535 || batch * time > 0x7fffffff ||
      (time + tf::kTT - 1) / tf::kTT > 65535)
    return TF_ERR_SHAPE;
  for (const void* p : {cn, static_cast<const void*>(mn), an, static_cast<const void*>(y), w, bias})
    if (!tf::a16(p)) return TF_ERR_SHAPE;
  if (batch * time == 0) return TF_OK;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int chunks = static_cast<int>((d / 8 + 63) / 64);
  const dim3 grid(static_cast<uint32_t>(3 * chunks), static_cast<uint32_t>((time + tf::kTT - 1) / tf::kTT),
                  static_cast<uint32_t>(batch));
#define TF_MC(KV)                                                                                                 \
  if (k == KV) {                                                                                                   \
    hipLaunchKernelGGL((tf::merge_conv_kernel<KV, tf::kTT>), grid, dim3(64), 0, s,                                \
                       static_cast<const uint16_t*>(cn), mn, static_cast<const uint16_t*>(an),                    \
                       static_cast<const uint16_t*>(g), static_cast<const uint16_t*>(w),                          \
                       static_cast<const uint16_t*>(bias), lengths, static_cast<uint16_t*>(y),                    \
                       static_cast<int>(time), static_cast<int>(d), chunks);                                      \
    return tf::launch_status();                                                                                   \
  }
  TF_MC(3)
#undef TF_MC
  return TF_ERR_SHAPE;
}
