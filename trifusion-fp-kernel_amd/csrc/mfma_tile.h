// Matrix-core tile helpers and the kernel-side operand block shared by the
// gfx950 recurrence kernels (mamba_mfma.hip, mamba_pipe.hip).
//
// MFMA 32x32x16 register layout (lane l, c32 = l & 31, hh = l >> 5):
//   A[i][k]: lane i + 32*(k/8), element k%8
//   B[k][j]: lane j + 32*(k/8), element k%8
//   D[i][j]: lane j + 32*((i/4)%2), element (i/8)*4 + i%4
// Writing both operands as rows ("row forms"), mfma(X, Y) accumulates
// D[i][j] += sum_k X[i][k] Y[j][k]: the lane indexes Y's row j = c32, the 16
// D values index X's rows i = drow(e, hh). Contraction indices are permuted the
// same way on both sides, slot j of k-step s holding k = kidx(s, hh, j), which
// makes the D values of one product directly usable as the K slots of the next
// product's operand.
#pragma once

#include "mamba_internal.h"

namespace tf {

typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8;
typedef __attribute__((ext_vector_type(16))) float f32x16;
typedef __attribute__((ext_vector_type(4))) uint32_t u32x4;
typedef __attribute__((ext_vector_type(2))) uint32_t u32x2;

__device__ __forceinline__ f32x16 mfma(const u32x4& x, const u32x4& y, const f32x16& acc) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, x), __builtin_bit_cast(bf16x8, y),
                                                 acc, 0, 0, 0);
}

__device__ __forceinline__ f32x16 zero16() {
  f32x16 z;
#pragma unroll
  for (int i = 0; i < 16; ++i) z[i] = 0.f;
  return z;
}

// Row (within a 32-row tile) held in D element e by lane half hh.
__device__ __forceinline__ int drow(int e, int hh) { return 8 * (e >> 2) + 4 * hh + (e & 3); }

// Contraction index held in slot j of k-step s (16 indices per step) by lane half hh.
__device__ __forceinline__ int kidx(int s, int hh, int j) {
  return 32 * (s >> 1) + 16 * (s & 1) + 8 * (j >> 2) + 4 * hh + (j & 3);
}

typedef __attribute__((ext_vector_type(2))) __bf16 bf16x2;

// Two fp32 -> packed bf16 pair, round to nearest even (v_cvt_pk_bf16_f32).
__device__ __forceinline__ uint32_t pack2(float lo, float hi) {
  const bf16x2 v = {static_cast<__bf16>(lo), static_cast<__bf16>(hi)};
  return __builtin_bit_cast(uint32_t, v);
}
__device__ __forceinline__ float lo_f(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float hi_f(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }
__device__ __forceinline__ float slot_f(const u32x4& x, int j) {
  const uint32_t w = x[j >> 1];
  return (j & 1) ? hi_f(w) : lo_f(w);
}

// gfx9 DPP lane moves (no LDS traffic): row_shr:n shifts within 16-lane rows,
// row_bcast:15 / row_bcast:31 pass a row's last lane on to the following
// rows. Lanes without a source, or outside ROW_MASK, receive 0.
template <int CTRL, int ROW_MASK = 0xf>
__device__ __forceinline__ uint32_t dpp_u32(uint32_t x) {
  return static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(x), CTRL, ROW_MASK, 0xf, true));
}
template <int CTRL, int ROW_MASK = 0xf>
__device__ __forceinline__ float dpp_f32(float x) {
  return __builtin_bit_cast(float, dpp_u32<CTRL, ROW_MASK>(__builtin_bit_cast(uint32_t, x)));
}
constexpr int kDppRowShr = 0x110;  // + n: row_shr:n

// Sum over each aligned group of 8 lanes, in every lane of the group:
// quad_perm [1,0,3,2] and [2,3,0,1] sum the quads, row_half_mirror (lane i of
// an 8-lane half-row reads lane 7 - i) adds the other quad. Each step adds the
// same two values in every lane, so all 8 lanes hold the same bits.
__device__ __forceinline__ float group8_sum(float x) {
  x += dpp_f32<0xB1>(x);
  x += dpp_f32<0x4E>(x);
  x += dpp_f32<0x141>(x);
  return x;
}
constexpr int kDppRowBcast15 = 0x142;
constexpr int kDppRowBcast31 = 0x143;

// Inclusive prefix sum over the 64 lanes of the wave on DPP.
__device__ __forceinline__ float wave_scan_dpp(float x) {
  x += dpp_f32<kDppRowShr + 1>(x);
  x += dpp_f32<kDppRowShr + 2>(x);
  x += dpp_f32<kDppRowShr + 4>(x);
  x += dpp_f32<kDppRowShr + 8>(x);
  x += dpp_f32<kDppRowBcast15, 0xa>(x);  // rows 1, 3 += last lane of rows 0, 2
  x += dpp_f32<kDppRowBcast31, 0xc>(x);  // rows 2, 3 += lane 31
  return x;
}

// Inclusive prefix sum over the 64 lanes of the wave on DPP, wrapping uint32.
__device__ __forceinline__ uint32_t wave_scan_u32(uint32_t x) {
  x += dpp_u32<kDppRowShr + 1>(x);
  x += dpp_u32<kDppRowShr + 2>(x);
  x += dpp_u32<kDppRowShr + 4>(x);
  x += dpp_u32<kDppRowShr + 8>(x);
  x += dpp_u32<kDppRowBcast15, 0xa>(x);
  x += dpp_u32<kDppRowBcast31, 0xc>(x);
  return x;
}

// Inclusive prefix sum within each group of G consecutive lanes (G = 8 or 16),
// wrapping uint32 arithmetic, on DPP.
template <int G>
__device__ __forceinline__ uint32_t group_scan_dpp(uint32_t x, int lane) {
  static_assert(G == 8 || G == 16, "group size");
  const int j = lane & (G - 1);
  uint32_t o = dpp_u32<kDppRowShr + 1>(x);
  x += j >= 1 ? o : 0u;
  o = dpp_u32<kDppRowShr + 2>(x);
  x += j >= 2 ? o : 0u;
  o = dpp_u32<kDppRowShr + 4>(x);
  x += j >= 4 ? o : 0u;
  if constexpr (G == 16) x += dpp_u32<kDppRowShr + 8>(x);
  return x;
}

// Inclusive prefix sum over each 32-lane half of the wave.
template <typename F>
__device__ __forceinline__ F half_scan(F v, int c32) {
#pragma unroll
  for (int off = 1; off < 32; off <<= 1) {
    const F o = __shfl_up(v, off, 32);
    if (c32 >= off) v += o;
  }
  return v;
}

template <typename F>
__device__ __forceinline__ F half_last(F v) {
  return __shfl(v, 31, 32);
}

// Orders this wave's LDS accesses: earlier writes before later reads of other
// lanes' data, earlier reads before later writes to the same cells.
__device__ __forceinline__ void wave_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// Workgroup barrier ordering LDS accesses only. Waves exchange data through LDS
// alone, so global loads in flight (the next super-chunk's inputs) stay
// outstanding across it instead of being drained as a full fence would.
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

__device__ __forceinline__ float sigmoid_fast(float x) {
  return __builtin_amdgcn_rcpf(1.f + __builtin_amdgcn_exp2f(-x * kLog2e));
}

// Identity operand for a 32-wide tile: slot j of k-step parity sp is 1.0 where
// kidx(sp, hh, j) == c32.
__device__ __forceinline__ u32x4 identity_rows(int sp, int hh, int c32) {
  u32x4 r;
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int j = 2 * q;
    const uint32_t lo = (16 * sp + 8 * (j >> 2) + 4 * hh + (j & 3)) == c32 ? 0x3f80u : 0u;
    const uint32_t hi = (16 * sp + 8 * ((j + 1) >> 2) + 4 * hh + ((j + 1) & 3)) == c32 ? 0x3f80u : 0u;
    r[q] = lo | (hi << 16);
  }
  return r;
}

// Elements k0..k0+3 and k0+8..k0+11 of one bf16 row (two 8-byte loads).
__device__ __forceinline__ u32x4 load_row8(const uint16_t* row, int k0) {
  const u32x2 x = *reinterpret_cast<const u32x2*>(row + k0);
  const u32x2 y = *reinterpret_cast<const u32x2*>(row + k0 + 8);
  u32x4 r;
  r[0] = x[0];
  r[1] = x[1];
  r[2] = y[0];
  r[3] = y[1];
  return r;
}

__device__ __forceinline__ u32x4 as_u4(const float4& f) { return __builtin_bit_cast(u32x4, f); }
__device__ __forceinline__ float4 as_f4(const u32x4& u) { return __builtin_bit_cast(float4, u); }

// tanh for |x| < 0.625 by the odd polynomial of the Cephes single-precision
// tanhf (S. L. Moshier, Cephes Math Library), else 1 - 2/(exp(2|x|) + 1) with the
// hardware exp2/rcp, evaluated only when some lane of the wave needs it. (The
// exp form alone is biased by ~1e-7 near 0, which the phase cumsum carries
// into a visible error after a few thousand steps.)
__device__ __forceinline__ float tanh_fast(float x) {
  const float ax = fabsf(x);
  const float z = x * x;
  float r = ((((-5.70498872745e-3f * z + 2.06390887954e-2f) * z - 5.37397155531e-2f) * z + 1.33314422036e-1f) * z -
             3.33332819422e-1f) * z * ax + ax;
  if (__any(ax >= 0.625f)) {
    const float e = __builtin_amdgcn_exp2f(2.f * kLog2e * fminf(ax, 40.f));
    const float big = 1.f - 2.f * __builtin_amdgcn_rcpf(e + 1.f);
    r = ax < 0.625f ? r : big;
  }
  return copysignf(r, x);
}

// Kernel-side operand block: per-tensor element strides as int32 (the host
// checks every offset fits) so addressing stays in few registers.
struct MfmaParams {
  const uint16_t* q;
  const uint16_t* k;
  const uint16_t* v;
  const uint16_t* z;
  const void* adt;  // adt and dt, or the raw a and ddt columns (ctl_raw)
  const void* dt;
  const void* trap;
  const void* angles;
  const float* qb;
  const float* kb;
  const float* d;
  void* out;
  const int64_t* lengths;
  int q_sb, q_st, q_sh;
  int k_sb, k_st, k_sh;
  int v_sb, v_st, v_sh;
  int z_sb, z_st, z_sh;
  int o_sb, o_st, o_sh;
  int g_sb, g_st, g_sh, g_sr;
  int a_sb, a_sh, a_st;
  int d_sb, d_sh, d_st;
  int r_sb, r_sh, r_st;
  int T, H, group, R, xcd_per;
  // State dim of q/k (16 runs the N = 32 kernel on zero-padded channels)
  int n_real;
  int out_f32, trap_bf16, angles_dtype;
  // Raw controls: adt/dt hold the in-projection's a/ddt columns (bf16 when
  // ctl_bf16), turned into the step and decay in the prologue.
  int ctl_raw, ctl_bf16;
  float a_floor;
  const float* dt_bias;
  // Reverse: step t < L of a unit reads and writes row L-1-t. The host negates
  // every time stride; the kernel moves each unit's bases to row L-1.
  int rev;
  // Chunk-parallel form: the time axis of each of the `units` (batch, head)
  // units is cut into G segments of SC chunks, one workgroup per (segment,
  // unit). Scratch: per (unit, chunk) the phase sum per pair ([NC][64] fp64,
  // from the phase pre-pass); per record rec = unit * G + segment the state
  // ([kF4] float4 in kernel layout: the contribution from zero written by the
  // summary pass, replaced by the state entering the segment by the segment
  // scan) and the log2 decay. G = 1: no scratch.
  float4* seg_state;
  double* chunk_phase;
  float* seg_decay;
  int units, G, SC, NC;
  // Pipelined kernel's chunk-parallel form: per (unit, segment) and rotary
  // pair the wrapping sum of its fixed-point phase increments ([G][32]),
  // written by the summary pass beside the segment's record.
  uint32_t* phase_fx;
  // Pipelined kernel, unsegmented varlen walks: deal batch rows longest first.
  int lpt;
  // Fused B/C RMSNorm: q and k are raw rows, each normalised as it is loaded,
  // round(x * rsqrt(mean(x^2) + norm_eps) * w), with w = qn_w / kn_w ([N]).
  int qk_norm;
  float norm_eps;
  const float* qn_w;
  const float* kn_w;
};

// One step of the segment scan, S 2^dec + summary, as explicit fused
// multiply-adds (the same rounding wherever it is inlined).
__device__ __forceinline__ float4 state_step(const float4& s, float m, const float4& d) {
  return make_float4(__builtin_fmaf(s.x, m, d.x), __builtin_fmaf(s.y, m, d.y), __builtin_fmaf(s.z, m, d.z),
                     __builtin_fmaf(s.w, m, d.w));
}

// The segment scan of one unit's records, float4 f of each: record g (the
// state segment g leaves from zero state; log2 decay dec[g]) is replaced by
// the state entering segment g: S_0 = 0, S_{g+1} = S_g 2^dec[g] + record g.
// Loads run ahead of the serial chain in batches of 16 records.
__device__ __forceinline__ void scan_unit_records(float4* st, const float* dec, int kf4, int G, int f) {
  constexpr int kBatch = 16;
  float4 run = make_float4(0.f, 0.f, 0.f, 0.f);
  for (int g0 = 0; g0 < G; g0 += kBatch) {
    float4 d[kBatch];
    float m[kBatch];
#pragma unroll
    for (int j = 0; j < kBatch; ++j) {
      if (g0 + j < G) {
        d[j] = st[static_cast<size_t>(g0 + j) * kf4 + f];
        m[j] = fast_exp2(dec[g0 + j]);
      }
    }
#pragma unroll
    for (int j = 0; j < kBatch; ++j) {
      if (g0 + j < G) {
        st[static_cast<size_t>(g0 + j) * kf4 + f] = run;
        run = state_step(run, m[j], d[j]);
      }
    }
  }
}

// Element i of a control tensor (fp32, or bf16 for raw controls).
__device__ __forceinline__ float ctl_value(const void* base, int bf16, int i) {
  return bf16 ? to_f32(static_cast<const bf16_t*>(base)[i]) : static_cast<const float*>(base)[i];
}

// Scores^T[u][t] = kr_u . qr_t of one 32x32 tile times the decay
// 2^min(cs_t - cs_u, 0), strictly causal on a diagonal tile (an off-diagonal
// tile must have every t > u), rounded to bf16 as the Y operand of the
// score . v product (rows t, K = u; mamba_fused.py:144-146). The clamp caps a
// weight at 1 where the signed decay is positive somewhere between u and t.
__device__ __forceinline__ void score_tile(const f32x16& acc, float cst, const float* csu_base, bool diag, int c32,
                                           int hh, u32x4 (&out)[2]) {
#pragma unroll
  for (int g = 0; g < 4; ++g) {
    const float4 csu = *reinterpret_cast<const float4*>(csu_base + 8 * g + 4 * hh);
    const float cu[4] = {csu.x, csu.y, csu.z, csu.w};
    float vals[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int e = 4 * g + q;
      // masked elements (t <= u) may overflow here; the select below drops them
      const float x = acc[e] * fast_exp2(fminf(cst - cu[q], 0.f));
      vals[q] = (!diag || c32 > drow(e, hh)) ? x : 0.f;
    }
    out[g >> 1][2 * (g & 1)] = pack2(vals[0], vals[1]);
    out[g >> 1][2 * (g & 1) + 1] = pack2(vals[2], vals[3]);
  }
}

bool aligned(const void* p, int bytes);
// Rows of 4-dim tensor `p` (strides `st`, innermost unit stride) can be read in
// `vec_bytes` pieces.
bool rows_vectorisable(const void* p, const int64_t* st, int elem_bytes, int vec_bytes);
// Every element offset of the operands fits the kernels' int32 addressing.
bool offsets_fit(const tf_mamba_args& a);
// Kernel operand block of `a`: int32 strides, time strides negated for reverse.
MfmaParams make_params(const tf_mamba_args& a);

}  // namespace tf
