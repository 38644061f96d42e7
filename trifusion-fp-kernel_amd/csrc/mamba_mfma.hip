// Chunked-scan fused Mamba-3 SISO recurrence on gfx950 bf16 MFMA.
//
// Same arithmetic and bf16 rounding points as the reference kernel
// (src/trifusion_l4/mamba_fused.py:72-152), reorganised for CDNA4:
//
//   * One workgroup per (batch, head) unit, W waves. The sequence is walked in
//     "super-chunks" of W chunks of 64 steps; wave w owns chunk g*W + w, so the
//     chunk-local work of W chunks (loads, controls, phase scan, rotary, the
//     intra-chunk C.B^T score, score.v and the chunk's state contribution dS)
//     runs on all SIMDs at once instead of one chunk after another.
//   * The only serial dependency, the fp32 state S <- S*2^tot + dS, is a
//     prefix scan over the W chunk contributions held in LDS: every thread of
//     the workgroup owns a slice of the P x N state and walks the W slots,
//     replacing each dS_c with the exclusive state S_c entering chunk c. Wave w
//     then adds 2^cs * qr . bf16(S_c)^T to its outputs.
//   * All contractions run on v_mfma_f32_32x32x16_bf16. Operands come straight
//     from global memory in MFMA register layout (8-byte loads of four
//     consecutive elements); the two transposes the contractions over time need
//     (v^T and kr^T) are products with an identity tile on the matrix core,
//     which is exact for bf16 values.
//   * The rotary phase is accumulated in fp64 and rounded to fp32 once.
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
#include "mamba_internal.h"

namespace tf {
namespace {

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

// Orders this wave's LDS writes before its later LDS reads of other lanes' data.
__device__ __forceinline__ void wave_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
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

// tanh for |x| < 0.625 by the odd polynomial of the Cephes single-precision
// tanhf (S. L. Moshier, Cephes Math Library), else 1 - 2/(exp(2|x|) + 1) with
// the hardware exp2/rcp; a few ulp, no branches.
__device__ __forceinline__ float tanh_fast(float x) {
  const float ax = fabsf(x);
  const float z = x * x;
  const float poly =
      ((((-5.70498872745e-3f * z + 2.06390887954e-2f) * z - 5.37397155531e-2f) * z + 1.33314422036e-1f) * z -
       3.33332819422e-1f) * z * ax + ax;
  const float e = __builtin_amdgcn_exp2f(2.f * kLog2e * fminf(ax, 40.f));
  const float big = 1.f - 2.f * __builtin_amdgcn_rcpf(e + 1.f);
  return copysignf(ax < 0.625f ? poly : big, x);
}

// Raw angles of rows [seg*rp, seg*rp + rp) of pair pp, all loads issued before
// use (0 past L or for pp >= R).
template <int RPMAX, typename E>
__device__ __forceinline__ void load_angles(const E* p, int64_t st, int t0, int L, int seg, int rp, bool on,
                                            float (&th)[RPMAX]) {
#pragma unroll
  for (int r = 0; r < RPMAX; ++r) {
    const int t = t0 + seg * rp + r;
    th[r] = (on && r < rp && t < L) ? to_f32(p[t * st]) : 0.f;
  }
}

// Pass 1: increments pi*tanh(theta)*dt of the lane's rows -> phs[row*rs + pp]
// (fp32); returns their fp64 sum.
template <int RPMAX>
__device__ __forceinline__ double phase_pass1(const tf_mamba_args& a, int64_t go, int t0, int L, int pp, int seg,
                                              int rp, int R, int rs, const float* dtw, float* phs) {
  float th[RPMAX];
  const bool on = pp < R;
  const int64_t st = a.angles_stride[1];
  const int64_t off = go + pp * a.angles_stride[3];
  if (a.angles_dtype == TF_FLOAT32)
    load_angles<RPMAX>(static_cast<const float*>(a.angles) + off, st, t0, L, seg, rp, on, th);
  else if (a.angles_dtype == TF_BFLOAT16)
    load_angles<RPMAX>(static_cast<const bf16_t*>(a.angles) + off, st, t0, L, seg, rp, on, th);
  else
    load_angles<RPMAX>(static_cast<const f16_t*>(a.angles) + off, st, t0, L, seg, rp, on, th);
  double sum = 0.0;
#pragma unroll
  for (int r = 0; r < RPMAX; ++r) {
    if (r < rp) {
      const int row = seg * rp + r;
      const float om = tanh_fast(th[r]) * kPi * dtw[row];
      if (on) phs[row * rs + pp] = om;
      sum += static_cast<double>(om);
    }
  }
  return sum;
}

// Pass 2: fp64 cumsum of the increments from `start`, replacing each with its
// phase reduced to [0, 2pi) as fp32.
template <int RPMAX>
__device__ __forceinline__ void phase_pass2(int pp, int seg, int rp, int R, int rs, double start, float* phs) {
  if (pp >= R) return;
  float om[RPMAX];
#pragma unroll
  for (int r = 0; r < RPMAX; ++r) om[r] = r < rp ? phs[(seg * rp + r) * rs + pp] : 0.f;
  double cum = start;
#pragma unroll
  for (int r = 0; r < RPMAX; ++r) {
    if (r < rp) {
      cum += static_cast<double>(om[r]);
      phs[(seg * rp + r) * rs + pp] = static_cast<float>(cum - kTwoPiD * floor(cum * (1.0 / kTwoPiD)));
    }
  }
}

template <int NT, int PT, int W>
struct Smem {
  static constexpr int kTiles = NT * PT;
  static constexpr int kF4 = kTiles * 4 * 64;  // float4 per chunk state
  float4 state[W][kF4];  // [slot][tile][g][lane] = D elements 4g..4g+3 of tile (nt, pt)
  float cs[W][kChunk];   // cumulative log2 decay of each wave's chunk
  float dt[W][kChunk];   // dt of each wave's chunk rows
  float tot[W];
  double wsum[W][64];    // phase increment of each chunk per rotary pair
  double carry[64];      // phase carry entering the super-chunk
  float qb[32 * NT];
  float kb[32 * NT];
};

template <int NT, int PT, int W>
__global__ __launch_bounds__(W * 64) void mamba_mfma_kernel(const tf_mamba_args a, const int xcd_per) {
  constexpr int N = 32 * NT;
  constexpr int KS = N / 16;  // k-steps over the state dim
  constexpr int PS = PT * 2;  // k-steps over the head dim
  using Sm = Smem<NT, PT, W>;
  constexpr int kF4 = Sm::kF4;
  constexpr int SPT = (kF4 + W * 64 - 1) / (W * 64);  // float4 of the running state per thread
  __shared__ Sm sh;

  const int lane = threadIdx.x & 63;
  const int w = threadIdx.x >> 6;
  const int c32 = lane & 31;
  const int hh = lane >> 5;
  const int H = static_cast<int>(a.heads);
  const int unit = xcd_per > 0 ? (blockIdx.x & 7) * xcd_per + (blockIdx.x >> 3) : static_cast<int>(blockIdx.x);
  const int b = unit / H;
  const int h = unit - b * H;
  const int qh = h / (H / static_cast<int>(a.qk_heads));
  const int T = static_cast<int>(a.time);
  const int L = valid_length(a, b);
  const int R = static_cast<int>(a.rotary);
  const int nvalid = (L + kChunk - 1) / kChunk;
  // phase lanes: pair pp = lane % rp over rows [seg*rp, seg*rp + rp), rp = pow2 >= R
  int rp = 1;
  while (rp < R) rp <<= 1;
  const int pp = lane & (rp - 1);
  const int seg = lane / rp;
  const int rs = (R + 1) & ~1;  // row stride of the staged phases (even: 8-byte pair reads)

  const uint16_t* qbase = static_cast<const uint16_t*>(a.q) + b * a.q_stride[0] + qh * a.q_stride[2];
  const uint16_t* kbase = static_cast<const uint16_t*>(a.k) + b * a.k_stride[0] + qh * a.k_stride[2];
  const uint16_t* vbase = static_cast<const uint16_t*>(a.v) + b * a.v_stride[0] + h * a.v_stride[2];
  const uint16_t* zbase = static_cast<const uint16_t*>(a.z) + b * a.z_stride[0] + h * a.z_stride[2];
  const int64_t go = b * a.angles_stride[0] + h * a.angles_stride[2];
  const int64_t ao = b * a.adt_stride[0] + h * a.adt_stride[1];
  const int64_t dto = b * a.dt_stride[0] + h * a.dt_stride[1];
  const int64_t tro = b * a.trap_stride[0] + h * a.trap_stride[1];
  const int64_t oo = b * a.out_stride[0] + h * a.out_stride[2];
  const float skip = a.d[h];

  for (int i = threadIdx.x; i < 64; i += W * 64) sh.carry[i] = 0.0;
  for (int i = threadIdx.x; i < N; i += W * 64) {
    sh.qb[i] = a.qb[h * N + i];
    sh.kb[i] = a.kb[h * N + i];
  }
  float4 run[SPT];
#pragma unroll
  for (int r = 0; r < SPT; ++r) run[r] = make_float4(0.f, 0.f, 0.f, 0.f);
  const u32x4 ident0 = identity_rows(0, hh, c32);
  const u32x4 ident1 = identity_rows(1, hh, c32);
  __syncthreads();

  for (int g0 = 0; g0 < nvalid; g0 += W) {
    const bool active = g0 + w < nvalid;  // wave-uniform; idle waves recompute the last chunk
    const int c = active ? g0 + w : nvalid - 1;
    const int nact = min(W, nvalid - g0);
    const int t0 = c * kChunk;
    float* phs = reinterpret_cast<float*>(&sh.state[w][0]);  // [row][pair] staging, free until dS

    // ---------------- phase A: chunk-local work ----------------
    float csr[2], gam[2], scl[2], dtr[2];
    bool ok[2];
    u32x4 qrow[2][KS], krow[2][KS], vrow[2][PS];
    {
      float da[2];
#pragma unroll
      for (int rt = 0; rt < 2; ++rt) {
        const int t = t0 + 32 * rt + c32;
        const bool valid = t < L;
        const bool next = t + 1 < T;
        ok[rt] = valid;
        const float* dtp = static_cast<const float*>(a.dt) + dto;
        const float dt = valid ? dtp[t * a.dt_stride[2]] : 0.f;
        const float dn = next ? dtp[(t + 1) * a.dt_stride[2]] : 0.f;
        const float tr = sigmoid_fast(valid ? load_f32(a.trap, a.trap_dtype, tro + t * a.trap_stride[2]) : 0.f);
        const float tn =
            sigmoid_fast(next ? load_f32(a.trap, a.trap_dtype, tro + (t + 1) * a.trap_stride[2]) : 0.f);
        gam[rt] = dt * tr;
        scl[rt] = dn * (1.f - tn) + gam[rt];
        dtr[rt] = dt;
        da[rt] = valid ? static_cast<const float*>(a.adt)[ao + t * a.adt_stride[2]] * kLog2e : 0.f;
      }
#pragma unroll
      for (int rt = 0; rt < 2; ++rt) {
        const int64_t t = ok[rt] ? t0 + 32 * rt + c32 : 0;  // invalid rows read row 0 and are zeroed
        const uint16_t* q_row = qbase + t * a.q_stride[1];
        const uint16_t* k_row = kbase + t * a.k_stride[1];
        const uint16_t* v_row = vbase + t * a.v_stride[1];
#pragma unroll
        for (int s = 0; s < KS; ++s) {
          qrow[rt][s] = load_row8(q_row, kidx(s, hh, 0));
          krow[rt][s] = load_row8(k_row, kidx(s, hh, 0));
        }
#pragma unroll
        for (int s = 0; s < PS; ++s) {
          const u32x4 x = load_row8(v_row, kidx(s, hh, 0));
          vrow[rt][s] = ok[rt] ? x : u32x4{0u, 0u, 0u, 0u};
        }
      }
      // cumulative log2 decay over the chunk; both lane halves hold all 64 rows
      const float cs0 = half_scan(da[0], c32);
      const float cs1 = half_scan(da[1], c32) + half_last(cs0);
      csr[0] = cs0;
      csr[1] = cs1;
      if (hh == 0) {
        sh.cs[w][c32] = cs0;
        sh.cs[w][32 + c32] = cs1;
        sh.dt[w][c32] = dtr[0];
        sh.dt[w][32 + c32] = dtr[1];
      }
      const float chunk_tot = half_last(cs1);  // shuffle with every lane active
      if (lane == 0) sh.tot[w] = chunk_tot;
      wave_sync();
    }
    // rotary phase increments pi*tanh(theta)*dt: lane (pair pp, segment seg) sums
    // rows [seg*rp, seg*rp + rp) in fp64; the chunk sum per pair goes to LDS
    const double seg_part = phase_pass1<16 * NT>(a, go, t0, L, pp, seg, rp, R, rs, sh.dt[w], phs);
    {
      double sum = seg_part;
      for (int off = rp; off < 64; off <<= 1) sum += __shfl_xor(sum, off);
      if (seg == 0 && pp < R) sh.wsum[w][pp] = sum;
    }
    __syncthreads();  // barrier 1: chunk phase sums visible

    f32x16 yacc[PT][2];  // y^T tiles (pt, tt): lane = t, elements = p
    {
      // skip-term partial sums gamma * (q + qb).(k + kb) over this lane's n, from
      // the unrotated biased values inside the rotation loop (mamba_fused.py:124)
      float part[2] = {0.f, 0.f};
      // rotary phase: carry of the preceding chunks + exclusive segment prefix +
      // serial fp64 cumsum, reduced mod 2pi and staged as fp32 [row][pair] in this
      // wave's state slot (free until dS is written)
      {
        double carry = 0.0;
        if (pp < R) {
          carry = sh.carry[pp];
          for (int j = 0; j < w; ++j) carry += sh.wsum[j][pp];
        }
        double pre = seg_part;  // inclusive scan over segments of the same pair
        for (int off = rp; off < 64; off <<= 1) {
          const double o = __shfl_up(pre, off);
          if (seg * rp >= off) pre += o;
        }
        phase_pass2<16 * NT>(pp, seg, rp, R, rs, carry + pre - seg_part, phs);
      }
      wave_sync();
#pragma unroll
      for (int s = 0; s < KS; ++s) {
        float co[2][4], si[2][4];
#pragma unroll
        for (int rt = 0; rt < 2; ++rt)
#pragma unroll
          for (int u = 0; u < 4; ++u) {
            co[rt][u] = 1.f;
            si[rt][u] = 0.f;
          }
        if (8 * s < R) {  // wave-uniform: pairs >= R are not rotated
#pragma unroll
          for (int rt = 0; rt < 2; ++rt) {
            const float* row = phs + (32 * rt + c32) * rs;
#pragma unroll
            for (int half = 0; half < 2; ++half) {
              const int pr = 8 * s + 2 * hh + 4 * half;
              const float2 ph = *reinterpret_cast<const float2*>(row + pr);
#pragma unroll
              for (int u = 0; u < 2; ++u) {
                const float x = u ? ph.y : ph.x;
                if (pr + u < R) {
                  co[rt][2 * half + u] = __builtin_amdgcn_cosf(x * kInvTwoPi);
                  si[rt][2 * half + u] = __builtin_amdgcn_sinf(x * kInvTwoPi);
                }
              }
            }
          }
        }
#pragma unroll
        for (int q4 = 0; q4 < 4; ++q4) {
          const int j = 2 * q4;
          const float qb0 = sh.qb[kidx(s, hh, j)], qb1 = sh.qb[kidx(s, hh, j + 1)];
          const float kb0 = sh.kb[kidx(s, hh, j)], kb1 = sh.kb[kidx(s, hh, j + 1)];
#pragma unroll
          for (int rt = 0; rt < 2; ++rt) {
            const uint32_t qw = qrow[rt][s][q4];
            const uint32_t kw = krow[rt][s][q4];
            const float q0 = lo_f(qw) + qb0, q1 = hi_f(qw) + qb1;
            const float k0 = lo_f(kw) + kb0, k1 = hi_f(kw) + kb1;
            part[rt] += q0 * k0 + q1 * k1;
            const float c = co[rt][q4], sn = si[rt][q4], sc = scl[rt];
            const uint32_t qn = pack2(q0 * c - q1 * sn, q0 * sn + q1 * c);
            const uint32_t kn = pack2((k0 * c - k1 * sn) * sc, (k0 * sn + k1 * c) * sc);
            qrow[rt][s][q4] = ok[rt] ? qn : 0u;
            krow[rt][s][q4] = ok[rt] ? kn : 0u;
          }
        }
      }

      float delta[2];
#pragma unroll
      for (int rt = 0; rt < 2; ++rt) delta[rt] = gam[rt] * (part[rt] + __shfl_xor(part[rt], 32));

      // scores^T[u][t] = kr_u . qr_t on tiles (ut, tt) with ut <= tt, then the
      // strictly causal decay mask, rounded to bf16 (mamba_fused.py:144-146)
      u32x4 scy[2][4];  // Y rows t, K = u
      {
        f32x16 sacc[3] = {zero16(), zero16(), zero16()};
#pragma unroll
        for (int s = 0; s < KS; ++s) {
          sacc[0] = mfma(krow[0][s], qrow[0][s], sacc[0]);
          sacc[1] = mfma(krow[0][s], qrow[1][s], sacc[1]);
          sacc[2] = mfma(krow[1][s], qrow[1][s], sacc[2]);
        }
#pragma unroll
        for (int tile = 0; tile < 3; ++tile) {
          const int ut = tile == 2 ? 1 : 0;
          const int tt = tile == 0 ? 0 : 1;
          const int tl = 32 * tt + c32;
          const float cst = csr[tt];
#pragma unroll
          for (int g = 0; g < 4; ++g) {
            const float4 csu = *reinterpret_cast<const float4*>(&sh.cs[w][32 * ut + 8 * g + 4 * hh]);
            const float cu[4] = {csu.x, csu.y, csu.z, csu.w};
            float vals[4];
#pragma unroll
            for (int q = 0; q < 4; ++q) {
              const int e = 4 * g + q;
              const int ul = 32 * ut + drow(e, hh);
              vals[q] = tl > ul ? sacc[tile][e] * fast_exp2(fminf(cst - cu[q], 0.f)) : 0.f;
            }
            scy[tt][2 * ut + (g >> 1)][2 * (g & 1)] = pack2(vals[0], vals[1]);
            scy[tt][2 * ut + (g >> 1)][2 * (g & 1) + 1] = pack2(vals[2], vals[3]);
          }
        }
      }

      // kr^T via the identity tile: D[u][n] = kr[u][n] -> X rows n, K = u
      u32x4 ktx[NT][4];
#pragma unroll
      for (int nt = 0; nt < NT; ++nt)
#pragma unroll
        for (int ut = 0; ut < 2; ++ut) {
          f32x16 d = mfma(krow[ut][2 * nt], ident0, zero16());
          d = mfma(krow[ut][2 * nt + 1], ident1, d);
#pragma unroll
          for (int sp = 0; sp < 2; ++sp)
#pragma unroll
            for (int q = 0; q < 4; ++q) ktx[nt][2 * ut + sp][q] = pack2(d[8 * sp + 2 * q], d[8 * sp + 2 * q + 1]);
        }

      // v^T via the identity tile: D[u][p] = v[u][p] -> X rows p, K = u; and the
      // decay-scaled copy rounded to bf16 (mamba_fused.py:151) -> Y rows p, K = u
      const float tot = sh.tot[w];
      u32x4 vtx[PT][4], vsy[PT][4];
#pragma unroll
      for (int ut = 0; ut < 2; ++ut) {
        float sc16[16];
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const float4 csu = *reinterpret_cast<const float4*>(&sh.cs[w][32 * ut + 8 * g + 4 * hh]);
          sc16[4 * g] = fast_exp2(tot - csu.x);
          sc16[4 * g + 1] = fast_exp2(tot - csu.y);
          sc16[4 * g + 2] = fast_exp2(tot - csu.z);
          sc16[4 * g + 3] = fast_exp2(tot - csu.w);
        }
#pragma unroll
        for (int pt = 0; pt < PT; ++pt) {
          f32x16 d = mfma(vrow[ut][2 * pt], ident0, zero16());
          d = mfma(vrow[ut][2 * pt + 1], ident1, d);
#pragma unroll
          for (int sp = 0; sp < 2; ++sp)
#pragma unroll
            for (int q = 0; q < 4; ++q) {
              const int e = 8 * sp + 2 * q;
              vtx[pt][2 * ut + sp][q] = pack2(d[e], d[e + 1]);
              vsy[pt][2 * ut + sp][q] = pack2(d[e] * sc16[e], d[e + 1] * sc16[e + 1]);
            }
        }
      }

      // y_intra^T[p][t] = (D + delta_t) v[t][p] + sum_u v^T[p][u] score[t][u]
#pragma unroll
      for (int pt = 0; pt < PT; ++pt) {
#pragma unroll
        for (int tt = 0; tt < 2; ++tt) {
          const float coef = skip + delta[tt];
#pragma unroll
          for (int e = 0; e < 16; ++e) yacc[pt][tt][e] = coef * slot_f(vrow[tt][2 * pt + (e >> 3)], e & 7);
        }
        yacc[pt][0] = mfma(vtx[pt][0], scy[0][0], yacc[pt][0]);
        yacc[pt][0] = mfma(vtx[pt][1], scy[0][1], yacc[pt][0]);
#pragma unroll
        for (int k = 0; k < 4; ++k) yacc[pt][1] = mfma(vtx[pt][k], scy[1][k], yacc[pt][1]);
      }

      // dS^T[n][p] = sum_u kr^T[n][u] vs[p][u] -> LDS slot w (lane = p, elements = n)
#pragma unroll
      for (int nt = 0; nt < NT; ++nt)
#pragma unroll
        for (int pt = 0; pt < PT; ++pt) {
          f32x16 d = zero16();
#pragma unroll
          for (int k = 0; k < 4; ++k) d = mfma(ktx[nt][k], vsy[pt][k], d);
          float4* dst = &sh.state[w][(nt * PT + pt) * 256];
#pragma unroll
          for (int g = 0; g < 4; ++g)
            dst[g * 64 + lane] = make_float4(d[4 * g], d[4 * g + 1], d[4 * g + 2], d[4 * g + 3]);
        }
    }
    __syncthreads();  // barrier 2: every dS in LDS

    // gate operand, loaded while the state scan runs
    u32x4 zrow[2][PS];
    {
#pragma unroll
      for (int rt = 0; rt < 2; ++rt) {
        const int64_t t = ok[rt] ? t0 + 32 * rt + c32 : 0;
        const uint16_t* z_row = zbase + t * a.z_stride[1];
#pragma unroll
        for (int s = 0; s < PS; ++s) zrow[rt][s] = load_row8(z_row, kidx(s, hh, 0));
      }
    }

    // ---------------- phase B: state scan over the W chunks ----------------
    {
      float dec[W];
#pragma unroll
      for (int j = 0; j < W; ++j) dec[j] = j < nact ? fast_exp2(sh.tot[j]) : 1.f;
#pragma unroll
      for (int r = 0; r < SPT; ++r) {
        const int f = threadIdx.x + r * W * 64;
        if (f >= kF4) break;
        float4 s = run[r];
#pragma unroll
        for (int j = 0; j < W; ++j) {
          if (j < nact) {
            const float4 d = sh.state[j][f];
            sh.state[j][f] = s;
            s = make_float4(s.x * dec[j] + d.x, s.y * dec[j] + d.y, s.z * dec[j] + d.z, s.w * dec[j] + d.w);
          }
        }
        run[r] = s;
      }
      if (threadIdx.x < R) {
        double cr = sh.carry[threadIdx.x];
        for (int j = 0; j < nact; ++j) cr += sh.wsum[j][threadIdx.x];
        sh.carry[threadIdx.x] = cr - kTwoPiD * floor(cr * (1.0 / kTwoPiD));
      }
    }
    __syncthreads();  // barrier 3: exclusive states in LDS

    // ---------------- phase C: inter-chunk term, gate, store ----------------
    {
#pragma unroll
      for (int pt = 0; pt < PT; ++pt) {
        f32x16 yi[2] = {zero16(), zero16()};
#pragma unroll
        for (int s = 0; s < KS; ++s) {
          // X rows p, K = n: D elements 8*(s&1) .. +7 of tile (s>>1, pt)
          const float4* src = &sh.state[w][((s >> 1) * PT + pt) * 256];
          const float4 lo = src[(2 * (s & 1)) * 64 + lane];
          const float4 hi = src[(2 * (s & 1) + 1) * 64 + lane];
          u32x4 sx;
          sx[0] = pack2(lo.x, lo.y);
          sx[1] = pack2(lo.z, lo.w);
          sx[2] = pack2(hi.x, hi.y);
          sx[3] = pack2(hi.z, hi.w);
          yi[0] = mfma(sx, qrow[0][s], yi[0]);
          yi[1] = mfma(sx, qrow[1][s], yi[1]);
        }
#pragma unroll
        for (int tt = 0; tt < 2; ++tt) {
          const int t = t0 + 32 * tt + c32;
          if (active && t < T) {
            const float decay = fast_exp2(csr[tt]);
#pragma unroll
            for (int g = 0; g < 4; ++g) {
              float y[4];
#pragma unroll
              for (int q = 0; q < 4; ++q) {
                const int e = 4 * g + q;
                const float zz = slot_f(zrow[tt][2 * pt + (e >> 3)], e & 7);
                const float acc = yacc[pt][tt][e] + yi[tt][e] * decay;
                y[q] = ok[tt] ? acc * (zz * sigmoid_fast(zz)) : 0.f;
              }
              const int p0 = 32 * pt + 8 * g + 4 * hh;
              if (a.out_dtype == TF_FLOAT32) {
                float* dst = static_cast<float*>(a.out) + oo + t * a.out_stride[1] + p0;
                *reinterpret_cast<float4*>(dst) = make_float4(y[0], y[1], y[2], y[3]);
              } else {
                uint16_t* dst = static_cast<uint16_t*>(a.out) + oo + t * a.out_stride[1] + p0;
                u32x2 pk;
                pk[0] = pack2(y[0], y[1]);
                pk[1] = pack2(y[2], y[3]);
                *reinterpret_cast<u32x2*>(dst) = pk;
              }
            }
          }
        }
      }
    }
  }
  // rows past the last valid chunk (only when lengths < T)
  const int P = 32 * PT;
  for (int e = nvalid * kChunk * P + threadIdx.x; e < T * P; e += W * 64) {
    const int t = e / P, p = e - t * P;
    store_f32(a.out, a.out_dtype, oo + t * a.out_stride[1] + p, 0.f);
  }
}

bool aligned(const void* p, int bytes) { return (reinterpret_cast<uintptr_t>(p) % bytes) == 0; }

bool rows_vectorisable(const void* p, const int64_t* st, int elem_bytes, int vec_bytes) {
  const int64_t m = vec_bytes / elem_bytes;
  return aligned(p, vec_bytes) && st[3] == 1 && st[0] % m == 0 && st[1] % m == 0 && st[2] % m == 0;
}

template <int NT, int PT, int W>
int launch_shape(const tf_mamba_args& a, hipStream_t stream) {
  const int64_t units = a.batch * a.heads;
  // Units sharing q/k rows (same batch) land on one XCD (workgroups are dealt
  // to the 8 XCDs round-robin), so their L2 serves the shared rows.
  const int xcd_per = (units % 8 == 0 && units >= 64) ? static_cast<int>(units / 8) : 0;
  hipLaunchKernelGGL((mamba_mfma_kernel<NT, PT, W>), dim3(static_cast<uint32_t>(units)), dim3(W * 64), 0, stream,
                     a, xcd_per);
  return launch_status();
}

// Four waves (one per SIMD, up to 512 registers each): the chunk-local working
// set of a 64-step chunk does not fit the 256 registers a wave gets at two
// waves per SIMD without spilling.
template <int NT, int PT>
int launch_waves(const tf_mamba_args& a, hipStream_t stream) {
  return launch_shape<NT, PT, 4>(a, stream);
}

}  // namespace

bool mfma_supported(const tf_mamba_args& a) {
  if (a.q_dtype != TF_BFLOAT16 || a.k_dtype != TF_BFLOAT16 || a.v_dtype != TF_BFLOAT16 || a.z_dtype != TF_BFLOAT16)
    return false;
  if (a.out_dtype != TF_BFLOAT16 && a.out_dtype != TF_FLOAT32) return false;
  if (!(a.state == 32 || a.state == 64 || a.state == 128)) return false;
  if (!(a.head_dim == 32 || a.head_dim == 64)) return false;
  if (a.batch * a.heads > 0x7fffffff) return false;
  if (!rows_vectorisable(a.q, a.q_stride, 2, 8) || !rows_vectorisable(a.k, a.k_stride, 2, 8) ||
      !rows_vectorisable(a.v, a.v_stride, 2, 8) || !rows_vectorisable(a.z, a.z_stride, 2, 8))
    return false;
  const int ob = a.out_dtype == TF_FLOAT32 ? 4 : 2;
  if (!rows_vectorisable(a.out, a.out_stride, ob, 4 * ob)) return false;
  return true;
}

int launch_mfma(const tf_mamba_args& a, hipStream_t stream) {
  const int nt = static_cast<int>(a.state / 32);
  const int pt = static_cast<int>(a.head_dim / 32);
  if (nt == 1 && pt == 1) return launch_waves<1, 1>(a, stream);
  if (nt == 1 && pt == 2) return launch_waves<1, 2>(a, stream);
  if (nt == 2 && pt == 1) return launch_waves<2, 1>(a, stream);
  if (nt == 2 && pt == 2) return launch_waves<2, 2>(a, stream);
  if (nt == 4 && pt == 1) return launch_waves<4, 1>(a, stream);
  if (nt == 4 && pt == 2) return launch_waves<4, 2>(a, stream);
  return TF_ERR_SHAPE;
}

}  // namespace tf
