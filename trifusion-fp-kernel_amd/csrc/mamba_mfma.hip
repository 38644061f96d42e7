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
// tanhf (S. L. Moshier, Cephes Math Library), else 1 - 2/(exp(2|x|) + 1) with the
// hardware exp2/rcp, evaluated only when some lane of the wave needs it.
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
  const float* adt;
  const float* dt;
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
  int out_f32, trap_bf16, angles_dtype;
};

// Global inputs of one wave's chunk, loaded ahead of use (rows c32 and c32+32 of
// the chunk in MFMA row form; phase lane (pp, seg) raw angles of its rows).
template <int KS, int PS, int RPMAX>
struct ChunkInputs {
  u32x4 q[2][KS], k[2][KS], v[2][PS];
  float dt[2], dn[2], tr[2], tn[2], adt[2];
  float th[RPMAX];
};

template <int RPMAX, typename E>
__device__ __forceinline__ void load_angles(const E* p, int st, int t0, int L, int seg, int rp, bool on,
                                            float (&th)[RPMAX]) {
  const int first = t0 + seg * rp;
  const E* row = p + first * st;
#pragma unroll
  for (int r = 0; r < RPMAX; ++r) {
    th[r] = (on && r < rp && first + r < L) ? to_f32(*row) : 0.f;
    row += st;
  }
}

template <int KS, int PS, int RPMAX>
__device__ __forceinline__ void load_chunk(const MfmaParams& P, ChunkInputs<KS, PS, RPMAX>& in, int b, int h, int qh,
                                           int t0, int L, int c32, int hh, int pp, int seg, int rp) {
  const float* dtp = P.dt + b * P.d_sb + h * P.d_sh;
  const float* adtp = P.adt + b * P.a_sb + h * P.a_sh;
  const int tro = b * P.r_sb + h * P.r_sh;
#pragma unroll
  for (int rt = 0; rt < 2; ++rt) {
    const int t = t0 + 32 * rt + c32;
    const bool valid = t < L;
    const bool next = t + 1 < P.T;
    in.dt[rt] = valid ? dtp[t * P.d_st] : 0.f;
    in.dn[rt] = next ? dtp[(t + 1) * P.d_st] : 0.f;
    in.adt[rt] = valid ? adtp[t * P.a_st] : 0.f;
    if (P.trap_bf16) {
      const bf16_t* tp = static_cast<const bf16_t*>(P.trap) + tro;
      in.tr[rt] = valid ? to_f32(tp[t * P.r_st]) : 0.f;
      in.tn[rt] = next ? to_f32(tp[(t + 1) * P.r_st]) : 0.f;
    } else {
      const float* tp = static_cast<const float*>(P.trap) + tro;
      in.tr[rt] = valid ? tp[t * P.r_st] : 0.f;
      in.tn[rt] = next ? tp[(t + 1) * P.r_st] : 0.f;
    }
    // rows past L read row t0 (in bounds) and never reach the outputs or the state
    const int tl = valid ? t : t0;
    const uint16_t* q_row = P.q + b * P.q_sb + qh * P.q_sh + tl * P.q_st;
    const uint16_t* k_row = P.k + b * P.k_sb + qh * P.k_sh + tl * P.k_st;
    const uint16_t* v_row = P.v + b * P.v_sb + h * P.v_sh + tl * P.v_st;
#pragma unroll
    for (int s = 0; s < KS; ++s) {
      in.q[rt][s] = load_row8(q_row, kidx(s, hh, 0));
      in.k[rt][s] = load_row8(k_row, kidx(s, hh, 0));
    }
#pragma unroll
    for (int s = 0; s < PS; ++s) in.v[rt][s] = load_row8(v_row, kidx(s, hh, 0));
  }
  const bool on = pp < P.R;
  const int go = b * P.g_sb + h * P.g_sh + (on ? pp : 0) * P.g_sr;
  if (P.angles_dtype == TF_FLOAT32)
    load_angles<RPMAX>(static_cast<const float*>(P.angles) + go, P.g_st, t0, L, seg, rp, on, in.th);
  else
    load_angles<RPMAX>(static_cast<const bf16_t*>(P.angles) + go, P.g_st, t0, L, seg, rp, on, in.th);
}

template <int NT, int PT, int W>
struct Smem {
  static constexpr int kTiles = NT * PT;
  static constexpr int kF4 = kTiles * 4 * 64;  // float4 per chunk state
  float4 state[W][kF4];  // [slot][tile][g][lane] = D elements 4g..4g+3 of tile (nt, pt)
  float cs[W][kChunk];   // cumulative log2 decay of each wave's chunk
  float dt[W][kChunk];   // dt of each wave's chunk rows
  float wv[W][kChunk];   // 2^(tot - cs): decay from each row to the chunk end
  float tot[W];
  double wsum[W][64];    // phase increment of each chunk per rotary pair
  double carry[64];      // phase carry entering the super-chunk
  float qb[32 * NT];
  float kb[32 * NT];
};

template <int NT, int PT, int W>
__global__ __launch_bounds__(W * 64) void mamba_mfma_kernel(const MfmaParams P) {
  constexpr int N = 32 * NT;
  constexpr int KS = N / 16;        // k-steps over the state dim
  constexpr int PS = PT * 2;        // k-steps over the head dim
  constexpr int RPMAX = N / 2;      // rows per phase lane at most (R <= N/2)
  using Sm = Smem<NT, PT, W>;
  constexpr int kF4 = Sm::kF4;
  constexpr int SPT = (kF4 + W * 64 - 1) / (W * 64);  // float4 of the running state per thread
  __shared__ Sm sh;

  const int lane = threadIdx.x & 63;
  const int w = threadIdx.x >> 6;
  const int c32 = lane & 31;
  const int hh = lane >> 5;
  const int unit = P.xcd_per > 0 ? (blockIdx.x & 7) * P.xcd_per + (blockIdx.x >> 3) : static_cast<int>(blockIdx.x);
  const int b = unit / P.H;
  const int h = unit - b * P.H;
  const int qh = h / P.group;
  const int T = P.T;
  const int R = P.R;
  int L = T;
  if (P.lengths != nullptr) {
    const int64_t l = P.lengths[b];
    L = l < 0 ? 0 : (l > T ? T : static_cast<int>(l));
  }
  const int nvalid = (L + kChunk - 1) / kChunk;
  // phase lanes: pair pp = lane % rp over rows [seg*rp, seg*rp + rp), rp = pow2 >= R
  int rp = 1;
  while (rp < R) rp <<= 1;
  const int pp = lane & (rp - 1);
  const int seg = lane / rp;
  const int rs = (R + 1) & ~1;  // row stride of the staged phases (even: 8-byte pair reads)
  const float skip = P.d[h];

  for (int i = threadIdx.x; i < 64; i += W * 64) sh.carry[i] = 0.0;
  for (int i = threadIdx.x; i < N; i += W * 64) {
    sh.qb[i] = P.qb[h * N + i];
    sh.kb[i] = P.kb[h * N + i];
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
    ChunkInputs<KS, PS, RPMAX> cur;
    load_chunk(P, cur, b, h, qh, t0, L, c32, hh, pp, seg, rp);

    // ---------------- phase A: chunk-local work ----------------
    float csr[2], gam[2], scl[2];
    {
      float da[2];
#pragma unroll
      for (int rt = 0; rt < 2; ++rt) {
        const float tr = sigmoid_fast(cur.tr[rt]);
        const float tn = sigmoid_fast(cur.tn[rt]);
        gam[rt] = cur.dt[rt] * tr;
        scl[rt] = cur.dn[rt] * (1.f - tn) + gam[rt];
        da[rt] = cur.adt[rt] * kLog2e;
      }
      // cumulative log2 decay over the chunk; both lane halves hold all 64 rows
      const float cs0 = half_scan(da[0], c32);
      const float cs1 = half_scan(da[1], c32) + half_last(cs0);
      const float tot = half_last(cs1);  // shuffle with every lane active
      csr[0] = cs0;
      csr[1] = cs1;
      if (hh == 0) {
        sh.cs[w][c32] = cs0;
        sh.cs[w][32 + c32] = cs1;
        sh.dt[w][c32] = cur.dt[0];
        sh.dt[w][32 + c32] = cur.dt[1];
        sh.wv[w][c32] = fast_exp2(tot - cs0);
        sh.wv[w][32 + c32] = fast_exp2(tot - cs1);
      }
      if (lane == 0) sh.tot[w] = tot;
      wave_sync();
    }
    // rotary phase, pass 1: increments pi*tanh(theta)*dt of the lane's rows to the
    // staging area and their fp64 sum; the chunk sum per pair goes to LDS
    double seg_part = 0.0;
    if (pp < R) {
      float* cell = phs + seg * rp * rs + pp;
      const float* dtr = &sh.dt[w][seg * rp];
#pragma unroll
      for (int r = 0; r < RPMAX; ++r) {
        if (r < rp) {
          const float om = tanh_fast(cur.th[r]) * kPi * dtr[r];
          *cell = om;
          seg_part += static_cast<double>(om);
        }
        cell += rs;
      }
    }
    {
      double sum = seg_part;
      for (int off = rp; off < 64; off <<= 1) sum += __shfl_xor(sum, off);
      if (seg == 0 && pp < R) sh.wsum[w][pp] = sum;
    }
    __syncthreads();  // barrier 1: chunk phase sums visible

    f32x16 yacc[PT][2];  // y^T tiles (pt, tt): lane = t, elements = p
    u32x4 qrow[2][KS];   // rotated q rows (Y operand over n)
    {
      // pass 2: carry of the preceding chunks + exclusive segment prefix + serial
      // fp64 cumsum, reduced to [0, 2pi) and staged as fp32 [row][pair]
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
        if (pp < R) {
          float* base = phs + seg * rp * rs + pp;
          float om[RPMAX];
#pragma unroll
          for (int r = 0; r < RPMAX; ++r) om[r] = r < rp ? base[r * rs] : 0.f;
          double cum = carry + pre - seg_part;
#pragma unroll
          for (int r = 0; r < RPMAX; ++r) {
            if (r < rp) {
              cum += static_cast<double>(om[r]);
              base[r * rs] = static_cast<float>(cum - kTwoPiD * floor(cum * (1.0 / kTwoPiD)));
            }
          }
        }
      }
      wave_sync();

      // bias + rotary + scale + bf16 rounding of q and k (mamba_fused.py:112-135),
      // with the skip-term partial sums gamma * (q + qb).(k + kb) over this lane's n
      // from the unrotated biased values (mamba_fused.py:124)
      u32x4 krow[2][KS];
      float part[2] = {0.f, 0.f};
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
        const bool rot = 8 * s < R;  // wave-uniform: pairs >= R are not rotated
        if (rot) {
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
            const uint32_t qw = cur.q[rt][s][q4];
            const uint32_t kw = cur.k[rt][s][q4];
            const float q0 = lo_f(qw) + qb0, q1 = hi_f(qw) + qb1;
            const float k0 = lo_f(kw) + kb0, k1 = hi_f(kw) + kb1;
            part[rt] += q0 * k0 + q1 * k1;
            const float sc = scl[rt];
            if (rot) {
              const float c = co[rt][q4], sn = si[rt][q4];
              qrow[rt][s][q4] = pack2(q0 * c - q1 * sn, q0 * sn + q1 * c);
              krow[rt][s][q4] = pack2((k0 * c - k1 * sn) * sc, (k0 * sn + k1 * c) * sc);
            } else {
              qrow[rt][s][q4] = pack2(q0, q1);
              krow[rt][s][q4] = pack2(k0 * sc, k1 * sc);
            }
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
          const float cst = csr[tt];
#pragma unroll
          for (int g = 0; g < 4; ++g) {
            const float4 csu = *reinterpret_cast<const float4*>(&sh.cs[w][32 * ut + 8 * g + 4 * hh]);
            const float cu[4] = {csu.x, csu.y, csu.z, csu.w};
            float vals[4];
#pragma unroll
            for (int q = 0; q < 4; ++q) {
              const int e = 4 * g + q;
              const float x = sacc[tile][e] * fast_exp2(fminf(cst - cu[q], 0.f));
              // the off-diagonal tile (u < 32 <= t) is entirely below the diagonal
              vals[q] = (tile == 1 || c32 > drow(e, hh)) ? x : 0.f;
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
      // decay-scaled copy rounded to bf16 (mamba_fused.py:151) -> Y rows p, K = u.
      // Rows past L carry v = 0, so they add nothing to the state.
#pragma unroll
      for (int rt = 0; rt < 2; ++rt)
        if (t0 + 32 * rt + c32 >= L)
#pragma unroll
          for (int s = 0; s < PS; ++s) cur.v[rt][s] = u32x4{0u, 0u, 0u, 0u};
      u32x4 vtx[PT][4], vsy[PT][4];
#pragma unroll
      for (int ut = 0; ut < 2; ++ut) {
        float sc16[16];
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const float4 wu = *reinterpret_cast<const float4*>(&sh.wv[w][32 * ut + 8 * g + 4 * hh]);
          sc16[4 * g] = wu.x;
          sc16[4 * g + 1] = wu.y;
          sc16[4 * g + 2] = wu.z;
          sc16[4 * g + 3] = wu.w;
        }
#pragma unroll
        for (int pt = 0; pt < PT; ++pt) {
          f32x16 d = mfma(cur.v[ut][2 * pt], ident0, zero16());
          d = mfma(cur.v[ut][2 * pt + 1], ident1, d);
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
    
      // y_intra^T[p][t] = (D + delta_t) v[t][p] + sum_u v^T[p][u] score[t][u]
#pragma unroll
      for (int pt = 0; pt < PT; ++pt) {
#pragma unroll
        for (int tt = 0; tt < 2; ++tt) {
          const float coef = skip + delta[tt];
#pragma unroll
          for (int e = 0; e < 16; ++e) yacc[pt][tt][e] = coef * slot_f(cur.v[tt][2 * pt + (e >> 3)], e & 7);
        }
        yacc[pt][0] = mfma(vtx[pt][0], scy[0][0], yacc[pt][0]);
        yacc[pt][0] = mfma(vtx[pt][1], scy[0][1], yacc[pt][0]);
#pragma unroll
        for (int k = 0; k < 4; ++k) yacc[pt][1] = mfma(vtx[pt][k], scy[1][k], yacc[pt][1]);
      }

    }
    __syncthreads();  // barrier 2: every dS in LDS

    // gate operand of this chunk and all inputs of the next super-chunk, loaded
    // while the state scan and the output phase run
    u32x4 zrow[2][PS];
#pragma unroll
    for (int rt = 0; rt < 2; ++rt) {
      const int t = t0 + 32 * rt + c32;
      const uint16_t* z_row = P.z + b * P.z_sb + h * P.z_sh + (t < L ? t : t0) * P.z_st;
#pragma unroll
      for (int s = 0; s < PS; ++s) zrow[rt][s] = load_row8(z_row, kidx(s, hh, 0));
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
          const bool ok = t < L;
          const float decay = fast_exp2(csr[tt]);
#pragma unroll
          for (int g = 0; g < 4; ++g) {
            float y[4];
#pragma unroll
            for (int q = 0; q < 4; ++q) {
              const int e = 4 * g + q;
              const float zz = slot_f(zrow[tt][2 * pt + (e >> 3)], e & 7);
              const float acc = yacc[pt][tt][e] + yi[tt][e] * decay;
              y[q] = ok ? acc * (zz * sigmoid_fast(zz)) : 0.f;
            }
            const int p0 = 32 * pt + 8 * g + 4 * hh;
            const int off = b * P.o_sb + h * P.o_sh + t * P.o_st + p0;
            if (P.out_f32) {
              *reinterpret_cast<float4*>(static_cast<float*>(P.out) + off) = make_float4(y[0], y[1], y[2], y[3]);
            } else {
              u32x2 pk;
              pk[0] = pack2(y[0], y[1]);
              pk[1] = pack2(y[2], y[3]);
              *reinterpret_cast<u32x2*>(static_cast<uint16_t*>(P.out) + off) = pk;
            }
          }
        }
      }
    }
  }
  // rows past the last valid chunk (only when lengths < T)
  constexpr int PD = 32 * PT;
  for (int e = nvalid * kChunk * PD + threadIdx.x; e < T * PD; e += W * 64) {
    const int t = e / PD, p = e - t * PD;
    const int off = b * P.o_sb + h * P.o_sh + t * P.o_st + p;
    if (P.out_f32)
      static_cast<float*>(P.out)[off] = 0.f;
    else
      static_cast<uint16_t*>(P.out)[off] = 0;
  }
}

bool aligned(const void* p, int bytes) { return (reinterpret_cast<uintptr_t>(p) % bytes) == 0; }

bool rows_vectorisable(const void* p, const int64_t* st, int elem_bytes, int vec_bytes) {
  const int64_t m = vec_bytes / elem_bytes;
  return aligned(p, vec_bytes) && st[3] == 1 && st[0] % m == 0 && st[1] % m == 0 && st[2] % m == 0;
}

// Largest element offset reachable through `n` dims of sizes/strides; strides
// must be non-negative.
bool fits_int32(const int64_t* sizes, const int64_t* strides, int n) {
  int64_t off = 0;
  for (int i = 0; i < n; ++i) {
    if (strides[i] < 0 || strides[i] > 0x7fffffff) return false;
    if (sizes[i] > 0) off += (sizes[i] - 1) * strides[i];
  }
  return off < 0x7fffffff - 64;
}

bool offsets_fit(const tf_mamba_args& a) {
  const int64_t qs[4] = {a.batch, a.time, a.qk_heads, a.state};
  const int64_t vs[4] = {a.batch, a.time, a.heads, a.head_dim};
  const int64_t gs[4] = {a.batch, a.time, a.heads, a.rotary};
  const int64_t cs[3] = {a.batch, a.heads, a.time + 1};
  return fits_int32(qs, a.q_stride, 4) && fits_int32(qs, a.k_stride, 4) && fits_int32(vs, a.v_stride, 4) &&
         fits_int32(vs, a.z_stride, 4) && fits_int32(vs, a.out_stride, 4) && fits_int32(gs, a.angles_stride, 4) &&
         fits_int32(cs, a.adt_stride, 3) && fits_int32(cs, a.dt_stride, 3) && fits_int32(cs, a.trap_stride, 3);
}

MfmaParams make_params(const tf_mamba_args& a) {
  MfmaParams P;
  P.q = static_cast<const uint16_t*>(a.q);
  P.k = static_cast<const uint16_t*>(a.k);
  P.v = static_cast<const uint16_t*>(a.v);
  P.z = static_cast<const uint16_t*>(a.z);
  P.adt = static_cast<const float*>(a.adt);
  P.dt = static_cast<const float*>(a.dt);
  P.trap = a.trap;
  P.angles = a.angles;
  P.qb = a.qb;
  P.kb = a.kb;
  P.d = a.d;
  P.out = a.out;
  P.lengths = a.lengths;
  P.q_sb = static_cast<int>(a.q_stride[0]), P.q_st = static_cast<int>(a.q_stride[1]), P.q_sh = static_cast<int>(a.q_stride[2]);
  P.k_sb = static_cast<int>(a.k_stride[0]), P.k_st = static_cast<int>(a.k_stride[1]), P.k_sh = static_cast<int>(a.k_stride[2]);
  P.v_sb = static_cast<int>(a.v_stride[0]), P.v_st = static_cast<int>(a.v_stride[1]), P.v_sh = static_cast<int>(a.v_stride[2]);
  P.z_sb = static_cast<int>(a.z_stride[0]), P.z_st = static_cast<int>(a.z_stride[1]), P.z_sh = static_cast<int>(a.z_stride[2]);
  P.o_sb = static_cast<int>(a.out_stride[0]), P.o_st = static_cast<int>(a.out_stride[1]), P.o_sh = static_cast<int>(a.out_stride[2]);
  P.g_sb = static_cast<int>(a.angles_stride[0]), P.g_st = static_cast<int>(a.angles_stride[1]);
  P.g_sh = static_cast<int>(a.angles_stride[2]), P.g_sr = static_cast<int>(a.angles_stride[3]);
  P.a_sb = static_cast<int>(a.adt_stride[0]), P.a_sh = static_cast<int>(a.adt_stride[1]), P.a_st = static_cast<int>(a.adt_stride[2]);
  P.d_sb = static_cast<int>(a.dt_stride[0]), P.d_sh = static_cast<int>(a.dt_stride[1]), P.d_st = static_cast<int>(a.dt_stride[2]);
  P.r_sb = static_cast<int>(a.trap_stride[0]), P.r_sh = static_cast<int>(a.trap_stride[1]), P.r_st = static_cast<int>(a.trap_stride[2]);
  P.T = static_cast<int>(a.time);
  P.H = static_cast<int>(a.heads);
  P.group = static_cast<int>(a.heads / a.qk_heads);
  P.R = static_cast<int>(a.rotary);
  const int64_t units = a.batch * a.heads;
  // Units sharing q/k rows (same batch) land on one XCD (workgroups are dealt
  // to the 8 XCDs round-robin), so their L2 serves the shared rows.
  P.xcd_per = (units % 8 == 0 && units >= 64) ? static_cast<int>(units / 8) : 0;
  P.out_f32 = a.out_dtype == TF_FLOAT32;
  P.trap_bf16 = a.trap_dtype == TF_BFLOAT16;
  P.angles_dtype = a.angles_dtype;
  return P;
}

template <int NT, int PT, int W>
int launch_shape(const tf_mamba_args& a, hipStream_t stream) {
  const int64_t units = a.batch * a.heads;
  hipLaunchKernelGGL((mamba_mfma_kernel<NT, PT, W>), dim3(static_cast<uint32_t>(units)), dim3(W * 64), 0, stream,
                     make_params(a));
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
  if (a.adt_dtype != TF_FLOAT32 || a.dt_dtype != TF_FLOAT32) return false;
  if (a.trap_dtype != TF_FLOAT32 && a.trap_dtype != TF_BFLOAT16) return false;
  if (a.angles_dtype != TF_FLOAT32 && a.angles_dtype != TF_BFLOAT16) return false;
  if (a.out_dtype != TF_BFLOAT16 && a.out_dtype != TF_FLOAT32) return false;
  if (!(a.state == 32 || a.state == 64 || a.state == 128)) return false;
  if (!(a.head_dim == 32 || a.head_dim == 64)) return false;
  // the phase staging area [64 rows][R rounded up to even] lives in a state slot
  if (64 * ((a.rotary + 1) & ~int64_t(1)) > (a.state / 32) * (a.head_dim / 32) * 1024) return false;
  if (a.batch * a.heads > 0x7fffffff) return false;
  if (!rows_vectorisable(a.q, a.q_stride, 2, 8) || !rows_vectorisable(a.k, a.k_stride, 2, 8) ||
      !rows_vectorisable(a.v, a.v_stride, 2, 8) || !rows_vectorisable(a.z, a.z_stride, 2, 8))
    return false;
  const int ob = a.out_dtype == TF_FLOAT32 ? 4 : 2;
  if (!rows_vectorisable(a.out, a.out_stride, ob, 4 * ob)) return false;
  return offsets_fit(a);
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
