// Chunked-scan fused Mamba-3 SISO recurrence on gfx950 bf16 MFMA.
//
// Same arithmetic and bf16 rounding points as the reference kernel
// (src/trifusion_l4/mamba_fused.py:72-152), reorganised for CDNA4:
//
//   * One workgroup per (batch, head) unit. The sequence is walked in
//     "super-chunks" of CW chunks of 64 steps. Each chunk is split over two
//     waves, one per 32-step half, so a workgroup runs 2*CW waves (two per SIMD
//     for CW = 4): every wave works on one 32-row MFMA tile, which keeps its
//     working set inside the 256 registers a wave gets at two waves per SIMD,
//     and the second wave on each SIMD hides the first one's memory and
//     dependency latency.
//   * Chunk semantics are unchanged: the cumulative decay, the causal score
//     mask, the state contribution dS and the bf16 rounding of the state all
//     follow 64-step chunks. The half-1 wave receives the half-0 wave's rotated
//     k rows and v^T tile through LDS for its off-diagonal score tile and y
//     term; each half writes its share of dS, and the state scan adds the two.
//   * The only serial dependency, the fp32 state S <- S*2^tot + dS, is a
//     prefix scan over the CW chunk contributions held in LDS: every thread of
//     the workgroup owns a slice of the P x N state and walks the CW chunks,
//     replacing each chunk's dS with the exclusive state S_c entering it. Each
//     wave then adds 2^cs * qr . bf16(S_c)^T to its outputs.
//   * All contractions run on v_mfma_f32_32x32x16_bf16. Operands come straight
//     from global memory in MFMA register layout (8-byte loads of four
//     consecutive elements); the transposes the contractions over time need
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
// product's operand (mfma_tile.h).
#include "mfma_tile.h"

namespace tf {
namespace {

template <int NT, int PT, int CW>
struct Smem {
  static constexpr int kF4 = NT * PT * 256;  // float4 per chunk state ([tile][g][lane])
  // Per chunk slot, in the order of use within a super-chunk:
  //   a: half-0 -> half-1 exchange (kr rows, v^T tile), then half 1's dS, then
  //      the exclusive state S_c read by the output phase;
  //   b: rotary phase staging [row][pair], then half 0's dS.
  float4 a[CW][kF4];
  float4 b[CW][kF4];
  float cs[CW][kChunk];  // cumulative log2 decay over the chunk
  float dt[CW][kChunk];  // dt of the chunk rows
  float wv[CW][kChunk];  // 2^(tot - cs): decay from each row to the chunk end
  float htot[2 * CW];    // log2 decay of each half (wave) on its own
  double wsum[2 * CW][64];  // phase increment of each half per rotary pair
  double carry[64];         // phase carry entering the super-chunk
  float qb[32 * NT];
  float kb[32 * NT];
  float qw[32 * NT];  // B/C norm weights (fused norms only)
  float kw[32 * NT];
};

// Global inputs of one wave's 32 rows, in two parts loaded at different
// times. Rows past L read a valid row; their dt is 0, so they reach neither the
// outputs nor the state.
//   HalfRows: row t of the lane in MFMA row form (q for the output pass, k, v),
//     loaded at the start of the super-chunk that uses them (first needed after
//     the controls and phase pass 1, which cover their latency);
//   HalfCtl: the controls of row t and, for the phase lane, the raw angles of
//     rows first .. first+RPL-1 of its rotary pair (column offset gcol),
//     prefetched one super-chunk ahead (needed first thing).
template <int KS, int PS>
struct HalfRows {
  u32x4 q[KS], k[KS], v[PS];
};

template <int RPL>
struct HalfCtl {
  float th[RPL];
  float dt, dn, adt, tr, tn;
};

template <bool WITH_Q, int KS, int PS>
__device__ __forceinline__ void load_rows(const MfmaParams& P, HalfRows<KS, PS>& in, const uint16_t* qbase,
                                          const uint16_t* kbase, const uint16_t* vbase, int t0, int t, int L,
                                          int hh) {
  const int tl = t < L ? t : t0;
  const uint16_t* q_row = qbase + tl * P.q_st;
  const uint16_t* k_row = kbase + tl * P.k_st;
  const uint16_t* v_row = vbase + tl * P.v_st;
#pragma unroll
  for (int s = 0; s < KS; ++s) {
    // k-steps past a 16-channel state are the zero padding (nothing to load)
    if (16 * s < P.n_real) {
      if constexpr (WITH_Q) in.q[s] = load_row8(q_row, kidx(s, hh, 0));
      in.k[s] = load_row8(k_row, kidx(s, hh, 0));
    } else {
      if constexpr (WITH_Q) in.q[s] = u32x4{0u, 0u, 0u, 0u};
      in.k[s] = u32x4{0u, 0u, 0u, 0u};
    }
  }
#pragma unroll
  for (int s = 0; s < PS; ++s) in.v[s] = load_row8(v_row, kidx(s, hh, 0));
}


// Loads row t's controls (raw values when P.ctl_raw; converted where used, so
// the loads stay in flight) and the halo step t + 1 when t + 1 < tlim: T, or
// the valid length of a reversed unit, whose step L has no row.
template <int RPL>
__device__ __forceinline__ void load_ctl(const MfmaParams& P, HalfCtl<RPL>& in, int dto, int ado, int trb,
                                         int gcol, int t, int first, int L, int tlim) {
  const bool valid = t < L;
  const bool next = t + 1 < tlim;
  in.dt = valid ? ctl_value(P.dt, P.ctl_bf16, dto + t * P.d_st) : 0.f;
  in.dn = next ? ctl_value(P.dt, P.ctl_bf16, dto + (t + 1) * P.d_st) : 0.f;
  in.adt = valid ? ctl_value(P.adt, P.ctl_bf16, ado + t * P.a_st) : 0.f;
  if (P.trap_bf16) {
    const bf16_t* tp = static_cast<const bf16_t*>(P.trap) + trb;
    in.tr = valid ? to_f32(tp[t * P.r_st]) : 0.f;
    in.tn = next ? to_f32(tp[(t + 1) * P.r_st]) : 0.f;
  } else {
    const float* tp = static_cast<const float*>(P.trap) + trb;
    in.tr = valid ? tp[t * P.r_st] : 0.f;
    in.tn = next ? tp[(t + 1) * P.r_st] : 0.f;
  }
  if (P.angles_dtype == TF_FLOAT32) {
    const float* ap = static_cast<const float*>(P.angles) + gcol;
#pragma unroll
    for (int r = 0; r < RPL; ++r) in.th[r] = ap[min(first + r, L - 1) * P.g_st];
  } else {
    const bf16_t* ap = static_cast<const bf16_t*>(P.angles) + gcol;
#pragma unroll
    for (int r = 0; r < RPL; ++r) in.th[r] = to_f32(ap[min(first + r, L - 1) * P.g_st]);
  }
}

// WIDE: R in (N/4, N/2], else R <= N/4. The phase lanes of a wave take pair
// pp = lane % RP over RPL consecutive rows of the wave's half, segment
// seg = lane / RP (64 / RP segments of RPL rows cover the 32 rows).
// MODE 0 computes the outputs of the workgroup's chunks, starting from the
// state and phase carry entering its time segment (zero, or the segment
// scan's record). MODE 1 is the summary pass of the chunk-parallel form: from
// zero it computes only the segment's state contribution, log2 decay and phase
// sum (no q, z, scores or outputs) and writes them to the segment's record.
template <int NT, int PT, int CW, bool WIDE, int MODE>
__global__ __launch_bounds__(CW * 128) void mamba_mfma_kernel(const MfmaParams P) {
  constexpr int W = 2 * CW;         // waves: two per chunk
  constexpr int N = 32 * NT;
  constexpr int KS = N / 16;        // k-steps over the state dim
  constexpr int PS = PT * 2;        // k-steps over the head dim
  constexpr int RPL = WIDE ? N / 4 : N / 8;  // phase rows per lane
  constexpr int RP = 2 * RPL;                // pairs covered by the phase lanes (>= R)
  using Sm = Smem<NT, PT, CW>;
  constexpr int kF4 = Sm::kF4;
  constexpr int SPT = (kF4 + W * 64 - 1) / (W * 64);  // float4 of the running state per thread
  static_assert((KS + 2 * PT) * 64 <= kF4, "exchange tile does not fit its slot");
  __shared__ Sm sh;

  const int w = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
  const int cw = w % CW;        // chunk slot
  const int hf = w / CW;        // half: rows 32*hf .. 32*hf + 31 of the chunk
  const int sub = 2 * cw + hf;  // time order of the wave's rows within the super-chunk
  // work item = (time segment, unit), units fastest, so the units sharing a
  // segment's q/k rows sit next to each other and land on one XCD
  const int item = P.xcd_per > 0 ? (blockIdx.x & 7) * P.xcd_per + (blockIdx.x >> 3) : static_cast<int>(blockIdx.x);
  const int tseg = item / P.units;
  const int unit = item - tseg * P.units;
  const int rec = unit * P.G + tseg;
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
  // chunks [c_begin, c_end) are this workgroup's; those below c_stop are valid
  const int c_begin = tseg * P.SC;
  const int c_end = min(c_begin + P.SC, (T + kChunk - 1) / kChunk);
  const int c_stop = min(c_end, nvalid);
  // Row stride of the staged phases: even (8-byte pair reads) and, where the
  // slot has room, 2 more than a multiple of 4 floats, so that the rows of one
  // read (lane = row) fall on distinct LDS banks; a multiple of 16 floats would
  // put 16 rows on the same bank.
  const int rs0 = (R + 1) & ~1;
  const int rs = (rs0 % 4 == 0 && 64 * (rs0 + 2) <= 4 * kF4) ? rs0 + 2 : rs0;
  const float skip = P.d[h];
  const int tlim = P.rev ? L : T;  // steps that have a row (halo bound)

  // per-unit bases, at row L-1 for a reversed unit (the time strides are
  // negated, so step t lands on row L-1-t)
  const int roff = P.rev ? max(L - 1, 0) : 0;
  const uint16_t* qbase = P.q + b * P.q_sb + qh * P.q_sh - roff * P.q_st;
  const uint16_t* kbase = P.k + b * P.k_sb + qh * P.k_sh - roff * P.k_st;
  const uint16_t* vbase = P.v + b * P.v_sb + h * P.v_sh - roff * P.v_st;
  const uint16_t* zbase = P.z + b * P.z_sb + h * P.z_sh - roff * P.z_st;
  const int dto = b * P.d_sb + h * P.d_sh - roff * P.d_st;
  const int ado = b * P.a_sb + h * P.a_sh - roff * P.a_st;
  const int trb = b * P.r_sb + h * P.r_sh - roff * P.r_st;
  const int gbase = b * P.g_sb + h * P.g_sh - roff * P.g_st;
  const int obase = b * P.o_sb + h * P.o_sh - roff * P.o_st;
  const float step_bias = P.ctl_raw ? P.dt_bias[h] : 0.f;

  // Phase carry entering the segment (both passes): the fp64 sum of the
  // preceding chunks' phase sums, reduced mod 2pi. kr depends on the absolute
  // phase, so even the summary pass needs it. State entering the segment
  // (output pass only): the segment scan's record.
  const bool seeded = MODE == 0 && P.G > 1;
  for (int i = threadIdx.x; i < 64; i += W * 64) {
    double acc = 0.0;
    if (P.G > 1 && i < R) {
      const double* cp = P.chunk_phase + static_cast<size_t>(unit) * P.NC * 64 + i;
#pragma unroll 8
      for (int c = 0; c < c_begin; ++c) acc += cp[c * 64];
      acc -= kTwoPiD * floor(acc * (1.0 / kTwoPiD));
    }
    sh.carry[i] = acc;
  }
  // biases and norm weights; a 16-channel state's padding channels get 0, so
  // they stay 0 through bias, norm, rotation and scale
  for (int i = threadIdx.x; i < N; i += W * 64) {
    const bool real = i < P.n_real;
    sh.qb[i] = real ? P.qb[h * P.n_real + i] : 0.f;
    sh.kb[i] = real ? P.kb[h * P.n_real + i] : 0.f;
    if (P.qk_norm) {
      sh.qw[i] = real ? P.qn_w[i] : 0.f;
      sh.kw[i] = real ? P.kn_w[i] : 0.f;
    }
  }
  float4 run[SPT];
#pragma unroll
  for (int r = 0; r < SPT; ++r) {
    const int f = threadIdx.x + r * W * 64;
    run[r] = (seeded && f < kF4) ? P.seg_state[static_cast<size_t>(rec) * kF4 + f] : make_float4(0.f, 0.f, 0.f, 0.f);
  }
  float seg_log2 = 0.f;  // log2 decay over the segment (summary pass)
  const u32x4 ident0 = identity_rows(0, (threadIdx.x >> 5) & 1, threadIdx.x & 31);
  const u32x4 ident1 = identity_rows(1, (threadIdx.x >> 5) & 1, threadIdx.x & 31);

  // controls and angles of the first super-chunk; later ones are prefetched one
  // super-chunk ahead, while the state scan and the output phase run
  using Ctl = HalfCtl<RPL>;
  Ctl cur = {};
  if (c_begin + cw < c_stop) {
    const int ln = threadIdx.x & 63;
    const int p0 = ln & (RP - 1);
    const int r0 = (c_begin + cw) * kChunk + 32 * hf;
    load_ctl(P, cur, dto, ado, trb, gbase + (p0 < R ? p0 : 0) * P.g_sr, r0 + (ln & 31), r0 + (ln / RP) * RPL, L,
             tlim);
  }

  lds_barrier();

  // Half 0's q/k/v rows of the next super-chunk, issued before the state scan of
  // this one (the scan and the output phase cover their latency). Half 1 keeps
  // loading its rows after phase pass 1, which staggers the two halves' bursts;
  // prefetching both halves, or issuing the next controls before the scan, was
  // slower.
  // N = 128, P = 64 with one chunk per super-chunk runs at one wave per SIMD
  // and spills into AGPRs; the next chunk's rows are loaded where used instead
  // of being held across the chunk.
  constexpr bool kPrefetch = !(NT == 4 && PT == 2 && CW == 1);
  HalfRows<KS, PS> pre = {};
  for (int g0 = c_begin; g0 < c_stop; g0 += CW) {
    // Lane-derived indices are rebuilt from an index the compiler cannot see
    // through each iteration: hoisted out of the loop, the dozens of per-lane
    // addresses they feed would stay live across it and spill.
    int tid = static_cast<int>(threadIdx.x);
    asm volatile("" : "+v"(tid));
    const int lane = tid & 63;
    const int c32 = lane & 31;
    const int hh = lane >> 5;
    const int pp = lane & (RP - 1);
    const int seg = lane / RP;
    const bool pair_on = pp < R;
    const int nact = min(CW, c_stop - g0);
    const bool active = cw < nact;  // wave-uniform; idle waves only join the barriers
    const int t0 = (g0 + cw) * kChunk;
    const int t = t0 + 32 * hf + c32;  // row of this lane in the row-form tiles
    float* stg = reinterpret_cast<float*>(&sh.b[cw][0]);  // [64][rs] phase staging

    // Values carried from one "if (active)" region to a later one are given a
    // definition on the idle path too: left undefined there, the compiler
    // carries them around the loop and holds their registers through every phase.
    // Row loads are issued at two points: half 0 here, half 1 after its phase
    // pass 1. Load issue stalls while the chip-wide burst drains; staggered, one
    // wave of each SIMD computes while the other waits.
    HalfRows<KS, PS> rows = {};
    if (active && hf == 0) {
      if (g0 == c_begin || !kPrefetch)
        load_rows<MODE == 0>(P, rows, qbase, kbase, vbase, t0, t, L, hh);
      else
        rows = pre;
    }
    u32x4 (&q)[KS] = rows.q;
    u32x4 (&k)[KS] = rows.k;
    u32x4 (&v)[PS] = rows.v;
    float (&th)[RPL] = cur.th;
    float dtv = cur.dt;
    float csr = 0.f, gam = 0.f, scl = 0.f;
    double seg_part = 0.0;
    // ---------------- controls, phase pass 1 ----------------
    if (active) {
      float dnv = cur.dn, adv = cur.adt;
      if (P.ctl_raw) {
        // step and decay from the raw columns (primitives.py:209-214); rows
        // without a step keep dt = adt = 0
        dtv = t < L ? control_step(dtv, step_bias) : 0.f;
        dnv = t + 1 < tlim ? control_step(dnv, step_bias) : 0.f;
        adv = t < L ? control_decay(adv, dtv, P.a_floor) : 0.f;
      }
      // controls (mamba_fused.py:98-110) and the half's cumulative log2 decay
      gam = dtv * sigmoid_fast(cur.tr);
      scl = dnv * (1.f - sigmoid_fast(cur.tn)) + gam;
      csr = half_scan(adv * kLog2e, c32);
      const float ltot = half_last(csr);
      if (hh == 0) {
        sh.dt[cw][32 * hf + c32] = dtv;
        if (hf == 0) sh.cs[cw][c32] = csr;  // final for half 0
      }
      if (lane == 0) sh.htot[w] = ltot;
      wave_sync();

      // rotary phase, pass 1: increments pi*tanh(theta)*dt of the lane's rows
      // (kept in th[]) and their fp64 sum; the half's sum per pair goes to LDS
      const float* dtr = &sh.dt[cw][32 * hf + seg * RPL];
#pragma unroll
      for (int r = 0; r < RPL; ++r) {
        th[r] = tanh_fast(th[r]) * kPi * dtr[r];
        seg_part += static_cast<double>(th[r]);
      }
      if (!pair_on) seg_part = 0.0;
      double sum = seg_part;
      for (int off = RP; off < 64; off <<= 1) sum += __shfl_xor(sum, off);
      if (seg == 0 && pair_on) sh.wsum[sub][pp] = sum;
      if (hf == 1) load_rows<MODE == 0>(P, rows, qbase, kbase, vbase, t0, t, L, hh);
    }
    lds_barrier();  // barrier 1: half sums of decay and phase visible

    u32x4 qrow[KS] = {};  // rotated q rows (Y operand over n)
    u32x4 scy_d[2] = {};  // diagonal score tile (Y rows t, K = u of this half)
    u32x4 ktx[NT][2] = {}, vtx[PT][2] = {}, vsy[PT][2] = {};
    float csf = 0.f, delta = 0.f;
    // ---------------- phase pass 2, rotary, own-half products ----------------
    if (active) {
      const float tot = sh.htot[CW + cw] + sh.htot[cw];  // chunk total, same sum as half 1's last cs
      csf = hf ? csr + sh.htot[cw] : csr;
      if (hh == 0) {
        if (hf) sh.cs[cw][32 + c32] = csf;
        sh.wv[cw][32 * hf + c32] = fast_exp2(tot - csf);
      }
      // pass 2: carry of the preceding halves + exclusive segment prefix + serial
      // fp64 cumsum, reduced to [0, 2pi) and staged as fp32 [row][pair]
      {
        const int ppc = pair_on ? pp : 0;
        double carry = sh.carry[ppc];
#pragma unroll
        for (int j = 0; j < 2 * CW; ++j) {  // independent reads, summed in order
          const double x = sh.wsum[j][ppc];
          carry += j < sub ? x : 0.0;
        }
        double pre = seg_part;  // inclusive scan over the segments of the same pair
        for (int off = RP; off < 64; off <<= 1) {
          const double o = __shfl_up(pre, off);
          if (lane >= off) pre += o;
        }
        double cum = carry + pre - seg_part;
        float* cell = stg + (32 * hf + seg * RPL) * rs + pp;
        if (pair_on) {
#pragma unroll
          for (int r = 0; r < RPL; ++r) {
            cum += static_cast<double>(th[r]);
            cell[r * rs] = static_cast<float>(cum - kTwoPiD * floor(cum * (1.0 / kTwoPiD)));
          }
        }
      }
      wave_sync();

      // bias + rotary + scale + bf16 rounding of q and k (mamba_fused.py:112-135),
      // with the skip-term partial sums gamma * (q + qb).(k + kb) over this lane's n
      // from the unrotated biased values (mamba_fused.py:124)
      u32x4 krow[KS];
      float part = 0.f;
      // zero the compiler cannot see through: keeps the bias reads inside the
      // loop instead of 4*N registers held across it
      int bias_off = 0;
      asm volatile("" : "+v"(bias_off));
      const float* prow = stg + (32 * hf + c32) * rs;
      // Fused B/C RMSNorm (mamba.py:56-57): the row's sum of squares over this
      // lane's half of the state dim and the other half's (lane ^ 32), then
      // each element x -> bf16(x * rsqrt(mean(x^2) + eps) * w) before its bias.
      // The multiply-adds are spelled out, so the summary pass (MODE 1) and
      // the output pass normalise a key row to the same bits.
      float rq = 0.f, rk = 0.f;
      if (P.qk_norm) {
        float sq = 0.f, sk = 0.f;
#pragma unroll
        for (int s = 0; s < KS; ++s) {
#pragma unroll
          for (int q4 = 0; q4 < 4; ++q4) {
            if constexpr (MODE == 0) {
              sq = __builtin_fmaf(lo_f(q[s][q4]), lo_f(q[s][q4]), sq);
              sq = __builtin_fmaf(hi_f(q[s][q4]), hi_f(q[s][q4]), sq);
            }
            sk = __builtin_fmaf(lo_f(k[s][q4]), lo_f(k[s][q4]), sk);
            sk = __builtin_fmaf(hi_f(k[s][q4]), hi_f(k[s][q4]), sk);
          }
        }
        if constexpr (MODE == 0) sq += __shfl_xor(sq, 32);
        sk += __shfl_xor(sk, 32);
        rq = rsqrtf(sq / static_cast<float>(P.n_real) + P.norm_eps);
        rk = rsqrtf(sk / static_cast<float>(P.n_real) + P.norm_eps);
      }
#pragma unroll
      for (int s = 0; s < KS; ++s) {
        float co[4] = {1.f, 1.f, 1.f, 1.f}, si[4] = {0.f, 0.f, 0.f, 0.f};
        const bool rot = 8 * s < R;  // wave-uniform: pairs >= R are not rotated
        if (rot) {
#pragma unroll
          for (int half = 0; half < 2; ++half) {
            const int pr = 8 * s + 2 * hh + 4 * half;
            const float2 ph = *reinterpret_cast<const float2*>(prow + min(pr, rs - 2));
#pragma unroll
            for (int u = 0; u < 2; ++u) {
              const float x = u ? ph.y : ph.x;
              if (pr + u < R) {
                co[2 * half + u] = __builtin_amdgcn_cosf(x * kInvTwoPi);
                si[2 * half + u] = __builtin_amdgcn_sinf(x * kInvTwoPi);
              }
            }
          }
        }
        // biases of the lane's 8 state indices (two 16-byte LDS reads each)
        const float4 qbl = *reinterpret_cast<const float4*>(&sh.qb[kidx(s, hh, 0) + bias_off]);
        const float4 qbh = *reinterpret_cast<const float4*>(&sh.qb[kidx(s, hh, 4) + bias_off]);
        const float4 kbl = *reinterpret_cast<const float4*>(&sh.kb[kidx(s, hh, 0) + bias_off]);
        const float4 kbh = *reinterpret_cast<const float4*>(&sh.kb[kidx(s, hh, 4) + bias_off]);
        const float qbs[8] = {qbl.x, qbl.y, qbl.z, qbl.w, qbh.x, qbh.y, qbh.z, qbh.w};
        const float kbs[8] = {kbl.x, kbl.y, kbl.z, kbl.w, kbh.x, kbh.y, kbh.z, kbh.w};
        float qns[8] = {}, kns[8] = {};
        if (P.qk_norm) {
          const float4 ql = *reinterpret_cast<const float4*>(&sh.qw[kidx(s, hh, 0) + bias_off]);
          const float4 qh4 = *reinterpret_cast<const float4*>(&sh.qw[kidx(s, hh, 4) + bias_off]);
          const float4 kl = *reinterpret_cast<const float4*>(&sh.kw[kidx(s, hh, 0) + bias_off]);
          const float4 kh4 = *reinterpret_cast<const float4*>(&sh.kw[kidx(s, hh, 4) + bias_off]);
          const float qa[8] = {ql.x, ql.y, ql.z, ql.w, qh4.x, qh4.y, qh4.z, qh4.w};
          const float ka[8] = {kl.x, kl.y, kl.z, kl.w, kh4.x, kh4.y, kh4.z, kh4.w};
#pragma unroll
          for (int j = 0; j < 8; ++j) qns[j] = qa[j], kns[j] = ka[j];
        }
#pragma unroll
        for (int q4 = 0; q4 < 4; ++q4) {
          const float qb0 = qbs[2 * q4], qb1 = qbs[2 * q4 + 1];
          const float kb0 = kbs[2 * q4], kb1 = kbs[2 * q4 + 1];
          uint32_t qw = q[s][q4];
          uint32_t kw = k[s][q4];
          if (P.qk_norm) {
            if constexpr (MODE == 0)
              qw = pack2(lo_f(qw) * rq * qns[2 * q4], hi_f(qw) * rq * qns[2 * q4 + 1]);
            kw = pack2(lo_f(kw) * rk * kns[2 * q4], hi_f(kw) * rk * kns[2 * q4 + 1]);
          }
          const float q0 = lo_f(qw) + qb0, q1 = hi_f(qw) + qb1;
          const float k0 = lo_f(kw) + kb0, k1 = hi_f(kw) + kb1;
          if constexpr (MODE == 0) part += q0 * k0 + q1 * k1;
          if (rot) {
            const float c = co[q4], sn = si[q4];
            if constexpr (MODE == 0) qrow[s][q4] = pack2(q0 * c - q1 * sn, q0 * sn + q1 * c);
            krow[s][q4] = pack2((k0 * c - k1 * sn) * scl, (k0 * sn + k1 * c) * scl);
          } else {
            if constexpr (MODE == 0) qrow[s][q4] = pack2(q0, q1);
            krow[s][q4] = pack2(k0 * scl, k1 * scl);
          }
        }
      }
      float4* ex = &sh.a[cw][0];
      if constexpr (MODE == 0) {
        delta = gam * (part + __shfl_xor(part, 32));
        if (hf == 0) {
#pragma unroll
          for (int s = 0; s < KS; ++s) ex[s * 64 + lane] = as_f4(krow[s]);
        }
        // diagonal score tile of this half
        f32x16 sacc = zero16();
#pragma unroll
        for (int s = 0; s < KS; ++s) sacc = mfma(krow[s], qrow[s], sacc);
        score_tile(sacc, csf, &sh.cs[cw][32 * hf], true, c32, hh, scy_d);
      }
      // kr^T via the identity tile: D[u][n] = kr[u][n] -> X rows n, K = u
#pragma unroll
      for (int nt = 0; nt < NT; ++nt) {
        f32x16 d = mfma(krow[2 * nt], ident0, zero16());
        d = mfma(krow[2 * nt + 1], ident1, d);
#pragma unroll
        for (int sp = 0; sp < 2; ++sp)
#pragma unroll
          for (int q4 = 0; q4 < 4; ++q4) ktx[nt][sp][q4] = pack2(d[8 * sp + 2 * q4], d[8 * sp + 2 * q4 + 1]);
      }
      // v^T via the identity tile: D[u][p] = v[u][p] -> X rows p, K = u; and the
      // decay-scaled copy rounded to bf16 (mamba_fused.py:151) -> Y rows p, K = u.
      // Rows past L carry v = 0, so they add nothing to the state.
      if (t >= L) {
#pragma unroll
        for (int s = 0; s < PS; ++s) v[s] = u32x4{0u, 0u, 0u, 0u};
      }
      float sc16[16];
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const float4 wu = *reinterpret_cast<const float4*>(&sh.wv[cw][32 * hf + 8 * g + 4 * hh]);
        sc16[4 * g] = wu.x;
        sc16[4 * g + 1] = wu.y;
        sc16[4 * g + 2] = wu.z;
        sc16[4 * g + 3] = wu.w;
      }
#pragma unroll
      for (int pt = 0; pt < PT; ++pt) {
        f32x16 d = mfma(v[2 * pt], ident0, zero16());
        d = mfma(v[2 * pt + 1], ident1, d);
#pragma unroll
        for (int sp = 0; sp < 2; ++sp)
#pragma unroll
          for (int q4 = 0; q4 < 4; ++q4) {
            const int e = 8 * sp + 2 * q4;
            if constexpr (MODE == 0) vtx[pt][sp][q4] = pack2(d[e], d[e + 1]);
            vsy[pt][sp][q4] = pack2(d[e] * sc16[e], d[e + 1] * sc16[e + 1]);
          }
      }
      if (MODE == 0 && hf == 0) {
#pragma unroll
        for (int pt = 0; pt < PT; ++pt)
#pragma unroll
          for (int sp = 0; sp < 2; ++sp) ex[(KS + 2 * pt + sp) * 64 + lane] = as_f4(vtx[pt][sp]);
      }
    }
    lds_barrier();  // barrier 2: exchange tiles visible, phase staging no longer read

    // gate operand of this half, loaded while the products and the state scan run
    u32x4 zrow[PS] = {};
    if (MODE == 0 && active) {
      const uint16_t* z_row = zbase + (t < L ? t : t0) * P.z_st;
#pragma unroll
      for (int s = 0; s < PS; ++s) zrow[s] = load_row8(z_row, kidx(s, hh, 0));
    }

    f32x16 yacc[PT] = {};  // y^T tiles: lane = t, elements = p
    if (active) {
      u32x4 scy_o[2];
      u32x4 exv[PT][2];
      const float4* ex = &sh.a[cw][0];
      if (MODE == 0 && hf) {
        // off-diagonal score tile: u in half 0, t in half 1 (entirely causal)
        f32x16 sacc = zero16();
#pragma unroll
        for (int s = 0; s < KS; ++s) sacc = mfma(as_u4(ex[s * 64 + lane]), qrow[s], sacc);
        score_tile(sacc, csf, &sh.cs[cw][0], false, c32, hh, scy_o);
#pragma unroll
        for (int pt = 0; pt < PT; ++pt)
#pragma unroll
          for (int sp = 0; sp < 2; ++sp) exv[pt][sp] = as_u4(ex[(KS + 2 * pt + sp) * 64 + lane]);
        wave_sync();  // exchange reads before this wave's dS overwrites the slot
      }
      // this half's share of dS^T[n][p] = sum_u kr^T[n][u] vs[p][u] (lane = p, elements = n)
      float4* dsl = hf ? &sh.a[cw][0] : &sh.b[cw][0];
#pragma unroll
      for (int nt = 0; nt < NT; ++nt)
#pragma unroll
        for (int pt = 0; pt < PT; ++pt) {
          f32x16 d = mfma(ktx[nt][0], vsy[pt][0], zero16());
          d = mfma(ktx[nt][1], vsy[pt][1], d);
          float4* dst = dsl + (nt * PT + pt) * 256;
#pragma unroll
          for (int g = 0; g < 4; ++g)
            dst[g * 64 + lane] = make_float4(d[4 * g], d[4 * g + 1], d[4 * g + 2], d[4 * g + 3]);
        }
      // y_intra^T[p][t] = (D + delta_t) v[t][p] + sum_{u < t} v^T[p][u] score[t][u]
      if constexpr (MODE == 0) {
        const float coef = skip + delta;
#pragma unroll
        for (int pt = 0; pt < PT; ++pt) {
#pragma unroll
          for (int e = 0; e < 16; ++e) yacc[pt][e] = coef * slot_f(v[2 * pt + (e >> 3)], e & 7);
          if (hf) {
            yacc[pt] = mfma(exv[pt][0], scy_o[0], yacc[pt]);
            yacc[pt] = mfma(exv[pt][1], scy_o[1], yacc[pt]);
          }
          yacc[pt] = mfma(vtx[pt][0], scy_d[0], yacc[pt]);
          yacc[pt] = mfma(vtx[pt][1], scy_d[1], yacc[pt]);
        }
      }
    }
    lds_barrier();  // barrier 3: every dS share in LDS
    pre = {};
    if (kPrefetch && hf == 0 && g0 + CW + cw < c_stop) {
      const int t0n = (g0 + CW + cw) * kChunk;
      load_rows<MODE == 0>(P, pre, qbase, kbase, vbase, t0n, t0n + c32, L, hh);
    }

    // controls and angles of the same half of the next super-chunk
    Ctl nxt = {};
    if (g0 + CW + cw < c_stop) {
      const int tn = (g0 + CW + cw) * kChunk;
      load_ctl(P, nxt, dto, ado, trb, gbase + (pair_on ? pp : 0) * P.g_sr, tn + 32 * hf + c32,
               tn + 32 * hf + seg * RPL, L, tlim);
    }

    // ---------------- state scan over the CW chunks ----------------
    {
      float dec[CW];
#pragma unroll
      for (int j = 0; j < CW; ++j) {
        const float tj = sh.htot[CW + j] + sh.htot[j];
        dec[j] = j < nact ? fast_exp2(tj) : 1.f;
        if (MODE == 1 && j < nact) seg_log2 += tj;
      }
#pragma unroll
      for (int r = 0; r < SPT; ++r) {
        const int f = tid + r * W * 64;
        if (f >= kF4) break;
        float4 s = run[r];
#pragma unroll
        for (int j = 0; j < CW; ++j) {
          if (j < nact) {
            const float4 d0 = sh.b[j][f];
            const float4 d1 = sh.a[j][f];
            if constexpr (MODE == 0) sh.a[j][f] = s;
            s = make_float4(s.x * dec[j] + (d0.x + d1.x), s.y * dec[j] + (d0.y + d1.y),
                            s.z * dec[j] + (d0.z + d1.z), s.w * dec[j] + (d0.w + d1.w));
          }
        }
        run[r] = s;
      }
      if (tid < R) {
        double cr = sh.carry[tid];
        for (int j = 0; j < 2 * nact; ++j) cr += sh.wsum[j][tid];
        sh.carry[tid] = cr - kTwoPiD * floor(cr * (1.0 / kTwoPiD));
      }
    }
    lds_barrier();  // barrier 4: exclusive states in LDS

    // ---------------- inter-chunk term, gate, store ----------------
    if (MODE == 0 && active) {
      const float decay = fast_exp2(csf);
#pragma unroll
      for (int pt = 0; pt < PT; ++pt) {
        f32x16 yi = zero16();
#pragma unroll
        for (int s = 0; s < KS; ++s) {
          // X rows p, K = n: D elements 8*(s&1) .. +7 of tile (s>>1, pt)
          const float4* src = &sh.a[cw][((s >> 1) * PT + pt) * 256];
          const float4 lo = src[(2 * (s & 1)) * 64 + lane];
          const float4 hi = src[(2 * (s & 1) + 1) * 64 + lane];
          u32x4 sx;
          sx[0] = pack2(lo.x, lo.y);
          sx[1] = pack2(lo.z, lo.w);
          sx[2] = pack2(hi.x, hi.y);
          sx[3] = pack2(hi.z, hi.w);
          yi = mfma(sx, qrow[s], yi);
        }
        float yv[16];
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          const float zz = slot_f(zrow[2 * pt + (e >> 3)], e & 7);
          yv[e] = (yacc[pt][e] + yi[e] * decay) * (zz * sigmoid_fast(zz));
        }
        if (t < L) {  // rows in [L, T) are zero-filled after the loop
#pragma unroll
          for (int g = 0; g < 4; ++g) {
            const float y[4] = {yv[4 * g], yv[4 * g + 1], yv[4 * g + 2], yv[4 * g + 3]};
            const int off = obase + t * P.o_st + 32 * pt + 8 * g + 4 * hh;
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
    cur = nxt;
  }
  if constexpr (MODE == 1) {
    // the segment's contribution: state from zero and log2 decay
#pragma unroll
    for (int r = 0; r < SPT; ++r) {
      const int f = threadIdx.x + r * W * 64;
      if (f < kF4) P.seg_state[static_cast<size_t>(rec) * kF4 + f] = run[r];
    }
    if (threadIdx.x == 0) P.seg_decay[rec] = seg_log2;
  } else {
    // rows of this segment in [L, T) (only when lengths < T); they are the same
    // rows in either direction, addressed with the unreversed base and stride
    constexpr int PD = 32 * PT;
    const int row_end = min(c_end * kChunk, T);
    const int o_st = P.rev ? -P.o_st : P.o_st;
    const int obase_fwd = b * P.o_sb + h * P.o_sh;
    for (int e = max(c_begin * kChunk, L) * PD + threadIdx.x; e < row_end * PD; e += W * 64) {
      const int tt = e / PD, p = e - tt * PD;
      const int off = obase_fwd + tt * o_st + p;
      if (P.out_f32)
        static_cast<float*>(P.out)[off] = 0.f;
      else
        static_cast<uint16_t*>(P.out)[off] = 0;
    }
  }
}

// Exclusive scan of the segment state records of each unit: record g's
// contribution dS_g (state from zero, log2 decay T_g) is replaced by the state
// entering segment g,
//   S_0 = 0,  S_{g+1} = S_g 2^{T_g} + dS_g,
// the composition the serial walk applies chunk by chunk. Workgroup
// (unit, slice) takes kScanSlice float4 of the unit's state, so the few units of a
// long sequence still spread over many CUs.
constexpr int kScanSlice = 64;  // one wave per slice (256 float4 per slice: 1 us slower at B1 L7200)

__global__ __launch_bounds__(kScanSlice) void segment_scan_kernel(float4* state, const float* decay, int kf4, int G) {
  const int slices = kf4 / kScanSlice;
  const int unit = blockIdx.x / slices;
  const int f = (blockIdx.x - unit * slices) * kScanSlice + threadIdx.x;
  scan_unit_records(state + static_cast<size_t>(unit) * G * kf4, decay + unit * G, kf4, G, f);
}

// Phase increments of each (unit, chunk): per rotary pair, the fp64 sum over
// the chunk's valid rows of pi * tanh(theta) * dt, each increment formed in
// fp32 exactly as the recurrence forms it (mamba_fused.py:102-109). Lanes of a
// row group take consecutive pairs (one row's angles are contiguous), the
// 256 / rpad row groups interleaved rows; LDS adds the group partials.
__global__ __launch_bounds__(256) void chunk_phase_kernel(const MfmaParams P) {
  __shared__ double part[256];
  const int unit = blockIdx.x / P.NC;
  const int chunk = blockIdx.x - unit * P.NC;
  const int b = unit / P.H;
  const int h = unit - b * P.H;
  const int T = P.T;
  int L = T;
  if (P.lengths != nullptr) {
    const int64_t l = P.lengths[b];
    L = l < 0 ? 0 : (l > T ? T : static_cast<int>(l));
  }
  int rpad = 16;
  while (rpad < P.R) rpad <<= 1;  // R <= 64
  const int r = threadIdx.x & (rpad - 1);
  const int grp = threadIdx.x / rpad;
  const int ngrp = 256 / rpad;
  const int t_begin = chunk * kChunk;
  const int t_end = min(min(t_begin + kChunk, T), L);
  const int roff = P.rev ? max(L - 1, 0) : 0;  // reversed unit: step t reads row L-1-t
  const int dto = b * P.d_sb + h * P.d_sh - roff * P.d_st;
  const float step_bias = P.ctl_raw ? P.dt_bias[h] : 0.f;
  double acc = 0.0;
  if (r < P.R) {
    const int g0 = b * P.g_sb + h * P.g_sh + r * P.g_sr - roff * P.g_st;
    // unrolled so that several rows' loads are in flight before the first use
    for (int t = t_begin + grp; t < t_end; t += ngrp) {
      const float th = P.angles_dtype == TF_FLOAT32 ? static_cast<const float*>(P.angles)[g0 + t * P.g_st]
                                                    : to_f32(static_cast<const bf16_t*>(P.angles)[g0 + t * P.g_st]);
      float dt = ctl_value(P.dt, P.ctl_bf16, dto + t * P.d_st);
      if (P.ctl_raw) dt = control_step(dt, step_bias);
      acc += static_cast<double>(tanh_fast(th) * kPi * dt);
    }
  }
  part[threadIdx.x] = acc;
  __syncthreads();
  if (threadIdx.x < 64) {
    double sum = 0.0;
    if (static_cast<int>(threadIdx.x) < P.R)
      for (int g = 0; g < ngrp; ++g) sum += part[g * rpad + threadIdx.x];
    P.chunk_phase[(static_cast<size_t>(unit) * P.NC + chunk) * 64 + threadIdx.x] = sum;
  }
}

}  // namespace

bool aligned(const void* p, int bytes) { return (reinterpret_cast<uintptr_t>(p) % bytes) == 0; }

bool rows_vectorisable(const void* p, const int64_t* st, int elem_bytes, int vec_bytes) {
  const int64_t m = vec_bytes / elem_bytes;
  return aligned(p, vec_bytes) && st[3] == 1 && st[0] % m == 0 && st[1] % m == 0 && st[2] % m == 0;
}

namespace {

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

}  // namespace

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
  P.adt = a.adt;
  P.dt = a.dt;
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
  P.n_real = static_cast<int>(a.state);
  P.out_f32 = a.out_dtype == TF_FLOAT32;
  P.trap_bf16 = a.trap_dtype == TF_BFLOAT16;
  P.angles_dtype = a.angles_dtype;
  P.units = static_cast<int>(a.batch * a.heads);
  P.G = 1;
  P.SC = static_cast<int>((a.time + kChunk - 1) / kChunk);
  P.NC = P.SC;
  P.seg_state = nullptr;
  P.chunk_phase = nullptr;
  P.seg_decay = nullptr;
  P.phase_fx = nullptr;
  P.lpt = 0;
  P.ctl_raw = a.dt_bias != nullptr;
  P.ctl_bf16 = a.dt_dtype == TF_BFLOAT16;
  P.a_floor = a.a_floor;
  P.dt_bias = a.dt_bias;
  P.qk_norm = a.q_norm != nullptr;
  P.norm_eps = a.norm_eps;
  P.qn_w = a.q_norm;
  P.kn_w = a.k_norm;
  P.rev = a.reverse != 0;
  if (P.rev) {
    P.q_st = -P.q_st, P.k_st = -P.k_st, P.v_st = -P.v_st, P.z_st = -P.z_st, P.o_st = -P.o_st;
    P.g_st = -P.g_st, P.a_st = -P.a_st, P.d_st = -P.d_st, P.r_st = -P.r_st;
  }
  return P;
}

namespace {

// Chunk-parallel plan: with fewer (batch, head) units than half the CUs, each
// unit's time axis is cut into G segments of SC chunks (whole super-chunks) so
// about one workgroup per CU runs. The cost is a phase pre-pass over the
// angles, a second, lighter pass over the inputs (the summary) and a tiny
// scan; a unit walked serially by one workgroup would leave the other CUs idle.
// Scratch layout: states [units][G][kf4] float4, chunk phase sums
// [units][chunks][64] fp64, decays [units][G] fp32, each block 256-byte aligned.
struct SegPlan {
  int G = 1;
  int SC = 0;
  int64_t phase_off = 0, decay_off = 0, bytes = 0;
};

constexpr int64_t kTargetGroups = 256;  // one workgroup per CU (MI355X: 256 CUs)

SegPlan plan_segments(const tf_mamba_args& a, int cw, int kf4) {
  SegPlan p;
  const int64_t units = a.batch * a.heads;
  const int64_t chunks = (a.time + kChunk - 1) / kChunk;
  p.SC = static_cast<int>(chunks);
  if (units <= 0 || chunks <= 0 || units > kTargetGroups / 2) return p;
  int64_t g = kTargetGroups / units;
  int64_t sc = (chunks + g - 1) / g;
  sc = (sc + cw - 1) / cw * cw;
  g = (chunks + sc - 1) / sc;
  if (g < 2) return p;
  p.G = static_cast<int>(g);
  p.SC = static_cast<int>(sc);
  const int64_t recs = units * g;
  auto up = [](int64_t x) { return (x + 255) & ~int64_t(255); };
  p.phase_off = up(recs * kf4 * 16);
  p.decay_off = p.phase_off + up(units * chunks * 64 * 8);
  p.bytes = p.decay_off + up(recs * 4);
  return p;
}

int shape_cw(const tf_mamba_args& a) { return a.state == 128 ? 2 : 4; }

// State dim the kernel runs at: N = 16 runs the N = 32 kernel, its upper 16
// channels zero.
int64_t padded_state(const tf_mamba_args& a) { return a.state < 32 ? 32 : a.state; }

template <int NT, int PT, int CW, bool WIDE>
int launch_modes(MfmaParams P, hipStream_t stream) {
  constexpr int kF4 = NT * PT * 256;
  const int64_t items = static_cast<int64_t>(P.units) * P.G;
  // Work items sharing q/k rows (same batch row and segment) are consecutive;
  // dealing contiguous ranges to the 8 XCDs (workgroups go round-robin) keeps
  // them on one L2.
  P.xcd_per = (items % 8 == 0 && items >= 64) ? static_cast<int>(items / 8) : 0;
  const dim3 grid(static_cast<uint32_t>(items)), block(CW * 128);
  if (P.G > 1) {
    // chunk phase sums -> segment state contributions (seeded with the phase
    // carry) -> scan of the states -> outputs
    hipLaunchKernelGGL(chunk_phase_kernel, dim3(static_cast<uint32_t>(P.units) * P.NC), dim3(256), 0, stream, P);
    if (const int rc = launch_status()) return rc;
    hipLaunchKernelGGL((mamba_mfma_kernel<NT, PT, CW, WIDE, 1>), grid, block, 0, stream, P);
    if (const int rc = launch_status()) return rc;
    static_assert(kF4 % kScanSlice == 0, "state slices");
    hipLaunchKernelGGL(segment_scan_kernel, dim3(static_cast<uint32_t>(P.units) * (kF4 / kScanSlice)),
                       dim3(kScanSlice), 0, stream,
                       P.seg_state, P.seg_decay, kF4, P.G);
    if (const int rc = launch_status()) return rc;
  }
  hipLaunchKernelGGL((mamba_mfma_kernel<NT, PT, CW, WIDE, 0>), grid, block, 0, stream, P);
  return launch_status();
}

template <int NT, int PT, int CW>
int launch_shape(const tf_mamba_args& a, hipStream_t stream) {
  MfmaParams P = make_params(a);
  const SegPlan plan = plan_segments(a, CW, NT * PT * 256);
  if (plan.G > 1 && a.workspace != nullptr && aligned(a.workspace, 256) && a.workspace_bytes >= plan.bytes) {
    char* ws = static_cast<char*>(a.workspace);
    P.G = plan.G;
    P.SC = plan.SC;
    P.seg_state = reinterpret_cast<float4*>(ws);
    P.chunk_phase = reinterpret_cast<double*>(ws + plan.phase_off);
    P.seg_decay = reinterpret_cast<float*>(ws + plan.decay_off);
  }
  // WIDE: R above a quarter of the kernel's state dim (8 NT)
  if (a.rotary > 8 * NT) return launch_modes<NT, PT, CW, true>(P, stream);
  return launch_modes<NT, PT, CW, false>(P, stream);
}

}  // namespace

int64_t mfma_workspace_bytes(const tf_mamba_args& a) {
  if (!mfma_supported(a)) return 0;
  const SegPlan plan = plan_segments(a, shape_cw(a), static_cast<int>((padded_state(a) / 32) * (a.head_dim / 32) * 256));
  return plan.G > 1 ? plan.bytes : 0;
}

bool mfma_supported(const tf_mamba_args& a) {
  if (a.q_dtype != TF_BFLOAT16 || a.k_dtype != TF_BFLOAT16 || a.v_dtype != TF_BFLOAT16 || a.z_dtype != TF_BFLOAT16)
    return false;
  if (a.dt_bias == nullptr) {
    if (a.adt_dtype != TF_FLOAT32 || a.dt_dtype != TF_FLOAT32) return false;
  } else if (a.adt_dtype != a.dt_dtype || (a.dt_dtype != TF_FLOAT32 && a.dt_dtype != TF_BFLOAT16)) {
    return false;
  }
  if (a.trap_dtype != TF_FLOAT32 && a.trap_dtype != TF_BFLOAT16) return false;
  if (a.angles_dtype != TF_FLOAT32 && a.angles_dtype != TF_BFLOAT16) return false;
  if (a.out_dtype != TF_BFLOAT16 && a.out_dtype != TF_FLOAT32) return false;
  if (!(a.state == 16 || a.state == 32 || a.state == 64 || a.state == 128)) return false;
  if (!(a.head_dim == 32 || a.head_dim == 64)) return false;
  if (a.rotary < 0 || a.rotary > a.state / 2) return false;
  // the phase staging area [64 rows][R rounded up to even] lives in a state slot
  if (64 * ((a.rotary + 1) & ~int64_t(1)) > (padded_state(a) / 32) * (a.head_dim / 32) * 1024) return false;
  if (a.batch * a.heads > 0x7fffffff) return false;
  if (!rows_vectorisable(a.q, a.q_stride, 2, 8) || !rows_vectorisable(a.k, a.k_stride, 2, 8) ||
      !rows_vectorisable(a.v, a.v_stride, 2, 8) || !rows_vectorisable(a.z, a.z_stride, 2, 8))
    return false;
  const int ob = a.out_dtype == TF_FLOAT32 ? 4 : 2;
  if (!rows_vectorisable(a.out, a.out_stride, ob, 4 * ob)) return false;
  return offsets_fit(a);
}

// Four chunks (eight waves, two per SIMD) per super-chunk. N=128 keeps two
// chunks (four waves, one per SIMD): its working set needs the 512 registers a
// lone wave gets, and with P=64 its two LDS slots per chunk would not fit four.
// With more (batch, head) units than CUs, N=128, P=64 takes one chunk per
// super-chunk: its 69 KB of LDS lets two workgroups share a CU, so every unit
// runs in one round instead of two (the model's 16 x 32 units: 37.8 -> 34.2 us).
int launch_mfma(const tf_mamba_args& a, hipStream_t stream) {
  const int nt = static_cast<int>(padded_state(a) / 32);
  const int pt = static_cast<int>(a.head_dim / 32);
  if (nt == 1 && pt == 1) return launch_shape<1, 1, 4>(a, stream);
  if (nt == 1 && pt == 2) return launch_shape<1, 2, 4>(a, stream);
  if (nt == 2 && pt == 1) return launch_shape<2, 1, 4>(a, stream);
  if (nt == 2 && pt == 2) return launch_shape<2, 2, 4>(a, stream);
  if (nt == 4 && pt == 1) return launch_shape<4, 1, 2>(a, stream);
  if (nt == 4 && pt == 2) {
    if (a.batch * a.heads > kTargetGroups) return launch_shape<4, 2, 1>(a, stream);
    return launch_shape<4, 2, 2>(a, stream);
  }
  return TF_ERR_SHAPE;
}

}  // namespace tf
