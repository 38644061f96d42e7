// Pipelined fused Mamba-3 SISO recurrence on gfx950 bf16 MFMA (N = P = 64).
//
// Same arithmetic and bf16 rounding points as the reference kernel
// (src/trifusion_l4/mamba_fused.py:72-152). One workgroup of twelve waves
// (three per SIMD) walks one (batch, head) unit chunk by chunk (64 steps). A
// chunk's work is cut into stages that run in the two intervals (A, B) between
// the workgroup barriers of consecutive iterations, so the stages of
// neighbouring chunks overlap:
//
//   stage of chunk c       interval   waves                    lane layout
//   controls               A(c-1)     prologue wave 3          lane = row
//   phase, cos/sin         B(c-1)     prologue waves           lane = (pair, row segment)
//   [B/C norm,] bias, rot. A(c)       output + state waves     lane = (row, 8 channels)
//   state S_{c+1}          B(c)       state waves              one 32x32 tile of S each
//   scores                 A(c+1)     prologue waves 0-2       one 32x32 score tile each
//   skip, inter-chunk      A(c+1)     output waves             one 32x32 tile of y each
//   scores . v, gate       B(c+1)     output waves             the same tile
//
// By role index w: waves 0-3 are output waves (time half th = w >> 1, head-dim
// tile pt = w & 1), waves 4-7 state waves (s = w - 4: state tile nt = s >> 1,
// pt = s & 1) and waves 8-11 prologue waves, so each SIMD holds one of each
// (the unseeded walk runs the prologue role on the first-dispatched hardware
// waves; w and the hardware wave share their SIMD). The fp32 state S
// (64 x 64) lives in the state waves' registers for the whole walk: each holds
// one 32 x 32 tile in MFMA accumulator layout and applies S <- S 2^tot + dS
// once per chunk; there is no scan and no state in LDS other than the bf16
// copies the outputs read.
//
// Chunk-local operands pass through LDS as bf16 rows (rotated q, rotated and
// scaled k, v, decay-scaled v) and are read back either as MFMA row operands
// (8-byte pieces) or transposed with ds_read_b64_tr_b16, which gives each lane
// four consecutive rows of one column: the transposes the contractions over
// time need (v^T, kr^T, vs^T) cost no VALU work.
//
// The rotary phase is kept exactly: each increment tanh(theta) dt / 2 (in
// revolutions) is reduced to [-1/2, 1/2] and converted to 32-bit fixed point,
// whose wrapping integer sums are the phase mod one revolution; v_sin/v_cos
// take revolutions directly.
#include "mfma_tile.h"

namespace tf {

namespace {

// Floats per row of a cos/sin table: 32 pairs x 2 + 2 pad. Rows 4 apart (the
// walk's phase lanes) land 8 banks apart, consecutive rows (the summary's) 2.
constexpr int kTrigStride = 66;

// Fourth word of a raw (unswizzled, stride 0) buffer descriptor on gfx9-family
// parts: 32-bit data format; loads and stores past num_records are dropped.
constexpr int kRawBufferWord3 = 0x00020000;
constexpr int kOutOfRange = static_cast<int>(0x80000000u);  // a lane offset no buffer here reaches
// Cache policy of the output stores: nt (streaming). The walk never reads its
// output back; streaming stores took 0.3-0.4 us off a clip call and 1 us off a
// long-clip call against write-back stores (sc0 sc1 write-through: 3-4 us
// slower). Non-temporal loads of the operand rows were slower and are not used.
constexpr int kStreamStore = 2;

typedef __attribute__((ext_vector_type(4))) short s16x4;
typedef __attribute__((address_space(3))) s16x4 lds_s16x4;

// Element offset of 8-byte unit u (0..15) of row t (0..63) in a [64][64] bf16
// row buffer. Units are XOR-swizzled by the row, so that the access patterns
// each touch 16 distinct units (all 32 banks once) per 16 lanes: row-form
// reads (16 rows, one unit), transposing reads (4 rows x 4 units) and the
// rotary's row writes (rows t and t + 4, units 2 ng (+1) of ng = 0..7: bit 0
// of the swizzle differs between the two rows, so one writes even units and
// the other odd ones).
__device__ __forceinline__ int rb_off(int t, int u) {
  const int swz = ((t & 3) << 2) | ((t >> 2) & 3);
  return t * 64 + ((u ^ swz) << 2);
}

// Row (0..7) of an eight-row block held by lanes 8 j .. 8 j + 7: j / 2 + 4 (j % 2),
// so the two rows of each 16 lanes are four apart (conflict-free row writes).
__device__ __forceinline__ int row8_of_lane(int lane) { return (lane >> 4) + 4 * ((lane >> 3) & 1); }

__device__ __forceinline__ u32x2 rb_read(const uint16_t* buf, int t, int u) {
  return *reinterpret_cast<const u32x2*>(buf + rb_off(t, u));
}

// Row-form MFMA operand of k-step s (contraction over the 64 columns) of row t:
// slots j hold columns kidx(s, hh, j).
__device__ __forceinline__ u32x4 row_operand(const uint16_t* buf, int t, int s, int hh) {
  const int u = 8 * (s >> 1) + 4 * (s & 1) + hh;
  const u32x2 lo = rb_read(buf, t, u), hi = rb_read(buf, t, u + 2);
  return u32x4{lo[0], lo[1], hi[0], hi[1]};
}

// Transposed MFMA operand of k-step s (contraction over the 64 rows) for the
// 32 columns of column tile `tile`: lane (c32, hh) receives column
// 32 tile + c32 at rows kidx(s, hh, j). Within each 16-lane group the source
// lane i = 4k + c reads row r0 + k, unit u0 + c, and the transposing read
// hands output lane j column 4 u0 + j of rows r0 .. r0 + 3.
__device__ __forceinline__ u32x4 tr_operand(const uint16_t* buf, int tile, int s, int lane) {
  const int g = lane >> 4;
  const int i = lane & 15;
  const int r0 = 32 * (s >> 1) + 16 * (s & 1) + 4 * (g >> 1) + (i >> 2);
  const int u = 8 * tile + 4 * (g & 1) + (i & 3);
  const uint16_t* p0 = buf + rb_off(r0, u);
  const uint16_t* p1 = buf + rb_off(r0 + 8, u);
  const s16x4 a = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(p0));
  const s16x4 b = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(p1));
  const u32x2 ua = __builtin_bit_cast(u32x2, a), ub = __builtin_bit_cast(u32x2, b);
  return u32x4{ua[0], ua[1], ub[0], ub[1]};
}

// As tr_operand, over the 32 rows of one time half (k-steps s = 0, 1 of rows
// 32 half .. 32 half + 31).
__device__ __forceinline__ u32x4 tr_operand_half(const uint16_t* buf, int tile, int half, int s, int lane) {
  return tr_operand(buf, tile, 2 * half + s, lane);
}

__device__ __forceinline__ void rb_write16(uint16_t* buf, int t, int u, const u32x4& x) {
  *reinterpret_cast<u32x2*>(buf + rb_off(t, u)) = u32x2{x[0], x[1]};
  *reinterpret_cast<u32x2*>(buf + rb_off(t, u + 1)) = u32x2{x[2], x[3]};
}

struct PipeSmem {
  uint16_t qr[2][64 * 64];  // bf16(rot(q + qb))
  uint16_t kr[2][64 * 64];  // bf16(rot(k + kb) * s)
  uint16_t v[2][64 * 64];   // v (0 past the valid length)
  uint16_t vs[2][64 * 64];  // bf16(v * 2^(tot - cs))
  float trig[2][64 * kTrigStride];  // [row][pair] (cos, sin)
  u32x4 sb[3][4][2][64];     // bf16 S_c (c mod 3): tiles (nt, pt), k-step halves, in MFMA operand order
  u32x4 score[2][3][2][64];  // bf16 score tiles (0,0), (1,0), (1,1), k-steps, in operand order
  float dt[3][64];
  float sc[3][64];   // trapezoid scale s_t of the keys
  float cs[3][64];   // inclusive log2 decay within the chunk
  float wv[3][64];   // 2^(tot - cs_t)
  float gam[3][64];  // dt_t sigmoid(trap_t)
  float skip[3][64];  // (q + qb).(k + kb) of each row
  float tot[3][4];    // [0]: the chunk's total log2 decay
  float nw[2][64];    // fused B/C norm weights of q and k
};

struct PipeCtl {
  float dt, dn, adt, tr, tn;
};

// Fused B/C RMSNorm (mamba.py:56-57, kernels/__init__.py:10-12) of a row of 64
// bf16 channels held as 8 channels by each of 8 neighbouring lanes:
// x -> bf16(x rsqrt(mean(x^2) + eps) w), the rounding of the separate norm's
// bf16 output. w8: the lane's 8 weights (LDS). The walk and the summary pass
// both call this, so a row is normalised to the same bits in either.
__device__ __forceinline__ u32x4 norm_row8(const u32x4& x, const float* w8, float eps) {
  float ss = 0.f;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    ss = __builtin_fmaf(lo_f(x[j]), lo_f(x[j]), ss);
    ss = __builtin_fmaf(hi_f(x[j]), hi_f(x[j]), ss);
  }
  const float r = rsqrtf(group8_sum(ss) / 64.f + eps);
  const float4 wa = reinterpret_cast<const float4*>(w8)[0], wb = reinterpret_cast<const float4*>(w8)[1];
  const float w[8] = {wa.x, wa.y, wa.z, wa.w, wb.x, wb.y, wb.z, wb.w};
  u32x4 y;
#pragma unroll
  for (int j = 0; j < 4; ++j) y[j] = pack2(lo_f(x[j]) * r * w[2 * j], hi_f(x[j]) * r * w[2 * j + 1]);
  return y;
}

template <bool BF16>
__device__ __forceinline__ float load_elem(const void* base, int i) {
  if constexpr (BF16)
    return bf16_to_f32(static_cast<const uint16_t*>(base)[i]);
  else
    return static_cast<const float*>(base)[i];
}

// Controls of row t and its halo step t + 1 (raw values when P.ctl_raw). Rows
// are clamped to ones that exist and masked where used, so no load sits behind
// a branch and the loads stay in flight until then.
template <bool CTL16, bool TRAP16>
__device__ __forceinline__ PipeCtl load_pipe_ctl(const MfmaParams& P, int dto, int ado, int trb, int t, int L,
                                                 int tlim) {
  const int tc = min(t, L - 1);
  const int tn = min(t + 1, tlim - 1);
  PipeCtl c;
  c.dt = load_elem<CTL16>(P.dt, dto + tc * P.d_st);
  c.dn = load_elem<CTL16>(P.dt, dto + tn * P.d_st);
  c.adt = load_elem<CTL16>(P.adt, ado + tc * P.a_st);
  c.tr = load_elem<TRAP16>(P.trap, trb + tc * P.r_st);
  c.tn = load_elem<TRAP16>(P.trap, trb + tn * P.r_st);
  return c;
}

// Phase lanes: lane = pi * (64 / RPW) + sg takes pair s * RPW + pi over the
// RPW rows sg * RPW .. sg * RPW + RPW - 1 of the chunk, so the segments of one
// pair are consecutive lanes (a DPP scan). Lanes of pairs >= R read pair 0's
// column and are never used.
template <int RPW, bool ANG16>
__device__ __forceinline__ void load_pipe_angles(const MfmaParams& P, float (&th)[RPW], int gbase, int pair,
                                                 int row0, int L) {
  const int col = gbase + (pair < P.R ? pair : 0) * P.g_sr;
#pragma unroll
  for (int i = 0; i < RPW; ++i) th[i] = load_elem<ANG16>(P.angles, col + min(row0 + i, L - 1) * P.g_st);
}

// Segment summaries a thread of the seeded walk loads per round trip.
constexpr int kSeedBatch = 8;

// First chunk of segment g of a unit's time axis: the ceil(T / 64) chunks
// split as evenly as G segments allow, the first (chunks mod G) segments one
// chunk longer. A later segment's walk first scans the summaries of every
// segment before it, so the segments that scan the most walk the fewest chunks.
__device__ __forceinline__ int seg_start(const MfmaParams& P, int g) {
  const int chunks = (P.T + kChunk - 1) / kChunk;
  const int base = chunks / P.G, extra = chunks % P.G;
  return g * base + min(g, extra);
}

// Raw 16-byte row pieces of the wave's eight channels (lane = row).
struct PipeRows {
  u32x4 q, k, v;
};

// Work item of workgroup blockIdx.x: (batch row, segment, head). The heads of
// one batch row and segment read the same q/k rows, so they are consecutive
// items, and items are dealt to the 8 XCDs in contiguous ranges so that those
// heads share an L2. A segment's state record is [unit][segment].
struct PipeItem {
  int b, h, seg, unit, rec;
};

__device__ __forceinline__ PipeItem pipe_item(const MfmaParams& P) {
  const int item = P.xcd_per > 0 ? (blockIdx.x & 7) * P.xcd_per + (blockIdx.x >> 3) : static_cast<int>(blockIdx.x);
  const int bseg = item / P.H;
  PipeItem it;
  it.h = item - bseg * P.H;
  it.b = bseg / P.G;
  it.seg = bseg - it.b * P.G;
  it.unit = it.b * P.H + it.h;
  it.rec = it.unit * P.G + it.seg;
  return it;
}

// Work item of an unsegmented varlen walk with P.lpt set (B <= 64, B % 8 ==
// 0, more units than CUs): the batch rows ranked by chunk count (more first,
// then lower index), rank r dealt to XCD r mod 8 in snake order (r = 8 k + x,
// or 8 k + 7 - x on odd rounds k), and each XCD's rows taken in rank order,
// all heads of a row together. The longest units take the first CU slots and
// the short ones fill in behind them. Every wave ranks the rows itself (lane
// = batch row), so the result is wave-uniform with no exchange.
__device__ __forceinline__ PipeItem pipe_item_lpt(const MfmaParams& P, int lane) {
  const int x = static_cast<int>(blockIdx.x & 7), pos = static_cast<int>(blockIdx.x >> 3);
  const int k = pos / P.H;
  PipeItem it;
  it.h = pos - k * P.H;
  const int r = 8 * k + ((k & 1) ? 7 - x : x);
  const int B = P.units / P.H;
  int c = -1;  // chunk count of batch row `lane`
  if (lane < B) {
    const int64_t l = P.lengths[lane];
    c = static_cast<int>(((l < 0 ? 0 : (l > P.T ? P.T : l)) + kChunk - 1) / kChunk);
  }
  int rank = 0;
  for (int u = 0; u < B; ++u) {
    const int cu = __builtin_amdgcn_readlane(c, u);
    rank += (cu > c || (cu == c && u < lane)) ? 1 : 0;
  }
  const uint64_t hit = __ballot(lane < B && rank == r);
  it.b = __builtin_amdgcn_readfirstlane(static_cast<int>(__builtin_ctzll(hit)));
  it.seg = 0;
  it.unit = it.b * P.H + it.h;
  it.rec = it.unit;
  return it;
}

// Fixed-point phase increment of one (row, pair): pi tanh(theta) dt radians
// (mamba_fused.py:102-109) = tanh(theta) dt / 2 revolutions, reduced to
// [-1/2, 1/2] and scaled by 2^32. A row without a step (dt = 0) adds 0.
__device__ __forceinline__ uint32_t phase_inc(float th, float dt) {
  float om = tanh_fast(th) * dt * 0.5f;
  om -= rintf(om);
  const float x = fminf(om * 4294967296.f, 2147483520.f);
  return static_cast<uint32_t>(static_cast<int>(x));
}

// (cos, sin) of a fixed-point phase (2^-32 revolutions): v_cos/v_sin take revolutions.
__device__ __forceinline__ float2 phase_trig(uint32_t ph) {
  const float rev = static_cast<float>(static_cast<int>(ph)) * 2.3283064365386963e-10f;
  return make_float2(__builtin_amdgcn_cosf(rev), __builtin_amdgcn_sinf(rev));
}

// Rows (2 rp, 2 rp + 1) and (2 rp + 2, 2 rp + 3) of a state record, the rotary
// pairs rp and rp + 1, turned by phases ph (the key rotation of key_pair,
// applied to the rows kr contributes to); pairs >= R are left as they are.
__device__ __forceinline__ float4 turn_rows(const float4& d, uint2 ph, int rp, int R) {
  float4 o = d;
  if (rp < R) {
    const float2 a = phase_trig(ph.x);
    o.x = __builtin_fmaf(d.x, a.x, -(d.y * a.y));
    o.y = __builtin_fmaf(d.x, a.y, d.y * a.x);
  }
  if (rp + 1 < R) {
    const float2 a = phase_trig(ph.y);
    o.z = __builtin_fmaf(d.z, a.x, -(d.w * a.y));
    o.w = __builtin_fmaf(d.z, a.y, d.w * a.x);
  }
  return o;
}

// Controls of one chunk, one wave, lane = row (mamba_fused.py:96-101, 139-142):
// step, key scale, inclusive log2 decay, 2^(tot - cs), dt sigmoid(trap), and
// the chunk's total log2 decay (every lane).
struct RowControls {
  float dt, sc, cs, wv, gam, tot;
};

__device__ __forceinline__ RowControls row_controls(const MfmaParams& P, const PipeCtl& raw, bool valid, bool next,
                                                    float step_bias) {
  float dtv = raw.dt, dnv = raw.dn, adv = raw.adt;
  if (P.ctl_raw) {
    // step and decay from the raw columns (primitives.py:209-214)
    dtv = control_step(dtv, step_bias);
    dnv = control_step(dnv, step_bias);
    adv = control_decay(adv, dtv, P.a_floor);
  }
  // rows without a step keep dt = adt = 0, and a missing halo step loads 0
  dtv = valid ? dtv : 0.f;
  adv = valid ? adv : 0.f;
  dnv = next ? dnv : 0.f;
  const float trv = valid ? raw.tr : 0.f;
  const float tnv = next ? raw.tn : 0.f;
  RowControls r;
  r.dt = dtv;
  r.gam = dtv * sigmoid_fast(trv);
  r.sc = __builtin_fmaf(dnv, 1.f - sigmoid_fast(tnv), r.gam);
  r.cs = wave_scan_dpp(adv * kLog2e);
  r.tot = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, r.cs), 63));
  r.wv = fast_exp2(r.tot - r.cs);
  return r;
}

// bf16 pair of a key rotated by (cv, sv) and scaled by the trapezoid scale
// (mamba_fused.py:126-131), and of a value scaled by 2^(tot - cs) (:151).
// The fused multiply-adds are spelled out, so that every kernel rounds a key
// the same way whatever the compiler would contract in its context.
__device__ __forceinline__ uint32_t key_pair(float k0, float k1, float cv, float sv, float scl) {
  return pack2(__builtin_fmaf(k0, cv, -(k1 * sv)) * scl, __builtin_fmaf(k0, sv, k1 * cv) * scl);
}
__device__ __forceinline__ uint32_t scaled_pair(uint32_t vw, float wvt) {
  return pack2(lo_f(vw) * wvt, hi_f(vw) * wvt);
}

// Walks the unit (or, SEEDED with P.G > 1, one time segment of it, from the
// state and phase entering the segment) and writes the outputs.
template <int RPW, bool CTL16, bool TRAP16, bool ANG16, bool OUT32, bool SEEDED>
__global__ __launch_bounds__(768) void mamba_pipe_kernel(const MfmaParams P) {
  __shared__ PipeSmem sh;
  // Role index w of hardware wave hw. Unseeded, the prologue role (w 8-11)
  // carries the start's longest chain (chunk c0's controls and phase, behind
  // its loads), so it runs on the first waves dispatched (hw 0-3), which
  // start ~1.7 k cycles before the last. Seeded, the segment scan on w 0-7 is
  // the longer chain, and w = hw. Either way w % 4 == hw % 4 (same SIMD).
  const int hw = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
  const int w = SEEDED ? hw : (hw < 4 ? hw + 8 : hw - 4);
  const int lane = static_cast<int>(threadIdx.x & 63);
  const int c32 = lane & 31;
  const int hh = lane >> 5;
  const bool out_wave = w < 4;
  const bool state_wave = w >= 4 && w < 8;
  const int s_idx = w - 4;  // state wave index (state waves)
  const int p_idx = w - 8;  // prologue wave index (prologue waves)
  const PipeItem it = (!SEEDED && P.lpt) ? pipe_item_lpt(P, lane) : pipe_item(P);
  const int b = it.b, h = it.h, seg = it.seg, unit = it.unit;
  const int qh = h / P.group;
  const int T = P.T;
  const int R = P.R;
  int L = T;
  if (P.lengths != nullptr) {
    const int64_t l = P.lengths[b];
    L = l < 0 ? 0 : (l > T ? T : static_cast<int>(l));
  }
  const int nvalid = (L + kChunk - 1) / kChunk;
  // the segment's chunks [c0, c1) of the valid prefix
  const int c0 = min(seg_start(P, seg), nvalid);
  const int c1 = min(seg_start(P, seg + 1), nvalid);
  const int tlim = P.rev ? L : T;
  const int roff = P.rev ? max(L - 1, 0) : 0;
  const uint16_t* qbase = P.q + b * P.q_sb + qh * P.q_sh - roff * P.q_st;
  const uint16_t* kbase = P.k + b * P.k_sb + qh * P.k_sh - roff * P.k_st;
  const uint16_t* vbase = P.v + b * P.v_sb + h * P.v_sh - roff * P.v_st;
  const uint16_t* zbase = P.z + b * P.z_sb + h * P.z_sh - roff * P.z_st;
  const int dto = b * P.d_sb + h * P.d_sh - roff * P.d_st;
  const int ado = b * P.a_sb + h * P.a_sh - roff * P.a_st;
  const int trb = b * P.r_sb + h * P.r_sh - roff * P.r_st;
  const int gbase = b * P.g_sb + h * P.g_sh - roff * P.g_st;
  const float step_bias = P.ctl_raw ? P.dt_bias[h] : 0.f;
  const float skip_d = P.d[h];

  if (c1 > c0) {
    constexpr int NSEG = 64 / RPW;  // row segments per pair
    const int pi = lane / NSEG;
    const int sg = lane & (NSEG - 1);
    const int pair = p_idx * RPW + pi;                // phase pair of a prologue wave's lane
    const bool phase_wave = w >= 8 && p_idx * RPW < R;  // wave-uniform

    // rotary tasks of the output and state waves: row rrow of the chunk,
    // channel group ng; eight rows per wave (output waves rows 0-31, state
    // waves rows 32-63), a row's eight channel groups on eight neighbouring
    // lanes, so a wave's row load is eight whole 128-byte rows and a row's
    // reductions (the B/C norms, the skip term) stay within its lanes
    const int rrow = 8 * (state_wave ? 4 + s_idx : w) + row8_of_lane(lane);
    const int ng = lane & 7;
    auto load_rows = [&](int c) {
      const int t = min(c * kChunk + rrow, L - 1);
      PipeRows r;
      r.q = *reinterpret_cast<const u32x4*>(qbase + t * P.q_st + 8 * ng);
      r.k = *reinterpret_cast<const u32x4*>(kbase + t * P.k_st + 8 * ng);
      r.v = *reinterpret_cast<const u32x4*>(vbase + t * P.v_st + 8 * ng);
      return r;
    };

    // controls of chunk c (state wave 3, lane = row)
    auto controls = [&](const PipeCtl& raw, int c) {
      const int t = c * kChunk + lane;
      const RowControls rc = row_controls(P, raw, t < L, t + 1 < tlim, step_bias);
      const int cr = c % 3;
      sh.dt[cr][lane] = rc.dt;
      sh.sc[cr][lane] = rc.sc;
      sh.cs[cr][lane] = rc.cs;
      sh.wv[cr][lane] = rc.wv;
      sh.gam[cr][lane] = rc.gam;
      if (lane == 0) sh.tot[cr][0] = rc.tot;
    };

    // rotary phase and cos/sin of chunk c (phase waves)
    uint32_t carry = 0;  // phase entering the chunk, pair `pair`, 2^-32 revolutions
    if (SEEDED && phase_wave) {
      // a segment's walk starts from the phase of the segments before it: the
      // wrapping sum of their fixed-point sums (the same integers the serial
      // walk adds), lanes of a pair splitting the segments
      uint32_t part = 0;
      if (pair < R)
        for (int g = sg; g < seg; g += NSEG) part += P.phase_fx[(static_cast<size_t>(unit) * P.G + g) * 32 + pair];
      const uint32_t incl = group_scan_dpp<NSEG>(part, lane);
#pragma unroll
      for (int j = 0; j < RPW; ++j) {
        const uint32_t tj = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(incl), NSEG * j + NSEG - 1));
        carry = pi == j ? tj : carry;
      }
    }
    auto phase_steps = [&](const float (&th)[RPW], const float (&dts)[RPW], int c) {
      uint32_t loc[RPW];
      uint32_t run = 0;
#pragma unroll
      for (int i = 0; i < RPW; ++i) {
        run += phase_inc(th[i], dts[i]);
        loc[i] = run;
      }
      const uint32_t incl = group_scan_dpp<NSEG>(run, lane);  // over the segments of the pair
      const uint32_t base = carry + (incl - run);
      // the chunk's sum for the pair: the last segment's inclusive sum
      uint32_t total = 0;
#pragma unroll
      for (int j = 0; j < RPW; ++j) {
        const uint32_t tj = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(incl), NSEG * j + NSEG - 1));
        total = pi == j ? tj : total;
      }
      carry += total;
      if (pair < R) {
        float* tg = &sh.trig[c & 1][0];
#pragma unroll
        for (int i = 0; i < RPW; ++i)
          *reinterpret_cast<float2*>(tg + (sg * RPW + i) * kTrigStride + 2 * pair) = phase_trig(base + loc[i]);
      }
    };
    auto phase = [&](const float (&th)[RPW], int c) {
      const int cr = c % 3;
      float dts[RPW];
#pragma unroll
      for (int i = 0; i < RPW; ++i) dts[i] = sh.dt[cr][sg * RPW + i];
      phase_steps(th, dts, c);
    };

    // biases of the wave's eight channels, wave-uniform, kept for the whole walk
    float qbv[8], kbv[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      qbv[j] = P.qb[h * 64 + 8 * ng + j];
      kbv[j] = P.kb[h * 64 + 8 * ng + j];
    }

    // bias, rotation, scaling and bf16 rounding of chunk c's rows (lane = row
    // rrow, channels 8 ng .. 8 ng + 7; mamba_fused.py:112-135, 151), after the
    // fused B/C RMSNorm when P.qk_norm (mamba.py:56-57: x -> bf16(x rsqrt(
    // mean(x^2) + eps) w), the separate norm's output rounding). One
    // branch-free form for every lane: pairs 4 ng + j >= R turn by the
    // identity, x * 1 - y * 0 being x exactly.
    auto rotary = [&](const PipeRows& in, int c) {
      const int cb = c & 1, cr = c % 3;
      const bool valid = c * kChunk + rrow < L;
      const float scl = sh.sc[cr][rrow];
      const float wvt = sh.wv[cr][rrow];
      u32x4 qin = in.q, kin = in.k;
      if (P.qk_norm) {
        qin = norm_row8(qin, &sh.nw[0][8 * ng], P.norm_eps);
        kin = norm_row8(kin, &sh.nw[1][8 * ng], P.norm_eps);
      }
      u32x4 qo, ko, vo, vso;
      float part = 0.f;
      const float2* tg = reinterpret_cast<const float2*>(&sh.trig[cb][rrow * kTrigStride + 8 * ng]);
      const float2 t0 = tg[0], t1 = tg[1], t2 = tg[2], t3 = tg[3];
      const float cosv[4] = {t0.x, t1.x, t2.x, t3.x}, sinv[4] = {t0.y, t1.y, t2.y, t3.y};
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const bool on = 4 * ng + j < R;
        const float cv = on ? cosv[j] : 1.f, sv = on ? sinv[j] : 0.f;
        const float q0 = lo_f(qin[j]) + qbv[2 * j], q1 = hi_f(qin[j]) + qbv[2 * j + 1];
        const float k0 = lo_f(kin[j]) + kbv[2 * j], k1 = hi_f(kin[j]) + kbv[2 * j + 1];
        part += q0 * k0 + q1 * k1;
        qo[j] = pack2(q0 * cv - q1 * sv, q0 * sv + q1 * cv);
        ko[j] = key_pair(k0, k1, cv, sv, scl);
      }
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const uint32_t vw = valid ? in.v[j] : 0u;
        vo[j] = vw;
        vso[j] = scaled_pair(vw, wvt);
      }
      rb_write16(sh.qr[cb], rrow, 2 * ng, qo);
      rb_write16(sh.kr[cb], rrow, 2 * ng, ko);
      rb_write16(sh.v[cb], rrow, 2 * ng, vo);
      rb_write16(sh.vs[cb], rrow, 2 * ng, vso);
      part = group8_sum(part);
      if (ng == 0) sh.skip[cr][rrow] = part;
    };

    // Each role runs its own copy of the walk, with the same two barriers per
    // iteration, and issues its global loads (and, output waves, its stores)
    // unconditionally: rows clamped to ones that exist, stores past the length
    // dropped by the buffer's range check. So the wait the compiler places
    // before each use counts exactly the role's own younger memory operations
    // and never waits for one issued later than the one it needs.
    // Loads ahead of use: rows and z of chunk c at A(c-1), controls at A(c-2),
    // angles at the start of A(c).
    float th[RPW];
#pragma unroll
    for (int i = 0; i < RPW; ++i) th[i] = 0.f;
    PipeRows rows = {};
    PipeCtl ctl_next = {};
    // The start's loads, all issued before any of them is used (a wave's loads
    // complete in order): the prologue waves' controls, angles and steps of
    // chunk c0 (every prologue wave loads the controls rows, wave 11 uses
    // them, so their count in each wave's outstanding loads is the same on
    // every path), then the rows of the output and state waves, then a
    // seeded segment's summaries.
    PipeCtl ctl0 = {};
    // controls are formed by prologue wave 3 (lane = row); the other prologue
    // waves issue the same loads (so every wave of the role counts the same
    // outstanding operations) at one row for all lanes: one cache line per
    // load instead of 32
    const int ctl_lane = p_idx == 3 ? lane : 0;
    float dts[RPW];
    if (w >= 8) {
      ctl0 = load_pipe_ctl<CTL16, TRAP16>(P, dto, ado, trb, c0 * kChunk + ctl_lane, L, tlim);
      ctl_next = load_pipe_ctl<CTL16, TRAP16>(P, dto, ado, trb, (c0 + 1) * kChunk + ctl_lane, L, tlim);
      load_pipe_angles<RPW, ANG16>(P, th, gbase, pair, c0 * kChunk + sg * RPW, L);
      // chunk c0's steps for the phase, read here rather than from the
      // controls' LDS rows, so that the phase does not wait for a barrier
#pragma unroll
      for (int i = 0; i < RPW; ++i)
        dts[i] = load_elem<CTL16>(P.dt, dto + min(c0 * kChunk + sg * RPW + i, L - 1) * P.d_st);
    }
    if (w < 8) rows = load_rows(c0);
    // fused B/C norm weights, read by the rotary from the first chunk on
    if (w < 2 && P.qk_norm) sh.nw[w][lane] = (w == 0 ? P.qn_w : P.kn_w)[lane];
    // A seeded segment's entering state: the segment scan of the unit's
    // summaries of the segments before it, S <- S 2^dec_g + turn_g(summary_g)
    // for g < seg, float4 f = 64 w + lane and 64 w + lane + 512 of the record
    // layout on waves 0-7 (the prologue waves go straight to the chunk-0
    // controls and phase), left in the second chunk's qr/kr buffers (tiles
    // 0-1, 2-3) for the state waves. Summary g is formed in segment g's phase
    // frame (phase 0 at its start); turn_g rotates its rotary row pairs by the
    // phase entering the segment, the wrapping sum of the earlier segments'
    // phase sums (kr of the unit's frame is that rotation of kr of the
    // segment's frame). Segment 0 starts at phase 0 and is used as it is.
    [[maybe_unused]] float4* seed_lds[2] = {reinterpret_cast<float4*>(sh.qr[(c0 + 1) & 1]),
                                            reinterpret_cast<float4*>(sh.kr[(c0 + 1) & 1])};
    if (SEEDED && w < 8) {
      const int f0 = 64 * w + lane, f1 = f0 + 512;
      const float4* sums = P.seg_state + static_cast<size_t>(unit) * P.G * 1024;
      const float* decs = P.seg_decay + unit * P.G;
      const uint2* phs = reinterpret_cast<const uint2*>(P.phase_fx + static_cast<size_t>(unit) * P.G * 32);
      // float4 f holds rows 32 (f >> 9) + 8 ((f >> 6) & 3) + 4 ((f >> 5) & 1)
      // + 0..3 of the record's S^T (the 32 x 32 tile layout): rotary pairs
      // rp(f) and rp(f) + 1
      const int rp0 = 16 * (f0 >> 9) + 4 * ((f0 >> 6) & 3) + 2 * ((f0 >> 5) & 1);
      const int rp1 = 16 * (f1 >> 9) + 4 * ((f1 >> 6) & 3) + 2 * ((f1 >> 5) & 1);
      // only pairs < R turn: the second float4 (rows >= 32, pairs >= 16) never
      // does when R <= 16 (RPW 4)
      const bool turn0 = rp0 < R;
      const bool turn1 = RPW > 4 && rp1 < R;
      float4 run0 = make_float4(0.f, 0.f, 0.f, 0.f), run1 = run0;
      uint2 ph0 = make_uint2(0u, 0u), ph1 = ph0;  // phase entering segment g, pairs rp, rp + 1
      for (int g0 = 0; g0 < seg; g0 += kSeedBatch) {
        float4 d0[kSeedBatch], d1[kSeedBatch];
        uint2 s0[kSeedBatch], s1[kSeedBatch];
        float m[kSeedBatch];
#pragma unroll
        for (int j = 0; j < kSeedBatch; ++j) {
          if (g0 + j < seg) {
            d0[j] = sums[static_cast<size_t>(g0 + j) * 1024 + f0];
            if (turn0) s0[j] = phs[(g0 + j) * 16 + rp0 / 2];
            d1[j] = sums[static_cast<size_t>(g0 + j) * 1024 + f1];
            if (turn1) s1[j] = phs[(g0 + j) * 16 + rp1 / 2];
            m[j] = fast_exp2(decs[g0 + j]);
          }
        }
#pragma unroll
        for (int j = 0; j < kSeedBatch; ++j) {
          if (g0 + j < seg) {
            if (turn0) {
              if (g0 + j > 0) d0[j] = turn_rows(d0[j], ph0, rp0, R);
              ph0 = make_uint2(ph0.x + s0[j].x, ph0.y + s0[j].y);
            }
            if (turn1) {
              if (g0 + j > 0) d1[j] = turn_rows(d1[j], ph1, rp1, R);
              ph1 = make_uint2(ph1.x + s1[j].x, ph1.y + s1[j].y);
            }
            run0 = state_step(run0, m[j], d0[j]);
            run1 = state_step(run1, m[j], d1[j]);
          }
        }
      }
      seed_lds[0][f0] = run0;
      seed_lds[1][f0] = run1;
    }
    if (w >= 8) {
#pragma unroll
      for (int i = 0; i < RPW; ++i) {
        float d = dts[i];
        if (P.ctl_raw) d = control_step(d, step_bias);
        dts[i] = c0 * kChunk + sg * RPW + i < L ? d : 0.f;
      }
      if (w == 11) controls(ctl0, c0);
      if (phase_wave) phase_steps(th, dts, c0);
    }
    lds_barrier();

    if (out_wave) {
      const int th_o = w >> 1, opt = w & 1;
      // the unit's valid output rows as one buffer: memory row r (r = t, or
      // L - 1 - t reversed) at element r * o_row from memory row 0; its size
      // ends with row L - 1, so any row t >= L is out of range
      const int o_row = P.rev ? -P.o_st : P.o_st;
      constexpr int esz = OUT32 ? 4 : 2;
      const __amdgpu_buffer_rsrc_t out_rsrc = __builtin_amdgcn_make_buffer_rsrc(
          static_cast<char*>(P.out) + static_cast<int64_t>(b * P.o_sb + h * P.o_sh) * esz, static_cast<short>(0),
          ((L - 1) * o_row + 64) * esz, kRawBufferWord3);
      // gate rows of chunk c (lane = row 32 th + c32 of the chunk, the tile's
      // columns), loaded at A(c) and turned into silu factors at A(c + 1)
      // (lane c32 + 32 hh holds 32 contiguous bytes of its row: columns
      // 32 opt + 16 hh .. + 15; the gate stage trades halves with lane ^ 32)
      auto load_z = [&](int c, u32x4 (&zr)[2]) {
        const int t = min(c * kChunk + 32 * th_o + c32, L - 1);
        const uint16_t* zrow = zbase + t * P.z_st + 32 * opt + 16 * hh;
        zr[0] = *reinterpret_cast<const u32x4*>(zrow);
        zr[1] = *reinterpret_cast<const u32x4*>(zrow + 8);
      };
      // rows (above), z, then stores: the order of every later iteration
      __builtin_amdgcn_sched_barrier(0);
      u32x4 zr[2];
      load_z(c0, zr);
      __builtin_amdgcn_sched_barrier(0);
      // dropped stores, so the walk starts with the same outstanding
      // operations (rows, z, stores) as every later iteration
#pragma unroll
      for (int g = 0; g < (OUT32 ? 4 : 2); ++g)
        __builtin_amdgcn_raw_buffer_store_b128(u32x4{0u, 0u, 0u, 0u}, out_rsrc, kOutOfRange, 0, kStreamStore);
      float gate[16];           // silu(z) of the chunk being finished (mamba_fused.py:148)
      f32x16 ybase = zero16();  // skip and inter-chunk terms of the chunk being finished
#pragma unroll
      for (int e = 0; e < 16; ++e) gate[e] = 0.f;
      for (int i = c0; i <= c1; ++i) {
        // ---------------- interval A(i) ----------------
        if (i > c0) {
          // silu factors of chunk i - 1 from its gate rows (loaded at A(i - 1))
          // columns 8 g + 4 hh .. + 3 of the tile layout: hh = 0 keeps its
          // g = 0, 1 pieces and takes g = 2, 3 from lane ^ 32, hh = 1 the
          // reverse. v_permlane32_swap(a, b) trades a's upper 32 lanes with
          // b's lower 32, so one swap per word pair does it in registers.
          u32x2 zt[4];
#pragma unroll
          for (int k = 0; k < 2; ++k) {
#pragma unroll
            for (int m = 0; m < 2; ++m) {
              const auto x = __builtin_amdgcn_permlane32_swap(zr[k][m], zr[k][m + 2], false, false);
              zt[k][m] = x[0];
              zt[k + 2][m] = x[1];
            }
          }
#pragma unroll
          for (int g = 0; g < 4; ++g) {
#pragma unroll
            for (int q = 0; q < 4; ++q) {
              const uint32_t zw = zt[g][q >> 1];
              const float zz = (q & 1) ? hi_f(zw) : lo_f(zw);
              gate[4 * g + q] = zz * sigmoid_fast(zz);
            }
          }
          // computed here, in interval A: left to itself the compiler sinks
          // this next to its use in B, which keeps the old gate rows live past
          // the next load_z and adds a copy that waits for those loads
#pragma unroll
          for (int e = 0; e < 16; ++e) asm volatile("" : "+v"(gate[e]));
        }
        load_z(i, zr);
        // rows 0-31 of chunk i (the state waves take rows 32-63)
        if (i < c1) rotary(rows, i);
        rows = load_rows(i + 1);
        if (i > c0) {
          // chunk c = i - 1, tile (th, pt) of y^T[p][t]: (D + gamma (q + qb).(k + kb)) v
          // (mamba_fused.py:124, 147) + 2^cs qr . bf16(S_c)^T (mamba_fused.py:143)
          const int c = i - 1;
          const int cb = c & 1, cr = c % 3;
          const int tl = 32 * th_o + c32;
          u32x4 sx[4], qy[4];
          u32x2 vv[4];
#pragma unroll
          for (int s = 0; s < 4; ++s) {
            sx[s] = sh.sb[cr][2 * (s >> 1) + opt][s & 1][lane];
            qy[s] = row_operand(sh.qr[cb], tl, s, hh);
          }
#pragma unroll
          for (int g = 0; g < 4; ++g) vv[g] = rb_read(sh.v[cb], tl, 8 * opt + 2 * g + hh);
          const float coef = skip_d + sh.gam[cr][tl] * sh.skip[cr][tl];
          const float decay = fast_exp2(sh.cs[cr][tl]);
          f32x16 yi = zero16();
#pragma unroll
          for (int s = 0; s < 4; ++s) yi = mfma(sx[s], qy[s], yi);
#pragma unroll
          for (int g = 0; g < 4; ++g) {
            ybase[4 * g] = coef * lo_f(vv[g][0]) + yi[4 * g] * decay;
            ybase[4 * g + 1] = coef * hi_f(vv[g][0]) + yi[4 * g + 1] * decay;
            ybase[4 * g + 2] = coef * lo_f(vv[g][1]) + yi[4 * g + 2] * decay;
            ybase[4 * g + 3] = coef * hi_f(vv[g][1]) + yi[4 * g + 3] * decay;
          }
        }
        lds_barrier();

        // ---------------- interval B(i) ----------------
        // chunk c = i - 1: intra-chunk scores . v (mamba_fused.py:144-146), gate, store
        const int c = i - 1;
        const int t = c * kChunk + 32 * th_o + c32;
        float yv[16];
#pragma unroll
        for (int e = 0; e < 16; ++e) yv[e] = 0.f;
        if (i > c0) {
          const int cb = c & 1;
          f32x16 y = ybase;
          if (th_o == 0) {
            const u32x4 s0 = sh.score[cb][0][0][lane], s1 = sh.score[cb][0][1][lane];
            const u32x4 v0 = tr_operand_half(sh.v[cb], opt, 0, 0, lane);
            const u32x4 v1 = tr_operand_half(sh.v[cb], opt, 0, 1, lane);
            y = mfma(v0, s0, y);
            y = mfma(v1, s1, y);
          } else {
            const u32x4 s0 = sh.score[cb][1][0][lane], s1 = sh.score[cb][1][1][lane];
            const u32x4 s2 = sh.score[cb][2][0][lane], s3 = sh.score[cb][2][1][lane];
            const u32x4 v0 = tr_operand_half(sh.v[cb], opt, 0, 0, lane);
            const u32x4 v1 = tr_operand_half(sh.v[cb], opt, 0, 1, lane);
            const u32x4 v2 = tr_operand_half(sh.v[cb], opt, 1, 0, lane);
            const u32x4 v3 = tr_operand_half(sh.v[cb], opt, 1, 1, lane);
            y = mfma(v0, s0, y);
            y = mfma(v1, s1, y);
            y = mfma(v2, s2, y);
            y = mfma(v3, s3, y);
          }
#pragma unroll
          for (int e = 0; e < 16; ++e) yv[e] = y[e] * gate[e];
        }
        // Every lane stores in every iteration, through the unit's range-checked
        // output buffer: rows t >= L (and the whole first iteration, which has
        // no chunk to finish) take an offset past any buffer size and the
        // hardware drops them; rows in [L, T) are zero-filled after the walk.
        const int mrow = P.rev ? L - 1 - t : t;  // row in memory order
        const bool live = i > c0 && t < L;
        if constexpr (OUT32) {
          const int lane_off = live ? (mrow * o_row + 32 * opt + 4 * hh) * esz : kOutOfRange;
#pragma unroll
          for (int g = 0; g < 4; ++g)
            __builtin_amdgcn_raw_buffer_store_b128(
                u32x4{__builtin_bit_cast(uint32_t, yv[4 * g]), __builtin_bit_cast(uint32_t, yv[4 * g + 1]),
                      __builtin_bit_cast(uint32_t, yv[4 * g + 2]), __builtin_bit_cast(uint32_t, yv[4 * g + 3])},
                out_rsrc, lane_off + 32 * g, 0, kStreamStore);
        } else {
          // bf16 pieces g (columns 8 g + 4 hh .. + 3) traded with lane ^ 32 into
          // 32 contiguous bytes per lane, columns 16 hh .. 16 hh + 15: after
          // swapping pieces k and k + 2 (one v_permlane32_swap per word),
          // both halves hold (first, second) piece of their 16 bytes k
          u32x2 pw[4];
#pragma unroll
          for (int g = 0; g < 4; ++g) pw[g] = u32x2{pack2(yv[4 * g], yv[4 * g + 1]), pack2(yv[4 * g + 2], yv[4 * g + 3])};
          const int lane_off = live ? (mrow * o_row + 32 * opt + 16 * hh) * esz : kOutOfRange;
#pragma unroll
          for (int k = 0; k < 2; ++k) {
            const auto x0 = __builtin_amdgcn_permlane32_swap(pw[k][0], pw[k + 2][0], false, false);
            const auto x1 = __builtin_amdgcn_permlane32_swap(pw[k][1], pw[k + 2][1], false, false);
            __builtin_amdgcn_raw_buffer_store_b128(u32x4{x0[0], x1[0], x0[1], x1[1]}, out_rsrc, lane_off + 16 * k, 0,
                                                   kStreamStore);
          }
        }
        lds_barrier();
      }
    } else if (state_wave) {
      const int nt = (s_idx >> 1) & 1, spt = s_idx & 1;
      // tile (nt, pt) of S^T[n][p]; a seeded segment starts from its entering
      // state (zero otherwise)
      f32x16 S = zero16();
      if constexpr (SEEDED) {
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const int f = s_idx * 256 + q * 64 + lane;
          const float4 x = seed_lds[f >> 9][f & 511];
          S[4 * q] = x.x, S[4 * q + 1] = x.y, S[4 * q + 2] = x.z, S[4 * q + 3] = x.w;
        }
      }
      {
        u32x4 lo, hi;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          lo[q] = pack2(S[2 * q], S[2 * q + 1]);
          hi[q] = pack2(S[8 + 2 * q], S[8 + 2 * q + 1]);
        }
        sh.sb[c0 % 3][s_idx][0][lane] = lo;  // bf16 S_c0 (read by the outputs of chunk c0)
        sh.sb[c0 % 3][s_idx][1][lane] = hi;
      }
      for (int i = c0; i <= c1; ++i) {
        // ---------------- interval A(i) ----------------
        if (i < c1) rotary(rows, i);
        rows = load_rows(i + 1);
        lds_barrier();

        // ---------------- interval B(i) ----------------
        // the walk needs S_{i+1} for a later chunk
        if (i + 1 < c1) {
          // S_{i+1} = S_i 2^tot + kr^T . bf16(v 2^(tot - cs)) of chunk i (mamba_fused.py:150-152)
          const int cb = i & 1;
          u32x4 kx[4], vy[4];
#pragma unroll
          for (int s = 0; s < 4; ++s) {
            kx[s] = tr_operand(sh.kr[cb], nt, s, lane);
            vy[s] = tr_operand(sh.vs[cb], spt, s, lane);
          }
          const float dec = fast_exp2(sh.tot[i % 3][0]);
          f32x16 d = zero16();
#pragma unroll
          for (int s = 0; s < 4; ++s) d = mfma(kx[s], vy[s], d);
#pragma unroll
          for (int e = 0; e < 16; ++e) S[e] = S[e] * dec + d[e];
          u32x4 lo, hi;
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            lo[q] = pack2(S[2 * q], S[2 * q + 1]);
            hi[q] = pack2(S[8 + 2 * q], S[8 + 2 * q + 1]);
          }
          sh.sb[(i + 1) % 3][s_idx][0][lane] = lo;
          sh.sb[(i + 1) % 3][s_idx][1][lane] = hi;
        }
        lds_barrier();
      }
    } else {
      // The prologue waves carry each interval's longest chain (the score
      // tiles and controls in A, the phase in B) but are the workgroup's
      // youngest waves, so oldest-first issue would serve them last: raise
      // their issue priority over the output and state waves on their SIMD.
      __builtin_amdgcn_s_setprio(2);
      for (int i = c0; i <= c1; ++i) {
        // ---------------- interval A(i) ----------------
        // angles of chunk i + 1, for the phase at B(i)
        load_pipe_angles<RPW, ANG16>(P, th, gbase, pair, (i + 1) * kChunk + sg * RPW, L);
        if (p_idx < 3 && i > c0) {
          // scores of chunk i - 1: tile (th, uh) = (0,0), (1,0), (1,1)
          const int c = i - 1;
          const int cb = c & 1;
          const int sth = p_idx > 0 ? 1 : 0;
          const int suh = p_idx > 1 ? 1 : 0;
          u32x4 kx[4], qy[4];
#pragma unroll
          for (int s = 0; s < 4; ++s) {
            kx[s] = row_operand(sh.kr[cb], 32 * suh + c32, s, hh);
            qy[s] = row_operand(sh.qr[cb], 32 * sth + c32, s, hh);
          }
          f32x16 acc = zero16();
#pragma unroll
          for (int s = 0; s < 4; ++s) acc = mfma(kx[s], qy[s], acc);
          u32x4 sc[2];
          const float* csr = sh.cs[c % 3];
          score_tile(acc, csr[32 * sth + c32], csr + 32 * suh, sth == suh, c32, hh, sc);
          sh.score[cb][p_idx][0][lane] = sc[0];
          sh.score[cb][p_idx][1][lane] = sc[1];
        }
        if (p_idx == 3 && i + 1 < c1) controls(ctl_next, i + 1);
        ctl_next = load_pipe_ctl<CTL16, TRAP16>(P, dto, ado, trb, (i + 2) * kChunk + ctl_lane, L, tlim);
        lds_barrier();

        // ---------------- interval B(i) ----------------
        if (phase_wave && i + 1 < c1) phase(th, i + 1);
        lds_barrier();
      }
    }
  }

  {
    // rows in [L, T) of the segment's time range (the whole range with one
    // segment), the same rows in either direction: unreversed base and
    // stride; 16 pieces per row (16 bytes of fp32, 8 bytes of bf16: the
    // alignment the output rows are checked for)
    const int o_st = P.rev ? -P.o_st : P.o_st;
    const int obase_fwd = b * P.o_sb + h * P.o_sh;
    const int r0 = max(L, seg_start(P, seg) * kChunk);
    const int r1 = seg == P.G - 1 ? T : min(T, seg_start(P, seg + 1) * kChunk);
    for (int e = r0 * 16 + static_cast<int>(threadIdx.x); e < r1 * 16; e += 768) {
      const int tt = e >> 4, piece = e & 15;
      const int off = obase_fwd + tt * o_st + 4 * piece;
      // streaming stores, as the walk's (varlen batches: 24.4 -> 23.3 us)
      if constexpr (OUT32)
        __builtin_nontemporal_store(u32x4{0u, 0u, 0u, 0u}, reinterpret_cast<u32x4*>(static_cast<float*>(P.out) + off));
      else
        __builtin_nontemporal_store(u32x2{0u, 0u}, reinterpret_cast<u32x2*>(static_cast<uint16_t*>(P.out) + off));
    }
  }
}

// LDS of the summary pass: a batch of four chunks (256 rows).
template <int PAIRS>
struct SummarySmem {
  union {
    float trig[256 * kTrigStride];  // [row][pair] (cos, sin)
    float4 dstate[4][1024];         // dS of each chunk, in record layout
  } a;
  union {
    uint32_t inc[PAIRS][260];  // fixed-point phase increments [pair][row]
    struct {
      uint16_t kr[4][64 * 64];  // bf16(rot(k + kb) * s), row buffers
      uint16_t vs[4][64 * 64];  // bf16(v * 2^(tot - cs))
    } t;
  } b;
  float sc[256];
  float wv[256];
  float tot[2][4];  // the chunks' total log2 decays, by batch parity
  float kw[64];     // fused B norm weights
};

// Summary pass of the chunk-parallel form, parallel over the chunks of the
// segment: the state the segment leaves from zero state, S <- S 2^tot_c + dS_c
// over its chunks c (mamba_fused.py:150-152), where dS_c = bf16(v_c 2^(tot_c -
// cs))^T . kr_c needs only chunk c's rows and the phase entering it. Chunks go
// in batches of four (1024 threads, 16 waves):
//   - every thread forms the fixed-point phase increments of rows x pairs of
//     the batch (lane = pair, so a wave's angle loads are whole rows), and the
//     first waves the controls of one chunk each (lane = row); the batch's
//     loads were issued during the previous batch;
//   - wave j scans pair j's increments over the batch's rows, from the phase
//     entering the batch (0 at the segment's start), into the cos/sin table;
//   - every thread rotates and scales the keys of one channel group and
//     scales the values, for two rows (8 lanes per row);
//   - wave w computes the 32 x 32 tile w mod 4 of dS for chunk w / 4;
//   - thread f folds float4 f of the four dS_c into the state, in chunk order.
// These are the serial walk's operations, in its order (its shared helpers,
// with the multiply-adds spelled out), so the record is the one a serial walk
// of the segment from zero state and phase leaves: for the first segment, the
// serial walk's own state after it. The record of a later segment is in that
// segment's phase frame, and the walks turn it by the phase entering the
// segment, which they form from the wrapping phase sums this pass also
// writes (the same integers the serial walk adds).
template <bool CTL16, bool TRAP16, bool ANG16, int PAIRS>
__global__ __launch_bounds__(1024) void pipe_summary_kernel(const MfmaParams P) {
  constexpr int kBatch = 4;                      // chunks per batch
  constexpr int kRowLanes = 1024 / PAIRS;        // phase row lanes per pair
  constexpr int kRowsPer = 256 / kRowLanes;      // phase rows per thread
  constexpr int kSlots = PAIRS / 16;             // pairs per scanning wave
  __shared__ SummarySmem<PAIRS> sh;
  const int tid = static_cast<int>(threadIdx.x);
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63;
  const PipeItem it = pipe_item(P);
  const int b = it.b, h = it.h;
  const int qh = h / P.group;
  const int T = P.T;
  const int R = P.R;
  int L = T;
  if (P.lengths != nullptr) {
    const int64_t l = P.lengths[b];
    L = l < 0 ? 0 : (l > T ? T : static_cast<int>(l));
  }
  const int nvalid = (L + kChunk - 1) / kChunk;
  const int c0 = min(seg_start(P, it.seg), nvalid);
  const int c1 = min(seg_start(P, it.seg + 1), nvalid);
  const int tlim = P.rev ? L : T;
  const int roff = P.rev ? max(L - 1, 0) : 0;
  const uint16_t* kbase = P.k + b * P.k_sb + qh * P.k_sh - roff * P.k_st;
  const uint16_t* vbase = P.v + b * P.v_sb + h * P.v_sh - roff * P.v_st;
  const int dto = b * P.d_sb + h * P.d_sh - roff * P.d_st;
  const int ado = b * P.a_sb + h * P.a_sh - roff * P.a_st;
  const int trb = b * P.r_sb + h * P.r_sh - roff * P.r_st;
  const int gbase = b * P.g_sb + h * P.g_sh - roff * P.g_st;
  const float step_bias = P.ctl_raw ? P.dt_bias[h] : 0.f;

  // phase of the wave's scan pairs from the segment's start (the segment's
  // own frame; the walks turn the record into the unit's frame)
  uint32_t carry[kSlots] = {};
  const int t_stop = min(L, c1 * kChunk);  // rows past the segment add no phase
  const int pj = tid % PAIRS;   // phase lanes: pair
  const int prl = tid / PAIRS;  // and row lane
  // key rotation tasks: channel group ng of batch rows rsub and rsub + 128
  // (8 lanes per row, so a wave's row loads are 8 whole 128-byte rows)
  const int ng = lane & 7;
  const int rsub = w * 8 + row8_of_lane(lane);
  float kbv[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) kbv[j] = P.kb[h * 64 + 8 * ng + j];

  float4 S = make_float4(0.f, 0.f, 0.f, 0.f);
  float seg_log2 = 0.f;
  int parity = 0;
  // a batch's loads (rows clamped to ones that exist), issued one batch ahead
  float th[kRowsPer], dts[kRowsPer];
  PipeCtl raw = {};
  u32x4 kin[2], vin[2];
  auto issue_loads = [&](int cb0) {
    const int t_lo = cb0 * kChunk;
    if (pj < R) {
#pragma unroll
      for (int i = 0; i < kRowsPer; ++i) {
        const int tc = min(t_lo + prl + kRowLanes * i, L - 1);
        dts[i] = load_elem<CTL16>(P.dt, dto + tc * P.d_st);
        th[i] = load_elem<ANG16>(P.angles, gbase + pj * P.g_sr + tc * P.g_st);
      }
    }
    // waves 4-15 do not form controls: one row for all lanes (one cache line
    // per load instead of 32)
    raw = load_pipe_ctl<CTL16, TRAP16>(P, dto, ado, trb, (cb0 + (w & 3)) * kChunk + (w < kBatch ? lane : 0), L, tlim);
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int tc = min(t_lo + rsub + 128 * i, L - 1);
      kin[i] = *reinterpret_cast<const u32x4*>(kbase + tc * P.k_st + 8 * ng);
      vin[i] = *reinterpret_cast<const u32x4*>(vbase + tc * P.v_st + 8 * ng);
    }
  };
  if (c0 < c1) issue_loads(c0);
  // fused B norm weights, read by the key rotation (after two barriers)
  if (w == 0 && P.qk_norm) sh.kw[lane] = P.kn_w[lane];
  for (int cb0 = c0; cb0 < c1; cb0 += kBatch, parity ^= 1) {
    const int nb = min(kBatch, c1 - cb0);
    const int t_lo = cb0 * kChunk;

    // phase increments (rows past the length have no step and add 0)
    if (pj < R) {
#pragma unroll
      for (int i = 0; i < kRowsPer; ++i) {
        const int r = prl + kRowLanes * i;
        float d = dts[i];
        if (P.ctl_raw) d = control_step(d, step_bias);
        sh.b.inc[pj][r] = phase_inc(th[i], t_lo + r < t_stop ? d : 0.f);
      }
    }
    // controls of chunk cb0 + w
    if (w < nb) {
      const int t = (cb0 + w) * kChunk + lane;
      const RowControls rc = row_controls(P, raw, t < L, t + 1 < tlim, step_bias);
      sh.sc[w * kChunk + lane] = rc.sc;
      sh.wv[w * kChunk + lane] = rc.wv;
      if (lane == 0) sh.tot[parity][w] = rc.tot;
    }
    lds_barrier();

    // per pair: phase of every row of the batch, then cos/sin
#pragma unroll
    for (int k = 0; k < kSlots; ++k) {
      const int j = w + 16 * k;
      if (j < R) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int r = lane + 64 * i;
          const uint32_t incl = wave_scan_u32(sh.b.inc[j][r]);
          *reinterpret_cast<float2*>(&sh.a.trig[r * kTrigStride + 2 * j]) = phase_trig(carry[k] + incl);
          carry[k] += static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(incl), 63));
        }
      }
    }
    lds_barrier();

    // keys: bias, rotation, scale; values: decay scale (mamba_fused.py:112-131, 151)
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int r = rsub + 128 * i;
      const int cc = r >> 6;
      if (cc < nb) {
        const bool valid = t_lo + r < L;
        const float scl = sh.sc[r];
        const float wvt = sh.wv[r];
        u32x4 ko, vso;
        // the walk's norm of the raw key row (cc is wave-uniform: a wave's
        // rows lie in one chunk)
        if (P.qk_norm) kin[i] = norm_row8(kin[i], &sh.kw[8 * ng], P.norm_eps);
        if (4 * ng < R) {
          // pairs 4 ng + j >= R turn by the identity
          const float2* tg = reinterpret_cast<const float2*>(&sh.a.trig[r * kTrigStride + 8 * ng]);
          const float2 t0 = tg[0], t1 = tg[1], t2 = tg[2], t3 = tg[3];
          const float cosv[4] = {t0.x, t1.x, t2.x, t3.x}, sinv[4] = {t0.y, t1.y, t2.y, t3.y};
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            const bool on = 4 * ng + j < R;
            const float k0 = lo_f(kin[i][j]) + kbv[2 * j], k1 = hi_f(kin[i][j]) + kbv[2 * j + 1];
            ko[j] = key_pair(k0, k1, on ? cosv[j] : 1.f, on ? sinv[j] : 0.f, scl);
          }
        } else {
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            const float k0 = lo_f(kin[i][j]) + kbv[2 * j], k1 = hi_f(kin[i][j]) + kbv[2 * j + 1];
            ko[j] = pack2(k0 * scl, k1 * scl);
          }
        }
#pragma unroll
        for (int j = 0; j < 4; ++j) vso[j] = scaled_pair(valid ? vin[i][j] : 0u, wvt);
        rb_write16(sh.b.t.kr[cc], r & 63, 2 * ng, ko);
        rb_write16(sh.b.t.vs[cc], r & 63, 2 * ng, vso);
      }
    }
    if (cb0 + kBatch < c1) issue_loads(cb0 + kBatch);
    lds_barrier();

    // dS_c = kr^T . vs tile (nt, pt) of S^T[n][p], in the walk's tile layout
    {
      const int cc = w >> 2, st = w & 3;
      if (cc < nb) {
        const int nt = st >> 1, spt = st & 1;
        u32x4 kx[4], vy[4];
#pragma unroll
        for (int s = 0; s < 4; ++s) {
          kx[s] = tr_operand(sh.b.t.kr[cc], nt, s, lane);
          vy[s] = tr_operand(sh.b.t.vs[cc], spt, s, lane);
        }
        f32x16 d = zero16();
#pragma unroll
        for (int s = 0; s < 4; ++s) d = mfma(kx[s], vy[s], d);
#pragma unroll
        for (int q = 0; q < 4; ++q)
          sh.a.dstate[cc][st * 256 + q * 64 + lane] = make_float4(d[4 * q], d[4 * q + 1], d[4 * q + 2], d[4 * q + 3]);
      }
    }
    lds_barrier();

    // S <- S 2^tot_c + dS_c, chunk by chunk
    for (int cc = 0; cc < nb; ++cc) {
      const float tot = sh.tot[parity][cc];
      const float dec = fast_exp2(tot);
      const float4 x = sh.a.dstate[cc][tid];
      S = make_float4(S.x * dec + x.x, S.y * dec + x.y, S.z * dec + x.z, S.w * dec + x.w);
      seg_log2 += tot;
    }
  }
  P.seg_state[static_cast<size_t>(it.rec) * 1024 + tid] = S;
  if (tid == 0) P.seg_decay[it.rec] = seg_log2;
  // the segment's phase sum per pair (0 for pairs >= R)
  if (lane == 0) {
#pragma unroll
    for (int k = 0; k < kSlots; ++k) P.phase_fx[static_cast<size_t>(it.rec) * 32 + w + 16 * k] = carry[k];
    if constexpr (PAIRS == 16) P.phase_fx[static_cast<size_t>(it.rec) * 32 + w + 16] = 0u;
  }
}

// Chunk-parallel plan: with at most 128 (batch, head) units, each unit's time
// axis is cut into G segments of at most SC chunks (seg_start) so that
// units * G is about one workgroup per CU. Scratch: states [units][G][4096] fp32, phase sums
// [units][G][32] uint32, decays [units][G] fp32, each 256-byte aligned.
constexpr int64_t kMinSegmentChunks = 4;

struct PipePlan {
  int G = 1;
  int SC = 0;
  int64_t phase_off = 0, decay_off = 0, bytes = 0;
};

PipePlan pipe_plan(const tf_mamba_args& a) {
  PipePlan p;
  const int64_t units = a.batch * a.heads;
  const int64_t chunks = (a.time + kChunk - 1) / kChunk;
  p.SC = static_cast<int>(chunks);
  if (units <= 0 || chunks <= 0 || units > 128) return p;
  int64_t g = 256 / units;
  // at least kMinSegmentChunks per segment: shorter walks gain less from the
  // extra workgroups than the two extra passes cost
  const int64_t sc = std::max<int64_t>((chunks + g - 1) / g, kMinSegmentChunks);
  g = (chunks + sc - 1) / sc;
  if (g < 2) return p;
  p.G = static_cast<int>(g);
  p.SC = static_cast<int>(sc);
  auto up = [](int64_t x) { return (x + 255) & ~int64_t(255); };
  const int64_t recs = units * g;
  p.phase_off = up(recs * 4096 * 4);
  p.decay_off = p.phase_off + up(recs * 32 * 4);
  p.bytes = p.decay_off + up(recs * 4);
  return p;
}

}  // namespace

bool pipe_supported(const tf_mamba_args& a) {
  if (a.state != 64 || a.head_dim != 64) return false;
  if (a.rotary < 0 || a.rotary > 32) return false;
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
  if (a.batch * a.heads > 0x7fffffff) return false;
  // q, k, v rows in 16-byte pieces; z and out rows in 8-byte (bf16) or 16-byte (fp32) pieces
  if (!rows_vectorisable(a.q, a.q_stride, 2, 16) || !rows_vectorisable(a.k, a.k_stride, 2, 16) ||
      !rows_vectorisable(a.v, a.v_stride, 2, 16) || !rows_vectorisable(a.z, a.z_stride, 2, 8))
    return false;
  const int ob = a.out_dtype == TF_FLOAT32 ? 4 : 2;
  if (!rows_vectorisable(a.out, a.out_stride, ob, 4 * ob)) return false;
  // output rows through a range-checked buffer: rows apart by at least one
  // row (so a row past the length is out of range) and a byte range below 2^31
  if (a.out_stride[1] < 64 || a.out_stride[3] != 1) return false;
  if ((a.time * a.out_stride[1] + 64) * ob >= (int64_t(1) << 31)) return false;
  return offsets_fit(a);
}

namespace {

template <int RPW, bool CTL16, bool TRAP16, bool ANG16>
int launch_pipe_kernel(const MfmaParams& P, hipStream_t stream) {
  const dim3 grid(static_cast<uint32_t>(P.units) * P.G), block(768);
  if (P.G > 1) {
    // segment summaries (from zero state, each in its segment's phase frame,
    // with the segment's phase sums) -> the seeded walks, which scan the
    // summaries before their segment and write the outputs
    if (P.R <= 16)
      hipLaunchKernelGGL((pipe_summary_kernel<CTL16, TRAP16, ANG16, 16>), grid, dim3(1024), 0, stream, P);
    else
      hipLaunchKernelGGL((pipe_summary_kernel<CTL16, TRAP16, ANG16, 32>), grid, dim3(1024), 0, stream, P);
    if (const int rc = launch_status()) return rc;
  }
  if (P.G > 1) {
    if (P.out_f32)
      hipLaunchKernelGGL((mamba_pipe_kernel<RPW, CTL16, TRAP16, ANG16, true, true>), grid, block, 0, stream, P);
    else
      hipLaunchKernelGGL((mamba_pipe_kernel<RPW, CTL16, TRAP16, ANG16, false, true>), grid, block, 0, stream, P);
  } else if (P.out_f32) {
    hipLaunchKernelGGL((mamba_pipe_kernel<RPW, CTL16, TRAP16, ANG16, true, false>), grid, block, 0, stream, P);
  } else {
    hipLaunchKernelGGL((mamba_pipe_kernel<RPW, CTL16, TRAP16, ANG16, false, false>), grid, block, 0, stream, P);
  }
  return launch_status();
}

template <int RPW>
int launch_pipe_rpw(const MfmaParams& P, hipStream_t stream) {
  const int key = (P.ctl_bf16 ? 4 : 0) | (P.trap_bf16 ? 2 : 0) | (P.angles_dtype == TF_BFLOAT16 ? 1 : 0);
  switch (key) {
    case 0: return launch_pipe_kernel<RPW, false, false, false>(P, stream);
    case 1: return launch_pipe_kernel<RPW, false, false, true>(P, stream);
    case 2: return launch_pipe_kernel<RPW, false, true, false>(P, stream);
    case 3: return launch_pipe_kernel<RPW, false, true, true>(P, stream);
    case 4: return launch_pipe_kernel<RPW, true, false, false>(P, stream);
    case 5: return launch_pipe_kernel<RPW, true, false, true>(P, stream);
    case 6: return launch_pipe_kernel<RPW, true, true, false>(P, stream);
    default: return launch_pipe_kernel<RPW, true, true, true>(P, stream);
  }
}

}  // namespace

int64_t pipe_workspace_bytes(const tf_mamba_args& a) {
  if (!pipe_supported(a)) return 0;
  const PipePlan plan = pipe_plan(a);
  return plan.G > 1 ? plan.bytes : 0;
}

int launch_pipe(const tf_mamba_args& a, hipStream_t stream) {
  MfmaParams P = make_params(a);
  if (a.rotary == 0) {
    // no angles to read: the (unused) angle loads read q's rows of the unit's
    // batch row instead, so every load address exists
    P.angles = a.q;
    P.angles_dtype = TF_BFLOAT16;
    P.g_sb = P.q_sb, P.g_st = P.q_st, P.g_sh = 0, P.g_sr = 1;
  }
  const PipePlan plan = pipe_plan(a);
  if (plan.G > 1 && a.workspace != nullptr && aligned(a.workspace, 256) && a.workspace_bytes >= plan.bytes) {
    char* ws = static_cast<char*>(a.workspace);
    P.G = plan.G;
    P.SC = plan.SC;
    P.seg_state = reinterpret_cast<float4*>(ws);
    P.phase_fx = reinterpret_cast<uint32_t*>(ws + plan.phase_off);
    P.seg_decay = reinterpret_cast<float*>(ws + plan.decay_off);
  }
  const int64_t items = static_cast<int64_t>(P.units) * P.G;
  P.xcd_per = (items % 8 == 0 && items >= 64) ? static_cast<int>(items / 8) : 0;
  // unsegmented varlen walks over more units than CUs: longest rows first
  P.lpt = (a.lengths != nullptr && P.G == 1 && a.batch <= 64 && a.batch % 8 == 0 && items > 256) ? 1 : 0;
  return a.rotary <= 16 ? launch_pipe_rpw<4>(P, stream) : launch_pipe_rpw<8>(P, stream);
}

}  // namespace tf

