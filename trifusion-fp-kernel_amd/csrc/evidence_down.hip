// Evidence down-projection of the TriFusion block:
//   z = bf16(silu(bf16(cat(cn, an) w^T + bias)))
// the reference's silu(e_down(torch.cat((cn, an), -1))) under bf16 autocast
// (src/trifusion_l4/model.py:161): the concatenation is never formed, the
// linear and the SiLU are one launch instead of a copy, a library GEMM of
// r = 64 output columns and an elementwise pass.
//
// At the model's shapes the product is tiny (B T = 1616 rows, K = 2d = 2048,
// r = 64) and the time goes to moving cn, an and w into the compute units.
// Loading MFMA operands straight from memory reads 32 rows of 32 bytes per
// wave instruction, and a workgroup then streams at about a quarter of what
// whole cache lines give. The staged kernel (d <= 1024) instead copies
// 128-column chunks of its 32 rows and 32 weight rows into LDS with whole-line
// loads, keeping four chunks in flight in registers (the chunk loop is unrolled
// at compile time so every wait names one chunk's loads), and feeds the MFMAs
// from LDS. Wider d runs the direct-load kernel.
//
// Both kernels: one workgroup of four waves per 32 rows; wave q contracts a
// quarter of the k-steps against the matching w columns (tiles of
// v_mfma_f32_32x32x16_bf16; a tile's columns past r read w row r - 1 and are
// dropped). Lane (c32, hh) feeds row c32 and output column c32 with the 8
// contiguous k values 8 hh .. 8 hh + 7 of each 16-wide k-step, the same k order
// in both operands. The four partial tiles meet in LDS; each thread then sums
// them for neighbouring columns of one row, adds the bias, rounds to bf16 as the
// linear's output is, and applies SiLU as x / (1 + exp(-x)) in fp32, rounded to
// bf16.
#include "mfma_tile.h"

namespace tf {
namespace {

constexpr int kDownRows = 32;

template <int R>  // output columns: 16, 32, 48 or 64
__global__ __launch_bounds__(256) void evidence_down_kernel(const uint16_t* __restrict__ cn,
                                                            const uint16_t* __restrict__ an,
                                                            const uint16_t* __restrict__ w,
                                                            const uint16_t* __restrict__ bias,
                                                            uint16_t* __restrict__ z, int rows, int d) {
  constexpr int NT = (R + 31) / 32;  // 32-column tiles
  __shared__ float part[4][NT][16][64];  // partial tiles in MFMA accumulator layout
  const int wave = static_cast<int>(threadIdx.x >> 6);
  const int lane = static_cast<int>(threadIdx.x & 63);
  const int c32 = lane & 31, hh = lane >> 5;
  const int row0 = static_cast<int>(blockIdx.x) * kDownRows;
  const int kq = d / 2;  // k columns per wave
  // rows past the last are read as the last row and never stored
  const int row = min(row0 + c32, rows - 1);
  const uint16_t* arow = (wave < 2 ? cn : an) + static_cast<int64_t>(row) * d + (wave & 1) * kq + 8 * hh;
  const uint16_t* wrow[NT];
#pragma unroll
  for (int nt = 0; nt < NT; ++nt)
    wrow[nt] = w + static_cast<int64_t>(min(32 * nt + c32, R - 1)) * (2 * d) + wave * kq + 8 * hh;

  f32x16 acc[NT];
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) acc[nt] = zero16();
  constexpr int kUnroll = 4;
  for (int k = 0; k < kq; k += 16 * kUnroll) {
    u32x4 a[kUnroll], b[kUnroll][NT];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      a[u] = *reinterpret_cast<const u32x4*>(arow + k + 16 * u);
#pragma unroll
      for (int nt = 0; nt < NT; ++nt) b[u][nt] = *reinterpret_cast<const u32x4*>(wrow[nt] + k + 16 * u);
    }
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
#pragma unroll
      for (int nt = 0; nt < NT; ++nt) acc[nt] = mfma(a[u], b[u][nt], acc[nt]);
    }
  }
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) {
#pragma unroll
    for (int e = 0; e < 16; ++e) part[wave][nt][e][lane] = acc[nt][e];
  }
  __syncthreads();

  // thread -> row i of the group, columns j0 .. j0 + CPT - 1
  constexpr int CPT = R * kDownRows / 256;  // r / 8: 2, 4, 6 or 8
  const int t = static_cast<int>(threadIdx.x);
  const int i = t / (R / CPT);
  const int j0 = (t % (R / CPT)) * CPT;
  // accumulator element of row i: e = 4 (i / 8) + i % 4 in lane half (i / 4) % 2
  const int e = 4 * (i >> 3) + (i & 3);
  const int half = (i >> 2) & 1;
  uint32_t packed[CPT / 2];
#pragma unroll
  for (int c = 0; c < CPT; c += 2) {
    float v[2];
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int j = j0 + c + u;
      const int nt = j >> 5, ln = (j & 31) + 32 * half;
      const float s = part[0][nt][e][ln] + part[1][nt][e][ln] + part[2][nt][e][ln] + part[3][nt][e][ln];
      const float x = round_bf16(s + bf16_to_f32(bias[j]));
      v[u] = x / (1.f + expf(-x));
    }
    packed[c / 2] = pack2(v[0], v[1]);
  }
  if (row0 + i < rows) {
    uint16_t* out = z + static_cast<int64_t>(row0 + i) * R + j0;
    if constexpr (CPT == 8) {
      *reinterpret_cast<u32x4*>(out) = u32x4{packed[0], packed[1], packed[2], packed[3]};
    } else if constexpr (CPT == 4) {
      *reinterpret_cast<u32x2*>(out) = u32x2{packed[0], packed[1]};
    } else {
#pragma unroll
      for (int c = 0; c < CPT / 2; ++c) reinterpret_cast<uint32_t*>(out)[c] = packed[c];
    }
  }
}


// Staged kernel: workgroup (row block, 32-column block of z); KC-column chunks
// of the concatenated row, NCH = 2 d / KC of them.
constexpr int kChunk = 128;
constexpr int kRing = 4;  // chunks in flight

template <int NCH>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, 1))) void evidence_down_staged_kernel(
    const uint16_t* __restrict__ cn, const uint16_t* __restrict__ an, const uint16_t* __restrict__ w,
    const uint16_t* __restrict__ bias, uint16_t* __restrict__ z, int rows, int r) {
  constexpr int d = NCH * kChunk / 2, K = 2 * d;
  constexpr int P = NCH < kRing ? NCH : kRing;
  constexpr int LD = kChunk + 8;        // LDS row pitch in elements (16-byte pad)
  constexpr int UPR = kChunk / 8;       // 16-byte units per row of a chunk
  constexpr int U = 32 * UPR / 256;     // units per thread, for both operands
  constexpr int SPW = kChunk / 16 / 4;  // k-steps per wave per chunk
  __shared__ __align__(16) uint16_t As[2][32][LD];
  __shared__ __align__(16) uint16_t Ws[2][32][LD];
  __shared__ float part[4][16][64];
  const int t = static_cast<int>(threadIdx.x), wave = t >> 6, lane = t & 63;
  const int c32 = lane & 31, hh = lane >> 5;
  const int row0 = static_cast<int>(blockIdx.x) * kDownRows, col0 = static_cast<int>(blockIdx.y) * 32;
  // unit i of thread t: row (t + 256 i) / UPR of the chunk, 16-byte column (t + 256 i) % UPR;
  // a wave's 64 units are whole 128-byte lines
  int64_t aoff[U];
  const uint16_t* wrow[U];
#pragma unroll
  for (int i = 0; i < U; ++i) {
    const int u = t + 256 * i, rr = u / UPR, cu = u % UPR;
    aoff[i] = static_cast<int64_t>(min(row0 + rr, rows - 1)) * d + 8 * cu;
    wrow[i] = w + static_cast<int64_t>(min(col0 + rr, r - 1)) * K + 8 * cu;
  }
  u32x4 ra[P][U], rw[P][U];
  auto gload = [&](int c, u32x4* a, u32x4* b) {
    const int k0 = c * kChunk;
    const uint16_t* src = k0 < d ? cn + k0 : an + (k0 - d);
#pragma unroll
    for (int i = 0; i < U; ++i) {
      a[i] = *reinterpret_cast<const u32x4*>(src + aoff[i]);
      b[i] = *reinterpret_cast<const u32x4*>(wrow[i] + k0);
    }
  };
  auto swrite = [&](int buf, const u32x4* a, const u32x4* b) {
#pragma unroll
    for (int i = 0; i < U; ++i) {
      const int u = t + 256 * i, rr = u / UPR, cu = u % UPR;
      *reinterpret_cast<u32x4*>(&As[buf][rr][8 * cu]) = a[i];
      *reinterpret_cast<u32x4*>(&Ws[buf][rr][8 * cu]) = b[i];
    }
  };
  f32x16 acc = zero16();
#pragma unroll
  for (int p = 0; p < P; ++p) gload(p, ra[p], rw[p]);
  // chunk c sits in LDS buffer c % 2; the barrier after writing chunk c + 1
  // also orders every wave's reads of chunk c - 1 before buffer (c + 1) % 2 is
  // rewritten
#pragma unroll
  for (int c = 0; c < NCH; ++c) {
    const int p = c % P, buf = c & 1;
    swrite(buf, ra[p], rw[p]);
    __syncthreads();
    if (c + P < NCH) gload(c + P, ra[p], rw[p]);
#pragma unroll
    for (int s = 0; s < SPW; ++s) {
      const int kk = 16 * (wave * SPW + s) + 8 * hh;
      const u32x4 a = *reinterpret_cast<const u32x4*>(&As[buf][c32][kk]);
      const u32x4 b = *reinterpret_cast<const u32x4*>(&Ws[buf][c32][kk]);
      acc = mfma(a, b, acc);
    }
  }
#pragma unroll
  for (int e = 0; e < 16; ++e) part[wave][e][lane] = acc[e];
  __syncthreads();

  // thread -> row i of the block, columns j0 .. j0 + 3 of the 32
  const int i = t >> 3, j0 = (t & 7) * 4;
  const int e = 4 * (i >> 3) + (i & 3), half = (i >> 2) & 1;
  if (row0 + i >= rows || col0 + j0 >= r) return;  // r is a multiple of 16: all four or none
  uint32_t packed[2];
#pragma unroll
  for (int c = 0; c < 4; c += 2) {
    float v[2];
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int ln = j0 + c + u + 32 * half;
      const float sum = part[0][e][ln] + part[1][e][ln] + part[2][e][ln] + part[3][e][ln];
      const float x = round_bf16(sum + bf16_to_f32(bias[col0 + j0 + c + u]));
      v[u] = x / (1.f + expf(-x));
    }
    packed[c / 2] = pack2(v[0], v[1]);
  }
  *reinterpret_cast<u32x2*>(z + static_cast<int64_t>(row0 + i) * r + col0 + j0) = u32x2{packed[0], packed[1]};
}

}  // namespace
}  // namespace tf

extern "C" int tf_evidence_down(const void* cn, const void* an, const void* w, const void* bias, void* z,
                                int64_t rows, int64_t d, int64_t r, void* stream) {
  if (rows < 0 || d < 0) return TF_ERR_SHAPE;
  if (rows == 0) return TF_OK;
  if (!cn || !an || !w || !bias || !z) return TF_ERR_NULL;
  // k quarters of whole 64-element steps; r a multiple of 16 up to 64
  if (d < 128 || d % 128 || r < 16 || r > 64 || r % 16 || rows > 0x7fffffff / 2 || d > (1 << 20))
    return TF_ERR_SHAPE;
  for (const void* p : {cn, an, w, static_cast<const void*>(z)})
    if (reinterpret_cast<uintptr_t>(p) % 16) return TF_ERR_STRIDE;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const auto* cp = static_cast<const uint16_t*>(cn);
  const auto* ap = static_cast<const uint16_t*>(an);
  const auto* wp = static_cast<const uint16_t*>(w);
  const auto* bp = static_cast<const uint16_t*>(bias);
  auto* zp = static_cast<uint16_t*>(z);
  const int n = static_cast<int>(rows), k = static_cast<int>(d), m = static_cast<int>(r);
  const uint32_t blocks = static_cast<uint32_t>((rows + tf::kDownRows - 1) / tf::kDownRows);
  if (d <= 1024) {
    const dim3 grid(blocks, static_cast<uint32_t>((r + 31) / 32)), block(256);
    switch (d / 128) {
#define TF_STAGED(Q) \
  case Q: hipLaunchKernelGGL(tf::evidence_down_staged_kernel<2 * Q>, grid, block, 0, s, cp, ap, wp, bp, zp, n, m); break;
      TF_STAGED(1) TF_STAGED(2) TF_STAGED(3) TF_STAGED(4) TF_STAGED(5) TF_STAGED(6) TF_STAGED(7) TF_STAGED(8)
#undef TF_STAGED
    }
    return tf::launch_status();
  }
  const dim3 grid(blocks), block(256);
  switch (r) {
    case 16: hipLaunchKernelGGL(tf::evidence_down_kernel<16>, grid, block, 0, s, cp, ap, wp, bp, zp, n, k); break;
    case 32: hipLaunchKernelGGL(tf::evidence_down_kernel<32>, grid, block, 0, s, cp, ap, wp, bp, zp, n, k); break;
    case 48: hipLaunchKernelGGL(tf::evidence_down_kernel<48>, grid, block, 0, s, cp, ap, wp, bp, zp, n, k); break;
    default: hipLaunchKernelGGL(tf::evidence_down_kernel<64>, grid, block, 0, s, cp, ap, wp, bp, zp, n, k); break;
  }
  return tf::launch_status();
}
