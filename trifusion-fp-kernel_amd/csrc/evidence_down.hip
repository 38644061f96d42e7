// Evidence down-projection of the TriFusion block:
//   z = bf16(silu(bf16(cat(cn, an) w^T + bias)))
// the reference's silu(e_down(torch.cat((cn, an), -1))) under bf16 autocast
// (src/trifusion_l4/model.py:161): the concatenation is never formed, the
// linear and the SiLU are one launch instead of a copy, a library GEMM of
// r = 64 output columns and an elementwise pass.
//
// One workgroup of four waves per 32 rows. The concatenated row has K = 2d
// columns; wave q contracts quarter q of them (waves 0-1 read cn, 2-3 read an)
// against the matching quarter of every w row, for all r output columns
// (ceil(r / 32) tiles of v_mfma_f32_32x32x16_bf16; a tile's columns past r read
// w row r - 1 and are dropped). Lane (c32, hh) feeds row c32 and output column
// c32 of each tile with the 8 contiguous k values 8 hh .. 8 hh + 7 of each
// 16-wide k-step, the same k order in both operands. The four partial tiles
// meet in LDS; each thread then sums them for r / 8 neighbouring columns of one
// row, adds the bias, rounds to bf16 as the linear's output is, and applies
// SiLU as x / (1 + exp(-x)) in fp32, rounded to bf16.
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
  const dim3 grid(static_cast<uint32_t>((rows + tf::kDownRows - 1) / tf::kDownRows)), block(256);
  hipStream_t s = static_cast<hipStream_t>(stream);
  const auto* cp = static_cast<const uint16_t*>(cn);
  const auto* ap = static_cast<const uint16_t*>(an);
  const auto* wp = static_cast<const uint16_t*>(w);
  const auto* bp = static_cast<const uint16_t*>(bias);
  auto* zp = static_cast<uint16_t*>(z);
  const int n = static_cast<int>(rows), k = static_cast<int>(d);
  switch (r) {
    case 16: hipLaunchKernelGGL(tf::evidence_down_kernel<16>, grid, block, 0, s, cp, ap, wp, bp, zp, n, k); break;
    case 32: hipLaunchKernelGGL(tf::evidence_down_kernel<32>, grid, block, 0, s, cp, ap, wp, bp, zp, n, k); break;
    case 48: hipLaunchKernelGGL(tf::evidence_down_kernel<48>, grid, block, 0, s, cp, ap, wp, bp, zp, n, k); break;
    default: hipLaunchKernelGGL(tf::evidence_down_kernel<64>, grid, block, 0, s, cp, ap, wp, bp, zp, n, k); break;
  }
  return tf::launch_status();
}
