// Query reads of the TriFusion decoder (decoder.py:17-32): NQ learned queries
// per head attend, with fp32 softmax, to a sequence's keys j < key_length[b];
// queries q [NQ, H, D] (shared by every batch row), keys and values the two
// halves of one projection kv [B, T, 2 H D] (bf16). Split over keys as in
// flash decoding: pass 1, one wave per (64-key tile, head, batch row), scores
// every query against its tile, takes the tile's softmax max and sum per query
// and the tile's unnormalised output; pass 2 merges the tiles of each (head,
// batch row) and writes y [B, NQ, H D] in bf16 (the head-merged layout the out
// projection reads). With no valid key a query row is 0 (SDPA would give NaN).
#include "common.h"

namespace tf {
namespace {

constexpr int kTile = 64;

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, 64));
  return v;
}

// Partial record of one (tile, head, batch row): per query max, sum, D outputs.
template <int D>
constexpr int rec_floats(int nq) { return nq * (D + 2); }

template <int NQ, int D>
__global__ __launch_bounds__(64) void query_read_tiles_kernel(const uint16_t* __restrict__ q,
                                                              const uint16_t* __restrict__ kv,
                                                              const int64_t* __restrict__ key_lengths,
                                                              float* __restrict__ part, int T, int H, int S,
                                                              float scale) {
  __shared__ float qs[NQ * D];
  __shared__ float ps[NQ * kTile];
  __shared__ float vs[kTile * (D + 1)];
  const int lane = threadIdx.x;
  const int s = blockIdx.x, h = blockIdx.y, b = blockIdx.z;
  int64_t lk = key_lengths[b];
  lk = lk < 0 ? 0 : (lk > T ? T : lk);
  for (int i = lane; i < NQ * D; i += 64) {
    const int qi = i / D, d = i - qi * D;
    qs[i] = bf16_to_f32(q[(qi * H + h) * D + d]);
  }
  const int j = s * kTile + lane;
  const bool valid = j < lk;
  float kr[D];
  const int64_t row = (static_cast<int64_t>(b) * T + (valid ? j : 0)) * 2 * H * D + static_cast<int64_t>(h) * D;
  const uint4* kp = reinterpret_cast<const uint4*>(kv + row);
  const uint4* vp = reinterpret_cast<const uint4*>(kv + row + static_cast<int64_t>(H) * D);
#pragma unroll
  for (int c = 0; c < D / 8; ++c) {
    const uint4 kk = valid ? kp[c] : make_uint4(0u, 0u, 0u, 0u);
    const uint4 vv = valid ? vp[c] : make_uint4(0u, 0u, 0u, 0u);
    const uint32_t kw[4] = {kk.x, kk.y, kk.z, kk.w}, vw[4] = {vv.x, vv.y, vv.z, vv.w};
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      kr[8 * c + 2 * e] = __uint_as_float(kw[e] << 16);
      kr[8 * c + 2 * e + 1] = __uint_as_float(kw[e] & 0xffff0000u);
      vs[lane * (D + 1) + 8 * c + 2 * e] = __uint_as_float(vw[e] << 16);
      vs[lane * (D + 1) + 8 * c + 2 * e + 1] = __uint_as_float(vw[e] & 0xffff0000u);
    }
  }
  __syncthreads();
  float mq[NQ], lq[NQ];
#pragma unroll
  for (int qi = 0; qi < NQ; ++qi) {
    float sc = 0.f;
#pragma unroll
    for (int d = 0; d < D; ++d) sc += qs[qi * D + d] * kr[d];
    sc = valid ? sc * scale : -INFINITY;
    const float m = wave_max(sc);
    const float p = m == -INFINITY ? 0.f : expf(sc - m);
    mq[qi] = m;
    lq[qi] = wave_sum(p);
    ps[qi * kTile + lane] = p;
  }
  __syncthreads();
  float* rec = part + ((static_cast<int64_t>(b) * H + h) * S + s) * rec_floats<D>(NQ);
  if (lane < NQ) {
    float m = 0.f, l = 0.f;
#pragma unroll
    for (int qi = 0; qi < NQ; ++qi)
      if (qi == lane) m = mq[qi], l = lq[qi];
    rec[lane * (D + 2)] = m;
    rec[lane * (D + 2) + 1] = l;
  }
  for (int o = lane; o < NQ * D; o += 64) {
    const int qi = o / D, d = o - qi * D;
    float acc = 0.f;
#pragma unroll 8
    for (int jj = 0; jj < kTile; ++jj) acc += ps[qi * kTile + jj] * vs[jj * (D + 1) + d];
    rec[qi * (D + 2) + 2 + d] = acc;
  }
}

// One thread per (query, dim) of one (head, batch row): merge the S tiles.
template <int NQ, int D>
__global__ __launch_bounds__(NQ * D) void query_read_merge_kernel(const float* __restrict__ part,
                                                                  uint16_t* __restrict__ y, int H, int S) {
  const int h = blockIdx.x, b = blockIdx.y;
  const int qi = threadIdx.x / D, d = threadIdx.x - qi * D;
  const float* base = part + (static_cast<int64_t>(b) * H + h) * S * rec_floats<D>(NQ) + qi * (D + 2);
  float m = -INFINITY;
  for (int s = 0; s < S; ++s) m = fmaxf(m, base[s * rec_floats<D>(NQ)]);
  float l = 0.f, o = 0.f;
  if (m != -INFINITY) {
    for (int s = 0; s < S; ++s) {
      const float* r = base + s * rec_floats<D>(NQ);
      const float w = r[0] == -INFINITY ? 0.f : expf(r[0] - m);
      l += w * r[1];
      o += w * r[2 + d];
    }
  }
  y[(static_cast<int64_t>(b) * NQ + qi) * H * D + h * D + d] = f32_to_bf16(l > 0.f ? o / l : 0.f);
}

}  // namespace
}  // namespace tf

extern "C" int64_t tf_query_read_workspace_size(int64_t batch, int64_t time, int64_t heads, int64_t queries,
                                                int64_t head_dim) {
  if (batch < 0 || time < 0 || heads < 1 || queries < 1 || head_dim < 1) return 0;
  const int64_t tiles = (time + tf::kTile - 1) / tf::kTile;
  return batch * heads * tiles * queries * (head_dim + 2) * static_cast<int64_t>(sizeof(float));
}

extern "C" int tf_query_read(const void* q, const void* kv, const int64_t* key_lengths, void* y, void* workspace,
                             int64_t workspace_bytes, int64_t batch, int64_t time, int64_t heads, int64_t queries,
                             int64_t head_dim, void* stream) {
  if (!q || !kv || !key_lengths || !y || !workspace) return TF_ERR_NULL;
  if (batch < 0 || time < 1 || heads < 1 || heads > 65535 || batch > 65535 || queries != 10 || head_dim != 32 ||
      batch * time * 2 * heads * head_dim > (int64_t(1) << 40))
    return TF_ERR_SHAPE;
  if (workspace_bytes < tf_query_read_workspace_size(batch, time, heads, queries, head_dim)) return TF_ERR_SHAPE;
  if ((reinterpret_cast<uintptr_t>(kv) & 15) || (reinterpret_cast<uintptr_t>(workspace) & 3)) return TF_ERR_SHAPE;
  if (batch == 0) return TF_OK;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int tiles = static_cast<int>((time + tf::kTile - 1) / tf::kTile);
  if (tiles > 65535 * 16) return TF_ERR_SHAPE;
  float* part = static_cast<float*>(workspace);
  const float scale = 1.0f / sqrtf(static_cast<float>(head_dim));
  hipLaunchKernelGGL((tf::query_read_tiles_kernel<10, 32>),
                     dim3(static_cast<uint32_t>(tiles), static_cast<uint32_t>(heads), static_cast<uint32_t>(batch)),
                     dim3(64), 0, s, static_cast<const uint16_t*>(q), static_cast<const uint16_t*>(kv), key_lengths,
                     part, static_cast<int>(time), static_cast<int>(heads), tiles, scale);
  if (const int rc = tf::launch_status()) return rc;
  hipLaunchKernelGGL((tf::query_read_merge_kernel<10, 32>),
                     dim3(static_cast<uint32_t>(heads), static_cast<uint32_t>(batch)), dim3(10 * 32), 0, s, part,
                     static_cast<uint16_t*>(y), static_cast<int>(heads), tiles);
  return tf::launch_status();
}
