// Generic fused Mamba-3 SISO recurrence: fp32 FMA arithmetic in LDS, any
// operand dtype (fp32/bf16/fp16), N <= 128 (even), P <= 64, R <= N/2.
//
// One workgroup per (head, batch) walks the sequence in 64-step chunks, the
// way the reference kernel does (src/trifusion_l4/mamba_fused.py:72-152), and
// rounds intermediate values to the operand dtypes at the same points:
// qr -> q dtype, kr -> k dtype (:127-132), the state copy used by qr.S^T -> q
// dtype (:143), the decayed score -> v dtype (:146) and the decay-scaled v ->
// k dtype (:151-152). It is the kernel for shapes and dtypes the MFMA path does
// not take (fp32 operands, odd sizes) and an independent second implementation
// the MFMA kernel is tested against. Raw controls and the reversed walk follow
// the MFMA kernel's definitions (computed per step; row L-1-t for step t).
#include "mamba_internal.h"

// Every product and sum is rounded on its own, as the elementwise reference
// formulation rounds it: a multiply-add fused here or not, depending on how
// the compiler happens to schedule the surrounding code, moves the inputs of
// the bf16 rounding points by an ulp and flips rounded q/k elements.
#pragma clang fp contract(off)

namespace tf {
namespace {

constexpr int kThreads = 256;

// sigmoid with the correctly rounded-to-1-ulp expf rather than the fast
// hardware exp: the trapezoid weights feed the bf16 rounding of kr.
__device__ __forceinline__ float sigmoid_exact(float x) { return 1.0f / (1.0f + expf(-x)); }
constexpr int kNMax = 128;
constexpr int kPMax = 64;
constexpr int kStatePerThread = kNMax * kPMax / kThreads;

struct GenericShared {
  float qr[kChunk][kNMax + 1];
  float kr[kChunk][kNMax + 1];
  float v[kChunk][kPMax + 1];
  float sc[kChunk][kChunk + 1];
  float sr[kPMax][kNMax + 1];  // state rounded to q's dtype
  float cs[kChunk];
  float gamma[kChunk];
  float scale[kChunk];
  float qk[kChunk];
  float dt[kChunk];
  float rn[2][kChunk];  // B/C norm scales of the chunk's q and k rows
};

__global__ __launch_bounds__(kThreads) void mamba_generic_kernel(const tf_mamba_args a) {
  __shared__ GenericShared sh;
  const int h = blockIdx.x;
  const int b = blockIdx.y;
  const int tid = threadIdx.x;
  const int n_state = static_cast<int>(a.state);
  const int p_dim = static_cast<int>(a.head_dim);
  const int rot = static_cast<int>(a.rotary);
  const int T = static_cast<int>(a.time);
  const int qh = h / static_cast<int>(a.heads / a.qk_heads);
  const int L = valid_length(a, b);
  // reverse: step t < L reads and writes row L-1-t; steps >= L have no row
  const bool rev = a.reverse != 0;
  const int tlim = rev ? L : T;
  auto row = [&](int t) -> int64_t { return rev ? L - 1 - t : t; };
  const bool raw = a.dt_bias != nullptr;
  const bool norm = a.q_norm != nullptr;
  const float step_bias = raw ? a.dt_bias[h] : 0.f;

  const int64_t qo = b * a.q_stride[0] + qh * a.q_stride[2];
  const int64_t ko = b * a.k_stride[0] + qh * a.k_stride[2];
  const int64_t vo = b * a.v_stride[0] + h * a.v_stride[2];
  const int64_t zo = b * a.z_stride[0] + h * a.z_stride[2];
  const int64_t oo = b * a.out_stride[0] + h * a.out_stride[2];
  const int64_t go = b * a.angles_stride[0] + h * a.angles_stride[2];
  const int64_t ao = b * a.adt_stride[0] + h * a.adt_stride[1];
  const int64_t dto = b * a.dt_stride[0] + h * a.dt_stride[1];
  const int64_t tro = b * a.trap_stride[0] + h * a.trap_stride[1];

  float state[kStatePerThread];
#pragma unroll
  for (int j = 0; j < kStatePerThread; ++j) state[j] = 0.f;
  for (int e = tid; e < kPMax * (kNMax + 1); e += kThreads) (&sh.sr[0][0])[e] = 0.f;
  double carry = 0.0;  // phase carry of pair `tid` (tid < N/2), kept in fp64
  const float skip = a.d[h];
  const int nchunks = (L + kChunk - 1) / kChunk;

  for (int c = 0; c < nchunks; ++c) {
    const int t0 = c * kChunk;
    if (tid < kChunk) {
      const int t = t0 + tid;
      const bool valid = t < L;
      const bool next = t + 1 < tlim;
      float dt = valid ? load_f32(a.dt, a.dt_dtype, dto + row(t) * a.dt_stride[2]) : 0.f;
      float dn = next ? load_f32(a.dt, a.dt_dtype, dto + row(t + 1) * a.dt_stride[2]) : 0.f;
      float ad = valid ? load_f32(a.adt, a.adt_dtype, ao + row(t) * a.adt_stride[2]) : 0.f;
      if (raw) {  // controls from the raw a/ddt columns (primitives.py:209-214)
        dt = valid ? control_step(dt, step_bias) : 0.f;
        dn = next ? control_step(dn, step_bias) : 0.f;
        ad = valid ? control_decay(ad, dt, a.a_floor) : 0.f;
      }
      const float tr =
          sigmoid_exact(valid ? load_f32(a.trap, a.trap_dtype, tro + row(t) * a.trap_stride[2]) : 0.f);
      const float tn =
          sigmoid_exact(next ? load_f32(a.trap, a.trap_dtype, tro + row(t + 1) * a.trap_stride[2]) : 0.f);
      const float gamma = dt * tr;
      const float da = ad * kLog2e;
      sh.cs[tid] = wave_inclusive_scan(da);
      sh.gamma[tid] = gamma;
      sh.scale[tid] = dn * (1.f - tn) + gamma;
      sh.dt[tid] = dt;
    }
    for (int e = tid; e < kChunk * n_state; e += kThreads) {
      const int r = e / n_state, n = e - r * n_state;
      const int t = t0 + r;
      const bool valid = t < L;
      sh.qr[r][n] = valid ? load_f32(a.q, a.q_dtype, qo + row(t) * a.q_stride[1] + n * a.q_stride[3]) : 0.f;
      sh.kr[r][n] = valid ? load_f32(a.k, a.k_dtype, ko + row(t) * a.k_stride[1] + n * a.k_stride[3]) : 0.f;
    }
    for (int e = tid; e < kChunk * p_dim; e += kThreads) {
      const int r = e / p_dim, p = e - r * p_dim;
      const int t = t0 + r;
      sh.v[r][p] = t < L ? load_f32(a.v, a.v_dtype, vo + row(t) * a.v_stride[1] + p * a.v_stride[3]) : 0.f;
    }
    __syncthreads();
    if (norm) {
      // B/C RMSNorm of the raw rows (mamba.py:56-57, kernels/__init__.py:10-12):
      // one thread per row of q (tid < 64) and of k
      if (tid < 2 * kChunk) {
        const int r = tid & (kChunk - 1);
        const float* x = tid < kChunk ? sh.qr[r] : sh.kr[r];
        float ss = 0.f;
        for (int n = 0; n < n_state; ++n) ss += x[n] * x[n];
        sh.rn[tid >> 6][r] = rsqrtf(ss / static_cast<float>(n_state) + a.norm_eps);
      }
      __syncthreads();
    }
    // biases, after the norm rounded to the operand dtype as the norm's output is
    for (int e = tid; e < kChunk * n_state; e += kThreads) {
      const int r = e / n_state, n = e - r * n_state;
      float qv = sh.qr[r][n], kv = sh.kr[r][n];
      if (norm) {
        qv = round_to(qv * sh.rn[0][r] * a.q_norm[n], a.q_dtype);
        kv = round_to(kv * sh.rn[1][r] * a.k_norm[n], a.k_dtype);
      }
      sh.qr[r][n] = qv + a.qb[h * n_state + n];
      sh.kr[r][n] = kv + a.kb[h * n_state + n];
    }
    __syncthreads();
    // skip term from the unrotated biased vectors (mamba_fused.py:124)
    if (tid < kChunk) {
      float s = 0.f;
      for (int n = 0; n < n_state; ++n) s += sh.qr[tid][n] * sh.kr[tid][n];
      sh.qk[tid] = s * sh.gamma[tid];
    }
    __syncthreads();
    // phase scan + rotary + scale + rounding, one thread per pair (mamba_fused.py:102-135).
    // The phase is accumulated in fp64 and rounded to fp32 once, so it carries no
    // fp32 summation noise into the bf16 rounding of qr/kr.
    if (tid < n_state / 2) {
      const int i = tid;
      double cum = 0.0;
      for (int r = 0; r < kChunk; ++r) {
        const int t = t0 + r;
        const bool valid = t < L;
        float co = 1.f, si = 0.f;
        if (i < rot) {
          const float th =
              valid ? load_f32(a.angles, a.angles_dtype, go + row(t) * a.angles_stride[1] + i * a.angles_stride[3])
                    : 0.f;
          cum += tanh(static_cast<double>(th)) * kPiD * static_cast<double>(sh.dt[r]);
          const float ph = static_cast<float>(mod_two_pi_d(cum + carry));
          co = cosf(ph);
          si = sinf(ph);
        }
        const float q0 = sh.qr[r][2 * i], q1 = sh.qr[r][2 * i + 1];
        const float k0 = sh.kr[r][2 * i], k1 = sh.kr[r][2 * i + 1];
        const float s = sh.scale[r];
        sh.qr[r][2 * i] = valid ? round_to(q0 * co - q1 * si, a.q_dtype) : 0.f;
        sh.qr[r][2 * i + 1] = valid ? round_to(q0 * si + q1 * co, a.q_dtype) : 0.f;
        sh.kr[r][2 * i] = valid ? round_to((k0 * co - k1 * si) * s, a.k_dtype) : 0.f;
        sh.kr[r][2 * i + 1] = valid ? round_to((k0 * si + k1 * co) * s, a.k_dtype) : 0.f;
      }
      if (i < rot) carry = mod_two_pi_d(carry + cum);
    }
    __syncthreads();
    // strictly causal decayed scores, rounded to v's dtype (mamba_fused.py:144-146)
    for (int e = tid; e < kChunk * kChunk; e += kThreads) {
      const int t = e / kChunk, u = e - t * kChunk;
      float val = 0.f;
      if (u < t) {
        float s = 0.f;
        for (int n = 0; n < n_state; ++n) s += sh.qr[t][n] * sh.kr[u][n];
        val = round_to(s * exp2f(fminf(sh.cs[t] - sh.cs[u], 0.f)), a.v_dtype);
      }
      sh.sc[t][u] = val;
    }
    __syncthreads();
    // outputs (mamba_fused.py:143-149)
    for (int e = tid; e < kChunk * p_dim; e += kThreads) {
      const int r = e / p_dim, p = e - r * p_dim;
      const int t = t0 + r;
      if (t >= T) continue;
      float y = 0.f;
      if (t < L) {
        float inter = 0.f;
        for (int n = 0; n < n_state; ++n) inter += sh.qr[r][n] * sh.sr[p][n];
        float intra = 0.f;
        for (int u = 0; u < r; ++u) intra += sh.sc[r][u] * sh.v[u][p];
        y = inter * exp2f(sh.cs[r]) + intra + (skip + sh.qk[r]) * sh.v[r][p];
        const float zz = load_f32(a.z, a.z_dtype, zo + row(t) * a.z_stride[1] + p * a.z_stride[3]);
        y *= zz * sigmoidf(zz);
      }
      // rows in [L, T) are the same rows in either direction
      store_f32(a.out, a.out_dtype, oo + (t < L ? row(t) : t) * a.out_stride[1] + p * a.out_stride[3], y);
    }
    // state update S <- S*2^tot + round_k(v*2^(tot-cs))^T kr (mamba_fused.py:150-152)
    const float tot = sh.cs[kChunk - 1];
    const float decay = exp2f(tot);
#pragma unroll
    for (int j = 0; j < kStatePerThread; ++j) {
      const int e = tid + j * kThreads;
      if (e < p_dim * n_state) {
        const int p = e / n_state, n = e - p * n_state;
        float acc = 0.f;
        for (int u = 0; u < kChunk; ++u)
          acc += round_to(sh.v[u][p] * exp2f(tot - sh.cs[u]), a.k_dtype) * sh.kr[u][n];
        state[j] = state[j] * decay + acc;
      }
    }
    __syncthreads();
#pragma unroll
    for (int j = 0; j < kStatePerThread; ++j) {
      const int e = tid + j * kThreads;
      if (e < p_dim * n_state) {
        const int p = e / n_state, n = e - p * n_state;
        sh.sr[p][n] = round_to(state[j], a.q_dtype);
      }
    }
    __syncthreads();
  }
  // rows past the last processed chunk (only when lengths < T)
  for (int e = nchunks * kChunk * p_dim + tid; e < T * p_dim; e += kThreads) {
    const int t = e / p_dim, p = e - t * p_dim;
    store_f32(a.out, a.out_dtype, oo + t * a.out_stride[1] + p * a.out_stride[3], 0.f);
  }
}

}  // namespace

bool generic_supported(const tf_mamba_args& a) {
  return a.state <= kNMax && a.head_dim <= kPMax;
}

int launch_generic(const tf_mamba_args& a, hipStream_t stream) {
  hipLaunchKernelGGL(mamba_generic_kernel, dim3(static_cast<uint32_t>(a.heads), static_cast<uint32_t>(a.batch)),
                     dim3(kThreads), 0, stream, a);
  return launch_status();
}

}  // namespace tf
