/*
 * C ABI of the MI355X (gfx950) TriFusion-FP inference kernels.
 *
 * Every entry point takes plain pointers, element counts and element strides,
 * enqueues its kernels on the given HIP stream (a hipStream_t passed as void*;
 * NULL is the legacy default stream) and returns a tf_status. Nothing is
 * allocated, nothing is synchronised and no host memory is read after the
 * call returns, so every entry point may be recorded into a HIP graph.
 * Concurrent calls on different streams are independent; the library keeps no
 * mutable global state besides a once-initialised device-property cache.
 *
 * Strides are in elements (not bytes) and may be 0 (broadcast) or any other
 * value; dtypes are tf_dtype codes.
 */
#ifndef TRIFUSION_AMD_H
#define TRIFUSION_AMD_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef enum tf_dtype {
  TF_FLOAT32 = 0,
  TF_BFLOAT16 = 1,
  TF_FLOAT16 = 2,
} tf_dtype;

typedef enum tf_status {
  TF_OK = 0,
  TF_ERR_NULL = 1,        /* a required pointer is NULL */
  TF_ERR_SHAPE = 2,       /* unsupported or inconsistent dimensions */
  TF_ERR_DTYPE = 3,       /* unsupported dtype code or combination */
  TF_ERR_STRIDE = 4,      /* layout the selected kernel cannot read */
  TF_ERR_VARIANT = 5,     /* requested kernel variant cannot run these arguments */
  TF_ERR_LAUNCH = 6,      /* the HIP runtime rejected the launch */
  TF_ERR_WORKSPACE = 7,   /* needs more scratch than tf_fused_mamba_static holds */
} tf_status;

/* Kernel selection for tf_fused_mamba. */
typedef enum tf_mamba_variant {
  TF_MAMBA_AUTO = 0,      /* pipelined kernel when supported, else the chunked
                             kernel when supported, else generic */
  TF_MAMBA_GENERIC = 1,   /* fp32-FMA kernel: any dtype, N <= 128, P <= 64 */
  TF_MAMBA_MFMA = 2,      /* bf16 MFMA chunked-scan kernel (gfx950) */
  TF_MAMBA_PIPE = 3,      /* bf16 MFMA pipelined walk, N = P = 64 (gfx950) */
} tf_mamba_variant;

/*
 * Operands of the fused Mamba-3 SISO recurrence. Shapes (reference
 * src/trifusion_l4/mamba_fused.py:155-191 and docs/api.md:61-74):
 *   q, k          [B, T, Hq, N]   C and B projections (H % Hq == 0)
 *   v, z          [B, T, H, P]    x and gate
 *   adt, dt, trap [B, H, T]       signed decay*dt, softplus(dt), pre-sigmoid trap
 *   qb, kb        [H, N]          fp32, contiguous (C and B biases)
 *   angles        [B, T, H, R]    raw pre-tanh rotary controls, R <= N/2
 *   d             [H]             fp32, contiguous (skip D)
 *   out           [B, T, H, P]
 *   lengths       [B] int64 or NULL: rows t >= lengths[b] are written as 0 and
 *                 chunks wholly past the length are skipped (extension; NULL
 *                 reproduces the reference exactly).
 *   workspace     device scratch of workspace_bytes, or NULL/0 (extension).
 *                 When it holds at least tf_fused_mamba_workspace_size(args)
 *                 bytes (> 0), long sequences over few (batch, head) units run
 *                 chunk-parallel: the time axis is cut into segments that run
 *                 on separate workgroups, joined by a scan of their states.
 *                 Otherwise each unit is walked by one workgroup.
 *   dt_bias       [H] fp32 or NULL (extension). Non-NULL selects raw controls:
 *                 adt and dt then point at the raw `a` and `ddt` columns of
 *                 the in-projection (fp32 or bf16, both of one dtype, any
 *                 [B, H, T] strides), and each step's controls are computed in
 *                 the recurrence as mamba_controls computes them
 *                 (src/trifusion_l4/kernels/primitives.py:190-216):
 *                   dt  = softplus(ddt + dt_bias[h])   (linear above 20)
 *                   adt = min(-(relu(a) + 1/(1 - min(a, 0))), -a_floor) * dt
 *                 so no [B, H, T] control tensors are written or read.
 *   a_floor       decay floor of the raw controls (the reference uses 1e-4).
 *   reverse       1 (extension): each batch row runs over its valid prefix
 *                 (L = lengths[b], or T) in reverse. Step t < L reads row
 *                 L-1-t of every time-indexed operand and writes row L-1-t of
 *                 out; rows t >= L are written as 0. The result equals the
 *                 reference's reverse_valid(fused_mamba(reverse_valid(...)))
 *                 of the backward direction (src/trifusion_l4/model.py:174-179,
 *                 kernels/__init__.py:44-55) with no reversed copies.
 *   q_norm, k_norm [N] fp32, contiguous, or both NULL (extension). Non-NULL:
 *                 q and k are the raw C and B columns of the in-projection, and
 *                 the block's C/B RMSNorm (src/trifusion_l4/mamba.py:56-57,
 *                 kernels/__init__.py:10-12) is applied to each row as it is
 *                 loaded, rounded to the operand dtype as the separate norm's
 *                 output is:
 *                   x <- round(x * rsqrt(mean_n(x^2) + norm_eps) * w)
 *                 so no normalised [B, T, Hq, N] copies are written or read.
 *   norm_eps      epsilon of those norms (the reference uses 1e-5).
 * Stride arrays follow the dimension order above.
 */
typedef struct tf_mamba_args {
  const void *q, *k, *v, *adt, *dt, *trap, *angles, *z;
  const float *qb, *kb, *d;
  void *out;
  const int64_t *lengths;
  int32_t q_dtype, k_dtype, v_dtype, z_dtype;
  int32_t adt_dtype, dt_dtype, trap_dtype, angles_dtype, out_dtype;
  int32_t variant;
  int64_t q_stride[4], k_stride[4], v_stride[4], z_stride[4];
  int64_t angles_stride[4], out_stride[4];
  int64_t adt_stride[3], dt_stride[3], trap_stride[3];
  int64_t batch, time, heads, qk_heads, state, head_dim, rotary;
  void *workspace;
  int64_t workspace_bytes;
  const float *dt_bias;
  float a_floor;
  int32_t reverse;
  const float *q_norm, *k_norm;
  float norm_eps;
} tf_mamba_args;

/*
 * Fused recurrence forward. Replaces the Triton launch of `_fused` in
 * src/trifusion_l4/mamba_fused.py:155-191 (shape check :159-160, launch
 * :162-190), generalised to N in {16,32,64,128}, P in {32,64}, R <= N/2.
 */
int tf_fused_mamba(const tf_mamba_args *args, void *stream);

/*
 * Scratch bytes the chunk-parallel path wants for these arguments, or 0 when
 * one workgroup per unit is used (short sequences, many units, or a kernel
 * without a segmented form). The reference has no counterpart: its Triton
 * kernel always walks a unit serially (src/trifusion_l4/mamba_fused.py:93-152).
 * Negative: a tf_status for invalid arguments.
 */
int64_t tf_fused_mamba_workspace_size(const tf_mamba_args *args);

/* Which kernel TF_MAMBA_AUTO would run for these arguments (1, 2 or 3), or a
 * negative tf_status if no kernel can run them. */
int tf_fused_mamba_variant(const tf_mamba_args *args);

/*
 * tf_fused_mamba without a caller workspace, for callers that cannot allocate
 * (code under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc). No counterpart in the reference. args->workspace is ignored: the
 * chunk-parallel form takes its scratch from a library-owned device array of
 * tf_fused_mamba_static_scratch_bytes() (16 MiB) that every device holds until
 * the process ends. Arguments whose tf_fused_mamba_workspace_size exceeds it
 * return TF_ERR_WORKSPACE and launch nothing. Calls allocate nothing; the
 * first call on a device that needs scratch looks up that device's copy of the
 * array (hipGetSymbolAddress, which may load the library's code object): make
 * that first call outside graph capture. A failed lookup returns TF_ERR_LAUNCH
 * and is tried again on the next call. Every call
 * on one device shares that device's array, and the kernels rewrite all of the
 * scratch they read within the call (nothing needs to start at zero), so calls
 * that overlap on one device (different streams, no ordering) race: serialise
 * them. Outputs equal tf_fused_mamba's for the same arguments.
 */
int tf_fused_mamba_static(const tf_mamba_args *args, void *stream);

/* Size in bytes of the scratch array tf_fused_mamba_static uses. */
int64_t tf_fused_mamba_static_scratch_bytes(void);

/*
 * Row RMSNorm: y[r,:] = x[r,:] * rsqrt(mean(x[r,:]^2) + eps) * w, fp32
 * statistics. Row r of x starts at x + r * x_row_stride (elements; the row
 * itself is contiguous, so strided column slices of a projection need no
 * copy); y is contiguous [rows, d]; w fp32 [d]; d <= 4096.
 * Replaces `_norm` MODE 0 / `rms` (src/trifusion_l4/kernels/native.py:8-39,
 * 42-70) and RMSNorm.forward (src/trifusion_l4/kernels/__init__.py:15-28).
 */
int tf_rmsnorm(const void *x, int32_t x_dtype, int64_t x_row_stride, const float *w,
               void *y, int32_t y_dtype, int64_t rows, int64_t d, float eps,
               void *stream);

/*
 * Residual add fused with the following RMSNorm:
 *   s = (a + b) * mask[row]   (fp32 math, stored as s_dtype)
 *   y = rmsnorm(s) * w        (stored as y_dtype)
 * mask is uint8 [rows] or NULL; all tensors contiguous [rows, d], d <= 4096.
 * The norm reads s as stored. Combines `add` (native.py:81-100) and the next
 * block's `_norm` MODE 0 (native.py:8-39) in one pass over the rows.
 */
int tf_add_rmsnorm(const void *a, int32_t a_dtype, const void *b, int32_t b_dtype,
                   const uint8_t *mask, const float *w, void *s, int32_t s_dtype,
                   void *y, int32_t y_dtype, int64_t rows, int64_t d, float eps,
                   void *stream);

/*
 * SwiGLU: y[r, j] = silu(x[r, j]) * x[r, d + j], fp32 math. x contiguous
 * [rows, 2d], y contiguous [rows, d]. Replaces `swiglu`/`_swiglu`
 * (src/trifusion_l4/kernels/__init__.py:31-41, kernels/primitives.py:25-37).
 */
int tf_swiglu(const void *x, void *y, int32_t dtype, int64_t rows, int64_t d,
              void *stream);

/*
 * Row mask: y[r,:] = mask[r] ? x[r,:] : 0 over contiguous [rows, d].
 * Replaces `mask_buffer`/`_mask` (src/trifusion_l4/kernels/buffers.py:6-10,
 * kernels/primitives.py:65-70).
 */
int tf_mask_rows(const void *x, void *y, int32_t dtype, const uint8_t *mask,
                 int64_t rows, int64_t d, void *stream);

/*
 * y = a + b in fp32 (rows with mask[r] == 0 give 0 when mask is non-NULL),
 * stored as y_dtype; contiguous [rows, d]. Replaces `add`/`_add`
 * (src/trifusion_l4/kernels/native.py:81-100).
 */
int tf_add(const void *a, int32_t a_dtype, const void *b, int32_t b_dtype,
           const uint8_t *mask, void *y, int32_t y_dtype, int64_t rows, int64_t d,
           void *stream);

/*
 * Mamba-3 controls: for a, ddt read as [B, T, H] with strides (sb, st, 1):
 *   dt  = softplus(ddt + bias[h])  (linear above 20)
 *   adt = -max(relu(a) + 1/(1 - min(a, 0)), floor) * dt
 * written as contiguous fp32 [B, H, T]. Replaces `mamba_controls`/`_controls`
 * (src/trifusion_l4/kernels/buffers.py:82-101, kernels/primitives.py:190-216).
 */
int tf_mamba_controls(const void *a, const void *ddt, int32_t dtype, int64_t sb,
                      int64_t st, const float *bias, float *adt, float *dt,
                      int64_t batch, int64_t time, int64_t heads, float floor_,
                      void *stream);

/*
 * Masked mean over time: y[b, :] = sum_{t < lengths[b]} x[b, t, :] / lengths[b]
 * in fp32; x contiguous [B, T, D], y fp32 [B, D]. Replaces the global-feature
 * pooling of src/trifusion_l4/decoder.py:60-62.
 * When B * D is too small to occupy the whole GPU with one workgroup per
 * 128-byte column slice, the time axis is split and the partial sums go to
 * `workspace` (tf_masked_mean_workspace_size bytes, 4-byte aligned), then are
 * added in split order. With a NULL or smaller workspace the mean is computed
 * without the split. For a given split, the result does not depend on timing.
 */
int tf_masked_mean(const void *x, int32_t dtype, const int64_t *lengths, float *y,
                   int64_t batch, int64_t time, int64_t d, void *workspace,
                   int64_t workspace_bytes, void *stream);

/* Workspace bytes tf_masked_mean uses for these sizes (0: no time split). */
int64_t tf_masked_mean_workspace_size(int32_t dtype, int64_t batch, int64_t time, int64_t d);

/* Row mask from lengths: mask[b*T + t] = t < lengths[b] (uint8). Replaces
 * time_mask (src/trifusion_l4/masking.py:6-7) on the device. */
int tf_time_mask(const int64_t *lengths, uint8_t *mask, int64_t batch, int64_t time,
                 void *stream);

/*
 * Valid-prefix reversal: for x, y contiguous [B, T, D],
 *   y[b, t, :] = x[b, L-1-t, :] for t < L = clamp(lengths[b], 0, T), else 0.
 * Replaces reverse_valid/_reverse (src/trifusion_l4/kernels/__init__.py:44-55,
 * kernels/primitives.py:40-47). x and y must not overlap.
 */
int tf_reverse_valid(const void *x, void *y, int32_t dtype, const int64_t *lengths,
                     int64_t batch, int64_t time, int64_t d, void *stream);

/*
 * Mean of the two directions fused with RMSNorm:
 *   s = (a + b) * 0.5 (fp32),  y = s * rsqrt(mean(s^2) + eps) * w  (fp32 out)
 * over contiguous [rows, d], d <= 4096. Replaces mean_norm (`_norm` MODE 2,
 * src/trifusion_l4/kernels/native.py:8-39,77-78).
 */
int tf_mean_rmsnorm(const void *a, int32_t a_dtype, const void *b, int32_t b_dtype,
                    const float *w, float *y, int64_t rows, int64_t d, float eps,
                    void *stream);

/*
 * RMSNorm of a masked row, writing the masked row too:
 *   s = mask[row] ? x : 0   (stored fp32),   y = rmsnorm(s) * w   (y_dtype)
 * over contiguous [rows, d], d <= 4096; mask uint8 [rows] or NULL. The first
 * residual of the encoder: the masked stem output (masking.py:10-11) and the
 * first block's `_norm` MODE 0 (src/trifusion_l4/kernels/native.py:8-39) in one
 * pass.
 */
int tf_mask_rmsnorm(const void *x, int32_t x_dtype, const uint8_t *mask, const float *w, float *s,
                    void *y, int32_t y_dtype, int64_t rows, int64_t d, float eps, void *stream);

/*
 * Two RMSNorms per row: row r holds two groups of d elements at
 * x + r * x_row_stride (0 = 2d); group g is normalised with w_g into the
 * contiguous y[r, g, :]. The B and C norms of the Mamba-3 block
 * (src/trifusion_l4/mamba.py:56-57: B_norm and C_norm over adjacent columns of
 * the in-projection) in one launch instead of two.
 */
int tf_rmsnorm_pair(const void *x, int32_t x_dtype, int64_t x_row_stride, const float *w0,
                    const float *w1, void *y, int32_t y_dtype, int64_t rows, int64_t d, float eps,
                    void *stream);

/*
 * Channel mix and framing of the encoder's strided Conv1d stem: for audio fp32
 * contiguous [B, C, N] and channels int64 [B],
 *   mono[b, n] = sum_{c < min(channels[b], C)} audio[b, c, n] / channels[b],
 *   framed[b, t, k] = bf16(mono[b, t*stride + k - pad]) for k < kernel (0 outside
 *   [0, N)), and 0 for kernel <= k < width,
 * into contiguous bf16 [B, frames, width] (width % 8 == 0, 16-byte aligned),
 * frames = (N + 2 pad - kernel) / stride + 1. The stem is then one GEMM.
 * No counterpart in the reference, whose front end is an STFT
 * (src/trifusion_l4/front.py); this is the front of the benchmark encoder.
 */
int tf_frame_audio(const float *audio, const int64_t *channels, void *framed, int64_t batch,
                   int64_t chans, int64_t samples, int64_t frames, int64_t kernel, int64_t width,
                   int64_t stride, int64_t pad, void *stream);

/*
 * Valid frames and row mask from sample lengths:
 *   frames[b] = clamp(floor(lengths[b] / stride), 1, T),  mask[b, t] = t < frames[b]
 * (int64 [B] and uint8 [B, T]). The hop-count frame lengths the reference front
 * end derives from sample lengths (src/trifusion_l4/front.py:62-67,90:
 * floor division by the 160-sample hop) fused with time_mask
 * (src/trifusion_l4/masking.py:6-7).
 */
int tf_frames_mask(const int64_t *lengths, int64_t stride, int64_t *frames, uint8_t *mask,
                   int64_t batch, int64_t time, void *stream);

/*
 * Small bf16 linear layer on an fp32 input, as an autocast forward computes it:
 *   y[b, o] = bf16(sum_k bf16(x[b, k]) * bf16(w[o, k]) + bf16(bias[o]))  (fp32 out)
 * x fp32 [B, D], w [O, D] and bias [O] (or NULL) of w_dtype. One launch for the
 * encoder head's cast, GEMM and cast; the reference's classifier heads are torch
 * Linear layers under autocast (src/trifusion_l4/decoder.py).
 */
int tf_small_linear(const float *x, const void *w, const void *bias, int32_t w_dtype, float *y,
                    int64_t batch, int64_t out_features, int64_t in_features, void *stream);

/* ---- Kernels of the TriFusion block and front end (reference model path) ---- */

/*
 * Masked depthwise convolution over time, "same" padding:
 *   y[b, t, c] = t < L_b ? sum_k x[b, t + k - K/2, c] * w[c, k] + bias[c] : 0
 * (sources outside [0, T) read 0; fp32 products and sums, each rounded; stored
 * in dtype). x, y contiguous [B, T, D]; w [D, K] (the Conv1d weight [D, 1, K]),
 * bias [D], both of dtype. Replaces depthwise_masked/_dw_forward
 * (src/trifusion_l4/kernels/buffers.py:13-32, kernels/primitives.py:74-88).
 */
int tf_depthwise_masked(const void *x, const void *w, const void *bias, int32_t dtype,
                        const int64_t *lengths, void *y, int64_t batch, int64_t time, int64_t d,
                        int64_t k, void *stream);

/*
 * 4:1 masked average over time: y[b, j, c] = sum_{k<4, 4j+k < L_b} x[b, 4j+k, c] /
 * max(min(L_b - 4j, 4), 1), y contiguous [B, ceil(T/4), D]. Replaces Pool4
 * (src/trifusion_l4/kernels/buffers.py:35-44, kernels/primitives.py:91-114).
 */
int tf_pool4(const void *x, int32_t dtype, const int64_t *lengths, void *y, int64_t batch, int64_t time,
             int64_t d, void *stream);

/*
 * Rotary Q/K/V packing: x contiguous [B, T, 3 H D] -> y [3, B, H, T, D]; for q and
 * k each interleaved pair (a, z) becomes (a cos - z sin, a sin + z cos) with
 * cos/sin fp32 [T, D/2]; v is copied. Replaces RotaryQKV/_rotary_qkv
 * (src/trifusion_l4/kernels/buffers.py:46-56, kernels/primitives.py:117-151).
 */
int tf_rotary_qkv(const void *x, int32_t dtype, const float *cos_t, const float *sin_t, void *y,
                  int64_t batch, int64_t time, int64_t heads, int64_t head_dim, void *stream);

/*
 * Channel RMSNorm of a [B, C, T, F] map with element strides strides[4], written
 * contiguous [B, T, F, C]: rows with t >= L_b are 0; y = round(x r w) and, when
 * silu is non-zero, y * sigmoid(y) (C <= 256). Replaces front_norm/_front_norm
 * (src/trifusion_l4/kernels/buffers.py:58-80, kernels/primitives.py:154-188).
 */
int tf_front_norm(const void *x, int32_t dtype, const int64_t *strides, const float *w,
                  const int64_t *lengths, void *y, int64_t batch, int64_t chans, int64_t time,
                  int64_t freq, float eps, int32_t silu, void *stream);

/*
 * Linear interpolation from the pooled grid back to frames:
 *   y[b, t, c] = t < L_b ? a + (z - a) * alpha[b, t] : 0,
 *   a = low[b, left[b, t], c], z = low[b, right[b, t], c]
 * low [B, LT, D], left/right int64 [B, T], alpha fp32 [B, T], y [B, T, D].
 * Replaces interpolate/_interpolate (src/trifusion_l4/kernels/native.py:104-133).
 */
int tf_interpolate(const void *low, int32_t dtype, const int64_t *left, const int64_t *right,
                   const float *alpha, const int64_t *lengths, void *y, int64_t batch, int64_t time,
                   int64_t low_time, int64_t d, void *stream);

/*
 * tf_interpolate followed by RMSNorm of each output row, in one pass:
 *   v = dtype(interpolated row), y = dtype(v rsqrt(mean(v^2) + eps) w)
 * w fp32 [D]; D a multiple of 8 up to 4096; low, y and w 16-byte aligned. The
 * same values as tf_interpolate then tf_rmsnorm. Replaces self.an(attention(h))
 * of the TriFusion block, whose attention ends in grids.interpolate
 * (src/trifusion_l4/model.py:104,160).
 */
int tf_interpolate_rmsnorm(const void *low, int32_t dtype, const int64_t *left, const int64_t *right,
                           const float *alpha, const int64_t *lengths, const float *w, float eps, void *y,
                           int64_t batch, int64_t time, int64_t low_time, int64_t d, void *stream);

/*
 * Eight frequency bands of a [B, C, T, F] map (strides[4]), written contiguous
 * [B, T, 8, C]: band i averages frequencies floor(i F/8) .. ceil((i+1) F/8) - 1,
 * the adaptive average pool of src/trifusion_l4/front.py:94-101. Replaces
 * bands/_bands (src/trifusion_l4/kernels/native.py:142-163). F >= 8.
 */
int tf_bands(const void *x, int32_t dtype, const int64_t *strides, void *y, int64_t batch, int64_t chans,
             int64_t time, int64_t freq, void *stream);

/*
 * Evidence-gated RMSNorm: s = mask[r] ? x + a * 2 sigmoid(g) : 0 (fp32),
 * y = s rsqrt(mean(s^2) + eps) w, computed in fp32 and stored as y_dtype (fp32, or
 * bf16 for a consumer that casts it); x and y contiguous [rows, d] (x fp32); a and g
 * of ag_dtype, rows of d elements ag_stride apart (both halves of one [rows, 2d]
 * projection, or contiguous with ag_stride = d); mask uint8 [rows] or NULL.
 * Replaces evidence_norm (`_norm` MODE 1, src/trifusion_l4/kernels/native.py:9-39,73-74).
 */
int tf_evidence_norm(const float *x, const void *a, const void *g, int32_t ag_dtype, int64_t ag_stride,
                     const uint8_t *mask, const float *w, void *y, int32_t y_dtype, int64_t rows, int64_t d,
                     float eps, void *stream);

/*
 * Sigmoid-gated concatenation: y[r, k d + j] = x[r, k d + j] * 2 sigmoid(gate[r, k])
 * for the three branches k < 3; x, y [rows, 3 d], gate [rows, 3], one dtype.
 * Replaces gated_concat/_gate (src/trifusion_l4/kernels/__init__.py:58-82,
 * kernels/primitives.py:51-63).
 */
int tf_gated_concat(const void *x, const void *gate, int32_t dtype, void *y, int64_t rows, int64_t d,
                    void *stream);

/*
 * First half of a front-end CNN stage, channels-last: y = silu(norm(mask(conv(x))))
 * with conv the 3x3 convolution of stride (stride, 2) and padding 1 and norm the
 * channel RMSNorm with weight norm_w and eps; rows t >= L_b of the output grid are 0.
 * The convolution output and the norm output are rounded to bf16, as in the bf16
 * autocast forward. x is fp32 [B, Ti, Fi] (cin == 1, rounded to bf16 on read) or bf16
 * [B, Ti, Fi, cin] (cin 32 or 64); w bf16 [9, cout, cin] (tap-major: tap = 3 dy + dx);
 * y bf16 [B, To, Fo, cout], To = (Ti - 1) / stride + 1, Fo = (Fi - 1) / 2 + 1;
 * cout 32 (cin 1) or 32, 64, 128. Replaces conv1 + front_norm(silu=True) of
 * CNNStage.forward (src/trifusion_l4/front.py:19-36, kernels/buffers.py:58-80).
 */
int tf_front_conv1(const void *x, int32_t x_dtype, const void *w, const float *norm_w,
                   const int64_t *lengths, void *y, int64_t batch, int64_t time_in, int64_t freq_in,
                   int64_t cin, int64_t cout, int64_t stride, float eps, void *stream);

/*
 * Second half of a front-end CNN stage: y = mask(silu(norm(mask(conv(h))) + mask(skip(x))))
 * with conv the 3x3 convolution (stride 1, padding 1) of h, the first half's output
 * [B, To, Fo, cout] bf16 with weight w bf16 [9, cout, cout], and skip the 1x1
 * convolution of stride (stride, 2) of the stage input x (fp32 [B, Ti, Fi] with cin 1,
 * or bf16 [B, Ti, Fi, cin] with cin 32 or 64) with weight w_skip bf16 [cout, cin].
 * Every intermediate is rounded to bf16 as in the autocast forward; y bf16
 * [B, To, Fo, cout], cout 32, 64 or 128. Replaces conv2 + front_norm + the skip,
 * residual and SiLU of CNNStage.forward (src/trifusion_l4/front.py:19-43).
 */
int tf_front_conv2(const void *h, const void *w, const float *norm_w, const void *x, int32_t x_dtype,
                   const void *w_skip, const int64_t *lengths, void *y, int64_t batch, int64_t time_in,
                   int64_t freq_in, int64_t cin, int64_t cout, int64_t stride, float eps, void *stream);

/*
 * Start of a TriFusion block under bf16 autocast: xm = mask(x) (rows t >= L_b zero,
 * fp32), h = bf16(RMSNorm(xm) w) [B, T, d], and the 4:1 pooled grid
 * p = bf16(mean of the fp32 norm rows 4j .. 4j+3 below L_b) [B, ceil(T/4), d].
 * d % 8 == 0, d <= 4096; 16-byte aligned pointers. Replaces mask_buffer + pre +
 * Grids.pool and the casts before local.up and attention.qkv
 * (src/trifusion_l4/model.py:144-160, masking.py:59-67, kernels/buffers.py:13-44).
 */
int tf_block_pre(const float *x, const int64_t *lengths, const float *w, float eps, float *xm, void *h, void *p,
                 int64_t batch, int64_t time, int64_t d, void *stream);

/*
 * tf_block_pre of x + addend (addend bf16 [B, T, d], added in fp32 before the
 * mask): the previous block's closing masked residual add (tf_add of the
 * residual and the FFN down-projection, src/trifusion_l4/model.py:199) and this
 * block's start in one launch, the values of the two.
 */
int tf_block_pre_add(const float *x, const void *addend, const int64_t *lengths, const float *w, float eps,
                     float *xm, void *h, void *p, int64_t batch, int64_t time, int64_t d, void *stream);

/*
 * RMSNorm of bf16 rows [rows, d] rounded to bf16, then SiLU rounded to bf16.
 * Replaces F.silu(self.norm(h)) of LocalCNN (src/trifusion_l4/model.py:74).
 */
int tf_norm_silu(const void *x, const float *w, void *y, int64_t rows, int64_t d, float eps, void *stream);

/*
 * F.glu over the last dim of up [B, T, 2d] (bf16(a sigmoid(b))), then the masked
 * depthwise conv of kernel k (3 or 7, padding k/2; w bf16 [d, k], bias bf16 [d]):
 * y [B, T, d] bf16, rows t >= L_b zero. Replaces F.glu + depthwise_masked of
 * LocalCNN (src/trifusion_l4/model.py:73, kernels/buffers.py:13-32).
 */
int tf_glu_depthwise(const void *up, const void *w, const void *bias, const int64_t *lengths, void *y,
                     int64_t batch, int64_t time, int64_t d, int64_t k, void *stream);

/*
 * tf_glu_depthwise followed by tf_norm_silu in one launch (d a multiple of 8 up
 * to 1024, k 3 or 7; norm_w fp32 [d], 16-byte aligned): the values of the two
 * launches. Replaces the LocalCNN's glu -> depthwise conv -> norm -> silu
 * (src/trifusion_l4/model.py:73-76, kernels/buffers.py:13-32).
 */
int tf_glu_depthwise_norm_silu(const void *up, const void *w, const void *bias, const int64_t *lengths,
                               const float *norm_w, float eps, void *y, int64_t batch, int64_t time, int64_t d,
                               int64_t k, void *stream);

/*
 * Attention on the pooled grid: qkv bf16 [B, T, 3, H, D] (D 32 or 64); q and k
 * rotated by interleaved pairs with cos/sin fp32 [T, D/2] (contiguous, 16-byte
 * aligned, as qkv and y are) and rounded to bf16;
 * softmax(q k^T / sqrt(D)) v in fp32 over keys j < low_lengths[b]; y bf16
 * [B, T, H D]. Replaces RotaryQKV + masked_attention + the head merge of
 * GlobalAttention (src/trifusion_l4/model.py:84-104, attention.py:8-18).
 */
int tf_pooled_attention(const void *qkv, const float *cos_t, const float *sin_t, const int64_t *low_lengths,
                        void *y, int64_t batch, int64_t low_time, int64_t heads, int64_t head_dim, void *stream);

/*
 * Merge of the two Mamba directions and the 3-way gate: mn = RMSNorm((mf + mb) / 2) w
 * (fp32 [rows, d]), g = bf16(cat(cn, bf16(mn), an) gate_w^T + gate_b) (bf16
 * [rows, 3]); cn, mf, mb, an bf16 [rows, d]; gate_w bf16 [3, 3d], gate_b bf16 [3].
 * Replaces mean_norm + torch.cat + the gate linear (src/trifusion_l4/model.py:180-186).
 */
int tf_merge_gate(const void *cn, const void *mf, const void *mb, const void *an, const float *norm_w, float eps,
                  const void *gate_w, const void *gate_b, float *mn, void *g, int64_t rows, int64_t d,
                  void *stream);

/*
 * Evidence down-projection: z = bf16(silu(bf16(cat(cn, an) w^T + bias))), cn, an
 * bf16 [rows, d] (contiguous, 16-byte aligned), w bf16 [r, 2d] (the Linear's
 * weight), bias bf16 [r], z bf16 [rows, r]; d a multiple of 128, r one of 16, 32, 48, 64.
 * Replaces torch.cat + e_down + F.silu (src/trifusion_l4/model.py:161).
 */
int tf_evidence_down(const void *cn, const void *an, const void *w, const void *bias, void *z, int64_t rows,
                     int64_t d, int64_t r, void *stream);

/*
 * Gated concatenation, masked depthwise merge and residual add: v = cat(cn, mn, an)
 * * 2 sigmoid(g) (fp32), c = masked depthwise conv (kernel k = 3; w bf16 [3d, k],
 * bias bf16 [3d]) of bf16(v), rounded to bf16, zero at t >= L_b; y = bf16(v + c)
 * [B, T, 3d]. Replaces gated_concat + merge_dw + add(bf16=True)
 * (src/trifusion_l4/model.py:187-196).
 */
int tf_merge_conv(const void *cn, const float *mn, const void *an, const void *g, const void *w, const void *bias,
                  const int64_t *lengths, void *y, int64_t batch, int64_t time, int64_t d, int64_t k,
                  void *stream);

/*
 * Query read of the decoder: y[b, i, h D + d] = softmax_j(q_i,h . k_j,h / sqrt(D)) v_j,h
 * in fp32 over keys j < key_lengths[b], rounded to bf16; q bf16 [queries, heads, D]
 * (the same for every batch row), kv bf16 [B, T, 2, heads, D] (keys, then values; 16-byte
 * aligned), y bf16 [B, queries, heads D]. queries = 10 and D = 32 (the decoder's shape).
 * A query row with no valid key is 0. workspace: caller-allocated fp32 scratch of at least
 * tf_query_read_workspace_size(...) bytes (per 64-key tile partial softmax records).
 * Replaces QueryRead's masked_attention call (src/trifusion_l4/decoder.py:24-32,
 * attention.py:8-18).
 */
int64_t tf_query_read_workspace_size(int64_t batch, int64_t time, int64_t heads, int64_t queries,
                                     int64_t head_dim);
int tf_query_read(const void *q, const void *kv, const int64_t *key_lengths, void *y, void *workspace,
                  int64_t workspace_bytes, int64_t batch, int64_t time, int64_t heads, int64_t queries,
                  int64_t head_dim, void *stream);

/*
 * Front-end preparations (src/trifusion_l4/front.py:62-90, masking.py:14-57), one launch each:
 *  - tf_mask_audio: y[b, c, n] = n < lengths[b] && c < channels[b] ? audio[b, c, n] : 0 (fp32,
 *    contiguous [B, C, N]);
 *  - tf_log_power: y[b, f, k] = f < lengths[b] / hop + 1 ? log(1e-6 + sum_c |spec[b C + c, k, f]|^2
 *    / channels[b]) : 0, spec complex64 (interleaved) with element strides[3] (complex units),
 *    y fp32 contiguous [B, frames, bins];
 *  - tf_front_lengths: out[0] = n / hop + 1 (frames), out[i + 1] = ceil(out[i] / strides[i]), int64
 *    [4, B];
 *  - tf_grids: mask[b, t] = t < L_b, low_lengths = ceil(L / 4), low_mask[b, j] = j < low_b, and the
 *    interpolation grid pos = min(max((t + 0.5) low / L - 0.5, 0), low - 1) (fp32, op by op),
 *    left = trunc(pos), right = min(left + 1, low - 1), alpha = pos - left; masks are bytes.
 * Replace the elementwise torch runs of Frontend.spectrogram, the stage length updates and
 * Grids.make (src/trifusion_l4/front.py:62-90,105-110, masking.py:29-57).
 */
int tf_mask_audio(const float *audio, const int64_t *lengths, const int64_t *channels, float *y, int64_t batch,
                  int64_t chans, int64_t samples, void *stream);
int tf_log_power(const void *spec, const int64_t *strides, const int64_t *channels, const int64_t *sample_lengths,
                 float *y, int64_t batch, int64_t chans, int64_t bins, int64_t frames, int64_t hop, void *stream);
int tf_front_lengths(const int64_t *sample_lengths, int64_t *out, int64_t batch, int64_t hop,
                     const int64_t *strides, void *stream);
int tf_grids(const int64_t *lengths, void *mask, int64_t *low_lengths, void *low_mask, int64_t *left,
             int64_t *right, float *alpha, int64_t batch, int64_t time, void *stream);

/* Library version string (static storage). */
const char *tf_version(void);

#ifdef __cplusplus
}
#endif

#endif /* TRIFUSION_AMD_H */
