// C-ABI entry points of the fused recurrence: argument validation and kernel
// selection. Mirrors the checks of the reference wrapper
// (src/trifusion_l4/mamba_fused.py:155-161), generalised to the shapes the
// kernels here support; the Python wrapper maps the status codes to
// ValueError/TypeError/RuntimeError before anything is launched.
#include <mutex>

#include "mamba_internal.h"

namespace tf {
namespace {

// Library-owned scratch of tf_fused_mamba_static: the chunk-parallel forms'
// segment states, chunk phase sums and segment decays, for callers that cannot
// allocate. Each device holds its own copy for the life of the process. In
// host code `scratch` names a host-side stand-in, never the device memory:
// host code uses only the per-device address that hipGetSymbolAddress returns.
constexpr int64_t kStaticScratchBytes = int64_t(16) << 20;
__device__ __align__(256) char scratch[kStaticScratchBytes];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mutex;
void* g_scratch_ptr[kMaxDevices] = {};

// Device address of `scratch` on `device`, looked up with that device current
// (the previous current device is restored). A successful lookup is kept; a
// failed one returns NULL and is tried again on the next call.
void* static_scratch(int device) {
  if (device < 0 || device >= kMaxDevices) return nullptr;
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  if (g_scratch_ptr[device] != nullptr) return g_scratch_ptr[device];
  int prev = -1;
  hipError_t rc = hipGetDevice(&prev);
  if (rc == hipSuccess && prev != device) rc = hipSetDevice(device);
  void* ptr = nullptr;
  if (rc == hipSuccess) rc = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
  if (prev >= 0 && prev != device) (void)hipSetDevice(prev);
  if (rc == hipSuccess) g_scratch_ptr[device] = ptr;
  return rc == hipSuccess ? ptr : nullptr;
}

bool empty(const tf_mamba_args* a) { return a->batch == 0 || a->time == 0; }

int validate(const tf_mamba_args* a) {
  if (a == nullptr) return TF_ERR_NULL;
  const int dts[] = {a->q_dtype,    a->k_dtype,     a->v_dtype,     a->z_dtype,     a->adt_dtype,
                     a->dt_dtype,   a->trap_dtype,  a->angles_dtype, a->out_dtype};
  for (int d : dts)
    if (!dtype_ok(d)) return TF_ERR_DTYPE;
  if (a->batch < 0 || a->time < 0 || a->heads < 1 || a->qk_heads < 1) return TF_ERR_SHAPE;
  if (a->heads % a->qk_heads) return TF_ERR_SHAPE;
  if (a->state < 2 || a->state % 2 || a->head_dim < 1) return TF_ERR_SHAPE;
  if (a->rotary < 0 || a->rotary > a->state / 2) return TF_ERR_SHAPE;
  if (a->batch > 65535 || a->heads > 65535 || a->time > (int64_t(1) << 30)) return TF_ERR_SHAPE;
  if (a->variant < TF_MAMBA_AUTO || a->variant > TF_MAMBA_PIPE) return TF_ERR_VARIANT;
  if (a->reverse != 0 && a->reverse != 1) return TF_ERR_SHAPE;
  // the fused B/C norms come as a pair
  if ((a->q_norm == nullptr) != (a->k_norm == nullptr)) return TF_ERR_NULL;
  // empty tensors may carry NULL data pointers
  if (!empty(a) && (!a->q || !a->k || !a->v || !a->adt || !a->dt || !a->trap || !a->angles ||
                    !a->z || !a->qb || !a->kb || !a->d || !a->out))
    return TF_ERR_NULL;
  return TF_OK;
}

int select(const tf_mamba_args* a) {
  const int rc = validate(a);
  if (rc != TF_OK) return -rc;
  if (a->variant == TF_MAMBA_PIPE) return pipe_supported(*a) ? TF_MAMBA_PIPE : -TF_ERR_VARIANT;
  if (a->variant == TF_MAMBA_MFMA) return mfma_supported(*a) ? TF_MAMBA_MFMA : -TF_ERR_VARIANT;
  if (a->variant == TF_MAMBA_GENERIC) return generic_supported(*a) ? TF_MAMBA_GENERIC : -TF_ERR_SHAPE;
  if (pipe_supported(*a)) return TF_MAMBA_PIPE;
  if (mfma_supported(*a)) return TF_MAMBA_MFMA;
  if (generic_supported(*a)) return TF_MAMBA_GENERIC;
  return -TF_ERR_SHAPE;
}

}  // namespace
}  // namespace tf

extern "C" int tf_fused_mamba_variant(const tf_mamba_args* a) { return tf::select(a); }

extern "C" int tf_fused_mamba(const tf_mamba_args* a, void* stream) {
  const int which = tf::select(a);
  if (which < 0) return -which;
  if (tf::empty(a)) return TF_OK;
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (which == TF_MAMBA_PIPE) return tf::launch_pipe(*a, s);
  return which == TF_MAMBA_MFMA ? tf::launch_mfma(*a, s) : tf::launch_generic(*a, s);
}

extern "C" int64_t tf_fused_mamba_workspace_size(const tf_mamba_args* a) {
  const int which = tf::select(a);
  if (which < 0) return which;
  if (tf::empty(a)) return 0;
  if (which == TF_MAMBA_PIPE) return tf::pipe_workspace_bytes(*a);
  return which == TF_MAMBA_MFMA ? tf::mfma_workspace_bytes(*a) : 0;
}

extern "C" int tf_fused_mamba_static(const tf_mamba_args* a, void* stream) {
  const int which = tf::select(a);
  if (which < 0) return -which;
  if (tf::empty(a)) return TF_OK;
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (which == TF_MAMBA_GENERIC) return tf::launch_generic(*a, s);
  const int64_t need = which == TF_MAMBA_PIPE ? tf::pipe_workspace_bytes(*a) : tf::mfma_workspace_bytes(*a);
  tf_mamba_args local = *a;
  local.workspace = nullptr;
  local.workspace_bytes = 0;
  if (need > 0) {
    if (need > tf::kStaticScratchBytes) return TF_ERR_WORKSPACE;
    int device = -1;
    hipError_t rc = s != nullptr ? hipStreamGetDevice(s, &device) : hipGetDevice(&device);
    if (rc != hipSuccess) return TF_ERR_LAUNCH;
    void* ptr = tf::static_scratch(device);
    if (ptr == nullptr) return TF_ERR_LAUNCH;
    local.workspace = ptr;
    local.workspace_bytes = tf::kStaticScratchBytes;
  }
  return which == TF_MAMBA_PIPE ? tf::launch_pipe(local, s) : tf::launch_mfma(local, s);
}

extern "C" int64_t tf_fused_mamba_static_scratch_bytes(void) { return tf::kStaticScratchBytes; }

extern "C" const char* tf_version(void) { return "trifusion_amd 0.1.0 (gfx950)"; }
