// C-ABI entry points of the fused recurrence: argument validation and kernel
// selection. Mirrors the checks of the reference wrapper
// (src/trifusion_l4/mamba_fused.py:155-161), generalised to the shapes the
// kernels here support; the Python wrapper maps the status codes to
// ValueError/TypeError/RuntimeError before anything is launched.
#include "mamba_internal.h"

namespace tf {
namespace {

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
  if (a->variant < TF_MAMBA_AUTO || a->variant > TF_MAMBA_MFMA) return TF_ERR_VARIANT;
  if (a->reverse != 0 && a->reverse != 1) return TF_ERR_SHAPE;
  // empty tensors may carry NULL data pointers
  if (!empty(a) && (!a->q || !a->k || !a->v || !a->adt || !a->dt || !a->trap || !a->angles ||
                    !a->z || !a->qb || !a->kb || !a->d || !a->out))
    return TF_ERR_NULL;
  return TF_OK;
}

int select(const tf_mamba_args* a) {
  const int rc = validate(a);
  if (rc != TF_OK) return -rc;
  if (a->variant == TF_MAMBA_MFMA) return mfma_supported(*a) ? TF_MAMBA_MFMA : -TF_ERR_VARIANT;
  if (a->variant == TF_MAMBA_GENERIC) return generic_supported(*a) ? TF_MAMBA_GENERIC : -TF_ERR_SHAPE;
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
  return which == TF_MAMBA_MFMA ? tf::launch_mfma(*a, s) : tf::launch_generic(*a, s);
}

extern "C" int64_t tf_fused_mamba_workspace_size(const tf_mamba_args* a) {
  const int which = tf::select(a);
  if (which < 0) return which;
  if (tf::empty(a) || which != TF_MAMBA_MFMA) return 0;
  return tf::mfma_workspace_bytes(*a);
}

extern "C" const char* tf_version(void) { return "trifusion_amd 0.1.0 (gfx950)"; }
