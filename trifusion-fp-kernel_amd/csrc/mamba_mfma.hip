// placeholder: MFMA chunked-scan kernel
#include "mamba_internal.h"
namespace tf {
bool mfma_supported(const tf_mamba_args&) { return false; }
int launch_mfma(const tf_mamba_args&, hipStream_t) { return TF_ERR_VARIANT; }
}
