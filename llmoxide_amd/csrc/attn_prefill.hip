// Placeholder: the MFMA prefill kernel is not in yet; every batch takes the
// split-K path.
#include "common.hpp"

namespace lmx {

bool prefill_supported(const lmx_attn_params*, lmx_dtype) { return false; }

lmx_status prefill_fwd(const lmx_attn_params*, const void*, lmx_dtype, const void*, const void*,
                       const void*, const void*, float*, hipStream_t) {
    return LMX_E_UNSUPPORTED;
}

}  // namespace lmx
