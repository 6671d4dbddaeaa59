// Decode kernels for f16 queries, batched addressing (see attn_decode.hpp).
#include "attn_decode.hpp"

namespace lmx {
template lmx_status launch_mode<f16, kModeBatched>(const DecodeArgs&, const DecodePlan&, int, hipStream_t);
}  // namespace lmx
