// Decode kernels for f32 queries, batched addressing (see attn_decode.hpp).
#include "attn_decode.hpp"

namespace lmx {
template lmx_status launch_mode<float, kModeBatched>(const DecodeArgs&, const DecodePlan&, int, hipStream_t);
}  // namespace lmx
