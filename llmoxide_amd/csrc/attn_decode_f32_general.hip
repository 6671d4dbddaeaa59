// Decode kernels for f32 queries, general addressing (see attn_decode.hpp).
#include "attn_decode.hpp"

namespace lmx {
template lmx_status launch_mode<float, kModeGeneral>(const DecodeArgs&, const DecodePlan&, int, hipStream_t);
}  // namespace lmx
