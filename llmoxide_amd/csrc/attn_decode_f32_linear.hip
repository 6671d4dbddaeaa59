// Decode kernels for f32 queries, linear addressing (see attn_decode.hpp).
#include "attn_decode.hpp"

namespace lmx {
template lmx_status launch_mode<float, kModeLinear>(const DecodeArgs&, const DecodePlan&, int, hipStream_t);
}  // namespace lmx
