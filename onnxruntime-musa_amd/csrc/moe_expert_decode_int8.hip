// moe_expert_decode_int8.hip -- int8 instantiations of the decode expert kernels
// (kernel templates: moe_expert_decode.h, moe_expert_stream.h).
#include "moe_expert_stream.h"

namespace moe {
namespace decode {

hipError_t launch_int8(const Stage& st, const ExpertArgs& a, bool fc1, bool gated, hipStream_t stream) {
  return launch_quant<kInt8>(st, a, fc1, gated, stream);
}

hipError_t launch_stream_int8(const StreamStage& ss, const ExpertArgs& a, bool fc1, bool gated, hipStream_t stream) {
  return launch_stream_fmt<kInt8>(ss, a, fc1, gated, stream);
}

}  // namespace decode
}  // namespace moe
