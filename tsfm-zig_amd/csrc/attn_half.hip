#include "launch.hpp"
namespace tsfm {
hipError_t launch_attn_half(const Params&, bool, int, int, bool, hipStream_t) { return hipErrorNotSupported; }
}
