#include "launch.hpp"
namespace tsfm {
hipError_t launch_kv_append(const KvLayout&, bool, const void*, int64_t, int64_t, const void*, int64_t, int64_t, int32_t, int32_t, hipStream_t) { return hipErrorNotSupported; }
hipError_t launch_kv_attend(const KvLayout&, bool, const void*, int64_t, int64_t, void*, int64_t, int64_t, int32_t, int32_t, int32_t, float, hipStream_t) { return hipErrorNotSupported; }
}
