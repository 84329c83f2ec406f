// Helpers shared by the translation units that implement the extern "C" ABI (abi.cpp,
// timestral_abi.cpp): the thread's last-error message, one-time device set-up, and the
// sub-allocation plan of scratch buffers.
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>
#include <functional>
#include <initializer_list>

namespace tsfm {
namespace abi {

// Records this thread's error message (tsfm_attn_last_error) and returns `code`.
int fail(int code, const char* fmt, ...);
// Device set-up, once per process; TSFM_OK or TSFM_E_UNAVAILABLE.
int ensure_ready();
// fail() for a HIP error: TSFM_E_UNSUPPORTED for hipErrorNotSupported, else TSFM_E_DEVICE.
int hip_fail(hipError_t e, const char* what);

inline bool aligned(const void* p, size_t a) { return (reinterpret_cast<uintptr_t>(p) & (a - 1)) == 0; }

// Sub-allocation plan over one scratch buffer (256-byte aligned pieces).
struct Plan {
    size_t off = 0;
    size_t take(size_t bytes) {
        const size_t at = off;
        off = (off + bytes + 255) & ~size_t(255);
        return at;
    }
};

// Scratch of the device-pointer entry points (abi.cpp): one slot per entry point.
enum ScratchSlot { kSlotEncode, kSlotChronos2Forward, kSlotChronos2Forecast, kSlotBoltForward, kSlotBoltForecast,
                   kSlotBoltHorizon, kSlotTimestralForecast, kSlotProject };
// A buffer of at least `bytes` for work queued on `stream` by the calling thread, kept between
// calls; *owned: a stream-ordered allocation instead, to be released with hipFreeAsync.
hipError_t scratch_acquire(hipStream_t stream, int slot, size_t bytes, char** out, bool* owned);

// TSFM_FORECAST_HOST_IO: a host array of `bytes` bytes and the device-pointer field that takes its
// copy (host may be NULL with bytes 0: the field is set to NULL).
struct HostArray {
    const void* host;
    size_t bytes;
    const void** dev;
};
// Uploads every `in` on the calling thread's stream, points its field at the copy, gives every `out`
// a device buffer, runs body(stream), downloads the outs and synchronises. Returns body's code, or
// a copy / allocation error.
int run_host_io(std::initializer_list<HostArray> ins, std::initializer_list<HostArray> outs,
                const std::function<int(hipStream_t)>& body);

}  // namespace abi
}  // namespace tsfm
