// Host-only stand-ins for the kernel launches of the sampling library, so that the C ABI
// layer (api.cpp) can be built with the address and undefined-behaviour sanitizers and
// driven without a GPU.  The launches record their arguments instead of launching.
#include <stdint.h>

#include "internal.h"
#include "stubs.h"

namespace stub {
kls::Args last_args;
kls::HeadArgs last_head;
int launches = 0;
int fills = 0;
alignas(256) unsigned char scratch[1 << 16];
size_t scratch_bytes = sizeof(scratch);
}  // namespace stub

namespace kls {

hipError_t launch_sample(const Args &a, int32_t, hipStream_t, const PhaseEvents *) {
    stub::last_args = a;
    ++stub::launches;
    return hipSuccess;
}

hipError_t launch_lmhead(const Args &a, const HeadArgs &h, hipStream_t) {
    stub::last_args = a;
    stub::last_head = h;
    ++stub::launches;
    return hipSuccess;
}

hipError_t launch_zero_fill(void *, size_t, hipStream_t) {
    ++stub::fills;
    return hipSuccess;
}

hipError_t scratch_workspace(hipStream_t, void **ptr) {
    *ptr = stub::scratch;
    return hipSuccess;
}

}  // namespace kls

extern "C" const char *hipGetErrorString(hipError_t) { return "stub HIP error"; }
