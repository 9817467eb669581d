// Causal paged prefill on MFMA: placeholder until the gfx950 kernel lands.
#include "common.h"

using namespace kvflux_hip;

extern "C" int kvflux_paged_prefill(const void*, const void*, uint64_t, uint64_t, uint64_t,
                                    uint64_t, int, const uint64_t*, uint64_t, uint64_t, uint64_t,
                                    uint64_t, const float*, float*, void*) {
    return fail(KVFLUX_ERR_UNSUPPORTED, "paged prefill: MFMA kernel not available");
}
