// attention.hip — placeholder until the causal GQA attention kernels land.
#include "ta_common.hpp"
extern "C" {
int ta_sdpa_fwd(const uint16_t*, const uint16_t*, const uint16_t*, uint16_t*, float*, int, int,
                int, int, int, void*) {
    return ta::set_error(-9, "sdpa_fwd: not built yet");
}
int ta_sdpa_bwd(const uint16_t*, const uint16_t*, const uint16_t*, const uint16_t*, const float*,
                uint16_t*, uint16_t*, uint16_t*, int, int, int, int, int, void*) {
    return ta::set_error(-9, "sdpa_bwd: not built yet");
}
}
