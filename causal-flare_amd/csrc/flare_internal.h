// flare_internal.h -- host-side declarations shared between the library's translation units.
#pragma once
#include <stdint.h>

namespace flare {
int64_t default_chunk(int64_t B, int64_t N, int64_t H, int64_t M, int64_t Dv);
}
