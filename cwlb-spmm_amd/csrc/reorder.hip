// Degree reordering on the GPU (reference main.cpp:197-278, produced there
// on the host with oneDPL).  Placeholder until the device sort lands.
#include "internal.h"

namespace cwlb {

cwlb_status launch_reorder(cwlb_ctx*, int32_t, int64_t, const int32_t*, const int32_t*,
                           const float*, int32_t*, int32_t*, int32_t*, float*)
{
    return fail(CWLB_UNSUPPORTED, "cwlb_reorder_by_degree_device: not available in this build");
}

}  // namespace cwlb
