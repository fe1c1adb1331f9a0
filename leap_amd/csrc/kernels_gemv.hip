// fp32 projection GEMV instances (see kernels.hpp).
#include "kernels.hpp"

namespace leap_kernels {

// RB rows per workgroup keep 128 KiB of weights in flight per workgroup (64
// KiB and 256 KiB measured slower at Llama-3-8B).
template <int NC>
constexpr int proj_rows() { return 32 / NC; }

bool pick_proj(int dim, QkvFn *qkv, ProjFn *proj, int *rb, GemvFloorFn *floor)
{
#define LEAP_PROJ(NC)                                                             \
    if (dim == 1024 * NC) {                                                       \
        *qkv = leap::qkv_kernel<proj_rows<NC>(), NC>;                             \
        *proj = leap::proj_residual_kernel<proj_rows<NC>(), NC>;                  \
        *rb = proj_rows<NC>();                                                    \
        if (floor) *floor = leap::gemv_floor_kernel<proj_rows<NC>(), NC>;         \
        return true;                                                              \
    }
    LEAP_PROJ(2) LEAP_PROJ(3) LEAP_PROJ(4) LEAP_PROJ(5) LEAP_PROJ(8)
#undef LEAP_PROJ
    return false;
}

}  // namespace leap_kernels
