// Decode kernel instances: head_dim 128, PART = true, with the 2-wave instances
// (see kernels_decode_table.hpp).
#include "kernels_decode_table.hpp"

namespace leap_kernels {
template KernelFn pick_decode<128, true>(int g, bool valu, int kvs, int waves);
}  // namespace leap_kernels
