// Host-side layout of a LEAP checkpoint (.bin), shared by checkpoint.cpp and
// the upload entry point in leap_hip_attention.hip.
#pragma once

#include <stddef.h>
#include <stdint.h>

#include "leap_hip_attention.h"

namespace leap {

// Byte offsets, from the start of the file, of one layer's attention
// weights.  For int8 checkpoints each projection is its int8 values followed
// by its group scales (init_quantized_tensors, QuantizedTransformer.cpp:88-100).
struct CkptLayer {
    size_t rms_att;
    size_t wq, wk, wv, wo;          // fp32 matrices, or int8 values
    size_t wq_s, wk_s, wv_s, wo_s;  // int8 only: the scales
};

// Offsets of layer `layer`'s weights in a checkpoint described by `c`, and
// the number of bytes the file must hold for every layer's attention weights
// to be inside it.  Returns false if the sizes overflow.
__attribute__((visibility("hidden"))) bool ckpt_layer(const leap_hip_attention_checkpoint &c, int layer,
                                                     CkptLayer *out, size_t *needed);

}  // namespace leap
