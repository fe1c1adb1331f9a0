// Host-side RoPE table, built once per handle and uploaded.
//
// The formula is the reference's precompute_freqs
// (src/inference/FloatTransformer.cpp:56-72): for even i,
//   freq = 1 / theta^(i/head_size), angle = (float)pos * freq,
// stored as fp32 cos/sin.  This file is compiled by the host C++ compiler with
// the reference's release flags (-O3 -ffast-math, CMakeLists.txt:33), and the
// reference's base 500000 is kept a compile-time constant, so the compiler
// evaluates the power the way it does in the reference and the tables agree
// bit for bit.  Device sin/cos are never used for the table: at long context
// the fp32 rounding of pos*freq must match the engine's own table.
#include <cmath>
#include <cstddef>

extern "C" void leap_rope_table_host(int seq_len, int head_size, float theta, float *cos_tab,
                                     float *sin_tab)
{
    const int half = head_size / 2;
    for (int pos = 0; pos < seq_len; pos++) {
        for (int j = 0; j < half; j++) {  // the even i of the reference's loop, one table entry each
            const int i = 2 * j;
            float freq;
            if (theta == 500000.0f)
                freq = 1.0f / std::pow(500000.0f, static_cast<float>(i) / static_cast<float>(head_size));
            else
                freq = 1.0f / std::pow(theta, static_cast<float>(i) / static_cast<float>(head_size));
            const float val = static_cast<float>(pos) * freq;
            const size_t idx = static_cast<size_t>(pos) * half + static_cast<size_t>(j);
            cos_tab[idx] = std::cos(val);
            sin_tab[idx] = std::sin(val);
        }
    }
}
