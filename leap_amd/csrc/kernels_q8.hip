// int8 W8A8 projection GEMV instances (see kernels.hpp).
#include "kernels.hpp"

namespace leap_kernels {

// The int8 projection kernels by (values per thread E, lanes per group
// L = gs/E, rows per team RPT, input kind, threads per team that own values
// ACT; n = ACT * E).  RPT is compiled in (every load of a thread is then
// unconditional); a launch takes the smallest instantiated RPT that covers
// its rows with one workgroup per CU.
struct Q8Entry {
    int e, l, rpt, kind, act;
    Q8Fn fn;
    Q8Fn floor;  // the same grid streaming the weights alone (measurement)
};

#define LEAP_Q8_K(E, L, R, K, A) \
    {E, L, R, K, A, leap::q8_gemv_kernel<E, L, R, K, K != leap::kQ8InRms, A>, leap::q8_floor_kernel<E, L, R, A>},
#define LEAP_Q8_QKV(E, L, A) LEAP_Q8_K(E, L, 2, leap::kQ8InRms, A) LEAP_Q8_K(E, L, 3, leap::kQ8InRms, A) \
    LEAP_Q8_K(E, L, 4, leap::kQ8InRms, A) LEAP_Q8_K(E, L, 6, leap::kQ8InRms, A)                      \
    LEAP_Q8_K(E, L, 8, leap::kQ8InRms, A) LEAP_Q8_K(E, L, 10, leap::kQ8InRms, A)
#define LEAP_Q8_PROJ(E, L, A) LEAP_Q8_K(E, L, 2, leap::kQ8InF32, A) LEAP_Q8_K(E, L, 4, leap::kQ8InF32, A) \
    LEAP_Q8_K(E, L, 8, leap::kQ8InF32, A)
#define LEAP_Q8_ALL(E, L, A) LEAP_Q8_QKV(E, L, A) LEAP_Q8_PROJ(E, L, A)
const Q8Entry kQ8Kernels[] = {
    // dim 2048, 4096, 8192: every thread of a team owns E = dim/256 values
    LEAP_Q8_ALL(8, 4, 256) LEAP_Q8_ALL(8, 8, 256) LEAP_Q8_ALL(8, 16, 256)
    LEAP_Q8_ALL(16, 2, 256) LEAP_Q8_ALL(16, 4, 256) LEAP_Q8_ALL(16, 8, 256) LEAP_Q8_ALL(16, 16, 256)
    LEAP_Q8_ALL(32, 2, 256) LEAP_Q8_ALL(32, 4, 256) LEAP_Q8_ALL(32, 8, 256)
    // dim 3072 (Llama-3.2-3B): 192 threads of 16 values; dim 5120 (Llama-2-13B): 160 of 32
    LEAP_Q8_ALL(16, 2, 192) LEAP_Q8_ALL(16, 4, 192) LEAP_Q8_ALL(16, 8, 192)
    LEAP_Q8_ALL(32, 2, 160) LEAP_Q8_ALL(32, 4, 160)
};
#undef LEAP_Q8_ALL
#undef LEAP_Q8_PROJ
#undef LEAP_Q8_QKV
#undef LEAP_Q8_K

// True if (dim, gs) has int8 kernels.
bool q8_supported(int dim, int gs)
{
    for (const Q8Entry &k : kQ8Kernels)
        if (k.act * k.e == dim && k.l * k.e == gs) return true;
    return false;
}

// The kernel of `kind` for `rows` rows: the smallest RPT with 4 * RPT * n_cu
// >= rows, else the largest; *rpt receives it.
Q8Fn pick_q8(int dim, int gs, int kind, int rows, int n_cu, int *rpt, Q8Fn *floor)
{
    const int need = (rows + leap::kQ8Teams * n_cu - 1) / (leap::kQ8Teams * n_cu);
    const Q8Entry *best = nullptr;
    for (const Q8Entry &k : kQ8Kernels) {
        if (k.act * k.e != dim || k.l * k.e != gs || k.kind != kind) continue;
        const bool covers = k.rpt >= need, best_covers = best && best->rpt >= need;
        if (!best || (covers && (!best_covers || k.rpt < best->rpt)) || (!covers && !best_covers && k.rpt > best->rpt))
            best = &k;
    }
    if (!best) return nullptr;
    *rpt = best->rpt;
    if (floor) *floor = best->floor;
    return best->fn;
}

}  // namespace leap_kernels
