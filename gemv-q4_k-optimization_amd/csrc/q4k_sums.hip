// q4k_sums.hip -- the parity variants (SUMS) of the Q4_K GEMV kernels: the
// product kernels of q4k_gemv_kernels.h that also store every lane's int32
// sub-block sums and the staging's int32 activation sums.  Instantiated in a
// translation unit of their own for the launch shapes the automatic
// geometry picks for plain products (one row per tile, 8 or 16 waves, 1 or 2
// slots, prologue 0, 1 or 3; the block-per-lane kernel at 4 or 8 waves; the
// matrix-core kernel for 1..8 columns; the K-split kernels in every shape they
// are instantiated in); q4k_gemv.hip launches them with the
// product's own geometry.
#include <hip/hip_runtime.h>

#include "q4k_gemv_kernels.h"
#include "q4k_ksplit.h"
#include "q4k_ksplit_nc.h"
#include "q4k_mfma.h"
#include "q4k_runtime.h"

namespace q4k {
namespace {

template <int NC, int WAVES, int S>
const void *tile_sums(int pro) {
    if (pro == 0) return reinterpret_cast<const void *>(&gemv_q4k_kernel<NC, 1, WAVES, 0, S, kEpiNone, false, true>);
    if (pro == 1) return reinterpret_cast<const void *>(&gemv_q4k_kernel<NC, 1, WAVES, 1, S, kEpiNone, false, true>);
    if constexpr (S == 2) {
        if (pro == 3)
            return reinterpret_cast<const void *>(&gemv_q4k_kernel<NC, 1, WAVES, 3, S, kEpiNone, false, true>);
    }
    return nullptr;
}

template <int WAVES, int S>
const void *tile_sums_nc(int nc, int pro) {
    switch (nc) {
        case 1: return tile_sums<1, WAVES, S>(pro);
        case 2: return tile_sums<2, WAVES, S>(pro);
        case 3: return tile_sums<3, WAVES, S>(pro);
        case 4: return tile_sums<4, WAVES, S>(pro);
        case 5: return tile_sums<5, WAVES, S>(pro);
        case 6: return tile_sums<6, WAVES, S>(pro);
        case 7: return tile_sums<7, WAVES, S>(pro);
        case 8: return tile_sums<8, WAVES, S>(pro);
        default: return nullptr;
    }
}

}  // namespace

const void *q4k_sums_kernel(int nc, int waves, int pro, int slots) {
    if (slots != 1 && slots != 2) return nullptr;
    if (waves <= 8) return slots == 1 ? tile_sums_nc<8, 1>(nc, pro) : tile_sums_nc<8, 2>(nc, pro);
    return slots == 1 ? tile_sums_nc<16, 1>(nc, pro) : tile_sums_nc<16, 2>(nc, pro);
}

template <int WAVES>
static const void *mfma_sums_nc(int nc) {
    switch (nc) {
        case 1: return reinterpret_cast<const void *>(&gemv_q4k_mfma_kernel<1, WAVES, true>);
        case 2: return reinterpret_cast<const void *>(&gemv_q4k_mfma_kernel<2, WAVES, true>);
        case 3: return reinterpret_cast<const void *>(&gemv_q4k_mfma_kernel<3, WAVES, true>);
        case 4: return reinterpret_cast<const void *>(&gemv_q4k_mfma_kernel<4, WAVES, true>);
        case 5: return reinterpret_cast<const void *>(&gemv_q4k_mfma_kernel<5, WAVES, true>);
        case 6: return reinterpret_cast<const void *>(&gemv_q4k_mfma_kernel<6, WAVES, true>);
        case 7: return reinterpret_cast<const void *>(&gemv_q4k_mfma_kernel<7, WAVES, true>);
        case 8: return reinterpret_cast<const void *>(&gemv_q4k_mfma_kernel<8, WAVES, true>);
        default: return nullptr;
    }
}

const void *q4k_mfma_sums_kernel(int nc, int waves) {
    return waves > 8 ? mfma_sums_nc<16>(nc) : mfma_sums_nc<8>(nc);
}

template <int NIF>
static const void *mfma_ga_sums_nc(int nc) {
    switch (nc) {
        case 1: return reinterpret_cast<const void *>(&gemv_q4k_mfma_kernel<1, 8, true, true, NIF>);
        case 2: return reinterpret_cast<const void *>(&gemv_q4k_mfma_kernel<2, 8, true, true, NIF>);
        case 3: return reinterpret_cast<const void *>(&gemv_q4k_mfma_kernel<3, 8, true, true, NIF>);
        case 4: return reinterpret_cast<const void *>(&gemv_q4k_mfma_kernel<4, 8, true, true, NIF>);
        case 5: return reinterpret_cast<const void *>(&gemv_q4k_mfma_kernel<5, 8, true, true, NIF>);
        case 6: return reinterpret_cast<const void *>(&gemv_q4k_mfma_kernel<6, 8, true, true, NIF>);
        case 7: return reinterpret_cast<const void *>(&gemv_q4k_mfma_kernel<7, 8, true, true, NIF>);
        case 8: return reinterpret_cast<const void *>(&gemv_q4k_mfma_kernel<8, 8, true, true, NIF>);
        default: return nullptr;
    }
}

const void *q4k_mfma_ga_sums_kernel(int nc, int waves, int nif) {
    if (waves != 8) return nullptr;
    return nif == 4 ? mfma_ga_sums_nc<4>(nc) : mfma_ga_sums_nc<2>(nc);
}

const void *q4k_ksplit_sums_kernel(int sbw, int waves, int slots, int G) {
    return ksplit_kernel<true>(sbw, waves, slots, G);
}

const void *q4k_ksplit_long_sums_kernel(int sbw, int waves, int slots, int G) {
    return ksplit_long_kernel<true>(sbw, waves, slots, G);
}

const void *q4k_ksplit_nc_sums_kernel(int nc, int sbw, int waves, int slots, int G, bool staged) {
    return ksplit_nc_kernel<true>(nc, sbw, waves, slots, G, staged);
}

const void *q4k_ksplit_nc_long_sums_kernel(int nc, int p, int sbw, int waves, int slots) {
    return ksplit_nc_long_kernel<true>(nc, p, sbw, waves, slots);
}

const void *q4k_bpl_sums_kernel(int waves) {
    return waves == 8 ? reinterpret_cast<const void *>(&gemv_q4k_bpl_kernel<8, true>)
                      : reinterpret_cast<const void *>(&gemv_q4k_bpl_kernel<4, true>);
}

}  // namespace q4k
