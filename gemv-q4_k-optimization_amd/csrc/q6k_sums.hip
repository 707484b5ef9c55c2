// q6k_sums.hip -- the parity variants (SUMS) of the Q6_K GEMV kernels: the
// product kernels of q6k_kernels.h and q6k_mfma.h that also store every
// lane's int32 group sums.  Instantiated for the launch shapes the automatic
// geometry picks for plain products (8 or 16 waves; the tile kernel with one
// slot and prologue 0 or 1; the K-split kernel in every shape it is
// instantiated in); q6k_gemv.hip launches them with the product's own
// geometry.
#include <hip/hip_runtime.h>

#include "q4k_runtime.h"
#include "q6k_kernels.h"
#include "q6k_ksplit.h"
#include "q6k_ksplit_nc.h"
#include "q6k_mfma.h"

namespace q4k {
namespace {

template <int NC, int WAVES, bool DENSE = false>
const void *q6_sums(int pro) {
    if (pro == 0)
        return reinterpret_cast<const void *>(&gemv_q6k_kernel<NC, WAVES, 0, 1, kEpiNone, false, true, DENSE>);
    if (pro == 1)
        return reinterpret_cast<const void *>(&gemv_q6k_kernel<NC, WAVES, 1, 1, kEpiNone, false, true, DENSE>);
    return nullptr;
}

// the dense-layout kernels (5 to 8 columns)
template <int WAVES>
const void *q6_sums_dense(int nc, int pro) {
    switch (nc) {
        case 5: return q6_sums<5, WAVES, true>(pro);
        case 6: return q6_sums<6, WAVES, true>(pro);
        case 7: return q6_sums<7, WAVES, true>(pro);
        case 8: return q6_sums<8, WAVES, true>(pro);
        default: return nullptr;
    }
}

template <int WAVES>
const void *q6_sums_nc(int nc, int pro) {
    switch (nc) {
        case 1: return q6_sums<1, WAVES>(pro);
        case 2: return q6_sums<2, WAVES>(pro);
        case 3: return q6_sums<3, WAVES>(pro);
        case 4: return q6_sums<4, WAVES>(pro);
        case 5: return q6_sums<5, WAVES>(pro);
        case 6: return q6_sums<6, WAVES>(pro);
        case 7: return q6_sums<7, WAVES>(pro);
        case 8: return q6_sums<8, WAVES>(pro);
        default: return nullptr;
    }
}

template <int WAVES>
const void *q6_mfma_sums_nc(int nc) {
    switch (nc) {
        case 1: return reinterpret_cast<const void *>(&gemv_q6k_mfma_kernel<1, WAVES, true>);
        case 2: return reinterpret_cast<const void *>(&gemv_q6k_mfma_kernel<2, WAVES, true>);
        case 3: return reinterpret_cast<const void *>(&gemv_q6k_mfma_kernel<3, WAVES, true>);
        case 4: return reinterpret_cast<const void *>(&gemv_q6k_mfma_kernel<4, WAVES, true>);
        case 5: return reinterpret_cast<const void *>(&gemv_q6k_mfma_kernel<5, WAVES, true>);
        case 6: return reinterpret_cast<const void *>(&gemv_q6k_mfma_kernel<6, WAVES, true>);
        case 7: return reinterpret_cast<const void *>(&gemv_q6k_mfma_kernel<7, WAVES, true>);
        case 8: return reinterpret_cast<const void *>(&gemv_q6k_mfma_kernel<8, WAVES, true>);
        default: return nullptr;
    }
}

}  // namespace

const void *q6k_mfma_sums_kernel(int nc, int waves) {
    return waves > 8 ? q6_mfma_sums_nc<16>(nc) : q6_mfma_sums_nc<8>(nc);
}

const void *q6k_mfma_ga_sums_kernel(int nc, int waves) {
    if (waves != 8) return nullptr;
    switch (nc) {
        case 1: return reinterpret_cast<const void *>(&gemv_q6k_mfma_kernel<1, 8, true, true>);
        case 2: return reinterpret_cast<const void *>(&gemv_q6k_mfma_kernel<2, 8, true, true>);
        case 3: return reinterpret_cast<const void *>(&gemv_q6k_mfma_kernel<3, 8, true, true>);
        case 4: return reinterpret_cast<const void *>(&gemv_q6k_mfma_kernel<4, 8, true, true>);
        case 5: return reinterpret_cast<const void *>(&gemv_q6k_mfma_kernel<5, 8, true, true>);
        case 6: return reinterpret_cast<const void *>(&gemv_q6k_mfma_kernel<6, 8, true, true>);
        case 7: return reinterpret_cast<const void *>(&gemv_q6k_mfma_kernel<7, 8, true, true>);
        case 8: return reinterpret_cast<const void *>(&gemv_q6k_mfma_kernel<8, 8, true, true>);
        default: return nullptr;
    }
}

const void *q6k_ksplit_sums_kernel(int sbw, int waves, int slots, int G) {
    return q6_ksplit_kernel<true>(sbw, waves, slots, G);
}

const void *q6k_ksplit_nc_sums_kernel(int nc, int p, int sbw, int waves, int slots) {
    return q6_ksplit_nc_kernel<true>(nc, p, sbw, waves, slots);
}

const void *q6k_ksplit_long_sums_kernel(int sbw, int waves, int slots, int G) {
    return q6_ksplit_long_kernel<true>(sbw, waves, slots, G);
}

const void *q6k_sums_kernel(int nc, int waves, int pro, int slots, bool dense) {
    if (slots != 1) return nullptr;
    if (dense) return waves <= 8 ? q6_sums_dense<8>(nc, pro) : q6_sums_dense<16>(nc, pro);
    return waves <= 8 ? q6_sums_nc<8>(nc, pro) : q6_sums_nc<16>(nc, pro);
}

}  // namespace q4k
