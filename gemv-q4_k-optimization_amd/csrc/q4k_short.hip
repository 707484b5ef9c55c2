// q4k_short.hip -- the long-row K-split kernels (one F32 column) with short
// teams, for rows of 3 to 14 super-blocks (K = 768 .. 3584 values): a team
// of KW = 16/SBW waves would leave the waves past the row's super-blocks
// without work, so a team is only as many waves as the row needs
// (ksplit_short_team).  Instantiated in translation units of
// their own (this one with Q6 = false for Q4_K, q6k_short.hip for Q6_K), in
// the shapes ksplit_short_exists lists: plain, parity (SUMS), fused (bias;
// gate weight + GLU) and batched launches; with them the several-column
// short-team kernels (two to four F32 columns, plain and parity) in the
// shapes ksplit_short_nc_exists lists.
#include <hip/hip_runtime.h>

#include <type_traits>

#include "q4k_ksplit.h"
#include "q4k_runtime.h"
#include "q6k_ksplit.h"

namespace q4k {
namespace {

template <bool Q6, int SBW, int KT, int W, int S, bool SUMS, int EPI, bool BATCH>
const void *short_sym() {
    if constexpr (ksplit_short_exists(Q6, SBW, KT, W, S, SUMS, EPI, BATCH)) {
        if constexpr (Q6)
            return reinterpret_cast<const void *>(&gemv_q6k_ksplit_long_kernel<SBW, W, S, 1, SUMS, EPI, BATCH, KT>);
        else
            return reinterpret_cast<const void *>(&gemv_q4k_ksplit_long_kernel<SBW, W, S, 1, SUMS, EPI, BATCH, KT>);
    }
    return nullptr;
}

template <bool Q6, int SBW, int KT, int W, int S>
const void *short_by_kind(bool sums, int epi, bool batch) {
    if (sums) return (epi == kEpiNone && !batch) ? short_sym<Q6, SBW, KT, W, S, true, kEpiNone, false>() : nullptr;
    switch (epi) {
        case kEpiNone:
            return batch ? short_sym<Q6, SBW, KT, W, S, false, kEpiNone, true>()
                         : short_sym<Q6, SBW, KT, W, S, false, kEpiNone, false>();
        case kEpiBias:
            return batch ? short_sym<Q6, SBW, KT, W, S, false, kEpiBias, true>()
                         : short_sym<Q6, SBW, KT, W, S, false, kEpiBias, false>();
        case kEpiGlu:
            return batch ? short_sym<Q6, SBW, KT, W, S, false, kEpiGlu, true>()
                         : short_sym<Q6, SBW, KT, W, S, false, kEpiGlu, false>();
        default: return nullptr;
    }
}

template <bool Q6, int SBW, int KT>
const void *short_by_shape(int waves, int slots, bool sums, int epi, bool batch) {
    auto by_s = [&](auto w_c) -> const void * {
        constexpr int W = decltype(w_c)::value;
        if (slots == 1) return short_by_kind<Q6, SBW, KT, W, 1>(sums, epi, batch);
        if (slots == 2) return short_by_kind<Q6, SBW, KT, W, 2>(sums, epi, batch);
        return nullptr;
    };
    if constexpr ((KT & (KT - 1)) == 0) {
        if (waves == 4) return by_s(std::integral_constant<int, 4>{});
        if (waves == 8) return by_s(std::integral_constant<int, 8>{});
        if (waves == 16) return by_s(std::integral_constant<int, 16>{});
    } else {
        if (waves == KT) return by_s(std::integral_constant<int, KT>{});
        if (waves == 2 * KT) return by_s(std::integral_constant<int, 2 * KT>{});
        if constexpr (4 * KT <= 16)
            if (waves == 4 * KT) return by_s(std::integral_constant<int, 4 * KT>{});
    }
    return nullptr;
}

template <bool Q6>
const void *short_kernel(int sbw, int kt, int waves, int slots, bool sums, int epi, bool batch) {
    if (sbw == 1 && kt == 4) return short_by_shape<Q6, 1, 4>(waves, slots, sums, epi, batch);
    if (sbw == 1 && kt == 8) return short_by_shape<Q6, 1, 8>(waves, slots, sums, epi, batch);
    if (sbw == 2 && kt == 2) return short_by_shape<Q6, 2, 2>(waves, slots, sums, epi, batch);
    if (sbw == 2 && kt == 4) return short_by_shape<Q6, 2, 4>(waves, slots, sums, epi, batch);
    if (sbw == 2 && kt == 5) return short_by_shape<Q6, 2, 5>(waves, slots, sums, epi, batch);
    if (sbw == 2 && kt == 6) return short_by_shape<Q6, 2, 6>(waves, slots, sums, epi, batch);
    if (sbw == 2 && kt == 7) return short_by_shape<Q6, 2, 7>(waves, slots, sums, epi, batch);
    if (sbw == 4 && kt == 1) return short_by_shape<Q6, 4, 1>(waves, slots, sums, epi, batch);
    if (sbw == 4 && kt == 2) return short_by_shape<Q6, 4, 2>(waves, slots, sums, epi, batch);
    if (sbw == 4 && kt == 3) return short_by_shape<Q6, 4, 3>(waves, slots, sums, epi, batch);
    return nullptr;
}

}  // namespace

namespace {
template <bool Q6, int NC, int SBW, int KT, int P = 2>
const void *short_nc_sym(int waves, int slots, bool sums) {
    auto by_s = [&](auto w_c) -> const void * {
        constexpr int W = decltype(w_c)::value;
        auto pick = [&](auto s_c) -> const void * {
            constexpr int S = decltype(s_c)::value;
            if constexpr (ksplit_short_nc_exists(NC, SBW, KT, W, S, P)) {
                if constexpr (Q6)
                    return sums ? reinterpret_cast<const void *>(
                                      &gemv_q6k_ksplit_short_nc_kernel<NC, SBW, W, S, KT, true, P>)
                                : reinterpret_cast<const void *>(
                                      &gemv_q6k_ksplit_short_nc_kernel<NC, SBW, W, S, KT, false, P>);
                else
                    return sums ? reinterpret_cast<const void *>(
                                      &gemv_q4k_ksplit_short_nc_kernel<NC, SBW, W, S, KT, true, P>)
                                : reinterpret_cast<const void *>(
                                      &gemv_q4k_ksplit_short_nc_kernel<NC, SBW, W, S, KT, false, P>);
            }
            return nullptr;
        };
        if (slots == 1) return pick(std::integral_constant<int, 1>{});
        if (slots == 2) return pick(std::integral_constant<int, 2>{});
        return nullptr;
    };
    if (waves == 4) return by_s(std::integral_constant<int, 4>{});
    if (waves == 8) return by_s(std::integral_constant<int, 8>{});
    if (waves == 16) return by_s(std::integral_constant<int, 16>{});
    return nullptr;
}

template <bool Q6>
const void *short_nc_kernel(int nc, int sbw, int kt, int waves, int slots, bool sums, int p) {
    if (p == 4) {  // residue classes mod 4 (three or four columns of rows of 5 to 8 blocks)
        if (nc == 3 && sbw == 2 && kt == 4) return short_nc_sym<Q6, 3, 2, 4, 4>(waves, slots, sums);
        if (nc == 4 && sbw == 2 && kt == 4) return short_nc_sym<Q6, 4, 2, 4, 4>(waves, slots, sums);
        return nullptr;
    }
    if (nc == 2 && sbw == 2 && kt == 2) return short_nc_sym<Q6, 2, 2, 2>(waves, slots, sums);
    if (nc == 2 && sbw == 2 && kt == 4) return short_nc_sym<Q6, 2, 2, 4>(waves, slots, sums);
    if (nc == 2 && sbw == 4 && kt == 1) return short_nc_sym<Q6, 2, 4, 1>(waves, slots, sums);
    if (nc == 2 && sbw == 4 && kt == 2) return short_nc_sym<Q6, 2, 4, 2>(waves, slots, sums);
    if (nc == 3 && sbw == 4 && kt == 1) return short_nc_sym<Q6, 3, 4, 1>(waves, slots, sums);
    if (nc == 4 && sbw == 4 && kt == 1) return short_nc_sym<Q6, 4, 4, 1>(waves, slots, sums);
    return nullptr;
}
}  // namespace

#ifndef Q4K_SHORT_Q6
const void *q4k_ksplit_short_kernel(int sbw, int kt, int waves, int slots, bool sums, int epi, bool batch) {
    return short_kernel<false>(sbw, kt, waves, slots, sums, epi, batch);
}
const void *q4k_ksplit_short_nc_kernel(int nc, int sbw, int kt, int waves, int slots, bool sums, int p) {
    return short_nc_kernel<false>(nc, sbw, kt, waves, slots, sums, p);
}
#else
const void *q6k_ksplit_short_kernel(int sbw, int kt, int waves, int slots, bool sums, int epi, bool batch) {
    return short_kernel<true>(sbw, kt, waves, slots, sums, epi, batch);
}
const void *q6k_ksplit_short_nc_kernel(int nc, int sbw, int kt, int waves, int slots, bool sums, int p) {
    return short_nc_kernel<true>(nc, sbw, kt, waves, slots, sums, p);
}
#endif

}  // namespace q4k
