// q6k_ksplit_nc.h -- the K-split Q6_K GEMV kernel for two to four F32
// activation columns, rows of up to 8 groups of 16 super-blocks: the plan of
// the Q4_K several-column long-row kernel (q4k_ksplit_nc.h) with the Q6_K
// tile kernel's lane map, loads and per-lane arithmetic (q6k_kernels.h).
//
// The Q6_K tile kernel reduces its lanes with the same several-column tree
// (column_sums: g ^ 8, with three or four columns g ^ 4, then the lane's
// half h and 16-value part j', then the low bits of g), and its lanes are
// laid out alike (lane = 4g + 2h + j'), so the waves own the same residue
// classes of super-blocks and reduce with the same DPP steps:
//
//   lane = 4*SBW*r + 4*s + 2h + j'   r: row of the step, s: slice position
//                                    (super-block ksn_block(w, s)), h, j'
//
// The activation is staged once per workgroup with the tile kernel's Q6_K
// staging arithmetic into the K-split Q6K layout (super-block positions
// permuted so that a wave's lanes read one contiguous span, auxiliary terms
// of whole groups); each step's lanes read their four 16-value groups, the
// d8 of blocks 4h..4h+3 and the four -32 * sum(q8) starting values there.
//
// Reference: kernels/mmvq.cu:150-344 (ncols_dst 2-4) with the Q6_K vec-dot
// of kernels/vecdotq.cuh:867-891 and :580-600.
#pragma once

#include <hip/hip_runtime.h>

#include <type_traits>

#include "q4k_ksplit_nc.h"
#include "q6k_kernels.h"

namespace q4k {

// LDS bytes of the staged activation of nc columns of K values in the Q6K
// K-split layouts: per column the q8 of whole groups (4096 bytes each) and
// 3 * 128 auxiliary words per group.
__host__ __device__ constexpr int q6_ksn_stage_bytes(int K, int nc) {
    return nc * ((K + 4095) / 4096) * (4096 + 3 * 128 * 4);
}

// What lane (slot sl, h, j') reads of staged column c, group i; a lane past
// the row's end (in_row false) takes the auxiliary terms of the group's
// first super-block (never-written slots could hold a NaN).
template <int LAYOUT>
__device__ __forceinline__ Q6Act q6_ksn_act(int i, int c, int sl, int h, int jp, bool in_row, int qcol, int pb,
                                            const int8_t *q8s, const uint8_t *aux) {
    const int8_t *qa = q8s + c * qcol + i * 4096 + (4 * sl + 2 * h + jp) * 16;
    Q6Act a;
#pragma unroll
    for (int m = 0; m < 4; ++m) a.a[m] = *reinterpret_cast<const u32x4 *>(qa + 1024 * m);
    const int at = 16 * i + (in_row ? sl : 0);
    const float *dq = reinterpret_cast<const float *>(aux) + c * 3 * pb;
    a.d8 = *reinterpret_cast<const float4 *>(dq + at * 8 + 4 * h);
    a.s0 = *reinterpret_cast<const int4 *>(reinterpret_cast<const int *>(dq + pb) + at * 16 + 4 * (2 * h + jp));
    return a;
}

// NC: columns (2..4); P: the tile kernel's tree column count (2 or 4; 2 for
// four columns when its launches take two); SBW: super-blocks per wave and
// group (2 or 4, at least P); WAVES: whole teams of 16/SBW waves; S: steps
// in flight.  p.ring_off: LDS offset of the partials (after the staged
// activation).  SUMS: the parity variant (every lane's four int32 group
// sums at sums[(c*M + row)*(K/16) + 16kb + 8h + j' + 2m]).
template <int NC, int P, int SBW, int WAVES, int S, bool SUMS = false>
__global__ __launch_bounds__(kWave *WAVES) void gemv_q6k_ksplit_nc_kernel(Q4K_GEMV_KERNEL_ARGS) {
    static_assert(P == 2 || P == 4, "two- or four-column trees");
    static_assert(NC >= 2 && NC <= 4 && SBW >= P && SBW <= 4, "two to four columns, 2 or 4 super-blocks");
    constexpr int KW = 16 / SBW;
    constexpr int TR = 16 / SBW;
    constexpr int TEAMS = WAVES / KW;
    static_assert(TEAMS >= 1 && WAVES % KW == 0, "whole teams");
    constexpr int kLayout = P == 2 ? kLayoutQ6KS2 : kLayoutQ6KS4;
    p = with_head(p, Q4K_GEMV_HEAD_VALUES);
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    int8_t *q8s = reinterpret_cast<int8_t *>(lds);
    uint8_t *aux = lds + NC * p.qcol;
    float *part = reinterpret_cast<float *>(lds + p.ring_off);

    const int lane = threadIdx.x & (kWave - 1);
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int slice = wave % KW, team = wave / KW;
    const int r = lane / (4 * SBW), s = (lane >> 2) & (SBW - 1);
    const int h = (lane >> 1) & 1, jp = lane & 1;
    const int G = p.G;

    const int b = (int)blockIdx.x;
    const int wg_beg = b * p.rows_base + min(b, p.rows_extra);
    const int n = p.rows_base + (b < p.rows_extra ? 1 : 0);
    const int nt = (n + TR - 1) / TR;
    const int tq = nt / TEAMS, trem = nt - tq * TEAMS;
    const int tb = team * tq + min(team, trem);
    const int ntiles = tq + (team < trem ? 1 : 0);
    const int kb0 = ksn_block<P, SBW>(slice, s);  // the lane's super-block within each group
    const int wkb = ksn_block<P, SBW>(slice, 0);  // the wave's first one
    const int sl = q4k_slot<kLayout>(kb0);
    const int pb = (p.K / 32 + 127) & ~127;

    // 1. the staging loads of every wave, queued ahead of the weight loads
    constexpr int kLPB = stage_lpb(NC);
    constexpr int kPreR = pre_rounds(NC, kWave * WAVES);
    ActStage<kLPB, kPreR> xs;
    stage_f32_issue<kLPB, kWave * WAVES>(p.x, p.ldx, p.K, NC, true, p.nblk32, xs);
    __syncthreads();

    // 2. the first S steps' weights
    const __amdgpu_buffer_rsrc_t rs = make_rsrc(p.w + (int64_t)wg_beg * p.row_stride, (uint32_t)(n * p.row_stride));
    Q6Lane ln;
    ln.lane = lane;
    ln.g = kb0;
    ln.h = h;
    ln.jp = jp;
    const uint32_t blk = (uint32_t)r * (uint32_t)p.row_stride + (uint32_t)kb0 * kQ6Bytes;
    ln.o_lo = blk + 64u * (uint32_t)h + 16u * (uint32_t)jp;
    ln.o_hi = blk + 128u + 32u * (uint32_t)h + 16u * (uint32_t)jp;
    ln.o_sc = blk + 192u + 8u * (uint32_t)h;
    ln.o_d = blk + 206u;
    const uint32_t tile_bytes = (uint32_t)TR * (uint32_t)p.row_stride;
    auto load_step = [&](Step st, Q6Regs &w) {
        const bool ok = st.tile < ntiles && 16 * st.i + kb0 < p.nb;
        q6_load(rs, ln, (uint32_t)(tb + st.tile) * tile_bytes + (uint32_t)st.i * (16u * kQ6Bytes), ok, w);
    };
    Step st[S];
    Q6Regs w[S];
    st[0] = Step{0, 0};
#pragma unroll
    for (int k = 1; k < S; ++k) st[k] = next_step(st[k - 1], G);
#pragma unroll
    for (int k = 0; k < S; ++k) load_step(st[k], w[k]);

    // 3. quantise into LDS (the tile kernel's Q6_K staging arithmetic)
    stage_f32_finish<kLayout, kLPB, kWave * WAVES, NC < 4 ? 1 : kFinishRounds>(p.x, p.ldx, p.K, NC, true, p.nblk32,
                                                                                xs, p.qcol, q8s, aux);
    __syncthreads();

    // 4. the (tile, group) steps, S in flight
    float acc[NC];
#pragma unroll
    for (int c = 0; c < NC; ++c) acc[c] = 0.0f;
    int remaining = ntiles * G;
    if (remaining > 0) {
        for (;;) {
#pragma unroll
            for (int k = 0; k < S; ++k) {
                const int rl = (tb + st[k].tile) * TR + r;
                if (16 * st[k].i + wkb < p.nb) {  // the wave's slice reaches this group
                    uint32_t v[4][4];
                    int sc[4];
                    q6_values(w[k], v);
                    q6_scales(w[k], jp, sc);
                    const float d = half_bits_to_float(w[k].dw >> 16);
                    const bool in_row = 16 * st[k].i + kb0 < p.nb;
#pragma unroll
                    for (int c = 0; c < NC; ++c) {
                        const Q6Act a = q6_ksn_act<kLayout>(st[k].i, c, sl, h, jp, in_row, p.qcol, pb, q8s, aux);
                        int gs[4];
                        q6_accumulate(v, sc, d, a, acc[c], gs);
                        if constexpr (SUMS) {
                            const int kb = 16 * st[k].i + kb0;
                            if (st[k].tile < ntiles && rl < n && kb < p.nb) {
                                int32_t *o = p.sums + ((int64_t)c * p.M + wg_beg + rl) * (p.K / 16) + kb * 16 +
                                             8 * h + jp;
#pragma unroll
                                for (int m = 0; m < 4; ++m) o[2 * m] = gs[m];
                            }
                        }
                    }
                }
                if (st[k].i == G - 1) {
                    const bool wr = ks_writer<SBW>(lane) && st[k].tile < ntiles && rl < n;
#pragma unroll
                    for (int c = 0; c < NC; ++c) {
                        const float q = ksn_reduce<P, SBW>(acc[c]);
                        if (wr) part[(rl * NC + c) * KW + slice] = q;
                        acc[c] = 0.0f;
                    }
                }
                st[k] = next_step(st[(k + S - 1) % S], G);
                load_step(st[k], w[k]);
            }
            remaining -= S;
            if (remaining <= 0) break;
        }
    }
    __syncthreads();
    for (int e = (int)threadIdx.x; e < n * NC; e += kWave * WAVES) {
        const int row = e / NC, c = e - row * NC;
        float q[KW];
#pragma unroll
        for (int k = 0; k < KW; ++k) q[k] = part[e * KW + k];
#pragma unroll
        for (int hh = KW / 2; hh >= 1; hh /= 2)
#pragma unroll
            for (int t = 0; t < hh; ++t) q[t] = q[2 * t] + q[2 * t + 1];
        p.dst[c * p.ld_dst + wg_beg + row] = q[0];
    }
}

// The instantiated variants (those of the Q4_K long-row form).
constexpr bool q6_ksplit_nc_exists(int nc, int p, int sbw, int waves, int slots) {
    return ksplit_nc_long_exists(nc, p, sbw, waves, slots);
}

// The kernel for nc = 2..4 columns and a p-column tree, or null.
template <bool SUMS>
const void *q6_ksplit_nc_kernel(int nc, int p, int sbw, int waves, int slots) {
    auto pick = [&](auto nc_c, auto p_c, auto sbw_c) -> const void * {
        constexpr int NC = decltype(nc_c)::value, PP = decltype(p_c)::value, B = decltype(sbw_c)::value;
        auto by_slots = [&](auto waves_c) -> const void * {
            constexpr int W = decltype(waves_c)::value;
            if constexpr (q6_ksplit_nc_exists(NC, PP, B, W, 1))
                if (slots == 1) return reinterpret_cast<const void *>(&gemv_q6k_ksplit_nc_kernel<NC, PP, B, W, 1, SUMS>);
            if constexpr (q6_ksplit_nc_exists(NC, PP, B, W, 2))
                if (slots == 2) return reinterpret_cast<const void *>(&gemv_q6k_ksplit_nc_kernel<NC, PP, B, W, 2, SUMS>);
            return nullptr;
        };
        if (waves == 4) return by_slots(std::integral_constant<int, 4>{});
        if (waves == 8) return by_slots(std::integral_constant<int, 8>{});
        if (waves == 16) return by_slots(std::integral_constant<int, 16>{});
        return nullptr;
    };
    using I2 = std::integral_constant<int, 2>;
    using I3 = std::integral_constant<int, 3>;
    using I4 = std::integral_constant<int, 4>;
    auto by_sbw = [&](auto nc_c, auto p_c) -> const void * {
        if (sbw == 2) return pick(nc_c, p_c, I2{});
        if (sbw == 4) return pick(nc_c, p_c, I4{});
        return nullptr;
    };
    if (nc == 2 && p == 2) return by_sbw(I2{}, I2{});
    if (nc == 3 && p == 4) return by_sbw(I3{}, I4{});
    if (nc == 4 && p == 2) return by_sbw(I4{}, I2{});
    if (nc == 4 && p == 4) return by_sbw(I4{}, I4{});
    return nullptr;
}

}  // namespace q4k
