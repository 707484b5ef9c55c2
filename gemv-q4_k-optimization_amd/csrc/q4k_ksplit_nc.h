// q4k_ksplit_nc.h -- the K-split Q4_K GEMV kernels for two to four F32
// activation columns: rows of one or two 16-block groups (K = 4096 or 8192),
// and rows of other lengths up to 8 groups (the long-row form).
//
// The one-column K-split kernel (q4k_ksplit.h) with NC accumulators per
// lane.  What changes is which super-blocks a wave owns, so that the
// outputs stay the tile kernel's bits.  With several columns the tile
// kernel reduces a wave's lanes in another order than with one
// (column_sums): first super-blocks g and g^8 (lane bit 5), with three or
// four columns then g and g^4 (lane bit 4), then the four chunks of a
// super-block, then the remaining bits of g from the lowest up.  So a wave
// here owns whole residue classes of super-blocks: with P = 2 (two columns)
// the C = SBW/2 super-blocks [C*w, +C) of slice w and the same ones 8
// further on, with P = 4 (three or four columns, SBW = 4) super-block w and
// those 4, 8 and 12 further on.  Its DPP steps (ksn_reduce) are column_sums'
// levels that stay inside the wave, in column_sums' order; the balanced tree
// over the KW slices of a row forms the rest (the low bits of g).  Each
// column's output is therefore the tile kernel's, for every launch shape
// (tested).
//
// Lanes: lane = 4*SBW*r + 4*s + j as in the one-column kernel; position s of
// slice w is super-block ksn_block(w, s) of each group.
//
// Activation.  Either each wave quantises its own slices in registers and
// hands the lanes their sub-blocks through ds_bpermute, as the one-column
// kernel (every team quantises the whole activation), or (STAGED) the
// workgroup quantises the activation once into LDS with the tile kernel's
// staging (arithmetic and barriers; the layout with the super-block
// positions permuted so that a wave's lanes read one contiguous span) and
// each lane reads its sub-blocks there: with three or four columns the
// per-team quantisation costs more than the barrier.
//
// Reference: kernels/mmvq.cu:150-344 (ncols_dst 2-4) with the vec-dot of
// kernels/vecdotq.cuh:775-819 and :457-483.
#pragma once

#include <hip/hip_runtime.h>

#include "q4k_ksplit.h"

namespace q4k {

// Super-block of slice position s of slice w, within a group.
template <int P, int SBW>
__device__ __forceinline__ int ksn_block(int w, int s) {
    constexpr int C = SBW / P, L = 16 / P;
    return C * w + (s % C) + L * (s / C);
}

// Block b (0 .. 8*SBW-1) of the slice of group i, as a block index of the row.
template <int P, int SBW>
struct KsnBlocks {
    int i, w;
    __device__ int operator()(int b) const { return (16 * i + ksn_block<P, SBW>(w, b >> 3)) * 8 + (b & 7); }
};

// The in-wave levels of column_sums' tree for one column's lane values,
// valid in the ks_writer lanes (a row rotation by 4 pairs a lane with lane
// bit 2 set with the one 4 below it).
//  P = 2, SBW = 2: g ^ 8 (lane bit 2), the chunks;
//  P = 2, SBW = 4: g ^ 8 (lane bit 3), the chunks, g ^ 1 (lane bit 2);
//  P = 4, SBW = 4: g ^ 8 (lane bit 3), g ^ 4 (lane bit 2), the chunks.
template <int P, int SBW>
__device__ __forceinline__ float ksn_reduce(float v) {
    if constexpr (SBW == 4) v += dppf<kDppRor8>(v);
    if constexpr (P == 4 || SBW == 2) v += dppf<kDppRor4>(v);
    v += dppf<kDppXor1>(v);
    v += dppf<kDppXor2>(v);
    if constexpr (P == 2 && SBW == 4) v += dppf<kDppRor4>(v);
    return v;
}

// What a lane reads of a staged column in the K-split layouts: the q8 of
// sub-blocks 2j, 2j+1 of the super-block at slot sl of group i and their
// (d8, d8 * sum q8) pairs (pb: the column's padded block count).  A lane
// whose super-block lies past the row's end (in_row false; its weights read
// as zero) takes the pairs of the group's first super-block: the slots past
// the row are never written, and stale LDS contents could hold an infinity
// or NaN that a zero weight would not cancel.
__device__ __forceinline__ LaneAct ksn_lane_act(int i, int c, int sl, int j, bool in_row, int qcol, int pb,
                                                const int8_t *q8s, const float2 *dks) {
    const int8_t *qa = q8s + c * qcol + i * 4096 + (4 * sl + j) * 16;
    LaneAct a;
    a.a0 = *reinterpret_cast<const u32x4 *>(qa);
    a.a1 = *reinterpret_cast<const u32x4 *>(qa + 1024);
    a.b0 = *reinterpret_cast<const u32x4 *>(qa + 2048);
    a.b1 = *reinterpret_cast<const u32x4 *>(qa + 3072);
    a.dk = *reinterpret_cast<const float4 *>(dks + c * pb + (16 * i + (in_row ? sl : 0)) * 8 + 2 * j);
    return a;
}

// LDS bytes of the staged activation of nc columns of K values in the
// K-split layouts (q8 and auxiliary pairs of whole groups).
__host__ __device__ constexpr int ksn_stage_bytes(int K, int nc) {
    return nc * ((K + 4095) / 4096 * 4096) * 5 / 4;
}

// NC: columns (2..4); SBW: super-blocks per wave and group (2 or 4 for two
// columns, 4 for three or four); WAVES: whole teams of 16/SBW waves; S: row
// tiles in flight per wave; G: groups per row; STAGED: the activation
// quantised once per workgroup into LDS (the partials then start at
// p.ring_off).  SUMS: the parity variant.
template <int NC, int SBW, int WAVES, int S, int G, bool STAGED, bool SUMS = false>
__global__ __launch_bounds__(kWave *WAVES) void gemv_q4k_ksplit_nc_kernel(Q4K_GEMV_KERNEL_ARGS) {
    constexpr int P = NC <= 2 ? 2 : 4;
    constexpr int KW = 16 / SBW;  // waves sharing a row
    constexpr int TR = 16 / SBW;  // rows per wave step
    constexpr int TEAMS = WAVES / KW;
    constexpr int kLayout = P == 2 ? kLayoutQ4KS2 : kLayoutQ4KS4;  // the staged activation's layout
    constexpr int V = 4 * SBW;    // activation values per lane, group and column
    static_assert(NC >= 2 && NC <= 4 && SBW >= P && SBW <= 4, "two to four columns, 2 or 4 super-blocks");
    static_assert(TEAMS >= 1 && WAVES % KW == 0, "whole teams");
    p = with_head(p, Q4K_GEMV_HEAD_VALUES);
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    float *part = reinterpret_cast<float *>(lds + (STAGED ? p.ring_off : 0));

    const int lane = threadIdx.x & (kWave - 1);
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int slice = wave % KW, team = wave / KW;
    const int r = lane / (4 * SBW), s = (lane >> 2) & (SBW - 1), j = lane & 3;

    const int b = (int)blockIdx.x;
    const int wg_beg = b * p.rows_base + min(b, p.rows_extra);
    const int n = p.rows_base + (b < p.rows_extra ? 1 : 0);
    const int nt = (n + TR - 1) / TR;
    const int tq = nt / TEAMS, trem = nt - tq * TEAMS;
    const int tb = team * tq + min(team, trem);
    const int ntiles = tq + (team < trem ? 1 : 0);
    const int kb0 = ksn_block<P, SBW>(slice, s);  // the lane's super-block within each group

    // 1. the slice's activation values of every column, issued first: lane
    //    L holds values [L*V, +V) of the slice's super-blocks taken in
    //    position order (16-byte loads; the host launches this kernel for
    //    16-byte aligned columns)
    //    (STAGED: the tile kernel's staging loads, every wave's queued ahead
    //    of the weight loads by a barrier)
    const int xsb = lane / (64 / SBW);  // the slice position the lane's values lie in
    const int xoff = ksn_block<P, SBW>(slice, xsb) * kQK + (lane * V) % kQK;
    constexpr int kLPB = stage_lpb(NC);
    constexpr int kPreR = pre_rounds(NC, kWave * WAVES);
    float xv[STAGED ? 1 : G][NC][V];
    ActStage<kLPB, kPreR> xs;
    if constexpr (STAGED) {
        stage_f32_issue<kLPB, kWave * WAVES>(p.x, p.ldx, p.K, NC, true, p.nblk32, xs);
        __syncthreads();
    } else {
#pragma unroll
        for (int i = 0; i < G; ++i)
#pragma unroll
            for (int c = 0; c < NC; ++c) {
                const float4 *src = reinterpret_cast<const float4 *>(p.x + c * p.ldx + 16 * i * kQK + xoff);
#pragma unroll
                for (int k = 0; k < V / 4; ++k) {
                    const float4 a = src[k];
                    xv[i][c][4 * k] = a.x;
                    xv[i][c][4 * k + 1] = a.y;
                    xv[i][c][4 * k + 2] = a.z;
                    xv[i][c][4 * k + 3] = a.w;
                }
            }
    }

    // 2. the first S tiles' weights
    const __amdgpu_buffer_rsrc_t rs = make_rsrc(p.w + (int64_t)wg_beg * p.row_stride, (uint32_t)(n * p.row_stride));
    const uint32_t lh = (uint32_t)r * (uint32_t)p.row_stride + (uint32_t)(kb0 * kBlockBytes);
    const uint32_t lq = lh + 16u + 32u * (uint32_t)j;
    const uint32_t tile_bytes = (uint32_t)TR * (uint32_t)p.row_stride;
    auto load_tile = [&](int t, RowRegs(&w)[G]) {
        const bool ok = t < ntiles;
        const uint32_t base = (uint32_t)(tb + t) * tile_bytes;
#pragma unroll
        for (int i = 0; i < G; ++i) {
            const uint32_t gi = (uint32_t)i * (16u * kBlockBytes);
            const uint32_t oh = ok ? base + gi + lh : kOOB;
            const uint32_t oq = ok ? base + gi + lq : kOOB;
            w[i].h = load16(rs, oh);
            w[i].q0 = load16(rs, oq);
            w[i].q1 = load16(rs, oq + 16u);
        }
    };
    int tk[S];
    RowRegs w[S][G];
#pragma unroll
    for (int k = 0; k < S; ++k) {
        tk[k] = k;
        load_tile(k, w[k]);
    }

    // 3. quantise the slices and hand each lane its sub-blocks (STAGED: the
    //    workgroup's staging, then each lane reads what the tile kernel's
    //    lane 4*kb0 + j reads)
    const int sl = q4k_slot<kLayout>(kb0);  // its slot in the staged layout
    const int pb = (p.K / 32 + 127) & ~127;
    Lane ln;
    ln.lane = 4 * sl + j;
    ln.g = kb0;
    ln.j = j;
    ln.sel = make_scale_sel(j);
    LaneAct act[G][NC];
    if constexpr (STAGED) {
        int8_t *q8s = reinterpret_cast<int8_t *>(lds);
        float2 *dks = reinterpret_cast<float2 *>(lds + NC * p.qcol);
        stage_f32_finish<kLayout, kLPB, kWave * WAVES, NC < 4 ? 1 : kFinishRounds>(
            p.x, p.ldx, p.K, NC, true, p.nblk32, xs, p.qcol, q8s, dks, SUMS ? p.sq : nullptr);
        __syncthreads();
#pragma unroll
        for (int i = 0; i < G; ++i)
#pragma unroll
            for (int c = 0; c < NC; ++c) act[i][c] = ksn_lane_act(i, c, sl, j, true, p.qcol, pb, q8s, dks);
    } else {
#pragma unroll
        for (int i = 0; i < G; ++i)
#pragma unroll
            for (int c = 0; c < NC; ++c)
                act[i][c] = ks_stage<SBW>(xv[i][c], lane, s, j, SUMS ? p.sq + c * (p.K / 32) : nullptr,
                                          KsnBlocks<P, SBW>{i, slice});
    }
    // 4. the tiles, S in flight
    int remaining = ntiles;
    if (remaining > 0) {
        for (;;) {
#pragma unroll
            for (int k = 0; k < S; ++k) {
                const int rl = (tb + tk[k]) * TR + r;
                float acc[NC];
#pragma unroll
                for (int c = 0; c < NC; ++c) acc[c] = 0.0f;
#pragma unroll
                for (int i = 0; i < G; ++i) {
                    const RowScales sc = row_scales(w[k][i], ln);
#pragma unroll
                    for (int c = 0; c < NC; ++c) {
                        int sa, sb;
                        accumulate(w[k][i], sc, act[i][c], acc[c], sa, sb);
                        if constexpr (SUMS) {
                            if (tk[k] < ntiles && rl < n) {
                                int32_t *o = p.sums + ((int64_t)c * p.M + wg_beg + rl) * (p.K / 32) +
                                             (16 * i + kb0) * 8 + 2 * j;
                                o[0] = sa;
                                o[1] = sb;
                            }
                        }
                    }
                }
                const bool wr = ks_writer<SBW>(lane) && tk[k] < ntiles && rl < n;
#pragma unroll
                for (int c = 0; c < NC; ++c) {
                    const float q = ksn_reduce<P, SBW>(acc[c]);
                    if (wr) part[(rl * NC + c) * KW + slice] = q;
                }
                tk[k] += S;
                load_tile(tk[k], w[k]);
            }
            remaining -= S;
            if (remaining <= 0) break;
        }
    }
    __syncthreads();
    // 5. each (row, column): the balanced tree over its KW slice sums
    for (int e = (int)threadIdx.x; e < n * NC; e += kWave * WAVES) {
        const int row = e / NC, c = e - row * NC;
        float q[KW];
#pragma unroll
        for (int k = 0; k < KW; ++k) q[k] = part[e * KW + k];
#pragma unroll
        for (int h = KW / 2; h >= 1; h /= 2)
#pragma unroll
            for (int t = 0; t < h; ++t) q[t] = q[2 * t] + q[2 * t + 1];
        p.dst[c * p.ld_dst + wg_beg + row] = q[0];
    }
}

// LDS bytes of the (row, column, slice) partials of the largest workgroup
// share (STAGED launches: after the staged activation).
__host__ __device__ constexpr int ksplit_nc_part_bytes(int rows_per_wg, int nc, int sbw) {
    return rows_per_wg * nc * (16 / sbw) * 4;
}

// The instantiated variants: those whose registers fit the launch bounds
// without spilling (16-wave workgroups: rows of one group, and one tile in
// flight with four columns); the STAGED ones for three or four columns.
constexpr bool ksplit_nc_exists(int nc, int sbw, int waves, int slots, int G) {
    return nc >= 2 && nc <= 4 && (sbw == 4 || (sbw == 2 && nc == 2)) && (waves == 4 || waves == 8 || waves == 16) &&
           waves % (16 / sbw) == 0 && (slots == 1 || slots == 2) && (G == 1 || G == 2) &&
           (waves < 16 || (G == 1 && (nc < 4 || slots == 1)));
}

template <bool SUMS, int NC, int SBW, int WAVES>
const void *ksplit_nc_sym(int slots, int G, bool staged) {
    auto one = [&](auto s_c, auto g_c) -> const void * {
        constexpr int S = decltype(s_c)::value, GG = decltype(g_c)::value;
        if constexpr (ksplit_nc_exists(NC, SBW, WAVES, S, GG)) {
            if (!staged)
                return reinterpret_cast<const void *>(&gemv_q4k_ksplit_nc_kernel<NC, SBW, WAVES, S, GG, false, SUMS>);
            if constexpr (NC >= 3)
                return reinterpret_cast<const void *>(&gemv_q4k_ksplit_nc_kernel<NC, SBW, WAVES, S, GG, true, SUMS>);
        }
        return nullptr;
    };
    using I1 = std::integral_constant<int, 1>;
    using I2 = std::integral_constant<int, 2>;
    if (slots == 1) return G == 1 ? one(I1{}, I1{}) : (G == 2 ? one(I1{}, I2{}) : nullptr);
    if (slots == 2) return G == 1 ? one(I2{}, I1{}) : (G == 2 ? one(I2{}, I2{}) : nullptr);
    return nullptr;
}

// ------------------------------------------------------------------------
// Rows of any other length up to 8 groups (the last one possibly partial):
// the activation is staged once per workgroup as in the STAGED variant, and
// each step's lanes read their sub-blocks of the step's group from LDS (as
// the tile kernel's lanes do at each group); steps walk (tile, group)
// pairs, S in flight, as in the one-column long-row kernel.  A lane whose
// super-block lies past the row's end reads zero weights (outside the
// workgroup's buffer) and adds exactly zero, as the tile kernel's lane of
// that super-block does; a wave whose first super-block of a group lies
// past the end skips the group.
// P: the reduction tree's column count (2 or 4), that of the tile kernel's
// launches for the same product: NC rounded up, or 2 for four columns when
// the tile kernel's LDS holds only two of them per launch (then each column
// gets that launch's two-column tree).
// ------------------------------------------------------------------------
template <int NC, int P, int SBW, int WAVES, int S, bool SUMS = false>
__global__ __launch_bounds__(kWave *WAVES) void gemv_q4k_ksplit_nc_long_kernel(Q4K_GEMV_KERNEL_ARGS) {
    static_assert(P == 2 || P == 4, "two- or four-column trees");
    constexpr int KW = 16 / SBW;
    constexpr int TR = 16 / SBW;
    constexpr int TEAMS = WAVES / KW;
    constexpr int kLayout = P == 2 ? kLayoutQ4KS2 : kLayoutQ4KS4;  // the staged activation's layout
    static_assert(NC >= 2 && NC <= 4 && SBW >= P && SBW <= 4, "two to four columns, 2 or 4 super-blocks");
    static_assert(TEAMS >= 1 && WAVES % KW == 0, "whole teams");
    p = with_head(p, Q4K_GEMV_HEAD_VALUES);
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    int8_t *q8s = reinterpret_cast<int8_t *>(lds);
    float2 *dks = reinterpret_cast<float2 *>(lds + NC * p.qcol);
    float *part = reinterpret_cast<float *>(lds + p.ring_off);

    const int lane = threadIdx.x & (kWave - 1);
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int slice = wave % KW, team = wave / KW;
    const int r = lane / (4 * SBW), s = (lane >> 2) & (SBW - 1), j = lane & 3;
    const int G = p.G;

    const int b = (int)blockIdx.x;
    const int wg_beg = b * p.rows_base + min(b, p.rows_extra);
    const int n = p.rows_base + (b < p.rows_extra ? 1 : 0);
    const int nt = (n + TR - 1) / TR;
    const int tq = nt / TEAMS, trem = nt - tq * TEAMS;
    const int tb = team * tq + min(team, trem);
    const int ntiles = tq + (team < trem ? 1 : 0);
    const int kb0 = ksn_block<P, SBW>(slice, s);       // the lane's super-block within each group
    const int wkb = ksn_block<P, SBW>(slice, 0);       // the wave's first one

    // 1. the staging loads of every wave, queued ahead of the weight loads
    constexpr int kLPB = stage_lpb(NC);
    constexpr int kPreR = pre_rounds(NC, kWave * WAVES);
    ActStage<kLPB, kPreR> xs;
    stage_f32_issue<kLPB, kWave * WAVES>(p.x, p.ldx, p.K, NC, true, p.nblk32, xs);
    __syncthreads();

    // 2. the first S steps' weights
    const __amdgpu_buffer_rsrc_t rs = make_rsrc(p.w + (int64_t)wg_beg * p.row_stride, (uint32_t)(n * p.row_stride));
    const uint32_t lh = (uint32_t)r * (uint32_t)p.row_stride + (uint32_t)(kb0 * kBlockBytes);
    const uint32_t lq = lh + 16u + 32u * (uint32_t)j;
    const uint32_t tile_bytes = (uint32_t)TR * (uint32_t)p.row_stride;
    auto load_step = [&](Step st, RowRegs &w) {
        const bool ok = st.tile < ntiles && 16 * st.i + kb0 < p.nb;
        const uint32_t base = (uint32_t)(tb + st.tile) * tile_bytes + (uint32_t)st.i * (16u * kBlockBytes);
        const uint32_t oh = ok ? base + lh : kOOB;
        const uint32_t oq = ok ? base + lq : kOOB;
        w.h = load16(rs, oh);
        w.q0 = load16(rs, oq);
        w.q1 = load16(rs, oq + 16u);
    };
    Step st[S];
    RowRegs w[S];
    st[0] = Step{0, 0};
#pragma unroll
    for (int k = 1; k < S; ++k) st[k] = next_step(st[k - 1], G);
#pragma unroll
    for (int k = 0; k < S; ++k) load_step(st[k], w[k]);

    // 3. quantise into LDS (the tile kernel's layout and arithmetic)
    stage_f32_finish<kLayout, kLPB, kWave * WAVES, NC < 4 ? 1 : kFinishRounds>(
        p.x, p.ldx, p.K, NC, true, p.nblk32, xs, p.qcol, q8s, dks, SUMS ? p.sq : nullptr);
    __syncthreads();

    const int sl = q4k_slot<kLayout>(kb0);  // its slot in the staged layout
    const int pb = (p.K / 32 + 127) & ~127;
    Lane ln;
    ln.lane = 4 * sl + j;
    ln.g = kb0;
    ln.j = j;
    ln.sel = make_scale_sel(j);
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
                    const RowScales sc = row_scales(w[k], ln);
#pragma unroll
                    for (int c = 0; c < NC; ++c) {
                        const LaneAct a =
                            ksn_lane_act(st[k].i, c, sl, j, 16 * st[k].i + kb0 < p.nb, p.qcol, pb, q8s, dks);
                        int sa, sb;
                        accumulate(w[k], sc, a, acc[c], sa, sb);
                        if constexpr (SUMS) {
                            const int kb = 16 * st[k].i + kb0;
                            if (st[k].tile < ntiles && rl < n && kb < p.nb) {
                                int32_t *o = p.sums + ((int64_t)c * p.M + wg_beg + rl) * (p.K / 32) + kb * 8 + 2 * j;
                                o[0] = sa;
                                o[1] = sb;
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
        for (int h = KW / 2; h >= 1; h /= 2)
#pragma unroll
            for (int t = 0; t < h; ++t) q[t] = q[2 * t] + q[2 * t + 1];
        p.dst[c * p.ld_dst + wg_beg + row] = q[0];
    }
}

// The instantiated long-row variants (P: 2 for two columns, 4 for three,
// 2 or 4 for four).
constexpr bool ksplit_nc_long_exists(int nc, int p, int sbw, int waves, int slots) {
    return ((nc == 2 && p == 2) || (nc == 3 && p == 4) || (nc == 4 && (p == 2 || p == 4))) && sbw >= p &&
           (sbw == 2 || sbw == 4) && (waves == 4 || waves == 8 || waves == 16) && waves % (16 / sbw) == 0 &&
           (slots == 1 || slots == 2);
}

// The long-row K-split kernel for nc = 2..4 columns and a p-column tree, or null.
template <bool SUMS>
const void *ksplit_nc_long_kernel(int nc, int p, int sbw, int waves, int slots) {
    auto pick = [&](auto nc_c, auto p_c, auto sbw_c) -> const void * {
        constexpr int NC = decltype(nc_c)::value, PP = decltype(p_c)::value, B = decltype(sbw_c)::value;
        auto by_slots = [&](auto waves_c) -> const void * {
            constexpr int W = decltype(waves_c)::value;
            if constexpr (ksplit_nc_long_exists(NC, PP, B, W, 1))
                if (slots == 1)
                    return reinterpret_cast<const void *>(&gemv_q4k_ksplit_nc_long_kernel<NC, PP, B, W, 1, SUMS>);
            if constexpr (ksplit_nc_long_exists(NC, PP, B, W, 2))
                if (slots == 2)
                    return reinterpret_cast<const void *>(&gemv_q4k_ksplit_nc_long_kernel<NC, PP, B, W, 2, SUMS>);
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

// The K-split kernel for nc = 2..4 columns, or null.
template <bool SUMS>
const void *ksplit_nc_kernel(int nc, int sbw, int waves, int slots, int G, bool staged) {
    auto by_waves = [&](auto nc_c, auto sbw_c) -> const void * {
        constexpr int NC = decltype(nc_c)::value, B = decltype(sbw_c)::value;
        if (waves == 4) return ksplit_nc_sym<SUMS, NC, B, 4>(slots, G, staged);
        if (waves == 8) return ksplit_nc_sym<SUMS, NC, B, 8>(slots, G, staged);
        if (waves == 16) return ksplit_nc_sym<SUMS, NC, B, 16>(slots, G, staged);
        return nullptr;
    };
    using B2 = std::integral_constant<int, 2>;
    using B4 = std::integral_constant<int, 4>;
    switch (nc) {
        case 2: return sbw == 2 ? by_waves(std::integral_constant<int, 2>{}, B2{})
                                : (sbw == 4 ? by_waves(std::integral_constant<int, 2>{}, B4{}) : nullptr);
        case 3: return sbw == 4 ? by_waves(std::integral_constant<int, 3>{}, B4{}) : nullptr;
        case 4: return sbw == 4 ? by_waves(std::integral_constant<int, 4>{}, B4{}) : nullptr;
        default: return nullptr;
    }
}

}  // namespace q4k
