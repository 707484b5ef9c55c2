// q6k_ksplit.h -- the K-split Q6_K GEMV kernel for gfx950: one F32
// activation column, rows of one or two 16-block groups (K = 4096 or 8192),
// on the plan of the Q4_K K-split kernel (q4k_ksplit.h).
//
// A team of KW = 16/SBW waves shares every row the team walks: wave w of the
// team owns the SBW super-blocks [16i + SBW*w, +SBW) of each group i; a wave
// step covers TR = 16/SBW rows of that slice, four lanes per super-block with
// the Q6_K tile kernel's lane map (q6k_kernels.h):
//
//   lane = 4*SBW*r + 4*s + 2h + j'   r: row of the step, s: super-block of
//                                    the slice, h: half of the block, j': l
//                                    in [16j', 16j' + 16)
//
// so a lane loads ql, qh, its half's scales and d of one super-block and
// forms four whole scale-group sums (weights 128h + 32m + 16j' + [0, 16),
// m = 0..3; kernels/vecdotq.cuh:867-891 and :580-600 compute the same sums
// over another partition).
//
// Activation: each lane loads 4*SBW consecutive values of the wave's slice
// and the wave quantises them in registers (Q8_1 arithmetic); ds_bpermute
// hands each lane its 64 q8, the d8 of blocks 4h..4h+3 and the -32 * (sum of
// q8) starting values of its four 16-value groups.  No LDS staging, no
// barrier before the weight loads; the (row, slice) partials meet in LDS
// after the last step.
//
// Summation order: the tile kernel's lane value (q6_accumulate, the same fma
// chain over the row's groups), then wave_sum's tree over the 16 super-block
// positions of a group, split between the DPP steps inside a wave and the
// balanced tree over the slices: the outputs are the tile kernel's bits.
#pragma once

#include <hip/hip_runtime.h>

#include "q4k_ksplit.h"
#include "q6k_kernels.h"

namespace q4k {

// The wave's activation slice of one group (lane L holds the 4*SBW values
// [L*4*SBW, +4*SBW) of the slice) -> what lane (r, s, h, j') reads.  sq
// (unused: the Q6_K parity variants store group sums only) is not taken.
template <int SBW>
__device__ __forceinline__ Q6Act q6_ks_stage(const float (&v)[4 * SBW], int s, int h, int jp) {
    constexpr int V = 4 * SBW;
    constexpr int LPB = 32 / V;  // lanes per 32-value block (8, 4, 2)
    static_assert(V <= 16, "16-value halves span whole lanes");
    uint32_t word[V / 4];
    float d8;
    int qs, hs;
    ks_quantize_part<V>(v, word, d8, qs, hs);
    Q6Act a;
    // dword t of group m = values 256s + 128h + 32m + 16j' + 4t: word t % SBW
    // of lane (64s + 32h + 8m + 4j' + t) / SBW
    const int base = 64 * s + 32 * h + 4 * jp;
#pragma unroll
    for (int m = 0; m < 4; ++m) {
        uint32_t q[4];
#pragma unroll
        for (int t = 0; t < 4; ++t) q[t] = bperm((base + 8 * m + t) / SBW, word[t % SBW]);
        a.a[m] = u32x4{q[0], q[1], q[2], q[3]};
    }
    // block 8s + 4h + m starts in lane (8s + 4h + m) * LPB; its half j' in
    // lane + j' * LPB / 2
    float d[4];
    int hsum[4];
#pragma unroll
    for (int m = 0; m < 4; ++m) {
        const int l0 = (8 * s + 4 * h + m) * LPB;
        d[m] = bpermf(l0, d8);
        hsum[m] = (int)bperm(l0 + jp * (LPB / 2), (uint32_t)hs);
    }
    a.d8 = make_float4(d[0], d[1], d[2], d[3]);
    a.s0 = make_int4(-32 * hsum[0], -32 * hsum[1], -32 * hsum[2], -32 * hsum[3]);
    return a;
}

// SBW: super-blocks per wave and group (1, 2, 4), WAVES: waves per
// workgroup (whole teams of 16/SBW), S: row tiles in flight per wave, G:
// groups per row.  SUMS: the parity variant, which also stores every lane's
// four int32 group sums.  Rows: the workgroup's share, tiles of TR rows
// split contiguously over the teams.
// EPI, BATCH: the fused epilogue and batched launches, as in the Q4_K
// K-split kernels (ks_epilogue, batch_activation / batch_weights).
template <int SBW, int WAVES, int S, int G, bool SUMS = false, int EPI = kEpiNone, bool BATCH = false>
__global__ __launch_bounds__(kWave *WAVES) void gemv_q6k_ksplit_kernel(Q4K_GEMV_KERNEL_ARGS) {
    constexpr int KW = 16 / SBW;
    constexpr int TR = 16 / SBW;
    constexpr int TEAMS = WAVES / KW;
    constexpr int V = 4 * SBW;
    constexpr int NW = EPI == kEpiGlu ? 2 : 1;  // weights per step (the weight, the gate weight)
    static_assert(TEAMS >= 1 && WAVES % KW == 0, "whole teams");
    static_assert(!SUMS || (EPI == kEpiNone && !BATCH), "parity variants of the plain product only");
    p = with_head(p, Q4K_GEMV_HEAD_VALUES);
    if constexpr (BATCH) batch_activation(p);
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    float *part = reinterpret_cast<float *>(lds);

    const int lane = threadIdx.x & (kWave - 1);
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int slice = wave % KW, team = wave / KW;
    const int r = lane / (4 * SBW), s = (lane >> 2) & (SBW - 1);
    const int h = (lane >> 1) & 1, jp = lane & 1;

    const int b = (int)blockIdx.x;
    const int wg_beg = b * p.rows_base + min(b, p.rows_extra);
    const int n = p.rows_base + (b < p.rows_extra ? 1 : 0);
    const int nt = (n + TR - 1) / TR;
    const int tq = nt / TEAMS, trem = nt - tq * TEAMS;
    const int tb = team * tq + min(team, trem);
    const int ntiles = tq + (team < trem ? 1 : 0);

    // 1. the slice's activation (16-byte loads: the host launches this
    //    kernel for 16-byte aligned activations), issued first
    float xv[G][V];
#pragma unroll
    for (int i = 0; i < G; ++i) {
        const float4 *src = reinterpret_cast<const float4 *>(p.x + (16 * i + SBW * slice) * kQK + lane * V);
#pragma unroll
        for (int k = 0; k < V / 4; ++k) {
            const float4 a = src[k];
            xv[i][4 * k] = a.x;
            xv[i][4 * k + 1] = a.y;
            xv[i][4 * k + 2] = a.z;
            xv[i][4 * k + 3] = a.w;
        }
    }

    // 2. the first S tiles' weights (GLU: and the gate weight's, at the same
    //    offsets; BATCH: of the workgroup's weight matrix, none if absent)
    if constexpr (BATCH) batch_weights(p);
    const uint32_t wbytes = BATCH && p.w_absent ? 0u : (uint32_t)(n * p.row_stride);
    __amdgpu_buffer_rsrc_t rsw[NW];
    rsw[0] = make_rsrc(p.w + (int64_t)wg_beg * p.row_stride, wbytes);
    if constexpr (NW == 2) rsw[NW - 1] = make_rsrc(p.gate + (int64_t)wg_beg * p.row_stride, wbytes);
    Q6Lane ln;
    ln.lane = lane;
    ln.g = SBW * slice + s;
    ln.h = h;
    ln.jp = jp;
    const uint32_t blk = (uint32_t)r * (uint32_t)p.row_stride + (uint32_t)ln.g * kQ6Bytes;
    ln.o_lo = blk + 64u * (uint32_t)h + 16u * (uint32_t)jp;
    ln.o_hi = blk + 128u + 32u * (uint32_t)h + 16u * (uint32_t)jp;
    ln.o_sc = blk + 192u + 8u * (uint32_t)h;
    ln.o_d = blk + 206u;
    const uint32_t tile_bytes = (uint32_t)TR * (uint32_t)p.row_stride;
    auto load_tile = [&](int t, Q6Regs(&w)[G][NW]) {
        const bool ok = t < ntiles;
        const uint32_t base = (uint32_t)(tb + t) * tile_bytes;
#pragma unroll
        for (int i = 0; i < G; ++i)
#pragma unroll
            for (int u = 0; u < NW; ++u) q6_load(rsw[u], ln, base + (uint32_t)i * (16u * kQ6Bytes), ok, w[i][u]);
    };
    int tk[S];
    Q6Regs w[S][G][NW];
#pragma unroll
    for (int k = 0; k < S; ++k) {
        tk[k] = k;
        load_tile(k, w[k]);
    }

    // 3. quantise the slice and hand each lane its groups
    Q6Act act[G];
#pragma unroll
    for (int i = 0; i < G; ++i) act[i] = q6_ks_stage<SBW>(xv[i], s, h, jp);

    // 4. the tiles, S in flight
    int remaining = ntiles;
    if (remaining > 0) {
        for (;;) {
#pragma unroll
            for (int k = 0; k < S; ++k) {
                float acc[NW];
#pragma unroll
                for (int u = 0; u < NW; ++u) acc[u] = 0.0f;
#pragma unroll
                for (int i = 0; i < G; ++i) {
                    int gs[4];
#pragma unroll
                    for (int u = 0; u < NW; ++u) {
                        uint32_t v[4][4];
                        int sc[4];
                        q6_values(w[k][i][u], v);
                        q6_scales(w[k][i][u], jp, sc);
                        q6_accumulate(v, sc, half_bits_to_float(w[k][i][u].dw >> 16), act[i], acc[u], gs);
                    }
                    if constexpr (SUMS) {
                        const int rl = (tb + tk[k]) * TR + r;
                        if (tk[k] < ntiles && rl < n) {
                            int32_t *o = p.sums + (int64_t)(wg_beg + rl) * (p.K / 16) + (16 * i + ln.g) * 16 + 8 * h + jp;
#pragma unroll
                            for (int m = 0; m < 4; ++m) o[2 * m] = gs[m];
                        }
                    }
                }
                const int rl = (tb + tk[k]) * TR + r;
                const bool wr = ks_writer<SBW>(lane) && tk[k] < ntiles && rl < n;
#pragma unroll
                for (int u = 0; u < NW; ++u) {
                    const float q = ks_reduce<SBW>(acc[u]);
                    if (wr) part[(rl * NW + u) * KW + slice] = q;
                }
                tk[k] += S;
                load_tile(tk[k], w[k]);
            }
            remaining -= S;
            if (remaining <= 0) break;
        }
    }
    __syncthreads();
    // 5. each row: the balanced tree over its KW slice sums
    for (int row = (int)threadIdx.x; row < n; row += kWave * WAVES) {
        float out[NW];
#pragma unroll
        for (int u = 0; u < NW; ++u) {
            float q[KW];
#pragma unroll
            for (int k = 0; k < KW; ++k) q[k] = part[(row * NW + u) * KW + k];
#pragma unroll
            for (int hh = KW / 2; hh >= 1; hh /= 2)
#pragma unroll
                for (int t = 0; t < hh; ++t) q[t] = q[2 * t] + q[2 * t + 1];
            out[u] = q[0];
        }
        p.dst[wg_beg + row] = ks_epilogue<EPI>(p, wg_beg + row, out);
    }
}

// ------------------------------------------------------------------------
// Rows of other lengths (up to 8 groups, the last one partial): the Q4_K
// long-row plan (q4k_ksplit.h).  Each wave quantises its slice of every
// group the row has into its own LDS area once, then walks (tile, group)
// steps reading the slice back; the lane map, the per-lane fma chain over
// the groups and the trees are the K-split kernel's, so the outputs are the
// tile kernel's bits (super-blocks past the row, which the tile kernel adds
// as exact zeros, are skipped).
// ------------------------------------------------------------------------

// LDS bytes of one wave's slice of one group: the q8, d8 per 32-value
// block, then the -32 * sum(q8) starting values per 16 values (first halves
// of the slice's blocks, then second halves).
__host__ __device__ constexpr int q6_ks_slice_bytes(int sbw) { return 352 * sbw; }

template <int SBW>
__device__ __forceinline__ void q6_ks_stage_lds(const float (&v)[4 * SBW], int lane, uint8_t *area) {
    constexpr int V = 4 * SBW;
    constexpr int LPB = 32 / V;
    uint32_t word[V / 4];
    float d8;
    int qs, hs;
    ks_quantize_part<V>(v, word, d8, qs, hs);
    uint32_t *q = reinterpret_cast<uint32_t *>(area + lane * V);
#pragma unroll
    for (int w = 0; w < V / 4; ++w) q[w] = word[w];
    const int b = lane / LPB;
    if ((lane & (LPB - 1)) == 0) reinterpret_cast<float *>(area + 256 * SBW)[b] = d8;
    if ((lane & (LPB / 2 - 1)) == 0) {
        const int half = (lane / (LPB / 2)) & 1;
        reinterpret_cast<int *>(area + 288 * SBW)[8 * SBW * half + b] = -32 * hs;
    }
}

// What lane (s, h, j') reads of a staged slice: its four 16-value groups of
// q8 (blocks 8s + 4h + m, half j'), their d8 and starting values.
__device__ __forceinline__ Q6Act q6_ks_read_lds(const uint8_t *area, int sbw, int s, int h, int jp) {
    Q6Act a;
    const uint8_t *q = area + 256 * s + 128 * h + 16 * jp;
#pragma unroll
    for (int m = 0; m < 4; ++m) a.a[m] = *reinterpret_cast<const u32x4 *>(q + 32 * m);
    a.d8 = *reinterpret_cast<const float4 *>(area + 256 * sbw + 4 * (8 * s + 4 * h));
    a.s0 = *reinterpret_cast<const int4 *>(area + 288 * sbw + 4 * (8 * sbw * jp + 8 * s + 4 * h));
    return a;
}

// SBW: 1, 2 or 4 super-blocks per wave and group; GMAX: the most groups per
// row (K <= 4096 GMAX); p.ring_off: LDS offset of the wave areas (after the
// partials).  KT: waves per team for rows shorter than one group (GMAX =
// 1), 0 for the whole 16/SBW, as in the Q4_K kernel.
template <int SBW, int WAVES, int S, int GMAX, bool SUMS = false, int EPI = kEpiNone, bool BATCH = false,
          int KT = 0>
__global__ __launch_bounds__(kWave *WAVES) void gemv_q6k_ksplit_long_kernel(Q4K_GEMV_KERNEL_ARGS) {
    constexpr int KW = 16 / SBW;
    constexpr int KS = KT > 0 ? KT : KW;  // slices a team computes
    constexpr int TR = 16 / SBW;
    constexpr int TEAMS = WAVES / KS;
    constexpr int V = 4 * SBW;
    constexpr int NW = EPI == kEpiGlu ? 2 : 1;  // weights per step (the weight, the gate weight)
    static_assert(TEAMS >= 1 && WAVES % KS == 0, "whole teams");
    static_assert(KS <= KW && (KS == KW || GMAX == 1), "short teams for rows of one partial group only");
    static_assert(!SUMS || (EPI == kEpiNone && !BATCH), "parity variants of the plain product only");
    p = with_head(p, Q4K_GEMV_HEAD_VALUES);
    if constexpr (BATCH) batch_activation(p);
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    float *part = reinterpret_cast<float *>(lds);

    const int lane = threadIdx.x & (kWave - 1);
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int slice = wave % KS, team = wave / KS;
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

    // 1. the slice's activation in every group, issued first; past the row:
    //    zeros (buffer loads; the whole vector is cast, see the Q4_K kernel)
    const __amdgpu_buffer_rsrc_t rx = make_rsrc(p.x, (uint32_t)p.K * 4u);
    float xv[GMAX][V];
#pragma unroll
    for (int i = 0; i < GMAX; ++i) {
        const uint32_t off = (uint32_t)(((16 * i + SBW * slice) * kQK + lane * V) * 4);
#pragma unroll
        for (int k = 0; k < V / 4; ++k) {
            const f32x4 a = __builtin_bit_cast(f32x4, load16(rx, off + 16u * k));
            xv[i][4 * k] = a[0];
            xv[i][4 * k + 1] = a[1];
            xv[i][4 * k + 2] = a[2];
            xv[i][4 * k + 3] = a[3];
        }
    }

    // 2. the first S steps' weights (GLU: and the gate weight's; BATCH: of
    //    the workgroup's weight matrix, none if absent)
    if constexpr (BATCH) batch_weights(p);
    const uint32_t wbytes = BATCH && p.w_absent ? 0u : (uint32_t)(n * p.row_stride);
    __amdgpu_buffer_rsrc_t rsw[NW];
    rsw[0] = make_rsrc(p.w + (int64_t)wg_beg * p.row_stride, wbytes);
    if constexpr (NW == 2) rsw[NW - 1] = make_rsrc(p.gate + (int64_t)wg_beg * p.row_stride, wbytes);
    Q6Lane ln;
    ln.lane = lane;
    ln.g = SBW * slice + s;  // the lane's super-block within each group
    ln.h = h;
    ln.jp = jp;
    const uint32_t blk = (uint32_t)r * (uint32_t)p.row_stride + (uint32_t)ln.g * kQ6Bytes;
    ln.o_lo = blk + 64u * (uint32_t)h + 16u * (uint32_t)jp;
    ln.o_hi = blk + 128u + 32u * (uint32_t)h + 16u * (uint32_t)jp;
    ln.o_sc = blk + 192u + 8u * (uint32_t)h;
    ln.o_d = blk + 206u;
    const uint32_t tile_bytes = (uint32_t)TR * (uint32_t)p.row_stride;
    auto load_step = [&](Step st, Q6Regs(&w)[NW]) {
        const bool ok = st.tile < ntiles && 16 * st.i + ln.g < p.nb;
#pragma unroll
        for (int u = 0; u < NW; ++u)
            q6_load(rsw[u], ln, (uint32_t)(tb + st.tile) * tile_bytes + (uint32_t)st.i * (16u * kQ6Bytes), ok, w[u]);
    };
    Step st[S];
    Q6Regs w[S][NW];
    st[0] = Step{0, 0};
#pragma unroll
    for (int k = 1; k < S; ++k) st[k] = next_step(st[k - 1], G);
#pragma unroll
    for (int k = 0; k < S; ++k) load_step(st[k], w[k]);

    // 3. quantise group 0 of the slice into the wave's LDS area, the other
    //    groups just before the step that first reads them (group 0
    //    unconditionally, so its load stays ahead of the weights)
    uint8_t *area = lds + p.ring_off + wave * G * q6_ks_slice_bytes(SBW);
    auto stage = [&](int i) {
        q6_ks_stage_lds<SBW>(xv[i], lane, area + i * q6_ks_slice_bytes(SBW));
        // lanes read what other lanes of the wave wrote
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    };
    // p.rpw: groups quantised before the first step (1, or all of them)
#pragma unroll
    for (int i = 0; i < GMAX; ++i)
        if (i == 0 || (i < p.rpw && i < G && 16 * i + SBW * slice < p.nb)) stage(i);
    int staged = max(1, min(p.rpw, G));  // groups staged so far

    // 4. the (tile, group) steps, S in flight
    float acc[NW];
#pragma unroll
    for (int u = 0; u < NW; ++u) acc[u] = 0.0f;
    int remaining = ntiles * G;
    if (remaining > 0) {
        for (;;) {
#pragma unroll
            for (int k = 0; k < S; ++k) {
                if (st[k].i >= staged) {  // the first tile reaches a new group
#pragma unroll
                    for (int i = 1; i < GMAX; ++i)
                        if (i >= staged && i <= st[k].i && i < G && 16 * i + SBW * slice < p.nb) stage(i);
                    staged = st[k].i + 1;
                }
                if (16 * st[k].i + SBW * slice < p.nb) {  // the wave's slice reaches this group
                    const Q6Act a = q6_ks_read_lds(area + st[k].i * q6_ks_slice_bytes(SBW), SBW, s, h, jp);
                    int gs[4];
#pragma unroll
                    for (int u = 0; u < NW; ++u) {
                        uint32_t v[4][4];
                        int sc[4];
                        q6_values(w[k][u], v);
                        q6_scales(w[k][u], jp, sc);
                        q6_accumulate(v, sc, half_bits_to_float(w[k][u].dw >> 16), a, acc[u], gs);
                    }
                    if constexpr (SUMS) {
                        const int rl = (tb + st[k].tile) * TR + r;
                        const int kb = 16 * st[k].i + ln.g;
                        if (st[k].tile < ntiles && rl < n && kb < p.nb) {
                            int32_t *o = p.sums + (int64_t)(wg_beg + rl) * (p.K / 16) + kb * 16 + 8 * h + jp;
#pragma unroll
                            for (int m = 0; m < 4; ++m) o[2 * m] = gs[m];
                        }
                    }
                }
                if (st[k].i == G - 1) {
                    const int rl = (tb + st[k].tile) * TR + r;
                    const bool wr = ks_writer<SBW>(lane) && st[k].tile < ntiles && rl < n;
#pragma unroll
                    for (int u = 0; u < NW; ++u) {
                        const float q = ks_reduce<SBW>(acc[u]);
                        if (wr) part[(rl * NW + u) * KS + slice] = q;
                        acc[u] = 0.0f;
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
    for (int row = (int)threadIdx.x; row < n; row += kWave * WAVES) {
        float out[NW];
#pragma unroll
        for (int u = 0; u < NW; ++u) {
            float q[KW];
#pragma unroll
            for (int k = 0; k < KW; ++k) q[k] = k < KS ? part[(row * NW + u) * KS + k] : 0.0f;
#pragma unroll
            for (int hh = KW / 2; hh >= 1; hh /= 2)
#pragma unroll
                for (int t = 0; t < hh; ++t) q[t] = q[2 * t] + q[2 * t + 1];
            out[u] = q[0];
        }
        p.dst[wg_beg + row] = ks_epilogue<EPI>(p, wg_beg + row, out);
    }
}

__host__ __device__ constexpr int q6_ksplit_long_lds_bytes(int rows_per_wg, int sbw, int waves, int G, int nw = 1,
                                                           int kt = 0) {
    return ksplit_long_part_bytes(rows_per_wg, sbw, nw, kt) + waves * G * q6_ks_slice_bytes(sbw);
}

// Several Q6_K columns of rows shorter than one group in short teams (two
// columns of rows of 3 to 8 blocks, three or four of 3 or 4): the Q6_K tile
// kernel reduces several columns in the Q4_K tile kernel's order, so for
// these rows its tree is the one-column tree (the reasoning of
// gemv_q4k_ksplit_short_nc_kernel), and this is the one-column short-team
// kernel with NC accumulators per lane.  p.ring_off: LDS offset of the wave
// areas (after the rows x NC x KT partials).
__host__ __device__ constexpr int q6_ksplit_short_nc_lds_bytes(int rows_per_wg, int nc, int sbw, int kt, int waves) {
    return ksplit_short_nc_part_bytes(rows_per_wg, nc, kt) + waves * nc * q6_ks_slice_bytes(sbw);
}

template <int NC, int SBW, int WAVES, int S, int KT, bool SUMS = false, int P = 2>
__global__ __launch_bounds__(kWave *WAVES) void gemv_q6k_ksplit_short_nc_kernel(Q4K_GEMV_KERNEL_ARGS) {
    constexpr int KW = 16 / SBW;
    constexpr int TR = 16 / SBW;
    constexpr int TEAMS = WAVES / KT;
    constexpr int V = 4 * SBW;
    constexpr bool RC4 = P == 4;  // wave w: super-blocks w and w + 4 (gemv_q4k_ksplit_short_nc_kernel)
    static_assert(NC >= 2 && NC <= 4 && TEAMS >= 1 && WAVES % KT == 0 && KT < KW, "short teams, 2-4 columns");
    static_assert(!RC4 || (SBW == 2 && KT == 4 && NC >= 3), "residue classes mod 4: rows of 5 to 8 blocks");
    p = with_head(p, Q4K_GEMV_HEAD_VALUES);
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    float *part = reinterpret_cast<float *>(lds);

    const int lane = threadIdx.x & (kWave - 1);
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int slice = wave % KT, team = wave / KT;
    const int r = lane / (4 * SBW), s = (lane >> 2) & (SBW - 1);
    const int h = (lane >> 1) & 1, jp = lane & 1;

    const int b = (int)blockIdx.x;
    const int wg_beg = b * p.rows_base + min(b, p.rows_extra);
    const int n = p.rows_base + (b < p.rows_extra ? 1 : 0);
    const int nt = (n + TR - 1) / TR;
    const int tq = nt / TEAMS, trem = nt - tq * TEAMS;
    const int tb = team * tq + min(team, trem);
    const int ntiles = tq + (team < trem ? 1 : 0);

    // 1. the slice of every column, issued first; past the row: zeros
    float xv[NC][V];
#pragma unroll
    for (int c = 0; c < NC; ++c) {
        const __amdgpu_buffer_rsrc_t rx = make_rsrc(p.x + (int64_t)c * p.ldx, (uint32_t)p.K * 4u);
        const uint32_t off = RC4 ? (uint32_t)(((slice + 4 * (lane >> 5)) * kQK + (lane & 31) * V) * 4)
                                 : (uint32_t)(((SBW * slice) * kQK + lane * V) * 4);
#pragma unroll
        for (int k = 0; k < V / 4; ++k) {
            const f32x4 a = __builtin_bit_cast(f32x4, load16(rx, off + 16u * k));
            xv[c][4 * k] = a[0];
            xv[c][4 * k + 1] = a[1];
            xv[c][4 * k + 2] = a[2];
            xv[c][4 * k + 3] = a[3];
        }
    }

    // 2. the first S tiles' weights (past the workgroup's rows or the row's
    //    blocks: zeros)
    const __amdgpu_buffer_rsrc_t rsw = make_rsrc(p.w + (int64_t)wg_beg * p.row_stride, (uint32_t)(n * p.row_stride));
    Q6Lane ln;
    ln.lane = lane;
    ln.g = RC4 ? slice + 4 * s : SBW * slice + s;
    ln.h = h;
    ln.jp = jp;
    const uint32_t blk = (uint32_t)r * (uint32_t)p.row_stride + (uint32_t)ln.g * kQ6Bytes;
    ln.o_lo = blk + 64u * (uint32_t)h + 16u * (uint32_t)jp;
    ln.o_hi = blk + 128u + 32u * (uint32_t)h + 16u * (uint32_t)jp;
    ln.o_sc = blk + 192u + 8u * (uint32_t)h;
    ln.o_d = blk + 206u;
    const uint32_t tile_bytes = (uint32_t)TR * (uint32_t)p.row_stride;
    auto load_tile = [&](int t, Q6Regs &w) {
        const bool ok = t < ntiles && ln.g < p.nb;
        q6_load(rsw, ln, (uint32_t)(tb + t) * tile_bytes, ok, w);
    };
    int tk[S];
    Q6Regs w[S];
#pragma unroll
    for (int k = 0; k < S; ++k) {
        tk[k] = k;
        load_tile(k, w[k]);
    }

    // 3. quantise every column's slice into the wave's LDS areas
    uint8_t *area = lds + p.ring_off + wave * NC * q6_ks_slice_bytes(SBW);
#pragma unroll
    for (int c = 0; c < NC; ++c) q6_ks_stage_lds<SBW>(xv[c], lane, area + c * q6_ks_slice_bytes(SBW));
    // lanes read what other lanes of the wave wrote
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");

    // 4. the tiles, S in flight
    int remaining = ntiles;
    if (remaining > 0) {
        for (;;) {
#pragma unroll
            for (int k = 0; k < S; ++k) {
                uint32_t v[4][4];
                int sc[4];
                q6_values(w[k], v);
                q6_scales(w[k], jp, sc);
                const float d = half_bits_to_float(w[k].dw >> 16);
                const int rl = (tb + tk[k]) * TR + r;
                float acc[NC];
#pragma unroll
                for (int c = 0; c < NC; ++c) {
                    acc[c] = 0.0f;
                    const Q6Act a = q6_ks_read_lds(area + c * q6_ks_slice_bytes(SBW), SBW, s, h, jp);
                    int gs[4];
                    q6_accumulate(v, sc, d, a, acc[c], gs);
                    if constexpr (SUMS) {
                        if (tk[k] < ntiles && rl < n && ln.g < p.nb) {
                            int32_t *o =
                                p.sums + ((int64_t)c * p.M + wg_beg + rl) * (p.K / 16) + ln.g * 16 + 8 * h + jp;
#pragma unroll
                            for (int m = 0; m < 4; ++m) o[2 * m] = gs[m];
                        }
                    }
                }
                const bool wr = ks_writer<SBW>(lane) && tk[k] < ntiles && rl < n;
#pragma unroll
                for (int c = 0; c < NC; ++c) {
                    const float q = RC4 ? ks_reduce_rc4(acc[c]) : ks_reduce<SBW>(acc[c]);
                    if (wr) part[(rl * NC + c) * KT + slice] = q;
                }
                tk[k] += S;
                load_tile(tk[k], w[k]);
            }
            remaining -= S;
            if (remaining <= 0) break;
        }
    }
    __syncthreads();
    // 5. each (row, column): the balanced tree over the 16/SBW slice sums
    //    (+0 for the slices past the team)
    for (int e = (int)threadIdx.x; e < n * NC; e += kWave * WAVES) {
        const int row = e / NC, c = e - row * NC;
        float q[KW];
#pragma unroll
        for (int k = 0; k < KW; ++k) q[k] = k < KT ? part[(row * NC + c) * KT + k] : 0.0f;
#pragma unroll
        for (int hh = KW / 2; hh >= 1; hh /= 2)
#pragma unroll
            for (int t = 0; t < hh; ++t) q[t] = q[2 * t] + q[2 * t + 1];
        p.dst[(int64_t)c * p.ld_dst + wg_beg + row] = q[0];
    }
}

// The long-row variants: those of the Q4_K kernel (SBW 1 or 2 for rows of
// up to 8 groups, 4 for rows of up to 4; three or four steps in flight in
// workgroups of up to 8 waves).
constexpr bool q6_ksplit_long_exists(int sbw, int waves, int slots, int gmax) {
    return ksplit_long_exists(sbw, waves, slots, gmax);
}

template <bool SUMS, int SBW, int WAVES, int S>
const void *q6_ksplit_long_sym_g(int gmax) {
    if constexpr (q6_ksplit_long_exists(SBW, WAVES, S, 4))
        if (gmax == 4) return reinterpret_cast<const void *>(&gemv_q6k_ksplit_long_kernel<SBW, WAVES, S, 4, SUMS>);
    if constexpr (q6_ksplit_long_exists(SBW, WAVES, S, 8))
        if (gmax == 8) return reinterpret_cast<const void *>(&gemv_q6k_ksplit_long_kernel<SBW, WAVES, S, 8, SUMS>);
    return nullptr;
}

// The Q6_K long-row K-split kernel for rows of G groups (G <= 8), or null.
template <bool SUMS>
const void *q6_ksplit_long_kernel(int sbw, int waves, int slots, int G) {
    const int gmax = G <= 4 ? 4 : 8;
    if (G > 8) return nullptr;
    auto pick = [&](auto sbw_c) -> const void * {
        constexpr int B = decltype(sbw_c)::value;
        auto by_slots = [&](auto waves_c) -> const void * {
            constexpr int W = decltype(waves_c)::value;
            switch (slots) {
                case 1: return q6_ksplit_long_sym_g<SUMS, B, W, 1>(gmax);
                case 2: return q6_ksplit_long_sym_g<SUMS, B, W, 2>(gmax);
                case 3: return q6_ksplit_long_sym_g<SUMS, B, W, 3>(gmax);
                case 4: return q6_ksplit_long_sym_g<SUMS, B, W, 4>(gmax);
                default: return nullptr;
            }
        };
        if (waves == 4) return by_slots(std::integral_constant<int, 4>{});
        if (waves == 8) return by_slots(std::integral_constant<int, 8>{});
        if (waves == 16) return by_slots(std::integral_constant<int, 16>{});
        return nullptr;
    };
    if (sbw == 1) return pick(std::integral_constant<int, 1>{});
    if (sbw == 2) return pick(std::integral_constant<int, 2>{});
    if (sbw == 4) return pick(std::integral_constant<int, 4>{});
    return nullptr;
}

// The instantiated variants: SBW 1, 2, 4 in whole teams, one or two tiles in
// flight, rows of one or two groups (two tiles of two-group rows not at 16
// waves, where they would spill registers).
constexpr bool q6_ksplit_exists(int sbw, int waves, int slots, int G) {
    return (sbw == 1 || sbw == 2 || sbw == 4) && (waves == 4 || waves == 8 || waves == 16) && waves % (16 / sbw) == 0 &&
           (slots == 1 || slots == 2) && (G == 1 || G == 2) && !(G == 2 && slots == 2 && waves == 16);
}

template <bool SUMS, int SBW, int WAVES, int S>
const void *q6_ksplit_sym_g(int G) {
    if constexpr (q6_ksplit_exists(SBW, WAVES, S, 1))
        if (G == 1) return reinterpret_cast<const void *>(&gemv_q6k_ksplit_kernel<SBW, WAVES, S, 1, SUMS>);
    if constexpr (q6_ksplit_exists(SBW, WAVES, S, 2))
        if (G == 2) return reinterpret_cast<const void *>(&gemv_q6k_ksplit_kernel<SBW, WAVES, S, 2, SUMS>);
    return nullptr;
}

template <bool SUMS, int SBW>
const void *q6_ksplit_sym_w(int waves, int slots, int G) {
    if (waves == 4) return slots == 2 ? q6_ksplit_sym_g<SUMS, SBW, 4, 2>(G) : q6_ksplit_sym_g<SUMS, SBW, 4, 1>(G);
    if (waves == 8) return slots == 2 ? q6_ksplit_sym_g<SUMS, SBW, 8, 2>(G) : q6_ksplit_sym_g<SUMS, SBW, 8, 1>(G);
    if (waves == 16) return slots == 2 ? q6_ksplit_sym_g<SUMS, SBW, 16, 2>(G) : q6_ksplit_sym_g<SUMS, SBW, 16, 1>(G);
    return nullptr;
}

// The fused-epilogue variants (EPI = kEpiBias or kEpiGlu): the plain
// kernels' shapes with one step in flight, or two in workgroups of up to 8
// waves; with a gate weight 16-wave workgroups only at one super-block per
// wave (elsewhere the gate weight's registers spilled).
constexpr bool q6_ksplit_epi_exists(int sbw, int waves, int slots, int G, bool glu) {
    return (slots == 1 || (slots == 2 && waves <= 8)) && !(glu && waves == 16 && sbw != 1) &&
           q6_ksplit_exists(sbw, waves, slots, G);
}
constexpr bool q6_ksplit_long_epi_exists(int sbw, int waves, int slots, int gmax, bool glu) {
    return (slots == 1 || (slots == 2 && waves <= 8)) && !(glu && waves == 16 && sbw != 1) &&
           q6_ksplit_long_exists(sbw, waves, slots, gmax);
}

// The batched variants: in the shapes the automatic rules pick (4
// super-blocks per wave in 4-wave workgroups, 2 in 8-wave ones).
constexpr bool q6_ksplit_batch_ok(int sbw, int waves) { return (sbw == 4 && waves == 4) || (sbw == 2 && waves == 8); }

// The fused (EPI kEpiBias, kEpiGlu) or batched (BATCH; any EPI) Q6_K K-split
// kernel (rows of 1 or 2 groups, long = false; any other length up to 8
// groups, long = true) of a launch shape, or null.
template <int EPI, bool BATCH = false>
const void *q6_ksplit_kernel_epi(bool lng, int sbw, int waves, int slots, int G) {
    const int gsel = lng ? (G <= 4 ? 4 : 8) : G;
    if (lng ? G > 8 : (G != 1 && G != 2)) return nullptr;
    auto pick = [&](auto sbw_c) -> const void * {
        constexpr int B = decltype(sbw_c)::value;
        auto by = [&](auto waves_c, auto s_c, auto g_c) -> const void * {
            constexpr int W = decltype(waves_c)::value, SS = decltype(s_c)::value, GG = decltype(g_c)::value;
            if constexpr (GG <= 2) {
                if constexpr (q6_ksplit_epi_exists(B, W, SS, GG, EPI == kEpiGlu) && (!BATCH || q6_ksplit_batch_ok(B, W)))
                    if (!lng)
                        return reinterpret_cast<const void *>(&gemv_q6k_ksplit_kernel<B, W, SS, GG, false, EPI, BATCH>);
            } else {
                if constexpr (q6_ksplit_long_epi_exists(B, W, SS, GG, EPI == kEpiGlu) &&
                              (!BATCH || q6_ksplit_batch_ok(B, W)))
                    if (lng)
                        return reinterpret_cast<const void *>(
                            &gemv_q6k_ksplit_long_kernel<B, W, SS, GG, false, EPI, BATCH>);
            }
            return nullptr;
        };
        auto by_g = [&](auto waves_c, auto s_c) -> const void * {
            switch (gsel) {
                case 1: return by(waves_c, s_c, std::integral_constant<int, 1>{});
                case 2: return by(waves_c, s_c, std::integral_constant<int, 2>{});
                case 4: return by(waves_c, s_c, std::integral_constant<int, 4>{});
                case 8: return by(waves_c, s_c, std::integral_constant<int, 8>{});
                default: return nullptr;
            }
        };
        auto by_w = [&](auto waves_c) -> const void * {
            if (slots == 1) return by_g(waves_c, std::integral_constant<int, 1>{});
            if (slots == 2) return by_g(waves_c, std::integral_constant<int, 2>{});
            return nullptr;
        };
        if (waves == 4) return by_w(std::integral_constant<int, 4>{});
        if (waves == 8) return by_w(std::integral_constant<int, 8>{});
        if (waves == 16) return by_w(std::integral_constant<int, 16>{});
        return nullptr;
    };
    if (sbw == 1) return pick(std::integral_constant<int, 1>{});
    if (sbw == 2) return pick(std::integral_constant<int, 2>{});
    if (sbw == 4) return pick(std::integral_constant<int, 4>{});
    return nullptr;
}

// The Q6_K K-split kernel of a launch shape, or null when not instantiated.
template <bool SUMS>
const void *q6_ksplit_kernel(int sbw, int waves, int slots, int G) {
    switch (sbw) {
        case 1: return q6_ksplit_sym_w<SUMS, 1>(waves, slots, G);
        case 2: return q6_ksplit_sym_w<SUMS, 2>(waves, slots, G);
        case 4: return q6_ksplit_sym_w<SUMS, 4>(waves, slots, G);
        default: return nullptr;
    }
}

}  // namespace q4k
