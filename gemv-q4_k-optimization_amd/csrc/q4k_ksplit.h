// q4k_ksplit.h -- the K-split Q4_K GEMV kernel for gfx950: one F32
// activation column, rows of one or two 16-block groups (K = 4096 or 8192).
//
// The waves of a workgroup split each row's super-blocks between them rather
// than its rows.  A team of KW = 16/SBW waves shares every row the team
// walks: wave w of the team owns the SBW super-blocks [16i + SBW*w, +SBW) of
// each group i.  A wave step covers TR = 16/SBW rows of that slice, four
// lanes per super-block as in the tile kernel:
//
//   lane = 4*SBW*r + 4*s + j    r: row of the step (0..TR-1)
//                               s: super-block of the slice (0..SBW-1)
//                               j: 32-byte qs chunk (sub-blocks 2j, 2j+1)
//
// so a lane again owns two whole sub-blocks of one super-block and forms
// complete int32 sub-block sums.
//
// Activation.  A wave needs only its own slice, SBW*256 values per group.
// Each lane loads 4*SBW consecutive values with 16-byte loads, the wave
// quantises them in registers with the Q8_1 arithmetic of the other kernels
// (32/(4*SBW) lanes per 32-value block; ggml's quantize_q8_1, called at
// kernels/mmvq.cu:734), and ds_bpermute hands each lane the 64 q8 of its
// two sub-blocks and their (d8, d8 * sum q8).  Those are cross-lane reads
// through the LDS crossbar: no LDS memory and no barrier.  So every wave
// issues its activation load and then its first weight loads as soon as it
// starts, and the quantisation runs while the weights are in flight.  LDS
// holds only the (row, slice) partials, which meet once, after the last
// step, behind the kernel's only barrier.
//
// Summation order.  A lane's value is the fma chain over the row's groups
// that a tile-kernel lane owning the same super-block and chunk forms
// (accumulate).  The four chunks of a super-block, the super-blocks of a
// slice and the slices of a row then combine in the balanced tree over the
// 16 super-block positions of a group that the tile kernel's wave_sum forms
// (at every level pairs (2t, 2t+1)): the DPP steps inside a wave are
// wave_sum's first steps, and the tree over the slices finishes it.  The
// outputs are therefore bit for bit the tile kernel's, for every SBW, team
// count and workgroup count (tested).
//
// Reference: the product is kernels/mmvq.cu:150-344 with the vec-dot of
// kernels/vecdotq.cuh:775-819 and :457-483, for one column.
#pragma once

#include <hip/hip_runtime.h>

#include <type_traits>

#include "q4k_gemv_kernels.h"

namespace q4k {

// One lane's V <= 32 values, part of one 32-value block spread over the
// 32/V lanes of an aligned lane group: V/4 packed q8 dwords, the block's
// half(d) widened, and the int32 sum of its 32 q8 (in every lane of the
// group) and of the 16-value half the lane's values lie in (V <= 16).  The
// arithmetic and reduction trees are quantize_block_part's.
template <int V>
__device__ __forceinline__ void ks_quantize_part(const float (&v)[V], uint32_t (&word)[V / 4], float &d8,
                                                 int &qsum, int &hsum) {
    constexpr int LPB = 32 / V;
    float amax = 0.0f;
#pragma unroll
    for (int k = 0; k < V; ++k) amax = fmaxf(amax, fabsf(v[k]));
    if constexpr (LPB >= 2) amax = dpp_max_xor1(amax);
    if constexpr (LPB >= 4) amax = dpp_max_xor2(amax);
    if constexpr (LPB >= 8) amax = dpp_max_half_mirror(amax);
    const float d = div127(amax);
    int s[1];
    if (amax != 0.0f) {
        quantize_values<V, 1>(v, d, __builtin_amdgcn_rcpf(d), word, s);
    } else {
#pragma unroll
        for (int w = 0; w < V / 4; ++w) word[w] = 0;
        s[0] = 0;
    }
    int t = s[0];
    if constexpr (LPB >= 4) t += dpp<kDppXor1>(t);
    if constexpr (LPB >= 8) t += dpp<kDppXor2>(t);
    hsum = t;
    if constexpr (LPB == 2) t += dpp<kDppXor1>(t);
    if constexpr (LPB == 4) t += dpp<kDppXor2>(t);
    if constexpr (LPB == 8) t += dpp<kDppHalfMirror>(t);
    qsum = t;
    d8 = (float)(_Float16)d;
}

__device__ __forceinline__ uint32_t bperm(int src_lane, uint32_t v) {
    return (uint32_t)__builtin_amdgcn_ds_bpermute(src_lane * 4, (int)v);
}
__device__ __forceinline__ float bpermf(int src_lane, float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_ds_bpermute(src_lane * 4, __builtin_bit_cast(int, v)));
}

// Block b of a slice of consecutive super-blocks starting at block blk0.
struct KsBlocks {
    int blk0;
    __device__ int operator()(int b) const { return blk0 + b; }
};

// The wave's activation slice of one group: lane L holds the 4*SBW values
// [L*4*SBW, +4*SBW) of the slice; returns what lane (r, s, j) reads (the q8
// of sub-blocks 2j and 2j+1 of super-block s and their (d8, d8 * sum q8)).
// sq (parity variants; null in the product kernels) gets the int32 sums of
// the slice's blocks, from each block's first lane, at sq[blk(b)] (blk:
// the row's block index of the slice's block b).
template <int SBW, class BlockOf = KsBlocks>
__device__ __forceinline__ LaneAct ks_stage(const float (&v)[4 * SBW], int lane, int s, int j, int32_t *sq,
                                            BlockOf blk) {
    constexpr int V = 4 * SBW;
    LaneAct a;
    if constexpr (V <= 32) {
        constexpr int LPB = 32 / V;
        uint32_t word[V / 4];
        float d8;
        int qs, hs;
        ks_quantize_part<V>(v, word, d8, qs, hs);
        if (sq && (lane & (LPB - 1)) == 0) sq[blk(lane / LPB)] = qs;
        // dword t of lane (s, j) = values 256s + 64j + 4t: word t % SBW of
        // lane (64s + 16j + t) / SBW
        const int base = 64 * s + 16 * j;
        uint32_t q[16];
#pragma unroll
        for (int t = 0; t < 16; ++t) q[t] = bperm((base + t) / SBW, word[t % SBW]);
        a.a0 = u32x4{q[0], q[1], q[2], q[3]};
        a.a1 = u32x4{q[4], q[5], q[6], q[7]};
        a.b0 = u32x4{q[8], q[9], q[10], q[11]};
        a.b1 = u32x4{q[12], q[13], q[14], q[15]};
        // block 8s + 2j + h starts in lane (8s + 2j + h) * LPB
        const int l0 = (8 * s + 2 * j) * LPB, l1 = l0 + LPB;
        const float d8a = bpermf(l0, d8), d8b = bpermf(l1, d8);
        const int sa = (int)bperm(l0, (uint32_t)qs), sb = (int)bperm(l1, (uint32_t)qs);
        a.dk = make_float4(d8a, d8a * (float)sa, d8b, d8b * (float)sb);
    } else {  // SBW = 16: a lane's 64 values are its own two sub-blocks
        float v0[32], v1[32];
#pragma unroll
        for (int k = 0; k < 32; ++k) {
            v0[k] = v[k];
            v1[k] = v[32 + k];
        }
        uint32_t w0[8], w1[8];
        float d0, d1;
        int s0, s1, h0, h1;
        ks_quantize_part<32>(v0, w0, d0, s0, h0);
        ks_quantize_part<32>(v1, w1, d1, s1, h1);
        if (sq) {
            sq[blk(2 * lane)] = s0;
            sq[blk(2 * lane + 1)] = s1;
        }
        a.a0 = u32x4{w0[0], w0[1], w0[2], w0[3]};
        a.a1 = u32x4{w0[4], w0[5], w0[6], w0[7]};
        a.b0 = u32x4{w1[0], w1[1], w1[2], w1[3]};
        a.b1 = u32x4{w1[4], w1[5], w1[6], w1[7]};
        a.dk = make_float4(d0, d0 * (float)s0, d1, d1 * (float)s1);
    }
    return a;
}

// Sum of a step row's slice: the four chunks of each super-block (quad),
// then the SBW super-blocks of the slice -- wave_sum's first steps; valid in
// the last lane of each 4*SBW-lane row group (ks_writer).
template <int SBW>
__device__ __forceinline__ float ks_reduce(float v) {
    v += dppf<kDppXor1>(v);
    v += dppf<kDppXor2>(v);
    if constexpr (SBW >= 2) v += dppf<kDppRor4>(v);
    if constexpr (SBW >= 4) v += dppf<kDppRor8>(v);
    if constexpr (SBW >= 8) v += dppf_rows<kDppBcast15, 0xa>(v);
    if constexpr (SBW >= 16) v += dppf_rows<kDppBcast31, 0xc>(v);
    return v;
}

// Two super-blocks per wave that lie 4 apart in the row (residue classes
// mod 4): the pair first, then the chunks -- the several-column tile
// kernel's order for a four-column tree (column_sums: g and g^4, then the
// chunks).  The sum lands in the last lane of each 8-lane row group.
__device__ __forceinline__ float ks_reduce_rc4(float v) {
    v += dppf<kDppRor4>(v);
    v += dppf<kDppXor1>(v);
    v += dppf<kDppXor2>(v);
    return v;
}

template <int SBW>
__device__ __forceinline__ bool ks_writer(int lane) {
    return (lane & (4 * SBW - 1)) == 4 * SBW - 1;
}

// The fused epilogues of the one-column K-split kernels (EPI: kEpiBias,
// kEpiGlu), applied where a row's slice sums meet: the tile kernel's
// ring_flush arithmetic on the same products.  q[0]: the product with the
// weight, q[1] (GLU): the product with the gate weight.
template <int EPI>
__device__ __forceinline__ float ks_epilogue(const GemvParams &p, int row, const float (&q)[EPI == kEpiGlu ? 2 : 1]) {
    if constexpr (EPI == kEpiGlu) {
        const float up = p.bias ? q[0] + p.bias[row] : q[0];
        const float g = p.gate_bias ? q[1] + p.gate_bias[row] : q[1];
        return glu_apply(p.glu_op, up, g);
    } else if constexpr (EPI == kEpiBias) {
        return q[0] + p.bias[row];
    } else {
        return q[0];
    }
}

// SBW: super-blocks per wave and group (1, 2, 4, 16), WAVES: waves per
// workgroup (whole teams of 16/SBW), S: row tiles in flight per wave, G:
// groups per row (K = 4096 G).  SUMS: the parity variant, which also stores
// every lane's int32 sub-block sums and the activation's block sums.  EPI:
// the fused epilogue (kEpiBias: dst = product + bias; kEpiGlu: each step
// also loads the same rows of the gate weight p.gate, and dst = glu(product
// + bias, gate product + gate bias); kernels/mmvq.cu:254-262, :309-336).
// BATCH: one launch over dst channels (grid y) and samples (grid z), each
// workgroup first selecting its activation and dst slice and, after its
// activation loads, its weight matrix (batch_activation, batch_weights, as
// the tile kernel).  Rows: the workgroup's share (rows_base / rows_extra, as
// the tile kernel), tiles of TR rows split contiguously over the teams.
template <int SBW, int WAVES, int S, int G, bool SUMS = false, int EPI = kEpiNone, bool BATCH = false>
__global__ __launch_bounds__(kWave *WAVES) void gemv_q4k_ksplit_kernel(Q4K_GEMV_KERNEL_ARGS) {
    constexpr int KW = 16 / SBW;  // waves sharing a row
    constexpr int TR = 16 / SBW;  // rows per wave step
    constexpr int TEAMS = WAVES / KW;
    constexpr int V = 4 * SBW;    // activation values per lane and group
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
    const int r = lane / (4 * SBW), s = (lane >> 2) & (SBW - 1), j = lane & 3;

    // the workgroup's rows, and the team's tiles of TR rows among them
    const int b = (int)blockIdx.x;
    const int wg_beg = b * p.rows_base + min(b, p.rows_extra);
    const int n = p.rows_base + (b < p.rows_extra ? 1 : 0);
    const int nt = (n + TR - 1) / TR;
    const int tq = nt / TEAMS, trem = nt - tq * TEAMS;
    const int tb = team * tq + min(team, trem);
    const int ntiles = tq + (team < trem ? 1 : 0);

    // 1. the slice's activation values, issued first (a CU returns vector
    //    loads in order, and these come from L2); 16-byte loads only (the
    //    host launches this kernel for 16-byte aligned activations: with an
    //    element-load path beside them the compiler waited for every
    //    activation load before issuing the first weight load)
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

    // 2. the first S tiles' weights: the workgroup's rows as one buffer, so
    //    rows past its share read zeros without memory traffic (GLU: the
    //    same rows of the gate weight, at the same offsets; BATCH: of the
    //    workgroup's weight matrix, none for an absent expert)
    if constexpr (BATCH) batch_weights(p);
    const uint32_t wbytes = BATCH && p.w_absent ? 0u : (uint32_t)(n * p.row_stride);
    __amdgpu_buffer_rsrc_t rsw[NW];
    rsw[0] = make_rsrc(p.w + (int64_t)wg_beg * p.row_stride, wbytes);
    if constexpr (NW == 2) rsw[NW - 1] = make_rsrc(p.gate + (int64_t)wg_beg * p.row_stride, wbytes);
    const uint32_t lrow = (uint32_t)r * (uint32_t)p.row_stride;
    const uint32_t lh = lrow + (uint32_t)((SBW * slice + s) * kBlockBytes);
    const uint32_t lq = lh + 16u + 32u * (uint32_t)j;
    const uint32_t tile_bytes = (uint32_t)TR * (uint32_t)p.row_stride;
    auto load_tile = [&](int t, RowRegs(&w)[G][NW]) {
        const bool ok = t < ntiles;
        const uint32_t base = (uint32_t)(tb + t) * tile_bytes;
#pragma unroll
        for (int i = 0; i < G; ++i) {
            const uint32_t gi = (uint32_t)i * (16u * kBlockBytes);
            const uint32_t oh = ok ? base + gi + lh : kOOB;
            const uint32_t oq = ok ? base + gi + lq : kOOB;
#pragma unroll
            for (int u = 0; u < NW; ++u) {
                w[i][u].h = load16(rsw[u], oh);
                w[i][u].q0 = load16(rsw[u], oq);
                w[i][u].q1 = load16(rsw[u], oq + 16u);
            }
        }
    };
    int tk[S];
    RowRegs w[S][G][NW];
#pragma unroll
    for (int k = 0; k < S; ++k) {
        tk[k] = k;
        load_tile(k, w[k]);
    }

    // 3. quantise the slice and hand each lane its sub-blocks
    LaneAct act[G];
#pragma unroll
    for (int i = 0; i < G; ++i)
        act[i] = ks_stage<SBW>(xv[i], lane, s, j, SUMS ? p.sq : nullptr, KsBlocks{(16 * i + SBW * slice) * 8});

    Lane ln;
    ln.lane = lane;
    ln.g = SBW * slice + s;
    ln.j = j;
    ln.sel = make_scale_sel(j);
    // 4. the tiles, S in flight; slot k is consumed and then reloaded with
    //    the tile S further on (past the team's tiles: zeros, no traffic)
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
                    int sa, sb;
#pragma unroll
                    for (int u = 0; u < NW; ++u) {
                        const RowScales sc = row_scales(w[k][i][u], ln);
                        accumulate(w[k][i][u], sc, act[i], acc[u], sa, sb);
                    }
                    if constexpr (SUMS) {
                        const int rl = (tb + tk[k]) * TR + r;
                        if (tk[k] < ntiles && rl < n) {
                            int32_t *o = p.sums + (int64_t)(wg_beg + rl) * (p.K / 32) + (16 * i + ln.g) * 8 + 2 * j;
                            o[0] = sa;
                            o[1] = sb;
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
    // 5. each row: the balanced tree over its KW slice sums, then the epilogue
    for (int row = (int)threadIdx.x; row < n; row += kWave * WAVES) {
        float out[NW];
#pragma unroll
        for (int u = 0; u < NW; ++u) {
            float q[KW];
#pragma unroll
            for (int k = 0; k < KW; ++k) q[k] = part[(row * NW + u) * KW + k];
#pragma unroll
            for (int h = KW / 2; h >= 1; h /= 2)
#pragma unroll
                for (int t = 0; t < h; ++t) q[t] = q[2 * t] + q[2 * t + 1];
            out[u] = q[0];
        }
        p.dst[wg_beg + row] = ks_epilogue<EPI>(p, wg_beg + row, out);
    }
}

// LDS bytes of a K-split launch: the (row, slice) partials of the largest
// workgroup share (nw: 2 with a gate weight, else 1).
__host__ __device__ constexpr int ksplit_lds_bytes(int rows_per_wg, int sbw, int nw = 1) {
    return rows_per_wg * (16 / sbw) * 4 * nw;
}

// ------------------------------------------------------------------------
// Rows of any length: G groups of 16 super-blocks (G <= GMAX), the last one
// possibly partial.  The activation of G groups would not fit the
// registers, so each wave keeps its quantised slice of every group in a
// wave-private LDS area -- the slice's q8, linear, then one (d8, d8 * sum
// q8) pair per 32-value block -- written once by the wave and read back by
// each lane at each step.  No other wave reads it, so there is still no
// barrier before the weight loads.  The activation is read through a buffer
// descriptor of exactly K floats: groups past the row read zeros, so every
// load is issued unconditionally (the compiler then waits for exactly the
// loads a step needs).  Steps walk (tile, group) pairs, S in flight.
// Super-blocks past the row's end hold zero weights; a tile-kernel lane
// adds exactly zero for them (its accumulator is never -0), so the wave
// skips groups its slice does not reach and the sums stay the tile
// kernel's bits.
// ------------------------------------------------------------------------

// LDS bytes of one wave's quantised slice of one group (q8, then a float2
// per 32-value block).
__host__ __device__ constexpr int ks_slice_bytes(int sbw) { return 320 * sbw; }

// The wave's slice of one group, quantised (lane L: values [L*V, +V)), into
// its LDS area; sq (parity variants) gets the int32 sums of the blocks that
// lie inside the row (blk0: the slice's first block in the row; blk_hi, two
// super-blocks per wave: how many blocks further on the second one lies).
template <int SBW>
__device__ __forceinline__ void ks_stage_lds(const float (&v)[4 * SBW], int lane, uint8_t *area, int32_t *sq,
                                             int blk0, int nblk, int blk_hi = 0) {
    constexpr int V = 4 * SBW;
    constexpr int LPB = 32 / V;
    uint32_t word[V / 4];
    float d8;
    int qs, hs;
    ks_quantize_part<V>(v, word, d8, qs, hs);
    uint32_t *q = reinterpret_cast<uint32_t *>(area + lane * V);
#pragma unroll
    for (int w = 0; w < V / 4; ++w) q[w] = word[w];
    if ((lane & (LPB - 1)) == 0) {
        const int b = lane / LPB;
        reinterpret_cast<float2 *>(area + 256 * SBW)[b] = make_float2(d8, d8 * (float)qs);
        const int bi = blk0 + b + (b >> 3) * blk_hi;  // (blk_hi: the second super-block's blocks moved)
        if (sq && bi < nblk) sq[bi] = qs;
    }
}

// What lane (s, j) reads of a staged slice: the q8 of sub-blocks 2j, 2j+1
// of super-block s and their two (d8, d8 * sum q8) pairs.
__device__ __forceinline__ LaneAct ks_read_lds(const uint8_t *area, int sbw, int s, int j) {
    const uint8_t *q = area + 256 * s + 64 * j;
    LaneAct a;
    a.a0 = *reinterpret_cast<const u32x4 *>(q);
    a.a1 = *reinterpret_cast<const u32x4 *>(q + 16);
    a.b0 = *reinterpret_cast<const u32x4 *>(q + 32);
    a.b1 = *reinterpret_cast<const u32x4 *>(q + 48);
    a.dk = *reinterpret_cast<const float4 *>(area + 256 * sbw + (8 * s + 2 * j) * 8);
    return a;
}

// SBW: 1, 2 or 4 super-blocks per wave and group; GMAX: the most groups per
// row (K <= 4096 GMAX); p.ring_off: LDS offset of the wave areas (after the
// partials); EPI, BATCH: the fused epilogue and batched launches, as in
// gemv_q4k_ksplit_kernel.
// KT (rows shorter than one group, GMAX = 1): waves per team, 0 for the
// whole KW = 16/SBW.  A team of KT < KW waves covers the super-blocks [0,
// SBW*KT), which hold the row's nb; the slices it leaves out would hold
// only super-blocks past the row, whose tile-kernel sums are exact zeros,
// so the tree over the KW slice sums takes +0 there and the bits stay the
// tile kernel's.
template <int SBW, int WAVES, int S, int GMAX, bool SUMS = false, int EPI = kEpiNone, bool BATCH = false,
          int KT = 0>
__global__ __launch_bounds__(kWave *WAVES) void gemv_q4k_ksplit_long_kernel(Q4K_GEMV_KERNEL_ARGS) {
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
    const int r = lane / (4 * SBW), s = (lane >> 2) & (SBW - 1), j = lane & 3;
    const int G = p.G;

    const int b = (int)blockIdx.x;
    const int wg_beg = b * p.rows_base + min(b, p.rows_extra);
    const int n = p.rows_base + (b < p.rows_extra ? 1 : 0);
    const int nt = (n + TR - 1) / TR;
    const int tq = nt / TEAMS, trem = nt - tq * TEAMS;
    const int tb = team * tq + min(team, trem);
    const int ntiles = tq + (team < trem ? 1 : 0);

    // 1. the slice's activation in every group, issued first; past the row: zeros
    const __amdgpu_buffer_rsrc_t rx = make_rsrc(p.x, (uint32_t)p.K * 4u);
    float xv[GMAX][V];
#pragma unroll
    for (int i = 0; i < GMAX; ++i) {
        const uint32_t off = (uint32_t)(((16 * i + SBW * slice) * kQK + lane * V) * 4);
#pragma unroll
        for (int k = 0; k < V / 4; ++k) {
            // the whole vector is cast: this clang's bit_cast of one element
            // of an ext_vector lvalue reads element 0
            const f32x4 a = __builtin_bit_cast(f32x4, load16(rx, off + 16u * k));
            xv[i][4 * k] = a[0];
            xv[i][4 * k + 1] = a[1];
            xv[i][4 * k + 2] = a[2];
            xv[i][4 * k + 3] = a[3];
        }
    }

    // 2. the first S steps' weights (GLU: and the gate weight's; BATCH: of
    //    the workgroup's weight matrix, none for an absent expert)
    if constexpr (BATCH) batch_weights(p);
    const uint32_t wbytes = BATCH && p.w_absent ? 0u : (uint32_t)(n * p.row_stride);
    __amdgpu_buffer_rsrc_t rsw[NW];
    rsw[0] = make_rsrc(p.w + (int64_t)wg_beg * p.row_stride, wbytes);
    if constexpr (NW == 2) rsw[NW - 1] = make_rsrc(p.gate + (int64_t)wg_beg * p.row_stride, wbytes);
    const uint32_t lrow = (uint32_t)r * (uint32_t)p.row_stride;
    const uint32_t lh = lrow + (uint32_t)((SBW * slice + s) * kBlockBytes);
    const uint32_t lq = lh + 16u + 32u * (uint32_t)j;
    const uint32_t tile_bytes = (uint32_t)TR * (uint32_t)p.row_stride;
    const int kb0 = SBW * slice + s;  // the lane's super-block within each group
    auto load_step = [&](Step st, RowRegs(&w)[NW]) {
        const bool ok = st.tile < ntiles && 16 * st.i + kb0 < p.nb;
        const uint32_t base = (uint32_t)(tb + st.tile) * tile_bytes + (uint32_t)st.i * (16u * kBlockBytes);
        const uint32_t oh = ok ? base + lh : kOOB;
        const uint32_t oq = ok ? base + lq : kOOB;
#pragma unroll
        for (int u = 0; u < NW; ++u) {
            w[u].h = load16(rsw[u], oh);
            w[u].q0 = load16(rsw[u], oq);
            w[u].q1 = load16(rsw[u], oq + 16u);
        }
    };
    Step st[S];
    RowRegs w[S][NW];
    st[0] = Step{0, 0};
#pragma unroll
    for (int k = 1; k < S; ++k) st[k] = next_step(st[k - 1], G);
#pragma unroll
    for (int k = 0; k < S; ++k) load_step(st[k], w[k]);

    // 3. quantise group 0 of the slice into the wave's LDS area, the other
    // groups just before the step that first reads them (the first tile
    // walks the groups in order); group 0 unconditionally (a slice past the
    // row quantises zeros and writes no sums), so its load is not sunk below
    // the weight loads
    uint8_t *area = lds + p.ring_off + wave * G * ks_slice_bytes(SBW);
    auto stage = [&](int i) {
        ks_stage_lds<SBW>(xv[i], lane, area + i * ks_slice_bytes(SBW), SUMS ? p.sq : nullptr,
                          (16 * i + SBW * slice) * 8, p.K / 32);
        // lanes read what other lanes of the wave wrote: keep the reads
        // below (a wave's LDS operations complete in order)
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    };
    // p.rpw: groups quantised before the first step (1, or all of them)
#pragma unroll
    for (int i = 0; i < GMAX; ++i)
        if (i == 0 || (i < p.rpw && i < G && 16 * i + SBW * slice < p.nb)) stage(i);
    int staged = max(1, min(p.rpw, G));  // groups staged so far

    Lane ln;
    ln.lane = lane;
    ln.g = kb0;
    ln.j = j;
    ln.sel = make_scale_sel(j);
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
                    const LaneAct a = ks_read_lds(area + st[k].i * ks_slice_bytes(SBW), SBW, s, j);
                    int sa, sb;
#pragma unroll
                    for (int u = 0; u < NW; ++u) {
                        const RowScales sc = row_scales(w[k][u], ln);
                        accumulate(w[k][u], sc, a, acc[u], sa, sb);
                    }
                    if constexpr (SUMS) {
                        const int rl = (tb + st[k].tile) * TR + r;
                        const int kb = 16 * st[k].i + kb0;
                        if (st[k].tile < ntiles && rl < n && kb < p.nb) {
                            int32_t *o = p.sums + (int64_t)(wg_beg + rl) * (p.K / 32) + kb * 8 + 2 * j;
                            o[0] = sa;
                            o[1] = sb;
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
            for (int h = KW / 2; h >= 1; h /= 2)
#pragma unroll
                for (int t = 0; t < h; ++t) q[t] = q[2 * t] + q[2 * t + 1];
            out[u] = q[0];
        }
        p.dst[wg_beg + row] = ks_epilogue<EPI>(p, wg_beg + row, out);
    }
}

// ------------------------------------------------------------------------
// Several columns of rows shorter than one group, in short teams (one
// partial group: nb <= 8 blocks for two columns, nb <= 4 for three or four).
// The several-column tile kernel sums a wave's lanes first over super-blocks
// g and g^8 (and, with three or four columns, g^4), then over the chunks,
// then over the low bits of g (column_sums).  Positions past the row hold
// exact zeros there (a lane's accumulator is never -0), so for such rows the
// g^8 and g^4 levels add +0 and the tree left is the one-column tree: the
// chunks, then pairs (2t, 2t+1) of positions.  So this kernel is the
// one-column short-team kernel with NC accumulators per lane: each wave
// stages its slice of every column once (ks_stage_lds), each step loads the
// weights once and accumulates every column, and the (row, column, slice)
// partials meet in the balanced tree over the slices.
// ------------------------------------------------------------------------

// LDS bytes of the partials (rows x NC x KT floats, padded to 16 bytes).
__host__ __device__ constexpr int ksplit_short_nc_part_bytes(int rows_per_wg, int nc, int kt) {
    return (rows_per_wg * nc * kt * 4 + 15) / 16 * 16;
}
__host__ __device__ constexpr int ksplit_short_nc_lds_bytes(int rows_per_wg, int nc, int sbw, int kt, int waves) {
    return ksplit_short_nc_part_bytes(rows_per_wg, nc, kt) + waves * nc * ks_slice_bytes(sbw);
}

// NC: columns (2..4), SBW: super-blocks per wave, WAVES: waves per
// workgroup (whole teams of KT), S: row tiles in flight per wave.  SUMS: the
// parity variant (every lane's int32 sub-block sums and the activation's
// block sums, per column).  p.ring_off: LDS offset of the wave areas.
template <int NC, int SBW, int WAVES, int S, int KT, bool SUMS = false, int P = 2>
__global__ __launch_bounds__(kWave *WAVES) void gemv_q4k_ksplit_short_nc_kernel(Q4K_GEMV_KERNEL_ARGS) {
    constexpr int KW = 16 / SBW;
    constexpr int TR = 16 / SBW;
    constexpr int TEAMS = WAVES / KT;
    constexpr int V = 4 * SBW;
    constexpr bool RC4 = P == 4;  // wave w: super-blocks w and w + 4
    static_assert(NC >= 2 && NC <= 4 && TEAMS >= 1 && WAVES % KT == 0 && KT < KW, "short teams, 2-4 columns");
    static_assert(!RC4 || (SBW == 2 && KT == 4 && NC >= 3), "residue classes mod 4: rows of 5 to 8 blocks");
    p = with_head(p, Q4K_GEMV_HEAD_VALUES);
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    float *part = reinterpret_cast<float *>(lds);

    const int lane = threadIdx.x & (kWave - 1);
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int slice = wave % KT, team = wave / KT;
    const int r = lane / (4 * SBW), s = (lane >> 2) & (SBW - 1), j = lane & 3;

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
            // the whole vector is cast (see the one-column long-row kernel)
            const f32x4 a = __builtin_bit_cast(f32x4, load16(rx, off + 16u * k));
            xv[c][4 * k] = a[0];
            xv[c][4 * k + 1] = a[1];
            xv[c][4 * k + 2] = a[2];
            xv[c][4 * k + 3] = a[3];
        }
    }

    // 2. the first S tiles' weights (rows past the workgroup's share: zeros)
    const __amdgpu_buffer_rsrc_t rsw = make_rsrc(p.w + (int64_t)wg_beg * p.row_stride, (uint32_t)(n * p.row_stride));
    const int kb0 = RC4 ? slice + 4 * s : SBW * slice + s;  // the lane's super-block
    const uint32_t lh = (uint32_t)r * (uint32_t)p.row_stride + (uint32_t)(kb0 * kBlockBytes);
    const uint32_t lq = lh + 16u + 32u * (uint32_t)j;
    const uint32_t tile_bytes = (uint32_t)TR * (uint32_t)p.row_stride;
    auto load_tile = [&](int t, RowRegs &w) {
        const bool ok = t < ntiles && kb0 < p.nb;
        const uint32_t base = (uint32_t)(tb + t) * tile_bytes;
        const uint32_t oh = ok ? base + lh : kOOB;
        const uint32_t oq = ok ? base + lq : kOOB;
        w.h = load16(rsw, oh);
        w.q0 = load16(rsw, oq);
        w.q1 = load16(rsw, oq + 16u);
    };
    int tk[S];
    RowRegs w[S];
#pragma unroll
    for (int k = 0; k < S; ++k) {
        tk[k] = k;
        load_tile(k, w[k]);
    }

    // 3. quantise every column's slice into the wave's LDS areas
    uint8_t *area = lds + p.ring_off + wave * NC * ks_slice_bytes(SBW);
#pragma unroll
    for (int c = 0; c < NC; ++c)
        ks_stage_lds<SBW>(xv[c], lane, area + c * ks_slice_bytes(SBW),
                          SUMS ? p.sq + (int64_t)c * (p.K / 32) : nullptr, (RC4 ? slice : SBW * slice) * 8,
                          p.K / 32, RC4 ? 24 : 0);
    // lanes read what other lanes of the wave wrote
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");

    Lane ln;
    ln.lane = lane;
    ln.g = kb0;
    ln.j = j;
    ln.sel = make_scale_sel(j);
    // 4. the tiles, S in flight
    int remaining = ntiles;
    if (remaining > 0) {
        for (;;) {
#pragma unroll
            for (int k = 0; k < S; ++k) {
                const RowScales sc = row_scales(w[k], ln);
                const int rl = (tb + tk[k]) * TR + r;
                float acc[NC];
#pragma unroll
                for (int c = 0; c < NC; ++c) {
                    acc[c] = 0.0f;
                    const LaneAct a = ks_read_lds(area + c * ks_slice_bytes(SBW), SBW, s, j);
                    int sa, sb;
                    accumulate(w[k], sc, a, acc[c], sa, sb);
                    if constexpr (SUMS) {
                        if (tk[k] < ntiles && rl < n && kb0 < p.nb) {
                            int32_t *o = p.sums + ((int64_t)c * p.M + wg_beg + rl) * (p.K / 32) + kb0 * 8 + 2 * j;
                            o[0] = sa;
                            o[1] = sb;
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
        for (int h = KW / 2; h >= 1; h /= 2)
#pragma unroll
            for (int t = 0; t < h; ++t) q[t] = q[2 * t] + q[2 * t + 1];
        p.dst[(int64_t)c * p.ld_dst + wg_beg + row] = q[0];
    }
}

// The instantiated several-column short-team variants: two columns at 2 or
// 4 super-blocks per wave for rows of 5 to 8 blocks (teams of 4 or 2) and
// of 3 or 4 (teams of 2 or 1), three or four columns at 4 per wave for rows
// of 3 or 4 blocks (teams of 1); 4, 8 or 16 waves; one or two tiles in
// flight.
constexpr bool ksplit_short_nc_exists(int nc, int sbw, int kt, int waves, int slots, int p = 2) {
    const bool shape = p == 4 ? (nc == 3 || nc == 4) && sbw == 2 && kt == 4
                       : nc == 2 ? ((sbw == 2 && (kt == 2 || kt == 4)) || (sbw == 4 && (kt == 1 || kt == 2)))
                                 : ((nc == 3 || nc == 4) && sbw == 4 && kt == 1);
    return shape && (waves == 4 || waves == 8 || waves == 16) && waves % kt == 0 && (slots == 1 || slots == 2);
}

// LDS bytes of a long-row K-split launch: the partials, padded to 16 bytes,
// then every wave's slice of every group (nw: 2 with a gate weight).
// (kt: waves per team, 0 for 16/sbw).
__host__ __device__ constexpr int ksplit_long_part_bytes(int rows_per_wg, int sbw, int nw = 1, int kt = 0) {
    return (rows_per_wg * (kt > 0 ? kt : 16 / sbw) * 4 * nw + 15) / 16 * 16;
}
__host__ __device__ constexpr int ksplit_long_lds_bytes(int rows_per_wg, int sbw, int waves, int G, int nw = 1,
                                                        int kt = 0) {
    return ksplit_long_part_bytes(rows_per_wg, sbw, nw, kt) + waves * G * ks_slice_bytes(sbw);
}

// Rows of 3 to 14 super-blocks (K = 768 .. 3584 values): the rows the
// short-team variants serve at 2 super-blocks per wave.
__host__ __device__ constexpr bool ksplit_short_rows(int64_t K) {
    return K % 256 == 0 && K >= 3 * 256 && K <= 14 * 256;
}

// The instantiated team sizes (waves per team) of the short-team variants
// at sbw super-blocks per wave: powers of two below 16/sbw for rows of 3 to
// 8 blocks, and 5, 6, 7 (sbw 2) or 3 (sbw 4) for rows of 9 to 14.
__host__ __device__ constexpr bool ksplit_short_kt_ok(int sbw, int kt) {
    return (sbw == 1 && (kt == 4 || kt == 8)) || (sbw == 2 && (kt == 2 || (kt >= 4 && kt <= 7))) ||
           (sbw == 4 && kt >= 1 && kt <= 3);
}

// Waves per team of the long-row kernel for rows of nb super-blocks at sbw
// per wave: for rows shorter than one group the fewest that cover the row
// where that team size is instantiated, else the next power of two; 0 (the
// whole 16/sbw) otherwise or where that is no fewer.
__host__ __device__ constexpr int ksplit_short_team(int nb, int sbw) {
    if (nb >= 16 || sbw <= 0) return 0;
    int kt = (nb + sbw - 1) / sbw;
    if (!ksplit_short_kt_ok(sbw, kt)) {
        int p = 1;
        while (p < kt) p *= 2;
        kt = p;
    }
    return kt < 16 / sbw && ksplit_short_kt_ok(sbw, kt) ? kt : 0;
}

// The instantiated K-split variants: whole teams per workgroup; two groups
// per row only up to SBW = 4 (at 16 the raw activation of two groups alone
// would take 128 registers), and no SBW = 8 (its 32 values per lane led the
// compiler to quantise them before issuing the first weight load).
constexpr bool ksplit_exists(int sbw, int waves, int slots, int G) {
    return (sbw == 1 || sbw == 2 || sbw == 4 || sbw == 16) && (waves == 4 || waves == 8 || waves == 16) &&
           waves % (16 / sbw) == 0 && !(sbw == 16 && waves == 16) &&
           (slots == 1 || slots == 2 || ((slots == 3 || slots == 4) && G == 1 && sbw <= 4)) &&
           (G == 1 || (G == 2 && sbw <= 4));
}

template <bool SUMS, int SBW, int WAVES, int S>
const void *ksplit_sym_g(int G) {
    if constexpr (ksplit_exists(SBW, WAVES, S, 1))
        if (G == 1) return reinterpret_cast<const void *>(&gemv_q4k_ksplit_kernel<SBW, WAVES, S, 1, SUMS>);
    if constexpr (ksplit_exists(SBW, WAVES, S, 2))
        if (G == 2) return reinterpret_cast<const void *>(&gemv_q4k_ksplit_kernel<SBW, WAVES, S, 2, SUMS>);
    return nullptr;
}

template <bool SUMS, int SBW, int WAVES>
const void *ksplit_sym_s(int slots, int G) {
    switch (slots) {
        case 1: return ksplit_sym_g<SUMS, SBW, WAVES, 1>(G);
        case 2: return ksplit_sym_g<SUMS, SBW, WAVES, 2>(G);
        case 3: return ksplit_sym_g<SUMS, SBW, WAVES, 3>(G);
        case 4: return ksplit_sym_g<SUMS, SBW, WAVES, 4>(G);
        default: return nullptr;
    }
}

template <bool SUMS, int SBW>
const void *ksplit_sym_w(int waves, int slots, int G) {
    if (waves == 4) return ksplit_sym_s<SUMS, SBW, 4>(slots, G);
    if (waves == 8) return ksplit_sym_s<SUMS, SBW, 8>(slots, G);
    if (waves == 16) return ksplit_sym_s<SUMS, SBW, 16>(slots, G);
    return nullptr;
}

// The long-row variants: SBW 1 or 2 in whole teams of 8 or 16 waves for rows
// of up to 4 or 8 groups, SBW 4 in teams of 4 waves (4, 8 or 16 per
// workgroup) for rows of up to 4 groups (its 16 values per lane and group
// held for 8 groups would take 128 registers); one or two steps in flight,
// or three or four in workgroups of up to 8 waves.
constexpr bool ksplit_long_exists(int sbw, int waves, int slots, int gmax) {
    return (((sbw == 1 || sbw == 2) && (waves == 8 || waves == 16) && (gmax == 4 || gmax == 8)) ||
           (sbw == 4 && (waves == 4 || waves == 8 || waves == 16) && gmax == 4)) &&
           waves % (16 / sbw) == 0 && (slots == 1 || slots == 2 || ((slots == 3 || slots == 4) && waves <= 8));
}

template <bool SUMS, int SBW, int WAVES, int S>
const void *ksplit_long_sym_g(int gmax) {
    if constexpr (ksplit_long_exists(SBW, WAVES, S, 4))
        if (gmax == 4) return reinterpret_cast<const void *>(&gemv_q4k_ksplit_long_kernel<SBW, WAVES, S, 4, SUMS>);
    if constexpr (ksplit_long_exists(SBW, WAVES, S, 8))
        if (gmax == 8) return reinterpret_cast<const void *>(&gemv_q4k_ksplit_long_kernel<SBW, WAVES, S, 8, SUMS>);
    return nullptr;
}

// The long-row K-split kernel for rows of G groups (G <= 8), or null.
template <bool SUMS>
const void *ksplit_long_kernel(int sbw, int waves, int slots, int G) {
    const int gmax = G <= 4 ? 4 : 8;
    if (G > 8) return nullptr;
    auto pick = [&](auto sbw_c) -> const void * {
        constexpr int B = decltype(sbw_c)::value;
        auto by_slots = [&](auto waves_c) -> const void * {
            constexpr int W = decltype(waves_c)::value;
            switch (slots) {
                case 1: return ksplit_long_sym_g<SUMS, B, W, 1>(gmax);
                case 2: return ksplit_long_sym_g<SUMS, B, W, 2>(gmax);
                case 3: return ksplit_long_sym_g<SUMS, B, W, 3>(gmax);
                case 4: return ksplit_long_sym_g<SUMS, B, W, 4>(gmax);
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

// The short-team variants of the long-row kernel (rows of one partial group;
// q4k_short.hip, q6k_short.hip): the team sizes of ksplit_short_kt_ok in
// workgroups of 4, 8 or 16 waves (power-of-two teams) or of one, two or
// four teams (the others, up to 16 waves); q6: the Q6_K kernel.
constexpr bool ksplit_short_exists(bool q6, int sbw, int kt, int waves, int slots, bool sums, int epi, bool batch) {
    const bool pow2 = (kt & (kt - 1)) == 0;
    const bool shape = ksplit_short_kt_ok(sbw, kt) &&
                       (pow2 ? (waves == 4 || waves == 8 || waves == 16)
                             : (waves == kt || waves == 2 * kt || waves == 4 * kt)) &&
                       waves <= 16 && waves % kt == 0 && (slots == 1 || slots == 2);
    if (!shape) return false;
    if (sums) return !batch && epi == kEpiNone;
    if (epi == kEpiNone && !batch) return true;
    // fused and batched: one step in flight (a gate weight at 16 waves
    // spills the Q6_K kernel's registers)
    return slots == 1 && !(q6 && epi == kEpiGlu && waves == 16);
}

// The fused-epilogue variants (EPI = kEpiBias or kEpiGlu), in the shapes of
// the plain kernels with 2 or 4 super-blocks per wave (short rows) or 1, 2
// or 4 (long rows) and one or two steps in flight, where their registers fit
// the launch bounds: not two steps in flight at 16 waves (the gate weight's
// registers spilled there).
constexpr bool ksplit_epi_exists(int sbw, int waves, int slots, int G) {
    return (sbw == 2 || sbw == 4) && (slots == 1 || (slots == 2 && waves <= 8)) &&
           ksplit_exists(sbw, waves, slots, G);
}
constexpr bool ksplit_long_epi_exists(int sbw, int waves, int slots, int gmax) {
    return (slots == 1 || (slots == 2 && waves <= 8)) && ksplit_long_exists(sbw, waves, slots, gmax);
}

// The batched variants (broadcasting and MUL_MAT_ID, with or without a
// fused epilogue): in the shapes the automatic rules pick -- 4 super-blocks
// per wave in 4-wave workgroups, 2 in 8-wave ones (or 16 with one step in
// flight), and for long rows also 1 in 16-wave workgroups.
constexpr bool ksplit_batch_exists(int sbw, int waves, int slots, int G) {
    return ksplit_epi_exists(sbw, waves, slots, G) &&
           ((sbw == 4 && waves == 4) || (sbw == 2 && (waves == 8 || (waves == 16 && slots == 1))));
}
constexpr bool ksplit_long_batch_exists(int sbw, int waves, int slots, int gmax) {
    return ksplit_long_epi_exists(sbw, waves, slots, gmax) &&
           ((sbw == 4 && waves == 4) || (sbw == 2 && waves == 8) || (sbw == 1 && waves == 16 && slots == 1));
}

// The fused (EPI kEpiBias, kEpiGlu) or batched (BATCH; any EPI) K-split
// kernel of a launch shape, or null.
template <int EPI, bool BATCH = false>
const void *ksplit_kernel_epi(int sbw, int waves, int slots, int G) {
    auto pick = [&](auto sbw_c) -> const void * {
        constexpr int B = decltype(sbw_c)::value;
        auto by = [&](auto waves_c, auto s_c, auto g_c) -> const void * {
            constexpr int W = decltype(waves_c)::value, SS = decltype(s_c)::value, GG = decltype(g_c)::value;
            if constexpr (BATCH ? ksplit_batch_exists(B, W, SS, GG) : ksplit_epi_exists(B, W, SS, GG))
                return reinterpret_cast<const void *>(&gemv_q4k_ksplit_kernel<B, W, SS, GG, false, EPI, BATCH>);
            return nullptr;
        };
        auto by_w = [&](auto waves_c) -> const void * {
            using I1 = std::integral_constant<int, 1>;
            using I2 = std::integral_constant<int, 2>;
            if (slots == 1) return G == 1 ? by(waves_c, I1{}, I1{}) : (G == 2 ? by(waves_c, I1{}, I2{}) : nullptr);
            if (slots == 2) return G == 1 ? by(waves_c, I2{}, I1{}) : (G == 2 ? by(waves_c, I2{}, I2{}) : nullptr);
            return nullptr;
        };
        if (waves == 4) return by_w(std::integral_constant<int, 4>{});
        if (waves == 8) return by_w(std::integral_constant<int, 8>{});
        if (waves == 16) return by_w(std::integral_constant<int, 16>{});
        return nullptr;
    };
    if (sbw == 2) return pick(std::integral_constant<int, 2>{});
    if (sbw == 4) return pick(std::integral_constant<int, 4>{});
    return nullptr;
}

template <int EPI, bool BATCH = false>
const void *ksplit_long_kernel_epi(int sbw, int waves, int slots, int G) {
    const int gmax = G <= 4 ? 4 : 8;
    if (G > 8) return nullptr;
    auto pick = [&](auto sbw_c) -> const void * {
        constexpr int B = decltype(sbw_c)::value;
        auto by = [&](auto waves_c, auto s_c, auto g_c) -> const void * {
            constexpr int W = decltype(waves_c)::value, SS = decltype(s_c)::value, GM = decltype(g_c)::value;
            if constexpr (BATCH ? ksplit_long_batch_exists(B, W, SS, GM) : ksplit_long_epi_exists(B, W, SS, GM))
                return reinterpret_cast<const void *>(&gemv_q4k_ksplit_long_kernel<B, W, SS, GM, false, EPI, BATCH>);
            return nullptr;
        };
        auto by_w = [&](auto waves_c) -> const void * {
            using I1 = std::integral_constant<int, 1>;
            using I2 = std::integral_constant<int, 2>;
            using I4 = std::integral_constant<int, 4>;
            using I8 = std::integral_constant<int, 8>;
            if (slots == 1) return gmax == 4 ? by(waves_c, I1{}, I4{}) : by(waves_c, I1{}, I8{});
            if (slots == 2) return gmax == 4 ? by(waves_c, I2{}, I4{}) : by(waves_c, I2{}, I8{});
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

// The K-split kernel of a launch shape, or null when it is not instantiated.
template <bool SUMS>
const void *ksplit_kernel(int sbw, int waves, int slots, int G) {
    switch (sbw) {
        case 1: return ksplit_sym_w<SUMS, 1>(waves, slots, G);
        case 2: return ksplit_sym_w<SUMS, 2>(waves, slots, G);
        case 4: return ksplit_sym_w<SUMS, 4>(waves, slots, G);
        case 16: return ksplit_sym_w<SUMS, 16>(waves, slots, G);
        default: return nullptr;
    }
}

}  // namespace q4k
