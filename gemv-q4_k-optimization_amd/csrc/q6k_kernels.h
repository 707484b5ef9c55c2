// q6k_kernels.h -- the gfx950 Q6_K GEMV tile kernel (template), shared by
// q6k_gemv.hip, which instantiates the product variants and launches them,
// and q4k_sums.hip, which instantiates its parity variants (SUMS).
//
// block_q6_K, 210 bytes per 256 weights: ql[128] (low 4 bits), qh[64] (high
// 2 bits), scales[16] (int8, one per 16 weights), d (fp16);
// w = d * scales[e / 16] * (q - 32) with the 6-bit q in [0, 63].  Within half
// h of the block (weights 128h.., ql[64h..], qh[32h..], scales[8h..]), for
// l in [0, 32):
//   weight 128h + l       low  nibble of ql[64h + l]       qh[32h + l] bits 0-1
//   weight 128h + 32 + l  low  nibble of ql[64h + 32 + l]  bits 2-3
//   weight 128h + 64 + l  high nibble of ql[64h + l]       bits 4-5
//   weight 128h + 96 + l  high nibble of ql[64h + 32 + l]  bits 6-7
// -- the byte and bit positions that kernels/vecdotq.cuh:867-891 computes from
// (iqs, QI6_K = 32, QR6_K = 2) and combines at :580-600.
//
// Tile kernel lane map (wave64, one group = 16 consecutive super-blocks of a
// row per step, four lanes per super-block):
//   lane = 4g + 2h + j'    g: super-block of the group, h: half, j': l in [16j', 16j' + 16)
//   loads per row:         ql[64h + 16j' ..+16), ql[64h + 32 + 16j' ..+16),
//                          qh[32h + 16j' ..+16), scales[8h ..+8), bytes 206..209 (d)
//   its 64 weights:        for m = 0..3, the 16 weights 128h + 32m + 16j' + [0, 16),
//                          which share scales[8h + 2m + j']
// so every lane's integer dot products are whole scale groups, computed as
// sum over 16 of q * q8 starting from -32 * (sum of the 16 q8), a term the
// activation staging provides.  Every weight byte is loaded once per row.
// Blocks sit at a 210-byte pitch, so every other block's loads are 2-byte
// aligned: gfx9 vector memory instructions serve them in the unaligned access
// mode of the HSA runtime's queues.
#pragma once

#include <hip/hip_runtime.h>

#include "q4k_tile.h"

namespace q4k {


constexpr int kQ6Bytes = 210;  // block_q6_K

typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

__device__ __forceinline__ u32x2 load8(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    return __builtin_amdgcn_raw_buffer_load_b64(r, off, 0, 0);
}
__device__ __forceinline__ uint32_t load4(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    return __builtin_amdgcn_raw_buffer_load_b32(r, off, 0, 0);
}

// One row's share of a group in a lane's registers.
struct Q6Regs {
    u32x4 lo0;     // ql[64h + 16j' ..+16): low nibbles -> m = 0, high -> m = 2
    u32x4 lo1;     // ql[64h + 32 + 16j' ..+16): low -> m = 1, high -> m = 3
    u32x4 hi;      // qh[32h + 16j' ..+16): bit pairs 0-1, 2-3, 4-5, 6-7 -> m = 0..3
    u32x2 sc;      // scales[8h ..+8)
    uint32_t dw;   // block bytes 206..209: scales[14], scales[15], d
};

// Per-lane constants of the lane map.
struct Q6Lane {
    int lane, g, h, jp;
    uint32_t o_lo, o_hi, o_sc, o_d;  // byte offsets of the lane's loads in a group
};

__device__ __forceinline__ Q6Lane q6_lane(int lane) {
    Q6Lane ln;
    ln.lane = lane;
    ln.g = lane >> 2;
    ln.h = (lane >> 1) & 1;
    ln.jp = lane & 1;
    const uint32_t blk = (uint32_t)ln.g * kQ6Bytes;
    ln.o_lo = blk + 64u * (uint32_t)ln.h + 16u * (uint32_t)ln.jp;
    ln.o_hi = blk + 128u + 32u * (uint32_t)ln.h + 16u * (uint32_t)ln.jp;
    ln.o_sc = blk + 192u + 8u * (uint32_t)ln.h;
    ln.o_d = blk + 206u;
    return ln;
}

// Loads the lane's share of group `i` of the row at byte offset `row` of the
// buffer; rows past the buffer (offset kOOB) and blocks past the row's end
// (ok false) read as 0 without memory traffic.
__device__ __forceinline__ void q6_load(__amdgpu_buffer_rsrc_t rs, const Q6Lane &ln, uint32_t row,
                                        bool ok, Q6Regs &w) {
    const uint32_t ob = ok ? row : kOOB;
    w.lo0 = load16(rs, ob + ln.o_lo);
    w.lo1 = load16(rs, ob + ln.o_lo + 32u);
    w.hi = load16(rs, ob + ln.o_hi);
    w.sc = load8(rs, ob + ln.o_sc);
    w.dw = load4(rs, ob + ln.o_d);
}

// The 6-bit values of scale group m, dword k (weights 128h + 32m + 16j' + 4k
// + [0, 4)), as bytes in [0, 63] -- kernels/vecdotq.cuh:587-591 without the
// -32, which the dot product's starting value carries.
__device__ __forceinline__ void q6_values(const Q6Regs &w, uint32_t (&v)[4][4]) {
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        v[0][k] = (w.lo0[k] & 0x0f0f0f0fu) | ((w.hi[k] << 4) & 0x30303030u);
        v[1][k] = (w.lo1[k] & 0x0f0f0f0fu) | ((w.hi[k] << 2) & 0x30303030u);
        v[2][k] = ((w.lo0[k] >> 4) & 0x0f0f0f0fu) | (w.hi[k] & 0x30303030u);
        v[3][k] = ((w.lo1[k] >> 4) & 0x0f0f0f0fu) | ((w.hi[k] >> 2) & 0x30303030u);
    }
}

// scales[8h + 2m + j'] sign-extended, m = 0..3.
__device__ __forceinline__ void q6_scales(const Q6Regs &w, int jp, int (&sc)[4]) {
    const uint32_t sh = 8u * (uint32_t)jp;
    sc[0] = (int)(int8_t)(w.sc[0] >> sh);
    sc[1] = (int)(int8_t)(w.sc[0] >> (sh + 16u));
    sc[2] = (int)(int8_t)(w.sc[1] >> sh);
    sc[3] = (int)(int8_t)(w.sc[1] >> (sh + 16u));
}

// The activation of one lane for a group and column (Q6K staging layout):
// the q8 of its four scale groups, d8 of the 32-value blocks 4h + m, and the
// -32 * sum(q8) starting values of the four groups.
struct Q6Act {
    u32x4 a[4];
    float4 d8;
    int4 s0;
};

// FULL: group i is stored with its chunks 1 KB apart (immediate offsets): a
// whole 16-block group, or any group of the padded layout; else the row's
// last, partial group of the dense layout (chunks 64 bytes per block apart).
template <bool FULL = true>
__device__ __forceinline__ Q6Act q6_act(const GemvParams &p, const Q6Lane &ln, int i, int c, int ncols,
                                        const int8_t *q8s, const uint8_t *aux) {
    const int kb = 16 * i + ln.g;
    const int kbc = kb < p.nb ? kb : 0;  // blocks past the row's end: weights read as 0
    const int8_t *qa = q8s + c * p.qcol + i * 4096;
    Q6Act a;
    if constexpr (FULL) {
        qa += ln.lane * 16;
#pragma unroll
        for (int m = 0; m < 4; ++m) a.a[m] = *reinterpret_cast<const u32x4 *>(qa + 1024 * m);
    } else {
        const int cs = (p.nb & 15) * 64;
        qa += kb < p.nb ? ln.lane * 16 : (ln.lane & 3) * 16;  // lanes past the row's end read block 0
#pragma unroll
        for (int m = 0; m < 4; ++m) a.a[m] = *reinterpret_cast<const u32x4 *>(qa + cs * m);
    }
    const int nblk = p.K / 32;
    a.d8 = *reinterpret_cast<const float4 *>(reinterpret_cast<const float *>(aux) + c * nblk + kbc * 8 + 4 * ln.h);
    a.s0 = *reinterpret_cast<const int4 *>(reinterpret_cast<const int *>(aux) + ncols * nblk + c * 2 * nblk +
                                           kbc * 16 + 4 * (2 * ln.h + ln.jp));
    return a;
}

// int32 sums over the lane's four scale groups: sum of (q - 32) * q8.
__device__ __forceinline__ void q6_lane_sums(const uint32_t (&v)[4][4], const Q6Act &a, int (&s)[4]) {
    s[0] = a.s0.x;
    s[1] = a.s0.y;
    s[2] = a.s0.z;
    s[3] = a.s0.w;
#pragma unroll
    for (int m = 0; m < 4; ++m)
#pragma unroll
        for (int k = 0; k < 4; ++k) s[m] = __builtin_amdgcn_sdot4((int)v[m][k], (int)a.a[m][k], s[m], false);
}

// acc += d * sum over the lane's four scale groups of d8 * (S * sc), S the
// group sums (returned in s): the float combine of every kernel with this
// lane map.  |S| <= 16*32*127 and |sc| <= 128: the 24-bit products are exact
// in f32; explicit fmas fix the rounding for every launch geometry.
__device__ __forceinline__ void q6_accumulate(const uint32_t (&v)[4][4], const int (&sc)[4], float d, const Q6Act &a,
                                              float &acc, int (&s)[4]) {
    q6_lane_sums(v, a, s);
    float f = a.d8.x * (float)__mul24(s[0], sc[0]);
    f = __builtin_fmaf(a.d8.y, (float)__mul24(s[1], sc[1]), f);
    f = __builtin_fmaf(a.d8.z, (float)__mul24(s[2], sc[2]), f);
    f = __builtin_fmaf(a.d8.w, (float)__mul24(s[3], sc[3]), f);
    acc = __builtin_fmaf(d, f, acc);
}

// A wave's rows as one buffer, as for Q4_K (and the same rows of the gate
// weight when the launch fuses one).
struct Q6Stream {
    __amdgpu_buffer_rsrc_t rs, rs_gate;
    int ntiles;
};

// Loads one step: the row's group into w[0] and, with GLU, the gate row's
// group into w[1].
template <int R>
__device__ __forceinline__ void q6_load_step(const GemvParams &p, const Q6Lane &ln, const Q6Stream &ws,
                                             Step st, Q6Regs (&w)[R]) {
    const uint32_t row = (uint32_t)st.tile * (uint32_t)p.row_stride + (uint32_t)st.i * (16 * kQ6Bytes);
    const bool ok = st.tile < ws.ntiles && 16 * st.i + ln.g < p.nb;
    q6_load(ws.rs, ln, row, ok, w[0]);
    if (R == 2) q6_load(ws.rs_gate, ln, row, ok, w[R - 1]);
}

// Parity variants (SUMS): the lane's four int32 group sums of wave row `tr`,
// block kb, column c, stored where the oracle keeps them
// (sums[(c*M + row)*(K/16) + 16kb + 8h + j' + 2m]); steps past the wave's
// rows or the row's blocks store nothing.
template <bool SUMS>
__device__ __forceinline__ void q6_record_sums(const GemvParams &p, const Q6Lane &ln, const ResultRing &rr, int tr,
                                               int kb, int c, const int (&s)[4]) {
    if constexpr (SUMS) {
        const int row = rr.beg + tr;
        if (row < rr.end && kb < p.nb) {
            int32_t *o = p.sums + ((int64_t)c * p.M + row) * (p.K / 16) + kb * 16 + 8 * ln.h + ln.jp;
#pragma unroll
            for (int m = 0; m < 4; ++m) o[2 * m] = s[m];
        }
    }
}

// Consumes one group held in w (one row, or the row and its gate row); at
// the tile's last group moves the R x NC sums to the result ring.
// FULL: group st.i has its chunks 1 KB apart (see q6_act).
template <int NC, int R, bool SUMS, bool FULL>
__device__ __forceinline__ void q6_process_group_as(const GemvParams &p, const Q6Lane &ln, Step st,
                                                    const int8_t *q8s, const uint8_t *aux, const Q6Regs (&w)[R],
                                                    float (&acc)[R][NC], const ResultRing &rr) {
    uint32_t v[R][4][4];
    int sc[R][4];
    float d[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
        q6_values(w[r], v[r]);
        q6_scales(w[r], ln.jp, sc[r]);
        d[r] = half_bits_to_float(w[r].dw >> 16);
    }
#pragma unroll
    for (int c = 0; c < NC; ++c) {
        const Q6Act a = q6_act<FULL>(p, ln, st.i, c, NC, q8s, aux);
#pragma unroll
        for (int r = 0; r < R; ++r) {
            int s[4];
            q6_accumulate(v[r], sc[r], d[r], a, acc[r][c], s);
            if (R == 1) q6_record_sums<SUMS>(p, ln, rr, st.tile, 16 * st.i + ln.g, c, s);
        }
    }
}

// DENSE: the activation is staged in the dense layout (the branch on the
// group kind is taken once per group, wave-uniformly).
template <int NC, int R, int EPI, bool SUMS = false, bool DENSE = false>
__device__ __forceinline__ void q6_process_group(const GemvParams &p, const Q6Lane &ln, Step st,
                                                 const int8_t *q8s, const uint8_t *aux, const Q6Regs (&w)[R],
                                                 float (&acc)[R][NC], ResultRing &rr) {
    if (!DENSE || __builtin_amdgcn_readfirstlane(16 * (st.i + 1) <= p.nb))
        q6_process_group_as<NC, R, SUMS, true>(p, ln, st, q8s, aux, w, acc, rr);
    else
        q6_process_group_as<NC, R, SUMS, false>(p, ln, st, q8s, aux, w, acc, rr);
    if (st.i == p.G - 1) tile_to_ring<NC, R, EPI>(p, ln.lane, acc, rr);
}

// Rows that are one group long: q6_process_group with the lane's activation
// slices (the same in every step) held in registers.
template <int NC, int EPI, bool SUMS = false>
__device__ __forceinline__ void q6_process_reg(const GemvParams &p, const Q6Lane &ln, Step st, const Q6Act (&a)[NC],
                                               const Q6Regs (&w)[1], float (&acc)[1][NC], ResultRing &rr) {
    uint32_t v[4][4];
    int sc[4];
    q6_values(w[0], v);
    q6_scales(w[0], ln.jp, sc);
    const float d = half_bits_to_float(w[0].dw >> 16);
#pragma unroll
    for (int c = 0; c < NC; ++c) {
        int s[4];
        q6_accumulate(v, sc, d, a[c], acc[0][c], s);
        q6_record_sums<SUMS>(p, ln, rr, st.tile, ln.g, c, s);
    }
    tile_to_ring<NC, 1, EPI>(p, ln.lane, acc, rr);
}

// Tile kernel: any K, 1..8 columns; one row per tile.  The structure of the
// Q4_K tile kernel: one workgroup per CU, activation loads first, then the
// barrier, the early weight slots (PRO 0: min(S, 2) slots before the
// activation is quantised, 1: none), quantisation into LDS, the barrier, and
// the S-slot stream with unconditional loads and the result ring.  GLU (one
// column): each tile also streams the same row of the gate weight, and the
// ring flush applies the biases and the GLU.
// BATCH: channels and samples over grid y and z, as in the Q4_K kernel.
// EPI: the epilogue (kEpiNone, kEpiBias, kEpiGlu; the fused ones are one
// column).
// SUMS: the parity variant of a plain launch, which also stores every lane's
// int32 group sums (p.sums).
// DENSE: the activation columns take K bytes each in LDS (kLayoutQ6KDense)
// instead of whole 16-block groups.
template <int NC, int WAVES, int PRO, int S, int EPI = kEpiNone, bool BATCH = false, bool SUMS = false,
          bool DENSE = false>
__global__ __launch_bounds__(kWave *WAVES) void gemv_q6k_kernel(Q4K_GEMV_KERNEL_ARGS) {
    constexpr bool GLU = EPI == kEpiGlu;
    static_assert(!SUMS || (EPI == kEpiNone && !BATCH), "parity variants of the plain product only");
    static_assert(!DENSE || EPI == kEpiNone, "the dense layout is for several columns");
    constexpr int kLayout = DENSE ? kLayoutQ6KDense : kLayoutQ6K;
    static_assert(EPI == kEpiNone || NC == 1, "the fused epilogue is one-column");
    constexpr int R = GLU ? 2 : 1;
    p = with_head(p, Q4K_GEMV_HEAD_VALUES);
    if constexpr (BATCH) batch_activation(p);
    constexpr int kEarly = early_slots(PRO, S);
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    int8_t *q8s = reinterpret_cast<int8_t *>(lds);
    uint8_t *aux = lds + NC * p.qcol;

    const Q6Lane ln = q6_lane(threadIdx.x & (kWave - 1));
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const WaveRows wr = wave_rows<WAVES>(p, wave);
    constexpr int kLPB = stage_lpb(NC);
    constexpr int kPreR = pre_rounds(NC, kWave * WAVES);
    ActStage<kLPB, kPreR> xs;
    Q81Stage<kPreR> ys;
    if constexpr (BATCH) {
        if (p.x) stage_f32_issue<kLPB, kWave * WAVES>(p.x, p.ldx, p.K, NC, p.vec_ok != 0, p.nblk32, xs);
        else stage_q81_issue<kWave * WAVES>(p.y, p.stride_col_y, p.K, NC, p.nblk32, ys);
        batch_weights(p);
    }
    Q6Stream ws;
    const uint32_t wave_bytes = BATCH && p.w_absent ? 0u : (uint32_t)((wr.end - wr.beg) * p.row_stride);
    ws.rs = make_rsrc(p.w + (int64_t)wr.beg * p.row_stride, wave_bytes);
    ws.rs_gate = GLU ? make_rsrc(p.gate + (int64_t)wr.beg * p.row_stride, wave_bytes) : ws.rs;
    ws.ntiles = wr.end - wr.beg;
    int remaining = ws.ntiles * p.G;

    if constexpr (!BATCH) {
        if (p.x) stage_f32_issue<kLPB, kWave * WAVES>(p.x, p.ldx, p.K, NC, p.vec_ok != 0, p.nblk32, xs);
        else stage_q81_issue<kWave * WAVES>(p.y, p.stride_col_y, p.K, NC, p.nblk32, ys);
    }
    __syncthreads();  // all activation loads of this CU are queued first

    Step st[S];
    Q6Regs w[S][R];
    st[0] = Step{0, 0};
#pragma unroll
    for (int k = 1; k < S; ++k) st[k] = next_step(st[k - 1], p.G);
#pragma unroll
    for (int k = 0; k < kEarly; ++k) q6_load_step<R>(p, ln, ws, st[k], w[k]);
    if (p.x)
        stage_f32_finish<kLayout, kLPB, kWave * WAVES, NC < 4 ? 1 : kFinishRounds>(
            p.x, p.ldx, p.K, NC, p.vec_ok != 0, p.nblk32, xs, p.qcol, q8s, aux);
    else
        stage_q81_finish<kLayout, kWave * WAVES, NC < 4 ? 1 : kFinishRounds>(
            p.y, p.stride_col_y, p.K, NC, p.nblk32, ys, p.qcol, q8s, aux);
    __syncthreads();
    if (remaining == 0) return;  // no barrier below this point
#pragma unroll
    for (int k = kEarly; k < S; ++k) q6_load_step<R>(p, ln, ws, st[k], w[k]);

    float acc[R][NC];
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
        for (int c = 0; c < NC; ++c) acc[r][c] = 0.0f;
    const int cap = ring_cap(p.ring_off, NC, WAVES);
    ResultRing rr{reinterpret_cast<float *>(lds + p.ring_off) + wave * cap, wr.beg, wr.end, 0, 0, cap};

    // (one column at 16 waves, eight at 8 waves: wider variants would spill
    // registers)
    if constexpr ((NC == 1 || WAVES == 8) && R == 1 && S <= 2 && !DENSE) {
        if (p.G == 1) {  // every step reads the same activation slice: keep it in registers
            Q6Act a0[NC];
#pragma unroll
            for (int c = 0; c < NC; ++c) a0[c] = q6_act(p, ln, 0, c, NC, q8s, aux);
            for (;;) {
#pragma unroll
                for (int k = 0; k < S; ++k) {
                    q6_process_reg<NC, EPI, SUMS>(p, ln, st[k], a0, w[k], acc, rr);
                    st[k] = next_step(st[(k + S - 1) % S], p.G);
                    q6_load_step<R>(p, ln, ws, st[k], w[k]);
                }
                remaining -= S;
                if (remaining <= 0) break;
            }
            ring_flush<NC, EPI>(p, ln.lane, rr);
            return;
        }
    }
    for (;;) {
#pragma unroll
        for (int k = 0; k < S; ++k) {
            q6_process_group<NC, R, EPI, SUMS, DENSE>(p, ln, st[k], q8s, aux, w[k], acc, rr);
            st[k] = next_step(st[(k + S - 1) % S], p.G);
            q6_load_step<R>(p, ln, ws, st[k], w[k]);
        }
        remaining -= S;
        if (remaining <= 0) break;
    }
    ring_flush<NC, EPI>(p, ln.lane, rr);
}

}  // namespace q4k
