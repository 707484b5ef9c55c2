// q4k_gemv_kernels.h -- the gfx950 Q4_K GEMV kernels (templates), shared by
// q4k_gemv.hip, which instantiates the product variants and launches them,
// and q4k_sums.hip, which instantiates their parity variants (SUMS: each
// lane also stores the int32 sums its dot products form).
//
//   gemv_q4k_kernel        Q4_K x Q8 product.  Each workgroup first stages the
//                          activation as int8 + f32 scales in LDS, quantising
//                          it from F32 itself (one launch per op) or copying an
//                          already-quantised AoS Q8_1 buffer.  Each wave then
//                          owns tiles of R rows and streams them group by group
//                          (16 super-blocks x 144 B per row per step, four
//                          lanes per super-block) with 16-byte buffer loads,
//                          the next step's loads issued before the current
//                          step's arithmetic.
//   gemv_q4k_bpl_kernel    block-per-lane kernel (one column, 16..64 blocks per row)
//   gemv_q4k_blk_kernel    the same arithmetic with coalesced loads through LDS
#pragma once

#include <hip/hip_runtime.h>

#include "q4k_tile.h"

namespace q4k {

// One row's share of a group in a lane's registers: the block header and the
// lane's 32 qs bytes.
struct RowRegs {
    u32x4 h, q0, q1;
};

// Loads group i (16 super-blocks) of rows [row0, row0 + nrows), nrows <= R;
// the rows past nrows (all rows when nrows <= 0) and blocks past the row's
// end read as 0 and cost no memory traffic.
template <int R>
__device__ __forceinline__ void load_group(const GemvParams &p, int row0, int nrows, int i, int g,
                                           int j, RowRegs (&w)[R]) {
    const uint8_t *base = p.w + (int64_t)row0 * p.row_stride;
    const __amdgpu_buffer_rsrc_t rs = make_rsrc(base, nrows > 0 ? (uint32_t)(nrows * p.row_stride) : 0u);
    const int kb = 16 * i + g;
    const uint32_t off = kb < p.nb ? (uint32_t)kb * kBlockBytes : kOOB;
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const uint32_t ro = off + (uint32_t)(r * p.row_stride);
        w[r].h = load16(rs, ro);
        w[r].q0 = load16(rs, ro + 16u + 32u * (uint32_t)j);
        w[r].q1 = load16(rs, ro + 32u + 32u * (uint32_t)j);
    }
}

// Per-lane constants of the lane map (lane = 4g + j).
struct Lane {
    int lane, g, j;
    ScaleSel sel;
};

// A wave's rows as one buffer (the host keeps them under 2^31 bytes): a load
// past them or past a row's last block reads 0 without memory traffic.
struct WaveStream {
    __amdgpu_buffer_rsrc_t rs;
    int ntiles;
    uint32_t lh, lq;  // the lane's byte offsets of its header and qs loads in a group
};

__device__ __forceinline__ WaveStream wave_stream(const GemvParams &p, const Lane &ln,
                                                  const WaveRows &wr, int R, bool absent = false) {
    WaveStream ws;
    ws.rs = make_rsrc(p.w + (int64_t)wr.beg * p.row_stride,
                      absent ? 0u : (uint32_t)((wr.end - wr.beg) * p.row_stride));
    ws.ntiles = (wr.end - wr.beg + R - 1) / R;
    ws.lh = (uint32_t)ln.g * kBlockBytes;
    ws.lq = ws.lh + 16u + 32u * (uint32_t)ln.j;
    return ws;
}

// Loads one step: R rows of the tile, or with GLU (R = 2) one row of the
// weight (w[0]) and the same row of the gate weight (w[1], buffer rs_gate).
template <int R, bool GLU>
__device__ __forceinline__ void load_step(const GemvParams &p, const Lane &ln, const WaveStream &ws,
                                          __amdgpu_buffer_rsrc_t rs_gate, Step st, RowRegs (&w)[R]) {
    constexpr int kRowsPerTile = GLU ? 1 : R;
    const uint32_t base =
        (uint32_t)(st.tile * kRowsPerTile) * (uint32_t)p.row_stride + (uint32_t)st.i * (16 * kBlockBytes);
    const bool ok = st.tile < ws.ntiles && 16 * st.i + ln.g < p.nb;
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const uint32_t ro = GLU ? base : base + (uint32_t)(r * p.row_stride);
        const __amdgpu_buffer_rsrc_t rs = GLU && r == 1 ? rs_gate : ws.rs;
        const uint32_t oh = ok ? ro + ws.lh : kOOB;
        const uint32_t oq = ok ? ro + ws.lq : kOOB;
        w[r].h = load16(rs, oh);
        w[r].q0 = load16(rs, oq);
        w[r].q1 = load16(rs, oq + 16u);
    }
}

// The activation a lane needs for one group and column: the q8 of sub-blocks
// 2j (a0, a1) and 2j+1 (b0, b1) of its super-block, and their (d8, d8*sum q8).
struct LaneAct {
    u32x4 a0, a1, b0, b1;
    float4 dk;  // d8a, kma, d8b, kmb
};

__device__ __forceinline__ LaneAct lane_act(const GemvParams &p, const Lane &ln, int i, int c,
                                            const int8_t *q8s, const float2 *dks) {
    const int kb = 16 * i + ln.g;
    const int kbc = kb < p.nb ? kb : 0;  // blocks past the row's end: weights read as 0
    const int8_t *qa = q8s + c * p.qcol + i * 4096 + ln.lane * 16;
    LaneAct a;
    a.a0 = *reinterpret_cast<const u32x4 *>(qa);
    a.a1 = *reinterpret_cast<const u32x4 *>(qa + 1024);
    a.b0 = *reinterpret_cast<const u32x4 *>(qa + 2048);
    a.b1 = *reinterpret_cast<const u32x4 *>(qa + 3072);
    a.dk = *reinterpret_cast<const float4 *>(dks + c * (p.K / 32) + kbc * 8 + ln.j * 2);
    return a;
}

// The lane's scale and min fields of one row's block (sub-blocks 2j, 2j+1)
// and the block's d and dmin.
struct RowScales {
    int sca, scb;
    float maf, mbf, d, dmin;
};

__device__ __forceinline__ RowScales row_scales(const RowRegs &w, const Lane &ln) {
    const uint32_t scm = unpack_scale_min(w.h, ln.sel);
    return RowScales{(int)(scm & 0xffu), (int)((scm >> 8) & 0xffu), (float)((scm >> 16) & 0xffu),
                     (float)(scm >> 24), half_bits_to_float(w.h[0]), half_bits_to_float(w.h[0] >> 16)};
}

// acc += the lane's share of one row's block times one activation column;
// sa, sb: its two int32 sub-block sums.
__device__ __forceinline__ void accumulate(const RowRegs &w, const RowScales &s, const LaneAct &a, float &acc,
                                           int &sa, int &sb) {
    lane_qdot(w.q0, w.q1, a.a0, a.a1, a.b0, a.b1, sa, sb);
    // |sa|, |sb| <= 32*15*127 and sc <= 63: 24-bit products are exact.
    // Explicit fmas: every kernel variant rounds identically, so the result
    // does not depend on the launch geometry.
    const float xs = __builtin_fmaf(a.dk.x, (float)__mul24(sa, s.sca), a.dk.z * (float)__mul24(sb, s.scb));
    const float ms = __builtin_fmaf(a.dk.y, s.maf, a.dk.w * s.mbf);
    acc = fmaf(s.d, xs, acc);
    acc = fmaf(-s.dmin, ms, acc);
}

// Parity variants (SUMS): the lane's two int32 sub-block sums of row tile
// row `tr` of the wave, block kb, column c, stored where the oracle keeps
// them (sums[(c*M + row)*(K/32) + 8kb + 2j + {0, 1}]); steps past the
// wave's rows or the row's blocks store nothing.
template <bool SUMS>
__device__ __forceinline__ void record_sums(const GemvParams &p, const Lane &ln, const ResultRing &rr, int tr,
                                            int kb, int c, int sa, int sb) {
    if constexpr (SUMS) {
        const int row = rr.beg + tr;
        if (row < rr.end && kb < p.nb) {
            int32_t *o = p.sums + ((int64_t)c * p.M + row) * (p.K / 32) + kb * 8 + ln.j * 2;
            o[0] = sa;
            o[1] = sb;
        }
    }
}

// Consumes one group (16 super-blocks of R rows) held in w; on the last group
// of a tile reduces the R x NC sums over the wave into the result ring.
template <int NC, int R, int EPI, bool SUMS = false>
__device__ __forceinline__ void process_group(const GemvParams &p, const Lane &ln, Step st,
                                              const int8_t *q8s, const float2 *dks,
                                              const RowRegs (&w)[R], float (&acc)[R][NC],
                                              ResultRing &rr) {
    RowScales sc[R];
#pragma unroll
    for (int r = 0; r < R; ++r) sc[r] = row_scales(w[r], ln);
#pragma unroll
    for (int c = 0; c < NC; ++c) {
        const LaneAct a = lane_act(p, ln, st.i, c, q8s, dks);
#pragma unroll
        for (int r = 0; r < R; ++r) {
            int sa, sb;
            accumulate(w[r], sc[r], a, acc[r][c], sa, sb);
            record_sums<SUMS>(p, ln, rr, st.tile * R + r, 16 * st.i + ln.g, c, sa, sb);
        }
    }
    if (st.i == p.G - 1) tile_to_ring<NC, R, EPI>(p, ln.lane, acc, rr);
}

// The same for rows that are one group long, with the
// lane's activation slices (the same in every step) held in registers.
template <int NC, int R, int EPI, bool SUMS = false>
__device__ __forceinline__ void process_row_tile(const GemvParams &p, const Lane &ln, Step st,
                                                 const LaneAct (&a)[NC], const RowRegs (&w)[R],
                                                 float (&acc)[R][NC], ResultRing &rr) {
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const RowScales sc = row_scales(w[r], ln);
#pragma unroll
        for (int c = 0; c < NC; ++c) {
            int sa, sb;
            accumulate(w[r], sc, a[c], acc[r][c], sa, sb);
            record_sums<SUMS>(p, ln, rr, st.tile * R + r, ln.g, c, sa, sb);
        }
    }
    tile_to_ring<NC, R, EPI>(p, ln.lane, acc, rr);
}

// Tile kernel: any K, 1..8 columns.  One workgroup per CU (the launch asks
// for enough LDS to keep a second one off the CU); each wave owns a
// contiguous range of rows and walks it R rows x one group at a time, with S
// groups in flight in S register slots.  Every wave issues its activation
// loads and the workgroup passes a barrier before any weight load is
// issued: a CU serves vector memory requests in order, so an activation load
// queued behind the weight stream would stall the whole workgroup's
// prologue.  PRO selects when the weight loads start: 0 -- the first two
// slots before the activation is quantised (it needs at most PRE staging
// rounds, so no activation load is issued after them) and the rest after,
// 1 -- all after, 2 -- all before, 3 -- one slot before.  Weight requests issued early overlap the quantisation
// but queue in the memory system ahead of other CUs' activation loads, so
// only part of the pipeline goes out early.
//
// Every weight load is issued unconditionally (steps past the wave's last
// one read zeros from outside the buffer) and results go to LDS, not
// memory, inside the loop: with no branch around a vector memory
// instruction, the compiler waits for exactly the group being consumed
// while the others stay in flight.
//
// GLU (one column, R = 2): each tile is one row of the weight and the same
// row of the gate weight (kernels/mmvq.cu:254-262 computes both products
// from the same activation); the ring holds the pair and its flush applies
// the biases and the GLU.
//
// BATCH: one launch over dst channels (grid y) and samples (grid z); each
// workgroup first selects its activation channel and dst slice, and, after
// its activation loads are issued, its weight matrix (batch_weights).
//
// EPI: the epilogue (kEpiNone, kEpiBias, kEpiGlu; the fused ones are one
// column).
//
// SUMS: the parity variant of a plain launch -- the same kernel that also
// stores every lane's int32 sub-block sums (p.sums) and the staging's int32
// activation sums (p.sq).
template <int NC, int R, int WAVES, int PRO, int S, int EPI = kEpiNone, bool BATCH = false, bool SUMS = false>
__global__ __launch_bounds__(kWave *WAVES) void gemv_q4k_kernel(Q4K_GEMV_KERNEL_ARGS) {
    constexpr bool GLU = EPI == kEpiGlu;
    static_assert(!SUMS || (EPI == kEpiNone && !BATCH), "parity variants of the plain product only");
    int32_t *const sq_out = SUMS ? p.sq : nullptr;
    static_assert(!GLU || (NC == 1 && R == 2), "the fused epilogue pairs one row of each weight");
    static_assert(EPI != kEpiBias || (NC == 1 && R == 1), "the bias epilogue is one column, one row per tile");
    p = with_head(p, Q4K_GEMV_HEAD_VALUES);
    if constexpr (BATCH) batch_activation(p);
    // slots loaded before quantisation
    constexpr int kEarly = early_slots(PRO, S);
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    int8_t *q8s = reinterpret_cast<int8_t *>(lds);
    float2 *dks = reinterpret_cast<float2 *>(lds + NC * p.qcol);

    Lane ln;
    ln.lane = threadIdx.x & (kWave - 1);
    ln.g = ln.lane >> 2;
    ln.j = ln.lane & 3;
    ln.sel = make_scale_sel(ln.j);

    // the wave index is wave-uniform; readfirstlane lets the compiler keep
    // row numbers and buffer descriptors in scalar registers
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const WaveRows wr = wave_rows<WAVES>(p, wave);
    constexpr int kLPB = stage_lpb(NC);  // activation lanes per 32-value block
    constexpr int kPreR = pre_rounds(NC, kWave * WAVES);
    ActStage<kLPB, kPreR> xs;
    Q81Stage<kPreR> ys;
    if constexpr (BATCH) {
        if (p.x) stage_f32_issue<kLPB, kWave * WAVES>(p.x, p.ldx, p.K, NC, p.vec_ok != 0, p.nblk32, xs);
        else stage_q81_issue<kWave * WAVES>(p.y, p.stride_col_y, p.K, NC, p.nblk32, ys);
        batch_weights(p);
    }
    const bool absent = BATCH && p.w_absent;
    const WaveStream ws = wave_stream(p, ln, wr, GLU ? 1 : R, absent);
    const __amdgpu_buffer_rsrc_t rs_gate =
        GLU ? make_rsrc(p.gate + (int64_t)wr.beg * p.row_stride,
                        absent ? 0u : (uint32_t)((wr.end - wr.beg) * p.row_stride))
            : ws.rs;
    int remaining = ws.ntiles * p.G;  // steps of this wave

    if constexpr (!BATCH) {
        if (p.x) stage_f32_issue<kLPB, kWave * WAVES>(p.x, p.ldx, p.K, NC, p.vec_ok != 0, p.nblk32, xs);
        else stage_q81_issue<kWave * WAVES>(p.y, p.stride_col_y, p.K, NC, p.nblk32, ys);
    }
    __syncthreads();  // all activation loads of this CU are queued first

    Step st[S];
    RowRegs w[S][R];
    st[0] = Step{0, 0};
#pragma unroll
    for (int k = 1; k < S; ++k) st[k] = next_step(st[k - 1], p.G);
#pragma unroll
    for (int k = 0; k < kEarly; ++k) load_step<R, GLU>(p, ln, ws, rs_gate, st[k], w[k]);
    float acc[R][NC];
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
        for (int c = 0; c < NC; ++c) acc[r][c] = 0.0f;
    const int cap = ring_cap(p.ring_off, NC, WAVES);
    ResultRing rr{reinterpret_cast<float *>(lds + p.ring_off) + wave * cap, wr.beg, wr.end, 0, 0, cap};

    // Rows of two groups (4096 < K <= 8192), one column and row, both slots
    // loaded early (the gate-weight variant would spill registers): each
    // quantisation round is one group, so a wave consumes its first early
    // step as soon as group 0 is staged and issues its next load then,
    // instead of after the whole activation.  Steps past the wave's rows
    // read zeros and their results are dropped, as in the loop.  Measured
    // on MI355X: 14336 x 8192 14.2 -> 13.6 us, 8192 x 8192 9.37 -> 9.14 us;
    // with longer rows (four groups) the waves wait between rounds for
    // early weights still in flight and 4096 x 14336 went 9.07 -> 9.41 us.
    constexpr bool kStream = NC == 1 && R == 1 && PRO == 0 && S == 2 && kEarly == 2 && WAVES == 16;
    if (kStream && p.x && p.G == 2) {
        stage_f32_rounds<kLayoutQ4K, kLPB, kWave * WAVES, 0, 1>(p.K, NC, p.nblk32, xs, p.qcol, q8s, dks, sq_out);
        __syncthreads();
        process_group<NC, R, EPI, SUMS>(p, ln, st[0], q8s, dks, w[0], acc, rr);
        st[0] = next_step(st[S - 1], p.G);
        load_step<R, GLU>(p, ln, ws, rs_gate, st[0], w[0]);
        stage_f32_rounds<kLayoutQ4K, kLPB, kWave * WAVES, 1, 2>(p.K, NC, p.nblk32, xs, p.qcol, q8s, dks, sq_out);
        __syncthreads();
        process_group<NC, R, EPI, SUMS>(p, ln, st[1], q8s, dks, w[1], acc, rr);
        st[1] = next_step(st[0], p.G);
        load_step<R, GLU>(p, ln, ws, rs_gate, st[1], w[1]);
        remaining -= 2;
        if (remaining <= 0) {  // no barrier below this point
            ring_flush<NC, EPI>(p, ln.lane, rr);
            return;
        }
    } else {
        if (p.x)
            stage_f32_finish<kLayoutQ4K, kLPB, kWave * WAVES, NC < 4 ? 1 : kFinishRounds>(
                p.x, p.ldx, p.K, NC, p.vec_ok != 0, p.nblk32, xs, p.qcol, q8s, dks, sq_out);
        else
            stage_q81_finish<kLayoutQ4K, kWave * WAVES, NC < 4 ? 1 : kFinishRounds>(
                p.y, p.stride_col_y, p.K, NC, p.nblk32, ys, p.qcol, q8s, dks, sq_out);
        __syncthreads();
        if (remaining == 0) return;  // no barrier below this point
#pragma unroll
        for (int k = kEarly; k < S; ++k) load_step<R, GLU>(p, ln, ws, rs_gate, st[k], w[k]);
    }

    // Slot k is consumed, then reloaded with the step after the newest one in
    // flight.  Steps go S at a time with one exit test; a count that is not a
    // multiple of S ends with steps past the wave's rows, whose zeros add
    // nothing and whose results the final flush drops.
    // (up to two columns at 16 waves, eight at 8 waves: wider variants would
    // spill registers)
    if constexpr ((NC <= 2 || WAVES == 8) && R == 1 && S <= 2) {
        if (p.G == 1) {  // every step reads the same activation slice: keep it in registers
            LaneAct a0[NC];
#pragma unroll
            for (int c = 0; c < NC; ++c) a0[c] = lane_act(p, ln, 0, c, q8s, dks);
            for (;;) {
#pragma unroll
                for (int k = 0; k < S; ++k) {
                    process_row_tile<NC, R, EPI, SUMS>(p, ln, st[k], a0, w[k], acc, rr);
                    st[k] = next_step(st[(k + S - 1) % S], p.G);
                    load_step<R, GLU>(p, ln, ws, rs_gate, st[k], w[k]);
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
            process_group<NC, R, EPI, SUMS>(p, ln, st[k], q8s, dks, w[k], acc, rr);
            st[k] = next_step(st[(k + S - 1) % S], p.G);
            load_step<R, GLU>(p, ln, ws, rs_gate, st[k], w[k]);
        }
        remaining -= S;
        if (remaining <= 0) break;
    }
    ring_flush<NC, EPI>(p, ln.lane, rr);
}

// ------------------------------------------------------------------------
// Block-per-lane kernel (one activation column, nb <= 64 super-blocks per row)
//
// Lane l owns super-block kb = l % nb of row l / nb in each "pass" of rpw
// rows (rpw = 64/nb for nb = 16 or 32, else 1 with lanes >= nb idle).  Its
// 144 weight bytes arrive as nine 16-byte loads and the matching 256-value
// activation slice stays in registers for the whole kernel, so the per-block
// work -- scale/min unpack, eight sub-block scalings, the min term -- is paid
// once per 144 bytes instead of once per 16.
// ------------------------------------------------------------------------

__device__ __forceinline__ void load_pass(const GemvParams &p, int pass, int rr, int kb, bool lane_on,
                                          u32x4 (&w)[9]) {
    const int row0 = pass * p.rpw;
    const int nrows = min(p.rpw, p.M - row0);
    const uint8_t *base = p.w + (int64_t)row0 * p.row_stride;
    const __amdgpu_buffer_rsrc_t rs = make_rsrc(base, (uint32_t)(nrows * p.row_stride));
    const uint32_t off = lane_on ? (uint32_t)(rr * p.row_stride) + (uint32_t)kb * kBlockBytes : kOOB;
#pragma unroll
    for (int t = 0; t < 9; ++t) w[t] = load16(rs, off + 16u * t);
}

// Sum over the nb lanes of each row segment (nb = 16, 32 or the whole wave);
// the result is valid in the segment's first lane.
__device__ __forceinline__ float segment_sum(float v, int nb) {
    v += dppf<kDppXor1>(v);
    v += dppf<kDppXor2>(v);
    v += dppf<kDppRor4>(v);
    v += dppf<kDppRor8>(v);
    if (nb == 16) return v;
    v += swizzle_xor<16>(v);
    if (nb == 32) return v;
    const float hi = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 32));
    return v + hi;
}

struct BlockAct {
    u32x4 q[16];   // 256 int8 activation values of the lane's super-block
    float d8[8];   // per sub-block scale
    float km[8];   // d8 * sum of the sub-block's q8 (the min term's factor)
};

// sums: the lane's eight int32 sub-block sums (S_qq of sub-blocks 0..7).
__device__ __forceinline__ float block_dot(const u32x4 (&w)[9], const BlockAct &a, int (&sums)[8]) {
    const u32x4 h = w[0];
    const uint32_t sc03 = h[1] & 0x3f3f3f3fu;
    const uint32_t m03 = h[2] & 0x3f3f3f3fu;
    const uint32_t sc47 = (h[3] & 0x0f0f0f0fu) | ((h[1] >> 2) & 0x30303030u);
    const uint32_t m47 = ((h[3] >> 4) & 0x0f0f0f0fu) | ((h[2] >> 2) & 0x30303030u);
    float xs = 0.0f, ys = 0.0f;
#pragma unroll
    for (int c = 0; c < 4; ++c) {  // 32-byte chunk c: sub-blocks 2c (low) and 2c+1 (high)
        int slo = 0, shi = 0;
#pragma unroll
        for (int hh = 0; hh < 2; ++hh) {
            const u32x4 wv = w[1 + 2 * c + hh];
            const u32x4 alo = a.q[4 * c + hh];
            const u32x4 ahi = a.q[4 * c + 2 + hh];
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                slo = __builtin_amdgcn_sdot4((int)(wv[k] & 0x0f0f0f0fu), (int)alo[k], slo, false);
                shi = __builtin_amdgcn_sdot4((int)((wv[k] >> 4) & 0x0f0f0f0fu), (int)ahi[k], shi, false);
            }
        }
        const int s0 = 2 * c, s1 = 2 * c + 1;
        sums[s0] = slo;
        sums[s1] = shi;
        const uint32_t scw = s0 < 4 ? sc03 : sc47;
        const uint32_t mw = s0 < 4 ? m03 : m47;
        const int sh0 = 8 * (s0 & 3), sh1 = 8 * (s1 & 3);
        const int sc0 = (int)((scw >> sh0) & 0xffu), sc1 = (int)((scw >> sh1) & 0xffu);
        xs = fmaf(a.d8[s0], (float)__mul24(slo, sc0), xs);
        xs = fmaf(a.d8[s1], (float)__mul24(shi, sc1), xs);
        ys = fmaf(a.km[s0], (float)((mw >> sh0) & 0xffu), ys);
        ys = fmaf(a.km[s1], (float)((mw >> sh1) & 0xffu), ys);
    }
    const float d = half_bits_to_float(h[0]);
    const float dmin = half_bits_to_float(h[0] >> 16);
    return fmaf(d, xs, -dmin * ys);
}

template <bool SUMS = false>
__device__ __forceinline__ void finish_pass(const GemvParams &p, int pass, int rr, int kb, bool lane_on,
                                            float part, const int (&sums)[8]) {
    const float s = segment_sum(part, p.nb);
    const int row = pass * p.rpw + rr;
    if (lane_on && kb == 0 && row < p.M) p.dst[row] = s;
    if constexpr (SUMS) {  // parity variant: the block's eight sub-block sums
        if (lane_on && row < p.M) {
            int32_t *o = p.sums + (int64_t)row * (p.K / 32) + kb * 8;
#pragma unroll
            for (int t = 0; t < 8; ++t) o[t] = sums[t];
        }
    }
}

// SUMS: the parity variant (also stores the int32 sub-block and activation
// sums, as the tile kernel's).
template <int WAVES, bool SUMS = false>
__global__ __launch_bounds__(kWave *WAVES) void gemv_q4k_bpl_kernel(Q4K_GEMV_KERNEL_ARGS) {
    p = with_head(p, Q4K_GEMV_HEAD_VALUES);
    int32_t *const sq_out = SUMS ? p.sq : nullptr;
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    int8_t *q8s = reinterpret_cast<int8_t *>(lds);
    float2 *dks = reinterpret_cast<float2 *>(lds + p.K);
    const int lane = threadIdx.x & (kWave - 1);
    const int rr = lane / p.nb;
    const int kb = lane - rr * p.nb;
    const bool lane_on = rr < p.rpw;

    const int tstride = gridDim.x * WAVES;
    int pa = blockIdx.x * WAVES + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const bool active = pa < p.ntiles;
    int pb = pa + tstride;
    bool vb = active && pb < p.ntiles;

    // activation loads first (the whole workgroup), then the weight loads of
    // each wave's first two passes
    ActStage<8, pre_rounds(1, kWave * WAVES)> xs;
    Q81Stage<pre_rounds(1, kWave * WAVES)> ys;
    if (p.x) stage_f32_issue<8, kWave * WAVES>(p.x, p.ldx, p.K, 1, p.vec_ok != 0, p.nblk32, xs);
    else stage_q81_issue<kWave * WAVES>(p.y, p.stride_col_y, p.K, 1, p.nblk32, ys);
    __syncthreads();
    u32x4 wa[9], wb[9];
    if (active) load_pass(p, pa, rr, kb, lane_on, wa);
    if (vb) load_pass(p, pb, rr, kb, lane_on, wb);
    if (p.x)
        stage_f32_finish<kLayoutLinear, 8, kWave * WAVES, 1>(p.x, p.ldx, p.K, 1, p.vec_ok != 0, p.nblk32, xs, p.K, q8s,
                                                          dks, sq_out);
    else
        stage_q81_finish<kLayoutLinear, kWave * WAVES, 1>(p.y, p.stride_col_y, p.K, 1, p.nblk32, ys, p.K, q8s, dks,
                                                       sq_out);
    __syncthreads();
    if (!active) return;  // no barrier below this point

    BlockAct act;
    {
        const int8_t *src = q8s + kb * kQK;
#pragma unroll
        for (int t = 0; t < 16; ++t) act.q[t] = *reinterpret_cast<const u32x4 *>(src + 16 * t);
#pragma unroll
        for (int s = 0; s < 8; ++s) {
            const float2 dk = dks[kb * 8 + s];
            act.d8[s] = dk.x;
            act.km[s] = dk.y;
        }
    }

    int sums[8];
    for (;;) {
        {
            const float part = block_dot(wa, act, sums);
            finish_pass<SUMS>(p, pa, rr, kb, lane_on, part, sums);
        }
        if (!vb) break;
        const int pa2 = pb + tstride;
        const bool va2 = pa2 < p.ntiles;
        if (va2) load_pass(p, pa2, rr, kb, lane_on, wa);
        {
            const float part = block_dot(wb, act, sums);
            finish_pass<SUMS>(p, pb, rr, kb, lane_on, part, sums);
        }
        if (!va2) break;
        const int pb2 = pa2 + tstride;
        vb = pb2 < p.ntiles;
        if (vb) load_pass(p, pb2, rr, kb, lane_on, wb);
        pa = pa2;
        pb = pb2;
    }
}

// ------------------------------------------------------------------------
// Block kernel: the block-per-lane arithmetic with coalesced loads.
//
// A pass (rpw rows x nb super-blocks, at most 64 blocks = 9216 bytes) is
// loaded with nine fully coalesced 16-byte loads -- lane l gets bytes
// [1024t + 16l, +16) of the pass -- written unchanged into a wave-private LDS
// slot, and read back by each lane as its own 144-byte block (stride 144 B
// is free of bank conflicts for 16-byte LDS reads).  Two passes are in
// flight per wave.
// ------------------------------------------------------------------------

constexpr int kSlotBytes = 64 * kBlockBytes;  // 9216

struct PassOffsets {
    uint32_t o[9];  // buffer offset of each of the lane's nine loads
};

__device__ __forceinline__ PassOffsets pass_offsets(const GemvParams &p, int lane) {
    const int row_bytes = p.nb * kBlockBytes;
    const int span = p.rpw * row_bytes;
    PassOffsets po;
#pragma unroll
    for (int t = 0; t < 9; ++t) {
        const int lin = 1024 * t + 16 * lane;
        int r = 0;
        while (r + 1 < p.rpw && lin >= (r + 1) * row_bytes) ++r;
        po.o[t] = lin < span ? (uint32_t)(r * p.row_stride + (lin - r * row_bytes)) : kOOB;
    }
    return po;
}

__device__ __forceinline__ void load_pass_coalesced(const GemvParams &p, int pass, const PassOffsets &po,
                                                    u32x4 (&w)[9]) {
    const int row0 = pass * p.rpw;
    const int nrows = min(p.rpw, p.M - row0);
    const __amdgpu_buffer_rsrc_t rs =
        make_rsrc(p.w + (int64_t)row0 * p.row_stride, (uint32_t)(nrows * p.row_stride));
#pragma unroll
    for (int t = 0; t < 9; ++t) w[t] = load16(rs, po.o[t]);
}

// landing registers -> LDS slot (pass order) -> this lane's 144-byte block
__device__ __forceinline__ void transpose_pass(uint8_t *slot, int lane, const u32x4 (&w)[9],
                                               u32x4 (&blk)[9]) {
#pragma unroll
    for (int t = 0; t < 9; ++t) *reinterpret_cast<u32x4 *>(slot + 1024 * t + 16 * lane) = w[t];
#pragma unroll
    for (int t = 0; t < 9; ++t) blk[t] = *reinterpret_cast<const u32x4 *>(slot + kBlockBytes * lane + 16 * t);
}

template <int WAVES>
__global__ __launch_bounds__(kWave *WAVES) void gemv_q4k_blk_kernel(Q4K_GEMV_KERNEL_ARGS) {
    p = with_head(p, Q4K_GEMV_HEAD_VALUES);
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    int8_t *q8s = reinterpret_cast<int8_t *>(lds);
    float2 *dks = reinterpret_cast<float2 *>(lds + p.K);
    const int act_bytes = p.K + p.K / 4;  // a multiple of 16: K % 256 == 0
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    uint8_t *slot = lds + act_bytes + wave * kSlotBytes;
    const int lane = threadIdx.x & (kWave - 1);
    const int rr = lane / p.nb;
    const int kb = lane - rr * p.nb;
    const bool lane_on = rr < p.rpw;

    const int tstride = gridDim.x * WAVES;
    int pa = blockIdx.x * WAVES + wave;
    const bool active = pa < p.ntiles;
    int pb = pa + tstride;
    bool vb = active && pb < p.ntiles;
    const PassOffsets po = pass_offsets(p, lane);

    // activation loads first (the whole workgroup), then the weight loads of
    // each wave's first two passes
    ActStage<8, pre_rounds(1, kWave * WAVES)> xs;
    Q81Stage<pre_rounds(1, kWave * WAVES)> ys;
    if (p.x) stage_f32_issue<8, kWave * WAVES>(p.x, p.ldx, p.K, 1, p.vec_ok != 0, p.nblk32, xs);
    else stage_q81_issue<kWave * WAVES>(p.y, p.stride_col_y, p.K, 1, p.nblk32, ys);
    __syncthreads();
    u32x4 wa[9], wb[9];
    if (active) load_pass_coalesced(p, pa, po, wa);
    if (vb) load_pass_coalesced(p, pb, po, wb);
    if (p.x) stage_f32_finish<kLayoutLinear, 8, kWave * WAVES, 1>(p.x, p.ldx, p.K, 1, p.vec_ok != 0, p.nblk32, xs, p.K, q8s, dks);
    else stage_q81_finish<kLayoutLinear, kWave * WAVES, 1>(p.y, p.stride_col_y, p.K, 1, p.nblk32, ys, p.K, q8s, dks);
    __syncthreads();
    if (!active) return;  // no barrier below this point

    BlockAct act;
    {
        const int8_t *src = q8s + kb * kQK;
#pragma unroll
        for (int t = 0; t < 16; ++t) act.q[t] = *reinterpret_cast<const u32x4 *>(src + 16 * t);
#pragma unroll
        for (int s = 0; s < 8; ++s) {
            const float2 dk = dks[kb * 8 + s];
            act.d8[s] = dk.x;
            act.km[s] = dk.y;
        }
    }

    u32x4 blk[9];
    for (;;) {
        transpose_pass(slot, lane, wa, blk);
        const int pa2 = pb + tstride;
        const bool va2 = vb && pa2 < p.ntiles;
        if (va2) load_pass_coalesced(p, pa2, po, wa);
        {
            int sums[8];
            const float part = block_dot(blk, act, sums);
            finish_pass(p, pa, rr, kb, lane_on, part, sums);
        }
        if (!vb) break;
        transpose_pass(slot, lane, wb, blk);
        const int pb2 = pa2 + tstride;
        const bool vb2 = va2 && pb2 < p.ntiles;
        if (vb2) load_pass_coalesced(p, pb2, po, wb);
        {
            int sums[8];
            const float part = block_dot(blk, act, sums);
            finish_pass(p, pb, rr, kb, lane_on, part, sums);
        }
        if (!va2) break;
        pa = pa2;
        pb = pb2;
        vb = vb2;
    }
}

}  // namespace q4k
