// q6k_gemv.hip -- gfx950 kernels of the Q6_K matrix-vector product and its
// C ABI (declared in include/q4k_gemv.h next to the Q4_K entry points).
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
#include <hip/hip_runtime.h>

#include <cstring>

#include "../../include/q4k_gemv.h"
#include "q4k_runtime.h"
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

__device__ __forceinline__ Q6Act q6_act(const GemvParams &p, const Q6Lane &ln, int i, int c, int ncols,
                                        const int8_t *q8s, const uint8_t *aux) {
    const int kb = 16 * i + ln.g;
    const int kbc = kb < p.nb ? kb : 0;  // blocks past the row's end: weights read as 0
    const int8_t *qa = q8s + c * p.qcol + i * 4096 + ln.lane * 16;
    Q6Act a;
#pragma unroll
    for (int m = 0; m < 4; ++m) a.a[m] = *reinterpret_cast<const u32x4 *>(qa + 1024 * m);
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

// Consumes one group held in w (one row, or the row and its gate row); at
// the tile's last group moves the R x NC sums to the result ring.
template <int NC, int R, int EPI>
__device__ __forceinline__ void q6_process_group(const GemvParams &p, const Q6Lane &ln, Step st,
                                                 const int8_t *q8s, const uint8_t *aux, const Q6Regs (&w)[R],
                                                 float (&acc)[R][NC], ResultRing &rr) {
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
        const Q6Act a = q6_act(p, ln, st.i, c, NC, q8s, aux);
#pragma unroll
        for (int r = 0; r < R; ++r) {
            int s[4];
            q6_lane_sums(v[r], a, s);
            // |s| <= 16*32*127 and |sc| <= 128: the 24-bit products are exact
            // in f32.  Explicit fmas fix the rounding for every launch geometry.
            float f = a.d8.x * (float)__mul24(s[0], sc[r][0]);
            f = __builtin_fmaf(a.d8.y, (float)__mul24(s[1], sc[r][1]), f);
            f = __builtin_fmaf(a.d8.z, (float)__mul24(s[2], sc[r][2]), f);
            f = __builtin_fmaf(a.d8.w, (float)__mul24(s[3], sc[r][3]), f);
            acc[r][c] = __builtin_fmaf(d[r], f, acc[r][c]);
        }
    }
    if (st.i == p.G - 1) tile_to_ring<NC, R, EPI>(p, ln.lane, acc, rr);
}

// Rows that are one group long: q6_process_group with the lane's activation
// slices (the same in every step) held in registers.
template <int NC, int EPI>
__device__ __forceinline__ void q6_process_reg(const GemvParams &p, const Q6Lane &ln, const Q6Act (&a)[NC],
                                               const Q6Regs (&w)[1], float (&acc)[1][NC], ResultRing &rr) {
    uint32_t v[4][4];
    int sc[4];
    q6_values(w[0], v);
    q6_scales(w[0], ln.jp, sc);
    const float d = half_bits_to_float(w[0].dw >> 16);
#pragma unroll
    for (int c = 0; c < NC; ++c) {
        int s[4];
        q6_lane_sums(v, a[c], s);
        float f = a[c].d8.x * (float)__mul24(s[0], sc[0]);
        f = __builtin_fmaf(a[c].d8.y, (float)__mul24(s[1], sc[1]), f);
        f = __builtin_fmaf(a[c].d8.z, (float)__mul24(s[2], sc[2]), f);
        f = __builtin_fmaf(a[c].d8.w, (float)__mul24(s[3], sc[3]), f);
        acc[0][c] = __builtin_fmaf(d, f, acc[0][c]);
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
template <int NC, int WAVES, int PRO, int S, int EPI = kEpiNone, bool BATCH = false>
__global__ __launch_bounds__(kWave *WAVES) void gemv_q6k_kernel(Q4K_GEMV_KERNEL_ARGS) {
    constexpr bool GLU = EPI == kEpiGlu;
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
        stage_f32_finish<kLayoutQ6K, kLPB, kWave * WAVES>(p.x, p.ldx, p.K, NC, p.vec_ok != 0, p.nblk32, xs,
                                                          p.qcol, q8s, aux);
    else
        stage_q81_finish<kLayoutQ6K, kWave * WAVES>(p.y, p.stride_col_y, p.K, NC, p.nblk32, ys, p.qcol, q8s,
                                                    aux);
    __syncthreads();
    if (remaining == 0) return;  // no barrier below this point
#pragma unroll
    for (int k = kEarly; k < S; ++k) q6_load_step<R>(p, ln, ws, st[k], w[k]);

    float acc[R][NC];
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
        for (int c = 0; c < NC; ++c) acc[r][c] = 0.0f;
    ResultRing rr{reinterpret_cast<float *>(lds + p.ring_off) + wave * ring_floats(NC), wr.beg, wr.end, 0, 0};

    // (one column at 16 waves, eight at 8 waves: wider variants would spill
    // registers)
    if constexpr ((NC == 1 || WAVES == 8) && R == 1 && S <= 2) {
        if (p.G == 1) {  // every step reads the same activation slice: keep it in registers
            Q6Act a0[NC];
#pragma unroll
            for (int c = 0; c < NC; ++c) a0[c] = q6_act(p, ln, 0, c, NC, q8s, aux);
            for (;;) {
#pragma unroll
                for (int k = 0; k < S; ++k) {
                    q6_process_reg<NC, EPI>(p, ln, a0, w[k], acc, rr);
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
            q6_process_group<NC, R, EPI>(p, ln, st[k], q8s, aux, w[k], acc, rr);
            st[k] = next_step(st[(k + S - 1) % S], p.G);
            q6_load_step<R>(p, ln, ws, st[k], w[k]);
        }
        remaining -= S;
        if (remaining <= 0) break;
    }
    ring_flush<NC, EPI>(p, ln.lane, rr);
}

// Parity probe: the int32 sums over every 16-weight scale group of
// (q - 32) * q8, from the tile kernel's lane map, staging and dot routine.
// One wave per (row, group); one activation column per launch.
struct Q6SumsParams {
    const uint8_t *w;
    int64_t row_stride;
    const uint8_t *y;  // one column of AoS Q8_1
    int32_t *s16;      // [M][K/16] for this column
    int M, K, nb, G, qcol;
    FastDiv nblk32;
};

__global__ __launch_bounds__(256) void q6_group_sums_kernel(Q6SumsParams p) {
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    int8_t *q8s = reinterpret_cast<int8_t *>(lds);
    uint8_t *aux = lds + p.qcol;
    stage_from_q8_1<kLayoutQ6K, 256>(p.y, 0, p.K, 1, p.nblk32, p.qcol, q8s, aux);
    __syncthreads();
    GemvParams gp{};
    gp.K = p.K;
    gp.nb = p.nb;
    gp.qcol = p.qcol;
    const Q6Lane ln = q6_lane(threadIdx.x & 63);
    const int nitems = p.M * p.G;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const __amdgpu_buffer_rsrc_t rs = make_rsrc(p.w, (uint32_t)(p.M * p.row_stride));
    for (int item = blockIdx.x * 4 + wave; item < nitems; item += gridDim.x * 4) {
        const int row = item / p.G;
        const int i = item - row * p.G;
        const int kb = 16 * i + ln.g;
        Q6Regs w;
        q6_load(rs, ln, (uint32_t)row * (uint32_t)p.row_stride + (uint32_t)i * (16 * kQ6Bytes), kb < p.nb, w);
        uint32_t v[4][4];
        q6_values(w, v);
        const Q6Act a = q6_act(gp, ln, i, 0, 1, q8s, aux);
        int s[4];
        q6_lane_sums(v, a, s);
        if (kb < p.nb) {
            int32_t *o = p.s16 + (int64_t)row * (p.K / 16) + kb * 16 + 8 * ln.h + ln.jp;
#pragma unroll
            for (int m = 0; m < 4; ++m) o[2 * m] = s[m];
        }
    }
}

// ------------------------------------------------------------------------
// host side
// ------------------------------------------------------------------------

// LDS of the staged activation: q8 columns in the Q6K layout, d8 per
// 32-value block (K/8 bytes per column), the -32*sum(q8) terms per 16 values
// (K/4 bytes per column), then a result ring per wave.
static int q6_act_bytes(int K, int nc) { return nc * (q8_col_bytes(K) + K / 8 + K / 4); }
static int q6_tile_lds_bytes(int K, int nc, int waves) { return q6_act_bytes(K, nc) + waves * ring_floats(nc) * 4; }

struct Q6Geometry {
    int waves = 16;
    int grid = 0;
    int lds = 0;
    int lds_launch = 0;
    int nc_chunk = 1;
    int rows_base = 0;
    int rows_extra = 0;
    int prologue = 0;
    int slots = 2;
};

// One workgroup per CU; one group (3360 bytes per wave) in flight per wave;
// 8 waves unless the activation is long (more than 8192 values over all
// columns: 16 waves quantise it in half the rounds) and the workgroup has 16
// or more steps; weight loads before quantisation when the activation fits
// the staging rounds issued ahead of them.  Measured on MI355X: with 210-byte blocks, more
// weight requests in flight (16 waves x 2 groups, 27.5 MB over the chip)
// delay the activation loads more than they hide latency.
static Q6Geometry pick_geometry_q6(const DeviceInfo &di, int64_t K, int64_t M, int64_t N, int64_t mats = 1,
                                   int fused = kFusedNone) {
    Q6Geometry g;
    const int max_lds = di.max_lds > 0 ? di.max_lds : 65536;
    const int cus = di.cus > 0 ? di.cus : 1;
    int nc = (int)N;
    while (nc > 1 && q6_tile_lds_bytes((int)K, nc, 16) > max_lds) nc = (nc + 1) / 2;
    g.nc_chunk = nc;
    const int owaves = g_ovr_waves.load(), owgs = g_ovr_wgs.load(), oslots = g_ovr_slots.load();
    g.grid = owgs > 0 ? owgs : grid_per_matrix(cus, mats, M);
    const int64_t steps_per_wg = (M + g.grid - 1) / g.grid * ((K / kQK + 15) / 16);
    g.waves = steps_per_wg >= 16 && (int64_t)nc * K > 8192 ? 16 : 8;
    // Six or more columns with rows of one group and >= 256 rows per
    // workgroup: 8 waves, whose registers hold every column's activation
    // slices (the step loop then reads no LDS), as in the Q4_K kernel.
    // Measured on MI355X: 128256 x 4096 N=8 126 -> 121 us; even at 128 rows
    // per workgroup (32768 x 4096) and 2 % slower at 56 (14336 x 4096).
    if (N >= 6 && K <= 16 * kQK && fused == kFusedNone && mats == 1 && (M + g.grid - 1) / g.grid >= 256)
        g.waves = 8;
    if (owaves >= 1 && owaves <= 16) g.waves = owaves > 8 ? 16 : 8;
    // One group in flight per wave, except in launches over several weight
    // matrices (MUL_MAT_ID, broadcasting) whose waves stream four or more
    // groups: there a second slot measured faster (Mixtral down 22.7 ->
    // 21.9 us, 2048 x 768 x 8 experts 9.35 -> 8.2 us), while on every
    // single-matrix shape it measured slower (1024 x 4096: 3.71 -> 4.71 us).
    g.slots = mats > 1 && steps_per_wg >= 4 * (int64_t)g.waves ? 2 : 1;
    if (oslots == 1 || oslots == 2) g.slots = oslots;
    g.rows_base = (int)(M / g.grid);
    g.rows_extra = (int)(M % g.grid);
    g.lds = q6_tile_lds_bytes((int)K, nc, g.waves);
    g.lds_launch = g.lds;
    if (owgs == 0 && g.lds_launch <= max_lds / 2) g.lds_launch = max_lds / 2 + 256;
    const bool pro0_ok = (int64_t)nc * (K / 32) <= (int64_t)stage_capacity(stage_lpb(nc), g.waves * kWave, nc);
    g.prologue = pro0_ok ? 0 : 1;
    const int opro = g_ovr_prologue.load();
    if (opro == 1 || (opro == 0 && pro0_ok)) g.prologue = opro;
    return g;
}

template <int NC, int WAVES, int S, int EPI, bool BATCH>
static const void *q6_sym(int pro) {
    return pro == 0 ? reinterpret_cast<const void *>(&gemv_q6k_kernel<NC, WAVES, 0, S, EPI, BATCH>)
                    : reinterpret_cast<const void *>(&gemv_q6k_kernel<NC, WAVES, 1, S, EPI, BATCH>);
}

template <int WAVES, int S, bool BATCH>
static const void *q6_sym_nc(int nc, int pro) {
    switch (nc) {
        case 1: return q6_sym<1, WAVES, S, kEpiNone, BATCH>(pro);
        case 2: return q6_sym<2, WAVES, S, kEpiNone, BATCH>(pro);
        case 3: return q6_sym<3, WAVES, S, kEpiNone, BATCH>(pro);
        case 4: return q6_sym<4, WAVES, S, kEpiNone, BATCH>(pro);
        case 5: return q6_sym<5, WAVES, S, kEpiNone, BATCH>(pro);
        case 6: return q6_sym<6, WAVES, S, kEpiNone, BATCH>(pro);
        case 7: return q6_sym<7, WAVES, S, kEpiNone, BATCH>(pro);
        case 8: return q6_sym<8, WAVES, S, kEpiNone, BATCH>(pro);
        default: return nullptr;
    }
}

template <int EPI, bool BATCH>
static const void *q6_kernel_epi(int waves, int pro, int slots) {
    if (waves <= 8) return slots == 1 ? q6_sym<1, 8, 1, EPI, BATCH>(pro) : q6_sym<1, 8, 2, EPI, BATCH>(pro);
    return slots == 1 ? q6_sym<1, 16, 1, EPI, BATCH>(pro) : q6_sym<1, 16, 2, EPI, BATCH>(pro);
}

template <bool BATCH>
static const void *q6_kernel_for(int nc, int waves, int pro, int slots, int fused) {
    if (pro != 0 && pro != 1) return nullptr;
    if (fused) {
        if (nc != 1) return nullptr;
        return fused == kFusedGate ? q6_kernel_epi<kEpiGlu, BATCH>(waves, pro, slots)
                                   : q6_kernel_epi<kEpiBias, BATCH>(waves, pro, slots);
    }
    if (waves <= 8) return slots == 1 ? q6_sym_nc<8, 1, BATCH>(nc, pro) : q6_sym_nc<8, 2, BATCH>(nc, pro);
    return slots == 1 ? q6_sym_nc<16, 1, BATCH>(nc, pro) : q6_sym_nc<16, 2, BATCH>(nc, pro);
}

int check_weight_q6(const void *src0, int64_t ne00, int64_t ne01, int64_t nb01) {
    if (ne00 <= 0 || ne00 % kQK != 0 || ne01 < 0) return Q4K_EINVAL;
    const int64_t row_bytes = ne00 / kQK * kQ6Bytes;
    if (nb01 < row_bytes || nb01 % kQ6Bytes != 0) return Q4K_EINVAL;
    if (ne01 > 0 && !src0) return Q4K_EINVAL;
    if (!aligned(src0, 2)) return Q4K_EINVAL;  // fp16 fields
    if (nb01 > (int64_t)1 << 28 || ne01 > ((int64_t)1 << 31) - 8 || ne00 > (1 << 24))
        return Q4K_EUNSUPPORTED;
    return Q4K_OK;
}

int run_gemv_q6(const void *src0, int64_t ne00, int64_t ne01, int64_t nb01, const float *x, int64_t ldx,
                const uint8_t *y, int64_t stride_col_y, int64_t ncols, float *dst, int64_t ld_dst,
                hipStream_t stream, const Epilogue *ep, const BatchLaunch *bl) {
    DeviceInfo *di = nullptr;
    int st = device_info(&di);
    if (st != Q4K_OK) return st;
    const int fused = fused_kind(ep);
    if (fused && ncols != 1) return Q4K_EINVAL;
    if (bl && ((int64_t)bl->nch > 65535 || (int64_t)bl->nsmp > 65535)) return Q4K_EUNSUPPORTED;
    const int64_t mats = bl ? (int64_t)bl->nch * bl->nsmp : 1;
    const Q6Geometry geo = pick_geometry_q6(*di, ne00, ne01, ncols, mats, fused);
    if (geo.lds > di->max_lds) return Q4K_EUNSUPPORTED;  // one column exceeds the LDS
    // a wave's rows are addressed with 31-bit offsets; column strides travel
    // as 32-bit kernel arguments
    if ((int64_t)(geo.rows_base / geo.waves + 2) * nb01 >= ((int64_t)1 << 31)) return Q4K_EUNSUPPORTED;
    if (ldx > INT32_MAX || stride_col_y > INT32_MAX) return Q4K_EUNSUPPORTED;
    for (int64_t c0 = 0; c0 < ncols; c0 += geo.nc_chunk) {
        const int nc = (int)(ncols - c0 < geo.nc_chunk ? ncols - c0 : geo.nc_chunk);
        int lds_launch = geo.lds_launch;
        const int lds = q6_tile_lds_bytes((int)ne00, nc, geo.waves);
        if (lds_launch < lds) lds_launch = lds;
        GemvParams p{};
        p.w = static_cast<const uint8_t *>(src0);
        p.row_stride = nb01;
        p.x = x ? x + c0 * ldx : nullptr;
        p.ldx = ldx;
        p.y = y ? y + c0 * stride_col_y * kQ81Bytes : nullptr;
        p.stride_col_y = stride_col_y;
        p.dst = dst + c0 * ld_dst;
        p.ld_dst = ld_dst;
        p.M = (int)ne01;
        p.K = (int)ne00;
        p.nb = (int)(ne00 / kQK);
        p.G = (p.nb + 15) / 16;
        p.qcol = q8_col_bytes((int)ne00);
        p.vec_ok = x && aligned(p.x, 16) && (ldx % 4 == 0);
        p.rows_base = geo.rows_base;
        p.rows_extra = geo.rows_extra;
        p.ring_off = q6_act_bytes(p.K, nc);
        p.nblk32 = fastdiv_init((uint32_t)(ne00 / 32));
        if (fused) {
            p.gate = ep->gate;
            p.bias = ep->bias;
            p.gate_bias = ep->gate ? ep->gate_bias : nullptr;
            p.glu_op = ep->glu_op;
        }
        const void *fn = bl ? q6_kernel_for<true>(nc, geo.waves, geo.prologue, geo.slots, fused)
                            : q6_kernel_for<false>(nc, geo.waves, geo.prologue, geo.slots, fused);
        if (bl) p.bt = bl->bt;
        if (!fn) return Q4K_EINVAL;
        st = ensure_lds(di, fn, lds_launch);
        if (st != Q4K_OK) return st;
        int32_t ldx32 = (int32_t)p.ldx, scy32 = (int32_t)p.stride_col_y;
        void *args[] = {&p.x, &p.y, &p.w, &p.row_stride, &ldx32, &scy32, &p.K, &p.vec_ok,
                        &p.rows_base, &p.rows_extra, &p.nb, &p.qcol, &p};
        const dim3 grid((unsigned)geo.grid, bl ? (unsigned)bl->nch : 1u, bl ? (unsigned)bl->nsmp : 1u);
        // the launch's own status, as in the Q4_K launch
        const hipError_t e = hipLaunchKernel(fn, grid, dim3(kWave * geo.waves), args, (size_t)lds_launch, stream);
        if (e != hipSuccess) return hip_fail(e);
    }
    return Q4K_OK;
}

}  // namespace q4k

using namespace q4k;

extern "C" {

int q6k_mul_mat_vec_q(const void *src0, int64_t ne00, int64_t ne01, int64_t nb01, const float *src1,
                      int64_t ne11, int64_t nb11, float *dst, int64_t nb1, void *workspace,
                      size_t workspace_bytes, void *stream) {
    int st = check_weight_q6(src0, ne00, ne01, nb01);
    if (st != Q4K_OK) return st;
    if (ne11 < 0 || ne11 > Q4K_MAX_BATCH) return Q4K_EINVAL;
    if (ne01 == 0 || ne11 == 0) return Q4K_OK;
    if (!src1 || !dst) return Q4K_EINVAL;
    if (nb11 % 4 != 0 || nb1 % 4 != 0) return Q4K_EINVAL;
    if (ne11 > 1 && (nb11 < ne00 * 4 || nb1 < ne01 * 4)) return Q4K_EINVAL;
    if (!aligned(src1, 4) || !aligned(dst, 4)) return Q4K_EINVAL;
    DeviceInfo *di = nullptr;
    st = device_info(&di);
    if (st != Q4K_OK) return st;
    const hipStream_t s = (hipStream_t)stream;
    const Q6Geometry geo = pick_geometry_q6(*di, ne00, ne01, ne11);
    const int64_t ldx = nb11 / 4, ldd = nb1 / 4;
    const size_t need = q4k_q8_1_bytes(ne00, ne11);
    const bool ws_fits = workspace && workspace_bytes >= need && aligned(workspace, 4);
    if (geo.nc_chunk >= ne11 && !(ws_fits && prefer_prequantised(ne00, ne11)))
        return run_gemv_q6(src0, ne00, ne01, nb01, src1, ldx, nullptr, 0, ne11, dst, ldd, s);
    // activation too large for one workgroup's LDS at this column count, or
    // (with a workspace) too many values for every workgroup to quantise:
    // quantise once to a Q8_1 buffer and run the GEMV on it
    void *buf = workspace;
    bool owned = false;
    if (buf) {
        if (workspace_bytes < need || !aligned(buf, 4)) return Q4K_EINVAL;
    } else {
        hipError_t e = hipMallocAsync(&buf, need, s);
        if (e != hipSuccess) {
            g_last_hip_error = (int32_t)e;
            return Q4K_ENOMEM;
        }
        owned = true;
    }
    const int64_t kp = pad512(ne00);
    st = q4k_quantize_row_q8_1(src1, buf, ne00, ldx, kp, ne11, stream);
    if (st == Q4K_OK)
        st = run_gemv_q6(src0, ne00, ne01, nb01, nullptr, 0, static_cast<const uint8_t *>(buf), kp / 32, ne11,
                         dst, ldd, s);
    if (owned) {
        hipError_t e = hipFreeAsync(buf, s);
        if (e != hipSuccess && st == Q4K_OK) st = hip_fail(e);
    }
    return st;
}

int q6k_op_mul_mat_vec_q(const void *src0_dd_i, int64_t ne00, int64_t row_low, int64_t row_high,
                         const void *src1_ddq_i, int64_t src1_ncols, int64_t src1_padded_row_size,
                         float *dst_dd_i, int64_t nrows_dst, void *stream) {
    if (row_low < 0 || row_high < row_low) return Q4K_EINVAL;
    const int64_t row_diff = row_high - row_low;
    if (ne00 <= 0 || ne00 % kQK != 0) return Q4K_EINVAL;
    int st = check_weight_q6(src0_dd_i, ne00, row_diff, ne00 / kQK * kQ6Bytes);
    if (st != Q4K_OK) return st;
    if (src1_ncols < 0 || src1_ncols > Q4K_MAX_BATCH) return Q4K_EINVAL;
    if (row_diff == 0 || src1_ncols == 0) return Q4K_OK;
    if (!src1_ddq_i || !dst_dd_i) return Q4K_EINVAL;
    if (src1_padded_row_size < ne00 || src1_padded_row_size % 32 != 0) return Q4K_EINVAL;
    if (nrows_dst < row_diff) return Q4K_EINVAL;
    if (!aligned(src1_ddq_i, 4) || !aligned(dst_dd_i, 4)) return Q4K_EINVAL;
    return run_gemv_q6(src0_dd_i, ne00, row_diff, ne00 / kQK * kQ6Bytes, nullptr, 0,
                       static_cast<const uint8_t *>(src1_ddq_i), src1_padded_row_size / 32, src1_ncols, dst_dd_i,
                       nrows_dst, (hipStream_t)stream);
}

int q6k_group_sums(const void *src0, int64_t ne00, int64_t ne01, int64_t nb01, const void *q8_1,
                   int64_t ncols, int64_t stride_col_y, int32_t *s16, void *stream) {
    int st = check_weight_q6(src0, ne00, ne01, nb01);
    if (st != Q4K_OK) return st;
    if (ncols < 0 || ncols > Q4K_MAX_BATCH) return Q4K_EINVAL;
    if (ne01 == 0 || ncols == 0) return Q4K_OK;
    if (!q8_1 || !s16 || stride_col_y < ne00 / 32 || !aligned(q8_1, 4) || !aligned(s16, 4)) return Q4K_EINVAL;
    if (ne01 * nb01 >= ((int64_t)1 << 31)) return Q4K_EUNSUPPORTED;  // one buffer descriptor
    DeviceInfo *di = nullptr;
    st = device_info(&di);
    if (st != Q4K_OK) return st;
    const int lds = q6_act_bytes((int)ne00, 1);
    if (lds > di->max_lds) return Q4K_EUNSUPPORTED;
    st = ensure_lds(di, reinterpret_cast<const void *>(&q6_group_sums_kernel), lds);
    if (st != Q4K_OK) return st;
    const int nb = (int)(ne00 / kQK);
    for (int64_t c = 0; c < ncols; ++c) {
        Q6SumsParams p{};
        p.w = static_cast<const uint8_t *>(src0);
        p.row_stride = nb01;
        p.y = static_cast<const uint8_t *>(q8_1) + c * stride_col_y * kQ81Bytes;
        p.s16 = s16 + c * ne01 * (ne00 / 16);
        p.M = (int)ne01;
        p.K = (int)ne00;
        p.nb = nb;
        p.G = (nb + 15) / 16;
        p.qcol = q8_col_bytes((int)ne00);
        p.nblk32 = fastdiv_init((uint32_t)(ne00 / 32));
        const int64_t items = ne01 * p.G;
        int grid = (int)((items + 3) / 4);
        if (grid > di->cus * 8) grid = di->cus * 8;
        void *args[] = {&p};
        const hipError_t e = hipLaunchKernel(reinterpret_cast<const void *>(&q6_group_sums_kernel), dim3(grid),
                                             dim3(256), args, (size_t)lds, (hipStream_t)stream);
        if (e != hipSuccess) return hip_fail(e);
    }
    return Q4K_OK;
}

int q6k_gemv_geometry(int64_t ne00, int64_t ne01, int64_t ne11, int32_t out[8]) {
    if (!out || ne00 <= 0 || ne00 % kQK != 0 || ne01 < 0 || ne11 < 1 || ne11 > Q4K_MAX_BATCH)
        return Q4K_EINVAL;
    DeviceInfo *di = nullptr;
    const int st = device_info(&di);
    if (st != Q4K_OK) return st;
    const Q6Geometry g = pick_geometry_q6(*di, ne00, ne01, ne11);
    out[0] = 1;
    out[1] = g.waves;
    out[2] = g.grid;
    out[3] = g.lds_launch;
    out[4] = g.nc_chunk;
    out[5] = g.nc_chunk >= ne11 ? 1 : 0;
    out[6] = 1;
    out[7] = g.slots;
    return Q4K_OK;
}

}  // extern "C"
