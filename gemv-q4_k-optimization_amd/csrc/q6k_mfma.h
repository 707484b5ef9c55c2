// q6k_mfma.h -- the Q6_K GEMV for several activation columns on the matrix
// cores: v_mfma_i32_16x16x64_i8 forms the int32 sums of every 16-weight scale
// group of a tile of 16 weight rows against up to 8 columns; the VALU unpacks
// the 6-bit weights and applies the per-(row, column, group) scales.
//
// The k dimension of one MFMA is 64 weights: lane group g = lane / 16 holds
// 16 of them (bytes t = 0..15), so one MFMA can keep four scale groups apart
// when each lane group carries one group and every A row has data in one
// lane group only.  For chunk j (0..3) of super-block kb:
//   lane group g  the scale group s = 4g + j, weights 64g + 16j + t of the
//                 super-block (ql[64h + 16j + t], nibble g & 1, qh[32h +
//                 16(j & 1) + t] bits 4(g & 1) + 2(j >> 1), h = g / 2);
//   A row i       activation column 4q + i % 4 (q: the MFMA's half of the
//                 eight columns) in lane group i / 4, zeros in the other
//                 three (read from a zero area of LDS);
//   B col r       weight row r of the tile, its 16 weights in lane group g as
//                 the bytes 4 (w - 32) (below);
//   D             D[i][r] = 4 S(r, 4q + i % 4, s = 4 (i / 4) + j), and lane l
//                 holds D[4(l / 16) + v][l % 16]: row l % 16, its own lane
//                 group's scale group, columns 4q + v.
// The weight byte is 4 (w - 32) = (w XOR 32) << 2 read as a signed byte: the
// 6-bit w with its top bit flipped is w - 32 as a 6-bit two's complement
// number, and the shift by two puts that sign bit at the byte's top.  The
// MFMA sums are then 4 times the sums of (w - 32) q8 that ggml's
// vec_dot_q6_K_q8_1 forms (kernels/vecdotq.cuh:580-600), exact, and no
// activation sums are needed.
//
// Scaling: scale groups 2b' and 2b'+1 of 32-value block b' share d8, and they
// are one lane's chunks j = 2b'' and 2b''+1 (b' = 2g + b''), so per column
// I = sc0 D0 + sc1 D1 is formed in int32 (|I| < 2^26, a multiple of 4:
// exact in float) and t += d8 * I; the row's d / 4 scales the item.
//
// Work split, summation segments, rounds and the reduction are those of the
// Q4_K matrix-core kernel (q4k_mfma.h): the result depends on K alone.  As
// there, the GA variants (pre-quantised route) bring each item's activation
// (super-block kb of the columns, 288 contiguous bytes of each) into an
// activation slot of the wave with the item's weights, and the LDS holds
// only the d8 table besides; chunk j of column c is q8 bytes 16 (j & 1) ..
// of block 2g + j / 2 of the column's 288.  A
// lane's eight column accumulators are summed over the four lane groups of
// its row at each segment end (two lane swaps), leaving lane l the columns
// 2(l / 16) and 2(l / 16) + 1 of row l % 16.
#pragma once

#include <hip/hip_runtime.h>

#include "q4k_mfma.h"
#include "q6k_kernels.h"

namespace q4k {

// per-wave partial results of a round: 64 lanes x 2 columns, two buffers
__host__ __device__ constexpr int q6m_part_bytes(int waves) { return 2 * waves * 64 * 8; }

// LDS layout (bytes from the start): NC q8 columns of qcol = K + 16 bytes,
// d8 of every 32-value block for 8 columns ([block][column], float), the
// zero area, the partials and one weight slot per wave.
__host__ __device__ constexpr int q6m_dk_off(int K, int nc) { return nc * mfma_qcol(K); }
__host__ __device__ constexpr int q6m_zero_off(int K, int nc) { return q6m_dk_off(K, nc) + (K / 32) * kMfmaCols * 4; }
__host__ __device__ constexpr int q6m_part_off(int K, int nc) { return q6m_zero_off(K, nc) + kMfmaZeroBytes; }
// Weight staging: an item (16 rows x one super-block, 16 x 210 bytes) arrives
// with four 64-lane x 16-byte loads and goes to the wave's LDS slot, rows 224
// bytes apart: chunk c = lane + 64i is row c / 14, o = c % 14, bytes
// [16o, +16) of its block for o < 13 and the block's last 16 bytes [194, 210)
// for o = 13 (no load reaches past a block, so a row at the end of the
// buffer is read whole), stored at 16o of the slot row: the scales at 192..207,
// d at 222..223.
constexpr int kQ6SlotPitch = 224;
constexpr int kQ6SlotBytes = kMfmaRows * kQ6SlotPitch;
constexpr int kQ6Chunks = kMfmaRows * kQ6SlotPitch / 16;  // 224
__host__ __device__ constexpr int q6m_slot_off(int K, int nc, int waves) {
    return q6m_part_off(K, nc) + q6m_part_bytes(waves);
}
__host__ __device__ constexpr int q6m_lds_bytes(int K, int nc, int waves) {
    return q6m_slot_off(K, nc, waves) + waves * kQ6SlotBytes;
}

// One item in flight: the lane's four 16-byte chunks.
struct Q6MLoad {
    u32x4 v[4];
};

// Per-lane constants.
struct Q6MLane {
    int lane;
    int wrow;          // weight row in the tile (B column, D column)
    int g;             // lane group: its scale groups 4g + j
    uint32_t rot_ql;   // rotation that moves its nibble to bits 2..5
    uint32_t rot_qh0;  // rotation that moves its qh bit pair to bits 6..7 (chunks 0, 1)
    uint32_t rot_qh1;  // (chunks 2, 3)
    int a_off[2];      // LDS byte offset of its A operand of super-block 0, chunk 0, column half q
    int a_step[2];     // its advance per chunk (16 (kb * 16 + j) from there): 16 (data lanes) or 0
    int dk_off;        // LDS byte offset of d8 of its block 2g, super-block 0, column 0
    uint32_t g_off[4]; // its chunks of an item: byte offsets from the item's first row
    int ar_off[2];       // GA: its A operand of chunk 0, column half q: offset in the activation slot
    bool a_data[2];      // GA: the lane carries activation in half q (else it reads the zero area)
    uint32_t ya_off[3];  // GA: its chunks of an item's activation, byte offsets from the item's first block
};

template <int NC, bool GA = false>
__device__ __forceinline__ Q6MLane q6m_lane(int K, int64_t stride_col_y = 0) {
    Q6MLane m;
    const int l = threadIdx.x & (kWave - 1);
    const int g = l >> 4;
    m.lane = l;
    m.wrow = l & 15;
    m.g = g;
    const uint32_t hi = (uint32_t)(g & 1);
    m.rot_ql = (4u * hi + 30u) & 31u;          // rotate right by 4 hi - 2
    m.rot_qh0 = (4u * hi + 26u) & 31u;         // by 4 hi - 6
    m.rot_qh1 = (4u * hi + 2u + 26u) & 31u;    // by 4 hi + 2 - 6
    // A: row i = l % 16 -> column 4q + i % 4, data in lane group i / 4
    const int i = l & 15;
    const bool data = (i >> 2) == g;
#pragma unroll
    for (int q = 0; q < 2; ++q) {
        const int c = 4 * q + (i & 3);
        const bool dq = data && c < NC;
        m.a_off[q] = dq ? c * mfma_qcol(K) + 64 * g : q6m_zero_off(K, NC) + 16 * (l & 7);
        m.a_step[q] = dq ? 16 : 0;
        m.ar_off[q] = c * kGaSuperBytes + 2 * g * kQ81Bytes + 4;
        m.a_data[q] = dq;
    }
#pragma unroll
    for (int i = 0; i < 3; ++i) {
        const int c = l + 64 * i, col = c / 18, o = c - 18 * col;
        m.ya_off[i] = col < NC ? (uint32_t)(col * stride_col_y) * (uint32_t)kQ81Bytes + 16u * (uint32_t)o : kOOB;
    }
    m.dk_off = (GA ? 0 : q6m_dk_off(K, NC)) + (2 * g) * kMfmaCols * 4;
    return m;
}

// GA LDS layout: the d8 table ([block][8 columns], float: K bytes), a zero
// area, the partials, one weight slot and one activation slot per wave.
__host__ __device__ constexpr int q6m_ga_zero_off(int K) { return K; }
__host__ __device__ constexpr int q6m_ga_part_off(int K) { return K + kGaZeroBytes; }
__host__ __device__ constexpr int q6m_ga_slot_off(int K, int waves) { return q6m_ga_part_off(K) + q6m_part_bytes(waves); }
__host__ __device__ constexpr int q6m_ga_aslot_off(int K, int waves) {
    return q6m_ga_slot_off(K, waves) + waves * kQ6SlotBytes;
}
__host__ __device__ constexpr int q6m_ga_lds_bytes(int K, int waves) {
    return q6m_ga_aslot_off(K, waves) + waves * kGaSlotBytes;
}

// GA: the lane's chunks of the activation of super-block kb (zeros past the
// NC columns).
__device__ __forceinline__ void q6m_load_act(__amdgpu_buffer_rsrc_t ry, const Q6MLane &ln, int kb, MfmaLoad &a) {
    const uint32_t o = (uint32_t)kb * (uint32_t)kGaSuperBytes;
#pragma unroll
    for (int i = 0; i < 3; ++i) a.v[i] = load16(ry, o + ln.ya_off[i]);
}

// The lane's chunk offsets of an item (rows row_stride bytes apart); chunks
// past the item's 224 get kOOB (their loads read zeros, nothing is written).
// In the slot, chunk c sits at 16c (the pitch is 14 chunks).
__device__ __forceinline__ void q6m_chunks(Q6MLane &m, int64_t row_stride) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int c = m.lane + 64 * i, r = c / 14, o = c - 14 * (c / 14);
        m.g_off[i] = c < kQ6Chunks ? (uint32_t)(r * row_stride) + 16u * (uint32_t)o - (o == 13 ? 14u : 0u) : kOOB;
    }
}

// Loads one item: one super-block of 16 rows whose first row's block starts
// at byte offset off of the workgroup's buffer (2-byte aligned), or zeros
// when off is kOOB.  As in the Q4_K kernel the sums need no selects: the
// buffer is under 2^31 bytes, so off + kOOB and kOOB + g_off read zeros, and
// kOOB + kOOB wraps to 0 only for chunks past the item's 224, which are
// never written to the slot.
__device__ __forceinline__ void q6m_load(__amdgpu_buffer_rsrc_t rs, uint32_t off, const Q6MLane &ln,
                                         Q6MLoad &w) {
#pragma unroll
    for (int i = 0; i < 4; ++i) w.v[i] = load16(rs, off + ln.g_off[i]);
}

// Writes an item to the wave's slot (GA: and its activation to the
// activation slot); the wait and the compiler barrier keep the lanes' reads
// of other lanes' bytes behind the writes.
template <bool GA = false>
__device__ __forceinline__ void q6m_stage(uint8_t *slot, const Q6MLane &ln, const Q6MLoad &w, uint8_t *aslot = nullptr,
                                          const MfmaLoad *a = nullptr, int nc = 0) {
    asm volatile("" ::: "memory");
#pragma unroll
    for (int i = 0; i < 4; ++i)
        if (i < 3 || ln.lane + 192 < kQ6Chunks) *reinterpret_cast<u32x4 *>(slot + 16 * ln.lane + 1024 * i) = w.v[i];
    if constexpr (GA) {
#pragma unroll
        for (int i = 0; i < 3; ++i)
            if (ln.lane + 64 * i < 18 * nc) *reinterpret_cast<u32x4 *>(aslot + 16 * (ln.lane + 64 * i)) = a->v[i];
    }
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
}

// 4 (w - 32) as signed bytes for four weights: ql dword (its nibble moved to
// bits 2..5 by rot_ql) and qh dword (pre-flipped by 0xaaaaaaaa, its bit pair
// moved to bits 6..7 by rot_qh).
__device__ __forceinline__ uint32_t q6m_bytes(uint32_t ql, uint32_t qhx, uint32_t rot_ql, uint32_t rot_qh) {
    const uint32_t lo = __builtin_amdgcn_alignbit(ql, ql, rot_ql) & 0x3c3c3c3cu;
    const uint32_t hi = __builtin_amdgcn_alignbit(qhx, qhx, rot_qh) & 0xc0c0c0c0u;
    return lo | hi;
}

// One item: eight MFMAs (four for up to four columns) and the scaling of
// their outputs into acc (the lane's row and scale groups, eight columns).
// SUMS: also stores the int32 group sums.
template <int NC, bool SUMS, bool GA = false>
__device__ __forceinline__ void q6m_item(const GemvParams &p, const Q6MLane &ln, const uint8_t *lds,
                                         const uint8_t *slot, int kb, float (&acc)[kMfmaCols], int row,
                                         bool row_ok, const uint8_t *const (&pa)[2]) {
    constexpr int NQ = NC > 4 ? 2 : 1;
    const uint8_t *wr = slot + ln.wrow * kQ6SlotPitch;
    const int h = ln.g >> 1;
    // qh bytes of chunks 0, 2 (jj = 0) and 1, 3 (jj = 1), their bit pairs'
    // top bits flipped
    u32x4 qh[2];
#pragma unroll
    for (int jj = 0; jj < 2; ++jj) {
        qh[jj] = *reinterpret_cast<const u32x4 *>(wr + 128 + 32 * h + 16 * jj);
#pragma unroll
        for (int e = 0; e < 4; ++e) qh[jj][e] ^= 0xaaaaaaaau;
    }
    const uint32_t scw = *reinterpret_cast<const uint32_t *>(wr + 192 + 4 * ln.g);
    const uint32_t dw = *reinterpret_cast<const uint32_t *>(wr + 220);  // d in the high half
    const float *dk = reinterpret_cast<const float *>(lds + ln.dk_off + kb * (8 * kMfmaCols * 4));
    float t[kMfmaCols];
#pragma unroll
    for (int c = 0; c < kMfmaCols; ++c) t[c] = 0.0f;
#pragma unroll
    for (int bb = 0; bb < 2; ++bb) {  // 32-value block 2g + bb: chunks 2bb, 2bb + 1
        const uint32_t rq = bb == 0 ? ln.rot_qh0 : ln.rot_qh1;
        i32x4 s[2][NQ];
#pragma unroll
        for (int jj = 0; jj < 2; ++jj) {
            const int j = 2 * bb + jj;
            const u32x4 ql = *reinterpret_cast<const u32x4 *>(wr + 64 * h + 16 * j);
            u32x4 bv;
#pragma unroll
            for (int e = 0; e < 4; ++e) bv[e] = q6m_bytes(ql[e], qh[jj][e], ln.rot_ql, rq);
#pragma unroll
            for (int q = 0; q < NQ; ++q) {
                u32x4 av;
                if constexpr (GA) {  // 4-byte aligned in the activation slot (data lanes)
                    const uint32_t *qa =
                        reinterpret_cast<const uint32_t *>(pa[q] + (ln.a_data[q] ? 36 * (j >> 1) + 16 * (j & 1) : 0));
                    av = u32x4{qa[0], qa[1], qa[2], qa[3]};
                } else {
                    av = *reinterpret_cast<const u32x4 *>(lds + ln.a_off[q] + ln.a_step[q] * (16 * kb + j));
                }
                s[jj][q] = __builtin_amdgcn_mfma_i32_16x16x64_i8(__builtin_bit_cast(i32x4, av),
                                                                 __builtin_bit_cast(i32x4, bv),
                                                                 i32x4{0, 0, 0, 0}, 0, 0, 0);
            }
        }
        // scales of groups 4g + 2bb, 4g + 2bb + 1 (signed bytes)
        const int sc0 = __builtin_amdgcn_sbfe((int)scw, 16u * bb, 8u);
        const int sc1 = __builtin_amdgcn_sbfe((int)scw, 16u * bb + 8u, 8u);
#pragma unroll
        for (int q = 0; q < NQ; ++q) {
            const float4 d8 = *reinterpret_cast<const float4 *>(dk + bb * kMfmaCols + 4 * q);
            const float d8v[4] = {d8.x, d8.y, d8.z, d8.w};
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                // |4S| < 2^18 and |sc| <= 128: 24-bit products; |I| < 2^26
                // and a multiple of 4, so exact in f32
                const int I = __mul24(s[0][q][v], sc0) + __mul24(s[1][q][v], sc1);
                t[4 * q + v] = __builtin_fmaf(d8v[v], (float)I, t[4 * q + v]);
            }
        }
        if constexpr (SUMS) {
            if (row_ok) {
#pragma unroll
                for (int jj = 0; jj < 2; ++jj)
#pragma unroll
                    for (int q = 0; q < NQ; ++q)
#pragma unroll
                        for (int v = 0; v < 4; ++v) {
                            const int c = 4 * q + v;
                            if (c < NC)
                                p.sums[((int64_t)c * p.M + row) * (p.K / 16) + kb * 16 + 4 * ln.g + 2 * bb + jj] =
                                    s[jj][q][v] / 4;
                        }
            }
        }
    }
    const float d4 = 0.25f * half_bits_to_float(dw >> 16);
#pragma unroll
    for (int c = 0; c < kMfmaCols; ++c) acc[c] = __builtin_fmaf(d4, t[c], acc[c]);
}

// Segment end: the lane's eight column sums over the four lane groups of its
// row; lane group g keeps columns 2g, 2g + 1 (v[0], v[1]); acc is cleared.
__device__ __forceinline__ void q6m_segment_sums(float (&acc)[kMfmaCols], float (&v)[2]) {
    float u[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {  // lanes 0..31 keep columns 0..3, 32..63 columns 4..7
        float a = acc[k], b = acc[k + 4];
        permlane32_swap(a, b);
        u[k] = a + b;
    }
#pragma unroll
    for (int k = 0; k < 2; ++k) {  // even 16-lane rows keep u[k], odd rows u[k + 2]
        float a = u[k], b = u[k + 2];
        permlane16_swap(a, b);
        v[k] = a + b;
    }
#pragma unroll
    for (int c = 0; c < kMfmaCols; ++c) acc[c] = 0.0f;
}

__device__ __forceinline__ void q6m_tree_push(int t, float (&v)[2], float (&l1)[2], float (&l2)[2], float (&l4)[2]) {
    if (t & 1) {
#pragma unroll
        for (int k = 0; k < 2; ++k) v[k] = l1[k] + v[k];
        if (t & 2) {
#pragma unroll
            for (int k = 0; k < 2; ++k) v[k] = l2[k] + v[k];
            if (t & 4) {
#pragma unroll
                for (int k = 0; k < 2; ++k) v[k] = l4[k] + v[k];
            } else {
#pragma unroll
                for (int k = 0; k < 2; ++k) l4[k] = v[k];
            }
        } else {
#pragma unroll
            for (int k = 0; k < 2; ++k) l2[k] = v[k];
        }
    } else {
#pragma unroll
        for (int k = 0; k < 2; ++k) l1[k] = v[k];
    }
}

// The kernel.  rows_base / rows_extra are the tile split: each workgroup
// owns rows_base tiles of 16 rows, the first rows_extra one more;
// p.rpw: KS, the waves that share one tile (1, 2, 4 or 8, at most S);
// p.ntiles: S, the segments of a row.  GA: the A operand from the Q8_1
// buffer p.y (which the GA variants require).
template <int NC, int WAVES, bool SUMS = false, bool GA = false>
__global__ __launch_bounds__(kWave *WAVES) void gemv_q6k_mfma_kernel(Q4K_GEMV_KERNEL_ARGS) {
    static_assert(NC >= 1 && NC <= kMfmaCols, "up to 8 columns");
    static_assert(WAVES == 8 || WAVES == 16, "8 or 16 waves");
    constexpr int NT = kWave * WAVES;
    p = with_head(p, Q4K_GEMV_HEAD_VALUES);
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    int8_t *q8s = reinterpret_cast<int8_t *>(lds);
    float *dks = reinterpret_cast<float *>(lds + q6m_dk_off(p.K, NC));

    Q6MLane ln = q6m_lane<NC, GA>(p.K, p.stride_col_y);
    q6m_chunks(ln, p.row_stride);
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int KS = p.rpw, S = p.ntiles;
    const int group = wave / KS, ks = wave - group * KS;
    const int ngroups = WAVES / KS;
    const int segs = S / KS, seg0 = ks * segs;  // the wave's run of segments
    const int b = (int)blockIdx.x;
    const int t0 = b * p.rows_base + min(b, p.rows_extra);
    const int nt = p.rows_base + (b < p.rows_extra ? 1 : 0);
    const int rounds = (nt + ngroups - 1) / ngroups;
    const int kb0 = seg0 * p.nb / S, kb1 = (seg0 + segs) * p.nb / S;  // kb1 > kb0 (S <= nb)
    const int items = rounds * (kb1 - kb0);
    const int row0 = t0 * kMfmaRows;
    const int nrows = min(nt * kMfmaRows, p.M - row0);
    const __amdgpu_buffer_rsrc_t rs =
        make_rsrc(p.w + (int64_t)row0 * p.row_stride, nrows > 0 ? (uint32_t)(nrows * p.row_stride) : 0u);

    constexpr int NQ = NC > 4 ? 2 : 1;
    constexpr int kLPB = stage_lpb(NC);
    constexpr int kPreR = GA ? 1 : pre_rounds(NC, NT);
    ActStage<kLPB, kPreR> xs;
    Q81Stage<kPreR> ys;
    if constexpr (!GA) {
        if (p.x) stage_f32_issue<kLPB, NT>(p.x, p.ldx, p.K, NC, p.vec_ok != 0, p.nblk32, xs);
        else stage_q81_issue<NT>(p.y, p.stride_col_y, p.K, NC, p.nblk32, ys);
        __syncthreads();  // all activation loads of this CU are queued first
    }
    const __amdgpu_buffer_rsrc_t ry =
        make_rsrc(p.y, GA ? (uint32_t)((int64_t)(NC - 1) * p.stride_col_y * kQ81Bytes + (p.K / 32) * kQ81Bytes) : 0u);

    auto next = [&](MfmaPos q) -> MfmaPos { return q.kb + 1 < kb1 ? MfmaPos{q.r, q.kb + 1} : MfmaPos{q.r + 1, kb0}; };
    auto item_off = [&](MfmaPos q) -> uint32_t {
        const int tile = group + ngroups * q.r;
        if (q.r >= rounds || tile >= nt) return kOOB;
        return (uint32_t)(tile * kMfmaRows * p.row_stride) + (uint32_t)q.kb * kQ6Bytes;
    };
    MfmaPos cur{0, kb0};
    MfmaPos ahead = cur;
    Q6MLoad w[2];
    MfmaLoad av[GA ? 2 : 1];
#pragma unroll
    for (int k = 0; k < 2; ++k) {
        q6m_load(rs, item_off(ahead), ln, w[k]);
        if constexpr (GA) q6m_load_act(ry, ln, ahead.kb, av[GA ? k : 0]);
        ahead = next(ahead);
    }

    if constexpr (GA) {
        // d8 of every (block, column); zeros for the padding columns
        float *d8s = reinterpret_cast<float *>(lds);
        for (int q = (int)threadIdx.x; q < (p.K / 32) * kMfmaCols; q += NT) {
            const int blk = q >> 3, c = q & 7;
            float dv = 0.0f;
            if (c < NC)
                dv = half_bits_to_float(
                    *reinterpret_cast<const uint32_t *>(p.y + ((int64_t)c * p.stride_col_y + blk) * kQ81Bytes));
            d8s[q] = dv;
        }
        // the zero area the A operand's zero lanes read
        if (threadIdx.x < kGaZeroBytes / 16)
            reinterpret_cast<u32x4 *>(lds + q6m_ga_zero_off(p.K))[threadIdx.x] = u32x4{0u, 0u, 0u, 0u};
    } else {
        if (p.x)
            stage_f32_finish<kLayoutMfmaQ6, kLPB, NT>(p.x, p.ldx, p.K, NC, p.vec_ok != 0, p.nblk32, xs,
                                                      mfma_qcol(p.K), q8s, dks);
        else
            stage_q81_finish<kLayoutMfmaQ6, NT>(p.y, p.stride_col_y, p.K, NC, p.nblk32, ys, mfma_qcol(p.K), q8s,
                                                dks);
        // the zero area of the A operand, and d8 of the padding columns (their
        // outputs are dropped; zeros keep them finite)
        if (threadIdx.x < kMfmaZeroBytes / 16)
            reinterpret_cast<u32x4 *>(lds + q6m_zero_off(p.K, NC))[threadIdx.x] = u32x4{0u, 0u, 0u, 0u};
        if constexpr (NC < kMfmaCols) {
            for (int q = (int)threadIdx.x; q < (p.K / 32) * (kMfmaCols - NC); q += NT) {
                const int blk = q / (kMfmaCols - NC), c = NC + q - blk * (kMfmaCols - NC);
                dks[blk * kMfmaCols + c] = 0.0f;
            }
        }
    }
    __syncthreads();

    float acc[kMfmaCols];
#pragma unroll
    for (int c = 0; c < kMfmaCols; ++c) acc[c] = 0.0f;
    float l1[2] = {0.0f, 0.0f}, l2[2] = {0.0f, 0.0f}, l4[2] = {0.0f, 0.0f};
    float *part = reinterpret_cast<float *>(lds + (GA ? q6m_ga_part_off(p.K) : q6m_part_off(p.K, NC)));
    uint8_t *slot = lds + (GA ? q6m_ga_slot_off(p.K, WAVES) : q6m_slot_off(p.K, NC, WAVES)) + wave * kQ6SlotBytes;
    uint8_t *aslot = lds + q6m_ga_aslot_off(p.K, WAVES) + wave * kGaSlotBytes;  // GA only
    const uint8_t *const pa[2] = {GA && ln.a_data[0] ? aslot + ln.ar_off[0] : lds + q6m_ga_zero_off(p.K),
                                  GA && ln.a_data[1] ? aslot + ln.ar_off[1] : lds + q6m_ga_zero_off(p.K)};
    int t = 0;                            // local segment of the current item
    int seg_end = (seg0 + 1) * p.nb / S;  // its end (super-block)
    // items go two at a time (load slot k holds item it); an odd count ends
    // with one item past the wave's, whose zeros add nothing
    for (int it = 0; it < items;) {
#pragma unroll
        for (int k = 0; k < 2; ++k, ++it) {
            const int tile = group + ngroups * cur.r;
            const int row = row0 + tile * kMfmaRows + ln.wrow;
            if constexpr (GA) {
                q6m_stage<true>(slot, ln, w[k], aslot, &av[GA ? k : 0], NC);
                q6m_load(rs, item_off(ahead), ln, w[k]);
                q6m_load_act(ry, ln, ahead.kb, av[GA ? k : 0]);
                q6m_item<NC, SUMS, true>(p, ln, lds, slot, cur.kb, acc, row,
                                         SUMS && it < items && tile < nt && row < p.M, pa);
            } else {
                q6m_stage(slot, ln, w[k]);
                q6m_load(rs, item_off(ahead), ln, w[k]);
                q6m_item<NC, SUMS>(p, ln, lds, slot, cur.kb, acc, row, SUMS && it < items && tile < nt && row < p.M,
                                   pa);
            }
            ahead = next(ahead);
            const MfmaPos done = cur;
            cur = next(cur);
            if (it < items && done.kb + 1 == seg_end) {
                float v[2];
                q6m_segment_sums(acc, v);
                q6m_tree_push(t, v, l1, l2, l4);
                ++t;
                if (t < segs) {
                    seg_end = (seg0 + t + 1) * p.nb / S;
                    continue;
                }
                // round end: v is the wave's subtree of the tile
                t = 0;
                seg_end = (seg0 + 1) * p.nb / S;
                const int buf = done.r & 1;
                *reinterpret_cast<float2 *>(part + ((buf * WAVES + wave) * 64 + ln.lane) * 2) = make_float2(v[0], v[1]);
                __syncthreads();
                // outputs of this round: tile group q, column c, row rr;
                // consecutive threads write consecutive rows of a column.
                // The KS subtrees combine in the same balanced tree.
                for (int o = (int)threadIdx.x; o < ngroups * kMfmaRows * kMfmaCols; o += NT) {
                    const int rr = o & 15, c = (o >> 4) & 7, q = o >> 7;
                    const int otile = q + ngroups * done.r;
                    const int orow = row0 + otile * kMfmaRows + rr;
                    if (c < NC && otile < nt && orow < p.M) {
                        const int l64 = rr + 16 * (c >> 1);
                        const float *src = part + ((buf * WAVES + q * KS) * 64 + l64) * 2 + (c & 1);
                        float pv[kMfmaMaxSegs];
#pragma unroll
                        for (int j = 0; j < kMfmaMaxSegs; ++j) pv[j] = j < KS ? src[j * 64 * 2] : 0.0f;
#pragma unroll
                        for (int wdt = 1; wdt < kMfmaMaxSegs; wdt *= 2)
#pragma unroll
                            for (int j = 0; j + wdt < kMfmaMaxSegs; j += 2 * wdt)
                                if (j + wdt < KS) pv[j] = pv[j] + pv[j + wdt];
                        p.dst[(int64_t)c * p.ld_dst + orow] = pv[0];
                    }
                }
            }
        }
    }
}

}  // namespace q4k
