// q4k_device.h -- device building blocks of the gfx950 Q4_K GEMV.
//
// Wave64 lane map of the tile kernel.  A wave consumes one "group" of 16
// consecutive Q4_K super-blocks of a weight row per step, four lanes per
// super-block:
//
//   lane = 4*g + j        g = super-block within the group (0..15)
//                         j = 32-byte chunk of the block's 128 qs bytes (0..3)
//   qs bytes [32j, 32j+32) of block kb = 16*i + g, as two 16-byte loads:
//     low  nibbles -> elements 64j + [0,32)       (sub-block 2j)
//     high nibbles -> elements 64j + 32 + [0,32)  (sub-block 2j+1)
//
// so each lane holds two whole sub-blocks: its integer dot products are the
// complete sub-block sums and the scale/min unpack and float scaling are paid
// once per 32 bytes.  The 16-byte block header (d, dmin, scales) is a third
// load per lane, shared by the block's four lanes.  Nibble order and
// sub-block pairing are those of kernels/vecdotq.cuh:785-794; the (sc, m)
// unpack is kernels/vecdotq.cuh:796-807 done with byte permutes.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace q4k {

constexpr int kQK = 256;          // weights per super-block
constexpr int kBlockBytes = 144;  // block_q4_K
constexpr int kQ81Bytes = 36;     // block_q8_1
constexpr int kWave = 64;
constexpr uint32_t kOOB = 0x80000000u;  // buffer offset that is always out of range

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

// gfx9 buffer descriptor word 3: 32-bit data format, no swizzle.
constexpr int kBufferWord3 = 0x00020000;

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void *base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), (short)0, (int)bytes,
                                             kBufferWord3);
}

// 16-byte buffer load; offsets at or beyond the descriptor's size return 0.
__device__ __forceinline__ u32x4 load16(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    return __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0);
}

// Signed 4 x int8 dot product starting a sum: the three-operand
// v_dot4_i32_i8 with an inline 0 (the compiler otherwise emits v_dot4c with
// the accumulator zeroed by a separate move).
__device__ __forceinline__ int sdot4_first(uint32_t a, uint32_t b) {
    int r;
    asm("v_dot4_i32_i8 %0, %1, %2, 0" : "=v"(r) : "v"(a), "v"(b));
    return r;
}

__device__ __forceinline__ float half_bits_to_float(uint32_t bits) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)(bits & 0xffffu));
}

template <int CTRL>
__device__ __forceinline__ int dpp(int v) {
    return __builtin_amdgcn_update_dpp(0, v, CTRL, 0xf, 0xf, true);
}
template <int CTRL>
__device__ __forceinline__ float dppf(float v) {
    return __builtin_bit_cast(float, dpp<CTRL>(__builtin_bit_cast(int, v)));
}

constexpr int kDppXor1 = 0xB1;   // quad_perm [1,0,3,2]
constexpr int kDppXor2 = 0x4E;   // quad_perm [2,3,0,1]
constexpr int kDppRor4 = 0x124;  // row_ror:4
constexpr int kDppRor8 = 0x128;  // row_ror:8
constexpr int kDppHalfMirror = 0x141;  // row_half_mirror: lane i <-> 7-i within 8 lanes

template <int XOR_MASK>
__device__ __forceinline__ float swizzle_xor(float v) {
    // ds_swizzle bit mode inside 32-lane halves: and_mask 0x1f, xor_mask
    return __builtin_bit_cast(
        float, __builtin_amdgcn_ds_swizzle(__builtin_bit_cast(int, v), 0x1f | (XOR_MASK << 10)));
}

constexpr int kDppBcast15 = 0x142;  // row_bcast:15 -- lane 15 of each row to the next row
constexpr int kDppBcast31 = 0x143;  // row_bcast:31 -- lane 31 to rows 2 and 3

// DPP move into the rows of ROW_MASK only; the other rows read 0.
template <int CTRL, int ROW_MASK>
__device__ __forceinline__ float dppf_rows(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL,
                                                                 ROW_MASK, 0xf, false));
}

// Sum over the 64 lanes, all in DPP (no LDS round trip); the result is
// wave-uniform.  After the four row steps every lane holds its 16-lane row's
// sum; the two broadcasts accumulate rows 0..3 into lane 63.
__device__ __forceinline__ float wave_sum(float v) {
    v += dppf<kDppXor1>(v);
    v += dppf<kDppXor2>(v);
    v += dppf<kDppRor4>(v);
    v += dppf<kDppRor8>(v);
    v += dppf_rows<kDppBcast15, 0xa>(v);
    v += dppf_rows<kDppBcast31, 0xc>(v);
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 63));
}

// Per-lane constants of the scale/min unpack for sub-block pair jp.
struct ScaleSel {
    uint32_t sel_x;  // bytes (2j', 2j'+1) of scales[0..3] and of scales[4..7]
    uint32_t sel_y;  // bytes (2j', 2j'+1) of scales[8..11], twice
    bool high;       // jp >= 2: 4+2 bit split fields
};

__device__ __forceinline__ ScaleSel make_scale_sel(int jp) {
    const uint32_t j = (uint32_t)(jp & 1) * 2u;
    ScaleSel s;
    s.sel_x = j | ((j + 1u) << 8) | ((j + 4u) << 16) | ((j + 5u) << 24);
    s.sel_y = j | ((j + 1u) << 8) | (j << 16) | ((j + 1u) << 24);
    s.high = jp >= 2;
    return s;
}

// Header dwords: h[0] = d | dmin << 16, h[1..3] = scales[0..11].
// Returns bytes {sc[2jp], sc[2jp+1], m[2jp], m[2jp+1]} (each 0..63).
__device__ __forceinline__ uint32_t unpack_scale_min(u32x4 h, const ScaleSel &s) {
    const uint32_t x = __builtin_amdgcn_perm(h[2], h[1], s.sel_x);
    const uint32_t y = __builtin_amdgcn_perm(h[3], h[3], s.sel_y);
    const uint32_t low = x & 0x3f3f3f3fu;
    const uint32_t split = (y & 0x00000f0fu) | ((y >> 4) & 0x0f0f0000u) | ((x >> 2) & 0x30303030u);
    return s.high ? split : low;
}

// The int32 sums over the lane's two whole sub-blocks: w0/w1 = its 32 qs
// bytes, a0/a1 = the 32 q8 of sub-block 2j, b0/b1 = those of sub-block 2j+1.
__device__ __forceinline__ void lane_qdot(u32x4 w0, u32x4 w1, u32x4 a0, u32x4 a1, u32x4 b0, u32x4 b1,
                                          int &sa, int &sb) {
    int a = sdot4_first(w0[0] & 0x0f0f0f0fu, a0[0]);
    int b = sdot4_first((w0[0] >> 4) & 0x0f0f0f0fu, b0[0]);
#pragma unroll
    for (int k = 1; k < 4; ++k) {
        a = __builtin_amdgcn_sdot4((int)(w0[k] & 0x0f0f0f0fu), (int)a0[k], a, false);
        b = __builtin_amdgcn_sdot4((int)((w0[k] >> 4) & 0x0f0f0f0fu), (int)b0[k], b, false);
    }
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        a = __builtin_amdgcn_sdot4((int)(w1[k] & 0x0f0f0f0fu), (int)a1[k], a, false);
        b = __builtin_amdgcn_sdot4((int)((w1[k] >> 4) & 0x0f0f0f0fu), (int)b1[k], b, false);
    }
    sa = a;
    sb = b;
}

__device__ __forceinline__ int byte_sum16(u32x4 a) {
    int s = 0;
#pragma unroll
    for (int k = 0; k < 4; ++k) s = __builtin_amdgcn_sdot4((int)a[k], 0x01010101, s, false);
    return s;
}

// ------------------------------------------------------------------------
// Activation staging into LDS.  Per column c (qcol bytes apart) the int8 q8
// values, followed after all columns by per-block auxiliary terms whose form
// depends on the weight type (LAYOUT):
//
//   linear    element e at c*qcol + e (qcol = K)
//   Q4K tile  the Q4_K tile kernel's read order: element e of super-block
//             kb = 16i + g, position 64j + 16k + t in the block, at
//             c*qcol + 4096i + 1024k + 16(4g + j) + t (qcol = 4096*ceil(K/4096)),
//             so that the 64 lanes of a wave reading chunk k of their blocks
//             read one contiguous, bank-conflict-free 1 KB.
//   Q4K K-split  the Q4K tile layout with the 16 super-block positions g of
//             a group permuted, at slot (g mod 8)*2 + g/8 (two-column tree)
//             or (g mod 4)*4 + g/4 (four-column tree): the several-column
//             K-split kernels' waves own positions {w, w+8} or {w, w+4, w+8,
//             w+12}, which the tile order puts 512 or 256 bytes apart, in
//             the same banks; permuted, a wave's lanes again read one
//             contiguous span.  Their auxiliary pairs are permuted alike
//             and padded to whole groups: dk[c*pb + 128i + 8*slot + s] for
//             block s of position g of group i (pb = K/32 rounded up to a
//             multiple of 128).
//   Q6K tile  the Q6_K tile kernel's read order: position 128h + 32m + 16j' + t
//             of super-block kb = 16i + g at c*qcol + 4096i + 1024m +
//             16(4g + 2h + j') + t -- lane 4g + 2h + j' reads, for each m, the 16
//             values that share one Q6_K scale.
//   Q6K K-split  the Q6K tile layout with the super-block positions
//             permuted as in the Q4K K-split layouts; per column its d8 of
//             whole groups, dq[c*3pb + 128i + 8*slot + s], then its -32 *
//             sum(q8) values, at c*3pb + pb + 16*(16i + slot) + 4(2h + j') + m
//             (int units from the start of the auxiliary area).
//   Q6K dense the Q6K tile layout with qcol = K: the row's last, partial
//             16-block group packs its four chunks 64 bytes per block apart
//             (1024m becomes cs*m, cs = 64*(nb mod 16); group_chunk_stride),
//             for column counts whose padded columns would not fit the LDS.
//   MFMA      linear q8 columns (qcol = K + 16: the skew puts eight columns'
//             16-byte reads at one offset in different banks) for the
//             matrix-core kernel; its auxiliary pairs are stored
//             [block][column] for 8 columns, dk[8b + c], so a lane reads the
//             pairs of four consecutive columns in two 16-byte reads.
//   MFMA Q6   the MFMA layout with d8 alone as the auxiliary term, d8[8b + c]
//             (the Q6_K matrix-core kernel folds the -32 offset into its
//             weight bytes, so it needs no activation sums).
//
// Auxiliary terms for the linear and Q4K layouts: per 32-value block b of
// column c, dk[c*K/32 + b] = (d8, d8 * sum of the block's q8) as a float2 --
// the second term is the factor of the Q4_K min correction, so the GEMV needs
// no per-lane byte sums.  For the Q6K layout: d8 as a float per 32-value
// block (float d8f[ncols*K/32]), then one int per 16-value half block,
// -32 * (sum of its q8) -- the Q6_K offset correction, the starting value of
// the lane's dot product -- at sq[ncols*K/32 + c*K/16 + 16kb + 4(2h + j') + m]
// (int units from the start of the auxiliary area), so a lane's four values
// are one 16-byte read.
// ------------------------------------------------------------------------
constexpr int kLayoutLinear = 0;
constexpr int kLayoutQ4K = 1;
constexpr int kLayoutQ6K = 2;
constexpr int kLayoutQ6KDense = 3;
constexpr int kLayoutMfma = 4;  // linear q8 columns; (d8, d8*sum) per [block][column] of 8 columns
constexpr int kLayoutMfmaQ6 = 5;  // linear q8 columns; d8 per [block][column] of 8 columns
constexpr int kLayoutQ4KS2 = 6;   // Q4K, positions permuted for the two-column K-split tree
constexpr int kLayoutQ4KS4 = 7;   // Q4K, positions permuted for the four-column K-split tree
constexpr int kLayoutQ6KS2 = 8;   // Q6K, positions permuted for the two-column K-split tree
constexpr int kLayoutQ6KS4 = 9;   // Q6K, positions permuted for the four-column K-split tree

constexpr bool is_q6_split_layout(int layout) { return layout == kLayoutQ6KS2 || layout == kLayoutQ6KS4; }

// Slot of super-block position g (0..15) of a group in the Q4K and Q6K layouts.
template <int LAYOUT>
__host__ __device__ constexpr int q4k_slot(int g) {
    return LAYOUT == kLayoutQ4KS2 || LAYOUT == kLayoutQ6KS2
               ? (g & 7) * 2 + (g >> 3)
               : (LAYOUT == kLayoutQ4KS4 || LAYOUT == kLayoutQ6KS4 ? (g & 3) * 4 + (g >> 2) : g);
}

constexpr bool is_q6_layout(int layout) { return layout == kLayoutQ6K || layout == kLayoutQ6KDense; }

// Chunk stride of 16-block group i of a row of nb super-blocks in the dense
// layout: 1024 bytes for a full group, 64 per block for a partial last one.
__host__ __device__ constexpr int group_chunk_stride(int i, int nb) {
    return 16 * (i + 1) <= nb ? 1024 : (nb & 15) * 64;
}

// LDS offset of values [4e, 4e+4) of 32-value block b of column c (rows of
// nb super-blocks).
template <int LAYOUT>
__device__ __forceinline__ int q8_offset(int c, int qcol, int nb, int b, int e) {
    if (LAYOUT == kLayoutLinear || LAYOUT == kLayoutMfma || LAYOUT == kLayoutMfmaQ6) return c * qcol + b * 32 + e * 4;
    const int kb = b >> 3, s = b & 7;
    if (LAYOUT == kLayoutQ4K || LAYOUT == kLayoutQ4KS2 || LAYOUT == kLayoutQ4KS4)
        return c * qcol + (kb >> 4) * 4096 + ((s & 1) * 2 + (e >> 2)) * 1024 +
               (q4k_slot<LAYOUT>(kb & 15) * 4 + (s >> 1)) * 16 + (e & 3) * 4;
    const int cs = LAYOUT == kLayoutQ6KDense ? group_chunk_stride(kb >> 4, nb) : 1024;
    // Q6K: s = 4h + m, values 16j' + 4(e & 3) + [0, 4) with j' = e >> 2
    return c * qcol + (kb >> 4) * 4096 + (s & 3) * cs +
           (q4k_slot<LAYOUT>(kb & 15) * 4 + (s >> 2) * 2 + (e >> 2)) * 16 + (e & 3) * 4;
}

// Int index (from the start of the auxiliary area) of the Q6K offset
// correction of half `half` of 32-value block b of column c; total = ncols*K/32.
__device__ __forceinline__ int q6_sq_index(int total, int nblk, int c, int b, int half) {
    const int kb = b >> 3, s = b & 7;
    return total + c * 2 * nblk + kb * 16 + ((s >> 2) * 2 + half) * 4 + (s & 3);
}

// Stores the auxiliary terms of 32-value block b (qb = c*nblk + b) from the
// lane holding values 16*half.. of it: d8 = half(d) widened, qsum = sum of
// all 32 q8 (Q4K/linear), hsum = sum of the lane's 16-value half (Q6K).
template <int LAYOUT>
__device__ __forceinline__ void store_aux(void *aux, int total, int nblk, int c, int b, int qb, int half,
                                          float d8, int qsum, int hsum) {
    if (is_q6_split_layout(LAYOUT)) {
        const int kb = b >> 3, s = b & 7, pb = (nblk + 127) & ~127;
        const int at = (kb >> 4) * 16 + q4k_slot<LAYOUT>(kb & 15);  // 16i + slot
        if (half == 0) reinterpret_cast<float *>(aux)[c * 3 * pb + at * 8 + s] = d8;
        reinterpret_cast<int *>(aux)[c * 3 * pb + pb + at * 16 + ((s >> 2) * 2 + half) * 4 + (s & 3)] = -32 * hsum;
    } else if (is_q6_layout(LAYOUT)) {
        if (half == 0) reinterpret_cast<float *>(aux)[qb] = d8;
        reinterpret_cast<int *>(aux)[q6_sq_index(total, nblk, c, b, half)] = -32 * hsum;
    } else if (LAYOUT == kLayoutMfma) {
        if (half == 0) reinterpret_cast<float2 *>(aux)[b * 8 + c] = make_float2(d8, d8 * (float)qsum);
    } else if (LAYOUT == kLayoutMfmaQ6) {
        if (half == 0) reinterpret_cast<float *>(aux)[b * 8 + c] = d8;
    } else if (LAYOUT == kLayoutQ4KS2 || LAYOUT == kLayoutQ4KS4) {
        if (half == 0) {
            const int kb = b >> 3, pb = (nblk + 127) & ~127;
            reinterpret_cast<float2 *>(aux)[c * pb + (kb >> 4) * 128 + q4k_slot<LAYOUT>(kb & 15) * 8 + (b & 7)] =
                make_float2(d8, d8 * (float)qsum);
        }
    } else if (half == 0) {
        reinterpret_cast<float2 *>(aux)[qb] = make_float2(d8, d8 * (float)qsum);
    }
}

// n / d for n < 2^31 as (umulhi(n, mul) + n) >> shift, with mul and shift
// from fastdiv_init on the host (Granlund-Montgomery round-up method).
struct FastDiv {
    uint32_t d, mul, shift;
};

__host__ __device__ inline FastDiv fastdiv_init(uint32_t d) {
    uint32_t l = 0;
    while (l < 32 && (1ull << l) < d) ++l;
    FastDiv f;
    f.d = d;
    f.shift = l;
    f.mul = (uint32_t)(((1ull << 32) * ((1ull << l) - d)) / d + 1);
    return f;
}

__device__ __forceinline__ uint32_t fastdiv(uint32_t n, const FastDiv &f) {
    return (__umulhi(n, f.mul) + n) >> f.shift;
}

// q[k] = roundf(v[k] / d) with the correctly rounded quotient, as ggml-cuda's
// quantize_q8_1 computes it.  y = v * rcp(d) is within 127 (2^-23 + 2^-24) <
// 2^-15.4 of v/d (|v/d| <= 127, v_rcp_f32 is 1-ulp accurate) and the rounded
// quotient within 2^-17 of it, so rint(y) is the answer unless y lies within
// 2^-15 of a half-integer; a lane with a value within 2^-14 of one (twice
// the margin; or a NaN) recomputes all its values with the exact division.
// One branch per lane instead of one per value.  rint(y) comes from adding
// 1.5 * 2^23: the sum is exact in its integer part for |y| < 2^22, so its low
// mantissa bits hold rint(y) (round-to-nearest-even, like the add itself)
// and subtracting the constant back gives it as a float.  Contraction is off
// so y is rounded on its own before the add.
template <int V, int H>
__device__ __forceinline__ bool quantize_pack(const float (&v)[V], float d, float rd, bool exact,
                                              uint32_t (&word)[V / 4], int (&hsum)[H]) {
#pragma clang fp contract(off)
    constexpr float kMagic = 12582912.0f;  // 1.5 * 2^23
    bool fast = true;
#pragma unroll
    for (int w = 0; w < V / 4; ++w) word[w] = 0;
#pragma unroll
    for (int h = 0; h < H; ++h) hsum[h] = 0;
#pragma unroll
    for (int k = 0; k < V; ++k) {
        int q;
        if (exact) {
            q = (int)roundf(v[k] / d);
        } else {
            const float y = v[k] * rd;
            const float m = y + kMagic;
            q = __builtin_bit_cast(int, m) - 0x4B400000;
            fast = fast && fabsf(y - (m - kMagic)) <= 0.5f - 0x1p-14f;
        }
        hsum[k * H / V] += q;
        word[k / 4] |= (uint32_t)(q & 0xff) << (8 * (k % 4));
    }
    return fast;
}

// The q8 of one lane's V values packed four to a dword, and the sums over
// its H halves of the block: the fast rounding, and the exact division when
// the lane has a value near a tie.  The bytes are packed as they are
// computed, so only the values, the packed words and the sums stay live.
template <int V, int H>
__device__ __forceinline__ void quantize_values(const float (&v)[V], float d, float rd,
                                                uint32_t (&word)[V / 4], int (&hsum)[H]) {
    if (!quantize_pack<V, H>(v, d, rd, false, word, hsum)) quantize_pack<V, H>(v, d, rd, true, word, hsum);
}

// F32 activation -> Q8_1 values with ggml-cuda's quantize_q8_1 arithmetic
// (call site kernels/mmvq.cu:734): per 32 values d = amax/127,
// q = amax == 0 ? 0 : roundf(x/d), and the kernel consumes half(d).
// LPB lanes per 32-value block (8 or 4), 32/LPB values per lane, consecutive
// lanes reading consecutive 16 bytes (fewer lanes per block, each reading
// 64-128 contiguous bytes, cut the quantisation's instructions but spread a
// wave's loads over 4-8 times the cache lines and measured slower): 8 lets a
// 16-wave workgroup cover a 4096-value column in one round, 4 halves the
// per-block overhead when several columns need several rounds (stage_lpb).
// Staging is split in two: issue() loads the first PRE rounds of values
// into registers, to be called before the kernel's first weight loads
// (vector loads complete in issue order, so values loaded after the weights
// would wait for them); finish() quantises them into LDS and handles any
// further rounds.  issue() loads unconditionally (lanes past the end re-read
// the last block): with no branches around them the compiler's wait for
// these values counts exactly the weight loads issued after them instead of
// waiting for all loads.
// PRE is 4, or, for workgroups of fewer than 1024 threads staging three or
// more columns, the rounds that 4096-value columns take (a round left to
// finish() waits for its loads behind the weight stream; a round past the
// values re-reads the last block, which measured slower too).
__host__ __device__ constexpr int pre_rounds(int ncols, int nt) { return nt >= 1024 || ncols <= 2 ? 4 : ncols; }
__host__ __device__ constexpr int stage_lpb(int ncols) { return ncols == 1 ? 8 : 4; }
// Blocks of 32 values the rounds issued ahead of the weight loads cover in a
// workgroup of nt threads.
__host__ __device__ constexpr int stage_capacity(int lpb, int nt, int ncols) {
    return pre_rounds(ncols, nt) * (nt / lpb);
}
// Weight slots a tile kernel issues before quantising the activation.
__host__ __device__ constexpr int early_slots(int pro, int slots) {
    return pro == 0 ? (slots < 2 ? slots : 2) : (pro == 2 ? slots : (pro == 3 ? 1 : 0));
}

// Rounds past the first PRE that finish() loads together (its CHUNK).  Two
// halve the memory round trips of the several-column launches whose
// activation outgrows the rounds issued ahead (4096 x 14336 N=8 24.1 ->
// 22.6 us, 1024 x 8192 N=8 11.4 -> 10.8 on MI355X); chunks of 4 and 8
// measured no better.  Kernels of up to three columns pass 1, one round at
// a time: they rarely have rounds left over; with one column the chunk's
// registers would take the kernel past the 64 that let two 16-wave (or four
// 8-wave) workgroups share a CU, and three columns measured 1-2 % faster
// without it (4096 x 4096 N=3 6.12 -> 5.99 us, 14336 x 4096 N=3 10.39 ->
// 10.21).
constexpr int kFinishRounds = 2;

template <int LPB, int PRE>
struct ActStage {
    float v[PRE][32 / LPB];
};

// amax / 127 rounded to nearest, as the IEEE division: the product with
// the rounded reciprocal corrected by one exact fma residual.  Equal to
// amax / 127.0f for every finite non-negative float (checked exhaustively).
__device__ __forceinline__ float div127(float a) {
    constexpr float kRcp127 = (float)(1.0 / 127.0);
    const float q0 = a * kRcp127;
    const float r = __builtin_fmaf(-q0, 127.0f, a);
    return __builtin_fmaf(r, kRcp127, q0);
}

// max(v, v of the lane that the DPP control names), as one v_max_f32 with
// the DPP source (through fmaxf the compiler inserts a canonicalising
// v_max after each DPP move).  The s_nop covers a VALU write of v right
// before.  NaN handling is v_max_f32's, as with fmaxf.
#define Q4K_DPP_MAX(CTRL)                                                                        \
    __device__ __forceinline__ float dpp_max_##CTRL(float v) {                                   \
        float r;                                                                                 \
        asm("s_nop 1\n\tv_max_f32_dpp %0, %1, %1 " Q4K_DPP_##CTRL " row_mask:0xf bank_mask:0xf" \
            : "=v"(r)                                                                            \
            : "v"(v));                                                                           \
        return r;                                                                                \
    }
#define Q4K_DPP_xor1 "quad_perm:[1,0,3,2]"
#define Q4K_DPP_xor2 "quad_perm:[2,3,0,1]"
#define Q4K_DPP_half_mirror "row_half_mirror"
Q4K_DPP_MAX(xor1)
Q4K_DPP_MAX(xor2)
Q4K_DPP_MAX(half_mirror)

// Reductions over the LPB lanes of a 32-value block (aligned lane groups).
template <int LPB>
__device__ __forceinline__ float block_max(float v) {
    v = dpp_max_xor1(v);
    v = dpp_max_xor2(v);
    if (LPB == 8) v = dpp_max_half_mirror(v);
    return v;
}

// Integer sums over the LPB lanes of a 32-value block: `half` over the lanes
// holding the lane's 16-value half of the block, `full` over all 32 values.
template <int LPB>
__device__ __forceinline__ void block_sums(int v, int &half, int &full) {
    v += dpp<kDppXor1>(v);
    if (LPB == 8) v += dpp<kDppXor2>(v);
    half = v;
    v += LPB == 8 ? dpp<kDppHalfMirror>(v) : dpp<kDppXor2>(v);
    full = v;
}

// sq_out (parity variants only; a literal null in the product kernels, so the
// store compiles away): the int32 sum of the block's 32 q8 at sq_out[qb].
template <int LAYOUT, int LPB>
__device__ __forceinline__ void quantize_block_part(const float (&v)[32 / LPB], int e, int qcol, int c,
                                                    int b, int qb, int total, int nblk, int8_t *q8s,
                                                    void *aux, int32_t *sq_out = nullptr) {
    constexpr int V = 32 / LPB;
    float amax = 0.0f;
#pragma unroll
    for (int k = 0; k < V; ++k) amax = fmaxf(amax, fabsf(v[k]));
    amax = block_max<LPB>(amax);
    const float d = div127(amax);
    const float rd = __builtin_amdgcn_rcpf(d);
    uint32_t word[V / 4];
    int qsum[1];
    if (amax != 0.0f) {
        quantize_values<V, 1>(v, d, rd, word, qsum);
    } else {
#pragma unroll
        for (int w = 0; w < V / 4; ++w) word[w] = 0;
        qsum[0] = 0;
    }
    int hsum, fsum;
    block_sums<LPB>(qsum[0], hsum, fsum);
    int8_t *dst = q8s + q8_offset<LAYOUT>(c, qcol, nblk >> 3, b, e * (V / 4));
    if (V == 4) *reinterpret_cast<uint32_t *>(dst) = word[0];
    else *reinterpret_cast<uint2 *>(dst) = make_uint2(word[0], word[V / 4 - 1]);
    const float d8 = (float)(_Float16)d;
    if ((e & (LPB / 2 - 1)) == 0) store_aux<LAYOUT>(aux, total, nblk, c, b, qb, e / (LPB / 2), d8, fsum, hsum);
    if (sq_out && e == 0) sq_out[qb] = fsum;
}

template <int V>
__device__ __forceinline__ void load_xv(const float *src, bool vec_ok, float (&v)[V]) {
    if (vec_ok) {
#pragma unroll
        for (int k = 0; k < V; k += 4) {
            const float4 a = *reinterpret_cast<const float4 *>(src + k);
            v[k] = a.x; v[k + 1] = a.y; v[k + 2] = a.z; v[k + 3] = a.w;
        }
    } else {
#pragma unroll
        for (int k = 0; k < V; ++k) v[k] = src[k];
    }
}

// NT: threads per workgroup, a compile-time constant of every kernel (reading
// blockDim would put a dependent kernel-argument load ahead of the first
// activation load).
template <int LPB, int NT, int PRE>
__device__ __forceinline__ void stage_f32_issue(const float *__restrict__ x, int64_t ldx, int K,
                                                int ncols, bool vec_ok, const FastDiv &fd,
                                                ActStage<LPB, PRE> &st) {
    constexpr int V = 32 / LPB;
    const int nblk = K / 32;
    const int total = ncols * nblk;
    const int e = threadIdx.x & (LPB - 1);
    constexpr int step = NT / LPB;
#pragma unroll
    for (int j = 0; j < PRE; ++j) {
        if (j >= 4 && j * step >= total) break;  // uniform: rounds past the values are not loaded
        const int qb = min((int)(threadIdx.x / LPB) + j * step, total - 1);
        const int c = ncols == 1 ? 0 : (int)fastdiv((uint32_t)qb, fd);
        const int b = qb - c * nblk;
        load_xv<V>(x + c * ldx + b * 32 + e * V, vec_ok, st.v[j]);
    }
}

template <int LAYOUT, int LPB, int NT, int CHUNK = kFinishRounds, int PRE>
__device__ __forceinline__ void stage_f32_finish(const float *__restrict__ x, int64_t ldx, int K,
                                                 int ncols, bool vec_ok, const FastDiv &fd,
                                                 const ActStage<LPB, PRE> &st, int qcol, int8_t *q8s,
                                                 void *aux, int32_t *sq_out = nullptr) {
    constexpr int V = 32 / LPB;
    const int nblk = K / 32;
    const int total = ncols * nblk;
    const int e = threadIdx.x & (LPB - 1);
    constexpr int step = NT / LPB;
#pragma unroll
    for (int j = 0; j < PRE; ++j) {
        const int qb = (int)(threadIdx.x / LPB) + j * step;
        if (qb < total) {
            const int c = ncols == 1 ? 0 : (int)fastdiv((uint32_t)qb, fd);
            quantize_block_part<LAYOUT, LPB>(st.v[j], e, qcol, c, qb - c * nblk, qb, total, nblk, q8s, aux,
                                             sq_out);
        }
    }
    // Further rounds a chunk at a time: all their loads first, then their
    // quantisation, so a chunk costs one memory round trip rather than one
    // per round.  A round past every block of the wave's lanes is not
    // loaded (q0w, the wave's first active lane, holds its smallest block);
    // in the others, lanes past the end re-read the last block.
    constexpr int kChunk = CHUNK;
    for (int q0 = (int)(threadIdx.x / LPB) + PRE * step; q0 < total; q0 += kChunk * step) {
        const int q0w = __builtin_amdgcn_readfirstlane(q0);
        float v[kChunk][V];
#pragma unroll
        for (int j = 0; j < kChunk; ++j) {
            if (j > 0 && q0w + j * step >= total) break;
            const int qb = min(q0 + j * step, total - 1);
            const int c = ncols == 1 ? 0 : (int)fastdiv((uint32_t)qb, fd);
            load_xv<V>(x + c * ldx + (qb - c * nblk) * 32 + e * V, vec_ok, v[j]);
        }
#pragma unroll
        for (int j = 0; j < kChunk; ++j) {
            const int qb = q0 + j * step;
            if (qb < total) {
                const int c = ncols == 1 ? 0 : (int)fastdiv((uint32_t)qb, fd);
                quantize_block_part<LAYOUT, LPB>(v[j], e, qcol, c, qb - c * nblk, qb, total, nblk, q8s, aux,
                                                 sq_out);
            }
        }
    }
}

// Rounds [J0, J1) of stage_f32_finish (J1 <= PRE: values already in
// registers), for a caller that interleaves the rounds with other work.
// With one column and NT / LPB = 128, round j is the 4096 values of
// 16-block group j.
template <int LAYOUT, int LPB, int NT, int J0, int J1, int PRE>
__device__ __forceinline__ void stage_f32_rounds(int K, int ncols, const FastDiv &fd, const ActStage<LPB, PRE> &st,
                                                 int qcol, int8_t *q8s, void *aux, int32_t *sq_out = nullptr) {
    static_assert(0 <= J0 && J0 <= J1 && J1 <= PRE, "rounds held in registers");
    const int nblk = K / 32;
    const int total = ncols * nblk;
    const int e = threadIdx.x & (LPB - 1);
    constexpr int step = NT / LPB;
#pragma unroll
    for (int j = J0; j < J1; ++j) {
        const int qb = (int)(threadIdx.x / LPB) + j * step;
        if (qb < total) {
            const int c = ncols == 1 ? 0 : (int)fastdiv((uint32_t)qb, fd);
            quantize_block_part<LAYOUT, LPB>(st.v[j], e, qcol, c, qb - c * nblk, qb, total, nblk, q8s, aux,
                                             sq_out);
        }
    }
}

// Already-quantised AoS block_q8_1 (column stride stride_col_y blocks) -> LDS,
// in the same two phases: the first PRE rounds' bytes are loaded by issue().
template <int PRE>
struct Q81Stage {
    uint32_t w[PRE][2];
    uint32_t ds[PRE];
};

template <int NT, int PRE>
__device__ __forceinline__ void stage_q81_issue(const uint8_t *__restrict__ y, int64_t stride_col_y,
                                                int K, int ncols, const FastDiv &fd, Q81Stage<PRE> &st) {
    const int nblk = K / 32;
    const int total = ncols * nblk;
    const int quarter = threadIdx.x & 3;
    constexpr int step = NT / 4;
#pragma unroll
    for (int j = 0; j < PRE; ++j) {
        if (j >= 4 && j * step >= total) break;  // uniform, as above
        const int qb = min((int)(threadIdx.x >> 2) + j * step, total - 1);  // unconditional, as above
        const int c = (int)fastdiv((uint32_t)qb, fd);
        const uint8_t *blk = y + ((int64_t)c * stride_col_y + (qb - c * nblk)) * kQ81Bytes;
        st.w[j][0] = *reinterpret_cast<const uint32_t *>(blk + 4 + quarter * 8);
        st.w[j][1] = *reinterpret_cast<const uint32_t *>(blk + 8 + quarter * 8);
        st.ds[j] = *reinterpret_cast<const uint32_t *>(blk);
    }
}

template <int LAYOUT>
__device__ __forceinline__ void store_q81_part(uint32_t w0, uint32_t w1, uint32_t ds, int quarter,
                                               int qcol, int c, int b, int qb, int total, int nblk,
                                               int8_t *q8s, void *aux, int32_t *sq_out = nullptr) {
    int hsum, fsum;
    block_sums<4>(__builtin_amdgcn_sdot4((int)w0, 0x01010101, __builtin_amdgcn_sdot4((int)w1, 0x01010101, 0, false),
                                         false),
                  hsum, fsum);
    *reinterpret_cast<uint2 *>(q8s + q8_offset<LAYOUT>(c, qcol, nblk >> 3, b, 2 * quarter)) = make_uint2(w0, w1);
    if ((quarter & 1) == 0)
        store_aux<LAYOUT>(aux, total, nblk, c, b, qb, quarter >> 1, half_bits_to_float(ds), fsum, hsum);
    if (sq_out && quarter == 0) sq_out[qb] = fsum;
}

template <int LAYOUT, int NT, int CHUNK = kFinishRounds, int PRE>
__device__ __forceinline__ void stage_q81_finish(const uint8_t *__restrict__ y, int64_t stride_col_y,
                                                 int K, int ncols, const FastDiv &fd,
                                                 const Q81Stage<PRE> &st, int qcol, int8_t *q8s,
                                                 void *aux, int32_t *sq_out = nullptr) {
    const int nblk = K / 32;
    const int total = ncols * nblk;
    const int quarter = threadIdx.x & 3;
    constexpr int step = NT / 4;
#pragma unroll
    for (int j = 0; j < PRE; ++j) {
        const int qb = (threadIdx.x >> 2) + j * step;
        if (qb < total) {
            const int c = (int)fastdiv((uint32_t)qb, fd);
            store_q81_part<LAYOUT>(st.w[j][0], st.w[j][1], st.ds[j], quarter, qcol, c, qb - c * nblk, qb,
                                   total, nblk, q8s, aux, sq_out);
        }
    }
    // further rounds CHUNK at a time, loads first, as in stage_f32_finish
    constexpr int kChunk = CHUNK;
    for (int q0 = (threadIdx.x >> 2) + PRE * step; q0 < total; q0 += kChunk * step) {
        const int q0w = __builtin_amdgcn_readfirstlane(q0);
        uint32_t w[kChunk][2], ds[kChunk];
#pragma unroll
        for (int j = 0; j < kChunk; ++j) {
            if (j > 0 && q0w + j * step >= total) break;
            const int qb = min(q0 + j * step, total - 1);
            const int c = (int)fastdiv((uint32_t)qb, fd);
            const uint8_t *blk = y + ((int64_t)c * stride_col_y + (qb - c * nblk)) * kQ81Bytes;
            w[j][0] = *reinterpret_cast<const uint32_t *>(blk + 4 + quarter * 8);
            w[j][1] = *reinterpret_cast<const uint32_t *>(blk + 8 + quarter * 8);
            ds[j] = *reinterpret_cast<const uint32_t *>(blk);
        }
#pragma unroll
        for (int j = 0; j < kChunk; ++j) {
            const int qb = q0 + j * step;
            if (qb < total) {
                const int c = (int)fastdiv((uint32_t)qb, fd);
                store_q81_part<LAYOUT>(w[j][0], w[j][1], ds[j], quarter, qcol, c, qb - c * nblk, qb, total, nblk,
                                       q8s, aux, sq_out);
            }
        }
    }
}

// One-call form (issue + finish) for kernels with no loads to overlap.
template <int LAYOUT, int NT>
__device__ __forceinline__ void stage_from_q8_1(const uint8_t *__restrict__ y, int64_t stride_col_y,
                                                int K, int ncols, const FastDiv &fd, int qcol,
                                                int8_t *q8s, void *aux) {
    Q81Stage<4> st;
    stage_q81_issue<NT>(y, stride_col_y, K, ncols, fd, st);
    stage_q81_finish<LAYOUT, NT>(y, stride_col_y, K, ncols, fd, st, qcol, q8s, aux);
}

}  // namespace q4k
