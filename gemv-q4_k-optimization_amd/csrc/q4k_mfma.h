// q4k_mfma.h -- the Q4_K GEMV for several activation columns on the matrix
// cores: v_mfma_i32_16x16x64_i8 forms the int32 sub-block sums of a tile of
// 16 weight rows against up to 8 columns, the VALU only unpacks nibbles and
// applies the per-(row, column, sub-block) scales.
//
// Operands of one MFMA (chunk jj of super-block kb: qs bytes [32jj, 32jj+32)
// of each row, i.e. sub-blocks 2jj (low nibbles) and 2jj+1 (high nibbles)).
// The instruction's 64 k-slots are lane group g = lane/16, byte t; A row i
// and B column j of lane l are l % 16, and D element v of lane l is
// D[4(l/16) + v][l % 16] (checked on the device).  Here
//   k-slots   g = 0, 1: sub-block 2jj, values 16g + t; g = 2, 3: sub-block
//             2jj+1, values 16(g-2) + t;
//   A row i   activation column i % 8 for sub-block 2jj (i < 8) or 2jj+1
//             (i >= 8): its q8 in the slots of its own sub-block, zeros in
//             the other two lane groups (read from a zero area of LDS);
//   B col r   weight row r of the tile: the nibbles of its 32 qs bytes;
//   D         D[i][r] = the int32 sum S_qq of row r, column i % 8, sub-block
//             2jj + i/8: every output is one the product needs.
// So lane l ends up with one weight row (l % 16), one sub-block parity
// (l / 32) and four columns (4((l/16) & 1) + v): the row's scale and min
// are unpacked once per lane and used for four columns.
//
// Work split: tiles of 16 rows, split evenly over the workgroups (one per
// CU, 8 or 16 waves).  The waves of a workgroup form 8/KS groups of KS waves; in
// each round every group takes one tile and its KS waves take equal shares
// of the tile's super-blocks.  At the end of a round each wave leaves its
// partial results in LDS and, after a barrier, the workgroup combines the KS
// partials of each tile and writes the outputs.
//
// A operand from the Q8_1 buffer (GA variants, pre-quantised activation):
// instead of an LDS copy of the whole activation, each item's activation --
// super-block kb of the NC columns, 8 AoS block_q8_1 of 36 bytes (288
// contiguous bytes) per column -- arrives with the item's weights, in three
// 64-lane x 16-byte loads (chunk c = lane + 64i is bytes [16 (c % 18), +16)
// of column c / 18), goes to a second LDS slot of the wave as it lies in
// memory, and the MFMA lanes read their A operands from there.  The LDS
// holds only the d8 of every (block, column) besides, so the length of the
// rows is not bounded by the LDS (eight 14336-value columns staged would
// take 170 KB of its 160).  The sum of each block's q8, which the staged layout keeps
// beside d8, comes from a second MFMA of the same A operand against a B of
// ones (D[i][r] = the sum of A row i); d8 * that sum is the staged product,
// so both variants compute the same bits.
//
// Summation order: a row's super-blocks form S = min(8, 2^floor(log2 nb))
// segments [s nb/S, (s+1) nb/S), each summed in order; the segment sums are
// combined in a fixed balanced binary tree.  A wave owns an aligned run of
// S/KS segments and forms that subtree itself; the reduction completes the
// tree across the KS waves.  So the result depends on K alone -- not on the
// number of rows, the tiles per workgroup or KS -- and row slices of a
// product reproduce it bit for bit.
#pragma once

#include <hip/hip_runtime.h>

#include "q4k_tile.h"

namespace q4k {

typedef int i32x4 __attribute__((ext_vector_type(4)));

constexpr int kMfmaRows = 16;   // weight rows per tile
constexpr int kMfmaCols = 8;    // activation columns of one MFMA (padded)
constexpr int kMfmaMaxSegs = 8; // summation segments of a row, at most
constexpr int kMfmaZeroBytes = 512;
// per-wave partial results of a round: 32 lanes x 4 columns, two buffers
__host__ __device__ constexpr int mfma_part_bytes(int waves) { return 2 * waves * 32 * 16; }

// LDS layout (bytes from the start): NC q8 columns of qcol = K + 16 bytes
// (the 16-byte skew puts the eight columns' reads of one lane octet in
// different banks), then the (d8, d8*sum q8) pairs of every 32-value block
// for 8 columns ([block][column], float2), the zero area, the partials and
// one weight slot per wave.
__host__ __device__ constexpr int mfma_qcol(int K) { return K + 16; }
__host__ __device__ constexpr int mfma_dk_off(int K, int nc) { return nc * mfma_qcol(K); }
__host__ __device__ constexpr int mfma_zero_off(int K, int nc) { return mfma_dk_off(K, nc) + (K / 32) * kMfmaCols * 8; }
__host__ __device__ constexpr int mfma_part_off(int K, int nc) { return mfma_zero_off(K, nc) + kMfmaZeroBytes; }
// Weight staging: an item (16 rows x one super-block, 2304 bytes) arrives
// with three contiguous 64-lane x 16-byte loads (chunk c = lane + 64i is
// bytes [16 (c % 9), +16) of row c / 9; loads that each touch one or two
// rows stream as fast as the tile kernel's, where loads touching all 16 rows
// reached half that), goes to the wave's LDS slot as it lies in memory (row
// pitch 144 bytes = 36 dwords: the 16-byte reads of 16 rows at one offset
// fall in distinct banks, and the writes are one contiguous run) and the
// MFMA operands are read from there.
constexpr int kMfmaSlotPitch = kBlockBytes;
constexpr int kMfmaSlotBytes = kMfmaRows * kMfmaSlotPitch;
constexpr int kMfmaChunks = kMfmaRows * kBlockBytes / 16;  // 144
__host__ __device__ constexpr int mfma_slot_off(int K, int nc, int waves) {
    return mfma_part_off(K, nc) + mfma_part_bytes(waves);
}
__host__ __device__ constexpr int mfma_lds_bytes(int K, int nc, int waves) {
    return mfma_slot_off(K, nc, waves) + waves * kMfmaSlotBytes;
}
// GA variants: d8 of every (block, column) ([block][8 columns], float: K
// bytes), a zero area, the partials, one weight slot and one activation
// slot (8 columns x 288 bytes) per wave.
constexpr int kGaZeroBytes = 256;
constexpr int kGaSuperBytes = 8 * kQ81Bytes;  // one super-block of one Q8_1 column
constexpr int kGaSlotBytes = kMfmaCols * kGaSuperBytes;
__host__ __device__ constexpr int mfma_ga_zero_off(int K) { return K; }
__host__ __device__ constexpr int mfma_ga_part_off(int K) { return K + kGaZeroBytes; }
__host__ __device__ constexpr int mfma_ga_slot_off(int K, int waves) { return mfma_ga_part_off(K) + mfma_part_bytes(waves); }
__host__ __device__ constexpr int mfma_ga_aslot_off(int K, int waves) {
    return mfma_ga_slot_off(K, waves) + waves * kMfmaSlotBytes;
}
__host__ __device__ constexpr int mfma_ga_lds_bytes(int K, int waves) {
    return mfma_ga_aslot_off(K, waves) + waves * kGaSlotBytes;
}

// One super-block's weights as the MFMA lane needs them: the header of row
// l % 16 and the 16 qs bytes of each chunk jj the lane's lane group reads.
struct MfmaRegs {
    u32x4 h;
    u32x4 q[4];
};

// One item in flight: the lane's three 16-byte chunks of the contiguous loads.
struct MfmaLoad {
    u32x4 v[3];
};

// Per-lane constants.
struct MfmaLane {
    int lane;
    int wrow;         // weight row in the tile (B column, D column)
    int half;         // which 16 bytes of a chunk the lane loads (lane group & 1)
    uint32_t nshift;  // 0: low nibbles (lane groups 0, 1), 4: high nibbles
    int hid;          // D: sub-block parity of the lane's outputs (lane / 32)
    int c0;           // D: first of the lane's four columns
    int a_off;        // LDS byte offset of the lane's A operand for super-block 0
    int a_inc;        // per super-block: 256 (data lanes) or 0 (zero lanes)
    int dk_off;       // LDS byte offset of its (d8, d8*sum) pairs for super-block 0
    uint32_t selx, sely;  // byte selectors of its scales (sub-blocks hid, 2+hid, ...)
    uint32_t g_off[3];    // its chunks of an item: byte offsets from the item's first row
    int s_off[3];         // and in the wave's slot
    uint32_t ya_off[3];   // GA: its chunks of an item's activation, byte offsets from the item's first block
    int ar_off;           // GA: its A operand of chunk 0 in the activation slot (data lanes)
    int ar_step;          // GA: per chunk (2 blocks) in the slot: 72 (data lanes) or 0 (zero lanes)
    bool a_data;          // GA: the lane carries activation (else it reads the zero area)
};

template <int NC>
__device__ __forceinline__ MfmaLane mfma_lane(int K, int64_t stride_col_y = 0) {
    MfmaLane m;
    const int l = threadIdx.x & (kWave - 1);
    const int g = l >> 4;
    m.lane = l;
    m.wrow = l & 15;
    m.half = g & 1;
    m.nshift = (uint32_t)(g >> 1) * 4u;
    m.hid = l >> 5;
    m.c0 = 4 * (g & 1);
    // A: row i = l % 16 -> column i % 8, sub-block parity i / 8; it holds
    // data in the lane groups of its own sub-block, zeros elsewhere
    const int ca = l & 7, hia = (l >> 3) & 1;
    const bool data = (g >> 1) == hia && ca < NC;
    m.a_off = data ? ca * mfma_qcol(K) + 32 * hia + 16 * (g & 1) : mfma_zero_off(K, NC) + 16 * (l & 7);
    m.a_inc = data ? kQK : 0;
    m.dk_off = mfma_dk_off(K, NC) + (m.hid * kMfmaCols + m.c0) * 8;
    const uint32_t h = (uint32_t)m.hid;
    m.selx = h | ((h + 2u) << 8) | ((h + 4u) << 16) | ((h + 6u) << 24);
    m.sely = h | ((h + 2u) << 8) | (h << 16) | ((h + 2u) << 24);
    // GA: chunk c = l + 64i of an item's activation is bytes [16 (c % 18),
    // +16) of column c / 18 (kOOB past the NC columns); the A operand of
    // chunk jj is q8 bytes 16 (g & 1) .. of block 2jj + hia of column ca
#pragma unroll
    for (int i = 0; i < 3; ++i) {
        const int c = l + 64 * i, col = c / 18, o = c - 18 * col;
        m.ya_off[i] = col < NC ? (uint32_t)(col * stride_col_y) * (uint32_t)kQ81Bytes + 16u * (uint32_t)o : kOOB;
    }
    m.a_data = data;
    m.ar_off = ca * kGaSuperBytes + hia * kQ81Bytes + 4 + 16 * (g & 1);
    m.ar_step = data ? 2 * kQ81Bytes : 0;
    return m;
}

// The lane's chunk offsets of an item (rows row_stride bytes apart); chunks
// past the item's 144 get no offset (their loads read zeros, nothing is
// written).
__device__ __forceinline__ void mfma_chunks(MfmaLane &m, int64_t row_stride) {
#pragma unroll
    for (int i = 0; i < 3; ++i) {
        const int c = m.lane + 64 * i, r = c / 9, o = c - 9 * (c / 9);
        m.g_off[i] = c < kMfmaChunks ? (uint32_t)(r * row_stride) + 16u * (uint32_t)o : kOOB;
        m.s_off[i] = r * kMfmaSlotPitch + 16 * o;
    }
}

// Loads one item: one super-block of 16 rows whose first row's block
// starts at byte offset off of the workgroup's buffer, or zeros when off is
// kOOB.  The sums need no selects: the buffer is under 2^31 bytes and off
// under 2^31 or kOOB, so off + kOOB and kOOB + g_off (g_off < 2^31) fall
// outside it and read zeros; kOOB + kOOB wraps to 0 and reads bytes, but
// only for chunks past the item's 144, which are never written to the slot.
__device__ __forceinline__ void mfma_load(__amdgpu_buffer_rsrc_t rs, uint32_t off, const MfmaLane &ln,
                                          MfmaLoad &w) {
#pragma unroll
    for (int i = 0; i < 3; ++i) w.v[i] = load16(rs, off + ln.g_off[i]);
}

// Writes an item to the wave's slot and reads the lane's operands back.
// The lanes read bytes other lanes wrote: the wait and the compiler barrier
// keep the reads behind the writes.
__device__ __forceinline__ MfmaRegs mfma_stage(uint8_t *slot, const MfmaLane &ln, const MfmaLoad &w) {
    asm volatile("" ::: "memory");
#pragma unroll
    for (int i = 0; i < 3; ++i)
        if (i < 2 || ln.lane + 128 < kMfmaChunks) *reinterpret_cast<u32x4 *>(slot + ln.s_off[i]) = w.v[i];
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    MfmaRegs r;
    const uint8_t *row = slot + ln.wrow * kMfmaSlotPitch;
    r.h = *reinterpret_cast<const u32x4 *>(row);
#pragma unroll
    for (int jj = 0; jj < 4; ++jj) r.q[jj] = *reinterpret_cast<const u32x4 *>(row + 16 + 16 * ln.half + 32 * jj);
    return r;
}

// The lane's (sc, m) of sub-blocks hid + 2jj, jj = 0..3: low = {sc(hid),
// sc(2+hid), m(hid), m(2+hid)}, split = the same for 4+hid, 6+hid (the
// 4+2-bit fields of get_scale_min_k4).
__device__ __forceinline__ void mfma_scales(u32x4 h, const MfmaLane &ln, uint32_t &low, uint32_t &split) {
    const uint32_t x = __builtin_amdgcn_perm(h[2], h[1], ln.selx);
    const uint32_t y = __builtin_amdgcn_perm(h[3], h[3], ln.sely);
    low = x & 0x3f3f3f3fu;
    split = (y & 0x00000f0fu) | ((y >> 4) & 0x0f0f0000u) | ((x >> 2) & 0x30303030u);
}

// One item: four MFMAs and the scaling of their outputs into acc (the
// lane's row, four columns).  SUMS: also stores the int32 sums.
template <int NC, bool SUMS>
__device__ __forceinline__ void mfma_item(const GemvParams &p, const MfmaLane &ln, const uint8_t *lds, int kb,
                                          const MfmaRegs &w, float (&acc)[4], int row, bool row_ok) {
    const uint8_t *pa = lds + ln.a_off + ln.a_inc * kb;
    const uint8_t *pk = lds + ln.dk_off + kb * (8 * kMfmaCols * 8);
    // the four products first (independent), then their scaling
    i32x4 s[4];
#pragma unroll
    for (int jj = 0; jj < 4; ++jj) {
        const u32x4 av = *reinterpret_cast<const u32x4 *>(pa + 64 * jj);
        u32x4 bv;
#pragma unroll
        for (int e = 0; e < 4; ++e) bv[e] = (w.q[jj][e] >> ln.nshift) & 0x0f0f0f0fu;
        s[jj] = __builtin_amdgcn_mfma_i32_16x16x64_i8(__builtin_bit_cast(i32x4, av), __builtin_bit_cast(i32x4, bv),
                                                      i32x4{0, 0, 0, 0}, 0, 0, 0);
    }
    uint32_t low, split;
    mfma_scales(w.h, ln, low, split);
    const float d = half_bits_to_float(w.h[0]), dmin = half_bits_to_float(w.h[0] >> 16);
    float t[4] = {0.0f, 0.0f, 0.0f, 0.0f}, u[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int jj = 0; jj < 4; ++jj) {
        // (d8, d8*sum q8) of the lane's four columns, sub-block 2jj + hid
        const float4 k01 = *reinterpret_cast<const float4 *>(pk + 2 * kMfmaCols * 8 * jj);
        const float4 k23 = *reinterpret_cast<const float4 *>(pk + 2 * kMfmaCols * 8 * jj + 16);
        const uint32_t scm = jj < 2 ? low : split;
        const int sc = (int)((scm >> (8 * (jj & 1))) & 0xffu);
        const float mf = (float)((scm >> (16 + 8 * (jj & 1))) & 0xffu);
        const float d8[4] = {k01.x, k01.z, k23.x, k23.z};
        const float km[4] = {k01.y, k01.w, k23.y, k23.w};
#pragma unroll
        for (int v = 0; v < 4; ++v) {
            // |s| <= 32*15*127 and sc <= 63: the 24-bit product is exact in f32
            t[v] = __builtin_fmaf(d8[v], (float)__mul24(s[jj][v], sc), t[v]);
            u[v] = __builtin_fmaf(km[v], mf, u[v]);
        }
        if constexpr (SUMS) {
            if (row_ok) {
#pragma unroll
                for (int v = 0; v < 4; ++v)
                    if (ln.c0 + v < NC)
                        p.sums[((int64_t)(ln.c0 + v) * p.M + row) * (p.K / 32) + kb * 8 + 2 * jj + ln.hid] = s[jj][v];
            }
        }
    }
#pragma unroll
    for (int v = 0; v < 4; ++v) {
        acc[v] = __builtin_fmaf(d, t[v], acc[v]);
        acc[v] = __builtin_fmaf(-dmin, u[v], acc[v]);
    }
}

// GA: the lane's chunks of the activation of super-block kb (zeros past the
// NC columns: kOOB + 288 kb stays outside the buffer).
__device__ __forceinline__ void mfma_load_act(__amdgpu_buffer_rsrc_t ry, const MfmaLane &ln, int kb, MfmaLoad &a) {
    const uint32_t o = (uint32_t)kb * (uint32_t)kGaSuperBytes;
#pragma unroll
    for (int i = 0; i < 3; ++i) a.v[i] = load16(ry, o + ln.ya_off[i]);
}

// GA: writes an item's weights and activation to the wave's two slots and
// reads the lane's weight operands back (the A operands are read in
// mfma_item_ga); as mfma_stage.
__device__ __forceinline__ MfmaRegs mfma_stage_ga(uint8_t *slot, uint8_t *aslot, const MfmaLane &ln,
                                                  const MfmaLoad &w, const MfmaLoad &a, int nc) {
    asm volatile("" ::: "memory");
#pragma unroll
    for (int i = 0; i < 3; ++i) {
        if (i < 2 || ln.lane + 128 < kMfmaChunks) *reinterpret_cast<u32x4 *>(slot + ln.s_off[i]) = w.v[i];
        if (ln.lane + 64 * i < 18 * nc) *reinterpret_cast<u32x4 *>(aslot + 16 * (ln.lane + 64 * i)) = a.v[i];
    }
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    MfmaRegs r;
    const uint8_t *row = slot + ln.wrow * kMfmaSlotPitch;
    r.h = *reinterpret_cast<const u32x4 *>(row);
#pragma unroll
    for (int jj = 0; jj < 4; ++jj) r.q[jj] = *reinterpret_cast<const u32x4 *>(row + 16 + 16 * ln.half + 32 * jj);
    return r;
}

// mfma_item with the A operand in registers (GA): d8 from the LDS table,
// d8 * sum q8 from the ones product.  SQ: also stores the block sums of q8
// (lanes of weight row 0 hold them for their four columns).
// pa: the lane's A operand of chunk 0 (in the activation slot, 4-byte
// aligned, or the zero area), pa + ar_step * jj that of chunk jj.
template <int NC, bool SUMS>
__device__ __forceinline__ void mfma_item_ga(const GemvParams &p, const MfmaLane &ln, const uint8_t *lds, int kb,
                                             const MfmaRegs &w, const uint8_t *pa, float (&acc)[4], int row,
                                             bool row_ok, bool sq_ok) {
    const float *pd = reinterpret_cast<const float *>(lds) + (kb * 8 + ln.hid) * kMfmaCols + ln.c0;
    i32x4 s[4], z[4];
#pragma unroll
    for (int jj = 0; jj < 4; ++jj) {
        u32x4 bv;
#pragma unroll
        for (int e = 0; e < 4; ++e) bv[e] = (w.q[jj][e] >> ln.nshift) & 0x0f0f0f0fu;
        const uint32_t *q = reinterpret_cast<const uint32_t *>(pa + ln.ar_step * jj);
        const i32x4 av = i32x4{(int)q[0], (int)q[1], (int)q[2], (int)q[3]};
        s[jj] = __builtin_amdgcn_mfma_i32_16x16x64_i8(av, __builtin_bit_cast(i32x4, bv), i32x4{0, 0, 0, 0}, 0, 0, 0);
        z[jj] = __builtin_amdgcn_mfma_i32_16x16x64_i8(av, i32x4{0x01010101, 0x01010101, 0x01010101, 0x01010101},
                                                      i32x4{0, 0, 0, 0}, 0, 0, 0);
    }
    uint32_t low, split;
    mfma_scales(w.h, ln, low, split);
    const float d = half_bits_to_float(w.h[0]), dmin = half_bits_to_float(w.h[0] >> 16);
    float t[4] = {0.0f, 0.0f, 0.0f, 0.0f}, u[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int jj = 0; jj < 4; ++jj) {
        // d8 of the lane's four columns, sub-block 2jj + hid
        const float4 d4 = *reinterpret_cast<const float4 *>(pd + 2 * kMfmaCols * jj);
        const uint32_t scm = jj < 2 ? low : split;
        const int sc = (int)((scm >> (8 * (jj & 1))) & 0xffu);
        const float mf = (float)((scm >> (16 + 8 * (jj & 1))) & 0xffu);
        const float d8[4] = {d4.x, d4.y, d4.z, d4.w};
#pragma unroll
        for (int v = 0; v < 4; ++v) {
            const float km = d8[v] * (float)z[jj][v];
            t[v] = __builtin_fmaf(d8[v], (float)__mul24(s[jj][v], sc), t[v]);
            u[v] = __builtin_fmaf(km, mf, u[v]);
        }
        if constexpr (SUMS) {
            if (row_ok) {
#pragma unroll
                for (int v = 0; v < 4; ++v)
                    if (ln.c0 + v < NC)
                        p.sums[((int64_t)(ln.c0 + v) * p.M + row) * (p.K / 32) + kb * 8 + 2 * jj + ln.hid] = s[jj][v];
            }
            if (sq_ok && ln.wrow == 0) {
#pragma unroll
                for (int v = 0; v < 4; ++v)
                    if (ln.c0 + v < NC) p.sq[(ln.c0 + v) * (p.K / 32) + kb * 8 + 2 * jj + ln.hid] = z[jj][v];
            }
        }
    }
#pragma unroll
    for (int v = 0; v < 4; ++v) {
        acc[v] = __builtin_fmaf(d, t[v], acc[v]);
        acc[v] = __builtin_fmaf(-dmin, u[v], acc[v]);
    }
}

// Adds segment value v (the sum of one segment, local index t in the wave's
// run) into the wave's subtree: l1, l2, l4 hold the pending left subtrees of
// 1, 2 and 4 segments; returns the subtree that ends at t.
__device__ __forceinline__ void mfma_tree_push(int t, float (&v)[4], float (&l1)[4], float (&l2)[4],
                                               float (&l4)[4]) {
    if (t & 1) {
#pragma unroll
        for (int k = 0; k < 4; ++k) v[k] = l1[k] + v[k];
        if (t & 2) {
#pragma unroll
            for (int k = 0; k < 4; ++k) v[k] = l2[k] + v[k];
            if (t & 4) {
#pragma unroll
                for (int k = 0; k < 4; ++k) v[k] = l4[k] + v[k];
            } else {
#pragma unroll
                for (int k = 0; k < 4; ++k) l4[k] = v[k];
            }
        } else {
#pragma unroll
            for (int k = 0; k < 4; ++k) l2[k] = v[k];
        }
    } else {
#pragma unroll
        for (int k = 0; k < 4; ++k) l1[k] = v[k];
    }
}

// A wave's position in its items: round r (tile group + ngroups * r) and
// super-block kb of the tile.
struct MfmaPos {
    int r, kb;
};

// The kernel.  rows_base / rows_extra are the tile split: each workgroup
// owns rows_base tiles of 16 rows, the first rows_extra one more;
// p.rpw: KS, the waves that share one tile (1, 2, 4 or 8, at most S);
// p.ntiles: S, the segments of a row.  GA: the A operand from the Q8_1
// buffer p.y (which the GA variants require).  NIF: items in flight per
// wave (2, or 4 in the GA variants).
template <int NC, int WAVES, bool SUMS = false, bool GA = false, int NIF = 2>
__global__ __launch_bounds__(kWave *WAVES) void gemv_q4k_mfma_kernel(Q4K_GEMV_KERNEL_ARGS) {
    static_assert(NC >= 1 && NC <= kMfmaCols, "up to 8 columns");
    static_assert(WAVES == 8 || WAVES == 16, "8 or 16 waves");
    constexpr int NT = kWave * WAVES;
    int32_t *const sq_out = SUMS ? p.sq : nullptr;
    p = with_head(p, Q4K_GEMV_HEAD_VALUES);
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    int8_t *q8s = reinterpret_cast<int8_t *>(lds);
    float2 *dks = reinterpret_cast<float2 *>(lds + mfma_dk_off(p.K, NC));

    MfmaLane ln = mfma_lane<NC>(p.K, p.stride_col_y);
    mfma_chunks(ln, p.row_stride);
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int KS = p.rpw, S = p.ntiles;
    const int group = wave / KS, ks = wave - group * KS;
    const int ngroups = WAVES / KS;
    const int segs = S / KS, seg0 = ks * segs;  // the wave's run of segments
    // this workgroup's tiles and this wave's super-blocks of each
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

    constexpr int kLPB = stage_lpb(NC);
    constexpr int kPreR = GA ? 1 : pre_rounds(NC, NT);
    ActStage<kLPB, kPreR> xs;
    Q81Stage<kPreR> ys;
    if constexpr (!GA) {
        if (p.x) stage_f32_issue<kLPB, NT>(p.x, p.ldx, p.K, NC, p.vec_ok != 0, p.nblk32, xs);
        else stage_q81_issue<NT>(p.y, p.stride_col_y, p.K, NC, p.nblk32, ys);
        __syncthreads();  // all activation loads of this CU are queued first
    }
    // GA: the Q8_1 columns as one buffer (columns stride_col_y blocks apart;
    // the host keeps it under 2^31 bytes)
    const __amdgpu_buffer_rsrc_t ry =
        make_rsrc(p.y, GA ? (uint32_t)((int64_t)(NC - 1) * p.stride_col_y * kQ81Bytes + (p.K / 32) * kQ81Bytes) : 0u);

    // items in order: rounds, and super-blocks kb0..kb1-1 of each; loads of
    // positions past the wave's last round or the workgroup's tiles read zeros
    auto next = [&](MfmaPos q) -> MfmaPos { return q.kb + 1 < kb1 ? MfmaPos{q.r, q.kb + 1} : MfmaPos{q.r + 1, kb0}; };
    auto item_off = [&](MfmaPos q) -> uint32_t {
        const int tile = group + ngroups * q.r;
        if (q.r >= rounds || tile >= nt) return kOOB;
        return (uint32_t)(tile * kMfmaRows * p.row_stride) + (uint32_t)q.kb * kBlockBytes;
    };
    static_assert(NIF == 2 || (GA && NIF == 4), "items in flight");
    MfmaPos cur{0, kb0};
    MfmaPos ahead = cur;
    MfmaLoad w[NIF];
    MfmaLoad av[GA ? NIF : 1];
#pragma unroll
    for (int k = 0; k < NIF; ++k) {
        mfma_load(rs, item_off(ahead), ln, w[k]);
        if constexpr (GA) mfma_load_act(ry, ln, ahead.kb, av[GA ? k : 0]);
        ahead = next(ahead);
    }

    if constexpr (GA) {
        // d8 of every (block, column); zeros for the padding columns (their
        // outputs are dropped; zeros keep them finite)
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
            reinterpret_cast<u32x4 *>(lds + mfma_ga_zero_off(p.K))[threadIdx.x] = u32x4{0u, 0u, 0u, 0u};
    } else {
        if (p.x)
            stage_f32_finish<kLayoutMfma, kLPB, NT>(p.x, p.ldx, p.K, NC, p.vec_ok != 0, p.nblk32, xs,
                                                    mfma_qcol(p.K), q8s, dks, sq_out);
        else
            stage_q81_finish<kLayoutMfma, NT>(p.y, p.stride_col_y, p.K, NC, p.nblk32, ys, mfma_qcol(p.K), q8s,
                                              dks, sq_out);
        // the zero area of the A operand, and the pairs of the padding columns
        // (their outputs are dropped; zeros keep them finite)
        if (threadIdx.x < kMfmaZeroBytes / 16)
            reinterpret_cast<u32x4 *>(lds + mfma_zero_off(p.K, NC))[threadIdx.x] = u32x4{0u, 0u, 0u, 0u};
        if constexpr (NC < kMfmaCols) {
            for (int q = (int)threadIdx.x; q < (p.K / 32) * (kMfmaCols - NC); q += NT) {
                const int blk = q / (kMfmaCols - NC), c = NC + q - blk * (kMfmaCols - NC);
                dks[blk * kMfmaCols + c] = make_float2(0.0f, 0.0f);
            }
        }
    }
    __syncthreads();

    float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    float l1[4] = {0.0f, 0.0f, 0.0f, 0.0f}, l2[4] = {0.0f, 0.0f, 0.0f, 0.0f}, l4[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    float *part = reinterpret_cast<float *>(lds + (GA ? mfma_ga_part_off(p.K) : mfma_part_off(p.K, NC)));
    uint8_t *slot =
        lds + (GA ? mfma_ga_slot_off(p.K, WAVES) : mfma_slot_off(p.K, NC, WAVES)) + wave * kMfmaSlotBytes;
    uint8_t *aslot = lds + mfma_ga_aslot_off(p.K, WAVES) + wave * kGaSlotBytes;  // GA only
    const uint8_t *pa = GA && ln.a_data ? aslot + ln.ar_off : lds + mfma_ga_zero_off(p.K);
    int t = 0;                            // local segment of the current item
    int seg_end = (seg0 + 1) * p.nb / S;  // its end (super-block)
    // items go NIF at a time (registers k hold item it); a count that is
    // not a multiple ends with items past the wave's, whose zeros add nothing
    for (int it = 0; it < items;) {
#pragma unroll
        for (int k = 0; k < NIF; ++k, ++it) {
            const int tile = group + ngroups * cur.r;
            const int row = row0 + tile * kMfmaRows + ln.wrow;
            if constexpr (GA) {
                const MfmaRegs wr = mfma_stage_ga(slot, aslot, ln, w[k], av[GA ? k : 0], NC);
                mfma_load(rs, item_off(ahead), ln, w[k]);
                mfma_load_act(ry, ln, ahead.kb, av[GA ? k : 0]);
                // sq: the group of waves holding tile 0 of workgroup 0 covers
                // every super-block once
                mfma_item_ga<NC, SUMS>(p, ln, lds, cur.kb, wr, pa, acc, row, SUMS && it < items && tile < nt && row < p.M,
                                       SUMS && blockIdx.x == 0 && group == 0 && cur.r == 0 && it < items);
            } else {
                const MfmaRegs wr = mfma_stage(slot, ln, w[k]);
                mfma_load(rs, item_off(ahead), ln, w[k]);
                mfma_item<NC, SUMS>(p, ln, lds, cur.kb, wr, acc, row, SUMS && it < items && tile < nt && row < p.M);
            }
            ahead = next(ahead);
            const MfmaPos done = cur;
            cur = next(cur);
            if (it < items && done.kb + 1 == seg_end) {
                // segment end: its value is the sum of the two sub-block
                // parities of each (row, column), in lanes l and l + 32
                float v[4];
#pragma unroll
                for (int c = 0; c < 4; ++c) {
                    float hi = acc[c];
                    permlane32_swap(acc[c], hi);
                    v[c] = acc[c] + hi;
                    acc[c] = 0.0f;
                }
                mfma_tree_push(t, v, l1, l2, l4);
                ++t;
                if (t < segs) {
                    seg_end = (seg0 + t + 1) * p.nb / S;
                    continue;
                }
                // round end: v is the wave's subtree of the tile
                t = 0;
                seg_end = (seg0 + 1) * p.nb / S;
                const int buf = done.r & 1;
                if (ln.lane < 32)
                    *reinterpret_cast<float4 *>(part + ((buf * WAVES + wave) * 32 + ln.lane) * 4) =
                        make_float4(v[0], v[1], v[2], v[3]);
                __syncthreads();
                // outputs of this round: tile group q, column c, row rr;
                // consecutive threads write consecutive rows of a column.
                // The KS subtrees combine in the same balanced tree.
                for (int o = (int)threadIdx.x; o < ngroups * kMfmaRows * kMfmaCols; o += NT) {
                    const int rr = o & 15, c = (o >> 4) & 7, q = o >> 7;
                    const int otile = q + ngroups * done.r;
                    const int orow = row0 + otile * kMfmaRows + rr;
                    if (c < NC && otile < nt && orow < p.M) {
                        const int l32 = rr + 16 * (c >> 2);
                        const float *src = part + ((buf * WAVES + q * KS) * 32 + l32) * 4 + (c & 3);
                        float pv[kMfmaMaxSegs];
#pragma unroll
                        for (int j = 0; j < kMfmaMaxSegs; ++j) pv[j] = j < KS ? src[j * 32 * 4] : 0.0f;
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
