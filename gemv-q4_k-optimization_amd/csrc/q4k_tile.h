// q4k_tile.h -- pieces shared by the gfx950 tile kernels of the K-quant
// GEMVs (Q4_K and Q6_K): launch parameters, the split of a product's rows
// over workgroups and waves, the walk over (row tile, group) steps and the
// per-wave result ring.
#pragma once

#include "q4k_device.h"

namespace q4k {

struct GemvParams {
    const uint8_t *w;        // weight rows (Q4_K)
    int64_t row_stride;      // bytes between rows
    const float *x;          // F32 activation (staged with quantisation) or null
    int64_t ldx;             // floats between activation columns
    const uint8_t *y;        // AoS Q8_1 activation when x is null
    int64_t stride_col_y;    // blocks between Q8_1 columns
    float *dst;
    int64_t ld_dst;          // floats between output columns
    int M;                   // rows
    int K;                   // values per row
    int nb;                  // super-blocks per row (K/256)
    int G;                   // groups of 16 super-blocks per row
    int qcol;                // LDS bytes between the staged q8 columns
    int ntiles;              // ceil(M / R) (ceil(M / rpw) for the block-per-lane kernel)
    int vec_ok;              // F32 activation 16-B aligned with ldx % 4 == 0
    int rpw;                 // block-per-lane kernel: rows per wave pass (64/nb or 1)
    int rows_base;           // tile kernel: each workgroup owns rows_base rows,
    int rows_extra;          //   the first rows_extra workgroups one more
    int ring_off;            // tile kernel: LDS byte offset of the per-wave result rings
    FastDiv nblk32;          // division by K/32 (Q8_1 blocks per column)
};

// The GEMV kernels take the fields their first memory requests need as
// leading scalar arguments (16 dwords), ahead of the GemvParams block, so
// they arrive in one kernel-argument fetch and can be preloaded into scalar
// registers (-mllvm -amdgpu-kernarg-preload-count=16; measured neutral to
// slightly slower on MI355X for the 14336 x 4096 product, so not enabled).
#define Q4K_GEMV_KERNEL_ARGS                                                                      \
    const float *x_, const uint8_t *y_, const uint8_t *w_, int64_t row_stride_, int ldx_,        \
        int stride_col_y_, int K_, int vec_ok_, int rows_base_, int rows_extra_, int nb_, int qcol_, \
        GemvParams p
#define Q4K_GEMV_HEAD_VALUES \
    x_, y_, w_, row_stride_, ldx_, stride_col_y_, K_, vec_ok_, rows_base_, rows_extra_, nb_, qcol_

__device__ __forceinline__ GemvParams with_head(GemvParams p, const float *x, const uint8_t *y,
                                                const uint8_t *w, int64_t row_stride, int ldx,
                                                int stride_col_y, int K, int vec_ok, int rows_base,
                                                int rows_extra, int nb, int qcol) {
    p.x = x;
    p.y = y;
    p.w = w;
    p.row_stride = row_stride;
    p.ldx = ldx;
    p.stride_col_y = stride_col_y;
    p.K = K;
    p.vec_ok = vec_ok;
    p.rows_base = rows_base;
    p.rows_extra = rows_extra;
    p.nb = nb;
    p.G = (nb + 15) >> 4;
    p.qcol = qcol;
    return p;
}

// Position of a wave in its sequence of (row tile, group) steps.
struct Step {
    int tile;
    int i;
};

__device__ __forceinline__ Step next_step(Step s, int G) {
    return s.i + 1 == G ? Step{s.tile + 1, 0} : Step{s.tile, s.i + 1};
}

// The contiguous rows [beg, end) a wave owns: the M rows split as evenly as
// possible over the workgroups (rows_base each, the first rows_extra one
// more), and each workgroup's share as evenly over its waves.  Every CU gets
// the same work to within one row and reads one contiguous range.
struct WaveRows {
    int beg, end;
};

template <int WAVES>
__device__ __forceinline__ WaveRows wave_rows(const GemvParams &p, int wave) {
    const int b = (int)blockIdx.x;
    const int wg_beg = b * p.rows_base + min(b, p.rows_extra);
    const int n = p.rows_base + (b < p.rows_extra ? 1 : 0);
    const int q = n / WAVES, rem = n - q * WAVES;
    const int beg = wg_beg + wave * q + min(wave, rem);
    return WaveRows{beg, beg + q + (wave < rem ? 1 : 0)};
}

// Results of a wave, buffered in LDS and written to dst in coalesced runs:
// entry e is column e % NC of row beg + e / NC.
constexpr int kRing = 256;  // floats per wave

struct ResultRing {
    float *buf;   // this wave's kRing floats of LDS
    int beg;      // first row of the wave
    int end;      // one past its last row
    int base;     // entries already written out
    int n;        // entries buffered
};

// Writes the buffered entries to dst (entries of rows >= end are dropped).
template <int NC>
__device__ __forceinline__ void ring_flush(const GemvParams &p, int lane, ResultRing &rr) {
    for (int k = lane; k < rr.n; k += kWave) {
        const int idx = rr.base + k;
        const int row = rr.beg + idx / NC;
        const int c = idx - (idx / NC) * NC;
        if (row < rr.end) p.dst[(int64_t)c * p.ld_dst + row] = rr.buf[k];
    }
    rr.base += rr.n;
    rr.n = 0;
}

// End of a row tile: the R x NC lane partials of the tile, reduced over the
// wave, go to the result ring (lane r*NC + c writes entry r*NC + c).
template <int NC, int R>
__device__ __forceinline__ void tile_to_ring(const GemvParams &p, int lane, float (&acc)[R][NC],
                                             ResultRing &rr) {
    float out = 0.0f;
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
        for (int c = 0; c < NC; ++c) {
            const float s = wave_sum(acc[r][c]);
            if (lane == r * NC + c) out = s;
            acc[r][c] = 0.0f;
        }
    if (lane < R * NC) rr.buf[rr.n + lane] = out;
    rr.n += R * NC;
    // rare (a wave's rows x NC above kRing): global stores inside the
    // loop make the compiler's load waits conservative
    if (rr.n + R * NC > kRing) ring_flush<NC>(p, lane, rr);
}

}  // namespace q4k
