// q4k_tile.h -- pieces shared by the gfx950 tile kernels of the K-quant
// GEMVs (Q4_K and Q6_K): launch parameters, the split of a product's rows
// over workgroups and waves, the walk over (row tile, group) steps and the
// per-wave result ring.
#pragma once

#include "q4k_device.h"

namespace q4k {

// Channels and samples of a batched launch (grid y = dst channel, z = dst
// sample; kernels/mmvq.cu:174-180): the weight matrix is ids[channel]
// (MUL_MAT_ID) or channel / channel_ratio, the activation channel is
// channel % nchannels_y (MUL_MAT_ID) or the channel itself.
struct BatchParams {
    const int32_t *ids;      // MUL_MAT_ID: weight matrix of each dst channel, or null
    int64_t w_channel;       // bytes between weight matrices
    int64_t w_sample;
    int64_t x_channel;       // activation: floats (F32) or Q8_1 blocks
    int64_t x_sample;
    int64_t dst_channel;     // floats (biases are indexed like dst)
    int64_t dst_sample;
    int channel_ratio;       // dst channels per weight matrix (without ids)
    int sample_ratio;        // dst samples per weight sample
    int nchannels_y;         // MUL_MAT_ID: activation channels (1 or the number of ids)
    int nexperts;            // MUL_MAT_ID: weight matrices; other ids read no weights
};

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
    // fused epilogue (one column): gate weight rows (same layout as w), the
    // biases of the two products (indexed like dst) and the GLU op
    const uint8_t *gate;
    const float *bias;
    const float *gate_bias;
    int glu_op;
    BatchParams bt;          // batched launches only
    int w_absent;            // batched: this workgroup's weight matrix is absent (bad id)
    // parity variants (SUMS) only: the int32 sums the kernel forms, where
    // the oracle keeps them (Q4_K: sums[(c*M + row)*(K/32) + 8kb + s],
    // sq[c*(K/32) + b]; Q6_K: sums[(c*M + row)*(K/16) + 16kb + t])
    int32_t *sums;
    int32_t *sq;
};

// A batched launch: its BatchParams and the dst channels and samples (grid
// y and z); nch = nsmp = 1 with bt.ids null is the plain 2-D product.
struct BatchLaunch {
    BatchParams bt{};
    int nch = 1;
    int nsmp = 1;
};

// Batched launches, step 1 (before the activation loads): this workgroup's
// activation channel, dst and bias slices.  Only kernel arguments and the
// block index: no memory access.
__device__ __forceinline__ void batch_activation(GemvParams &p) {
    const int ch = (int)blockIdx.y, smp = (int)blockIdx.z;
    const int cy = p.bt.ids ? ch % p.bt.nchannels_y : ch;
    const int64_t xo = (int64_t)smp * p.bt.x_sample + (int64_t)cy * p.bt.x_channel;
    if (p.x) p.x += xo;
    else p.y += xo * kQ81Bytes;
    const int64_t dofs = (int64_t)smp * p.bt.dst_sample + (int64_t)ch * p.bt.dst_channel;
    p.dst += dofs;
    if (!p.bt.ids) {  // biases per dst channel; with ids per weight matrix (step 2)
        if (p.bias) p.bias += dofs;
        if (p.gate_bias) p.gate_bias += dofs;
    }
}

// Batched launches, step 2 (after the activation loads are issued): the
// weight matrix.  The expert id is read with a vector load, which returns
// after the activation loads issued before it, then made wave-uniform.  An
// id outside [0, nexperts) selects no matrix: the workgroup's weight loads
// read zeros and its biases are dropped.
__device__ __forceinline__ void batch_weights(GemvParams &p) {
    const int ch = (int)blockIdx.y, smp = (int)blockIdx.z;
    int cx;
    if (p.bt.ids) {
        const __amdgpu_buffer_rsrc_t ri = make_rsrc(p.bt.ids, (uint32_t)(ch + 1) * 4u);
        cx = __builtin_amdgcn_readfirstlane((int)__builtin_amdgcn_raw_buffer_load_b32(ri, (uint32_t)ch * 4u, 0, 0));
        const bool ok = cx >= 0 && cx < p.bt.nexperts;
        p.w_absent = !ok;
        const int64_t bo = (int64_t)smp * p.bt.dst_sample + (int64_t)cx * p.bt.dst_channel;
        p.bias = p.bias && ok ? p.bias + bo : nullptr;
        p.gate_bias = p.gate_bias && ok ? p.gate_bias + bo : nullptr;
        if (!ok) cx = 0;
    } else {
        cx = ch / p.bt.channel_ratio;
    }
    const int64_t wo = (int64_t)(smp / p.bt.sample_ratio) * p.bt.w_sample + (int64_t)cx * p.bt.w_channel;
    p.w += wo;
    if (p.gate) p.gate += wo;
}

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

// Epilogue of a tile kernel variant, a compile-time choice: the plain
// kernels never read the epilogue's kernel arguments (a kernel-argument
// cache line first touched at the loop's entry costs the whole launch a
// memory round trip).
constexpr int kEpiNone = 0;  // dst = product
constexpr int kEpiBias = 1;  // dst = product + bias
constexpr int kEpiGlu = 2;   // dst = glu(product + bias, gate product + gate bias)

// GLU ops of the fused epilogue (values of ggml's enum ggml_glu_op).
constexpr int kGluGeglu = 1;
constexpr int kGluSwiglu = 2;
constexpr int kGluSwigluOai = 3;

// The epilogue of kernels/mmvq.cu:309-336 for one output: `up` (the product
// with the weight, bias added) gated by `g` (the product with the gate
// weight, its bias added): SWIGLU up * silu(g), GEGLU up * gelu(g) (tanh
// form), SWIGLU_OAI with alpha 1.702 and limit 7 (ggml's
// ggml_cuda_op_*_single formulas; expf and tanhf are the device library's).
__device__ __forceinline__ float glu_apply(int op, float up, float g) {
    if (op == kGluSwiglu) return up * (g / (1.0f + expf(-g)));
    if (op == kGluGeglu) {
        const float kSqrt2OverPi = 0.79788456080286535588f;
        return up * (0.5f * g * (1.0f + tanhf(kSqrt2OverPi * g * (1.0f + 0.044715f * g * g))));
    }
    if (op == kGluSwigluOai) {
        const float x = fminf(g, 7.0f);
        const float u = fmaxf(fminf(up, 7.0f), -7.0f);
        return x / (1.0f + expf(-x * 1.702f)) * (1.0f + u);
    }
    return up * g;
}

// Results of a wave, buffered in LDS and written to dst in coalesced runs:
// entry e is column e % NC of row beg + e / NC; with a gate (GLU), entries
// 2t and 2t + 1 are the products of row beg + t with the weight and the gate.
// Floats per wave: 256, or 64 (eight rows) from five columns on, which lets
// eight 14336-value columns and the rings of 16 waves share one
// workgroup's 160 KB of LDS.
__host__ __device__ constexpr int ring_floats(int nc) { return nc <= 4 ? 256 : 64; }

// The ring of a launch: ring_floats(nc) floats per wave, or, from three
// columns on, 64 where those rings and an activation of act bytes would not
// fit a gfx950 workgroup's 160 KB of LDS (three or four columns of ~26,000
// values or more: Q6_K 8192 x 28672 at N=4 then runs in one launch instead
// of two).  A ring holds at least one step's R * NC <= 32 entries.  The
// kernels derive it from the ring offset (the activation's size), which they
// read anyway.  One and two columns keep the compile-time size: with the
// size a run-time value the fused Q6_K gate/up launch measured 4 % slower
// (14336 x 4096: 20.7 -> 21.6 us), and their rings always fit.
constexpr int kLdsBytes = 160 * 1024;
__host__ __device__ constexpr int ring_cap(int act, int nc, int waves) {
    return nc <= 2 || act + waves * ring_floats(nc) * 4 <= kLdsBytes ? ring_floats(nc) : 64;
}

struct ResultRing {
    float *buf;   // this wave's cap floats of LDS
    int beg;      // first row of the wave
    int end;      // one past its last row
    int base;     // entries already written out
    int n;        // entries buffered
    int cap;      // floats in buf
};

// Writes the buffered entries to dst (entries of rows >= end are dropped),
// applying the variant's epilogue.
template <int NC, int EPI>
__device__ __forceinline__ void ring_flush(const GemvParams &p, int lane, ResultRing &rr) {
    if (EPI == kEpiGlu) {
        for (int k = lane; 2 * k < rr.n; k += kWave) {
            const int row = rr.beg + rr.base / 2 + k;
            if (row < rr.end) {
                const float2 v = *reinterpret_cast<const float2 *>(rr.buf + 2 * k);
                const float up = p.bias ? v.x + p.bias[row] : v.x;
                const float g = p.gate_bias ? v.y + p.gate_bias[row] : v.y;
                p.dst[row] = glu_apply(p.glu_op, up, g);
            }
        }
    } else {
        for (int k = lane; k < rr.n; k += kWave) {
            const int idx = rr.base + k;
            const int row = rr.beg + idx / NC;
            const int c = idx - (idx / NC) * NC;
            if (row < rr.end) {
                const int64_t o = (int64_t)c * p.ld_dst + row;
                p.dst[o] = EPI == kEpiBias ? rr.buf[k] + p.bias[o] : rr.buf[k];
            }
        }
    }
    rr.base += rr.n;
    rr.n = 0;
}

// v_permlane32_swap_b32 a, b: lanes 32..63 of a trade places with lanes 0..31
// of b; v_permlane16_swap_b32 a, b: the odd 16-lane rows of a trade places
// with the even rows of b.  Inline assembly: clang's builtins for them keep
// only the first of the two results.  The s_nop covers a VALU write of
// either operand right before.
__device__ __forceinline__ void permlane32_swap(float &a, float &b) {
    asm volatile("s_nop 1\n\tv_permlane32_swap_b32 %0, %1" : "+v"(a), "+v"(b));
}
__device__ __forceinline__ void permlane16_swap(float &a, float &b) {
    asm volatile("s_nop 1\n\tv_permlane16_swap_b32 %0, %1" : "+v"(a), "+v"(b));
}

// Sums of NC (2..8) lane values over the wave, reduce-scatter style: with P
// the power of two >= NC, each lane-swap halves the values a lane holds
// (lane bit 5, then 4, then 3 select which half it keeps), so that lane l
// ends with the sum of value (l >> (6 - log2 P)) over the 64 lanes, and the
// butterfly over the remaining low lane bits costs one step per bit for all
// values together.  Every value is summed over a fixed tree, the same in
// every workgroup and wave.
template <int NC>
__device__ __forceinline__ float column_sums(const float (&v)[NC], int lane) {
    constexpr int P = NC <= 2 ? 2 : (NC <= 4 ? 4 : 8);
    static_assert(NC >= 2 && NC <= 8, "two to eight values");
    float u[P];
#pragma unroll
    for (int i = 0; i < P; ++i) u[i] = i < NC ? v[i] : 0.0f;
#pragma unroll
    for (int i = 0; i < P / 2; ++i) {  // lane bit 5: lanes 0..31 keep value i, 32..63 value i + P/2
        float a = u[i], b = u[i + P / 2];
        permlane32_swap(a, b);
        u[i] = a + b;
    }
    if constexpr (P >= 4) {
#pragma unroll
        for (int i = 0; i < P / 4; ++i) {  // lane bit 4: even rows keep u[i], odd rows u[i + P/4]
            float a = u[i], b = u[i + P / 4];
            permlane16_swap(a, b);
            u[i] = a + b;
        }
    }
    float s = u[0];
    if constexpr (P == 8) {  // lane bit 3: the lane keeps u[bit3] and adds its partner's
        const bool hi = (lane & 8) != 0;
        const float keep = hi ? u[1] : u[0];
        const float send = hi ? u[0] : u[1];
        s = keep + dppf<kDppRor8>(send);
    }
    s += dppf<kDppXor1>(s);
    s += dppf<kDppXor2>(s);
    s += dppf<kDppHalfMirror>(s);
    if constexpr (P <= 4) s += dppf<kDppRor8>(s);
    if constexpr (P == 2) {  // lane bit 4: a + b = s + s(lane ^ 16) in every lane
        float a = s, b = s;
        permlane16_swap(a, b);
        s = a + b;
    }
    return s;
}

// End of a row tile: the R x NC lane partials of the tile, reduced over the
// wave, go to the result ring (entry r*NC + c; with one column lane r writes
// entry r, with several the lanes of column_sums' map).
template <int NC, int R, int EPI>
__device__ __forceinline__ void tile_to_ring(const GemvParams &p, int lane, float (&acc)[R][NC],
                                             ResultRing &rr) {
    if constexpr (NC == 1) {
        float out = 0.0f;
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const float s = wave_sum(acc[r][0]);
            if (lane == r) out = s;
            acc[r][0] = 0.0f;
        }
        if (lane < R) rr.buf[rr.n + lane] = out;
    } else {
        constexpr int P = NC <= 2 ? 2 : (NC <= 4 ? 4 : 8);
        constexpr int kShift = P == 2 ? 5 : (P == 4 ? 4 : 3);
        const int c = lane >> kShift;
        const bool writer = (lane & ((1 << kShift) - 1)) == 0 && c < NC;
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const float s = column_sums<NC>(acc[r], lane);
            if (writer) rr.buf[rr.n + r * NC + c] = s;
#pragma unroll
            for (int k = 0; k < NC; ++k) acc[r][k] = 0.0f;
        }
    }
    rr.n += R * NC;
    // rare (a wave's rows x NC above the ring): global stores inside the
    // loop make the compiler's load waits conservative
    if (rr.n + R * NC > rr.cap) ring_flush<NC, EPI>(p, lane, rr);
}

}  // namespace q4k
