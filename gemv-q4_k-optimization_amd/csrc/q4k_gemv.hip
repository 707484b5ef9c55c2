// q4k_gemv.hip -- the Q4_K matrix-vector product's launches and the C ABI
// declared in include/q4k_gemv.h.
//
// Kernels defined here
//   quantize_q8_1_kernel   F32 -> AoS block_q8_1 (the standalone quantiser,
//                          kernels/mmvq.cu:728-735 calls its counterpart)
//   subblock_sums_kernel   parity probe: the int32 sub-block sums computed with
//                          the GEMV's lane map and dot routines, one wave per
//                          (row, group)
// and instantiated here: the product variants of the GEMV kernels of
// q4k_gemv_kernels.h (their parity variants are in q4k_sums.hip).
#include <hip/hip_runtime.h>

#include <atomic>
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <vector>

#include "../../include/q4k_gemv.h"
#include "q4k_runtime.h"
#include "q4k_gemv_kernels.h"
#include "q4k_ksplit.h"
#include "q4k_ksplit_nc.h"
#include "q4k_mfma.h"
#include "q4k_tile.h"

namespace q4k {

// F32 -> AoS block_q8_1 with ggml-cuda's quantize_q8_1 arithmetic (call site
// kernels/mmvq.cu:728-735): per 32 values d = amax/127 (div127, the IEEE
// quotient), q = roundf(x/d) (quantize_values), ds = (half(d), half(sum x)).
// Eight lanes per block, four values (one 16-byte load) per lane, 32 blocks
// per 256-thread workgroup.  amax is order-free; the sum follows the tree of
// ggml's 32-lane warp_reduce_sum (partners at element distance 16, 8, 4, 2,
// 1), which with element 4e + k in lane e is lane distance 4, 2, 1 and then
// k ^ 2, k ^ 1 inside the lane, so ds.y is bit for bit ggml's.
__global__ __launch_bounds__(256) void quantize_q8_1_kernel(const float *__restrict__ x,
                                                            uint8_t *__restrict__ vy, int64_t ne00,
                                                            int64_t s01, int64_t nblk_col, int vec_ok) {
    const int64_t blk = (int64_t)blockIdx.x * 32 + (threadIdx.x >> 3);
    if (blk >= nblk_col) return;  // whole 8-lane groups leave together
    const int e = threadIdx.x & 7;
    const int64_t col = blockIdx.y;
    const int64_t i0 = blk * 32 + 4 * e;
    const float *src = x + col * s01 + i0;
    float v[4];
    if (vec_ok && i0 + 4 <= ne00) {
        const float4 a = *reinterpret_cast<const float4 *>(src);
        v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
    } else {
#pragma unroll
        for (int k = 0; k < 4; ++k) v[k] = i0 + k < ne00 ? src[k] : 0.0f;
    }
    float amax = fmaxf(fmaxf(fabsf(v[0]), fabsf(v[1])), fmaxf(fabsf(v[2]), fabsf(v[3])));
    amax = block_max<8>(amax);
    float t[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) t[k] = v[k] + swizzle_xor<4>(v[k]);
#pragma unroll
    for (int k = 0; k < 4; ++k) t[k] += dppf<kDppXor2>(t[k]);
#pragma unroll
    for (int k = 0; k < 4; ++k) t[k] += dppf<kDppXor1>(t[k]);
    const float sum = (t[0] + t[2]) + (t[1] + t[3]);
    const float d = div127(amax);
    uint32_t word[1] = {0u};
    int qsum[1];
    if (amax != 0.0f) quantize_values<4, 1>(v, d, __builtin_amdgcn_rcpf(d), word, qsum);
    uint8_t *out = vy + (col * nblk_col + blk) * kQ81Bytes;
    *reinterpret_cast<uint32_t *>(out + 4 + 4 * e) = word[0];
    if (e == 0) {
        const uint16_t dh = __builtin_bit_cast(uint16_t, (_Float16)d);
        const uint16_t sh = __builtin_bit_cast(uint16_t, (_Float16)sum);
        *reinterpret_cast<uint32_t *>(out) = (uint32_t)dh | ((uint32_t)sh << 16);
    }
}

struct SumsParams {
    const uint8_t *w;
    int64_t row_stride;
    const uint8_t *y;  // one column of AoS Q8_1
    int32_t *sqq;      // [M][K/32] for this column
    int32_t *sq;       // [K/32] for this column
    int M, K, nb, G, qcol;
    FastDiv nblk32;
};

// One wave per (row, group): the GEMV's lane map, swizzled activation layout,
// loads and lane_qdot; each lane's two sums are whole sub-blocks.
__global__ __launch_bounds__(256) void subblock_sums_kernel(SumsParams p) {
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    int8_t *q8s = reinterpret_cast<int8_t *>(lds);
    float2 *dks = reinterpret_cast<float2 *>(lds + p.qcol);
    stage_from_q8_1<kLayoutQ4K, 256>(p.y, 0, p.K, 1, p.nblk32, p.qcol, q8s, dks);
    __syncthreads();
    GemvParams gp{};
    gp.w = p.w;
    gp.row_stride = p.row_stride;
    gp.M = p.M;
    gp.K = p.K;
    gp.nb = p.nb;
    gp.qcol = p.qcol;
    Lane ln;
    ln.lane = threadIdx.x & 63;
    ln.g = ln.lane >> 2;
    ln.j = ln.lane & 3;
    ln.sel = make_scale_sel(ln.j);
    const int nitems = p.M * p.G;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    for (int item = blockIdx.x * 4 + wave; item < nitems; item += gridDim.x * 4) {
        const int row = item / p.G;
        const int i = item - row * p.G;
        RowRegs w[1];
        load_group<1>(gp, row, 1, i, ln.g, ln.j, w);
        const LaneAct a = lane_act(gp, ln, i, 0, q8s, dks);
        int sa, sb;
        lane_qdot(w[0].q0, w[0].q1, a.a0, a.a1, a.b0, a.b1, sa, sb);
        const int kb = 16 * i + ln.g;
        if (kb < p.nb) {
            int32_t *o = p.sqq + (int64_t)row * (p.K / 32) + kb * 8 + ln.j * 2;
            o[0] = sa;
            o[1] = sb;
            if (row == 0) {
                p.sq[kb * 8 + ln.j * 2] = byte_sum16(a.a0) + byte_sum16(a.a1);
                p.sq[kb * 8 + ln.j * 2 + 1] = byte_sum16(a.b0) + byte_sum16(a.b1);
            }
        }
    }
}

// ------------------------------------------------------------------------
// host side
// ------------------------------------------------------------------------

thread_local int32_t g_last_hip_error = 0;

int hip_fail(hipError_t e) {
    g_last_hip_error = (int32_t)e;
    return Q4K_EHIP;
}

static DeviceInfo g_dev[kMaxDevices];

int device_info(DeviceInfo **out) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return hip_fail(e);
    if (dev < 0 || dev >= kMaxDevices) return Q4K_EUNSUPPORTED;
    DeviceInfo &di = g_dev[dev];
    std::call_once(di.once, [&]() {
        hipDeviceProp_t prop;
        if (hipGetDeviceProperties(&prop, dev) != hipSuccess) return;
        di.cus = prop.multiProcessorCount;
        int lds = 0;
        if (hipDeviceGetAttribute(&lds, hipDeviceAttributeMaxSharedMemoryPerBlock, dev) != hipSuccess)
            lds = 65536;
        di.max_lds = lds;
        di.supported = std::strncmp(prop.gcnArchName, "gfx950", 6) == 0;
        di.ok = true;
    });
    if (!di.ok) return hip_fail(hipErrorInvalidDevice);
    if (!di.supported) return Q4K_EUNSUPPORTED;
    *out = &di;
    return Q4K_OK;
}

int ensure_lds(DeviceInfo *di, const void *fn, int bytes) {
    if (bytes <= 65536) return Q4K_OK;
    std::lock_guard<std::mutex> lk(di->attr_mu);
    for (const void *f : di->attr_done)
        if (f == fn) return Q4K_OK;
    hipError_t e = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, di->max_lds);
    if (e != hipSuccess) return hip_fail(e);
    di->attr_done.push_back(fn);
    return Q4K_OK;
}

// Geometry overrides for tuning sweeps (0 = automatic; prologue -1 =
// automatic), set only through q4k_set_geometry_override and
// q4k_set_pipeline_override: nothing is read from the environment.
std::atomic<int> g_ovr_rows{0}, g_ovr_waves{0}, g_ovr_wgs{0}, g_ovr_kernel{0};
std::atomic<int> g_ovr_prologue{-1}, g_ovr_slots{0};

struct Geometry {
    int R = 2;          // tile kernel: rows per wave tile
    int waves = 16;     // waves per workgroup
    int grid = 0;       // workgroups
    int lds = 0;        // LDS bytes the activation needs
    int lds_launch = 0; // LDS bytes requested at launch (>= lds)
    int nc_chunk = 1;   // columns per launch
    int ntiles = 0;     // block-per-lane kernel: passes
    int bpl = 0;        // 1: block-per-lane kernel
    int rpw = 0;        // block-per-lane kernel: rows per pass
    int rows_base = 0;  // tile kernel: rows per workgroup (first rows_extra +1)
    int rows_extra = 0;
    int prologue = 0;   // tile kernel: when the first weight loads go out (PRO)
    int slots = 2;      // tile kernel: groups in flight per wave (S)
    int mfma = 0;       // 1: matrix-core kernel (tiles of 16 rows; rows_base/rows_extra count tiles)
    int mfma_ga = 0;    // matrix-core kernel: A operand from the Q8_1 buffer (pre-quantised route)
    int ks = 1;         // matrix-core kernel: waves sharing one tile
    int segs = 1;       // matrix-core kernel: summation segments of a row
    int ksplit = 0;     // K-split kernel: super-blocks per wave and group (0: another kernel)
    int ks_long = 0;    // K-split kernel for rows of any length (activation slices in LDS)
    int ks_staged = 0;  // several-column K-split kernel: activation quantised once per workgroup into LDS
    int ks_p = 0;       // several-column K-split kernel: columns of its reduction tree (2 or 4)
    int ks_kt = 0;      // long-row K-split kernel, rows shorter than one group: waves per team (0: 16/SBW)
    int colsplit = 0;   // several columns as one launch over one-column channels (the columns; 0: not)
    int ks_snc = 0;     // several columns of rows shorter than one group in short teams: the tree's columns (2, 4)
};

// Tile kernel variants that are instantiated: those whose registers fit the
// launch bounds without spilling (16 waves per workgroup leave 128 VGPRs per
// lane, 8 waves 256), with 2 or 4 groups in flight.
static constexpr bool tile_fits(int nc, int R, int waves, int slots) {
    if (slots == 8) return waves <= 8 && R == 1 && nc <= 2;
    if (slots == 1) return R == 1;
    if (slots == 4)
        return waves > 8 ? (R == 1 && nc <= 4) : (R == 1 || (R == 2 && nc <= 4));
    return waves > 8 ? (R == 1 || (R == 2 && nc <= 2)) : (R <= 2 || (R == 4 && nc <= 5));
}

// Rows per pass of the block-per-lane kernel, 0 when it does not apply.
static int bpl_rows_per_pass(int64_t nb) {
    if (nb == 16) return 4;
    if (nb == 32) return 2;
    if (nb > 32 && nb <= 64) return 1;
    return 0;
}

// LDS bytes of the staged activation: q8 columns (swizzled, padded to whole
// 16-block groups, for the tile kernel; linear for the one-column block
// kernels) followed by the per-32-value (d8, d8*sum q8) pairs.
static int lds_bytes(int K, int nc) { return nc * (q8_col_bytes(K) + K / 4); }
// The tile kernel adds a result ring per wave after the activation.
static int tile_lds_bytes(int K, int nc, int waves) {
    const int act = lds_bytes(K, nc);
    return act + waves * ring_cap(act, nc, waves) * 4;
}
static int lds_bytes_linear(int K) { return K + K / 4; }

// Products that run on the matrix-core kernel when no override says
// otherwise (all columns in one launch, which the caller checks).  Measured
// on MI355X against the tile kernel (interleaved, one process; us):
//  - rows of 4096 values: eight columns from 896 row tiles (14336 rows), six
//    to eight from 4096 tiles: 128256 x 4096 N=8 64.5 against 83.4, N=6
//    63.6 against 73.2; 28672 x 4096 N=8 21.1 against 22.9; 14336 x 4096 N=8
//    14.1 against 15.7.  Slower with fewer rows (4096 x 4096 N=8 10.2
//    against 8.6; 11008 x 4096 N=8 13.7 against 12.9) or fewer columns
//    (14336 x 4096 N=6 13.8 against 13.3; 128256 x 4096 N=4 62.7 against
//    57.6: padded columns cost scaling work).
//  - longer rows (two or more 16-block groups, where the tile kernel reads
//    every column's activation from LDS at each step): six to eight columns
//    from 512 tiles, five from 864: 8192 x 8192 N=8 17.8 against 22.0, N=6
//    17.0 against 19.4; 13824 x 5120 N=8 18.2 against 26.0, N=5 16.6 against
//    18.0; 28672 x 10240 N=5 43.4 against 50.1.  Slower at 5120 x 5120 and
//    below (N=7 13.0 against 12.5), at five columns of 8192 x 5120 or 6144
//    (13.1 against 12.9) and at four columns (8192 x 8192 14.5 against 13.3).
//  - shorter rows: the tile kernel (18944 x 3584 N=8 17.7 against 18.7).
// Rows longer than ~10,700 values need two launches for eight columns and
// are left to the tile kernel (4096 x 14336 N=8).  Four items in flight per
// wave instead of two measured slower on every shape.
static bool use_mfma(int64_t M, int64_t N, int64_t K) {
    const int64_t tiles = (M + kMfmaRows - 1) / kMfmaRows;
    if (K < 4096) return false;
    if (K == 4096) return (N == 8 && tiles >= 896) || (N >= 6 && tiles >= 4096);
    return (N >= 6 && tiles >= 512) || (N == 5 && tiles >= 864);
}

// Where the pre-quantised route runs the matrix-core kernel with its A
// operand read from the Q8_1 buffer (GA): rows longer than 8192 values,
// five to eight columns, a tile per CU or more, where (the caller checks)
// the staged matrix-core kernel is not chosen or cannot hold the columns.
// Measured on MI355X (us per op with a Q8_1 workspace, the quantiser launch
// included; GA against the tile kernel): 4096 x 14336 N=8 18.35 against
// 22.84, N=6 17.66 / 19.86, N=5 17.38 / 18.16; 8192 x 28672 N=8 44.07 /
// 66.95, N=6 42.65 / 62.90.  Slower at four columns (8192 x 28672 39.40 /
// 37.62) and than the staged matrix-core kernel where that is chosen and
// holds the columns (13824 x 5120 N=8 24.74 against 17.87, 8192 x 8192
// N=8 17.54 / 17.34, 28672 x 4096 N=8 22.99 / 21.70).  Two items in flight
// per wave, not four (4096 x 14336 N=8 18.35 against 20.07); weights
// through the slot, not loaded straight into the lanes' registers in MFMA
// order (4096 x 14336 N=6 17.57 against 21.43).
static bool use_mfma_ga(int64_t M, int64_t N, int64_t K) {
    const int64_t tiles = (M + kMfmaRows - 1) / kMfmaRows;
    return K > 8192 && N >= 5 && tiles >= 256;
}

// The matrix-core kernel: one workgroup per CU (at most one per tile) of 8
// or 16 waves, the tiles of 16 rows split evenly over the workgroups, and as
// many waves sharing a tile (KS) as leave every wave group a tile in the
// first round -- KS at most the S summation segments of a row (S = min(8,
// the largest power of two <= the super-blocks per row), a function of K
// alone, which fixes the summation order).
static Geometry pick_geometry_mfma(const DeviceInfo &di, int64_t K, int64_t M, int nc, int owgs, int owaves,
                                   bool ga = false) {
    Geometry g;
    const int max_lds = di.max_lds > 0 ? di.max_lds : 65536;
    const int cus = di.cus > 0 ? di.cus : 1;
    const int64_t tiles = (M + kMfmaRows - 1) / kMfmaRows;
    g.mfma = 1;
    g.R = kMfmaRows;
    g.slots = 2;
    g.nc_chunk = nc;
    const int64_t wgs = owgs > 0 ? owgs : cus;
    g.grid = (int)(tiles < wgs ? tiles : wgs);
    if (g.grid < 1) g.grid = 1;
    g.rows_base = (int)(tiles / g.grid);
    g.rows_extra = (int)(tiles % g.grid);
    const int64_t nt = g.rows_base + (g.rows_extra ? 1 : 0);
    g.waves = 16;  // measured faster than 8 where the kernel is chosen
    if (owaves >= 1 && owaves <= 16) g.waves = owaves > 8 ? 16 : 8;
    if (ga) {  // GA: its A operands in flight take 146 registers at 2 items
        g.waves = 8;
        const int os = g_ovr_slots.load();
        g.slots = os == 2 || os == 4 ? os : 2;
    }
    const int64_t nb = K / kQK;
    g.segs = 1;
    while (g.segs < kMfmaMaxSegs && 2 * g.segs <= nb) g.segs *= 2;
    int groups = 1;
    while (groups < g.waves && 2 * groups <= nt) groups *= 2;
    g.ks = g.waves / groups;
    while (g.ks > g.segs) g.ks /= 2;
    g.mfma_ga = ga ? 1 : 0;
    g.lds = ga ? mfma_ga_lds_bytes((int)K, g.waves) : mfma_lds_bytes((int)K, nc, g.waves);
    g.lds_launch = g.lds <= max_lds / 2 ? max_lds / 2 + 256 : g.lds;  // one workgroup per CU
    return g;
}

// The K-split kernel: rows_per_step TR = 16 / SBW rows per wave step (1, 4,
// 8, 16; SBW super-blocks per wave and group; rows of other lengths than
// 4096 and 8192 values: 4 for up to 4 groups, 8, 16), waves per workgroup
// (whole teams of TR waves), workgroups (default one per CU) and row tiles
// in flight per wave (1 or 2).
static Geometry pick_geometry_ksplit(const DeviceInfo &di, int64_t K, int64_t M, int rows_per_step, int waves,
                                     int wgs, int slots, int N = 1, int staged = 0, int P = 0, int fused = 0,
                                     bool batch = false) {
    Geometry g;
    const int cus = di.cus > 0 ? di.cus : 1;
    if (N >= 2) {  // two to four columns
        const bool lng = K != 4096 && K != 8192;  // rows of other lengths: the long-row form (staged)
        const int G = lng ? (int)((K / kQK + 15) / 16) : (int)(K / 4096);
        g.ks_long = lng ? 1 : 0;
        g.ks_p = lng && P == 2 ? 2 : (N <= 2 ? 2 : 4);  // rows of 1 or 2 groups: the columns rounded up
        g.ksplit = g.ks_p == 2 && rows_per_step == 8 ? 2 : 4;
        g.R = 16 / g.ksplit;
        g.waves = waves == 4 || waves == 8 || waves == 16 ? waves : 8;
        if (g.waves < g.R) g.waves = g.R;
        g.slots = slots == 1 || slots == 2 ? slots : 2;
        auto exists = [&]() {
            return lng ? ksplit_nc_long_exists(N, g.ks_p, g.ksplit, g.waves, g.slots)
                       : ksplit_nc_exists(N, g.ksplit, g.waves, g.slots, G);
        };
        if (!exists()) g.slots = 1;
        if (!exists()) {
            g.waves = 8;
            g.slots = 2;
        }
        // rows of 1 or 2 groups, three or four columns: the activation
        // quantised once per workgroup (prologue override 0) or by every
        // wave for its own slices (2); otherwise as `staged` says
        const int opro = g_ovr_prologue.load();
        g.ks_staged = lng || (N >= 3 && (opro == 0 || (opro != 2 && staged))) ? 1 : 0;
        int64_t grid = wgs > 0 ? wgs : cus;
        if (grid > M) grid = M;
        g.grid = grid < 1 ? 1 : (int)grid;
        g.rows_base = (int)(M / g.grid);
        g.rows_extra = (int)(M % g.grid);
        g.lds = ksplit_nc_part_bytes(g.rows_base + (g.rows_extra ? 1 : 0), N, g.ksplit) +
                (g.ks_staged ? ksn_stage_bytes((int)K, N) : 0);
        g.lds_launch = g.lds;
        g.nc_chunk = N;
        return g;
    }
    const int tr = rows_per_step == 1 || rows_per_step == 4 || rows_per_step == 8 || rows_per_step == 16
                       ? rows_per_step
                       : 16;
    const bool lng = K != 4096 && K != 8192;  // rows of other lengths: the long-row variant
    const int G = (int)((K / kQK + 15) / 16), gmax = G <= 4 ? 4 : 8;
    g.ks_long = lng ? 1 : 0;
    g.ksplit = 16 / tr;
    // long rows: 4 super-blocks per wave for up to 4 groups, else at most 2
    if (lng && g.ksplit > (G <= 4 ? 4 : 2)) g.ksplit = G <= 4 ? 4 : 2;
    g.R = 16 / g.ksplit;
    g.waves = waves >= 1 && waves <= 16 ? waves : 16;
    g.slots = slots >= 1 && slots <= 4 ? slots : 1;
    // rows shorter than one group: teams of only the waves the row needs,
    // where that variant is instantiated (else the whole team; team sizes
    // other than powers of two take workgroups of whole teams)
    const int epi = fused == kFusedGate ? kEpiGlu : (fused == kFusedBias ? kEpiBias : kEpiNone);
    int kt = lng ? ksplit_short_team((int)(K / kQK), g.ksplit) : 0;
    if (kt) {
        if (g.waves < kt) g.waves = kt;
        if (!ksplit_short_exists(false, g.ksplit, kt, g.waves, g.slots, false, epi, batch)) g.slots = 1;
        if (!ksplit_short_exists(false, g.ksplit, kt, g.waves, g.slots, false, epi, batch)) kt = 0;
    }
    g.ks_kt = kt;
    if (!kt) {
        if (g.waves != 4 && g.waves != 8 && g.waves != 16) g.waves = 16;
        if (g.waves < g.R) g.waves = g.R;
        if (lng ? !ksplit_long_exists(g.ksplit, g.waves, g.slots, gmax)
                : !ksplit_exists(g.ksplit, g.waves, g.slots, (int)(K / 4096)))
            g.slots = 2;
    }
    int64_t grid = wgs > 0 ? wgs : cus;
    if (grid > M) grid = M;
    g.grid = grid < 1 ? 1 : (int)grid;
    g.rows_base = (int)(M / g.grid);
    g.rows_extra = (int)(M % g.grid);
    const int rows = g.rows_base + (g.rows_extra ? 1 : 0);
    // fused epilogue or batched launch: the variants that exist (else
    // ksplit = 0: the caller takes the tile kernel); with a gate two
    // partials per (row, slice)
    if ((fused || batch) && !kt) {
        const int gk = lng ? gmax : (int)(K / 4096);
        auto ok = [&]() {
            return batch ? (lng ? ksplit_long_batch_exists(g.ksplit, g.waves, g.slots, gk)
                                : ksplit_batch_exists(g.ksplit, g.waves, g.slots, gk))
                         : (lng ? ksplit_long_epi_exists(g.ksplit, g.waves, g.slots, gk)
                                : ksplit_epi_exists(g.ksplit, g.waves, g.slots, gk));
        };
        if (g.slots > 2 || !ok()) g.slots = 1;
        if (!ok()) g.ksplit = 0;
    }
    const int nw = fused == kFusedGate ? 2 : 1;
    g.lds = lng ? ksplit_long_lds_bytes(rows, g.ksplit ? g.ksplit : 1, g.waves, G, nw, kt)
                : ksplit_lds_bytes(rows, g.ksplit ? g.ksplit : 1, nw);
    g.lds_launch = g.lds;
    g.nc_chunk = 1;
    return g;
}

// The several-column short-team kernel (gemv_q4k_ksplit_short_nc_kernel) for
// N columns of rows of nb blocks: rows_per_step 8 or 4 (2 or 4 super-blocks
// per wave), waves, workgroups (default one per CU), tiles in flight; the
// team is the fewest waves that cover the row.  ksplit = 0 where that
// variant is not instantiated.
static Geometry pick_geometry_short_nc(const DeviceInfo &di, int64_t K, int64_t M, int N, int rows_per_step,
                                       int waves, int wgs, int slots) {
    Geometry g;
    const int cus = di.cus > 0 ? di.cus : 1;
    const int nb = (int)(K / kQK);
    const bool rc4 = N > 2 && nb > 4;  // the four-column tree: super-blocks w and w + 4 per wave
    g.ksplit = rc4 ? 2 : (rows_per_step == 4 || N > 2 ? 4 : 2);
    g.R = 16 / g.ksplit;
    g.ks_kt = rc4 ? 4 : ksplit_short_team(nb, g.ksplit);
    g.waves = waves == 4 || waves == 8 || waves == 16 ? waves : 8;
    g.slots = slots == 1 || slots == 2 ? slots : 1;
    if (!g.ks_kt || !ksplit_short_nc_exists(N, g.ksplit, g.ks_kt, g.waves, g.slots, rc4 ? 4 : 2)) {
        g.ksplit = 0;
        return g;
    }
    g.ks_long = 1;
    g.ks_snc = rc4 ? 4 : 2;
    int64_t grid = wgs > 0 ? wgs : cus;
    if (grid > M) grid = M;
    g.grid = grid < 1 ? 1 : (int)grid;
    g.rows_base = (int)(M / g.grid);
    g.rows_extra = (int)(M % g.grid);
    g.lds = ksplit_short_nc_lds_bytes(g.rows_base + (g.rows_extra ? 1 : 0), N, g.ksplit, g.ks_kt, g.waves);
    g.lds_launch = g.lds;
    if (g.lds > (di.max_lds > 0 ? di.max_lds : 65536)) g.ksplit = 0;
    g.nc_chunk = N;
    return g;
}

// Whether N columns of rows of K values can take the several-column
// short-team kernel: rows of 3 to 8 blocks (with two columns, or three or
// four over 3 or 4 blocks, the tile kernel's tree reduces to the one-column
// tree; three or four columns over 5 to 8 blocks pair super-blocks w and
// w + 4 first) and the tile kernel launches all N at once.
static bool short_nc_ok(int64_t K, int N, int tile_nc) {
    const int64_t nb = K / kQK;
    return tile_nc == N && K % kQK == 0 && nb >= 3 && nb <= 8 && N >= 2 && N <= 4;
}

// The several-column short-team kernel's automatic launch shape (aligned F32
// columns whose rows short_nc_ok admits), one workgroup per CU; false where the
// column split or the tile kernel measured faster.  Rows per CU rho: two
// columns at 2 super-blocks per wave, 4 waves to rho 16, 8 to 24, then two
// tiles in flight (16 waves at rho 41 to 48); three or four columns at 4 per
// wave, 4 waves, from rho 13 (below: the column split), two tiles in flight
// from rho 17, 8 waves beyond rho 64.  Measured on
// MI355X, us, before -> after: two columns 512 x 2048 3.09 -> 2.86, 2048 x 2048
// 4.14 -> 3.05, 1536 x 1536 4.04 -> 3.03, 2048 x 1024 3.59 -> 2.98, 3072 x 1024
// 4.22 -> 3.05, 4096 x 768 4.38 -> 3.04, 6144 x 2048 5.22 -> 4.09, 8192 x 2048
// 5.63 -> 4.53, 8960 x 1536 5.75 -> 4.62, 11008 x 2048 6.42 -> 5.22, 12288 x
// 768 6.52 -> 4.11, 14336 x 1024 6.80 -> 4.50, 16384 x 2048 7.88 -> 5.98; three
// columns 4096 x 768 4.87 -> 4.11, 5120 x 1024 5.25 -> 4.65, 6144 x 1024 5.51
// -> 4.67, 8192 x 768 6.39 -> 4.66; four columns 4096 x 768 5.18 -> 4.79, 5120
// x 1024 5.54 -> 5.47, 6144 x 1024 5.81 -> 5.48, 8192 x 768 6.95 -> 5.48. Many
// rows per CU: two columns 24576 x 2048 9.57 -> 7.59, 32768 x 2048 11.29 ->
// 8.89, 65536 x 2048 19.01 -> 15.26, 128256 x 2048 32.49 -> 27.50, 32768 x 768
// 10.71 -> 5.55; three columns 12288 x 1024 7.83 -> 5.70, 16384 x 768 8.08 ->
// 5.72; four 12288 x 1024 8.51 -> 6.74, 16384 x 768 9.10 -> 6.80; 151936 x 1024
// two columns 35.79 -> 18.36, 65536 x 1024 three 22.05 -> 11.31 and four 25.29
// -> 13.74 (8 waves beyond rho 64).  Three or four columns of rows of 5 to 8
// blocks (super-blocks w and w + 4 per wave) from rho 5, 4 waves up to rho 32,
// 8 beyond, two tiles in flight from rho 9: 2048 x 2048 three 3.93 -> 3.42,
// four 4.75 -> 4.05, 3072 x 2048 three 4.83 -> 3.93, 8192 x 2048 three 6.48
// -> 4.97, four 7.52 -> 5.59, 8960 x 1536 three 6.59 -> 5.38, 16384 x 2048
// four 9.80 -> 7.72, 128256 x 2048 three 41.36 -> 29.06.  Measured up to rho
// 594; past it the LDS of the partials bounds the rows per workgroup
// (pick_geometry_short_nc).
static bool short_nc_auto(int64_t M, int N, int nb, int cus, int &rows_per_step, int &waves, int &slots) {
    const int64_t rho = (M + cus - 1) / cus;
    slots = 1;
    if (N > 2 && nb > 4) {  // super-blocks w and w + 4 per wave: from 5 rows per CU (below: the column split)
        rows_per_step = 8;
        waves = rho > 32 ? 8 : 4;
        slots = rho > 8 ? 2 : 1;
        return rho > 4;
    }
    if (N == 2) {
        rows_per_step = 8;
        waves = rho <= 16 ? 4 : (rho > 40 && rho <= 48 ? 16 : 8);
        if (rho > 24 && waves == 8) slots = 2;
        return true;
    }
    rows_per_step = 4;
    waves = rho > 64 ? 8 : 4;
    if (rho > 16) slots = 2;
    return rho > 12;
}

// The K-split kernel's automatic launch shape for one aligned F32 column of
// rows of up to 8 groups, one workgroup per CU; false where the tile kernel
// measured faster.  rho = rows per CU.  Measured on MI355X (us, interleaved
// graph timings of 200 calls; K-split against the tile kernel):
//  - K = 4096: up to 4 rows per CU, 4 rows per step and 4 waves (1024 x
//    4096 2.87 against 3.14); up to 8, 8 rows and 8 waves (2048 x 4096 3.19
//    against 3.36).  Beyond, 8 rows per step: with an odd number of 8-row
//    tiles per CU up to 64 rows, two 8-wave teams with one tile in flight
//    (4608 x 4096 4.33 against 4.59, 6144 x 4096 4.69 / 5.02, 13312 x 4096
//    7.39 / 7.60, 14336 x 4096 7.71 / 7.80), otherwise one 8-wave team with
//    two tiles in flight (4096 x 4096 3.98 / 4.37, 7168 x 4096 5.14 / 5.39,
//    12288 x 4096 6.90 / 7.28, 16384 x 4096 8.44 / 8.71, 28672 x 4096
//    13.03 / 13.62, 128256 x 4096 50.30 / 50.79 on the block-per-lane
//    kernel); the two shapes swap at the other parity (14336 x 4096: 7.97
//    against 7.71; 16384 x 4096: 8.45 against 8.44).  160 to 400 rows per
//    CU stay on the tile kernel's four 8-wave workgroups per CU (65536 x
//    4096 26.50 against 26.71-26.84).
//  - K = 8192: the same up to 8 rows per CU (1024 x 8192 3.95 against 4.58,
//    2048 x 8192 4.38 / 5.03), then 4 rows per step, 4 waves and two tiles
//    in flight (4096 x 8192 5.51 / 5.87, 14336 x 8192 12.91 / 13.45, 28672 x
//    8192 23.33 / 24.27).
//  - other lengths up to 8 groups (the long-row variant): up to 4 rows per
//    CU and 4 groups, 4 rows, 4 waves, one step in flight (1024 x 14336
//    5.48 against 5.60 with two and 5.65 on the next shape); up to 8 rows per CU, 8 rows, 8
//    waves, two steps (1024 x 14336 5.56 against 6.65 on the tile kernel,
//    2048 x 14336 5.79 / 7.21, 1024 x 28672 9.33 / 11.11, 2048 x 11008 5.88
//    / 6.09); three or four steps in flight measured slower everywhere but
//    at 1024 x 14336 (4096 x 14336 8.69 and 9.09 against 8.35, 14336 x 14336
//    22.64 and 22.12 against 21.61, 1024 x 14336 at 4 rows 5.40 against
//    5.48); from 9 to 16 rows per CU, 16 rows
//    and 16 waves, one step (4096 x 14336 8.32 / 8.54, 4096 x 11008 6.97 /
//    7.42, 4096 x 5120 4.81 / 5.53, 3584 x 18944 9.91 / 11.89, 3072 x 14336
//    7.47 / 8.02, 2816 x 11008 6.20 / 6.50, 2304 x 9216 5.77 / 6.14; 8 rows,
//    8 waves, two steps 10.28 and 8.19 at the first two, which that rule
//    took only with at most one row in eight idle); beyond, 8 rows, 8
//    waves, two steps where 8-row tiles leave at most one row in eight idle
//    (8192 x 28672
//    25.50 / 28.62, 14336 x 14336 21.55 / 22.46, 13824 x 5120 9.97 / 10.17,
//    32000 x 5120 19.32 / 19.77), the tile kernel otherwise (5120 x 13824,
//    20 rows per CU: 10.23 against 9.50; 16 rows and 16 waves 11.31; 4608 x
//    14336, 18 rows, 10.06 / 9.24) and over 160 rows per CU (not measured);
//    rows under 4096 values as below.
//  - rows of 3 to 8 blocks (768 .. 2048 values; the long-row kernel with
//    teams of only the waves a row needs): 8 rows per step, one step in
//    flight, 4 waves up to 16 rows per CU (512 x 2048 2.60 against 2.88 on
//    the tile kernel, 2048 x 2048 2.81 / 3.15, 4096 x 1024 2.85 / 3.64,
//    1024 x 768 2.51 / 2.81), 8 up to 24 (6144 x 2048 3.84 / 4.40), 16
//    beyond (8960 x 1536 4.13 / 4.90, 16384 x 2048 5.37 / 6.69, 8192 x 2048
//    4.22 / 4.72, 32768 x 2048 8.57 / 9.74, 128256 x 2048 26.44 / 30.31).
//  - rows of 9 to 14 blocks (2304 .. 3584 values): 8 rows per step, two
//    teams of ceil(blocks / 2) waves and one step in flight (2304 x 2304
//    3.60 / 3.82, 9216 x 2304 5.10 / 5.15, 2560 x 2560 3.62 / 3.85, 9728 x
//    2560 5.25 / 5.41, 3072 x 3072 3.73 / 3.83, 8192 x 3072 4.89 / 5.13),
//    one team up to 8 rows per CU (2048 x 2304 3.23 against 3.30 with two,
//    3.24 on the tile kernel); teams of 7 one per workgroup with two steps
//    (3584 x 3584 3.94 / 4.13, 18944 x 3584 8.78 / 9.40); the tile kernel
//    up to 4 rows per CU (512 x 3584 3.07 against 3.17) and over 160
//    (151936 x 2560 40.01 against 40.81).
static bool ksplit_short_auto(int64_t K, int64_t rho, bool glu, int &tr, int &waves, int &slots) {
    const int nb = (int)(K / kQK);
    tr = 8;
    slots = 1;
    if (nb <= 8) {
        waves = rho <= 16 ? 4 : (rho <= 24 || glu ? 8 : 16);
        return true;
    }
    const int kt = (nb + 1) / 2;
    waves = kt == 7 || rho <= 8 ? kt : 2 * kt;
    if (kt == 7 && !glu) slots = 2;
    return rho > 4 && rho <= 160;
}

static bool ksplit_auto(int64_t K, int64_t M, int cus, int &tr, int &waves, int &slots) {
    const int64_t rho = (M + cus - 1) / cus;
    slots = 1;
    if (ksplit_short_rows(K)) return ksplit_short_auto(K, rho, false, tr, waves, slots);
    if (K != 4096 && K != 8192) {
        if (rho <= 4 && K <= 4 * 4096) {
            tr = waves = 4;
            slots = 1;
            return true;
        }
        if (rho > 8 && rho <= 16) {
            tr = waves = 16;
            return true;
        }
        tr = waves = 8;
        slots = 2;
        return rho <= 8 || (rho <= 160 && ((rho + 7) / 8 * 8 - rho) * 8 <= rho);
    }
    if (rho <= 4) {
        tr = 4;
        waves = 4;
        return true;
    }
    if (rho <= 8) {
        tr = 8;
        waves = 8;
        return true;
    }
    if (K == 8192) {
        tr = 4;
        waves = 4;
        slots = 2;
        return true;
    }
    if (rho > 160 && rho <= 400) return false;
    tr = 8;
    if (rho <= 64 && ((rho + 7) / 8) % 2 == 1) {
        waves = 16;
    } else {
        waves = 8;
        slots = 2;
    }
    return true;
}

// The K-split kernel's automatic launch shape for one aligned F32 column
// with a gate weight and the GLU (two weights' rows per step); false where
// the tile kernel is kept.  rho = rows per CU.  Measured on MI355X (us per
// fused op, one process, K-split against the fused tile kernel): rows of
// 4096 values up to 16 rows per CU 8 rows per step and 8 waves, one tile in
// flight (4096 x 4096 5.68 against 6.10), beyond 4 rows, 4 waves, two tiles
// (14336 x 4096 13.45 / 13.71, 11008 x 4096 11.27 / 11.90 -- 4 rows and 8
// waves 10.94 there, 13.98 at 14336 rows); 8192 values 4 rows, 4 waves, one
// tile (28672 x 8192 45.05 / 48.40); other lengths 8 rows, 8 waves, one step
// (4096 x 14336 13.96 / 17.40).  Rows of 4096 values or more, up to 160
// rows per CU: the range measured; rows of 3 to 8 blocks (short teams) 8
// rows per step, 4 waves up to 16 rows per CU, else 8 (2048 x 2048 3.53 /
// 3.97, 5632 x 2048 4.85 / 6.27, 6144 x 2048 5.13 / 6.32, 8192 x 2048 5.93
// / 7.46; MUL_MAT_ID of eight 768 x 2048 experts 5.09 / 6.62); rows of 9 to
// 14 blocks two teams of ceil(blocks / 2) waves (teams of 7: one), one step
// (2560 x 2560 4.66 / 4.81, 9728 x 2560 7.44 / 8.89, 8192 x 3072 7.74 /
// 8.07, 18944 x 3584 15.86 / 16.55).
static bool ksplit_glu_auto(int64_t K, int64_t M, int cus, int &tr, int &waves, int &slots) {
    const int64_t rho = (M + cus - 1) / cus;
    slots = 1;
    if (ksplit_short_rows(K)) return ksplit_short_auto(K, rho, true, tr, waves, slots);
    if (rho > 160 || K < 4096) return false;  // (other rows under 4096 values: not measured)
    if (K == 4096) {
        if (rho <= 16) {
            tr = waves = 8;
        } else {
            tr = waves = 4;
            slots = 2;
        }
        return true;
    }
    tr = waves = K == 8192 ? 4 : 8;
    return true;
}

// The several-column K-split kernel's automatic launch shape (N = 2..4
// aligned F32 columns, rows of 4096 or 8192 values, one workgroup per CU;
// staged: the activation quantised once per workgroup into LDS); false
// where the tile kernel measured faster.  rho = rows per CU.  Measured on
// MI355X (us, interleaved timings of 200 ops; K-split against the tile
// kernel, whose outputs are the same bits):
//  - two columns, K = 4096: up to 16 rows per CU 8 rows per step, 8 waves,
//    one tile in flight (1024 x 4096 3.97 against 4.09, 2048 x 4096 4.12 /
//    4.30, 4096 x 4096 4.86 / 5.26); beyond, an odd number of 8-row tiles
//    per CU up to 64 rows two 8-wave teams with one tile in flight (6144 x
//    4096 5.85 / 6.09, 14336 x 4096 8.53 / 8.94), otherwise one team with
//    two (8192 x 4096 6.00 / 6.82, 16384 x 4096 9.03 / 10.07, 28672 x 4096
//    13.56 / 15.13, 128256 x 4096 52.08 / 54.82); the activation
//    quantised by every wave in registers (staged in LDS: 4096 x 4096 5.29,
//    14336 x 4096 8.86).
//  - two columns, K = 8192: up to 4 rows per CU 4 rows per step and 4
//    waves (1024 x 8192 5.40 / 5.91), else 8 rows and 8 waves, one tile in
//    flight (4096 x 8192 6.78 / 7.25, 14336 x 8192 14.55 / 15.61, 28672 x
//    8192 26.00 / 27.49).
//  - three columns: 4 rows per step, 8 waves, staged; 8192 values up to 4
//    rows per CU, one tile in flight (1024 x 8192 7.11 / 8.09; 4096 x 8192
//    stays on the tile kernel: 9.57 against 8.37); 4096 values over 4 and
//    up to 16 rows per CU, two (4096 x 4096 5.52 / 5.69 over three
//    alternations; 1024 x 4096 stays on the tile kernel: 4.62 against
//    4.51).
//  - three or four columns, K = 8192, 96 rows per CU or more: 4 rows, 4
//    waves, two tiles in flight, in registers (28672 x 8192 N=3 28.63 /
//    29.19, N=4 30.28 / 32.03).
//  - rows of other lengths over 8192 values (the long-row form, staged): 4 rows per step
//    and 16 waves (four teams; two columns: 4 super-blocks per wave).  Two
//    columns: two tiles in flight where a wave's steps are even in number,
//    else one (4096 x 14336 10.52 against 10.94, 1024 x 14336 7.90 / 8.94,
//    14336 x 14336 24.82 / 25.20, 8192 x 28672 30.44 / 31.54, 4096 x 11008
//    9.06 / 9.30); three or four columns up to 16384 values, one tile in
//    flight, two up to 4 rows per CU (4096 x 14336 N=3 13.15 against 14.5-15.9
//    with the quantiser launch, N=4 16.11 / 17.29, 1024 x 14336 N=4 11.51 /
//    11.97, 4096 x 11008 N=4 12.29 / 13.75; 8192 x 28672 N=4 40.02 / 38.17
//    stays on the tile kernel).  Staged in the tile kernel's layout, with
//    the super-block positions unpermuted, the reads of the four-column tree
//    conflicted four ways (4096 x 14336 N=4 18.39, 8192 x 28672 N=4 47.37).
//  The tile kernel elsewhere: four columns of 4096 values (14336 x 4096
//  10.97 staged against 10.68, 4096 x 4096 6.47 / 6.29), 56 rows per CU of
//  8192 values (14336 x 8192 N=3 17.54 / 16.77, N=4 19.06 / 18.88).
//  Up to 12 rows per CU (8 with two columns) split_columns comes first: the
//  columns as one-column channels of one launch.
static bool ksplit_nc_auto(int64_t K, int64_t M, int64_t N, int cus, int &tr, int &waves, int &slots,
                           int &staged) {
    const int64_t rho = (M + cus - 1) / cus;
    if (K != 4096 && K != 8192) {
        if (K < 8192) return false;  // rows shorter than two groups: not measured
        tr = 4;
        waves = 16;
        staged = 1;
        if (N == 2) {
            const int64_t G = (K / kQK + 15) / 16;
            const int64_t steps = ((rho + 3) / 4 + 3) / 4 * G;  // per wave: tiles per team x groups
            slots = steps % 2 == 0 ? 2 : 1;
            return true;
        }
        slots = rho <= 4 ? 2 : 1;
        return K <= 16384;
    }
    staged = 0;
    slots = 1;
    if (N == 2) {
        if (K == 8192) {
            tr = waves = rho <= 4 ? 4 : 8;
            return true;
        }
        tr = 8;
        waves = 8;
        if (rho <= 16) return true;
        if (rho <= 64 && ((rho + 7) / 8) % 2 == 1) waves = 16;
        else slots = 2;
        return true;
    }
    tr = 4;
    if (N == 3 && (K == 8192 ? rho <= 4 : rho > 4 && rho <= 16)) {
        waves = 8;
        staged = 1;
        slots = rho <= 4 ? 1 : 2;
        return true;
    }
    if (K == 8192 && rho >= 96) {
        waves = 4;
        slots = 2;
        return true;
    }
    return false;
}

// Several columns over few rows per CU: every workgroup of a several-column
// launch quantises (or stages) all N columns for its few rows, so the
// columns go to one launch of one-column products instead, column c as
// dst channel c of a broadcast batched launch (the weight shared, grid y =
// columns), whose workgroups quantise one column each.  Each column then
// carries the one-column product's bits, on both routes (F32: the
// one-column K-split kernel; pre-quantised: the one-column tile kernel).
// Measured on MI355X (us, N columns in one launch against N one-column
// channels, same buffers): 512 x 4096 N=4 4.97 -> 3.56, N=8 7.27 -> 3.93;
// 1024 x 4096 N=2 3.98 -> 3.59, N=3 4.48 -> 4.18, N=4 5.16 -> 3.98, N=8
// 7.29 -> 4.69; 2048 x 4096 N=3 5.48 -> 5.20, N=4 5.41 -> 4.75, N=8 7.65 ->
// 6.23; 3072 x 4096 N=4 6.01 -> 5.58, N=8 8.12 -> 7.76; 1024 x 8192 N=4
// 8.02 -> 5.44; 1024 x 14336 N=4 11.95 -> 7.23, N=8 16.00 -> 10.21; 1024 x
// 2048 N=8 5.57 -> 5.11; Q6_K 1024 x 4096 N=4 5.59 -> 5.01, N=8 7.92 ->
// 6.64.  Not at 4096 rows (4096 x 4096 N=2 4.86 -> 5.08, N=4 6.29 -> 6.42)
// nor beyond; two columns only up to 8 rows per CU (2048 x 4096: 4.12 ->
// 4.11).
bool split_columns(int64_t K, int64_t M, int64_t N, int cus) {
    if (N < 2 || N > Q4K_MAX_BATCH || cus < 1) return false;
    const int64_t rho = (M + cus - 1) / cus;
    // rows shorter than one group of 5 or more blocks: up to 4 rows per CU
    // (from 5 the tile kernel measured faster: 2048 x 2048 N=3 4.46 against
    // 3.91 us, N=4 5.15 / 4.71, 1536 x 1536 N=3 4.37 / 3.89, 2048 x 3584 N=3
    // 5.79 / 4.44, N=2 4.35 / 4.06, 2048 x 2304 N=2 4.08 / 3.86, Q6_K 2048 x
    // 2048 N=3 4.81 / 4.26; at up to 4 the split: 512 x 2048 N=4 3.08 / 4.04,
    // 1024 x 2560 N=4 4.18 / 4.53)
    const int64_t lim = K < 4096 && K > 1024 ? 4 : (N == 2 ? 8 : 12);
    return rho <= lim && K <= 8 * 4096 && (K >= 4096 || ksplit_short_rows(K));
}

// Launch geometry for an (M, K, N) product.
//  tile kernel: one workgroup per CU (requesting just over half the CU's LDS
//    keeps a second one away), 8 or 16 waves, the M rows split evenly over
//    all waves, one row per tile and two groups in flight per wave (larger
//    tiles and deeper pipelines measured slower on MI355X: the activation
//    prologue is the critical path and more weight requests in flight delay
//    its loads).
//  block-per-lane kernel (one column, 16..64 super-blocks per row): 4-wave
//    workgroups, 2 per CU, two passes per wave in flight.
//  fused epilogue (bias and/or gate, one column): the tile kernel only; with
//    a gate each tile pairs one row of both weights (R = 2, one or two
//    groups in flight).
static Geometry pick_geometry(const DeviceInfo &di, int64_t K, int64_t M, int64_t N, int fused = 0,
                              int64_t mats = 1, bool f32_vec = true, bool q81 = false) {
    Geometry g;
    const int max_lds = di.max_lds > 0 ? di.max_lds : 65536;
    const int cus = di.cus > 0 ? di.cus : 1;
    int nc = (int)N;
    while (nc > 1 && tile_lds_bytes((int)K, nc, 16) > max_lds) nc = (nc + 1) / 2;
    g.nc_chunk = nc;
    g.lds = tile_lds_bytes((int)K, nc, 16);
    const int orows = g_ovr_rows.load(), owaves = g_ovr_waves.load(), owgs = g_ovr_wgs.load();
    const int okern = g_ovr_kernel.load();
    const int rpw = bpl_rows_per_pass(K / kQK);
    // several columns of rows shorter than one group: short teams (aligned
    // F32 columns, automatic only; before the column split, which these
    // shapes measured slower)
    if (!fused && mats == 1 && okern == 0 && orows == 0 && owaves == 0 && owgs == 0 && f32_vec && N >= 2 &&
        N <= 4 && short_nc_ok(K, (int)N, nc)) {
        int tr = 0, w = 0, s = 0;
        if (short_nc_auto(M, (int)N, (int)(K / kQK), cus, tr, w, s)) {
            const Geometry gs = pick_geometry_short_nc(di, K, M, (int)N, tr, w, 0, s);
            if (gs.ksplit) return gs;
        }
    }
    // several columns over few rows: one-column channels (automatic only;
    // where the aligned F32 column takes the K-split kernel, so both routes
    // decide alike)
    if (!fused && mats == 1 && okern == 0 && orows == 0 && owaves == 0 && owgs == 0 && split_columns(K, M, N, cus) &&
        pick_geometry(di, K, M, 1, 0, N, true, false).ksplit) {
        Geometry g1 = pick_geometry(di, K, M, 1, 0, N, f32_vec, q81);
        g1.colsplit = (int)N;
        g1.nc_chunk = (int)N;
        return g1;
    }
    // K-split kernel: one 16-byte aligned F32 column of rows of up to 8
    // groups (4096 or 8192 values: activation in registers; other lengths:
    // the long-row variant); the tile kernel, whose outputs are the same
    // bits, takes the rest
    // (fused epilogues and batched launches included; a batched launch's
    // workgroups per weight matrix: grid_per_matrix.  Batched, rows of 4096
    // values or more and rows of 3 to 8 blocks (short teams): MUL_MAT_ID
    // measured on MI355X, Mixtral 8x7B gate/up with SWIGLU, Q4_K, 26.61 ->
    // 25.27 us, down, Q6_K, 22.27 -> 19.64; Qwen3-30B-A3B-like gate/up 6.62
    // -> 5.09, down 7.73 -> 4.43; other lengths under 4096 values not
    // measured)
    const bool ks_ok = N == 1 && f32_vec && K <= 8 * 4096 &&
                       (mats == 1 || K >= 4096 || okern == 5 || ksplit_short_rows(K));
    const int cus_m = mats > 1 ? grid_per_matrix(cus, mats, M) : cus;
    // two to four columns: the K-split kernel for rows of 1 or 2 groups
    // (the tile kernel's launches, whose bits these are: all columns in one,
    // or four columns two by two)
    const bool ksn_ok = N >= 2 && N <= 4 && !fused && mats == 1 && f32_vec && K <= 8 * 4096 &&
                        (nc == N || (nc == 2 && N == 4));
    const int ksn_p = nc <= 2 ? 2 : 4;
    // several columns of rows shorter than one group: short teams
    const bool snc_ok = ksn_ok && short_nc_ok(K, (int)N, nc);
    if (snc_ok && okern == 5) {
        const Geometry gs = pick_geometry_short_nc(di, K, M, (int)N, orows, owaves, owgs, g_ovr_slots.load());
        if (gs.ksplit) return gs;
    }
    if (ksn_ok && okern == 5)
        return pick_geometry_ksplit(di, K, M, orows, owaves, owgs, g_ovr_slots.load(), (int)N, 1, ksn_p);
    if (ks_ok && okern == 5) {
        const Geometry gk = pick_geometry_ksplit(di, K, M, orows, owaves, owgs > 0 ? owgs : (mats > 1 ? cus_m : 0),
                                                 g_ovr_slots.load(), 1, 0, 0, fused, mats > 1);
        if (gk.ksplit) return gk;
    }
    // (automatic: where the partials fit the LDS)
    if (ks_ok && okern == 0 && orows == 0 && owaves == 0 && owgs == 0) {
        int tr = 0, kw = 0, ks = 0;
        if (fused == kFusedGate ? ksplit_glu_auto(K, M, cus_m, tr, kw, ks) : ksplit_auto(K, M, cus_m, tr, kw, ks)) {
            const int os = g_ovr_slots.load();
            const Geometry gk = pick_geometry_ksplit(di, K, M, tr, kw, mats > 1 ? cus_m : 0,
                                                     os >= 1 && os <= 4 ? os : ks, 1, 0, 0, fused, mats > 1);
            if (gk.ksplit && gk.lds <= max_lds && (mats == 1 || K >= 4096 || gk.ks_kt)) return gk;
        }
    }
    if (ksn_ok && okern == 0 && orows == 0 && owaves == 0 && owgs == 0) {
        int tr = 0, kw = 0, ks = 0, st = 0;
        if (ksplit_nc_auto(K, M, N, cus, tr, kw, ks, st)) {
            const int os = g_ovr_slots.load();
            const Geometry gk =
                pick_geometry_ksplit(di, K, M, tr, kw, 0, os == 1 || os == 2 ? os : ks, (int)N, st, ksn_p);
            if (gk.lds <= max_lds) return gk;
        }
    }
    if (N == 1 && rpw > 0 && okern == 3 && !fused && mats == 1) {
        // block kernel: ~2 waves per SIMD; activation + one 9216-byte LDS
        // slot per wave
        g.bpl = 2;
        g.rpw = rpw;
        g.waves = 8;  // the kernel's compile-time workgroup size
        g.ntiles = (int)((M + rpw - 1) / rpw);
        const int wg_needed = (g.ntiles + g.waves - 1) / g.waves;
        int wgs = cus;
        if (owgs > 0) wgs = owgs;
        g.grid = wg_needed < wgs ? wg_needed : wgs;
        g.lds = lds_bytes_linear((int)K);
        g.lds_launch = g.lds + g.waves * kSlotBytes;
        return g;
    }
    // The block-per-lane kernel (override 2) measured 0.2-1 % faster than
    // the tile kernel on one column of >= 256 MB of 4096-value rows (128256
    // x 4096 50.70 against 50.90 us), but sums in another order; it is not
    // chosen automatically, so the pre-quantised route (tile kernel) gives
    // the F32 route's (K-split kernel's) bits there too.
    const int64_t weight_bytes = M * (K / kQK) * kBlockBytes;
    if (N == 1 && rpw > 0 && okern == 2 && !fused && mats == 1) {
        // ~173 VGPRs: two waves per SIMD; 4-wave workgroups, two per CU
        g.bpl = 1;
        g.rpw = rpw;
        g.waves = (owaves == 4 || owaves == 8) ? owaves : 4;
        g.ntiles = (int)((M + rpw - 1) / rpw);
        const int wg_needed = (g.ntiles + g.waves - 1) / g.waves;
        int wgs = cus * (8 / g.waves);
        if (owgs > 0) wgs = owgs;
        g.grid = wg_needed < wgs ? wg_needed : wgs;
        g.lds = lds_bytes_linear((int)K);
        g.lds_launch = g.lds;
        return g;
    }
    // the matrix-core kernel with its A operand from the Q8_1 buffer: the
    // pre-quantised route, up to 8 columns in one launch
    if (q81 && !fused && mats == 1 && N <= kMfmaCols &&
        (okern == 6 || (okern == 0 && use_mfma_ga(M, N, K) &&
                         !(use_mfma(M, N, K) && mfma_lds_bytes((int)K, (int)N, 16) <= max_lds))))
        return pick_geometry_mfma(di, K, M, (int)N, owgs, owaves, true);
    if (!fused && mats == 1 && (okern == 4 || (okern == 0 && use_mfma(M, N, K)))) {
        int mc = (int)N;
        while (mc > 1 && mfma_lds_bytes((int)K, mc, 16) > max_lds) mc = (mc + 1) / 2;
        if (mfma_lds_bytes((int)K, mc, 16) <= max_lds && (okern == 4 || mc == N))
            return pick_geometry_mfma(di, K, M, mc, owgs, owaves);
    }
    g.grid = owgs > 0 ? owgs : grid_per_matrix(cus, mats, M);
    // One column with rows of at most 8192 values and ~500 KB or more of
    // weight per CU: four 8-wave workgroups per CU, all resident, keep
    // twice the weight requests in flight of one 16-wave workgroup, which
    // pays off once the stream is long enough to amortise the extra
    // activation staging (measured on MI355X: 28672 x 8192 27.2 -> 25.2 us,
    // 32768 x 8192 28.6 -> 27.5 us; 20480 x 8192 even, and slower for
    // shorter streams, longer rows or several columns).
    const bool four_per_cu = owgs == 0 && owaves == 0 && N == 1 && !fused && mats == 1 && K <= 8192 &&
                             weight_bytes >= (int64_t)500000 * cus;
    if (four_per_cu) g.grid = 4 * cus;
    // One column with rows of three or more groups and >= 192 steps per CU:
    // two 16-wave workgroups per CU with one group in flight per wave
    // (measured on MI355X: 8192 x 28672 30.0 -> 28.5 us, 14336 x 14336
    // 23.4 -> 22.7 us; 8192 x 14336, 128 steps, 5 % slower).
    const int64_t G = (K / kQK + 15) / 16;
    const bool two_per_cu = owgs == 0 && owaves == 0 && N == 1 && !fused && mats == 1 && !four_per_cu && G >= 3 &&
                            (M + cus - 1) / cus * G >= 192;
    if (two_per_cu) g.grid = 2 * cus;
    // 16 waves per CU unless the product is small (under 12 steps per
    // workgroup; 12-15 steps measured 2-4 % faster at 16 than at 8, e.g.
    // 3584 x 3584 4.38 -> 4.24 us, and 4 steps 6 % slower); two groups in
    // flight per wave once a wave has four or more to stream, else one (a
    // second slot would mostly run past the wave's rows).  Measured on MI355X.
    // Small products with an activation of 32768 or more values (all
    // columns) take 16 waves too: they halve the quantisation rounds that
    // dominate them (1024 x 8192 N=4 9.44 -> 8.30 us, N=8 13.24 -> 11.52;
    // 1024 x 4096 N=8 7.60 -> 7.31; at 28672 values 1 % slower).
    const int64_t steps_per_wg = (M + g.grid - 1) / g.grid * ((K / kQK + 15) / 16);
    g.waves = (steps_per_wg >= 12 || N * K >= 32768) && !four_per_cu ? 16 : 8;
    // Three or more columns with rows of one group and >= 96 rows per
    // workgroup (>= 48 from six columns on): 8 waves, whose registers hold
    // the lane's activation slices of every column, so the step loop reads
    // no LDS (at 16 waves it reads the whole activation from LDS once per
    // row, ~14 bytes per weight byte at 8 columns).  Measured on MI355X:
    // 128256 x 4096 N=8 96 -> 83 us, N=4 63.6 -> 59.3 us, 28672 x 4096 N=4
    // 20.6 -> 16.9 us, 14336 x 4096 N=8 16.5 -> 15.8 us; N=3..5 at
    // 14336 x 4096 (56 rows) even to 3 % slower.
    // From 64 rows per workgroup at three to five columns (18944 x 4096 N=3
    // 13.4 -> 11.6 us, N=4 14.9 -> 13.1; 18944 x 3584 N=4 14.4 -> 12.4).
    const int64_t rows_per_wg = (M + g.grid - 1) / g.grid;
    if (N >= 3 && K <= 16 * kQK && !fused && mats == 1 && (rows_per_wg >= 64 || (N >= 6 && rows_per_wg >= 48)))
        g.waves = 8;
    // Two columns with rows of two groups and at most 32 rows per workgroup:
    // 8 waves (5120 x 5120 7.67 -> 7.02 us, 5120 x 8192 9.2 -> 8.8, 8192 x
    // 5120 8.8 -> 8.2, 8192 x 8192 10.9 -> 10.5; 56 rows and more 1-2 %
    // slower that way).
    if (N == 2 && G == 2 && !fused && mats == 1 && rows_per_wg <= 32) g.waves = 8;
    if (owaves >= 1 && owaves <= 16) g.waves = owaves > 8 ? 16 : 8;  // the instantiated sizes
    g.slots = steps_per_wg >= 4 * (int64_t)g.waves ? 2 : 1;
    if (two_per_cu) g.slots = 1;
    // One column with rows of one group: one slot up to 8 steps per wave
    // (20480 x 4096 10.87 -> 10.53 us, 18944 x 3584 9.71 -> 9.52 us; rows of
    // four groups keep two: 5120 x 13824 9.60 against 11.13 us).
    if (N == 1 && !fused && mats == 1 && !four_per_cu && g.waves == 16 && G == 1 && steps_per_wg < 128)
        g.slots = 1;
    // One column, rows of two groups, at most 8 rows per workgroup: 8 waves
    // with both of a row's groups in flight (2048 x 8192 5.21 -> 4.63 us,
    // 1024 x 8192 4.72 -> 4.33 us; 16 rows, 4096 x 8192, 2 % slower).
    if (N == 1 && !fused && mats == 1 && owaves == 0 && G == 2 && rows_per_wg <= 8) {
        g.waves = 8;
        g.slots = 2;
    }
    g.R = 1;
    if (orows == 1 || orows == 2 || orows == 4) g.R = orows;
    const int oslots = g_ovr_slots.load();
    if (oslots == 1 || oslots == 2 || oslots == 4 || oslots == 8) g.slots = oslots;
    // only the variants that fit the register file without spilling exist
    if (!tile_fits(nc, g.R, g.waves, g.slots)) g.waves = 8;  // (8 fits every R, slots <= 4 variant)
    if (!tile_fits(nc, g.R, g.waves, g.slots)) g.slots = g.slots == 8 ? 4 : 2;
    if (!tile_fits(nc, g.R, g.waves, g.slots)) g.slots = 2;
    if (!tile_fits(nc, g.R, g.waves, g.slots)) g.R = 2;
    if (fused) {
        g.R = fused == kFusedGate ? 2 : 1;  // with a gate: the weight row and the gate row
        if (g.slots > 2) g.slots = 2;
    }
    // With a gate and under 96 rows per CU: 8 waves, one (row, gate row)
    // step in flight per wave, and from 48 rows per CU two workgroups per CU
    // (measured on MI355X: 4096 x 4096 6.84 -> 6.18 us, 11008 x 4096
    // 12.27 -> 11.90, 14336 x 4096 14.31 -> 14.00, 14336 x 8192 25.35 ->
    // 24.64; 28672 x 8192, 112 rows per CU, 3 % slower that way).
    bool glu_two = false;
    const int64_t rows_per_cu = (M + cus - 1) / cus;
    if (fused == kFusedGate && mats == 1 && owaves == 0 && owgs == 0 && rows_per_cu < 96) {
        g.waves = 8;
        g.slots = 1;
        if (rows_per_cu >= 48) {
            g.grid = 2 * cus;
            glu_two = true;
        }
    }
    const bool glu = fused != kFusedNone;
    // rows per workgroup (the kernel splits each share over its waves)
    g.rows_base = (int)(M / g.grid);
    g.rows_extra = (int)(M % g.grid);
    g.lds = tile_lds_bytes((int)K, nc, g.waves);
    g.lds_launch = g.lds;
    if (owgs == 0 && !four_per_cu && !two_per_cu && !glu_two && g.lds_launch <= max_lds / 2)
        g.lds_launch = max_lds / 2 + 256;
    // weight loads before quantisation only when every activation load fits
    // the staging rounds issued ahead of them
    const bool pro0_ok = (int64_t)nc * (K / 32) <= (int64_t)stage_capacity(stage_lpb(nc), g.waves * kWave, nc);
    g.prologue = pro0_ok ? 0 : 1;
    // One column and two slots on streams of under 8 steps per wave: one
    // early group instead of two (measured on MI355X: 4096 x 14336 9.06 ->
    // 8.63 us, 5120 x 13824 10.13 -> 9.63, 20480 x 4096 11.16 -> 10.85,
    // 8192 x 8192 9.61 -> 8.85 (against the streamed prologue below),
    // 11008 x 8192 11.42 -> 11.18; 8192 x 28672, 14 steps per wave, 1 %
    // slower).  Longer two-group streams keep the streamed prologue.
    if (pro0_ok && nc == 1 && g.slots == 2 && !glu && steps_per_wg < 8 * g.waves) g.prologue = 3;
    const int opro = g_ovr_prologue.load();
    if (opro == 1 || ((opro == 0 || (opro == 2 && g.slots >= 4) || (opro == 3 && g.slots == 2 && !glu)) && pro0_ok))
        g.prologue = opro;
    return g;
}

template <int NC, int R, int WAVES, int S>
static const void *gemv_sym(int pro) {
    if constexpr (tile_fits(NC, R, WAVES, S)) {
        if (pro == 0) return reinterpret_cast<const void *>(&gemv_q4k_kernel<NC, R, WAVES, 0, S, kEpiNone>);
        if (pro == 1) return reinterpret_cast<const void *>(&gemv_q4k_kernel<NC, R, WAVES, 1, S, kEpiNone>);
        if constexpr (S >= 4) {
            if (pro == 2) return reinterpret_cast<const void *>(&gemv_q4k_kernel<NC, R, WAVES, 2, S, kEpiNone>);
        }
        if constexpr (S == 2) {
            if (pro == 3) return reinterpret_cast<const void *>(&gemv_q4k_kernel<NC, R, WAVES, 3, S, kEpiNone>);
        }
    }
    return nullptr;
}

template <int R, int WAVES, int S>
static const void *gemv_sym_nc(int nc, int pro) {
    switch (nc) {
        case 1: return gemv_sym<1, R, WAVES, S>(pro);
        case 2: return gemv_sym<2, R, WAVES, S>(pro);
        case 3: return gemv_sym<3, R, WAVES, S>(pro);
        case 4: return gemv_sym<4, R, WAVES, S>(pro);
        case 5: return gemv_sym<5, R, WAVES, S>(pro);
        case 6: return gemv_sym<6, R, WAVES, S>(pro);
        case 7: return gemv_sym<7, R, WAVES, S>(pro);
        case 8: return gemv_sym<8, R, WAVES, S>(pro);
        default: return nullptr;
    }
}

template <int WAVES, int S>
static const void *gemv_sym_r(int nc, int R, int pro) {
    if (R == 1) return gemv_sym_nc<1, WAVES, S>(nc, pro);
    if (R == 2) return gemv_sym_nc<2, WAVES, S>(nc, pro);
    return gemv_sym_nc<4, WAVES, S>(nc, pro);
}

// Instantiations: R in {1, 2, 4}; launch bounds of 8 or 16 waves; 2 or 4
// slots (see tile_fits); both prologue orders.
template <int EPI, int WAVES, int S, bool BATCH>
static const void *gemv_sym_epi(int pro) {
    constexpr int R = EPI == kEpiGlu ? 2 : 1;
    return pro == 0 ? reinterpret_cast<const void *>(&gemv_q4k_kernel<1, R, WAVES, 0, S, EPI, BATCH>)
                    : reinterpret_cast<const void *>(&gemv_q4k_kernel<1, R, WAVES, 1, S, EPI, BATCH>);
}

// The fused-epilogue variants (bias, or gate + GLU): one column, 8 or 16
// waves, 1 or 2 slots, both prologue orders, plain or batched.
template <int EPI, bool BATCH>
static const void *gemv_kernel_epi(int waves, int pro, int slots) {
    if (pro != 0 && pro != 1) return nullptr;
    if (waves <= 8) return slots == 1 ? gemv_sym_epi<EPI, 8, 1, BATCH>(pro) : gemv_sym_epi<EPI, 8, 2, BATCH>(pro);
    return slots == 1 ? gemv_sym_epi<EPI, 16, 1, BATCH>(pro) : gemv_sym_epi<EPI, 16, 2, BATCH>(pro);
}

template <int NC, int WAVES, int S>
static const void *gemv_sym_batch(int pro) {
    return pro == 0 ? reinterpret_cast<const void *>(&gemv_q4k_kernel<NC, 1, WAVES, 0, S, kEpiNone, true>)
                    : reinterpret_cast<const void *>(&gemv_q4k_kernel<NC, 1, WAVES, 1, S, kEpiNone, true>);
}

template <int WAVES, int S>
static const void *gemv_sym_batch_nc(int nc, int pro) {
    switch (nc) {
        case 1: return gemv_sym_batch<1, WAVES, S>(pro);
        case 2: return gemv_sym_batch<2, WAVES, S>(pro);
        case 3: return gemv_sym_batch<3, WAVES, S>(pro);
        case 4: return gemv_sym_batch<4, WAVES, S>(pro);
        case 5: return gemv_sym_batch<5, WAVES, S>(pro);
        case 6: return gemv_sym_batch<6, WAVES, S>(pro);
        case 7: return gemv_sym_batch<7, WAVES, S>(pro);
        case 8: return gemv_sym_batch<8, WAVES, S>(pro);
        default: return nullptr;
    }
}

// Batched variants (channels/samples, MUL_MAT_ID): one row per tile, 8 or
// 16 waves, 1 or 2 slots, both prologue orders.
static const void *gemv_kernel_batch(int nc, int waves, int pro, int slots) {
    if (pro != 0 && pro != 1) return nullptr;
    if (waves <= 8) return slots == 1 ? gemv_sym_batch_nc<8, 1>(nc, pro) : gemv_sym_batch_nc<8, 2>(nc, pro);
    return slots == 1 ? gemv_sym_batch_nc<16, 1>(nc, pro) : gemv_sym_batch_nc<16, 2>(nc, pro);
}

static const void *gemv_kernel_for(int nc, int R, int waves, int pro, int slots) {
    if (waves <= 8) {
        if (slots == 8) return gemv_sym_r<8, 8>(nc, R, pro);
        if (slots == 1) return gemv_sym_r<8, 1>(nc, R, pro);
        return slots == 4 ? gemv_sym_r<8, 4>(nc, R, pro) : gemv_sym_r<8, 2>(nc, R, pro);
    }
    if (slots == 1) return gemv_sym_r<16, 1>(nc, R, pro);
    return slots == 4 ? gemv_sym_r<16, 4>(nc, R, pro) : gemv_sym_r<16, 2>(nc, R, pro);
}

template <int WAVES>
static const void *mfma_kernel_nc(int nc) {
    switch (nc) {
        case 1: return reinterpret_cast<const void *>(&gemv_q4k_mfma_kernel<1, WAVES>);
        case 2: return reinterpret_cast<const void *>(&gemv_q4k_mfma_kernel<2, WAVES>);
        case 3: return reinterpret_cast<const void *>(&gemv_q4k_mfma_kernel<3, WAVES>);
        case 4: return reinterpret_cast<const void *>(&gemv_q4k_mfma_kernel<4, WAVES>);
        case 5: return reinterpret_cast<const void *>(&gemv_q4k_mfma_kernel<5, WAVES>);
        case 6: return reinterpret_cast<const void *>(&gemv_q4k_mfma_kernel<6, WAVES>);
        case 7: return reinterpret_cast<const void *>(&gemv_q4k_mfma_kernel<7, WAVES>);
        case 8: return reinterpret_cast<const void *>(&gemv_q4k_mfma_kernel<8, WAVES>);
        default: return nullptr;
    }
}

static const void *mfma_kernel_for(int nc, int waves) {
    return waves > 8 ? mfma_kernel_nc<16>(nc) : mfma_kernel_nc<8>(nc);
}

template <int NIF>
static const void *mfma_ga_kernel_nc(int nc) {
    switch (nc) {
        case 1: return reinterpret_cast<const void *>(&gemv_q4k_mfma_kernel<1, 8, false, true, NIF>);
        case 2: return reinterpret_cast<const void *>(&gemv_q4k_mfma_kernel<2, 8, false, true, NIF>);
        case 3: return reinterpret_cast<const void *>(&gemv_q4k_mfma_kernel<3, 8, false, true, NIF>);
        case 4: return reinterpret_cast<const void *>(&gemv_q4k_mfma_kernel<4, 8, false, true, NIF>);
        case 5: return reinterpret_cast<const void *>(&gemv_q4k_mfma_kernel<5, 8, false, true, NIF>);
        case 6: return reinterpret_cast<const void *>(&gemv_q4k_mfma_kernel<6, 8, false, true, NIF>);
        case 7: return reinterpret_cast<const void *>(&gemv_q4k_mfma_kernel<7, 8, false, true, NIF>);
        case 8: return reinterpret_cast<const void *>(&gemv_q4k_mfma_kernel<8, 8, false, true, NIF>);
        default: return nullptr;
    }
}

// GA: 8-wave workgroups, 2 or 4 items in flight per wave
static const void *mfma_ga_kernel_for(int nc, int waves, int nif) {
    if (waves != 8) return nullptr;
    return nif == 4 ? mfma_ga_kernel_nc<4>(nc) : mfma_ga_kernel_nc<2>(nc);
}

static int launch_gemv(DeviceInfo *di, const Geometry &geo, GemvParams p, int nc, hipStream_t stream,
                       const BatchLaunch *bl = nullptr) {
    const void *fn = nullptr;
    const bool batch = bl != nullptr;
    if (batch && geo.bpl) return Q4K_EINVAL;
    if ((p.gate || p.bias) && !geo.ksplit) {
        if (nc != 1 || geo.bpl || geo.R != (p.gate ? 2 : 1)) return Q4K_EINVAL;
        if (p.gate)
            fn = batch ? gemv_kernel_epi<kEpiGlu, true>(geo.waves, geo.prologue, geo.slots)
                       : gemv_kernel_epi<kEpiGlu, false>(geo.waves, geo.prologue, geo.slots);
        else
            fn = batch ? gemv_kernel_epi<kEpiBias, true>(geo.waves, geo.prologue, geo.slots)
                       : gemv_kernel_epi<kEpiBias, false>(geo.waves, geo.prologue, geo.slots);
        p.rows_base = geo.rows_base;
        p.rows_extra = geo.rows_extra;
        p.ring_off = lds_bytes(p.K, nc);
    } else if (batch && !geo.ksplit) {
        if (geo.R != 1) return Q4K_EINVAL;
        fn = gemv_kernel_batch(nc, geo.waves, geo.prologue, geo.slots);
        p.rows_base = geo.rows_base;
        p.rows_extra = geo.rows_extra;
        p.ring_off = lds_bytes(p.K, nc);
    } else if (geo.ksplit) {
        if (!p.x || !p.vec_ok) return Q4K_EINVAL;
        if (nc > 1 && geo.ks_snc) {
            if (nc != geo.nc_chunk) return Q4K_EINVAL;
            fn = q4k_ksplit_short_nc_kernel(nc, geo.ksplit, geo.ks_kt, geo.waves, geo.slots, p.sums != nullptr,
                                            geo.ks_snc);
            p.ring_off = ksplit_short_nc_part_bytes(geo.rows_base + (geo.rows_extra ? 1 : 0), nc, geo.ks_kt);
        } else if (nc > 1) {
            if (nc != geo.nc_chunk) return Q4K_EINVAL;
            if (geo.ks_long)
                fn = p.sums ? q4k_ksplit_nc_long_sums_kernel(nc, geo.ks_p, geo.ksplit, geo.waves, geo.slots)
                            : ksplit_nc_long_kernel<false>(nc, geo.ks_p, geo.ksplit, geo.waves, geo.slots);
            else
                fn = p.sums ? q4k_ksplit_nc_sums_kernel(nc, geo.ksplit, geo.waves, geo.slots, p.G, geo.ks_staged != 0)
                            : ksplit_nc_kernel<false>(nc, geo.ksplit, geo.waves, geo.slots, p.G, geo.ks_staged != 0);
            p.ring_off = geo.ks_staged ? ksn_stage_bytes(p.K, nc) : 0;
        } else if (geo.ks_long && geo.ks_kt) {
            const int epi = p.gate ? kEpiGlu : (p.bias ? kEpiBias : kEpiNone);
            fn = q4k_ksplit_short_kernel(geo.ksplit, geo.ks_kt, geo.waves, geo.slots, p.sums != nullptr, epi, batch);
            p.ring_off = ksplit_long_part_bytes(geo.rows_base + (geo.rows_extra ? 1 : 0), geo.ksplit,
                                                p.gate ? 2 : 1, geo.ks_kt);
            p.rpw = 1;
        } else if (geo.ks_long) {
            if (batch)
                fn = p.gate   ? ksplit_long_kernel_epi<kEpiGlu, true>(geo.ksplit, geo.waves, geo.slots, p.G)
                     : p.bias ? ksplit_long_kernel_epi<kEpiBias, true>(geo.ksplit, geo.waves, geo.slots, p.G)
                              : ksplit_long_kernel_epi<kEpiNone, true>(geo.ksplit, geo.waves, geo.slots, p.G);
            else if (p.gate)
                fn = ksplit_long_kernel_epi<kEpiGlu>(geo.ksplit, geo.waves, geo.slots, p.G);
            else if (p.bias)
                fn = ksplit_long_kernel_epi<kEpiBias>(geo.ksplit, geo.waves, geo.slots, p.G);
            else
                fn = p.sums ? q4k_ksplit_long_sums_kernel(geo.ksplit, geo.waves, geo.slots, p.G)
                            : ksplit_long_kernel<false>(geo.ksplit, geo.waves, geo.slots, p.G);
            p.ring_off = ksplit_long_part_bytes(geo.rows_base + (geo.rows_extra ? 1 : 0), geo.ksplit, p.gate ? 2 : 1);
            // groups quantised before the first step: all of them for one
            // super-block per wave and group (4096 x 14336 8.27 against 8.39
            // us, 4096 x 11008 6.97 / 7.02), else one, the others just before
            // the first step that reads them (8192 x 28672 25.10 against
            // 25.60); the pipeline override's prologue 2 forces all, 0, 1 or 3
            // one
            const int opro = g_ovr_prologue.load();
            p.rpw = (opro == 2 || (opro < 0 && geo.ksplit == 1)) ? p.G : 1;
        } else if (batch) {
            fn = p.gate   ? ksplit_kernel_epi<kEpiGlu, true>(geo.ksplit, geo.waves, geo.slots, p.G)
                 : p.bias ? ksplit_kernel_epi<kEpiBias, true>(geo.ksplit, geo.waves, geo.slots, p.G)
                          : ksplit_kernel_epi<kEpiNone, true>(geo.ksplit, geo.waves, geo.slots, p.G);
        } else if (p.gate) {
            fn = ksplit_kernel_epi<kEpiGlu>(geo.ksplit, geo.waves, geo.slots, p.G);
        } else if (p.bias) {
            fn = ksplit_kernel_epi<kEpiBias>(geo.ksplit, geo.waves, geo.slots, p.G);
        } else {
            fn = p.sums ? q4k_ksplit_sums_kernel(geo.ksplit, geo.waves, geo.slots, p.G)
                        : ksplit_kernel<false>(geo.ksplit, geo.waves, geo.slots, p.G);
        }
        p.rows_base = geo.rows_base;
        p.rows_extra = geo.rows_extra;
    } else if (geo.mfma) {
        if (geo.mfma_ga && (p.x || !p.y)) return Q4K_EINVAL;  // GA reads the Q8_1 buffer
        fn = geo.mfma_ga ? (p.sums ? q4k_mfma_ga_sums_kernel(nc, geo.waves, geo.slots)
                                   : mfma_ga_kernel_for(nc, geo.waves, geo.slots))
                         : (p.sums ? q4k_mfma_sums_kernel(nc, geo.waves) : mfma_kernel_for(nc, geo.waves));
        p.rows_base = geo.rows_base;
        p.rows_extra = geo.rows_extra;
        p.rpw = geo.ks;
        p.ntiles = geo.segs;
    } else if (geo.bpl == 2 && nc == 1) {
        if (p.sums) return Q4K_EUNSUPPORTED;  // no parity variant of the override-only kernel
        fn = reinterpret_cast<const void *>(&gemv_q4k_blk_kernel<8>);
        p.rpw = geo.rpw;
    } else if (geo.bpl == 1 && nc == 1) {
        if (p.sums) fn = q4k_bpl_sums_kernel(geo.waves);
        else
            fn = geo.waves == 8 ? reinterpret_cast<const void *>(&gemv_q4k_bpl_kernel<8>)
                                : reinterpret_cast<const void *>(&gemv_q4k_bpl_kernel<4>);
        p.rpw = geo.rpw;
    } else {
        if (p.sums) {
            fn = geo.R == 1 ? q4k_sums_kernel(nc, geo.waves, geo.prologue, geo.slots) : nullptr;
            if (!fn) return Q4K_EUNSUPPORTED;  // a launch shape with no parity variant (overrides)
        } else {
            fn = gemv_kernel_for(nc, geo.R, geo.waves, geo.prologue, geo.slots);
        }
        p.rows_base = geo.rows_base;
        p.rows_extra = geo.rows_extra;
        p.ring_off = lds_bytes(p.K, nc);
    }
    if (!fn) return Q4K_EINVAL;
    int st = ensure_lds(di, fn, geo.lds_launch);
    if (st != Q4K_OK) return st;
    // leading arguments: column strides as 32-bit values (run_gemv checks the range)
    int32_t ldx32 = (int32_t)p.ldx, scy32 = (int32_t)p.stride_col_y;
    void *args[] = {&p.x, &p.y, &p.w, &p.row_stride, &ldx32, &scy32, &p.K, &p.vec_ok,
                    &p.rows_base, &p.rows_extra, &p.nb, &p.qcol, &p};
    if (batch) p.bt = bl->bt;
    const dim3 grid((unsigned)geo.grid, batch ? (unsigned)bl->nch : 1u, batch ? (unsigned)bl->nsmp : 1u);
    // the launch's own status (hipGetLastError would also report, and clear,
    // an error a caller's earlier unrelated call left behind)
    const hipError_t e = hipLaunchKernel(fn, grid, dim3(kWave * geo.waves), args, (size_t)geo.lds_launch, stream);
    if (e != hipSuccess) return hip_fail(e);
    return Q4K_OK;
}

// Shared checks of the weight operand.
static int check_weight(const void *src0, int64_t ne00, int64_t ne01, int64_t nb01) {
    if (ne00 <= 0 || ne00 % kQK != 0 || ne01 < 0) return Q4K_EINVAL;
    const int64_t row_bytes = ne00 / kQK * kBlockBytes;
    if (nb01 < row_bytes || nb01 % kBlockBytes != 0) return Q4K_EINVAL;
    if (ne01 > 0 && !src0) return Q4K_EINVAL;
    if (!aligned(src0, 16)) return Q4K_EUNSUPPORTED;
    // 32-bit buffer offsets within a 4-row tile; int row/K arithmetic
    if (nb01 > (int64_t)1 << 28 || ne01 > ((int64_t)1 << 31) - 8 || ne00 > (1 << 24))
        return Q4K_EUNSUPPORTED;
    return Q4K_OK;
}

static int run_gemv(const void *src0, int64_t ne00, int64_t ne01, int64_t nb01, const float *x,
                    int64_t ldx, const uint8_t *y, int64_t stride_col_y, int64_t ncols, float *dst,
                    int64_t ld_dst, hipStream_t stream, const Epilogue *ep = nullptr,
                    const BatchLaunch *bl = nullptr, const SumsOut *so = nullptr) {
    DeviceInfo *di = nullptr;
    int st = device_info(&di);
    if (st != Q4K_OK) return st;
    const int fused = fused_kind(ep);
    if (fused && ncols != 1) return Q4K_EINVAL;
    if (bl && ((int64_t)bl->nch > 65535 || (int64_t)bl->nsmp > 65535)) return Q4K_EUNSUPPORTED;
    const int64_t mats = bl ? (int64_t)bl->nch * bl->nsmp : 1;
    // (batched: every channel's and sample's activation 16-byte aligned too)
    const bool f32_vec = x && aligned(x, 16) && ldx % 4 == 0 &&
                         (!bl || (bl->bt.x_channel % 4 == 0 && bl->bt.x_sample % 4 == 0));
    Geometry geo = pick_geometry(*di, ne00, ne01, ncols, fused, mats, f32_vec, !x && y);
    if ((bl || fused || geo.colsplit) && !geo.ksplit) {  // the batched and fused tile variants: 1 or 2 slots, prologue 0 or 1
        if (fused != kFusedGate) geo.R = 1;
        if (geo.slots > 2) geo.slots = 2;
        if (geo.prologue > 1) geo.prologue = 0;
    }
    if (geo.lds > di->max_lds) return Q4K_EUNSUPPORTED;  // one column exceeds the LDS
    // the tile kernel addresses a wave's rows with 31-bit offsets; column
    // strides travel as 32-bit kernel arguments
    // (the K-split kernel: a workgroup's rows and one step past them)
    if (geo.mfma ? (int64_t)(geo.rows_base + 1) * kMfmaRows * nb01 >= ((int64_t)1 << 31)
                 : geo.ksplit ? (int64_t)(geo.rows_base + 17) * nb01 >= ((int64_t)1 << 31)
                              : !geo.bpl && (int64_t)(geo.rows_base / geo.waves + 2) * nb01 >= ((int64_t)1 << 31))
        return Q4K_EUNSUPPORTED;
    if (ldx > INT32_MAX || stride_col_y > INT32_MAX) return Q4K_EUNSUPPORTED;
    // GA: the Q8_1 columns of a launch as one buffer of 32-bit offsets
    if (geo.mfma_ga && (int64_t)geo.nc_chunk * stride_col_y * kQ81Bytes >= ((int64_t)1 << 31))
        return Q4K_EUNSUPPORTED;
    if (geo.colsplit) {  // the columns as one-column channels of one launch
        if (bl || fused || geo.colsplit != ncols) return Q4K_EINVAL;
        GemvParams p{};
        p.w = static_cast<const uint8_t *>(src0);
        p.row_stride = nb01;
        p.ldx = ldx;
        p.stride_col_y = stride_col_y;
        p.ld_dst = ld_dst;
        p.M = (int)ne01;
        p.K = (int)ne00;
        p.nb = (int)(ne00 / kQK);
        p.G = (p.nb + 15) / 16;
        p.qcol = q8_col_bytes((int)ne00);
        p.ntiles = geo.ntiles;
        p.nblk32 = fastdiv_init((uint32_t)(ne00 / 32));
        if (so) {  // parity variant: each column's launch on its own, same geometry and kernel
            for (int64_t c = 0; c < ncols; ++c) {
                GemvParams pc = p;
                pc.x = x ? x + c * ldx : nullptr;
                pc.y = y ? y + c * stride_col_y * kQ81Bytes : nullptr;
                pc.dst = dst + c * ld_dst;
                pc.vec_ok = x && aligned(pc.x, 16) && (ldx % 4 == 0);
                pc.sums = so->sums + c * ne01 * (ne00 / 32);
                pc.sq = so->sq + c * (ne00 / 32);
                st = launch_gemv(di, geo, pc, 1, stream, nullptr);
                if (st != Q4K_OK) return st;
            }
            return Q4K_OK;
        }
        p.x = x;
        p.y = y;
        p.dst = dst;
        p.vec_ok = x && aligned(x, 16) && (ldx % 4 == 0);
        BatchLaunch cb;
        cb.nch = (int)ncols;
        cb.nsmp = 1;
        cb.bt.ids = nullptr;
        cb.bt.w_channel = 0;
        cb.bt.w_sample = 0;
        cb.bt.x_channel = x ? ldx : stride_col_y;
        cb.bt.x_sample = 0;
        cb.bt.dst_channel = ld_dst;
        cb.bt.dst_sample = 0;
        cb.bt.channel_ratio = (int)ncols;
        cb.bt.sample_ratio = 1;
        cb.bt.nchannels_y = (int)ncols;
        cb.bt.nexperts = 1;
        return launch_gemv(di, geo, p, 1, stream, &cb);
    }
    for (int64_t c0 = 0; c0 < ncols; c0 += geo.nc_chunk) {
        const int nc = (int)(ncols - c0 < geo.nc_chunk ? ncols - c0 : geo.nc_chunk);
        Geometry g2 = geo;
        if (!geo.bpl && !geo.ksplit && !geo.mfma_ga) {
            g2.lds = geo.mfma ? mfma_lds_bytes((int)ne00, nc, geo.waves) : tile_lds_bytes((int)ne00, nc, geo.waves);
            if (g2.lds_launch < g2.lds) g2.lds_launch = g2.lds;
        }
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
        p.ntiles = geo.ntiles;
        p.vec_ok = x && aligned(p.x, 16) && (ldx % 4 == 0);
        p.nblk32 = fastdiv_init((uint32_t)(ne00 / 32));
        if (fused) {
            p.gate = ep->gate;
            p.bias = ep->bias;
            p.gate_bias = ep->gate ? ep->gate_bias : nullptr;
            p.glu_op = ep->glu_op;
        }
        if (so) {  // parity variant: this chunk's columns of the sums
            if (fused || bl) return Q4K_EINVAL;
            p.sums = so->sums + c0 * ne01 * (ne00 / 32);
            p.sq = so->sq + c0 * (ne00 / 32);
        }
        st = launch_gemv(di, g2, p, nc, stream, bl);
        if (st != Q4K_OK) return st;
    }
    return Q4K_OK;
}

}  // namespace q4k

using namespace q4k;

extern "C" {

int32_t q4k_version(void) { return 100; }

const char *q4k_strerror(int status) {
    switch (status) {
        case Q4K_OK: return "ok";
        case Q4K_EUNSUPPORTED: return "unsupported shape, layout or device (fall back)";
        case Q4K_EINVAL: return "invalid argument";
        case Q4K_EHIP: return "HIP runtime error";
        case Q4K_ENOMEM: return "out of memory";
        case Q4K_EIO: return "file could not be opened, read or mapped";
        case Q4K_EFORMAT: return "not a valid GGUF v2/v3 file";
        case Q4K_ESCRATCH: return "the activation's Q8_1 copy exceeds the allocation-free entry point's 1 MiB scratch";
        default: return "unknown status";
    }
}

int32_t q4k_last_hip_error(void) { return g_last_hip_error; }

size_t q4k_q8_1_bytes(int64_t ne10, int64_t ne11) {
    // 0 also for sizes whose byte count would not fit 63 bits
    if (ne10 < 0 || ne11 < 0 || ne10 > ((int64_t)1 << 40) || ne11 > ((int64_t)1 << 16)) return 0;
    return (size_t)(ne11 * (pad512(ne10) / 32) * kQ81Bytes);
}

int q4k_quantize_row_q8_1(const float *x, void *vy, int64_t ne00, int64_t s01, int64_t ne0,
                          int64_t ne1, void *stream) {
    if (ne00 < 0 || ne1 < 0 || ne0 < ne00 || ne0 % 32 != 0) return Q4K_EINVAL;
    if (ne0 == 0 || ne1 == 0) return Q4K_OK;
    if (!x || !vy || (ne1 > 1 && s01 < ne00) || ne1 > 65535) return Q4K_EINVAL;
    if (ne0 > ((int64_t)1 << 38)) return Q4K_EUNSUPPORTED;  // grid.x = ne0 / 1024 < 2^31
    if (!aligned(vy, 4)) return Q4K_EINVAL;
    DeviceInfo *di = nullptr;
    int st = device_info(&di);
    if (st != Q4K_OK) return st;
    int64_t nblk_col = ne0 / 32;
    int vec_ok = aligned(x, 16) && s01 % 4 == 0;
    uint8_t *y = static_cast<uint8_t *>(vy);
    void *args[] = {&x, &y, &ne00, &s01, &nblk_col, &vec_ok};
    // the launch's own status (hipGetLastError would also report, and clear,
    // an error a caller's earlier unrelated call left behind)
    const hipError_t e = hipLaunchKernel(reinterpret_cast<const void *>(&quantize_q8_1_kernel),
                                         dim3((unsigned)((nblk_col + 31) / 32), (unsigned)ne1), dim3(256), args,
                                         0, (hipStream_t)stream);
    if (e != hipSuccess) return hip_fail(e);
    return Q4K_OK;
}

}  // extern "C"

// q4k_mul_mat_vec_q, and with `so` its parity form (the same routes and
// geometry, the SUMS kernels).
static int mul_mat_vec_q_q4k(const void *src0, int64_t ne00, int64_t ne01, int64_t nb01, const float *src1,
                             int64_t ne11, int64_t nb11, float *dst, int64_t nb1, void *workspace,
                             size_t workspace_bytes, void *stream, const SumsOut *so) {
    int st = check_weight(src0, ne00, ne01, nb01);
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
    const Geometry geo = pick_geometry(*di, ne00, ne01, ne11);
    const int64_t ldx = nb11 / 4, ldd = nb1 / 4;
    const size_t need = q4k_q8_1_bytes(ne00, ne11);
    const bool ws_fits = workspace && workspace_bytes >= need && aligned(workspace, 4);
    // the matrix-core kernel that reads its A operand from a Q8_1 copy is
    // reached through that copy, with or without a workspace (so both give
    // the pre-quantised entry point's bits)
    const bool ga_route = pick_geometry(*di, ne00, ne01, ne11, 0, 1, false, true).mfma_ga != 0;
    if (geo.nc_chunk >= ne11 && !ga_route && (geo.ksplit || !(ws_fits && prefer_prequantised(ne00, ne11)))) {
        // quantisation inside the GEMV launch (always for the K-split
        // kernels, the one route they have)
        return run_gemv(src0, ne00, ne01, nb01, src1, ldx, nullptr, 0, ne11, dst, ldd, s, nullptr, nullptr, so);
    }
    // activation too large for one workgroup's LDS at this column count,
    // (with a workspace) too many values for every workgroup to quantise, or
    // the matrix-core kernel with its A operand in the Q8_1 copy:
    // quantise once to a Q8_1 buffer and run the GEMV on it (in column
    // chunks when the columns do not fit the LDS together).
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
        st = run_gemv(src0, ne00, ne01, nb01, nullptr, 0, static_cast<const uint8_t *>(buf), kp / 32,
                      ne11, dst, ldd, s, nullptr, nullptr, so);
    if (owned) {
        hipError_t e = hipFreeAsync(buf, s);
        if (e != hipSuccess && st == Q4K_OK) st = hip_fail(e);
    }
    return st;
}

extern "C" {

int q4k_mul_mat_vec_q(const void *src0, int64_t ne00, int64_t ne01, int64_t nb01, const float *src1,
                      int64_t ne11, int64_t nb11, float *dst, int64_t nb1, void *workspace,
                      size_t workspace_bytes, void *stream) {
    return mul_mat_vec_q_q4k(src0, ne00, ne01, nb01, src1, ne11, nb11, dst, nb1, workspace, workspace_bytes,
                             stream, nullptr);
}

int q4k_mul_mat_vec_q_sums(const void *src0, int64_t ne00, int64_t ne01, int64_t nb01, const float *src1,
                           int64_t ne11, int64_t nb11, float *dst, int64_t nb1, void *workspace,
                           size_t workspace_bytes, int32_t *sums, int32_t *sq, void *stream) {
    if (!sums || !sq || !aligned(sums, 4) || !aligned(sq, 4)) return Q4K_EINVAL;
    const SumsOut so{sums, sq};
    return mul_mat_vec_q_q4k(src0, ne00, ne01, nb01, src1, ne11, nb11, dst, nb1, workspace, workspace_bytes,
                             stream, &so);
}

}  // extern "C"

namespace q4k {

// Scratch of the allocation-free entry point: the Q8_1 copy of the
// activation, in a file-scope device array instead of a workspace or a
// stream-ordered temporary.  Every device holds its own copy until the
// process ends.  Host code never uses the array's name (a host-side stand-in,
// not a device address) but the address hipGetSymbolAddress returns for the
// current device, looked up once per device.
constexpr size_t kNoAllocScratchBytes = (size_t)1 << 20;
static __device__ __align__(256) uint8_t scratch[kNoAllocScratchBytes];

struct ScratchSlot {
    std::once_flag once;
    void *ptr = nullptr;
    hipError_t err = hipSuccess;
};
static ScratchSlot g_scratch[kMaxDevices];

static int scratch_for_current_device(void **out) {
    int dev = 0;
    const hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return hip_fail(e);
    if (dev < 0 || dev >= kMaxDevices) return Q4K_EUNSUPPORTED;
    ScratchSlot &sl = g_scratch[dev];
    std::call_once(sl.once, [&sl]() {
        void *p = nullptr;
        sl.err = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (sl.err == hipSuccess) sl.ptr = p;
    });
    if (sl.err != hipSuccess) return hip_fail(sl.err);
    if (!sl.ptr) return hip_fail(hipErrorInvalidSymbol);
    *out = sl.ptr;
    return Q4K_OK;
}

}  // namespace q4k

extern "C" {

int q4k_mul_mat_vec_q_noalloc(const void *src0, int64_t ne00, int64_t ne01, int64_t nb01, const float *src1,
                              int64_t ne11, int64_t nb11, float *dst, int64_t nb1, void *stream) {
    int st = check_weight(src0, ne00, ne01, nb01);
    if (st != Q4K_OK) return st;
    if (ne11 < 0 || ne11 > Q4K_MAX_BATCH) return Q4K_EINVAL;
    if (ne01 == 0 || ne11 == 0) return Q4K_OK;
    if (q4k_q8_1_bytes(ne00, ne11) > kNoAllocScratchBytes) return Q4K_ESCRATCH;
    DeviceInfo *di = nullptr;
    st = device_info(&di);
    if (st != Q4K_OK) return st;
    void *ws = nullptr;
    st = scratch_for_current_device(&ws);
    if (st != Q4K_OK) return st;
    // with a workspace that holds the Q8_1 copy, q4k_mul_mat_vec_q never
    // allocates: it quantises in-launch or into the workspace
    return q4k_mul_mat_vec_q(src0, ne00, ne01, nb01, src1, ne11, nb11, dst, nb1, ws, kNoAllocScratchBytes,
                             stream);
}

int q4k_op_mul_mat_vec_q(const void *src0_dd_i, int64_t ne00, int64_t row_low, int64_t row_high,
                         const void *src1_ddq_i, int64_t src1_ncols, int64_t src1_padded_row_size,
                         float *dst_dd_i, int64_t nrows_dst, void *stream) {
    if (row_low < 0 || row_high < row_low) return Q4K_EINVAL;
    const int64_t row_diff = row_high - row_low;
    if (ne00 <= 0 || ne00 % kQK != 0) return Q4K_EINVAL;
    int st = check_weight(src0_dd_i, ne00, row_diff, ne00 / kQK * kBlockBytes);
    if (st != Q4K_OK) return st;
    if (src1_ncols < 0 || src1_ncols > Q4K_MAX_BATCH) return Q4K_EINVAL;
    if (row_diff == 0 || src1_ncols == 0) return Q4K_OK;
    if (!src1_ddq_i || !dst_dd_i) return Q4K_EINVAL;
    if (src1_padded_row_size < ne00 || src1_padded_row_size % 32 != 0) return Q4K_EINVAL;
    if (nrows_dst < row_diff) return Q4K_EINVAL;
    if (!aligned(src1_ddq_i, 4) || !aligned(dst_dd_i, 4)) return Q4K_EINVAL;
    return run_gemv(src0_dd_i, ne00, row_diff, ne00 / kQK * kBlockBytes, nullptr, 0,
                    static_cast<const uint8_t *>(src1_ddq_i), src1_padded_row_size / 32, src1_ncols,
                    dst_dd_i, nrows_dst, (hipStream_t)stream);
}

int q4k_mul_mat_vec_q_fused(int32_t src0_type, const void *src0, int64_t ne00, int64_t ne01, int64_t nb01,
                            const float *src1, const q4k_fusion *fusion, float *dst, void *stream) {
    const bool q6 = src0_type == Q4K_GGML_TYPE_Q6_K;
    if (!q6 && src0_type != Q4K_GGML_TYPE_Q4_K) return Q4K_EUNSUPPORTED;
    int st = q6 ? check_weight_q6(src0, ne00, ne01, nb01) : check_weight(src0, ne00, ne01, nb01);
    if (st != Q4K_OK) return st;
    if (ne01 == 0) return Q4K_OK;
    if (!src1 || !dst || !aligned(src1, 4) || !aligned(dst, 4)) return Q4K_EINVAL;
    Epilogue ep;
    if (fusion) {
        ep.gate = static_cast<const uint8_t *>(fusion->gate);
        ep.bias = fusion->x_bias;
        ep.gate_bias = fusion->gate ? fusion->gate_bias : nullptr;  // kernels/mmvq.cu:191
        ep.glu_op = fusion->glu_op;
    }
    if (ep.gate) {
        if (ep.glu_op != kGluGeglu && ep.glu_op != kGluSwiglu && ep.glu_op != kGluSwigluOai)
            return Q4K_EUNSUPPORTED;
        if (!aligned(ep.gate, q6 ? 2 : 16)) return q6 ? Q4K_EINVAL : Q4K_EUNSUPPORTED;
    }
    if (!aligned(ep.bias, 4) || !aligned(ep.gate_bias, 4)) return Q4K_EINVAL;
    const hipStream_t s = (hipStream_t)stream;
    const Epilogue *e = fused_kind(&ep) ? &ep : nullptr;
    return q6 ? run_gemv_q6(src0, ne00, ne01, nb01, src1, ne00, nullptr, 0, 1, dst, ne01, s, e)
              : run_gemv(src0, ne00, ne01, nb01, src1, ne00, nullptr, 0, 1, dst, ne01, s, e);
}

// Same shape and strides (ggml_are_same_shape and ggml_are_same_stride).
static bool same_layout(const q4k_tensor *a, const q4k_tensor *b) {
    for (int d = 0; d < 4; ++d)
        if (a->ne[d] != b->ne[d] || a->nb[d] != b->nb[d]) return false;
    return true;
}

// A bias of the fused epilogue: F32, dst->ne[0] values per row, and (the
// kernel indexes it with dst's strides, as kernels/mmvq.cu:201-218 does) the
// strides of dst in every further dimension the launch walks.
static int check_bias(const q4k_tensor *b, const q4k_tensor *dst, const q4k_tensor *src0, bool ids) {
    if (b->type != Q4K_GGML_TYPE_F32 || b->ne[0] != dst->ne[0] || b->nb[0] != 4) return Q4K_EINVAL;
    if (ids) {
        if (b->ne[1] != src0->ne[2]) return Q4K_EINVAL;  // one bias row per weight matrix
        if (b->ne[1] > 1 && b->nb[1] != dst->nb[1]) return Q4K_EUNSUPPORTED;
        if (dst->ne[3] > 1 && (b->ne[3] != dst->ne[3] || b->nb[3] != dst->nb[3])) return Q4K_EUNSUPPORTED;
        return Q4K_OK;
    }
    for (int d = 2; d < 4; ++d)
        if (dst->ne[d] > 1 && (b->ne[d] != dst->ne[d] || b->nb[d] != dst->nb[d])) return Q4K_EUNSUPPORTED;
    return Q4K_OK;
}

int q4k_ggml_mul_mat_vec_q(const q4k_tensor *src0, const q4k_tensor *src1, const q4k_tensor *ids,
                           q4k_tensor *dst, const q4k_fusion_args *fusion, void *workspace,
                           size_t workspace_bytes, void *stream) {
    if (!src0 || !src1 || !dst) return Q4K_EINVAL;
    if (src1->type != Q4K_GGML_TYPE_F32 || dst->type != Q4K_GGML_TYPE_F32) return Q4K_EINVAL;
    if (src0->type != Q4K_GGML_TYPE_Q4_K && src0->type != Q4K_GGML_TYPE_Q6_K) return Q4K_EUNSUPPORTED;
    const bool q6 = src0->type == Q4K_GGML_TYPE_Q6_K;
    const size_t block_bytes = q6 ? Q4K_BLOCK_Q6_K_BYTES : (size_t)kBlockBytes;
    if (src0->nb[0] != block_bytes || src1->nb[0] != 4 || dst->nb[0] != 4) return Q4K_EINVAL;
    if (ids && (ids->type != Q4K_GGML_TYPE_I32 || ids->nb[0] != 4)) return Q4K_EINVAL;  // :671, :685
    if (src1->ne[0] != src0->ne[0] || dst->ne[0] != src0->ne[1]) return Q4K_EINVAL;
    for (int d = 1; d < 4; ++d)
        if (src0->nb[d] % 2 || src1->nb[d] % 4 || dst->nb[d] % 4) return Q4K_EINVAL;
    const int64_t ne00 = src0->ne[0], ne01 = src0->ne[1], ne02 = src0->ne[2], ne03 = src0->ne[3];
    const int64_t ne11 = src1->ne[1], ne12 = src1->ne[2], ne13 = src1->ne[3];
    if (ne02 < 1 || ne03 < 1) return Q4K_EINVAL;

    // fused epilogue, under the reference's checks (kernels/mmvq.cu:694-715)
    const bool want_fusion = fusion && (fusion->x_bias || fusion->gate);
    Epilogue ep;
    if (want_fusion) {
        if (ids ? dst->ne[2] != 1 : dst->ne[1] != 1) return Q4K_EINVAL;
        int st;
        if (fusion->x_bias) {
            if ((st = check_bias(fusion->x_bias, dst, src0, ids != nullptr)) != Q4K_OK) return st;
            ep.bias = static_cast<const float *>(fusion->x_bias->data);
        }
        if (fusion->gate) {
            if (fusion->gate->type != src0->type || !same_layout(fusion->gate, src0)) return Q4K_EINVAL;
            if (fusion->glu_op != kGluGeglu && fusion->glu_op != kGluSwiglu && fusion->glu_op != kGluSwigluOai)
                return Q4K_EUNSUPPORTED;
            ep.gate = static_cast<const uint8_t *>(fusion->gate->data);
            ep.glu_op = fusion->glu_op;
            if (fusion->gate_bias) {
                if ((st = check_bias(fusion->gate_bias, dst, src0, ids != nullptr)) != Q4K_OK) return st;
                ep.gate_bias = static_cast<const float *>(fusion->gate_bias->data);
            }
        }
        if (!aligned(ep.gate, q6 ? 2 : 16)) return q6 ? Q4K_EINVAL : Q4K_EUNSUPPORTED;
    }
    const Epilogue *e = want_fusion ? &ep : nullptr;
    const int64_t nb01 = (int64_t)src0->nb[1];
    const float *x = static_cast<const float *>(src1->data);
    float *d = static_cast<float *>(dst->data);

    BatchLaunch bl;
    int64_t ncols, ldx, ldd;
    if (!ids) {
        if (dst->ne[1] != ne11 || dst->ne[2] != ne12 || dst->ne[3] != ne13) return Q4K_EINVAL;
        if (ne12 % ne02 != 0 || ne13 % ne03 != 0) return Q4K_EINVAL;  // broadcast (ggml_can_mul_mat)
        if (ne12 == 1 && ne13 == 1) {
            // the 2-D product
            if (e) {
                q4k_fusion f{ep.bias, ep.gate, ep.gate_bias, ep.glu_op};
                return q4k_mul_mat_vec_q_fused(src0->type, src0->data, ne00, ne01, nb01, x, &f, d, stream);
            }
            return (q6 ? q6k_mul_mat_vec_q : q4k_mul_mat_vec_q)(src0->data, ne00, ne01, nb01, x, ne11,
                                                                 (int64_t)src1->nb[1], d, (int64_t)dst->nb[1],
                                                                 workspace, workspace_bytes, stream);
        }
        bl.nch = (int)ne12;
        bl.nsmp = (int)ne13;
        bl.bt.channel_ratio = (int)(ne12 / ne02);
        bl.bt.sample_ratio = (int)(ne13 / ne03);
        bl.bt.x_channel = (int64_t)src1->nb[2] / 4;
        bl.bt.dst_channel = (int64_t)dst->nb[2] / 4;
        ncols = ne11;
        ldx = (int64_t)src1->nb[1] / 4;
        ldd = (int64_t)dst->nb[1] / 4;
    } else {
        // MUL_MAT_ID: dst column j of token 0 = src0[ids[j]] . src1 column j % ne11
        if (ne12 != 1) return Q4K_EINVAL;  // :675 (batch size 1)
        if (ids->ne[0] != dst->ne[1] || ids->ne[1] != ne12 || dst->ne[2] != ne12 || dst->ne[3] != ne13)
            return Q4K_EINVAL;
        if (ne13 % ne03 != 0) return Q4K_EINVAL;
        if (!aligned(ids->data, 4)) return Q4K_EINVAL;
        bl.nch = (int)dst->ne[1];
        bl.nsmp = (int)ne13;
        bl.bt.ids = static_cast<const int32_t *>(ids->data);
        bl.bt.nchannels_y = (int)ne11;
        bl.bt.nexperts = (int)ne02;
        bl.bt.channel_ratio = 1;
        bl.bt.sample_ratio = (int)(ne13 / ne03);
        bl.bt.x_channel = (int64_t)src1->nb[1] / 4;
        bl.bt.dst_channel = (int64_t)dst->nb[1] / 4;
        ncols = 1;
        ldx = (int64_t)src1->nb[2] / 4;
        ldd = (int64_t)dst->nb[2] / 4;
    }
    if (ne01 == 0 || ne11 == 0 || bl.nch == 0 || bl.nsmp == 0) return Q4K_OK;  // empty product
    if (ncols > Q4K_MAX_BATCH) return Q4K_EINVAL;
    if (!x || !d || !aligned(x, 4) || !aligned(d, 4)) return Q4K_EINVAL;
    bl.bt.w_channel = (int64_t)src0->nb[2];
    bl.bt.w_sample = (int64_t)src0->nb[3];
    bl.bt.x_sample = (int64_t)src1->nb[3] / 4;
    bl.bt.dst_sample = (int64_t)dst->nb[3] / 4;
    int st = q6 ? check_weight_q6(src0->data, ne00, ne01, nb01) : check_weight(src0->data, ne00, ne01, nb01);
    if (st != Q4K_OK) return st;
    if (!q6 && ((bl.bt.w_channel % 16) || (bl.bt.w_sample % 16))) return Q4K_EUNSUPPORTED;
    const hipStream_t s = (hipStream_t)stream;
    return q6 ? run_gemv_q6(src0->data, ne00, ne01, nb01, x, ldx, nullptr, 0, ncols, d, ldd, s, e, &bl)
              : run_gemv(src0->data, ne00, ne01, nb01, x, ldx, nullptr, 0, ncols, d, ldd, s, e, &bl);
}

int q4k_subblock_sums(const void *src0, int64_t ne00, int64_t ne01, int64_t nb01, const void *q8_1,
                      int64_t ncols, int64_t stride_col_y, int32_t *sqq, int32_t *sq, void *stream) {
    int st = check_weight(src0, ne00, ne01, nb01);
    if (st != Q4K_OK) return st;
    if (ncols < 0 || ncols > Q4K_MAX_BATCH) return Q4K_EINVAL;
    if (ne01 == 0 || ncols == 0) return Q4K_OK;
    if (!q8_1 || !sqq || !sq || stride_col_y < ne00 / 32 || !aligned(q8_1, 4)) return Q4K_EINVAL;
    DeviceInfo *di = nullptr;
    st = device_info(&di);
    if (st != Q4K_OK) return st;
    const int lds = lds_bytes((int)ne00, 1);
    if (lds > di->max_lds) return Q4K_EUNSUPPORTED;
    st = ensure_lds(di, reinterpret_cast<const void *>(&subblock_sums_kernel), lds);
    if (st != Q4K_OK) return st;
    const int nb = (int)(ne00 / kQK);
    for (int64_t c = 0; c < ncols; ++c) {
        SumsParams p{};
        p.w = static_cast<const uint8_t *>(src0);
        p.row_stride = nb01;
        p.y = static_cast<const uint8_t *>(q8_1) + c * stride_col_y * kQ81Bytes;
        p.sqq = sqq + c * ne01 * (ne00 / 32);
        p.sq = sq + c * (ne00 / 32);
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
        const hipError_t e = hipLaunchKernel(reinterpret_cast<const void *>(&subblock_sums_kernel), dim3(grid),
                                             dim3(256), args, (size_t)lds, (hipStream_t)stream);
        if (e != hipSuccess) return hip_fail(e);
    }
    return Q4K_OK;
}

int q4k_set_geometry_override(int32_t rows_per_tile, int32_t waves_per_wg, int32_t workgroups,
                              int32_t kernel) {
    if (rows_per_tile < 0 || waves_per_wg < 0 || workgroups < 0) return Q4K_EINVAL;
    if (kernel < 0 || kernel > 6) return Q4K_EINVAL;
    if (rows_per_tile != 0 && rows_per_tile != 1 && rows_per_tile != 2 && rows_per_tile != 4 &&
        !(kernel == 5 && (rows_per_tile == 8 || rows_per_tile == 16)))
        return Q4K_EINVAL;
    if (waves_per_wg < 0 || waves_per_wg > 16) return Q4K_EINVAL;
    g_ovr_rows.store(rows_per_tile);
    g_ovr_waves.store(waves_per_wg);
    g_ovr_wgs.store(workgroups);
    g_ovr_kernel.store(kernel);
    return Q4K_OK;
}

int q4k_set_pipeline_override(int32_t slots, int32_t prologue) {
    if (slots < 0 || slots > 8 || (slots > 4 && slots != 8)) return Q4K_EINVAL;
    if (prologue < -1 || prologue > 3) return Q4K_EINVAL;
    g_ovr_slots.store(slots);
    g_ovr_prologue.store(prologue);
    return Q4K_OK;
}

static void fill_geometry_out(const Geometry &g, int64_t ne11, bool q81, int32_t out[8]) {
    out[0] = g.R;
    out[1] = g.waves;
    out[2] = g.grid;
    out[3] = g.lds_launch;
    out[4] = g.colsplit ? 1 : g.nc_chunk;  // (column split: one column per channel, all in one launch)
    out[5] = g.colsplit || g.nc_chunk >= ne11 ? 1 : 0;
    out[6] = g.ksplit ? 5 : (g.mfma_ga ? 6 : (g.mfma ? 4 : (g.bpl == 2 ? 3 : (g.bpl ? 2 : 1))));
    out[7] = g.bpl ? g.rpw : g.R;
    if (q81) out[5] = 0;
}

static int gemv_geometry(int64_t ne00, int64_t ne01, int64_t ne11, bool q81, int32_t out[8]) {
    if (!out || ne00 <= 0 || ne00 % kQK != 0 || ne01 < 0 || ne11 < 1 || ne11 > Q4K_MAX_BATCH)
        return Q4K_EINVAL;
    DeviceInfo *di = nullptr;
    int st = device_info(&di);
    if (st != Q4K_OK) return st;
    Geometry g = pick_geometry(*di, ne00, ne01, ne11, 0, 1, !q81, q81);
    if (!q81) {  // the F32 entry reaches the GA kernel through a Q8_1 copy
        const Geometry gq = pick_geometry(*di, ne00, ne01, ne11, 0, 1, false, true);
        if (gq.mfma_ga) {
            g = gq;
            q81 = true;
        }
    }
    fill_geometry_out(g, ne11, q81, out);
    return Q4K_OK;
}

int q4k_gemv_geometry(int64_t ne00, int64_t ne01, int64_t ne11, int32_t out[8]) {
    return gemv_geometry(ne00, ne01, ne11, false, out);
}

int q4k_gemv_geometry_q8_1(int64_t ne00, int64_t ne01, int64_t ne11, int32_t out[8]) {
    return gemv_geometry(ne00, ne01, ne11, true, out);
}

int q4k_gemv_geometry_fused(int64_t ne00, int64_t ne01, int32_t with_gate, int32_t out[8]) {
    if (!out || ne00 <= 0 || ne00 % kQK != 0 || ne01 < 0) return Q4K_EINVAL;
    DeviceInfo *di = nullptr;
    int st = device_info(&di);
    if (st != Q4K_OK) return st;
    Geometry g = pick_geometry(*di, ne00, ne01, 1, with_gate ? kFusedGate : kFusedBias, 1, true, false);
    if (!g.ksplit) {  // the tile variants' adjustments (run_gemv)
        if (!with_gate) g.R = 1;
        if (g.slots > 2) g.slots = 2;
    }
    fill_geometry_out(g, 1, false, out);
    return Q4K_OK;
}

}  // extern "C"
