// q6k_gemv.hip -- the Q6_K matrix-vector product's launches and its C ABI
// (declared in include/q4k_gemv.h next to the Q4_K entry points).  The tile
// kernel is in q6k_kernels.h, the matrix-core kernel in q6k_mfma.h: their
// product variants are instantiated here, their parity variants in
// q6k_sums.hip.
#include <hip/hip_runtime.h>

#include <cstring>

#include "../../include/q4k_gemv.h"
#include "q4k_runtime.h"
#include "q4k_tile.h"
#include "q6k_kernels.h"
#include "q6k_ksplit.h"
#include "q6k_ksplit_nc.h"
#include "q6k_mfma.h"

namespace q4k {

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
static int q6_act_bytes(int K, int nc, bool dense) { return nc * (q8_col_bytes(K, dense) + K / 8 + K / 4); }
static int q6_tile_lds_bytes(int K, int nc, int waves, bool dense) {
    const int act = q6_act_bytes(K, nc, dense);
    return act + waves * ring_cap(act, nc, waves) * 4;
}

// Column counts with dense-layout kernels: from 5 columns up, where halving
// the column count (two launches, each streaming the whole weight matrix) is
// what the dense layout's saving of up to 4095 bytes per column avoids.
constexpr int kDenseMinCols = 5;

struct Q6Geometry {
    int waves = 16;
    int grid = 0;
    int lds = 0;
    int lds_launch = 0;
    int nc_chunk = 1;
    bool dense = false;  // nc_chunk columns fit the LDS only in the dense layout
    int rows_base = 0;
    int rows_extra = 0;
    int prologue = 0;
    int slots = 2;
    int mfma = 0;  // 1: matrix-core kernel (tiles of 16 rows; rows_base/rows_extra count tiles)
    int ks = 1;    // matrix-core kernel: waves sharing one tile
    int segs = 1;  // matrix-core kernel: summation segments of a row
    int ksplit = 0;  // K-split kernel: super-blocks per wave and group (0: another kernel)
    int ks_tr = 0;   // K-split kernel: rows per wave step (16 / ksplit)
    int ks_long = 0; // K-split kernel for rows of any length (activation slices in LDS)
    int mfma_ga = 0; // matrix-core kernel: A operand from the Q8_1 buffer (pre-quantised route)
    int ks_nc_p = 0; // several-column K-split kernel: columns of its reduction tree (2 or 4; 0: not it)
    int ks_kt = 0;   // long-row K-split kernel, rows shorter than one group: waves per team (0: 16/SBW)
    int colsplit = 0; // several columns as one launch over one-column channels (the columns; 0: not)
    int ks_snc = 0;   // several columns of rows shorter than one group in short teams: waves per team
    int ks_snc_p = 2; // (and the tile kernel's tree columns, 2 or 4)
};

// Columns per launch of the tile kernel for N columns of K values (halved
// until they fit the LDS, or all of five or more in the dense layout).
static int q6_tile_chunk(int64_t K, int64_t N, int max_lds, bool &dense) {
    int nc = (int)N;
    dense = false;
    while (nc > 1 && q6_tile_lds_bytes((int)K, nc, 16, false) > max_lds) {
        if (nc >= kDenseMinCols && q6_tile_lds_bytes((int)K, nc, 16, true) <= max_lds) {
            dense = true;
            break;
        }
        nc = (nc + 1) / 2;
    }
    return nc;
}

// The several-column K-split kernel's launch shape (N = 2..4 aligned F32
// columns; P: the tile kernel's tree column count): rows_per_step 8 (two
// super-blocks per wave; P = 2) or 4, waves per workgroup (whole teams),
// workgroups (default one per CU), steps in flight (1, 2).
static Q6Geometry pick_geometry_q6_ksplit_nc(const DeviceInfo &di, int64_t K, int64_t M, int rows_per_step,
                                             int waves, int wgs, int slots, int N, int P) {
    Q6Geometry g;
    const int cus = di.cus > 0 ? di.cus : 1;
    g.ks_nc_p = P;
    g.ksplit = P == 2 && rows_per_step == 8 ? 2 : 4;
    g.ks_tr = 16 / g.ksplit;
    g.waves = waves == 4 || waves == 8 || waves == 16 ? waves : 16;
    if (g.waves < g.ks_tr) g.waves = g.ks_tr;
    g.slots = slots == 1 || slots == 2 ? slots : 1;
    if (!q6_ksplit_nc_exists(N, P, g.ksplit, g.waves, g.slots)) {
        g.waves = 16;
        g.slots = 1;
    }
    int64_t grid = wgs > 0 ? wgs : cus;
    if (grid > M) grid = M;
    g.grid = grid < 1 ? 1 : (int)grid;
    g.rows_base = (int)(M / g.grid);
    g.rows_extra = (int)(M % g.grid);
    g.lds = q6_ksn_stage_bytes((int)K, N) +
            ksplit_nc_part_bytes(g.rows_base + (g.rows_extra ? 1 : 0), N, g.ksplit);
    g.lds_launch = g.lds;
    g.nc_chunk = N;
    return g;
}

// The several-column short-team kernel (gemv_q6k_ksplit_short_nc_kernel)
// for N columns of rows of K values: rows_per_step 8 or 4 (2 or 4
// super-blocks per wave; three or four columns: 4), waves, workgroups
// (default one per CU), tiles in flight; ksplit = 0 where the rows do not
// qualify (3 to 8 blocks), the variant is not instantiated or its LDS does
// not fit.
static Q6Geometry pick_geometry_q6_short_nc(const DeviceInfo &di, int64_t K, int64_t M, int N, int rows_per_step,
                                            int waves, int wgs, int slots) {
    Q6Geometry g;
    const int cus = di.cus > 0 ? di.cus : 1;
    const int64_t nb = K / kQK;
    if (K % kQK || nb < 3 || nb > 8 || N < 2 || N > 4) return g;
    const bool rc4 = N > 2 && nb > 4;  // the four-column tree: super-blocks w and w + 4 per wave
    g.ksplit = rc4 ? 2 : (rows_per_step == 4 || N > 2 ? 4 : 2);
    g.ks_tr = 16 / g.ksplit;
    g.ks_snc = rc4 ? 4 : ksplit_short_team((int)nb, g.ksplit);
    g.ks_snc_p = rc4 ? 4 : 2;
    g.waves = waves == 4 || waves == 8 || waves == 16 ? waves : 8;
    g.slots = slots == 1 || slots == 2 ? slots : 1;
    if (!g.ks_snc || !ksplit_short_nc_exists(N, g.ksplit, g.ks_snc, g.waves, g.slots, g.ks_snc_p)) {
        g.ksplit = 0;
        return g;
    }
    int64_t grid = wgs > 0 ? wgs : cus;
    if (grid > M) grid = M;
    g.grid = grid < 1 ? 1 : (int)grid;
    g.rows_base = (int)(M / g.grid);
    g.rows_extra = (int)(M % g.grid);
    g.lds = q6_ksplit_short_nc_lds_bytes(g.rows_base + (g.rows_extra ? 1 : 0), N, g.ksplit, g.ks_snc, g.waves);
    g.lds_launch = g.lds;
    g.nc_chunk = N;
    if (g.lds > (di.max_lds > 0 ? di.max_lds : 65536)) g.ksplit = 0;
    return g;
}

// The K-split kernel's launch shape: rows_per_step TR = 16 / SBW (4, 8, 16;
// rows of other lengths than 4096 and 8192 values: the long-row variant, 8
// or 16), waves per workgroup (whole teams of TR waves; long rows: 8 or 16),
// workgroups (default one per CU), tiles in flight (1, 2).
static Q6Geometry pick_geometry_q6_ksplit(const DeviceInfo &di, int64_t K, int64_t M, int rows_per_step, int waves,
                                          int wgs, int slots, int fused = kFusedNone, bool batch = false) {
    Q6Geometry g;
    const int cus = di.cus > 0 ? di.cus : 1;
    const bool lng = K != 4096 && K != 8192;
    const int G = (int)((K / kQK + 15) / 16);
    g.ks_long = lng ? 1 : 0;
    g.ks_tr = rows_per_step == 4 || rows_per_step == 8 || rows_per_step == 16 ? rows_per_step : 8;
    if (lng && g.ks_tr == 4 && G > 4) g.ks_tr = 8;  // 4 rows per step: rows of up to 4 groups
    g.ksplit = 16 / g.ks_tr;
    g.waves = waves >= 1 && waves <= 16 ? waves : 16;
    g.slots = slots >= 1 && slots <= (lng ? 4 : 2) ? slots : 1;
    // rows shorter than one group: teams of only the waves the row needs,
    // where that variant is instantiated (else the whole team; team sizes
    // other than powers of two take workgroups of whole teams)
    const int epi = fused == kFusedGate ? kEpiGlu : (fused == kFusedBias ? kEpiBias : kEpiNone);
    int kt = lng ? ksplit_short_team((int)(K / kQK), g.ksplit) : 0;
    if (kt) {
        if (g.waves < kt) g.waves = kt;
        if (!ksplit_short_exists(true, g.ksplit, kt, g.waves, g.slots, false, epi, batch)) g.slots = 1;
        if (!ksplit_short_exists(true, g.ksplit, kt, g.waves, g.slots, false, epi, batch)) kt = 0;
    }
    g.ks_kt = kt;
    if (!kt) {
        if (g.waves != 4 && g.waves != 8 && g.waves != 16) g.waves = 16;
        if (g.waves < g.ks_tr) g.waves = g.ks_tr;
        if (lng ? !q6_ksplit_long_exists(g.ksplit, g.waves, g.slots, G <= 4 ? 4 : 8)
                : !q6_ksplit_exists(g.ksplit, g.waves, g.slots, (int)(K / 4096)))
            g.slots = lng ? 2 : 1;
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
    if ((fused != kFusedNone || batch) && !kt) {
        const bool glu = fused == kFusedGate;
        auto ok = [&]() {
            return (!batch || q6_ksplit_batch_ok(g.ksplit, g.waves)) &&
                   (lng ? q6_ksplit_long_epi_exists(g.ksplit, g.waves, g.slots, G <= 4 ? 4 : 8, glu)
                        : q6_ksplit_epi_exists(g.ksplit, g.waves, g.slots, (int)(K / 4096), glu));
        };
        if (g.slots > 2 || !ok()) g.slots = 1;
        if (!ok()) g.ksplit = 0;
    }
    const int nw = fused == kFusedGate ? 2 : 1;
    const int sbw = g.ksplit ? g.ksplit : 1;
    g.lds = lng ? q6_ksplit_long_lds_bytes(rows, sbw, g.waves, G, nw, kt) : ksplit_lds_bytes(rows, sbw, nw);
    g.lds_launch = g.lds;
    g.nc_chunk = 1;
    return g;
}

// The K-split kernel's automatic shape for one aligned F32 column of rows
// of up to 8 groups, one workgroup per CU; false where the tile kernel
// measured faster.  rho = rows per CU.  Measured on MI355X (us, interleaved
// graph timings of 200 calls; K-split against the tile kernel): up to 4
// rows per CU, 4 rows per step and 4 waves (1024 x 4096 3.10 against 3.69,
// 1024 x 8192 4.71 / 5.42); up to 8, 8 rows and 8 waves (2048 x 4096 3.61 /
// 4.25); beyond, 4 rows per step, 4 waves and two tiles in flight (4096 x
// 4096 4.79 / 5.75, 14336 x 4096 10.57 / 11.49, 32768 x 4096 21.87 / 22.19,
// 65536 x 4096 39.54 / 41.35, 4096 x 8192 7.96 / 8.60, 28672 x 8192 35.92 /
// 36.60), except over 256 rows per CU at 4096 values (128256 x 4096: 76.10
// against 75.10 on the tile kernel).  Rows of other lengths up to 8 groups
// (the long-row variant): 8 rows per step, 8 waves, one step in flight up
// to 160 rows per CU (4096 x 14336 12.10 against 12.36 with two in flight
// and 13.58 on the tile kernel, 8192 x 28672 37.15 / 39.13 / 42.46,
// 4096 x 11008 9.93 / 10.44 / 10.84, 14336 x 14336 33.75 / 33.84 / 35.93;
// with two: 2048 x 14336 7.84 / 9.17, 13824 x 5120 15.26 / 17.32, 5120 x
// 13824 14.92 / 14.95), 4 rows, 4 waves and two steps up to 4 rows per CU
// and 4 groups (1024 x 14336 6.26 against 6.32), 16 rows and 16 waves from
// 9 to 11 rows per CU (2304 x 9216 7.46 against 7.93 on 8 rows and 8.03 on
// the tile kernel, 2560 x 9728 7.87 / 8.30 / 8.25; at 12 and 14 rows 8 rows
// stay faster: 3072 x 14336 10.73 / 10.88, 3584 x 18944 14.15 / 15.19);
// three or four steps in flight, 16 waves or two workgroups per CU measured
// slower at 16 rows (4096 x 14336 13.29, 13.32, 13.34, 13.12 against
// 12.10).
// Rows of 3 to 8 blocks (768 .. 2048 values; short teams): 8 rows per
// step, one step in flight, 4 waves up to 16 rows per CU (2048 x 768 2.88
// against 3.49 on the tile kernel, 2048 x 2048 3.16 / 3.65), 8 beyond
// (16384 x 768 4.68 / 9.40, 128256 x 2048 38.75 / 57.98; MUL_MAT_ID of
// eight 2048 x 768 experts 4.43 / 7.73).  Rows of 9 to 14 blocks: teams of
// ceil(blocks / 2) waves, one per workgroup up to 16 rows per CU (1024 x
// 2560 3.12 / 3.37, 3584 x 3584 4.71 / 5.33), else two (teams of 7: one;
// 151936 x 2560 57.15 / 72.32, 128256 x 3072 60.09 / 64.66).
static bool q6_ksplit_auto(int64_t K, int64_t M, int cus, int &tr, int &waves, int &slots) {
    const int64_t rho = (M + cus - 1) / cus;
    slots = 1;
    if (ksplit_short_rows(K)) {
        const int nb = (int)(K / kQK), kt = (nb + 1) / 2;
        tr = 8;
        waves = nb <= 8 ? (rho <= 16 ? 4 : 8) : (rho <= 16 || kt == 7 ? kt : 2 * kt);
        return true;
    }
    if (K != 4096 && K != 8192) {
        const bool small = rho <= 4 && K <= 4 * 4096;
        tr = waves = small ? 4 : (rho >= 9 && rho <= 11 ? 16 : 8);
        slots = small ? 2 : 1;
        return rho <= 160;
    }
    if (rho <= 4) {
        tr = waves = 4;
        return true;
    }
    if (rho <= 8) {
        tr = waves = 8;
        return true;
    }
    if (K == 4096 && rho > 256) return false;
    tr = waves = 4;
    slots = 2;
    return true;
}

// Where the matrix-core kernel is chosen (all columns in one launch, which
// the caller checks).  Measured on MI355X against the tile kernel (graph
// replays, us):
//  - rows of up to 4096 values: eight columns from 896 row tiles, six or more
//    from 2048: 128256 x 4096 N=8 117.0 -> 93.5, N=6 106.7 -> 92.4;
//    65536 x 4096 N=6 55.6 -> 49.5; 32768 x 4096 N=8 36.4 -> 29.1, N=6
//    30.3 -> 28.5; 14336 x 4096 N=8 19.1 -> 18.3; 28672 x 3584 N=8 30.0 ->
//    26.7.  Slower at four columns (128256 x 4096: 86.2 against 88.5), at
//    14336 x 4096 N=6, 13824 x 3584 N=8 and on small products.
//  - longer rows: seven or eight columns from 512 tiles (8192 x 8192 N=8
//    24.7 -> 22.2, 8192 x 5120 N=7 19.4 -> 16.5, 28672 x 8192 N=7 53.3 ->
//    51.9); at 5120 values also six columns from 512 tiles and five from 864
//    (13824 x 5120 N=5 21.7 -> 21.0, 28672 x 5120 N=5 39.8 -> 33.3).  At 8192
//    values five or six columns are slower (28672 x 8192 N=6 48.9 against
//    51.4), and 4096 rows are slower everywhere.
// Where the pre-quantised route runs the matrix-core kernel with its A
// operand read from the Q8_1 buffer (GA): rows longer than 8192 values, a
// tile per CU or more, six to eight columns, or five of rows longer than
// 16384 values, where (the caller checks) the staged matrix-core kernel is
// not chosen or cannot hold the columns.  Measured on MI355X (us per op
// with a Q8_1 workspace, the quantiser launch included; GA against the tile
// kernel): 4096 x 14336 N=8 21.88 against 24.52, N=6 20.94 / 21.59;
// 8192 x 28672 N=8 55.79 / 89.89, N=5 52.27 / 85.27.  Even at 4096 x 14336
// with five columns (20.75 / 20.65); slower with four (20.79 / 20.13).
static bool use_mfma_q6_ga(int64_t M, int64_t N, int64_t K) {
    const int64_t tiles = (M + kMfmaRows - 1) / kMfmaRows;
    return K > 8192 && tiles >= 256 && (N >= 6 || (N == 5 && K > 16384));
}

static bool use_mfma_q6(int64_t M, int64_t N, int64_t K) {
    const int64_t tiles = (M + kMfmaRows - 1) / kMfmaRows;
    if (K <= 4096) return (N == 8 && tiles >= 896) || (N >= 6 && tiles >= 2048);
    if (N >= 7 && tiles >= 512) return true;
    return K <= 5120 && ((N == 6 && tiles >= 512) || (N == 5 && tiles >= 864));
}

// The matrix-core kernel's geometry, as for Q4_K: one workgroup per CU (at
// most one per tile) of 8 or 16 waves, the tiles split evenly over the
// workgroups, and KS waves sharing a tile, KS at most the S summation
// segments of a row (a function of K alone, which fixes the summation order).
static Q6Geometry pick_geometry_q6_mfma(const DeviceInfo &di, int64_t K, int64_t M, int nc, int owgs, int owaves,
                                        bool ga = false) {
    Q6Geometry g;
    const int max_lds = di.max_lds > 0 ? di.max_lds : 65536;
    const int cus = di.cus > 0 ? di.cus : 1;
    const int64_t tiles = (M + kMfmaRows - 1) / kMfmaRows;
    g.mfma = 1;
    g.slots = 2;
    g.nc_chunk = nc;
    const int64_t wgs = owgs > 0 ? owgs : cus;
    g.grid = (int)(tiles < wgs ? tiles : wgs);
    if (g.grid < 1) g.grid = 1;
    g.rows_base = (int)(tiles / g.grid);
    g.rows_extra = (int)(tiles % g.grid);
    const int64_t nt = g.rows_base + (g.rows_extra ? 1 : 0);
    g.waves = 16;
    if (owaves >= 1 && owaves <= 16) g.waves = owaves > 8 ? 16 : 8;
    if (ga) g.waves = 8;  // GA: its A operands in flight need more than 16 waves' registers
    const int64_t nb = K / kQK;
    g.segs = 1;
    while (g.segs < kMfmaMaxSegs && 2 * g.segs <= nb) g.segs *= 2;
    int groups = 1;
    while (groups < g.waves && 2 * groups <= nt) groups *= 2;
    g.ks = g.waves / groups;
    while (g.ks > g.segs) g.ks /= 2;
    g.mfma_ga = ga ? 1 : 0;
    g.lds = ga ? q6m_ga_lds_bytes((int)K, g.waves) : q6m_lds_bytes((int)K, nc, g.waves);
    g.lds_launch = g.lds <= max_lds / 2 ? max_lds / 2 + 256 : g.lds;  // one workgroup per CU
    return g;
}

// One workgroup per CU; one group (3360 bytes per wave) in flight per wave;
// 8 waves unless the activation is long (more than 8192 values over all
// columns: 16 waves quantise it in half the rounds) and the workgroup has 16
// or more steps; weight loads before quantisation when the activation fits
// the staging rounds issued ahead of them.  Measured on MI355X: with 210-byte blocks, more
// weight requests in flight (16 waves x 2 groups, 27.5 MB over the chip)
// delay the activation loads more than they hide latency.
// The K-split kernel's automatic shape for one aligned F32 column with a
// gate weight and the GLU; false where the tile kernel is kept.  Measured on
// MI355X (us per fused op, one process, K-split against the fused tile
// kernel): rows of 4096 or 8192 values 4 rows per step, 4 waves, one tile in
// flight (4096 x 4096 7.57 against 8.88, 14336 x 4096 19.71 / 21.55, 28672 x
// 8192 69.51 / 72.01, where the one-column rule's shape, two tiles in
// flight, took 74.51); other lengths 8 rows, 8 waves, one step (4096 x
// 14336 21.94 / 23.63).  Rows of 4096 values or more, up to 160 rows per CU.
static bool q6_ksplit_glu_auto(int64_t K, int64_t M, int cus, int &tr, int &waves, int &slots) {
    const int64_t rho = (M + cus - 1) / cus;
    if (ksplit_short_rows(K)) return q6_ksplit_auto(K, M, cus, tr, waves, slots);  // (the plain rule's shapes)
    if (rho > 160 || K < 4096) return false;
    tr = waves = K == 4096 || K == 8192 ? 4 : 8;
    slots = 1;
    return true;
}

// The several-column short-team kernel's automatic launch shape (aligned F32
// columns of rows that pick_geometry_q6_short_nc admits), one workgroup per
// CU; false where the column split or the tile kernel measured faster.  Rows
// per CU rho: one tile in flight up to rho 16, two beyond; two columns at 2
// super-blocks per wave, 4 waves, three or four at 4 per wave from rho 13
// (below: the column split), 4 waves up to rho 64, 8 beyond.  Measured on
// MI355X, us, before -> after: two columns 512 x 2048 3.46 -> 3.22, 2048 x
// 2048 4.50 -> 3.33, 8192 x 2048 7.37 -> 5.21, 16384 x 768 10.38 -> 4.89,
// 128256 x 2048 62.59 -> 40.44, 151936 x 1024 68.59 -> 25.84; three columns
// 4096 x 768 5.07 -> 4.23, 151936 x 1024 74.63 -> 28.49; four 8192 x 768 7.96
// -> 5.74, 151936 x 1024 80.71 -> 33.98.  Measured up to rho 594; past it the
// LDS of the partials bounds the rows per workgroup.
static bool q6_short_nc_auto(int64_t M, int N, int nb, int cus, int &rows_per_step, int &waves, int &slots) {
    const int64_t rho = (M + cus - 1) / cus;
    if (N > 2 && nb > 4) {  // super-blocks w and w + 4 per wave (the Q4_K rule): 2048 x 1536 three 4.20 ->
                            // 3.61 us, 8192 x 2048 four 8.75 -> 6.98, 128256 x 2048 four 73.16 -> 46.76
        rows_per_step = 8;
        waves = rho > 32 ? 8 : 4;
        slots = rho > 8 ? 2 : 1;
        return rho > 4;
    }
    rows_per_step = N == 2 ? 8 : 4;
    waves = N > 2 && rho > 64 ? 8 : 4;
    slots = rho > 16 ? 2 : 1;
    return N == 2 || rho > 12;
}

static Q6Geometry pick_geometry_q6(const DeviceInfo &di, int64_t K, int64_t M, int64_t N, int64_t mats = 1,
                                   int fused = kFusedNone, bool f32_vec = true, bool q81 = false) {
    Q6Geometry g;
    const int max_lds = di.max_lds > 0 ? di.max_lds : 65536;
    const int cus = di.cus > 0 ? di.cus : 1;
    const int okern = g_ovr_kernel.load();
    // several columns of rows shorter than one group: short teams (aligned
    // F32 columns, the tile kernel launching all N at once; automatic only,
    // before the column split, which these shapes measured slower)
    if (fused == kFusedNone && mats == 1 && okern == 0 && g_ovr_rows.load() == 0 && g_ovr_waves.load() == 0 &&
        g_ovr_wgs.load() == 0 && f32_vec && N >= 2 && N <= 4) {
        bool dense = false;
        int tr = 0, w = 0, sl = 0;
        if (q6_tile_chunk(K, N, max_lds, dense) == N && !dense && q6_short_nc_auto(M, (int)N, (int)(K / kQK), cus, tr, w, sl)) {
            const Q6Geometry gs = pick_geometry_q6_short_nc(di, K, M, (int)N, tr, w, 0, sl);
            if (gs.ksplit) return gs;
        }
    }
    // several columns over few rows per CU: one launch of one-column channels
    // (split_columns; automatic only)
    if (fused == kFusedNone && mats == 1 && okern == 0 && g_ovr_rows.load() == 0 && g_ovr_waves.load() == 0 &&
        g_ovr_wgs.load() == 0 && split_columns(K, M, N, cus) &&
        pick_geometry_q6(di, K, M, 1, N, kFusedNone, true, false).ksplit) {
        Q6Geometry g1 = pick_geometry_q6(di, K, M, 1, N, kFusedNone, f32_vec, q81);
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
    // 25.27 us, down, Q6_K, 22.27 -> 19.64; Qwen3-30B-A3B-like down 7.73 ->
    // 4.43)
    const bool ks_ok = N == 1 && f32_vec && K <= 8 * 4096 &&
                       (mats == 1 || K >= 4096 || okern == 5 || ksplit_short_rows(K));
    const int cus_m = mats > 1 ? grid_per_matrix(cus, mats, M) : cus;
    // two to four columns: the several-column K-split kernel, whose outputs
    // are the bits of the tile kernel's launches (all columns in one, or
    // four two by two; not the dense layout).  Through the override only:
    // measured on MI355X no faster than the tile kernel (4096 x 14336 N=2
    // 15.58 against 15.26 us, N=4 20.25 / 19.93, 1024 x 4096 N=4 5.77 /
    // 5.61, 4096 x 4096 N=2 6.58 / 6.56) -- a Q6_K step reads six 16-byte
    // LDS chunks per column and unpacks more per weight byte, so spreading
    // rows over more waves buys nothing.
    bool tdense = false;
    const int tchunk = q6_tile_chunk(K, N, max_lds, tdense);
    const bool ksn_ok = N >= 2 && N <= 4 && mats == 1 && fused == kFusedNone && f32_vec && K <= 8 * 4096 &&
                        !tdense && (tchunk == N || (tchunk == 2 && N == 4));
    const int ksn_p = tchunk <= 2 ? 2 : 4;
    // several columns of rows shorter than one group: short teams (the tile
    // kernel launching all N columns at once)
    if (ksn_ok && tchunk == N && okern == 5) {
        const Q6Geometry gs = pick_geometry_q6_short_nc(di, K, M, (int)N, g_ovr_rows.load(), g_ovr_waves.load(),
                                                        g_ovr_wgs.load(), g_ovr_slots.load());
        if (gs.ksplit) return gs;
    }
    if (ksn_ok && okern == 5)
        return pick_geometry_q6_ksplit_nc(di, K, M, g_ovr_rows.load(), g_ovr_waves.load(), g_ovr_wgs.load(),
                                          g_ovr_slots.load(), (int)N, ksn_p);
    if (ks_ok && okern == 5) {
        const int ow = g_ovr_wgs.load();
        const Q6Geometry gk = pick_geometry_q6_ksplit(di, K, M, g_ovr_rows.load(), g_ovr_waves.load(),
                                                      ow > 0 ? ow : (mats > 1 ? cus_m : 0), g_ovr_slots.load(), fused,
                                                      mats > 1);
        if (gk.ksplit) return gk;
    }
    if (ks_ok && okern == 0 && g_ovr_rows.load() == 0 && g_ovr_waves.load() == 0 && g_ovr_wgs.load() == 0) {
        int tr = 0, kw = 0, ks = 0;
        if (fused == kFusedGate ? q6_ksplit_glu_auto(K, M, cus_m, tr, kw, ks) : q6_ksplit_auto(K, M, cus_m, tr, kw, ks)) {
            const int os = g_ovr_slots.load();
            Q6Geometry gk = pick_geometry_q6_ksplit(di, K, M, tr, kw, mats > 1 ? cus_m : 0,
                                                    os >= 1 && os <= 4 ? os : ks, fused, mats > 1);
            if (!gk.ksplit && tr == 16)  // (no batched 16-row variant: the 8-row shape)
                gk = pick_geometry_q6_ksplit(di, K, M, 8, 8, mats > 1 ? cus_m : 0, os >= 1 && os <= 4 ? os : ks,
                                             fused, mats > 1);
            if (gk.ksplit && gk.lds <= max_lds && (mats == 1 || K >= 4096 || gk.ks_kt)) return gk;
        }
    }
    // the matrix-core kernel with its A operand from the Q8_1 buffer: the
    // pre-quantised route, up to 8 columns in one launch
    if (q81 && fused == kFusedNone && mats == 1 && N <= kMfmaCols &&
        (okern == 6 ||
         (okern == 0 && use_mfma_q6_ga(M, N, K) &&
          !(use_mfma_q6(M, N, K) && q6m_lds_bytes((int)K, (int)N, 16) <= max_lds))))
        return pick_geometry_q6_mfma(di, K, M, (int)N, g_ovr_wgs.load(), g_ovr_waves.load(), true);
    if (fused == kFusedNone && mats == 1 && (okern == 4 || (okern == 0 && use_mfma_q6(M, N, K)))) {
        int mc = (int)N;
        while (mc > 1 && q6m_lds_bytes((int)K, mc, 16) > max_lds) mc = (mc + 1) / 2;
        if (q6m_lds_bytes((int)K, mc, 16) <= max_lds && (okern == 4 || mc == N))
            return pick_geometry_q6_mfma(di, K, M, mc, g_ovr_wgs.load(), g_ovr_waves.load());
    }
    int nc = (int)N;
    // Measured on MI355X: 4096 x 14336 at 8 columns, one dense launch 26.8 us
    // against two padded 4-column launches 34.5 us.
    while (nc > 1 && q6_tile_lds_bytes((int)K, nc, 16, false) > max_lds) {
        if (nc >= kDenseMinCols && q6_tile_lds_bytes((int)K, nc, 16, true) <= max_lds) {
            g.dense = true;
            break;
        }
        nc = (nc + 1) / 2;
    }
    g.nc_chunk = nc;
    const int owaves = g_ovr_waves.load(), owgs = g_ovr_wgs.load(), oslots = g_ovr_slots.load();
    g.grid = owgs > 0 ? owgs : grid_per_matrix(cus, mats, M);
    const int64_t steps_per_wg = (M + g.grid - 1) / g.grid * ((K / kQK + 15) / 16);
    g.waves = steps_per_wg >= 16 && (int64_t)nc * K > 8192 ? 16 : 8;
    // Small products with an activation of 32768 or more values: 16 waves,
    // which halve the quantisation rounds that dominate them (1024 x 8192
    // N=4 9.82 -> 8.81 us, N=8 14.45 -> 12.56; 1024 x 4096 N=8 8.33 -> 8.0).
    if ((int64_t)nc * K >= 32768) g.waves = 16;
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
    if (g.dense) g.slots = 1;  // the dense kernels are one-slot
    g.rows_base = (int)(M / g.grid);
    g.rows_extra = (int)(M % g.grid);
    g.lds = q6_tile_lds_bytes((int)K, nc, g.waves, g.dense);
    g.lds_launch = g.lds;
    if (owgs == 0 && g.lds_launch <= max_lds / 2) g.lds_launch = max_lds / 2 + 256;
    const bool pro0_ok = (int64_t)nc * (K / 32) <= (int64_t)stage_capacity(stage_lpb(nc), g.waves * kWave, nc);
    g.prologue = pro0_ok ? 0 : 1;
    const int opro = g_ovr_prologue.load();
    if (opro == 1 || (opro == 0 && pro0_ok)) g.prologue = opro;
    return g;
}

template <int NC, int WAVES, int S, int EPI, bool BATCH, bool DENSE = false>
static const void *q6_sym(int pro) {
    return pro == 0 ? reinterpret_cast<const void *>(&gemv_q6k_kernel<NC, WAVES, 0, S, EPI, BATCH, false, DENSE>)
                    : reinterpret_cast<const void *>(&gemv_q6k_kernel<NC, WAVES, 1, S, EPI, BATCH, false, DENSE>);
}

template <int WAVES, bool BATCH>
static const void *q6_sym_dense(int nc, int pro) {
    static_assert(kDenseMinCols == 5, "dense kernels for 5..8 columns");
    switch (nc) {
        case 5: return q6_sym<5, WAVES, 1, kEpiNone, BATCH, true>(pro);
        case 6: return q6_sym<6, WAVES, 1, kEpiNone, BATCH, true>(pro);
        case 7: return q6_sym<7, WAVES, 1, kEpiNone, BATCH, true>(pro);
        case 8: return q6_sym<8, WAVES, 1, kEpiNone, BATCH, true>(pro);
        default: return nullptr;
    }
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
static const void *q6_kernel_for(int nc, int waves, int pro, int slots, int fused, bool dense) {
    if (pro != 0 && pro != 1) return nullptr;
    if (dense) {
        if (fused || slots != 1) return nullptr;
        return waves <= 8 ? q6_sym_dense<8, BATCH>(nc, pro) : q6_sym_dense<16, BATCH>(nc, pro);
    }
    if (fused) {
        if (nc != 1) return nullptr;
        return fused == kFusedGate ? q6_kernel_epi<kEpiGlu, BATCH>(waves, pro, slots)
                                   : q6_kernel_epi<kEpiBias, BATCH>(waves, pro, slots);
    }
    if (waves <= 8) return slots == 1 ? q6_sym_nc<8, 1, BATCH>(nc, pro) : q6_sym_nc<8, 2, BATCH>(nc, pro);
    return slots == 1 ? q6_sym_nc<16, 1, BATCH>(nc, pro) : q6_sym_nc<16, 2, BATCH>(nc, pro);
}

template <int WAVES>
static const void *q6_mfma_kernel_nc(int nc) {
    switch (nc) {
        case 1: return reinterpret_cast<const void *>(&gemv_q6k_mfma_kernel<1, WAVES>);
        case 2: return reinterpret_cast<const void *>(&gemv_q6k_mfma_kernel<2, WAVES>);
        case 3: return reinterpret_cast<const void *>(&gemv_q6k_mfma_kernel<3, WAVES>);
        case 4: return reinterpret_cast<const void *>(&gemv_q6k_mfma_kernel<4, WAVES>);
        case 5: return reinterpret_cast<const void *>(&gemv_q6k_mfma_kernel<5, WAVES>);
        case 6: return reinterpret_cast<const void *>(&gemv_q6k_mfma_kernel<6, WAVES>);
        case 7: return reinterpret_cast<const void *>(&gemv_q6k_mfma_kernel<7, WAVES>);
        case 8: return reinterpret_cast<const void *>(&gemv_q6k_mfma_kernel<8, WAVES>);
        default: return nullptr;
    }
}

static const void *q6_mfma_kernel_for(int nc, int waves) {
    return waves > 8 ? q6_mfma_kernel_nc<16>(nc) : q6_mfma_kernel_nc<8>(nc);
}

// GA: 8-wave workgroups
static const void *q6_mfma_ga_kernel_for(int nc, int waves) {
    if (waves != 8) return nullptr;
    switch (nc) {
        case 1: return reinterpret_cast<const void *>(&gemv_q6k_mfma_kernel<1, 8, false, true>);
        case 2: return reinterpret_cast<const void *>(&gemv_q6k_mfma_kernel<2, 8, false, true>);
        case 3: return reinterpret_cast<const void *>(&gemv_q6k_mfma_kernel<3, 8, false, true>);
        case 4: return reinterpret_cast<const void *>(&gemv_q6k_mfma_kernel<4, 8, false, true>);
        case 5: return reinterpret_cast<const void *>(&gemv_q6k_mfma_kernel<5, 8, false, true>);
        case 6: return reinterpret_cast<const void *>(&gemv_q6k_mfma_kernel<6, 8, false, true>);
        case 7: return reinterpret_cast<const void *>(&gemv_q6k_mfma_kernel<7, 8, false, true>);
        case 8: return reinterpret_cast<const void *>(&gemv_q6k_mfma_kernel<8, 8, false, true>);
        default: return nullptr;
    }
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
                hipStream_t stream, const Epilogue *ep, const BatchLaunch *bl, const SumsOut *so,
                int64_t geo_mats) {
    DeviceInfo *di = nullptr;
    int st = device_info(&di);
    if (st != Q4K_OK) return st;
    const int fused = fused_kind(ep);
    if (fused && ncols != 1) return Q4K_EINVAL;
    if (bl && ((int64_t)bl->nch > 65535 || (int64_t)bl->nsmp > 65535)) return Q4K_EUNSUPPORTED;
    if (geo_mats < 1 || (geo_mats > 1 && (bl || ncols != 1))) return Q4K_EINVAL;
    const int64_t mats = bl ? (int64_t)bl->nch * bl->nsmp : geo_mats;
    // (batched: every channel's and sample's activation 16-byte aligned too)
    const bool f32_vec = x && aligned(x, 16) && ldx % 4 == 0 &&
                         (!bl || (bl->bt.x_channel % 4 == 0 && bl->bt.x_sample % 4 == 0));
    const Q6Geometry geo = pick_geometry_q6(*di, ne00, ne01, ncols, mats, fused, f32_vec, !x && y);
    if (geo.colsplit) {  // the columns as one-column channels of one launch
        if (bl || fused || geo.colsplit != ncols) return Q4K_EINVAL;
        if (so) {  // parity variant: each column's launch on its own, same geometry and kernel
            for (int64_t c = 0; c < ncols; ++c) {
                const SumsOut sc{so->sums + c * ne01 * (ne00 / 16), nullptr};
                st = run_gemv_q6(src0, ne00, ne01, nb01, x ? x + c * ldx : nullptr, ldx,
                                 y ? y + c * stride_col_y * kQ81Bytes : nullptr, stride_col_y, 1, dst + c * ld_dst,
                                 ld_dst, stream, nullptr, nullptr, &sc, ncols);
                if (st != Q4K_OK) return st;
            }
            return Q4K_OK;
        }
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
        return run_gemv_q6(src0, ne00, ne01, nb01, x, ldx, y, stride_col_y, 1, dst, ld_dst, stream, nullptr, &cb);
    }
    if (geo.lds > di->max_lds) return Q4K_EUNSUPPORTED;  // one column exceeds the LDS
    // a wave's rows (the matrix-core kernel: a workgroup's tiles; the K-split
    // kernel: a workgroup's rows and one step past them) are addressed with
    // 31-bit offsets; column strides travel as 32-bit kernel arguments
    if (geo.mfma      ? (int64_t)(geo.rows_base + 1) * kMfmaRows * nb01 >= ((int64_t)1 << 31)
        : geo.ksplit ? (int64_t)(geo.rows_base + 17) * nb01 >= ((int64_t)1 << 31)
                     : (int64_t)(geo.rows_base / geo.waves + 2) * nb01 >= ((int64_t)1 << 31))
        return Q4K_EUNSUPPORTED;
    if (ldx > INT32_MAX || stride_col_y > INT32_MAX) return Q4K_EUNSUPPORTED;
    // GA: the Q8_1 columns of a launch as one buffer of 32-bit offsets
    if (geo.mfma_ga && (int64_t)geo.nc_chunk * stride_col_y * kQ81Bytes >= ((int64_t)1 << 31))
        return Q4K_EUNSUPPORTED;
    for (int64_t c0 = 0; c0 < ncols; c0 += geo.nc_chunk) {
        const int nc = (int)(ncols - c0 < geo.nc_chunk ? ncols - c0 : geo.nc_chunk);
        // a last chunk of under kDenseMinCols columns is staged padded
        const bool dense = geo.dense && nc >= kDenseMinCols;
        int lds_launch = geo.lds_launch;
        const int lds = geo.mfma_ga  ? geo.lds
                        : geo.mfma   ? q6m_lds_bytes((int)ne00, nc, geo.waves)
                        : geo.ksplit ? geo.lds
                                     : q6_tile_lds_bytes((int)ne00, nc, geo.waves, dense);
        if (lds > di->max_lds) return Q4K_EUNSUPPORTED;
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
        p.qcol = q8_col_bytes((int)ne00, dense);
        p.vec_ok = x && aligned(p.x, 16) && (ldx % 4 == 0);
        p.rows_base = geo.rows_base;
        p.rows_extra = geo.rows_extra;
        p.ring_off = q6_act_bytes(p.K, nc, dense);
        p.nblk32 = fastdiv_init((uint32_t)(ne00 / 32));
        if (fused) {
            p.gate = ep->gate;
            p.bias = ep->bias;
            p.gate_bias = ep->gate ? ep->gate_bias : nullptr;
            p.glu_op = ep->glu_op;
        }
        const int epi = fused == kFusedGate ? kEpiGlu : (fused == kFusedBias ? kEpiBias : kEpiNone);
        const void *fn = geo.ks_snc ? q6k_ksplit_short_nc_kernel(nc, geo.ksplit, geo.ks_snc, geo.waves, geo.slots, false, geo.ks_snc_p)
                         : geo.ks_nc_p  ? q6_ksplit_nc_kernel<false>(nc, geo.ks_nc_p, geo.ksplit, geo.waves, geo.slots)
                         : geo.ks_kt
                             ? q6k_ksplit_short_kernel(geo.ksplit, geo.ks_kt, geo.waves, geo.slots, false, epi, bl != nullptr)
                         : geo.ksplit && bl && fused == kFusedGate
                             ? q6_ksplit_kernel_epi<kEpiGlu, true>(geo.ks_long != 0, geo.ksplit, geo.waves, geo.slots, p.G)
                         : geo.ksplit && bl && fused == kFusedBias
                             ? q6_ksplit_kernel_epi<kEpiBias, true>(geo.ks_long != 0, geo.ksplit, geo.waves, geo.slots, p.G)
                         : geo.ksplit && bl
                             ? q6_ksplit_kernel_epi<kEpiNone, true>(geo.ks_long != 0, geo.ksplit, geo.waves, geo.slots, p.G)
                         : geo.ksplit && fused == kFusedGate
                             ? q6_ksplit_kernel_epi<kEpiGlu>(geo.ks_long != 0, geo.ksplit, geo.waves, geo.slots, p.G)
                         : geo.ksplit && fused == kFusedBias
                             ? q6_ksplit_kernel_epi<kEpiBias>(geo.ks_long != 0, geo.ksplit, geo.waves, geo.slots, p.G)
                         : geo.ks_long  ? q6_ksplit_long_kernel<false>(geo.ksplit, geo.waves, geo.slots, p.G)
                         : geo.ksplit ? q6_ksplit_kernel<false>(geo.ksplit, geo.waves, geo.slots, p.G)
                         : geo.mfma_ga ? q6_mfma_ga_kernel_for(nc, geo.waves)
                         : geo.mfma ? q6_mfma_kernel_for(nc, geo.waves)
                         : bl       ? q6_kernel_for<true>(nc, geo.waves, geo.prologue, geo.slots, fused, dense)
                                    : q6_kernel_for<false>(nc, geo.waves, geo.prologue, geo.slots, fused, dense);
        const bool several = geo.ks_nc_p || geo.ks_snc;
        if (geo.ksplit && (nc != (several ? geo.nc_chunk : 1) || ((fused || bl) && several) || !p.x || !p.vec_ok))
            return Q4K_EINVAL;
        if (geo.ks_nc_p) p.ring_off = q6_ksn_stage_bytes(p.K, nc);
        if (geo.ks_snc)
            p.ring_off = ksplit_short_nc_part_bytes(geo.rows_base + (geo.rows_extra ? 1 : 0), nc, geo.ks_snc);
        if (geo.mfma) {
            if (fused || bl) return Q4K_EINVAL;
            if (geo.mfma_ga && (p.x || !p.y)) return Q4K_EINVAL;  // GA reads the Q8_1 buffer
            p.rpw = geo.ks;
            p.ntiles = geo.segs;
        }
        if (so) {  // parity variant: this chunk's columns of the group sums
            if (fused || bl) return Q4K_EINVAL;
            fn = geo.ks_snc ? q6k_ksplit_short_nc_kernel(nc, geo.ksplit, geo.ks_snc, geo.waves, geo.slots, true, geo.ks_snc_p)
                 : geo.ks_nc_p  ? q6k_ksplit_nc_sums_kernel(nc, geo.ks_nc_p, geo.ksplit, geo.waves, geo.slots)
                 : geo.ks_kt    ? q6k_ksplit_short_kernel(geo.ksplit, geo.ks_kt, geo.waves, geo.slots, true, kEpiNone, false)
                 : geo.ks_long  ? q6k_ksplit_long_sums_kernel(geo.ksplit, geo.waves, geo.slots, p.G)
                 : geo.ksplit ? q6k_ksplit_sums_kernel(geo.ksplit, geo.waves, geo.slots, p.G)
                 : geo.mfma_ga ? q6k_mfma_ga_sums_kernel(nc, geo.waves)
                 : geo.mfma ? q6k_mfma_sums_kernel(nc, geo.waves)
                            : q6k_sums_kernel(nc, geo.waves, geo.prologue, geo.slots, dense);
            if (!fn) return Q4K_EUNSUPPORTED;  // a launch shape with no parity variant (overrides)
            p.sums = so->sums + c0 * ne01 * (ne00 / 16);
        }
        if (bl) p.bt = bl->bt;
        if (geo.ks_long) {
            p.ring_off = ksplit_long_part_bytes(geo.rows_base + (geo.rows_extra ? 1 : 0), geo.ksplit,
                                                fused == kFusedGate ? 2 : 1, geo.ks_kt);
            // groups quantised before the first step: one, the others just
            // before the first step that reads them (4096 x 14336 12.08
            // against 12.14 us with all before, 8192 x 28672 37.04 / 38.42);
            // the pipeline override's prologue 2 forces all
            p.rpw = g_ovr_prologue.load() == 2 ? p.G : 1;
        }
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

}  // extern "C"

// q6k_mul_mat_vec_q, and with `so` its parity form (the same routes and
// geometry, the SUMS kernels).
static int mul_mat_vec_q_q6k(const void *src0, int64_t ne00, int64_t ne01, int64_t nb01, const float *src1,
                             int64_t ne11, int64_t nb11, float *dst, int64_t nb1, void *workspace,
                             size_t workspace_bytes, void *stream, const SumsOut *so) {
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
    // the matrix-core kernel that reads its A operand from a Q8_1 copy is
    // reached through that copy, with or without a workspace (so both give
    // the pre-quantised entry point's bits)
    const bool ga_route = pick_geometry_q6(*di, ne00, ne01, ne11, 1, kFusedNone, false, true).mfma_ga != 0;
    // (the K-split kernels quantise inside the launch: their one route)
    if (geo.nc_chunk >= ne11 && !ga_route && (geo.ksplit || !(ws_fits && prefer_prequantised(ne00, ne11))))
        return run_gemv_q6(src0, ne00, ne01, nb01, src1, ldx, nullptr, 0, ne11, dst, ldd, s, nullptr, nullptr, so);
    // activation too large for one workgroup's LDS at this column count,
    // (with a workspace) too many values for every workgroup to quantise, or
    // the matrix-core kernel with its A operand in the Q8_1 copy:
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
                         dst, ldd, s, nullptr, nullptr, so);
    if (owned) {
        hipError_t e = hipFreeAsync(buf, s);
        if (e != hipSuccess && st == Q4K_OK) st = hip_fail(e);
    }
    return st;
}

extern "C" {

int q6k_mul_mat_vec_q(const void *src0, int64_t ne00, int64_t ne01, int64_t nb01, const float *src1,
                      int64_t ne11, int64_t nb11, float *dst, int64_t nb1, void *workspace,
                      size_t workspace_bytes, void *stream) {
    return mul_mat_vec_q_q6k(src0, ne00, ne01, nb01, src1, ne11, nb11, dst, nb1, workspace, workspace_bytes,
                             stream, nullptr);
}

int q6k_mul_mat_vec_q_sums(const void *src0, int64_t ne00, int64_t ne01, int64_t nb01, const float *src1,
                           int64_t ne11, int64_t nb11, float *dst, int64_t nb1, void *workspace,
                           size_t workspace_bytes, int32_t *s16, void *stream) {
    if (!s16 || !aligned(s16, 4)) return Q4K_EINVAL;
    const SumsOut so{s16, nullptr};
    return mul_mat_vec_q_q6k(src0, ne00, ne01, nb01, src1, ne11, nb11, dst, nb1, workspace, workspace_bytes,
                             stream, &so);
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
    const int lds = q6_act_bytes((int)ne00, 1, false);
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

static int gemv_geometry_q6(int64_t ne00, int64_t ne01, int64_t ne11, bool q81, int32_t out[8]) {
    if (!out || ne00 <= 0 || ne00 % kQK != 0 || ne01 < 0 || ne11 < 1 || ne11 > Q4K_MAX_BATCH)
        return Q4K_EINVAL;
    DeviceInfo *di = nullptr;
    const int st = device_info(&di);
    if (st != Q4K_OK) return st;
    Q6Geometry g = pick_geometry_q6(*di, ne00, ne01, ne11, 1, kFusedNone, !q81, q81);
    if (!q81) {  // the F32 entry reaches the GA kernel through a Q8_1 copy
        const Q6Geometry gq = pick_geometry_q6(*di, ne00, ne01, ne11, 1, kFusedNone, false, true);
        if (gq.mfma_ga) {
            g = gq;
            q81 = true;
        }
    }
    out[0] = g.ksplit ? g.ks_tr : (g.mfma ? kMfmaRows : 1);
    out[1] = g.waves;
    out[2] = g.grid;
    out[3] = g.lds_launch;
    out[4] = g.colsplit ? 1 : g.nc_chunk;  // (column split: one column per channel, all in one launch)
    out[5] = g.colsplit || g.nc_chunk >= ne11 ? 1 : 0;
    out[6] = g.ksplit ? 5 : (g.mfma_ga ? 6 : (g.mfma ? 4 : 1));
    out[7] = g.slots;
    if (q81) out[5] = 0;
    return Q4K_OK;
}

int q6k_gemv_geometry(int64_t ne00, int64_t ne01, int64_t ne11, int32_t out[8]) {
    return gemv_geometry_q6(ne00, ne01, ne11, false, out);
}

int q6k_gemv_geometry_q8_1(int64_t ne00, int64_t ne01, int64_t ne11, int32_t out[8]) {
    return gemv_geometry_q6(ne00, ne01, ne11, true, out);
}

int q6k_gemv_geometry_fused(int64_t ne00, int64_t ne01, int32_t with_gate, int32_t out[8]) {
    if (!out || ne00 <= 0 || ne00 % kQK != 0 || ne01 < 0) return Q4K_EINVAL;
    DeviceInfo *di = nullptr;
    const int st = device_info(&di);
    if (st != Q4K_OK) return st;
    const Q6Geometry g = pick_geometry_q6(*di, ne00, ne01, 1, 1, with_gate ? kFusedGate : kFusedBias, true, false);
    out[0] = g.ksplit ? g.ks_tr : (g.mfma ? kMfmaRows : 1);
    out[1] = g.waves;
    out[2] = g.grid;
    out[3] = g.lds_launch;
    out[4] = g.nc_chunk;
    out[5] = 1;
    out[6] = g.ksplit ? 5 : (g.mfma ? 4 : 1);
    out[7] = g.slots;
    return Q4K_OK;
}

}  // extern "C"
