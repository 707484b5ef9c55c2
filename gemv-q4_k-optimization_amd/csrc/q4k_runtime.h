// q4k_runtime.h -- host-side state and helpers shared by the K-quant GEMV
// entry points (Q4_K in q4k_gemv.hip, Q6_K in q6k_gemv.hip): per-device
// properties, the dynamic-LDS attribute, the last HIP error, the tuning
// overrides and small layout helpers.
#pragma once

#include <hip/hip_runtime.h>

#include <atomic>
#include <cstdint>
#include <mutex>
#include <vector>

#include "../../include/q4k_gemv.h"
#include "q4k_tile.h"

namespace q4k {

// hipError_t of the most recent Q4K_EHIP on this thread
extern thread_local int32_t g_last_hip_error;
// records e and returns Q4K_EHIP
int hip_fail(hipError_t e);

struct DeviceInfo {
    bool ok = false;
    bool supported = false;
    int cus = 0;
    int max_lds = 0;
    std::once_flag once;
    // dynamic-LDS attribute already raised for a kernel (by address)
    std::mutex attr_mu;
    std::vector<const void *> attr_done;
};

constexpr int kMaxDevices = 64;

// The current device's properties, read once per device; Q4K_EUNSUPPORTED on
// anything but gfx950.
int device_info(DeviceInfo **out);
// Raises a kernel's dynamic-LDS limit once when it asks for more than 64 KB.
int ensure_lds(DeviceInfo *di, const void *fn, int bytes);

// Geometry overrides for tuning sweeps (0 = automatic, prologue -1 =
// automatic), set through the q4k_set_*_override entry points only.
extern std::atomic<int> g_ovr_rows, g_ovr_waves, g_ovr_wgs, g_ovr_kernel;
extern std::atomic<int> g_ovr_prologue, g_ovr_slots;

// Fused epilogue of a one-column product (the fields of ggml's
// ggml_cuda_mm_fusion_args_device, kernels/mmvq.cu:692-715): an optional
// gate weight with the layout of the weight, optional biases of the two
// products, and the GLU op that combines them.
struct Epilogue {
    const uint8_t *gate = nullptr;
    const float *bias = nullptr;
    const float *gate_bias = nullptr;
    int glu_op = 0;
};
constexpr int kFusedNone = 0;
constexpr int kFusedBias = 1;  // bias only
constexpr int kFusedGate = 2;  // gate weight (+ biases) and GLU
inline int fused_kind(const Epilogue *e) {
    return !e ? kFusedNone : (e->gate ? kFusedGate : (e->bias ? kFusedBias : kFusedNone));
}

inline bool aligned(const void *p, uintptr_t a) { return ((uintptr_t)p & (a - 1)) == 0; }

// Parity outputs of the *_sums entry points: launches with them run the
// SUMS variants of the product kernels (same geometry, same results) that
// also store the int32 sums.
struct SumsOut {
    int32_t *sums;  // Q4_K [N][M][K/32] sub-block sums; Q6_K [N][M][K/16] group sums
    int32_t *sq;    // Q4_K [N][K/32] activation sums (Q6_K: unused)
};

// The SUMS kernels (q4k_sums.hip, q6k_sums.hip): the variant of the launch
// shape given, or null when it is not instantiated (only the shapes the
// automatic geometry picks for plain products are).
const void *q4k_sums_kernel(int nc, int waves, int pro, int slots);
const void *q4k_bpl_sums_kernel(int waves);
const void *q4k_mfma_sums_kernel(int nc, int waves);
const void *q4k_ksplit_sums_kernel(int sbw, int waves, int slots, int G);
const void *q4k_ksplit_long_sums_kernel(int sbw, int waves, int slots, int G);
const void *q4k_ksplit_nc_sums_kernel(int nc, int sbw, int waves, int slots, int G, bool staged);
const void *q4k_ksplit_nc_long_sums_kernel(int nc, int p, int sbw, int waves, int slots);
const void *q4k_mfma_ga_sums_kernel(int nc, int waves, int nif);
const void *q6k_mfma_sums_kernel(int nc, int waves);
const void *q6k_ksplit_sums_kernel(int sbw, int waves, int slots, int G);
const void *q6k_ksplit_long_sums_kernel(int sbw, int waves, int slots, int G);
const void *q6k_ksplit_nc_sums_kernel(int nc, int p, int sbw, int waves, int slots);
const void *q6k_mfma_ga_sums_kernel(int nc, int waves);
const void *q6k_sums_kernel(int nc, int waves, int pro, int slots, bool dense);

// The long-row K-split kernels with short teams (q4k_short.hip): the variant
// of the launch shape and kind given (sums: the parity variant; epi:
// kEpiNone, kEpiBias, kEpiGlu; batch: broadcasting / MUL_MAT_ID), or null
// where ksplit_short_exists says it is not instantiated.
const void *q4k_ksplit_short_kernel(int sbw, int kt, int waves, int slots, bool sums, int epi, bool batch);
const void *q6k_ksplit_short_kernel(int sbw, int kt, int waves, int slots, bool sums, int epi, bool batch);
// The several-column short-team kernels (q4k_short.hip, q6k_short.hip), or null.
// (p: columns of the tile kernel's reduction tree, 2, or 4 for rows of 5 to 8
// blocks in three or four columns: super-blocks w and w + 4 per wave)
const void *q4k_ksplit_short_nc_kernel(int nc, int sbw, int kt, int waves, int slots, bool sums, int p = 2);
const void *q6k_ksplit_short_nc_kernel(int nc, int sbw, int kt, int waves, int slots, bool sums, int p = 2);

// Q6_K weight checks and launch (q6k_gemv.hip), for the type-dispatching
// entry points of q4k_gemv.hip.
int check_weight_q6(const void *src0, int64_t ne00, int64_t ne01, int64_t nb01);
// (geo_mats: the geometry of a launch over that many one-column channels,
// for the parity variant's per-column launches of a column-split product)
int run_gemv_q6(const void *src0, int64_t ne00, int64_t ne01, int64_t nb01, const float *x, int64_t ldx,
                const uint8_t *y, int64_t stride_col_y, int64_t ncols, float *dst, int64_t ld_dst,
                hipStream_t stream, const Epilogue *ep = nullptr, const BatchLaunch *bl = nullptr,
                const SumsOut *so = nullptr, int64_t geo_mats = 1);

// Whether N columns of an (M, K) product run as one launch of N one-column
// channels (q4k_gemv.hip: the measured rule), on cus CUs.
bool split_columns(int64_t K, int64_t M, int64_t N, int cus);

// Workgroups per weight matrix of a launch over `mats` matrices of M rows:
// the CUs shared among the matrices, at least one, at most one per row; 16
// or more rounded down to a multiple of 8.  Workgroups go to the 8 XCDs
// (each with its own L2) round robin by linear id, so with such a count
// workgroup x of every channel runs on the same XCD, and channels that
// share a weight matrix (broadcasting, several columns as channels) read
// its rows through one L2 (1024 x 4096, three columns as channels: 85
// workgroups each fetched 7.56 MB from beyond the L2s for a 2.36 MB
// weight, against 2.69 MB at two columns and 128).
inline int grid_per_matrix(int cus, int64_t mats, int64_t M) {
    int64_t g = mats > 1 ? cus / mats : cus;
    if (mats > 1 && g >= 16) g -= g % 8;
    if (mats > 1 && g > M) g = M;
    return g < 1 ? 1 : (int)g;
}
inline int64_t pad512(int64_t k) { return (k + 511) / 512 * 512; }
// A 2-D product with a caller workspace quantises the activation in a
// launch of its own and runs the GEMV on the Q8_1 buffer when every
// workgroup's in-launch quantisation of all ncols x K values would cost
// more than that launch (~2 us per call on MI355X): measured crossover
// near 40,000 values (4096 x 14336 at 3 columns even, 4 columns 15.7 vs
// 16.8 us, 8 columns 27.2 vs 35.5 us; 8192 x 28672 at 2 columns 32.0 vs
// 33.2 us; 4096-value rows up to 8 columns stay in one launch).
inline bool prefer_prequantised(int64_t K, int64_t ncols) { return K * ncols > 40960; }
// LDS bytes of one staged q8 column in a tile layout: whole 16-block groups,
// or exactly K in the dense Q6_K layout (whose last, partial group packs its
// chunks 64 bytes per block apart)
inline int q8_col_bytes(int K, bool dense = false) { return dense ? K : (K + 4095) / 4096 * 4096; }

}  // namespace q4k
