// q4k_gemv.hip -- gfx950 kernels of the Q4_K matrix-vector product and the
// C ABI declared in include/q4k_gemv.h.
//
// Kernels
//   quantize_q8_1_kernel   F32 -> AoS block_q8_1 (the standalone quantiser,
//                          kernels/mmvq.cu:728-735 calls its counterpart)
//   gemv_q4k_kernel        Q4_K x Q8 product.  Each workgroup first stages the
//                          activation as int8 + f32 scales in LDS, quantising
//                          it from F32 itself (one launch per op) or copying an
//                          already-quantised AoS Q8_1 buffer.  Each wave then
//                          owns tiles of R rows and streams them group by group
//                          (8 super-blocks x 144 B per row per step) with
//                          16-byte buffer loads, the next step's loads issued
//                          before the current step's arithmetic.
//   subblock_sums_kernel   parity probe: the int32 sub-block sums computed with
//                          the GEMV's lane map and dot routines.
#include <hip/hip_runtime.h>

#include <atomic>
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <vector>

#include "../../include/q4k_gemv.h"
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
    int G;                   // groups of 8 super-blocks per row
    int ntiles;              // ceil(M / R)
    int vec_ok;              // F32 activation 16-B aligned with ldx % 4 == 0
};

template <int R>
__device__ __forceinline__ void load_group(const GemvParams &p, int tile, int i, int g, int part,
                                           u32x4 (&wq)[R], u32x4 (&wh)[R]) {
    const int row0 = tile * R;
    const int nrows = min(R, p.M - row0);
    const uint8_t *base = p.w + (int64_t)row0 * p.row_stride;
    const __amdgpu_buffer_rsrc_t rs = make_rsrc(base, (uint32_t)(nrows * p.row_stride));
    const int kb = 8 * i + g;
    const uint32_t off = kb < p.nb ? (uint32_t)kb * kBlockBytes : kOOB;
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const uint32_t ro = off + (uint32_t)(r * p.row_stride);
        wh[r] = load16(rs, ro);
        wq[r] = load16(rs, ro + 16u + 16u * (uint32_t)part);
    }
}

template <int NC, int R, int WAVES>
__global__ __launch_bounds__(kWave *WAVES) void gemv_q4k_kernel(GemvParams p) {
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    int8_t *q8s = reinterpret_cast<int8_t *>(lds);
    float *d8s = reinterpret_cast<float *>(lds + NC * p.K);

    if (p.x) {
        stage_from_f32(p.x, p.ldx, p.K, NC, p.vec_ok != 0, q8s, d8s);
    } else {
        stage_from_q8_1(p.y, p.stride_col_y, p.K, NC, q8s, d8s);
    }
    __syncthreads();

    const int lane = threadIdx.x & (kWave - 1);
    const int g = lane >> 3;
    const int part = lane & 7;
    const int jp = part >> 1;
    const int h = part & 1;
    const ScaleSel sel = make_scale_sel(jp);
    const int K = p.K;
    const int nblk32 = K / 32;

    // the wave index is wave-uniform; readfirstlane lets the compiler keep
    // tile numbers and buffer descriptors in scalar registers
    int tile = blockIdx.x * WAVES + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int tstride = gridDim.x * WAVES;
    if (tile >= p.ntiles) return;  // no barrier below this point

    u32x4 wq[R], wh[R];
    load_group<R>(p, tile, 0, g, part, wq, wh);
    int i = 0;
    float acc[R][NC];
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
        for (int c = 0; c < NC; ++c) acc[r][c] = 0.0f;

    for (;;) {
        int ni = i + 1, ntile = tile;
        if (ni == p.G) {
            ni = 0;
            ntile += tstride;
        }
        const bool more = ntile < p.ntiles;
        u32x4 nq[R], nh[R];
        if (more) load_group<R>(p, ntile, ni, g, part, nq, nh);

        // activation slice of this lane for group i
        const int kb = 8 * i + g;
        const int kbc = kb < p.nb ? kb : 0;
        u32x4 alo[NC], ahi[NC];
        float d8a[NC], d8b[NC], ka[NC], kbv[NC];
#pragma unroll
        for (int c = 0; c < NC; ++c) {
            const int8_t *qa = q8s + c * K + kbc * kQK + jp * 64 + h * 16;
            alo[c] = *reinterpret_cast<const u32x4 *>(qa);
            ahi[c] = *reinterpret_cast<const u32x4 *>(qa + 32);
            const float2 dd = *reinterpret_cast<const float2 *>(d8s + c * nblk32 + kbc * 8 + jp * 2);
            d8a[c] = dd.x;
            d8b[c] = dd.y;
            ka[c] = dd.x * (float)byte_sum16(alo[c]);
            kbv[c] = dd.y * (float)byte_sum16(ahi[c]);
        }

#pragma unroll
        for (int r = 0; r < R; ++r) {
            const uint32_t scm = unpack_scale_min(wh[r], sel);
            const int sca = (int)(scm & 0xffu);
            const int scb = (int)((scm >> 8) & 0xffu);
            const float maf = (float)((scm >> 16) & 0xffu);
            const float mbf = (float)(scm >> 24);
            const float d = half_bits_to_float(wh[r][0]);
            const float dmin = half_bits_to_float(wh[r][0] >> 16);
#pragma unroll
            for (int c = 0; c < NC; ++c) {
                int sa, sb;
                lane_qdot(wq[r], alo[c], ahi[c], sa, sb);
                const float xs = d8a[c] * (float)(sa * sca) + d8b[c] * (float)(sb * scb);
                const float ms = ka[c] * maf + kbv[c] * mbf;
                acc[r][c] = fmaf(d, xs, acc[r][c]);
                acc[r][c] = fmaf(-dmin, ms, acc[r][c]);
            }
        }

        if (i == p.G - 1) {
            float out = 0.0f;
#pragma unroll
            for (int r = 0; r < R; ++r)
#pragma unroll
                for (int c = 0; c < NC; ++c) {
                    const float s = wave_sum(acc[r][c]);
                    if (lane == r * NC + c) out = s;
                    acc[r][c] = 0.0f;
                }
            const int r = lane / NC;
            const int c = lane - r * NC;
            const int row = tile * R + r;
            if (lane < R * NC && row < p.M) p.dst[(int64_t)c * p.ld_dst + row] = out;
        }
        if (!more) break;
#pragma unroll
        for (int r = 0; r < R; ++r) {
            wq[r] = nq[r];
            wh[r] = nh[r];
        }
        tile = ntile;
        i = ni;
    }
}

// ggml-cuda quantize_q8_1 arithmetic, one value per lane, 32 lanes per block:
// amax and sum reduced over the 32 lanes with xor distances 16, 8, 4, 2, 1.
__global__ __launch_bounds__(256) void quantize_q8_1_kernel(const float *__restrict__ x,
                                                            uint8_t *__restrict__ vy, int64_t ne00,
                                                            int64_t s01, int64_t ne0) {
    const int64_t i0 = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i0 >= ne0) return;  // ne0 % 32 == 0: whole 32-lane groups leave together
    const int64_t col = blockIdx.y;
    const float xi = i0 < ne00 ? x[col * s01 + i0] : 0.0f;
    float amax = fabsf(xi);
    float sum = xi;
    amax = fmaxf(amax, swizzle_xor<16>(amax)); sum += swizzle_xor<16>(sum);
    amax = fmaxf(amax, swizzle_xor<8>(amax));  sum += swizzle_xor<8>(sum);
    amax = fmaxf(amax, swizzle_xor<4>(amax));  sum += swizzle_xor<4>(sum);
    amax = fmaxf(amax, swizzle_xor<2>(amax));  sum += swizzle_xor<2>(sum);
    amax = fmaxf(amax, swizzle_xor<1>(amax));  sum += swizzle_xor<1>(sum);
    const float d = amax / 127.0f;
    const int q = amax == 0.0f ? 0 : (int)roundf(xi / d);
    const int64_t ic = col * ne0 + i0;
    uint8_t *blk = vy + (ic / 32) * kQ81Bytes;
    const int iqs = (int)(ic & 31);
    blk[4 + iqs] = (uint8_t)(int8_t)q;
    if (iqs == 0) {
        const uint16_t dh = __builtin_bit_cast(uint16_t, (_Float16)d);
        const uint16_t sh = __builtin_bit_cast(uint16_t, (_Float16)sum);
        *reinterpret_cast<uint32_t *>(blk) = (uint32_t)dh | ((uint32_t)sh << 16);
    }
}

struct SumsParams {
    const uint8_t *w;
    int64_t row_stride;
    const uint8_t *y;  // one column of AoS Q8_1
    int32_t *sqq;      // [M][K/32] for this column
    int32_t *sq;       // [K/32] for this column
    int M, K, nb, G;
};

// One wave per (row, group): the GEMV's lane map and lane_qdot, then the two
// lanes that share a sub-block (p and p^1) are added.
__global__ __launch_bounds__(256) void subblock_sums_kernel(SumsParams p) {
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    int8_t *q8s = reinterpret_cast<int8_t *>(lds);
    float *d8s = reinterpret_cast<float *>(lds + p.K);
    stage_from_q8_1(p.y, 0, p.K, 1, q8s, d8s);
    __syncthreads();
    const int lane = threadIdx.x & 63;
    const int g = lane >> 3, part = lane & 7, jp = part >> 1, h = part & 1;
    const int nitems = p.M * p.G;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    for (int item = blockIdx.x * 4 + wave; item < nitems; item += gridDim.x * 4) {
        const int row = item / p.G;
        const int i = item - row * p.G;
        u32x4 wq[1], wh[1];
        GemvParams gp{};
        gp.w = p.w;
        gp.row_stride = p.row_stride;
        gp.M = p.M;
        gp.nb = p.nb;
        load_group<1>(gp, row, i, g, part, wq, wh);
        const int kb = 8 * i + g;
        const int kbc = kb < p.nb ? kb : 0;
        const int8_t *qa = q8s + kbc * kQK + jp * 64 + h * 16;
        const u32x4 alo = *reinterpret_cast<const u32x4 *>(qa);
        const u32x4 ahi = *reinterpret_cast<const u32x4 *>(qa + 32);
        int sa, sb;
        lane_qdot(wq[0], alo, ahi, sa, sb);
        int qa_sum = byte_sum16(alo), qb_sum = byte_sum16(ahi);
        sa += dpp<kDppXor1>(sa);
        sb += dpp<kDppXor1>(sb);
        qa_sum += dpp<kDppXor1>(qa_sum);
        qb_sum += dpp<kDppXor1>(qb_sum);
        if (h == 0 && kb < p.nb) {
            int32_t *o = p.sqq + (int64_t)row * (p.K / 32) + kb * 8 + jp * 2;
            o[0] = sa;
            o[1] = sb;
            if (row == 0) {
                p.sq[kb * 8 + jp * 2] = qa_sum;
                p.sq[kb * 8 + jp * 2 + 1] = qb_sum;
            }
        }
    }
}

// ------------------------------------------------------------------------
// host side
// ------------------------------------------------------------------------

static thread_local int32_t g_last_hip_error = 0;

static int hip_fail(hipError_t e) {
    g_last_hip_error = (int32_t)e;
    return Q4K_EHIP;
}

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

static constexpr int kMaxDevices = 64;
static DeviceInfo g_dev[kMaxDevices];

static int device_info(DeviceInfo **out) {
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

static int ensure_lds(DeviceInfo *di, const void *fn, int bytes) {
    if (bytes <= 65536) return Q4K_OK;
    std::lock_guard<std::mutex> lk(di->attr_mu);
    for (const void *f : di->attr_done)
        if (f == fn) return Q4K_OK;
    hipError_t e = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, di->max_lds);
    if (e != hipSuccess) return hip_fail(e);
    di->attr_done.push_back(fn);
    return Q4K_OK;
}

static int env_int(const char *name, int dflt) {
    const char *v = std::getenv(name);
    return v && *v ? std::atoi(v) : dflt;
}

struct Geometry {
    int R = 4;
    int waves = 4;
    int grid = 0;
    int lds = 0;
    int nc_chunk = 1;
    int ntiles = 0;
};

static int lds_bytes(int K, int nc) { return nc * (K + K / 8); }

// Rows per wave tile, waves per workgroup and grid for an (M, K, N) product.
// Environment overrides for sweeps: Q4K_ROWS (1, 2, 4), Q4K_WAVES (4, 8),
// Q4K_WGS (workgroups), Q4K_WGS_PER_CU.
static Geometry pick_geometry(const DeviceInfo &di, int64_t K, int64_t M, int64_t N) {
    Geometry g;
    const int max_lds = di.max_lds > 0 ? di.max_lds : 65536;
    int nc = (int)N;
    while (nc > 1 && lds_bytes((int)K, nc) > max_lds) nc = (nc + 1) / 2;
    g.nc_chunk = nc;
    g.lds = lds_bytes((int)K, nc);
    g.R = nc == 1 ? 4 : 2;
    g.waves = g.lds > 40 * 1024 ? 8 : 4;
    g.R = env_int("Q4K_ROWS", g.R);
    if (g.R != 1 && g.R != 2 && g.R != 4) g.R = 2;
    g.waves = env_int("Q4K_WAVES", g.waves);
    if (g.waves != 4 && g.waves != 8) g.waves = 4;
    g.ntiles = (int)((M + g.R - 1) / g.R);
    const int wg_needed = (g.ntiles + g.waves - 1) / g.waves;
    int per_cu = max_lds / (g.lds > 0 ? g.lds : 1);
    if (per_cu < 1) per_cu = 1;
    if (per_cu > 8) per_cu = 8;
    per_cu = env_int("Q4K_WGS_PER_CU", per_cu);
    int wgs = di.cus * per_cu;
    wgs = env_int("Q4K_WGS", wgs);
    if (wgs < 1) wgs = 1;
    g.grid = wg_needed < wgs ? wg_needed : wgs;
    return g;
}

typedef void (*gemv_fn_t)(GemvParams);

template <int NC, int R, int WAVES>
static const void *gemv_sym() {
    return reinterpret_cast<const void *>(&gemv_q4k_kernel<NC, R, WAVES>);
}

template <int R, int WAVES>
static const void *gemv_sym_nc(int nc) {
    switch (nc) {
        case 1: return gemv_sym<1, R, WAVES>();
        case 2: return gemv_sym<2, R, WAVES>();
        case 3: return gemv_sym<3, R, WAVES>();
        case 4: return gemv_sym<4, R, WAVES>();
        case 5: return gemv_sym<5, R, WAVES>();
        case 6: return gemv_sym<6, R, WAVES>();
        case 7: return gemv_sym<7, R, WAVES>();
        case 8: return gemv_sym<8, R, WAVES>();
        default: return nullptr;
    }
}

static const void *gemv_kernel_for(int nc, int R, int waves) {
    if (waves == 4) {
        if (R == 1) return gemv_sym_nc<1, 4>(nc);
        if (R == 2) return gemv_sym_nc<2, 4>(nc);
        return gemv_sym_nc<4, 4>(nc);
    }
    if (R == 1) return gemv_sym_nc<1, 8>(nc);
    if (R == 2) return gemv_sym_nc<2, 8>(nc);
    return gemv_sym_nc<4, 8>(nc);
}

static int launch_gemv(DeviceInfo *di, const Geometry &geo, GemvParams p, int nc, hipStream_t stream) {
    const void *fn = gemv_kernel_for(nc, geo.R, geo.waves);
    if (!fn) return Q4K_EINVAL;
    int st = ensure_lds(di, fn, geo.lds);
    if (st != Q4K_OK) return st;
    void *args[] = {&p};
    hipError_t e = hipLaunchKernel(fn, dim3(geo.grid), dim3(kWave * geo.waves), args, (size_t)geo.lds,
                                   stream);
    if (e != hipSuccess) return hip_fail(e);
    e = hipGetLastError();
    if (e != hipSuccess) return hip_fail(e);
    return Q4K_OK;
}

static bool aligned(const void *p, uintptr_t a) { return ((uintptr_t)p & (a - 1)) == 0; }

static int64_t pad512(int64_t k) { return (k + 511) / 512 * 512; }

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
                    int64_t ld_dst, hipStream_t stream) {
    DeviceInfo *di = nullptr;
    int st = device_info(&di);
    if (st != Q4K_OK) return st;
    const Geometry geo = pick_geometry(*di, ne00, ne01, ncols);
    for (int64_t c0 = 0; c0 < ncols; c0 += geo.nc_chunk) {
        const int nc = (int)(ncols - c0 < geo.nc_chunk ? ncols - c0 : geo.nc_chunk);
        Geometry g2 = geo;
        g2.lds = lds_bytes((int)ne00, nc);
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
        p.G = (p.nb + 7) / 8;
        p.ntiles = geo.ntiles;
        p.vec_ok = x && aligned(p.x, 16) && (ldx % 4 == 0);
        st = launch_gemv(di, g2, p, nc, stream);
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
        case Q4K_ENOMEM: return "out of device memory";
        default: return "unknown status";
    }
}

int32_t q4k_last_hip_error(void) { return g_last_hip_error; }

size_t q4k_q8_1_bytes(int64_t ne10, int64_t ne11) {
    if (ne10 < 0 || ne11 < 0) return 0;
    return (size_t)(ne11 * (pad512(ne10) / 32) * kQ81Bytes);
}

int q4k_quantize_row_q8_1(const float *x, void *vy, int64_t ne00, int64_t s01, int64_t ne0,
                          int64_t ne1, void *stream) {
    if (ne00 < 0 || ne1 < 0 || ne0 < ne00 || ne0 % 32 != 0) return Q4K_EINVAL;
    if (ne0 == 0 || ne1 == 0) return Q4K_OK;
    if (!x || !vy || (ne1 > 1 && s01 < ne00) || ne1 > 65535) return Q4K_EINVAL;
    if (!aligned(vy, 4)) return Q4K_EINVAL;
    DeviceInfo *di = nullptr;
    int st = device_info(&di);
    if (st != Q4K_OK) return st;
    const dim3 grid((unsigned)((ne0 + 255) / 256), (unsigned)ne1);
    hipLaunchKernelGGL(quantize_q8_1_kernel, grid, dim3(256), 0, (hipStream_t)stream, x,
                       static_cast<uint8_t *>(vy), ne00, s01, ne0);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return hip_fail(e);
    return Q4K_OK;
}

int q4k_mul_mat_vec_q(const void *src0, int64_t ne00, int64_t ne01, int64_t nb01, const float *src1,
                      int64_t ne11, int64_t nb11, float *dst, int64_t nb1, void *workspace,
                      size_t workspace_bytes, void *stream) {
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
    if (geo.nc_chunk >= ne11) {
        // quantisation inside the GEMV launch
        return run_gemv(src0, ne00, ne01, nb01, src1, ldx, nullptr, 0, ne11, dst, ldd, s);
    }
    // activation too large for one workgroup's LDS at this column count:
    // quantise once to a Q8_1 buffer and run the GEMV in column chunks.
    const size_t need = q4k_q8_1_bytes(ne00, ne11);
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
                      ne11, dst, ldd, s);
    if (owned) {
        hipError_t e = hipFreeAsync(buf, s);
        if (e != hipSuccess && st == Q4K_OK) st = hip_fail(e);
    }
    return st;
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

int q4k_ggml_mul_mat_vec_q(const q4k_tensor *src0, const q4k_tensor *src1, const q4k_tensor *ids,
                           q4k_tensor *dst, const void *fusion, void *workspace,
                           size_t workspace_bytes, void *stream) {
    if (!src0 || !src1 || !dst) return Q4K_EINVAL;
    if (src1->type != Q4K_GGML_TYPE_F32 || dst->type != Q4K_GGML_TYPE_F32) return Q4K_EINVAL;
    if (src0->type != Q4K_GGML_TYPE_Q4_K) return Q4K_EUNSUPPORTED;
    if (src0->nb[0] != (size_t)kBlockBytes || src1->nb[0] != 4 || dst->nb[0] != 4) return Q4K_EINVAL;
    if (ids || fusion) return Q4K_EUNSUPPORTED;
    for (int d = 2; d < 4; ++d)
        if (src0->ne[d] != 1 || src1->ne[d] != 1 || dst->ne[d] != 1) return Q4K_EUNSUPPORTED;
    if (src1->ne[0] != src0->ne[0] || dst->ne[0] != src0->ne[1] || dst->ne[1] != src1->ne[1])
        return Q4K_EINVAL;
    // ggml's nb00 is the block size: ne00 counts values, ne00/256 blocks per row
    return q4k_mul_mat_vec_q(src0->data, src0->ne[0], src0->ne[1], (int64_t)src0->nb[1],
                             static_cast<const float *>(src1->data), src1->ne[1],
                             (int64_t)src1->nb[1], static_cast<float *>(dst->data),
                             (int64_t)dst->nb[1], workspace, workspace_bytes, stream);
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
        p.G = (nb + 7) / 8;
        const int64_t items = ne01 * p.G;
        int grid = (int)((items + 3) / 4);
        if (grid > di->cus * 8) grid = di->cus * 8;
        hipLaunchKernelGGL(subblock_sums_kernel, dim3(grid), dim3(256), (size_t)lds,
                           (hipStream_t)stream, p);
        hipError_t e = hipGetLastError();
        if (e != hipSuccess) return hip_fail(e);
    }
    return Q4K_OK;
}

int q4k_gemv_geometry(int64_t ne00, int64_t ne01, int64_t ne11, int32_t out[6]) {
    if (!out || ne00 <= 0 || ne00 % kQK != 0 || ne01 < 0 || ne11 < 1 || ne11 > Q4K_MAX_BATCH)
        return Q4K_EINVAL;
    DeviceInfo *di = nullptr;
    int st = device_info(&di);
    if (st != Q4K_OK) return st;
    const Geometry g = pick_geometry(*di, ne00, ne01, ne11);
    out[0] = g.R;
    out[1] = g.waves;
    out[2] = g.grid;
    out[3] = g.lds;
    out[4] = g.nc_chunk;
    out[5] = g.nc_chunk >= ne11 ? 1 : 0;
    return Q4K_OK;
}

}  // extern "C"
