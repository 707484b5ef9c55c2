// q4k_probe.hip -- a plain streaming read of device memory, the ceiling the
// GEMV kernels are measured against (bench.py --read-ceiling).  Not part of
// the GEMV path: the product entry points never launch it.
//
// Wave w of the grid reads bytes [w*per_wave, (w+1)*per_wave) of the buffer
// with 16-byte loads, 64 lanes x 16 B = 1 KB per load instruction, INFL
// instructions in flight at a time (issued together, then consumed), and
// folds the data into one word per lane; lane 0 of each wave stores the
// wave's xor into sink[w], so no load is dead.  Loads past the buffer end
// read zeros (buffer descriptor), so any grid is in bounds.
#include <hip/hip_runtime.h>

#include "../../include/q4k_gemv.h"
#include "q4k_device.h"
#include "q4k_runtime.h"

namespace q4k {

template <int WAVES, int INFL>
__global__ __launch_bounds__(kWave *WAVES) void read_probe_kernel(const uint8_t *__restrict__ src, uint32_t bytes,
                                                                   uint32_t per_wave, uint32_t *__restrict__ sink) {
    const int lane = threadIdx.x & (kWave - 1);
    const uint32_t wave = blockIdx.x * WAVES + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const __amdgpu_buffer_rsrc_t rs = make_rsrc(src, bytes);
    const uint32_t beg = wave * per_wave;
    uint32_t acc = 0;
    for (uint32_t o = 0; o < per_wave; o += INFL * 1024u) {
        u32x4 v[INFL];
#pragma unroll
        for (int k = 0; k < INFL; ++k) {
            const uint32_t off = beg + o + 1024u * k + 16u * lane;
            v[k] = load16(rs, o + 1024u * k < per_wave ? off : kOOB);
        }
#pragma unroll
        for (int k = 0; k < INFL; ++k) acc ^= v[k][0] ^ v[k][1] ^ v[k][2] ^ v[k][3];
    }
    acc = (uint32_t)__builtin_amdgcn_readfirstlane((int)acc) ^ (uint32_t)lane;
    if (lane == 0) sink[wave] = acc;
}

template <int WAVES>
static const void *read_probe_sym(int infl) {
    switch (infl) {
        case 1: return reinterpret_cast<const void *>(&read_probe_kernel<WAVES, 1>);
        case 2: return reinterpret_cast<const void *>(&read_probe_kernel<WAVES, 2>);
        case 4: return reinterpret_cast<const void *>(&read_probe_kernel<WAVES, 4>);
        case 8: return reinterpret_cast<const void *>(&read_probe_kernel<WAVES, 8>);
        default: return nullptr;
    }
}

}  // namespace q4k

using namespace q4k;

extern "C" int q4k_read_probe(const void *src, size_t bytes, int32_t workgroups, int32_t waves_per_wg,
                              int32_t bytes_per_wave, int32_t loads_in_flight, uint32_t *sink, void *stream) {
    if (!src || !sink || bytes == 0 || bytes >= ((size_t)1 << 31) || workgroups < 1 || bytes_per_wave < 1024 ||
        bytes_per_wave % 1024 != 0)
        return Q4K_EINVAL;
    if ((int64_t)workgroups * waves_per_wg * bytes_per_wave >= ((int64_t)1 << 32)) return Q4K_EINVAL;
    const void *fn = waves_per_wg == 4    ? read_probe_sym<4>(loads_in_flight)
                     : waves_per_wg == 8  ? read_probe_sym<8>(loads_in_flight)
                     : waves_per_wg == 16 ? read_probe_sym<16>(loads_in_flight)
                                          : nullptr;
    if (!fn) return Q4K_EINVAL;
    uint32_t b = (uint32_t)bytes, pw = (uint32_t)bytes_per_wave;
    void *args[] = {(void *)&src, &b, &pw, &sink};
    const hipError_t e =
        hipLaunchKernel(fn, dim3((unsigned)workgroups), dim3(kWave * waves_per_wg), args, 0, (hipStream_t)stream);
    if (e != hipSuccess) return hip_fail(e);
    return Q4K_OK;
}
