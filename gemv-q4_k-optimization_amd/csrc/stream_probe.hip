// stream_probe.hip -- measurement aid, not part of the GEMV library.
//
// A read-only streaming kernel with the GEMV's memory shape: each wave reads
// a contiguous span of `bytes_per_wave` bytes with coalesced 16-byte buffer
// loads, `depth` loads in flight per lane, and folds the data into one word.
// Timing it over the same number of bytes as a GEMV (one launch, inputs in
// HBM) gives the bandwidth a kernel of that size can reach on the device:
// launch, ramp-up and drain included.  Built into libq4k_stream_probe.so by
// build.py and used by bench.py --stream-probe.
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

template <int DEPTH>
__global__ __launch_bounds__(256) void stream_read_kernel(const uint8_t *__restrict__ src,
                                                          uint64_t bytes, uint32_t bytes_per_wave,
                                                          uint32_t *__restrict__ out) {
    const uint32_t lane = threadIdx.x & 63;
    const uint64_t wave = (uint64_t)blockIdx.x * (blockDim.x >> 6) +
                          __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint64_t begin = wave * bytes_per_wave;
    if (begin >= bytes) return;
    const uint64_t span = bytes - begin < bytes_per_wave ? bytes - begin : bytes_per_wave;
    const __amdgpu_buffer_rsrc_t rs =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t *>(src + begin), (short)0,
                                          (int)span, 0x00020000);
    uint32_t acc = 0;
    for (uint32_t off = 0; off < span; off += 1024u * DEPTH) {
        u32x4 v[DEPTH];
#pragma unroll
        for (int k = 0; k < DEPTH; ++k)
            v[k] = __builtin_amdgcn_raw_buffer_load_b128(rs, off + 1024u * k + 16u * lane, 0, 0);
#pragma unroll
        for (int k = 0; k < DEPTH; ++k) acc ^= v[k][0] ^ v[k][1] ^ v[k][2] ^ v[k][3];
    }
    if (acc == 0x9e3779b9u) out[wave] = acc;  // keeps the loads alive
}

}  // namespace

extern "C" int q4k_probe_stream_read(const void *src, uint64_t bytes, uint32_t bytes_per_wave,
                                     int depth, void *out, void *stream) {
    if (!src || !out || bytes_per_wave == 0 || bytes_per_wave % 1024 != 0) return 2;
    const uint64_t waves = (bytes + bytes_per_wave - 1) / bytes_per_wave;
    const dim3 grid((unsigned)((waves + 3) / 4));
    const hipStream_t s = (hipStream_t)stream;
    const uint8_t *p = static_cast<const uint8_t *>(src);
    uint32_t *o = static_cast<uint32_t *>(out);
    switch (depth) {
        case 4: hipLaunchKernelGGL(stream_read_kernel<4>, grid, dim3(256), 0, s, p, bytes, bytes_per_wave, o); break;
        case 8: hipLaunchKernelGGL(stream_read_kernel<8>, grid, dim3(256), 0, s, p, bytes, bytes_per_wave, o); break;
        case 16: hipLaunchKernelGGL(stream_read_kernel<16>, grid, dim3(256), 0, s, p, bytes, bytes_per_wave, o); break;
        default: return 2;
    }
    return hipGetLastError() == hipSuccess ? 0 : 3;
}
