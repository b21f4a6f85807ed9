// hbm_probe.hip - a read-only streaming kernel: the ceiling against which the
// read-dominated attention passes are measured (a device copy moves as many
// bytes out as in, so it is no bound for a pass that reads 1000x what it
// writes).
//
// Each workgroup reads one contiguous range with non-temporal 16-byte loads,
// eight in flight per lane (consecutive lanes on consecutive words: 1 KB per
// wave and load), four workgroups per CU; the XOR of everything read leaves
// as one word per wave, so the loads cannot be dropped.  Measured on MI355X
// over 2 GiB, this shape reads at 6.8-7.1 TB/s; grid-stride loops over the
// whole buffer, cached loads or more workgroups per CU read at 5.3-6.2.

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdio.h>

#include "q8_common.h"

using namespace gfa;

namespace {

constexpr int SR_THREADS = 256;
constexpr int SR_WGS_PER_CU = 4;
constexpr int SR_UNROLL = 8;

__global__ __launch_bounds__(SR_THREADS) void stream_read_kernel(const u32x4 *src, int64_t n, uint32_t *out) {
    const int64_t per = (n + gridDim.x - 1) / gridDim.x;
    const int64_t b0 = min((int64_t)blockIdx.x * per, n), b1 = min(b0 + per, n);
    uint32_t acc = 0;
    int64_t i = b0 + threadIdx.x;
    for (; i + (SR_UNROLL - 1) * SR_THREADS < b1; i += SR_UNROLL * SR_THREADS) {
        u32x4 x = {0u, 0u, 0u, 0u};
#pragma unroll
        for (int u = 0; u < SR_UNROLL; ++u) x ^= __builtin_nontemporal_load(src + i + u * SR_THREADS);
        acc ^= (x[0] ^ x[1]) ^ (x[2] ^ x[3]);
    }
    for (; i < b1; i += SR_THREADS) {
        const u32x4 x = __builtin_nontemporal_load(src + i);
        acc ^= (x[0] ^ x[1]) ^ (x[2] ^ x[3]);
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) acc ^= (uint32_t)__shfl_xor((int)acc, off);
    if ((threadIdx.x & 63) == 0) out[((int64_t)blockIdx.x * SR_THREADS + threadIdx.x) >> 6] = acc;
}

}  // namespace

extern "C" int gfx906_fa_amd_stream_read_words(void) {
    int dev = 0, cus = 256;
    if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        cus <= 0)
        cus = 256;
    return cus * SR_WGS_PER_CU * (SR_THREADS / 64);  // one word per wave
}

extern "C" hipError_t gfx906_fa_amd_stream_read(const void *src, int64_t bytes, uint32_t *out, int out_words,
                                                hipStream_t stream) {
    if (bytes == 0) return hipSuccess;
    const int need = gfx906_fa_amd_stream_read_words();
    if (src == nullptr || out == nullptr || bytes < 0 || (bytes & 15) || ((uintptr_t)src & 15) ||
        out_words < need) {
        fprintf(stderr,
                "[gfx906_fa_amd] stream_read: need a 16-byte aligned source, a byte count that is a multiple of "
                "16 and %d output words (got %d)\n", need, out_words);
        return hipErrorInvalidValue;
    }
    const int grid = need / (SR_THREADS / 64);
    stream_read_kernel<<<grid, SR_THREADS, 0, stream>>>(static_cast<const u32x4 *>(src), bytes / 16, out);
    return hipGetLastError();
}
