// probe.hip -- a bare streaming read, the achievable-bandwidth line that the
// GEMV rooflines are read against (measurement aid; no counterpart in the
// reference).  Every thread issues its four 16-byte loads before using any,
// the words are XOR-combined and written only in the (practically
// impossible) case that the combination hits a fixed constant, so the loads
// cannot be removed and nothing else is written.
#include "common.hpp"
#include "internal.hpp"

namespace cri {
namespace dev {

constexpr int kProbePer = 4;  // 16-byte loads per thread

__global__ __launch_bounds__(256) void stream_read_kernel(const u32x4* __restrict__ src, long n16,
                                                          uint32_t* __restrict__ sink) {
    const long base = static_cast<long>(blockIdx.x) * 256 * kProbePer + threadIdx.x;
    u32x4 v[kProbePer];
#pragma unroll
    for (int i = 0; i < kProbePer; ++i) {
        const long idx = base + 256L * i;
        v[i] = src[idx < n16 ? idx : n16 - 1];  // past the end: the last chunk again (in bounds)
    }
    uint32_t x = 0;
#pragma unroll
    for (int i = 0; i < kProbePer; ++i) x ^= v[i].x ^ v[i].y ^ v[i].z ^ v[i].w;
    if (x == 0x9E3779B9u) sink[0] = x;
}

}  // namespace dev

namespace detail {

int launch_stream_read(const void* src, long n_bytes, uint32_t* sink, hipStream_t stream) {
    const long n16 = n_bytes / 16;
    const long blocks = (n16 + 256L * dev::kProbePer - 1) / (256L * dev::kProbePer);
    if (blocks > 0x7FFFFFFFL) return -1;
    hipLaunchKernelGGL(dev::stream_read_kernel, dim3(static_cast<unsigned>(blocks)), dim3(256), 0, stream,
                       static_cast<const dev::u32x4*>(src), n16, sink);
    return 0;
}

}  // namespace detail
}  // namespace cri
