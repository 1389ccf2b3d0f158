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

// PER 16-byte loads per thread, all issued before any is used.  One-shot
// (stride 0): the grid covers the buffer once, each block a contiguous
// 256 * PER * 16 bytes.  Grid-stride (stride = grid size in threads): every
// thread walks the buffer in rounds of PER loads.
template <int PER>
__global__ __launch_bounds__(256) void stream_read_kernel(const u32x4* __restrict__ src, long n16, long stride,
                                                          uint32_t* __restrict__ sink) {
    uint32_t x = 0;
    const long first = static_cast<long>(blockIdx.x) * 256 * PER + threadIdx.x;
    const long step = stride == 0 ? n16 : stride * PER;  // one round when one-shot
    const long lane_step = stride == 0 ? 256 : stride;
    for (long base = stride == 0 ? first : static_cast<long>(blockIdx.x) * 256 + threadIdx.x; base < n16;
         base += step) {
        u32x4 v[PER];
#pragma unroll
        for (int i = 0; i < PER; ++i) {
            const long idx = base + lane_step * i;
            v[i] = src[idx < n16 ? idx : n16 - 1];  // past the end: the last chunk again (in bounds)
        }
#pragma unroll
        for (int i = 0; i < PER; ++i) x ^= v[i].x ^ v[i].y ^ v[i].z ^ v[i].w;
    }
    if (x == 0x9E3779B9u) sink[0] = x;
}

// The GPU's constant-rate clock (100 MHz, s_memrealtime) written to *dst by
// one lane: a timestamp between the kernels of a captured graph.
__global__ void timestamp_kernel(unsigned long long* __restrict__ dst) {
    if (threadIdx.x == 0) *dst = wall_clock64();
}

}  // namespace dev

namespace detail {

int launch_timestamp(unsigned long long* dst, hipStream_t stream) {
    hipLaunchKernelGGL(dev::timestamp_kernel, dim3(1), dim3(64), 0, stream, dst);
    return 0;
}

template <int PER>
static int launch_read(const void* src, long n16, long blocks, long stride, uint32_t* sink, hipStream_t stream) {
    hipLaunchKernelGGL(dev::stream_read_kernel<PER>, dim3(static_cast<unsigned>(blocks)), dim3(256), 0, stream,
                       static_cast<const dev::u32x4*>(src), n16, stride, sink);
    return 0;
}

int launch_stream_read_ex(const void* src, long n_bytes, uint32_t* sink, int per, long grid_blocks,
                          hipStream_t stream) {
    const long n16 = n_bytes / 16;
    long blocks = grid_blocks;
    long stride = 0;
    if (grid_blocks <= 0)
        blocks = (n16 + 256L * per - 1) / (256L * per);
    else
        stride = grid_blocks * 256;
    if (blocks < 1 || blocks > 0x7FFFFFFFL) return kDeclined;
    switch (per) {
        case 1: return launch_read<1>(src, n16, blocks, stride, sink, stream);
        case 2: return launch_read<2>(src, n16, blocks, stride, sink, stream);
        case 4: return launch_read<4>(src, n16, blocks, stride, sink, stream);
        case 8: return launch_read<8>(src, n16, blocks, stride, sink, stream);
        case 16: return launch_read<16>(src, n16, blocks, stride, sink, stream);
    }
    return kDeclined;
}

int launch_stream_read(const void* src, long n_bytes, uint32_t* sink, hipStream_t stream) {
    return launch_stream_read_ex(src, n_bytes, sink, 4, 0, stream);
}

}  // namespace detail
}  // namespace cri
