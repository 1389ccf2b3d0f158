// dequant.hip -- standalone block -> fp32 dequantisation.
//
// Replaces kernel_dequantize_{q8_0,q4_0,q5_0,q6_k,q4_k}
// (ref:src/kernels/dequantize.cu:34-336).  Output-bandwidth bound (4 bytes
// written per element), so each thread produces 8 consecutive floats with two
// 16-byte stores and a wave writes 2 KiB of contiguous output per step.  The
// element formulas are the reference's, so results are bit-identical.
#include "common.hpp"
#include "decode.hpp"
#include "internal.hpp"

namespace cri {
namespace dev {

template <int FMT, int BE, int BB>
__global__ __launch_bounds__(256) void dequant_kernel(const uint8_t* __restrict__ src, float* __restrict__ dst,
                                                      long n_groups) {
    const long g = static_cast<long>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (g >= n_groups) return;
    const long e0 = g * 8;  // first element
    const long b = e0 / BE;
    const int e = static_cast<int>(e0 - b * BE);
    const uint8_t* blk = src + b * BB;
    float v[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        if constexpr (FMT == kFmtQ8_0) v[i] = decode_q8_0(blk, e + i);
        else if constexpr (FMT == kFmtQ4_0) v[i] = decode_q4_0(blk, e + i);
        else if constexpr (FMT == kFmtQ5_0) v[i] = decode_q5_0(blk, e + i);
        else if constexpr (FMT == kFmtQ4_K) v[i] = decode_q4_k(blk, e + i);
        else v[i] = decode_q6_k(blk, e + i);
    }
    f32x4_a4* out = reinterpret_cast<f32x4_a4*>(dst + e0);  // dst only needs float alignment
    out[0] = f32x4_a4{v[0], v[1], v[2], v[3]};
    out[1] = f32x4_a4{v[4], v[5], v[6], v[7]};
}

}  // namespace dev

namespace detail {

template <int FMT, int BE, int BB>
static void launch_dq(const void* src, float* dst, long n_blocks, hipStream_t stream) {
    const long groups = n_blocks * BE / 8;
    const long blocks = (groups + 255) / 256;
    hipLaunchKernelGGL((dev::dequant_kernel<FMT, BE, BB>), dim3(static_cast<unsigned>(blocks)), dim3(256), 0,
                       stream, static_cast<const uint8_t*>(src), dst, groups);
}

int launch_dequant(int fmt, const void* src, float* dst, long n_blocks, hipStream_t stream) {
    if (n_blocks <= 0) return 0;
    switch (fmt) {
        case kFmtQ8_0: launch_dq<kFmtQ8_0, 32, 34>(src, dst, n_blocks, stream); return 0;
        case kFmtQ4_0: launch_dq<kFmtQ4_0, 32, 18>(src, dst, n_blocks, stream); return 0;
        case kFmtQ5_0: launch_dq<kFmtQ5_0, 32, 22>(src, dst, n_blocks, stream); return 0;
        case kFmtQ4_K: launch_dq<kFmtQ4_K, 256, 144>(src, dst, n_blocks, stream); return 0;
        case kFmtQ6_K: launch_dq<kFmtQ6_K, 256, 210>(src, dst, n_blocks, stream); return 0;
    }
    return -1;
}

}  // namespace detail
}  // namespace cri
