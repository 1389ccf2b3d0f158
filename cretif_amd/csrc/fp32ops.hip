// fp32ops.hip -- the two fp32 neighbours of the fused path.
//
// matmul_transposed_b: C = A * B^T with B [N,K] fp32 (the tied LM head,
//   ref:src/embedding.cu:85-135).  M == 1 runs the streaming GEMV (one pass over
//   B with coalesced 16-byte loads, activations in VGPRs); other shapes use the
//   LDS-tiled fallback.
// batched_matmul_gqa: C[h] = A[h] * B[h / G] with A [H,M,K], B [Hkv,K,N]
//   (ref:src/attention.cu:192-218).  One block serves all G query heads of a KV
//   head, so each B tile is read once per group instead of once per head; when
//   the (kv head, n tile) grid alone is too small to fill the GPU the K range is
//   split across blocks and partial sums are combined with fp32 atomics into a
//   zero-filled C.
#include "common.hpp"
#include "internal.hpp"

namespace cri {
namespace dev {

__global__ __launch_bounds__(256) void fill_zero_kernel(float* __restrict__ p, long n) {
    const long i = static_cast<long>(blockIdx.x) * blockDim.x + threadIdx.x;
    const long stride = static_cast<long>(gridDim.x) * blockDim.x;
    for (long j = i; j < n; j += stride) p[j] = 0.0f;
}

constexpr int kQTN = 64;  // n per tile
constexpr int kQTR = 16;  // (head, m) rows per tile
constexpr int kQTK = 32;  // k per LDS stage

__global__ __launch_bounds__(256) void gqa_kernel(const float* __restrict__ A, const float* __restrict__ B,
                                                  float* __restrict__ C, int G, int M, int N, int K,
                                                  int k_split, int splits, int atomic) {
    __shared__ float as[kQTR][kQTK + 1];
    __shared__ float bs[kQTK][kQTN];
    const int tid = threadIdx.x;
    const int n0 = blockIdx.x * kQTN;
    const int r0 = blockIdx.y * kQTR;
    const int kv = blockIdx.z / splits;
    const int split = blockIdx.z - kv * splits;
    const int kb = split * k_split;
    const int ke = min(K, kb + k_split);
    const int R = G * M;  // rows of this KV group: (head in group, m)
    const float* Bk = B + static_cast<long>(kv) * K * N;
    const int tn = tid & 63, tr = (tid >> 6) * 4;
    float acc[4] = {0.f, 0.f, 0.f, 0.f};

    for (int k0 = kb; k0 < ke; k0 += kQTK) {
        // A tile: 16 rows x 32 k, 2 floats per thread
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const int idx = tid + 256 * i;
            const int rr = idx >> 5, kk = idx & 31;
            const int r = r0 + rr, k = k0 + kk;
            float v = 0.0f;
            if (r < R && k < ke) {
                const int head = kv * G + r / M, m = r - (r / M) * M;
                v = A[(static_cast<long>(head) * M + m) * K + k];
            }
            as[rr][kk] = v;
        }
        // B tile: 32 k x 64 n, coalesced along n
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const int kk = (tid >> 6) + 4 * i, nn = tid & 63;
            const int k = k0 + kk, n = n0 + nn;
            bs[kk][nn] = (k < ke && n < N) ? Bk[static_cast<long>(k) * N + n] : 0.0f;
        }
        __syncthreads();
#pragma unroll 8
        for (int kk = 0; kk < kQTK; ++kk) {
            const float b = bs[kk][tn];
#pragma unroll
            for (int i = 0; i < 4; ++i) acc[i] = __builtin_fmaf(as[tr + i][kk], b, acc[i]);
        }
        __syncthreads();
    }
    const int n = n0 + tn;
    if (n >= N) return;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int r = r0 + tr + i;
        if (r >= R) continue;
        const int head = kv * G + r / M, m = r - (r / M) * M;
        float* dst = C + (static_cast<long>(head) * M + m) * N + n;
        if (atomic) atomicAdd(dst, acc[i]);
        else *dst = acc[i];
    }
}

}  // namespace dev

namespace detail {

void launch_fill_zero(float* C, long n, hipStream_t stream) {
    if (n <= 0) return;
    const long blocks = (n + 255) / 256 < 4096 ? (n + 255) / 256 : 4096;
    hipLaunchKernelGGL(dev::fill_zero_kernel, dim3(static_cast<unsigned>(blocks)), dim3(256), 0, stream, C, n);
}

int launch_transposed_b(const float* A, const float* B, float* C, int M, int N, int K, hipStream_t stream) {
    if (M == 1 && gemv_supported(kFmtF32, K, B)) return launch_gemv(kFmtF32, A, B, C, N, K, stream);
    return launch_generic_matmul(kFmtF32, A, B, C, M, N, K, stream);
}

int launch_gqa(const float* A, const float* B, float* C, int n_heads, int n_kv_heads, int M, int N, int K,
               hipStream_t stream) {
    const int G = n_heads / n_kv_heads;
    const int R = G * M;
    const int n_tiles = (N + dev::kQTN - 1) / dev::kQTN;
    const int r_tiles = (R + dev::kQTR - 1) / dev::kQTR;
    const long base = static_cast<long>(n_tiles) * r_tiles * n_kv_heads;
    int splits = 1;
    const int k_stages = (K + dev::kQTK - 1) / dev::kQTK;
    while (base * splits < 512 && splits * 2 <= k_stages) splits *= 2;
    const int k_split = ((k_stages + splits - 1) / splits) * dev::kQTK;
    splits = (K + k_split - 1) / k_split;
    const int atomic = splits > 1;
    if (atomic) launch_fill_zero(C, static_cast<long>(n_heads) * M * N, stream);
    const dim3 grid(n_tiles, r_tiles, n_kv_heads * splits);
    hipLaunchKernelGGL(dev::gqa_kernel, grid, dim3(256), 0, stream, A, B, C, G, M, N, K, k_split, splits, atomic);
    return 0;
}

}  // namespace detail
}  // namespace cri
