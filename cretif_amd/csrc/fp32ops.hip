// fp32ops.hip -- the two fp32 neighbours of the fused path.
//
// matmul_transposed_b: C = A * B^T with B [N,K] fp32 (the tied LM head,
//   ref:src/embedding.cu:85-135).  M == 1 runs the streaming GEMV (one pass over
//   B with coalesced 16-byte loads, activations in VGPRs); 2 <= M <= 16 (a
//   decode batch) streams B once through v_mfma_f32_16x16x4_f32, fp32 products
//   summed in fp32, with the M activation rows staged in LDS (below); other
//   shapes use the LDS-tiled fallback.
// batched_matmul_gqa: C[h] = A[h] * B[h / G] with A [H,M,K], B [Hkv,K,N]
//   (ref:src/attention.cu:192-218).  The G query heads sharing a KV head are
//   served together, so each B element is read once per row tile of its KV
//   group (the repeats hit the caches):
//   a block owns 64 columns (one per lane) x RT (4 or 8) (head, m) rows of one KV
//   group; its four waves take interleaved 16-column k slices of each 64-k
//   stage (row values broadcast from LDS, B read once, coalesced along n) and
//   add their partial sums through LDS in a fixed order.  Short K (QK^T over
//   head_dim) has enough (column tile, row tile, KV head) blocks and stores
//   plainly (deterministic); long K (PV over the cache length) is also split
//   over blocks until ~8 blocks per CU run, and those partial tiles are added
//   with fp32 atomics into a zero-filled C.
#include <atomic>

#include "common.hpp"
#include "internal.hpp"

namespace cri {
namespace dev {

// p[0 .. n) = 0: 16-byte stores over the 16-byte aligned body, single floats at the ends
__global__ __launch_bounds__(256) void fill_zero_kernel(float* __restrict__ p, long n) {
    const long i = static_cast<long>(blockIdx.x) * blockDim.x + threadIdx.x;
    const long stride = static_cast<long>(gridDim.x) * blockDim.x;
    const long head = static_cast<long>((16 - (reinterpret_cast<uintptr_t>(p) & 15)) & 15) / 4;  // p is 4-aligned
    const long lead = head < n ? head : n;
    const long nv = (n - lead) / 4;
    f32x4* body = reinterpret_cast<f32x4*>(p + lead);
    for (long j = i; j < nv; j += stride) body[j] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    if (i < lead) p[i] = 0.0f;
    const long tail = lead + 4 * nv;
    if (tail + i < n) p[tail + i] = 0.0f;
}

// ---- GQA kernel -----------------------------------------------------------------
// RT rows per block: 4 when a KV group has at most 4 (head, m) rows (one query
// token), else 8.  Fewer rows per block mean more blocks in flight, which these
// latency-bound products need (T = 2048, 32/8 heads: Q K^T 4.7 -> 3.4 us at M = 1,
// 8.8 -> 7.4 at M = 16 against 16 rows; 32 rows was slower still).
constexpr int kGsKC = 16;  // k per wave per LDS stage (a stage is 4 waves x 16 k)

template <int RT>
__global__ __launch_bounds__(256) void gqa_split_kernel(const float* __restrict__ A, const float* __restrict__ B,
                                                        float* __restrict__ C, int G, int M, int N, int K,
                                                        int k_split, int atomic) {
    __shared__ float qs[RT][4 * kGsKC + 4];
    __shared__ float red[3][RT][64];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int n = blockIdx.x * 64 + lane;
    const int kv = blockIdx.y;
    const int rt = blockIdx.z % ((G * M + RT - 1) / RT);
    const int split = blockIdx.z / ((G * M + RT - 1) / RT);
    const int r0 = rt * RT;
    const int R = G * M;
    const int kb = split * k_split, ke = min(K, kb + k_split);
    const float* Bk = B + static_cast<long>(kv) * K * N + min(n, N - 1);
    float acc[RT];
#pragma unroll
    for (int r = 0; r < RT; ++r) acc[r] = 0.0f;
    // each stage: 4 waves x kGsKC k; wave w takes k [k0 + w * kGsKC, +kGsKC).  The
    // wave's B loads are issued before the row values are staged, so the two
    // latencies overlap.
    for (int k0 = kb; k0 < ke; k0 += 4 * kGsKC) {
        const int kw = k0 + wave * kGsKC;
        float b[kGsKC];
#pragma unroll
        for (int kk = 0; kk < kGsKC; ++kk) b[kk] = kw + kk < ke ? Bk[static_cast<long>(kw + kk) * N] : 0.0f;
        for (int e = tid; e < RT * 4 * kGsKC; e += 256) {
            const int rr = e / (4 * kGsKC), kk = e - rr * (4 * kGsKC), r = r0 + rr, k = k0 + kk;
            float v = 0.0f;
            if (r < R && k < ke) {
                const int head = kv * G + r / M, m = r - (r / M) * M;
                v = A[(static_cast<long>(head) * M + m) * K + k];
            }
            qs[rr][kk] = v;
        }
        __syncthreads();
#pragma unroll
        for (int kk = 0; kk < kGsKC; kk += 4)
#pragma unroll
            for (int r = 0; r < RT; ++r) {
                const f32x4 q = *reinterpret_cast<const f32x4*>(&qs[r][wave * kGsKC + kk]);
                acc[r] = __builtin_fmaf(q.x, b[kk], acc[r]);
                acc[r] = __builtin_fmaf(q.y, b[kk + 1], acc[r]);
                acc[r] = __builtin_fmaf(q.z, b[kk + 2], acc[r]);
                acc[r] = __builtin_fmaf(q.w, b[kk + 3], acc[r]);
            }
        __syncthreads();
    }
    // add the four waves' partial sums (fixed order)
    if (wave > 0)
#pragma unroll
        for (int r = 0; r < RT; ++r) red[wave - 1][r][lane] = acc[r];
    __syncthreads();
    if (wave != 0 || n >= N) return;
#pragma unroll
    for (int rr = 0; rr < RT; ++rr) {
        const int r = r0 + rr;
        if (r >= R) break;
        const float v = ((acc[rr] + red[0][rr][lane]) + red[1][rr][lane]) + red[2][rr][lane];
        const int head = kv * G + r / M, m = r - (r / M) * M;
        float* dst = C + (static_cast<long>(head) * M + m) * N + n;
        if (atomic) atomicAdd(dst, v);
        else *dst = v;
    }
}


// ---- batched_matmul_gqa at prefill M: fp32 matrix cores ----
// The G query heads of one KV head are consecutive in A and C, so per KV head
// the product is one GEMM C_kv [R = G M, N] = A_kv [R, K] * B_kv [K, N].  A
// workgroup owns a 64 x 64 tile of it, its four waves one 32 x 32
// v_mfma_f32_32x32x2_f32 tile each (fp32 products summed in fp32).  Each k
// stage (KS columns) of A (rows) and B (stored transposed, [n][k]) goes
// through double-buffered LDS, so each lane's KS / 2 k values of a stage are
// 16-byte reads; lane (i, h) feeds k = (KS / 2) h + j to the j-th MFMA of the
// stage in both operands (a k order of its own, the same products and sums).
// The global loads run D stages ahead of the stage being computed (D register
// sets): short K (Q K^T over head_dim) takes 16-column stages two deep, long K
// (P V over the keys) 32-column stages four deep, where one workgroup per CU
// has to keep enough requests in flight.
// Requires K, N >= 4, K % 4 == 0, N % 4 == 0 and 16-byte aligned A, B; every
// load address is clamped into its row, k past K stages zero activations, rows
// past R and columns past N are computed from clamped values and not stored.
typedef float gm_f16v __attribute__((ext_vector_type(16)));
constexpr int kGmT = 64;

// KS: k per stage (16 or 32); D: stages of loads in flight (2 or 4 register sets)
template <int KS, int D>
__global__ __launch_bounds__(256) void gqa_mfma_kernel(const float* __restrict__ A, const float* __restrict__ B,
                                                       float* __restrict__ C, int R, int N, int K) {
    constexpr int LD = KS + 4;   // LDS row stride (floats): 16-byte reads of 16 rows fall in distinct bank groups
    constexpr int AP = KS / 16;  // staged pieces per thread and operand
    __shared__ __attribute__((aligned(16))) float sa[2][kGmT * LD];
    __shared__ __attribute__((aligned(16))) float sb[2][kGmT * LD];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int kv = blockIdx.y;
    const int r0 = blockIdx.z * kGmT, n0 = blockIdx.x * kGmT;
    const float* Akv = A + static_cast<long>(kv) * R * K;
    const float* Bkv = B + static_cast<long>(kv) * K * N;
    float* Ckv = C + static_cast<long>(kv) * R * N;

    // staging, AP pieces per thread and operand: A rows ai + (256 / (KS / 4)) p, columns
    // 4 aq .. + 3 of the stage; B rows (k) bk + 16 p, columns 4 bc .. + 3
    constexpr int APR = KS / 4;            // 16-byte pieces per staged A row
    constexpr int AROWS = 256 / APR;       // A rows per pass of the 256 threads
    const int ai = tid / APR, aq = tid % APR, bk = tid >> 4, bc = tid & 15;
    const float* arow[AP];
#pragma unroll
    for (int p = 0; p < AP; ++p) arow[p] = Akv + static_cast<long>(min(r0 + ai + AROWS * p, R - 1)) * K;
    const float* bcol = Bkv + min(n0 + 4 * bc, N - 4);
    const int nsteps = (K + KS - 1) / KS;
    struct Regs {
        f32x4 a[AP], b[AP];
    };
    // every load is unconditional (a clamped in-bounds address; values past K are zeroed
    // after the load), so the compiler knows how many are in flight
    auto gload = [&](Regs& g, int s) {
        const int k0 = s * KS;
        const bool in = k0 + 4 * aq < K;
        const int ka = min(k0 + 4 * aq, K - 4);  // within the row (K >= 4); = k0 + 4 aq whenever in
        const f32x4 z = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int p = 0; p < AP; ++p) {
            const f32x4 v = ld_f32x4(arow[p] + ka);
            g.a[p] = in ? v : z;
            g.b[p] = ld_f32x4(bcol + static_cast<long>(min(k0 + bk + 16 * p, K - 1)) * N);
        }
    };
    auto swrite = [&](const Regs& g, int buf) {
#pragma unroll
        for (int p = 0; p < AP; ++p) {
            *reinterpret_cast<f32x4*>(&sa[buf][(ai + AROWS * p) * LD + 4 * aq]) = g.a[p];
            float* t = &sb[buf][(4 * bc) * LD + bk + 16 * p];
            t[0] = g.b[p].x;
            t[LD] = g.b[p].y;
            t[2 * LD] = g.b[p].z;
            t[3 * LD] = g.b[p].w;
        }
    };
    const int wr = wave >> 1, wc = wave & 1, i = lane & 31, h = lane >> 5;
    constexpr int KH = KS / 2;  // k per half-wave per stage
    const int aoff = (32 * wr + i) * LD + KH * h, boff = (32 * wc + i) * LD + KH * h;
    gm_f16v acc;
#pragma unroll
    for (int v = 0; v < 16; ++v) acc[v] = 0.0f;
    auto compute = [&](int buf) {
#pragma unroll
        for (int c = 0; c < KH / 4; ++c) {
            const f32x4 a = *reinterpret_cast<const f32x4*>(&sa[buf][aoff + 4 * c]);
            const f32x4 b = *reinterpret_cast<const f32x4*>(&sb[buf][boff + 4 * c]);
            acc = __builtin_amdgcn_mfma_f32_32x32x2f32(a.x, b.x, acc, 0, 0, 0);
            acc = __builtin_amdgcn_mfma_f32_32x32x2f32(a.y, b.y, acc, 0, 0, 0);
            acc = __builtin_amdgcn_mfma_f32_32x32x2f32(a.z, b.z, acc, 0, 0, 0);
            acc = __builtin_amdgcn_mfma_f32_32x32x2f32(a.w, b.w, acc, 0, 0, 0);
        }
    };

    // Iteration s: stage s is in LDS buffer s & 1, stages s + 1 .. s + D - 1 are in the
    // register sets other than set s % D, which receives stage s + D's loads; it computes
    // stage s, writes stage s + 1 to the other buffer and syncs once.  The stage count is
    // padded to a multiple of D with stages past K, which hold zero activations.
    const int nstepsD = (nsteps + D - 1) / D * D;
    Regs g[D];
#pragma unroll
    for (int d = 0; d < D; ++d) gload(g[d], d);
    swrite(g[0], 0);
    __syncthreads();
    for (int s = 0; s < nstepsD; s += D) {
#pragma unroll
        for (int d = 0; d < D; ++d) {
            gload(g[d], s + d + D);
            __builtin_amdgcn_sched_barrier(0);  // the loads go out before this stage's work
            compute((s + d) & 1);
            swrite(g[(d + 1) % D], (s + d + 1) & 1);
            __syncthreads();
        }
    }

    // lane (i, h), accumulator v: row 32 wr + 8 (v >> 2) + 4 h + (v & 3), column 32 wc + i
    const int n = n0 + 32 * wc + i;
    if (n >= N) return;
#pragma unroll
    for (int v = 0; v < 16; ++v) {
        const int r = r0 + 32 * wr + 8 * (v >> 2) + 4 * h + (v & 3);
        if (r < R) Ckv[static_cast<long>(r) * N + n] = acc[v];
    }
}

// ---- A * B^T for 2 <= M <= 16: one pass over B on the fp32 matrix cores ----
// A wave owns 16 rows of B (one 16 x 16 output tile: B rows x activation rows,
// the activation rows past M are zeros) and walks K in groups of 16 columns:
// lane (i, q) = (lane & 15, lane >> 4) loads B[n0 + i][k + 4q .. + 3] (16 bytes;
// the 64 lanes cover 16 rows x 64 contiguous bytes) and reads A[i][k + 4q .. + 3]
// from LDS, and element j of both feeds the j-th of four MFMAs -- the k order
// inside a group differs from k order, the products and their fp32 sums are
// the reference's.  Weight loads run eight groups ahead (two register sets).
// The activation rows are staged per chunk of up to kTbChunk columns; with more
// than one chunk (K > kTbChunk) every row task restages them.
constexpr int kTbChunk = 2048;
constexpr int kTbLd = kTbChunk + 4;  // LDS row stride (floats): the 16 rows' chunks fall in distinct bank groups
constexpr int kTbThreads = 512;
constexpr int kTbBatch = 8;          // 16-column groups per batch of weight loads
constexpr int kTbLdsBytes = 16 * kTbLd * 4;

__global__ __launch_bounds__(kTbThreads) void tb_stream_kernel(const float* __restrict__ A, const float* __restrict__ B,
                                                               float* __restrict__ C, int M, int N, int K,
                                                               int tasks_per_wave) {
    extern __shared__ __attribute__((aligned(16))) float xs[];  // 16 rows x kTbLd
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int li = lane & 15, q = lane >> 4;
    const long nwaves = static_cast<long>(gridDim.x) * (kTbThreads / 64);
    const long ngroups = (static_cast<long>(N) + 15) / 16;
    const int nchunks = (K + kTbChunk - 1) / kTbChunk;
    const float* xrow = xs + li * kTbLd + 4 * q;

    for (int t = 0; t < tasks_per_wave; ++t) {
        const long g = static_cast<long>(blockIdx.x) * (kTbThreads / 64) + wave + t * nwaves;
        const long n0 = (g < ngroups ? g : ngroups - 1) * 16;  // idle waves repeat the last group (no store)
        const float* wrow = B + min(n0 + li, static_cast<long>(N) - 1) * K + 4 * q;
        f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
        for (int c = 0; c < nchunks; ++c) {
            const int k0 = c * kTbChunk, kc = min(kTbChunk, K - k0);
            if (nchunks > 1 || t == 0) {  // uniform over the workgroup
                __syncthreads();
                const int per = kc >> 2;  // 16-byte pieces per row
                for (int e = tid; e < 16 * per; e += kTbThreads) {
                    const int m = e / per, j = e - m * per;
                    const f32x4 v = m < M ? ld_f32x4(A + static_cast<long>(m) * K + k0 + 4 * j)
                                          : f32x4{0.0f, 0.0f, 0.0f, 0.0f};
                    *reinterpret_cast<f32x4*>(xs + m * kTbLd + 4 * j) = v;
                }
                __syncthreads();
            }
            const int ng = kc >> 4;  // 16-column groups in this chunk
            const float* wp = wrow + k0;
            auto load = [&](f32x4 (&w)[kTbBatch], int s0) {
#pragma unroll
                for (int u = 0; u < kTbBatch; ++u) w[u] = ld_f32x4(wp + 16 * min(s0 + u, ng - 1));  // in bounds
            };
            auto mma = [&](const f32x4 (&w)[kTbBatch], int s0) {
#pragma unroll
                for (int u = 0; u < kTbBatch; ++u) {
                    if (s0 + u >= ng) break;  // uniform
                    const f32x4 x = *reinterpret_cast<const f32x4*>(xrow + 16 * (s0 + u));
                    acc = __builtin_amdgcn_mfma_f32_16x16x4f32(w[u].x, x.x, acc, 0, 0, 0);
                    acc = __builtin_amdgcn_mfma_f32_16x16x4f32(w[u].y, x.y, acc, 0, 0, 0);
                    acc = __builtin_amdgcn_mfma_f32_16x16x4f32(w[u].z, x.z, acc, 0, 0, 0);
                    acc = __builtin_amdgcn_mfma_f32_16x16x4f32(w[u].w, x.w, acc, 0, 0, 0);
                }
            };
            f32x4 wa[kTbBatch], wb[kTbBatch];
            load(wa, 0);
            for (int s0 = 0; s0 < ng; s0 += 2 * kTbBatch) {
                load(wb, s0 + kTbBatch);
                mma(wa, s0);
                load(wa, s0 + 2 * kTbBatch);
                mma(wb, s0 + kTbBatch);
            }
        }
        // lane (i, q): C[m = i][n0 + 4q + r], r = 0..3
        if (g < ngroups && li < M) {
            const long n = n0 + 4 * q;
            float* cp = C + static_cast<long>(li) * N + n;
            if (n + 0 < N) cp[0] = acc.x;
            if (n + 1 < N) cp[1] = acc.y;
            if (n + 2 < N) cp[2] = acc.z;
            if (n + 3 < N) cp[3] = acc.w;
        }
    }
}

}  // namespace dev

namespace detail {

void launch_fill_zero(float* C, long n, hipStream_t stream) {
    if (n <= 0) return;
    const long vec = (n + 3) / 4;  // one 16-byte store per thread and pass
    const long blocks = (vec + 255) / 256 < 2048 ? (vec + 255) / 256 : 2048;
    hipLaunchKernelGGL(dev::fill_zero_kernel, dim3(static_cast<unsigned>(blocks)), dim3(256), 0, stream, C, n);
}

// the streaming kernel uses more than the default 64 KB of LDS: the limit is raised once per device
static int launch_tb_stream(const float* A, const float* B, float* C, int M, int N, int K, hipStream_t stream) {
    constexpr int kMaxDevices = 64;
    static std::atomic<bool> ready[kMaxDevices];
    int devid = 0;
    if (hipGetDevice(&devid) != hipSuccess || devid < 0 || devid >= kMaxDevices) return kFailed;
    if (!ready[devid].load(std::memory_order_acquire)) {
        if (hipFuncSetAttribute(reinterpret_cast<const void*>(&dev::tb_stream_kernel),
                                hipFuncAttributeMaxDynamicSharedMemorySize, dev::kTbLdsBytes) != hipSuccess)
            return kFailed;
        ready[devid].store(true, std::memory_order_release);
    }
    const long groups = (static_cast<long>(N) + 15) / 16;
    constexpr int kWavesPerBlock = dev::kTbThreads / 64;
    long blocks = (groups + kWavesPerBlock - 1) / kWavesPerBlock;
    if (blocks > 256) blocks = 256;  // one workgroup per CU (the staged rows fill most of its LDS)
    const long waves = blocks * kWavesPerBlock;
    const int tasks = static_cast<int>((groups + waves - 1) / waves);
    hipLaunchKernelGGL(dev::tb_stream_kernel, dim3(static_cast<unsigned>(blocks)), dim3(dev::kTbThreads),
                       dev::kTbLdsBytes, stream, A, B, C, M, N, K, tasks);
    return 0;
}

int launch_transposed_b(const float* A, const float* B, float* C, int M, int N, int K, hipStream_t stream) {
    if (M == 1 && gemv_supported(kFmtF32, K, B)) return launch_gemv(kFmtF32, A, B, C, N, K, stream);
    const bool aligned = ((reinterpret_cast<uintptr_t>(A) | reinterpret_cast<uintptr_t>(B)) & 15) == 0;
    if (M >= 2 && M <= 16 && K % 16 == 0 && aligned) return launch_tb_stream(A, B, C, M, N, K, stream);
    return launch_generic_matmul(kFmtF32, A, B, C, M, N, K, stream);
}

int launch_gqa(const float* A, const float* B, float* C, int n_heads, int n_kv_heads, int M, int N, int K,
               hipStream_t stream) {
    const int G = n_heads / n_kv_heads;
    const long R = static_cast<long>(G) * M;
    // prefill (many rows per KV head): the matrix-core tiles
    const bool aligned = ((reinterpret_cast<uintptr_t>(A) | reinterpret_cast<uintptr_t>(B)) & 15) == 0;
    if (M >= 32 && K >= 4 && N >= 4 && K % 4 == 0 && N % 4 == 0 && aligned && (R + 63) / 64 <= 65535) {
        const dim3 grid((N + 63) / 64, n_kv_heads, static_cast<unsigned>((R + 63) / 64));
        if (K <= 128)
            hipLaunchKernelGGL((dev::gqa_mfma_kernel<16, 2>), grid, dim3(256), 0, stream, A, B, C,
                               static_cast<int>(R), N, K);
        else
            hipLaunchKernelGGL((dev::gqa_mfma_kernel<32, 4>), grid, dim3(256), 0, stream, A, B, C,
                               static_cast<int>(R), N, K);
        return 0;
    }
    // split K over blocks while (column tiles x row tiles x KV heads) gives fewer than ~8
    // blocks per CU: a block's stages run one after another, so several resident blocks
    // per CU hide each other's load latency (P V at M = 16 with 16-row blocks: 21.2 us
    // with ~1 block per CU, 14.2 with 2, 12.5 with 4, despite 4x the atomic adds; with
    // 8-row blocks 10.6 us at 4 and 10.2 at 8)
    const int RT = R <= 4 ? 4 : 8;
    const long rtiles = (R + RT - 1) / RT;
    const long base = static_cast<long>((N + 63) / 64) * rtiles * n_kv_heads;
    const int stage = 4 * dev::kGsKC;
    const int stages = (K + stage - 1) / stage;
    int splits = 1;
    while (base * splits < 2048 && splits * 2 <= stages) splits *= 2;
    const int k_split = ((stages + splits - 1) / splits) * stage;
    splits = (K + k_split - 1) / k_split;
    if (rtiles * splits > 65535) return -1;
    const int atomic = splits > 1;
    if (atomic) launch_fill_zero(C, static_cast<long>(n_heads) * M * N, stream);
    const dim3 grid((N + 63) / 64, n_kv_heads, static_cast<unsigned>(rtiles * splits));
    if (RT == 4)
        hipLaunchKernelGGL(dev::gqa_split_kernel<4>, grid, dim3(256), 0, stream, A, B, C, G, M, N, K, k_split, atomic);
    else
        hipLaunchKernelGGL(dev::gqa_split_kernel<8>, grid, dim3(256), 0, stream, A, B, C, G, M, N, K, k_split, atomic);
    return 0;
}

}  // namespace detail
}  // namespace cri
