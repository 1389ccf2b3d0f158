// attention.hip -- fused decode attention: one query token, grouped-query heads,
// over the fp32 KV cache in its [kv_len, n_kv_heads, head_dim] layout
// (ref:src/attention.cu:410-511 computes the same softmax(q K^T * scale) V with
// one block per query head walking the positions one at a time).
//
// The call has no workspace (the reference's signature), so partial softmax
// states cannot be merged across workgroups: a workgroup owns complete outputs.
// It is one query head h and a slice of 8 output dims, and walks every
// position of its KV head.  Launch shape for Llama-3.2-1B (32 heads, 8 KV heads,
// head_dim 64): 8 slices of 8 dims -> 256 workgroups, and the 32 workgroups of
// one KV head are mapped onto one XCD, so that head's K/V (1 MB at 2048
// positions) comes from HBM once and the repeats hit that XCD's L2.
//
// Per wave and tile of 64 positions:
//   * scores: 4 lanes per position, each lane holding 4-float slices of the
//     query (dims 4r + 16i) and loading the same slices of the K row (16-byte
//     loads, 64 contiguous bytes per lane quad); a 2-step quad reduction gives
//     the dot products of 16 positions per load round, 4 rounds per tile; lane
//     (quad q, r) keeps position 16 r + q, so the tile's 64 scores sit one per lane;
//   * online softmax in base 2 (the query is pre-scaled by scale * log2 e): the
//     tile max is a wave reduction, the rescale factor is wave-uniform and each
//     lane updates its own running sum and its 8 accumulators with the V
//     values of its own position;
// and at the end the wave's lanes, then the workgroup's waves, are merged
// (max, rescale, sum) in a fixed order.
#include <atomic>

#include "common.hpp"
#include "internal.hpp"

// Partial softmax records of cri_fused_decode_attention_noalloc: one array per
// GPU, held until the process ends.  Host code never uses this name as an
// address (in host code it is a stand-in, not device memory): the device
// address comes from hipGetSymbolAddress, once per device (noalloc_scratch).
static __device__ __align__(256) float scratch[cri::detail::kNoallocScratchBytes / sizeof(float)];

namespace cri {
namespace dev {

constexpr int kAttWaves = 8;   // waves per workgroup; wave w takes tiles w, w + 8, ...
constexpr int kAttTile = 64;   // positions per wave tile
constexpr int kAttDs = 8;      // output dims per workgroup (one slice)

// NQ: 4-float query slices per lane (head_dim <= 16 NQ).  VEC: head_dim % 4 == 0
// and 16-byte aligned Q / K / V, so the slices load as 16-byte vectors.  One
// workgroup per CU gives two waves per SIMD: registers go to loads in flight,
// not to occupancy.
template <int NQ, bool VEC>
__global__ __launch_bounds__(64 * kAttWaves) __attribute__((amdgpu_waves_per_eu(1, 2))) void decode_attn_kernel(
    const float* __restrict__ Q, const float* __restrict__ Kc, const float* __restrict__ Vc, float* __restrict__ out,
    int G, int kvd, int D, int T, float qscale, int n_slices, int remap) {
    constexpr int DS = kAttDs;
    // position groups (16 positions each) whose K slices are loaded as one batch
    constexpr int GB = NQ <= 4 ? 4 : (NQ == 8 ? 2 : 1);
    // query slices per batch (scalar loads of head_dim > 128 in two halves)
    constexpr int IB = (!VEC && NQ == 16) ? 8 : NQ;
    __shared__ float red[kAttWaves][2 + DS];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    int L = blockIdx.x;
    if (remap) {  // gridDim.x % 8 == 0: logical index L runs on XCD L / (gridDim.x / 8)
        const int per = gridDim.x >> 3;
        L = (blockIdx.x & 7) * per + (blockIdx.x >> 3);
    }
    const int h = L / n_slices, sl = L - h * n_slices;
    const int kvh = h / G;
    const int d0 = sl * DS;
    const int q4 = lane >> 2, r = lane & 3;
    const float* Kh = Kc + static_cast<long>(kvh) * D;
    const float* Vh = Vc + static_cast<long>(kvh) * D;

    // Every load is unconditional, from an address clamped into the row (a
    // guarded load becomes a branch with its own wait); values past head_dim
    // are zeroed by a select or meet a zero query value.
    f32x4 qv[NQ];
#pragma unroll
    for (int i = 0; i < NQ; ++i) {
        const int d = 4 * r + 16 * i;
        if constexpr (VEC) {
            const f32x4 v = ld_f32x4(Q + static_cast<long>(h) * D + min(d, D - 4)) * qscale;
            qv[i] = d < D ? v : f32x4{0.f, 0.f, 0.f, 0.f};
        } else {
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const float v = Q[static_cast<long>(h) * D + min(d + e, D - 1)] * qscale;
                qv[i][e] = d + e < D ? v : 0.0f;
            }
        }
    }

    float m = -INFINITY, l = 0.0f;
    float acc[DS];
#pragma unroll
    for (int e = 0; e < DS; ++e) acc[e] = 0.0f;
    const int ntiles = (T + kAttTile - 1) / kAttTile;

    // V slice of the lane's own position (its address does not depend on the scores)
    auto load_v = [&](float (&vv)[DS], int base) {
        const float* vp = Vh + static_cast<long>(min(base + 16 * r + q4, T - 1)) * kvd;
        if constexpr (VEC) {
#pragma unroll
            for (int e = 0; e < DS; e += 4) {
                const f32x4 v = ld_f32x4(vp + min(d0 + e, D - 4));  // 4 | D and 4 | d0
                vv[e] = v.x; vv[e + 1] = v.y; vv[e + 2] = v.z; vv[e + 3] = v.w;
            }
        } else {
#pragma unroll
            for (int e = 0; e < DS; ++e) vv[e] = vp[min(d0 + e, D - 1)];
        }
    };
    // K slices (query slices i0 .. i0+IB) of position group g of a tile
    auto load_k = [&](f32x4 (&kv)[IB], int base, int g, int i0) {
        const float* kp = Kh + static_cast<long>(min(base + 16 * g + q4, T - 1)) * kvd;
#pragma unroll
        for (int i = 0; i < IB; ++i) {
            const int d = 4 * r + 16 * (i0 + i);
            if constexpr (VEC) {
                kv[i] = ld_f32x4(kp + min(d, D - 4));
            } else {
#pragma unroll
                for (int e = 0; e < 4; ++e) kv[i][e] = kp[min(d + e, D - 1)];
            }
        }
    };
    auto dot = [&](float part, const f32x4 (&kv)[IB], int i0) {
#pragma unroll
        for (int i = 0; i < IB; ++i) {
            part = __builtin_fmaf(qv[i0 + i].x, kv[i].x, part);
            part = __builtin_fmaf(qv[i0 + i].y, kv[i].y, part);
            part = __builtin_fmaf(qv[i0 + i].z, kv[i].z, part);
            part = __builtin_fmaf(qv[i0 + i].w, kv[i].w, part);
        }
        return part;
    };
    // lane (quad q, r) keeps the score of position 16 r + q of the tile
    auto own_score = [&](float& s_own, float part, int base, int g, int limit) {
        part += dpp<kQuadPerm1032>(part);
        part += dpp<kQuadPerm2301>(part);
        const int pos = base + 16 * g + q4;
        if (g == r) s_own = pos < limit ? part : -INFINITY;
    };
    // online-softmax update with the tile's scores and the V slices of the lanes' positions
    auto update = [&](float s_own, const float (&vraw)[DS]) {
        // every processed tile has a valid position, so tmax and m_new are finite
        const float tmax = wave_max(s_own);
        const float m_new = fmaxf(m, tmax);
        const float c = exp2f(m - m_new);  // 0 on the wave's first tile
        const float p = exp2f(s_own - m_new);
        l = __builtin_fmaf(l, c, p);
#pragma unroll
        for (int e = 0; e < DS; ++e) {
            const float v = d0 + e < D ? vraw[e] : 0.0f;
            acc[e] = __builtin_fmaf(p, v, acc[e] * c);
        }
        m = m_new;
    };

    if constexpr (NQ <= 4) {
        // one tile at a time: its 18 loads (2 V + 16 K) are issued as one batch
        // (a software pipeline over two tiles measured slower: the bound is the
        // CU's vector-memory throughput, and the clamped prefetch past the end
        // adds instructions)
        for (int tile = wave; tile < ntiles; tile += kAttWaves) {
            const int base = tile * kAttTile;
            float vv[DS];
            load_v(vv, base);
            f32x4 kv[4][IB];
#pragma unroll
            for (int g = 0; g < 4; ++g) load_k(kv[g], base, g, 0);
            __builtin_amdgcn_sched_barrier(0);  // the batch above stays in flight together
            float s_own = -INFINITY;
#pragma unroll
            for (int g = 0; g < 4; ++g) own_score(s_own, dot(0.0f, kv[g], 0), base, g, T);
            update(s_own, vv);
        }
    } else {
        // head_dim > 64: one tile at a time, K in batches of GB position groups
        for (int tile = wave; tile < ntiles; tile += kAttWaves) {
            const int base = tile * kAttTile;
            float vv[DS];
            load_v(vv, base);
            float s_own = -INFINITY;
#pragma unroll
            for (int g0 = 0; g0 < 4; g0 += GB) {
                float part[GB];
#pragma unroll
                for (int gb = 0; gb < GB; ++gb) part[gb] = 0.0f;
#pragma unroll
                for (int i0 = 0; i0 < NQ; i0 += IB) {
                    f32x4 kv[GB][IB];
#pragma unroll
                    for (int gb = 0; gb < GB; ++gb) load_k(kv[gb], base, g0 + gb, i0);
                    __builtin_amdgcn_sched_barrier(0);  // the batch above stays in flight together
#pragma unroll
                    for (int gb = 0; gb < GB; ++gb) part[gb] = dot(part[gb], kv[gb], i0);
                }
#pragma unroll
                for (int gb = 0; gb < GB; ++gb) own_score(s_own, part[gb], base, g0 + gb, T);
            }
            update(s_own, vv);
        }
    }

    // merge: lanes of the wave (same m), then the waves (rescaled to the common max)
    l = group_sum_t<6>(l);
#pragma unroll
    for (int e = 0; e < DS; ++e) acc[e] = group_sum_t<6>(acc[e]);
    if (lane == 0) {
        red[wave][0] = m;
        red[wave][1] = l;
#pragma unroll
        for (int e = 0; e < DS; ++e) red[wave][2 + e] = acc[e];
    }
    __syncthreads();
    const int e = threadIdx.x;
    if (e < DS && d0 + e < D) {
        float M = -INFINITY;
#pragma unroll
        for (int w = 0; w < kAttWaves; ++w) M = fmaxf(M, red[w][0]);
        float num = 0.0f, den = 0.0f;
#pragma unroll
        for (int w = 0; w < kAttWaves; ++w) {
            const float f = exp2f(red[w][0] - M);  // 0 for a wave without tiles (m = -inf)
            num = __builtin_fmaf(f, red[w][2 + e], num);
            den = __builtin_fmaf(f, red[w][1], den);
        }
        out[static_cast<long>(h) * D + d0 + e] = num / den;
    }
}

// ---- split form (caller workspace) ---------------------------------------------
//
// A workgroup is KV head kvh, a quad of its query heads (one wave per head;
// measured faster than two or four heads per wave, whose longer per-wave VALU
// chains dominate a one-tile chunk), a chunk of the positions in tiles of 32,
// and one query row m (blockIdx.y).  The waves read each tile's K and V rows 4
// lanes per position (dims 4 r + 16 i, 16-byte loads); the four waves of a quad
// hit the same lines, so the cache is read from memory once per query row (the
// rows of one call re-read it from the caches).  Per head: the scores of the
// tile's 32 positions end on lanes r = 0, 1 (position 16 r + q), online softmax
// as above, and P.V in the same lane layout as the loads (the weight of position
// 16 g + q is broadcast from lane (q, g) inside its quad).  The chunk's (max,
// sum, acc[D]) per (row, head) go to the workspace, and the combine kernel
// merges the chunks of each (row, head).
//
// Query row m sees the first kv0 + m positions, plus *kv_dev when kv_dev is
// not null (causal: the rows are consecutive tokens whose keys are already in
// the cache; a position counter read from device memory keeps a captured graph
// of the call valid as the sequence grows).  The
// positions of a row are cut into nchunks chunks of whole tiles, the chunk
// length computed from the row's length (a chunk past the end writes an empty
// record: max -inf, sum 0).  head_dim <= 16 NQ, a multiple of 4, and 16-byte
// aligned Q, K, V.
constexpr int kSplitTile = 32;

template <int HQ, int NQ>
__global__ __launch_bounds__(256 / HQ) void decode_attn_split_kernel(const float* __restrict__ Q,
                                                                     const float* __restrict__ Kc,
                                                                     const float* __restrict__ Vc,
                                                                     float* __restrict__ ws, int G, int kvd, int D,
                                                                     const int* __restrict__ kv_dev, int kv0,
                                                                     float qscale, int nchunks, int nhq, long ldq) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int c = blockIdx.x % nchunks;
    const int hq = (blockIdx.x / nchunks) % nhq;
    const int kvh = blockIdx.x / (nchunks * nhq);
    const int mrow = blockIdx.y;
    const int H = G * (gridDim.x / (nchunks * nhq));
    const int T = (kv_dev ? *kv_dev : 0) + kv0 + mrow;  // positions this row attends to
    const int Tc = kSplitTile * ((((T + kSplitTile - 1) / kSplitTile) + nchunks - 1) / nchunks);
    const int q4 = lane >> 2, r = lane & 3;
    const int t0 = c * Tc, t1 = min(T, t0 + Tc);
    const float* Kh = Kc + static_cast<long>(kvh) * D;
    const float* Vh = Vc + static_cast<long>(kvh) * D;
    const float* Qm = Q + mrow * ldq;

    f32x4 qv[HQ][NQ];
#pragma unroll
    for (int j = 0; j < HQ; ++j) {
        const int hg = hq * 4 + wave * HQ + j;  // head index inside the KV group
        const int h = kvh * G + min(hg, G - 1);
#pragma unroll
        for (int i = 0; i < NQ; ++i) {
            const int d = 4 * r + 16 * i;
            const f32x4 v = ld_f32x4(Qm + static_cast<long>(h) * D + min(d, D - 4)) * qscale;
            qv[j][i] = d < D && hg < G ? v : f32x4{0.f, 0.f, 0.f, 0.f};
        }
    }
    float m[HQ], l[HQ];
    f32x4 acc[HQ][NQ];
#pragma unroll
    for (int j = 0; j < HQ; ++j) {
        m[j] = -INFINITY;
        l[j] = 0.0f;
#pragma unroll
        for (int i = 0; i < NQ; ++i) acc[j][i] = f32x4{0.f, 0.f, 0.f, 0.f};
    }

    // a tile: positions base + 16 g + q4 (clamped to T - 1) for g = 0, 1
    auto load_tile = [&](f32x4 (&kv)[2][NQ], f32x4 (&vv)[2][NQ], int base) {
#pragma unroll
        for (int g = 0; g < 2; ++g) {
            const long row = static_cast<long>(min(base + 16 * g + q4, T - 1)) * kvd;
#pragma unroll
            for (int i = 0; i < NQ; ++i) {
                const int d = min(4 * r + 16 * i, D - 4);
                kv[g][i] = ld_f32x4(Kh + row + d);
                vv[g][i] = ld_f32x4(Vh + row + d);
            }
        }
    };
    auto run_tile = [&](const f32x4 (&kv)[2][NQ], const f32x4 (&vv)[2][NQ], int base) {
#pragma unroll
        for (int j = 0; j < HQ; ++j) {
            float s_own = -INFINITY;  // lanes r = 2, 3 own no position of a 32-position tile
#pragma unroll
            for (int g = 0; g < 2; ++g) {
                float part = 0.0f;
#pragma unroll
                for (int i = 0; i < NQ; ++i) {
                    part = __builtin_fmaf(qv[j][i].x, kv[g][i].x, part);
                    part = __builtin_fmaf(qv[j][i].y, kv[g][i].y, part);
                    part = __builtin_fmaf(qv[j][i].z, kv[g][i].z, part);
                    part = __builtin_fmaf(qv[j][i].w, kv[g][i].w, part);
                }
                part += dpp<kQuadPerm1032>(part);
                part += dpp<kQuadPerm2301>(part);
                const int pos = base + 16 * g + q4;
                if (g == r) s_own = pos < t1 ? part : -INFINITY;
            }
            // the tile has a valid position, so tmax and m_new are finite
            const float tmax = wave_max(s_own);
            const float m_new = fmaxf(m[j], tmax);
            const float cf = exp2f(m[j] - m_new);
            const float p = exp2f(s_own - m_new);
            l[j] = __builtin_fmaf(l[j], cf, p);
            m[j] = m_new;
            const float p0 = dpp<0x00>(p);  // quad_perm [0,0,0,0]: weight of position 16 * 0 + q
            const float p1 = dpp<0x55>(p);  // quad_perm [1,1,1,1]: weight of position 16 * 1 + q
#pragma unroll
            for (int i = 0; i < NQ; ++i) {
                f32x4 a = acc[j][i] * cf;
                a.x = __builtin_fmaf(p0, vv[0][i].x, a.x);
                a.y = __builtin_fmaf(p0, vv[0][i].y, a.y);
                a.z = __builtin_fmaf(p0, vv[0][i].z, a.z);
                a.w = __builtin_fmaf(p0, vv[0][i].w, a.w);
                a.x = __builtin_fmaf(p1, vv[1][i].x, a.x);
                a.y = __builtin_fmaf(p1, vv[1][i].y, a.y);
                a.z = __builtin_fmaf(p1, vv[1][i].z, a.z);
                a.w = __builtin_fmaf(p1, vv[1][i].w, a.w);
                acc[j][i] = a;
            }
        }
    };
    f32x4 k0[2][NQ], v0[2][NQ];
    if (t1 - t0 == 2 * kSplitTile) {  // two tiles: both requested before the first is computed
        f32x4 k1[2][NQ], v1[2][NQ];
        load_tile(k0, v0, t0);
        load_tile(k1, v1, t0 + kSplitTile);
        __builtin_amdgcn_sched_barrier(0);
        run_tile(k0, v0, t0);
        run_tile(k1, v1, t0 + kSplitTile);
    } else {
        for (int base = t0; base < t1; base += kSplitTile) {
            load_tile(k0, v0, base);
            __builtin_amdgcn_sched_barrier(0);  // the tile's loads stay in flight together
            run_tile(k0, v0, base);
        }
    }

    // sums over the 16 quads (lanes with the same r) and, for l, over all lanes
    const int stride = D + 4;  // record: m, l, 2 pad, acc[D] (16-byte aligned)
#pragma unroll
    for (int j = 0; j < HQ; ++j) {
        const int hg = hq * 4 + wave * HQ + j;
        const float lsum = group_sum_t<6>(l[j]);
        float* rec = ws + ((static_cast<long>(mrow) * H + kvh * G + min(hg, G - 1)) * nchunks + c) * stride;
#pragma unroll
        for (int i = 0; i < NQ; ++i) {
            f32x4 a = acc[j][i];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                float v = a[e];
                v += dpp<0x124>(v);  // row_ror:4
                v += dpp<0x128>(v);  // row_ror:8
                v += swizzle_xor16(v);
                v += shfl_xor32(v);
                a[e] = v;
            }
            const int d = 4 * r + 16 * i;
            if (hg < G && q4 == 0 && d < D) *reinterpret_cast<f32x4*>(rec + 4 + d) = a;
        }
        if (hg < G && lane == 0) {
            rec[0] = m[j];
            rec[1] = lsum;
        }
    }
}

// ---- multi-row split form on the fp32 matrix cores (head_dim 64) ---------------
//
// For a batch of M query rows (consecutive tokens) one workgroup takes 32
// queries -- q = m G + g over the rows m and the G query heads of KV head kvh --
// and one chunk of positions; its kMrWaves waves take the chunk's 32-position
// tiles in turn (wave w: tiles w, w + kMrWaves, ...), so each K and V row of the
// chunk is read once for all 32 queries.  The products run transposed, so that a
// lane owns one query.  Per tile:
//   * S^T = K Q^T, 32 positions x 32 queries, as 32 v_mfma_f32_32x32x2_f32: the
//     u-th takes dim 32 h + u from lane (i, h) for key i (A) and for query i (B);
//     lane (j, h) receives query j's scores at positions 8 (v >> 2) + 4 h + (v & 3),
//     v = 0..15 (fp32 products, fp32 sums);
//   * causal mask (query row m sees positions < Tb + m), online softmax in base
//     2: the query's tile max is over the lane's 16 scores and the other
//     half-wave's 16, each lane keeps its partial sum;
//   * O^T += V^T P^T, 64 dims x 32 queries as two 32 x 32 tiles of 16 MFMAs: the
//     s-th takes position 8 (s >> 2) + 4 h + (s & 3) from lane (i, h), which is
//     exactly the probability lane (j, h) holds in its register s, so P stays in
//     registers;
// then the waves' (max, sum, acc) meet in LDS and the workgroup writes one
// record per (row, head) -- the per-row kernel's format, merged by the same
// combine kernel -- adding the waves' parts in wave order.  All rows share one
// chunk length (from the longest row); chunks past a row's end write empty
// records (max -inf, sum 0).
//
// Workgroup order: the query halves of one (KV head, chunk) are consecutive
// work indices, and when the grid is a multiple of the 8 XCDs each XCD
// (workgroup id mod 8) takes a contiguous range of work indices, so both halves
// read the chunk's K and V through the same L2.
constexpr int kMrD = 64;
constexpr int kMrWaves = 4;
constexpr int kMrAld = kMrD + 4;  // LDS row stride of a wave's accumulators (floats)
constexpr int kXcds = 8;

template <bool PAIR>
__global__ __launch_bounds__(64 * kMrWaves) void decode_attn_mrow_kernel(
    const float* __restrict__ Q, const float* __restrict__ Kc, const float* __restrict__ Vc, float* __restrict__ ws,
    int G, int n_kv, int M, const int* __restrict__ kv_dev, int kv0, float qscale, int nchunks, long ldq,
    float* __restrict__ out, long ldo) {
    __shared__ __attribute__((aligned(16))) float acc_s[kMrWaves][32 * kMrAld];
    __shared__ float mx_s[kMrWaves][32];
    __shared__ float l_s[kMrWaves][32];
    typedef float mr_f16v __attribute__((ext_vector_type(16)));
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, i = lane & 31, h = lane >> 5;
    const int nq = M * G, nqh = (nq + 31) / 32;
    const int nb = static_cast<int>(gridDim.x), b = static_cast<int>(blockIdx.x);
    const int wi = nb % kXcds == 0 ? (b % kXcds) * (nb / kXcds) + b / kXcds : b;
    // PAIR (one chunk, direct output): workgroup p of a KV head takes query groups nqh - 1 - p,
    // then p -- a causal prompt's longest and shortest, so every workgroup does about the same
    // number of tiles
    const int npair = (nqh + 1) / 2;
    const int qh_a = PAIR ? nqh - 1 - wi % npair : wi % nqh;
    const int qh_b = PAIR && wi % npair != nqh - 1 - wi % npair ? wi % npair : -1;
    const int c = PAIR ? 0 : (wi / nqh) % nchunks, kvh = PAIR ? wi / npair : wi / (nqh * nchunks);
    const int H = G * n_kv, kvd = n_kv * kMrD;
    const int Tb = (kv_dev ? *kv_dev : 0) + kv0;  // row m attends to positions [0, Tb + m)
    const int Tmax = Tb + M - 1;
    const int Tc = kSplitTile * ((((Tmax + kSplitTile - 1) / kSplitTile) + nchunks - 1) / nchunks);
    const int t0 = c * Tc, t1 = min(Tmax, t0 + Tc);

    auto run_group = [&](const int qh) {
    // the lane's query (column i of S^T and O^T): row qm, head qg; positions below lim are visible
    const int q = qh * 32 + i;
    const bool qok = q < nq;
    const int qm = qok ? q / G : 0, qg = qok ? q - qm * G : 0;
    const int lim = qok ? min(Tb + qm, t1) : 0;
    float qb[32];  // B operand of S^T: dims 32 h .. + 31 of the query, scaled into base 2
    {
        const float* qp = Q + static_cast<long>(qm) * ldq + static_cast<long>(kvh * G + qg) * kMrD + 32 * h;
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            const f32x4 v = ld_f32x4(qp + 4 * u) * qscale;
            qb[4 * u] = qok ? v.x : 0.0f;
            qb[4 * u + 1] = qok ? v.y : 0.0f;
            qb[4 * u + 2] = qok ? v.z : 0.0f;
            qb[4 * u + 3] = qok ? v.w : 0.0f;
        }
    }
    float mx = -INFINITY, l = 0.0f;
    mr_f16v o0, o1;
#pragma unroll
    for (int v = 0; v < 16; ++v) {
        o0[v] = 0.0f;
        o1[v] = 0.0f;
    }
    const float* Kh = Kc + static_cast<long>(kvh) * kMrD;
    const float* Vh = Vc + static_cast<long>(kvh) * kMrD;

    // one tile's operands: key i's dims 32 h .. + 31 (A of S^T) and, for k slot s, dims i and 32 + i of
    // position 8 (s >> 2) + 4 h + (s & 3) (A of O^T); positions past the end read the last row
    struct Tile {
        f32x4 k[8];
        float v0[16], v1[16];
    };
    auto load_tile = [&](Tile& T, int tb) {
        const float* kp = Kh + static_cast<long>(min(tb + i, Tmax - 1)) * kvd + 32 * h;
#pragma unroll
        for (int u = 0; u < 8; ++u) T.k[u] = ld_f32x4(kp + 4 * u);
#pragma unroll
        for (int s = 0; s < 16; ++s) {
            const float* vp = Vh + static_cast<long>(min(tb + 8 * (s >> 2) + 4 * h + (s & 3), Tmax - 1)) * kvd + i;
            T.v0[s] = vp[0];
            T.v1[s] = vp[32];
        }
    };
    auto run_tile = [&](const Tile& T, int tb) {
        mr_f16v sa, sb;  // two independent chains (even and odd dims)
#pragma unroll
        for (int v = 0; v < 16; ++v) {
            sa[v] = 0.0f;
            sb[v] = 0.0f;
        }
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            sa = __builtin_amdgcn_mfma_f32_32x32x2f32(T.k[u].x, qb[4 * u], sa, 0, 0, 0);
            sb = __builtin_amdgcn_mfma_f32_32x32x2f32(T.k[u].y, qb[4 * u + 1], sb, 0, 0, 0);
            sa = __builtin_amdgcn_mfma_f32_32x32x2f32(T.k[u].z, qb[4 * u + 2], sa, 0, 0, 0);
            sb = __builtin_amdgcn_mfma_f32_32x32x2f32(T.k[u].w, qb[4 * u + 3], sb, 0, 0, 0);
        }
        float p[16];
        float tmax = -INFINITY;
#pragma unroll
        for (int v = 0; v < 16; ++v) {
            p[v] = tb + 8 * (v >> 2) + 4 * h + (v & 3) < lim ? sa[v] + sb[v] : -INFINITY;
            tmax = fmaxf(tmax, p[v]);
        }
        tmax = fmaxf(tmax, shfl_xor32(tmax));  // the query's other 16 positions
        const float mnew = fmaxf(mx, tmax);
        const float base = mnew == -INFINITY ? 0.0f : mnew;  // no visible position yet: every factor 0
        const float cf = __builtin_amdgcn_exp2f(mx - base);
        mx = mnew;
        float ps = 0.0f;
#pragma unroll
        for (int v = 0; v < 16; ++v) {
            p[v] = __builtin_amdgcn_exp2f(p[v] - base);
            ps += p[v];
        }
        l = __builtin_fmaf(l, cf, ps);
        o0 *= cf;
        o1 *= cf;
#pragma unroll
        for (int s = 0; s < 16; ++s) {
            o0 = __builtin_amdgcn_mfma_f32_32x32x2f32(T.v0[s], p[s], o0, 0, 0, 0);
            o1 = __builtin_amdgcn_mfma_f32_32x32x2f32(T.v1[s], p[s], o1, 0, 0, 0);
        }
    };
    // the wave's tiles: the next one's loads are in flight while the current one is computed.
    // They end where the workgroup's last query row stops seeing positions: a prompt's early rows
    // see few, and a tile no query sees would add exact zeros (a causal prompt's query groups
    // skip about half the tiles of the chunk)
    const int te = min(t1, Tb + min(nq - 1, qh * 32 + 31) / G);
    constexpr int kStep = kMrWaves * kSplitTile;
    int tb = t0 + w * kSplitTile;
    if (tb < te) {
        Tile T0, T1;
        load_tile(T0, tb);
        while (true) {
            if (tb + kStep >= te) {
                run_tile(T0, tb);
                break;
            }
            load_tile(T1, tb + kStep);
            run_tile(T0, tb);
            tb += kStep;
            if (tb + kStep >= te) {
                run_tile(T1, tb);
                break;
            }
            load_tile(T0, tb + kStep);
            run_tile(T1, tb);
            tb += kStep;
        }
    }

    // the waves meet in LDS: max and sum per query, accumulators per (query, dim)
    const float lq = l + shfl_xor32(l);
    if (h == 0) {
        mx_s[w][i] = mx;
        l_s[w][i] = lq;
    }
    float* a = acc_s[w] + i * kMrAld + 4 * h;
#pragma unroll
    for (int g = 0; g < 4; ++g) {
        *reinterpret_cast<f32x4*>(a + 8 * g) = f32x4{o0[4 * g], o0[4 * g + 1], o0[4 * g + 2], o0[4 * g + 3]};
        *reinterpret_cast<f32x4*>(a + 32 + 8 * g) = f32x4{o1[4 * g], o1[4 * g + 1], o1[4 * g + 2], o1[4 * g + 3]};
    }
    __syncthreads();
    // records: eight threads per query, eight dims each
    const int rq = tid >> 3, d0 = 8 * (tid & 7), qq = qh * 32 + rq;
    if (qq >= nq) return;
    float mw[kMrWaves], Mx = -INFINITY;
#pragma unroll
    for (int u = 0; u < kMrWaves; ++u) {
        mw[u] = mx_s[u][rq];
        Mx = fmaxf(Mx, mw[u]);
    }
    float L = 0.0f;
    f32x4 r0 = {0.0f, 0.0f, 0.0f, 0.0f}, r1 = r0;
#pragma unroll
    for (int u = 0; u < kMrWaves; ++u) {
        const float f = mw[u] == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(mw[u] - Mx);
        L = __builtin_fmaf(f, l_s[u][rq], L);
        const float* src = acc_s[u] + rq * kMrAld + d0;
        r0 += f * *reinterpret_cast<const f32x4*>(src);
        r1 += f * *reinterpret_cast<const f32x4*>(src + 4);
    }
    const int m = qq / G, g = qq - m * G;
    if (out) {  // one chunk: the merged output itself, as the combine kernel would divide it
        float* o = out + m * ldo + static_cast<long>(kvh * G + g) * kMrD + d0;
        *reinterpret_cast<f32x4*>(o) = f32x4{r0.x / L, r0.y / L, r0.z / L, r0.w / L};
        *reinterpret_cast<f32x4*>(o + 4) = f32x4{r1.x / L, r1.y / L, r1.z / L, r1.w / L};
        return;
    }
    float* rec = ws + ((static_cast<long>(m) * H + kvh * G + g) * nchunks + c) * (kMrD + 4);
    *reinterpret_cast<f32x4*>(rec + 4 + d0) = r0;
    *reinterpret_cast<f32x4*>(rec + 8 + d0) = r1;
    if (d0 == 0) {
        rec[0] = Mx;
        rec[1] = L;
    }
    };
    run_group(qh_a);
    if constexpr (PAIR) {
        if (qh_b >= 0) {
            __syncthreads();  // the first group's merge has read the LDS accumulators
            run_group(qh_b);
        }
    }
}

// out[m][h][d] = sum_c 2^(m_c - M) acc_c[d] / sum_c 2^(m_c - M) l_c, M = max_c m_c,
// for query row m = blockIdx.y (output rows ldo floats apart).  One workgroup of
// kCombineWaves waves per (row, head): its threads take the chunks for the max and
// the sum (their loads are independent), the factors go through LDS; wave w adds up
// the accumulators of chunks w, w + kCombineWaves, ... (eight loads in flight), and
// the waves' partial numerators are added in wave order.  Empty chunks (max -inf)
// get the factor 0; chunk 0 always holds a position.
constexpr int kCombineMaxChunks = 4096;
constexpr int kCombineWaves = 4;

__global__ __launch_bounds__(64 * kCombineWaves) void decode_attn_combine_kernel(const float* __restrict__ ws,
                                                                                 float* __restrict__ out, int D,
                                                                                 int nchunks, long ldo) {
    constexpr int kT = 64 * kCombineWaves;
    __shared__ float fs[kCombineMaxChunks];
    __shared__ float red[kCombineWaves];
    __shared__ float part[kCombineWaves][detail::kDecodeAttnSplitMaxHeadDim];
    const int h = blockIdx.x, mrow = blockIdx.y, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int stride = D + 4;
    const float* P = ws + (static_cast<long>(mrow) * gridDim.x + h) * nchunks * stride;
    float mloc = -INFINITY;
    for (int c = tid; c < nchunks; c += kT) mloc = fmaxf(mloc, P[static_cast<long>(c) * stride]);
    mloc = wave_max(mloc);
    if (lane == 0) red[wave] = mloc;
    __syncthreads();
    float M = red[0];
#pragma unroll
    for (int w = 1; w < kCombineWaves; ++w) M = fmaxf(M, red[w]);
    __syncthreads();  // red is reused below
    float lloc = 0.0f;
    for (int c = tid; c < nchunks; c += kT) {
        const float f = exp2f(P[static_cast<long>(c) * stride] - M);
        fs[c] = f;
        lloc = __builtin_fmaf(f, P[static_cast<long>(c) * stride + 1], lloc);
    }
    lloc = group_sum_t<6>(lloc);
    if (lane == 0) red[wave] = lloc;
    __syncthreads();
    float den = red[0];
#pragma unroll
    for (int w = 1; w < kCombineWaves; ++w) den += red[w];
    for (int d0 = 0; d0 < D; d0 += 64) {
        const int d = min(d0 + lane, D - 1);
        float num = 0.0f;
#pragma unroll 8
        for (int c = wave; c < nchunks; c += kCombineWaves)
            num = __builtin_fmaf(fs[c], P[static_cast<long>(c) * stride + 4 + d], num);
        if (d0 + lane < D) part[wave][d0 + lane] = num;
    }
    __syncthreads();
    float* o = out + mrow * ldo + static_cast<long>(h) * D;
    for (int d = tid; d < D; d += kT) {
        float num = part[0][d];
#pragma unroll
        for (int w = 1; w < kCombineWaves; ++w) num += part[w][d];
        o[d] = num / den;
    }
}

// The same merge for head_dim 64 and at most 32 chunks (the decode steps' shapes) in one round
// trip: thread t takes chunk t / 8 and dims 8 (t % 8) .. + 8 and issues its record loads (max,
// sum, 8 accumulators) before anything is reduced; the chunk factors stay in registers, each
// wave adds its 8 chunks with cross-lane sums (lanes t, t ^ 8, t ^ 16, t ^ 32 hold the same dims),
// and the four waves' parts are added in wave order through LDS.  The general kernel above
// loads the maxima, reduces them, and only then loads the accumulators.
constexpr int kCombine64MaxChunks = 32;

__global__ __launch_bounds__(256) void decode_attn_combine64_kernel(const float* __restrict__ ws,
                                                                    float* __restrict__ out, int nchunks, long ldo) {
    constexpr int D = 64, stride = D + 4;
    __shared__ float red[2][4];
    __shared__ float part[4][D];
    const int h = blockIdx.x, mrow = blockIdx.y, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int c = tid >> 3, j = tid & 7;
    const float* rec = ws + ((static_cast<long>(mrow) * gridDim.x + h) * nchunks + min(c, nchunks - 1)) * stride;
    const bool live = c < nchunks;
    const float mc = live ? rec[0] : -INFINITY;
    const float lc = live ? rec[1] : 0.0f;
    const f32x4 a0 = ld_f32x4(rec + 4 + 8 * j), a1 = ld_f32x4(rec + 8 + 8 * j);
    const float wm = wave_max(mc);
    if (lane == 0) red[0][wave] = wm;
    __syncthreads();
    const float M = fmaxf(fmaxf(red[0][0], red[0][1]), fmaxf(red[0][2], red[0][3]));
    const float f = live ? exp2f(mc - M) : 0.0f;  // empty chunks (max -inf): 0
    const float ls = group_sum_t<6>(j == 0 ? f * lc : 0.0f);
    float v[8] = {f * a0.x, f * a0.y, f * a0.z, f * a0.w, f * a1.x, f * a1.y, f * a1.z, f * a1.w};
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        float x = v[e];
        x += dpp<0x128>(x);  // row_ror:8 (lane ^ 8 inside a row of 16)
        x += swizzle_xor16(x);
        x += shfl_xor32(x);
        v[e] = x;
    }
    if (lane < 8) {
#pragma unroll
        for (int e = 0; e < 8; ++e) part[wave][8 * lane + e] = v[e];
    }
    if (lane == 0) red[1][wave] = ls;
    __syncthreads();
    if (tid < D) {
        const float den = ((red[1][0] + red[1][1]) + red[1][2]) + red[1][3];
        const float num = ((part[0][tid] + part[1][tid]) + part[2][tid]) + part[3][tid];
        out[mrow * ldo + static_cast<long>(h) * D + tid] = num / den;
    }
}

}  // namespace dev

namespace detail {

// merge the chunk records of every (row, head)
static void launch_combine(const float* ws, float* out, int n_heads, int rows, int D, int nchunks, long ldo,
                           hipStream_t stream) {
    const dim3 grid(n_heads, static_cast<unsigned>(rows));
    if (D == 64 && nchunks <= dev::kCombine64MaxChunks)
        hipLaunchKernelGGL(dev::decode_attn_combine64_kernel, grid, dim3(256), 0, stream, ws, out, nchunks, ldo);
    else
        hipLaunchKernelGGL(dev::decode_attn_combine_kernel, grid, dim3(64 * dev::kCombineWaves), 0, stream, ws, out,
                           D, nchunks, ldo);
}

template <int NQ>
static void launch_att(bool vec, dim3 grid, hipStream_t stream, const float* Q, const float* K, const float* V,
                       float* out, int G, int kvd, int D, int T, float qscale, int n_slices, int remap) {
    if (vec)
        hipLaunchKernelGGL((dev::decode_attn_kernel<NQ, true>), grid, dim3(64 * dev::kAttWaves), 0, stream, Q, K, V,
                           out, G, kvd, D, T, qscale, n_slices, remap);
    else
        hipLaunchKernelGGL((dev::decode_attn_kernel<NQ, false>), grid, dim3(64 * dev::kAttWaves), 0, stream, Q, K, V,
                           out, G, kvd, D, T, qscale, n_slices, remap);
}

constexpr int kSplitHeadsPerWave = 1;  // 4 waves per workgroup, one query head each
constexpr int kMrowMinRows = 4;        // from this many query rows on, head_dim 64 takes the matrix-core form

// Split form: number of chunks (of whole 32-position tiles) that gives ~256
// workgroups per query row at kv_len positions (measured: 512 or 1024 smaller
// chunks are no faster at 2048 positions, slower at 8192); fewer chunks when the
// workspace (ws_floats >= 0) is smaller.  The kernel recomputes the chunk
// length from the row's own length.
static int split_chunks(int n_heads, int n_kv_heads, int D, int kv_len, int rows, long ws_floats) {
    const int G = n_heads / n_kv_heads, nhq = (G + 3) / 4;
    const long groups = static_cast<long>(n_kv_heads) * nhq;
    const long tiles = (kv_len + dev::kSplitTile - 1) / dev::kSplitTile;
    long per = (tiles * groups + 255) / 256;  // tiles per chunk
    if (per < 1) per = 1;
    long nchunks = (tiles + per - 1) / per;
    if (nchunks > dev::kCombineMaxChunks) nchunks = dev::kCombineMaxChunks;  // the combine kernel's factor array
    const long rec = static_cast<long>(rows) * n_heads * (D + 4);
    if (ws_floats >= 0 && nchunks * rec > ws_floats) nchunks = ws_floats / rec;
    return static_cast<int>(nchunks);
}

// The multi-row (matrix-core) form gives each workgroup's kMrWaves waves one
// 32-position tile each per chunk, up to kMrowMaxChunks chunks (at 2048 positions:
// 16 chunks x 8 KV heads x 2 query halves = 256 workgroups for a batch of 16).
constexpr int kMrowMaxChunks = 16;

static bool use_mrow(int rows, int head_dim) { return head_dim == dev::kMrD && rows >= kMrowMinRows; }

bool decode_attention_split_supported(const float* Q, const float* K, const float* V, int head_dim) {
    auto a16 = [](const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; };
    return head_dim >= 4 && head_dim <= kDecodeAttnSplitMaxHeadDim && head_dim % 4 == 0 && a16(Q) && a16(K) &&
           a16(V);
}

long decode_attention_workspace_bytes(int n_heads, int n_kv_heads, int head_dim, int kv_len) {
    const int nchunks = split_chunks(n_heads, n_kv_heads, head_dim, kv_len, 1, -1);
    return static_cast<long>(nchunks) * n_heads * (head_dim + 4) * 4;
}

int launch_decode_attention_rows(const float* Q, long ldq, const float* K, const float* V, float* out, long ldo,
                                 int rows, int n_heads, int n_kv_heads, int head_dim, const int* kv_dev, int kv0,
                                 int nchunks, float scale, float* ws, hipStream_t stream) {
    const int D = head_dim, G = n_heads / n_kv_heads, nhq = (G + 3) / 4;
    if (nchunks < 1 || nchunks > dev::kCombineMaxChunks || rows < 1 || rows > 65535) return kDeclined;
    // the record and combine layouts, and the kernels' 16-byte loads of Q rows (ldq floats apart), K and V
    if (!decode_attention_split_supported(Q, K, V, D) || ldq % 4 != 0) return kDeclined;
    const long blocks = static_cast<long>(n_kv_heads) * nhq * nchunks;
    if (blocks > 0x7FFFFFFFL) return kDeclined;
    const float qscale = scale * 1.44269504088896341f;
    if (use_mrow(rows, D)) {
        // several query rows: the rows share each chunk's K / V reads on the matrix cores
        const long nqh = (static_cast<long>(rows) * G + 31) / 32;
        const long wgs = static_cast<long>(n_kv_heads) * nchunks * nqh;
        if (wgs > 0x7FFFFFFFL) return kDeclined;
        // one chunk (a prompt's many query groups fill the GPU alone): the kernel writes the output
        const bool direct = nchunks == 1 && ldo % 4 == 0 && (reinterpret_cast<uintptr_t>(out) & 15u) == 0;
        // one chunk: query groups in pairs, the longest with the shortest (half the workgroups)
        const long pwgs = static_cast<long>(n_kv_heads) * ((nqh + 1) / 2);
        if (direct)
            hipLaunchKernelGGL(dev::decode_attn_mrow_kernel<true>, dim3(static_cast<unsigned>(pwgs)),
                               dim3(64 * dev::kMrWaves), 0, stream, Q, K, V, ws, G, n_kv_heads, rows, kv_dev, kv0,
                               qscale, nchunks, ldq, out, ldo);
        else
            hipLaunchKernelGGL(dev::decode_attn_mrow_kernel<false>, dim3(static_cast<unsigned>(wgs)),
                               dim3(64 * dev::kMrWaves), 0, stream, Q, K, V, ws, G, n_kv_heads, rows, kv_dev, kv0,
                               qscale, nchunks, ldq, nullptr, ldo);
        if (!direct) launch_combine(ws, out, n_heads, rows, D, nchunks, ldo, stream);
        return 0;
    }
    const dim3 grid(static_cast<unsigned>(blocks), static_cast<unsigned>(rows));
    if (D <= 64)
        hipLaunchKernelGGL((dev::decode_attn_split_kernel<kSplitHeadsPerWave, 4>), grid, dim3(256 / kSplitHeadsPerWave),
                           0, stream, Q, K, V, ws, G, n_kv_heads * D, D, kv_dev, kv0, qscale, nchunks, nhq, ldq);
    else
        hipLaunchKernelGGL((dev::decode_attn_split_kernel<kSplitHeadsPerWave, 8>), grid, dim3(256 / kSplitHeadsPerWave),
                           0, stream, Q, K, V, ws, G, n_kv_heads * D, D, kv_dev, kv0, qscale, nchunks, nhq, ldq);
    launch_combine(ws, out, n_heads, rows, D, nchunks, ldo, stream);
    return 0;
}

bool decode_attention_rows_mrow(int rows, int head_dim) { return use_mrow(rows, head_dim); }

int decode_attention_rows_chunks(int n_heads, int n_kv_heads, int head_dim, int max_kv_len, int rows) {
    if (use_mrow(rows, head_dim)) {
        const int tiles = (max_kv_len + dev::kSplitTile - 1) / dev::kSplitTile;
        const int per_wg = (tiles + dev::kMrWaves - 1) / dev::kMrWaves;
        int n = per_wg < 1 ? 1 : (per_wg < kMrowMaxChunks ? per_wg : kMrowMaxChunks);
        // many query groups (a prompt: rows x heads / 32 of them per KV head) already fill the GPU:
        // fewer, longer chunks (about 512 workgroups in all), down to one, whose workgroups write
        // the output without records or a combine launch
        const long groups = static_cast<long>(n_kv_heads) * ((static_cast<long>(rows) * (n_heads / n_kv_heads) + 31) / 32);
        const long cap = (512 + groups - 1) / groups;
        if (cap < n) n = static_cast<int>(cap);
        return n;
    }
    return split_chunks(n_heads, n_kv_heads, head_dim, max_kv_len, 1, -1);
}

int launch_decode_attention_split(const float* Q, const float* K, const float* V, float* out, int n_heads,
                                  int n_kv_heads, int head_dim, int kv_len, float scale, float* ws, long ws_bytes,
                                  hipStream_t stream) {
    const int nchunks = split_chunks(n_heads, n_kv_heads, head_dim, kv_len, 1, ws_bytes / 4);
    if (nchunks < 1) return -2;  // workspace too small for one record per head
    return launch_decode_attention_rows(Q, 0, K, V, out, 0, 1, n_heads, n_kv_heads, head_dim, nullptr, kv_len,
                                        nchunks, scale, ws, stream);
}

int noalloc_scratch(float** out) {
    constexpr int kMaxDevices = 64;
    static std::atomic<float*> ptrs[kMaxDevices];
    int devid = 0;
    if (hipGetDevice(&devid) != hipSuccess || devid < 0 || devid >= kMaxDevices) return kFailed;
    float* p = ptrs[devid].load(std::memory_order_acquire);
    if (!p) {
        void* addr = nullptr;
        // with this device current: its own copy of the array
        if (hipGetSymbolAddress(&addr, HIP_SYMBOL(scratch)) != hipSuccess || !addr) return kFailed;
        p = static_cast<float*>(addr);
        ptrs[devid].store(p, std::memory_order_release);
    }
    *out = p;
    return 0;
}

int launch_decode_attention(const float* Q, const float* K, const float* V, float* out, int n_heads, int n_kv_heads,
                            int head_dim, int kv_len, float scale, hipStream_t stream) {
    const int D = head_dim;
    if (D < 1 || D > kDecodeAttnMaxHeadDim || kv_len < 1) return -1;
    const int G = n_heads / n_kv_heads, kvd = n_kv_heads * D;
    const int n_slices = (D + dev::kAttDs - 1) / dev::kAttDs;
    const long blocks = static_cast<long>(n_heads) * n_slices;
    if (blocks > 0x7FFFFFFFL) return -1;
    auto a16 = [](const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; };
    const bool vec = D % 4 == 0 && a16(Q) && a16(K) && a16(V);
    const int remap = blocks % 8 == 0;
    const float qscale = scale * 1.44269504088896341f;  // log2(e): the kernel works in base 2
    const dim3 grid(static_cast<unsigned>(blocks));
    if (D <= 16) launch_att<1>(vec, grid, stream, Q, K, V, out, G, kvd, D, kv_len, qscale, n_slices, remap);
    else if (D <= 32) launch_att<2>(vec, grid, stream, Q, K, V, out, G, kvd, D, kv_len, qscale, n_slices, remap);
    else if (D <= 64) launch_att<4>(vec, grid, stream, Q, K, V, out, G, kvd, D, kv_len, qscale, n_slices, remap);
    else if (D <= 128) launch_att<8>(vec, grid, stream, Q, K, V, out, G, kvd, D, kv_len, qscale, n_slices, remap);
    else launch_att<16>(vec, grid, stream, Q, K, V, out, G, kvd, D, kv_len, qscale, n_slices, remap);
    return 0;
}

}  // namespace detail
}  // namespace cri
