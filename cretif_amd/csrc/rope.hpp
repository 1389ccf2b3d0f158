// rope.hpp -- the fused q/k/v projection's epilogue for one decode token: RoPE on q and k
// (ref:src/kernels/elementwise.cu:232-257, the angle read from the step's (cos, sin) table) and
// the KV-cache append (ref:src/kv_cache.cu:157-211), shared by the batch-1 GEMV kernels.
#pragma once

#include "common.hpp"
#include "internal.hpp"

namespace cri {
namespace dev {

// Output column n (value x, its pair partner xp) of the fused q/k/v projection: q and k
// rotated by the angle of (position, pair) as the RoPE kernel does, q to q_out, k and v to
// cache row pos.
__device__ __forceinline__ void rope_out(const RopeOut& R, float* q_out, int n, float x, float xp) {
    const int pos = *R.pos;
    const long kvrow = static_cast<long>(pos) * R.kvd;
    if (n < R.qd + R.kvd) {
        const int nn = n < R.qd ? n : n - R.qd;
        const int lp = (nn % (2 * R.half)) >> 1;
        const f32x2 cs = reinterpret_cast<const f32x2*>(R.rot)[static_cast<long>(pos) * R.half + lp];
        const bool odd = n & 1;
        const float x0 = odd ? xp : x, x1 = odd ? x : xp;
        const float v = odd ? __fadd_rn(__fmul_rn(x0, cs.y), __fmul_rn(x1, cs.x))
                            : __fsub_rn(__fmul_rn(x0, cs.x), __fmul_rn(x1, cs.y));
        if (n < R.qd)
            q_out[n] = v;
        else
            R.kc[kvrow + nn] = v;
    } else {
        R.vc[kvrow + (n - R.qd - R.kvd)] = x;
    }
}

}  // namespace dev
}  // namespace cri
