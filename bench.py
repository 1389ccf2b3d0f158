#!/usr/bin/env python3
"""Benchmark of the fused dequant+matmul path on one MI355X.

Headline (the `value` of the JSON line): weight GB/s of the batch-1 Q4_K
decode GEMV at the Llama-3.2-1B FFN gate/up shape (N=8192, K=2048).  One
"step" is one GEMV launch over one batch of synthetic input.  The weights are
rotated over enough distinct copies (>= 2x the 256 MB Infinity Cache) that each
launch streams its matrix from HBM; the launches are captured once in a HIP
graph and replayed, and the timed region is bracketed by HIP events on the
replay stream plus device synchronisation.

GB/s counts algorithmic bytes only: N*(K/bs)*block_bytes + 4*M*K + 4*M*N.

    python bench.py [--steps K] [--warmup W] [--workload NAME] [--no-cpu] [--no-details]
"""
from __future__ import annotations

import argparse
import json
import os
import platform
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

import numpy as np  # noqa: E402

HBM_PEAK_GBS = 8000.0
FP16_MFMA_PEAK_TFLOPS = 2500.0  # MI355X dense fp16 matrix peak
MALL_BYTES = 256 << 20

# Multi-token prefill GEMMs: name -> (fmt, M, N, K); reported in TFLOP/s.
PREFILL_WORKLOADS = {
    "q8_0_prefill": ("q8_0", 512, 8192, 2048),
    "q8_0_prefill_down": ("q8_0", 512, 2048, 8192),
    "q4_k_prefill": ("q4_k", 512, 8192, 2048),
    "q4_k_prefill_down": ("q4_k", 512, 2048, 8192),
}

GEMV_WORKLOADS = {
    # name: (fmt, N, K)
    "q4_k_gemv": ("q4_k", 8192, 2048),
    "q8_0_gemv": ("q8_0", 8192, 2048),
    "q4_0_gemv": ("q4_0", 8192, 2048),
    "q5_0_gemv": ("q5_0", 8192, 2048),
    "q6_k_gemv": ("q6_k", 2048, 2048),
    "fp16_gemv": ("fp16", 8192, 2048),
    "q4_k_gemv_down": ("q4_k", 2048, 8192),
    "q8_0_gemv_down": ("q8_0", 2048, 8192),
    "q6_k_lm_head": ("q6_k", 128256, 2048),
    # the reference's tied LM head: the token table dequantized to fp32 and multiplied by
    # matmul_transposed_b (ref:src/model.cu:1027-1029); against q6_k_lm_head / q8_0_lm_head it
    # shows what keeping the tied table quantized saves
    "fp32_tied_lm_head": ("fp32", 128256, 2048),
    "q8_0_lm_head": ("q8_0", 128256, 2048),
}


def algo_bytes(fmt, M, N, K):
    from cretif_amd import quant

    return N * quant.row_bytes(fmt, K) + 4 * M * K + 4 * M * N


class GemvRig:
    """Weights replicated over `copies` device buffers, launches captured in a graph."""

    def __init__(self, fmt, N, K, M=1, seed=1, min_bytes=2 * MALL_BYTES, max_copies=64):
        import torch

        import cretif_amd as cri
        from cretif_amd import quant

        self.fmt, self.N, self.K, self.M = fmt, N, K, M
        w = tiled_weights(fmt, N, K, seed=seed) if fmt != "fp32" else \
            quant.randn(N * K, seed=seed).astype(np.float32).view(np.uint8)
        self.wbytes = w.size
        self.copies = int(max(1, min(max_copies, -(-min_bytes // w.size))))
        base = torch.from_numpy(w).cuda()
        self.W = [base] + [base.clone() for _ in range(self.copies - 1)]
        self.x = torch.from_numpy(quant.randn(M * K, seed=seed + 1).reshape(M, K)).cuda()
        self.y = torch.empty(M, N, device="cuda")
        self.cri = cri
        torch.cuda.synchronize()
        self.graph = torch.cuda.CUDAGraph()
        side = torch.cuda.Stream()
        def run(Wi):
            if fmt == "fp32":
                cri.matmul_transposed_b(self.x, Wi, self.y, M, N, K)
            else:
                cri.matmul(fmt, self.x, Wi, self.y, M, N, K)

        with torch.cuda.stream(side):
            for Wi in self.W:  # eager warm-up on the side stream
                run(Wi)
        side.synchronize()
        with torch.cuda.graph(self.graph, stream=side):
            for Wi in self.W:
                run(Wi)
        torch.cuda.synchronize()

    def bytes_per_launch(self):
        return algo_bytes(self.fmt, self.M, self.N, self.K)

    def time(self, steps, warmup):
        """Returns (ms per launch, launches timed)."""
        import torch

        reps = max(1, -(-steps // self.copies))
        wreps = max(1, -(-warmup // self.copies))
        for _ in range(wreps):
            self.graph.replay()
        torch.cuda.synchronize()
        start = torch.cuda.Event(enable_timing=True)
        end = torch.cuda.Event(enable_timing=True)
        start.record()
        for _ in range(reps):
            self.graph.replay()
        end.record()
        torch.cuda.synchronize()
        launches = reps * self.copies
        return start.elapsed_time(end) / launches, launches

    def free(self):
        self.W = None
        self.graph = None


class StreamRig:
    """The achievable streaming-read line: cri_stream_read over `copies` buffers of n_bytes (rotated
    over >= 2x the Infinity Cache, as the GEMVs), launches captured in a graph, timed as GemvRig."""

    def __init__(self, n_bytes, min_bytes=2 * MALL_BYTES, max_copies=64):
        import torch

        import cretif_amd as cri

        self.n_bytes = n_bytes
        self.copies = int(max(1, min(max_copies, -(-min_bytes // n_bytes))))
        base = torch.zeros(n_bytes, dtype=torch.uint8, device="cuda")
        self.W = [base] + [base.clone() for _ in range(self.copies - 1)]
        self.sink = torch.zeros(1, dtype=torch.int32, device="cuda")
        side = torch.cuda.Stream()
        with torch.cuda.stream(side):
            for Wi in self.W:
                cri.stream_read(Wi, n_bytes, self.sink)
        side.synchronize()
        self.graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(self.graph, stream=side):
            for Wi in self.W:
                cri.stream_read(Wi, n_bytes, self.sink)
        torch.cuda.synchronize()

    time = GemvRig.time

    def free(self):
        self.W = None
        self.graph = None


def tiled_weights(fmt, N, K, seed, max_rows=8192):
    """Synthetic weights of N rows built from at most `max_rows` quantized rows
    repeated (rows are independent, so the bytes streamed per launch are the
    same; the large Q6_K lm_head would otherwise take ~40 s of host
    quantization)."""
    from cretif_amd import quant

    if N <= max_rows:
        return quant.synthetic_weights(fmt, N, K, seed=seed)
    rows = next(r for r in range(max_rows, 0, -1) if N % r == 0)
    base = quant.synthetic_weights(fmt, rows, K, seed=seed).reshape(rows, -1)
    return np.ascontiguousarray(np.tile(base, (N // rows, 1))).ravel()


class DecodeStepRig:
    """Synthetic Llama-3.2-1B-shaped decode step for M
    tokens: 16 layers of Q4_K q (2048x2048), k and v (512x2048), o (2048x2048),
    gate and up (8192x2048), down (2048x8192) plus the GQA QK^T and PV products
    over an fp32 KV cache of T = 2048 positions (32 query heads over 8 KV heads,
    head_dim 64), then the Q6_K lm_head (128256x2048).  The step is the path's
    own kernels only (norms, RoPE, softmax and SiLU are not on the path); every
    layer has its own weight and cache buffers, and the whole step is captured
    as one HIP graph and replayed.  As inference engines do, the q/k/v weights
    of a layer are stored as one [3072, 2048] matrix and gate/up as one
    [16384, 2048] matrix, so a layer is 4 weight launches (same bytes, fewer
    launches).  Buffers are reused between layers: the timing covers the
    products at their real shapes; the values are not chained semantically.
    attention='fused' (M = 1) replaces the two GQA products by the fused decode
    attention (softmax included) over a [T, 8, 64] cache, in its split form
    with a preallocated workspace, as the reference's decode path calls
    fused_decode_attention (ref:src/model.cu:928-943)."""

    LAYERS, D, H, HKV, HD, FF, VOCAB, T = 16, 2048, 32, 8, 64, 8192, 128256, 2048

    def __init__(self, M, seed=1100, attention="gqa", elementwise="none"):
        import torch

        import cretif_amd as cri

        if attention not in ("gqa", "fused") or (attention == "fused" and M != 1):
            raise ValueError("attention is 'gqa', or 'fused' for M = 1 (one query token)")
        if elementwise not in ("none", "separate", "fused") or (elementwise == "separate" and M != 1):
            raise ValueError("elementwise is 'none', 'fused', or 'separate' for M = 1")
        self.M, self.attention, self.elementwise = M, attention, elementwise
        D, FF, T, H, HKV, HD = self.D, self.FF, self.T, self.H, self.HKV, self.HD
        shapes = {"qkv": (D + 2 * HKV * HD, D), "o": (D, D), "gateup": (2 * FF, D), "down": (D, FF)}
        base = {name: torch.from_numpy(tiled_weights("q4_k", n, k, seed + i)).cuda()
                for i, (name, (n, k)) in enumerate(shapes.items())}
        self.layers = [{name: base[name].clone() for name in shapes} for _ in range(self.LAYERS)]
        del base
        self.lm_head = torch.from_numpy(tiled_weights("q6_k", self.VOCAB, D, seed + 99)).cuda()
        g = torch.Generator(device="cuda").manual_seed(3000)
        if attention == "gqa":
            # batched_matmul_gqa operands: K^T [Hkv, HD, T] and V [Hkv, T, HD] per layer
            self.kT = [torch.randn(HKV, HD, T, device="cuda", generator=g) for _ in range(self.LAYERS)]
            self.vc = [torch.randn(HKV, T, HD, device="cuda", generator=g) for _ in range(self.LAYERS)]
        else:
            # fused decode attention reads the cache layout [T, Hkv, HD] directly
            self.kT = [torch.randn(T, HKV, HD, device="cuda", generator=g) for _ in range(self.LAYERS)]
            self.vc = [torch.randn(T, HKV, HD, device="cuda", generator=g) for _ in range(self.LAYERS)]
            self.ws = torch.empty(cri.decode_attention_workspace_size(H, HKV, HD, T) // 4, device="cuda")
        self.x = torch.randn(M, D, device="cuda", generator=g)
        self.qkv = torch.empty(M, D + 2 * HKV * HD, device="cuda")
        self.scores = torch.empty(H, M, T, device="cuda")
        self.ctx = torch.empty(H, M, HD, device="cuda")
        self.h = torch.empty(M, D, device="cuda")
        self.ff = torch.empty(M, 2 * FF, device="cuda")
        # residual stream and norms (elementwise != "none"): two hidden buffers (the fused
        # form writes hidden + residual to the other one), RMSNorm weights ~ 1 + N(0, 0.1)
        self.hid = [torch.randn(M, D, device="cuda", generator=g) for _ in range(2)]
        self.attn_out = torch.empty(M, D, device="cuda")
        self.ffn_out = torch.empty(M, D, device="cuda")
        self.normed = torch.empty(M, D, device="cuda")
        self.act = torch.empty(M, FF, device="cuda")
        self.norm_w = [1.0 + 0.1 * torch.randn(D, device="cuda", generator=g) for _ in range(2 * self.LAYERS + 1)]
        self.logits = torch.empty(M, self.VOCAB, device="cuda")
        self.weight_bytes = sum(t.numel() for L in self.layers for t in L.values()) + self.lm_head.numel()
        self.kv_bytes = sum(t.numel() * 4 for t in self.kT) + sum(t.numel() * 4 for t in self.vc)
        self.cri = cri
        side = torch.cuda.Stream()
        with torch.cuda.stream(side):
            self.step()
        side.synchronize()
        self.graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(self.graph, stream=side):
            self.step()
        torch.cuda.synchronize()

    def step(self):
        if self.elementwise != "none":
            return self.step_with_norms()
        cri, M, D, FF, HKV, HD = self.cri, self.M, self.D, self.FF, self.HKV, self.HD
        x = self.x
        for li, L in enumerate(self.layers):
            cri.matmul("q4_k", x, L["qkv"], self.qkv, M, D + 2 * HKV * HD, D)
            # the first 32*M*64 values of the qkv output read as [32, M, 64] queries; 'fused' is
            # softmax(q K^T / 8) V in one call (its split form)
            self.attend(li)
            cri.matmul("q4_k", self.ctx, L["o"], self.h, M, D, D)
            cri.matmul("q4_k", self.h, L["gateup"], self.ff, M, 2 * FF, D)
            # the first M*8192 values of the gate/up output read as the [M, 8192] down input
            cri.matmul("q4_k", self.ff, L["down"], self.h, M, D, FF)
            x = self.h
        cri.matmul("q6_k", x, self.lm_head, self.logits, M, self.VOCAB, D)

    def attend(self, li):
        cri, M, H, HKV, HD, T = self.cri, self.M, self.H, self.HKV, self.HD, self.T
        if self.attention == "gqa":
            cri.batched_matmul_gqa(self.qkv, self.kT[li], self.scores, H, HKV, M, T, HD)
            cri.batched_matmul_gqa(self.scores, self.vc[li], self.ctx, H, HKV, M, HD, T)
        else:
            cri.fused_decode_attention_ws(self.qkv, self.kT[li], self.vc[li], self.ctx, H, HKV, HD, T, 0.125, self.ws)

    def step_with_norms(self):
        """The layer with its elementwise neighbours, as the reference's decode loop runs it
        (ref:src/model.cu:894-1018): h += ffn_out; n = RMSNorm(h); q/k/v; attention; o;
        h += attn_out; n = RMSNorm(h); gate/up; silu(gate) * up; down; and after the last
        layer h += ffn_out; n = RMSNorm(h); lm_head.  'separate' launches rmsnorm_residual
        and silu_mul; 'fused' folds them into the next matmul's activation staging."""
        cri, M, D, FF, HKV, HD = self.cri, self.M, self.D, self.FF, self.HKV, self.HD
        fused = self.elementwise == "fused"
        cur, res = 0, None  # hidden buffer in use; residual still to be added (none before layer 0)
        eps = 1e-5

        def norm_then(w, Wq, out, N, fmt="q4_k"):
            nonlocal cur
            if fused:
                cri.matmul_rmsnorm(fmt, self.hid[cur], res, w, self.hid[1 - cur], Wq, out, M, N, D, eps)
                cur = 1 - cur
            else:
                cri.rmsnorm_residual(self.hid[cur], res, w, self.hid[cur], self.normed, M, D, eps)
                cri.matmul(fmt, self.normed, Wq, out, M, N, D)

        for li, L in enumerate(self.layers):
            norm_then(self.norm_w[2 * li], L["qkv"], self.qkv, D + 2 * HKV * HD)
            self.attend(li)
            cri.matmul("q4_k", self.ctx, L["o"], self.attn_out, M, D, D)
            res = self.attn_out
            norm_then(self.norm_w[2 * li + 1], L["gateup"], self.ff, 2 * FF)
            if fused:
                cri.matmul_swiglu("q4_k", self.ff, self.ff.data_ptr() + 4 * FF, 2 * FF, L["down"], self.ffn_out, M,
                                  D, FF)
            else:
                cri.silu_mul(self.ff, self.ff.data_ptr() + 4 * FF, self.act, M * FF)  # M = 1
                cri.matmul("q4_k", self.act, L["down"], self.ffn_out, M, D, FF)
            res = self.ffn_out
        if fused:
            cri.matmul_rmsnorm("q6_k", self.hid[cur], res, self.norm_w[-1], None, self.lm_head, self.logits, M,
                               self.VOCAB, D, eps)
        else:
            norm_then(self.norm_w[-1], self.lm_head, self.logits, self.VOCAB, fmt="q6_k")

    def time(self, reps=20, warmup=3):
        import torch

        for _ in range(warmup):
            self.graph.replay()
        torch.cuda.synchronize()
        start = torch.cuda.Event(enable_timing=True)
        end = torch.cuda.Event(enable_timing=True)
        start.record()
        for _ in range(reps):
            self.graph.replay()
        end.record()
        torch.cuda.synchronize()
        return start.elapsed_time(end) / reps

    def free(self):
        self.layers = self.lm_head = self.kT = self.vc = self.graph = None


class AttentionRig:
    """Fused decode attention of one token (32 query heads over 8 KV heads,
    head_dim 64) over an fp32 cache of T positions in the [T, 8, 64] layout, for
    `copies` distinct caches (>= 2 x the MALL) captured in one graph and replayed.
    form 'plain' is cri_fused_decode_attention (reference signature), 'ws' its
    split form with a workspace."""

    H, HKV, HD = 32, 8, 64

    def __init__(self, form, T=2048, min_bytes=2 * MALL_BYTES):
        import torch

        import cretif_amd as cri

        H, HKV, HD = self.H, self.HKV, self.HD
        self.T, self.form = T, form
        cache = T * HKV * HD * 4
        self.copies = int(max(2, -(-min_bytes // (2 * cache))))
        g = torch.Generator(device="cuda").manual_seed(3000)
        self.K = [torch.randn(T, HKV, HD, device="cuda", generator=g) for _ in range(self.copies)]
        self.V = [torch.randn(T, HKV, HD, device="cuda", generator=g) for _ in range(self.copies)]
        self.q = torch.randn(H * HD, device="cuda", generator=g)
        self.out = torch.empty(H * HD, device="cuda")
        self.ws = torch.empty(max(4, cri.decode_attention_workspace_size(H, HKV, HD, T) // 4), device="cuda")

        def run():
            for k, v in zip(self.K, self.V):
                if form == "plain":
                    cri.fused_decode_attention(self.q, k, v, self.out, H, HKV, HD, T, 0.125)
                else:
                    cri.fused_decode_attention_ws(self.q, k, v, self.out, H, HKV, HD, T, 0.125, self.ws)

        side = torch.cuda.Stream()
        with torch.cuda.stream(side):
            run()
        side.synchronize()
        self.graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(self.graph, stream=side):
            run()
        torch.cuda.synchronize()

    def bytes_per_call(self):
        # algorithmic: q, out and every K and V value of the T positions, once
        return 4 * (2 * self.H * self.HD + 2 * self.T * self.HKV * self.HD)

    def time(self, reps=20):
        """ms per call."""
        import torch

        self.graph.replay()
        torch.cuda.synchronize()
        start = torch.cuda.Event(enable_timing=True)
        end = torch.cuda.Event(enable_timing=True)
        start.record()
        for _ in range(reps):
            self.graph.replay()
        end.record()
        torch.cuda.synchronize()
        return start.elapsed_time(end) / (reps * self.copies)

    def free(self):
        self.K = self.V = self.graph = None


class GqaRig:
    """batched_matmul_gqa (32 query heads over 8 KV heads, head_dim 64, T = 2048):
    'qk' is Q K^T (A [32, M, 64], B [8, 64, T]), 'pv' is P V (A [32, M, T],
    B [8, T, 64]).  Both operands rotate over `copies` distinct buffers (>= 2 x
    the MALL) in one captured graph.  Algorithmic bytes: 4 (H M K + Hkv K N + H M N)."""

    H, HKV, HD, T = 32, 8, 64, 2048

    def __init__(self, product, M, min_bytes=2 * MALL_BYTES):
        import torch

        import cretif_amd as cri

        H, HKV = self.H, self.HKV
        self.M = M
        self.K, self.N = (self.HD, self.T) if product == "qk" else (self.T, self.HD)
        K, N = self.K, self.N
        per = 4 * (H * M * K + HKV * K * N)
        self.copies = int(max(2, min(256, -(-min_bytes // per))))
        g = torch.Generator(device="cuda").manual_seed(3000 + M)
        self.A = [torch.randn(H, M, K, device="cuda", generator=g) for _ in range(self.copies)]
        self.B = [torch.randn(HKV, K, N, device="cuda", generator=g) for _ in range(self.copies)]
        self.C = torch.empty(H, M, N, device="cuda")

        def run():
            for a_, b_ in zip(self.A, self.B):
                cri.batched_matmul_gqa(a_, b_, self.C, H, HKV, M, N, K)

        side = torch.cuda.Stream()
        with torch.cuda.stream(side):
            run()
        side.synchronize()
        self.graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(self.graph, stream=side):
            run()
        torch.cuda.synchronize()

    def bytes_per_call(self):
        return 4 * (self.H * self.M * self.K + self.HKV * self.K * self.N + self.H * self.M * self.N)

    time = AttentionRig.time

    def free(self):
        self.A = self.B = self.graph = None


def measured_traffic(workload):
    """HBM bytes per launch from the committed rocprofv3 --pmc summary of this
    workload (profiles/<kernel>_<shape>.md, line `traffic_bytes_per_launch:`), or None."""
    import glob
    import re

    fmt, N, K = GEMV_WORKLOADS[workload]
    for path in glob.glob(os.path.join(ROOT, "profiles", "*%s_gemv_%dx%d*.md" % (fmt.replace("_", ""), N, K))):
        m = re.search(r"^traffic_bytes_per_launch:\s*(\d+)", open(path).read(), re.M)
        if m:
            return int(m.group(1))
    return None


def cpu_baseline(fmt, N, K, budget_s=12.0):
    """The reference's CPU path (dequant + sequential fp32 matmul, restated in
    oracle/oracle.c) on this host, single-threaded, on a bounded sample."""
    import oracle as orc
    from cretif_amd import quant

    rows = min(N, 2048)
    w = quant.synthetic_weights(fmt, rows, K, seed=7)
    x = quant.randn(K, seed=8).reshape(1, K)
    orc.matmul_quant(fmt, x, w, rows, K)  # warm
    t0 = time.perf_counter()
    calls = []
    while True:
        t = time.perf_counter()
        orc.matmul_quant(fmt, x, w, rows, K)
        calls.append(time.perf_counter() - t)
        el = time.perf_counter() - t0
        if el >= budget_s and len(calls) >= 5:
            break
    per_call = float(np.median(calls))  # median of the calls, as the reference's benchmarks report
    gbs = algo_bytes(fmt, 1, rows, K) / per_call / 1e9
    return {
        "value": round(gbs, 3),
        "unit": "GB/s",
        "cores": 1,
        "kind": "port",
        "sample": "%s GEMV M=1, %d of %d rows x K=%d, median of %d calls over %.1f s (oracle/oracle.c, gcc -O2 "
        "-ffp-contract=off, 1 thread; host %s, %d logical CPUs visible)" % (
            fmt, rows, N, K, len(calls), el, cpu_model(), os.cpu_count() or 0),
    }


def cpu_model():
    """The host CPU's model name (from /proc/cpuinfo), else the platform's machine string."""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or platform.machine()


def main():
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=12800)
    ap.add_argument("--warmup", type=int, default=640)
    ap.add_argument("--workload", default="q4_k_gemv", choices=sorted(GEMV_WORKLOADS))
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--no-details", action="store_true", help="skip the per-format side measurements")
    ap.add_argument("--prefill", default=None, choices=sorted(PREFILL_WORKLOADS),
                    help="only time one prefill GEMM workload (for profiling) and print its figures")
    ap.add_argument("--decode-step", type=int, default=None, metavar="M",
                    help="only time the synthetic decode step for M tokens (for profiling)")
    ap.add_argument("--step-attention", default="gqa", choices=["gqa", "fused"],
                    help="attention of --decode-step: the two GQA products (default) or the fused kernel (M = 1)")
    ap.add_argument("--step-elementwise", default="none", choices=["none", "separate", "fused"],
                    help="--decode-step with the layer's RMSNorm / SiLU work: separate launches or fused prologues")
    ap.add_argument("--attention", default=None, choices=["plain", "ws"],
                    help="only time the fused decode attention at 2048 positions (for profiling)")
    ap.add_argument("--launch-floor", action="store_true",
                    help="only time the headline kernel on a one-tile problem (Q4_K, 16 x 256) in the same graph "
                         "rig: the per-launch cost with no data to stream, with and without a profiler")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="only run ten 64 MiB device copies (known bytes, for scaling rocprofv3 FETCH_SIZE/WRITE_SIZE)")
    args = ap.parse_args()

    if args.copy_calibration:
        import torch

        a = torch.empty(64 << 20, dtype=torch.uint8, device="cuda").fill_(1)
        b = torch.empty_like(a)
        for _ in range(10):
            b.copy_(a)
        torch.cuda.synchronize()
        print("copied 10 x %d bytes" % a.numel())
        return

    if args.gpus != 1:
        print("bench.py measures one GPU only: this build has no multi-GPU path (the kernels shard by "
              "output rows without communication). Run with --gpus 1.", file=sys.stderr)
        sys.exit(2)

    import torch

    import cretif_amd as cri

    cri.lib()
    if args.launch_floor:
        r = GemvRig("q4_k", 16, 256, M=1, max_copies=57)
        ms, n = r.time(args.steps, args.warmup)
        print(json.dumps({"workload": "launch_floor q4_k 16x256 M=1", "launches": n, "copies": r.copies,
                          "us_per_launch": round(ms * 1e3, 3)}))
        return
    if args.attention:
        r = AttentionRig(args.attention)
        ms_call = r.time(reps=max(3, args.steps // r.copies))
        print(json.dumps({"workload": "decode_attention_" + args.attention, "T": r.T, "calls": r.copies,
                          "us": round(ms_call * 1e3, 3),
                          "GB/s": round(r.bytes_per_call() / (ms_call * 1e-3) / 1e9, 1)}))
        return
    if args.decode_step:
        r = DecodeStepRig(args.decode_step, attention=args.step_attention, elementwise=args.step_elementwise)
        ms_step = r.time(reps=max(3, args.steps // 1000))
        print(json.dumps({"workload": "decode_step", "M": args.decode_step, "attention": args.step_attention,
                          "elementwise": args.step_elementwise,
                          "ms_per_step": round(ms_step, 4),
                          "tokens/s": round(args.decode_step / (ms_step * 1e-3), 1)}))
        return
    if args.prefill:
        f, m_, n, k = PREFILL_WORKLOADS[args.prefill]
        r = GemvRig(f, n, k, M=m_, max_copies=16)
        m, launches = r.time(max(args.steps // 100, 2 * r.copies), 16)
        print(json.dumps({"workload": args.prefill, "M": m_, "N": n, "K": k, "launches": launches,
                          "us": round(m * 1e3, 3), "TFLOP/s": round(2.0 * m_ * n * k / (m * 1e-3) / 1e12, 1)}))
        return
    fmt, N, K = GEMV_WORKLOADS[args.workload]
    rig = GemvRig(fmt, N, K)
    ms, launches = rig.time(args.steps, args.warmup)
    bpl = rig.bytes_per_launch()
    gbs = bpl / (ms * 1e-3) / 1e9
    copies = rig.copies
    rig.free()
    torch.cuda.empty_cache()

    details = {}
    if not args.no_details:
        # achievable line: a bare 16-byte streaming read of the headline's weight bytes and of the
        # Q6_K lm_head's (one launch each, same rig)
        for name, nb in (("stream_read_9.4MB", 9437184), ("stream_read_215MB", 215470080)):
            r = StreamRig(nb)
            m, _ = r.time(max(640, 4 * r.copies), 64)
            details[name] = {"GB/s": round(nb / (m * 1e-3) / 1e9, 1), "us": round(m * 1e3, 3), "copies": r.copies}
            r.free()
            torch.cuda.empty_cache()
        for name, (f, n, k) in GEMV_WORKLOADS.items():
            if name == args.workload:
                continue
            r = GemvRig(f, n, k, max_copies=64)
            m, _ = r.time(max(640, 4 * r.copies), 64)
            details[name] = {"GB/s": round(r.bytes_per_launch() / (m * 1e-3) / 1e9, 1), "us": round(m * 1e3, 3),
                             "copies": r.copies}
            r.free()
            torch.cuda.empty_cache()
        # batched decode (BASELINE config 5 at M = 16): reported against the HBM and the fp16 MFMA roofs
        for name, (f, m_, n, k) in (("q4_k_gemv_m16", ("q4_k", 16, 8192, 2048)),
                                    ("q4_k_gemv_down_m16", ("q4_k", 16, 2048, 8192))):
            r = GemvRig(f, n, k, M=m_, max_copies=64)
            m, _ = r.time(max(640, 4 * r.copies), 64)
            details[name] = {"GB/s": round(r.bytes_per_launch() / (m * 1e-3) / 1e9, 1),
                             "TFLOP/s": round(2.0 * m_ * n * k / (m * 1e-3) / 1e12, 2), "us": round(m * 1e3, 3),
                             "M": m_, "copies": r.copies}
            r.free()
            torch.cuda.empty_cache()
        for name, (f, m_, n, k) in PREFILL_WORKLOADS.items():
            r = GemvRig(f, n, k, M=m_, max_copies=16)
            m, _ = r.time(max(64, 2 * r.copies), 16)
            details[name] = {"TFLOP/s": round(2.0 * m_ * n * k / (m * 1e-3) / 1e12, 1), "us": round(m * 1e3, 3),
                             "M": m_, "copies": r.copies, "fraction_of_fp16_mfma_peak": round(
                                 2.0 * m_ * n * k / (m * 1e-3) / 1e12 / FP16_MFMA_PEAK_TFLOPS, 4)}
            r.free()
            torch.cuda.empty_cache()
        for form in ("plain", "ws"):
            r = AttentionRig(form)
            ms_call = r.time()
            details["decode_attention_%s_T2048" % form] = {
                "us": round(ms_call * 1e3, 3), "GB/s": round(r.bytes_per_call() / (ms_call * 1e-3) / 1e9, 1),
                "copies": r.copies}
            r.free()
            torch.cuda.empty_cache()
        for product in ("qk", "pv"):
            for m_ in (1, 16):
                r = GqaRig(product, m_)
                ms_call = r.time()
                details["gqa_%s_m%d_T2048" % (product, m_)] = {
                    "us": round(ms_call * 1e3, 3), "GB/s": round(r.bytes_per_call() / (ms_call * 1e-3) / 1e9, 1),
                    "copies": r.copies}
                r.free()
                torch.cuda.empty_cache()
        for m_, attn, ew in ((1, "gqa", "none"), (16, "gqa", "none"), (1, "fused", "none"), (1, "fused", "separate"),
                             (1, "fused", "fused"), (16, "gqa", "fused")):
            r = DecodeStepRig(m_, attention=attn, elementwise=ew)
            ms_step = r.time()
            key = "decode_step_m%d" % m_ + ("_fused_attention" if attn == "fused" else "") + (
                "" if ew == "none" else "_norms_" + ew)
            details[key] = {
                "tokens/s": round(m_ / (ms_step * 1e-3), 1), "ms_per_step": round(ms_step, 4),
                "weight_GB/s": round(r.weight_bytes / (ms_step * 1e-3) / 1e9, 1),
                "weight+kv_GB/s": round((r.weight_bytes + r.kv_bytes) / (ms_step * 1e-3) / 1e9, 1)}
            r.free()
            torch.cuda.empty_cache()

    line = {
        "metric": "weight GB/s (% of HBM peak) for Q4_K/Q8_0 decode GEMV; prefill GEMM TFLOP/s",
        "value": round(gbs, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": launches,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp32",
        "data": "synthetic: w ~ N(0, 0.02) quantised to %s, x ~ N(0, 1)" % fmt,
        "config": {"workload": "%s decode GEMV M=1" % fmt.upper(), "N": N, "K": K, "M": 1,
                   "weight_copies": copies, "rotation_bytes": copies * (bpl - 4 * K - 4 * N),
                   "timing": "HIP graph of %d launches replayed; hipEvents on the replay stream" % copies},
        "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": measured_traffic(args.workload)},
    }
    if not args.no_cpu:
        line["cpu_baseline"] = cpu_baseline(fmt, N, K)
    if details:
        line["details"] = details
    print(json.dumps(line))


if __name__ == "__main__":
    main()
