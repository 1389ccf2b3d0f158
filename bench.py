#!/usr/bin/env python3
"""Benchmark of the fused dequant+matmul path on one MI355X.

Headline (the `value` of the JSON line): weight GB/s of the batch-1 Q4_K
decode GEMV at the Llama-3.2-1B FFN gate/up shape (N=8192, K=2048).  One
"step" is one GEMV launch over one batch of synthetic input.  The weights are
rotated over enough distinct copies (>= 2x the 256 MB Infinity Cache) that each
launch streams its matrix from HBM; the launches are captured in one HIP graph
with a device timestamp kernel between samples (so no graph boundary falls
inside a sample), and the timed replay is bracketed by HIP events on the replay
stream plus device synchronisation.  Every line in `details` is timed the same
way.

GB/s counts algorithmic bytes only: N*(K/bs)*block_bytes + 4*M*K + 4*M*N.

    python bench.py [--steps K] [--warmup W] [--samples S] [--workload NAME] [--no-cpu] [--no-details]

A timed sample is exactly K launches (--steps); S samples (>= 5) are taken back to
back and the median sample gives `value` and `ms_per_step`.
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
    "q6_k_prefill": ("q6_k", 512, 8192, 2048),
    "q6_k_prefill_down": ("q6_k", 512, 2048, 8192),
    "q4_0_prefill": ("q4_0", 512, 8192, 2048),
    "q4_0_prefill_down": ("q4_0", 512, 2048, 8192),
    "q5_0_prefill": ("q5_0", 512, 8192, 2048),
    "q5_0_prefill_down": ("q5_0", 512, 2048, 8192),
    # FP16 on the register-decode kernel, copied per step with global_load_lds
    "fp16_prefill": ("fp16", 512, 8192, 2048),
    # through cri_matmul_ws: the down shape's K split (four ways, 64 output tiles) stores its
    # partial sums in the workspace and a second launch adds them in order, instead of fp32
    # atomics into a zero-filled C
    "q4_k_prefill_down_ws": ("q4_k", 512, 2048, 8192),
    "q8_0_prefill_down_ws": ("q8_0", 512, 2048, 8192),
}

# batched decode GEMVs (BASELINE config 5 at M = 16): name -> (fmt, M, N, K)
SKINNY_WORKLOADS = {
    "q4_k_gemv_m16": ("q4_k", 16, 8192, 2048),
    "q4_k_gemv_down_m16": ("q4_k", 16, 2048, 8192),
    # the same through cri_matmul_ws: the K split's partial sums added in a fixed order (the same
    # bits every call) instead of with atomics
    "q4_k_gemv_m16_ws": ("q4_k", 16, 8192, 2048),
    "q4_k_gemv_down_m16_ws": ("q4_k", 16, 2048, 8192),
    # the tied fp32 LM head at decode batch 16 (matmul_transposed_b, ref:src/embedding.cu:85-135)
    "fp32_tied_lm_head_m16": ("fp32", 16, 128256, 2048),
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
    # the other BASELINE GEMV shapes: config 1 (SmolLM2-135M FFN up), config 2 (FFN down),
    # config 3 (q/o and k/v projections)
    "q8_0_gemv_1536x576": ("q8_0", 1536, 576),
    "q4_0_gemv_down": ("q4_0", 2048, 8192),
    "q5_0_gemv_down": ("q5_0", 2048, 8192),
    "q4_k_gemv_2048x2048": ("q4_k", 2048, 2048),
    "q4_k_gemv_512x2048": ("q4_k", 512, 2048),
    "q6_k_gemv_512x2048": ("q6_k", 512, 2048),
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


def rotation_plan(steps, need, max_nodes=20000):
    """(copies, graphs, continuous): `graphs` graphs of exactly `steps` launches each, graph
    r using weight copies (r * steps + i) % copies, so that replaying them in turn walks one
    continuous rotation over >= `need` copies and no launch finds its weights in the
    Infinity Cache.  Falls back to one graph whose rotation restarts every sample when a
    continuous plan would need more than max_nodes launches."""
    import math

    if steps <= need:
        copies = -(-need // steps) * steps
        return copies, copies // steps, True
    for c in range(need, 2 * need + 1):
        if steps % c == 0:
            return c, 1, True
    graphs = need // math.gcd(need, steps)
    if graphs * steps <= max_nodes:
        return need, graphs, True
    return need, 1, False


def time_graphs(graphs, samples, warmup_steps, steps, stream):
    """ms of each of `samples` consecutive graph replays (graphs taken in turn), after
    ceil(warmup_steps / steps) untimed replays; HIP events on the replay stream between
    the replays, which are all enqueued before the one synchronisation."""
    import torch

    torch.cuda.synchronize()
    gi = 0
    for _ in range(max(1, -(-warmup_steps // steps))):
        graphs[gi % len(graphs)].replay()
        gi += 1
    torch.cuda.synchronize()
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(samples + 1)]
    with torch.cuda.stream(stream):
        ev[0].record(stream)
        for i in range(samples):
            graphs[gi % len(graphs)].replay()
            gi += 1
            ev[i + 1].record(stream)
    torch.cuda.synchronize()
    return [ev[i].elapsed_time(ev[i + 1]) for i in range(samples)]


def chain_samples(call, steps, samples, stream):
    """ms per call of each of `samples` consecutive samples of exactly `steps` calls, all in one
    captured graph with a device timestamp kernel (cri_timestamp, 100 MHz clock) between the
    samples, so no graph boundary falls inside the timed region (each boundary costs ~13 us on
    this box, which a sample of a few large launches would otherwise carry).  call(n) enqueues
    call n of the weight rotation, which continues through the samples.  The graph runs once
    untimed, once timed.  Also returns the hipEvent time of the whole timed replay (ms), which
    brackets the samples."""
    import torch

    import cretif_amd as cri

    ts = torch.zeros(samples + 1, dtype=torch.int64, device="cuda")
    g = torch.cuda.CUDAGraph()
    n = 0
    with torch.cuda.graph(g, stream=stream):
        for i in range(samples):
            cri.timestamp(ts.data_ptr() + 8 * i)
            for _ in range(steps):
                call(n)
                n += 1
        cri.timestamp(ts.data_ptr() + 8 * samples)
    torch.cuda.synchronize()
    g.replay()  # warm-up pass
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    with torch.cuda.stream(stream):
        e0.record(stream)
        g.replay()
        e1.record(stream)
    torch.cuda.synchronize()
    t = ts.cpu().numpy().astype(np.int64)
    per = [(t[i + 1] - t[i]) * 1e-5 / steps for i in range(samples)]  # 100 MHz ticks -> ms per call
    del g
    return per, e0.elapsed_time(e1)


class ChainTimed:
    """time(): warm-up replays of the rig's graphs, then the median of chain_samples.  A rig
    defines call(n), steps, stream and graphs."""

    def samples(self, samples, warmup):
        """ms per call of each sample (one replay = `steps` calls, events between replays)."""
        return [t / self.steps for t in time_graphs(self.graphs, samples, warmup, self.steps, self.stream)]

    def chain_samples(self, samples):
        return chain_samples(self.call, self.steps, samples, self.stream)

    def time(self, samples=9, warmup=64):
        """Median ms per call over `samples` samples of `steps` calls each."""
        self.samples(1, warmup)  # untimed warm-up
        return float(np.median(self.chain_samples(samples)[0]))


class GemvRig(ChainTimed):
    """Weights replicated over enough device copies that each launch streams from HBM;
    `steps` launches per captured graph (see rotation_plan)."""

    def __init__(self, fmt, N, K, M=1, seed=1, min_bytes=2 * MALL_BYTES, max_copies=64, steps=None,
                 workspace=False):
        import torch

        import cretif_amd as cri
        from cretif_amd import quant

        self.fmt, self.N, self.K, self.M = fmt, N, K, M
        w = tiled_weights(fmt, N, K, seed=seed) if fmt != "fp32" else \
            quant.randn(N * K, seed=seed).astype(np.float32).view(np.uint8)
        self.wbytes = w.size
        need = int(max(1, min(max_copies, -(-min_bytes // w.size))))
        self.steps = steps or need
        self.copies, ngraphs, self.continuous = rotation_plan(self.steps, need)
        base = torch.from_numpy(w).cuda()
        self.W = [base] + [base.clone() for _ in range(self.copies - 1)]
        self.x = torch.from_numpy(quant.randn(M * K, seed=seed + 1).reshape(M, K)).cuda()
        self.y = torch.empty(M, N, device="cuda")
        self.cri = cri
        wsb = cri.matmul_workspace_bytes(fmt, M, N, K) if workspace else 0
        self.ws = torch.empty(max(1, wsb // 4), dtype=torch.float32, device="cuda") if wsb else None
        torch.cuda.synchronize()
        self.stream = torch.cuda.Stream()

        def run(Wi):
            if fmt == "fp32":
                cri.matmul_transposed_b(self.x, Wi, self.y, M, N, K)
            elif self.ws is not None:
                cri.matmul_ws(fmt, self.x, Wi, self.y, M, N, K, self.ws)
            else:
                cri.matmul(fmt, self.x, Wi, self.y, M, N, K)

        self._run = run
        with torch.cuda.stream(self.stream):
            for Wi in self.W:  # eager warm-up on the side stream
                run(Wi)
        self.stream.synchronize()
        self.graphs = []
        for r in range(ngraphs):
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g, stream=self.stream):
                for i in range(self.steps):
                    run(self.W[(r * self.steps + i) % self.copies])
            self.graphs.append(g)
        torch.cuda.synchronize()

    def bytes_per_launch(self):
        return algo_bytes(self.fmt, self.M, self.N, self.K)

    def call(self, n):
        self._run(self.W[n % self.copies])

    def free(self):
        self.W = None
        self.graphs = None


class StreamRig(ChainTimed):
    """The achievable streaming-read line: cri_stream_read_ex over `copies` buffers of n_bytes
    (rotated over >= 2x the Infinity Cache, as the GEMVs) in the shape the read sweep found
    fastest at the headline's size: one 16-byte load per thread, one pass of the buffer."""

    def __init__(self, n_bytes, min_bytes=2 * MALL_BYTES, max_copies=64):
        import torch

        import cretif_amd as cri

        self.n_bytes = n_bytes
        self.copies = self.steps = int(max(1, min(max_copies, -(-min_bytes // n_bytes))))
        base = torch.zeros(n_bytes, dtype=torch.uint8, device="cuda")
        self.W = [base] + [base.clone() for _ in range(self.copies - 1)]
        self.sink = torch.zeros(1, dtype=torch.int32, device="cuda")
        self.stream = torch.cuda.Stream()
        self.cri = cri
        with torch.cuda.stream(self.stream):
            for n in range(self.copies):
                self.call(n)
        self.stream.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=self.stream):
            for n in range(self.copies):
                self.call(n)
        self.graphs = [g]
        torch.cuda.synchronize()

    def call(self, n):
        self.cri.stream_read_ex(self.W[n % self.copies], self.n_bytes, self.sink, 1, 0)

    def free(self):
        self.W = None
        self.graphs = None


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


def hip_memcpy(dst, src, nbytes, kind):
    """hipMemcpy through the HIP runtime torch loaded (kind 1: host to device, 3: device to device)."""
    import ctypes

    path = next(ln.split()[-1] for ln in open("/proc/self/maps") if "libamdhip64" in ln)
    h = ctypes.CDLL(path)
    h.hipMemcpy.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int]
    if h.hipMemcpy(dst, src, nbytes, kind) != 0:
        raise RuntimeError("hipMemcpy failed")


class VendorGemmRig(ChainTimed):
    """A point of comparison, not part of the library: torch.mm on fp16 operands with fp32
    output (hipBLASLt on this image, its default heuristic) at a prefill workload's shape,
    C[M, N] = A[M, K] B[N, K]^T -- the vendor library's plain fp16 GEMM with the weights
    already fp16, so no dequantization and no activation conversion.  The weights rotate over
    `copies` device copies in one captured graph, like the prefill rig's."""

    def __init__(self, M, N, K, copies=16):
        import torch

        g = torch.Generator(device="cuda").manual_seed(4000)
        self.A = torch.randn(M, K, device="cuda", dtype=torch.float16, generator=g)
        self.W = [(torch.randn(N, K, device="cuda", dtype=torch.float16, generator=g) * 0.02) for _ in range(copies)]
        self.steps = copies

        def call(n):
            torch.mm(self.A, self.W[n % copies].t(), out_dtype=torch.float32)

        def run():
            for n in range(copies):
                call(n)

        self.call = call
        self.stream = torch.cuda.Stream()
        with torch.cuda.stream(self.stream):
            run()
        self.stream.synchronize()
        gr = torch.cuda.CUDAGraph()
        with torch.cuda.graph(gr, stream=self.stream):
            run()
        self.graphs = [gr]
        torch.cuda.synchronize()


class DecodeStepRig:
    """BASELINE config 5 through the product decode step (cri_decoder_*, C++
    cuinfer::DecodeStep): a synthetic Llama-3.2-1B -- 16 layers of Q4_K q (2048x2048),
    k and v (512x2048), o (2048x2048), gate and up (8192x2048), down (2048x8192), RMSNorm
    weights ~ 1 + N(0, 0.1), a Q8_0 token table and a Q6_K 128256x2048 LM head --
    with an fp32 KV cache ~ N(0, 1) filled to 2048 positions.  One step is M tokens:
    embedding, per layer RMSNorm + q/k/v (one stacked matrix), RoPE + cache append,
    attention over the cache (32 query heads over 8 KV heads, head_dim 64), o,
    residual + RMSNorm + gate/up (one stacked matrix), SiLU * up + down, then the final
    RMSNorm, the LM head and the greedy token of each row, values chained throughout;
    captured once as a HIP graph.  Each timed replay runs at position 2048 - M (the last
    row sees all 2048 positions); the position is reset by a kernel outside the timed
    events.  Every layer has its own weight copy (the same bytes: weights are N(0, 0.02)
    rows quantized once and tiled)."""

    LAYERS, D, H, HKV, HD, FF, VOCAB, T = 16, 2048, 32, 8, 64, 8192, 128256, 2048

    def __init__(self, M, seed=1100, capture=True):
        import torch

        import cretif_amd as cri

        D, FF, H, HKV, HD, V, T = self.D, self.FF, self.H, self.HKV, self.HD, self.VOCAB, self.T
        self.M = M
        shapes = {"q": (H * HD, D), "k": (HKV * HD, D), "v": (HKV * HD, D), "o": (D, H * HD), "gate": (FF, D),
                  "up": (FF, D), "down": (D, FF)}
        w = {n: ("q4_k", tiled_weights("q4_k", r, c, seed + i)) for i, (n, (r, c)) in enumerate(shapes.items())}
        rng = np.random.default_rng(seed)
        self.dec = dec = cri.Decoder(self.LAYERS, D, H, HKV, HD, FF, V, T, max_batch=max(16, M),
                                     rope_theta=500000.0)
        for li in range(self.LAYERS):
            dec.set_layer(li, (1 + 0.1 * rng.standard_normal(D)).astype(np.float32),
                          (1 + 0.1 * rng.standard_normal(D)).astype(np.float32), **w)
        dec.set_embedding("q8_0", tiled_weights("q8_0", V, D, seed + 98))
        dec.set_output((1 + 0.1 * rng.standard_normal(D)).astype(np.float32),
                       ("q6_k", tiled_weights("q6_k", V, D, seed + 99)))
        g = torch.Generator(device="cuda").manual_seed(3000)
        for li in range(self.LAYERS):
            ka, va = dec.kv_cache(li)
            for addr in (ka, va):
                t = torch.randn(T * HKV * HD, device="cuda", generator=g)
                torch.cuda.synchronize()
                hip_memcpy(addr, t.data_ptr(), t.numel() * 4, 3)
        # the bytes one step reads: every layer's weights and norms, the LM head and the M token rows
        # (not the whole token table, which the step only gathers from)
        self.weight_bytes = dec.step_weight_bytes(M)
        self.kv_bytes = 2 * self.LAYERS * T * HKV * HD * 4
        self.ids = torch.from_numpy(rng.integers(0, V, M).astype(np.int32)).cuda()
        self.logits = torch.empty(M, V, device="cuda")
        self.next_ids = torch.empty(M, dtype=torch.int32, device="cuda")
        self.stream = torch.cuda.Stream()
        self.pos0 = T - M
        torch.cuda.synchronize()
        if capture:
            dec.capture(self.ids, M, self.logits, self.next_ids, stream=self.stream)

    def prompt_samples(self, samples=5, warmup=1, last_only=False):
        """ms of each of `samples` eager steps of the M tokens at position 0 (a prompt into an empty
        cache: the attention spans only the positions the prompt sees).  last_only: cri_decoder_prefill,
        the LM head and argmax of the last token only (what the reference's generate() reads)."""
        import torch

        s = self.stream
        ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(samples)]
        for i in range(warmup + samples):
            self.dec.set_position(0, stream=s)
            if i >= warmup:
                ev[i - warmup][0].record(s)
            if last_only:
                self.dec.prefill(self.ids, self.M, self.logits, self.next_ids, stream=s)
            else:
                self.dec.forward(self.ids, self.M, self.logits, self.next_ids, stream=s)
            if i >= warmup:
                ev[i - warmup][1].record(s)
        torch.cuda.synchronize()
        return [a.elapsed_time(b) for a, b in ev]

    def samples(self, samples=9, warmup=3):
        """ms of each of `samples` replays at position 2048 - M."""
        import torch

        s = self.stream
        for _ in range(warmup):
            self.dec.set_position(self.pos0, stream=s)
            self.dec.replay(stream=s)
        torch.cuda.synchronize()
        ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(samples)]
        for a, b in ev:
            self.dec.set_position(self.pos0, stream=s)
            a.record(s)
            self.dec.replay(stream=s)
            b.record(s)
        torch.cuda.synchronize()
        return [a.elapsed_time(b) for a, b in ev]

    def time(self, samples=9, warmup=3):
        return float(np.median(self.samples(samples, warmup)))

    def free(self):
        self.dec.close()
        self.dec = None


class AttentionRig(ChainTimed):
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

        def call(n):
            k, v = self.K[n % self.copies], self.V[n % self.copies]
            if form == "plain":
                cri.fused_decode_attention(self.q, k, v, self.out, H, HKV, HD, T, 0.125)
            else:
                cri.fused_decode_attention_ws(self.q, k, v, self.out, H, HKV, HD, T, 0.125, self.ws)

        def run():
            for n in range(self.copies):
                call(n)

        self.call = call

        self.stream = torch.cuda.Stream()
        with torch.cuda.stream(self.stream):
            run()
        self.stream.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=self.stream):
            run()
        self.graphs, self.steps = [g], self.copies
        torch.cuda.synchronize()

    def bytes_per_call(self):
        # algorithmic: q, out and every K and V value of the T positions, once
        return 4 * (2 * self.H * self.HD + 2 * self.T * self.HKV * self.HD)

    def free(self):
        self.K = self.V = self.graphs = None


class GqaRig(ChainTimed):
    """batched_matmul_gqa (32 query heads over 8 KV heads, head_dim 64, T keys):
    'qk' is Q K^T (A [32, M, 64], B [8, 64, T]), 'pv' is P V (A [32, M, T],
    B [8, T, 64]).  Both operands rotate over `copies` distinct buffers (>= 2 x
    the MALL) in one captured graph.  Algorithmic bytes: 4 (H M K + Hkv K N + H M N);
    flops 2 H M K N."""

    H, HKV, HD = 32, 8, 64

    def __init__(self, product, M, T=2048, min_bytes=2 * MALL_BYTES):
        import torch

        import cretif_amd as cri

        H, HKV = self.H, self.HKV
        self.M = M
        self.T = T
        self.K, self.N = (self.HD, T) if product == "qk" else (T, self.HD)
        K, N = self.K, self.N
        per = 4 * (H * M * K + HKV * K * N)
        self.copies = int(max(2, min(256, -(-min_bytes // per))))
        g = torch.Generator(device="cuda").manual_seed(3000 + M)
        self.A = [torch.randn(H, M, K, device="cuda", generator=g) for _ in range(self.copies)]
        self.B = [torch.randn(HKV, K, N, device="cuda", generator=g) for _ in range(self.copies)]
        self.C = torch.empty(H, M, N, device="cuda")

        def call(n):
            cri.batched_matmul_gqa(self.A[n % self.copies], self.B[n % self.copies], self.C, H, HKV, M, N, K)

        def run():
            for n in range(self.copies):
                call(n)

        self.call = call

        self.stream = torch.cuda.Stream()
        with torch.cuda.stream(self.stream):
            run()
        self.stream.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=self.stream):
            run()
        self.graphs, self.steps = [g], self.copies
        torch.cuda.synchronize()

    def bytes_per_call(self):
        return 4 * (self.H * self.M * self.K + self.HKV * self.K * self.N + self.H * self.M * self.N)

    def flops_per_call(self):
        return 2.0 * self.H * self.M * self.K * self.N

    def free(self):
        self.A = self.B = self.graphs = None


def read_probe_us(nb, per, grid, samples=7):
    """us per launch of cri_stream_read_ex over nb bytes (per 16-byte loads per thread, issued
    before any is used; grid 0 = one-shot, one pass of the buffer, else that many workgroups
    striding over it), the buffers rotated over >= 2x the Infinity Cache (chain_samples)."""
    import torch

    import cretif_amd as cri

    copies = int(max(2, min(256, -(-2 * MALL_BYTES // nb))))
    base = torch.zeros(nb, dtype=torch.uint8, device="cuda")
    W = [base] + [base.clone() for _ in range(copies - 1)]
    sink = torch.zeros(1, dtype=torch.int32, device="cuda")
    s = torch.cuda.Stream()
    with torch.cuda.stream(s):
        for w in W:
            cri.stream_read_ex(w, nb, sink, per, grid)
    s.synchronize()
    t, _ = chain_samples(lambda n: cri.stream_read_ex(W[n % copies], nb, sink, per, grid), copies, samples, s)
    del W
    torch.cuda.empty_cache()
    return float(np.median(t)) * 1e3


def read_sweep():
    """The achievable read rate at the headline's size, and how it grows with size: one JSON
    line per point, then the best 9.4 MB shape and the fraction of 8 TB/s it reaches."""
    nb, best = 9437184, None
    for per in (1, 2, 4, 8, 16):
        for grid in (0, 256, 512, 1024, 2048, 4096):
            us = read_probe_us(nb, per, grid)
            print(json.dumps({"read_sweep": "9.4MB", "loads_per_thread": per, "grid": grid or "one-shot",
                              "us": round(us, 3), "GB/s": round(nb / us / 1e3, 1)}), flush=True)
            if best is None or us < best[0]:
                best = (us, per, grid)
    us, per, grid = best
    for mb in (0.25, 0.5, 1, 2, 4.7, 9.4, 18.9, 37.7, 75.5, 151, 302, 604):
        n = int(mb * 1e6) // 4096 * 4096
        t = read_probe_us(n, per, grid)
        print(json.dumps({"read_sweep": "size", "MB": mb, "loads_per_thread": per, "grid": grid or "one-shot",
                          "us": round(t, 3), "GB/s": round(n / t / 1e3, 1)}), flush=True)
    print(json.dumps({"read_sweep": "best_9.4MB", "us": round(us, 3), "GB/s": round(nb / us / 1e3, 1),
                      "fraction_of_8TB/s": round(nb / us / 1e3 / 8000, 3),
                      "us_needed_for_70pct": round(nb / (0.7 * 8000) / 1e3, 3)}), flush=True)


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


def cpu_baseline_prefill(fmt, M, N, K, cols=64, budget_s=6.0):
    """The reference's CPU path for a BASELINE config-4 prefill GEMM (M activation rows, weights
    [N, K]) on a column sample: the first `cols` output columns for all M rows, single-threaded,
    median of >= 3 calls (ref:tests/test_matmul_quant.cu:30-41 restated in oracle/oracle.c)."""
    import oracle as orc
    from cretif_amd import quant

    w = quant.synthetic_weights(fmt, cols, K, seed=9)
    x = quant.randn(M * K, seed=10).reshape(M, K)
    calls = []
    t0 = time.perf_counter()
    while True:
        t = time.perf_counter()
        orc.matmul_quant(fmt, x, w, cols, K)
        calls.append(time.perf_counter() - t)
        el = time.perf_counter() - t0
        if el >= budget_s and len(calls) >= 3:
            break
    per_call = float(np.median(calls))
    return {
        "value": round(2.0 * M * cols * K / per_call / 1e9, 3),
        "unit": "GFLOP/s",
        "cores": 1,
        "kind": "port",
        "sample": "%s prefill GEMM M=%d, %d of %d output columns x K=%d, median of %d calls over %.1f s "
        "(oracle/oracle.c, gcc -O2 -ffp-contract=off, 1 thread; host %s)" % (
            fmt, M, cols, N, K, len(calls), el, cpu_model()),
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
    ap.add_argument("--steps", type=int, default=400, help="launches per timed sample of the headline GEMV")
    ap.add_argument("--warmup", type=int, default=400, help="untimed launches before the samples")
    ap.add_argument("--samples", type=int, default=25, help="timed samples (>= 5); the median is reported")
    ap.add_argument("--workload", default="q4_k_gemv", choices=sorted(GEMV_WORKLOADS))
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--no-details", action="store_true", help="skip the per-format side measurements")
    ap.add_argument("--gqa", default=None, help="time one batched_matmul_gqa shape: qk|pv,M,T")
    ap.add_argument("--read-sweep", action="store_true",
                    help="the read probe (cri_stream_read_ex) over loads per thread x grid shapes at the "
                         "headline's 9.4 MB, then the best shape over sizes 0.25 MB .. 604 MB")
    ap.add_argument("--prefill", default=None, choices=sorted(PREFILL_WORKLOADS),
                    help="only time one prefill GEMM workload (for profiling) and print its figures")
    ap.add_argument("--vendor-gemm", default=None, choices=sorted(PREFILL_WORKLOADS),
                    help="only time the vendor library's plain fp16 GEMM (torch.mm, fp32 output) at that prefill "
                         "workload's shape, as a point of comparison for the fused kernels")
    ap.add_argument("--gemv", default=None, choices=sorted(GEMV_WORKLOADS) + sorted(SKINNY_WORKLOADS),
                    help="only time one GEMV workload (for profiling) and print its figures")
    ap.add_argument("--decode-step", type=int, default=None, metavar="M",
                    help="only time the synthetic Llama-3.2-1B decode step for M tokens (for profiling)")
    ap.add_argument("--prompt", type=int, default=None, metavar="M",
                    help="time an M-token prompt (eager steps at position 0) through the 16-layer decode step")
    ap.add_argument("--prompt-last-row", action="store_true",
                    help="with --prompt: cri_decoder_prefill (the LM head of the last token only)")
    ap.add_argument("--attention", default=None, choices=["plain", "ws"],
                    help="only time the fused decode attention at 2048 positions (for profiling)")
    ap.add_argument("--launch-floor", action="store_true",
                    help="only time the headline kernel on a one-tile problem (Q4_K, 16 x 256) in the same graph "
                         "rig: the per-launch cost with no data to stream, with and without a profiler")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="only run ten 64 MiB device copies (known bytes, for scaling rocprofv3 FETCH_SIZE/WRITE_SIZE)")
    args = ap.parse_args()
    # a sample is exactly --steps launches; the timed graph holds samples x steps of them
    samples = max(5, min(args.samples, 40000 // max(1, args.steps)))

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
        ms = r.time(samples, args.warmup)
        print(json.dumps({"workload": "launch_floor q4_k 16x256 M=1", "launches_per_sample": r.steps,
                          "samples": samples, "us_per_launch": round(ms * 1e3, 3)}))
        return
    if args.attention:
        r = AttentionRig(args.attention)
        ms_call = r.time(samples)
        print(json.dumps({"workload": "decode_attention_" + args.attention, "T": r.T, "calls_per_sample": r.copies,
                          "us": round(ms_call * 1e3, 3),
                          "GB/s": round(r.bytes_per_call() / (ms_call * 1e-3) / 1e9, 1)}))
        return
    if args.decode_step:
        r = DecodeStepRig(args.decode_step)
        ms_step = r.time(samples)
        print(json.dumps({"workload": "decode_step", "M": args.decode_step, "ms_per_step": round(ms_step, 4),
                          "tokens/s": round(args.decode_step / (ms_step * 1e-3), 1),
                          "weight_GB/s": round(r.weight_bytes / (ms_step * 1e-3) / 1e9, 1),
                          "weight_frac_of_hbm_peak": round(r.weight_bytes / (ms_step * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)}))
        return
    if args.prompt:
        r = DecodeStepRig(args.prompt, capture=False)
        ms = float(np.median(r.prompt_samples(samples, last_only=args.prompt_last_row)))
        print(json.dumps({"workload": "prompt", "M": args.prompt, "ms_per_prompt": round(ms, 4),
                          "prompt_tokens/s": round(args.prompt / (ms * 1e-3), 1)}))
        return
    if args.read_sweep:
        read_sweep()
        return
    if args.gqa:
        product, m_, t_ = args.gqa.split(",")
        r = GqaRig(product, int(m_), T=int(t_))
        ms_call = r.time(samples)
        print(json.dumps({"workload": "gqa_%s" % product, "M": int(m_), "T": int(t_), "us": round(ms_call * 1e3, 3),
                          "TFLOP/s": round(r.flops_per_call() / (ms_call * 1e-3) / 1e12, 2)}))
        return
    if args.prefill:
        f, m_, n, k = PREFILL_WORKLOADS[args.prefill]
        r = GemvRig(f, n, k, M=m_, max_copies=16, workspace=args.prefill.endswith("_ws"))
        m = r.time(samples, 16)
        print(json.dumps({"workload": args.prefill, "M": m_, "N": n, "K": k, "launches_per_sample": r.steps,
                          "us": round(m * 1e3, 3), "TFLOP/s": round(2.0 * m_ * n * k / (m * 1e-3) / 1e12, 1)}))
        return
    if args.vendor_gemm:
        _, m_, n, k = PREFILL_WORKLOADS[args.vendor_gemm]
        r = VendorGemmRig(m_, n, k)
        m = r.time(samples, 16)
        print(json.dumps({"workload": "vendor_fp16_gemm " + args.vendor_gemm, "M": m_, "N": n, "K": k,
                          "launches_per_sample": r.steps, "us": round(m * 1e3, 3),
                          "TFLOP/s": round(2.0 * m_ * n * k / (m * 1e-3) / 1e12, 1)}))
        return
    if args.gemv:
        if args.gemv in SKINNY_WORKLOADS:
            f, m_, n, k = SKINNY_WORKLOADS[args.gemv]
        else:
            (f, n, k), m_ = GEMV_WORKLOADS[args.gemv], 1
        r = GemvRig(f, n, k, M=m_, max_copies=1024, workspace=args.gemv.endswith("_ws"))
        m = r.time(samples, 64)
        print(json.dumps({"workload": args.gemv, "M": m_, "N": n, "K": k, "launches_per_sample": r.steps,
                          "us": round(m * 1e3, 3), "GB/s": round(r.bytes_per_launch() / (m * 1e-3) / 1e9, 1)}))
        return
    fmt, N, K = GEMV_WORKLOADS[args.workload]
    rig = GemvRig(fmt, N, K, steps=max(1, args.steps))
    rig.samples(1, args.warmup)  # W untimed warm-up launches
    per_launch, event_ms = rig.chain_samples(samples)
    ms_launch = float(np.median(per_launch))
    bpl = rig.bytes_per_launch()
    gbs = bpl / (ms_launch * 1e-3) / 1e9
    copies = rig.copies
    rig.free()
    torch.cuda.empty_cache()

    details = {}
    if not args.no_details:
        def gemv_line(r, m):
            return {"GB/s": round(r.bytes_per_launch() / (m * 1e-3) / 1e9, 1), "us": round(m * 1e3, 3),
                    "copies": r.copies}

        # achievable line: a bare 16-byte streaming read of the headline's weight bytes and of the
        # Q6_K lm_head's (one launch each, same rig)
        for name, nb in (("stream_read_9.4MB", 9437184), ("stream_read_215MB", 215470080)):
            r = StreamRig(nb)
            m = r.time(9, 64)
            details[name] = {"GB/s": round(nb / (m * 1e-3) / 1e9, 1), "us": round(m * 1e3, 3), "copies": r.copies}
            r.free()
            torch.cuda.empty_cache()
        for name, (f, n, k) in GEMV_WORKLOADS.items():
            if name == args.workload:
                continue
            r = GemvRig(f, n, k, max_copies=1024)  # small matrices too rotate over >= 2x the MALL
            details[name] = gemv_line(r, r.time(9, 64))
            r.free()
            torch.cuda.empty_cache()
        # batched decode (BASELINE config 5 at M = 16): reported against the HBM and the fp16 MFMA roofs
        for name, (f, m_, n, k) in SKINNY_WORKLOADS.items():
            r = GemvRig(f, n, k, M=m_, workspace=name.endswith("_ws"))
            m = r.time(9, 64)
            details[name] = dict(gemv_line(r, m), M=m_, **{"TFLOP/s": round(2.0 * m_ * n * k / (m * 1e-3) / 1e12, 2)})
            r.free()
            torch.cuda.empty_cache()
        for name, (f, m_, n, k) in PREFILL_WORKLOADS.items():
            r = GemvRig(f, n, k, M=m_, max_copies=16, workspace=name.endswith("_ws"))
            m = r.time(9, 16)
            tf = 2.0 * m_ * n * k / (m * 1e-3) / 1e12
            details[name] = {"TFLOP/s": round(tf, 1), "us": round(m * 1e3, 3), "M": m_, "copies": r.copies,
                             "fraction_of_fp16_mfma_peak": round(tf / FP16_MFMA_PEAK_TFLOPS, 4)}
            r.free()
            torch.cuda.empty_cache()
        for form in ("plain", "ws"):
            r = AttentionRig(form)
            ms_call = r.time(9)
            details["decode_attention_%s_T2048" % form] = {
                "us": round(ms_call * 1e3, 3), "GB/s": round(r.bytes_per_call() / (ms_call * 1e-3) / 1e9, 1),
                "copies": r.copies}
            r.free()
            torch.cuda.empty_cache()
        for product in ("qk", "pv"):
            for m_ in (1, 16):
                r = GqaRig(product, m_)
                ms_call = r.time(9)
                details["gqa_%s_m%d_T2048" % (product, m_)] = {
                    "us": round(ms_call * 1e3, 3), "GB/s": round(r.bytes_per_call() / (ms_call * 1e-3) / 1e9, 1),
                    "copies": r.copies}
                r.free()
                torch.cuda.empty_cache()
            # prefill: a 512-token prompt attends to itself (ref:src/attention.cu:837-861), fp32 products
            r = GqaRig(product, 512, T=512)
            ms_call = r.time(9)
            details["gqa_%s_m512_T512" % product] = {
                "us": round(ms_call * 1e3, 3), "TFLOP/s": round(r.flops_per_call() / (ms_call * 1e-3) / 1e12, 2),
                "GB/s": round(r.bytes_per_call() / (ms_call * 1e-3) / 1e9, 1), "copies": r.copies}
            r.free()
            torch.cuda.empty_cache()
        for m_ in (1, 16):
            r = DecodeStepRig(m_)
            ms_step = r.time(9)
            details["decode_step_m%d" % m_] = {
                "tokens/s": round(m_ / (ms_step * 1e-3), 1), "ms_per_step": round(ms_step, 4),
                "step_weight_bytes": r.weight_bytes,
                "weight_GB/s": round(r.weight_bytes / (ms_step * 1e-3) / 1e9, 1),
                "weight_frac_of_hbm_peak": round(r.weight_bytes / (ms_step * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
                "weight+kv_GB/s": round((r.weight_bytes + r.kv_bytes) / (ms_step * 1e-3) / 1e9, 1),
                "timing": "median of 9 replays of the captured cri_decoder step at position %d" % r.pos0}
            r.free()
            torch.cuda.empty_cache()
        # a 512-token prompt (BASELINE config 4's M) through the same step: the prefill GEMMs and the
        # reference's prefill attention on batched_matmul_gqa, eager steps at position 0
        r = DecodeStepRig(512, capture=False)
        ms_prompt = float(np.median(r.prompt_samples(5)))
        details["prompt_m512"] = {"prompt_tokens/s": round(512 / (ms_prompt * 1e-3), 1),
                                  "ms_per_prompt": round(ms_prompt, 4),
                                  "timing": "median of 5 eager cri_decoder steps of 512 tokens at position 0"}
        # the same prompt as generate() consumes it (ref:src/model.cu:1063-1078): every layer on the
        # 512 tokens, the LM head and argmax of the last one only (cri_decoder_prefill)
        ms_gen = float(np.median(r.prompt_samples(5, last_only=True)))
        details["prompt_m512_last_row"] = {"prompt_tokens/s": round(512 / (ms_gen * 1e-3), 1),
                                           "ms_per_prompt": round(ms_gen, 4),
                                           "timing": "median of 5 eager cri_decoder_prefill calls of 512 tokens "
                                                     "at position 0"}
        r.free()
        torch.cuda.empty_cache()

    line = {
        "metric": "weight GB/s (% of HBM peak) for Q4_K/Q8_0 decode GEMV; prefill GEMM TFLOP/s",
        "value": round(gbs, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": rig.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_launch, 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp32",
        "data": "synthetic: w ~ N(0, 0.02) quantised to %s, x ~ N(0, 1)" % fmt,
        "config": {"workload": "%s decode GEMV M=1" % fmt.upper(), "N": N, "K": K, "M": 1,
                   "weight_copies": copies, "rotation_bytes": copies * (bpl - 4 * K - 4 * N),
                   "samples": samples,
                   "us_per_launch_min_median_max": [round(min(per_launch) * 1e3, 3), round(ms_launch * 1e3, 3),
                                                    round(max(per_launch) * 1e3, 3)],
                   "event_ms_all_samples": round(event_ms, 4),
                   "timing": "%d back-to-back samples of exactly %d launches in one captured graph, a device "
                             "timestamp (100 MHz clock) between samples; value from the median sample; the "
                             "hipEvents around the whole replay give event_ms_all_samples" % (samples, rig.steps)},
        "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": measured_traffic(args.workload)},
    }
    if not args.no_cpu:
        line["cpu_baseline"] = cpu_baseline(fmt, N, K)
        if not args.no_details:
            # the CPU path for the metric's other half (the Q8_0 GEMV) and for config 4 (prefill), beside
            # the GPU lines in details
            details["cpu_baseline_q8_0_gemv"] = cpu_baseline("q8_0", 8192, 2048, budget_s=6.0)
            details["cpu_baseline_q4_k_prefill"] = cpu_baseline_prefill("q4_k", 512, 8192, 2048)
    if details:
        line["details"] = details
    print(json.dumps(line))


if __name__ == "__main__":
    main()
