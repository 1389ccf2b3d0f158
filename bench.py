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
MALL_BYTES = 256 << 20

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
        w = quant.synthetic_weights(fmt, N, K, seed=seed)
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
        with torch.cuda.stream(side):
            for Wi in self.W:  # eager warm-up on the side stream
                cri.matmul(fmt, self.x, Wi, self.y, M, N, K)
        side.synchronize()
        with torch.cuda.graph(self.graph, stream=side):
            for Wi in self.W:
                cri.matmul(fmt, self.x, Wi, self.y, M, N, K)
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


def measured_traffic(workload):
    """HBM bytes per launch from the committed rocprofv3 --pmc summary of this
    workload (profiles/<kernel>_<shape>.md, line `traffic_bytes_per_launch:`), or None."""
    import glob
    import re

    fmt, N, K = GEMV_WORKLOADS[workload]
    for path in glob.glob(os.path.join(ROOT, "profiles", "*%s*%dx%d*.md" % (fmt.replace("_", ""), N, K))):
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
    n = 0
    while True:
        orc.matmul_quant(fmt, x, w, rows, K)
        n += 1
        el = time.perf_counter() - t0
        if el >= budget_s:
            break
    per_call = el / n
    gbs = algo_bytes(fmt, 1, rows, K) / per_call / 1e9
    return {
        "value": round(gbs, 3),
        "unit": "GB/s",
        "cores": 1,
        "kind": "port",
        "sample": "%s GEMV M=1, %d of %d rows x K=%d, %d calls in %.1f s (oracle/oracle.c, gcc -O2 "
        "-ffp-contract=off, 1 thread, %s)" % (fmt, rows, N, K, n, el, platform.processor() or platform.machine()),
    }


def main():
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=12800)
    ap.add_argument("--warmup", type=int, default=640)
    ap.add_argument("--workload", default="q4_k_gemv", choices=sorted(GEMV_WORKLOADS))
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--no-details", action="store_true", help="skip the per-format side measurements")
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
              "output rows without communication; see DESIGN.md). Run with --gpus 1.", file=sys.stderr)
        sys.exit(2)

    import torch

    import cretif_amd as cri

    cri.lib()
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
        for name, (f, n, k) in GEMV_WORKLOADS.items():
            if name == args.workload:
                continue
            r = GemvRig(f, n, k, max_copies=64)
            m, _ = r.time(max(640, 4 * r.copies), 64)
            details[name] = {"GB/s": round(r.bytes_per_launch() / (m * 1e-3) / 1e9, 1), "us": round(m * 1e3, 3),
                             "copies": r.copies}
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
