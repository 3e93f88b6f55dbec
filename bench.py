"""Benchmark of flock's attention hot path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload NAME]

Prints ONE JSON line on stdout (progress goes to stderr). A step is one pass
of the hot path over one batch of synthetic, HBM-resident input:

  decode32k  (default) Long-context GQA decode, all 28 Qwen3-0.6B layers:
             per layer one fused launch of per-head q/k RMSNorm + RoPE (theta
             1e6) + K/V append at position 32768 + split-K decode attention
             over 32769 keys (16 q / 8 kv heads, d 128, f32).
             value = algorithmic HBM bytes / step time (GB/s).
  prefill2k  Causal prefill of 2048 tokens: fused prologue + K/V write, then
             MFMA flash attention. value = causal flops / step time (TFLOP/s).
  ragged     64 independent sequences, n_keys ~ U[1025, 16385] (seeded),
             ragged decode attention in one launch. value in GB/s.
  chunk32k   64-token chunk at pos0 32768 onto a 32768-key cache, 28 layers:
             prologue + chunked prefill attention. value in TFLOP/s.
  decode512  One layer, 513 keys (fits in the 256 MB MALL: "effective" GB/s).

The default run also measures prefill2k (the metric's second half) and reports
it under "prefill". Inputs are N(0, 1) from a seeded generator (gains
N(1, 0.1)); the K/V caches are written on the device before timing starts.
"""
from __future__ import annotations

import argparse
import json
import os
import re
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "decode-attn HBM GB/s (% peak) @32k ctx; prefill-attn TFLOP/s (% MFMA peak) @2k"
HBM_PEAK_GBS = 8000.0          # MI355X HBM3E
FP32_MFMA_PEAK_TFLOPS = 157.3  # MI355X dense fp32 matrix
H, HKV, D = 16, 8, 128
EPS = 9.999999974752427e-7
PROFILES = os.path.join(ROOT, "profiles")


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def traffic_from_profiles(name: str):
    """HBM bytes per launch measured by rocprofv3 --pmc (committed summary)."""
    path = os.path.join(PROFILES, name)
    if not os.path.exists(path):
        return None
    m = re.search(r"traffic_bytes_per_launch:\s*([0-9.eE+]+)", open(path).read())
    return float(m.group(1)) if m else None


class Timer:
    """HIP events on the benchmark stream around whole steps and single launches."""

    def __init__(self, torch, stream):
        self.torch, self.stream = torch, stream

    def event(self):
        e = self.torch.cuda.Event(enable_timing=True)
        e.record(self.stream)
        return e


# ------------------------------------------------------------------ workloads
class Decode32k:
    name = "decode32k"

    def __init__(self, torch, ops, layers=28, n_keys=32769):
        self.torch, self.ops = torch, ops
        self.L, self.nk = layers, n_keys
        self.pos = n_keys - 1
        self.maxk = n_keys
        dev = "cuda"
        g = torch.Generator(device=dev)
        g.manual_seed(2026)
        rows = self.maxk * HKV * D
        log(f"[{self.name}] allocating {2 * layers * rows * 4 / 1e9:.2f} GB of K/V cache")
        self.kc = [torch.randn(rows, device=dev, generator=g) for _ in range(layers)]
        self.vc = [torch.randn(rows, device=dev, generator=g) for _ in range(layers)]
        self.q = torch.randn(layers, H * D, device=dev, generator=g)
        self.k = torch.randn(layers, HKV * D, device=dev, generator=g)
        self.v = torch.randn(layers, HKV * D, device=dev, generator=g)
        self.gq = 1 + 0.1 * torch.randn(layers, D, device=dev, generator=g)
        self.gk = 1 + 0.1 * torch.randn(layers, D, device=dev, generator=g)
        self.inv = torch.tensor(ops.rope_inv_freq(D, 1e6), device=dev)
        self.qn = torch.empty(layers, H * D, device=dev)
        self.o = torch.empty(layers, H * D, device=dev)
        self.ws = ops.Workspace(H, HKV, D, self.maxk)
        # Algorithmic bytes per layer: K and V rows of every key once, q in,
        # o out, the new k and v rows.
        self.bytes_per_launch = 2 * n_keys * HKV * D * 4 + 2 * H * D * 4 + 2 * HKV * D * 4
        self.work_per_step = layers * self.bytes_per_launch
        self.launches_per_step = layers

    def launch(self, l):
        ops = self.ops
        ops.decode_layer(self.q[l], self.k[l], self.v[l], self.gq[l], self.gk[l], self.inv, EPS,
                         "neox", self.qn[l], self.kc[l], self.vc[l], self.o[l], self.pos, H, HKV,
                         D, self.maxk, self.ws)

    def step(self):
        for l in range(self.L):
            self.launch(l)

    def value(self, ms):
        return self.work_per_step / (ms * 1e-3) / 1e9

    unit = "GB/s"

    def config(self):
        return {"workload": f"GQA decode, {self.L} layers x {self.nk} keys (pos {self.pos}), "
                            "fused q/k RMSNorm + RoPE + K/V append + split-K attention",
                "layers": self.L, "n_keys": self.nk, "n_heads": H, "n_kv_heads": HKV,
                "head_dim": D, "batch": 1, "kv_cache_bytes": 2 * self.L * self.maxk * HKV * D * 4}

    def roofline(self, launch_ms, traffic):
        achieved = self.bytes_per_launch / (launch_ms * 1e-3) / 1e9
        return {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS,
                "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": traffic,
                "kernel": "decode_kernel<128,2> (flk_decode_layer)",
                "bytes_per_launch": self.bytes_per_launch,
                "avg_launch_us": round(launch_ms * 1e3, 2)}

    def cpu_baseline(self, seconds=12.0):
        """The oracle's attention slice of one layer (1 thread), repeated."""
        import oracle
        oracle.set_threads(1)
        rng = np.random.default_rng(5)
        nk = self.nk
        kc = rng.standard_normal(nk * HKV * D, dtype=np.float32)
        vc = rng.standard_normal(nk * HKV * D, dtype=np.float32)
        q = rng.standard_normal(H * D, dtype=np.float32)
        k = rng.standard_normal(HKV * D, dtype=np.float32)
        v = rng.standard_normal(HKV * D, dtype=np.float32)
        gq = rng.normal(1, 0.1, D).astype(np.float32)
        gk = rng.normal(1, 0.1, D).astype(np.float32)
        inv = oracle.rope_inv_freq(D)
        oracle.layer_attn_decode(q, k, v, gq, gk, inv, kc, vc, nk - 1, H, HKV, D)  # warm-up
        n, t0 = 0, time.perf_counter()
        while True:
            oracle.layer_attn_decode(q, k, v, gq, gk, inv, kc, vc, nk - 1, H, HKV, D)
            n += 1
            if time.perf_counter() - t0 > seconds:
                break
        dt = time.perf_counter() - t0
        return {"value": round(n * self.bytes_per_launch / dt / 1e9, 3), "unit": "GB/s",
                "cores": 1, "kind": "port",
                "sample": f"{n} x one layer of this workload (oracle layer_attn_decode, "
                          f"{nk} keys, f32, 1 thread): {dt / n * 1e3:.1f} ms per layer, "
                          f"{dt:.1f} s total"}


class Prefill2k:
    name = "prefill2k"
    unit = "TFLOP/s"

    def __init__(self, torch, ops, n=2048, pos0=0, layers=1, cache_rows=None):
        self.torch, self.ops = torch, ops
        self.n, self.pos0, self.L = n, pos0, layers
        self.maxk = cache_rows or (pos0 + n)
        dev = "cuda"
        g = torch.Generator(device=dev)
        g.manual_seed(4096 + n + pos0)
        rows = self.maxk * HKV * D
        self.kc = [torch.randn(rows, device=dev, generator=g) for _ in range(layers)]
        self.vc = [torch.randn(rows, device=dev, generator=g) for _ in range(layers)]
        self.q = torch.randn(layers, n * H * D, device=dev, generator=g)
        self.k = torch.randn(layers, n * HKV * D, device=dev, generator=g)
        self.v = torch.randn(layers, n * HKV * D, device=dev, generator=g)
        self.gq = 1 + 0.1 * torch.randn(layers, D, device=dev, generator=g)
        self.gk = 1 + 0.1 * torch.randn(layers, D, device=dev, generator=g)
        self.inv = torch.tensor(ops.rope_inv_freq(D, 1e6), device=dev)
        self.qn = torch.empty(layers, n * H * D, device=dev)
        self.o = torch.empty(layers, n * H * D, device=dev)
        self.ws = ops.Workspace(H, HKV, D, self.maxk, n)
        causal_keys = n * pos0 + n * (n + 1) // 2
        self.flops_per_launch = 4 * H * D * causal_keys
        self.work_per_step = layers * self.flops_per_launch
        self.launches_per_step = layers

    def launch(self, l):
        ops = self.ops
        ops.qk_prologue(self.q[l], self.k[l], self.v[l], self.gq[l], self.gk[l], self.inv, EPS,
                        "neox", self.qn[l], self.kc[l], self.vc[l], self.n, self.pos0, H, HKV, D,
                        self.maxk)
        ops.attn_prefill(self.qn[l], self.kc[l], self.vc[l], self.o[l], H, HKV, D, self.n,
                         self.pos0, self.ws)

    def step(self):
        for l in range(self.L):
            self.launch(l)

    def value(self, ms):
        return self.work_per_step / (ms * 1e-3) / 1e12

    def config(self):
        return {"workload": f"causal GQA prefill, {self.n} tokens at pos0 {self.pos0}, "
                            f"{self.L} layer(s): fused prologue + K/V write + MFMA attention",
                "layers": self.L, "n_queries": self.n, "pos0": self.pos0, "n_heads": H,
                "n_kv_heads": HKV, "head_dim": D}

    def roofline(self, launch_ms, traffic):
        achieved = self.flops_per_launch / (launch_ms * 1e-3) / 1e12
        return {"bound": "mfma", "achieved": round(achieved, 2), "peak": FP32_MFMA_PEAK_TFLOPS,
                "unit": "TFLOP/s", "frac": round(achieved / FP32_MFMA_PEAK_TFLOPS, 4),
                "traffic": traffic, "kernel": "qk_prologue + prefill_kernel<128> (+ merge)",
                "flops_per_launch": self.flops_per_launch,
                "avg_launch_us": round(launch_ms * 1e3, 2)}

    def cpu_baseline(self, seconds=10.0):
        """The oracle's prefill slice on a bounded prefix of the prompt (1 thread)."""
        import oracle
        oracle.set_threads(1)
        rng = np.random.default_rng(6)
        n = min(self.n, 384)
        pos0 = self.pos0
        nk = pos0 + n
        kc = np.zeros(nk * HKV * D, np.float32)
        vc = np.zeros_like(kc)
        kc[:pos0 * HKV * D] = rng.standard_normal(pos0 * HKV * D, dtype=np.float32)
        vc[:pos0 * HKV * D] = rng.standard_normal(pos0 * HKV * D, dtype=np.float32)
        q = rng.standard_normal(n * H * D, dtype=np.float32)
        k = rng.standard_normal(n * HKV * D, dtype=np.float32)
        v = rng.standard_normal(n * HKV * D, dtype=np.float32)
        gq = rng.normal(1, 0.1, D).astype(np.float32)
        gk = rng.normal(1, 0.1, D).astype(np.float32)
        inv = oracle.rope_inv_freq(D)
        flops = 4 * H * D * (n * pos0 + n * (n + 1) // 2)
        reps, t0 = 0, time.perf_counter()
        while True:
            oracle.layer_attn_prefill(q, k, v, gq, gk, inv, kc.copy(), vc.copy(), n, pos0, H,
                                      HKV, D)
            reps += 1
            if time.perf_counter() - t0 > seconds:
                break
        dt = time.perf_counter() - t0
        return {"value": round(reps * flops / dt / 1e12, 6), "unit": "TFLOP/s", "cores": 1,
                "kind": "port",
                "sample": f"{reps} x oracle layer_attn_prefill of the first {n} tokens "
                          f"(pos0 {pos0}, f32, 1 thread), {dt:.1f} s"}


class Chunk32k(Prefill2k):
    name = "chunk32k"

    def __init__(self, torch, ops):
        super().__init__(torch, ops, n=64, pos0=32768, layers=28, cache_rows=32768 + 64)


class Ragged:
    name = "ragged"
    unit = "GB/s"

    def __init__(self, torch, ops, n_seqs=64, seed=3):
        self.torch, self.ops = torch, ops
        rng = np.random.default_rng(seed)
        lens = rng.integers(1024, 16385, n_seqs).astype(np.uint32)  # cached keys
        self.n_keys = (lens + 1).astype(np.uint32)                  # + the new token
        offs = np.concatenate([[0], np.cumsum(self.n_keys.astype(np.uint64))[:-1]])
        rows = int(self.n_keys.astype(np.uint64).sum())
        dev = "cuda"
        g = torch.Generator(device=dev)
        g.manual_seed(77)
        log(f"[ragged] {n_seqs} sequences, {rows} cache rows ({2 * rows * HKV * D * 4 / 1e9:.2f} GB)")
        self.kc = torch.randn(rows * HKV * D, device=dev, generator=g)
        self.vc = torch.randn(rows * HKV * D, device=dev, generator=g)
        self.q = torch.randn(n_seqs * H * D, device=dev, generator=g)
        self.o = torch.empty(n_seqs * H * D, device=dev)
        self.offs = torch.tensor(offs.astype(np.int64), device=dev)
        self.nkd = torch.tensor(self.n_keys.astype(np.int32), device=dev)
        self.B, self.maxn = n_seqs, int(self.n_keys.max())
        self.ws = ops.Workspace(H, HKV, D, self.maxn, 0, n_seqs)
        self.bytes_per_launch = 2 * rows * HKV * D * 4 + 2 * n_seqs * H * D * 4
        self.work_per_step = self.bytes_per_launch
        self.launches_per_step = 1

    def launch(self, l=0):
        self.ops.attn_decode_ragged(self.q, self.kc, self.vc, self.offs, self.nkd, self.o, self.B,
                                    self.maxn, H, HKV, D, self.ws)

    def step(self):
        self.launch()

    def value(self, ms):
        return self.work_per_step / (ms * 1e-3) / 1e9

    def config(self):
        return {"workload": f"ragged GQA decode, {self.B} sequences, n_keys U[1025,16385] "
                            f"(sum {int(self.n_keys.astype(np.uint64).sum())})",
                "n_seqs": self.B, "sum_n_keys": int(self.n_keys.astype(np.uint64).sum()),
                "n_heads": H, "n_kv_heads": HKV, "head_dim": D}

    def roofline(self, launch_ms, traffic):
        achieved = self.bytes_per_launch / (launch_ms * 1e-3) / 1e9
        return {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS,
                "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": traffic,
                "kernel": "decode_kernel<128,2> (flk_attn_decode_ragged)",
                "bytes_per_launch": self.bytes_per_launch,
                "avg_launch_us": round(launch_ms * 1e3, 2)}

    def cpu_baseline(self, seconds=10.0):
        return None


class Decode512(Decode32k):
    name = "decode512"

    def __init__(self, torch, ops):
        super().__init__(torch, ops, layers=1, n_keys=513)


WORKLOADS = {c.name: c for c in (Decode32k, Prefill2k, Ragged, Chunk32k, Decode512)}


def measure(torch, stream, w, steps, warmup):
    """Time `steps` steps (events around the whole region) and, in a second
    pass, every launch of the dominant kernel (events around each launch)."""
    for _ in range(warmup):
        w.step()
    torch.cuda.synchronize()
    tm = Timer(torch, stream)
    start = tm.event()
    t0 = time.perf_counter()
    for _ in range(steps):
        w.step()
    end = tm.event()
    torch.cuda.synchronize()
    wall_ms = (time.perf_counter() - t0) * 1e3 / steps
    ms = start.elapsed_time(end) / steps
    # Per-launch pass.
    pairs = []
    for _ in range(max(1, min(steps, 10))):
        for l in range(w.launches_per_step):
            a = tm.event()
            w.launch(l)
            b = tm.event()
            pairs.append((a, b))
    torch.cuda.synchronize()
    launch_ms = float(np.mean([a.elapsed_time(b) for a, b in pairs]))
    return ms, wall_ms, launch_ms


def main():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--workload", default="decode32k", choices=sorted(WORKLOADS))
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-secondary", action="store_true",
                    help="skip the prefill2k measurement of the default run")
    args = ap.parse_args()

    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU: this path has no multi-GPU mode "
              f"(asked for --gpus {args.gpus}). Run with --gpus 1.", file=sys.stderr)
        sys.exit(2)

    import torch
    from flock_amd import ops

    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        sys.exit(1)
    stream = torch.cuda.Stream()
    ops.set_stream(stream)
    with torch.cuda.stream(stream):
        w = WORKLOADS[args.workload](torch, ops)
        torch.cuda.synchronize()
        log(f"[{w.name}] warmup {args.warmup}, timing {args.steps} steps")
        ms, wall_ms, launch_ms = measure(torch, stream, w, args.steps, args.warmup)
        value = w.value(ms)
        log(f"[{w.name}] {ms:.3f} ms/step (host wall {wall_ms:.3f}), {value:.2f} {w.unit}, "
            f"avg launch {launch_ms * 1e3:.2f} us")
        traffic = traffic_from_profiles(f"{w.name}_pmc.md")
        out = {
            "metric": METRIC, "value": round(value, 3), "unit": w.unit, "n_gpus": 1,
            "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms, 4),
            "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "f32",
            "data": "synthetic: seeded N(0,1) q/k/v and K/V caches, norm gains N(1,0.1); "
                    "no weights (attention path only)",
            "config": w.config(), "roofline": w.roofline(launch_ms, traffic),
        }
        if w.unit == "GB/s":
            out["frac_of_hbm_peak"] = round(value / HBM_PEAK_GBS, 4)
        else:
            out["frac_of_fp32_mfma_peak"] = round(value / FP32_MFMA_PEAK_TFLOPS, 4)
        del w
        torch.cuda.empty_cache()

        if args.workload == "decode32k" and not args.no_secondary:
            p = Prefill2k(torch, ops)
            torch.cuda.synchronize()
            pms, _, plaunch = measure(torch, stream, p, max(5, args.steps), args.warmup)
            pv = p.value(pms)
            log(f"[prefill2k] {pms:.3f} ms/step, {pv:.2f} TFLOP/s")
            out["prefill"] = {"workload": p.config()["workload"], "value": round(pv, 3),
                              "unit": "TFLOP/s", "ms_per_step": round(pms, 4),
                              "frac_of_fp32_mfma_peak": round(pv / FP32_MFMA_PEAK_TFLOPS, 4),
                              "roofline": p.roofline(plaunch, traffic_from_profiles("prefill2k_pmc.md"))}
            if not args.no_cpu_baseline:
                log("[prefill2k] CPU baseline (oracle port)")
                out["prefill"]["cpu_baseline"] = p.cpu_baseline()
            del p

    if not args.no_cpu_baseline:
        log(f"[{args.workload}] CPU baseline (oracle port, 1 thread)")
        cb = WORKLOADS[args.workload].cpu_baseline(_Shape(args.workload))
        out["cpu_baseline"] = cb
    print(json.dumps(out), flush=True)


class _Shape:
    """The workload's sizes without its device buffers (for the CPU baseline)."""

    def __init__(self, name):
        proto = {"decode32k": (28, 32769, None), "decode512": (1, 513, None),
                 "prefill2k": (1, None, (2048, 0)), "chunk32k": (28, None, (64, 32768))}
        L, nk, pre = proto.get(name, (1, 1, None))
        self.L = L
        if nk:
            self.nk, self.pos, self.maxk = nk, nk - 1, nk
            self.bytes_per_launch = 2 * nk * HKV * D * 4 + 2 * H * D * 4 + 2 * HKV * D * 4
        if pre:
            self.n, self.pos0 = pre


if __name__ == "__main__":
    main()
