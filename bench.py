"""Benchmark of flock's attention hot path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload NAME]

Prints ONE JSON line on stdout (progress goes to stderr). A step is one pass
of the hot path over one batch of synthetic, HBM-resident input:

  decode32k  (default) Long-context GQA decode, all 28 Qwen3-0.6B layers:
             per layer one flk_decode_layer call = per-head q/k RMSNorm + RoPE
             (theta 1e6) + K/V append at position 32768 + split-K decode
             attention over 32769 keys (16 q / 8 kv heads, d 128, f32).
             value = algorithmic HBM bytes / step time (GB/s).
  prefill2k  Causal prefill of 2048 tokens at position 0: fused prologue
             (norm + RoPE + K/V write), then MFMA flash attention.
             value = causal attention flops / step time (TFLOP/s).
  ragged     64 independent sequences, n_keys ~ U[1025, 16385] (seeded), one
             decode step for all of them in one flk_decode_layer_ragged call:
             per sequence q/k RMSNorm + RoPE at position n_keys - 1, the K/V
             append, and attention. value in GB/s.
  chunk32k   A 64-token chunk at position 32768 onto a 32768-key cache, 28
             layers: prologue + chunked prefill attention. value in TFLOP/s.
  decode512  The same 28-layer step at 513 keys (4.2 MB per layer: it fits in
             the 256 MB MALL, so the figure is an "effective" GB/s), the 28
             calls replayed from one captured HIP graph (launch-bound).
  copy       1 GiB device-to-device copy (torch): the reference kernel of
             known traffic that calibrates the FETCH_SIZE / WRITE_SIZE
             counters in profiles/.
  q8lmhead   The Q8_0 projection next to the path at its largest: the
             151936 x 1024 LM head, one token (flk_q8_matvec). GB/s.
  q8proj     The seven Q8_0 projections of all 28 layers for one decode
             token (196 flk_q8_matvec calls). GB/s.
  token32k   One greedy decode token through the whole model: 28 decoder
             layers (DecoderLayer: fused projections + attention over 32769
             keys) + output norm + LM head + argmax. GB/s and tokens/s.
  token512   The same at 513 keys (launch-bound).
  gen32k     Greedy generation with the captured one-token HIP graph
             (flock_amd.model): 32 tokens per step from position 32768.
             GB/s and tokens/s.
  gen512     The same from position 512.
  q8prefill  The largest prefill projection: ffn_norm + gate/up (2 x 3072 x
             1024) + SwiGLU over 2048 tokens in one call (the weight-reusing
             tile kernel). TFLOP/s against the fp32 vector peak.
  prompt2k   Time to first token: a 2048-token prompt through Model.step
             (28 layers in prefill + head). tokens/s and ms per prompt.
  replay32k  Chunked replay: a 64-id chunk at position 32768 through Model.step
             (28 layers of prefill onto the cache + head). tokens/s.

The default run also measures, each under its own key with its own roofline:
prefill2k ("prefill", the metric's second half), decode512 ("decode512"),
ragged ("ragged"), chunk32k ("chunk32k", in TFLOP/s and in GB/s of K/V
read), the LM-head projection ("q8_lm_head"),
greedy generation at 32k context ("generate") and the 2048-token prompt
("prompt"). Inputs are N(0, 1) from a seeded generator (gains N(1, 0.1));
caches are written on the device before timing starts.

CPU leg (after every GPU measurement). After a workload's timed region its
inputs and outputs for one layer (the whole batch for ragged) are copied to
the host; the oracle (oracle/, C) then runs on exactly those values. That run
is both the CPU baseline -- 1 thread (value, cores 1) and OpenMP on the host's
share of cores ("openmp"), with the host's CPU model and nproc -- and the
parity check: "parity" holds max_abs and relErr of the GPU against the
oracle, both distances from the float64 closed form, the clause of the bar
that decided, the per-row argmax agreement, and bit-exactness of qn and the
appended cache rows. Decode at 32k runs its layer 28 times on 1 thread (one
whole step); prefill2k and ragged run in full; chunk32k runs one of its 28
layers and states the x28 extrapolation.

Timing: HIP events recorded on the stream the kernels are launched on bracket
the K timed steps (after a synchronize). The roofline's average call duration
is events around R back-to-back calls of the dominant entry point, divided by
R. One flk_decode_layer call is the split kernel plus its merge kernel; one
flk_attn_prefill call is the prefill kernel, plus a merge kernel when the
plan splits keys (chunk32k).
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
# MI355X's published fp32 vector peak; VALU rooflines divide by it. It counts
# packed-fp32 instructions (two flops per lane per cycle), which this library
# never emits, so its VALU code can reach at most half of it: VALU rooflines
# also report the fraction of that unpacked ceiling.
FP32_VECTOR_PEAK_TFLOPS = 157.3
FP32_UNPACKED_VALU_TFLOPS = 78.6
H, HKV, D = 16, 8, 128
EPS = 9.999999974752427e-7
PROFILES = os.path.join(ROOT, "profiles")


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def traffic_from_profiles(name: str):
    """HBM bytes per call measured by rocprofv3 --pmc (committed summary)."""
    path = os.path.join(PROFILES, name)
    if not os.path.exists(path):
        return None
    m = re.search(r"traffic_bytes_per_launch:\s*([0-9.eE+]+)", open(path).read())
    return float(m.group(1)) if m else None


def rng_inputs(torch, seed, shapes):
    g = torch.Generator(device="cuda")
    g.manual_seed(seed)
    return [torch.randn(n, device="cuda", generator=g) for n in shapes], g


# ------------------------------------------------------------------ workloads
class Workload:
    """One benchmark: step() is the timed unit, call(i) the dominant call."""

    name = ""
    unit = "GB/s"
    bound = "hbm"
    calls_per_step = 1
    graph_step = False  # step() replays a captured graph: call time = step time / calls
    roofline_note = None
    data = ("synthetic: seeded N(0,1) q/k/v and K/V caches, norm gains N(1,0.1); no weights "
            "(attention path only)")

    def value(self, ms):
        scale = 1e9 if self.unit == "GB/s" else 1e12
        return self.work_per_step / (ms * 1e-3) / scale

    def roofline(self, call_ms, traffic):
        if self.bound == "hbm":
            achieved = self.work_per_call / (call_ms * 1e-3) / 1e9
            peak, unit, key = HBM_PEAK_GBS, "GB/s", "bytes_per_launch"
        elif self.bound in ("valu", "mixed"):
            achieved = self.work_per_call / (call_ms * 1e-3) / 1e12
            peak, unit, key = FP32_VECTOR_PEAK_TFLOPS, "TFLOP/s", "flops_per_launch"
        else:
            achieved = self.work_per_call / (call_ms * 1e-3) / 1e12
            peak, unit, key = FP32_MFMA_PEAK_TFLOPS, "TFLOP/s", "flops_per_launch"
        out = {"bound": self.bound, "achieved": round(achieved, 2), "peak": peak, "unit": unit,
               "frac": round(achieved / peak, 4), "traffic": traffic, "kernel": self.kernel,
               key: self.work_per_call, "avg_launch_us": round(call_ms * 1e3, 2)}
        if self.bound in ("valu", "mixed"):
            out["frac_of_unpacked_valu"] = round(achieved / FP32_UNPACKED_VALU_TFLOPS, 4)
        if self.bound == "mixed":
            out["note"] = ("flops of fp32-MFMA attention and VALU projections together, against "
                           "the fp32 vector peak")
        if self.roofline_note:
            out["note"] = self.roofline_note
        return out

    # CPU leg: capture() keeps host copies of the timed inputs and the GPU's
    # outputs (self.host); cpu_sample(threads) runs the oracle on them and
    # returns (work done, seconds, what ran), keeping the oracle's outputs of
    # its first run in self.ref; parity() compares the two.
    cpu_sample = None
    cpu_parallel = True
    host = None
    ref = None

    def capture(self):
        pass

    def parity(self):
        return None

    def cpu_leg(self, baseline=True):
        """The oracle on this host's cores over the captured inputs: the CPU
        baseline -- 1 thread (the primary figure, as the reference's
        single-threaded TypeScript oracle), then OpenMP on the host's share
        of cores -- and the parity of the GPU's outputs against it. Returns
        (cpu_baseline or None, parity or None)."""
        if self.cpu_sample is None:
            return None, None
        import oracle
        model, nproc, share = cpu_info()
        scale = 1e9 if self.unit == "GB/s" else 1e12
        out = None
        legs = (1, share) if baseline else (share,)
        for th in legs:
            oracle.set_threads(th)
            work, dt, what = self.cpu_sample(th)
            entry = {"value": round(work / dt / scale, 6), "unit": self.unit, "cores": th,
                     "kind": "port", "sample": f"{what}; f32, {th} thread(s), {dt:.1f} s"}
            if out is None:
                out = dict(entry, nproc=nproc, cpu_model=model)
            else:
                out["openmp"] = entry
            if share == 1 or not self.cpu_parallel:
                break
        oracle.set_threads(share)
        par = self.parity()
        oracle.set_threads(1)
        return (out if baseline else None), par


def host(x):
    """A device tensor's values as a host numpy array (ordered after the work
    queued on the current stream)."""
    return x.detach().cpu().numpy().copy()


def parity_entry(m, ids, inputs, **extra):
    """The parity object of one workload: the bar's numbers (oracle/parity.py)."""
    from oracle.parity import clause
    out = {k: float(f"{m[k]:.3e}") for k in ("max_abs", "rel", "gpu_abs_vs_f64",
                                               "oracle_abs_vs_f64") if k in m}
    out["clause"] = clause(m)
    out.update(ids)
    out.update(extra)
    out["inputs"] = inputs
    return out


def cpu_info():
    """(CPU model, logical CPUs, threads for the all-cores leg). The threads
    are the host's share for this GPU (OMP_NUM_THREADS when set), at most 16."""
    model = ""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    nproc = os.cpu_count() or 1
    share = int(os.environ.get("OMP_NUM_THREADS", "0") or 0) or nproc
    return model, nproc, max(1, min(share, nproc, 16))


def timed(fn, min_seconds, reps=None):
    """Run fn() exactly `reps` times, or (reps None) until min_seconds have
    passed, at least once; returns (reps, seconds)."""
    n, t0 = 0, time.perf_counter()
    while True:
        fn()
        n += 1
        dt = time.perf_counter() - t0
        if (reps is not None and n >= reps) or (reps is None and dt >= min_seconds):
            return n, dt


class Decode32k(Workload):
    name = "decode32k"
    kernel = ("flk_decode_layer: decode_split_kernel<128,2,8> + decode_merge_kernel<128> "
              "(one call per layer)")

    def __init__(self, torch, ops, layers=28, n_keys=32769):
        self.torch, self.ops = torch, ops
        self.L, self.nk = layers, n_keys
        self.pos = n_keys - 1
        self.maxk = n_keys
        rows = self.maxk * HKV * D
        log(f"[{self.name}] allocating {2 * layers * rows * 4 / 1e9:.2f} GB of K/V cache")
        caches, g = rng_inputs(torch, 2026, [rows] * (2 * layers))
        self.kc, self.vc = caches[:layers], caches[layers:]
        self.q = torch.randn(layers, H * D, device="cuda", generator=g)
        self.k = torch.randn(layers, HKV * D, device="cuda", generator=g)
        self.v = torch.randn(layers, HKV * D, device="cuda", generator=g)
        self.gq = 1 + 0.1 * torch.randn(layers, D, device="cuda", generator=g)
        self.gk = 1 + 0.1 * torch.randn(layers, D, device="cuda", generator=g)
        self.inv = torch.tensor(ops.rope_inv_freq(D, 1e6), device="cuda")
        self.qn = torch.empty(layers, H * D, device="cuda")
        self.o = torch.empty(layers, H * D, device="cuda")
        self.ws = ops.Workspace(H, HKV, D, self.maxk)
        # Algorithmic bytes of one call: every K and V row of the kv heads
        # once, q in, o out, the new k and v rows (read raw, written once).
        self.work_per_call = 2 * n_keys * HKV * D * 4 + 2 * H * D * 4 + 2 * HKV * D * 4
        self.work_per_step = layers * self.work_per_call
        self.calls_per_step = layers

    def call(self, l):
        self.ops.decode_layer(self.q[l], self.k[l], self.v[l], self.gq[l], self.gk[l], self.inv,
                              EPS, "neox", self.qn[l], self.kc[l], self.vc[l], self.o[l],
                              self.pos, H, HKV, D, self.maxk, self.ws)

    def step(self):
        for l in range(self.L):
            self.call(l)

    def config(self):
        how = ", the layers' calls replayed from one captured HIP graph" if self.graph_step else ""
        return {"workload": f"GQA decode, {self.L} layers x {self.nk} keys (new token at position "
                            f"{self.pos}), per layer fused q/k RMSNorm + RoPE + K/V append + "
                            f"split-K attention{how}",
                "layers": self.L, "n_keys": self.nk, "n_heads": H, "n_kv_heads": HKV,
                "head_dim": D, "batch": 1, "kv_cache_bytes": 2 * self.L * self.maxk * HKV * D * 4}

    def capture(self, l=0):
        """Layer l's timed inputs and the GPU's outputs, on the host."""
        self.torch.cuda.synchronize()
        h = {k: host(getattr(self, k)[l]) for k in ("q", "k", "v", "gq", "gk", "kc", "vc", "qn",
                                                      "o")}
        h["inv"] = host(self.inv)
        row = HKV * D
        p = self.pos * row
        h["k_row"], h["v_row"] = h["kc"][p:p + row].copy(), h["vc"][p:p + row].copy()
        self.host = h

    def cpu_sample(self, threads):
        """oracle layer_attn_decode (norm, RoPE, append, attention) of layer 0
        of the timed step, on its inputs: 1 thread, once per layer of the step
        (the full step's work); more threads, repeated for >= 3 s."""
        import oracle
        h = self.host
        layer = lambda: oracle.layer_attn_decode(h["q"], h["k"], h["v"], h["gq"], h["gk"], h["inv"],
                                                 h["kc"], h["vc"], self.pos, H, HKV, D)
        first = layer()  # also the warm-up (pages the cache in)
        if self.ref is None:
            self.ref = first
        nk = self.nk
        if threads == 1 and self.L > 1:
            n, dt = timed(layer, 0.0, reps=self.L)
            what = (f"oracle layer_attn_decode x {n} (one whole step's work) over {nk} keys, on "
                    "the timed step's layer-0 inputs")
        else:
            n, dt = timed(layer, 3.0)
            what = f"oracle layer_attn_decode x {n} over {nk} keys, on the timed layer-0 inputs"
        return n * self.work_per_call, dt, what

    def parity(self):
        from oracle import closed_form as cf
        from oracle.parity import ids_check, metrics, projection_ids
        h = self.host
        qn, o = self.ref
        m = metrics(h["o"], o, cf.attention(qn, h["kc"], h["vc"], H, HKV, D, 1, self.pos))
        row, p = HKV * D, self.pos * HKV * D
        return parity_entry(
            m, ids_check(h["o"], o, H, m["max_abs"]),
            "layer 0 of the timed step: its q/k/v, gains, cache and the GPU's qn, o and "
            "appended row, copied to the host after the timed region",
            projection_id_equal=projection_ids(h["o"])[0] == projection_ids(o)[0],
            qn_bit_exact=bool(np.array_equal(h["qn"], qn)),
            appended_row_bit_exact=bool(np.array_equal(h["k_row"], h["kc"][p:p + row]) and
                                        np.array_equal(h["v_row"], h["vc"][p:p + row])))


class Decode512(Decode32k):
    """The same layer call at 513 keys (4.2 MB per layer: it fits in the 256 MB
    MALL, so the figure is an effective GB/s). A call costs about as much as
    its launches here, so the step -- one call per layer of 28 -- is captured
    once into a HIP graph and replayed, as a host decoding many tokens would
    (Model.replay); the call time is the step time / 28."""

    name = "decode512"
    kernel = ("flk_decode_layer x 28 replayed from one HIP graph: decode_split_kernel<128,2,8> + "
              "decode_merge_kernel<128> per call")
    graph_step = True
    roofline_note = ("latency-bound: a call reads 4.2 MB, which HBM would deliver in ~0.5 us; "
                     "the two kernels' launch and memory latency set its time")

    def __init__(self, torch, ops):
        super().__init__(torch, ops, layers=28, n_keys=513)
        self.graph = None

    def step(self):
        if self.graph is None:
            with self.ops.Graph() as g:
                for l in range(self.L):
                    self.call(l)
            self.graph = g
        self.graph.launch()


class Prefill2k(Workload):
    name = "prefill2k"
    unit = "TFLOP/s"
    bound = "mfma"
    kernel = "flk_attn_prefill: prefill_kernel<128> (paired q tiles, no merge launch)"

    def __init__(self, torch, ops, n=2048, pos0=0, layers=1):
        self.torch, self.ops = torch, ops
        self.n, self.pos0, self.L = n, pos0, layers
        self.maxk = pos0 + n
        rows = self.maxk * HKV * D
        caches, g = rng_inputs(torch, 4096 + n + pos0, [rows] * (2 * layers))
        self.kc, self.vc = caches[:layers], caches[layers:]
        self.q = torch.randn(layers, n * H * D, device="cuda", generator=g)
        self.k = torch.randn(layers, n * HKV * D, device="cuda", generator=g)
        self.v = torch.randn(layers, n * HKV * D, device="cuda", generator=g)
        self.gq = 1 + 0.1 * torch.randn(layers, D, device="cuda", generator=g)
        self.gk = 1 + 0.1 * torch.randn(layers, D, device="cuda", generator=g)
        self.inv = torch.tensor(ops.rope_inv_freq(D, 1e6), device="cuda")
        self.qn = torch.empty(layers, n * H * D, device="cuda")
        self.o = torch.empty(layers, n * H * D, device="cuda")
        self.ws = ops.Workspace(H, HKV, D, self.maxk, n)
        # Causal attention flops: QK^T and PV, 2 flops per multiply-add each,
        # over the keys each query sees (pos0 + i + 1 for query i).
        causal_keys = n * pos0 + n * (n + 1) // 2
        self.work_per_call = 4 * H * D * causal_keys
        self.work_per_step = layers * self.work_per_call
        self.calls_per_step = layers

    def prologue_line(self, torch, stream, reps=20):
        """The step's other kernel, timed on its own: the flk_qk_prologue calls
        of the step's layers captured once into a HIP graph (so a short call
        is not timed at the host's launch rate), replayed R times between
        events. Its bytes: raw q, k, v read, qn and the k, v cache rows
        written."""
        torch.cuda.synchronize()
        per = max(self.L, 8)
        with self.ops.Graph() as g:
            for i in range(per):
                self.prologue(i % self.L)
        g.launch()
        torch.cuda.synchronize()
        start = torch.cuda.Event(enable_timing=True)
        end = torch.cuda.Event(enable_timing=True)
        start.record(stream)
        for _ in range(reps):
            g.launch()
        end.record(stream)
        torch.cuda.synchronize()
        g.free()
        us = start.elapsed_time(end) * 1e3 / (reps * per)
        b = 2 * self.n * (H + 2 * HKV) * D * 4
        gbs = b / (us * 1e-6) / 1e9
        return {"prologue": {"kernel": "flk_qk_prologue: qk_prologue_kernel<128> (one workgroup "
                                       "per token)", "bound": "hbm", "bytes_per_launch": b,
                             "avg_launch_us": round(us, 2), "achieved": round(gbs, 2),
                             "unit": "GB/s", "peak": HBM_PEAK_GBS,
                             "frac": round(gbs / HBM_PEAK_GBS, 4),
                             "share_of_step": round(us * self.L / 1e3 / self.step_ms, 4)}}

    def prologue(self, l):
        self.ops.qk_prologue(self.q[l], self.k[l], self.v[l], self.gq[l], self.gk[l], self.inv,
                             EPS, "neox", self.qn[l], self.kc[l], self.vc[l], self.n, self.pos0,
                             H, HKV, D, self.maxk)

    def call(self, l):
        self.ops.attn_prefill(self.qn[l], self.kc[l], self.vc[l], self.o[l], H, HKV, D, self.n,
                              self.pos0, self.ws)

    def step(self):
        for l in range(self.L):
            self.prologue(l)
            self.call(l)

    def config(self):
        return {"workload": f"causal GQA prefill, {self.n} tokens at position {self.pos0}, "
                            f"{self.L} layer(s): fused q/k RMSNorm + RoPE + K/V write, then "
                            "fp32-MFMA flash attention",
                "layers": self.L, "n_queries": self.n, "pos0": self.pos0, "n_heads": H,
                "n_kv_heads": HKV, "head_dim": D}

    def capture(self, l=0):
        """Layer l's timed inputs and the GPU's outputs, on the host."""
        self.torch.cuda.synchronize()
        h = {k: host(getattr(self, k)[l]) for k in ("q", "k", "v", "gq", "gk", "kc", "vc", "qn",
                                                      "o")}
        h["inv"] = host(self.inv)
        p = self.pos0 * HKV * D
        h["k_rows"], h["v_rows"] = h["kc"][p:].copy(), h["vc"][p:].copy()
        self.host = h

    def cpu_sample(self, threads):
        """oracle layer_attn_prefill (norm, RoPE, append, causal attention) of
        layer 0 of the timed step, on its inputs, once; more threads, repeated
        for >= 2 s."""
        import oracle
        h = self.host
        n, pos0 = self.n, self.pos0
        layer = lambda: oracle.layer_attn_prefill(h["q"], h["k"], h["v"], h["gq"], h["gk"],
                                                  h["inv"], h["kc"], h["vc"], n, pos0, H, HKV, D)
        reps, dt = 0, 0.0
        if self.ref is None:  # the first run is timed too: same work every time
            t0 = time.perf_counter()
            self.ref = layer()
            reps, dt = 1, time.perf_counter() - t0
        if threads != 1 or reps == 0:
            r2, dt2 = timed(layer, 0.0 if threads == 1 else 2.0)
            reps, dt = r2, dt2
        what = (f"oracle layer_attn_prefill x {reps}: {n} tokens at position {pos0}, layer 0 "
                f"of {self.L} of the timed step")
        if self.L > 1:
            what += f" (the {self.L}-layer step extrapolates to {dt / reps * self.L:.1f} s)"
        return reps * self.work_per_call, dt, what

    def parity(self):
        from oracle import closed_form as cf
        from oracle.parity import ids_check, metrics, projection_ids
        h = self.host
        qn, o = self.ref
        n, pos0 = self.n, self.pos0
        m = metrics(h["o"], o, cf.attention(qn, h["kc"], h["vc"], H, HKV, D, n, pos0))
        p = pos0 * HKV * D
        last = H * D  # the last token's output, what an LM head reads
        return parity_entry(
            m, ids_check(h["o"], o, n * H, m["max_abs"]),
            "layer 0 of the timed step: its q/k/v, gains, cache and the GPU's qn, o and "
            "appended rows, copied to the host after the timed region",
            projection_id_equal=projection_ids(h["o"][-last:])[0] == projection_ids(o[-last:])[0],
            qn_bit_exact=bool(np.array_equal(h["qn"], qn)),
            appended_rows_bit_exact=bool(np.array_equal(h["k_rows"], h["kc"][p:]) and
                                         np.array_equal(h["v_rows"], h["vc"][p:])))


class Chunk32k(Prefill2k):
    name = "chunk32k"
    kernel = "flk_attn_prefill: prefill_kernel<128> (key splits) + prefill_merge_kernel<128>"

    def __init__(self, torch, ops):
        super().__init__(torch, ops, n=64, pos0=32768, layers=28)
        # Bytes an attention call must move: every K and V row of the cache
        # (pos0 + n keys, 8 kv heads) once, q in and o out.
        self.bytes_per_call = (2 * self.maxk * HKV * D * 4) + 2 * self.n * H * D * 4

    def extra(self, ms, call_ms):
        return {"hbm": {"bytes_per_launch": self.bytes_per_call,
                        "achieved": round(self.bytes_per_call / (call_ms * 1e-3) / 1e9, 2),
                        "unit": "GB/s", "peak": HBM_PEAK_GBS,
                        "frac": round(self.bytes_per_call / (call_ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)}}


class Ragged(Workload):
    name = "ragged"
    kernel = ("flk_decode_layer_ragged: qk_prologue_kernel<128,true> (norm + RoPE + append per "
              "sequence; resets the item counters) + decode_batch_kernel<128,2,8> (persistent, "
              "claimed items) + decode_merge_kernel<128,64>")

    def __init__(self, torch, ops, n_seqs=64, seed=3):
        self.torch, self.ops = torch, ops
        rng = np.random.default_rng(seed)
        lens = rng.integers(1024, 16385, n_seqs).astype(np.uint32)  # cached keys
        self.n_keys = (lens + 1).astype(np.uint32)                  # + the new token
        offs = np.concatenate([[0], np.cumsum(self.n_keys.astype(np.uint64))[:-1]])
        self.rows = rows = int(self.n_keys.astype(np.uint64).sum())
        log(f"[ragged] {n_seqs} sequences, {rows} cache rows "
            f"({2 * rows * HKV * D * 4 / 1e9:.2f} GB)")
        (self.kc, self.vc, self.q, self.k, self.v), g = rng_inputs(
            torch, 77, [rows * HKV * D, rows * HKV * D, n_seqs * H * D, n_seqs * HKV * D,
                        n_seqs * HKV * D])
        self.gq = 1 + 0.1 * torch.randn(D, device="cuda", generator=g)
        self.gk = 1 + 0.1 * torch.randn(D, device="cuda", generator=g)
        self.inv = torch.tensor(ops.rope_inv_freq(D, 1e6), device="cuda")
        self.qn = torch.empty(n_seqs * H * D, device="cuda")
        self.o = torch.empty(n_seqs * H * D, device="cuda")
        self.offs_h = offs.astype(np.uint64)
        self.offs = torch.tensor(offs.astype(np.int64), device="cuda")
        self.nkd = torch.tensor(self.n_keys.astype(np.int32), device="cuda")
        self.B, self.maxn = n_seqs, int(self.n_keys.max())
        self.ws = ops.Workspace(H, HKV, D, self.maxn, 0, n_seqs)
        # Algorithmic bytes: every K and V row once (the new one written), and
        # per sequence raw q, k, v in and o out.
        self.work_per_call = (2 * rows * HKV * D * 4
                              + n_seqs * (2 * H * D * 4 + 2 * HKV * D * 4))
        self.work_per_step = self.work_per_call

    def call(self, l=0):
        self.ops.decode_layer_ragged(self.q, self.k, self.v, self.gq, self.gk, self.inv, EPS,
                                     "neox", self.qn, self.kc, self.vc, self.offs, self.nkd,
                                     self.o, self.B, self.maxn, H, HKV, D, self.ws)

    def step(self):
        self.call()

    def config(self):
        return {"workload": f"ragged GQA decode step, {self.B} sequences, n_keys U[1025,16385] "
                            f"(sum {self.rows}): per sequence q/k RMSNorm + RoPE at position "
                            "n_keys - 1 + K/V append + split-K attention, one call",
                "n_seqs": self.B, "sum_n_keys": self.rows, "n_heads": H, "n_kv_heads": HKV,
                "head_dim": D}

    def capture(self):
        self.torch.cuda.synchronize()
        h = {k: host(getattr(self, k)) for k in ("q", "k", "v", "gq", "gk", "inv", "kc", "vc",
                                                  "qn", "o")}
        row = HKV * D
        last = [(int(self.offs_h[b]) + int(self.n_keys[b]) - 1) * row for b in range(self.B)]
        h["k_rows"] = np.stack([h["kc"][p:p + row] for p in last])
        h["v_rows"] = np.stack([h["vc"][p:p + row] for p in last])
        self.host = h

    def _seq(self, b):
        h, row = self.host, HKV * D
        s, n = int(self.offs_h[b]) * row, int(self.n_keys[b])
        return (h["q"][b * H * D:(b + 1) * H * D], h["k"][b * row:(b + 1) * row],
                h["v"][b * row:(b + 1) * row], h["kc"][s:s + n * row], h["vc"][s:s + n * row], n)

    def cpu_sample(self, threads):
        """oracle layer_attn_decode (norm, RoPE, append, attention) of every
        sequence of the timed batch in order, on its inputs; more threads, the
        batch repeated for >= 2 s."""
        import oracle
        h = self.host

        def batch():
            outs = []
            for b in range(self.B):
                q, k, v, kc, vc, n = self._seq(b)  # cache views: appended in place
                outs.append(oracle.layer_attn_decode(q, k, v, h["gq"], h["gk"], h["inv"], kc, vc,
                                                     n - 1, H, HKV, D))
            return outs

        reps, dt = 0, 0.0
        if self.ref is None:
            t0 = time.perf_counter()
            self.ref = batch()
            reps, dt = 1, time.perf_counter() - t0
        if threads != 1 or reps == 0:
            reps, dt = timed(batch, 0.0 if threads == 1 else 2.0)
        return reps * self.work_per_call, dt, (
            f"oracle layer_attn_decode over all {self.B} sequences of the timed batch "
            f"({self.rows} keys) x {reps}")

    def parity(self):
        from oracle import closed_form as cf
        from oracle.parity import clause, ids_check, metrics
        h, row = self.host, HKV * D
        worst, clauses, ids_ok, ties, qn_ok, rows_ok = None, {}, True, 0, True, True
        for b in range(self.B):
            q, k, v, kc, vc, n = self._seq(b)
            qn, o = self.ref[b]
            got = h["o"][b * H * D:(b + 1) * H * D]
            m = metrics(got, o, cf.attention(qn, kc, vc, H, HKV, D, 1, n - 1))
            c = clause(m)
            clauses[c] = clauses.get(c, 0) + 1
            ids = ids_check(got, o, H, m["max_abs"])
            ids_ok &= ids["argmax_equal"]
            ties += ids["near_tie_rows"]
            qn_ok &= bool(np.array_equal(h["qn"][b * H * D:(b + 1) * H * D], qn))
            rows_ok &= bool(np.array_equal(h["k_rows"][b], kc[(n - 1) * row:]) and
                            np.array_equal(h["v_rows"][b], vc[(n - 1) * row:]))
            if worst is None or m["rel"] > worst[1]["rel"]:
                worst = (b, m)
        return parity_entry(
            worst[1], {"argmax_equal": ids_ok, "argmax_rows": self.B * H, "near_tie_rows": ties},
            "every sequence of the timed batch: its q/k/v, gains, cache and the GPU's qn, o and "
            "appended rows, copied to the host after the timed region; numbers of the sequence "
            "with the largest relErr",
            worst_seq=worst[0], worst_seq_n_keys=int(self.n_keys[worst[0]]),
            clauses_over_sequences=clauses, qn_bit_exact=qn_ok, appended_rows_bit_exact=rows_ok)


class Copy(Workload):
    name = "copy"
    data = "synthetic: a 1 GiB N(0,1) buffer"
    kernel = "torch Tensor.copy_ (device to device)"

    def __init__(self, torch, ops, nbytes=1 << 30):
        self.src = torch.empty(nbytes // 4, device="cuda").normal_()
        self.dst = torch.empty_like(self.src)
        self.work_per_call = 2 * nbytes
        self.work_per_step = self.work_per_call

    def call(self, l=0):
        self.dst.copy_(self.src)

    def step(self):
        self.call()

    def config(self):
        return {"workload": f"device-to-device copy of {self.src.numel() * 4} bytes"}


class Q8LmHead(Workload):
    """Qwen3-0.6B's tied LM head as one Q8_0 matvec: 151936 x 1024."""

    data = ("synthetic: random Q8_0 weights of the Qwen3-0.6B shapes (seeded quants, f16 "
            "scales), seeded N(0,1) inputs, zeroed or seeded caches")

    name = "q8lmhead"
    kernel = ("flk_q8_matvec: q8_matvec1k_kernel (coop(64) order, 1024-column rows read "
              "contiguously)")
    rows, cols, copies = 151936, 1024, 3

    def __init__(self, torch, ops):
        self.torch, self.ops = torch, ops
        g = torch.Generator(device="cuda")
        g.manual_seed(151936)
        n = self.rows * self.cols
        # Three weight copies (496 MB) rotate so the 256 MB MALL cannot hold them.
        self.qs = [torch.randint(-128, 128, (n,), device="cuda", generator=g, dtype=torch.int8)
                   for _ in range(self.copies)]
        self.sc = [(torch.rand(n // 32, device="cuda", generator=g) * 8e-4 + 1e-5)
                   .to(torch.float16).view(torch.int16) for _ in range(self.copies)]
        self.x = torch.randn(self.cols, device="cuda", generator=g)
        self.o = torch.empty(self.rows, device="cuda")
        self.work_per_call = self.rows * self.cols * 34 // 32 + 4 * (self.cols + self.rows)
        self.work_per_step = self.work_per_call
        self.calls_per_step = 1
        self.i = 0

    def call(self, l=0):
        c = self.i % self.copies
        self.i += 1
        self.ops.q8_matvec(None, self.x, self.o, 1, qs=self.qs[c], scales=self.sc[c],
                           n_rows=self.rows, n_cols=self.cols)

    def step(self):
        self.call()

    def config(self):
        return {"workload": f"Q8_0 matvec {self.rows} x {self.cols} (LM head), 1 token",
                "rows": self.rows, "cols": self.cols, "weight_bytes": self.rows * self.cols * 34 // 32}

    def capture(self):
        """The weights, x and output of the last timed call, on the host."""
        self.torch.cuda.synchronize()
        c = (self.i - 1) % self.copies
        blocks = np.empty((self.rows * self.cols // 32, 34), np.uint8)
        blocks[:, :2] = host(self.sc[c]).view(np.uint8).reshape(-1, 2)
        blocks[:, 2:] = host(self.qs[c]).view(np.uint8).reshape(-1, 32)
        self.host = {"packed": blocks.ravel(), "x": host(self.x), "o": host(self.o)}

    def cpu_sample(self, threads):
        """oracle.q8_matvec (coop(64); a serial loop, so 1 thread) of the whole
        head on the last timed call's weights and x, for >= 5 s."""
        import oracle
        h = self.host
        run = lambda: oracle.q8_matvec(h["packed"], h["x"], self.rows, self.cols, 64)
        if self.ref is None:
            self.ref = run()
        n, dt = timed(run, 5.0)
        return n * self.work_per_call, dt, (f"oracle q8_matvec of the whole {self.rows} x "
                                            f"{self.cols} head (the last timed call's weights) "
                                            f"x {n}")

    def parity(self):
        from oracle.parity import metrics
        from oracle import argmax
        h, want = self.host, self.ref
        m = metrics(h["o"], want)
        return parity_entry(
            m, {"argmax_equal": argmax(h["o"]) == argmax(want)},
            "the last timed call's weights, x and output, copied to the host after the timed "
            "region", bit_exact=bool(np.array_equal(h["o"], want)))

    cpu_parallel = False  # the q8 oracle has no parallel loop


class Q8Proj(Workload):
    """The seven Q8_0 projections of every Qwen3-0.6B layer, one decode token,
    28 layers: q 2048x1024, k and v 1024x1024, o 1024x2048, gate and up
    3072x1024, down 1024x3072."""

    data = ("synthetic: random Q8_0 weights of the Qwen3-0.6B shapes (seeded quants, f16 "
            "scales), seeded N(0,1) inputs, zeroed or seeded caches")

    name = "q8proj"
    kernel = "flk_q8_matvec (7 calls per layer; mean over the calls)"
    shapes = [(2048, 1024), (1024, 1024), (1024, 1024), (1024, 2048), (3072, 1024),
              (3072, 1024), (1024, 3072)]
    layers = 28

    def __init__(self, torch, ops):
        self.torch, self.ops = torch, ops
        g = torch.Generator(device="cuda")
        g.manual_seed(28)
        self.w = []
        for _ in range(self.layers):
            for r, c in self.shapes:
                qs = torch.randint(-128, 128, (r * c,), device="cuda", generator=g, dtype=torch.int8)
                sc = (torch.rand(r * c // 32, device="cuda", generator=g) * 8e-4 + 1e-5).to(
                    torch.float16).view(torch.int16)
                self.w.append((qs, sc, r, c))
        self.x = torch.randn(3072, device="cuda", generator=g)
        self.o = torch.empty(3072, device="cuda")
        per = [r * c * 34 // 32 + 4 * (r + c) for r, c in self.shapes]
        self.work_per_step = self.layers * sum(per)
        self.calls_per_step = self.layers * len(self.shapes)
        self.work_per_call = self.work_per_step / self.calls_per_step

    def call(self, i):
        qs, sc, r, c = self.w[i]
        self.ops.q8_matvec(None, self.x, self.o, 1, qs=qs, scales=sc, n_rows=r, n_cols=c)

    def step(self):
        for i in range(self.calls_per_step):
            self.call(i)

    def config(self):
        return {"workload": "Q8_0 projections of 28 Qwen3-0.6B layers (q, k, v, o, gate, up, "
                            "down), 1 decode token", "layers": self.layers,
                "shapes": self.shapes, "weight_bytes": self.layers * sum(
                    r * c * 34 // 32 for r, c in self.shapes)}


def random_q8(rng, rows, cols, scale=8e-4):
    """Q8_0 bytes (34-byte blocks) with random quants and f16 scales."""
    blocks = np.empty((rows * cols // 32, 34), np.uint8)
    blocks[:, :2] = (rng.random(blocks.shape[0]) * scale + 1e-5).astype(
        np.float16).view(np.uint8).reshape(-1, 2)
    blocks[:, 2:] = rng.integers(0, 256, (blocks.shape[0], 32), dtype=np.uint8)
    return blocks.ravel()


class Q8Prefill(Workload):
    """The largest projection of a 2048-token prefill: ffn_norm, then gate and
    up (3072 x 1024 each, rows interleaved) with SwiGLU, in one
    flk_q8_gate_up_swiglu call over 2048 tokens -- the weight-reusing tile
    kernel (q8_mm_kernel), exact to the coop(64) order. VALU-bound: the
    exact summation order rules out MFMA."""

    data = ("synthetic: random Q8_0 weights of the Qwen3-0.6B shapes (seeded quants, f16 "
            "scales), seeded N(0,1) inputs, zeroed or seeded caches")

    name = "q8prefill"
    unit = "TFLOP/s"
    bound = "valu"
    kernel = ("flk_q8_gate_up_swiglu: q8_mm1_kernel<kMmNorm> (32 rows x 8 tokens per tile, "
              "8 row tiles per workgroup)")
    n_tokens, ffn, hid = 2048, 3072, 1024

    def __init__(self, torch, ops):
        self.torch, self.ops = torch, ops
        rng = np.random.default_rng(29)
        gq, gs = ops.q8_split(random_q8(rng, self.ffn, self.hid), self.ffn, self.hid)
        uq, us = ops.q8_split(random_q8(rng, self.ffn, self.hid), self.ffn, self.hid)
        self.w = ops.Q8Matrix(ops.interleave_rows(gq, uq, self.ffn, self.hid),
                              ops.interleave_rows(gs, us, self.ffn, self.hid // 32),
                              2 * self.ffn, self.hid)
        self.x = ops.DeviceBuffer.from_array(
            rng.standard_normal(self.n_tokens * self.hid).astype(np.float32))
        self.gain = ops.DeviceBuffer.from_array((1 + 0.1 * rng.standard_normal(self.hid)).astype(np.float32))
        self.act = ops.DeviceBuffer(self.n_tokens * self.ffn * 4)
        self.work_per_call = 2 * (2 * self.ffn) * self.hid * self.n_tokens  # 2 flops per MAC
        self.work_per_step = self.work_per_call

    def call(self, i=0):
        self.ops.q8_gate_up_swiglu(self.w, self.x, self.act, self.n_tokens, norm_gain=self.gain,
                                   eps=EPS)

    def step(self):
        self.call()

    def config(self):
        return {"workload": "Q8_0 gate+up (2 x 3072 x 1024, interleaved) with ffn_norm in and "
                            "SwiGLU out, 2048 tokens", "rows": 2 * self.ffn, "cols": self.hid,
                "tokens": self.n_tokens}


class Prompt2k(Workload):
    """Time to first token: a 2048-token prompt through flock_amd.model.Model.step
    (embedding, 28 Qwen3-0.6B layers in prefill -- Q8_0 tile projections with
    fused norms and SwiGLU, q/k norm + RoPE + K/V write, fp32-MFMA causal
    attention -- then the head and argmax on the last row, read back)."""

    data = ("synthetic: random Q8_0 weights of the Qwen3-0.6B shapes (seeded quants, f16 "
            "scales), seeded N(0,1) inputs, zeroed or seeded caches")

    name = "prompt2k"
    unit = "tokens/s"
    bound = "mixed"
    kernel = "Model.step(2048 ids): embed, 28 x encodePrefill, lm_head"
    n_tokens = 2048

    def __init__(self, torch, ops):
        from flock_amd.decoder import DecoderConfig
        from flock_amd.model import Model
        self.torch, self.ops = torch, ops
        rng = np.random.default_rng(30)
        cfg = DecoderConfig(maxKeys=self.n_tokens, maxPrefill=self.n_tokens)
        log(f"[{self.name}] building the model (random Q8_0 weights)")
        layers = []
        for _ in range(28):
            w = {n: random_q8(rng, r, c) for n, (r, c) in cfg.shapes().items()}
            for n, sz in (("attn_norm.weight", cfg.hidden), ("ffn_norm.weight", cfg.hidden),
                          ("attn_q_norm.weight", cfg.headDim), ("attn_k_norm.weight", cfg.headDim)):
                w[n] = (1 + 0.1 * rng.standard_normal(sz)).astype(np.float32)
            layers.append(w)
        self.vocab = 151936
        self.model = Model(cfg, layers, random_q8(rng, self.vocab, cfg.hidden, 0.02),
                           (1 + 0.1 * rng.standard_normal(cfg.hidden)).astype(np.float32),
                           self.vocab, max_generate=1)
        del layers
        self.ids = rng.integers(0, self.vocab, self.n_tokens).astype(np.uint32)
        macs = sum(r * c for r, c in cfg.shapes().values())
        n, H, d = self.n_tokens, cfg.nHeads, cfg.headDim
        attn = 4 * H * d * n * (n + 1) // 2  # QK^T and PV over the causal triangle
        self.work_per_call = 28 * (2 * macs * n + attn) + 2 * self.vocab * cfg.hidden
        self.work_per_step = self.work_per_call

    def value(self, ms):
        return self.n_tokens / (ms * 1e-3)

    def call(self, i=0):
        self.model.reset()
        self.model.step(self.ids)

    def step(self):
        self.call()

    def extra(self, ms, call_ms):
        return {"ms_per_prompt": round(ms, 3)}

    def config(self):
        return {"workload": "time to first token: 2048-token prompt at position 0 through 28 "
                            "Qwen3-0.6B layers (prefill) + output norm + LM head + argmax",
                "layers": 28, "tokens": self.n_tokens, "vocab": self.vocab,
                "flops_per_prompt": self.work_per_call}


class Replay32k(Prompt2k):
    """Chunked replay through the whole model (FLOCK_REPLAY_CHUNK = 64): a
    64-id chunk appended at position 32768 onto a 32768-key cache by
    Model.step -- 28 layers of prefill (Q8_0 tile projections, chunk
    attention over the cache with split keys) + head. The caches are zeroed
    once; each step rewinds to position 32768."""

    name = "replay32k"
    kernel = "Model.step(64 ids at position 32768): embed, 28 x encodePrefill, lm_head"
    n_tokens = 64
    n_keys = 32768

    def __init__(self, torch, ops):
        from flock_amd.decoder import DecoderConfig
        from flock_amd.model import Model
        self.torch, self.ops = torch, ops
        rng = np.random.default_rng(31)
        cfg = DecoderConfig(maxKeys=self.n_keys + self.n_tokens, maxPrefill=self.n_tokens)
        log(f"[{self.name}] building the model (random Q8_0 weights)")
        layers = []
        for _ in range(28):
            w = {n: random_q8(rng, r, c) for n, (r, c) in cfg.shapes().items()}
            for n, sz in (("attn_norm.weight", cfg.hidden), ("ffn_norm.weight", cfg.hidden),
                          ("attn_q_norm.weight", cfg.headDim), ("attn_k_norm.weight", cfg.headDim)):
                w[n] = (1 + 0.1 * rng.standard_normal(sz)).astype(np.float32)
            layers.append(w)
        self.vocab = 151936
        self.model = Model(cfg, layers, random_q8(rng, self.vocab, cfg.hidden, 0.02),
                           (1 + 0.1 * rng.standard_normal(cfg.hidden)).astype(np.float32),
                           self.vocab, max_generate=1)
        del layers
        for layer in self.model.layers:
            layer.buf["kcache"].zero()
            layer.buf["vcache"].zero()
        self.ids = rng.integers(0, self.vocab, self.n_tokens).astype(np.uint32)
        macs = sum(r * c for r, c in cfg.shapes().values())
        n, H, d = self.n_tokens, cfg.nHeads, cfg.headDim
        attn = 4 * H * d * sum(self.n_keys + i + 1 for i in range(n))  # QK^T and PV, causal
        self.work_per_call = 28 * (2 * macs * n + attn) + 2 * self.vocab * cfg.hidden
        self.work_per_step = self.work_per_call

    def call(self, i=0):
        m = self.model
        m.nKeys = self.n_keys
        for layer in m.layers:
            layer.nKeys = self.n_keys
        m.step(self.ids)

    def extra(self, ms, call_ms):
        return {"ms_per_chunk": round(ms, 3)}

    def config(self):
        return {"workload": "chunked replay: a 64-id chunk at position 32768 through 28 "
                            "Qwen3-0.6B layers (prefill onto a 32768-key cache) + head",
                "layers": 28, "tokens": self.n_tokens, "n_keys": self.n_keys,
                "vocab": self.vocab, "flops_per_chunk": self.work_per_call}


class Token(Workload):
    """One greedy decode token through all 28 Qwen3-0.6B layers and the head:
    per layer the five DecoderLayer calls (fused projections + the attention
    slice), then flk_lm_head (output norm, tied 151936 x 1024 projection,
    argmax). Random Q8_0 weights, zeroed caches at position n_keys - 1."""

    data = ("synthetic: random Q8_0 weights of the Qwen3-0.6B shapes (seeded quants, f16 "
            "scales), seeded N(0,1) inputs, zeroed or seeded caches")

    unit = "GB/s"
    kernel = ("DecoderLayer.encode x 28 + flk_lm_head (q8_matvec1k_kernel, q8_matvec_kernel, "
              "decode_split/merge, argmax_final_kernel)")
    n_keys = 32769
    layers = 28

    def __init__(self, torch, ops):
        from flock_amd.decoder import DecoderConfig, DecoderLayer
        self.torch, self.ops = torch, ops
        rng = np.random.default_rng(12)
        cfg = DecoderConfig(maxKeys=self.n_keys, maxPrefill=1)
        log(f"[{self.name}] building {self.layers} layers (random Q8_0 weights)")

        def packed(rows, cols):
            blocks = np.empty((rows * cols // 32, 34), np.uint8)
            blocks[:, :2] = (rng.random(blocks.shape[0]) * 8e-4 + 1e-5).astype(
                np.float16).view(np.uint8).reshape(-1, 2)
            blocks[:, 2:] = rng.integers(0, 256, (blocks.shape[0], 32), dtype=np.uint8)
            return blocks.ravel()

        self.L = []
        for _ in range(self.layers):
            w = {n: packed(r, c) for n, (r, c) in cfg.shapes().items()}
            for n, sz in (("attn_norm.weight", cfg.hidden), ("ffn_norm.weight", cfg.hidden),
                          ("attn_q_norm.weight", cfg.headDim), ("attn_k_norm.weight", cfg.headDim)):
                w[n] = (1 + 0.1 * rng.standard_normal(sz)).astype(np.float32)
            layer = DecoderLayer.create(cfg, w)
            layer.buf["kcache"].zero()
            layer.buf["vcache"].zero()
            self.L.append(layer)
        self.vocab, self.hid = 151936, cfg.hidden
        self.head = ops.Q8Matrix.from_packed(packed(self.vocab, self.hid), self.vocab, self.hid)
        self.gout = ops.DeviceBuffer.from_array((1 + 0.1 * rng.standard_normal(self.hid)).astype(np.float32))
        self.normed = ops.DeviceBuffer(self.hid * 4)
        self.tok_v, self.tok_i = ops.DeviceBuffer(4), ops.DeviceBuffer(4)
        self.hws = ops.DeviceBuffer(ops.lm_head_ws_bytes(self.vocab, self.hid))
        self.x = ops.DeviceBuffer.from_array(rng.standard_normal(self.hid).astype(np.float32))
        layer_w = sum(r * c * 34 // 32 for r, c in cfg.shapes().values())
        kv = 2 * self.n_keys * cfg.nKvHeads * cfg.headDim * 4
        self.work_per_call = self.layers * (layer_w + kv) + self.vocab * self.hid * 34 // 32
        self.work_per_step = self.work_per_call
        self.calls_per_step = 1

    def call(self, l=0):
        src = self.x
        for layer in self.L:
            layer.nKeys = self.n_keys - 1
            layer.encode(src=src)
            src = layer.outputBuffer()
        self.ops.lm_head(src, self.gout, EPS, self.head, self.normed, None, self.tok_v, self.tok_i,
                         self.hws)

    def step(self):
        self.call()

    def extra(self, ms, call_ms):
        return {"tokens_per_s": round(1e3 / ms, 2), "ms_per_token": round(ms, 4)}

    def config(self):
        return {"workload": f"greedy decode of one token at position {self.n_keys - 1}: 28 "
                            "Qwen3-0.6B layers (fused Q8_0 projections, norms, SwiGLU, attention "
                            "over the cache) + output norm + LM head + argmax",
                "layers": self.layers, "n_keys": self.n_keys, "hidden": self.hid,
                "vocab": self.vocab, "bytes_per_token": self.work_per_call}


class Token32k(Token):
    name = "token32k"


class Token512(Token):
    name = "token512"
    n_keys = 513


class Gen(Workload):
    """Greedy generation through the whole model with the captured one-token
    HIP graph (flock_amd.model.Model.replay): 28 Qwen3-0.6B layers + head, the
    position, fed-back token and token log on the device. A step is 32 tokens
    decoded from position n_keys - 1 (the caches are rewound between steps)."""

    data = ("synthetic: random Q8_0 weights of the Qwen3-0.6B shapes (seeded quants, f16 "
            "scales), seeded N(0,1) inputs, zeroed or seeded caches")

    unit = "GB/s"
    kernel = "Model.replay: one hipGraphLaunch per token (embed, 28 x 6 kernels, head, advance)"
    n_keys = 32769
    tokens = 32

    def __init__(self, torch, ops):
        from flock_amd.decoder import DecoderConfig
        from flock_amd.model import Model
        self.torch, self.ops = torch, ops
        rng = np.random.default_rng(13)
        cfg = DecoderConfig(maxKeys=self.n_keys + self.tokens, maxPrefill=1)
        log(f"[{self.name}] building the model (random Q8_0 weights)")

        def packed(rows, cols, scale=8e-4):
            blocks = np.empty((rows * cols // 32, 34), np.uint8)
            blocks[:, :2] = (rng.random(blocks.shape[0]) * scale + 1e-5).astype(
                np.float16).view(np.uint8).reshape(-1, 2)
            blocks[:, 2:] = rng.integers(0, 256, (blocks.shape[0], 32), dtype=np.uint8)
            return blocks.ravel()

        layers = []
        for _ in range(28):
            w = {n: packed(r, c) for n, (r, c) in cfg.shapes().items()}
            for n, sz in (("attn_norm.weight", cfg.hidden), ("ffn_norm.weight", cfg.hidden),
                          ("attn_q_norm.weight", cfg.headDim), ("attn_k_norm.weight", cfg.headDim)):
                w[n] = (1 + 0.1 * rng.standard_normal(sz)).astype(np.float32)
            layers.append(w)
        self.vocab = 151936
        self.model = Model(cfg, layers, packed(self.vocab, cfg.hidden, 0.02),
                           (1 + 0.1 * rng.standard_normal(cfg.hidden)).astype(np.float32),
                           self.vocab, max_generate=self.tokens)
        del layers
        for layer in self.model.layers:
            layer.buf["kcache"].zero()
            layer.buf["vcache"].zero()
        layer_w = sum(r * c * 34 // 32 for r, c in cfg.shapes().values())
        kv = 2 * self.n_keys * cfg.nKvHeads * cfg.headDim * 4
        self.work_per_token = 28 * (layer_w + kv) + self.vocab * cfg.hidden * 34 // 32
        self.work_per_step = self.tokens * self.work_per_token
        self.work_per_call = self.work_per_step
        self.calls_per_step = 1

    def call(self, l=0):
        m = self.model
        m.nKeys = self.n_keys - 1
        m.replay(17, self.tokens, read=False)

    def step(self):
        self.call()

    def extra(self, ms, call_ms):
        return {"tokens_per_s": round(self.tokens * 1e3 / ms, 2),
                "ms_per_token": round(ms / self.tokens, 4)}

    def config(self):
        return {"workload": f"greedy generation, {self.tokens} tokens per step from position "
                            f"{self.n_keys - 1}: 28 Qwen3-0.6B layers + head per token, one HIP "
                            "graph replay per token", "layers": 28, "n_keys": self.n_keys,
                "tokens_per_step": self.tokens, "vocab": self.vocab,
                "bytes_per_token": self.work_per_token}


class Gen32k(Gen):
    name = "gen32k"


class Gen512(Gen):
    name = "gen512"
    n_keys = 513


WORKLOADS = {c.name: c for c in (Decode32k, Prefill2k, Ragged, Chunk32k, Decode512, Copy,
                                 Q8LmHead, Q8Proj, Q8Prefill, Prompt2k, Replay32k, Token32k,
                                 Token512, Gen32k, Gen512)}


def settle_clocks(torch, w, seconds=0.5):
    """Untimed steps until `seconds` have passed, so the GPU is at its working
    clock when the W warmup steps start (an idle GPU drops its clocks; the CPU
    baselines and input generation leave it idle or differently loaded)."""
    t0 = time.perf_counter()
    while time.perf_counter() - t0 < seconds:
        w.step()
        torch.cuda.synchronize()


def measure(torch, stream, w, steps, warmup, calls=None):
    """(ms per step, host wall ms per step, ms per dominant call)."""
    settle_clocks(torch, w)
    for _ in range(warmup):
        w.step()
    torch.cuda.synchronize()
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    start.record(stream)
    t0 = time.perf_counter()
    for _ in range(steps):
        w.step()
    end.record(stream)
    torch.cuda.synchronize()
    wall_ms = (time.perf_counter() - t0) * 1e3 / steps
    ms = start.elapsed_time(end) / steps
    if w.graph_step:  # the calls are only launched inside the graph
        return ms, wall_ms, ms / w.calls_per_step
    # Dominant call: R back-to-back calls between two events.
    calls = calls or max(steps * w.calls_per_step, 20)
    torch.cuda.synchronize()
    start.record(stream)
    for i in range(calls):
        w.call(i % w.calls_per_step)
    end.record(stream)
    torch.cuda.synchronize()
    call_ms = start.elapsed_time(end) / calls
    return ms, wall_ms, call_ms


def run(torch, ops, stream, name, steps, warmup):
    """Measure one workload; returns its JSON fields and its CPU-baseline thunk."""
    w = WORKLOADS[name](torch, ops)
    torch.cuda.synchronize()
    log(f"[{name}] warmup {warmup}, timing {steps} steps")
    ms, wall_ms, call_ms = measure(torch, stream, w, steps, warmup)
    value = w.value(ms)
    log(f"[{name}] {ms:.3f} ms/step (host wall {wall_ms:.3f}), {value:.2f} {w.unit}; "
        f"dominant call {call_ms * 1e3:.2f} us")
    out = {"value": round(value, 3), "unit": w.unit, "ms_per_step": round(ms, 4),
           "data": w.data, "config": w.config(),
           "roofline": w.roofline(call_ms, traffic_from_profiles(f"{name}_pmc.md"))}
    if hasattr(w, "extra"):
        out.update(w.extra(ms, call_ms))
    if hasattr(w, "prologue_line"):
        w.step_ms = ms
        out.update(w.prologue_line(torch, stream))
    w.capture()  # host copies of the timed inputs and outputs for the CPU leg
    # Drop the device buffers; the CPU leg needs only the host copies.
    if getattr(w, "graph", None) is not None:
        w.graph.free()
        w.graph = None
    if hasattr(w, "model"):
        w.model.free()
    for k in [k for k, v in vars(w).items()
              if isinstance(v, (torch.Tensor, list, ops.Workspace, ops.DeviceBuffer, ops.Q8Matrix))
              or k == "model"]:
        delattr(w, k)
    ops.sync()  # also releases the dropped buffers
    torch.cuda.empty_cache()
    return out, w.cpu_leg


def main():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--workload", default="decode32k", choices=sorted(WORKLOADS))
    ap.add_argument("--no-cpu-baseline", action="store_true",
                    help="skip the CPU baseline timing (the parity check still runs)")
    ap.add_argument("--no-parity", action="store_true",
                    help="skip the whole CPU leg: no CPU baseline and no parity check")
    ap.add_argument("--no-secondary", action="store_true",
                    help="measure only the main workload (the default run also measures "
                         "prefill2k, decode512, ragged, chunk32k, q8lmhead, gen32k, prompt2k)")
    args = ap.parse_args()

    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print(f"bench.py measures one GPU (asked for --gpus {args.gpus}): flock_amd's attention "
              "path runs on a single MI355X and has no multi-GPU mode. Run with --gpus 1.",
              file=sys.stderr)
        sys.exit(2)

    import torch
    from flock_amd import ops

    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        sys.exit(1)
    stream = torch.cuda.Stream()
    ops.set_stream(stream)
    with torch.cuda.stream(stream):
        main_res, main_cpu = run(torch, ops, stream, args.workload, args.steps, args.warmup)
        out = {"metric": METRIC, "value": main_res["value"], "unit": main_res["unit"],
               "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
               "ms_per_step": main_res["ms_per_step"], "higher_is_better": True,
               "scaling": "weak", "vs_baseline": None, "dtype": "f32",
               "data": main_res["data"],
               "config": main_res["config"], "roofline": main_res["roofline"]}
        for k in ("tokens_per_s", "ms_per_token"):
            if k in main_res:
                out[k] = main_res[k]
        if main_res["unit"] == "GB/s":
            out["frac_of_hbm_peak"] = round(main_res["value"] / HBM_PEAK_GBS, 4)
        elif main_res["unit"] == "TFLOP/s" and main_res["roofline"]["bound"] == "mfma":
            out["frac_of_fp32_mfma_peak"] = round(main_res["value"] / FP32_MFMA_PEAK_TFLOPS, 4)
        elif main_res["unit"] == "TFLOP/s":
            out["frac_of_fp32_vector_peak"] = round(main_res["value"] / FP32_VECTOR_PEAK_TFLOPS, 4)
        for k in ("ms_per_prompt", "ms_per_chunk"):
            if k in main_res:
                out[k] = main_res[k]
        # The other benchmark workloads and the rows next to the path,
        # each with its own roofline (and CPU baseline where it has one).
        secondary = []
        if args.workload == "decode32k" and not args.no_secondary:
            for key, name, steps, warm in (
                    ("prefill", "prefill2k", max(5, args.steps), args.warmup),
                    ("decode512", "decode512", max(20, args.steps), args.warmup),
                    ("ragged", "ragged", max(5, args.steps // 2), args.warmup),
                    ("chunk32k", "chunk32k", max(5, args.steps // 2), args.warmup),
                    ("q8_lm_head", "q8lmhead", max(5, args.steps), args.warmup),
                    ("generate", "gen32k", 5, 2),
                    ("prompt", "prompt2k", 3, 1)):
                res, cpu = run(torch, ops, stream, name, steps, warm)
                b = res["roofline"]["bound"]
                if res["unit"] == "GB/s":
                    res["frac_of_hbm_peak"] = round(res["value"] / HBM_PEAK_GBS, 4)
                elif res["unit"] == "TFLOP/s" and b == "mfma":
                    res["frac_of_fp32_mfma_peak"] = round(res["value"] / FP32_MFMA_PEAK_TFLOPS, 4)
                out[key] = res
                secondary.append((key, name, cpu))
    # The CPU leg last, with the GPU measurements done: the oracle on the
    # timed inputs, as the CPU baseline and as the parity check.
    if not args.no_parity:
        baseline = not args.no_cpu_baseline
        for key, name, cpu in [(None, args.workload, main_cpu)] + secondary:
            log(f"[{name}] CPU leg: oracle on the timed inputs"
                f"{' (baseline + parity)' if baseline else ' (parity)'}")
            cb, par = cpu(baseline)
            dst = out if key is None else out[key]
            if cb is not None:
                dst["cpu_baseline"] = cb
            if par is not None:
                dst["parity"] = par
                log(f"[{name}] parity: {par['clause']}, max_abs {par.get('max_abs')}, "
                    f"rel {par.get('rel')}")
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
