#!/usr/bin/env python3
"""tiler-hip benchmark on one MI355X.

A "step" is one launch of the hot path over one batch of synthetic input that
is already resident in HBM.  The headline line measures BASELINE.json's metric
on configs[1] (RMS normalization, bf16 [8192 x 4096], w bf16 [4096], eps 1e-5,
f32 accumulation, bf16 output) as achieved HBM GB/s of algorithmic bytes; the
other four configs are measured the same way and reported under "families".

Measurement rules: fixed seeds; input/output buffer sets are rotated so more
than the 256 MB Infinity Cache is touched per sweep; W untimed warm-up
launches and at least SETTLE_S of untimed graph replays, then K back-to-back
launches (one graph replay) between HIP events recorded on the context stream
the kernels run on (median/p10/p90 from an eager pass with per-launch event
pairs).  The CPU baseline is the oracle's restatement of
the reference loops (strict binary32 folds, no FMA) on the GPU box's host,
single-threaded, on a bounded sample.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload NAME]
                       [--no-families] [--no-cpu-baseline] [--calibration-copy]
                       [--vendor-gemm] [--no-reference-cells]

"reference_cells" times this library on the reference's own published
benchmark cells (its strict f32 contraction cells and its reduction dispatch
crossover cells), each beside the reference's Apple-GPU figure.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0          # MI355X HBM3E, GB/s
# Host threads for the CPU baseline: the GPU box's CPU share per GPU is 16,
# whatever os.cpu_count() reports there.
CPU_THREADS = max(1, min(16, int(os.environ.get("OMP_NUM_THREADS", "0") or 0) or (os.cpu_count() or 1)))
MFMA_BF16_PEAK_TFLOPS = 2500.0  # dense bf16 MFMA, TFLOP/s
EPS_BITS = 0x3727C5AC           # 1e-5 as binary32 (config eps)
SETTLE_S = 0.05                 # untimed graph replays before the timed one
METRIC = "achieved HBM GB/s (% peak) for RMSNorm/softmax/gather; bf16 GEMM TFLOP/s"


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def to_bf16(x: np.ndarray) -> np.ndarray:
    """binary32 -> bf16 bit patterns, round to nearest even (NaN -> 0x7fc0):
    synthetic-input generation only (the oracle stays the checker)."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32)
    r = ((u + (np.uint32(0x7FFF) + ((u >> 16) & np.uint32(1)))) >> 16).astype(np.uint16)
    return np.where(np.isnan(x), np.uint16(0x7FC0), r)


class Workload:
    name = ""
    kernel = ""  # the dominant kernel, whose measured HBM traffic is reported
    bound = "hbm"
    unit = "GB/s"

    def __init__(self, ctx):
        self.ctx = ctx
        self.buffers = []

    def _keep(self, *bufs):
        self.buffers.extend(bufs)
        return bufs if len(bufs) > 1 else bufs[0]

    def teardown(self):
        for b in self.buffers:
            b.free()
        self.buffers = []


class RmsNorm(Workload):
    """RMS normalization over rows."""
    name = "rms_norm"
    kernel = "tiler_rms_norm_bf16_ch8_full"
    rows, extent = 8192, 4096
    sets = 6  # 6 x 128 MiB touched per sweep

    def config(self):
        return {"workload": "rms_norm bf16 [8192 x 4096] x w[4096] eps=1e-5, f32 accumulation, bf16 out",
                "rows": self.rows, "hidden": self.extent, "storage": "bf16", "eps_bits": hex(EPS_BITS),
                "buffer_sets": self.sets}

    def work(self):  # algorithmic bytes per launch
        return self.rows * self.extent * 2 * 2 + self.extent * 2

    def setup(self):
        from tiler_amd import _lib as L
        self.L = L
        rng = np.random.default_rng(1)
        w = to_bf16(rng.normal(1.0, 0.1, self.extent).astype(np.float32))
        self.w = self._keep(self.ctx.to_device(w))
        self.sets_ = []
        for s in range(self.sets):
            x = to_bf16(rng.standard_normal((self.rows, self.extent), dtype=np.float32))
            self.sets_.append(self._keep(self.ctx.to_device(x), self.ctx.alloc(x.nbytes)))
        return len(self.sets_)

    def launch(self, i):
        x, y = self.sets_[i % len(self.sets_)]
        self.ctx.rms_norm(self.L.BF16, x, self.w, self.rows, self.extent, EPS_BITS, y,
                          weight_broadcast=True)

    def cpu_baseline(self, budget_s):
        """The oracle's strict RMSNorm (widen, normalize, narrow) on whole rows:
        timed on one thread for half the budget, then on CPU_THREADS threads
        (independent 512-row blocks; the oracle is plain C called through
        ctypes, which releases the GIL) for the other half.  The threaded
        figure is the baseline; the single-thread one is reported beside it."""
        import oracle
        from concurrent.futures import ThreadPoolExecutor
        rows = 512
        wb = oracle.bf16_narrow(np.random.default_rng(7).normal(1.0, 0.1, self.extent).astype(np.float32))
        wfull = np.broadcast_to(oracle.bf16_widen(wb), (rows, self.extent)).copy()

        def worker(seed, seconds):
            xb = oracle.bf16_narrow(np.random.default_rng(seed).standard_normal((rows, self.extent),
                                                                                dtype=np.float32))
            done, t0 = 0, time.perf_counter()
            while True:
                y = oracle.rms_norm_f32(oracle.bf16_widen(xb), wfull, (rows, self.extent), 1, EPS_BITS)
                oracle.bf16_narrow(y)
                done += rows
                if time.perf_counter() - t0 >= seconds:
                    return done

        def rate(done_rows, seconds):
            return (done_rows * self.extent * 4 + self.extent * 2) / seconds / 1e9

        t0 = time.perf_counter()
        single = worker(7, budget_s / 2)
        single_s = time.perf_counter() - t0
        threads = CPU_THREADS
        t0 = time.perf_counter()
        with ThreadPoolExecutor(threads) as pool:
            done = sum(pool.map(lambda i: worker(100 + i, budget_s / 2), range(threads)))
        threaded_s = time.perf_counter() - t0
        return {"value": rate(done, threaded_s), "unit": "GB/s", "cores": threads, "kind": "port",
                "sample": f"{done} rows x {self.extent} of the config in {threaded_s:.1f} s on {threads} threads "
                          "(oracle rms_norm_f32 over widened bf16, then narrowing; independent 512-row blocks)",
                "single_thread": {"value": rate(single, single_s), "unit": "GB/s", "cores": 1,
                                  "sample": f"{single} rows in {single_s:.1f} s"}}


class RmsNormStrict(RmsNorm):
    """configs[1] under the strict contract (no PERMITS_REASSOCIATION): the
    reference's serial fold of the squares, bit for bit with
    rms_norm.rs:134-195 on the exactly widened values (the rows held in
    registers, tiler_rms_norm_bf16_strict_rr8_p16), realized through
    tiler_hip_realize and run through the RuntimeAdapter stages."""
    name = "rms_norm_strict"
    kernel = "tiler_rms_norm_bf16_strict_rr8_p16"

    def config(self):
        c = super().config()
        c["workload"] += ", strict contract (serial fold of the squares in the reference's order)"
        return c

    def setup(self):
        from tiler_amd import _lib as L
        from tiler_amd.realize import prepare_route, realize
        n = super().setup()
        rz = realize(L.PROGRAM_RMS_NORM, (self.rows, self.extent), dtype=L.BF16, scalars=(EPS_BITS,),
                     flags=L.REGION_ALIGNED16 | L.REGION_OPERAND_BROADCAST, ctx=self.ctx)
        if rz.symbols != [self.kernel]:
            raise RuntimeError(f"strict rms_norm realized as {rz.symbols}, not {self.kernel}")
        self.plans = [prepare_route(self.ctx, rz, [x, self.w, y]) for x, y in self.sets_]
        return n

    def launch(self, i):
        self.plans[i % len(self.plans)].enqueue()

    def teardown(self):
        for pl in getattr(self, "plans", []):
            pl.release()
        self.plans = []
        super().teardown()


class Sum(Workload):
    """f32[2^24] -> scalar, the two-level tree."""
    name = "sum"
    kernel = "tiler_sum_f32_grid"
    n = 1 << 24
    sets = 6

    def config(self):
        out = {"workload": "serial-sum f32[2^24] ~U[-1,1] -> f32 scalar (two-level tree)",
               "buffer_sets": self.sets}
        if hasattr(self, "conditioning"):
            out["conditioning"] = self.conditioning
        return out

    def work(self):
        return self.n * 4 + 4

    def setup(self):
        rng = np.random.default_rng(0)
        self.xs = []
        for s in range(self.sets):
            x = rng.uniform(-1, 1, self.n).astype(np.float32)
            if s == 0:
                # Condition of the sum: sum|x| / |sum x| (f64), and the device's
                # relative error on this set against the f64 sum.
                exact = float(np.sum(x, dtype=np.float64))
                self.conditioning = {"set": 0, "sum_f64": exact,
                                     "sum_abs_f64": float(np.sum(np.abs(x), dtype=np.float64)),
                                     "condition_number": float(np.sum(np.abs(x), dtype=np.float64)) / abs(exact)}
            self.xs.append(self._keep(self.ctx.to_device(x)))
        self.out = self._keep(self.ctx.alloc(4))
        from tiler_amd import _lib as L
        # the reassociating tree: the sum under a REASSOCIATE_F32 contract
        self.topology = L.SUM_TREE
        self.ctx.sum_f32(self.xs[0], 1, self.n, self.out, topology=self.topology)
        got = float(self.out.download(np.float32, (1,))[0])
        exact = self.conditioning["sum_f64"]
        self.conditioning["device_sum"] = got
        self.conditioning["relative_error_vs_f64"] = abs(got - exact) / abs(exact)
        return self.sets

    def launch(self, i):
        self.ctx.sum_f32(self.xs[i % self.sets], 1, self.n, self.out, topology=self.topology)

    def cpu_baseline(self, budget_s):
        import oracle
        x = np.random.default_rng(0).uniform(-1, 1, self.n).astype(np.float32)
        done, t0 = 0, time.perf_counter()
        while True:
            oracle.strict_sum(x, (self.n,), 0)
            done += 1
            el = time.perf_counter() - t0
            if el >= budget_s:
                break
        return {"value": done * self.work() / el / 1e9, "unit": "GB/s", "cores": 1, "kind": "port",
                "sample": f"{done} x strict_sum over 2^24 in {el:.1f} s, single thread"}


class Softmax(Workload):
    """f32 [32 x 2048 x 2048] softmax over the last axis."""
    name = "softmax"
    kernel = "tiler_softmax_f32_ch8_full"
    rows, extent = 32 * 2048, 2048
    sets = 2

    def config(self):
        return {"workload": "softmax f32 [32 x 2048 x 2048] ~N(0,3), last axis", "buffer_sets": self.sets}

    def work(self):
        return self.rows * self.extent * 4 * 2

    def setup(self):
        rng = np.random.default_rng(3)
        self.sets_ = []
        for _ in range(self.sets):
            x = rng.standard_normal((self.rows, self.extent), dtype=np.float32) * np.float32(3.0)
            self.sets_.append(self._keep(self.ctx.to_device(x), self.ctx.alloc(x.nbytes)))
        return self.sets

    def launch(self, i):
        x, y = self.sets_[i % self.sets]
        self.ctx.softmax_f32(x, self.rows, self.extent, y)

    def cpu_baseline(self, budget_s):
        import oracle
        rows = 256
        x = np.random.default_rng(3).standard_normal((rows, self.extent), dtype=np.float32) * np.float32(3.0)
        done, t0 = 0, time.perf_counter()
        while True:
            oracle.softmax_f32(x, (rows, self.extent), 1)
            done += rows
            el = time.perf_counter() - t0
            if el >= budget_s:
                break
        return {"value": done * self.extent * 8 / el / 1e9, "unit": "GB/s", "cores": 1, "kind": "port",
                "sample": f"{done} rows x {self.extent} in {el:.1f} s, single thread (certified exp)"}


class SoftmaxStrict(Workload):
    """configs[2]'s shape under the strict contract (no PERMITS_REASSOCIATION):
    the reference's serial exponent sum, bit for bit with softmax.rs:237-315
    (the rows held in registers, tiler_softmax_f32_strict_rr8_p16), realized
    through tiler_hip_realize and run through the RuntimeAdapter stages."""
    name = "softmax_strict"
    kernel = "tiler_softmax_f32_strict_rr8_p16"
    rows, extent = 32 * 2048, 2048
    sets = 2

    def config(self):
        return {"workload": "softmax f32 [32 x 2048 x 2048] ~N(0,3), last axis, strict contract "
                            "(serial exponent sum in the reference's order)", "buffer_sets": self.sets}

    def work(self):
        return self.rows * self.extent * 4 * 2

    def setup(self):
        from tiler_amd import _lib as L
        from tiler_amd.realize import prepare_route, realize
        rz = realize(L.PROGRAM_SOFTMAX, (self.rows, self.extent), flags=L.REGION_ALIGNED16, ctx=self.ctx)
        if rz.symbols != [self.kernel]:
            raise RuntimeError(f"strict softmax realized as {rz.symbols}, not {self.kernel}")
        rng = np.random.default_rng(3)
        self.plans = []
        for _ in range(self.sets):
            x = rng.standard_normal((self.rows, self.extent), dtype=np.float32) * np.float32(3.0)
            bufs = self._keep(self.ctx.to_device(x), self.ctx.alloc(x.nbytes))
            self.plans.append(prepare_route(self.ctx, rz, list(bufs)))
        return self.sets

    def launch(self, i):
        self.plans[i % self.sets].enqueue()

    def teardown(self):
        for pl in getattr(self, "plans", []):
            pl.release()
        self.plans = []
        super().teardown()

    def cpu_baseline(self, budget_s):
        return Softmax(self.ctx).cpu_baseline(budget_s)  # the oracle's softmax is the strict fold


class SoftmaxDecode(Workload):
    """Few long rows: f32 [32 heads x 131072 keys] softmax over the keys (the
    shape of decode-attention scores).  16 segments a row, 512 workgroups:
    the row-synchronized form runs (one launch, x read once); 16 buffer sets
    (512 MiB) keep the working set out of the 256 MB last-level cache."""
    name = "softmax_decode"
    kernel = "tiler_softmax_f32_rowsync_a"
    rows, extent = 32, 131072
    sets = 16

    def config(self):
        return {"workload": "softmax f32 [32 x 131072] ~N(0,3), last axis (split rows)",
                "buffer_sets": self.sets}

    def work(self):
        return self.rows * self.extent * 4 * 2

    def setup(self):
        rng = np.random.default_rng(4)
        self.sets_ = []
        for _ in range(self.sets):
            x = rng.standard_normal((self.rows, self.extent), dtype=np.float32) * np.float32(3.0)
            self.sets_.append(self._keep(self.ctx.to_device(x), self.ctx.alloc(x.nbytes)))
        return self.sets

    def launch(self, i):
        x, y = self.sets_[i % self.sets]
        self.ctx.softmax_f32(x, self.rows, self.extent, y)

    def cpu_baseline(self, budget_s):
        import oracle
        x = np.random.default_rng(4).standard_normal((2, self.extent), dtype=np.float32) * np.float32(3.0)
        done, t0 = 0, time.perf_counter()
        while True:
            oracle.softmax_f32(x, (2, self.extent), 1)
            done += 2
            el = time.perf_counter() - t0
            if el >= budget_s:
                break
        return {"value": done * self.extent * 8 / el / 1e9, "unit": "GB/s", "cores": 1, "kind": "port",
                "sample": f"{done} rows x {self.extent} in {el:.1f} s, single thread (certified exp)"}


class Gather(Workload):
    """tied embedding gather."""
    name = "gather"
    kernel = "tiler_gather_u128"
    vocab, hidden, count = 128256, 4096, 16384
    sets = 6

    def config(self):
        return {"workload": "gather bf16 [128256 x 4096] by int32[16384] -> bf16 [16384 x 4096]",
                "index_sets": self.sets}

    def work(self):
        return self.count * self.hidden * 2 * 2 + self.count * 4

    def setup(self):
        rng = np.random.default_rng(4)
        table = np.empty((self.vocab, self.hidden), np.uint16)
        for lo in range(0, self.vocab, 16384):
            hi = min(self.vocab, lo + 16384)
            table[lo:hi] = to_bf16(
                rng.standard_normal((hi - lo, self.hidden), dtype=np.float32) * np.float32(0.02))
        self.table = self._keep(self.ctx.to_device(table))
        del table
        self.idx = [self._keep(self.ctx.to_device(rng.integers(0, self.vocab, self.count).astype(np.int32)))
                    for _ in range(self.sets)]
        self.outs = [self._keep(self.ctx.alloc(self.count * self.hidden * 2)) for _ in range(2)]
        return self.sets

    def launch(self, i):
        self.ctx.gather(self.table, 1, self.vocab, self.hidden, 2, self.idx[i % self.sets], self.count,
                        self.outs[i % 2], index_signed=True)

    def cpu_baseline(self, budget_s):
        import oracle
        rng = np.random.default_rng(4)
        vocab = 8192
        table = rng.integers(0, 65535, (vocab, self.hidden), dtype=np.uint16)
        idx = rng.integers(0, vocab, self.count).astype(np.int32)
        done, t0 = 0, time.perf_counter()
        while True:
            oracle.gather(table.reshape(-1), 1, vocab, self.hidden, idx.view(np.uint32), index_signed=True)
            done += 1
            el = time.perf_counter() - t0
            if el >= budget_s:
                break
        return {"value": done * self.work() / el / 1e9, "unit": "GB/s", "cores": 1, "kind": "port",
                "sample": f"{done} x {self.count}-row gather (table of {vocab} rows) in {el:.1f} s"}


class Contract(Workload):
    """bf16 4096^3 contraction with fused SiLU."""
    name = "contract"
    kernel = "tiler_contract_bf16_silu_t256_kf"
    bound = "mfma"
    unit = "TFLOP/s"
    m = n = k = 4096
    sets = 4

    def config(self):
        return {"workload": "contraction bf16 A[4096x4096] . B[4096x4096]^T, f32 acc, fused SiLU, bf16 C",
                "buffer_sets": self.sets}

    def work(self):  # flops per launch
        return 2 * self.m * self.n * self.k

    def operands(self):
        """The seeded bf16 operand sets (A [m,k], B [n,k]) every leg uses."""
        rng = np.random.default_rng(5)
        for _ in range(self.sets):
            a = to_bf16(rng.standard_normal((self.m, self.k), dtype=np.float32) / np.float32(64.0))
            b = to_bf16(rng.standard_normal((self.n, self.k), dtype=np.float32) / np.float32(64.0))
            yield a, b

    def setup(self):
        from tiler_amd import _lib as L
        self.L = L
        self.sets_ = []
        for a, b in self.operands():
            self.sets_.append(self._keep(self.ctx.to_device(a), self.ctx.to_device(b),
                                         self.ctx.alloc(self.m * self.n * 2)))
        return self.sets

    def vendor_reference(self, steps, warmup):
        """The vendor library's bf16 GEMM on the same operands, for comparison
        only: torch.matmul(A, B^T) (hipBLASLt), no epilogue, bf16 out, its
        K launches captured in a torch CUDA graph, settled, and one replay
        timed between events on torch's stream."""
        import torch
        dev = torch.device("cuda", 0)
        sets = [(torch.from_numpy(a.view(np.int16)).to(dev).view(torch.bfloat16),
                 torch.from_numpy(b.view(np.int16)).to(dev).view(torch.bfloat16))
                for a, b in self.operands()]
        outs = [torch.empty((self.m, self.n), device=dev, dtype=torch.bfloat16) for _ in sets]

        def run(i):
            a, b = sets[i % len(sets)]
            torch.matmul(a, b.t(), out=outs[i % len(sets)])
        for i in range(warmup):
            run(i)
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            for i in range(steps):
                run(i)
        t_settle = time.perf_counter()
        while time.perf_counter() - t_settle < SETTLE_S:
            g.replay()
            torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        g.replay()
        e1.record()
        e1.synchronize()
        ms = e0.elapsed_time(e1) / steps
        return {"library": f"hipBLASLt via torch.matmul(A, B^T) (torch {torch.__version__})",
                "epilogue": "none", "value": self.work() / (ms / 1e3) / 1e12, "unit": "TFLOP/s",
                "ms_per_step": ms, "steps": steps}

    def launch(self, i):
        a, b, c = self.sets_[i % self.sets]
        self.ctx.contract_bf16(a, b, self.m, self.n, self.k, c, self.L.EPILOGUE_SILU)

    def cpu_baseline(self, budget_s):
        import oracle
        rng = np.random.default_rng(5)
        a = rng.standard_normal((self.m, self.k), dtype=np.float32) / np.float32(64.0)
        b = rng.standard_normal((self.n, self.k), dtype=np.float32) / np.float32(64.0)
        done, rows, t0 = 0, 2, time.perf_counter()
        while True:
            oracle.contract_strict_f32(a[done % self.m:done % self.m + rows], b, rows, self.n, self.k,
                                       threads=1)
            done += rows
            el = time.perf_counter() - t0
            if el >= budget_s:
                break
        flops = 2.0 * done * self.n * self.k
        return {"value": flops / el / 1e12, "unit": "TFLOP/s", "cores": 1, "kind": "port",
                "sample": f"{done} output rows of the strict f32 fold (x{self.n}, k={self.k}) in {el:.1f} s, "
                          "single thread; extrapolated per row"}


class Convert(Workload):
    """The binary32 -> bf16 narrowing family (ADR 0091 decision 2) over
    f32[2^26]: not a BASELINE config, measured as a family of its own."""
    name = "convert"
    kernel = "tiler_narrow_f32_bf16_v8"
    n = 1 << 26
    sets = 2  # 2 x 384 MiB touched per sweep

    def config(self):
        return {"workload": "narrow f32[2^26] ~N(0,1) -> bf16 (RNE, canonical NaN)", "buffer_sets": self.sets}

    def work(self):  # algorithmic bytes per launch
        return self.n * 4 + self.n * 2

    def setup(self):
        from tiler_amd import _lib as L
        self.L = L
        rng = np.random.default_rng(6)
        self.sets_ = [self._keep(self.ctx.to_device(rng.standard_normal(self.n, dtype=np.float32)),
                                 self.ctx.alloc(self.n * 2)) for _ in range(self.sets)]
        return self.sets

    def launch(self, i):
        x, y = self.sets_[i % self.sets]
        self.ctx.convert(self.L.CONVERT_NARROW_F32_BF16, x, self.n, y)

    def cpu_baseline(self, budget_s):
        import oracle
        x = np.random.default_rng(6).standard_normal(1 << 22, dtype=np.float32)
        done, t0 = 0, time.perf_counter()
        while time.perf_counter() - t0 < budget_s:
            oracle.bf16_narrow(x)
            done += x.size
        el = time.perf_counter() - t0
        return {"value": done * 6 / el / 1e9, "unit": "GB/s", "cores": 1, "kind": "port",
                "sample": f"{done} elements of the oracle's narrowing in {el:.1f} s, single thread"}


class Expression(Workload):
    """A pointwise f32 expression DAG (ScalarProgram::PointwiseF32) over three
    inputs of f32[2^26]: y = (x0 * x1 + x2) * 0.5, one rounding per node, one
    fused launch.  Not a BASELINE config, measured as a family of its own."""
    name = "expression"
    kernel = "tiler_expr_f32_r16_i3"
    n = 1 << 26
    sets = 2  # 2 x 1 GiB touched per sweep
    nodes = [(0, 0, 0), (0, 1, 0), (0, 2, 0), (3, 0, 1), (2, 3, 2), (1, 0x3F000000, 0), (3, 4, 5)]

    def config(self):
        return {"workload": "f32 expression y = (x0 * x1 + x2) * 0.5 over 3 x f32[2^26] ~N(0,1)",
                "nodes": len(self.nodes), "inputs": 3, "buffer_sets": self.sets}

    def work(self):  # algorithmic bytes per launch: three inputs read, one output written
        return self.n * 4 * 4

    def setup(self):
        from tiler_amd import _lib as L
        self.L = L
        rng = np.random.default_rng(8)
        self.sets_ = []
        for _ in range(self.sets):
            ins = [self._keep(self.ctx.to_device(rng.standard_normal(self.n, dtype=np.float32))) for _ in range(3)]
            self.sets_.append((ins, self._keep(self.ctx.alloc(self.n * 4))))
        return self.sets

    def launch(self, i):
        ins, y = self.sets_[i % self.sets]
        self.ctx.expression(self.L.F32, self.nodes, ins, self.n, y)

    def cpu_baseline(self, budget_s):
        import oracle
        rng = np.random.default_rng(8)
        xs = [rng.standard_normal(1 << 20, dtype=np.float32) for _ in range(3)]
        done, t0 = 0, time.perf_counter()
        while time.perf_counter() - t0 < budget_s:
            oracle.expression_f32(self.nodes, xs)
            done += xs[0].size
        el = time.perf_counter() - t0
        return {"value": done * 16 / el / 1e9, "unit": "GB/s", "cores": 1, "kind": "port",
                "sample": f"{done} elements of the oracle's expression evaluator in {el:.1f} s, single thread"}


class Dequantize(Workload):
    """Strict-affine U4 -> f32 dequantization (ScalarProgram::
    StrictAffineU4Dequantize) of 2^28 codes packed LSB-first: 0.5 B read and
    4 B written per element.  Not a BASELINE config, measured as a family of
    its own."""
    name = "dequantize"
    kernel = "tiler_dequantize_u4_f32_w"
    n = 1 << 28
    scale_bits, zero_point = 0x3C23D70A, 8  # 0.01, zero point 8
    sets = 2  # 2 x 1.125 GiB touched per sweep

    def config(self):
        return {"workload": "dequantize strict-affine U4[2^28] (packed LSB-first, uniform codes) -> f32, "
                            "scale 0.01, zero point 8", "buffer_sets": self.sets}

    def work(self):  # algorithmic bytes per launch
        return self.n // 2 + self.n * 4

    def setup(self):
        rng = np.random.default_rng(9)
        self.sets_ = [self._keep(self.ctx.to_device(rng.integers(0, 256, self.n // 2, dtype=np.uint8)),
                                 self.ctx.alloc(self.n * 4)) for _ in range(self.sets)]
        return self.sets

    def launch(self, i):
        codes, y = self.sets_[i % self.sets]
        self.ctx.dequantize_u4(codes, self.n, self.scale_bits, self.zero_point, y)

    def cpu_baseline(self, budget_s):
        import oracle
        packed = np.random.default_rng(9).integers(0, 256, 1 << 21, dtype=np.uint8)
        done, t0 = 0, time.perf_counter()
        while time.perf_counter() - t0 < budget_s:
            oracle.dequantize_u4(packed, packed.size * 2, self.scale_bits, self.zero_point)
            done += packed.size * 2
        el = time.perf_counter() - t0
        return {"value": done * 4.5 / el / 1e9, "unit": "GB/s", "cores": 1, "kind": "port",
                "sample": f"{done} elements of the oracle's dequantization in {el:.1f} s, single thread"}


WORKLOADS = {w.name: w for w in (RmsNorm, RmsNormStrict, Sum, Softmax, SoftmaxStrict, SoftmaxDecode, Gather,
                                 Contract, Convert, Expression, Dequantize)}


TRAFFIC_FILE = os.path.join(ROOT, "profiles", "hbm_traffic_all_families.md")


def measured_traffic() -> dict:
    """Calibrated HBM bytes per launch by kernel, from the committed rocprofv3
    FETCH_SIZE / WRITE_SIZE summary (rows '| `kernel` | ... | bytes |', the last
    column the calibrated total).  Empty when the summary is absent."""
    out = {}
    if not os.path.exists(TRAFFIC_FILE):
        return out
    with open(TRAFFIC_FILE) as f:
        for line in f:
            cells = [c.strip() for c in line.strip().strip("|").split("|")]
            if len(cells) >= 2 and cells[0].startswith("`tiler_"):
                try:
                    out[cells[0].strip("`")] = int(cells[-1].replace(",", ""))
                except ValueError:
                    pass
    return out


def calibration_copy(ctx, nbytes=256 << 20, times=3):
    """A plain device-to-device copy of known size, for scaling the FETCH_SIZE
    and WRITE_SIZE counters of a rocprofv3 --pmc run of this script."""
    src, dst = ctx.alloc(nbytes), ctx.alloc(nbytes)
    ctx.fill_u32(src, 0x3f800000, nbytes // 4)
    for _ in range(times):
        ctx.copy(dst, src, nbytes)
    ctx.synchronize()
    src.free()
    dst.free()


def measure(ctx, wl, steps, warmup):
    """W eager warm-up launches; then the K timed launches are captured once
    into a HIP graph (so Python's launch cost is not in the timed region),
    replayed untimed for at least SETTLE_S, and replayed once more between two
    events on the context stream: that replay is the K timed steps.  A second,
    eager pass with an event pair around every launch gives median/p10/p90."""
    log(f"{wl.name}: preparing synthetic inputs")
    wl.setup()
    for i in range(warmup):
        wl.launch(i)
    ctx.synchronize()
    ctx.capture_begin()
    for i in range(steps):
        wl.launch(warmup + i)
    graph = ctx.capture_end()
    # Settle: replay the graph for at least SETTLE_S.  Clocks dip for a few
    # milliseconds after sustained load begins and recover; timing one replay
    # right after the first would land in that dip.
    settle = 0
    t_settle = time.perf_counter()
    while settle < 3 or time.perf_counter() - t_settle < SETTLE_S:
        ctx.graph_launch(graph)
        ctx.synchronize()
        settle += 1
    e0, e1 = ctx.event(), ctx.event()
    log(f"{wl.name}: timing {steps} launches (graph replay)")
    t0 = time.perf_counter()
    ctx.record(e0)
    ctx.graph_launch(graph)
    ctx.record(e1)
    ctx.synchronize()
    wall = time.perf_counter() - t0
    total_ms = ctx.elapsed_ms(e0, e1)
    ctx.graph_destroy(graph)
    events = [ctx.event() for _ in range(steps + 1)]
    for i in range(steps):
        ctx.record(events[i])
        wl.launch(warmup + i)
    ctx.record(events[steps])
    ctx.synchronize()
    per = np.asarray([ctx.elapsed_ms(events[i], events[i + 1]) for i in range(steps)])
    for e in events + [e0, e1]:
        ctx.destroy_event(e)
    wl.teardown()
    mean_ms = total_ms / steps
    work = wl.work()
    if wl.bound == "hbm":
        achieved = work / (mean_ms / 1e3) / 1e9
        peak = HBM_PEAK_GBS
    else:
        achieved = work / (mean_ms / 1e3) / 1e12
        peak = MFMA_BF16_PEAK_TFLOPS
    return {
        "value": achieved, "unit": wl.unit, "ms_per_step": mean_ms,
        "median_ms": float(np.median(per)), "p10_ms": float(np.percentile(per, 10)),
        "p90_ms": float(np.percentile(per, 90)), "wall_s": wall,
        "roofline": {"bound": wl.bound, "achieved": achieved, "peak": peak,
                     "unit": wl.unit, "frac": achieved / peak,
                     "traffic": measured_traffic().get(wl.kernel),
                     "work_per_launch": work, "kernel": wl.kernel},
        "config": wl.config(),
    }


# The reference's own published device timings, Apple GPUs (context: other
# hardware, other memory system; not targets).  Strict f32 contraction cells
# of spikes/scheduling/metal_contraction_vertical/results/2026-07-31-timing-
# apple9-f32-msl4-macos26-m3pro-metal32023.883/timing-summary.tsv, realization
# `tiled` (the strict first-product fold): (cell, m, n, k, settled min us,
# GFLOP/s, line).
REFERENCE_CONTRACTION_CELLS = [
    ("w_decode_kv", 1, 1024, 1024, 60.500, 34.7, 3),
    ("w_prefill_q", 10, 2048, 1024, 148.958, 281.6, 9),
    ("w_prefill_mlp_in", 128, 3072, 1024, 1601.833, 502.7, 15),
    ("w_prefill_mlp_out", 128, 1024, 3072, 1599.459, 503.5, 21),
    ("w_prefill_o", 128, 1024, 2048, 1051.458, 510.6, 27),
    ("w_vocab_slice", 1, 8192, 1024, 523.500, 32.0, 33),
    ("t_vocab_full", 1, 151936, 1024, 9668.583, 32.2, 39),
    ("t_prefill_mlp_512", 512, 3072, 1024, 6395.375, 503.7, 45),
]
# Reduction dispatch crossover at 2^24 elements, Apple M4 Max, amortized p50 us
# (spikes/program-planning/reduction-dispatch-crossover/results/2026-08-07-
# apple-m4-max-macos27.0-26A5388g/sweep.tsv): (rows, extent, strategy, us, line).
REFERENCE_REDUCTION_CELLS = [
    (1024, 16384, "serial-fold", 1493.1444, 208),
    (1024, 16384, "single-workgroup-tree", 891.5083, 209),
    (1024, 16384, "multi-pass-split", 891.0139, 210),
    (4096, 4096, "serial-fold", 865.2778, 235),
    (4096, 4096, "single-workgroup-tree", 851.6889, 236),
    (4096, 4096, "multi-pass-split", 852.9639, 237),
    (65536, 256, "serial-fold", 860.7167, 274),
    (65536, 256, "single-workgroup-tree", 830.7334, 275),
    (65536, 256, "multi-pass-split", 836.9389, 276),
]


def time_launches(ctx, launch, steps, warmup, graph=True):
    """Mean ms per launch of `launch(i)`: W eager warm-ups, then K launches
    captured into a graph, replayed once untimed and once between events
    (graph=False: K eager launches between events, for a family that
    allocates per call and so refuses capture)."""
    for i in range(warmup):
        launch(i)
    ctx.synchronize()
    g = None
    if graph:
        ctx.capture_begin()
        try:
            for i in range(steps):
                launch(warmup + i)
        finally:
            g = ctx.capture_end()
        ctx.graph_launch(g)
        ctx.synchronize()
    e0, e1 = ctx.event(), ctx.event()
    ctx.record(e0)
    if g is not None:
        ctx.graph_launch(g)
    else:
        for i in range(steps):
            launch(warmup + i)
    ctx.record(e1)
    ctx.synchronize()
    ms = ctx.elapsed_ms(e0, e1) / steps
    for e in (e0, e1):
        ctx.destroy_event(e)
    if g is not None:
        ctx.graph_destroy(g)
    return ms


def reference_cells(ctx, steps, warmup):
    """This library on the reference's own published benchmark cells, with the
    same semantics.
    * The strict f32 contraction cells (tiler_contract_strict_f32, the
      first-product fold bit for bit).
    * The dispatch crossover's reduction cells with the reference's own
      program (reduction-dispatch-crossover/src/main.rs:999-1028): x * 1.0 +
      0.0 into a sum over the trailing axis, FusedMultiplyAddSerialSum, under
      FLUSH_AND_REASSOCIATE_F32 (permits_reassociation, both subnormal modes
      flushing to the signed zero), realized through tiler_hip_realize and run
      through the RuntimeAdapter stages: the serial fold, the single-workgroup
      tree (the cooperative workgroup at the balanced partition the
      2026-08-07 sweep dispatched) and the multi-pass split (the same
      partition).  Operands are all ones, as in the sweep, so every grouping
      gives the contributor count exactly; each cell's every output is
      checked against it before it is timed.  Inputs rotate over 5 sets of
      64 MiB (more than the Infinity Cache holds)."""
    from tiler_amd import _lib as L
    from tiler_amd.calibrate import split_partitions
    from tiler_amd.realize import prepare_route, realize
    out = {"contraction": [], "reduction": [],
           "reference_hardware": {"contraction": "Apple M3 Pro", "reduction": "Apple M4 Max"},
           "reduction_program": "FusedMultiplyAddSerialSum x*1.0+0.0 over the trailing axis, "
                                "FLUSH_AND_REASSOCIATE_F32, all-ones operands, via tiler_hip_realize"}
    rng = np.random.default_rng(3)
    for cell, m, n, k, ref_us, ref_gflops, line in REFERENCE_CONTRACTION_CELLS:
        a = ctx.to_device(rng.standard_normal((m, k)).astype(np.float32))
        b = ctx.to_device(rng.standard_normal((n, k)).astype(np.float32))
        c = ctx.alloc(m * n * 4)
        try:
            ms = time_launches(ctx, lambda i: ctx.contract_strict_f32(a, b, m, n, k, c), max(5, steps // 4), warmup)
        finally:
            for x in (a, b, c):
                x.free()
        gflops = 2.0 * m * n * k / (ms * 1e-3) / 1e9
        out["contraction"].append({"cell": cell, "m": m, "n": n, "k": k, "us": ms * 1e3, "gflop_per_s": gflops,
                                   "reference_us": ref_us, "reference_gflop_per_s": ref_gflops,
                                   "reference_line": line})
        log(f"reference cell {cell} {m}x{n}x{k}: {ms * 1e3:.1f} us ({gflops:.0f} GFLOP/s; reference {ref_us} us)")
    n_elem = 1 << 24
    ones = np.ones(n_elem, np.float32)
    xs = [ctx.to_device(ones) for _ in range(5)]
    o = ctx.alloc(65536 * 4)
    contract = dict(permissions=L.PERMITS_REASSOCIATION, input_subnormals=L.SUBNORMALS_FLUSH_SIGN,
                    result_subnormals=L.SUBNORMALS_FLUSH_SIGN, variant=L.FOLD_FMA, rank=2,
                    scalars=(0x3F800000, 0x00000000), flags=L.REGION_ALIGNED16)
    try:
        for rows, extent, strategy, ref_us, line in REFERENCE_REDUCTION_CELLS:
            p = split_partitions(extent)
            if strategy == "serial-fold":
                kw = dict(topology=L.SUM_SERIAL, grouping=(2,))
            elif strategy == "single-workgroup-tree":
                kw = dict(topology=L.SUM_COOPERATIVE, grouping=(2, p, extent // p))
            else:
                kw = dict(topology=L.SUM_MULTIPASS, grouping=(2, p, extent // p))
            rz = realize(L.PROGRAM_FOLD, (rows, extent), ctx=ctx, **kw, **contract)
            plans = [prepare_route(ctx, rz, [x, o] + [None] * (len(rz.slots) - 2)) for x in xs]
            try:
                plans[0].dispatch()
                got = o.download(np.float32, (rows,))
                if not (got == np.float32(extent)).all():
                    raise RuntimeError(f"reduction cell {rows}x{extent} {strategy}: outputs differ from {extent}")
                ms = time_launches(ctx, lambda i: plans[i % 5].enqueue(), max(10, steps // 4), warmup)
            finally:
                for pl in plans:
                    pl.release()
            out["reduction"].append({"rows": rows, "extent": extent, "strategy": strategy, "us": ms * 1e3,
                                     "kernels": rz.symbols, "reference_us": ref_us, "reference_line": line})
            log(f"reference cell {rows}x{extent} {strategy} {rz.symbols}: {ms * 1e3:.1f} us (reference {ref_us} us)")
    finally:
        for x in xs + [o]:
            x.free()
    return out


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--workload", default="rms_norm", choices=sorted(WORKLOADS))
    ap.add_argument("--no-families", action="store_true")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-reference-cells", action="store_true",
                    help="skip timing the reference's own published benchmark cells")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--vendor-gemm", action="store_true",
                    help="also time the vendor bf16 GEMM (torch.matmul) on the contraction operands")
    ap.add_argument("--vendor-gemm-child", action="store_true", help=argparse.SUPPRESS)
    ap.add_argument("--calibration-copy", action="store_true",
                    help="first run a 256 MiB device copy (counter calibration under rocprofv3 --pmc)")
    args = ap.parse_args()
    if args.gpus != 1:
        print("tiler-hip bench runs on one GPU: this build has no multi-GPU path "
              "(the reference has no multi-device notion); run with --gpus 1", file=sys.stderr)
        sys.exit(2)

    if args.vendor_gemm_child:  # torch's own HIP runtime, in a process without tiler-hip's
        print(json.dumps(Contract(None).vendor_reference(max(20, args.steps // 2), args.warmup)))
        return
    vendor = None
    if args.vendor_gemm:
        # Before this process touches the GPU: the vendor leg runs as a child
        # process, because torch's HIP runtime and the one tiler-hip links
        # cannot share a process.
        import subprocess
        log("vendor bf16 GEMM on the contraction operands (child process)")
        r = subprocess.run([sys.executable, os.path.abspath(__file__), "--vendor-gemm-child",
                            "--steps", str(args.steps), "--warmup", str(args.warmup)],
                           stdout=subprocess.PIPE, text=True, timeout=600)
        if r.returncode != 0:
            log(f"vendor leg failed with status {r.returncode}")
            sys.exit(r.returncode)
        vendor = json.loads(r.stdout.strip().splitlines()[-1])
        log(f"vendor: {vendor['value']:.1f} TFLOP/s ({vendor['ms_per_step'] * 1e3:.1f} us)")

    import tiler_amd
    ctx = tiler_amd.Context(0)
    log(f"device {ctx.environment['device_name']} {ctx.environment['gcn_arch_name']} "
        f"CUs={ctx.environment['compute_units']}")

    if args.calibration_copy:
        calibration_copy(ctx)
    head = measure(ctx, WORKLOADS[args.workload](ctx), args.steps, args.warmup)
    families = {}
    if not args.no_families:
        for name, cls in WORKLOADS.items():
            if name == args.workload:
                continue
            r = measure(ctx, cls(ctx), max(20, args.steps // 2), args.warmup)
            families[name] = {k: r[k] for k in ("value", "unit", "ms_per_step", "median_ms", "roofline", "config")}
            log(f"{name}: {r['value']:.1f} {r['unit']} ({100 * r['roofline']['frac']:.1f}% of peak)")

    cells = None
    if not args.no_reference_cells:
        cells = reference_cells(ctx, args.steps, args.warmup)

    cpu = None
    if not args.no_cpu_baseline:
        log(f"cpu baseline ({args.workload}), ~{args.cpu_seconds:.0f} s")
        cpu = WORKLOADS[args.workload](ctx).cpu_baseline(args.cpu_seconds)

    line = {
        "metric": METRIC,
        "value": head["value"],
        "unit": head["unit"],
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": head["ms_per_step"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32" if args.workload != "contract" else "bf16",
        "data": "synthetic (seeded numpy; BASELINE.json config shapes and distributions)",
        "config": head["config"],
        "timing": {"graph_replay_mean_ms": head["ms_per_step"],
                   "eager_median_ms": head["median_ms"], "eager_p10_ms": head["p10_ms"],
                   "eager_p90_ms": head["p90_ms"]},
        "roofline": head["roofline"],
        "cpu_baseline": cpu,
        "families": families,
        **({"reference_cells": cells} if cells else {}),
        **({"vendor_gemm": vendor} if vendor else {}),
        "device": {k: ctx.environment[k] for k in ("device_name", "gcn_arch_name", "compute_units")},
    }
    ctx.close()
    print(json.dumps(line))


if __name__ == "__main__":
    main()
