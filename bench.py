"""Benchmark of the fused LoRA linear on one MI355X.

Headline (the JSON line's `value`): BASELINE config 2 — Qwen3-0.6B-shaped prefill
projections in bf16, M = 8192 tokens, 7 projections x 28 layers per step, one shared
base weight set, per-layer rank-32 LoRA (scale 2). A step is one pass over the 196
projections, captured once as a HIP graph and replayed. The projections that read one
activation (q|k|v, gate|up) run as one grouped launch each (wsl_lora_linear_grouped_fwd;
each group's output is bit-identical to its own launch), so a layer is 4 launches; the same
inputs with one launch per projection (7 per layer) are reported beside it. value =
algorithmic TFLOP/s, FLOPs = sum over projections of 2*M*(N*K + r*(K+N)).

Also reported (same JSON line, key "extra"): config 3 decode GB/s (cold and warm
weights), config 4 weight-shared Qwen3 greedy decode tokens/s, config 5 fp8-base
projections, and the CPU baseline (the reference's fp32 arithmetic on host cores).

Usage: python bench.py [--gpus 1] [--steps 20] [--warmup 5] [--no-extra] [--no-cpu]
                      [--only c1|c2|c2single|c2_1p7b|c3|c4|c5|c5paths|emb|vendor|backward|medium|shape]
                      [--shape M,N,K,r]
                      [--vendor]
                      [--copy-calibration]

--only runs one section and prints its JSON alone (for profiling one workload).
--only vendor times the same shapes through torch.matmul (hipBLASLt): the plain GEMM and
the unfused three-call LoRA linear, beside the fused op.
--only shape runs five eager launches of one M,N,K,r shape (the fused op, or with
--vendor torch.matmul's plain GEMM), for rocprofv3 counter runs of a single kernel.
--copy-calibration first runs a plain device copy of COPY_BYTES bytes (three launches),
the reference point against which rocprofv3's FETCH_SIZE / WRITE_SIZE counters are
scaled to HBM bytes.
"""
from __future__ import annotations

import argparse
import json
import os
import re
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

import torch  # noqa: E402

METRIC = "fused-LoRA linear TFLOP/s (% MFMA peak); weight-shared Qwen3 decode tok/s"
BF16_PEAK_TFLOPS = 2500.0   # MI355X dense bf16 MFMA
FP8_PEAK_TFLOPS = 5000.0    # MI355X dense fp8 MFMA
HBM_PEAK_GBS = 8000.0       # MI355X HBM3E
COPY_BYTES = 256 << 20      # size of the calibration copy (--copy-calibration)
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "prefill_kernel_c2_hbm_traffic.md")

# (name, N, K) of the seven projections, as functions of (hidden, q_out, kv_out, ffn)
def proj_shapes(hidden, q_out, kv_out, ffn):
    return [("wq", q_out, hidden), ("wk", kv_out, hidden), ("wv", kv_out, hidden),
            ("wo", hidden, q_out), ("w1", ffn, hidden), ("w3", ffn, hidden), ("w2", hidden, ffn)]


QWEN3_0P6B = proj_shapes(1024, 2048, 1024, 3072)
QWEN3_1P7B = proj_shapes(2048, 2048, 1024, 6144)
QWEN3_8B = proj_shapes(4096, 4096, 1024, 12288)


def lora_flops(M, N, K, r):
    return 2.0 * M * (N * K + r * (K + N))


def lora_bytes(M, N, K, r, w_bytes=2, scales=False):
    return 2 * M * K + w_bytes * N * K + (4 * N if scales else 0) + 2 * r * K + 2 * N * r + 2 * M * N


class ProjectionStack:
    """Inputs of `layers` x 7 projections: one x per distinct K, `copies` sets of shared
    base weights (layer l uses copy l % copies), per-layer LoRA A/B. Drawn from one seeded
    generator in the order x, W (per copy, per projection), then A, B layer-major."""

    def __init__(self, shapes, M, r, layers, dev, seed=0, copies=1, fp8=False, scale=2.0):
        g = torch.Generator(device=dev).manual_seed(seed)
        self.shapes, self.M, self.r, self.layers, self.copies, self.scale = shapes, M, r, layers, copies, scale
        self.fp8 = fp8
        self.x = {}
        for _, _, K in shapes:
            if K not in self.x:
                self.x[K] = torch.randn(M, K, device=dev, generator=g).bfloat16()
        self.W, self.S = [], []
        for _ in range(copies):
            wl, sl = [], []
            for _, N, K in shapes:
                w = torch.randn(N, K, device=dev, generator=g) * 0.02
                if fp8:
                    from weightshared_torchtitan_amd import quantize_fp8_per_channel
                    q, s = quantize_fp8_per_channel(w)
                    wl.append(q)
                    sl.append(s)
                else:
                    wl.append(w.bfloat16())
                    sl.append(None)
                del w
            self.W.append(wl)
            self.S.append(sl)
        self.A, self.B = [], []
        for _ in range(layers):
            al, bl = [], []
            for _, N, K in shapes:
                al.append((torch.randn(r, K, device=dev, generator=g) * 0.02).bfloat16() if r else None)
                bl.append((torch.randn(N, r, device=dev, generator=g) * 0.02).bfloat16() if r else None)
            self.A.append(al)
            self.B.append(bl)

    def run(self):
        from weightshared_torchtitan_amd import lora_linear
        for l in range(self.layers):
            c = l % self.copies
            for p, (_, N, K) in enumerate(self.shapes):
                lora_linear(self.x[K], self.W[c][p], self.A[l][p], self.B[l][p], self.scale, w_scale=self.S[c][p])

    # Projections that read the same activation, run as one grouped launch each
    # (wsl_lora_linear_grouped_fwd): q|k|v and gate|up. Indices into `shapes`.
    GROUPS = ((0, 1, 2), (3,), (4, 5), (6,))

    def stack_groups(self):
        """Stacked operands of the grouped run, built once from the same tensors: per
        weight copy [W_q; W_k; W_v] and [W_1; W_3], per layer the A and B factors likewise."""
        def cat(ts):
            if len(ts) == 1:
                return ts[0]
            if ts[0].dtype == torch.float8_e4m3fn:  # stacked as bytes
                return torch.cat([t.view(torch.uint8) for t in ts], 0).view(torch.float8_e4m3fn)
            return torch.cat(ts, 0).contiguous()
        self.gW = [[cat([self.W[c][p] for p in grp]) for grp in self.GROUPS] for c in range(self.copies)]
        self.gS = [[cat([self.S[c][p] for p in grp]) if self.fp8 else None for grp in self.GROUPS]
                   for c in range(self.copies)]
        self.gA = [[cat([self.A[l][p] for p in grp]) if self.r else None for grp in self.GROUPS]
                   for l in range(self.layers)]
        self.gB = [[cat([self.B[l][p] for p in grp]) if self.r else None for grp in self.GROUPS]
                   for l in range(self.layers)]
        self.gN = [[self.shapes[p][1] for p in grp] for grp in self.GROUPS]
        self.gK = [self.shapes[grp[0]][2] for grp in self.GROUPS]

    def run_grouped(self):
        from weightshared_torchtitan_amd import ops
        for l in range(self.layers):
            c = l % self.copies
            for q in range(len(self.GROUPS)):
                ops.lora_linear_grouped_op(self.x[self.gK[q]], self.gW[c][q], self.gS[c][q], self.gA[l][q],
                                           self.gB[l][q], self.scale, self.gN[q])

    def prepare_chain(self, layers_per_chain=2):
        """Chains (wsl_lora_linear_chain_fwd) of the grouped launches' projections as
        independent stages, `layers_per_chain` layers (4 stages each) per launch: the inputs
        are synthetic, so no stage reads another's output. Outputs are allocated once. False
        where the library does not take it."""
        from weightshared_torchtitan_amd import ops
        self.stack_groups()
        dev = self.x[self.gK[0]].device
        self.chains = []
        st = []
        for l in range(self.layers):
            c = l % self.copies
            for q in range(len(self.GROUPS)):
                y = torch.empty(self.M, sum(self.gN[q]), dtype=torch.bfloat16, device=dev)
                st.append(ops.ChainStage(self.x[self.gK[q]], self.gW[c][q], self.gA[l][q], self.gB[l][q], self.scale,
                                         y, group_n=self.gN[q]))
            if (l + 1) % layers_per_chain == 0 or l + 1 == self.layers:
                if self.fp8 or not ops.chain_supported(st, self.M):
                    return False
                self.chains.append(st)
                st = []
        return True

    def run_chain(self):
        from weightshared_torchtitan_amd import ops
        for st in self.chains:
            ops.lora_linear_chain(st, self.M)

    def flops(self):
        return self.layers * sum(lora_flops(self.M, N, K, self.r) for _, N, K in self.shapes)

    def bytes(self):
        wb = 1 if self.fp8 else 2
        return self.layers * sum(lora_bytes(self.M, N, K, self.r, wb, self.fp8) for _, N, K in self.shapes)


class VendorStack(ProjectionStack):
    """The same inputs run through torch.matmul (hipBLASLt on this image): the plain
    base GEMM x . W^T, and the unfused LoRA linear x . W^T + s (x . A^T) . B^T (three
    library calls, the reference's arithmetic)."""

    def run_plain(self):
        for l in range(self.layers):
            c = l % self.copies
            for p, (_, N, K) in enumerate(self.shapes):
                torch.matmul(self.x[K], self.W[c][p].t())

    def run_plain_grouped(self):
        """The plain GEMM on the stacked q|k|v and gate|up weights (stack_groups first)."""
        for l in range(self.layers):
            c = l % self.copies
            for q in range(len(self.GROUPS)):
                torch.matmul(self.x[self.gK[q]], self.gW[c][q].t())

    def run_lora(self):
        for l in range(self.layers):
            c = l % self.copies
            for p, (_, N, K) in enumerate(self.shapes):
                x = self.x[K]
                torch.addmm(torch.matmul(x, self.W[c][p].t()), torch.matmul(x, self.A[l][p].t()),
                            self.B[l][p].t(), alpha=self.scale)


def bench_vendor(dev, steps, warmup):
    """Vendor-library comparison on the headline shapes, in one process: the fused op
    against torch.matmul's plain GEMM and the unfused three-call LoRA linear, each
    captured as a HIP graph of the same launches. Prefill: configs 2 (0.6B, 28 layers)
    and the 1.7B shapes (4 layers), M = 8192, r = 32, TFLOP/s of the LoRA linear's FLOPs
    (the plain GEMM's own FLOPs for the plain line). Decode: config 3 (1.7B, r = 64,
    28 layers, 6 rotating weight copies), GB/s of the LoRA linear's bytes. Each also with
    q|k|v and gate|up grouped: the fused op's grouped launches, and the plain GEMM on the
    stacked weights."""
    out = {}
    for name, shapes, layers in (("c2_qwen3_0.6b_prefill", QWEN3_0P6B, 28), ("qwen3_1.7b_prefill", QWEN3_1P7B, 4)):
        st = VendorStack(shapes, M=8192, r=32, layers=layers, dev=dev, seed=2)
        st.stack_groups()
        plain_flops = layers * sum(2.0 * 8192 * N * K for _, N, K in shapes)
        row = {}
        for label, fn, fl in (("wsl_fused", st.run, st.flops()), ("wsl_fused_grouped", st.run_grouped, st.flops()),
                              ("torch_plain_gemm", st.run_plain, plain_flops),
                              ("torch_plain_gemm_grouped", st.run_plain_grouped, plain_flops),
                              ("torch_unfused_lora", st.run_lora, st.flops())):
            g = graph_of(fn)
            ms = time_replays(g, steps, warmup)
            row[label] = {"ms": round(ms, 4), "TFLOP/s": round(fl / ms / 1e9, 1)}
            del g
        out[name] = row
        del st
        torch.cuda.empty_cache()
    dec = {}
    for M in (1, 8, 32, 64):
        st = VendorStack(QWEN3_1P7B, M=M, r=64, layers=28, dev=dev, seed=3, copies=6)
        st.stack_groups()
        row = {}
        for label, fn in (("wsl_fused", st.run), ("wsl_fused_grouped", st.run_grouped),
                          ("torch_plain_gemm", st.run_plain), ("torch_plain_gemm_grouped", st.run_plain_grouped),
                          ("torch_unfused_lora", st.run_lora)):
            g = graph_of(fn)
            ms = time_replays(g, steps, warmup)
            row[label] = {"ms_per_28_layers": round(ms, 4), "GB/s": round(st.bytes() / ms / 1e6, 1)}
            del g
        dec[f"M={M}"] = row
        del st
        torch.cuda.empty_cache()
    out["c3_qwen3_1.7b_decode_cold"] = dec
    return out


def run_shape(dev, shape, vendor):
    """Five eager launches of one shape (for rocprofv3 runs of a single kernel):
    wsl.lora_linear, or with `vendor` torch.matmul's plain GEMM."""
    M, N, K, r = shape
    g = torch.Generator(device=dev).manual_seed(0)
    x = torch.randn(M, K, device=dev, generator=g).bfloat16()
    W = (torch.randn(N, K, device=dev, generator=g) * 0.02).bfloat16()
    A = (torch.randn(r, K, device=dev, generator=g) * 0.02).bfloat16() if r else None
    B = (torch.randn(N, r, device=dev, generator=g) * 0.02).bfloat16() if r else None
    from weightshared_torchtitan_amd import lora_linear
    for _ in range(5):
        if vendor:
            torch.matmul(x, W.t())
        else:
            lora_linear(x, W, A, B, 2.0)
    torch.cuda.synchronize()
    return {"M": M, "N": N, "K": K, "r": r, "launches": 5, "vendor": bool(vendor)}


def graph_of(fn):
    """Captures fn() once as a HIP graph (after one eager warm-up on a side stream)."""
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        fn()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):  # the warm-up stream: its workspaces exist already
        fn()
    torch.cuda.synchronize()
    return g


def time_replays(graph, steps, warmup):
    """Mean ms per replay over `steps` replays, bracketed by synchronize + HIP events on
    the stream the replays run on."""
    for _ in range(warmup):
        graph.replay()
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream()
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for _ in range(steps):
        graph.replay()
    e1.record(stream)
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / steps


# ------------------------------------------------------------------------------ configs
def bench_c2(dev, steps, warmup, grouped=True, single=True):
    """Config 2 on the same inputs, two ways: q|k|v and gate|up (the projections that read
    one activation) as grouped launches, 4 per layer, 112 per step (the headline), and one
    launch per projection, 7 per layer, 196 per step. Returns (FLOPs, ms grouped, ms single);
    a way not run gives None."""
    st = ProjectionStack(QWEN3_0P6B, M=8192, r=32, layers=28, dev=dev, seed=2)
    ms_grouped = ms_single = None
    if grouped:
        st.stack_groups()
        g = graph_of(st.run_grouped)
        ms_grouped = time_replays(g, steps, warmup)
        del g
    if single:
        g = graph_of(st.run)
        ms_single = time_replays(g, steps, warmup)
        del g
    del st
    torch.cuda.empty_cache()
    return lora_flops_c2(), ms_grouped, ms_single


# Prefill launches of configs 2 and 1.7B for side-by-side timing of the path switches (name,
# M, group widths, K); every launch at r = 32.
AB_SHAPES = [("c2 q|k|v", 8192, (2048, 1024, 1024), 1024), ("c2 o", 8192, (1024,), 2048),
             ("c2 gate|up", 8192, (3072, 3072), 1024), ("c2 down", 8192, (1024,), 3072),
             ("1.7b q|k|v", 8192, (2048, 1024, 1024), 2048), ("1.7b o", 8192, (2048,), 2048),
             ("1.7b gate|up", 8192, (6144, 6144), 2048), ("1.7b down", 8192, (2048,), 6144)]


def bench_data(dev, names=("c2 q|k|v", "1.7b gate|up", "1.7b down"), launches=28, rounds=6):
    """The same prefill launches (the fused op, and torch.mm on hipBLASLt for the base GEMM
    alone) on operands of different value statistics and identical shapes, layouts and
    memory traffic: x ~ N(0, 1) and W ~ N(0, 0.02^2) as every benchmark here uses, x zero,
    W zero, x all ones, half of x's rows zero. The chip's clock is set by its power budget,
    and the power drawn depends on how many operand bits switch, so these times differ while
    the work does not. One HIP graph of `launches` launches per variant, the graphs
    replayed in alternating order, the median of `rounds` rounds (us per launch)."""
    from weightshared_torchtitan_amd import ops
    out = {}
    for name, M, ns, K in AB_SHAPES:
        if name not in names:
            continue
        r = 32
        g = torch.Generator(device=dev).manual_seed(M + sum(ns) + K)
        xr = torch.randn(M, K, device=dev, generator=g).bfloat16()
        wr = (torch.randn(sum(ns), K, device=dev, generator=g) * 0.02).bfloat16()
        a = (torch.randn(len(ns) * r, K, device=dev, generator=g) * 0.02).bfloat16()
        b = (torch.randn(sum(ns), r, device=dev, generator=g) * 0.02).bfloat16()
        half = (torch.rand(M, 1, device=dev, generator=g) < 0.5).bfloat16()
        data = {"randn": (xr, wr), "x_zero": (torch.zeros_like(xr), wr), "w_zero": (xr, torch.zeros_like(wr)),
                "x_ones": (torch.ones_like(xr), wr), "x_half_rows_zero": (xr * half, wr)}
        graphs = {}
        for v, (x, w) in data.items():
            if len(ns) > 1:
                fn = lambda x=x, w=w: ops.lora_linear_grouped_op(x, w, None, a, b, 2.0, list(ns))  # noqa: E731
            else:
                fn = lambda x=x, w=w: ops.lora_linear_op(x, w, None, a, b, 2.0)  # noqa: E731
            graphs["wsl " + v] = graph_of(lambda fn=fn: [fn() for _ in range(launches)])
            if v in ("randn", "x_zero"):
                wt = w.t()
                graphs["hipblaslt_base_gemm " + v] = graph_of(lambda x=x, wt=wt: [torch.mm(x, wt) for _ in range(launches)])
        times = {k: [] for k in graphs}
        for _ in range(rounds):
            for k, gr in graphs.items():
                times[k].append(time_replays(gr, 3, 1) * 1e3 / launches)
        fl = sum(lora_flops(M, n, K, r) for n in ns)  # the base GEMM alone: r = 0
        flb = sum(lora_flops(M, n, K, 0) for n in ns)
        out[name] = {k: {"us": round(sorted(t)[len(t) // 2], 2),
                         "TFLOP/s": round((flb if k.startswith("hipblaslt") else fl) / (sorted(t)[len(t) // 2] * 1e-6) / 1e12, 1)}
                     for k, t in times.items()}
        del graphs, data, xr, wr, a, b
        torch.cuda.empty_cache()
    return out


def bench_env_ab(dev, modes, names=None, launches=28, rounds=6):
    """Side-by-side timing of libwsl's path overrides (ops.path_options: prefill_strips,
    prefill_split, ...): per launch shape one HIP graph of `launches` launches is captured
    under each mode's overrides, and the graphs are replayed in alternating order over
    `rounds` rounds (5 replays each, HIP events), so clock drift falls on every mode alike.
    Returns the median us per launch per mode."""
    from weightshared_torchtitan_amd import ops
    out = {}
    for name, M, ns, K in AB_SHAPES:
        if names is not None and name not in names:
            continue
        r = 32
        g = torch.Generator(device=dev).manual_seed(M + sum(ns) + K)
        x = torch.randn(M, K, device=dev, generator=g).bfloat16()
        w = (torch.randn(sum(ns), K, device=dev, generator=g) * 0.02).bfloat16()
        a = (torch.randn(len(ns) * r, K, device=dev, generator=g) * 0.02).bfloat16()
        b = (torch.randn(sum(ns), r, device=dev, generator=g) * 0.02).bfloat16()
        if len(ns) > 1:
            fn = lambda: ops.lora_linear_grouped_op(x, w, None, a, b, 2.0, list(ns))  # noqa: E731
        else:
            fn = lambda: ops.lora_linear_op(x, w, None, a, b, 2.0)  # noqa: E731
        graphs = {}
        for mode, opts in modes.items():
            with ops.path_options(**opts):
                graphs[mode] = graph_of(lambda: [fn() for _ in range(launches)])
        times = {m: [] for m in modes}
        order = list(modes)
        for it in range(rounds):
            for m in (order if it % 2 == 0 else order[::-1]):
                times[m].append(time_replays(graphs[m], 5, 1) * 1e3 / launches)
        out[name] = {m: round(sorted(v)[len(v) // 2], 2) for m, v in times.items()}
        del graphs
    torch.cuda.empty_cache()
    return out


STAMP_PHASES = ("first_fill", "k_loop", "lora_up", "stage", "store_issue")


def bench_stamps(dev, names=None):
    """Where a prefill tile's time goes, from the instrumented library's per-workgroup
    wall-clock stamps (WSL_LIB=<repo>/weightshared_torchtitan_amd/libwsl_stamps.so, built by
    `python -m weightshared_torchtitan_amd.build --stamps`). One launch per shape of
    AB_SHAPES (and of MEDIUM_STAMP_SHAPES) after three warm-up launches; per tile of a strip
    (q = 0, 1, ...), or for split-K launches per last split and other splits, the median and
    maximum over workgroups of each phase's duration (us at the 100 MHz constant clock), the
    spread of tile starts, and the span from the first start to the last store beside the
    HIP-event time of the same launch."""
    import ctypes
    import numpy as np
    from weightshared_torchtitan_amd import _native, ops
    lib = _native.lib()
    if not hasattr(lib, "wsl_prefill_stamps"):
        raise SystemExit("--only stamps needs WSL_LIB=<repo>/weightshared_torchtitan_amd/libwsl_stamps.so "
                         "(python -m weightshared_torchtitan_amd.build --stamps)")
    lib.wsl_prefill_stamps.restype = ctypes.c_int
    lib.wsl_prefill_stamps.argtypes = [ctypes.c_void_p, ctypes.c_size_t]
    recs = 4096
    buf = np.zeros(recs * 8, dtype=np.uint64)
    out = {}
    for name, M, ns, K, r in [(*sh, 32) for sh in AB_SHAPES] + MEDIUM_STAMP_SHAPES:
        if names is not None and name not in names:
            continue
        g = torch.Generator(device=dev).manual_seed(M + sum(ns) + K)
        x = torch.randn(M, K, device=dev, generator=g).bfloat16()
        w = (torch.randn(sum(ns), K, device=dev, generator=g) * 0.02).bfloat16()
        a = (torch.randn(len(ns) * r, K, device=dev, generator=g) * 0.02).bfloat16()
        b = (torch.randn(sum(ns), r, device=dev, generator=g) * 0.02).bfloat16()
        if len(ns) > 1:
            fn = lambda: ops.lora_linear_grouped_op(x, w, None, a, b, 2.0, list(ns))  # noqa: E731
        else:
            fn = lambda: ops.lora_linear_op(x, w, None, a, b, 2.0)  # noqa: E731
        for _ in range(3):
            fn()
        torch.cuda.synchronize()
        lib.wsl_prefill_stamps(buf.ctypes.data, recs)  # clears the stamps
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        e0.record()
        fn()
        e1.record()
        torch.cuda.synchronize()
        rc = lib.wsl_prefill_stamps(buf.ctypes.data, recs)
        if rc != 0:
            raise RuntimeError(f"wsl_prefill_stamps failed: {rc}")
        st = buf.reshape(recs, 8).astype(np.int64)
        valid = st[:, 0] > 0
        t0 = st[valid, 0].min()
        plan = ops.plan(M, K, r, list(ns))
        res = {"plan": {k: plan[k] for k in ("path", "tile_m", "tile_n", "k_splits", "workgroups")},
               "event_us": round(e0.elapsed_time(e1) * 1e3, 2),
               "span_us": round((st[valid, 5].max() - t0) / 100.0, 2)}
        if plan["k_splits"] > 1:
            # split-K: the last split of each tile runs every phase (the reduction falls in
            # "stage"); the others stop after the up-projection of their own part
            groups = [("last_split", valid & (st[:, 5] > 0), len(STAMP_PHASES)),
                      ("other_splits", valid & (st[:, 5] == 0), 3)]
        else:
            groups = [(f"tile{q}", (np.arange(recs) % 4 == q) & valid, len(STAMP_PHASES)) for q in range(4)]
        for label, sel, nph in groups:
            rows = st[sel]
            if len(rows) == 0:
                continue
            d = {"workgroups": int(len(rows)),
                 "start_after_first_us": [round(float(np.median(rows[:, 0] - t0)) / 100, 2),
                                          round(float((rows[:, 0] - t0).max()) / 100, 2)]}
            for k, ph in enumerate(STAMP_PHASES[:nph], start=1):
                dd = (rows[:, k] - rows[:, k - 1]) / 100.0
                d[ph + "_us"] = [round(float(np.median(dd)), 2), round(float(dd.max()), 2)]
            res[label] = d
        out[name] = res
        del x, w, a, b
    if names is None or any(n in names for n, *_ in DECODE_STAMP_SHAPES):
        out.update(decode_stamps(dev, lib, names))
    return out


# Medium-M launches (1.7B shapes, r = 64, the in-launch split-K form) for the prefill
# kernel's phase stamps: name, M, group widths, K, rank.
MEDIUM_STAMP_SHAPES = [("1.7b q|k|v M=256", 256, (2048, 1024, 1024), 2048, 64),
                       ("1.7b down M=512", 512, (2048,), 6144, 64)]


# Decode launches (config 3 shapes, r = 64) for the decode kernel's phase stamps: name, M,
# group widths, K.
DECODE_STAMP_SHAPES = [("c3 o M=1", 1, (2048,), 2048), ("c3 gate|up M=1", 1, (6144, 6144), 2048),
                       ("c3 down M=1", 1, (2048,), 6144), ("c3 o M=8", 8, (2048,), 2048),
                       ("c3 gate|up M=64", 64, (6144, 6144), 2048)]


def decode_stamps(dev, lib, names=None, copies=6):
    """Per-workgroup phase times of one decode launch per shape (cold weights: `copies`
    weight sets, the first ones for the warm-up launches, the last for the stamped one),
    in us after the launch's first workgroup start (median / max): T workgroups' T
    published; W workgroups' W stream and cross-wave reduction done, K-split reduction done,
    T gathered, outputs stored."""
    import ctypes
    import numpy as np
    from weightshared_torchtitan_amd import ops
    lib.wsl_decode_stamps.restype = ctypes.c_int
    lib.wsl_decode_stamps.argtypes = [ctypes.c_void_p, ctypes.c_size_t]
    recs = 4096
    buf = np.zeros(recs * 8, dtype=np.uint64)
    out = {}
    for name, M, ns, K in DECODE_STAMP_SHAPES:
        if names is not None and name not in names:
            continue
        r = 64
        g = torch.Generator(device=dev).manual_seed(M + sum(ns) + K)
        x = torch.randn(M, K, device=dev, generator=g).bfloat16()
        sets = []
        for _ in range(copies):
            sets.append(((torch.randn(sum(ns), K, device=dev, generator=g) * 0.02).bfloat16(),
                         (torch.randn(len(ns) * r, K, device=dev, generator=g) * 0.02).bfloat16(),
                         (torch.randn(sum(ns), r, device=dev, generator=g) * 0.02).bfloat16()))

        def run(wab):
            w, a, b = wab
            if len(ns) > 1:
                return ops.lora_linear_grouped_op(x, w, None, a, b, 2.0, list(ns))
            return ops.lora_linear_op(x, w, None, a, b, 2.0)

        for q in range(copies - 1):
            run(sets[q])
        torch.cuda.synchronize()
        lib.wsl_decode_stamps(buf.ctypes.data, recs)  # clears the stamps
        run(sets[-1])
        torch.cuda.synchronize()
        rc = lib.wsl_decode_stamps(buf.ctypes.data, recs)
        if rc != 0:
            raise RuntimeError(f"wsl_decode_stamps failed: {rc}")
        st = buf.reshape(recs, 8).astype(np.int64)
        kind = st[:, 7]
        t0 = st[kind > 0, 0].min()

        def mm(v):
            v = (v - t0) / 100.0
            return [round(float(np.median(v)), 2), round(float(v.max()), 2)]

        tw, ww = st[kind == 1], st[kind == 2]
        res = {"t_workgroups": int(len(tw)), "w_workgroups": int(len(ww)),
               "start": mm(st[kind > 0, 0]),
               "t_published": mm(tw[tw[:, 2] > 0, 2]) if (tw[:, 2] > 0).any() else None,
               "w_stream_reduced": mm(ww[:, 1]),
               "w_split_reduced": mm(ww[ww[:, 2] > 0, 2]) if (ww[:, 2] > 0).any() else None,
               "w_t_gathered": mm(ww[ww[:, 3] > 0, 3]) if (ww[:, 3] > 0).any() else None,
               "w_stored": mm(ww[ww[:, 4] > 0, 4]) if (ww[:, 4] > 0).any() else None}
        out[name] = res
        del sets, x
    return out


def lora_flops_c2():
    return 28 * sum(lora_flops(8192, N, K, 32) for _, N, K in QWEN3_0P6B)


def bench_c2_1p7b(dev, steps, warmup):
    st = ProjectionStack(QWEN3_1P7B, M=8192, r=32, layers=4, dev=dev, seed=21)
    g = graph_of(st.run)
    ms = time_replays(g, steps, warmup)
    del g
    st.stack_groups()
    g = graph_of(st.run_grouped)
    ms_grouped = time_replays(g, steps, warmup)
    del g, st
    torch.cuda.empty_cache()
    return ms, ms_grouped


def c2_1p7b_extra(dev, steps, warmup):
    """The Qwen3-1.7B prefill shapes (the north star's >= 70 % target): 4 layers of the 7
    projections, M = 8192, r = 32, one launch per projection and grouped."""
    ms17, ms17g = bench_c2_1p7b(dev, steps, warmup)
    f17 = 4 * sum(lora_flops(8192, N, K, 32) for _, N, K in QWEN3_1P7B)
    return {"TFLOP/s": round(f17 / ms17 / 1e9, 1), "frac_mfma": round(f17 / ms17 / 1e9 / BF16_PEAK_TFLOPS, 4),
            "ms_per_4_layers": round(ms17, 4), "grouped_qkv_gateup_TFLOP/s": round(f17 / ms17g / 1e9, 1),
            "grouped_frac_mfma": round(f17 / ms17g / 1e9 / BF16_PEAK_TFLOPS, 4),
            "grouped_ms_per_4_layers": round(ms17g, 4)}


def bench_c3(dev, steps, warmup):
    """Config 3 per M: one launch per projection with cold weights (6 rotating copies) and
    warm (one copy), cold with q|k|v and gate|up as grouped launches (4 per layer), and cold
    with two layers' grouped launches as the independent stages of one chain launch (up to 16
    tokens)."""
    out = {}
    for M in (1, 8, 32, 64):
        row = {}
        for label, copies, grouped in (("cold", 6, False), ("warm", 1, False), ("cold_grouped", 6, True),
                                       ("cold_chain", 6, "chain")):
            st = ProjectionStack(QWEN3_1P7B, M=M, r=64, layers=28, dev=dev, seed=3, copies=copies)
            if grouped == "chain":
                if not st.prepare_chain():
                    continue
                fn = st.run_chain
            elif grouped:
                st.stack_groups()
                fn = st.run_grouped
            else:
                fn = st.run
            g = graph_of(fn)
            ms = time_replays(g, steps, warmup)
            row[label] = {"ms_per_28_layers": round(ms, 4), "GB/s": round(st.bytes() / ms / 1e6, 1),
                          "frac_hbm": round(st.bytes() / ms / 1e6 / HBM_PEAK_GBS, 4)}
            del g, st
            torch.cuda.empty_cache()
        out[f"M={M}"] = row
    return out


def bench_medium(dev, steps, warmup):
    """Medium M (above the decode path's fused forms, up to a thousand tokens) at the
    Qwen3-1.7B projection shapes, r = 64, cold weights (6 rotating copies), 28 layers per
    graph, grouped q|k|v and gate|up, each way the library can run them on the same inputs:
    the decode path (the default up to 64 tokens; its wide form from 65 to 72 with the
    decode_wide override at 1), the prefill path's in-launch split-K form (the default from 65
    tokens) and its unsplit tiles (prefill_split and prefill_medium at -1, which keep the
    split forms off); from 128 tokens also torch.matmul (hipBLASLt) on the same
    inputs: the plain GEMM on the stacked weights (no LoRA term) and the unfused three-call
    LoRA linear (the reference's arithmetic)."""
    from weightshared_torchtitan_amd import ops
    out = {}
    ways = (("decode", {"decode_wide": 1}),
            ("split_k", {}),
            ("unsplit", {"prefill_split": -1, "prefill_medium": -1}))
    for M in (64, 65, 72, 96, 128, 160, 192, 256, 512, 1024):
        row = {}
        for label, opts in ways:
            if (label == "decode" and M > 72) or (label != "decode" and M <= 64):
                continue  # decode runs up to 72 tokens, the prefill forms above 64
            with ops.path_options(**opts):
                st = ProjectionStack(QWEN3_1P7B, M=M, r=64, layers=28, dev=dev, seed=3, copies=6)
                st.stack_groups()
                g = graph_of(st.run_grouped)
            ms = time_replays(g, steps, warmup)
            row[label] = {"ms_per_28_layers": round(ms, 4), "GB/s": round(st.bytes() / ms / 1e6, 1),
                          "TFLOP/s": round(st.flops() / ms / 1e9, 1)}
            del g, st
            torch.cuda.empty_cache()
        if M >= 128:
            st = VendorStack(QWEN3_1P7B, M=M, r=64, layers=28, dev=dev, seed=3, copies=6)
            st.stack_groups()
            for label, fn in (("torch_plain_gemm_grouped", st.run_plain_grouped), ("torch_unfused_lora", st.run_lora)):
                g = graph_of(fn)
                ms = time_replays(g, steps, warmup)
                row[label] = {"ms_per_28_layers": round(ms, 4)}
                del g
            del st
            torch.cuda.empty_cache()
        out[f"M={M}"] = row
    return out


def bench_c5_paths(dev, steps, warmup):
    """Config 5 at M = 4096 on each fp8 prefill path, same inputs: the default (two activation
    terms on the fp8 matrix cores for launches wider than one wave of 256 x 256 tiles, W
    decoded onto the bf16 matrix cores for the rest), every launch on the fp8 matrix cores
    with two terms (the fp8_prefill override at 2), with one term (the opt-in
    WSL_DTYPE_FP8_E4M3_ACT8), and every launch with W decoded (the override at 1)."""
    from weightshared_torchtitan_amd import ops
    st = ProjectionStack(QWEN3_8B, M=4096, r=128, layers=1, dev=dev, seed=5, copies=1, fp8=True, scale=1.0)
    st.stack_groups()
    base = st.layers * sum(2.0 * 4096 * N * K for _, N, K in st.shapes)
    lora = st.flops() - base
    t_min = base / (FP8_PEAK_TFLOPS * 1e12) + lora / (BF16_PEAK_TFLOPS * 1e12)
    out = {}
    saved = ops.FP8_ACTIVATIONS
    try:
        for name, act8, weight_only in (("default", False, 0), ("fp8_mfma_two_term", False, 2),
                                        ("fp8_mfma_one_term", True, 0), ("weight_only_bf16_mfma", False, 1)):
            ops.FP8_ACTIVATIONS = act8
            row = {}
            for label, fn in (("per_projection", st.run), ("grouped_qkv_gateup", st.run_grouped)):
                with ops.path_options(fp8_prefill=weight_only):
                    g = graph_of(fn)
                ms = time_replays(g, steps, warmup)
                del g
                row[label] = {"ms": round(ms, 4), "TFLOP/s": round(st.flops() / ms / 1e9, 1),
                              "frac_mixed_mfma_roofline": round(t_min * 1e3 / ms, 4)}
            out[name] = row
    finally:
        ops.FP8_ACTIVATIONS = saved
    del st
    torch.cuda.empty_cache()
    return out


def bench_c5(dev, steps, warmup):
    out = {}
    for M in (16, 4096):
        copies = 3 if M == 16 else 1
        st = ProjectionStack(QWEN3_8B, M=M, r=128, layers=4 if M == 16 else 1, dev=dev, seed=5,
                             copies=copies, fp8=True, scale=1.0)
        g = graph_of(st.run)
        ms = time_replays(g, steps, warmup)
        del g
        st.stack_groups()
        g = graph_of(st.run_grouped)
        ms_g = time_replays(g, steps, warmup)
        base = st.layers * sum(2.0 * M * N * K for _, N, K in st.shapes)
        lora = st.flops() - base
        t_min = base / (FP8_PEAK_TFLOPS * 1e12) + lora / (BF16_PEAK_TFLOPS * 1e12)
        out[f"M={M}"] = {"ms": round(ms, 4), "TFLOP/s": round(st.flops() / ms / 1e9, 1),
                         "GB/s": round(st.bytes() / ms / 1e6, 1),
                         "frac_mixed_mfma_roofline": round(t_min * 1e3 / ms, 4),
                         "frac_hbm": round(st.bytes() / ms / 1e6 / HBM_PEAK_GBS, 4),
                         "grouped_qkv_gateup": {"ms": round(ms_g, 4), "TFLOP/s": round(st.flops() / ms_g / 1e9, 1),
                                                "GB/s": round(st.bytes() / ms_g / 1e6, 1),
                                                "frac_mixed_mfma_roofline": round(t_min * 1e3 / ms_g, 4),
                                                "frac_hbm": round(st.bytes() / ms_g / 1e6 / HBM_PEAK_GBS, 4)}}
        del g, st
        torch.cuda.empty_cache()
    return out


def lora_backward_flops(M, N, K, r):
    """dx = gy.W + s(gy.B).A, dW = gy^T.x, dA = s(gy.B)^T.x, dB = s gy^T.(x.A^T): U = gy.B
    and T = x.A^T counted once each."""
    return 2.0 * M * (2 * N * K + 2 * r * (N + K) + r * N + r * K)


def bench_backward(dev, steps, warmup, layers=4, M=8192, r=32):
    """Backward of the config-2 projections (Qwen3-0.6B, M = 8192, r = 32) over `layers`
    layers that share one base W set, every tensor requiring grad (the weight-shared
    trainer's case; each layer has its own inputs, the three projections of a layer that
    read one activation share it, as q/k/v and gate/up do). Timed eagerly with HIP events around loss.backward() only; the
    forward runs untimed before each step. Three paths on the same inputs: the fused op
    (dx on the fused kernel, weight gradients by wsl_lora_linear_bwd_weights), the grouped
    op for q|k|v and gate|up (stacked parameters), and torch autograd of the reference's
    unfused arithmetic x.W^T + s (x.A^T).B^T. "weight_grads" times dW, dA and dB alone per
    projection shape: the HIP entry point against the same three products on torch GEMMs
    (hipBLASLt)."""
    from weightshared_torchtitan_amd import lora_linear
    g = torch.Generator(device=dev).manual_seed(12)
    Ws = [(torch.randn(N, K, device=dev, generator=g) * 0.02).bfloat16().requires_grad_(True)
          for _, N, K in QWEN3_0P6B]
    xs = [{K: torch.randn(M, K, device=dev, generator=g).bfloat16().requires_grad_(True)
           for K in sorted({K for _, _, K in QWEN3_0P6B})} for _ in range(layers)]
    lor = [[((torch.randn(r, K, device=dev, generator=g) * 0.02).bfloat16().requires_grad_(True),
             (torch.randn(N, r, device=dev, generator=g) * 0.02).bfloat16().requires_grad_(True))
            for _, N, K in QWEN3_0P6B] for _ in range(layers)]
    gys = [torch.randn(M, N, device=dev, generator=g).bfloat16() for _, N, _ in QWEN3_0P6B]

    def fused():
        return [lora_linear(xs[l][K], Ws[i], *lor[l][i], 2.0)
                for l in range(layers) for i, (_, _, K) in enumerate(QWEN3_0P6B)]

    def unfused():
        return [xs[l][K] @ Ws[i].t() + 2.0 * (xs[l][K] @ lor[l][i][0].t()) @ lor[l][i][1].t()
                for l in range(layers) for i, (_, _, K) in enumerate(QWEN3_0P6B)]

    # grouped: q|k|v and gate|up as one op each, on stacked leaves holding the same values
    # (a trainer that keeps the stacked tensors as its parameters)
    groups = ProjectionStack.GROUPS
    leaf = lambda ts: torch.cat([t.detach() for t in ts], 0).requires_grad_(True)
    gWs = [leaf([Ws[i] for i in grp]) for grp in groups]
    glor = [[(leaf([lor[l][i][0] for i in grp]), leaf([lor[l][i][1] for i in grp])) for grp in groups]
            for l in range(layers)]
    gN = [[QWEN3_0P6B[i][1] for i in grp] for grp in groups]
    gK = [QWEN3_0P6B[grp[0]][2] for grp in groups]
    ggys = [torch.cat([gys[i] for i in grp], 1) for grp in groups]

    def grouped():
        from weightshared_torchtitan_amd import ops
        return [ops.lora_linear_grouped_op(xs[l][gK[q]], gWs[q], None, glor[l][q][0], glor[l][q][1], 2.0, gN[q])
                for l in range(layers) for q in range(len(groups))]

    params = ([v for d in xs for v in d.values()] + Ws + [p for pr in lor for ab in pr for p in ab] + gWs
              + [p for pr in glor for ab in pr for p in ab])

    def timed(fwd, grads):
        total = 0.0
        for it in range(warmup + steps):
            for t in params:
                t.grad = None
            ys = fwd()
            torch.cuda.synchronize()
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            torch.autograd.backward(ys, [grads[i % len(grads)] for i in range(len(ys))])
            e1.record()
            e1.synchronize()
            if it >= warmup:
                total += e0.elapsed_time(e1)
        return total / steps

    def graphed(fwd, grads):
        """The GPU time of the backward without the host's launch work: forward + backward
        captured as one HIP graph and the forward alone as another (both after eager warm-ups
        on the capture stream, gradients allocated by the capture); the backward is the
        difference of their mean replay times."""
        def step():
            ys = fwd()
            torch.autograd.backward(ys, [grads[i % len(grads)] for i in range(len(ys))])

        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            for _ in range(2):
                for t in params:
                    t.grad = None
                step()
        torch.cuda.current_stream().wait_stream(s)
        torch.cuda.synchronize()
        for t in params:
            t.grad = None
        g_fb, g_f = torch.cuda.CUDAGraph(), torch.cuda.CUDAGraph()
        with torch.cuda.graph(g_fb, stream=s):
            step()
        with torch.cuda.graph(g_f, stream=s):
            fwd()
        torch.cuda.synchronize()
        t_fb = time_replays(g_fb, steps, warmup)
        t_f = time_replays(g_f, steps, warmup)
        del g_fb, g_f
        for t in params:
            t.grad = None
        torch.cuda.synchronize()
        return t_fb - t_f, t_f

    fl = layers * sum(lora_backward_flops(M, N, K, r) for _, N, K in QWEN3_0P6B)
    out = {"layers": layers, "M": M, "r": r}
    for name, fwd, grads in (("wsl_fused", fused, gys), ("wsl_grouped_qkv_gateup", grouped, ggys),
                             ("torch_unfused_autograd", unfused, gys)):
        ms = timed(fwd, grads)
        out[name] = {"ms": round(ms, 4), "TFLOP/s": round(fl / ms / 1e9, 1),
                     "frac_mfma": round(fl / ms / 1e9 / BF16_PEAK_TFLOPS, 4)}
        try:
            gms, fms = graphed(fwd, grads)
            out[name].update({"graph_ms": round(gms, 4), "graph_TFLOP/s": round(fl / gms / 1e9, 1),
                              "graph_frac_mfma": round(fl / gms / 1e9 / BF16_PEAK_TFLOPS, 4),
                              "graph_forward_ms": round(fms, 4)})
        except RuntimeError as e:  # a capture the path does not support: the eager figure stands
            torch.cuda.synchronize()
            out[name]["graph_error"] = str(e)[:200]
    from weightshared_torchtitan_amd import ops

    def torch_weight_grads(x2, gy2, a, b, s):
        """The same three products on torch GEMMs (hipBLASLt), the vendor comparison:
        dW = gy^T x, dA = s (gy B)^T x, dB = s gy^T (x A^T)."""
        gt = gy2.t()
        dw = gt @ x2
        da = ((gy2 @ b) * s).t() @ x2
        db = gt @ ((x2 @ a.t()) * s)
        return dw, da, db

    def wg_ms(fn):
        for _ in range(warmup):
            fn()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(steps):
            fn()
        e1.record()
        e1.synchronize()
        return e0.elapsed_time(e1) / steps

    wg = {}
    tot_hip = tot_torch = 0.0
    for i, (name, N, K) in enumerate(QWEN3_0P6B):
        x2, gy2 = xs[0][K].detach(), gys[i]
        a, b = lor[0][i][0].detach(), lor[0][i][1].detach()
        hip = wg_ms(lambda: ops.lora_linear_weight_grads_op(x2, gy2, a, b, 2.0, True, True, True))
        tch = wg_ms(lambda: torch_weight_grads(x2, gy2, a, b, 2.0))
        fl = 2.0 * M * (N * K + r * (N + K)) + 2.0 * M * r * (N + K)  # dW, dA, dB + the T, U pre-passes
        wg[name] = {"N": N, "K": K, "hip_ms": round(hip, 4), "torch_ms": round(tch, 4),
                    "hip_TFLOP/s": round(fl / hip / 1e9, 1), "torch_TFLOP/s": round(fl / tch / 1e9, 1)}
        tot_hip += hip
        tot_torch += tch
    # config 2's own projection shape (N = K = 4096)
    x2 = torch.randn(M, 4096, device=dev, generator=g).bfloat16()
    gy2 = torch.randn(M, 4096, device=dev, generator=g).bfloat16()
    a = (torch.randn(r, 4096, device=dev, generator=g) * 0.02).bfloat16()
    b = (torch.randn(4096, r, device=dev, generator=g) * 0.02).bfloat16()
    hip = wg_ms(lambda: ops.lora_linear_weight_grads_op(x2, gy2, a, b, 2.0, True, True, True))
    tch = wg_ms(lambda: torch_weight_grads(x2, gy2, a, b, 2.0))
    fl = 2.0 * M * (4096 * 4096 + r * 8192) + 2.0 * M * r * 8192
    out["weight_grads"] = {"per_projection": wg, "layer_hip_ms": round(tot_hip, 4),
                           "layer_torch_ms": round(tot_torch, 4),
                           "c2_N4096_K4096": {"hip_ms": round(hip, 4), "torch_ms": round(tch, 4),
                                              "hip_TFLOP/s": round(fl / hip / 1e9, 1),
                                              "torch_TFLOP/s": round(fl / tch / 1e9, 1)}}
    del x2, gy2, a, b
    del Ws, xs, lor, gys, gWs, glor, ggys, params
    torch.cuda.empty_cache()
    return out


def bench_embedding(dev, steps, warmup):
    """The factorized embedding at config 4's prefill: 8 x 512 token ids, E [151936, 256],
    P [1024, 256] -> [4096, 1024] bf16 (wsl_factorized_embedding_fwd). Algorithmic bytes:
    the gathered E rows, P, the ids and the output; FLOPs 2 * tokens * 256 * 1024."""
    from weightshared_torchtitan_amd import factorized_embedding
    g = torch.Generator(device=dev).manual_seed(11)
    V, k, H, T = 151936, 256, 1024, 4096
    emb = (torch.randn(V, k, device=dev, generator=g) * 0.02).bfloat16()
    proj = (torch.randn(H, k, device=dev, generator=g) * 0.02).bfloat16()
    ids = torch.randint(0, V, (T,), device=dev, generator=g)
    L = 16
    graph = graph_of(lambda: [factorized_embedding(ids, emb, proj) for _ in range(L)])
    ms = time_replays(graph, steps, warmup) / L
    nbytes = T * k * 2 + H * k * 2 + T * 8 + T * H * 2
    return {"tokens": T, "us": round(ms * 1e3, 3), "Mtok/s": round(T / ms / 1e3, 1),
            "GB/s": round(nbytes / ms / 1e6, 1), "frac_hbm": round(nbytes / ms / 1e6 / HBM_PEAK_GBS, 4),
            "TFLOP/s": round(2.0 * T * k * H / ms / 1e9, 1)}


def c4_step_bytes(a, batch, prompt, n_new):
    """Algorithmic HBM bytes of one config-4 decode step, averaged over the steps: the KV
    cache read at every position up to the step's (K and V, kv heads x head_dim bf16 per
    sequence per layer), each unique block's base weights once, every layer's LoRA factors,
    the embedding table E and P (the tied head reads all of E), and, as a second figure,
    with every layer's base weights counted (no reuse across the 7 layers of a block)."""
    sh = a.proj_shapes()
    base = sum(o * i for o, i in sh.values()) * 2  # one block, bf16
    lora = sum(a.lora_rank * (o + i) for o, i in sh.values()) * 2 * a.n_layers
    emb = a.vocab_size * a.embed_rank * 2 + a.dim * a.embed_rank * 2
    kv_pos = 2 * a.n_kv_heads * a.head_dim * 2 * batch * a.n_layers  # bytes per cached position
    steps = n_new - 1
    mean_len = sum(prompt + i + 1 for i in range(steps)) / steps  # positions 0..pos read at pos
    kv = kv_pos * mean_len
    act = batch * a.dim * 2 * 4 * a.n_layers  # activations in and out of the launches (small)
    unique = kv + base * a.n_unique_blocks + lora + emb + act
    every = kv + base * a.n_layers + lora + emb + act
    return {"unique": unique, "every_layer": every,
            "terms": {"kv_cache": kv, "base_unique": base * a.n_unique_blocks, "lora": lora, "embedding": emb,
                      "activations": act}}


def bench_c4(dev):
    from weightshared_torchtitan_amd.qwen3_shared import SharedQwen3, qwen3_0p6b_shared
    args = qwen3_0p6b_shared()
    args.max_seq_len = 1024
    model = SharedQwen3(args).to(dev)
    model.init_random(seed=4)
    model = model.to(torch.bfloat16)
    g = torch.Generator().manual_seed(4)
    prompt = torch.randint(0, args.vocab_size, (8, 512), generator=g).to(dev)
    model.generate(prompt[:, :16], 4)  # warm-up (allocations, kernel load)
    torch.cuda.synchronize()
    toks, t = model.generate(prompt, 256)
    n_new = 256
    steps = n_new - 1  # the first new token comes from the prefill
    step_ms = t["decode_ms"] / steps
    by = c4_step_bytes(args, batch=8, prompt=512, n_new=n_new)
    res = {"batch": 8, "prompt": 512, "new_tokens": n_new,
           "decode_tok_s": round(8 * n_new / (t["decode_ms"] / 1e3), 1),
           "prefill_ms": round(t["prefill_ms"], 2), "decode_ms": round(t["decode_ms"], 2),
           "ms_per_step": round(step_ms, 4),
           "reference_formula_tok_s": round(8 * (512 + n_new) / ((t["prefill_ms"] + t["decode_ms"]) / 1e3), 1),
           "roofline": {"bound": "hbm", "bytes_per_step": round(by["unique"]),
                        "achieved_GB/s": round(by["unique"] / step_ms / 1e6, 1),
                        "frac": round(by["unique"] / step_ms / 1e6 / HBM_PEAK_GBS, 4),
                        "bytes_per_step_every_layer_weights": round(by["every_layer"]),
                        "frac_every_layer_weights": round(by["every_layer"] / step_ms / 1e6 / HBM_PEAK_GBS, 4),
                        "terms_MB": {k: round(v / 1e6, 2) for k, v in by["terms"].items()}}}
    # the same decode with chains (2 launches per layer: the attention step and one chain of
    # o, gate|up, down and the next layer's q|k|v) instead of one launch per fused projection
    model.decode_chain = True
    _, t2 = model.generate(prompt, n_new)
    res["with_chain"] = {"decode_tok_s": round(8 * n_new / (t2["decode_ms"] / 1e3), 1),
                         "ms_per_step": round(t2["decode_ms"] / steps, 4)}
    del model
    torch.cuda.empty_cache()
    return res


def cpu_threads():
    """Every CPU this process may run on (its affinity set, the box's CPU share), bounded by
    OMP_NUM_THREADS when the environment sets it."""
    try:
        n = len(os.sched_getaffinity(0))
    except AttributeError:
        n = os.cpu_count() or 1
    omp = os.environ.get("OMP_NUM_THREADS", "")
    if omp.isdigit() and int(omp) > 0:
        n = min(n, int(omp))
    return max(1, n)


def cpu_model():
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def bench_c1(dev, steps, warmup):
    """Config 1 exactly: one LoRA linear, x [2048,1024] ~ N(0,1), W [1024,1024], A [16,1024],
    B [1024,16] ~ N(0, 0.02^2), alpha 32 / rank 16 = scale 2, all from one seed.
    CPU: the reference's fp32 arithmetic (F.linear(x,W) + F.linear(F.linear(x,A),B)*s,
    torchtitan/models/llama3/model/model.py:189-192,392-398) on every available host core,
    torch.utils.benchmark median. GPU: the fused op on the same values in bf16, HIP-event
    mean over a graph of 64 launches."""
    import torch.utils.benchmark as tb
    from oracle.qwen3_ref import reference_lora_linear
    from weightshared_torchtitan_amd import lora_linear
    M, N, K, r = 2048, 1024, 1024, 16
    g = torch.Generator().manual_seed(1)
    x = torch.randn(M, K, generator=g)
    W = torch.randn(N, K, generator=g) * 0.02
    A = torch.randn(r, K, generator=g) * 0.02
    B = torch.randn(N, r, generator=g) * 0.02
    threads = cpu_threads()
    torch.set_num_threads(threads)
    t = tb.Timer("f(x, W, A, B, 2.0)", globals={"f": reference_lora_linear, "x": x, "W": W, "A": A, "B": B},
                 num_threads=threads)
    cpu_s = t.blocked_autorange(min_run_time=2.0).median
    fl = lora_flops(M, N, K, r)
    xd, Wd, Ad, Bd = (v.to(dev).bfloat16() for v in (x, W, A, B))
    L = 64
    graph = graph_of(lambda: [lora_linear(xd, Wd, Ad, Bd, 2.0) for _ in range(L)])
    gpu_ms = time_replays(graph, steps, warmup) / L
    del graph
    return {"shape": "x [2048,1024], W [1024,1024], A [16,1024], B [1024,16], scale 2",
            "cpu_fp32": {"us": round(cpu_s * 1e6, 1), "TFLOP/s": round(fl / cpu_s / 1e12, 4), "threads": threads,
                         "cpu_model": cpu_model(), "kind": "reference arithmetic (F.linear x3 + mul + add)"},
            "mi355x_bf16": {"us": round(gpu_ms * 1e3, 3), "TFLOP/s": round(fl / gpu_ms / 1e9, 1),
                            "GB/s": round(lora_bytes(M, N, K, r) / gpu_ms / 1e6, 1)}}


def cpu_baseline(seconds=10.0):
    """The reference's fp32 CPU arithmetic (F.linear(x,W) + F.linear(F.linear(x,A),B)*s),
    timed on every available host core over a bounded sample of the config-2 projections."""
    from oracle.qwen3_ref import reference_lora_linear
    threads = cpu_threads()
    torch.set_num_threads(threads)
    g = torch.Generator().manual_seed(0)
    M = 8192
    xs = {K: torch.randn(M, K, generator=g) for _, _, K in QWEN3_0P6B}
    Ws = [torch.randn(N, K, generator=g) * 0.02 for _, N, K in QWEN3_0P6B]
    As = [torch.randn(32, K, generator=g) * 0.02 for _, _, K in QWEN3_0P6B]
    Bs = [torch.randn(N, 32, generator=g) * 0.02 for _, N, _ in QWEN3_0P6B]
    reference_lora_linear(xs[1024][:256], Ws[0], As[0], Bs[0], 2.0)  # warm-up
    flops, n = 0.0, 0
    t0 = time.perf_counter()
    while True:
        p = n % 7
        _, N, K = QWEN3_0P6B[p]
        reference_lora_linear(xs[K], Ws[p], As[p], Bs[p], 2.0)
        flops += lora_flops(M, N, K, 32)
        n += 1
        el = time.perf_counter() - t0
        if el >= seconds and n >= 7:
            break
    return {"value": round(flops / el / 1e12, 4), "unit": "TFLOP/s", "cores": threads, "kind": "port",
            "cpu_model": cpu_model(), "host_cpus": os.cpu_count(),
            "sample": f"{n} config-2 projections (M=8192, hidden 1024, r=32) in fp32, {el:.1f} s"}


def measured_traffic():
    """HBM bytes per prefill launch at config 2, as recorded from the rocprofv3
    FETCH_SIZE + WRITE_SIZE passes (line `traffic_bytes_per_launch: N`), else None."""
    try:
        with open(TRAFFIC_FILE) as f:
            m = re.search(r"^traffic_bytes_per_launch:\s*([0-9.eE+]+)", f.read(), re.M)
        return float(m.group(1)) if m else None
    except OSError:
        return None


def copy_calibration(dev):
    """A plain copy of COPY_BYTES bytes, three times: reads and writes COPY_BYTES each."""
    src = torch.ones(COPY_BYTES // 2, dtype=torch.bfloat16, device=dev)
    dst = torch.empty_like(src)
    for _ in range(3):
        dst.copy_(src)
    torch.cuda.synchronize()
    del src, dst
    torch.cuda.empty_cache()


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--no-extra", action="store_true")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--only", choices=("c1", "c2", "c2single", "c2_1p7b", "c3", "c4", "c5", "c5paths", "emb",
                                       "vendor", "backward", "medium", "shape", "envab", "stamps", "data"), default=None)
    ap.add_argument("--shape", default="8192,2048,6144,0", help="M,N,K,r for --only shape")
    ap.add_argument("--vendor", action="store_true", help="--only shape: torch.matmul instead of the fused op")
    ap.add_argument("--copy-calibration", action="store_true")
    ap.add_argument("--ab", default='{"default": {}, "strips_off": {"prefill_strips": -1}}',
                    help="--only envab: JSON {mode: {option: value}} of the path overrides timed side by side")
    ap.add_argument("--ab-shapes", default=None, help="--only envab / stamps: comma-separated names from AB_SHAPES (stamps: also "
                         "MEDIUM_STAMP_SHAPES, DECODE_STAMP_SHAPES)")
    ap.add_argument("--opt", action="append", default=[], metavar="NAME=VALUE",
                    help="a libwsl path override for the whole run (ops.path_options names), repeatable")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU only: this build has no multi-GPU path "
              "(the fused LoRA linear is row-independent; see the sharding design).", file=sys.stderr)
        sys.exit(2)
    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        sys.exit(2)
    import weightshared_torchtitan_amd  # noqa: F401  (loads libwsl; fails loudly if missing)
    from weightshared_torchtitan_amd import _native
    for kv in args.opt:
        name, _, val = kv.partition("=")
        _native.set_option(name, int(val))

    dev = torch.device("cuda:0")
    torch.cuda.synchronize()
    if args.copy_calibration:
        copy_calibration(dev)
    if args.only is not None and args.only not in ("c2", "c2single"):
        fn = {"c1": lambda: bench_c1(dev, args.steps, args.warmup),
              "c2_1p7b": lambda: c2_1p7b_extra(dev, args.steps, args.warmup),
              "c3": lambda: bench_c3(dev, args.steps, args.warmup),
              "c4": lambda: bench_c4(dev),
              "c5": lambda: bench_c5(dev, args.steps, args.warmup),
              "c5paths": lambda: bench_c5_paths(dev, args.steps, args.warmup),
              "emb": lambda: bench_embedding(dev, args.steps, args.warmup),
              "vendor": lambda: bench_vendor(dev, args.steps, args.warmup),
              "medium": lambda: bench_medium(dev, min(args.steps, 10), min(args.warmup, 3)),
              "backward": lambda: bench_backward(dev, min(args.steps, 10), min(args.warmup, 3)),
              "shape": lambda: run_shape(dev, tuple(int(v) for v in args.shape.split(",")), args.vendor),
              "envab": lambda: bench_env_ab(dev, json.loads(args.ab),
                                            args.ab_shapes.split(",") if args.ab_shapes else None),
              "stamps": lambda: bench_stamps(dev, args.ab_shapes.split(",") if args.ab_shapes else None),
              "data": lambda: bench_data(dev)}[args.only]
        print(json.dumps({args.only: fn()}), flush=True)
        return
    flops, ms, ms_single = bench_c2(dev, args.steps, args.warmup, grouped=args.only != "c2single",
                                    single=args.only in (None, "c2single"))
    if args.only == "c2single":
        print(json.dumps({"c2single": {"TFLOP/s": round(flops / ms_single / 1e9, 2), "ms_per_step": round(ms_single, 4),
                                       "launches": 7 * 28, "avg_launch_us": round(ms_single * 1e3 / 196, 3)}}),
              flush=True)
        return
    tflops = flops / ms / 1e9
    launches = 4 * 28
    res = {
        "metric": METRIC,
        "value": round(tflops, 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (x ~ N(0,1); W, A, B ~ N(0, 0.02^2); seeded)",
        "config": {"workload": "config 2: Qwen3-0.6B prefill projections, M=8192, 7 proj x 28 layers, "
                               "one shared base W set, per-layer rank-32 LoRA, scale 2; the projections that "
                               "read one activation (q|k|v, gate|up) run as one grouped launch each",
                   "M": 8192, "hidden": 1024, "rank": 32, "layers": 28, "projections": 7,
                   "launches_per_layer": 4},
        "roofline": {"bound": "mfma", "achieved": round(tflops, 2), "peak": BF16_PEAK_TFLOPS,
                     "unit": "TFLOP/s", "frac": round(tflops / BF16_PEAK_TFLOPS, 4), "traffic": measured_traffic(),
                     "kernel": "prefill_kernel (112 launches per step: q|k|v, o, gate|up, down per layer)",
                     "avg_launch_us": round(ms * 1e3 / launches, 3)},
    }
    extra = {}
    if ms_single is not None:
        extra["c2_one_launch_per_projection"] = {"TFLOP/s": round(flops / ms_single / 1e9, 1),
                                                 "frac_mfma": round(flops / ms_single / 1e9 / BF16_PEAK_TFLOPS, 4),
                                                 "ms_per_step": round(ms_single, 4), "launches": 7 * 28}
    if not args.no_extra and args.only is None:
        extra["c1_exact"] = bench_c1(dev, args.steps, args.warmup)
        extra["c2_qwen3_1.7b_prefill"] = c2_1p7b_extra(dev, args.steps, args.warmup)
        extra["c3_qwen3_1.7b_decode"] = bench_c3(dev, args.steps, args.warmup)
        extra["c5_qwen3_8b_fp8_base"] = bench_c5(dev, args.steps, args.warmup)
        extra["c5_qwen3_8b_fp8_base"]["M=4096_paths"] = bench_c5_paths(dev, args.steps, args.warmup)
        extra["c4_weightshared_qwen3_0.6b_decode"] = bench_c4(dev)
        extra["factorized_embedding_c4_prefill"] = bench_embedding(dev, args.steps, args.warmup)
        extra["c2_backward"] = bench_backward(dev, min(args.steps, 10), min(args.warmup, 3))
        extra["medium_m_qwen3_1.7b"] = bench_medium(dev, min(args.steps, 10), min(args.warmup, 3))
    if extra:
        res["extra"] = extra
    if not args.no_cpu and args.only is None:
        res["cpu_baseline"] = cpu_baseline()
    print(json.dumps(res), flush=True)


if __name__ == "__main__":
    main()
