"""Benchmark of the fused per-layer elementwise path on one MI355X.

A step is one pass of the path over one batch at the Llama-3-8B 512-token
prefill shape, as a model loop runs it: the Q4_K token-embedding gather with
the first RMSNorm in one kernel (512 rows of 4096: x and h written), NeoX
RoPE on q (512 x 32 x 128) and k (512 x 8 x 128) at positions 0..511, the
residual add with the next RMSNorm in one kernel (512 x 4096), and SwiGLU on
gate/up (512 x 14336). Inputs are synthetic (seeded), resident in HBM before
timing starts, and rotated over --sets buffer sets (> 1 GiB together) so no
launch reads data the 256 MiB Infinity Cache still holds from the previous
use of its set.

A step replays a recorded plan (aero_hip_plan_launch: the four kernels
issued from C, one host call per step). `value` is the whole step's
algorithmic HBM bytes / wall time per step over the timed region (GB/s).
`ops` also reports the unfused gather and RMSNorm the two fused kernels
replace. Each entry of `ops` gives two device timings of the op: per
dispatch (`kernel_us`, `frac`: the median dispatch, the mean beside it; a
second region of the same run replays plans of the ops with an event pair
recorded by each kernel's own dispatch, hipExtLaunchKernel; events per
kernel serialise the host side, so that region times kernels, not steps)
and sustained (`sustained_us`,
`sustained_frac`: the op alone, launched back to back on one stream over its
own > 1 GiB rotation of buffers, with one HIP event pair on that stream
around the whole region; mean duration = region / launches). `roofline` is
the dominant kernel (SwiGLU, 88 MB per launch): algorithmic bytes / its
median per-dispatch duration, the figure a rocprofv3 kernel trace of the
same command reproduces (the mean and the sustained figure are kept beside
it). `cpu_baseline`
is the same step on the host: the reference's own C++ (built into
oracle/_ref) when present, else the oracle's restatement, single-threaded
like the reference, over a bounded sample, with the reference's threaded
dequant over the same rows beside it.

    python bench.py [--steps K] [--warmup W] [--sets S] [--cpu-seconds T]
    python bench.py --all-shapes        # per-op table over every layer shape
    python bench.py --all-shapes --only OP   # one op over every layer shape
    python bench.py --variants          # every op variant at the 512-token shape
    python bench.py --gemv              # quantised GEMV (decode projections)
    python bench.py --gemm              # quantised GEMM (prefill projections)
    python bench.py --fused             # fused decode GEMVs vs the launches they replace
    python bench.py --layer-gemm        # prefill add+norm folded into the GEMMs vs unfused
    python bench.py --layer             # one decoder block, all fusions on / off
    python bench.py --attention         # attention over a KV cache (decode, prefill)
    python bench.py --gguf              # GGUF parse, upload to HBM, device row addressing
    python bench.py --ssm               # gated DeltaNet scan and conv
    python bench.py --ssm-layer         # one gated-DeltaNet layer (projections .. out)
    python bench.py --only OP --steps K # one kernel only (for counter runs)
    python bench.py --copy-calibration  # a plain copy of known size
    python bench.py --copy-sweep        # copy kernel, runtime copy, fill: 2 MiB to 1 GiB
    python bench.py --sweep             # streaming ops under alternative launch shapes
"""
from __future__ import annotations

import argparse
import ctypes
import json
import os
import re
import statistics
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0  # MI355X HBM3E
SUSTAINED_ROTATION = 5 << 28  # bytes one rotation of buffer sets moves (1.25 GiB)
SUSTAINED_REPS = 8            # rotations timed per op
METRIC = "fused-op HBM GB/s (% of MI355X peak) + rows/s vs CPU ref, Llama-3-8B shapes"
# the ops of the path as separate kernels, and the data-flow fusions that
# replace the gather and the norms in a model loop
UNFUSED_OPS = ("embed_gather", "rmsnorm", "rope_qk", "swiglu")
FUSED_OPS = ("embed_rmsnorm", "add_rmsnorm")
OPS = UNFUSED_OPS + FUSED_OPS
# one layer's elementwise path as a model loop runs it: gather + first norm,
# RoPE on q/k, residual add + norm, act-mul
STEP_OPS = ("embed_rmsnorm", "rope_qk", "add_rmsnorm", "swiglu")


def parse_args(argv=None):
    p = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=200)
    p.add_argument("--warmup", type=int, default=20)
    p.add_argument("--sets", type=int, default=10)
    p.add_argument("--shape", default=None)
    p.add_argument("--cpu-seconds", type=float, default=10.0)
    p.add_argument("--no-cpu", action="store_true")
    p.add_argument("--all-shapes", action="store_true")
    p.add_argument("--shapes", default=None, help="comma list for --all-shapes / --variants")
    p.add_argument("--variants", action="store_true",
                   help="every op variant at the Llama-3-8B 512-token geometry")
    p.add_argument("--gemv", action="store_true", help="quantised GEMV cases")
    p.add_argument("--ssm", action="store_true",
                   help="gated DeltaNet scan and causal conv (Qwen3-Next heads)")
    p.add_argument("--ssm-layer", action="store_true",
                   help="one gated-DeltaNet layer at Qwen3-Next's size (prefill and decode)")
    p.add_argument("--gguf", action="store_true",
                   help="GGUF parse, file-to-HBM upload and device row addressing")
    p.add_argument("--attention", action="store_true",
                   help="attention over a KV cache (decode and causal prefill)")
    p.add_argument("--fused", action="store_true",
                   help="fused decode GEMVs (norm + q/k/v, norm + gate/up + act) vs separate")
    p.add_argument("--layer", action="store_true",
                   help="one decoder block, fused and unfused (decode and 512-token prefill)")
    p.add_argument("--layer-gemm", action="store_true",
                   help="norm -> projections, unfused vs folded into the GEMM (512 tokens)")
    p.add_argument("--gemm", action="store_true",
                   help="quantised GEMM cases (prefill token counts)")
    p.add_argument("--only", choices=OPS + ("gated_norm", "post_norm_add"), default=None)
    p.add_argument("--copy-calibration", action="store_true")
    p.add_argument("--copy-sweep", action="store_true",
                   help="plain copy at 2 MiB .. 1 GiB: the streaming ceiling per size")
    p.add_argument("--host-abi", action="store_true",
                   help="PCIe-inclusive rate of the reference-compatible host ABI")
    p.add_argument("--sweep", action="store_true",
                   help="the streaming ops under every alternative launch shape (tuning knobs)")
    p.add_argument("--launch-floor", action="store_true",
                   help="device duration of a one-block launch")
    return p.parse_args(argv)


# ---------------------------------------------------------------- GPU side
class StepBuffers:
    """One buffer set of a step, in HBM."""

    def __init__(self, s, d_table, rng, only=None):
        from aero_amd.device import DeviceArray as DA

        R = s.n_tok

        def normal(*shape):
            return DA.from_numpy(rng.standard_normal(shape, dtype=np.float32))

        def want(op):
            return only is None or only == op

        if want("embed_gather"):
            self.ids = DA.from_numpy(rng.integers(0, s.vocab, R).astype(np.int32))
            self.emb_out = DA.empty((R, s.hidden))
        if want("rmsnorm"):
            self.x = normal(R, s.hidden)
            self.h = DA.empty((R, s.hidden))
        if want("embed_rmsnorm"):
            self.eids = DA.from_numpy(rng.integers(0, s.vocab, R).astype(np.int32))
            self.ex = DA.empty((R, s.hidden))
            self.eh = DA.empty((R, s.hidden))
        if want("add_rmsnorm"):
            self.rx = normal(R, s.hidden)
            self.rd = normal(R, s.hidden)
            self.rh = DA.empty((R, s.hidden))
        if want("rope_qk"):
            self.q = normal(R, s.hq, s.head_dim)
            self.k = normal(R, s.hk, s.head_dim)
        if want("swiglu"):
            self.gate = normal(R, s.ffn)
            self.up = normal(R, s.ffn)
            self.act_out = DA.empty((R, s.ffn))
        if s.unit_offset and want("post_norm_add"):
            self.py = normal(R, s.hidden)
            self.px = normal(R, s.hidden)
            self.ph = DA.empty((R, s.hidden))
        if s.gated and want("gated_norm"):
            n_v, dd = s.gated
            self.gx = normal(R, n_v * dd)
            self.gz = normal(R, n_v * dd)
            self.gout = DA.empty((R, n_v * dd))
        self.table = d_table

    INPUTS = {"embed_gather": (("ids",), ("emb_out",)), "rmsnorm": (("x",), ("h",)),
              "embed_rmsnorm": (("eids",), ("ex", "eh")), "add_rmsnorm": (("rx", "rd"), ("rh",)),
              "rope_qk": (("q", "k"), ()), "swiglu": (("gate", "up"), ("act_out",)),
              "gated_norm": (("gx", "gz"), ("gout",)),
              "post_norm_add": (("py", "px"), ("ph",))}

    @classmethod
    def copy_for(cls, src, op, rng, vocab):
        """A new set of `op`'s buffers: device copies of `src`'s activations,
        fresh token ids (so no two sets read the same table rows), fresh
        outputs."""
        from aero_amd.device import DeviceArray as DA

        b = cls.__new__(cls)
        ins, outs = cls.INPUTS[op]
        for n in ins:
            a = getattr(src, n)
            setattr(b, n, DA.from_numpy(rng.integers(0, vocab, a.shape).astype(np.int32))
                    if n in ("ids", "eids") else a.clone())
        for n in outs:
            setattr(b, n, DA.empty(getattr(src, n).shape))
        b.table = src.table
        return b


class Path:
    """The ops of one shape, bound to device constants."""

    def __init__(self, name, sets, seed=0, shape=None, only=None):
        from aero_amd import ops
        from aero_amd import workloads as W
        from aero_amd.device import DeviceArray as DA

        self.ops, self.W = ops, W
        s = shape if shape is not None else W.SHAPES[name]
        self.s = s
        self.only = only
        rng = np.random.default_rng(seed)
        bv, bb = W.BLOCK[s.emb_type]
        self.table = self.table_host = None
        if only in (None, "embed_gather", "embed_rmsnorm"):
            self.table_host = W.make_table(s.emb_type, s.vocab * (s.hidden // bv), rng)
            self.table = DA.from_numpy(self.table_host)
        w = rng.standard_normal(s.hidden, dtype=np.float32) * np.float32(0.1)
        self.w = DA.from_numpy(w if s.unit_offset else np.float32(1) + w)
        self.pos_host = W.positions(s, rng)
        self.pos = DA.from_numpy(self.pos_host)
        n_rot, inv = ops.rope_inv_freq(s.n_rot, s.n_rot, s.theta)
        self.inv = DA.from_numpy(inv)
        self.tab = None
        if s.rope_table:
            # the dense position-indexed table, built on the device
            dense = DA.from_numpy(np.arange(s.rope_table, dtype=np.int32))
            half = s.n_rot // 2
            self.tab = (DA.empty((s.rope_table, half)), DA.empty((s.rope_table, half)))
            ops.rope_tables(dense, self.inv, self.tab[0], self.tab[1])
        self.qk_w = None
        if s.qk_norm:
            self.qk_w = (DA.from_numpy(np.float32(0) + rng.standard_normal(s.head_dim,
                                                                           dtype=np.float32) * 0.1),
                         DA.from_numpy(rng.standard_normal(s.head_dim, dtype=np.float32) * 0.1))
        if s.gated:
            self.gw = DA.from_numpy(np.float32(1) + rng.standard_normal(s.gated[1],
                                                                        dtype=np.float32) * 0.1)
        self.sets = [StepBuffers(s, self.table, rng, only) for _ in range(sets)]
        self.scale = float(np.float32(np.sqrt(s.hidden))) if s.emb_scale else 0.0

    def bytes(self):
        W, s = self.W, self.s
        b = {
            "embed_gather": W.bytes_embed(s.n_tok, s.hidden, s.emb_type),
            "rmsnorm": W.bytes_rmsnorm(s.n_tok, s.hidden),
            "rope_qk": W.bytes_rope(s.n_tok, s.hq + s.hk, s.head_dim, s.n_rot, s.qk_norm,
                                    True, bool(s.rope_table)) + (4 * s.head_dim if s.qk_norm
                                                                 else 0),
            "swiglu": W.bytes_act(s.n_tok, s.ffn),
            "embed_rmsnorm": W.bytes_embed_rmsnorm(s.n_tok, s.hidden, s.emb_type),
            "add_rmsnorm": W.bytes_add_rmsnorm(s.n_tok, s.hidden),
        }
        if s.gated:
            b["gated_norm"] = W.bytes_gated(s.n_tok, s.gated[0] * s.gated[1], s.gated[1])
        if s.unit_offset:
            b["post_norm_add"] = W.bytes_post_norm_add(s.n_tok, s.hidden)
        return b

    def rows(self):
        s = self.s
        r = {"embed_gather": s.n_tok, "rmsnorm": s.n_tok, "rope_qk": s.n_tok * (s.hq + s.hk),
             "swiglu": s.n_tok, "embed_rmsnorm": s.n_tok, "add_rmsnorm": s.n_tok}
        if s.gated:
            r["gated_norm"] = s.n_tok
        if s.unit_offset:
            r["post_norm_add"] = s.n_tok
        return r

    def run(self, op, i, stream=None):
        ops, s, b = self.ops, self.s, self.sets[i % len(self.sets)]
        if op == "embed_gather":
            ops.embed_gather(s.emb_type, b.table, s.vocab, s.hidden, b.ids, b.emb_out,
                             scale=self.scale, stream=stream)
        elif op == "rmsnorm":
            ops.rmsnorm(b.x, self.w, b.h, s.n_tok, s.hidden, s.eps, unit_offset=s.unit_offset,
                        stream=stream)
        elif op == "rope_qk":
            kw = {"cos_tab": self.tab[0], "sin_tab": self.tab[1]} if self.tab else {
                "inv_freq": self.inv}
            ops.qk_norm_rope(b.q, s.hq, s.n_tok, s.head_dim, s.n_rot, k=b.k, n_k_heads=s.hk,
                             q_norm_w=self.qk_w[0] if self.qk_w else None,
                             k_norm_w=self.qk_w[1] if self.qk_w else None, eps=s.eps,
                             unit_offset=s.unit_offset, mode=s.rope_mode, pos=self.pos,
                             stream=stream, **kw)
        elif op == "swiglu":
            ops.act_mul(s.act, b.gate, b.up, b.act_out, stream=stream)
        elif op == "embed_rmsnorm":
            ops.embed_rmsnorm(s.emb_type, b.table, s.vocab, s.hidden, b.eids, b.ex, b.eh,
                              self.w, s.eps, scale=self.scale, unit_offset=s.unit_offset,
                              stream=stream)
        elif op == "add_rmsnorm":
            ops.add_rmsnorm(b.rx, b.rd, self.w, b.rh, s.n_tok, s.hidden, s.eps,
                            unit_offset=s.unit_offset, stream=stream)
        elif op == "post_norm_add":
            ops.post_norm_add(b.py, b.px, self.w, self.w, b.ph, s.n_tok, s.hidden, s.eps,
                              ds=0.5, unit_offset=s.unit_offset, stream=stream)
        elif op == "gated_norm":
            ops.gated_rmsnorm_silu(b.gx, b.gz, self.gw, b.gout, s.n_tok,
                                   s.gated[0] * s.gated[1], s.eps, stream=stream)
        else:
            raise ValueError(op)

    def step_ops(self):
        """The kernels a model loop runs for one layer's elementwise path."""
        if self.only:
            return [self.only]
        return list(STEP_OPS) + (["gated_norm"] if self.s.gated else []) + (
            ["post_norm_add"] if self.s.unit_offset else [])

    def report_ops(self):
        """The step's kernels and the unfused ops they replace."""
        if self.only:
            return [self.only]
        return self.step_ops() + [op for op in UNFUSED_OPS if op not in STEP_OPS]


def build_plans(path, ops_list):
    """One recorded plan per buffer set: the given ops in order."""
    from aero_amd.device import Plan

    plans = []
    for i in range(len(path.sets)):
        p = Plan()
        with p:
            for op in ops_list:
                path.run(op, i)
        plans.append(p)
    return plans, ops_list


def kernel_kinds(path, ops_list):
    """Op name of each kernel a step records (an op may record two)."""
    from aero_amd.device import Plan

    kinds = []
    for op in ops_list:
        probe = Plan()
        with probe:
            path.run(op, 0)
        kinds += [op] * len(probe)
        probe.destroy()
    return kinds


def timed_steps(path, steps, warmup):
    """The timed region: `warmup` untimed step replays, then exactly `steps`
    replays (one plan launch, one C call each) bracketed by a stream
    synchronize on both sides. Returns wall ms per step."""
    from aero_amd.device import Stream

    stream = Stream()
    plans, _ = build_plans(path, path.step_ops())
    for i in range(warmup):
        plans[i % len(plans)].launch(stream)
    stream.synchronize()
    t0 = time.perf_counter()
    for i in range(steps):
        plans[(warmup + i) % len(plans)].launch(stream)
    stream.synchronize()
    wall = (time.perf_counter() - t0) * 1e3 / steps
    stream.destroy()
    for p in plans:
        p.destroy()
    return wall


def kernel_times(path, steps, warmup, ops_list):
    """The kernel-timing region: the same replays with every kernel recording
    its own device begin/end (hipExtLaunchKernel events on the stream it runs
    on). Recording events per kernel serialises the host side, so this region
    gives kernel durations, not step throughput. Returns {op: [ms per step]}."""
    from aero_amd.device import Event, Stream, synchronize

    stream = Stream()
    plans, ops_list = build_plans(path, ops_list)
    kinds = kernel_kinds(path, ops_list)
    n_k = len(plans[0])
    assert len(kinds) == n_k
    for i in range(warmup):
        plans[i % len(plans)].launch(stream)
    stream.synchronize()
    evs = [([Event() for _ in range(n_k)], [Event() for _ in range(n_k)]) for _ in range(steps)]
    arrs = [plans[0].event_arrays(a, b) for a, b in evs]
    for i in range(steps):
        plans[(warmup + i) % len(plans)].launch(stream, arrs[i])
    stream.synchronize()
    synchronize()
    ker = {op: [] for op in ops_list}
    for a, b in evs:
        per = {}
        for k in range(n_k):
            per[kinds[k]] = per.get(kinds[k], 0.0) + a[k].elapsed_ms(b[k])
        for op, ms in per.items():
            ker[op].append(ms)
    stream.destroy()
    for p in plans:
        p.destroy()
    return ker


def sustained_times(path, ops_list, reps):
    """Back-to-back launches of one op: a plan issues the op once on each of
    its own buffer sets (together > 1 GiB, or 256 sets for ops under 5 MB,
    so the 256 MiB Infinity Cache holds no set of a large op from its
    previous use) and is replayed `reps` times between
    one event pair on the stream. Returns {op: mean µs per launch}. No event
    is recorded per kernel, so this is the op's cost inside a busy stream."""
    from aero_amd.device import Event, Plan, Stream

    out = {}
    rng = np.random.default_rng(1)
    step_sets = path.sets
    for op in ops_list:
        n = min(256, max(4, -(-SUSTAINED_ROTATION // max(1, path.bytes()[op]))))
        path.sets = [StepBuffers.copy_for(step_sets[i % len(step_sets)], op, rng, path.s.vocab)
                     for i in range(n)]
        plan = Plan()
        with plan:
            for i in range(n):
                path.run(op, i)
        per_plan = len(plan) // n
        stream = Stream()
        for _ in range(2):
            plan.launch(stream)
        e0, e1 = Event(), Event()
        e0.record(stream)
        for _ in range(reps):
            plan.launch(stream)
        e1.record(stream)
        e1.synchronize()
        out[op] = e0.elapsed_ms(e1) * 1e3 / (reps * n)
        assert per_plan >= 1
        plan.destroy()
        stream.destroy()
        path.sets = None  # frees this op's sets before the next op allocates
    path.sets = step_sets
    return out


def op_entry(b, rows, ms_per_dispatch, us_sustained):
    """Per-op figures: per dispatch (events on each kernel; `kernel_us` and
    `frac` from the median dispatch, the mean beside them: a few slow
    dispatches pull the mean) and sustained (back-to-back launches)."""
    us = statistics.median(ms_per_dispatch) * 1e3
    mean = statistics.mean(ms_per_dispatch) * 1e3
    e = {"kernel_us": round(us, 3), "bytes": b,
         "GB/s": round(b / (us * 1e-6) / 1e9, 1),
         "frac": round(b / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
         "kernel_us_mean": round(mean, 3),
         "frac_mean": round(b / (mean * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
         "rows_per_s": round(rows / (us * 1e-6), 1)}
    if us_sustained is not None:
        g = b / (us_sustained * 1e-6) / 1e9
        e.update({"sustained_us": round(us_sustained, 3), "sustained_GB/s": round(g, 1),
                  "sustained_frac": round(g / HBM_PEAK_GBS, 4)})
    return e


# ---------------------------------------------------------------- CPU side
def cpu_baseline(path, seconds):
    """The same step on the host, single-threaded, timed per op around the
    reference's own C entry points (oracle/_ref) or the oracle's."""
    import ctypes
    from ctypes import POINTER, c_float, c_int32, c_uint8

    from oracle import cpuref, refbind

    s, W = path.s, path.W
    use_ref = refbind.available()
    K = refbind.kernels() if use_ref else None
    T = refbind.transformer() if use_ref else None
    C = cpuref.lib()
    fp = lambda a: a.ctypes.data_as(POINTER(c_float))  # noqa: E731
    ip = lambda a: a.ctypes.data_as(POINTER(c_int32))  # noqa: E731
    rng = np.random.default_rng(1)
    R = s.n_tok
    bv, bb = W.BLOCK[s.emb_type]
    rb = (s.hidden // bv) * bb
    table = path.table_host
    ids = rng.integers(0, s.vocab, R).astype(np.int32)
    emb = np.empty((R, s.hidden), np.float32)
    x = rng.standard_normal((R, s.hidden), dtype=np.float32)
    w = (np.float32(1) + rng.standard_normal(s.hidden, dtype=np.float32) * np.float32(0.1))
    h = np.empty_like(x)
    q0 = rng.standard_normal((R, s.hq, s.head_dim), dtype=np.float32)
    k0 = rng.standard_normal((R, s.hk, s.head_dim), dtype=np.float32)
    half = s.n_rot // 2
    pos = path.pos_host.astype(np.int32)
    # a dense 0..max_pos table, as the reference's attention layer builds it
    # (src/attention_layer.cpp:127-135), read by position in apply_rope
    allpos = np.arange(int(pos.max()) + 1, dtype=np.int32)
    n_tab = allpos.size
    cos = np.empty((n_tab, half), np.float32)
    sin = np.empty((n_tab, half), np.float32)
    qpos = np.repeat(pos, s.hq).astype(np.int32)
    kpos = np.repeat(pos, s.hk).astype(np.int32)
    g0 = rng.standard_normal((R, s.ffn), dtype=np.float32)
    up = rng.standard_normal((R, s.ffn), dtype=np.float32)
    tbase = table.ctypes.data

    def embed():
        for i in range(R):
            src = ctypes.cast(tbase + int(ids[i]) * rb, POINTER(c_uint8))
            dst = ctypes.cast(emb.ctypes.data + i * s.hidden * 4, POINTER(c_float))
            if use_ref:
                K.aero_dequant_ref(s.emb_type, src, rb, dst, s.hidden)
            else:
                C.cr_dequant(s.emb_type, src, rb, dst, s.hidden)

    def norm():
        if use_ref:
            T.aero_rmsnorm_rows(fp(x), fp(w), fp(h), R, s.hidden, s.eps)
        else:
            C.cr_rmsnorm_rows(fp(x), fp(w), fp(h), R, s.hidden, s.eps, 0)

    def rope(q, k):
        # the table is rebuilt per call, as the reference's attention layer does
        if use_ref:
            T.aero_rope_tables(s.n_rot, ip(allpos), n_tab, s.theta, s.n_rot, None, 0, fp(cos),
                               fp(sin))
            T.aero_apply_rope(fp(q), R * s.hq, s.head_dim, s.n_rot, fp(cos), fp(sin), ip(qpos), 0)
            T.aero_apply_rope(fp(k), R * s.hk, s.head_dim, s.n_rot, fp(cos), fp(sin), ip(kpos), 0)
        else:
            C.cr_rope_tables(s.n_rot, ip(allpos), n_tab, s.theta, s.n_rot, None, 0, fp(cos),
                             fp(sin))
            C.cr_apply_rope(fp(q), R * s.hq, s.head_dim, s.n_rot, fp(cos), fp(sin), ip(qpos), 0)
            C.cr_apply_rope(fp(k), R * s.hk, s.head_dim, s.n_rot, fp(cos), fp(sin), ip(kpos), 0)

    def swiglu(g):
        if use_ref:
            T.aero_swiglu(fp(g), fp(up), g.size)
        else:
            C.cr_act_mul(0, fp(g), fp(up), fp(g), g.size)

    # the residual add of src/model.cpp:279 (an elementwise loop there; numpy
    # here), then the norm of the sum
    rx0 = rng.standard_normal((R, s.hidden), dtype=np.float32)
    rd = rng.standard_normal((R, s.hidden), dtype=np.float32)

    def add_norm(rx):
        np.add(rx, rd, out=rx)
        if use_ref:
            T.aero_rmsnorm_rows(fp(rx), fp(w), fp(h), R, s.hidden, s.eps)
        else:
            C.cr_rmsnorm_rows(fp(rx), fp(w), fp(h), R, s.hidden, s.eps, 0)

    def embed_norm():
        embed()
        if use_ref:
            T.aero_rmsnorm_rows(fp(emb), fp(w), fp(h), R, s.hidden, s.eps)
        else:
            C.cr_rmsnorm_rows(fp(emb), fp(w), fp(h), R, s.hidden, s.eps, 0)

    times = {op: [] for op in OPS}
    t_end = time.perf_counter() + seconds
    reps = 0
    while reps < 3 or time.perf_counter() < t_end:
        q, k, g, rx = q0.copy(), k0.copy(), g0.copy(), rx0.copy()  # outside the timing
        for op, fn in (("embed_gather", embed), ("rmsnorm", norm),
                       ("rope_qk", lambda: rope(q, k)), ("swiglu", lambda: swiglu(g)),
                       ("embed_rmsnorm", embed_norm), ("add_rmsnorm", lambda: add_norm(rx))):
            t0 = time.perf_counter_ns()
            fn()
            times[op].append((time.perf_counter_ns() - t0) * 1e-6)
        reps += 1
    med = {op: statistics.median(v) for op, v in times.items()}

    # the threaded dequant row (src/kernels.cpp:463-494 at min(hw, 8) threads,
    # src/kernels.cpp:541-548): the same rows' blocks, copied into one
    # contiguous buffer outside the timing, dequantised by the reference's
    # aero_dequant_threaded (or the oracle's restatement of it)
    threads = min(os.cpu_count() or 1, 8)
    raw = np.concatenate([table[int(t) * rb:(int(t) + 1) * rb] for t in ids])
    flat = np.empty(R * s.hidden, np.float32)
    rawp = raw.ctypes.data_as(POINTER(c_uint8))
    thr = []
    t_end = time.perf_counter() + min(seconds, 3.0)
    while len(thr) < 5 or time.perf_counter() < t_end:
        t0 = time.perf_counter_ns()
        ok = (K.aero_dequant_threaded if use_ref else C.cr_dequant_threaded)(
            s.emb_type, rawp, raw.size, fp(flat), flat.size, threads)
        thr.append((time.perf_counter_ns() - t0) * 1e-6)
        assert ok
    assert np.array_equal(flat.reshape(R, s.hidden).view(np.uint32), emb.view(np.uint32))
    threaded = {"ms": round(statistics.median(thr), 3), "threads": threads,
                "reps": len(thr), "entry": "aero_dequant_threaded" if use_ref
                else "cr_dequant_threaded"}
    return med, reps, ("reference" if use_ref else "port"), threaded


# ---------------------------------------------------------------- reports
def traffic_from_profiles(kernel_tag):
    """HBM bytes per launch of the dominant kernel (SwiGLU) from the committed
    counter summary (FETCH_SIZE + WRITE_SIZE, calibrated), or None."""
    path = os.path.join(ROOT, "profiles", "llama3_8b_prefill_counters.md")
    if not os.path.exists(path):
        return None
    m = re.search(r"traffic_bytes_per_launch:\s*([0-9.]+)", open(path).read())
    return float(m.group(1)) if m else None


def main(argv=None):
    a = parse_args(argv)
    if a.gpus != 1:
        print(f"bench.py measures one GPU; --gpus {a.gpus} is not supported "
              "(every op of the path is row-independent, so N GPUs each take 1/N of the rows).",
              file=sys.stderr)
        return 2
    from aero_amd import _lib, workloads as W

    if not _lib.available():
        print(f"HIP path unavailable: {_lib.unavailable_reason()}", file=sys.stderr)
        return 1
    if a.copy_calibration:
        return copy_calibration(a)
    if a.copy_sweep:
        return copy_sweep(a)
    if a.host_abi:
        return host_abi(a)
    if a.launch_floor:
        return launch_floor(a)
    if a.sweep:
        return shape_sweep(a)
    if a.all_shapes:
        return all_shapes(a)
    if a.variants:
        return variants(a)
    if a.gemv:
        return gemv(a)
    if a.gemm:
        return gemm(a)
    if a.layer_gemm:
        return layer_gemm(a)
    if a.layer:
        return layer_bench(a)
    if a.fused:
        return fused(a)
    if a.attention:
        return attention_bench(a)
    if a.gguf:
        return gguf_bench(a)
    if a.ssm:
        return ssm_bench(a)
    if a.ssm_layer:
        return ssm_layer_bench(a)

    name = a.shape or W.HEADLINE
    if a.only:
        # only that op's buffers (two sets beyond 4096 tokens)
        path = Path(name, a.sets if W.SHAPES[name].n_tok <= 4096 else 2, only=a.only)
    else:
        path = Path(name, a.sets)
    if a.only:
        ker = kernel_times(path, a.steps, a.warmup, [a.only])
        b = path.bytes()[a.only]
        med = statistics.median(ker[a.only])
        print(json.dumps({"op": a.only, "shape": name, "kernel_us": round(med * 1e3, 3),
                          "kernel_us_mean": round(statistics.mean(ker[a.only]) * 1e3, 3),
                          "GB/s": round(b / (med * 1e-3) / 1e9, 1), "bytes": b}))
        return 0
    wall = timed_steps(path, a.steps, a.warmup)
    ker = kernel_times(path, a.steps, a.warmup, path.report_ops())
    sus = sustained_times(path, path.report_ops(), SUSTAINED_REPS)
    bts = path.bytes()
    rows = path.rows()
    total = sum(bts[op] for op in path.step_ops())
    value = total / (wall * 1e-3) / 1e9
    per_op = {}
    for op in path.report_ops():
        per_op[op] = op_entry(bts[op], rows[op], ker[op], sus[op])
    dom = "swiglu"
    ach = per_op[dom]["GB/s"]
    out = {
        "metric": METRIC, "value": round(value, 1), "unit": "GB/s", "n_gpus": 1,
        "steps": a.steps, "warmup": a.warmup, "ms_per_step": round(wall, 5),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "f32",
        "data": "synthetic",
        "config": {"workload": f"{name}: one layer's elementwise path as the model loop "
                               f"runs it: Q4_K embedding gather + first RMSNorm (one kernel), "
                               f"NeoX RoPE on q and k, residual add + RMSNorm (one kernel), "
                               f"SwiGLU",
                   "tokens": path.s.n_tok, "hidden": path.s.hidden, "heads": [path.s.hq,
                                                                              path.s.hk],
                   "head_dim": path.s.head_dim, "ffn": path.s.ffn, "buffer_sets": a.sets},
        "rows_per_s": round(path.s.n_tok / (wall * 1e-3), 1),
        "roofline": {"bound": "hbm", "achieved": ach, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(ach / HBM_PEAK_GBS, 4), "traffic": traffic_from_profiles(dom),
                     "kernel": "act_vec_kernel<silu> (SwiGLU 512x14336)",
                     "bytes_per_launch": bts[dom], "launch_us": per_op[dom]["kernel_us"],
                     "launch_us_mean": per_op[dom]["kernel_us_mean"],
                     "frac_mean": per_op[dom]["frac_mean"], "duration": "median dispatch",
                     "sustained_GB/s": per_op[dom]["sustained_GB/s"],
                     "sustained_frac": per_op[dom]["sustained_frac"]},
        "ops": per_op,
    }
    if not a.no_cpu:
        med, reps, kind, threaded = cpu_baseline(path, a.cpu_seconds)
        cpu_ms = sum(med[op] for op in path.step_ops())
        emb_b = bts["embed_gather"]
        out["cpu_baseline"] = {
            "value": round(total / (cpu_ms * 1e-3) / 1e9, 3), "unit": "GB/s", "cores": 1,
            "kind": kind, "rows_per_s": round(path.s.n_tok / (cpu_ms * 1e-3), 1),
            "ms_per_step": round(cpu_ms, 3),
            "ops_ms": {k: round(v, 3) for k, v in med.items()},
            "threaded_dequant": {**threaded, "GB/s": round(emb_b / (threaded["ms"] * 1e-3)
                                                          / 1e9, 3),
                                 "single_thread_ms": round(med["embed_gather"], 3)},
            "sample": f"the full step ({path.s.n_tok} tokens) and the unfused ops, repeated "
                      f"{reps} times (~{a.cpu_seconds:.0f} s), median per op, single thread "
                      f"(the threaded dequant row: {threaded['threads']} threads over the "
                      f"same {path.s.n_tok} rows' blocks), os.cpu_count()={os.cpu_count()}"}
        out["speedup_vs_cpu"] = round(out["value"] / out["cpu_baseline"]["value"], 1)
    print(json.dumps(out))
    return 0


def all_shapes(a):
    """Per-op kernel time, GB/s and fraction of peak for every layer shape."""
    from aero_amd import workloads as W

    res = {}
    names = a.shapes.split(",") if a.shapes else list(W.SHAPES)
    for name in names:
        sets = a.sets if W.SHAPES[name].n_tok <= 4096 else 2
        path = Path(name, sets)
        ops_list = [a.only] if a.only else path.report_ops()
        if (a.only == "gated_norm" and not path.s.gated) or (
                a.only == "post_norm_add" and not path.s.unit_offset):
            continue
        ker = kernel_times(path, max(20, a.steps // 4), 5, ops_list)
        sus = sustained_times(path, ops_list, SUSTAINED_REPS)
        bts, rows = path.bytes(), path.rows()
        res[name] = {}
        for op in ops_list:
            res[name][op] = op_entry(bts[op], rows[op], ker[op], sus[op])
        print(json.dumps({"shape": name, "ops": res[name]}), flush=True)
        del path
    return 0


# The alternative launch shapes of the streaming kernels (AERO_HIP_TUNE keys):
# norm_loop = a persistent grid of that many workgroups per CU (weights in
# registers, next row's loads before this row's stores); norm_vmax = float4 a
# lane before another lane is added to a row (16, 32: one or two waves a row
# at 4096-8192 columns); act_grid = a persistent act grid of that many
# workgroups per CU; act_bs / act_u = lanes per workgroup / float4 per lane.
SWEEP_SHAPES = ("llama3_8b_prefill", "gemma3_4b_prefill", "qwen3next_hybrid",
                "llama3_70b_prefill16k")
SWEEP = (
    (("rmsnorm", "add_rmsnorm", "gated_norm"),
     ({}, {"norm_loop": 1}, {"norm_loop": 2}, {"norm_loop": 4}, {"norm_vmax": 8},
      {"norm_vmax": 16}, {"norm_vmax": 32})),
    (("swiglu",),
     ({}, {"act_grid": 4}, {"act_grid": 16}, {"act_bs": 256}, {"act_bs": 256, "act_grid": 4},
      {"act_u": 2})),
)


def shape_sweep(a):
    """Each streaming op at each large shape under every alternative launch
    shape of SWEEP, set in-process (aero_hip_tune_set) and dropped again:
    median per-dispatch and sustained time, one JSON line per case, the
    default shape first."""
    from aero_amd import workloads as W
    from aero_amd.device import tune_set

    names = a.shapes.split(",") if a.shapes else list(SWEEP_SHAPES)
    for name in names:
        s = W.SHAPES[name]
        for ops_list, knob_sets in SWEEP:
            for op in ops_list:
                if op == "gated_norm" and not s.gated:
                    continue
                path = Path(name, 2 if s.n_tok > 4096 else 4, only=op)
                b = path.bytes()[op]
                for kn in knob_sets:
                    for k, v in kn.items():
                        tune_set(k, v)
                    try:
                        ker = kernel_times(path, 30, 5, [op])[op]
                        sus = sustained_times(path, [op], 4)[op]
                    finally:
                        for k in kn:
                            tune_set(k, None)
                    med = statistics.median(ker) * 1e3
                    print(json.dumps({"shape": name, "op": op, "knobs": kn, "bytes": b,
                                      "kernel_us": round(med, 3),
                                      "frac": round(b / (med * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
                                      "sustained_us": round(sus, 3),
                                      "sustained_frac": round(b / (sus * 1e-6) / 1e9
                                                              / HBM_PEAK_GBS, 4)}), flush=True)
                del path
    return 0


def variants(a):
    """Every op variant at the Llama-3-8B 512-token geometry: per-dispatch and
    sustained time, GB/s and fraction of peak, one JSON line per variant."""
    from aero_amd import workloads as W

    names = a.shapes.split(",") if a.shapes else list(W.VARIANTS)
    unknown = [n for n in names if n not in W.VARIANTS]
    if unknown:
        print(f"--variants: unknown variant(s) {unknown}; one of {list(W.VARIANTS)}",
              file=sys.stderr)
        return 2
    for name in names:
        shape, op = W.VARIANTS[name]
        path = Path(name, a.sets, shape=shape, only=op)
        ker = kernel_times(path, max(20, a.steps // 4), 5, [op])
        sus = sustained_times(path, [op], SUSTAINED_REPS)
        e = op_entry(path.bytes()[op], path.rows()[op], ker[op], sus[op])
        print(json.dumps({"variant": name, "op": op, **e}), flush=True)
        del path
    return 0


GEMV_CASES = [
    # (name, dtype, n_rows, n_cols): Llama-3-8B decode projections in Q4_K, and
    # each block type at the 4096 x 4096 / 14336 x 4096 shapes
    ("attn_q_4096x4096", 12, 4096, 4096), ("attn_kv_1024x4096", 12, 1024, 4096),
    ("ffn_gate_14336x4096", 12, 14336, 4096), ("ffn_down_4096x14336", 12, 4096, 14336),
    ("q8_0_4096x4096", 8, 4096, 4096), ("q8_0_14336x4096", 8, 14336, 4096),
    ("q5_k_14336x4096", 13, 14336, 4096), ("q6_k_14336x4096", 14, 14336, 4096),
    ("iq4_xs_14336x4096", 23, 14336, 4096),
    # hidden 2048 (Qwen3-Next, Llama-3.2-1B): rows of half a 4096-column step
    ("q4_k_8192x2048", 12, 8192, 2048), ("q4_k_2048x8192", 12, 2048, 8192),
    ("q8_0_8192x2048", 8, 8192, 2048),
]


def cpu_matmul_us(t, n_rows, n_cols, n_tok, seconds=1.0):
    """The reference's own matmul (oracle/_ref, src/kernels.cpp:497-538) or
    else the oracle's, one thread, on a sample of rows of the same shape:
    returns (estimated us for all rows, kind, sample description)."""
    import time
    from aero_amd import workloads as W
    from oracle import cpuref, refbind

    use_ref = refbind.available()
    mm = refbind.matmul if use_ref else cpuref.matmul
    rng = np.random.default_rng(2)
    bv, bb = W.BLOCK[t]
    rows = max(1, min(n_rows, (1 << 26) // max(1, n_cols * n_tok)))
    w = W.make_table(t, rows * n_cols // bv, rng)
    X = rng.standard_normal((n_tok, n_cols)).astype(np.float32)
    mm(t, w, X, rows)
    reps, t0 = 0, time.perf_counter()
    while time.perf_counter() - t0 < seconds:
        mm(t, w, X, rows)
        reps += 1
    per_row = (time.perf_counter() - t0) / (reps * rows)
    return (per_row * n_rows * 1e6, "reference" if use_ref else "port",
            f"{rows} of {n_rows} rows x {n_tok} tokens, {reps} calls, one thread")


def gemv(a):
    """Quantised GEMV: sustained time per launch (back to back over a > 1 GiB
    rotation of weight copies), weight GB/s and fraction of HBM peak, for 1, 4
    and 8 tokens per launch."""
    from aero_amd import ops, workloads as W
    from aero_amd.device import DeviceArray as DA, Event, Plan, Stream

    rng = np.random.default_rng(0)
    names = a.shapes.split(",") if a.shapes else [c[0] for c in GEMV_CASES]
    for name, t, n_rows, n_cols in GEMV_CASES:
        if name not in names:
            continue
        bv, bb = W.BLOCK[t]
        w0 = DA.from_numpy(W.make_table(t, n_rows * n_cols // bv, rng))
        wbytes = w0.nbytes
        n_sets = min(256, max(4, -(-SUSTAINED_ROTATION // wbytes)))
        ws = [w0] + [w0.clone() for _ in range(n_sets - 1)]
        res = {"case": name, "dtype": t, "n_rows": n_rows, "n_cols": n_cols,
               "weight_bytes": wbytes}
        for n_tok in (1, 4, 8):
            X = DA.from_numpy(rng.standard_normal((n_tok, n_cols)).astype(np.float32))
            Y = DA.empty((n_tok, n_rows))
            plan = Plan()
            with plan:
                for w in ws:
                    ops.matvec(t, w, X, Y, n_rows, n_cols, n_tok)
            stream = Stream()
            plan.launch(stream)
            e0, e1 = Event(), Event()
            e0.record(stream)
            for _ in range(SUSTAINED_REPS):
                plan.launch(stream)
            e1.record(stream)
            e1.synchronize()
            us = e0.elapsed_ms(e1) * 1e3 / (SUSTAINED_REPS * len(ws))
            b = wbytes + 4 * n_tok * (n_cols + n_rows)
            gbs = b / (us * 1e-6) / 1e9
            res[f"t{n_tok}"] = {"us": round(us, 3), "GB/s": round(gbs, 1),
                                "frac": round(gbs / HBM_PEAK_GBS, 4)}
            plan.destroy()
            stream.destroy()
        if not a.no_cpu:
            cu, kind, sample = cpu_matmul_us(t, n_rows, n_cols, 1)
            res["cpu_baseline"] = {"us_t1": round(cu, 1), "kind": kind, "cores": 1,
                                   "sample": sample}
            res["speedup_vs_cpu_t1"] = round(cu / res["t1"]["us"], 1)
        print(json.dumps(res), flush=True)
        del ws, w0
    return 0


FUSED_CASES = [
    # (name, kind, rows of each matrix, n_cols): Llama-3-8B decode, Q4_K
    ("qkv_4096", "qkv", (4096, 1024, 1024), 4096),
    ("gate_up_silu_14336", "gate_up", (14336, 14336), 4096),
]


def fused(a):
    """Fused decode GEMVs against the separate launches they replace:
    RMSNorm + q/k/v (aero_hip_norm_matvec) vs rmsnorm + three GEMVs, and
    RMSNorm + gate/up + SiLU·mul (aero_hip_norm_gate_up) vs rmsnorm + two GEMVs
    + act_mul; and with a residual input, the same launches with the add in
    their prologue (norm_matmul / norm_matmul_gate_up below 32 tokens) vs
    add_rmsnorm + the fused GEMV without a norm. Sustained time per step
    (recorded plans, back to back over a > 1 GiB rotation of weight sets),
    weight GB/s of the fused launch."""
    from aero_amd import ops, workloads as W
    from aero_amd.device import DeviceArray as DA, Event, Plan, Stream

    t = W.Q4_K
    rng = np.random.default_rng(0)
    names = a.shapes.split(",") if a.shapes else [c[0] for c in FUSED_CASES]
    for name, kind, rows, n_cols in FUSED_CASES:
        if name not in names:
            continue
        w0 = [DA.from_numpy(W.make_table(t, nr * n_cols // 256, rng)) for nr in rows]
        set_bytes = sum(w.nbytes for w in w0)
        n_sets = min(128, max(4, -(-SUSTAINED_ROTATION // set_bytes)))
        sets = [w0] + [[w.clone() for w in w0] for _ in range(n_sets - 1)]
        nw = DA.from_numpy((1 + 0.1 * rng.standard_normal(n_cols)).astype(np.float32))
        res = {"case": name, "dtype": t, "rows": list(rows), "n_cols": n_cols,
               "weight_bytes": set_bytes}
        for n_tok in (1, 2, 4):
            X = DA.from_numpy(rng.standard_normal((n_tok, n_cols)).astype(np.float32))
            H = DA.empty((n_tok, n_cols))
            Ys = [DA.empty((n_tok, nr)) for nr in rows]
            O = DA.empty((n_tok, rows[0]))
            D = DA.from_numpy(rng.standard_normal((n_tok, n_cols)).astype(np.float32))
            XO = DA.empty((n_tok, n_cols))
            out = {}
            for path in ("fused", "separate", "resid_fused", "resid_separate"):
                plan = Plan()
                with plan:
                    for ws in sets:
                        if path == "resid_fused":
                            # x_out = x + d, then the same launch with the add
                            # in its prologue (norm_matmul below 32 tokens)
                            if kind == "qkv":
                                ops.norm_matmul(t, ws, X, Ys, list(rows), n_cols, n_tok,
                                                norm_w=nw, eps=1e-5, d=D, x_out=XO)
                            else:
                                ops.norm_matmul_gate_up(t, ws[0], ws[1], X, O, rows[0], n_cols,
                                                        n_tok, act="silu", norm_w=nw, eps=1e-5,
                                                        d=D, x_out=XO)
                        elif path == "resid_separate":
                            # add + norm, then the fused GEMV on h without a norm
                            ops.add_rmsnorm(X, D, nw, H, n_tok, n_cols, 1e-5, x_out=XO)
                            if kind == "qkv":
                                ops.norm_matvec(t, ws, H, Ys, list(rows), n_cols, n_tok,
                                                norm=False)
                            else:
                                ops.norm_gate_up(t, ws[0], ws[1], H, O, rows[0], n_cols, n_tok,
                                                 act="silu", norm=False)
                        elif kind == "qkv":
                            if path == "fused":
                                ops.norm_matvec(t, ws, X, Ys, list(rows), n_cols, n_tok,
                                                norm_w=nw, eps=1e-5)
                            else:
                                ops.rmsnorm(X, nw, H, n_tok, n_cols, 1e-5)
                                for w, y, nr in zip(ws, Ys, rows):
                                    ops.matvec(t, w, H, y, nr, n_cols, n_tok)
                        else:
                            if path == "fused":
                                ops.norm_gate_up(t, ws[0], ws[1], X, O, rows[0], n_cols, n_tok,
                                                 act="silu", norm_w=nw, eps=1e-5)
                            else:
                                ops.rmsnorm(X, nw, H, n_tok, n_cols, 1e-5)
                                ops.matvec(t, ws[0], H, Ys[0], rows[0], n_cols, n_tok)
                                ops.matvec(t, ws[1], H, Ys[1], rows[1], n_cols, n_tok)
                                ops.act_mul("silu", Ys[0], Ys[1], O, n_tok * rows[0])
                stream = Stream()
                plan.launch(stream)
                e0, e1 = Event(), Event()
                e0.record(stream)
                for _ in range(SUSTAINED_REPS):
                    plan.launch(stream)
                e1.record(stream)
                e1.synchronize()
                us = e0.elapsed_ms(e1) * 1e3 / (SUSTAINED_REPS * len(sets))
                out[path] = us
                plan.destroy()
                stream.destroy()
            gbs = set_bytes / (out["fused"] * 1e-6) / 1e9
            res[f"t{n_tok}"] = {"fused_us": round(out["fused"], 3),
                                "separate_us": round(out["separate"], 3),
                                "speedup": round(out["separate"] / out["fused"], 3),
                                "weight_GB/s": round(gbs, 1),
                                "frac": round(gbs / HBM_PEAK_GBS, 4),
                                "resid_fused_us": round(out["resid_fused"], 3),
                                "resid_separate_us": round(out["resid_separate"], 3),
                                "resid_speedup": round(out["resid_separate"] /
                                                       out["resid_fused"], 3)}
        print(json.dumps(res), flush=True)
        del sets, w0
    return 0


GEMM_CASES = [
    # (name, dtype, n_rows, n_cols, tokens): Llama-3-8B prefill projections
    ("attn_q_4096x4096", 12, 4096, 4096, 512), ("ffn_gate_14336x4096", 12, 14336, 4096, 512),
    ("ffn_down_4096x14336", 12, 4096, 14336, 512), ("q8_0_14336x4096", 8, 14336, 4096, 512),
    ("q6_k_14336x4096", 14, 14336, 4096, 512), ("q6_k_4096x14336", 14, 4096, 14336, 512),
    ("iq4_xs_14336x4096", 23, 14336, 4096, 512),
    ("q6_k_14336x4096_t5", 14, 14336, 4096, 5), ("q6_k_14336x4096_t8", 14, 14336, 4096, 8),
    ("q6_k_14336x4096_t16", 14, 14336, 4096, 16), ("q8_0_14336x4096_t5", 8, 14336, 4096, 5),
    ("iq4_xs_14336x4096_t5", 23, 14336, 4096, 5), ("iq4_xs_14336x4096_t8", 23, 14336, 4096, 8),
    ("q6_k_4096x4096_t8", 14, 4096, 4096, 8), ("q8_0_4096x4096_t8", 8, 4096, 4096, 8),
    ("ffn_down_4096x14336_t3", 12, 4096, 14336, 3), ("ffn_down_4096x14336_t4", 12, 4096, 14336, 4),
    ("q8_0_4096x14336_t4", 8, 4096, 14336, 4), ("attn_o_4096x8192_t4", 12, 4096, 8192, 4),
    ("ffn_gate_14336x4096_t64", 12, 14336, 4096, 64),
    ("q8_0_4096x4096", 8, 4096, 4096, 512), ("q8_0_4096x14336", 8, 4096, 14336, 512),
    ("q8_0_14336x4096_t8", 8, 14336, 4096, 8), ("q8_0_14336x4096_t16", 8, 14336, 4096, 16),
    ("q8_0_14336x4096_t32", 8, 14336, 4096, 32), ("q8_0_4096x4096_t16", 8, 4096, 4096, 16),
    # few tokens (speculative decoding, small batches): the GEMV below the
    # split GEMM's token threshold
    ("ffn_gate_14336x4096_t8", 12, 14336, 4096, 8), ("ffn_gate_14336x4096_t16", 12, 14336, 4096, 16),
    ("ffn_gate_14336x4096_t24", 12, 14336, 4096, 24), ("attn_q_4096x4096_t16", 12, 4096, 4096, 16),
    ("ffn_down_4096x14336_t16", 12, 4096, 14336, 16),
    ("ffn_gate_14336x4096_t4", 12, 14336, 4096, 4), ("ffn_gate_14336x4096_t5", 12, 14336, 4096, 5),
    ("ffn_gate_14336x4096_t6", 12, 14336, 4096, 6), ("ffn_down_4096x14336_t8", 12, 4096, 14336, 8),
    ("attn_q_4096x4096_t8", 12, 4096, 4096, 8), ("attn_q_4096x4096_t12", 12, 4096, 4096, 12),
    ("attn_q_4096x4096_t6", 12, 4096, 4096, 6), ("attn_kv_1024x4096_t8", 12, 1024, 4096, 8),
    ("attn_kv_1024x4096_t12", 12, 1024, 4096, 12), ("attn_kv_1024x4096_t16", 12, 1024, 4096, 16),
]
MFMA_FP32_PEAK_TFLOPS = 157.3
MFMA_FP16_PEAK_TFLOPS = 2500.0   # dense fp16 matrix peak of MI355X


def split_parts():
    """fp16 parts the library's split GEMM cuts x into (2, or 3 in a build with
    -DAERO_SPLIT_PARTS=3), read off its workspace size for 32 tokens of 256
    columns: 32*256*2 bytes a part plus 1280 bytes of sums and scales."""
    from aero_amd import _lib
    return (int(_lib.lib().aero_hip_matmul_workspace(12, 256, 32)) - 1280) // (32 * 256 * 2)


def gemm(a):
    """Quantised GEMM (many tokens): time per launch (events around a few
    back-to-back launches over rotating weight copies), TFLOP/s and the
    fraction of the fp32 matrix peak it runs at."""
    from aero_amd import ops, workloads as W
    from aero_amd.device import DeviceArray as DA, Event, Stream

    rng = np.random.default_rng(0)
    names = a.shapes.split(",") if a.shapes else [c[0] for c in GEMM_CASES]
    for name, t, n_rows, n_cols, n_tok in GEMM_CASES:
        if name not in names:
            continue
        bv, bb = W.BLOCK[t]
        ws = [DA.from_numpy(W.make_table(t, n_rows * n_cols // bv, rng)) for _ in range(4)]
        X = DA.from_numpy(rng.standard_normal((n_tok, n_cols)).astype(np.float32))
        Y = DA.empty((n_tok, n_rows))
        stream = Stream()
        # Q4_K / Q5_K / Q8_0 / Q6_K / IQ4_XS: the split-x fp16 GEMM (the default), then the call
        # without a workspace: the fp32 GEMM from 32 tokens, the GEMV below
        plain = "fp32" if n_tok >= 32 else "gemv"
        paths = ["split_fp16", plain] if t in (W.Q4_K, W.Q5_K, W.Q8_0, W.Q6_K, W.IQ4_XS) else [plain]
        for path in paths:
            split = path == "split_fp16"
            for w in ws:
                ops.matvec(t, w, X, Y, n_rows, n_cols, n_tok, stream=stream, split=split)
            reps = 5
            e0, e1 = Event(), Event()
            e0.record(stream)
            for _ in range(reps):
                for w in ws:
                    ops.matvec(t, w, X, Y, n_rows, n_cols, n_tok, stream=stream, split=split)
            e1.record(stream)
            e1.synchronize()
            us = e0.elapsed_ms(e1) * 1e3 / (reps * len(ws))
            tf = 2.0 * n_rows * n_cols * n_tok / (us * 1e-6) / 1e12
            res = {"case": name, "path": path, "dtype": t, "n_rows": n_rows, "n_cols": n_cols,
                   "tokens": n_tok, "us": round(us, 2), "TFLOP/s": round(tf, 1),
                   "frac_fp32_mfma": round(tf / MFMA_FP32_PEAK_TFLOPS, 4)}
            if split:
                parts = split_parts()
                res["x_parts"] = parts
                res["frac_fp16_mfma_parts"] = round(parts * tf / MFMA_FP16_PEAK_TFLOPS, 4)
            if not a.no_cpu and path == paths[0]:
                cu, kind, sample = cpu_matmul_us(t, n_rows, n_cols, n_tok)
                res["cpu_baseline"] = {"us": round(cu, 1), "kind": kind, "cores": 1,
                                       "sample": sample}
                res["speedup_vs_cpu"] = round(cu / us, 1)
            print(json.dumps(res), flush=True)
        stream.destroy()
        del ws
    return 0


def layer_gemm(a):
    """The prefill layer's two norm -> projection steps at the Llama-3-8B
    512-token shape over Q4_K weights, unfused (add + RMSNorm kernel, then
    the split GEMM per matrix, then act-mul) against the folded forms
    (aero_hip_norm_matmul, aero_hip_norm_matmul_gate_up). Each form is a
    recorded plan replayed back to back over 4 weight sets (> 256 MiB
    together); mean µs per call between one event pair."""
    from aero_amd import ops, workloads as W
    from aero_amd.device import DeviceArray as DA, Event, Plan, Stream

    s = W.SHAPES[W.HEADLINE]
    T, N, F = s.n_tok, s.hidden, s.ffn
    rng = np.random.default_rng(0)
    t = W.Q4_K
    rows = [s.hq * s.head_dim, s.hk * s.head_dim, s.hk * s.head_dim]

    def mat(r):
        return DA.from_numpy(W.make_table(t, r * N // 256, rng))

    sets = [{"qkv": [mat(r) for r in rows], "g": mat(F), "u": mat(F)} for _ in range(4)]
    x = DA.from_numpy(rng.standard_normal((T, N), dtype=np.float32))
    d = DA.from_numpy(rng.standard_normal((T, N), dtype=np.float32))
    w = DA.from_numpy(np.float32(1) + rng.standard_normal(N, dtype=np.float32) * np.float32(0.1))
    h = DA.empty((T, N))
    ys = [DA.empty((T, r)) for r in rows]
    g, u = DA.empty((T, F)), DA.empty((T, F))

    def attn_unfused(m):
        ops.add_rmsnorm(x, d, w, h, T, N, s.eps)
        for wm, y, r in zip(m["qkv"], ys, rows):
            ops.matvec(t, wm, h, y, r, N, T)

    def attn_fused(m):
        ops.norm_matmul(t, m["qkv"], x, ys, rows, N, T, norm_w=w, eps=s.eps, d=d)

    def ffn_unfused(m):
        ops.add_rmsnorm(x, d, w, h, T, N, s.eps)
        ops.matvec(t, m["g"], h, g, F, N, T)
        ops.matvec(t, m["u"], h, u, F, N, T)
        ops.act_mul("silu", g, u, g)

    def ffn_fused(m):
        ops.norm_matmul_gate_up(t, m["g"], m["u"], x, g, F, N, T, act="silu", norm_w=w,
                                eps=s.eps, d=d)

    flops = {"attn": 2.0 * T * N * sum(rows), "ffn": 2.0 * T * N * 2 * F}
    res = {}
    for name, fn in (("attn_unfused", attn_unfused), ("attn_fused", attn_fused),
                     ("ffn_unfused", ffn_unfused), ("ffn_fused", ffn_fused)):
        plan = Plan()
        with plan:
            for m in sets:
                fn(m)
        stream = Stream()
        plan.launch(stream)
        reps = max(5, a.steps // 20)
        e0, e1 = Event(), Event()
        e0.record(stream)
        for _ in range(reps):
            plan.launch(stream)
        e1.record(stream)
        e1.synchronize()
        us = e0.elapsed_ms(e1) * 1e3 / (reps * len(sets))
        kinds = len(plan) // len(sets)
        res[name] = us
        tf = flops[name.split("_")[0]] / (us * 1e-6) / 1e12
        print(json.dumps({"case": name, "us": round(us, 2), "launches": kinds,
                          "TFLOP/s": round(tf, 1), "shape": f"{T}x{N} Q4_K"}), flush=True)
        plan.destroy()
        stream.destroy()
    print(json.dumps({"attn_speedup": round(res["attn_unfused"] / res["attn_fused"], 3),
                      "ffn_speedup": round(res["ffn_unfused"] / res["ffn_fused"], 3),
                      "saved_us": round(res["attn_unfused"] - res["attn_fused"] +
                                        res["ffn_unfused"] - res["ffn_fused"], 2)}), flush=True)
    return 0


LAYER_CASES = [
    # (name, layer geometry, weight type, tokens, earlier cache positions)
    ("qwen2_0p5b_decode", "qwen2_0p5b_decode", 8, 1, 37),
    ("llama3_8b_prefill", "llama3_8b_prefill", 12, 512, 0),
    ("llama3_8b_decode", "llama3_8b_prefill", 12, 1, 4095),    # one token at 4095
    ("llama3_8b_t16", "llama3_8b_prefill", 12, 16, 4080),      # 16 tokens (speculative step)
    # the 512-token prefill in the other split-GEMM types
    ("llama3_8b_prefill_q8_0", "llama3_8b_prefill", 8, 512, 0),
    ("llama3_8b_prefill_q6_k", "llama3_8b_prefill", 14, 512, 0),
    # Gemma blocks (sandwich norms, layer output scale on the deltas) at the
    # Gemma-3-4B-style geometry, 2048-token prefill and one-token decode; a
    # 65536-row embedding table (the gather reads T rows of it)
    ("gemma3_4b_sandwich_prefill", "gemma3_4b_prefill", 12, 2048, 0,
     {"post_norms": True, "out_scale_mode": 1, "vocab": 65536}),
    ("gemma3_4b_sandwich_decode", "gemma3_4b_prefill", 12, 1, 4095,
     {"post_norms": True, "out_scale_mode": 1, "vocab": 65536}),
    # the Qwen3-Next attention layer (output gate, V norm) at 512 tokens
    ("qwen3next_gated_attn_t512", "qwen3next_hybrid", 8, 512, 0,
     {"attn_gate": True, "v_norm": True, "vocab": 65536}),
]


def layer_bench(a):
    """One decoder block (aero_amd.layer.LayerStep: embedding, q/k/v, QK-norm +
    RoPE, attention, o, residual + norm, gate/up + act, down, output norm)
    at the Qwen2-0.5B decode, Llama-3-8B 512-token prefill, Llama-3-8B
    one-token decode (4095 cached positions) and Llama-3-8B 16-token
    (4080 cached positions) shapes, Gemma blocks (sandwich norms) at the
    Gemma-3-4B-style 2048-token prefill and one-token decode, and the
    Qwen3-Next gated attention block at 512 tokens, with
    every fusion on and with every fusion off. Four blocks with their own
    weights (rotated, so weights come from HBM as in a deep model), each
    recorded as a plan; µs per block = region / blocks run, between one
    event pair on the stream. Then the same four blocks as one 4-layer stack
    (one plan; a block's residual add folded into the next block's first
    norm): µs per layer."""
    from aero_amd import layer, select, workloads as W
    from aero_amd.device import Event, Plan, Stream

    names = a.shapes.split(",") if a.shapes else [c[0] for c in LAYER_CASES]
    for case in LAYER_CASES:
        shape, geom, wtype, T, kv_len = case[:5]
        opts = dict(case[5]) if len(case) > 5 else {}
        if shape not in names:
            continue
        vocab = opts.pop("vocab", None)
        cfg = layer.BlockConfig.from_shape(W.SHAPES[geom], wtype, vocab=vocab, **opts)
        weights = [layer.BlockWeights(cfg, seed=i) for i in range(4)]
        rng = np.random.default_rng(5)
        ids = rng.integers(0, cfg.vocab, T).astype(np.int32)
        res = {}
        for mode in ("fused", "unfused"):
            fus = None if mode == "fused" else {f: False for f in select.FUSIONS}
            steps = [layer.LayerStep(cfg, w, T, kv_len + T, fusions=fus) for w in weights]
            plans = []
            for st in steps:
                st.prepare(ids, kv_len)
                p = Plan()
                with p:
                    st.forward(T, kv_len)
                plans.append(p)
            stream = Stream()
            reps = max(3, a.steps // 10)
            for _ in range(reps):          # warm-up as long as the timed region
                for p in plans:
                    p.launch(stream)
            e0, e1 = Event(), Event()
            e0.record(stream)
            for _ in range(reps):
                for p in plans:
                    p.launch(stream)
            e1.record(stream)
            e1.synchronize()
            us = e0.elapsed_ms(e1) * 1e3 / (reps * len(plans))
            res[mode] = us
            print(json.dumps({"layer": shape, "mode": mode, "weight_type": wtype,
                              "tokens": T, "kv_len": kv_len, "us_per_block": round(us, 2),
                              "launches": len(plans[0]),
                              "tokens_per_s_per_block": round(T / (us * 1e-6), 1)}),
                  flush=True)
            for p in plans:
                p.destroy()
            stream.destroy()
            del steps
        print(json.dumps({"layer": shape, "fused_speedup": round(res["unfused"] / res["fused"],
                                                                 3)}), flush=True)
        # the four blocks as one 4-layer stack: one embedding and one output
        # norm, each block's FFN output added by the next block's first norm
        st = layer.LayerStep(cfg, weights, T, kv_len + T)
        st.prepare(ids, kv_len)
        p = Plan()
        with p:
            st.forward(T, kv_len)
        stream = Stream()
        reps = max(3, a.steps // 10)
        for _ in range(reps):
            p.launch(stream)
        e0, e1 = Event(), Event()
        e0.record(stream)
        for _ in range(reps):
            p.launch(stream)
        e1.record(stream)
        e1.synchronize()
        us = e0.elapsed_ms(e1) * 1e3 / (reps * len(weights))
        print(json.dumps({"layer": shape, "mode": "stack", "layers": len(weights),
                          "weight_type": wtype, "tokens": T, "kv_len": kv_len,
                          "us_per_layer": round(us, 2), "launches": len(p),
                          "tokens_per_s_per_layer": round(T / (us * 1e-6), 1)}), flush=True)
        p.destroy()
        stream.destroy()
        del st
    return 0


ATTN_CASES = [
    # (name, query tokens, cached keys, KV type 0 fp32 / 1 int8 / 2 int4[,
    # (query heads, kv heads, head_dim)]); Llama-3-8B heads by default: 32 query
    # heads, 8 kv heads, head_dim 128
    ("decode_s4096_f32", 1, 4096, 0), ("decode_s4096_int8", 1, 4096, 1),
    ("decode_s4096_int4", 1, 4096, 2), ("decode_s16384_f32", 1, 16384, 0),
    ("decode_s32768_int8", 1, 32768, 1), ("prefill_t512_causal_f32", 512, 512, 0),
    # Gemma-3-4B heads (8 / 4, head_dim 256) and Qwen3-Next's attention heads
    # (16 / 2, head_dim 256)
    ("prefill_t2048_causal_f32_gemma3", 2048, 2048, 0, (8, 4, 256)),
    ("prefill_t512_causal_f32_qwen3next", 512, 512, 0, (16, 2, 256)),
    ("decode_s4096_f32_gemma3", 1, 4096, 0, (8, 4, 256)),
    ("decode_s4096_int8_gemma3", 1, 4096, 1, (8, 4, 256)),
]


def cpu_attention_us(T, S, H, HK, D, seconds):
    """The reference's attention_tiled (oracle/_ref, src/transformer.cpp:120-203)
    or else the oracle's, one thread, on the same shape over an fp32 cache."""
    from oracle import cpuref, refbind

    use_ref = refbind.available()
    at = refbind.attention_tiled if use_ref else cpuref.attention_tiled
    rng = np.random.default_rng(3)
    q = rng.standard_normal((T, H, D)).astype(np.float32)
    k = rng.standard_normal((S, HK, D)).astype(np.float32)
    v = rng.standard_normal((S, HK, D)).astype(np.float32)
    qpos = np.arange(S - T, S, dtype=np.int32)
    reps, t0 = 0, time.perf_counter()
    while reps == 0 or time.perf_counter() - t0 < seconds:
        at(q, k, v, 1.0 / np.sqrt(D), qpos=qpos)
        reps += 1
    us = (time.perf_counter() - t0) / reps * 1e6
    return us, "reference" if use_ref else "port", f"the full call, {reps} repeats, one thread"


def attention_bench(a):
    """Attention over a KV cache: mean time per call (a recorded plan of calls
    over rotating caches of > 1 GiB together, one event pair around the
    replays), per-kernel dispatch times (an event pair per kernel), algorithmic
    bytes (K, V and their scales read once, q and out) and, for prefill, flops."""
    from aero_amd import ops
    from aero_amd.device import DeviceArray as DA, Event, Plan, Stream

    rng = np.random.default_rng(0)
    names = a.shapes.split(",") if a.shapes else [c[0] for c in ATTN_CASES]
    for name, T, S, dt, *heads in ATTN_CASES:
        if name not in names:
            continue
        H, HK, D = heads[0] if heads else (32, 8, 128)
        vb = ops.kv_vec_bytes(dt, D)
        kv_bytes = 2 * S * HK * (vb + (4 if dt else 0))
        n_sets = min(64, max(2, -(-SUSTAINED_ROTATION // kv_bytes)))
        src = DA.from_numpy(rng.standard_normal((S, HK, D)).astype(np.float32))
        sets = []
        for _ in range(n_sets):
            if dt == 0:
                sets.append((src.clone(), src.clone(), None, None))
            else:
                side = []
                for _s in range(2):
                    qb, sc = DA.empty(S * HK * vb, np.uint8), DA.empty(S * HK)
                    ops.kv_write(dt, src, S, HK, D, qb, sc, 0, S)
                    side.append((qb, sc))
                sets.append((side[0][0], side[1][0], side[0][1], side[1][1]))
        q = DA.from_numpy(rng.standard_normal((T, H, D)).astype(np.float32))
        out = DA.empty((T, H, D))
        qpos = DA.from_numpy(np.arange(S - T, S, dtype=np.int32))
        scale = 1.0 / np.sqrt(D)
        plan = Plan()
        with plan:
            for k, v, ks, vs in sets:
                ops.attention(q, k, v, out, T, H, HK, D, D, S, scale, qpos=qpos, kv_dt=dt,
                              k_scale=ks, v_scale=vs)
        per_call = len(plan) // n_sets
        stream = Stream()
        plan.launch(stream)
        e0, e1 = Event(), Event()
        reps = max(2, SUSTAINED_REPS // 2)
        e0.record(stream)
        for _ in range(reps):
            plan.launch(stream)
        e1.record(stream)
        e1.synchronize()
        us = e0.elapsed_ms(e1) * 1e3 / (reps * n_sets)
        starts = [Event() for _ in range(len(plan))]
        stops = [Event() for _ in range(len(plan))]
        ev = plan.event_arrays(starts, stops)
        kern = [[] for _ in range(per_call)]
        for _ in range(2):
            plan.launch(stream, ev)
            stream.synchronize()
            for i, (x, y) in enumerate(zip(starts, stops)):
                kern[i % per_call].append(x.elapsed_ms(y) * 1e3)
        kus = [statistics.mean(x) for x in kern]
        b = kv_bytes + 4 * T * H * 2 * D + 4 * T
        pairs = sum(min(S, S - T + t + 1) for t in range(T))
        flops = 2.0 * H * 2 * D * pairs
        gbs = b / (kus[0] * 1e-6) / 1e9
        res = {"case": name, "heads": [H, HK], "head_dim": D, "tokens": T, "keys": S,
               "kv": ["f32", "int8", "int4"][dt], "bytes": b, "us_per_call": round(us, 3),
               "GB/s_per_call": round(b / (us * 1e-6) / 1e9, 1),
               "attn_kernel_us": round(kus[0], 3),
               "roofline": {"bound": "hbm" if T == 1 else "mfma", "achieved": round(
                   gbs if T == 1 else flops / (kus[0] * 1e-6) / 1e12, 2),
                   "peak": HBM_PEAK_GBS if T == 1 else MFMA_FP32_PEAK_TFLOPS,
                   "unit": "GB/s" if T == 1 else "TFLOP/s"}}
        res["roofline"]["frac"] = round(res["roofline"]["achieved"] / res["roofline"]["peak"], 4)
        if per_call > 1:
            res["combine_kernel_us"] = round(kus[1], 3)
        if T > 1:
            res["flops"] = flops
        if not a.no_cpu:
            cu, kind, sample = cpu_attention_us(T, S, H, HK, D, a.cpu_seconds / len(names))
            res["cpu_baseline"] = {"us": round(cu, 1), "kind": kind, "cores": 1,
                                   "sample": sample + ("" if dt == 0 else
                                                       "; fp32 cache, dequantisation not timed")}
            res["speedup_vs_cpu"] = round(cu / us, 1)
        print(json.dumps(res), flush=True)
        plan.destroy()
        stream.destroy()
        del sets, src
    return 0


PCIE_GEN5_X16_GBS = 64.0  # host link, one direction


def gguf_image(meta, tensors, alignment: int = 32) -> bytes:
    """The bytes of a GGUF v3 file. `meta`: (key, value type, value) in file
    order, an array value being (element type, items); `tensors`: (name,
    row-major shape, GGML type, raw bytes). The data section starts at the
    first multiple of `alignment` after the index, each tensor at a multiple
    of it within the section, and the file ends on one."""
    import struct

    from aero_amd import gguf as AG

    packed = {AG.GGUF_UINT8: "B", AG.GGUF_INT8: "b", AG.GGUF_UINT16: "H", AG.GGUF_INT16: "h",
              AG.GGUF_UINT32: "I", AG.GGUF_INT32: "i", AG.GGUF_FLOAT32: "f", AG.GGUF_BOOL: "?",
              AG.GGUF_UINT64: "Q", AG.GGUF_INT64: "q", AG.GGUF_FLOAT64: "d"}
    buf = bytearray()

    def text(s):
        b = s.encode("utf-8")
        buf.extend(struct.pack("<Q", len(b)))
        buf.extend(b)

    def value(t, v):
        if t == AG.GGUF_STRING:
            text(v)
        elif t == AG.GGUF_ARRAY:
            et, items = v
            buf.extend(struct.pack("<IQ", et, len(items)))
            if et in packed:
                buf.extend(struct.pack(f"<{len(items)}{packed[et]}", *items))
            else:
                for it in items:
                    value(et, it)
        else:
            buf.extend(struct.pack("<" + packed[t], v))

    def pad():
        buf.extend(bytes(-len(buf) % alignment))

    buf.extend(b"GGUF")
    buf.extend(struct.pack("<IQQ", 3, len(tensors), len(meta)))
    for key, t, v in meta:
        text(key)
        buf.extend(struct.pack("<I", t))
        value(t, v)
    rel = 0
    for name, shape, t, raw in tensors:
        text(name)
        buf.extend(struct.pack(f"<I{len(shape)}QIQ", len(shape), *shape[::-1], t, rel))
        rel += len(raw) + (-len(raw) % alignment)
    pad()
    for _name, _shape, _t, raw in tensors:
        buf.extend(raw)
        pad()
    return bytes(buf)


def llama3_gguf(path: str, rng) -> dict:
    """A synthetic Llama-3-8B GGUF file: the model's metadata and tokenizer
    sizes (128256 tokens, 280147 merges), its 291 tensor records with their
    names, the Q4_K token embedding table at full size (128256 x 4096, 295 MB)
    and the norms at full size; the per-layer projections carry one Q4_K block
    each (the index is the model's, the file is not 4.9 GB)."""
    from aero_amd import gguf as AG, workloads as W

    meta = [("general.architecture", AG.GGUF_STRING, "llama"),
            ("general.alignment", AG.GGUF_UINT32, 32)]
    for k, v in (("block_count", 32), ("context_length", 8192), ("embedding_length", 4096),
                 ("feed_forward_length", 14336), ("attention.head_count", 32),
                 ("attention.head_count_kv", 8), ("vocab_size", 128256)):
        meta.append((f"llama.{k}", AG.GGUF_UINT32, v))
    meta += [("llama.rope.freq_base", AG.GGUF_FLOAT32, 500000.0),
             ("llama.attention.layer_norm_rms_epsilon", AG.GGUF_FLOAT32, 1e-5),
             ("tokenizer.ggml.model", AG.GGUF_STRING, "gpt2"),
             ("tokenizer.ggml.tokens", AG.GGUF_ARRAY,
              (AG.GGUF_STRING, [f"\u0120tok{i}" for i in range(128256)])),
             ("tokenizer.ggml.token_type", AG.GGUF_ARRAY, (AG.GGUF_INT32, [1] * 128256)),
             ("tokenizer.ggml.merges", AG.GGUF_ARRAY,
              (AG.GGUF_STRING, [f"\u0120t {i}" for i in range(280147)])),
             ("tokenizer.ggml.bos_token_id", AG.GGUF_UINT32, 128000)]
    emb = W.make_table(12, 128256 * 16, rng).tobytes()
    norm = np.ones(4096, np.float32).tobytes()
    block = W.make_table(12, 1, rng).tobytes()
    tensors = [("token_embd.weight", (128256, 4096), 12, emb)]
    for i in range(32):
        tensors += [(f"blk.{i}.attn_norm.weight", (4096,), 0, norm),
                    (f"blk.{i}.ffn_norm.weight", (4096,), 0, norm)]
        tensors += [(f"blk.{i}.{t}.weight", (1, 256), 12, block)
                    for t in ("attn_q", "attn_k", "attn_v", "attn_output", "ffn_gate", "ffn_up",
                              "ffn_down")]
    tensors += [("output_norm.weight", (4096,), 0, norm), ("output.weight", (1, 256), 12, block)]
    with open(path, "wb") as f:
        f.write(gguf_image(meta, tensors, 32))
    return {"tensors": len(tensors), "file_bytes": os.path.getsize(path),
            "table_bytes": len(emb)}


def gguf_bench(a):
    """GGUF on MI355X: parse time, file-to-HBM upload rate, and device row
    addressing (tensor_rows and the id gather) over the resident table."""
    import tempfile

    from aero_amd import _lib, gguf as AG
    from aero_amd.device import DeviceArray as DA, Event, Stream, time_next_kernel

    rng = np.random.default_rng(0)
    tmp = tempfile.mkdtemp(prefix="aero_gguf_")
    path = os.path.join(tmp, "llama3_8b_q4k.gguf")
    try:
        t0 = time.perf_counter()
        meta = llama3_gguf(path, rng)
        write_s = time.perf_counter() - t0
        L = _lib.load()
        # parse: the library's C++ parse alone, and the full Python reader
        parse_us = []
        for _ in range(5):
            t0 = time.perf_counter()
            h = L.aero_gguf_open(path.encode())
            parse_us.append((time.perf_counter() - t0) * 1e6)
            L.aero_gguf_close(h)
        reader_us = []
        for _ in range(3):
            t0 = time.perf_counter()
            r = AG.GGUFReader(path)
            reader_us.append((time.perf_counter() - t0) * 1e6)
            r.close()
        res = {"case": "parse", "workload": "Llama-3-8B GGUF index (291 tensors, 128256-token "
               "vocabulary, 280147 merges)", "file_bytes": meta["file_bytes"],
               "parse_us": round(statistics.median(parse_us), 1),
               "reader_us": round(statistics.median(reader_us), 1)}
        if not a.no_cpu:
            from oracle import refbind
            Lr = refbind.gguf()
            if Lr is not None:
                ref_us = []
                err = ctypes.create_string_buffer(256)
                for _ in range(5):
                    t0 = time.perf_counter()
                    hr = Lr.rg_open(path.encode(), err, 256)
                    ref_us.append((time.perf_counter() - t0) * 1e6)
                    Lr.rg_close(hr)
                res["cpu_baseline"] = {"us": round(statistics.median(ref_us), 1),
                                       "kind": "reference", "cores": 1,
                                       "sample": "GgufReader constructor (src/gguf.cpp), "
                                                 "median of 5"}
        print(json.dumps(res), flush=True)

        r = AG.GGUFReader(path)
        info = r.tensors["token_embd.weight"]
        up_s = []
        for _ in range(3):
            r.release("token_embd.weight")
            t0 = time.perf_counter()
            dt = r.to_device("token_embd.weight")
            up_s.append(time.perf_counter() - t0)
        gbs = info.nbytes / statistics.median(up_s) / 1e9
        print(json.dumps({"case": "upload", "tensor": "token_embd.weight Q4_K 128256x4096",
                          "bytes": info.nbytes, "s": round(statistics.median(up_s), 4),
                          "GB/s": round(gbs, 2), "of_pcie_gen5_x16": round(gbs / PCIE_GEN5_X16_GBS, 3),
                          "write_s": round(write_s, 2),
                          "note": "pread from the page cache (file just written) into pinned "
                                  "buffers, host-to-device copies overlapped"}), flush=True)

        stream = Stream()
        n = 512
        out = DA.empty((n, 4096))
        ids = DA.from_numpy(rng.integers(0, 128256, n).astype(np.int32))
        row_bytes = info.nbytes // 128256
        b = n * row_bytes + n * 4096 * 4
        for name, run in (("tensor_rows_512", lambda: dt.rows(64000, 64000 + n, out, stream)),
                          ("gather_512", lambda: dt.gather(ids, out, stream=stream))):
            for _ in range(a.warmup):
                run()
            pairs = []
            for _ in range(a.steps):
                e0, e1 = Event(), Event()
                time_next_kernel(e0, e1)
                run()
                pairs.append((e0, e1))
            stream.synchronize()
            us = statistics.mean(x.elapsed_ms(y) * 1e3 for x, y in pairs)
            g = b / (us * 1e-6) / 1e9
            res = {"case": name, "rows": n, "bytes": b, "kernel_us": round(us, 3),
                   "roofline": {"bound": "hbm", "achieved": round(g, 1), "peak": HBM_PEAK_GBS,
                                "unit": "GB/s", "frac": round(g / HBM_PEAK_GBS, 4)}}
            if not a.no_cpu:
                from oracle import refbind
                raw = np.frombuffer(r.tensor_bytes(info), np.uint8)
                rows = raw[64000 * row_bytes:(64000 + n) * row_bytes]
                deq = refbind.dequant if refbind.kernels() is not None else None
                if deq is not None:
                    reps, t0 = 0, time.perf_counter()
                    while reps == 0 or time.perf_counter() - t0 < 1.0:
                        deq(12, rows, n * 4096)
                        reps += 1
                    cu = (time.perf_counter() - t0) / reps * 1e6
                    res["cpu_baseline"] = {"us": round(cu, 1), "kind": "reference", "cores": 1,
                                           "sample": f"aero_dequant_ref of the {n} rows' bytes "
                                                     f"(the core of tensor_rows), {reps} calls"}
            print(json.dumps(res), flush=True)
        stream.destroy()
        r.close()
    finally:
        try:
            os.remove(path)
            os.rmdir(tmp)
        except OSError:
            pass
    return 0


SSM_CASES = [
    # (name, tokens, key heads, value heads, head dim): Qwen3-Next's linear
    # attention is 16 key heads, 32 value heads, d 128; the same prefill at
    # head dims 64 and 256. The qkv conv (8192 channels, kernel 4) is timed
    # beside each.
    ("decode", 1, 16, 32, 128), ("prefill_4096", 4096, 16, 32, 128),
    ("prefill_4096_d64", 4096, 16, 32, 64), ("prefill_4096_d256", 4096, 8, 16, 256),
]


def ssm_bench(a):
    """Gated DeltaNet: per-kernel device times (an event pair per kernel) of
    the prep pass, the scan and the conv; decode against the HBM bytes of the
    state it reads and writes, prefill per token; the reference's C++ on a
    bounded sample of the same shapes beside it."""
    from aero_amd import ops
    from aero_amd.device import DeviceArray as DA, Event, Stream, time_next_kernel

    C, K = 8192, 4
    rng = np.random.default_rng(0)
    stream = Stream()
    for name, T, n_k, n_v, d in SSM_CASES:
        f = lambda *s: DA.from_numpy(rng.standard_normal(s).astype(np.float32))
        q, k, v = f(T, n_k, d), f(T, n_k, d), f(T, n_v, d)
        al, bt = f(T, n_v), f(T, n_v)
        a_log = DA.from_numpy((-np.abs(rng.standard_normal(n_v)) * 0.5).astype(np.float32))
        dtb = f(n_v)
        # decode rotates over 64 layer states (> 256 MB together) so no state
        # is still in the 256 MiB cache from its previous step
        n_states = 64 if T == 1 else 1
        states = [DA.from_numpy((rng.standard_normal((n_v, d, d)) * 0.1).astype(np.float32))
                  for _ in range(n_states)]
        outs = DA.empty((T, n_v, d))
        x, w = f(T, C), f(C, K)
        tail = DA.empty((K - 1) * C)
        cout = DA.empty((T, C))
        reps = a.steps if T == 1 else max(3, a.steps // 20)
        times = {"prep": [], "conv": []}
        for it in range(a.warmup + reps):
            st = states[it % n_states]
            pp, pc = (Event(), Event()), (Event(), Event())
            time_next_kernel(*pp)          # the op's first kernel: the prep pass
            ops.ssm_scan(q, k, v, al, bt, a_log, dtb, st, outs, T, n_k, n_v, d,
                         1.0 / np.sqrt(d), stream=stream)
            time_next_kernel(*pc)          # the conv kernel
            ops.ssm_conv(x, w, tail, K - 1 if it else 0, tail, cout, T, C, K, stream=stream)
            stream.synchronize()
            if it >= a.warmup:
                times["prep"].append(pp[0].elapsed_ms(pp[1]) * 1e3)
                times["conv"].append(pc[0].elapsed_ms(pc[1]) * 1e3)
        # the whole op (prep + scan) back to back; the scan is the rest
        e0, e1 = Event(), Event()
        e0.record(stream)
        for it in range(reps):
            ops.ssm_scan(q, k, v, al, bt, a_log, dtb, states[it % n_states], outs, T, n_k, n_v,
                         d, 1.0 / np.sqrt(d), stream=stream)
        e1.record(stream)
        e1.synchronize()
        op_us = e0.elapsed_ms(e1) * 1e3 / reps
        # short scans (up to 16 tokens) are one kernel, whose time the first
        # event pair measured; longer ones a prep pass and the scan (from 128
        # tokens the chunked scan: chunk pre-pass + state pass)
        fused = T <= 16
        chunked = T >= 128 and os.environ.get("AERO_HIP_TUNE", "").find("ssm_chunk=0") < 0
        n_kern = 1 if fused else (3 if chunked else 2)
        prep_us = 0.0 if fused else statistics.mean(times["prep"])
        scan_us = op_us - prep_us
        conv_us = statistics.mean(times["conv"])
        state_bytes = 2 * n_v * d * d * 4
        io_bytes = 4 * T * (2 * n_k * d + 2 * n_v * d + 2 * n_v)
        conv_bytes = 4 * (2 * T * C + C * K)
        res = {"case": name, "tokens": T, "heads": [n_k, n_v], "d": d,
               "form": "fused" if fused else ("chunked" if chunked else "per-token"),
               "ssm_op_us": round(op_us, 3), "kernels": n_kern,
               "prep_us": round(prep_us, 3), "scan_us": round(scan_us, 3),
               "conv_us": round(conv_us, 3),
               "conv_GB/s": round(conv_bytes / (conv_us * 1e-6) / 1e9, 1)}
        if T == 1:
            g = (state_bytes + io_bytes) / (op_us * 1e-6) / 1e9
            res["roofline"] = {"bound": "hbm", "achieved": round(g, 1), "peak": HBM_PEAK_GBS,
                               "unit": "GB/s", "frac": round(g / HBM_PEAK_GBS, 4),
                               "bytes": state_bytes + io_bytes,
                               "note": "state read + written once, q/k/v/out; whole op"}
        else:
            res["us_per_token"] = round(op_us / T, 4)
            g = conv_bytes / (conv_us * 1e-6) / 1e9
            res["roofline"] = {"bound": "hbm", "achieved": round(g, 1), "peak": HBM_PEAK_GBS,
                               "unit": "GB/s", "frac": round(g / HBM_PEAK_GBS, 4),
                               "kernel": "ssm_conv_kernel", "bytes": conv_bytes}
        if not a.no_cpu:
            from oracle import refbind
            if refbind.ssm() is not None:
                Ts = min(T, 8)
                hq = rng.standard_normal((Ts, n_k, d)).astype(np.float32)
                hv = rng.standard_normal((Ts, n_v, d)).astype(np.float32)
                ha = rng.standard_normal((Ts, n_v)).astype(np.float32)
                hs = (rng.standard_normal((n_v, d, d)) * 0.1).astype(np.float32)
                hl = (-np.abs(rng.standard_normal(n_v)) * 0.5).astype(np.float32)
                reps_c, t0 = 0, time.perf_counter()
                while reps_c == 0 or time.perf_counter() - t0 < 1.0:
                    refbind.ssm_scan(hq, hq, hv, ha, ha, hl, hl, hs, 0.088)
                    reps_c += 1
                per_tok = (time.perf_counter() - t0) / (reps_c * Ts) * 1e6
                hx = rng.standard_normal((Ts, C)).astype(np.float32)
                hw = rng.standard_normal((C, K)).astype(np.float32)
                reps_v, t0 = 0, time.perf_counter()
                while reps_v == 0 or time.perf_counter() - t0 < 0.5:
                    refbind.ssm_conv(hx, hw, None, 0)
                    reps_v += 1
                conv_tok = (time.perf_counter() - t0) / (reps_v * Ts) * 1e6
                res["cpu_baseline"] = {"scan_us": round(per_tok * T, 1),
                                       "conv_us": round(conv_tok * T, 1), "kind": "reference",
                                       "cores": 1,
                                       "sample": f"aero_ssm_scan / aero_ssm_conv on {Ts} tokens "
                                                 f"({reps_c} / {reps_v} calls), per token x {T}"}
                res["speedup_vs_cpu_scan"] = round(per_tok * T / op_us, 1)
        print(json.dumps(res), flush=True)
    stream.destroy()
    return 0


SSM_LAYER_CASES = [
    # (name, tokens): Qwen3-Next's linear-attention layer, hidden 2048, 16 key
    # and 32 value heads of 128, conv kernel 4, Q4_K projections
    ("prefill_4096", 4096), ("decode", 1),
]


def ssm_layer_bench(a):
    """One gated-DeltaNet layer (aero_amd.ssm_layer, aero_ssm_forward_q of
    src/ssm.cpp:262-352) recorded as a plan: mean time per layer over plan
    replays, per-launch device times (an event pair a launch), the weight
    bytes a call streams; the reference's aero_ssm_forward_q on a bounded
    sample of tokens on one host core beside it."""
    from aero_amd import ssm_layer as S
    from aero_amd import workloads as W
    from aero_amd.device import Event, Plan, Stream

    cfg = S.SsmConfig(2048, 16, 32, 128, 4, (W.Q4_K,) * 5)
    wts = S.SsmWeights(cfg, seed=0)
    w_bytes = sum(wts.host[n].nbytes for n in S.PROJ)
    rng = np.random.default_rng(0)
    for name, T in SSM_LAYER_CASES:
        step = S.SsmStep(cfg, wts, max_tokens=T)
        step.x.view((T, cfg.hidden)).copy_from(rng.standard_normal((T, cfg.hidden),
                                                                   dtype=np.float32))
        # eager steps until the conv history holds kernel - 1 rows (a plan
        # records the history length it was made with)
        while step.tail_len < cfg.conv_kernel - 1:
            step.forward(T)
        stream = Stream()
        plan = Plan()
        with plan:
            step.forward(T, stream=stream)
        n = len(plan)
        reps = a.steps if T == 1 else max(5, a.steps // 10)
        for _ in range(a.warmup):
            plan.launch(stream)
        e0, e1 = Event(), Event()
        e0.record(stream)
        for _ in range(reps):
            plan.launch(stream)
        e1.record(stream)
        e1.synchronize()
        us = e0.elapsed_ms(e1) * 1e3 / reps
        starts, stops = [Event() for _ in range(n)], [Event() for _ in range(n)]
        ev = plan.event_arrays(starts, stops)
        kern = [[] for _ in range(n)]
        for _ in range(3):
            plan.launch(stream, ev)
            stream.synchronize()
            for i, (x, y) in enumerate(zip(starts, stops)):
                kern[i].append(x.elapsed_ms(y) * 1e3)
        res = {"case": name, "tokens": T, "hidden": cfg.hidden, "heads": [cfg.n_k, cfg.n_v],
               "d": cfg.head_dim, "weights": "Q4_K", "launches": n,
               "us_per_layer": round(us, 2), "us_per_token": round(us / T, 4),
               "launch_us": [round(statistics.mean(k), 2) for k in kern],
               "weight_bytes": w_bytes,
               "weight_GB/s": round(w_bytes / (us * 1e-6) / 1e9, 1)}
        if not a.no_cpu:
            from oracle import refbind
            if refbind.ssm() is not None:
                h = wts.host
                Ts = min(T, 2)
                case = dict(dts=list(cfg.wtypes), weights=[h[k] for k in S.PROJ],
                            a_log=h["a_log"], dt_bias=h["dt_bias"], conv1d=h["conv1d"],
                            norm=h["norm"], n_k=cfg.n_k, d=cfg.head_dim, inner=cfg.inner,
                            eps=cfg.eps, norm_eps=cfg.norm_eps)
                x = rng.standard_normal((Ts, cfg.hidden)).astype(np.float32)
                tail = np.zeros((cfg.conv_kernel - 1, cfg.qkv), np.float32)
                st = np.zeros((cfg.n_v, cfg.head_dim, cfg.head_dim), np.float32)
                calls, t0 = 0, time.perf_counter()
                while calls == 0 or time.perf_counter() - t0 < min(a.cpu_seconds, 5.0):
                    refbind.ssm_forward(x, tail=tail, tail_len=0, state=st, threads=1, **case)
                    calls += 1
                per_tok = (time.perf_counter() - t0) / (calls * Ts) * 1e6
                res["cpu_baseline"] = {"us": round(per_tok * T, 1), "kind": "reference",
                                       "cores": 1,
                                       "sample": f"aero_ssm_forward_q on {Ts} tokens ({calls} "
                                                 f"calls), per token x {T}"}
                res["speedup_vs_cpu"] = round(per_tok * T / us, 1)
        print(json.dumps(res), flush=True)
        plan.destroy()
        stream.destroy()
    return 0


def copy_calibration(a):
    """A plain fp32 copy of 256 MiB, for scaling FETCH_SIZE / WRITE_SIZE."""
    from aero_amd import ops
    from aero_amd.device import DeviceArray as DA, Event, synchronize, time_next_kernel

    n = 64 * 1024 * 1024
    bufs = [(DA.empty(n), DA.empty(n)) for _ in range(4)]
    ts = []
    for i in range(a.warmup + a.steps):
        src, dst = bufs[i % 4]
        e0, e1 = Event(), Event()
        time_next_kernel(e0, e1)
        ops.copy_f32(src, dst)
        if i >= a.warmup:
            ts.append((e0, e1))
    synchronize()
    m = statistics.mean(x.elapsed_ms(y) for x, y in ts)
    print(json.dumps({"copy_bytes_read": 4 * n, "copy_bytes_written": 4 * n,
                      "kernel_us": round(m * 1e3, 2),
                      "GB/s": round(8 * n / (m * 1e-3) / 1e9, 1)}))
    return 0


def copy_sweep(a):
    """The streaming ceiling at each launch size, three ways: this library's
    plain fp32 copy kernel (`aero_hip_copy_f32`, the act kernel's access
    pattern: one read and one write per element), the HIP runtime's own
    device-to-device copy (`hipMemcpyAsync`, which runs the runtime's blit
    kernel), and a store-only fill (`aero_hip_fill_f32`, the ceiling of a
    kernel whose bytes are nearly all writes, like the embedding gathers),
    each of total traffic 2 MiB .. 1 GiB, rotated over buffers of > 1.5 GiB
    together. The kernels are timed per dispatch by their own events; the
    runtime copy by an event pair on its stream around each call (a
    rocprofv3 kernel trace of the same command times all three alike). One
    JSON line per size and copy."""
    from aero_amd import _lib, ops
    from aero_amd.device import DeviceArray as DA, Event, Stream, synchronize, time_next_kernel

    L = _lib.lib()
    stream = Stream()
    for mib in (2, 4, 8, 16, 32, 64, 128, 256, 512, 1024):
        n = mib * (1 << 20) // 8                 # floats per buffer (read + write = mib)
        k = max(2, -(-(3 << 29) // (8 * n)))     # buffer pairs over 1.5 GiB
        bufs = [(DA.empty(n), DA.empty(n)) for _ in range(k)]
        fills = [DA.empty(2 * n) for _ in range(k)]
        for how in ("kernel", "hipMemcpyAsync", "fill"):
            ts = []
            for i in range(a.warmup + a.steps):
                src, dst = bufs[i % k]
                e0, e1 = Event(), Event()
                if how == "kernel":
                    time_next_kernel(e0, e1)
                    ops.copy_f32(src, dst, stream=stream)
                elif how == "fill":
                    # write-only, the same byte count as the copy's read + write
                    time_next_kernel(e0, e1)
                    ops.fill_f32(fills[i % k], 1.0, stream=stream)
                else:
                    e0.record(stream)
                    _lib.check(L.aero_hip_memcpy_dtod(dst.ptr, src.ptr, 4 * n, stream.handle),
                               "memcpy D2D")
                    e1.record(stream)
                if i >= a.warmup:
                    ts.append((e0, e1))
            synchronize()
            us = [x.elapsed_ms(y) * 1e3 for x, y in ts]
            m = statistics.mean(us)
            med = statistics.median(us)
            print(json.dumps({"copy": how, "copy_bytes": 8 * n, "kernel_us": round(m, 3),
                              "kernel_us_median": round(med, 3),
                              "GB/s": round(8 * n / (m * 1e-6) / 1e9, 1),
                              "frac_median": round(8 * n / (med * 1e-6) / 1e9 / HBM_PEAK_GBS,
                                                   4)}), flush=True)
        del bufs, fills, ts
    stream.destroy()
    return 0


def host_abi(a):
    """The reference-compatible host-pointer entry points at the 512-token
    shape: algorithmic bytes / wall time of the whole call, PCIe both ways
    included, beside the reference's own C++ (oracle/_ref, one thread) on the
    same arrays. Inputs an op modifies in place are fresh copies made outside
    the timing."""
    from aero_amd import native as NK, tensor_native as TN, transformer_native as N
    from aero_amd import workloads as W
    from oracle import refbind

    s = W.SHAPES[W.HEADLINE]
    rng = np.random.default_rng(0)
    x = rng.standard_normal((s.n_tok, s.hidden), dtype=np.float32)
    w = np.float32(1) + rng.standard_normal(s.hidden, dtype=np.float32) * np.float32(0.1)
    g = rng.standard_normal((s.n_tok, s.ffn), dtype=np.float32)
    u = rng.standard_normal((s.n_tok, s.ffn), dtype=np.float32)
    q = rng.standard_normal((s.n_tok * s.hq, s.head_dim), dtype=np.float32)
    c, si = N.rope_tables(s.head_dim, np.arange(s.n_tok), s.theta)
    qpos = np.repeat(np.arange(s.n_tok), s.hq).astype(np.int32)
    raw = W.make_table(s.emb_type, s.n_tok * (s.hidden // 256), rng).tobytes()
    raw_np = np.frombuffer(raw, np.uint8)
    use_ref = refbind.available()
    reps = max(3, a.steps // 20)
    cases = [
        ("transformer_native.rmsnorm_rows", lambda _: N.rmsnorm_rows(x, w, s.eps),
         (lambda _: refbind.rmsnorm_rows(x, w, s.eps)) if use_ref else None, None,
         W.bytes_rmsnorm(s.n_tok, s.hidden)),
        ("tensor_native.swiglu", lambda gi: TN.swiglu(gi, u),
         (lambda gi: refbind.swiglu(gi, u)) if use_ref else None, g, W.bytes_act(s.n_tok, s.ffn)),
        ("transformer_native.apply_rope(q)", lambda _: N.apply_rope(q, c, si, qpos),
         (lambda _: refbind.apply_rope(q, c, si, qpos)) if use_ref else None, None,
         8 * q.size),
        ("native.dequant(Q4_K, 512 rows)",
         lambda _: NK.dequant(s.emb_type, raw, (s.n_tok, s.hidden)),
         (lambda _: refbind.dequant(s.emb_type, raw_np, s.n_tok * s.hidden)) if use_ref
         else None, None, W.bytes_embed(s.n_tok, s.hidden, s.emb_type)),
    ]

    def timed(fn, fresh):
        fn(None if fresh is None else fresh.copy())
        ts = []
        for _ in range(reps):
            arg = None if fresh is None else fresh.copy()
            t0 = time.perf_counter()
            fn(arg)
            ts.append(time.perf_counter() - t0)
        return statistics.median(ts)

    out = {}
    for name, fn, ref, fresh, b in cases:
        m = timed(fn, fresh)
        e = {"ms": round(m * 1e3, 3), "GB/s_incl_pcie": round(b / m / 1e9, 2)}
        if ref is not None:
            r = timed(ref, fresh)
            e.update({"reference_cpu_ms": round(r * 1e3, 3), "speedup_vs_cpu": round(r / m, 2)})
        out[name] = e
    print(json.dumps({"host_abi_llama3_8b_prefill": out, "reps": reps,
                      "cpu": "reference C++ (oracle/_ref), one thread" if use_ref else None}))
    return 0


def launch_floor(a):
    """Device duration of a one-block launch (act_mul on 4 floats)."""
    from aero_amd import ops
    from aero_amd.device import DeviceArray as DA, Event, synchronize, time_next_kernel

    g, u, o = DA.empty(4), DA.empty(4), DA.empty(4)
    pairs = []
    for i in range(a.warmup + a.steps):
        e0, e1 = Event(), Event()
        time_next_kernel(e0, e1)
        ops.act_mul("silu", g, u, o)
        if i >= a.warmup:
            pairs.append((e0, e1))
    synchronize()
    ts = sorted(x.elapsed_ms(y) * 1e3 for x, y in pairs)
    print(json.dumps({"one_block_kernel_us_median": round(ts[len(ts) // 2], 3),
                      "min_us": round(ts[0], 3)}))
    return 0


if __name__ == "__main__":
    sys.exit(main())
