"""Device-resident gated-DeltaNet layers: the SSM counterpart of layer.py.

One linear-attention layer of the reference, aero_ssm_forward_q
(src/ssm.cpp:262-352), over quantised weights resident in HBM, with its
recurrent state and conv history kept on the device between calls:

    qkv, gate, alpha, beta = x Wqkv, x Wgate, x Walpha, x Wbeta   :289-315
    c = silu(conv(tail ++ qkv))      causal depthwise, kernel K     :297-301
    o = scan(q, k, v slices of c, alpha, beta; state)               :316-320
    o = rmsnorm(o over the whole row) * norm[c % d] * silu(gate)    :322-340
    out = o Wout                                                    :343-348

x is the layer's input, already normed (the reference's caller passes it so).
Projections of one weight type that read x go to the GPU in one launch (up
to four matrices); the silu runs in the conv's store, and the scan reads
q, k and v as strided slices of the conv output (scan_strided, :128-142),
so five launches carry the layer (the scan adds its prep pass and, from 128
tokens, the chunk pre-pass). The gated norm runs inside the output
projection (fusion "norm_gemm"): in its GEMV prologue at one or two tokens,
in the split GEMM's x pre-pass on that path. At one or two tokens the conv
also writes its history, and at one token (fusion "conv_gemm": one weight
type for the four input projections) the conv and silu run on the qkv rows
in the projections' GEMV epilogue: three launches. The gated norm site consults aero_amd.select
(op "gated_norm") like the decoder block's sites; the projections, conv and
scan have no host path. With every op on the GPU, `forward` can be recorded
as a Plan once the conv history is full (kernel - 1 rows, from the second
call on): the history length is a launch argument, so a recording refuses
a shorter one rather than replay it.
"""
from __future__ import annotations

from dataclasses import dataclass

import numpy as np

from . import ops, select
from . import workloads as W
from .device import DeviceArray as DA, Stream, recording_plan

# projection order of aero_ssm_forward_q's weight descriptors (src/ssm.cpp:224-225)
PROJ = ("qkv", "gate", "alpha", "beta", "out")


@dataclass(frozen=True)
class SsmConfig:
    hidden: int          # n_embd
    n_k: int             # key heads (n_group)
    n_v: int             # value heads (time_step_rank)
    head_dim: int        # state_size d: 64, 128 or 256
    conv_kernel: int
    wtypes: tuple        # ggml types of (qkv, gate, alpha, beta, out)
    eps: float = 1e-6        # q / k l2-norm floor
    norm_eps: float = 1e-6   # the gated norm's

    @property
    def inner(self) -> int:
        return self.n_v * self.head_dim

    @property
    def qkv(self) -> int:
        return 2 * self.n_k * self.head_dim + self.inner

    def shapes(self) -> dict:
        """(rows, columns) of each projection."""
        N, I = self.hidden, self.inner
        return {"qkv": (self.qkv, N), "gate": (I, N), "alpha": (self.n_v, N),
                "beta": (self.n_v, N), "out": (N, I)}


class SsmWeights:
    """Synthetic weights of one layer (seeded): quantised projections of
    trained-like scale, the conv taps, a_log < 0, dt_bias, the norm weight;
    kept on the host (`host`) and in HBM (`dev`)."""

    def __init__(self, cfg: SsmConfig, seed: int = 0):
        rng = np.random.default_rng(seed)
        h = {}
        for (name, (r, c)), t in zip(cfg.shapes().items(), cfg.wtypes):
            if c % W.BLOCK[t][0]:
                raise ValueError(f"{name}: {c} columns are not whole {W.BLOCK[t][0]}-value blocks")
            h[name] = W.weight_table(t, r, c, rng)
        f = lambda *s: rng.standard_normal(s, dtype=np.float32)
        h["conv1d"] = (f(cfg.qkv, cfg.conv_kernel) * np.float32(0.5)).astype(np.float32)
        h["a_log"] = (-np.abs(f(cfg.n_v)) * np.float32(0.5)).astype(np.float32)
        h["dt_bias"] = f(cfg.n_v)
        h["norm"] = (np.float32(1) + f(cfg.head_dim) * np.float32(0.1)).astype(np.float32)
        self.host = h
        self.dev = {k: DA.from_numpy(v) for k, v in h.items()}


class SsmStep:
    """One gated-DeltaNet layer over device buffers sized for `max_tokens`
    tokens a call, with its state [n_v, d, d] and conv history [K-1, qkv] in
    HBM (both zero at the start; `reset()` zeroes them again).

        step = SsmStep(cfg, SsmWeights(cfg), max_tokens=4096)
        step.x.view((T, cfg.hidden)).copy_from(h)   # the normed layer input
        step.forward(T)                             # or record it in a Plan
        out = step.out                              # [T, hidden], in HBM
    """

    def __init__(self, cfg: SsmConfig, weights: SsmWeights, max_tokens: int,
                 gpu_ops: dict | None = None, fusions: dict | None = None,
                 hooks: dict | None = None):
        if cfg.head_dim not in (64, 128, 256):
            raise ValueError(f"head dim {cfg.head_dim}: the device scan takes 64, 128 or 256")
        if cfg.n_v % cfg.n_k:
            raise ValueError(f"{cfg.n_v} value heads are not a multiple of {cfg.n_k} key heads")
        if not 1 <= cfg.conv_kernel <= 16:
            raise ValueError(f"conv kernel {cfg.conv_kernel} outside 1..16")
        self.cfg, self.w = cfg, weights
        self.gpu_ops, self.fusions, self.hooks = gpu_ops or {}, fusions or {}, hooks or {}
        T, N, I, Q = max_tokens, cfg.hidden, cfg.inner, cfg.qkv
        self.max_tokens = T
        self.x, self.out = DA.empty((T, N)), DA.empty((T, N))
        self.qkv, self.conv = DA.empty((T, Q)), DA.empty((T, Q))
        self.gate, self.o, self.on = DA.empty((T, I)), DA.empty((T, I)), DA.empty((T, I))
        self.alpha, self.beta = DA.empty((T, cfg.n_v)), DA.empty((T, cfg.n_v))
        self.state = DA.empty((cfg.n_v, cfg.head_dim, cfg.head_dim))
        self.tail = DA.empty((max(cfg.conv_kernel - 1, 1), Q))
        self.scale = float(np.float32(1.0) / np.sqrt(np.float32(cfg.head_dim)))
        # projections of x, grouped by weight type (one launch a group)
        outs = {"qkv": self.qkv, "gate": self.gate, "alpha": self.alpha, "beta": self.beta}
        groups: dict = {}
        for name, t in zip(PROJ[:4], cfg.wtypes[:4]):
            groups.setdefault(t, []).append(name)
        self.groups = [(t, names, [outs[n] for n in names]) for t, names in groups.items()]
        # decode folds the conv into the projections' GEMV: one weight type for
        # the four, kernel 4, rows of whole 16 bytes (the 64-column lane GEMV)
        bv, bb = W.BLOCK[cfg.wtypes[0]]
        self.conv_fold = (len(self.groups) == 1 and cfg.conv_kernel == 4 and
                          cfg.hidden % bv == 0 and (cfg.hidden // bv * bb) % 16 == 0)
        self.reset()

    def reset(self) -> None:
        """Zero the state and forget the conv history."""
        self.state.copy_from(np.zeros(self.state.shape, np.float32))
        self.tail_len = 0

    def gpu(self, op: str) -> bool:
        if select.enabled(op, self.gpu_ops.get(op), default=True):
            return True
        if op in self.hooks:
            return False
        raise select.HostPathRequired(
            f"op {op!r} is off the GPU ({select.ENV}) and no host hook was given for it")

    def forward(self, T: int, stream: Stream | None = None) -> None:
        """The layer on the first T rows of self.x; out in self.out."""
        cfg, dev = self.cfg, self.w.dev
        if not 0 < T <= self.max_tokens:
            raise ValueError(f"{T} tokens: outside 1..{self.max_tokens}")
        if recording_plan() is not None and self.tail_len < cfg.conv_kernel - 1:
            # the history length is a launch argument: a recording made now
            # would replay this short history on every later step
            raise ValueError(f"forward: recording a plan with {self.tail_len} rows of conv "
                             f"history (fewer than {cfg.conv_kernel - 1}); record it once "
                             f"the history is full")
        shapes = cfg.shapes()
        x = self.x.view((T, cfg.hidden))
        if T == 1 and self.conv_fold and select.fusion_enabled("conv_gemm",
                                                               self.fusions.get("conv_gemm")):
            # one token: the conv and silu on the qkv rows in the projections'
            # GEMV epilogue, the history moved on there too
            (t, names, ys), = self.groups
            self.tail_len = ops.ssm_proj_conv(t, [dev[n] for n in names], x, ys,
                                              [shapes[n][0] for n in names], cfg.hidden,
                                              dev["conv1d"], self.tail, self.tail_len, self.conv,
                                              stream=stream)
        else:
            for t, names, ys in self.groups:
                ops.norm_matmul(t, [dev[n] for n in names], x, ys,
                                [shapes[n][0] for n in names], cfg.hidden, T, norm=False,
                                stream=stream)
            self.tail_len = ops.ssm_conv(self.qkv, dev["conv1d"], self.tail, self.tail_len,
                                         self.tail, self.conv, T, cfg.qkv, cfg.conv_kernel,
                                         silu=True, stream=stream)
        nk_d = cfg.n_k * cfg.head_dim
        ops.ssm_scan(self.conv, self.conv, self.conv, self.alpha, self.beta, dev["a_log"],
                     dev["dt_bias"], self.state, self.o, T, cfg.n_k, cfg.n_v, cfg.head_dim,
                     self.scale, cfg.eps, strides=(cfg.qkv, cfg.qkv, cfg.qkv), q_off=0,
                     k_off=nk_d, v_off=2 * nk_d, stream=stream)
        if self.gpu("gated_norm") and select.fusion_enabled("norm_gemm",
                                                            self.fusions.get("norm_gemm")):
            # the gated norm in the output projection: its GEMV prologue at
            # decode, its x pre-pass on the split GEMM's path, else a gated
            # norm pass into the projection's workspace
            ops.gated_norm_matmul(cfg.wtypes[4], dev["out"], self.o, self.gate, dev["norm"],
                                  self.out, cfg.hidden, cfg.inner, T, cfg.norm_eps,
                                  stream=stream)
            return
        if self.gpu("gated_norm"):
            ops.gated_rmsnorm_silu(self.o, self.gate, dev["norm"], self.on, T, cfg.inner,
                                   cfg.norm_eps, stream=stream)
        else:
            if stream is not None:
                stream.synchronize()
            host = self.hooks["gated_norm"](self.o.view((T, cfg.inner)).numpy(),
                                            self.gate.view((T, cfg.inner)).numpy(),
                                            self.w.host["norm"], cfg.norm_eps)
            self.on.view((T, cfg.inner)).copy_from(np.ascontiguousarray(host, np.float32))
        ops.norm_matmul(cfg.wtypes[4], [dev["out"]], self.on.view((T, cfg.inner)),
                        [self.out], [cfg.hidden], cfg.inner, T, norm=False, stream=stream)
