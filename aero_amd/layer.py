"""Device-resident decoder blocks: the model-loop counterpart of the fused ops.

Qwen-style blocks of the reference (src/model.cpp:234-287, with the
attention hook of src/attention_layer.cpp:60-240 and the FFN of
src/model.cpp:166-178), one or a stack, over quantised weights resident in
HBM, every activation kept on the device. Per block:

    x = embed(ids) (* scale)                      src/model.cpp:297-316
    h = rmsnorm(x, attn_norm)                     :244-245
    q, k, v = h Wq, h Wk, h Wv                    attention_layer.cpp
    q, k = qk_norm(q, k); rope(q, k)              :89-156
    k, v -> KV cache rows kv_len .. kv_len+T-1    :158-200
    a = attention(q, K, V), causal                :202-225
    x += a Wo                                     src/model.cpp:279
    h = rmsnorm(x, ffn_norm)                      :280-282
    x += (act(h Wg) * (h Wu)) Wd                  :166-178, 284
    h_out = rmsnorm(x, out_norm)                  :329

In a stack the FFN output of a block is added to x by the next block's
attention norm (and after the last block by the output norm), so that add
folds into the next projections like the o-projection's does.

Each elementwise site asks aero_amd.select whether its op runs on the GPU
(AERO_GPU_OPS; unset means every op, for this device-resident loop) and which
fusions apply (AERO_GPU_FUSE; unset means all): the gather with the first
norm (embed_norm), norms and residual adds folded into the projections that
consume them (norm_gemm), the act-mul folded into the gate/up projection
(act_gemm), the per-head norms and RoPE in the epilogue of the q/k
projection (rope_gemm), the embedding rows read by the first q/k/v
projection's pre-pass (embed_gemm). At 512 Llama-3-8B tokens a block is then
10 launches: pre-pass + q/k/v GEMM (with the gather, norm, RoPE), attention,
and a pre-pass + GEMM each for o, gate/up (+ act) and down, and the output
norm. An op off the GPU runs the caller's host hook for it, as the
reference's model loop keeps its own code for the ops it does not hand to a
library; with no hook the block raises select.HostPathRequired, since the
library has no CPU path. With every op on the GPU, `forward` can be recorded
as a Plan and replayed with one call a step.
"""
from __future__ import annotations

import math
from dataclasses import dataclass

import numpy as np

from . import ops, select
from . import workloads as W
from .device import DeviceArray as DA, Stream

@dataclass(frozen=True)
class BlockConfig:
    hidden: int
    n_head: int
    n_head_kv: int
    head_dim: int
    ffn: int
    eps: float
    theta: float
    n_rot: int
    act: str            # "silu" | "gelu" | "gelu_tanh"
    wtype: int          # projection weights' ggml type
    emb_type: int
    vocab: int
    qk_norm: bool = False
    unit_offset: bool = False
    emb_scale: bool = False
    # Gemma blocks (src/model.cpp:181-232): a post-norm on the attention and
    # on the FFN output before each residual add, and the layer output scale
    # applied to the deltas (out_scale_mode 1) or to the whole sum (2)
    post_norms: bool = False
    out_scale_mode: int = 0
    # the attention layer's options (src/attention_layer.cpp:60-156,262-263):
    # q rows interleaved per head with a gate [q_h | gate_h] and a sigmoid
    # output gate; a weightless per-head V norm; V := K (no V projection);
    # RoPE frequency factors
    attn_gate: bool = False
    v_norm: bool = False
    v_from_k: bool = False
    freq_factors: tuple | None = None

    @classmethod
    def from_shape(cls, s: W.Shape, wtype: int, vocab: int | None = None,
                   **options) -> "BlockConfig":
        return cls(s.hidden, s.hq, s.hk, s.head_dim, s.ffn, s.eps, s.theta, s.n_rot, s.act,
                   wtype, s.emb_type, s.vocab if vocab is None else vocab, s.qk_norm,
                   s.unit_offset, s.emb_scale, **options)


class BlockWeights:
    """Synthetic weights of one block (seeded): quantised projections of
    trained-like scale (values of rms ~1/sqrt(columns)), the embedding table,
    fp32 norm weights; kept on the host (`host`) and in HBM."""

    def __init__(self, cfg: BlockConfig, seed: int = 0):
        rng = np.random.default_rng(seed)
        N, D, F = cfg.hidden, cfg.head_dim, cfg.ffn
        HD, KD = cfg.n_head * D, cfg.n_head_kv * D
        bv, bb = W.BLOCK[cfg.wtype]
        # with the output gate, wq holds 2*HD rows, [q_h | gate_h] per head,
        # as the reference's file stores it
        shapes = {"wq": (2 * HD if cfg.attn_gate else HD, N), "wk": (KD, N), "wv": (KD, N),
                  "wo": (N, HD), "wg": (F, N), "wu": (F, N), "wd": (N, F)}
        self.MATS = tuple(m for m in ("wq", "wk", "wv", "wo", "wg", "wu", "wd")
                          if not (m == "wv" and cfg.v_from_k))
        h = {}
        for name in self.MATS:
            r, c = shapes[name]
            if c % bv:
                raise ValueError(f"{name}: {c} columns are not whole {bv}-value blocks")
            h[name] = W.weight_table(cfg.wtype, r, c, rng)
        self.shapes = shapes
        h["emb"] = W.make_table(cfg.emb_type, cfg.vocab * (N // W.BLOCK[cfg.emb_type][0]), rng)

        def norm_w(n):
            w = rng.standard_normal(n, dtype=np.float32) * np.float32(0.1)
            return w if cfg.unit_offset else (np.float32(1) + w).astype(np.float32)

        for name in ("attn_norm", "ffn_norm", "out_norm") + (
                ("post_attn_norm", "post_ffw_norm") if cfg.post_norms else ()):
            h[name] = norm_w(N)
        if cfg.qk_norm:
            h["q_norm"], h["k_norm"] = norm_w(D), norm_w(D)
        # the layer output scale (a per-layer scalar of the file)
        self.out_scale = float(np.float32(rng.uniform(0.5, 1.5))) if cfg.out_scale_mode else 1.0
        self.host = h
        dev = {k: DA.from_numpy(v) for k, v in h.items() if k != "wq" or not cfg.attn_gate}
        if cfg.attn_gate:
            # the q and the gate rows of each head, regrouped once at upload
            # into two matrices (row bytes are whole blocks, so this moves
            # bytes only), so the projection writes q and the gate to their
            # own buffers and no split pass runs per step
            rb = (N // bv) * bb
            rows = h["wq"].reshape(cfg.n_head, 2, D, rb)
            dev["wq"] = DA.from_numpy(np.ascontiguousarray(rows[:, 0]).reshape(-1))
            dev["wq_gate"] = DA.from_numpy(np.ascontiguousarray(rows[:, 1]).reshape(-1))
        self.dev = dev


class LayerStep:
    """Embedding, one block or a stack of them (`weights` a BlockWeights or a
    list, one a layer, each with its own KV cache) and the output norm, over
    device buffers sized for `max_tokens` tokens a step and KV caches of
    `kv_cap` positions (fp32).

        step = LayerStep(cfg, BlockWeights(cfg), max_tokens=512, kv_cap=4096)
        step.prepare(ids, kv_len)          # token ids and positions to HBM
        step.forward(len(ids), kv_len)     # or record it: with plan: ...
        x, h_out = step.x, step.h_out      # [T, hidden] each, in HBM
    """

    def __init__(self, cfg: BlockConfig, weights, max_tokens: int,
                 kv_cap: int, gpu_ops: dict | None = None, fusions: dict | None = None,
                 hooks: dict | None = None):
        self.layers = list(weights) if isinstance(weights, (list, tuple)) else [weights]
        if not self.layers:
            raise ValueError("LayerStep needs the weights of at least one block")
        self.cfg = cfg
        self.w = self.layers[0]
        self.gpu_ops, self.fusions, self.hooks = gpu_ops or {}, fusions or {}, hooks or {}
        N, D, F = cfg.hidden, cfg.head_dim, cfg.ffn
        T = max_tokens
        self.max_tokens, self.kv_cap = T, kv_cap
        HD, KD = cfg.n_head * D, cfg.n_head_kv * D
        self.x, self.h, self.h_out = DA.empty((T, N)), DA.empty((T, N)), DA.empty((T, N))
        # x and a second residual buffer: below 32 tokens a projection that
        # folds the residual add stores x + d into the other one (its
        # workgroups still read x); the output norm leaves x in self.x
        self.xs = (self.x, DA.empty((T, N)))
        self._cur = 0
        self.q, self.att = DA.empty((T, HD)), DA.empty((T, HD))
        self.qgate = DA.empty((T, HD)) if cfg.attn_gate else None
        # the pending post-norm of a Gemma block's FFN output, applied by the
        # next norm site: (post_ffw_norm weight, ds, ss)
        self._post = None
        self.o = DA.empty((T, N))
        self.dn = DA.empty((T, N))
        self.g, self.u = DA.empty((T, F)), DA.empty((T, F))
        self.ids, self.pos = DA.empty((T,), np.int32), DA.empty((T,), np.int32)
        # one KV cache a layer; K, V are the first layer's
        self.kv = [(DA.empty((kv_cap, KD)), DA.empty((kv_cap, KD))) for _ in self.layers]
        self.K, self.V = self.kv[0]
        n_rot, inv = ops.rope_inv_freq(D, cfg.n_rot, cfg.theta,
                                       None if cfg.freq_factors is None
                                       else np.asarray(cfg.freq_factors, np.float32))
        self.n_rot, self.inv = n_rot, DA.from_numpy(inv)
        self.scale = float(np.float32(math.sqrt(N))) if cfg.emb_scale else 0.0
        rb = (N // W.BLOCK[cfg.wtype][0]) * W.BLOCK[cfg.wtype][1]
        # rows fit the fused decode GEMVs: whole 16 bytes, or Q8_0 rows of
        # whole 8 bytes in matrices (allocated to size) ending on a 16-byte
        # boundary
        rows_n = (cfg.n_head * D, cfg.n_head_kv * D, F)
        self.rows16 = rb % 16 == 0 or (cfg.wtype == W.Q8_0 and rb % 8 == 0 and
                                       all(n * rb % 16 == 0 for n in rows_n))

    # ------------------------------------------------------------ selection
    def gpu(self, op: str) -> bool:
        if select.enabled(op, self.gpu_ops.get(op), default=True):
            return True
        if op in self.hooks:
            return False
        raise select.HostPathRequired(
            f"op {op!r} is off the GPU ({select.ENV}) and no host hook was given for it")

    def fuse(self, name: str) -> bool:
        return select.fusion_enabled(name, self.fusions.get(name))

    def uses_host(self) -> bool:
        """True when some op runs a host hook (the step then cannot be recorded)."""
        return any(not self.gpu(op) for op in ("embed", "rmsnorm", "rope", "act") +
                   (("qk_norm",) if self.cfg.qk_norm else ()))

    # ------------------------------------------------------------ host side
    def prepare(self, ids, kv_len: int, positions=None) -> None:
        """Token ids and their positions (default kv_len ..) to HBM."""
        ids = np.ascontiguousarray(ids, np.int32).reshape(-1)
        T = ids.size
        if not 0 < T <= self.max_tokens or kv_len < 0 or kv_len + T > self.kv_cap:
            raise ValueError(f"{T} tokens at kv_len {kv_len}: outside max_tokens "
                             f"{self.max_tokens} / kv_cap {self.kv_cap}")
        pos = (np.arange(kv_len, kv_len + T, dtype=np.int32) if positions is None
               else np.ascontiguousarray(positions, np.int32).reshape(-1))
        self.ids.view((T,)).copy_from(ids)
        self.pos.view((T,)).copy_from(pos)

    def _host(self, a: DA, shape):
        return a.view(shape).numpy()

    def _put(self, a: DA, v) -> None:
        a.view(np.shape(v)).copy_from(np.ascontiguousarray(v, np.float32))

    # ------------------------------------------------------------ the blocks
    def forward(self, T: int, kv_len: int, stream: Stream | None = None) -> None:
        """Embedding, every block, the output norm. A block's FFN output is not
        added to x at its end: the next block's first norm takes it as the
        residual input (folded into its q/k/v pre-pass where it can be), and
        after the last block the output norm does (src/model.cpp:284,
        244-245, 329)."""
        c = self.cfg
        N = c.hidden
        if not 0 < T <= self.max_tokens or kv_len + T > self.kv_cap:
            raise ValueError("forward: tokens or KV span outside the buffers")
        s = stream
        x, h = self.x.view((T, N)), self.h.view((T, N))
        self._cur = 0
        self._post = None
        w0 = self.layers[0]

        # embedding (+ the first block's attention norm when its projections
        # need h); or read by the first q/k/v projection's pre-pass
        h_ready = False
        emb_fold = self._folds_emb(T)
        if emb_fold:
            pass
        elif self.gpu("embed"):
            if not self._folds_norm(T) and self.fuse("embed_norm") and self.gpu("rmsnorm"):
                ops.embed_rmsnorm(c.emb_type, w0.dev["emb"], c.vocab, N, self.ids, x, h,
                                  w0.dev["attn_norm"], c.eps, scale=self.scale,
                                  unit_offset=c.unit_offset, n_ids=T, stream=s)
                h_ready = True
            else:
                ops.embed_gather(c.emb_type, w0.dev["emb"], c.vocab, N, self.ids, x,
                                 scale=self.scale, n_ids=T, stream=s)
        else:
            self._put(x, self.hooks["embed"](self._host(self.ids, (T,))))

        resid = None
        for li, w in enumerate(self.layers):
            resid = self._block(w, li, T, kv_len, resid, h_ready, s, emb=emb_fold and li == 0)
            h_ready = False
        self._norm(self.layers[-1], self._x(T), resid, "out_norm", self.h_out.view((T, N)), T,
                   s, x_out=x)

    def _block(self, w: BlockWeights, li: int, T: int, kv_len: int, resid, h_ready: bool,
               s, emb: bool = False) -> DA:
        """One block on x (+ resid, the previous block's FFN output; emb: x is
        the embedding rows, read by the q/k/v projection's pre-pass). Returns
        this block's FFN output, to be added by the next norm."""
        c, d = self.cfg, w.dev
        N, H, HK, D, F = c.hidden, c.n_head, c.n_head_kv, c.head_dim, c.ffn
        Kc, Vc = self.kv[li]
        kv0 = kv_len * HK * D * 4
        kq = Kc.view((T, HK * D), offset_bytes=kv0)
        vq = Vc.view((T, HK * D), offset_bytes=kv0)
        q = self.q.view((T, H * D))

        # x += resid (or x = the embedding rows); q, k, v (k and v straight
        # into the cache rows of these positions), with the per-head norms and
        # RoPE on q and k in the projection's epilogue where that folds
        # V := K projects K's matrix again into the V cache rows (the raw
        # projection, before the k norm and RoPE, as src/attention_layer.cpp:
        # 67-69 copies it); with the output gate a fourth matrix writes the
        # gate rows
        mats = [d["wq"], d["wk"], d["wk"] if c.v_from_k else d["wv"]]
        ys, rows = [q, kq, vq], [H * D, HK * D, HK * D]
        if c.attn_gate:
            mats.append(d["wq_gate"])
            ys.append(self.qgate.view((T, H * D)))
            rows.append(H * D)
        rope = None
        if not h_ready and self._folds_norm(T):
            rope = self._rope_args(w)
            xi, xo = self._advance(T, resid)
            first = self.layers[0].dev
            ops.attn_input(c.wtype, mats, ys, rows, N, T, x_out=xo, x=None if emb else xi,
                           d=resid,
                           emb={"type": c.emb_type, "table": first["emb"], "vocab": c.vocab,
                                "ids": self.ids, "scale": self.scale} if emb else None,
                           norm_w=d["attn_norm"], eps=c.eps, unit_offset=c.unit_offset,
                           rope=rope, stream=s)
        else:
            self._project(w, resid, "attn_norm", mats, ys, rows, T, h_ready, s)

        # the weightless per-head V norm (src/attention_layer.cpp:109-114; not
        # on a V taken from K), in the cache rows
        if c.v_norm and not c.v_from_k:
            if self.gpu("rmsnorm"):
                ops.rmsnorm(vq, None, vq, T * HK, D, c.eps, stream=s)
            else:
                _, vn = self.hooks["rmsnorm"](self._host(vq, (T * HK, D)), None,
                                              np.ones(D, np.float32), c.eps, False)
                self._put(vq, vn)

        # per-head norms and RoPE, in place (the cache rows of k included),
        # unless the projection's epilogue rotated q and k
        if rope is None:
            if self.gpu("rope") and (not c.qk_norm or self.gpu("qk_norm")):
                ops.qk_norm_rope(q, H, T, D, self.n_rot, k=kq, n_k_heads=HK,
                                 q_norm_w=d.get("q_norm"), k_norm_w=d.get("k_norm"), eps=c.eps,
                                 unit_offset=c.unit_offset, pos=self.pos, inv_freq=self.inv,
                                 stream=s)
            else:
                qh, kh = self.hooks["rope"](self._host(q, (T, H, D)),
                                            self._host(kq, (T, HK, D)), self._host(self.pos, (T,)))
                self._put(q, qh)
                self._put(kq, kh)

        # causal attention over the cache, then the output projection
        att = self.att.view((T, H * D))
        ops.attention(q, Kc, Vc, att, T, H, HK, D, D, kv_len + T, 1.0 / math.sqrt(D),
                      qpos=self.pos, stream=s)
        if c.attn_gate:
            # att *= sigmoid(gate) (src/attention_layer.cpp:262-263)
            ops.act_mul("sigmoid", self.qgate.view((T, H * D)), att, att, stream=s)
        o = self.o.view((T, N))
        ops.matvec(c.wtype, d["wo"], att, o, N, H * D, T, stream=s)

        # x += o; h = rmsnorm(x); g = act(h Wg) * (h Wu). Gemma: x += ds *
        # post_attn_norm(o) before that norm (src/model.cpp:213-219)
        g = self.g.view((T, F))
        if c.post_norms:
            h = self.h.view((T, N))
            ds = w.out_scale if c.out_scale_mode == 1 else 1.0
            self._norm(w, self._x(T), o, "ffn_norm", h, T, s,
                       post=(d["post_attn_norm"], ds, 1.0))
            self._gate_up(w, h, g, T, s)
        elif self._folds_norm(T) and self.fuse("act_gemm") and self.gpu("act"):
            xi, xo = self._advance(T, o)
            ops.norm_matmul_gate_up(c.wtype, d["wg"], d["wu"], xi, g, F, N, T, act=c.act,
                                    norm_w=d["ffn_norm"], eps=c.eps, unit_offset=c.unit_offset,
                                    d=o, x_out=xo, stream=s)
        else:
            h = self.h.view((T, N))
            self._norm(w, self._x(T), o, "ffn_norm", h, T, s)
            if self.gpu("act") and self.fuse("act_gemm") and T < 32 and self.rows16:
                ops.norm_gate_up(c.wtype, d["wg"], d["wu"], h, g, F, N, T, act=c.act,
                                 norm=False, stream=s)
            else:
                u = self.u.view((T, F))
                ops.matvec(c.wtype, d["wg"], h, g, F, N, T, stream=s)
                ops.matvec(c.wtype, d["wu"], h, u, F, N, T, stream=s)
                if self.gpu("act"):
                    ops.act_mul(c.act, g, u, g, stream=s)
                else:
                    self._put(g, self.hooks["act"](self._host(g, (T, F)), self._host(u, (T, F))))

        # the down projection (the next norm adds it to x; this block's own
        # residual input in dn was consumed by its first norm)
        dn = self.dn.view((T, N))
        ops.matvec(c.wtype, d["wd"], g, dn, N, F, T, stream=s)
        if c.post_norms:
            # the next norm site adds (x + ds * post_ffw_norm(dn)) * ss
            # (src/model.cpp:228-231)
            self._post = (d["post_ffw_norm"],
                          w.out_scale if c.out_scale_mode == 1 else 1.0,
                          w.out_scale if c.out_scale_mode == 2 else 1.0)
        return dn

    def _gate_up(self, w: BlockWeights, h, g, T: int, s) -> None:
        """g = act(h Wg) * (h Wu) for a normalised h: one launch (the split
        GEMM's act epilogue, or the fused decode GEMV) when act-mul folds."""
        c, d = self.cfg, w.dev
        F, N = c.ffn, c.hidden
        if self.gpu("act") and self.fuse("act_gemm"):
            ops.norm_matmul_gate_up(c.wtype, d["wg"], d["wu"], h, g, F, N, T, act=c.act,
                                    norm=False, stream=s)
            return
        u = self.u.view((T, F))
        ops.matvec(c.wtype, d["wg"], h, g, F, N, T, stream=s)
        ops.matvec(c.wtype, d["wu"], h, u, F, N, T, stream=s)
        if self.gpu("act"):
            ops.act_mul(c.act, g, u, g, stream=s)
        else:
            self._put(g, self.hooks["act"](self._host(g, (T, F)), self._host(u, (T, F))))

    def _folds_norm(self, T: int) -> bool:
        """True when the norm (and residual add) before a projection folds into
        it: the split GEMM's pre-pass at 32+ tokens, when the library's own
        rule (ops.split_ok) gives the split path to this type and shape (the
        call itself takes it from 5-16 tokens where it is faster), the fused
        decode GEMV's prologue below that."""
        c = self.cfg
        if not (self.fuse("norm_gemm") and self.gpu("rmsnorm")) or c.post_norms:
            # Gemma's sites take a second norm of the sublayer output first:
            # their own kernel (post_norm_add), then the projection on h
            return False
        if T >= 32:
            return ops.split_ok(c.wtype, c.hidden,
                                ((2 if c.attn_gate else 1) * c.n_head + 2 * c.n_head_kv)
                                * c.head_dim, T)
        return self.rows16

    def _rope_args(self, w: BlockWeights) -> dict | None:
        """The per-head norms and RoPE of q and k for the folded q/k/v
        projection (ops.attn_input), or None when they run apart: their ops
        on the GPU and the rope_gemm fusion on. The library folds them into
        the projection's epilogue where the path taken allows (the split
        GEMM: heads of up to 128 rows; the fused decode GEMV: every channel
        rotated, no per-head norm) and runs the per-head pass otherwise."""
        c, d = self.cfg, w.dev
        if not (self.fuse("rope_gemm") and self.gpu("rope") and
                (not c.qk_norm or self.gpu("qk_norm"))):
            return None
        return {"n": 2, "head_dim": c.head_dim, "n_rot": self.n_rot, "mode": ops.ROPE_NEOX,
                "pos": self.pos, "inv_freq": self.inv, "q_norm_w": d.get("q_norm"),
                "k_norm_w": d.get("k_norm"), "eps": c.eps, "unit_offset": c.unit_offset}

    def _folds_emb(self, T: int) -> bool:
        """True when the first block's q/k/v pre-pass reads the embedding
        rows itself (the split GEMM at 32+ tokens, a table type its pre-pass
        dequantises), so no embedding launch runs."""
        c = self.cfg
        return (T >= 32 and self.gpu("embed") and self.fuse("embed_gemm") and
                self._folds_norm(T) and c.emb_type in (W.Q8_0, W.Q4_K, W.Q5_K, W.Q6_K, W.IQ4_XS))

    def _x(self, T: int) -> DA:
        """The residual stream x as it stands (one of the two x buffers)."""
        return self.xs[self._cur].view((T, self.cfg.hidden))

    def _advance(self, T: int, resid):
        """(x, x_out) for a projection folding x += resid: in place at 32+
        tokens (the split GEMM's pre-pass owns each token's row), else into
        the other x buffer, which then holds x."""
        xi = self._x(T)
        if resid is None or T >= 32:
            return xi, xi
        self._cur ^= 1
        return xi, self._x(T)

    def _norm(self, wts: BlockWeights, x, resid, wname, h, T, s, x_out=None,
              post=None) -> None:
        """x_out = x + resid (resid given; x_out None: x in place); h =
        rmsnorm of that (or of x) * the norm weight `wname`. Gemma blocks:
        x_out = (x + ds * rmsnorm(resid) * w_post) * ss with (w_post, ds, ss)
        = `post`, or the pending post-norm of the previous block's FFN."""
        c = self.cfg
        w = wts.dev[wname]
        if resid is None and x_out is not None and x_out.ptr != x.ptr:
            raise ValueError("_norm: x_out without a residual input")
        if resid is not None and c.post_norms:
            post = post if post is not None else self._post
            if not self.gpu("rmsnorm"):
                raise select.HostPathRequired("the Gemma post-norm sites run on the GPU only")
            ops.post_norm_add(resid, x, post[0], w, h, T, c.hidden, c.eps, ds=post[1],
                              ss=post[2], unit_offset=c.unit_offset, x_out=x_out, stream=s)
            return
        if self.gpu("rmsnorm"):
            if resid is not None:
                ops.add_rmsnorm(x, resid, w, h, T, c.hidden, c.eps, c.unit_offset, x_out=x_out,
                                stream=s)
            else:
                ops.rmsnorm(x, w, h, T, c.hidden, c.eps, c.unit_offset, stream=s)
            return
        xn, hn = self.hooks["rmsnorm"](self._host(x, (T, c.hidden)),
                                       None if resid is None else self._host(resid, (T, c.hidden)),
                                       wts.host[wname], c.eps, c.unit_offset)
        self._put(x if x_out is None else x_out, xn)
        self._put(h, hn)

    def _project(self, wts: BlockWeights, resid, wname, mats, ys, rows, T, h_ready,
                 s) -> None:
        """ys[m] = rmsnorm(x (+ resid)) W_m^T with the norm as its own pass
        (or h already normed): the sites whose norm does not fold."""
        c = self.cfg
        h = self.h.view((T, c.hidden))
        if not h_ready:
            self._norm(wts, self._x(T), resid, wname, h, T, s)
        if self.fuse("norm_gemm") and T < 32 and self.rows16 and len(mats) <= 3:
            ops.norm_matvec(c.wtype, mats, h, ys, rows, c.hidden, T, norm=False, stream=s)
        elif self.fuse("norm_gemm"):
            # every matrix in one launch where the shape allows (split GEMM,
            # fused GEMV), with x as is
            ops.norm_matmul(c.wtype, mats, h, ys, rows, c.hidden, T, norm=False, stream=s)
        else:
            for m, y, r in zip(mats, ys, rows):
                ops.matvec(c.wtype, m, h, y, r, c.hidden, T, stream=s)
