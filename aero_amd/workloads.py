"""The five layer shapes of the elementwise path, as seeded synthetic inputs.

Each op's inputs come from a fresh numpy.random.default_rng(seed) (seed 0 by
default), drawn in the order written in each generator, so the GPU run, the
CPU baseline and the tests see identical bytes. Quant tables follow the GGML
block layouts with random quants and realistic fp16 scales (a random fp16
scale would be inf/NaN half the time).

Shapes:
  qwen2_0p5b_decode   1 token, hidden 896, 14/2 heads x 64, FFN 4864,
                      NeoX theta 1e6 at position 37, Q8_0 table 151936 x 896
  llama3_8b_prefill   512 tokens, hidden 4096, 32/8 heads x 128, FFN 14336,
                      eps 1e-5, NeoX theta 5e5, Q4_K table 128256 x 4096
  gemma3_4b_prefill   2048 tokens, hidden 2560, 8/4 heads x 256, FFN 10240,
                      (1+w) norms, QK-norm fused with RoPE theta 1e6, GeGLU
                      tanh, Q6_K table 262144 x 2560 scaled by sqrt(2560)
  qwen3next_hybrid    4096 tokens, hidden 2048: gated norm over 32 x 128,
                      16/2 heads x 256 with partial NeoX RoPE on 64 dims
                      (theta 1e7), SwiGLU FFN 5120, Q8_0 table 151936 x 2048
  llama3_70b_decode64 64 tokens at positions U[0, 32767], hidden 8192,
                      64/8 heads x 128, FFN 28672, RoPE from a dense 32768-row
                      table, Q4_K table 128256 x 8192
  llama3_70b_prefill16k  the same shapes over 16384 tokens at 0..16383
"""
from __future__ import annotations

import math
from dataclasses import dataclass, field, replace

import numpy as np

F32, F16, Q8_0, Q4_K, Q5_K, Q6_K, IQ4_XS, BF16 = 0, 1, 8, 12, 13, 14, 23, 30
BLOCK = {Q8_0: (32, 34), Q4_K: (256, 144), Q5_K: (256, 176), Q6_K: (256, 210),
         IQ4_XS: (256, 136)}


@dataclass(frozen=True)
class Shape:
    name: str
    n_tok: int
    hidden: int
    hq: int
    hk: int
    head_dim: int
    ffn: int
    eps: float
    theta: float
    n_rot: int
    positions: str          # "const:37", "range", "uniform:32768"
    act: str                # "silu" | "gelu_tanh"
    emb_type: int
    vocab: int
    unit_offset: bool = False
    qk_norm: bool = False
    rope_table: int = 0     # rows of a dense pre-computed table, 0 = computed angle
    emb_scale: bool = False
    gated: tuple = ()       # (n_v, d) of the gated norm, when the shape has one
    rope_mode: int = 0      # 0 NeoX, 1 interleaved
    extra: dict = field(default_factory=dict)


SHAPES = {
    "qwen2_0p5b_decode": Shape("qwen2_0p5b_decode", 1, 896, 14, 2, 64, 4864, 1e-6, 1e6, 64,
                               "const:37", "silu", Q8_0, 151936),
    "llama3_8b_prefill": Shape("llama3_8b_prefill", 512, 4096, 32, 8, 128, 14336, 1e-5, 5e5,
                               128, "range", "silu", Q4_K, 128256),
    "gemma3_4b_prefill": Shape("gemma3_4b_prefill", 2048, 2560, 8, 4, 256, 10240, 1e-6, 1e6,
                               256, "range", "gelu_tanh", Q6_K, 262144, unit_offset=True,
                               qk_norm=True, emb_scale=True),
    "qwen3next_hybrid": Shape("qwen3next_hybrid", 4096, 2048, 16, 2, 256, 5120, 1e-6, 1e7, 64,
                              "range", "silu", Q8_0, 151936, gated=(32, 128)),
    "llama3_70b_decode64": Shape("llama3_70b_decode64", 64, 8192, 64, 8, 128, 28672, 1e-5, 5e5,
                                 128, "uniform:32768", "silu", Q4_K, 128256, rope_table=32768),
    "llama3_70b_prefill16k": Shape("llama3_70b_prefill16k", 16384, 8192, 64, 8, 128, 28672,
                                   1e-5, 5e5, 128, "range", "silu", Q4_K, 128256,
                                   rope_table=32768),
}

# the shape the headline metric is quoted on
HEADLINE = "llama3_8b_prefill"


def _l8b(name, **kw):
    return replace(SHAPES[HEADLINE], name=name, **kw)


# Every op variant of the path at the Llama-3-8B 512-token geometry
# (R=512, N=4096, 32/8 heads x 128, FFN 14336): name -> (shape, op).
VARIANTS = {
    "rmsnorm": (SHAPES[HEADLINE], "rmsnorm"),
    "rmsnorm_unit_offset": (_l8b("rmsnorm_unit_offset", unit_offset=True), "rmsnorm"),
    "gated_norm_32x128": (_l8b("gated_norm_32x128", gated=(32, 128)), "gated_norm"),
    "rope_neox": (SHAPES[HEADLINE], "rope_qk"),
    "rope_interleaved": (_l8b("rope_interleaved", rope_mode=1), "rope_qk"),
    "rope_partial64_in_place": (_l8b("rope_partial64_in_place", n_rot=64), "rope_qk"),
    "rope_table": (_l8b("rope_table", rope_table=512), "rope_qk"),
    "qk_norm_rope": (_l8b("qk_norm_rope", qk_norm=True), "rope_qk"),
    "swiglu": (SHAPES[HEADLINE], "swiglu"),
    "geglu_erf": (_l8b("geglu_erf", act="gelu"), "swiglu"),
    "geglu_tanh": (_l8b("geglu_tanh", act="gelu_tanh"), "swiglu"),
    "gather_q4_k": (SHAPES[HEADLINE], "embed_gather"),
    "gather_q8_0": (_l8b("gather_q8_0", emb_type=Q8_0), "embed_gather"),
    "gather_q6_k_scaled": (_l8b("gather_q6_k_scaled", emb_type=Q6_K, emb_scale=True),
                           "embed_gather"),
}


def positions(s: Shape, rng) -> np.ndarray:
    if s.positions.startswith("const:"):
        return np.full(s.n_tok, int(s.positions[6:]), dtype=np.int32)
    if s.positions == "range":
        return np.arange(s.n_tok, dtype=np.int32)
    if s.positions.startswith("uniform:"):
        return rng.integers(0, int(s.positions[8:]), size=s.n_tok).astype(np.int32)
    raise ValueError(s.positions)


# ----------------------------------------------------------------- fp32 ops
def rmsnorm_inputs(s: Shape, seed: int = 0, rows: int | None = None):
    """x [R, hidden] ~ N(0,1); w ~ N(1, 0.1), or N(0, 0.1) applied as (1+w)."""
    rng = np.random.default_rng(seed)
    R = s.n_tok if rows is None else rows
    x = rng.standard_normal((R, s.hidden), dtype=np.float32)
    if s.unit_offset:
        w = (rng.standard_normal(s.hidden, dtype=np.float32) * np.float32(0.1))
    else:
        w = (np.float32(1) + rng.standard_normal(s.hidden, dtype=np.float32) * np.float32(0.1))
    return {"x": x, "w": w.astype(np.float32), "eps": s.eps, "unit_offset": s.unit_offset}


def rope_inputs(s: Shape, seed: int = 0, rows: int | None = None):
    """q [R, hq, D], k [R, hk, D] ~ N(0,1); positions; QK-norm weights when the
    shape has them (same recipe as the row norm)."""
    rng = np.random.default_rng(seed)
    R = s.n_tok if rows is None else rows
    q = rng.standard_normal((R, s.hq, s.head_dim), dtype=np.float32)
    k = rng.standard_normal((R, s.hk, s.head_dim), dtype=np.float32)
    pos = positions(s, rng)[:R]
    out = {"q": q, "k": k, "pos": pos, "n_rot": s.n_rot, "theta": s.theta, "eps": s.eps,
           "unit_offset": s.unit_offset, "table_rows": s.rope_table}
    if s.qk_norm:
        base = np.float32(0) if s.unit_offset else np.float32(1)
        out["q_w"] = (base + rng.standard_normal(s.head_dim, dtype=np.float32) * np.float32(0.1))
        out["k_w"] = (base + rng.standard_normal(s.head_dim, dtype=np.float32) * np.float32(0.1))
    return out


def act_inputs(s: Shape, seed: int = 0, rows: int | None = None):
    """gate, up [R, ffn] ~ N(0,1)."""
    rng = np.random.default_rng(seed)
    R = s.n_tok if rows is None else rows
    g = rng.standard_normal((R, s.ffn), dtype=np.float32)
    u = rng.standard_normal((R, s.ffn), dtype=np.float32)
    return {"gate": g, "up": u, "act": s.act}


def gated_inputs(s: Shape, seed: int = 0, rows: int | None = None):
    """x, z [R, n_v*d] ~ N(0,1); w [d] ~ N(1, 0.1)."""
    rng = np.random.default_rng(seed)
    R = s.n_tok if rows is None else rows
    n_v, d = s.gated
    x = rng.standard_normal((R, n_v * d), dtype=np.float32)
    z = rng.standard_normal((R, n_v * d), dtype=np.float32)
    w = np.float32(1) + rng.standard_normal(d, dtype=np.float32) * np.float32(0.1)
    return {"x": x, "z": z, "w": w.astype(np.float32), "eps": s.eps}


# ------------------------------------------------------------ quant tables
def _f16_bytes(v: np.ndarray) -> np.ndarray:
    return np.ascontiguousarray(v.astype(np.float16)).view(np.uint8).reshape(-1, 2)


# Root mean square of a dequantised value per unit of the random block scale
# (d, and dmin alike) make_table draws, from the distributions below: Q8_0
# rms(q) over U{-127..127}; the K-quants rms(sc*q) with 6-bit sc and 4-, 5-
# or 6-bit q (the min term is an order of magnitude smaller); IQ4_XS the
# codebook times its 6-bit signed scales. Used to draw weights of a chosen
# scale (weight_table).
_RMS_PER_D = {Q8_0: 73.3 * 0.02 / 127, Q4_K: 323.0 * 0.01, Q5_K: 659.0 * 0.01,
              Q6_K: 1365.0 * 0.01, IQ4_XS: 1080.0 * 0.001}


def weight_table(t: int, n_rows: int, n_cols: int, rng) -> np.ndarray:
    """A synthetic weight matrix of type t whose values have an rms of about
    1/sqrt(n_cols), as trained projections do, so that activations stay of
    unit scale through a block (attention scores of order one)."""
    return make_table(t, n_rows * n_cols // BLOCK[t][0], rng,
                      d_scale=1.0 / (_RMS_PER_D[t] * math.sqrt(n_cols)))


def make_table(t: int, n_blocks: int, rng, d_scale: float = 1.0) -> np.ndarray:
    """n_blocks GGML blocks of type t as a flat uint8 array (block scales
    drawn as below, times d_scale)."""
    bv, bb = BLOCK[t]
    ds = np.float32(d_scale)
    if t == Q8_0:
        # int8 quants U{-127..127}; d = fp16(|N(0, 0.02)| / 127)
        blk = np.empty((n_blocks, bb), dtype=np.uint8)
        q = rng.integers(-127, 128, size=(n_blocks, 32), dtype=np.int8)
        d = np.abs(rng.standard_normal(n_blocks, dtype=np.float32) * np.float32(0.02)) / np.float32(127) * ds
        blk[:, 0:2] = _f16_bytes(d)
        blk[:, 2:] = q.view(np.uint8)
        return blk.reshape(-1)
    if t == Q4_K:
        # every byte random, then d, dmin = fp16(|N(0, 0.01)|)
        blk = rng.integers(0, 256, size=(n_blocks, bb), dtype=np.uint8)
        dd = np.abs(rng.standard_normal((n_blocks, 2), dtype=np.float32) * np.float32(0.01)) * ds
        blk[:, 0:4] = np.ascontiguousarray(dd.astype(np.float16)).view(np.uint8).reshape(-1, 4)
        return blk.reshape(-1)
    if t == Q6_K:
        # ql/qh random bytes, int8 scales U{-128..127}, d = fp16(|N(0, 0.01)|)
        blk = rng.integers(0, 256, size=(n_blocks, bb), dtype=np.uint8)
        d = np.abs(rng.standard_normal(n_blocks, dtype=np.float32) * np.float32(0.01)) * ds
        blk[:, 208:210] = _f16_bytes(d)
        return blk.reshape(-1)
    if t == Q5_K:
        # as Q4_K: random bytes (scales, qh, qs), d, dmin = fp16(|N(0, 0.01)|)
        blk = rng.integers(0, 256, size=(n_blocks, bb), dtype=np.uint8)
        dd = np.abs(rng.standard_normal((n_blocks, 2), dtype=np.float32) * np.float32(0.01)) * ds
        blk[:, 0:4] = np.ascontiguousarray(dd.astype(np.float16)).view(np.uint8).reshape(-1, 4)
        return blk.reshape(-1)
    if t == IQ4_XS:
        # random scale and quant bytes, d = fp16(|N(0, 0.001)|) (x codebook up to 127)
        blk = rng.integers(0, 256, size=(n_blocks, bb), dtype=np.uint8)
        d = np.abs(rng.standard_normal(n_blocks, dtype=np.float32) * np.float32(0.001)) * ds
        blk[:, 0:2] = _f16_bytes(d)
        return blk.reshape(-1)
    raise ValueError(t)


def embed_inputs(s: Shape, seed: int = 0, vocab: int | None = None, rows: int | None = None):
    """The quantised table (vocab rows), then ids ~ U[0, vocab)."""
    rng = np.random.default_rng(seed)
    V = s.vocab if vocab is None else vocab
    R = s.n_tok if rows is None else rows
    bv, bb = BLOCK[s.emb_type]
    nbr = s.hidden // bv
    table = make_table(s.emb_type, V * nbr, rng)
    ids = rng.integers(0, V, size=R).astype(np.int32)
    scale = float(np.float32(math.sqrt(s.hidden))) if s.emb_scale else 0.0
    return {"type": s.emb_type, "table": table, "vocab": V, "n_embd": s.hidden, "ids": ids,
            "scale": scale, "row_bytes": nbr * bb}


# ------------------------------------------------- algorithmic HBM bytes
def bytes_rmsnorm(R: int, N: int) -> int:
    return 4 * (2 * R * N + N)


def bytes_gated(R: int, inner: int, d: int) -> int:
    return 4 * (3 * R * inner + d)


def bytes_rope(R: int, heads: int, D: int, n_rot: int, norm: bool, in_place: bool,
               table: bool) -> int:
    """Read + write of every touched channel (all D with a norm or a copy, the
    rotated n_rot otherwise), the norm weights once, table rows when used."""
    ch = D if (norm or not in_place) else n_rot
    b = 8 * R * heads * ch
    if norm:
        b += 4 * D
    if table:
        b += 4 * R * n_rot
    return b


def bytes_act(R: int, F: int) -> int:
    return 12 * R * F


def bytes_embed(R: int, N: int, t: int) -> int:
    bv, bb = BLOCK[t]
    return R * (N // bv) * bb + 4 * R * N + 4 * R


def bytes_embed_rmsnorm(R: int, N: int, t: int) -> int:
    """Fused gather + first RMSNorm: table rows and ids read, x and h written,
    the norm weight once."""
    return bytes_embed(R, N, t) + 4 * R * N + 4 * N


def bytes_add_rmsnorm(R: int, N: int) -> int:
    """Residual add + RMSNorm: x and d read, x + d and h written, the weight once."""
    return 16 * R * N + 4 * N


def bytes_post_norm_add(R: int, N: int) -> int:
    """Gemma's sandwich-norm site: y and x read, x' and h written, both weights once."""
    return 16 * R * N + 8 * N
