"""GPU parity: the device-resident block (aero_amd.layer.LayerStep) against the
oracle's composition of the same block (src/model.cpp:234-287,297-316,329 with
the attention hook of src/attention_layer.cpp:89-225): the oracle's embedding
gather, rmsnorm_rows, qk_norm_rope, attention_tiled and act_mul, and float64
products over the oracle's dequantised weights for the projections (the
oracle's matmul equals that product to ~1e-6 of scale, tests/test_gpu_gemm16.py).

Checked at the Qwen2-0.5B decode shape (one token at position 37 over a
cache of 37 earlier positions; Q8_0 weights, whose 952-byte rows of 896
values take the fused decode GEMVs), the Llama-3-8B 512-token prefill (Q4_K
weights: the split GEMM with the norms folded), a Llama-3-8B one-token
decode over 1023 cached positions (the fused decode GEMVs with RoPE in the
epilogue, chunked attention), 16 Llama-3-8B tokens over 100 cached
positions (the split GEMMs below 32 tokens) and a Gemma-style 64-token
prefill (QK-norm, (1+w) norms, GeGLU tanh, scaled embedding), with every
fusion on and with every fusion off, and with host hooks standing in for
ops taken off the GPU.
Stacks of 2-3 blocks (each with its own weights and KV cache) are checked
at the same shapes against the oracle's blocks in turn.
Tolerance 1e-5 of each output's scale; x is the residual stream after the
last block, h_out its output norm.
"""
import math

import numpy as np
import pytest

from conftest import RTOL, rel_to_scale
from aero_amd import layer, select
from aero_amd import workloads as W

pytestmark = pytest.mark.gpu

ACT = {"silu": 0, "gelu": 1, "gelu_tanh": 2}

CASES = {
    # name: (shape, weight type, vocab, tokens, earlier cache positions)
    "qwen2_0p5b_decode": ("qwen2_0p5b_decode", W.Q8_0, 4096, 1, 37),
    "llama3_8b_prefill": ("llama3_8b_prefill", W.Q4_K, 4096, 512, 0),
    "gemma_like_prefill": ("gemma3_4b_prefill", W.Q4_K, 2048, 64, 0),
    # one token over 1023 cached positions at the Llama-3-8B geometry: the
    # fused decode GEMVs (16-byte Q4_K rows) and the chunked attention
    "llama3_8b_decode": ("llama3_8b_prefill", W.Q4_K, 4096, 1, 1023),
    # 16 tokens over 100 cached positions (a speculative-decoding step): the
    # projections take the split GEMM with the norms folded below 32 tokens
    "llama3_8b_t16": ("llama3_8b_prefill", W.Q4_K, 4096, 16, 100),
    # the 512-token prefill in the other split-GEMM types: the norms and
    # residual adds fold into the pre-pass for these too (Q6_K: rows of 4096
    # and 14336 columns are whole 2048-value groups)
    "llama3_8b_prefill_q8_0": ("llama3_8b_prefill", W.Q8_0, 4096, 512, 0),
    "llama3_8b_prefill_q6_k": ("llama3_8b_prefill", W.Q6_K, 4096, 512, 0),
}

# Blocks with the options of src/model.cpp:181-232 (Gemma's sandwich norms
# and layer output scale) and src/attention_layer.cpp:60-156,262-263 (the
# per-head output gate, the weightless V norm, V := K, RoPE frequency
# factors), at the config-3 (Gemma-3-4B-style) and config-4 (Qwen3-Next
# attention) layer geometries: (CASES entry, BlockConfig options)
OPTION_CASES = {
    "gemma_sandwich_prefill": (("gemma3_4b_prefill", W.Q4_K, 2048, 64, 0),
                               {"post_norms": True, "out_scale_mode": 1}),
    "gemma_sandwich_decode": (("gemma3_4b_prefill", W.Q4_K, 2048, 1, 40),
                              {"post_norms": True, "out_scale_mode": 2}),
    "gemma_v_from_k_prefill": (("gemma3_4b_prefill", W.Q8_0, 2048, 48, 16),
                               {"post_norms": True, "v_from_k": True}),
    # Q8_0 (zero-mean weights): with the Q4_K tables' non-zero row means the
    # stacked residual stream of this geometry grows to ~1e4 on some tokens
    # and near-cancelling rows make the output norm ill-conditioned
    "qwen3next_gated_attn_prefill": (("qwen3next_hybrid", W.Q8_0, 2048, 64, 0),
                                     {"attn_gate": True, "v_norm": True,
                                      "freq_factors": "random"}),
    "qwen3next_gated_attn_decode": (("qwen3next_hybrid", W.Q8_0, 2048, 1, 33),
                                    {"attn_gate": True, "v_norm": True}),
}


def dq(oracle, t, raw, rows, cols):
    return oracle.dequant(t, raw, rows * cols).reshape(rows, cols).astype(np.float64)


def oracle_block(oracle, cfg, wts, ids, kv_len, K0, V0):
    return oracle_stack(oracle, cfg, [wts], ids, kv_len, [K0], [V0])


def oracle_stack(oracle, cfg, layers, ids, kv_len, K0s, V0s):
    """The blocks in turn on the embedded tokens, then the last block's output
    norm; layer i attends over its own cache K0s[i], V0s[i]. The block is the
    reference's qwen_block (src/model.cpp:234-287) or, with post_norms, its
    gemma_block (:181-232), around its attention layer (src/attention_layer.
    cpp:60-263): q/gate split per head, V := K, the weightless V norm, q/k
    norms, RoPE with frequency factors, the sigmoid output gate."""
    N, H, HK, D = cfg.hidden, cfg.n_head, cfg.n_head_kv, cfg.head_dim
    T = ids.size
    pos = np.arange(kv_len, kv_len + T, dtype=np.int32)
    scale = float(np.float32(math.sqrt(N))) if cfg.emb_scale else 0.0
    ff = None if cfg.freq_factors is None else np.asarray(cfg.freq_factors, np.float32)
    h0 = layers[0].host
    x = oracle.embed_gather(cfg.emb_type, h0["emb"], cfg.vocab, N, ids, scale)
    for wts, K0, V0 in zip(layers, K0s, V0s):
        h_ = wts.host
        mats = {k: dq(oracle, cfg.wtype, h_[k], *wts.shapes[k]) for k in wts.MATS}
        ds = np.float32(wts.out_scale if cfg.out_scale_mode == 1 else 1.0)
        ss = np.float32(wts.out_scale if cfg.out_scale_mode == 2 else 1.0)

        def mm(name, a):
            return (a.astype(np.float64) @ mats[name].T).astype(np.float32)

        def norm(a, name):
            return oracle.rmsnorm_rows(a, h_[name], cfg.eps, cfg.unit_offset)

        h = norm(x, "attn_norm")
        q, k = mm("wq", h), mm("wk", h)
        v = k.copy() if cfg.v_from_k else mm("wv", h)
        gate = None
        if cfg.attn_gate:
            qg = q.reshape(T, H, 2, D)
            q, gate = np.ascontiguousarray(qg[:, :, 0]), np.ascontiguousarray(qg[:, :, 1])
        if cfg.v_norm and not cfg.v_from_k:
            v = oracle.rmsnorm_rows(v.reshape(T * HK, D), None, cfg.eps)
        q = oracle.qk_norm_rope(q, T, H, D, cfg.n_rot, pos, cfg.theta, 0, h_.get("q_norm"),
                                cfg.eps, cfg.unit_offset, ff=ff)
        k = oracle.qk_norm_rope(k, T, HK, D, cfg.n_rot, pos, cfg.theta, 0, h_.get("k_norm"),
                                cfg.eps, cfg.unit_offset, ff=ff)
        Kc = np.concatenate([K0[:kv_len], k.reshape(T, HK * D)]).reshape(-1, HK, D)
        Vc = np.concatenate([V0[:kv_len], v.reshape(T, HK * D)]).reshape(-1, HK, D)
        att = oracle.attention_tiled(q.reshape(T, H, D), Kc, Vc, 1.0 / math.sqrt(D), qpos=pos,
                                     kpos=np.arange(kv_len + T, dtype=np.int32))
        att = att.reshape(T, H * D)
        if gate is not None:
            att = oracle.act_mul(oracle.ACT_SIGMOID, gate.reshape(T, H * D), att)
        o = mm("wo", att)
        if cfg.post_norms:
            x = x + ds * norm(o, "post_attn_norm")
        else:
            x = x + o
        h = norm(x, "ffn_norm")
        g = oracle.act_mul(ACT[cfg.act], mm("wg", h), mm("wu", h))
        dn = mm("wd", g)
        if cfg.post_norms:
            x = (x + ds * norm(dn, "post_ffw_norm")) * ss
        else:
            x = x + dn
    return x, oracle.rmsnorm_rows(x, layers[-1].host["out_norm"], cfg.eps, cfg.unit_offset)


def block_options(name):
    if name not in OPTION_CASES:
        return CASES[name], {}
    case, opts = OPTION_CASES[name]
    opts = dict(opts)
    if opts.get("freq_factors") == "random":
        n_rot = W.SHAPES[case[0]].n_rot
        ff = np.random.default_rng(5).uniform(0.5, 4.0, n_rot // 2).astype(np.float32)
        opts["freq_factors"] = tuple(float(f) for f in ff)
    return case, opts


def setup(name, seed=0, n_layers=1, **kw):
    (shape, wtype, vocab, T, kv_len), opts = block_options(name)
    cfg = layer.BlockConfig.from_shape(W.SHAPES[shape], wtype, vocab=vocab, **opts)
    layers = [layer.BlockWeights(cfg, seed=seed + 17 * i) for i in range(n_layers)]
    step = layer.LayerStep(cfg, layers if n_layers > 1 else layers[0], max_tokens=T,
                           kv_cap=kv_len + T, **kw)
    rng = np.random.default_rng(seed + 1)
    ids = rng.integers(0, vocab, T).astype(np.int32)
    KD = cfg.n_head_kv * cfg.head_dim
    K0s, V0s = [], []
    for Kd, Vd in step.kv:
        K0 = rng.standard_normal((kv_len + T, KD), dtype=np.float32)
        V0 = rng.standard_normal((kv_len + T, KD), dtype=np.float32)
        Kd.copy_from(K0)
        Vd.copy_from(V0)
        K0s.append(K0)
        V0s.append(V0)
    if n_layers == 1:
        return cfg, layers[0], step, ids, kv_len, K0s[0], V0s[0]
    return cfg, layers, step, ids, kv_len, K0s, V0s


def run_and_check(oracle, name, n_layers=1, **kw):
    cfg, wts, step, ids, kv_len, K0, V0 = setup(name, n_layers=n_layers, **kw)
    T = ids.size
    print(f"layer {name} layers={n_layers} tokens={T} kv_len={kv_len} wtype={cfg.wtype} {kw}",
          flush=True)
    step.prepare(ids, kv_len)
    step.forward(T, kv_len)
    if n_layers == 1:
        want_x, want_h = oracle_block(oracle, cfg, wts, ids, kv_len, K0, V0)
    else:
        want_x, want_h = oracle_stack(oracle, cfg, wts, ids, kv_len, K0, V0)
    got_x = step.x.view((T, cfg.hidden)).numpy()
    got_h = step.h_out.view((T, cfg.hidden)).numpy()
    ex, eh = rel_to_scale(got_x, want_x), rel_to_scale(got_h, want_h)
    print(f"  rel x {ex:.2e} h_out {eh:.2e}", flush=True)
    assert ex <= RTOL and eh <= RTOL
    return step


@pytest.mark.parametrize("name", list(OPTION_CASES))
@pytest.mark.parametrize("fused", [True, False])
@pytest.mark.parametrize("n_layers", [1, 2])
def test_block_options_vs_oracle(hip, oracle, name, fused, n_layers):
    """Gemma sandwich norms with the layer output scale on the deltas or the
    whole sum, V := K, the gated attention with the V norm and frequency
    factors: one block and a 2-block stack (the post-norm of a block's FFN
    output applied at the next block's first norm) against the oracle's
    composition, with every fusion on and off."""
    fus = None if fused else {f: False for f in select.FUSIONS}
    step = run_and_check(oracle, name, n_layers=n_layers, fusions=fus)
    assert not step.uses_host()


@pytest.mark.parametrize("name", list(CASES))
@pytest.mark.parametrize("fused", [True, False])
def test_layer_vs_oracle(hip, oracle, name, fused):
    fus = None if fused else {f: False for f in select.FUSIONS}
    step = run_and_check(oracle, name, fusions=fus)
    assert not step.uses_host()
    if fused and CASES[name][3] >= 32:
        # the fold decision follows the library's split rule for every type
        assert step._folds_norm(CASES[name][3])


@pytest.mark.parametrize("name,n_layers", [("qwen2_0p5b_decode", 3), ("llama3_8b_prefill", 2),
                                           ("llama3_8b_decode", 2), ("gemma_like_prefill", 2)])
@pytest.mark.parametrize("fused", [True, False])
def test_layer_stack_vs_oracle(hip, oracle, name, n_layers, fused):
    """A stack of blocks, each with its own weights and KV cache: a block's
    FFN output is added to x by the next block's attention norm (at 32+ tokens
    in the q/k/v GEMMs' pre-pass), and by the output norm after the last."""
    fus = None if fused else {f: False for f in select.FUSIONS}
    step = run_and_check(oracle, name, n_layers=n_layers, fusions=fus)
    assert not step.uses_host()


def test_layer_plan_replay(hip, oracle):
    """The step recorded as a plan and replayed twice gives the oracle's
    result both times (a replay starts from the embedding gather and writes
    the same KV cache rows, so nothing carries over between replays)."""
    from aero_amd.device import Plan, Stream, synchronize

    cfg, wts, step, ids, kv_len, K0, V0 = setup("llama3_8b_prefill")
    T = ids.size
    step.prepare(ids, kv_len)
    plan = Plan()
    with plan:
        step.forward(T, kv_len)
    want_x, want_h = oracle_block(oracle, cfg, wts, ids, kv_len, K0, V0)
    stream = Stream()
    for _ in range(2):
        plan.launch(stream)
        stream.synchronize()
        synchronize()
        assert rel_to_scale(step.h_out.view((T, cfg.hidden)).numpy(), want_h) <= RTOL
        assert rel_to_scale(step.x.view((T, cfg.hidden)).numpy(), want_x) <= RTOL
    plan.destroy()
    stream.destroy()


def test_layer_host_hooks(hip, oracle):
    """rope and act taken off the GPU: the caller's host code (here the
    oracle's) runs at those sites, the rest stays on the GPU."""
    cfg = layer.BlockConfig.from_shape(W.SHAPES["qwen2_0p5b_decode"], W.Q8_0, vocab=4096)

    def rope(q, k, pos):
        T, H, D = q.shape
        qo = oracle.qk_norm_rope(q, T, H, D, cfg.n_rot, pos, cfg.theta)
        ko = oracle.qk_norm_rope(k, T, k.shape[1], D, cfg.n_rot, pos, cfg.theta)
        return qo, ko

    def act(g, u):
        return oracle.act_mul(ACT[cfg.act], g, u)

    step = run_and_check(oracle, "qwen2_0p5b_decode", gpu_ops={"rope": False, "act": False},
                         hooks={"rope": rope, "act": act})
    assert step.uses_host()


def test_layer_refuses_without_host_path(hip):
    cfg, wts, step, ids, kv_len, _, _ = setup("qwen2_0p5b_decode", gpu_ops={"rmsnorm": False})
    step.prepare(ids, kv_len)
    with pytest.raises(select.HostPathRequired):
        step.forward(ids.size, kv_len)


def test_layer_decode_rope_fold(hip, oracle):
    """At one token the q/k/v GEMV rotates q and k in its epilogue: the
    Llama-3-8B decode block records one launch fewer than with rope_gemm
    off, and both match the oracle."""
    from aero_amd.device import Plan

    counts = {}
    for fold in (True, False):
        step = run_and_check(oracle, "llama3_8b_decode", fusions={"rope_gemm": fold})
        cfg = step.cfg
        plan = Plan()
        with plan:
            step.forward(1, CASES["llama3_8b_decode"][4])
        counts[fold] = len(plan)
        plan.destroy()
    assert counts[True] == counts[False] - 1, counts


def test_layer_prefill_ten_launches(hip, oracle):
    """At 512 Llama-3-8B tokens the q/k/v pre-pass reads the embedding rows
    and the q/k/v GEMM's epilogue runs RoPE: the block records 10 launches,
    12 with embed_gemm and rope_gemm off, and both match the oracle."""
    from aero_amd.device import Plan

    counts = {}
    for fold in (True, False):
        step = run_and_check(oracle, "llama3_8b_prefill",
                             fusions={"rope_gemm": fold, "embed_gemm": fold})
        plan = Plan()
        with plan:
            step.forward(512, 0)
        counts[fold] = len(plan)
        plan.destroy()
    assert counts == {True: 10, False: 12}, counts


def test_stack_prefill_then_decode(hip, oracle):
    """A 2-layer Llama-3-8B stack run as a model runs it: 16 prompt tokens at
    positions 0-15 (the split GEMMs with the norms folded), then 3 decode
    tokens at positions 16, 17, 18 (the fused decode GEMVs with RoPE in the
    epilogue), each step attending over the K/V rows the earlier steps wrote.
    The oracle keeps its own K/V cache from its own projections; every
    step's x and h_out match it to 1e-5 of scale."""
    shape, wtype, vocab = "llama3_8b_prefill", W.Q4_K, 4096
    cfg = layer.BlockConfig.from_shape(W.SHAPES[shape], wtype, vocab=vocab)
    layers = [layer.BlockWeights(cfg, seed=40 + i) for i in range(2)]
    n_prompt, n_dec = 16, 3
    cap = n_prompt + n_dec
    step = layer.LayerStep(cfg, layers, max_tokens=n_prompt, kv_cap=cap)
    KD = cfg.n_head_kv * cfg.head_dim
    Ks = [np.zeros((cap, KD), np.float32) for _ in layers]
    Vs = [np.zeros((cap, KD), np.float32) for _ in layers]
    rng = np.random.default_rng(7)
    prompt = rng.integers(0, vocab, n_prompt).astype(np.int32)
    N, H, HK, D = cfg.hidden, cfg.n_head, cfg.n_head_kv, cfg.head_dim

    def oracle_step(ids, kv_len):
        """The stack on ids at positions kv_len.., extending Ks / Vs."""
        T = ids.size
        pos = np.arange(kv_len, kv_len + T, dtype=np.int32)
        x = oracle.embed_gather(cfg.emb_type, layers[0].host["emb"], cfg.vocab, N, ids, 0.0)
        for li, wts in enumerate(layers):
            h_ = wts.host
            mats = {k: dq(oracle, cfg.wtype, h_[k], *wts.shapes[k]) for k in wts.MATS}

            def mm(name, a):
                return (a.astype(np.float64) @ mats[name].T).astype(np.float32)

            h = oracle.rmsnorm_rows(x, h_["attn_norm"], cfg.eps, cfg.unit_offset)
            q, k, v = mm("wq", h), mm("wk", h), mm("wv", h)
            q = oracle.qk_norm_rope(q, T, H, D, cfg.n_rot, pos, cfg.theta, 0)
            k = oracle.qk_norm_rope(k, T, HK, D, cfg.n_rot, pos, cfg.theta, 0)
            Ks[li][kv_len:kv_len + T] = k.reshape(T, KD)
            Vs[li][kv_len:kv_len + T] = v.reshape(T, KD)
            S = kv_len + T
            att = oracle.attention_tiled(q.reshape(T, H, D), Ks[li][:S].reshape(S, HK, D),
                                         Vs[li][:S].reshape(S, HK, D), 1.0 / math.sqrt(D),
                                         qpos=pos, kpos=np.arange(S, dtype=np.int32))
            x = x + mm("wo", att.reshape(T, H * D))
            h = oracle.rmsnorm_rows(x, h_["ffn_norm"], cfg.eps, cfg.unit_offset)
            x = x + mm("wd", oracle.act_mul(ACT[cfg.act], mm("wg", h), mm("wu", h)))
        return x, oracle.rmsnorm_rows(x, layers[-1].host["out_norm"], cfg.eps, cfg.unit_offset)

    def check(T, kv_len, ids, what):
        step.prepare(ids, kv_len)
        step.forward(T, kv_len)
        want_x, want_h = oracle_step(ids, kv_len)
        ex = rel_to_scale(step.x.view((T, N)).numpy(), want_x)
        eh = rel_to_scale(step.h_out.view((T, N)).numpy(), want_h)
        print(f"  {what}: rel x {ex:.2e} h_out {eh:.2e}", flush=True)
        assert ex <= RTOL and eh <= RTOL, what
        return want_h

    print("stack prefill 16 then decode 3", flush=True)
    check(n_prompt, 0, prompt, "prompt")
    for i in range(n_dec):
        tok = np.array([rng.integers(0, vocab)], np.int32)
        check(1, n_prompt + i, tok, f"decode {i}")
    # the caches the GPU steps wrote hold the oracle's rows
    for li in range(len(layers)):
        Kd, Vd = step.kv[li]
        assert rel_to_scale(Kd.numpy(), Ks[li]) <= RTOL
        assert rel_to_scale(Vd.numpy(), Vs[li]) <= RTOL
