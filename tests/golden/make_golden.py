"""Write the golden fixtures under tests/golden/ (run in the build container,
where the reference tree exists):

    make -C oracle ref && python tests/golden/make_golden.py

1. kat_quant.npz -- hand-built quant blocks from the reference's own tests,
   rebuilt here from the constructions those tests describe, with the values
   the tests assert:
     * Q4_K, d=1, dmin=0, scales [1,1,1,1,0,0,0,0,1,1,1,1],
       qs[i] = (i & 15) | ((31-i) & 15) << 4  ->  output = the nibbles
       (tests/test_quant.py:72-93), and the same block with dmin=2 (no-op);
     * Q4_K make_q4k packer: sc = 1..8, mn = 8..1, quants (3i) & 0xFF,
       d = 1 with dmin = 0 and 1 -> d*sc*q - dmin*mn (tests/test_kernels.cpp:
       80-154);
     * Q6_K all-zero bits -> -32, all-one bits -> 31, low-nibble pattern ->
       -17 / -32 (tests/test_quant.py:96-124);
     * Q8_0 d = 0.5, q = 0..31 -> 0.5*i (tests/test_quant.py:127-131).
2. ref_vectors.npz -- inputs and outputs of the reference's own C++ (built
   into oracle/_ref/ from src/kernels.cpp, src/transformer.cpp and
   src/tensor.cpp) on small seeded inputs: row norms, activations, RoPE tables
   and rotation, Q8_0 / Q4_K / Q5_K / Q6_K / IQ4_XS dequant, matvec /
   matmul over each of those block types, row softmax, GQA attention (causal
   with positions, a window, shuffled key positions) and the int8 / int4 KV
   vector quantisers. These pin the oracle and the GPU
   path on machines where the reference build is absent.
"""
from __future__ import annotations

import os
import struct
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)


def f16(v: float) -> bytes:
    return struct.pack("<e", v)


def kat_blocks() -> dict:
    out = {}
    # tests/test_quant.py:72-93
    scales = bytes([1, 1, 1, 1, 0, 0, 0, 0, 1, 1, 1, 1])
    qs = bytes([(i & 0x0F) | (((31 - i) & 0x0F) << 4) for i in range(128)])
    blk = f16(1.0) + f16(0.0) + scales + qs
    lo = np.array([i & 0x0F for i in range(128)], np.float32)
    hi = np.array([(31 - i) & 0x0F for i in range(128)], np.float32)
    want = np.empty(256, np.float32)
    for j in range(4):
        want[j * 64:j * 64 + 32] = lo[j * 32:(j + 1) * 32]
        want[j * 64 + 32:j * 64 + 64] = hi[j * 32:(j + 1) * 32]
    out["q4k_nibbles_raw"] = np.frombuffer(blk, np.uint8)
    out["q4k_nibbles_want"] = want
    out["q4k_nibbles_dmin2_raw"] = np.frombuffer(f16(1.0) + f16(2.0) + scales + qs, np.uint8)

    # tests/test_kernels.cpp:80-154 (make_q4k)
    sc = [1, 2, 3, 4, 5, 6, 7, 8]
    mn = [8, 7, 6, 5, 4, 3, 2, 1]
    quants = [(i * 3) & 0xFF for i in range(128)]
    for dmin in (0.0, 1.0):
        b = bytearray(144)
        b[0:2] = f16(1.0)
        b[2:4] = f16(dmin)
        for j in range(4):
            b[4 + j] = (sc[j] & 0x3F) | (((sc[j + 4] >> 4) & 0x03) << 6)
            b[8 + j] = (mn[j] & 0x3F) | (((mn[j + 4] >> 4) & 0x03) << 6)
            b[12 + j] = (sc[j + 4] & 0x0F) | ((mn[j + 4] & 0x0F) << 4)
        b[16:144] = bytes(quants)
        vals = np.empty(256, np.float32)
        col = 0
        for j in range(0, 256, 64):
            for half in range(2):
                sb = j // 32 + half
                for i in range(32):
                    byte = quants[col + i]
                    q = (byte & 0x0F) if half == 0 else (byte >> 4)
                    vals[j + half * 32 + i] = (np.float32(1.0) * np.float32(sc[sb]) * np.float32(q)
                                               - np.float32(dmin) * np.float32(mn[sb]))
            col += 32
        tag = f"q4k_pack_dmin{int(dmin)}"
        out[tag + "_raw"] = np.frombuffer(bytes(b), np.uint8)
        out[tag + "_want"] = vals

    # tests/test_quant.py:96-124
    sc6 = bytes([1] * 16)
    out["q6k_zero_raw"] = np.frombuffer(bytes(128) + bytes(64) + sc6 + f16(1.0), np.uint8)
    out["q6k_zero_want"] = np.full(256, -32.0, np.float32)
    out["q6k_ones_raw"] = np.frombuffer(bytes([0xFF] * 192) + sc6 + f16(1.0), np.uint8)
    out["q6k_ones_want"] = np.full(256, 31.0, np.float32)
    out["q6k_lownib_raw"] = np.frombuffer(bytes([0x0F] * 128) + bytes(64) + sc6 + f16(1.0),
                                          np.uint8)
    w6 = np.empty(256, np.float32)
    for half in range(2):
        b0 = half * 128
        w6[b0:b0 + 64] = -17.0
        w6[b0 + 64:b0 + 128] = -32.0
    out["q6k_lownib_want"] = w6

    # tests/test_quant.py:127-131
    out["q8_0_ramp_raw"] = np.frombuffer(f16(0.5) + bytes(range(32)), np.uint8)
    out["q8_0_ramp_want"] = np.arange(32, dtype=np.float32) * np.float32(0.5)
    return out


def ref_vectors() -> dict:
    from oracle import refbind as R

    if not R.available():
        raise SystemExit("oracle/_ref not built: run `make -C oracle ref` first")
    rng = np.random.default_rng(20261015)
    v = {}
    # norms (tests/test_transformer_native.py:112-121 style inputs, more rows)
    x = (rng.standard_normal((9, 48)) * 2.0).astype(np.float32)
    w = (rng.standard_normal(48) + 2.0).astype(np.float32)
    v["norm_x"], v["norm_w"] = x, w
    v["rms_out"] = R.rmsnorm_rows(x, w, 1e-6)
    v["rms_out_noweight"] = R.rmsnorm_rows(x, None, 1e-6)
    v["l2_out"] = R.l2norm_rows(x, w, 1e-6)
    big = rng.standard_normal((3, 4096)).astype(np.float32)
    wb = (1 + 0.1 * rng.standard_normal(4096)).astype(np.float32)
    v["rms4096_x"], v["rms4096_w"] = big, wb
    v["rms4096_out"] = R.rmsnorm_rows(big, wb, 1e-5)
    # activations over [-6, 6] and random
    z = np.concatenate([np.linspace(-6, 6, 401, dtype=np.float32),
                        (rng.standard_normal(1024) * 5).astype(np.float32)])
    up = rng.standard_normal(z.size).astype(np.float32)
    v["act_z"], v["act_up"] = z, up
    v["silu_out"] = R.act("silu", z)
    v["gelu_out"] = R.act("gelu", z)
    v["swiglu_out"] = R.swiglu(z, up)
    v["mul_out"] = R.mul(z, up)
    # RoPE tables: full / partial / proportional, large positions
    pos = rng.integers(0, 32768, size=37).astype(np.int32)
    v["rope_pos"] = pos
    for tag, hd, nd, base, ff in (("full128", 128, None, 500000.0, None),
                                  ("partial64of256", 256, 64, 1e7, None),
                                  ("ff64", 64, None, 10000.0,
                                   np.concatenate([np.ones(16, np.float32),
                                                   np.full(16, 1e30, np.float32)]))):
        c, s = R.rope_tables(hd, pos, base, nd, ff)
        v[f"tab_{tag}_cos"], v[f"tab_{tag}_sin"] = c, s
    # apply_rope on a dense table, NeoX / interleaved / partial
    T, H, D = 6, 3, 32
    xr = rng.standard_normal((T * H, D)).astype(np.float32)
    c, s = R.rope_tables(D, np.arange(T, dtype=np.int32), 10000.0)
    rowpos = np.repeat(np.arange(T), H).astype(np.int32)
    v["apply_x"], v["apply_cos"], v["apply_sin"], v["apply_pos"] = xr, c, s, rowpos
    v["apply_neox"] = R.apply_rope(xr, c, s, rowpos, 0)
    v["apply_inter"] = R.apply_rope(xr, c, s, rowpos, 1)
    c8, s8 = R.rope_tables(D, np.arange(T, dtype=np.int32), 10000.0, 8)
    v["apply_cos8"], v["apply_sin8"] = c8, s8
    v["apply_partial8"] = R.apply_rope(xr, c8, s8, rowpos, 0)
    # dequant: random blocks with realistic fp16 scales
    for t, bb, nb in ((8, 34, 40), (12, 144, 12), (14, 210, 12)):
        raw = rng.integers(0, 256, nb * bb, dtype=np.uint8).reshape(nb, bb)
        if t == 8:
            raw[:, 0:2] = np.frombuffer((np.abs(rng.standard_normal(nb) * 0.02) / 127)
                                        .astype(np.float16).tobytes(), np.uint8).reshape(nb, 2)
        elif t == 12:
            raw[:, 0:4] = np.frombuffer(np.abs(rng.standard_normal(2 * nb) * 0.01)
                                        .astype(np.float16).tobytes(), np.uint8).reshape(nb, 4)
        else:
            raw[:, 208:210] = np.frombuffer(np.abs(rng.standard_normal(nb) * 0.01)
                                            .astype(np.float16).tobytes(), np.uint8).reshape(nb, 2)
        raw = raw.reshape(-1)
        bv = 32 if t == 8 else 256
        v[f"deq{t}_raw"] = raw
        v[f"deq{t}_out"] = R.dequant(t, raw, nb * bv)
    # Q5_K and IQ4_XS dequant; matvec and matmul of every block type
    from aero_amd import workloads as W
    for t in (W.Q5_K, W.IQ4_XS):
        raw = W.make_table(t, 12, rng)
        v[f"deq{t}_raw"] = raw
        v[f"deq{t}_out"] = R.dequant(t, raw, 12 * 256)
    for t in (W.Q8_0, W.Q4_K, W.Q5_K, W.Q6_K, W.IQ4_XS):
        n_rows, n_cols = 24, 512
        bv, bb = W.BLOCK[t]
        w = W.make_table(t, n_rows * n_cols // bv, rng)
        X = rng.standard_normal((3, n_cols)).astype(np.float32)
        v[f"mv{t}_w"], v[f"mv{t}_x"] = w, X
        v[f"mv{t}_y"] = R.matvec(t, w, X[0], n_rows)
        v[f"mm{t}_y"] = R.matmul(t, w, X, n_rows)
    # softmax rows and GQA attention (src/tensor.cpp:167-178,
    # src/transformer.cpp:120-214): prefill-style causal with positions, a
    # window, a fully masked query (position below every key), and decode
    sm = (rng.standard_normal((6, 37)) * 4).astype(np.float32)
    v["softmax_x"], v["softmax_y"] = sm, R.softmax(sm)
    T, H, HK, D, DV, S = 7, 8, 2, 64, 48, 50
    q = rng.standard_normal((T, H, D)).astype(np.float32)
    k = rng.standard_normal((S, HK, D)).astype(np.float32)
    vv = rng.standard_normal((S, HK, DV)).astype(np.float32)
    qpos = np.array([0, 5, 17, 31, 49, 49, -1], np.int32)
    v["att_q"], v["att_k"], v["att_v"], v["att_qpos"] = q, k, vv, qpos
    v["att_out"] = R.attention_tiled(q, k, vv, 0.125, qpos=qpos, block=16)
    v["att_out_win8"] = R.attention_tiled(q, k, vv, 0.125, qpos=qpos, block=16, window=8)
    kpos = rng.permutation(S).astype(np.int32)
    v["att_kpos"] = kpos
    v["att_out_kpos"] = R.attention_tiled(q, k, vv, 0.125, qpos=qpos, kpos=kpos, block=1024)
    # KV quantisers (src/kv.cpp:13-46)
    kvx = (rng.standard_normal((5, 64)) * np.array([1, 1e-3, 30, 0, 7], np.float32)[:, None])
    kvx = kvx.astype(np.float32)
    v["kv_x"] = kvx
    for dt in (1, 2):
        qs, sc = zip(*(R.kv_write_vec(dt, row) for row in kvx))
        v[f"kv{dt}_q"] = np.stack(qs)
        v[f"kv{dt}_scale"] = np.array(sc, np.float32)
    # gated DeltaNet scan and causal conv (src/ssm.cpp:69-210): 6 tokens,
    # 2 k-heads, 4 v-heads, d = 32; a conv over 8 channels in two chunks
    T, NK, NV, D = 6, 2, 4, 32
    sq = rng.standard_normal((T, NK, D)).astype(np.float32)
    sk = rng.standard_normal((T, NK, D)).astype(np.float32)
    sv = rng.standard_normal((T, NV, D)).astype(np.float32)
    sal = rng.standard_normal((T, NV)).astype(np.float32)
    sbt = rng.standard_normal((T, NV)).astype(np.float32)
    sa = (-np.abs(rng.standard_normal(NV)) * 0.5).astype(np.float32)
    sdt = rng.standard_normal(NV).astype(np.float32)
    s0 = (rng.standard_normal((NV, D, D)) * 0.1).astype(np.float32)
    for name, arr in (("q", sq), ("k", sk), ("v", sv), ("alpha", sal), ("beta", sbt),
                      ("a_log", sa), ("dt_bias", sdt), ("state", s0)):
        v[f"ssm_{name}"] = arr
    v["ssm_out"], v["ssm_state_out"] = R.ssm_scan(sq, sk, sv, sal, sbt, sa, sdt, s0, 0.125)
    cx = rng.standard_normal((9, 8)).astype(np.float32)
    cw = rng.standard_normal((8, 4)).astype(np.float32)
    o1, t1, l1 = R.ssm_conv(cx[:2], cw, None, 0)
    o2, t2, l2 = R.ssm_conv(cx[2:], cw, t1, l1)
    v["conv_x"], v["conv_w"] = cx, cw
    v["conv_out"], v["conv_tail"] = np.concatenate([o1, o2]), t2
    return v


def main():
    np.savez_compressed(os.path.join(HERE, "kat_quant.npz"), **kat_blocks())
    np.savez_compressed(os.path.join(HERE, "ref_vectors.npz"), **ref_vectors())
    print("wrote", os.path.join(HERE, "kat_quant.npz"), os.path.join(HERE, "ref_vectors.npz"))


if __name__ == "__main__":
    main()
