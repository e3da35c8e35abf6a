/* oracle/cpuref.c -- fp32 part of the CPU restatement (norms, activations,
 * RoPE, gated norm).
 *
 * TEST INFRASTRUCTURE: the oracle of the HIP path, and the "port" CPU
 * baseline. Built with gcc -O2 -ffp-contract=off and no -ffast-math, as the
 * reference builds its fp32 libraries (Makefile:74-76,144-154), so every
 * multiply and add rounds separately and summation is serial in fp32.
 *
 * How each function is pinned (tests/test_oracle.py):
 *   cr_rmsnorm_rows    float64 closed form x/sqrt(mean(x^2)+eps)*w; "ones in ->
 *                      weight out" (tests/test_tensor.cpp:98-104); weight=NULL
 *                      bit-identical to ones (tests/test_transformer_cpp.cpp:
 *                      289-294); compiled reference src/transformer.cpp when
 *                      it builds (bit-exact).
 *   cr_l2norm_rows     float64 closed form with the max(norm, eps) floor; the
 *                      sub-eps floor case of tests/test_tensor_native.py:
 *                      154-181; compiled reference (bit-exact).
 *   cr_gated_rmsnorm_silu  float64 closed form of src/ssm.cpp:327-343;
 *                      invariants (z -> +inf with w = 1 gives unit RMS over the
 *                      group; group = inner has no per-head effect). The
 *                      reference only reaches this arithmetic inside
 *                      aero_ssm_forward_q: the layer composed around it
 *                      (cpuref.py ssm_forward) equals that function compiled
 *                      from the reference within 1e-5 of scale.
 *   cr_act / cr_act_mul  math.erf / math.tanh / exp closed forms in float64;
 *                      spot values of tests/test_tensor_native.py:118-132;
 *                      compiled reference (bit-exact for silu/gelu/swiglu/mul).
 *                      gelu_tanh has no reference function: closed form only.
 *                      sigmoid (kind 4, the attention output gate): float64
 *                      closed form, and v * sigmoid(v) is the compiled
 *                      reference's silu bit for bit.
 *   cr_dense_matvec / cr_dense_matmul  compiled reference src/tensor.cpp
 *                      (bit-exact, 1-5 tokens, ragged widths); float64 product
 *                      to 5e-6 of scale; a planted regrouping of the sum (one
 *                      product at a time in the matvec) is caught by the
 *                      bit-exact check.
 *   cr_argmax          compiled reference (bit-exact) on ties, NaN at 0 and
 *                      elsewhere, signed zeros, infinities; np.argmax on
 *                      NaN-free input.
 *   cr_rope_*          compiled reference (bit-exact); relative-position
 *                      invariance, norm preservation, tail pass-through and
 *                      freq_factor 1e30 => cos 1, sin 0
 *                      (tests/test_transformer_cpp.cpp:137-257); float64
 *                      closed form of the angle.
 */
#include "cpuref.h"

#include <math.h>
#include <stddef.h>
#include <stdlib.h>
#include <string.h>

/* ------------------------------------------------------------------ norms */

/* src/tensor.cpp:128-134 (rmsnorm) applied per row as src/transformer.cpp:
 * 98-104 does. ss accumulates serially in fp32, inv = 1/sqrt(ss/n + eps), and
 * out = (x*inv)*w. unit_offset = 1 is the Gemma-style (1+w) composition:
 * w' = 1 + w in fp32, then the same expression (the reference has no such
 * function; this is rms_norm(x, np.float32(1) + w)). out may alias x. */
void cr_rmsnorm_rows(const float* x, const float* w, float* out, int64_t rows,
                     int64_t cols, float eps, int unit_offset) {
    for (int64_t r = 0; r < rows; ++r) {
        const float* xr = x + r * cols;
        float* o = out + r * cols;
        float ss = 0.0f;
        for (int64_t c = 0; c < cols; ++c) ss += xr[c] * xr[c];
        const float inv = 1.0f / sqrtf(ss / (float)cols + eps);
        for (int64_t c = 0; c < cols; ++c) {
            const float v = xr[c] * inv;
            if (w == NULL) {
                o[c] = v * 1.0f;
            } else {
                const float wc = unit_offset ? 1.0f + w[c] : w[c];
                o[c] = v * wc;
            }
        }
    }
}

/* src/tensor.cpp:136-154 (l2norm) per row as src/transformer.cpp:106-113:
 * denominator max(||x||, eps), weighted iff w != NULL. */
void cr_l2norm_rows(const float* x, const float* w, float* out, int64_t rows,
                    int64_t cols, float eps) {
    for (int64_t r = 0; r < rows; ++r) {
        const float* xr = x + r * cols;
        float* o = out + r * cols;
        float ss = 0.0f;
        for (int64_t c = 0; c < cols; ++c) ss += xr[c] * xr[c];
        const float nrm = sqrtf(ss);
        const float inv = 1.0f / (nrm > eps ? nrm : eps);
        for (int64_t c = 0; c < cols; ++c)
            o[c] = xr[c] * inv * (w ? w[c] : 1.0f);
    }
}

/* silu in the division form of src/ssm.cpp:17. */
static float silu_div(float v) { return v / (1.0f + expf(-v)); }

/* Gated RMSNorm * silu, src/ssm.cpp:327-343 (numpy twin engine/ssm.py:
 * 346-348). For each `group`-long slice of a row: ss over the slice,
 * denom = sqrt(ss/group + eps), out = ((x/denom) * w[col % w_len]) * silu(z),
 * where col is the column inside the `inner`-long row. group = inner is the
 * reference (whole-row RMS over the inner dimension); a smaller group that divides
 * inner is the per-head reading. */
void cr_gated_rmsnorm_silu(const float* x, const float* z, const float* w,
                           int64_t w_len, float* out, int64_t rows,
                           int64_t inner, int64_t group, float eps) {
    const int64_t gpr = inner / group;
    for (int64_t r = 0; r < rows; ++r) {
        for (int64_t g = 0; g < gpr; ++g) {
            const int64_t off = r * inner + g * group;
            const float* xr = x + off;
            const float* zr = z + off;
            float* o = out + off;
            float ss = 0.0f;
            for (int64_t c = 0; c < group; ++c) ss += xr[c] * xr[c];
            ss /= (float)group;
            const float denom = sqrtf(ss + eps);
            for (int64_t c = 0; c < group; ++c) {
                const float wn = w[(g * group + c) % w_len];
                o[c] = (xr[c] / denom) * wn * silu_div(zr[c]);
            }
        }
    }
}

/* ------------------------------------------------------------ activations */

/* src/tensor.cpp:47 */
static float sigmoid_recip(float v) { return 1.0f / (1.0f + expf(-v)); }

/* Abramowitz & Stegun 7.1.26 erf (published constants), evaluated in the
 * order of src/tensor.cpp:52-59. */
static float erf_as(float v) {
    const float s = copysignf(1.0f, v);
    const float a = fabsf(v);
    const float t = 1.0f / (1.0f + 0.3275911f * a);
    const float p = ((((1.061405429f * t - 1.453152027f) * t + 1.421413741f) * t
                      - 0.284496736f) * t + 0.254829592f) * t;
    return s * (1.0f - p * expf(-a * a));
}

static float act1(int kind, float v) {
    switch (kind) {
    case 0: /* src/tensor.cpp:104-106: v *= sigmoid(v) */
        return v * sigmoid_recip(v);
    case 1: /* src/tensor.cpp:108-114 */
        return 0.5f * v * (1.0f + erf_as(v * 0.7071067811865476f));
    case 2: /* tanh-approximate GELU: no reference function; closed form */
        return 0.5f * v *
               (1.0f + tanhf(0.7978845608028654f * (v + 0.044715f * v * v * v)));
    case 4: /* src/attention_layer.cpp:262-263: the output gate 1/(1+exp(-g)) */
        return sigmoid_recip(v);
    default:
        return v;
    }
}

void cr_act(int kind, float* v, int64_t n) {
    for (int64_t i = 0; i < n; ++i) v[i] = act1(kind, v[i]);
}

/* out = act(gate) * up. kind 0 is swiglu_ (src/tensor.cpp:120-125,
 * (g*sigmoid(g))*u); kind 1 is gelu_ then mul_ (src/tensor.cpp:108-118, as
 * src/model.cpp:224-225 calls them); kind 3 is mul_ alone. */
void cr_act_mul(int kind, const float* gate, const float* up, float* out,
                int64_t n) {
    for (int64_t i = 0; i < n; ++i) {
        const float a = act1(kind, gate[i]);
        out[i] = up ? a * up[i] : a;
    }
}

/* ------------------------------------------------------------------- RoPE */

/* The per-pair inverse frequency of src/transformer.cpp:34-47:
 * n = head dim or min(n_dims, head_dim), rounded down to even;
 * inv[p] = 1/powf(base, (float)p*2/(float)n), divided by ff[p] when given.
 * Returns n (the rotated width) or -1 on the reference's refusals. */
int64_t cr_rope_inv_freq(int64_t head_dim, int64_t n_dims, float base,
                         const float* ff, int64_t n_ff, float* inv_out) {
    if (head_dim <= 0) return -1;
    int64_t n = (n_dims <= 0) ? head_dim : (n_dims < head_dim ? n_dims : head_dim);
    n -= n % 2;
    const int64_t half = n / 2;
    if (half <= 0) return n;
    if (ff != NULL && n_ff < half) return -1;
    for (int64_t p = 0; p < half; ++p) {
        const float e = (float)((float)p * 2.0f / (float)n);
        float inv = 1.0f / powf(base, e);
        if (ff != NULL) inv /= ff[p];
        inv_out[p] = inv;
    }
    return n;
}

/* src/transformer.cpp:27-61. ROW-indexed: row t holds (float)pos[t]*inv[p]. */
int64_t cr_rope_tables(int64_t head_dim, const int32_t* pos, int64_t n_pos,
                       float base, int64_t n_dims, const float* ff,
                       int64_t n_ff, float* cos_out, float* sin_out) {
    if (head_dim <= 0 || n_pos < 0 || pos == NULL) return -1;
    float inv[4096];
    int64_t n = (n_dims <= 0) ? head_dim : (n_dims < head_dim ? n_dims : head_dim);
    n -= n % 2;
    if (n / 2 > 4096) return -1;
    const int64_t got = cr_rope_inv_freq(head_dim, n_dims, base, ff, n_ff, inv);
    if (got < 0) return -1;
    const int64_t half = got / 2;
    for (int64_t t = 0; t < n_pos; ++t) {
        for (int64_t p = 0; p < half; ++p) {
            const float ang = (float)pos[t] * inv[p];
            cos_out[t * half + p] = cosf(ang);
            sin_out[t * half + p] = sinf(ang);
        }
    }
    return got;
}

/* src/transformer.cpp:63-96. In place; row r reads table row pos[r] (or r):
 * POSITION-indexed. mode 0 = NeoX (x[p], x[p+half]); anything else pairs
 * (x[2p], x[2p+1]). Channels >= 2*half are untouched. */
void cr_apply_rope(float* x, int64_t n_rows, int64_t head_dim, int64_t n_rot,
                   const float* cos_tab, const float* sin_tab,
                   const int32_t* pos, int mode) {
    const int64_t half = n_rot / 2;
    if (half <= 0 || head_dim <= 0) return;
    for (int64_t r = 0; r < n_rows; ++r) {
        float* xr = x + r * head_dim;
        const int64_t pi = pos ? (int64_t)pos[r] : r;
        const float* c = cos_tab + pi * half;
        const float* s = sin_tab + pi * half;
        for (int64_t p = 0; p < half; ++p) {
            const int64_t i0 = (mode == 0) ? p : 2 * p;
            const int64_t i1 = (mode == 0) ? p + half : 2 * p + 1;
            const float x0 = xr[i0];
            const float x1 = xr[i1];
            xr[i0] = x0 * c[p] - x1 * s[p];
            xr[i1] = x0 * s[p] + x1 * c[p];
        }
    }
}

/* ------------------------------------------------------------ softmax */
/* src/tensor.cpp:167-178: max, exp(v - max) summed serially, times 1/sum
 * (0 when the sum is not positive). */
static float cr_fmax_(float a, float b) { return (a < b) ? b : a; }  /* std::max */

void cr_softmax(float* v, int64_t n) {
    if (n <= 0) return;
    float m = v[0];
    for (int64_t i = 1; i < n; ++i) m = cr_fmax_(m, v[i]);
    float s = 0.0f;
    for (int64_t i = 0; i < n; ++i) {
        v[i] = expf(v[i] - m);
        s += v[i];
    }
    const float inv = (s > 0.0f) ? 1.0f / s : 0.0f;
    for (int64_t i = 0; i < n; ++i) v[i] *= inv;
}

void cr_softmax_rows(float* v, int64_t n_rows, int64_t n_cols) {
    for (int64_t r = 0; r < n_rows; ++r) cr_softmax(v + r * n_cols, n_cols);
}

/* ------------------------------------------------------ dense fp32 */
/* src/tensor.cpp:65-81 matvec: per row, four products summed left to right
 * and added to acc at a time, then the tail one product at a time. */
void cr_dense_matvec(const float* w, const float* x, float* y, int64_t n_rows,
                     int64_t n_cols) {
    for (int64_t r = 0; r < n_rows; ++r) {
        const float* wr = w + r * n_cols;
        float acc = 0.0f;
        int64_t c = 0;
        for (; c + 4 <= n_cols; c += 4) {
            float g = wr[c] * x[c];
            g = g + wr[c + 1] * x[c + 1];
            g = g + wr[c + 2] * x[c + 2];
            g = g + wr[c + 3] * x[c + 3];
            acc = acc + g;
        }
        for (; c < n_cols; ++c) acc = acc + wr[c] * x[c];
        y[r] = acc;
    }
}

/* src/tensor.cpp:83-92 matmul: one token is the matvec; several sum each
 * row's products one at a time. Y is [n_tok, n_rows]. */
void cr_dense_matmul(const float* w, const float* x, float* y, int64_t n_tok, int64_t n_rows,
                     int64_t n_cols) {
    if (n_tok == 1) {
        cr_dense_matvec(w, x, y, n_rows, n_cols);
        return;
    }
    for (int64_t r = 0; r < n_rows; ++r)
        for (int64_t t = 0; t < n_tok; ++t) {
            float acc = 0.0f;
            for (int64_t c = 0; c < n_cols; ++c) acc = acc + w[r * n_cols + c] * x[t * n_cols + c];
            y[t * n_rows + r] = acc;
        }
}

/* src/tensor.cpp:180-186 argmax: start at v[0], move on only to a strictly
 * larger value (so the first of equal maxima wins and NaN is never taken). */
int cr_argmax(const float* v, int64_t n) {
    int best = 0;
    float bv = v[0];
    for (int64_t i = 1; i < n; ++i)
        if (v[i] > bv) {
            bv = v[i];
            best = (int)i;
        }
    return best;
}

/* ---------------------------------------------------------- attention */
/* src/transformer.cpp:120-203: grouped-query attention with an online softmax
 * over key blocks. Query t (position qpos[t] or t), head h reads kv head
 * h / (n_head / n_head_kv); key j (position kpos[j] or j) is kept when
 * kp <= qp and, with window > 0, qp - kp < window; its score is
 * (sum_d q[d]*k[d]) * scale. Per block: m_new = max(m, block max), the running
 * sum and accumulator are scaled by exp(m - m_new) (0 while m is -inf), each
 * kept key adds p = exp(s - m_new) and p*v. out = acc / max(l, 1e-30).
 * Returns 0 for the reference's refusals. */
int cr_attention_tiled(const float* q, const float* k, const float* v, float* out, int64_t n_q,
                       int64_t n_head, int64_t n_head_kv, int64_t head_dim, int64_t value_dim,
                       float scale, const int32_t* qpos, const int32_t* kpos, int64_t n_kv,
                       int window, int64_t block) {
    if (n_q <= 0 || n_head <= 0 || n_head_kv <= 0 || head_dim <= 0 || value_dim <= 0 ||
        n_kv <= 0)
        return 0;
    if (n_head % n_head_kv) return 0;
    const int64_t rep = n_head / n_head_kv;
    if (block <= 0) block = n_kv;
    const int64_t rows = n_q * n_head;
    float* acc = (float*)calloc((size_t)(rows * value_dim), sizeof(float));
    float* l = (float*)calloc((size_t)rows, sizeof(float));
    float* m = (float*)malloc((size_t)rows * sizeof(float));
    float* sb = (float*)malloc((size_t)block * sizeof(float));
    if (!acc || !l || !m || !sb) {
        free(acc); free(l); free(m); free(sb);
        return 0;
    }
    for (int64_t i = 0; i < rows; ++i) m[i] = -INFINITY;
    for (int64_t b0 = 0; b0 < n_kv; b0 += block) {
        const int64_t b1 = (b0 + block < n_kv) ? b0 + block : n_kv;
        const int64_t nb = b1 - b0;
        for (int64_t t = 0; t < n_q; ++t) {
            const int64_t qp = qpos ? (int64_t)qpos[t] : t;
            for (int64_t h = 0; h < n_head; ++h) {
                const int64_t kh = h / rep;
                const float* qv = q + (t * n_head + h) * head_dim;
                float* a = acc + (t * n_head + h) * value_dim;
                float* lp = l + t * n_head + h;
                float* mp = m + t * n_head + h;
                float bmax = -INFINITY;
                for (int64_t j = 0; j < nb; ++j) {
                    const int64_t kp = kpos ? (int64_t)kpos[b0 + j] : b0 + j;
                    int keep = kp <= qp;
                    if (window > 0) keep = keep && (qp - kp) < window;
                    float sj = -INFINITY;
                    if (keep) {
                        const float* kj = k + ((b0 + j) * n_head_kv + kh) * head_dim;
                        float dot = 0.0f;
                        for (int64_t d = 0; d < head_dim; ++d) dot += qv[d] * kj[d];
                        sj = dot * scale;
                    }
                    sb[j] = sj;
                    bmax = cr_fmax_(bmax, sj);
                }
                const float m_new = cr_fmax_(*mp, bmax);
                const int finite_m = isfinite(*mp);
                const float m_safe = finite_m ? *mp : 0.0f;
                const float mn_safe = isfinite(m_new) ? m_new : 0.0f;
                const float alpha = finite_m ? expf(m_safe - mn_safe) : 0.0f;
                *lp *= alpha;
                for (int64_t d = 0; d < value_dim; ++d) a[d] *= alpha;
                float lsum = 0.0f;
                for (int64_t j = 0; j < nb; ++j) {
                    const float p = isfinite(sb[j]) ? expf(sb[j] - mn_safe) : 0.0f;
                    lsum += p;
                    const float* vj = v + ((b0 + j) * n_head_kv + kh) * value_dim;
                    for (int64_t d = 0; d < value_dim; ++d) a[d] += p * vj[d];
                }
                *lp += lsum;
                *mp = m_new;
            }
        }
    }
    for (int64_t i = 0; i < rows; ++i) {
        const float den = cr_fmax_(l[i], 1e-30f);
        for (int64_t d = 0; d < value_dim; ++d) out[i * value_dim + d] = acc[i * value_dim + d] / den;
    }
    free(acc); free(l); free(m); free(sb);
    return 1;
}

/* src/transformer.cpp:205-214: one query at position n_kv - 1 against keys
 * at positions 0..n_kv-1, one block. */
int cr_attention(const float* q, const float* k, const float* v, float* out, int64_t n_head,
                 int64_t n_head_kv, int64_t head_dim, int64_t value_dim, float scale,
                 int64_t n_kv, int window) {
    if (n_kv <= 0) return 0;
    const int32_t qp = (int32_t)(n_kv - 1);
    int32_t* kp = (int32_t*)malloc((size_t)n_kv * sizeof(int32_t));
    if (!kp) return 0;
    for (int64_t j = 0; j < n_kv; ++j) kp[j] = (int32_t)j;
    const int ok = cr_attention_tiled(q, k, v, out, 1, n_head, n_head_kv, head_dim, value_dim,
                                      scale, &qp, kp, n_kv, window, n_kv);
    free(kp);
    return ok;
}

/* ------------------------------------------------------- KV quantisers */
/* include/aero/kv.hpp:62-103: symmetric per-vector scale amax/127 (int8) or
 * amax/7 (int4), 1 when amax is 0; q = round(x / scale) clipped; int4 packs
 * two per byte, low nibble first, as (q & 15), sign-extended on unpack. */
void cr_kv_quant_i8(const float* x, int64_t dim, int8_t* q, float* s) {
    float amax = 0.0f;
    for (int64_t i = 0; i < dim; ++i) amax = cr_fmax_(amax, fabsf(x[i]));
    const float sc = amax > 0.0f ? amax / 127.0f : 1.0f;
    *s = sc;
    for (int64_t i = 0; i < dim; ++i) {
        float v = roundf(x[i] / sc);
        if (v > 127.0f) v = 127.0f;
        if (v < -127.0f) v = -127.0f;
        q[i] = (int8_t)v;
    }
}

void cr_kv_quant_i4(const float* x, int64_t dim, uint8_t* q, float* s) {
    float amax = 0.0f;
    for (int64_t i = 0; i < dim; ++i) amax = cr_fmax_(amax, fabsf(x[i]));
    const float sc = amax > 0.0f ? amax / 7.0f : 1.0f;
    *s = sc;
    for (int64_t i = 0; i < dim; i += 2) {
        float a = roundf(x[i] / sc), b = roundf(x[i + 1] / sc);
        if (a > 7.0f) a = 7.0f;
        if (a < -7.0f) a = -7.0f;
        if (b > 7.0f) b = 7.0f;
        if (b < -7.0f) b = -7.0f;
        q[i / 2] = (uint8_t)(((int)a & 0x0F) | (((int)b & 0x0F) << 4));
    }
}

/* src/kv.cpp:29-46: dequantise one vector (0 fp32 copy, 1 int8, 2 int4). */
int cr_kv_read_vec(int dt, const void* q, const float* scale, int64_t dim, float* out) {
    if (!q || !scale || !out || dim <= 0) return 0;
    if (dt == 0) {
        memcpy(out, q, (size_t)dim * sizeof(float));
    } else if (dt == 1) {
        const int8_t* v = (const int8_t*)q;
        for (int64_t i = 0; i < dim; ++i) out[i] = (float)v[i] * (*scale);
    } else if (dt == 2) {
        if (dim % 2) return 0;
        const uint8_t* b = (const uint8_t*)q;
        for (int64_t i = 0; i < dim; i += 2) {
            const int lo = b[i / 2] & 0x0F, hi = (b[i / 2] >> 4) & 0x0F;
            out[i] = (float)(lo >= 8 ? lo - 16 : lo) * (*scale);
            out[i + 1] = (float)(hi >= 8 ? hi - 16 : hi) * (*scale);
        }
    } else {
        return 0;
    }
    return 1;
}

/* src/kv.cpp:13-26: quantise one vector. */
int cr_kv_write_vec(int dt, const float* x, int64_t dim, void* q, float* scale) {
    if (!x || !q || !scale || dim <= 0) return 0;
    if (dt == 0) memcpy(q, x, (size_t)dim * sizeof(float));
    else if (dt == 1) cr_kv_quant_i8(x, dim, (int8_t*)q, scale);
    else if (dt == 2) {
        if (dim % 2) return 0;
        cr_kv_quant_i4(x, dim, (uint8_t*)q, scale);
    } else return 0;
    return 1;
}

/* ------------------------------------------------------ gated DeltaNet */
/* src/ssm.cpp:17-24: silu / sigmoid / softplus(x) = log1p(exp(-|x|)) +
 * max(x, 0). */
float cr_ssm_softplus(float x) {
    return log1pf(expf(-fabsf(x))) + (x > 0.0f ? x : 0.0f);
}

static float cr_sigmoid(float x) { return 1.0f / (1.0f + expf(-x)); }

/* src/ssm.cpp:28-34: x / max(||x||, eps), the sum of squares serial. */
static void cr_l2_row(const float* x, int64_t n, float eps, float* out) {
    float ss = 0.0f;
    for (int64_t i = 0; i < n; ++i) ss += x[i] * x[i];
    float nv = sqrtf(ss);
    if (nv < eps) nv = eps;
    for (int64_t i = 0; i < n; ++i) out[i] = x[i] / nv;
}

/* src/ssm.cpp:69-126: one token of the gated delta rule. v-head h reads
 * k-head h % n_k; g = a_log[h] * softplus(alpha[h] + dt_bias[h]) clamped to
 * <= 0, S *= exp(g), v_pred = kn^T S, v_new = (v - v_pred) * sigmoid(beta[h]),
 * S += kn v_new^T, out = scale * qn^T S. state [n_v][d][d] row-major (row i =
 * key element, column e = value element). */
void cr_ssm_delta_step_grouped(const float* q, const float* k, const float* v,
                               const float* alpha, const float* beta, const float* a_log,
                               const float* dt_bias, float* state, int64_t n_k, int64_t n_v,
                               int64_t d, float scale, float eps, float* out) {
    float* qn = (float*)malloc(sizeof(float) * (size_t)(n_v * d));
    float* kn = (float*)malloc(sizeof(float) * (size_t)(n_v * d));
    float* vpred = (float*)malloc(sizeof(float) * (size_t)d);
    float* vnew = (float*)malloc(sizeof(float) * (size_t)d);
    for (int64_t h = 0; h < n_v; ++h) {
        const int64_t kk = h % n_k;
        cr_l2_row(q + kk * d, d, eps, qn + h * d);
        cr_l2_row(k + kk * d, d, eps, kn + h * d);
    }
    for (int64_t h = 0; h < n_v; ++h) {
        float g = a_log[h] * cr_ssm_softplus(alpha[h] + dt_bias[h]);
        if (g > 0.0f) g = 0.0f;
        const float dec = expf(g);
        const float b = cr_sigmoid(beta[h]);
        float* S = state + h * d * d;
        const float* knh = kn + h * d;
        const float* qnh = qn + h * d;
        const float* vh = v + h * d;
        float* oh = out + h * d;
        for (int64_t i = 0; i < d * d; ++i) S[i] *= dec;
        for (int64_t e = 0; e < d; ++e) {
            float s = 0.0f;
            for (int64_t i = 0; i < d; ++i) s += knh[i] * S[i * d + e];
            vpred[e] = s;
        }
        for (int64_t e = 0; e < d; ++e) vnew[e] = (vh[e] - vpred[e]) * b;
        for (int64_t i = 0; i < d; ++i) {
            const float ki = knh[i];
            for (int64_t e = 0; e < d; ++e) S[i * d + e] += ki * vnew[e];
        }
        for (int64_t e = 0; e < d; ++e) {
            float s = 0.0f;
            for (int64_t i = 0; i < d; ++i) s += qnh[i] * S[i * d + e];
            oh[e] = scale * s;
        }
    }
    free(qn);
    free(kn);
    free(vpred);
    free(vnew);
}

/* src/ssm.cpp:128-142,163-171: T tokens; q, k [T][n_k][d], v [T][n_v][d],
 * alpha, beta [T][n_v], outs [T][n_v][d]. */
void cr_ssm_scan(const float* q, const float* k, const float* v, const float* alpha,
                 const float* beta, const float* a_log, const float* dt_bias, float* state,
                 int64_t T, int64_t n_k, int64_t n_v, int64_t d, float scale, float eps,
                 float* outs) {
    for (int64_t t = 0; t < T; ++t)
        cr_ssm_delta_step_grouped(q + t * n_k * d, k + t * n_k * d, v + t * n_v * d,
                                  alpha + t * n_v, beta + t * n_v, a_log, dt_bias, state, n_k,
                                  n_v, d, scale, eps, outs + t * n_v * d);
}

/* src/ssm.cpp:173-210: causal depthwise conv over [tail; x] (tail_len rows of
 * history), w [channels][kernel] with tap 0 on the oldest input; out [T][C];
 * the tail becomes the last min(kernel - 1, tail_len + T) rows. */
void cr_ssm_conv(const float* x, const float* w, float* tail, int* tail_len, float* out,
                 int64_t T, int64_t channels, int64_t kernel) {
    const int64_t tl = *tail_len;
    const int64_t n = tl + T;
    float* buf = (float*)malloc(sizeof(float) * (size_t)((n > 0 ? n : 1) * channels));
    if (tl > 0) memcpy(buf, tail, sizeof(float) * (size_t)(tl * channels));
    memcpy(buf + tl * channels, x, sizeof(float) * (size_t)(T * channels));
    for (int64_t t = 0; t < T; ++t) {
        const int64_t end = n - T + t + 1;
        const int64_t start = end - kernel;
        for (int64_t c = 0; c < channels; ++c) {
            float acc = 0.0f;
            for (int64_t j = 0; j < kernel; ++j) {
                const int64_t idx = start + j;
                if (idx >= 0 && idx < n) acc += buf[idx * channels + c] * w[c * kernel + j];
            }
            out[t * channels + c] = acc;
        }
    }
    int64_t keep = kernel - 1;
    if (keep < 0) keep = 0;
    if (keep > n) keep = n;
    if (keep > 0) memcpy(tail, buf + (n - keep) * channels, sizeof(float) * (size_t)(keep * channels));
    *tail_len = (int)keep;
    free(buf);
}
