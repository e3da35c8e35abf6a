/* oracle/cpuref_quant.c -- GGUF block dequant and embedding row gather.
 *
 * TEST INFRASTRUCTURE: the oracle of the HIP gather/dequant kernels and the
 * "port" CPU baseline. Built with -O2 -ffast-math -fno-math-errno -pthread as
 * the reference builds src/kernels.cpp (Makefile:29), plus -ffp-contract=off
 * so d*q and f*q - g round as separate IEEE operations.
 *
 * The block layouts are the GGML on-disk formats; they must be byte-for-byte
 * the same as the reference's because they are a file format.
 *
 * How each function is pinned (tests/test_oracle.py):
 *   cr_f16_to_f32   exhaustively, all 65536 half patterns against numpy's
 *                   IEEE float16 -> float32 conversion.
 *   Q8_0            tests/test_quant.py:127-131 (d = 0.5, q = 0..31);
 *                   compiled reference src/kernels.cpp (bit-exact).
 *   Q4_K            tests/test_quant.py:72-93 (output == nibbles) and the
 *                   make_q4k packer of tests/test_kernels.cpp:80-154 (sc 1..8,
 *                   mn 8..1, d/dmin in {0,1}); compiled reference (bit-exact).
 *   Q6_K            tests/test_quant.py:96-124 (all-zero -> -32, all-one ->
 *                   31, low-nibble pattern -> -17/-32); compiled reference.
 *   Q5_K, IQ4_XS    compiled reference (bit-exact) on random blocks; Q5_K
 *                   with qh = 0 equals Q4_K of the same bytes, with qh all
 *                   ones adds 16*(d*sc) to every value; IQ4_XS with one
 *                   nibble value per block reproduces the codebook times dl.
 *   cr_matvec,      the compiled reference's aero_matvec/aero_matmul (within
 *   cr_matmul       1e-6 of scale: its -ffast-math may reorder sums) and the
 *                   float64 product dequant(W) @ x; matmul rows == matvec
 *                   (tests/test_kernels.cpp:289-314).
 *   cr_embed_gather brute-force row selection on tiny tables; refusals of
 *                   src/model.cpp:297-316.
 */
#include "cpuref.h"

#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

/* Exact IEEE half -> single (src/kernels.cpp:29-52 states the same map with
 * bit surgery; here the value is rebuilt arithmetically, which is exact
 * because every half is a small integer times a power of two). */
float cr_f16_to_f32(uint16_t h) {
    const int sign = (h >> 15) & 1;
    const int e = (h >> 10) & 31;
    const int m = h & 1023;
    float v;
    if (e == 0) {
        v = ldexpf((float)m, -24);                 /* zero and subnormals */
    } else if (e == 31) {
        uint32_t bits = 0x7F800000u | ((uint32_t)m << 13);
        memcpy(&v, &bits, sizeof v);               /* inf / nan, payload kept */
    } else {
        v = ldexpf((float)(m | 1024), e - 25);
    }
    return sign ? -v : v;
}

void cr_f16_to_f32_n(const uint16_t* h, float* out, int64_t n) {
    for (int64_t i = 0; i < n; ++i) out[i] = cr_f16_to_f32(h[i]);
}

static float bf16_to_f32(uint16_t h) {
    const uint32_t bits = (uint32_t)h << 16;
    float v;
    memcpy(&v, &bits, sizeof v);
    return v;
}

static uint16_t rd16(const uint8_t* p) { return (uint16_t)(p[0] | (p[1] << 8)); }

/* src/kernels.cpp:286-313 (dtype_block_bytes / dtype_block_values) */
int64_t cr_block_bytes(int type) {
    switch (type) {
    case CR_F32: return 4;
    case CR_F16: case CR_BF16: return 2;
    case CR_Q8_0: return 34;
    case CR_Q4_K: return 144;
    case CR_Q5_K: return 176;
    case CR_Q6_K: return 210;
    case CR_IQ4_XS: return 136;
    default: return 0;
    }
}

int64_t cr_block_values(int type) {
    switch (type) {
    case CR_F32: case CR_F16: case CR_BF16: return 1;
    case CR_Q8_0: return 32;
    case CR_Q4_K: case CR_Q5_K: case CR_Q6_K: case CR_IQ4_XS: return 256;
    default: return 0;
    }
}

/* Q8_0, src/kernels.cpp:364-373: 34 bytes = fp16 d + 32 int8; y = d*q. */
static void deq_q8_0(const uint8_t* blk, float* o) {
    const float d = cr_f16_to_f32(rd16(blk));
    const int8_t* q = (const int8_t*)(blk + 2);
    for (int i = 0; i < 32; ++i) o[i] = d * (float)q[i];
}

/* The 6-bit (scale, min) pair of sub-block k in the 12-byte Q4_K scale
 * field (src/kernels.cpp:65-73). */
static void q4k_scale_min(int k, const uint8_t* s, int* sc, int* mn) {
    if (k < 4) {
        *sc = s[k] & 63;
        *mn = s[k + 4] & 63;
    } else {
        *sc = (s[k + 4] & 15) | ((s[k - 4] >> 6) << 4);
        *mn = (s[k + 4] >> 4) | ((s[k] >> 6) << 4);
    }
}

/* Q4_K, src/kernels.cpp:337-363: 144 bytes = d, dmin (fp16), 12 scale bytes,
 * 128 quant bytes. Group j covers values 64j..64j+63: the low nibbles of
 * qs[32j..32j+31] with sub-block 2j, then the high nibbles with 2j+1;
 * y = (d*sc)*q - (dmin*m). */
static void deq_q4_k(const uint8_t* blk, float* o) {
    const float d = cr_f16_to_f32(rd16(blk));
    const float dmin = cr_f16_to_f32(rd16(blk + 2));
    const uint8_t* sc = blk + 4;
    const uint8_t* qs = blk + 16;
    for (int j = 0; j < 4; ++j) {
        int s1, m1, s2, m2;
        q4k_scale_min(2 * j, sc, &s1, &m1);
        q4k_scale_min(2 * j + 1, sc, &s2, &m2);
        const float f1 = d * (float)s1, g1 = dmin * (float)m1;
        const float f2 = d * (float)s2, g2 = dmin * (float)m2;
        for (int i = 0; i < 32; ++i) {
            const uint8_t b = qs[32 * j + i];
            o[64 * j + i] = f1 * (float)(b & 15) - g1;
            o[64 * j + 32 + i] = f2 * (float)(b >> 4) - g2;
        }
    }
}

/* Q6_K, src/kernels.cpp:427-458: 210 bytes = ql[128], qh[64], int8 sc[16],
 * fp16 d at 208. Half h, l < 32: four 6-bit values from ql[64h+l],
 * ql[64h+l+32] (low then high nibbles) and 2-bit fields of qh[32h+l];
 * y[128h + l + 32k] = (d*sc[8h + l/16 + 2k]) * (q_k - 32). */
static void deq_q6_k(const uint8_t* blk, float* o) {
    const uint8_t* ql = blk;
    const uint8_t* qh = blk + 128;
    const int8_t* sc = (const int8_t*)(blk + 192);
    const float d = cr_f16_to_f32(rd16(blk + 208));
    for (int h = 0; h < 2; ++h) {
        for (int l = 0; l < 32; ++l) {
            const int lo = ql[64 * h + l];
            const int hi = ql[64 * h + l + 32];
            const int hb = qh[32 * h + l];
            const int q[4] = {
                (lo & 15) | ((hb & 3) << 4),
                (hi & 15) | (((hb >> 2) & 3) << 4),
                (lo >> 4) | (((hb >> 4) & 3) << 4),
                (hi >> 4) | (((hb >> 6) & 3) << 4),
            };
            for (int k = 0; k < 4; ++k)
                o[128 * h + l + 32 * k] =
                    d * (float)sc[8 * h + l / 16 + 2 * k] * (float)(q[k] - 32);
        }
    }
}

/* Q5_K, src/kernels.cpp:374-404: 176 bytes = d, dmin (fp16), 12 scale bytes
 * (the Q4_K 6-bit packing), qh[32], qs[128]. As Q4_K, plus a fifth bit: value
 * i of group j takes bit 2j (low nibbles) or 2j+1 (high nibbles) of qh[i];
 * y = (d*sc)*(nibble | bit<<4) - (dmin*m). */
static void deq_q5_k(const uint8_t* blk, float* o) {
    const float d = cr_f16_to_f32(rd16(blk));
    const float dmin = cr_f16_to_f32(rd16(blk + 2));
    const uint8_t* sc = blk + 4;
    const uint8_t* qh = blk + 16;
    const uint8_t* qs = blk + 48;
    for (int j = 0; j < 4; ++j) {
        int s1, m1, s2, m2;
        q4k_scale_min(2 * j, sc, &s1, &m1);
        q4k_scale_min(2 * j + 1, sc, &s2, &m2);
        const float f1 = d * (float)s1, g1 = dmin * (float)m1;
        const float f2 = d * (float)s2, g2 = dmin * (float)m2;
        for (int i = 0; i < 32; ++i) {
            const uint8_t b = qs[32 * j + i];
            const int h1 = (qh[i] >> (2 * j)) & 1;
            const int h2 = (qh[i] >> (2 * j + 1)) & 1;
            o[64 * j + i] = f1 * (float)((b & 15) | (h1 << 4)) - g1;
            o[64 * j + 32 + i] = f2 * (float)((b >> 4) | (h2 << 4)) - g2;
        }
    }
}

/* IQ4_XS codebook (src/kernels.cpp:212-215): the GGML IQ4_NL non-linear
 * 4-bit levels, a file-format constant. */
static const float kIq4nl[16] = {-127.f, -104.f, -83.f, -65.f, -49.f, -35.f, -22.f, -10.f,
                                 1.f,    13.f,   25.f,  38.f,  53.f,  69.f,  89.f,  113.f};

/* 6-bit scale of IQ4_XS sub-block ib: low 4 bits from scales_l (two per
 * byte), high 2 bits from the 16-bit scales_h (src/kernels.cpp:405-425). */
static int iq4xs_scale(const uint8_t* blk, int ib) {
    const unsigned sh = (unsigned)rd16(blk + 2);
    const uint8_t* sl = blk + 4;
    return ((sl[ib >> 1] >> (4 * (ib & 1))) & 15) | (int)(((sh >> (2 * ib)) & 3u) << 4);
}

/* IQ4_XS: 136 bytes = fp16 d, scales_h (2), scales_l (4), qs[128]. Sub-block
 * ib of 32 values: dl = d*(ls-32); values j < 16 are the low nibbles of
 * qs[16ib + j], values 16..31 the high nibbles; y = dl*codebook[nibble]. */
static void deq_iq4_xs(const uint8_t* blk, float* o) {
    const float d = cr_f16_to_f32(rd16(blk));
    const uint8_t* qs = blk + 8;
    for (int ib = 0; ib < 8; ++ib) {
        const float dl = d * (float)(iq4xs_scale(blk, ib) - 32);
        const uint8_t* q = qs + 16 * ib;
        for (int j = 0; j < 16; ++j) {
            o[32 * ib + j] = dl * kIq4nl[q[j] & 15];
            o[32 * ib + 16 + j] = dl * kIq4nl[q[j] >> 4];
        }
    }
}

static int deq_blocks(int type, const uint8_t* raw, float* out, int64_t b0,
                      int64_t b1) {
    const int64_t bb = cr_block_bytes(type), bv = cr_block_values(type);
    for (int64_t b = b0; b < b1; ++b) {
        const uint8_t* blk = raw + b * bb;
        float* o = out + b * bv;
        switch (type) {
        case CR_Q8_0: deq_q8_0(blk, o); break;
        case CR_Q4_K: deq_q4_k(blk, o); break;
        case CR_Q6_K: deq_q6_k(blk, o); break;
        case CR_Q5_K: deq_q5_k(blk, o); break;
        case CR_IQ4_XS: deq_iq4_xs(blk, o); break;
        case CR_F16: o[0] = cr_f16_to_f32(rd16(blk)); break;
        case CR_BF16: o[0] = bf16_to_f32(rd16(blk)); break;
        case CR_F32: memcpy(o, blk, 4); break;
        default: return 0;
        }
    }
    return 1;
}

static int is_block_quant(int type) {
    return type == CR_Q8_0 || type == CR_Q4_K || type == CR_Q5_K || type == CR_Q6_K ||
           type == CR_IQ4_XS;
}

static int supported(int type) {
    return type == CR_F32 || type == CR_F16 || type == CR_BF16 || is_block_quant(type);
}

/* dequant_ref, src/kernels.cpp:315-323: refuse a short buffer, then
 * dequantise floor(n/bv) whole blocks. */
int cr_dequant(int type, const uint8_t* raw, int64_t raw_len, float* out,
               int64_t n_values) {
    if (!supported(type) || raw == NULL || out == NULL) return 0;
    const int64_t bb = cr_block_bytes(type), bv = cr_block_values(type);
    if (raw_len < (n_values / bv) * bb) return 0;
    return deq_blocks(type, raw, out, 0, n_values / bv);
}

/* dequant_threaded, src/kernels.cpp:463-494 with parallel_for :253-268:
 * block b goes to thread b % t. Used as the threaded CPU-baseline row. */
struct deq_job {
    int type, k, t;
    const uint8_t* raw;
    float* out;
    int64_t nblocks;
};

static void* deq_worker(void* arg) {
    const struct deq_job* j = (const struct deq_job*)arg;
    for (int64_t b = j->k; b < j->nblocks; b += j->t)
        deq_blocks(j->type, j->raw, j->out, b, b + 1);
    return NULL;
}

int cr_dequant_threaded(int type, const uint8_t* raw, int64_t raw_len,
                        float* out, int64_t n_values, int threads) {
    if (!supported(type) || raw == NULL || out == NULL) return 0;
    const int64_t bb = cr_block_bytes(type), bv = cr_block_values(type);
    if (raw_len < (n_values / bv) * bb) return 0;
    const int64_t nb = n_values / bv;
    if (threads <= 1 || nb <= 1 || type == CR_F32)
        return deq_blocks(type, raw, out, 0, nb);
    const int t = (int)(threads < nb ? threads : nb);
    pthread_t th[64];
    struct deq_job jobs[64];
    const int tt = t > 64 ? 64 : t;
    for (int k = 0; k < tt; ++k) {
        jobs[k] = (struct deq_job){type, k, tt, raw, out, nb};
        pthread_create(&th[k], NULL, deq_worker, &jobs[k]);
    }
    for (int k = 0; k < tt; ++k) pthread_join(th[k], NULL);
    return 1;
}

/* Token-embedding gather, src/model.cpp:297-316: row bytes
 * rb = (n_embd/bv)*bb; refuse n_embd % bv and out-of-range ids; dequantise
 * each requested row; then, when scale > 0, multiply every value by scale in
 * a second pass (the reference's x *= embed_scale). */
int cr_embed_gather(int type, const uint8_t* table, int64_t vocab,
                    int64_t n_embd, const int32_t* ids, int64_t n_ids,
                    float scale, float* out) {
    const int64_t bb = cr_block_bytes(type), bv = cr_block_values(type);
    if (!supported(type) || bv <= 0 || n_embd % bv != 0) return 0;
    const int64_t rb = (n_embd / bv) * bb;
    for (int64_t i = 0; i < n_ids; ++i) {
        const int64_t tok = ids[i];
        if (tok < 0 || tok >= vocab) return 0;
        if (!cr_dequant(type, table + tok * rb, rb, out + i * n_embd, n_embd))
            return 0;
    }
    if (scale > 0.0f)
        for (int64_t i = 0; i < n_ids * n_embd; ++i) out[i] *= scale;
    return 1;
}

/* ------------------------------------------------------------ block dots
 * One block of a quantised weight row dotted with the matching x values,
 * in the reference's accumulation order (src/kernels.cpp:78-250). */

/* src/kernels.cpp:78-84: d * sum(q*x). */
static float dot_q8_0(const uint8_t* blk, const float* x) {
    const float d = cr_f16_to_f32(rd16(blk));
    const int8_t* q = (const int8_t*)(blk + 2);
    float acc = 0.0f;
    for (int i = 0; i < 32; ++i) acc += (float)q[i] * x[i];
    return d * acc;
}

/* Q4_K (src/kernels.cpp:123-156) and Q5_K (:90-121, fifth bit from qh):
 * per group j, qx = sum(q*x) and sx = sum(x) over each 32-value half;
 * acc += (d*sc)*qx - (dmin*m)*sx. */
static float dot_q45_k(const uint8_t* blk, const float* x, int five) {
    const float d = cr_f16_to_f32(rd16(blk));
    const float dmin = cr_f16_to_f32(rd16(blk + 2));
    const uint8_t* sc = blk + 4;
    const uint8_t* qh = blk + 16;
    const uint8_t* qs = blk + (five ? 48 : 16);
    float acc = 0.0f;
    for (int j = 0; j < 4; ++j) {
        int s1, m1, s2, m2;
        q4k_scale_min(2 * j, sc, &s1, &m1);
        q4k_scale_min(2 * j + 1, sc, &s2, &m2);
        float qx1 = 0.0f, sx1 = 0.0f, qx2 = 0.0f, sx2 = 0.0f;
        for (int i = 0; i < 32; ++i) {
            const uint8_t b = qs[32 * j + i];
            const float xlo = x[64 * j + i], xhi = x[64 * j + 32 + i];
            const int h1 = five ? (qh[i] >> (2 * j)) & 1 : 0;
            const int h2 = five ? (qh[i] >> (2 * j + 1)) & 1 : 0;
            qx1 += (float)((b & 15) | (h1 << 4)) * xlo;
            sx1 += xlo;
            qx2 += (float)((b >> 4) | (h2 << 4)) * xhi;
            sx2 += xhi;
        }
        acc += (d * (float)s1) * qx1 - (dmin * (float)m1) * sx1;
        acc += (d * (float)s2) * qx2 - (dmin * (float)m2) * sx2;
    }
    return acc;
}

/* src/kernels.cpp:170-200: acc += d*sc*(q-32)*x, four values per (h, l). */
static float dot_q6_k(const uint8_t* blk, const float* x) {
    const uint8_t* ql = blk;
    const uint8_t* qh = blk + 128;
    const int8_t* sc = (const int8_t*)(blk + 192);
    const float d = cr_f16_to_f32(rd16(blk + 208));
    float acc = 0.0f;
    for (int h = 0; h < 2; ++h) {
        for (int l = 0; l < 32; ++l) {
            const int lo = ql[64 * h + l], hi = ql[64 * h + l + 32], hb = qh[32 * h + l];
            const int is = l >> 4;
            const float v0 = (float)(((lo & 15) | ((hb & 3) << 4)) - 32);
            const float v1 = (float)(((hi & 15) | (((hb >> 2) & 3) << 4)) - 32);
            const float v2 = (float)(((lo >> 4) | (((hb >> 4) & 3) << 4)) - 32);
            const float v3 = (float)(((hi >> 4) | (((hb >> 6) & 3) << 4)) - 32);
            const float* xb = x + 128 * h + l;
            acc += d * (float)sc[8 * h + is] * v0 * xb[0];
            acc += d * (float)sc[8 * h + is + 2] * v1 * xb[32];
            acc += d * (float)sc[8 * h + is + 4] * v2 * xb[64];
            acc += d * (float)sc[8 * h + is + 6] * v3 * xb[96];
        }
    }
    return acc;
}

/* src/kernels.cpp:217-238: per sub-block, dl * sum(codebook[q]*x). */
static float dot_iq4_xs(const uint8_t* blk, const float* x) {
    const float d = cr_f16_to_f32(rd16(blk));
    const uint8_t* qs = blk + 8;
    float acc = 0.0f;
    for (int ib = 0; ib < 8; ++ib) {
        const float dl = d * (float)(iq4xs_scale(blk, ib) - 32);
        const uint8_t* q = qs + 16 * ib;
        const float* xb = x + 32 * ib;
        float sub = 0.0f;
        for (int j = 0; j < 16; ++j) {
            sub += kIq4nl[q[j] & 15] * xb[j];
            sub += kIq4nl[q[j] >> 4] * xb[j + 16];
        }
        acc += dl * sub;
    }
    return acc;
}

static float block_dot(int type, const uint8_t* blk, const float* x) {
    switch (type) {
    case CR_Q8_0: return dot_q8_0(blk, x);
    case CR_Q4_K: return dot_q45_k(blk, x, 0);
    case CR_Q5_K: return dot_q45_k(blk, x, 1);
    case CR_Q6_K: return dot_q6_k(blk, x);
    case CR_IQ4_XS: return dot_iq4_xs(blk, x);
    default: return 0.0f;
    }
}

/* matvec, src/kernels.cpp:497-515: y[r] = sum over blocks in order of the
 * block dot of row r; refuses non-quantised types and n_cols % bv. */
int cr_matvec(int type, const uint8_t* w, const float* x, float* y, int64_t n_rows,
              int64_t n_cols) {
    if (!is_block_quant(type) || w == NULL || x == NULL || y == NULL) return 0;
    const int64_t bv = cr_block_values(type), bb = cr_block_bytes(type);
    if (n_cols % bv != 0) return 0;
    const int64_t rb = (n_cols / bv) * bb;
    for (int64_t r = 0; r < n_rows; ++r) {
        float acc = 0.0f;
        for (int64_t c = 0; c < n_cols; c += bv) acc += block_dot(type, w + r * rb + (c / bv) * bb, x + c);
        y[r] = acc;
    }
    return 1;
}

/* matmul, src/kernels.cpp:517-538: Y[t, r] = matvec of token t. */
int cr_matmul(int type, const uint8_t* w, const float* X, float* Y, int64_t n_tok,
              int64_t n_rows, int64_t n_cols) {
    if (!is_block_quant(type) || X == NULL || Y == NULL) return 0;
    float* tmp = (float*)malloc((size_t)(n_rows > 0 ? n_rows : 1) * sizeof(float));
    if (tmp == NULL) return 0;
    int ok = 1;
    for (int64_t t = 0; t < n_tok && ok; ++t) {
        ok = cr_matvec(type, w, X + t * n_cols, tmp, n_rows, n_cols);
        for (int64_t r = 0; ok && r < n_rows; ++r) Y[t * n_rows + r] = tmp[r];
    }
    free(tmp);
    return ok;
}
