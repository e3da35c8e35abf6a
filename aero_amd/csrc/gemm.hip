// Quantised GEMM for many tokens on gfx950 (prefill): y[t, r] = sum_c W[r, c] * x[t, c]
// with W in GGML blocks and x, y fp32 — the reference's matmul
// (src/kernels.cpp:520-538) for token counts where re-reading W for every few
// tokens (the GEMV kernels) would dominate.
//
// A workgroup (4 waves) computes a BM-row x BN-token tile of y. For each
// BK-column chunk of the rows it dequantises its BM rows into LDS as fp32 —
// the reference's dequantised values bit for bit (the arithmetic of
// quant_blocks.hpp) — and stages the BN tokens' x, then each wave runs fp32
// matrix FMAs (v_mfma_f32_16x16x4_f32) over a (BM/2) x (BN/2) sub-tile: exact
// products, fp32 accumulation, so results differ from the reference's serial
// dots only in summation order. The next chunk's weights and x are loaded
// before the current chunk's matrix steps run.
//
// Weight staging: with W 16-byte aligned and rows a multiple of 16 bytes (8
// for IQ4_XS) a thread dequantises one 32-value sub-block per chunk from
// 16-byte loads (2-byte aligned Q8_0 / Q6_K blocks are shifted into place
// with byte permutes); otherwise four values at a time from 2- and 4-byte
// loads.
//
// LDS tiles hold element (i, k) of a chunk at i*(BK+4) + (k%4)*(BK/4) + k/4:
// a lane's operands for four consecutive matrix steps (k = 4s + lane/16) are
// one 16-byte read, and the 4-float row pad puts the 16 rows a read touches
// in 16 different bank groups.
//
// HBM bytes per launch: W once per BN-token tile, x once per BM-row tile
// (mostly from L2), y once.
#include "quant_blocks.hpp"

#pragma clang fp contract(off)

namespace aero {

namespace {

struct GemmParams {
    const uint8_t* w;  // n_rows rows of rb bytes
    const float* x;    // n_tok rows of x_stride floats
    float* y;          // n_tok rows of y_stride floats
    int64_t n_rows;
    int n_cols;
    int64_t rb;
    int n_tok;
    int64_t x_stride, y_stride;
};

// ------------------------------------------------- 32-value sub-blocks
// Values c0 .. c0+31 of a row (c0 a multiple of 32), loaded with wide loads
// (load) and dequantised (decode) with the reference's arithmetic.
template <int TYPE> struct Sub32;

// Q4_K (src/kernels.cpp:65-73,337-363): sub-block k = nibble k%2 of qs
// bytes 32(k/2) .. +31; y = (d*sc)*q - (dmin*m).
template <> struct Sub32<AERO_DTYPE_Q4_K> {
    uint4 hd, q[2];
    int k;
    __device__ __forceinline__ void load(const uint8_t* rowp, int c0) {
        const uint8_t* b = rowp + (int64_t)(c0 >> 8) * 144;
        k = (c0 & 255) >> 5;
        hd = ld128(b);
        q[0] = ld128(b + 16 + 32 * (k >> 1));
        q[1] = ld128(b + 32 + 32 * (k >> 1));
    }
    __device__ __forceinline__ void decode(float (&v)[32]) const {
        uint32_t sc, mn;
        kq_scale_min(hd.y, hd.z, hd.w, k, sc, mn);
        const float f = half_bits_to_float(hd.x & 0xFFFFu) * (float)sc;
        const float g = half_bits_to_float(hd.x >> 16) * (float)mn;
        const int sh = (k & 1) ? 4 : 0;
#pragma unroll
        for (int m = 0; m < 8; ++m) {
            const uint32_t w = wd(q, m) >> sh;
#pragma unroll
            for (int e = 0; e < 4; ++e) v[4 * m + e] = f * (float)((w >> (8 * e)) & 15u) - g;
        }
    }
};

// Q5_K (src/kernels.cpp:374-404): Q4_K plus bit k of qh[i] as bit 4.
template <> struct Sub32<AERO_DTYPE_Q5_K> {
    uint4 hd, h[2], q[2];
    int k;
    __device__ __forceinline__ void load(const uint8_t* rowp, int c0) {
        const uint8_t* b = rowp + (int64_t)(c0 >> 8) * 176;
        k = (c0 & 255) >> 5;
        hd = ld128(b);
        h[0] = ld128(b + 16);
        h[1] = ld128(b + 32);
        q[0] = ld128(b + 48 + 32 * (k >> 1));
        q[1] = ld128(b + 64 + 32 * (k >> 1));
    }
    __device__ __forceinline__ void decode(float (&v)[32]) const {
        uint32_t sc, mn;
        kq_scale_min(hd.y, hd.z, hd.w, k, sc, mn);
        const float f = half_bits_to_float(hd.x & 0xFFFFu) * (float)sc;
        const float g = half_bits_to_float(hd.x >> 16) * (float)mn;
        const int sh = (k & 1) ? 4 : 0;
#pragma unroll
        for (int m = 0; m < 8; ++m) {
            const uint32_t w = wd(q, m) >> sh, hb = wd(h, m) >> k;
#pragma unroll
            for (int e = 0; e < 4; ++e)
                v[4 * m + e] =
                    f * (float)(((w >> (8 * e)) & 15u) | (((hb >> (8 * e)) & 1u) << 4)) - g;
        }
    }
};

// Q8_0 (src/kernels.cpp:364-373): one block, 34 bytes at a 2-byte aligned
// offset, from the 48 aligned bytes around it; y = d*q.
template <> struct Sub32<AERO_DTYPE_Q8_0> {
    uint4 c[3];
    uint32_t ph;
    __device__ __forceinline__ void load(const uint8_t* rowp, int c0) {
        const uint32_t ob = (uint32_t)(c0 >> 5) * 34u;
        ph = ob & 15u;
        const uint8_t* b = rowp + (ob - ph);
#pragma unroll
        for (int i = 0; i < 3; ++i) c[i] = ld128(b + 16 * i);
    }
    __device__ __forceinline__ void decode(float (&v)[32]) const {
        uint32_t w[9];
        shifted_words<9, 3>(c, ph, w);
        const float d = half_bits_to_float(w[0] & 0xFFFFu);
#pragma unroll
        for (int m = 0; m < 8; ++m) {
            const uint32_t q = __builtin_amdgcn_alignbyte(w[m + 1], w[m], 2);
#pragma unroll
            for (int e = 0; e < 4; ++e) v[4 * m + e] = d * (float)(int8_t)((q >> (8 * e)) & 0xFFu);
        }
    }
};

// Q6_K (src/kernels.cpp:427-458): quarter kq of half h: nibble kq/2 of
// ql[64h + 32(kq%2) + i], bits 2kq of qh[32h + i]; scale sc[8h + 2kq + i/16];
// y = (d*sc)*(q-32). ql and qh from the 48 aligned bytes around each.
template <> struct Sub32<AERO_DTYPE_Q6_K> {
    uint4 l3[3], h3[3];
    uint32_t ph, sc, d;
    int kq;
    __device__ __forceinline__ void load(const uint8_t* rowp, int c0) {
        const uint32_t ob = (uint32_t)(c0 >> 8) * 210u;
        const int h = (c0 >> 7) & 1;
        kq = (c0 >> 5) & 3;
        ph = ob & 15u;
        const uint8_t* b = rowp + (ob - ph);
#pragma unroll
        for (int i = 0; i < 3; ++i) {
            l3[i] = ld128(b + 64 * h + 32 * (kq & 1) + 16 * i);
            h3[i] = ld128(b + 128 + 32 * h + 16 * i);
        }
        sc = ld_u16(rowp + ob + 192 + 8 * h + 2 * kq);
        d = ld_u16(rowp + ob + 208);
    }
    __device__ __forceinline__ void decode(float (&v)[32]) const {
        uint32_t wl[8], wh[8];
        shifted_words<8, 3>(l3, ph, wl);
        shifted_words<8, 3>(h3, ph, wh);
        const float df = half_bits_to_float(d);
        const float f0 = df * (float)(int8_t)(sc & 0xFFu);
        const float f1 = df * (float)(int8_t)((sc >> 8) & 0xFFu);
        const int sl = kq >= 2 ? 4 : 0, shh = 2 * kq;
#pragma unroll
        for (int m = 0; m < 8; ++m) {
            const uint32_t lb = wl[m] >> sl, hb = wh[m] >> shh;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int q = (int)(((lb >> (8 * e)) & 15u) | (((hb >> (8 * e)) & 3u) << 4));
                v[4 * m + e] = (m < 4 ? f0 : f1) * (float)(q - 32);
            }
        }
    }
};

// IQ4_XS (src/kernels.cpp:405-425): sub-block ib: values 0..15 from the low
// nibbles of qs[16ib ..], 16..31 from the high; y = d*(ls-32)*codebook[q].
template <> struct Sub32<AERO_DTYPE_IQ4_XS> {
    uint2 hd, q[2];
    int ib;
    __device__ __forceinline__ void load(const uint8_t* rowp, int c0) {
        const uint8_t* b = rowp + (int64_t)(c0 >> 8) * 136;
        ib = (c0 & 255) >> 5;
        hd = *reinterpret_cast<const uint2*>(b);
        q[0] = *reinterpret_cast<const uint2*>(b + 8 + 16 * ib);
        q[1] = *reinterpret_cast<const uint2*>(b + 16 + 16 * ib);
    }
    __device__ __forceinline__ void decode(float (&v)[32]) const {
        const float d = half_bits_to_float(hd.x & 0xFFFFu);
        const uint32_t sh = hd.x >> 16;
        const uint32_t ls = ((byte_of(hd.y, ib >> 1) >> (4 * (ib & 1))) & 15u) |
                            (((sh >> (2 * ib)) & 3u) << 4);
        const float dl = d * (float)((int)ls - 32);
#pragma unroll
        for (int m = 0; m < 4; ++m) {
            const uint32_t w = (m & 1) ? q[m >> 1].y : q[m >> 1].x;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                v[4 * m + e] = dl * iq4_level((w >> (8 * e)) & 15u);
                v[16 + 4 * m + e] = dl * iq4_level((w >> (8 * e + 4)) & 15u);
            }
        }
    }
};

// ------------------------------------------------------ weight staging
// FAST: one 32-value sub-block per unit from wide loads (W 16-byte aligned,
// rows a multiple of 16 bytes, 8 for IQ4_XS). Otherwise 16 values per unit,
// four at a time with load_raw / decode.
template <int TYPE, bool FAST, int BM, int BK> struct StageW;

template <int TYPE, int BM, int BK>
struct StageW<TYPE, true, BM, BK> {
    static constexpr int GR = BK / 32;       // sub-blocks per row chunk
    static constexpr int U = BM * GR / 256;  // units per thread
    static_assert(U >= 1 && BM * GR % 256 == 0, "tile");
    Sub32<TYPE> s[U];
    const uint8_t* rowp[U];
    int grp;
    bool valid;
    __device__ __forceinline__ void init(const GemmParams& p, int64_t r0, int tid) {
        grp = tid % GR;
#pragma unroll
        for (int u = 0; u < U; ++u)
            rowp[u] = p.w + min(r0 + (tid + 256 * u) / GR, p.n_rows - 1) * p.rb;
    }
    __device__ __forceinline__ void load(const GemmParams& p, int kc) {
        const int c = kc * BK + 32 * grp;
        valid = c < p.n_cols;  // n_cols is a multiple of 32
        const int cc = min(c, p.n_cols - 32);
#pragma unroll
        for (int u = 0; u < U; ++u) s[u].load(rowp[u], cc);
    }
    __device__ __forceinline__ void store(float* As, int tid) const {
        constexpr int RowF = BK + 4;
        const float4 z = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
        for (int u = 0; u < U; ++u) {
            float v[32];
            s[u].decode(v);
            float* row = As + ((tid + 256 * u) / GR) * RowF + 8 * grp;
#pragma unroll
            for (int kk = 0; kk < 4; ++kk) {
                // past n_cols (the last chunk of a Q8_0 row whose length is
                // not a multiple of 128): zeros, replacing the values of the
                // clamped block (a multiply by zero would keep inf / nan)
                float4 a = make_float4(v[kk], v[kk + 4], v[kk + 8], v[kk + 12]);
                float4 b = make_float4(v[kk + 16], v[kk + 20], v[kk + 24], v[kk + 28]);
                if (!valid) a = b = z;
                *reinterpret_cast<float4*>(row + kk * (BK / 4)) = a;
                *reinterpret_cast<float4*>(row + kk * (BK / 4) + 4) = b;
            }
        }
    }
};

template <int TYPE, int BM, int BK>
struct StageW<TYPE, false, BM, BK> {
    static constexpr int GR = BK / 16;  // 16-value groups per row chunk
    static constexpr int U = BM * GR / 256;
    static_assert(U >= 1 && BM * GR % 256 == 0, "tile");
    using Raw = typename QT<TYPE>::Raw;
    Raw raw[U][4];
    const uint8_t* rowp[U];
    int grp, cc;
    bool valid;
    __device__ __forceinline__ void init(const GemmParams& p, int64_t r0, int tid) {
        grp = tid % GR;
#pragma unroll
        for (int u = 0; u < U; ++u)
            rowp[u] = p.w + min(r0 + (tid + 256 * u) / GR, p.n_rows - 1) * p.rb;
    }
    __device__ __forceinline__ void load(const GemmParams& p, int kc) {
        const int c = kc * BK + 16 * grp;
        valid = c < p.n_cols;
        cc = min(c, p.n_cols - 16);
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const int cq = cc + 4 * q;
#pragma unroll
            for (int u = 0; u < U; ++u)
                load_raw(rowp[u] + (int64_t)(cq / QT<TYPE>::BV) * QT<TYPE>::BB,
                         (cq % QT<TYPE>::BV) / 4, raw[u][q]);
        }
    }
    __device__ __forceinline__ void store(float* As, int tid) const {
        constexpr int RowF = BK + 4;
        const float4 z = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
        for (int u = 0; u < U; ++u) {
            float4 w4[4];
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const float4 dq = decode(raw[u][q], ((cc + 4 * q) % QT<TYPE>::BV) / 4);
                w4[q] = valid ? dq : z;  // decode unconditional: a select, not a branch
            }
            float* row = As + ((tid + 256 * u) / GR) * RowF + 4 * grp;
            *reinterpret_cast<float4*>(row + 0 * BK / 4) = make_float4(w4[0].x, w4[1].x, w4[2].x, w4[3].x);
            *reinterpret_cast<float4*>(row + 1 * BK / 4) = make_float4(w4[0].y, w4[1].y, w4[2].y, w4[3].y);
            *reinterpret_cast<float4*>(row + 2 * BK / 4) = make_float4(w4[0].z, w4[1].z, w4[2].z, w4[3].z);
            *reinterpret_cast<float4*>(row + 3 * BK / 4) = make_float4(w4[0].w, w4[1].w, w4[2].w, w4[3].w);
        }
    }
};

// x staging: 16 consecutive floats of a token per unit.
template <int BN, int BK>
struct StageX {
    static constexpr int GR = BK / 16;
    static constexpr int U = BN * GR / 256;
    static_assert(U >= 1 && BN * GR % 256 == 0, "tile");
    float4 v[U][4];
    const float* xrow[U];
    int grp;
    bool valid;
    __device__ __forceinline__ void init(const GemmParams& p, int t0, int tid) {
        grp = tid % GR;
#pragma unroll
        for (int u = 0; u < U; ++u)
            xrow[u] = p.x + (int64_t)min(t0 + (tid + 256 * u) / GR, p.n_tok - 1) * p.x_stride;
    }
    __device__ __forceinline__ void load(const GemmParams& p, int kc) {
        const int c = kc * BK + 16 * grp;
        valid = c < p.n_cols;
        const int cc = min(c, p.n_cols - 16);
#pragma unroll
        for (int u = 0; u < U; ++u)
#pragma unroll
            for (int q = 0; q < 4; ++q)
                v[u][q] = *reinterpret_cast<const float4*>(xrow[u] + cc + 4 * q);
    }
    __device__ __forceinline__ void store(float* Bs, int tid) const {
        constexpr int RowF = BK + 4;
        const float4 z = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
        for (int u = 0; u < U; ++u) {
            float4 x4[4];
#pragma unroll
            for (int q = 0; q < 4; ++q) x4[q] = valid ? v[u][q] : z;
            float* row = Bs + ((tid + 256 * u) / GR) * RowF + 4 * grp;
            *reinterpret_cast<float4*>(row + 0 * BK / 4) = make_float4(x4[0].x, x4[1].x, x4[2].x, x4[3].x);
            *reinterpret_cast<float4*>(row + 1 * BK / 4) = make_float4(x4[0].y, x4[1].y, x4[2].y, x4[3].y);
            *reinterpret_cast<float4*>(row + 2 * BK / 4) = make_float4(x4[0].z, x4[1].z, x4[2].z, x4[3].z);
            *reinterpret_cast<float4*>(row + 3 * BK / 4) = make_float4(x4[0].w, x4[1].w, x4[2].w, x4[3].w);
        }
    }
};

// ---------------------------------------------------------------- kernel
// 4 waves in a 2 x 2 grid, each owning (BM/2) x (BN/2) as 16 x 16 tiles.
template <int TYPE, bool FAST, int BM, int BN, int BK>
__global__ __launch_bounds__(256) void gemm_kernel(GemmParams p) {
    constexpr int RowF = BK + 4;               // floats per padded LDS tile row
    constexpr int MI = BM / 32, NI = BN / 32;  // matrix tiles per wave
    __shared__ __align__(16) float As[BM * RowF];
    __shared__ __align__(16) float Bs[BN * RowF];

    const int tid = threadIdx.x;
    const int l = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave & 1, wn = wave >> 1;
    const int64_t r0 = (int64_t)blockIdx.x * BM;
    const int t0 = blockIdx.y * BN;
    const int n_k = (p.n_cols + BK - 1) / BK;

    v4f acc[MI][NI];
#pragma unroll
    for (int i = 0; i < MI; ++i)
#pragma unroll
        for (int j = 0; j < NI; ++j) acc[i][j] = v4f{0.f, 0.f, 0.f, 0.f};

    StageW<TYPE, FAST, BM, BK> sw;
    StageX<BN, BK> sx;
    sw.init(p, r0, tid);
    sx.init(p, t0, tid);

    sx.load(p, 0);
    sw.load(p, 0);
    sw.store(As, tid);
    sx.store(Bs, tid);
    __syncthreads();
    const float* ap = As + ((BM / 2) * wm + (l & 15)) * RowF + (l >> 4) * (BK / 4);
    const float* bp = Bs + ((BN / 2) * wn + (l & 15)) * RowF + (l >> 4) * (BK / 4);
    for (int kc = 0; kc < n_k; ++kc) {
        // the next chunk's loads go out before this chunk's matrix steps
        const int kn = min(kc + 1, n_k - 1);
        sx.load(p, kn);
        sw.load(p, kn);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int sg = 0; sg < BK / 16; ++sg) {
            float4 a[MI], b[NI];
#pragma unroll
            for (int i = 0; i < MI; ++i)
                a[i] = *reinterpret_cast<const float4*>(ap + 16 * i * RowF + 4 * sg);
#pragma unroll
            for (int j = 0; j < NI; ++j)
                b[j] = *reinterpret_cast<const float4*>(bp + 16 * j * RowF + 4 * sg);
#pragma unroll
            for (int e = 0; e < 4; ++e)
#pragma unroll
                for (int i = 0; i < MI; ++i)
#pragma unroll
                    for (int j = 0; j < NI; ++j)
                        acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[i][e], b[j][e],
                                                                         acc[i][j], 0, 0, 0);
        }
        if (kc + 1 >= n_k) break;
        __syncthreads();  // every wave is done reading this chunk
        sw.store(As, tid);
        sx.store(Bs, tid);
        __syncthreads();
    }

    // acc[i][j] holds rows 4(l/16)+v, token l%16 of matrix tile (i, j)
#pragma unroll
    for (int i = 0; i < MI; ++i)
#pragma unroll
        for (int j = 0; j < NI; ++j) {
            const int64_t row = r0 + (BM / 2) * wm + 16 * i + 4 * (l >> 4);
            const int tok = t0 + (BN / 2) * wn + 16 * j + (l & 15);
            if (tok < p.n_tok) {
                float* yp = p.y + (int64_t)tok * p.y_stride;
#pragma unroll
                for (int v = 0; v < 4; ++v)
                    if (row + v < p.n_rows) yp[row + v] = acc[i][j][v];
            }
        }
}

using GemmKernel = void (*)(GemmParams);

template <bool FAST>
GemmKernel pick_gemm(int dtype) {
    constexpr int BM = 64, BN = 64, BK = 128;
    switch (dtype) {
    case AERO_DTYPE_Q8_0: return gemm_kernel<AERO_DTYPE_Q8_0, FAST, BM, BN, BK>;
    case AERO_DTYPE_Q4_K: return gemm_kernel<AERO_DTYPE_Q4_K, FAST, BM, BN, BK>;
    case AERO_DTYPE_Q5_K: return gemm_kernel<AERO_DTYPE_Q5_K, FAST, BM, BN, BK>;
    case AERO_DTYPE_Q6_K: return gemm_kernel<AERO_DTYPE_Q6_K, FAST, BM, BN, BK>;
    case AERO_DTYPE_IQ4_XS: return gemm_kernel<AERO_DTYPE_IQ4_XS, FAST, BM, BN, BK>;
    default: return nullptr;
    }
}

}  // namespace

// Called by gemv_dev after its argument checks (W's size and 4-byte
// alignment, x 16-byte aligned, n_cols a multiple of the block), for
// launches of many tokens.
bool gemm_dev(int dtype, const uint8_t* w, const float* x, float* y, int64_t n_rows,
              int64_t n_cols, int64_t rb, int64_t n_tok, hipStream_t s) {
    const int64_t row_tiles = (n_rows + 63) / 64, tok_tiles = (n_tok + 63) / 64;
    const bool fast = dtype == AERO_DTYPE_IQ4_XS
                          ? (reinterpret_cast<uintptr_t>(w) & 7u) == 0 && rb % 8 == 0
                          : aligned16(w) && rb % 16 == 0;
    GemmKernel k = (fast && tune("gemm_fast", 1)) ? pick_gemm<true>(dtype) : pick_gemm<false>(dtype);
    if (k == nullptr || row_tiles > 0x7fffffff || tok_tiles > 65535 || n_cols % 32 != 0) {
        set_error("matmul: no GEMM for dtype %d at %lld x %lld, %lld tokens", dtype,
                  (long long)n_rows, (long long)n_cols, (long long)n_tok);
        return false;
    }
    GemmParams p{w, x, y, n_rows, (int)n_cols, rb, (int)n_tok, n_cols, n_rows};
    return launch("gemm_kernel", k, dim3((unsigned)row_tiles, (unsigned)tok_tiles), dim3(256), 0,
                  s, p);
}

}  // namespace aero
