// Quantised GEMM for many tokens on gfx950 (prefill): y[t, r] = sum_c W[r, c] * x[t, c]
// with W in GGML blocks and x, y fp32 — the reference's matmul
// (src/kernels.cpp:520-538) for token counts where re-reading W for every few
// tokens (the GEMV kernels) would dominate.
//
// A workgroup (4 waves) computes a 64-row x 64-token tile of y. For each
// 128-column chunk of the row it dequantises its 64 rows into LDS as fp32 —
// the reference's dequantised values bit for bit (quant_blocks.hpp decode) —
// and stages the 64 tokens' x, then each wave runs fp32 matrix FMAs
// (v_mfma_f32_16x16x4_f32) over a 32 x 32 sub-tile: exact products, fp32
// accumulation, so results differ from the reference's serial dots only in
// summation order.
//
// LDS tiles hold element (i, k) of a 128-column chunk at i*132 + (k%4)*32 +
// k/4: a lane's operands for four consecutive matrix steps (k = 4s + lane/16,
// s = s0..s0+3) are one 16-byte read, and the 4-float row pad puts the 16
// rows a read touches in 16 different bank groups.
//
// HBM bytes per launch: W once per 64-token tile, x once per 64-row tile
// (mostly from L2), y once.
#include "quant_blocks.hpp"

#pragma clang fp contract(off)

namespace aero {

namespace {

constexpr int kBM = 64, kBN = 64, kBK = 128;
constexpr int kRowF = kBK + 4;  // floats per padded LDS tile row

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

// Four dequantised weights at columns c..c+3 of a row (c a multiple of 4).
template <int TYPE>
__device__ __forceinline__ float4 dequant_quad(const uint8_t* rowp, int c) {
    using Q = QT<TYPE>;
    const int blk = c / Q::BV;
    const int l = (c % Q::BV) / 4;
    typename Q::Raw raw;
    load_raw(rowp + (int64_t)blk * Q::BB, l, raw);
    return decode(raw, l);
}

template <int TYPE>
__global__ __launch_bounds__(256) void gemm_kernel(GemmParams p) {
    __shared__ __align__(16) float As[kBM * kRowF];
    __shared__ __align__(16) float Bs[kBN * kRowF];

    const int tid = threadIdx.x;
    const int l = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave & 1, wn = wave >> 1;
    const int64_t r0 = (int64_t)blockIdx.x * kBM;
    const int t0 = blockIdx.y * kBN;
    const int n_k = (p.n_cols + kBK - 1) / kBK;

    v4f acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) acc[i][j] = v4f{0.f, 0.f, 0.f, 0.f};

    // staging units: (tile row or token, 16-column group), two per thread
    int srow[2], sgrp[2];
    const uint8_t* wrow[2];
    const float* xrow[2];
#pragma unroll
    for (int u = 0; u < 2; ++u) {
        const int unit = tid + 256 * u;
        srow[u] = unit >> 3;
        sgrp[u] = unit & 7;
        wrow[u] = p.w + min(r0 + srow[u], p.n_rows - 1) * p.rb;
        xrow[u] = p.x + (int64_t)min(t0 + srow[u], p.n_tok - 1) * p.x_stride;
    }

    for (int kc = 0; kc < n_k; ++kc) {
        float4 wv[2][4], xv[2][4];
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            const int c = kc * kBK + 16 * sgrp[u];
            const bool valid = c < p.n_cols;  // n_cols is a multiple of 32: whole groups
            const int cc = min(c, p.n_cols - 16);
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const float4 a = dequant_quad<TYPE>(wrow[u], cc + 4 * q);
                const float4 b = *reinterpret_cast<const float4*>(xrow[u] + cc + 4 * q);
                const float4 z = make_float4(0.f, 0.f, 0.f, 0.f);
                wv[u][q] = valid ? a : z;
                xv[u][q] = valid ? b : z;
            }
        }
        __syncthreads();  // the previous chunk's matrix steps are done with LDS
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            float* ar = As + srow[u] * kRowF + 4 * sgrp[u];
            float* br = Bs + srow[u] * kRowF + 4 * sgrp[u];
            *reinterpret_cast<float4*>(ar + 0) = make_float4(wv[u][0].x, wv[u][1].x, wv[u][2].x, wv[u][3].x);
            *reinterpret_cast<float4*>(ar + 32) = make_float4(wv[u][0].y, wv[u][1].y, wv[u][2].y, wv[u][3].y);
            *reinterpret_cast<float4*>(ar + 64) = make_float4(wv[u][0].z, wv[u][1].z, wv[u][2].z, wv[u][3].z);
            *reinterpret_cast<float4*>(ar + 96) = make_float4(wv[u][0].w, wv[u][1].w, wv[u][2].w, wv[u][3].w);
            *reinterpret_cast<float4*>(br + 0) = make_float4(xv[u][0].x, xv[u][1].x, xv[u][2].x, xv[u][3].x);
            *reinterpret_cast<float4*>(br + 32) = make_float4(xv[u][0].y, xv[u][1].y, xv[u][2].y, xv[u][3].y);
            *reinterpret_cast<float4*>(br + 64) = make_float4(xv[u][0].z, xv[u][1].z, xv[u][2].z, xv[u][3].z);
            *reinterpret_cast<float4*>(br + 96) = make_float4(xv[u][0].w, xv[u][1].w, xv[u][2].w, xv[u][3].w);
        }
        __syncthreads();

        const float* ap = As + (32 * wm + (l & 15)) * kRowF + (l >> 4) * 32;
        const float* bp = Bs + (32 * wn + (l & 15)) * kRowF + (l >> 4) * 32;
#pragma unroll
        for (int sg = 0; sg < kBK / 16; ++sg) {
            float4 a[2], b[2];
#pragma unroll
            for (int i = 0; i < 2; ++i) {
                a[i] = *reinterpret_cast<const float4*>(ap + 16 * i * kRowF + 4 * sg);
                b[i] = *reinterpret_cast<const float4*>(bp + 16 * i * kRowF + 4 * sg);
            }
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const float ae[2] = {e == 0 ? a[0].x : e == 1 ? a[0].y : e == 2 ? a[0].z : a[0].w,
                                     e == 0 ? a[1].x : e == 1 ? a[1].y : e == 2 ? a[1].z : a[1].w};
                const float be[2] = {e == 0 ? b[0].x : e == 1 ? b[0].y : e == 2 ? b[0].z : b[0].w,
                                     e == 0 ? b[1].x : e == 1 ? b[1].y : e == 2 ? b[1].z : b[1].w};
#pragma unroll
                for (int i = 0; i < 2; ++i)
#pragma unroll
                    for (int j = 0; j < 2; ++j)
                        acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(ae[i], be[j], acc[i][j], 0, 0, 0);
            }
        }
    }

    // acc[i][j] holds rows 4(l/16)+v, token l%16 of sub-tile (i, j)
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const int64_t row = r0 + 32 * wm + 16 * i + 4 * (l >> 4);
            const int tok = t0 + 32 * wn + 16 * j + (l & 15);
            if (tok < p.n_tok) {
                float* yp = p.y + (int64_t)tok * p.y_stride;
#pragma unroll
                for (int v = 0; v < 4; ++v)
                    if (row + v < p.n_rows) yp[row + v] = acc[i][j][v];
            }
        }
}

using GemmKernel = void (*)(GemmParams);

GemmKernel pick_gemm(int dtype) {
    switch (dtype) {
    case AERO_DTYPE_Q8_0: return gemm_kernel<AERO_DTYPE_Q8_0>;
    case AERO_DTYPE_Q4_K: return gemm_kernel<AERO_DTYPE_Q4_K>;
    case AERO_DTYPE_Q5_K: return gemm_kernel<AERO_DTYPE_Q5_K>;
    case AERO_DTYPE_Q6_K: return gemm_kernel<AERO_DTYPE_Q6_K>;
    case AERO_DTYPE_IQ4_XS: return gemm_kernel<AERO_DTYPE_IQ4_XS>;
    default: return nullptr;
    }
}

}  // namespace

// Called by gemv_dev after its argument checks (W's size and alignment, block
// multiple of n_cols), for launches of many tokens.
bool gemm_dev(int dtype, const uint8_t* w, const float* x, float* y, int64_t n_rows,
              int64_t n_cols, int64_t rb, int64_t n_tok, hipStream_t s) {
    GemmKernel k = pick_gemm(dtype);
    const int64_t row_tiles = (n_rows + kBM - 1) / kBM, tok_tiles = (n_tok + kBN - 1) / kBN;
    if (k == nullptr || row_tiles > 0x7fffffff || tok_tiles > 65535 || n_cols % 32 != 0) {
        set_error("matmul: no GEMM for dtype %d at %lld x %lld, %lld tokens", dtype,
                  (long long)n_rows, (long long)n_cols, (long long)n_tok);
        return false;
    }
    GemmParams p{w, x, y, n_rows, (int)n_cols, rb, (int)n_tok, n_cols, n_rows};
    return launch("gemm_kernel", k, dim3((unsigned)row_tiles, (unsigned)tok_tiles), dim3(256), 0, s,
                  p);
}

}  // namespace aero
