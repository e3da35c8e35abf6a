// Quantised GEMV / small-batch GEMM on gfx950: y[t, r] = sum_c W[r, c] * x[t, c]
// with W in GGML blocks (Q8_0, Q4_K, Q5_K, Q6_K, IQ4_XS), x and y fp32 — the
// reference's matvec / matmul (src/kernels.cpp:497-538) with its block dots
// (:78-250), which it calls between the elementwise ops of a layer.
//
// One wave (a 64-thread workgroup) owns R consecutive output rows. It walks
// the columns in chunks of U 256-value steps: the chunk's quant blocks of each
// of its rows (contiguous in W) are loaded with coalesced 32-bit loads, all
// issued before any is used, and staged in LDS; then in each step lane l takes
// values 4l..4l+3 (the gather's lane layout, quant_blocks.hpp), loads one
// float4 of x per token, and for each row expands its four weights into
// (q[4], f, g) and accumulates f*sum(q*x) - g*sum(x) — the factoring of the
// reference's block dots, so sum(x) is shared by all R rows and a row costs
// four multiply-adds per lane per step. x is read once per step for R rows.
// At the end each (row, token) sum is an xor-butterfly over the wave.
//
// HBM bytes per launch: the weight blocks once (n_rows * n_cols/bv * bb) plus
// x and y; x is re-read from L2 by every wave. Results differ from the
// reference's serial sums only in summation order.
#include "quant_blocks.hpp"

#pragma clang fp contract(off)

namespace aero {

int64_t dtype_block_bytes(int t);
int64_t dtype_block_values(int t);

namespace {

struct GemvParams {
    const uint8_t* w;  // n_rows rows of rb bytes
    const float* x;    // n_tok rows of x_stride floats (the first n_cols used)
    float* y;          // n_tok rows of y_stride floats (the first n_rows written)
    int64_t n_rows;
    int n_cols;
    int64_t rb;
    int n_tok;         // tokens this launch handles (<= T)
    int64_t x_stride, y_stride;
};

template <int TYPE, int R, int U, int T>
__global__ __launch_bounds__(64) void gemv_kernel(GemvParams p) {
    using Q = QT<TYPE>;
    constexpr int BPS = 256 / Q::BV;                           // blocks per step
    constexpr int MAX_DW = (U * BPS * Q::BB + 3 + 3) / 4;     // + misalignment
    constexpr int PER = (MAX_DW + 63) / 64;
    __shared__ __align__(16) uint32_t stage[R][PER * 64];

    const int l = threadIdx.x;
    const int64_t r0 = (int64_t)blockIdx.x * R;
    const int steps = (p.n_cols + 255) / 256;

    float acc[R][T];
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
        for (int t = 0; t < T; ++t) acc[r][t] = 0.0f;

    for (int s0 = 0; s0 < steps; s0 += U) {
        const int nv = min(U * 256, p.n_cols - s0 * 256);  // values in this chunk
        const int nbytes = (nv / Q::BV) * Q::BB;
        // Each row's chunk: the 4-byte words covering it (aligned down; rows of
        // Q8_0 / Q6_K may start 2 bytes past a word). Rows past the end re-read
        // the last row, and lanes past the chunk its last word, so every load is
        // unconditional and all are in flight together.
        int off[R];
        uint32_t wv[R][PER];
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const int64_t row = min(r0 + r, p.n_rows - 1);
            const uint8_t* g = p.w + row * p.rb + (int64_t)(s0 * 256 / Q::BV) * Q::BB;
            off[r] = (int)(reinterpret_cast<uintptr_t>(g) & 3u);
            const uint32_t* g4 = reinterpret_cast<const uint32_t*>(g - off[r]);
            const int n_dw = (off[r] + nbytes + 3) >> 2;
#pragma unroll
            for (int i = 0; i < PER; ++i) wv[r][i] = g4[min(l + 64 * i, n_dw - 1)];
        }
        __syncthreads();  // the previous chunk's LDS reads are done
#pragma unroll
        for (int r = 0; r < R; ++r)
#pragma unroll
            for (int i = 0; i < PER; ++i) stage[r][l + 64 * i] = wv[r][i];
        __syncthreads();

#pragma unroll
        for (int st = 0; st < U; ++st) {
            const int v0 = st * 256 + 4 * l;
            if (v0 >= nv) break;
            float4 xv[T];
            float sx[T];
#pragma unroll
            for (int t = 0; t < T; ++t) {
                const int tt = t < p.n_tok ? t : 0;
                xv[t] = *reinterpret_cast<const float4*>(p.x + tt * p.x_stride + s0 * 256 + v0);
                sx[t] = ((xv[t].x + xv[t].y) + xv[t].z) + xv[t].w;
            }
#pragma unroll
            for (int r = 0; r < R; ++r) {
                typename Q::Raw raw;
                load_raw(reinterpret_cast<const uint8_t*>(stage[r]) + off[r] + (v0 / Q::BV) * Q::BB,
                         l, raw);
                const Quad w4 = expand(raw, l);
#pragma unroll
                for (int t = 0; t < T; ++t) {
                    float qx = w4.q[0] * xv[t].x;
                    qx = __builtin_fmaf(w4.q[1], xv[t].y, qx);
                    qx = __builtin_fmaf(w4.q[2], xv[t].z, qx);
                    qx = __builtin_fmaf(w4.q[3], xv[t].w, qx);
                    acc[r][t] = __builtin_fmaf(w4.f, qx, acc[r][t]);
                    if (HasMin<TYPE>::value) acc[r][t] = __builtin_fmaf(-w4.g, sx[t], acc[r][t]);
                }
            }
        }
    }

#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
        for (int t = 0; t < T; ++t) {
            const float v = group_sum<64>(acc[r][t]);
            if (l == 0 && r0 + r < p.n_rows && t < p.n_tok) p.y[t * p.y_stride + r0 + r] = v;
        }
}

using GemvKernel = void (*)(GemvParams);

template <int TYPE, int R, int U>
GemvKernel pick_t(int T) {
    switch (T) {
    case 1: return gemv_kernel<TYPE, R, U, 1>;
    case 2: return gemv_kernel<TYPE, R, U, 2>;
    case 4: return gemv_kernel<TYPE, R, U, 4>;
    case 8: return gemv_kernel<TYPE, R, U, 8>;
    default: return nullptr;
    }
}

// Steps per chunk: 16 (Q8_0: 8, its blocks take 1.9x the LDS of Q4_K's).
template <int TYPE> constexpr int chunk_steps() { return TYPE == AERO_DTYPE_Q8_0 ? 8 : 16; }

template <int TYPE>
GemvKernel pick_r(int R, int T) {
    constexpr int U = chunk_steps<TYPE>();
    switch (R) {
    case 1: return pick_t<TYPE, 1, U>(T);
    case 2: return pick_t<TYPE, 2, U>(T);
    case 4: return pick_t<TYPE, 4, U>(T);
    default: return nullptr;
    }
}

GemvKernel pick_gemv(int dtype, int R, int T) {
    switch (dtype) {
    case AERO_DTYPE_Q8_0: return pick_r<AERO_DTYPE_Q8_0>(R, T);
    case AERO_DTYPE_Q4_K: return pick_r<AERO_DTYPE_Q4_K>(R, T);
    case AERO_DTYPE_Q5_K: return pick_r<AERO_DTYPE_Q5_K>(R, T);
    case AERO_DTYPE_Q6_K: return pick_r<AERO_DTYPE_Q6_K>(R, T);
    case AERO_DTYPE_IQ4_XS: return pick_r<AERO_DTYPE_IQ4_XS>(R, T);
    default: return nullptr;
    }
}

}  // namespace

// y[t, r] for t < n_tok: tokens are taken in groups of up to 8 per launch
// (each group re-reads W; a token-tiled GEMM is the prefill path).
bool gemv_dev(int dtype, const uint8_t* w, int64_t w_bytes, const float* x, float* y,
              int64_t n_rows, int64_t n_cols, int64_t n_tok, hipStream_t s) {
    const int64_t bv = dtype_block_values(dtype), bb = dtype_block_bytes(dtype);
    const bool quant = dtype == AERO_DTYPE_Q8_0 || dtype == AERO_DTYPE_Q4_K ||
                       dtype == AERO_DTYPE_Q5_K || dtype == AERO_DTYPE_Q6_K ||
                       dtype == AERO_DTYPE_IQ4_XS;
    if (!quant) {
        set_error("matvec: dtype %d has no quantised GEMV (Q8_0, Q4_K, Q5_K, Q6_K, IQ4_XS)",
                  dtype);
        return false;
    }
    if (w == nullptr || x == nullptr || y == nullptr || n_rows < 0 || n_cols <= 0 ||
        n_tok < 0 || n_cols % bv != 0 || n_cols > (int64_t)1 << 30) {
        set_error("matvec: bad arguments (n_rows=%lld n_cols=%lld n_tok=%lld; n_cols must "
                  "be a positive multiple of %lld)", (long long)n_rows, (long long)n_cols,
                  (long long)n_tok, (long long)bv);
        return false;
    }
    const int64_t rb = (n_cols / bv) * bb;
    if (w_bytes < n_rows * rb) {
        set_error("matvec: w_bytes %lld < n_rows*row_bytes %lld", (long long)w_bytes,
                  (long long)(n_rows * rb));
        return false;
    }
    if ((reinterpret_cast<uintptr_t>(w) & 3u) || !aligned16(x)) {
        set_error("matvec: w must be 4-byte and x 16-byte aligned");
        return false;
    }
    if (n_rows == 0 || n_tok == 0) return true;
    // rows per wave: share each x load across more rows while the grid keeps
    // >= 1024 waves
    int R = n_rows >= 4 * 1024 ? 4 : (n_rows >= 2 * 1024 ? 2 : 1);
    R = tune("gemv_r", R);
    const int64_t waves = (n_rows + R - 1) / R;
    if (waves > 0x7fffffff) {
        set_error("matvec: grid too large");
        return false;
    }
    for (int64_t t0 = 0; t0 < n_tok; t0 += 8) {
        const int nt = (int)std::min<int64_t>(8, n_tok - t0);
        const int T = nt == 1 ? 1 : (nt == 2 ? 2 : (nt <= 4 ? 4 : 8));
        GemvKernel k = pick_gemv(dtype, R, T);
        if (k == nullptr) {
            set_error("matvec: no kernel for rows/wave %d", R);
            return false;
        }
        GemvParams p{w, x + t0 * n_cols, y + t0 * n_rows, n_rows, (int)n_cols, rb, nt,
                     n_cols, n_rows};
        if (!launch("gemv_kernel", k, dim3((unsigned)waves), dim3(64), 0, s, p)) return false;
    }
    return true;
}

}  // namespace aero

extern "C" {

int aero_hip_matvec(int dtype, const uint8_t* w, int64_t w_bytes, const float* x, float* y,
                    int64_t n_rows, int64_t n_cols, int64_t n_tok, void* stream) {
    return aero::gemv_dev(dtype, w, w_bytes, x, y, n_rows, n_cols, n_tok,
                          (hipStream_t)stream) ? 1 : 0;
}

}  // extern "C"
