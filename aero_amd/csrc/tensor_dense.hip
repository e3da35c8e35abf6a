// The reference's fp32 tensor primitives that are not elementwise: the dense
// matvec / matmul and argmax of src/tensor.cpp (:65-92, :180-186), behind
// its C ABI aero_tensor_matvec / aero_tensor_matmul / aero_tensor_argmax
// (:209-231, :298-302) in dropin.hip. They complete that ABI so the
// reference's own loader binds this library; they are not on the fused
// path and are built for exact agreement, not for speed (the host-pointer
// calls they serve move W over PCIe, which dominates).
//
// Results equal the reference's bit for bit: one lane a (token, row) sums
// the row in the reference's order with contraction off. matvec (and
// matmul of one token) adds four products at a time, acc += ((w0*x0 +
// w1*x1) + w2*x2) + w3*x3, then the tail one by one; matmul of several
// tokens adds one product at a time. Adjacent lanes take adjacent rows, so
// a wave's load touches 64 rows at one column; the rows' cache lines serve
// the following columns.
//
// argmax is the first index of the largest value, NaN never chosen, as the
// reference's strict '>' scan from v[0] gives (0 when v[0] is NaN).
#include "common.hpp"
#include "aero_hip.h"

#include <cmath>

#pragma clang fp contract(off)

namespace aero {
namespace {

constexpr int kDenseBlock = 256;

template <bool GROUPED, bool VEC>
__global__ __launch_bounds__(kDenseBlock)
void dense_rows_kernel(const float* w, const float* x, float* y, int64_t n_rows,
                       int64_t n_cols, int64_t n_tok) {
    const int64_t i = (int64_t)blockIdx.x * kDenseBlock + threadIdx.x;
    if (i >= n_rows * n_tok) return;
    const int64_t t = i / n_rows, r = i - t * n_rows;
    const float* wr = w + r * n_cols;
    const float* xt = x + t * n_cols;
    float acc = 0.0f;
    int64_t c = 0;
    if constexpr (GROUPED) {
        for (; c + 4 <= n_cols; c += 4) {
            float4 a, b;
            if constexpr (VEC) {
                a = *reinterpret_cast<const float4*>(wr + c);
                b = *reinterpret_cast<const float4*>(xt + c);
            } else {
                a = make_float4(wr[c], wr[c + 1], wr[c + 2], wr[c + 3]);
                b = make_float4(xt[c], xt[c + 1], xt[c + 2], xt[c + 3]);
            }
            acc += a.x * b.x + a.y * b.y + a.z * b.z + a.w * b.w;
        }
    } else if constexpr (VEC) {
        for (; c + 4 <= n_cols; c += 4) {
            const float4 a = *reinterpret_cast<const float4*>(wr + c);
            const float4 b = *reinterpret_cast<const float4*>(xt + c);
            acc += a.x * b.x;
            acc += a.y * b.y;
            acc += a.z * b.z;
            acc += a.w * b.w;
        }
    }
    for (; c < n_cols; ++c) acc += wr[c] * xt[c];
    y[t * n_rows + r] = acc;
}

struct Best {
    float v;
    int64_t i;
    bool has;
};

__device__ __forceinline__ Best pick(Best a, Best b) {
    if (!b.has) return a;
    if (!a.has) return b;
    return (b.v > a.v || (b.v == a.v && b.i < a.i)) ? b : a;
}

// One workgroup over the whole vector: lane l scans l, l + 1024, ... in
// order (keeping its first largest), then a tree of (value, index) pairs
// keeps the largest value and, among equals, the lowest index.
constexpr int kArgmaxBlock = 1024;

__global__ __launch_bounds__(kArgmaxBlock)
void argmax_kernel(const float* v, int64_t n, int32_t* out) {
    __shared__ float sv[kArgmaxBlock];
    __shared__ int64_t si[kArgmaxBlock];
    __shared__ int sh[kArgmaxBlock];
    const int tid = threadIdx.x;
    Best b{0.0f, 0, false};
    for (int64_t i = tid; i < n; i += kArgmaxBlock) {
        const float e = v[i];
        if (!isnan(e) && (!b.has || e > b.v)) b = Best{e, i, true};
    }
    sv[tid] = b.v;
    si[tid] = b.i;
    sh[tid] = b.has ? 1 : 0;
    __syncthreads();
    for (int s = kArgmaxBlock / 2; s > 0; s >>= 1) {
        if (tid < s) {
            const Best o = pick(Best{sv[tid], si[tid], sh[tid] != 0},
                                Best{sv[tid + s], si[tid + s], sh[tid + s] != 0});
            sv[tid] = o.v;
            si[tid] = o.i;
            sh[tid] = o.has ? 1 : 0;
        }
        __syncthreads();
    }
    if (tid == 0) out[0] = (isnan(v[0]) || !sh[0]) ? 0 : (int32_t)si[0];
}

}  // namespace

bool dense_matmul_dev(const float* w, const float* x, float* y, int64_t n_rows, int64_t n_cols,
                      int64_t n_tok, hipStream_t s) {
    if (w == nullptr || x == nullptr || y == nullptr || n_rows <= 0 || n_cols <= 0 ||
        n_tok <= 0) {
        set_error("dense matmul: null or non-positive dims");
        return false;
    }
    const int64_t blocks = (n_rows * n_tok + kDenseBlock - 1) / kDenseBlock;
    if (blocks > 0x7fffffff) {
        set_error("dense matmul: too many outputs");
        return false;
    }
    const bool vec = n_cols % 4 == 0 && aligned16(w) && aligned16(x);
    const dim3 g((unsigned)blocks), b(kDenseBlock);
    if (n_tok == 1)
        return vec ? launch("dense_rows_kernel", dense_rows_kernel<true, true>, g, b, 0, s, w, x,
                            y, n_rows, n_cols, n_tok)
                   : launch("dense_rows_kernel", dense_rows_kernel<true, false>, g, b, 0, s, w,
                            x, y, n_rows, n_cols, n_tok);
    return vec ? launch("dense_rows_kernel", dense_rows_kernel<false, true>, g, b, 0, s, w, x, y,
                        n_rows, n_cols, n_tok)
               : launch("dense_rows_kernel", dense_rows_kernel<false, false>, g, b, 0, s, w, x,
                        y, n_rows, n_cols, n_tok);
}

bool argmax_dev(const float* v, int64_t n, int32_t* out, hipStream_t s) {
    if (v == nullptr || out == nullptr || n <= 0 || n > (int64_t)0x7fffffff) {
        set_error("argmax: null, n <= 0 or n beyond an int index");
        return false;
    }
    return launch("argmax_kernel", argmax_kernel, dim3(1), dim3(kArgmaxBlock), 0, s, v, n, out);
}

}  // namespace aero
