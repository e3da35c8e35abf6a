// KV cache vectors read back from their quantised form, and the
// quantisation error of a written span (src/kv.cpp:30-46, 72-88). The
// writer is kv_write_kernel (attention.hip). Codes: dt 0 fp32, 1 int8 (one
// scale a vector), 2 int4 packed two a byte, low nibble first, sign-extended
// from 4 bits. The value is float(code) * scale, as the reference computes
// it, so reads are bit-exact; the span error's maxima are order-free, so it
// is bit-exact too.
#include "common.hpp"
#include "aero_hip.h"

#include <cmath>

#pragma clang fp contract(off)

namespace aero {
namespace {

template <int DT>
__device__ __forceinline__ float kv_code(const void* q, int64_t vec, int64_t dim, int64_t i) {
    if constexpr (DT == 0) {
        return static_cast<const float*>(q)[vec * dim + i];
    } else if constexpr (DT == 1) {
        return (float)static_cast<const int8_t*>(q)[vec * dim + i];
    } else {
        const uint8_t b = static_cast<const uint8_t*>(q)[vec * (dim / 2) + i / 2];
        const int n = (i & 1) ? (b >> 4) & 15 : b & 15;
        return (float)(n >= 8 ? n - 16 : n);
    }
}

// one 64-lane workgroup a vector: out[v][i] = code * scale[v] (fp32: a copy)
template <int DT>
__global__ __launch_bounds__(64) void kv_read_kernel(const void* q, const float* scale,
                                                     int64_t dim, float* out) {
    const int64_t v = blockIdx.x;
    const float s = DT == 0 ? 1.0f : scale[v];
    for (int64_t i = threadIdx.x; i < dim; i += 64) {
        const float c = kv_code<DT>(q, v, dim, i);
        out[v * dim + i] = DT == 0 ? c : c * s;
    }
}

// one 256-lane workgroup: max |read - x| / max |x| (1e-9 when x is all zero)
template <int DT>
__global__ __launch_bounds__(256) void kv_span_error_kernel(const void* q, const float* scale,
                                                            int64_t dim, const float* x,
                                                            float* out) {
    __shared__ float se[4], sx[4];
    const float s = DT == 0 ? 1.0f : scale[0];
    float me = 0.0f, mx = 0.0f;
    for (int64_t i = threadIdx.x; i < dim; i += 256) {
        const float c = kv_code<DT>(q, 0, dim, i);
        const float back = DT == 0 ? c : c * s;
        me = fmaxf(me, fabsf(back - x[i]));
        mx = fmaxf(mx, fabsf(x[i]));
    }
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) {
        me = fmaxf(me, __shfl_xor(me, off, 64));
        mx = fmaxf(mx, __shfl_xor(mx, off, 64));
    }
    if ((threadIdx.x & 63) == 0) {
        se[threadIdx.x >> 6] = me;
        sx[threadIdx.x >> 6] = mx;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        me = fmaxf(fmaxf(se[0], se[1]), fmaxf(se[2], se[3]));
        mx = fmaxf(fmaxf(sx[0], sx[1]), fmaxf(sx[2], sx[3]));
        out[0] = me / (mx > 0.0f ? mx : 1e-9f);
    }
}

}  // namespace

bool kv_read_dev(int dt, const void* q, const float* scale, int64_t n_vec, int64_t dim,
                 float* out, hipStream_t s) {
    if (q == nullptr || out == nullptr || n_vec < 0 || dim <= 0 || dt < 0 || dt > 2 ||
        (dt != 0 && scale == nullptr) || (dt == 2 && dim % 2) || n_vec > 0x7fffffff) {
        set_error("kv_read: bad arguments (dt=%d n_vec=%lld dim=%lld)", dt, (long long)n_vec,
                  (long long)dim);
        return false;
    }
    if (n_vec == 0) return true;
    const dim3 g((unsigned)n_vec), b(64);
    switch (dt) {
    case 0: return launch("kv_read_kernel", kv_read_kernel<0>, g, b, 0, s, q, scale, dim, out);
    case 1: return launch("kv_read_kernel", kv_read_kernel<1>, g, b, 0, s, q, scale, dim, out);
    default: return launch("kv_read_kernel", kv_read_kernel<2>, g, b, 0, s, q, scale, dim, out);
    }
}

bool kv_span_error_dev(int dt, const void* q, const float* scale, int64_t dim, const float* x,
                       float* out, hipStream_t s) {
    if (q == nullptr || x == nullptr || out == nullptr || dim <= 0 || dt < 0 || dt > 2 ||
        (dt != 0 && scale == nullptr) || (dt == 2 && dim % 2)) {
        set_error("kv_span_error: bad arguments (dt=%d dim=%lld)", dt, (long long)dim);
        return false;
    }
    const dim3 g(1), b(256);
    switch (dt) {
    case 0:
        return launch("kv_span_error_kernel", kv_span_error_kernel<0>, g, b, 0, s, q, scale, dim,
                      x, out);
    case 1:
        return launch("kv_span_error_kernel", kv_span_error_kernel<1>, g, b, 0, s, q, scale, dim,
                      x, out);
    default:
        return launch("kv_span_error_kernel", kv_span_error_kernel<2>, g, b, 0, s, q, scale, dim,
                      x, out);
    }
}

}  // namespace aero
