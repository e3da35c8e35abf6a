// Row norms on gfx950: RMSNorm (plain, Gemma (1+w), weightless), the L2
// variant, and the gated-DeltaNet norm(x)*silu(z).
//
// One kernel template covers all of them. A row (or a `group`-long slice of
// a row) is owned by TPR consecutive lanes; each lane keeps V float4 of the
// row in VGPRs, so x (and z) are read from HBM exactly once with 128-bit
// coalesced loads (nontemporal: each element is used once). The sum of
// squares is reduced with a wave64 xor butterfly
// and, when a row spans several waves, one LDS step. The output is written
// once with 128-bit stores. HBM bytes per row: 4*(2*cols) (+4*cols for z);
// the weight vector is re-read from L2, not HBM.
//
// Arithmetic follows the reference operation by operation with contraction
// disabled: inv = 1/sqrtf(ss/n + eps), out = (x*inv)*w (src/tensor.cpp:
// 128-134); L2: inv = 1/max(sqrtf(ss), eps) (src/tensor.cpp:136-154). The
// summation order of ss differs (tree instead of serial). The gated norm,
// out = ((x/denom)*w)*(z/(1+expf(-z))) in the reference (src/ssm.cpp:17,
// 327-343), multiplies by 1/denom and takes silu from the hardware exp and
// reciprocal (a few ulp from the division form; see the vector kernel).
#include <algorithm>

#include "common.hpp"
#include "aero_hip.h"

#pragma clang fp contract(off)

namespace aero {
namespace {

struct NormParams {
    const float* x;
    const float* z;      // gated only
    const float* w;      // may be null (ones)
    float* out;          // may alias x
    int64_t rows;        // number of normalised slices
    int cols;            // slice length
    int gpr;             // slices per original row (weight offset)
    int w_len;           // weight period
    float eps;
    int flags;
    float* xo;           // residual form: x + z written here (may alias x or z)
};

// Kernel forms: plain / L2 norm, gated norm*silu(z), residual add then norm.
constexpr int kPlain = 0, kGated = 1, kResid = 2;


__device__ __forceinline__ float norm_scale(float ss, const NormParams& p) {
    if (p.flags & AERO_NORM_L2) {
        const float nrm = sqrtf(ss);
        return 1.0f / (nrm > p.eps ? nrm : p.eps);
    }
    return 1.0f / sqrtf(ss / (float)p.cols + p.eps);
}

__device__ __forceinline__ float apply_w(float v, const float* w, int idx, int flags) {
    if (w == nullptr) return v;
    const float wc = (flags & AERO_NORM_UNIT_OFFSET) ? 1.0f + w[idx] : w[idx];
    return v * wc;
}

template <int TPR, int V, int MODE>
__global__ __launch_bounds__(TPR > 256 ? TPR : 256)
void norm_vec_kernel(NormParams p) {
    constexpr bool GATED = MODE == kGated;
    constexpr bool RESID = MODE == kResid;
    constexpr int BS = TPR > 256 ? TPR : 256;
    constexpr int RPB = BS / TPR;
    const int tid = threadIdx.x;
    const int lr = tid / TPR;
    const int t = tid % TPR;
    const int64_t row = (int64_t)blockIdx.x * RPB + lr;
    const bool ok = row < p.rows;
    const int nv = p.cols >> 2;
    const int64_t base = ok ? row * (int64_t)p.cols : 0;
    const float* xr = p.x + base;
    const float* zr = (GATED || RESID) ? p.z + base : p.x;

    // The gated norm loads its weights here, with the row: stores count in
    // the same vector-memory counter as loads, so a load issued after the
    // first store waits for every store before it (measured: 40.1 -> 36.4 us
    // at 4096 x 4096). So does the residual form, which stores x + d before
    // its reduction, at up to 4 float4 a lane (512 x 4096: 6.3 -> 5.9 us,
    // 16384 x 8192: 364.5 -> 351.8 us on MI355X; at 5 a lane the extra
    // registers cost a wave a SIMD: 2048 x 2560 14.3 -> 15.1 us). The plain
    // norm keeps its weight load beside each store: moving it here, or after
    // the reduction, made 2048 x 2560 and 4096 x 2048 ~20% slower on MI355X
    // (7.7 -> 9.5 us, 11.0 -> 13.3 us) and gained 2-4% elsewhere; an explicit
    // wait after each store did not recover it. Rows of 512 lanes (8192
    // columns and more) take it: 16384 x 8192 182.5 -> 177.0 us a dispatch
    // (at 256 lanes, 512 x 4096, per-dispatch and back-to-back times moved in
    // opposite directions).
    constexpr bool W_EARLY = V <= 4 && (RESID || (!GATED && TPR >= 512));
    float4 xv[V];
    float4 zv[V];
    float4 wv[V];
    const int col0 = GATED ? (int)((ok ? row : 0) % p.gpr) * p.cols : 0;
#pragma unroll
    for (int i = 0; i < V; ++i) {
        const int c = i * TPR + t;
        wv[i] = make_float4(1.f, 1.f, 1.f, 1.f);
        if (ok && c < nv) {
            xv[i] = ld_stream(xr + 4 * c);
            if (GATED) {
                zv[i] = ld_stream(zr + 4 * c);
                wv[i] = *reinterpret_cast<const float4*>(p.w + (col0 + 4 * c) % p.w_len);
            }
            if (RESID) zv[i] = ld_stream(zr + 4 * c);
            if (W_EARLY && p.w != nullptr) wv[i] = *reinterpret_cast<const float4*>(p.w + 4 * c);
        } else {
            xv[i] = make_float4(0.f, 0.f, 0.f, 0.f);
            if (GATED || RESID) zv[i] = xv[i];
        }
    }
    if constexpr (RESID) {
        // x + d is the new residual stream: stored at once, before the
        // reduction, so the stores overlap the cross-wave step
        const int64_t r0 = (int64_t)blockIdx.x * RPB;
        const StreamOut ox(p.xo + r0 * p.cols, (p.rows - r0) * (int64_t)p.cols * 4);
        const uint32_t xb = (uint32_t)(lr * p.cols) * 4u;
#pragma unroll
        for (int i = 0; i < V; ++i) {
            xv[i].x = xv[i].x + zv[i].x;
            xv[i].y = xv[i].y + zv[i].y;
            xv[i].z = xv[i].z + zv[i].z;
            xv[i].w = xv[i].w + zv[i].w;
            const int c = i * TPR + t;
            if (ok && c < nv) ox.store(xb + 16u * c, xv[i]);
        }
    }
    float ss = 0.0f;
#pragma unroll
    for (int i = 0; i < V; ++i) {
        ss += xv[i].x * xv[i].x;
        ss += xv[i].y * xv[i].y;
        ss += xv[i].z * xv[i].z;
        ss += xv[i].w * xv[i].w;
    }
    if constexpr (TPR <= 64) {
        ss = group_sum<TPR>(ss);
    } else {
        constexpr int WPR = TPR / 64;  // waves per row
        __shared__ float part[BS / 64];
        ss = group_sum<64>(ss);
        if ((tid & 63) == 0) part[tid >> 6] = ss;
        __syncthreads();
        const int w0 = lr * WPR;
        ss = part[w0];
#pragma unroll
        for (int k = 1; k < WPR; ++k) ss += part[w0 + k];
    }
    // every lane of the block shares the descriptor based at its first row
    const int64_t row0 = (int64_t)blockIdx.x * RPB;
    const StreamOut os(p.out + row0 * p.cols, (p.rows - row0) * (int64_t)p.cols * 4);
    const uint32_t obase = (uint32_t)(lr * p.cols) * 4u;
    if (!ok) return;

    if constexpr (GATED) {
        // one division a row, then multiplies; silu with the hardware exp and
        // reciprocal. The gated norm is bound by its instructions, not its
        // bytes, with the division form (x/denom, z/(1+expf(-z))): 35.0 ->
        // 33.6 us at 4096 x 4096 and 7.2 -> 5.5 us at 512 x 4096 on MI355X,
        // within 1.5e-6 of the reference's division form.
        const float rinv = 1.0f / sqrtf(ss / (float)p.cols + p.eps);
        auto out4 = [&](int i) {
            float4 o;
            o.x = ((xv[i].x * rinv) * wv[i].x) * silu_fast(zv[i].x);
            o.y = ((xv[i].y * rinv) * wv[i].y) * silu_fast(zv[i].y);
            o.z = ((xv[i].z * rinv) * wv[i].z) * silu_fast(zv[i].z);
            o.w = ((xv[i].w * rinv) * wv[i].w) * silu_fast(zv[i].w);
            return o;
        };
        if (nv == V * TPR) {
            // whole rows of V float4 per lane: no per-element branch, so the
            // compiler waits for z and w once, not before every store
#pragma unroll
            for (int i = 0; i < V; ++i) os.store(obase + 16u * (i * TPR + t), out4(i));
        } else {
#pragma unroll
            for (int i = 0; i < V; ++i) {
                const int c = i * TPR + t;
                if (c < nv) os.store(obase + 16u * c, out4(i));
            }
        }
    } else {
        const float inv = norm_scale(ss, p);
#pragma unroll
        for (int i = 0; i < V; ++i) {
            const int c = i * TPR + t;
            if (c >= nv) continue;
            float4 o = make_float4(xv[i].x * inv, xv[i].y * inv, xv[i].z * inv,
                                   xv[i].w * inv);
            if (p.w != nullptr) {
                float4 w4 = W_EARLY ? wv[i] : reinterpret_cast<const float4*>(p.w)[c];
                if (p.flags & AERO_NORM_UNIT_OFFSET) {
                    w4.x = 1.0f + w4.x; w4.y = 1.0f + w4.y;
                    w4.z = 1.0f + w4.z; w4.w = 1.0f + w4.w;
                }
                o.x = o.x * w4.x; o.y = o.y * w4.y; o.z = o.z * w4.z; o.w = o.w * w4.w;
            }
            os.store(obase + 16u * c, o);
        }
    }
}

// Read-only stand-in weight for a weightless norm, read with stride 0
// (global memory, so the select between it and p.w stays a global load).
__device__ float kOnes[4] = {1.0f, 1.0f, 1.0f, 1.0f};

// Persistent form of norm_vec_kernel for many rows: a grid of a few
// workgroups per CU, each looping over row groups blockIdx.x, +gridDim.x, ...
// (`iters` rounds, the last one partial). Two differences from the per-row
// form:
//  - the lane's weight chunks are loaded once, into registers, for every row
//    it sees; the per-row form re-reads them from L2 for every row, half as
//    many extra L2 requests as the row's own loads and stores;
//  - the next row group's loads are issued before this one's reduction and
//    stores, so each wave keeps a row in flight across its own reduction.
// Loads are unconditional, from clamped row and chunk indices (a branch
// around a load makes the compiler wait for every load before it); chunks
// past the row's end are zeroed by a select and never stored, and a round
// past the last group only loads (the clamped last group) and stores
// nothing. Gated slices need cols % w_len == 0, so every slice has the same
// weight phase. Same arithmetic and summation order as norm_vec_kernel.
template <int TPR, int V, int MODE>
__global__ __launch_bounds__(TPR > 256 ? TPR : 256)
void norm_loop_kernel(NormParams p, int iters) {
    constexpr bool GATED = MODE == kGated;
    constexpr bool RESID = MODE == kResid;
    constexpr bool TWO = GATED || RESID;
    constexpr int BS = TPR > 256 ? TPR : 256;
    constexpr int RPB = BS / TPR;
    constexpr int NW = BS / 64;
    __shared__ float part[2][NW];
    const int tid = threadIdx.x;
    const int lr = tid / TPR;
    const int t = tid % TPR;
    const int nv = p.cols >> 2;
    const int64_t last = p.rows - 1;
    const int64_t ngroups = (p.rows + RPB - 1) / RPB;

    int cc[V];
#pragma unroll
    for (int i = 0; i < V; ++i) cc[i] = min(i * TPR + t, nv - 1);

    const bool has_w = p.w != nullptr;
    const float* wb = has_w ? p.w : kOnes;
    const int wst = has_w ? 1 : 0;
    const bool unit = has_w && (p.flags & AERO_NORM_UNIT_OFFSET) != 0;
    float4 wv[V];
#pragma unroll
    for (int i = 0; i < V; ++i) {
        const int wi = GATED ? (4 * cc[i]) % p.w_len : 4 * cc[i];
        wv[i] = *reinterpret_cast<const float4*>(wb + wst * wi);
    }

    auto load_rows = [&](int64_t g, float4 (&xv)[V], float4 (&zv)[V]) {
        const int64_t row = min(g * RPB + lr, last);
        const float* xr = p.x + row * (int64_t)p.cols;
        const float* zr = (TWO ? p.z : p.x) + row * (int64_t)p.cols;
#pragma unroll
        for (int i = 0; i < V; ++i) {
            xv[i] = ld_stream(xr + 4 * cc[i]);
            if (TWO) zv[i] = ld_stream(zr + 4 * cc[i]);
        }
    };

    auto process = [&](int64_t g, int k, float4 (&xv)[V], float4 (&zv)[V]) {
        const int64_t row0 = g * RPB;
        const bool ok = row0 + lr < p.rows;
        const uint32_t obase = (uint32_t)(lr * p.cols) * 4u;
        if constexpr (RESID) {
            const StreamOut ox(p.xo + row0 * p.cols, (p.rows - row0) * (int64_t)p.cols * 4);
#pragma unroll
            for (int i = 0; i < V; ++i) {
                xv[i].x = xv[i].x + zv[i].x;
                xv[i].y = xv[i].y + zv[i].y;
                xv[i].z = xv[i].z + zv[i].z;
                xv[i].w = xv[i].w + zv[i].w;
                const int c = i * TPR + t;
                if (ok && c < nv) ox.store(obase + 16u * c, xv[i]);
            }
        }
        float ss = 0.0f;
#pragma unroll
        for (int i = 0; i < V; ++i) {
            const bool in = i * TPR + t < nv;
            const float a = in ? xv[i].x : 0.0f, b = in ? xv[i].y : 0.0f;
            const float c = in ? xv[i].z : 0.0f, d = in ? xv[i].w : 0.0f;
            ss += a * a;
            ss += b * b;
            ss += c * c;
            ss += d * d;
        }
        if constexpr (TPR <= 64) {
            ss = group_sum<TPR>(ss);
        } else {
            constexpr int WPR = TPR / 64;
            ss = group_sum<64>(ss);
            if ((tid & 63) == 0) part[k & 1][tid >> 6] = ss;
            __syncthreads();
            const int w0 = lr * WPR;
            ss = part[k & 1][w0];
#pragma unroll
            for (int q = 1; q < WPR; ++q) ss += part[k & 1][w0 + q];
        }
        const StreamOut os(p.out + row0 * p.cols, (p.rows - row0) * (int64_t)p.cols * 4);
        if (!ok) return;
        if constexpr (GATED) {
            const float rinv = 1.0f / sqrtf(ss / (float)p.cols + p.eps);
#pragma unroll
            for (int i = 0; i < V; ++i) {
                const int c = i * TPR + t;
                if (c >= nv) continue;
                float4 o;
                o.x = ((xv[i].x * rinv) * wv[i].x) * silu_fast(zv[i].x);
                o.y = ((xv[i].y * rinv) * wv[i].y) * silu_fast(zv[i].y);
                o.z = ((xv[i].z * rinv) * wv[i].z) * silu_fast(zv[i].z);
                o.w = ((xv[i].w * rinv) * wv[i].w) * silu_fast(zv[i].w);
                os.store(obase + 16u * c, o);
            }
        } else {
            const float inv = norm_scale(ss, p);
#pragma unroll
            for (int i = 0; i < V; ++i) {
                const int c = i * TPR + t;
                if (c >= nv) continue;
                float4 w4 = wv[i];
                if (unit) {
                    w4.x = 1.0f + w4.x; w4.y = 1.0f + w4.y;
                    w4.z = 1.0f + w4.z; w4.w = 1.0f + w4.w;
                }
                float4 o = make_float4(xv[i].x * inv, xv[i].y * inv, xv[i].z * inv,
                                       xv[i].w * inv);
                o.x = o.x * w4.x; o.y = o.y * w4.y; o.z = o.z * w4.z; o.w = o.w * w4.w;
                os.store(obase + 16u * c, o);
            }
        }
    };

    const int64_t G = gridDim.x;
    int64_t g = blockIdx.x;
    float4 xa[V], za[V];
    load_rows(g, xa, za);
    for (int k = 0; k < iters - 1; ++k) {
        float4 xb[V], zb[V];
        load_rows(min(g + G, ngroups - 1), xb, zb);
        process(g, k, xa, za);
#pragma unroll
        for (int i = 0; i < V; ++i) {
            xa[i] = xb[i];
            if (TWO) za[i] = zb[i];
        }
        g += G;
    }
    if (g < ngroups) process(g, iters - 1, xa, za);
}

// Any shape / alignment: one 256-thread block per slice, two passes over the
// slice (the second pass hits L2). Same arithmetic as the vector kernel.
template <int MODE>
__global__ __launch_bounds__(256) void norm_scalar_kernel(NormParams p) {
    constexpr bool GATED = MODE == kGated;
    const int64_t row = blockIdx.x;
    const int tid = threadIdx.x;
    const int64_t base = row * (int64_t)p.cols;
    const float* xr = p.x + base;
    float ss = 0.0f;
    if constexpr (MODE == kResid) {
        // each thread reads back only the sums it wrote itself
        float* xo = p.xo + base;
        const float* dr = p.z + base;
        for (int c = tid; c < p.cols; c += 256) {
            const float v = xr[c] + dr[c];
            xo[c] = v;
            ss += v * v;
        }
        xr = xo;
    } else {
        for (int c = tid; c < p.cols; c += 256) ss += xr[c] * xr[c];
    }
    __shared__ float part[4];
    ss = group_sum<64>(ss);
    if ((tid & 63) == 0) part[tid >> 6] = ss;
    __syncthreads();
    ss = ((part[0] + part[1]) + part[2]) + part[3];
    float* o = p.out + base;
    if constexpr (GATED) {
        const float rinv = 1.0f / sqrtf(ss / (float)p.cols + p.eps);
        const float* zr = p.z + base;
        const int64_t col0 = (row % p.gpr) * (int64_t)p.cols;
        for (int c = tid; c < p.cols; c += 256) {
            const float wn = p.w[(col0 + c) % p.w_len];
            o[c] = ((xr[c] * rinv) * wn) * silu_fast(zr[c]);
        }
    } else {
        const float inv = norm_scale(ss, p);
        for (int c = tid; c < p.cols; c += 256)
            o[c] = apply_w(xr[c] * inv, p.w, c, p.flags);
    }
}

// ---------------------------------------------- Gemma sandwich-norm sites
// After a Gemma block's attention and after its FFN (src/model.cpp:213-215,
// 224-231), the sublayer output y is normalised with its post-norm weight,
// scaled by ds, added to the residual stream x, the sum scaled by ss (1 at
// the attention site), and the next norm taken of the result:
//   a = (y * inv(y)) * w1,  x' = (x + ds * a) * ss,  h = (x' * inv(x')) * w2
// with inv(v) = 1/sqrtf(mean(v^2) + eps) and (1+w) weights under
// AERO_NORM_UNIT_OFFSET. One pass reads y and x and writes x' and h, the
// four streams of add + norm, where the reference makes four passes (norm,
// add, norm, and the output-scale pass). Lanes own row chunks as
// norm_vec_kernel; two cross-wave sums.
struct PostParams {
    const float* y;
    const float* x;
    const float* w1;     // post-norm weight (null: ones)
    const float* w2;     // next norm's weight (null: ones)
    float* xo;           // x' (may alias x)
    float* h;
    int64_t rows;
    int cols;
    float eps, ds, ss;
    int flags;
};

__device__ __forceinline__ float4 w4_at(const float* w, int c, int flags) {
    if (w == nullptr) return make_float4(1.f, 1.f, 1.f, 1.f);
    float4 v = reinterpret_cast<const float4*>(w)[c];
    if (flags & AERO_NORM_UNIT_OFFSET) {
        v.x = 1.0f + v.x; v.y = 1.0f + v.y; v.z = 1.0f + v.z; v.w = 1.0f + v.w;
    }
    return v;
}

template <int TPR>
__device__ __forceinline__ float row_sum(float ss, float* part, int tid, int lr) {
    if constexpr (TPR <= 64) {
        return group_sum<TPR>(ss);
    } else {
        constexpr int WPR = TPR / 64;
        ss = group_sum<64>(ss);
        if ((tid & 63) == 0) part[tid >> 6] = ss;
        __syncthreads();
        const int w0 = lr * WPR;
        ss = part[w0];
#pragma unroll
        for (int k = 1; k < WPR; ++k) ss += part[w0 + k];
        return ss;
    }
}

template <int TPR, int V>
__global__ __launch_bounds__(TPR > 256 ? TPR : 256)
void post_norm_add_kernel(PostParams p) {
    constexpr int BS = TPR > 256 ? TPR : 256;
    constexpr int RPB = BS / TPR;
    __shared__ float part1[BS / 64], part2[BS / 64];
    const int tid = threadIdx.x;
    const int lr = tid / TPR;
    const int t = tid % TPR;
    const int64_t row = (int64_t)blockIdx.x * RPB + lr;
    const bool ok = row < p.rows;
    const int nv = p.cols >> 2;
    const int64_t base = ok ? row * (int64_t)p.cols : 0;
    float4 yv[V], xv[V], w1[V];
#pragma unroll
    for (int i = 0; i < V; ++i) {
        const int c = i * TPR + t;
        if (ok && c < nv) {
            yv[i] = ld_stream(p.y + base + 4 * c);
            xv[i] = ld_stream(p.x + base + 4 * c);
            w1[i] = w4_at(p.w1, c, p.flags);
        } else {
            yv[i] = xv[i] = make_float4(0.f, 0.f, 0.f, 0.f);
            w1[i] = make_float4(1.f, 1.f, 1.f, 1.f);
        }
    }
    float s1 = 0.0f;
#pragma unroll
    for (int i = 0; i < V; ++i) {
        s1 += yv[i].x * yv[i].x;
        s1 += yv[i].y * yv[i].y;
        s1 += yv[i].z * yv[i].z;
        s1 += yv[i].w * yv[i].w;
    }
    s1 = row_sum<TPR>(s1, part1, tid, lr);
    const float inv1 = 1.0f / sqrtf(s1 / (float)p.cols + p.eps);
    const int64_t r0 = (int64_t)blockIdx.x * RPB;
    const StreamOut ox(p.xo + r0 * p.cols, (p.rows - r0) * (int64_t)p.cols * 4);
    const uint32_t ob = (uint32_t)(lr * p.cols) * 4u;
    auto step = [&](float y, float w, float x) {
        const float a = (y * inv1) * w;
        return (x + p.ds * a) * p.ss;
    };
    float s2 = 0.0f;
#pragma unroll
    for (int i = 0; i < V; ++i) {
        xv[i].x = step(yv[i].x, w1[i].x, xv[i].x);
        xv[i].y = step(yv[i].y, w1[i].y, xv[i].y);
        xv[i].z = step(yv[i].z, w1[i].z, xv[i].z);
        xv[i].w = step(yv[i].w, w1[i].w, xv[i].w);
        const int c = i * TPR + t;
        if (ok && c < nv) ox.store(ob + 16u * c, xv[i]);
        else xv[i] = make_float4(0.f, 0.f, 0.f, 0.f);
        s2 += xv[i].x * xv[i].x;
        s2 += xv[i].y * xv[i].y;
        s2 += xv[i].z * xv[i].z;
        s2 += xv[i].w * xv[i].w;
    }
    s2 = row_sum<TPR>(s2, part2, tid, lr);
    const float inv2 = 1.0f / sqrtf(s2 / (float)p.cols + p.eps);
    const StreamOut oh(p.h + r0 * p.cols, (p.rows - r0) * (int64_t)p.cols * 4);
    if (!ok) return;
#pragma unroll
    for (int i = 0; i < V; ++i) {
        const int c = i * TPR + t;
        if (c >= nv) continue;
        const float4 w = w4_at(p.w2, c, p.flags);
        const float4 o = make_float4((xv[i].x * inv2) * w.x, (xv[i].y * inv2) * w.y,
                                     (xv[i].z * inv2) * w.z, (xv[i].w * inv2) * w.w);
        oh.store(ob + 16u * c, o);
    }
}

// Any shape / alignment: one 256-lane workgroup a row, the same arithmetic;
// x' is read back only by the lane that wrote it.
__global__ __launch_bounds__(256) void post_norm_add_scalar_kernel(PostParams p) {
    const int64_t row = blockIdx.x;
    const int tid = threadIdx.x;
    const int64_t base = row * (int64_t)p.cols;
    __shared__ float part[4];
    auto wv = [&](const float* w, int c) {
        if (w == nullptr) return 1.0f;
        return (p.flags & AERO_NORM_UNIT_OFFSET) ? 1.0f + w[c] : w[c];
    };
    float s1 = 0.0f;
    for (int c = tid; c < p.cols; c += 256) s1 += p.y[base + c] * p.y[base + c];
    s1 = group_sum<64>(s1);
    if ((tid & 63) == 0) part[tid >> 6] = s1;
    __syncthreads();
    s1 = ((part[0] + part[1]) + part[2]) + part[3];
    __syncthreads();
    const float inv1 = 1.0f / sqrtf(s1 / (float)p.cols + p.eps);
    float s2 = 0.0f;
    for (int c = tid; c < p.cols; c += 256) {
        const float a = (p.y[base + c] * inv1) * wv(p.w1, c);
        const float v = (p.x[base + c] + p.ds * a) * p.ss;
        p.xo[base + c] = v;
        s2 += v * v;
    }
    s2 = group_sum<64>(s2);
    if ((tid & 63) == 0) part[tid >> 6] = s2;
    __syncthreads();
    s2 = ((part[0] + part[1]) + part[2]) + part[3];
    const float inv2 = 1.0f / sqrtf(s2 / (float)p.cols + p.eps);
    for (int c = tid; c < p.cols; c += 256)
        p.h[base + c] = (p.xo[base + c] * inv2) * wv(p.w2, c);
}

using PostKernel = void (*)(PostParams);

template <int TPR>
PostKernel pick_post_v(int v) {
    switch (v) {
    case 1: return post_norm_add_kernel<TPR, 1>;
    case 2: return post_norm_add_kernel<TPR, 2>;
    case 3: return post_norm_add_kernel<TPR, 3>;
    case 4: return post_norm_add_kernel<TPR, 4>;
    case 5: return post_norm_add_kernel<TPR, 5>;
    case 6: return post_norm_add_kernel<TPR, 6>;
    case 7: return post_norm_add_kernel<TPR, 7>;
    case 8: return post_norm_add_kernel<TPR, 8>;
    default: return nullptr;
    }
}

PostKernel pick_post(int tpr, int v) {
    switch (tpr) {
    case 8: return pick_post_v<8>(v);
    case 16: return pick_post_v<16>(v);
    case 32: return pick_post_v<32>(v);
    case 64: return pick_post_v<64>(v);
    case 128: return pick_post_v<128>(v);
    case 256: return pick_post_v<256>(v);
    case 512: return pick_post_v<512>(v);
    case 1024: return pick_post_v<1024>(v);
    default: return nullptr;
    }
}

using NormKernel = void (*)(NormParams);
using NormLoopKernel = void (*)(NormParams, int);

template <int MODE, int TPR>
NormLoopKernel pick_loop_v(int v) {
    switch (v) {
    case 1: return norm_loop_kernel<TPR, 1, MODE>;
    case 2: return norm_loop_kernel<TPR, 2, MODE>;
    case 3: return norm_loop_kernel<TPR, 3, MODE>;
    case 4: return norm_loop_kernel<TPR, 4, MODE>;
    case 8: return norm_loop_kernel<TPR, 8, MODE>;
    default: return nullptr;
    }
}

template <int MODE>
NormLoopKernel pick_loop(int tpr, int v) {
    switch (tpr) {
    case 8: return pick_loop_v<MODE, 8>(v);
    case 16: return pick_loop_v<MODE, 16>(v);
    case 32: return pick_loop_v<MODE, 32>(v);
    case 64: return pick_loop_v<MODE, 64>(v);
    case 128: return pick_loop_v<MODE, 128>(v);
    case 256: return pick_loop_v<MODE, 256>(v);
    case 512: return pick_loop_v<MODE, 512>(v);
    case 1024: return pick_loop_v<MODE, 1024>(v);
    default: return nullptr;
    }
}

template <int MODE, int TPR>
NormKernel pick_v(int v) {
    switch (v) {
    case 1: return norm_vec_kernel<TPR, 1, MODE>;
    case 2: return norm_vec_kernel<TPR, 2, MODE>;
    case 3: return norm_vec_kernel<TPR, 3, MODE>;
    case 4: return norm_vec_kernel<TPR, 4, MODE>;
    case 5: return norm_vec_kernel<TPR, 5, MODE>;
    case 6: return norm_vec_kernel<TPR, 6, MODE>;
    case 7: return norm_vec_kernel<TPR, 7, MODE>;
    case 8: return norm_vec_kernel<TPR, 8, MODE>;
    default: return nullptr;
    }
}

// one or two waves a row with 16 or 32 float4 a lane (wide rows, no or one
// cross-wave step)
template <int MODE, int TPR>
NormKernel pick_wide(int v) {
    if (v <= 8) return pick_v<MODE, TPR>(v);
    if (v <= 16) return norm_vec_kernel<TPR, 16, MODE>;
    if (v <= 32) return norm_vec_kernel<TPR, 32, MODE>;
    return nullptr;
}

template <int MODE>
NormKernel pick(int tpr, int v) {
    switch (tpr) {
    case 8: return pick_v<MODE, 8>(v);
    case 16: return pick_v<MODE, 16>(v);
    case 32: return pick_v<MODE, 32>(v);
    case 64: return pick_wide<MODE, 64>(v);
    case 128: return pick_wide<MODE, 128>(v);
    case 256: return pick_v<MODE, 256>(v);
    case 512: return pick_v<MODE, 512>(v);
    case 1024: return pick_v<MODE, 1024>(v);
    default: return nullptr;
    }
}

// Lanes per slice: the smallest power of two (8..1024) that keeps each lane
// at <= vmax float4 (4 by default, so a lane has four 128-bit loads, eight
// when gated, in flight); V then covers the rest.
void choose_shape(int nv, int vmax, int* tpr, int* v) {
    int t = 8;
    // more than 8 float4 a lane exist for whole-wave rows only (64 or 128 lanes)
    while (t < 1024 && (t * vmax < nv || (vmax > 8 && t < 64))) t *= 2;
    // a row that t lanes leave ragged but half as many fit exactly (2560
    // columns: 256 x 3 float4 leave a sixth of the lanes idle, 128 x 5 fit)
    // takes the exact fit: 15.84 -> 15.08 us for add + RMSNorm at 2048 x 2560
    // on MI355X, RMSNorm the same
    if (vmax <= 4 && nv % t != 0 && t >= 16 && nv % (t / 2) == 0 && nv / (t / 2) <= 8) t /= 2;
    *tpr = t;
    *v = (nv + t - 1) / t;
}

bool run_norm(NormParams p, int mode, hipStream_t stream) {
    if (p.rows == 0) return true;
    const bool vec = (p.cols % 4 == 0) && aligned16(p.x) && aligned16(p.out) &&
                     (p.w == nullptr || aligned16(p.w)) &&
                     (mode != kGated || (aligned16(p.z) && p.w_len % 4 == 0)) &&
                     (mode != kResid || (aligned16(p.z) && aligned16(p.xo)));
    int tpr = 0, v = 0;
    if (vec) choose_shape(p.cols / 4, tune("norm_vmax", 4), &tpr, &v);
    if (vec && (v <= 8 || ((tpr == 64 || tpr == 128) && v <= 32))) {
        const int bs = tpr > 256 ? tpr : 256;
        const int rpb = bs / tpr;
        const int64_t blocks = (p.rows + rpb - 1) / rpb;
        // many rows: the persistent form, `norm_loop` workgroups per CU
        const int per_cu = tune("norm_loop", 0);
        const int64_t G = (int64_t)per_cu * cu_count();
        if (per_cu > 0 && blocks > G && (v <= 4 || v == 8) &&
            (mode != kGated || p.cols % p.w_len == 0)) {
            NormLoopKernel k = mode == kGated ? pick_loop<kGated>(tpr, v)
                               : mode == kResid ? pick_loop<kResid>(tpr, v)
                                                : pick_loop<kPlain>(tpr, v);
            const int iters = (int)((blocks + G - 1) / G);
            return launch("norm_loop_kernel", k, dim3((unsigned)G), dim3(bs), 0, stream, p,
                          iters);
        }
        NormKernel k = mode == kGated ? pick<kGated>(tpr, v)
                       : mode == kResid ? pick<kResid>(tpr, v) : pick<kPlain>(tpr, v);
        return launch("norm_vec_kernel", k, dim3((unsigned)blocks), dim3(bs), 0,
                      stream, p);
    }
    NormKernel k = mode == kGated ? norm_scalar_kernel<kGated>
                   : mode == kResid ? norm_scalar_kernel<kResid> : norm_scalar_kernel<kPlain>;
    return launch("norm_scalar_kernel", k, dim3((unsigned)p.rows), dim3(256), 0,
                  stream, p);
}

bool run_post_norm_add(const PostParams& p, hipStream_t stream) {
    if (p.rows == 0) return true;
    const bool vec = (p.cols % 4 == 0) && aligned16(p.y) && aligned16(p.x) && aligned16(p.xo) &&
                     aligned16(p.h) && (p.w1 == nullptr || aligned16(p.w1)) &&
                     (p.w2 == nullptr || aligned16(p.w2));
    int tpr = 0, v = 0;
    if (vec) choose_shape(p.cols / 4, 4, &tpr, &v);
    if (vec && v <= 8) {
        const int bs = tpr > 256 ? tpr : 256;
        const int64_t blocks = (p.rows + bs / tpr - 1) / (bs / tpr);
        return launch("post_norm_add_kernel", pick_post(tpr, v), dim3((unsigned)blocks), dim3(bs),
                      0, stream, p);
    }
    return launch("post_norm_add_scalar_kernel", post_norm_add_scalar_kernel,
                  dim3((unsigned)p.rows), dim3(256), 0, stream, p);
}

}  // namespace

// Used by the host-pointer ABI (dropin.hip).
bool norm_rows(const float* x, const float* w, float* out, int64_t rows,
               int64_t cols, float eps, int flags, hipStream_t stream) {
    if (x == nullptr || out == nullptr || rows < 0 || cols <= 0 ||
        cols > (int64_t)0x7fffffff || rows > (int64_t)0x7fffffff) {
        set_error("rmsnorm: bad arguments (rows=%lld cols=%lld)", (long long)rows,
                  (long long)cols);
        return false;
    }
    NormParams p{x, nullptr, w, out, rows, (int)cols, 1, (int)cols, eps, flags, nullptr};
    return run_norm(p, kPlain, stream);
}

}  // namespace aero

extern "C" {

int aero_hip_rmsnorm(const float* x, const float* w, float* out, int64_t rows,
                     int64_t cols, float eps, int flags, void* stream) {
    return aero::norm_rows(x, w, out, rows, cols, eps, flags, (hipStream_t)stream)
               ? 1 : 0;
}

int aero_hip_gated_rmsnorm_silu(const float* x, const float* z, const float* w,
                                int64_t w_len, float* out, int64_t rows,
                                int64_t inner, int64_t group, float eps,
                                void* stream) {
    if (!x || !z || !w || !out || rows < 0 || inner <= 0 || group <= 0 ||
        w_len <= 0 || inner % group != 0 || inner > (int64_t)0x7fffffff) {
        aero::set_error("gated_rmsnorm_silu: bad arguments (rows=%lld inner=%lld "
                        "group=%lld w_len=%lld)", (long long)rows, (long long)inner,
                        (long long)group, (long long)w_len);
        return 0;
    }
    const int64_t slices = rows * (inner / group);
    if (slices > (int64_t)0x7fffffff) {
        aero::set_error("gated_rmsnorm_silu: too many slices (%lld)", (long long)slices);
        return 0;
    }
    aero::NormParams p{x, z, w, out, slices, (int)group, (int)(inner / group),
                       (int)w_len, eps, 0, nullptr};
    return aero::run_norm(p, aero::kGated, (hipStream_t)stream) ? 1 : 0;
}

int aero_hip_add_rmsnorm(const float* x, const float* d, float* x_out, const float* w,
                         float* h, int64_t rows, int64_t cols, float eps, int flags,
                         void* stream) {
    if (!x || !d || !x_out || !h || rows < 0 || cols <= 0 || cols > (int64_t)0x7fffffff ||
        rows > (int64_t)0x7fffffff || (flags & ~AERO_NORM_UNIT_OFFSET) != 0) {
        aero::set_error("add_rmsnorm: bad arguments (rows=%lld cols=%lld flags=%d)",
                        (long long)rows, (long long)cols, flags);
        return 0;
    }
    if (h == x || h == d || h == x_out) {
        aero::set_error("add_rmsnorm: h must not alias x, d or x_out");
        return 0;
    }
    aero::NormParams p{x, d, w, h, rows, (int)cols, 1, (int)cols, eps, flags, x_out};
    return aero::run_norm(p, aero::kResid, (hipStream_t)stream) ? 1 : 0;
}

int aero_hip_post_norm_add(const float* y, const float* x, float* x_out, const float* w_post,
                           float ds, float ss, const float* w_next, float* h, int64_t rows,
                           int64_t cols, float eps, int flags, void* stream) {
    if (!y || !x || !x_out || !h || rows < 0 || cols <= 0 || cols > (int64_t)0x7fffffff ||
        rows > (int64_t)0x7fffffff || (flags & ~AERO_NORM_UNIT_OFFSET) != 0) {
        aero::set_error("post_norm_add: bad arguments (rows=%lld cols=%lld flags=%d)",
                        (long long)rows, (long long)cols, flags);
        return 0;
    }
    if (h == y || h == x || h == x_out || y == x_out) {
        aero::set_error("post_norm_add: h must not alias y, x or x_out, nor x_out y");
        return 0;
    }
    aero::PostParams p{y, x, w_post, w_next, x_out, h, rows, (int)cols, eps, ds, ss, flags};
    return aero::run_post_norm_add(p, (hipStream_t)stream) ? 1 : 0;
}

}  // extern "C"
