// Activation * multiply on gfx950: SwiGLU (silu(g)*u), GeGLU with the erf
// GELU of the reference (Abramowitz & Stegun 7.1.26) or the tanh
// approximation, unary silu/gelu, and the plain product.
//
// Pure streaming: each lane loads one float4 of gate and of up with the
// nontemporal hint and writes one float4 back the same way; occupancy (many
// 64-lane blocks) keeps the loads in flight. HBM bytes per element: 12
// (gate, up, out), 8 unary.
// One pass replaces the reference's gelu_ then mul_ two-pass sequence.
//
// Arithmetic follows src/tensor.cpp:47-59,104-125 with contraction off:
// silu(g) = g * (1/(1+expf(-g))); gelu(g) = (0.5*g)*(1+erf(g*0.70710678))
// with the A&S polynomial evaluated in the reference's order; then *up.
#include "act_ops.hpp"

#pragma clang fp contract(off)

namespace aero {
namespace {

template <int KIND, bool UP>
__device__ __forceinline__ float4 act4(float4 g, float4 u) {
    float4 o;
    o.x = act<KIND>(g.x);
    o.y = act<KIND>(g.y);
    o.z = act<KIND>(g.z);
    o.w = act<KIND>(g.w);
    if constexpr (UP) {
        o.x = o.x * u.x; o.y = o.y * u.y; o.z = o.z * u.z; o.w = o.w * u.w;
    }
    return o;
}

constexpr int kActBlock = 256;  // scalar-tail block

// n4 float4 elements; block b covers [b*BS*U, (b+1)*BS*U) with lane stride
// BS, so each load instruction of a wave touches 1 KiB contiguous. gate and
// up stream in and out stream back with the nontemporal hint.
template <int KIND, bool UP, int U, int BS>
__global__ __launch_bounds__(BS)
void act_vec_kernel(const float* g, const float* u, float* out, int64_t n4) {
    const int64_t base = (int64_t)blockIdx.x * (BS * U) + threadIdx.x;
    float4 gv[U];
    float4 uv[U];
#pragma unroll
    for (int i = 0; i < U; ++i) {
        const int64_t idx = base + (int64_t)i * BS;
        if (idx < n4) {
            gv[i] = ld_stream(g + 4 * idx);
            if constexpr (UP) uv[i] = ld_stream(u + 4 * idx);
        }
    }
    const int64_t first = (int64_t)blockIdx.x * (BS * U);
    const StreamOut o(out + 4 * first, (n4 - first) * 16);
#pragma unroll
    for (int i = 0; i < U; ++i) {
        const int64_t idx = base + (int64_t)i * BS;
        if (idx < n4)
            o.store((uint32_t)((idx - first) * 16), act4<KIND, UP>(gv[i], UP ? uv[i] : gv[i]));
    }
}

// Persistent form: a grid of a few workgroups per CU, workgroup b taking
// chunks b, b + G, ... of BS float4 (`iters` rounds, the last one partial),
// with the next chunk's loads issued before this chunk's stores. Loads read
// clamped indices unconditionally; stores past the end are skipped.
template <int KIND, bool UP, int BS>
__global__ __launch_bounds__(BS)
void act_loop_kernel(const float* g, const float* u, float* out, int64_t n4, int iters) {
    const int64_t G = gridDim.x;
    int64_t chunk = blockIdx.x;
    auto ld = [&](int64_t c, float4& gv, float4& uv) {
        const int64_t idx = min(c * BS + threadIdx.x, n4 - 1);
        gv = ld_stream(g + 4 * idx);
        if constexpr (UP) uv = ld_stream(u + 4 * idx);
    };
    auto st = [&](int64_t c, float4 gv, float4 uv) {
        const int64_t first = c * BS;
        const StreamOut o(out + 4 * first, (n4 - first) * 16);
        if (first + threadIdx.x < n4)
            o.store((uint32_t)threadIdx.x * 16u, act4<KIND, UP>(gv, UP ? uv : gv));
    };
    float4 ga, ua = make_float4(0.f, 0.f, 0.f, 0.f);
    ld(chunk, ga, ua);
    const int64_t nchunks = (n4 + BS - 1) / BS;
    for (int k = 0; k < iters - 1; ++k) {
        float4 gb, ub = make_float4(0.f, 0.f, 0.f, 0.f);
        ld(min(chunk + G, nchunks - 1), gb, ub);
        st(chunk, ga, ua);
        ga = gb;
        ua = ub;
        chunk += G;
    }
    if (chunk < nchunks) st(chunk, ga, ua);
}

// Store-only stream (dst = value): the write-only counterpart of the copy,
// one float4 a lane in 256-lane blocks (64-lane blocks of one store each
// measured 0.60 of peak at 1 GiB, 256-lane blocks 0.84, the copy's rate),
// NT stores like every output here.
__global__ __launch_bounds__(256) void fill_kernel(float* out, float value, int64_t n4) {
    const int64_t first = (int64_t)blockIdx.x * 256;
    const StreamOut o(out + 4 * first, (n4 - first) * 16);
    if (first + threadIdx.x < n4)
        o.store((uint32_t)threadIdx.x * 16u, make_float4(value, value, value, value));
}

// Scalar form for unaligned pointers and the n % 4 tail.
template <int KIND, bool UP>
__global__ __launch_bounds__(kActBlock)
void act_scalar_kernel(const float* g, const float* u, float* out, int64_t n) {
    const int64_t i = (int64_t)blockIdx.x * kActBlock + threadIdx.x;
    if (i >= n) return;
    const float a = act<KIND>(g[i]);
    out[i] = UP ? a * u[i] : a;
}

template <int KIND, bool UP, int U>
bool launch_vec(int bs, const float* g, const float* u, float* out, int64_t n4, hipStream_t s) {
    const int64_t per_block = (int64_t)bs * U;
    const int64_t blocks = (n4 + per_block - 1) / per_block;
    if (blocks > 0x7fffffff) {
        set_error("act_mul: too many elements (%lld float4)", (long long)n4);
        return false;
    }
    switch (bs) {
    case 64:
        return launch("act_vec_kernel", act_vec_kernel<KIND, UP, U, 64>, dim3((unsigned)blocks),
                      dim3(64), 0, s, g, u, out, n4);
    case 128:
        return launch("act_vec_kernel", act_vec_kernel<KIND, UP, U, 128>, dim3((unsigned)blocks),
                      dim3(128), 0, s, g, u, out, n4);
    default:
        return launch("act_vec_kernel", act_vec_kernel<KIND, UP, U, 256>, dim3((unsigned)blocks),
                      dim3(256), 0, s, g, u, out, n4);
    }
}

// Launch shape: one float4 of each input per lane and 64-lane blocks (the
// measured best on MI355X from 88 MB to 5.6 GB per launch).
template <int KIND, bool UP>
bool run_act(const float* g, const float* u, float* out, int64_t n, hipStream_t s) {
    const bool vec = aligned16(g) && aligned16(out) && (!UP || aligned16(u));
    int64_t done = 0;
    if (vec) {
        const int64_t n4 = n / 4;
        if (n4 > 0) {
            const int bs = tune("act_bs", 64);
            const int per_cu = tune("act_grid", 0);
            const int64_t G = (int64_t)per_cu * cu_count();
            const int64_t chunks = (n4 + bs - 1) / bs;
            if (per_cu > 0 && chunks > G) {
                const int iters = (int)((chunks + G - 1) / G);
                bool ok2;
                if (bs == 256)
                    ok2 = launch("act_loop_kernel", act_loop_kernel<KIND, UP, 256>,
                                 dim3((unsigned)G), dim3(256), 0, s, g, u, out, n4, iters);
                else
                    ok2 = launch("act_loop_kernel", act_loop_kernel<KIND, UP, 64>,
                                 dim3((unsigned)G), dim3(64), 0, s, g, u, out, n4, iters);
                if (!ok2) return false;
                done = n4 * 4;
                goto tail;
            }
            const bool ok = tune("act_u", 1) == 2
                                ? launch_vec<KIND, UP, 2>(bs, g, u, out, n4, s)
                                : launch_vec<KIND, UP, 1>(bs, g, u, out, n4, s);
            if (!ok) return false;
        }
        done = n4 * 4;
    }
tail:
    const int64_t rest = n - done;
    if (rest > 0) {
        const int64_t blocks = (rest + kActBlock - 1) / kActBlock;
        if (blocks > 0x7fffffff) {
            set_error("act_mul: n too large (%lld)", (long long)n);
            return false;
        }
        return launch("act_scalar_kernel", act_scalar_kernel<KIND, UP>,
                      dim3((unsigned)blocks), dim3(kActBlock), 0, s, g + done,
                      UP ? u + done : u, out + done, rest);
    }
    return true;
}

template <int KIND>
bool run_act_kind(const float* g, const float* u, float* out, int64_t n, hipStream_t s) {
    return u ? run_act<KIND, true>(g, u, out, n, s) : run_act<KIND, false>(g, u, out, n, s);
}

}  // namespace

bool act_mul(int kind, const float* g, const float* u, float* out, int64_t n,
             hipStream_t s) {
    if (g == nullptr || out == nullptr || n < 0) {
        set_error("act_mul: bad arguments");
        return false;
    }
    if (n == 0) return true;
    switch (kind) {
    case AERO_ACT_SILU: return run_act_kind<AERO_ACT_SILU>(g, u, out, n, s);
    case AERO_ACT_GELU: return run_act_kind<AERO_ACT_GELU>(g, u, out, n, s);
    case AERO_ACT_GELU_TANH: return run_act_kind<AERO_ACT_GELU_TANH>(g, u, out, n, s);
    case AERO_ACT_SIGMOID: return run_act_kind<AERO_ACT_SIGMOID>(g, u, out, n, s);
    case AERO_ACT_IDENTITY:
        if (u == nullptr) {
            set_error("act_mul: identity needs `up`");
            return false;
        }
        return run_act_kind<AERO_ACT_IDENTITY>(g, u, out, n, s);
    default:
        set_error("act_mul: unknown kind %d", kind);
        return false;
    }
}

}  // namespace aero

extern "C" {

int aero_hip_act_mul(int kind, const float* gate, const float* up, float* out,
                     int64_t n, void* stream) {
    return aero::act_mul(kind, gate, up, out, n, (hipStream_t)stream) ? 1 : 0;
}

int aero_hip_copy_f32(const float* src, float* dst, int64_t n, void* stream) {
    if (!src || !dst || n < 0 || n % 4 != 0 || !aero::aligned16(src) ||
        !aero::aligned16(dst)) {
        aero::set_error("copy_f32: needs 16-byte aligned pointers and n %% 4 == 0");
        return 0;
    }
    // unary identity through the streaming kernel: a plain read-once,
    // write-once copy with the same access pattern as act_mul
    return aero::run_act<AERO_ACT_IDENTITY, false>(src, nullptr, dst, n, (hipStream_t)stream)
               ? 1 : 0;
}

int aero_hip_fill_f32(float* dst, float value, int64_t n, void* stream) {
    if (!dst || n < 0 || n % 4 != 0 || !aero::aligned16(dst) || n / 4 / 256 >= 0x7fffffff) {
        aero::set_error("fill_f32: needs a 16-byte aligned pointer and n %% 4 == 0");
        return 0;
    }
    if (n == 0) return 1;
    const int64_t blocks = (n / 4 + 255) / 256;
    return aero::launch("fill_kernel", aero::fill_kernel, dim3((unsigned)blocks), dim3(256), 0,
                        (hipStream_t)stream, dst, value, n / 4) ? 1 : 0;
}

}  // extern "C"
