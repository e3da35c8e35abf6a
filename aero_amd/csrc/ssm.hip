// Gated DeltaNet on gfx950: the reference's delta-rule scan and causal
// depthwise conv (src/ssm.cpp:17-210).
//
// Per token t and value head h (key head kk = h % n_k):
//   qn, kn = q[t, kk], k[t, kk] / max(||.||, eps)
//   dec = exp(min(a_log[h] * softplus(alpha[t, h] + dt_bias[h]), 0))
//   b = sigmoid(beta[t, h])
//   S_h = dec * S_h;  v_new = (v[t, h] - kn^T S_h) * b;  S_h += kn v_new^T
//   out[t, h] = scale * qn^T S_h
// S_h is d x d (row i = key element, column e = value element). Column e of
// S_h evolves on its own: it needs only kn, qn, v[e], dec and b. So the scan
// keeps each column in registers for the whole call: P lanes share a column
// (each holding d/P of its rows), a wave holds 64/P columns, a workgroup of
// four waves 256/P columns of one head. A token costs each lane d/P
// multiplies, three d/P-long dot/update passes and two log2(P)-step lane
// reductions; the state is read and written once per call.
//
// ssm_prep_kernel computes qn, kn, dec and b for every token first (one wave
// a token and key head), so the serial loop only streams them.
//
// Sums run in another order than the reference's serial loops, and exp /
// log1p / sqrt are the GPU's: <= 1e-5 relative to the output's scale. The conv
// adds its taps in the reference's order with separate multiplies and adds:
// bit-exact.
#include "common.hpp"
#include "aero_hip.h"

#include <cmath>

namespace aero {

namespace {

constexpr int kScanThreads = 256;

__device__ __forceinline__ float softplus_dev(float x) {
    return log1pf(expf(-fabsf(x))) + (x > 0.0f ? x : 0.0f);
}

// One wave per (token t, key head kk): qn, kn; the wave of kk == 0 also
// writes dec and b of token t for every value head.
__global__ __launch_bounds__(64) void ssm_prep_kernel(
    const float* __restrict__ q, const float* __restrict__ k, const float* __restrict__ alpha,
    const float* __restrict__ beta, const float* __restrict__ a_log,
    const float* __restrict__ dt_bias, float* __restrict__ qn, float* __restrict__ kn,
    float* __restrict__ dec, float* __restrict__ bb, int64_t n_k, int64_t n_v, int64_t d,
    float eps) {
    const int64_t row = blockIdx.x;  // t * n_k + kk
    const int64_t t = row / n_k, kk = row % n_k;
    const int lane = threadIdx.x;
    const float* qr = q + row * d;
    const float* kr = k + row * d;
    float sq = 0.0f, sk = 0.0f;
    for (int64_t i = lane; i < d; i += 64) {
        sq += qr[i] * qr[i];
        sk += kr[i] * kr[i];
    }
    sq = group_sum<64>(sq);
    sk = group_sum<64>(sk);
    const float nq = fmaxf(sqrtf(sq), eps), nk = fmaxf(sqrtf(sk), eps);
    for (int64_t i = lane; i < d; i += 64) {
        qn[row * d + i] = qr[i] / nq;
        kn[row * d + i] = kr[i] / nk;
    }
    if (kk == 0) {
        for (int64_t h = lane; h < n_v; h += 64) {
            float g = a_log[h] * softplus_dev(alpha[t * n_v + h] + dt_bias[h]);
            if (g > 0.0f) g = 0.0f;
            dec[t * n_v + h] = expf(g);
            bb[t * n_v + h] = 1.0f / (1.0f + expf(-beta[t * n_v + h]));
        }
    }
}

// P lanes a column, RPT = D / P rows each; lane = part * CPW + ci.
template <int D, int P>
__global__ __launch_bounds__(kScanThreads) void ssm_scan_kernel(
    const float* __restrict__ qn, const float* __restrict__ kn, const float* __restrict__ v,
    const float* __restrict__ dec, const float* __restrict__ bb, float* __restrict__ state,
    float* __restrict__ outs, int64_t T, int64_t n_k, int64_t n_v, float scale) {
    constexpr int RPT = D / P;        // rows a lane holds
    constexpr int CPW = 64 / P;       // columns a wave holds
    constexpr int CW = 4 * CPW;       // columns a workgroup holds
    static_assert(RPT % 4 == 0, "rows a lane must be whole float4s");
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int part = lane / CPW, ci = lane % CPW;
    const int64_t h = blockIdx.x;
    const int64_t kk = h % n_k;
    const int e = (int)blockIdx.y * CW + wave * CPW + ci;  // this lane's column
    const int i0 = part * RPT;                              // its first row

    float* S = state + h * (int64_t)D * D;
    float s[RPT];
#pragma unroll
    for (int j = 0; j < RPT; ++j) s[j] = S[(int64_t)(i0 + j) * D + e];

    // token t's operands; the next token's are loaded while t is computed
    // (the last token's again at the end: in bounds, no branch)
    float kc[RPT], qc[RPT], kx[RPT], qx[RPT];
    float vc, dc, bc, vx, dx, bx;
    auto load = [&](int64_t t, float (&kr)[RPT], float (&qr)[RPT], float& vr, float& dr,
                    float& br) {
        const float4* k4 = reinterpret_cast<const float4*>(kn + (t * n_k + kk) * D + i0);
        const float4* q4 = reinterpret_cast<const float4*>(qn + (t * n_k + kk) * D + i0);
#pragma unroll
        for (int j = 0; j < RPT / 4; ++j) {
            const float4 a = k4[j], c = q4[j];
            kr[4 * j] = a.x; kr[4 * j + 1] = a.y; kr[4 * j + 2] = a.z; kr[4 * j + 3] = a.w;
            qr[4 * j] = c.x; qr[4 * j + 1] = c.y; qr[4 * j + 2] = c.z; qr[4 * j + 3] = c.w;
        }
        vr = v[(t * n_v + h) * D + e];
        dr = dec[t * n_v + h];
        br = bb[t * n_v + h];
    };
    load(0, kc, qc, vc, dc, bc);
    for (int64_t t = 0; t < T; ++t) {
        load(min(t + 1, T - 1), kx, qx, vx, dx, bx);
        float p0 = 0.0f, p1 = 0.0f;
#pragma unroll
        for (int j = 0; j < RPT; j += 2) {
            s[j] *= dc;
            s[j + 1] *= dc;
            p0 = __builtin_fmaf(kc[j], s[j], p0);
            p1 = __builtin_fmaf(kc[j + 1], s[j + 1], p1);
        }
        float vp = p0 + p1;
#pragma unroll
        for (int m = CPW; m < 64; m <<= 1) vp += __shfl_xor(vp, m);
        const float vnew = (vc - vp) * bc;
        float o0 = 0.0f, o1 = 0.0f;
#pragma unroll
        for (int j = 0; j < RPT; j += 2) {
            s[j] = __builtin_fmaf(kc[j], vnew, s[j]);
            s[j + 1] = __builtin_fmaf(kc[j + 1], vnew, s[j + 1]);
            o0 = __builtin_fmaf(qc[j], s[j], o0);
            o1 = __builtin_fmaf(qc[j + 1], s[j + 1], o1);
        }
        float o = o0 + o1;
#pragma unroll
        for (int m = CPW; m < 64; m <<= 1) o += __shfl_xor(o, m);
        if (part == 0) outs[(t * n_v + h) * D + e] = scale * o;
#pragma unroll
        for (int j = 0; j < RPT; ++j) {
            kc[j] = kx[j];
            qc[j] = qx[j];
        }
        vc = vx;
        dc = dx;
        bc = bx;
    }
#pragma unroll
    for (int j = 0; j < RPT; ++j) S[(int64_t)(i0 + j) * D + e] = s[j];
}

// out[t, c] = sum_j buf[tl + t + 1 - K + j, c] * w[c, j] over the rows that
// exist, buf = [tail (tl rows); x], taps in order, tap 0 the oldest.
__global__ __launch_bounds__(256) void ssm_conv_kernel(const float* __restrict__ x,
                                                       const float* __restrict__ w,
                                                       const float* __restrict__ tail,
                                                       float* __restrict__ out, int64_t tl,
                                                       int64_t T, int64_t C, int K) {
    const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (idx >= T * C) return;
    const int64_t t = idx / C, c = idx % C;
    float acc = 0.0f;
    for (int j = 0; j < K; ++j) {
        const int64_t b = tl + t + 1 - K + j;
        if (b < 0) continue;
        const float in = b < tl ? tail[b * C + c] : x[(b - tl) * C + c];
        acc = acc + in * w[c * K + j];
    }
    out[idx] = acc;
}

// The new tail: the last keep rows of buf, per channel; a lane reads all of
// its channel's rows before writing any, so tail_out may be tail.
constexpr int kMaxConvKeep = 15;
__global__ __launch_bounds__(256) void ssm_conv_tail_kernel(const float* __restrict__ x,
                                                            const float* tail, float* tail_out,
                                                            int64_t tl, int64_t T, int64_t C,
                                                            int keep) {
    const int64_t c = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (c >= C) return;
    const int64_t n = tl + T;
    float r[kMaxConvKeep];
#pragma unroll
    for (int i = 0; i < kMaxConvKeep; ++i) {
        if (i >= keep) break;
        const int64_t b = n - keep + i;
        r[i] = b < tl ? tail[b * C + c] : x[(b - tl) * C + c];
    }
#pragma unroll
    for (int i = 0; i < kMaxConvKeep; ++i) {
        if (i >= keep) break;
        tail_out[(int64_t)i * C + c] = r[i];
    }
}

using ScanKernel = void (*)(const float*, const float*, const float*, const float*,
                            const float*, float*, float*, int64_t, int64_t, int64_t, float);

ScanKernel pick_scan(int64_t d, int p) {
    if (d == 128) return p == 16 ? ssm_scan_kernel<128, 16> : ssm_scan_kernel<128, 8>;
    if (d == 64) return p == 16 ? ssm_scan_kernel<64, 16> : ssm_scan_kernel<64, 8>;
    if (d == 256) return ssm_scan_kernel<256, 16>;
    return nullptr;
}

}  // namespace

int64_t ssm_workspace_bytes(int64_t T, int64_t n_k, int64_t n_v, int64_t d) {
    if (T <= 0 || n_k <= 0 || n_v <= 0 || d <= 0) return 0;
    const auto up = [](int64_t b) { return (b + 255) / 256 * 256; };
    return 2 * up(T * n_k * d * 4) + 2 * up(T * n_v * 4);
}

bool ssm_scan_dev(const float* q, const float* k, const float* v, const float* alpha,
                  const float* beta, const float* a_log, const float* dt_bias, float* state,
                  int64_t T, int64_t n_k, int64_t n_v, int64_t d, float scale, float eps,
                  float* outs, void* workspace, int64_t ws_bytes, hipStream_t s) {
    if (T < 0 || n_k <= 0 || n_v <= 0 || n_v % n_k || d <= 0) {
        set_error("ssm_scan: bad sizes (T=%lld n_k=%lld n_v=%lld d=%lld)", (long long)T,
                  (long long)n_k, (long long)n_v, (long long)d);
        return false;
    }
    if (T == 0) return true;
    if (!q || !k || !v || !alpha || !beta || !a_log || !dt_bias || !state || !outs) {
        set_error("ssm_scan: null pointer");
        return false;
    }
    const int p = tune("ssm_parts", 8);
    ScanKernel kern = pick_scan(d, p);
    if (kern == nullptr) {
        set_error("ssm_scan: head dim %lld not in {64, 128, 256}", (long long)d);
        return false;
    }
    const int P = d == 256 ? 16 : (p == 16 ? 16 : 8);
    if (!aligned16(q) || !aligned16(k) || !aligned16(state) || !aligned16(workspace)) {
        set_error("ssm_scan: q, k, state and workspace must be 16-byte aligned");
        return false;
    }
    const int64_t need = ssm_workspace_bytes(T, n_k, n_v, d);
    if (workspace == nullptr || ws_bytes < need) {
        set_error("ssm_scan: workspace %lld bytes < %lld needed", (long long)ws_bytes,
                  (long long)need);
        return false;
    }
    if (T * n_k > 0x7fffffff || n_v > 65535) {
        set_error("ssm_scan: grid too large");
        return false;
    }
    const auto up = [](int64_t b) { return (b + 255) / 256 * 256; };
    char* w = static_cast<char*>(workspace);
    float* qn = reinterpret_cast<float*>(w);
    float* kn = reinterpret_cast<float*>(w + up(T * n_k * d * 4));
    float* dc = reinterpret_cast<float*>(w + 2 * up(T * n_k * d * 4));
    float* bb = reinterpret_cast<float*>(w + 2 * up(T * n_k * d * 4) + up(T * n_v * 4));
    if (!launch("ssm_prep_kernel", ssm_prep_kernel, dim3((unsigned)(T * n_k)), dim3(64), 0, s,
                q, k, alpha, beta, a_log, dt_bias, qn, kn, dc, bb, n_k, n_v, d, eps))
        return false;
    const int64_t cw = 4 * (64 / P);
    return launch("ssm_scan_kernel", kern, dim3((unsigned)n_v, (unsigned)(d / cw)),
                  dim3(kScanThreads), 0, s, qn, kn, v, dc, bb, state, outs, T, n_k, n_v, scale);
}

bool ssm_conv_dev(const float* x, const float* w, const float* tail, int64_t tail_len,
                  float* tail_out, float* out, int64_t T, int64_t C, int64_t K,
                  int64_t* new_tail_len, hipStream_t s) {
    if (T < 0 || C <= 0 || K <= 0 || K - 1 > kMaxConvKeep || tail_len < 0 ||
        tail_len > K - 1 || (T > 0 && (x == nullptr || out == nullptr)) || w == nullptr ||
        (tail_len > 0 && tail == nullptr)) {
        set_error("ssm_conv: bad arguments (T=%lld C=%lld K=%lld tail_len=%lld)", (long long)T,
                  (long long)C, (long long)K, (long long)tail_len);
        return false;
    }
    const int64_t n = tail_len + T;
    const int64_t keep = std::min<int64_t>(K - 1, n);
    if (keep > 0 && tail_out == nullptr) {
        set_error("ssm_conv: null tail_out");
        return false;
    }
    if (T * C > ((int64_t)0x7fffffff) * 256) {
        set_error("ssm_conv: too large");
        return false;
    }
    if (T > 0 && !launch("ssm_conv_kernel", ssm_conv_kernel, dim3((unsigned)((T * C + 255) / 256)),
                         dim3(256), 0, s, x, w, tail, out, tail_len, T, C, (int)K))
        return false;
    if (keep > 0 && !launch("ssm_conv_tail_kernel", ssm_conv_tail_kernel,
                            dim3((unsigned)((C + 255) / 256)), dim3(256), 0, s, x, tail,
                            tail_out, tail_len, T, C, (int)keep))
        return false;
    if (new_tail_len) *new_tail_len = keep;
    return true;
}

}  // namespace aero

extern "C" {

int64_t aero_hip_ssm_workspace(int64_t T, int64_t n_k, int64_t n_v, int64_t d) {
    return aero::ssm_workspace_bytes(T, n_k, n_v, d);
}

int aero_hip_ssm_scan(const float* q, const float* k, const float* v, const float* alpha,
                      const float* beta, const float* a_log, const float* dt_bias, float* state,
                      int64_t T, int64_t n_k, int64_t n_v, int64_t d, float scale, float eps,
                      float* outs, void* workspace, int64_t ws_bytes, void* stream) {
    aero::clear_error();
    return aero::ssm_scan_dev(q, k, v, alpha, beta, a_log, dt_bias, state, T, n_k, n_v, d,
                              scale, eps, outs, workspace, ws_bytes, (hipStream_t)stream) ? 1 : 0;
}

int aero_hip_ssm_conv(const float* x, const float* w, const float* tail, int64_t tail_len,
                      float* tail_out, float* out, int64_t T, int64_t channels, int64_t kernel,
                      int64_t* new_tail_len, void* stream) {
    aero::clear_error();
    return aero::ssm_conv_dev(x, w, tail, tail_len, tail_out, out, T, channels, kernel,
                              new_tail_len, (hipStream_t)stream) ? 1 : 0;
}

}  // extern "C"
