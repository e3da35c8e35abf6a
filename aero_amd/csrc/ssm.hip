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
// ssm_prep_kernel computes qn, kn, dec and b for every token first (d / 4 lanes
// a token and key head), so the serial loop only streams them. Scans of 128
// or more tokens take the chunked (WY) form instead (ssm_chunk_prep_kernel +
// ssm_chunk_scan_kernel, below).
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
constexpr int kDepth = 4;  // tokens whose operands a lane has in flight

__device__ __forceinline__ float softplus_dev(float x) {
    return log1pf(expf(-fabsf(x))) + (x > 0.0f ? x : 0.0f);
}

// G = d / 4 lanes per (token t, key head kk) row, each normalising 4
// adjacent elements of q and k (one 16-byte load of each; token rows
// q_stride / k_stride floats apart), 256 / G rows a workgroup; qn and kn are
// written contiguous [T][n_k][d]; the group of kk == 0 also writes dec and b of token t for every
// value head (log_dec: the log of the decay, g <= 0, in place of exp(g), for
// the chunked scan).
template <int G>
__global__ __launch_bounds__(256) void ssm_prep_kernel(
    const float* __restrict__ q, const float* __restrict__ k, const float* __restrict__ alpha,
    const float* __restrict__ beta, const float* __restrict__ a_log,
    const float* __restrict__ dt_bias, float* __restrict__ qn, float* __restrict__ kn,
    float* __restrict__ dec, float* __restrict__ bb, int64_t n_rows, int64_t n_k, int64_t n_v,
    int64_t q_stride, int64_t k_stride, float eps, int log_dec) {
    constexpr int D = 4 * G;
    const int lane = threadIdx.x % G;
    const int64_t row = (int64_t)blockIdx.x * (256 / G) + threadIdx.x / G;  // t * n_k + kk
    if (row >= n_rows) return;   // whole groups: the sums below stay inside a group
    const int64_t t = row / n_k, kk = row % n_k;
    const v4f qv = *reinterpret_cast<const v4f*>(q + t * q_stride + kk * D + 4 * lane);
    const v4f kv = *reinterpret_cast<const v4f*>(k + t * k_stride + kk * D + 4 * lane);
    float sq = 0.0f, sk = 0.0f;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        sq += qv[e] * qv[e];
        sk += kv[e] * kv[e];
    }
    sq = group_sum<G>(sq);
    sk = group_sum<G>(sk);
    const float nq = fmaxf(sqrtf(sq), eps), nk = fmaxf(sqrtf(sk), eps);
    v4f qo, ko;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        qo[e] = qv[e] / nq;
        ko[e] = kv[e] / nk;
    }
    *reinterpret_cast<v4f*>(qn + row * D + 4 * lane) = qo;
    *reinterpret_cast<v4f*>(kn + row * D + 4 * lane) = ko;
    if (kk == 0) {
        for (int64_t h = lane; h < n_v; h += G) {
            float g = a_log[h] * softplus_dev(alpha[t * n_v + h] + dt_bias[h]);
            if (g > 0.0f) g = 0.0f;
            dec[t * n_v + h] = log_dec ? g : expf(g);
            bb[t * n_v + h] = 1.0f / (1.0f + expf(-beta[t * n_v + h]));
        }
    }
}

// Sum over each aligned group of G (8 or 16) lanes, every lane getting the
// sum, through DPP lane moves (no LDS path): lane ^ 1, lane ^ 2 within a
// quad, then the 8-lane and 16-lane mirrors.
template <int CTRL>
__device__ __forceinline__ float dpp_mov(float v) {
    return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), CTRL, 0xF, 0xF, true));
}
template <int G>
__device__ __forceinline__ float lane_group_sum(float v) {
    static_assert(G == 8 || G == 16, "DPP groups of 8 or 16 lanes");
    v += dpp_mov<0xB1>(v);   // quad_perm [1,0,3,2]
    v += dpp_mov<0x4E>(v);   // quad_perm [2,3,0,1]
    v += dpp_mov<0x141>(v);  // row_half_mirror
    if constexpr (G == 16) v += dpp_mov<0x140>(v);  // row_mirror
    return v;
}

struct ScanArgs {
    const float* q;        // [T][n_k][D]: raw (FUSED) or normalised (workspace)
    const float* k;
    const float* v;        // [T][n_v][D]
    int64_t qs, ks, vs;    // floats from one token's q / k / v row to the next
    const float* alpha;    // [T][n_v]: raw alpha (FUSED) or the decay (workspace)
    const float* beta;     // [T][n_v]: raw beta (FUSED) or the gate (workspace)
    const float* a_log;    // [n_v] (FUSED)
    const float* dt_bias;  // [n_v] (FUSED)
    float* state;          // [n_v][D][D]
    float* outs;           // [T][n_v][D]
    int64_t T, n_k, n_v;
    float scale, eps;
};

// One token's operands for a lane: its RPT rows of kn and qn, v of its column,
// the head's decay and gate.
template <int D, int RPT>
struct TokenOps {
    float k[RPT], q[RPT];
    float v, dec, b;
};

// A token's loads (q / k raw when FUSED, else normalised by ssm_prep_kernel;
// alpha / beta raw when FUSED, else the decay and gate).
template <int D, int RPT, bool FUSED>
__device__ __forceinline__ void load_token(const ScanArgs& a, int64_t t, int64_t h, int64_t kk,
                                           int e, int i0, TokenOps<D, RPT>& o) {
    const float4* k4 = reinterpret_cast<const float4*>(a.k + t * a.ks + kk * D + i0);
    const float4* q4 = reinterpret_cast<const float4*>(a.q + t * a.qs + kk * D + i0);
#pragma unroll
    for (int j = 0; j < RPT / 4; ++j) {
        const float4 x = k4[j], y = q4[j];
        o.k[4 * j] = x.x; o.k[4 * j + 1] = x.y; o.k[4 * j + 2] = x.z; o.k[4 * j + 3] = x.w;
        o.q[4 * j] = y.x; o.q[4 * j + 1] = y.y; o.q[4 * j + 2] = y.z; o.q[4 * j + 3] = y.w;
    }
    o.v = a.v[t * a.vs + h * D + e];
    o.dec = a.alpha[t * a.n_v + h];
    o.b = a.beta[t * a.n_v + h];
}

// FUSED (short scans): normalise q / k (a wave reduction for each norm) and
// compute the decay and gate, when the token is used.
template <int D, int RPT, bool FUSED>
__device__ __forceinline__ void finish_token(const ScanArgs& a, int64_t t, int64_t h,
                                             int64_t kk, int lane, TokenOps<D, RPT>& o) {
    if constexpr (FUSED) {
        const float* kr = a.k + t * a.ks + kk * D;
        const float* qr = a.q + t * a.qs + kk * D;
        float sk = 0.0f, sq = 0.0f;
#pragma unroll
        for (int i = lane; i < D; i += 64) {
            sk += kr[i] * kr[i];
            sq += qr[i] * qr[i];
        }
        sk = group_sum<64>(sk);
        sq = group_sum<64>(sq);
        const float nk = fmaxf(sqrtf(sk), a.eps), nq = fmaxf(sqrtf(sq), a.eps);
#pragma unroll
        for (int j = 0; j < RPT; ++j) {
            o.k[j] = o.k[j] / nk;
            o.q[j] = o.q[j] / nq;
        }
        float g = a.a_log[h] * softplus_dev(o.dec + a.dt_bias[h]);
        if (g > 0.0f) g = 0.0f;
        o.dec = expf(g);
        o.b = 1.0f / (1.0f + expf(-o.b));
    }
}

// P adjacent lanes share a column (lane = ci * P + part), each holding RPT =
// D / P consecutive rows; a wave holds CPW = 64 / P columns, the workgroup CW
// = 4 * CPW. The state tile passes through LDS at the start and the end, so
// its global reads and writes are row-contiguous.
template <int D, int P, bool FUSED>
__global__ __launch_bounds__(kScanThreads) void ssm_scan_kernel(ScanArgs a) {
    constexpr int RPT = D / P;
    constexpr int CPW = 64 / P;
    constexpr int CW = 4 * CPW;
    constexpr int LD = D + 4;  // LDS column stride (floats)
    static_assert(RPT % 4 == 0, "rows a lane must be whole float4s");
    __shared__ __align__(16) float tile[CW * LD];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int part = lane % P, ci = lane / P;
    const int64_t h = blockIdx.x;
    const int64_t kk = h % a.n_k;
    const int e0 = (int)blockIdx.y * CW;
    const int c = wave * CPW + ci;  // this lane's column within the tile
    const int e = e0 + c;
    const int i0 = part * RPT;

    float* S = a.state + h * (int64_t)D * D;
    for (int f = threadIdx.x; f < D * CW; f += kScanThreads) {
        const int i = f / CW, cc = f % CW;
        tile[cc * LD + i] = S[(int64_t)i * D + e0 + cc];
    }
    __syncthreads();
    float s[RPT];
#pragma unroll
    for (int j = 0; j < RPT; j += 4) {
        const float4 x = *reinterpret_cast<const float4*>(&tile[c * LD + i0 + j]);
        s[j] = x.x; s[j + 1] = x.y; s[j + 2] = x.z; s[j + 3] = x.w;
    }

    // the delta-rule update of this lane's rows for one token
    auto step = [&](TokenOps<D, RPT>& o, int64_t t) __attribute__((always_inline)) {
        finish_token<D, RPT, FUSED>(a, t, h, kk, lane, o);
        float p0 = 0.0f, p1 = 0.0f;
#pragma unroll
        for (int j = 0; j < RPT; j += 2) {
            s[j] *= o.dec;
            s[j + 1] *= o.dec;
            p0 = __builtin_fmaf(o.k[j], s[j], p0);
            p1 = __builtin_fmaf(o.k[j + 1], s[j + 1], p1);
        }
        const float vp = lane_group_sum<P>(p0 + p1);
        const float vnew = (o.v - vp) * o.b;
        float o0 = 0.0f, o1 = 0.0f;
#pragma unroll
        for (int j = 0; j < RPT; j += 2) {
            s[j] = __builtin_fmaf(o.k[j], vnew, s[j]);
            s[j + 1] = __builtin_fmaf(o.k[j + 1], vnew, s[j + 1]);
            o0 = __builtin_fmaf(o.q[j], s[j], o0);
            o1 = __builtin_fmaf(o.q[j + 1], s[j + 1], o1);
        }
        const float r = lane_group_sum<P>(o0 + o1);
        if (part == 0) a.outs[(t * a.n_v + h) * D + e] = a.scale * r;
    };
    // a ring of kDepth tokens' operands in flight: slot u holds token t + u
    // and is refilled with token t + u + kDepth once used (clamped to the last
    // token: in bounds, no branch); slots are static in the unrolled body
    TokenOps<D, RPT> ring[kDepth];
#pragma unroll
    for (int u = 0; u < kDepth; ++u)
        load_token<D, RPT, FUSED>(a, min((int64_t)u, a.T - 1), h, kk, e, i0, ring[u]);
    int64_t t = 0;
    for (; t + kDepth <= a.T; t += kDepth) {
#pragma unroll
        for (int u = 0; u < kDepth; ++u) {
            step(ring[u], t + u);
            load_token<D, RPT, FUSED>(a, min(t + u + kDepth, a.T - 1), h, kk, e, i0, ring[u]);
        }
    }
#pragma unroll
    for (int u = 0; u < kDepth; ++u)
        if (t + u < a.T) step(ring[u], t + u);

#pragma unroll
    for (int j = 0; j < RPT; j += 4)
        *reinterpret_cast<float4*>(&tile[c * LD + i0 + j]) = make_float4(s[j], s[j + 1],
                                                                           s[j + 2], s[j + 3]);
    __syncthreads();
    for (int f = threadIdx.x; f < D * CW; f += kScanThreads) {
        const int i = f / CW, cc = f % CW;
        S[(int64_t)i * D + e0 + cc] = tile[cc * LD + i];
    }
}

// silu (src/ssm.cpp:17), applied to the conv's outputs when the SSM layer
// asks for it (src/ssm.cpp:298-301)
template <bool SILU>
__device__ __forceinline__ float conv_out(float v) {
    if constexpr (SILU) return silu_fast(v);
    return v;
}

// out[t, c] = sum_j buf[tl + t + 1 - K + j, c] * w[c, j] over the rows that
// exist, buf = [tail (tl rows); x], taps in order, tap 0 the oldest.
template <bool SILU>
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
    out[idx] = conv_out<SILU>(acc);
}

// The same conv with K fixed: a lane owns channel c for TB consecutive
// tokens, holding its K weights and a sliding window of K inputs in
// registers, so each input is loaded once (plus K - 1 rows of halo a block).
// Taps before the start of the history are skipped, as above. With one
// block of tokens (T <= TB) and tail_out given, the lane also writes its
// channel's new history, the last keep rows of [tail; x], from the window
// after its last token: it has read every history row of the channel by
// then, so tail_out may be tail.
template <int K, int TB, bool SILU>
__global__ __launch_bounds__(256) void ssm_conv_k_kernel(const float* x, const float* __restrict__ w,
                                                         const float* tail, float* __restrict__ out,
                                                         int64_t tl, int64_t T, int64_t C,
                                                         float* tail_out, int keep) {
    const int64_t c = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (c >= C) return;
    const int64_t t0 = (int64_t)blockIdx.y * TB;
    float wr[K];
#pragma unroll
    for (int j = 0; j < K; ++j) wr[j] = w[c * K + j];
    float win[K];
    bool ok[K];
    auto fetch = [&](int64_t b, float& val, bool& has) {
        has = b >= 0;
        val = b < 0 ? 0.0f : (b < tl ? tail[b * C + c] : x[(b - tl) * C + c]);
    };
#pragma unroll
    for (int j = 0; j < K - 1; ++j) fetch(tl + t0 + 1 - K + j, win[j], ok[j]);
    for (int tt = 0; tt < TB; ++tt) {
        const int64_t t = t0 + tt;
        if (t >= T) break;
        fetch(tl + t, win[K - 1], ok[K - 1]);
        float acc = 0.0f;
#pragma unroll
        for (int j = 0; j < K; ++j)
            if (ok[j]) acc = acc + win[j] * wr[j];
        out[t * C + c] = conv_out<SILU>(acc);
#pragma unroll
        for (int j = 0; j < K - 1; ++j) {
            win[j] = win[j + 1];
            ok[j] = ok[j + 1];
        }
    }
    // the window now holds rows tl + T - (K - 1) .. tl + T - 1 of [tail; x]
    if (tail_out != nullptr) {
#pragma unroll
        for (int i = 0; i < K - 1; ++i)
            if (i < keep) tail_out[(int64_t)i * C + c] = win[K - 1 - keep + i];
    }
}

// K = 4 with 4 adjacent channels a lane (C % 4 == 0, 16-byte aligned x, w
// and out): a block whose taps all lie in x (t0 >= 3, the whole block inside
// T) loads its TB + 3 rows as 16-byte loads up front, so the loads overlap;
// other blocks take the per-channel sliding window of ssm_conv_k_kernel.
// Same tap order, separate multiply and add from 0: bit-identical results.
template <int TB, bool SILU>
__global__ __launch_bounds__(256) void ssm_conv4_kernel(const float* __restrict__ x,
                                                        const float* __restrict__ w,
                                                        const float* __restrict__ tail,
                                                        float* __restrict__ out, int64_t tl,
                                                        int64_t T, int64_t C) {
    constexpr int K = 4;
    const int64_t c = ((int64_t)blockIdx.x * 256 + threadIdx.x) * 4;
    if (c >= C) return;
    const int64_t t0 = (int64_t)blockIdx.y * TB;
    v4f wv[4];   // wv[e]: the K taps of channel c + e
#pragma unroll
    for (int e = 0; e < 4; ++e) wv[e] = *reinterpret_cast<const v4f*>(w + (c + e) * K);
    if (t0 >= K - 1 && t0 + TB <= T) {
        v4f in[TB + K - 1];
#pragma unroll
        for (int i = 0; i < TB + K - 1; ++i)
            in[i] = *reinterpret_cast<const v4f*>(x + (t0 - (K - 1) + i) * C + c);
#pragma unroll
        for (int tt = 0; tt < TB; ++tt) {
            v4f acc;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                float s = 0.0f;
#pragma unroll
                for (int j = 0; j < K; ++j) s = s + in[tt + j][e] * wv[e][j];
                acc[e] = conv_out<SILU>(s);
            }
            *reinterpret_cast<v4f*>(out + (t0 + tt) * C + c) = acc;
        }
        return;
    }
    for (int e = 0; e < 4; ++e) {
        const int64_t ch = c + e;
        float win[K];
        bool ok[K];
        auto fetch = [&](int64_t b, float& val, bool& has) {
            has = b >= 0;
            val = b < 0 ? 0.0f : (b < tl ? tail[b * C + ch] : x[(b - tl) * C + ch]);
        };
#pragma unroll
        for (int j = 0; j < K - 1; ++j) fetch(tl + t0 + 1 - K + j, win[j], ok[j]);
        for (int tt = 0; tt < TB; ++tt) {
            const int64_t t = t0 + tt;
            if (t >= T) break;
            fetch(tl + t, win[K - 1], ok[K - 1]);
            float acc = 0.0f;
#pragma unroll
            for (int j = 0; j < K; ++j)
                if (ok[j]) acc = acc + win[j] * wv[e][j];
            out[t * C + ch] = conv_out<SILU>(acc);
#pragma unroll
            for (int j = 0; j < K - 1; ++j) {
                win[j] = win[j + 1];
                ok[j] = ok[j + 1];
            }
        }
    }
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

using ScanKernel = void (*)(ScanArgs);

template <int D, int P>
ScanKernel pick_scan_f(bool fused) {
    return fused ? ssm_scan_kernel<D, P, true> : ssm_scan_kernel<D, P, false>;
}

// P = lanes a column: 16 (8 rows a lane) by default; 8 keeps 16 rows a lane.
ScanKernel pick_scan(int64_t d, int p, bool fused) {
    if (d == 128) return p == 8 ? pick_scan_f<128, 8>(fused) : pick_scan_f<128, 16>(fused);
    if (d == 64) return p == 8 ? pick_scan_f<64, 8>(fused) : pick_scan_f<64, 16>(fused);
    if (d == 256) return pick_scan_f<256, 16>(fused);
    return nullptr;
}

// ---------------------------------------------------------- chunked scan
// The delta rule over chunks of C = 64 tokens (the WY form of the gated
// delta rule), algebraically the per-token recurrence above:
//   S_t = g_t S_{t-1} + k_t d_t^T,  d_t = b_t (v_t - g_t S_{t-1}^T k_t),
//   o_t = scale S_t^T q_t.
// With L_t = sum_{r<=t} log g_r inside the chunk, G_t = exp(L_t) and
// Gam_ts = exp(L_t - L_s) <= 1 (no overflow), the chunk's d rows satisfy
//   (I + A) Dlt = diag(b) (V - diag(G) K S0),  A_ts = b_t Gam_ts (k_t . k_s) (s < t)
// so Dlt = U - W S0 with U = (I+A)^-1 diag(b) V, W = (I+A)^-1 diag(b G) K, and
//   O = scale (diag(G) Q S0 + P Dlt),  P_ts = Gam_ts (q_t . k_s) (s <= t),
//   S_end = G_n S0 + sum_s exp(L_n - L_s) k_s d_s^T.
// ssm_chunk_prep_kernel computes U, W, P and the decay factors of every
// (chunk, value head) in parallel; the state pass (ssm_chunk_split_kernel at
// head dims 64 and 128, ssm_chunk_scan_kernel at 256) carries the state
// through the chunks on the fp32 matrix cores, 16 state columns a workgroup.
// Results differ from the per-token scan by fp32 rounding (the chunked form
// of a 512-token scan: ~6e-7 of the output's scale).
constexpr int kChunk = 64;

struct ChunkArgs {
    const float* qn;    // [T][n_k][D] normalised
    const float* kn;
    const float* v;     // [T][n_v][D], token rows vs floats apart
    int64_t vs;
    const float* lg;    // [T][n_v] log decay (<= 0)
    const float* bb;    // [T][n_v] gate
    float* U;           // [n_v][nc][C][D]
    float* W;           // [n_v][nc][C][D] in operand order (op_index)
    float* P;           // [n_v][nc][C][C] in operand order
    float* Qop;         // [n_k][nc][C][D]: normalised q in operand order
    float* Kop;         // [n_k][nc][C][D]: keys in the state pass's operand order
    float* gam;         // [n_v][nc][C]: G_t (0 past the chunk's last token)
    float* kfac;        // [n_v][nc][C]: exp(L_n - L_t) (0 past the last token)
    float* gC;          // [n_v][nc]: G_n
    float* state;       // [n_v][D][D]
    float* outs;        // [T][n_v][D]
    int64_t T, n_k, n_v;
    int nc;
    float scale;
};

// The scan's A operands (rows of W, Q, P) are stored in the order its waves
// load them: element (t, k) of a chunk's C x K block (t = 16w + r, k =
// 4g + 16j + e) at ((w * K/16 + j) * 64 + 16g + r) * 4 + e, so wave w's j-th
// 16-byte load of lane 16g + r reads 1 KB of contiguous memory.
__device__ __forceinline__ int op_index(int t, int k, int K) {
    return (((t >> 4) * (K >> 4) + (k >> 4)) * 64 + ((k >> 2) & 3) * 16 + (t & 15)) * 4 + (k & 3);
}

// One workgroup a (chunk c, value head h), four waves, every product on the
// fp32 matrix cores (16x16x4: lane (r, g) = (l % 16, l / 16) supplies A[r][g]
// and B[g][r] and receives D[4g + v][r]):
//  1. K K^T (strictly lower) and Q K^T (lower) in 16x16 tiles, five tile
//     products a wave; A = diag(b) Gam (K K^T) to LDS, P = Gam (Q K^T) out.
//     Lane group g supplies the reduction indices (D/4) g + 4 jj + e.
//  2. T = (I + A)^-1 by 16x16 blocks: the four unit lower-triangular diagonal
//     blocks by substitution (a wave each), then
//     T_ij = -T_ii sum_{j<=k<i} A_ik T_kj along the sub-diagonals.
//  3. U = T diag(b) V (waves 0, 1) and W = T diag(b G) K (waves 2, 3), skipping
//     T's zero blocks; the column scaling is folded into T's operand. From
//     D = 128 the two waves of a product split its columns (D / 2 each, in
//     groups of 64); at D = 64 they split its row tiles ({3, 0} and {2, 1},
//     equal work under the triangle).
// The keys are also stored in the order the state pass loads them, from one
// value head of each key head: entry ((((w * D/64 + it) * 4 + j) * 64 +
// 16g + r) * 4 + e) holds K[16j + 4g + e][(D/4) w + 16 it + r].
template <int D>
__global__ __launch_bounds__(256) void ssm_chunk_prep_kernel(ChunkArgs a) {
    constexpr int C = kChunk, KP = D + 4, AP = C + 4;
    constexpr int NJ = D / 16;                  // 16-byte loads a lane a 16-row tile
    constexpr int NG = D >= 128 ? D / 128 : 1;  // 64-column groups a wave in step 3
    constexpr int NT = D >= 128 ? 4 : 2;        // row tiles a wave in step 3
    constexpr int NPRE = 2 * NJ > 16 * NG ? 2 * NJ : 16 * NG;
    static_assert((D == 64 || D == 128 || D == 256) && C == 64, "tile layout");
    __shared__ __align__(16) float Ks[C * KP];   // keys [s][i], rows past n zero
    __shared__ __align__(16) float As[C * AP];   // A [t][s]
    __shared__ __align__(16) float Ts[C * AP];   // (I + A)^-1 [t][s]
    __shared__ double Ls[C];
    __shared__ float Bs[C], Fs[C];
    const int tid = threadIdx.x, l = tid & 63, r = l & 15, g = l >> 4;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int c = blockIdx.x;
    const int64_t h = blockIdx.y, kk = h % a.n_k;
    const int64_t t0 = (int64_t)c * C;
    const int n = (int)min<int64_t>(C, a.T - t0);
    const int64_t base = h * a.nc + c;

    // roles: waves 0, 1 form K K^T (row tiles {3, 0} / {2, 1}) and U; waves
    // 2, 3 form Q K^T and W. Each wave's rows from memory (V for U, Q rows
    // for Q K^T) are loaded here, before the first barrier, with the keys.
    const bool qw = wave >= 2;
    const int i_hi = (wave & 1) ? 2 : 3;
    v4f pre[NPRE];
    if (qw) {
#pragma unroll
        for (int which = 0; which < 2; ++which) {
            const int i = which ? 3 - i_hi : i_hi;
            const float* qrow = a.qn + ((t0 + min(16 * i + r, n - 1)) * a.n_k + kk) * D + (D / 4) * g;
#pragma unroll
            for (int jj = 0; jj < NJ; ++jj) pre[NJ * which + jj] = *reinterpret_cast<const v4f*>(qrow + 4 * jj);
        }
    } else {
        // rows past n: T's column scale (b) is zero there; any finite row
#pragma unroll
        for (int cg = 0; cg < NG; ++cg) {
            const int c0 = D >= 128 ? (D / 2) * (wave & 1) + 64 * cg : 0;
            const float* vsrc = a.v + h * D + c0 + 4 * r;
#pragma unroll
            for (int ks = 0; ks < C / 4; ++ks)
                pre[16 * cg + ks] = *reinterpret_cast<const v4f*>(vsrc + (t0 + min(4 * ks + g, n - 1)) * a.vs);
        }
    }
    // the chunk's normalised keys (rows past n zero)
#pragma unroll
    for (int i = 0; i < C * D / 4 / 256; ++i) {
        const int idx = tid + 256 * i, row = idx / (D / 4), c4 = idx % (D / 4);
        v4f kv = v4f{0.f, 0.f, 0.f, 0.f};
        if (row < n) kv = *reinterpret_cast<const v4f*>(a.kn + ((t0 + row) * a.n_k + kk) * D + 4 * c4);
        *reinterpret_cast<v4f*>(Ks + row * KP + 4 * c4) = kv;
    }
    // inclusive prefix sum of the log decays over the chunk, and the gates.
    // In float64: under strong decay L reaches -1e3 within a chunk, where a
    // float32 sum resolves 6e-5, and every factor below is exp of a
    // difference L_t - L_s of nearby tokens.
    if (wave == 0) {
        double lg = l < n ? (double)a.lg[(t0 + l) * a.n_v + h] : 0.0;
        const float b = l < n ? a.bb[(t0 + l) * a.n_v + h] : 0.0f;
#pragma unroll
        for (int o = 1; o < 64; o <<= 1) {
            const double u = __shfl_up(lg, o, 64);
            if (l >= o) lg += u;
        }
        Ls[l] = lg;
        Bs[l] = b;
        Fs[l] = b * expf((float)lg);
    }
    __syncthreads();

    if (h < a.n_k) {   // one value head of each key head copies the keys
        float* kop = a.Kop + (kk * a.nc + c) * C * D;
#pragma unroll
        for (int m = 0; m < C * D / 4 / 256; ++m) {
            // entry idx holds K[s][i] for e = 0..3
            const int idx = tid + 256 * m, lane = idx & 63, rest = idx >> 6;
            const int j = rest & 3, wit = rest >> 2;
            const int i = (wit / (D / 64)) * (D / 4) + (wit % (D / 64)) * 16 + (lane & 15);
            const int s0 = 16 * j + 4 * (lane >> 4);
            *reinterpret_cast<v4f*>(kop + 4 * idx) =
                v4f{Ks[s0 * KP + i], Ks[(s0 + 1) * KP + i], Ks[(s0 + 2) * KP + i], Ks[(s0 + 3) * KP + i]};
        }
    }

    // 1. K K^T (waves 0, 1) or Q K^T (waves 2, 3) for two row tiles each
    {
        const bool isq = qw;
#pragma unroll
        for (int which = 0; which < 2; ++which) {
            const int i = which ? 3 - i_hi : i_hi;
            v4f ar[NJ];
            if (isq) {
#pragma unroll
                for (int jj = 0; jj < NJ; ++jj) ar[jj] = pre[NJ * which + jj];
                if (h < a.n_k) {   // one value head of each key head copies q
                    float* qop = a.Qop + (kk * a.nc + c) * C * D;
#pragma unroll
                    for (int jj = 0; jj < NJ; ++jj)
                        *reinterpret_cast<v4f*>(qop + op_index(16 * i + r, (D / 4) * g + 4 * jj, D)) = ar[jj];
                }
            } else {
#pragma unroll
                for (int jj = 0; jj < NJ; ++jj)
                    ar[jj] = *reinterpret_cast<const v4f*>(Ks + (16 * i + r) * KP + (D / 4) * g + 4 * jj);
            }
            for (int j = 0; j < C / 16; ++j) {
                v4f acc = v4f{0.f, 0.f, 0.f, 0.f};
                if (j <= i) {
#pragma unroll
                    for (int jj = 0; jj < NJ; ++jj) {
                        const v4f kb = *reinterpret_cast<const v4f*>(Ks + (16 * j + r) * KP + (D / 4) * g + 4 * jj);
#pragma unroll
                        for (int e = 0; e < 4; ++e)
                            acc = __builtin_amdgcn_mfma_f32_16x16x4f32(ar[jj][e], kb[e], acc, 0, 0, 0);
                    }
                } else if (!isq) {
                    continue;   // A above the diagonal is never read
                }
#pragma unroll
                for (int vv = 0; vv < 4; ++vv) {
                    const int t = 16 * i + 4 * g + vv, sidx = 16 * j + r;
                    const float gm = (sidx <= t && t < n) ? expf((float)(Ls[t] - Ls[sidx])) : 0.0f;
                    if (isq)
                        a.P[base * C * C + op_index(t, sidx, C)] = sidx <= t ? gm * acc[vv] : 0.0f;
                    else
                        As[t * AP + sidx] = sidx < t ? Bs[t] * (gm * acc[vv]) : 0.0f;
                }
            }
        }
    }
    if (tid < C) {
        const bool live = tid < n;
        a.gam[base * C + tid] = live ? expf((float)Ls[tid]) : 0.0f;
        a.kfac[base * C + tid] = live ? expf((float)(Ls[n - 1] - Ls[tid])) : 0.0f;
        if (tid == 0) a.gC[base] = expf((float)Ls[n - 1]);
    }
    __syncthreads();

    // 2a. diagonal block w of T: column r by substitution (rows above r zero)
    {
        const int b0 = 16 * wave;
        float x[16];
#pragma unroll
        for (int t = 0; t < 16; ++t) {
            float acc = t == r ? 1.0f : 0.0f;
#pragma unroll
            for (int s4 = 0; s4 < t; s4 += 4) {
                const v4f av = *reinterpret_cast<const v4f*>(As + (b0 + t) * AP + b0 + s4);
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    if (s4 + e < t) acc -= av[e] * x[s4 + e];
            }
            x[t] = acc;
        }
        if (g == 0) {
#pragma unroll
            for (int t = 0; t < 16; ++t) Ts[(b0 + t) * AP + b0 + r] = x[t];
        }
    }
    __syncthreads();
    // 2b. T_ij = -T_ii X, X = sum_{j<=k<i} A_ik T_kj; X in the output layout is
    // the B operand of the second product with T_ii's columns taken as 4g + v
    auto off_diag = [&](int i, int j) __attribute__((always_inline)) {
        v4f xa = v4f{0.f, 0.f, 0.f, 0.f};
        for (int k = j; k < i; ++k)
#pragma unroll
            for (int q = 0; q < 4; ++q)
                xa = __builtin_amdgcn_mfma_f32_16x16x4f32(As[(16 * i + r) * AP + 16 * k + 4 * q + g],
                                                          Ts[(16 * k + 4 * q + g) * AP + 16 * j + r],
                                                          xa, 0, 0, 0);
        const v4f tii = *reinterpret_cast<const v4f*>(Ts + (16 * i + r) * AP + 16 * i + 4 * g);
        v4f y = v4f{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int vv = 0; vv < 4; ++vv)
            y = __builtin_amdgcn_mfma_f32_16x16x4f32(tii[vv], xa[vv], y, 0, 0, 0);
#pragma unroll
        for (int vv = 0; vv < 4; ++vv) Ts[(16 * i + 4 * g + vv) * AP + 16 * j + r] = -y[vv];
    };
    if (wave < 3) off_diag(wave + 1, wave);
    __syncthreads();
    if (wave < 2) off_diag(wave + 2, wave);
    __syncthreads();
    if (wave == 0) off_diag(3, 0);
    __syncthreads();

    // 3. U = T diag(b) V (waves 0, 1), W = T diag(b G) K (waves 2, 3): lane r
    // of column tile ct holds column c0 + 4r + ct, so each lane loads and
    // stores 4 adjacent columns
    const bool isw = qw;
#pragma unroll
    for (int cg = 0; cg < NG; ++cg) {
        const int c0 = D >= 128 ? (D / 2) * (wave & 1) + 64 * cg : 0;
        v4f acc[NT][4];
#pragma unroll
        for (int ti = 0; ti < NT; ++ti)
#pragma unroll
            for (int ct = 0; ct < 4; ++ct) acc[ti][ct] = v4f{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int ks = 0; ks < C / 4; ++ks) {
            const int sidx = 4 * ks + g;
            const v4f bv = isw ? *reinterpret_cast<const v4f*>(Ks + sidx * KP + c0 + 4 * r) : pre[16 * cg + ks];
            const float fs = isw ? Fs[sidx] : Bs[sidx];
#pragma unroll
            for (int ti = 0; ti < NT; ++ti) {
                const int i = NT == 4 ? ti : (ti ? 3 - i_hi : i_hi);
                if (NT == 4 ? ks / 4 > ti : ks / 4 > i) continue;   // T is lower triangular
                const float ta = Ts[(16 * i + r) * AP + sidx] * fs;
#pragma unroll
                for (int ct = 0; ct < 4; ++ct)
                    acc[ti][ct] = __builtin_amdgcn_mfma_f32_16x16x4f32(ta, bv[ct], acc[ti][ct], 0, 0, 0);
            }
        }
        // U row-major; W in operand order (4 adjacent columns stay adjacent)
        float* dst = (isw ? a.W : a.U) + base * C * D;
#pragma unroll
        for (int ti = 0; ti < NT; ++ti)
#pragma unroll
            for (int vv = 0; vv < 4; ++vv) {
                const int i = NT == 4 ? ti : (ti ? 3 - i_hi : i_hi);
                const int t = 16 * i + 4 * g + vv, col = c0 + 4 * r;
                *reinterpret_cast<v4f*>(dst + (isw ? op_index(t, col, D) : t * D + col)) =
                    v4f{acc[ti][0][vv], acc[ti][1][vv], acc[ti][2][vv], acc[ti][3][vv]};
            }
    }
}

// The state pass, for head dims 64, 128 and 256. One workgroup a (value head
// h, 16 CT state columns from e0) carries that block of the state in LDS
// through the chunks in order. Per chunk, on the fp32 matrix cores:
//  (a) W S0 and Q S0 for each wave's 16 tokens;
//  then d = U - W S0 and kfac d go to LDS (one barrier), and
//  (b) P d, giving O = scale (diag(G) Q S0 + P d);
//  (c) the state update, computed transposed, S0^T <- G_n S0^T + (kfac d)^T K,
//      so the keys are its B operand.
// The registers a chunk holds are cut to what head dim 256 allows (512 a
// lane):
// - the keys come from Kop, already in the order (c) consumes them, so no key
//   buffer sits in LDS (at D = 256 two would take 133 KB);
// - the state tile streams from LDS into (a), 16 bytes a step;
// - the next chunk's rows of W and Q are loaded right after (a), when this
//   chunk's are dead, and land during (b) and (c); its rows of P and the keys
//   after (c), landing during the next (a); U and the decay factors at the
//   chunk's start. At D = 256 (QLATE) a chunk's Q rows load at its own start,
//   behind W S0, so that two chunks' Q rows are never held at once.
// Wave w owns token rows 16w..16w+15 of a chunk and state rows
// (D/4) w..(D/4)(w+1)-1 (D/64 tiles of 16).
template <int D>
struct ChunkWQ {
    v4f w[D / 16], q[D / 16];
};
template <int D, int CT>
struct ChunkOps {
    v4f p[4], kb[D / 16];
    float u[CT][4], gm[4], kf[4];
    float gc;
};

template <int D, int CT>
__global__ __launch_bounds__(256) void ssm_chunk_scan_kernel(ChunkArgs a) {
    constexpr int C = kChunk, SP = D + 4, TP = C + 4, NC = 16 * CT, NJ = D / 16, IT = D / 64;
    constexpr bool QLATE = D == 256;
    static_assert((D == 64 || D == 128 || D == 256) && C == 64, "wave layout");
    __shared__ __align__(16) float St[NC * SP];   // state block, St[col][i]
    __shared__ __align__(16) float Dt[NC * TP];   // d^T: Dt[col][s]
    __shared__ __align__(16) float Dk[NC * TP];   // (kfac d)^T
    const int tid = threadIdx.x, l = tid & 63, r = l & 15, g = l >> 4;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int64_t h = blockIdx.x, kk = h % a.n_k;
    const int e0 = NC * blockIdx.y;
    float* Sg = a.state + h * D * D;
#pragma unroll
    for (int i = 0; i < D * NC / 256; ++i) {
        const int idx = tid + 256 * i, row = idx / NC, col = idx % NC;
        St[col * SP + row] = Sg[(int64_t)row * D + e0 + col];
    }

    // rows of W and Q in operand order (op_index): 1 KB contiguous a load
    auto load_w = [&](int c, ChunkWQ<D>& o) __attribute__((always_inline)) {
        const float* wr = a.W + (h * a.nc + c) * C * D + (wave * NJ * 64 + l) * 4;
#pragma unroll
        for (int j = 0; j < NJ; ++j) o.w[j] = *reinterpret_cast<const v4f*>(wr + 256 * j);
    };
    auto load_q = [&](int c, ChunkWQ<D>& o) __attribute__((always_inline)) {
        const float* qr = a.Qop + (kk * a.nc + c) * C * D + (wave * NJ * 64 + l) * 4;
#pragma unroll
        for (int j = 0; j < NJ; ++j) o.q[j] = *reinterpret_cast<const v4f*>(qr + 256 * j);
    };
    // rows of P and the keys, used by (b) and (c)
    auto load_pk = [&](int c, ChunkOps<D, CT>& o) __attribute__((always_inline)) {
        const int64_t base = h * a.nc + c;
        const float* pr = a.P + base * C * C + (wave * (C / 16) * 64 + l) * 4;
        const float* kr = a.Kop + (kk * a.nc + c) * C * D + (wave * IT * 4 * 64 + l) * 4;
#pragma unroll
        for (int j = 0; j < 4; ++j) o.p[j] = *reinterpret_cast<const v4f*>(pr + 256 * j);
#pragma unroll
        for (int m = 0; m < NJ; ++m) o.kb[m] = *reinterpret_cast<const v4f*>(kr + 256 * m);
    };
    // U and the per-token factors
    auto load_ops = [&](int c, ChunkOps<D, CT>& o) __attribute__((always_inline)) {
        const int64_t base = h * a.nc + c;
#pragma unroll
        for (int vv = 0; vv < 4; ++vv) {
            const int t = 16 * wave + 4 * g + vv;
#pragma unroll
            for (int ct = 0; ct < CT; ++ct) o.u[ct][vv] = a.U[(base * C + t) * D + e0 + 16 * ct + r];
            o.gm[vv] = a.gam[base * C + t];
            o.kf[vv] = a.kfac[base * C + t];
        }
        o.gc = a.gC[base];
    };
    auto chunk = [&](int c, ChunkWQ<D>& o, ChunkWQ<D>& nwq, const ChunkOps<D, CT>& op,
                     ChunkOps<D, CT>& nop) __attribute__((always_inline)) {
        const int64_t t0 = (int64_t)c * C;
        const int n = (int)min<int64_t>(C, a.T - t0);
        const int cn = min(c + 1, a.nc - 1);
        load_ops(cn, nop);
        // (a) W S0 and Q S0 for the wave's 16 tokens and each column tile:
        // B[i][col] = S0[i][e0 + 16 ct + r], i = 4g + 16j + e. With QLATE the
        // chunk's Q rows load here and W S0 runs first, over their latency.
        v4f ws[CT], qs[CT];
#pragma unroll
        for (int ct = 0; ct < CT; ++ct) ws[ct] = qs[ct] = v4f{0.f, 0.f, 0.f, 0.f};
        if constexpr (QLATE) {
            load_q(c, o);
#pragma unroll
            for (int j = 0; j < NJ; ++j)
#pragma unroll
                for (int ct = 0; ct < CT; ++ct) {
                    const v4f sv = *reinterpret_cast<const v4f*>(St + (16 * ct + r) * SP + 4 * g + 16 * j);
#pragma unroll
                    for (int e = 0; e < 4; ++e)
                        ws[ct] = __builtin_amdgcn_mfma_f32_16x16x4f32(o.w[j][e], sv[e], ws[ct], 0, 0, 0);
                }
            __builtin_amdgcn_sched_barrier(0);
            load_w(cn, nwq);
#pragma unroll
            for (int j = 0; j < NJ; ++j)
#pragma unroll
                for (int ct = 0; ct < CT; ++ct) {
                    const v4f sv = *reinterpret_cast<const v4f*>(St + (16 * ct + r) * SP + 4 * g + 16 * j);
#pragma unroll
                    for (int e = 0; e < 4; ++e)
                        qs[ct] = __builtin_amdgcn_mfma_f32_16x16x4f32(o.q[j][e], sv[e], qs[ct], 0, 0, 0);
                }
        } else {
#pragma unroll
            for (int j = 0; j < NJ; ++j)
#pragma unroll
                for (int ct = 0; ct < CT; ++ct) {
                    const v4f sv = *reinterpret_cast<const v4f*>(St + (16 * ct + r) * SP + 4 * g + 16 * j);
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        ws[ct] = __builtin_amdgcn_mfma_f32_16x16x4f32(o.w[j][e], sv[e], ws[ct], 0, 0, 0);
                        qs[ct] = __builtin_amdgcn_mfma_f32_16x16x4f32(o.q[j][e], sv[e], qs[ct], 0, 0, 0);
                    }
                }
        }
        // the wave's own state entries, for the update after the barrier
        float sold[CT][IT][4];
#pragma unroll
        for (int ct = 0; ct < CT; ++ct)
#pragma unroll
            for (int it = 0; it < IT; ++it)
#pragma unroll
                for (int vv = 0; vv < 4; ++vv)
                    sold[ct][it][vv] = St[(16 * ct + 4 * g + vv) * SP + (D / 4) * wave + 16 * it + r];
        __builtin_amdgcn_sched_barrier(0);
        if constexpr (!QLATE) {
            load_w(cn, nwq);
            load_q(cn, nwq);
        }
        // d = U - W S0 (rows 16w + 4g + v, column r of each tile); kfac d
#pragma unroll
        for (int ct = 0; ct < CT; ++ct) {
            v4f dl, dk;
#pragma unroll
            for (int vv = 0; vv < 4; ++vv) {
                dl[vv] = op.u[ct][vv] - ws[ct][vv];
                dk[vv] = op.kf[vv] * dl[vv];
            }
            *reinterpret_cast<v4f*>(Dt + (16 * ct + r) * TP + 16 * wave + 4 * g) = dl;
            *reinterpret_cast<v4f*>(Dk + (16 * ct + r) * TP + 16 * wave + 4 * g) = dk;
        }
        __syncthreads();
        v4f dt[CT][4], dkv[CT][4];
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int ct = 0; ct < CT; ++ct) {
                dt[ct][j] = *reinterpret_cast<const v4f*>(Dt + (16 * ct + r) * TP + 4 * g + 16 * j);
                dkv[ct][j] = *reinterpret_cast<const v4f*>(Dk + (16 * ct + r) * TP + 4 * g + 16 * j);
            }
        // (b) P d and (c) S0^T <- G_n S0^T + (kfac d)^T K for the wave's state
        // rows: A[col][s] = (kfac d)[s][col], B[s][i] = K[s][i] from kb
        v4f pd[CT], sd[CT][IT];
#pragma unroll
        for (int ct = 0; ct < CT; ++ct) {
            pd[ct] = v4f{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int it = 0; it < IT; ++it) sd[ct][it] = v4f{0.f, 0.f, 0.f, 0.f};
        }
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int e = 0; e < 4; ++e)
#pragma unroll
                for (int ct = 0; ct < CT; ++ct) {
                    pd[ct] = __builtin_amdgcn_mfma_f32_16x16x4f32(op.p[j][e], dt[ct][j][e], pd[ct], 0, 0, 0);
#pragma unroll
                    for (int it = 0; it < IT; ++it)
                        sd[ct][it] = __builtin_amdgcn_mfma_f32_16x16x4f32(dkv[ct][j][e], op.kb[4 * it + j][e],
                                                                          sd[ct][it], 0, 0, 0);
                }
        // O = scale (G Q S0 + P d)
#pragma unroll
        for (int ct = 0; ct < CT; ++ct)
#pragma unroll
            for (int vv = 0; vv < 4; ++vv) {
                const int t = 16 * wave + 4 * g + vv;
                if (t < n)
                    a.outs[((t0 + t) * a.n_v + h) * D + e0 + 16 * ct + r] =
                        a.scale * (op.gm[vv] * qs[ct][vv] + pd[ct][vv]);
            }
#pragma unroll
        for (int ct = 0; ct < CT; ++ct)
#pragma unroll
            for (int it = 0; it < IT; ++it)
#pragma unroll
                for (int vv = 0; vv < 4; ++vv)
                    St[(16 * ct + 4 * g + vv) * SP + (D / 4) * wave + 16 * it + r] =
                        op.gc * sold[ct][it][vv] + sd[ct][it][vv];
        __builtin_amdgcn_sched_barrier(0);
        load_pk(cn, nop);
        __syncthreads();
    };

    ChunkWQ<D> wa, wb;
    ChunkOps<D, CT> oa, ob;
    load_w(0, wa);
    if constexpr (!QLATE) load_q(0, wa);
    load_ops(0, oa);
    load_pk(0, oa);
    __syncthreads();
    for (int c = 0; c < a.nc; c += 2) {
        chunk(c, wa, wb, oa, ob);
        if (c + 1 >= a.nc) break;
        chunk(c + 1, wb, wa, ob, oa);
    }
#pragma unroll
    for (int i = 0; i < D * NC / 256; ++i) {
        const int idx = tid + 256 * i, row = idx / NC, col = idx % NC;
        Sg[(int64_t)row * D + e0 + col] = St[col * SP + row];
    }
}

// The state pass with two waves a SIMD (head dims 64 and 128): the four
// state waves carry the chain W S0 -> d -> state update, and four output
// waves take Q S0 and P d off it. Per chunk:
//   state wave w:  W S0 (its 16 tokens) | d, kfac d -> LDS | barrier |
//                  (c) on its D/4 state rows | barrier
//   output wave w: Q S0 (its 16 tokens) |                  | barrier |
//                  P d, the outputs      | barrier
// St is read by every wave before the first barrier and written by the
// state waves after it; Dt / Dk written before it and read after. Each
// wave's operands for the next chunk load at the chunk's start.
template <int D>
struct SplitStateOps {
    v4f w[D / 16], kb[D / 16];
    float u[4], kf[4];
    float gc;
};
template <int D>
struct SplitOutOps {
    v4f q[D / 16], p[4];
    float gm[4];
};

template <int D>
__global__ __launch_bounds__(512) void ssm_chunk_split_kernel(ChunkArgs a) {
    constexpr int C = kChunk, SP = D + 4, TP = C + 4, NC = 16, NJ = D / 16, IT = D / 64;
    static_assert((D == 64 || D == 128) && C == 64, "wave layout");
    __shared__ __align__(16) float St[NC * SP];   // state block, St[col][i]
    __shared__ __align__(16) float Dt[NC * TP];   // d^T: Dt[col][s]
    __shared__ __align__(16) float Dk[NC * TP];   // (kfac d)^T
    const int tid = threadIdx.x, l = tid & 63, r = l & 15, g = l >> 4;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6), wq = wave & 3;
    const int64_t h = blockIdx.x, kk = h % a.n_k;
    const int e0 = NC * blockIdx.y;
    float* Sg = a.state + h * D * D;
#pragma unroll
    for (int i = 0; i < D * NC / 512; ++i) {
        const int idx = tid + 512 * i, row = idx / NC, col = idx % NC;
        St[col * SP + row] = Sg[(int64_t)row * D + e0 + col];
    }
    // B[i][col] = S0[i][e0 + r], i = 4g + 16j + e, against A rows x[j]
    auto s0_product = [&](const v4f* x) __attribute__((always_inline)) {
        v4f acc = v4f{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int j = 0; j < NJ; ++j) {
            const v4f sv = *reinterpret_cast<const v4f*>(St + r * SP + 4 * g + 16 * j);
#pragma unroll
            for (int e = 0; e < 4; ++e) acc = __builtin_amdgcn_mfma_f32_16x16x4f32(x[j][e], sv[e], acc, 0, 0, 0);
        }
        return acc;
    };

    if (wave < 4) {
        auto load = [&](int c, SplitStateOps<D>& o) __attribute__((always_inline)) {
            const int64_t base = h * a.nc + c;
            const float* wr = a.W + base * C * D + (wq * NJ * 64 + l) * 4;
            const float* kr = a.Kop + (kk * a.nc + c) * C * D + (wq * IT * 4 * 64 + l) * 4;
#pragma unroll
            for (int j = 0; j < NJ; ++j) {
                o.w[j] = *reinterpret_cast<const v4f*>(wr + 256 * j);
                o.kb[j] = *reinterpret_cast<const v4f*>(kr + 256 * j);
            }
#pragma unroll
            for (int vv = 0; vv < 4; ++vv) {
                const int t = 16 * wq + 4 * g + vv;
                o.u[vv] = a.U[(base * C + t) * D + e0 + r];
                o.kf[vv] = a.kfac[base * C + t];
            }
            o.gc = a.gC[base];
        };
        auto chunk = [&](int c, const SplitStateOps<D>& o, SplitStateOps<D>& nx) __attribute__((always_inline)) {
            load(min(c + 1, a.nc - 1), nx);
            const v4f ws = s0_product(o.w);
            float sold[IT][4];
#pragma unroll
            for (int it = 0; it < IT; ++it)
#pragma unroll
                for (int vv = 0; vv < 4; ++vv) sold[it][vv] = St[(4 * g + vv) * SP + (D / 4) * wq + 16 * it + r];
            v4f dl, dk;
#pragma unroll
            for (int vv = 0; vv < 4; ++vv) {
                dl[vv] = o.u[vv] - ws[vv];
                dk[vv] = o.kf[vv] * dl[vv];
            }
            *reinterpret_cast<v4f*>(Dt + r * TP + 16 * wq + 4 * g) = dl;
            *reinterpret_cast<v4f*>(Dk + r * TP + 16 * wq + 4 * g) = dk;
            __syncthreads();
            v4f dkv[4];
#pragma unroll
            for (int j = 0; j < 4; ++j) dkv[j] = *reinterpret_cast<const v4f*>(Dk + r * TP + 4 * g + 16 * j);
            // (c) S0^T <- G_n S0^T + (kfac d)^T K on state rows (D/4) wq + 16 it + r
            v4f sd[IT];
#pragma unroll
            for (int it = 0; it < IT; ++it) sd[it] = v4f{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int j = 0; j < 4; ++j)
#pragma unroll
                for (int e = 0; e < 4; ++e)
#pragma unroll
                    for (int it = 0; it < IT; ++it)
                        sd[it] = __builtin_amdgcn_mfma_f32_16x16x4f32(dkv[j][e], o.kb[4 * it + j][e], sd[it], 0, 0, 0);
#pragma unroll
            for (int it = 0; it < IT; ++it)
#pragma unroll
                for (int vv = 0; vv < 4; ++vv)
                    St[(4 * g + vv) * SP + (D / 4) * wq + 16 * it + r] = o.gc * sold[it][vv] + sd[it][vv];
            __syncthreads();
        };
        SplitStateOps<D> oa, ob;
        load(0, oa);
        __syncthreads();
        for (int c = 0; c < a.nc; c += 2) {
            chunk(c, oa, ob);
            if (c + 1 >= a.nc) break;
            chunk(c + 1, ob, oa);
        }
    } else {
        auto load = [&](int c, SplitOutOps<D>& o) __attribute__((always_inline)) {
            const int64_t base = h * a.nc + c;
            const float* qr = a.Qop + (kk * a.nc + c) * C * D + (wq * NJ * 64 + l) * 4;
            const float* pr = a.P + base * C * C + (wq * (C / 16) * 64 + l) * 4;
#pragma unroll
            for (int j = 0; j < NJ; ++j) o.q[j] = *reinterpret_cast<const v4f*>(qr + 256 * j);
#pragma unroll
            for (int j = 0; j < 4; ++j) o.p[j] = *reinterpret_cast<const v4f*>(pr + 256 * j);
#pragma unroll
            for (int vv = 0; vv < 4; ++vv) o.gm[vv] = a.gam[base * C + 16 * wq + 4 * g + vv];
        };
        auto chunk = [&](int c, const SplitOutOps<D>& o, SplitOutOps<D>& nx) __attribute__((always_inline)) {
            const int64_t t0 = (int64_t)c * C;
            const int n = (int)min<int64_t>(C, a.T - t0);
            load(min(c + 1, a.nc - 1), nx);
            const v4f qs = s0_product(o.q);
            __syncthreads();
            v4f dt[4];
#pragma unroll
            for (int j = 0; j < 4; ++j) dt[j] = *reinterpret_cast<const v4f*>(Dt + r * TP + 4 * g + 16 * j);
            v4f pd = v4f{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int j = 0; j < 4; ++j)
#pragma unroll
                for (int e = 0; e < 4; ++e) pd = __builtin_amdgcn_mfma_f32_16x16x4f32(o.p[j][e], dt[j][e], pd, 0, 0, 0);
            // O = scale (G Q S0 + P d)
#pragma unroll
            for (int vv = 0; vv < 4; ++vv) {
                const int t = 16 * wq + 4 * g + vv;
                if (t < n)
                    a.outs[((t0 + t) * a.n_v + h) * D + e0 + r] = a.scale * (o.gm[vv] * qs[vv] + pd[vv]);
            }
            __syncthreads();
        };
        SplitOutOps<D> oa, ob;
        load(0, oa);
        __syncthreads();
        for (int c = 0; c < a.nc; c += 2) {
            chunk(c, oa, ob);
            if (c + 1 >= a.nc) break;
            chunk(c + 1, ob, oa);
        }
    }
#pragma unroll
    for (int i = 0; i < D * NC / 512; ++i) {
        const int idx = tid + 512 * i, row = idx / NC, col = idx % NC;
        Sg[(int64_t)row * D + e0 + col] = St[col * SP + row];
    }
}

}  // namespace

// Long scans take the chunked form (measured faster on MI355X from a few
// chunks on).
static bool use_chunked(int64_t T, int64_t d) {
    return (d == 64 || d == 128 || d == 256) && T >= tune("ssm_chunk_min", 128) &&
           tune("ssm_chunk", 1) != 0;
}

int64_t ssm_workspace_bytes(int64_t T, int64_t n_k, int64_t n_v, int64_t d) {
    if (T <= 0 || n_k <= 0 || n_v <= 0 || d <= 0) return 0;
    const auto up = [](int64_t b) { return (b + 255) / 256 * 256; };
    int64_t b = 2 * up(T * n_k * d * 4) + 2 * up(T * n_v * 4);
    if (use_chunked(T, d)) {
        const int64_t nc = (T + kChunk - 1) / kChunk, rows = n_v * nc * kChunk;
        b += 2 * up(rows * d * 4) + up(rows * kChunk * 4) + 2 * up(rows * 4) + up(n_v * nc * 4) +
             2 * up(n_k * nc * kChunk * d * 4);
    }
    return b;
}

// q, k and v token rows qs, ks, vs floats apart (the reference's
// scan_strided, src/ssm.cpp:128-142: the SSM layer scans slices of its packed
// qkv rows); outs contiguous [T][n_v][d].
bool ssm_scan_strided_dev(const float* q, int64_t qs, const float* k, int64_t ks, const float* v,
                          int64_t vs, const float* alpha, const float* beta, const float* a_log,
                          const float* dt_bias, float* state, int64_t T, int64_t n_k, int64_t n_v,
                          int64_t d, float scale, float eps, float* outs, void* workspace,
                          int64_t ws_bytes, hipStream_t s) {
    if (T < 0 || n_k <= 0 || n_v <= 0 || n_v % n_k || d <= 0) {
        set_error("ssm_scan: bad sizes (T=%lld n_k=%lld n_v=%lld d=%lld)", (long long)T,
                  (long long)n_k, (long long)n_v, (long long)d);
        return false;
    }
    if (qs < n_k * d || ks < n_k * d || vs < n_v * d || qs % 4 || ks % 4 || vs % 4) {
        set_error("ssm_scan: row strides (q %lld, k %lld, v %lld) must cover a token's heads "
                  "and be multiples of 4 floats", (long long)qs, (long long)ks, (long long)vs);
        return false;
    }
    if (T == 0) return true;
    if (!q || !k || !v || !alpha || !beta || !a_log || !dt_bias || !state || !outs) {
        set_error("ssm_scan: null pointer");
        return false;
    }
    const int P = (d == 256 || tune("ssm_parts", 16) != 8) ? 16 : 8;
    const bool fused = T <= tune("ssm_fuse_tokens", 16);
    ScanKernel kern = pick_scan(d, P, fused);
    if (kern == nullptr) {
        set_error("ssm_scan: head dim %lld not in {64, 128, 256}", (long long)d);
        return false;
    }
    if (!aligned16(q) || !aligned16(k) || !aligned16(state) || !aligned16(workspace)) {
        set_error("ssm_scan: q, k, state and workspace must be 16-byte aligned");
        return false;
    }
    if (n_v > 0x7fffffff || T * n_k > 0x7fffffff) {
        set_error("ssm_scan: grid too large");
        return false;
    }
    const int64_t cw = 4 * (64 / P);
    const dim3 grid((unsigned)n_v, (unsigned)(d / cw));
    if (fused) {
        ScanArgs sa{q, k, v, qs, ks, vs, alpha, beta, a_log, dt_bias, state, outs, T, n_k, n_v,
                    scale, eps};
        return launch("ssm_scan_kernel", kern, grid, dim3(kScanThreads), 0, s, sa);
    }
    const int64_t need = ssm_workspace_bytes(T, n_k, n_v, d);
    if (workspace == nullptr || ws_bytes < need) {
        set_error("ssm_scan: workspace %lld bytes < %lld needed", (long long)ws_bytes,
                  (long long)need);
        return false;
    }
    const auto up = [](int64_t b) { return (b + 255) / 256 * 256; };
    char* w = static_cast<char*>(workspace);
    float* qn = reinterpret_cast<float*>(w);
    float* kn = reinterpret_cast<float*>(w + up(T * n_k * d * 4));
    float* dc = reinterpret_cast<float*>(w + 2 * up(T * n_k * d * 4));
    float* bb = reinterpret_cast<float*>(w + 2 * up(T * n_k * d * 4) + up(T * n_v * 4));
    const bool chunked = use_chunked(T, d);
    {
        const int64_t rows = T * n_k, per = 1024 / d;   // 256 threads, d / 4 a row
        const dim3 pg((unsigned)((rows + per - 1) / per));
        const int ld = chunked ? 1 : 0;
        const bool ok =
            d == 64 ? launch("ssm_prep_kernel", ssm_prep_kernel<16>, pg, dim3(256), 0, s, q, k, alpha,
                             beta, a_log, dt_bias, qn, kn, dc, bb, rows, n_k, n_v, qs, ks, eps, ld)
            : d == 128 ? launch("ssm_prep_kernel", ssm_prep_kernel<32>, pg, dim3(256), 0, s, q, k,
                                alpha, beta, a_log, dt_bias, qn, kn, dc, bb, rows, n_k, n_v, qs, ks,
                                eps, ld)
                       : launch("ssm_prep_kernel", ssm_prep_kernel<64>, pg, dim3(256), 0, s, q, k,
                                alpha, beta, a_log, dt_bias, qn, kn, dc, bb, rows, n_k, n_v, qs, ks,
                                eps, ld);
        if (!ok) return false;
    }
    if (chunked) {
        const int64_t nc = (T + kChunk - 1) / kChunk, rows = n_v * nc * kChunk;
        if (nc > 0x7fffffff || n_v > 65535) {
            set_error("ssm_scan: too many chunks or heads for the chunked scan");
            return false;
        }
        char* cw = w + 2 * up(T * n_k * d * 4) + 2 * up(T * n_v * 4);
        ChunkArgs ca{};
        ca.qn = qn;
        ca.kn = kn;
        ca.v = v;
        ca.vs = vs;
        ca.lg = dc;
        ca.bb = bb;
        ca.U = reinterpret_cast<float*>(cw);
        ca.W = reinterpret_cast<float*>(cw + up(rows * d * 4));
        ca.P = reinterpret_cast<float*>(cw + 2 * up(rows * d * 4));
        ca.gam = reinterpret_cast<float*>(cw + 2 * up(rows * d * 4) + up(rows * kChunk * 4));
        ca.kfac = reinterpret_cast<float*>(cw + 2 * up(rows * d * 4) + up(rows * kChunk * 4) +
                                           up(rows * 4));
        ca.gC = reinterpret_cast<float*>(cw + 2 * up(rows * d * 4) + up(rows * kChunk * 4) +
                                         2 * up(rows * 4));
        ca.Qop = reinterpret_cast<float*>(cw + 2 * up(rows * d * 4) + up(rows * kChunk * 4) +
                                          2 * up(rows * 4) + up(n_v * nc * 4));
        ca.state = state;
        ca.outs = outs;
        ca.T = T;
        ca.n_k = n_k;
        ca.n_v = n_v;
        ca.nc = (int)nc;
        ca.scale = scale;
        if (!aligned16(v) || !aligned16(outs)) {
            set_error("ssm_scan: v and outs must be 16-byte aligned for the chunked scan");
            return false;
        }
        ca.Kop = reinterpret_cast<float*>(reinterpret_cast<char*>(ca.Qop) + up(n_k * nc * kChunk * d * 4));
        // chunk pre-pass: one workgroup a (chunk, value head); state pass: one
        // a (value head, 16 state columns), 256 at Qwen3-Next's 32 heads of 128
        const dim3 pgrid((unsigned)nc, (unsigned)n_v), sgrid((unsigned)n_v, (unsigned)(d / 16));
        // head dims 64 and 128: two waves a SIMD (AERO_HIP_TUNE ssm_split=0:
        // the one-wave form, measured 3-7% slower on MI355X)
        const bool split = tune("ssm_split", 1) != 0;
        if (d == 64)
            return launch("ssm_chunk_prep_kernel", ssm_chunk_prep_kernel<64>, pgrid, dim3(256), 0, s, ca) &&
                   (split ? launch("ssm_chunk_split_kernel", ssm_chunk_split_kernel<64>, sgrid, dim3(512), 0, s, ca)
                          : launch("ssm_chunk_scan_kernel", ssm_chunk_scan_kernel<64, 1>, sgrid, dim3(256), 0, s, ca));
        if (d == 256)
            return launch("ssm_chunk_prep_kernel", ssm_chunk_prep_kernel<256>, pgrid, dim3(256), 0, s, ca) &&
                   launch("ssm_chunk_scan_kernel", ssm_chunk_scan_kernel<256, 1>, sgrid, dim3(256), 0, s, ca);
        return launch("ssm_chunk_prep_kernel", ssm_chunk_prep_kernel<128>, pgrid, dim3(256), 0, s, ca) &&
               (split ? launch("ssm_chunk_split_kernel", ssm_chunk_split_kernel<128>, sgrid, dim3(512), 0, s, ca)
                      : launch("ssm_chunk_scan_kernel", ssm_chunk_scan_kernel<128, 1>, sgrid, dim3(256), 0, s, ca));
    }
    ScanArgs sa{qn, kn, v, n_k * d, n_k * d, vs, dc, bb, nullptr, nullptr, state, outs, T, n_k,
                n_v, scale, eps};
    return launch("ssm_scan_kernel", kern, grid, dim3(kScanThreads), 0, s, sa);
}

bool ssm_scan_dev(const float* q, const float* k, const float* v, const float* alpha,
                  const float* beta, const float* a_log, const float* dt_bias, float* state,
                  int64_t T, int64_t n_k, int64_t n_v, int64_t d, float scale, float eps,
                  float* outs, void* workspace, int64_t ws_bytes, hipStream_t s) {
    return ssm_scan_strided_dev(q, n_k * d, k, n_k * d, v, n_v * d, alpha, beta, a_log, dt_bias,
                                state, T, n_k, n_v, d, scale, eps, outs, workspace, ws_bytes, s);
}

// silu: out = silu(conv) (the SSM layer's order, src/ssm.cpp:298-301)
bool ssm_conv_act_dev(const float* x, const float* w, const float* tail, int64_t tail_len,
                      float* tail_out, float* out, int64_t T, int64_t C, int64_t K, bool silu,
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
    constexpr int kTB = 32, kTB4 = 16;
    bool tail_done = false;
    // the 4-channel form from 64 tokens (short calls are all boundary blocks:
    // the one-channel form spreads them over 4x the lanes)
    if (T >= 4 * kTB4 && K == 4 && C % 4 == 0 && aligned16(x) && aligned16(w) &&
        aligned16(out) && (T + kTB4 - 1) / kTB4 <= 65535) {
        const dim3 grid((unsigned)((C / 4 + 255) / 256), (unsigned)((T + kTB4 - 1) / kTB4));
        if (!launch("ssm_conv_kernel", silu ? ssm_conv4_kernel<kTB4, true> : ssm_conv4_kernel<kTB4, false>,
                    grid, dim3(256), 0, s, x, w, tail, out, tail_len, T, C))
            return false;
    } else if (T > 0) {
        const dim3 gk((unsigned)((C + 255) / 256), (unsigned)((T + kTB - 1) / kTB));
        const dim3 g1((unsigned)((T * C + 255) / 256));
        // one block of tokens: the conv kernel writes the new history itself
        tail_done = K == 4 && T <= kTB;
        float* to = tail_done ? tail_out : nullptr;
        const bool ok =
            (K == 4 && (T + kTB - 1) / kTB <= 65535)
                ? launch("ssm_conv_kernel", silu ? ssm_conv_k_kernel<4, kTB, true> : ssm_conv_k_kernel<4, kTB, false>,
                         gk, dim3(256), 0, s, x, w, tail, out, tail_len, T, C, to, (int)keep)
                : launch("ssm_conv_kernel", silu ? ssm_conv_kernel<true> : ssm_conv_kernel<false>, g1,
                         dim3(256), 0, s, x, w, tail, out, tail_len, T, C, (int)K);
        if (!ok) return false;
    }
    if (keep > 0 && !tail_done && !launch("ssm_conv_tail_kernel", ssm_conv_tail_kernel,
                            dim3((unsigned)((C + 255) / 256)), dim3(256), 0, s, x, tail,
                            tail_out, tail_len, T, C, (int)keep))
        return false;
    if (new_tail_len) *new_tail_len = keep;
    return true;
}

bool ssm_conv_dev(const float* x, const float* w, const float* tail, int64_t tail_len,
                  float* tail_out, float* out, int64_t T, int64_t C, int64_t K,
                  int64_t* new_tail_len, hipStream_t s) {
    return ssm_conv_act_dev(x, w, tail, tail_len, tail_out, out, T, C, K, false, new_tail_len, s);
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

int aero_hip_ssm_scan_strided(const float* q, int64_t q_stride, const float* k, int64_t k_stride,
                              const float* v, int64_t v_stride, const float* alpha,
                              const float* beta, const float* a_log, const float* dt_bias,
                              float* state, int64_t T, int64_t n_k, int64_t n_v, int64_t d,
                              float scale, float eps, float* outs, void* workspace,
                              int64_t ws_bytes, void* stream) {
    aero::clear_error();
    return aero::ssm_scan_strided_dev(q, q_stride, k, k_stride, v, v_stride, alpha, beta, a_log,
                                      dt_bias, state, T, n_k, n_v, d, scale, eps, outs, workspace,
                                      ws_bytes, (hipStream_t)stream) ? 1 : 0;
}

int aero_hip_ssm_conv_silu(const float* x, const float* w, const float* tail, int64_t tail_len,
                           float* tail_out, float* out, int64_t T, int64_t channels,
                           int64_t kernel, int64_t* new_tail_len, void* stream) {
    aero::clear_error();
    return aero::ssm_conv_act_dev(x, w, tail, tail_len, tail_out, out, T, channels, kernel, true,
                                  new_tail_len, (hipStream_t)stream) ? 1 : 0;
}

}  // extern "C"
