// RoPE on gfx950, fused with the per-head RMSNorm that precedes it
// (src/attention_layer.cpp:89-156: q/k norm per head, then NeoX rotation at
// the token's position).
//
// Layout: q [n_tok, hq, D] and k [n_tok, hk, D]; a token's hq + hk head rows
// share its position. A workgroup takes one token and a range of its heads.
// Its first `half` lanes produce the token's cos/sin pairs once (fp32 angle
// (float)pos*inv[p] then sincos, or a gather from a position-indexed table)
// into LDS, so the transcendental work is per token, not per head row.
//
// Each head row is owned by L lanes (L = D/8 when the whole row is touched,
// n_rot/8 otherwise); every lane holds two float4 chunks:
//   NeoX rotation lane j:        x[4j..4j+3]   and x[half+4j..half+4j+3]
//   interleaved rotation lane j: x[8j..8j+3]   and x[8j+4..8j+7]
//   pass-through lane j:         x[n_rot+8m .. n_rot+8m+7], m = j - n_rot/8
// so both members of every rotated pair sit in the same lane and no shuffle
// is needed for the rotation; the norm's sum of squares is an xor butterfly
// over the L lanes. All loads of a lane's rows are issued before the LDS
// barrier, and each element is read once and written once: HBM bytes per
// head row 8*D (4*D read + 4*D written; 8*n_rot for an in-place partial
// rotation without norm, which touches only the rotated channels).
//
// Arithmetic with contraction off, in the reference's order:
// norm (x*inv)*w with inv = 1/sqrtf(ss/D + eps) (src/tensor.cpp:128-134);
// rotation x0*c - x1*s, x0*s + x1*c (src/transformer.cpp:77-93).
#include "common.hpp"
#include "aero_hip.h"

#include <cmath>

#pragma clang fp contract(off)

namespace aero {
namespace {

struct RopeParams {
    float* q;
    float* q_out;
    const float* q_w;
    float* k;
    float* k_out;
    const float* k_w;
    int hq, hk;
    int64_t n_tok;
    int D, n_rot, mode;
    float eps;
    int norm_flags;
    const int32_t* pos;
    const float* inv;
    const float* ctab;
    const float* stab;
    int64_t n_tab;
    int hpw;      // heads per workgroup
    int n_hg;     // workgroups per token
    int do_tail;  // lanes beyond n_rot/8 carry the pass-through channels
};

constexpr int kRopeBlock = 256;

__device__ __forceinline__ float4 ld4(const float* p) {
    return *reinterpret_cast<const float4*>(p);
}

__device__ __forceinline__ float4 wmul(float4 v, float inv, const float* w, int flags) {
    float4 o = make_float4(v.x * inv, v.y * inv, v.z * inv, v.w * inv);
    float4 wv = ld4(w);
    if (flags & AERO_NORM_UNIT_OFFSET) {
        wv.x = 1.0f + wv.x; wv.y = 1.0f + wv.y; wv.z = 1.0f + wv.z; wv.w = 1.0f + wv.w;
    }
    o.x = o.x * wv.x; o.y = o.y * wv.y; o.z = o.z * wv.z; o.w = o.w * wv.w;
    return o;
}

__device__ __forceinline__ void rot2(float& x0, float& x1, float c, float s) {
    const float a = x0, b = x1;
    x0 = a * c - b * s;
    x1 = a * s + b * c;
}

template <int L, int RPS>
__global__ __launch_bounds__(kRopeBlock)
void rope_vec_kernel(RopeParams p) {
    constexpr int S = kRopeBlock / L;
    __shared__ float4 cs_c[64];
    __shared__ float4 cs_s[64];

    const int tid = threadIdx.x;
    const int64_t t = blockIdx.x / p.n_hg;
    const int hg = blockIdx.x % p.n_hg;
    const int NH = p.hq + p.hk;
    const int h0 = hg * p.hpw;
    const int h1 = min(h0 + p.hpw, NH);
    const int s = tid / L;
    const int j = tid % L;
    const int half = p.n_rot >> 1;
    const int r8 = p.n_rot >> 3;

    const int64_t pt = p.pos ? (int64_t)p.pos[t] : t;
    if (p.inv == nullptr && (pt < 0 || pt >= p.n_tab)) return;  // uniform per block

    // element offsets of this lane's two chunks inside a head row
    const bool rot = j < r8;
    const bool active = rot || (p.do_tail && j < (p.D >> 3));
    int a0, b0;
    if (rot) {
        a0 = p.mode == AERO_ROPE_NEOX ? 4 * j : 8 * j;
        b0 = p.mode == AERO_ROPE_NEOX ? half + 4 * j : 8 * j + 4;
    } else {
        a0 = p.n_rot + 8 * (j - r8);
        b0 = a0 + 4;
    }

    float4 A[RPS], B[RPS];
    const float* wrow[RPS];
    int rowoff[RPS];   // element offset of the row inside its token's q or k block
    bool isq_row[RPS];
    bool valid[RPS];
#pragma unroll
    for (int i = 0; i < RPS; ++i) {
        const int h = h0 + s + S * i;
        valid[i] = active && h < h1;
        A[i] = make_float4(0.f, 0.f, 0.f, 0.f);
        B[i] = A[i];
        wrow[i] = nullptr;
        rowoff[i] = 0;
        isq_row[i] = true;
        if (h < h1) {
            const bool isq = h < p.hq;
            isq_row[i] = isq;
            rowoff[i] = (isq ? h : h - p.hq) * p.D;
            const int64_t roff = t * (int64_t)(isq ? p.hq : p.hk) * p.D + rowoff[i];
            const float* src = (isq ? p.q : p.k) + roff;
            wrow[i] = isq ? p.q_w : p.k_w;
            if (valid[i]) {
                A[i] = ld_stream(src + a0);
                B[i] = ld_stream(src + b0);
            }
        }
    }

    // the token's cos/sin for pairs 0..half-1, once per workgroup
    if (tid < half) {
        float c, sn;
        if (p.inv != nullptr) {
            const float ang = (float)pt * p.inv[tid];
            sincosf(ang, &sn, &c);
        } else {
            c = p.ctab[pt * half + tid];
            sn = p.stab[pt * half + tid];
        }
        reinterpret_cast<float*>(cs_c)[tid] = c;
        reinterpret_cast<float*>(cs_s)[tid] = sn;
    }
    __syncthreads();

    // this token's q rows and k rows, each a contiguous block of heads x D
    const StreamOut oq(p.q_out + t * (int64_t)p.hq * p.D, (int64_t)p.hq * p.D * 4);
    const StreamOut ok_(p.hk > 0 ? p.k_out + t * (int64_t)p.hk * p.D : p.q_out,
                        (int64_t)p.hk * p.D * 4);

    float4 c4 = make_float4(1.f, 1.f, 1.f, 1.f), s4 = make_float4(0.f, 0.f, 0.f, 0.f);
    if (rot) {
        c4 = cs_c[j];
        s4 = cs_s[j];
    }

#pragma unroll
    for (int i = 0; i < RPS; ++i) {
        // sum of squares over the whole head row (all L lanes of the slot)
        float ss = 0.0f;
        ss += A[i].x * A[i].x; ss += A[i].y * A[i].y;
        ss += A[i].z * A[i].z; ss += A[i].w * A[i].w;
        ss += B[i].x * B[i].x; ss += B[i].y * B[i].y;
        ss += B[i].z * B[i].z; ss += B[i].w * B[i].w;
        ss = group_sum<L>(ss);
        if (!valid[i]) continue;
        if (wrow[i] != nullptr) {
            const float inv = 1.0f / sqrtf(ss / (float)p.D + p.eps);
            A[i] = wmul(A[i], inv, wrow[i] + a0, p.norm_flags);
            B[i] = wmul(B[i], inv, wrow[i] + b0, p.norm_flags);
        }
        if (rot) {
            if (p.mode == AERO_ROPE_NEOX) {
                rot2(A[i].x, B[i].x, c4.x, s4.x);
                rot2(A[i].y, B[i].y, c4.y, s4.y);
                rot2(A[i].z, B[i].z, c4.z, s4.z);
                rot2(A[i].w, B[i].w, c4.w, s4.w);
            } else {
                rot2(A[i].x, A[i].y, c4.x, s4.x);
                rot2(A[i].z, A[i].w, c4.y, s4.y);
                rot2(B[i].x, B[i].y, c4.z, s4.z);
                rot2(B[i].z, B[i].w, c4.w, s4.w);
            }
        }
        const uint32_t off = (uint32_t)(rowoff[i] + a0) * 4u;
        const uint32_t offb = (uint32_t)(rowoff[i] + b0) * 4u;
        if (isq_row[i]) {
            oq.store(off, A[i]);
            oq.store(offb, B[i]);
        } else {
            ok_.store(off, A[i]);
            ok_.store(offb, B[i]);
        }
    }
}

// Any head_dim / n_rot / alignment: one wave per head row. Pass 1 writes the
// normalised (or copied) row to its destination, pass 2 rotates pairs there.
__global__ __launch_bounds__(64) void rope_scalar_kernel(RopeParams p) {
    const int lane = threadIdx.x;
    const int NH = p.hq + p.hk;
    const int64_t t = blockIdx.x / NH;
    const int h = blockIdx.x % NH;
    const int64_t pt = p.pos ? (int64_t)p.pos[t] : t;
    if (p.inv == nullptr && (pt < 0 || pt >= p.n_tab)) return;
    const bool isq = h < p.hq;
    const int64_t roff = (t * (isq ? p.hq : p.hk) + (isq ? h : h - p.hq)) * (int64_t)p.D;
    const float* src = (isq ? p.q : p.k) + roff;
    float* dst = (isq ? p.q_out : p.k_out) + roff;
    const float* w = isq ? p.q_w : p.k_w;
    if (w != nullptr) {
        float ss = 0.0f;
        for (int c = lane; c < p.D; c += 64) ss += src[c] * src[c];
        ss = group_sum<64>(ss);
        const float inv = 1.0f / sqrtf(ss / (float)p.D + p.eps);
        for (int c = lane; c < p.D; c += 64) {
            const float wc = (p.norm_flags & AERO_NORM_UNIT_OFFSET) ? 1.0f + w[c] : w[c];
            dst[c] = (src[c] * inv) * wc;
        }
    } else if (dst != src) {
        for (int c = lane; c < p.D; c += 64) dst[c] = src[c];
    }
    __syncthreads();
    const int half = p.n_rot >> 1;
    for (int q = lane; q < half; q += 64) {
        float c, sn;
        if (p.inv != nullptr) {
            sincosf((float)pt * p.inv[q], &sn, &c);
        } else {
            c = p.ctab[pt * half + q];
            sn = p.stab[pt * half + q];
        }
        const int i0 = p.mode == AERO_ROPE_NEOX ? q : 2 * q;
        const int i1 = p.mode == AERO_ROPE_NEOX ? q + half : 2 * q + 1;
        float x0 = dst[i0], x1 = dst[i1];
        rot2(x0, x1, c, sn);
        dst[i0] = x0;
        dst[i1] = x1;
    }
}

__global__ __launch_bounds__(256)
void rope_tables_kernel(const int32_t* pos, int64_t n_pos, const float* inv,
                        int half, float* cos_out, float* sin_out) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= n_pos * half) return;
    const int64_t t = i / half;
    const int q = (int)(i % half);
    float sn, c;
    sincosf((float)pos[t] * inv[q], &sn, &c);
    cos_out[i] = c;
    sin_out[i] = sn;
}

using RopeKernel = void (*)(RopeParams);

template <int L>
RopeKernel pick_rps(int rps) {
    switch (rps) {
    case 1: return rope_vec_kernel<L, 1>;
    case 2: return rope_vec_kernel<L, 2>;
    case 3: return rope_vec_kernel<L, 3>;
    case 4: return rope_vec_kernel<L, 4>;
    case 5: return rope_vec_kernel<L, 5>;
    case 6: return rope_vec_kernel<L, 6>;
    case 7: return rope_vec_kernel<L, 7>;
    case 8: return rope_vec_kernel<L, 8>;
    default: return nullptr;
    }
}

RopeKernel pick_rope(int L, int rps) {
    switch (L) {
    case 2: return pick_rps<2>(rps);
    case 4: return pick_rps<4>(rps);
    case 8: return pick_rps<8>(rps);
    case 16: return pick_rps<16>(rps);
    case 32: return pick_rps<32>(rps);
    case 64: return pick_rps<64>(rps);
    default: return nullptr;
    }
}

int next_pow2(int v) {
    int p = 1;
    while (p < v) p <<= 1;
    return p;
}

}  // namespace

bool qk_norm_rope(RopeParams p, hipStream_t stream) {
    const int NH = p.hq + p.hk;
    if (p.n_tok == 0 || NH == 0) return true;
    const bool norm = p.q_w != nullptr || p.k_w != nullptr;
    const bool out_of_place = p.q_out != p.q || (p.k != nullptr && p.k_out != p.k);
    if (p.n_rot == 0 && !norm && !out_of_place) return true;
    p.do_tail = (norm || out_of_place) ? 1 : 0;

    bool vec = p.D % 8 == 0 && p.n_rot % 8 == 0 && aligned16(p.q) && aligned16(p.q_out) &&
               (p.k == nullptr || (aligned16(p.k) && aligned16(p.k_out))) &&
               (p.q_w == nullptr || aligned16(p.q_w)) &&
               (p.k_w == nullptr || aligned16(p.k_w));
    int L = 0;
    if (vec) {
        L = p.do_tail ? p.D / 8 : next_pow2(p.n_rot / 8);
        vec = L >= 2 && L <= 64 && (L & (L - 1)) == 0 && (!p.do_tail || L * 8 == p.D);
    }
    const int64_t blocks_cap = 0x7fffffff;
    if (vec) {
        const int S = kRopeBlock / L;
        const int need = (NH + S - 1) / S;
        const int rps_max = tune("rope_rps_max", 8);
        const int64_t min_wg = tune("rope_min_wg", 1024);
        int rps = need < rps_max ? need : rps_max;
        if (rps < 1) rps = 1;
        int n_hg = 1;
        for (;; --rps) {
            n_hg = (NH + S * rps - 1) / (S * rps);
            if (rps == 1 || p.n_tok * n_hg >= min_wg) break;
        }
        p.n_hg = n_hg;
        p.hpw = (NH + n_hg - 1) / n_hg;
        rps = (p.hpw + S - 1) / S;
        if (rps > 8) {  // more heads than 8 slots per lane group: add groups
            p.n_hg = (NH + S * 8 - 1) / (S * 8);
            p.hpw = (NH + p.n_hg - 1) / p.n_hg;
            rps = (p.hpw + S - 1) / S;
        }
        const int64_t blocks = p.n_tok * p.n_hg;
        if (blocks > blocks_cap) {
            set_error("qk_norm_rope: grid too large");
            return false;
        }
        return launch("rope_vec_kernel", pick_rope(L, rps), dim3((unsigned)blocks),
                      dim3(kRopeBlock), 0, stream, p);
    }
    const int64_t blocks = p.n_tok * NH;
    if (blocks > blocks_cap) {
        set_error("qk_norm_rope: grid too large");
        return false;
    }
    return launch("rope_scalar_kernel", rope_scalar_kernel, dim3((unsigned)blocks),
                  dim3(64), 0, stream, p);
}

bool rope_tables_dev(const int32_t* pos, int64_t n_pos, const float* inv, int64_t half,
                     float* c, float* s, hipStream_t stream) {
    if (n_pos == 0 || half == 0) return true;
    const int64_t total = n_pos * half;
    const int64_t blocks = (total + 255) / 256;
    if (blocks > 0x7fffffff) {
        set_error("rope_tables: too large");
        return false;
    }
    return launch("rope_tables_kernel", rope_tables_kernel, dim3((unsigned)blocks),
                  dim3(256), 0, stream, pos, n_pos, inv, (int)half, c, s);
}

// src/transformer.cpp:34-47, evaluated on the host in fp32 with the same
// expression so that the device angle (float)pos*inv matches bit for bit.
int64_t rope_inv_freq_host(int64_t head_dim, int64_t n_dims, float base,
                           const float* ff, int64_t n_ff, float* inv_out) {
    if (head_dim <= 0) return -1;
    int64_t n = (n_dims <= 0) ? head_dim : (n_dims < head_dim ? n_dims : head_dim);
    n -= n % 2;
    const int64_t half = n / 2;
    if (half <= 0) return n;
    if (ff != nullptr && n_ff < half) return -1;
    for (int64_t q = 0; q < half; ++q) {
        const float e = (float)((float)q * 2.0f / (float)n);
        float inv = 1.0f / std::pow(base, e);
        if (ff != nullptr) inv /= ff[q];
        inv_out[q] = inv;
    }
    return n;
}

}  // namespace aero

extern "C" {

int64_t aero_hip_rope_inv_freq(int64_t head_dim, int64_t n_dims, float base,
                               const float* freq_factors, int64_t n_ff,
                               float* inv_out) {
    if (inv_out == nullptr) {
        aero::set_error("rope_inv_freq: null output");
        return -1;
    }
    const int64_t n = aero::rope_inv_freq_host(head_dim, n_dims, base, freq_factors,
                                               n_ff, inv_out);
    if (n < 0) aero::set_error("rope_inv_freq: refused (head_dim or freq_factors)");
    return n;
}

int aero_hip_rope_tables(const int32_t* pos, int64_t n_pos, const float* inv,
                         int64_t half, float* cos_out, float* sin_out, void* stream) {
    if (!pos || !inv || !cos_out || !sin_out || n_pos < 0 || half < 0 ||
        half > (1 << 24)) {
        aero::set_error("rope_tables: bad arguments");
        return 0;
    }
    return aero::rope_tables_dev(pos, n_pos, inv, half, cos_out, sin_out,
                                 (hipStream_t)stream) ? 1 : 0;
}

int aero_hip_qk_norm_rope(float* q, float* q_out, int64_t n_q_heads, float* k,
                          float* k_out, int64_t n_k_heads, const float* q_norm_w,
                          const float* k_norm_w, float eps, int norm_flags,
                          int64_t n_tok, int64_t head_dim, int64_t n_rot, int mode,
                          const int32_t* pos, const float* inv_freq,
                          const float* cos_tab, const float* sin_tab, int64_t n_tab,
                          void* stream) {
    if (q == nullptr || n_q_heads < 0 || n_k_heads < 0 || n_tok < 0 || head_dim <= 0 ||
        n_rot < 0 || n_rot > head_dim || n_rot > 512 || head_dim > (1 << 20) ||
        n_q_heads + n_k_heads > (1 << 20) || (n_k_heads > 0 && k == nullptr) ||
        (mode != AERO_ROPE_NEOX && mode != AERO_ROPE_INTERLEAVED)) {
        aero::set_error("qk_norm_rope: bad arguments (heads=%lld/%lld D=%lld n_rot=%lld "
                        "mode=%d)", (long long)n_q_heads, (long long)n_k_heads,
                        (long long)head_dim, (long long)n_rot, mode);
        return 0;
    }
    const bool have_inv = inv_freq != nullptr;
    const bool have_tab = cos_tab != nullptr || sin_tab != nullptr;
    if (n_rot >= 2 && have_inv == have_tab) {
        aero::set_error("qk_norm_rope: give exactly one of inv_freq or cos/sin tables");
        return 0;
    }
    if (have_tab && (cos_tab == nullptr || sin_tab == nullptr || n_tab < 0)) {
        aero::set_error("qk_norm_rope: table needs cos, sin and n_tab >= 0");
        return 0;
    }
    aero::RopeParams p{};
    p.q = q;
    p.q_out = q_out ? q_out : q;
    p.q_w = q_norm_w;
    p.k = n_k_heads > 0 ? k : nullptr;
    p.k_out = n_k_heads > 0 ? (k_out ? k_out : k) : nullptr;
    p.k_w = n_k_heads > 0 ? k_norm_w : nullptr;
    p.hq = (int)n_q_heads;
    p.hk = (int)n_k_heads;
    p.n_tok = n_tok;
    p.D = (int)head_dim;
    p.n_rot = (int)(n_rot & ~int64_t(1));
    p.mode = mode;
    p.eps = eps;
    p.norm_flags = norm_flags;
    p.pos = pos;
    p.inv = have_tab ? nullptr : inv_freq;
    p.ctab = cos_tab;
    p.stab = sin_tab;
    p.n_tab = have_tab ? n_tab : 0;
    if (p.n_rot < 2 && p.inv == nullptr && !have_tab) {
        // nothing rotates: keep the norm/copy path (it never reads a table)
        p.n_tab = (int64_t)1 << 62;
        p.pos = nullptr;
    }
    return aero::qk_norm_rope(p, (hipStream_t)stream) ? 1 : 0;
}

}  // extern "C"
