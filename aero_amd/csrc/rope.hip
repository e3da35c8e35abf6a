// RoPE on gfx950, fused with the per-head RMSNorm that precedes it
// (src/attention_layer.cpp:89-156: q/k norm per head, then NeoX rotation at
// the token's position).
//
// Layout: q [n_tok, hq, D] and k [n_tok, hk, D]; a token's hq + hk head rows
// share its position. A workgroup takes a tile of TW consecutive tokens and
// a group of their heads (TW x heads rows). Its lanes first produce the cos/sin
// pairs of the tile's tokens (fp32 angle (float)pos*inv[p] then sincos, or a
// gather from a position-indexed table) into LDS, so the transcendental work
// is per token, not per head row.
//
// Each head row is owned by L lanes (L = D/8 when the whole row is touched,
// n_rot/8 rounded up to a power of two otherwise), each holding two float4
// chunks (chunk c = x[4c..4c+3]) chosen so that every load instruction of a
// wave reads contiguous 16-byte chunks and both members of every rotated pair
// sit in the same lane (no shuffle for the rotation):
//   NeoX, rotating lane j < n_rot/8:   chunks j and j + n_rot/8 (x[p], x[p+half])
//   NeoX, pass-through lane j:         chunks n_rot/4 + m and n_rot/4 + m + (L - n_rot/8),
//                                      m = j - n_rot/8
//   interleaved lane j:                chunks j and j + span (span = L, or n_rot/8
//                                      in place), each rotated iff below n_rot
// The norm's sum of squares is an xor butterfly over the L lanes. A lane owns
// up to RPS rows of the tile; all their loads are issued before the LDS
// barrier, and each element is read once and written once: HBM bytes per head
// row 8*D (4*D read + 4*D written; 8*n_rot for an in-place partial rotation
// without norm, which touches only the rotated channels).
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
    int n_hg;     // head groups per token tile
    int tw;       // tokens per tile
    int do_tail;  // lanes beyond n_rot/8 carry the pass-through channels
};

constexpr int kRopeBlock = 256;
constexpr int kRopeLds = kRopeBlock;  // cos (and sin) floats of one tile: TW * n_rot/2
constexpr int kRopeMaxTw = 64;  // tokens per tile
// Read-only stand-in for an absent positions array.
// Global (not constant) memory on purpose: a select between them and a kernel
// argument pointer then stays a global load (a constant-space address would
// turn it into a flat load, which the compiler can only wait for with the
// whole vector-memory counter).
__device__ int32_t kZeroInt[1] = {0};

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

// TABLE: angles from the position-indexed cos/sin table (else computed from
// p.inv); one path per instantiation keeps the load counts exact.
template <int L, int RPS, bool TABLE>
__global__ __launch_bounds__(kRopeBlock)
void rope_vec_kernel(RopeParams p) {
    constexpr int S = kRopeBlock / L;
    __shared__ __align__(16) float cs_c[kRopeLds];
    __shared__ __align__(16) float cs_s[kRopeLds];
    static_assert(kRopeLds <= kRopeBlock, "one cos/sin entry per lane");
    __shared__ int tok_ok[kRopeMaxTw];

    const int tid = threadIdx.x;
    const int tile = (int)(blockIdx.x / p.n_hg);
    const int hg = (int)(blockIdx.x - (unsigned)tile * p.n_hg);
    const int64_t t0 = (int64_t)tile * p.tw;
    const int tw = (int)min((int64_t)p.tw, p.n_tok - t0);
    const int NH = p.hq + p.hk;
    const int h0 = hg * p.hpw;
    const int hn = min(h0 + p.hpw, NH) - h0;
    const int rows = tw * hn;
    const int s = tid / L;
    const int j = tid % L;
    const int half = p.n_rot >> 1;
    const int r8 = p.n_rot >> 3;

    int cA, cB;
    bool rotA, rotB;
    if (p.mode == AERO_ROPE_NEOX) {
        if (j < r8) {
            cA = j; cB = j + r8; rotA = rotB = true;
        } else {
            cA = 2 * r8 + (j - r8); cB = cA + (L - r8); rotA = rotB = false;
        }
    } else {
        const int span = p.do_tail ? L : r8;
        cA = j; cB = j + span;
        rotA = cA < 2 * r8; rotB = cB < 2 * r8;
    }
    const bool active = p.do_tail || j < r8;
    const int a0 = 4 * cA, b0 = 4 * cB;

    // The position (and inverse frequency) of this lane's cos/sin entry is
    // loaded first, from a clamped index, and used only after the row loads
    // are issued: the vector-memory counter retires in order, so the angle is
    // computed while the rows are in flight. Without positions the load reads
    // a one-element stand-in with stride 0, so no branch separates the load
    // from its use.
    const int n_fill = tw * half;  // <= kRopeBlock: one entry per lane
    const int fidx = min(tid, n_fill > 0 ? n_fill - 1 : 0);
    const int hdiv = half > 0 ? half : 1;
    const int fti = fidx / hdiv;
    const int fq = fidx - fti * hdiv;
    const int32_t* pos_base = p.pos != nullptr ? p.pos + t0 : kZeroInt;
    const int pos_step = p.pos != nullptr ? 1 : 0;
    const int fpos = pos_base[fti * pos_step];
    const float finv = TABLE ? 0.0f : p.inv[fq];
    const int my_pos = pos_base[min(tid, tw - 1) * pos_step];  // token `tid` of the tile

    // Row loads are unconditional too (a lane past the tile's rows re-reads
    // its last row, an idle lane reads chunk 0), so the compiler knows how
    // many loads follow the position loads; invalid values are masked later.
    float4 A[RPS], B[RPS];
#pragma unroll
    for (int i = 0; i < RPS; ++i) {
        const int r = min(s + S * i, rows - 1);
        const int ti = p.tw == 1 ? 0 : r / hn;
        const int h = h0 + (r - ti * hn);
        const bool isq = h < p.hq;
        const int64_t roff = ((t0 + ti) * (isq ? p.hq : p.hk) + (isq ? h : h - p.hq)) *
                             (int64_t)p.D;
        const float* src = (isq ? p.q : p.k) + roff;
        A[i] = ld_stream(src + (active ? a0 : 0));
        B[i] = ld_stream(src + (active ? b0 : 0));
    }

    // cos/sin of pairs 0..half-1 for each token of the tile (lanes past the
    // tile's entries compute a copy of the last one and do not store it)
    if (tid < tw) {  // a token outside its table is left untouched
        const int64_t pt = p.pos != nullptr ? (int64_t)my_pos : t0 + tid;
        tok_ok[tid] = !TABLE || (pt >= 0 && pt < p.n_tab);
    }
    if (n_fill > 0) {
        const int64_t pt = p.pos != nullptr ? (int64_t)fpos : t0 + fti;
        float c = 1.0f, sn = 0.0f;
        if (!TABLE) {
            const float ang = (float)pt * finv;
            sincosf(ang, &sn, &c);
        } else if (p.n_tab > 0) {  // clamped read; out-of-table tokens are skipped
            const int64_t pc = pt < 0 ? 0 : (pt >= p.n_tab ? p.n_tab - 1 : pt);
            c = p.ctab[pc * half + fq];
            sn = p.stab[pc * half + fq];
        }
        if (tid < n_fill) {
            cs_c[tid] = c;
            cs_s[tid] = sn;
        }
    }
    __syncthreads();

    // the tile's q rows and k rows, each a contiguous block of tokens x heads x D
    const StreamOut oq(p.q_out + t0 * p.hq * (int64_t)p.D, (int64_t)tw * p.hq * p.D * 4);
    const StreamOut ok_(p.hk > 0 ? p.k_out + t0 * p.hk * (int64_t)p.D : p.q_out,
                        (int64_t)tw * p.hk * p.D * 4);

#pragma unroll
    for (int i = 0; i < RPS; ++i) {
        const int r = s + S * i;
        if (!active || r >= rows) {
            A[i] = make_float4(0.f, 0.f, 0.f, 0.f);
            B[i] = A[i];
        }
        // sum of squares over the whole head row (all L lanes of the slot)
        float ss = 0.0f;
        ss += A[i].x * A[i].x; ss += A[i].y * A[i].y;
        ss += A[i].z * A[i].z; ss += A[i].w * A[i].w;
        ss += B[i].x * B[i].x; ss += B[i].y * B[i].y;
        ss += B[i].z * B[i].z; ss += B[i].w * B[i].w;
        ss = group_sum<L>(ss);
        if (!active || r >= rows) continue;
        const int ti = p.tw == 1 ? 0 : r / hn;
        const int h = h0 + (r - ti * hn);
        const bool isq = h < p.hq;
        if (!tok_ok[ti]) continue;
        const float* w = isq ? p.q_w : p.k_w;
        if (w != nullptr) {
            const float inv = 1.0f / sqrtf(ss / (float)p.D + p.eps);
            A[i] = wmul(A[i], inv, w + a0, p.norm_flags);
            B[i] = wmul(B[i], inv, w + b0, p.norm_flags);
        }
        const float* cc = cs_c + ti * half;
        const float* sc = cs_s + ti * half;
        if (p.mode == AERO_ROPE_NEOX) {
            if (rotA) {
                const float4 c4 = *reinterpret_cast<const float4*>(cc + 4 * j);
                const float4 s4 = *reinterpret_cast<const float4*>(sc + 4 * j);
                rot2(A[i].x, B[i].x, c4.x, s4.x);
                rot2(A[i].y, B[i].y, c4.y, s4.y);
                rot2(A[i].z, B[i].z, c4.z, s4.z);
                rot2(A[i].w, B[i].w, c4.w, s4.w);
            }
        } else {
            if (rotA) {
                const float2 c2 = *reinterpret_cast<const float2*>(cc + 2 * cA);
                const float2 s2 = *reinterpret_cast<const float2*>(sc + 2 * cA);
                rot2(A[i].x, A[i].y, c2.x, s2.x);
                rot2(A[i].z, A[i].w, c2.y, s2.y);
            }
            if (rotB) {
                const float2 c2 = *reinterpret_cast<const float2*>(cc + 2 * cB);
                const float2 s2 = *reinterpret_cast<const float2*>(sc + 2 * cB);
                rot2(B[i].x, B[i].y, c2.x, s2.x);
                rot2(B[i].z, B[i].w, c2.y, s2.y);
            }
        }
        const uint32_t row_off =
            (uint32_t)((ti * (isq ? p.hq : p.hk) + (isq ? h : h - p.hq)) * p.D);
        const uint32_t offa = (row_off + (uint32_t)a0) * 4u;
        const uint32_t offb = (row_off + (uint32_t)b0) * 4u;
        if (isq) {
            oq.store(offa, A[i]);
            oq.store(offb, B[i]);
        } else {
            ok_.store(offa, A[i]);
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

template <int L, bool TABLE>
RopeKernel pick_rps(int rps) {
    switch (rps) {
    case 1: return rope_vec_kernel<L, 1, TABLE>;
    case 2: return rope_vec_kernel<L, 2, TABLE>;
    case 3: return rope_vec_kernel<L, 3, TABLE>;
    case 4: return rope_vec_kernel<L, 4, TABLE>;
    case 5: return rope_vec_kernel<L, 5, TABLE>;
    case 6: return rope_vec_kernel<L, 6, TABLE>;
    case 7: return rope_vec_kernel<L, 7, TABLE>;
    case 8: return rope_vec_kernel<L, 8, TABLE>;
    default: return nullptr;
    }
}

template <bool TABLE>
RopeKernel pick_l(int L, int rps) {
    switch (L) {
    case 2: return pick_rps<2, TABLE>(rps);
    case 4: return pick_rps<4, TABLE>(rps);
    case 8: return pick_rps<8, TABLE>(rps);
    case 16: return pick_rps<16, TABLE>(rps);
    case 32: return pick_rps<32, TABLE>(rps);
    case 64: return pick_rps<64, TABLE>(rps);
    default: return nullptr;
    }
}

RopeKernel pick_rope(int L, int rps, bool table) {
    return table ? pick_l<true>(L, rps) : pick_l<false>(L, rps);
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
        // Heads of one token are split into groups only when they exceed
        // rps_max rows per lane, or to reach min_wg workgroups on short inputs.
        const int S = kRopeBlock / L;
        const int rps_max = std::min(8, std::max(1, tune("rope_rps_max", 8)));
        const int64_t min_wg = tune("rope_min_wg", 1024);
        const int half = p.n_rot / 2;
        int n_hg = (NH + S * rps_max - 1) / (S * rps_max);
        while (p.n_tok * n_hg < min_wg && (NH + n_hg - 1) / n_hg > S) ++n_hg;
        p.hpw = (NH + n_hg - 1) / n_hg;
        p.n_hg = (NH + p.hpw - 1) / p.hpw;
        // Tiles of several tokens only pay when one token per workgroup already
        // gives several rounds of workgroups (>= 4096): then tiles grow while a
        // workgroup moves < 64 KB and the grid keeps >= 512 workgroups. Swept
        // on MI355X over 1/2/4/8 tokens: 4096 x 18 heads, in-place 64/256
        // partial rotation 10.1 -> 8.6 us at 8 tokens; every other layer shape
        // equal or slower with tiles.
        const int64_t row_bytes = 8 * (int64_t)(p.do_tail ? p.D : p.n_rot);
        int tw = 1;
        if (p.n_tok * p.n_hg >= 4096)
            while (2 * tw <= kRopeMaxTw && 2 * tw * (half > 0 ? half : 1) <= kRopeLds &&
                   (2 * tw * p.hpw + S - 1) / S <= rps_max &&
                   (int64_t)tw * p.hpw * row_bytes < 65536 &&
                   ((p.n_tok + 2 * tw - 1) / (2 * tw)) * p.n_hg >= 512)
                tw *= 2;
        // an override is clamped to what fits: LDS, 8 rows per lane, 64 tokens
        int t = tune("rope_tw", tw);
        while (t > 1 && (t > kRopeMaxTw || t * half > kRopeLds || (t * p.hpw + S - 1) / S > 8))
            t /= 2;
        p.tw = t < 1 ? 1 : t;
        const int64_t hmax = p.hq > p.hk ? p.hq : p.hk;
        if ((int64_t)p.tw * hmax * p.D * 4 >= ((int64_t)1 << 31)) vec = false;
    }
    if (vec) {
        const int S = kRopeBlock / L;
        const int rps = (p.tw * p.hpw + S - 1) / S;
        const int half = p.n_rot / 2;
        if (rps < 1 || rps > 8 || p.tw < 1 || p.tw > kRopeMaxTw || p.tw * half > kRopeLds) {
            set_error("qk_norm_rope: tile of %d tokens does not fit", p.tw);
            return false;
        }
        const int64_t blocks = ((p.n_tok + p.tw - 1) / p.tw) * p.n_hg;
        if (blocks > blocks_cap) {
            set_error("qk_norm_rope: grid too large");
            return false;
        }
        // without inv_freq: a table, or nothing rotates (n_rot < 2, no table,
        // every token valid), which the table kernel handles without reads
        const bool table = p.inv == nullptr;
        return launch("rope_vec_kernel", pick_rope(L, rps, table), dim3((unsigned)blocks),
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
    if (p.n_rot < 2) {
        // nothing rotates: the norm/copy path reads no angle source, and every
        // token counts as inside the (absent) table
        p.inv = nullptr;
        p.ctab = p.stab = nullptr;
        p.n_tab = (int64_t)1 << 62;
        p.pos = nullptr;
    }
    return aero::qk_norm_rope(p, (hipStream_t)stream) ? 1 : 0;
}

}  // extern "C"
