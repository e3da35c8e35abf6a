// GGML quant block formats on gfx950: the raw words one lane needs for four
// consecutive values of a 256-value step, and their decode. Shared by the
// embedding gather / dequant (quant.hip) and the quantised GEMV (gemv.hip).
//
// In each 256-value step, lane l of a wave handles values 4l..4l+3: for the
// 256-value K-quants and IQ4_XS those of the step's one block, for Q8_0 values
// 4(l%8).. of the step's block l/8. load_raw reads a lane's words from a block
// (in LDS or global memory): Q8_0 and Q6_K blocks may start at even byte
// offsets and are read in 16-bit pieces; Q4_K, Q5_K and IQ4_XS blocks start at
// multiples of 4 in a 4-byte aligned buffer.
//
// Arithmetic is the reference's, operation by operation (callers compile with
// contraction off), so dequantised values are bit-identical: Q8_0 d*q
// (src/kernels.cpp:364-373); Q4_K (d*sc)*q - (dmin*m) with the 6-bit unpacking
// of src/kernels.cpp:65-73,337-363; Q5_K the same with a fifth bit
// (:374-404); Q6_K (d*sc)*(q-32) (:427-458); IQ4_XS dl*codebook[q]
// (:405-425). fp16 scales are decoded exactly (subnormals included).
#pragma once
#include "common.hpp"
#include "aero_hip.h"

#pragma clang fp contract(off)

namespace aero {
namespace {

__device__ __forceinline__ uint32_t ld_u16(const uint8_t* p) {
    return *reinterpret_cast<const uint16_t*>(p);
}
// 4 bytes at a 2-byte aligned address, little endian
__device__ __forceinline__ uint32_t ld_u32_a2(const uint8_t* p) {
    return ld_u16(p) | (ld_u16(p + 2) << 16);
}
__device__ __forceinline__ uint32_t ld_u32(const uint8_t* p) {
    return *reinterpret_cast<const uint32_t*>(p);
}
__device__ __forceinline__ uint32_t byte_of(uint32_t w, int k) {
    return (w >> (8 * k)) & 0xFFu;
}

// Raw words one lane needs for its four values of one unit.
struct RawQ8 { uint32_t d, q0, q1; };        // fp16 d, quant bytes as 2 x 16 bit
struct RawQ4 { uint32_t dd, s0, s1, s2, q; }; // d|dmin, 12 scale bytes, 4 quant bytes
struct RawQ6 { uint32_t ql0, ql1, qh0, qh1, sc, d; };
struct RawQ5 { uint32_t dd, s0, s1, s2, h, q; };  // as Q4_K plus 4 qh bytes
struct RawIQ4 { uint32_t dsh, sl, q; };           // d|scales_h, scales_l, 4 quant bytes

// Q8_0 lanes work per block: lane l covers values 4(l%8).. of its block.
__device__ __forceinline__ void load_raw(const uint8_t* blk, int l, RawQ8& r) {
    const int k = l & 7;
    r.d = ld_u16(blk);
    r.q0 = ld_u16(blk + 2 + 4 * k);
    r.q1 = ld_u16(blk + 4 + 4 * k);
}
__device__ __forceinline__ void load_raw(const uint8_t* blk, int l, RawQ4& r) {
    const int j = l >> 4, i0 = (l & 7) * 4;
    r.dd = ld_u32(blk);
    r.s0 = ld_u32(blk + 4);
    r.s1 = ld_u32(blk + 8);
    r.s2 = ld_u32(blk + 12);
    r.q = ld_u32(blk + 16 + 32 * j + i0);
}
__device__ __forceinline__ void load_raw(const uint8_t* blk, int l, RawQ6& r) {
    const int h = l >> 5, k = (l >> 3) & 3, lq = (l & 7) * 4;
    const uint8_t* ql = blk + 64 * h + lq + 32 * (k & 1);
    const uint8_t* qh = blk + 128 + 32 * h + lq;
    r.ql0 = ld_u16(ql);
    r.ql1 = ld_u16(ql + 2);
    r.qh0 = ld_u16(qh);
    r.qh1 = ld_u16(qh + 2);
    r.sc = blk[192 + 8 * h + (lq >> 4) + 2 * k];
    r.d = ld_u16(blk + 208);
}

__device__ __forceinline__ void load_raw(const uint8_t* blk, int l, RawQ5& r) {
    const int j = l >> 4, i0 = (l & 7) * 4;
    r.dd = ld_u32(blk);
    r.s0 = ld_u32(blk + 4);
    r.s1 = ld_u32(blk + 8);
    r.s2 = ld_u32(blk + 12);
    r.h = ld_u32(blk + 16 + i0);
    r.q = ld_u32(blk + 48 + 32 * j + i0);
}
__device__ __forceinline__ void load_raw(const uint8_t* blk, int l, RawIQ4& r) {
    const int ib = l >> 3, jj = (l & 7) * 4;
    r.dsh = ld_u32(blk);
    r.sl = ld_u32(blk + 4);
    r.q = ld_u32(blk + 8 + 16 * ib + (jj & 15));
}

// Q8_0, src/kernels.cpp:364-373: y = d*q.
__device__ __forceinline__ float4 decode(const RawQ8& r, int) {
    const float d = half_bits_to_float(r.d);
    const uint32_t q = r.q0 | (r.q1 << 16);
    float4 v;
    v.x = d * (float)(int8_t)byte_of(q, 0);
    v.y = d * (float)(int8_t)byte_of(q, 1);
    v.z = d * (float)(int8_t)byte_of(q, 2);
    v.w = d * (float)(int8_t)byte_of(q, 3);
    return v;
}

// Q4_K, src/kernels.cpp:65-73,337-363: group j = l/16 covers values
// 64j..64j+63, low nibbles (sub-block 2j) then high nibbles (2j+1);
// y = (d*sc)*q - (dmin*m).
__device__ __forceinline__ float4 decode(const RawQ4& r, int l) {
    const float d = half_bits_to_float(r.dd & 0xFFFFu);
    const float dmin = half_bits_to_float(r.dd >> 16);
    const int j = l >> 4;
    const int hi = (l >> 3) & 1;
    const int k = 2 * j + hi;
    // byte idx of the 12-byte scale field, selected from registers
    const uint32_t s0 = r.s0, s1 = r.s1, s2 = r.s2;
    auto sb = [s0, s1, s2](int idx) {
        const uint32_t w = idx < 4 ? s0 : (idx < 8 ? s1 : s2);
        return byte_of(w, idx & 3);
    };
    uint32_t sc, mn;
    if (k < 4) {
        sc = sb(k) & 63u;
        mn = sb(k + 4) & 63u;
    } else {
        sc = (sb(k + 4) & 15u) | ((sb(k - 4) >> 6) << 4);
        mn = (sb(k + 4) >> 4) | ((sb(k) >> 6) << 4);
    }
    const float f = d * (float)sc;
    const float g = dmin * (float)mn;
    const int sh = hi ? 4 : 0;
    float4 v;
    v.x = f * (float)((byte_of(r.q, 0) >> sh) & 15u) - g;
    v.y = f * (float)((byte_of(r.q, 1) >> sh) & 15u) - g;
    v.z = f * (float)((byte_of(r.q, 2) >> sh) & 15u) - g;
    v.w = f * (float)((byte_of(r.q, 3) >> sh) & 15u) - g;
    return v;
}

// Q6_K, src/kernels.cpp:427-458: half h = l/32, quarter k = (l/8)%4 (values
// 128h + 32k + lq .. +3, lq = 4*(l%8)); y = (d*sc)*(q-32).
__device__ __forceinline__ float4 decode(const RawQ6& r, int l) {
    const int k = (l >> 3) & 3;
    const uint32_t ql = r.ql0 | (r.ql1 << 16);
    const uint32_t qh = r.qh0 | (r.qh1 << 16);
    const float f = half_bits_to_float(r.d) * (float)(int8_t)r.sc;
    const int shl = (k >= 2) ? 4 : 0;
    const int shh = 2 * k;
    float qv[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        const int q = (int)(((byte_of(ql, e) >> shl) & 15u) |
                            (((byte_of(qh, e) >> shh) & 3u) << 4));
        qv[e] = f * (float)(q - 32);
    }
    return make_float4(qv[0], qv[1], qv[2], qv[3]);
}

// The (sc, m) pair of sub-block k from the three words of the 12-byte K-quant
// scale field (src/kernels.cpp:65-73).
__device__ __forceinline__ void kq_scale_min(uint32_t s0, uint32_t s1, uint32_t s2, int k,
                                             uint32_t& sc, uint32_t& mn) {
    auto sb = [s0, s1, s2](int idx) {
        const uint32_t w = idx < 4 ? s0 : (idx < 8 ? s1 : s2);
        return byte_of(w, idx & 3);
    };
    if (k < 4) {
        sc = sb(k) & 63u;
        mn = sb(k + 4) & 63u;
    } else {
        sc = (sb(k + 4) & 15u) | ((sb(k - 4) >> 6) << 4);
        mn = (sb(k + 4) >> 4) | ((sb(k) >> 6) << 4);
    }
}

// Q5_K, src/kernels.cpp:374-404: Q4_K's layout plus qh[32] at byte 16 (quants
// at 48); value i of group j adds bit 2j (low nibbles) or 2j+1 (high) of
// qh[i] as bit 4; y = (d*sc)*q - (dmin*m).
__device__ __forceinline__ float4 decode(const RawQ5& r, int l) {
    const float d = half_bits_to_float(r.dd & 0xFFFFu);
    const float dmin = half_bits_to_float(r.dd >> 16);
    const int j = l >> 4;
    const int hi = (l >> 3) & 1;
    const int k = 2 * j + hi;
    uint32_t sc, mn;
    kq_scale_min(r.s0, r.s1, r.s2, k, sc, mn);
    const float f = d * (float)sc;
    const float g = dmin * (float)mn;
    const int sh = hi ? 4 : 0;
    float qv[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        const uint32_t q = ((byte_of(r.q, e) >> sh) & 15u) | (((byte_of(r.h, e) >> k) & 1u) << 4);
        qv[e] = f * (float)q - g;
    }
    return make_float4(qv[0], qv[1], qv[2], qv[3]);
}

// IQ4_XS codebook (src/kernels.cpp:212-215; the GGML IQ4_NL levels, a file
// format constant), as four words of packed int8 so a lookup stays in
// registers.
__device__ __forceinline__ float iq4_level(uint32_t nib) {
    constexpr uint32_t W0 = 0xBFAD9881u;  // -127, -104,  -83,  -65
    constexpr uint32_t W1 = 0xF6EADDCFu;  //  -49,  -35,  -22,  -10
    constexpr uint32_t W2 = 0x26190D01u;  //    1,   13,   25,   38
    constexpr uint32_t W3 = 0x71594535u;  //   53,   69,   89,  113
    const uint32_t w = nib < 8 ? (nib < 4 ? W0 : W1) : (nib < 12 ? W2 : W3);
    return (float)(int8_t)((w >> (8 * (nib & 3))) & 0xFFu);
}

// IQ4_XS, src/kernels.cpp:405-425: sub-block ib = l/8 of 32 values,
// dl = d*(ls-32) with ls = 4 low bits from scales_l and 2 high bits from
// scales_h; lanes 0..3 of a sub-block take low nibbles of qs[16ib..], lanes
// 4..7 the high nibbles; y = dl*codebook[q].
__device__ __forceinline__ float4 decode(const RawIQ4& r, int l) {
    const int ib = l >> 3;
    const int hi = (l & 7) >= 4;
    const float d = half_bits_to_float(r.dsh & 0xFFFFu);
    const uint32_t sh = r.dsh >> 16;
    const uint32_t ls = ((byte_of(r.sl, ib >> 1) >> (4 * (ib & 1))) & 15u) |
                        (((sh >> (2 * ib)) & 3u) << 4);
    const float dl = d * (float)((int)ls - 32);
    float qv[4];
#pragma unroll
    for (int e = 0; e < 4; ++e)
        qv[e] = dl * iq4_level((byte_of(r.q, e) >> (hi ? 4 : 0)) & 15u);
    return make_float4(qv[0], qv[1], qv[2], qv[3]);
}

// 16- and 8-byte loads, and word k of an array of 16-byte chunks.
__device__ __forceinline__ uint4 ld128(const uint8_t* p) {
    return *reinterpret_cast<const uint4*>(p);
}
__device__ __forceinline__ uint2 ld64(const uint8_t* p) {
    return *reinterpret_cast<const uint2*>(p);
}
template <int N>
__device__ __forceinline__ uint32_t wd(const uint4 (&c)[N], int k) {
    const uint4& v = c[k >> 2];
    return (k & 3) == 0 ? v.x : ((k & 3) == 1 ? v.y : ((k & 3) == 2 ? v.z : v.w));
}
// Words of the 16-byte chunks c starting at byte `ph` (even, 0..14, the same
// for all outputs), out[i] = bytes ph+4i .. ph+4i+3: shifts by 8 and by 4
// bytes (byte permutes of two words) and by ph & 3 (a byte align). Permutes
// rather than selects: the compiler turns a select between two array
// elements into a load from a selected address, which sends the array to
// scratch memory.
template <int N, int C>
__device__ __forceinline__ void shifted_words(const uint4 (&c)[C], uint32_t ph,
                                              uint32_t (&out)[N]) {
    // words ph/4 .. ph/4 + N (the last only with a byte shift) must lie in c;
    // reads past c are clamped (and unused when ph & 3 == 0)
    static_assert(4 * C >= N + 3, "window too small");
    const uint32_t sel8 = (ph & 8u) ? 0x07060504u : 0x03020100u;
    const uint32_t sel4 = (ph & 4u) ? 0x07060504u : 0x03020100u;
    uint32_t a[N + 2], b[N + 1];
#pragma unroll
    for (int i = 0; i < N + 2; ++i)
        a[i] = __builtin_amdgcn_perm(wd(c, min(i + 2, 4 * C - 1)), wd(c, i), sel8);
#pragma unroll
    for (int i = 0; i < N + 1; ++i) b[i] = __builtin_amdgcn_perm(a[i + 1], a[i], sel4);
#pragma unroll
    for (int i = 0; i < N; ++i) out[i] = __builtin_amdgcn_alignbyte(b[i + 1], b[i], ph & 3u);
}

template <int TYPE> struct QT;
template <> struct QT<AERO_DTYPE_Q8_0> { static constexpr int BV = 32, BB = 34; using Raw = RawQ8; };
template <> struct QT<AERO_DTYPE_Q4_K> { static constexpr int BV = 256, BB = 144; using Raw = RawQ4; };
template <> struct QT<AERO_DTYPE_Q6_K> { static constexpr int BV = 256, BB = 210; using Raw = RawQ6; };
template <> struct QT<AERO_DTYPE_Q5_K> { static constexpr int BV = 256, BB = 176; using Raw = RawQ5; };
template <> struct QT<AERO_DTYPE_IQ4_XS> { static constexpr int BV = 256, BB = 136; using Raw = RawIQ4; };

// A lane's four weights of one step for a dot product, factored the way the
// reference's block dots are (src/kernels.cpp:78-250): the block's weights are
// f*q[e] - g, so sum(w*x) = f*sum(q*x) - g*sum(x). g is zero for the types
// without a min (HAS_MIN false).
struct Quad {
    float q[4];
    float f, g;
};

// Q8_0 (src/kernels.cpp:78-84): d * sum(q*x).
__device__ __forceinline__ Quad expand(const RawQ8& r, int) {
    const uint32_t q = r.q0 | (r.q1 << 16);
    Quad o;
#pragma unroll
    for (int e = 0; e < 4; ++e) o.q[e] = (float)(int8_t)byte_of(q, e);
    o.f = half_bits_to_float(r.d);
    o.g = 0.0f;
    return o;
}

// Q4_K (src/kernels.cpp:123-156): (d*sc)*sum(q*x) - (dmin*m)*sum(x) per
// 32-value half.
__device__ __forceinline__ Quad expand(const RawQ4& r, int l) {
    const int j = l >> 4, hi = (l >> 3) & 1;
    uint32_t sc, mn;
    kq_scale_min(r.s0, r.s1, r.s2, 2 * j + hi, sc, mn);
    Quad o;
#pragma unroll
    for (int e = 0; e < 4; ++e) o.q[e] = (float)((byte_of(r.q, e) >> (hi ? 4 : 0)) & 15u);
    o.f = half_bits_to_float(r.dd & 0xFFFFu) * (float)sc;
    o.g = half_bits_to_float(r.dd >> 16) * (float)mn;
    return o;
}

// Q5_K (src/kernels.cpp:90-121): Q4_K with the fifth bit from qh.
__device__ __forceinline__ Quad expand(const RawQ5& r, int l) {
    const int j = l >> 4, hi = (l >> 3) & 1, k = 2 * j + hi;
    uint32_t sc, mn;
    kq_scale_min(r.s0, r.s1, r.s2, k, sc, mn);
    Quad o;
#pragma unroll
    for (int e = 0; e < 4; ++e)
        o.q[e] = (float)(((byte_of(r.q, e) >> (hi ? 4 : 0)) & 15u) |
                         (((byte_of(r.h, e) >> k) & 1u) << 4));
    o.f = half_bits_to_float(r.dd & 0xFFFFu) * (float)sc;
    o.g = half_bits_to_float(r.dd >> 16) * (float)mn;
    return o;
}

// Q6_K (src/kernels.cpp:170-200): (d*sc)*sum((q-32)*x); a lane's four values
// share one 16-value scale.
__device__ __forceinline__ Quad expand(const RawQ6& r, int l) {
    const int k = (l >> 3) & 3;
    const uint32_t ql = r.ql0 | (r.ql1 << 16);
    const uint32_t qh = r.qh0 | (r.qh1 << 16);
    const int shl = (k >= 2) ? 4 : 0, shh = 2 * k;
    Quad o;
#pragma unroll
    for (int e = 0; e < 4; ++e)
        o.q[e] = (float)((int)(((byte_of(ql, e) >> shl) & 15u) |
                               (((byte_of(qh, e) >> shh) & 3u) << 4)) - 32);
    o.f = half_bits_to_float(r.d) * (float)(int8_t)r.sc;
    o.g = 0.0f;
    return o;
}

// IQ4_XS (src/kernels.cpp:217-238): dl * sum(codebook[q]*x).
__device__ __forceinline__ Quad expand(const RawIQ4& r, int l) {
    const int ib = l >> 3, hi = (l & 7) >= 4;
    const uint32_t sh = r.dsh >> 16;
    const uint32_t ls = ((byte_of(r.sl, ib >> 1) >> (4 * (ib & 1))) & 15u) |
                        (((sh >> (2 * ib)) & 3u) << 4);
    Quad o;
#pragma unroll
    for (int e = 0; e < 4; ++e) o.q[e] = iq4_level((byte_of(r.q, e) >> (hi ? 4 : 0)) & 15u);
    o.f = half_bits_to_float(r.dsh & 0xFFFFu) * (float)((int)ls - 32);
    o.g = 0.0f;
    return o;
}

template <int TYPE> struct HasMin { static constexpr bool value = false; };
template <> struct HasMin<AERO_DTYPE_Q4_K> { static constexpr bool value = true; };
template <> struct HasMin<AERO_DTYPE_Q5_K> { static constexpr bool value = true; };

}  // namespace
}  // namespace aero
