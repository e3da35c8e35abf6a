// Quantised GEMV / small-batch GEMM on gfx950: y[t, r] = sum_c W[r, c] * x[t, c]
// with W in GGML blocks (Q8_0, Q4_K, Q5_K, Q6_K, IQ4_XS), x and y fp32 — the
// reference's matvec / matmul (src/kernels.cpp:497-538) with its block dots
// (:78-250), which it calls between the elementwise ops of a layer.
//
// One wave (a 64-thread workgroup) owns R consecutive output rows. It walks
// the columns in chunks of U 256-value steps (U*T = 8): the chunk's quant
// blocks of each of its rows (contiguous in W) are loaded with coalesced
// 32-bit loads and staged in LDS, and the lane's x float4 of every step of the
// chunk is loaded into registers; the next chunk's loads are issued before the
// current chunk is computed, so one chunk is always in flight. In each step
// lane l takes values 4l..4l+3 (the gather's lane layout, quant_blocks.hpp)
// and for each row expands its four weights into (q[4], f, g) and accumulates
// f*sum(q*x) - g*sum(x) — the factoring of the reference's block dots, so
// sum(x) is shared by all R rows and a row costs four multiply-adds per lane
// per step. At the end each (row, token) sum is an xor-butterfly over the wave.
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

// ------------------------------------------------------------ lane groups
// A super-step is 2048 consecutive columns; lane l takes the 32-value group
// at columns 32l..32l+31 of it: group l%8 of block l/8 for the 256-value
// types, block l for Q8_0. A lane loads only its group's words (the 8 lanes
// of a block share the header through L1) and turns each quant byte into a
// float with one byte-convert (unsigned forms; signed types are offset by
// 128 or 32 and corrected through sum(x)). Its contribution is
//     f0*sum(u*x)[0:16] + f1*sum(u*x)[16:32] - g0*sum(x)[0:16] - g1*sum(x)[16:32]
// which is the reference's block dot for the group with q = u - offset.
// Loading is split from expanding (RawG::load only issues loads, RawG::expand
// is ALU), so the next super-step's words can be in flight while this one is
// computed.
struct Group {
    uint32_t u[8];         // 32 unsigned bytes, value i in byte i%4 of u[i/4]
    float f0, f1, g0, g1;
};

__device__ __forceinline__ uint32_t ld32(const uint8_t* p) {
    return *reinterpret_cast<const uint32_t*>(p);
}
__device__ __forceinline__ uint32_t ld16(const uint8_t* p) {
    return *reinterpret_cast<const uint16_t*>(p);
}
// fp16 scale -> fp32 with the hardware conversion: exact for every finite
// half (subnormals included: fp16 denormals are not flushed); only a
// signalling NaN's payload could differ from the reference's bit copy.
__device__ __forceinline__ float f16f(uint32_t h) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)(h & 0xFFFFu));
}

// The (sc, m) pair of K-quant sub-block k (0..7, per lane) from the 12-byte
// scale field (src/kernels.cpp:65-73), without branches.
__device__ __forceinline__ void kq_scale_min_sel(uint32_t s0, uint32_t s1, uint32_t s2, int k,
                                                 uint32_t& sc, uint32_t& mn) {
    const bool lo = k < 4;
    const int kk = k & 3;
    const uint32_t a = lo ? s0 : s1;                 // byte k   (k < 4) / byte k (k >= 4)
    const uint32_t b = lo ? s1 : s2;                 // byte k+4
    const uint32_t bk = (a >> (8 * kk)) & 0xFFu;     // b[k]
    const uint32_t bk4 = (b >> (8 * kk)) & 0xFFu;    // b[k+4]
    const uint32_t bkm4 = (s0 >> (8 * kk)) & 0xFFu;  // b[k-4] (k >= 4)
    sc = lo ? (bk & 63u) : ((bk4 & 15u) | ((bkm4 >> 6) << 4));
    mn = lo ? (bk4 & 63u) : ((bk4 >> 4) | ((bk >> 6) << 4));
}

// Byte e of w as a float, with the byte-convert instruction (one VALU op).
#ifndef AERO_CVT_ASM
#define AERO_CVT_ASM asm
#endif
template <int E>
__device__ __forceinline__ float cvt_ub(uint32_t w) {
#ifdef AERO_CVT_C
    return (float)((w >> (8 * E)) & 0xFFu);
#endif
    float r;
    if constexpr (E == 0) AERO_CVT_ASM("v_cvt_f32_ubyte0 %0, %1" : "=v"(r) : "v"(w));
    else if constexpr (E == 1) AERO_CVT_ASM("v_cvt_f32_ubyte1 %0, %1" : "=v"(r) : "v"(w));
    else if constexpr (E == 2) AERO_CVT_ASM("v_cvt_f32_ubyte2 %0, %1" : "=v"(r) : "v"(w));
    else AERO_CVT_ASM("v_cvt_f32_ubyte3 %0, %1" : "=v"(r) : "v"(w));
    return r;
}

// Multiply-adds of one quant word per row: al[t] += sum_e byte_e(lo) *
// xl[e][t] and ah[t] += sum_e byte_e(hi) * xh[e][t], each byte turned into a
// float with the byte-convert instruction right before its multiply-adds.
// Written as one instruction group so that every convert stays next to its
// uses (as separate operations the compiler hoists all converts of a step
// ahead of the multiply-adds and runs out of registers).
template <int T>
__device__ __forceinline__ void word_fma(uint32_t lo, uint32_t hi, const float (&xl)[4][T],
                                         const float (&xh)[4][T], float (&al)[T],
                                         float (&ah)[T]) {
    float t0, t1;
    if constexpr (T == 1) {
        asm("v_cvt_f32_ubyte0 %0, %4\n\t"
            "v_fmac_f32 %2, %0, %6\n\t"
            "v_cvt_f32_ubyte0 %1, %5\n\t"
            "v_fmac_f32 %3, %1, %10\n\t"
            "v_cvt_f32_ubyte1 %0, %4\n\t"
            "v_fmac_f32 %2, %0, %7\n\t"
            "v_cvt_f32_ubyte1 %1, %5\n\t"
            "v_fmac_f32 %3, %1, %11\n\t"
            "v_cvt_f32_ubyte2 %0, %4\n\t"
            "v_fmac_f32 %2, %0, %8\n\t"
            "v_cvt_f32_ubyte2 %1, %5\n\t"
            "v_fmac_f32 %3, %1, %12\n\t"
            "v_cvt_f32_ubyte3 %0, %4\n\t"
            "v_fmac_f32 %2, %0, %9\n\t"
            "v_cvt_f32_ubyte3 %1, %5\n\t"
            "v_fmac_f32 %3, %1, %13"
            : "=&v"(t0), "=&v"(t1), "+v"(al[0]), "+v"(ah[0])
            : "v"(lo), "v"(hi), "v"(xl[0][0]), "v"(xl[1][0]), "v"(xl[2][0]), "v"(xl[3][0]), "v"(xh[0][0]), "v"(xh[1][0]), "v"(xh[2][0]), "v"(xh[3][0]));
    } else if constexpr (T == 2) {
        asm("v_cvt_f32_ubyte0 %0, %6\n\t"
            "v_fmac_f32 %2, %0, %8\n\t"
            "v_fmac_f32 %3, %0, %9\n\t"
            "v_cvt_f32_ubyte0 %1, %7\n\t"
            "v_fmac_f32 %4, %1, %16\n\t"
            "v_fmac_f32 %5, %1, %17\n\t"
            "v_cvt_f32_ubyte1 %0, %6\n\t"
            "v_fmac_f32 %2, %0, %10\n\t"
            "v_fmac_f32 %3, %0, %11\n\t"
            "v_cvt_f32_ubyte1 %1, %7\n\t"
            "v_fmac_f32 %4, %1, %18\n\t"
            "v_fmac_f32 %5, %1, %19\n\t"
            "v_cvt_f32_ubyte2 %0, %6\n\t"
            "v_fmac_f32 %2, %0, %12\n\t"
            "v_fmac_f32 %3, %0, %13\n\t"
            "v_cvt_f32_ubyte2 %1, %7\n\t"
            "v_fmac_f32 %4, %1, %20\n\t"
            "v_fmac_f32 %5, %1, %21\n\t"
            "v_cvt_f32_ubyte3 %0, %6\n\t"
            "v_fmac_f32 %2, %0, %14\n\t"
            "v_fmac_f32 %3, %0, %15\n\t"
            "v_cvt_f32_ubyte3 %1, %7\n\t"
            "v_fmac_f32 %4, %1, %22\n\t"
            "v_fmac_f32 %5, %1, %23"
            : "=&v"(t0), "=&v"(t1), "+v"(al[0]), "+v"(al[1]), "+v"(ah[0]), "+v"(ah[1])
            : "v"(lo), "v"(hi), "v"(xl[0][0]), "v"(xl[0][1]), "v"(xl[1][0]), "v"(xl[1][1]), "v"(xl[2][0]), "v"(xl[2][1]), "v"(xl[3][0]), "v"(xl[3][1]), "v"(xh[0][0]), "v"(xh[0][1]), "v"(xh[1][0]), "v"(xh[1][1]), "v"(xh[2][0]), "v"(xh[2][1]), "v"(xh[3][0]), "v"(xh[3][1]));
    } else {
        static_assert(T == 4, "T is 1, 2 or 4");
        asm("v_cvt_f32_ubyte0 %0, %6\n\t"
            "v_fmac_f32 %2, %0, %7\n\t"
            "v_fmac_f32 %3, %0, %8\n\t"
            "v_fmac_f32 %4, %0, %9\n\t"
            "v_fmac_f32 %5, %0, %10\n\t"
            "v_cvt_f32_ubyte1 %1, %6\n\t"
            "v_fmac_f32 %2, %1, %11\n\t"
            "v_fmac_f32 %3, %1, %12\n\t"
            "v_fmac_f32 %4, %1, %13\n\t"
            "v_fmac_f32 %5, %1, %14\n\t"
            "v_cvt_f32_ubyte2 %0, %6\n\t"
            "v_fmac_f32 %2, %0, %15\n\t"
            "v_fmac_f32 %3, %0, %16\n\t"
            "v_fmac_f32 %4, %0, %17\n\t"
            "v_fmac_f32 %5, %0, %18\n\t"
            "v_cvt_f32_ubyte3 %1, %6\n\t"
            "v_fmac_f32 %2, %1, %19\n\t"
            "v_fmac_f32 %3, %1, %20\n\t"
            "v_fmac_f32 %4, %1, %21\n\t"
            "v_fmac_f32 %5, %1, %22"
            : "=&v"(t0), "=&v"(t1), "+v"(al[0]), "+v"(al[1]), "+v"(al[2]), "+v"(al[3])
            : "v"(lo), "v"(xl[0][0]), "v"(xl[0][1]), "v"(xl[0][2]), "v"(xl[0][3]), "v"(xl[1][0]), "v"(xl[1][1]), "v"(xl[1][2]), "v"(xl[1][3]), "v"(xl[2][0]), "v"(xl[2][1]), "v"(xl[2][2]), "v"(xl[2][3]), "v"(xl[3][0]), "v"(xl[3][1]), "v"(xl[3][2]), "v"(xl[3][3]));
        asm("v_cvt_f32_ubyte0 %0, %6\n\t"
            "v_fmac_f32 %2, %0, %7\n\t"
            "v_fmac_f32 %3, %0, %8\n\t"
            "v_fmac_f32 %4, %0, %9\n\t"
            "v_fmac_f32 %5, %0, %10\n\t"
            "v_cvt_f32_ubyte1 %1, %6\n\t"
            "v_fmac_f32 %2, %1, %11\n\t"
            "v_fmac_f32 %3, %1, %12\n\t"
            "v_fmac_f32 %4, %1, %13\n\t"
            "v_fmac_f32 %5, %1, %14\n\t"
            "v_cvt_f32_ubyte2 %0, %6\n\t"
            "v_fmac_f32 %2, %0, %15\n\t"
            "v_fmac_f32 %3, %0, %16\n\t"
            "v_fmac_f32 %4, %0, %17\n\t"
            "v_fmac_f32 %5, %0, %18\n\t"
            "v_cvt_f32_ubyte3 %1, %6\n\t"
            "v_fmac_f32 %2, %1, %19\n\t"
            "v_fmac_f32 %3, %1, %20\n\t"
            "v_fmac_f32 %4, %1, %21\n\t"
            "v_fmac_f32 %5, %1, %22"
            : "=&v"(t0), "=&v"(t1), "+v"(ah[0]), "+v"(ah[1]), "+v"(ah[2]), "+v"(ah[3])
            : "v"(hi), "v"(xh[0][0]), "v"(xh[0][1]), "v"(xh[0][2]), "v"(xh[0][3]), "v"(xh[1][0]), "v"(xh[1][1]), "v"(xh[1][2]), "v"(xh[1][3]), "v"(xh[2][0]), "v"(xh[2][1]), "v"(xh[2][2]), "v"(xh[2][3]), "v"(xh[3][0]), "v"(xh[3][1]), "v"(xh[3][2]), "v"(xh[3][3]));
    }
}

// 32 bytes at a 2-byte aligned address as 9 aligned words; the 9th is read
// only when the bytes straddle it (else the 8th again), so no load touches a
// word that holds none of the 32 bytes.
struct Span32 {
    uint32_t w[9];
    uint32_t sh;
    __device__ __forceinline__ void load(const uint8_t* p) {
        const uintptr_t a = reinterpret_cast<uintptr_t>(p);
        sh = (uint32_t)(a & 3u);
        const uint32_t* q = reinterpret_cast<const uint32_t*>(a - sh);
#pragma unroll
        for (int i = 0; i < 8; ++i) w[i] = q[i];
        w[8] = q[sh ? 8 : 7];
    }
    __device__ __forceinline__ uint32_t word(int m) const {
        return __builtin_amdgcn_alignbyte(w[m + 1], w[m], sh);
    }
};

template <int TYPE> struct RawG;

// Q8_0 (src/kernels.cpp:78-84): block = group (bytes 0..33: d, q[32]);
// u = q ^ 0x80 = q + 128.
template <> struct RawG<AERO_DTYPE_Q8_0> {
    uint32_t d;
    Span32 q;
    __device__ __forceinline__ void load(const uint8_t* blk, int) {
        d = ld16(blk);
        q.load(blk + 2);
    }
    __device__ __forceinline__ Group expand(int) const {
        Group g;
#pragma unroll
        for (int m = 0; m < 8; ++m) g.u[m] = q.word(m) ^ 0x80808080u;
        g.f0 = g.f1 = f16f(d);
        g.g0 = g.g1 = g.f0 * 128.0f;
        return g;
    }
};

// Q4_K (src/kernels.cpp:123-156): group k = sub-block k; nibbles of
// qs[32(k/2) ..], low for even k, high for odd.
template <> struct RawG<AERO_DTYPE_Q4_K> {
    uint32_t dd, s0, s1, s2, q[8];
    __device__ __forceinline__ void load(const uint8_t* blk, int k) {
        dd = ld32(blk); s0 = ld32(blk + 4); s1 = ld32(blk + 8); s2 = ld32(blk + 12);
        const uint8_t* qs = blk + 16 + 32 * (k >> 1);
#pragma unroll
        for (int m = 0; m < 8; ++m) q[m] = ld32(qs + 4 * m);
    }
    __device__ __forceinline__ Group expand(int k) const {
        uint32_t sc, mn;
        kq_scale_min_sel(s0, s1, s2, k, sc, mn);
        const int sh = (k & 1) ? 4 : 0;
        Group g;
#pragma unroll
        for (int m = 0; m < 8; ++m) g.u[m] = (q[m] >> sh) & 0x0F0F0F0Fu;
        g.f0 = g.f1 = f16f(dd) * (float)sc;
        g.g0 = g.g1 = f16f(dd >> 16) * (float)mn;
        return g;
    }
};

// Q5_K (src/kernels.cpp:90-121): Q4_K plus bit k of qh[i] as bit 4.
template <> struct RawG<AERO_DTYPE_Q5_K> {
    uint32_t dd, s0, s1, s2, h[8], q[8];
    __device__ __forceinline__ void load(const uint8_t* blk, int k) {
        dd = ld32(blk); s0 = ld32(blk + 4); s1 = ld32(blk + 8); s2 = ld32(blk + 12);
        const uint8_t* qs = blk + 48 + 32 * (k >> 1);
#pragma unroll
        for (int m = 0; m < 8; ++m) {
            h[m] = ld32(blk + 16 + 4 * m);
            q[m] = ld32(qs + 4 * m);
        }
    }
    __device__ __forceinline__ Group expand(int k) const {
        uint32_t sc, mn;
        kq_scale_min_sel(s0, s1, s2, k, sc, mn);
        const int sh = (k & 1) ? 4 : 0;
        Group g;
#pragma unroll
        for (int m = 0; m < 8; ++m)
            g.u[m] = ((q[m] >> sh) & 0x0F0F0F0Fu) | (((h[m] >> k) & 0x01010101u) << 4);
        g.f0 = g.f1 = f16f(dd) * (float)sc;
        g.g0 = g.g1 = f16f(dd >> 16) * (float)mn;
        return g;
    }
};

// Q6_K (src/kernels.cpp:170-200): group k = half h = k/4, quarter kq = k%4:
// low (kq < 2) or high nibbles of ql[64h + 32(kq&1) ..] and bits 2kq of
// qh[32h ..]; scale sc[8h + 2kq] for the first 16 values, sc[8h + 2kq + 1]
// for the next; u = q + 32.
template <> struct RawG<AERO_DTYPE_Q6_K> {
    Span32 ql, qh;
    uint32_t scw, d;
    __device__ __forceinline__ void load(const uint8_t* blk, int k) {
        const int h = k >> 2, kq = k & 3;
        ql.load(blk + 64 * h + 32 * (kq & 1));
        qh.load(blk + 128 + 32 * h);
        scw = ld16(blk + 192 + 8 * h + 2 * kq);
        d = ld16(blk + 208);
    }
    __device__ __forceinline__ Group expand(int k) const {
        const int kq = k & 3;
        const int sl = kq >= 2 ? 4 : 0, shh = 2 * kq;
        Group g;
#pragma unroll
        for (int m = 0; m < 8; ++m)
            g.u[m] = ((ql.word(m) >> sl) & 0x0F0F0F0Fu) | (((qh.word(m) >> shh) & 0x03030303u) << 4);
        const float df = f16f(d);
        g.f0 = df * (float)(int8_t)(scw & 0xFFu);
        g.f1 = df * (float)(int8_t)((scw >> 8) & 0xFFu);
        g.g0 = g.f0 * 32.0f;
        g.g1 = g.f1 * 32.0f;
        return g;
    }
};

// IQ4_XS (src/kernels.cpp:217-238): sub-block k; values 0..15 from the low
// nibbles of q[16k ..], 16..31 from the high nibbles; u = codebook + 128,
// looked up with byte permutes of the packed codebook.
__device__ __forceinline__ uint32_t iq4_bytes(uint32_t nib) {  // 4 nibbles, one per byte
    constexpr uint32_t C0 = 0xBFAD9881u ^ 0x80808080u, C1 = 0xF6EADDCFu ^ 0x80808080u;
    constexpr uint32_t C2 = 0x26190D01u ^ 0x80808080u, C3 = 0x71594535u ^ 0x80808080u;
    const uint32_t sel = nib & 0x07070707u;
    const uint32_t lo = __builtin_amdgcn_perm(C1, C0, sel);  // entries 0..7
    const uint32_t hi = __builtin_amdgcn_perm(C3, C2, sel);  // entries 8..15
    const uint32_t m = ((nib >> 3) & 0x01010101u) * 0xFFu;
    return (lo & ~m) | (hi & m);
}
template <> struct RawG<AERO_DTYPE_IQ4_XS> {
    uint32_t w0, sl, q[4];
    __device__ __forceinline__ void load(const uint8_t* blk, int k) {
        w0 = ld32(blk); sl = ld32(blk + 4);
#pragma unroll
        for (int m = 0; m < 4; ++m) q[m] = ld32(blk + 8 + 16 * k + 4 * m);
    }
    __device__ __forceinline__ Group expand(int k) const {
        const uint32_t shw = w0 >> 16;
        const uint32_t ls = ((byte_of(sl, k >> 1) >> (4 * (k & 1))) & 15u) |
                            (((shw >> (2 * k)) & 3u) << 4);
        Group g;
#pragma unroll
        for (int m = 0; m < 4; ++m) {
            g.u[m] = iq4_bytes(q[m] & 0x0F0F0F0Fu);
            g.u[m + 4] = iq4_bytes((q[m] >> 4) & 0x0F0F0F0Fu);
        }
        g.f0 = g.f1 = f16f(w0) * (float)((int)ls - 32);
        g.g0 = g.g1 = g.f0 * 128.0f;
        return g;
    }
};

constexpr int kGemvWaves = 4;  // waves per workgroup, sharing each x slice

// Lane-group coordinates of super-step ss (clamped into the row).
template <int TYPE>
__device__ __forceinline__ void lane_group(const GemvParams& p, int ss, int l, int& blk, int& k,
                                           bool& live) {
    using Q = QT<TYPE>;
    const int col = ss * 2048 + 32 * l;
    live = col < p.n_cols;
    const int colc = live ? col : p.n_cols - 32;
    blk = colc / Q::BV;
    k = (colc % Q::BV) / 32;
}

// x of one super-step: per token 2048 floats in 128 runs of 16; a thread
// stages XG runs (its four float4 are loaded into registers one step ahead)
// and also stores each run's sum, so lanes read sum(x) instead of adding it.
template <int T> struct XStage {
    static constexpr int XG = T >= 2 ? T / 2 : 1;  // runs per thread (128*T / 256, at least 1)
};

template <int TYPE, int R, int T>
__device__ __forceinline__ void load_step(const GemvParams& p, int ss, int l, int64_t r0,
                                          int tid, RawG<TYPE> (&w)[R],
                                          float4 (&xr)[XStage<T>::XG][4]) {
    using Q = QT<TYPE>;
    // this thread's runs of the x slice first, then the wave's weight groups
#pragma unroll
    for (int i = 0; i < XStage<T>::XG; ++i) {
        const int run = min(tid + 64 * kGemvWaves * i, 128 * T - 1);  // [0, 128*T)
        const int t = run >> 7, j = run & 127;
        const int tt = t < p.n_tok ? t : 0;
#pragma unroll
        for (int m = 0; m < 4; ++m) {
            const int c = min(ss * 2048 + 16 * j + 4 * m, p.n_cols - 4);
            xr[i][m] = *reinterpret_cast<const float4*>(p.x + tt * p.x_stride + c);
        }
    }
    int blk, k;
    bool live;
    lane_group<TYPE>(p, ss, l, blk, k, live);
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const int64_t row = min(r0 + r, p.n_rows - 1);
        w[r].load(p.w + row * p.rb + (int64_t)blk * Q::BB, k);
    }
}

template <int T>
__device__ __forceinline__ void store_x(float4 (*xs)[512], float (*xsum)[128],
                                        const float4 (&xr)[XStage<T>::XG][4], int tid) {
#pragma unroll
    for (int i = 0; i < XStage<T>::XG; ++i) {
        const int run = tid + 64 * kGemvWaves * i;
        if (run < 128 * T) {
            const int t = run >> 7, j = run & 127;
            float sum = 0.0f;
#pragma unroll
            for (int m = 0; m < 4; ++m) {
                xs[t][4 * j + m] = xr[i][m];
                sum += (xr[i][m].x + xr[i][m].y) + (xr[i][m].z + xr[i][m].w);
            }
            xsum[t][j] = sum;
        }
    }
}

template <int TYPE, int R, int T>
__device__ __forceinline__ void compute_step(const GemvParams& p, int ss, int l,
                                             const RawG<TYPE> (&w)[R], const float4 (*xs)[512],
                                             const float (*xsum)[128], float (&acc)[R][T]) {
    int blk, k;
    bool live;
    lane_group<TYPE>(p, ss, l, blk, k, live);
    Group g[R];
#pragma unroll
    for (int r = 0; r < R; ++r) g[r] = w[r].expand(k);
#pragma unroll
    for (int t = 0; t < T; ++t) {
        float4 xv[8];
#pragma unroll
        for (int m = 0; m < 8; ++m) xv[m] = xs[t][8 * l + m];
        const float2 sx = *reinterpret_cast<const float2*>(&xsum[t][2 * l]);
#pragma unroll
        for (int r = 0; r < R; ++r) {
            float q0 = 0.0f, q1 = 0.0f;
#pragma unroll
            for (int m = 0; m < 4; ++m) {
                q0 = __builtin_fmaf(cvt_ub<0>(g[r].u[m]), xv[m].x, q0);
                q0 = __builtin_fmaf(cvt_ub<1>(g[r].u[m]), xv[m].y, q0);
                q0 = __builtin_fmaf(cvt_ub<2>(g[r].u[m]), xv[m].z, q0);
                q0 = __builtin_fmaf(cvt_ub<3>(g[r].u[m]), xv[m].w, q0);
                q1 = __builtin_fmaf(cvt_ub<0>(g[r].u[m + 4]), xv[m + 4].x, q1);
                q1 = __builtin_fmaf(cvt_ub<1>(g[r].u[m + 4]), xv[m + 4].y, q1);
                q1 = __builtin_fmaf(cvt_ub<2>(g[r].u[m + 4]), xv[m + 4].z, q1);
                q1 = __builtin_fmaf(cvt_ub<3>(g[r].u[m + 4]), xv[m + 4].w, q1);
            }
            float a = acc[r][t];
            a = __builtin_fmaf(g[r].f0, q0, a);
            a = __builtin_fmaf(g[r].f1, q1, a);
            a = __builtin_fmaf(-g[r].g0, sx.x, a);
            a = __builtin_fmaf(-g[r].g1, sx.y, a);
            acc[r][t] = live ? a : acc[r][t];
        }
    }
}

// A workgroup of kGemvWaves waves covers kGemvWaves*R rows; each wave owns R
// of them. Per super-step the workgroup stages the 2048-column x slice of
// every token in LDS (double-buffered) and each wave reads its lanes' 32
// columns from there. Loads run one super-step ahead: the next slice of x
// and the next weight groups are issued (x first) before the current step is
// computed, always for super-step min(ss+1, last) so that every load is
// unconditional and the compiler's wait counts stay exact.
template <int TYPE, int R, int T>
__global__ __launch_bounds__(64 * kGemvWaves) void gemv_kernel(GemvParams p) {
    __shared__ __align__(16) float4 xs[2][T][512];
    __shared__ __align__(16) float xsum[2][T][128];

    const int tid = threadIdx.x;
    const int l = tid & 63;
    const int64_t r0 = ((int64_t)blockIdx.x * kGemvWaves + (tid >> 6)) * R;
    const int n_ss = (p.n_cols + 2047) / 2048;

    float acc[R][T];
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
        for (int t = 0; t < T; ++t) acc[r][t] = 0.0f;

    RawG<TYPE> wa[R], wb[R];
    float4 xr[XStage<T>::XG][4];
    load_step<TYPE, R, T>(p, 0, l, r0, tid, wa, xr);
    store_x<T>(xs[0], xsum[0], xr, tid);
    __syncthreads();
    for (int ss = 0; ss < n_ss; ss += 2) {
        load_step<TYPE, R, T>(p, min(ss + 1, n_ss - 1), l, r0, tid, wb, xr);
        compute_step<TYPE, R, T>(p, ss, l, wa, xs[0], xsum[0], acc);
        store_x<T>(xs[1], xsum[1], xr, tid);
        __syncthreads();
        if (ss + 1 >= n_ss) break;
        load_step<TYPE, R, T>(p, min(ss + 2, n_ss - 1), l, r0, tid, wa, xr);
        compute_step<TYPE, R, T>(p, ss + 1, l, wb, xs[1], xsum[1], acc);
        store_x<T>(xs[0], xsum[0], xr, tid);
        __syncthreads();
    }

#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
        for (int t = 0; t < T; ++t) {
            const float v = group_sum<64>(acc[r][t]);
            if (l == 0 && r0 + r < p.n_rows && t < p.n_tok) p.y[t * p.y_stride + r0 + r] = v;
        }
}

// ------------------------------------------------------- 64-column lanes
// Kernel for 16-byte aligned Q4_K rows. A step is 4096 columns (16 blocks);
// lane l owns the step's columns [64l, 64l+64): sub-block pair j = l%4 of
// block l/4, whose 32 quant bytes are two aligned 16-byte chunks (low
// nibbles: sub-block 2j, high: 2j+1) next to the block's 16-byte header
// (d, dmin, scales). Every load is a 16-byte load, a wave's loads of a row
// step cover 2304 contiguous bytes, and the scale decoding is paid once per
// 64 weights. A workgroup of kGemvWaves waves owns kGemvWaves*R rows (R per
// wave) and stages each step's x in LDS in lane order (float4 q of lane l at
// [q][l], so a wave's reads are consecutive) with its 32-column sums.
constexpr int kLaneCols = 64;
constexpr int kStepCols = 64 * kLaneCols;

template <int T>
struct XStep {
    float4 v[T][16][64];  // v[t][q][l] = x[t][64l + 4q .. 64l + 4q + 4)
    float s[T][128];      // s[t][2l + h] = sum of x[t][64l + 32h .. 64l + 32h + 32)
};

// Thread tid stages columns [16 tid, 16 tid + 16) of the step for each token.
template <int T>
struct XStepRegs {
    float4 v[T][4];
};

template <int T>
__device__ __forceinline__ void xstep_load(const GemvParams& p, int st, int tid,
                                           XStepRegs<T>& xr) {
    const int c0 = min(st * kStepCols + 16 * tid, p.n_cols - 16);
#pragma unroll
    for (int t = 0; t < T; ++t) {
        const int tt = t < p.n_tok ? t : 0;
        const float* src = p.x + tt * p.x_stride + c0;
#pragma unroll
        for (int m = 0; m < 4; ++m) xr.v[t][m] = *reinterpret_cast<const float4*>(src + 4 * m);
    }
}

// Columns past n_cols (the last step of a row that is not a whole step) hold
// x of the row's last columns: finite and never used, those lanes are not
// accumulated. The two halves of a sub-block sit in adjacent lanes, which add
// their sums.
template <int T>
__device__ __forceinline__ void xstep_store(XStep<T>& X, const XStepRegs<T>& xr, int tid) {
    const int sb = tid >> 1, half = tid & 1;
    const int l = sb >> 1, q0 = 8 * (sb & 1) + 4 * half;
#pragma unroll
    for (int t = 0; t < T; ++t) {
        float s4[4];
#pragma unroll
        for (int m = 0; m < 4; ++m) {
            X.v[t][q0 + m][l] = xr.v[t][m];
            s4[m] = (xr.v[t][m].x + xr.v[t][m].y) + (xr.v[t][m].z + xr.v[t][m].w);
        }
        float sum = (s4[0] + s4[1]) + (s4[2] + s4[3]);
        const float other = __shfl_xor(sum, 1, 64);
        sum = half ? other + sum : sum + other;  // same order in both lanes
        if (half == 0) X.s[t][sb] = sum;
    }
}

// One row's share of a step for a lane: header chunk and the two quant chunks.
struct Q4KLane {
    uint4 hd, q0, q1;
    __device__ __forceinline__ void load(const uint8_t* rowp, uint32_t off_h, uint32_t off_q) {
        hd = *reinterpret_cast<const uint4*>(rowp + off_h);
        q0 = *reinterpret_cast<const uint4*>(rowp + off_q);
        q1 = *reinterpret_cast<const uint4*>(rowp + off_q + 16);
    }
    __device__ __forceinline__ uint32_t word(int m) const {
        const uint4& c = m < 4 ? q0 : q1;
        const int k = m & 3;
        return k == 0 ? c.x : (k == 1 ? c.y : (k == 2 ? c.z : c.w));
    }
};

template <int R, int T>
__device__ __forceinline__ void q4k_step(const Q4KLane (&u)[R], const XStep<T>& X, int l,
                                         bool live, float (&acc)[R][T]) {
    float al[R][T], ah[R][T];
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
        for (int t = 0; t < T; ++t) al[r][t] = ah[r][t] = 0.0f;
    float4 xl[2][T], xh[2][T];
#pragma unroll
    for (int t = 0; t < T; ++t) {
        xl[0][t] = X.v[t][0][l];
        xh[0][t] = X.v[t][8][l];
    }
#pragma unroll
    for (int m = 0; m < 8; ++m) {
        if (m + 1 < 8) {
#pragma unroll
            for (int t = 0; t < T; ++t) {
                xl[(m + 1) & 1][t] = X.v[t][m + 1][l];
                xh[(m + 1) & 1][t] = X.v[t][9 + m][l];
            }
        }
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const uint32_t w = u[r].word(m);
            const uint32_t lo = w & 0x0F0F0F0Fu, hi = w & 0xF0F0F0F0u;  // hi bytes are 16*q
            float x4[4][T], y4[4][T];
#pragma unroll
            for (int t = 0; t < T; ++t) {
                x4[0][t] = xl[m & 1][t].x; x4[1][t] = xl[m & 1][t].y;
                x4[2][t] = xl[m & 1][t].z; x4[3][t] = xl[m & 1][t].w;
                y4[0][t] = xh[m & 1][t].x; y4[1][t] = xh[m & 1][t].y;
                y4[2][t] = xh[m & 1][t].z; y4[3][t] = xh[m & 1][t].w;
            }
            word_fma<T>(lo, hi, x4, y4, al[r], ah[r]);
        }
    }
    // (sc, m) of sub-blocks 2j, 2j+1 (src/kernels.cpp:65-73) as whole-word
    // byte operations: bytes 0..3 of SC/MN are sub-blocks 0..3 (j < 2) or
    // 4..7 (j >= 2); the pair is bytes 2(j%2), 2(j%2)+1.
    const int j = l & 3;
    const bool upper = j >= 2;
    const uint32_t mA = upper ? 0x0F0F0F0Fu : 0x3F3F3F3Fu;
    const uint32_t mB = upper ? 0x30303030u : 0u;
    const int shB = upper ? 4 : 0, sel = 16 * (j & 1);
    float2 sx[T];
#pragma unroll
    for (int t = 0; t < T; ++t) sx[t] = *reinterpret_cast<const float2*>(&X.s[t][2 * l]);
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const uint32_t dd = u[r].hd.x, s0 = u[r].hd.y, s1 = u[r].hd.z, s2 = u[r].hd.w;
        const uint32_t sc = (((upper ? s2 : s0) & mA) | ((s0 >> 2) & mB)) >> sel;
        const uint32_t mn = ((((upper ? s2 : s1) >> shB) & mA) | ((s1 >> 2) & mB)) >> sel;
        const float d = f16f(dd), dm = f16f(dd >> 16);
        const float f_lo = d * cvt_ub<0>(sc), f_hi = (d * 0.0625f) * cvt_ub<1>(sc);
        const float g_lo = dm * cvt_ub<0>(mn), g_hi = dm * cvt_ub<1>(mn);
#pragma unroll
        for (int t = 0; t < T; ++t) {
            float a = acc[r][t];
            a = __builtin_fmaf(f_lo, al[r][t], a);
            a = __builtin_fmaf(f_hi, ah[r][t], a);
            a = __builtin_fmaf(-g_lo, sx[t].x, a);
            a = __builtin_fmaf(-g_hi, sx[t].y, a);
            acc[r][t] = live ? a : acc[r][t];
        }
    }
}

// Offsets of lane l's chunks in step st (its block clamped into the row, so
// every load is in bounds; lanes past the row's end are not accumulated).
__device__ __forceinline__ void q4k_offsets(int st, int l, int n_blk, uint32_t& off_h,
                                            uint32_t& off_q, bool& live) {
    const int kb = st * 16 + (l >> 2);
    live = kb < n_blk;
    const uint32_t kc = (uint32_t)min(kb, n_blk - 1);
    off_h = kc * 144u;
    off_q = off_h + 16u + 32u * (uint32_t)(l & 3);
}


// Stage x: 16-column run u (token t, step st, run j of the step) is loaded by
// thread u % threads; runs past n_cols are stored as zeros. The two halves of
// a sub-block sit in adjacent lanes, which add their sums.
template <int R>
__device__ __forceinline__ void q4k_load(const uint8_t* const (&rowp)[R], int st, int l,
                                         int n_blk, Q4KLane (&u)[R], bool& live) {
    uint32_t oh, oq;
    q4k_offsets(st, l, n_blk, oh, oq, live);
#pragma unroll
    for (int r = 0; r < R; ++r) u[r].load(rowp[r], oh, oq);
}

// Each step's x is loaded before its weight chunks: loads complete in order,
// so the wait for x before the barrier does not also wait for the weights.
// PIPE (rows of more than one step): the next step's x and chunks are loaded
// before the current step is computed, for step min(st+1, last) so that every
// load is unconditional.
template <int R, int T, bool PIPE>
__global__ __launch_bounds__(64 * kGemvWaves) void gemv_q4k_kernel(GemvParams p) {
    __shared__ __align__(16) XStep<T> xs[PIPE ? 2 : 1];

    const int tid = threadIdx.x;
    const int l = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int64_t r0 = ((int64_t)blockIdx.x * kGemvWaves + wave) * R;
    const int n_blk = p.n_cols / 256;
    const int n_st = (n_blk + 15) / 16;

    const uint8_t* rowp[R];
#pragma unroll
    for (int r = 0; r < R; ++r) rowp[r] = p.w + min(r0 + r, p.n_rows - 1) * p.rb;

    float acc[R][T];
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
        for (int t = 0; t < T; ++t) acc[r][t] = 0.0f;

    XStepRegs<T> xr;
    Q4KLane ua[R];
    bool live_a;
    xstep_load<T>(p, 0, tid, xr);
    q4k_load<R>(rowp, 0, l, n_blk, ua, live_a);
    xstep_store<T>(xs[0], xr, tid);
    __syncthreads();

    if constexpr (!PIPE) {
        q4k_step<R, T>(ua, xs[0], l, live_a, acc);  // rows of one step
    } else {
        Q4KLane ub[R];
        bool live_b;
        for (int st = 0; st < n_st; st += 2) {
            const int s1 = min(st + 1, n_st - 1);
            xstep_load<T>(p, s1, tid, xr);
            q4k_load<R>(rowp, s1, l, n_blk, ub, live_b);
            live_b = live_b && st + 1 < n_st;
            __builtin_amdgcn_sched_barrier(0);
            q4k_step<R, T>(ua, xs[0], l, live_a, acc);
            xstep_store<T>(xs[1], xr, tid);
            __syncthreads();
            if (st + 1 >= n_st) break;
            const int s2 = min(st + 2, n_st - 1);
            xstep_load<T>(p, s2, tid, xr);
            q4k_load<R>(rowp, s2, l, n_blk, ua, live_a);
            live_a = live_a && st + 2 < n_st;
            __builtin_amdgcn_sched_barrier(0);
            q4k_step<R, T>(ub, xs[1], l, live_b, acc);
            xstep_store<T>(xs[0], xr, tid);
            __syncthreads();
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

template <int R, bool PIPE>
GemvKernel pick_q4k_t(int T) {
    switch (T) {
    case 1: return gemv_q4k_kernel<R, 1, PIPE>;
    case 2: return gemv_q4k_kernel<R, 2, PIPE>;
    case 4: return gemv_q4k_kernel<R, 4, PIPE>;
    default: return nullptr;
    }
}

template <bool PIPE>
GemvKernel pick_q4k(int R, int T) {
    switch (R) {
    case 1: return pick_q4k_t<1, PIPE>(T);
    case 2: return pick_q4k_t<2, PIPE>(T);
    case 4: return pick_q4k_t<4, PIPE>(T);
    default: return nullptr;
    }
}

template <int TYPE, int R>
GemvKernel pick_t(int T) {
    switch (T) {
    case 1: return gemv_kernel<TYPE, R, 1>;
    case 2: return gemv_kernel<TYPE, R, 2>;
    case 4: return gemv_kernel<TYPE, R, 4>;
    default: return nullptr;
    }
}

template <int TYPE>
GemvKernel pick_r(int R, int T) {
    switch (R) {
    case 1: return pick_t<TYPE, 1>(T);
    case 2: return pick_t<TYPE, 2>(T);
    case 4: return pick_t<TYPE, 4>(T);
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

// y[t, r] for t < n_tok: tokens are taken in groups of up to 4 per launch
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
    if (dtype == AERO_DTYPE_Q4_K && aligned16(w) && tune("gemv_lanes64", 1)) {
        const bool pipe = n_cols > kStepCols;
        for (int64_t t0 = 0; t0 < n_tok; t0 += 4) {
            const int nt = (int)std::min<int64_t>(4, n_tok - t0);
            const int T = nt == 1 ? 1 : (nt == 2 ? 2 : 4);
            // rows per wave (measured on MI355X): 2 while that leaves >= 256
            // workgroups, else 1; four tokens share the weight decoding over
            // 4 rows when that leaves >= 512 workgroups (>= 256 for rows of
            // several steps)
            auto wgs_of = [&](int r) { return (n_rows + r * kGemvWaves - 1) / (r * kGemvWaves); };
            int R = wgs_of(2) >= 256 ? 2 : 1;
            if (T == 4 && (wgs_of(4) >= 512 || (pipe && wgs_of(4) >= 256))) R = 4;
            R = tune("gemv_r", R);
            const int64_t wgs =
                (n_rows + (int64_t)R * kGemvWaves - 1) / ((int64_t)R * kGemvWaves);
            GemvKernel k = pipe ? pick_q4k<true>(R, T) : pick_q4k<false>(R, T);
            if (k == nullptr || wgs > 0x7fffffff) {
                set_error("matvec: no Q4_K kernel for rows/wave %d", R);
                return false;
            }
            GemvParams p{w, x + t0 * n_cols, y + t0 * n_rows, n_rows, (int)n_cols, rb, nt,
                         n_cols, n_rows};
            if (!launch("gemv_q4k_kernel", k, dim3((unsigned)wgs), dim3(64 * kGemvWaves), 0, s,
                        p))
                return false;
        }
        return true;
    }
    // rows per wave: up to 4 (2 for the 2-byte aligned Q8_0 / Q6_K blocks, whose
    // words take two loads each) while the grid keeps >= 512 workgroups
    int R = (dtype == AERO_DTYPE_Q8_0 || dtype == AERO_DTYPE_Q6_K) ? 2 : 4;
    while (R > 1 && (n_rows + R * kGemvWaves - 1) / (R * kGemvWaves) < 512) R /= 2;
    R = tune("gemv_r", R);
    const int64_t wgs = (n_rows + (int64_t)R * kGemvWaves - 1) / ((int64_t)R * kGemvWaves);
    if (wgs > 0x7fffffff) {
        set_error("matvec: grid too large");
        return false;
    }
    for (int64_t t0 = 0; t0 < n_tok; t0 += 4) {
        const int nt = (int)std::min<int64_t>(4, n_tok - t0);
        const int T = nt == 1 ? 1 : (nt == 2 ? 2 : 4);
        GemvKernel k = pick_gemv(dtype, R, T);
        if (k == nullptr) {
            set_error("matvec: no kernel for rows/wave %d", R);
            return false;
        }
        GemvParams p{w, x + t0 * n_cols, y + t0 * n_rows, n_rows, (int)n_cols, rb, nt,
                     n_cols, n_rows};
        if (!launch("gemv_kernel", k, dim3((unsigned)wgs), dim3(64 * kGemvWaves), 0, s, p))
            return false;
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
