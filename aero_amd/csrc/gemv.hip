// Quantised GEMV / small-batch GEMM on gfx950: y[t, r] = sum_c W[r, c] * x[t, c]
// with W in GGML blocks (Q8_0, Q4_K, Q5_K, Q6_K, IQ4_XS), x and y fp32 — the
// reference's matvec / matmul (src/kernels.cpp:497-538) with its block dots
// (:78-250), which it calls between the elementwise ops of a layer.
//
// Two kernels, both workgroups of kGemvWaves waves that share x through LDS:
//   gemv64_kernel (rows of a multiple of 16 bytes, Q8_0 rows also of 8, W
//     16-byte aligned: every common shape): lane l of a 4096-column step
//     owns columns 64l..64l+63 and loads only its bytes of each row with
//     16-byte loads;
//   gemv_kernel (any row length, W 4-byte aligned): lane l of a 2048-column
//     step owns a 32-value group, loaded as 4-byte words.
// Each wave owns R rows; the row sums are xor-butterflies over the wave.
//
// HBM bytes per launch: the weight blocks once (n_rows * n_cols/bv * bb) plus
// x and y; x is re-read from L2 by every workgroup. Results differ from the
// reference's serial sums only in summation order.
#include "quant_blocks.hpp"
#include "act_ops.hpp"

#pragma clang fp contract(off)

namespace aero {

int64_t dtype_block_bytes(int t);
bool gemm_dev(int dtype, const uint8_t* w, const float* x, float* y, int64_t n_rows,
              int64_t n_cols, int64_t rb, int64_t n_tok, hipStream_t s);
int64_t split_gemm_workspace(int dtype, int64_t n_cols, int64_t n_tok);
bool split_tokens_ok(int64_t n_tok, int64_t n_rows, int64_t n_cols);
bool split_gemm_dev(int dtype, const uint8_t* w, const float* x, float* y, int64_t n_rows,
                    int64_t n_cols, int64_t rb, int64_t n_tok, void* ws, int64_t ws_bytes,
                    hipStream_t s, bool* ran);
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
    int sub;           // gemv64_kernel: rows of <= 2048 (1) / 1024 (2) columns, a row a 64 >> sub lanes
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
// Kernels for rows whose byte length is a multiple of 16 (16-byte aligned
// W). A step is 4096 columns (16 blocks of 256, 128 of 32); lane l owns the
// step's columns [64l, 64l+64) and loads only its own bytes of each row, in
// 16-byte (8-byte for IQ4_XS) loads:
//   Q4_K / Q5_K: sub-block pair j = l%4 of block l/4: the pair's 32 quant
//       bytes (low nibbles sub-block 2j, high 2j+1), the 16-byte header and
//       (Q5_K) the 32 high-bit bytes;
//   IQ4_XS: the 32 bytes of sub-blocks 2j, 2j+1 of block l/4 and its header;
//   Q8_0: blocks 2l, 2l+1 (68 bytes at a 4-byte aligned offset, taken from
//       the 80 aligned bytes around them);
//   Q6_K: ql bytes [64h+32a, +32) and qh bytes [32h, +32) of block l/4
//       (h = j/2, a = j%2: quarters a and a+2 of half h, whose columns start
//       in lanes l-a and l-a+1), from the 48 aligned bytes around each.
// Quant values become unsigned bytes (signed types offset by 128 or 32,
// corrected through sums of x), so each converts to a float with one
// instruction; a row's share of a block dot is
//     sum_g scale_g * (sum(u * x)_g - offset * sum(x)_g)
// the factoring of the reference's block dots (src/kernels.cpp:78-250).
// A workgroup of kGemvWaves waves owns kGemvWaves*R rows (R per wave) and
// stages each step's x in LDS in lane order (float4 q of lane l at [q][l], so
// a wave's reads are consecutive) with its 32- and 16-column sums.
constexpr int kLaneCols = 64;
constexpr int kStepCols = 64 * kLaneCols;

template <int T>
struct XStep {
    float4 v[T][16][64];  // v[t][q][l] = x[t][64l + 4q .. 64l + 4q + 4)
    float s[T][128];      // s[t][2l + h] = sum of x[t][64l + 32h .. 64l + 32h + 32)
    float s16[T][256];    // s16[t][i] = sum of x[t][16i .. 16i + 16)
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
// accumulated. The two halves of a 32-column run sit in adjacent lanes, which
// add their sums.
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
        X.s16[t][tid] = sum;
        const float other = __shfl_xor(sum, 1, 64);
        sum = half ? other + sum : sum + other;  // same order in both lanes
        if (half == 0) X.s[t][sb] = sum;
    }
}

__device__ __forceinline__ uint32_t rotr(uint32_t v, uint32_t s) {
    return __builtin_amdgcn_alignbit(v, v, s);
}

// x operands of word m: float4 lanes/rows chosen by the lane type.
template <int T>
__device__ __forceinline__ void x_words(const XStep<T>& X, int q_lo, int lane_lo, int q_hi,
                                        int lane_hi, float (&xl)[4][T], float (&xh)[4][T]) {
#pragma unroll
    for (int t = 0; t < T; ++t) {
        const float4 a = X.v[t][q_lo][lane_lo], b = X.v[t][q_hi][lane_hi];
        xl[0][t] = a.x; xl[1][t] = a.y; xl[2][t] = a.z; xl[3][t] = a.w;
        xh[0][t] = b.x; xh[1][t] = b.y; xh[2][t] = b.z; xh[3][t] = b.w;
    }
}

// The word loop shared by the lane types: for m = 0..7 and each row, the lo
// and hi unsigned-byte words wf(r, m) are multiplied with the x float4 rows
// q_lo(m) (lane lane_lo) and q_hi(m) (lane lane_hi) and added to accumulator
// group g(m). The next word's x is read before the current one is used.
template <int R, int T, int G, typename WF, typename QF, typename GF>
__device__ __forceinline__ void word_loop(const XStep<T>& X, int lane_lo, int lane_hi, WF wf,
                                          QF qf, GF gf, float (&al)[R][G][T],
                                          float (&ah)[R][G][T]) {
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
        for (int g = 0; g < G; ++g)
#pragma unroll
            for (int t = 0; t < T; ++t) al[r][g][t] = ah[r][g][t] = 0.0f;
    float xl[2][4][T], xh[2][4][T];
    {
        int ql, qh;
        qf(0, ql, qh);
        x_words<T>(X, ql, lane_lo, qh, lane_hi, xl[0], xh[0]);
    }
#pragma unroll
    for (int m = 0; m < 8; ++m) {
        if (m + 1 < 8) {
            int ql, qh;
            qf(m + 1, ql, qh);
            x_words<T>(X, ql, lane_lo, qh, lane_hi, xl[(m + 1) & 1], xh[(m + 1) & 1]);
        }
        const int g = gf(m);
#pragma unroll
        for (int r = 0; r < R; ++r) {
            uint32_t lo, hi;
            wf(r, m, lo, hi);
            word_fma<T>(lo, hi, xl[m & 1], xh[m & 1], al[r][g], ah[r][g]);
        }
    }
}

// Scale and minimum of K-quant sub-blocks 2j and 2j+1 (src/kernels.cpp:65-73)
// as whole-word byte operations: bytes 0..3 of sc/mn hold sub-blocks 0..3
// (j < 2) or 4..7 (j >= 2); the pair is bytes 2(j%2), 2(j%2)+1.
__device__ __forceinline__ void kq_pair_scales(uint32_t s0, uint32_t s1, uint32_t s2, int j,
                                               float& sc_lo, float& sc_hi, float& mn_lo,
                                               float& mn_hi) {
    const bool upper = j >= 2;
    const uint32_t mA = upper ? 0x0F0F0F0Fu : 0x3F3F3F3Fu;
    const uint32_t mB = upper ? 0x30303030u : 0u;
    const int shB = upper ? 4 : 0, sel = 16 * (j & 1);
    const uint32_t sc = (((upper ? s2 : s0) & mA) | ((s0 >> 2) & mB)) >> sel;
    const uint32_t mn = ((((upper ? s2 : s1) >> shB) & mA) | ((s1 >> 2) & mB)) >> sel;
    sc_lo = cvt_ub<0>(sc);
    sc_hi = cvt_ub<1>(sc);
    mn_lo = cvt_ub<0>(mn);
    mn_hi = cvt_ub<1>(mn);
}

// Lambdas passed to word_loop are inlined so that their row / word
// indices stay compile-time constants (else arrays they index go to scratch).
#define AERO_INLINE __attribute__((always_inline))

template <int TYPE> struct Lane64;

// Q4_K (src/kernels.cpp:123-156). Low nibbles are masked in place; high
// nibbles are kept as 16*q (exact), their scale carries the 1/16.
template <> struct Lane64<AERO_DTYPE_Q4_K> {
    uint4 hd, q[2];
    __device__ __forceinline__ void load(const uint8_t* rowp, int st, int l, int n_blk) {
        const uint32_t kc = (uint32_t)min(st * 16 + (l >> 2), n_blk - 1);
        const uint32_t oh = kc * 144u, oq = oh + 16u + 32u * (uint32_t)(l & 3);
        hd = ld128(rowp + oh);
        q[0] = ld128(rowp + oq);
        q[1] = ld128(rowp + oq + 16);
    }
    template <int R, int T>
    static __device__ __forceinline__ void step(const Lane64 (&u)[R], const XStep<T>& X, int l,
                                                bool live, float (&acc)[R][T]) {
        float al[R][1][T], ah[R][1][T];
        word_loop<R, T, 1>(
            X, l, l,
            [&](int r, int m, uint32_t& lo, uint32_t& hi) AERO_INLINE {
                const uint32_t w = wd(u[r].q, m);
                lo = w & 0x0F0F0F0Fu;
                hi = w & 0xF0F0F0F0u;
            },
            [](int m, int& ql, int& qh) AERO_INLINE { ql = m; qh = 8 + m; }, [](int) AERO_INLINE { return 0; }, al, ah);
        float2 sx[T];
#pragma unroll
        for (int t = 0; t < T; ++t) sx[t] = *reinterpret_cast<const float2*>(&X.s[t][2 * l]);
#pragma unroll
        for (int r = 0; r < R; ++r) {
            float sc_lo, sc_hi, mn_lo, mn_hi;
            kq_pair_scales(u[r].hd.y, u[r].hd.z, u[r].hd.w, l & 3, sc_lo, sc_hi, mn_lo, mn_hi);
            const float d = f16f(u[r].hd.x), dm = f16f(u[r].hd.x >> 16);
            const float f_lo = d * sc_lo, f_hi = (d * 0.0625f) * sc_hi;
            const float g_lo = dm * mn_lo, g_hi = dm * mn_hi;
#pragma unroll
            for (int t = 0; t < T; ++t) {
                float a = acc[r][t];
                a = __builtin_fmaf(f_lo, al[r][0][t], a);
                a = __builtin_fmaf(f_hi, ah[r][0][t], a);
                a = __builtin_fmaf(-g_lo, sx[t].x, a);
                a = __builtin_fmaf(-g_hi, sx[t].y, a);
                acc[r][t] = live ? a : acc[r][t];
            }
        }
    }
};

// Q5_K (src/kernels.cpp:90-121): Q4_K plus bit k of qh[i] as bit 4 of value
// i of sub-block k, moved there with a rotate of the qh word.
template <> struct Lane64<AERO_DTYPE_Q5_K> {
    uint4 hd, h[2], q[2];
    __device__ __forceinline__ void load(const uint8_t* rowp, int st, int l, int n_blk) {
        const uint32_t kc = (uint32_t)min(st * 16 + (l >> 2), n_blk - 1);
        const uint32_t oh = kc * 176u, oq = oh + 48u + 32u * (uint32_t)(l & 3);
        hd = ld128(rowp + oh);
        h[0] = ld128(rowp + oh + 16);
        h[1] = ld128(rowp + oh + 32);
        q[0] = ld128(rowp + oq);
        q[1] = ld128(rowp + oq + 16);
    }
    template <int R, int T>
    static __device__ __forceinline__ void step(const Lane64 (&u)[R], const XStep<T>& X, int l,
                                                bool live, float (&acc)[R][T]) {
        const int j = l & 3;
        const uint32_t s_lo = (uint32_t)(2 * j - 4) & 31u, s_hi = (uint32_t)(2 * j - 3) & 31u;
        float al[R][1][T], ah[R][1][T];
        word_loop<R, T, 1>(
            X, l, l,
            [&](int r, int m, uint32_t& lo, uint32_t& hi) AERO_INLINE {
                const uint32_t w = wd(u[r].q, m), hb = wd(u[r].h, m);
                lo = (w & 0x0F0F0F0Fu) | (rotr(hb, s_lo) & 0x10101010u);
                hi = ((w >> 4) & 0x0F0F0F0Fu) | (rotr(hb, s_hi) & 0x10101010u);
            },
            [](int m, int& ql, int& qh) AERO_INLINE { ql = m; qh = 8 + m; }, [](int) AERO_INLINE { return 0; }, al, ah);
        float2 sx[T];
#pragma unroll
        for (int t = 0; t < T; ++t) sx[t] = *reinterpret_cast<const float2*>(&X.s[t][2 * l]);
#pragma unroll
        for (int r = 0; r < R; ++r) {
            float sc_lo, sc_hi, mn_lo, mn_hi;
            kq_pair_scales(u[r].hd.y, u[r].hd.z, u[r].hd.w, j, sc_lo, sc_hi, mn_lo, mn_hi);
            const float d = f16f(u[r].hd.x), dm = f16f(u[r].hd.x >> 16);
            const float f_lo = d * sc_lo, f_hi = d * sc_hi;
            const float g_lo = dm * mn_lo, g_hi = dm * mn_hi;
#pragma unroll
            for (int t = 0; t < T; ++t) {
                float a = acc[r][t];
                a = __builtin_fmaf(f_lo, al[r][0][t], a);
                a = __builtin_fmaf(f_hi, ah[r][0][t], a);
                a = __builtin_fmaf(-g_lo, sx[t].x, a);
                a = __builtin_fmaf(-g_hi, sx[t].y, a);
                acc[r][t] = live ? a : acc[r][t];
            }
        }
    }
};

// IQ4_XS (src/kernels.cpp:217-238): sub-block k uses q[16k .. 16k+16):
// values 0..15 from low nibbles, 16..31 from high; u = codebook + 128 by
// byte permutes of the packed codebook.
template <> struct Lane64<AERO_DTYPE_IQ4_XS> {
    uint2 hd, q[4];
    __device__ __forceinline__ void load(const uint8_t* rowp, int st, int l, int n_blk) {
        const uint32_t kc = (uint32_t)min(st * 16 + (l >> 2), n_blk - 1);
        const uint32_t oh = kc * 136u, oq = oh + 8u + 32u * (uint32_t)(l & 3);
        hd = ld64(rowp + oh);
#pragma unroll
        for (int i = 0; i < 4; ++i) q[i] = ld64(rowp + oq + 8 * i);
    }
    __device__ __forceinline__ uint32_t word(int m) const {
        return (m & 1) ? q[m >> 1].y : q[m >> 1].x;
    }
    template <int R, int T>
    static __device__ __forceinline__ void step(const Lane64 (&u)[R], const XStep<T>& X, int l,
                                                bool live, float (&acc)[R][T]) {
        // words 0..3: sub-block 2j (columns 0..31 of the lane), 4..7: 2j+1
        float al[R][2][T], ah[R][2][T];
        word_loop<R, T, 2>(
            X, l, l,
            [&](int r, int m, uint32_t& lo, uint32_t& hi) AERO_INLINE {
                const uint32_t w = u[r].word(m);
                lo = iq4_bytes(w & 0x0F0F0F0Fu);
                hi = iq4_bytes((w >> 4) & 0x0F0F0F0Fu);
            },
            [](int m, int& ql, int& qh) AERO_INLINE {
                ql = (m & 3) + 8 * (m >> 2);
                qh = ql + 4;
            },
            [](int m) AERO_INLINE { return m >> 2; }, al, ah);
        const int j = l & 3;
        float2 sx[T];
#pragma unroll
        for (int t = 0; t < T; ++t) sx[t] = *reinterpret_cast<const float2*>(&X.s[t][2 * l]);
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const uint32_t shw = u[r].hd.x >> 16, slw = u[r].hd.y;
            const uint32_t ls0 = ((slw >> (8 * j)) & 15u) | (((shw >> (4 * j)) & 3u) << 4);
            const uint32_t ls1 = ((slw >> (8 * j + 4)) & 15u) | (((shw >> (4 * j + 2)) & 3u) << 4);
            const float d = f16f(u[r].hd.x);
            const float f0 = d * (float)((int)ls0 - 32), f1 = d * (float)((int)ls1 - 32);
#pragma unroll
            for (int t = 0; t < T; ++t) {
                float a = acc[r][t];
                a = __builtin_fmaf(f0, al[r][0][t] + ah[r][0][t], a);
                a = __builtin_fmaf(f1, al[r][1][t] + ah[r][1][t], a);
                a = __builtin_fmaf(-128.0f * f0, sx[t].x, a);
                a = __builtin_fmaf(-128.0f * f1, sx[t].y, a);
                acc[r][t] = live ? a : acc[r][t];
            }
        }
    }
};

// Q8_0 (src/kernels.cpp:78-84): the lane's two blocks are 68 bytes at byte
// 68l of the step, loaded as the five 16-byte-aligned chunks around them;
// u = q ^ 0x80 = q + 128. Rows start on 8-byte boundaries at least (the
// 896-column rows of 952 bytes alternate between 16- and 8-byte aligned),
// so the blocks' absolute address is 4-byte aligned and ph in {0,4,8,12}.
template <> struct Lane64<AERO_DTYPE_Q8_0> {
    uint4 c[5];
    uint32_t ph;  // byte offset of the blocks within c
    __device__ __forceinline__ void load(const uint8_t* rowp, int st, int l, int n_blk) {
        // n_blk is a multiple of 4: clamp to the last even block pair
        const uint32_t kc = (uint32_t)min(st * 128 + 2 * l, n_blk - 2);
        const uint32_t ob = kc * 34u;
        // the 16-byte boundary at or below the blocks' absolute address (ph
        // may exceed ob on a row that starts 8 bytes past a boundary, so the
        // base is not formed as rowp + (ob - ph) in 32-bit arithmetic)
        const uintptr_t a = reinterpret_cast<uintptr_t>(rowp) + ob;
        ph = (uint32_t)(a & 15u);
        const uint8_t* base = reinterpret_cast<const uint8_t*>(a - ph);
#pragma unroll
        for (int i = 0; i < 5; ++i) c[i] = ld128(base + 16 * i);
    }
    template <int R, int T>
    static __device__ __forceinline__ void step(const Lane64 (&u)[R], const XStep<T>& X, int l,
                                                bool live, float (&acc)[R][T]) {
        uint32_t qa[R][8], qb[R][8], da[R], db[R];
#pragma unroll
        for (int r = 0; r < R; ++r) {
            uint32_t w[17];
            shifted_words<17, 5>(u[r].c, u[r].ph, w);
            da[r] = w[0];
            db[r] = w[8] >> 16;
#pragma unroll
            for (int m = 0; m < 8; ++m) {
                qa[r][m] = __builtin_amdgcn_alignbyte(w[m + 1], w[m], 2) ^ 0x80808080u;
                qb[r][m] = w[9 + m] ^ 0x80808080u;
            }
        }
        float al[R][1][T], ah[R][1][T];
        word_loop<R, T, 1>(
            X, l, l,
            [&](int r, int m, uint32_t& lo, uint32_t& hi) AERO_INLINE {
                lo = qa[r][m];
                hi = qb[r][m];
            },
            [](int m, int& ql, int& qh) AERO_INLINE { ql = m; qh = 8 + m; }, [](int) AERO_INLINE { return 0; }, al, ah);
        float2 sx[T];
#pragma unroll
        for (int t = 0; t < T; ++t) sx[t] = *reinterpret_cast<const float2*>(&X.s[t][2 * l]);
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const float fa = f16f(da[r]), fb = f16f(db[r]);
#pragma unroll
            for (int t = 0; t < T; ++t) {
                float a = acc[r][t];
                a = __builtin_fmaf(fa, al[r][0][t], a);
                a = __builtin_fmaf(fb, ah[r][0][t], a);
                a = __builtin_fmaf(-128.0f * fa, sx[t].x, a);
                a = __builtin_fmaf(-128.0f * fb, sx[t].y, a);
                acc[r][t] = live ? a : acc[r][t];
            }
        }
    }
};

// Q6_K (src/kernels.cpp:170-200): lane j = 2h + a of a block takes quarters
// a and a+2 of half h: low / high nibbles of ql[64h + 32a + i] with qh[32h + i]
// bits 2a and 4+2a as bits 4-5; scale sc[8h + 2*quarter + i/16]; u = q + 32.
template <> struct Lane64<AERO_DTYPE_Q6_K> {
    uint4 l3[3], h3[3];
    uint32_t ph, sa, sb, d;
    __device__ __forceinline__ void load(const uint8_t* rowp, int st, int l, int n_blk) {
        const uint32_t kc = (uint32_t)min(st * 16 + (l >> 2), n_blk - 1);
        const uint32_t j = (uint32_t)(l & 3), h = j >> 1, a = j & 1;
        const uint32_t ob = kc * 210u;
        ph = ob & 15u;
        const uint8_t* bl = rowp + (ob - ph);
#pragma unroll
        for (int i = 0; i < 3; ++i) {
            l3[i] = ld128(bl + 64 * h + 32 * a + 16 * i);
            h3[i] = ld128(bl + 128 + 32 * h + 16 * i);
        }
        const uint8_t* sc = rowp + ob + 192 + 8 * h + 2 * a;
        sa = *reinterpret_cast<const uint16_t*>(sc);
        sb = *reinterpret_cast<const uint16_t*>(sc + 4);
        d = *reinterpret_cast<const uint16_t*>(rowp + ob + 208);
    }
    template <int R, int T>
    static __device__ __forceinline__ void step(const Lane64 (&u)[R], const XStep<T>& X, int l,
                                                bool live, float (&acc)[R][T]) {
        const int a = l & 1;
        const uint32_t sl = 4 - 2 * a, sr = 2 * a;
        uint32_t lo[R][8], hi[R][8];
#pragma unroll
        for (int r = 0; r < R; ++r) {
            uint32_t wl[8], wh[8];
            shifted_words<8, 3>(u[r].l3, u[r].ph, wl);
            shifted_words<8, 3>(u[r].h3, u[r].ph, wh);
#pragma unroll
            for (int m = 0; m < 8; ++m) {
                lo[r][m] = (wl[m] & 0x0F0F0F0Fu) | ((wh[m] << sl) & 0x30303030u);
                hi[r][m] = ((wl[m] >> 4) & 0x0F0F0F0Fu) | ((wh[m] >> sr) & 0x30303030u);
            }
        }
        // quarter a: columns in lane l-a, quarter a+2: lane l-a+1; x rows
        // 8a.. of those lanes; groups: values 0..15 / 16..31 of each quarter
        float al[R][2][T], ah[R][2][T];
        word_loop<R, T, 2>(
            X, l - a, l - a + 1,
            [&](int r, int m, uint32_t& lw, uint32_t& hw) AERO_INLINE {
                lw = lo[r][m];
                hw = hi[r][m];
            },
            [a](int m, int& ql, int& qh) AERO_INLINE { ql = qh = 8 * a + m; }, [](int m) AERO_INLINE { return m >> 2; },
            al, ah);
        float2 sq_a[T], sq_b[T];
#pragma unroll
        for (int t = 0; t < T; ++t) {
            sq_a[t] = *reinterpret_cast<const float2*>(&X.s16[t][4 * l - 2 * a]);
            sq_b[t] = *reinterpret_cast<const float2*>(&X.s16[t][4 * l - 2 * a + 4]);
        }
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const float df = f16f(u[r].d);
            const float f0 = df * (float)(int8_t)(u[r].sa & 0xFFu);
            const float f1 = df * (float)(int8_t)((u[r].sa >> 8) & 0xFFu);
            const float f2 = df * (float)(int8_t)(u[r].sb & 0xFFu);
            const float f3 = df * (float)(int8_t)((u[r].sb >> 8) & 0xFFu);
#pragma unroll
            for (int t = 0; t < T; ++t) {
                float v = acc[r][t];
                v = __builtin_fmaf(f0, al[r][0][t], v);
                v = __builtin_fmaf(f1, al[r][1][t], v);
                v = __builtin_fmaf(f2, ah[r][0][t], v);
                v = __builtin_fmaf(f3, ah[r][1][t], v);
                v = __builtin_fmaf(-32.0f * f0, sq_a[t].x, v);
                v = __builtin_fmaf(-32.0f * f1, sq_a[t].y, v);
                v = __builtin_fmaf(-32.0f * f2, sq_b[t].x, v);
                v = __builtin_fmaf(-32.0f * f3, sq_b[t].y, v);
                acc[r][t] = live ? v : acc[r][t];
            }
        }
    }
};

// Each step's x is loaded before its weights: loads complete in order, so
// the wait for x before the barrier does not also wait for the weights.
// PIPE (rows of more than one step): the next step's x and weights are
// loaded before the current step is computed, for step min(st+1, last) so
// that every load is unconditional.
// Rows of at most 1024 / 2048 columns fill only 16 / 32 of a wave's lanes:
// with sub = 2 / 1 each group of 64 >> sub lanes takes a row of its own (lane
// l: row slot l >> (6 - sub), column slot l & ((64 >> sub) - 1)); a row's sum
// is a butterfly over its group.
__device__ __forceinline__ float sub_sum(float v, int sub) {
    return sub == 0 ? group_sum<64>(v) : (sub == 1 ? group_sum<32>(v) : group_sum<16>(v));
}
// the width of rows a wave's sub-groups take whole (0: one row a wave)
inline int gemv_sub(int64_t n_cols) {
    if (!tune("gemv_half", 1)) return 0;
    return n_cols <= kStepCols / 4 ? 2 : (n_cols <= kStepCols / 2 ? 1 : 0);
}

template <int TYPE, int R, int T, bool PIPE, bool SUBR = false>
__global__ __launch_bounds__(64 * kGemvWaves) void gemv64_kernel(GemvParams p) {
    using L = Lane64<TYPE>;
    constexpr int BV = QT<TYPE>::BV;
    __shared__ __align__(16) XStep<T> xs[PIPE ? 2 : 1];

    const int tid = threadIdx.x;
    const int l = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    // p.sub: each group of 64 >> sub lanes takes a row (R << sub rows a
    // wave); lc is the lane's 64-column slot within its row
    const int sub = SUBR && !PIPE ? p.sub : 0;   // SUBR: rows of one step or less
    const int lc = l & ((64 >> sub) - 1), lrow = l >> (6 - sub);
    const int64_t r0 = (((int64_t)blockIdx.x * kGemvWaves + wave) * R) << sub;
    const int n_blk = p.n_cols / BV;
    const int n_st = (p.n_cols + kStepCols - 1) / kStepCols;

    const uint8_t* rowp[R];
#pragma unroll
    for (int r = 0; r < R; ++r)
        rowp[r] = p.w + min(r0 + (r << sub) + lrow, p.n_rows - 1) * p.rb;

    float acc[R][T];
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
        for (int t = 0; t < T; ++t) acc[r][t] = 0.0f;

    XStepRegs<T> xr;
    L ua[R];
    xstep_load<T>(p, 0, tid, xr);
#pragma unroll
    for (int r = 0; r < R; ++r) ua[r].load(rowp[r], 0, lc, n_blk);
    bool live_a = kLaneCols * lc < p.n_cols;
    xstep_store<T>(xs[0], xr, tid);
    __syncthreads();

    if constexpr (!PIPE) {
        L::template step<R, T>(ua, xs[0], lc, live_a, acc);  // rows of one step
    } else {
        L ub[R];
        bool live_b;
        for (int st = 0; st < n_st; st += 2) {
            const int s1 = min(st + 1, n_st - 1);
            xstep_load<T>(p, s1, tid, xr);
#pragma unroll
            for (int r = 0; r < R; ++r) ub[r].load(rowp[r], s1, lc, n_blk);
            live_b = st + 1 < n_st && s1 * kStepCols + kLaneCols * lc < p.n_cols;
            __builtin_amdgcn_sched_barrier(0);
            L::template step<R, T>(ua, xs[0], lc, live_a, acc);
            xstep_store<T>(xs[1], xr, tid);
            __syncthreads();
            if (st + 1 >= n_st) break;
            const int s2 = min(st + 2, n_st - 1);
            xstep_load<T>(p, s2, tid, xr);
#pragma unroll
            for (int r = 0; r < R; ++r) ua[r].load(rowp[r], s2, lc, n_blk);
            live_a = st + 2 < n_st && s2 * kStepCols + kLaneCols * lc < p.n_cols;
            __builtin_amdgcn_sched_barrier(0);
            L::template step<R, T>(ub, xs[1], lc, live_b, acc);
            xstep_store<T>(xs[0], xr, tid);
            __syncthreads();
        }
    }

#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
        for (int t = 0; t < T; ++t) {
            const float v = sub_sum(acc[r][t], sub);
            const int64_t row = r0 + (r << sub) + lrow;
            if (lc == 0 && row < p.n_rows && t < p.n_tok) p.y[t * p.y_stride + row] = v;
        }
}

// ------------------------------------------------ fused decode variants
// gemv64_kernel with its neighbours of a decoder layer folded in (the
// reference runs them as separate passes: rmsnorm_rows src/transformer.cpp:
// 98-104, matvec src/kernels.cpp:497-518, act_mul src/tensor.cpp:104-125):
//   * RMSNorm of x in the prologue: every workgroup sums x^2 of its tokens
//     over the row (from L2), inv = 1/sqrtf(ss/n + eps) as the norm kernels,
//     and stages (x*inv)*w (w, or 1+w with AERO_NORM_UNIT_OFFSET) in LDS in
//     place of x; norm < 0: x as is;
//   * MULTI: up to four matrices of one type and width sharing x in one
//     launch (q, k, v; a DeltaNet layer's qkv, gate, alpha, beta):
//     workgroups [blk[m], blk[m+1]) take matrix m;
//   * PAIR: row i of w[0] (gate) and of w[1] (up) in the same wave, written
//     as act(gate . x) * (up . x) (the act·mul op's arithmetic);
//   * RESID: the residual add before the norm (src/model.cpp:244-245, 284):
//     every x load also loads d and uses x + d (one fp32 add, as add_rmsnorm),
//     and workgroup 0 stores x + d to xo, which overlaps neither x nor d (the
//     other workgroups still read them);
//   * GATED: the gated-DeltaNet norm in place of the RMSNorm (src/ssm.cpp:
//     322-340): x / sqrt(mean(x^2) + eps) * norm_w[c % w_len] * silu(z[c]),
//     the row's sum of squares as the RMSNorm's, z loaded with x;
//   * RoPE on the outputs of matrices m < rope_mats (q, k; the rotation of
//     src/attention_layer.cpp:120-156 over every channel of heads of
//     rope_D rows, angle (float)pos * inv[p] as the RoPE kernel): NeoX
//     pairs (i, i + D/2) are 64 or 32 rows apart, so a workgroup of such a
//     matrix owns 2R rows of a head's first half (waves 0, 1) and the same
//     2R rows of its second half (waves 2, 3), and the partners' sums meet
//     in LDS; interleaved pairs (2i, 2i+1) are two rows of one wave.
// Two rows a wave, as gemv64_kernel<.., 2, ..>.
struct GemvFuse {
    const uint8_t* w[4];
    float* y[4];          // y[m][t * n_rows[m] + r]; PAIR: y[0]
    int64_t n_rows[4];    // PAIR: n_rows[0] rows of each of gate and up
    int blk[5];           // MULTI: first workgroup of each matrix, blk[4] = total
    const float* x;       // [n_tok][n_cols]
    const float* norm_w;  // nullable (ones)
    const float* d;       // RESID: [n_tok][n_cols], added to x
    float* xo;            // RESID: x + d, written by workgroup 0
    const float* z;       // GATED: [n_tok][n_cols], the gate
    int w_len;            // GATED: norm_w's length, tiled over the row
    float eps;
    int norm;             // < 0: no norm; else AERO_NORM_UNIT_OFFSET or 0
    int act;              // PAIR: AERO_ACT_*
    int n_cols;
    int64_t rb;
    int n_tok;            // tokens this launch handles (<= T)
    int rope_mats;        // matrices 0 .. rope_mats-1 rotate their outputs (0: none)
    int rope_D;           // rows a head (every channel rotates)
    int rope_mode;        // AERO_ROPE_NEOX / AERO_ROPE_INTERLEAVED
    const int32_t* pos;   // [n_tok] positions of this launch's tokens
    const float* inv;     // [rope_D / 2] inverse frequencies
    int sub;              // rows of <= 2048 (1) / 1024 (2) columns, no RoPE: a row a 64 >> sub lanes
    // one token, matrix 0 = a DeltaNet layer's qkv projection: its rows go
    // through the causal conv (kernel 4) and silu instead of to y[0]
    const float* conv_w;  // [n_rows[0]][4] taps, or null
    float* conv_tail;     // [3][n_rows[0]] history, conv_tl rows valid; updated
    float* conv_out;      // [n_rows[0]]
    int64_t conv_tl;
};

// Channel c of a DeltaNet layer's causal depthwise conv (kernel 4) over
// [history; v] for one new token v, silu in the store, and the channel's
// history moved on by one: the arithmetic of ssm_conv_k_kernel (ssm.hip) at
// T = 1 (src/ssm.cpp:297-301), the history read before it is written.
__device__ __forceinline__ void conv_fold(const GemvFuse& f, int64_t c, float v) {
    constexpr int K = 4;
    const int64_t C = f.n_rows[0], tl = f.conv_tl;
    float win[K];
    float acc = 0.0f;
#pragma unroll
    for (int j = 0; j < K; ++j) {
        const int64_t b = tl + 1 - K + j;
        win[j] = j == K - 1 ? v : (b < 0 ? 0.0f : f.conv_tail[b * C + c]);
        if (b >= 0) acc = acc + win[j] * f.conv_w[c * K + j];
    }
    f.conv_out[c] = silu_fast(acc);
    const int keep = (int)(tl + 1 < K - 1 ? tl + 1 : K - 1);
#pragma unroll
    for (int i = 0; i < K - 1; ++i)
        if (i < keep) f.conv_tail[i * C + c] = win[K - keep + i];
}

__device__ __forceinline__ float act_rt(int kind, float v) {
    switch (kind) {
    case AERO_ACT_SILU: return act<AERO_ACT_SILU>(v);
    case AERO_ACT_GELU: return act<AERO_ACT_GELU>(v);
    case AERO_ACT_GELU_TANH: return act<AERO_ACT_GELU_TANH>(v);
    default: return v;
    }
}

// R rows a wave: 4 in PAIR mode (2 of gate, the same 2 of up) and for 4
// tokens, else 2 (as gemv64_kernel picks for these shapes). The first
// step's weights are requested before the norm is computed (after x, which
// the norm waits for); for rows of one step the x loaded for the norm is the
// x staged.
template <int TYPE, int T, bool PIPE, bool PAIR, bool RESID, bool GATED = false,
          bool SUBR = false>
__global__ __launch_bounds__(64 * kGemvWaves) void gemv64_fused_kernel(GemvFuse f) {
    using L = Lane64<TYPE>;
    constexpr int R = (PAIR || T == 4) ? 4 : 2;
    constexpr int BV = QT<TYPE>::BV;
    __shared__ __align__(16) XStep<T> xs[PIPE ? 2 : 1];
    __shared__ float red[kGemvWaves][T];
    __shared__ float rot[kGemvWaves][R][T];   // RoPE: each wave's row sums

    const int tid = threadIdx.x;
    const int l = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    // f.sub: each group of 64 >> sub lanes takes a row, so a wave covers
    // R << sub rows; lc is the lane's 64-column slot within its row
    const int sub = SUBR && !PIPE ? f.sub : 0;   // SUBR: rows of one step or less
    const int lc = l & ((64 >> sub) - 1), lrow = l >> (6 - sub);
    const int n_blk = f.n_cols / BV;
    const int n_st = (f.n_cols + kStepCols - 1) / kStepCols;

    int m = 0;
    int64_t r0;
    int pair0 = 0;  // NeoX RoPE: the pair index (within the head) of the wave's first row
    const uint8_t* rowp[R];
    if constexpr (PAIR) {
        // rows r0 .. r0 + R/2 of gate (r < R/2) and of up (r >= R/2)
        r0 = (((int64_t)blockIdx.x * kGemvWaves + wave) * (R / 2)) << sub;
#pragma unroll
        for (int r = 0; r < R; ++r)
            rowp[r] = f.w[r < R / 2 ? 0 : 1] +
                      min(r0 + ((r % (R / 2)) << sub) + lrow, f.n_rows[0] - 1) * f.rb;
    } else {
        const int b = blockIdx.x;
        m = __builtin_amdgcn_readfirstlane((b >= f.blk[1]) + (b >= f.blk[2]) + (b >= f.blk[3]));
        if (m < f.rope_mats && f.rope_mode == AERO_ROPE_NEOX) {
            // 2R pairs a workgroup: rows p0 .. p0+2R-1 of the head's first
            // half (waves 0, 1) and of its second half (waves 2, 3)
            const int P = f.rope_D / 2, per_head = P / (2 * R);
            const int bl = b - f.blk[m];
            const int h = bl / per_head;
            pair0 = (bl % per_head) * (2 * R) + (wave & 1) * R;
            r0 = (int64_t)h * f.rope_D + (wave >= 2 ? P : 0) + pair0;
        } else {
            r0 = (((int64_t)(b - f.blk[m]) * kGemvWaves + wave) * R) << sub;
        }
#pragma unroll
        for (int r = 0; r < R; ++r)
            rowp[r] = f.w[m] + min(r0 + (r << sub) + lrow, f.n_rows[m] - 1) * f.rb;
    }
    GemvParams p{nullptr, f.x, nullptr, 0, f.n_cols, f.rb, f.n_tok, f.n_cols, 0};
    GemvParams pd = p;
    pd.x = f.d;
    GemvParams pz = p;
    pz.x = f.z;
    XStepRegs<T> zr;   // GATED: the gate of the step held in xr
    auto load_z = [&](int st) AERO_INLINE {
        if constexpr (GATED) xstep_load<T>(pz, st, tid, zr);
    };
    // this thread's 16 columns of step st for each token: x, or x + d
    auto load_x = [&](int st, XStepRegs<T>& xq) AERO_INLINE {
        xstep_load<T>(p, st, tid, xq);
        if constexpr (RESID) {
            XStepRegs<T> dv;
            xstep_load<T>(pd, st, tid, dv);
#pragma unroll
            for (int t = 0; t < T; ++t)
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const float4 a = xq.v[t][q], b = dv.v[t][q];
                    xq.v[t][q] = make_float4(a.x + b.x, a.y + b.y, a.z + b.z, a.w + b.w);
                }
        }
    };
    // RESID: workgroup 0 stores x + d of its columns (the last step's clamped
    // copies and the padding tokens are not stored)
    auto store_x = [&](int st, const XStepRegs<T>& xq) AERO_INLINE {
        if constexpr (RESID) {
            const int c = st * kStepCols + 16 * tid;
            if (blockIdx.x != 0 || c >= f.n_cols) return;
#pragma unroll
            for (int t = 0; t < T; ++t) {
                if (t >= f.n_tok) break;
                float* dst = f.xo + (int64_t)t * f.n_cols + c;
#pragma unroll
                for (int q = 0; q < 4; ++q) *reinterpret_cast<float4*>(dst + 4 * q) = xq.v[t][q];
            }
        }
    };

    float inv[T], den[T];
#pragma unroll
    for (int t = 0; t < T; ++t) inv[t] = den[t] = 1.0f;
    // (x * inv) * w (or 1 + w) for this thread's 16 columns of step st; the
    // weights of a step are loaded with its x (load_w), before they are used
    // (branch-free: a load under a branch makes the next wait a full one;
    // without a weight every thread reads the first 64 bytes of x, unused)
    const bool has_w = f.norm >= 0 && f.norm_w != nullptr;
    const bool unit = has_w && (f.norm & AERO_NORM_UNIT_OFFSET);
    const float* wsrc = has_w ? f.norm_w : f.x;
    auto load_w = [&](int st, v4f (&wv)[4]) AERO_INLINE {
        int c0 = has_w ? min(st * kStepCols + 16 * tid, f.n_cols - 16) : 0;
        if constexpr (GATED) c0 %= f.w_len;   // 16 columns inside one period
#pragma unroll
        for (int q = 0; q < 4; ++q) wv[q] = *reinterpret_cast<const v4f*>(wsrc + c0 + 4 * q);
    };
    auto norm_x = [&](v4f (&wv)[4], XStepRegs<T>& xv) AERO_INLINE {
        if constexpr (GATED) {
#pragma unroll
            for (int t = 0; t < T; ++t)
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const float4 v = xv.v[t][q], z = zr.v[t][q];
                    xv.v[t][q] = make_float4(((v.x / den[t]) * wv[q].x) * silu_fast(z.x),
                                             ((v.y / den[t]) * wv[q].y) * silu_fast(z.y),
                                             ((v.z / den[t]) * wv[q].z) * silu_fast(z.z),
                                             ((v.w / den[t]) * wv[q].w) * silu_fast(z.w));
                }
            return;
        }
        if (f.norm < 0) return;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const v4f one = v4f{1.0f, 1.0f, 1.0f, 1.0f};
            wv[q] = has_w ? (unit ? one + wv[q] : wv[q]) : one;
        }
#pragma unroll
        for (int t = 0; t < T; ++t)
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const float4 v = xv.v[t][q];
                xv.v[t][q] = make_float4((v.x * inv[t]) * wv[q].x, (v.y * inv[t]) * wv[q].y,
                                         (v.z * inv[t]) * wv[q].z, (v.w * inv[t]) * wv[q].w);
            }
    };

    // x, then the norm weights, then the matrix weights: loads complete in
    // order, so waiting for x (the norm, the staging) does not wait for W
    XStepRegs<T> xr;
    load_x(0, xr);
    load_z(0);
    v4f wv[4];
    load_w(0, wv);
    __builtin_amdgcn_sched_barrier(0);  // keeps every x load ahead of the weights
    L ua[R];
#pragma unroll
    for (int r = 0; r < R; ++r) ua[r].load(rowp[r], 0, lc, n_blk);

    // the norm of each token's x: squares of this thread's 16 columns of
    // each step (the last step's columns clamped to the row: counted once),
    // a tree sum over the workgroup
    if (f.norm >= 0) {
        float ss[T];
        auto add_sq = [&](int st, const XStepRegs<T>& xq) AERO_INLINE {
            const bool own = st * kStepCols + 16 * tid < f.n_cols;  // not a clamped copy
#pragma unroll
            for (int t = 0; t < T; ++t) {
                float a = 0.0f;
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const float4 v = xq.v[t][q];
                    a += v.x * v.x + v.y * v.y + v.z * v.z + v.w * v.w;
                }
                ss[t] += own ? a : 0.0f;
            }
        };
#pragma unroll
        for (int t = 0; t < T; ++t) ss[t] = 0.0f;
        add_sq(0, xr);
        store_x(0, xr);
        if constexpr (PIPE) {
            for (int st = 1; st < n_st; ++st) {
                XStepRegs<T> xq;
                load_x(st, xq);
                add_sq(st, xq);
                store_x(st, xq);
            }
        }
#pragma unroll
        for (int t = 0; t < T; ++t) {
            ss[t] = group_sum<64>(ss[t]);
            if (l == 0) red[wave][t] = ss[t];
        }
        __syncthreads();
#pragma unroll
        for (int t = 0; t < T; ++t) {
            float a = 0.0f;
#pragma unroll
            for (int w = 0; w < kGemvWaves; ++w) a += red[w][t];
            den[t] = sqrtf(a / (float)f.n_cols + f.eps);
            inv[t] = 1.0f / den[t];
        }
    }
    float acc[R][T];
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
        for (int t = 0; t < T; ++t) acc[r][t] = 0.0f;

    norm_x(wv, xr);
    bool live_a = kLaneCols * lc < f.n_cols;
    xstep_store<T>(xs[0], xr, tid);
    __syncthreads();

    if constexpr (!PIPE) {
        L::template step<R, T>(ua, xs[0], lc, live_a, acc);
    } else {
        L ub[R];
        bool live_b;
        for (int st = 0; st < n_st; st += 2) {
            const int s1 = min(st + 1, n_st - 1);
            load_x(s1, xr);
            load_z(s1);
            load_w(s1, wv);
#pragma unroll
            for (int r = 0; r < R; ++r) ub[r].load(rowp[r], s1, lc, n_blk);
            live_b = st + 1 < n_st && s1 * kStepCols + kLaneCols * lc < f.n_cols;
            __builtin_amdgcn_sched_barrier(0);
            L::template step<R, T>(ua, xs[0], lc, live_a, acc);
            norm_x(wv, xr);
            xstep_store<T>(xs[1], xr, tid);
            __syncthreads();
            if (st + 1 >= n_st) break;
            const int s2 = min(st + 2, n_st - 1);
            load_x(s2, xr);
            load_z(s2);
            load_w(s2, wv);
#pragma unroll
            for (int r = 0; r < R; ++r) ua[r].load(rowp[r], s2, lc, n_blk);
            live_a = st + 2 < n_st && s2 * kStepCols + kLaneCols * lc < f.n_cols;
            __builtin_amdgcn_sched_barrier(0);
            L::template step<R, T>(ub, xs[1], lc, live_b, acc);
            norm_x(wv, xr);
            xstep_store<T>(xs[0], xr, tid);
            __syncthreads();
        }
    }

#pragma unroll
    for (int t = 0; t < T; ++t) {
        if constexpr (PAIR) {
#pragma unroll
            for (int r = 0; r < R / 2; ++r) {
                const float g = sub_sum(acc[r][t], sub);
                const float u = sub_sum(acc[R / 2 + r][t], sub);
                const int64_t row = r0 + (r << sub) + lrow;
                if (lc == 0 && row < f.n_rows[0] && t < f.n_tok)
                    f.y[0][t * f.n_rows[0] + row] = act_rt(f.act, g) * u;
            }
        } else if (m >= f.rope_mats) {
#pragma unroll
            for (int r = 0; r < R; ++r) {
                const float v = sub_sum(acc[r][t], sub);
                const int64_t row = r0 + (r << sub) + lrow;
                if (lc == 0 && row < f.n_rows[m] && t < f.n_tok) {
                    if (!PAIR && !GATED && T == 1 && m == 0 && f.conv_w != nullptr)
                        conv_fold(f, row, v);
                    else
                        f.y[m][t * f.n_rows[m] + row] = v;
                }
            }
        }
    }
    if constexpr (!PAIR) {
        if (m < f.rope_mats) {  // uniform: the workgroup's matrix
            float v[R][T];
#pragma unroll
            for (int t = 0; t < T; ++t)
#pragma unroll
                for (int r = 0; r < R; ++r) v[r][t] = group_sum<64>(acc[r][t]);
            const bool neox = f.rope_mode == AERO_ROPE_NEOX;
            if (neox) {
                if (l == 0) {
#pragma unroll
                    for (int t = 0; t < T; ++t)
#pragma unroll
                        for (int r = 0; r < R; ++r) rot[wave][r][t] = v[r][t];
                }
                __syncthreads();
            }
            if (l == 0) {
#pragma unroll
                for (int t = 0; t < T; ++t) {
                    if (t >= f.n_tok) break;
                    const float pt = (float)f.pos[t];
#pragma unroll
                    for (int r = 0; r < R; ++r) {
                        float o;
                        if (neox) {
                            // x'[i] = x[i] c - x[i+P] s; x'[i+P] = x[i+P] c + x[i] s
                            float sn, c;
                            sincosf(pt * f.inv[pair0 + r], &sn, &c);
                            const float other = rot[wave ^ 2][r][t];
                            o = wave < 2 ? v[r][t] * c - other * sn : v[r][t] * c + other * sn;
                        } else {
                            // x'[2i] = x[2i] c - x[2i+1] s; x'[2i+1] = x[2i] s + x[2i+1] c
                            const int rr = r & ~1;
                            float sn, c;
                            sincosf(pt * f.inv[(int)((r0 + rr) % f.rope_D) / 2], &sn, &c);
                            o = (r & 1) == 0 ? v[rr][t] * c - v[rr + 1][t] * sn
                                             : v[rr][t] * sn + v[rr + 1][t] * c;
                        }
                        if (r0 + r < f.n_rows[m]) f.y[m][t * f.n_rows[m] + r0 + r] = o;
                    }
                }
            }
        }
    }
}

using GemvFusedKernel = void (*)(GemvFuse);

template <int TYPE, bool PAIR, bool RESID>
GemvFusedKernel pick_fused_t(int T, bool pipe, bool subr) {
    if (pipe) {
        switch (T) {
        case 1: return gemv64_fused_kernel<TYPE, 1, true, PAIR, RESID>;
        case 2: return gemv64_fused_kernel<TYPE, 2, true, PAIR, RESID>;
        default: return nullptr;
        }
    }
    switch (T) {
    case 1: return subr ? gemv64_fused_kernel<TYPE, 1, false, PAIR, RESID, false, true>
                        : gemv64_fused_kernel<TYPE, 1, false, PAIR, RESID>;
    case 2: return subr ? gemv64_fused_kernel<TYPE, 2, false, PAIR, RESID, false, true>
                        : gemv64_fused_kernel<TYPE, 2, false, PAIR, RESID>;
    case 4: return subr ? gemv64_fused_kernel<TYPE, 4, false, PAIR, RESID, false, true>
                        : gemv64_fused_kernel<TYPE, 4, false, PAIR, RESID>;
    default: return nullptr;
    }
}

template <bool PAIR, bool RESID>
GemvFusedKernel pick_fused_r(int dtype, int T, bool pipe, bool subr) {
    switch (dtype) {
    case AERO_DTYPE_Q8_0: return pick_fused_t<AERO_DTYPE_Q8_0, PAIR, RESID>(T, pipe, subr);
    case AERO_DTYPE_Q4_K: return pick_fused_t<AERO_DTYPE_Q4_K, PAIR, RESID>(T, pipe, subr);
    case AERO_DTYPE_Q5_K: return pick_fused_t<AERO_DTYPE_Q5_K, PAIR, RESID>(T, pipe, subr);
    case AERO_DTYPE_Q6_K: return pick_fused_t<AERO_DTYPE_Q6_K, PAIR, RESID>(T, pipe, subr);
    case AERO_DTYPE_IQ4_XS: return pick_fused_t<AERO_DTYPE_IQ4_XS, PAIR, RESID>(T, pipe, subr);
    default: return nullptr;
    }
}

template <int TYPE>
GemvFusedKernel pick_gated_t(int T, bool pipe) {
    if (T == 1) return pipe ? gemv64_fused_kernel<TYPE, 1, true, false, false, true>
                            : gemv64_fused_kernel<TYPE, 1, false, false, false, true>;
    if (T == 2) return pipe ? gemv64_fused_kernel<TYPE, 2, true, false, false, true>
                            : gemv64_fused_kernel<TYPE, 2, false, false, false, true>;
    return nullptr;
}

GemvFusedKernel pick_gated(int dtype, int T, bool pipe) {
    switch (dtype) {
    case AERO_DTYPE_Q8_0: return pick_gated_t<AERO_DTYPE_Q8_0>(T, pipe);
    case AERO_DTYPE_Q4_K: return pick_gated_t<AERO_DTYPE_Q4_K>(T, pipe);
    case AERO_DTYPE_Q5_K: return pick_gated_t<AERO_DTYPE_Q5_K>(T, pipe);
    case AERO_DTYPE_Q6_K: return pick_gated_t<AERO_DTYPE_Q6_K>(T, pipe);
    case AERO_DTYPE_IQ4_XS: return pick_gated_t<AERO_DTYPE_IQ4_XS>(T, pipe);
    default: return nullptr;
    }
}

GemvFusedKernel pick_fused(bool pair, bool resid, int dtype, int T, bool pipe, bool subr) {
    if (pair)
        return resid ? pick_fused_r<true, true>(dtype, T, pipe, subr)
                     : pick_fused_r<true, false>(dtype, T, pipe, subr);
    return resid ? pick_fused_r<false, true>(dtype, T, pipe, subr)
                 : pick_fused_r<false, false>(dtype, T, pipe, subr);
}

using GemvKernel = void (*)(GemvParams);

template <int TYPE, int R, bool PIPE, bool SUBR>
GemvKernel pick64_t(int T) {
    switch (T) {
    case 1: return gemv64_kernel<TYPE, R, 1, PIPE, SUBR>;
    case 2: return gemv64_kernel<TYPE, R, 2, PIPE, SUBR>;
    case 4:
        if constexpr (!PIPE) return gemv64_kernel<TYPE, R, 4, PIPE, SUBR>;
        return nullptr;
    default: return nullptr;
    }
}

template <int TYPE, bool PIPE, bool SUBR>
GemvKernel pick64_r(int R, int T) {
    switch (R) {
    case 1: return pick64_t<TYPE, 1, PIPE, SUBR>(T);
    case 2: return pick64_t<TYPE, 2, PIPE, SUBR>(T);
    case 4: return pick64_t<TYPE, 4, PIPE, SUBR>(T);
    default: return nullptr;
    }
}

// SUBR: the sub-wave row layout (rows of one step or less, GemvParams::sub)
template <bool PIPE, bool SUBR = false>
GemvKernel pick64(int dtype, int R, int T) {
    switch (dtype) {
    case AERO_DTYPE_Q8_0: return pick64_r<AERO_DTYPE_Q8_0, PIPE, SUBR>(R, T);
    case AERO_DTYPE_Q4_K: return pick64_r<AERO_DTYPE_Q4_K, PIPE, SUBR>(R, T);
    case AERO_DTYPE_Q5_K: return pick64_r<AERO_DTYPE_Q5_K, PIPE, SUBR>(R, T);
    case AERO_DTYPE_Q6_K: return pick64_r<AERO_DTYPE_Q6_K, PIPE, SUBR>(R, T);
    case AERO_DTYPE_IQ4_XS: return pick64_r<AERO_DTYPE_IQ4_XS, PIPE, SUBR>(R, T);
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
// Whether a matrix takes the 64-column lane kernels (gemv64_kernel and the
// fused decode GEMVs): W 16-byte aligned with rows of whole 16 bytes, or a
// Q8_0 matrix with rows of whole 8 bytes whose lane windows are placed from
// the absolute address. The window of the last row's final block pair ends
// at the first 16-byte boundary at or past that row (up to 8 bytes beyond
// it), which must lie inside w_bytes.
bool lanes64_ok(int dtype, const uint8_t* w, int64_t rb, int64_t n_rows, int64_t w_bytes) {
    if (!aligned16(w)) return false;
    if (rb % 16 == 0) return true;
    if (dtype != AERO_DTYPE_Q8_0 || rb % 8 != 0 || n_rows <= 0) return false;
    const int64_t end = n_rows * rb;
    return w_bytes >= end + ((16 - (end & 15)) & 15);
}

bool gemv_dev(int dtype, const uint8_t* w, int64_t w_bytes, const float* x, float* y,
              int64_t n_rows, int64_t n_cols, int64_t n_tok, hipStream_t s, void* ws,
              int64_t ws_bytes) {
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
    // several tokens: the matrix-core GEMMs. The split-x fp16 one when a
    // workspace is given and the type has it (from 5-16 tokens by the
    // matrix size, split_tokens_ok), else the fp32 one from 32 tokens (W
    // once per 64).
    if (ws != nullptr && n_tok <= (int64_t)1 << 30 && split_tokens_ok(n_tok, n_rows, n_cols)) {
        bool ran = false;
        if (!split_gemm_dev(dtype, w, x, y, n_rows, n_cols, rb, n_tok, ws, ws_bytes, s, &ran))
            return false;
        if (ran) return true;
    }
    if (n_tok >= tune("gemm_min_tokens", 32) && n_tok <= (int64_t)1 << 30)
        return gemm_dev(dtype, w, x, y, n_rows, n_cols, rb, n_tok, s);
    if (lanes64_ok(dtype, w, rb, n_rows, w_bytes) && tune("gemv_lanes64", 1)) {
        const bool pipe = n_cols > kStepCols;
        const int t_max = pipe ? 2 : 4;  // double-buffered x of 4 tokens would fill LDS
        for (int64_t t0 = 0; t0 < n_tok; t0 += t_max) {
            const int nt = (int)std::min<int64_t>(t_max, n_tok - t0);
            const int T = nt == 1 ? 1 : (nt == 2 ? 2 : 4);
            // rows per wave (measured on MI355X): 2 while that leaves >= 256
            // workgroups, else 1; four tokens share the weight decoding over
            // 4 rows when that leaves >= 512 workgroups (>= 256 for rows of
            // several steps)
            // rows of at most 2048 / 1024 columns: a row a half / quarter wave
            const int hf = 1 << gemv_sub(n_cols);
            auto wgs_of = [&](int r) {
                return (n_rows + r * hf * kGemvWaves - 1) / (r * hf * kGemvWaves);
            };
            int R = wgs_of(2) >= 256 ? 2 : 1;
            if (T == 4 && wgs_of(4) >= 512) R = 4;
            // one Q8_0 token of one-step rows: a row a wave (its 80-byte
            // windows leave the wave's loads fewer; twice the workgroups keep
            // more in flight): 4096 x 4096 7.72 -> 6.29 us, 14336 x 4096
            // 17.80 -> 15.67 us on MI355X (Q4_K, Q5_K, Q6_K, IQ4_XS: equal or
            // slower)
            if (dtype == AERO_DTYPE_Q8_0 && T == 1 && !pipe && hf == 1) R = 1;
            R = tune("gemv_r", R);
            const int64_t wgs = wgs_of(R);
            GemvKernel k = pipe ? pick64<true>(dtype, R, T)
                                : (hf > 1 ? pick64<false, true>(dtype, R, T)
                                          : pick64<false>(dtype, R, T));
            if (k == nullptr || wgs > 0x7fffffff) {
                set_error("matvec: no kernel for dtype %d, rows/wave %d", dtype, R);
                return false;
            }
            GemvParams p{w, x + t0 * n_cols, y + t0 * n_rows, n_rows, (int)n_cols, rb, nt,
                         n_cols, n_rows, gemv_sub(n_cols)};
            if (!launch("gemv64_kernel", k, dim3((unsigned)wgs), dim3(64 * kGemvWaves), 0, s, p))
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

// Whether RoPE on the outputs of matrices 0 .. rope.mats-1 folds into the
// fused GEMV: plain (not gate/up) matrices whose rows are whole heads of D
// rows, D even; NeoX needs D a multiple of 16 (a workgroup takes 2R of a
// head's pairs, R up to 4); positions and inverse frequencies given; every
// channel rotates and no per-head norm comes first.
bool rope_fold_ok(const RopeFold& rope, bool pair, int n_mat, const int64_t* n_rows) {
    if (pair || rope.mats < 1 || rope.mats > n_mat || rope.pos == nullptr ||
        rope.inv == nullptr || rope.D < 2 || rope.D % 2 || rope.D > 1024 ||
        rope.rot() != rope.D || rope.qk_norm() ||
        (rope.mode != AERO_ROPE_NEOX && rope.mode != AERO_ROPE_INTERLEAVED) ||
        (rope.mode == AERO_ROPE_NEOX && rope.D % 16))
        return false;
    for (int m = 0; m < rope.mats; ++m)
        if (n_rows[m] % rope.D) return false;
    return true;
}

// The fused decode GEMVs (gemv64_fused_kernel): argument checks, token
// groups of up to 4 (2 for rows of more than one 4096-column step), one
// launch a group. Matrices must take gemv64 (16-byte aligned, rows a
// multiple of 16 bytes). w_bytes[m] >= n_rows[m] * row bytes.
// The gated-DeltaNet norm as the prologue (GATED): the gate z [n_tok][n_cols]
// and the length of the tiled norm weight.
struct GatedIn {
    const float* z;
    int64_t w_len;
};

// a DeltaNet layer's conv (kernel 4) on matrix 0's rows (one token)
struct ConvIn {
    const float* w;
    float* tail;
    int64_t tail_len;
    float* out;
};

static bool gemv_fused_impl(int dtype, bool pair, int n_mat, const uint8_t* const* w,
                            const int64_t* w_bytes, const int64_t* n_rows, float* const* y,
                            const float* x, const float* norm_w, float eps, int norm, int act,
                            int64_t n_cols, int64_t n_tok, hipStream_t s, const float* d,
                            float* xo, const RopeFold* rope, const GatedIn* gated,
                            const ConvIn* conv = nullptr) {
    const char* what = gated ? "gated_norm_matvec" : (pair ? "norm_gate_up" : "norm_matvec");
    const bool quant = dtype == AERO_DTYPE_Q8_0 || dtype == AERO_DTYPE_Q4_K ||
                       dtype == AERO_DTYPE_Q5_K || dtype == AERO_DTYPE_Q6_K ||
                       dtype == AERO_DTYPE_IQ4_XS;
    if (!quant) {
        set_error("%s: dtype %d has no quantised GEMV", what, dtype);
        return false;
    }
    const int64_t bv = dtype_block_values(dtype), bb = dtype_block_bytes(dtype);
    if (n_mat < 1 || n_mat > 4 || (pair && n_mat != 2) || w == nullptr || w_bytes == nullptr ||
        n_rows == nullptr || y == nullptr || x == nullptr || n_cols <= 0 || n_cols % bv != 0 ||
        n_cols > (int64_t)1 << 30 || n_tok < 0 || norm > AERO_NORM_UNIT_OFFSET || act < 0 ||
        act > AERO_ACT_IDENTITY) {
        set_error("%s: bad arguments (n_mat=%d n_cols=%lld n_tok=%lld norm=%d act=%d)", what,
                  n_mat, (long long)n_cols, (long long)n_tok, norm, act);
        return false;
    }
    const int64_t rb = (n_cols / bv) * bb;
    if (!aligned16(x) || (norm_w != nullptr && !aligned16(norm_w))) {
        set_error("%s: x and the norm weight must be 16-byte aligned", what);
        return false;
    }
    if (d != nullptr) {
        // x + d is stored by one workgroup while the others read x and d
        const int64_t nb = n_tok * n_cols * 4;
        auto apart = [nb](const void* a, const void* b) {
            const uintptr_t ua = reinterpret_cast<uintptr_t>(a), ub = reinterpret_cast<uintptr_t>(b);
            return ua + nb <= ub || ub + nb <= ua;
        };
        if (xo == nullptr || norm < 0 || !aligned16(d) || !aligned16(xo) || !apart(xo, x) ||
            !apart(xo, d)) {
            set_error("%s: the residual add needs a norm and x_out 16-byte aligned, overlapping "
                      "neither x nor d", what);
            return false;
        }
    }
    for (int m = 0; m < n_mat; ++m) {
        if (w[m] == nullptr || y[pair ? 0 : m] == nullptr || n_rows[m] < 0 ||
            n_rows[m] > (int64_t)1 << 31 || w_bytes[m] < n_rows[m] * rb ||
            !lanes64_ok(dtype, w[m], rb, n_rows[m], w_bytes[m]) ||
            (pair && n_rows[m] != n_rows[0])) {
            set_error("%s: matrix %d: null, short, rows differ, or not 16-byte aligned with rows "
                      "of whole 16 bytes (Q8_0: 8, with the last row's 16-byte window inside "
                      "w_bytes)", what, m);
            return false;
        }
    }
    if (rope != nullptr && rope->mats > 0 && !rope_fold_ok(*rope, pair, n_mat, n_rows)) {
        set_error("%s: RoPE on %d matrices of heads of %d rows (mode %d) cannot fold", what,
                  rope->mats, rope->D, rope->mode);
        return false;
    }
    if (gated != nullptr &&
        (pair || d != nullptr || (rope != nullptr && rope->mats > 0) || norm != 0 ||
         norm_w == nullptr || gated->z == nullptr || !aligned16(gated->z) ||
         gated->w_len < 16 || gated->w_len % 16 || n_cols % gated->w_len || n_tok > 2)) {
        set_error("%s: the gated norm takes a 16-byte aligned gate, a norm weight whose length "
                  "is a multiple of 16 dividing the row, and at most 2 tokens (n_tok=%lld)",
                  what, (long long)n_tok);
        return false;
    }
    if (conv != nullptr &&
        (pair || d != nullptr || gated != nullptr || (rope != nullptr && rope->mats > 0) ||
         n_tok != 1 || conv->w == nullptr || conv->tail == nullptr || conv->out == nullptr ||
         conv->tail_len < 0 || conv->tail_len > 3)) {
        set_error("%s: the conv fold takes one token, no residual, RoPE or gated norm, and a "
                  "history of 0-3 rows (tail_len=%lld)", what, (long long)conv->tail_len);
        return false;
    }
    if (conv != nullptr) {
        // every workgroup reads x, the weights and the conv weights while
        // single lanes write conv_out[c] and the history rows: those two
        // must be apart from each other and from everything read or written
        // by the other workgroups
        const int64_t C = n_rows[0];
        struct Span {
            const void* p;
            int64_t bytes;
        };
        auto meets = [](Span a, Span b) {
            const uintptr_t ua = reinterpret_cast<uintptr_t>(a.p);
            const uintptr_t ub = reinterpret_cast<uintptr_t>(b.p);
            return a.bytes > 0 && b.bytes > 0 && ua < ub + (uintptr_t)b.bytes &&
                   ub < ua + (uintptr_t)a.bytes;
        };
        const Span out{conv->out, C * 4}, hist{conv->tail, 3 * C * 4};
        bool clash = meets(out, hist) || meets(out, {x, n_cols * 4}) ||
                     meets(hist, {x, n_cols * 4}) || meets(out, {conv->w, C * 16}) ||
                     meets(hist, {conv->w, C * 16});
        for (int m = 0; m < n_mat && !clash; ++m) {
            const Span wm{w[m], w_bytes[m]};
            clash = meets(out, wm) || meets(hist, wm);
            if (m > 0) {
                const Span ym{y[m], n_rows[m] * 4};
                clash = clash || meets(out, ym) || meets(hist, ym);
            }
        }
        if (clash) {
            set_error("%s: conv_out and the history tail must overlap neither each other nor x, "
                      "the weights, the conv weights or the other outputs", what);
            return false;
        }
    }
    if (n_tok == 0) return true;
    GemvFuse f{};
    if (gated != nullptr) f.w_len = (int)gated->w_len;
    if (conv != nullptr) {
        f.conv_w = conv->w;
        f.conv_tail = conv->tail;
        f.conv_out = conv->out;
        f.conv_tl = conv->tail_len;
    }
    if (rope != nullptr && rope->mats > 0) {
        f.rope_mats = rope->mats;
        f.rope_D = rope->D;
        f.rope_mode = rope->mode;
        f.inv = rope->inv;
    }
    // rows of at most 2048 / 1024 columns fill only half / a quarter of a
    // wave's 64-column lanes: each half / quarter wave then takes a row of its
    // own (not with RoPE, whose row pairs follow the one-row-a-wave layout)
    f.sub = f.rope_mats == 0 && gated == nullptr ? gemv_sub(n_cols) : 0;
    // workgroups of a launch of T tokens: rows a wave as the kernel's R, times
    // 2^sub
    auto grid_of = [&](int T, GemvFuse& g) -> int64_t {
        const int R = ((pair || T == 4) ? 4 : 2) << f.sub;
        int64_t tot = 0;
        if (pair) return (n_rows[0] + (int64_t)kGemvWaves * (R / 2) - 1) / (kGemvWaves * (R / 2));
        for (int m = 0; m < 4; ++m) {
            g.blk[m] = (int)std::min<int64_t>(tot, 0x7fffffff);
            if (m < n_mat) tot += (n_rows[m] + (int64_t)kGemvWaves * R - 1) / (kGemvWaves * R);
        }
        for (int m = n_mat; m < 4; ++m) g.blk[m] = 0x7fffffff;  // never reached
        g.blk[4] = (int)std::min<int64_t>(tot, 0x7fffffff);
        return tot;
    };
    for (int m = 0; m < n_mat; ++m) {
        f.w[m] = w[m];
        f.n_rows[m] = n_rows[m];
    }
    f.norm_w = norm_w;
    f.eps = eps;
    f.norm = norm;
    f.act = act;
    f.n_cols = (int)n_cols;
    f.rb = rb;
    const bool pipe = n_cols > kStepCols;
    const int t_max = pipe ? 2 : 4;
    for (int64_t t0 = 0; t0 < n_tok; t0 += t_max) {
        const int nt = (int)std::min<int64_t>(t_max, n_tok - t0);
        const int T = nt == 1 ? 1 : (nt == 2 ? 2 : 4);
        GemvFusedKernel k = gated ? pick_gated(dtype, T, pipe)
                              : pick_fused(pair, d != nullptr, dtype, T, pipe, f.sub > 0);
        if (k == nullptr) {
            set_error("%s: no kernel for %d tokens", what, T);
            return false;
        }
        f.x = x + t0 * n_cols;
        f.pos = f.rope_mats > 0 ? rope->pos + t0 : nullptr;
        f.d = d ? d + t0 * n_cols : nullptr;
        f.xo = d ? xo + t0 * n_cols : nullptr;
        f.z = gated ? gated->z + t0 * n_cols : nullptr;
        f.n_tok = nt;
        for (int m = 0; m < (pair ? 1 : n_mat); ++m) f.y[m] = y[m] + t0 * n_rows[m];
        const int64_t total = grid_of(T, f);
        if (total == 0) continue;
        if (total > 0x7fffffff) {
            set_error("%s: grid too large", what);
            return false;
        }
        if (!launch(pair ? "gemv64_fused_kernel<pair>" : "gemv64_fused_kernel", k,
                    dim3((unsigned)total), dim3(64 * kGemvWaves), 0, s, f))
            return false;
    }
    return true;
}

bool gemv_fused_dev(int dtype, bool pair, int n_mat, const uint8_t* const* w,
                    const int64_t* w_bytes, const int64_t* n_rows, float* const* y,
                    const float* x, const float* norm_w, float eps, int norm, int act,
                    int64_t n_cols, int64_t n_tok, hipStream_t s, const float* d,
                    float* xo, const RopeFold* rope) {
    return gemv_fused_impl(dtype, pair, n_mat, w, w_bytes, n_rows, y, x, norm_w, eps, norm, act,
                           n_cols, n_tok, s, d, xo, rope, nullptr);
}

bool gemv_conv_dev(int dtype, int n_mat, const uint8_t* const* w, const int64_t* w_bytes,
                   const int64_t* n_rows, float* const* y, const float* x, int64_t n_cols,
                   const float* conv_w, float* tail, int64_t tail_len, float* conv_out,
                   hipStream_t s) {
    const ConvIn c{conv_w, tail, tail_len, conv_out};
    return gemv_fused_impl(dtype, false, n_mat, w, w_bytes, n_rows, y, x, nullptr, 0.f, -1,
                           AERO_ACT_IDENTITY, n_cols, 1, s, nullptr, nullptr, nullptr, nullptr,
                           &c);
}

bool gemv_gated_dev(int dtype, const uint8_t* w, int64_t w_bytes, int64_t n_rows, float* y,
                    const float* x, const float* z, const float* norm_w, int64_t w_len,
                    float eps, int64_t n_cols, int64_t n_tok, hipStream_t s) {
    const GatedIn g{z, w_len};
    return gemv_fused_impl(dtype, false, 1, &w, &w_bytes, &n_rows, &y, x, norm_w, eps, 0,
                           AERO_ACT_IDENTITY, n_cols, n_tok, s, nullptr, nullptr, nullptr, &g);
}

}  // namespace aero

extern "C" {

int aero_hip_matvec(int dtype, const uint8_t* w, int64_t w_bytes, const float* x, float* y,
                    int64_t n_rows, int64_t n_cols, int64_t n_tok, void* stream) {
    return aero::gemv_dev(dtype, w, w_bytes, x, y, n_rows, n_cols, n_tok,
                          (hipStream_t)stream, nullptr, 0) ? 1 : 0;
}

int aero_hip_norm_matvec(int dtype, int n_mat, const uint8_t* const* w, const int64_t* w_bytes,
                         const int64_t* n_rows, float* const* y, const float* x,
                         const float* norm_w, float eps, int norm, int64_t n_cols,
                         int64_t n_tok, void* stream) {
    return aero::gemv_fused_dev(dtype, false, n_mat, w, w_bytes, n_rows, y, x, norm_w, eps, norm,
                                AERO_ACT_IDENTITY, n_cols, n_tok, (hipStream_t)stream, nullptr,
                                nullptr, nullptr) ? 1 : 0;
}

int aero_hip_ssm_proj_conv(int dtype, int n_mat, const uint8_t* const* w, const int64_t* w_bytes,
                           const int64_t* n_rows, float* const* y, const float* x,
                           int64_t n_cols, const float* conv_w, float* tail, int64_t tail_len,
                           float* conv_out, void* stream) {
    aero::clear_error();
    if (w == nullptr || w_bytes == nullptr || n_rows == nullptr || y == nullptr || n_mat < 1 ||
        n_mat > 4) {
        aero::set_error("ssm_proj_conv: 1-4 matrices with their sizes and outputs");
        return 0;
    }
    return aero::gemv_conv_dev(dtype, n_mat, w, w_bytes, n_rows, y, x, n_cols, conv_w, tail,
                               tail_len, conv_out, (hipStream_t)stream) ? 1 : 0;
}

int aero_hip_gated_norm_matvec(int dtype, const uint8_t* w, int64_t w_bytes, int64_t n_rows,
                               float* y, const float* x, const float* z, const float* norm_w,
                               int64_t w_len, float eps, int64_t n_cols, int64_t n_tok,
                               void* stream) {
    aero::clear_error();
    return aero::gemv_gated_dev(dtype, w, w_bytes, n_rows, y, x, z, norm_w, w_len, eps, n_cols,
                                n_tok, (hipStream_t)stream) ? 1 : 0;
}

int aero_hip_norm_gate_up(int dtype, const uint8_t* w_gate, const uint8_t* w_up, int64_t w_bytes,
                          const float* x, const float* norm_w, float eps, int norm, int act,
                          float* out, int64_t n_ff, int64_t n_cols, int64_t n_tok,
                          void* stream) {
    const uint8_t* w[2] = {w_gate, w_up};
    const int64_t wb[2] = {w_bytes, w_bytes};
    const int64_t nr[2] = {n_ff, n_ff};
    float* y[2] = {out, out};
    return aero::gemv_fused_dev(dtype, true, 2, w, wb, nr, y, x, norm_w, eps, norm, act, n_cols,
                                n_tok, (hipStream_t)stream, nullptr, nullptr, nullptr) ? 1 : 0;
}

int64_t aero_hip_matmul_workspace(int dtype, int64_t n_cols, int64_t n_tok) {
    return aero::split_gemm_workspace(dtype, n_cols, n_tok);
}

int aero_hip_matmul(int dtype, const uint8_t* w, int64_t w_bytes, const float* x, float* y,
                    int64_t n_rows, int64_t n_cols, int64_t n_tok, void* ws, int64_t ws_bytes,
                    void* stream) {
    return aero::gemv_dev(dtype, w, w_bytes, x, y, n_rows, n_cols, n_tok, (hipStream_t)stream,
                          ws, ws_bytes) ? 1 : 0;
}

}  // extern "C"
