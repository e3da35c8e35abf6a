// Quantised GEMM on the fp16 matrix cores with x split into three fp16 parts
// (prefill): y[t, r] = sum_c W[r, c] * x[t, c], W in Q4_K / Q5_K blocks, x and
// y fp32 — the reference's matmul (src/kernels.cpp:520-538) over its block
// dots (:78-250), at fp32-grade accuracy on the fp16 matrix rate.
//
// Arithmetic. A Q4_K / Q5_K value is (d*sc)*q - (dmin*m) with per-256-value
// fp16 scales d, dmin and per-32-value 6-bit sc, m (src/kernels.cpp:337-404).
// sc*q <= 63*31 is an integer below 2048, exact in fp16, so per super-block
//   sum_c w_c x_c = d * sum_c (sc*q)_c x_c  -  dmin * sum_g m_g * S_g
// with S_g the sum of x over sub-block g. Each token's x is scaled by a power
// of two 2^(15-e) (e the exponent of its largest finite |x|, so the scaled
// values lie below 2^15) and split into three fp16 parts hi + mid + lo: every
// value of at least 2^-16 of the token's largest is represented exactly,
// smaller ones to 2^-25 absolute in the scaled units (2^-39 of the largest).
// Products of fp16 integers and fp16 parts are exact; the matrix cores add
// them in fp32. The reference dequantises each value to fp32 and sums the
// rounded products serially; results differ from it by fp32 rounding only.
//
// Kernels:
//   xscale_kernel   one workgroup a token: the per-token scale and the
//                   sub-block sums S of the scaled x (fp32);
//   xsplit_kernel   the fp16 parts of x in matrix-operand order, padded to
//                   32 tokens with zeros;
//   split_gemm_kernel  4 waves, 256 rows x 32 tokens. y^T is computed as
//                   x^T W^T so that the weights are the B operand: lane l
//                   holds B[k][n = l%16] for k = 8(l/16)..+7, i.e. 8 values
//                   of ONE weight row, and decodes them itself from 16-byte
//                   loads of that row (no LDS for W); its accumulator lanes
//                   hold 4 tokens of the same row, so the row's d, dmin and m
//                   are lane-local. The x parts (A operand) are staged in LDS,
//                   double-buffered per 128-column chunk, shared by the four
//                   waves.
//
// Operand order. Lane group g = l/16 of a row owns qs bytes 32g..32g+31 of
// each super-block: sub-block 2g in the low nibbles, 2g+1 in the high. At
// step s (0..7) of the super-block it uses byte dword s, and its 8 operand
// values are, in order, columns 64g + 4s + {0, 2, 1, 3} (low nibbles) and
// 64g + 32 + 4s + {0, 2, 1, 3} (high): the order in which two masks of a
// dword place nibbles in the halves of fp16 pairs. xsplit_kernel writes x in
// the same order. A nibble pair becomes fp16 (1024 + q) by or-ing in the
// exponent bits, and one packed fp16 FMA (1024 + q)*sc - 1024*sc gives sc*q
// exactly (one rounding of an exactly representable result).
#include "quant_blocks.hpp"

#pragma clang fp contract(off)

namespace aero {

namespace {

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef uint32_t u4 __attribute__((ext_vector_type(4)));  // 16 bytes, kept in registers

constexpr int kParts = 3;          // fp16 parts of x
constexpr int kTokTile = 32;       // tokens a workgroup
constexpr int kChunkSteps = 4;     // 32-column steps a staged chunk
constexpr int kScaleMax = 15;      // scaled |x| < 2^15

__device__ __forceinline__ h2 as_h2(uint32_t u) { return __builtin_bit_cast(h2, u); }
// fp16 bits to fp32 with the hardware conversion (exact, subnormals included)
__device__ __forceinline__ float f16_lo(uint32_t u) { return (float)as_h2(u)[0]; }
__device__ __forceinline__ float f16_hi(uint32_t u) { return (float)as_h2(u)[1]; }
__device__ __forceinline__ uint32_t as_u32(h2 h) { return __builtin_bit_cast(uint32_t, h); }

// ------------------------------------------------------------ x prepass
// Workgroup t: e = exponent of the largest finite |x[t, :]| (frexp), the
// scale 2^(15-e) (1 for an all-zero token), xinv[t] = its inverse, and the
// sums of the scaled x over each 32-column sub-block. Tokens t >= n_tok (the
// padding to 32) get scale 1 and zero sums.
__global__ __launch_bounds__(256) void xscale_kernel(const float* __restrict__ x, int n_tok,
                                                      int n_cols, float* __restrict__ xsum,
                                                      float* __restrict__ xinv) {
    __shared__ float red[4];
    const int t = blockIdx.x;
    const int tid = threadIdx.x;
    const float* xr = x + (int64_t)t * n_cols;
    float amax = 0.f;
    if (t < n_tok) {
        for (int c = 4 * tid; c < n_cols; c += 1024) {
            const float4 v = *reinterpret_cast<const float4*>(xr + c);
            const float a[4] = {fabsf(v.x), fabsf(v.y), fabsf(v.z), fabsf(v.w)};
#pragma unroll
            for (int i = 0; i < 4; ++i) amax = a[i] <= 3.4028235e38f ? fmaxf(amax, a[i]) : amax;
        }
    }
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) amax = fmaxf(amax, __shfl_xor(amax, o));
    if ((tid & 63) == 0) red[tid >> 6] = amax;
    __syncthreads();
    amax = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    int e = 0;
    if (amax > 0.f) {
        frexpf(amax, &e);
        e = min(max(e, -111), 128);  // keeps 2^(15-e) and 2^(e-15) normal
    } else {
        e = kScaleMax;
    }
    const float scale = ldexpf(1.f, kScaleMax - e);
    if (tid == 0) xinv[t] = ldexpf(1.f, e - kScaleMax);
    const int n_g = n_cols >> 5;
    for (int g = tid; g < n_g; g += 256) {
        float s = 0.f;
        if (t < n_tok) {
#pragma unroll
            for (int q = 0; q < 8; ++q) {
                const float4 v = *reinterpret_cast<const float4*>(xr + 32 * g + 4 * q);
                s += v.x * scale;
                s += v.y * scale;
                s += v.z * scale;
                s += v.w * scale;
            }
        }
        xsum[(int64_t)t * n_g + g] = s;
    }
}

// Parts of one scaled value: hi = fp16(v), mid = fp16(v - hi), lo =
// fp16(v - hi - mid); both differences are exact in fp32. Non-finite values
// keep hi = fp16(v) and zero mid / lo.
__device__ __forceinline__ void split3(float v, _Float16& hi, _Float16& mid, _Float16& lo) {
    hi = (_Float16)v;
    const float r1 = v - (float)hi;
    mid = (_Float16)r1;
    const float r2 = r1 - (float)mid;
    lo = (_Float16)r2;
    if (!(fabsf(v) <= 3.4028235e38f)) mid = lo = (_Float16)0.f;
}

// xp[((mt*nK + K)*3 + p)*64 + lane] = 8 fp16 values of part p for token
// 16mt + lane%16, step K, lane group lane/16, in the operand order above.
// Grid (tok_pad/16, nK/4); wave w of a workgroup writes step 4*blockIdx.y + w.
__global__ __launch_bounds__(256) void xsplit_kernel(const float* __restrict__ x, int n_tok,
                                                      int n_cols, const float* __restrict__ xinv,
                                                      uint4* __restrict__ xp) {
    const int tid = threadIdx.x;
    const int l = tid & 63;
    const int K = 4 * blockIdx.y + (tid >> 6);
    const int nK = n_cols >> 5;
    const int mt = blockIdx.x;
    const int t = 16 * mt + (l & 15), g = l >> 4;
    float v[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    if (t < n_tok) {
        const float scale = 1.f / xinv[t];  // a power of two: exact
        const float* xr = x + (int64_t)t * n_cols + 256 * (K >> 3) + 64 * g + 4 * (K & 7);
        const float4 a = *reinterpret_cast<const float4*>(xr);
        const float4 b = *reinterpret_cast<const float4*>(xr + 32);
        v[0] = a.x * scale; v[1] = a.z * scale; v[2] = a.y * scale; v[3] = a.w * scale;
        v[4] = b.x * scale; v[5] = b.z * scale; v[6] = b.y * scale; v[7] = b.w * scale;
    }
    h8 parts[kParts];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        _Float16 hi, mid, lo;
        split3(v[i], hi, mid, lo);
        parts[0][i] = hi;
        parts[1][i] = mid;
        parts[2][i] = lo;
    }
    uint4* dst = xp + ((int64_t)mt * nK + K) * (kParts * 64) + l;
#pragma unroll
    for (int p = 0; p < kParts; ++p) dst[64 * p] = __builtin_bit_cast(uint4, parts[p]);
}

// ---------------------------------------------------------- the GEMM
struct SplitParams {
    const uint8_t* w;     // n_rows rows of rb bytes, 16-byte aligned
    const uint4* xp;      // x parts (xsplit_kernel)
    const float* xsum;    // [tok_pad][n_cols/32] sub-block sums of the scaled x
    const float* xinv;    // [tok_pad] inverse token scales
    float* y;             // [n_tok][n_rows]
    int64_t n_rows;
    int n_cols;
    int64_t rb;
    int n_tok;
};

// sc*q for the 4 fp16 pairs of one dword of quants (Q5_K: with the fifth
// bits of the matching qh dword, bits 2g / 2g+1 of each byte).
template <bool Q5>
__device__ __forceinline__ h8 weight_operand(uint32_t w, uint32_t h, int g, h2 s_lo, h2 b_lo,
                                             h2 s_hi, h2 b_hi) {
    constexpr uint32_t M = 0x000F000Fu, E = 0x64006400u;
    uint32_t p0 = (w & M) | E, p1 = ((w >> 8) & M) | E;
    uint32_t p2 = ((w >> 4) & M) | E, p3 = ((w >> 12) & M) | E;
    if (Q5) {
        const uint32_t h0 = h >> (2 * g), h1 = h >> (2 * g + 1);
        p0 |= (h0 & 0x00010001u) << 4;
        p1 |= ((h0 >> 8) & 0x00010001u) << 4;
        p2 |= (h1 & 0x00010001u) << 4;
        p3 |= ((h1 >> 8) & 0x00010001u) << 4;
    }
    const h2 a0 = __builtin_elementwise_fma(as_h2(p0), s_lo, b_lo);
    const h2 a1 = __builtin_elementwise_fma(as_h2(p1), s_lo, b_lo);
    const h2 a2 = __builtin_elementwise_fma(as_h2(p2), s_hi, b_hi);
    const h2 a3 = __builtin_elementwise_fma(as_h2(p3), s_hi, b_hi);
    return __builtin_bit_cast(h8, make_uint4(as_u32(a0), as_u32(a1), as_u32(a2), as_u32(a3)));
}

// kq_scale_min for a sub-block index that differs between lanes: both
// unpackings computed and selected, no branch (src/kernels.cpp:65-73).
__device__ __forceinline__ void kq_scale_min_lanes(uint32_t s0, uint32_t s1, uint32_t s2, int k,
                                                   uint32_t& sc, uint32_t& mn) {
    const uint32_t sh = 8u * (uint32_t)(k & 3);
    const uint32_t a0 = (s0 >> sh) & 0xFFu, a1 = (s1 >> sh) & 0xFFu, a2 = (s2 >> sh) & 0xFFu;
    sc = k < 4 ? (a0 & 63u) : ((a2 & 15u) | ((a0 >> 6) << 4));
    mn = k < 4 ? (a1 & 63u) : ((a2 >> 4) | ((a1 >> 6) << 4));
}

// The x parts and sub-block sums of one chunk on their way to LDS: thread
// tid stages uint4 tid + 256i of the chunk, i < 3 from the first token tile,
// i >= 3 from the second (each chunk of a token tile is 768 contiguous
// uint4 of xp), and float4 tid of the super-block's sums.
struct XStage {
    static constexpr int CSTEP = kChunkSteps * kParts * 64;
    u4 r[6];
    v4f s;
    const u4* b0;
    const u4* b1;
    const v4f* sb;
    int n_chunks;
    __device__ __forceinline__ void init(const uint4* xp, const float* xsum, int tt, int nK,
                                         int tid) {
        b0 = reinterpret_cast<const u4*>(xp) + (int64_t)(2 * tt) * nK * (kParts * 64) + tid;
        b1 = b0 + (int64_t)nK * (kParts * 64);
        sb = reinterpret_cast<const v4f*>(xsum) +
             ((int64_t)(kTokTile * tt + ((tid & 63) >> 1)) * nK) / 4 + (tid & 1);
        n_chunks = nK / kChunkSteps;
    }
    // chunk c, clamped: past the end the last chunk is read again, unused
    __device__ __forceinline__ void load(int c) {
        c = min(c, n_chunks - 1);
        const int64_t o = (int64_t)c * CSTEP;
#pragma unroll
        for (int i = 0; i < 3; ++i) {
            r[i] = b0[o + 256 * i];
            r[3 + i] = b1[o + 256 * i];
        }
        s = sb[2 * (c >> 1)];
    }
    __device__ __forceinline__ void store(u4* xs, v4f* ss, int tid) const {
#pragma unroll
        for (int i = 0; i < 6; ++i) xs[tid + 256 * i] = r[i];
        if (ss != nullptr && tid < 2 * kTokTile) ss[tid] = s;
    }
};

__device__ __forceinline__ uint32_t comp(const uint4& v, int i) {
    return i == 0 ? v.x : (i == 1 ? v.y : (i == 2 ? v.z : v.w));
}

// NT matrix tiles of 16 rows a wave; a workgroup covers 4 x 16NT rows.
template <int TYPE, int NT>
__global__ __launch_bounds__(256) void split_gemm_kernel(SplitParams p) {
    constexpr bool Q5 = TYPE == AERO_DTYPE_Q5_K;
    constexpr int BB = Q5 ? 176 : 144;          // bytes a super-block
    constexpr int QOFF = Q5 ? 48 : 16;          // quants within the block
    constexpr int kRowsWave = 16 * NT;
    constexpr int MT = kTokTile / 16;           // matrix tiles over tokens (2)
    constexpr int CHUNK = MT * XStage::CSTEP;   // uint4 a chunk (1536)
    static_assert(MT == 2 && CHUNK == 6 * 256, "staging split");
    __shared__ u4 xs[2][CHUNK];                 // 2 x 24 KB, by chunk parity
    __shared__ v4f ss[2][kTokTile * 2];         // sub-block sums, by super-block parity

    const int tid = threadIdx.x;
    const int l = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int r = l & 15, g = l >> 4;
    const int64_t row0 = (int64_t)blockIdx.x * (4 * kRowsWave) + wave * kRowsWave;
    const int tt = blockIdx.y;
    const int nK = p.n_cols >> 5, n_g = nK;
    const int n_chunks = nK / kChunkSteps, n_sb = n_chunks / 2;

    // rows past n_rows read the last row (their results are not stored)
    const uint8_t* wbase = p.w + row0 * p.rb;
    int woff[NT];
#pragma unroll
    for (int j = 0; j < NT; ++j)
        woff[j] = (int)((min(row0 + 16 * j + r, p.n_rows - 1) - row0) * p.rb);

    XStage xst;
    xst.init(p.xp, p.xsum, tt, nK, tid);

    uint4 q[NT], hq[NT], hd[NT];
    auto load_q = [&](int sb, int half, uint4 (&qq)[NT], uint4 (&hh)[NT]) {
        const uint8_t* b = wbase + (int64_t)min(sb, n_sb - 1) * BB;
#pragma unroll
        for (int j = 0; j < NT; ++j) {
            qq[j] = ld128(b + woff[j] + QOFF + 32 * g + 16 * half);
            if (Q5) hh[j] = ld128(b + woff[j] + 16 + 16 * half);
        }
    };
    auto load_hd = [&](int sb, uint4 (&dd)[NT]) {
        const uint8_t* b = wbase + (int64_t)min(sb, n_sb - 1) * BB;
#pragma unroll
        for (int j = 0; j < NT; ++j) dd[j] = ld128(b + woff[j]);
    };

    v4f acc[MT][NT], part[MT][NT];
#pragma unroll
    for (int m = 0; m < MT; ++m)
#pragma unroll
        for (int j = 0; j < NT; ++j) acc[m][j] = v4f{0.f, 0.f, 0.f, 0.f};

    h2 s_lo[NT], b_lo[NT], s_hi[NT], b_hi[NT];
    // the 4 steps of one chunk from LDS buffer xb with quants qq
    auto run_steps = [&](const u4* xb, const uint4 (&qq)[NT], const uint4 (&hh)[NT]) {
#pragma unroll
        for (int s = 0; s < kChunkSteps; ++s) {
            h8 B[NT], A[MT][kParts];
#pragma unroll
            for (int j = 0; j < NT; ++j)
                B[j] = weight_operand<Q5>(comp(qq[j], s), Q5 ? comp(hh[j], s) : 0u, g, s_lo[j],
                                          b_lo[j], s_hi[j], b_hi[j]);
#pragma unroll
            for (int m = 0; m < MT; ++m)
#pragma unroll
                for (int pp = 0; pp < kParts; ++pp)
                    A[m][pp] = __builtin_bit_cast(
                        h8, xb[((m * kChunkSteps + s) * kParts + pp) * 64 + l]);
            // small parts first into each tile's super-block sum
#pragma unroll
            for (int pp = kParts - 1; pp >= 0; --pp)
#pragma unroll
                for (int m = 0; m < MT; ++m)
#pragma unroll
                    for (int j = 0; j < NT; ++j)
                        part[m][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(A[m][pp], B[j],
                                                                            part[m][j], 0, 0, 0);
            // keeps the next step's operand reads from being hoisted here
            // (4 steps of operands at once exceed the register file)
            __builtin_amdgcn_sched_barrier(0);
        }
    };

    // prologue: chunk 0 (super-block 0, first half) staged, chunk 1 in flight
    xst.load(0);
    load_q(0, 0, q, hq);
    load_hd(0, hd);
    xst.store(xs[0], ss[0], tid);
    xst.load(1);
    __syncthreads();

    for (int sb = 0; sb < n_sb; ++sb) {
        // ---- first half: chunk 2sb in xs[0]
        uint4 qn[NT], hqn[NT], hdn[NT];
        load_q(sb, 1, qn, hqn);
#pragma unroll
        for (int j = 0; j < NT; ++j) {
            uint32_t sc0, sc1, mn;
            kq_scale_min_lanes(hd[j].y, hd[j].z, hd[j].w, 2 * g, sc0, mn);
            kq_scale_min_lanes(hd[j].y, hd[j].z, hd[j].w, 2 * g + 1, sc1, mn);
            const _Float16 f0 = (_Float16)(float)sc0, f1 = (_Float16)(float)sc1;
            const _Float16 n0 = (_Float16)(-1024.f * (float)sc0);
            const _Float16 n1 = (_Float16)(-1024.f * (float)sc1);
            s_lo[j] = h2{f0, f0};
            s_hi[j] = h2{f1, f1};
            b_lo[j] = h2{n0, n0};
            b_hi[j] = h2{n1, n1};
        }
#pragma unroll
        for (int m = 0; m < MT; ++m)
#pragma unroll
            for (int j = 0; j < NT; ++j) part[m][j] = v4f{0.f, 0.f, 0.f, 0.f};
        run_steps(xs[0], q, hq);
        xst.store(xs[1], nullptr, tid);   // chunk 2sb+1 (loaded a chunk ago)
        xst.load(2 * sb + 2);
        __syncthreads();

        // ---- second half: chunk 2sb+1 in xs[1]
        load_q(sb + 1, 0, q, hq);   // next super-block (clamped)
        load_hd(sb + 1, hdn);
        run_steps(xs[1], qn, hqn);
        // acc += d * part - dmin * sum_k m_k S_k: the row's d, dmin and m are
        // lane-local; a token's 8 sums are read once for all row tiles
        const v4f* sp = ss[sb & 1];
        float d[NT], dm[NT], mf[NT][8];
#pragma unroll
        for (int j = 0; j < NT; ++j) {
            d[j] = f16_lo(hd[j].x);
            dm[j] = f16_hi(hd[j].x);
#pragma unroll
            for (int k = 0; k < 8; ++k) {
                uint32_t sc, mn;
                kq_scale_min(hd[j].y, hd[j].z, hd[j].w, k, sc, mn);
                mf[j][k] = (float)mn;
            }
        }
#pragma unroll
        for (int m = 0; m < MT; ++m)
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                const int tk = 16 * m + 4 * g + v;
                const v4f s0 = sp[2 * tk], s1 = sp[2 * tk + 1];
#pragma unroll
                for (int j = 0; j < NT; ++j) {
                    float ms = mf[j][0] * s0.x;
                    ms = fmaf(mf[j][1], s0.y, ms);
                    ms = fmaf(mf[j][2], s0.z, ms);
                    ms = fmaf(mf[j][3], s0.w, ms);
                    ms = fmaf(mf[j][4], s1.x, ms);
                    ms = fmaf(mf[j][5], s1.y, ms);
                    ms = fmaf(mf[j][6], s1.z, ms);
                    ms = fmaf(mf[j][7], s1.w, ms);
                    const float a = fmaf(d[j], part[m][j][v], acc[m][j][v]);
                    acc[m][j][v] = fmaf(-dm[j], ms, a);
                }
                __builtin_amdgcn_sched_barrier(0);  // one token's sums at a time
            }
        xst.store(xs[0], ss[(sb + 1) & 1], tid);  // chunk 2sb+2: the next super-block
        xst.load(2 * sb + 3);
#pragma unroll
        for (int j = 0; j < NT; ++j) hd[j] = hdn[j];
        __syncthreads();
    }

    // acc[m][j][v]: token 32tt + 16m + 4g + v, row row0 + 16j + r
#pragma unroll
    for (int m = 0; m < MT; ++m)
#pragma unroll
        for (int v = 0; v < 4; ++v) {
            const int tok = kTokTile * tt + 16 * m + 4 * g + v;
            if (tok >= p.n_tok) continue;
            const float inv = p.xinv[tok];
            float* yp = p.y + (int64_t)tok * p.n_rows;
#pragma unroll
            for (int j = 0; j < NT; ++j) {
                const int64_t row = row0 + 16 * j + r;
                if (row < p.n_rows) yp[row] = acc[m][j][v] * inv;
            }
        }
}

inline int64_t align256(int64_t b) { return (b + 255) & ~(int64_t)255; }

}  // namespace

// Workspace bytes of the split-x GEMM for n_tok tokens of n_cols (0 when the
// type or shape has no split path): the x parts, the sub-block sums and the
// token scales.
int64_t split_gemm_workspace(int dtype, int64_t n_cols, int64_t n_tok) {
    if ((dtype != AERO_DTYPE_Q4_K && dtype != AERO_DTYPE_Q5_K) || n_cols <= 0 ||
        n_cols % 256 != 0 || n_cols / 128 > 65535 || n_tok <= 0)
        return 0;
    const int64_t tp = (n_tok + kTokTile - 1) / kTokTile * kTokTile;
    return align256(tp * n_cols * 2 * kParts) + align256(tp * (n_cols / 32) * 4) +
           align256(tp * 4);
}

// Called by the matmul entry after its argument checks; false (without an
// error) when this path does not apply, so the caller takes another GEMM.
bool split_gemm_dev(int dtype, const uint8_t* w, const float* x, float* y, int64_t n_rows,
                    int64_t n_cols, int64_t rb, int64_t n_tok, void* ws, int64_t ws_bytes,
                    hipStream_t s, bool* ran) {
    *ran = false;
    const int64_t need = split_gemm_workspace(dtype, n_cols, n_tok);
    const int64_t tp = (n_tok + kTokTile - 1) / kTokTile * kTokTile;
    // rows a wave: 64 while that leaves >= 512 workgroups, else 32
    // (measured on MI355X)
    const int64_t tok_tiles = tp / kTokTile;
    int nt = (n_rows + 255) / 256 * tok_tiles >= 512 ? 4 : 2;
    nt = tune("gemm16_nt", nt) == 4 ? 4 : 2;
    const int64_t row_tiles = (n_rows + 64 * nt - 1) / (64 * nt);
    if (need == 0 || ws == nullptr || ws_bytes < need || !aligned16(w) || rb % 16 != 0 ||
        !aligned16(ws) || tok_tiles > 65535 || row_tiles > 0x7fffffff || tp > 0x7fffffff ||
        !tune("gemm16", 1))
        return true;
    uint8_t* base = static_cast<uint8_t*>(ws);
    uint4* xp = reinterpret_cast<uint4*>(base);
    float* xsum = reinterpret_cast<float*>(base + align256(tp * n_cols * 2 * kParts));
    float* xinv = reinterpret_cast<float*>(base + align256(tp * n_cols * 2 * kParts) +
                                           align256(tp * (n_cols / 32) * 4));
    if (!launch("xscale_kernel", xscale_kernel, dim3((unsigned)tp), dim3(256), 0, s, x,
                (int)n_tok, (int)n_cols, xsum, xinv))
        return false;
    if (!launch("xsplit_kernel", xsplit_kernel, dim3((unsigned)(tp / 16), (unsigned)(n_cols / 128)),
                dim3(256), 0, s, x, (int)n_tok, (int)n_cols, (const float*)xinv, xp))
        return false;
    SplitParams p{w, xp, xsum, xinv, y, n_rows, (int)n_cols, rb, (int)n_tok};
    const bool q5 = dtype == AERO_DTYPE_Q5_K;
    auto k = nt == 4 ? (q5 ? split_gemm_kernel<AERO_DTYPE_Q5_K, 4> : split_gemm_kernel<AERO_DTYPE_Q4_K, 4>)
                     : (q5 ? split_gemm_kernel<AERO_DTYPE_Q5_K, 2> : split_gemm_kernel<AERO_DTYPE_Q4_K, 2>);
    if (!launch("split_gemm_kernel", k, dim3((unsigned)row_tiles, (unsigned)tok_tiles), dim3(256),
                0, s, p))
        return false;
    *ran = true;
    return true;
}

}  // namespace aero
