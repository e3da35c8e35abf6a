// Quantised GEMM on the fp16 matrix cores with x split into fp16 parts
// (prefill): y[t, r] = sum_c W[r, c] * x[t, c], W in Q4_K / Q5_K blocks, x and
// y fp32 — the reference's matmul (src/kernels.cpp:520-538) over its block
// dots (:78-250), at fp32-grade accuracy on the fp16 matrix rate.
//
// Arithmetic. A Q4_K / Q5_K value is (d*sc)*q - (dmin*m) with per-256-value
// fp16 scales d, dmin and per-32-value 6-bit sc, m (src/kernels.cpp:337-404).
// sc*q <= 63*31 is an integer below 2048, exact in fp16, so per super-block
//   sum_c w_c x_c = d * sum_c (sc*q)_c x_c  -  dmin * sum_g m_g * S_g
// with S_g the sum of x over sub-block g. Each token's x is scaled, per
// super-block, by a power of two 2^(15-e) (e the exponent of the block's
// largest finite |x|, so the scaled values lie below 2^15) and split into
// two fp16 parts hi + lo: 22 significant bits of each value (relative error
// at most 2^-22; fp32 holds 24), and values below 2^-3 in the scaled units
// to 2^-25 absolute (2^-39 of the block's largest). A build with
// -DAERO_SPLIT_PARTS=3 adds a third part (hi + mid + lo): every value of at
// least 2^-16 of the block's largest is then exact, for half again the
// matrix work. Products of fp16 integers and fp16 parts are exact; the
// matrix cores add them in fp32, and each super-block's sum is scaled back
// (by 2^(e-15)) as it is added to the row's fp32 total. The reference
// dequantises each value to fp32 and sums the rounded products serially; on
// the layer shapes both differ from the exact product by 2-5e-7 of the
// output's scale (measured), the reference's own fp32 rounding level.
//
// Kernels:
//   xsplit_kernel   one workgroup a 16-token tile and super-block: the scale,
//                   the fp16 parts of x in matrix-operand order (padded to
//                   32 tokens with zeros) and the sub-block sums S of the
//                   scaled x (fp32);
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
// Operand order. At step s (0..3) of half h (0..1) of a super-block, lane
// group g = l/16 of a row uses quant dword s of the 16 bytes 64h + 16g ..
// +15 of the block's qs (one contiguous 64-byte run a row and half): the
// bytes of sub-block pair P = 2h + g/2 (sub-block 2P in the low nibbles,
// 2P+1 in the high) at value offset 16(g%2) + 4s. Its 8 operand values are,
// in order, columns 64P + 16(g%2) + 4s + {0, 2, 1, 3} (low nibbles) and the
// same + 32 (high): the order in which two masks of a dword place nibbles in
// the halves of fp16 pairs. xsplit_kernel writes x in the same order. A
// nibble pair becomes fp16 (1024 + q) by or-ing in the exponent bits, and
// one packed fp16 FMA (1024 + q)*sc - 1024*sc gives sc*q exactly (one
// rounding of an exactly representable result).
#include <mutex>

#include "act_ops.hpp"
#include "quant_blocks.hpp"

#pragma clang fp contract(off)

namespace aero {

// block sizes of the ggml types (quant.hip)
int64_t dtype_block_bytes(int t);
int64_t dtype_block_values(int t);

namespace {

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef uint32_t u4 __attribute__((ext_vector_type(4)));  // 16 bytes, kept in registers

#ifndef AERO_SPLIT_PARTS
#define AERO_SPLIT_PARTS 2
#endif
constexpr int kParts = AERO_SPLIT_PARTS;  // fp16 parts of x (2 or 3)
static_assert(kParts == 2 || kParts == 3, "x is split into two or three fp16 parts");
constexpr int kTokTile = 32;       // tokens a workgroup
constexpr int kChunkSteps = 4;     // 32-column steps a staged chunk
constexpr int kScaleMax = 15;      // scaled |x| < 2^15

__device__ __forceinline__ h2 as_h2(uint32_t u) { return __builtin_bit_cast(h2, u); }
// fp16 bits to fp32 with the hardware conversion (exact, subnormals included)
__device__ __forceinline__ float f16_lo(uint32_t u) { return (float)as_h2(u)[0]; }
__device__ __forceinline__ float f16_hi(uint32_t u) { return (float)as_h2(u)[1]; }
__device__ __forceinline__ uint32_t as_u32(h2 h) { return __builtin_bit_cast(uint32_t, h); }

// ------------------------------------------------------------ x prepass
// Parts of one scaled value: hi = fp16(v), mid = fp16(v - hi), lo =
// fp16(v - hi - mid); both differences are exact in fp32. Non-finite values
// keep hi = fp16(v) and zero mid / lo. The two-part split keeps hi and mid.
__device__ __forceinline__ void split3(float v, _Float16& hi, _Float16& mid, _Float16& lo) {
    hi = (_Float16)v;
    const float r1 = v - (float)hi;
    mid = (_Float16)r1;
    const float r2 = r1 - (float)mid;
    lo = (_Float16)r2;
    if (!(fabsf(v) <= 3.4028235e38f)) mid = lo = (_Float16)0.f;
}

// One workgroup a (16-token tile mt, super-block sb); grid (tok_pad/16,
// n_cols/256). For token t of the tile: e = exponent of the largest finite
// |x| of the super-block (frexp), scale 2^(15-e) (1 when all are zero, and
// for the padding tokens t >= n_tok), xinv[t][sb] = 2^(e-15);
// xp[((mt*nK + K)*kParts + p)*64 + lane] = 8 fp16 values of part p of the scaled x
// of token 16mt + lane%16 at step K = 8sb + 4h + s, lane group lane/16, in
// the operand order above; xsum[t][8sb + k] = the sum of the scaled x over
// sub-block k (fp32, in column order). x is read coalesced into LDS and
// read back in operand order.
//
// Folded steps of the model loop (the reference runs them as separate
// passes before its matmul, src/model.cpp:244-245,279-282):
//   RESID: x = x + d, and the sum is stored to x_out (the residual stream);
//   EMB:   x = the embedding rows of the token ids (a ggml type EMB, times
//          emb_scale when that is > 0, src/model.cpp:297-316), stored to
//          x_out; dequantised as the gather does (bit for bit), an id
//          outside the vocabulary giving a zero row;
//   NORM:  ssq[t][sb] = the sum of x^2 over the super-block, and x is
//          multiplied by the norm weight w (or 1 + w) before the split. The
//          GEMM multiplies each token's sums by 1/sqrtf(sum_sb ssq/n + eps),
//          so y = W (x*inv*w) without the normalised x ever reaching HBM.
struct XsplitArgs {
    const float* x;
    const float* d;       // RESID
    float* x_out;         // RESID
    const float* w;       // NORM (null: ones)
    float* ssq;           // NORM: [tok_pad][n_cols/256]
    int unit_offset;      // NORM: w applied as 1 + w
    int n_tok;
    int n_cols;
    uint4* xp;
    float* xsum;
    float* xinv;
    const float* z;       // NORM, gated (src/ssm.cpp:322-340): x * w[c % w_len] * silu(z)
    int w_len;
    int order;            // operand order: 0 Q4_K / Q5_K, 1 Q8_0, 2 Q6_K, 3 IQ4_XS
    const uint8_t* emb;   // EMB: the table, rows of emb_rb bytes
    const int32_t* ids;   // EMB: [n_tok]
    int64_t vocab;
    int64_t emb_rb;
    float emb_scale;
};

template <bool NORM, bool RESID, int EMB>
__global__ __launch_bounds__(256) void xsplit_kernel(XsplitArgs a) {
    constexpr int RowF = 256 + 4;
    __shared__ float xl[16 * RowF];
    const int tid = threadIdx.x;
    const int mt = blockIdx.x, sb = blockIdx.y;
    const int n_cols = a.n_cols;
    const int nK = n_cols >> 5, n_sb = n_cols >> 8;
    uint4* __restrict__ xp = a.xp;
    float* __restrict__ xsum = a.xsum;
    // token tk = tid / 16 of the tile, columns 16 (tid % 16) .. +15
    const int tk = tid >> 4, cq = tid & 15;
    const int t = 16 * mt + tk;
    float4 v[4];
    float amax = 0.f, ss = 0.f;
#pragma unroll
    for (int i = 0; i < 4; ++i) v[i] = make_float4(0.f, 0.f, 0.f, 0.f);
    if (t < a.n_tok) {
        const int64_t off = (int64_t)t * n_cols + 256 * sb + 16 * cq;
        if constexpr (EMB != 0) {
            // values 16 cq .. +15 of the row's super-block sb: the gather's
            // lanes 4 cq .. 4 cq + 3 of that 256-value step
            using Q = QT<EMB>;
            const int64_t id = a.ids[t];
            if (id >= 0 && id < a.vocab) {
                const uint8_t* rowp = a.emb + id * a.emb_rb;
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int vl = 4 * cq + i;
                    typename Q::Raw raw;
                    load_raw(rowp + ((256 * sb + 4 * vl) / Q::BV) * Q::BB, vl, raw);
                    v[i] = decode(raw, vl);
                    if (a.emb_scale > 0.0f) {
                        v[i].x = v[i].x * a.emb_scale; v[i].y = v[i].y * a.emb_scale;
                        v[i].z = v[i].z * a.emb_scale; v[i].w = v[i].w * a.emb_scale;
                    }
                }
            }
            // (stored at once: measured faster here than after the norm's
            // weight loads)
#pragma unroll
            for (int i = 0; i < 4; ++i)
                __builtin_nontemporal_store(v4f{v[i].x, v[i].y, v[i].z, v[i].w},
                                            reinterpret_cast<v4f*>(a.x_out + off + 4 * i));
        } else {
            const float* xr = a.x + off;
#pragma unroll
            for (int i = 0; i < 4; ++i) v[i] = ld_stream(xr + 4 * i);
        }
        // the residual, the norm's weights and the gate are loaded before x + d
        // is stored: stores count in the same vector-memory counter as loads,
        // so a load issued after a store waits for that store too (the
        // residual pre-pass at 512 x 4096: 16.7 -> 10.5 us on MI355X)
        float4 dv[4], w4[4], z4[4];
        if constexpr (RESID) {
            const float* dr = a.d + off;
#pragma unroll
            for (int i = 0; i < 4; ++i) dv[i] = ld_stream(dr + 4 * i);
        }
        const int wc = 256 * sb + 16 * cq;
        const bool has_w = NORM && a.w != nullptr, has_z = NORM && a.z != nullptr;
        if (has_w) {
            const float* wr = a.w + (a.z != nullptr ? wc % a.w_len : wc);
#pragma unroll
            for (int i = 0; i < 4; ++i) w4[i] = *reinterpret_cast<const float4*>(wr + 4 * i);
        }
        if (has_z) {
            const float* zr = a.z + off;
#pragma unroll
            for (int i = 0; i < 4; ++i) z4[i] = ld_stream(zr + 4 * i);
        }
        __builtin_amdgcn_sched_barrier(0);
        if constexpr (RESID) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                v[i].x = v[i].x + dv[i].x; v[i].y = v[i].y + dv[i].y;
                v[i].z = v[i].z + dv[i].z; v[i].w = v[i].w + dv[i].w;
                __builtin_nontemporal_store(v4f{v[i].x, v[i].y, v[i].z, v[i].w},
                                            reinterpret_cast<v4f*>(a.x_out + off + 4 * i));
            }
        }
        if constexpr (NORM) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                ss += v[i].x * v[i].x;
                ss += v[i].y * v[i].y;
                ss += v[i].z * v[i].z;
                ss += v[i].w * v[i].w;
            }
            if (has_w) {
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    float4 wv = w4[i];
                    if (a.unit_offset) {
                        wv.x = 1.0f + wv.x; wv.y = 1.0f + wv.y;
                        wv.z = 1.0f + wv.z; wv.w = 1.0f + wv.w;
                    }
                    v[i].x = v[i].x * wv.x; v[i].y = v[i].y * wv.y;
                    v[i].z = v[i].z * wv.z; v[i].w = v[i].w * wv.w;
                }
            }
            if (has_z) {   // gated: silu of the gate
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    v[i].x = v[i].x * silu_fast(z4[i].x);
                    v[i].y = v[i].y * silu_fast(z4[i].y);
                    v[i].z = v[i].z * silu_fast(z4[i].z);
                    v[i].w = v[i].w * silu_fast(z4[i].w);
                }
            }
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const float q[4] = {fabsf(v[i].x), fabsf(v[i].y), fabsf(v[i].z), fabsf(v[i].w)};
#pragma unroll
            for (int k = 0; k < 4; ++k) amax = q[k] <= 3.4028235e38f ? fmaxf(amax, q[k]) : amax;
        }
    }
#pragma unroll
    for (int o = 1; o < 16; o <<= 1) amax = fmaxf(amax, __shfl_xor(amax, o));
    if constexpr (NORM) {
        ss = group_sum<16>(ss);
        if (cq == 0) a.ssq[(int64_t)t * n_sb + sb] = ss;
    }
    int e = kScaleMax;
    if (amax > 0.f) {
        frexpf(amax, &e);
        e = min(max(e, -111), 128);  // keeps 2^(15-e) and 2^(e-15) normal
    }
    const float scale = ldexpf(1.f, kScaleMax - e);
    if (cq == 0) a.xinv[(int64_t)t * n_sb + sb] = ldexpf(1.f, e - kScaleMax);
    float* row = xl + tk * RowF + 16 * cq;
#pragma unroll
    for (int i = 0; i < 4; ++i)
        *reinterpret_cast<float4*>(row + 4 * i) =
            make_float4(v[i].x * scale, v[i].y * scale, v[i].z * scale, v[i].w * scale);
    __syncthreads();

    // operand (step 8sb + s8, lane l): thread tid makes s8 = tid/64 and tid/64 + 4
    const int l = tid & 63, lt = l & 15, g = l >> 4;
#pragma unroll
    for (int rep = 0; rep < 2; ++rep) {
        const int s8 = (tid >> 6) + 4 * rep;
        float w[8];
        if (a.order == 1) {
            // Q8_0 block s8: values (2 + 8s + i) % 32 of even blocks, 8s + i of
            // odd, s = 2(g&1) + g/2
            const float* xr = xl + lt * RowF + 32 * s8;
            const int sg = ((g & 1) << 1) | (g >> 1);
            const int o = (s8 & 1) ? 8 * sg : 2 + 8 * sg;
#pragma unroll
            for (int i = 0; i < 8; ++i) w[i] = xr[(o + i) & 31];
        } else if (a.order == 3) {
            // IQ4_XS sub-block s8: values 4k + i and 16 + 4k + i, k = 3 - g
            const float* xr = xl + lt * RowF + 32 * s8 + 4 * (3 - g);
            const float4 va = *reinterpret_cast<const float4*>(xr);
            const float4 vb = *reinterpret_cast<const float4*>(xr + 16);
            w[0] = va.x; w[1] = va.y; w[2] = va.z; w[3] = va.w;
            w[4] = vb.x; w[5] = vb.y; w[6] = vb.z; w[7] = vb.w;
        } else if (a.order == 2) {
            // Q6_K quarter s8 % 4 of half s8 / 4: values 8t .. 8t+7, t = (1, 3, 0, 2)[g]
            const int t6 = (0x2031 >> (4 * g)) & 3;
            const float* xr = xl + lt * RowF + 32 * s8 + 8 * t6;
            const float4 va = *reinterpret_cast<const float4*>(xr);
            const float4 vb = *reinterpret_cast<const float4*>(xr + 4);
            w[0] = va.x; w[1] = va.y; w[2] = va.z; w[3] = va.w;
            w[4] = vb.x; w[5] = vb.y; w[6] = vb.z; w[7] = vb.w;
        } else {
            const int c0 = 128 * (s8 >> 2) + 64 * (g >> 1) + 16 * (g & 1) + 4 * (s8 & 3);
            const float* xr = xl + lt * RowF + c0;
            const float4 va = *reinterpret_cast<const float4*>(xr);
            const float4 vb = *reinterpret_cast<const float4*>(xr + 32);
            w[0] = va.x; w[1] = va.z; w[2] = va.y; w[3] = va.w;
            w[4] = vb.x; w[5] = vb.z; w[6] = vb.y; w[7] = vb.w;
        }
        h8 parts[kParts];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            _Float16 hi, mid, lo;
            split3(w[i], hi, mid, lo);
            parts[0][i] = hi;
            parts[1][i] = mid;
            if constexpr (kParts == 3) parts[2][i] = lo;
        }
        uint4* dst = xp + ((int64_t)mt * nK + 8 * sb + s8) * (kParts * 64) + l;
#pragma unroll
        for (int p = 0; p < kParts; ++p) dst[64 * p] = __builtin_bit_cast(uint4, parts[p]);
    }
    // sub-block sums: thread tid < 128 sums sub-block tid % 8 of token tid / 8
    if (tid < 128) {
        const int st = tid >> 3, k = tid & 7;
        const float* xr = xl + st * RowF + 32 * k;
        float sum = 0.f;
#pragma unroll
        for (int i = 0; i < 32; i += 4) {
            const float4 q = *reinterpret_cast<const float4*>(xr + i);
            sum += q.x;
            sum += q.y;
            sum += q.z;
            sum += q.w;
        }
        xsum[(int64_t)(16 * mt + st) * nK + 8 * sb + k] = sum;
    }
}

// ---------------------------------------------------------- the GEMM
// Up to kMaxMats matrices of one type and width sharing x (q, k, v) run in
// one launch: the row tiles of matrix m are workgroups tile0[m] ..
// tile0[m+1]-1 along x, so small matrices (k, v) fill the GPU together with
// the large one.
constexpr int kMaxMats = 4;

struct SplitParams {
    const uint8_t* w[kMaxMats];   // n_rows[m] rows of rb bytes, 16-byte aligned
    float* y[kMaxMats];           // [n_tok][n_rows[m]]
    int64_t n_rows[kMaxMats];
    int tile0[kMaxMats + 1];      // first row tile of each matrix; tile0[n_mat] = all
    int n_mat;
    const uint4* xp;      // x parts (xsplit_kernel)
    const float* xsum;    // [tok_pad][n_cols/32] sub-block sums of the scaled x
    const float* xinv;    // [tok_pad][n_cols/256] inverse scales a token and super-block
    int n_cols;
    int64_t rb;
    int n_tok;
    const uint8_t* w2;    // gate/up form: the up matrix (w[0] is the gate)
    const float* ssq;     // folded norm: [tok_pad][n_cols/256] sums of x^2, else null
    float eps;
    // split over columns (ksplit > 1): workgroup z of the grid's third
    // dimension takes super-blocks [z, z+1) * n_sb/ksplit and writes its raw
    // sums to part[z][token][roff[m] + row] (gate/up: gate rows, then up
    // rows), which split_reduce_kernel adds up
    int ksplit;
    float* part;
    int64_t roff[kMaxMats];
    int64_t r_all;        // partial rows a token
    // per-head RMSNorm and RoPE on the outputs of matrices 0 .. rope_mats-1
    // (heads of rope_D rows, whole heads a workgroup), in the epilogue
    int rope_mats;
    int rope_D;
    int rope_rot;         // rotated channels
    int rope_mode;        // AERO_ROPE_NEOX / AERO_ROPE_INTERLEAVED
    const int32_t* pos;   // [n_tok]
    const float* rinv;    // [rope_rot / 2] inverse frequencies
    const float* qk_w[2]; // per-head norm weights of matrices 0 and 1, or null
    float qk_eps;
    int qk_flags;
};

// Epilogue forms: y = acc (kEpiPlain), or the gate/up form: out =
// act(gate) * up with act an AERO_ACT_* kind (src/tensor.cpp:104-125).
constexpr int kEpiPlain = -1;

// sc*q for the 4 fp16 pairs of one dword of quants of sub-block pair P
// (Q5_K: with the fifth bits of the matching qh dword, bits 2P / 2P+1), in
// the pair order (b0, b2), (b1, b3) of the dword's bytes b0..b3, low nibbles
// then high. Q4_K: the low nibbles of b0 and b2 sit at bits 0-3 and 16-19,
// so or-ing in 0x6400 makes fp16 1024 + q; the high nibbles sit at bits 4-7
// and 20-23, mantissa bits worth 1 under the exponent of 64, so or-ing in
// 0x5400 makes 64 + q (b1, b3 the same after a shift by 8): one and-or a
// pair. Q5_K: the nibbles with their fifth bit placed by byte permutes as
// (b0, 0x64, b2, 0x64) and (b1, 0x64, b3, 0x64), fp16 pairs 1024 + q.
// s_lo / s_hi: packed (sc, sc) of sub-blocks 2P / 2P+1; b_lo: -1024 sc,
// b_hi: -64 sc (Q4_K) or -1024 sc (Q5_K). One packed fp16 FMA a pair gives
// sc*q exactly (one rounding of an exactly representable result).
// e_lo / e_hi: 0x64006400 / 0x54005400 held in VGPRs (one and-or a pair:
// the mask is its one scalar operand).
template <bool Q5>
__device__ __forceinline__ h8 weight_operand(uint32_t w, uint32_t h, int P, h2 s_lo, h2 b_lo,
                                             h2 s_hi, h2 b_hi, uint32_t e_lo, uint32_t e_hi) {
    if constexpr (!Q5) {
        const uint32_t w8 = w >> 8;
        const h2 a0 = __builtin_elementwise_fma(as_h2((w & 0x000F000Fu) | e_lo), s_lo, b_lo);
        const h2 a1 = __builtin_elementwise_fma(as_h2((w8 & 0x000F000Fu) | e_lo), s_lo, b_lo);
        const h2 a2 = __builtin_elementwise_fma(as_h2((w & 0x00F000F0u) | e_hi), s_hi, b_hi);
        const h2 a3 = __builtin_elementwise_fma(as_h2((w8 & 0x00F000F0u) | e_hi), s_hi, b_hi);
        return __builtin_bit_cast(h8, make_uint4(as_u32(a0), as_u32(a1), as_u32(a2), as_u32(a3)));
    }
    constexpr uint32_t E = 0x64646464u, EVEN = 0x04020400u, ODD = 0x04030401u;
    uint32_t lo = w & 0x0F0F0F0Fu, hi = (w >> 4) & 0x0F0F0F0Fu;
    if (Q5) {
        lo |= ((h >> (2 * P)) << 4) & 0x10101010u;
        hi |= ((h >> (2 * P + 1)) << 4) & 0x10101010u;
    }
    const h2 a0 = __builtin_elementwise_fma(as_h2(__builtin_amdgcn_perm(E, lo, EVEN)), s_lo, b_lo);
    const h2 a1 = __builtin_elementwise_fma(as_h2(__builtin_amdgcn_perm(E, lo, ODD)), s_lo, b_lo);
    const h2 a2 = __builtin_elementwise_fma(as_h2(__builtin_amdgcn_perm(E, hi, EVEN)), s_hi, b_hi);
    const h2 a3 = __builtin_elementwise_fma(as_h2(__builtin_amdgcn_perm(E, hi, ODD)), s_hi, b_hi);
    return __builtin_bit_cast(h8, make_uint4(as_u32(a0), as_u32(a1), as_u32(a2), as_u32(a3)));
}

// The two sub-block scales of pair P = 2h + G of a K-quant header as packed
// fp16 (sc_2P, sc_2P+1), for G = 0 / 1 and half h = 0 / 1 (sub-blocks 2G,
// 2G+1 and 4+2G, 5+2G; src/kernels.cpp:65-73): the 6-bit values unpacked two
// bytes at a time and turned into fp16 as 1024 + sc - 1024 (exact).
__device__ __forceinline__ h2 kq_scale_pair(uint32_t s0, uint32_t s2, int G, int h) {
    const uint32_t u0 = s0 >> (16 * G);
    const uint32_t sc = h == 0 ? (u0 & 0x3F3Fu)
                               : (((s2 >> (16 * G)) & 0x0F0Fu) | ((u0 >> 2) & 0x3030u));
    const h2 v = as_h2(__builtin_amdgcn_perm(0x64646464u, sc, 0x04010400u));
    return v + h2{(_Float16)-1024.f, (_Float16)-1024.f};
}

// The mins m_g and m_{g+4} of a K-quant header for sub-blocks g < 4 and g + 4
// (src/kernels.cpp:65-73).
__device__ __forceinline__ void kq_min_pair(uint32_t s1, uint32_t s2, int g, uint32_t& m0,
                                            uint32_t& m1) {
    const uint32_t b1 = (s1 >> (8 * g)) & 0xFFu, b2 = (s2 >> (8 * g)) & 0xFFu;
    m0 = b1 & 63u;
    m1 = (b2 >> 4) | ((b1 >> 6) << 4);
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

// The x parts, sub-block sums and inverse scales of one chunk of MT
// 16-token tiles (TT tokens) on their way to LDS: thread tid stages uint4
// tid + 256i of the chunk, kParts of them from each tile (each chunk of a
// token tile is 256 * kParts contiguous uint4 of xp); threads < 2TT float4
// tid of the super-block's sums, threads 2TT .. 3TT-1 the inverse scale of
// token tid - 2TT.
template <int MT>
struct XStage {
    static constexpr int TT = 16 * MT;
    static constexpr int CSTEP = kChunkSteps * kParts * 64;   // uint4 a tile's chunk
    static_assert(CSTEP == 256 * kParts && 3 * TT <= 256, "staging split");
    u4 r[MT * kParts];
    v4f s;
    float iv;
    const u4* b;          // tile 0; tile m at + m * tstride
    int64_t tstride;
    const v4f* sb;
    const float* ib;
    int n_chunks;
    __device__ __forceinline__ void init(const uint4* xp, const float* xsum, const float* xinv,
                                         int tt, int nK, int tid) {
        tstride = (int64_t)nK * (kParts * 64);
        b = reinterpret_cast<const u4*>(xp) + (int64_t)(MT * tt) * tstride + tid;
        sb = reinterpret_cast<const v4f*>(xsum) +
             ((int64_t)(TT * tt + ((tid & (2 * TT - 1)) >> 1)) * nK) / 4 + (tid & 1);
        ib = xinv + (int64_t)(TT * tt + (tid & (TT - 1))) * (nK / 8);
        n_chunks = nK / kChunkSteps;
    }
    // chunk c, clamped: past the end the last chunk is read again, unused
    __device__ __forceinline__ void load(int c) {
        c = min(c, n_chunks - 1);
        const int64_t o = (int64_t)c * CSTEP;
#pragma unroll
        for (int m = 0; m < MT; ++m)
#pragma unroll
            for (int i = 0; i < kParts; ++i) r[m * kParts + i] = b[m * tstride + o + 256 * i];
        s = sb[2 * (c >> 1)];
        iv = ib[c >> 1];
    }
    __device__ __forceinline__ void store(u4* xs, v4f* ss, float* si, int tid) const {
#pragma unroll
        for (int i = 0; i < MT * kParts; ++i) xs[tid + 256 * i] = r[i];
        if (ss != nullptr && tid < 2 * TT) ss[tid] = s;
        if (ss != nullptr && tid >= 2 * TT && tid < 3 * TT) si[tid - 2 * TT] = iv;
    }
};

__device__ __forceinline__ uint32_t comp(const uint4& v, int i) {
    return i == 0 ? v.x : (i == 1 ? v.y : (i == 2 ? v.z : v.w));
}

// Q8_0 (src/kernels.cpp:364-373): 34-byte blocks of an fp16 scale d and 32
// int8 quants, value d*q. Here a super-block is 8 blocks (272 bytes) and
// step s of half h is block 4h + s. A block pair (68 bytes: d0 q0[32] d1
// q1[32]; dword k = bytes 4k..4k+3) starts 4-byte aligned. Lane group g
// loads dwords 4g+1 .. 4g+4 of each pair (16 bytes: the pair's bytes 4..67
// over the four groups) and one dword of the half's scale dwords (0 and 8
// of both pairs). Two lane swaps between the halves of the wave leave each
// group two dwords of each block: group g, s(g) = 2(g&1) + g/2, holds
//   even block: q0[2+8s .. 9+8s] (s = 3: q0[26..29], and q0[30], q0[31],
//               q0[0], q0[1] from dwords 8 and 0),
//   odd block:  q1[8s .. 8s+7],
// and three more swaps give every lane the four scale dwords. xsplit_kernel
// writes x in this order. q is exact in fp16 and so is each product with an
// x part; d scales each block's sum (fp32) after its matrix steps,
// lane-locally since an accumulator lane holds one row.
__device__ __forceinline__ uint32_t ld_w1(const uint8_t* p) {
    return *reinterpret_cast<const uint32_t*>(p);
}
typedef uint32_t u4a __attribute__((ext_vector_type(4), aligned(4)));
__device__ __forceinline__ u4a ld_w4(const uint8_t* p) {   // 4-byte aligned
    return *reinterpret_cast<const u4a*>(p);
}
// 8 int8 quants (bytes of w0, then w1) as fp16: each byte offset by 128 and
// placed under the exponent bits of 1024 by a byte permute, then 1152
// subtracted (exact).
__device__ __forceinline__ h8 q8_operand(uint32_t w0, uint32_t w1) {
    constexpr uint32_t E = 0x64646464u, LO = 0x04010400u, HI = 0x04030402u;
    const h2 off{(_Float16)-1152.f, (_Float16)-1152.f};
    const uint32_t u0 = w0 ^ 0x80808080u, u1 = w1 ^ 0x80808080u;
    const h2 a0 = as_h2(__builtin_amdgcn_perm(E, u0, LO)) + off;
    const h2 a1 = as_h2(__builtin_amdgcn_perm(E, u0, HI)) + off;
    const h2 a2 = as_h2(__builtin_amdgcn_perm(E, u1, LO)) + off;
    const h2 a3 = as_h2(__builtin_amdgcn_perm(E, u1, HI)) + off;
    return __builtin_bit_cast(h8, make_uint4(as_u32(a0), as_u32(a1), as_u32(a2), as_u32(a3)));
}

// Q6_K (src/kernels.cpp:427-458): 210-byte blocks of ql[128] (low 4 bits),
// qh[64] (high 2 bits), 16 int8 scales and an fp16 d; value d*sc*(q - 32)
// with sc per 16 values. Step s of half h is quarter s: values
// 128h + 32s + l, l < 32, from ql[64h + l + 32(s&1)] (low nibble for s < 2,
// high for s >= 2), bits 2s..2s+1 of qh[32h + l], scale sc[8h + 2s + l/16].
// Lane group g takes l = 8t .. 8t+7, t = (1, 3, 0, 2)[g]: it loads 16 bytes
// of the half's ql (ql[64h + 16g ..]), which two lane swaps across the wave's
// halves turn into ql[64h + 8t ..] and ql[64h + 32 + 8t ..]; 8 bytes of qh
// and the half's 8 scales. Blocks of odd index start 2 bytes past a 4-byte
// boundary: their words are loaded from 2 bytes earlier and funnel-shifted.
// sc*(q-32) reaches 4096, beyond fp16's exact integers (2048): it is split
// as w_hi = fp16(sc*(q-32)) (rounded) and w_lo = sc*(q-32) - w_hi (exact,
// |w_lo| <= 1), and each x part meets w_hi, the largest part w_lo as well.
// 8 quants of one quarter: low nibbles (ns = 0) or high (ns = 4) of the ql
// words, bits 2s..2s+1 of the qh words as bits 4-5, then q - 32 as fp16
// pairs (exponent bits of 1024 placed by byte permutes, 1056 subtracted).
__device__ __forceinline__ void q6_quants(uint32_t l0, uint32_t l1, uint32_t h0, uint32_t h1,
                                          int ns, int s, h2 (&q)[4]) {
    constexpr uint32_t E = 0x64646464u, LO = 0x04010400u, HI = 0x04030402u;
    const h2 off{(_Float16)-1056.f, (_Float16)-1056.f};
    const uint32_t u0 = ((l0 >> ns) & 0x0F0F0F0Fu) | (((h0 >> (2 * s)) << 4) & 0x30303030u);
    const uint32_t u1 = ((l1 >> ns) & 0x0F0F0F0Fu) | (((h1 >> (2 * s)) << 4) & 0x30303030u);
    q[0] = as_h2(__builtin_amdgcn_perm(E, u0, LO)) + off;
    q[1] = as_h2(__builtin_amdgcn_perm(E, u0, HI)) + off;
    q[2] = as_h2(__builtin_amdgcn_perm(E, u1, LO)) + off;
    q[3] = as_h2(__builtin_amdgcn_perm(E, u1, HI)) + off;
}

// IQ4_XS (src/kernels.cpp:405-425): 136-byte blocks of an fp16 d, 2+6 bits
// of scale ls a 32-value sub-block (scales_h, scales_l) and 128 quant bytes,
// value d*(ls - 32)*codebook[q]. A step is one sub-block; lane group g takes
// quant dword k = 3 - g of it: values 4k .. 4k+3 (low nibbles) and 16 + 4k ..
// +3 (high). Each lane loads 16 bytes (a whole sub-block) and a 4 x 4
// transpose by lane swaps hands it its dword of each. The codebook (int8,
// offset by 128) is looked up by byte permutes from two 8-entry halves,
// then made fp16 as for Q8_0; d*(ls - 32) scales each sub-block's sums.
__device__ __forceinline__ uint32_t iq4_lookup(uint32_t u) {   // 4 nibbles in bytes
    constexpr uint32_t T0 = 0xBFAD9881u ^ 0x80808080u, T1 = 0xF6EADDCFu ^ 0x80808080u;
    constexpr uint32_t T2 = 0x26190D01u ^ 0x80808080u, T3 = 0x71594535u ^ 0x80808080u;
    const uint32_t sel = u & 0x07070707u;
    const uint32_t lo = __builtin_amdgcn_perm(T1, T0, sel), hi = __builtin_amdgcn_perm(T3, T2, sel);
    const uint32_t m = ((u >> 3) & 0x01010101u) * 0xFFu;
    return (hi & m) | (lo & ~m);
}
__device__ __forceinline__ h8 iq4_operand(uint32_t w) {
    constexpr uint32_t E = 0x64646464u, LO = 0x04010400u, HI = 0x04030402u;
    const h2 off{(_Float16)-1152.f, (_Float16)-1152.f};
    const uint32_t a = iq4_lookup(w & 0x0F0F0F0Fu), b = iq4_lookup((w >> 4) & 0x0F0F0F0Fu);
    const h2 a0 = as_h2(__builtin_amdgcn_perm(E, a, LO)) + off;
    const h2 a1 = as_h2(__builtin_amdgcn_perm(E, a, HI)) + off;
    const h2 a2 = as_h2(__builtin_amdgcn_perm(E, b, LO)) + off;
    const h2 a3 = as_h2(__builtin_amdgcn_perm(E, b, HI)) + off;
    return __builtin_bit_cast(h8, make_uint4(as_u32(a0), as_u32(a1), as_u32(a2), as_u32(a3)));
}
// d*(ls - 32) of sub-block ib from the header words h0 (d, scales_h) and h1
// (scales_l), as the reference forms dl (src/kernels.cpp:413-415)
__device__ __forceinline__ float iq4_scale(uint32_t h0, uint32_t h1, int ib) {
    const int ls = (int)(((h1 >> (4 * ib)) & 0xFu) | (((h0 >> (16 + 2 * ib)) & 3u) << 4));
    return f16_lo(h0) * (float)(ls - 32);
}

// NT matrix tiles of 16 rows a wave; a workgroup covers 4 x 16NT rows. In
// the gate/up form (EPI >= 0, NT = 2) tile 0 holds 16 rows of the gate
// matrix and tile 1 the same 16 rows of the up matrix, so each lane ends
// with gate and up of the same (token, row) and writes act(gate) * up: a
// workgroup covers 4 x 16 output rows.
template <int TYPE, int NT, int EPI, int MT>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(NT == 4 ? 1 : 2)))
void split_gemm_kernel(SplitParams p) {
    constexpr bool Q5 = TYPE == AERO_DTYPE_Q5_K;
    constexpr bool Q8 = TYPE == AERO_DTYPE_Q8_0;
    constexpr bool Q6 = TYPE == AERO_DTYPE_Q6_K;
    constexpr bool IQ4 = TYPE == AERO_DTYPE_IQ4_XS;
    constexpr bool GU = EPI != kEpiPlain;
    static_assert(!GU || NT == 2, "gate/up pairs one gate and one up tile");
    constexpr int BB = Q8 ? 272 : (Q6 ? 210 : (Q5 ? 176 : (IQ4 ? 136 : 144)));   // bytes a super-block
    constexpr int QOFF = Q5 ? 48 : 16;          // quants within the block
    constexpr int kRowsWave = GU ? 16 : 16 * NT;
    constexpr int TT = 16 * MT;                 // tokens a workgroup (MT matrix tiles)
    constexpr int CHUNK = MT * XStage<MT>::CSTEP;   // uint4 a chunk
    __shared__ u4 xs[2][CHUNK];                 // 2 x 16 KB (MT = 2), by chunk parity
    __shared__ v4f ss[2][TT * 2];               // sub-block sums, by super-block parity
    __shared__ __align__(16) float si[2][TT];   // inverse scales, by super-block parity

    const int tid = threadIdx.x;
    const int l = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int r = l & 15, g = l >> 4;
    // the exponent bits of the Q4_K operand decode, kept in VGPRs (a VALU
    // instruction here takes one scalar or literal operand, the mask)
    uint32_t e_lo, e_hi;
    asm("v_mov_b32 %0, 0x64006400" : "=v"(e_lo));
    asm("v_mov_b32 %0, 0x54005400" : "=v"(e_hi));
    // this workgroup's matrix and its row tile within it (uniform)
    int mi = 0;
#pragma unroll
    for (int k = 1; k < kMaxMats; ++k) mi += (k < p.n_mat && (int)blockIdx.x >= p.tile0[k]);
    const uint8_t* const W = p.w[mi];
    float* const Y = p.y[mi];
    const int64_t n_rows = p.n_rows[mi];
    const int64_t row0 = (int64_t)((int)blockIdx.x - p.tile0[mi]) * (4 * kRowsWave) +
                         wave * kRowsWave;
    const int tt = blockIdx.y;
    const int nK = p.n_cols >> 5;
    const int n_chunks = nK / kChunkSteps, n_sb = n_chunks / 2;
    // this workgroup's super-blocks (all of them unless split over columns)
    const int sb_per = n_sb / p.ksplit;
    const int sb0 = (int)blockIdx.z * sb_per, sb1 = sb0 + sb_per;

    // rows past n_rows read the last row (their results are not stored)
    const uint8_t* wbase[NT];
    int woff[NT];
#pragma unroll
    for (int j = 0; j < NT; ++j) {
        wbase[j] = (GU && j == 1 ? p.w2 : W) + row0 * p.rb;
        const int64_t rj = GU ? row0 + r : row0 + 16 * j + r;
        woff[j] = (int)((min(rj, n_rows - 1) - row0) * p.rb);
    }

    XStage<MT> xst;
    xst.init(p.xp, p.xsum, p.xinv, tt, nK, tid);

    // quants of both halves of a super-block (Q5_K: the qh bytes, the same for
    // both halves) and its 16-byte header, loaded a super-block ahead
    uint4 q[2][NT], hq[NT], hd[NT];
    auto load_w = [&](int sb, uint4 (&qq)[2][NT], uint4 (&hh)[NT], uint4 (&dd)[NT]) {
        const int64_t sbo = (int64_t)min(sb, n_sb - 1) * BB;
#pragma unroll
        for (int j = 0; j < NT; ++j) {
            const uint8_t* b = wbase[j] + sbo;
            qq[0][j] = ld128(b + woff[j] + QOFF + 16 * g);
            qq[1][j] = ld128(b + woff[j] + QOFF + 64 + 16 * g);
            if (Q5) hh[j] = ld128(b + woff[j] + 16 + 16 * (g & 1));
            dd[j] = ld128(b + woff[j]);
        }
    };

    v4f acc[MT][NT], part[MT][NT];
#pragma unroll
    for (int m = 0; m < MT; ++m)
#pragma unroll
        for (int j = 0; j < NT; ++j) acc[m][j] = v4f{0.f, 0.f, 0.f, 0.f};

    h2 s_lo[NT], b_lo[NT], s_hi[NT], b_hi[NT];
    // sc of the lane's sub-block pair P = 2 half + g/2 of each row tile
    // (headers hh), as packed fp16 factors (sc, sc) and offsets (-1024 sc
    // for the low nibbles, -64 sc or Q5_K's -1024 sc for the high)
    auto set_scales = [&](int half, const uint4 (&hh)[NT]) {
#pragma unroll
        for (int j = 0; j < NT; ++j) {
            const h2 sp = kq_scale_pair(hh[j].y, hh[j].w, g >> 1, half);
            const h2 nb = sp * h2{(_Float16)-1024.f, (_Float16)(Q5 ? -1024.f : -64.f)};
            s_lo[j] = h2{sp[0], sp[0]};
            s_hi[j] = h2{sp[1], sp[1]};
            b_lo[j] = h2{nb[0], nb[0]};
            b_hi[j] = h2{nb[1], nb[1]};
        }
    };
    // the 4 steps of one chunk (half `half` of a super-block) from LDS
    // buffer xb with quants qq. Software-pipelined by one step: while the
    // matrix steps of step s run, the weights of step s+1 are decoded (VALU)
    // and its x operands read from LDS (two register sets of each), one matrix
    // step, two VALU instructions and (six times) one LDS read at a time.
    auto run_steps = [&](const u4* xb, int half, const uint4 (&qq)[NT],
                         const uint4 (&hh)[NT]) {
        const int P = 2 * half + (g >> 1);
        auto read_a = [&](int s, h8 (&a)[MT][kParts]) {
#pragma unroll
            for (int m = 0; m < MT; ++m)
#pragma unroll
                for (int pp = 0; pp < kParts; ++pp)
                    a[m][pp] = __builtin_bit_cast(
                        h8, xb[((m * kChunkSteps + s) * kParts + pp) * 64 + l]);
        };
        auto decode_b = [&](int s, h8 (&b)[NT]) {
#pragma unroll
            for (int j = 0; j < NT; ++j)
                b[j] = weight_operand<Q5>(comp(qq[j], s), Q5 ? comp(hh[j], s) : 0u, P, s_lo[j],
                                          b_lo[j], s_hi[j], b_hi[j], e_lo, e_hi);
        };
        if constexpr (MT == 4) {
            // 64 tokens: one register set of x operands, each tile's refilled
            // for the next step as soon as its matrix steps are issued
            h8 A[MT][kParts], B[2][NT];
            read_a(0, A);
            decode_b(0, B[0]);
#pragma unroll
            for (int s = 0; s < kChunkSteps; ++s) {
                if (s + 1 < kChunkSteps) decode_b(s + 1, B[(s + 1) & 1]);
#pragma unroll
                for (int m = 0; m < MT; ++m) {
                    // small parts first into each tile's super-block sum
#pragma unroll
                    for (int pp = kParts - 1; pp >= 0; --pp)
#pragma unroll
                        for (int j = 0; j < NT; ++j)
                            part[m][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(
                                A[m][pp], B[s & 1][j], part[m][j], 0, 0, 0);
                    if (s + 1 < kChunkSteps) {
#pragma unroll
                        for (int pp = 0; pp < kParts; ++pp)
                            A[m][pp] = __builtin_bit_cast(
                                h8, xb[((m * kChunkSteps + s + 1) * kParts + pp) * 64 + l]);
                    }
                }
#pragma unroll
                for (int i = 0; i < kParts * MT * NT; ++i) {
                    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // one matrix step
                    __builtin_amdgcn_sched_group_barrier(0x002, 1, 0);  // one VALU
                    if (i % (kParts * NT) == kParts * NT - 1)
                        __builtin_amdgcn_sched_group_barrier(0x100, kParts, 0);  // LDS reads
                }
                __builtin_amdgcn_sched_barrier(0);
            }
            return;
        }
        h8 A[2][MT][kParts], B[2][NT];
        read_a(0, A[0]);
        decode_b(0, B[0]);
#pragma unroll
        for (int s = 0; s < kChunkSteps; ++s) {
            if (s + 1 < kChunkSteps) {
                read_a(s + 1, A[(s + 1) & 1]);
                decode_b(s + 1, B[(s + 1) & 1]);
            }
            // small parts first into each tile's super-block sum
#pragma unroll
            for (int pp = kParts - 1; pp >= 0; --pp)
#pragma unroll
                for (int m = 0; m < MT; ++m)
#pragma unroll
                    for (int j = 0; j < NT; ++j)
                        part[m][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(
                            A[s & 1][m][pp], B[s & 1][j], part[m][j], 0, 0, 0);
            constexpr int kMfma = kParts * MT * NT, kReads = MT * kParts;
#pragma unroll
            for (int i = 0; i < kMfma; ++i) {
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // one matrix step
                __builtin_amdgcn_sched_group_barrier(0x002, 2, 0);  // two VALU
                if (i < kReads) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // LDS read
            }
            __builtin_amdgcn_sched_barrier(0);
        }
    };

    // Q8_0: half `half` of super-block sb as loaded (dwords 4g+1 .. 4g+4 of
    // each pair, then the scale dword g); arranged by arrange_w8 before use
    auto load_w8 = [&](int sb, int half, uint32_t (&dst)[NT][12]) {
        const int64_t o = (int64_t)min(sb, n_sb - 1) * BB + 136 * half;
#pragma unroll
        for (int j = 0; j < NT; ++j) {
            const uint8_t* e = wbase[j] + woff[j] + o;
#pragma unroll
            for (int pr = 0; pr < 2; ++pr) {
                const u4a v = ld_w4(e + 68 * pr + 4 + 16 * g);
                dst[j][4 * pr + 0] = v[0];
                dst[j][4 * pr + 1] = v[1];
                dst[j][4 * pr + 2] = v[2];
                dst[j][4 * pr + 3] = v[3];
            }
            dst[j][8] = ld_w1(e + 68 * (g >> 1) + 32 * (g & 1));
        }
    };
    // in place: per pair, dwords 0-1 the even block's operand words, 2-3 the
    // odd block's; 8-11 the scale dwords 0 and 8 of pair 0, then of pair 1
    auto arrange_w8 = [&](uint32_t (&w)[NT][12]) {
#pragma unroll
        for (int j = 0; j < NT; ++j) {
#pragma unroll
            for (int pr = 0; pr < 2; ++pr) {
                uint32_t* v = w[j] + 4 * pr;
                const auto a = __builtin_amdgcn_permlane32_swap(v[0], v[2], false, false);
                const auto b = __builtin_amdgcn_permlane32_swap(v[1], v[3], false, false);
                v[0] = a[0];
                v[2] = a[1];
                v[1] = b[0];
                v[3] = b[1];
            }
            const uint32_t x = w[j][8];
            const auto c = __builtin_amdgcn_permlane16_swap(x, x, false, false);
            const auto e = __builtin_amdgcn_permlane32_swap(c[0], c[0], false, false);
            const auto f = __builtin_amdgcn_permlane32_swap(c[1], c[1], false, false);
            w[j][8] = e[0];
            w[j][9] = f[0];
            w[j][10] = e[1];
            w[j][11] = f[1];
        }
    };
    // IQ4_XS: half `half` of super-block sb: dwords 0-3 the 16 quant bytes
    // 64 half + 16 g of the block's qs (sub-block 4 half + g), 4-5 its header
    auto load_iq4 = [&](int sb, int half, uint32_t (&dst)[NT][12]) {
        const int64_t o = (int64_t)min(sb, n_sb - 1) * BB;
#pragma unroll
        for (int j = 0; j < NT; ++j) {
            const uint8_t* e = wbase[j] + woff[j] + o;
            const u4a v = ld_w4(e + 8 + 64 * half + 16 * g);
            const uint2 h = ld64(e);
            dst[j][0] = v[0];
            dst[j][1] = v[1];
            dst[j][2] = v[2];
            dst[j][3] = v[3];
            dst[j][4] = h.x;
            dst[j][5] = h.y;
        }
    };
    auto load_wb = [&](int sb, int half, uint32_t (&dst)[NT][12]) {
        if constexpr (IQ4) load_iq4(sb, half, dst);
        else load_w8(sb, half, dst);
    };
    // in place, a 4 x 4 transpose over the lane groups: dword 3 - s becomes
    // quant dword 3 - g of sub-block 4 half + s
    auto arrange_iq4 = [&](uint32_t (&w)[NT][12]) {
#pragma unroll
        for (int j = 0; j < NT; ++j) {
            uint32_t* v = w[j];
            const auto a = __builtin_amdgcn_permlane32_swap(v[2], v[0], false, false);
            const auto b = __builtin_amdgcn_permlane32_swap(v[3], v[1], false, false);
            const auto c = __builtin_amdgcn_permlane16_swap(b[1], a[1], false, false);
            const auto e = __builtin_amdgcn_permlane16_swap(b[0], a[0], false, false);
            v[1] = c[0];
            v[0] = c[1];
            v[3] = e[0];
            v[2] = e[1];
        }
    };
    // the 4 blocks of one half from LDS buffer xb: each block's matrix steps
    // into P from zero, then sacc += d * P a step later (pipelined as
    // run_steps, with the block's d conversion and scaling among the VALU)
    v4f sacc[MT][NT];
    auto run_q8 = [&](const u4* xb, uint32_t (&wq)[NT][12], int half) {
        if constexpr (IQ4) arrange_iq4(wq);
        else arrange_w8(wq);
        h8 A[2][MT][kParts], B[2][NT];
        v4f P[2][MT][NT];
        auto read_a = [&](int s, h8 (&a)[MT][kParts]) {
#pragma unroll
            for (int m = 0; m < MT; ++m)
#pragma unroll
                for (int pp = 0; pp < kParts; ++pp)
                    a[m][pp] = __builtin_bit_cast(
                        h8, xb[((m * kChunkSteps + s) * kParts + pp) * 64 + l]);
        };
        auto decode = [&](int s, h8 (&b)[NT]) {
#pragma unroll
            for (int j = 0; j < NT; ++j) {
                if constexpr (IQ4) {
                    b[j] = iq4_operand(wq[j][3 - s]);
                    continue;
                }
                const uint32_t* w = wq[j] + 4 * (s >> 1);
                const uint32_t d0 = wq[j][8 + 2 * (s >> 1)], d8 = wq[j][9 + 2 * (s >> 1)];
                if (s & 1) {
                    b[j] = q8_operand(w[2], w[3]);
                } else {
                    const uint32_t w1 = g == 3 ? __builtin_amdgcn_perm(d8, d0, 0x03020504u) : w[1];
                    b[j] = q8_operand(w[0], w1);
                }
            }
        };
        auto scale_in = [&](int s) {
#pragma unroll
            for (int j = 0; j < NT; ++j) {
                float d;
                if constexpr (IQ4) {
                    d = iq4_scale(wq[j][4], wq[j][5], 4 * half + s);
                } else {
                    const uint32_t dw = wq[j][8 + 2 * (s >> 1) + (s & 1)];
                    d = (s & 1) ? f16_hi(dw) : f16_lo(dw);
                }
#pragma unroll
                for (int m = 0; m < MT; ++m)
#pragma unroll
                    for (int v = 0; v < 4; ++v)
                        sacc[m][j][v] = fmaf(d, P[s & 1][m][j][v], sacc[m][j][v]);
            }
        };
        read_a(0, A[0]);
        decode(0, B[0]);
#pragma unroll
        for (int s = 0; s < kChunkSteps; ++s) {
            if (s + 1 < kChunkSteps) {
                read_a(s + 1, A[(s + 1) & 1]);
                decode(s + 1, B[(s + 1) & 1]);
            }
#pragma unroll
            for (int pp = kParts - 1; pp >= 0; --pp)
#pragma unroll
                for (int m = 0; m < MT; ++m)
#pragma unroll
                    for (int j = 0; j < NT; ++j)
                        P[s & 1][m][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(
                            A[s & 1][m][pp], B[s & 1][j],
                            pp == kParts - 1 ? v4f{0.f, 0.f, 0.f, 0.f} : P[s & 1][m][j], 0, 0,
                            0);
            if (s > 0) scale_in(s - 1);
            constexpr int kMfma = kParts * MT * NT, kReads = MT * kParts;
#pragma unroll
            for (int i = 0; i < kMfma; ++i) {
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // one matrix step
                __builtin_amdgcn_sched_group_barrier(0x002, 5, 0);  // five VALU
                if (i < kReads) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // LDS read
            }
            __builtin_amdgcn_sched_barrier(0);
        }
        scale_in(kChunkSteps - 1);
    };

    // Q6_K: half `half` of super-block sb as loaded: 4-byte aligned words from
    // sh = 2 (odd blocks) or 0 bytes before each field: ql 16 bytes (5 words),
    // qh 8 (3 words), the half's 8 scales (3 words)
    typedef uint32_t u3a __attribute__((ext_vector_type(3), aligned(4)));
    auto load_w6 = [&](int sb, int half, uint32_t (&dst)[NT][11]) {
        const int sbc = min(sb, n_sb - 1);
        const int64_t o = (int64_t)sbc * BB - 2 * (sbc & 1);
        const int t6 = (0x2031 >> (4 * g)) & 3;
#pragma unroll
        for (int j = 0; j < NT; ++j) {
            const uint8_t* e = wbase[j] + woff[j] + o;
            const u4a v = ld_w4(e + 64 * half + 16 * g);
            const u3a h = *reinterpret_cast<const u3a*>(e + 128 + 32 * half + 8 * t6);
            const u3a c = *reinterpret_cast<const u3a*>(e + 192 + 8 * half);
            dst[j][0] = v[0];
            dst[j][1] = v[1];
            dst[j][2] = v[2];
            dst[j][3] = v[3];
            dst[j][4] = ld_w1(e + 64 * half + 16 * g + 16);
            dst[j][5] = h[0];
            dst[j][6] = h[1];
            dst[j][7] = h[2];
            dst[j][8] = c[0];
            dst[j][9] = c[1];
            dst[j][10] = c[2];
        }
    };
    // the 4 quarters of one half from LDS buffer xb into part (raw words wq
    // of a block starting sh bytes past a 4-byte boundary); pipelined as
    // run_steps, three matrix steps a tile and quarter
    auto run_q6 = [&](const u4* xb, const uint32_t (&wq)[NT][11], int sh) {
        // ql: (lq[2], lq[3]) = ql[.. + 8t ..], (lq[0], lq[1]) = ql[.. + 32 + 8t ..]
        uint32_t lq[NT][4], hq6[NT][2], sq[NT][2];
        const int t6 = (0x2031 >> (4 * g)) & 3;
#pragma unroll
        for (int j = 0; j < NT; ++j) {
            uint32_t f[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) f[i] = __builtin_amdgcn_alignbyte(wq[j][i + 1], wq[j][i], sh);
            const auto a = __builtin_amdgcn_permlane32_swap(f[2], f[0], false, false);
            const auto b = __builtin_amdgcn_permlane32_swap(f[3], f[1], false, false);
            lq[j][2] = a[0];
            lq[j][0] = a[1];
            lq[j][3] = b[0];
            lq[j][1] = b[1];
            hq6[j][0] = __builtin_amdgcn_alignbyte(wq[j][6], wq[j][5], sh);
            hq6[j][1] = __builtin_amdgcn_alignbyte(wq[j][7], wq[j][6], sh);
            sq[j][0] = __builtin_amdgcn_alignbyte(wq[j][9], wq[j][8], sh) ^ 0x80808080u;
            sq[j][1] = __builtin_amdgcn_alignbyte(wq[j][10], wq[j][9], sh) ^ 0x80808080u;
        }
        h8 A[2][MT][kParts], Bh[2][NT], Bl[2][NT];
        auto read_a = [&](int s, h8 (&a)[MT][kParts]) {
#pragma unroll
            for (int m = 0; m < MT; ++m)
#pragma unroll
                for (int pp = 0; pp < kParts; ++pp)
                    a[m][pp] = __builtin_bit_cast(
                        h8, xb[((m * kChunkSteps + s) * kParts + pp) * 64 + l]);
        };
        auto decode = [&](int s, h8 (&bh)[NT], h8 (&bl)[NT]) {
            // the lane's scale sc[8h + 2s + t/2] as a packed fp16 pair
            const uint32_t k = 2 * (s & 1) + (t6 >> 1);
            const uint32_t sel = k | (4u << 8) | (k << 16) | (4u << 24);
#pragma unroll
            for (int j = 0; j < NT; ++j) {
                h2 q[4];
                q6_quants(lq[j][(s & 1) ? 0 : 2], lq[j][(s & 1) ? 1 : 3], hq6[j][0], hq6[j][1],
                          (s >> 1) * 4, s, q);
                const h2 sc = as_h2(__builtin_amdgcn_perm(0x64646464u, sq[j][s >> 1], sel)) +
                              h2{(_Float16)-1152.f, (_Float16)-1152.f};
                h2 hi[4], lo[4];
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    hi[i] = q[i] * sc;
                    lo[i] = __builtin_elementwise_fma(q[i], sc, -hi[i]);
                }
                bh[j] = __builtin_bit_cast(h8, make_uint4(as_u32(hi[0]), as_u32(hi[1]),
                                                          as_u32(hi[2]), as_u32(hi[3])));
                bl[j] = __builtin_bit_cast(h8, make_uint4(as_u32(lo[0]), as_u32(lo[1]),
                                                          as_u32(lo[2]), as_u32(lo[3])));
            }
        };
        read_a(0, A[0]);
        decode(0, Bh[0], Bl[0]);
#pragma unroll
        for (int s = 0; s < kChunkSteps; ++s) {
            if (s + 1 < kChunkSteps) {
                read_a(s + 1, A[(s + 1) & 1]);
                decode(s + 1, Bh[(s + 1) & 1], Bl[(s + 1) & 1]);
            }
            // small parts first: x's lower parts with w_hi, x's largest with
            // w_lo, then with w_hi
#pragma unroll
            for (int pp = kParts - 1; pp >= 1; --pp)
#pragma unroll
                for (int m = 0; m < MT; ++m)
#pragma unroll
                    for (int j = 0; j < NT; ++j)
                        part[m][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(
                            A[s & 1][m][pp], Bh[s & 1][j], part[m][j], 0, 0, 0);
#pragma unroll
            for (int m = 0; m < MT; ++m)
#pragma unroll
                for (int j = 0; j < NT; ++j) {
                    part[m][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(
                        A[s & 1][m][0], Bl[s & 1][j], part[m][j], 0, 0, 0);
                    part[m][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(
                        A[s & 1][m][0], Bh[s & 1][j], part[m][j], 0, 0, 0);
                }
            constexpr int kMfma = (kParts + 1) * MT * NT, kReads = MT * kParts;
#pragma unroll
            for (int i = 0; i < kMfma; ++i) {
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // one matrix step
                __builtin_amdgcn_sched_group_barrier(0x002, 5, 0);  // five VALU
                if (i < kReads) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // LDS read
            }
            __builtin_amdgcn_sched_barrier(0);
        }
    };

    if constexpr (Q6) {
        uint32_t wa[NT][11];
        xst.load(2 * sb0);
        load_w6(sb0, 0, wa);
        xst.store(xs[0], ss[sb0 & 1], si[sb0 & 1], tid);
        xst.load(2 * sb0 + 1);
        __syncthreads();
        for (int sb = sb0; sb < sb1; ++sb) {
            uint32_t wb[NT][11];
            load_w6(sb, 1, wb);
            const int sh = 2 * (sb & 1);
#pragma unroll
            for (int m = 0; m < MT; ++m)
#pragma unroll
                for (int j = 0; j < NT; ++j) part[m][j] = v4f{0.f, 0.f, 0.f, 0.f};
            run_q6(xs[0], wa, sh);
            xst.store(xs[1], nullptr, nullptr, tid);
            xst.load(2 * sb + 2);
            __syncthreads();
            load_w6(sb + 1, 0, wa);   // the next super-block's first half (clamped)
            run_q6(xs[1], wb, sh);
            // acc += inv * d * part: d in the second half's scale words (block
            // bytes 208-209: the low half of the last word, or its high half
            // when the words start 2 bytes early)
            const float* ip = si[sb & 1];
#pragma unroll
            for (int j = 0; j < NT; ++j) {
                const float d = sh ? f16_hi(wb[j][10]) : f16_lo(wb[j][10]);
#pragma unroll
                for (int m = 0; m < MT; ++m) {
                    const v4f inv = *reinterpret_cast<const v4f*>(ip + 16 * m + 4 * g);
#pragma unroll
                    for (int v = 0; v < 4; ++v)
                        acc[m][j][v] = fmaf(inv[v], d * part[m][j][v], acc[m][j][v]);
                }
            }
            xst.store(xs[0], ss[(sb + 1) & 1], si[(sb + 1) & 1], tid);
            xst.load(2 * sb + 3);
            __syncthreads();
        }
    } else if constexpr (Q8 || IQ4) {
        uint32_t wa[NT][12];
        xst.load(2 * sb0);
        load_wb(sb0, 0, wa);
        xst.store(xs[0], ss[sb0 & 1], si[sb0 & 1], tid);
        xst.load(2 * sb0 + 1);
        __syncthreads();
        for (int sb = sb0; sb < sb1; ++sb) {
            uint32_t wb[NT][12];
            load_wb(sb, 1, wb);
#pragma unroll
            for (int m = 0; m < MT; ++m)
#pragma unroll
                for (int j = 0; j < NT; ++j) sacc[m][j] = v4f{0.f, 0.f, 0.f, 0.f};
            run_q8(xs[0], wa, 0);
            xst.store(xs[1], nullptr, nullptr, tid);
            xst.load(2 * sb + 2);
            __syncthreads();
            load_wb(sb + 1, 0, wa);   // the next super-block's first half (clamped)
            run_q8(xs[1], wb, 1);
            // acc += inv * sacc, inv the token's inverse scale of this super-block
            const float* ip = si[sb & 1];
#pragma unroll
            for (int m = 0; m < MT; ++m) {
                const v4f inv = *reinterpret_cast<const v4f*>(ip + 16 * m + 4 * g);
#pragma unroll
                for (int j = 0; j < NT; ++j)
#pragma unroll
                    for (int v = 0; v < 4; ++v)
                        acc[m][j][v] = fmaf(inv[v], sacc[m][j][v], acc[m][j][v]);
            }
            xst.store(xs[0], ss[(sb + 1) & 1], si[(sb + 1) & 1], tid);
            xst.load(2 * sb + 3);
            __syncthreads();
        }
    } else {
    // prologue: chunk 2 sb0 (super-block sb0, first half) staged, the next in
    // flight
    xst.load(2 * sb0);
    load_w(sb0, q, hq, hd);
    xst.store(xs[0], ss[sb0 & 1], si[sb0 & 1], tid);
    xst.load(2 * sb0 + 1);
    __syncthreads();

    // one super-block with its weights in (qc, hqc, hdc) while the next one's
    // load into (qn, hqn, hdn); the loop alternates the two register sets
    auto sb_body = [&](int sb, const uint4 (&qc)[2][NT], const uint4 (&hqc)[NT],
                       const uint4 (&hdc)[NT], uint4 (&qn)[2][NT], uint4 (&hqn)[NT],
                       uint4 (&hdn)[NT]) {
        load_w(sb + 1, qn, hqn, hdn);   // the next super-block (clamped)
        // ---- first half: chunk 2sb in xs[0]
        set_scales(0, hdc);
#pragma unroll
        for (int m = 0; m < MT; ++m)
#pragma unroll
            for (int j = 0; j < NT; ++j) part[m][j] = v4f{0.f, 0.f, 0.f, 0.f};
        run_steps(xs[0], 0, qc[0], hqc);
        xst.store(xs[1], nullptr, nullptr, tid);   // chunk 2sb+1 (loaded a chunk ago)
        xst.load(2 * sb + 2);
        __syncthreads();

        // ---- second half: chunk 2sb+1 in xs[1]
        set_scales(1, hdc);
        run_steps(xs[1], 1, qc[1], hqc);
        // acc += inv * (d * part + mins), inv the token's inverse scale for
        // this super-block and mins = -dmin * sum_k m_k S_k on the fp32 matrix
        // cores: A[token][k] = S of sub-block k (k = g, then g + 4), B[k][row]
        // = -dmin * m_k of the lane's row (lane-local), D in part's layout
        const float* sp = reinterpret_cast<const float*>(ss[sb & 1]);
        const float* ip = si[sb & 1];
        float sa[MT][2];
#pragma unroll
        for (int m = 0; m < MT; ++m) {
            sa[m][0] = sp[8 * (16 * m + r) + g];
            sa[m][1] = sp[8 * (16 * m + r) + g + 4];
        }
#pragma unroll
        for (int j = 0; j < NT; ++j) {
            const float d = f16_lo(hdc[j].x);
            const float ndm = -f16_hi(hdc[j].x);
            uint32_t m0, m1;
            kq_min_pair(hdc[j].z, hdc[j].w, g, m0, m1);
            const float b0 = ndm * (float)m0, b1 = ndm * (float)m1;
#pragma unroll
            for (int m = 0; m < MT; ++m) {
                v4f mins = __builtin_amdgcn_mfma_f32_16x16x4f32(sa[m][0], b0,
                                                                v4f{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
                mins = __builtin_amdgcn_mfma_f32_16x16x4f32(sa[m][1], b1, mins, 0, 0, 0);
                const v4f inv = *reinterpret_cast<const v4f*>(ip + 16 * m + 4 * g);
#pragma unroll
                for (int v = 0; v < 4; ++v)
                    acc[m][j][v] = fmaf(inv[v], fmaf(d, part[m][j][v], mins[v]), acc[m][j][v]);
            }
        }
        xst.store(xs[0], ss[(sb + 1) & 1], si[(sb + 1) & 1], tid);  // chunk 2sb+2
        xst.load(2 * sb + 3);
        __syncthreads();
    };
    uint4 q2[2][NT], hq2[NT], hd2[NT];
    for (int sb = sb0; sb < sb1; sb += 2) {
        sb_body(sb, q, hq, hd, q2, hq2, hd2);
        if (sb + 1 < sb1) sb_body(sb + 1, q2, hq2, hd2, q, hq, hd);
    }
    }

    // split over columns: the raw sums go to the partials (the norm's scale
    // and the gate/up act follow the reduction)
    if (p.ksplit > 1) {
        float* P = p.part + (int64_t)blockIdx.z * p.n_tok * p.r_all;
#pragma unroll
        for (int m = 0; m < MT; ++m)
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                const int tok = TT * tt + 16 * m + 4 * g + v;
                if (tok >= p.n_tok) continue;
                float* pp = P + (int64_t)tok * p.r_all;
                if constexpr (GU) {
                    const int64_t row = row0 + r;
                    if (row < n_rows) {
                        pp[row] = acc[m][0][v];
                        pp[n_rows + row] = acc[m][1][v];
                    }
                } else {
#pragma unroll
                    for (int j = 0; j < NT; ++j) {
                        const int64_t row = row0 + 16 * j + r;
                        if (row < n_rows) pp[p.roff[mi] + row] = acc[m][j][v];
                    }
                }
            }
        return;
    }

    // folded norm: each token's sums times 1/sqrtf(sum of x^2 / n + eps),
    // the sum of its super-block partials (8 lanes a token, in a fixed order;
    // 64-token tiles take two rounds)
    __shared__ float tinv[TT];
    if (p.ssq != nullptr) {
#pragma unroll
        for (int h = 0; h < MT / 2; ++h) {
            const int k = 32 * h + (tid >> 3), part = tid & 7;
            const float* sp = p.ssq + (int64_t)(TT * tt + k) * n_sb;
            float sum = 0.f;
            for (int i = part; i < n_sb; i += 8) sum += sp[i];
            sum = group_sum<8>(sum);
            if (part == 0) tinv[k] = 1.0f / sqrtf(sum / (float)p.n_cols + p.eps);
        }
        __syncthreads();
    }

    // q / k heads: the per-head norm and RoPE on the workgroup's whole heads
    // (src/attention_layer.cpp:89-156). The tile goes through LDS (the x
    // staging buffers, free after the loop's last barrier) so that each
    // thread holds SLOTS channel pairs of one (token, head): NeoX pairs
    // (i, i + rot/2) for i < rot/2, then the unrotated channels two at a
    // time; interleaved pairs (2i, 2i + 1). Threads of one (token, head)
    // are TPU adjacent lanes; the norm's sum of squares is theirs.
    if constexpr (!GU) {
        if (mi < p.rope_mats) {   // uniform: the workgroup's matrix
            constexpr int RW = 4 * kRowsWave;            // rows a workgroup
            constexpr int LD = NT == 2 ? RW + 4 : RW;    // tile row stride (floats)
            constexpr int SLOTS = TT * RW / 512;         // pairs a thread
            static_assert(TT * LD * 4 <= (int)sizeof(xs), "rope tile fits the staging");
            float* tile = reinterpret_cast<float*>(&xs[0][0]);
#pragma unroll
            for (int m = 0; m < MT; ++m)
#pragma unroll
                for (int v = 0; v < 4; ++v) {
                    const int tk = 16 * m + 4 * g + v;
                    const float inv = p.ssq != nullptr ? tinv[tk] : 1.0f;
#pragma unroll
                    for (int j = 0; j < NT; ++j)
                        tile[tk * LD + wave * kRowsWave + 16 * j + r] =
                            p.ssq != nullptr ? acc[m][j][v] * inv : acc[m][j][v];
                }
            __syncthreads();
            const int D = p.rope_D, half = p.rope_rot / 2;
            const int tpu = D / (2 * SLOTS);             // threads a (token, head)
            const int hpw = RW / D;                      // heads a workgroup
            const int u = tid / tpu, k = tid - u * tpu;
            const int tk = u / hpw, hl = u - tk * hpw;
            const int tok = TT * tt + tk;
            const int64_t hrow = (int64_t)((int)blockIdx.x - p.tile0[mi]) * RW + hl * D;
            const bool neox = p.rope_mode == AERO_ROPE_NEOX;
            float a[SLOTS], b[SLOTS];
            int c0[SLOTS], c1[SLOTS];
#pragma unroll
            for (int i = 0; i < SLOTS; ++i) {
                const int qi = k * SLOTS + i;
                if (neox) {
                    c0[i] = qi < half ? qi : p.rope_rot + 2 * (qi - half);
                    c1[i] = qi < half ? qi + half : c0[i] + 1;
                } else {
                    c0[i] = 2 * qi;
                    c1[i] = 2 * qi + 1;
                }
                a[i] = tile[tk * LD + hl * D + c0[i]];
                b[i] = tile[tk * LD + hl * D + c1[i]];
            }
            const float* qw = p.qk_w[mi < 2 ? mi : 0];
            if (qw != nullptr) {   // uniform
                float ss = 0.f;
#pragma unroll
                for (int i = 0; i < SLOTS; ++i) {
                    ss += a[i] * a[i];
                    ss += b[i] * b[i];
                }
                for (int o = 1; o < tpu; o <<= 1) ss += __shfl_xor(ss, o);
                const float ninv = 1.0f / sqrtf(ss / (float)D + p.qk_eps);
                const bool uo = (p.qk_flags & AERO_NORM_UNIT_OFFSET) != 0;
#pragma unroll
                for (int i = 0; i < SLOTS; ++i) {
                    const float w0 = uo ? 1.0f + qw[c0[i]] : qw[c0[i]];
                    const float w1 = uo ? 1.0f + qw[c1[i]] : qw[c1[i]];
                    a[i] = (a[i] * ninv) * w0;
                    b[i] = (b[i] * ninv) * w1;
                }
            }
            if (tok < p.n_tok && hrow < n_rows) {
                const float pt = (float)p.pos[tok];
                float* yp = Y + (int64_t)tok * n_rows + hrow;
#pragma unroll
                for (int i = 0; i < SLOTS; ++i) {
                    const int qi = k * SLOTS + i;
                    float o0 = a[i], o1 = b[i];
                    if (qi < half) {
                        // x0 c - x1 s, x0 s + x1 c (src/transformer.cpp:77-93)
                        float sn, c;
                        sincosf(pt * p.rinv[qi], &sn, &c);
                        o0 = a[i] * c - b[i] * sn;
                        o1 = a[i] * sn + b[i] * c;
                    }
                    yp[c0[i]] = o0;
                    yp[c1[i]] = o1;
                }
            }
            return;
        }
    }

    // acc[m][j][v]: token TT tt + 16m + 4g + v, row row0 + 16j + r (gate/up:
    // row row0 + r of the gate (j = 0) and the up (j = 1) matrix)
#pragma unroll
    for (int m = 0; m < MT; ++m)
#pragma unroll
        for (int v = 0; v < 4; ++v) {
            const int tk = 16 * m + 4 * g + v;
            const int tok = TT * tt + tk;
            if (tok >= p.n_tok) continue;
            const float inv = p.ssq != nullptr ? tinv[tk] : 1.0f;
            float* yp = Y + (int64_t)tok * n_rows;
            if constexpr (GU) {
                const int64_t row = row0 + r;
                float gv = acc[m][0][v], uv = acc[m][1][v];
                if (p.ssq != nullptr) {
                    gv = gv * inv;
                    uv = uv * inv;
                }
                if (row < n_rows) yp[row] = act<GU ? EPI : 0>(gv) * uv;
            } else {
#pragma unroll
                for (int j = 0; j < NT; ++j) {
                    const int64_t row = row0 + 16 * j + r;
                    const float y = p.ssq != nullptr ? acc[m][j][v] * inv : acc[m][j][v];
                    if (row < n_rows) yp[row] = y;
                }
            }
        }
}

// Sum of the column splits' partials of split_gemm_kernel, in split order,
// then the epilogue the unsplit kernel applies: each token's sums times its
// 1/sqrtf(sum of x^2 / n + eps) (folded norm; the super-block partials
// summed by 8 lanes in the kernel's order), and y = sum, or (gate/up) out =
// act(gate) * up. Thread (x, token) owns one output: every partial load is
// issued at once (clamped, at most kMaxSplits), then added in order.
constexpr int kMaxSplits = 16;
struct ReduceArgs {
    const float* part;    // [ksplit][n_tok][r_all]
    int ksplit;
    int n_tok;
    int64_t r_all;
    const float* ssq;     // [tok_pad][n_sb] or null
    int n_sb;
    int n_cols;
    float eps;
    int n_mat;            // plain form
    float* y[kMaxMats];
    int64_t n_rows[kMaxMats];
    int64_t roff[kMaxMats + 1];
};

template <int EPI>
__global__ __launch_bounds__(256) void split_reduce_kernel(ReduceArgs a) {
    constexpr bool GU = EPI != kEpiPlain;
    const int tid = threadIdx.x;
    const int tok = blockIdx.y;
    __shared__ float tinv;
    if (tid < 8) {
        float sum = 0.f;
        if (a.ssq != nullptr) {
            const float* sp = a.ssq + (int64_t)tok * a.n_sb;
            for (int i = tid; i < a.n_sb; i += 8) sum += sp[i];
        }
        sum = group_sum<8>(sum);
        if (tid == 0) tinv = a.ssq != nullptr ? 1.0f / sqrtf(sum / (float)a.n_cols + a.eps) : 1.f;
    }
    const int64_t n_out = GU ? a.r_all / 2 : a.r_all;
    const int64_t o = (int64_t)blockIdx.x * 256 + tid;
    const int64_t oc = o < n_out ? o : n_out - 1;
    const int64_t stride = (int64_t)a.n_tok * a.r_all;
    const float* pt = a.part + (int64_t)tok * a.r_all + oc;
    float pg[kMaxSplits], pu[GU ? kMaxSplits : 1];
#pragma unroll
    for (int z = 0; z < kMaxSplits; ++z) {
        const int64_t zo = (int64_t)min(z, a.ksplit - 1) * stride;
        pg[z] = pt[zo];
        if constexpr (GU) pu[z] = pt[zo + n_out];
    }
    __syncthreads();
    const float inv = tinv;
    if (o >= n_out) return;
    float gv = 0.f, uv = 0.f;
#pragma unroll
    for (int z = 0; z < kMaxSplits; ++z) {
        if (z < a.ksplit) {
            gv += pg[z];
            if constexpr (GU) uv += pu[z];
        }
    }
    if (a.ssq != nullptr) {
        gv = gv * inv;
        if constexpr (GU) uv = uv * inv;
    }
    if constexpr (GU) {
        a.y[0][(int64_t)tok * n_out + o] = act<GU ? EPI : 0>(gv) * uv;
    } else {
        int m = 0;
#pragma unroll
        for (int i = 1; i < kMaxMats; ++i) m += (i < a.n_mat && o >= a.roff[i]);
        a.y[m][(int64_t)tok * a.n_rows[m] + (o - a.roff[m])] = gv;
    }
}

inline int64_t align256(int64_t b) { return (b + 255) & ~(int64_t)255; }

// Workspace layout of the split-x GEMM for tp (padded) tokens of n_cols:
// the x parts, the sub-block sums, the inverse scales and, with a folded
// norm, the per-super-block sums of x^2.
struct SplitWs {
    uint4* xp;
    float* xsum;
    float* xinv;
    float* ssq;
};

int64_t split_ws_bytes(int64_t tp, int64_t n_cols, bool norm) {
    return align256(tp * n_cols * 2 * kParts) + align256(tp * (n_cols / 32) * 4) +
           align256(tp * (n_cols / 256) * 4) + (norm ? align256(tp * (n_cols / 256) * 4) : 0);
}

SplitWs split_ws(void* ws, int64_t tp, int64_t n_cols) {
    uint8_t* b = static_cast<uint8_t*>(ws);
    SplitWs w;
    w.xp = reinterpret_cast<uint4*>(b);
    b += align256(tp * n_cols * 2 * kParts);
    w.xsum = reinterpret_cast<float*>(b);
    b += align256(tp * (n_cols / 32) * 4);
    w.xinv = reinterpret_cast<float*>(b);
    b += align256(tp * (n_cols / 256) * 4);
    w.ssq = reinterpret_cast<float*>(b);
    return w;
}

int64_t pad_tokens(int64_t n_tok) { return (n_tok + kTokTile - 1) / kTokTile * kTokTile; }

// The shape part of whether the split path applies (types with it, whole
// super-blocks a row, grid limits); alignment is checked at the call.
bool split_shape_ok(int dtype, int64_t n_cols, int64_t n_tok) {
    // Q6_K: 210-byte blocks, rows 16-byte aligned from 8 blocks; IQ4_XS: 136
    // bytes, from 2
    return (dtype == AERO_DTYPE_Q4_K || dtype == AERO_DTYPE_Q5_K || dtype == AERO_DTYPE_Q8_0 ||
            (dtype == AERO_DTYPE_Q6_K && n_cols % 2048 == 0) ||
            (dtype == AERO_DTYPE_IQ4_XS && n_cols % 512 == 0)) &&
           n_cols > 0 &&
           n_cols % 256 == 0 && n_cols / 256 <= 65535 && n_tok > 0 &&
           pad_tokens(n_tok) / kTokTile <= 65535 && pad_tokens(n_tok) <= 0x7fffffff;
}

// One folded pre-pass, then the GEMM launches: n_mat plain products
// y[m] = W_m x', or (w_up != null) one gate/up launch out = act(W x') * (U x').
struct SplitJob {
    int dtype;
    const float* x;
    const float* d;        // residual input (x' = x + d, stored to x_out) or null
    float* x_out;
    const float* norm_w;   // folded RMSNorm weight (null: ones)
    int norm;              // < 0: no norm; else 0 / AERO_NORM_UNIT_OFFSET
    float eps;
    int n_mat;
    const uint8_t* const* w;
    const uint8_t* w_up;   // gate/up form when non-null (w[0] is the gate)
    int act;
    const int64_t* n_rows;
    float* const* y;
    int64_t n_cols;
    int64_t rb;
    int64_t n_tok;
    void* ws;
    RopeFold rope;         // RoPE on the first rope.mats outputs (norm_matmul_rope)
    int64_t ws_bytes;      // room beyond split_ws_bytes lets few tokens split the columns
    const float* z;        // gated norm (gated_norm_matmul): the gate, norm_w tiled
    int64_t w_len;         //   with period w_len
    // x from the embedding rows of ids (attn_input): x is unused and x_out
    // receives the rows
    const uint8_t* emb;
    int emb_type;
    int64_t emb_bytes;
    int64_t vocab;
    const int32_t* ids;
    float emb_scale;
};

template <bool NORM, bool RESID, int EMB = 0>
bool launch_xsplit(const XsplitArgs& a, int64_t tp, hipStream_t s) {
    return launch("xsplit_kernel", xsplit_kernel<NORM, RESID, EMB>,
                  dim3((unsigned)(tp / 16), (unsigned)(a.n_cols / 256)), dim3(256), 0, s, a);
}

// The pre-pass reading x from the embedding rows (with the norm).
bool launch_xsplit_emb(int emb_type, const XsplitArgs& a, int64_t tp, hipStream_t s) {
    switch (emb_type) {
    case AERO_DTYPE_Q8_0: return launch_xsplit<true, false, AERO_DTYPE_Q8_0>(a, tp, s);
    case AERO_DTYPE_Q4_K: return launch_xsplit<true, false, AERO_DTYPE_Q4_K>(a, tp, s);
    case AERO_DTYPE_Q5_K: return launch_xsplit<true, false, AERO_DTYPE_Q5_K>(a, tp, s);
    case AERO_DTYPE_Q6_K: return launch_xsplit<true, false, AERO_DTYPE_Q6_K>(a, tp, s);
    case AERO_DTYPE_IQ4_XS: return launch_xsplit<true, false, AERO_DTYPE_IQ4_XS>(a, tp, s);
    default:
        set_error("split pre-pass: embedding type %d has no device dequant here", emb_type);
        return false;
    }
}

template <int TYPE, int MT>
void* pick_split_gemm_mt(int nt, int epi) {
    switch (epi) {
    case kEpiPlain:
        if (nt == 1 && MT == 4) return (void*)split_gemm_kernel<TYPE, 1, kEpiPlain, 4>;
        return nt == 4 && MT == 2 ? (void*)split_gemm_kernel<TYPE, 4, kEpiPlain, 2>
                                  : (void*)split_gemm_kernel<TYPE, 2, kEpiPlain, MT>;
    case AERO_ACT_SILU: return (void*)split_gemm_kernel<TYPE, 2, AERO_ACT_SILU, MT>;
    case AERO_ACT_GELU: return (void*)split_gemm_kernel<TYPE, 2, AERO_ACT_GELU, MT>;
    case AERO_ACT_GELU_TANH: return (void*)split_gemm_kernel<TYPE, 2, AERO_ACT_GELU_TANH, MT>;
    case AERO_ACT_IDENTITY: return (void*)split_gemm_kernel<TYPE, 2, AERO_ACT_IDENTITY, MT>;
    default: return nullptr;
    }
}

template <int TYPE>
void* pick_split_gemm(int nt, int epi, int mt) {
    if constexpr (TYPE == AERO_DTYPE_Q4_K || TYPE == AERO_DTYPE_Q6_K)
        if (mt == 4) return pick_split_gemm_mt<TYPE, 4>(nt, epi);
    // Q8_0: 64-token workgroups only with 16-row waves (32-row waves would
    // spill)
    if constexpr (TYPE == AERO_DTYPE_Q8_0)
        if (mt == 4 && nt == 1 && epi == kEpiPlain)
            return (void*)split_gemm_kernel<TYPE, 1, kEpiPlain, 4>;
    return pick_split_gemm_mt<TYPE, 2>(nt, epi);
}

// Column splits for a launch of base_wgs workgroups over n_sb super-blocks:
// for launches of fewer than 128 workgroups (half the CUs; the reduction is
// a launch more, which a launch of 224 workgroups does not repay: gate
// 14336 x 4096 at 64 tokens 40.4 us unsplit, 44.9 in two; AERO_HIP_TUNE
// gemm16_ksplit_below=N moves the limit),
// the largest divisor d of n_sb (at most 16) that keeps d * base_wgs within
// 512 workgroups and two super-blocks a split, when room holds the d
// partials of part_bytes each; 1 otherwise. Measured on MI355X, Q4_K, 16
// tokens, with the reduction: 4096 x 14336 108.6 -> 27.1 us (14 splits),
// 4096 x 4096 35.5 -> 15.5 (8), 14336 x 4096 37.6 -> 26.9 (4).
// AERO_HIP_TUNE gemm16_ksplit=N caps it (1: never split).
int pick_ksplit(int64_t base_wgs, int n_sb, int64_t part_bytes, int64_t room) {
    const int cap = std::min(kMaxSplits, tune("gemm16_ksplit", kMaxSplits));
    int ks = 1;
    if (base_wgs >= tune("gemm16_ksplit_below", 128)) return 1;
    for (int d = 2; d <= cap; ++d) {
        if (n_sb % d || n_sb / d < 2 || base_wgs * d > 512) continue;
        if (room < (int64_t)d * part_bytes) break;
        ks = d;
    }
    return ks;
}

// Bytes of the column-split partials beyond split_ws_bytes for a call over
// n_rows rows in all (gate/up: both matrices) of n_cols columns and n_tok
// tokens: the most pick_ksplit can use (0 when the call never splits).
int64_t split_partials_bytes(int64_t n_rows, int64_t n_cols, int64_t n_tok) {
    if (n_rows <= 0 || n_cols % 256 || n_tok <= 0) return 0;
    const int n_sb = (int)(n_cols / 256);
    // the fewest workgroups such a call can have (128 rows each), so the most splits
    const int64_t base = (n_rows + 127) / 128 * ((pad_tokens(n_tok) + kTokTile - 1) / kTokTile);
    const int ks = pick_ksplit(base, n_sb, 1, INT64_MAX);
    return ks > 1 ? (int64_t)ks * n_tok * n_rows * 4 : 0;
}

// Below 16 tokens the split GEMM beats the GEMV only with its columns split
// over more workgroups (MI355X, Q4_K, 4096 x 14336: 108.6 us unsplit at 16
// tokens or fewer, 27.1 split 14 ways; the GEMV 31.6 us at 4 tokens, 62.2 at
// 8): such a call takes the split path only when `room` (the workspace
// beyond the split GEMM's own) holds every partial it would write.
bool split_room_ok(int64_t n_rows, int64_t n_cols, int64_t n_tok, int64_t room) {
    if (n_tok >= 16) return true;
    return room >= split_partials_bytes(n_rows, n_cols, n_tok);
}

// Whether the per-head norm and RoPE of j.rope run in the split GEMM's
// epilogue: plain matrices of whole heads, each workgroup's rows (rows_wg)
// whole heads of D rows with D / (rows_wg / 8) lanes a head, an even rotated
// width, positions and inverse frequencies given, no column split.
bool split_rope_ok(const SplitJob& j, int rows_wg, int ks, int mt) {
    const RopeFold& r = j.rope;
    const int D = r.D, pairs = mt * rows_wg / 32;   // channel pairs a thread
    if (r.mats < 1 || j.w_up != nullptr || ks != 1 || r.mats > j.n_mat || r.mats > 2 ||
        r.pos == nullptr || r.inv == nullptr || D < 2 * pairs || D > rows_wg ||
        rows_wg % D || D % (2 * pairs) || r.rot() < 2 || r.rot() > D || r.rot() % 2 ||
        (r.mode != AERO_ROPE_NEOX && r.mode != AERO_ROPE_INTERLEAVED))
        return false;
    for (int m = 0; m < r.mats; ++m)
        if (j.n_rows[m] % D) return false;
    return true;
}

bool split_run(const SplitJob& j, hipStream_t s, bool* rope_done = nullptr) {
    if (rope_done != nullptr) *rope_done = false;
    const int64_t tp = pad_tokens(j.n_tok);
    const bool norm = j.norm >= 0;
    const SplitWs w = split_ws(j.ws, tp, j.n_cols);
    XsplitArgs a{j.x, j.d, j.x_out, j.norm_w, w.ssq, norm && (j.norm & AERO_NORM_UNIT_OFFSET),
                 (int)j.n_tok, (int)j.n_cols, w.xp, w.xsum, w.xinv, j.z, (int)j.w_len,
                 j.dtype == AERO_DTYPE_Q8_0   ? 1
                 : j.dtype == AERO_DTYPE_Q6_K ? 2
                 : j.dtype == AERO_DTYPE_IQ4_XS ? 3 : 0};
    if (j.emb != nullptr) {
        a.emb = j.emb;
        a.ids = j.ids;
        a.vocab = j.vocab;
        a.emb_rb = j.n_cols / dtype_block_values(j.emb_type) * dtype_block_bytes(j.emb_type);
        a.emb_scale = j.emb_scale;
    }
    const bool ok = j.emb != nullptr ? launch_xsplit_emb(j.emb_type, a, tp, s)
                    : norm ? (j.d ? launch_xsplit<true, true>(a, tp, s)
                                  : launch_xsplit<true, false>(a, tp, s))
                           : (j.d ? launch_xsplit<false, true>(a, tp, s)
                                  : launch_xsplit<false, false>(a, tp, s));
    if (!ok) return false;
    const bool gu = j.w_up != nullptr;
    // rows a wave: 32 (two waves a SIMD); 64 (AERO_HIP_TUNE gemm16_nt=4) runs
    // one wave a SIMD and measured slower on MI355X at every prefill shape
    int nt = gu ? 2 : (tune("gemm16_nt", 2) == 4 ? 4 : 2);
    const int epi = gu ? j.act : kEpiPlain;
    // one launch for every matrix: row tiles of matrix m follow those of m-1
    SplitParams p{};
    const int n_mat = gu ? 1 : j.n_mat;
    p.n_mat = n_mat;
    auto count_tiles = [&](int rows_wg) {
        int64_t t = 0;
        for (int m = 0; m < n_mat; ++m) t += (j.n_rows[m] + rows_wg - 1) / rows_wg;
        return t;
    };
    int rows_wg = gu ? 64 : 64 * nt;
    int64_t tiles = count_tiles(rows_wg);
    // 16 rows a wave and 64 tokens a workgroup for plain Q6_K and Q8_0
    // launches that have two such workgroups a CU but not two of 32-row waves
    // (4096-row matrices at 512 tokens): the decode of a weight is then shared
    // by twice the tokens. Measured on MI355X at 512 tokens, 4096 x 14336:
    // Q6_K 325.8 -> 286.3 us, Q8_0 280.7 -> 270.2 (4096 x 4096 82.4 -> 77.5);
    // Q4_K 228.6 -> 255.2 (its x reads from LDS, twice as many a matrix step,
    // cost more than the decode saved), so Q4_K keeps 32 rows (AERO_HIP_TUNE
    // gemm16_nt1=1 / 0 forces / forbids).
    const bool kq = j.dtype == AERO_DTYPE_Q4_K || j.dtype == AERO_DTYPE_Q6_K;
    const bool nt1_ok = kq || j.dtype == AERO_DTYPE_Q8_0;
    const int nt1 = tune("gemm16_nt1", j.dtype == AERO_DTYPE_Q4_K ? 0 : 1);
    // (not where it would lose a per-head epilogue the 32-row waves take)
    const bool keeps_rope = j.rope.mats == 0 || split_rope_ok(j, 64, 1, 4) ||
                            !split_rope_ok(j, 128, 1, 2);
    if (!gu && nt == 2 && nt1_ok && tp % 64 == 0 && nt1 == 1 && keeps_rope &&
        tiles * (tp / 64) < 2 * cu_count() && count_tiles(64) * (tp / 64) >= 2 * cu_count()) {
        nt = 1;
        rows_wg = 64;
        tiles = count_tiles(64);
    }
    if (tiles > 0x7fffffff) {
        set_error("split GEMM: too many rows");
        return false;
    }
    {
        int64_t t0 = 0;
        for (int m = 0; m < n_mat; ++m) {
            p.w[m] = j.w[m];
            p.y[m] = j.y[m];
            p.n_rows[m] = j.n_rows[m];
            p.tile0[m] = (int)t0;
            t0 += (j.n_rows[m] + rows_wg - 1) / rows_wg;
        }
    }
    for (int m = n_mat; m <= kMaxMats; ++m) p.tile0[m] = (int)tiles;
    if (tiles == 0) return true;
    p.xp = w.xp;
    p.xsum = w.xsum;
    p.xinv = w.xinv;
    p.n_cols = (int)j.n_cols;
    p.rb = j.rb;
    p.n_tok = (int)j.n_tok;
    p.w2 = gu ? j.w_up : nullptr;
    p.ssq = norm ? w.ssq : nullptr;
    p.eps = j.eps;
    // few tokens leave workgroups idle: split the columns when the
    // workspace holds the partials
    int64_t r_all = 0;
    for (int m = 0; m < n_mat; ++m) {
        p.roff[m] = r_all;
        r_all += j.n_rows[m];
    }
    if (gu) r_all = 2 * j.n_rows[0];
    const int64_t base_wgs = tiles * (tp / kTokTile);
    const int n_sb = (int)(j.n_cols / 256);
    const int64_t part_off = split_ws_bytes(tp, j.n_cols, norm);
    const int ks = pick_ksplit(base_wgs, n_sb, j.n_tok * r_all * 4, j.ws_bytes - part_off);
    p.ksplit = ks;
    p.r_all = r_all;
    p.part = ks > 1 ? reinterpret_cast<float*>(static_cast<uint8_t*>(j.ws) + part_off) : nullptr;
    // 64 tokens a workgroup (each decoded weight serving twice the matrix
    // steps) for Q4_K and Q6_K (the others would spill registers) where the
    // launch still has two workgroups a CU (512 tokens of gate/up or of a
    // 14336-row matrix), or one on (nearly) every CU instead of two (o and
    // down at 4096 rows and 512 tokens: Q4_K 4096 x 4096 68.0 -> 66.4 us,
    // 4096 x 14336 232.5 -> 220.9 us on MI355X); not where one CU in two
    // would hold a second (q/k/v, 6144 rows: 86.9 -> 90.1 us). AERO_HIP_TUNE
    // gemm16_mt=2 keeps 32, gemm16_mt=4 takes 64 wherever the shape allows.
    const int mt_knob = tune("gemm16_mt", 0);
    const int64_t w64 = tiles * (tp / 64), cus = cu_count();
    const int mt = nt == 1 || (kq && nt == 2 && ks == 1 && tp % 64 == 0 && mt_knob != 2 &&
                               (mt_knob == 4 || w64 >= 2 * cus ||
                                (w64 <= cus && w64 >= cus - cus / 8)))
                       ? 4 : 2;
    void* kp = j.dtype == AERO_DTYPE_Q5_K   ? pick_split_gemm<AERO_DTYPE_Q5_K>(nt, epi, mt)
               : j.dtype == AERO_DTYPE_Q8_0 ? pick_split_gemm<AERO_DTYPE_Q8_0>(nt, epi, mt)
               : j.dtype == AERO_DTYPE_Q6_K ? pick_split_gemm<AERO_DTYPE_Q6_K>(nt, epi, mt)
               : j.dtype == AERO_DTYPE_IQ4_XS ? pick_split_gemm<AERO_DTYPE_IQ4_XS>(nt, epi, mt)
                                            : pick_split_gemm<AERO_DTYPE_Q4_K>(nt, epi, mt);
    if (kp == nullptr) {
        set_error("split GEMM: unknown activation %d", j.act);
        return false;
    }
    auto k = reinterpret_cast<void (*)(SplitParams)>(kp);
    if (split_rope_ok(j, rows_wg, ks, mt)) {
        p.rope_mats = j.rope.mats;
        p.rope_D = j.rope.D;
        p.rope_rot = j.rope.rot();
        p.rope_mode = j.rope.mode;
        p.pos = j.rope.pos;
        p.rinv = j.rope.inv;
        p.qk_w[0] = j.rope.qk_w[0];
        p.qk_w[1] = j.rope.qk_w[1];
        p.qk_eps = j.rope.qk_eps;
        p.qk_flags = j.rope.qk_flags;
        if (rope_done != nullptr) *rope_done = true;
    }
    if (!launch("split_gemm_kernel", k,
                dim3((unsigned)tiles, (unsigned)(tp / (16 * mt)), (unsigned)ks), dim3(256), 0, s,
                p))
        return false;
    if (ks == 1) return true;
    ReduceArgs ra{};
    ra.part = p.part;
    ra.ksplit = ks;
    ra.n_tok = (int)j.n_tok;
    ra.r_all = r_all;
    ra.ssq = p.ssq;
    ra.n_sb = n_sb;
    ra.n_cols = (int)j.n_cols;
    ra.eps = j.eps;
    ra.n_mat = n_mat;
    for (int m = 0; m < n_mat; ++m) {
        ra.y[m] = j.y[m];
        ra.n_rows[m] = j.n_rows[m];
        ra.roff[m] = p.roff[m];
    }
    for (int m = n_mat; m <= kMaxMats; ++m) ra.roff[m] = r_all;
    const int64_t n_out = gu ? r_all / 2 : r_all;
    const dim3 rg((unsigned)((n_out + 255) / 256), (unsigned)j.n_tok);
    switch (epi) {
    case kEpiPlain:
        return launch("split_reduce_kernel", split_reduce_kernel<kEpiPlain>, rg, dim3(256), 0, s, ra);
    case AERO_ACT_SILU:
        return launch("split_reduce_kernel", split_reduce_kernel<AERO_ACT_SILU>, rg, dim3(256), 0, s,
                      ra);
    case AERO_ACT_GELU:
        return launch("split_reduce_kernel", split_reduce_kernel<AERO_ACT_GELU>, rg, dim3(256), 0, s,
                      ra);
    case AERO_ACT_GELU_TANH:
        return launch("split_reduce_kernel", split_reduce_kernel<AERO_ACT_GELU_TANH>, rg, dim3(256),
                      0, s, ra);
    default:
        return launch("split_reduce_kernel", split_reduce_kernel<AERO_ACT_IDENTITY>, rg, dim3(256),
                      0, s, ra);
    }
}

}  // namespace

// The fewest tokens with which a call over n_rows rows (every matrix of the
// call) of n_cols columns takes the split GEMM rather than the GEMV (the
// shape and a workspace permitting). The GEMV converts and multiply-adds
// each weight once per token and streams the matrix once per 4 tokens; the
// split GEMM decodes each weight once per 32 tokens and runs the products
// on the matrix cores (small grids split over columns). Measured on MI355X,
// Q4_K, split / GEMV, µs: 14336 x 4096 at 4 tokens 24.9 / 23.2, 5: 25.1 /
// 31.0; 4096 x 4096 at 6 tokens 14.5 / 14.2, 8: 14.6 / 17.6; 1024 x 4096
// at 8 tokens 13.3 / 10.6, 12: 13.4 / 15.8. So: 5 tokens from 32M
// weights, 7 from 8M, 10 from 2M, 16 below. Rows longer than one 4096-column
// GEMV step run as GEMV launches of two tokens at most, so there 4 tokens
// from 32M weights: 4096 x 14336 at 4 tokens 25.9 / 31.6 (Q8_0 33.3 /
// 39.7), at 3 25.7 / 26.1. AERO_HIP_TUNE gemm_split_min_tokens=N sets one
// threshold instead.
int split_min_tokens(int64_t n_rows, int64_t n_cols) {
    const int fixed = tune("gemm_split_min_tokens", 0);
    if (fixed > 0) return fixed;
    const int64_t weights = n_rows * n_cols;
    if (n_cols > 4096 && weights >= ((int64_t)32 << 20)) return 4;
    return weights >= ((int64_t)32 << 20) ? 5
                                          : weights >= ((int64_t)8 << 20) ? 7
                                                                          : weights >= ((int64_t)2 << 20) ? 10 : 16;
}

bool split_tokens_ok(int64_t n_tok, int64_t n_rows, int64_t n_cols) {
    return n_tok >= split_min_tokens(n_rows, n_cols);
}

// Workspace bytes of the split-x GEMM for n_tok tokens of n_cols (0 when the
// type or shape has no split path): the x parts, the sub-block sums and the
// inverse scales.
int64_t split_gemm_workspace(int dtype, int64_t n_cols, int64_t n_tok) {
    if (!split_shape_ok(dtype, n_cols, n_tok)) return 0;
    return split_ws_bytes(pad_tokens(n_tok), n_cols, false);
}

// Called by the matmul entry after its argument checks; false (without an
// error) when this path does not apply, so the caller takes another GEMM.
bool split_gemm_dev(int dtype, const uint8_t* w, const float* x, float* y, int64_t n_rows,
                    int64_t n_cols, int64_t rb, int64_t n_tok, void* ws, int64_t ws_bytes,
                    hipStream_t s, bool* ran) {
    *ran = false;
    const int64_t need = split_gemm_workspace(dtype, n_cols, n_tok);
    if (need == 0 || ws == nullptr || ws_bytes < need || !aligned16(w) || rb % 16 != 0 ||
        !aligned16(ws) || !tune("gemm16", 1))
        return true;
    if (!split_room_ok(n_rows, n_cols, n_tok, ws_bytes - need)) return true;
    SplitJob j{dtype, x, nullptr, nullptr, nullptr, -1, 0.f, 1, &w, nullptr, 0, &n_rows, &y,
               n_cols, rb, n_tok, ws, {}, ws_bytes};
    if (!split_run(j, s)) return false;
    *ran = true;
    return true;
}

// the quantised GEMV / GEMM dispatch and the fused decode GEMVs (gemv.hip)
bool gemv_dev(int dtype, const uint8_t* w, int64_t w_bytes, const float* x, float* y,
              int64_t n_rows, int64_t n_cols, int64_t n_tok, hipStream_t s, void* ws,
              int64_t ws_bytes);
bool lanes64_ok(int dtype, const uint8_t* w, int64_t rb, int64_t n_rows, int64_t w_bytes);
bool gemv_fused_dev(int dtype, bool pair, int n_mat, const uint8_t* const* w,
                    const int64_t* w_bytes, const int64_t* n_rows, float* const* y,
                    const float* x, const float* norm_w, float eps, int norm, int act,
                    int64_t n_cols, int64_t n_tok, hipStream_t s, const float* d, float* xo,
                    const RopeFold* rope);
bool gemv_gated_dev(int dtype, const uint8_t* w, int64_t w_bytes, int64_t n_rows, float* y,
                    const float* x, const float* z, const float* norm_w, int64_t w_len,
                    float eps, int64_t n_cols, int64_t n_tok, hipStream_t s);

// ------------------------------------------------ allocation-free matmul
// The split GEMM's workspace in a file-scope device array, for callers that
// cannot allocate (code under HIP graph capture, serving loops, harnesses
// that forbid hipMalloc). Each GPU the library runs on holds its own copy
// of kScratchBytes until the process ends. The array's name is a host-side
// stand-in; its device address on the current GPU comes from
// hipGetSymbolAddress, taken once per device and kept.
constexpr int64_t kScratchBytes = 32ll << 20;
constexpr int kScratchDevices = 64;
static __device__ __align__(256) uint8_t scratch[kScratchBytes];

namespace {

std::mutex g_scratch_mu;
void* g_scratch_ptr[kScratchDevices] = {};
// The last call's stream on each device and an event recorded after it, so
// a call on another stream while that one may still run is refused rather
// than left to race on the shared array.
struct ScratchUse {
    hipEvent_t done = nullptr;
    hipStream_t stream = nullptr;
    bool used = false;
};
ScratchUse g_scratch_use[kScratchDevices];

// The current device's scratch address, looked up on its first use.
void* scratch_ptr() {
    int dev = -1;
    if (!hip_ok(hipGetDevice(&dev), "hipGetDevice")) return nullptr;
    if (dev < 0 || dev >= kScratchDevices) {
        set_error("matmul_noalloc: device %d outside the %d the scratch table holds", dev,
                  kScratchDevices);
        return nullptr;
    }
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    if (g_scratch_ptr[dev] == nullptr) {
        void* p = nullptr;
        if (!hip_ok(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)), "hipGetSymbolAddress(scratch)"))
            return nullptr;
        g_scratch_ptr[dev] = p;
    }
    return g_scratch_ptr[dev];
}

}  // namespace

int64_t matmul_scratch_bytes() { return kScratchBytes; }

bool matmul_noalloc(int dtype, const uint8_t* w, int64_t w_bytes, const float* x, float* y,
                    int64_t n_rows, int64_t n_cols, int64_t n_tok, hipStream_t s) {
    const int64_t need = split_gemm_workspace(dtype, n_cols, n_tok);
    if (need > kScratchBytes) {
        set_error("matmul_noalloc: %lld tokens of %lld columns need %lld bytes of scratch, "
                  "more than the %lld the library holds a device; use aero_hip_matmul with a "
                  "workspace", (long long)n_tok, (long long)n_cols, (long long)need,
                  (long long)kScratchBytes);
        return false;
    }
    void* ws = nullptr;
    if (need > 0) {
        ws = scratch_ptr();
        if (ws == nullptr) return false;
    }
    if (need == 0)
        return gemv_dev(dtype, w, w_bytes, x, y, n_rows, n_cols, n_tok, s, nullptr, 0);
    // Overlap check (eager calls only: a call recorded into a plan or a HIP
    // graph runs later, so there is nothing to compare it with now): a call
    // on a stream other than the last call's, while that call may still
    // run, is refused.
    hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
    const bool eager = recording_plan() == nullptr &&
                       hipStreamIsCapturing(s, &cap) == hipSuccess &&
                       cap == hipStreamCaptureStatusNone;
    int dev = 0;
    if (!hip_ok(hipGetDevice(&dev), "hipGetDevice")) return false;
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    ScratchUse& u = g_scratch_use[dev];
    if (eager && u.used && u.stream != s) {
        const hipError_t q = hipEventQuery(u.done);
        if (q == hipErrorNotReady) {
            set_error("matmul_noalloc: the previous call on this GPU (another stream) may still "
                      "be using its scratch; order the calls on one stream or wait for it");
            return false;
        }
        if (!hip_ok(q, "hipEventQuery")) return false;
    }
    // the whole array is the call's room: a few-token call writes its
    // column splits' partials there too (they are far smaller than the
    // array: 14 x 16 tokens x 4096 rows x 4 bytes = 3.7 MB at most)
    if (!gemv_dev(dtype, w, w_bytes, x, y, n_rows, n_cols, n_tok, s, ws, kScratchBytes))
        return false;
    if (eager) {
        if (u.done == nullptr &&
            !hip_ok(hipEventCreateWithFlags(&u.done, hipEventDisableTiming), "hipEventCreate"))
            return false;
        if (!hip_ok(hipEventRecord(u.done, s), "hipEventRecord")) return false;
        u.stream = s;
        u.used = true;
    }
    return true;
}

// ------------------------------------ norm (and residual) folded into GEMMs
// The prefill forms of the model loop's "norm -> projections" and "norm ->
// gate/up -> act" steps (src/model.cpp:166-178,244-245,279-282): the split
// path folds the residual add and the RMSNorm into the x pre-pass and the
// act-mul into the GEMM epilogue (from the token counts split_tokens_ok
// gives). With fewer tokens, rows the lane GEMVs take go to the fused
// decode GEMVs (every matrix, or gate/up with the act-mul in
// the epilogue, in one launch): at one token (two without a residual) with
// the norm and the residual add (x_out apart from x and d) in their
// prologue, else after an add + norm pass into the workspace. Other types and shapes run the same
// steps as separate launches (add+norm into the workspace, the library
// GEMM, the act-mul), so every type and token count is accepted.
// Sized for the path the shape takes with 16-byte aligned weights (as the
// GGUF loader and the ops allocate them); a call whose weights are not
// aligned takes the separate launches and refuses, with the size it needs,
// a workspace too small for them.
int64_t norm_matmul_workspace(int dtype, int64_t n_cols, int64_t n_ff, int64_t n_tok) {
    if (n_cols <= 0 || n_tok <= 0 || n_ff < 0) return 0;
    const int64_t sep = align256(n_tok * n_cols * 4) + (n_ff > 0 ? align256(n_tok * n_ff * 4) : 0);
    // the rows (unknown here) decide the path between the largest and the
    // smallest threshold: room for both
    if (!split_shape_ok(dtype, n_cols, n_tok) ||
        n_tok < split_min_tokens((int64_t)1 << 40, 1 << 20))
        return sep;
    const int64_t spl = split_ws_bytes(pad_tokens(n_tok), n_cols, true);
    return n_tok >= split_min_tokens(1, 1) ? spl : std::max(spl, sep);
}

namespace {

// The fused decode GEMVs take the call's matrices in one launch (a group of
// up to 4 tokens): few tokens, matrices the 64-column lane kernels take
// (lanes64_ok: 16-byte aligned rows of whole 16 bytes, Q8_0 also of 8), at
// most 3 matrices (or the gate/up pair).
bool fused_gemv_rows_ok(const SplitJob& j, bool gu, const int64_t* w_bytes) {
    if (j.n_tok >= tune("gemm_min_tokens", 32) || (!gu && j.n_mat > 4) ||
        !tune("gemv_lanes64", 1) || !tune("fused_gemv", 1))
        return false;
    for (int m = 0; m < (gu ? 1 : j.n_mat); ++m)
        if (!lanes64_ok(j.dtype, j.w[m], j.rb, j.n_rows[m], w_bytes[m])) return false;
    return !gu || lanes64_ok(j.dtype, j.w_up, j.rb, j.n_rows[0], w_bytes[0]);
}

// ... and also the norm (and residual add) in their prologue: every
// workgroup sums x^2 of its tokens over the row (and loads d), which pays
// at few tokens a launch. Measured on MI355X at the Llama-3-8B decode
// shapes: the norm alone up to 2 tokens, the add + norm at 1; beyond that
// the add + norm pass plus the GEMV on h is as fast or faster. A residual
// add only with a norm and an x_out apart from x and d (one workgroup
// stores x + d while the others read x and d).
bool fused_prologue_ok(const SplitJob& j) {
    if (j.n_tok > tune("fused_norm_max_tokens", j.d ? 1 : 2)) return false;
    if (j.d == nullptr) return true;
    const uintptr_t nb = (uintptr_t)(j.n_tok * j.n_cols * 4);
    auto apart = [nb](const void* a, const void* b) {
        const uintptr_t ua = reinterpret_cast<uintptr_t>(a), ub = reinterpret_cast<uintptr_t>(b);
        return ua + nb <= ub || ub + nb <= ua;
    };
    return j.norm >= 0 && apart(j.x_out, j.x) && apart(j.x_out, j.d);
}

// One fused-GEMV launch per token group over x (norm / residual per the
// arguments) for the call's matrices, or its gate/up pair with the act-mul;
// the RoPE of j.rope in its epilogue when that folds (*rope_done).
bool fused_gemv_run(const SplitJob& j, bool gu, const int64_t* w_bytes, const float* x,
                    int norm, const float* d, hipStream_t s, bool* rope_done) {
    const uint8_t* w[3] = {j.w[0], gu ? j.w_up : nullptr, nullptr};
    int64_t wb[3] = {w_bytes[0], w_bytes[0], 0}, nr[3] = {j.n_rows[0], j.n_rows[0], 0};
    float* y[3] = {j.y[0], j.y[0], nullptr};
    if (!gu) {
        for (int m = 1; m < j.n_mat; ++m) {
            w[m] = j.w[m];
            wb[m] = w_bytes[m];
            nr[m] = j.n_rows[m];
            y[m] = j.y[m];
        }
    }
    const bool fold = j.rope.mats > 0 && rope_fold_ok(j.rope, gu, j.n_mat, j.n_rows);
    if (!gemv_fused_dev(j.dtype, gu, gu ? 2 : j.n_mat, w, wb, nr, y, x, j.norm_w, j.eps, norm,
                        gu ? j.act : AERO_ACT_IDENTITY, j.n_cols, j.n_tok, s, d,
                        d ? j.x_out : nullptr, fold ? &j.rope : nullptr))
        return false;
    *rope_done = fold;
    return true;
}

// The embedding rows as x: checks, and the gather into x_out first where
// the split pre-pass or the gather + norm pass cannot read the table
// themselves (no norm, a type without their dequant, rows beyond 16384
// values); j then reads x from x_out.
bool emb_input(SplitJob& j, hipStream_t s) {
    const int64_t ebv = dtype_block_values(j.emb_type), ebb = dtype_block_bytes(j.emb_type);
    if (ebv <= 0 || j.ids == nullptr || j.x_out == nullptr || j.d != nullptr ||
        j.z != nullptr || j.vocab <= 0 || j.n_cols <= 0 || j.n_cols % ebv != 0 ||
        j.emb_bytes < j.vocab * (j.n_cols / ebv) * ebb || !aligned16(j.x_out)) {
        set_error("attn_input: bad embedding arguments (type %d, vocab %lld, %lld bytes for "
                  "%lld columns; ids and a 16-byte aligned x_out needed, no residual input)",
                  j.emb_type, (long long)j.vocab, (long long)j.emb_bytes, (long long)j.n_cols);
        return false;
    }
    const bool direct = j.norm >= 0 && j.n_cols <= 8 * 8 * 256 &&
                        (j.emb_type == AERO_DTYPE_Q8_0 || j.emb_type == AERO_DTYPE_Q4_K ||
                         j.emb_type == AERO_DTYPE_Q5_K || j.emb_type == AERO_DTYPE_Q6_K ||
                         j.emb_type == AERO_DTYPE_IQ4_XS);
    if (direct || j.n_tok == 0) return true;
    if (!aero_hip_embed_gather(j.emb_type, j.emb, j.emb_bytes, j.vocab, j.n_cols, j.ids,
                               j.n_tok, j.emb_scale, j.x_out, nullptr, s))
        return false;
    j.x = j.x_out;
    j.emb = nullptr;
    return true;
}

bool norm_matmul_run(SplitJob j, const int64_t* w_bytes, int64_t n_ff, int64_t ws_bytes,
                     hipStream_t s, bool* rope_done) {
    *rope_done = false;
    j.ws_bytes = ws_bytes;
    const int64_t bv = dtype_block_values(j.dtype), bb = dtype_block_bytes(j.dtype);
    const bool gu = j.w_up != nullptr;
    if (j.emb != nullptr && !emb_input(j, s)) return false;
    const bool emb = j.emb != nullptr;   // x from the table (the split pre-pass or gather + norm)
    if (bv <= 0 || (j.x == nullptr && !emb) || j.n_cols <= 0 || j.n_tok < 0 ||
        j.n_cols % bv != 0 ||
        j.n_cols > (int64_t)1 << 30 || j.n_tok > 0x7fffffff || (j.d && !j.x_out) ||
        j.norm > AERO_NORM_UNIT_OFFSET || j.n_mat < 1 || j.n_mat > 4 ||
        (j.norm_w && !aligned16(j.norm_w)) || (!emb && !aligned16(j.x)) ||
        (j.d && !aligned16(j.d)) ||
        (j.x_out && !aligned16(j.x_out))) {
        set_error("norm_matmul: bad arguments (n_cols=%lld n_tok=%lld n_mat=%d norm=%d; x, d, "
                  "x_out, norm_w 16-byte aligned, n_cols a multiple of %lld, d needs x_out)",
                  (long long)j.n_cols, (long long)j.n_tok, j.n_mat, j.norm, (long long)bv);
        return false;
    }
    if (j.z != nullptr &&
        (gu || j.n_mat != 1 || j.d != nullptr || j.norm != 0 || j.norm_w == nullptr ||
         !aligned16(j.z) || j.w_len < 16 || j.w_len % 16 || j.n_cols % j.w_len)) {
        set_error("gated_norm_matmul: one matrix, a 16-byte aligned gate and a norm weight whose "
                  "length is a multiple of 16 dividing the row (w_len=%lld, n_cols=%lld)",
                  (long long)j.w_len, (long long)j.n_cols);
        return false;
    }
    j.rb = (j.n_cols / bv) * bb;
    for (int m = 0; m < (gu ? 1 : j.n_mat); ++m) {
        if (j.w[m] == nullptr || j.y[m] == nullptr || j.n_rows[m] < 0 ||
            w_bytes[m] < j.n_rows[m] * j.rb) {
            set_error("norm_matmul: matrix %d: null, or w_bytes %lld < n_rows*row_bytes %lld", m,
                      (long long)w_bytes[m], (long long)(j.n_rows[m] * j.rb));
            return false;
        }
    }
    if (j.n_tok == 0) return true;
    // the path decides the workspace: the split GEMM's parts, or the separate
    // launches' h (and up) buffers
    int64_t all_rows = gu ? 2 * n_ff : 0;
    for (int m = 0; m < (gu ? 0 : j.n_mat); ++m) all_rows += j.n_rows[m];
    bool split = split_shape_ok(j.dtype, j.n_cols, j.n_tok) &&
                 split_tokens_ok(j.n_tok, all_rows, j.n_cols) && j.rb % 16 == 0 &&
                 tune("gemm16", 1) &&
                 split_room_ok(all_rows, j.n_cols, j.n_tok,
                               ws_bytes - split_ws_bytes(pad_tokens(j.n_tok), j.n_cols, true));
    for (int m = 0; m < (gu ? 1 : j.n_mat); ++m) split = split && aligned16(j.w[m]);
    if (gu) split = split && aligned16(j.w_up);
    const bool fused = !split && fused_gemv_rows_ok(j, gu, w_bytes);
    if (fused && j.z != nullptr && j.n_tok <= 2)   // the gated norm in the GEMV's prologue
        return gemv_gated_dev(j.dtype, j.w[0], w_bytes[0], j.n_rows[0], j.y[0], j.x, j.z,
                              j.norm_w, j.w_len, j.eps, j.n_cols, j.n_tok, s);
    if (fused && j.z == nullptr && !emb && fused_prologue_ok(j))
        return fused_gemv_run(j, gu, w_bytes, j.x, j.norm, j.d, s, rope_done);
    const int64_t need = split ? split_ws_bytes(pad_tokens(j.n_tok), j.n_cols, true)
                               : align256(j.n_tok * j.n_cols * 4) +
                                     (gu && !fused ? align256(j.n_tok * n_ff * 4) : 0);
    if (j.ws == nullptr || ws_bytes < need || !aligned16(j.ws)) {
        set_error("norm_matmul: workspace of %lld bytes (16-byte aligned) needed, %lld given",
                  (long long)need, (long long)ws_bytes);
        return false;
    }
    if (split) return split_run(j, s, rope_done);

    // separate launches: x' (= x + d, or the embedding rows) and h =
    // rmsnorm(x') in the workspace;
    // without a norm the add still runs through the add + norm kernel (its h
    // is left unused) and h is x'
    const float* h = j.d ? j.x_out : j.x;
    float* hb = static_cast<float*>(j.ws);
    if (emb) {   // with a norm (emb_input gathered the other cases)
        if (!aero_hip_embed_rmsnorm(j.emb_type, j.emb, j.emb_bytes, j.vocab, j.n_cols, j.ids,
                                    j.n_tok, j.emb_scale, j.x_out, j.norm_w, j.eps, j.norm, hb,
                                    nullptr, s))
            return false;
        h = hb;
    } else if (j.z != nullptr) {
        if (!aero_hip_gated_rmsnorm_silu(j.x, j.z, j.norm_w, j.w_len, hb, j.n_tok, j.n_cols,
                                         j.n_cols, j.eps, s))
            return false;
        h = hb;
    } else if (j.d) {
        if (!aero_hip_add_rmsnorm(j.x, j.d, j.x_out, j.norm_w, hb, j.n_tok, j.n_cols, j.eps,
                                  j.norm >= 0 ? j.norm : 0, s))
            return false;
        if (j.norm >= 0) h = hb;
    } else if (j.norm >= 0) {
        if (!aero_hip_rmsnorm(j.x, j.norm_w, hb, j.n_tok, j.n_cols, j.eps, j.norm, s))
            return false;
        h = hb;
    }
    // the matrices (or the gate/up pair with its act-mul) in one fused launch
    // on h when their rows allow it
    if (fused) return fused_gemv_run(j, gu, w_bytes, h, -1, nullptr, s, rope_done);
    if (!gu) {
        for (int m = 0; m < j.n_mat; ++m)
            if (!gemv_dev(j.dtype, j.w[m], w_bytes[m], h, j.y[m], j.n_rows[m], j.n_cols,
                          j.n_tok, s, nullptr, 0))
                return false;
        return true;
    }
    float* ub = reinterpret_cast<float*>(static_cast<uint8_t*>(j.ws) +
                                         align256(j.n_tok * j.n_cols * 4));
    return gemv_dev(j.dtype, j.w[0], w_bytes[0], h, j.y[0], n_ff, j.n_cols, j.n_tok, s,
                    nullptr, 0) &&
           gemv_dev(j.dtype, j.w_up, w_bytes[0], h, ub, n_ff, j.n_cols, j.n_tok, s, nullptr,
                    0) &&
           aero_hip_act_mul(j.act, j.y[0], ub, j.y[0], j.n_tok * n_ff, s) == 1;
}

}  // namespace

}  // namespace aero

extern "C" {

int aero_hip_split_ok(int dtype, int64_t n_cols, int64_t n_rows, int64_t n_tok) {
    const int64_t bv = aero::dtype_block_values(dtype), bb = aero::dtype_block_bytes(dtype);
    if (bv <= 1 || n_cols <= 0 || n_rows <= 0 || n_tok <= 0 || n_cols % bv != 0) return 0;
    const int64_t rb = (n_cols / bv) * bb;
    return aero::split_shape_ok(dtype, n_cols, n_tok) && rb % 16 == 0 &&
                   aero::split_tokens_ok(n_tok, n_rows, n_cols) && aero::tune("gemm16", 1)
               ? 1 : 0;
}

int64_t aero_hip_split_partials_bytes(int64_t n_rows, int64_t n_cols, int64_t n_tok) {
    return aero::split_partials_bytes(n_rows, n_cols, n_tok);
}

int64_t aero_hip_norm_matmul_workspace(int dtype, int64_t n_cols, int64_t n_ff, int64_t n_tok) {
    return aero::norm_matmul_workspace(dtype, n_cols, n_ff, n_tok);
}

int aero_hip_norm_matmul(int dtype, int n_mat, const uint8_t* const* w, const int64_t* w_bytes,
                         const int64_t* n_rows, float* const* y, const float* x, const float* d,
                         float* x_out, const float* norm_w, float eps, int norm, int64_t n_cols,
                         int64_t n_tok, void* ws, int64_t ws_bytes, void* stream) {
    if (w == nullptr || w_bytes == nullptr || n_rows == nullptr || y == nullptr) {
        aero::set_error("norm_matmul: null matrix arrays");
        return 0;
    }
    aero::SplitJob j{dtype, x, d, x_out, norm_w, norm, eps, n_mat, w, nullptr, 0, n_rows, y,
                     n_cols, 0, n_tok, ws, {}};
    bool rope_done;
    return aero::norm_matmul_run(j, w_bytes, 0, ws_bytes, (hipStream_t)stream, &rope_done) ? 1
                                                                                           : 0;
}

int aero_hip_gated_norm_matmul(int dtype, const uint8_t* w, int64_t w_bytes, int64_t n_rows,
                               float* y, const float* x, const float* z, const float* norm_w,
                               int64_t w_len, float eps, int64_t n_cols, int64_t n_tok,
                               void* ws, int64_t ws_bytes, void* stream) {
    aero::clear_error();
    aero::SplitJob j{dtype, x, nullptr, nullptr, norm_w, 0, eps, 1, &w, nullptr, 0, &n_rows, &y,
                     n_cols, 0, n_tok, ws, {}};
    j.z = z;
    j.w_len = w_len;
    if (z == nullptr) {
        aero::set_error("gated_norm_matmul: null gate");
        return 0;
    }
    bool rope_done;
    return aero::norm_matmul_run(j, &w_bytes, 0, ws_bytes, (hipStream_t)stream, &rope_done) ? 1
                                                                                            : 0;
}

int aero_hip_norm_matmul_rope(int dtype, int n_mat, const uint8_t* const* w,
                              const int64_t* w_bytes, const int64_t* n_rows, float* const* y,
                              const float* x, const float* d, float* x_out, const float* norm_w,
                              float eps, int norm, int64_t n_cols, int64_t n_tok, int n_rope,
                              int64_t head_dim, int rope_mode, const int32_t* pos,
                              const float* inv_freq, void* ws, int64_t ws_bytes, void* stream) {
    if (w == nullptr || w_bytes == nullptr || n_rows == nullptr || y == nullptr) {
        aero::set_error("norm_matmul_rope: null matrix arrays");
        return 0;
    }
    if (n_rope < 1 || n_rope > 2 || n_rope > n_mat || head_dim < 2 || head_dim % 2 ||
        head_dim > 512 || pos == nullptr || inv_freq == nullptr ||
        (rope_mode != AERO_ROPE_NEOX && rope_mode != AERO_ROPE_INTERLEAVED)) {
        aero::set_error("norm_matmul_rope: bad RoPE arguments (n_rope=%d of %d matrices, "
                        "head_dim=%lld, mode=%d, pos and inv_freq required)", n_rope, n_mat,
                        (long long)head_dim, rope_mode);
        return 0;
    }
    for (int m = 0; m < n_rope; ++m) {
        if (n_rows[m] % head_dim) {
            aero::set_error("norm_matmul_rope: matrix %d has %lld rows, not whole heads of %lld",
                            m, (long long)n_rows[m], (long long)head_dim);
            return 0;
        }
    }
    aero::SplitJob j{dtype, x, d, x_out, norm_w, norm, eps, n_mat, w, nullptr, 0, n_rows, y,
                     n_cols, 0, n_tok, ws,
                     {n_rope, (int)head_dim, rope_mode, pos, inv_freq}};
    bool rope_done = false;
    if (!aero::norm_matmul_run(j, w_bytes, 0, ws_bytes, (hipStream_t)stream, &rope_done))
        return 0;
    if (rope_done || n_tok == 0) return 1;
    // the path taken has no RoPE epilogue: the RoPE pass on q (and k)
    return aero_hip_qk_norm_rope(y[0], nullptr, n_rows[0] / head_dim, n_rope > 1 ? y[1] : nullptr,
                                 nullptr, n_rope > 1 ? n_rows[1] / head_dim : 0, nullptr,
                                 nullptr, 0.f, 0, n_tok, head_dim, head_dim, rope_mode, pos,
                                 inv_freq, nullptr, nullptr, 0, stream);
}

int aero_hip_attn_input(const aero_attn_input_t* a, void* ws, int64_t ws_bytes, void* stream) {
    if (a == nullptr || a->w == nullptr || a->w_bytes == nullptr || a->n_rows == nullptr ||
        a->y == nullptr) {
        aero::set_error("attn_input: null arguments or matrix arrays");
        return 0;
    }
    const bool rope = a->n_rope > 0;
    if (a->n_rope < 0 || a->n_rope > 2 || a->n_rope > a->n_mat ||
        (rope && (a->head_dim < 2 || a->head_dim % 2 || a->head_dim > 512 || a->n_rot < 0 ||
                  a->n_rot > a->head_dim || a->n_rot % 2 || a->pos == nullptr ||
                  (a->n_rot > 0 && a->inv_freq == nullptr) ||
                  (a->rope_mode != AERO_ROPE_NEOX && a->rope_mode != AERO_ROPE_INTERLEAVED) ||
                  (a->qk_flags & ~AERO_NORM_UNIT_OFFSET) != 0))) {
        aero::set_error("attn_input: bad RoPE arguments (n_rope=%d of %d matrices, head_dim=%lld, "
                        "n_rot=%lld, mode=%d; pos and inv_freq required)", a->n_rope, a->n_mat,
                        (long long)a->head_dim, (long long)a->n_rot, a->rope_mode);
        return 0;
    }
    for (int m = 0; m < a->n_rope; ++m) {
        if (a->n_rows[m] % a->head_dim) {
            aero::set_error("attn_input: matrix %d has %lld rows, not whole heads of %lld", m,
                            (long long)a->n_rows[m], (long long)a->head_dim);
            return 0;
        }
    }
    aero::SplitJob j{a->dtype, a->x, a->d, a->x_out, a->norm_w, a->norm, a->eps, a->n_mat, a->w,
                     nullptr, 0, a->n_rows, a->y, a->n_cols, 0, a->n_tok, ws, {}};
    if (rope && a->n_rot > 0) {
        j.rope = aero::RopeFold{a->n_rope, (int)a->head_dim, a->rope_mode, a->pos, a->inv_freq};
        j.rope.n_rot = (int)a->n_rot;
        j.rope.qk_w[0] = a->q_norm_w;
        j.rope.qk_w[1] = a->n_rope > 1 ? a->k_norm_w : nullptr;
        j.rope.qk_eps = a->qk_eps;
        j.rope.qk_flags = a->qk_flags;
    }
    j.emb = a->emb;
    j.emb_type = a->emb_type;
    j.emb_bytes = a->emb_bytes;
    j.vocab = a->vocab;
    j.ids = a->ids;
    j.emb_scale = a->emb_scale;
    bool rope_done = false;
    if (!aero::norm_matmul_run(j, a->w_bytes, 0, ws_bytes, (hipStream_t)stream, &rope_done))
        return 0;
    const bool norms = a->q_norm_w != nullptr || (a->n_rope > 1 && a->k_norm_w != nullptr);
    if (rope_done || a->n_tok == 0 || !rope || (a->n_rot == 0 && !norms)) return 1;
    // the path taken has no such epilogue: the per-head norm + RoPE pass
    return aero_hip_qk_norm_rope(
        a->y[0], nullptr, a->n_rows[0] / a->head_dim, a->n_rope > 1 ? a->y[1] : nullptr, nullptr,
        a->n_rope > 1 ? a->n_rows[1] / a->head_dim : 0, a->q_norm_w,
        a->n_rope > 1 ? a->k_norm_w : nullptr, a->qk_eps, a->qk_flags, a->n_tok, a->head_dim,
        a->n_rot, a->rope_mode, a->pos, a->n_rot > 0 ? a->inv_freq : nullptr, nullptr, nullptr,
        0, stream);
}

int aero_hip_norm_matmul_gate_up(int dtype, const uint8_t* w_gate, const uint8_t* w_up,
                                 int64_t w_bytes, const float* x, const float* d, float* x_out,
                                 const float* norm_w, float eps, int norm, int act, float* out,
                                 int64_t n_ff, int64_t n_cols, int64_t n_tok, void* ws,
                                 int64_t ws_bytes, void* stream) {
    if (w_up == nullptr || act < AERO_ACT_SILU || act > AERO_ACT_IDENTITY) {
        aero::set_error("norm_matmul_gate_up: null up matrix or unknown activation %d", act);
        return 0;
    }
    const uint8_t* const ws_g[1] = {w_gate};
    const int64_t wb[1] = {w_bytes};
    const int64_t nr[1] = {n_ff};
    float* const ys[1] = {out};
    aero::SplitJob j{dtype, x, d, x_out, norm_w, norm, eps, 1, ws_g, w_up, act, nr, ys,
                     n_cols, 0, n_tok, ws, {}};
    bool rope_done;
    return aero::norm_matmul_run(j, wb, n_ff, ws_bytes, (hipStream_t)stream, &rope_done) ? 1
                                                                                         : 0;
}

int aero_hip_matmul_noalloc(int dtype, const uint8_t* w, int64_t w_bytes, const float* x,
                            float* y, int64_t n_rows, int64_t n_cols, int64_t n_tok,
                            void* stream) {
    return aero::matmul_noalloc(dtype, w, w_bytes, x, y, n_rows, n_cols, n_tok,
                                (hipStream_t)stream) ? 1 : 0;
}

int64_t aero_hip_matmul_noalloc_max_bytes(void) { return aero::matmul_scratch_bytes(); }

}  // extern "C"
