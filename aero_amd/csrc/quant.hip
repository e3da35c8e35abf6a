// GGUF token-embedding row gather with Q8_0 / Q4_K / Q6_K dequant on gfx950,
// and the same kernels as a whole-buffer dequant.
//
// Work is split by quant block: a Q4_K or Q6_K block (256 values) is one
// wave, each lane producing one float4 of consecutive outputs; a Q8_0 block
// (32 values) is eight lanes. A lane reads only the bytes its four values
// need (a 32-bit word of quants plus the block header, which every lane of
// the block shares through L1), unpacks the 6-bit / 4-bit scales in
// registers and writes one 128-bit store, so a wave writes 1 KiB of
// contiguous output. HBM bytes per gathered row: (n_embd/bv)*bb read +
// 4*n_embd written.
//
// Arithmetic is the reference's, operation by operation with contraction
// off, so results are bit-identical: Q8_0 d*q (src/kernels.cpp:364-373);
// Q4_K (d*sc)*q - (dmin*m) with the 6-bit unpacking of src/kernels.cpp:65-73,
// 337-363; Q6_K (d*sc)*(q-32) (src/kernels.cpp:427-458). fp16 scales are
// decoded exactly (subnormals included). The optional embedding scale is a
// separate multiply, as the reference's second pass (src/model.cpp:315-316).
#include "common.hpp"
#include "aero_hip.h"

#pragma clang fp contract(off)

namespace aero {
namespace {

struct GatherParams {
    const uint8_t* table;
    const int32_t* ids;  // null: output row r reads table row r
    int64_t vocab;
    int64_t n_rows;
    int64_t nbr;         // quant blocks per row
    int64_t rb;          // bytes per table row
    float* out;
    float scale;         // applied when > 0
    uint32_t* bad;       // optional count of out-of-range ids
};

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

template <int TYPE> struct QType;
template <> struct QType<AERO_DTYPE_Q8_0> { static constexpr int BV = 32, BB = 34, LPB = 8; };
template <> struct QType<AERO_DTYPE_Q4_K> { static constexpr int BV = 256, BB = 144, LPB = 64; };
template <> struct QType<AERO_DTYPE_Q6_K> { static constexpr int BV = 256, BB = 210, LPB = 64; };

// Values 4l..4l+3 of one Q8_0 block.
__device__ __forceinline__ float4 dec_q8_0(const uint8_t* blk, int l) {
    const float d = half_bits_to_float(ld_u16(blk));
    const uint32_t q = ld_u32_a2(blk + 2 + 4 * l);
    float4 v;
    v.x = d * (float)(int8_t)byte_of(q, 0);
    v.y = d * (float)(int8_t)byte_of(q, 1);
    v.z = d * (float)(int8_t)byte_of(q, 2);
    v.w = d * (float)(int8_t)byte_of(q, 3);
    return v;
}

// Values 4l..4l+3 of one Q4_K block: group j = l/16 covers values 64j..64j+63,
// low nibbles first (sub-block 2j) then high nibbles (sub-block 2j+1).
__device__ __forceinline__ float4 dec_q4_k(const uint8_t* blk, int l) {
    const uint32_t dd = ld_u32(blk);
    const float d = half_bits_to_float(dd & 0xFFFFu);
    const float dmin = half_bits_to_float(dd >> 16);
    const uint32_t s0 = ld_u32(blk + 4), s1 = ld_u32(blk + 8), s2 = ld_u32(blk + 12);
    const int j = l >> 4;
    const int hi = (l >> 3) & 1;
    const int i0 = (l & 7) * 4;
    const int k = 2 * j + hi;
    // byte idx of the 12-byte scale field, selected without a private array
    auto sb = [&](int idx) {
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
    const uint32_t q = ld_u32(blk + 16 + 32 * j + i0);
    const int sh = hi ? 4 : 0;
    float4 v;
    v.x = f * (float)((byte_of(q, 0) >> sh) & 15u) - g;
    v.y = f * (float)((byte_of(q, 1) >> sh) & 15u) - g;
    v.z = f * (float)((byte_of(q, 2) >> sh) & 15u) - g;
    v.w = f * (float)((byte_of(q, 3) >> sh) & 15u) - g;
    return v;
}

// Values 4l..4l+3 of one Q6_K block: half h = l/32, quarter k = (l/8)%4
// (values 128h + 32k + lq .. +3, lq = 4*(l%8)).
__device__ __forceinline__ float4 dec_q6_k(const uint8_t* blk, int l) {
    const int h = l >> 5;
    const int k = (l >> 3) & 3;
    const int lq = (l & 7) * 4;
    const uint32_t ql = ld_u32_a2(blk + 64 * h + lq + 32 * (k & 1));
    const uint32_t qh = ld_u32_a2(blk + 128 + 32 * h + lq);
    const int sc = (int8_t)blk[192 + 8 * h + (lq >> 4) + 2 * k];
    const float d = half_bits_to_float(ld_u16(blk + 208));
    const float f = d * (float)sc;
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

template <int TYPE>
__global__ __launch_bounds__(256) void gather_kernel(GatherParams p) {
    using Q = QType<TYPE>;
    const int64_t g = (int64_t)blockIdx.x * 256 + threadIdx.x;
    const int64_t gb = g / Q::LPB;
    const int l = (int)(g % Q::LPB);
    if (gb >= p.n_rows * p.nbr) return;
    const int64_t row = gb / p.nbr;
    const int64_t b = gb % p.nbr;
    const int64_t tok = p.ids ? (int64_t)p.ids[row] : row;
    float* o = p.out + gb * Q::BV + 4 * l;
    if (tok < 0 || tok >= p.vocab) {
        st_stream(o, make_float4(0.f, 0.f, 0.f, 0.f));
        if (p.bad != nullptr && b == 0 && l == 0) atomicAdd(p.bad, 1u);
        return;
    }
    const uint8_t* blk = p.table + tok * p.rb + b * Q::BB;
    float4 v;
    if constexpr (TYPE == AERO_DTYPE_Q8_0) v = dec_q8_0(blk, l);
    else if constexpr (TYPE == AERO_DTYPE_Q4_K) v = dec_q4_k(blk, l);
    else v = dec_q6_k(blk, l);
    if (p.scale > 0.0f) {
        v.x = v.x * p.scale; v.y = v.y * p.scale; v.z = v.z * p.scale; v.w = v.w * p.scale;
    }
    st_stream(o, v);
}

// F16 / BF16 element-wise decode for whole-buffer dequant.
template <bool BF>
__global__ __launch_bounds__(256)
void dequant_half_kernel(const uint16_t* raw, float* out, int64_t n) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= n) return;
    const uint32_t h = raw[i];
    out[i] = BF ? __builtin_bit_cast(float, h << 16) : half_bits_to_float(h);
}

int block_values(int t) {
    switch (t) {
    case AERO_DTYPE_F32: case AERO_DTYPE_F16: case AERO_DTYPE_BF16: return 1;
    case AERO_DTYPE_Q8_0: return 32;
    case AERO_DTYPE_Q4_K: case 13: case AERO_DTYPE_Q6_K: case 23: return 256;
    default: return 0;
    }
}

int block_bytes(int t) {
    switch (t) {
    case AERO_DTYPE_F32: return 4;
    case AERO_DTYPE_F16: case AERO_DTYPE_BF16: return 2;
    case AERO_DTYPE_Q8_0: return 34;
    case AERO_DTYPE_Q4_K: return 144;
    case 13: return 176;
    case AERO_DTYPE_Q6_K: return 210;
    case 23: return 136;
    default: return 0;
    }
}

bool is_block_quant(int t) {
    return t == AERO_DTYPE_Q8_0 || t == AERO_DTYPE_Q4_K || t == AERO_DTYPE_Q6_K;
}

bool run_gather(int dtype, GatherParams p, hipStream_t s) {
    const int64_t nb = p.n_rows * p.nbr;
    if (nb == 0) return true;
    const int lpb = dtype == AERO_DTYPE_Q8_0 ? 8 : 64;
    const int64_t blocks = (nb * lpb + 255) / 256;
    if (blocks > 0x7fffffff) {
        set_error("gather: grid too large");
        return false;
    }
    switch (dtype) {
    case AERO_DTYPE_Q8_0:
        return launch("gather_kernel<Q8_0>", gather_kernel<AERO_DTYPE_Q8_0>,
                      dim3((unsigned)blocks), dim3(256), 0, s, p);
    case AERO_DTYPE_Q4_K:
        return launch("gather_kernel<Q4_K>", gather_kernel<AERO_DTYPE_Q4_K>,
                      dim3((unsigned)blocks), dim3(256), 0, s, p);
    case AERO_DTYPE_Q6_K:
        return launch("gather_kernel<Q6_K>", gather_kernel<AERO_DTYPE_Q6_K>,
                      dim3((unsigned)blocks), dim3(256), 0, s, p);
    default:
        set_error("gather: unsupported dtype %d", dtype);
        return false;
    }
}

}  // namespace

int64_t dtype_block_bytes(int t) { return block_bytes(t); }
int64_t dtype_block_values(int t) { return block_values(t); }

bool dequant_dev(int dtype, const uint8_t* raw, int64_t raw_len, float* out,
                 int64_t n_values, hipStream_t s) {
    const bool known = dtype == AERO_DTYPE_F32 || dtype == AERO_DTYPE_F16 ||
                       dtype == AERO_DTYPE_BF16 || is_block_quant(dtype);
    if (!known) {
        set_error("dequant: dtype %d has no GPU dequantiser", dtype);
        return false;
    }
    if (raw == nullptr || out == nullptr || n_values < 0) {
        set_error("dequant: bad arguments");
        return false;
    }
    const int64_t bv = block_values(dtype), bb = block_bytes(dtype);
    const int64_t nblocks = n_values / bv;
    if (raw_len < nblocks * bb) {
        set_error("dequant: raw_len %lld < %lld bytes needed", (long long)raw_len,
                  (long long)(nblocks * bb));
        return false;
    }
    if (nblocks == 0) return true;
    if (dtype == AERO_DTYPE_F32) return async_copy(out, raw, (size_t)(nblocks * 4), s);
    if (dtype == AERO_DTYPE_F16 || dtype == AERO_DTYPE_BF16) {
        if (reinterpret_cast<uintptr_t>(raw) & 1u) {
            set_error("dequant: fp16 input must be 2-byte aligned");
            return false;
        }
        const int64_t blocks = (nblocks + 255) / 256;
        if (blocks > 0x7fffffff) {
            set_error("dequant: too large");
            return false;
        }
        if (dtype == AERO_DTYPE_F16)
            return launch("dequant_half_kernel", dequant_half_kernel<false>,
                          dim3((unsigned)blocks), dim3(256), 0, s,
                          reinterpret_cast<const uint16_t*>(raw), out, nblocks);
        return launch("dequant_half_kernel", dequant_half_kernel<true>,
                      dim3((unsigned)blocks), dim3(256), 0, s,
                      reinterpret_cast<const uint16_t*>(raw), out, nblocks);
    }
    if ((reinterpret_cast<uintptr_t>(raw) & 3u) || !aligned16(out)) {
        set_error("dequant: raw must be 4-byte and out 16-byte aligned");
        return false;
    }
    GatherParams p{raw, nullptr, 1, 1, nblocks, nblocks * bb, out, 0.0f, nullptr};
    return run_gather(dtype, p, s);
}

bool embed_gather(int dtype, const uint8_t* table, int64_t table_bytes, int64_t vocab,
                  int64_t n_embd, const int32_t* ids, int64_t n_ids, float scale,
                  float* out, uint32_t* bad, hipStream_t s) {
    if (!is_block_quant(dtype)) {
        set_error("embed_gather: dtype %d not supported (Q8_0, Q4_K, Q6_K)", dtype);
        return false;
    }
    const int64_t bv = block_values(dtype), bb = block_bytes(dtype);
    if (table == nullptr || out == nullptr || (n_ids > 0 && ids == nullptr) ||
        vocab <= 0 || n_embd <= 0 || n_ids < 0 || n_embd % bv != 0) {
        set_error("embed_gather: bad arguments (vocab=%lld n_embd=%lld n_ids=%lld)",
                  (long long)vocab, (long long)n_embd, (long long)n_ids);
        return false;
    }
    const int64_t rb = (n_embd / bv) * bb;
    if (table_bytes < vocab * rb) {
        set_error("embed_gather: table_bytes %lld < vocab*row_bytes %lld",
                  (long long)table_bytes, (long long)(vocab * rb));
        return false;
    }
    if ((reinterpret_cast<uintptr_t>(table) & 3u) || !aligned16(out)) {
        set_error("embed_gather: table must be 4-byte and out 16-byte aligned");
        return false;
    }
    GatherParams p{table, ids, vocab, n_ids, n_embd / bv, rb, out, scale, bad};
    return run_gather(dtype, p, s);
}

}  // namespace aero

extern "C" {

int aero_hip_embed_gather(int dtype, const uint8_t* table, int64_t table_bytes,
                          int64_t vocab, int64_t n_embd, const int32_t* ids,
                          int64_t n_ids, float scale, float* out, uint32_t* bad_count,
                          void* stream) {
    return aero::embed_gather(dtype, table, table_bytes, vocab, n_embd, ids, n_ids,
                              scale, out, bad_count, (hipStream_t)stream) ? 1 : 0;
}

int aero_hip_dequant(int dtype, const uint8_t* raw, int64_t raw_len, float* out,
                     int64_t n_values, void* stream) {
    return aero::dequant_dev(dtype, raw, raw_len, out, n_values, (hipStream_t)stream)
               ? 1 : 0;
}

int64_t aero_dtype_block_bytes(int t) { return aero::dtype_block_bytes(t); }
int64_t aero_dtype_block_values(int t) { return aero::dtype_block_values(t); }

}  // extern "C"
