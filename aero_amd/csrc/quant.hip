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
template <> struct QType<AERO_DTYPE_Q4_K> { static constexpr int BV = 256, BB = 144; };
template <> struct QType<AERO_DTYPE_Q6_K> { static constexpr int BV = 256, BB = 210; };

// A "unit" is 256 consecutive output values. For Q4_K / Q6_K a unit is one
// block and lane l of a wave produces values 4l..4l+3 of it. For Q8_0 a unit
// is eight consecutive blocks of the flattened (row, block) sequence (rows of
// any block count): lane l produces values 4(l%8).. of block l/8. Each wave
// takes NB consecutive units, issues the loads of all of them first (raw
// words into registers), then decodes and stores, so a wave has NB units of
// loads in flight and writes NB KiB.

// Raw words one lane needs for its four values of one unit.
struct RawQ8 { uint32_t d, q0, q1; };        // fp16 d, quant bytes as 2 x 16 bit
struct RawQ4 { uint32_t dd, s0, s1, s2, q; }; // d|dmin, 12 scale bytes, 4 quant bytes
struct RawQ6 { uint32_t ql0, ql1, qh0, qh1, sc, d; };

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

template <int TYPE, typename RAW, int NB>
__global__ __launch_bounds__(256) void gather_kernel(GatherParams p) {
    using Q = QType<TYPE>;
    static_assert(Q::BV == 256, "one block per unit");
    const int l = threadIdx.x & 63;
    const int64_t wave = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    const int64_t upr = p.nbr;            // units per row
    const int64_t n_units = p.n_rows * upr;
    RAW raw[NB];
    bool ok[NB];
    int64_t unit[NB];
#pragma unroll
    for (int i = 0; i < NB; ++i) {
        unit[i] = wave * NB + i;
        ok[i] = false;
        if (unit[i] < n_units) {
            const int64_t row = unit[i] / upr;
            const int64_t u = unit[i] % upr;
            const int64_t tok = p.ids ? (int64_t)p.ids[row] : row;
            if (tok >= 0 && tok < p.vocab) {
                ok[i] = true;
                load_raw(p.table + tok * p.rb + u * Q::BB, l, raw[i]);
            } else if (p.bad != nullptr && u == 0 && l == 0) {
                atomicAdd(p.bad, 1u);
            }
        }
    }
    const int64_t u0 = wave * NB;  // first unit of the wave
    const StreamOut o(p.out + u0 * 256, (n_units - u0) * 1024);
#pragma unroll
    for (int i = 0; i < NB; ++i) {
        if (unit[i] >= n_units) continue;
        float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
        if (ok[i]) {
            v = decode(raw[i], l);
            if (p.scale > 0.0f) {
                v.x = v.x * p.scale; v.y = v.y * p.scale;
                v.z = v.z * p.scale; v.w = v.w * p.scale;
            }
        }
        o.store((uint32_t)(((unit[i] - u0) * 256 + 4 * l) * 4), v);
    }
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

template <int NB>
__global__ __launch_bounds__(256) void gather_q8_0_kernel(GatherParams p) {
    const int l = threadIdx.x & 63;
    const int64_t wave = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    const int64_t n_blocks = p.n_rows * p.nbr;
    RawQ8 raw[NB];
    bool ok[NB];
    int64_t gb[NB];
#pragma unroll
    for (int i = 0; i < NB; ++i) {
        gb[i] = (wave * NB + i) * 8 + (l >> 3);
        ok[i] = false;
        if (gb[i] < n_blocks) {
            const int64_t row = gb[i] / p.nbr;
            const int64_t b = gb[i] % p.nbr;
            const int64_t tok = p.ids ? (int64_t)p.ids[row] : row;
            if (tok >= 0 && tok < p.vocab) {
                ok[i] = true;
                load_raw(p.table + tok * p.rb + b * 34, l, raw[i]);
            } else if (p.bad != nullptr && b == 0 && (l & 7) == 0) {
                atomicAdd(p.bad, 1u);
            }
        }
    }
    const int64_t gb0 = wave * NB * 8;  // first block of the wave
    const StreamOut o(p.out + gb0 * 32, (n_blocks - gb0) * 128);
#pragma unroll
    for (int i = 0; i < NB; ++i) {
        if (gb[i] >= n_blocks) continue;
        float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
        if (ok[i]) {
            v = decode(raw[i], l);
            if (p.scale > 0.0f) {
                v.x = v.x * p.scale; v.y = v.y * p.scale;
                v.z = v.z * p.scale; v.w = v.w * p.scale;
            }
        }
        o.store((uint32_t)(((gb[i] - gb0) * 32 + 4 * (l & 7)) * 4), v);
    }
}

template <int TYPE, typename RAW>
bool launch_gather(const char* name, GatherParams p, int64_t n_units, hipStream_t s) {
    // Small gathers want many short waves (latency), large ones want more
    // bytes in flight per wave: measured crossover ~128K units on MI355X.
    const int nb = tune("gather_nb", n_units >= 131072 ? 2 : 1);
    const int per_wave = nb >= 4 ? 4 : (nb >= 2 ? 2 : 1);
    const int64_t waves = (n_units + per_wave - 1) / per_wave;
    const int64_t blocks = (waves + 3) / 4;
    if (blocks > 0x7fffffff) {
        set_error("gather: grid too large");
        return false;
    }
    if constexpr (TYPE == AERO_DTYPE_Q8_0) {
        switch (per_wave) {
        case 4: return launch(name, gather_q8_0_kernel<4>, dim3((unsigned)blocks), dim3(256), 0, s, p);
        case 2: return launch(name, gather_q8_0_kernel<2>, dim3((unsigned)blocks), dim3(256), 0, s, p);
        default: return launch(name, gather_q8_0_kernel<1>, dim3((unsigned)blocks), dim3(256), 0, s, p);
        }
    } else {
        switch (per_wave) {
        case 4: return launch(name, gather_kernel<TYPE, RAW, 4>, dim3((unsigned)blocks), dim3(256), 0, s, p);
        case 2: return launch(name, gather_kernel<TYPE, RAW, 2>, dim3((unsigned)blocks), dim3(256), 0, s, p);
        default: return launch(name, gather_kernel<TYPE, RAW, 1>, dim3((unsigned)blocks), dim3(256), 0, s, p);
        }
    }
}

bool run_gather(int dtype, GatherParams p, hipStream_t s) {
    const int64_t nb = p.n_rows * p.nbr;
    if (nb == 0) return true;
    switch (dtype) {
    case AERO_DTYPE_Q8_0:  // units of 8 blocks of the flattened sequence
        return launch_gather<AERO_DTYPE_Q8_0, RawQ8>("gather_q8_0_kernel", p, (nb + 7) / 8, s);
    case AERO_DTYPE_Q4_K:
        return launch_gather<AERO_DTYPE_Q4_K, RawQ4>("gather_kernel<Q4_K>", p, nb, s);
    case AERO_DTYPE_Q6_K:
        return launch_gather<AERO_DTYPE_Q6_K, RawQ6>("gather_kernel<Q6_K>", p, nb, s);
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
