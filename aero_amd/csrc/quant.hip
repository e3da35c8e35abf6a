// GGUF token-embedding row gather with Q8_0 / Q4_K / Q5_K / Q6_K / IQ4_XS
// dequant on gfx950, and the same kernel as a whole-buffer dequant.
//
// One wave (a 64-thread workgroup) takes a run of U*256 consecutive values of
// one output row. It reads the row's token id once, loads the run's quant
// blocks (contiguous in the table) with coalesced 32-bit loads, one per lane
// per 256 bytes, stages them in LDS, and then each lane decodes four values
// per 256-value step from LDS (block header plus the quant bytes of its four
// values, unpacking 6-bit / 4-bit scales in registers) and writes one
// 128-bit store, so each step of a wave writes 1 KiB of contiguous output.
// HBM bytes per gathered row: (n_embd/bv)*bb read + 4*n_embd written.
//
// Values are the reference's dequant bit for bit (quant_blocks.hpp). The
// optional embedding scale is a separate multiply, as the reference's second
// pass (src/model.cpp:315-316).
#include <algorithm>

#include "quant_blocks.hpp"

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
    case AERO_DTYPE_Q4_K: case AERO_DTYPE_Q5_K: case AERO_DTYPE_Q6_K:
    case AERO_DTYPE_IQ4_XS: return 256;
    default: return 0;
    }
}

int block_bytes(int t) {
    switch (t) {
    case AERO_DTYPE_F32: return 4;
    case AERO_DTYPE_F16: case AERO_DTYPE_BF16: return 2;
    case AERO_DTYPE_Q8_0: return 34;
    case AERO_DTYPE_Q4_K: return 144;
    case AERO_DTYPE_Q5_K: return 176;
    case AERO_DTYPE_Q6_K: return 210;
    case AERO_DTYPE_IQ4_XS: return 136;
    default: return 0;
    }
}

bool is_block_quant(int t) {
    return t == AERO_DTYPE_Q8_0 || t == AERO_DTYPE_Q4_K || t == AERO_DTYPE_Q5_K ||
           t == AERO_DTYPE_Q6_K || t == AERO_DTYPE_IQ4_XS;
}


// Wave w covers values [c*U*256, min((c+1)*U*256, n_embd)) of output row
// r = w / cpr (c = w % cpr). Every branch on r, the token or the run length
// is uniform across the wave.
template <int TYPE, int U>
__global__ __launch_bounds__(64) void gather_rows_kernel(GatherParams p, int cpr) {
    using Q = QT<TYPE>;
    constexpr int BPS = 256 / Q::BV;                   // blocks per 256-value step
    constexpr int MAX_DW = (U * BPS * Q::BB + 3 + 3) / 4;  // + up to 3 bytes of misalignment
    constexpr int PER = (MAX_DW + 63) / 64;
    __shared__ __align__(16) uint32_t stage[PER * 64];

    const int l = threadIdx.x;
    const int row = (int)blockIdx.x / cpr;
    const int c = (int)blockIdx.x - row * cpr;
    const int64_t n_embd = p.nbr * Q::BV;
    const int64_t v_begin = (int64_t)c * (U * 256);
    const int nv = (int)min((int64_t)(U * 256), n_embd - v_begin);  // values in this run
    const StreamOut o(p.out + (int64_t)row * n_embd + v_begin, (int64_t)nv * 4);

    const int64_t tok = p.ids ? (int64_t)p.ids[row] : (int64_t)row;
    if (tok < 0 || tok >= p.vocab) {
        if (p.bad != nullptr && c == 0 && l == 0) atomicAdd(p.bad, 1u);
#pragma unroll
        for (int st = 0; st < U; ++st)
            if (st * 256 + 4 * l < nv)
                o.store((uint32_t)(st * 256 + 4 * l) * 4u, make_float4(0.f, 0.f, 0.f, 0.f));
        return;
    }

    // The run's blocks are contiguous: load the 4-byte words that cover them.
    // The first word is aligned down, so the loads stay inside the words that
    // hold the run's bytes (no access beyond the table's last word).
    const uint8_t* g = p.table + tok * p.rb + (v_begin / Q::BV) * Q::BB;
    const int off = (int)(reinterpret_cast<uintptr_t>(g) & 3u);
    const uint32_t* g4 = reinterpret_cast<const uint32_t*>(g - off);
    const int n_dw = (off + (nv / Q::BV) * Q::BB + 3) >> 2;
    // Indices past the run re-read its last word, so every load is issued
    // unconditionally and all of them are in flight together.
    uint32_t w[PER];
#pragma unroll
    for (int i = 0; i < PER; ++i) w[i] = g4[min(l + 64 * i, n_dw - 1)];
#pragma unroll
    for (int i = 0; i < PER; ++i) stage[l + 64 * i] = w[i];
    __syncthreads();

    const uint8_t* run = reinterpret_cast<const uint8_t*>(stage) + off;
#pragma unroll
    for (int st = 0; st < U; ++st) {
        const int v0 = st * 256 + 4 * l;
        if (v0 >= nv) break;
        typename Q::Raw raw;
        load_raw(run + (v0 / Q::BV) * Q::BB, l, raw);
        float4 v = decode(raw, l);
        if (p.scale > 0.0f) {
            v.x = v.x * p.scale; v.y = v.y * p.scale;
            v.z = v.z * p.scale; v.w = v.w * p.scale;
        }
        o.store((uint32_t)v0 * 4u, v);
    }
}

template <int TYPE>
bool launch_rows(const char* name, GatherParams p, hipStream_t s) {
    const int64_t n_embd = p.nbr * QT<TYPE>::BV;
    const int64_t steps_per_row = (n_embd + 255) / 256;
    // Run length, from a sweep of 1..16 on MI355X over the layer shapes:
    // up to 64K steps, the shortest run that brings the grid down to 4096
    // waves, widened to a whole row when it would leave a short last run in
    // each row; beyond that, runs of 4 steps (16K x 8192 Q4_K: 98 us at 4,
    // 110 us at 16, 135 us at 2).
    const int64_t total = p.n_rows * steps_per_row;
    int u = 4;
    if (total <= 65536) {
        u = 1;
        while (u < 16 && p.n_rows * ((steps_per_row + u - 1) / u) > 4096) u *= 2;
        if (steps_per_row % u != 0 && u < steps_per_row) {
            int whole = 1;
            while (whole < steps_per_row) whole *= 2;
            if (whole <= 16) u = whole;
        }
    }
    u = tune("gather_u", u);
    const int64_t cpr = (steps_per_row + u - 1) / u;
    const int64_t waves = p.n_rows * cpr;
    if (waves > 0x7fffffff || cpr > 0x7fffffff) {
        set_error("gather: grid too large (%lld waves)", (long long)waves);
        return false;
    }
    const dim3 grid((unsigned)waves), block(64);
    switch (u) {
    case 16: return launch(name, gather_rows_kernel<TYPE, 16>, grid, block, 0, s, p, (int)cpr);
    case 8: return launch(name, gather_rows_kernel<TYPE, 8>, grid, block, 0, s, p, (int)cpr);
    case 4: return launch(name, gather_rows_kernel<TYPE, 4>, grid, block, 0, s, p, (int)cpr);
    case 2: return launch(name, gather_rows_kernel<TYPE, 2>, grid, block, 0, s, p, (int)cpr);
    case 1: return launch(name, gather_rows_kernel<TYPE, 1>, grid, block, 0, s, p, (int)cpr);
    default:
        set_error("gather: run length %d not in {1,2,4,8,16}", u);
        return false;
    }
}

bool run_gather(int dtype, GatherParams p, hipStream_t s) {
    if (p.n_rows * p.nbr == 0) return true;
    switch (dtype) {
    case AERO_DTYPE_Q8_0: return launch_rows<AERO_DTYPE_Q8_0>("gather_rows_kernel<Q8_0>", p, s);
    case AERO_DTYPE_Q4_K: return launch_rows<AERO_DTYPE_Q4_K>("gather_rows_kernel<Q4_K>", p, s);
    case AERO_DTYPE_Q6_K: return launch_rows<AERO_DTYPE_Q6_K>("gather_rows_kernel<Q6_K>", p, s);
    case AERO_DTYPE_Q5_K: return launch_rows<AERO_DTYPE_Q5_K>("gather_rows_kernel<Q5_K>", p, s);
    case AERO_DTYPE_IQ4_XS:
        return launch_rows<AERO_DTYPE_IQ4_XS>("gather_rows_kernel<IQ4_XS>", p, s);
    default:
        set_error("gather: unsupported dtype %d", dtype);
        return false;
    }
}

// ------------------------------------------------ gather + first RMSNorm
// The model loop's first two steps in one pass (src/model.cpp:297-316, then
// norm_row of the first block, :244-245): x = dequant(table row ids[r])
// (* scale), h = (x * 1/sqrtf(mean(x^2)+eps)) * w. A workgroup of W waves
// owns one row; wave wv decodes the U consecutive 256-value steps starting
// at step wv*U (staged through its own LDS slice as in gather_rows_kernel),
// keeps them in VGPRs, stores x at once, and after one cross-wave sum of
// squares stores h, so the row is read from the table once and x is never
// read back. HBM bytes per row: (n_embd/bv)*bb + 8*n_embd.
constexpr int kEmbedNormMaxWaves = 8;

struct EmbedNormParams {
    GatherParams g;      // g.out is x
    const float* w;      // norm weight, null = ones
    float* h;
    float eps;
    int flags;           // AERO_NORM_UNIT_OFFSET
};

template <int TYPE, int U>
__global__ __launch_bounds__(64 * kEmbedNormMaxWaves)
void embed_norm_kernel(EmbedNormParams p) {
    using Q = QT<TYPE>;
    constexpr int BPS = 256 / Q::BV;
    constexpr int MAX_DW = (U * BPS * Q::BB + 3 + 3) / 4;
    constexpr int PER = (MAX_DW + 63) / 64;
    __shared__ __align__(16) uint32_t stage[kEmbedNormMaxWaves][PER * 64];
    __shared__ float part[kEmbedNormMaxWaves];

    const int l = threadIdx.x & 63;
    const int wv = threadIdx.x >> 6;
    const int nw = blockDim.x >> 6;
    const int64_t row = blockIdx.x;
    const int64_t n_embd = p.g.nbr * Q::BV;
    const int64_t v_begin = (int64_t)wv * (U * 256);
    // values this wave owns (<= 0: a wave past the row's end, which only
    // joins the barriers)
    const int nv = (int)max(min((int64_t)(U * 256), n_embd - v_begin), (int64_t)0);
    const int64_t tok = p.g.ids ? (int64_t)p.g.ids[row] : row;
    const bool good = tok >= 0 && tok < p.g.vocab;
    if (!good && p.g.bad != nullptr && threadIdx.x == 0) atomicAdd(p.g.bad, 1u);

    const int off = good ? (int)(reinterpret_cast<uintptr_t>(
                               p.g.table + tok * p.g.rb + (v_begin / Q::BV) * Q::BB) & 3u)
                         : 0;
    if (good && nv > 0) {
        const uint8_t* g = p.g.table + tok * p.g.rb + (v_begin / Q::BV) * Q::BB;
        const uint32_t* g4 = reinterpret_cast<const uint32_t*>(g - off);
        const int n_dw = (off + (nv / Q::BV) * Q::BB + 3) >> 2;
        uint32_t wd[PER];
#pragma unroll
        for (int i = 0; i < PER; ++i) wd[i] = g4[min(l + 64 * i, n_dw - 1)];
#pragma unroll
        for (int i = 0; i < PER; ++i) stage[wv][l + 64 * i] = wd[i];
    }
    __syncthreads();

    const int64_t rowoff = row * n_embd + v_begin;
    const int64_t left = (int64_t)max(nv, 0) * 4;
    const StreamOut ox(p.g.out + rowoff, left);
    const StreamOut oh(p.h + rowoff, left);
    const uint8_t* run = reinterpret_cast<const uint8_t*>(stage[wv]) + off;
    float4 xv[U];
    float ss = 0.0f;
#pragma unroll
    for (int st = 0; st < U; ++st) {
        const int v0 = st * 256 + 4 * l;
        float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
        if (v0 < nv) {
            if (good) {
                typename Q::Raw raw;
                load_raw(run + (v0 / Q::BV) * Q::BB, l, raw);
                v = decode(raw, l);
                if (p.g.scale > 0.0f) {
                    v.x = v.x * p.g.scale; v.y = v.y * p.g.scale;
                    v.z = v.z * p.g.scale; v.w = v.w * p.g.scale;
                }
            }
            ox.store((uint32_t)v0 * 4u, v);
        }
        xv[st] = v;
        ss += v.x * v.x;
        ss += v.y * v.y;
        ss += v.z * v.z;
        ss += v.w * v.w;
    }
    ss = group_sum<64>(ss);
    if (l == 0) part[wv] = ss;
    __syncthreads();
    ss = part[0];
    for (int k = 1; k < nw; ++k) ss += part[k];
    const float inv = 1.0f / sqrtf(ss / (float)n_embd + p.eps);
#pragma unroll
    for (int st = 0; st < U; ++st) {
        const int v0 = st * 256 + 4 * l;
        if (v0 >= nv) break;
        float4 o = make_float4(xv[st].x * inv, xv[st].y * inv, xv[st].z * inv,
                               xv[st].w * inv);
        if (p.w != nullptr) {
            float4 w4 = *reinterpret_cast<const float4*>(p.w + v_begin + v0);
            if (p.flags & AERO_NORM_UNIT_OFFSET) {
                w4.x = 1.0f + w4.x; w4.y = 1.0f + w4.y;
                w4.z = 1.0f + w4.z; w4.w = 1.0f + w4.w;
            }
            o.x = o.x * w4.x; o.y = o.y * w4.y; o.z = o.z * w4.z; o.w = o.w * w4.w;
        }
        oh.store((uint32_t)v0 * 4u, o);
    }
}

// Steps a wave and waves a row: the fewest steps a wave (1, 2, 4, 8) that
// keep the row within `maxw` waves, so short rows still spread over several
// waves and long rows keep <= 8 float4 a lane. maxw is 8 up to 1024 rows
// and 4 beyond (sweep on MI355X: 512 x 4096 Q4_K 5.1 us at 8, 5.7 at 4;
// 2048 x 2560 Q6_K 8.8 us at 4, 10.3 at 8; 4096 x 2048 Q8_0 13.2 at 4, 17.2
// at 8; 16384 x 8192 Q4_K within 3% either way).
template <int TYPE>
bool launch_embed_norm(EmbedNormParams p, hipStream_t s) {
    const int64_t n_embd = p.g.nbr * QT<TYPE>::BV;
    const int64_t steps = (n_embd + 255) / 256;
    const int maxw = std::min(std::max(tune("embed_norm_waves", p.g.n_rows <= 1024 ? 8 : 4), 1),
                              kEmbedNormMaxWaves);
    int u = 1;
    while (u < 8 && (steps + u - 1) / u > maxw) u *= 2;
    u = tune("embed_norm_u", u);
    const int64_t waves = (steps + u - 1) / u;
    if (waves > kEmbedNormMaxWaves) {
        set_error("embed_rmsnorm: row of %lld values needs %lld waves (max %d)",
                  (long long)n_embd, (long long)waves, kEmbedNormMaxWaves);
        return false;
    }
    if (p.g.n_rows > 0x7fffffff) {
        set_error("embed_rmsnorm: too many rows (%lld)", (long long)p.g.n_rows);
        return false;
    }
    const dim3 grid((unsigned)p.g.n_rows), block((unsigned)(64 * waves));
    const char* name = "embed_norm_kernel";
    switch (u) {
    case 1: return launch(name, embed_norm_kernel<TYPE, 1>, grid, block, 0, s, p);
    case 2: return launch(name, embed_norm_kernel<TYPE, 2>, grid, block, 0, s, p);
    case 4: return launch(name, embed_norm_kernel<TYPE, 4>, grid, block, 0, s, p);
    case 8: return launch(name, embed_norm_kernel<TYPE, 8>, grid, block, 0, s, p);
    default:
        set_error("embed_rmsnorm: steps per wave %d not in {1,2,4,8}", u);
        return false;
    }
}

}  // namespace

bool embed_rmsnorm(int dtype, const uint8_t* table, int64_t table_bytes, int64_t vocab,
                   int64_t n_embd, const int32_t* ids, int64_t n_ids, float scale,
                   float* x_out, const float* norm_w, float eps, int norm_flags,
                   float* h_out, uint32_t* bad, hipStream_t s) {
    if (!is_block_quant(dtype)) {
        set_error("embed_rmsnorm: dtype %d not supported (Q8_0, Q4_K, Q5_K, Q6_K, IQ4_XS)",
                  dtype);
        return false;
    }
    const int64_t bv = block_values(dtype), bb = block_bytes(dtype);
    if (table == nullptr || x_out == nullptr || h_out == nullptr ||
        (n_ids > 0 && ids == nullptr) || vocab <= 0 || n_embd <= 0 || n_ids < 0 ||
        n_embd % bv != 0 || (norm_flags & ~AERO_NORM_UNIT_OFFSET) != 0) {
        set_error("embed_rmsnorm: bad arguments (vocab=%lld n_embd=%lld n_ids=%lld "
                  "flags=%d)", (long long)vocab, (long long)n_embd, (long long)n_ids,
                  norm_flags);
        return false;
    }
    if (x_out == h_out) {
        set_error("embed_rmsnorm: x_out and h_out must be different buffers");
        return false;
    }
    const int64_t rb = (n_embd / bv) * bb;
    if (table_bytes < vocab * rb) {
        set_error("embed_rmsnorm: table_bytes %lld < vocab*row_bytes %lld",
                  (long long)table_bytes, (long long)(vocab * rb));
        return false;
    }
    if ((reinterpret_cast<uintptr_t>(table) & 3u) || !aligned16(x_out) || !aligned16(h_out) ||
        (norm_w != nullptr && !aligned16(norm_w))) {
        set_error("embed_rmsnorm: table must be 4-byte and x_out, h_out, norm_w 16-byte "
                  "aligned");
        return false;
    }
    if (n_ids == 0) return true;
    EmbedNormParams p{{table, ids, vocab, n_ids, n_embd / bv, rb, x_out, scale, bad},
                      norm_w, h_out, eps, norm_flags};
    switch (dtype) {
    case AERO_DTYPE_Q8_0: return launch_embed_norm<AERO_DTYPE_Q8_0>(p, s);
    case AERO_DTYPE_Q4_K: return launch_embed_norm<AERO_DTYPE_Q4_K>(p, s);
    case AERO_DTYPE_Q5_K: return launch_embed_norm<AERO_DTYPE_Q5_K>(p, s);
    case AERO_DTYPE_Q6_K: return launch_embed_norm<AERO_DTYPE_Q6_K>(p, s);
    default: return launch_embed_norm<AERO_DTYPE_IQ4_XS>(p, s);
    }
}

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
        set_error("embed_gather: dtype %d not supported (Q8_0, Q4_K, Q5_K, Q6_K, IQ4_XS)",
                  dtype);
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

// Rows [r0, r1) of a resident tensor of n_rows rows of n_per_row values
// (whole blocks a row), dequantised to out [(r1 - r0) x n_per_row]: the row
// addressing of engine/gguf.py:278-314 over HBM. Block types go through the
// row gather (any row alignment: it loads the aligned words around a row),
// F32 / F16 / BF16 through the element decode.
bool tensor_rows_dev(int dtype, const uint8_t* table, int64_t table_bytes, int64_t n_rows,
                     int64_t n_per_row, int64_t r0, int64_t r1, float* out, hipStream_t s) {
    const bool known = dtype == AERO_DTYPE_F32 || dtype == AERO_DTYPE_F16 ||
                       dtype == AERO_DTYPE_BF16 || is_block_quant(dtype);
    if (!known) {
        set_error("tensor_rows: dtype %d has no GPU dequantiser", dtype);
        return false;
    }
    const int64_t bv = block_values(dtype), bb = block_bytes(dtype);
    if (table == nullptr || out == nullptr || n_rows < 0 || n_per_row <= 0 ||
        n_per_row % bv != 0) {
        set_error("tensor_rows: bad arguments (n_rows=%lld n_per_row=%lld)", (long long)n_rows,
                  (long long)n_per_row);
        return false;
    }
    if (r0 < 0 || r1 < r0 || r1 > n_rows) {
        set_error("tensor_rows: row range [%lld,%lld) outside [0,%lld)", (long long)r0,
                  (long long)r1, (long long)n_rows);
        return false;
    }
    const int64_t rb = (n_per_row / bv) * bb;
    if (table_bytes < n_rows * rb) {
        set_error("tensor_rows: table_bytes %lld < n_rows*row_bytes %lld",
                  (long long)table_bytes, (long long)(n_rows * rb));
        return false;
    }
    if ((reinterpret_cast<uintptr_t>(table) & 3u) || !aligned16(out)) {
        set_error("tensor_rows: table must be 4-byte and out 16-byte aligned");
        return false;
    }
    const int64_t n = r1 - r0;
    if (n == 0) return true;
    const uint8_t* first = table + r0 * rb;
    if (!is_block_quant(dtype)) return dequant_dev(dtype, first, n * rb, out, n * n_per_row, s);
    GatherParams p{first, nullptr, n, n, n_per_row / bv, rb, out, 0.0f, nullptr};
    return run_gather(dtype, p, s);
}

}  // namespace aero

extern "C" {

int aero_hip_tensor_rows(int dtype, const uint8_t* table, int64_t table_bytes, int64_t n_rows,
                         int64_t n_per_row, int64_t r0, int64_t r1, float* out, void* stream) {
    aero::clear_error();
    return aero::tensor_rows_dev(dtype, table, table_bytes, n_rows, n_per_row, r0, r1, out,
                                 (hipStream_t)stream) ? 1 : 0;
}

int aero_hip_embed_gather(int dtype, const uint8_t* table, int64_t table_bytes,
                          int64_t vocab, int64_t n_embd, const int32_t* ids,
                          int64_t n_ids, float scale, float* out, uint32_t* bad_count,
                          void* stream) {
    return aero::embed_gather(dtype, table, table_bytes, vocab, n_embd, ids, n_ids,
                              scale, out, bad_count, (hipStream_t)stream) ? 1 : 0;
}

int aero_hip_embed_rmsnorm(int dtype, const uint8_t* table, int64_t table_bytes,
                           int64_t vocab, int64_t n_embd, const int32_t* ids, int64_t n_ids,
                           float scale, float* x_out, const float* norm_w, float eps,
                           int norm_flags, float* h_out, uint32_t* bad_count,
                           void* stream) {
    return aero::embed_rmsnorm(dtype, table, table_bytes, vocab, n_embd, ids, n_ids, scale,
                               x_out, norm_w, eps, norm_flags, h_out, bad_count,
                               (hipStream_t)stream) ? 1 : 0;
}

int aero_hip_dequant(int dtype, const uint8_t* raw, int64_t raw_len, float* out,
                     int64_t n_values, void* stream) {
    return aero::dequant_dev(dtype, raw, raw_len, out, n_values, (hipStream_t)stream)
               ? 1 : 0;
}

int64_t aero_dtype_block_bytes(int t) { return aero::dtype_block_bytes(t); }
int64_t aero_dtype_block_values(int t) { return aero::dtype_block_values(t); }

}  // extern "C"
