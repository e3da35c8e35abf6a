// Attention core and KV cache on gfx950: the reference's grouped-query
// attention with an online softmax (src/transformer.cpp:120-214), its row
// softmax (src/tensor.cpp:167-178) and the KV cache vector quantisers
// (include/aero/kv.hpp:62-103, src/kv.cpp:13-46).
//
// attn_kernel: a workgroup (4 waves) takes one kv head, QV = 4 query vectors
// of that head's group (query vector u = token u / rep, head kh*rep + u % rep)
// and one chunk of the keys. 16 lanes own a key at a time (lane i holds
// elements E*i .. E*i+E-1 of the head dimension), so a wave walks 4 keys per
// step and each K / V element is loaded once for the 4 queries. Each lane
// group keeps an online softmax (running max m, sum l, accumulator) per
// query; the 16 groups of the workgroup are merged through LDS at the end,
// and with several key chunks (decode: one query, many keys) the chunks'
// (m, l, acc) are merged by attn_combine_kernel. K / V are read in the
// cache's format (fp32, or int8 / int4 with one fp32 scale per vector) and
// dequantised in registers exactly as the reference's read_vec.
//
// Masking as the reference: key j (position kpos[j] or j) is kept for query
// position qp when kp <= qp and, with window > 0, qp - kp < window; a query
// with no kept key gives zeros. When kpos is absent, keys past the tile's
// largest query position (or before its smallest window start) are skipped.
//
// Results differ from the reference's serial loops in summation order and in
// the exp of the GPU's math library: <= 1e-5 relative to the output's scale.
#include "common.hpp"
#include "aero_hip.h"

#include <cmath>

namespace aero {

namespace {

constexpr int kQV = 4;           // query vectors per workgroup
constexpr int kAttnWaves = 4;
constexpr int kKeysPerStep = 4 * kAttnWaves;  // 4 lane groups of 16 per wave

struct AttnParams {
    const float* q;        // [n_q, n_head, head_dim]
    const void* k;         // [n_kv, n_head_kv, head_dim] in kv_dt
    const float* k_scale;  // [n_kv, n_head_kv] (int8 / int4)
    const void* v;         // [n_kv, n_head_kv, value_dim] in kv_dt
    const float* v_scale;
    float* out;            // [n_q, n_head, value_dim]
    float* part;           // [n_chunks, n_q * n_head, value_dim + 2] (several chunks)
    const int32_t* qpos;   // [n_q] or null (= t)
    const int32_t* kpos;   // [n_kv] or null (= j)
    int64_t n_q, n_head, n_head_kv, head_dim, value_dim, n_kv;
    int rep;               // n_head / n_head_kv
    int window;
    float scale;
    int64_t chunk_len;     // keys per chunk (multiple of kKeysPerStep)
    int n_chunks;
};

// E consecutive elements [e0, e0+E) of vector `vec` of a cache side, as fp32
// (zeros past `dim`). DT 0 fp32, 1 int8, 2 int4 (low nibble first).
template <int DT, int E>
__device__ __forceinline__ void load_vec(const void* base, const float* scales, int64_t vec,
                                         int64_t dim, int e0, float (&o)[E]) {
    if constexpr (DT == 0) {
        const float* p = static_cast<const float*>(base) + vec * dim + e0;
#pragma unroll
        for (int e = 0; e < E; e += 4) {
            if (e0 + e + 4 <= dim) {
                const float4 f = *reinterpret_cast<const float4*>(p + e);
                o[e] = f.x; o[e + 1] = f.y; o[e + 2] = f.z; o[e + 3] = f.w;
            } else {
#pragma unroll
                for (int i = 0; i < 4; ++i) o[e + i] = (e0 + e + i < dim) ? p[e + i] : 0.0f;
            }
        }
    } else if constexpr (DT == 1) {
        const int8_t* p = static_cast<const int8_t*>(base) + vec * dim + e0;
        const float s = scales[vec];
#pragma unroll
        for (int e = 0; e < E; ++e) o[e] = (e0 + e < dim) ? (float)p[e] * s : 0.0f;
    } else {
        const uint8_t* p = static_cast<const uint8_t*>(base) + vec * (dim / 2) + e0 / 2;
        const float s = scales[vec];
#pragma unroll
        for (int e = 0; e < E; e += 2) {
            const uint32_t b = (e0 + e < dim) ? p[e / 2] : 0u;
            const int lo = (int)(b & 15u), hi = (int)((b >> 4) & 15u);
            o[e] = (float)(lo >= 8 ? lo - 16 : lo) * s;
            o[e + 1] = (float)(hi >= 8 ? hi - 16 : hi) * s;
        }
    }
}

__device__ __forceinline__ bool key_kept(int64_t kp, int64_t qp, int window) {
    bool keep = kp <= qp;
    if (window > 0) keep = keep && (qp - kp) < window;
    return keep;
}

// MERGE_OUT: one chunk, write out directly; else write the chunk's partials.
template <int DT, int E, bool MERGE_OUT>
__global__ __launch_bounds__(64 * kAttnWaves) void attn_kernel(AttnParams p) {
    constexpr int DVP = 16 * E;  // padded value width
    __shared__ float sm[kAttnWaves * 4][kQV];
    __shared__ float sl[kAttnWaves * 4][kQV];
    __shared__ float sacc[kAttnWaves * 4][kQV][DVP];

    const int tid = threadIdx.x;
    const int grp = tid >> 4;   // lane group (0..15) of the workgroup
    const int li = tid & 15;    // lane within the group
    const int e0 = E * li;
    const int chunk = blockIdx.x;
    const int kh = blockIdx.y;
    const int64_t n_vec = p.n_q * p.rep;  // query vectors of this kv head

    // this workgroup's query vectors
    int64_t qrow[kQV];  // row of q / out: t * n_head + h
    int64_t qp[kQV];
    bool qvalid[kQV];
    float qv[kQV][E];
    int64_t qp_min = INT64_MAX, qp_max = INT64_MIN;
#pragma unroll
    for (int i = 0; i < kQV; ++i) {
        const int64_t u = (int64_t)blockIdx.z * kQV + i;
        qvalid[i] = u < n_vec;
        const int64_t uc = qvalid[i] ? u : n_vec - 1;
        const int64_t t = uc / p.rep, h = (int64_t)kh * p.rep + uc % p.rep;
        qrow[i] = t * p.n_head + h;
        qp[i] = p.qpos ? (int64_t)p.qpos[t] : t;
        qp_min = min(qp_min, qp[i]);
        qp_max = max(qp_max, qp[i]);
#pragma unroll
        for (int e = 0; e < E; ++e) qv[i][e] = 0.0f;
        const float* qsrc = p.q + qrow[i] * p.head_dim;
#pragma unroll
        for (int e = 0; e < E; ++e)
            if (e0 + e < p.head_dim) qv[i][e] = qsrc[e0 + e];
    }

    // key range of this chunk; without explicit key positions, keys past the
    // largest query position (and before the earliest window) are masked
    int64_t j0 = (int64_t)chunk * p.chunk_len;
    int64_t j1 = min(j0 + p.chunk_len, p.n_kv);
    if (p.kpos == nullptr) {
        j1 = min(j1, qp_max + 1);
        if (p.window > 0) j0 = max(j0, qp_min - p.window + 1);
    }

    float m[kQV], l[kQV], acc[kQV][E];
#pragma unroll
    for (int i = 0; i < kQV; ++i) {
        m[i] = -INFINITY;
        l[i] = 0.0f;
#pragma unroll
        for (int e = 0; e < E; ++e) acc[i][e] = 0.0f;
    }

    const int64_t vstride = p.n_head_kv;
    for (int64_t jb = j0; jb < j1; jb += kKeysPerStep) {
        const int64_t j = jb + grp;
        const bool in = j < j1;
        const int64_t jc = in ? j : j0;  // an in-range key for the loads
        const int64_t vec = jc * vstride + kh;
        float kv[E], vv[E];
        load_vec<DT, E>(p.k, p.k_scale, vec, p.head_dim, e0, kv);
        load_vec<DT, E>(p.v, p.v_scale, vec, p.value_dim, e0, vv);
        const int64_t kp = p.kpos ? (int64_t)p.kpos[jc] : jc;
#pragma unroll
        for (int i = 0; i < kQV; ++i) {
            float d = 0.0f;
#pragma unroll
            for (int e = 0; e < E; ++e) d = __builtin_fmaf(qv[i][e], kv[e], d);
            d += __shfl_xor(d, 8, 16);
            d += __shfl_xor(d, 4, 16);
            d += __shfl_xor(d, 2, 16);
            d += __shfl_xor(d, 1, 16);
            const bool keep = in && key_kept(kp, qp[i], p.window);
            if (keep) {
                const float s = d * p.scale;
                const float mn = fmaxf(m[i], s);
                const float alpha = (m[i] == -INFINITY) ? 0.0f : expf(m[i] - mn);
                const float pr = expf(s - mn);
                l[i] = l[i] * alpha + pr;
#pragma unroll
                for (int e = 0; e < E; ++e) acc[i][e] = __builtin_fmaf(pr, vv[e], acc[i][e] * alpha);
                m[i] = mn;
            }
        }
    }

    // merge the 16 lane groups through LDS
#pragma unroll
    for (int i = 0; i < kQV; ++i) {
        if (li == 0) {
            sm[grp][i] = m[i];
            sl[grp][i] = l[i];
        }
#pragma unroll
        for (int e = 0; e < E; ++e) sacc[grp][i][e0 + e] = acc[i][e];
    }
    __syncthreads();
    // thread (query i, element d) for i < kQV, d < DVP: 4 * DVP <= 1024 work
    for (int w = tid; w < kQV * DVP; w += 64 * kAttnWaves) {
        const int i = w / DVP, d = w % DVP;
        float mt = -INFINITY;
#pragma unroll
        for (int g = 0; g < kAttnWaves * 4; ++g) mt = fmaxf(mt, sm[g][i]);
        float lt = 0.0f, at = 0.0f;
#pragma unroll
        for (int g = 0; g < kAttnWaves * 4; ++g) {
            const float wg = (sm[g][i] == -INFINITY) ? 0.0f : expf(sm[g][i] - mt);
            lt = __builtin_fmaf(sl[g][i], wg, lt);
            at = __builtin_fmaf(sacc[g][i][d], wg, at);
        }
        if (!qvalid[i] || d >= p.value_dim) continue;
        if constexpr (MERGE_OUT) {
            p.out[qrow[i] * p.value_dim + d] = at / fmaxf(lt, 1e-30f);
        } else {
            float* pr = p.part + ((int64_t)chunk * p.n_q * p.n_head + qrow[i]) * (p.value_dim + 2);
            pr[2 + d] = at;
            if (d == 0) {
                pr[0] = mt;
                pr[1] = lt;
            }
        }
    }
}

// Merge the chunks' (m, l, acc) of every (token, head): one thread per
// output element.
__global__ __launch_bounds__(256) void attn_combine_kernel(AttnParams p) {
    const int64_t rows = p.n_q * p.n_head;
    const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (idx >= rows * p.value_dim) return;
    const int64_t row = idx / p.value_dim, d = idx % p.value_dim;
    const int64_t cstride = rows * (p.value_dim + 2);
    const float* base = p.part + row * (p.value_dim + 2);
    float mt = -INFINITY;
    for (int c = 0; c < p.n_chunks; ++c) mt = fmaxf(mt, base[c * cstride]);
    float lt = 0.0f, at = 0.0f;
    for (int c = 0; c < p.n_chunks; ++c) {
        const float mc = base[c * cstride];
        const float wg = (mc == -INFINITY) ? 0.0f : expf(mc - mt);
        lt = __builtin_fmaf(base[c * cstride + 1], wg, lt);
        at = __builtin_fmaf(base[c * cstride + 2 + d], wg, at);
    }
    p.out[row * p.value_dim + d] = at / fmaxf(lt, 1e-30f);
}

using AttnKernel = void (*)(AttnParams);

template <int DT, bool MERGE_OUT>
AttnKernel pick_attn_e(int E) {
    switch (E) {
    case 4: return attn_kernel<DT, 4, MERGE_OUT>;
    case 8: return attn_kernel<DT, 8, MERGE_OUT>;
    case 16: return attn_kernel<DT, 16, MERGE_OUT>;
    default: return nullptr;
    }
}

AttnKernel pick_attn(int dt, int E, bool merge_out) {
    switch (dt) {
    case 0: return merge_out ? pick_attn_e<0, true>(E) : pick_attn_e<0, false>(E);
    case 1: return merge_out ? pick_attn_e<1, true>(E) : pick_attn_e<1, false>(E);
    case 2: return merge_out ? pick_attn_e<2, true>(E) : pick_attn_e<2, false>(E);
    default: return nullptr;
    }
}

struct AttnPlan {
    int E;
    int64_t q_tiles, chunk_len;
    int n_chunks;
};

bool attn_plan(int64_t n_q, int64_t n_head, int64_t n_head_kv, int64_t head_dim,
               int64_t value_dim, int64_t n_kv, AttnPlan& pl) {
    const int64_t width = std::max(head_dim, value_dim);
    pl.E = width <= 64 ? 4 : (width <= 128 ? 8 : (width <= 256 ? 16 : 0));
    if (pl.E == 0) return false;
    const int64_t rep = n_head / n_head_kv;
    pl.q_tiles = (n_q * rep + kQV - 1) / kQV;
    // enough workgroups to fill the chip: split the keys when the query
    // tiles alone do not (decode), chunks of at least 64 keys
    const int64_t base = n_head_kv * pl.q_tiles;
    const int64_t target = tune("attn_wgs", 1024);
    int64_t nc = std::max<int64_t>(1, (target + base - 1) / base);
    nc = std::min<int64_t>(nc, std::max<int64_t>(1, (n_kv + 63) / 64));
    int64_t cl = (n_kv + nc - 1) / nc;
    cl = (cl + kKeysPerStep - 1) / kKeysPerStep * kKeysPerStep;
    pl.chunk_len = cl;
    pl.n_chunks = (int)((n_kv + cl - 1) / cl);
    return true;
}

// ------------------------------------------------------------ KV writes
// One wave per vector: amax over the vector, scale amax/127 (int8) or amax/7
// (int4), 1 for a zero vector; q = round(x / scale) clipped; int4 packs two
// per byte, low nibble first (include/aero/kv.hpp:62-92). Row r of x
// (token t = r / heads, head h = r % heads) goes to vector
// ((phys0 + t) mod cap) * heads + h of the slot.
template <int DT>
__global__ __launch_bounds__(64) void kv_write_kernel(const float* x, int64_t n_rows,
                                                      int64_t heads, int64_t dim, int64_t phys0,
                                                      int64_t cap, void* q, float* scale) {
    const int64_t r = blockIdx.x;
    const int lane = threadIdx.x;
    const float* xr = x + r * dim;
    const int64_t t = r / heads, h = r % heads;
    const int64_t vec = ((phys0 + t) % cap) * heads + h;
    if constexpr (DT == 0) {
        float* o = static_cast<float*>(q) + vec * dim;
        for (int64_t i = lane; i < dim; i += 64) o[i] = xr[i];
        return;
    } else {
        float amax = 0.0f;
        for (int64_t i = lane; i < dim; i += 64) amax = fmaxf(amax, fabsf(xr[i]));
#pragma unroll
        for (int off = 32; off >= 1; off >>= 1) amax = fmaxf(amax, __shfl_xor(amax, off, 64));
        constexpr float qmax = DT == 1 ? 127.0f : 7.0f;
        const float sc = amax > 0.0f ? amax / qmax : 1.0f;
        if (lane == 0) scale[vec] = sc;
        if constexpr (DT == 1) {
            int8_t* o = static_cast<int8_t*>(q) + vec * dim;
            for (int64_t i = lane; i < dim; i += 64) {
                const float v = fminf(fmaxf(roundf(xr[i] / sc), -127.0f), 127.0f);
                o[i] = (int8_t)v;
            }
        } else {
            uint8_t* o = static_cast<uint8_t*>(q) + vec * (dim / 2);
            for (int64_t i = lane; i < dim / 2; i += 64) {
                const float a = fminf(fmaxf(roundf(xr[2 * i] / sc), -7.0f), 7.0f);
                const float b = fminf(fmaxf(roundf(xr[2 * i + 1] / sc), -7.0f), 7.0f);
                o[i] = (uint8_t)(((int)a & 15) | (((int)b & 15) << 4));
            }
        }
    }
}

// ------------------------------------------------------------- softmax
// One workgroup of 256 per row: max, then exp(v - max) and its sum, then the
// product with 1/sum (0 when the sum is not positive), src/tensor.cpp:167-178.
__global__ __launch_bounds__(256) void softmax_rows_kernel(const float* x, float* y,
                                                           int64_t n_cols) {
    __shared__ float red[4];
    const float* xr = x + (int64_t)blockIdx.x * n_cols;
    float* yr = y + (int64_t)blockIdx.x * n_cols;
    const int tid = threadIdx.x;
    float m = -INFINITY;
    for (int64_t i = tid; i < n_cols; i += 256) m = fmaxf(m, xr[i]);
    m = fmaxf(m, __shfl_xor(m, 32, 64));
    m = fmaxf(m, __shfl_xor(m, 16, 64));
    m = fmaxf(m, __shfl_xor(m, 8, 64));
    m = fmaxf(m, __shfl_xor(m, 4, 64));
    m = fmaxf(m, __shfl_xor(m, 2, 64));
    m = fmaxf(m, __shfl_xor(m, 1, 64));
    if ((tid & 63) == 0) red[tid >> 6] = m;
    __syncthreads();
    m = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    __syncthreads();
    float s = 0.0f;
    for (int64_t i = tid; i < n_cols; i += 256) s += expf(xr[i] - m);
    s = group_sum<64>(s);
    if ((tid & 63) == 0) red[tid >> 6] = s;
    __syncthreads();
    s = (red[0] + red[1]) + (red[2] + red[3]);
    const float inv = s > 0.0f ? 1.0f / s : 0.0f;
    for (int64_t i = tid; i < n_cols; i += 256) yr[i] = expf(xr[i] - m) * inv;
}

}  // namespace

int64_t attn_workspace_bytes(int64_t n_q, int64_t n_head, int64_t n_head_kv, int64_t head_dim,
                             int64_t value_dim, int64_t n_kv) {
    AttnPlan pl;
    if (n_q <= 0 || n_head <= 0 || n_head_kv <= 0 || n_head % n_head_kv || n_kv <= 0 ||
        !attn_plan(n_q, n_head, n_head_kv, head_dim, value_dim, n_kv, pl))
        return 0;
    if (pl.n_chunks <= 1) return 0;
    return (int64_t)pl.n_chunks * n_q * n_head * (value_dim + 2) * 4;
}

bool attention_dev(const float* q, int kv_dt, const void* k, const float* k_scale, const void* v,
                   const float* v_scale, float* out, int64_t n_q, int64_t n_head,
                   int64_t n_head_kv, int64_t head_dim, int64_t value_dim, float scale,
                   const int32_t* qpos, const int32_t* kpos, int64_t n_kv, int window,
                   void* workspace, int64_t ws_bytes, hipStream_t s) {
    if (n_q <= 0 || n_head <= 0 || n_head_kv <= 0 || head_dim <= 0 || value_dim <= 0 ||
        n_kv <= 0 || n_head % n_head_kv) {
        set_error("attention: bad sizes (n_q=%lld n_head=%lld n_head_kv=%lld head_dim=%lld "
                  "value_dim=%lld n_kv=%lld)", (long long)n_q, (long long)n_head,
                  (long long)n_head_kv, (long long)head_dim, (long long)value_dim,
                  (long long)n_kv);
        return false;
    }
    if (q == nullptr || k == nullptr || v == nullptr || out == nullptr || kv_dt < 0 ||
        kv_dt > 2 || (kv_dt != 0 && (k_scale == nullptr || v_scale == nullptr)) ||
        (kv_dt == 2 && (head_dim % 2 || value_dim % 2))) {
        set_error("attention: bad pointers or kv dtype %d", kv_dt);
        return false;
    }
    if (kv_dt == 0 && (!aligned16(k) || !aligned16(v) || head_dim % 4 || value_dim % 4)) {
        set_error("attention: fp32 K/V must be 16-byte aligned with dims a multiple of 4");
        return false;
    }
    AttnPlan pl;
    if (!attn_plan(n_q, n_head, n_head_kv, head_dim, value_dim, n_kv, pl)) {
        set_error("attention: head_dim/value_dim %lld/%lld above 256", (long long)head_dim,
                  (long long)value_dim);
        return false;
    }
    const int64_t need = pl.n_chunks > 1
                             ? (int64_t)pl.n_chunks * n_q * n_head * (value_dim + 2) * 4 : 0;
    if (need > ws_bytes || (need > 0 && workspace == nullptr)) {
        set_error("attention: workspace %lld bytes < %lld needed", (long long)ws_bytes,
                  (long long)need);
        return false;
    }
    if (pl.q_tiles > 65535 || n_head_kv > 65535) {
        set_error("attention: grid too large");
        return false;
    }
    AttnParams p{q, k, k_scale, v, v_scale, out, static_cast<float*>(workspace), qpos, kpos,
                 n_q, n_head, n_head_kv, head_dim, value_dim, n_kv,
                 (int)(n_head / n_head_kv), window, scale, pl.chunk_len, pl.n_chunks};
    AttnKernel kern = pick_attn(kv_dt, pl.E, pl.n_chunks == 1);
    if (!launch("attn_kernel", kern, dim3((unsigned)pl.n_chunks, (unsigned)n_head_kv,
                                          (unsigned)pl.q_tiles),
                dim3(64 * kAttnWaves), 0, s, p))
        return false;
    if (pl.n_chunks > 1) {
        const int64_t n = n_q * n_head * value_dim;
        if (!launch("attn_combine_kernel", attn_combine_kernel, dim3((unsigned)((n + 255) / 256)),
                    dim3(256), 0, s, p))
            return false;
    }
    return true;
}

bool kv_write_dev(int dt, const float* x, int64_t n_tok, int64_t heads, int64_t dim,
                  int64_t phys0, int64_t cap, void* q, float* scale, hipStream_t s) {
    if (x == nullptr || q == nullptr || n_tok < 0 || heads <= 0 || dim <= 0 || cap <= 0 ||
        phys0 < 0 || dt < 0 || dt > 2 || (dt != 0 && scale == nullptr) || (dt == 2 && dim % 2) ||
        n_tok > cap) {
        set_error("kv_write: bad arguments (dt=%d n_tok=%lld heads=%lld dim=%lld cap=%lld)", dt,
                  (long long)n_tok, (long long)heads, (long long)dim, (long long)cap);
        return false;
    }
    const int64_t rows = n_tok * heads;
    if (rows == 0) return true;
    if (rows > 0x7fffffff) {
        set_error("kv_write: too many vectors");
        return false;
    }
    switch (dt) {
    case 0:
        return launch("kv_write_kernel", kv_write_kernel<0>, dim3((unsigned)rows), dim3(64), 0, s,
                      x, rows, heads, dim, phys0, cap, q, scale);
    case 1:
        return launch("kv_write_kernel", kv_write_kernel<1>, dim3((unsigned)rows), dim3(64), 0, s,
                      x, rows, heads, dim, phys0, cap, q, scale);
    default:
        return launch("kv_write_kernel", kv_write_kernel<2>, dim3((unsigned)rows), dim3(64), 0, s,
                      x, rows, heads, dim, phys0, cap, q, scale);
    }
}

bool softmax_rows_dev(const float* x, float* y, int64_t n_rows, int64_t n_cols, hipStream_t s) {
    if (x == nullptr || y == nullptr || n_rows < 0 || n_cols <= 0 || n_rows > 0x7fffffff) {
        set_error("softmax: bad arguments");
        return false;
    }
    if (n_rows == 0) return true;
    return launch("softmax_rows_kernel", softmax_rows_kernel, dim3((unsigned)n_rows), dim3(256), 0,
                  s, x, y, n_cols);
}

}  // namespace aero

extern "C" {

int64_t aero_hip_attention_workspace(int64_t n_q, int64_t n_head, int64_t n_head_kv,
                                     int64_t head_dim, int64_t value_dim, int64_t n_kv) {
    return aero::attn_workspace_bytes(n_q, n_head, n_head_kv, head_dim, value_dim, n_kv);
}

int aero_hip_attention(const float* q, int kv_dt, const void* k, const float* k_scale,
                       const void* v, const float* v_scale, float* out, int64_t n_q,
                       int64_t n_head, int64_t n_head_kv, int64_t head_dim, int64_t value_dim,
                       float scale, const int32_t* qpos, const int32_t* kpos, int64_t n_kv,
                       int window, void* workspace, int64_t ws_bytes, void* stream) {
    aero::clear_error();
    return aero::attention_dev(q, kv_dt, k, k_scale, v, v_scale, out, n_q, n_head, n_head_kv,
                               head_dim, value_dim, scale, qpos, kpos, n_kv, window, workspace,
                               ws_bytes, (hipStream_t)stream) ? 1 : 0;
}

int aero_hip_kv_write(int dt, const float* x, int64_t n_tok, int64_t heads, int64_t dim,
                      int64_t phys0, int64_t cap, void* q, float* scale, void* stream) {
    aero::clear_error();
    return aero::kv_write_dev(dt, x, n_tok, heads, dim, phys0, cap, q, scale,
                              (hipStream_t)stream) ? 1 : 0;
}

int aero_hip_softmax_rows(const float* x, float* y, int64_t n_rows, int64_t n_cols,
                          void* stream) {
    aero::clear_error();
    return aero::softmax_rows_dev(x, y, n_rows, n_cols, (hipStream_t)stream) ? 1 : 0;
}

}  // extern "C"
