// Attention core and KV cache on gfx950: the reference's grouped-query
// attention with an online softmax (src/transformer.cpp:120-214), its row
// softmax (src/tensor.cpp:167-178) and the KV cache vector quantisers
// (include/aero/kv.hpp:62-103, src/kv.cpp:13-46).
//
// Two attention kernels share one plan. Keys are split into chunks when the
// query tiles alone do not fill the chip (decode: one query, many keys); each
// chunk's (max m, sum l, accumulator) is merged by attn_combine_kernel.
//  * attn_mfma_kernel (head_dim == value_dim in {64, 128, 256}): scores and
//    the value sum on the fp32 matrix cores, a wave per 16-key tile, the
//    workgroup's four waves sharing one 16-query tile.
//  * attn_kernel (any other width up to 256): 16-lane groups own a key, the
//    dot product is reduced with lane shuffles, four query vectors a
//    workgroup.
// K / V are read in the cache's format (fp32, or int8 / int4 with one fp32
// scale per vector).
//
// Masking as the reference: key j (position kpos[j] or j) is kept for query
// position qp when kp <= qp and, with window > 0, qp - kp < window; a query
// with no kept key gives zeros. When kpos is absent, keys past the tile's
// largest query position (or before its earliest window start) are skipped.
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
    float* part;           // several chunks: acc [n_chunks][n_q * n_head][value_dim],
                           // then (m, l) [n_chunks][n_q * n_head][2]
    const int32_t* qpos;   // [n_q] or null (= t)
    const int32_t* kpos;   // [n_kv] or null (= j)
    int64_t n_q, n_head, n_head_kv, head_dim, value_dim, n_kv;
    int rep;               // n_head / n_head_kv
    int window;
    float scale;
    int64_t chunk_len;     // keys per chunk (a multiple of the kernel's keys per step)
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
            const int64_t pi = (int64_t)chunk * p.n_q * p.n_head + qrow[i];
            p.part[pi * p.value_dim + d] = at;
            if (d == 0) {
                float* ml = p.part + (int64_t)p.n_chunks * p.n_q * p.n_head * p.value_dim + 2 * pi;
                ml[0] = mt;
                ml[1] = lt;
            }
        }
    }
}

// ------------------------------------------------------------ MFMA path
// Scores and the value sum on the fp32 matrix cores. v_mfma_f32_16x16x4f32:
// lane l (g = l / 16, c = l % 16) supplies A[c][g] and B[g][c] and receives
// D[4g + r][c], r = 0..3. A wave owns a tile of 16 query vectors (column c =
// query vector) and walks the keys 16 at a time:
//  * S^T = K . Q^T with A = K (row = key c) and B = Q^T. The head dimension is
//    permuted (a dot product does not depend on the order of its terms): lane
//    group g owns D/4 elements of key c and of query c, taken as 16-byte
//    pieces that interleave with the other groups' (kdim), so the four
//    groups' loads of one key are adjacent.
//  * Lane l then holds the scores of query c against keys 4g + r, which is
//    the A operand of O += P . V when the value step r takes keys
//    {4g + r : g = 0..3}. B = V[key 4g + r][...]: lane c of the group owns
//    DV/16 value elements, 16-byte pieces interleaved across the 16 lanes
//    (vdim), so a row's loads are contiguous.
//  * Output tile t, lane l: O[query 4g + r][vdim(c, t)].
// Integer caches multiply the integer codes (exact in fp32); the key scale
// multiplies the score and the value scale the probability.
//
// The four waves of a workgroup share one query tile and take every fourth
// key tile of the chunk (balanced under a causal mask); their (m, l, acc) are
// merged through LDS. Workgroups run the last query tiles (in causal prefill
// the longest) first.
template <int DT>
constexpr int kv_bits() { return DT == 0 ? 32 : (DT == 1 ? 8 : 4); }

// Loaded in place of an absent position array: the loads of positions stay
// unconditional (a load under a branch makes the compiler wait for every
// load in flight where the branches join) and the value is selected after.
__device__ int32_t g_no_position = 0;

__device__ __forceinline__ int32_t position_or(const int32_t* pos, int64_t i, int64_t dflt) {
    const int32_t* a = pos ? pos + i : &g_no_position;
    const int32_t v = *a;
    return pos ? v : (int32_t)dflt;
}

// N bytes (4-byte multiple, or 2) at p into words.
template <int N>
__device__ __forceinline__ void load_words(const uint8_t* p, uint32_t* w) {
    if constexpr (N % 16 == 0) {
#pragma unroll
        for (int i = 0; i < N / 16; ++i) {
            const uint4 x = *reinterpret_cast<const uint4*>(p + 16 * i);
            w[4 * i] = x.x; w[4 * i + 1] = x.y; w[4 * i + 2] = x.z; w[4 * i + 3] = x.w;
        }
    } else if constexpr (N % 8 == 0) {
#pragma unroll
        for (int i = 0; i < N / 8; ++i) {
            const uint2 x = *reinterpret_cast<const uint2*>(p + 8 * i);
            w[2 * i] = x.x; w[2 * i + 1] = x.y;
        }
    } else if constexpr (N % 4 == 0) {
#pragma unroll
        for (int i = 0; i < N / 4; ++i) w[i] = reinterpret_cast<const uint32_t*>(p)[i];
    } else {
        static_assert(N == 2, "slice size");
        w[0] = *reinterpret_cast<const uint16_t*>(p);
    }
}

// element e of a slice held as words: fp32 bits, int8 or int4 (low nibble first)
template <int DT>
__device__ __forceinline__ float slice_elem(const uint32_t* w, int e) {
    if constexpr (DT == 0) {
        return __uint_as_float(w[e]);
    } else if constexpr (DT == 1) {
        return (float)((int32_t)(w[e >> 2] << (24 - 8 * (e & 3))) >> 24);
    } else {
        return (float)((int32_t)(w[e >> 3] << (28 - 4 * (e & 7))) >> 28);
    }
}

template <int DT, int D, int DV>
struct KvTile {
    static constexpr int KS = D / 4, VS = DV / 16;
    static constexpr int KB = KS * kv_bits<DT>() / 8, VB = VS * kv_bits<DT>() / 8;
    static constexpr int KW = (KB + 3) / 4, VW = (VB + 3) / 4;
    // bytes and elements per load, loads per lane
    static constexpr int KLB = KB < 16 ? KB : 16, KLE = KLB * 8 / kv_bits<DT>(), KNI = KB / KLB;
    static constexpr int VLB = VB < 16 ? VB : 16, VLE = VLB * 8 / kv_bits<DT>(), VNI = VB / VLB;
    // head-dimension index of element j of lane group g's key / query slice
    static __device__ __forceinline__ int kdim(int g, int j) {
        return (j / KLE) * (4 * KLE) + g * KLE + j % KLE;
    }
    // value index of element t of lane c's value slice (and output column)
    static __device__ __forceinline__ int vdim(int c, int t) {
        return (t / VLE) * (16 * VLE) + c * VLE + t % VLE;
    }
    uint32_t k[KW];
    uint32_t v[4][VW];
    // scales (integer caches) and position of key c; lanes 4g + r hand them
    // to the lanes that need key 4g + r
    float ks, vs;
    int32_t kp;

    // keys kb .. kb + 15, clamped to < j1 for the loads
    __device__ __forceinline__ void load(const AttnParams& p, int64_t kb, int64_t j1, int g,
                                         int c, int kh) {
        const int64_t hk = p.n_head_kv;
        constexpr int64_t KVEC = (int64_t)D * kv_bits<DT>() / 8;
        constexpr int64_t VVEC = (int64_t)DV * kv_bits<DT>() / 8;
        const int64_t kk = min(kb + c, j1 - 1);
        const uint8_t* kr = static_cast<const uint8_t*>(p.k) + (kk * hk + kh) * KVEC;
#pragma unroll
        for (int i = 0; i < KNI; ++i) load_words<KLB>(kr + (4 * i + g) * KLB, k + i * KLB / 4);
        if constexpr (DT != 0) {
            ks = p.k_scale[kk * hk + kh];
            vs = p.v_scale[kk * hk + kh];
        }
        kp = position_or(p.kpos, kk, 0);
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int64_t kv = min(kb + 4 * g + r, j1 - 1);
            const uint8_t* vr = static_cast<const uint8_t*>(p.v) + (kv * hk + kh) * VVEC;
#pragma unroll
            for (int i = 0; i < VNI; ++i)
                load_words<VLB>(vr + (16 * i + c) * VLB, v[r] + i * VLB / 4);
        }
    }
};

// The four waves' (m, l, acc) of one 16-query tile merged through LDS, then
// the output (one chunk) or the chunk's partials written. The 16 queries'
// merge weights, sums and output rows are computed once (64 threads: wave x,
// query qi), then each thread writes elements d of query vectors qi.
template <typename Tile, int DV, bool MERGE_OUT>
__device__ __forceinline__ void merge_tile(const AttnParams& p, float m, float ls,
                                           const v4f (&acc)[DV / 16], int64_t tile,
                                           int64_t n_vec, int chunk, int kh, int wave, int g,
                                           int c) {
    constexpr int VS = DV / 16;
    ls += __shfl_xor(ls, 16);
    ls += __shfl_xor(ls, 32);
    __shared__ float sm[4][16], sl[4][16], sw[4][16], smt[16], slt[16];
    __shared__ int32_t srow[16];
    __shared__ float sacc[4][16][DV + 4];
    if (g == 0) {
        sm[wave][c] = m;
        sl[wave][c] = ls;
    }
#pragma unroll
    for (int r = 0; r < 4; ++r)
#pragma unroll
        for (int t = 0; t < VS; ++t) sacc[wave][4 * g + r][Tile::vdim(c, t)] = acc[t][r];
    __syncthreads();
    const int tid = threadIdx.x;
    if (tid < 64) {
        const int x = tid >> 4, qi = tid & 15;
        const float mt = fmaxf(fmaxf(sm[0][qi], sm[1][qi]), fmaxf(sm[2][qi], sm[3][qi]));
        const float wg = (sm[x][qi] == -INFINITY) ? 0.0f : expf(sm[x][qi] - mt);
        sw[x][qi] = wg;
        float lw = sl[x][qi] * wg;
        lw += __shfl_xor(lw, 16);
        lw += __shfl_xor(lw, 32);
        if (x == 0) {
            smt[qi] = mt;
            slt[qi] = lw;
            const int64_t uq = tile * 16 + qi;
            srow[qi] = uq < n_vec ? (int32_t)((uq / p.rep) * p.n_head + (int64_t)kh * p.rep +
                                              uq % p.rep)
                                  : -1;
        }
    }
    __syncthreads();
    const int64_t rows = p.n_q * p.n_head;
#pragma unroll
    for (int w0 = 0; w0 < 16 * DV; w0 += 256) {
        const int w = w0 + tid;
        const int qi = w / DV, d = w % DV;
        const int32_t row = srow[qi];
        if (row < 0) break;  // rows past the last vector: qi only grows
        float at = 0.0f;
#pragma unroll
        for (int x = 0; x < 4; ++x) at = __builtin_fmaf(sacc[x][qi][d], sw[x][qi], at);
        const float lt = slt[qi];
        if constexpr (MERGE_OUT) {
            p.out[(int64_t)row * DV + d] = at / fmaxf(lt, 1e-30f);
        } else {
            const int64_t pi = (int64_t)chunk * rows + row;
            p.part[pi * DV + d] = at;
            if (d == 0) {
                float* ml = p.part + (int64_t)p.n_chunks * rows * DV + 2 * pi;
                ml[0] = smt[qi];
                ml[1] = lt;
            }
        }
    }
}

template <int DT, int D, int DV, bool MERGE_OUT>
__global__ __launch_bounds__(256) void attn_mfma_kernel(AttnParams p) {
    using Tile = KvTile<DT, D, DV>;
    constexpr int KS = Tile::KS, VS = Tile::VS;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int g = lane >> 4, c = lane & 15;
    const int chunk = blockIdx.x, kh = blockIdx.y;
    const int64_t n_vec = p.n_q * p.rep;
    const int64_t tile = (int64_t)(gridDim.z - 1 - blockIdx.z);
    constexpr int64_t istep = 4;

    // this chunk's keys (every load stays below c1); the wave's first key
    // tile is issued before the query positions, which may narrow the range,
    // arrive: one memory round trip instead of two
    const int64_t c0 = (int64_t)chunk * p.chunk_len;
    const int64_t c1 = min(c0 + p.chunk_len, p.n_kv);
    const int64_t tiles_c = (c1 - c0 + 15) / 16;
    const int64_t i_spec = wave;
    // the next tile is loaded while this one is used: integer caches (two
    // tiles of int8 / int4 fit in the registers one fp32 tile takes) and
    // single-chunk calls (prefill) at head dim 256, which runs one wave a SIMD
    // either way (2048-token Gemma-3 prefill 288 -> 253 us on MI355X). Not at
    // head dim 128, where an fp32 prefetch costs the second wave a SIMD (the
    // 512-token prefill measured slower), nor for decode chunks, whose waves
    // take one tile and would load it again (the next tile is clamped to the
    // chunk's last). The next tile is copied into this one's registers: at
    // head dim 256 two alternating register sets would not fit without spills.
    constexpr bool PF = DT != 0 || (D == 256 && MERGE_OUT);
    Tile tl, nx;
    tl.load(p, c0 + 16 * min(i_spec, tiles_c - 1), c1, g, c, kh);

    // query vector of column c: token t, head kh * rep + u % rep
    const int64_t u = tile * 16 + c;
    const bool qok = u < n_vec;
    const int64_t uc = qok ? u : n_vec - 1;
    const int64_t tq = uc / p.rep;
    const int64_t qrow = tq * p.n_head + (int64_t)kh * p.rep + uc % p.rep;
    const int64_t qp = position_or(p.qpos, tq, tq);
    float qs[KS];
    {
        const float* src = p.q + qrow * D;
#pragma unroll
        for (int e = 0; e < KS; e += 4) {
            const float4 f = *reinterpret_cast<const float4*>(src + Tile::kdim(g, e));
            qs[e] = qok ? f.x : 0.0f;
            qs[e + 1] = qok ? f.y : 0.0f;
            qs[e + 2] = qok ? f.z : 0.0f;
            qs[e + 3] = qok ? f.w : 0.0f;
        }
    }
    int64_t qmin = qp, qmax = qp;
#pragma unroll
    for (int off = 8; off >= 1; off >>= 1) {
        qmin = min(qmin, (int64_t)__shfl_xor(qmin, off, 16));
        qmax = max(qmax, (int64_t)__shfl_xor(qmax, off, 16));
    }

    // key tiles [i_lo, i_hi) of the chunk can hold kept keys: without key
    // positions, none past the tile's last query position or before its
    // earliest window
    int64_t i_lo = 0, i_hi = tile * 16 < n_vec ? tiles_c : 0;
    if (p.kpos == nullptr) {
        i_hi = min(i_hi, max<int64_t>(0, (qmax + 1 - c0 + 15) / 16));
        if (p.window > 0) i_lo = max<int64_t>(0, (qmin - p.window + 1 - c0) / 16);
    }
    int64_t i = i_lo + (((wave - i_lo) % 4) + 4) % 4;
    if (i != i_spec && i < i_hi) tl.load(p, c0 + 16 * i, c1, g, c, kh);

    float m = -INFINITY, ls = 0.0f;
    v4f acc[VS];
#pragma unroll
    for (int t = 0; t < VS; ++t) acc[t] = v4f{0.f, 0.f, 0.f, 0.f};

    while (i < i_hi) {
        const int64_t kb = c0 + 16 * i;
        // (clamped to the chunk's last tile: in bounds, and no branch for the
        // wait counters to merge)
        if constexpr (PF) nx.load(p, c0 + 16 * min(i + istep, tiles_c - 1), c1, g, c, kh);
        v4f s0 = {0.f, 0.f, 0.f, 0.f}, s1 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int j = 0; j < KS; j += 2) {
            s0 = __builtin_amdgcn_mfma_f32_16x16x4f32(slice_elem<DT>(tl.k, j), qs[j], s0, 0,
                                                      0, 0);
            s1 = __builtin_amdgcn_mfma_f32_16x16x4f32(slice_elem<DT>(tl.k, j + 1), qs[j + 1],
                                                      s1, 0, 0, 0);
        }
        float sc[4];
        float tm = -INFINITY;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int64_t kj = kb + 4 * g + r;
            const int64_t kp = p.kpos ? (int64_t)__shfl(tl.kp, 4 * g + r) : kj;
            const bool keep = qok && kj < c1 && key_kept(kp, qp, p.window);
            float y = (s0[r] + s1[r]);
            if constexpr (DT != 0) y *= __shfl(tl.ks, 4 * g + r);
            sc[r] = keep ? y * p.scale : -INFINITY;
            tm = fmaxf(tm, sc[r]);
        }
        tm = fmaxf(tm, __shfl_xor(tm, 16));
        tm = fmaxf(tm, __shfl_xor(tm, 32));
        const float mn = fmaxf(m, tm);
        const float alpha = (m == -INFINITY) ? 0.0f : expf(m - mn);
        float pr[4];
        float psum = 0.0f;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            pr[r] = (sc[r] == -INFINITY) ? 0.0f : expf(sc[r] - mn);
            psum += pr[r];
            if constexpr (DT != 0) pr[r] *= __shfl(tl.vs, 4 * g + r);
        }
        ls = ls * alpha + psum;
        m = mn;
        // rescale the rows of query 4g + r by that query's alpha (lane 4g + r)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const float ar = __shfl(alpha, 4 * g + r);
#pragma unroll
            for (int t = 0; t < VS; ++t) acc[t][r] *= ar;
        }
#pragma unroll
        for (int r = 0; r < 4; ++r)
#pragma unroll
            for (int t = 0; t < VS; ++t)
                acc[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(
                    pr[r], slice_elem<DT>(tl.v[r], t), acc[t], 0, 0, 0);
        i += istep;
        if (i >= i_hi) break;
        if constexpr (PF)
            tl = nx;
        else
            tl.load(p, c0 + 16 * i, c1, g, c, kh);
    }
    merge_tile<Tile, DV, MERGE_OUT>(p, m, ls, acc, tile, n_vec, chunk, kh, wave, g, c);
}

// ---------------------------------------------------- integer caches, fp16
// Integer caches on the fp16 matrix cores (v_mfma_f32_16x16x32_f16: lane
// (r, g) supplies A[r][8g..8g+7] and B[8g..8g+7][r], receives D[4g+v][r]).
// The codes are exact in fp16: a code c becomes the fp16 bits 0x6400 | u of
// 1024 + u, u = c + 128 (int8) or c + 8 (int4), minus 1152 or 1032. q, scaled
// by 2^(14-e) per query (|q| < 2^15), and each tile's probabilities times the
// value scales, scaled by 2^(14-e) of the tile's largest value scale, are
// split into two fp16 parts (hi = fp16(v), lo = fp16(v - hi)): every product
// is exact and the fp32 sums carry about 22 bits of each operand. A wave
// takes 32 keys a step, two halves of 16 loaded as attn_mfma_kernel's tiles:
//  * scores: D[key][query] over K = 32 dimensions a matrix step; lane group
//    g's 8 values of a step are elements 8s..8s+7 of its key slice (the
//    order of int4 nibbles within a dword: 0, 4, 2, 6, 1, 5, 3, 7);
//  * value sum: D[query][value dim] over the 32 keys in one matrix step a
//    value tile, lane group g's k-slots being keys 4g..4g+3 of each half:
//    the probabilities the lane holds after the scores, and the codes of
//    those keys' value rows it loaded.
typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef unsigned int v2u __attribute__((ext_vector_type(2)));

__device__ __forceinline__ h2 u32_h2(uint32_t u) { return __builtin_bit_cast(h2, u); }
__device__ __forceinline__ uint32_t h2_u32(h2 h) { return __builtin_bit_cast(uint32_t, h); }

// the 8 codes of key-slice step s as fp16, in the order described above
template <int DT>
__device__ __forceinline__ h8 key_codes(const uint32_t* k, int s) {
    constexpr uint32_t E = 0x64646464u;
    if constexpr (DT == 1) {
        const h2 off = h2{(_Float16)-1152.f, (_Float16)-1152.f};
        const uint32_t u0 = k[2 * s] ^ 0x80808080u, u1 = k[2 * s + 1] ^ 0x80808080u;
        const h2 a0 = u32_h2(__builtin_amdgcn_perm(E, u0, 0x04010400u)) + off;
        const h2 a1 = u32_h2(__builtin_amdgcn_perm(E, u0, 0x04030402u)) + off;
        const h2 a2 = u32_h2(__builtin_amdgcn_perm(E, u1, 0x04010400u)) + off;
        const h2 a3 = u32_h2(__builtin_amdgcn_perm(E, u1, 0x04030402u)) + off;
        return __builtin_bit_cast(h8, make_uint4(h2_u32(a0), h2_u32(a1), h2_u32(a2), h2_u32(a3)));
    } else {
        const h2 off = h2{(_Float16)-1032.f, (_Float16)-1032.f};
        const uint32_t u = k[s] ^ 0x88888888u;
        const uint32_t lo = u & 0x0F0F0F0Fu, hi = (u >> 4) & 0x0F0F0F0Fu;
        const h2 a0 = u32_h2(__builtin_amdgcn_perm(E, lo, 0x04020400u)) + off;  // 0, 4
        const h2 a1 = u32_h2(__builtin_amdgcn_perm(E, lo, 0x04030401u)) + off;  // 2, 6
        const h2 a2 = u32_h2(__builtin_amdgcn_perm(E, hi, 0x04020400u)) + off;  // 1, 5
        const h2 a3 = u32_h2(__builtin_amdgcn_perm(E, hi, 0x04030401u)) + off;  // 3, 7
        return __builtin_bit_cast(h8, make_uint4(h2_u32(a0), h2_u32(a1), h2_u32(a2), h2_u32(a3)));
    }
}

// element i of a key-slice operand is slice element 8s + key_order(i)
template <int DT>
__device__ __forceinline__ constexpr int key_order(int i) {
    return DT == 1 ? i : ((i & 1) ? 4 : 0) + ((i >> 1) & 1) * 2 + (i >> 2);
}

// codes of element t of two value rows (words a, b of those rows) as fp16
// (code_a, code_b)
template <int DT>
__device__ __forceinline__ uint32_t value_pair(const uint32_t* a, const uint32_t* b, int t) {
    if constexpr (DT == 1) {
        const uint32_t byte = (uint32_t)(t & 3);
        const uint32_t sel = 0x0C000C00u | ((4u + byte) << 16) | byte;
        const uint32_t x = __builtin_amdgcn_perm(b[t >> 2], a[t >> 2], sel) ^ 0x64806480u;
        return h2_u32(u32_h2(x) + h2{(_Float16)-1152.f, (_Float16)-1152.f});
    } else {
        const uint32_t byte = (uint32_t)((t >> 1) & 3);
        const uint32_t sel = 0x0C000C00u | ((4u + byte) << 16) | byte;
        uint32_t x = __builtin_amdgcn_perm(b[t >> 3], a[t >> 3], sel);
        x = ((t & 1) ? (x >> 4) : x) & 0x000F000Fu;
        return h2_u32(u32_h2(x ^ 0x64086408u) + h2{(_Float16)-1032.f, (_Float16)-1032.f});
    }
}

// v = 2^scale-shifted value split into fp16 hi and lo
__device__ __forceinline__ void split2(float v, _Float16& hi, _Float16& lo) {
    hi = (_Float16)v;
    lo = (_Float16)(v - (float)hi);
}

// One kv head's keys [c0, c0 + n) of an integer cache, read through buffer
// descriptors. A 16-key tile's descriptors start at its first key and end at
// the chunk's last one, so a lane's byte offsets within a tile are fixed (no
// per-step address arithmetic: the tile's place is wave-uniform), and a key
// at or past the chunk's end reads as zero codes, scales and positions (the
// hardware's range check) instead of being clamped to the last key. Lane
// (g, c) loads key c's slice (the scores' operand), the value rows of keys
// 4g + r (the value sum's operand), and those keys' scales and positions.
// The host keeps a chunk's bytes below 2^31.
template <int DT, int D, bool KPOS>
struct IntKv {
    using Tile = KvTile<DT, D, D>;
    static constexpr int KVEC = D * kv_bits<DT>() / 8;  // bytes of a key or value vector
    static constexpr int KW = Tile::KW, VW = Tile::VW, KLB = Tile::KLB, KNI = Tile::KNI;
    static constexpr int VLB = Tile::VLB, VNI = Tile::VNI;
    struct T {
        uint32_t k[KW];
        uint32_t v[4][VW];
        float ks[4], vs[4];
        int32_t kp[4];
    };
    const uint8_t* kb;
    const uint8_t* vb;
    const uint8_t* ksb;
    const uint8_t* vsb;
    const uint8_t* kpb;
    uint32_t kstride, sstride;   // bytes from one key to the next: n_head_kv * KVEC, * 4
    int32_t n;                   // keys in the chunk
    uint32_t ko, vo[4], so[4], po[4];

    __device__ __forceinline__ IntKv(const AttnParams& p, int64_t c0, int64_t c1, int kh, int g,
                                     int c) {
        const int64_t hk = p.n_head_kv;
        kb = static_cast<const uint8_t*>(p.k) + (c0 * hk + kh) * KVEC;
        vb = static_cast<const uint8_t*>(p.v) + (c0 * hk + kh) * KVEC;
        ksb = reinterpret_cast<const uint8_t*>(p.k_scale + c0 * hk + kh);
        vsb = reinterpret_cast<const uint8_t*>(p.v_scale + c0 * hk + kh);
        kpb = KPOS ? reinterpret_cast<const uint8_t*>(p.kpos + c0) : nullptr;
        kstride = (uint32_t)(hk * KVEC);
        sstride = (uint32_t)(hk * 4);
        n = (int32_t)(c1 - c0);
        ko = (uint32_t)c * kstride + (uint32_t)(g * KLB);
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            vo[r] = (uint32_t)(4 * g + r) * kstride + (uint32_t)(c * VLB);
            so[r] = (uint32_t)(4 * g + r) * sstride;
            po[r] = (uint32_t)(4 * g + r) * 4u;
        }
    }

    // descriptor over [base + j0 * stride, the end of the chunk's last vector)
    static __device__ __forceinline__ __amdgpu_buffer_rsrc_t rsrc(const uint8_t* base, int32_t j0,
                                                                   int32_t n, uint32_t stride,
                                                                   uint32_t vec) {
        const int32_t left = n - j0;
        const uint32_t bytes = left > 0 ? (uint32_t)(left - 1) * stride + vec : 0u;
        return __builtin_amdgcn_make_buffer_rsrc(
            const_cast<uint8_t*>(base) + (int64_t)j0 * stride, 0, (int)bytes, kBufferDword3);
    }

    template <int N>
    static __device__ __forceinline__ void words(__amdgpu_buffer_rsrc_t r, uint32_t off,
                                                 uint32_t* w) {
        if constexpr (N == 16) {
            const v4u x = __builtin_amdgcn_raw_buffer_load_b128(r, (int)off, 0, 0);
            w[0] = x.x; w[1] = x.y; w[2] = x.z; w[3] = x.w;
        } else if constexpr (N == 8) {
            const v2u x = __builtin_amdgcn_raw_buffer_load_b64(r, (int)off, 0, 0);
            w[0] = x.x; w[1] = x.y;
        } else if constexpr (N == 4) {
            w[0] = __builtin_amdgcn_raw_buffer_load_b32(r, (int)off, 0, 0);
        } else {
            static_assert(N == 2, "slice size");
            w[0] = __builtin_amdgcn_raw_buffer_load_b16(r, (int)off, 0, 0);
        }
    }

    static __device__ __forceinline__ float word_f(__amdgpu_buffer_rsrc_t r, uint32_t off) {
        return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, (int)off, 0, 0));
    }

    // keys c0 + j0 .. c0 + j0 + 15 (j0 wave-uniform)
    __device__ __forceinline__ void load(T& t, int32_t j0) const {
        const __amdgpu_buffer_rsrc_t rk = rsrc(kb, j0, n, kstride, KVEC);
        const __amdgpu_buffer_rsrc_t rv = rsrc(vb, j0, n, kstride, KVEC);
        const __amdgpu_buffer_rsrc_t rks = rsrc(ksb, j0, n, sstride, 4);
        const __amdgpu_buffer_rsrc_t rvs = rsrc(vsb, j0, n, sstride, 4);
#pragma unroll
        for (int i = 0; i < KNI; ++i)
            words<KLB>(rk, ko + (uint32_t)(4 * i * KLB), t.k + i * KLB / 4);
#pragma unroll
        for (int r = 0; r < 4; ++r)
#pragma unroll
            for (int i = 0; i < VNI; ++i)
                words<VLB>(rv, vo[r] + (uint32_t)(16 * i * VLB), t.v[r] + i * VLB / 4);
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            t.ks[r] = word_f(rks, so[r]);
            t.vs[r] = word_f(rvs, so[r]);
        }
        if constexpr (KPOS) {
            const __amdgpu_buffer_rsrc_t rp = rsrc(kpb, j0, n, 4, 4);
#pragma unroll
            for (int r = 0; r < 4; ++r)
                t.kp[r] = (int32_t)__builtin_amdgcn_raw_buffer_load_b32(rp, (int)po[r], 0, 0);
        }
    }
};

// 2^e as a float, e in [-126, 127]
__device__ __forceinline__ float pow2i(int e) { return __builtin_bit_cast(float, (uint32_t)(e + 127) << 23); }

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;

// Per 32-key step:
//  * the scores are kept in log2 units (the softmax scale times log2(e)
//    folded into the query's scale) and exponentiated with the hardware's
//    exp2; m is returned in natural units for the merges;
//  * a step whose 32 keys are all inside the chunk and kept for every query
//    of the tile (no key positions, past the window's start, before the
//    tile's earliest query) skips the per-key masks (a wave-uniform branch);
//    a query column past the tile's last vector holds a real query's copy
//    (finite scores) and is never written out;
//  * the value sum accumulates in the matrix cores' accumulator in units of
//    2^(e - 6), and the probabilities are taken against a reference max m
//    that may sit up to 8 (log2 units) below the running max: p <= 2^8, so
//    p * value scale * 2^(6 - e) < 2^14 while e is at least the exponent of
//    the step's largest value scale. The reference max and e move (and the
//    sums are rescaled by 2^(m_old - m_new) * 2^(e_old - e_new)) only when
//    some query's max passes m + 8, a value scale passes 2^e, or the step's
//    largest value scale falls 2^8 below it (then e follows it as far as the
//    rescaled sums stay below 2^100): most steps of a long decode rescale
//    nothing;
//  * the tiles alternate between two register sets (the loop body twice),
//    so the next step's loads land without copies.
template <int DT, int D, bool MERGE_OUT, bool KPOS>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2))) void attn_f16_kernel(AttnParams p) {
    static_assert(DT == 1 || DT == 2, "integer caches");
    using Tile = KvTile<DT, D, D>;
    using Kv = IntKv<DT, D, KPOS>;
    using KT = typename Kv::T;
    constexpr int KS = Tile::KS, VS = Tile::VS, NS = KS / 8;
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int g = lane >> 4, c = lane & 15;
    const int chunk = blockIdx.x, kh = blockIdx.y;
    const int64_t n_vec = p.n_q * p.rep;
    const int64_t tile = (int64_t)(gridDim.z - 1 - blockIdx.z);
    constexpr int istep = 4;

    // this chunk's keys in 32-key steps
    const int64_t c0 = (int64_t)chunk * p.chunk_len;
    const int64_t c1 = min(c0 + p.chunk_len, p.n_kv);
    const int tiles_c = (int)((c1 - c0 + 31) / 32);
    const Kv kv(p, c0, c1, kh, g, c);
    KT ta, tb, na, nb;
    const int i_spec = min(wave, tiles_c - 1);
    const int64_t u = tile * 16 + c;
    const int64_t uc = u < n_vec ? u : n_vec - 1;
    const int64_t tq = uc / p.rep;
    const int64_t qrow = tq * p.n_head + (int64_t)kh * p.rep + uc % p.rep;
    float qs[KS];
    {
        const float* src = p.q + qrow * D;
#pragma unroll
        for (int e = 0; e < KS; e += 4) {
            const float4 f = *reinterpret_cast<const float4*>(src + Tile::kdim(g, e));
            qs[e] = f.x; qs[e + 1] = f.y; qs[e + 2] = f.z; qs[e + 3] = f.w;
        }
    }
    // the wave's first step is issued after the query (loads complete in
    // order: the split waits for q only) and before the query position
    // (which may narrow the range and is only used after the split)
    __builtin_amdgcn_sched_barrier(0);
    kv.load(ta, 32 * i_spec);
    kv.load(tb, 32 * i_spec + 16);
    // (a buffer load: a flat one would make every wait a full one)
    const __amdgpu_buffer_rsrc_t rqp = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<int32_t*>(p.qpos), 0, p.qpos ? 0x7fffffff : 0, kBufferDword3);
    const int32_t qp_raw = (int32_t)__builtin_amdgcn_raw_buffer_load_b32(rqp, (int)(tq * 4), 0, 0);
    __builtin_amdgcn_sched_barrier(0);
    float qmax = 0.0f;
#pragma unroll
    for (int e = 0; e < KS; ++e) qmax = fmaxf(qmax, fabsf(qs[e]));
    qmax = fmaxf(qmax, __shfl_xor(qmax, 16));
    qmax = fmaxf(qmax, __shfl_xor(qmax, 32));
    int eq = 0;
    if (qmax > 0.0f && qmax <= 3.4028235e38f) frexpf(qmax, &eq);
    const float qsc = ldexpf(1.0f, 14 - eq);
    const float qsl = ldexpf(p.scale * kLog2e, eq - 14);
    h8 qhi[NS], qlo[NS];
#pragma unroll
    for (int st = 0; st < NS; ++st)
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            _Float16 hi, lo;
            split2(qs[8 * st + key_order<DT>(i)] * qsc, hi, lo);
            qhi[st][i] = hi;
            qlo[st][i] = lo;
        }
    // (the split stays here, ahead of the wait for the query position and
    // the first step, rather than being sunk into the loop's preheader)
#pragma unroll
    for (int st = 0; st < NS; ++st) asm volatile("" : "+v"(qhi[st]), "+v"(qlo[st]));
    __builtin_amdgcn_sched_barrier(0);
    const int64_t qp = p.qpos ? (int64_t)qp_raw : tq;
    int64_t qmin = qp, qmx = qp;
#pragma unroll
    for (int off = 8; off >= 1; off >>= 1) {
        qmin = min(qmin, (int64_t)__shfl_xor(qmin, off, 16));
        qmx = max(qmx, (int64_t)__shfl_xor(qmx, off, 16));
    }
    // (every lane group holds the 16 columns' positions: wave-uniform)
    qmin = (int64_t)__builtin_amdgcn_readfirstlane((uint32_t)qmin) |
           ((int64_t)__builtin_amdgcn_readfirstlane((uint32_t)((uint64_t)qmin >> 32)) << 32);
    qmx = (int64_t)__builtin_amdgcn_readfirstlane((uint32_t)qmx) |
          ((int64_t)__builtin_amdgcn_readfirstlane((uint32_t)((uint64_t)qmx >> 32)) << 32);

    // 32-key steps [i_lo, i_hi) of the chunk can hold kept keys (as
    // attn_mfma_kernel's 16-key tiles)
    int64_t i_lo = 0, i_hi = tile * 16 < n_vec ? tiles_c : 0;
    if constexpr (!KPOS) {
        i_hi = min(i_hi, max<int64_t>(0, (qmx + 1 - c0 + 31) / 32));
        if (p.window > 0) i_lo = max<int64_t>(0, (qmin - p.window + 1 - c0) / 32);
    }
    int i = (int)(i_lo + (((wave - i_lo) % 4) + 4) % 4);
    if (i != i_spec && i < i_hi) {
        kv.load(ta, 32 * i);
        kv.load(tb, 32 * i + 16);
    }

    float m = -INFINITY, ls = 0.0f;   // reference max (log2 units), sum of p
    int e_acc = -1000;                 // the sums' exponent (none yet)
    v4f acc[VS];
#pragma unroll
    for (int t = 0; t < VS; ++t) acc[t] = v4f{0.f, 0.f, 0.f, 0.f};

    auto body = [&](const KT& A, const KT& B, int64_t kb) __attribute__((always_inline)) {
        // scores of keys kb + 16 h + 4g + r for query c, h = 0, 1
        v4f sa = {0.f, 0.f, 0.f, 0.f}, sb = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int st = 0; st < NS; ++st) {
            const h8 ka = key_codes<DT>(A.k, st), kbv = key_codes<DT>(B.k, st);
            sa = __builtin_amdgcn_mfma_f32_16x16x32_f16(ka, qlo[st], sa, 0, 0, 0);
            sb = __builtin_amdgcn_mfma_f32_16x16x32_f16(kbv, qlo[st], sb, 0, 0, 0);
            sa = __builtin_amdgcn_mfma_f32_16x16x32_f16(ka, qhi[st], sa, 0, 0, 0);
            sb = __builtin_amdgcn_mfma_f32_16x16x32_f16(kbv, qhi[st], sb, 0, 0, 0);
        }
        float sc[8];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            sc[r] = sa[r] * (qsl * A.ks[r]);
            sc[4 + r] = sb[r] * (qsl * B.ks[r]);
        }
        const bool full = !KPOS && kb + 32 <= c1 && kb + 31 <= qmin &&
                          (p.window <= 0 || qmx - kb < p.window);
        if (!full) {
#pragma unroll
            for (int h = 0; h < 2; ++h)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int64_t kj = kb + 16 * h + 4 * g + r;
                    const int64_t kp = KPOS ? (int64_t)(h ? B.kp[r] : A.kp[r]) : kj;
                    const bool keep = kj < c1 && key_kept(kp, qp, p.window);
                    sc[4 * h + r] = keep ? sc[4 * h + r] : -INFINITY;
                }
        }
        float tm = sc[0];
#pragma unroll
        for (int k = 1; k < 8; ++k) tm = fmaxf(tm, sc[k]);
        tm = fmaxf(tm, __shfl_xor(tm, 16));
        tm = fmaxf(tm, __shfl_xor(tm, 32));
        // the step's largest value scale (lane group g holds the scales of
        // keys 4g .. 4g + 3 of both halves)
        float vmax = fmaxf(fmaxf(fmaxf(A.vs[0], A.vs[1]), fmaxf(A.vs[2], A.vs[3])),
                           fmaxf(fmaxf(B.vs[0], B.vs[1]), fmaxf(B.vs[2], B.vs[3])));
        vmax = fmaxf(vmax, __shfl_xor(vmax, 16));
        vmax = fmaxf(vmax, __shfl_xor(vmax, 32));
        int ev = 0;
        if (vmax > 0.0f && vmax <= 3.4028235e38f) frexpf(vmax, &ev);
        ev = __builtin_amdgcn_readfirstlane(ev);
        int e_new = e_acc;
        if (ev > e_acc) {
            e_new = ev;
        } else if (ev < e_acc - 8) {
            // down to ev, as far as the sums (times 2^(e_acc - e_new)) stay
            // below 2^100 (the later steps add < 2^53 to them)
            float amax = 0.0f;
#pragma unroll
            for (int t = 0; t < VS; ++t)
#pragma unroll
                for (int r = 0; r < 4; ++r) amax = fmaxf(amax, fabsf(acc[t][r]));
#pragma unroll
            for (int off = 32; off >= 1; off >>= 1) amax = fmaxf(amax, __shfl_xor(amax, off));
            int ea = -1000;
            if (amax > 0.0f) frexpf(amax, &ea);
            ea = __builtin_amdgcn_readfirstlane(ea);
            e_new = max(ev, e_acc - (100 - ea));
        }
        e_new = min(max(e_new, -120), 128);   // 2^(6 - e) and 2^(e - 6) normal
        if (__any(tm > m + 8.0f) || e_new != e_acc) {
            const float mn = fmaxf(m, tm);
            // (before the first step's sums (e_acc -1000, wave-uniform) the
            // sums and l are zero: nothing to rescale)
            if (e_acc != -1000) {
                const float alpha = (m == -INFINITY) ? 0.0f : __builtin_amdgcn_exp2f(m - mn);
                ls = ls * alpha;
                // rescale the rows of query 4g + r by that query's alpha
                // (lane 4g + r), then all by 2^(e_acc - e_new)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const float ar = __shfl(alpha, 4 * g + r);
#pragma unroll
                    for (int t = 0; t < VS; ++t) acc[t][r] *= ar;
                }
                const int d = e_acc - e_new;
                if (d != 0) {
#pragma unroll
                    for (int t = 0; t < VS; ++t)
#pragma unroll
                        for (int r = 0; r < 4; ++r) acc[t][r] = ldexpf(acc[t][r], d);
                }
            }
            m = mn;
            e_acc = e_new;
        }
        const float msafe = (m == -INFINITY) ? 0.0f : m;   // p = 0 for a masked key
        const float psc = pow2i(6 - e_acc);
        h8 phi, plo;
        float psum = 0.0f;
#pragma unroll
        for (int h = 0; h < 2; ++h)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const float pr = __builtin_amdgcn_exp2f(sc[4 * h + r] - msafe);
                psum += pr;
                _Float16 hi, lo;
                split2(pr * (h ? B.vs[r] : A.vs[r]) * psc, hi, lo);
                phi[4 * h + r] = hi;
                plo[4 * h + r] = lo;
            }
        ls = ls + psum;
        // value sum: B = codes of element vdim(c, t) of the 8 keys' rows
#pragma unroll
        for (int t = 0; t < VS; ++t) {
            const h8 vbv = __builtin_bit_cast(
                h8, make_uint4(value_pair<DT>(A.v[0], A.v[1], t), value_pair<DT>(A.v[2], A.v[3], t),
                               value_pair<DT>(B.v[0], B.v[1], t), value_pair<DT>(B.v[2], B.v[3], t)));
            acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(plo, vbv, acc[t], 0, 0, 0);
            acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(phi, vbv, acc[t], 0, 0, 0);
        }
    };

    // steps i, i + 4, ...: ta/tb hold step i, na/nb receive the next (a
    // wave-uniform branch: the last step loads nothing)
    while (i < (int)i_hi) {
        if (i + istep < (int)i_hi) {
            kv.load(na, 32 * (i + istep));
            kv.load(nb, 32 * (i + istep) + 16);
        }
        body(ta, tb, c0 + 32 * (int64_t)i);
        i += istep;
        if (i >= (int)i_hi) break;
        if (i + istep < (int)i_hi) {
            kv.load(ta, 32 * (i + istep));
            kv.load(tb, 32 * (i + istep) + 16);
        }
        body(na, nb, c0 + 32 * (int64_t)i);
        i += istep;
    }
    // back to natural units: the sums times 2^(e - 6), m times ln 2
    const float back = e_acc < -120 ? 0.0f : pow2i(e_acc - 6);
#pragma unroll
    for (int t = 0; t < VS; ++t)
#pragma unroll
        for (int r = 0; r < 4; ++r) acc[t][r] *= back;
    m = m * kLn2;
    merge_tile<Tile, D, MERGE_OUT>(p, m, ls, acc, tile, n_vec, chunk, kh, wave, g, c);
}

// Merge the chunks' (m, l, acc) of one (token, head) row per workgroup. Thread
// (part q, element d) loads (m, l, acc[d]) of chunks q, q + P, ... all at once
// (clamped indices, no branch between the loads), merges them in registers,
// and the parts are merged through LDS: one memory round trip.
constexpr int kMaxChunks = 1024;
constexpr int kCombineBatch = 16;
__global__ __launch_bounds__(512) void attn_combine_kernel(AttnParams p) {
    __shared__ float sm[512], sl[512], sa[512];
    const int tid = threadIdx.x;
    const int64_t rows = p.n_q * p.n_head;
    const int64_t row = blockIdx.x;
    const int64_t DV = p.value_dim;
    const int nc = p.n_chunks;
    const int P = (int)max<int64_t>(1, 512 / DV);
    const float* ml = p.part + (int64_t)nc * rows * DV;
    float M = -INFINITY, L = 0.0f, A = 0.0f;
    if (tid < P * DV) {
        const int64_t d = tid % DV;
        const int q = tid / (int)DV;
        for (int c0 = q; c0 < nc; c0 += kCombineBatch * P) {
            float mc[kCombineBatch], lc[kCombineBatch], ac[kCombineBatch];
#pragma unroll
            for (int i = 0; i < kCombineBatch; ++i) {
                const int c = min(c0 + i * P, nc - 1);
                const int64_t pi = (int64_t)c * rows + row;
                mc[i] = ml[2 * pi];
                lc[i] = ml[2 * pi + 1];
                ac[i] = p.part[pi * DV + d];
            }
            float mb = M;
#pragma unroll
            for (int i = 0; i < kCombineBatch; ++i)
                if (c0 + i * P < nc) mb = fmaxf(mb, mc[i]);
            const float sc = (M == -INFINITY) ? 0.0f : expf(M - mb);
            L *= sc;
            A *= sc;
#pragma unroll
            for (int i = 0; i < kCombineBatch; ++i) {
                const bool ok = c0 + i * P < nc && mc[i] != -INFINITY;
                const float w = ok ? expf(mc[i] - mb) : 0.0f;
                L = __builtin_fmaf(lc[i], w, L);
                A = __builtin_fmaf(ac[i], w, A);
            }
            M = mb;
        }
    }
    sm[tid] = M;
    sl[tid] = L;
    sa[tid] = A;
    __syncthreads();
    for (int64_t d = tid; d < DV; d += 512) {
        float mt = -INFINITY;
        for (int q = 0; q < P; ++q) mt = fmaxf(mt, sm[q * DV + d]);
        float lt = 0.0f, at = 0.0f;
        for (int q = 0; q < P; ++q) {
            const float mq = sm[q * DV + d];
            const float w = (mq == -INFINITY) ? 0.0f : expf(mq - mt);
            lt = __builtin_fmaf(sl[q * DV + d], w, lt);
            at = __builtin_fmaf(sa[q * DV + d], w, at);
        }
        p.out[row * DV + d] = at / fmaxf(lt, 1e-30f);
    }
}

// The same merge for value widths that are a multiple of 4 (16-byte aligned
// partials and output): lane d4 of lane group grp (DV / 4 lanes a group,
// G = 512 / (DV / 4) groups) loads elements 4 d4 .. 4 d4 + 3 of chunks grp,
// grp + G, ... as one float4 each and the chunk's (m, l) as one float2, a
// batch of chunks at once: an eighth of the load instructions of
// attn_combine_kernel. Each group then scales its (l, acc) by its weight
// against the groups' max (one LDS pass), and DV / 4 threads add the
// groups' scaled sums.
constexpr int kCombineBatch4 = 8;
__global__ __launch_bounds__(512) void attn_combine4_kernel(AttnParams p) {
    __shared__ float sm[512], sl[512];
    __shared__ float4 sa[512];
    const int tid = threadIdx.x;
    const int64_t rows = p.n_q * p.n_head;
    const int64_t row = blockIdx.x;
    const int DV = (int)p.value_dim;
    const int lpr = DV / 4;
    const int G = 512 / lpr;
    const int nc = p.n_chunks;
    const float2* ml = reinterpret_cast<const float2*>(p.part + (int64_t)nc * rows * DV);
    const int d4 = tid % lpr, grp = tid / lpr;
    float M = -INFINITY, L = 0.0f;
    float4 A = make_float4(0.f, 0.f, 0.f, 0.f);
    if (grp < G) {
        for (int c0 = grp; c0 < nc; c0 += kCombineBatch4 * G) {
            float2 mc[kCombineBatch4];
            float4 ac[kCombineBatch4];
#pragma unroll
            for (int i = 0; i < kCombineBatch4; ++i) {
                const int c = min(c0 + i * G, nc - 1);
                const int64_t pi = (int64_t)c * rows + row;
                mc[i] = ml[pi];
                ac[i] = *reinterpret_cast<const float4*>(p.part + pi * DV + 4 * d4);
            }
            float mb = M;
#pragma unroll
            for (int i = 0; i < kCombineBatch4; ++i)
                if (c0 + i * G < nc) mb = fmaxf(mb, mc[i].x);
            const float sc = (M == -INFINITY) ? 0.0f : expf(M - mb);
            L *= sc;
            A.x *= sc; A.y *= sc; A.z *= sc; A.w *= sc;
#pragma unroll
            for (int i = 0; i < kCombineBatch4; ++i) {
                const bool ok = c0 + i * G < nc && mc[i].x != -INFINITY;
                const float w = ok ? expf(mc[i].x - mb) : 0.0f;
                L = __builtin_fmaf(mc[i].y, w, L);
                A.x = __builtin_fmaf(ac[i].x, w, A.x);
                A.y = __builtin_fmaf(ac[i].y, w, A.y);
                A.z = __builtin_fmaf(ac[i].z, w, A.z);
                A.w = __builtin_fmaf(ac[i].w, w, A.w);
            }
            M = mb;
        }
        if (d4 == 0) sm[grp] = M;
    }
    __syncthreads();
    if (grp < G) {
        float mt = -INFINITY;
        for (int k = 0; k < G; ++k) mt = fmaxf(mt, sm[k]);
        const float w = (M == -INFINITY) ? 0.0f : expf(M - mt);
        sa[tid] = make_float4(A.x * w, A.y * w, A.z * w, A.w * w);
        if (d4 == 0) sl[grp] = L * w;
    }
    __syncthreads();
    if (tid < lpr) {
        float lt = 0.0f;
        float4 at = make_float4(0.f, 0.f, 0.f, 0.f);
        for (int k = 0; k < G; ++k) {
            const float4 a = sa[k * lpr + tid];
            lt += sl[k];
            at.x += a.x; at.y += a.y; at.z += a.z; at.w += a.w;
        }
        const float r = 1.0f / fmaxf(lt, 1e-30f);
        *reinterpret_cast<float4*>(p.out + row * DV + 4 * tid) =
            make_float4(at.x * r, at.y * r, at.z * r, at.w * r);
    }
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

template <int DT, int D>
AttnKernel pick_mfma_d(bool merge_out) {
    return merge_out ? attn_mfma_kernel<DT, D, D, true> : attn_mfma_kernel<DT, D, D, false>;
}

template <int DT>
AttnKernel pick_mfma_dt(int D, bool merge_out) {
    switch (D) {
    case 64: return pick_mfma_d<DT, 64>(merge_out);
    case 128: return pick_mfma_d<DT, 128>(merge_out);
    case 256: return pick_mfma_d<DT, 256>(merge_out);
    default: return nullptr;
    }
}

AttnKernel pick_mfma(int dt, int D, bool merge_out) {
    switch (dt) {
    case 0: return pick_mfma_dt<0>(D, merge_out);
    case 1: return pick_mfma_dt<1>(D, merge_out);
    case 2: return pick_mfma_dt<2>(D, merge_out);
    default: return nullptr;
    }
}

template <int DT, int D>
AttnKernel pick_f16_d(bool merge_out, bool kpos) {
    if (kpos) return merge_out ? attn_f16_kernel<DT, D, true, true> : attn_f16_kernel<DT, D, false, true>;
    return merge_out ? attn_f16_kernel<DT, D, true, false> : attn_f16_kernel<DT, D, false, false>;
}

template <int DT>
AttnKernel pick_f16_dt(int D, bool merge_out, bool kpos) {
    if (D == 64) return pick_f16_d<DT, 64>(merge_out, kpos);
    if (D == 128) return pick_f16_d<DT, 128>(merge_out, kpos);
    return nullptr;
}

AttnKernel pick_f16(int dt, int D, bool merge_out, bool kpos) {
    return dt == 1 ? pick_f16_dt<1>(D, merge_out, kpos)
                   : (dt == 2 ? pick_f16_dt<2>(D, merge_out, kpos) : nullptr);
}

struct AttnPlan {
    bool mfma;
    bool f16;              // integer caches on the fp16 matrix cores (attn_f16_kernel)
    int E;                 // VALU kernel: elements per lane
    int64_t grid_z;        // query tiles (4 vectors: VALU kernel, 16: MFMA kernel)
    int64_t chunk_len;
    int n_chunks;
};

// The matrix-core kernel takes head_dim == value_dim in {64, 128} with
// 16-byte aligned operands; other shapes take the vector kernel.
bool attn_plan(int64_t n_q, int64_t n_head, int64_t n_head_kv, int64_t head_dim,
               int64_t value_dim, int64_t n_kv, bool aligned, int kv_dt, AttnPlan& pl) {
    const int64_t width = std::max(head_dim, value_dim);
    pl.E = width <= 64 ? 4 : (width <= 128 ? 8 : (width <= 256 ? 16 : 0));
    if (pl.E == 0) return false;
    const int64_t rep = n_head / n_head_kv;
    const int64_t n_vec = n_q * rep;
    // (head dim 256: one wave a SIMD, 320-481 registers by cache type)
    pl.mfma = aligned && head_dim == value_dim &&
              (head_dim == 64 || head_dim == 128 || head_dim == 256) &&
              tune("attn_mfma", 1) != 0;
    // integer caches at head dims 64 and 128: 32-key steps a wave on the fp16
    // matrix cores (at 256 the fp32 matrix-core kernel reads their codes)
    pl.f16 = pl.mfma && kv_dt != 0 && head_dim != 256 && tune("attn_f16", 1) != 0;
    int64_t step;  // keys a workgroup walks per step
    if (pl.mfma) {
        pl.grid_z = (n_vec + 15) / 16;
        step = pl.f16 ? 128 : 64;
    } else {
        pl.grid_z = (n_vec + kQV - 1) / kQV;
        step = kKeysPerStep;
    }
    // enough workgroups to fill the chip: split the keys when the query tiles
    // alone do not (decode), at least min_chunk keys a chunk
    const int64_t base = n_head_kv * pl.grid_z;
    const int64_t target = tune("attn_wgs", 512);
    const int64_t min_chunk = std::max<int64_t>(step, tune("attn_min_chunk", 64));
    int64_t nc = std::max<int64_t>(1, (target + base - 1) / base);
    nc = std::min<int64_t>(nc, std::max<int64_t>(1, (n_kv + min_chunk - 1) / min_chunk));
    nc = std::min<int64_t>(nc, kMaxChunks);
    int64_t cl = (n_kv + nc - 1) / nc;
    cl = (cl + step - 1) / step * step;
    pl.chunk_len = cl;
    pl.n_chunks = (int)((n_kv + cl - 1) / cl);
    // the fp16 kernel addresses a chunk of one kv head with 32-bit offsets
    const int64_t vec_bytes = head_dim * (kv_dt == 1 ? 8 : 4) / 8;
    if (pl.f16 && cl * n_head_kv * vec_bytes >= (int64_t(1) << 31)) pl.f16 = false;
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
    // the size for the vector kernel bounds the matrix-core kernel's
    if (n_q <= 0 || n_head <= 0 || n_head_kv <= 0 || n_head % n_head_kv || n_kv <= 0 ||
        !attn_plan(n_q, n_head, n_head_kv, head_dim, value_dim, n_kv, true, 0, pl))
        return 0;
    AttnPlan pv;   // (the fp16 plan's 128-key steps give no more chunks)
    attn_plan(n_q, n_head, n_head_kv, head_dim, value_dim, n_kv, false, 0, pv);
    if (pv.n_chunks > pl.n_chunks) pl = pv;
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
    const bool aligned = aligned16(q) && aligned16(k) && aligned16(v) && aligned16(out) &&
                         aligned16(workspace);
    if (!attn_plan(n_q, n_head, n_head_kv, head_dim, value_dim, n_kv, aligned, kv_dt, pl)) {
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
    if (pl.grid_z > 65535 || n_head_kv > 65535 || n_q * n_head > 0x7fffffff) {
        set_error("attention: grid too large");
        return false;
    }
    AttnParams p{q, k, k_scale, v, v_scale, out, static_cast<float*>(workspace), qpos, kpos,
                 n_q, n_head, n_head_kv, head_dim, value_dim, n_kv,
                 (int)(n_head / n_head_kv), window, scale, pl.chunk_len, pl.n_chunks};
    const bool one = pl.n_chunks == 1;
    AttnKernel kern = pl.f16 ? pick_f16(kv_dt, (int)head_dim, one, kpos != nullptr)
                      : pl.mfma ? pick_mfma(kv_dt, (int)head_dim, one)
                                : pick_attn(kv_dt, pl.E, one);
    if (!launch(pl.f16 ? "attn_f16_kernel" : (pl.mfma ? "attn_mfma_kernel" : "attn_kernel"), kern,
                dim3((unsigned)pl.n_chunks, (unsigned)n_head_kv, (unsigned)pl.grid_z),
                dim3(64 * kAttnWaves), 0, s, p))
        return false;
    // (value widths of a multiple of 4 up to 256 here: DV / 4 <= 512 lanes)
    const bool c4 = value_dim % 4 == 0 && aligned16(workspace) && aligned16(out) &&
                    tune("attn_combine4", 1) != 0;
    if (!one && !launch(c4 ? "attn_combine4_kernel" : "attn_combine_kernel",
                        c4 ? attn_combine4_kernel : attn_combine_kernel,
                        dim3((unsigned)(n_q * n_head)), dim3(512), 0, s, p))
        return false;
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
