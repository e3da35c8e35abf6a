// Internal helpers shared by the libaero_hip translation units: error state,
// launch wrapper with optional per-kernel device timing, wave-level
// reductions and exact fp16 decoding. gfx950 only (wave64).
#pragma once

#include <hip/hip_runtime.h>
#include <hip/hip_ext.h>

#include <cstdint>
#include <cstdio>
#include <functional>
#include <vector>

namespace aero {

// ---------------------------------------------------------------- errors
// Thread-local "why was this refused" string returned by aero_hip_last_error.
void set_error(const char* fmt, ...) __attribute__((format(printf, 1, 2)));
void clear_error();
bool hip_ok(hipError_t e, const char* what);

// ---------------------------------------------------------------- timing
// Per-thread arming set by aero_hip_time_next_kernel; consumed by launch().
struct TimingSlot {
    hipEvent_t start = nullptr;
    hipEvent_t stop = nullptr;
};
TimingSlot& timing_slot();

// ------------------------------------------------------------------ plans
// A plan is a recorded list of launches replayed by aero_hip_plan_launch.
// While a plan records on this thread, launch() appends a closure holding the
// kernel, its launch shape and its arguments by value instead of launching,
// so the host-side checks and kernel choice of every op run once, at record
// time, and a replay is a tight loop of hipLaunchKernel calls.
struct PlanEntry {
    const char* name;
    std::function<void(hipStream_t, hipEvent_t, hipEvent_t)> run;
};
struct Plan {
    std::vector<PlanEntry> entries;
};
Plan*& recording_plan();

// Launch `kernel` on `stream` (or record it into the plan this thread is
// recording). When per-kernel timing is armed the launch goes through
// hipExtLaunchKernelGGL so the events carry the kernel's own begin/end
// timestamps. Returns false (with the error set) on failure.
template <typename... KArgs, typename... Args>
bool launch(const char* name, void (*kernel)(KArgs...), dim3 grid, dim3 block,
            uint32_t shmem, hipStream_t stream, Args... args) {
    if (Plan* plan = recording_plan()) {
        plan->entries.push_back(
            {name, [=](hipStream_t s, hipEvent_t a, hipEvent_t b) {
                 if (a != nullptr)
                     hipExtLaunchKernelGGL(kernel, grid, block, shmem, s, a, b, 0,
                                           static_cast<KArgs>(args)...);
                 else
                     hipLaunchKernelGGL(kernel, grid, block, shmem, s,
                                        static_cast<KArgs>(args)...);
             }});
        return true;
    }
    TimingSlot& ts = timing_slot();
    if (ts.start != nullptr) {
        hipEvent_t a = ts.start, b = ts.stop;
        ts.start = ts.stop = nullptr;
        hipExtLaunchKernelGGL(kernel, grid, block, shmem, stream, a, b, 0,
                              static_cast<KArgs>(args)...);
    } else {
        hipLaunchKernelGGL(kernel, grid, block, shmem, stream,
                           static_cast<KArgs>(args)...);
    }
    return hip_ok(hipGetLastError(), name);
}

// Device-to-device copy that is recorded like a launch while a plan records.
bool async_copy(void* dst, const void* src, size_t bytes, hipStream_t stream);

// ------------------------------------------------------------------ tuning
// Launch-shape knobs (block sizes, lanes per row, rows per lane). Defaults
// are the measured best; AERO_HIP_TUNE="key=value,..." (read once per
// process) or tune_set overrides them for sweeps.
int tune(const char* key, int dflt);
// Set (or, with erase, drop) one knob for the rest of the process: lets a
// sweep change launch shapes without a new process. Thread-safe.
bool tune_set(const char* key, int value, bool erase);

// Compute units of the current device (256 on MI355X), cached per device.
int cu_count();

inline bool aligned16(const void* p) {
    return (reinterpret_cast<uintptr_t>(p) & 15u) == 0;
}

// RoPE folded into a projection's epilogue (the fused decode GEMV's,
// gemv.hip, or the split GEMM's, gemm16.hip): the outputs of matrices
// 0 .. mats-1 are heads of D rows, channels rotated at the token's position,
// angle (float)pos * inv[p]. The split GEMM also takes a per-head RMSNorm
// before the rotation (qk_w) and a partial rotation (n_rot < D); the GEMV
// fold takes neither.
struct RopeFold {
    int mats;             // 0: none
    int D;
    int mode;             // AERO_ROPE_NEOX / AERO_ROPE_INTERLEAVED
    const int32_t* pos;   // [n_tok]
    const float* inv;     // [n_rot / 2]
    int n_rot = 0;        // rotated channels (0: all D)
    const float* qk_w[2] = {nullptr, nullptr};  // per-head norm weights of matrices 0, 1 [D]
    float qk_eps = 0.f;
    int qk_flags = 0;     // 0 or AERO_NORM_UNIT_OFFSET
    bool qk_norm() const { return qk_w[0] != nullptr || qk_w[1] != nullptr; }
    int rot() const { return n_rot > 0 ? n_rot : D; }
};
bool rope_fold_ok(const RopeFold& rope, bool pair, int n_mat, const int64_t* n_rows);

// silu(v) = v / (1 + exp(-v)) with the hardware exp and reciprocal (about 1
// ulp each), where silu sits in a pass that is limited by its instructions
// (the conv's store, the split GEMM's x pre-pass, the gated GEMV prologue);
// -inf gives NaN, as the division form does.
__device__ __forceinline__ float silu_fast(float v) {
    return v * __builtin_amdgcn_rcpf(1.0f + __expf(-v));
}

// ------------------------------------------------- streaming loads/stores
// Data read once or written once (activations) moves with the nontemporal
// hint, so it streams through the caches without evicting what is reused
// (weights, tables, the cos/sin of a token). Measured on MI355X: +10-15%
// HBM throughput for the streaming kernels at 88-400 MB per launch.
typedef float v4f __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float4 ld_stream(const float* p) {
    const v4f v = __builtin_nontemporal_load(reinterpret_cast<const v4f*>(p));
    return make_float4(v.x, v.y, v.z, v.w);
}

// Output stores through a buffer descriptor: the hardware drops any store
// at or past `bytes` from the base, so a wrong offset cannot write outside
// the output. The descriptor is built from a base the caller guarantees is
// the same for every lane of the wave (it is read from lane 0); offsets are
// 32-bit bytes from that base. The cache policy is NT (streaming), which on
// MI355X measured equal to nontemporal global stores and faster than
// device-scope SC1 stores for the gathers (1.7x at 16384 rows).
typedef unsigned int v4u __attribute__((ext_vector_type(4)));
constexpr int kBufferDword3 = 0x00020000;  // raw buffer, 32-bit data format (gfx9)
constexpr int kStorePolicy = 2;  // cache-policy operand (gfx950: 1 SC0, 2 NT, 16 SC1)

struct StreamOut {
    __amdgpu_buffer_rsrc_t rsrc;
    __device__ __forceinline__ StreamOut(float* wave_uniform_base, int64_t bytes) {
        const uint64_t a = reinterpret_cast<uint64_t>(wave_uniform_base);
        const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)a);
        const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(a >> 32));
        const int64_t cl = bytes < 0 ? 0 : (bytes > 0xFFFFFFFFll ? 0xFFFFFFFFll : bytes);
        const uint32_t n = __builtin_amdgcn_readfirstlane((uint32_t)cl);
        rsrc = __builtin_amdgcn_make_buffer_rsrc(
            reinterpret_cast<void*>(((uint64_t)hi << 32) | lo), 0, (int)n, kBufferDword3);
    }
    __device__ __forceinline__ void store(uint32_t byte_off, float4 v) const {
        const v4u d = {__builtin_bit_cast(uint32_t, v.x), __builtin_bit_cast(uint32_t, v.y),
                       __builtin_bit_cast(uint32_t, v.z), __builtin_bit_cast(uint32_t, v.w)};
        __builtin_amdgcn_raw_buffer_store_b128(d, rsrc, (int)byte_off, 0, kStorePolicy);
    }
    __device__ __forceinline__ void store1(uint32_t byte_off, float v) const {
        __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, v), rsrc, (int)byte_off,
                                              0, kStorePolicy);
    }
};

// ------------------------------------------------------- device helpers
// Sum across aligned groups of W lanes (W a power of two, W <= 64) with an
// xor butterfly. Every lane of a group ends with the identical bit pattern
// (fp add is commutative), so every lane derives the same scale factor.
template <int W>
__device__ __forceinline__ float group_sum(float v) {
#pragma unroll
    for (int off = W / 2; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
    return v;
}

// Exact IEEE half -> single from the raw 16 bits, subnormals included
// (v_cvt_f32_f16 would also be exact; the integer form keeps the result
// independent of the wave's fp16 denormal mode).
__host__ __device__ __forceinline__ float half_bits_to_float(uint32_t h) {
    const uint32_t sign = (h & 0x8000u) << 16;
    const uint32_t e = (h >> 10) & 31u;
    uint32_t m = h & 1023u;
    uint32_t bits;
    if (e == 31u) {
        bits = sign | 0x7F800000u | (m << 13);
    } else if (e != 0u) {
        bits = sign | ((e + 112u) << 23) | (m << 13);
    } else if (m == 0u) {
        bits = sign;
    } else {
        // subnormal: m * 2^-24 with m < 1024; normalise so bit 10 is set
#if defined(__HIP_DEVICE_COMPILE__)
        const int lz = __clz(m) - 21;  // leading zeros within 11 bits
#else
        const int lz = __builtin_clz(m) - 21;
#endif
        m <<= lz;
        bits = sign | ((uint32_t)(113 - lz) << 23) | ((m & 1023u) << 13);
    }
    return __builtin_bit_cast(float, bits);
}

}  // namespace aero
