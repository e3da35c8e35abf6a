// Reference-compatible host-pointer ABI of libaero_hip.so.
//
// Each entry point keeps the name, signature and status convention of the
// reference symbol it replaces (src/tensor.cpp:205-304, src/transformer.cpp:
// 223-284, src/kernels.cpp:560-603): buffers are host memory and the call is
// synchronous. Inputs are staged into a per-device HBM arena (grown on
// demand, reused across calls, freed at exit), the same device kernels as
// the aero_hip_* entry points run on a library-owned stream, and the result
// is copied back before returning. Calls from several threads serialise on
// the arena lock.
//
// Host buffers are pageable (numpy arrays), and a DMA from pageable memory
// goes through the driver's own single-threaded staging (6-7 GB/s measured).
// Large transfers instead move in 4 MiB chunks through two pinned buffers
// per device: a pool of host threads copies chunk i between the caller's
// memory and one pinned buffer while the DMA engine moves chunk i-1 from or
// to the other, each buffer guarded by an event of its last DMA. Bad arguments are refused before any device work. The
// `void` entry points clear the error string on entry; after a refusal or a
// HIP error they return with aero_hip_last_error() saying why, so a caller
// detects failure by a non-empty error string.
#include "common.hpp"
#include "aero_hip.h"

#include <algorithm>
#include <condition_variable>
#include <cstring>
#include <functional>
#include <mutex>
#include <new>
#include <thread>
#include <vector>

namespace aero {

bool norm_rows(const float* x, const float* w, float* out, int64_t rows, int64_t cols,
               float eps, int flags, hipStream_t stream);
bool act_mul(int kind, const float* g, const float* u, float* out, int64_t n,
             hipStream_t s);
int64_t rope_inv_freq_host(int64_t head_dim, int64_t n_dims, float base,
                           const float* ff, int64_t n_ff, float* inv_out);
bool rope_tables_dev(const int32_t* pos, int64_t n_pos, const float* inv, int64_t half,
                     float* c, float* s, hipStream_t stream);
bool dequant_dev(int dtype, const uint8_t* raw, int64_t raw_len, float* out,
                 int64_t n_values, hipStream_t s);
int64_t dtype_block_bytes(int t);
int64_t dtype_block_values(int t);
bool gemv_dev(int dtype, const uint8_t* w, int64_t w_bytes, const float* x, float* y,
              int64_t n_rows, int64_t n_cols, int64_t n_tok, hipStream_t s, void* ws,
              int64_t ws_bytes);
int64_t split_gemm_workspace(int dtype, int64_t n_cols, int64_t n_tok);
bool attention_dev(const float* q, int kv_dt, const void* k, const float* k_scale, const void* v,
                   const float* v_scale, float* out, int64_t n_q, int64_t n_head,
                   int64_t n_head_kv, int64_t head_dim, int64_t value_dim, float scale,
                   const int32_t* qpos, const int32_t* kpos, int64_t n_kv, int window,
                   void* workspace, int64_t ws_bytes, hipStream_t s);
int64_t attn_workspace_bytes(int64_t n_q, int64_t n_head, int64_t n_head_kv, int64_t head_dim,
                             int64_t value_dim, int64_t n_kv);
bool kv_write_dev(int dt, const float* x, int64_t n_tok, int64_t heads, int64_t dim,
                  int64_t phys0, int64_t cap, void* q, float* scale, hipStream_t s);
bool softmax_rows_dev(const float* x, float* y, int64_t n_rows, int64_t n_cols, hipStream_t s);
int64_t ssm_workspace_bytes(int64_t T, int64_t n_k, int64_t n_v, int64_t d);
bool ssm_scan_dev(const float* q, const float* k, const float* v, const float* alpha,
                  const float* beta, const float* a_log, const float* dt_bias, float* state,
                  int64_t T, int64_t n_k, int64_t n_v, int64_t d, float scale, float eps,
                  float* outs, void* workspace, int64_t ws_bytes, hipStream_t s);
bool ssm_conv_dev(const float* x, const float* w, const float* tail, int64_t tail_len,
                  float* tail_out, float* out, int64_t T, int64_t C, int64_t K,
                  int64_t* new_tail_len, hipStream_t s);
bool dense_matmul_dev(const float* w, const float* x, float* y, int64_t n_rows, int64_t n_cols,
                      int64_t n_tok, hipStream_t s);
bool argmax_dev(const float* v, int64_t n, int32_t* out, hipStream_t s);
bool kv_read_dev(int dt, const void* q, const float* scale, int64_t n_vec, int64_t dim,
                 float* out, hipStream_t s);
bool kv_span_error_dev(int dt, const void* q, const float* scale, int64_t dim, const float* x,
                       float* out, hipStream_t s);

// A KV slot (src/kv.cpp:92-133, include/aero/kv.hpp:35-60) resident in HBM:
// codes [cap, heads, dim] (fp32, int8, or int4 two a byte) and one fp32
// scale a (position, head) for int8/int4, zeroed at creation, on the device
// that was current then. aero_hip_kv_slot_view hands the device pointers to
// the attention entry point.
struct KvSlotDev {
    int64_t cap, heads, dim;
    int dt;
    int ring;
    int device;
    void* q;
    float* scale;
    int64_t vec_bytes() const { return dt == 2 ? dim / 2 : (dt == 1 ? dim : dim * 4); }
    int64_t bytes() const { return cap * heads * vec_bytes() + (dt != 0 ? cap * heads * 4 : 0); }
};

namespace {

// ------------------------------------------------------ host copy pool
// A fixed pool of host threads for large memcpys between pageable and
// pinned memory: copy(dst, src, n) splits n into one part a worker (plus the
// caller) and returns when every part is done. Workers start on first use
// and are joined at exit.
class CopyPool {
public:
    static CopyPool& get() {
        static CopyPool pool;
        return pool;
    }
    void copy(void* dst, const void* src, size_t n) {
        std::lock_guard<std::mutex> call(call_mu_);   // one copy at a time
        const int parts = (int)std::min<size_t>(workers_.size() + 1, std::max<size_t>(1, n >> 19));
        if (parts <= 1) {
            std::memcpy(dst, src, n);
            return;
        }
        const size_t per = ((n + parts - 1) / parts + 63) & ~size_t(63);
        char* d = static_cast<char*>(dst);
        const char* sp = static_cast<const char*>(src);
        {
            std::lock_guard<std::mutex> lk(mu_);
            pending_ = 0;
            for (int i = 1; i < parts; ++i) {
                const size_t o = (size_t)i * per;
                if (o >= n) break;
                jobs_.push_back({d + o, sp + o, std::min(per, n - o)});
                ++pending_;
            }
        }
        cv_.notify_all();
        std::memcpy(d, sp, std::min(per, n));
        std::unique_lock<std::mutex> lk(mu_);
        done_.wait(lk, [&] { return pending_ == 0; });
    }
    ~CopyPool() {
        {
            std::lock_guard<std::mutex> lk(mu_);
            stop_ = true;
        }
        cv_.notify_all();
        for (auto& t : workers_) t.join();
    }

private:
    struct Job {
        char* d;
        const char* s;
        size_t n;
    };
    CopyPool() {
        const unsigned hc = std::thread::hardware_concurrency();
        const int n = (int)std::min(hc == 0 ? 1u : hc, 8u) - 1;
        for (int i = 0; i < n; ++i) workers_.emplace_back([this] { run(); });
    }
    void run() {
        for (;;) {
            Job j;
            {
                std::unique_lock<std::mutex> lk(mu_);
                cv_.wait(lk, [&] { return stop_ || !jobs_.empty(); });
                if (stop_ && jobs_.empty()) return;
                j = jobs_.back();
                jobs_.pop_back();
            }
            std::memcpy(j.d, j.s, j.n);
            std::lock_guard<std::mutex> lk(mu_);
            if (--pending_ == 0) done_.notify_all();
        }
    }
    std::vector<std::thread> workers_;
    std::vector<Job> jobs_;
    std::mutex call_mu_;
    std::mutex mu_;
    std::condition_variable cv_, done_;
    int pending_ = 0;
    bool stop_ = false;
};

constexpr size_t kChunk = 4u << 20;      // bytes a pinned transfer chunk
constexpr size_t kDirect = 1u << 20;     // below this, plain async copies

struct Arena {
    std::mutex mu;
    void* buf = nullptr;
    size_t cap = 0;
    hipStream_t stream = nullptr;
    void* pinned[2] = {nullptr, nullptr};    // kChunk bytes each
    hipEvent_t done[2] = {nullptr, nullptr}; // the last DMA of each buffer
    bool busy[2] = {false, false};           // an event is recorded on it
};

constexpr int kMaxDevices = 64;
Arena g_arena[kMaxDevices];

// Holds the current device's arena for the duration of one host call and
// carves 256-byte aligned sub-buffers out of it.
class Staging {
public:
    Staging() {
        // A host-pointer call runs and copies back at once; under plan
        // recording its kernels would be recorded instead of run, the call
        // would copy back the unmodified input, and the plan would hold
        // pointers into this arena, which a later larger call reallocates.
        if (recording_plan() != nullptr) {
            set_error("host-pointer entry points cannot be recorded into a plan; "
                      "use the aero_hip_* device-pointer ops inside a plan");
            return;
        }
        int dev = 0;
        ok_ = hip_ok(hipGetDevice(&dev), "hipGetDevice");
        if (ok_ && (dev < 0 || dev >= kMaxDevices)) {
            set_error("device index %d out of range", dev);
            ok_ = false;
        }
        a_ = &g_arena[ok_ ? dev : 0];
        lock_ = std::unique_lock<std::mutex>(a_->mu);
        if (ok_ && a_->stream == nullptr)
            ok_ = hip_ok(hipStreamCreate(&a_->stream), "hipStreamCreate");
    }
    bool ok() const { return ok_; }
    hipStream_t stream() const { return a_ ? a_->stream : nullptr; }

    // Reserve sizes[i] bytes for each i; pointers land in out[i].
    bool reserve(std::initializer_list<size_t> sizes, void** out) {
        if (!ok_) return false;
        size_t total = 0;
        for (size_t s : sizes) total += (s + 255) & ~size_t(255);
        if (total == 0) total = 256;
        if (total > a_->cap) {
            if (a_->buf != nullptr) {
                (void)hipStreamSynchronize(a_->stream);
                (void)hipFree(a_->buf);
                a_->buf = nullptr;
                a_->cap = 0;
            }
            if (!hip_ok(hipMalloc(&a_->buf, total), "hipMalloc(staging)")) return false;
            a_->cap = total;
        }
        char* p = static_cast<char*>(a_->buf);
        int i = 0;
        for (size_t s : sizes) {
            out[i++] = p;
            p += (s + 255) & ~size_t(255);
        }
        return true;
    }

    // host -> device: returns once every chunk is in a pinned buffer and its
    // DMA queued on the stream
    bool h2d(void* d, const void* h, size_t n) {
        if (!ok_) return false;
        if (n < kDirect || !pinned())
            return n == 0 || hip_ok(hipMemcpyAsync(d, h, n, hipMemcpyHostToDevice, a_->stream),
                                    "hipMemcpyAsync H2D");
        for (size_t o = 0, i = 0; o < n; o += kChunk, ++i) {
            const int b = (int)(i & 1);
            const size_t len = std::min(kChunk, n - o);
            if (!wait(b)) return false;
            CopyPool::get().copy(a_->pinned[b], static_cast<const char*>(h) + o, len);
            if (!hip_ok(hipMemcpyAsync(static_cast<char*>(d) + o, a_->pinned[b], len,
                                       hipMemcpyHostToDevice, a_->stream), "hipMemcpyAsync H2D") ||
                !record(b))
                return false;
        }
        return true;
    }
    // device -> host, after the work queued before it: returns with the data
    // in host memory
    bool d2h(void* h, const void* d, size_t n) {
        if (!ok_) return false;
        if (n < kDirect || !pinned())
            return n == 0 || hip_ok(hipMemcpyAsync(h, d, n, hipMemcpyDeviceToHost, a_->stream),
                                    "hipMemcpyAsync D2H");
        const size_t nc = (n + kChunk - 1) / kChunk;
        auto issue = [&](size_t i) {
            const int b = (int)(i & 1);
            const size_t o = i * kChunk, len = std::min(kChunk, n - o);
            return wait(b) &&
                   hip_ok(hipMemcpyAsync(a_->pinned[b], static_cast<const char*>(d) + o, len,
                                         hipMemcpyDeviceToHost, a_->stream),
                          "hipMemcpyAsync D2H") &&
                   record(b);
        };
        if (!issue(0)) return false;
        for (size_t i = 0; i < nc; ++i) {
            const int b = (int)(i & 1);
            // the next chunk's DMA runs while this one is copied out
            if (i + 1 < nc) {
                // the other buffer's last DMA must land before it is reused:
                // its contents (chunk i-1) were copied out in the previous turn
                if (!issue(i + 1)) return false;
            }
            if (!wait(b)) return false;
            const size_t o = i * kChunk, len = std::min(kChunk, n - o);
            CopyPool::get().copy(static_cast<char*>(h) + o, a_->pinned[b], len);
        }
        return true;
    }
    bool finish() { return ok_ && hip_ok(hipStreamSynchronize(a_->stream), "hipStreamSynchronize"); }

private:
    // the two pinned chunk buffers and their events, made on first use
    bool pinned() {
        if (a_->pinned[0] != nullptr) return true;
        for (int b = 0; b < 2; ++b) {
            if (!hip_ok(hipHostMalloc(&a_->pinned[b], kChunk, hipHostMallocDefault),
                        "hipHostMalloc(staging)") ||
                !hip_ok(hipEventCreateWithFlags(&a_->done[b], hipEventDisableTiming),
                        "hipEventCreate")) {
                for (int c = 0; c < 2; ++c) {
                    if (a_->pinned[c] != nullptr) (void)hipHostFree(a_->pinned[c]);
                    if (a_->done[c] != nullptr) (void)hipEventDestroy(a_->done[c]);
                    a_->pinned[c] = nullptr;
                    a_->done[c] = nullptr;
                }
                clear_error();   // fall back to the driver's pageable copies
                return false;
            }
        }
        return true;
    }
    bool wait(int b) {
        if (!a_->busy[b]) return true;
        a_->busy[b] = false;
        return hip_ok(hipEventSynchronize(a_->done[b]), "hipEventSynchronize");
    }
    bool record(int b) {
        a_->busy[b] = true;
        return hip_ok(hipEventRecord(a_->done[b], a_->stream), "hipEventRecord");
    }

    Arena* a_ = nullptr;
    std::unique_lock<std::mutex> lock_;
    bool ok_ = false;
};

// out = f(in) for an n-float buffer (optionally with a second input).
bool host_act(int kind, float* g, const float* u, int64_t n) {
    Staging st;
    void* p[2];
    const size_t bytes = (size_t)n * sizeof(float);
    if (!st.reserve({bytes, u ? bytes : 0}, p)) return false;
    float* dg = static_cast<float*>(p[0]);
    float* du = u ? static_cast<float*>(p[1]) : nullptr;
    return st.h2d(dg, g, bytes) && (!u || st.h2d(du, u, bytes)) &&
           act_mul(kind, dg, du, dg, n, st.stream()) && st.d2h(g, dg, bytes) && st.finish();
}

// Y = X W^T for host W [n_rows, n_cols] and X [n_tok, n_cols] (fp32).
bool host_dense(const float* w, const float* x, float* y, int64_t n_tok, int64_t n_rows,
                int64_t n_cols) {
    Staging st;
    void* p[3];
    const size_t wb = (size_t)(n_rows * n_cols) * 4, xb = (size_t)(n_tok * n_cols) * 4,
                 yb = (size_t)(n_tok * n_rows) * 4;
    if (!st.reserve({wb, xb, yb}, p)) return false;
    float* dw = static_cast<float*>(p[0]);
    float* dx = static_cast<float*>(p[1]);
    float* dy = static_cast<float*>(p[2]);
    return st.h2d(dw, w, wb) && st.h2d(dx, x, xb) &&
           dense_matmul_dev(dw, dx, dy, n_rows, n_cols, n_tok, st.stream()) &&
           st.d2h(y, dy, yb) && st.finish();
}

bool host_norm(const float* x, const float* w, float* out, int64_t rows, int64_t cols,
               float eps, int flags) {
    Staging st;
    void* p[2];
    const size_t bytes = (size_t)(rows * cols) * sizeof(float);
    const size_t wbytes = w ? (size_t)cols * sizeof(float) : 0;
    if (!st.reserve({bytes, wbytes}, p)) return false;
    float* dx = static_cast<float*>(p[0]);
    float* dw = w ? static_cast<float*>(p[1]) : nullptr;
    return st.h2d(dx, x, bytes) && (!w || st.h2d(dw, w, wbytes)) &&
           norm_rows(dx, dw, dx, rows, cols, eps, flags, st.stream()) &&
           st.d2h(out, dx, bytes) && st.finish();
}

}  // namespace

bool qk_norm_rope_public(float* q, float* q_out, int64_t hq, float* k, float* k_out,
                         int64_t hk, const float* qw, const float* kw, float eps,
                         int flags, int64_t n_tok, int64_t D, int64_t n_rot, int mode,
                         const int32_t* pos, const float* inv, const float* ct,
                         const float* stb, int64_t n_tab, hipStream_t s) {
    return aero_hip_qk_norm_rope(q, q_out, hq, k, k_out, hk, qw, kw, eps, flags, n_tok, D,
                                 n_rot, mode, pos, inv, ct, stb, n_tab, s) == 1;
}

}  // namespace aero

using aero::set_error;

extern "C" {

// ------------------------------------------------------ src/tensor.cpp ABI
int aero_tensor_silu(float* v, int64_t n) {
    if (!v || n <= 0) { set_error("aero_tensor_silu: null or n <= 0"); return 0; }
    return aero::host_act(AERO_ACT_SILU, v, nullptr, n) ? 1 : 0;
}

int aero_tensor_gelu(float* v, int64_t n) {
    if (!v || n <= 0) { set_error("aero_tensor_gelu: null or n <= 0"); return 0; }
    return aero::host_act(AERO_ACT_GELU, v, nullptr, n) ? 1 : 0;
}

int aero_tensor_mul(float* a, const float* b, int64_t n) {
    if (!a || !b || n <= 0) { set_error("aero_tensor_mul: null or n <= 0"); return 0; }
    return aero::host_act(AERO_ACT_IDENTITY, a, b, n) ? 1 : 0;
}

int aero_tensor_swiglu(float* gate, const float* up, int64_t n) {
    if (!gate || !up || n <= 0) { set_error("aero_tensor_swiglu: null or n <= 0"); return 0; }
    return aero::host_act(AERO_ACT_SILU, gate, up, n) ? 1 : 0;
}

int aero_tensor_rmsnorm(const float* x, const float* weight, float* out, int64_t n,
                        float eps) {
    if (!x || !weight || !out || n <= 0) {
        set_error("aero_tensor_rmsnorm: null or n <= 0");
        return 0;
    }
    return aero::host_norm(x, weight, out, 1, n, eps, 0) ? 1 : 0;
}

int aero_tensor_l2norm(const float* x, const float* weight, float* out, int64_t n,
                       float eps, int weighted) {
    if (!x || !out || n <= 0 || (weighted && !weight)) {
        set_error("aero_tensor_l2norm: null, n <= 0 or weighted without weight");
        return 0;
    }
    return aero::host_norm(x, weighted ? weight : nullptr, out, 1, n, eps, AERO_NORM_L2)
               ? 1 : 0;
}

int aero_tensor_rmsnorm_rows(float* t, int64_t rows, int64_t cols, float eps) {
    if (!t || rows <= 0 || cols <= 0) {
        set_error("aero_tensor_rmsnorm_rows: null or non-positive dims");
        return 0;
    }
    return aero::host_norm(t, nullptr, t, rows, cols, eps, 0) ? 1 : 0;
}

// src/tensor.cpp:207 aero_tensor_threads: the thread count the reference's
// native layer would pick (hardware threads, at most 8). The GPU entry
// points below take and ignore a `threads` argument.
int aero_tensor_threads(void) {
    const unsigned hc = std::thread::hardware_concurrency();
    return (int)std::min(hc == 0 ? 1u : hc, 8u);
}

// src/tensor.cpp:209-218 aero_tensor_matvec: y[r] = dot(W.row(r), x), fp32,
// summed in the reference's order (bit-identical for any `threads`).
int aero_tensor_matvec(const float* w, const float* x, float* y, int64_t n_rows, int64_t n_cols,
                       int threads) {
    (void)threads;
    aero::clear_error();
    if (!w || !x || !y || n_rows <= 0 || n_cols <= 0) {
        set_error("aero_tensor_matvec: null or non-positive dims");
        return 0;
    }
    return aero::host_dense(w, x, y, 1, n_rows, n_cols) ? 1 : 0;
}

// src/tensor.cpp:220-231 aero_tensor_matmul: Y[t][r] = dot(W.row(r),
// X.row(t)); one token is the matvec.
int aero_tensor_matmul(const float* w, const float* X, float* Y, int64_t n_tokens,
                       int64_t n_rows, int64_t n_cols, int threads) {
    (void)threads;
    aero::clear_error();
    if (!w || !X || !Y || n_tokens <= 0 || n_rows <= 0 || n_cols <= 0) {
        set_error("aero_tensor_matmul: null or non-positive dims");
        return 0;
    }
    return aero::host_dense(w, X, Y, n_tokens, n_rows, n_cols) ? 1 : 0;
}

// src/tensor.cpp:298-302 aero_tensor_argmax: index of the first largest
// value (NaN never chosen; 0 when v[0] is NaN); -1 when refused.
int aero_tensor_argmax(const float* v, int64_t n) {
    aero::clear_error();
    if (!v || n <= 0) {
        set_error("aero_tensor_argmax: null or n <= 0");
        return -1;
    }
    aero::Staging st;
    void* p[2];
    const size_t vb = (size_t)n * 4;
    int32_t best = -1;
    if (!st.reserve({vb, 4}, p) || !st.h2d(p[0], v, vb) ||
        !aero::argmax_dev(static_cast<const float*>(p[0]), n, static_cast<int32_t*>(p[1]),
                          st.stream()) ||
        !st.d2h(&best, p[1], 4) || !st.finish())
        return -1;
    return best;
}

// ------------------------------------------------- src/transformer.cpp ABI
int64_t aero_rope_tables(int64_t head_dim, const int32_t* positions, int64_t n_pos,
                         float base, int64_t n_dims, const float* freq_factors,
                         int64_t n_ff, float* cos_out, float* sin_out) {
    if (head_dim <= 0 || n_pos < 0 || positions == nullptr) {
        set_error("aero_rope_tables: head_dim <= 0, n_pos < 0 or null positions");
        return -1;
    }
    std::vector<float> inv((size_t)head_dim / 2 + 1);
    const int64_t n = aero::rope_inv_freq_host(head_dim, n_dims, base, freq_factors, n_ff,
                                               inv.data());
    if (n < 0) {
        set_error("aero_rope_tables: freq_factors shorter than n_rot/2");
        return -1;
    }
    const int64_t half = n / 2;
    if (half <= 0 || n_pos == 0) return n;
    if (cos_out == nullptr || sin_out == nullptr) {
        set_error("aero_rope_tables: null output");
        return -1;
    }
    aero::Staging st;
    void* p[4];
    const size_t tb = (size_t)(n_pos * half) * sizeof(float);
    if (!st.reserve({(size_t)n_pos * 4, (size_t)half * 4, tb, tb}, p)) return -1;
    const bool ok = st.h2d(p[0], positions, (size_t)n_pos * 4) &&
                    st.h2d(p[1], inv.data(), (size_t)half * 4) &&
                    aero::rope_tables_dev(static_cast<int32_t*>(p[0]), n_pos,
                                          static_cast<float*>(p[1]), half,
                                          static_cast<float*>(p[2]),
                                          static_cast<float*>(p[3]), st.stream()) &&
                    st.d2h(cos_out, p[2], tb) && st.d2h(sin_out, p[3], tb) && st.finish();
    return ok ? n : -1;
}

void aero_apply_rope(float* x, int64_t n_rows, int64_t head_dim, int64_t n_rot,
                     const float* cos_tab, const float* sin_tab, const int32_t* positions,
                     int mode) {
    aero::clear_error();
    const int64_t half = n_rot / 2;
    if (half <= 0 || head_dim <= 0 || n_rows <= 0) return;
    if (!x || !cos_tab || !sin_tab || n_rot > head_dim) {
        set_error("aero_apply_rope: null buffer or n_rot > head_dim");
        return;
    }
    // The table must cover every position read (POSITION-indexed).
    int64_t n_tab = n_rows;
    if (positions != nullptr) {
        int64_t mx = -1;
        for (int64_t r = 0; r < n_rows; ++r) {
            if (positions[r] < 0) {
                set_error("aero_apply_rope: negative position %d at row %lld",
                          positions[r], (long long)r);
                return;
            }
            mx = std::max<int64_t>(mx, positions[r]);
        }
        n_tab = mx + 1;
    }
    aero::Staging st;
    void* p[4];
    const size_t xb = (size_t)(n_rows * head_dim) * 4;
    const size_t tb = (size_t)(n_tab * half) * 4;
    if (!st.reserve({xb, tb, tb, positions ? (size_t)n_rows * 4 : 0}, p)) return;
    float* dx = static_cast<float*>(p[0]);
    int32_t* dpos = positions ? static_cast<int32_t*>(p[3]) : nullptr;
    const int m = mode == 0 ? AERO_ROPE_NEOX : AERO_ROPE_INTERLEAVED;
    (void)(st.h2d(dx, x, xb) && st.h2d(p[1], cos_tab, tb) && st.h2d(p[2], sin_tab, tb) &&
           (!positions || st.h2d(dpos, positions, (size_t)n_rows * 4)) &&
           aero::qk_norm_rope_public(dx, nullptr, 1, nullptr, nullptr, 0, nullptr, nullptr,
                                     0.0f, 0, n_rows, head_dim, 2 * half, m, dpos, nullptr,
                                     static_cast<float*>(p[1]), static_cast<float*>(p[2]),
                                     n_tab, st.stream()) &&
           st.d2h(x, dx, xb) && st.finish());
}

void aero_rmsnorm_rows(const float* x, const float* weight, float* out, int64_t n_rows,
                       int64_t n_cols, float eps) {
    aero::clear_error();
    if (!x || !out || n_rows <= 0 || n_cols <= 0) {
        set_error("aero_rmsnorm_rows: null or non-positive dims");
        return;
    }
    (void)aero::host_norm(x, weight, out, n_rows, n_cols, eps, 0);
}

void aero_l2norm_rows(const float* x, const float* weight, float* out, int64_t n_rows,
                      int64_t n_cols, float eps) {
    aero::clear_error();
    if (!x || !out || n_rows <= 0 || n_cols <= 0) {
        set_error("aero_l2norm_rows: null or non-positive dims");
        return;
    }
    (void)aero::host_norm(x, weight, out, n_rows, n_cols, eps, AERO_NORM_L2);
}

void aero_gelu(float* v, int64_t n) {
    aero::clear_error();
    if (!v || n <= 0) return;
    (void)aero::host_act(AERO_ACT_GELU, v, nullptr, n);
}

void aero_silu(float* v, int64_t n) {
    aero::clear_error();
    if (!v || n <= 0) return;
    (void)aero::host_act(AERO_ACT_SILU, v, nullptr, n);
}

void aero_swiglu(float* gate, const float* up, int64_t n) {
    aero::clear_error();
    if (!gate || !up || n <= 0) return;
    (void)aero::host_act(AERO_ACT_SILU, gate, up, n);
}

// ------------------------------------------------------ src/kernels.cpp ABI
int aero_hardware_threads(void) {
    const unsigned hc = std::thread::hardware_concurrency();
    return (int)std::min(hc == 0 ? 1u : hc, 8u);
}

int aero_dequant_ref(int t, const uint8_t* raw, int64_t raw_len, float* out,
                     int64_t n_values) {
    const int64_t bv = aero::dtype_block_values(t), bb = aero::dtype_block_bytes(t);
    const bool known = t == AERO_DTYPE_F32 || t == AERO_DTYPE_F16 || t == AERO_DTYPE_BF16 ||
                       t == AERO_DTYPE_Q8_0 || t == AERO_DTYPE_Q4_K || t == AERO_DTYPE_Q5_K ||
                       t == AERO_DTYPE_Q6_K || t == AERO_DTYPE_IQ4_XS;
    if (!known || bv <= 0 || !raw || !out || n_values < 0) {
        set_error("aero_dequant_ref: dtype %d not supported on the GPU path or bad args", t);
        return 0;
    }
    const int64_t nblocks = n_values / bv;
    if (raw_len < nblocks * bb) {
        set_error("aero_dequant_ref: raw_len %lld < %lld", (long long)raw_len,
                  (long long)(nblocks * bb));
        return 0;
    }
    if (nblocks == 0) return 1;
    aero::Staging st;
    void* p[2];
    const size_t rbytes = (size_t)(nblocks * bb);
    const size_t obytes = (size_t)(nblocks * bv) * 4;
    if (!st.reserve({rbytes, obytes}, p)) return 0;
    const bool ok = st.h2d(p[0], raw, rbytes) &&
                    aero::dequant_dev(t, static_cast<uint8_t*>(p[0]), (int64_t)rbytes,
                                      static_cast<float*>(p[1]), n_values, st.stream()) &&
                    st.d2h(out, p[1], obytes) && st.finish();
    return ok ? 1 : 0;
}

// src/kernels.cpp:497-538 through :605-615: refuse what the reference refuses
// (a type without a block dot, n_cols % bv), stage W and X, one GEMV launch
// per call.
static int host_gemv(int t, const uint8_t* w, const float* X, float* Y, int64_t n_tok,
                     int64_t n_rows, int64_t n_cols) {
    aero::clear_error();
    const bool quant = t == AERO_DTYPE_Q8_0 || t == AERO_DTYPE_Q4_K || t == AERO_DTYPE_Q5_K ||
                       t == AERO_DTYPE_Q6_K || t == AERO_DTYPE_IQ4_XS;
    const int64_t bv = aero::dtype_block_values(t), bb = aero::dtype_block_bytes(t);
    if (!quant || n_cols < 0 || n_cols % bv != 0 || n_rows < 0 || n_tok < 0) {
        set_error("aero_matvec: dtype %d / n_cols %lld refused", t, (long long)n_cols);
        return 0;
    }
    if (n_rows == 0 || n_tok == 0) return 1;
    if (w == nullptr || X == nullptr || Y == nullptr) {
        set_error("aero_matvec: null pointer");
        return 0;
    }
    if (n_cols == 0) {  // empty dot products, as the reference's loop leaves them
        std::memset(Y, 0, (size_t)(n_tok * n_rows) * sizeof(float));
        return 1;
    }
    const size_t wbytes = (size_t)(n_rows * (n_cols / bv) * bb);
    const size_t xbytes = (size_t)(n_tok * n_cols) * 4, ybytes = (size_t)(n_tok * n_rows) * 4;
    // many tokens of Q4_K / Q5_K: the split-x GEMM's workspace as a fourth buffer
    const int64_t wsb = n_tok >= 32 ? aero::split_gemm_workspace(t, n_cols, n_tok) : 0;
    aero::Staging st;
    void* p[4] = {nullptr, nullptr, nullptr, nullptr};
    if (!(wsb > 0 ? st.reserve({wbytes, xbytes, ybytes, (size_t)wsb}, p)
                  : st.reserve({wbytes, xbytes, ybytes}, p)))
        return 0;
    const bool ok = st.h2d(p[0], w, wbytes) && st.h2d(p[1], X, xbytes) &&
                    aero::gemv_dev(t, static_cast<uint8_t*>(p[0]), (int64_t)wbytes,
                                   static_cast<float*>(p[1]), static_cast<float*>(p[2]), n_rows,
                                   n_cols, n_tok, st.stream(), p[3], wsb) &&
                    st.d2h(Y, p[2], ybytes) && st.finish();
    return ok ? 1 : 0;
}

int aero_matvec(int t, const uint8_t* w, const float* x, float* y, int64_t n_rows,
                int64_t n_cols, int threads) {
    (void)threads;
    return host_gemv(t, w, x, y, 1, n_rows, n_cols);
}

int aero_matmul(int t, const uint8_t* w, const float* X, float* Y, int64_t n_tokens,
                int64_t n_rows, int64_t n_cols, int threads) {
    (void)threads;
    return host_gemv(t, w, X, Y, n_tokens, n_rows, n_cols);
}

int aero_dequant_threaded(int t, const uint8_t* raw, int64_t raw_len, float* out,
                          int64_t n_values, int threads) {
    (void)threads;
    return aero_dequant_ref(t, raw, raw_len, out, n_values);
}


// ------------------------------------------- src/transformer.cpp:259-284 ABI
void aero_softmax(float* v, int64_t n) {
    aero::clear_error();
    if (v == nullptr || n <= 0) return;
    aero::Staging st;
    void* p[1];
    const size_t bytes = (size_t)n * 4;
    if (st.reserve({bytes}, p) && st.h2d(p[0], v, bytes) &&
        aero::softmax_rows_dev(static_cast<float*>(p[0]), static_cast<float*>(p[0]), 1, n,
                               st.stream()))
        (void)(st.d2h(v, p[0], bytes) && st.finish());
}

void aero_softmax_rows(float* v, int64_t n_rows, int64_t n_cols) {
    aero::clear_error();
    if (v == nullptr || n_rows <= 0 || n_cols <= 0) return;
    aero::Staging st;
    void* p[1];
    const size_t bytes = (size_t)(n_rows * n_cols) * 4;
    if (st.reserve({bytes}, p) && st.h2d(p[0], v, bytes) &&
        aero::softmax_rows_dev(static_cast<float*>(p[0]), static_cast<float*>(p[0]), n_rows,
                               n_cols, st.stream()))
        (void)(st.d2h(v, p[0], bytes) && st.finish());
}

// src/tensor.cpp:246-249 aero_tensor_softmax (flat vector, in place).
int aero_tensor_softmax(float* v, int64_t n) {
    if (v == nullptr || n <= 0) {
        aero::clear_error();
        set_error("aero_tensor_softmax: refused");
        return 0;
    }
    aero_softmax(v, n);
    return aero_hip_last_error()[0] == 0 ? 1 : 0;
}

// src/transformer.cpp:120-203 through :266-273. The reference's refusals
// (non-positive sizes, n_head not a multiple of n_head_kv) return 0; `block`
// only changes the reference's rounding and is not needed on the GPU.
int aero_attention_tiled(const float* q, const float* k, const float* v, float* out,
                         int64_t n_q, int64_t n_head, int64_t n_head_kv, int64_t head_dim,
                         int64_t value_dim, float scale, const int32_t* qpos,
                         const int32_t* kpos, int64_t n_kv, int window, int64_t block) {
    (void)block;
    aero::clear_error();
    if (n_q <= 0 || n_head <= 0 || n_head_kv <= 0 || head_dim <= 0 || value_dim <= 0 ||
        n_kv <= 0 || n_head % n_head_kv) {
        set_error("aero_attention_tiled: refused sizes");
        return 0;
    }
    if (q == nullptr || k == nullptr || v == nullptr || out == nullptr) {
        set_error("aero_attention_tiled: null pointer");
        return 0;
    }
    const size_t qb = (size_t)(n_q * n_head * head_dim) * 4;
    const size_t kb = (size_t)(n_kv * n_head_kv * head_dim) * 4;
    const size_t vb = (size_t)(n_kv * n_head_kv * value_dim) * 4;
    const size_t ob = (size_t)(n_q * n_head * value_dim) * 4;
    const size_t qpb = qpos ? (size_t)n_q * 4 : 0, kpb = kpos ? (size_t)n_kv * 4 : 0;
    const int64_t wsb = aero::attn_workspace_bytes(n_q, n_head, n_head_kv, head_dim, value_dim,
                                                   n_kv);
    aero::Staging st;
    void* p[7];
    if (!st.reserve({qb, kb, vb, ob, qpb, kpb, (size_t)wsb}, p)) return 0;
    const bool ok =
        st.h2d(p[0], q, qb) && st.h2d(p[1], k, kb) && st.h2d(p[2], v, vb) &&
        (!qpos || st.h2d(p[4], qpos, qpb)) && (!kpos || st.h2d(p[5], kpos, kpb)) &&
        aero::attention_dev(static_cast<float*>(p[0]), 0, p[1], nullptr, p[2], nullptr,
                            static_cast<float*>(p[3]), n_q, n_head, n_head_kv, head_dim,
                            value_dim, scale, qpos ? static_cast<int32_t*>(p[4]) : nullptr,
                            kpos ? static_cast<int32_t*>(p[5]) : nullptr, n_kv, window,
                            wsb > 0 ? p[6] : nullptr, wsb, st.stream()) &&
        st.d2h(out, p[3], ob) && st.finish();
    return ok ? 1 : 0;
}

// src/transformer.cpp:205-214: one query at position n_kv - 1; keys at
// positions 0..n_kv-1 (the default key positions).
int aero_attention(const float* q, const float* k, const float* v, float* out, int64_t n_head,
                   int64_t n_head_kv, int64_t head_dim, int64_t value_dim, float scale,
                   int64_t n_kv, int window) {
    if (n_kv <= 0) {
        aero::clear_error();
        set_error("aero_attention: n_kv <= 0");
        return 0;
    }
    const int32_t qp = (int32_t)(n_kv - 1);
    return aero_attention_tiled(q, k, v, out, 1, n_head, n_head_kv, head_dim, value_dim, scale,
                                &qp, nullptr, n_kv, window, n_kv);
}

// ---------------------------------------------------- src/kv.cpp:13-46 ABI
// One vector through the device quantiser (dt 0 fp32, 1 int8, 2 int4).
int aero_kv_write_vec(int dt, const float* x, int64_t dim, void* q, float* scale) {
    aero::clear_error();
    if (x == nullptr || q == nullptr || scale == nullptr || dim <= 0 || dt < 0 || dt > 2 ||
        (dt == 2 && dim % 2)) {
        set_error("aero_kv_write_vec: refused");
        return 0;
    }
    const size_t xb = (size_t)dim * 4;
    const size_t qb = dt == 0 ? xb : (dt == 1 ? (size_t)dim : (size_t)dim / 2);
    aero::Staging st;
    void* p[3];
    if (!st.reserve({xb, qb, 4}, p)) return 0;
    const bool ok = st.h2d(p[0], x, xb) &&
                    aero::kv_write_dev(dt, static_cast<float*>(p[0]), 1, 1, dim, 0, 1, p[1],
                                       static_cast<float*>(p[2]), st.stream()) &&
                    st.d2h(q, p[1], qb) && (dt == 0 || st.d2h(scale, p[2], 4)) && st.finish();
    return ok ? 1 : 0;
}
// src/kv.cpp:28-46 aero_kv_read_vec: one vector back to fp32 (code * scale).
int aero_kv_read_vec(int dt, const void* q, const float* scale, int64_t dim, float* out) {
    aero::clear_error();
    if (q == nullptr || scale == nullptr || out == nullptr || dim <= 0 || dt < 0 || dt > 2 ||
        (dt == 2 && dim % 2)) {
        set_error("aero_kv_read_vec: refused");
        return 0;
    }
    const size_t ob = (size_t)dim * 4;
    const size_t qb = dt == 0 ? ob : (dt == 1 ? (size_t)dim : (size_t)dim / 2);
    aero::Staging st;
    void* p[3];
    if (!st.reserve({qb, 4, ob}, p)) return 0;
    const bool ok = st.h2d(p[0], q, qb) && (dt == 0 || st.h2d(p[1], scale, 4)) &&
                    aero::kv_read_dev(dt, p[0], static_cast<float*>(p[1]), 1, dim,
                                      static_cast<float*>(p[2]), st.stream()) &&
                    st.d2h(out, p[2], ob) && st.finish();
    return ok ? 1 : 0;
}

// src/kv.cpp:48-56 aero_kv_ring_indices: 0 .. n-1 (a ring that has not
// wrapped); index bookkeeping on the host.
int aero_kv_ring_indices(int64_t cap, int64_t n, int64_t* out) {
    if (cap <= 0 || n < 0 || out == nullptr || n > cap) return 0;
    for (int64_t i = 0; i < n; ++i) out[i] = i;
    return 1;
}

// src/kv.cpp:58-64 aero_kv_ring_rotate: the physical indices of the first n
// positions in chronological order, (start + i) % cap.
int aero_kv_ring_rotate(int64_t cap, int64_t start, int64_t n, int64_t* out) {
    if (cap <= 0 || n < 0 || out == nullptr || start < 0 || start >= cap || n > cap) return 0;
    for (int64_t i = 0; i < n; ++i) out[i] = (start + i) % cap;
    return 1;
}

// src/kv.cpp:66-82 aero_kv_span_error: max|x - read(q)| / max|x| (1e-9 for
// an all-zero x) of one written vector.
int aero_kv_span_error(int dt, const void* q, const float* scale, int64_t dim, const float* x,
                       float* out) {
    aero::clear_error();
    if (q == nullptr || scale == nullptr || x == nullptr || out == nullptr || dim <= 0 ||
        dt < 0 || dt > 2 || (dt == 2 && dim % 2)) {
        set_error("aero_kv_span_error: refused");
        return 0;
    }
    const size_t xb = (size_t)dim * 4;
    const size_t qb = dt == 0 ? xb : (dt == 1 ? (size_t)dim : (size_t)dim / 2);
    aero::Staging st;
    void* p[4];
    if (!st.reserve({qb, 4, xb, 4}, p)) return 0;
    const bool ok = st.h2d(p[0], q, qb) && (dt == 0 || st.h2d(p[1], scale, 4)) &&
                    st.h2d(p[2], x, xb) &&
                    aero::kv_span_error_dev(dt, p[0], static_cast<float*>(p[1]), dim,
                                            static_cast<float*>(p[2]),
                                            static_cast<float*>(p[3]), st.stream()) &&
                    st.d2h(out, p[3], 4) && st.finish();
    return ok ? 1 : 0;
}

// src/kv.cpp:92-108 aero_kv_slot_new: a slot in HBM on the current device
// (NULL when refused or out of memory).
void* aero_kv_slot_new(int64_t cap, int64_t heads, int64_t dim, int dt, int ring) {
    aero::clear_error();
    if (cap <= 0 || heads <= 0 || dim <= 0 || dt < 0 || dt > 2 || (dt == 2 && dim % 2)) {
        set_error("aero_kv_slot_new: refused (cap=%lld heads=%lld dim=%lld dt=%d)",
                  (long long)cap, (long long)heads, (long long)dim, dt);
        return nullptr;
    }
    auto* sl = new (std::nothrow) aero::KvSlotDev{cap, heads, dim, dt, ring != 0, 0, nullptr,
                                                 nullptr};
    if (sl == nullptr) return nullptr;
    const size_t qb = (size_t)(cap * heads * sl->vec_bytes());
    const size_t sb = dt != 0 ? (size_t)(cap * heads) * 4 : 0;
    bool ok = aero::hip_ok(hipGetDevice(&sl->device), "hipGetDevice") &&
              aero::hip_ok(hipMalloc(&sl->q, qb), "hipMalloc(kv slot)") &&
              aero::hip_ok(hipMemset(sl->q, 0, qb), "hipMemset(kv slot)");
    if (ok && sb) {
        void* sp = nullptr;
        ok = aero::hip_ok(hipMalloc(&sp, sb), "hipMalloc(kv slot scales)") &&
             aero::hip_ok(hipMemset(sp, 0, sb), "hipMemset(kv slot scales)");
        sl->scale = static_cast<float*>(sp);
    }
    if (!ok) {
        if (sl->q) (void)hipFree(sl->q);
        if (sl->scale) (void)hipFree(sl->scale);
        delete sl;
        return nullptr;
    }
    return sl;
}

// src/kv.cpp:110 aero_kv_slot_free (NULL is ignored).
void aero_kv_slot_free(void* s) {
    auto* sl = static_cast<aero::KvSlotDev*>(s);
    if (sl == nullptr) return;
    (void)hipDeviceSynchronize();
    if (sl->q) (void)hipFree(sl->q);
    if (sl->scale) (void)hipFree(sl->scale);
    delete sl;
}

// src/kv.cpp:112-115 aero_kv_slot_bytes: the reference's KvSlot::bytes()
// (codes plus int8/int4 scales); -1 for NULL.
int64_t aero_kv_slot_bytes(void* s) {
    auto* sl = static_cast<aero::KvSlotDev*>(s);
    return sl ? sl->bytes() : -1;
}

// src/kv.cpp:117-124 aero_kv_slot_write: quantise host x into the slot's
// (phys, head) vector; the head is checked too (the reference checks phys
// only).
int aero_kv_slot_write(void* s, int64_t phys, int64_t head, const float* x) {
    auto* sl = static_cast<aero::KvSlotDev*>(s);
    aero::clear_error();
    if (sl == nullptr || x == nullptr || phys < 0 || phys >= sl->cap || head < 0 ||
        head >= sl->heads) {
        set_error("aero_kv_slot_write: refused");
        return 0;
    }
    int dev = -1;
    if (!aero::hip_ok(hipGetDevice(&dev), "hipGetDevice")) return 0;
    if (dev != sl->device) {
        set_error("aero_kv_slot_write: the slot lives on device %d, device %d is current", sl->device,
                  dev);
        return 0;
    }
    const int64_t vec = phys * sl->heads + head;
    const size_t xb = (size_t)sl->dim * 4;
    aero::Staging st;
    void* p[1];
    if (!st.reserve({xb}, p)) return 0;
    void* qv = static_cast<uint8_t*>(sl->q) + vec * sl->vec_bytes();
    const bool ok = st.h2d(p[0], x, xb) &&
                    aero::kv_write_dev(sl->dt, static_cast<float*>(p[0]), 1, 1, sl->dim, 0, 1,
                                       qv, sl->scale ? sl->scale + vec : nullptr, st.stream()) &&
                    st.finish();
    return ok ? 1 : 0;
}

// src/kv.cpp:126-131 aero_kv_slot_read: the slot's (phys, head) vector as
// fp32 into host out.
int aero_kv_slot_read(void* s, int64_t phys, int64_t head, float* out) {
    auto* sl = static_cast<aero::KvSlotDev*>(s);
    aero::clear_error();
    if (sl == nullptr || out == nullptr || phys < 0 || phys >= sl->cap || head < 0 ||
        head >= sl->heads) {
        set_error("aero_kv_slot_read: refused");
        return 0;
    }
    int dev = -1;
    if (!aero::hip_ok(hipGetDevice(&dev), "hipGetDevice")) return 0;
    if (dev != sl->device) {
        set_error("aero_kv_slot_read: the slot lives on device %d, device %d is current", sl->device,
                  dev);
        return 0;
    }
    const int64_t vec = phys * sl->heads + head;
    const size_t ob = (size_t)sl->dim * 4;
    aero::Staging st;
    void* p[1];
    if (!st.reserve({ob}, p)) return 0;
    const void* qv = static_cast<const uint8_t*>(sl->q) + vec * sl->vec_bytes();
    const bool ok = aero::kv_read_dev(sl->dt, qv, sl->scale ? sl->scale + vec : nullptr, 1,
                                      sl->dim, static_cast<float*>(p[0]), st.stream()) &&
                    st.d2h(out, p[0], ob) && st.finish();
    return ok ? 1 : 0;
}

int aero_hip_kv_slot_view(void* s, void** q, float** scale, int64_t* cap, int64_t* heads,
                          int64_t* dim, int* dt, int* ring) {
    auto* sl = static_cast<aero::KvSlotDev*>(s);
    aero::clear_error();
    if (sl == nullptr) {
        set_error("aero_hip_kv_slot_view: NULL slot");
        return 0;
    }
    if (q) *q = sl->q;
    if (scale) *scale = sl->scale;
    if (cap) *cap = sl->cap;
    if (heads) *heads = sl->heads;
    if (dim) *dim = sl->dim;
    if (dt) *dt = sl->dt;
    if (ring) *ring = sl->ring;
    return 1;
}

// ------------------------------------------------------- gated DeltaNet
// src/ssm.cpp:151-210. Host arrays, synchronous; the void entries report a
// refusal through aero_hip_last_error() and leave the outputs unwritten.

// softplus(x) = log1p(exp(-|x|)) + max(x, 0) (src/ssm.cpp:22-24): a scalar
// helper of the ABI, evaluated on the host.
float aero_ssm_softplus(float x) { return log1pf(expf(-fabsf(x))) + (x > 0.0f ? x : 0.0f); }

static bool host_ssm_scan(const float* q, const float* k, const float* v, const float* alpha,
                          const float* beta, const float* a_log, const float* dt_bias,
                          float* state, int64_t T, int64_t n_k, int64_t n_v, int64_t d,
                          float scale, float eps, float* outs) {
    if (T < 0 || n_k <= 0 || n_v <= 0 || d <= 0 || n_v % n_k || !q || !k || !v || !alpha ||
        !beta || !a_log || !dt_bias || !state || !outs) {
        set_error("aero_ssm_scan: refused arguments");
        return false;
    }
    const size_t qb = (size_t)(T * n_k * d) * 4, vb = (size_t)(T * n_v * d) * 4;
    const size_t ab = (size_t)(T * n_v) * 4, hb = (size_t)n_v * 4;
    const size_t sb = (size_t)(n_v * d * d) * 4;
    const int64_t wsb = aero::ssm_workspace_bytes(T, n_k, n_v, d);
    aero::Staging st;
    void* p[10];
    if (!st.reserve({qb, qb, vb, ab, ab, hb, hb, sb, vb, (size_t)wsb}, p)) return false;
    float** f = reinterpret_cast<float**>(p);
    return st.h2d(f[0], q, qb) && st.h2d(f[1], k, qb) && st.h2d(f[2], v, vb) &&
           st.h2d(f[3], alpha, ab) && st.h2d(f[4], beta, ab) && st.h2d(f[5], a_log, hb) &&
           st.h2d(f[6], dt_bias, hb) && st.h2d(f[7], state, sb) &&
           aero::ssm_scan_dev(f[0], f[1], f[2], f[3], f[4], f[5], f[6], f[7], T, n_k, n_v, d,
                              scale, eps, f[8], p[9], wsb, st.stream()) &&
           st.d2h(outs, f[8], vb) && st.d2h(state, f[7], sb) && st.finish();
}

// One token with q/k already tiled to n_heads (src/ssm.cpp:153-161).
void aero_ssm_delta_step(const float* q, const float* k, const float* v, const float* alpha,
                         const float* beta, const float* a_log, const float* dt_bias,
                         float* state, int n_heads, int d, float scale, float eps, float* out) {
    aero::clear_error();
    (void)host_ssm_scan(q, k, v, alpha, beta, a_log, dt_bias, state, 1, n_heads, n_heads, d,
                        scale, eps, out);
}

// T tokens, v-head h reading k-head h % n_k (src/ssm.cpp:163-171).
void aero_ssm_scan(const float* qh, const float* kh, const float* vh, const float* alpha,
                   const float* beta, const float* a_log, const float* dt_bias, float* state,
                   int T, int n_k, int n_v, int d, float scale, float eps, float* outs) {
    aero::clear_error();
    (void)host_ssm_scan(qh, kh, vh, alpha, beta, a_log, dt_bias, state, T, n_k, n_v, d, scale,
                        eps, outs);
}

// Causal depthwise conv over [tail; x]; tail (kernel - 1 rows of room) and
// *tail_len are updated in place (src/ssm.cpp:173-210).
void aero_ssm_conv(const float* x, const float* w, float* tail, int* tail_len, float* out,
                   int T, int channels, int kernel) {
    aero::clear_error();
    if (tail_len == nullptr || x == nullptr || w == nullptr || out == nullptr || T < 0 ||
        channels <= 0 || kernel <= 0 || *tail_len < 0 || *tail_len > kernel - 1 ||
        (kernel > 1 && tail == nullptr)) {
        set_error("aero_ssm_conv: refused arguments");
        return;
    }
    const int64_t tl = *tail_len;
    const size_t xb = (size_t)T * channels * 4, wb = (size_t)channels * kernel * 4;
    const size_t tb = (size_t)(kernel > 1 ? kernel - 1 : 0) * channels * 4;
    aero::Staging st;
    void* p[4];
    if (!st.reserve({xb, wb, tb, xb}, p)) return;
    float** f = reinterpret_cast<float**>(p);
    int64_t keep = 0;
    if (st.h2d(f[0], x, xb) && st.h2d(f[1], w, wb) &&
        st.h2d(f[2], tail, (size_t)tl * channels * 4) &&
        aero::ssm_conv_dev(f[0], f[1], f[2], tl, f[2], f[3], T, channels, kernel, &keep,
                           st.stream()) &&
        st.d2h(out, f[3], xb) && st.d2h(tail, f[2], (size_t)keep * channels * 4) && st.finish())
        *tail_len = (int)keep;
}

}  // extern "C"
