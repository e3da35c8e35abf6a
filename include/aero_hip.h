/* aero_hip.h -- C ABI of libaero_hip.so, the MI355X (gfx950) implementation of
 * Aero's fused per-layer elementwise path: RMSNorm (plain, (1+w), per-head
 * QK-norm, gated norm*silu), act*mul (SwiGLU, GeGLU erf/tanh), RoPE (NeoX and
 * interleaved, full and partial, computed angle or pre-computed table) and
 * GGUF embedding row gather with Q8_0 / Q4_K / Q6_K dequant.
 *
 * Three groups of entry points:
 *
 *  1. Reference-compatible host-pointer symbols. Same names, signatures and
 *     status conventions as the reference's C ABI, so the reference's ctypes
 *     bindings can load this library in place of libaero_tensor /
 *     libaero_transformer / libaero_kernels for these ops. Buffers are host
 *     memory; each call stages them through HBM, runs the kernel, copies the
 *     result back and returns when it is complete (synchronous, like the
 *     reference). Citations name the reference function each one replaces.
 *
 *  2. Device-pointer entry points (aero_hip_*). All buffers are HBM pointers;
 *     work is enqueued on `stream` (NULL = the null stream) and the call
 *     returns without waiting. They return 1 on success and 0 on refusal
 *     (bad shape, misaligned pointer, HIP error); aero_hip_last_error()
 *     then describes why. Nothing is allocated; the caller owns every buffer.
 *
 *  3. Runtime helpers (device memory, streams, events, per-kernel timing)
 *     so that a host without PyTorch can drive the device path.
 *
 * Layouts are row-major fp32 unless stated. Pointers must be 16-byte aligned
 * where a vectorised kernel applies (any hipMalloc pointer is); unaligned or
 * odd-sized inputs take a scalar kernel with the same arithmetic.
 */
#ifndef AERO_HIP_H
#define AERO_HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ------------------------------------------------------------------------
 * 1. Reference-compatible host-pointer ABI
 * ---------------------------------------------------------------------- */

/* src/tensor.cpp:207 aero_tensor_threads: the default thread count of the
 * reference's native layer (hardware threads, at most 8); the GPU entry
 * points take and ignore `threads`. */
int aero_tensor_threads(void);
/* src/tensor.cpp:209-218 aero_tensor_matvec: y[r] = dot(W.row(r), x), W
 * [n_rows, n_cols] fp32, summed in the reference's order (four products at
 * a time): bit-identical. 1 = ok, 0 = refused (null or dims <= 0). */
int aero_tensor_matvec(const float* w, const float* x, float* y, int64_t n_rows,
                       int64_t n_cols, int threads);
/* src/tensor.cpp:220-231 aero_tensor_matmul: Y[t][r] = dot(W.row(r), X.row(t)),
 * X [n_tokens, n_cols], Y [n_tokens, n_rows]; one token is the matvec,
 * several sum one product at a time as the reference: bit-identical. */
int aero_tensor_matmul(const float* w, const float* X, float* Y, int64_t n_tokens,
                       int64_t n_rows, int64_t n_cols, int threads);
/* src/tensor.cpp:298-302 aero_tensor_argmax: index of the first largest
 * value (NaN never chosen; 0 when v[0] is NaN), -1 = refused. */
int aero_tensor_argmax(const float* v, int64_t n);
/* src/tensor.cpp:234-238 aero_tensor_silu: v[i] *= sigmoid(v[i]), in place.
 * 1 = ok, 0 = refused (null or n <= 0). */
int aero_tensor_silu(float* v, int64_t n);
/* src/tensor.cpp:240-244 aero_tensor_gelu: erf-form GELU (A&S 7.1.26), in place. */
int aero_tensor_gelu(float* v, int64_t n);
/* src/tensor.cpp:252-257 aero_tensor_mul: a[i] *= b[i]. */
int aero_tensor_mul(float* a, const float* b, int64_t n);
/* src/tensor.cpp:259-264 aero_tensor_swiglu: gate[i] = silu(gate[i])*up[i]. */
int aero_tensor_swiglu(float* gate, const float* up, int64_t n);
/* src/tensor.cpp:266-275 aero_tensor_rmsnorm: out = x/sqrt(mean(x^2)+eps)*w. */
int aero_tensor_rmsnorm(const float* x, const float* weight, float* out,
                        int64_t n, float eps);
/* src/tensor.cpp:277-288 aero_tensor_l2norm: out = x/max(||x||,eps)*w
 * (weighted = 1) or weightless (weighted = 0, weight may be NULL). */
int aero_tensor_l2norm(const float* x, const float* weight, float* out,
                       int64_t n, float eps, int weighted);
/* src/tensor.cpp:290-296 aero_tensor_rmsnorm_rows: weightless per-row RMS
 * over a rows x cols block, in place. */
int aero_tensor_rmsnorm_rows(float* t, int64_t rows, int64_t cols, float eps);

/* src/transformer.cpp:227-233 aero_rope_tables: cos/sin [n_pos, n_rot/2],
 * ROW-indexed (row t = positions[t]). Returns n_rot, or -1 when head_dim <= 0,
 * n_pos < 0, positions == NULL or freq_factors is shorter than n_rot/2
 * (and -1 on a HIP failure, which the reference cannot have). */
int64_t aero_rope_tables(int64_t head_dim, const int32_t* positions,
                         int64_t n_pos, float base, int64_t n_dims,
                         const float* freq_factors, int64_t n_ff,
                         float* cos_out, float* sin_out);
/* src/transformer.cpp:235-240 aero_apply_rope: rotate x [n_rows, head_dim]
 * in place; row r reads table row positions[r] (or r when NULL). mode 0 =
 * NeoX, otherwise interleaved. Rows with a negative position are refused as
 * a whole (nothing is written; aero_hip_last_error says why). */
void aero_apply_rope(float* x, int64_t n_rows, int64_t head_dim, int64_t n_rot,
                     const float* cos_tab, const float* sin_tab,
                     const int32_t* positions, int mode);
/* src/transformer.cpp:242-245 aero_rmsnorm_rows: out (may alias x) =
 * per-row RMSNorm; weight NULL = ones. */
void aero_rmsnorm_rows(const float* x, const float* weight, float* out,
                       int64_t n_rows, int64_t n_cols, float eps);
/* src/transformer.cpp:247-250 aero_l2norm_rows. */
void aero_l2norm_rows(const float* x, const float* weight, float* out,
                      int64_t n_rows, int64_t n_cols, float eps);
/* src/transformer.cpp:252-253 aero_gelu / aero_silu (in place, void). */
void aero_gelu(float* v, int64_t n);
void aero_silu(float* v, int64_t n);
/* src/transformer.cpp:255-257 aero_swiglu (in place on gate, void). */
void aero_swiglu(float* gate, const float* up, int64_t n);

/* src/kernels.cpp:560-565 block geometry of a ggml type id; 0 if unknown. */
int64_t aero_dtype_block_bytes(int t);
int64_t aero_dtype_block_values(int t);
/* src/kernels.cpp:566 aero_hardware_threads: min(host cores, 8). Kept for the
 * reference binding's auto-thread rule; the GPU path ignores it. */
int aero_hardware_threads(void);
/* src/kernels.cpp:568-584 aero_dequant_ref: dequantise floor(n/bv) blocks of
 * type t (F32, F16, BF16, Q8_0, Q4_K, Q5_K, Q6_K, IQ4_XS). Refuses (0) a raw_len shorter
 * than the blocks need, or any other type. */
int aero_dequant_ref(int t, const uint8_t* raw, int64_t raw_len, float* out,
                     int64_t n_values);
/* src/kernels.cpp:587-603 aero_dequant_threaded: same result; `threads` is
 * accepted for signature compatibility and ignored. */
int aero_dequant_threaded(int t, const uint8_t* raw, int64_t raw_len,
                          float* out, int64_t n_values, int threads);
/* src/kernels.cpp:605-609 aero_matvec: y = W @ x, W n_rows rows of quant
 * blocks of type t (Q8_0, Q4_K, Q5_K, Q6_K, IQ4_XS). 1 = done; 0 = refused
 * (another type, n_cols % block size, a null pointer). W is uploaded per call;
 * `threads` is ignored. */
int aero_matvec(int t, const uint8_t* w, const float* x, float* y, int64_t n_rows,
                int64_t n_cols, int threads);
/* src/kernels.cpp:611-615 aero_matmul: Y[t*n_rows + r] = row r of W dotted
 * with token t of X, for n_tokens tokens. Same refusals as aero_matvec. */
int aero_matmul(int t, const uint8_t* w, const float* X, float* Y, int64_t n_tokens,
                int64_t n_rows, int64_t n_cols, int threads);

/* src/tensor.cpp:246-249 aero_tensor_softmax (in place; 0 = refused). */
int aero_tensor_softmax(float* v, int64_t n);
/* src/transformer.cpp:259-263 aero_softmax / aero_softmax_rows (in place). */
void aero_softmax(float* v, int64_t n);
void aero_softmax_rows(float* v, int64_t n_rows, int64_t n_cols);
/* src/transformer.cpp:266-273 aero_attention_tiled: GQA attention with an
 * online softmax, q [n_q, n_head, head_dim], k [n_kv, n_head_kv, head_dim],
 * v [n_kv, n_head_kv, value_dim] -> out [n_q, n_head, value_dim]; key j kept
 * for query t when kpos[j] <= qpos[t] (and qpos - kpos < window when
 * window > 0); null positions mean t / j. 1 = done, 0 = refused (non-positive
 * sizes, n_head % n_head_kv). `block` is accepted and not needed. */
int aero_attention_tiled(const float* q, const float* k, const float* v, float* out,
                         int64_t n_q, int64_t n_head, int64_t n_head_kv, int64_t head_dim,
                         int64_t value_dim, float scale, const int32_t* qpos,
                         const int32_t* kpos, int64_t n_kv, int window, int64_t block);
/* src/transformer.cpp:276-281 aero_attention: one query at position n_kv-1. */
int aero_attention(const float* q, const float* k, const float* v, float* out, int64_t n_head,
                   int64_t n_head_kv, int64_t head_dim, int64_t value_dim, float scale,
                   int64_t n_kv, int window);
/* src/kv.cpp:13-26 aero_kv_write_vec: quantise one vector (dt 0 fp32 copy,
 * 1 int8 with scale amax/127, 2 int4 low-nibble-first with scale amax/7). */
int aero_kv_write_vec(int dt, const float* x, int64_t dim, void* q, float* scale);
/* src/kv.cpp:28-46 aero_kv_read_vec: one vector back to fp32, code * scale
 * (bit-exact). 0 = refused. */
int aero_kv_read_vec(int dt, const void* q, const float* scale, int64_t dim, float* out);
/* src/kv.cpp:48-56 aero_kv_ring_indices: out[i] = i for i < n <= cap. */
int aero_kv_ring_indices(int64_t cap, int64_t n, int64_t* out);
/* src/kv.cpp:58-64 aero_kv_ring_rotate: out[i] = (start + i) % cap, the
 * chronological physical order of a wrapped ring. */
int aero_kv_ring_rotate(int64_t cap, int64_t start, int64_t n, int64_t* out);
/* src/kv.cpp:66-82 aero_kv_span_error: *out = max|x - read(q)| / max|x|
 * (1e-9 for an all-zero x), bit-exact. */
int aero_kv_span_error(int dt, const void* q, const float* scale, int64_t dim, const float* x,
                       float* out);
/* src/kv.cpp:92-133 the KV slot, here resident in HBM on the device current
 * at creation: codes [cap, heads, dim] (dt 0 fp32, 1 int8, 2 int4) plus one
 * fp32 scale a vector for int8/int4, zeroed. new returns NULL when refused;
 * bytes is the reference's KvSlot::bytes() (-1 for NULL); write quantises a
 * host vector into (phys, head), read returns it as fp32; both refuse a phys
 * or head out of range (the reference checks phys only) and another current
 * device. A ring slot's wrap is the caller's, as in the reference. */
void*   aero_kv_slot_new(int64_t cap, int64_t heads, int64_t dim, int dt, int ring);
void    aero_kv_slot_free(void* slot);
int64_t aero_kv_slot_bytes(void* slot);
int     aero_kv_slot_write(void* slot, int64_t phys, int64_t head, const float* x);
int     aero_kv_slot_read(void* slot, int64_t phys, int64_t head, float* out);
/* The device side of a slot: its codes and scales in HBM (the k / v and
 * k_scale / v_scale arguments of aero_hip_attention, vector (phys, head) at
 * phys * heads + head) and its shape. No counterpart in the reference. */
int aero_hip_kv_slot_view(void* slot, void** q, float** scale, int64_t* cap, int64_t* heads,
                          int64_t* dim, int* dt, int* ring);

/* ------------------------------------------------------------------------
 * 2. Device-pointer fused ops (HBM pointers, asynchronous on `stream`)
 * ---------------------------------------------------------------------- */

#define AERO_NORM_UNIT_OFFSET 1 /* weight is applied as (1 + w) (Gemma)      */
#define AERO_NORM_L2          2 /* divisor max(||x||, eps) instead of RMS     */

/* Per-row RMSNorm: out[r] = x[r] * (1/sqrt(mean(x[r]^2)+eps)) * w.
 * Replaces src/tensor.cpp:128-134 / src/transformer.cpp:98-104 (rows) and,
 * with rows = T*H and cols = head_dim, the per-head QK-norm of
 * src/attention_layer.cpp:89-108. w may be NULL (ones); out may alias x. */
int aero_hip_rmsnorm(const float* x, const float* w, float* out, int64_t rows,
                     int64_t cols, float eps, int flags, void* stream);

/* Gated RMSNorm * silu (src/ssm.cpp:327-343): x, z, out are [rows, inner];
 * for each group-long slice: denom = sqrt(mean(x^2)+eps),
 * out = ((x/denom) * w[col % w_len]) * z/(1+exp(-z)). group = inner is the
 * reference's whole-row RMS; group must divide inner. out may alias x. */
int aero_hip_gated_rmsnorm_silu(const float* x, const float* z, const float* w,
                                int64_t w_len, float* out, int64_t rows,
                                int64_t inner, int64_t group, float eps,
                                void* stream);

/* A Gemma block's sandwich-norm site in one pass (src/model.cpp:213-215,
 * 224-231): the sublayer output y is normalised with its post-norm weight,
 * scaled by ds and added to the residual stream, the sum scaled by ss, and
 * the next norm taken of it:
 *   a = rmsnorm(y) * w_post;  x_out = (x + ds * a) * ss;
 *   h = rmsnorm(x_out) * w_next
 * rmsnorm as aero_hip_rmsnorm (same eps; flags 0 or AERO_NORM_UNIT_OFFSET
 * for both weights; NULL weights are ones). After attention ss = 1 and
 * w_next is the FFN norm; after the FFN, ss is the layer output scale and
 * w_next the next block's attention norm (or the output norm). x_out may
 * alias x; h must not alias y, x or x_out, nor x_out y. [rows, cols] fp32. */
int aero_hip_post_norm_add(const float* y, const float* x, float* x_out, const float* w_post,
                           float ds, float ss, const float* w_next, float* h, int64_t rows,
                           int64_t cols, float eps, int flags, void* stream);

/* Residual add + RMSNorm in one pass: x_out = x + d (the residual stream),
 * h = rmsnorm(x_out) * w as aero_hip_rmsnorm (flags 0 or
 * AERO_NORM_UNIT_OFFSET; w NULL = ones). Replaces the reference block's
 * `x_[i] += o_[i]` followed by norm_row(x_, w, h_) (src/model.cpp:279-282),
 * and the end of a block (`x_ += d_`, :284) followed by the next block's
 * first norm_row (:244-245). x_out may alias x or d (x_out == x: in place,
 * as the reference); h must be a different buffer. [rows, cols] fp32. */
int aero_hip_add_rmsnorm(const float* x, const float* d, float* x_out, const float* w,
                         float* h, int64_t rows, int64_t cols, float eps, int flags,
                         void* stream);

#define AERO_ACT_SILU      0 /* g*sigmoid(g)           src/tensor.cpp:104-106,120-125 */
#define AERO_ACT_GELU      1 /* erf GELU, A&S 7.1.26   src/tensor.cpp:52-59,108-114   */
#define AERO_ACT_GELU_TANH 2 /* tanh-approximate GELU (no reference function)        */
#define AERO_ACT_IDENTITY  3 /* plain product (mul_)   src/tensor.cpp:116-118         */
#define AERO_ACT_SIGMOID   4 /* sigmoid(g), the attention output gate
                                src/attention_layer.cpp:262-263 (act-mul only)      */

/* out[i] = act(gate[i]) * up[i] (up == NULL: out = act(gate)). n elements.
 * out may alias gate or up. Replaces swiglu_ / gelu_+mul_ / silu_ / mul_. */
int aero_hip_act_mul(int kind, const float* gate, const float* up, float* out,
                     int64_t n, void* stream);

/* Host-side arithmetic only (no device work): the per-pair inverse
 * frequencies of src/transformer.cpp:34-47, inv[p] = 1/powf(base,
 * (float)p*2/(float)n) (/ ff[p]), written to host inv_out[n/2]. Returns n
 * (the rotated width, even) or -1. Computing them on the host with the same
 * expression keeps (float)pos*inv bit-identical to the reference's angle. */
int64_t aero_hip_rope_inv_freq(int64_t head_dim, int64_t n_dims, float base,
                               const float* freq_factors, int64_t n_ff,
                               float* inv_out);

/* Device rope_tables: cos/sin[t*half + p] = cos/sin((float)pos[t]*inv[p]).
 * pos [n_pos] int32, inv [half] (from aero_hip_rope_inv_freq). */
int aero_hip_rope_tables(const int32_t* pos, int64_t n_pos, const float* inv,
                         int64_t half, float* cos_out, float* sin_out,
                         void* stream);

#define AERO_ROPE_NEOX        0 /* pairs (x[p], x[p+n_rot/2]) */
#define AERO_ROPE_INTERLEAVED 1 /* pairs (x[2p], x[2p+1])      */

/* Fused per-head RMSNorm -> RoPE on q [n_tok, n_q_heads, head_dim] and
 * (optionally) k [n_tok, n_k_heads, head_dim], one pass per head row.
 * Reproduces src/attention_layer.cpp:89-156: optional RMSNorm over the head
 * (q_norm_w / k_norm_w [head_dim], NULL = no norm for that tensor;
 * norm_flags as for aero_hip_rmsnorm), then RoPE on the first n_rot
 * channels at the token's position (every head of a token shares it):
 *   - angle source: inv_freq [n_rot/2] (angle = (float)pos*inv[p], fp32,
 *     accurate sincos) or a POSITION-indexed table cos_tab/sin_tab
 *     [n_tab, n_rot/2] (exactly one of the two must be given);
 *   - pos [n_tok] int32 (NULL = token index); a token whose position falls
 *     outside [0, n_tab) of a table is left unchanged;
 *   - channels >= n_rot pass through (normalised when a norm is applied).
 * q_out / k_out NULL = in place. n_k_heads may be 0 with k == NULL. */
int aero_hip_qk_norm_rope(float* q, float* q_out, int64_t n_q_heads,
                          float* k, float* k_out, int64_t n_k_heads,
                          const float* q_norm_w, const float* k_norm_w,
                          float eps, int norm_flags, int64_t n_tok,
                          int64_t head_dim, int64_t n_rot, int mode,
                          const int32_t* pos, const float* inv_freq,
                          const float* cos_tab, const float* sin_tab,
                          int64_t n_tab, void* stream);

/* ggml type ids accepted by the gather / dequant entry points */
#define AERO_DTYPE_F32  0
#define AERO_DTYPE_F16  1
#define AERO_DTYPE_Q8_0 8
#define AERO_DTYPE_Q4_K 12
#define AERO_DTYPE_Q5_K 13
#define AERO_DTYPE_Q6_K 14
#define AERO_DTYPE_IQ4_XS 23
#define AERO_DTYPE_BF16 30

/* Token-embedding row gather + dequant (src/model.cpp:297-316 with
 * dequant_ref, src/kernels.cpp:315-458): out[i, :] = dequant(table row
 * ids[i]) (* scale when scale > 0, a separate fp32 multiply as the reference's
 * second pass). table holds vocab rows of (n_embd/bv)*bb bytes (table_bytes
 * >= that, base 4-byte aligned); types Q8_0, Q4_K, Q5_K, Q6_K, IQ4_XS. An id outside
 * [0, vocab) yields a zero row and, when bad_count != NULL, adds 1 to
 * *bad_count (device uint32; the caller clears it). */
int aero_hip_embed_gather(int dtype, const uint8_t* table, int64_t table_bytes,
                          int64_t vocab, int64_t n_embd, const int32_t* ids,
                          int64_t n_ids, float scale, float* out,
                          uint32_t* bad_count, void* stream);

/* Embedding gather + the first block's RMSNorm in one pass: x_out[i] =
 * dequant(table row ids[i]) (* scale when scale > 0), exactly as
 * aero_hip_embed_gather, and h_out[i] = rmsnorm(x_out[i]) * norm_w as
 * aero_hip_rmsnorm (norm_flags 0 or AERO_NORM_UNIT_OFFSET; norm_w NULL =
 * ones). Replaces the reference's embedding loop and scale pass
 * (src/model.cpp:297-316) followed by norm_row(x_, attn_norm, h_)
 * (src/model.cpp:244-245). x_out, h_out, norm_w 16-byte aligned; x_out !=
 * h_out; n_embd <= 8*8*256 values. Out-of-range ids as embed_gather (zero
 * x and h rows, *bad_count += 1). */
int aero_hip_embed_rmsnorm(int dtype, const uint8_t* table, int64_t table_bytes,
                           int64_t vocab, int64_t n_embd, const int32_t* ids, int64_t n_ids,
                           float scale, float* x_out, const float* norm_w, float eps,
                           int norm_flags, float* h_out, uint32_t* bad_count,
                           void* stream);

/* Rows [r0, r1) of a resident tensor (n_rows rows of n_per_row values, whole
 * blocks a row, table 4-byte aligned) dequantised to out [(r1-r0) x
 * n_per_row] (16-byte aligned): the device form of the row addressing of
 * engine/gguf.py:278-314 (GGUFReader.tensor_rows). Types F32, F16, BF16,
 * Q8_0, Q4_K, Q5_K, Q6_K, IQ4_XS; 0 with a reason for a range outside
 * [0, n_rows) or a short table. */
int aero_hip_tensor_rows(int dtype, const uint8_t* table, int64_t table_bytes, int64_t n_rows,
                         int64_t n_per_row, int64_t r0, int64_t r1, float* out, void* stream);

/* Whole-buffer dequant (the device form of aero_dequant_ref): floor(n/bv)
 * blocks of raw -> out. Types F32, F16, BF16, Q8_0, Q4_K, Q5_K, Q6_K, IQ4_XS. */
int aero_hip_dequant(int dtype, const uint8_t* raw, int64_t raw_len, float* out,
                     int64_t n_values, void* stream);

/* Quantised GEMV / small-batch GEMM, the device form of the reference's
 * matvec / matmul (src/kernels.cpp:497-538, block dots :78-250):
 * y[t*n_rows + r] = sum_c W[r, c] * x[t*n_cols + c] for t < n_tok, W =
 * n_rows rows of (n_cols/bv)*bb bytes of type dtype (Q8_0, Q4_K, Q5_K, Q6_K,
 * IQ4_XS; w_bytes >= that, base 4-byte aligned), x fp32 16-byte aligned.
 * n_cols must be a multiple of the block size. Sums run in a different order
 * from the reference's serial loop (equal to ~1e-6 of the output scale). */
int aero_hip_matvec(int dtype, const uint8_t* w, int64_t w_bytes, const float* x,
                    float* y, int64_t n_rows, int64_t n_cols, int64_t n_tok,
                    void* stream);

/* aero_hip_matvec with a workspace, the same call as the reference's matmul
 * (src/kernels.cpp:520-538). With enough tokens of Q4_K, Q5_K, Q8_0,
 * Q6_K (rows a multiple of 2048 columns) or IQ4_XS (of 512) (5 for matrices
 * of 32M+ weights, 4 when their rows are longer than 4096 columns, 7 for 8M+,
 * 10 for 2M+, else 16: where measured faster)
 * and
 * `ws` 16-byte aligned of at least aero_hip_matmul_workspace(dtype, n_cols,
 * n_tok) bytes (W 16-byte aligned), the GEMM runs on the fp16 matrix cores
 * with x split into two fp16 parts per token and 256 columns (22
 * significant bits of x, exact products, fp32 sums; ws holds the parts);
 * otherwise it is aero_hip_matvec. Below 16 tokens the split GEMM is taken
 * only when ws also holds aero_hip_split_partials_bytes for its column
 * splits (unsplit it is slower than the GEMV there). Calls sharing one
 * workspace must be ordered on one stream. */
/* Decode steps of a decoder layer in one launch each. The reference runs
 * them as separate passes: rmsnorm_rows (src/transformer.cpp:98-104, or
 * src/tensor.cpp:128-134), matvec (src/kernels.cpp:497-518) per matrix,
 * act_mul (src/tensor.cpp:104-125); each result equals that composition to
 * 1e-5 of its scale.
 *   aero_hip_norm_matvec: y[m][t*n_rows[m] + r] = sum_c W_m[r, c] * xn[t, c]
 *     for up to 4 matrices of one type and width sharing x (q, k, v; a
 *     DeltaNet layer's qkv, gate, alpha, beta);
 *   aero_hip_norm_gate_up: out[t*n_ff + r] = act(Wg[r] . xn[t]) * (Wu[r] . xn[t]).
 * xn = x normalised as aero_hip_rmsnorm with weight norm_w (nullable: ones)
 * and flags `norm` (0 or AERO_NORM_UNIT_OFFSET); norm < 0: xn = x. act is an
 * AERO_ACT_* kind. Weights 16-byte aligned with rows of a multiple of 16
 * bytes (the gemv fast path; Q8_0 rows of a multiple of 8 bytes too, such
 * as the 952-byte rows of 896 columns, when w_bytes also covers the 16-byte
 * boundary at or after the last row's end), x and norm_w 16-byte aligned;
 * tokens are taken up to 4 a launch. */
int aero_hip_norm_matvec(int dtype, int n_mat, const uint8_t* const* w,
                         const int64_t* w_bytes, const int64_t* n_rows, float* const* y,
                         const float* x, const float* norm_w, float eps, int norm,
                         int64_t n_cols, int64_t n_tok, void* stream);
int aero_hip_norm_gate_up(int dtype, const uint8_t* w_gate, const uint8_t* w_up,
                          int64_t w_bytes, const float* x, const float* norm_w, float eps,
                          int norm, int act, float* out, int64_t n_ff, int64_t n_cols,
                          int64_t n_tok, void* stream);
/* A gated-DeltaNet layer's input projections and its causal conv for one
 * token (decode), in one launch: matrices 0 .. n_mat-1 (1-4, one type and
 * width, weights as aero_hip_norm_matvec) times x as aero_hip_norm_matvec with
 * no norm, except that matrix 0's rows (the qkv projection, n_rows[0]
 * channels) go through the conv of kernel 4 over the channel's history and
 * silu: conv_out[c] = silu(sum_j conv_w[c*4 + j] * [tail; row][tail_len - 3
 * + j]) (rows before the history count as absent), and the history tail
 * [3][n_rows[0]] (tail_len rows valid) is moved on by one row in place
 * (min(3, tail_len + 1) rows valid after). It replaces the projections
 * (src/ssm.cpp:289-315) and the conv (:297-301) of aero_ssm_forward_q, as
 * aero_hip_norm_matvec followed by aero_hip_ssm_conv_silu; y[0] is not
 * written. conv_out and tail must overlap neither each other nor x, the
 * weights, conv_w or y[1..] (refused otherwise). */
int aero_hip_ssm_proj_conv(int dtype, int n_mat, const uint8_t* const* w, const int64_t* w_bytes,
                           const int64_t* n_rows, float* const* y, const float* x,
                           int64_t n_cols, const float* conv_w, float* tail, int64_t tail_len,
                           float* conv_out, void* stream);
/* The gated-DeltaNet norm folded into the next projection's GEMV:
 * y[t*n_rows + r] = sum_c W[r, c] * on[t, c], with
 * on[t, c] = x[t, c] / sqrt(mean_c x[t]^2 + eps) * norm_w[c % w_len] * silu(z[t, c])
 * over the whole row, as aero_hip_gated_rmsnorm_silu with group = n_cols. It
 * replaces the gated norm (src/ssm.cpp:322-340) and the output projection
 * (:343-348) of aero_ssm_forward_q for up to 2 tokens (decode); w_len a
 * multiple of 16 that divides n_cols; x, z, norm_w 16-byte aligned; weights as
 * aero_hip_norm_matvec. Equals that composition to 1e-5 of scale. */
int aero_hip_gated_norm_matvec(int dtype, const uint8_t* w, int64_t w_bytes, int64_t n_rows,
                               float* y, const float* x, const float* z, const float* norm_w,
                               int64_t w_len, float eps, int64_t n_cols, int64_t n_tok,
                               void* stream);
/* The same for any token count, with the workspace of aero_hip_norm_matmul
 * (aero_hip_norm_matmul_workspace(dtype, n_cols, 0, n_tok) plus
 * aero_hip_split_partials_bytes(n_rows, n_cols, n_tok)): up to 2 tokens the
 * fused GEMV above; on the split GEMM's path (aero_hip_matmul's types, from 5-16 tokens by
 * matrix size) the gated norm in its x pre-pass, the inverse RMS in its
 * epilogue; otherwise the gated norm into the workspace, then the projection. */
int aero_hip_gated_norm_matmul(int dtype, const uint8_t* w, int64_t w_bytes, int64_t n_rows,
                               float* y, const float* x, const float* z, const float* norm_w,
                               int64_t w_len, float eps, int64_t n_cols, int64_t n_tok,
                               void* ws, int64_t ws_bytes, void* stream);

int64_t aero_hip_matmul_workspace(int dtype, int64_t n_cols, int64_t n_tok);
int aero_hip_matmul(int dtype, const uint8_t* w, int64_t w_bytes, const float* x,
                    float* y, int64_t n_rows, int64_t n_cols, int64_t n_tok,
                    void* ws, int64_t ws_bytes, void* stream);

/* Prefill forms of the decode steps above, any token count: one pass that
 * folds the residual add and the RMSNorm into the GEMM's x pre-pass, then
 * the projections. The reference runs these as separate passes: `x_ +=
 * o_`, norm_row (src/model.cpp:244-245,279-282), matmul per matrix
 * (src/kernels.cpp:520-538) and act-mul (src/model.cpp:172-175). x is
 * [n_tok, n_cols] fp32; with d != NULL, x' = x + d is the residual stream
 * and is stored to x_out (may alias x or d), else x' = x. h = x' normalised
 * as aero_hip_rmsnorm (weight norm_w, NULL = ones; flags `norm` 0 or
 * AERO_NORM_UNIT_OFFSET; norm < 0: h = x').
 *   aero_hip_norm_matmul: y[m][t*n_rows[m] + r] = W_m[r] . h[t] for up to 4
 *     matrices of one type and width (q, k, v);
 *   aero_hip_norm_matmul_gate_up: out[t*n_ff + r] = act(Wg[r] . h[t]) *
 *     (Wu[r] . h[t]), act an AERO_ACT_* kind.
 * The split GEMM's types (aero_hip_matmul) with enough tokens (5 when the
 * call's matrices hold 32M+ weights together (4 for rows of more than 4096
 * columns), 7 for 8M+, 10 for 2M+, else 16; weights 16-byte
 * aligned) run the
 * split-x fp16 GEMM with h never written: each token's sums are scaled by
 * its 1/sqrt(mean(x'^2)+eps) and act(gate)*up is formed in the GEMM
 * epilogue. Fewer tokens, with rows the fused decode GEMVs take (above), run the fused
 * decode GEMVs, every matrix (or gate/up with the act-mul) in one launch: at
 * one token (two without d) with the add and the norm in their prologue
 * (x_out then must overlap neither x nor d; otherwise the add + norm pass
 * runs first). Other types and shapes run add+norm into the workspace, the
 * library GEMM per matrix and the act-mul. Each result equals that
 * composition to 1e-5 of its scale. ws (16-byte aligned) of at least
 * aero_hip_norm_matmul_workspace(dtype, n_cols, n_ff (0 for the plain
 * form), n_tok) bytes, sized for 16-byte aligned weights (weights that are
 * not take the separate launches, and a call whose workspace is too small
 * for them is refused with the size needed); x, d, x_out, norm_w 16-byte
 * aligned; h, y and out must not overlap x, d or x_out. */
int64_t aero_hip_norm_matmul_workspace(int dtype, int64_t n_cols, int64_t n_ff, int64_t n_tok);

/* Extra workspace bytes that let a split-path call of few tokens split its
 * columns over more workgroups: n_rows is the call's rows in all (every
 * matrix; gate/up: both), n_cols its columns. A workspace of
 * aero_hip_matmul_workspace / aero_hip_norm_matmul_workspace plus this
 * many bytes lets the call write each split's partial sums there and add
 * them in a second launch (in split order: deterministic); with less it
 * runs unsplit. 0 when the call would not split. No counterpart in the
 * reference, whose matmul runs on the CPU. */
int64_t aero_hip_split_partials_bytes(int64_t n_rows, int64_t n_cols, int64_t n_tok);
/* 1 when a matmul (or norm_matmul) of n_tok tokens over n_rows rows (all
 * matrices together) of n_cols columns of `dtype` takes the split-x fp16
 * GEMM, whose pre-pass folds a residual add and an RMSNorm, given 16-byte
 * aligned pointers and the workspace; 0 when it runs as separate launches.
 * Lets a model loop decide whether to fold its norm into the projection
 * from the library's own rule. No counterpart in the reference. */
int aero_hip_split_ok(int dtype, int64_t n_cols, int64_t n_rows, int64_t n_tok);
int aero_hip_norm_matmul(int dtype, int n_mat, const uint8_t* const* w, const int64_t* w_bytes,
                         const int64_t* n_rows, float* const* y, const float* x, const float* d,
                         float* x_out, const float* norm_w, float eps, int norm, int64_t n_cols,
                         int64_t n_tok, void* ws, int64_t ws_bytes, void* stream);
int aero_hip_norm_matmul_gate_up(int dtype, const uint8_t* w_gate, const uint8_t* w_up,
                                 int64_t w_bytes, const float* x, const float* d, float* x_out,
                                 const float* norm_w, float eps, int norm, int act, float* out,
                                 int64_t n_ff, int64_t n_cols, int64_t n_tok, void* ws,
                                 int64_t ws_bytes, void* stream);

/* aero_hip_norm_matmul, then RoPE on the outputs of its first n_rope (1 or
 * 2) matrices, q [n_tok, n_rows[0]] and k [n_tok, n_rows[1]] as heads of
 * head_dim rows: every channel rotated (n_rot = head_dim) at positions pos
 * [n_tok] with inv_freq [head_dim/2], mode AERO_ROPE_NEOX or
 * AERO_ROPE_INTERLEAVED. That is the projection and rotation of
 * src/attention_layer.cpp:60-156 without the per-head norms, and equals
 * aero_hip_norm_matmul followed by aero_hip_qk_norm_rope (no norm weights,
 * n_rot = head_dim). When the call takes the fused decode GEMV (below 32
 * tokens; NeoX heads a multiple of 16 rows) the rotation runs in its
 * epilogue: the partner rows of a pair are computed by the same workgroup
 * and meet in LDS. When it takes the split GEMM with workgroups of whole
 * heads (head_dim 16-128) the rotation runs in that GEMM's epilogue.
 * Otherwise the RoPE pass follows the projections. */
int aero_hip_norm_matmul_rope(int dtype, int n_mat, const uint8_t* const* w,
                              const int64_t* w_bytes, const int64_t* n_rows, float* const* y,
                              const float* x, const float* d, float* x_out, const float* norm_w,
                              float eps, int norm, int64_t n_cols, int64_t n_tok, int n_rope,
                              int64_t head_dim, int rope_mode, const int32_t* pos,
                              const float* inv_freq, void* ws, int64_t ws_bytes, void* stream);

/* The attention sublayer's input in one call, the steps of
 * src/model.cpp:244-245,297-316 and src/attention_layer.cpp:60-156:
 *   1. x' = the embedding rows of ids (ggml type emb_type, emb_bytes of
 *      table, times emb_scale when > 0) when emb is set, else x + d (d NULL:
 *      x); x' is stored to x_out (required with emb or d);
 *   2. h = rmsnorm(x') * norm_w (norm: -1 none, else 0 / AERO_NORM_UNIT_OFFSET);
 *   3. y[m] = h W_m^T for the n_mat (1-4) matrices of one type sharing h;
 *   4. on the first n_rope (0-2) outputs, q and k as heads of head_dim rows:
 *      the per-head RMSNorm (q_norm_w / k_norm_w [head_dim], NULL: none;
 *      qk_eps, qk_flags 0 / AERO_NORM_UNIT_OFFSET), then RoPE on the first
 *      n_rot channels (0: none) at positions pos [n_tok], inv_freq
 *      [n_rot/2], mode AERO_ROPE_NEOX / AERO_ROPE_INTERLEAVED.
 * Results equal aero_hip_embed_rmsnorm (or aero_hip_add_rmsnorm), the
 * projections and aero_hip_qk_norm_rope to fp32 re-association. With the
 * split GEMM (aero_hip_split_ok) the embedding rows are dequantised in its
 * x pre-pass (Q8_0, Q4_K, Q5_K, Q6_K, IQ4_XS tables; bit-identical to the
 * gather; an id outside the vocabulary gives a zero row) and, for
 * workgroups of whole heads (head_dim 16-128), step 4 runs in the GEMM's
 * epilogue: one pre-pass and one GEMM launch for all four steps. Otherwise
 * the steps take the gather + norm pass, the projections and the per-head
 * pass. Workspace: as aero_hip_norm_matmul. Plain C struct, no padding
 * assumptions beyond the platform ABI. */
typedef struct aero_attn_input {
    int dtype;
    int n_mat;
    const uint8_t* const* w;
    const int64_t* w_bytes;
    const int64_t* n_rows;
    float* const* y;
    int64_t n_cols;
    int64_t n_tok;
    const float* x;
    const float* d;
    float* x_out;
    int emb_type;
    const uint8_t* emb;
    int64_t emb_bytes;
    int64_t vocab;
    const int32_t* ids;
    float emb_scale;
    const float* norm_w;
    float eps;
    int norm;
    int n_rope;
    int64_t head_dim;
    int64_t n_rot;
    int rope_mode;
    const int32_t* pos;
    const float* inv_freq;
    const float* q_norm_w;
    const float* k_norm_w;
    float qk_eps;
    int qk_flags;
} aero_attn_input_t;
int aero_hip_attn_input(const aero_attn_input_t* a, void* ws, int64_t ws_bytes, void* stream);

/* aero_hip_matmul without a workspace argument and without allocating: the
 * split-x GEMM's workspace is a device array inside the library, of
 * aero_hip_matmul_noalloc_max_bytes() (32 MiB) a GPU, held by each GPU the
 * library runs on until the process ends. No counterpart in the reference:
 * it is for callers that cannot call hipMalloc (code under HIP graph
 * capture, serving loops, harnesses that forbid allocation). Results equal
 * aero_hip_matmul's with a workspace of aero_hip_matmul_workspace +
 * aero_hip_split_partials_bytes bytes bit for bit (the array is the call's
 * room, column-split partials included). Returns 0 with a reason when the
 * call would need more scratch than the maximum (n_tok * n_cols * 4 bytes
 * and a little more for the split path's types). Every call on one GPU
 * shares that GPU's array: calls ordered on one stream are safe; an eager
 * call on another stream while the last call may still run is refused
 * (0, "another stream"); calls recorded into a plan or captured into a HIP
 * graph are not checked, and such calls that overlap on one GPU race.
 * Nothing in the array needs clearing between calls. */
int aero_hip_matmul_noalloc(int dtype, const uint8_t* w, int64_t w_bytes, const float* x,
                            float* y, int64_t n_rows, int64_t n_cols, int64_t n_tok,
                            void* stream);
int64_t aero_hip_matmul_noalloc_max_bytes(void);

/* Attention over a KV cache, the device form of aero_attention_tiled
 * (src/transformer.cpp:120-214): q [n_q, n_head, head_dim] fp32; K / V
 * [n_kv, n_head_kv, dim] in kv_dt (0 fp32, 16-byte aligned, dims a multiple
 * of 4; 1 int8 or 2 int4 with one fp32 scale per (position, head) vector in
 * k_scale / v_scale, read as the reference's aero_kv_read_vec); out
 * [n_q, n_head, value_dim]. head_dim, value_dim <= 256. Decode shapes split
 * the keys into chunks whose partial softmax states go to `workspace`
 * (aero_hip_attention_workspace bytes; 0 when one chunk suffices). */
int64_t aero_hip_attention_workspace(int64_t n_q, int64_t n_head, int64_t n_head_kv,
                                     int64_t head_dim, int64_t value_dim, int64_t n_kv);
int aero_hip_attention(const float* q, int kv_dt, const void* k, const float* k_scale,
                       const void* v, const float* v_scale, float* out, int64_t n_q,
                       int64_t n_head, int64_t n_head_kv, int64_t head_dim, int64_t value_dim,
                       float scale, const int32_t* qpos, const int32_t* kpos, int64_t n_kv,
                       int window, void* workspace, int64_t ws_bytes, void* stream);
/* Append to a KV cache slot (include/aero/kv.hpp:62-126, src/kv.cpp:13-26):
 * row (t, h) of x [n_tok, heads, dim] is quantised (dt 0 fp32, 1 int8, 2
 * int4) into vector ((phys0 + t) % cap) * heads + h of the slot q (and its
 * scale), so a ring slot wraps. */
int aero_hip_kv_write(int dt, const float* x, int64_t n_tok, int64_t heads, int64_t dim,
                      int64_t phys0, int64_t cap, void* q, float* scale, void* stream);
/* Row softmax (src/tensor.cpp:167-178): y[r] = softmax(x[r]); y may alias x. */
int aero_hip_softmax_rows(const float* x, float* y, int64_t n_rows, int64_t n_cols,
                          void* stream);

/* Plain fp32 copy kernel (dst = src, n elements): the known-size reference
 * workload used to calibrate HBM byte counters. */
int aero_hip_copy_f32(const float* src, float* dst, int64_t n, void* stream);
/* Store-only fill (dst[i] = value, n % 4 == 0, 16-byte aligned): the
 * write-only streaming ceiling, beside the copy's read + write one. No
 * counterpart in the reference (measurement only). */
int aero_hip_fill_f32(float* dst, float value, int64_t n, void* stream);

/* ------------------------------------------------------------------------
 * 3. Runtime helpers
 * ---------------------------------------------------------------------- */
const char* aero_hip_last_error(void);  /* thread-local, "" when none       */
const char* aero_hip_version(void);
int   aero_hip_device_count(void);      /* 0 when no GPU / no driver        */
int   aero_hip_set_device(int device);
void* aero_hip_malloc(int64_t bytes);   /* NULL on failure                  */
int   aero_hip_free(void* p);
int   aero_hip_memcpy_htod(void* dst, const void* src, int64_t bytes);
int   aero_hip_memcpy_dtoh(void* dst, const void* src, int64_t bytes);
int   aero_hip_memcpy_dtod(void* dst, const void* src, int64_t bytes,
                           void* stream);
int   aero_hip_memset(void* dst, int value, int64_t bytes);  /* synchronous */
/* Launch-shape knob override for sweeps (the AERO_HIP_TUNE keys, e.g.
 * "norm_loop", "act_bs"): sets `key` to `value`, or drops it when `erase` is
 * nonzero so the built-in default applies again. Plans keep the kernel
 * choice they recorded. No counterpart in the reference (tuning only). */
int   aero_hip_tune_set(const char* key, int value, int erase);
void* aero_hip_stream_create(void);     /* default priority                 */
int   aero_hip_stream_destroy(void* stream);
int   aero_hip_stream_synchronize(void* stream);
int   aero_hip_device_synchronize(void);
void* aero_hip_event_create(void);
int   aero_hip_event_destroy(void* ev);
int   aero_hip_event_record(void* ev, void* stream);
int   aero_hip_event_synchronize(void* ev);
/* Milliseconds between two recorded events; negative on error. */
float aero_hip_event_elapsed_ms(void* start, void* stop);
/* Plans: record a sequence of aero_hip_* device ops once, replay it many
 * times. Between plan_begin and plan_end on one thread, every aero_hip_*
 * device op is checked and resolved to its kernel and launch shape as usual
 * but recorded (with its pointer and size arguments) instead of launched;
 * plan_launch then issues the recorded kernels in order on `stream` with no
 * per-op host work. starts / stops (nullable) are arrays of plan_size()
 * events: entry i then records the device begin/end of its own kernel.
 * The recorded buffers must stay allocated while the plan is used. */
void*   aero_hip_plan_create(void);
int     aero_hip_plan_begin(void* plan);
int     aero_hip_plan_end(void* plan);
int64_t aero_hip_plan_size(void* plan);
int     aero_hip_plan_launch(void* plan, void* stream, void** starts, void** stops);
int     aero_hip_plan_destroy(void* plan);

/* Arm per-kernel timing: the next kernel this thread launches through any
 * aero_hip_* op records `start` when it begins and `stop` when it ends on the
 * device (hipExtLaunchKernel), then the arming is cleared. */
int   aero_hip_time_next_kernel(void* start, void* stop);

/* ------------------------------------------------------- gated DeltaNet
 * The delta-rule scan and causal conv of src/ssm.cpp:17-210 (engine/ssm.py
 * recurrence). Per token t and value head h (key head h % n_k): qn, kn =
 * q, k / max(||.||, eps); dec = exp(min(a_log[h] * softplus(alpha + dt_bias),
 * 0)); b = sigmoid(beta); S_h = dec S_h; v_new = (v - kn^T S_h) b;
 * S_h += kn v_new^T; out = scale qn^T S_h. state [n_v][d][d] (row = key
 * element) is updated in place. */

/* Reference-compatible host ABI (host arrays, synchronous). The void
 * entries leave their outputs unwritten and set aero_hip_last_error() when
 * they refuse (sizes, null pointers, head dim not in {64, 128, 256}). */
float aero_ssm_softplus(float x);                                   /* src/ssm.cpp:151 */
void  aero_ssm_delta_step(const float* q, const float* k, const float* v,
                          const float* alpha, const float* beta, const float* a_log,
                          const float* dt_bias, float* state, int n_heads, int d,
                          float scale, float eps, float* out);       /* src/ssm.cpp:153-161 */
void  aero_ssm_scan(const float* qh, const float* kh, const float* vh, const float* alpha,
                    const float* beta, const float* a_log, const float* dt_bias,
                    float* state, int T, int n_k, int n_v, int d, float scale, float eps,
                    float* outs);                                    /* src/ssm.cpp:163-171 */
void  aero_ssm_conv(const float* x, const float* w, float* tail, int* tail_len, float* out,
                    int T, int channels, int kernel);                /* src/ssm.cpp:173-210 */

/* Device ABI. q, k [T][n_k][d]; v, outs [T][n_v][d]; alpha, beta [T][n_v];
 * a_log, dt_bias [n_v]; state [n_v][d][d]; d in {64, 128, 256}; q, k, state
 * and workspace 16-byte aligned; workspace of aero_hip_ssm_workspace bytes
 * (normalised q / k and the per-token decay and gate; from 128 tokens also
 * the chunked form's per-chunk operands, about (2 n_v + n_k) T d + n_v T 64
 * floats, plus n_k T d at d = 64 and 256; v and outs then 16-byte aligned
 * too). */
int64_t aero_hip_ssm_workspace(int64_t T, int64_t n_k, int64_t n_v, int64_t d);
int     aero_hip_ssm_scan(const float* q, const float* k, const float* v, const float* alpha,
                          const float* beta, const float* a_log, const float* dt_bias,
                          float* state, int64_t T, int64_t n_k, int64_t n_v, int64_t d,
                          float scale, float eps, float* outs, void* workspace,
                          int64_t ws_bytes, void* stream);
/* Causal depthwise conv: x, out [T][channels], w [channels][kernel] (tap 0
 * the oldest input), tail [tail_len][channels] of history (tail_len <
 * kernel <= 16); the new history (the last min(kernel-1, tail_len+T) rows of
 * [tail; x]) goes to tail_out, which may be tail, and its length to
 * *new_tail_len (host). */
int     aero_hip_ssm_conv(const float* x, const float* w, const float* tail, int64_t tail_len,
                          float* tail_out, float* out, int64_t T, int64_t channels,
                          int64_t kernel, int64_t* new_tail_len, void* stream);
/* The scan over q, k, v token rows q_stride, k_stride, v_stride floats apart
 * (each a multiple of 4, at least the token's heads): slices of one packed
 * [T][qkv] buffer, as the SSM layer scans them. Replaces scan_strided
 * (src/ssm.cpp:128-142) as aero_ssm_forward_q calls it (:316-320); same
 * workspace and alignment as aero_hip_ssm_scan. */
int     aero_hip_ssm_scan_strided(const float* q, int64_t q_stride, const float* k,
                                  int64_t k_stride, const float* v, int64_t v_stride,
                                  const float* alpha, const float* beta, const float* a_log,
                                  const float* dt_bias, float* state, int64_t T, int64_t n_k,
                                  int64_t n_v, int64_t d, float scale, float eps, float* outs,
                                  void* workspace, int64_t ws_bytes, void* stream);
/* aero_hip_ssm_conv with silu(x) = x / (1 + exp(-x)) applied to every output:
 * the conv then silu of aero_ssm_forward_q (src/ssm.cpp:298-301) in one pass. */
int     aero_hip_ssm_conv_silu(const float* x, const float* w, const float* tail,
                               int64_t tail_len, float* tail_out, float* out, int64_t T,
                               int64_t channels, int64_t kernel, int64_t* new_tail_len,
                               void* stream);

/* ---------------------------------------------------------------- GGUF
 * A GGUF file parsed on the host (src/gguf.cpp:150-354, the reference's
 * GgufReader; engine/gguf.py:166-233, GGUFReader._parse_index) and its tensors
 * uploaded to HBM. The file is mapped read-only; header, metadata and tensor
 * index are parsed with bounds checks. Handles are not thread-safe. */

/* Open and parse (GgufReader::GgufReader, src/gguf.cpp:150-168). NULL with
 * aero_hip_last_error() for a missing or unreadable file, bad magic, a
 * version other than 2 or 3, a truncated header, metadata or index, an
 * unknown metadata type, a general.alignment that is not a power of two,
 * n_dims > 4, an element count that is not whole blocks, or tensor data past
 * the end of the file (src/gguf.cpp:173-275). */
void*       aero_gguf_open(const char* path);
void        aero_gguf_close(void* h);                   /* GgufReader::~GgufReader */
int64_t     aero_gguf_file_size(void* h);               /* GgufReader::file_size */
int         aero_gguf_version(void* h);                 /* GGUFReader.version */
int64_t     aero_gguf_alignment(void* h);               /* GGUFReader.alignment */
int64_t     aero_gguf_data_offset(void* h);             /* GGUFReader.data_offset */
const char* aero_gguf_arch(void* h);                    /* GgufReader::arch */

/* Metadata in file order: n_kv keys; each value's GGUF type (0 u8 ... 12 f64,
 * -1 absent). Lookups take a key verbatim or, as the reference's C++ reader,
 * the part after its first dot unless the key starts with "tokenizer" or
 * "general." (the first entry for a name wins; src/gguf.cpp:205-218). */
int64_t     aero_gguf_n_kv(void* h);
const char* aero_gguf_kv_key(void* h, int64_t i);
int         aero_gguf_kv_type(void* h, const char* key);                  /* has :284 */
int         aero_gguf_get_int(void* h, const char* key, int64_t* out);    /* get_int :286-294 */
int         aero_gguf_get_float(void* h, const char* key, double* out);   /* get_float :296-304 */
const char* aero_gguf_get_str(void* h, const char* key, int64_t* len);    /* get_str :306-310 */
int64_t     aero_gguf_array_len(void* h, const char* key);
int64_t     aero_gguf_array_ints(void* h, const char* key, int64_t* out, int64_t n);   /* get_int_array :312-316 */
int64_t     aero_gguf_array_floats(void* h, const char* key, double* out, int64_t n);
const char* aero_gguf_array_str(void* h, const char* key, int64_t i, int64_t* len); /* get_str_array :318-322 */
/* Every metadata entry as JSON, [[key, type, value], ...] in file order (bytes
 * >= 0x80 of strings as \u00XX, one code point per byte): the metadata dict of
 * GGUFReader.kv (engine/gguf.py:186-198) in one call. Valid until close. */
const char* aero_gguf_kv_json(void* h, int64_t* len);

/* Tensor index (GgufReader::tensors / find, src/gguf.cpp:223-275,336-345): the
 * tensor's ggml type, dims in GGUF order (fastest first, unused = 0), offset
 * in the data section and size in bytes (-1 for a type whose block size is
 * not known). Returns the tensor's index, -1 if absent. */
int64_t     aero_gguf_n_tensors(void* h);
const char* aero_gguf_tensor_name(void* h, int64_t i);
int64_t     aero_gguf_tensor_info(void* h, const char* name, int* type, int* n_dims,
                                  int64_t* dims, int64_t* offset, int64_t* nbytes);
/* Host pointer to a tensor's bytes in the mapping (GgufReader::tensor_data,
 * src/gguf.cpp:347-349). */
const void* aero_gguf_tensor_data(void* h, const char* name);
/* Copy bytes [byte0, byte0+nbytes) of a tensor to host memory
 * (GGUFReader.tensor_bytes / _pread, engine/gguf.py:145-164,232-237). */
int         aero_gguf_read(void* h, const char* name, int64_t byte0, int64_t nbytes, void* dst);
/* Copy bytes [byte0, byte0+nbytes) of a tensor to device memory dst_dev on
 * `stream`: four threads pread 8 MiB chunks into pinned host buffers (two
 * per thread, 64 MiB, allocated on the handle's first upload) and queue each
 * chunk's host-to-device copy while reading the next. Returns once the bytes
 * are in HBM. No reference counterpart: the reference reads tensors into host
 * memory only. */
int         aero_gguf_upload(void* h, const char* name, int64_t byte0, int64_t nbytes,
                             void* dst_dev, void* stream);

#ifdef __cplusplus
}
#endif
#endif /* AERO_HIP_H */
