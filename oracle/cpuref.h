/* oracle/cpuref.h -- CPU restatement of Aero's fused per-layer elementwise path.
 *
 * TEST INFRASTRUCTURE. This library checks the product and is never part of it: only
 * tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may load it.
 * The GPU path in aero_amd/ never calls it and has no CPU fallback.
 *
 * Every function restates the reference algorithm in plain C, in the
 * reference's fp32 operation order, and cites the file:line it follows
 * (paths relative to the BattleCrusader/aero tree). See cpuref.c for how each
 * function's parity is pinned.
 */
#ifndef AERO_CPUREF_H
#define AERO_CPUREF_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ggml type ids (include/aero/kernels.hpp:40-49) */
enum {
    CR_F32 = 0, CR_F16 = 1, CR_Q8_0 = 8, CR_Q4_K = 12, CR_Q5_K = 13,
    CR_Q6_K = 14, CR_IQ4_XS = 23, CR_BF16 = 30
};

/* ---- quant (cpuref_quant.c) ------------------------------------------- */
float   cr_f16_to_f32(uint16_t h);
void    cr_f16_to_f32_n(const uint16_t* h, float* out, int64_t n);
int64_t cr_block_bytes(int type);
int64_t cr_block_values(int type);
int     cr_dequant(int type, const uint8_t* raw, int64_t raw_len, float* out,
                   int64_t n_values);
int     cr_dequant_threaded(int type, const uint8_t* raw, int64_t raw_len,
                            float* out, int64_t n_values, int threads);
int     cr_matvec(int type, const uint8_t* w, const float* x, float* y,
                  int64_t n_rows, int64_t n_cols);
int     cr_matmul(int type, const uint8_t* w, const float* X, float* Y,
                  int64_t n_tok, int64_t n_rows, int64_t n_cols);
int     cr_embed_gather(int type, const uint8_t* table, int64_t vocab,
                        int64_t n_embd, const int32_t* ids, int64_t n_ids,
                        float scale, float* out);

/* ---- fp32 path (cpuref.c) --------------------------------------------- */
void cr_rmsnorm_rows(const float* x, const float* w, float* out, int64_t rows,
                     int64_t cols, float eps, int unit_offset);
void cr_l2norm_rows(const float* x, const float* w, float* out, int64_t rows,
                    int64_t cols, float eps);
void cr_gated_rmsnorm_silu(const float* x, const float* z, const float* w,
                           int64_t w_len, float* out, int64_t rows,
                           int64_t inner, int64_t group, float eps);

/* act kinds: 0 silu, 1 gelu (erf, A&S 7.1.26), 2 gelu (tanh), 3 identity */
void cr_act(int kind, float* v, int64_t n);
void cr_act_mul(int kind, const float* gate, const float* up, float* out,
                int64_t n);

int64_t cr_rope_inv_freq(int64_t head_dim, int64_t n_dims, float base,
                         const float* ff, int64_t n_ff, float* inv_out);
int64_t cr_rope_tables(int64_t head_dim, const int32_t* pos, int64_t n_pos,
                       float base, int64_t n_dims, const float* ff,
                       int64_t n_ff, float* cos_out, float* sin_out);
void    cr_apply_rope(float* x, int64_t n_rows, int64_t head_dim, int64_t n_rot,
                      const float* cos_tab, const float* sin_tab,
                      const int32_t* pos, int mode);

/* softmax, GQA attention (src/tensor.cpp:167-178, src/transformer.cpp:120-214) */
void cr_dense_matvec(const float* w, const float* x, float* y, int64_t n_rows, int64_t n_cols);
void cr_dense_matmul(const float* w, const float* x, float* y, int64_t n_tok, int64_t n_rows,
                     int64_t n_cols);
int cr_argmax(const float* v, int64_t n);
void cr_softmax(float* v, int64_t n);
void cr_softmax_rows(float* v, int64_t n_rows, int64_t n_cols);
int  cr_attention_tiled(const float* q, const float* k, const float* v, float* out, int64_t n_q,
                        int64_t n_head, int64_t n_head_kv, int64_t head_dim, int64_t value_dim,
                        float scale, const int32_t* qpos, const int32_t* kpos, int64_t n_kv,
                        int window, int64_t block);
int  cr_attention(const float* q, const float* k, const float* v, float* out, int64_t n_head,
                  int64_t n_head_kv, int64_t head_dim, int64_t value_dim, float scale,
                  int64_t n_kv, int window);

/* KV cache vectors (include/aero/kv.hpp:62-103, src/kv.cpp:13-46) */
void cr_kv_quant_i8(const float* x, int64_t dim, int8_t* q, float* s);
void cr_kv_quant_i4(const float* x, int64_t dim, uint8_t* q, float* s);
int  cr_kv_read_vec(int dt, const void* q, const float* scale, int64_t dim, float* out);
int  cr_kv_write_vec(int dt, const float* x, int64_t dim, void* q, float* scale);

/* gated DeltaNet (src/ssm.cpp:17-210) */
float cr_ssm_softplus(float x);
void  cr_ssm_delta_step_grouped(const float* q, const float* k, const float* v,
                                const float* alpha, const float* beta, const float* a_log,
                                const float* dt_bias, float* state, int64_t n_k, int64_t n_v,
                                int64_t d, float scale, float eps, float* out);
void  cr_ssm_scan(const float* q, const float* k, const float* v, const float* alpha,
                  const float* beta, const float* a_log, const float* dt_bias, float* state,
                  int64_t T, int64_t n_k, int64_t n_v, int64_t d, float scale, float eps,
                  float* outs);
void  cr_ssm_conv(const float* x, const float* w, float* tail, int* tail_len, float* out,
                  int64_t T, int64_t channels, int64_t kernel);

#ifdef __cplusplus
}
#endif
#endif
