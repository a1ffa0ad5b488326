/*
 * CPU oracle for the attention-matching compaction path.
 *
 * TEST INFRASTRUCTURE ONLY. This is a plain-C restatement of the reference
 * CPU path (src/kv-compact-api.cpp, include/kv-compact-math.h,
 * include/kv-compact-state.h) that keeps the reference's fp32 operation
 * order, so that, compiled like the reference (-O3, no -march: no FMA
 * contraction) and linked against the same libm, it reproduces the
 * reference's outputs bit for bit. Only tests/, __graft_entry__.smoke() and
 * bench.py's cpu_baseline leg may load it, and only as the checker. The
 * product library never links or calls it.
 *
 * Pinning: every function here is checked bit-exactly against the compiled
 * reference (oracle/_ref) on the committed golden fixtures
 * (tests/golden fixtures) and, where mathematics fixes the answer, against
 * closed forms (see tests/test_oracle.py).
 */
#pragma once
#include <stddef.h>
#include <stdint.h>
#include "../include/kv-compact-api.h"
#include "../include/kvc-state.h"

#ifdef __cplusplus
extern "C" {
#endif

/* full entry points, same signatures and semantics as the reference ABI */
kv_compact_params orc_params_default(void);
int  orc_kv_compact(const float * K, const float * V, const float * Q,
                    int T, int n_q, int H, int d_k, int d_v,
                    const kv_compact_params * params, kv_compact_result * res);
int  orc_kv_compact_multi_round(const float * K, const float * V, const float * Q,
                                int T, int n_q, int H, int d_k, int d_v,
                                const kv_compact_params * params, int n_rounds,
                                kv_compact_result * res, kv_compact_stats * per_round);
void orc_result_free(kv_compact_result * res);
int  orc_kv_compact_quantized(const uint8_t * Kq, const uint8_t * Vq, const float * Q,
                              int k_type, int v_type, size_t k_rb, size_t v_rb,
                              int T, int n_q, int H, int d_k, int d_v,
                              const kv_compact_params * params,
                              kv_compact_quant_result * res);
void orc_quant_result_free(kv_compact_quant_result * res);

/* codec (reference include/kv-compact-state.h:326-629) */
float    orc_f16_to_f32(uint16_t h);
uint16_t orc_f32_to_f16(float f);
int      orc_quant_row_elements(int type, size_t row_bytes);
size_t   orc_quant_row_bytes(int type, int n_elements);
int      orc_dequantize_row(const uint8_t * src, int type, size_t row_bytes, float * dst, int max_el);
size_t   orc_quantize_row(const float * src, int type, int n, uint8_t * dst);

/* building blocks, exposed for known-answer tests */
float orc_expf_replica(float x);   /* glibc-expf algorithm restated (see .c) */
void  orc_scores(const float * Q, const float * K, float * S, int n_q, int T,
                 int d, int stride_q, int stride_k, float scale);
void  orc_mat_mul_AB(const float * A, const float * B, float * C, int m, int k, int n, int ldb);
void  orc_softmax_importance(const float * S, float * attn, float * imp,
                             float * exp_out, float * row_sums, int m, int n, int agg);
void  orc_softmax_rows(float * x, int m, int n);
int   orc_select_topk(const float * imp, int T, int t, int n_prefix, int * out_sorted);
int   orc_select_diverse(const float * imp, const float * K, int T, int t, int n_embd,
                         float strength, int n_prefix, int * out_sorted, int * out_order);
void  orc_ls_solve(const float * A, const float * b, float * x, int m, int n, int p, float ridge);
void  orc_nnls_lh(const float * A, const float * b, float * w, int m, int n, int max_iter);
void  orc_nnls_clamped(const float * A, const float * b, float * w, int m, int n, float eps);
void  orc_nnls_pgd(const float * A, const float * b, float * w, int m, int n, float eps, int iters);
float orc_head_sensitivity(const float * attn, int n_q, int T);
void  orc_omp_select(const float * E, const float * rs, int T, int n_q, int t, int * sel_out, float * w_out,
                     int k_choice, int refit_interval, int nnls_iters);
void  orc_quality_stats(const float * K, const float * V, const float * Q, int T, int n_q,
                        int H, int d_k, int d_v, const kv_compact_result * r,
                        kv_compact_stats * st);
/* chunk plan of one call: returns n_chunks and fills chunk size; t of chunk c
 * by orc_chunk_t(); exact float arithmetic of reference api.cpp:396-437 */
int   orc_chunk_plan(int T, const kv_compact_params * p, int * chunk_size_out);
int   orc_target_count(int T, const kv_compact_params * p);

/* llama.cpp state blob compaction (state.h:104-222, 645-810; kv-compact.cpp:380-690) */
int  orc_state_parse_info(const uint8_t * blob, size_t size, uint32_t n_pos_per_embd, kvc_state_info * info);
int  orc_state_compact(const uint8_t * blob, size_t size, const kvc_state_params * sp,
                       uint8_t ** out, size_t * out_size, int32_t * selected);
void orc_state_free(uint8_t * p);

#ifdef __cplusplus
}
#endif
