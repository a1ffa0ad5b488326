/*
 * kv-compact accelerator plug-in ABI (reference: include/kv-compact-accel.h).
 *
 * The reference routes two GEMMs of its CPU path through these five
 * symbols (rocBLAS strided-batched SGEMM in src/kv-compact-hip.hip). This
 * library exports the same symbols, implemented on its own HIP kernels with
 * the CPU path's sequential fp32 accumulation, so a build of the reference
 * orchestrator linked against this library gets bit-identical scores.
 * Pointers are host memory (the reference copies them through a managed
 * pool); the calls are thread-safe here. Return 0 on success, -1 when no
 * GPU is usable.
 */
#pragma once

#ifdef __cplusplus
extern "C" {
#endif

int kv_compact_hip_available(void);                              /* ref accel.h:22 */

/* C[m x n] = scale * A[m x k] * B[n x k]^T                          ref accel.h:24 */
int kv_compact_hip_mat_mul_ABt_scaled(const float * A, const float * B, float * C,
                                      int m, int n, int k, float scale);

/* scores_out[h][qi*T + ki] = scale * <Q_ref[qi, h, :], K_all[ki, h, :]>
 * Q_ref [n_q x H*d_k], K_all [T x H*d_k] interleaved; scores_out[h] host
 * buffers of n_q*T floats.                                          ref accel.h:38 */
int kv_compact_hip_score_all_heads(const float * Q_ref, const float * K_all, float ** scores_out,
                                   int n_q, int T, int n_head_kv, int d_k, float scale);

/* Y_out[h] [n_q x d_v] = W_per_head[h] [n_q x T] * V_h, V_all [T x H*d_v]  ref accel.h:50 */
int kv_compact_hip_refit_target_all_heads(const float * const * W_per_head, const float * V_all,
                                          float ** Y_out, int n_q, int T, int n_head_kv, int d_v);

void kv_compact_hip_pool_free(void);                              /* ref accel.h:55 */

#ifdef __cplusplus
}
#endif
