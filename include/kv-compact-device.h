/*
 * kv-compact device-resident batch API (MI355X). Additive to the reference
 * ABI (include/kv-compact-api.h): the reference has no counterpart; its
 * callers loop kv_compact() over layers with host buffers (reference
 * src/kv-compact.cpp:499-648, tests/bench-throughput-large.cpp:55-62).
 *
 * One call compacts L layers that share T, n_q, H, d_k, d_v and params.
 * All pointers are device (HBM) memory. Layer l of K is K + l*ldK (elements;
 * ldK >= T*H*d_k), likewise V/ldV and Q_ref/ldQ. Results, per layer l:
 *   indices + l*t_total              [t_total]          kept positions, ascending
 *   beta    + l*H*t_total            [H][t_total]
 *   C_v     + l*H*t_total*d_v        [H][t_total][d_v]
 *   stats   + 3*l                    avg_cosine_sim, avg_mse, avg_agreement
 * Each layer's results equal kv_compact() on that layer bit for bit.
 * token_weight (device float[T], may be NULL) holds the R-KV multiplier of
 * each position; when NULL and params->reasoning has a classifier, the
 * classifier is evaluated on the host. The call is synchronous with respect
 * to `stream` (NULL: the library's stream). Returns the kv_compact codes.
 */
#pragma once
#include "kv-compact-api.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef struct kvc_device_out {
    int   * indices;
    float * beta;
    float * C_v;
    float * stats;
} kvc_device_out;

/* Chunk plan of a call (same arithmetic as kv_compact): number of kept
 * tokens per layer and number of chunks. */
int kvc_plan(int T, int n_q, int q_ref_given, const kv_compact_params * params,
             int * t_total, int * n_chunks);

int kvc_compact_layers_device(const float * K, const float * V, const float * Q_ref,
                              int L, int T, int n_q, int n_head_kv, int d_k, int d_v,
                              long long ldK, long long ldV, long long ldQ,
                              const kv_compact_params * params, const float * token_weight,
                              kvc_device_out * out, void * stream);

/* Allocation-free variant of kvc_compact_layers_device (no counterpart in the
 * reference). For callers that cannot allocate device memory (tight serving
 * loops, harnesses that forbid hipMalloc): same
 * arguments, outputs and results bit for bit, but the workspace is a fixed
 * device array of KVC_NOALLOC_SCRATCH_BYTES per GPU that the library holds
 * from load until the process ends, and the call makes no hipMalloc/hipFree
 * (nor any other allocating library call). A call whose workspace exceeds the
 * array returns KVC_E_SCRATCH without launching anything. Every call on one
 * GPU uses that GPU's array and leaves its contents behind (each call writes
 * what it reads, and clears its status flag with a kernel): calls on one GPU
 * must not overlap — this library serializes its own calls per device, so
 * overlapping calls can only come from elsewhere (another copy of the library
 * in the process) and would race on the array. The call is not capturable
 * into a HIP graph: like kvc_compact_layers_device it synchronizes its
 * stream and copies a status word to the host before it returns. */
#define KVC_NOALLOC_SCRATCH_BYTES (64u << 20)
#define KVC_E_SCRATCH (-7)
int kvc_compact_layers_device_noalloc(const float * K, const float * V, const float * Q_ref,
                                      int L, int T, int n_q, int n_head_kv, int d_k, int d_v,
                                      long long ldK, long long ldV, long long ldQ,
                                      const kv_compact_params * params, const float * token_weight,
                                      kvc_device_out * out, void * stream);

/* Device-resident quantized pipeline (reference api.cpp:1182-1257 for each
 * layer): L layers of K/V rows in the given codecs (device; layer l of K at
 * K_quant + l * ldKq bytes, likewise V; Q_ref layers ldQ floats apart) are
 * dequantized into the library's workspace, compacted as by
 * kvc_compact_layers_device, and the kept K rows and refitted V rows
 * requantized into K_out / V_out (device, [L][t_total][row bytes]); indices,
 * beta, C_v and stats as above. Each layer's outputs equal
 * kv_compact_quantized() on that layer bit for bit. */
int kvc_compact_quantized_layers_device(const uint8_t * K_quant, const uint8_t * V_quant, const float * Q_ref,
                                        int L, int k_type, int v_type, size_t k_row_bytes, size_t v_row_bytes,
                                        int T, int n_q, int n_head_kv, int d_k, int d_v,
                                        long long ldKq, long long ldVq, long long ldQ,
                                        const kv_compact_params * params, kvc_device_out * out,
                                        uint8_t * K_out, uint8_t * V_out, void * stream);

/* The same for one layer (L = 1). */
int kvc_compact_quantized_device(const uint8_t * K_quant, const uint8_t * V_quant, const float * Q_ref,
                                 int k_type, int v_type, size_t k_row_bytes, size_t v_row_bytes,
                                 int T, int n_q, int n_head_kv, int d_k, int d_v,
                                 const kv_compact_params * params, kvc_device_out * out,
                                 uint8_t * K_out, uint8_t * V_out, void * stream);

/* Device time in ms of each pipeline stage of the last call on the current
 * device, measured with HIP events on that call's stream. Stages, in order:
 * 0 scores, 1 chunk softmax + importance, 2 refit target Y = A V,
 * 3 selection, 4 beta fit, 5 compacted softmax X, 6 normal equations,
 * 7 LU elimination with partial pivoting, 8 forward + back substitution,
 * 9 refinement rounds, 10 quality statistics, and for the quantized entries
 * 11 dequantization of the K and V rows, 12 requantization of the kept K
 * rows and refitted V rows (0 after an unquantized call). After a call that
 * took the fused scoring kernel (KVC_FUSED=1), stage 0 is that kernel and
 * stages 1 and 2 read 0. Returns the number written. */
int kvc_stage_times(float * out_ms, int n);

/* Release the library's cached device workspace of the current device, and
 * its pinned host ring for transfers from and to pageable host memory (both
 * are allocated again by the next call that needs them). */
void kvc_release_workspace(void);

/* Number of HIP streams, events and pinned host buffers the library holds,
 * over all devices (no counterpart in the reference). It stays constant
 * across calls once the library is set up, including calls that fail part
 * of the way through a set-up; a test of the error paths reads it. */
int kvc_live_objects(void);

#ifdef __cplusplus
}
#endif
