/*
 * kv-compact C API — attention-matching KV-cache compaction on MI355X.
 *
 * Drop-in replacement for the reference library's public header
 * (reference: include/kv-compact-api.h). Every type, field, enum value and
 * function below keeps the reference's name, order, size and meaning so that
 * existing callers (C/C++ code, ctypes bindings) link and run unchanged.
 * Struct layouts on x86-64: kv_compact_params 104 B, kv_compact_reasoning
 * 32 B, kv_compact_stats 40 B, kv_compact_result 72 B,
 * kv_compact_quant_result 112 B.
 *
 * Data layout of one layer (row-major, heads concatenated per token):
 *   K_all     [T   x n_head_kv*d_k]
 *   V_all     [T   x n_head_kv*d_v]
 *   Q_ref_all [n_q x n_head_kv*d_k]
 * Inputs may be host or device (HBM) pointers; results are always host
 * memory obtained with malloc() and released with kv_compact_result_free().
 *
 * Return codes: 0 ok, -1 NULL argument, -2 bad dimension, -3 bad round
 * count, -4 quantized row size mismatch (all as the reference), and the
 * additional codes KV_COMPACT_E_UNSUPPORTED (-5: an option this library
 * does not implement on the GPU) and KV_COMPACT_E_DEVICE (-6: no usable
 * GPU, a HIP runtime failure, or a failed host allocation of the result).
 * There is no CPU fallback.
 */
#pragma once

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define KV_COMPACT_E_UNSUPPORTED (-5)
#define KV_COMPACT_E_DEVICE      (-6)

/* ---- layer filters (reference: include/kv-compact-api.h:51-87) ---------- */

typedef int (*kv_layer_filter_fn)(int layer_idx, int n_layers, void * user_data);

static inline int kv_layer_filter_all(int layer_idx, int n_layers, void * user_data) {
    (void)layer_idx; (void)n_layers; (void)user_data;
    return 1;
}

/* user_data carries the attention interval; layer i is kept when
 * (i + 1) is a multiple of it (interval <= 0 keeps every layer). */
static inline int kv_layer_filter_periodic(int layer_idx, int n_layers, void * user_data) {
    (void)n_layers;
    int every = (int)(intptr_t)user_data;
    if (every <= 0) return 1;
    return ((layer_idx + 1) % every) == 0 ? 1 : 0;
}

typedef struct kv_layer_list {
    const int * layers;   /* ascending layer indices */
    int         n_layers;
} kv_layer_list;

static inline int kv_layer_filter_explicit(int layer_idx, int n_layers, void * user_data) {
    (void)n_layers;
    const kv_layer_list * lst = (const kv_layer_list *)user_data;
    if (!lst || !lst->layers) return 1;
    for (int i = 0; i < lst->n_layers; i++) {
        if (lst->layers[i] == layer_idx) return 1;
        if (lst->layers[i] > layer_idx) break;
    }
    return 0;
}

/* ---- reasoning-aware weighting, R-KV (reference: api.h:98-127) ---------- */

typedef enum {
    KV_TOKEN_ANSWER     = 0,
    KV_TOKEN_THINKING   = 1,
    KV_TOKEN_TRANSITION = 2
} kv_token_type;

typedef int (*kv_token_classifier_fn)(int token_pos, void * user_data);

typedef struct kv_compact_reasoning {
    kv_token_classifier_fn classifier;       /* NULL disables weighting */
    void *                 classifier_data;
    float                  thinking_weight;   /* importance multiplier, THINKING */
    float                  transition_weight; /* importance multiplier, TRANSITION */
    int                    token_offset;      /* added to the position before classifying */
} kv_compact_reasoning;

/* ---- parameters (reference: api.h:133-215; defaults api.cpp:333-358) ---- */

typedef struct kv_compact_params {
    float target_ratio;        /* fraction kept (default 0.5) */
    int   target_count;        /* > 0 overrides target_ratio */
    int   use_sensitivity;     /* per-head sensitivity weighting (unsupported: -5) */
    float ridge;               /* ridge of the value refit (default 1e-6) */
    int   nnls_max_iter;       /* Lawson-Hanson iteration cap (default 200) */
    int   refine_rounds;       /* swap-worst-for-best rounds (default 0) */
    int   use_diversity;       /* cosine-diversity greedy selection */
    float diversity_strength;  /* default 0.5 */
    int   n_shared_prefix;     /* leading positions always kept */
    int   use_cheap_qref;      /* reference queries sampled from K */
    int   skip_beta;           /* beta = 0, no NNLS (default 1) */
    int   score_method;        /* 0 max, 1 RMS (default), 2 mean */
    int   use_omp;             /* OMP selection (unsupported: -5) */
    int   omp_k_choice;
    int   omp_refit_interval;
    int   nnls_method;         /* 0 Lawson-Hanson, 1 clamped LS (default) */
    int   nnls_pgd_iters;      /* > 0 unsupported: -5 */
    int   chunk_size;          /* 0 auto, -1 never, > 0 explicit */
    int   n_threads;           /* accepted; only affects host-side work */
    kv_layer_filter_fn     layer_filter;
    void *                 layer_filter_data;
    kv_compact_reasoning * reasoning;
} kv_compact_params;

/* ---- results (reference: api.h:221-241) --------------------------------- */

typedef struct kv_compact_stats {
    float  avg_cosine_sim;
    float  avg_mse;
    float  avg_agreement;
    double elapsed_ms;
    double scoring_ms;
    double nnls_ms;
} kv_compact_stats;

typedef struct kv_compact_result {
    int      t;
    int      n_head_kv;
    int *    selected_indices;  /* [t], ascending */
    float ** beta;              /* [n_head_kv][t] */
    float ** C_v;               /* [n_head_kv][t * d_v] */
    kv_compact_stats stats;
} kv_compact_result;

kv_compact_params kv_compact_params_default(void);          /* ref api.cpp:333 */

int kv_compact(const float * K_all, const float * V_all, const float * Q_ref_all,
               int T, int n_q, int n_head_kv, int d_k, int d_v,
               const kv_compact_params * params,
               kv_compact_result * result);                  /* ref api.cpp:360 */

int kv_compact_multi_round(const float * K_all, const float * V_all,
                           const float * Q_ref_all,
                           int T, int n_q, int n_head_kv, int d_k, int d_v,
                           const kv_compact_params * params, int n_rounds,
                           kv_compact_result * result,
                           kv_compact_stats * per_round_stats); /* ref api.cpp:980 */

void kv_compact_result_free(kv_compact_result * result);      /* ref api.cpp:1113 */

/* ---- quantized KV (reference: api.h:306-378; api.cpp:1150-1266) --------- */

typedef enum {
    KV_TYPE_F32  = 0,
    KV_TYPE_F16  = 1,
    KV_TYPE_Q4_0 = 2,
    KV_TYPE_Q4_1 = 3,
    KV_TYPE_Q8_0 = 8,
    /* Extension, no counterpart in the reference: bfloat16 rows (ggml's
     * value for the type). Decode is exact (the upper 16 bits of the float);
     * encode rounds to nearest, ties to even; NaN stays a quiet NaN. */
    KV_TYPE_BF16 = 30
} kv_data_type;

#define KV_COMPACT_BLOCK_SIZE 32

typedef struct kv_compact_quant_result {
    kv_compact_result base;
    int       k_type;
    int       v_type;
    uint8_t * K_out;        /* [t x k_row_bytes] */
    uint8_t * V_out;        /* [t x v_row_bytes] */
    size_t    k_row_bytes;
    size_t    v_row_bytes;
} kv_compact_quant_result;

int kv_compact_quantized(const uint8_t * K_quant, const uint8_t * V_quant,
                         const float * Q_ref_all, int k_type, int v_type,
                         size_t k_row_bytes, size_t v_row_bytes,
                         int T, int n_q, int n_head_kv, int d_k, int d_v,
                         const kv_compact_params * params,
                         kv_compact_quant_result * result);   /* ref api.cpp:1182 */

void kv_compact_quant_result_free(kv_compact_quant_result * result); /* ref api.cpp:1259 */

int    kv_dequantize_row(const uint8_t * src, int type, size_t row_bytes,
                         float * dst, int max_elements);       /* ref api.cpp:1169 */
size_t kv_quantize_row(const float * src, int type, int n_elements,
                       uint8_t * dst);                          /* ref api.cpp:1177 */
int    kv_quant_row_elements(int type, size_t row_bytes);       /* ref api.cpp:1155 */
size_t kv_quant_row_bytes(int type, int n_elements);            /* ref api.cpp:1159 */

static inline int kv_compact_count_layers(kv_layer_filter_fn filter,
                                          void * filter_data, int n_layers) {
    if (!filter) return n_layers;
    int n = 0;
    for (int l = 0; l < n_layers; l++) n += filter(l, n_layers, filter_data) ? 1 : 0;
    return n;
}

static inline int kv_compact_should_compact_layer(const kv_compact_params * params,
                                                  int layer_idx, int n_layers) {
    if (!params || !params->layer_filter) return 1;
    return params->layer_filter(layer_idx, n_layers, params->layer_filter_data);
}

#ifdef __cplusplus
}
#endif
