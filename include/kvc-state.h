/* Compaction of a llama.cpp sequence state blob on MI355X.
 *
 * The reference's parsed_kv_state / build_compacted_state
 * (include/kv-compact-state.h:104-222, :645-810) are C++ header code driven
 * by its CLI (src/kv-compact.cpp:380-790): parse the blob written by
 * llama_state_seq_get_data, score every selected layer's heads with the last
 * n_ref keys as queries, take one top-t set of cells across all layers and
 * heads (max of the per-head importances, or the sensitivity-weighted sum),
 * refit each head's values by ridge least squares (beta = 0), compute each
 * head's beta direction, and write a blob of the t kept cells that
 * llama_state_seq_set_data accepts. This header exposes that sequence as one
 * C call over host or device memory; the work runs on the GPU.
 *
 * Blob layout (state.h:6-14):
 *   u32 n_stream; per stream: u32 cell_count; if cell_count > 0:
 *     per cell: i32 pos, u32 n_seq_id, [i32 x, i32 y when n_pos_per_embd > 1],
 *               i32 seq_id[n_seq_id]
 *     u32 v_trans, u32 n_layer
 *     per layer: i32 k_type, u64 k_size_row, cell_count rows of k_size_row bytes
 *     per layer, v_trans == 0: i32 v_type, u64 v_size_row, cell_count rows
 *     per layer, v_trans == 1: i32 v_type, u32 v_size_el, u32 n_embd_v_gqa,
 *               n_embd_v_gqa * cell_count * v_size_el bytes ([embd][cell])
 *   then any trailing bytes (e.g. a recurrent-state section), copied as is.
 *
 * Element types: F32 (0), F16 (1), Q4_0 (2), Q4_1 (3), Q8_0 (8) with the
 * reference's own codec (state.h:326-629).
 *
 * Scope of this build (each refusal returns KV_COMPACT_E_UNSUPPORTED = -5):
 *  - stream 0 is compacted; any other stream must be empty;
 *  - every layer has layer 0's K and V row widths (the reference reads every
 *    layer with layer 0's widths, src/kv-compact.cpp:403-404, :622);
 *  - other element types (the reference would zero them and write rows of no
 *    bytes, state.h:419, :628);
 *  - more than 8192 reference queries.
 */
#ifndef KVC_STATE_H
#define KVC_STATE_H

#include <stddef.h>
#include <stdint.h>

#include "kv-compact-api.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef struct kvc_state_params {
    float    compact_ratio;      /* t = max(1, (int)(cell_count * compact_ratio)), kv-compact.cpp:269 */
    int32_t  n_ref_queries;      /* <= 0: max(16, cell_count / 4); then min(., cell_count), kv-compact.cpp:274-277 */
    int32_t  n_head_kv;          /* heads per layer: d_k = n_embd_k / n_head_kv */
    uint32_t n_pos_per_embd;     /* 1, or > 1 for M-RoPE / IMROPE cells (x, y), state.h:104-130 */
    int32_t  sensitivity_budget; /* 1: sum over layers and heads of sens * importance, kv-compact.cpp:532-571 */
    kv_layer_filter_fn layer_filter;  /* NULL: every layer; layers it rejects keep their values */
    void *   layer_filter_data;
} kvc_state_params;

typedef struct kvc_state_info {
    uint32_t n_stream;
    uint32_t cell_count;         /* stream 0 */
    uint32_t v_trans;
    uint32_t n_layer;
    int32_t  n_embd_k;           /* layer 0 K row width in elements */
    int32_t  n_embd_v;           /* layer 0 V row width in elements */
    uint64_t kv_bytes;           /* bytes up to the end of the KV section */
    uint64_t trailing_bytes;     /* bytes after it */
} kvc_state_info;

/* Host-side parse of the blob's layout (parsed_kv_state::parse, state.h:104-222).
 * 0, or -1 (NULL), -2 (malformed or empty). */
int kvc_state_parse_info(const void * blob, size_t size, uint32_t n_pos_per_embd, kvc_state_info * info);

/* Host blob in, malloc'd host blob out (*out, freed by kvc_state_free).
 * selected (optional, [t]): kept cell indices, ascending.
 * 0; -1 NULL; -2 malformed / empty / bad parameters; -5 outside the scope
 * above; -6 device error. */
int kvc_state_compact(const void * blob, size_t size, const kvc_state_params * sp,
                      void ** out, size_t * out_size, int32_t * selected);

/* Device blob in, device blob out: d_out must hold out_cap bytes. When the
 * compacted blob is larger, returns KVC_E_CAPACITY (-8) with *out_size set
 * to the size needed and writes nothing. Ordered on `stream` (NULL: the
 * library's stream); returns after the output is complete. */
int kvc_state_compact_device(const void * d_blob, size_t size, const kvc_state_params * sp,
                             void * d_out, size_t out_cap, size_t * out_size, int32_t * selected,
                             void * stream);

void kvc_state_free(void * out);

#define KVC_E_CAPACITY (-8)

#ifdef __cplusplus
}
#endif

#endif
