// Host-side launch wrappers for the kernels in kvc_kernels.hip.
#pragma once
#include "kvc_common.h"

namespace kvc {

hipError_t set_exp2_table(const uint64_t * tab32);

void launch_scores(const Geom & g, const ChunkDesc * chunks, int n_chunk_units, int Tc_max,
                   const float * K, const float * Q, float * S, int Hs, int nq_cap,
                   long long s_layer, long long s_head, long long s_row, int qmode, hipStream_t st,
                   const int * key_idx = nullptr, const float * beta = nullptr, unsigned * tmax = nullptr);
void launch_chunk_softmax(const Geom & g, const Work & w, hipStream_t st);
void launch_refit_target(const Geom & g, const Work & w, const float * V, hipStream_t st);
void launch_global_importance(const Geom & g, const Work & w, hipStream_t st);
void launch_select_topk(const Geom & g, const Work & w, hipStream_t st);
void launch_div_level(const Geom & g, const Work & w, const DivWork & dw, const float * K, hipStream_t st);
void launch_fill_int(int * p, int v, long long n, hipStream_t st);
// fill kernels stand in for hipMemsetAsync (a caller may capture the call in a graph)
void launch_fill_f32(float * p, float v, long long n, hipStream_t st);
void launch_refine_step(const Geom & g, const Work & w, hipStream_t st);
// Ssel (optional): the kept keys' scores [L][H][nq_max][t_total] in place of S[:, sel]
void launch_ls_softmax(const Geom & g, const Work & w, const float * beta, hipStream_t st,
                       const float * Ssel = nullptr);
// The scoring, chunk softmax, importance and refit target of a call in one
// kernel whose scores stay on chip (k_score_attend): chunks of at most 1280
// keys, at most 32 reference queries shared by every chunk, d_v = 128, fp32
// K and V with 16-byte aligned rows. S (optional) receives the raw scores of
// the heads h < mh (and w.smax their tile maxima) for the statistics.
bool score_attend_ok(const Geom & g, const float * K, const float * V, const float * Q, int Tc_max, int nq_max,
                     int qmode);
void launch_score_attend(const Geom & g, const Work & w, const float * K, const float * V, const float * Q,
                         float * S, int mh, hipStream_t st);
void launch_gather_exp(const Geom & g, const Work & w, hipStream_t st);
void launch_nnls_lh(const Geom & g, const Work & w, float * wout, int max_iter, int * status, hipStream_t st);
void launch_beta_log(float * wb, long long n, hipStream_t st);
// PGD steps of the beta fit on [AtA | Atb] in aug and M in X (wb refined in
// place; 3 tc_max + nq_max <= PGD_LDS_FLOATS)
constexpr int PGD_LDS_FLOATS = 40960 - 64;
void launch_nnls_pgd(const Geom & g, const Work & w, float * wb, int iters, hipStream_t st);
// query rows: the chunk softmax keeps two floats per row in LDS, OMP three
constexpr int SOFTMAX_MAXQ = 8192, OMP_MAXQ = 256;
// OMP selection into w.sel (rows of w.A and w.rowsum as the exp scores)
void launch_omp_select(const Geom & g, const Work & w, const OmpWork & ow, hipStream_t st);
// m_by_lu: k_ls_build leaves M = X^T X out where k_ge_lu can form it from X
// (the register LU's systems with nq * n <= 8192); launch_ge_lu must then
// be given the same flag
void launch_ls_build(const Geom & g, const Work & w, hipStream_t st, bool m_by_lu = false);
void launch_ge_lu(const Geom & g, const Work & w, hipStream_t st, bool m_by_lu = false);
void launch_ge_solve(const Geom & g, const Work & w, float * Cv, hipStream_t st);
// S_main: the main path's scores [L][H][nq_max][T], used (and overwritten by
// the sampled rows' softmax) when the statistics share its query set; else null
void launch_stats(const Geom & g, const Work & w, const StatWork & sw, const float * K,
                  const float * V, const float * Q, const float * beta, const float * Cv,
                  float * stats, hipStream_t st, float * S_main = nullptr);
// the same in parts: original attention (needs S and V only), compacted
// attention, then the statistics (needs both)
// beside_lu: it runs on a second stream beside the factorizations, so the
// sums with V take the form that shares a CU with a factorization block
void launch_stats_original(const Geom & g, const Work & w, const StatWork & sw, const float * K,
                           const float * V, const float * Q, hipStream_t st, float * S_main,
                           bool beside_lu = false);
void launch_stats_compacted(const Geom & g, const Work & w, const StatWork & sw, const float * K,
                            const float * V, const float * Q, const float * beta, const float * Cv,
                            float * stats, hipStream_t st);
void launch_stats_final(const Geom & g, const StatWork & sw, float * stats, hipStream_t st);
void launch_dequant_rows(const uint8_t * src, int type, long long row_bytes, int n_el, long long rows,
                         float * dst, hipStream_t st);
void launch_quant_rows(const float * src, long long src_ld, const int * idx, int type, int n_el,
                       long long rows, uint8_t * dst, long long row_bytes, hipStream_t st);
void launch_gather_cv_rows(const float * Cv, int H, int t, int dv, float * rows, hipStream_t st);
// whole-cache codec kernels (coalesced; Q8_0, Q4_0, F16, BF16, F32 when codec8_ok)
bool codec8_ok(int type, int n_el);
void launch_dequant8(const uint8_t * src, int type, long long row_bytes, long long src_ls, int n_el, int T, int L,
                     float * dst, hipStream_t st);
// mode 0: kept rows idx[l * idx_ls + j] of src (row stride src_ld, layer stride
// src_ls floats); mode 1: value rows assembled from C_v [L][H][rows][dv]
// sq.base != nullptr (mode 0): the kept rows are read in place from that
// quantized cache (src unused) and re-encoded
void launch_requant8(const float * src, long long src_ls, long long src_ld, const int * idx, long long idx_ls,
                     int mode, int H, int dv, int type, int n_el, int rows, int L, uint8_t * dst, long long row_bytes,
                     long long dst_ls, hipStream_t st, RowCodec sq = RowCodec{});
// state blobs: [rows][cols] -> [cols][rows]; kept key rows with the beta
// fold; transposed value columns; the reference-query rows of each head
void launch_transpose(const float * src, long long rows, long long cols, float * dst, hipStream_t st);
void launch_fold_rows(const float * K, int nk, const int * sel, int t, const float * beta, const float * dir, int H,
                      int dk, float scale, float * out, hipStream_t st);
void launch_value_columns(const float * Cv, const float * V, int nv, const int * sel, int H, int dv, int t,
                          float * col, hipStream_t st);
void launch_gather_qref(const float * K, long long ldK, int nk, int q0, int nq, int H, int dk, int L, float * out,
                        hipStream_t st);
void launch_iota(int * p, long long n, hipStream_t st);
void launch_gemm_abt(const float * A, long long lda, const float * B, long long ldb, float * C, long long ldc,
                     int m, int n, int k, float scale, long long sa, long long sb, long long sc, int batch,
                     hipStream_t st);
void launch_gemm_ab(const float * A, long long lda, const float * B, long long ldb, float * C, long long ldc,
                    int m, int n, int k, long long sa, long long sb, long long sc, int batch, hipStream_t st);

}  // namespace kvc
