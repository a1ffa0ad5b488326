// Fixture harness around the reference's header-only functions.
//
// TEST INFRASTRUCTURE ONLY. Built by `make -C oracle ref` from the reference
// headers where they lie (-I<reference>/include) into oracle/_ref/; never
// linked into the product. It gives the known-answer tests direct access to
// the reference's static building blocks (kv-compact-math.h,
// kv-compact-state.h), which its public API does not export.
#include <cmath>
#include <cstdint>
#include <cstring>
#include <algorithm>
#include <vector>

#include "kv-compact-math.h"
#include "kv-compact-state.h"

extern "C" {

void ref_least_squares_solve(const float * A, const float * b, float * x,
                             int m, int n, int p, float ridge) {
    least_squares_solve(A, b, x, m, n, p, ridge);
}

void ref_nnls_solve(const float * A, const float * b, float * w, int m, int n, int max_iter) {
    nnls_solve(A, b, w, m, n, max_iter);
}

void ref_nnls_pgd_solve(const float * A, const float * b, float * w, int m, int n,
                        float eps, int iters) {
    nnls_pgd_solve(A, b, w, m, n, eps, iters);
}

void ref_softmax_importance(const float * scores, float * attn, float * imp,
                            int m, int n, int agg) {
    softmax_importance_fused(scores, attn, imp, m, n, agg);
}

void ref_exp_softmax_importance(const float * scores, float * expo, float * rs,
                                float * attn, float * imp, int m, int n, int agg) {
    exp_softmax_importance_fused(scores, expo, rs, attn, imp, m, n, agg);
}

void ref_softmax_rows(float * x, int m, int n) { softmax_rows(x, m, n); }

void ref_mat_mul_ABt(const float * A, const float * B, float * C, int m, int n, int k) {
    mat_mul_ABt(A, B, C, m, n, k);
}

void ref_mat_mul_AB(const float * A, const float * B, float * C, int m, int k, int n) {
    mat_mul_AB(A, B, C, m, k, n);
}

size_t ref_convert_from_f32(const float * src, int type, uint8_t * dst, int n) {
    return convert_from_f32(src, type, dst, n);
}

void ref_convert_to_f32(const uint8_t * src, int type, float * dst, size_t n) {
    parsed_kv_state::convert_to_f32(src, type, dst, n);
}

float ref_f16_to_f32(uint16_t h) { return parsed_kv_state::f16_to_f32(h); }
uint16_t ref_f32_to_f16(float f) { return f32_to_f16(f); }

float ref_expf(float x) { return expf(x); }

// The CLI's stream-0 compaction (src/kv-compact.cpp:380-690) and write-back
// (:785-790) driven through the reference's own parse, math and blob writer.
// The glue follows the CLI's steps: queries = the last n_ref keys of each
// layer, max-aggregated importance (or the sensitivity-weighted sum) over all
// selected layers and heads, one partial_sort top-t, beta = 0, the LS value
// refit, beta directions, build_compacted_state. layers/n_layers: an explicit
// layer list (n_layers < 0: every layer). Returns 0, or -2 when the parse
// fails; *out is malloc'd.
int ref_state_compact(const uint8_t * blob, size_t size, uint32_t n_pos, int n_head_kv, float ratio, int n_ref,
                      int sens_budget, const int * layers, int n_layers, uint8_t ** out, size_t * out_size,
                      int * sel_out) {
    parsed_kv_state st;
    if (!st.parse(blob, size, n_pos)) return -2;
    const auto & sd = st.streams[0];
    const int T = (int)sd.cell_count, L = (int)sd.n_layer, H = n_head_kv;
    const int nk = sd.layers[0].n_embd_k_gqa(), nv = sd.layers[0].n_embd_v_gqa_computed();
    const int dk = nk / H, dv = nv / H;
    const int t = std::max(1, (int)(T * ratio));
    int nq = n_ref <= 0 ? std::max(16, T / 4) : n_ref;
    nq = std::min(nq, T);
    const int q0 = T - nq;
    auto on = [&](int l) {
        if (n_layers < 0) return true;
        for (int i = 0; i < n_layers; i++) if (layers[i] == l) return true;
        return false;
    };
    const float inv_sqrt = 1.0f / sqrtf((float)dk);
    std::vector<float> gimp(T, 0.0f), sens;
    std::vector<std::vector<float>> head_imp;
    std::vector<std::vector<std::vector<float>>> S(L), A(L);
    std::vector<float> qb((size_t)nq * dk), kb((size_t)T * dk), vb((size_t)T * dv);
    for (int l = 0; l < L; l++) {
        if (!on(l)) continue;
        const auto & ld = sd.layers[l];
        S[l].resize(H);
        A[l].resize(H);
        for (int h = 0; h < H; h++) {
            S[l][h].resize((size_t)nq * T);
            A[l][h].resize((size_t)nq * T);
            extract_head_contiguous(ld.K.data() + (size_t)q0 * nk, qb.data(), nq, dk, nk, h * dk);
            extract_head_contiguous(ld.K.data(), kb.data(), T, dk, nk, h * dk);
            mat_mul_ABt(qb.data(), kb.data(), S[l][h].data(), nq, T, dk);
            for (auto & x : S[l][h]) x *= inv_sqrt;
            std::vector<float> imp(T);
            softmax_importance_fused(S[l][h].data(), A[l][h].data(), imp.data(), nq, T);
            if (sens_budget) {
                sens.push_back(compute_head_sensitivity(A[l][h].data(), nq, T));
                head_imp.push_back(std::move(imp));
            } else {
                for (int j = 0; j < T; j++) if (imp[j] > gimp[j]) gimp[j] = imp[j];
            }
        }
    }
    if (sens_budget) accumulate_weighted_importance(head_imp, sens, T, (int)sens.size(), gimp.data());
    std::vector<int> idx(T);
    for (int j = 0; j < T; j++) idx[j] = j;
    std::partial_sort(idx.begin(), idx.begin() + t, idx.end(), [&](int a, int b) { return gimp[a] > gimp[b]; });
    std::vector<int> sel(idx.begin(), idx.begin() + t);
    std::sort(sel.begin(), sel.end());
    if (sel_out) std::copy(sel.begin(), sel.end(), sel_out);
    std::vector<std::vector<std::vector<float>>> cv(L), beta(L), dirs(L);
    for (int l = 0; l < L; l++) {
        const auto & ld = sd.layers[l];
        cv[l].resize(H);
        beta[l].assign(H, std::vector<float>(t, 0.0f));
        dirs[l].assign(H, std::vector<float>(dk, 0.0f));
        for (int h = 0; h < H; h++) {
            cv[l][h].resize((size_t)t * dv);
            if (!on(l)) {
                for (int j = 0; j < t; j++)
                    memcpy(cv[l][h].data() + (size_t)j * dv, ld.V.data() + (size_t)sel[j] * nv + h * dv, dv * 4);
                continue;
            }
            std::vector<float> X((size_t)nq * t);
            for (int i = 0; i < nq; i++)
                for (int j = 0; j < t; j++) X[(size_t)i * t + j] = S[l][h][(size_t)i * T + sel[j]] + beta[l][h][j];
            softmax_rows(X.data(), nq, t);
            extract_head_contiguous(ld.V.data(), vb.data(), T, dv, nv, h * dv);
            std::vector<float> Y((size_t)nq * dv);
            mat_mul_AB(A[l][h].data(), vb.data(), Y.data(), nq, T, dv);
            least_squares_solve(X.data(), Y.data(), cv[l][h].data(), nq, t, dv);
            std::vector<float> Qh((size_t)nq * dk);
            for (int i = 0; i < nq; i++) memcpy(Qh.data() + (size_t)i * dk, ld.K.data() + (size_t)(q0 + i) * nk + h * dk, dk * 4);
            compute_beta_direction(Qh.data(), nq, dk, dirs[l][h].data());
        }
    }
    std::vector<uint8_t> blob_out = build_compacted_state(st, sel, cv, H, dk, dv, n_pos, beta, dirs);
    *out = (uint8_t *)malloc(blob_out.size() + 1);
    memcpy(*out, blob_out.data(), blob_out.size());
    *out_size = blob_out.size();
    return 0;
}

void ref_free(void * p) { free(p); }

}  // extern "C"
