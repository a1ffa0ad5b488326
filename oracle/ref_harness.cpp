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

size_t ref_convert_from_f32(const float * src, int type, uint8_t * dst, int n) {
    return convert_from_f32(src, type, dst, n);
}

void ref_convert_to_f32(const uint8_t * src, int type, float * dst, size_t n) {
    parsed_kv_state::convert_to_f32(src, type, dst, n);
}

float ref_f16_to_f32(uint16_t h) { return parsed_kv_state::f16_to_f32(h); }
uint16_t ref_f32_to_f16(float f) { return f32_to_f16(f); }

float ref_expf(float x) { return expf(x); }

}  // extern "C"
