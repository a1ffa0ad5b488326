// Shared declarations between the host orchestrator and the HIP kernels of
// libkv-compact.so (MI355X / gfx950).
//
// Numerical contract: every kernel reproduces the reference CPU path's fp32
// operation order (sequential dot products, multiply and add rounded
// separately, the same expf/sqrtf/division semantics), so device results
// equal the reference's bit for bit. The whole library is compiled with
// -ffp-contract=off; division and sqrt use the correctly rounded sequences.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace kvc {

// How the reference queries of a chunk are obtained.
enum QMode : int {
    Q_PROVIDED = 0,      // caller's Q_ref rows (reference api.cpp:391-393)
    Q_CHEAP_GLOBAL = 1,  // rows of K sampled over the whole call (api.cpp:382-390)
    Q_CHEAP_LOCAL = 2,   // rows of K sampled inside each chunk (chunk regenerates, api.cpp:473-475)
};

// One chunk of the reference's chunk plan (api.cpp:417-499). All chunks of a
// call share the plan; every layer of a batch uses the same plan.
struct ChunkDesc {
    int start;    // first token of the chunk
    int Tc;       // tokens in the chunk
    int tc;       // tokens kept
    int prefix;   // forced leading positions
    int off;      // offset of the chunk's kept tokens in the merged output
    int nq;       // reference queries used by the chunk
};

// A quantized K or V cache read in place: the kernels that read the cache
// decode each block in registers as they load it (the same products as the
// whole-cache codec kernels). base == nullptr: the fp32 array is read.
// Block codecs only (Q8_0, Q4_0): 2-byte fields at even offsets of even row
// and layer strides.
struct RowCodec {
    const uint8_t * base;   // layer 0, row 0
    long long row_bytes;    // bytes per token row (all heads)
    long long layer_bytes;  // bytes per layer
    int type;               // KV_TYPE_Q8_0 (8) or KV_TYPE_Q4_0 (2)
};

// Geometry of a batch of layers sharing one plan.
struct Geom {
    int L, T, H, dk, dv;
    int n_chunks, t_total, nq_max, tc_max, Tc_max;
    int qmode, nq_global;       // query source; n_q of Q_CHEAP_GLOBAL/Q_PROVIDED
    long long ldK, ldV, ldQ;    // layer strides (elements)
    int score_method;           // 0 max, 1 rms, 2 mean
    float inv_sqrt_dk;
    float ridge;
    float zero_val;             // solution value of a skipped pivot (0 for C_v, eps for the beta weights)
    int lu_masked;              // 1: every register LU takes the masked variant (KVC_LU_MASKED=1, for tests)
    RowCodec kc, vc;            // in-place quantized K / V (base == nullptr: fp32 K / V)
};

// Device scratch for one batch (all pointers device memory).
struct Work {
    float * S;        // [L][H][nq_max][T]   scaled scores per chunk column range
    unsigned * smax;  // [L][H][nq_max][n_chunks][ceil(Tc_max/128)] order keys of the scoring tiles' row maxima
    float * A;        // [L][H][nq_max][T]   unnormalised exponentials e; the softmax weights are e * ainv[row]
    float * E;        // == A when beta is solved (the exp scores), else nullptr
    float * rowsum;   // [L][n_chunks][H][nq_max]
    float * ainv;     // [L][n_chunks][H][nq_max] 1 / (row sum + 1e-12f) of the chunk softmax
    float * imp;      // [L][H][T]           per-head importance
    float * amax;     // [L][H][T]           per-key maxima over queries of the softmax weights
                      //                     (sensitivity under the rms and mean score methods), or nullptr
    float * sens;     // [L][n_chunks][H]    head sensitivities (nullptr: max over heads)
    float * gimp;     // [L][T]              global importance (after R-KV weights)
    float * Y;        // [L][n_chunks][H][nq_max][dv]
    int   * sel;      // [L][t_total]        kept token positions (layer-local), ascending
    float * X;        // [L][H][nq_max][t_total] compacted softmax weights
    float * aug;      // GE workspace per (layer, chunk, head): M column-major [tc][tc], then B
                      // (tc x dv: row-major when tc <= 256, else column-major)
    int   * perm;     // [L][n_chunks][H][tc_max] pivot order of each system
    unsigned char * skip; // [L][n_chunks][H][tc_max] skipped-pivot flags by step
    float * LU;       // [L][n_chunks][H][256][256] by physical row: multipliers left of the row's
                      // pivot step, its U row from that step on (systems with tc <= 256)
    float * Bt;       // [L][n_chunks][H][256][dv] forward-substituted right-hand sides by logical row
    float * LU2;      // [L][n_chunks][H][128][128] trailing matrices of the split register LU
                      // (column-major), or nullptr: no split
    int   * map2;     // [L][n_chunks][H][128] physical row of each trailing-matrix row
    long long * aug_off; // [L][n_chunks][H] element offsets into aug
    float * gtmp;     // [L][n_chunks][H][tc_max + tc_max + dv] GE factor / pivot-row spill
    int   * cand;     // [L][n_chunks][Tc_max] selection candidates
    unsigned char * flags; // [L][n_chunks][Tc_max]
    float * wts;      // [T] R-KV weights (nullptr when disabled)
    int   * status;   // [1] nonzero: a kernel met a case this build refuses
    int   * refine_active; // [L][n_chunks] 1 while the unit's refinement rounds continue
    int   * lu_redo;  // [L][n_chunks][H] 1: the system's LU is redone with masked updates
    ChunkDesc * chunks;  // [n_chunks + 2]; then all T keys, then the kept keys (statistics)
    float * Qt;       // [L][H][dk][32] transposed reference queries (the fused scoring path), or nullptr
};

// Diversity selection scratch (api.cpp:175-233). One unit = (layer, chunk).
// A level runs candidate pruning, the candidates' Gram matrix and the greedy
// pass for the units whose gslot is >= 0.
enum DivState : int { DIV_PENDING = 0, DIV_DONE = 1, DIV_RETRY = 2, DIV_SHORT = 3 };
struct DivWork {
    float strength;   // diversity_strength
    float alpha;      // candidates: importance >= alpha * (t-th largest); 0 = every unused key
    int cap;          // candidate capacity of a unit at this level (<= DIV_MAX_CAND)
    int * state;      // [units] DivState
    int * gslot;      // [units] Gram slot of the unit at this level, -1 = not run
    int * count;      // [units] number of candidates
    float * maxnc;    // [units] largest importance among the pruned keys
    float * G;        // [slots][cap][cap] Gram matrix of the candidates' full key rows
};
constexpr int DIV_MAX_CAND = 1280;   // 20 candidates per lane in the greedy wave

// OMP key selection scratch (math.h:832-950). One unit = (layer, chunk).
struct OmpWork {
    float * ce;       // [L][nq_max][T]      exp scores summed over heads
    float * cs;       // [L][n_chunks][nq_max] row sums summed over heads
    float * corr;     // [L][T]              correlations with the residual
    unsigned char * mask; // [L][T]          1: key picked
    int * order;      // [L][t_total]        picks in pick order
    float * w;        // [L][t_total]        latest NNLS solution
    float * prev_w;   // [L][t_total]        weights of the residual (padded with 1e-12f between refits)
    float * G;        // [units][tc_max][tc_max] Gram matrix of the picked columns, pick order
    float * Atb;      // [units][tc_max]
    float * aug;      // [units][tc_max][tc_max + 1] the regularised system, solved in place
    float * vec;      // [units][4 tc_max + 1 + nq_max] PGD vectors (u, grad, v), GE pivot row and factors
    int k_choice, refit_interval, pgd_iters;
};

// Statistics scratch (api.cpp:239-325 sampling: h < min(H,4), qi < min(nq,32))
struct StatWork {
    int mh, mq, qmode;
    float * OS;   // [L][mh][mq][T]        original scores -> unnormalised softmax
    float * CS;   // [L][mh][mq][t_total]  compacted scores -> unnormalised softmax
    float * OI;   // [L][mh][mq]           1 / (row sum + 1e-12f) of the original rows
    float * CI;   // [L][mh][mq]           the same for the compacted rows
    float * OO;   // [L][mh][mq][dv]
    float * CO;   // [L][mh][mq][dv]
};

}  // namespace kvc
