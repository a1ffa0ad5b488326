// HIP kernels of the attention-matching compaction path for MI355X (gfx950).
//
// Every kernel keeps the reference CPU path's fp32 operation order so the
// device output equals the reference's bit for bit:
//   * dot products accumulate sequentially over the feature index, one
//     rounded multiply and one rounded add per term (built with
//     -ffp-contract=off), then one multiply by 1/sqrt(d_k);
//   * row softmax: max, e = expf(x - max) by the glibc algorithm restated
//     below, a sequential sum, 1/(sum + 1e-12f), one multiply;
//   * Gaussian elimination with partial pivoting in the reference's row and
//     column order (first maximal |pivot| wins, pivots below 1e-12 skipped).
// Parallelism comes from independent outputs (keys, queries, heads, chunks,
// layers); a sum whose order matters always runs in one thread.
#include "kvc_common.h"
#include "kvc_kernels.h"

#include <math.h>
#include <stdlib.h>

#include <algorithm>

#include <utility>

namespace kvc {

// ---------------------------------------------------------------------------
// expf as glibc computes it on x86-64 (FMA variant of the ARM optimized-
// routines method): exp(x) = 2^(k/32) * 2^(r/32), k = round(x*32/ln2),
// cubic polynomial in double. c_exp2_tab[i] = bits(2^(i/32)) - (i << 47),
// filled by the host at start-up. Verified against libm expf over every
// float in [-104, 0] (the softmax domain).
// ---------------------------------------------------------------------------
__constant__ uint64_t c_exp2_tab[32];

// tab: c_exp2_tab, or a copy of it in LDS. Kernels that store results
// between exponentials use the LDS copy: a lane-indexed lookup in constant
// memory is a vector memory load, and waiting for it also waits for every
// store in flight.
__device__ __forceinline__ float expf_ref(float x, const uint64_t * tab = c_exp2_tab) {
    if (x < -0x1.9fe368p6f) return 0.0f;
    if (x > 0x1.62e42ep6f) return __int_as_float(0x7f800000);
    const double N = 32.0;
    const double inv_ln2_n = 0x1.71547652b82fep+0 * N;
    const double shift = 0x1.8p+52;
    const double c0 = 0x1.c6af84b912394p-5 / N / N / N;
    const double c1 = 0x1.ebfce50fac4f3p-3 / N / N;
    const double c2 = 0x1.62e42ff0c52d6p-1 / N;
    double xd = (double)x;
    double z = inv_ln2_n * xd;
    double kd = z + shift;
    uint64_t ki = (uint64_t)__double_as_longlong(kd);
    kd -= shift;
    double r = __builtin_fma(inv_ln2_n, xd, -kd);
    uint64_t tb = tab[ki % 32] + (ki << 47);
    double s = __longlong_as_double((long long)tb);
    double p = __builtin_fma(c0, r, c1);
    double r2 = r * r;
    double y = __builtin_fma(c2, r, 1.0);
    y = __builtin_fma(p, r2, y);
    return (float)(y * s);
}

// The same value as expf_ref for every x, computed without branches: the
// general path always, then the two range results selected (for x below
// the lower or above the upper limit the general path's value is unused;
// NaN takes the general path in both forms).
__device__ __forceinline__ float expf_ref_sel(float x, const uint64_t * tab) {
    const double N = 32.0;
    const double inv_ln2_n = 0x1.71547652b82fep+0 * N;
    const double shift = 0x1.8p+52;
    const double c0 = 0x1.c6af84b912394p-5 / N / N / N;
    const double c1 = 0x1.ebfce50fac4f3p-3 / N / N;
    const double c2 = 0x1.62e42ff0c52d6p-1 / N;
    double xd = (double)x;
    double z = inv_ln2_n * xd;
    double kd = z + shift;
    uint64_t ki = (uint64_t)__double_as_longlong(kd);
    kd -= shift;
    double r = __builtin_fma(inv_ln2_n, xd, -kd);
    uint64_t tb = tab[ki % 32] + (ki << 47);
    double sc = __longlong_as_double((long long)tb);
    double p = __builtin_fma(c0, r, c1);
    double r2 = r * r;
    double y = __builtin_fma(c2, r, 1.0);
    y = __builtin_fma(p, r2, y);
    const float v = (float)(y * sc);
    return x < -0x1.9fe368p6f ? 0.0f : (x > 0x1.62e42ep6f ? __int_as_float(0x7f800000) : v);
}

// ---------------------------------------------------------------------------
// logf as glibc computes it on x86-64 (FMA variant of the ARM optimized-
// routines method): x = 2^k * z with z in [0x1.66p-1, 0x1.66p0), 16
// subintervals with a tabulated c ~ 1/invc and log(c), then
// log(x) = k ln2 + log(c) + log1p(r), r = z*invc - 1, with a cubic in double.
// Verified against libm logf over every non-negative finite float (the beta
// weights are >= 1e-12). Only finite positive normal inputs reach it here.
// ---------------------------------------------------------------------------
__device__ __forceinline__ float logf_ref(float x) {
    const double ln2 = 0x1.62e42fefa39efp-1;
    const double a0 = -0x1.00ea348b88334p-2, a1 = 0x1.5575b0be00b6ap-2, a2 = -0x1.ffffef20a4123p-2;
    const double invc_t[16] = {
        0x1.661ec79f8f3bep+0, 0x1.571ed4aaf883dp+0, 0x1.49539f0f010bp+0, 0x1.3c995b0b80385p+0,
        0x1.30d190c8864a5p+0, 0x1.25e227b0b8eap+0, 0x1.1bb4a4a1a343fp+0, 0x1.12358f08ae5bap+0,
        0x1.0953f419900a7p+0, 0x1p+0, 0x1.e608cfd9a47acp-1, 0x1.ca4b31f026aap-1,
        0x1.b2036576afce6p-1, 0x1.9c2d163a1aa2dp-1, 0x1.886e6037841edp-1, 0x1.767dcf5534862p-1};
    const double logc_t[16] = {
        -0x1.57bf7808caadep-2, -0x1.2bef0a7c06ddbp-2, -0x1.01eae7f513a67p-2, -0x1.b31d8a68224e9p-3,
        -0x1.6574f0ac07758p-3, -0x1.1aa2bc79c81p-3, -0x1.a4e76ce8c0e5ep-4, -0x1.1973c5a611ccp-4,
        -0x1.252f438e10c1ep-5, 0x0p+0, 0x1.aa5aa5df25984p-5, 0x1.c5e53aa362eb4p-4,
        0x1.526e57720db08p-3, 0x1.bc2860d22477p-3, 0x1.1058bc8a07ee1p-2, 0x1.4043057b6ee09p-2};
    uint32_t ix = __float_as_uint(x);
    if (ix == 0x3f800000u) return 0.0f;
    if (ix - 0x00800000u >= 0x7f800000u - 0x00800000u) {
        if (ix * 2u == 0u) return -__int_as_float(0x7f800000);
        if (ix == 0x7f800000u) return x;
        if ((ix & 0x80000000u) || ix * 2u >= 0xff000000u) return __int_as_float(0x7fc00000);
        ix = __float_as_uint(x * 0x1p23f) - (23u << 23);   // subnormal: normalise
    }
    const uint32_t tmp = ix - 0x3f330000u;
    const int i = (int)((tmp >> 19) % 16u);
    const int k = (int)tmp >> 23;
    const uint32_t iz = ix - (tmp & 0xff800000u);
    const double z = (double)__uint_as_float(iz);
    const double r = __builtin_fma(z, invc_t[i], -1.0);
    const double y0 = __builtin_fma((double)k, ln2, logc_t[i]);
    const double r2 = r * r;
    double y = __builtin_fma(a1, r, a2);
    y = __builtin_fma(a0, r2, y);
    y = __builtin_fma(y, r2, y0 + r);
    return (float)y;
}

// lane L of each 16-lane row of v, in every lane (DPP row_newbcast, folded
// into the instruction that uses it)
template <int L>
__device__ __forceinline__ float sb_bc(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x150 + L, 0xf, 0xf, false));
}

// cheap reference-query row (api.cpp:140-151): quadratic spacing over n rows
__device__ __forceinline__ int cheap_pos(int qi, int n, int T) {
    float f = (float)(qi + 1) / (float)(n + 1);
    f = f * f;
    int pos = (int)(f * (float)(T - 1));
    if (pos >= T) pos = T - 1;
    if (pos < 0) pos = 0;
    return pos;
}

// Row of the reference queries used by chunk c for query qi (head offset 0).
__device__ __forceinline__ const float * query_row(const Geom & g, const float * K, const float * Q,
                                                   int layer, const ChunkDesc & c, int qi, int qmode) {
    const long long ek = (long long)g.H * g.dk;
    if (qmode == Q_PROVIDED) return Q + layer * g.ldQ + (long long)qi * ek;
    if (qmode == Q_CHEAP_GLOBAL) return K + layer * g.ldK + (long long)cheap_pos(qi, g.nq_global, g.T) * ek;
    return K + layer * g.ldK + (long long)(c.start + cheap_pos(qi, c.nq, c.Tc)) * ek;
}

// In-place quantized rows (RowCodec), decoded with the whole-cache codec's
// products: Q8_0 d * q, Q4_0 d * (nibble - 8) with adjacent-pair nibbles
// (state.h:355-375). TYPE (KV_TYPE_Q8_0 = 8 or KV_TYPE_Q4_0 = 2) is fixed per
// kernel instance; codec_inst picks the instance for a RowCodec (0: fp32).
__device__ __forceinline__ float f16_to_f32_ref(uint16_t hv);

// f16 bits to f32, exact and without branches: the same bits as
// f16_to_f32_ref (subnormals are m * 2^-24, a normal f32; Inf and NaN keep
// their payload; zeros keep their sign)
__device__ __forceinline__ float f16_bits_f32(uint32_t h) {
    const uint32_t sign = (h & 0x8000u) << 16, e = (h >> 10) & 0x1Fu, m = h & 0x3FFu;
    const uint32_t sub = __float_as_uint((float)m * 0x1p-24f);
    const uint32_t nrm = ((e + 112u) << 23) | (m << 13);
    const uint32_t inf = 0x7F800000u | (m << 13);
    return __uint_as_float(sign | (e == 0u ? sub : (e == 31u ? inf : nrm)));
}

inline int codec_inst(const RowCodec & rc) { return rc.base ? rc.type : 0; }

__device__ __forceinline__ const uint8_t * codec_row(const RowCodec & rc, int l, long long r) {
    return rc.base + l * rc.layer_bytes + r * rc.row_bytes;
}

// The loads and the decode apart, so that a loader can keep the raw bits in
// registers while a tile is summed and decode them when it stores the next
// one: Q8_0 {scale, 2 bytes, 2 bytes}, Q4_0 {scale, 2 bytes}. Elements
// c .. c + 3 (c a multiple of 4: one block, aligned 2-byte fields) of a row
// from its first byte.
struct Raw4 {
    uint32_t x, y, z, w;
};
template <int TYPE>
__device__ __forceinline__ Raw4 codec_raw4_at(const uint8_t * row, int c) {
    const int o = c & 31;
    if constexpr (TYPE == 8) {
        const uint8_t * bl = row + (c >> 5) * 34;
        return Raw4{*reinterpret_cast<const uint16_t *>(bl), *reinterpret_cast<const uint16_t *>(bl + 2 + o),
                    *reinterpret_cast<const uint16_t *>(bl + 4 + o), 0u};
    } else {
        const uint8_t * bl = row + (c >> 5) * 18;
        return Raw4{*reinterpret_cast<const uint16_t *>(bl), *reinterpret_cast<const uint16_t *>(bl + 2 + (o >> 1)),
                    0u, 0u};
    }
}
template <int TYPE>
__device__ __forceinline__ Raw4 codec_raw4(const RowCodec & rc, int l, long long r, int c) {
    return codec_raw4_at<TYPE>(codec_row(rc, l, r), c);
}
template <int TYPE>
__device__ __forceinline__ float4 codec_dec4(const Raw4 & v) {
    const float d = f16_bits_f32(v.x);
    if constexpr (TYPE == 8)
        return make_float4(d * (float)(int8_t)(v.y & 0xFF), d * (float)(int8_t)(v.y >> 8),
                           d * (float)(int8_t)(v.z & 0xFF), d * (float)(int8_t)(v.z >> 8));
    else
        return make_float4(d * ((float)(v.y & 0xF) - 8.0f), d * ((float)((v.y >> 4) & 0xF) - 8.0f),
                           d * ((float)((v.y >> 8) & 0xF) - 8.0f), d * ((float)((v.y >> 12) & 0xF) - 8.0f));
}
template <int TYPE>
__device__ __forceinline__ float4 codec_load4(const RowCodec & rc, int l, long long r, int c) {
    return codec_dec4<TYPE>(codec_raw4<TYPE>(rc, l, r, c));
}
// element c (any) of row r of layer l
template <int TYPE>
__device__ __forceinline__ float codec_load1(const RowCodec & rc, int l, long long r, int c) {
    const uint8_t * row = codec_row(rc, l, r);
    const int o = c & 31;
    if constexpr (TYPE == 8) {
        const uint8_t * bl = row + (c >> 5) * 34;
        return f16_bits_f32(*reinterpret_cast<const uint16_t *>(bl)) * (float)(int8_t)bl[2 + o];
    } else {
        const uint8_t * bl = row + (c >> 5) * 18;
        const uint8_t b = bl[2 + (o >> 1)];
        return f16_bits_f32(*reinterpret_cast<const uint16_t *>(bl)) * ((float)((o & 1) ? (b >> 4) : (b & 0xF)) - 8.0f);
    }
}
// v where keep, else zero bits (per component: a select of the struct goes
// through memory). Zero bits decode to +0 or -0 in every codec.
__device__ __forceinline__ Raw4 raw_keep(bool keep, const Raw4 & v) {
    return Raw4{keep ? v.x : 0u, keep ? v.y : 0u, keep ? v.z : 0u, keep ? v.w : 0u};
}
// a 16-byte fp32 load as raw bits, and back
__device__ __forceinline__ Raw4 f32_raw4(const float * p) {
    const float4 x = *reinterpret_cast<const float4 *>(p);
    return Raw4{__float_as_uint(x.x), __float_as_uint(x.y), __float_as_uint(x.z), __float_as_uint(x.w)};
}
__device__ __forceinline__ float4 raw_f4(const Raw4 & v) {
    return make_float4(__uint_as_float(v.x), __uint_as_float(v.y), __uint_as_float(v.z), __uint_as_float(v.w));
}

// K row (token index) of reference query qi of chunk c in the cheap modes
__device__ __forceinline__ long long query_krow(const Geom & g, const ChunkDesc & c, int qi, int qmode) {
    if (qmode == Q_CHEAP_GLOBAL) return cheap_pos(qi, g.nq_global, g.T);
    return c.start + cheap_pos(qi, c.nq, c.Tc);
}

// order-preserving key of a float score (unsigned order = float order; NaN excluded by callers)
__device__ __forceinline__ unsigned score_key(float x) {
    const unsigned b = __float_as_uint(x);
    return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}

// Wave-wide max / min of a 32-bit unsigned value through DPP row shifts and
// row broadcasts (the result collects in lane 63).
template <bool MAX>
__device__ __forceinline__ unsigned dpp_reduce_u32(unsigned x) {
    // lanes without a source (row edge, masked row) see the identity, which
    // lets the move and the min/max fold into one DPP instruction
    constexpr int ident = MAX ? 0 : -1;
#define KVC_DPP_STEP(ctrl, rmask)                                                                  \
    {                                                                                              \
        const unsigned t = (unsigned)__builtin_amdgcn_update_dpp(ident, (int)x, ctrl, rmask, 0xf, false); \
        x = MAX ? (t > x ? t : x) : (t < x ? t : x);                                               \
    }
    KVC_DPP_STEP(0x111, 0xf)   // row_shr:1
    KVC_DPP_STEP(0x112, 0xf)   // row_shr:2
    KVC_DPP_STEP(0x114, 0xf)   // row_shr:4
    KVC_DPP_STEP(0x118, 0xf)   // row_shr:8
    KVC_DPP_STEP(0x142, 0xa)   // row_bcast:15
    KVC_DPP_STEP(0x143, 0xc)   // row_bcast:31
#undef KVC_DPP_STEP
    return (unsigned)__builtin_amdgcn_readlane((int)x, 63);
}

__device__ __forceinline__ long long lS(const Geom & g) { return (long long)g.H * g.nq_max * g.T; }
__device__ __forceinline__ long long hS(const Geom & g) { return (long long)g.nq_max * g.T; }

// ---------------------------------------------------------------------------
// Scores. S[l][h][qi][start + j] = (sum_d q[d] k_j[d]) * inv_sqrt_dk, the dot
// product sequential over d (math.h:44-54; the product a*b is symmetric).
// Block: 128 keys x 32 query rows; thread (tk, tr) owns keys 4 tk .. 4 tk + 3
// and rows 4 tr .. 4 tr + 3 (16 sums). Features are staged through LDS in
// slabs of 32, transposed (dimension-major) so each thread reads its 4 keys
// and its 4 rows as one 16-byte load each. grid = (ceil(Tc_max/128),
// n_chunks * Hs, L); query rows beyond 32 loop.
// tmax (optional): each block also writes, per query row, the order key
// (score_key) of its largest non-NaN stored score, or of -inf, at
// tmax[(((layer * Hs + h) * nq_max + qi) * n_chunks + chunk) * gridDim.x + blockIdx.x];
// the chunk softmax takes its row maxima from these instead of re-reading S.
// ---------------------------------------------------------------------------
constexpr int SC_KEYS = 128, SC_SLAB = 32, SC_ROWS = 32;

// max of x over lanes 0-31 in lane 31 and over lanes 32-63 in lane 63
__device__ __forceinline__ unsigned dpp_half_max_u32(unsigned x) {
#define KVC_DPP_STEP(ctrl, rmask)                                                                  \
    {                                                                                              \
        const unsigned t = (unsigned)__builtin_amdgcn_update_dpp(0, (int)x, ctrl, rmask, 0xf, false); \
        x = t > x ? t : x;                                                                         \
    }
    KVC_DPP_STEP(0x111, 0xf)   // row_shr:1
    KVC_DPP_STEP(0x112, 0xf)   // row_shr:2
    KVC_DPP_STEP(0x114, 0xf)   // row_shr:4
    KVC_DPP_STEP(0x118, 0xf)   // row_shr:8
    KVC_DPP_STEP(0x142, 0xa)   // row_bcast:15
#undef KVC_DPP_STEP
    return x;
}

// KC: 0, or the codec (8 Q8_0, 2 Q4_0) of a quantized K read in place (g.kc),
// decoded in registers
template <int KC>
__global__ void __launch_bounds__(256)
k_scores(Geom g, const ChunkDesc * __restrict__ chunks, const float * __restrict__ K,
         const float * __restrict__ Q, float * __restrict__ S, int Hs, int nq_cap,
         long long s_layer, long long s_head, long long s_row, int qmode,
         const int * __restrict__ key_idx, const float * __restrict__ beta, unsigned * __restrict__ tmax) {
    const int c_idx = blockIdx.y / Hs, h = blockIdx.y % Hs, layer = blockIdx.z;
    const ChunkDesc c = chunks[c_idx];
    const int key0 = blockIdx.x * SC_KEYS;
    if (key0 >= c.Tc) return;
    const int nq = min(c.nq, nq_cap);
    __shared__ __align__(16) float ks[SC_SLAB][SC_KEYS + 4];
    __shared__ __align__(16) float qs[SC_SLAB][SC_ROWS + 4];
    __shared__ const float * qptr[SC_ROWS];
    __shared__ long long qoff[SC_ROWS];
    const int tid = threadIdx.x;
    const int tk = tid & 31, tr = tid >> 5;
    const long long ek = (long long)g.H * g.dk;
    // K read in place from a quantized cache (uniform): the fast path below
    // decodes its tiles in registers; the host sends such K only when that
    // path is taken (d_k a multiple of 32, provided queries 16-byte aligned)
    constexpr bool kcod = KC != 0;
    // key_idx: keys are rows key_idx[layer * t_total + j] (compacted statistics)
    const float * Kl = kcod ? nullptr : K + layer * g.ldK + (key_idx ? 0 : (long long)c.start * ek) + (long long)h * g.dk;
    const int * kix = key_idx ? key_idx + (long long)layer * g.t_total : nullptr;
    const float * bh = beta ? beta + ((long long)layer * g.H + h) * g.t_total : nullptr;
    float * Sl = S + layer * s_layer + h * s_head + c.start;
    // scaled (+ beta) scores of rows q0 + 4 tr .. + 3 out to S, and each row's tile maximum to tmax
    auto store_tile = [&](const float (&acc)[4][4], int q0) {
        // fmaxf returns the other operand for a NaN, so mx is the largest
        // non-NaN score or -inf (a zero's sign may differ from a scan's
        // first-found zero, which leaves every s - max unchanged)
        float mx[4];
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int qi = q0 + 4 * tr + i;
            mx[i] = -INFINITY;
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const int key = key0 + 4 * tk + j;
                if (key < c.Tc) {
                    float v = acc[i][j] * g.inv_sqrt_dk;
                    if (bh) v = v + bh[key];
                    if (qi < nq) Sl[(long long)qi * s_row + key] = v;
                    mx[i] = fmaxf(mx[i], v);
                }
            }
        }
        if (tmax) {
            const long long nt = gridDim.x, ncu = gridDim.y / Hs;
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const unsigned m = dpp_half_max_u32(score_key(mx[i]));
                const int qi = q0 + 4 * tr + i;
                if ((tid & 31) == 31 && qi < nq)
                    tmax[((((long long)layer * Hs + h) * g.nq_max + qi) * ncu + c_idx) * nt + blockIdx.x] = m;
            }
        }
    };
    // tile loaders: 8 threads per key row (4 dims each, 16-byte loads when
    // aligned), keys (tid >> 3) + 32 u; query rows likewise
    const int ld = (tid & 7) * 4, lr = tid >> 3;
    const float * kp[4];
#pragma unroll
    for (int u = 0; u < 4; u++) {
        const int key = key0 + lr + 32 * u;
        const long long row = (key < c.Tc) ? (kix ? (long long)kix[key] : (long long)key) : -1;
        kp[u] = (row >= 0) ? Kl + row * ek : nullptr;
    }
    const bool vec = (g.dk & 3) == 0 &&
                     (kcod || ((ek & 3) == 0 && (reinterpret_cast<uintptr_t>(Kl) & 15) == 0)) &&
                     (qmode != Q_PROVIDED || ((reinterpret_cast<uintptr_t>(Q) & 15) == 0 && (g.ldQ & 3) == 0));
    if (vec && g.dk % SC_SLAB == 0) {
        // whole 16-byte slabs: every thread loads rows that exist (keys past
        // the chunk read its last key, query rows past nq read row 0; their
        // sums are not stored), with no branch around the loads, and the next
        // slab is loaded while this one is summed
        const float * kq[4];
        long long kr[4];   // token rows (quantized K)
#pragma unroll
        for (int u = 0; u < 4; u++) {
            const int key = min(key0 + lr + 32 * u, c.Tc - 1);
            kr[u] = kix ? (long long)kix[key] : (long long)c.start + key;
            kq[u] = kcod ? nullptr : Kl + (kix ? (long long)kix[key] : (long long)key) * ek + ld;
        }
        const int kc0 = h * g.dk + ld;   // this thread's first element of a quantized row
        const uint8_t * krp[4];
#pragma unroll
        for (int u = 0; u < 4; u++) krp[u] = kcod ? codec_row(g.kc, layer, kr[u]) : nullptr;
        // query rows as element offsets from qbase (a pointer kept in LDS
        // would make the row loads flat ones, which every LDS wait waits for),
        // or as K token rows when they are rows of a quantized K
        const bool qcod = kcod && qmode != Q_PROVIDED;
        const float * qbase = qmode == Q_PROVIDED ? Q : K;
        // raw loads (bits kept while a slab is summed), decoded at the LDS store
        auto kload = [&](int u, int dn) -> Raw4 {
            return kcod ? codec_raw4_at<KC>(krp[u], kc0 + dn) : f32_raw4(kq[u] + dn);
        };
        for (int q0 = 0; q0 < nq; q0 += SC_ROWS) {
            __syncthreads();
            if (tid < SC_ROWS) {
                const int qi = q0 + tid, qq = qi < nq ? qi : 0;
                qoff[tid] = qcod ? query_krow(g, c, qq, qmode)
                                 : (query_row(g, K, Q, layer, c, qq, qmode) - qbase) + (long long)h * g.dk;
            }
            __syncthreads();
            const long long qo = qoff[lr];
            const float * qp = qcod ? nullptr : qbase + qo + ld;
            const uint8_t * qrp = qcod ? codec_row(g.kc, layer, qo) : nullptr;
            auto qload = [&](int dn) -> Raw4 {
                return qcod ? codec_raw4_at<KC>(qrp, kc0 + dn) : f32_raw4(qp + dn);
            };
            float acc[4][4];
#pragma unroll
            for (int i = 0; i < 4; i++)
#pragma unroll
                for (int j = 0; j < 4; j++) acc[i][j] = 0.0f;
            Raw4 kx[4], qx;
#pragma unroll
            for (int u = 0; u < 4; u++) kx[u] = kload(u, 0);
            qx = qload(0);
            for (int d0 = 0; d0 < g.dk; d0 += SC_SLAB) {
                __syncthreads();
#pragma unroll
                for (int u = 0; u < 4; u++) {
                    const int kk = lr + 32 * u;
                    const float4 k4 = kcod ? codec_dec4<KC>(kx[u]) : raw_f4(kx[u]);
                    ks[ld][kk] = k4.x; ks[ld + 1][kk] = k4.y; ks[ld + 2][kk] = k4.z; ks[ld + 3][kk] = k4.w;
                }
                const float4 q4 = qcod ? codec_dec4<KC>(qx) : raw_f4(qx);
                qs[ld][lr] = q4.x; qs[ld + 1][lr] = q4.y; qs[ld + 2][lr] = q4.z; qs[ld + 3][lr] = q4.w;
                __syncthreads();
                // the next slab (the last one again at the end: no branch)
                const int dn = min(d0 + SC_SLAB, g.dk - SC_SLAB);
#pragma unroll
                for (int u = 0; u < 4; u++) kx[u] = kload(u, dn);
                qx = qload(dn);
                asm volatile("" ::: "memory");   // keeps the loads ahead of the sums, not sunk to their use
                // dimension dd + 1 is read from LDS while dd is summed
                float4 kv = *reinterpret_cast<const float4 *>(&ks[0][4 * tk]);
                float4 qv = *reinterpret_cast<const float4 *>(&qs[0][4 * tr]);
#pragma unroll
                for (int dd = 0; dd < SC_SLAB; dd++) {
                    float4 kn = kv, qn = qv;
                    if (dd + 1 < SC_SLAB) {
                        kn = *reinterpret_cast<const float4 *>(&ks[dd + 1][4 * tk]);
                        qn = *reinterpret_cast<const float4 *>(&qs[dd + 1][4 * tr]);
                    }
                    __builtin_amdgcn_sched_barrier(0);
                    const float kk[4] = {kv.x, kv.y, kv.z, kv.w}, qq[4] = {qv.x, qv.y, qv.z, qv.w};
#pragma unroll
                    for (int i = 0; i < 4; i++)
#pragma unroll
                        for (int j = 0; j < 4; j++) acc[i][j] = acc[i][j] + qq[i] * kk[j];
                    __builtin_amdgcn_sched_barrier(0);
                    kv = kn;
                    qv = qn;
                }
            }
            store_tile(acc, q0);
        }
        return;
    }
    for (int q0 = 0; q0 < nq; q0 += SC_ROWS) {
        __syncthreads();
        if (tid < SC_ROWS) {
            const int qi = q0 + tid;
            qptr[tid] = (qi < nq) ? query_row(g, K, Q, layer, c, qi, qmode) + (long long)h * g.dk : nullptr;
        }
        float acc[4][4];
#pragma unroll
        for (int i = 0; i < 4; i++)
#pragma unroll
            for (int j = 0; j < 4; j++) acc[i][j] = 0.0f;
        for (int d0 = 0; d0 < g.dk; d0 += SC_SLAB) {
            __syncthreads();
            const int dim = d0 + ld;
            const bool full = vec && dim + 3 < g.dk;
#pragma unroll
            for (int u = 0; u < 4; u++) {
                float4 x = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
                if (kp[u]) {
                    if (full) {
                        x = *reinterpret_cast<const float4 *>(kp[u] + dim);
                    } else {
                        if (dim < g.dk) x.x = kp[u][dim];
                        if (dim + 1 < g.dk) x.y = kp[u][dim + 1];
                        if (dim + 2 < g.dk) x.z = kp[u][dim + 2];
                        if (dim + 3 < g.dk) x.w = kp[u][dim + 3];
                    }
                }
                const int kk = lr + 32 * u;
                ks[ld][kk] = x.x; ks[ld + 1][kk] = x.y; ks[ld + 2][kk] = x.z; ks[ld + 3][kk] = x.w;
            }
            {
                const float * qp = qptr[lr];
                float4 x = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
                if (qp) {
                    if (full) {
                        x = *reinterpret_cast<const float4 *>(qp + dim);
                    } else {
                        if (dim < g.dk) x.x = qp[dim];
                        if (dim + 1 < g.dk) x.y = qp[dim + 1];
                        if (dim + 2 < g.dk) x.z = qp[dim + 2];
                        if (dim + 3 < g.dk) x.w = qp[dim + 3];
                    }
                }
                qs[ld][lr] = x.x; qs[ld + 1][lr] = x.y; qs[ld + 2][lr] = x.z; qs[ld + 3][lr] = x.w;
            }
            __syncthreads();
            const int dn = min(SC_SLAB, g.dk - d0);
            for (int dd = 0; dd < dn; dd++) {
                const float4 kv = *reinterpret_cast<const float4 *>(&ks[dd][4 * tk]);
                const float4 qv = *reinterpret_cast<const float4 *>(&qs[dd][4 * tr]);
                const float kk[4] = {kv.x, kv.y, kv.z, kv.w}, qq[4] = {qv.x, qv.y, qv.z, qv.w};
#pragma unroll
                for (int i = 0; i < 4; i++)
#pragma unroll
                    for (int j = 0; j < 4; j++) acc[i][j] = acc[i][j] + qq[i] * kk[j];
            }
        }
        store_tile(acc, q0);
    }
}

// ---------------------------------------------------------------------------
// Block reductions (blockDim.x a multiple of 64, at most 1024)
// ---------------------------------------------------------------------------
__device__ __forceinline__ float block_max(float v, float * red) {
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o));
    const int w = threadIdx.x >> 6;
    __syncthreads();
    if ((threadIdx.x & 63) == 0) red[w] = v;
    __syncthreads();
    float r = red[0];
    for (int i = 1; i < (int)(blockDim.x >> 6); i++) r = fmaxf(r, red[i]);
    return r;
}

// Row maximum in the reference's scan order: start from row[0], replace on
// strictly greater. Without NaN this is the plain maximum; a NaN at row[0]
// is kept, any other NaN is skipped.
__device__ __forceinline__ float ref_row_max(const float * row, int n, float * red) {
    float m = -INFINITY;
    for (int j = threadIdx.x; j < n; j += blockDim.x) {
        const float v = row[j];
        if (v == v) m = fmaxf(m, v);
    }
    m = block_max(m, red);
    const float r0 = row[0];
    if (r0 != r0) return r0;
    return (m > r0) ? m : r0;
}

// ---------------------------------------------------------------------------
// Chunk softmax + per-key importance (math.h:142-248).
//   A = e * inv, e = expf(s - max), inv = 1/(sum e + 1e-12f), sum sequential
//   imp[j] = max / rms / mean over rows, accumulated in row order
// E/rowsum are written when beta is solved. grid = (n_chunks * H, L)
// ---------------------------------------------------------------------------
// Row maximum in the reference's scan order for one row held by a wave:
// the largest non-NaN value (or -inf), unless row[0] is NaN (then NaN);
// every lane gets the result.
__device__ __forceinline__ float wave_ref_row_max(const float * row, int n, int lane) {
    float m = -INFINITY;
    int j = lane;
    for (; j + 192 < n; j += 256) {   // four loads in flight
        float v[4];
#pragma unroll
        for (int u = 0; u < 4; u++) v[u] = row[j + 64 * u];
#pragma unroll
        for (int u = 0; u < 4; u++)
            if (v[u] == v[u] && v[u] > m) m = v[u];
    }
    for (; j < n; j += 64) {
        const float v = row[j];
        if (v == v && v > m) m = v;
    }
    const unsigned k = dpp_reduce_u32<true>(score_key(m));
    const unsigned b = (k & 0x80000000u) ? (k & 0x7fffffffu) : ~k;   // inverse of score_key
    const float mm = __uint_as_float(b);
    const float r0 = row[0];
    if (r0 != r0) return r0;
    return (mm > r0) ? mm : r0;
}

// Workgroup barrier for data in LDS only: waits for this wave's LDS
// operations and leaves its global loads and stores in flight (a
// __syncthreads also waits for those). The empty asm statements keep the
// compiler from moving memory accesses across it.
__device__ __forceinline__ void lds_barrier() {
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_waitcnt(0xc07f);   // lgkmcnt(0), vmcnt and expcnt unchanged
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}

// Chunk softmax + per-key importance (math.h:142-248), for up to SOFTMAX_MAXQ rows
// (two floats per row in dynamic LDS):
//  1. row maxima, one wave per row;
//  2. e = expf(s - max) over 64-key tiles: written unnormalised to A, staged
//     in LDS so that one thread per row adds its tile in key order; the row's
//     inv = 1 / (sum + 1e-12f) goes to ainv (and the sum to rowsum, if given);
//  3. one thread per key: the weights a = e * inv row by row, importance
//     accumulated in row order (max / sum of squares / sum), finalised as the
//     reference. A keeps e: its consumers form a = e * inv themselves (the
//     same single rounding), and e itself is the beta fit's exp scores.
// grid = (n_chunks * H, L)
constexpr int SM_TILE = 64, SM_TROWS = 32;

__global__ void __launch_bounds__(256)
k_softmax_importance(Geom g, const ChunkDesc * __restrict__ chunks, const float * __restrict__ S,
                     const unsigned * __restrict__ smax, float * __restrict__ A, float * __restrict__ rowsum,
                     float * __restrict__ ainv, float * __restrict__ imp, float * __restrict__ amax) {
    const int c_idx = blockIdx.x / g.H, h = blockIdx.x % g.H, layer = blockIdx.y;
    const ChunkDesc c = chunks[c_idx];
    const long long rs = g.T;
    const float * Sh = S + layer * lS(g) + h * hS(g) + c.start;
    float * Ah = A + layer * lS(g) + h * hS(g) + c.start;
    extern __shared__ float sm_rows[];   // row maxima, then 1 / (row sum + 1e-12f): nq_max each
    float * rmax = sm_rows;
    float * rinv = sm_rows + g.nq_max;
    __shared__ float eb[SM_TROWS][SM_TILE + 1];
    __shared__ uint64_t etab[32];
    const int nq = c.nq, n = c.Tc;
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    if (tid < 32) etab[tid] = c_exp2_tab[tid];   // visible after the barrier below
    // 1. row maxima: from the scoring tiles' maxima (smax, see k_scores), or
    //    one wave per row over S
    if (smax) {
        const int nt = (g.Tc_max + SC_KEYS - 1) / SC_KEYS, ntc = (n + SC_KEYS - 1) / SC_KEYS;
        for (int r = tid; r < nq; r += blockDim.x) {
            const unsigned * sm = smax + ((((long long)layer * g.H + h) * g.nq_max + r) * g.n_chunks + c_idx) * nt;
            unsigned k = sm[0];
            for (int t = 1; t < ntc; t++) k = max(k, sm[t]);
            const float mm = __uint_as_float((k & 0x80000000u) ? (k & 0x7fffffffu) : ~k);
            const float r0 = Sh[r * rs];
            rmax[r] = (r0 != r0) ? r0 : ((mm > r0) ? mm : r0);
        }
    } else {
        for (int r = wv; r < nq; r += 4) {
            const float m = wave_ref_row_max(Sh + r * rs, n, lane);
            if (lane == 0) rmax[r] = m;
        }
    }
    __syncthreads();
    // 2. exponentials and ordered row sums, 32 rows at a time; the next tile's
    //    scores load while the row sums run (barriers for LDS only)
    const int kk = tid & 63;
    for (int r0 = 0; r0 < nq; r0 += SM_TROWS) {
        const int nr = min(SM_TROWS, nq - r0);
        float sum = 0.0f;   // row r0 + tid for tid < nr
        // this thread's rows wv, wv + 4, ... of tile t0, at clamped (in-bounds) rows and keys
        float sv[SM_TROWS / 4];
        auto load = [&](int t0) {
            const int j = t0 + min(kk, min(SM_TILE, n - t0) - 1);
#pragma unroll
            for (int u = 0; u < SM_TROWS / 4; u++)
                sv[u] = Sh[(long long)(r0 + min(wv + 4 * u, nr - 1)) * rs + j];
        };
        load(0);
        for (int t0 = 0; t0 < n; t0 += SM_TILE) {
            const int jn = min(SM_TILE, n - t0);
            if (kk < jn) {
#pragma unroll
                for (int u = 0; u < SM_TROWS / 4; u++) {
                    const int rr = wv + 4 * u;
                    if (rr < nr) {
                        const int r = r0 + rr;
                        const float e = expf_ref(sv[u] - rmax[r], etab);
                        eb[rr][kk] = e;
                        Ah[r * rs + t0 + kk] = e;
                    }
                }
            }
            lds_barrier();
            if (t0 + SM_TILE < n) load(t0 + SM_TILE);
            if (tid < nr) {
                int j = 0;
                for (; j + 16 <= jn; j += 16) {   // 16 reads in flight, then the adds in order
                    float e[16];
#pragma unroll
                    for (int k = 0; k < 16; k++) e[k] = eb[tid][j + k];
#pragma unroll
                    for (int k = 0; k < 16; k++) sum += e[k];
                }
                for (; j < jn; j++) sum += eb[tid][j];
            }
            lds_barrier();
        }
        if (tid < nr) {
            const int r = r0 + tid;
            const long long ro = (((long long)layer * g.n_chunks + c_idx) * g.H + h) * g.nq_max + r;
            if (rowsum) rowsum[ro] = sum;
            const float iv = 1.0f / (sum + 1e-12f);
            rinv[r] = iv;
            ainv[ro] = iv;
        }
    }
    __syncthreads();
    // 3. the weights per key, aggregated in row order
    float * imph = imp + ((long long)layer * g.H + h) * g.T + c.start;
    const float inv_m = 1.0f / (float)nq;
    float * amaxh = amax ? amax + ((long long)layer * g.H + h) * g.T + c.start : nullptr;
    for (int j = tid; j < n; j += blockDim.x) {
        float acc = 0.0f, mx = 0.0f;
        for (int q0 = 0; q0 < nq; q0 += 16) {
            // sixteen rows' loads in flight, then the row-ordered aggregation
            const int qn = min(16, nq - q0);
            float ev[16];
#pragma unroll
            for (int u = 0; u < 16; u++)
                if (u < qn) ev[u] = Ah[(q0 + u) * rs + j];
#pragma unroll
            for (int u = 0; u < 16; u++) {
                if (u < qn) {
                    const int qi = q0 + u;
                    const float a = ev[u] * rinv[qi];
                    if (g.score_method == 0) {
                        if (a > acc) acc = a;
                    } else if (g.score_method == 1) {
                        acc += a * a;
                    } else {
                        acc += a;
                    }
                    if (amaxh && a > mx) mx = a;
                }
            }
        }
        if (g.score_method == 1) acc = sqrtf(acc * inv_m);
        else if (g.score_method == 2) acc *= inv_m;
        imph[j] = acc;
        if (amaxh) amaxh[j] = mx;
    }
}

// ---------------------------------------------------------------------------
// Refit target Y = A V per (layer, chunk, head) (math.h:70-80): each output
// accumulated sequentially over the chunk's keys; keys are staged through LDS
// 32 at a time. The weights are formed on the way in as a = e * ascale[row]
// (the unnormalised exponentials times the row's 1 / (sum + 1e-12f), the
// chunk softmax's own product). grid (n_chunks*H, L)
// ---------------------------------------------------------------------------
constexpr int AS_KT = 32;

// Register-blocked tile: 256 threads as TQ x TV; thread (tq, tv) owns
// queries tq + TQ*i (i < QR) and columns tv + TV*k (k < VR) of a QB x VB
// output block (QB = TQ*QR, VB = TV*VR); every output is a sequential sum
// over the keys in order.
template <int QR, int VR, int TV, int VC>
__device__ __forceinline__ void attn_sum_tile(const float * __restrict__ a, const float * __restrict__ ascale,
                                              long long a_rs, int nq,
                                              const float * __restrict__ val, long long val_rs, int n,
                                              int vn, float * __restrict__ out, long long out_rs,
                                              const RowCodec & vq, int layer, long long vrow0, int ve0) {
    constexpr int TQ = 256 / TV, QB = TQ * QR, VB = TV * VR;
    __shared__ float as[QB][AS_KT + 1];
    __shared__ float vs[AS_KT][VB + 1];
    const int tq = threadIdx.x / TV, tv = threadIdx.x % TV;
    for (int v0 = 0; v0 < vn; v0 += VB) {
        const int vb = min(VB, vn - v0);
        for (int q0 = 0; q0 < nq; q0 += QB) {
            const int qb = min(QB, nq - q0);
            float acc[QR][VR];
#pragma unroll
            for (int i = 0; i < QR; i++)
#pragma unroll
                for (int k = 0; k < VR; k++) acc[i][k] = 0.0f;
            for (int j0 = 0; j0 < n; j0 += AS_KT) {
                const int jn = min(AS_KT, n - j0);
                __syncthreads();
                for (int e = threadIdx.x; e < QB * AS_KT; e += 256) {
                    const int qi = e / AS_KT, jj = e % AS_KT;
                    as[qi][jj] = (qi < qb && jj < jn) ? a[(long long)(q0 + qi) * a_rs + j0 + jj] * ascale[q0 + qi] : 0.0f;
                }
                for (int e = threadIdx.x; e < AS_KT * VB; e += 256) {
                    const int jj = e / VB, vv = e % VB;
                    // (a quantized V: token row vrow0 + j, element ve0 + column)
                    vs[jj][vv] = (jj < jn && vv < vb)
                                     ? (VC ? codec_load1<VC>(vq, layer, vrow0 + j0 + jj, ve0 + v0 + vv)
                                                : val[(long long)(j0 + jj) * val_rs + v0 + vv])
                                     : 0.0f;
                }
                __syncthreads();
                for (int jj = 0; jj < jn; jj++) {
                    float av[QR], vv[VR];
#pragma unroll
                    for (int i = 0; i < QR; i++) av[i] = as[tq + TQ * i][jj];
#pragma unroll
                    for (int k = 0; k < VR; k++) vv[k] = vs[jj][tv + TV * k];
#pragma unroll
                    for (int i = 0; i < QR; i++)
#pragma unroll
                        for (int k = 0; k < VR; k++) acc[i][k] += av[i] * vv[k];
                }
            }
#pragma unroll
            for (int i = 0; i < QR; i++) {
                const int qi = tq + TQ * i;
#pragma unroll
                for (int k = 0; k < VR; k++) {
                    const int vv = tv + TV * k;
                    if (qi < qb && vv < vb) out[(long long)(q0 + qi) * out_rs + v0 + vv] = acc[i][k];
                }
            }
        }
    }
}

// The same sums for vn == 128 with 16-byte aligned value rows: a 32 x 128
// output block, thread (tq, tv) = (tid / 32, tid % 32) owning queries
// 4 tq .. 4 tq + 3 and columns 4 tv .. 4 tv + 3, both read from LDS as one
// 16-byte load per key; the weights are staged key-major. Tile loads read
// rows that exist (clamped) and put zeros in registers for keys past n and
// queries past nq, with no branch around the loads; the next tile is loaded
// while this one is summed. A zero term leaves a sum unchanged: a sum that
// starts at +0 never becomes -0 (x + y is -0 only when both are -0), and
// x + (+0) = x for every other x.
template <int VC>
__device__ __forceinline__ void attn_sum_128(const float * __restrict__ a, const float * __restrict__ ascale,
                                             long long a_rs, int nq,
                                             const float * __restrict__ val, long long val_rs, int n,
                                             float * __restrict__ out, long long out_rs,
                                             const RowCodec & vq, int layer, long long vrow0, int ve0) {
    __shared__ __align__(16) float as[AS_KT][32];
    __shared__ __align__(16) float vs[AS_KT][128];
    const int tid = threadIdx.x, tq = tid >> 5, tv = tid & 31;
    // loaders: weights, thread -> query lq, keys 4 lk .. 4 lk + 3;
    // values, thread -> keys vk + 8 u, columns 4 vc .. 4 vc + 3
    const int lq = tid >> 3, lk = (tid & 7) * 4;
    const int vk = tid >> 5, vc = (tid & 31) * 4;
    for (int q0 = 0; q0 < nq; q0 += 32) {
        const bool qok = q0 + lq < nq;
        const float * arow = a + (long long)min(q0 + lq, nq - 1) * a_rs;
        const float sc = ascale[min(q0 + lq, nq - 1)];
        float ra[4];
        float4 rv[4];
        Raw4 rq[4];   // (quantized V) raw value bits, decoded at the LDS store
        // loads at clamped (valid) positions with no condition on them; the
        // row scale and the zeros for keys past n and queries past nq are
        // applied at the LDS store (a product or a select on a load here
        // would make each load wait for its data before the tile is summed)
        auto load = [&](int j0) {
#pragma unroll
            for (int u = 0; u < 4; u++) ra[u] = arow[min(j0 + lk + u, n - 1)];
#pragma unroll
            for (int u = 0; u < 4; u++) {
                const int j = min(j0 + vk + 8 * u, n - 1);
                if constexpr (VC != 0) {
                    rq[u] = codec_raw4<VC>(vq, layer, vrow0 + j, ve0 + vc);
                } else {
                    rv[u] = *reinterpret_cast<const float4 *>(val + (long long)j * val_rs + vc);
                }
            }
        };
        float acc[4][4];
#pragma unroll
        for (int i = 0; i < 4; i++)
#pragma unroll
            for (int k = 0; k < 4; k++) acc[i][k] = 0.0f;
        load(0);
        for (int j0 = 0; j0 < n; j0 += AS_KT) {
            __syncthreads();
#pragma unroll
            for (int u = 0; u < 4; u++) {
                const float x = ra[u] * sc;
                as[lk + u][lq] = (qok && j0 + lk + u < n) ? x : 0.0f;
            }
#pragma unroll
            for (int u = 0; u < 4; u++) {
                const bool in = j0 + vk + 8 * u < n;
                float4 x;
                if constexpr (VC != 0) x = codec_dec4<VC>(raw_keep(in, rq[u]));
                else x = in ? rv[u] : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
                *reinterpret_cast<float4 *>(&vs[vk + 8 * u][vc]) = x;
            }
            __syncthreads();
            load(j0 + AS_KT);   // past the end: clamped rows, zeros (not used)
            asm volatile("" ::: "memory");   // keeps the loads ahead of the sums
            float4 av = *reinterpret_cast<const float4 *>(&as[0][4 * tq]);
            float4 vv = *reinterpret_cast<const float4 *>(&vs[0][4 * tv]);
#pragma unroll
            for (int jj = 0; jj < AS_KT; jj++) {
                float4 an = av, vn = vv;
                if (jj + 1 < AS_KT) {
                    an = *reinterpret_cast<const float4 *>(&as[jj + 1][4 * tq]);
                    vn = *reinterpret_cast<const float4 *>(&vs[jj + 1][4 * tv]);
                }
                __builtin_amdgcn_sched_barrier(0);
                const float aa[4] = {av.x, av.y, av.z, av.w}, vx[4] = {vv.x, vv.y, vv.z, vv.w};
#pragma unroll
                for (int i = 0; i < 4; i++)
#pragma unroll
                    for (int k = 0; k < 4; k++) acc[i][k] = acc[i][k] + aa[i] * vx[k];
                __builtin_amdgcn_sched_barrier(0);
                av = an;
                vv = vn;
            }
        }
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int qi = q0 + 4 * tq + i;
            if (qi < nq)
                *reinterpret_cast<float4 *>(out + (long long)qi * out_rs + 4 * tv) =
                    make_float4(acc[i][0], acc[i][1], acc[i][2], acc[i][3]);
        }
    }
}

// Two kernels, so that each holds only its own LDS tiles: k_refit_target
// for d_v = 128 with 16-byte aligned value rows (chosen on the host), and
// k_refit_target_any for every other shape.
template <int VC>   // 0, or the codec of a quantized V read in place (g.vc)
__global__ void __launch_bounds__(256)
k_refit_target(Geom g, const ChunkDesc * __restrict__ chunks, const float * __restrict__ A,
               const float * __restrict__ ainv, const float * __restrict__ V, float * __restrict__ Y) {
    const int c_idx = blockIdx.x / g.H, h = blockIdx.x % g.H, layer = blockIdx.y;
    const ChunkDesc c = chunks[c_idx];
    const long long ev = (long long)g.H * g.dv;
    if (c.nq <= 0 || c.Tc <= 0) return;
    const float * sc = ainv + (((long long)layer * g.n_chunks + c_idx) * g.H + h) * g.nq_max;
    attn_sum_128<VC>(A + layer * lS(g) + h * hS(g) + c.start, sc, g.T, c.nq,
                 VC ? nullptr : V + layer * g.ldV + (long long)c.start * ev + (long long)h * g.dv, ev, c.Tc,
                 Y + ((((long long)layer * g.n_chunks + c_idx) * g.H + h) * g.nq_max) * g.dv, g.dv,
                 g.vc, layer, c.start, h * g.dv);
}

template <int VC>
__global__ void __launch_bounds__(256)
k_refit_target_any(Geom g, const ChunkDesc * __restrict__ chunks, const float * __restrict__ A,
                   const float * __restrict__ ainv, const float * __restrict__ V, float * __restrict__ Y) {
    const int c_idx = blockIdx.x / g.H, h = blockIdx.x % g.H, layer = blockIdx.y;
    const ChunkDesc c = chunks[c_idx];
    const long long ev = (long long)g.H * g.dv;
    const float * sc = ainv + (((long long)layer * g.n_chunks + c_idx) * g.H + h) * g.nq_max;
    attn_sum_tile<4, 4, 32, VC>(A + layer * lS(g) + h * hS(g) + c.start, sc, g.T, c.nq,
                            VC ? nullptr : V + layer * g.ldV + (long long)c.start * ev + (long long)h * g.dv,
                            ev, c.Tc, g.dv,
                            Y + ((((long long)layer * g.n_chunks + c_idx) * g.H + h) * g.nq_max) * g.dv, g.dv,
                            g.vc, layer, c.start, h * g.dv);
}

// ---------------------------------------------------------------------------
// Scoring, chunk softmax, per-key importance and the refit target in one pass
// per (layer, chunk, head), the chunk's scores held in registers so that
// neither the score matrix nor the softmax weights go to HBM (math.h:44-54,
// 142-248; api.cpp:618-628, 754-783). Thread t owns keys 2t and 2t + 1 of the
// chunk with all FA_ROWS query rows (64 values), FA_THREADS threads cover
// FA_KEYS keys; the registers this takes leave one block per CU. Every value
// is the reference's:
//   1. s = (sum_d q[d] k[d]) * inv_sqrt_dk, d ascending (the query columns
//      come from Qt [L][H][d_k][FA_ROWS], uniform over the block: scalar
//      operands; key rows in 64-byte segments), the same sums k_scores forms;
//   2. row maxima in the reference's scan semantics (largest non-NaN value,
//      or row[0] when it is NaN), from wave maxima of the order keys; each
//      wave's maxima are also the 128-key tile maxima the statistics' row
//      softmax reads (tmax, as k_scores writes them);
//   3. e = expf(s - max); row sums in key order: 64-key tiles of e go through
//      LDS and one thread per row adds them in order; inv = 1/(sum + 1e-12f);
//   4. a = e * inv; importance per key over the rows in row order (max, sum
//      of squares then sqrtf(acc * inv_m), or mean), as k_softmax_importance;
//   5. Y[i][v] = sum_j a[i][j] V[j][v], j ascending: 64-key tiles of a
//      (key-major) and V through LDS, double-buffered (the owners of the next
//      tile's keys and waves 8-9 fill it while threads 0..511, 2 rows x 4
//      columns each, sum this one; d_v = 128).
// S (optional): the raw scores of the heads h < mh are stored for the
// statistics (they read rows of S); other heads store nothing.
// grid (n_chunks * H, L); FA_THREADS threads.
// ---------------------------------------------------------------------------
constexpr int FA_THREADS = 640, FA_ROWS = 32, FA_KEYS = 2 * FA_THREADS, FA_TILE = 64;
constexpr int FA_WAVES = FA_THREADS / 64;

struct FaShared {
    union {
        float eb[2][FA_ROWS][FA_TILE + 1];   // e tiles for the ordered row sums
        struct {
            float at[2][FA_TILE][FA_ROWS];   // a tiles, key-major
            float vt[2][FA_TILE][128];       // V tiles
        } y;
    } u;
    unsigned red[FA_WAVES][FA_ROWS];         // per-wave row maxima (order keys)
    float rmax[FA_ROWS], rinv[FA_ROWS], r0[FA_ROWS];
    uint64_t etab[32];
};

__global__ void __launch_bounds__(FA_THREADS)
k_score_attend(Geom g, const ChunkDesc * __restrict__ chunks, const float * __restrict__ K,
               const float * __restrict__ Qt, const float * __restrict__ V, float * __restrict__ S, int mh,
               unsigned * __restrict__ tmax, float * __restrict__ imp, float * __restrict__ ainv,
               float * __restrict__ Y) {
    const int c_idx = blockIdx.x / g.H, h = blockIdx.x % g.H, layer = blockIdx.y;
    const ChunkDesc c = chunks[c_idx];
    const int n = c.Tc, nq = c.nq;
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    __shared__ __align__(16) FaShared sh;
    if (tid < 32) sh.etab[tid] = c_exp2_tab[tid];   // visible after the barriers below
    const long long ek = (long long)g.H * g.dk, ev = (long long)g.H * g.dv;
    const int j0 = 2 * tid;
    const bool ok0 = j0 < n, ok1 = j0 + 1 < n;
    // 1. scores (loads at clamped keys; the sums of keys past n are not used)
    const float * Kl = K + layer * g.ldK + (long long)c.start * ek + (long long)h * g.dk;
    const float4 * kp0 = reinterpret_cast<const float4 *>(Kl + (long long)min(j0, n - 1) * ek);
    const float4 * kp1 = reinterpret_cast<const float4 *>(Kl + (long long)min(j0 + 1, n - 1) * ek);
    const float * qt = Qt + ((long long)layer * g.H + h) * g.dk * FA_ROWS;
    float s0[FA_ROWS], s1[FA_ROWS];
#pragma unroll
    for (int i = 0; i < FA_ROWS; i++) s0[i] = s1[i] = 0.0f;
    // Each key row in 64-byte segments (16 dimensions, one cache line):
    // a thread's two segments sit in registers, and the next segment's first
    // half is loaded once this one's first eight dimensions are summed (its
    // second half after the rest), so the loads overlap the sums and every
    // line is read whole. Query column d: uniform scalar operands.
    const int nst = g.dk >> 4;   // (the host sends d_k % 16 == 0)
    float4 A[4], B[4];
#pragma unroll
    for (int k = 0; k < 4; k++) {
        A[k] = kp0[k];
        B[k] = kp1[k];
    }
    for (int st = 0; st < nst; st++) {
        const int nx = min(st + 1, nst - 1);
#pragma unroll
        for (int half = 0; half < 2; half++) {
#pragma unroll
            for (int dd = 0; dd < 8; dd++) {
                const int d = 16 * st + 8 * half + dd;
                const float a = (dd & 4) ? ((dd & 2) ? ((dd & 1) ? A[2 * half + 1].w : A[2 * half + 1].z)
                                                      : ((dd & 1) ? A[2 * half + 1].y : A[2 * half + 1].x))
                                         : ((dd & 2) ? ((dd & 1) ? A[2 * half].w : A[2 * half].z)
                                                      : ((dd & 1) ? A[2 * half].y : A[2 * half].x));
                const float b = (dd & 4) ? ((dd & 2) ? ((dd & 1) ? B[2 * half + 1].w : B[2 * half + 1].z)
                                                      : ((dd & 1) ? B[2 * half + 1].y : B[2 * half + 1].x))
                                         : ((dd & 2) ? ((dd & 1) ? B[2 * half].w : B[2 * half].z)
                                                      : ((dd & 1) ? B[2 * half].y : B[2 * half].x));
                const float * qd = qt + (long long)d * FA_ROWS;
#pragma unroll
                for (int i = 0; i < FA_ROWS; i++) {
                    const float q = qd[i];
                    s0[i] = s0[i] + q * a;
                    s1[i] = s1[i] + q * b;
                }
            }
            // this half's eight dimensions are summed: the next segment's
            // same half into their registers
            A[2 * half] = kp0[4 * nx + 2 * half];
            A[2 * half + 1] = kp0[4 * nx + 2 * half + 1];
            B[2 * half] = kp1[4 * nx + 2 * half];
            B[2 * half + 1] = kp1[4 * nx + 2 * half + 1];
            asm volatile("" ::: "memory");   // keeps the loads here, ahead of the next sums
        }
    }
#pragma unroll
    for (int i = 0; i < FA_ROWS; i++) {
        s0[i] = s0[i] * g.inv_sqrt_dk;
        s1[i] = s1[i] * g.inv_sqrt_dk;
    }
    if (S && h < mh) {
        float * Sh = S + layer * lS(g) + h * hS(g) + c.start;
#pragma unroll
        for (int i = 0; i < FA_ROWS; i++) {
            if (i < nq) {
                if (ok0) Sh[(long long)i * g.T + j0] = s0[i];
                if (ok1) Sh[(long long)i * g.T + j0 + 1] = s1[i];
            }
        }
    }
    if (tid == 0) {
#pragma unroll
        for (int i = 0; i < FA_ROWS; i++) sh.r0[i] = s0[i];
    }
    // 2. row maxima: wave maxima of the order keys of the largest non-NaN
    //    score (fmaxf skips NaN), then over the waves, then row[0]'s rule
    unsigned mine = 0u;
#pragma unroll
    for (int i = 0; i < FA_ROWS; i++) {
        float m = -INFINITY;
        if (ok0) m = fmaxf(m, s0[i]);
        if (ok1) m = fmaxf(m, s1[i]);
        const unsigned k = dpp_reduce_u32<true>(score_key(m));
        mine = lane == i ? k : mine;
    }
    if (lane < FA_ROWS) {
        sh.red[wv][lane] = mine;
        // this wave's 128 keys are one scoring tile of the statistics' row softmax
        if (tmax && h < mh && lane < nq && 128 * wv < n) {
            const long long nt = (g.Tc_max + SC_KEYS - 1) / SC_KEYS;
            tmax[((((long long)layer * g.H + h) * g.nq_max + lane) * g.n_chunks + c_idx) * nt + wv] = mine;
        }
    }
    __syncthreads();
    if (tid < FA_ROWS) {
        unsigned k = sh.red[0][tid];
        for (int w = 1; w < FA_WAVES; w++) k = max(k, sh.red[w][tid]);
        const float mm = __uint_as_float((k & 0x80000000u) ? (k & 0x7fffffffu) : ~k);
        const float a0 = sh.r0[tid];
        sh.rmax[tid] = (a0 != a0) ? a0 : ((mm > a0) ? mm : a0);
    }
    __syncthreads();
    // 3. exponentials (rows past nq and keys past n hold 0)
#pragma unroll
    for (int i = 0; i < FA_ROWS; i++) {
        const float m = sh.rmax[i];
        const float e0 = expf_ref_sel(s0[i] - m, sh.etab), e1 = expf_ref_sel(s1[i] - m, sh.etab);
        s0[i] = (ok0 && i < nq) ? e0 : 0.0f;
        s1[i] = (ok1 && i < nq) ? e1 : 0.0f;
    }
    //    the row sums in key order: tile p (keys 64 p ..) is written by
    //    threads 32 p .. 32 p + 31 while thread i < nq adds tile p - 1
    const int ntile = (n + FA_TILE - 1) / FA_TILE;
    auto put_e = [&](int p) {
        const int kk = j0 - FA_TILE * p;
        if (kk >= 0 && kk < FA_TILE) {
#pragma unroll
            for (int i = 0; i < FA_ROWS; i++) {
                sh.u.eb[p & 1][i][kk] = s0[i];
                sh.u.eb[p & 1][i][kk + 1] = s1[i];
            }
        }
    };
    float sum = 0.0f;
    put_e(0);
    __syncthreads();
    for (int p = 0; p < ntile; p++) {
        if (p + 1 < ntile) put_e(p + 1);
        if (tid < nq) {
            const int jn = min(FA_TILE, n - FA_TILE * p);
            const float * er = &sh.u.eb[p & 1][tid][0];
            int j = 0;
            for (; j + 16 <= jn; j += 16) {   // 16 reads in flight, then the adds in order
                float e[16];
#pragma unroll
                for (int k = 0; k < 16; k++) e[k] = er[j + k];
#pragma unroll
                for (int k = 0; k < 16; k++) sum += e[k];
            }
            for (; j < jn; j++) sum += er[j];
        }
        __syncthreads();
    }
    if (tid < nq) {
        const float iv = 1.0f / (sum + 1e-12f);
        sh.rinv[tid] = iv;
        ainv[(((long long)layer * g.n_chunks + c_idx) * g.H + h) * g.nq_max + tid] = iv;
    }
    __syncthreads();
    // 4. weights and importance, rows in order
    {
        const float inv_m = 1.0f / (float)nq;
        float acc0 = 0.0f, acc1 = 0.0f;
#pragma unroll
        for (int i = 0; i < FA_ROWS; i++) {
            if (i < nq) {
                const float iv = sh.rinv[i];
                const float a0 = s0[i] * iv, a1 = s1[i] * iv;
                s0[i] = a0;
                s1[i] = a1;
                if (g.score_method == 0) {
                    if (a0 > acc0) acc0 = a0;
                    if (a1 > acc1) acc1 = a1;
                } else if (g.score_method == 1) {
                    acc0 += a0 * a0;
                    acc1 += a1 * a1;
                } else {
                    acc0 += a0;
                    acc1 += a1;
                }
            }
        }
        if (g.score_method == 1) {
            acc0 = sqrtf(acc0 * inv_m);
            acc1 = sqrtf(acc1 * inv_m);
        } else if (g.score_method == 2) {
            acc0 *= inv_m;
            acc1 *= inv_m;
        }
        float * imph = imp + ((long long)layer * g.H + h) * g.T + c.start;
        if (ok0) imph[j0] = acc0;
        if (ok1) imph[j0 + 1] = acc1;
    }
    // 5. Y = A V over 64-key tiles, double-buffered in LDS: the owners of
    //    tile p + 1 write its weights and waves 8-9 load its V rows (four
    //    16-byte loads at a time, zeros past n) while threads 0..511 sum tile
    //    p, each owning rows 2 tq, 2 tq + 1 and columns 4 tv .. 4 tv + 3
    const float * Vl = V + layer * g.ldV + (long long)c.start * ev + (long long)h * g.dv;
    const bool yt = tid < 512;
    const int tq = (tid >> 5) & 15, tv = tid & 31;
    auto put_a = [&](int p) {
        const int kk = j0 - FA_TILE * p;
        if (kk >= 0 && kk < FA_TILE) {
#pragma unroll
            for (int i4 = 0; i4 < FA_ROWS / 4; i4++) {
                *reinterpret_cast<float4 *>(&sh.u.y.at[p & 1][kk][4 * i4]) =
                    make_float4(s0[4 * i4], s0[4 * i4 + 1], s0[4 * i4 + 2], s0[4 * i4 + 3]);
                *reinterpret_cast<float4 *>(&sh.u.y.at[p & 1][kk + 1][4 * i4]) =
                    make_float4(s1[4 * i4], s1[4 * i4 + 1], s1[4 * i4 + 2], s1[4 * i4 + 3]);
            }
        }
    };
    auto put_v = [&](int p) {   // waves 8-9: 128 threads, 16 rows of 4 keys x 32 columns each, all in flight
        const int lt = tid - 512, col = 4 * (lt & 31);
        float4 x[16];
#pragma unroll
        for (int u = 0; u < 16; u++) {
            const int kk = (lt >> 5) + 4 * u;
            x[u] = *reinterpret_cast<const float4 *>(Vl + (long long)min(FA_TILE * p + kk, n - 1) * ev + col);
        }
#pragma unroll
        for (int u = 0; u < 16; u++) {
            const int kk = (lt >> 5) + 4 * u;
            *reinterpret_cast<float4 *>(&sh.u.y.vt[p & 1][kk][col]) =
                FA_TILE * p + kk < n ? x[u] : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        }
    };
    float acc[2][4];
#pragma unroll
    for (int r = 0; r < 2; r++)
#pragma unroll
        for (int k = 0; k < 4; k++) acc[r][k] = 0.0f;
    __syncthreads();   // the row sums' tiles (same LDS) have been read
    put_a(0);
    if (!yt) put_v(0);
    __syncthreads();
    for (int p = 0; p < ntile; p++) {
        if (p + 1 < ntile) {
            put_a(p + 1);
            if (!yt) put_v(p + 1);
        }
        if (yt) {
            // keys in groups of four: the next group's LDS reads are in
            // flight while this group is summed (keys in order)
            const float (*at)[FA_ROWS] = sh.u.y.at[p & 1];
            const float (*vt)[128] = sh.u.y.vt[p & 1];
            float2 ag[4];
            float4 vg[4];
#pragma unroll
            for (int u = 0; u < 4; u++) {
                ag[u] = *reinterpret_cast<const float2 *>(&at[u][2 * tq]);
                vg[u] = *reinterpret_cast<const float4 *>(&vt[u][4 * tv]);
            }
#pragma unroll 4
            for (int j4 = 0; j4 < FA_TILE; j4 += 4) {
                float2 an[4];
                float4 vn[4];
                const int jn = min(j4 + 4, FA_TILE - 4);
#pragma unroll
                for (int u = 0; u < 4; u++) {
                    an[u] = *reinterpret_cast<const float2 *>(&at[jn + u][2 * tq]);
                    vn[u] = *reinterpret_cast<const float4 *>(&vt[jn + u][4 * tv]);
                }
                __builtin_amdgcn_sched_barrier(0);
#pragma unroll
                for (int u = 0; u < 4; u++) {
                    const float aa[2] = {ag[u].x, ag[u].y}, vx[4] = {vg[u].x, vg[u].y, vg[u].z, vg[u].w};
#pragma unroll
                    for (int r = 0; r < 2; r++)
#pragma unroll
                        for (int k = 0; k < 4; k++) acc[r][k] = acc[r][k] + aa[r] * vx[k];
                }
                __builtin_amdgcn_sched_barrier(0);
#pragma unroll
                for (int u = 0; u < 4; u++) {
                    ag[u] = an[u];
                    vg[u] = vn[u];
                }
            }
        }
        __syncthreads();
    }
    if (yt) {
        float * Yh = Y + ((((long long)layer * g.n_chunks + c_idx) * g.H + h) * g.nq_max) * g.dv;
#pragma unroll
        for (int r = 0; r < 2; r++) {
            const int qi = 2 * tq + r;
            if (qi < nq)
                *reinterpret_cast<float4 *>(Yh + (long long)qi * g.dv + 4 * tv) =
                    make_float4(acc[r][0], acc[r][1], acc[r][2], acc[r][3]);
        }
    }
}

// Qt[l][h][d][i] = component h * d_k + d of query row i (FA_ROWS rows; rows
// past nq are zero), the transposed query columns k_score_attend reads as
// uniform operands. grid (H, L), 256 threads.
__global__ void __launch_bounds__(256)
k_query_columns(Geom g, const ChunkDesc * __restrict__ chunks, const float * __restrict__ K,
                const float * __restrict__ Q, float * __restrict__ Qt) {
    const int h = blockIdx.x, layer = blockIdx.y;
    const ChunkDesc c = chunks[0];
    float * o = Qt + ((long long)layer * g.H + h) * g.dk * FA_ROWS;
    for (int e = threadIdx.x; e < g.dk * FA_ROWS; e += blockDim.x) {
        const int d = e / FA_ROWS, i = e % FA_ROWS;
        o[e] = i < c.nq ? query_row(g, K, Q, layer, c, i, g.qmode)[(long long)h * g.dk + d] : 0.0f;
    }
}

// ---------------------------------------------------------------------------
// Statistics attention outputs (api.cpp:270-293): out[q][v] = sum_j a[q][j] *
// val[j][v], j ascending, for the sampled heads and queries, over all T keys
// (original) or the t_total kept keys (compacted, val = C_v). Each output is a
// sequential sum, so the parallelism is the outputs: a block of 256 threads
// owns 16 queries x 64 columns, each thread one query x 4 columns (4
// independent sums; four waves per block keep two per SIMD busy); 64-key
// tiles of a and val are double-buffered in LDS.
// grid (mh * ceil(mq/16) * ceil(dv/64), L)
// ---------------------------------------------------------------------------
constexpr int SV_QB = 16, SV_VB = 64, SV_KT = 64, SV_THREADS = 256;

// LDS: As[2][SV_QB][SV_KT + 1] then Vs[2][SV_KT][SV_VB] (SV_LDS bytes), given
// at launch. At 80-86 VGPRs a block does not fit on a CU beside a k_ge_lu
// block (four waves per SIMD at 112 VGPRs leave 64): beside the
// factorizations the sums over an fp32 V take k_stats_values_lean, which
// does; this kernel serves the compacted statistics, a quantized V, and the
// calls that run the statistics after the solve.
constexpr int SV_LDS = (2 * SV_QB * (SV_KT + 1) + 2 * SV_KT * SV_VB) * 4;
// VC: 0, or the codec of a quantized V (mode 1) read in place (g.vc)
template <int VC>
__global__ void __launch_bounds__(SV_THREADS) __attribute__((amdgpu_waves_per_eu(5, 8)))
k_stats_values(Geom g, const float * __restrict__ a_all, const float * __restrict__ ascale, long long a_ls,
               long long a_hs, long long a_rs, int n,
               const float * __restrict__ V, const float * __restrict__ Cv, int mode, float * __restrict__ out_all,
               int mh, int mq) {
    const int nqb = (mq + SV_QB - 1) / SV_QB, nvb = (g.dv + SV_VB - 1) / SV_VB;
    const int layer = blockIdx.y;
    const int h = blockIdx.x / (nqb * nvb);
    const int q0 = ((blockIdx.x / nvb) % nqb) * SV_QB, v0 = (blockIdx.x % nvb) * SV_VB;
    const float * a = a_all + layer * a_ls + h * a_hs;   // row q at a + q * a_rs
    const float * val;
    long long vrs;
    // original attention over a quantized V: rows decoded in registers
    const bool vcod = VC != 0 && mode == 1;
    if (mode == 1) {
        vrs = (long long)g.H * g.dv;
        val = vcod ? nullptr : V + layer * g.ldV + (long long)h * g.dv;
    } else {
        vrs = g.dv;
        val = Cv + ((long long)layer * g.H + h) * g.t_total * g.dv;
    }
    float * out = out_all + (((long long)layer * mh + h) * mq) * g.dv;
    extern __shared__ __align__(16) float sv_lds[];
    float (*As)[SV_QB][SV_KT + 1] = reinterpret_cast<float (*)[SV_QB][SV_KT + 1]>(sv_lds);
    float (*Vs)[SV_KT][SV_VB] = reinterpret_cast<float (*)[SV_KT][SV_VB]>(sv_lds + 2 * SV_QB * (SV_KT + 1));
    const int tid = threadIdx.x, tq = tid >> 4, tv = tid & 15;
    const int qa = q0 + tq, vc = v0 + 4 * tv;
    // tile loaders: a: 16 x 64 (4 per thread); val: 64 x 64 (16 per thread, 4 float4)
    const bool vvec = (g.dv & 3) == 0 && (vcod || ((vrs & 3) == 0 && (reinterpret_cast<uintptr_t>(val) & 15) == 0));
    float ra[4];
    Raw4 rv[4];   // raw value bits (a quantized V is decoded at the LDS store)
    // row scales (the weights are a * ascale[row] when ascale is given),
    // applied at the LDS store: a product at the load would make each load
    // wait for its data before the next is issued
    float sc[4];
#pragma unroll
    for (int u = 0; u < 4; u++) {
        const int q = q0 + ((tid + SV_THREADS * u) >> 6);
        sc[u] = ascale ? ascale[((long long)layer * mh + h) * mq + min(q, mq - 1)] : 1.0f;
    }
    auto load = [&](int j0) {
#pragma unroll
        for (int u = 0; u < 4; u++) {
            const int e = tid + SV_THREADS * u, qi = e >> 6, jj = e & 63;
            const int q = q0 + qi, j = j0 + jj;
            ra[u] = (q < mq && j < n) ? a[(long long)q * a_rs + j] : 0.0f;
        }
#pragma unroll
        for (int u = 0; u < 4; u++) {
            const int e = tid + SV_THREADS * u, jj = e >> 4, c4 = (e & 15) * 4;
            const int j = j0 + jj, c = v0 + c4;
            Raw4 x{0u, 0u, 0u, 0u};
            if (j < n) {
                if (vcod && c + 3 < g.dv) {
                    x = codec_raw4<VC>(g.vc, layer, j, h * g.dv + c);
                } else if (vcod) {
                    // columns past d_v stay zero
                } else {
                    const float * src = val + (long long)j * vrs + c;
                    if (vvec && c + 3 < g.dv) {
                        x = f32_raw4(src);
                    } else {
                        if (c < g.dv) x.x = __float_as_uint(src[0]);
                        if (c + 1 < g.dv) x.y = __float_as_uint(src[1]);
                        if (c + 2 < g.dv) x.z = __float_as_uint(src[2]);
                        if (c + 3 < g.dv) x.w = __float_as_uint(src[3]);
                    }
                }
            }
            rv[u] = x;
        }
    };
    auto store = [&](int b) {
#pragma unroll
        for (int u = 0; u < 4; u++) {
            const int e = tid + SV_THREADS * u;
            As[b][e >> 6][e & 63] = ra[u] * sc[u];
        }
#pragma unroll
        for (int u = 0; u < 4; u++) {
            const int e = tid + SV_THREADS * u;
            // (zero bits: padded keys and columns, +0 or -0 in every codec)
            *reinterpret_cast<float4 *>(&Vs[b][e >> 4][(e & 15) * 4]) = vcod ? codec_dec4<VC>(rv[u]) : raw_f4(rv[u]);
        }
    };
    float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    const int ntiles = (n + SV_KT - 1) / SV_KT;
    if (ntiles > 0) {
        load(0);
        store(0);
    }
    __syncthreads();
    for (int t = 0; t < ntiles; t++) {
        const int b = t & 1;
        if (t + 1 < ntiles) load((t + 1) * SV_KT);
        const int jn = min(SV_KT, n - t * SV_KT);
        if (jn == SV_KT) {
#pragma unroll 4
            for (int jj = 0; jj < SV_KT; jj++) {
                const float a0 = As[b][tq][jj];
                const float4 x = *reinterpret_cast<const float4 *>(&Vs[b][jj][4 * tv]);
                acc[0] = acc[0] + a0 * x.x; acc[1] = acc[1] + a0 * x.y;
                acc[2] = acc[2] + a0 * x.z; acc[3] = acc[3] + a0 * x.w;
            }
        } else {
            for (int jj = 0; jj < jn; jj++) {
                const float a0 = As[b][tq][jj];
                const float4 x = *reinterpret_cast<const float4 *>(&Vs[b][jj][4 * tv]);
                acc[0] = acc[0] + a0 * x.x; acc[1] = acc[1] + a0 * x.y;
                acc[2] = acc[2] + a0 * x.z; acc[3] = acc[3] + a0 * x.w;
            }
        }
        if (t + 1 < ntiles) store(b ^ 1);
        __syncthreads();
    }
    if (qa < mq) {
#pragma unroll
        for (int k = 0; k < 4; k++)
            if (vc + k < g.dv) out[(long long)qa * g.dv + vc + k] = acc[k];
    }
}

// The same sums for grids that would leave most CUs idle (one layer): each
// thread one (query, column) output, so that a block's time is one sequential
// sum over the keys rather than four; blocks of 16 queries x 16 columns,
// 64-key tiles of a and val double-buffered in LDS. fp32 values only (a
// quantized V takes k_stats_values). grid (mh * ceil(mq/16) * ceil(dv/16), L).
constexpr int SVN_QB = 16, SVN_VB = 16;

__global__ void __launch_bounds__(SV_THREADS)
k_stats_values_narrow(Geom g, const float * __restrict__ a_all, const float * __restrict__ ascale, long long a_ls,
                      long long a_hs, long long a_rs, int n, const float * __restrict__ V,
                      const float * __restrict__ Cv, int mode, float * __restrict__ out_all, int mh, int mq) {
    const int nqb = (mq + SVN_QB - 1) / SVN_QB, nvb = (g.dv + SVN_VB - 1) / SVN_VB;
    const int layer = blockIdx.y;
    const int h = blockIdx.x / (nqb * nvb);
    const int q0 = ((blockIdx.x / nvb) % nqb) * SVN_QB, v0 = (blockIdx.x % nvb) * SVN_VB;
    const float * a = a_all + layer * a_ls + h * a_hs;   // row q at a + q * a_rs
    const float * val;
    long long vrs;
    if (mode == 1) {
        vrs = (long long)g.H * g.dv;
        val = V + layer * g.ldV + (long long)h * g.dv;
    } else {
        vrs = g.dv;
        val = Cv + ((long long)layer * g.H + h) * g.t_total * g.dv;
    }
    float * out = out_all + (((long long)layer * mh + h) * mq) * g.dv;
    __shared__ float As[2][SVN_QB][SV_KT + 1];
    __shared__ float Vs[2][SV_KT][SVN_VB];
    const int tid = threadIdx.x, tq = tid >> 4, tv = tid & 15;
    // tile loaders: a 16 x 64 and val 64 x 16, four elements per thread each
    float ra[4], rv[4], sc[4];
#pragma unroll
    for (int u = 0; u < 4; u++) {
        const int q = q0 + ((tid + SV_THREADS * u) >> 6);
        sc[u] = ascale ? ascale[((long long)layer * mh + h) * mq + min(q, mq - 1)] : 1.0f;
    }
    auto load = [&](int j0) {
#pragma unroll
        for (int u = 0; u < 4; u++) {
            const int e = tid + SV_THREADS * u, q = q0 + (e >> 6), j = j0 + (e & 63);
            ra[u] = (q < mq && j < n) ? a[(long long)q * a_rs + j] : 0.0f;
        }
#pragma unroll
        for (int u = 0; u < 4; u++) {
            const int e = tid + SV_THREADS * u, j = j0 + (e >> 4), c = v0 + (e & 15);
            rv[u] = (j < n && c < g.dv) ? val[(long long)j * vrs + c] : 0.0f;
        }
    };
    auto store = [&](int b) {
#pragma unroll
        for (int u = 0; u < 4; u++) {
            const int e = tid + SV_THREADS * u;
            As[b][e >> 6][e & 63] = ra[u] * sc[u];
            Vs[b][e >> 4][e & 15] = rv[u];
        }
    };
    float acc = 0.0f;
    const int ntiles = (n + SV_KT - 1) / SV_KT;
    if (ntiles > 0) {
        load(0);
        store(0);
    }
    __syncthreads();
    for (int t = 0; t < ntiles; t++) {
        const int b = t & 1;
        if (t + 1 < ntiles) load((t + 1) * SV_KT);
        const int jn = min(SV_KT, n - t * SV_KT);
        if (jn == SV_KT) {
#pragma unroll 8
            for (int jj = 0; jj < SV_KT; jj++) acc = acc + As[b][tq][jj] * Vs[b][jj][tv];
        } else {
            for (int jj = 0; jj < jn; jj++) acc = acc + As[b][tq][jj] * Vs[b][jj][tv];
        }
        if (t + 1 < ntiles) store(b ^ 1);
        __syncthreads();
    }
    const int q = q0 + tq, c = v0 + tv;
    if (q < mq && c < g.dv) out[(long long)q * g.dv + c] = acc;
}

// ---------------------------------------------------------------------------
// The original-attention sums (the k_stats_values arithmetic for mode 1 and
// an fp32 V: out[q][v] = sum_j (a[q][j] * ascale[q]) * V[j][v], j ascending)
// in a form that fits on a CU beside a k_ge_lu block, whose four waves per
// SIMD leave 32 VGPRs a lane, most of the VALU's issue slots and 90 KB of LDS:
// at most 32 VGPRs, one wave per SIMD, 48 KB of LDS. A block of four waves
// owns 32 queries x 64 columns of one (layer, head); a wave owns eight
// queries, lane = column, so each lane keeps eight independent sums. Tiles of
// 64 keys are copied to LDS with global_load_lds (no registers: each wave
// copies 16 rows of V, one 256-byte row an instruction, and its own eight
// weight rows), the next tile while the current one is summed. A lane reads
// the weight of query (l & 15) >> 1 for key jj + (l & 1) (l: its lane in the
// 16-lane row), scales it, and DPP broadcasts take each query's weight into
// the multiplies. Keys past the last whole tile come straight from memory.
// Offsets are 32-bit, the weight rows 16-byte aligned: the host checks both.
// grid (mh * ceil(mq / 32) * (dv / 64), L), dv a multiple of 64.
// ---------------------------------------------------------------------------
constexpr int SL_QW = 8, SL_QB = 4 * SL_QW, SL_KT = 64;
constexpr int SL_LDS = (2 * SL_KT * 64 + 4 * 2 * SL_QW * SL_KT) * 4;   // V tiles, then each wave's weight tiles

// key K of a pair: the weight of query Q sits in lane 2 Q + K of each
// 16-lane row of w
template <int K, int... Q>
__device__ __forceinline__ void sl_key(float (&acc)[SL_QW], float w, float v, std::integer_sequence<int, Q...>) {
    ((acc[Q] = acc[Q] + sb_bc<2 * Q + K>(w) * v), ...);
    // (one key's products at a time: the kernel has few registers)
    __builtin_amdgcn_sched_barrier(0);
}

template <class T>
__device__ __forceinline__ const T * sl_at(const T * base, unsigned byte_off) {
    return reinterpret_cast<const T *>(reinterpret_cast<const char *>(base) + byte_off);
}

__global__ void __launch_bounds__(256)
k_stats_values_lean(Geom g, const float * __restrict__ a_all, const float * __restrict__ ascale, long long a_ls,
                    long long a_hs, long long a_rs, int n, const float * __restrict__ V,
                    float * __restrict__ out_all, int mh, int mq) {
    const int nqb = (mq + SL_QB - 1) / SL_QB, nvb = g.dv / 64;
    const int layer = blockIdx.y;
    const int h = blockIdx.x / (nqb * nvb);
    const int wv = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int q0 = ((blockIdx.x / nvb) % nqb) * SL_QB + SL_QW * wv, c = (blockIdx.x % nvb) * 64 + lane;
    // the lane's weight row (rows past mq read row mq - 1; their sums are not
    // stored) and scale
    const int ql = min(q0 + ((lane & 15) >> 1), mq - 1);
    const float * __restrict__ ab = a_all + layer * a_ls + h * a_hs;
    const float sc = ascale ? ascale[((long long)layer * mh + h) * mq + ql] : 1.0f;
    const float * __restrict__ vb = V + layer * g.ldV + (long long)h * g.dv;
    const unsigned vrs4 = (unsigned)(g.H * g.dv) * 4u;   // bytes from one key's row of V to the next
    extern __shared__ __align__(16) float sl_lds[];
    float (*Vs)[SL_KT][64] = reinterpret_cast<float (*)[SL_KT][64]>(sl_lds);
    float (*Ws)[SL_QW][SL_KT] = reinterpret_cast<float (*)[SL_QW][SL_KT]>(sl_lds + 2 * SL_KT * 64) + 2 * wv;
    auto issue = [&](int t) {
        const int b = t & 1;
        const unsigned j0 = (unsigned)t * SL_KT;
#pragma unroll
        for (int k = 0; k < 16; k++) {
            const unsigned jj = 16u * wv + k;
            __builtin_amdgcn_global_load_lds(static_cast<const void *>(sl_at(vb, (j0 + jj) * vrs4 + 4u * c)),
                                             (__attribute__((address_space(3))) void *)&Vs[b][jj][0], 4, 0, 0);
        }
#pragma unroll
        for (int r = 0; r < 2; r++) {
            const int q = min(q0 + 4 * r + (lane >> 4), mq - 1);
            __builtin_amdgcn_global_load_lds(
                static_cast<const void *>(sl_at(ab, 4u * (unsigned)(q * a_rs + j0 + 4 * (lane & 15)))),
                (__attribute__((address_space(3))) void *)&Ws[b][4 * r][0], 16, 0, 0);
        }
    };
    float acc[SL_QW];
#pragma unroll
    for (int q = 0; q < SL_QW; q++) acc[q] = 0.0f;
    const int ntf = n / SL_KT;
    if (ntf > 0) issue(0);
    __syncthreads();   // (waits for the copies)
    for (int t = 0; t < ntf; t++) {
        const int b = t & 1;
        if (t + 1 < ntf) issue(t + 1);
#pragma unroll 2
        for (int jj = 0; jj < SL_KT; jj += 2) {
            const float w = Ws[b][(lane & 15) >> 1][jj + (lane & 1)] * sc;
            const float v0 = Vs[b][jj][lane], v1 = Vs[b][jj + 1][lane];
            sl_key<0>(acc, w, v0, std::make_integer_sequence<int, SL_QW>{});
            sl_key<1>(acc, w, v1, std::make_integer_sequence<int, SL_QW>{});
        }
        __syncthreads();   // tile t + 1 has landed; every wave is done with tile t
    }
    // the keys past the last whole tile
    const unsigned ao = (unsigned)(ql * a_rs);
    for (int j = ntf * SL_KT; j < n; j++) {
        const float w = ab[ao + (unsigned)j] * sc;
        sl_key<0>(acc, w, *sl_at(vb, (unsigned)j * vrs4 + 4u * c), std::make_integer_sequence<int, SL_QW>{});
    }
    float * out = out_all + (((long long)layer * mh + h) * mq) * g.dv;
#pragma unroll
    for (int q = 0; q < SL_QW; q++)
        if (q0 + q < mq) out[(long long)(q0 + q) * g.dv + c] = acc[q];
}

// ---------------------------------------------------------------------------
// Head sensitivity (math.h:579-594) of one (layer, chunk, head): over the
// chunk's keys, the largest of the per-key maxima over queries of the softmax
// weights (0 start, strictly greater replaces), over their mean (the sum runs
// in key order) plus 1e-12f. amax holds those per-key maxima [L][H][T] (the
// importance itself under the max score method). The wave walks the keys 64
// at a time and every lane adds the broadcast values in key order.
// grid = (n_chunks * H, L), 64 threads
// ---------------------------------------------------------------------------
__global__ void __launch_bounds__(64)
k_head_sensitivity(Geom g, const ChunkDesc * __restrict__ chunks, const float * __restrict__ amax,
                   float * __restrict__ sens) {
    const int c_idx = blockIdx.x / g.H, h = blockIdx.x % g.H, layer = blockIdx.y;
    const ChunkDesc c = chunks[c_idx];
    const float * src = amax + ((long long)layer * g.H + h) * g.T + c.start;
    const int n = c.Tc, lane = threadIdx.x;
    float sum = 0.0f, mx = 0.0f;
    for (int j0 = 0; j0 < n; j0 += 64) {
        const float x = (j0 + lane < n) ? src[j0 + lane] : 0.0f;
        const int cnt = min(64, n - j0);
        for (int k = 0; k < cnt; k++) {
            const float y = __shfl(x, k);
            sum += y;
            if (y > mx) mx = y;
        }
    }
    if (lane == 0) {
        const float mean = sum / (float)n;
        sens[((long long)layer * g.n_chunks + c_idx) * g.H + h] = mx / (mean + 1e-12f);
    }
}

// ---------------------------------------------------------------------------
// Global importance (api.cpp:656-684): max over heads (init 0, strictly
// greater replaces), or with sensitivity weighting (math.h:605-618) the sum
// over heads in order of sens_h * imp_h[j] from 0; then the R-KV weight.
// grid = (n_chunks, L)
// ---------------------------------------------------------------------------
__global__ void __launch_bounds__(256)
k_global_importance(Geom g, const ChunkDesc * __restrict__ chunks, const float * __restrict__ imp,
                    const float * __restrict__ wts, const float * __restrict__ sens, float * __restrict__ gimp) {
    const int c_idx = blockIdx.x, layer = blockIdx.y;
    const ChunkDesc c = chunks[c_idx];
    const float * sh = sens ? sens + ((long long)layer * g.n_chunks + c_idx) * g.H : nullptr;
    for (int j = threadIdx.x; j < c.Tc; j += blockDim.x) {
        float m = 0.0f;
        for (int h = 0; h < g.H; h++) {
            const float v = imp[((long long)layer * g.H + h) * g.T + c.start + j];
            if (sh) m = m + sh[h] * v;
            else if (v > m) m = v;
        }
        if (wts) m *= wts[c.start + j];
        gimp[(long long)layer * g.T + c.start + j] = m;
    }
}

// ---------------------------------------------------------------------------
// Top-t selection (api.cpp:716-744): the set std::partial_sort keeps under
// "greater importance first", written ascending. Without NaN and without a
// tie across the boundary that set is every candidate at or above the t-th
// largest importance, found by a block-wide bitwise search; otherwise
// libstdc++'s heap selection, restated here so that boundary ties resolve to
// the same members, runs on lane 0 over LDS copies (or global scratch for
// chunks beyond the LDS budget). grid = (n_chunks, L).
// ---------------------------------------------------------------------------
__device__ __forceinline__ bool heap_less(const float * imp, int a, int b) { return imp[a] > imp[b]; }

__device__ void heap_push(int * h, const float * imp, int hole, int top, int val) {
    int parent = (hole - 1) / 2;
    while (hole > top && heap_less(imp, h[parent], val)) {
        h[hole] = h[parent];
        hole = parent;
        parent = (hole - 1) / 2;
    }
    h[hole] = val;
}

__device__ void heap_adjust(int * h, const float * imp, int hole, int len, int val) {
    const int top = hole;
    int child = hole;
    while (child < (len - 1) / 2) {
        child = 2 * (child + 1);
        if (heap_less(imp, h[child], h[child - 1])) child--;
        h[hole] = h[child];
        hole = child;
    }
    if ((len & 1) == 0 && child == (len - 2) / 2) {
        child = 2 * (child + 1);
        h[hole] = h[child - 1];
        hole = child - 1;
    }
    heap_push(h, imp, hole, top, val);
}

__device__ void heap_select(int * a, int k, int n, const float * imp) {
    if (k >= 2) {
        int parent = (k - 2) / 2;
        for (;;) {
            const int v = a[parent];
            heap_adjust(a, imp, parent, k, v);
            if (parent == 0) break;
            parent--;
        }
    }
    for (int i = k; i < n; i++) {
        if (heap_less(imp, a[i], a[0])) {
            const int v = a[i];
            a[i] = a[0];
            heap_adjust(a, imp, 0, k, v);
        }
    }
}

// ascending write-out of flagged positions: block prefix sum over flags
__device__ void write_flagged(const unsigned char * fl, int n, int base, int * out) {
    __shared__ int wsum[16];
    __shared__ int carry;
    if (threadIdx.x == 0) carry = 0;
    __syncthreads();
    for (int j0 = 0; j0 < n; j0 += blockDim.x) {
        const int j = j0 + threadIdx.x;
        const int f = (j < n) ? (int)fl[j] : 0;
        int x = f;
        const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
        for (int o = 1; o < 64; o <<= 1) {
            const int y = __shfl_up(x, o);
            if (lane >= o) x += y;
        }
        if (lane == 63) wsum[w] = x;
        __syncthreads();
        int pre = carry;
        for (int i = 0; i < w; i++) pre += wsum[i];
        if (f) out[pre + x - 1] = base + j;
        __syncthreads();
        if (threadIdx.x == 0) {
            int tot = 0;
            for (int i = 0; i < (int)(blockDim.x >> 6); i++) tot += wsum[i];
            carry += tot;
        }
        __syncthreads();
    }
}

__global__ void __launch_bounds__(256)
k_select_topk(Geom g, const ChunkDesc * __restrict__ chunks, const float * __restrict__ gimp,
              int * __restrict__ cand_g, unsigned char * __restrict__ flags_g, int * __restrict__ sel,
              int lds_ok) {
    extern __shared__ unsigned char smem[];
    const int c_idx = blockIdx.x, layer = blockIdx.y;
    const ChunkDesc c = chunks[c_idx];
    const long long unit = (long long)layer * g.n_chunks + c_idx;
    const float * im_g = gimp + (long long)layer * g.T + c.start;
    const int pc = min(c.prefix, c.tc);
    const int rem = c.tc - pc;
    const int nc = c.Tc - pc;
    float * im;
    int * cand;
    unsigned char * fl;
    if (lds_ok) {
        im = reinterpret_cast<float *>(smem);
        cand = reinterpret_cast<int *>(smem + sizeof(float) * g.Tc_max);
        fl = smem + (sizeof(float) + sizeof(int)) * g.Tc_max;
        for (int j = threadIdx.x; j < c.Tc; j += blockDim.x) im[j] = im_g[j];
    } else {
        im = const_cast<float *>(im_g);
        cand = cand_g + unit * g.Tc_max;
        fl = flags_g + unit * g.Tc_max;
    }
    for (int j = threadIdx.x; j < nc; j += blockDim.x) cand[j] = pc + j;
    for (int j = threadIdx.x; j < c.Tc; j += blockDim.x) fl[j] = (j < pc) ? 1 : 0;
    __syncthreads();
    // The set a partial sort keeps is fixed by value unless the boundary
    // value ties: find the rem-th largest order key K (-0 counted as +0, the
    // comparator's equality) by a bitwise search over block counts; when no
    // candidate is NaN and exactly rem candidates reach K, they are the set.
    // Otherwise (NaN, or a tie across the boundary) the heap selection
    // decides which of the tied keys stay.
    bool fast = false;
    if (rem > 0) {
        __shared__ int s_wc[4];
        auto okey = [](float v) {
            const unsigned u = __float_as_uint(v == 0.0f ? 0.0f : v);
            return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
        };
        // candidates with key >= kt (nan: with a NaN importance instead)
        auto count = [&](unsigned kt, bool nan) {
            int cnt = 0;
            for (int j0 = 0; j0 < nc; j0 += blockDim.x) {
                const int j = j0 + threadIdx.x;
                const float v = j < nc ? im[pc + j] : 0.0f;
                const bool pr = j < nc && (nan ? v != v : okey(v) >= kt);
                cnt += __popcll(__ballot(pr));
            }
            if ((threadIdx.x & 63) == 0) s_wc[threadIdx.x >> 6] = cnt;
            __syncthreads();
            int tot = 0;
            for (int i = 0; i < (int)(blockDim.x >> 6); i++) tot += s_wc[i];
            __syncthreads();
            return tot;
        };
        if (count(0u, true) == 0) {
            unsigned K = 0u;
            for (int b = 31; b >= 0; b--) {
                const unsigned kt = K | (1u << b);
                if (count(kt, false) >= rem) K = kt;
            }
            fast = count(K, false) == rem;
            if (fast)
                for (int j = threadIdx.x; j < nc; j += blockDim.x)
                    if (okey(im[pc + j]) >= K) fl[pc + j] = 1;
        }
    }
    if (!fast) {
        if (threadIdx.x == 0 && rem > 0) heap_select(cand, rem, nc, im);
        __syncthreads();
        for (int j = threadIdx.x; j < rem; j += blockDim.x) fl[cand[j]] = 1;
    }
    __syncthreads();
    write_flagged(fl, c.Tc, c.start, sel + (long long)layer * g.t_total + c.off);
}


// ---------------------------------------------------------------------------
// Diversity selection (api.cpp:175-233). The reference's greedy pass picks,
// t - prefix times, the unused key of largest imp_j * (1 - s * pen_j) (first
// index on ties, scores must beat -1e30), then raises every unused key's
// penalty to its cosine with the pick, over the full H*d_k key row:
//   cos = dot(k_b, k_j) / ((sqrtf(|k_b|^2) + 1e-8) * sqrtf(|k_j|^2) + 1e-8),
// all sums sequential over the row. A sequential dot product is symmetric bit
// for bit (a*b == b*a), and |k_j|^2 is the Gram diagonal, so every value the
// pass needs is an entry of the candidates' Gram matrix.
//
// Pruning: while fewer than t keys are used, one of the t most important keys
// is unused, so the pick's score is at least about (1 - s) I_t (I_t = t-th
// largest importance) and at most its own importance (1 - s*pen <= 1). Keys
// below alpha * I_t are left out; the greedy pass then checks at every step
// that its pick beats the largest pruned importance (which bounds every pruned
// key's score) and flags the unit for a wider level otherwise, so the result
// is exact whatever alpha is.
// ---------------------------------------------------------------------------

// candidates of one (layer, chunk): ascending positions of the unused keys
// with importance >= alpha * I_t; grid (n_chunks, L), 256 threads
constexpr int DC_LDS = 4096;
__global__ void __launch_bounds__(256)
k_div_candidates(Geom g, const ChunkDesc * __restrict__ chunks, const float * __restrict__ gimp, DivWork dw,
                 int * __restrict__ cand_all) {
    const int c_idx = blockIdx.x, layer = blockIdx.y;
    const int unit = layer * g.n_chunks + c_idx;
    if (dw.gslot[unit] < 0) return;
    const ChunkDesc c = chunks[c_idx];
    const float * im = gimp + (long long)layer * g.T + c.start;
    const int pc = min(c.prefix, c.tc);
    const int need = c.tc - pc;
    const int tid = threadIdx.x;
    __shared__ int s_bad;
    __shared__ int wsum[4];
    __shared__ float s_im[DC_LDS];
    if (need <= 0) {   // the prefix fills the chunk: no greedy step
        if (tid == 0) {
            dw.maxnc[unit] = -INFINITY;
            dw.count[unit] = 0;
            dw.state[unit] = DIV_PENDING;
        }
        return;
    }
    if (tid == 0) s_bad = 0;
    __syncthreads();
    // pruning needs finite, non-negative importance and 0 <= s < 1
    float thr = -INFINITY;
    bool prune = dw.alpha > 0.0f && dw.strength >= 0.0f && dw.strength < 1.0f;
    if (prune) {
        for (int j = tid; j < c.Tc; j += blockDim.x) {
            const float v = im[j];
            if (!(v >= 0.0f && v <= 3.0e38f)) s_bad = 1;
        }
        __syncthreads();
        prune = s_bad == 0;
    }
    if (prune) {
        // I_t: the largest bit pattern x with #(imp >= x) >= tc (order of
        // non-negative floats = order of their bits), by bisection over
        // block counts (a ballot per wave, the waves' counts through LDS;
        // every thread takes the same bounds); the chunk's importances staged
        // in LDS when they fit
        const float * src = im;
        if (c.Tc <= DC_LDS) {
            for (int j = tid; j < c.Tc; j += blockDim.x) s_im[j] = im[j];
            __syncthreads();
            src = s_im;
        }
        unsigned lo = 0u, hi = 0x7f7fffffu;
        for (int it = 0; it < 32 && lo < hi; it++) {
            const unsigned mid = lo + (hi - lo + 1u) / 2u;
            int cnt = 0;
            for (int j0 = 0; j0 < c.Tc; j0 += blockDim.x) {
                const int j = j0 + tid;
                cnt += __popcll(__ballot(j < c.Tc && __float_as_uint(src[j < c.Tc ? j : 0]) >= mid));
            }
            if ((tid & 63) == 0) wsum[tid >> 6] = cnt;
            __syncthreads();
            const int tot = wsum[0] + wsum[1] + wsum[2] + wsum[3];
            __syncthreads();
            if (tot >= c.tc) lo = mid; else hi = mid - 1u;
        }
        thr = __uint_as_float(lo) * dw.alpha;
    }
    // flags, the largest pruned importance, then an ascending write-out
    int * cand = cand_all + (long long)unit * g.Tc_max;
    __shared__ int carry;
    if (tid == 0) carry = 0;
    __syncthreads();
    float mnc = -INFINITY;
    for (int j0 = 0; j0 < c.Tc; j0 += blockDim.x) {
        const int j = j0 + tid;
        int f = 0;
        if (j < c.Tc && j >= pc) {
            const float v = im[j];
            if (!prune || v >= thr) f = 1;
            else if (v > mnc) mnc = v;
        }
        const int lane = tid & 63, w = tid >> 6;
        const unsigned long long m = __ballot(f);
        const int pre_l = __popcll(m & ((1ull << lane) - 1ull));
        if (lane == 0) wsum[w] = __popcll(m);
        __syncthreads();
        int pre = carry;
        for (int i = 0; i < w; i++) pre += wsum[i];
        const int pos = pre + pre_l;
        if (f && pos < dw.cap) cand[pos] = j;
        __syncthreads();
        if (tid == 0) carry += wsum[0] + wsum[1] + wsum[2] + wsum[3];
        __syncthreads();
    }
    // block max of the pruned importances (non-negative or -inf)
    for (int o = 32; o > 0; o >>= 1) {
        const float y = __shfl_xor(mnc, o);
        if (y > mnc) mnc = y;
    }
    if ((tid & 63) == 0) wsum[tid >> 6] = __float_as_int(mnc);
    __syncthreads();
    if (tid == 0) {
        float m = -INFINITY;
        for (int i = 0; i < 4; i++) {
            const float y = __int_as_float(wsum[i]);
            if (y > m) m = y;
        }
        dw.maxnc[unit] = m;
        dw.count[unit] = carry;
        dw.state[unit] = (carry > dw.cap) ? DIV_RETRY : DIV_PENDING;
    }
}

// Gram matrix of one unit's candidates over the full key row (length H*d_k),
// each entry a sequential dot product. Tiles of 64 x 64 above the diagonal
// (mirrored on write); 256 threads, each 4 x 4 entries. A diagonal tile needs
// only its 136 sub-tiles on or above the diagonal: there threads 0..135 take
// them in order and the others only help stage the slabs (a wave with no
// sub-tile skips the sums). grid (8 ceil(units / 8) tile pairs), XCD-grouped.
constexpr int DG_TILE = 64, DG_SLAB = 32;

template <int KC>   // 0, or the codec of a quantized K read in place (g.kc)
__global__ void __launch_bounds__(256)
k_div_gram(Geom g, const ChunkDesc * __restrict__ chunks, const float * __restrict__ K, DivWork dw,
           const int * __restrict__ cand_all) {
    // The blocks of one unit are dealt to one XCD back to back (the
    // dispatcher gives consecutive blocks to the 8 XCDs in turn), so the
    // unit's candidate rows, which every tile pair re-reads, come from that
    // XCD's L2: block b is unit 8 (s / npairs) + b % 8, pair s % npairs,
    // s = b / 8. (In unit-major order the pairs of a unit ran far apart and
    // re-read their rows from HBM: 16 GB per step against 9 GB.)
    const int nt = (dw.cap + DG_TILE - 1) / DG_TILE, npairs = nt * (nt + 1) / 2;
    const int seq = blockIdx.x >> 3;
    const int unit = (seq / npairs) * 8 + (blockIdx.x & 7);
    if (unit >= g.L * g.n_chunks) return;
    const int slot = dw.gslot[unit];
    if (slot < 0 || dw.state[unit] != DIV_PENDING) return;
    const int C = dw.count[unit];
    // tile pair (ti <= tj) from the linear index
    int ti = 0, rem = seq % npairs;
    while (rem >= nt - ti) { rem -= nt - ti; ti++; }
    const int tj = ti + rem;
    if (ti * DG_TILE >= C || tj * DG_TILE >= C) return;
    const int layer = unit / g.n_chunks, c_idx = unit % g.n_chunks;
    const ChunkDesc c = chunks[c_idx];
    const int E = g.H * g.dk;
    const int * cand = cand_all + (long long)unit * g.Tc_max;
    constexpr bool kcod = KC != 0;   // rows of a quantized K, decoded in registers
    const float * Kl = kcod ? nullptr : K + (long long)layer * g.ldK + (long long)c.start * E;
    __shared__ __align__(16) float As[DG_SLAB][DG_TILE + 4];
    __shared__ __align__(16) float Bs[DG_SLAB][DG_TILE + 4];
    // rows from tile ta, columns from tile tb: the partial last tile, if in
    // the pair, gives the rows, so that a wave whose rows are all past C
    // skips the sums (the entries go out both ways, so the orientation is free)
    const bool swp = ti < tj && (tj + 1) * DG_TILE > C;
    const int ta = swp ? tj : ti, tb = swp ? ti : tj;
    const int tid = threadIdx.x;
    int tx = tid & 15, ty = tid >> 4;
    bool work = true;
    if (ti == tj) {
        // sub-tile k = tid of the upper triangle, row by row: row y holds 16 - y
        int k = tid, y = 0;
        while (y < 16 && k >= 16 - y) { k -= 16 - y; y++; }
        work = y < 16;
        ty = work ? y : 0;
        tx = work ? y + k : 0;
    }
    work = work && ta * DG_TILE + 4 * ty < C;
    const bool wave_work = __builtin_amdgcn_readfirstlane(__ballot(work) != 0ull) != 0;
    // loader: row lr of the tile, dims lq*8 .. lq*8+7 of the slab
    const int lr = tid >> 2, lq = tid & 3;
    const int ra = ta * DG_TILE + lr, rb = tb * DG_TILE + lr;
    const long long rra = c.start + cand[ra < C ? ra : C - 1], rrb = c.start + cand[rb < C ? rb : C - 1];
    const float * pa = kcod ? nullptr : Kl + (rra - c.start) * E + lq * 8;
    const float * pb = kcod ? nullptr : Kl + (rrb - c.start) * E + lq * 8;
    // (a quantized row holds whole 32-element blocks: E is a multiple of 32)
    const bool vec = kcod || ((E & 3) == 0 && (reinterpret_cast<uintptr_t>(Kl) & 15) == 0);
    float acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
        for (int j = 0; j < 4; j++) acc[i][j] = 0.0f;
    for (int d0 = 0; d0 < E; d0 += DG_SLAB) {
        float va[8], vb[8];
        if (vec && d0 + DG_SLAB <= E) {
            float4 a0, a1, b0, b1;
            if (kcod) {
                const int e0 = d0 + lq * 8;
                a0 = codec_load4<KC>(g.kc, layer, rra, e0); a1 = codec_load4<KC>(g.kc, layer, rra, e0 + 4);
                b0 = codec_load4<KC>(g.kc, layer, rrb, e0); b1 = codec_load4<KC>(g.kc, layer, rrb, e0 + 4);
            } else {
                a0 = *reinterpret_cast<const float4 *>(pa + d0); a1 = *reinterpret_cast<const float4 *>(pa + d0 + 4);
                b0 = *reinterpret_cast<const float4 *>(pb + d0); b1 = *reinterpret_cast<const float4 *>(pb + d0 + 4);
            }
            va[0] = a0.x; va[1] = a0.y; va[2] = a0.z; va[3] = a0.w; va[4] = a1.x; va[5] = a1.y; va[6] = a1.z; va[7] = a1.w;
            vb[0] = b0.x; vb[1] = b0.y; vb[2] = b0.z; vb[3] = b0.w; vb[4] = b1.x; vb[5] = b1.y; vb[6] = b1.z; vb[7] = b1.w;
        } else {
#pragma unroll
            for (int u = 0; u < 8; u++) {
                const int d = d0 + lq * 8 + u;
                va[u] = d < E ? pa[d0 + u] : 0.0f;
                vb[u] = d < E ? pb[d0 + u] : 0.0f;
            }
        }
        __syncthreads();
#pragma unroll
        for (int u = 0; u < 8; u++) {
            As[lq * 8 + u][lr] = va[u];
            Bs[lq * 8 + u][lr] = vb[u];
        }
        __syncthreads();
        const int dn = wave_work ? min(DG_SLAB, E - d0) : 0;
        for (int dd = 0; dd < dn; dd++) {
            const float4 a = *reinterpret_cast<const float4 *>(&As[dd][ty * 4]);
            const float4 b = *reinterpret_cast<const float4 *>(&Bs[dd][tx * 4]);
            const float av[4] = {a.x, a.y, a.z, a.w}, bv[4] = {b.x, b.y, b.z, b.w};
#pragma unroll
            for (int i = 0; i < 4; i++)
#pragma unroll
                for (int j = 0; j < 4; j++) acc[i][j] = acc[i][j] + av[i] * bv[j];
        }
    }
    float * G = dw.G + (long long)slot * dw.cap * dw.cap;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const int r = ta * DG_TILE + ty * 4 + i;
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const int q = tb * DG_TILE + tx * 4 + j;
            if (work && r < C && q < C) {
                G[(long long)r * dw.cap + q] = acc[i][j];
                G[(long long)q * dw.cap + r] = acc[i][j];
            }
        }
    }
}

// The greedy pass of one unit, one wave; candidate position p sits in lane
// p % 64, slot p / 64 (NS slots: the level's capacity is at most 64 NS).
// grid (units).
template <int NS>
__global__ void __launch_bounds__(64)
k_div_greedy(Geom g, const ChunkDesc * __restrict__ chunks, const float * __restrict__ gimp, DivWork dw,
             const int * __restrict__ cand_all, int * __restrict__ sel) {
    const int unit = blockIdx.x;
    const int slot_g = dw.gslot[unit];
    if (slot_g < 0 || dw.state[unit] != DIV_PENDING) return;
    const int layer = unit / g.n_chunks, c_idx = unit % g.n_chunks;
    const ChunkDesc c = chunks[c_idx];
    const int lane = threadIdx.x;
    const int pc = min(c.prefix, c.tc);
    const int need = c.tc - pc;
    const int C = dw.count[unit];
    const float s = dw.strength, maxnc = dw.maxnc[unit];
    const float * im = gimp + (long long)layer * g.T + c.start;
    const int * cand = cand_all + (long long)unit * g.Tc_max;
    const float * G = dw.G + (long long)slot_g * dw.cap * dw.cap;
    __shared__ unsigned char taken[DIV_MAX_CAND];   // by candidate position
    float imp[NS], pen[NS], sqn[NS], gv[NS];
    unsigned live = 0;   // bit k: slot k holds an unused candidate
    // Loads sit under wave-uniform slot guards with clamped indices, never
    // under a per-lane branch: a load inside a divergent branch is waited for
    // before the branch ends, which would serialize one memory round trip per
    // slot. Lanes past the candidates read a valid entry and discard it.
    const int nsl = (C + 63) >> 6;   // slots holding candidates
    int ci[NS];
#pragma unroll
    for (int k = 0; k < NS; k++) {
        const int p = min(lane + 64 * k, C - 1);
        ci[k] = k < nsl ? cand[p] : 0;
        gv[k] = k < nsl ? G[(long long)p * dw.cap + p] : 0.0f;
    }
#pragma unroll
    for (int k = 0; k < NS; k++) {
        const int p = lane + 64 * k;
        const bool v = p < C;
        const float x = k < nsl ? im[ci[k]] : 0.0f;
        imp[k] = v ? x : 0.0f;
        sqn[k] = v ? sqrtf(gv[k]) : 0.0f;
        pen[k] = 0.0f;
        if (v) live |= 1u << k;
        taken[p] = 0;
    }
    __builtin_amdgcn_wave_barrier();
    int state = DIV_DONE;
    for (int step = 0; step < need; step++) {
        float bs = -1e30f;
        int bp = -1;
#pragma unroll
        for (int k = 0; k < NS; k++) {
            if (k < nsl) {
                const float sc = imp[k] * (1.0f - s * pen[k]);
                if (((live >> k) & 1u) && sc > bs) { bs = sc; bp = lane + 64 * k; }
            }
        }
        const unsigned kmax = dpp_reduce_u32<true>(bp >= 0 ? score_key(bs) : 0u);
        const unsigned pmin = dpp_reduce_u32<false>((bp >= 0 && score_key(bs) == kmax) ? (unsigned)bp : 0xffffffffu);
        if (pmin == 0xffffffffu) { state = DIV_SHORT; break; }
        const int b = (int)pmin;
        const float best = __shfl(bs, b & 63);
        // a pruned key could have won only if its importance reaches the pick's score
        if (!(best > maxnc)) { state = DIV_RETRY; break; }
        if (lane == (b & 63)) {
            live &= ~(1u << (b >> 6));
            taken[b] = 1;
        }
        const float * Gb = G + (long long)b * dw.cap;
#pragma unroll
        for (int k = 0; k < NS; k++) gv[k] = k < nsl ? Gb[min(lane + 64 * k, C - 1)] : 0.0f;
        const float nsel = sqrtf(Gb[b]) + 1e-8f;
        // every slot's quotient is formed (no divergent branch); only unused
        // candidates take it
#pragma unroll
        for (int k = 0; k < NS; k++) {
            if (k < nsl) {
                const float cs = gv[k] / (nsel * sqn[k] + 1e-8f);
                if (((live >> k) & 1u) && cs > pen[k]) pen[k] = cs;
            }
        }
    }
    if (lane == 0) dw.state[unit] = state;
    if (state != DIV_DONE) return;
    __builtin_amdgcn_wave_barrier();
    // kept positions ascending: the prefix, then the picks in position order
    int * out = sel + (long long)layer * g.t_total + c.off;
    for (int j = lane; j < pc; j += 64) out[j] = c.start + j;
    int base = pc;
    for (int p0 = 0; p0 < C; p0 += 64) {
        const int p = p0 + lane;
        const int f = (p < C) ? (int)taken[p] : 0;
        const unsigned long long m = __ballot(f);
        if (f) out[base + __popcll(m & ((1ull << lane) - 1ull))] = c.start + cand[p];
        base += __popcll(m);
    }
}

// ---------------------------------------------------------------------------
// One refinement round's decision per (layer, chunk) (api.cpp:851-903).
// key_value[j] = sum_h (sum_qi X_h[qi][j]^2) / n_q, X = the current compacted
// softmax (the reference recomputes it per slot: same values). The worst slot
// is the first minimum (slot 0 when key_value[0] is NaN); the best unused
// position is the first maximum of the global importance above -1 among the
// unkept ones. The round stops the unit (for good) when there is none or when
// it is not above half the worst slot's importance; otherwise the worst kept
// position is replaced and the kept list stays ascending. grid (n_chunks, L).
// ---------------------------------------------------------------------------
__device__ __forceinline__ void block_argbest(unsigned key, int idx, bool want_max, unsigned & k_out, int & i_out) {
    // best key (max or min), smallest index among equal keys; 256 threads
    __shared__ unsigned rk[4];
    __shared__ int ri[4];
    unsigned k = want_max ? dpp_reduce_u32<true>(key) : dpp_reduce_u32<false>(key);
    const unsigned i = dpp_reduce_u32<false>(key == k ? (unsigned)idx : 0xffffffffu);
    if ((threadIdx.x & 63) == 0) { rk[threadIdx.x >> 6] = k; ri[threadIdx.x >> 6] = (int)i; }
    __syncthreads();
    unsigned bk = rk[0];
    int bi = ri[0];
    for (int wv = 1; wv < (int)(blockDim.x >> 6); wv++) {
        const bool better = want_max ? (rk[wv] > bk) : (rk[wv] < bk);
        if (better || (rk[wv] == bk && (unsigned)ri[wv] < (unsigned)bi)) { bk = rk[wv]; bi = ri[wv]; }
    }
    __syncthreads();
    k_out = bk;
    i_out = bi;
}

__global__ void __launch_bounds__(256)
k_refine_step(Geom g, const ChunkDesc * __restrict__ chunks, const float * __restrict__ X,
              const float * __restrict__ gimp, int * __restrict__ sel, unsigned char * __restrict__ flags_all,
              int * __restrict__ active) {
    const int c_idx = blockIdx.x, layer = blockIdx.y;
    const int unit = layer * g.n_chunks + c_idx;
    if (!active[unit]) return;
    const ChunkDesc c = chunks[c_idx];
    const int t = c.tc, nq = c.nq, tid = threadIdx.x;
    if (t >= c.Tc || t <= 0) {
        if (tid == 0) active[unit] = 0;
        return;
    }
    int * sl = sel + (long long)layer * g.t_total + c.off;
    const float * gi = gimp + (long long)layer * g.T;
    unsigned char * fl = flags_all + (long long)unit * g.Tc_max;
    const long long hsX = (long long)g.nq_max * g.t_total;
    // worst slot
    unsigned wk = 0xffffffffu;
    int wi = 0x7fffffff;
    __shared__ int s_kv0_nan;
    for (int j = tid; j < t; j += blockDim.x) {
        float kv = 0.0f;
        for (int h = 0; h < g.H; h++) {
            const float * xh = X + (long long)layer * g.H * hsX + h * hsX + c.off + j;
            float e = 0.0f;
            for (int qi = 0; qi < nq; qi++) {
                const float x = xh[(long long)qi * g.t_total];
                e = e + x * x;
            }
            kv = kv + e / (float)nq;
        }
        if (j == 0) s_kv0_nan = (kv != kv) ? 1 : 0;
        if (kv == kv) {
            const unsigned k = score_key(kv);
            if (k < wk) { wk = k; wi = j; }
        }
    }
    unsigned bk;
    int worst;
    block_argbest(wk, wi, false, bk, worst);
    if (s_kv0_nan || worst == 0x7fffffff) worst = 0;
    // best unused position
    for (int j = tid; j < c.Tc; j += blockDim.x) fl[j] = 0;
    __syncthreads();
    for (int k = tid; k < t; k += blockDim.x) fl[sl[k] - c.start] = 1;
    __syncthreads();
    unsigned uk = 0u;
    int ui = 0x7fffffff;
    for (int j = tid; j < c.Tc; j += blockDim.x) {
        const float v = gi[c.start + j];
        if (!fl[j] && v > -1.0f) {
            const unsigned k = score_key(v);
            if (k > uk) { uk = k; ui = j; }
        }
    }
    int best;
    block_argbest(uk, ui, true, bk, best);
    if (tid == 0) {
        if (bk == 0u) best = -1;
        const int wpos = sl[worst];
        if (best < 0 || gi[c.start + best] <= gi[wpos] * 0.5f) {
            active[unit] = 0;
        } else {
            const int np = c.start + best;
            for (int k = worst; k < t - 1; k++) sl[k] = sl[k + 1];
            int k = t - 1;
            while (k > 0 && sl[k - 1] > np) { sl[k] = sl[k - 1]; k--; }
            sl[k] = np;
        }
    }
}

// ---------------------------------------------------------------------------
// Least-squares system per (chunk, head): X = softmax_rows(S[:, sel] + beta)
// (api.cpp:833-840); aug = [X^T X + ridge I | X^T Y] (math.h:465-504),
// both sums sequential over the query index.
// ---------------------------------------------------------------------------
// Up to 32 rows x t_c columns at a time in LDS: gather S[:, sel] + beta, row
// maxima (one wave per row, the reference's scan semantics), exponentials,
// the sequential row sums (one thread per row over LDS), then X = e * inv.
// The dynamic LDS holds the chunk's selection and beta (2 t_c floats), then
// the rows at a stride of t_c + 1 floats; it is sized for the largest chunk
// (at most LSX_LDS_BYTES), and a chunk for which not even one row fits goes
// row by row through global memory.
constexpr int LSX_ROWS = 32, LSX_LDS_BYTES = 60 * 1024;

__host__ __device__ inline int lsx_rows(int t, int lds_floats) {
    return min(LSX_ROWS, (lds_floats - 2 * t) / (t + 1));
}

__global__ void __launch_bounds__(256)
k_ls_softmax(Geom g, const ChunkDesc * __restrict__ chunks, const float * __restrict__ S,
             const int * __restrict__ sel, const float * __restrict__ beta, float * __restrict__ X,
             int lds_floats, const float * __restrict__ Ssel) {
    const int c_idx = blockIdx.x / g.H, h = blockIdx.x % g.H, layer = blockIdx.y;
    const ChunkDesc c = chunks[c_idx];
    const int t = c.tc, nq = c.nq;
    // S[:, sel] from the main scores, or (Ssel) the kept keys' own scores:
    // row r of the chunk's kept key j at Sr[r * srs + sj]
    const float * Sh = Ssel ? Ssel + ((long long)layer * g.H + h) * g.nq_max * g.t_total + c.off
                            : S + layer * lS(g) + h * hS(g);
    const long long srs = Ssel ? g.t_total : g.T;
    const int * sl = sel + (long long)layer * g.t_total + c.off;
    const float * bh = beta + ((long long)layer * g.H + h) * g.t_total + c.off;
    const long long hsX = (long long)g.nq_max * g.t_total;
    float * Xh = X + (long long)layer * g.H * hsX + h * hsX + c.off;
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    __shared__ uint64_t etab[32];
    if (tid < 32) etab[tid] = c_exp2_tab[tid];   // visible after the barriers below
    const int rows = lsx_rows(t, lds_floats);
    if (rows < 1) {
        // large chunks: row by row through global memory
        __shared__ float red[16];
        __shared__ float rmax1, rinv1;
        for (int r = 0; r < nq; r++) {
            float * xr = Xh + (long long)r * g.t_total;
            const float * sr = Sh + (long long)r * srs;
            for (int j = tid; j < t; j += blockDim.x) xr[j] = sr[Ssel ? j : sl[j]] + bh[j];
            __syncthreads();
            const float m = ref_row_max(xr, t, red);
            if (tid == 0) rmax1 = m;
            __syncthreads();
            for (int j = tid; j < t; j += blockDim.x) xr[j] = expf_ref(xr[j] - rmax1, etab);
            __syncthreads();
            if (tid == 0) {
                float sum = 0.0f;
                for (int j = 0; j < t; j++) sum += xr[j];
                rinv1 = 1.0f / (sum + 1e-12f);
            }
            __syncthreads();
            for (int j = tid; j < t; j += blockDim.x) xr[j] = xr[j] * rinv1;
            __syncthreads();
        }
        return;
    }
    extern __shared__ float lsx_dyn[];
    __shared__ float rmax[LSX_ROWS], rinv[LSX_ROWS];
    int * sls = reinterpret_cast<int *>(lsx_dyn);
    float * bs = lsx_dyn + t;
    float * xs = lsx_dyn + 2 * t;
    const int ld = t + 1;
    for (int j = tid; j < t; j += blockDim.x) {
        sls[j] = Ssel ? j : sl[j];
        bs[j] = bh[j];
    }
    __syncthreads();
    for (int r0 = 0; r0 < nq; r0 += rows) {
        const int nr = min(rows, nq - r0);
        // gather: all rows' loads per thread in flight (at clamped rows: in
        // bounds, the extra ones unused); the LDS caps the block count, so
        // these registers cost no occupancy
        for (int j = tid; j < t; j += blockDim.x) {
            const int sj = sls[j];
            const float bj = bs[j];
            float v[LSX_ROWS];
#pragma unroll
            for (int u = 0; u < LSX_ROWS; u++) v[u] = Sh[(long long)(r0 + min(u, nr - 1)) * srs + sj];
#pragma unroll
            for (int u = 0; u < LSX_ROWS; u++)
                if (u < nr) xs[u * ld + j] = v[u] + bj;
        }
        __syncthreads();
        // maxima: largest non-NaN value, NaN when the first entry is NaN,
        // else the first entry unless a value exceeds it
        for (int r = wv; r < nr; r += 4) {
            float m = -INFINITY;
            for (int j = lane; j < t; j += 64) {
                const float v = xs[r * ld + j];
                if (v == v && v > m) m = v;
            }
            const unsigned k = dpp_reduce_u32<true>(score_key(m));
            const float mm = __uint_as_float((k & 0x80000000u) ? (k & 0x7fffffffu) : ~k);
            const float a0 = xs[r * ld];
            if (lane == 0) rmax[r] = (a0 != a0) ? a0 : ((mm > a0) ? mm : a0);
        }
        __syncthreads();
        for (int r = 0; r < nr; r++)
            for (int j = tid; j < t; j += blockDim.x) xs[r * ld + j] = expf_ref(xs[r * ld + j] - rmax[r], etab);
        __syncthreads();
        if (tid < nr) {
            float sum = 0.0f;
            int j = 0;
            for (; j + 16 <= t; j += 16) {   // 16 reads in flight, then the adds in order
                float e[16];
#pragma unroll
                for (int k = 0; k < 16; k++) e[k] = xs[tid * ld + j + k];
#pragma unroll
                for (int k = 0; k < 16; k++) sum += e[k];
            }
            for (; j < t; j++) sum += xs[tid * ld + j];
            rinv[tid] = 1.0f / (sum + 1e-12f);
        }
        __syncthreads();
        for (int r = 0; r < nr; r++) {
            const float iv = rinv[r];
            float * xr = Xh + (long long)(r0 + r) * g.t_total;
            for (int j = tid; j < t; j += blockDim.x) xr[j] = xs[r * ld + j] * iv;
        }
        __syncthreads();
    }
}

// beta fit input (api.cpp:812-831): M[k][j] = exp_scores[k][sel[j]] per
// (chunk, head), written in the compacted-softmax layout [L][H][nq][t_total]
__global__ void __launch_bounds__(256)
k_gather_exp(Geom g, const ChunkDesc * __restrict__ chunks, const float * __restrict__ E,
             const int * __restrict__ sel, float * __restrict__ M) {
    const int c_idx = blockIdx.x / g.H, h = blockIdx.x % g.H, layer = blockIdx.y;
    const ChunkDesc c = chunks[c_idx];
    const float * Eh = E + layer * lS(g) + h * hS(g);
    const int * sl = sel + (long long)layer * g.t_total + c.off;
    const long long hsX = (long long)g.nq_max * g.t_total;
    float * Mh = M + (long long)layer * g.H * hsX + h * hsX + c.off;
    for (int e = threadIdx.x; e < c.nq * c.tc; e += blockDim.x) {
        const int k = e / c.tc, j = e % c.tc;
        Mh[(long long)k * g.t_total + j] = Eh[(long long)k * g.T + sl[j]];
    }
}

// beta = logf(max(1e-12, w)) after the solvers' final clamp w < 1e-12 -> 1e-12
// (math.h:449-451, math.h:755-757, api.cpp:829). The clamp keeps NaN and
// std::max then returns 1e-12 for it, so together: w >= 1e-12 ? w : 1e-12.
// (Written as one comparison: the two selects in sequence were folded into
// the first alone, which keeps NaN.)
__global__ void __launch_bounds__(256)
k_beta_log(float * __restrict__ wb, long long n) {
    const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    const float w = wb[i];
    const float m = (w >= 1e-12f) ? w : 1e-12f;
    wb[i] = logf_ref(m);
}

// ---------------------------------------------------------------------------
// Lawson-Hanson NNLS for the beta weights (math.h:283-452), one wave per
// (layer, chunk, head). Input: aug = [AtA | Atb] (column-major n x (n+1), no
// ridge). The active-set loop is the reference's, step for step: the entering
// variable is the first largest -grad over the zero set; each inner pass
// solves the passive-set normal equations (+1e-10 on the diagonal) by
// Gaussian elimination with partial pivoting in LDS (rows r, r + 64 in lane r),
// interpolates back to the boundary when infeasible, and the gradient is
// AtA w - Atb with sequential sums. Writes w (the clamp and log follow in
// k_beta_log). Passive sets beyond LH_PMAX set *status (the host then
// refuses the call). n <= 256: lane l owns variables l, l+64, l+128, l+192.
// ---------------------------------------------------------------------------
constexpr int LH_PMAX = 128;   // passive-set capacity: rows lane and lane + 64 of the sub-problem

__global__ void __launch_bounds__(64)
k_nnls_lh(Geom g, const ChunkDesc * __restrict__ chunks, const float * __restrict__ aug,
          const long long * __restrict__ aug_off, float * __restrict__ wout, int max_iter, int * __restrict__ status) {
    const int c_idx = blockIdx.x / g.H, h = blockIdx.x % g.H, layer = blockIdx.y;
    const ChunkDesc c = chunks[c_idx];
    const int n = c.tc;
    const int lane = threadIdx.x;
    float * wo = wout + ((long long)layer * g.H + h) * g.t_total + c.off;
    if (n > 256) return;   // refused on the host
    const float * Ag = aug + aug_off[((long long)layer * g.n_chunks + c_idx) * g.H + h];
    __shared__ float w[256], grad[256], sv[256], atb[256];
    __shared__ unsigned char inP[256];
    __shared__ int pidx[LH_PMAX];
    __shared__ float sub[LH_PMAX][LH_PMAX + 2];
    __shared__ float sP[LH_PMAX];
    for (int i = lane; i < 256; i += 64) {
        const float b = i < n ? Ag[(long long)n * n + i] : 0.0f;
        atb[i] = b;
        w[i] = 0.0f;
        sv[i] = 0.0f;
        grad[i] = -b;
        inP[i] = 0;
    }
    __builtin_amdgcn_wave_barrier();
    for (int outer = 0; outer < max_iter; outer++) {
        // entering variable: first index of the largest -grad > 0 over the zero set
        unsigned bk = 0u;
        int bi = 0x7fffffff;
#pragma unroll
        for (int k = 0; k < 4; k++) {
            const int i = lane + 64 * k;
            if (i < n && !inP[i]) {
                const float d = -grad[i];
                if (d > 0.0f && __float_as_uint(d) > bk) { bk = __float_as_uint(d); bi = i; }
            }
        }
        const unsigned gk = dpp_reduce_u32<true>(bk);
        const unsigned gi = dpp_reduce_u32<false>((bk == gk && bk != 0u) ? (unsigned)bi : 0xffffffffu);
        if (gk == 0u || __uint_as_float(gk) < 1e-10f) break;
        const int t_idx = (int)gi;
        if (lane == 0) inP[t_idx] = 1;
        __builtin_amdgcn_wave_barrier();
        for (int inner = 0; inner < max_iter; inner++) {
            // passive set, ascending
            int pc = 0;
#pragma unroll
            for (int k = 0; k < 4; k++) {
                const int i = lane + 64 * k;
                const bool f = i < n && inP[i];
                const unsigned long long m = __ballot(f);
                const int pos = pc + __popcll(m & ((1ull << lane) - 1ull));
                if (f && pos < LH_PMAX) pidx[pos] = i;
                pc += __popcll(m);
            }
            if (pc > LH_PMAX) {
                if (lane == 0) atomicOr(status, 1);
                return;
            }
            __builtin_amdgcn_wave_barrier();
            // sub-problem [AtA_PP + 1e-10 I | Atb_P]; rows lane and lane + 64
#pragma unroll
            for (int q = 0; q < 2; q++) {
                const int r = lane + 64 * q;
                if (r < pc) {
                    const int pr = pidx[r];
                    for (int cc = 0; cc < pc; cc++) {
                        float v = Ag[(long long)pidx[cc] * n + pr];
                        if (cc == r) v = v + 1e-10f;
                        sub[r][cc] = v;
                    }
                    sub[r][pc] = atb[pr];
                }
            }
            __builtin_amdgcn_wave_barrier();
            for (int col = 0; col < pc; col++) {
                // pivot: first row below col of largest |a| strictly above |a[col][col]|
                const float a0 = fabsf(sub[col][col]);
                unsigned key = 0u;
                int kr = 0x7fffffff;
#pragma unroll
                for (int q = 0; q < 2; q++) {
                    const int r = lane + 64 * q;
                    if (r > col && r < pc) {
                        const float v = fabsf(sub[r][col]);
                        if (v > a0 && __float_as_uint(v) > key) { key = __float_as_uint(v); kr = r; }
                    }
                }
                const unsigned km = dpp_reduce_u32<true>(key);
                int mr = col;
                if (km != 0u) mr = (int)dpp_reduce_u32<false>((key == km) ? (unsigned)kr : 0xffffffffu);
                if (mr != col) {
                    for (int j = lane; j <= pc; j += 64) {
                        const float t0 = sub[col][j];
                        sub[col][j] = sub[mr][j];
                        sub[mr][j] = t0;
                    }
                }
                __builtin_amdgcn_wave_barrier();
                const float piv = sub[col][col];
                if (fabsf(piv) < 1e-12f) continue;
#pragma unroll
                for (int q = 0; q < 2; q++) {
                    const int r = lane + 64 * q;
                    if (r > col && r < pc) {
                        const float f = sub[r][col] / piv;
                        for (int j = col; j <= pc; j++) sub[r][j] = sub[r][j] - f * sub[col][j];
                    }
                }
                __builtin_amdgcn_wave_barrier();
            }
            if (lane == 0) {
                for (int r = 0; r < pc; r++) sP[r] = 0.0f;
                for (int col = pc - 1; col >= 0; col--) {
                    const float piv = sub[col][col];
                    if (fabsf(piv) < 1e-12f) continue;
                    float val = sub[col][pc];
                    for (int r = col + 1; r < pc; r++) val = val - sub[col][r] * sP[r];
                    sP[col] = val / piv;
                }
            }
            __builtin_amdgcn_wave_barrier();
            for (int i = lane; i < 256; i += 64) sv[i] = 0.0f;
            __builtin_amdgcn_wave_barrier();
            bool infeasible = false;
#pragma unroll
            for (int q = 0; q < 2; q++) {
                const int r = lane + 64 * q;
                if (r < pc) {
                    sv[pidx[r]] = sP[r];
                    infeasible = infeasible || (sP[r] <= 0.0f);
                }
            }
            __builtin_amdgcn_wave_barrier();
            if (__ballot(infeasible) == 0ull) {
                for (int i = lane; i < 256; i += 64) w[i] = sv[i];
                __builtin_amdgcn_wave_barrier();
                break;
            }
            // step to the boundary, in passive-set order
            if (lane == 0) {
                float alpha = 1.0f;
                for (int r = 0; r < pc; r++) {
                    const int idx = pidx[r];
                    if (sv[idx] <= 0.0f) {
                        const float a = w[idx] / (w[idx] - sv[idx] + 1e-30f);
                        if (a < alpha) alpha = a;
                    }
                }
                sP[0] = alpha;
            }
            __builtin_amdgcn_wave_barrier();
            const float alpha = sP[0];
            for (int i = lane; i < n; i += 64) w[i] = w[i] + alpha * (sv[i] - w[i]);
            __builtin_amdgcn_wave_barrier();
#pragma unroll
            for (int q = 0; q < 2; q++) {
                const int r = lane + 64 * q;
                if (r < pc) {
                    const int idx = pidx[r];
                    if (fabsf(w[idx]) < 1e-12f) {
                        w[idx] = 0.0f;
                        inP[idx] = 0;
                    }
                }
            }
            __builtin_amdgcn_wave_barrier();
        }
        // grad = AtA w - Atb, sequential over j
#pragma unroll
        for (int k = 0; k < 4; k++) {
            const int i = lane + 64 * k;
            if (i < n) {
                float sum = 0.0f;
                for (int j = 0; j < n; j++) sum = sum + Ag[(long long)j * n + i] * w[j];
                grad[i] = sum - atb[i];
            }
        }
        __builtin_amdgcn_wave_barrier();
    }
    for (int i = lane; i < n; i += 64) wo[i] = w[i];
}

// Right-hand side entry (row i, column v) of a system's [M | B] storage:
// row-major for the register-LU systems (n <= 256), whose solve reads one row
// of B across 64 columns at a time; column-major (B transposed) for larger
// ones, whose general elimination swaps rows in place. For p == 1 both are
// the same.
// The register LU forms M = X^T X from X itself, staging X through the LDS of
// its step ring in slabs of rows, when X has at most LU_X_MAXQ rows
// (lu_x_fits, defined with the LU's constants below): then k_ls_build writes
// B only.
__device__ __forceinline__ bool lu_x_fits(int n, int nq);

__device__ __forceinline__ long long rhs_at(int n, int p, int i, int v) {
    return (long long)n * n + (n <= 256 ? (long long)i * p + v : (long long)v * n + i);
}

// X (nq x n) and Y (nq x p) staged in (dynamic) LDS as rows X | Y of width
// wp = round_up(n + p, 4); 4 x 4 output tiles per thread over the block tile
// grid, upper-triangular tiles only for X^T X (a sequential dot product is
// symmetric bit for bit: the mirror entry is written from the same sum).
// When all nq rows fit the LDS budget, one block per system takes every
// tile. Otherwise (large systems: the unchunked refits of state blobs) the
// rows come through the LDS in slabs of ks and each thread keeps two tiles'
// sums across the slabs (k ascending throughout), the system's tiles spread
// over gridDim.z blocks, 512 tiles per block and pass. Rows wider than the
// budget allows (ks < 8): one output per thread straight from global memory.
constexpr int LB_LDS_FLOATS = 40960;   // 160 KB
constexpr int LB_TPT = 2;              // tiles per thread and pass (slab mode)

// SLAB: the instance for systems whose rows do not all fit (the launcher's
// choice), so that the other keeps its registers
template <bool SLAB>
__global__ void __launch_bounds__(256)
k_ls_build(Geom g, const ChunkDesc * __restrict__ chunks, const float * __restrict__ X,
           const float * __restrict__ Y, float * __restrict__ aug, const long long * __restrict__ aug_off,
           int lds_floats, int m_by_lu) {
    const int c_idx = blockIdx.x / g.H, h = blockIdx.x % g.H, layer = blockIdx.y;
    const ChunkDesc c = chunks[c_idx];
    const int n = c.tc, p = g.dv, w = n + p, nq = c.nq;
    // M is left to k_ge_lu, which forms it from X itself (lu_x_fits)
    const bool skip_m = m_by_lu && lu_x_fits(n, nq);
    float * Ag = aug + aug_off[((long long)layer * g.n_chunks + c_idx) * g.H + h];
    const long long hsX = (long long)g.nq_max * g.t_total;
    const float * Xh = X + (long long)layer * g.H * hsX + h * hsX + c.off;
    const float * Yh = Y + ((((long long)layer * g.n_chunks + c_idx) * g.H + h) * g.nq_max) * g.dv;
    extern __shared__ __align__(16) float xs[];
    const int wp = (w + 3) & ~3;
    const bool whole = (long long)nq * wp <= lds_floats;
    const int ks = whole ? nq : lds_floats / wp;   // rows per slab
    if (!whole && ks < 8) {
        if (blockIdx.z != 0) return;
        // column-major: entry (row i, column j) at Ag[j * n + i]
        const long long total = (long long)n * w;
        for (long long e = skip_m ? (long long)n * n + threadIdx.x : threadIdx.x; e < total; e += blockDim.x) {
            const int j = (int)(e / n), i = (int)(e % n);
            float s = 0.0f;
            if (j < n) {
                for (int k = 0; k < nq; k++) s += Xh[(long long)k * g.t_total + i] * Xh[(long long)k * g.t_total + j];
            } else {
                for (int k = 0; k < nq; k++) s += Xh[(long long)k * g.t_total + i] * Yh[(long long)k * g.dv + (j - n)];
            }
            if (i == j) s += g.ridge;
            Ag[j < n ? e : rhs_at(n, p, i, j - n)] = s;
        }
        return;
    }
    // rows k0 .. k0 + kn - 1 into xs: xs[k][0..n) = X row, xs[k][n..n+p) = Y row, zero padding to wp
    const bool v4 = (n & 3) == 0 && (p & 3) == 0 && (g.t_total & 3) == 0 && (g.dv & 3) == 0 &&
                    (reinterpret_cast<uintptr_t>(Xh) & 15) == 0 && (reinterpret_cast<uintptr_t>(Yh) & 15) == 0;
    auto stage = [&](int k0, int kn) {
        if (v4) {
            // 16-byte pieces, eight loads per thread in flight before their
            // LDS stores: pieces q < tx are X's, the rest Y's (w = wp here);
            // a slot past the end repeats the last piece (the same value to
            // the same place)
            const int n4 = n >> 2, p4 = p >> 2, tx = kn * n4, tot = tx + kn * p4;
            for (int q0 = threadIdx.x; q0 < tot; q0 += 8 * blockDim.x) {
                float4 v[8];
                int dst[8];
#pragma unroll
                for (int u = 0; u < 8; u++) {
                    const int q = min(q0 + u * (int)blockDim.x, tot - 1);
                    const bool isx = q < tx;
                    const int qq = isx ? q : q - tx, w4 = isx ? n4 : p4;
                    const int k = qq / w4, j4 = qq - k * w4;
                    const float * src = isx ? Xh + (long long)(k0 + k) * g.t_total + 4 * j4
                                            : Yh + (long long)(k0 + k) * g.dv + 4 * j4;
                    dst[u] = k * wp + (isx ? 0 : n) + 4 * j4;
                    v[u] = *reinterpret_cast<const float4 *>(src);
                }
#pragma unroll
                for (int u = 0; u < 8; u++) *reinterpret_cast<float4 *>(&xs[dst[u]]) = v[u];
            }
        } else {
            for (int e = threadIdx.x; e < kn * wp; e += blockDim.x) {
                const int k = e / wp, j = e % wp;
                float v = 0.0f;
                if (j < n) v = Xh[(long long)(k0 + k) * g.t_total + j];
                else if (j < w) v = Yh[(long long)(k0 + k) * g.dv + (j - n)];
                xs[e] = v;
            }
        }
    };
    const int nbi = (n + 3) >> 2, nbw = wp >> 2;
    // 16-byte stores need n, p multiples of 4, B row-major and an aligned base
    const bool vec = (n & 3) == 0 && (p & 3) == 0 && n <= 256 && (reinterpret_cast<uintptr_t>(Ag) & 15) == 0;
    // a 4 x 4 tile's sums over the staged rows 0 .. kn - 1 (k ascending),
    // continuing acc
    auto tile_acc = [&](float (&acc)[4][4], int ib, int jb, int kn) {
        const int i0 = 4 * ib, j0 = 4 * jb;
        // row k + 1 is read from LDS while row k is summed (the last row
        // again at the end: no branch around the reads)
        float4 xi = *reinterpret_cast<const float4 *>(&xs[i0]);
        float4 xj = *reinterpret_cast<const float4 *>(&xs[j0]);
        for (int k = 0; k < kn; k++) {
            const int kk = min(k + 1, kn - 1);
            const float4 xin = *reinterpret_cast<const float4 *>(&xs[kk * wp + i0]);
            const float4 xjn = *reinterpret_cast<const float4 *>(&xs[kk * wp + j0]);
            __builtin_amdgcn_sched_barrier(0);
            const float vi[4] = {xi.x, xi.y, xi.z, xi.w}, vj[4] = {xj.x, xj.y, xj.z, xj.w};
#pragma unroll
            for (int a = 0; a < 4; a++)
#pragma unroll
                for (int b = 0; b < 4; b++) acc[a][b] = acc[a][b] + vi[a] * vj[b];
            __builtin_amdgcn_sched_barrier(0);
            xi = xin;
            xj = xjn;
        }
    };
    auto tile_store = [&](float (&acc)[4][4], int ib, int jb) {
        const int i0 = 4 * ib, j0 = 4 * jb;
        if (vec && i0 + 3 < n && j0 + 3 < w && (j0 + 3 < n || j0 >= n)) {
            // whole tile inside M or inside B: 16-byte stores
            if (j0 < n) {
                if (skip_m) return;
                if (ib == jb) {
#pragma unroll
                    for (int a = 0; a < 4; a++) acc[a][a] = acc[a][a] + g.ridge;
                }
#pragma unroll
                for (int b = 0; b < 4; b++)   // column j0 + b, rows i0 .. i0 + 3
                    *reinterpret_cast<float4 *>(&Ag[(long long)(j0 + b) * n + i0]) =
                        make_float4(acc[0][b], acc[1][b], acc[2][b], acc[3][b]);
                if (ib < jb) {
#pragma unroll
                    for (int a = 0; a < 4; a++)   // mirror: column i0 + a, rows j0 .. j0 + 3
                        *reinterpret_cast<float4 *>(&Ag[(long long)(i0 + a) * n + j0]) =
                            make_float4(acc[a][0], acc[a][1], acc[a][2], acc[a][3]);
                }
            } else {
#pragma unroll
                for (int a = 0; a < 4; a++)   // row i0 + a of B, columns j0 - n ..
                    *reinterpret_cast<float4 *>(&Ag[rhs_at(n, p, i0 + a, j0 - n)]) =
                        make_float4(acc[a][0], acc[a][1], acc[a][2], acc[a][3]);
            }
            return;
        }
#pragma unroll
        for (int a = 0; a < 4; a++) {
            const int i = i0 + a;
            if (i >= n) continue;
#pragma unroll
            for (int b = 0; b < 4; b++) {
                const int j = j0 + b;
                if (j >= w || (skip_m && j < n)) continue;
                float v = acc[a][b];
                if (i == j) v += g.ridge;
                Ag[j < n ? (long long)j * n + i : rhs_at(n, p, i, j - n)] = v;
                if (j < n && j > i) Ag[(long long)i * n + j] = v;   // mirror (j, i)
            }
        }
    };
    // the tiles: those holding columns of M (upper triangle; column blocks
    // jb < nbm, consecutive row blocks to consecutive threads: column-major
    // stores), or with M left to the LU only the block that also holds the
    // first columns of B; then the tiles of B alone
    const int nbm = nbi, nbr = nbw - nbm;
    const int nmt = skip_m ? ((n & 3) ? nbi : 0) : nbi * nbm;
    const int njobs = nmt + nbi * nbr;
    // job -> tile (ib, jb); false: none (below the diagonal)
    auto job_tile = [&](int e, int & ib, int & jb) -> bool {
        if (e < nmt) {
            if (skip_m) { ib = e; jb = nbm - 1; return true; }
            jb = e / nbi;
            ib = e % nbi;
            return ib <= jb;
        }
        e -= nmt;
        ib = e / nbr;
        jb = nbm + e % nbr;
        return true;
    };
    if (!SLAB || whole) {
        if (blockIdx.z != 0 || !whole) return;
        stage(0, nq);
        __syncthreads();
        for (int e = threadIdx.x; e < njobs; e += blockDim.x) {
            int ib, jb;
            if (!job_tile(e, ib, jb)) continue;
            float acc[4][4];
#pragma unroll
            for (int a = 0; a < 4; a++)
#pragma unroll
                for (int b = 0; b < 4; b++) acc[a][b] = 0.0f;
            tile_acc(acc, ib, jb, nq);
            tile_store(acc, ib, jb);
        }
        return;
    }
    // slab mode: passes of LB_TPT * 256 jobs per block; every thread of the
    // block runs the same passes and slabs (the barriers are uniform)
    if constexpr (SLAB) {
    const int per_pass = LB_TPT * (int)blockDim.x;
    for (int p0 = (int)blockIdx.z * per_pass; p0 < njobs; p0 += (int)gridDim.z * per_pass) {
        int tib[LB_TPT], tjb[LB_TPT];
        bool act[LB_TPT];
        float acc[LB_TPT][4][4];
#pragma unroll
        for (int u = 0; u < LB_TPT; u++) {
            const int e = p0 + u * (int)blockDim.x + (int)threadIdx.x;
            act[u] = e < njobs && job_tile(e, tib[u], tjb[u]);
#pragma unroll
            for (int a = 0; a < 4; a++)
#pragma unroll
                for (int b = 0; b < 4; b++) acc[u][a][b] = 0.0f;
        }
        for (int k0 = 0; k0 < nq; k0 += ks) {
            const int kn = min(ks, nq - k0);
            __syncthreads();   // the previous slab is read
            stage(k0, kn);
            __syncthreads();
#pragma unroll
            for (int u = 0; u < LB_TPT; u++)
                if (act[u]) tile_acc(acc[u], tib[u], tjb[u], kn);
        }
#pragma unroll
        for (int u = 0; u < LB_TPT; u++)
            if (act[u]) tile_store(acc[u], tib[u], tjb[u]);
    }
    }
}

// ---------------------------------------------------------------------------
// Gaussian elimination with partial pivoting + back substitution on [M | B]
// (n x (n + p)), math.h:494-556. M is stored column-major (entry (r, j) at
// a[j * n + r]; M is symmetric), B after it as given by rhs_at.
//
// k_ge_lu (n <= 256): LU of the n x n matrix with the reference's partial
// pivoting, in registers, as a column-cyclic dataflow. Wave w owns columns
// w, w + 16, ..., w + 240; lane l owns rows l, l+64, l+128, l+192 (physical
// rows; swaps are a logical<->physical permutation kept in LDS). Step c is
// produced by the owner of column c: pivot search on that column (DPP
// reductions), the multipliers a[r][c] / pivot, which it publishes through a
// 32-slot LDS ring with a per-slot step flag. Every wave consumes the steps
// in order, applying step c to each of its columns j > c (a -= f * u, the
// pivot row's u read from its own registers), so each element receives
// exactly the reference's sequence of updates. The owner of column c + 1
// applies step c to that column first and publishes step c + 1 before it
// updates its other columns, so the serial chain per step is one column's
// update, one pivot search and one division per row; everything else runs
// beside it. A wave can be at most 17 steps behind the newest published step
// (it owns one of any 16 consecutive columns and publishes that step only
// after consuming the step before), so the 32-slot ring is never overwritten
// before every wave has read it, and every flag a wave waits for is
// published by a wave that only waits for earlier flags.
//
// Two variants. The unmasked one applies each step to every row with the
// published multiplier, which is 0 for the rows no longer below the pivot, so
// those rows (already final) see a -= 0 * u. That leaves them unchanged
// whenever u is finite and a is not -0: the input is checked for -0 and
// non-finite entries, and no entry ever becomes -0 (x - y is -0 only for
// x = -0), and a non-finite u would leave a non-finite final entry in its
// pivot row, so a system whose final entries are all finite was factored
// exactly. Any other system is flagged and redone by the masked variant,
// which skips the rows no longer below the pivot.
//
// Output per system: one 256 x 256 array by physical row r holding, left of
// the step at which r became the pivot, r's multipliers (by step; the
// producer stores them over the eliminated column in registers), and from
// that step on, r's U row; plus the final permutation and the skipped-pivot
// flags. The right-hand sides are not touched here: the reference's
// elimination of them is forward substitution with the final permutation
// (ascending steps), done with the back substitution in k_ge_solve.
// ---------------------------------------------------------------------------
constexpr int RG_ROWS = 256, RG_WAVES = 16, RG_COLS = 16, RG_SLOTS = 4;
constexpr int RG_THREADS = RG_WAVES * 64;
constexpr int LU_RING = 32;          // > 17 outstanding steps
constexpr int LU_TROWS = 64;         // rows per pass of the transposed output write
constexpr int LU_SPIN_LIMIT = 1 << 22;   // polls per wave over the whole factorization
constexpr int LU_X_FLOATS = LU_RING * 64 * 4;   // X staged in the ring's LDS, LU_X_FLOATS / n rows at a time
constexpr int LU_X_MAXQ = 1024;                 // rows of X beyond which k_ls_build forms M
#ifndef LU_POLL_SLEEP
#define LU_POLL_SLEEP 1   // s_sleep units (64 clocks) between polls of a wave with slack
#endif
constexpr int LU_SPLIT = 128;   // k_ge_lu<false, true> takes steps before this; k_ge_lu_tail the rest
// wave priorities in the register LU: the owners of the next LU_PRIO_HI
// steps at 2, of the steps up to LU_PRIO_MID ahead at 1
#ifndef LU_PRIO_HI
#define LU_PRIO_HI 4
#endif
#ifndef LU_PRIO_MID
#define LU_PRIO_MID 12
#endif

// the register LU forms M from X: a system it factors, and X of at most
// LU_X_MAXQ rows (staged through the ring's LDS in slabs of rows)
__device__ __forceinline__ bool lu_x_fits(int n, int nq) { return n <= RG_ROWS && nq >= 1 && nq <= LU_X_MAXQ; }

// (the small arrays first: their fixed addresses stay within the 16-bit
// offset field of the LDS instructions)
struct LuShared {
    int plog[RG_ROWS];               // step c's pivot row (+256: skipped); -1 until published
    union {
        struct {
            int4 inv[64];            // logical index of rows l, l+64, l+128, l+192 in inv[l]
            int phys[RG_ROWS];       // physical row of each logical index
        } p;
        int e[2 * RG_ROWS];          // the same as one array: inv entries, then phys
    } m;
    union {
        float4 fm[LU_RING][64];      // step c's multipliers in slot c % LU_RING: lane l's four rows
        float tile[LU_TROWS][RG_ROWS + 1];   // output staging at the end
        float xs[LU_X_FLOATS];       // X (nq x n) while the matrix is formed, when M comes from X
    } u;
    static_assert(sizeof(float) * LU_X_FLOATS <= sizeof(float4) * LU_RING * 64, "X staging exceeds the ring");
    static_assert(2 * LU_X_FLOATS <= LU_TROWS * (RG_ROWS + 1), "X and its column-grouped copy exceed the union");
};

__device__ __forceinline__ int lu_inv_elem(int r) { return (r & 63) * 4 + (r >> 6); }
constexpr int LU_PHYS0 = RG_ROWS;    // index of phys[0] in LuShared::m.e

// LDS byte offset of a __shared__ object
template <typename T>
__device__ __forceinline__ unsigned lu_lds(const T * p) {
    return (unsigned)(size_t)(const __attribute__((address_space(3))) T *)p;
}

// Four LDS reads issued back to back, in this order, then one wait: an entry
// of plog, then (same pass) a step's multipliers, this lane's logical indices
// and one entry of phys. A wave's LDS accesses execute in order, so when the
// plog entry reads as published, the other three read what its producer
// wrote before it.
__device__ __forceinline__ void lu_poll_read(unsigned a_plog, unsigned a_fm, unsigned a_inv, unsigned a_phys,
                                             int & pl, float4 & f4, int4 & iv, int & ph) {
    typedef float v4f __attribute__((ext_vector_type(4)));
    typedef int v4i __attribute__((ext_vector_type(4)));
    v4f x;
    v4i y;
    asm volatile("ds_read_b32 %0, %4\n\t"
                 "ds_read_b128 %1, %5\n\t"
                 "ds_read_b128 %2, %6\n\t"
                 "ds_read_b32 %3, %7\n\t"
                 "s_waitcnt lgkmcnt(0)"
                 : "=&v"(pl), "=&v"(x), "=&v"(y), "=&v"(ph)
                 : "v"(a_plog), "v"(a_fm), "v"(a_inv), "v"(a_phys)
                 : "memory");
    f4 = make_float4(x[0], x[1], x[2], x[3]);
    iv = make_int4(y[0], y[1], y[2], y[3]);
}

// v[s] for a uniform s, as selects (no branches)
__device__ __forceinline__ float lu_pick(const float (&v)[RG_SLOTS], int s) {
    const float lo = (s & 1) ? v[1] : v[0];
    const float hi = (s & 1) ? v[3] : v[2];
    return (s & 2) ? hi : lo;
}

// Floating-point class tests (one v_cmp_class each, no branches). The class
// masks: bit 0 signalling NaN, 1 quiet NaN, 2 -inf, 5 -0, 9 +inf.
constexpr int FP_CLASS_NONFINITE = 0x207;   // NaN or +-inf
constexpr int FP_CLASS_UNSAFE = 0x227;      // NaN, +-inf or -0
// -0, +-inf or NaN
__device__ __forceinline__ bool lu_unsafe(float x) { return __builtin_amdgcn_classf(x, FP_CLASS_UNSAFE); }
__device__ __forceinline__ bool lu_nonfinite(float x) { return __builtin_amdgcn_classf(x, FP_CLASS_NONFINITE); }

// Publish step c1 from its column's values col[] (steps < c1 applied), given
// the logical indices iv of this lane's rows (negative for rows past n) and
// the physical row physc at logical c1: pivot = first row in logical order of
// largest |a| among the rows not yet used (logical index >= c1), replacing the
// diagonal only when strictly larger and never NaN (a NaN diagonal keeps the
// diagonal, every comparison against it failing); pivots below 1e-12 in
// magnitude skip the step (math.h:507-527). The rows still below the pivot
// get their multipliers (0 for a skipped step) in col[]; every other row's
// published multiplier is 0. The multipliers and the permutation update go
// to LDS before the step's entry in plog, which consumers wait for.
// Unmasked (MASKED = false), NaN needs no handling: a system that meets one
// ends with a non-finite entry and is redone masked.
template <bool MASKED>
__device__ __forceinline__ void lu_produce(LuShared & sh, float (&col)[RG_SLOTS], int4 iv, int physc, int c1,
                                           int lane) {
    const int li[RG_SLOTS] = {iv.x, iv.y, iv.z, iv.w};
    bool live[RG_SLOTS];
    unsigned key[RG_SLOTS];
    bool nanc = false;
#pragma unroll
    for (int s = 0; s < RG_SLOTS; s++) {
        live[s] = li[s] >= c1;
        const float v = fabsf(col[s]);
        if (MASKED) {
            key[s] = (live[s] && v == v) ? __float_as_uint(v) : 0u;
            nanc = nanc || (li[s] == c1 && v != v);
        } else {
            key[s] = live[s] ? __float_as_uint(v) : 0u;
        }
    }
    const unsigned gmax = dpp_reduce_u32<true>(max(max(key[0], key[1]), max(key[2], key[3])));
    int mr, P;
    if ((MASKED && __ballot(nanc)) || gmax == 0u) {
        // every live row is +-0 (or NaN), or the diagonal is NaN: the diagonal stays
        mr = c1;
        P = physc;
    } else {
        // first logical index among the rows at the maximum, with its physical row
        unsigned cand = 0xffffu;
#pragma unroll
        for (int s = 0; s < RG_SLOTS; s++)
            cand = min(cand, key[s] == gmax ? (((unsigned)li[s] << 8) | (unsigned)(lane + 64 * s)) : 0xffffu);
        const unsigned long long m = __ballot(cand != 0xffffu);
        unsigned v;
        if ((m & (m - 1)) == 0ull) v = (unsigned)__builtin_amdgcn_readlane((int)cand, __builtin_ctzll(m));
        else v = dpp_reduce_u32<false>(cand);
        mr = (int)(v >> 8);
        P = (int)(v & 255u);
    }
    // swap logical c1 and mr: lanes 0-3 write inv[P], inv[physc], phys[c1],
    // phys[mr] in one instruction (equal addresses carry equal values when
    // mr == c1), issued before the division so that it completes beside it
    {
        const int e01 = lane == 0 ? lu_inv_elem(P) : lu_inv_elem(physc);
        const int e23 = LU_PHYS0 + (lane == 2 ? c1 : mr);
        const int v01 = lane == 0 ? c1 : mr;
        const int v23 = lane == 2 ? P : physc;
        if (lane < 4) sh.m.e[lane < 2 ? e01 : e23] = lane < 2 ? v01 : v23;
    }
    const float piv = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(lu_pick(col, P >> 6)), P & 63));
    const bool elim = !(fabsf(piv) < 1e-12f);
    float f[RG_SLOTS];
#pragma unroll
    for (int s = 0; s < RG_SLOTS; s++) {
        const bool below = live[s] && (lane + 64 * s) != P;
        const float q = col[s] / piv;
        f[s] = (elim && below) ? q : 0.0f;
        if (below) col[s] = f[s];
    }
    sh.u.fm[c1 & (LU_RING - 1)][lane] = make_float4(f[0], f[1], f[2], f[3]);
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    if (lane == 0) __hip_atomic_store(&sh.plog[c1], P | (elim ? 0 : 256), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}

// The owner of column c + 1 (register column Q): a copy of that column with
// step c applied, from which step c + 1 is published; the copy (multipliers
// below the new pivot) replaces the column after the wave's own update with
// step c, which computes the same values for it.
template <int Q, bool MASKED>
__device__ __forceinline__ void lu_next_column(LuShared & sh, const float (&a)[RG_SLOTS][RG_COLS],
                                               const bool (&live)[RG_SLOTS], const float (&f)[RG_SLOTS],
                                               bool skip, int P, int4 iv, int physc, int c1, int n, int lane,
                                               float (&col)[RG_SLOTS]) {
#pragma unroll
    for (int s = 0; s < RG_SLOTS; s++) col[s] = a[s][Q];
    if (!skip) {
        const float u = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(lu_pick(col, P >> 6)), P & 63));
#pragma unroll
        for (int s = 0; s < RG_SLOTS; s++) {
            if (MASKED) {
                if (live[s]) col[s] = col[s] - f[s] * u;
            } else {
                col[s] = col[s] - f[s] * u;
            }
        }
    }
    lu_produce<MASKED>(sh, col, iv, physc, c1, lane);
}

// u[q] = a[P][q] for the register columns q >= Q0 (pivot row in slot S, lane lP)
template <int S, int Q0, bool MASKED>
__device__ __forceinline__ void lu_read_row(const float (&a)[RG_SLOTS][RG_COLS], int lP, float (&u)[RG_COLS]) {
    if constexpr (!MASKED) {
        // each column's pivot entry broadcast from lane lP by ds_bpermute, so
        // that the multiplies read VGPRs only: fp32 multiplies with an SGPR
        // operand (a v_readlane result) issue at about half the rate
#pragma unroll
        for (int q = Q0; q < RG_COLS; q++)
            u[q] = __int_as_float(__builtin_amdgcn_ds_bpermute(lP << 2, __float_as_int(a[S][q])));
    } else {
        // (the masked variant, at its register limit, reads them into SGPRs)
#pragma unroll
        for (int q = Q0; q < RG_COLS; q++) u[q] = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(a[S][q]), lP));
    }
}

// Apply one step to the register columns q >= Q0: a[r][q] -= f[r] * a[P][q],
// for every row (f = 0 off the rows below) or, MASKED, for the rows below.
template <int Q0, bool MASKED>
__device__ __forceinline__ void lu_apply_any(float (&a)[RG_SLOTS][RG_COLS], const bool (&live)[RG_SLOTS],
                                             const float (&f)[RG_SLOTS], int P) {
    if constexpr (Q0 < RG_COLS) {
        const int lP = P & 63;
        float u[RG_COLS];
        switch (P >> 6) {
            case 0: lu_read_row<0, Q0, MASKED>(a, lP, u); break;
            case 1: lu_read_row<1, Q0, MASKED>(a, lP, u); break;
            case 2: lu_read_row<2, Q0, MASKED>(a, lP, u); break;
            default: lu_read_row<3, Q0, MASKED>(a, lP, u); break;
        }
#pragma unroll
        for (int s = 0; s < RG_SLOTS; s++) {
            if (MASKED) {
                if (live[s]) {
#pragma unroll
                    for (int q = Q0; q < RG_COLS; q++) a[s][q] = a[s][q] - f[s] * u[q];
                }
            } else {
#pragma unroll
                for (int q = Q0; q < RG_COLS; q++) a[s][q] = a[s][q] - f[s] * u[q];
            }
        }
    }
}

// Steps 16 B .. 16 B + 15 (register column B is the wave's column in that
// range). Step c goes to the columns j = w + 16 q > c: q > B always, q = B
// when w > i.
template <int B, bool MASKED>
__device__ __forceinline__ void lu_steps(LuShared & sh, float (&a)[RG_SLOTS][RG_COLS], bool (&live)[RG_SLOTS],
                                         int n, int w, int lane, int & spins, int * __restrict__ status) {
    for (int i = 0; i < RG_COLS; i++) {
        const int c = RG_COLS * B + i;
        if (c >= n) break;   // (a break, not a return: one exit path keeps the register assignment)
        const int slot = c & (LU_RING - 1);
        const bool prod = c + 1 < n && w == ((c + 1) & (RG_COLS - 1));
        // the owners of the next columns run ahead of the others on their
        // SIMDs: the owner of c + 1 publishes step c + 1 now, the owner of
        // c + 2 must be through step c by the time step c + 1 appears, and
        // waves that own a column a few steps ahead work off the updates they
        // still owe before their turn comes (at equal priority the SIMDs
        // favour older waves, and the younger ones would fall behind)
        const int ahead = (w - c) & (RG_COLS - 1);   // this wave next publishes step c + ahead
        if (ahead != 0 && ahead <= LU_PRIO_HI) __builtin_amdgcn_s_setprio(2);
        else if (ahead != 0 && ahead <= LU_PRIO_MID) __builtin_amdgcn_s_setprio(1);
        else __builtin_amdgcn_s_setprio(0);
        // wait for step c (bounded: past the limit the wave stops waiting and
        // reports through *status, which the host turns into a device error).
        // The next producer polls without sleeping and reads the step's
        // multipliers, its rows' logical indices and the row at logical c + 1
        // in the same pass: LDS accesses of one wave execute in order, and
        // the producer wrote them before the plog entry.
        int pv;
        float4 f4;
        int4 iv = make_int4(0, 0, 0, 0);
        int physc = 0;
        if (prod) {
            for (;;) {
                int pl;
                lu_poll_read(lu_lds(&sh.plog[c]), lu_lds(&sh.u.fm[slot][lane]), lu_lds(&sh.m.p.inv[lane]),
                             lu_lds(&sh.m.p.phys[c + 1]), pl, f4, iv, physc);
                pv = __builtin_amdgcn_readfirstlane(pl);
                if (pv >= 0) break;
                if (++spins > LU_SPIN_LIMIT) {
                    if (lane == 0) atomicOr(status, 2);
                    break;
                }
            }
        } else {
            for (;;) {
                pv = __builtin_amdgcn_readfirstlane(
                    __hip_atomic_load(&sh.plog[c], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP));
                if (pv >= 0) break;
                if (++spins > LU_SPIN_LIMIT) {
                    if (lane == 0) atomicOr(status, 2);
                    break;
                }
                // (the owner of column c + 2 publishes next after the
                // producer; the others have a step or more of slack and
                // wait longer between polls, which leaves the issue slots
                // of their SIMDs to the waves doing the work)
                if (w == ((c + 2) & (RG_COLS - 1))) __builtin_amdgcn_s_sleep(1);
                else __builtin_amdgcn_s_sleep(LU_POLL_SLEEP);
            }
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
            f4 = sh.u.fm[slot][lane];
        }
        physc = __builtin_amdgcn_readfirstlane(physc);
        const float f[RG_SLOTS] = {f4.x, f4.y, f4.z, f4.w};
        const int P = pv & 255;
        const bool skip = (pv & 256) != 0;
        if (MASKED) {
#pragma unroll
            for (int s = 0; s < RG_SLOTS; s++) live[s] = live[s] && (lane + 64 * s) != P;
        }
        float col[RG_SLOTS];
        if (prod) {
            __builtin_amdgcn_s_setprio(3);
            if (w != 0) lu_next_column<B, MASKED>(sh, a, live, f, skip, P, iv, physc, c + 1, n, lane, col);
            else if constexpr (B + 1 < RG_COLS)
                lu_next_column<B + 1, MASKED>(sh, a, live, f, skip, P, iv, physc, c + 1, n, lane, col);
            __builtin_amdgcn_s_setprio(2);
        }
        if (!skip) {
            if (w > i) lu_apply_any<B, MASKED>(a, live, f, P);
            else lu_apply_any<B + 1, MASKED>(a, live, f, P);
        }
        if (prod) {
            if (w != 0) {
#pragma unroll
                for (int s = 0; s < RG_SLOTS; s++) a[s][B] = col[s];
            } else if constexpr (B + 1 < RG_COLS) {
#pragma unroll
                for (int s = 0; s < RG_SLOTS; s++) a[s][B + 1] = col[s];
            }
        }
    }
    if constexpr (B + 1 < RG_COLS) lu_steps<B + 1, MASKED>(sh, a, live, n, w, lane, spins, status);
}

// grid (n_chunks * H, L), 1024 threads. MASKED = false: every system, sets
// redo[sys]; MASKED = true: only the systems with redo[sys] set.
// SPLIT (unmasked only): steps 0 .. 127 only. A system of n > 128 unknowns
// then leaves its rows not yet chosen as pivots (logical indices 128 ..
// n - 1) in the columns >= 128 to k_ge_lu_tail, which takes the remaining
// steps: that trailing matrix goes to T2[sys] column-major (entry (logical
// row 128 + k, column 128 + j) at j * 128 + k) and the physical row of each
// of its rows to map2[sys][k]; every other entry is final and written here.
template <bool MASKED, bool SPLIT>
__device__ __forceinline__ void
ge_lu_body(Geom g, const ChunkDesc * __restrict__ chunks, const float * __restrict__ aug,
           const long long * __restrict__ aug_off, const float * __restrict__ X, int * __restrict__ perm_out,
           unsigned char * __restrict__ skip_out, float * __restrict__ LU_all, int * __restrict__ redo,
           int * __restrict__ status, float * __restrict__ T2, int * __restrict__ map2) {
    static_assert(!(MASKED && SPLIT), "the split factorization is the unmasked one");
    const int c_idx = blockIdx.x / g.H, h = blockIdx.x % g.H, layer = blockIdx.y;
    const ChunkDesc c = chunks[c_idx];
    const int n = c.tc;
    if (n > RG_ROWS || n < 1) return;
    const long long sys = ((long long)layer * g.n_chunks + c_idx) * g.H + h;
    if (MASKED && redo[sys] == 0) return;
    if (!MASKED && g.lu_masked) {
        if (threadIdx.x == 0) redo[sys] = 1;
        return;
    }
    const float * A = aug + aug_off[sys];
    float * LU = LU_all + sys * (long long)RG_ROWS * RG_ROWS;
    const int tid = threadIdx.x, lane = tid & 63, w = __builtin_amdgcn_readfirstlane(tid >> 6);
    __shared__ LuShared sh;

    // rows and columns past n hold copies of row / column n - 1: those rows
    // are never live and those columns are never published or written out
    float a[RG_SLOTS][RG_COLS];
    bool live[RG_SLOTS];
    bool unsafe = false;
    if (X && lu_x_fits(n, c.nq)) {
        // M = X^T X (+ ridge on the diagonal) formed here, k_ls_build having
        // left it out: each entry the same sequential sum over the rows of X
        // (k ascending from +0, kept in registers across the slabs of rows
        // staged in LDS), the ridge added after it
        const int nq = c.nq;
        // rows per slab: at least 32; at most 32 with the second copy of the
        // slab (256 columns a row)
        constexpr bool XP = !MASKED;
        const int kb = XP ? LU_X_FLOATS / RG_ROWS : LU_X_FLOATS / n;
        const long long hsX = (long long)g.nq_max * g.t_total;
        const float * Xh = X + (long long)layer * g.H * hsX + h * hsX + c.off;
        int cc[RG_COLS];
#pragma unroll
        for (int q = 0; q < RG_COLS; q++) cc[q] = min(w + RG_WAVES * q, n - 1);
#pragma unroll
        for (int s = 0; s < RG_SLOTS; s++) {
            const int r = lane + 64 * s;
            live[s] = r < n;
#pragma unroll
            for (int q = 0; q < RG_COLS; q++) a[s][q] = 0.0f;
        }
        // rows of X as 16-byte pieces copied straight to LDS when they allow
        // it (global_load_lds: no registers, every piece of a slab in flight
        // at once; a wave's 64 pieces land contiguously at the LDS address
        // given for its first lane). The masked variant, at its register
        // limit, keeps the plain loads.
        const bool x4 = !MASKED && (n & 3) == 0 && (g.t_total & 3) == 0 &&
                        (reinterpret_cast<uintptr_t>(Xh) & 15) == 0;
        for (int k0 = 0; k0 < nq; k0 += kb) {
            const int nk = min(kb, nq - k0);
            if (k0 > 0) __syncthreads();   // the previous slab has been read
            if (x4) {
                constexpr int PER = LU_X_FLOATS / 4 / RG_THREADS;
                const int n4 = n >> 2, tot4 = (nk * n) >> 2;
#pragma unroll
                for (int u = 0; u < PER; u++) {
                    const int base = u * RG_THREADS + 64 * w;   // this wave's first piece
                    const int e4 = base + lane;
                    if (e4 < tot4) {
                        const int k = e4 / n4, i4 = e4 - k * n4;
                        __builtin_amdgcn_global_load_lds(
                            static_cast<const void *>(Xh + (long long)(k0 + k) * g.t_total + 4 * i4),
                            (__attribute__((address_space(3))) void *)(sh.u.xs + 4 * base), 16, 0, 0);
                    }
                }
            } else {
                for (int e = tid; e < nk * n; e += RG_THREADS) {
                    const int k = e / n, i = e - k * n;
                    sh.u.xs[e] = Xh[(long long)(k0 + k) * g.t_total + i];
                }
            }
            __syncthreads();
            // (unmasked) a second copy of the slab with each wave's 16 columns
            // side by side (entry (k, w + 16 q) at k * 256 + 16 w + q, clamped
            // like cc), so that a wave reads its column values as four
            // broadcast 16-byte reads per row of X
            float * xp = sh.u.xs + LU_X_FLOATS;
            if constexpr (XP) {
                for (int e = tid; e < nk * RG_ROWS; e += RG_THREADS) {
                    const int k = e >> 8, p = e & 255;
                    xp[e] = sh.u.xs[k * n + min((p >> 4) + RG_WAVES * (p & 15), n - 1)];
                }
                __syncthreads();
            }
            for (int k = 0; k < nk; k++) {
                const float * xk = sh.u.xs + k * n;
                float xr[RG_SLOTS], xc[RG_COLS];
#pragma unroll
                for (int s = 0; s < RG_SLOTS; s++) xr[s] = xk[min(lane + 64 * s, n - 1)];
                if constexpr (XP) {
                    const float4 * xq = reinterpret_cast<const float4 *>(xp + k * RG_ROWS + 16 * w);
#pragma unroll
                    for (int i = 0; i < RG_COLS / 4; i++) {
                        const float4 v = xq[i];
                        xc[4 * i] = v.x; xc[4 * i + 1] = v.y; xc[4 * i + 2] = v.z; xc[4 * i + 3] = v.w;
                    }
                } else {
#pragma unroll
                    for (int q = 0; q < RG_COLS; q++) xc[q] = xk[cc[q]];
                }
#pragma unroll
                for (int s = 0; s < RG_SLOTS; s++)
#pragma unroll
                    for (int q = 0; q < RG_COLS; q++) a[s][q] = a[s][q] + xr[s] * xc[q];
            }
        }
#pragma unroll
        for (int s = 0; s < RG_SLOTS; s++) {
            const int rc = min(lane + 64 * s, n - 1);
#pragma unroll
            for (int q = 0; q < RG_COLS; q++) {
                if (rc == cc[q]) a[s][q] = a[s][q] + g.ridge;
                if (!MASKED) unsafe |= lu_unsafe(a[s][q]);
            }
        }
        __syncthreads();   // X is dead: the LDS becomes the step ring
    } else {
#pragma unroll
        for (int s = 0; s < RG_SLOTS; s++) {
            const int r = lane + 64 * s;
            live[s] = r < n;
            const int rc = min(r, n - 1);
#pragma unroll
            for (int q = 0; q < RG_COLS; q++) {
                a[s][q] = A[(unsigned)(min(w + RG_WAVES * q, n - 1) * n + rc)];
                if (!MASKED) unsafe |= lu_unsafe(a[s][q]);
            }
        }
    }
    if (tid < RG_ROWS) {
        sh.m.p.phys[tid] = tid;
        sh.m.e[lu_inv_elem(tid)] = tid < n ? tid : -1;   // rows past n are never live
        sh.plog[tid] = -1;
    }
    if (!MASKED) {
        if (__syncthreads_or(unsafe)) {
            if (tid == 0) redo[sys] = 1;
            return;
        }
    } else {
        __syncthreads();
    }
    if (w == 0) {
        float col[RG_SLOTS];
#pragma unroll
        for (int s = 0; s < RG_SLOTS; s++) col[s] = a[s][0];
        lu_produce<MASKED>(sh, col, sh.m.p.inv[lane], 0, 0, lane);
#pragma unroll
        for (int s = 0; s < RG_SLOTS; s++) a[s][0] = col[s];
    }
    int spins = 0;
    // (SPLIT: the steps before LU_SPLIT only)
    const int nsteps = SPLIT ? min(n, LU_SPLIT) : n;
    const bool tail = SPLIT && n > LU_SPLIT;
    lu_steps<0, MASKED>(sh, a, live, nsteps, w, lane, spins, status);
    int li[RG_SLOTS] = {0, 0, 0, 0};
    if (tail) {
        __syncthreads();   // (the last step's permutation update)
        const int4 iv = sh.m.p.inv[lane];
        li[0] = iv.x; li[1] = iv.y; li[2] = iv.z; li[3] = iv.w;
    }
    if (!MASKED) {
        // a non-finite final entry: some step may have changed a finished row
        // (SPLIT: the entries final here, columns < 128 and the rows already
        // chosen as pivots)
        // (bitwise operators only: short-circuit ones compile to a branch per entry)
        bool bad = false;
#pragma unroll
        for (int s = 0; s < RG_SLOTS; s++) {
            const bool rin = lane + 64 * s < n;
            const bool rfin = rin & (!tail | (li[s] < LU_SPLIT));
#pragma unroll
            for (int q = 0; q < RG_COLS; q++) {
                // (column w + 16 q is below LU_SPLIT exactly when q is)
                const bool use = (w + RG_WAVES * q < n) & (q < LU_SPLIT / RG_WAVES ? rin : rfin);
                bad |= use & lu_nonfinite(a[s][q]);
            }
        }
        const bool redo_sys = __syncthreads_or(bad);
        if (tid == 0) redo[sys] = redo_sys ? 1 : 0;
        if (redo_sys) return;
    } else {
        __syncthreads();
    }
    if (tail) {
        // the trailing matrix and its rows' physical indices for k_ge_lu_tail
        float * T = T2 + sys * (long long)(LU_SPLIT * LU_SPLIT);
#pragma unroll
        for (int s = 0; s < RG_SLOTS; s++) {
            if (li[s] >= LU_SPLIT && li[s] < n) {
#pragma unroll
                for (int q = LU_SPLIT / RG_WAVES; q < RG_COLS; q++) {
                    const int j = w + RG_WAVES * q;
                    if (j < n) T[(unsigned)((j - LU_SPLIT) * LU_SPLIT + li[s] - LU_SPLIT)] = a[s][q];
                }
            }
        }
        if (tid < n - LU_SPLIT) map2[sys * LU_SPLIT + tid] = sh.m.p.phys[LU_SPLIT + tid];
    }
    if (tid < nsteps) {
        const int pl = sh.plog[tid];
        perm_out[sys * (long long)g.tc_max + tid] = pl & 255;
        skip_out[sys * (long long)g.tc_max + tid] = (unsigned char)(pl >> 8);
    }
    // every entry is final in registers: multipliers left of each row's pivot
    // step, U from it on; rows go out through LDS, TR at a time (LU_TROWS; 32 in the masked
    // variant, whose registers are at their limit), as
    // contiguous row segments of 256 entries, zero past column n (the
    // substitution reads whole blocks of a row without guards)
    constexpr int TR = MASKED ? 32 : LU_TROWS;
#pragma unroll
    for (int s = 0; s < RG_SLOTS; s++) {
#pragma unroll
        for (int half = 0; half < 64 / TR; half++) {
            const int r0 = 64 * s + TR * half;
            if (r0 >= n) break;
            const int lr = lane - TR * half;
            if (lr >= 0 && lr < TR) {
#pragma unroll
                for (int q = 0; q < RG_COLS; q++) sh.u.tile[lr][w + RG_WAVES * q] = a[s][q];
            }
            __syncthreads();
            // four entries a thread, one 16-byte store (a group never straddles
            // column 128; the last one of a row with n % 4 != 0 goes entry by
            // entry); the masked variant stores entry by entry
            if constexpr (MASKED) {
                for (int e = tid; e < TR * RG_ROWS; e += RG_THREADS) {
                    const int rr = e / RG_ROWS, j = e % RG_ROWS;
                    if (r0 + rr < n && j < n) LU[(unsigned)((r0 + rr) * RG_ROWS + j)] = sh.u.tile[rr][j];
                }
            } else for (int e4 = tid; e4 < TR * RG_ROWS / 4; e4 += RG_THREADS) {
                const int rr = e4 >> 6, j = (e4 & 63) * 4, r = r0 + rr;
                if (r < n && j < n && (!tail || j < LU_SPLIT || sh.m.e[lu_inv_elem(r)] < LU_SPLIT)) {
                    const float * t = &sh.u.tile[rr][j];
                    float * o = LU + (unsigned)(r * RG_ROWS + j);
                    if (j + 4 <= n) {
                        *reinterpret_cast<float4 *>(o) = make_float4(t[0], t[1], t[2], t[3]);
                    } else {
                        for (int k = 0; k < n - j; k++) o[k] = t[k];
                    }
                }
            }
            __syncthreads();
        }
    }
    // zeros past column n
    for (int e = tid; e < n * (RG_ROWS - n); e += RG_THREADS) {
        const int r = e / (RG_ROWS - n), j = n + e % (RG_ROWS - n);
        LU[(unsigned)(r * RG_ROWS + j)] = 0.0f;
    }
}

// The kernels. The unmasked ones are held to 112 VGPRs (amdgpu_num_vgpr
// counts a register pair on this GPU, so 56), one under what they use
// unconstrained and spill-free: four waves per SIMD then leave 64 VGPRs a
// lane, which lets a block of the original-attention statistics run on the
// same CU. The masked kernel keeps its registers.
template <bool MASKED, bool SPLIT = false>
__global__ void __launch_bounds__(RG_THREADS)
k_ge_lu(Geom g, const ChunkDesc * __restrict__ chunks, const float * __restrict__ aug,
        const long long * __restrict__ aug_off, const float * __restrict__ X, int * __restrict__ perm_out,
        unsigned char * __restrict__ skip_out, float * __restrict__ LU_all, int * __restrict__ redo,
        int * __restrict__ status, float * __restrict__ T2, int * __restrict__ map2) {
    ge_lu_body<MASKED, SPLIT>(g, chunks, aug, aug_off, X, perm_out, skip_out, LU_all, redo, status, T2, map2);
}
template <>
__global__ void __launch_bounds__(RG_THREADS) __attribute__((amdgpu_num_vgpr(56)))
k_ge_lu<false, true>(Geom g, const ChunkDesc * __restrict__ chunks, const float * __restrict__ aug,
        const long long * __restrict__ aug_off, const float * __restrict__ X, int * __restrict__ perm_out,
        unsigned char * __restrict__ skip_out, float * __restrict__ LU_all, int * __restrict__ redo,
        int * __restrict__ status, float * __restrict__ T2, int * __restrict__ map2) {
    ge_lu_body<false, true>(g, chunks, aug, aug_off, X, perm_out, skip_out, LU_all, redo, status, T2, map2);
}
template <>
__global__ void __launch_bounds__(RG_THREADS) __attribute__((amdgpu_num_vgpr(56)))
k_ge_lu<false, false>(Geom g, const ChunkDesc * __restrict__ chunks, const float * __restrict__ aug,
        const long long * __restrict__ aug_off, const float * __restrict__ X, int * __restrict__ perm_out,
        unsigned char * __restrict__ skip_out, float * __restrict__ LU_all, int * __restrict__ redo,
        int * __restrict__ status, float * __restrict__ T2, int * __restrict__ map2) {
    ge_lu_body<false, false>(g, chunks, aug, aug_off, X, perm_out, skip_out, LU_all, redo, status, T2, map2);
}

// ---------------------------------------------------------------------------
// The last steps of the split register LU. k_ge_lu<false, true> stops after
// step 127; from there a step only changes the rows not yet chosen as pivots
// (logical indices 128 .. n - 1) in the columns >= 128. That trailing matrix
// (at most 128 x 128, T2) is factored here, its rows in logical order, with
// k_ge_lu's pivot rules and update order, in 32 registers per lane of a
// 512-thread block: lane l holds rows l and l + 64, wave w columns w, w + 8,
// ... Such a block needs a quarter of the registers of a whole system, so
// several run on a CU at once and their pivot chains (each a series of
// dependent reductions, divisions and LDS hand-offs) overlap, where the
// whole-matrix kernel runs one system per CU.
// ---------------------------------------------------------------------------
constexpr int LP_WAVES = 8, LP_THREADS = 64 * LP_WAVES;
constexpr int LP_Q = LU_SPLIT / LP_WAVES;   // register columns per wave
constexpr int LP_TROWS = 32;               // rows per pass of the output

struct LtShared {
    float2 ring[LU_RING][64];              // step c's multipliers in slot c % LU_RING: lane l's two rows
    float tile[LP_TROWS][LU_SPLIT + 1];    // output staging
    int plog[LU_SPLIT];                    // step c's pivot row (+256: skipped); -1 until published
    int inv[2 * 64];                       // logical index of rows l, l + 64 at [2 l], [2 l + 1]
    int phys[LU_SPLIT];                    // row of each logical index
    int map[LU_SPLIT];                     // physical row (of the whole system) of each row
};

// S values of slot c of a ring, the plog entry and the lane's logical row
// indices, and phys[c + 1], read in this order with one wait (the wave's LDS
// reads execute in order, so a published plog entry means the rest is too)
template <int S>
__device__ __forceinline__ void lp_poll_read(unsigned a_plog, unsigned a_f, unsigned a_inv, unsigned a_phys,
                                             int & pl, float (&f)[S], int (&li)[S], int & ph) {
    if constexpr (S == 4) {
        typedef float v4f __attribute__((ext_vector_type(4)));
        typedef int v4i __attribute__((ext_vector_type(4)));
        v4f x;
        v4i y;
        asm volatile("ds_read_b32 %0, %4\n\t"
                     "ds_read_b128 %1, %5\n\t"
                     "ds_read_b128 %2, %6\n\t"
                     "ds_read_b32 %3, %7\n\t"
                     "s_waitcnt lgkmcnt(0)"
                     : "=&v"(pl), "=&v"(x), "=&v"(y), "=&v"(ph)
                     : "v"(a_plog), "v"(a_f), "v"(a_inv), "v"(a_phys)
                     : "memory");
        f[0] = x[0]; f[1] = x[1]; f[2] = x[2]; f[3] = x[3];
        li[0] = y[0]; li[1] = y[1]; li[2] = y[2]; li[3] = y[3];
    } else {
        typedef float v2f __attribute__((ext_vector_type(2)));
        typedef int v2i __attribute__((ext_vector_type(2)));
        v2f x;
        v2i y;
        asm volatile("ds_read_b32 %0, %4\n\t"
                     "ds_read_b64 %1, %5\n\t"
                     "ds_read_b64 %2, %6\n\t"
                     "ds_read_b32 %3, %7\n\t"
                     "s_waitcnt lgkmcnt(0)"
                     : "=&v"(pl), "=&v"(x), "=&v"(y), "=&v"(ph)
                     : "v"(a_plog), "v"(a_f), "v"(a_inv), "v"(a_phys)
                     : "memory");
        f[0] = x[0]; f[1] = x[1];
        li[0] = y[0]; li[1] = y[1];
    }
}

// v[s] for a uniform s, as selects of values (a conditional of the array
// elements themselves would select their addresses, and an array read
// through a selected address is kept in scratch memory)
template <int S>
__device__ __forceinline__ float lp_pick(const float (&v)[S], int s) {
    const float v0 = v[0], v1 = v[1];
    const float lo = (s & 1) ? v1 : v0;
    if constexpr (S == 4) {
        const float v2 = v[2], v3 = v[3];
        const float hi = (s & 1) ? v3 : v2;
        return (s & 2) ? hi : lo;
    } else {
        return lo;
    }
}

// Publish step c1 of a chain from its column col[] (steps < c1 applied):
// lu_produce's rules (first logical index among the largest |a| of the rows
// not yet used, the diagonal kept when all are zero, pivots below 1e-12
// skip the step), for S rows per lane. ring: [LU_RING][64][S]; inv: [64][S].
template <int S>
__device__ __forceinline__ void lp_produce(float * ring, int * plog, int * inv, int * phys, float (&col)[S],
                                           const int (&li)[S], int physc, int c1, int lane) {
    bool live[S];
    unsigned key[S];
#pragma unroll
    for (int s = 0; s < S; s++) {
        live[s] = li[s] >= c1;
        key[s] = live[s] ? __float_as_uint(fabsf(col[s])) : 0u;
    }
    unsigned km = key[0];
#pragma unroll
    for (int s = 1; s < S; s++) km = max(km, key[s]);
    const unsigned gmax = dpp_reduce_u32<true>(km);
    int mr, P;
    if (gmax == 0u) {
        mr = c1;
        P = physc;
    } else {
        unsigned cand = 0xffffffffu;
#pragma unroll
        for (int s = 0; s < S; s++)
            cand = min(cand, key[s] == gmax ? (((unsigned)li[s] << 8) | (unsigned)(lane + 64 * s)) : 0xffffffffu);
        const unsigned long long m = __ballot(cand != 0xffffffffu);
        unsigned v;
        if ((m & (m - 1)) == 0ull) v = (unsigned)__builtin_amdgcn_readlane((int)cand, __builtin_ctzll(m));
        else v = dpp_reduce_u32<false>(cand);
        mr = (int)(v >> 8);
        P = (int)(v & 255u);
    }
    // swap logical c1 and mr: inv[P] = c1, inv[physc] = mr, phys[c1] = P, phys[mr] = physc
    if (lane < 4) {
        const int ie = lane == 0 ? P : physc;
        const int e = lane < 2 ? (ie & 63) * S + (ie >> 6) : (lane == 2 ? c1 : mr);
        const int v = lane == 0 ? c1 : (lane == 1 ? mr : (lane == 2 ? P : physc));
        if (lane < 2) inv[e] = v;
        else phys[e] = v;
    }
    const float piv = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(lp_pick<S>(col, P >> 6)), P & 63));
    const bool elim = !(fabsf(piv) < 1e-12f);
    float f[S];
#pragma unroll
    for (int s = 0; s < S; s++) {
        const bool below = live[s] && (lane + 64 * s) != P;
        const float q = col[s] / piv;
        f[s] = (elim && below) ? q : 0.0f;
        if (below) col[s] = f[s];
    }
    float * slot = ring + ((c1 & (LU_RING - 1)) * 64 + lane) * S;
    if constexpr (S == 4) *reinterpret_cast<float4 *>(slot) = make_float4(f[0], f[1], f[2], f[3]);
    else *reinterpret_cast<float2 *>(slot) = make_float2(f[0], f[1]);
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    if (lane == 0) __hip_atomic_store(&plog[c1], P | (elim ? 0 : 256), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}

// a[r][q] -= f[r] * a[P][q] for the register columns q >= Q0 (pivot row in
// slot SL, lane lP): each column's pivot entry read from its lane just
// before the column is updated (v_readlane: the ds_bpermute broadcast of
// k_ge_lu needs registers that would cost this kernel a block per CU)
template <int S, int Q, int SL, int Q0>
__device__ __forceinline__ void lp_update_from(float (&a)[S][Q], const float (&f)[S], int lP) {
#pragma unroll
    for (int q = Q0; q < Q; q++) {
        const float u = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(a[SL][q]), lP));
#pragma unroll
        for (int s = 0; s < S; s++) a[s][q] = a[s][q] - f[s] * u;
    }
}

// one step applied to the register columns q >= Q0 (multiplier 0 off the rows below)
template <int S, int Q, int Q0>
__device__ __forceinline__ void lp_apply(float (&a)[S][Q], const float (&f)[S], int P) {
    if constexpr (Q0 < Q) {
        const int lP = P & 63;
        if constexpr (S == 4) {
            switch (P >> 6) {
                case 0: lp_update_from<S, Q, 0, Q0>(a, f, lP); break;
                case 1: lp_update_from<S, Q, 1, Q0>(a, f, lP); break;
                case 2: lp_update_from<S, Q, 2, Q0>(a, f, lP); break;
                default: lp_update_from<S, Q, 3, Q0>(a, f, lP); break;
            }
        } else {
            if (P >> 6) lp_update_from<S, Q, 1, Q0>(a, f, lP);
            else lp_update_from<S, Q, 0, Q0>(a, f, lP);
        }
    }
}

// The owner of column c + 1 (register column QN): a copy of it with step c
// applied, from which step c + 1 is published
template <int S, int Q, int QN>
__device__ __forceinline__ void lp_next_column(float * ring, int * plog, int * inv, int * phys, const float (&a)[S][Q],
                                               const float (&f)[S], bool skip, int P, const int (&li)[S], int physc,
                                               int c1, int lane, float (&col)[S]) {
#pragma unroll
    for (int s = 0; s < S; s++) col[s] = a[s][QN];
    if (!skip) {
        const float u = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(lp_pick<S>(col, P >> 6)), P & 63));
#pragma unroll
        for (int s = 0; s < S; s++) col[s] = col[s] - f[s] * u;
    }
    lp_produce<S>(ring, plog, inv, phys, col, li, physc, c1, lane);
}

// Step c = LP_WAVES B + i of a chain whose wave-relative column block is B: wait
// for it, publish step c + 1 if this wave owns column c + 1 (and c + 1 <
// nlim), apply it to the wave's columns > c (lu_steps' scheme).
template <int S, int Q, int B>
__device__ __forceinline__ void lp_step(float * ring, int * plog, int * inv, int * phys, float (&a)[S][Q], int c,
                                        int nlim, int wv, int lane, int & spins, int * __restrict__ status) {
    const int i = c - LP_WAVES * B;
    const int slot = c & (LU_RING - 1);
    const bool prod = c + 1 < nlim && wv == ((c + 1) & (LP_WAVES - 1));
    if (prod || wv == ((c + 2) & (LP_WAVES - 1))) __builtin_amdgcn_s_setprio(2);
    else __builtin_amdgcn_s_setprio(0);
    int pv;
    float f[S];
    int li[S];
    int physc = 0;
#pragma unroll
    for (int s = 0; s < S; s++) li[s] = 0;
    float * fs = ring + (slot * 64 + lane) * S;
    if (prod) {
        for (;;) {
            int pl;
            lp_poll_read<S>(lu_lds(&plog[c]), lu_lds(fs), lu_lds(&inv[lane * S]), lu_lds(&phys[c + 1]), pl, f, li,
                            physc);
            pv = __builtin_amdgcn_readfirstlane(pl);
            if (pv >= 0) break;
            if (++spins > LU_SPIN_LIMIT) {
                if (lane == 0) atomicOr(status, 2);
                break;
            }
        }
    } else {
        for (;;) {
            pv = __builtin_amdgcn_readfirstlane(
                __hip_atomic_load(&plog[c], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP));
            if (pv >= 0) break;
            if (++spins > LU_SPIN_LIMIT) {
                if (lane == 0) atomicOr(status, 2);
                break;
            }
            if (wv == ((c + 2) & (LP_WAVES - 1))) __builtin_amdgcn_s_sleep(1);
            else __builtin_amdgcn_s_sleep(LU_POLL_SLEEP);
        }
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
        if constexpr (S == 4) {
            const float4 v = *reinterpret_cast<const float4 *>(fs);
            f[0] = v.x; f[1] = v.y; f[2] = v.z; f[3] = v.w;
        } else {
            const float2 v = *reinterpret_cast<const float2 *>(fs);
            f[0] = v.x; f[1] = v.y;
        }
    }
    physc = __builtin_amdgcn_readfirstlane(physc);
    const int P = pv & 255;
    const bool skip = (pv & 256) != 0;
    float col[S];
#pragma unroll
    for (int s = 0; s < S; s++) col[s] = 0.0f;
    if (prod) {
        __builtin_amdgcn_s_setprio(3);
        if (wv != 0) lp_next_column<S, Q, B>(ring, plog, inv, phys, a, f, skip, P, li, physc, c + 1, lane, col);
        else if constexpr (B + 1 < Q)
            lp_next_column<S, Q, B + 1>(ring, plog, inv, phys, a, f, skip, P, li, physc, c + 1, lane, col);
        __builtin_amdgcn_s_setprio(2);
    }
    if (!skip) {
        if (wv > i) lp_apply<S, Q, B>(a, f, P);
        else lp_apply<S, Q, B + 1>(a, f, P);
    }
    // (value selects: stores under if / else to two elements would be merged
    // into one store through a selected address, which keeps the matrix in
    // scratch memory)
    const bool put0 = prod && wv != 0;
#pragma unroll
    for (int s = 0; s < S; s++) a[s][B] = put0 ? col[s] : a[s][B];
    if constexpr (B + 1 < Q) {
        const bool put1 = prod && wv == 0;
#pragma unroll
        for (int s = 0; s < S; s++) a[s][B + 1] = put1 ? col[s] : a[s][B + 1];
    }
}

// steps LP_WAVES B .. LP_WAVES B + LP_WAVES - 1 (below m)
template <int B>
__device__ __forceinline__ void lt_steps(LtShared & sh, float (&b)[2][LP_Q], int m, int w, int lane, int & spins,
                                         int * __restrict__ status) {
    for (int i = 0; i < LP_WAVES; i++) {
        const int c = LP_WAVES * B + i;
        if (c >= m) break;
        lp_step<2, LP_Q, B>(&sh.ring[0][0].x, sh.plog, sh.inv, sh.phys, b, c, m, w, lane, spins, status);
    }
    if constexpr (B + 1 < LP_Q) {
        if (LP_WAVES * (B + 1) < m) lt_steps<B + 1>(sh, b, m, w, lane, spins, status);
    }
}

// grid (n_chunks * H, L), LP_THREADS threads: the systems of more than 128
// unknowns that k_ge_lu<false, true> did not flag for the masked kernel
// (at most 64 VGPRs: eight waves per SIMD, four systems per CU)
__global__ void __launch_bounds__(LP_THREADS, 8)
k_ge_lu_tail(Geom g, const ChunkDesc * __restrict__ chunks, const float * __restrict__ T2,
             const int * __restrict__ map2, int * __restrict__ perm_out, unsigned char * __restrict__ skip_out,
             float * __restrict__ LU_all, int * __restrict__ redo, int * __restrict__ status) {
    const int c_idx = blockIdx.x / g.H, h = blockIdx.x % g.H, layer = blockIdx.y;
    const int n = chunks[c_idx].tc;
    if (n <= LU_SPLIT || n > RG_ROWS) return;
    const long long sys = ((long long)layer * g.n_chunks + c_idx) * g.H + h;
    if (redo[sys] != 0) return;
    const int m = n - LU_SPLIT;
    const int tid = threadIdx.x, lane = tid & 63, w = __builtin_amdgcn_readfirstlane(tid >> 6);
    __shared__ LtShared sh;
    // rows and columns past m hold zeros; those rows are never live and
    // those columns are never published or written out
    const float * T = T2 + sys * (long long)(LU_SPLIT * LU_SPLIT);
    float b[2][LP_Q];
#pragma unroll
    for (int s = 0; s < 2; s++)
#pragma unroll
        for (int q = 0; q < LP_Q; q++) {
            const int k = lane + 64 * s, j = w + LP_WAVES * q;
            b[s][q] = (k < m && j < m) ? T[j * LU_SPLIT + k] : 0.0f;
        }
    if (tid < LU_SPLIT) {
        sh.inv[(tid & 63) * 2 + (tid >> 6)] = tid < m ? tid : -1;
        sh.phys[tid] = tid;
        sh.plog[tid] = -1;
        sh.map[tid] = tid < m ? map2[sys * LU_SPLIT + tid] : 0;
    }
    __syncthreads();
    if (w == 0) {
        float col[2] = {b[0][0], b[1][0]};
        const int li[2] = {sh.inv[2 * lane], sh.inv[2 * lane + 1]};
        lp_produce<2>(&sh.ring[0][0].x, sh.plog, sh.inv, sh.phys, col, li, 0, 0, lane);
        b[0][0] = col[0];
        b[1][0] = col[1];
    }
    int spins = 0;
    lt_steps<0>(sh, b, m, w, lane, spins, status);
    __builtin_amdgcn_s_setprio(0);
    bool bad = false;
#pragma unroll
    for (int s = 0; s < 2; s++)
#pragma unroll
        for (int q = 0; q < LP_Q; q++)
            bad |= (lane + 64 * s < m) & (w + LP_WAVES * q < m) & lu_nonfinite(b[s][q]);
    const bool redo_sys = __syncthreads_or(bad);
    if (tid == 0) redo[sys] = redo_sys ? 1 : 0;
    if (redo_sys) return;
    if (tid < m) {
        const int pl = sh.plog[tid];
        perm_out[sys * (long long)g.tc_max + LU_SPLIT + tid] = sh.map[pl & 255];
        skip_out[sys * (long long)g.tc_max + LU_SPLIT + tid] = (unsigned char)(pl >> 8);
    }
    // row k's columns 128 .. n - 1 to its physical row, through LDS
    float * LU = LU_all + sys * (long long)RG_ROWS * RG_ROWS;
#pragma unroll
    for (int s = 0; s < 2; s++) {
#pragma unroll
        for (int part = 0; part < 64 / LP_TROWS; part++) {
            const int k0 = 64 * s + LP_TROWS * part;
            if (k0 >= m) break;
            const int lr = lane - LP_TROWS * part;
            if (lr >= 0 && lr < LP_TROWS) {
#pragma unroll
                for (int q = 0; q < LP_Q; q++) sh.tile[lr][w + LP_WAVES * q] = b[s][q];
            }
            __syncthreads();
            for (int e = tid; e < LP_TROWS * m; e += LP_THREADS) {
                const int kk = e / m, j = e - kk * m;
                if (k0 + kk < m) LU[(unsigned)(sh.map[k0 + kk] * RG_ROWS + LU_SPLIT + j)] = sh.tile[kk][j];
            }
            __syncthreads();
        }
    }
}

// Forward substitution y = L^-1 P b (the reference's elimination of the
// right-hand sides: row i receives the updates of steps 0..i-1 in order,
// skipped pivots contribute nothing), then back substitution (math.h:540-556)
// x[i] = (y[i] - sum_{r>i} U[i][r] x[r]) / U[i][i] with r ascending. One wave
// per 64 right-hand sides, lane v owns column v. The first 128 solved rows
// of each sweep move from LDS into registers and are then read through a
// statically unrolled loop; the other rows' earlier results come from LDS.
// Each row of L / U (and its right-hand-side value) is loaded one row ahead
// into registers, so its global-memory latency overlaps the previous row.
constexpr int BS_HIGH = 128;
constexpr int BS_PAD = 128;   // the row buffer holds entry k at rowb[BS_PAD - shift + k]
constexpr int BS_AHEAD = 8;   // backward rows in flight
constexpr int BS_FAHEAD = 4;  // forward 4-row blocks in flight
constexpr int BS_LQ = 6;      // forward: multipliers read ahead in the register part
constexpr int BS_UQ = 6;      // backward: float4 of U read ahead in the register part

// val -= rowp[t] * xsb[t][lane] for t = 0 .. n_terms-1, ascending and
// sequential. Sums of DS_B terms or more run in batches of DS_B: the first
// batch is read at term 0 and applies its first (n_terms % DS_B, else DS_B)
// terms, each later batch starts where the previous one stopped, and every
// batch is read while the one before it is applied (two register sets
// used in turn; a batch past the end is read at the last in-range start
// n_terms - DS_B and not applied, so no read leaves [0, n_terms) and the
// reads need no branches around them). The scheduling fences keep the
// reads ahead of the arithmetic, so the LDS latency overlaps a batch of
// the chain.
constexpr int DS_B = 16;
// val - r[0] * x[0] - r[1] * x[1] - ... in order: the products first, then
// the subtractions back to back (a subtraction issued right after the one
// it depends on waits less than one separated from it by a product).
template <int B>
__device__ __forceinline__ float sub_products(float val, const float (&r)[B], const float (&x)[B]) {
    float p[B];
#pragma unroll
    for (int u = 0; u < B; u++) p[u] = r[u] * x[u];
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int u = 0; u < B; u++) val = val - p[u];
    __builtin_amdgcn_sched_barrier(0);
    return val;
}
__device__ __forceinline__ void ds_load(float (&r)[DS_B], float (&x)[DS_B], const float * rowp,
                                        const float (*xsb)[64], int t0, int lane) {
#pragma unroll
    for (int u = 0; u < DS_B; u++) { r[u] = rowp[t0 + u]; x[u] = xsb[t0 + u][lane]; }
}
// the same batch with rowp + t0 16-byte aligned (float4 reads of rowp)
__device__ __forceinline__ void ds_load4(float (&r)[DS_B], float (&x)[DS_B], const float * rowp,
                                         const float (*xsb)[64], int t0, int lane) {
    const float4 * r4 = reinterpret_cast<const float4 *>(rowp + t0);
#pragma unroll
    for (int q = 0; q < DS_B / 4; q++) {
        const float4 a = r4[q];
        r[4 * q + 0] = a.x; r[4 * q + 1] = a.y; r[4 * q + 2] = a.z; r[4 * q + 3] = a.w;
    }
#pragma unroll
    for (int u = 0; u < DS_B; u++) x[u] = xsb[t0 + u][lane];
}
__device__ __forceinline__ float dot_seq(float val, const float * rowp, const float (*xsb)[64], int n_terms,
                                         int lane) {
    if (n_terms < DS_B) {
        float r[DS_B - 1], x[DS_B - 1];
#pragma unroll
        for (int u = 0; u < DS_B - 1; u++)
            if (u < n_terms) { r[u] = rowp[u]; x[u] = xsb[u][lane]; }
#pragma unroll
        for (int u = 0; u < DS_B - 1; u++)
            if (u < n_terms) val = val - r[u] * x[u];
        return val;
    }
    const int rem = n_terms & (DS_B - 1);
    const int first = rem ? rem : DS_B;
    const int lastb = n_terms - DS_B;
    float ra[DS_B], xa[DS_B], rb[DS_B], xb[DS_B];
    ds_load(ra, xa, rowp, xsb, 0, lane);
    int t = first;
    ds_load(rb, xb, rowp, xsb, min(t, lastb), lane);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int u = 0; u < DS_B; u++)
        if (u < first) val = val - ra[u] * xa[u];
    __builtin_amdgcn_sched_barrier(0);
    while (t < n_terms) {
        ds_load(ra, xa, rowp, xsb, min(t + DS_B, lastb), lane);
        __builtin_amdgcn_sched_barrier(0);
        val = sub_products(val, rb, xb);
        t += DS_B;
        if (t >= n_terms) break;
        ds_load(rb, xb, rowp, xsb, min(t + DS_B, lastb), lane);
        __builtin_amdgcn_sched_barrier(0);
        val = sub_products(val, ra, xa);
        t += DS_B;
    }
    return val;
}

// dot_seq for a number of terms n8 that is a multiple of 8, with rowp
// 16-byte aligned: an odd eighth first, then batches of DS_B read one batch
// ahead as in dot_seq (no partial batch, so no per-term selection).
__device__ __forceinline__ float dot_seq8(float val, const float * rowp, const float (*xsb)[64], int n8,
                                          int lane) {
    if (n8 <= 0) return val;
    const float4 * r4 = reinterpret_cast<const float4 *>(rowp);
    float r8[8], x8[8];
    if (n8 == 8) {
        const float4 a = r4[0], b = r4[1];
        r8[0] = a.x; r8[1] = a.y; r8[2] = a.z; r8[3] = a.w;
        r8[4] = b.x; r8[5] = b.y; r8[6] = b.z; r8[7] = b.w;
#pragma unroll
        for (int u = 0; u < 8; u++) x8[u] = xsb[u][lane];
        return sub_products(val, r8, x8);
    }
    float ra[DS_B], xa[DS_B], rb[DS_B], xb[DS_B];
    int t;
    if (n8 & 8) {
        const float4 a = r4[0], b = r4[1];
        r8[0] = a.x; r8[1] = a.y; r8[2] = a.z; r8[3] = a.w;
        r8[4] = b.x; r8[5] = b.y; r8[6] = b.z; r8[7] = b.w;
#pragma unroll
        for (int u = 0; u < 8; u++) x8[u] = xsb[u][lane];
        ds_load4(rb, xb, rowp, xsb, 8, lane);
        __builtin_amdgcn_sched_barrier(0);
        val = sub_products(val, r8, x8);
        t = 8;
    } else {
        ds_load4(rb, xb, rowp, xsb, 0, lane);
        t = 0;
    }
    const int lastb = n8 - DS_B;
    while (true) {
        ds_load4(ra, xa, rowp, xsb, min(t + DS_B, lastb), lane);
        __builtin_amdgcn_sched_barrier(0);
        val = sub_products(val, rb, xb);
        t += DS_B;
        if (t >= n8) break;
        ds_load4(rb, xb, rowp, xsb, min(t + DS_B, lastb), lane);
        __builtin_amdgcn_sched_barrier(0);
        val = sub_products(val, ra, xa);
        t += DS_B;
        if (t >= n8) break;
    }
    return val;
}

// Four rows at once: val[t] -= lt[j][t] * xsb[j - j1][lane] for j = j1 .. j2-1,
// each row's terms in ascending j (four independent sequential sums);
// lt holds the four rows' entries interleaved (16 bytes per j). Batches of
// D4_B steps, arranged and read ahead as in dot_seq.
constexpr int D4_B = 8;
__device__ __forceinline__ void d4_load(float4 (&l)[D4_B], float (&y)[D4_B], const float4 * lp,
                                        const float (*xsb)[64], int t0, int lane) {
#pragma unroll
    for (int u = 0; u < D4_B; u++) { l[u] = lp[t0 + u]; y[u] = xsb[t0 + u][lane]; }
}
__device__ __forceinline__ void d4_apply(float (&val)[4], const float4 (&l)[D4_B], const float (&y)[D4_B], int cnt) {
#pragma unroll
    for (int u = 0; u < D4_B; u++) {
        if (u < cnt) {
            val[0] = val[0] - l[u].x * y[u];
            val[1] = val[1] - l[u].y * y[u];
            val[2] = val[2] - l[u].z * y[u];
            val[3] = val[3] - l[u].w * y[u];
        }
    }
}
__device__ __forceinline__ void dot4_seq(float (&val)[4], const float4 * lt, const float (*xsb)[64], int j1, int j2,
                                         int lane) {
    const int n_terms = j2 - j1;
    const float4 * lp = lt + j1;
    if (n_terms < D4_B) {
        float4 l[D4_B];
        float y[D4_B];
#pragma unroll
        for (int u = 0; u < D4_B - 1; u++)
            if (u < n_terms) { l[u] = lp[u]; y[u] = xsb[u][lane]; }
        d4_apply(val, l, y, n_terms);
        return;
    }
    const int rem = n_terms & (D4_B - 1);
    const int first = rem ? rem : D4_B;
    const int lastb = n_terms - D4_B;
    float4 la[D4_B], lb[D4_B];
    float ya[D4_B], yb[D4_B];
    d4_load(la, ya, lp, xsb, 0, lane);
    int t = first;
    d4_load(lb, yb, lp, xsb, min(t, lastb), lane);
    __builtin_amdgcn_sched_barrier(0);
    d4_apply(val, la, ya, first);
    __builtin_amdgcn_sched_barrier(0);
    while (t < n_terms) {
        d4_load(la, ya, lp, xsb, min(t + D4_B, lastb), lane);
        __builtin_amdgcn_sched_barrier(0);
        d4_apply(val, lb, yb, D4_B);
        __builtin_amdgcn_sched_barrier(0);
        t += D4_B;
        if (t >= n_terms) break;
        d4_load(lb, yb, lp, xsb, min(t + D4_B, lastb), lane);
        __builtin_amdgcn_sched_barrier(0);
        d4_apply(val, la, ya, D4_B);
        __builtin_amdgcn_sched_barrier(0);
        t += D4_B;
    }
}

// the same sum without the terms of steps whose pivot was skipped (skp[t] == 0)
__device__ __forceinline__ float dot_seq_skip(float val, const float * rowp, const float (*xsb)[64], int n_terms,
                                              const float * skp, int lane) {
    for (int t = 0; t < n_terms; t++)
        if (skp[t] != 0.0f) val = val - rowp[t] * xsb[t][lane];
    return val;
}

__global__ void __launch_bounds__(64)
k_ge_solve(Geom g, const ChunkDesc * __restrict__ chunks, const float * __restrict__ aug,
           const long long * __restrict__ aug_off, const int * __restrict__ perm_in,
           const unsigned char * __restrict__ skip_in, const float * __restrict__ LU_all,
           float * __restrict__ Yt_all, float * __restrict__ Cv, int only_skip) {
    const int sysl = blockIdx.x;   // (layer, chunk, head)
    const int h = sysl % g.H, c_idx = (sysl / g.H) % g.n_chunks, layer = sysl / (g.H * g.n_chunks);
    const ChunkDesc c = chunks[c_idx];
    const int n = c.tc, p = g.dv;
    if (n > RG_ROWS || n < 1) return;
    const int lane = threadIdx.x;
    const int v = blockIdx.y * 64 + lane;
    const bool act = v < p;
    const int vc = act ? v : p - 1;   // in-range column for the loads of idle lanes
    // by physical row: multipliers left of the row's pivot step, U from it on
    const float * __restrict__ LU = LU_all + (long long)sysl * RG_ROWS * RG_ROWS;
    const float * __restrict__ B = aug + aug_off[sysl] + (long long)n * n;   // row-major RHS [r][v]
    float * Yt = Yt_all + (long long)sysl * RG_ROWS * g.dv;
    float * x = Cv + (((long long)layer * g.H + h) * g.t_total + c.off) * g.dv;
    __shared__ float xs[BS_HIGH][64];
    // the forward's interleaved multipliers and the row buffers share LDS:
    // rowb[0] holds the forward's rows when pivots were skipped, and the
    // backward alternates U rows between rowb[0] and rowb[1]
    __shared__ __align__(16) union {
        float4 lt[RG_ROWS];
        float rowb[2][BS_PAD + RG_ROWS];
    } srows;
    float * const rowb = srows.rowb[0];
    __shared__ float skf[RG_ROWS];   // 1 where the step eliminated, 0 where it was skipped
    __shared__ int permL[RG_ROWS];
    __shared__ int any_skip;
    if (lane == 0) any_skip = 0;
    __builtin_amdgcn_wave_barrier();
    for (int i = lane; i < RG_ROWS; i += 64) {
        const int sk = (i < n) ? skip_in[(long long)sysl * g.tc_max + i] : 0;
        skf[i] = sk ? 0.0f : 1.0f;
        permL[i] = (i < n) ? perm_in[(long long)sysl * g.tc_max + i] : 0;
        if (sk) any_skip = 1;
    }
    __builtin_amdgcn_wave_barrier();
    const bool sk = any_skip != 0;
    if (only_skip && !sk) return;         // k_ge_subst solved this system
    const float * frow = rowb + BS_PAD;   // forward rows, unshifted
    float4 * frow4 = reinterpret_cast<float4 *>(rowb + BS_PAD);

    float4 pf;
    float pb;
    if (!sk) {
        // ---- forward, four rows at a time (no skipped pivots): the rows'
        // multipliers sit interleaved in LDS; earlier results come from LDS
        // (rows below 128 until row 128, then from registers) and the four
        // sums run side by side; the 4 x 4 triangle finishes them in order.
        float4 * const lt = srows.lt;
        float yr[BS_HIGH];
        // rows and right-hand sides of the next BS_FAHEAD blocks in flight
        float4 qf[BS_FAHEAD][4];
        float qb[BS_FAHEAD][4];
        auto fetch = [&](int i0, float4 (&f)[4], float (&bb)[4]) {
#pragma unroll
            for (int t = 0; t < 4; t++) {
                const int r = permL[(i0 + t < n) ? i0 + t : i0];
                f[t] = reinterpret_cast<const float4 *>(LU + (unsigned)(r * RG_ROWS))[lane];
                bb[t] = B[(unsigned)(r * p + vc)];
            }
        };
#pragma unroll
        for (int k = 0; k < BS_FAHEAD; k++)
            if (4 * k < n) fetch(4 * k, qf[k], qb[k]);
        for (int ib = 0; ib < n; ib += 4 * BS_FAHEAD) {
#pragma unroll
        for (int k = 0; k < BS_FAHEAD; k++) {
            const int i0 = ib + 4 * k;
            if (i0 >= n) break;
            const int nr = min(4, n - i0);
            lt[4 * lane + 0] = make_float4(qf[k][0].x, qf[k][1].x, qf[k][2].x, qf[k][3].x);
            lt[4 * lane + 1] = make_float4(qf[k][0].y, qf[k][1].y, qf[k][2].y, qf[k][3].y);
            lt[4 * lane + 2] = make_float4(qf[k][0].z, qf[k][1].z, qf[k][2].z, qf[k][3].z);
            lt[4 * lane + 3] = make_float4(qf[k][0].w, qf[k][1].w, qf[k][2].w, qf[k][3].w);
            float val[4];
#pragma unroll
            for (int t = 0; t < 4; t++) val[t] = act ? qb[k][t] : 0.0f;
            fetch(min(i0 + 4 * BS_FAHEAD, n - 1), qf[k], qb[k]);   // unconditional, as in the backward ring
            __builtin_amdgcn_wave_barrier();
            if (i0 <= BS_HIGH) {
                dot4_seq(val, lt, xs, 0, i0, lane);
            } else {
                // entries read BS_LQ steps ahead of their use
                float4 lq[BS_HIGH];
#pragma unroll
                for (int j = 0; j < BS_LQ; j++) lq[j] = lt[j];
#pragma unroll
                for (int j = 0; j < BS_HIGH; j++) {
                    if (j + BS_LQ < BS_HIGH) lq[j + BS_LQ] = lt[j + BS_LQ];
                    __builtin_amdgcn_sched_barrier(0);
                    val[0] = val[0] - lq[j].x * yr[j];
                    val[1] = val[1] - lq[j].y * yr[j];
                    val[2] = val[2] - lq[j].z * yr[j];
                    val[3] = val[3] - lq[j].w * yr[j];
                    __builtin_amdgcn_sched_barrier(0);
                }
                dot4_seq(val, lt + BS_HIGH, xs, 0, i0 - BS_HIGH, lane);
            }
            // the block's own triangle, row by row
            float yn[4];
#pragma unroll
            for (int t = 0; t < 4; t++) {
#pragma unroll
                for (int q = 0; q < 4; q++)
                    if (q < t) val[t] = val[t] - reinterpret_cast<const float *>(&lt[i0 + q])[t] * yn[q];
                yn[t] = val[t];
            }
#pragma unroll
            for (int t = 0; t < 4; t++) {
                if (t >= nr) break;
                const int i = i0 + t;
                xs[i < BS_HIGH ? i : i - BS_HIGH][lane] = yn[t];
                if (act) Yt[(unsigned)(i * g.dv + v)] = yn[t];
            }
            __builtin_amdgcn_wave_barrier();
            if (i0 + 4 == BS_HIGH && n > BS_HIGH) {
#pragma unroll
                for (int j = 0; j < BS_HIGH; j++) yr[j] = xs[j][lane];
                __builtin_amdgcn_wave_barrier();
            }
        }
        }
    } else {
    // ---- forward: rows [0, lb) from LDS, then rows [lb, n) with [0, lb) in registers
    const int lb = n < BS_HIGH ? n : BS_HIGH;
    pf = reinterpret_cast<const float4 *>(LU + (unsigned)(permL[0] * RG_ROWS))[lane];
    pb = B[(unsigned)(permL[0] * p + vc)];
    for (int i = 0; i < lb; i++) {
        frow4[lane] = pf;
        float val = act ? pb : 0.0f;
        if (i + 1 < n) {
            const int rn = permL[i + 1];
            pf = reinterpret_cast<const float4 *>(LU + (unsigned)(rn * RG_ROWS))[lane];
            pb = B[(unsigned)(rn * p + vc)];
        }
        __builtin_amdgcn_wave_barrier();
        val = sk ? dot_seq_skip(val, frow, xs, i, skf, lane) : dot_seq(val, frow, xs, i, lane);
        xs[i][lane] = val;
        if (act) Yt[(unsigned)(i * g.dv + v)] = val;
        __builtin_amdgcn_wave_barrier();
    }
    if (n > BS_HIGH) {
        float yr[BS_HIGH];
#pragma unroll
        for (int j = 0; j < BS_HIGH; j++) yr[j] = xs[j][lane];
        for (int i = BS_HIGH; i < n; i++) {
            frow4[lane] = pf;
            float val = act ? pb : 0.0f;
            if (i + 1 < n) {
                const int rn = permL[i + 1];
                pf = reinterpret_cast<const float4 *>(LU + (unsigned)(rn * RG_ROWS))[lane];
                pb = B[(unsigned)(rn * p + vc)];
            }
            __builtin_amdgcn_wave_barrier();
            if (!sk) {
#pragma unroll
                for (int j = 0; j < BS_HIGH; j++) val -= frow[j] * yr[j];
                val = dot_seq(val, frow + BS_HIGH, xs, i - BS_HIGH, lane);
            } else {
#pragma unroll
                for (int j = 0; j < BS_HIGH; j++)
                    if (skf[j] != 0.0f) val -= frow[j] * yr[j];
                val = dot_seq_skip(val, frow + BS_HIGH, xs, i - BS_HIGH, skf + BS_HIGH, lane);
            }
            xs[i - BS_HIGH][lane] = val;
            if (act) Yt[(unsigned)(i * g.dv + v)] = val;
            __builtin_amdgcn_wave_barrier();
        }
    }
    }

    // ---- backward: rows [hb, n) first, then rows [0, hb) with [hb, n) in
    // registers (xh). Rows run in groups of BS_AHEAD from the top of each
    // part (n - hb is a multiple of BS_AHEAD), so a row's sum splits into
    // the rows above it in its own group (kept in registers, w), the earlier
    // groups of its part (from LDS, a multiple of 8 terms) and, below hb,
    // the register part; each piece ascends, in that order. Row col of U
    // sits at rowb[k & 1] + bsh (k = the row's place in its group), written
    // while the row before it runs; bsh places the entries of the earlier
    // groups (col0 + 1 on) 16-byte aligned and, when hb > 0, the register
    // part's entries (hb on) too. U rows and y values are loaded BS_AHEAD
    // rows ahead through a register ring.
    const int hb = n > BS_HIGH ? n - BS_HIGH : 0;
    const int bsh = BS_PAD - hb - (hb > 0 ? 0 : (n & 3));
    float xh[BS_HIGH];
    float w[BS_AHEAD];
    float4 rf[BS_AHEAD];
    float rb[BS_AHEAD];
#pragma unroll
    for (int k = 0; k < BS_AHEAD; k++) {
        const int r = max(n - 1 - k, 0);
        rf[k] = reinterpret_cast<const float4 *>(LU + (unsigned)(permL[r] * RG_ROWS))[lane];
        rb[k] = Yt[(unsigned)(r * g.dv + vc)];
    }
    {
        float * b0 = srows.rowb[0] + bsh;
        b0[4 * lane + 0] = rf[0].x;
        b0[4 * lane + 1] = rf[0].y;
        b0[4 * lane + 2] = rf[0].z;
        b0[4 * lane + 3] = rf[0].w;
    }
    for (int col0 = n - 1; col0 >= 0; col0 -= BS_AHEAD) {
        const bool upper = col0 >= hb;            // the whole group is on one side of hb
        const int xoff = upper ? hb : 0;           // row r's result sits at xs[r - xoff]
        const int n8 = (upper ? n : hb) - col0 - 1;   // earlier groups of this part
        // physical rows of the next group, lane k holding row col0 - BS_AHEAD - k
        const int pnext = permL[max(col0 - BS_AHEAD - (lane & (BS_AHEAD - 1)), 0)];
#pragma unroll
        for (int k = 0; k < BS_AHEAD; k++) {
            const int col = col0 - k;
            if (col < 0) break;
            if (col == hb - 1) {
                // entering the rows below hb: rows [hb, n) move to registers
#pragma unroll
                for (int i = 0; i < BS_HIGH; i++) xh[i] = xs[i][lane];
                __builtin_amdgcn_wave_barrier();
            }
            const float * brow = srows.rowb[k & 1] + bsh;
            const float * bhi = srows.rowb[k & 1] + BS_PAD;   // == brow + hb when hb > 0
            {
                // the next row's U (ring slot k + 1) into the other buffer
                float * bn = srows.rowb[(k + 1) & 1] + bsh;
                const float4 f = rf[(k + 1) % BS_AHEAD];
                bn[4 * lane + 0] = f.x;
                bn[4 * lane + 1] = f.y;
                bn[4 * lane + 2] = f.z;
                bn[4 * lane + 3] = f.w;
            }
            const float yv = rb[k];
            const float piv = brow[col];
            float ug[BS_AHEAD];   // U entries of the rows above col in the group
#pragma unroll
            for (int j = 0; j < k; j++) ug[j] = brow[col + 1 + j];
            float val = g.zero_val;
            if (!(fabsf(piv) < 1e-12f)) {
                val = act ? yv : 0.0f;
                if (k > 0) {
                    float pg[BS_AHEAD];
#pragma unroll
                    for (int j = 0; j < k; j++) pg[j] = ug[j] * w[k - 1 - j];
                    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
                    for (int j = 0; j < k; j++) val = val - pg[j];
                    __builtin_amdgcn_sched_barrier(0);
                }
                val = dot_seq8(val, brow + col0 + 1, xs + (col0 + 1 - xoff), n8, lane);
                if (!upper) {
                    // U entries read BS_UQ float4 ahead of their use
                    const float4 * bhi4 = reinterpret_cast<const float4 *>(bhi);
                    float4 uq[BS_HIGH / 4];
#pragma unroll
                    for (int q = 0; q < BS_UQ; q++) uq[q] = bhi4[q];
#pragma unroll
                    for (int q = 0; q < BS_HIGH / 4; q += 2) {
                        if (q + BS_UQ < BS_HIGH / 4) uq[q + BS_UQ] = bhi4[q + BS_UQ];
                        if (q + 1 + BS_UQ < BS_HIGH / 4) uq[q + 1 + BS_UQ] = bhi4[q + 1 + BS_UQ];
                        __builtin_amdgcn_sched_barrier(0);
                        const float r8[8] = {uq[q].x, uq[q].y, uq[q].z, uq[q].w,
                                             uq[q + 1].x, uq[q + 1].y, uq[q + 1].z, uq[q + 1].w};
                        const float x8[8] = {xh[4 * q + 0], xh[4 * q + 1], xh[4 * q + 2], xh[4 * q + 3],
                                             xh[4 * q + 4], xh[4 * q + 5], xh[4 * q + 6], xh[4 * q + 7]};
                        val = sub_products(val, r8, x8);
                    }
                }
                val = val / piv;
            }
            w[k] = val;
            xs[col - xoff][lane] = val;
            {
                // the slot's next row, refilled once its values are dead and
                // unconditionally (row 0 again near the end): otherwise the
                // slot holds two live values, and the copy that merges them
                // waits for every load in flight
                const int r = max(col - BS_AHEAD, 0);
                const int pr = __builtin_amdgcn_readlane(pnext, k);
                rf[k] = reinterpret_cast<const float4 *>(LU + (unsigned)(pr * RG_ROWS))[lane];
                rb[k] = Yt[(unsigned)(r * g.dv + vc)];
            }
            __builtin_amdgcn_wave_barrier();
        }
    }
    // the solution goes out after the sweep (stores inside it would make
    // the waits for the row loads drain every access in flight): rows
    // [0, hb) from LDS, rows [hb, n) from registers when n > BS_HIGH
    if (act) {
        for (int i = 0; i < (hb > 0 ? hb : n); i++) x[(unsigned)(i * g.dv + v)] = xs[i][lane];
        if (hb > 0) {
#pragma unroll
            for (int i = 0; i < BS_HIGH; i++) x[(unsigned)((hb + i) * g.dv + v)] = xh[i];
        }
    }
}

// ---------------------------------------------------------------------------
// Forward and back substitution of the register-LU systems (n <= 256). The
// forward pass is the reference's elimination of the right-hand-side columns
// (math.h:531-537): the row that ends at logical position i receives the
// updates of steps 0 .. i-1 in step order, y_i = b - f_0 y_0 - f_1 y_1 - ...,
// and a skipped step updates no row. The backward pass is math.h:540-556:
// x_i = (y_i - U[i][i+1] x_{i+1} - U[i][i+2] x_{i+2} - ...) / U[i][i], the
// solution value of a skipped pivot (|U[i][i]| < 1e-12) being zero_val.
//
// One wave per 64 right-hand-side columns (lane = column), the waves of a
// system in one block, two waves per SIMD. A column's 256 values sit in 32
// groups of eight rows: 23 groups in registers, 9 in LDS (the most that lets
// two waves share a SIMD with nothing spilled: the 23 groups take 184 of 256
// registers, and a tenth group in LDS would leave room for three blocks of
// four on the CU's 160 KB). Registers are only
// indexed statically, so they form a stack: a new group enters at block 0 and
// the others move down one block. Each pass reads the stack in a fixed order
// with a uniform guard per block:
//  - forward: block m holds group cnt-1-m (cnt = groups in registers), read
//    oldest first; groups 23-31 go to LDS (the earliest rows, read by every
//    later row, stay in registers);
//  - backward: block m holds the solution of group gb+1+m, read newest first,
//    and the bottom blocks hold the y groups still to be consumed, the next
//    one in the last block; once solved groups fill the stack the oldest
//    moves to the LDS slot of the y group just consumed.
// Between the passes the blocks are permuted statically into the backward's
// order. Entries of L and U are the same for every lane of a wave: they come
// in vector loads that replicate sixteen of them in each 16-lane row, and a
// DPP broadcast folds each into the multiply that uses it (an SGPR operand,
// which a scalar load would give, costs the multiply as much issue time, and
// scalar loads return out of order, so a pipeline of them waits on all at
// once; vector loads return in order and run several blocks ahead). The
// forward pass sums the eight rows of a group side by side (independent
// chains); the backward pass is one chain per column (each row's sum starts
// with the row solved just before it). Rows past n are processed
// as zero rows: their values stay zero and the factor array holds zeros in
// their columns, so their terms (0 * 0 subtracted from a sum that is never -0)
// change nothing and the sums need no guards.
// ---------------------------------------------------------------------------
constexpr int SB_G = 8;                     // rows per group (and entries per block)
constexpr int SB_NG = RG_ROWS / SB_G;       // groups of a column
constexpr int SB_RG = 23;                   // groups held in registers
constexpr int SB_LG = SB_NG - SB_RG;        // groups held in LDS
constexpr int SB_LDS = SB_LG * SB_G;        // stored LDS rows per lane
constexpr int SB_LROWS = SB_LDS + 1;        // plus one row for the sink of the cache warm-up loads

// N consecutive entries of a row of the factor array (uniform address: scalar loads)
template <int N>
__device__ __forceinline__ void sb_load(float (&u)[N], const float * __restrict__ row, int k0) {
#pragma unroll
    for (int j = 0; j < N; j++) u[j] = row[k0 + j];
}

// Scalar loads return out of order, so a wait covers every load in flight:
// the next block's loads are issued after the wait for the current block's
// and before its arithmetic.
__device__ __forceinline__ void sb_wait_scalar() {
    __builtin_amdgcn_s_waitcnt(0xc07f);   // lgkmcnt(0), vmcnt and expcnt unchanged
    __builtin_amdgcn_sched_barrier(0);
}

// slot s of the lanes' permutation entries (perm[l + 64 s] in lane l), for a
// uniform s; masks rather than a select chain, which the compiler may turn
// into an indexed private array
__device__ __forceinline__ int sb_pvslot(const int (&pv)[4], int s) {
    return (pv[0] & -(int)(s == 0)) | (pv[1] & -(int)(s == 1)) | (pv[2] & -(int)(s == 2)) | (pv[3] & -(int)(s == 3));
}

// perm[i] for a uniform i, from the lanes' entries
__device__ __forceinline__ int sb_perm(const int (&pv)[4], int i) {
    return __builtin_amdgcn_readlane(sb_pvslot(pv, i >> 6), i & 63);
}

// push a group onto the register stack
__device__ __forceinline__ void sb_push(float (&R)[SB_RG][SB_G], const float (&g)[SB_G]) {
#pragma unroll
    for (int m = SB_RG - 1; m > 0; m--)
#pragma unroll
        for (int j = 0; j < SB_G; j++) R[m][j] = R[m - 1][j];
#pragma unroll
    for (int j = 0; j < SB_G; j++) R[0][j] = g[j];
}

// Forward pass: the eight rows of a group side by side (eight independent
// sums share each y value). The entries of the eight L rows for the eight
// steps of one earlier group come in one 16-byte vector load per lane: lane l
// of every 16-lane row loads entries 8 G + 4 (l & 1) .. + 3 of row
// (l & 15) >> 1, so component q holds L[t][8 G + 4 j4 + q] in lane 2 t + j4
// of each 16-lane row, and a DPP broadcast folds it into the multiply. Vector
// loads return in order, so the loads run SB_FD groups ahead of the
// arithmetic (SB_FD + 1 buffers: a block issues its load into the buffer
// the block before it used, then works on its own) with no wait beyond the
// one for the group being used.
constexpr int SB_FD = 2;
constexpr int SB_FB = SB_FD + 1;
constexpr int SB_FSINK = 11;   // the block of the load sequence that issues the cache warm-up loads

__device__ __forceinline__ float4 sb_fload(const float * __restrict__ LU, unsigned off) {
    return *reinterpret_cast<const float4 *>(LU + off);
}

// L[T][8 G + J] from the group's load, in every lane
template <int J, int T>
__device__ __forceinline__ float sb_fl(const float4 & b) {
    constexpr int q = J & 3;
    return sb_bc<2 * T + (J >> 2)>(q == 0 ? b.x : q == 1 ? b.y : q == 2 ? b.z : b.w);
}

// val[t] -= L[t][8 G + J] * y for the eight rows t
template <int J, int... T>
__device__ __forceinline__ void sb_fstep(float (&val)[SB_G], const float4 & b, float y,
                                         std::integer_sequence<int, T...>) {
    float pr[SB_G];
    ((pr[T] = sb_fl<J, T>(b) * y), ...);
    ((val[T] = val[T] - pr[T]), ...);
}

// the eight steps of one earlier group, ascending
template <int... J>
__device__ __forceinline__ void sb_fterms(float (&val)[SB_G], const float4 & b, const float * y,
                                          std::integer_sequence<int, J...>) {
    (sb_fstep<J>(val, b, y[J], std::make_integer_sequence<int, SB_G>{}), ...);
}

// the group's own steps: row T takes steps 8 gi + R, R < T, ascending, from
// the rows finished before it
template <int T, int... R>
__device__ __forceinline__ void sb_ftri_row(float (&val)[SB_G], const float4 & b, std::integer_sequence<int, R...>) {
    ((val[T] = val[T] - sb_fl<R, T>(b) * val[R]), ...);
}
template <int... T>
__device__ __forceinline__ void sb_ftri(float (&val)[SB_G], const float4 & b, std::integer_sequence<int, T...>) {
    (sb_ftri_row<T>(val, b, std::make_integer_sequence<int, T>{}), ...);
}

// one group of the forward pass: its eight results in yg (zero past n). Rows
// 8 gi .. 8 gi + 7 take the steps of every earlier group (the register
// stack oldest first, then the LDS groups), then the group's own steps.
// rows 8 gi .. 8 gi + 7 of the right-hand sides (rows past n read row n - 1)
__device__ __forceinline__ void sb_bload(float (&b)[SB_G], const float * __restrict__ B, const int (&pv)[4], int gi,
                                         int n, int p, int vc) {
#pragma unroll
    for (int t = 0; t < SB_G; t++) {
        const int pr = sb_perm(pv, min(SB_G * gi + t, n - 1));
        b[t] = B[(unsigned)(pr * p + vc)];
    }
}

// bn: this group's right-hand-side values on entry (loaded during the group
// before), the next group's on exit
__device__ __forceinline__ void sb_fgroup(float (&yg)[SB_G], const float (&R)[SB_RG][SB_G], float (*zl)[64],
                                          const float * __restrict__ LU, const float * __restrict__ B,
                                          const int (&pv)[4], int gi, int n, int p, int vc, int lane, float & pf,
                                          float (&bn)[SB_G]) {
    if (SB_G * gi >= n) {
#pragma unroll
        for (int j = 0; j < SB_G; j++) yg[j] = 0.0f;
        return;
    }
    // the lane's L row for the group's loads (rows past n read row n - 1,
    // whose results are discarded); the group's rows share one 64-row slot
    // of the permutation
    const int rt = min(SB_G * gi + ((lane & 15) >> 1), n - 1);
    const int prow = __builtin_amdgcn_ds_bpermute(4 * (rt & 63), sb_pvslot(pv, gi >> 3));
    const unsigned vb = (unsigned)(prow * RG_ROWS + 4 * (lane & 1));
    float val[SB_G];
#pragma unroll
    for (int t = 0; t < SB_G; t++) val[t] = bn[t];
    int cnt = min(gi, SB_RG);
    // (opaque to the compiler, so that each block tests it afresh rather than
    // keeping 23 comparison results alive)
    asm volatile("" : "+s"(cnt));
    // Register groups, oldest first: block m holds group cnt - 1 - m. Block m
    // uses buffer m % SB_FB, which block m + SB_FD loaded: every block,
    // m = SB_RG + SB_FD - 1 .. 0, first loads the group SB_FD blocks on (its
    // index clamped to 0 .. gi) into the buffer of block m + 1, then (m <
    // cnt) works on its own. The blocks not in use load too, so that every
    // path through the sequence issues the same loads and each wait is for
    // exactly the load it needs. The last loads go past the register groups:
    // to the LDS groups, or to group gi (the group's own steps).
    float4 fb[SB_FB];
    float w[2], bnext[SB_G];
#pragma unroll
    for (int m = SB_RG + SB_FD - 1; m >= 0; m--) {
        const int G = min(max(cnt - 1 - m + SB_FD, 0), gi);
        fb[(m + 1) % SB_FB] = sb_fload(LU, vb + SB_G * G);
        if (m == SB_FSINK) {
            // the next group's eight L rows into the caches (lane l: line
            // l & 15 of row l >> 4 of each half; the values only feed the
            // sink, at the end of the group), so that its first loads hit
            // them, and its right-hand-side values into registers. Issued
            // here, mid-sequence, because the loads after them in the
            // in-order queue are not waited for until several blocks on.
            const int r = min(SB_G * (gi + 1) + (lane >> 4), n - 1);
            const int r2 = min(SB_G * (gi + 1) + 4 + (lane >> 4), n - 1);
            const int pr = __builtin_amdgcn_ds_bpermute(4 * (r & 63), sb_pvslot(pv, r >> 6));
            const int pr2 = __builtin_amdgcn_ds_bpermute(4 * (r2 & 63), sb_pvslot(pv, r2 >> 6));
            w[0] = LU[(unsigned)(pr * RG_ROWS + 16 * (lane & 15))];
            w[1] = LU[(unsigned)(pr2 * RG_ROWS + 16 * (lane & 15))];
            sb_bload(bnext, B, pv, min(gi + 1, SB_NG - 1), n, p, vc);
        }
        if (m < SB_RG && m < cnt)
            sb_fterms(val, fb[m % SB_FB], &R[m][0], std::make_integer_sequence<int, SB_G>{});
    }
    // blocks 1 and 0 loaded groups cnt and cnt + 1 (clamped to gi) into
    // buffers 2 and 1; the LDS groups SB_RG .. gi - 1 (present only when the
    // stack is full) continue the sequence, and the group after the last
    // one, gi, ends in cur
    static_assert(SB_FD == 2 && SB_FB == 3, "the buffer rotation assumes two groups in flight");
    float4 cur = fb[2], nxt = fb[1];
    for (int G = SB_RG; G < gi; G++) {
        const float4 fre = sb_fload(LU, vb + SB_G * min(G + SB_FD, gi));
        float y[SB_G];
#pragma unroll
        for (int j = 0; j < SB_G; j++) y[j] = zl[SB_G * (G - SB_RG) + j][lane];
        sb_fterms(val, cur, y, std::make_integer_sequence<int, SB_G>{});
        cur = nxt;
        nxt = fre;
    }
    sb_ftri(val, cur, std::make_integer_sequence<int, SB_G>{});
#pragma unroll
    for (int t = 0; t < SB_G; t++) yg[t] = SB_G * gi + t < n ? val[t] : 0.0f;
    pf = fmaxf(pf, fmaxf(w[0], w[1]));
#pragma unroll
    for (int t = 0; t < SB_G; t++) bn[t] = bnext[t];
}

__device__ __forceinline__ void sb_forward(float (&R)[SB_RG][SB_G], float (*zl)[64], const float * __restrict__ LU,
                                           const float * __restrict__ B, const int (&pv)[4], int n, int p, int vc,
                                           int lane, float & pf) {
    // groups 0 .. SB_RG - 1 onto the register stack, the rest into LDS
    float bn[SB_G];
    sb_bload(bn, B, pv, 0, n, p, vc);
    for (int gi = 0; gi < SB_RG; gi++) {
        float yg[SB_G];
        sb_fgroup(yg, R, zl, LU, B, pv, gi, n, p, vc, lane, pf, bn);
        sb_push(R, yg);
    }
    for (int gi = SB_RG; gi < SB_NG; gi++) {
        float yg[SB_G];
        sb_fgroup(yg, R, zl, LU, B, pv, gi, n, p, vc, lane, pf, bn);
#pragma unroll
        for (int j = 0; j < SB_G; j++) zl[SB_G * (gi - SB_RG) + j][lane] = yg[j];
    }
}

// Backward pass. On entry block m holds y group SB_LG + m and LDS slot s y
// group s; on exit block m holds x group m and LDS slot s x group SB_RG + s.
// A row's U entries come in vector loads from its group's first column g0,
// sixteen entries per register (register i: entries g0 + 16 i + 0..15, each
// in every 16-lane row), and a DPP broadcast folds each into its multiply.
// Registers 0..11 cover the register blocks (entries g0 + 8 .. g0 + 191),
// 12..15 the LDS slots (g0 + 192 .. g0 + 255). Loads past the row's end
// (g0 + 16 i + 15 > 255, at most 247 entries) read the next physical row, or
// for the last row of the last system the factor array's padding; those
// entries are never used. One address per row, the registers at immediate
// offsets. The next row's entries load while a row runs.
constexpr int SB_US = RG_ROWS / 16;

__device__ __forceinline__ void sb_uload(float (&us)[SB_US], const float * __restrict__ LU, const int (&pv)[4],
                                         int col, int lane) {
    const int g0 = col & ~(SB_G - 1);
    const float * __restrict__ rp = LU + (unsigned)(sb_perm(pv, col) * RG_ROWS + g0 + (lane & 15));
#pragma unroll
    for (int i = 0; i < SB_US; i++) us[i] = rp[16 * i];
}

// products of register block M (entries g0 + 8 (M + 1) + J) with its results
template <int M, int... J>
__device__ __forceinline__ void sb_bprod(float (&pr)[SB_G], const float (&us)[SB_US], const float (&R)[SB_RG][SB_G],
                                         std::integer_sequence<int, J...>) {
    ((pr[J] = sb_bc<(SB_G * (M + 1) + J) % 16>(us[(SB_G * (M + 1) + J) / 16]) * R[M][J]), ...);
}
template <int M>
__device__ __forceinline__ void sb_bblock(float & val, const float (&us)[SB_US], const float (&R)[SB_RG][SB_G],
                                          int nxr) {
    if (M < nxr) {
        float pr[SB_G];
        sb_bprod<M>(pr, us, R, std::make_integer_sequence<int, SB_G>{});
#pragma unroll
        for (int j = 0; j < SB_G; j++) val = val - pr[j];
    }
}
template <int... M>
__device__ __forceinline__ void sb_bblocks(float & val, const float (&us)[SB_US], const float (&R)[SB_RG][SB_G],
                                           int nxr, std::integer_sequence<int, M...>) {
    (sb_bblock<M>(val, us, R, nxr), ...);
}
// LDS slot gb + D (solved group gb + SB_RG + D, entries g0 + 8 (SB_RG + D) + J)
template <int D, int... J>
__device__ __forceinline__ void sb_bslot(float & val, const float (&us)[SB_US], float (*zl)[64], int gb, int lane,
                                         std::integer_sequence<int, J...>) {
    if (gb + D < SB_LG) {
        float x[SB_G], pr[SB_G];
        ((x[J] = zl[SB_G * (gb + D) + J][lane]), ...);
        ((pr[J] = sb_bc<(SB_G * (SB_RG + D) + J) % 16>(us[(SB_G * (SB_RG + D) + J) / 16]) * x[J]), ...);
        ((val = val - pr[J]), ...);
    }
}
template <int... D>
__device__ __forceinline__ void sb_bslots(float & val, const float (&us)[SB_US], float (*zl)[64], int gb, int lane,
                                          std::integer_sequence<int, D...>) {
    (sb_bslot<D + 1>(val, us, zl, gb, lane, std::make_integer_sequence<int, SB_G>{}), ...);
}
// the rows above row K of its group (entries g0 + J, J > K), ascending
template <int K, int... J>
__device__ __forceinline__ void sb_bgroup_terms(float & val, float us0, const float (&xw)[SB_G],
                                                std::integer_sequence<int, J...>) {
    ((J > K ? (void)(val = val - sb_bc<J>(us0) * xw[J]) : (void)0), ...);
}

// row K of group gb (logical row 8 gb + K; nothing past n): its result into
// xw[K]. us holds the row's U entries on entry and the next row's on exit.
template <int K>
__device__ __forceinline__ void sb_brow(float (&xw)[SB_G], float yk, const float (&R)[SB_RG][SB_G], float (*zl)[64],
                                        const float * __restrict__ LU, const int (&pv)[4], int gb, int nx, int n,
                                        float zero_val, int lane, float (&us)[SB_US]) {
    const int col = SB_G * gb + K;
    if (col >= n) return;
    // the next row's entries (the next group's first row after row 0) while
    // this row runs
    float un[SB_US];
    sb_uload(un, LU, pv, max(col - 1, 0), lane);
    const float piv = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(us[0]), K));
    float val = zero_val;
    if (!(fabsf(piv) < 1e-12f)) {
        val = yk;
        sb_bgroup_terms<K>(val, us[0], xw, std::make_integer_sequence<int, SB_G>{});
        // solved groups in registers, newest (lowest rows) first (nx opaque:
        // tested per row, not kept from the row before)
        int nxr = nx;
        asm volatile("" : "+s"(nxr));
        sb_bblocks(val, us, R, nxr, std::make_integer_sequence<int, SB_RG>{});
        // solved groups gb + SB_RG + 1 .. 31 in LDS slots gb + 1 .. SB_LG - 1
        sb_bslots(val, us, zl, gb, lane, std::make_integer_sequence<int, SB_LG - 1>{});
        val = val / piv;
    }
    xw[K] = val;
#pragma unroll
    for (int i = 0; i < SB_US; i++) us[i] = un[i];
}

// one group of the backward pass: its results xw from its y values yw, the
// rows from the last (the highest below n) to the first, each unrolled so
// that its place in the group is a constant (its y value a register); us
// holds the U entries of the group's first row on entry and those of the
// next group's first row on exit
template <int... K>
__device__ __forceinline__ void sb_bgroup(float (&xw)[SB_G], const float (&yw)[SB_G], const float (&R)[SB_RG][SB_G],
                                          float (*zl)[64], const float * __restrict__ LU, const int (&pv)[4],
                                          int gb, int n, float zero_val, int lane, float (&us)[SB_US],
                                          std::integer_sequence<int, K...>) {
    const int nx = min(SB_NG - 1 - gb, SB_RG);   // solved groups in registers
#pragma unroll
    for (int j = 0; j < SB_G; j++) xw[j] = 0.0f;
    (sb_brow<SB_G - 1 - K>(xw, yw[SB_G - 1 - K], R, zl, LU, pv, gb, nx, n, zero_val, lane, us), ...);
}

__device__ __forceinline__ void sb_backward(float (&R)[SB_RG][SB_G], float (*zl)[64], const float * __restrict__ LU,
                                            const int (&pv)[4], int n, float zero_val, int lane) {
    float us[SB_US];
    sb_uload(us, LU, pv, n - 1, lane);
    // groups 31 .. SB_LG: y from the bottom block, which the pushed result replaces
    for (int gb = SB_NG - 1; gb >= SB_LG; gb--) {
        float yw[SB_G], xw[SB_G];
#pragma unroll
        for (int j = 0; j < SB_G; j++) yw[j] = R[SB_RG - 1][j];
        sb_bgroup(xw, yw, R, zl, LU, pv, gb, n, zero_val, lane, us, std::make_integer_sequence<int, SB_G>{});
        sb_push(R, xw);
    }
    // groups SB_LG - 1 .. 0: y from LDS; the oldest solved group moves to its slot
    for (int gb = SB_LG - 1; gb >= 0; gb--) {
        float yw[SB_G], xw[SB_G];
#pragma unroll
        for (int j = 0; j < SB_G; j++) yw[j] = zl[SB_G * gb + j][lane];
        sb_bgroup(xw, yw, R, zl, LU, pv, gb, n, zero_val, lane, us, std::make_integer_sequence<int, SB_G>{});
#pragma unroll
        for (int j = 0; j < SB_G; j++) zl[SB_G * gb + j][lane] = R[SB_RG - 1][j];
        sb_push(R, xw);
    }
}

// grid (systems), block 64 * ceil(p / 64); dynamic LDS SB_LROWS rows x
// 64 lanes per wave
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2)))
k_ge_subst(Geom g, const ChunkDesc * __restrict__ chunks, const float * __restrict__ aug,
           const long long * __restrict__ aug_off, const int * __restrict__ perm_in,
           const unsigned char * __restrict__ skip_in, const float * __restrict__ LU_all, float * __restrict__ Cv) {
    const int sysl = blockIdx.x;   // (layer, chunk, head)
    const int h = sysl % g.H, c_idx = (sysl / g.H) % g.n_chunks, layer = sysl / (g.H * g.n_chunks);
    const ChunkDesc c = chunks[c_idx];
    const int n = c.tc, p = g.dv;
    if (n > RG_ROWS || n < 1) return;
    const int wv = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int v = wv * 64 + lane;
    const bool act = v < p;
    const int vc = act ? v : p - 1;
    const float * __restrict__ LU = LU_all + (long long)sysl * RG_ROWS * RG_ROWS;
    const float * __restrict__ B = aug + aug_off[sysl] + (long long)n * n;   // row-major RHS [r][v]
    float * __restrict__ x = Cv + (((long long)layer * g.H + h) * g.t_total + c.off) * g.dv;
    extern __shared__ float sb_lds[];
    float (*zl)[64] = reinterpret_cast<float (*)[64]>(sb_lds + (size_t)wv * SB_LROWS * 64);
    // permutation by logical row (lane l holds rows l, l + 64, ...); a system
    // with a skipped step is left to k_ge_solve
    int pv[4];
    bool sk = false;
#pragma unroll
    for (int s = 0; s < 4; s++) {
        const int i = lane + 64 * s;
        pv[s] = i < n ? perm_in[(long long)sysl * g.tc_max + i] : 0;
        sk = sk || (i < n && skip_in[(long long)sysl * g.tc_max + i] != 0);
    }
    if (__ballot(sk) != 0ull) return;
    float R[SB_RG][SB_G];
#pragma unroll
    for (int m = 0; m < SB_RG; m++)
#pragma unroll
        for (int j = 0; j < SB_G; j++) R[m][j] = 0.0f;
    float pf = 0.0f;   // sink of the cache warm-up loads
    sb_forward(R, zl, LU, B, pv, n, p, vc, lane, pf);
    // forward layout: block m = group SB_RG - 1 - m, LDS slot s = group
    // SB_RG + s; backward layout: block m = group SB_LG + m, LDS slot s =
    // group s
    {
        // one group at a time (a group's LDS slot is read before the
        // register group that replaces it is stored), so that no more than
        // one group is in flight beside the stack
        float Q[SB_RG][SB_G];
#pragma unroll
        for (int s = 0; s < SB_LG; s++) {
            float t[SB_G];
#pragma unroll
            for (int j = 0; j < SB_G; j++) t[j] = zl[SB_G * s + j][lane];
#pragma unroll
            for (int j = 0; j < SB_G; j++) zl[SB_G * s + j][lane] = R[SB_RG - 1 - s][j];
#pragma unroll
            for (int j = 0; j < SB_G; j++) Q[SB_RG - SB_LG + s][j] = t[j];
            __builtin_amdgcn_sched_barrier(0);
        }
#pragma unroll
        for (int m = 0; m < SB_RG - SB_LG; m++)
#pragma unroll
            for (int j = 0; j < SB_G; j++) Q[m][j] = R[SB_RG - SB_LG - 1 - m][j];
#pragma unroll
        for (int m = 0; m < SB_RG; m++)
#pragma unroll
            for (int j = 0; j < SB_G; j++) R[m][j] = Q[m][j];
    }
    sb_backward(R, zl, LU, pv, n, g.zero_val, lane);
    zl[SB_LDS][lane] = pf;
    // block m = x group m, LDS slot s = x group 24 + s
    if (act) {
#pragma unroll
        for (int m = 0; m < SB_RG; m++)
#pragma unroll
            for (int j = 0; j < SB_G; j++)
                if (SB_G * m + j < n) x[(unsigned)((SB_G * m + j) * g.dv + v)] = R[m][j];
        for (int r = SB_G * SB_RG; r < n; r++) x[(unsigned)(r * g.dv + v)] = zl[r - SB_G * SB_RG][lane];
    }
}

// general size: physical row swaps in global memory, column-major storage
__device__ void ge_solve_block(float * __restrict__ a, int n, int p, float * __restrict__ x,
                               long long ldx, float zero_val, float * prow, float * fac) {
    const int w = n + p;
    __shared__ float bv[16];
    __shared__ int bi[16];
    __shared__ int s_mr;
    for (int col = 0; col < n; col++) {
        float best = -1.0f;
        int brow = 0x7fffffff;
        const float a0 = fabsf(a[(long long)col * n + col]);
        for (int r = col + 1 + threadIdx.x; r < n; r += blockDim.x) {
            const float v = fabsf(a[(long long)col * n + r]);
            if (v == v && v > best) { best = v; brow = r; }
        }
        for (int o = 32; o > 0; o >>= 1) {
            const float ov = __shfl_xor(best, o);
            const int orow = __shfl_xor(brow, o);
            if (ov > best || (ov == best && orow < brow)) { best = ov; brow = orow; }
        }
        if ((threadIdx.x & 63) == 0) { bv[threadIdx.x >> 6] = best; bi[threadIdx.x >> 6] = brow; }
        __syncthreads();
        if (threadIdx.x == 0) {
            float b = bv[0];
            int r = bi[0];
            for (int i = 1; i < (int)(blockDim.x >> 6); i++)
                if (bv[i] > b || (bv[i] == b && bi[i] < r)) { b = bv[i]; r = bi[i]; }
            s_mr = (a0 == a0 && b > a0) ? r : col;
        }
        __syncthreads();
        const int mr = s_mr;
        if (mr != col) {
            for (int j = threadIdx.x; j < w; j += blockDim.x) {
                const float t0 = a[(long long)j * n + col];
                a[(long long)j * n + col] = a[(long long)j * n + mr];
                a[(long long)j * n + mr] = t0;
            }
        }
        __syncthreads();
        const float piv = a[(long long)col * n + col];
        if (fabsf(piv) < 1e-12f) continue;
        for (int j = col + threadIdx.x; j < w; j += blockDim.x) prow[j - col] = a[(long long)j * n + col];
        for (int r = col + 1 + threadIdx.x; r < n; r += blockDim.x) fac[r - col - 1] = a[(long long)col * n + r] / piv;
        __syncthreads();
        const int rows = n - col - 1, cols = w - col;
        const long long tot = (long long)rows * cols;
        for (long long e = threadIdx.x; e < tot; e += blockDim.x) {
            const int jj = (int)(e / rows), rr = (int)(e % rows);
            float * ap = a + (long long)(col + jj) * n + col + 1 + rr;
            *ap = *ap - fac[rr] * prow[jj];
        }
        __syncthreads();
    }
    for (int col = n - 1; col >= 0; col--) {
        const float piv = a[(long long)col * n + col];
        if (fabsf(piv) < 1e-12f) {
            for (int j = threadIdx.x; j < p; j += blockDim.x) x[(long long)col * ldx + j] = zero_val;
        } else {
            for (int j = threadIdx.x; j < p; j += blockDim.x) {
                float v = a[(long long)(n + j) * n + col];
                for (int r = col + 1; r < n; r++) v -= a[(long long)r * n + col] * x[(long long)r * ldx + j];
                x[(long long)col * ldx + j] = v / piv;
            }
        }
        __syncthreads();
    }
}

constexpr int GE_LDS_FLOATS = 8192;

// The same elimination in panels of pb steps (systems with n > 256): each
// element of [M | B] receives the same sequence of row swaps and updates
// a -= f * u, in step order, as in ge_solve_block, but the trailing columns
// are read and written once per panel instead of once per step.
//  1. Panel: columns c0 .. c0 + pb - 1, rows c0 .. n - 1, in LDS (P, one
//     column of nr = n - c0 rows each). Per step c: the pivot search over
//     column c (rows > c; the largest |a| that is not NaN, the first such row
//     on ties, taken only when it exceeds |a[c][c]| and that is not NaN), the
//     swap of rows c and mr in the panel, and, unless |pivot| < 1e-12 (a
//     skipped step), the multipliers F[s][r] = a[r][c] / pivot (rows r > c)
//     and their update of the panel's later columns. The panel's rows c0 ..
//     c0 + pb - 1 are final and go back to memory (the rows below the
//     diagonal are never read again).
//  2. Trailing columns c0 + pb .. w - 1 (the rest of M, then B), each by 16
//     lanes of one wave in an LDS column of its own: each panel step applied
//     in order, the row swap and then, unless skipped, a[r][j] -= F[s][r] *
//     a[c][j] for the rows r > c.
// Then the back substitution of ge_solve_block. Dynamic LDS: 3 pb nr floats
// (P, F and min(pb, blockDim.x / 16) trailing columns).
// Order this wave's LDS accesses around the call in program order (the
// hardware completes one wave's LDS operations in order; this keeps the
// compiler from moving them across).
__device__ __forceinline__ void lds_wave_order() {
    __builtin_amdgcn_wave_barrier();
    asm volatile("" ::: "memory");
}

__device__ void ge_solve_blocked(float * __restrict__ a, int n, int p, float * __restrict__ x, long long ldx,
                                 float zero_val, float * __restrict__ lds, int pb) {
    const int w = n + p, nt = blockDim.x, tid = threadIdx.x;
    __shared__ float bv[32];
    __shared__ int bi[32];
    __shared__ int s_mr[32];
    __shared__ unsigned char s_skip[32];
    for (int c0 = 0; c0 < n; c0 += pb) {
        const int np = min(pb, n - c0), nr = n - c0;
        float * P = lds;                    // P[jj * nr + (r - c0)]
        float * F = lds + pb * nr;          // F[s * nr + (r - c0)]
        float * Tt = lds + 2 * pb * nr;     // trailing tile, same layout as P
        __syncthreads();
        for (int e = tid; e < np * nr; e += nt) {
            const int jj = e / nr, rr = e - jj * nr;
            P[e] = a[(long long)(c0 + jj) * n + c0 + rr];
        }
        __syncthreads();
        for (int s = 0; s < np; s++) {
            const int c = c0 + s;
            const float * Pc = P + s * nr;
            // pivot search (as in ge_solve_block)
            float best = -1.0f;
            int brow = 0x7fffffff;
            for (int r = c + 1 + tid; r < n; r += nt) {
                const float v = fabsf(Pc[r - c0]);
                if (v == v && v > best) { best = v; brow = r; }
            }
            for (int o = 32; o > 0; o >>= 1) {
                const float ov = __shfl_xor(best, o);
                const int orow = __shfl_xor(brow, o);
                if (ov > best || (ov == best && orow < brow)) { best = ov; brow = orow; }
            }
            if ((tid & 63) == 0) { bv[tid >> 6] = best; bi[tid >> 6] = brow; }
            __syncthreads();
            if (tid == 0) {
                float b = bv[0];
                int r = bi[0];
                for (int i = 1; i < (nt >> 6); i++)
                    if (bv[i] > b || (bv[i] == b && bi[i] < r)) { b = bv[i]; r = bi[i]; }
                const float a0 = fabsf(Pc[s]);
                s_mr[s] = (a0 == a0 && b > a0) ? r : c;
            }
            __syncthreads();
            const int mr = s_mr[s];
            if (mr != c) {
                for (int jj = tid; jj < np; jj += nt) {
                    float * col = P + jj * nr;
                    const float t0 = col[s];
                    col[s] = col[mr - c0];
                    col[mr - c0] = t0;
                }
            }
            __syncthreads();
            const float piv = Pc[s];
            const bool skip = fabsf(piv) < 1e-12f;
            if (tid == 0) s_skip[s] = skip ? 1 : 0;
            if (!skip) {
                for (int r = c + 1 + tid; r < n; r += nt) F[s * nr + (r - c0)] = Pc[r - c0] / piv;
                __syncthreads();
                // 16 lanes per column, rows strided by 16
                for (int jj = s + 1 + (tid >> 4); jj < np; jj += nt >> 4) {
                    float * col = P + jj * nr;
                    const float u = col[s];
                    for (int rr = c + 1 - c0 + (tid & 15); rr < nr; rr += 16) col[rr] = col[rr] - F[s * nr + rr] * u;
                }
            }
            __syncthreads();
        }
        // the panel's rows c0 .. c0 + np - 1 are final: U in place on and
        // above the diagonal, and each U row also transposed below it (the
        // multipliers there are dead), so that row i's entries right of the
        // diagonal lie contiguously at a[i n + i + 1 ..]
        for (int e = tid; e < np * np; e += nt) {
            const int jj = e / np, rr = e - jj * np;
            a[(long long)(c0 + jj) * n + c0 + rr] = rr <= jj ? P[jj * nr + rr] : P[rr * nr + jj];
        }
        // trailing columns: each column by the 16 lanes of one column group
        // (rows strided by 16) in its own LDS column; the lanes of a group
        // are in one wave, whose LDS accesses complete in program order, so
        // the panel's steps need no block barrier here
        {
            const int cg = tid >> 4, cr = tid & 15, ngr = min(nt >> 4, pb);
            float * col = Tt + cg * nr;
            for (int j = c0 + np + cg; cg < ngr && j < w; j += ngr) {
                float * aj = a + (long long)j * n + c0;
                for (int rr = cr; rr < nr; rr += 16) col[rr] = aj[rr];
                lds_wave_order();
                for (int s = 0; s < np; s++) {
                    const int c = c0 + s, mr = s_mr[s];
                    if (mr != c) {
                        if (cr == 0) {
                            const float t0 = col[s];
                            col[s] = col[mr - c0];
                            col[mr - c0] = t0;
                        }
                        lds_wave_order();
                    }
                    if (!s_skip[s]) {
                        const float u = col[s];
                        const float * Fs = F + s * nr;
                        for (int rr = c + 1 - c0 + cr; rr < nr; rr += 16) col[rr] = col[rr] - Fs[rr] * u;
                        lds_wave_order();
                    }
                }
                for (int rr = cr; rr < nr; rr += 16) aj[rr] = col[rr];
                if (j < n)   // U rows c0 .. c0 + np - 1, transposed below the diagonal
                    for (int rr = cr; rr < np; rr += 16) a[(long long)(c0 + rr) * n + j] = col[rr];
                lds_wave_order();
            }
        }
        __syncthreads();
    }
    // back substitution (the order of ge_solve_block's) from LDS, in passes
    // of pc right-hand-side columns: the pass's y, then x in place, at
    // xl[r (pc + 1) + j]; U row col (contiguous at a[col n + col ..]) in one
    // of two LDS rows, the next row loaded by the whole block while this one
    // is solved
    const int pc_max = min(3 * pb - 3, nt);   // n (pc + 1) + 2 n <= 3 pb n
    if (pc_max >= 1) {
        const int passes = (p + pc_max - 1) / pc_max, pc = (p + passes - 1) / passes, ldl = pc + 1;
        float * ub = lds;
        float * xl = lds + 2 * n;
        constexpr int PF = 4;
        for (int j0 = 0; j0 < p; j0 += pc) {
            const int nc = min(pc, p - j0);
            __syncthreads();
            for (int e = tid; e < nc * n; e += nt) {
                const int j = e / n, r = e - j * n;
                xl[r * ldl + j] = a[(long long)(n + j0 + j) * n + r];
            }
            if (tid == 0) ub[((n - 1) & 1) * n + n - 1] = a[(long long)(n - 1) * n + n - 1];
            __syncthreads();
            for (int col = n - 1; col >= 0; col--) {
                // row col - 1 (entries col - 1 .. n - 1) toward the other buffer
                const int nld = col > 0 ? n - col + 1 : 0;
                const float * src = a + (long long)(col - 1) * n + (col - 1);
                float * dst = ub + ((col - 1) & 1) * n + (col - 1);
                const bool pf = nld <= PF * nt;
                float pre[PF];
#pragma unroll
                for (int k = 0; k < PF; k++) pre[k] = (pf && tid + k * nt < nld) ? src[tid + k * nt] : 0.0f;
                if (tid < nc) {
                    const float * u = ub + (col & 1) * n;
                    const float piv = u[col];
                    float v = zero_val;
                    if (!(fabsf(piv) < 1e-12f)) {
                        v = xl[col * ldl + tid];
                        // terms in order, eight at a time, the next eight's
                        // reads issued before this eight's arithmetic
                        int r = col + 1;
                        if (r + 8 <= n) {
                            float uc[8], xc[8];
#pragma unroll
                            for (int k = 0; k < 8; k++) { uc[k] = u[r + k]; xc[k] = xl[(r + k) * ldl + tid]; }
                            for (; r + 16 <= n; r += 8) {
                                float un[8], xn[8];
#pragma unroll
                                for (int k = 0; k < 8; k++) { un[k] = u[r + 8 + k]; xn[k] = xl[(r + 8 + k) * ldl + tid]; }
#pragma unroll
                                for (int k = 0; k < 8; k++) v -= uc[k] * xc[k];
#pragma unroll
                                for (int k = 0; k < 8; k++) { uc[k] = un[k]; xc[k] = xn[k]; }
                            }
#pragma unroll
                            for (int k = 0; k < 8; k++) v -= uc[k] * xc[k];
                            r += 8;
                        }
                        for (; r < n; r++) v -= u[r] * xl[r * ldl + tid];
                        v = v / piv;
                    }
                    xl[col * ldl + tid] = v;
                }
                if (pf) {
#pragma unroll
                    for (int k = 0; k < PF; k++)
                        if (tid + k * nt < nld) dst[tid + k * nt] = pre[k];
                } else {
                    for (int i = tid; i < nld; i += nt) dst[i] = src[i];
                }
                __syncthreads();
            }
            for (int e = tid; e < n * nc; e += nt) {
                const int r = e / nc, j = e - r * nc;
                x[(long long)r * ldx + j0 + j] = xl[r * ldl + j];
            }
        }
        return;
    }
    __syncthreads();
    for (int col = n - 1; col >= 0; col--) {
        const float piv = a[(long long)col * n + col];
        if (fabsf(piv) < 1e-12f) {
            for (int j = tid; j < p; j += nt) x[(long long)col * ldx + j] = zero_val;
        } else {
            for (int j = tid; j < p; j += nt) {
                float v = a[(long long)(n + j) * n + col];
                // U row col, transposed below the diagonal
                for (int r = col + 1; r < n; r++) v -= a[(long long)col * n + r] * x[(long long)r * ldx + j];
                x[(long long)col * ldx + j] = v / piv;
            }
        }
        __syncthreads();
    }
}

// panel width for n rows in GE_BLK_LDS floats (3 pb n), or 0: too large
constexpr int GE_BLK_LDS = 40960 - 256;
__host__ __device__ inline int ge_panel(int n) { return std::min(32, GE_BLK_LDS / (3 * n)); }

__global__ void __launch_bounds__(512)
k_ge_general(Geom g, const ChunkDesc * __restrict__ chunks, float * __restrict__ aug,
             const long long * __restrict__ aug_off, float * __restrict__ Cv, float * __restrict__ gtmp) {
    const int c_idx = blockIdx.x / g.H, h = blockIdx.x % g.H, layer = blockIdx.y;
    const ChunkDesc c = chunks[c_idx];
    if (c.tc <= RG_ROWS) return;
    const long long sys = ((long long)layer * g.n_chunks + c_idx) * g.H + h;
    float * Ag = aug + aug_off[sys];
    float * x = Cv + (((long long)layer * g.H + h) * g.t_total + c.off) * g.dv;
    extern __shared__ __align__(16) float ge_dyn[];
    const int n = c.tc, w = n + g.dv;
    // the panel width the launch sized the LDS for (3 pb tc_max floats): a
    // smaller chunk's own width could need more than that
    const int pb = ge_panel(g.tc_max);
    if (pb >= 1) {
        ge_solve_blocked(Ag, n, g.dv, x, g.dv, g.zero_val, ge_dyn, pb);
        return;
    }
    // (rows beyond the panel budget: step by step, the factors in LDS or in gtmp)
    float * prow;
    float * fac;
    if (w + n <= GE_LDS_FLOATS) {
        prow = ge_dyn;
        fac = ge_dyn + w;
    } else {
        prow = gtmp + sys * (long long)(2 * g.tc_max + g.dv);
        fac = prow + g.tc_max + g.dv;
    }
    ge_solve_block(Ag, n, g.dv, x, g.dv, g.zero_val, prow, fac);
}

// ---------------------------------------------------------------------------
// Projected-gradient NNLS (math.h:752-805), after the clamped least-squares
// solution: w < eps -> eps; then, for iters > 0, three power-iteration steps
// on M from u = 1 / sqrtf(n) (each stopped when a norm falls below 1e-12f),
// L = u^T (M^T M) u clamped to 1e-6f, eta = 1 / L, and iters steps
// w <- max(eps, w - eta (M^T M w - M^T b)). Every sum runs in index order
// (one thread per output, or thread 0 for the norms and L). One block; the
// vectors u (n), v (m) and grad (n) are the caller's scratch.
// ---------------------------------------------------------------------------
struct MatRows {    // M(i, j) = p[i * rs + j]
    const float * p;
    long long rs;
    __device__ __forceinline__ float operator()(int i, int j) const { return p[(long long)i * rs + j]; }
};
struct MatPicked {  // M(i, j) = p[i * rs + col[j]]
    const float * p;
    long long rs;
    const int * col;
    __device__ __forceinline__ float operator()(int i, int j) const { return p[(long long)i * rs + col[j]]; }
};

// AtA(i, j) at AtA[j * lda + i] (symmetric); w, u, v, grad visible to the block
template <class Mat>
__device__ void pgd_block(const Mat & M, int m, int n, const float * AtA, long long lda, const float * Atb,
                          float * w, float eps, int iters, float * u, float * v, float * grad) {
    __shared__ float s_val;
    const int tid = threadIdx.x, nt = blockDim.x;
    for (int i = tid; i < n; i += nt) {
        const float x = w[i];
        w[i] = (x < eps) ? eps : x;
    }
    __syncthreads();
    if (iters <= 0) return;
    const float u0 = 1.0f / sqrtf((float)n);
    for (int j = tid; j < n; j += nt) u[j] = u0;
    __syncthreads();
    for (int pw = 0; pw < 3; pw++) {
        for (int i = tid; i < m; i += nt) {
            float acc = 0.0f;
            for (int j = 0; j < n; j++) acc += M(i, j) * u[j];
            v[i] = acc;
        }
        __syncthreads();
        if (tid == 0) {
            float s = 0.0f;
            for (int i = 0; i < m; i++) s += v[i] * v[i];
            s_val = sqrtf(s);
        }
        __syncthreads();
        const float vn = s_val;
        if (vn < 1e-12f) break;
        for (int i = tid; i < m; i += nt) v[i] = v[i] / vn;
        __syncthreads();
        for (int j = tid; j < n; j += nt) {
            float acc = 0.0f;
            for (int i = 0; i < m; i++) acc += M(i, j) * v[i];
            u[j] = acc;
        }
        __syncthreads();
        if (tid == 0) {
            float s = 0.0f;
            for (int j = 0; j < n; j++) s += u[j] * u[j];
            s_val = sqrtf(s);
        }
        __syncthreads();
        const float un = s_val;
        if (un < 1e-12f) break;
        for (int j = tid; j < n; j += nt) u[j] = u[j] / un;
        __syncthreads();
    }
    for (int i = tid; i < n; i += nt) {
        float acc = 0.0f;
        for (int j = 0; j < n; j++) acc += AtA[(long long)j * lda + i] * u[j];
        grad[i] = acc;
    }
    __syncthreads();
    if (tid == 0) {
        float L = 0.0f;
        for (int i = 0; i < n; i++) L += u[i] * grad[i];
        if (L < 1e-6f) L = 1e-6f;
        s_val = 1.0f / L;
    }
    __syncthreads();
    const float eta = s_val;
    for (int it = 0; it < iters; it++) {
        for (int i = tid; i < n; i += nt) {
            float acc = 0.0f;
            for (int j = 0; j < n; j++) acc += AtA[(long long)j * lda + i] * w[j];
            grad[i] = acc - Atb[i];
        }
        __syncthreads();
        for (int i = tid; i < n; i += nt) {
            const float x = w[i] - eta * grad[i];
            w[i] = (x < eps) ? eps : x;
        }
        __syncthreads();
    }
}

// The beta fit's PGD steps (api.cpp:826 with nnls_pgd_iters > 0): per
// (layer, chunk, head), M = the gathered exp scores in X, [AtA | Atb] in aug
// (k_ls_build without ridge), w = the clamped LS solution in wb, refined in
// place. Dynamic LDS: w, u, grad (tc_max each), v (nq_max).
// grid = (n_chunks * H, L), 256 threads
__global__ void __launch_bounds__(256)
k_nnls_pgd(Geom g, const ChunkDesc * __restrict__ chunks, const float * __restrict__ X,
           const float * __restrict__ aug, const long long * __restrict__ aug_off, float * __restrict__ wb,
           int iters) {
    const int c_idx = blockIdx.x / g.H, h = blockIdx.x % g.H, layer = blockIdx.y;
    const ChunkDesc c = chunks[c_idx];
    const int n = c.tc, m = c.nq;
    const long long sys = ((long long)layer * g.n_chunks + c_idx) * g.H + h;
    const float * Ag = aug + aug_off[sys];
    const long long hsX = (long long)g.nq_max * g.t_total;
    const float * Xh = X + (long long)layer * g.H * hsX + h * hsX + c.off;
    float * wg = wb + ((long long)layer * g.H + h) * g.t_total + c.off;
    extern __shared__ float pv[];
    float * w = pv;
    float * u = pv + g.tc_max;
    float * grad = pv + 2 * g.tc_max;
    float * v = pv + 3 * g.tc_max;
    for (int i = threadIdx.x; i < n; i += blockDim.x) w[i] = wg[i];
    __syncthreads();
    pgd_block(MatRows{Xh, g.t_total}, m, n, Ag, n, Ag + (long long)n * n, w, 1e-12f, iters, u, v, grad);
    for (int i = threadIdx.x; i < n; i += blockDim.x) wg[i] = w[i];
}

// ---------------------------------------------------------------------------
// OMP key selection (math.h:832-950; api.cpp:690-711) of one (layer, chunk)
// on the exp scores and row sums summed over heads (in head order from 0):
// while fewer than t keys are picked, the residual r = b - cur, the
// correlations corr_j = sum_i E[i][j] r_i of the unpicked keys, then up to
// k_choice picks of the largest correlation (first index on ties; it must
// beat -1e30f). On refit iterations (every refit_interval-th, and the last)
// the NNLS of the picked columns in pick order (ridge 1e-10f, GE with partial
// pivoting, skipped pivots and the clamp at 1e-12f, then the PGD steps) gives
// the weights and cur = M w; between refits the new picks weigh 1e-12f. The
// Gram matrix grows by the new columns only (every entry is its own sum over
// the queries, the same whenever it is formed). Output: the picks ascending
// (fewer than t picks are padded with the chunk's first position). An
// iteration without a pick (every correlation NaN) sets status bit 4 and
// stops, where the reference would not return.
// grid = (n_chunks, L), 256 threads
// ---------------------------------------------------------------------------
__global__ void __launch_bounds__(256)
k_omp_select(Geom g, const ChunkDesc * __restrict__ chunks, const float * __restrict__ E,
             const float * __restrict__ rowsum, OmpWork ow, int * __restrict__ sel, int * __restrict__ status) {
    const int c_idx = blockIdx.x, layer = blockIdx.y;
    const ChunkDesc c = chunks[c_idx];
    const int T = c.Tc, nq = c.nq, t = c.tc, tid = threadIdx.x, nt = blockDim.x;
    const long long unit = (long long)layer * g.n_chunks + c_idx;
    const long long tm = g.tc_max;
    float * ce = ow.ce + (long long)layer * g.nq_max * g.T + c.start;   // row k at k * g.T
    float * corr = ow.corr + (long long)layer * g.T + c.start;
    unsigned char * mask = ow.mask + (long long)layer * g.T + c.start;
    int * order = ow.order + (long long)layer * g.t_total + c.off;
    float * w = ow.w + (long long)layer * g.t_total + c.off;
    float * prev_w = ow.prev_w + (long long)layer * g.t_total + c.off;
    float * G = ow.G + unit * tm * tm;            // column j at G + j * t
    float * Atb = ow.Atb + unit * tm;
    float * aug = ow.aug + unit * tm * (tm + 1);
    float * u = ow.vec + unit * (4 * tm + 1 + g.nq_max);
    float * grad = u + tm;
    float * v = grad + tm;
    float * prow = v + g.nq_max;
    float * fac = prow + tm + 1;
    __shared__ float cs[OMP_MAXQ], res[OMP_MAXQ], cur[OMP_MAXQ];
    __shared__ float rv[4];
    __shared__ int ri[4];
    __shared__ int s_best;
    for (long long e = tid; e < (long long)nq * T; e += nt) {
        const int k = (int)(e / T), j = (int)(e % T);
        float s = 0.0f;
        for (int h = 0; h < g.H; h++) s += E[layer * lS(g) + h * hS(g) + (long long)k * g.T + c.start + j];
        ce[(long long)k * g.T + j] = s;
    }
    for (int k = tid; k < nq; k += nt) {
        float s = 0.0f;
        for (int h = 0; h < g.H; h++) s += rowsum[(unit * g.H + h) * g.nq_max + k];
        cs[k] = s;
        cur[k] = 0.0f;
    }
    for (int j = tid; j < T; j += nt) mask[j] = 0;
    __syncthreads();
    const MatPicked M{ce, g.T, order};
    int ns = 0, n_prev = 0, ng = 0, iteration = 0;
    while (ns < t) {
        for (int i = tid; i < nq; i += nt) res[i] = cs[i] - cur[i];
        __syncthreads();
        for (int j = tid; j < T; j += nt) {
            float cc = 0.0f;
            if (!mask[j])
                for (int i = 0; i < nq; i++) cc += ce[(long long)i * g.T + j] * res[i];
            corr[j] = cc;
        }
        __syncthreads();
        int k_sel = min(ow.k_choice, t - ns);
        k_sel = min(k_sel, T - ns);
        if (k_sel <= 0) break;
        const int ns0 = ns;
        for (int k = 0; k < k_sel; k++) {
            float bv = -1e30f;
            int bi = -1;
            for (int j = tid; j < T; j += nt)
                if (!mask[j]) {
                    const float x = corr[j];
                    if (x > bv) { bv = x; bi = j; }
                }
            // largest value, then smallest index (-1, no candidate, ranks last)
            for (int o = 32; o > 0; o >>= 1) {
                const float ov = __shfl_xor(bv, o);
                const int oi = __shfl_xor(bi, o);
                if (ov > bv || (ov == bv && (unsigned)oi < (unsigned)bi)) { bv = ov; bi = oi; }
            }
            if ((tid & 63) == 0) { rv[tid >> 6] = bv; ri[tid >> 6] = bi; }
            __syncthreads();
            if (tid == 0) {
                float b = rv[0];
                int r = ri[0];
                for (int q = 1; q < (nt >> 6); q++)
                    if (rv[q] > b || (rv[q] == b && (unsigned)ri[q] < (unsigned)r)) { b = rv[q]; r = ri[q]; }
                s_best = r;
                if (r >= 0) {
                    order[ns] = r;
                    mask[r] = 1;
                }
            }
            __syncthreads();
            if (s_best < 0) break;
            ns++;
        }
        if (ns == ns0) {
            if (tid == 0) atomicOr(status, 4);
            return;
        }
        const int ct = ns;
        const bool solve = ow.refit_interval <= 1 || iteration % ow.refit_interval == 0 || ct == t;
        if (solve) {
            // Gram entries (i, jn) of the new columns jn, i <= jn, mirrored
            for (long long e = tid; e < (long long)(ct - ng) * ct; e += nt) {
                const int jn = ng + (int)(e / ct), i = (int)(e % ct);
                if (i > jn) continue;
                const int ci = order[i], cj = order[jn];
                float s = 0.0f;
                for (int k = 0; k < nq; k++) s += ce[(long long)k * g.T + ci] * ce[(long long)k * g.T + cj];
                G[(long long)jn * t + i] = s;
                G[(long long)i * t + jn] = s;
            }
            for (int jn = ng + tid; jn < ct; jn += nt) {
                const int cj = order[jn];
                float s = 0.0f;
                for (int k = 0; k < nq; k++) s += ce[(long long)k * g.T + cj] * cs[k];
                Atb[jn] = s;
            }
            ng = ct;
            __syncthreads();
            // [G + 1e-10 I | A^T b], column-major ct x (ct + 1)
            for (long long e = tid; e < (long long)ct * ct; e += nt) {
                const int j = (int)(e / ct), i = (int)(e % ct);
                float a = G[(long long)j * t + i];
                if (i == j) a += 1e-10f;
                aug[e] = a;
            }
            for (int i = tid; i < ct; i += nt) aug[(long long)ct * ct + i] = Atb[i];
            __syncthreads();
            ge_solve_block(aug, ct, 1, w, 1, 1e-12f, prow, fac);
            pgd_block(M, nq, ct, G, t, Atb, w, 1e-12f, ow.pgd_iters, u, v, grad);
            for (int j = tid; j < ct; j += nt) prev_w[j] = w[j];
            n_prev = ct;
            for (int i = tid; i < nq; i += nt) {
                float acc = 0.0f;
                for (int j = 0; j < ct; j++) acc += M(i, j) * w[j];
                cur[i] = acc;
            }
        } else {
            for (int j = n_prev + tid; j < ct; j += nt) prev_w[j] = 1e-12f;
            n_prev = ct;
            __syncthreads();
            for (int i = tid; i < nq; i += nt) {
                float acc = 0.0f;
                for (int j = 0; j < ct; j++) acc += M(i, j) * prev_w[j];
                cur[i] = acc;
            }
        }
        __syncthreads();
        iteration++;
    }
    // ascending (the picks are distinct: rank = number of smaller picks)
    int * out = sel + (long long)layer * g.t_total + c.off;
    for (int j = tid; j < ns; j += nt) {
        const int x = order[j];
        int r = 0;
        for (int k = 0; k < ns; k++) r += order[k] < x ? 1 : 0;
        out[r] = c.start + x;
    }
    for (int j = ns + tid; j < t; j += nt) out[j] = c.start;
}

// ---------------------------------------------------------------------------
// Quality statistics (api.cpp:239-325).
// ---------------------------------------------------------------------------
// In-place row softmax (math.h:83-100) of the statistics rows: row r of a
// layer is (h = r / mq, q = r % mq) at x + layer * ls + h * hs + q * rs. A
// block owns ROWS rows and sweeps them together, one column per thread,
// so that every row's load of a column is in flight at once:
//  1. maxima: the largest non-NaN value of each row (NaN when row[0] is NaN;
//     the reference's scan keeps row[0] otherwise unless a value exceeds it),
//     from the scoring tiles' maxima when the rows are the main scores (ms.tm),
//     else over the row;
//  2. RSM_TILE-column tiles, double-buffered in LDS: threads 64.. compute
//     expf(x - max) (written back in place) while lane r of wave 0 adds row
//     r's previous tile in column order, the reference's sequential sum;
//  3. inv = 1 / (sum + 1e-12f): to inv_out[layer][r] when given (the rows stay
//     unnormalised and their reader forms x * inv, the same product), else
//     x *= inv in place.
// grid (ceil(mh * mq / ROWS), L), RSM_THREADS threads. ROWS = RSM_ROWS, or
// RSM_ROWS_FEW when that grid would leave most CUs idle (one layer): each
// row's sequential sum then shares its block with fewer rows. RSM_ROWS_FEW
// also for the original-attention rows beside the factorizations: at 32
// VGPRs its blocks share CUs with k_ge_lu blocks, where the 70 of RSM_ROWS
// would keep them off the CUs they hold.
constexpr int RSM_ROWS = 16, RSM_ROWS_FEW = 4, RSM_TILE = 256, RSM_THREADS = 64 + RSM_TILE;

// tile maxima of the main scores (k_scores' tmax), for rows that are rows of S:
// row (h, q) of a layer at tm + layer * ls + h * hs + q * rs, chunk c's tiles
// from c * nt on, ceil(chunks[c].Tc / SC_KEYS) of them
struct RowMaxSrc {
    const unsigned * tm;
    const ChunkDesc * chunks;
    int nc, nt;
    long long ls, hs, rs;
};

template <int ROWS>
__global__ void __launch_bounds__(RSM_THREADS)
k_row_softmax(float * __restrict__ x, int n, long long ls, long long hs, long long rs, int mh, int mq,
              RowMaxSrc ms, float * __restrict__ inv_out) {
    const int layer = blockIdx.y, r0 = blockIdx.x * ROWS;
    const int nrows = min(ROWS, mh * mq - r0);
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    __shared__ float mx[ROWS], inv[ROWS];
    __shared__ float tile[2][ROWS][RSM_TILE + 1];
    __shared__ unsigned red[RSM_THREADS / 64][ROWS];
    __shared__ uint64_t etab[32];
    if (tid < 32) etab[tid] = c_exp2_tab[tid];   // visible after the barriers below
    float * rowp[ROWS];
#pragma unroll
    for (int r = 0; r < ROWS; r++) {
        const int rr = r0 + min(r, nrows - 1);
        rowp[r] = x + layer * ls + (long long)(rr / mq) * hs + (long long)(rr % mq) * rs;
    }
    // 1. maxima
    if (ms.tm) {
        if (tid < nrows) {
            const int rr = r0 + tid;
            const unsigned * p = ms.tm + layer * ms.ls + (long long)(rr / mq) * ms.hs + (long long)(rr % mq) * ms.rs;
            unsigned k = 0;
            for (int c = 0; c < ms.nc; c++) {
                const int ntc = (ms.chunks[c].Tc + SC_KEYS - 1) / SC_KEYS;
                for (int t = 0; t < ntc; t++) k = max(k, p[(long long)c * ms.nt + t]);
            }
            const float mm = __uint_as_float((k & 0x80000000u) ? (k & 0x7fffffffu) : ~k);
            const float a0 = rowp[tid][0];
            mx[tid] = (a0 != a0) ? a0 : ((mm > a0) ? mm : a0);
        }
        __syncthreads();
    } else {
        float m[ROWS];
#pragma unroll
        for (int r = 0; r < ROWS; r++) m[r] = -INFINITY;
        for (int j = tid; j < n; j += RSM_THREADS) {
            float v[ROWS];
#pragma unroll
            for (int r = 0; r < ROWS; r++) v[r] = rowp[r][j];
#pragma unroll
            for (int r = 0; r < ROWS; r++)
                if (v[r] == v[r] && v[r] > m[r]) m[r] = v[r];
        }
#pragma unroll
        for (int r = 0; r < ROWS; r++) {
            const unsigned k = dpp_reduce_u32<true>(score_key(m[r]));
            if (lane == 0) red[w][r] = k;
        }
        __syncthreads();
        if (tid < nrows) {
            unsigned k = red[0][tid];
            for (int i = 1; i < RSM_THREADS / 64; i++) k = max(k, red[i][tid]);
            const float mm = __uint_as_float((k & 0x80000000u) ? (k & 0x7fffffffu) : ~k);
            const float a0 = rowp[tid][0];
            mx[tid] = (a0 != a0) ? a0 : ((mm > a0) ? mm : a0);
        }
        __syncthreads();
    }
    // 2. exponentials and the sequential sums
    const int ntiles = (n + RSM_TILE - 1) / RSM_TILE;
    auto compute = [&](int t, int b) {   // threads 64 .. 64 + RSM_TILE - 1
        const int c = tid - 64, j = t * RSM_TILE + c;
        if (j >= n) return;
        float v[ROWS];
#pragma unroll
        for (int r = 0; r < ROWS; r++) v[r] = rowp[r][j];
#pragma unroll
        for (int r = 0; r < ROWS; r++) {
            if (r < nrows) {
                const float e = expf_ref(v[r] - mx[r], etab);
                rowp[r][j] = e;
                tile[b][r][c] = e;
            }
        }
    };
    float sum = 0.0f;
    if (w > 0) compute(0, 0);
    __syncthreads();
    for (int t = 0; t < ntiles; t++) {
        const int b = t & 1;
        if (w > 0) {
            if (t + 1 < ntiles) compute(t + 1, b ^ 1);
        } else if (lane < nrows) {
            const int jn = min(RSM_TILE, n - t * RSM_TILE);
            const float * tr = &tile[b][lane][0];
            int c = 0;
            for (; c + 16 <= jn; c += 16) {   // 16 reads in flight, then the adds in order
                float e[16];
#pragma unroll
                for (int k = 0; k < 16; k++) e[k] = tr[c + k];
#pragma unroll
                for (int k = 0; k < 16; k++) sum += e[k];
            }
            for (; c < jn; c++) sum += tr[c];
        }
        __syncthreads();
    }
    if (w == 0 && lane < nrows) {
        const float iv = 1.0f / (sum + 1e-12f);
        inv[lane] = iv;
        if (inv_out) inv_out[(long long)layer * mh * mq + r0 + lane] = iv;
    }
    if (inv_out) return;
    __syncthreads();
    // 3. normalisation
    float iv[ROWS];
#pragma unroll
    for (int r = 0; r < ROWS; r++) iv[r] = inv[min(r, nrows - 1)];
    for (int j = tid; j < n; j += RSM_THREADS) {
        float v[ROWS];
#pragma unroll
        for (int r = 0; r < ROWS; r++) v[r] = rowp[r][j];
#pragma unroll
        for (int r = 0; r < ROWS; r++)
            if (r < nrows) rowp[r][j] = v[r] * iv[r];
    }
}

// per (h, qi) terms in parallel (each sequential over d), then the
// reference's accumulation order over (h, qi) on lane 0
__global__ void __launch_bounds__(128)
k_stats_final(Geom g, const float * __restrict__ oo, const float * __restrict__ co,
              int mh, int mq, float * __restrict__ stats) {
    const int layer = blockIdx.x;
    __shared__ float t_cos[128], t_mse[128];
    __shared__ int t_agree[128];
    const int nt = mh * mq;
    for (int i = threadIdx.x; i < nt; i += blockDim.x) {
        const float * o = oo + ((long long)layer * nt + i) * g.dv;
        const float * c = co + ((long long)layer * nt + i) * g.dv;
        float dp = 0.0f, no = 0.0f, nc = 0.0f;
        for (int d = 0; d < g.dv; d++) { dp += o[d] * c[d]; no += o[d] * o[d]; nc += c[d] * c[d]; }
        t_cos[i] = dp / (sqrtf(no * nc) + 1e-8f);
        float mse = 0.0f;
        for (int d = 0; d < g.dv; d++) { const float df = o[d] - c[d]; mse += df * df; }
        t_mse[i] = mse / (float)g.dv;
        int ao = 0, ac = 0;
        for (int d = 1; d < g.dv; d++) {
            if (o[d] > o[ao]) ao = d;
            if (c[d] > c[ac]) ac = d;
        }
        t_agree[i] = (ao == ac) ? 1 : 0;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        float sum_cos = 0.0f, sum_mse = 0.0f;
        int agree = 0;
        for (int i = 0; i < nt; i++) { sum_cos += t_cos[i]; sum_mse += t_mse[i]; agree += t_agree[i]; }
        stats[layer * 3 + 0] = sum_cos / (float)nt;
        stats[layer * 3 + 1] = sum_mse / (float)nt;
        stats[layer * 3 + 2] = (float)agree / (float)nt;
    }
}

// ---------------------------------------------------------------------------
// Codec (state.h:326-629), bit-exact with the reference.
// ---------------------------------------------------------------------------
__device__ __forceinline__ float f16_to_f32_ref(uint16_t hv) {
    uint32_t sign = (uint32_t)(hv & 0x8000) << 16;
    uint32_t e = (hv >> 10) & 0x1F;
    uint32_t m = hv & 0x3FF;
    uint32_t bits;
    if (e == 0) {
        if (m == 0) {
            bits = sign;
        } else {
            e = 1;
            while (!(m & 0x400)) { m <<= 1; e--; }
            m &= 0x3FF;
            e = e + (127 - 15);
            bits = sign | (e << 23) | (m << 13);
        }
    } else if (e == 31) {
        bits = sign | 0x7F800000u | (m << 13);
    } else {
        e = e + (127 - 15);
        bits = sign | (e << 23) | (m << 13);
    }
    return __uint_as_float(bits);
}

__device__ __forceinline__ uint16_t f32_to_f16_ref(float val) {
    const uint32_t f = __float_as_uint(val);
    const uint32_t sign = (f >> 16) & 0x8000;
    const int32_t e = (int32_t)((f >> 23) & 0xFF) - 127 + 15;
    uint32_t m = (f >> 13) & 0x3FF;
    if (e <= 0) {
        if (e < -10) return (uint16_t)sign;
        m = (m | 0x400) >> (1 - e);
        return (uint16_t)(sign | m);
    } else if (e >= 31) {
        return (uint16_t)(sign | 0x7C00);
    }
    return (uint16_t)(sign | ((uint32_t)e << 10) | m);
}

__device__ __forceinline__ float fmax_std(float a, float b) { return (a < b) ? b : a; }
__device__ __forceinline__ float fmin_std(float a, float b) { return (b < a) ? b : a; }
__device__ __forceinline__ uint16_t load_u16(const uint8_t * p) { return (uint16_t)(p[0] | ((uint16_t)p[1] << 8)); }

// one work item per 32-element block (per element for F32/F16)
__global__ void __launch_bounds__(256)
k_dequant_rows(const uint8_t * __restrict__ src, int type, long long row_bytes, int n_el,
               long long rows, float * __restrict__ dst) {
    const long long nb = (type == 0 || type == 1 || type == 30) ? (long long)n_el : (long long)(n_el / 32);
    const long long total = rows * nb;
    for (long long e = (long long)blockIdx.x * blockDim.x + threadIdx.x; e < total;
         e += (long long)gridDim.x * blockDim.x) {
        const long long r = e / nb, b = e % nb;
        const uint8_t * s = src + r * row_bytes;
        float * o = dst + r * n_el;
        if (type == 0) {
            o[b] = __uint_as_float((uint32_t)s[4 * b] | ((uint32_t)s[4 * b + 1] << 8) |
                                   ((uint32_t)s[4 * b + 2] << 16) | ((uint32_t)s[4 * b + 3] << 24));
        } else if (type == 1) {
            o[b] = f16_to_f32_ref(load_u16(s + 2 * b));
        } else if (type == 30) {
            o[b] = __uint_as_float((uint32_t)load_u16(s + 2 * b) << 16);
        } else if (type == 8) {
            const uint8_t * bl = s + b * 34;
            const float d = f16_to_f32_ref(load_u16(bl));
            for (int i = 0; i < 32; i++) o[b * 32 + i] = d * (float)(int8_t)bl[2 + i];
        } else if (type == 2) {
            const uint8_t * bl = s + b * 18;
            const float d = f16_to_f32_ref(load_u16(bl));
            for (int i = 0; i < 16; i++) {
                o[b * 32 + 2 * i] = d * ((float)(bl[2 + i] & 0xF) - 8.0f);
                o[b * 32 + 2 * i + 1] = d * ((float)(bl[2 + i] >> 4) - 8.0f);
            }
        } else if (type == 3) {
            const uint8_t * bl = s + b * 20;
            const float d = f16_to_f32_ref(load_u16(bl)), m = f16_to_f32_ref(load_u16(bl + 2));
            for (int i = 0; i < 16; i++) {
                o[b * 32 + 2 * i] = d * (float)(bl[4 + i] & 0xF) + m;
                o[b * 32 + 2 * i + 1] = d * (float)(bl[4 + i] >> 4) + m;
            }
        }
    }
}

// bfloat16 encode: round to nearest, ties to even; NaN -> quiet NaN
__device__ __forceinline__ uint16_t f32_to_bf16(float x) {
    const uint32_t u = __float_as_uint(x);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
    return (uint16_t)((u + 0x7fffu + ((u >> 16) & 1u)) >> 16);
}

// quantize rows gathered by index (idx == nullptr: identity), src row stride src_ld
__global__ void __launch_bounds__(256)
k_quant_rows(const float * __restrict__ src, long long src_ld, const int * __restrict__ idx,
             int type, int n_el, long long rows, uint8_t * __restrict__ dst, long long row_bytes) {
    const long long nb = (type == 0 || type == 1 || type == 30) ? (long long)n_el : (long long)(n_el / 32);
    const long long total = rows * nb;
    for (long long e = (long long)blockIdx.x * blockDim.x + threadIdx.x; e < total;
         e += (long long)gridDim.x * blockDim.x) {
        const long long r = e / nb, b = e % nb;
        const long long sr = idx ? (long long)idx[r] : r;
        const float * x = src + sr * src_ld;
        uint8_t * o = dst + r * row_bytes;
        if (type == 0) {
            const uint32_t u = __float_as_uint(x[b]);
            o[4 * b] = u & 0xFF; o[4 * b + 1] = (u >> 8) & 0xFF; o[4 * b + 2] = (u >> 16) & 0xFF; o[4 * b + 3] = u >> 24;
        } else if (type == 1) {
            const uint16_t hv = f32_to_f16_ref(x[b]);
            o[2 * b] = hv & 0xFF; o[2 * b + 1] = hv >> 8;
        } else if (type == 30) {
            const uint16_t hv = f32_to_bf16(x[b]);
            o[2 * b] = hv & 0xFF; o[2 * b + 1] = hv >> 8;
        } else if (type == 8) {
            const float * xb = x + b * 32;
            uint8_t * ob = o + b * 34;
            float amax = 0.0f;
            for (int i = 0; i < 32; i++) { const float a = fabsf(xb[i]); if (a > amax) amax = a; }
            const float d = amax / 127.0f;
            const uint16_t hv = f32_to_f16_ref(d);
            ob[0] = hv & 0xFF; ob[1] = hv >> 8;
            const float id = (d != 0.0f) ? 127.0f / amax : 0.0f;
            for (int i = 0; i < 32; i++) {
                const float v = xb[i] * id;
                ob[2 + i] = (uint8_t)(int8_t)roundf(fmax_std(-128.0f, fmin_std(127.0f, v)));
            }
        } else if (type == 2) {
            const float * xb = x + b * 32;
            uint8_t * ob = o + b * 18;
            float amax = 0.0f;
            for (int i = 0; i < 32; i++) { const float a = fabsf(xb[i]); if (a > amax) amax = a; }
            const float d = amax / 7.0f;
            const uint16_t hv = f32_to_f16_ref(d);
            ob[0] = hv & 0xFF; ob[1] = hv >> 8;
            const float id = (d != 0.0f) ? 7.0f / amax : 0.0f;
            for (int i = 0; i < 16; i++) {
                const float v0 = xb[2 * i] * id + 8.0f;
                const float v1 = xb[2 * i + 1] * id + 8.0f;
                const uint8_t q0 = (uint8_t)fmax_std(0.0f, fmin_std(15.0f, roundf(v0)));
                const uint8_t q1 = (uint8_t)fmax_std(0.0f, fmin_std(15.0f, roundf(v1)));
                ob[2 + i] = (uint8_t)(q0 | (q1 << 4));
            }
        } else if (type == 3) {
            const float * xb = x + b * 32;
            uint8_t * ob = o + b * 20;
            float mn = xb[0], mx = xb[0];
            for (int i = 1; i < 32; i++) { if (xb[i] < mn) mn = xb[i]; if (xb[i] > mx) mx = xb[i]; }
            const float d = (mx - mn) / 15.0f;
            const uint16_t hd = f32_to_f16_ref(d), hm = f32_to_f16_ref(mn);
            ob[0] = hd & 0xFF; ob[1] = hd >> 8; ob[2] = hm & 0xFF; ob[3] = hm >> 8;
            const float id = (d != 0.0f) ? 15.0f / (mx - mn) : 0.0f;
            for (int i = 0; i < 16; i++) {
                const float v0 = (xb[2 * i] - mn) * id;
                const float v1 = (xb[2 * i + 1] - mn) * id;
                const uint8_t q0 = (uint8_t)fmax_std(0.0f, fmin_std(15.0f, roundf(v0)));
                const uint8_t q1 = (uint8_t)fmax_std(0.0f, fmin_std(15.0f, roundf(v1)));
                ob[4 + i] = (uint8_t)(q0 | (q1 << 4));
            }
        }
    }
}

// row j of the compacted V: concat over heads of C_v[h][j] (api.cpp:1243-1254)
__global__ void __launch_bounds__(256)
k_gather_cv_rows(const float * __restrict__ Cv, int H, int t, int dv, float * __restrict__ rows) {
    const long long total = (long long)t * H * dv;
    for (long long e = (long long)blockIdx.x * blockDim.x + threadIdx.x; e < total;
         e += (long long)gridDim.x * blockDim.x) {
        const long long j = e / ((long long)H * dv), r = e % ((long long)H * dv);
        const int h = (int)(r / dv), d = (int)(r % dv);
        rows[e] = Cv[((long long)h * t + j) * dv + d];
    }
}

// ---------------------------------------------------------------------------
// Whole-cache codec kernels (state.h:355-375, 528-567): eight elements per
// work item, the floats moved as 16-byte pieces, so a wave reads and writes
// contiguous memory. Quantization gives the four work items of a 32-element
// block to the four lanes of a quad, which reduce the block's largest
// magnitude between them (the largest non-NaN |x| from 0: one value in any
// order). Results equal k_dequant_rows / k_quant_rows bit for bit; Q4_1 and
// rows whose element count is not a multiple of 32 stay on those.
// ---------------------------------------------------------------------------

// rows [L][T] of codec `type` (row stride row_bytes, layer stride src_ls
// bytes) into dst [L][T][n_el] fp32
__global__ void __launch_bounds__(256)
k_dequant8(const uint8_t * __restrict__ src, int type, long long row_bytes, long long src_ls, int n_el, int T,
           int L, float * __restrict__ dst) {
    const int n8 = n_el >> 3;
    const long long total = (long long)L * T * n8;
    for (long long e = (long long)blockIdx.x * blockDim.x + threadIdx.x; e < total;
         e += (long long)gridDim.x * blockDim.x) {
        const long long rr = e / n8;
        const int q = (int)(e - rr * n8);
        const long long l = rr / T, r = rr - l * T;
        const uint8_t * s = src + l * src_ls + r * row_bytes;
        float v[8];
        // (block codecs: every 2-byte field sits at an even offset of an
        // even row stride, so it is read as one 2-byte load)
        if (type == 8) {          // Q8_0: d * q
            const uint8_t * bl = s + (q >> 2) * 34;
            const float d = f16_to_f32_ref(*reinterpret_cast<const uint16_t *>(bl));
            const uint16_t * qs = reinterpret_cast<const uint16_t *>(bl + 2 + 8 * (q & 3));
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const uint16_t w = qs[i];
                v[2 * i] = d * (float)(int8_t)(w & 0xFF);
                v[2 * i + 1] = d * (float)(int8_t)(w >> 8);
            }
        } else if (type == 2) {   // Q4_0: d * (nibble - 8), adjacent-pair nibbles
            const uint8_t * bl = s + (q >> 2) * 18;
            const float d = f16_to_f32_ref(*reinterpret_cast<const uint16_t *>(bl));
            const uint16_t * qs = reinterpret_cast<const uint16_t *>(bl + 2 + 4 * (q & 3));
#pragma unroll
            for (int i = 0; i < 2; i++) {
                const uint16_t w = qs[i];
                const uint8_t b0 = w & 0xFF, b1 = w >> 8;
                v[4 * i] = d * ((float)(b0 & 0xF) - 8.0f);
                v[4 * i + 1] = d * ((float)(b0 >> 4) - 8.0f);
                v[4 * i + 2] = d * ((float)(b1 & 0xF) - 8.0f);
                v[4 * i + 3] = d * ((float)(b1 >> 4) - 8.0f);
            }
        } else if (type == 1) {   // F16
#pragma unroll
            for (int i = 0; i < 8; i++) v[i] = f16_to_f32_ref(load_u16(s + 2 * (8 * q + i)));
        } else if (type == 30) {  // BF16
#pragma unroll
            for (int i = 0; i < 8; i++) v[i] = __uint_as_float((uint32_t)load_u16(s + 2 * (8 * q + i)) << 16);
        } else {                  // F32 (byte-assembled: rows need not be aligned)
#pragma unroll
            for (int i = 0; i < 8; i++) {
                const uint8_t * b = s + 4 * (8 * q + i);
                v[i] = __uint_as_float((uint32_t)b[0] | ((uint32_t)b[1] << 8) | ((uint32_t)b[2] << 16) |
                                       ((uint32_t)b[3] << 24));
            }
        }
        float4 * o = reinterpret_cast<float4 *>(dst + rr * n_el + 8 * q);
        o[0] = make_float4(v[0], v[1], v[2], v[3]);
        o[1] = make_float4(v[4], v[5], v[6], v[7]);
    }
}

// Quantize rows (l, j), j < rows, of L layers into codec `type` (row stride
// row_bytes, layer stride dst_ls bytes). Source row:
//   mode 0: src + l * src_ls + idx[l * idx_ls + j] * src_ld (kept rows of a cache)
//   mode 1: the concatenation over heads h of Cv[((l * H + h) * rows + j) * dv ..]
//           (a refitted value row, api.cpp:1243-1254; dv a multiple of 8)
__global__ void __launch_bounds__(256)
k_requant8(const float * __restrict__ src, long long src_ls, long long src_ld, const int * __restrict__ idx,
           long long idx_ls, int mode, int H, int dv, int type, int n_el, int rows, int L,
           uint8_t * __restrict__ dst, long long row_bytes, long long dst_ls, RowCodec sq) {
    const int n8 = n_el >> 3;
    const long long total = (long long)L * rows * n8;   // a multiple of 4: quads stay whole
    for (long long e = (long long)blockIdx.x * blockDim.x + threadIdx.x; e < total;
         e += (long long)gridDim.x * blockDim.x) {
        const long long rr = e / n8;
        const int q = (int)(e - rr * n8);
        const long long l = rr / rows, j = rr - l * rows;
        float4 a, b;
        if (mode == 0 && sq.base) {
            // kept rows of a quantized cache read in place: decoded, then re-encoded
            const long long r = idx[l * idx_ls + j];
            if (sq.type == 8) {
                a = codec_load4<8>(sq, (int)l, r, 8 * q);
                b = codec_load4<8>(sq, (int)l, r, 8 * q + 4);
            } else {
                a = codec_load4<2>(sq, (int)l, r, 8 * q);
                b = codec_load4<2>(sq, (int)l, r, 8 * q + 4);
            }
        } else {
            const float * x;
            if (mode == 0) {
                x = src + l * src_ls + (long long)idx[l * idx_ls + j] * src_ld + 8 * q;
            } else {
                const int h = (8 * q) / dv, v = 8 * q - h * dv;
                x = src + (((l * H + h) * rows + j) * dv + v);
            }
            a = reinterpret_cast<const float4 *>(x)[0];
            b = reinterpret_cast<const float4 *>(x)[1];
        }
        const float xv[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
        uint8_t * o = dst + l * dst_ls + j * row_bytes;
        if (type == 8 || type == 2) {
            float amax = 0.0f;
#pragma unroll
            for (int i = 0; i < 8; i++) {
                const float t = fabsf(xv[i]);
                if (t > amax) amax = t;
            }
            const float o1 = __shfl_xor(amax, 1);
            amax = o1 > amax ? o1 : amax;
            const float o2 = __shfl_xor(amax, 2);
            amax = o2 > amax ? o2 : amax;
            const int kq = q & 3;
            if (type == 8) {
                uint8_t * ob = o + (q >> 2) * 34;
                const float d = amax / 127.0f;
                const float id = (d != 0.0f) ? 127.0f / amax : 0.0f;
                if (kq == 0) {
                    const uint16_t hv = f32_to_f16_ref(d);
                    ob[0] = hv & 0xFF;
                    ob[1] = hv >> 8;
                }
                uint16_t * q16 = reinterpret_cast<uint16_t *>(ob + 2 + 8 * kq);   // 2-byte aligned
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const uint8_t q0 = (uint8_t)(int8_t)roundf(fmax_std(-128.0f, fmin_std(127.0f, xv[2 * i] * id)));
                    const uint8_t q1 =
                        (uint8_t)(int8_t)roundf(fmax_std(-128.0f, fmin_std(127.0f, xv[2 * i + 1] * id)));
                    q16[i] = (uint16_t)(q0 | ((uint16_t)q1 << 8));
                }
            } else {
                uint8_t * ob = o + (q >> 2) * 18;
                const float d = amax / 7.0f;
                const float id = (d != 0.0f) ? 7.0f / amax : 0.0f;
                if (kq == 0) {
                    const uint16_t hv = f32_to_f16_ref(d);
                    ob[0] = hv & 0xFF;
                    ob[1] = hv >> 8;
                }
                uint16_t * q16 = reinterpret_cast<uint16_t *>(ob + 2 + 4 * kq);
#pragma unroll
                for (int i = 0; i < 2; i++) {
                    uint8_t by[2];
#pragma unroll
                    for (int u = 0; u < 2; u++) {
                        const float v0 = xv[4 * i + 2 * u] * id + 8.0f;
                        const float v1 = xv[4 * i + 2 * u + 1] * id + 8.0f;
                        const uint8_t q0 = (uint8_t)fmax_std(0.0f, fmin_std(15.0f, roundf(v0)));
                        const uint8_t q1 = (uint8_t)fmax_std(0.0f, fmin_std(15.0f, roundf(v1)));
                        by[u] = (uint8_t)(q0 | (q1 << 4));
                    }
                    q16[i] = (uint16_t)(by[0] | ((uint16_t)by[1] << 8));
                }
            }
        } else if (type == 1 || type == 30) {
            uint16_t * o16 = reinterpret_cast<uint16_t *>(o) + 8 * q;   // rows of 2-byte elements
#pragma unroll
            for (int i = 0; i < 8; i++) o16[i] = type == 1 ? f32_to_f16_ref(xv[i]) : f32_to_bf16(xv[i]);
        } else {
#pragma unroll
            for (int i = 0; i < 8; i++) {
                const uint32_t u = __float_as_uint(xv[i]);
                uint8_t * b4 = o + 4 * (8 * q + i);
                b4[0] = u & 0xFF; b4[1] = (u >> 8) & 0xFF; b4[2] = (u >> 16) & 0xFF; b4[3] = u >> 24;
            }
        }
    }
}

// roundf (halves away from zero) for |y| < 2^23, as
// trunc(y + copysign(0.5 - 2^-25, y)): three instructions instead of six.
// Equal to roundf bit for bit on every float of that range (checked
// exhaustively: adding 0.5 - 2^-25 carries into the next integer exactly
// when the fraction is at least one half); a NaN gives a NaN.
__device__ __forceinline__ float roundf_small(float y) {
    return truncf(y + copysignf(0x1.fffffep-2f, y));
}

// One wave encodes up to 1024 elements of a row (32 blocks, Q8_0 or Q4_0,
// the reference's arithmetic, state.h:528-567): lane l holds elements
// 16 l .. 16 l + 15 in x (half of block l / 2; the block's amax comes from
// the lane pair), and lanes with `on` write the block's scale and their codes
// at so + (l / 2) * bytes-per-block. Every lane of the wave calls it.
template <int TYPE>
__device__ __forceinline__ void rq_encode16(const float (&x)[16], bool on, int lane, uint8_t * so) {
    constexpr int BB = TYPE == 8 ? 34 : 18;    // bytes per block
    float amax = 0.0f;
#pragma unroll
    for (int i = 0; i < 16; i++) {
        const float t = fabsf(x[i]);
        if (t > amax) amax = t;
    }
    const float o1 = __shfl_xor(amax, 1);
    amax = o1 > amax ? o1 : amax;
    const int b = lane >> 1, half = lane & 1;
    uint16_t * ob = reinterpret_cast<uint16_t *>(so + b * BB);   // 2-byte aligned
    if (on) {
        if constexpr (TYPE == 8) {
            const float d = amax / 127.0f;
            const float id = (d != 0.0f) ? 127.0f / amax : 0.0f;
            if (half == 0) ob[0] = f32_to_f16_ref(d);
#pragma unroll
            for (int i = 0; i < 8; i++) {
                const uint8_t q0 = (uint8_t)(int8_t)roundf_small(fmax_std(-128.0f, fmin_std(127.0f, x[2 * i] * id)));
                const uint8_t q1 =
                    (uint8_t)(int8_t)roundf_small(fmax_std(-128.0f, fmin_std(127.0f, x[2 * i + 1] * id)));
                ob[1 + 8 * half + i] = (uint16_t)(q0 | ((uint16_t)q1 << 8));
            }
        } else {
            const float d = amax / 7.0f;
            const float id = (d != 0.0f) ? 7.0f / amax : 0.0f;
            if (half == 0) ob[0] = f32_to_f16_ref(d);
#pragma unroll
            for (int i = 0; i < 4; i++) {
                uint8_t by[2];
#pragma unroll
                for (int u = 0; u < 2; u++) {
                    const float v0 = x[4 * i + 2 * u] * id + 8.0f;
                    const float v1 = x[4 * i + 2 * u + 1] * id + 8.0f;
                    const uint8_t q0 = (uint8_t)fmax_std(0.0f, fmin_std(15.0f, roundf_small(v0)));
                    const uint8_t q1 = (uint8_t)fmax_std(0.0f, fmin_std(15.0f, roundf_small(v1)));
                    by[u] = (uint8_t)(q0 | (q1 << 4));
                }
                ob[1 + 4 * half + i] = (uint16_t)(by[0] | ((uint16_t)by[1] << 8));
            }
        }
    }
}

// The same encodings (Q8_0 / Q4_0, the same arithmetic as k_requant8) one
// wave per row, for rows whose encoded bytes are whole 16-byte pieces at
// 16-byte aligned addresses. A row goes in chunks of up to 1024 elements:
// lane l takes elements 16 l .. 16 l + 15 of the chunk (half a 32-element
// block; the block's amax comes from the lane pair), writes its scale and
// codes into the wave's LDS copy of the chunk's encoded bytes, and the wave
// stores that copy as 16-byte pieces. Sources: MODE 0 gathered fp32 rows
// (src + l src_ls + idx[l idx_ls + j] src_ld), MODE 1 C_v [L][H][rows][dv],
// MODE 2 kept rows of a quantized cache (sq, rows staged into LDS as 16-byte
// pieces and decoded there).
constexpr int RQ_WAVES = 4;
constexpr int RQ_CHUNK = 1024;                 // elements per chunk
constexpr int RQ_BYTES = RQ_CHUNK / 32 * 34;   // encoded bytes of a chunk, at most (Q8_0)

template <int TYPE, int MODE>
__global__ void __launch_bounds__(64 * RQ_WAVES)
k_requant_rows(const float * __restrict__ src, long long src_ls, long long src_ld, const int * __restrict__ idx,
               long long idx_ls, int H, int dv, int n_el, int rows, int L, uint8_t * __restrict__ dst,
               long long row_bytes, long long dst_ls, RowCodec sq) {
    constexpr int BB = TYPE == 8 ? 34 : 18;    // bytes per block
    __shared__ __align__(16) uint8_t st_out[RQ_WAVES][RQ_BYTES];
    __shared__ __align__(16) uint8_t st_in[MODE == 2 ? RQ_WAVES : 1][MODE == 2 ? RQ_BYTES : 16];
    const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
    uint8_t * so = st_out[w];
    const long long nrows = (long long)L * rows;
    const long long step = (long long)gridDim.x * RQ_WAVES;
    // the raw source of one chunk of row rw (MODE 2: 16-byte pieces lane and
    // lane + 64 of the encoded row; else the lane's 16 values)
    auto fetch = [&](long long rw, int c0, float (&x)[16], uint4 & raw0, uint4 & raw1) {
        const int l = (int)(rw / rows);
        const long long j = rw - (long long)l * rows;
        const int ce = min(RQ_CHUNK, n_el - c0);
        if constexpr (MODE == 2) {
            const uint8_t * irow = codec_row(sq, l, idx[l * idx_ls + j]) + c0 / 32 * BB;
            const int np = ce / 32 * BB / 16;
            if (lane < np) raw0 = *reinterpret_cast<const uint4 *>(irow + 16 * lane);
            if (lane + 64 < np) raw1 = *reinterpret_cast<const uint4 *>(irow + 16 * (lane + 64));
        } else {
            const float * xs;
            if constexpr (MODE == 0) {
                xs = src + l * src_ls + (long long)idx[l * idx_ls + j] * src_ld + c0 + 16 * lane;
            } else {
                const int e = c0 + 16 * lane, h = e / dv, v = e - h * dv;
                xs = src + (((long long)l * H + h) * rows + j) * dv + v;
            }
            const bool on = lane < ce / 16;
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const float4 v = on ? reinterpret_cast<const float4 *>(xs)[i] : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
                x[4 * i] = v.x; x[4 * i + 1] = v.y; x[4 * i + 2] = v.z; x[4 * i + 3] = v.w;
            }
        }
    };
    // encode one chunk of row rw from its fetched source and store it
    auto put = [&](long long rw, int c0, float (&x)[16], const uint4 & raw0, const uint4 & raw1) {
        const int l = (int)(rw / rows);
        const long long j = rw - (long long)l * rows;
        const int ce = min(RQ_CHUNK, n_el - c0);   // a multiple of 256
        const int nb = ce / 32 * BB;                // encoded bytes (a multiple of 16)
        const bool on = lane < ce / 16;
        if constexpr (MODE == 2) {
            uint8_t * si = st_in[w];
            if (lane < nb / 16) *reinterpret_cast<uint4 *>(si + 16 * lane) = raw0;
            if (lane + 64 < nb / 16) *reinterpret_cast<uint4 *>(si + 16 * (lane + 64)) = raw1;
            __builtin_amdgcn_wave_barrier();
            __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront", "local");
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const float4 v = on ? codec_dec4<TYPE>(codec_raw4_at<TYPE>(si, 16 * lane + 4 * i))
                                    : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
                x[4 * i] = v.x; x[4 * i + 1] = v.y; x[4 * i + 2] = v.z; x[4 * i + 3] = v.w;
            }
        }
        rq_encode16<TYPE>(x, on, lane, so);
        // the wave's LDS writes are done before its reads of the copy
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront", "local");
        uint8_t * orow = dst + l * dst_ls + j * row_bytes + c0 / 32 * BB;
        for (int p = lane; p < nb / 16; p += 64)
            *reinterpret_cast<uint4 *>(orow + 16 * p) = *reinterpret_cast<const uint4 *>(so + 16 * p);
        // (the copies are rewritten for the next chunk or row only after these reads)
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront", "local");
    };
    const long long rw0 = (long long)blockIdx.x * RQ_WAVES + w;
    float x[16];
    uint4 raw0 = make_uint4(0, 0, 0, 0), raw1 = raw0;
    if (n_el <= RQ_CHUNK) {
        // one chunk a row: the next row's source is fetched before this row is encoded
        float xn[16];
        uint4 rn0 = raw0, rn1 = raw0;
        if (rw0 < nrows) fetch(rw0, 0, xn, rn0, rn1);
        for (long long rw = rw0; rw < nrows; rw += step) {
#pragma unroll
            for (int i = 0; i < 16; i++) x[i] = xn[i];
            raw0 = rn0;
            raw1 = rn1;
            if (rw + step < nrows) fetch(rw + step, 0, xn, rn0, rn1);
            put(rw, 0, x, raw0, raw1);
        }
    } else {
        for (long long rw = rw0; rw < nrows; rw += step)
            for (int c0 = 0; c0 < n_el; c0 += RQ_CHUNK) {
                fetch(rw, c0, x, raw0, raw1);
                put(rw, c0, x, raw0, raw1);
            }
    }
}

// ---------------------------------------------------------------------------
// Codec row tiles for the whole-cache decode (Q8_0 / Q4_0 rows whose byte
// length is a multiple of 16, at 16-byte aligned addresses): a block stages
// up to CT_ROWS whole rows in LDS, so HBM sees only 16-byte pieces, and
// writes one float4 per lane: every wave instruction reads or writes 1 KB
// of contiguous memory. The 2-byte scale and code fields are read in LDS,
// with the in-register decoders' products (codec_dec4, k_dequant8's values
// bit for bit).
// ---------------------------------------------------------------------------
constexpr int CT_THREADS = 256;
constexpr int CT_ROWS = 8;

// copy nr rows (row r at src_row(r), rb bytes, rb % 16 == 0) into LDS at
// lds + r * rb, four 16-byte loads per thread in flight. No load or store
// sits under a per-lane condition (under one, the loads were compiled into
// one at a time, each waited for): a piece index past the last stands for
// the last piece, read again and stored again with the same bytes.
template <class RowPtr>
__device__ __forceinline__ void ct_stage(uint8_t * lds, int nr, long long rb, RowPtr src_row) {
    const int pieces = (int)(rb >> 4), n = nr * pieces;
    for (int p0 = threadIdx.x; p0 < n; p0 += 4 * CT_THREADS) {
        int pp[4];
        uint4 v[4];
#pragma unroll
        for (int k = 0; k < 4; k++) {
            pp[k] = min(p0 + k * CT_THREADS, n - 1);
            const int rl = pp[k] / pieces, o = pp[k] - rl * pieces;
            v[k] = *reinterpret_cast<const uint4 *>(src_row(rl) + 16LL * o);
        }
#pragma unroll
        for (int k = 0; k < 4; k++) *reinterpret_cast<uint4 *>(lds + 16LL * pp[k]) = v[k];
    }
}

// rows [L][T] of codec TYPE (row stride row_bytes, layer stride src_ls
// bytes) into dst [L][T][n_el] fp32; grid (ceil(T / CT_ROWS), L): rows
// j0 .. j0 + nr - 1 of layer blockIdx.y per block
template <int TYPE>
__global__ void __launch_bounds__(CT_THREADS)
k_dequant_tile(const uint8_t * __restrict__ src, long long row_bytes, long long src_ls, int n_el, int T, int L,
               float * __restrict__ dst) {
    extern __shared__ __align__(16) uint8_t ct_lds[];
    const int j0 = blockIdx.x * CT_ROWS, l = blockIdx.y;
    const int nr = min(CT_ROWS, T - j0);
    const uint8_t * base = src + l * src_ls + (long long)j0 * row_bytes;
    ct_stage(ct_lds, nr, row_bytes, [&](int rl) { return base + rl * row_bytes; });
    __syncthreads();
    const int n4 = n_el >> 2;
    float4 * out = reinterpret_cast<float4 *>(dst + ((long long)l * T + j0) * n_el);
    for (int j = threadIdx.x; j < nr * n4; j += CT_THREADS) {
        const int rl = j / n4, c = 4 * (j - rl * n4);
        out[j] = codec_dec4<TYPE>(codec_raw4_at<TYPE>(ct_lds + rl * row_bytes, c));
    }
}

// Whether decoding a block and encoding it again gives back its own bytes,
// which holds for every block the encoder writes. Q8_0: with the scale d a
// positive normal f16 and the largest |q| exactly 127 (no q = -128), the
// decoded x = d q are exact (an 11-bit by 8-bit product), amax = 127 d, the
// new scale amax / 127 = d exactly (the same f16 bits), the inverse
// 127 / amax = fl(1 / d), and x fl(1 / d) = q (1 + e), |e| < 2^-22, which the
// clamp keeps and roundf takes back to q. Q4_0: the same with x = d (q - 8),
// every q in 1..15 and the largest |q - 8| exactly 7 (amax = 7 d), so
// x fl(1 / d) + 8 rounds back to q. Lane l tests half l & 1 of block l / 2
// of the encoded row at `row`; its pair's result is merged in, so each lane
// answers for the whole block (lanes without `on` answer true). Every lane
// of the wave calls it.
template <int TYPE>
__device__ __forceinline__ bool recode_is_identity(const uint8_t * row, bool on, int lane) {
    constexpr int BB = TYPE == 8 ? 34 : 18;
    const int half = lane & 1;
    const uint8_t * bl = row + (lane >> 1) * BB;
    int bad = 0, ext = 1;   // (lanes without `on`)
    bool scale_ok = true;
    if (on) {
        const uint32_t sb = *reinterpret_cast<const uint16_t *>(bl);
        scale_ok = sb >= 0x0400u && sb <= 0x7BFFu;
        ext = 0;
        if constexpr (TYPE == 8) {
            const uint16_t * c = reinterpret_cast<const uint16_t *>(bl + 2 + 16 * half);
#pragma unroll
            for (int i = 0; i < 8; i++) {
                const uint32_t w = c[i];
#pragma unroll
                for (int k = 0; k < 2; k++) {
                    const uint32_t q = (w >> (8 * k)) & 0xFFu;
                    bad |= q == 0x80u;
                    ext |= (q == 0x7Fu) | (q == 0x81u);
                }
            }
        } else {
            const uint16_t * c = reinterpret_cast<const uint16_t *>(bl + 2 + 8 * half);
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const uint32_t w = c[i];
#pragma unroll
                for (int k = 0; k < 4; k++) {
                    const uint32_t q = (w >> (4 * k)) & 0xFu;
                    bad |= q == 0u;
                    ext |= (q == 1u) | (q == 15u);
                }
            }
        }
    }
    bad |= __shfl_xor(bad, 1);
    ext |= __shfl_xor(ext, 1);
    return scale_ok && !bad && ext;
}

// Kept rows of a quantized cache decoded and re-encoded (the bytes of
// k_requant_rows MODE 2) a tile of rows at a time, for rows of at most 1024
// elements: the block gathers nrb whole rows (through idx) into LDS with
// ct_stage, 16-byte pieces, each wave decodes its rows there and writes the
// encoding over them (the wave issues all its reads of a row before its
// first write, since every code depends on the block's amax; a row whose
// blocks all pass recode_is_identity is left as it is), and the block
// stores the tile as 16-byte pieces. grid ceil(L * rows / nrb), nrb * (the
// encoded row bytes) <= RC_LDS, nrb <= CT_THREADS.
constexpr int RC_LDS = 16384;

template <int TYPE>
__global__ void __launch_bounds__(CT_THREADS)
k_recode_tile(const int * __restrict__ idx, long long idx_ls, int n_el, int rows, int L, int nrb,
              uint8_t * __restrict__ dst, long long row_bytes, long long dst_ls, RowCodec sq) {
    constexpr int BB = TYPE == 8 ? 34 : 18;
    __shared__ __align__(16) uint8_t lds[RC_LDS];
    __shared__ long long srco[CT_THREADS], dsto[CT_THREADS];   // byte offsets from sq.base and dst
    const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63;
    const long long nrows = (long long)L * rows, r0 = (long long)blockIdx.x * nrb;
    const int nr = (int)min((long long)nrb, nrows - r0);
    const int nb = n_el / 32 * BB, np = nb / 16;
    if (tid < nr) {
        const long long rw = r0 + tid;
        const int l = (int)(rw / rows);
        const long long j = rw - (long long)l * rows;
        srco[tid] = l * sq.layer_bytes + idx[l * idx_ls + j] * sq.row_bytes;
        dsto[tid] = l * dst_ls + j * row_bytes;
    }
    __syncthreads();
    ct_stage(lds, nr, nb, [&](int rl) { return sq.base + srco[rl]; });
    __syncthreads();
    const bool on = lane < n_el / 16;
    for (int rl = w; rl < nr; rl += CT_THREADS / 64) {
        uint8_t * row = lds + rl * nb;
        if (__all(recode_is_identity<TYPE>(row, on, lane))) continue;
        float x[16];
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const float4 v = on ? codec_dec4<TYPE>(codec_raw4_at<TYPE>(row, 16 * lane + 4 * i))
                                : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
            x[4 * i] = v.x; x[4 * i + 1] = v.y; x[4 * i + 2] = v.z; x[4 * i + 3] = v.w;
        }
        rq_encode16<TYPE>(x, on, lane, row);
    }
    __syncthreads();
    for (int p = tid; p < nr * np; p += CT_THREADS) {
        const int rl = p / np, o = p - rl * np;
        *reinterpret_cast<uint4 *>(dst + dsto[rl] + 16 * o) = *reinterpret_cast<const uint4 *>(lds + 16 * p);
    }
}

// ---------------------------------------------------------------------------
// llama.cpp state blobs (state.h:425-462, 645-810; kv-compact.cpp:659-685):
// the layout moves around the compaction itself.
// ---------------------------------------------------------------------------
// [rows][cols] -> [cols][rows], 32 x 32 tiles through LDS; grid (ceil(cols/32),
// ceil(rows/32)), 32 x 8 threads
__global__ void __launch_bounds__(256)
k_transpose(const float * __restrict__ src, long long rows, long long cols, float * __restrict__ dst) {
    __shared__ float tile[32][33];
    const long long r0 = (long long)blockIdx.y * 32, c0 = (long long)blockIdx.x * 32;
    const int tx = threadIdx.x & 31, ty = threadIdx.x >> 5;
    for (int i = ty; i < 32; i += 8) {
        const long long r = r0 + i, c = c0 + tx;
        tile[i][tx] = (r < rows && c < cols) ? src[r * cols + c] : 0.0f;
    }
    __syncthreads();
    for (int i = ty; i < 32; i += 8) {
        const long long c = c0 + i, r = r0 + tx;
        if (c < cols && r < rows) dst[c * rows + r] = tile[tx][i];
    }
}

// Kept key rows with the beta fold of the blob writer (state.h:714-728):
// out[j][h * dk + d] = K[sel[j]][h * dk + d] + (beta[h][j] * scale) * dir[h][d],
// other columns copied. grid (ceil(t * nk / 256))
__global__ void __launch_bounds__(256)
k_fold_rows(const float * __restrict__ K, int nk, const int * __restrict__ sel, int t, const float * __restrict__ beta,
            const float * __restrict__ dir, int H, int dk, float scale, float * __restrict__ out) {
    const long long total = (long long)t * nk;
    for (long long e = (long long)blockIdx.x * blockDim.x + threadIdx.x; e < total;
         e += (long long)gridDim.x * blockDim.x) {
        const int j = (int)(e / nk), c = (int)(e % nk);
        float x = K[(long long)sel[j] * nk + c];
        if (c < H * dk) {
            const int h = c / dk, d = c - h * dk;
            const float bs = beta[(long long)h * t + j] * scale;
            x = x + bs * dir[(long long)h * dk + d];
        }
        out[e] = x;
    }
}

// Transposed value columns of the blob writer (state.h:770-800): col[d][j] for
// d < H * dv, j < t, from C_v [H][t][dv] (Cv != nullptr) or, for a layer the
// filter keeps as is, from the original rows V[sel[j]][d] (row width nv).
__global__ void __launch_bounds__(256)
k_value_columns(const float * __restrict__ Cv, const float * __restrict__ V, int nv, const int * __restrict__ sel,
                int H, int dv, int t, float * __restrict__ col) {
    const long long total = (long long)H * dv * t;
    for (long long e = (long long)blockIdx.x * blockDim.x + threadIdx.x; e < total;
         e += (long long)gridDim.x * blockDim.x) {
        const int d = (int)(e / t), j = (int)(e % t);
        const int h = d / dv, c = d - h * dv;
        col[e] = Cv ? Cv[((long long)h * t + j) * dv + c] : V[(long long)sel[j] * nv + d];
    }
}

// Reference queries of the direction fit (kv-compact.cpp:674-681): rows
// q0 .. q0 + nq - 1 of each layer's keys, per head: out[l][h][i][d] =
// K[l][q0 + i][h * dk + d]. grid (ceil(H * nq * dk / 256), L)
__global__ void __launch_bounds__(256)
k_gather_qref(const float * __restrict__ K, long long ldK, int nk, int q0, int nq, int H, int dk,
              float * __restrict__ out) {
    const int l = blockIdx.y;
    const long long total = (long long)H * nq * dk;
    for (long long e = (long long)blockIdx.x * blockDim.x + threadIdx.x; e < total;
         e += (long long)gridDim.x * blockDim.x) {
        const int h = (int)(e / ((long long)nq * dk)), r = (int)(e % ((long long)nq * dk));
        const int i = r / dk, d = r - i * dk;
        out[(long long)l * total + e] = K[(long long)l * ldK + (long long)(q0 + i) * nk + h * dk + d];
    }
}

__global__ void __launch_bounds__(256) k_iota(int * __restrict__ p, long long n) {
    const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) p[i] = (int)i;
}

// ---------------------------------------------------------------------------
// Accelerator plug-in GEMMs (accel ABI), sequential accumulation.
// ---------------------------------------------------------------------------
__global__ void __launch_bounds__(256)
k_gemm_abt(const float * __restrict__ A, long long lda, const float * __restrict__ B, long long ldb,
           float * __restrict__ C, long long ldc, int m, int n, int k, float scale,
           long long sa, long long sb, long long sc) {
    const int bat = blockIdx.z;
    A += bat * sa; B += bat * sb; C += bat * sc;
    const int i = blockIdx.y * 16 + (threadIdx.x >> 4);
    const int j = blockIdx.x * 16 + (threadIdx.x & 15);
    if (i >= m || j >= n) return;
    float s = 0.0f;
    for (int l = 0; l < k; l++) s += A[(long long)i * lda + l] * B[(long long)j * ldb + l];
    C[(long long)i * ldc + j] = s * scale;
}

__global__ void __launch_bounds__(256)
k_gemm_ab(const float * __restrict__ A, long long lda, const float * __restrict__ B, long long ldb,
          float * __restrict__ C, long long ldc, int m, int n, int k,
          long long sa, long long sb, long long sc) {
    const int bat = blockIdx.z;
    A += bat * sa; B += bat * sb; C += bat * sc;
    const int i = blockIdx.y * 16 + (threadIdx.x >> 4);
    const int j = blockIdx.x * 16 + (threadIdx.x & 15);
    if (i >= m || j >= n) return;
    float s = 0.0f;
    for (int l = 0; l < k; l++) s += A[(long long)i * lda + l] * B[(long long)l * ldb + j];
    C[(long long)i * ldc + j] = s;
}

// ===========================================================================
// Host launch wrappers
// ===========================================================================
static inline unsigned cdiv(long long a, long long b) { return (unsigned)((a + b - 1) / b); }
static inline unsigned grid_cap(long long n, int bs) {
    long long g = (n + bs - 1) / bs;
    return (unsigned)(g < 1 ? 1 : (g > 65535 * 4 ? 65535 * 4 : g));
}

hipError_t set_exp2_table(const uint64_t * tab32) {
    return hipMemcpyToSymbol(HIP_SYMBOL(c_exp2_tab), tab32, 32 * sizeof(uint64_t));
}

void launch_scores(const Geom & g, const ChunkDesc * chunks, int n_chunk_units, int Tc_max,
                   const float * K, const float * Q, float * S, int Hs, int nq_cap,
                   long long s_layer, long long s_head, long long s_row, int qmode, hipStream_t st,
                   const int * key_idx, const float * beta, unsigned * tmax) {
    dim3 grid(cdiv(Tc_max, SC_KEYS), n_chunk_units * Hs, g.L);
    switch (codec_inst(g.kc)) {
    case 8:
        hipLaunchKernelGGL(k_scores<8>, grid, dim3(256), 0, st, g, chunks, K, Q, S, Hs, nq_cap,
                           s_layer, s_head, s_row, qmode, key_idx, beta, tmax);
        break;
    case 2:
        hipLaunchKernelGGL(k_scores<2>, grid, dim3(256), 0, st, g, chunks, K, Q, S, Hs, nq_cap,
                           s_layer, s_head, s_row, qmode, key_idx, beta, tmax);
        break;
    default:
        hipLaunchKernelGGL(k_scores<0>, grid, dim3(256), 0, st, g, chunks, K, Q, S, Hs, nq_cap,
                           s_layer, s_head, s_row, qmode, key_idx, beta, tmax);
    }
}

void launch_chunk_softmax(const Geom & g, const Work & w, hipStream_t st) {
    hipLaunchKernelGGL(k_softmax_importance, dim3(g.n_chunks * g.H, g.L), dim3(256),
                       (size_t)2 * g.nq_max * sizeof(float), st,
                       g, w.chunks, w.S, w.smax, w.A, w.E ? w.rowsum : nullptr, w.ainv, w.imp,
                       w.sens && g.score_method != 0 ? w.amax : nullptr);
    // sensitivity per (layer, chunk, head) from the per-key maxima over
    // queries (the importance itself under the max score method)
    if (w.sens)
        hipLaunchKernelGGL(k_head_sensitivity, dim3(g.n_chunks * g.H, g.L), dim3(64), 0, st,
                           g, w.chunks, g.score_method != 0 ? w.amax : w.imp, w.sens);
}

template <int VC>
void launch_refit_inst(const Geom & g, const Work & w, const float * V, bool v128, hipStream_t st) {
    const dim3 grid(g.n_chunks * g.H, g.L);
    if (v128)
        hipLaunchKernelGGL(k_refit_target<VC>, grid, dim3(256), 0, st, g, w.chunks, w.A, w.ainv, V, w.Y);
    else
        hipLaunchKernelGGL(k_refit_target_any<VC>, grid, dim3(256), 0, st, g, w.chunks, w.A, w.ainv, V, w.Y);
}

void launch_refit_target(const Geom & g, const Work & w, const float * V, hipStream_t st) {
    // every (layer, chunk, head) value row starts 16-byte aligned when V does
    // and the layer, token and head strides are multiples of four floats (a
    // quantized V read in place is decoded four elements at a time)
    const int vc = codec_inst(g.vc);
    const bool v128 = g.dv == 128 && (vc || ((reinterpret_cast<uintptr_t>(V) & 15) == 0 && (g.ldV & 3) == 0 &&
                                              (((long long)g.H * g.dv) & 3) == 0));
    if (vc == 8) launch_refit_inst<8>(g, w, V, v128, st);
    else if (vc == 2) launch_refit_inst<2>(g, w, V, v128, st);
    else launch_refit_inst<0>(g, w, V, v128, st);
}

void launch_global_importance(const Geom & g, const Work & w, hipStream_t st) {
    hipLaunchKernelGGL(k_global_importance, dim3(g.n_chunks, g.L), dim3(256), 0, st,
                       g, w.chunks, w.imp, w.wts, w.sens, w.gimp);
}

void launch_div_level(const Geom & g, const Work & w, const DivWork & dw, const float * K, hipStream_t st) {
    const unsigned units = (unsigned)(g.L * g.n_chunks);
    const int nt = cdiv(dw.cap, DG_TILE);
    hipLaunchKernelGGL(k_div_candidates, dim3(g.n_chunks, g.L), dim3(256), 0, st, g, w.chunks, w.gimp, dw, w.cand);
    const dim3 ggrid(cdiv((int)units, 8) * 8 * (nt * (nt + 1) / 2));   // XCD-grouped (k_div_gram)
    switch (codec_inst(g.kc)) {
    case 8: hipLaunchKernelGGL(k_div_gram<8>, ggrid, dim3(256), 0, st, g, w.chunks, K, dw, w.cand); break;
    case 2: hipLaunchKernelGGL(k_div_gram<2>, ggrid, dim3(256), 0, st, g, w.chunks, K, dw, w.cand); break;
    default: hipLaunchKernelGGL(k_div_gram<0>, ggrid, dim3(256), 0, st, g, w.chunks, K, dw, w.cand);
    }
    if (dw.cap <= 8 * 64)
        hipLaunchKernelGGL(k_div_greedy<8>, dim3(units), dim3(64), 0, st, g, w.chunks, w.gimp, dw, w.cand, w.sel);
    else
        hipLaunchKernelGGL(k_div_greedy<DIV_MAX_CAND / 64>, dim3(units), dim3(64), 0, st, g, w.chunks, w.gimp, dw,
                           w.cand, w.sel);
}

void launch_select_topk(const Geom & g, const Work & w, hipStream_t st) {
    const size_t lds = (size_t)g.Tc_max * (sizeof(float) + sizeof(int) + 1);
    const int lds_ok = lds <= 60 * 1024 ? 1 : 0;
    hipLaunchKernelGGL(k_select_topk, dim3(g.n_chunks, g.L), dim3(256), lds_ok ? lds : 0, st,
                       g, w.chunks, w.gimp, w.cand, w.flags, w.sel, lds_ok);
}

__global__ void __launch_bounds__(256) k_fill_int(int * __restrict__ p, int v, long long n) {
    const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) p[i] = v;
}

void launch_fill_int(int * p, int v, long long n, hipStream_t st) {
    if (n <= 0) return;
    hipLaunchKernelGGL(k_fill_int, dim3(cdiv(n, 256)), dim3(256), 0, st, p, v, n);
}

__global__ void __launch_bounds__(256) k_fill_f32(float * __restrict__ p, float v, long long n) {
    for (long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (long long)gridDim.x * blockDim.x)
        p[i] = v;
}

void launch_fill_f32(float * p, float v, long long n, hipStream_t st) {
    if (n <= 0) return;
    hipLaunchKernelGGL(k_fill_f32, dim3(grid_cap(n, 256)), dim3(256), 0, st, p, v, n);
}

void launch_refine_step(const Geom & g, const Work & w, hipStream_t st) {
    hipLaunchKernelGGL(k_refine_step, dim3(g.n_chunks, g.L), dim3(256), 0, st, g, w.chunks, w.X, w.gimp, w.sel,
                       w.flags, w.refine_active);
}

void launch_ls_softmax(const Geom & g, const Work & w, const float * beta, hipStream_t st, const float * Ssel) {
    // LDS for the largest chunk's rows (every smaller chunk then fits as many)
    const int W = g.tc_max;
    const int rows = lsx_rows(W, LSX_LDS_BYTES / 4);
    const size_t bytes = rows >= 1 ? sizeof(float) * (2 * (size_t)W + (size_t)rows * (W + 1)) : LSX_LDS_BYTES;
    hipLaunchKernelGGL(k_ls_softmax, dim3(g.n_chunks * g.H, g.L), dim3(256), bytes, st,
                       g, w.chunks, w.S, w.sel, beta, w.X, (int)(bytes / sizeof(float)), Ssel);
}

bool score_attend_ok(const Geom & g, const float * K, const float * V, const float * Q, int Tc_max, int nq_max,
                     int qmode) {
    const auto al16 = [](const void * p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; };
    return Tc_max <= FA_KEYS && nq_max >= 1 && nq_max <= FA_ROWS && qmode != Q_CHEAP_LOCAL && g.dv == 128 &&
           g.dk >= 16 && (g.dk & 15) == 0 && !g.kc.base && !g.vc.base && K && V && al16(K) && al16(V) &&
           (g.ldK & 3) == 0 && (g.ldV & 3) == 0 && ((long long)g.H * g.dk & 3) == 0 &&
           (qmode != Q_PROVIDED || Q);
}

void launch_score_attend(const Geom & g, const Work & w, const float * K, const float * V, const float * Q,
                         float * S, int mh, hipStream_t st) {
    hipLaunchKernelGGL(k_query_columns, dim3(g.H, g.L), dim3(256), 0, st, g, w.chunks, K, Q, w.Qt);
    hipLaunchKernelGGL(k_score_attend, dim3(g.n_chunks * g.H, g.L), dim3(FA_THREADS), 0, st,
                       g, w.chunks, K, w.Qt, V, S, mh, S ? w.smax : nullptr, w.imp, w.ainv, w.Y);
}

void launch_gather_exp(const Geom & g, const Work & w, hipStream_t st) {
    hipLaunchKernelGGL(k_gather_exp, dim3(g.n_chunks * g.H, g.L), dim3(256), 0, st, g, w.chunks, w.E, w.sel, w.X);
}

void launch_nnls_lh(const Geom & g, const Work & w, float * wout, int max_iter, int * status, hipStream_t st) {
    hipLaunchKernelGGL(k_nnls_lh, dim3(g.n_chunks * g.H, g.L), dim3(64), 0, st, g, w.chunks, w.aug, w.aug_off,
                       wout, max_iter, status);
}

void launch_nnls_pgd(const Geom & g, const Work & w, float * wb, int iters, hipStream_t st) {
    const size_t lds = (size_t)(3 * g.tc_max + g.nq_max) * sizeof(float);
    // beyond 64 KB of dynamic LDS the kernel needs the attribute (set once;
    // PGD_LDS_FLOATS leaves room for the kernel's static LDS)
    static bool lds_set = false;
    if (lds > 65536 && !lds_set)
        lds_set = hipFuncSetAttribute(reinterpret_cast<const void *>(k_nnls_pgd),
                                      hipFuncAttributeMaxDynamicSharedMemorySize,
                                      PGD_LDS_FLOATS * (int)sizeof(float)) == hipSuccess;
    hipLaunchKernelGGL(k_nnls_pgd, dim3(g.n_chunks * g.H, g.L), dim3(256), lds, st,
                       g, w.chunks, w.X, w.aug, w.aug_off, wb, iters);
}

void launch_omp_select(const Geom & g, const Work & w, const OmpWork & ow, hipStream_t st) {
    hipLaunchKernelGGL(k_omp_select, dim3(g.n_chunks, g.L), dim3(256), 0, st,
                       g, w.chunks, w.A, w.rowsum, ow, w.sel, w.status);
}

void launch_beta_log(float * wb, long long n, hipStream_t st) {
    if (n <= 0) return;
    hipLaunchKernelGGL(k_beta_log, dim3((unsigned)cdiv(n, 256)), dim3(256), 0, st, wb, n);
}

void launch_ls_build(const Geom & g, const Work & w, hipStream_t st, bool m_by_lu) {
    // dynamic LDS beyond 64 KB needs the kernel attribute (once per process)
    static int lds_cap = -1;
    if (lds_cap < 0)
        lds_cap = hipFuncSetAttribute(reinterpret_cast<const void *>(k_ls_build<false>),
                                      hipFuncAttributeMaxDynamicSharedMemorySize,
                                      LB_LDS_FLOATS * (int)sizeof(float)) == hipSuccess &&
                          hipFuncSetAttribute(reinterpret_cast<const void *>(k_ls_build<true>),
                                              hipFuncAttributeMaxDynamicSharedMemorySize,
                                              LB_LDS_FLOATS * (int)sizeof(float)) == hipSuccess
                      ? LB_LDS_FLOATS : 16384;
    const long long need = (long long)g.nq_max * ((g.tc_max + g.dv + 3) & ~3);
    // every system's rows fit: one block per system; else slabs of rows
    // through the whole budget, the tiles of a system over enough blocks to
    // give the GPU about 2048 of them
    const int wmax = (g.tc_max + g.dv + 3) & ~3;
    // (slabs of at least 8 rows in about 40 KB: four blocks per CU; whole
    // systems only up to 48 KB, three blocks per CU)
    const bool whole = need <= std::min(lds_cap, 12288);
    const int lds_floats = whole ? (int)need : std::min(lds_cap, std::max(8 * wmax, 10240));
    const long long systems = (long long)g.n_chunks * g.H * g.L;
    const int nz = whole ? 1 : (int)std::max<long long>(1, std::min<long long>(64, (2048 + systems - 1) / systems));
    if (whole)
        hipLaunchKernelGGL(k_ls_build<false>, dim3(g.n_chunks * g.H, g.L), dim3(256), (size_t)lds_floats * sizeof(float),
                           st, g, w.chunks, w.X, w.Y, w.aug, w.aug_off, lds_floats, m_by_lu ? 1 : 0);
    else
        hipLaunchKernelGGL(k_ls_build<true>, dim3(g.n_chunks * g.H, g.L, nz), dim3(256),
                           (size_t)lds_floats * sizeof(float), st, g, w.chunks, w.X, w.Y, w.aug, w.aug_off, lds_floats,
                           m_by_lu ? 1 : 0);
}

// KVC_LU_SPLIT=0 (read at every launch) factors every system in one pass of
// k_ge_lu instead of k_ge_lu<false, true> + k_ge_lu_tail
static bool lu_split_enabled() {
    const char * e = getenv("KVC_LU_SPLIT");
    return !(e && e[0] == '0');
}

void launch_ge_lu(const Geom & g, const Work & w, hipStream_t st, bool m_by_lu) {
    // unmasked pass over every system, then the masked pass over the flagged ones
    const float * X = m_by_lu ? w.X : nullptr;
    const dim3 grid(g.n_chunks * g.H, g.L);
    if (w.LU2 && g.tc_max > LU_SPLIT && lu_split_enabled()) {
        hipLaunchKernelGGL((k_ge_lu<false, true>), grid, dim3(RG_THREADS), 0, st,
                           g, w.chunks, w.aug, w.aug_off, X, w.perm, w.skip, w.LU, w.lu_redo, w.status, w.LU2, w.map2);
        hipLaunchKernelGGL(k_ge_lu_tail, grid, dim3(LP_THREADS), 0, st,
                           g, w.chunks, w.LU2, w.map2, w.perm, w.skip, w.LU, w.lu_redo, w.status);
    } else {
        hipLaunchKernelGGL((k_ge_lu<false, false>), grid, dim3(RG_THREADS), 0, st,
                           g, w.chunks, w.aug, w.aug_off, X, w.perm, w.skip, w.LU, w.lu_redo, w.status, nullptr,
                           nullptr);
    }
    hipLaunchKernelGGL((k_ge_lu<true, false>), grid, dim3(RG_THREADS), 0, st,
                       g, w.chunks, w.aug, w.aug_off, X, w.perm, w.skip, w.LU, w.lu_redo, w.status, nullptr, nullptr);
}

void launch_ge_solve(const Geom & g, const Work & w, float * Cv, hipStream_t st) {
    const unsigned systems = (unsigned)(g.L * g.n_chunks * g.H);
    // k_ge_subst solves every system without a skipped pivot step, k_ge_solve
    // the others (KVC_SOLVE_OLD=1: k_ge_solve all of them)
    static const bool old_solve = [] {
        const char * e = getenv("KVC_SOLVE_OLD");
        return e && e[0] == '1';
    }();
    if (!old_solve) {
        const unsigned nw = cdiv(g.dv, 64);
        const size_t lds = (size_t)nw * SB_LROWS * 64 * sizeof(float);
        static int lds_ok = -1;
        if (lds_ok < 0)
            lds_ok = hipFuncSetAttribute(reinterpret_cast<const void *>(k_ge_subst),
                                         hipFuncAttributeMaxDynamicSharedMemorySize,
                                         4 * SB_LROWS * 64 * (int)sizeof(float)) == hipSuccess;
        hipLaunchKernelGGL(k_ge_subst, dim3(systems), dim3(64 * nw), lds, st,
                           g, w.chunks, w.aug, w.aug_off, w.perm, w.skip, w.LU, Cv);
    }
    hipLaunchKernelGGL(k_ge_solve, dim3(systems, cdiv(g.dv, 64)), dim3(64), 0, st,
                       g, w.chunks, w.aug, w.aug_off, w.perm, w.skip, w.LU, w.Bt, Cv, old_solve ? 0 : 1);
    if (g.tc_max > RG_ROWS) {
        // dynamic LDS: the largest system's panels (3 pb n floats), or the
        // step-by-step factors; the attribute once per process
        static int ge_lds_ok = -1;
        if (ge_lds_ok < 0)
            ge_lds_ok = hipFuncSetAttribute(reinterpret_cast<const void *>(k_ge_general),
                                            hipFuncAttributeMaxDynamicSharedMemorySize,
                                            GE_BLK_LDS * (int)sizeof(float)) == hipSuccess;
        const int pb = ge_panel(g.tc_max);
        size_t lds = pb >= 1 ? (size_t)3 * pb * g.tc_max * sizeof(float) : (size_t)GE_LDS_FLOATS * sizeof(float);
        // without the attribute a launch above 64 KB fails, and run_batch's
        // error check turns that into -6 (the kernel is never run short of LDS)
        (void)ge_lds_ok;
        hipLaunchKernelGGL(k_ge_general, dim3(g.n_chunks * g.H, g.L), dim3(512), lds, st,
                           g, w.chunks, w.aug, w.aug_off, Cv, w.gtmp);
    }
}

// Original attention of the sampled queries over all T (outputs OO): needs
// only the main scores (or the statistics' own) and V, so it may run beside
// the compaction once the main path no longer reads S (row softmax rewrites
// the rows of S it uses in place).
// The statistics' sums take the narrow kernel when the wide grid would not
// give every CU a block.
bool stats_narrow(const Geom & g, unsigned sv_blocks) { return (long long)sv_blocks * g.L < 256; }

void launch_row_softmax(const Geom & g, float * x, int n, long long ls, long long hs, long long rs, int mh, int mq,
                        RowMaxSrc ms, float * inv_out, hipStream_t st, bool beside_lu = false) {
    const int rows = mh * mq;
    if (beside_lu || (long long)cdiv(rows, RSM_ROWS) * g.L < 256)
        hipLaunchKernelGGL(k_row_softmax<RSM_ROWS_FEW>, dim3(cdiv(rows, RSM_ROWS_FEW), g.L), dim3(RSM_THREADS), 0, st,
                           x, n, ls, hs, rs, mh, mq, ms, inv_out);
    else
        hipLaunchKernelGGL(k_row_softmax<RSM_ROWS>, dim3(cdiv(rows, RSM_ROWS), g.L), dim3(RSM_THREADS), 0, st,
                           x, n, ls, hs, rs, mh, mq, ms, inv_out);
}

void launch_stats_original(const Geom & g, const Work & w, const StatWork & sw, const float * K,
                           const float * V, const float * Q, hipStream_t st, float * S_main, bool beside_lu) {
    const ChunkDesc * whole = w.chunks + g.n_chunks;      // all T keys
    const long long osl = (long long)sw.mh * sw.mq * g.T;
    const unsigned sv_blocks = (unsigned)(sw.mh * cdiv(sw.mq, SV_QB) * cdiv(g.dv, SV_VB));
    // the main path's scores S [L][H][nq_max][T] hold exactly these rows when
    // the statistics use the main query set, else they are computed here
    float * os = sw.OS;
    long long o_ls = osl, o_hs = (long long)sw.mq * g.T;
    RowMaxSrc ms{};
    if (S_main) {
        os = S_main;
        o_ls = (long long)g.H * g.nq_max * g.T;
        o_hs = (long long)g.nq_max * g.T;
        if (w.smax) {
            ms.tm = w.smax;
            ms.chunks = w.chunks;
            ms.nc = g.n_chunks;
            ms.nt = cdiv(g.Tc_max, SC_KEYS);
            ms.rs = (long long)ms.nc * ms.nt;
            ms.hs = (long long)g.nq_max * ms.rs;
            ms.ls = (long long)g.H * ms.hs;
        }
    } else {
        launch_scores(g, whole, 1, g.T, K, Q, sw.OS, sw.mh, sw.mq, osl, (long long)sw.mq * g.T, g.T, sw.qmode, st,
                      nullptr, nullptr);
    }
    launch_row_softmax(g, os, g.T, o_ls, o_hs, (long long)g.T, sw.mh, sw.mq, ms, sw.OI, st, beside_lu);
    const dim3 sgrid(sv_blocks, g.L);
    if (codec_inst(g.vc) == 0 && stats_narrow(g, sv_blocks)) {
        hipLaunchKernelGGL(k_stats_values_narrow, dim3(sw.mh * cdiv(sw.mq, SVN_QB) * cdiv(g.dv, SVN_VB), g.L),
                           dim3(SV_THREADS), 0, st, g, os, sw.OI, o_ls, o_hs, (long long)g.T, g.T, V, nullptr, 1,
                           sw.OO, sw.mh, sw.mq);
        return;
    }
    // beside the factorizations: the form that shares a CU with a k_ge_lu
    // block (fp32 V, whole 64-column blocks, 16-byte aligned weight rows,
    // 32-bit offsets)
    const bool lean = beside_lu && codec_inst(g.vc) == 0 && g.dv % 64 == 0 && g.T % 4 == 0 &&
                      o_ls % 4 == 0 && o_hs % 4 == 0 && (reinterpret_cast<uintptr_t>(os) & 15) == 0 &&
                      ((long long)g.T + SL_KT) * g.H * g.dv * 4 < (1ll << 31) &&
                      (long long)sw.mq * g.T * 4 < (1ll << 31);
    if (lean) {
        hipLaunchKernelGGL(k_stats_values_lean, dim3(sw.mh * cdiv(sw.mq, SL_QB) * (g.dv / 64), g.L), dim3(256),
                           SL_LDS, st, g, os, sw.OI, o_ls, o_hs, (long long)g.T, g.T, V, sw.OO, sw.mh, sw.mq);
        return;
    }
    switch (codec_inst(g.vc)) {
    case 8:
        hipLaunchKernelGGL(k_stats_values<8>, sgrid, dim3(SV_THREADS), SV_LDS, st,
                           g, os, sw.OI, o_ls, o_hs, (long long)g.T, g.T, V, nullptr, 1, sw.OO, sw.mh, sw.mq);
        break;
    case 2:
        hipLaunchKernelGGL(k_stats_values<2>, sgrid, dim3(SV_THREADS), SV_LDS, st,
                           g, os, sw.OI, o_ls, o_hs, (long long)g.T, g.T, V, nullptr, 1, sw.OO, sw.mh, sw.mq);
        break;
    default:
        hipLaunchKernelGGL(k_stats_values<0>, sgrid, dim3(SV_THREADS), SV_LDS, st,
                           g, os, sw.OI, o_ls, o_hs, (long long)g.T, g.T, V, nullptr, 1, sw.OO, sw.mh, sw.mq);
    }
}

// Compacted attention over the kept keys with beta and C_v (outputs CO), then
// the statistics from OO and CO.
void launch_stats_compacted(const Geom & g, const Work & w, const StatWork & sw, const float * K,
                            const float * V, const float * Q, const float * beta, const float * Cv,
                            float * stats, hipStream_t st) {
    const ChunkDesc * kept = w.chunks + g.n_chunks + 1;   // the t_total kept keys
    const long long csl = (long long)sw.mh * sw.mq * g.t_total;
    const unsigned sv_blocks = (unsigned)(sw.mh * cdiv(sw.mq, SV_QB) * cdiv(g.dv, SV_VB));
    launch_scores(g, kept, 1, g.t_total, K, Q, sw.CS, sw.mh, sw.mq, csl, (long long)sw.mq * g.t_total, g.t_total,
                  sw.qmode, st, w.sel, beta);
    launch_row_softmax(g, sw.CS, g.t_total, csl, (long long)sw.mq * g.t_total, (long long)g.t_total, sw.mh, sw.mq,
                       RowMaxSrc{}, sw.CI, st);
    if (stats_narrow(g, sv_blocks))
        hipLaunchKernelGGL(k_stats_values_narrow, dim3(sw.mh * cdiv(sw.mq, SVN_QB) * cdiv(g.dv, SVN_VB), g.L),
                           dim3(SV_THREADS), 0, st, g, sw.CS, sw.CI, csl, (long long)sw.mq * g.t_total,
                           (long long)g.t_total, g.t_total, V, Cv, 2, sw.CO, sw.mh, sw.mq);
    else
        hipLaunchKernelGGL(k_stats_values<0>, dim3(sv_blocks, g.L), dim3(SV_THREADS), SV_LDS, st,
                           g, sw.CS, sw.CI, csl, (long long)sw.mq * g.t_total, (long long)g.t_total, g.t_total, V, Cv,
                           2, sw.CO, sw.mh, sw.mq);
}

void launch_stats_final(const Geom & g, const StatWork & sw, float * stats, hipStream_t st) {
    hipLaunchKernelGGL(k_stats_final, dim3(g.L), dim3(128), 0, st, g, sw.OO, sw.CO, sw.mh, sw.mq, stats);
}

void launch_stats(const Geom & g, const Work & w, const StatWork & sw, const float * K,
                  const float * V, const float * Q, const float * beta, const float * Cv,
                  float * stats, hipStream_t st, float * S_main) {
    launch_stats_original(g, w, sw, K, V, Q, st, S_main);
    launch_stats_compacted(g, w, sw, K, V, Q, beta, Cv, stats, st);
    launch_stats_final(g, sw, stats, st);
}

void launch_dequant_rows(const uint8_t * src, int type, long long row_bytes, int n_el, long long rows,
                         float * dst, hipStream_t st) {
    const long long nb = (type == 0 || type == 1 || type == 30) ? (long long)n_el : (long long)(n_el / 32);
    hipLaunchKernelGGL(k_dequant_rows, dim3(grid_cap(rows * nb, 256)), dim3(256), 0, st,
                       src, type, row_bytes, n_el, rows, dst);
}

void launch_quant_rows(const float * src, long long src_ld, const int * idx, int type, int n_el,
                       long long rows, uint8_t * dst, long long row_bytes, hipStream_t st) {
    const long long nb = (type == 0 || type == 1 || type == 30) ? (long long)n_el : (long long)(n_el / 32);
    hipLaunchKernelGGL(k_quant_rows, dim3(grid_cap(rows * nb, 256)), dim3(256), 0, st,
                       src, src_ld, idx, type, n_el, rows, dst, row_bytes);
}

bool codec8_ok(int type, int n_el) {
    if (type == 8 || type == 2) return n_el % 32 == 0;
    return (type == 0 || type == 1 || type == 30) && n_el % 8 == 0;
}

// Q8_0 / Q4_0 rows that are whole 16-byte pieces at 16-byte aligned addresses
static bool ct_rows_ok(int type, const void * base, long long row_bytes, long long layer_bytes, int n_el) {
    return (type == 8 || type == 2) && n_el % 32 == 0 && row_bytes % 16 == 0 && layer_bytes % 16 == 0 &&
           (reinterpret_cast<uintptr_t>(base) & 15) == 0 && CT_ROWS * row_bytes <= 32768;
}

void launch_dequant8(const uint8_t * src, int type, long long row_bytes, long long src_ls, int n_el, int T, int L,
                     float * dst, hipStream_t st) {
    if (ct_rows_ok(type, src, row_bytes, src_ls, n_el) && (reinterpret_cast<uintptr_t>(dst) & 15) == 0) {
        if ((long long)L * T <= 0) return;
        const dim3 grid(cdiv(T, CT_ROWS), L);
        const size_t lds = (size_t)CT_ROWS * row_bytes;
        if (type == 8)
            hipLaunchKernelGGL(k_dequant_tile<8>, grid, dim3(CT_THREADS), lds, st, src, row_bytes, src_ls, n_el, T, L,
                               dst);
        else
            hipLaunchKernelGGL(k_dequant_tile<2>, grid, dim3(CT_THREADS), lds, st, src, row_bytes, src_ls, n_el, T, L,
                               dst);
        return;
    }
    // one work item per thread (measured: 5.1 TB/s against 4.0 with the
    // grid capped and a strided loop)
    const long long total = (long long)L * T * (n_el / 8);
    const long long blocks = std::min<long long>((total + 255) / 256, 1LL << 30);
    hipLaunchKernelGGL(k_dequant8, dim3((unsigned)std::max<long long>(blocks, 1)), dim3(256), 0, st,
                       src, type, row_bytes, src_ls, n_el, T, L, dst);
}

void launch_requant8(const float * src, long long src_ls, long long src_ld, const int * idx, long long idx_ls,
                     int mode, int H, int dv, int type, int n_el, int rows, int L, uint8_t * dst, long long row_bytes,
                     long long dst_ls, hipStream_t st, RowCodec sq) {
    const long long total = (long long)L * rows * (n_el / 8);
    if (total <= 0) return;
    // one wave per row where the encoded rows are whole 16-byte pieces
    auto a16 = [](const void * p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; };
    if ((type == 8 || type == 2) && n_el % 256 == 0 && row_bytes % 16 == 0 && dst_ls % 16 == 0 && a16(dst)) {
        int m = -1;
        if (mode == 0 && sq.base) {
            if (sq.type == type && sq.row_bytes % 16 == 0 && sq.layer_bytes % 16 == 0 && a16(sq.base)) m = 2;
        } else if (mode == 0) {
            if (a16(src) && src_ls % 4 == 0 && src_ld % 4 == 0) m = 0;
        } else if (a16(src) && dv % 16 == 0) {
            m = 1;
        }
        if (m == 2 && n_el <= RQ_CHUNK) {
            const int nb = n_el / 32 * (type == 8 ? 34 : 18);
            const int nrb = std::min(CT_THREADS, RC_LDS / nb);
            const dim3 grid((unsigned)((L * (long long)rows + nrb - 1) / nrb));
            if (type == 8)
                hipLaunchKernelGGL(k_recode_tile<8>, grid, dim3(CT_THREADS), 0, st, idx, idx_ls, n_el, rows, L, nrb,
                                   dst, row_bytes, dst_ls, sq);
            else
                hipLaunchKernelGGL(k_recode_tile<2>, grid, dim3(CT_THREADS), 0, st, idx, idx_ls, n_el, rows, L, nrb,
                                   dst, row_bytes, dst_ls, sq);
            return;
        }
        if (m >= 0) {
            const long long nrows = (long long)L * rows;
            // (one row a wave: measured faster than a grid of 2048 blocks whose
            // waves fetch each next row while they encode the current one)
            const dim3 grid((unsigned)std::min<long long>((nrows + RQ_WAVES - 1) / RQ_WAVES, 1LL << 20));
            const dim3 blk(64 * RQ_WAVES);
#define KVC_RQ(T_, M_)                                                                                           \
    hipLaunchKernelGGL((k_requant_rows<T_, M_>), grid, blk, 0, st, src, src_ls, src_ld, idx, idx_ls, H, dv, n_el, \
                       rows, L, dst, row_bytes, dst_ls, sq)
            if (type == 8) {
                if (m == 0) KVC_RQ(8, 0); else if (m == 1) KVC_RQ(8, 1); else KVC_RQ(8, 2);
            } else {
                if (m == 0) KVC_RQ(2, 0); else if (m == 1) KVC_RQ(2, 1); else KVC_RQ(2, 2);
            }
#undef KVC_RQ
            return;
        }
    }
    const long long blocks = std::min<long long>((total + 255) / 256, 1LL << 30);
    hipLaunchKernelGGL(k_requant8, dim3((unsigned)blocks), dim3(256), 0, st,
                       src, src_ls, src_ld, idx, idx_ls, mode, H, dv, type, n_el, rows, L, dst, row_bytes, dst_ls, sq);
}

void launch_transpose(const float * src, long long rows, long long cols, float * dst, hipStream_t st) {
    if (rows <= 0 || cols <= 0) return;
    hipLaunchKernelGGL(k_transpose, dim3(cdiv(cols, 32), cdiv(rows, 32)), dim3(256), 0, st, src, rows, cols, dst);
}

void launch_fold_rows(const float * K, int nk, const int * sel, int t, const float * beta, const float * dir, int H,
                      int dk, float scale, float * out, hipStream_t st) {
    if (t <= 0) return;
    hipLaunchKernelGGL(k_fold_rows, dim3(grid_cap((long long)t * nk, 256)), dim3(256), 0, st,
                       K, nk, sel, t, beta, dir, H, dk, scale, out);
}

void launch_value_columns(const float * Cv, const float * V, int nv, const int * sel, int H, int dv, int t,
                          float * col, hipStream_t st) {
    if (t <= 0) return;
    hipLaunchKernelGGL(k_value_columns, dim3(grid_cap((long long)H * dv * t, 256)), dim3(256), 0, st,
                       Cv, V, nv, sel, H, dv, t, col);
}

void launch_gather_qref(const float * K, long long ldK, int nk, int q0, int nq, int H, int dk, int L, float * out,
                        hipStream_t st) {
    if (L <= 0) return;
    hipLaunchKernelGGL(k_gather_qref, dim3(grid_cap((long long)H * nq * dk, 256), L), dim3(256), 0, st,
                       K, ldK, nk, q0, nq, H, dk, out);
}

void launch_iota(int * p, long long n, hipStream_t st) {
    if (n <= 0) return;
    hipLaunchKernelGGL(k_iota, dim3(cdiv(n, 256)), dim3(256), 0, st, p, n);
}

void launch_gather_cv_rows(const float * Cv, int H, int t, int dv, float * rows, hipStream_t st) {
    hipLaunchKernelGGL(k_gather_cv_rows, dim3(grid_cap((long long)t * H * dv, 256)), dim3(256), 0, st,
                       Cv, H, t, dv, rows);
}

void launch_gemm_abt(const float * A, long long lda, const float * B, long long ldb, float * C, long long ldc,
                     int m, int n, int k, float scale, long long sa, long long sb, long long sc, int batch,
                     hipStream_t st) {
    hipLaunchKernelGGL(k_gemm_abt, dim3(cdiv(n, 16), cdiv(m, 16), batch), dim3(256), 0, st,
                       A, lda, B, ldb, C, ldc, m, n, k, scale, sa, sb, sc);
}

void launch_gemm_ab(const float * A, long long lda, const float * B, long long ldb, float * C, long long ldc,
                    int m, int n, int k, long long sa, long long sb, long long sc, int batch, hipStream_t st) {
    hipLaunchKernelGGL(k_gemm_ab, dim3(cdiv(n, 16), cdiv(m, 16), batch), dim3(256), 0, st,
                       A, lda, B, ldb, C, ldc, m, n, k, sa, sb, sc);
}

}  // namespace kvc
