// Host-code checks of libkv-compact built with sanitizers (tests/sanitize/Makefile):
// the state-blob parser over every truncation and seeded byte mutations of a
// valid blob, the argument validation of the C entry points, the pure host
// helpers, and concurrent calls from several threads. On a machine without a
// GPU the device entry points return KV_COMPACT_E_DEVICE before any launch;
// the parser and validation paths run in full. Exit status 0: every check held
// (the sanitizers abort the process on their own findings).
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <thread>
#include <vector>

#include "../../include/kv-compact-api.h"
#include "../../include/kv-compact-device.h"
#include "../../include/kvc-state.h"

static int failures = 0;
#define CHECK(c)                                                        \
    do {                                                                \
        if (!(c)) {                                                     \
            fprintf(stderr, "check failed: %s (line %d)\n", #c, __LINE__); \
            failures++;                                                 \
        }                                                               \
    } while (0)

template <class T> static void put(std::vector<uint8_t> & b, T v) {
    const uint8_t * p = reinterpret_cast<const uint8_t *>(&v);
    b.insert(b.end(), p, p + sizeof(T));
}

// a valid blob: one stream, T cells, L layers of F16 K and transposed F16 V
static std::vector<uint8_t> make_blob(int T, int L, int nk, uint32_t n_pos, bool vtrans) {
    std::vector<uint8_t> b;
    put<uint32_t>(b, 1);
    put<uint32_t>(b, (uint32_t)T);
    for (int i = 0; i < T; i++) {
        put<int32_t>(b, i);
        put<uint32_t>(b, 1 + i % 2);
        if (n_pos > 1) { put<int32_t>(b, i % 7); put<int32_t>(b, i % 5); }
        for (int k = 0; k < 1 + i % 2; k++) put<int32_t>(b, k);
    }
    put<uint32_t>(b, vtrans ? 1 : 0);
    put<uint32_t>(b, (uint32_t)L);
    uint64_t x = 88172645463325252ull;
    auto half = [&]() { x ^= x << 13; x ^= x >> 7; x ^= x << 17; return (uint16_t)(0x3000 + (x & 0x0fff)); };
    for (int l = 0; l < L; l++) {
        put<int32_t>(b, KV_TYPE_F16);
        put<uint64_t>(b, (uint64_t)nk * 2);
        for (int i = 0; i < T * nk; i++) put<uint16_t>(b, half());
    }
    for (int l = 0; l < L; l++) {
        put<int32_t>(b, KV_TYPE_F16);
        if (vtrans) { put<uint32_t>(b, 2); put<uint32_t>(b, (uint32_t)nk); }
        else put<uint64_t>(b, (uint64_t)nk * 2);
        for (int i = 0; i < T * nk; i++) put<uint16_t>(b, half());
    }
    for (int i = 0; i < 9; i++) put<uint8_t>(b, (uint8_t)i);
    return b;
}

static void parser_checks() {
    for (int vt = 0; vt < 2; vt++)
        for (uint32_t n_pos : {1u, 4u}) {
            std::vector<uint8_t> blob = make_blob(24, 2, 64, n_pos, vt != 0);
            kvc_state_info info;
            CHECK(kvc_state_parse_info(blob.data(), blob.size(), n_pos, &info) == 0);
            CHECK(info.cell_count == 24 && info.n_layer == 2 && info.n_embd_k == 64 && info.n_embd_v == 64);
            CHECK(info.trailing_bytes == 9 && info.kv_bytes + 9 == blob.size());
            // every truncation: either a clean error or (for cuts inside the
            // trailing bytes) a parse with fewer trailing bytes
            for (size_t cut = 0; cut < blob.size(); cut++) {
                std::vector<uint8_t> part(blob.begin(), blob.begin() + cut);
                const int rc = kvc_state_parse_info(part.empty() ? nullptr : part.data(), cut, n_pos, &info);
                if (cut == 0) CHECK(rc == -1);
                else if (cut < blob.size() - 9) CHECK(rc == -2);
                else CHECK(rc == 0);
            }
            // seeded byte mutations: any outcome but a crash or a sanitizer report
            uint64_t x = 0x9E3779B97F4A7C15ull + vt + n_pos;
            for (int it = 0; it < 4000; it++) {
                std::vector<uint8_t> m = blob;
                for (int k = 0; k < 4; k++) {
                    x ^= x << 13; x ^= x >> 7; x ^= x << 17;
                    m[(size_t)(x % m.size())] = (uint8_t)(x >> 32);
                }
                (void)kvc_state_parse_info(m.data(), m.size(), n_pos, &info);
            }
        }
}

static void api_checks() {
    kv_compact_params p = kv_compact_params_default();
    CHECK(p.target_ratio == 0.5f && p.skip_beta == 1 && p.score_method == 1 && p.nnls_method == 1);
    kv_compact_result r;
    memset(&r, 0, sizeof(r));
    float K[64] = {0}, V[64] = {0};
    CHECK(kv_compact(nullptr, V, nullptr, 4, 0, 1, 16, 16, &p, &r) == -1);
    CHECK(kv_compact(K, V, nullptr, 0, 0, 1, 16, 16, &p, &r) == -2);
    CHECK(kv_compact(K, V, K, 4, 0, 1, 16, 16, &p, &r) == -2);
    kv_compact_result_free(&r);
    kv_compact_result_free(&r);
    kv_compact_result_free(nullptr);
    CHECK(kv_compact_multi_round(K, V, nullptr, 4, 0, 1, 16, 16, &p, 0, &r, nullptr) == -3);
    CHECK(kv_quant_row_elements(KV_TYPE_Q8_0, 34 * 4) == 128);
    CHECK(kv_quant_row_bytes(KV_TYPE_Q4_0, 128) == 72);
    CHECK(kv_quant_row_bytes(KV_TYPE_Q4_1, 128) == 80);
    int t = 0, nc = 0;
    CHECK(kvc_plan(100000, 32, 1, &p, &t, &nc) == 0);
    p.target_ratio = 0.2f;
    CHECK(kvc_plan(100000, 32, 1, &p, &t, &nc) == 0 && nc == 79 && t == 20000);
    kvc_state_params sp;
    memset(&sp, 0, sizeof(sp));
    void * out = nullptr;
    size_t n = 0;
    CHECK(kvc_state_compact(nullptr, 0, &sp, &out, &n, nullptr) == -1);
    CHECK(kvc_state_parse_info(nullptr, 0, 1, nullptr) == -1);
}

int main() {
    parser_checks();
    api_checks();
    // several threads through the parser and the validation paths at once
    std::vector<std::thread> th;
    for (int i = 0; i < 8; i++)
        th.emplace_back([i]() {
            std::vector<uint8_t> blob = make_blob(16 + i, 2, 32, 1, i & 1);
            kvc_state_info info;
            for (int k = 0; k < 50; k++) CHECK(kvc_state_parse_info(blob.data(), blob.size(), 1, &info) == 0);
            kv_compact_params p = kv_compact_params_default();
            kv_compact_result r;
            memset(&r, 0, sizeof(r));
            CHECK(kv_compact(nullptr, nullptr, nullptr, 1, 0, 1, 1, 1, &p, &r) == -1);
        });
    for (auto & x : th) x.join();
    if (failures) {
        fprintf(stderr, "%d checks failed\n", failures);
        return 1;
    }
    printf("host checks ok\n");
    return 0;
}
