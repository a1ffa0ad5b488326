// Host orchestrator of libkv-compact.so: the reference's C ABI
// (include/kv-compact-api.h, include/kv-compact-accel.h) plus the additive
// device-resident batch API (include/kv-compact-device.h), all running on
// the HIP kernels of kvc_kernels.hip. There is no CPU compute path: when no
// GPU is usable the calls return KV_COMPACT_E_DEVICE.
//
// Call flow (reference src/kv-compact-api.cpp:360-978):
//   validate -> params/defaults -> query source -> target count -> chunk
//   plan -> [device] scores, chunk softmax + importance, refit target Y,
//   global importance (+R-KV) and top-t, LS system + Gaussian elimination,
//   quality statistics -> results.
// Every layer of a batch and every chunk of a layer is independent, so one
// launch of each kernel covers all (layer, chunk, head) units.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <atomic>
#include <chrono>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <functional>
#include <mutex>
#include <thread>
#include <vector>

#include <sys/mman.h>

#include "../../include/kv-compact-api.h"
#include "../../include/kv-compact-accel.h"
#include "../../include/kv-compact-device.h"
#include "../../include/kvc-state.h"
#include "kvc_common.h"
#include "kvc_kernels.h"

using namespace kvc;

namespace {

// ------------------------------------------------------------------ device

// Pipeline stages timed with events on the call's stream (kvc_stage_times)
enum Stage { ST_SCORES, ST_SOFTMAX, ST_REFIT, ST_SELECT, ST_BETA, ST_LS_SOFTMAX, ST_LS_BUILD, ST_LU, ST_SOLVE,
             ST_REFINE, ST_STATS, ST_BATCH_END,
             // the quantized entries' codec phases, around the batch
             ST_DEQUANT = ST_BATCH_END, ST_REQUANT, ST_COUNT };

// Fixed workspace of kvc_compact_layers_device_noalloc, one copy per GPU
// (each device that loads the library holds it until the process ends). Host
// code never uses this name as an address: DeviceCtx::scratch holds the
// device address, taken once per device with hipGetSymbolAddress.
static __device__ __align__(256) unsigned char scratch[KVC_NOALLOC_SCRATCH_BYTES];

// Pinned host ring for transfers between pageable host memory and the
// device: kPinThreads host threads, each with two buffers of kPinBytes.
constexpr int kPinThreads = 4, kPinBufs = 2 * kPinThreads;
constexpr size_t kPinBytes = (size_t)8 << 20;

struct DeviceCtx {
    std::mutex mu;
    // the pinned ring (allocated on the first large host transfer, kept
    // until the process ends; pin_failed: plain copies instead)
    void * pin[kPinBufs] = {};
    hipEvent_t pin_ev[kPinBufs] = {};
    bool pin_used[kPinBufs] = {};
    bool pin_ready = false, pin_failed = false;
    bool ready = false;
    char * scratch = nullptr;   // device address of `scratch` on this device (null if unavailable)
    hipStream_t stream = nullptr;
    // second stream (default priority, like stream) for work that runs beside
    // the main chain: the refit target during the selection, and the
    // original-attention statistics during the normal equations and
    // factorizations
    hipStream_t stream2 = nullptr;
    hipEvent_t fork_ev = nullptr, join_ev = nullptr;
    hipEvent_t refit_fork = nullptr, refit_join = nullptr;
    // host-pointer calls: V uploads on its own stream while the kernels
    // that read only K run; v_ev marks its last transfer
    hipStream_t up_stream = nullptr;
    hipEvent_t v_ev = nullptr;
    hipEvent_t cv_ev = nullptr;   // C_v written (its download, on up_stream, waits for it)
    hipEvent_t refit_t[2] = {};   // timing of the refit target on the second stream
    char * arena = nullptr;
    size_t arena_cap = 0;
    hipEvent_t ev[ST_BATCH_END + 1] = {};
    hipEvent_t q_ev[4] = {};      // dequantization and requantization phases
    float stage_ms[ST_COUNT] = {};
};

constexpr int kMaxDevices = 64;
DeviceCtx g_dev[kMaxDevices];
std::mutex g_init_mu;

void exp2_table(uint64_t tab[32]) {
    // tab[i] = bits(2^(i/32) rounded to double) - (i << 47)
    for (int i = 0; i < 32; i++) {
        long double v = exp2l((long double)i / 32.0L);
        double d = (double)v;
        uint64_t b;
        memcpy(&b, &d, 8);
        tab[i] = b - ((uint64_t)i << 47);
    }
}

// HIP streams, events and pinned host buffers the library holds, over all
// devices (kvc_live_objects): every creation below counts one, every destroy
// takes one back, so a failure path that leaks shows up in the count.
std::atomic<int> g_live{0};

bool made(hipError_t e) {
    if (e != hipSuccess) {
        (void)hipGetLastError();
        return false;
    }
    g_live++;
    return true;
}

template <class H, class F> void drop(H & h, F destroy) {
    if (!h) return;
    (void)destroy(h);
    h = nullptr;
    g_live--;
}

// Destroys the streams and events of a context (a device_ctx set-up that
// failed part of the way, so the next call starts again from nothing).
void destroy_ctx_objects(DeviceCtx * c) {
    drop(c->stream, hipStreamDestroy);
    drop(c->stream2, hipStreamDestroy);
    drop(c->fork_ev, hipEventDestroy);
    drop(c->join_ev, hipEventDestroy);
    drop(c->refit_fork, hipEventDestroy);
    drop(c->refit_join, hipEventDestroy);
    drop(c->up_stream, hipStreamDestroy);
    drop(c->v_ev, hipEventDestroy);
    drop(c->cv_ev, hipEventDestroy);
    for (hipEvent_t & e : c->refit_t) drop(e, hipEventDestroy);
    for (hipEvent_t & e : c->ev) drop(e, hipEventDestroy);
    for (hipEvent_t & e : c->q_ev) drop(e, hipEventDestroy);
}

bool forced_fault(const char * kind);

bool create_ctx_objects(DeviceCtx * c) {
    uint64_t tab[32];
    exp2_table(tab);
    if (set_exp2_table(tab) != hipSuccess) {
        (void)hipGetLastError();
        return false;
    }
    if (!made(hipStreamCreateWithFlags(&c->stream, hipStreamNonBlocking)) ||
        !made(hipStreamCreateWithFlags(&c->stream2, hipStreamNonBlocking)) ||
        !made(hipEventCreateWithFlags(&c->fork_ev, hipEventDisableTiming)) ||
        !made(hipEventCreateWithFlags(&c->join_ev, hipEventDisableTiming)))
        return false;
    // (KVC_FAULT=init: the set-up fails here, with part of its objects made)
    if (forced_fault("init")) return false;
    if (!made(hipEventCreateWithFlags(&c->refit_fork, hipEventDisableTiming)) ||
        !made(hipEventCreateWithFlags(&c->refit_join, hipEventDisableTiming)) ||
        !made(hipStreamCreateWithFlags(&c->up_stream, hipStreamNonBlocking)) ||
        !made(hipEventCreateWithFlags(&c->v_ev, hipEventDisableTiming)) ||
        !made(hipEventCreateWithFlags(&c->cv_ev, hipEventDisableTiming)))
        return false;
    for (hipEvent_t & e : c->refit_t)
        if (!made(hipEventCreate(&e))) return false;
    for (hipEvent_t & e : c->ev)
        if (!made(hipEventCreate(&e))) return false;
    for (hipEvent_t & e : c->q_ev)
        if (!made(hipEventCreate(&e))) return false;
    return true;
}

// Returns the context of the current device, initialised, or nullptr (then
// nothing of a partial set-up is kept, and the next call tries again).
DeviceCtx * device_ctx() {
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || n <= 0) {
        (void)hipGetLastError();
        return nullptr;
    }
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return nullptr;
    DeviceCtx * c = &g_dev[dev];
    std::lock_guard<std::mutex> lk(g_init_mu);
    if (!c->ready) {
        if (!create_ctx_objects(c)) {
            destroy_ctx_objects(c);
            return nullptr;
        }
        void * sp = nullptr;
        if (hipGetSymbolAddress(&sp, HIP_SYMBOL(scratch)) == hipSuccess) {
            c->scratch = static_cast<char *>(sp);
        } else {
            (void)hipGetLastError();
            c->scratch = nullptr;
        }
        c->ready = true;
    }
    return c;
}

// Bump allocator over the device arena (256-byte aligned pieces).
struct Carver {
    size_t off = 0;
    char * base = nullptr;
    template <class T> T * take(size_t n) {
        off = (off + 255) & ~(size_t)255;
        T * p = base ? reinterpret_cast<T *>(base + off) : nullptr;
        off += n * sizeof(T);
        return p;
    }
};

// Work an earlier call left on the second stream (it ended early, after the
// refit target or the statistics were launched there) may still read or
// write the workspace: the call's stream waits for it before any workspace
// write.
bool drain_second_stream(DeviceCtx * ctx, hipStream_t st) {
    if (!ctx->stream2) return true;
    return hipEventRecord(ctx->refit_join, ctx->stream2) == hipSuccess &&
           hipStreamWaitEvent(st, ctx->refit_join, 0) == hipSuccess;
}

// Host-forced faults for tests of the error paths, read at every call:
// KVC_FAULT=alloc fails every workspace allocation (as a failing hipMalloc
// would, whether or not the arena must grow); KVC_FAULT=launch stops each
// compaction's kernel sequence before its first launch with a device error.
bool forced_fault(const char * kind) {
    const char * e = getenv("KVC_FAULT");
    if (!e || strcmp(e, kind) != 0) return false;
    fprintf(stderr, "[kv-compact] forced %s failure (KVC_FAULT=%s)\n", kind, kind);
    return true;
}

bool ensure_arena(DeviceCtx * c, size_t bytes) {
    if (forced_fault("alloc")) return false;
    if (c->arena_cap >= bytes) return true;
    if (c->arena) {
        (void)hipStreamSynchronize(c->stream);
        (void)hipStreamSynchronize(c->stream2);
        (void)hipFree(c->arena);
        c->arena = nullptr;
        c->arena_cap = 0;
    }
    size_t want = bytes + bytes / 8 + (1u << 20);
    if (hipMalloc(&c->arena, want) != hipSuccess) {
        (void)hipGetLastError();
        c->arena = nullptr;
        return false;
    }
    c->arena_cap = want;
    return true;
}

bool is_device_ptr(const void * p) {
    if (!p) return false;
    hipPointerAttribute_t a;
    if (hipPointerGetAttributes(&a, p) != hipSuccess) {
        (void)hipGetLastError();
        return false;
    }
    return a.type == hipMemoryTypeDevice;
}

// One contiguous piece of a transfer between host and device memory.
struct HostSeg {
    void * host;
    void * dev;
    size_t bytes;
};

// Frees the pinned ring's buffers and events (after any transfer still
// queued from them).
void free_pin_ring(DeviceCtx * c) {
    for (int b = 0; b < kPinBufs; b++)
        if (c->pin_used[b] && c->pin_ev[b]) (void)hipEventSynchronize(c->pin_ev[b]);
    for (int b = 0; b < kPinBufs; b++) {
        drop(c->pin[b], hipHostFree);
        drop(c->pin_ev[b], hipEventDestroy);
        c->pin_used[b] = false;
    }
    c->pin_ready = false;
}

// Allocates the ring once; on a failure frees what it made and marks the
// ring failed (plain copies until kvc_release_workspace clears the mark).
bool pin_ring(DeviceCtx * c) {
    if (c->pin_ready) return true;
    if (c->pin_failed) return false;
    for (int b = 0; b < kPinBufs; b++) {
        // (KVC_FAULT=pin: the ring fails after its first buffer)
        if ((b == 1 && forced_fault("pin")) || !made(hipHostMalloc(&c->pin[b], kPinBytes, hipHostMallocDefault)) ||
            !made(hipEventCreateWithFlags(&c->pin_ev[b], hipEventDisableTiming))) {
            free_pin_ring(c);
            c->pin_failed = true;
            return false;
        }
    }
    c->pin_ready = true;
    return true;
}

// Copies the segments between pageable host memory and device memory on st,
// through the pinned ring: thread i moves pieces i, i + kPinThreads, ... (at
// most pin_piece_bytes() each, in segment order) through its two buffers. Host to
// device: a piece is copied into a buffer once the transfer that last read
// it has finished, then its transfer is queued on st; the data is on the
// device once st reaches that point. Device to host (data produced on st):
// the transfer of a thread's next piece is queued before the previous one is
// copied out, and the call returns with every piece in host memory. Without
// the ring (or for a single piece) the segments take plain copies. Returns
// false on a HIP error.
// Piece size of the pinned transfers: kPinBytes, or KVC_PIN_BYTES (a test
// switch, read at every call: 4096 .. kPinBytes) to run the ring on small
// inputs.
size_t pin_piece_bytes() {
    const char * e = getenv("KVC_PIN_BYTES");
    if (!e) return kPinBytes;
    const long long v = atoll(e);
    return (v >= 4096 && v <= (long long)kPinBytes) ? (size_t)v : kPinBytes;
}

bool host_transfer(DeviceCtx * c, const std::vector<HostSeg> & segs, bool to_device, hipStream_t st) {
    const size_t piece = pin_piece_bytes();
    std::vector<HostSeg> pieces;
    for (const HostSeg & sg : segs) {
        if (sg.bytes > 0 && is_device_ptr(sg.host)) {
            // (a device buffer passed where host memory is expected: copied directly)
            const hipError_t e = to_device ? hipMemcpyAsync(sg.dev, sg.host, sg.bytes, hipMemcpyDefault, st)
                                           : hipMemcpyAsync(sg.host, sg.dev, sg.bytes, hipMemcpyDefault, st);
            if (e != hipSuccess) return false;
            continue;
        }
        for (size_t off = 0; off < sg.bytes; off += piece)
            pieces.push_back({static_cast<char *>(sg.host) + off, static_cast<char *>(sg.dev) + off,
                              std::min(piece, sg.bytes - off)});
    }
    if (pieces.size() < 2 || !pin_ring(c)) {
        for (const HostSeg & pc : pieces) {
            const hipError_t e = to_device
                ? hipMemcpyAsync(pc.dev, pc.host, pc.bytes, hipMemcpyHostToDevice, st)
                : hipMemcpyAsync(pc.host, pc.dev, pc.bytes, hipMemcpyDeviceToHost, st);
            if (e != hipSuccess) return false;
        }
        return to_device || hipStreamSynchronize(st) == hipSuccess;
    }
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return false;
    std::atomic<bool> ok{true};
    auto worker = [&](int i) {
        if (hipSetDevice(dev) != hipSuccess) { ok = false; return; }
        int prev = -1, pb = -1;   // device to host: piece waiting to be copied out, and its buffer
        int k = 0;
        for (size_t q = (size_t)i; q < pieces.size() && ok; q += kPinThreads, k++) {
            const int b = 2 * i + (k & 1);
            const HostSeg & pc = pieces[q];
            if (to_device) {
                if (c->pin_used[b] && hipEventSynchronize(c->pin_ev[b]) != hipSuccess) { ok = false; break; }
                memcpy(c->pin[b], pc.host, pc.bytes);
                if (hipMemcpyAsync(pc.dev, c->pin[b], pc.bytes, hipMemcpyHostToDevice, st) != hipSuccess ||
                    hipEventRecord(c->pin_ev[b], st) != hipSuccess) { ok = false; break; }
                c->pin_used[b] = true;
            } else {
                if (hipMemcpyAsync(c->pin[b], pc.dev, pc.bytes, hipMemcpyDeviceToHost, st) != hipSuccess ||
                    hipEventRecord(c->pin_ev[b], st) != hipSuccess) { ok = false; break; }
                c->pin_used[b] = true;
                if (prev >= 0) {
                    if (hipEventSynchronize(c->pin_ev[pb]) != hipSuccess) { ok = false; break; }
                    memcpy(pieces[prev].host, c->pin[pb], pieces[prev].bytes);
                }
                prev = (int)q;
                pb = b;
            }
        }
        if (!to_device && prev >= 0 && ok) {
            if (hipEventSynchronize(c->pin_ev[pb]) != hipSuccess) ok = false;
            else memcpy(pieces[prev].host, c->pin[pb], pieces[prev].bytes);
        }
    };
    // (a worker whose thread cannot be started runs on this one: each moves
    // only its own pieces through its own buffers)
    std::vector<std::thread> th;
    int started = 1;
    try {
        for (; started < kPinThreads; started++) th.emplace_back(worker, started);
    } catch (...) {
    }
    worker(0);
    for (int i = started; i < kPinThreads; i++) worker(i);
    for (std::thread & t : th) t.join();
    // (device to host: also any direct copies queued above)
    if (!to_device && ok && hipStreamSynchronize(st) != hipSuccess) ok = false;
    return ok;
}

double now_ms() {
    return std::chrono::duration<double, std::milli>(
               std::chrono::steady_clock::now().time_since_epoch()).count();
}

// -------------------------------------------------------------------- plan

// Reference api.cpp:382-390 (cheap query count)
int cheap_count(int T) {
    int n = T / 2;
    if (n > 64) n = 64;
    if (n < 4) n = 4;
    if (n > T) n = T;
    return n;
}

// Reference api.cpp:396-409 (tokens kept by one call)
int target_count(int T, const kv_compact_params & p) {
    int t;
    if (p.target_count > 0) {
        t = p.target_count < T ? p.target_count : T;
    } else {
        t = (int)(T * p.target_ratio);
        if (t < 1) t = 1;
        if (t > T) t = T;
    }
    if (p.n_shared_prefix > t) t = p.n_shared_prefix < T ? p.n_shared_prefix : T;
    return t;
}

// Reference api.cpp:417-437 (auto chunk size)
int chunk_size(int T, const kv_compact_params & p) {
    int cs = p.chunk_size;
    if (cs == 0) {
        float r = (p.target_count > 0) ? (float)p.target_count / (float)T : p.target_ratio;
        if (r <= 0.0f) r = 0.5f;
        if (r > 1.0f) r = 1.0f;
        int est = (int)(T * r);
        if (est > 256) {
            cs = (int)(256.0f / r);
            if (cs < 64) cs = 64;
            if (cs >= T) cs = T;
        } else {
            cs = T;
        }
    } else if (cs < 0) {
        cs = T;
    }
    return cs;
}

struct Plan {
    int T = 0, n_chunks = 0, t_total = 0, nq_max = 0, tc_max = 0, Tc_max = 0;
    int qmode = Q_PROVIDED, nq_global = 0, stats_qmode = Q_PROVIDED;
    std::vector<ChunkDesc> chunks;  // n_chunks, then the two statistics pseudo-chunks
};

// Chunk plan of one call; the per-chunk recursion of api.cpp:466-499 is
// unrolled here (chunk params: chunk_size -1, prefix only in chunk 0).
void make_plan(int T, int n_q, bool q_given, const kv_compact_params & p, Plan & pl) {
    pl.T = T;
    const bool cheap = p.use_cheap_qref || !q_given;
    const int nq_outer = cheap ? cheap_count(T) : n_q;
    pl.nq_global = nq_outer;
    pl.stats_qmode = q_given && !p.use_cheap_qref ? Q_PROVIDED : Q_CHEAP_GLOBAL;
    const int cs = chunk_size(T, p);
    pl.chunks.clear();
    if (cs < T) {
        pl.n_chunks = (T + cs - 1) / cs;
        // inside a chunk call Q_ref is non-NULL: it regenerates only when the flag is set
        pl.qmode = p.use_cheap_qref ? Q_CHEAP_LOCAL : (q_given ? Q_PROVIDED : Q_CHEAP_GLOBAL);
        int off = 0;
        for (int c = 0; c < pl.n_chunks; c++) {
            ChunkDesc d;
            d.start = c * cs;
            d.Tc = std::min(T, d.start + cs) - d.start;
            kv_compact_params cp = p;
            cp.n_shared_prefix = (c > 0) ? 0 : std::min(p.n_shared_prefix, d.Tc);
            d.tc = target_count(d.Tc, cp);
            d.prefix = cp.n_shared_prefix;
            d.nq = (pl.qmode == Q_CHEAP_LOCAL) ? cheap_count(d.Tc) : nq_outer;
            d.off = off;
            off += d.tc;
            pl.chunks.push_back(d);
        }
        pl.t_total = off;
    } else {
        pl.n_chunks = 1;
        pl.qmode = cheap ? Q_CHEAP_GLOBAL : Q_PROVIDED;
        ChunkDesc d;
        d.start = 0;
        d.Tc = T;
        d.tc = target_count(T, p);
        d.prefix = p.n_shared_prefix;
        d.nq = nq_outer;
        d.off = 0;
        pl.chunks.push_back(d);
        pl.t_total = d.tc;
    }
    pl.nq_max = 0;
    pl.tc_max = 0;
    pl.Tc_max = 0;
    for (const ChunkDesc & d : pl.chunks) {
        pl.nq_max = std::max(pl.nq_max, d.nq);
        pl.tc_max = std::max(pl.tc_max, d.tc);
        pl.Tc_max = std::max(pl.Tc_max, d.Tc);
    }
    // statistics pseudo-chunks: all T keys, then the t_total kept keys
    ChunkDesc whole;
    whole.start = 0;
    whole.Tc = T;
    whole.tc = pl.t_total;
    whole.prefix = 0;
    whole.off = 0;
    whole.nq = nq_outer;
    pl.chunks.push_back(whole);
    whole.Tc = pl.t_total;
    pl.chunks.push_back(whole);
}

// KVC_FUSED=1 (read at every call) runs the scoring, chunk softmax,
// importance and refit target as one kernel whose scores never leave the
// chip (k_score_attend), where the call allows it; same results. It is not
// the default: holding a chunk's scores in registers leaves one block per CU,
// and at that occupancy the kernel takes longer (about 14.9 ms at 100k
// tokens x 32 layers) than the separate kernels with their HBM round trip
// (scores 5.4 + softmax 2.0 ms, the refit target beside the selection).
bool fused_enabled() {
    const char * e = getenv("KVC_FUSED");
    return e && e[0] == '1';
}

// Options this library implements; everything else is refused with -5
// rather than computed differently.
int check_supported(const kv_compact_params & p, int d_v) {
    if (d_v > 256) return KV_COMPACT_E_UNSUPPORTED;
    return 0;
}

// ------------------------------------------------------------ batch run

struct BatchIO {
    const float * K;   // device (nullptr when kc.base is set)
    const float * V;   // device (nullptr when vc.base is set)
    RowCodec kc, vc;   // quantized K / V read in place (base nullptr: K / V above)
    const float * Q;   // device or null
    long long ldK, ldV, ldQ;
    int L, T, n_q, H, dk, dv;
    const float * wts; // device [T] or null
    int * indices;     // device outputs
    float * beta;
    float * Cv;
    float * stats;
};

struct Timing {
    double scoring_ms = 0.0, nnls_ms = 0.0;
};

// candidate capacity of the first diversity level: twice the kept count
int div_cap1(const Plan & pl) {
    int c = std::max(2 * pl.tc_max, 256);
    c = (c + 63) / 64 * 64;
    return std::max(1, std::min(std::min(c, pl.Tc_max), DIV_MAX_CAND));
}

size_t div_g_floats(const Plan & pl, int L) {
    const size_t units = (size_t)L * pl.n_chunks;
    const size_t c1 = div_cap1(pl), cm = std::min(pl.Tc_max, DIV_MAX_CAND);
    return std::max(units * c1 * c1, cm * cm);
}

// p == nullptr: statistics-only workspace (no exp scores, no diversity)
size_t workspace_bytes(const Plan & pl, const BatchIO & io, const kv_compact_params * p, Carver * cv_out, Work * w,
                       StatWork * sw, DivWork * dw = nullptr, size_t * div_floats = nullptr, OmpWork * ow = nullptr) {
    // OMP reads the exp scores and row sums even when beta is skipped (api.cpp:634-643)
    const bool omp = p && p->use_omp;
    const bool need_e = p && (!p->skip_beta || omp);
    const bool div = p && p->use_diversity && !omp;
    const bool sens = p && p->use_sensitivity;
    Carver cv = cv_out ? *cv_out : Carver();
    const size_t L = io.L, H = io.H, T = io.T, nqm = pl.nq_max, nc = pl.n_chunks;
    const size_t tt = pl.t_total, dv = io.dv;
    Work ww{};
    ww.S = cv.take<float>(L * H * nqm * T);
    ww.smax = cv.take<unsigned>(L * H * nqm * nc * (((size_t)pl.Tc_max + 127) / 128));
    ww.A = cv.take<float>(L * H * nqm * T);
    ww.E = need_e ? ww.A : nullptr;   // A keeps the unnormalised exponentials
    ww.rowsum = cv.take<float>(L * nc * H * nqm);
    ww.ainv = cv.take<float>(L * nc * H * nqm);
    ww.imp = cv.take<float>(L * H * T);
    ww.sens = sens ? cv.take<float>(L * nc * H) : nullptr;
    ww.amax = sens && p->score_method != 0 ? cv.take<float>(L * H * T) : nullptr;
    ww.gimp = cv.take<float>(L * T);
    ww.Y = cv.take<float>(L * nc * H * nqm * dv);
    ww.sel = nullptr;
    ww.X = cv.take<float>(L * H * nqm * tt);
    size_t aug_elems = 0;
    for (int c = 0; c < pl.n_chunks; c++) aug_elems += (size_t)pl.chunks[c].tc * (pl.chunks[c].tc + dv);
    ww.aug = cv.take<float>(L * H * aug_elems);
    ww.aug_off = cv.take<long long>(L * nc * H);
    ww.perm = cv.take<int>(L * nc * H * (size_t)pl.tc_max);
    // register-LU systems (t_c <= 256) exist unless every chunk keeps more
    int tc_min = pl.tc_max;
    for (int c = 0; c < pl.n_chunks; c++) tc_min = std::min(tc_min, pl.chunks[c].tc);
    const size_t ut_rows = tc_min <= 256 ? 256 : 0;
    ww.skip = cv.take<unsigned char>(L * nc * H * (size_t)pl.tc_max);
    // (one row of padding: the back substitution's U-row loads run up to 247
    // entries past a row's end, values it never uses)
    ww.LU = cv.take<float>(L * nc * H * ut_rows * ut_rows + (ut_rows ? 256 : 0));
    ww.Bt = cv.take<float>(L * nc * H * ut_rows * dv);
    // trailing matrices of the split register LU (systems of 129 .. 256 unknowns)
    const bool split = ut_rows && pl.tc_max > 128;
    ww.LU2 = split ? cv.take<float>(L * nc * H * 128 * 128) : nullptr;
    ww.map2 = split ? cv.take<int>(L * nc * H * 128) : nullptr;
    ww.gtmp = cv.take<float>(L * nc * H * (2 * (size_t)pl.tc_max + dv));
    ww.cand = cv.take<int>(L * nc * (size_t)pl.Tc_max);
    ww.flags = cv.take<unsigned char>(L * nc * (size_t)pl.Tc_max);
    ww.chunks = cv.take<ChunkDesc>(pl.chunks.size());
    ww.Qt = cv.take<float>(L * H * (size_t)io.dk * 32);
    ww.status = cv.take<int>(1);
    ww.refine_active = cv.take<int>(L * nc);
    ww.lu_redo = cv.take<int>(L * nc * H);
    if (omp) {
        const size_t units = L * nc, tm = pl.tc_max;
        OmpWork o{};
        o.ce = cv.take<float>(L * nqm * T);
        o.cs = cv.take<float>(units * nqm);
        o.corr = cv.take<float>(L * T);
        o.mask = cv.take<unsigned char>(L * T);
        o.order = cv.take<int>(L * tt);
        o.w = cv.take<float>(L * tt);
        o.prev_w = cv.take<float>(L * tt);
        o.G = cv.take<float>(units * tm * tm);
        o.Atb = cv.take<float>(units * tm);
        o.aug = cv.take<float>(units * tm * (tm + 1));
        o.vec = cv.take<float>(units * (4 * tm + 1 + nqm));
        o.k_choice = p->omp_k_choice;
        o.refit_interval = p->omp_refit_interval;
        o.pgd_iters = p->nnls_pgd_iters;
        if (ow) *ow = o;
    }
    if (div) {
        const size_t units = L * nc;
        DivWork d{};
        d.state = cv.take<int>(units);
        d.gslot = cv.take<int>(units);
        d.count = cv.take<int>(units);
        d.maxnc = cv.take<float>(units);
        const size_t gf = div_g_floats(pl, io.L);
        d.G = cv.take<float>(gf);
        if (dw) *dw = d;
        if (div_floats) *div_floats = gf;
    }
    StatWork s{};
    s.mh = std::min(io.H, 4);
    s.mq = std::min(pl.nq_global, 32);
    s.qmode = pl.stats_qmode;
    // the original scores reuse S when the statistics share the main query set
    s.OS = (p && pl.qmode == pl.stats_qmode) ? nullptr : cv.take<float>(L * s.mh * s.mq * T);
    s.CS = cv.take<float>(L * s.mh * s.mq * std::max<size_t>(tt, 1));
    s.OI = cv.take<float>(L * s.mh * s.mq);
    s.CI = cv.take<float>(L * s.mh * s.mq);
    s.OO = cv.take<float>(L * s.mh * s.mq * dv);
    s.CO = cv.take<float>(L * s.mh * s.mq * dv);
    if (w) *w = ww;
    if (sw) *sw = s;
    if (cv_out) *cv_out = cv;
    return cv.off + 256;
}

// Diversity selection by levels of candidate pruning (each exact; a unit
// whose pruned greedy pass cannot certify its picks moves to the next,
// wider level): alpha = max(0.85, safe), then the safe bound
// (1 - 1.001 s)(1 - 1e-5), then every unused key.
int run_diversity(hipStream_t st, const Plan & pl, const kv_compact_params & p, const Geom & g, const Work & w,
                  DivWork dw, size_t g_floats, const float * K) {
    const int units = g.L * pl.n_chunks;
    const float s = p.diversity_strength;
    float safe = 0.0f;
    if (s >= 0.0f && s < 1.0f) safe = std::max(0.0f, (1.0f - 1.001f * s) * (1.0f - 1e-5f));
    struct Level { float alpha; int cap; };
    std::vector<Level> levels;
    const int cmax = std::min(pl.Tc_max, DIV_MAX_CAND);
    if (safe > 0.0f) {
        const float a1 = std::max(0.85f, safe);
        levels.push_back({a1, div_cap1(pl)});
        if (safe < a1) levels.push_back({safe, cmax});
    }
    levels.push_back({0.0f, cmax});
    dw.strength = s;
    std::vector<int> state(units, DIV_RETRY), slot(units, -1), got(units);
    for (const Level & lv : levels) {
        std::vector<int> todo;
        for (int u = 0; u < units; u++)
            if (state[u] == DIV_RETRY) todo.push_back(u);
        if (todo.empty()) break;
        const size_t per = std::max<size_t>(1, g_floats / ((size_t)lv.cap * lv.cap));
        dw.alpha = lv.alpha;
        dw.cap = lv.cap;
        for (size_t b0 = 0; b0 < todo.size(); b0 += per) {
            const size_t b1 = std::min(todo.size(), b0 + per);
            std::fill(slot.begin(), slot.end(), -1);
            for (size_t k = b0; k < b1; k++) slot[todo[k]] = (int)(k - b0);
            if (hipMemcpyAsync(dw.gslot, slot.data(), (size_t)units * sizeof(int), hipMemcpyHostToDevice, st) !=
                hipSuccess)
                return KV_COMPACT_E_DEVICE;
            launch_div_level(g, w, dw, K, st);
            if (hipMemcpyAsync(got.data(), dw.state, (size_t)units * sizeof(int), hipMemcpyDeviceToHost, st) !=
                    hipSuccess ||
                hipStreamSynchronize(st) != hipSuccess)
                return KV_COMPACT_E_DEVICE;
            for (size_t k = b0; k < b1; k++) state[todo[k]] = got[todo[k]];
        }
    }
    for (int u = 0; u < units; u++)
        if (state[u] != DIV_DONE) return KV_COMPACT_E_UNSUPPORTED;   // greedy stopped early or > DIV_MAX_CAND keys
    return 0;
}

// v_ready (host-pointer calls): V may still be arriving. It is called once,
// before the first kernel that reads V is queued, and returns once st waits
// for V (0) or an error code; the refit target then runs on st after the
// kernels that read only K, which overlap the upload of V.
// cv_done (host-pointer calls): called once C_v's last writer is queued on
// st (before the statistics), so that its download can start beside them.
int run_batch(DeviceCtx * ctx, hipStream_t st, const Plan & pl, const kv_compact_params & p,
              const BatchIO & io, Carver & carver, Timing * tm,
              const std::function<int()> & v_ready = std::function<int()>(),
              const std::function<void()> & cv_done = std::function<void()>()) {
    // the chunk softmax keeps each row's maximum and scale in LDS, OMP its residuals
    if (pl.nq_max > SOFTMAX_MAXQ || (p.use_omp && pl.nq_max > OMP_MAXQ)) return KV_COMPACT_E_UNSUPPORTED;
    // Lawson-Hanson keeps a system's passive set on one wave: refused before
    // anything is launched
    if (!p.skip_beta && p.nnls_method == 0 && pl.tc_max > 256) return KV_COMPACT_E_UNSUPPORTED;
    // the beta fit's PGD steps keep their vectors in LDS
    const bool pgd = !p.skip_beta && p.nnls_method != 0 && p.nnls_pgd_iters > 0;
    if (pgd && 3 * pl.tc_max + pl.nq_max > PGD_LDS_FLOATS) return KV_COMPACT_E_UNSUPPORTED;
    if (forced_fault("launch")) return KV_COMPACT_E_DEVICE;
    if (!drain_second_stream(ctx, st)) return KV_COMPACT_E_DEVICE;
    Work w{};
    StatWork sw{};
    DivWork dw{};
    OmpWork ow{};
    size_t div_floats = 0;
    workspace_bytes(pl, io, &p, &carver, &w, &sw, &dw, &div_floats, &ow);
    w.sel = io.indices;
    w.wts = const_cast<float *>(io.wts);
    (void)ctx;

    Geom g{};
    g.L = io.L; g.T = io.T; g.H = io.H; g.dk = io.dk; g.dv = io.dv;
    g.n_chunks = pl.n_chunks; g.t_total = pl.t_total; g.nq_max = pl.nq_max;
    g.tc_max = pl.tc_max; g.Tc_max = pl.Tc_max;
    g.qmode = pl.qmode; g.nq_global = pl.nq_global;
    g.ldK = io.ldK; g.ldV = io.ldV; g.ldQ = io.ldQ;
    g.kc = io.kc; g.vc = io.vc;
    g.score_method = p.score_method;
    g.inv_sqrt_dk = 1.0f / sqrtf((float)io.dk);
    g.ridge = p.ridge;
    {
        const char * e = getenv("KVC_LU_MASKED");
        g.lu_masked = (e && e[0] == '1') ? 1 : 0;
    }

    // aug offsets: [L][n_chunks][H]
    std::vector<long long> aug_off((size_t)io.L * pl.n_chunks * io.H);
    {
        long long o = 0;
        for (int l = 0; l < io.L; l++)
            for (int c = 0; c < pl.n_chunks; c++)
                for (int h = 0; h < io.H; h++) {
                    aug_off[((size_t)l * pl.n_chunks + c) * io.H + h] = o;
                    o += (long long)pl.chunks[c].tc * (pl.chunks[c].tc + io.dv);
                }
    }
    if (hipMemcpyAsync(w.chunks, pl.chunks.data(), pl.chunks.size() * sizeof(ChunkDesc),
                       hipMemcpyHostToDevice, st) != hipSuccess) return KV_COMPACT_E_DEVICE;
    if (hipMemcpyAsync(w.aug_off, aug_off.data(), aug_off.size() * sizeof(long long),
                       hipMemcpyHostToDevice, st) != hipSuccess) return KV_COMPACT_E_DEVICE;

    launch_fill_int(w.status, 0, 1, st);
    hipEvent_t * ev = ctx->ev;
    (void)hipEventRecord(ev[0], st);
    // Scoring, chunk softmax, importance and the refit target in one kernel
    // whose scores never leave the chip, where the call allows it (the
    // options that read the scores or weights again later keep them in HBM)
    const bool fused = p.skip_beta && !p.use_omp && !p.use_sensitivity && p.refine_rounds <= 0 && fused_enabled() &&
                       !v_ready &&
                       score_attend_ok(g, io.K, io.V, io.Q, pl.Tc_max, pl.nq_max, pl.qmode);
    if (fused) {
        // the statistics' original scores are rows of S (heads < 4) when they
        // share the main query set
        launch_score_attend(g, w, io.K, io.V, io.Q, pl.qmode == pl.stats_qmode ? w.S : nullptr,
                            std::min(io.H, 4), st);
        (void)hipEventRecord(ev[ST_SCORES + 1], st);
        (void)hipEventRecord(ev[ST_SOFTMAX + 1], st);
    } else {
        // 1. scores for every (layer, chunk, head)
        launch_scores(g, w.chunks, pl.n_chunks, pl.Tc_max, io.K, io.Q, w.S, io.H, pl.nq_max,
                      (long long)io.H * pl.nq_max * io.T, (long long)pl.nq_max * io.T, io.T, pl.qmode, st,
                      nullptr, nullptr, w.smax);
        (void)hipEventRecord(ev[ST_SCORES + 1], st);
        // 2. chunk softmax + per-head importance
        launch_chunk_softmax(g, w, st);
        (void)hipEventRecord(ev[ST_SOFTMAX + 1], st);
    }
    // 3. refit target Y = A V. Only the normal equations read Y, so it runs
    //    on the second stream beside the selection (whose greedy pass is one
    //    short serial chain per unit and leaves the chip mostly idle).
    const bool late_v = static_cast<bool>(v_ready);
    const bool refit_fork = !fused && !late_v && ctx->stream2 != nullptr;
    if (fused || late_v) {
    } else if (refit_fork) {
        if (hipEventRecord(ctx->refit_fork, st) != hipSuccess ||
            hipStreamWaitEvent(ctx->stream2, ctx->refit_fork, 0) != hipSuccess) return KV_COMPACT_E_DEVICE;
        (void)hipEventRecord(ctx->refit_t[0], ctx->stream2);
        launch_refit_target(g, w, io.V, ctx->stream2);
        (void)hipEventRecord(ctx->refit_t[1], ctx->stream2);
        if (hipEventRecord(ctx->refit_join, ctx->stream2) != hipSuccess) return KV_COMPACT_E_DEVICE;
    } else {
        launch_refit_target(g, w, io.V, st);
    }
    (void)hipEventRecord(ev[ST_REFIT + 1], st);
    // 4. global importance (+R-KV), then OMP, the diversity greedy pass or top-t
    //    (api.cpp:686-716)
    launch_global_importance(g, w, st);
    if (p.use_omp) {
        launch_omp_select(g, w, ow, st);
    } else if (p.use_diversity) {
        const int rc = run_diversity(st, pl, p, g, w, dw, div_floats, io.K);
        if (rc) return rc;
    } else {
        launch_select_topk(g, w, st);
    }
    (void)hipEventRecord(ev[ST_SELECT + 1], st);
    // 5. beta: zeros (skip_beta), or the NNLS mass fit on the exp scores
    //    (api.cpp:812-831): M = exp_scores[:, sel], b = row sums
    auto fit_beta = [&]() -> int {
        if (p.skip_beta) {
            launch_fill_f32(io.beta, 0.0f, (long long)io.L * io.H * pl.t_total, st);
            return 0;
        }
        launch_gather_exp(g, w, st);   // M into the X buffer
        Geom gb = g;
        gb.dv = 1;
        gb.zero_val = 1e-12f;
        Work wb = w;
        wb.Y = w.rowsum;
        if (p.nnls_method == 0) {
            gb.ridge = 0.0f;   // Lawson-Hanson adds its own 1e-10 to each sub-problem
            launch_ls_build(gb, wb, st);
            launch_nnls_lh(gb, wb, io.beta, p.nnls_max_iter, w.status, st);
        } else {
            gb.ridge = 1e-10f;   // clamped unconstrained LS, math.h:707-745
            launch_ls_build(gb, wb, st, true);
            launch_ge_lu(gb, wb, st, true);
            launch_ge_solve(gb, wb, io.beta, st);
            if (pgd) {
                // projected-gradient steps (math.h:752-805) on [AtA | Atb] without the ridge
                gb.ridge = 0.0f;
                launch_ls_build(gb, wb, st);
                launch_nnls_pgd(gb, wb, io.beta, p.nnls_pgd_iters, st);
            }
        }
        launch_beta_log(io.beta, (long long)io.L * io.H * pl.t_total, st);
        return 0;
    };
    int rc = fit_beta();
    if (rc) return rc;
    (void)hipEventRecord(ev[ST_BETA + 1], st);
    // 6. X = softmax(S[:, sel] + beta); without S in HBM, the kept keys'
    //    scores are computed again (the same sums) into the A buffer
    if (fused) {
        launch_scores(g, w.chunks + pl.n_chunks + 1, 1, pl.t_total, io.K, io.Q, w.A, io.H, pl.nq_max,
                      (long long)io.H * pl.nq_max * pl.t_total, (long long)pl.nq_max * pl.t_total, pl.t_total,
                      pl.qmode, st, w.sel, nullptr);
        launch_ls_softmax(g, w, io.beta, st, w.A);
    } else {
        launch_ls_softmax(g, w, io.beta, st);
    }
    (void)hipEventRecord(ev[ST_LS_SOFTMAX + 1], st);
    // V still arriving: the factorizations, which form their matrices from X
    // alone (every system's at most 256 x 256, from at most 1024 rows of X),
    // run before the wait too; the normal equations then write B only
    const bool lu_first = late_v && pl.tc_max <= 256 && pl.nq_max <= 1024;
    if (lu_first) launch_ge_lu(g, w, st, true);
    if (late_v) {
        rc = v_ready();
        if (rc) return rc;
        launch_refit_target(g, w, io.V, st);
    }
    // The original-attention statistics read S and V only and rewrite the rows
    // of S they use; without refinement rounds the main path reads S no more,
    // so they run from here on the second stream, beside the normal
    // equations, factorizations and substitutions.
    float * s_main = pl.qmode == pl.stats_qmode ? w.S : nullptr;
    const bool fork = p.refine_rounds <= 0 && ctx->stream2;
    if (fork) {
        if (hipEventRecord(ctx->fork_ev, st) != hipSuccess ||
            hipStreamWaitEvent(ctx->stream2, ctx->fork_ev, 0) != hipSuccess) return KV_COMPACT_E_DEVICE;
        launch_stats_original(g, w, sw, io.K, io.V, io.Q, ctx->stream2, s_main, true);
        if (hipEventRecord(ctx->join_ev, ctx->stream2) != hipSuccess) return KV_COMPACT_E_DEVICE;
    }
    // 7. normal equations and their solution
    if (refit_fork && hipStreamWaitEvent(st, ctx->refit_join, 0) != hipSuccess) return KV_COMPACT_E_DEVICE;
    launch_ls_build(g, w, st, true);
    (void)hipEventRecord(ev[ST_LS_BUILD + 1], st);
    if (!lu_first) launch_ge_lu(g, w, st, true);
    (void)hipEventRecord(ev[ST_LU + 1], st);
    launch_ge_solve(g, w, io.Cv, st);
    (void)hipEventRecord(ev[ST_SOLVE + 1], st);
    // refinement rounds (api.cpp:851-946): swap the worst kept key for the
    // best unused one, then refit beta and C_v (units that stopped refit to
    // the same values)
    if (p.refine_rounds > 0) {
        launch_fill_int(w.refine_active, 1, (long long)io.L * pl.n_chunks, st);
        for (int r = 0; r < p.refine_rounds; r++) {
            launch_refine_step(g, w, st);
            rc = fit_beta();
            if (rc) return rc;
            launch_ls_softmax(g, w, io.beta, st);
            launch_ls_build(g, w, st, true);
            launch_ge_lu(g, w, st, true);
            launch_ge_solve(g, w, io.Cv, st);
        }
    }
    (void)hipEventRecord(ev[ST_REFINE + 1], st);
    if (cv_done) cv_done();
    // 8. quality statistics against the full call
    // the statistics' original scores are rows of S when both use one query set
    if (!fork) launch_stats_original(g, w, sw, io.K, io.V, io.Q, st, s_main);
    launch_stats_compacted(g, w, sw, io.K, io.V, io.Q, io.beta, io.Cv, io.stats, st);
    if (fork && hipStreamWaitEvent(st, ctx->join_ev, 0) != hipSuccess) return KV_COMPACT_E_DEVICE;
    launch_stats_final(g, sw, io.stats, st);
    (void)hipEventRecord(ev[ST_STATS + 1], st);

    hipError_t err = hipGetLastError();
    if (err == hipSuccess) err = hipStreamSynchronize(st);
    if (err != hipSuccess) {
        fprintf(stderr, "[kv-compact] HIP error: %s\n", hipGetErrorString(err));
        return KV_COMPACT_E_DEVICE;
    }
    int status = 0;
    if (hipMemcpy(&status, w.status, sizeof(int), hipMemcpyDeviceToHost) != hipSuccess) return KV_COMPACT_E_DEVICE;
    if (status & 2) {
        fprintf(stderr, "[kv-compact] LU step wait exceeded its bound\n");
        return KV_COMPACT_E_DEVICE;
    }
    if (status & 4) fprintf(stderr, "[kv-compact] OMP selection found no pickable key (non-finite correlations)\n");
    if (status) return KV_COMPACT_E_UNSUPPORTED;
    for (int i = 0; i < ST_BATCH_END; i++) {
        float ms = 0.0f;
        (void)hipEventElapsedTime(&ms, ev[i], ev[i + 1]);
        ctx->stage_ms[i] = ms;
    }
    ctx->stage_ms[ST_DEQUANT] = ctx->stage_ms[ST_REQUANT] = 0.0f;
    // (the fused kernel's time is the scores stage's; the two stages it
    // absorbs read 0)
    if (fused) ctx->stage_ms[ST_SOFTMAX] = ctx->stage_ms[ST_REFIT] = 0.0f;
    if (refit_fork) {
        // the refit target's own time on the second stream (it overlaps the selection)
        float ms = 0.0f;
        (void)hipEventElapsedTime(&ms, ctx->refit_t[0], ctx->refit_t[1]);
        ctx->stage_ms[ST_REFIT] = ms;
    }
    if (tm) {
        tm->scoring_ms = ctx->stage_ms[ST_SCORES] + ctx->stage_ms[ST_SOFTMAX] + ctx->stage_ms[ST_SELECT];
        tm->nnls_ms = ctx->stage_ms[ST_REFIT] + ctx->stage_ms[ST_BETA] + ctx->stage_ms[ST_LS_SOFTMAX] +
                      ctx->stage_ms[ST_LS_BUILD] +
                      ctx->stage_ms[ST_LU] + ctx->stage_ms[ST_SOLVE] + ctx->stage_ms[ST_REFINE];
    }
    return 0;
}

// Host-evaluated R-KV weights (api.cpp:668-684) for positions [0, T)
bool rkv_weights(const kv_compact_params & p, int T, std::vector<float> & w) {
    if (!p.reasoning || !p.reasoning->classifier) return false;
    const kv_compact_reasoning * r = p.reasoning;
    w.resize(T);
    for (int j = 0; j < T; j++) {
        int ty = r->classifier(j + r->token_offset, r->classifier_data);
        float x = 1.0f;
        if (ty == KV_TOKEN_THINKING) x = r->thinking_weight;
        else if (ty == KV_TOKEN_TRANSITION) x = r->transition_weight;
        w[j] = x;
    }
    return true;
}

int validate(const float * K, const float * V, const void * res, int T, int n_q, int H, int dk, int dv,
             const float * Q, const kv_compact_params & p) {
    if (!K || !V || !res) return -1;
    if (T <= 0 || H <= 0 || dk <= 0 || dv <= 0) return -2;
    if (!(p.use_cheap_qref || !Q) && n_q <= 0) return -2;
    return 0;
}

// Host memory for a result array, freeable with free(): arrays of 4 MB or
// more are aligned to 2 MB and advised for transparent huge pages, so that
// first-touch faults (and the caller's later free) come per 2 MB rather than
// per 4 KB page; smaller ones come from malloc.
void * host_alloc(size_t bytes) {
    constexpr size_t kHuge = (size_t)2 << 20;
    if (bytes < 2 * kHuge) return malloc(bytes);
    void * p = nullptr;
    if (posix_memalign(&p, kHuge, bytes) != 0) return nullptr;
    (void)madvise(p, (bytes + kHuge - 1) & ~(kHuge - 1), MADV_HUGEPAGE);
    return p;
}

// Device-resident outputs of one layer copied into a malloc'd host result.
// The result's arrays (reference ownership: malloc'd, freed by
// kv_compact_result_free), contents not yet set. False (and nothing left
// allocated) when an allocation fails.
bool alloc_result(kv_compact_result * r, int t, int H, int dv) {
    r->t = t;
    r->n_head_kv = H;
    r->selected_indices = (int *)host_alloc((size_t)std::max(t, 1) * sizeof(int));
    r->beta = (float **)calloc((size_t)std::max(H, 1), sizeof(float *));
    r->C_v = (float **)calloc((size_t)std::max(H, 1), sizeof(float *));
    bool ok = r->selected_indices && r->beta && r->C_v;
    for (int h = 0; ok && h < H; h++) {
        r->beta[h] = (float *)host_alloc((size_t)std::max(t, 1) * sizeof(float));
        r->C_v[h] = (float *)host_alloc((size_t)std::max(t, 1) * dv * sizeof(float));
        ok = r->beta[h] && r->C_v[h];
    }
    if (!ok) {
        fprintf(stderr, "[kv-compact] host allocation of the result failed\n");
        if (!r->beta || !r->C_v) r->n_head_kv = 0;   // (entries freed only when both arrays exist)
        kv_compact_result_free(r);
    }
    return ok;
}

// Writes one byte of every page of some host arrays on helper threads, so
// that the pages are mapped (and zeroed by the kernel) while the device
// works rather than during the result download. The array contents are set
// afterwards; join() before anything else writes them.
class PageToucher {
public:
    void add(void * p, size_t bytes) {
        if (p && bytes) regions_.push_back({static_cast<char *>(p), bytes});
    }
    void start(int n_threads) {
        for (int i = 0; i < n_threads; i++) {
            try {
                th_.emplace_back([this, i, n_threads] { touch(i, n_threads); });
            } catch (...) {
                touch(i, n_threads);   // (a thread that cannot start: its share runs here)
            }
        }
    }
    void join() {
        for (std::thread & t : th_) t.join();
        th_.clear();
    }
    ~PageToucher() { join(); }

private:
    static constexpr size_t kPage = 4096;
    // thread i of n: the i-th contiguous part of each array (parts of whole
    // 2 MB units, so no two threads fault the same huge page)
    void touch(int i, int n) {
        constexpr size_t kUnit = (size_t)2 << 20;
        for (const auto & r : regions_) {
            const size_t units = (r.second + kUnit - 1) / kUnit;
            const size_t lo = std::min(r.second, units * i / n * kUnit);
            const size_t hi = std::min(r.second, units * (i + 1) / n * kUnit);
            for (size_t o = lo; o < hi; o += kPage) reinterpret_cast<volatile char *>(r.first)[o] = 0;
        }
    }
    std::vector<std::pair<char *, size_t>> regions_;
    std::vector<std::thread> th_;
};

bool fill_result(kv_compact_result * r, int t, int H, int dv, const std::vector<int> & idx,
                 const std::vector<float> & beta, const std::vector<float> & cv) {
    if (!alloc_result(r, t, H, dv)) return false;
    memcpy(r->selected_indices, idx.data(), (size_t)t * sizeof(int));
    for (int h = 0; h < H; h++) {
        memcpy(r->beta[h], beta.data() + (size_t)h * t, (size_t)t * sizeof(float));
        memcpy(r->C_v[h], cv.data() + (size_t)h * t * dv, (size_t)t * dv * sizeof(float));
    }
    return true;
}

// One layer with host or device inputs; results to host (kv_compact()).
// Host inputs: K is uploaded first; V then uploads on a second stream,
// driven by a helper thread, while the kernels that read only K run
// (scores, softmax, selection, the compacted softmax), and the kernels that
// read V wait for its last transfer. The result arrays are allocated at the
// start and their pages mapped by helper threads meanwhile, so C_v comes
// back through the pinned ring into memory that is already present.
int compact_one(const float * K, const float * V, const float * Q, int T, int n_q, int H, int dk, int dv,
                const kv_compact_params & p, kv_compact_result * res) {
    const double t0 = now_ms();
    DeviceCtx * ctx = device_ctx();
    if (!ctx) return KV_COMPACT_E_DEVICE;
    std::lock_guard<std::mutex> lk(ctx->mu);
    hipStream_t st = ctx->stream;
    if (!drain_second_stream(ctx, st)) return KV_COMPACT_E_DEVICE;
    Plan pl;
    const bool q_given = Q != nullptr;
    make_plan(T, n_q, q_given, p, pl);
    const long long ek = (long long)H * dk, ev = (long long)H * dv;
    const bool kd = is_device_ptr(K), vd = is_device_ptr(V), qd = q_given && is_device_ptr(Q);
    const bool use_q = q_given && !p.use_cheap_qref;
    std::vector<float> wts;
    const bool have_w = rkv_weights(p, T, wts);

    BatchIO io{};
    io.L = 1; io.T = T; io.n_q = n_q; io.H = H; io.dk = dk; io.dv = dv;
    io.ldK = (long long)T * ek; io.ldV = (long long)T * ev; io.ldQ = (long long)std::max(n_q, 1) * ek;

    // size the arena: inputs + outputs + workspace
    Carver sizer;
    float * dK = kd ? nullptr : sizer.take<float>((size_t)T * ek);
    float * dV = vd ? nullptr : sizer.take<float>((size_t)T * ev);
    float * dQ = (use_q && !qd) ? sizer.take<float>((size_t)n_q * ek) : nullptr;
    float * dW = have_w ? sizer.take<float>(T) : nullptr;
    int * dI = sizer.take<int>(std::max(pl.t_total, 1));
    float * dB = sizer.take<float>((size_t)H * std::max(pl.t_total, 1));
    float * dC = sizer.take<float>((size_t)H * std::max(pl.t_total, 1) * dv);
    float * dS = sizer.take<float>(3);
    (void)dK; (void)dV; (void)dQ; (void)dW; (void)dI; (void)dB; (void)dC; (void)dS;
    size_t need = workspace_bytes(pl, io, &p, &sizer, nullptr, nullptr);
    if (!ensure_arena(ctx, need)) return KV_COMPACT_E_DEVICE;

    // the result (freed again on every failure below), its pages mapped by
    // helper threads while the device works
    const int t = pl.t_total;
    if (!alloc_result(res, t, H, dv)) return KV_COMPACT_E_DEVICE;
    struct FreeOnFail {
        kv_compact_result * r;
        bool armed = true;
        ~FreeOnFail() { if (armed) kv_compact_result_free(r); }
    } guard{res};
    PageToucher touch;
    for (int h = 0; h < H; h++) {
        touch.add(res->C_v[h], (size_t)t * dv * sizeof(float));
        touch.add(res->beta[h], (size_t)t * sizeof(float));
    }
    touch.add(res->selected_indices, (size_t)t * sizeof(int));
    touch.start(4);

    Carver cv;
    cv.base = ctx->arena;
    float * K_dev = kd ? const_cast<float *>(K) : cv.take<float>((size_t)T * ek);
    float * V_dev = vd ? const_cast<float *>(V) : cv.take<float>((size_t)T * ev);
    float * Q_dev = nullptr;
    if (use_q) Q_dev = qd ? const_cast<float *>(Q) : cv.take<float>((size_t)n_q * ek);
    float * W_dev = have_w ? cv.take<float>(T) : nullptr;
    io.indices = cv.take<int>(std::max(pl.t_total, 1));
    io.beta = cv.take<float>((size_t)H * std::max(pl.t_total, 1));
    io.Cv = cv.take<float>((size_t)H * std::max(pl.t_total, 1) * dv);
    io.stats = cv.take<float>(3);
    // the small inputs directly, K through the pinned ring on the call's stream
    hipError_t e = hipSuccess;
    if (use_q && !qd) e = hipMemcpyAsync(Q_dev, Q, (size_t)n_q * ek * sizeof(float), hipMemcpyHostToDevice, st);
    if (e == hipSuccess && have_w) e = hipMemcpyAsync(W_dev, wts.data(), (size_t)T * sizeof(float), hipMemcpyHostToDevice, st);
    if (e != hipSuccess) return KV_COMPACT_E_DEVICE;
    if (!kd && !host_transfer(ctx, {{const_cast<float *>(K), K_dev, (size_t)T * ek * sizeof(float)}}, true, st))
        return KV_COMPACT_E_DEVICE;
    io.K = K_dev; io.V = V_dev; io.Q = Q_dev; io.wts = W_dev;

    // V on the upload stream from a helper thread (the ring is idle again:
    // host_transfer has queued every piece of K), unless it is on the device
    // or the fused scoring kernel (which reads V with K) is asked for
    std::thread v_thread;
    std::atomic<int> v_state{vd ? 1 : 0};   // 0 queued in progress, 1 done, -1 failed
    std::function<int()> v_ready;
    if (!vd && fused_enabled()) {
        if (!host_transfer(ctx, {{const_cast<float *>(V), V_dev, (size_t)T * ev * sizeof(float)}}, true, st))
            return KV_COMPACT_E_DEVICE;
        v_state = 1;
    } else if (!vd) {
        int dev = 0;
        if (hipGetDevice(&dev) != hipSuccess) return KV_COMPACT_E_DEVICE;
        auto upload_v = [ctx, dev, V, V_dev, T, ev, &v_state] {
            const bool ok = hipSetDevice(dev) == hipSuccess &&
                            host_transfer(ctx, {{const_cast<float *>(V), V_dev, (size_t)T * ev * sizeof(float)}}, true,
                                          ctx->up_stream) &&
                            hipEventRecord(ctx->v_ev, ctx->up_stream) == hipSuccess;
            v_state = ok ? 1 : -1;
        };
        try {
            v_thread = std::thread(upload_v);
        } catch (...) {
            upload_v();   // (no thread: V is queued now, before the kernels)
        }
        v_ready = [&]() -> int {
            if (v_thread.joinable()) v_thread.join();
            if (v_state != 1 || hipStreamWaitEvent(st, ctx->v_ev, 0) != hipSuccess) return KV_COMPACT_E_DEVICE;
            return 0;
        };
    }
    // C_v goes to the caller's arrays through the pinned ring as soon as its
    // last writer is queued: a helper thread queues the transfers on the
    // upload stream (after an event on st) while the statistics run
    std::vector<HostSeg> down;
    for (int h = 0; h < H; h++)
        down.push_back({res->C_v[h], io.Cv + (size_t)h * t * dv, (size_t)t * dv * sizeof(float)});
    std::thread d_thread;
    std::atomic<int> d_state{0};   // 0 not started, 1 done, -1 failed
    auto download = [ctx, &down, &d_state, &touch](int dev) {
        touch.join();   // (the pages are mapped before the ring writes them)
        const bool ok = hipSetDevice(dev) == hipSuccess && hipStreamWaitEvent(ctx->up_stream, ctx->cv_ev, 0) == hipSuccess &&
                        host_transfer(ctx, down, false, ctx->up_stream);
        d_state = ok ? 1 : -1;
    };
    std::function<void()> cv_done = [&]() {
        int dev = 0;
        if (hipGetDevice(&dev) != hipSuccess || hipEventRecord(ctx->cv_ev, st) != hipSuccess) {
            d_state = -1;
            return;
        }
        try {
            d_thread = std::thread(download, dev);
        } catch (...) {
            download(dev);
        }
    };
    Timing tm;
    int rc = run_batch(ctx, st, pl, p, io, cv, &tm, v_ready, cv_done);
    if (v_thread.joinable()) v_thread.join();   // (run_batch stopped before it needed V)
    if (d_thread.joinable()) d_thread.join();
    if (rc == 0 && v_state != 1) rc = KV_COMPACT_E_DEVICE;
    if (rc == 0 && d_state == 0) {
        touch.join();
        d_state = host_transfer(ctx, down, false, st) ? 1 : -1;   // (cv_done was not reached)
    }
    if (rc == 0 && d_state != 1) rc = KV_COMPACT_E_DEVICE;
    if (rc != 0) {
        // nothing queued may still read the pinned ring or the arena
        (void)hipStreamSynchronize(ctx->up_stream);
        (void)hipStreamSynchronize(st);
        return rc;
    }

    // the small results
    float stats[3];
    e = hipMemcpy(res->selected_indices, io.indices, (size_t)t * sizeof(int), hipMemcpyDeviceToHost);
    for (int h = 0; h < H; h++)
        if (e == hipSuccess)
            e = hipMemcpy(res->beta[h], io.beta + (size_t)h * t, (size_t)t * sizeof(float), hipMemcpyDeviceToHost);
    if (e == hipSuccess) e = hipMemcpy(stats, io.stats, sizeof(stats), hipMemcpyDeviceToHost);
    if (e != hipSuccess) return KV_COMPACT_E_DEVICE;
    res->stats.avg_cosine_sim = stats[0];
    res->stats.avg_mse = stats[1];
    res->stats.avg_agreement = stats[2];
    res->stats.scoring_ms = tm.scoring_ms;
    res->stats.nnls_ms = tm.nnls_ms;
    res->stats.elapsed_ms = now_ms() - t0;
    guard.armed = false;
    return 0;
}

kv_compact_params defaults() {
    kv_compact_params p;
    memset(&p, 0, sizeof(p));
    p.target_ratio = 0.5f;
    p.ridge = 1e-6f;
    p.nnls_max_iter = 200;
    p.diversity_strength = 0.5f;
    p.skip_beta = 1;
    p.score_method = 1;
    p.omp_k_choice = 1;
    p.omp_refit_interval = 1;
    p.nnls_method = 1;
    return p;
}

// Reference state.h:326-352 (row geometry of the codecs)
int block_bytes(int type) {
    if (type == KV_TYPE_F32) return 4;
    if (type == KV_TYPE_F16 || type == KV_TYPE_BF16) return 2;
    if (type == KV_TYPE_Q8_0) return 34;
    if (type == KV_TYPE_Q4_0) return 18;
    if (type == KV_TYPE_Q4_1) return 20;
    return 4;
}
bool is_block_type(int t) { return t == KV_TYPE_Q8_0 || t == KV_TYPE_Q4_0 || t == KV_TYPE_Q4_1; }
bool known_type(int t) { return t == KV_TYPE_F32 || t == KV_TYPE_F16 || t == KV_TYPE_BF16 || is_block_type(t); }

// Quantized caches of L layers (device memory; layer strides in bytes).
struct QuantIO {
    const uint8_t * Kq = nullptr;
    const uint8_t * Vq = nullptr;
    long long lsKq = 0, lsVq = 0;
    int k_type = 0, v_type = 0;
    size_t k_rb = 0, v_rb = 0;
    uint8_t * Kout = nullptr;   // [L][t][k_rb]
    uint8_t * Vout = nullptr;   // [L][t][v_rb]
};

// times of the dequantization and requantization phases of the last quantized call
void record_codec_times(DeviceCtx * ctx) {
    float a = 0.0f, b = 0.0f;
    (void)hipEventElapsedTime(&a, ctx->q_ev[0], ctx->q_ev[1]);
    (void)hipEventElapsedTime(&b, ctx->q_ev[2], ctx->q_ev[3]);
    ctx->stage_ms[ST_DEQUANT] = a;
    ctx->stage_ms[ST_REQUANT] = b;
}

// rows [L][T] of a codec into fp32 [L][T][n_el]
// The coalesced codec kernels read and write the 2-byte fields of Q8_0, Q4_0,
// F16 and BF16 rows as 2-byte accesses: they need even addresses (row strides
// of these codecs are even; base and layer strides are the caller's). Other
// layouts go through the per-row kernels, which move single bytes.
bool two_byte_ok(int type, const void * base, long long ls) {
    if (type != KV_TYPE_Q8_0 && type != KV_TYPE_Q4_0 && type != KV_TYPE_F16 && type != KV_TYPE_BF16) return true;
    return ((reinterpret_cast<uintptr_t>(base) | (uintptr_t)ls) & 1) == 0;
}

void dequant_cache(const uint8_t * src, int type, size_t rb, long long ls, int n_el, int T, int L, float * dst,
                   hipStream_t st) {
    // (the coalesced kernel assembles F16 / BF16 / F32 elements from bytes)
    const bool even = ((reinterpret_cast<uintptr_t>(src) | (uintptr_t)ls | (uintptr_t)rb) & 1) == 0;
    if (codec8_ok(type, n_el) && (even || (type != KV_TYPE_Q8_0 && type != KV_TYPE_Q4_0))) {
        launch_dequant8(src, type, (long long)rb, ls, n_el, T, L, dst, st);
        return;
    }
    for (int l = 0; l < L; l++)
        launch_dequant_rows(src + (long long)l * ls, type, (long long)rb, n_el, T, dst + (long long)l * T * n_el, st);
}

// Scratch the requantization of L layers may need (value rows gathered from
// C_v when the coalesced kernel does not apply).
size_t requant_floats(const QuantIO & qi, int t, int H, int dv) {
    const bool v8 = codec8_ok(qi.v_type, H * dv) && dv % 8 == 0;
    return v8 ? 0 : (size_t)t * H * dv;
}

// A quantized K or V that the kernels read in place, decoding each block in
// registers as they load it (no fp32 copy of the cache): Q8_0 and Q4_0 whose
// 2-byte fields are aligned (even base, row and layer strides); K with d_k a
// multiple of 32 (whole slabs of the scoring tiles) and, when queries are
// provided, 16-byte aligned query rows; V with d_v a multiple of 4.
// KVC_INPLACE=0 sends every cache through the whole-cache decode instead.
RowCodec inplace_codec(const uint8_t * base, int type, size_t row_bytes, long long layer_bytes, int d, bool is_k,
                       const float * Q, long long ldQ) {
    RowCodec rc{};
    const char * e = getenv("KVC_INPLACE");
    if (e && e[0] == '0') return rc;
    if (type != KV_TYPE_Q8_0 && type != KV_TYPE_Q4_0) return rc;
    if ((reinterpret_cast<uintptr_t>(base) & 1) || (row_bytes & 1) || (layer_bytes & 1)) return rc;
    if (is_k) {
        if (d % 32 != 0) return rc;
        if (Q && ((reinterpret_cast<uintptr_t>(Q) & 15) || (ldQ & 3))) return rc;
    } else if (d % 4 != 0) {
        return rc;
    }
    rc.base = base;
    rc.row_bytes = (long long)row_bytes;
    rc.layer_bytes = layer_bytes;
    rc.type = type;
    return rc;
}

// K_out: the kept rows of the dequantized K (api.cpp:1234-1241); V_out: the
// refitted rows assembled over heads from C_v (api.cpp:1243-1254).
void requant_outputs(const QuantIO & qi, const float * Kf, const int * idx, const float * Cv, int L, int T, int t,
                     int H, int dk, int dv, float * rows_tmp, hipStream_t st, const RowCodec & kc) {
    if (t <= 0) return;
    const int ek = H * dk, ev = H * dv;
    const bool cv_al = (reinterpret_cast<uintptr_t>(Cv) & 15) == 0;
    const bool k_even = two_byte_ok(qi.k_type, qi.Kout, 0), v_even = two_byte_ok(qi.v_type, qi.Vout, 0);
    if (kc.base) {
        // K read in place: its kept rows are decoded and re-encoded in one pass
        // (in place only with an even K_out)
        launch_requant8(nullptr, 0, 0, idx, t, 0, H, dk, qi.k_type, ek, t, L, qi.Kout, (long long)qi.k_rb,
                        (long long)t * qi.k_rb, st, kc);
    } else if (codec8_ok(qi.k_type, ek) && k_even) {
        launch_requant8(Kf, (long long)T * ek, ek, idx, t, 0, H, dk, qi.k_type, ek, t, L, qi.Kout,
                        (long long)qi.k_rb, (long long)t * qi.k_rb, st);
    } else {
        for (int l = 0; l < L; l++)
            launch_quant_rows(Kf + (long long)l * T * ek, ek, idx + (long long)l * t, qi.k_type, ek, t,
                              qi.Kout + (long long)l * t * qi.k_rb, (long long)qi.k_rb, st);
    }
    if (codec8_ok(qi.v_type, ev) && dv % 8 == 0 && cv_al && v_even) {
        launch_requant8(Cv, 0, 0, nullptr, 0, 1, H, dv, qi.v_type, ev, t, L, qi.Vout, (long long)qi.v_rb,
                        (long long)t * qi.v_rb, st);
    } else {
        for (int l = 0; l < L; l++) {
            launch_gather_cv_rows(Cv + (long long)l * H * t * dv, H, t, dv, rows_tmp, st);
            launch_quant_rows(rows_tmp, ev, nullptr, qi.v_type, ev, t, qi.Vout + (long long)l * t * qi.v_rb,
                              (long long)qi.v_rb, st);
        }
    }
}

}  // namespace

// ======================================================================
// Reference C ABI
// ======================================================================
extern "C" {

kv_compact_params kv_compact_params_default(void) { return defaults(); }

int kv_compact(const float * K_all, const float * V_all, const float * Q_ref_all,
               int T, int n_q, int n_head_kv, int d_k, int d_v,
               const kv_compact_params * params, kv_compact_result * result) {
    kv_compact_params p = params ? *params : defaults();
    int rc = validate(K_all, V_all, result, T, n_q, n_head_kv, d_k, d_v, Q_ref_all, p);
    if (rc) return rc;
    rc = check_supported(p, d_v);
    if (rc) return rc;
    return compact_one(K_all, V_all, Q_ref_all, T, n_q, n_head_kv, d_k, d_v, p, result);
}

void kv_compact_result_free(kv_compact_result * r) {
    if (!r) return;
    free(r->selected_indices);
    r->selected_indices = NULL;
    if (r->beta) {
        for (int h = 0; h < r->n_head_kv; h++) free(r->beta[h]);
        free(r->beta);
        r->beta = NULL;
    }
    if (r->C_v) {
        for (int h = 0; h < r->n_head_kv; h++) free(r->C_v[h]);
        free(r->C_v);
        r->C_v = NULL;
    }
    r->t = 0;
    r->n_head_kv = 0;
}

// Reference api.cpp:980-1111: repeated compaction of the previous round's
// kept keys and refitted values; indices map back to the original positions.
int kv_compact_multi_round(const float * K_all, const float * V_all, const float * Q_ref_all,
                           int T, int n_q, int n_head_kv, int d_k, int d_v,
                           const kv_compact_params * params, int n_rounds,
                           kv_compact_result * result, kv_compact_stats * per_round_stats) {
    if (!K_all || !V_all || !result) return -1;
    if (T <= 0 || n_head_kv <= 0 || d_k <= 0 || d_v <= 0) return -2;
    if (n_rounds < 1) return -3;
    kv_compact_params pc = params ? *params : defaults();
    if (!Q_ref_all && !pc.use_cheap_qref) return -1;
    if (Q_ref_all && n_q <= 0 && !pc.use_cheap_qref) return -2;
    int rc = check_supported(pc, d_v);
    if (rc) return rc;
    const int H = n_head_kv;
    const size_t ek = (size_t)H * d_k, ev = (size_t)H * d_v;
    // host copies: rounds chain on small compacted caches
    std::vector<float> Kh((size_t)T * ek), Vh((size_t)T * ev);
    if (is_device_ptr(K_all)) {
        if (hipMemcpy(Kh.data(), K_all, Kh.size() * 4, hipMemcpyDeviceToHost) != hipSuccess) return KV_COMPACT_E_DEVICE;
    } else {
        memcpy(Kh.data(), K_all, Kh.size() * 4);
    }
    if (is_device_ptr(V_all)) {
        if (hipMemcpy(Vh.data(), V_all, Vh.size() * 4, hipMemcpyDeviceToHost) != hipSuccess) return KV_COMPACT_E_DEVICE;
    } else {
        memcpy(Vh.data(), V_all, Vh.size() * 4);
    }
    std::vector<float> Qh;
    const float * Qm = Q_ref_all;
    int nqm = n_q;
    if (pc.use_cheap_qref || !Q_ref_all) {
        nqm = cheap_count(T);
        Qh.resize((size_t)nqm * ek);
        for (int qi = 0; qi < nqm; qi++) {
            float f = (float)(qi + 1) / (float)(nqm + 1);
            f = f * f;
            int pos = (int)(f * (T - 1));
            pos = std::min(std::max(pos, 0), T - 1);
            memcpy(Qh.data() + (size_t)qi * ek, Kh.data() + (size_t)pos * ek, ek * 4);
        }
        Qm = Qh.data();
    } else if (is_device_ptr(Q_ref_all)) {
        Qh.resize((size_t)n_q * ek);
        if (hipMemcpy(Qh.data(), Q_ref_all, Qh.size() * 4, hipMemcpyDeviceToHost) != hipSuccess) return KV_COMPACT_E_DEVICE;
        Qm = Qh.data();
    }
    std::vector<int> orig(T);
    for (int i = 0; i < T; i++) orig[i] = i;
    std::vector<float> cK = Kh, cV = Vh;
    int cT = T;
    for (int round = 0; round < n_rounds; round++) {
        const int nqr = std::min(nqm, cT);
        kv_compact_result rr;
        memset(&rr, 0, sizeof(rr));
        rc = kv_compact(cK.data(), cV.data(), Qm, cT, nqr, H, d_k, d_v, params, &rr);
        if (rc != 0) {
            kv_compact_result_free(&rr);
            return rc;
        }
        if (per_round_stats) per_round_stats[round] = rr.stats;
        const int nT = rr.t;
        std::vector<int> norig(nT);
        std::vector<float> nK((size_t)nT * ek), nV((size_t)nT * ev);
        for (int j = 0; j < nT; j++) {
            const int src = rr.selected_indices[j];
            norig[j] = orig[src];
            memcpy(nK.data() + (size_t)j * ek, cK.data() + (size_t)src * ek, ek * 4);
            for (int h = 0; h < H; h++)
                memcpy(nV.data() + (size_t)j * ev + (size_t)h * d_v, rr.C_v[h] + (size_t)j * d_v, (size_t)d_v * 4);
        }
        if (round == n_rounds - 1) {
            std::vector<float> b((size_t)H * nT), c((size_t)H * nT * d_v);
            for (int h = 0; h < H; h++) {
                memcpy(b.data() + (size_t)h * nT, rr.beta[h], (size_t)nT * 4);
                memcpy(c.data() + (size_t)h * nT * d_v, rr.C_v[h], (size_t)nT * d_v * 4);
            }
            if (!fill_result(result, nT, H, d_v, norig, b, c)) {
                kv_compact_result_free(&rr);
                return KV_COMPACT_E_DEVICE;
            }
            result->stats = rr.stats;
        }
        kv_compact_result_free(&rr);
        cK.swap(nK);
        cV.swap(nV);
        orig.swap(norig);
        cT = nT;
    }
    // final statistics against the original cache, on the GPU: evaluate the
    // result as a one-chunk call over the original data
    {
        DeviceCtx * ctx = device_ctx();
        if (!ctx) return KV_COMPACT_E_DEVICE;
        std::lock_guard<std::mutex> lk(ctx->mu);
        hipStream_t st = ctx->stream;
        if (!drain_second_stream(ctx, st)) return KV_COMPACT_E_DEVICE;
        Plan pl;
        kv_compact_params sp = pc;
        sp.chunk_size = -1;
        make_plan(T, nqm, true, sp, pl);
        pl.t_total = result->t;
        pl.chunks[pl.n_chunks].tc = result->t;
        pl.chunks[pl.n_chunks + 1].Tc = result->t;
        pl.chunks[pl.n_chunks + 1].tc = result->t;
        BatchIO io{};
        io.L = 1; io.T = T; io.n_q = nqm; io.H = H; io.dk = d_k; io.dv = d_v;
        io.ldK = (long long)T * ek; io.ldV = (long long)T * ev; io.ldQ = (long long)nqm * ek;
        Carver sizer;
        sizer.take<float>((size_t)T * ek); sizer.take<float>((size_t)T * ev); sizer.take<float>((size_t)nqm * ek);
        sizer.take<int>(std::max(result->t, 1)); sizer.take<float>((size_t)H * result->t);
        sizer.take<float>((size_t)H * result->t * d_v); sizer.take<float>(3);
        size_t need = workspace_bytes(pl, io, nullptr, &sizer, nullptr, nullptr);
        if (!ensure_arena(ctx, need)) return KV_COMPACT_E_DEVICE;
        Carver cv;
        cv.base = ctx->arena;
        float * dK = cv.take<float>((size_t)T * ek);
        float * dV = cv.take<float>((size_t)T * ev);
        float * dQ = cv.take<float>((size_t)nqm * ek);
        int * dI = cv.take<int>(std::max(result->t, 1));
        float * dB = cv.take<float>((size_t)H * result->t);
        float * dC = cv.take<float>((size_t)H * result->t * d_v);
        float * dS = cv.take<float>(3);
        Work w{};
        StatWork sw{};
        workspace_bytes(pl, io, nullptr, &cv, &w, &sw);
        sw.qmode = Q_PROVIDED;
        std::vector<float> b((size_t)H * result->t), c((size_t)H * result->t * d_v);
        for (int h = 0; h < H; h++) {
            memcpy(b.data() + (size_t)h * result->t, result->beta[h], (size_t)result->t * 4);
            memcpy(c.data() + (size_t)h * result->t * d_v, result->C_v[h], (size_t)result->t * d_v * 4);
        }
        hipError_t e = hipMemcpyAsync(dK, Kh.data(), Kh.size() * 4, hipMemcpyHostToDevice, st);
        if (e == hipSuccess) e = hipMemcpyAsync(dV, Vh.data(), Vh.size() * 4, hipMemcpyHostToDevice, st);
        if (e == hipSuccess) e = hipMemcpyAsync(dQ, Qm, (size_t)nqm * ek * 4, hipMemcpyHostToDevice, st);
        if (e == hipSuccess) e = hipMemcpyAsync(dI, result->selected_indices, (size_t)result->t * 4, hipMemcpyHostToDevice, st);
        if (e == hipSuccess) e = hipMemcpyAsync(dB, b.data(), b.size() * 4, hipMemcpyHostToDevice, st);
        if (e == hipSuccess) e = hipMemcpyAsync(dC, c.data(), c.size() * 4, hipMemcpyHostToDevice, st);
        if (e == hipSuccess) e = hipMemcpyAsync(w.chunks, pl.chunks.data(), pl.chunks.size() * sizeof(ChunkDesc), hipMemcpyHostToDevice, st);
        if (e != hipSuccess) return KV_COMPACT_E_DEVICE;
        Geom g{};
        g.L = 1; g.T = T; g.H = H; g.dk = d_k; g.dv = d_v;
        g.n_chunks = pl.n_chunks; g.t_total = result->t; g.nq_max = pl.nq_max;
        g.tc_max = pl.tc_max; g.Tc_max = pl.Tc_max; g.qmode = Q_PROVIDED; g.nq_global = nqm;
        g.ldK = io.ldK; g.ldV = io.ldV; g.ldQ = io.ldQ;
        g.score_method = pc.score_method; g.inv_sqrt_dk = 1.0f / sqrtf((float)d_k); g.ridge = pc.ridge;
        w.sel = dI;
        launch_stats(g, w, sw, dK, dV, dQ, dB, dC, dS, st);
        float s3[3];
        e = hipGetLastError();
        if (e == hipSuccess) e = hipMemcpyAsync(s3, dS, sizeof(s3), hipMemcpyDeviceToHost, st);
        if (e == hipSuccess) e = hipStreamSynchronize(st);
        if (e != hipSuccess) return KV_COMPACT_E_DEVICE;
        result->stats.avg_cosine_sim = s3[0];
        result->stats.avg_mse = s3[1];
        result->stats.avg_agreement = s3[2];
    }
    return 0;
}

// ---- codec (reference api.cpp:1150-1180; state.h:326-629) ----

int kv_quant_row_elements(int type, size_t row_bytes) {
    if (type == KV_TYPE_F32) return (int)(row_bytes / 4);
    if (type == KV_TYPE_F16 || type == KV_TYPE_BF16) return (int)(row_bytes / 2);
    if (is_block_type(type)) return (int)(row_bytes / (size_t)block_bytes(type)) * 32;
    return (int)(row_bytes / 4);
}

size_t kv_quant_row_bytes(int type, int n_elements) {
    if (type == KV_TYPE_F32) return (size_t)n_elements * 4;
    if (type == KV_TYPE_F16 || type == KV_TYPE_BF16) return (size_t)n_elements * 2;
    if (is_block_type(type)) return (size_t)(n_elements / 32) * (size_t)block_bytes(type);
    return (size_t)n_elements * 4;
}

int kv_dequantize_row(const uint8_t * src, int type, size_t row_bytes, float * dst, int max_elements) {
    int n = kv_quant_row_elements(type, row_bytes);
    if (n > max_elements) n = max_elements;
    if (n <= 0) return n;
    if (!known_type(type)) {
        memset(dst, 0, (size_t)n * sizeof(float));
        return n;
    }
    DeviceCtx * ctx = device_ctx();
    if (!ctx) return KV_COMPACT_E_DEVICE;
    std::lock_guard<std::mutex> lk(ctx->mu);
    const int n_conv = is_block_type(type) ? (n / 32) * 32 : n;
    if (!drain_second_stream(ctx, ctx->stream) || !ensure_arena(ctx, row_bytes + (size_t)n * 4 + 4096))
        return KV_COMPACT_E_DEVICE;
    uint8_t * ds = reinterpret_cast<uint8_t *>(ctx->arena);
    float * dd = reinterpret_cast<float *>(ctx->arena + ((row_bytes + 255) & ~(size_t)255));
    hipStream_t st = ctx->stream;
    if (hipMemcpyAsync(ds, src, row_bytes, hipMemcpyHostToDevice, st) != hipSuccess) return KV_COMPACT_E_DEVICE;
    if (n_conv > 0) launch_dequant_rows(ds, type, (long long)row_bytes, n_conv, 1, dd, st);
    if (n_conv > 0 && hipMemcpyAsync(dst, dd, (size_t)n_conv * 4, hipMemcpyDeviceToHost, st) != hipSuccess)
        return KV_COMPACT_E_DEVICE;
    if (hipStreamSynchronize(st) != hipSuccess) return KV_COMPACT_E_DEVICE;
    return n;
}

size_t kv_quantize_row(const float * src, int type, int n_elements, uint8_t * dst) {
    if (!known_type(type) || n_elements <= 0) return 0;
    const size_t nb = kv_quant_row_bytes(type, n_elements);
    if (nb == 0) return 0;
    DeviceCtx * ctx = device_ctx();
    if (!ctx) return 0;
    std::lock_guard<std::mutex> lk(ctx->mu);
    if (!drain_second_stream(ctx, ctx->stream) || !ensure_arena(ctx, (size_t)n_elements * 4 + nb + 4096)) return 0;
    float * ds = reinterpret_cast<float *>(ctx->arena);
    uint8_t * dd = reinterpret_cast<uint8_t *>(ctx->arena + (((size_t)n_elements * 4 + 255) & ~(size_t)255));
    hipStream_t st = ctx->stream;
    if (hipMemcpyAsync(ds, src, (size_t)n_elements * 4, hipMemcpyHostToDevice, st) != hipSuccess) return 0;
    const int n_conv = is_block_type(type) ? (n_elements / 32) * 32 : n_elements;
    launch_quant_rows(ds, 0, nullptr, type, n_conv, 1, dd, (long long)nb, st);
    if (hipMemcpyAsync(dst, dd, nb, hipMemcpyDeviceToHost, st) != hipSuccess) return 0;
    if (hipStreamSynchronize(st) != hipSuccess) return 0;
    return nb;
}

// Reference api.cpp:1182-1257: the quantized rows are uploaded into the
// workspace, dequantized there, compacted, and the kept K rows and refitted V
// rows requantized there; the host receives the results only.
int kv_compact_quantized(const uint8_t * K_quant, const uint8_t * V_quant, const float * Q_ref_all,
                         int k_type, int v_type, size_t k_row_bytes, size_t v_row_bytes,
                         int T, int n_q, int n_head_kv, int d_k, int d_v,
                         const kv_compact_params * params, kv_compact_quant_result * result) {
    if (!K_quant || !V_quant || !result) return -1;
    if (T <= 0 || n_head_kv <= 0 || d_k <= 0 || d_v <= 0) return -2;
    const int H = n_head_kv;
    const int ek = H * d_k, ev = H * d_v;
    if (kv_quant_row_elements(k_type, k_row_bytes) != ek || kv_quant_row_elements(v_type, v_row_bytes) != ev)
        return -4;
    kv_compact_params p = params ? *params : defaults();
    int rc = validate((const float *)K_quant, (const float *)V_quant, result, T, n_q, H, d_k, d_v, Q_ref_all, p);
    if (rc) return rc;
    memset(&result->base, 0, sizeof(result->base));
    rc = check_supported(p, d_v);
    if (rc) return rc;
    if (!known_type(k_type) || !known_type(v_type)) return KV_COMPACT_E_UNSUPPORTED;
    const double t0 = now_ms();
    DeviceCtx * ctx = device_ctx();
    if (!ctx) return KV_COMPACT_E_DEVICE;
    std::lock_guard<std::mutex> lk(ctx->mu);
    hipStream_t st = ctx->stream;
    if (!drain_second_stream(ctx, st)) return KV_COMPACT_E_DEVICE;
    Plan pl;
    const bool q_given = Q_ref_all != nullptr;
    make_plan(T, n_q, q_given, p, pl);
    const bool use_q = q_given && !p.use_cheap_qref;
    const bool qd = use_q && is_device_ptr(Q_ref_all);
    std::vector<float> wts;
    const bool have_w = rkv_weights(p, T, wts);
    const int t = pl.t_total;
    QuantIO qi;
    qi.k_type = k_type; qi.v_type = v_type; qi.k_rb = k_row_bytes; qi.v_rb = v_row_bytes;
    qi.lsKq = (long long)T * k_row_bytes; qi.lsVq = (long long)T * v_row_bytes;
    BatchIO io{};
    io.L = 1; io.T = T; io.n_q = n_q; io.H = H; io.dk = d_k; io.dv = d_v;
    io.ldK = (long long)T * ek; io.ldV = (long long)T * ev; io.ldQ = (long long)std::max(n_q, 1) * ek;
    // K / V read in place (the carve below places the quantized rows at
    // 256-byte boundaries, so only the strides and shapes decide)
    const bool k_in = inplace_codec(reinterpret_cast<const uint8_t *>(256), k_type, k_row_bytes, qi.lsKq, d_k, true,
                                    use_q ? reinterpret_cast<const float *>(qd ? Q_ref_all : nullptr) : nullptr,
                                    io.ldQ).base != nullptr;
    const bool v_in = inplace_codec(reinterpret_cast<const uint8_t *>(256), v_type, v_row_bytes, qi.lsVq, d_v, false,
                                    nullptr, 0).base != nullptr;
    // workspace: quantized rows, fp32 cache, query rows, weights, outputs, requantized rows, batch workspace
    auto carve = [&](Carver & cv, uint8_t *& dKq, uint8_t *& dVq, float *& dK, float *& dV, float *& dQ,
                     float *& dW, float *& tmp) {
        dKq = cv.take<uint8_t>((size_t)T * k_row_bytes);
        dVq = cv.take<uint8_t>((size_t)T * v_row_bytes);
        dK = k_in ? nullptr : cv.take<float>((size_t)T * ek);
        dV = v_in ? nullptr : cv.take<float>((size_t)T * ev);
        dQ = (use_q && !qd) ? cv.take<float>((size_t)n_q * ek) : nullptr;
        dW = have_w ? cv.take<float>(T) : nullptr;
        io.indices = cv.take<int>(std::max(t, 1));
        io.beta = cv.take<float>((size_t)H * std::max(t, 1));
        io.Cv = cv.take<float>((size_t)H * std::max(t, 1) * d_v);
        io.stats = cv.take<float>(3);
        qi.Kout = cv.take<uint8_t>((size_t)std::max(t, 1) * k_row_bytes);
        qi.Vout = cv.take<uint8_t>((size_t)std::max(t, 1) * v_row_bytes);
        tmp = cv.take<float>(std::max<size_t>(requant_floats(qi, t, H, d_v), 1));
    };
    uint8_t * dKq; uint8_t * dVq; float * dK; float * dV; float * dQ; float * dW; float * tmp;
    Carver sizer;
    carve(sizer, dKq, dVq, dK, dV, dQ, dW, tmp);
    const size_t need = workspace_bytes(pl, io, &p, &sizer, nullptr, nullptr);
    if (!ensure_arena(ctx, need)) return KV_COMPACT_E_DEVICE;
    Carver cv;
    cv.base = ctx->arena;
    carve(cv, dKq, dVq, dK, dV, dQ, dW, tmp);
    // the quantized rows through the pinned ring, the small inputs directly
    const std::vector<HostSeg> up{{const_cast<void *>(static_cast<const void *>(K_quant)), dKq, (size_t)T * k_row_bytes},
                                  {const_cast<void *>(static_cast<const void *>(V_quant)), dVq, (size_t)T * v_row_bytes}};
    if (!host_transfer(ctx, up, true, st)) return KV_COMPACT_E_DEVICE;
    hipError_t e = hipSuccess;
    if (dQ) e = hipMemcpyAsync(dQ, Q_ref_all, (size_t)n_q * ek * 4, hipMemcpyHostToDevice, st);
    if (e == hipSuccess && dW) e = hipMemcpyAsync(dW, wts.data(), (size_t)T * 4, hipMemcpyHostToDevice, st);
    if (e != hipSuccess) return KV_COMPACT_E_DEVICE;
    io.Q = use_q ? (qd ? Q_ref_all : dQ) : nullptr;
    io.kc = k_in ? inplace_codec(dKq, k_type, k_row_bytes, qi.lsKq, d_k, true, io.Q, io.ldQ) : RowCodec{};
    io.vc = v_in ? inplace_codec(dVq, v_type, v_row_bytes, qi.lsVq, d_v, false, nullptr, 0) : RowCodec{};
    if (k_in != (io.kc.base != nullptr) || v_in != (io.vc.base != nullptr)) return KV_COMPACT_E_DEVICE;
    (void)hipEventRecord(ctx->q_ev[0], st);
    if (!k_in) dequant_cache(dKq, k_type, k_row_bytes, qi.lsKq, ek, T, 1, dK, st);
    if (!v_in) dequant_cache(dVq, v_type, v_row_bytes, qi.lsVq, ev, T, 1, dV, st);
    (void)hipEventRecord(ctx->q_ev[1], st);
    io.K = dK; io.V = dV; io.wts = dW;
    Timing tm;
    rc = run_batch(ctx, st, pl, p, io, cv, &tm);
    if (rc != 0) return rc;
    (void)hipEventRecord(ctx->q_ev[2], st);
    requant_outputs(qi, dK, io.indices, io.Cv, 1, T, t, H, d_k, d_v, tmp, st, io.kc);
    (void)hipEventRecord(ctx->q_ev[3], st);
    // results straight into the caller's arrays (C_v and the requantized
    // rows through the pinned ring)
    float stats[3];
    result->K_out = (uint8_t *)malloc((size_t)std::max(t, 1) * k_row_bytes);
    result->V_out = (uint8_t *)malloc((size_t)std::max(t, 1) * v_row_bytes);
    if (!result->K_out || !result->V_out || !alloc_result(&result->base, t, H, d_v)) {
        free(result->K_out);
        free(result->V_out);
        result->K_out = result->V_out = NULL;
        kv_compact_result_free(&result->base);
        return KV_COMPACT_E_DEVICE;
    }
    e = hipGetLastError();
    if (e == hipSuccess) e = hipStreamSynchronize(st);
    if (e == hipSuccess) record_codec_times(ctx);
    if (e == hipSuccess)
        e = hipMemcpy(result->base.selected_indices, io.indices, (size_t)t * sizeof(int), hipMemcpyDeviceToHost);
    std::vector<HostSeg> down;
    for (int h = 0; h < H; h++) {
        if (e == hipSuccess)
            e = hipMemcpy(result->base.beta[h], io.beta + (size_t)h * t, (size_t)t * 4, hipMemcpyDeviceToHost);
        down.push_back({result->base.C_v[h], io.Cv + (size_t)h * t * d_v, (size_t)t * d_v * 4});
    }
    if (e == hipSuccess) e = hipMemcpy(stats, io.stats, sizeof(stats), hipMemcpyDeviceToHost);
    if (t > 0) {
        down.push_back({result->K_out, qi.Kout, (size_t)t * k_row_bytes});
        down.push_back({result->V_out, qi.Vout, (size_t)t * v_row_bytes});
    }
    if (e != hipSuccess || !host_transfer(ctx, down, false, st)) {
        free(result->K_out);
        free(result->V_out);
        result->K_out = result->V_out = NULL;
        kv_compact_result_free(&result->base);
        return KV_COMPACT_E_DEVICE;
    }
    result->base.stats.avg_cosine_sim = stats[0];
    result->base.stats.avg_mse = stats[1];
    result->base.stats.avg_agreement = stats[2];
    result->base.stats.scoring_ms = tm.scoring_ms;
    result->base.stats.nnls_ms = tm.nnls_ms;
    result->base.stats.elapsed_ms = now_ms() - t0;
    result->k_type = k_type;
    result->v_type = v_type;
    result->k_row_bytes = k_row_bytes;
    result->v_row_bytes = v_row_bytes;
    return 0;
}

void kv_compact_quant_result_free(kv_compact_quant_result * r) {
    if (!r) return;
    kv_compact_result_free(&r->base);
    free(r->K_out);
    r->K_out = NULL;
    free(r->V_out);
    r->V_out = NULL;
}

// ======================================================================
// Accelerator plug-in ABI (reference include/kv-compact-accel.h)
// ======================================================================

int kv_compact_hip_available(void) { return device_ctx() ? 1 : 0; }

int kv_compact_hip_mat_mul_ABt_scaled(const float * A, const float * B, float * C, int m, int n, int k,
                                      float scale) {
    DeviceCtx * ctx = device_ctx();
    if (!ctx || m <= 0 || n <= 0 || k <= 0) return -1;
    std::lock_guard<std::mutex> lk(ctx->mu);
    const size_t sa = (size_t)m * k, sb = (size_t)n * k, sc = (size_t)m * n;
    if (!drain_second_stream(ctx, ctx->stream) || !ensure_arena(ctx, (sa + sb + sc) * 4 + 1024)) return -1;
    Carver cv;
    cv.base = ctx->arena;
    float * dA = cv.take<float>(sa);
    float * dB = cv.take<float>(sb);
    float * dC = cv.take<float>(sc);
    hipStream_t st = ctx->stream;
    hipError_t e = hipMemcpyAsync(dA, A, sa * 4, hipMemcpyHostToDevice, st);
    if (e == hipSuccess) e = hipMemcpyAsync(dB, B, sb * 4, hipMemcpyHostToDevice, st);
    if (e != hipSuccess) return -1;
    launch_gemm_abt(dA, k, dB, k, dC, n, m, n, k, scale, 0, 0, 0, 1, st);
    e = hipMemcpyAsync(C, dC, sc * 4, hipMemcpyDeviceToHost, st);
    if (e == hipSuccess) e = hipStreamSynchronize(st);
    return e == hipSuccess ? 0 : -1;
}

int kv_compact_hip_score_all_heads(const float * Q_ref, const float * K_all, float ** scores_out,
                                   int n_q, int T, int n_head_kv, int d_k, float scale) {
    DeviceCtx * ctx = device_ctx();
    if (!ctx || n_q <= 0 || T <= 0 || n_head_kv <= 0 || d_k <= 0) return -1;
    std::lock_guard<std::mutex> lk(ctx->mu);
    const size_t ek = (size_t)n_head_kv * d_k;
    const size_t sq = (size_t)n_q * ek, sk = (size_t)T * ek, ss = (size_t)n_head_kv * n_q * T;
    if (!drain_second_stream(ctx, ctx->stream) || !ensure_arena(ctx, (sq + sk + ss) * 4 + 1024)) return -1;
    Carver cv;
    cv.base = ctx->arena;
    float * dQ = cv.take<float>(sq);
    float * dK = cv.take<float>(sk);
    float * dS = cv.take<float>(ss);
    hipStream_t st = ctx->stream;
    hipError_t e = hipMemcpyAsync(dQ, Q_ref, sq * 4, hipMemcpyHostToDevice, st);
    if (e == hipSuccess) e = hipMemcpyAsync(dK, K_all, sk * 4, hipMemcpyHostToDevice, st);
    if (e != hipSuccess) return -1;
    launch_gemm_abt(dQ, (long long)ek, dK, (long long)ek, dS, T, n_q, T, d_k, scale, d_k, d_k,
                    (long long)n_q * T, n_head_kv, st);
    for (int h = 0; h < n_head_kv && e == hipSuccess; h++)
        e = hipMemcpyAsync(scores_out[h], dS + (size_t)h * n_q * T, (size_t)n_q * T * 4, hipMemcpyDeviceToHost, st);
    if (e == hipSuccess) e = hipStreamSynchronize(st);
    return e == hipSuccess ? 0 : -1;
}

int kv_compact_hip_refit_target_all_heads(const float * const * W_per_head, const float * V_all,
                                          float ** Y_out, int n_q, int T, int n_head_kv, int d_v) {
    DeviceCtx * ctx = device_ctx();
    if (!ctx || n_q <= 0 || T <= 0 || n_head_kv <= 0 || d_v <= 0) return -1;
    std::lock_guard<std::mutex> lk(ctx->mu);
    const size_t ev = (size_t)n_head_kv * d_v;
    const size_t sw = (size_t)n_head_kv * n_q * T, sv = (size_t)T * ev, sy = (size_t)n_head_kv * n_q * d_v;
    if (!drain_second_stream(ctx, ctx->stream) || !ensure_arena(ctx, (sw + sv + sy) * 4 + 1024)) return -1;
    Carver cv;
    cv.base = ctx->arena;
    float * dW = cv.take<float>(sw);
    float * dV = cv.take<float>(sv);
    float * dY = cv.take<float>(sy);
    hipStream_t st = ctx->stream;
    hipError_t e = hipSuccess;
    for (int h = 0; h < n_head_kv && e == hipSuccess; h++)
        e = hipMemcpyAsync(dW + (size_t)h * n_q * T, W_per_head[h], (size_t)n_q * T * 4, hipMemcpyHostToDevice, st);
    if (e == hipSuccess) e = hipMemcpyAsync(dV, V_all, sv * 4, hipMemcpyHostToDevice, st);
    if (e != hipSuccess) return -1;
    launch_gemm_ab(dW, T, dV, (long long)ev, dY, d_v, n_q, d_v, T, (long long)n_q * T, d_v,
                   (long long)n_q * d_v, n_head_kv, st);
    for (int h = 0; h < n_head_kv && e == hipSuccess; h++)
        e = hipMemcpyAsync(Y_out[h], dY + (size_t)h * n_q * d_v, (size_t)n_q * d_v * 4, hipMemcpyDeviceToHost, st);
    if (e == hipSuccess) e = hipStreamSynchronize(st);
    return e == hipSuccess ? 0 : -1;
}

void kv_compact_hip_pool_free(void) { kvc_release_workspace(); }

// ======================================================================
// Device-resident batch API (include/kv-compact-device.h)
// ======================================================================

int kvc_plan(int T, int n_q, int q_ref_given, const kv_compact_params * params, int * t_total, int * n_chunks) {
    if (T <= 0) return -2;
    kv_compact_params p = params ? *params : defaults();
    Plan pl;
    make_plan(T, n_q, q_ref_given != 0, p, pl);
    if (t_total) *t_total = pl.t_total;
    if (n_chunks) *n_chunks = pl.n_chunks;
    return 0;
}

}  // extern "C"

namespace {

// kvc_compact_layers_device and its allocation-free variant: the workspace is
// the device arena (grown with hipMalloc when needed) or the fixed scratch.
int layers_device(const float * K, const float * V, const float * Q_ref, int L, int T, int n_q, int n_head_kv,
                  int d_k, int d_v, long long ldK, long long ldV, long long ldQ, const kv_compact_params * params,
                  const float * token_weight, kvc_device_out * out, void * stream, bool noalloc) {
    kv_compact_params p = params ? *params : defaults();
    int rc = validate(K, V, out, T, n_q, n_head_kv, d_k, d_v, Q_ref, p);
    if (rc) return rc;
    if (L <= 0) return -2;
    if (!out->indices || !out->beta || !out->C_v || !out->stats) return -1;
    rc = check_supported(p, d_v);
    if (rc) return rc;
    DeviceCtx * ctx = device_ctx();
    if (!ctx) return KV_COMPACT_E_DEVICE;
    std::lock_guard<std::mutex> lk(ctx->mu);
    hipStream_t st = stream ? (hipStream_t)stream : ctx->stream;
    Plan pl;
    make_plan(T, n_q, Q_ref != nullptr, p, pl);
    BatchIO io{};
    io.K = K; io.V = V; io.Q = (Q_ref && !p.use_cheap_qref) ? Q_ref : nullptr;
    io.ldK = ldK; io.ldV = ldV; io.ldQ = ldQ;
    io.L = L; io.T = T; io.n_q = n_q; io.H = n_head_kv; io.dk = d_k; io.dv = d_v;
    io.indices = out->indices; io.beta = out->beta; io.Cv = out->C_v; io.stats = out->stats;
    std::vector<float> wts;
    const bool host_w = !token_weight && rkv_weights(p, T, wts);
    Carver sizer;
    if (host_w) sizer.take<float>(T);
    const size_t need = workspace_bytes(pl, io, &p, &sizer, nullptr, nullptr);
    if (!drain_second_stream(ctx, st)) return KV_COMPACT_E_DEVICE;
    Carver cv;
    if (noalloc) {
        if (!ctx->scratch) return KV_COMPACT_E_DEVICE;
        if (need > (size_t)KVC_NOALLOC_SCRATCH_BYTES) {
            fprintf(stderr, "[kv-compact] kvc_compact_layers_device_noalloc: the call needs %zu bytes of workspace, "
                            "the fixed scratch holds %zu\n", need, (size_t)KVC_NOALLOC_SCRATCH_BYTES);
            return KVC_E_SCRATCH;
        }
        cv.base = ctx->scratch;
    } else {
        if (!ensure_arena(ctx, need)) return KV_COMPACT_E_DEVICE;
        cv.base = ctx->arena;
    }
    io.wts = token_weight;
    if (host_w) {
        float * dW = cv.take<float>(T);
        if (hipMemcpyAsync(dW, wts.data(), (size_t)T * 4, hipMemcpyHostToDevice, st) != hipSuccess)
            return KV_COMPACT_E_DEVICE;
        io.wts = dW;
    }
    return run_batch(ctx, st, pl, p, io, cv, nullptr);
}

}  // namespace

extern "C" {

int kvc_compact_layers_device(const float * K, const float * V, const float * Q_ref, int L, int T, int n_q,
                              int n_head_kv, int d_k, int d_v, long long ldK, long long ldV, long long ldQ,
                              const kv_compact_params * params, const float * token_weight,
                              kvc_device_out * out, void * stream) {
    return layers_device(K, V, Q_ref, L, T, n_q, n_head_kv, d_k, d_v, ldK, ldV, ldQ, params, token_weight, out,
                         stream, false);
}

int kvc_compact_layers_device_noalloc(const float * K, const float * V, const float * Q_ref, int L, int T, int n_q,
                                      int n_head_kv, int d_k, int d_v, long long ldK, long long ldV, long long ldQ,
                                      const kv_compact_params * params, const float * token_weight,
                                      kvc_device_out * out, void * stream) {
    return layers_device(K, V, Q_ref, L, T, n_q, n_head_kv, d_k, d_v, ldK, ldV, ldQ, params, token_weight, out,
                         stream, true);
}

int kvc_compact_quantized_layers_device(const uint8_t * K_quant, const uint8_t * V_quant, const float * Q_ref,
                                        int L, int k_type, int v_type, size_t k_row_bytes, size_t v_row_bytes,
                                        int T, int n_q, int n_head_kv, int d_k, int d_v,
                                        long long ldKq, long long ldVq, long long ldQ,
                                        const kv_compact_params * params, kvc_device_out * out,
                                        uint8_t * K_out, uint8_t * V_out, void * stream) {
    if (!K_quant || !V_quant || !out || !K_out || !V_out) return -1;
    if (T <= 0 || n_head_kv <= 0 || d_k <= 0 || d_v <= 0 || L <= 0) return -2;
    const int H = n_head_kv, ek = H * d_k, ev = H * d_v;
    if (kv_quant_row_elements(k_type, k_row_bytes) != ek || kv_quant_row_elements(v_type, v_row_bytes) != ev)
        return -4;
    if (!known_type(k_type) || !known_type(v_type)) return KV_COMPACT_E_UNSUPPORTED;
    if (!out->indices || !out->beta || !out->C_v || !out->stats) return -1;
    kv_compact_params p = params ? *params : defaults();
    int rc = validate((const float *)K_quant, (const float *)V_quant, out, T, n_q, H, d_k, d_v, Q_ref, p);
    if (rc) return rc;
    rc = check_supported(p, d_v);
    if (rc) return rc;
    DeviceCtx * ctx = device_ctx();
    if (!ctx) return KV_COMPACT_E_DEVICE;
    std::lock_guard<std::mutex> lk(ctx->mu);
    hipStream_t st = stream ? (hipStream_t)stream : ctx->stream;
    if (!drain_second_stream(ctx, st)) return KV_COMPACT_E_DEVICE;
    Plan pl;
    make_plan(T, n_q, Q_ref != nullptr, p, pl);
    const int t = pl.t_total;
    QuantIO qi;
    qi.Kq = K_quant; qi.Vq = V_quant; qi.lsKq = ldKq; qi.lsVq = ldVq;
    qi.k_type = k_type; qi.v_type = v_type; qi.k_rb = k_row_bytes; qi.v_rb = v_row_bytes;
    qi.Kout = K_out; qi.Vout = V_out;
    BatchIO io{};
    io.Q = (Q_ref && !p.use_cheap_qref) ? Q_ref : nullptr;
    io.ldK = (long long)T * ek; io.ldV = (long long)T * ev; io.ldQ = ldQ;
    io.L = L; io.T = T; io.n_q = n_q; io.H = H; io.dk = d_k; io.dv = d_v;
    io.indices = out->indices; io.beta = out->beta; io.Cv = out->C_v; io.stats = out->stats;
    std::vector<float> wts;
    const bool host_w = rkv_weights(p, T, wts);
    // (the kept rows of an in-place K are re-encoded with 2-byte stores: even K_out)
    io.kc = two_byte_ok(k_type, K_out, 0) ? inplace_codec(K_quant, k_type, k_row_bytes, ldKq, d_k, true, io.Q, io.ldQ)
                                          : RowCodec{};
    io.vc = inplace_codec(V_quant, v_type, v_row_bytes, ldVq, d_v, false, nullptr, 0);
    auto carve = [&](Carver & cv, float *& dK, float *& dV, float *& dW, float *& tmp) {
        dK = io.kc.base ? nullptr : cv.take<float>((size_t)L * T * ek);
        dV = io.vc.base ? nullptr : cv.take<float>((size_t)L * T * ev);
        dW = host_w ? cv.take<float>(T) : nullptr;
        tmp = cv.take<float>(std::max<size_t>(requant_floats(qi, t, H, d_v), 1));
    };
    float * dK; float * dV; float * dW; float * tmp;
    Carver sizer;
    carve(sizer, dK, dV, dW, tmp);
    const size_t need = workspace_bytes(pl, io, &p, &sizer, nullptr, nullptr);
    if (!ensure_arena(ctx, need)) return KV_COMPACT_E_DEVICE;
    Carver cv;
    cv.base = ctx->arena;
    carve(cv, dK, dV, dW, tmp);
    if (dW && hipMemcpyAsync(dW, wts.data(), (size_t)T * 4, hipMemcpyHostToDevice, st) != hipSuccess)
        return KV_COMPACT_E_DEVICE;
    (void)hipEventRecord(ctx->q_ev[0], st);
    if (!io.kc.base) dequant_cache(K_quant, k_type, k_row_bytes, ldKq, ek, T, L, dK, st);
    if (!io.vc.base) dequant_cache(V_quant, v_type, v_row_bytes, ldVq, ev, T, L, dV, st);
    (void)hipEventRecord(ctx->q_ev[1], st);
    io.K = dK; io.V = dV; io.wts = dW;
    rc = run_batch(ctx, st, pl, p, io, cv, nullptr);
    if (rc != 0) return rc;
    (void)hipEventRecord(ctx->q_ev[2], st);
    requant_outputs(qi, dK, io.indices, io.Cv, L, T, t, H, d_k, d_v, tmp, st, io.kc);
    (void)hipEventRecord(ctx->q_ev[3], st);
    hipError_t e = hipGetLastError();
    if (e == hipSuccess) e = hipStreamSynchronize(st);
    if (e == hipSuccess) record_codec_times(ctx);
    return e == hipSuccess ? 0 : KV_COMPACT_E_DEVICE;
}

int kvc_compact_quantized_device(const uint8_t * K_quant, const uint8_t * V_quant, const float * Q_ref,
                                 int k_type, int v_type, size_t k_row_bytes, size_t v_row_bytes,
                                 int T, int n_q, int n_head_kv, int d_k, int d_v,
                                 const kv_compact_params * params, kvc_device_out * out,
                                 uint8_t * K_out, uint8_t * V_out, void * stream) {
    return kvc_compact_quantized_layers_device(K_quant, V_quant, Q_ref, 1, k_type, v_type, k_row_bytes, v_row_bytes,
                                               T, n_q, n_head_kv, d_k, d_v, (long long)T * k_row_bytes,
                                               (long long)T * v_row_bytes,
                                               (long long)std::max(n_q, 1) * n_head_kv * d_k, params, out, K_out,
                                               V_out, stream);
}

int kvc_stage_times(float * out_ms, int n) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return 0;
    DeviceCtx * c = &g_dev[dev];
    std::lock_guard<std::mutex> lk(c->mu);
    const int m = std::min(n, (int)ST_COUNT);
    for (int i = 0; i < m; i++) out_ms[i] = c->stage_ms[i];
    return m;
}

void kvc_release_workspace(void) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return;
    DeviceCtx * c = &g_dev[dev];
    std::lock_guard<std::mutex> lk(c->mu);
    if (c->arena) {
        (void)hipStreamSynchronize(c->stream);
        (void)hipStreamSynchronize(c->stream2);
        (void)hipFree(c->arena);
        c->arena = nullptr;
        c->arena_cap = 0;
    }
    free_pin_ring(c);
    c->pin_failed = false;
}

int kvc_live_objects(void) { return g_live.load(); }

}  // extern "C"

// ------------------------------------------------------- llama.cpp state blobs
//
// kvc_state_compact / _device: the reference CLI's compaction of a sequence
// state (src/kv-compact.cpp:380-690) and its write-back blob
// (build_compacted_state, include/kv-compact-state.h:645-810). The blob's
// headers and cell records are walked on the host (parsed_kv_state::parse,
// state.h:104-222); every K/V payload is decoded, compacted and re-encoded on
// the device.
namespace {

// Reads of a blob in host or device memory; device reads go through a host
// window so that the walk over headers and cell records costs few copies.
struct BlobReader {
    const uint8_t * p = nullptr;
    size_t size = 0;
    bool dev = false;
    bool dev_err = false;
    std::vector<uint8_t> win;
    size_t win_off = 0, win_len = 0;
    bool read(size_t off, void * dst, size_t n) {
        if (off > size || n > size - off) return false;
        if (!dev) {
            memcpy(dst, p + off, n);
            return true;
        }
        if (off < win_off || off + n > win_off + win_len) {
            // the first window covers the cell records; later reads are the
            // layers' headers, megabytes apart: small windows
            const size_t len = std::min(size - off, std::max(n, win_len == 0 ? (size_t)1 << 20 : (size_t)1 << 16));
            win.resize(len);
            if (hipMemcpy(win.data(), p + off, len, hipMemcpyDeviceToHost) != hipSuccess) {
                (void)hipGetLastError();
                dev_err = true;
                return false;
            }
            win_off = off;
            win_len = len;
        }
        memcpy(dst, win.data() + (off - win_off), n);
        return true;
    }
};

struct StateLayer {
    int32_t k_type = 0, v_type = 0;
    uint64_t k_rb = 0, v_rb = 0;   // row bytes (V: row-major layout)
    uint32_t v_el = 0, v_ne = 0;   // transposed V: element size, n_embd_v_gqa
    size_t k_off = 0, v_off = 0;   // payload offsets in the blob
    int nk = 0, nv = 0;            // elements per K / V row
};

struct StateLayout {
    uint32_t n_stream = 0, cells = 0, v_trans = 0, n_layer = 0;
    std::vector<size_t> cell_at;    // offset of each cell record
    std::vector<uint32_t> cell_len; // its bytes: pos, n_seq_id, [x, y], seq ids
    std::vector<StateLayer> layers;
    size_t kv_end = 0;
    bool extra_streams = false;     // a stream after the first holds cells
};

// elements per row of a stored type (state.h:342-352)
int state_row_elements(int32_t type, uint64_t rb) {
    if (type == KV_TYPE_F32) return (int)(rb / 4);
    if (type == KV_TYPE_F16) return (int)(rb / 2);
    if (is_block_type(type)) return (int)(rb / (uint64_t)block_bytes(type)) * 32;
    return (int)(rb / 4);
}

bool state_type_ok(int32_t t) {
    return t == KV_TYPE_F32 || t == KV_TYPE_F16 || is_block_type(t);
}

// parsed_kv_state::parse (state.h:104-222) without the payload decode.
// 0, -2 malformed, -6 device read failed. Stops at a second stream that holds
// cells (extra_streams).
int parse_state(BlobReader & r, uint32_t n_pos, StateLayout & s) {
    size_t off = 0;
    auto rd = [&](void * v, size_t n) {
        if (!r.read(off, v, n)) return false;
        off += n;
        return true;
    };
    auto fail = [&]() { return r.dev_err ? KV_COMPACT_E_DEVICE : -2; };
    if (!rd(&s.n_stream, 4)) return fail();
    for (uint32_t st = 0; st < s.n_stream; st++) {
        uint32_t cc = 0;
        if (!rd(&cc, 4)) return fail();
        if (cc == 0) continue;
        if (st > 0) {
            s.extra_streams = true;
            return 0;
        }
        // every cell record takes at least 8 bytes: a count beyond the blob
        // is malformed (checked before anything is sized by it)
        if (cc > (r.size - off) / 8) return -2;
        s.cells = cc;
        s.cell_at.resize(cc);
        s.cell_len.resize(cc);
        for (uint32_t c = 0; c < cc; c++) {
            s.cell_at[c] = off;
            int32_t pos = 0;
            uint32_t ns = 0;
            if (!rd(&pos, 4) || !rd(&ns, 4)) return fail();
            if (n_pos > 1) off += 8;
            if (off > r.size || (r.size - off) / 4 < ns) return fail();
            off += (size_t)ns * 4;
            s.cell_len[c] = (uint32_t)(off - s.cell_at[c]);
        }
        if (!rd(&s.v_trans, 4) || !rd(&s.n_layer, 4)) return fail();
        if (s.n_layer > (r.size - off) / 24) return -2;   // two headers of >= 12 bytes per layer
        s.layers.assign(s.n_layer, StateLayer());
        for (uint32_t l = 0; l < s.n_layer; l++) {
            StateLayer & ld = s.layers[l];
            if (!rd(&ld.k_type, 4) || !rd(&ld.k_rb, 8)) return fail();
            const uint64_t bytes = (uint64_t)cc * ld.k_rb;
            if (ld.k_rb != 0 && bytes / ld.k_rb != cc) return -2;
            if (bytes > r.size - off) return -2;
            ld.nk = state_row_elements(ld.k_type, ld.k_rb);
            ld.k_off = off;
            off += bytes;
        }
        for (uint32_t l = 0; l < s.n_layer; l++) {
            StateLayer & ld = s.layers[l];
            if (!rd(&ld.v_type, 4)) return fail();
            if (!s.v_trans) {
                if (!rd(&ld.v_rb, 8)) return fail();
                const uint64_t bytes = (uint64_t)cc * ld.v_rb;
                if (ld.v_rb != 0 && bytes / ld.v_rb != cc) return -2;
                if (bytes > r.size - off) return -2;
                ld.nv = state_row_elements(ld.v_type, ld.v_rb);
                ld.v_off = off;
                off += bytes;
            } else {
                if (!rd(&ld.v_el, 4) || !rd(&ld.v_ne, 4)) return fail();
                const uint64_t bytes = (uint64_t)ld.v_ne * cc * ld.v_el;
                if (bytes > r.size - off) return -2;
                // the flat decode must stay inside the section (a smaller
                // v_size_el would make the reference read past it)
                if ((uint64_t)ld.v_ne * cc >= (1ULL << 31) ||
                    (uint64_t)kv_quant_row_bytes(ld.v_type, (int)((uint64_t)ld.v_ne * cc)) > bytes)
                    return -2;
                ld.nv = (int)ld.v_ne;
                ld.v_off = off;
                off += bytes;
            }
        }
    }
    s.kv_end = off;
    return 0;
}

size_t row_written(int32_t type, int n) { return (size_t)kv_quant_row_bytes(type, n); }

// The output blob's sections (state.h:660-808), laid out from the parse and
// the kept cells.
struct StateOut {
    size_t cells_off = 0, total = 0;
    std::vector<size_t> k_hdr, k_pay, v_hdr, v_pay;   // per layer
    std::vector<size_t> k_w, v_w;                     // bytes per written row (V transposed: per column)
    size_t tail_off = 0;                              // empty streams, then the trailing bytes
};

StateOut plan_state_out(const StateLayout & s, const std::vector<int> & sel, int t, int H, int dv, size_t size) {
    StateOut o;
    size_t off = 8;   // n_stream, t
    o.cells_off = off;
    for (int j = 0; j < t; j++) off += s.cell_len[sel[j]];
    off += 8;         // v_trans, n_layer
    const int L = (int)s.n_layer;
    o.k_hdr.resize(L); o.k_pay.resize(L); o.v_hdr.resize(L); o.v_pay.resize(L);
    o.k_w.resize(L); o.v_w.resize(L);
    for (int l = 0; l < L; l++) {
        const StateLayer & ld = s.layers[l];
        o.k_hdr[l] = off;
        o.k_pay[l] = off + 12;
        o.k_w[l] = row_written(ld.k_type, ld.nk);
        off += 12 + (size_t)t * o.k_w[l];
    }
    for (int l = 0; l < L; l++) {
        const StateLayer & ld = s.layers[l];
        o.v_hdr[l] = off;
        o.v_pay[l] = off + 12;
        if (!s.v_trans) {
            o.v_w[l] = row_written(ld.v_type, ld.nv);
            off += 12 + (size_t)t * o.v_w[l];
        } else {
            o.v_w[l] = row_written(ld.v_type, t);
            off += 12 + (size_t)H * dv * o.v_w[l];
        }
    }
    o.tail_off = off;
    off += (size_t)(s.n_stream - 1) * 4 + (size - s.kv_end);
    o.total = off;
    return o;
}

// Decode one stored section into fp32 rows [T][n] (rows of rb bytes, or the
// transposed [n][T] run decoded flat and transposed through tmp).
void decode_rows(const uint8_t * src, int32_t type, uint64_t rb, int n, int T, float * dst, hipStream_t st) {
    const bool even = ((reinterpret_cast<uintptr_t>(src) | rb) & 1) == 0;
    if (codec8_ok(type, n) && even)
        launch_dequant8(src, type, (long long)rb, 0, n, T, 1, dst, st);
    else
        launch_dequant_rows(src, type, (long long)rb, n, T, dst, st);
}

// rows [t][n] fp32 (gathered by idx, or in order when idx is null) into a
// section of rows of w bytes
void encode_rows(const float * src, long long ld, const int * idx, const int * iota, int32_t type, int n, int t,
                 uint8_t * dst, size_t w, hipStream_t st) {
    const bool even = ((reinterpret_cast<uintptr_t>(dst) | w) & 1) == 0;
    const bool al = (reinterpret_cast<uintptr_t>(src) & 15) == 0 && (ld & 3) == 0;
    if (codec8_ok(type, n) && even && al)
        launch_requant8(src, 0, ld, idx ? idx : iota, 0, 0, 0, 1, type, n, t, 1, dst, (long long)w, 0, st);
    else
        launch_quant_rows(src, ld, idx, type, n, t, dst, (long long)w, st);
}

struct StateRun {
    int rc = 0;
    std::vector<int> sel;
    size_t out_size = 0;
};

// The whole call: blob (host or device, `dev`), output to a host buffer
// (*host_out, malloc'd) or to device memory (d_out, out_cap).
StateRun state_compact_impl(const uint8_t * blob, size_t size, bool dev, const kvc_state_params & sp,
                            void ** host_out, uint8_t * d_out, size_t out_cap, hipStream_t user_st) {
    StateRun run;
    auto done = [&](int rc) { run.rc = rc; return run; };
    DeviceCtx * ctx = device_ctx();
    if (!ctx) return done(KV_COMPACT_E_DEVICE);
    std::lock_guard<std::mutex> lk(ctx->mu);
    hipStream_t st = user_st ? user_st : ctx->stream;
    BlobReader rd;
    rd.p = blob; rd.size = size; rd.dev = dev;
    StateLayout s;
    int rc = parse_state(rd, sp.n_pos_per_embd, s);
    if (rc) return done(rc);
    if (s.extra_streams) return done(KV_COMPACT_E_UNSUPPORTED);
    if (s.cells == 0 || s.n_layer == 0) return done(-2);
    const int T = (int)s.cells, L = (int)s.n_layer, H = sp.n_head_kv;
    const int nk = s.layers[0].nk, nv = s.layers[0].nv;
    if (H <= 0 || nk <= 0 || nv <= 0 || nk % H || nv % H) return done(-2);
    for (const StateLayer & ld : s.layers)
        if (!state_type_ok(ld.k_type) || !state_type_ok(ld.v_type) || ld.nk != nk || ld.nv != nv)
            return done(KV_COMPACT_E_UNSUPPORTED);
    const int dk = nk / H, dv = nv / H;
    int t = (int)(T * sp.compact_ratio);
    if (t < 1) t = 1;
    int nq = sp.n_ref_queries;
    if (nq <= 0) nq = std::max(16, T / 4);
    nq = std::min(nq, T);
    if (t > T) return done(-2);
    if (nq > SOFTMAX_MAXQ) return done(KV_COMPACT_E_UNSUPPORTED);
    if (s.v_trans && (long long)nv * T >= (1LL << 31)) return done(KV_COMPACT_E_UNSUPPORTED);
    const int q0 = T - nq;
    // compacted layers take the first slots of the fp32 caches, kept layers the rest
    std::vector<int> slot(L), order;
    for (int l = 0; l < L; l++)
        if (!sp.layer_filter || sp.layer_filter(l, L, sp.layer_filter_data)) order.push_back(l);
    const int Lc = (int)order.size();
    for (int l = 0; l < L; l++)
        if (!(!sp.layer_filter || sp.layer_filter(l, L, sp.layer_filter_data))) order.push_back(l);
    for (int i = 0; i < L; i++) slot[order[i]] = i;

    // plans: the compaction (one chunk of all T cells keeping t, nq queries)
    // and the direction fits (d_k unknowns, nq rows, one right-hand side)
    kv_compact_params p = defaults();
    p.skip_beta = 1;
    p.score_method = 0;
    p.use_sensitivity = sp.sensitivity_budget ? 1 : 0;
    Plan pl;
    {
        pl.T = T; pl.n_chunks = 1; pl.t_total = t; pl.nq_max = nq; pl.tc_max = t; pl.Tc_max = T;
        pl.qmode = Q_PROVIDED; pl.nq_global = nq; pl.stats_qmode = Q_PROVIDED;
        ChunkDesc d;
        d.start = 0; d.Tc = T; d.tc = t; d.prefix = 0; d.nq = nq; d.off = 0;
        pl.chunks = {d, d, d};
        pl.chunks[2].Tc = t;
    }
    Plan pd;
    {
        pd.T = dk; pd.n_chunks = 1; pd.t_total = dk; pd.nq_max = nq; pd.tc_max = dk; pd.Tc_max = dk;
        pd.qmode = Q_PROVIDED; pd.nq_global = nq; pd.stats_qmode = Q_PROVIDED;
        ChunkDesc d;
        d.start = 0; d.Tc = dk; d.tc = dk; d.prefix = 0; d.nq = nq; d.off = 0;
        pd.chunks = {d, d, d};
    }
    BatchIO io{};
    io.L = Lc; io.T = T; io.n_q = nq; io.H = H; io.dk = dk; io.dv = dv;
    io.ldK = (long long)T * nk; io.ldV = (long long)T * nv; io.ldQ = (long long)T * nk;
    BatchIO iod{};
    iod.L = Lc; iod.T = dk; iod.n_q = nq; iod.H = H; iod.dk = dk; iod.dv = 1;
    kv_compact_params pdp = defaults();
    pdp.skip_beta = 1;

    // arena: blob copy (host input), fp32 caches, outputs, then the two
    // workspaces (the same carving sizes the arena and places the buffers)
    struct Bufs {
        uint8_t * blob = nullptr;
        float * Kf = nullptr, * Vf = nullptr, * vt_tmp = nullptr;
        int * idx = nullptr, * iota = nullptr;
        float * zbeta = nullptr, * beta_c = nullptr, * Cv = nullptr, * stats = nullptr, * dirs = nullptr;
        float * rows = nullptr, * cols = nullptr;
        uint8_t * stage = nullptr;
        Work w{}, wd{};
    };
    auto carve = [&](Carver & c, Bufs & b) {
        if (!dev) b.blob = c.take<uint8_t>(size);
        b.Kf = c.take<float>((size_t)L * T * nk);
        b.Vf = c.take<float>((size_t)L * T * nv);
        b.vt_tmp = s.v_trans ? c.take<float>((size_t)nv * T) : nullptr;
        b.idx = c.take<int>((size_t)std::max(Lc, 1) * t);
        b.iota = c.take<int>((size_t)t);
        b.zbeta = c.take<float>((size_t)H * t);
        b.beta_c = c.take<float>((size_t)std::max(Lc, 1) * H * t);
        b.Cv = c.take<float>((size_t)std::max(Lc, 1) * H * t * dv);
        b.stats = c.take<float>((size_t)std::max(Lc, 1) * 3);
        b.dirs = c.take<float>((size_t)L * H * dk);
        b.rows = c.take<float>((size_t)t * std::max(nk, nv));
        b.cols = c.take<float>((size_t)nv * t);
        b.stage = c.take<uint8_t>(size);   // the compacted blob is never larger than the input
        if (Lc > 0) {
            StatWork sw{};
            workspace_bytes(pl, io, &p, &c, &b.w, &sw);
            workspace_bytes(pd, iod, &pdp, &c, &b.wd, &sw);
        }
    };
    Bufs b;
    {
        Carver sz;
        Bufs dummy;
        carve(sz, dummy);
        if (!drain_second_stream(ctx, st)) return done(KV_COMPACT_E_DEVICE);
        if (!ensure_arena(ctx, sz.off + 256)) return done(KV_COMPACT_E_DEVICE);
        Carver c;
        c.base = ctx->arena;
        carve(c, b);
    }
    const uint8_t * dblob = blob;
    if (!dev) {
        if (!host_transfer(ctx, {{const_cast<uint8_t *>(blob), b.blob, size}}, true, st))
            return done(KV_COMPACT_E_DEVICE);
        dblob = b.blob;
    }
    float * Kf = b.Kf, * Vf = b.Vf, * vt_tmp = b.vt_tmp, * zbeta = b.zbeta, * Cv = b.Cv, * dirs = b.dirs;
    float * rows = b.rows, * cols = b.cols;
    int * idx = b.idx, * iota = b.iota;
    uint8_t * stage = b.stage;

    if (forced_fault("launch")) return done(KV_COMPACT_E_DEVICE);
    // 1. decode every layer's K and V into fp32 rows (slot order)
    (void)hipEventRecord(ctx->q_ev[0], st);
    for (int l = 0; l < L; l++) {
        const StateLayer & ld = s.layers[l];
        float * kd = Kf + (size_t)slot[l] * T * nk;
        float * vd = Vf + (size_t)slot[l] * T * nv;
        decode_rows(dblob + ld.k_off, ld.k_type, ld.k_rb, nk, T, kd, st);
        if (!s.v_trans) {
            decode_rows(dblob + ld.v_off, ld.v_type, ld.v_rb, nv, T, vd, st);
        } else {
            // [nv][T] decoded as one flat run (state.h:447-453; a block-coded
            // run leaves its last n % 32 values 0), then transposed
            launch_fill_f32(vt_tmp, 0.0f, (long long)nv * T, st);
            launch_dequant_rows(dblob + ld.v_off, ld.v_type, 0, nv * T, 1, vt_tmp, st);
            launch_transpose(vt_tmp, nv, T, vd, st);
        }
    }
    (void)hipEventRecord(ctx->q_ev[1], st);
    launch_fill_f32(zbeta, 0.0f, (long long)H * t, st);
    launch_fill_f32(dirs, 0.0f, (long long)L * H * dk, st);
    launch_iota(iota, t, st);

    // 2. scores, softmax and importance of the compacted layers; one global
    //    importance over all their heads; top-t; values and directions
    if (Lc > 0) {
        io.K = Kf; io.V = Vf; io.Q = Kf + (size_t)q0 * nk;
        io.indices = idx; io.Cv = Cv; io.stats = b.stats; io.beta = b.beta_c;
        Work & w = b.w;
        Work & wd = b.wd;
        w.sel = idx;
        w.wts = nullptr;
        Geom g{};
        g.L = Lc; g.T = T; g.H = H; g.dk = dk; g.dv = dv;
        g.n_chunks = 1; g.t_total = t; g.nq_max = nq; g.tc_max = t; g.Tc_max = T;
        g.qmode = Q_PROVIDED; g.nq_global = nq;
        g.ldK = io.ldK; g.ldV = io.ldV; g.ldQ = io.ldQ;
        g.score_method = 0;
        g.inv_sqrt_dk = 1.0f / sqrtf((float)dk);
        g.ridge = 1e-6f;   // least_squares_solve's default (math.h:463-464)
        g.zero_val = 0.0f;
        {
            const char * e = getenv("KVC_LU_MASKED");
            g.lu_masked = (e && e[0] == '1') ? 1 : 0;
        }
        std::vector<long long> aoff((size_t)Lc * H), doff((size_t)Lc * H);
        for (size_t i = 0; i < aoff.size(); i++) {
            aoff[i] = (long long)i * t * (t + dv);
            doff[i] = (long long)i * dk * (dk + 1);
        }
        if (hipMemcpyAsync(w.chunks, pl.chunks.data(), pl.chunks.size() * sizeof(ChunkDesc), hipMemcpyHostToDevice,
                           st) != hipSuccess ||
            hipMemcpyAsync(w.aug_off, aoff.data(), aoff.size() * 8, hipMemcpyHostToDevice, st) != hipSuccess ||
            hipMemcpyAsync(wd.chunks, pd.chunks.data(), pd.chunks.size() * sizeof(ChunkDesc), hipMemcpyHostToDevice,
                           st) != hipSuccess ||
            hipMemcpyAsync(wd.aug_off, doff.data(), doff.size() * 8, hipMemcpyHostToDevice, st) != hipSuccess)
            return done(KV_COMPACT_E_DEVICE);
        launch_fill_int(w.status, 0, 1, st);
        launch_fill_int(wd.status, 0, 1, st);
        launch_scores(g, w.chunks, 1, T, io.K, io.Q, w.S, H, nq, (long long)H * nq * T, (long long)nq * T, T,
                      Q_PROVIDED, st, nullptr, nullptr, w.smax);
        launch_chunk_softmax(g, w, st);
        // every (layer, head) of the compacted layers as one head list
        Geom gg = g;
        gg.L = 1;
        gg.H = Lc * H;
        launch_global_importance(gg, w, st);
        launch_select_topk(gg, w, st);
        for (int l = 1; l < Lc; l++)
            if (hipMemcpyAsync(idx + (size_t)l * t, idx, (size_t)t * 4, hipMemcpyDeviceToDevice, st) != hipSuccess)
                return done(KV_COMPACT_E_DEVICE);
        launch_refit_target(g, w, io.V, st);
        launch_fill_f32(b.beta_c, 0.0f, (long long)Lc * H * t, st);
        launch_ls_softmax(g, w, b.beta_c, st);
        launch_ls_build(g, w, st, true);
        launch_ge_lu(g, w, st, true);
        launch_ge_solve(g, w, Cv, st);
        // beta directions: ridge LS of each head's reference queries against 1
        Geom gd{};
        gd.L = Lc; gd.T = dk; gd.H = H; gd.dk = dk; gd.dv = 1;
        gd.n_chunks = 1; gd.t_total = dk; gd.nq_max = nq; gd.tc_max = dk; gd.Tc_max = dk;
        gd.qmode = Q_PROVIDED; gd.nq_global = nq;
        gd.ridge = 1e-6f;
        gd.zero_val = 0.0f;
        gd.lu_masked = g.lu_masked;
        launch_gather_qref(Kf, io.ldK, nk, q0, nq, H, dk, Lc, wd.X, st);
        launch_fill_f32(wd.Y, 1.0f, (long long)Lc * H * nq, st);
        launch_ls_build(gd, wd, st, true);
        launch_ge_lu(gd, wd, st, true);
        launch_ge_solve(gd, wd, dirs, st);   // slots 0 .. Lc - 1 are the compacted layers
        int status[2] = {0, 0};
        if (hipStreamSynchronize(st) != hipSuccess ||
            hipMemcpy(&status[0], w.status, 4, hipMemcpyDeviceToHost) != hipSuccess ||
            hipMemcpy(&status[1], wd.status, 4, hipMemcpyDeviceToHost) != hipSuccess) {
            (void)hipGetLastError();
            return done(KV_COMPACT_E_DEVICE);
        }
        if ((status[0] | status[1]) & 2) {
            fprintf(stderr, "[kv-compact] LU step wait exceeded its bound\n");
            return done(KV_COMPACT_E_DEVICE);
        }
        if (status[0] | status[1]) return done(KV_COMPACT_E_UNSUPPORTED);
    } else {
        // no layer compacted: the importance is 0 everywhere, and partial_sort
        // over equal keys keeps the first t positions (its heap moves never
        // bring in an element that does not compare greater)
        run.sel.resize(t);
        for (int j = 0; j < t; j++) run.sel[j] = j;
        if (hipMemcpyAsync(idx, run.sel.data(), (size_t)t * 4, hipMemcpyHostToDevice, st) != hipSuccess ||
            hipStreamSynchronize(st) != hipSuccess)
            return done(KV_COMPACT_E_DEVICE);
    }
    if (run.sel.empty()) {
        run.sel.resize(t);
        if (hipMemcpyAsync(run.sel.data(), idx, (size_t)t * 4, hipMemcpyDeviceToHost, st) != hipSuccess ||
            hipStreamSynchronize(st) != hipSuccess)
            return done(KV_COMPACT_E_DEVICE);
    }

    // 3. the output blob, staged in device memory with the final offsets
    const StateOut o = plan_state_out(s, run.sel, t, H, dv, size);
    run.out_size = o.total;
    if (o.total > size) return done(-2);   // not reached: every section shrinks or keeps its size
    if (!host_out && o.total > out_cap) return done(KVC_E_CAPACITY);
    std::vector<uint8_t> hdr(o.k_hdr.empty() ? 16 : o.k_hdr[0]);
    {
        uint32_t v2[2] = {s.n_stream, (uint32_t)t};
        memcpy(hdr.data(), v2, 8);
        size_t off = o.cells_off;
        BlobReader cr;
        cr.p = blob; cr.size = size; cr.dev = dev;
        for (int j = 0; j < t; j++) {
            const int c = run.sel[j];
            if (!cr.read(s.cell_at[c], hdr.data() + off, s.cell_len[c])) return done(KV_COMPACT_E_DEVICE);
            off += s.cell_len[c];
        }
        v2[0] = s.v_trans;
        v2[1] = s.n_layer;
        memcpy(hdr.data() + off, v2, 8);
    }
    if (hipMemcpyAsync(stage, hdr.data(), hdr.size(), hipMemcpyHostToDevice, st) != hipSuccess)
        return done(KV_COMPACT_E_DEVICE);
    std::vector<uint8_t> lh((size_t)2 * L * 16);
    (void)hipEventRecord(ctx->q_ev[2], st);
    const float scale = sqrtf((float)dk);
    for (int l = 0; l < L; l++) {
        const StateLayer & ld = s.layers[l];
        uint8_t * kh = lh.data() + (size_t)l * 16;
        memcpy(kh, &ld.k_type, 4);
        memcpy(kh + 4, &ld.k_rb, 8);
        if (hipMemcpyAsync(stage + o.k_hdr[l], kh, 12, hipMemcpyHostToDevice, st) != hipSuccess)
            return done(KV_COMPACT_E_DEVICE);
        const int sl = slot[l];
        const int * sidx = idx;   // row 0: every layer keeps the same cells
        launch_fold_rows(Kf + (size_t)sl * T * nk, nk, sidx, t, zbeta, dirs + (size_t)sl * H * dk, H, dk, scale,
                         rows, st);
        encode_rows(rows, nk, nullptr, iota, ld.k_type, nk, t, stage + o.k_pay[l], o.k_w[l], st);
        // the fold reads `rows` before the value rows overwrite it: same stream
    }
    for (int l = 0; l < L; l++) {
        const StateLayer & ld = s.layers[l];
        uint8_t * vh = lh.data() + (size_t)(L + l) * 16;
        memcpy(vh, &ld.v_type, 4);
        const int sl = slot[l];
        const bool comp = sl < Lc;
        const float * cvl = comp ? Cv + (size_t)sl * H * t * dv : nullptr;
        const float * vl = Vf + (size_t)sl * T * nv;
        if (!s.v_trans) {
            memcpy(vh + 4, &ld.v_rb, 8);
            if (comp) {
                launch_gather_cv_rows(cvl, H, t, dv, rows, st);
                encode_rows(rows, nv, nullptr, iota, ld.v_type, nv, t, stage + o.v_pay[l], o.v_w[l], st);
            } else {
                encode_rows(vl, nv, idx, iota, ld.v_type, nv, t, stage + o.v_pay[l], o.v_w[l], st);
            }
        } else {
            const uint32_t ne = (uint32_t)(H * dv);
            memcpy(vh + 4, &ld.v_el, 4);
            memcpy(vh + 8, &ne, 4);
            launch_value_columns(cvl, vl, nv, idx, H, dv, t, cols, st);
            launch_quant_rows(cols, t, nullptr, ld.v_type, t, (long long)ne, stage + o.v_pay[l],
                              (long long)o.v_w[l], st);
        }
        if (hipMemcpyAsync(stage + o.v_hdr[l], vh, 12, hipMemcpyHostToDevice, st) != hipSuccess)
            return done(KV_COMPACT_E_DEVICE);
    }
    (void)hipEventRecord(ctx->q_ev[3], st);
    // empty streams and the trailing bytes
    std::vector<uint8_t> zeros((size_t)(s.n_stream - 1) * 4, 0);
    if (!zeros.empty() &&
        hipMemcpyAsync(stage + o.tail_off, zeros.data(), zeros.size(), hipMemcpyHostToDevice, st) != hipSuccess)
        return done(KV_COMPACT_E_DEVICE);
    const size_t trail = size - s.kv_end;
    if (trail && hipMemcpyAsync(stage + o.tail_off + zeros.size(), dblob + s.kv_end, trail,
                                hipMemcpyDeviceToDevice, st) != hipSuccess)
        return done(KV_COMPACT_E_DEVICE);
    if (host_out) {
        uint8_t * out = (uint8_t *)malloc(std::max<size_t>(o.total, 1));
        if (!out) return done(-1);
        if (!host_transfer(ctx, {{out, stage, o.total}}, false, st)) {
            free(out);
            return done(KV_COMPACT_E_DEVICE);
        }
        *host_out = out;
    } else {
        if (hipMemcpyAsync(d_out, stage, o.total, hipMemcpyDeviceToDevice, st) != hipSuccess ||
            hipStreamSynchronize(st) != hipSuccess)
            return done(KV_COMPACT_E_DEVICE);
    }
    record_codec_times(ctx);
    return done(0);
}

}  // namespace

extern "C" {

int kvc_state_parse_info(const void * blob, size_t size, uint32_t n_pos_per_embd, kvc_state_info * info) {
    if (!blob || !info) return -1;
    BlobReader rd;
    rd.p = static_cast<const uint8_t *>(blob);
    rd.size = size;
    rd.dev = is_device_ptr(blob);
    StateLayout s;
    const int rc = parse_state(rd, n_pos_per_embd, s);
    memset(info, 0, sizeof(*info));
    if (rc) return rc;
    if (s.extra_streams) return KV_COMPACT_E_UNSUPPORTED;
    info->n_stream = s.n_stream;
    info->cell_count = s.cells;
    info->v_trans = s.v_trans;
    info->n_layer = s.n_layer;
    if (s.n_layer > 0) {
        info->n_embd_k = s.layers[0].nk;
        info->n_embd_v = s.layers[0].nv;
    }
    info->kv_bytes = s.kv_end;
    info->trailing_bytes = size - s.kv_end;
    return 0;
}

int kvc_state_compact(const void * blob, size_t size, const kvc_state_params * sp, void ** out, size_t * out_size,
                      int32_t * selected) {
    if (!blob || !sp || !out || !out_size) return -1;
    *out = nullptr;
    *out_size = 0;
    StateRun r = state_compact_impl(static_cast<const uint8_t *>(blob), size, false, *sp, out, nullptr, 0, nullptr);
    if (r.rc) return r.rc;
    *out_size = r.out_size;
    if (selected) memcpy(selected, r.sel.data(), r.sel.size() * sizeof(int32_t));
    return 0;
}

int kvc_state_compact_device(const void * d_blob, size_t size, const kvc_state_params * sp, void * d_out,
                             size_t out_cap, size_t * out_size, int32_t * selected, void * stream) {
    if (!d_blob || !sp || !d_out || !out_size) return -1;
    if (!is_device_ptr(d_blob) || !is_device_ptr(d_out)) return -1;
    StateRun r = state_compact_impl(static_cast<const uint8_t *>(d_blob), size, true, *sp, nullptr,
                                    static_cast<uint8_t *>(d_out), out_cap, (hipStream_t)stream);
    *out_size = r.out_size;
    if (r.rc) return r.rc;
    if (selected) memcpy(selected, r.sel.data(), r.sel.size() * sizeof(int32_t));
    return 0;
}

void kvc_state_free(void * out) { free(out); }

}  // extern "C"
