// C ABI of the MI355X routed-expert lane: context, resident bank and the lane
// entry points. Host side of the drop-in boundary declared in include/crosslane.h.
//
// Reference interfaces replaced (engine/strata/...):
//   warm/runtime.hpp:10-16                 WarmRedirect (contains / compute / compute_many)
//   sycl/stage/wiring/hip_resident_bank.hpp HipResidentBank (load :38-142, expert :143-166,
//                                          enqueue_layer :170-236)
//   warm/runtime.cpp:180-188               fixed-order combine
//   sycl/stage/wiring/hip_q8k.hpp:6-10     q8k::{quantize, mv}
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <fstream>
#include <map>
#include <new>
#include <set>
#include <sstream>
#include <stdexcept>
#include <string>
#include <vector>

#include "../../include/crosslane.h"
#include "xl_format.hpp"
#include "xl_internal.hpp"

namespace {

struct Failure : std::runtime_error {
    int32_t code;
    Failure(int32_t c, const std::string& m) : std::runtime_error(m), code(c) {}
};

[[noreturn]] void fail(int32_t code, const char* fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    std::vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    throw Failure(code, buf);
}
void need(bool ok, int32_t code, const char* what) {
    if (!ok) fail(code, "%s", what);
}
void hip_check(hipError_t e, const char* what) {
    if (e != hipSuccess) fail(XL_E_HIP, "%s: %s", what, hipGetErrorString(e));
}

#include "xl_codebooks.inc"

uint64_t expand_codes(unsigned short code, bool iq1) {
    static const uint8_t mag[3] = {8, 25, 43};
    static const uint8_t tri[3] = {0xff, 0x00, 0x01};
    uint64_t v = 0;
    for (int j = 0; j < 8; ++j) {
        const unsigned s = (code >> (2 * j)) & 3u;
        if (s > 2) throw Failure(XL_E_STATE, "corrupt codebook symbol");
        v |= uint64_t(iq1 ? tri[s] : mag[s]) << (8 * j);
    }
    return v;
}
uint8_t ksigns(int i) { return uint8_t(i | ((__builtin_popcount(unsigned(i)) & 1) << 7)); }

// Device table rows: IQ2_XXS grid, IQ2_XS grid, IQ1 grid, 128 sign masks.
std::vector<uint64_t> device_tables() {
    std::vector<uint64_t> t;
    t.reserve(2944);
    for (int i = 0; i < 256; ++i) t.push_back(expand_codes(kIq2xxsCodes[i], false));
    for (int i = 0; i < 512; ++i) t.push_back(expand_codes(kIq2xsCodes[i], false));
    for (int i = 0; i < 2048; ++i) t.push_back(expand_codes(kIq1sCodes[i], true));
    for (int i = 0; i < 128; ++i) {
        const uint8_t s = ksigns(i);
        uint64_t m = 0;
        for (int j = 0; j < 8; ++j)
            if (s & (1u << j)) m |= uint64_t(0xff) << (8 * j);
        t.push_back(m);
    }
    return t;
}

// Expanded codebooks of the single-launch kernels (byte layout kG_* in
// xl_layer.hip), one copy each: sign rows {M, M & 0x01..01} where M has 0xff in
// the bytes of negative weights, then the IQ2_XXS, IQ2_XS and IQ1 grids, then
// the streaming kernels' IQ1_M value rows (at kTableIQ1X).
std::vector<uint64_t> layer_tables() {
    std::vector<uint64_t> t;
    t.reserve(xl::kTableBytes / 8);
    for (int i = 0; i < 128; ++i) {
        const uint8_t sg = ksigns(i);
        uint64_t m = 0;
        for (int j = 0; j < 8; ++j)
            if (sg & (1u << j)) m |= uint64_t(0xff) << (8 * j);
        t.push_back(m);
        t.push_back(m & 0x0101010101010101ull);
    }
    for (int i = 0; i < 256; ++i) t.push_back(expand_codes(kIq2xxsCodes[i], false));
    for (int i = 0; i < 512; ++i) t.push_back(expand_codes(kIq2xsCodes[i], false));
    for (int i = 0; i < 2048; ++i) t.push_back(expand_codes(kIq1sCodes[i], true));
    if (t.size() * 8 != size_t(xl::kLayer3TableBytes)) throw Failure(XL_E_STATE, "expanded table size");
    // IQ1_M value rows: row (nib << 8 | lo) holds 8 * grid[(nib & 7) << 8 | lo] + delta,
    // delta = -1 when bit 3 of the nibble is set, else +1 (one byte per weight)
    for (int nib = 0; nib < 16; ++nib)
        for (int lo = 0; lo < 256; ++lo) {
            const uint64_t g = expand_codes(kIq1sCodes[((nib & 7) << 8) | lo], true);
            uint64_t v = 0;
            for (int j = 0; j < 8; ++j) {
                const int s = int(int8_t(uint8_t(g >> (8 * j))));
                v |= uint64_t(uint8_t(int8_t(8 * s + ((nib & 8) ? -1 : 1)))) << (8 * j);
            }
            t.push_back(v);
        }
    if (t.size() * 8 != size_t(xl::kTableBytes)) throw Failure(XL_E_STATE, "expanded table size");
    return t;
}

int env_int(const char* name, int fallback) {
    const char* s = std::getenv(name);
    if (!s || !*s) return fallback;
    char* end = nullptr;
    const long v = std::strtol(s, &end, 10);
    if (*end || v < 0 || v > 1 << 20) fail(XL_E_ARG, "%s must be a non-negative integer", name);
    return int(v);
}

uint64_t matrix_blocks(int n, int k) { return uint64_t(n) * uint64_t(k / 256); }

}  // namespace

// A layer whose experts all share one type triple has every expert's three
// matrices at slab + id * estride + roff[role].
struct LayerShape {
    bool regular = false;
    uint64_t estride = 0, roff[3] = {0, 0, 0};
    int rtype[3] = {0, 0, 0};
};

struct xl_context {
    xl_config cfg{};
    int cus = 0;
    hipStream_t stream = nullptr;
    bool poisoned = false;
    xl_error last{};
    // workspace (one allocation, carved)
    void* ws = nullptr;
    uint64_t ws_bytes = 0;
    uint16_t* codes = nullptr;   // compact codebooks (2-bit symbols), expanded into LDS by the kernels
    int* err_flag = nullptr;
    float *x = nullptr, *xd = nullptr, *h = nullptr, *hd = nullptr, *g = nullptr, *u = nullptr, *y = nullptr;
    float *out = nullptr, *shared = nullptr, *w = nullptr, *mv_x = nullptr;
    int8_t *xq = nullptr, *hq = nullptr;
    int32_t* ids = nullptr;
    uint8_t* q8std = nullptr;
    int act_max = 0;  // longest vector the activation workspace holds
    // bank
    bool bank_ready = false, generated = false;
    std::vector<int32_t> types;
    std::vector<uint8_t*> slabs;
    std::vector<xl::ExpertDesc> descs;
    std::vector<int> gu_mask, dn_mask;   // per layer: block types among gate/up and among down matrices
    std::vector<LayerShape> layer_shape; // per layer: regular-layout addressing (see Layer3Args)
    xl::ExpertDesc* d_descs = nullptr;
    uint64_t payload = 0, allocated = 0;
    int grid_gu = 0, grid_down = 0;
    // Layer path: 1 = single launch (default: the streaming kernel of
    // xl_stream.hpp where it has an instance for the layer, else the all-types
    // kernel of xl_layer.hip, else separate launches), 3 = the all-types single
    // launch only, 4 = the streaming kernel only (a layer it cannot run is an
    // error), 0 = separate launches. XL_LAYER_PATH selects; shapes without a
    // single-launch instance use separate launches.
    int path = 1;
    // Grouped path: 1 = the MFMA kernels where the layer's types allow, else one
    // layer call per token (default); 0 = per-token calls only; 2 = the MFMA
    // kernels only (a layer they cannot run is an error). XL_GROUPED_PATH selects.
    int gpath = 1;
    float* hbuf = nullptr;      // streaming kernel's h exchange (2 x kHBufWords, sentinel-filled)
    // grouped path (xl_grouped.hip), sized by max_tokens * max_picks pairs
    struct Group {
        int32_t* ids = nullptr; float* w = nullptr; float* x = nullptr; float* shared = nullptr; float* out = nullptr;
        int8_t* xq = nullptr; float* xd = nullptr;
        int32_t* order = nullptr; int32_t* pos = nullptr; int4* tasks = nullptr; int32_t* n_tasks = nullptr;
        float* h = nullptr; int8_t* hq = nullptr; float* hd = nullptr; float* y = nullptr;
        uint64_t hq_bytes = 0;
    } grp;
    uint64_t* htag = nullptr;   // single-launch handoff buffers (Layer3Args)
    uint64_t* hqtag = nullptr;
    uint64_t* hdtag = nullptr;
    uint32_t* ctl = nullptr;
    uint64_t* tables = nullptr;
    float* p32d = nullptr;      // per32 scales: act_max / 32 of the input, then max_picks * ff / 32 of h
    uint64_t* timeline = nullptr;   // per-wave timestamps of the last profiled single launch
    uint64_t timeline_words = 0;
    // stage profiling (xl_profile_begin / xl_profile_end): events recorded
    // around every kernel of the layer calls, on the stream they run on.
    struct Prof {
        bool on = false;
        int max_calls = 0, calls = 0, stages = 0;
        std::vector<hipEvent_t> ev;      // max_calls * (kMaxStages + 1)
        std::vector<std::string> names;
    } prof;
    // Call ordering across streams: every device call records `done` on its
    // stream when it has been enqueued; a call on another stream first waits
    // for it, so the calls of one context never overlap whatever streams they
    // name (they share the workspace, the exchange buffers and the counters).
    hipEvent_t done = nullptr;
    hipStream_t last_stream = nullptr;
    bool has_last = false;
    // Layer calls by the way they ran (XL_LAUNCH_*), for xl_debug_launch_counts.
    int64_t launches[XL_LAUNCH_KINDS] = {};
};

namespace {

constexpr int kMaxStages = 8;

// Stage marks: call mark(ctx, s, i) before stage i (i = 0) and after it.
struct Marks {
    xl_context* ctx;
    hipStream_t s;
    int slot = -1, n = 0;
    Marks(xl_context* c, hipStream_t st) : ctx(c), s(st) {
        if (ctx->prof.on && ctx->prof.calls < ctx->prof.max_calls) slot = ctx->prof.calls++;
    }
    void operator()(const char* name) {
        if (slot < 0) return;
        if (n > 0 && int(ctx->prof.names.size()) < n) ctx->prof.names.emplace_back(name);
        if (n <= kMaxStages) hip_check(hipEventRecord(ctx->prof.ev[size_t(slot) * (kMaxStages + 1) + n], s), "event record");
        if (n > ctx->prof.stages) ctx->prof.stages = n;
        ++n;
    }
};

void set_error(xl_context* ctx, xl_error* err, int32_t code, const char* msg) {
    xl_error e{};
    e.code = code;
    std::snprintf(e.message, sizeof e.message, "%s", msg);
    if (ctx) ctx->last = e;
    if (err) *err = e;
}

template <class F>
int32_t guarded(xl_context* ctx, xl_error* err, F&& f) {
    try {
        if (err) { err->code = XL_OK; err->message[0] = 0; }
        f();
        return XL_OK;
    } catch (const Failure& e) {
        if (ctx && (e.code == XL_E_HIP || e.code == XL_E_DEVICE)) {
            // Poison: drain whatever is queued, refuse further compute.
            ctx->poisoned = true;
            if (ctx->stream) (void)hipStreamSynchronize(ctx->stream);
        }
        set_error(ctx, err, e.code, e.what());
        return e.code;
    } catch (const std::bad_alloc&) {
        set_error(ctx, err, XL_E_MEMORY, "host allocation failed");
        return XL_E_MEMORY;
    } catch (const std::exception& e) {
        set_error(ctx, err, XL_E_STATE, e.what());
        return XL_E_STATE;
    } catch (...) {
        set_error(ctx, err, XL_E_STATE, "unknown exception");
        return XL_E_STATE;
    }
}

void ready(const xl_context* ctx, bool need_bank) {
    need(ctx != nullptr, XL_E_ARG, "null context");
    need(!ctx->poisoned, XL_E_STATE, "context poisoned by an earlier device error; close it");
    if (need_bank) need(ctx->bank_ready, XL_E_STATE, "bank not created");
    hip_check(hipSetDevice(ctx->cfg.device), "hipSetDevice");
}

hipStream_t pick_stream(const xl_context* ctx, void* s) { return s ? static_cast<hipStream_t>(s) : ctx->stream; }

// Orders one call's device work after the context's previous call (see
// xl_context::done): waits on another stream's last call at construction,
// records this call's end at destruction (also when the call failed part way:
// what it enqueued is then ordered too).
struct Ordered {
    xl_context* ctx;
    hipStream_t s;
    bool carried = false;   // the call's last launch already carries `done` as its stop event
    Ordered(xl_context* c, hipStream_t st) : ctx(c), s(st) {
        if (ctx->has_last && ctx->last_stream != s) hip_check(hipStreamWaitEvent(s, ctx->done, 0), "order after the previous call");
    }
    // The single-launch layer calls hand `done` to the launch itself (no marker
    // packet between back-to-back layers); other calls record it here.
    hipEvent_t stop() const { return ctx->done; }
    void carried_by_launch(bool yes) { carried = yes; }
    ~Ordered() {
        if (carried || hipEventRecord(ctx->done, s) == hipSuccess) {
            ctx->last_stream = s;
            ctx->has_last = true;
        }
    }
    Ordered(const Ordered&) = delete;
    Ordered& operator=(const Ordered&) = delete;
};

// Reads and checks the device error flag after draining the stream.
void drain(xl_context* ctx, hipStream_t s) {
    hip_check(hipStreamSynchronize(s), "stream synchronize");
    int flag = 0;
    hip_check(hipMemcpy(&flag, ctx->err_flag, sizeof flag, hipMemcpyDeviceToHost), "error flag read");
    if (flag) {
        fail(XL_E_DEVICE, "device error flag 0x%x (%s%s%s%s)", flag, (flag & xl::kDevErrExpertId) ? "expert id out of range " : "",
             (flag & xl::kDevErrNonFinite) ? "non-finite activation " : "", (flag & xl::kDevErrType) ? "bad block type " : "", (flag & xl::kDevErrTimeout) ? "layer wait timeout" : "");
    }
}

// Whether byte ranges [p, p + pb) and [q, q + qb) are disjoint.
bool apart(const void* p, uint64_t pb, const void* q, uint64_t qb) {
    const uintptr_t a = reinterpret_cast<uintptr_t>(p), b = reinterpret_cast<uintptr_t>(q);
    return a <= b ? b - a >= pb : a - b >= qb;
}

void check_ids(const xl_context* ctx, const int32_t* ids, int32_t k) {
    need(ids != nullptr, XL_E_ARG, "null ids");
    need(k >= 1 && k <= ctx->cfg.max_picks, XL_E_ARG, "pick count outside 1..max_picks");
    std::set<int32_t> seen;
    for (int i = 0; i < k; ++i) {
        need(ids[i] >= 0 && ids[i] < ctx->cfg.n_experts, XL_E_ARG, "expert id out of range");
        need(seen.insert(ids[i]).second, XL_E_ARG, "duplicate expert id");
    }
}
void check_finite(const float* v, size_t n, const char* what) {
    need(v != nullptr, XL_E_ARG, what);
    for (size_t i = 0; i < n; ++i)
        if (!std::isfinite(v[i])) fail(XL_E_ARG, "%s: non-finite value at %zu", what, i);
}
void check_layer(const xl_context* ctx, int32_t layer) {
    need(layer >= 0 && layer < ctx->cfg.n_layers, XL_E_ARG, "layer out of range");
}

// Enqueues the routed-expert layer on stream s: Q8_K(x), gate/up + SwiGLU,
// Q8_K(h), down, fixed-order combine. All pointers are device pointers.
// Parity trace outputs of one single-launch layer call (Layer3Args::tq8x ...),
// and which kernel ran (1 streaming, 3 all-types).
struct LayerTrace {
    uint8_t* q8x = nullptr;
    uint8_t* q8h = nullptr;
    float* h = nullptr;
    int32_t* ints = nullptr;
    float* y = nullptr;   // per-pick (per-pair) rows before the combine
    int kernel = 0;
};

// Returns true when the layer ran as one launch carrying `stop` (recorded as it
// completes); false when it took separate launches, which leave `stop` alone.
// With `tr`, the layer must run as one launch (XL_E_ARG otherwise).
// Arguments of the single-launch layer kernels for one layer call.
xl::Layer3Args layer3_args(xl_context* ctx, int32_t layer, const int32_t* d_ids, const float* d_w, int32_t k,
                           const float* d_x, const float* d_shared, float* d_out, hipStream_t s, LayerTrace* tr) {
    const int E = ctx->cfg.n_experts;
    xl::Layer3Args a{};
    a.descs = ctx->d_descs + size_t(layer) * E; a.ids = d_ids; a.w = d_w; a.x = d_x; a.shared = d_shared; a.out = d_out;
    a.k = k; a.n_experts = E; a.dim = ctx->cfg.dim; a.ff = ctx->cfg.ff;
    a.htag = ctx->htag; a.hqtag = ctx->hqtag; a.hdtag = ctx->hdtag; a.ctl = ctx->ctl; a.err = ctx->err_flag;
    a.lim = ctx->cfg.swiglu_limit;
    a.tables = ctx->tables;
    a.hbuf = ctx->hbuf;
    if (ctx->prof.on && ctx->prof.calls <= ctx->prof.max_calls) {
        a.trace = ctx->timeline;
        hip_check(hipMemsetAsync(ctx->timeline, 0, size_t(ctx->cus) * 16 * 32 * 8, s), "timeline clear");
    }
    if (tr) { a.tq8x = tr->q8x; a.tq8h = tr->q8h; a.th = tr->h; a.tint = tr->ints; a.ty = tr->y; }
    const LayerShape& ls = ctx->layer_shape[size_t(layer)];
    if (ls.regular) {
        a.slab = ctx->slabs[size_t(layer)];
        a.estride = ls.estride;
        for (int r = 0; r < 3; ++r) { a.roff[r] = ls.roff[r]; a.rtype[r] = ls.rtype[r]; }
    }
    return a;
}

// A routed layer call as one streaming launch that routes in its prologue
// (every wave from the logits): true if launched (it records `stop`), false
// if this layer or expert count has no such launch, or while stages are
// profiled (the router then runs as its own stage).
bool enqueue_layer_routed(xl_context* ctx, int32_t layer, const float* d_logits, const float* d_bias, int32_t k,
                          float scale, const float* d_x, const float* d_shared, float* d_out, hipStream_t s,
                          hipEvent_t stop) {
    if (ctx->cfg.n_experts > xl::kStreamRouteMax || (ctx->path != 1 && ctx->path != 4) || ctx->prof.on) return false;
    // ids and w are not read when routed; valid buffers all the same
    xl::Layer3Args a = layer3_args(ctx, layer, ctx->ids, ctx->w, k, d_x, d_shared, d_out, s, nullptr);
    a.rlogits = d_logits;
    a.rbias = d_bias;
    a.rscale = scale;
    const hipError_t e = xl::dev::launch_stream(a, ctx->gu_mask[size_t(layer)], ctx->dn_mask[size_t(layer)], ctx->cus, s,
                                                stop);
    if (e == hipErrorNotSupported) {
        (void)hipGetLastError();
        return false;
    }
    hip_check(e, "routed streaming layer");
    ++ctx->launches[XL_LAUNCH_ROUTED];
    return true;
}

// A layer call whose x is the pre-norm of one stream, as one streaming launch
// that normalizes in its prologue (workgroup 0 writes x to d_x): true if
// launched (it records `stop`), false if this layer has no such launch, or
// while stages are profiled.
bool enqueue_layer_prenorm(xl_context* ctx, int32_t layer, const int32_t* d_ids, const float* d_w, int32_t k,
                           const float* d_h, const float* d_mix, const float* d_norm_w, float eps, float* d_x,
                           const float* d_shared, float* d_out, hipStream_t s, hipEvent_t stop) {
    if ((ctx->path != 1 && ctx->path != 4) || ctx->prof.on) return false;
    xl::Layer3Args a = layer3_args(ctx, layer, d_ids, d_w, k, d_x, d_shared, d_out, s, nullptr);
    a.pn_h = d_h;
    a.pn_mix = d_mix;
    a.pn_w = d_norm_w;
    a.pn_x = d_x;
    a.pn_eps = eps;
    const hipError_t e = xl::dev::launch_stream(a, ctx->gu_mask[size_t(layer)], ctx->dn_mask[size_t(layer)], ctx->cus, s,
                                                stop);
    if (e == hipErrorNotSupported) {
        (void)hipGetLastError();
        return false;
    }
    hip_check(e, "pre-normed streaming layer");
    ++ctx->launches[XL_LAUNCH_PRENORM];
    return true;
}

// A layer call followed by hc_post of its output, as one streaming launch
// whose combine applies hc_post to its rows: true if launched (it records
// `stop`), false if this layer has no such launch, or while stages are profiled.
bool enqueue_layer_post(xl_context* ctx, int32_t layer, const int32_t* d_ids, const float* d_w, int32_t k,
                        const float* d_x, const float* d_shared, float* d_out, const float* d_res, const float* d_post,
                        const float* d_comb, int32_t H, float* d_post_out, hipStream_t s, hipEvent_t stop) {
    if ((ctx->path != 1 && ctx->path != 4) || ctx->prof.on) return false;
    xl::Layer3Args a = layer3_args(ctx, layer, d_ids, d_w, k, d_x, d_shared, d_out, s, nullptr);
    a.po_res = d_res;
    a.po_post = d_post;
    a.po_comb = d_comb;
    a.po_out = d_post_out;
    a.po_H = H;
    const hipError_t e = xl::dev::launch_stream(a, ctx->gu_mask[size_t(layer)], ctx->dn_mask[size_t(layer)], ctx->cus, s,
                                                stop);
    if (e == hipErrorNotSupported) {
        (void)hipGetLastError();
        return false;
    }
    hip_check(e, "streaming layer with hc_post");
    ++ctx->launches[XL_LAUNCH_POST];
    return true;
}

bool enqueue_layer(xl_context* ctx, int32_t layer, const int32_t* d_ids, const float* d_w, int32_t k, const float* d_x,
                   const float* d_shared, float* d_out, hipStream_t s, float* g_dbg = nullptr,
                   float* u_dbg = nullptr, hipEvent_t stop = nullptr, LayerTrace* tr = nullptr) {
    const int dim = ctx->cfg.dim, ff = ctx->cfg.ff, E = ctx->cfg.n_experts;
    const xl::ExpertDesc* descs = ctx->d_descs + size_t(layer) * E;
    const int gu_mask = ctx->gu_mask[size_t(layer)], dn_mask = ctx->dn_mask[size_t(layer)];
    Marks mark(ctx, s);
    mark("");
    if ((ctx->path == 1 || ctx->path == 3 || ctx->path == 4) && !g_dbg && !u_dbg) {
        xl::Layer3Args a = layer3_args(ctx, layer, d_ids, d_w, k, d_x, d_shared, d_out, s, tr);
        if (d_out) {
            hipError_t e = hipErrorNotSupported;
            if (ctx->path == 1 || ctx->path == 4) {
                e = xl::dev::launch_stream(a, gu_mask, dn_mask, ctx->cus, s, stop);
                if (e != hipSuccess && e != hipErrorNotSupported) hip_check(e, "streaming layer");
                (void)hipGetLastError();
                if (e == hipSuccess) {
                    ++ctx->launches[XL_LAUNCH_STREAM];
                    if (tr) tr->kernel = 1;
                }
            }
            need(ctx->path != 4 || e == hipSuccess, XL_E_ARG, "XL_LAYER_PATH=4: no streaming-kernel instance for this layer");
            if (e == hipErrorNotSupported) {
                e = xl::dev::launch_layer3(a, gu_mask, dn_mask, ctx->cus, s, stop);
                if (e == hipSuccess) {
                    ++ctx->launches[XL_LAUNCH_ALLTYPES];
                    if (tr) tr->kernel = 3;
                }
            }
            if (e == hipSuccess) {
                if (a.trace) ctx->timeline_words = uint64_t(ctx->cus) * 16 * 32;
                mark("layer");
                return stop != nullptr;
            }
            if (e != hipErrorNotSupported) hip_check(e, "single-launch layer");
            (void)hipGetLastError();   // no instance for this shape: separate launches below
        }
    }
    need(tr == nullptr, XL_E_ARG, "trace: this layer does not run as a single launch (shape, path or output)");
    ++ctx->launches[XL_LAUNCH_SEPARATE];
    hip_check(xl::dev::launch_q8k(d_x, dim / 256, ctx->xq, ctx->xd, nullptr, ctx->err_flag, s), "Q8_K(x) launch");
    mark("q8k_x");
    hip_check(xl::dev::launch_gate_up(descs, d_ids, k, E, dim, ff, ctx->xq, ctx->xd, ctx->codes, ctx->h, g_dbg, u_dbg,
                                      ctx->err_flag, ctx->grid_gu, gu_mask, ctx->cfg.swiglu_limit, s),
              "gate/up launch");
    mark("gate_up");
    hip_check(xl::dev::launch_q8k(ctx->h, k * ff / 256, ctx->hq, ctx->hd, nullptr, ctx->err_flag, s), "Q8_K(h) launch");
    mark("q8k_h");
    hip_check(xl::dev::launch_down(descs, d_ids, k, E, dim, ff, ctx->hq, ctx->hd, ctx->codes, ctx->y, ctx->err_flag,
                                   ctx->grid_down, dn_mask, s),
              "down launch");
    mark("down");
    if (d_out) {
        hip_check(xl::dev::launch_combine(d_ids, d_w, k, ctx->y, dim, d_shared, d_out, s), "combine launch");
        mark("combine");
    }
    return false;
}

// The layer in the reference CPU lane's float order (xl_exact.hip): Q8_K(x),
// gate/up rows + SwiGLU, Q8_K(h), down rows, fixed-order combine; every float
// as q8k_core.hpp:76-95 computes it. Separate launches on stream s.
void enqueue_layer_exact(xl_context* ctx, int32_t layer, const int32_t* d_ids, const float* d_w, int32_t k,
                         const float* d_x, const float* d_shared, float* d_out, hipStream_t s) {
    const int dim = ctx->cfg.dim, ff = ctx->cfg.ff, E = ctx->cfg.n_experts;
    const xl::ExpertDesc* descs = ctx->d_descs + size_t(layer) * E;
    need(dim % 32 == 0 && ff % 32 == 0, XL_E_ARG, "exact rows: dim and ff must be multiples of 32");
    hip_check(xl::dev::launch_q8k(d_x, dim / 256, ctx->xq, ctx->xd, nullptr, ctx->err_flag, s), "Q8_K(x) launch");
    hip_check(xl::dev::launch_exact_rows(descs, d_ids, k, E, ff, dim, 0, ctx->xq, ctx->xd, ctx->tables, ctx->h,
                                         ctx->cfg.swiglu_limit, ctx->err_flag, s),
              "exact gate/up launch");
    hip_check(xl::dev::launch_q8k(ctx->h, k * ff / 256, ctx->hq, ctx->hd, nullptr, ctx->err_flag, s), "Q8_K(h) launch");
    hip_check(xl::dev::launch_exact_rows(descs, d_ids, k, E, dim, ff, 2, ctx->hq, ctx->hd, ctx->tables, ctx->y, 0.0f,
                                         ctx->err_flag, s),
              "exact down launch");
    hip_check(xl::dev::launch_combine(d_ids, d_w, k, ctx->y, dim, d_shared, d_out, s), "combine launch");
    ++ctx->launches[XL_LAUNCH_EXACT];
}

// A per32 matrix: planar IQ (xl_format.hpp) or raw dense ggml blocks.
xl::MatRef per32_matrix(int type, const void* base, int n, int k) {
    need(reinterpret_cast<uintptr_t>(base) % 16 == 0, XL_E_ARG, "matrix not 16-byte aligned");
    xl::MatRef m{};
    m.base = static_cast<const uint8_t*>(base);
    m.type = type;
    if (xl::dense_type(type)) {
        m.nb = k / xl::dense_block_values(type);
    } else {
        const auto P = xl::plane_layout(type, matrix_blocks(n, k));
        m.off1 = P.off[1];
        m.off2 = P.off[2];
        m.nb = k / 256;
    }
    return m;
}

// Shared-expert workspace of T tokens: g, u (T x ff floats), Q32(x) and Q32(h)
// quants and scales, each 256-byte aligned.
struct SharedWork {
    uint64_t g, u, xq, hq, xd, hd, bytes;
};
SharedWork shared_work(int dim, int ff, int T) {
    SharedWork w{};
    uint64_t at = 0;
    const auto take = [&](uint64_t bytes) { const uint64_t o = at; at += (bytes + 255) & ~uint64_t(255); return o; };
    const uint64_t t = uint64_t(T);
    w.g = take(t * ff * 4);
    w.u = take(t * ff * 4);
    w.xq = take(t * dim);
    w.hq = take(t * ff);
    w.xd = take(t * (dim / 32) * 4);
    w.hd = take(t * (ff / 32) * 4);
    w.bytes = at;
    return w;
}

// Enqueues the per32 layer (hip_resident_bank.hpp:185-200 with the kernels of
// hip_experts.hip): quant32(x), gate and up rows of every pick in one launch,
// SwiGLU, quant32(h) of every pick, down rows into y (k x dim), then the
// fixed-order combine into out when out is given.
void enqueue_per32(xl_context* ctx, int32_t layer, const int32_t* d_ids, const float* d_w, int32_t k, const float* d_x,
                   const float* d_shared, float* d_y, float* d_out, hipStream_t s) {
    const int dim = ctx->cfg.dim, ff = ctx->cfg.ff, E = ctx->cfg.n_experts;
    const xl::ExpertDesc* descs = ctx->d_descs + size_t(layer) * E;
    float* xd = ctx->p32d;
    float* hd = ctx->p32d + ctx->act_max / 32;
    const xl::MatRef none{};
    Marks mark(ctx, s);
    mark("");
    hip_check(xl::dev::launch_quant32(d_x, 1, dim, ctx->xq, xd, ctx->err_flag, s), "quant32(x) launch");
    mark("quant32_x");
    hip_check(xl::dev::launch_mv32(descs, d_ids, none, none, k, E, 0, 2, ff, dim, ctx->xq, 0, xd, 0, ctx->g, ctx->u,
                                   size_t(ff), ctx->tables, ctx->err_flag, s),
              "per32 gate/up launch");
    mark("gate_up32");
    hip_check(xl::dev::launch_swiglu_quant32(ctx->g, ctx->u, k, ff, ctx->cfg.swiglu_limit, ctx->hq, hd, s),
              "SwiGLU + quant32(h) launch");
    mark("swiglu_quant32");
    // the fixed-order combine (runtime.cpp:183-188) in the down launch's epilogue
    // when out is given: each workgroup holds every pick's value of its rows
    const xl::dev::Mv32Comb cb{d_w, d_shared, d_out};
    hip_check(xl::dev::launch_mv32(descs, d_ids, none, none, k, E, 2, 1, dim, ff, ctx->hq, size_t(ff), hd, size_t(ff / 32),
                                   d_y, nullptr, size_t(dim), ctx->tables, ctx->err_flag, s, nullptr,
                                   d_out ? &cb : nullptr),
              "per32 down launch");
    mark(d_out ? "down32_combine" : "down32");
}

}  // namespace

extern "C" {

uint32_t xl_abi_version(void) { return XL_ABI_VERSION; }

int32_t xl_open(uint32_t abi_version, const xl_config* cfg, xl_context** out, xl_error* err) {
    xl_context* ctx = nullptr;
    const int32_t rc = guarded(nullptr, err, [&] {
        need(out != nullptr, XL_E_ARG, "null output pointer");
        *out = nullptr;
        need(abi_version == XL_ABI_VERSION, XL_E_VERSION, "ABI version mismatch");
        need(cfg != nullptr, XL_E_ARG, "null config");
        need(cfg->struct_bytes == sizeof(xl_config), XL_E_VERSION, "xl_config size mismatch");
        int lpr, ppl;
        need(xl::row_shape(cfg->dim, lpr, ppl), XL_E_ARG,
             "dim not supported (256, 512, 768, 1024, 2048, 2304, 3072, 4096 or 5120)");
        need(xl::row_shape(cfg->ff, lpr, ppl), XL_E_ARG,
             "ff not supported (256, 512, 768, 1024, 2048, 2304, 3072, 4096 or 5120)");
        need(cfg->n_layers >= 1 && cfg->n_layers <= 4096, XL_E_ARG, "n_layers outside 1..4096");
        need(cfg->n_experts >= 1 && cfg->n_experts <= 65536, XL_E_ARG, "n_experts outside 1..65536");
        need(cfg->max_picks >= 1 && cfg->max_picks <= 16, XL_E_ARG, "max_picks outside 1..16");
        need(cfg->max_tokens >= 0 && cfg->max_tokens <= 65536, XL_E_ARG, "max_tokens outside 0..65536");
        need(std::isfinite(cfg->swiglu_limit), XL_E_ARG, "swiglu_limit not finite");
        int ndev = 0;
        hip_check(hipGetDeviceCount(&ndev), "hipGetDeviceCount");
        need(cfg->device >= 0 && cfg->device < ndev, XL_E_ARG, "device ordinal out of range");
        ctx = new xl_context();
        ctx->cfg = *cfg;
        hip_check(hipSetDevice(cfg->device), "hipSetDevice");
        hipDeviceProp_t prop{};
        hip_check(hipGetDeviceProperties(&prop, cfg->device), "hipGetDeviceProperties");
        ctx->cus = prop.multiProcessorCount;
        hip_check(hipStreamCreateWithFlags(&ctx->stream, hipStreamNonBlocking), "hipStreamCreate");
        hip_check(hipEventCreateWithFlags(&ctx->done, hipEventDisableTiming), "hipEventCreate");
        ctx->grid_gu = env_int("XL_WGS_GATE_UP", 4 * ctx->cus);
        ctx->grid_down = env_int("XL_WGS_DOWN", 4 * ctx->cus);

        const int P = cfg->max_picks, dim = cfg->dim, ff = cfg->ff;
        ctx->act_max = std::max({dim, ff, xl::kMaxRowK});
        struct Part { void** p; uint64_t bytes; };
        const uint64_t code_bytes = (256 + 512 + 2048) * 2;
        std::vector<Part> parts = {
            {reinterpret_cast<void**>(&ctx->codes), code_bytes},
            {reinterpret_cast<void**>(&ctx->err_flag), 256},
            {reinterpret_cast<void**>(&ctx->x), uint64_t(dim) * 4},
            {reinterpret_cast<void**>(&ctx->xq), uint64_t(ctx->act_max)},
            {reinterpret_cast<void**>(&ctx->xd), uint64_t(ctx->act_max / 256) * 4},
            {reinterpret_cast<void**>(&ctx->mv_x), uint64_t(ctx->act_max) * 4},
            {reinterpret_cast<void**>(&ctx->h), uint64_t(P) * ff * 4},
            {reinterpret_cast<void**>(&ctx->hq), uint64_t(P) * ff},
            {reinterpret_cast<void**>(&ctx->hd), uint64_t(P) * (ff / 256) * 4},
            {reinterpret_cast<void**>(&ctx->g), uint64_t(P) * ff * 4},
            {reinterpret_cast<void**>(&ctx->u), uint64_t(P) * ff * 4},
            {reinterpret_cast<void**>(&ctx->y), uint64_t(P) * dim * 4},
            {reinterpret_cast<void**>(&ctx->out), uint64_t(dim) * 4},
            {reinterpret_cast<void**>(&ctx->shared), uint64_t(dim) * 4},
            {reinterpret_cast<void**>(&ctx->w), 64 * 4},
            {reinterpret_cast<void**>(&ctx->ids), 64 * 4},
            {reinterpret_cast<void**>(&ctx->q8std), uint64_t(P) * (std::max(dim, ff) / 256) * 292},
            {reinterpret_cast<void**>(&ctx->htag), uint64_t(P) * ff * 8},
            {reinterpret_cast<void**>(&ctx->hqtag), uint64_t(P) * ff * 2},
            {reinterpret_cast<void**>(&ctx->hdtag), uint64_t(P) * (ff / 256) * 8},
            {reinterpret_cast<void**>(&ctx->ctl), 256},
            {reinterpret_cast<void**>(&ctx->hbuf), uint64_t(2) * xl::kHBufWords * 4},
            {reinterpret_cast<void**>(&ctx->tables), uint64_t(xl::kTableBytes)},
            {reinterpret_cast<void**>(&ctx->p32d), (uint64_t(ctx->act_max / 32) + uint64_t(P) * (ff / 32)) * 4},
            {reinterpret_cast<void**>(&ctx->timeline), uint64_t(ctx->cus) * 16 * 32 * 8},
        };
        if (cfg->max_tokens > 0) {
            const uint64_t T = uint64_t(cfg->max_tokens), GP = T * uint64_t(P);
            auto& g = ctx->grp;
            const uint64_t slots = 16 * uint64_t(xl::group_max_tasks(int64_t(GP), cfg->n_experts));
            g.hq_bytes = slots * uint64_t(ff);
            const std::vector<Part> gparts = {
                {reinterpret_cast<void**>(&g.ids), GP * 4},
                {reinterpret_cast<void**>(&g.w), GP * 4},
                {reinterpret_cast<void**>(&g.x), T * dim * 4},
                {reinterpret_cast<void**>(&g.shared), T * dim * 4},
                {reinterpret_cast<void**>(&g.out), T * dim * 4},
                {reinterpret_cast<void**>(&g.xq), slots * dim},
                {reinterpret_cast<void**>(&g.xd), T * (dim / 256) * 4},
                {reinterpret_cast<void**>(&g.order), slots * 4},
                {reinterpret_cast<void**>(&g.pos), GP * 4},
                {reinterpret_cast<void**>(&g.tasks), uint64_t(xl::group_max_tasks(int64_t(GP), cfg->n_experts)) * 16},
                {reinterpret_cast<void**>(&g.n_tasks), 256},
                {reinterpret_cast<void**>(&g.h), GP * ff * 4},
                {reinterpret_cast<void**>(&g.hq), g.hq_bytes},
                {reinterpret_cast<void**>(&g.hd), GP * (ff / 256) * 4},
                {reinterpret_cast<void**>(&g.y), GP * dim * 4},
            };
            parts.insert(parts.end(), gparts.begin(), gparts.end());
        }
        uint64_t total = 0;
        for (auto& p : parts) total += xl::align256(p.bytes);
        hip_check(hipMalloc(&ctx->ws, total), "workspace hipMalloc");
        ctx->ws_bytes = total;
        uint64_t at = 0;
        for (auto& p : parts) {
            *p.p = static_cast<uint8_t*>(ctx->ws) + at;
            at += xl::align256(p.bytes);
        }
        std::vector<uint16_t> codes;
        codes.insert(codes.end(), kIq2xxsCodes, kIq2xxsCodes + 256);
        codes.insert(codes.end(), kIq2xsCodes, kIq2xsCodes + 512);
        codes.insert(codes.end(), kIq1sCodes, kIq1sCodes + 2048);
        for (int i = 0; i < 256 + 512; ++i) (void)expand_codes(codes[size_t(i)], false);   // rejects a corrupt symbol
        hip_check(hipMemcpy(ctx->codes, codes.data(), code_bytes, hipMemcpyHostToDevice), "codebook upload");
        hip_check(hipMemset(ctx->err_flag, 0, 256), "error flag clear");
        hip_check(hipMemset(ctx->htag, 0, size_t(P) * ff * 8), "tag clear");
        hip_check(hipMemset(ctx->hdtag, 0, size_t(P) * (ff / 256) * 8), "tag clear");
        hip_check(hipMemset(ctx->hqtag, 0, size_t(P) * ff * 2), "tag clear");
        hip_check(hipMemset(ctx->ctl, 0, 256), "epoch clear");
        hip_check(hipMemset(ctx->hbuf, 0xff, size_t(2) * xl::kHBufWords * 4), "h exchange fill");
        const std::vector<uint64_t> tab = layer_tables();
        hip_check(hipMemcpy(ctx->tables, tab.data(), tab.size() * 8, hipMemcpyHostToDevice), "table upload");
        void* scratch = nullptr;   // the no-allocation scratch's address on this device, looked up once
        hip_check(xl::dev::noalloc_scratch(cfg->device, &scratch), "no-allocation scratch address");
        ctx->path = env_int("XL_LAYER_PATH", 1);
        need(ctx->path == 0 || ctx->path == 1 || ctx->path == 3 || ctx->path == 4, XL_E_ARG,
             "XL_LAYER_PATH must be 0, 1, 3 or 4");
        ctx->gpath = env_int("XL_GROUPED_PATH", 1);
        need(ctx->gpath >= 0 && ctx->gpath <= 2, XL_E_ARG, "XL_GROUPED_PATH must be 0, 1 or 2");
        *out = ctx;
    });
    if (rc != XL_OK && ctx) xl_close(ctx);
    return rc;
}

void xl_close(xl_context* ctx) {
    if (!ctx) return;
    (void)hipSetDevice(ctx->cfg.device);
    // The last call may have run on a caller stream: wait for it, then for the
    // context stream, before any memory goes back.
    if (ctx->done && ctx->has_last) (void)hipEventSynchronize(ctx->done);
    if (ctx->stream) (void)hipStreamSynchronize(ctx->stream);
    for (auto& e : ctx->prof.ev)   // profiling left active (xl_profile_end never called)
        if (e) (void)hipEventDestroy(e);
    ctx->prof.ev.clear();
    for (auto* s : ctx->slabs) (void)hipFree(s);
    if (ctx->d_descs) (void)hipFree(ctx->d_descs);
    if (ctx->ws) (void)hipFree(ctx->ws);
    if (ctx->done) (void)hipEventDestroy(ctx->done);
    if (ctx->stream) (void)hipStreamDestroy(ctx->stream);
    delete ctx;
}

int32_t xl_last_error(const xl_context* ctx, xl_error* err) {
    if (!ctx || !err) return XL_E_ARG;
    *err = ctx->last;
    return XL_OK;
}

int32_t xl_bank_create(xl_context* ctx, const int32_t* types, xl_error* err) {
    return guarded(ctx, err, [&] {
        ready(ctx, false);
        need(!ctx->bank_ready, XL_E_STATE, "bank already created");
        need(types != nullptr, XL_E_ARG, "null type map");
        const int L = ctx->cfg.n_layers, E = ctx->cfg.n_experts, dim = ctx->cfg.dim, ff = ctx->cfg.ff;
        const size_t n = size_t(L) * E * 3;
        for (size_t i = 0; i < n; ++i) need(xl::supported_type(types[i]), XL_E_ARG, "unsupported block type");
        for (size_t e = 0; e < size_t(L) * E; ++e)
            need(types[3 * e] == types[3 * e + 1], XL_E_ARG, "gate and up must share a block type");
        ctx->types.assign(types, types + n);
        ctx->gu_mask.assign(size_t(L), 0);
        ctx->dn_mask.assign(size_t(L), 0);
        for (int l = 0; l < L; ++l)
            for (int e = 0; e < E; ++e) {
                ctx->gu_mask[size_t(l)] |= xl::dev::type_bit(types[(size_t(l) * E + e) * 3]);
                ctx->dn_mask[size_t(l)] |= xl::dev::type_bit(types[(size_t(l) * E + e) * 3 + 2]);
            }
        ctx->descs.assign(size_t(L) * E, xl::ExpertDesc{});
        // One slab per layer, experts contiguous, each matrix's planes 256-B aligned.
        for (int l = 0; l < L; ++l) {
            uint64_t bytes = 0;
            for (int e = 0; e < E; ++e)
                for (int r = 0; r < 3; ++r) {
                    const int t = types[(size_t(l) * E + e) * 3 + r];
                    const int nr = r < 2 ? ff : dim, kk = r < 2 ? dim : ff;
                    bytes += xl::plane_layout(t, matrix_blocks(nr, kk)).bytes;
                    ctx->payload += matrix_blocks(nr, kk) * uint64_t(xl::block_bytes(t));
                }
            uint8_t* slab = nullptr;
            const hipError_t e = hipMalloc(&slab, bytes);
            if (e != hipSuccess) fail(XL_E_MEMORY, "bank slab %d (%llu bytes): %s", l, (unsigned long long)bytes, hipGetErrorString(e));
            ctx->slabs.push_back(slab);
            ctx->allocated += bytes;
            uint64_t at = 0;
            for (int e2 = 0; e2 < E; ++e2)
                for (int r = 0; r < 3; ++r) {
                    const int t = types[(size_t(l) * E + e2) * 3 + r];
                    const int nr = r < 2 ? ff : dim, kk = r < 2 ? dim : ff;
                    const auto P = xl::plane_layout(t, matrix_blocks(nr, kk));
                    xl::MatRef& m = ctx->descs[size_t(l) * E + e2].m[r];
                    m.base = slab + at;
                    m.off1 = P.off[1];
                    m.off2 = P.off[2];
                    m.type = t;
                    m.nb = kk / 256;
                    at += P.bytes;
                }
        }
        ctx->layer_shape.assign(size_t(L), LayerShape{});
        for (int l = 0; l < L; ++l) {
            LayerShape& ls = ctx->layer_shape[size_t(l)];
            const int32_t* t0 = types + size_t(l) * E * 3;
            bool same = true;
            for (int e = 1; e < E && same; ++e)
                for (int r = 0; r < 3; ++r) same = same && t0[3 * e + r] == t0[r];
            if (!same) continue;
            const uint8_t* b0 = ctx->descs[size_t(l) * E].m[0].base;
            uint64_t at = 0;
            for (int r = 0; r < 3; ++r) {
                ls.roff[r] = uint64_t(ctx->descs[size_t(l) * E].m[r].base - b0);
                ls.rtype[r] = t0[r];
                at += xl::plane_layout(t0[r], r < 2 ? matrix_blocks(ff, dim) : matrix_blocks(dim, ff)).bytes;
            }
            ls.estride = at;
            ls.regular = true;
            for (int e = 0; e < E && ls.regular; ++e)
                for (int r = 0; r < 3; ++r)
                    ls.regular = ls.regular && ctx->descs[size_t(l) * E + e].m[r].base == b0 + uint64_t(e) * at + ls.roff[r];
        }
        hip_check(hipMalloc(&ctx->d_descs, ctx->descs.size() * sizeof(xl::ExpertDesc)), "descriptor hipMalloc");
        hip_check(hipMemcpy(ctx->d_descs, ctx->descs.data(), ctx->descs.size() * sizeof(xl::ExpertDesc),
                            hipMemcpyHostToDevice),
                  "descriptor upload");
        ctx->bank_ready = true;
    });
}

int32_t xl_bank_generate(xl_context* ctx, uint64_t seed, xl_error* err) {
    return guarded(ctx, err, [&] {
        ready(ctx, true);
        const int L = ctx->cfg.n_layers, E = ctx->cfg.n_experts, dim = ctx->cfg.dim, ff = ctx->cfg.ff;
        Ordered ord(ctx, ctx->stream);
        for (int l = 0; l < L; ++l)
            for (int e = 0; e < E; ++e)
                for (int r = 0; r < 3; ++r) {
                    const xl::MatRef& m = ctx->descs[size_t(l) * E + e].m[r];
                    const int nr = r < 2 ? ff : dim, kk = r < 2 ? dim : ff;
                    hip_check(xl::dev::launch_generate(const_cast<uint8_t*>(m.base), m.type, nr, kk, seed, uint32_t(l),
                                                       uint32_t(e), uint32_t(r), ctx->stream),
                              "generate launch");
                }
        drain(ctx, ctx->stream);
        ctx->generated = true;
    });
}

int32_t xl_bank_upload(xl_context* ctx, int32_t layer, int32_t expert, int32_t role, const void* aos, uint64_t bytes,
                       xl_error* err) {
    return guarded(ctx, err, [&] {
        ready(ctx, true);
        check_layer(ctx, layer);
        need(expert >= 0 && expert < ctx->cfg.n_experts && role >= 0 && role < 3, XL_E_ARG, "expert/role out of range");
        need(aos != nullptr, XL_E_ARG, "null weights");
        const xl::MatRef& m = ctx->descs[size_t(layer) * ctx->cfg.n_experts + expert].m[role];
        const int nr = role < 2 ? ctx->cfg.ff : ctx->cfg.dim, kk = role < 2 ? ctx->cfg.dim : ctx->cfg.ff;
        const uint64_t nblk = matrix_blocks(nr, kk);
        need(bytes == nblk * uint64_t(xl::block_bytes(m.type)), XL_E_ARG, "weight byte extent differs from shape");
        const auto P = xl::plane_layout(m.type, nblk);
        std::vector<uint8_t> planar(P.bytes, 0);
        const auto* src = static_cast<const uint8_t*>(aos);
        for (uint64_t b = 0; b < nblk; ++b)
            xl::block_to_planes(m.type, src + b * xl::block_bytes(m.type), planar.data(), P, b);
        Ordered ord(ctx, ctx->stream);
        hip_check(hipMemcpyAsync(const_cast<uint8_t*>(m.base), planar.data(), P.bytes, hipMemcpyHostToDevice, ctx->stream),
                  "weight upload");
        hip_check(hipStreamSynchronize(ctx->stream), "weight upload drain");
    });
}

// ---- pack loader -----------------------------------------------------------------
// The reference's weight pack (sycl/stage/wiring/pack_source.cpp:144-186): a
// directory with ds4.txt ("key value" lines: model_dir, format, hidden_size,
// num_hidden_layers, n_routed_experts, num_experts_per_tok,
// moe_intermediate_size, ...) and tensors.txt ("file <i> <name>" and
// "t <name> <dtype> <file> <offset> <bytes> <shape...>" lines) over shard
// files in model_dir. Routed experts are layers.<l>.ffn.experts.<e>.w1 (gate),
// .w3 (up) and .w2 (down) .weight, raw ggml blocks (engine/strata/warm/
// test_mmvq.py:111-137 writes the same layout).
namespace {

struct PackTensor {
    std::string dtype;
    int file = -1;
    uint64_t offset = 0, bytes = 0;
};
struct Pack {
    std::string dir, model_dir;
    std::map<std::string, std::string> kv;
    std::vector<std::string> files;
    std::map<std::string, PackTensor> t;
    int num(const char* key) const {
        const auto it = kv.find(key);
        if (it == kv.end()) fail(XL_E_ARG, "pack ds4.txt: %s missing", key);
        char* end = nullptr;
        const long v = std::strtol(it->second.c_str(), &end, 10);
        if (*end || v < 0 || v > (1L << 30)) fail(XL_E_ARG, "pack ds4.txt: %s is not a count", key);
        return int(v);
    }
    double real(const char* key, double dflt) const {
        const auto it = kv.find(key);
        if (it == kv.end()) return dflt;
        char* end = nullptr;
        const double v = std::strtod(it->second.c_str(), &end);
        if (*end || !std::isfinite(v)) fail(XL_E_ARG, "pack ds4.txt: %s is not a finite number", key);
        return v;
    }
};

std::string slurp(const std::string& path) {
    std::ifstream f(path, std::ios::binary);
    if (!f) fail(XL_E_ARG, "pack: cannot read %s", path.c_str());
    std::ostringstream s;
    s << f.rdbuf();
    return s.str();
}

Pack read_pack(const char* dir) {
    need(dir != nullptr && *dir, XL_E_ARG, "null pack directory");
    Pack p;
    p.dir = dir;
    {
        std::istringstream f(slurp(p.dir + "/ds4.txt"));
        std::string line;
        while (std::getline(f, line)) {
            const size_t sp = line.find(' ');
            if (sp != std::string::npos) p.kv[line.substr(0, sp)] = line.substr(sp + 1);
        }
    }
    const auto fmt = p.kv.find("format");
    need(fmt != p.kv.end() && fmt->second == "gguf", XL_E_ARG, "pack: only the gguf format is admitted");
    const auto md = p.kv.find("model_dir");
    need(md != p.kv.end() && !md->second.empty(), XL_E_ARG, "pack ds4.txt: model_dir missing");
    p.model_dir = md->second[0] == '/' ? md->second : p.dir + "/" + md->second;
    std::istringstream f(slurp(p.dir + "/tensors.txt"));
    std::string line;
    while (std::getline(f, line)) {
        std::istringstream s(line);
        std::string tag;
        s >> tag;
        if (tag == "file") {
            int i = -1;
            std::string name;
            s >> i >> name;
            need(i >= 0 && i < (1 << 20) && !name.empty(), XL_E_ARG, "pack tensors.txt: bad file line");
            if (int(p.files.size()) <= i) p.files.resize(size_t(i) + 1);
            p.files[size_t(i)] = name;
        } else if (tag == "t") {
            std::string name;
            PackTensor x;
            s >> name >> x.dtype >> x.file >> x.offset >> x.bytes;
            need(!s.fail() && !name.empty(), XL_E_ARG, "pack tensors.txt: bad tensor line");
            need(p.t.emplace(name, x).second, XL_E_ARG, "pack tensors.txt: duplicate tensor");
        }
    }
    return p;
}

int32_t ggml_type_of(const std::string& dtype) {
    if (dtype == "IQ2_XXS") return xl::kIQ2_XXS;
    if (dtype == "IQ2_XS") return xl::kIQ2_XS;
    if (dtype == "IQ1_M") return xl::kIQ1_M;
    return -1;
}

const char* kRoleName[3] = {"w1", "w3", "w2"};   // gate, up, down

const PackTensor& expert_tensor(const Pack& p, int layer, int expert, int role) {
    const std::string name = "layers." + std::to_string(layer) + ".ffn.experts." + std::to_string(expert) + "." +
                             kRoleName[role] + ".weight";
    const auto it = p.t.find(name);
    if (it == p.t.end()) fail(XL_E_ARG, "pack: tensor %s missing", name.c_str());
    return it->second;
}

}  // namespace

int32_t xl_pack_meta_get(const char* pack_dir, xl_pack_meta* out, xl_error* err) {
    return guarded(nullptr, err, [&] {
        need(out != nullptr, XL_E_ARG, "null output");
        need(out->struct_bytes == sizeof(xl_pack_meta), XL_E_VERSION, "xl_pack_meta size mismatch");
        const Pack p = read_pack(pack_dir);
        out->dim = p.num("hidden_size");
        out->ff = p.num("moe_intermediate_size");
        out->n_layers = p.num("num_hidden_layers");
        out->n_experts = p.num("n_routed_experts");
        out->top_k = p.num("num_experts_per_tok");
        out->swiglu_limit = float(p.real("swiglu_limit", 0.0));
    });
}

int32_t xl_pack_types(const char* pack_dir, int32_t first_layer, int32_t n_layers, int32_t n_experts, int32_t* types,
                      xl_error* err) {
    return guarded(nullptr, err, [&] {
        need(types != nullptr && first_layer >= 0 && n_layers >= 1 && n_experts >= 1, XL_E_ARG, "bad layer window");
        const Pack p = read_pack(pack_dir);
        for (int l = 0; l < n_layers; ++l)
            for (int e = 0; e < n_experts; ++e)
                for (int r = 0; r < 3; ++r) {
                    const int32_t t = ggml_type_of(expert_tensor(p, first_layer + l, e, r).dtype);
                    need(t > 0, XL_E_ARG, "pack: an expert matrix is not IQ2_XXS / IQ2_XS / IQ1_M");
                    types[(size_t(l) * n_experts + e) * 3 + r] = t;
                }
    });
}

int32_t xl_bank_load_pack(xl_context* ctx, const char* pack_dir, int32_t first_layer, xl_error* err) {
    return guarded(ctx, err, [&] {
        ready(ctx, true);
        const Pack p = read_pack(pack_dir);
        need(p.num("hidden_size") == ctx->cfg.dim && p.num("moe_intermediate_size") == ctx->cfg.ff, XL_E_ARG,
             "pack: hidden_size / moe_intermediate_size differ from the context's dim / ff");
        need(p.num("n_routed_experts") == ctx->cfg.n_experts, XL_E_ARG, "pack: n_routed_experts differs from the context");
        need(first_layer >= 0 && first_layer + ctx->cfg.n_layers <= p.num("num_hidden_layers"), XL_E_ARG,
             "pack: layer window past num_hidden_layers");
        std::vector<uint8_t> buf;
        std::vector<std::ifstream> shards(p.files.size());
        for (int l = 0; l < ctx->cfg.n_layers; ++l)
            for (int e = 0; e < ctx->cfg.n_experts; ++e)
                for (int r = 0; r < 3; ++r) {
                    const PackTensor& x = expert_tensor(p, first_layer + l, e, r);
                    const xl::MatRef& m = ctx->descs[size_t(l) * ctx->cfg.n_experts + e].m[r];
                    need(ggml_type_of(x.dtype) == m.type, XL_E_ARG, "pack: a matrix type differs from the bank's");
                    need(x.file >= 0 && size_t(x.file) < p.files.size() && !p.files[size_t(x.file)].empty(), XL_E_ARG,
                         "pack: tensor names an unknown shard");
                    auto& sh = shards[size_t(x.file)];
                    if (!sh.is_open()) {
                        sh.open(p.model_dir + "/" + p.files[size_t(x.file)], std::ios::binary);
                        if (!sh) fail(XL_E_ARG, "pack: cannot open shard %s", p.files[size_t(x.file)].c_str());
                    }
                    buf.resize(x.bytes);
                    sh.seekg(std::streamoff(x.offset));
                    sh.read(reinterpret_cast<char*>(buf.data()), std::streamsize(x.bytes));
                    need(bool(sh) && uint64_t(sh.gcount()) == x.bytes, XL_E_ARG, "pack: tensor extent past shard end");
                    xl_error e2{};
                    const int32_t rc = xl_bank_upload(ctx, l, e, r, buf.data(), x.bytes, &e2);
                    if (rc != XL_OK) fail(rc, "pack: layer %d expert %d %s: %s", first_layer + l, e, kRoleName[r], e2.message);
                }
        ctx->generated = false;
    });
}

int32_t xl_bank_download(xl_context* ctx, int32_t layer, int32_t expert, int32_t role, void* aos, uint64_t bytes,
                         xl_error* err) {
    return guarded(ctx, err, [&] {
        ready(ctx, true);
        check_layer(ctx, layer);
        need(expert >= 0 && expert < ctx->cfg.n_experts && role >= 0 && role < 3, XL_E_ARG, "expert/role out of range");
        need(aos != nullptr, XL_E_ARG, "null output");
        const xl::MatRef& m = ctx->descs[size_t(layer) * ctx->cfg.n_experts + expert].m[role];
        const int nr = role < 2 ? ctx->cfg.ff : ctx->cfg.dim, kk = role < 2 ? ctx->cfg.dim : ctx->cfg.ff;
        const uint64_t nblk = matrix_blocks(nr, kk);
        need(bytes == nblk * uint64_t(xl::block_bytes(m.type)), XL_E_ARG, "output byte extent differs from shape");
        const auto P = xl::plane_layout(m.type, nblk);
        std::vector<uint8_t> planar(P.bytes);
        Ordered ord(ctx, ctx->stream);
        hip_check(hipMemcpyAsync(planar.data(), m.base, P.bytes, hipMemcpyDeviceToHost, ctx->stream), "weight download");
        hip_check(hipStreamSynchronize(ctx->stream), "weight download drain");
        auto* dst = static_cast<uint8_t*>(aos);
        for (uint64_t b = 0; b < nblk; ++b) xl::planes_to_block(m.type, planar.data(), P, b, dst + b * xl::block_bytes(m.type));
    });
}

int32_t xl_bank_info_get(const xl_context* ctx, xl_bank_info* out) {
    if (!ctx || !out) return XL_E_ARG;
    std::memset(out, 0, sizeof *out);
    out->payload_bytes = ctx->payload;
    out->allocated_bytes = ctx->allocated;
    out->workspace_bytes = ctx->ws_bytes;
    out->n_layers = ctx->cfg.n_layers;
    out->n_experts = ctx->cfg.n_experts;
    out->generated = ctx->generated ? 1 : 0;
    return XL_OK;
}

int32_t xl_contains(const xl_context* ctx, int32_t layer, int32_t expert) {
    return ctx && ctx->bank_ready && layer >= 0 && layer < ctx->cfg.n_layers && expert >= 0 &&
           expert < ctx->cfg.n_experts;
}

int32_t xl_experts_forward(xl_context* ctx, int32_t layer, const int32_t* ids, int32_t k, const float* x, float* ys,
                           xl_error* err) {
    return guarded(ctx, err, [&] {
        ready(ctx, true);
        check_layer(ctx, layer);
        check_ids(ctx, ids, k);
        check_finite(x, size_t(ctx->cfg.dim), "input vector");
        need(ys != nullptr, XL_E_ARG, "null output");
        hipStream_t s = ctx->stream;
        Ordered ord(ctx, s);
        hip_check(hipMemcpyAsync(ctx->ids, ids, sizeof(int32_t) * k, hipMemcpyHostToDevice, s), "ids upload");
        hip_check(hipMemcpyAsync(ctx->x, x, sizeof(float) * ctx->cfg.dim, hipMemcpyHostToDevice, s), "x upload");
        enqueue_layer(ctx, layer, ctx->ids, nullptr, k, ctx->x, nullptr, nullptr, s);
        hip_check(hipMemcpyAsync(ys, ctx->y, sizeof(float) * size_t(k) * ctx->cfg.dim, hipMemcpyDeviceToHost, s),
                  "output download");
        drain(ctx, s);
        for (size_t i = 0; i < size_t(k) * ctx->cfg.dim; ++i)
            if (!std::isfinite(ys[i])) fail(XL_E_DEVICE, "non-finite expert output");
    });
}

int32_t xl_expert_forward(xl_context* ctx, int32_t layer, int32_t expert, const float* x, float* y, xl_error* err) {
    const int32_t id = expert;
    return xl_experts_forward(ctx, layer, &id, 1, x, y, err);
}

namespace {

// Enqueues T tokens of layer `layer` on stream s: the grouped MFMA kernels when
// the layer's gate/up are IQ2_XXS and its down IQ2_XS, otherwise one layer
// call per token. All pointers are device pointers.
void enqueue_grouped(xl_context* ctx, int32_t layer, int32_t T, int32_t k, const int32_t* d_ids, const float* d_w,
                     const float* d_x, const float* d_shared, float* d_out, hipStream_t s, LayerTrace* tr = nullptr) {
    const int dim = ctx->cfg.dim, E = ctx->cfg.n_experts;
    const int gu_mask = ctx->gu_mask[size_t(layer)], dn_mask = ctx->dn_mask[size_t(layer)];
    Marks mark(ctx, s);
    mark("");
    if (ctx->gpath != 0 && gu_mask == 1 && dn_mask == 2) {
        xl::GroupArgs a{};
        a.descs = ctx->d_descs + size_t(layer) * E;
        a.ids = d_ids; a.w = d_w; a.x = d_x; a.shared = d_shared; a.out = d_out;
        a.T = T; a.k = k; a.n_experts = E; a.dim = dim; a.ff = ctx->cfg.ff;
        const auto& g = ctx->grp;
        a.xq = g.xq; a.xd = g.xd; a.order = g.order; a.pos = g.pos; a.tasks = g.tasks; a.n_tasks = g.n_tasks;
        a.h = g.h; a.hq = g.hq; a.hd = g.hd; a.y = g.y;
        a.tables = ctx->tables; a.err = ctx->err_flag;
        a.lim = ctx->cfg.swiglu_limit;
        if (tr) { a.tq8x = tr->q8x; a.tq8h = tr->q8h; a.tint = tr->ints; }
        const hipError_t e = xl::dev::launch_grouped(a, ctx->cus, s);
        if (e == hipSuccess) {
            if (tr && tr->h)   // the pairs' h as the gate/up kernel wrote it for Q8_K(h)
                hip_check(hipMemcpyAsync(tr->h, g.h, sizeof(float) * size_t(T) * k * ctx->cfg.ff,
                                         hipMemcpyDeviceToDevice, s), "trace h copy");
            if (tr && tr->y)   // the pairs' rows as the combine kernel read them
                hip_check(hipMemcpyAsync(tr->y, g.y, sizeof(float) * size_t(T) * k * dim, hipMemcpyDeviceToDevice, s),
                          "trace y copy");
            mark("grouped");
            return;
        }
        if (e != hipErrorNotSupported) hip_check(e, "grouped launch");
        (void)hipGetLastError();
    }
    need(ctx->gpath != 2, XL_E_ARG, "XL_GROUPED_PATH=2: the grouped MFMA kernels cannot run this layer");
    need(tr == nullptr, XL_E_ARG, "trace: this layer does not run on the grouped MFMA kernels");
    for (int t = 0; t < T; ++t)
        enqueue_layer(ctx, layer, d_ids + size_t(t) * k, d_w + size_t(t) * k, k, d_x + size_t(t) * dim,
                      d_shared ? d_shared + size_t(t) * dim : nullptr, d_out + size_t(t) * dim, s);
}

void check_grouped(const xl_context* ctx, int32_t T, int32_t k) {
    need(ctx->cfg.max_tokens > 0, XL_E_STATE, "grouped path unused: the context was opened with max_tokens = 0");
    need(T >= 1 && T <= ctx->cfg.max_tokens, XL_E_ARG, "token count outside 1..max_tokens");
    need(k >= 1 && k <= ctx->cfg.max_picks, XL_E_ARG, "pick count outside 1..max_picks");
}

}  // namespace

int32_t xl_grouped_forward(xl_context* ctx, int32_t layer, int32_t T, int32_t k, const int32_t* ids, const float* w,
                           const float* x, const float* shared_or_null, float* out, xl_error* err) {
    return guarded(ctx, err, [&] {
        ready(ctx, true);
        check_layer(ctx, layer);
        check_grouped(ctx, T, k);
        need(ids && w && x && out, XL_E_ARG, "null pointer");
        const int dim = ctx->cfg.dim;
        for (int t = 0; t < T; ++t) check_ids(ctx, ids + size_t(t) * k, k);
        check_finite(w, size_t(T) * k, "route weights");
        check_finite(x, size_t(T) * dim, "input vectors");
        if (shared_or_null) check_finite(shared_or_null, size_t(T) * dim, "shared vectors");
        hipStream_t s = ctx->stream;
        Ordered ord(ctx, s);
        auto& g = ctx->grp;
        const size_t P = size_t(T) * k, X = size_t(T) * dim;
        hip_check(hipMemcpyAsync(g.ids, ids, sizeof(int32_t) * P, hipMemcpyHostToDevice, s), "ids upload");
        hip_check(hipMemcpyAsync(g.w, w, sizeof(float) * P, hipMemcpyHostToDevice, s), "weights upload");
        hip_check(hipMemcpyAsync(g.x, x, sizeof(float) * X, hipMemcpyHostToDevice, s), "x upload");
        if (shared_or_null)
            hip_check(hipMemcpyAsync(g.shared, shared_or_null, sizeof(float) * X, hipMemcpyHostToDevice, s), "shared upload");
        enqueue_grouped(ctx, layer, T, k, g.ids, g.w, g.x, shared_or_null ? g.shared : nullptr, g.out, s);
        hip_check(hipMemcpyAsync(out, g.out, sizeof(float) * X, hipMemcpyDeviceToHost, s), "output download");
        drain(ctx, s);
    });
}

int32_t xl_grouped_forward_async(xl_context* ctx, int32_t layer, int32_t T, int32_t k, const int32_t* d_ids,
                                 const float* d_w, const float* d_x, const float* d_shared_or_null, float* d_out,
                                 void* stream, xl_error* err) {
    return guarded(ctx, err, [&] {
        ready(ctx, true);
        check_layer(ctx, layer);
        check_grouped(ctx, T, k);
        need(d_ids && d_w && d_x && d_out, XL_E_ARG, "null device pointer");
        hipStream_t s = pick_stream(ctx, stream);
        Ordered ord(ctx, s);
        enqueue_grouped(ctx, layer, T, k, d_ids, d_w, d_x, d_shared_or_null, d_out, s);
    });
}

int32_t xl_route_async(xl_context* ctx, const float* d_logits, int32_t T, int32_t stride, const float* d_bias_or_null,
                       int32_t n, int32_t k, float scale, int32_t* d_ids, float* d_w, void* stream, xl_error* err) {
    return guarded(ctx, err, [&] {
        ready(ctx, false);
        need(d_logits && d_ids && d_w, XL_E_ARG, "null device pointer");
        need(T >= 1, XL_E_ARG, "token count below 1");
        need(n >= 1 && n <= xl::kRouteMaxExperts, XL_E_ARG, "expert count outside 1..4096");
        need(k >= 1 && k <= 16 && k <= n, XL_E_ARG, "pick count outside 1..min(16, n)");
        need(stride >= n, XL_E_ARG, "logit stride below the expert count");
        need(std::isfinite(scale) && scale >= 0.0f, XL_E_ARG, "route scale must be finite and >= 0");
        hipStream_t s = pick_stream(ctx, stream);
        Ordered ord(ctx, s);
        hip_check(xl::dev::launch_route(d_logits, T, stride, d_bias_or_null, n, k, scale, d_ids, d_w, ctx->err_flag, s),
                  "route launch");
    });
}

int32_t xl_layer_forward_routed_async(xl_context* ctx, int32_t layer, const float* d_logits, const float* d_bias_or_null,
                                      int32_t k, float scale, const float* d_x, const float* d_shared_or_null,
                                      float* d_out, void* stream, xl_error* err) {
    return guarded(ctx, err, [&] {
        ready(ctx, true);
        check_layer(ctx, layer);
        need(k >= 1 && k <= ctx->cfg.max_picks, XL_E_ARG, "pick count outside 1..max_picks");
        need(k <= ctx->cfg.n_experts, XL_E_ARG, "router: more picks than experts");
        need(ctx->cfg.n_experts <= xl::kRouteMaxExperts, XL_E_ARG, "router: more than 4096 experts");
        need(std::isfinite(scale) && scale >= 0.0f, XL_E_ARG, "route scale must be finite and >= 0");
        need(d_logits && d_x && d_out, XL_E_ARG, "null device pointer");
        hipStream_t s = pick_stream(ctx, stream);
        Ordered ord(ctx, s);
        const int n = ctx->cfg.n_experts;
        // one launch that routes in its prologue where the streaming kernel has the
        // layer, else the router kernel and then the layer
        if (enqueue_layer_routed(ctx, layer, d_logits, d_bias_or_null, k, scale, d_x, d_shared_or_null, d_out, s,
                                 ord.stop())) {
            ord.carried_by_launch(true);
            return;
        }
        hip_check(xl::dev::launch_route(d_logits, 1, n, d_bias_or_null, n, k, scale, ctx->ids, ctx->w, ctx->err_flag, s),
                  "route launch");
        ord.carried_by_launch(enqueue_layer(ctx, layer, ctx->ids, ctx->w, k, d_x, d_shared_or_null, d_out, s, nullptr,
                                            nullptr, ord.stop()));
    });
}

int32_t xl_grouped_forward_routed_async(xl_context* ctx, int32_t layer, int32_t T, const float* d_logits,
                                        const float* d_bias_or_null, int32_t k, float scale, const float* d_x,
                                        const float* d_shared_or_null, float* d_out, void* stream, xl_error* err) {
    return guarded(ctx, err, [&] {
        ready(ctx, true);
        check_layer(ctx, layer);
        check_grouped(ctx, T, k);
        need(ctx->cfg.n_experts <= xl::kRouteMaxExperts, XL_E_ARG, "router: more than 4096 experts");
        need(std::isfinite(scale) && scale >= 0.0f, XL_E_ARG, "route scale must be finite and >= 0");
        need(d_logits && d_x && d_out, XL_E_ARG, "null device pointer");
        hipStream_t s = pick_stream(ctx, stream);
        Ordered ord(ctx, s);
        const int n = ctx->cfg.n_experts;
        auto& g = ctx->grp;
        hip_check(xl::dev::launch_route(d_logits, T, n, d_bias_or_null, n, k, scale, g.ids, g.w, ctx->err_flag, s),
                  "route launch");
        enqueue_grouped(ctx, layer, T, k, g.ids, g.w, d_x, d_shared_or_null, d_out, s);
    });
}

int32_t xl_layer_forward(xl_context* ctx, int32_t layer, const int32_t* ids, const float* w, int32_t k, const float* x,
                         const float* shared_or_null, float* out, xl_error* err) {
    return guarded(ctx, err, [&] {
        ready(ctx, true);
        check_layer(ctx, layer);
        check_ids(ctx, ids, k);
        check_finite(w, size_t(k), "route weights");
        check_finite(x, size_t(ctx->cfg.dim), "input vector");
        if (shared_or_null) check_finite(shared_or_null, size_t(ctx->cfg.dim), "shared vector");
        need(out != nullptr, XL_E_ARG, "null output");
        hipStream_t s = ctx->stream;
        Ordered ord(ctx, s);
        const int dim = ctx->cfg.dim;
        hip_check(hipMemcpyAsync(ctx->ids, ids, sizeof(int32_t) * k, hipMemcpyHostToDevice, s), "ids upload");
        hip_check(hipMemcpyAsync(ctx->w, w, sizeof(float) * k, hipMemcpyHostToDevice, s), "weights upload");
        hip_check(hipMemcpyAsync(ctx->x, x, sizeof(float) * dim, hipMemcpyHostToDevice, s), "x upload");
        if (shared_or_null)
            hip_check(hipMemcpyAsync(ctx->shared, shared_or_null, sizeof(float) * dim, hipMemcpyHostToDevice, s),
                      "shared upload");
        enqueue_layer(ctx, layer, ctx->ids, ctx->w, k, ctx->x, shared_or_null ? ctx->shared : nullptr, ctx->out, s);
        hip_check(hipMemcpyAsync(out, ctx->out, sizeof(float) * dim, hipMemcpyDeviceToHost, s), "output download");
        drain(ctx, s);
    });
}

int32_t xl_expert_trace(xl_context* ctx, int32_t layer, int32_t expert, const float* x, float* g, float* u, float* h,
                        void* q8h, float* y, xl_error* err) {
    return guarded(ctx, err, [&] {
        ready(ctx, true);
        check_layer(ctx, layer);
        const int32_t id = expert;
        check_ids(ctx, &id, 1);
        check_finite(x, size_t(ctx->cfg.dim), "input vector");
        hipStream_t s = ctx->stream;
        Ordered ord(ctx, s);
        const int dim = ctx->cfg.dim, ff = ctx->cfg.ff;
        hip_check(hipMemcpyAsync(ctx->ids, &id, sizeof id, hipMemcpyHostToDevice, s), "ids upload");
        hip_check(hipMemcpyAsync(ctx->x, x, sizeof(float) * dim, hipMemcpyHostToDevice, s), "x upload");
        enqueue_layer(ctx, layer, ctx->ids, nullptr, 1, ctx->x, nullptr, nullptr, s, ctx->g, ctx->u);
        // Standard 292-byte Q8_K blocks of h, same kernel as the hot path.
        hip_check(xl::dev::launch_q8k(ctx->h, ff / 256, ctx->hq, ctx->hd, ctx->q8std, ctx->err_flag, s), "Q8_K(h) launch");
        if (g) hip_check(hipMemcpyAsync(g, ctx->g, sizeof(float) * ff, hipMemcpyDeviceToHost, s), "g download");
        if (u) hip_check(hipMemcpyAsync(u, ctx->u, sizeof(float) * ff, hipMemcpyDeviceToHost, s), "u download");
        if (h) hip_check(hipMemcpyAsync(h, ctx->h, sizeof(float) * ff, hipMemcpyDeviceToHost, s), "h download");
        if (q8h) hip_check(hipMemcpyAsync(q8h, ctx->q8std, size_t(ff / 256) * 292, hipMemcpyDeviceToHost, s), "q8h download");
        if (y) hip_check(hipMemcpyAsync(y, ctx->y, sizeof(float) * dim, hipMemcpyDeviceToHost, s), "y download");
        drain(ctx, s);
    });
}

int32_t xl_layer_forward_async(xl_context* ctx, int32_t layer, const int32_t* d_ids, const float* d_w, int32_t k,
                               const float* d_x, const float* d_shared_or_null, float* d_out, void* stream,
                               xl_error* err) {
    return guarded(ctx, err, [&] {
        ready(ctx, true);
        check_layer(ctx, layer);
        need(k >= 1 && k <= ctx->cfg.max_picks, XL_E_ARG, "pick count outside 1..max_picks");
        need(d_ids && d_w && d_x && d_out, XL_E_ARG, "null device pointer");
        hipStream_t s = pick_stream(ctx, stream);
        Ordered ord(ctx, s);
        ord.carried_by_launch(enqueue_layer(ctx, layer, d_ids, d_w, k, d_x, d_shared_or_null, d_out, s, nullptr, nullptr,
                                            ord.stop()));
    });
}

int32_t xl_layer_forward_exact_async(xl_context* ctx, int32_t layer, const int32_t* d_ids, const float* d_w,
                                     int32_t k, const float* d_x, const float* d_shared_or_null, float* d_out,
                                     void* stream, xl_error* err) {
    return guarded(ctx, err, [&] {
        ready(ctx, true);
        check_layer(ctx, layer);
        need(k >= 1 && k <= ctx->cfg.max_picks, XL_E_ARG, "pick count outside 1..max_picks");
        need(d_ids && d_w && d_x && d_out, XL_E_ARG, "null device pointer");
        hipStream_t s = pick_stream(ctx, stream);
        Ordered ord(ctx, s);
        enqueue_layer_exact(ctx, layer, d_ids, d_w, k, d_x, d_shared_or_null, d_out, s);
    });
}

int32_t xl_layer_forward_prenorm_async(xl_context* ctx, int32_t layer, const int32_t* d_ids, const float* d_w,
                                       int32_t k, const float* d_h, int32_t H, const float* d_mix,
                                       const float* d_norm_w_or_null, float eps, float* d_x,
                                       const float* d_shared_or_null, float* d_out, void* stream, xl_error* err) {
    return guarded(ctx, err, [&] {
        ready(ctx, true);
        check_layer(ctx, layer);
        need(k >= 1 && k <= ctx->cfg.max_picks, XL_E_ARG, "pick count outside 1..max_picks");
        need(d_ids && d_w && d_h && d_mix && d_x && d_out, XL_E_ARG, "null device pointer");
        need(H >= 1 && H <= 4, XL_E_ARG, "hc geometry: H in 1..4");
        need(std::isfinite(eps) && eps > 0.0f, XL_E_ARG, "hc epsilon must be finite and positive");
        const uint64_t D = uint64_t(ctx->cfg.dim);
        // x is written while h, mix and the norm weights are read; out is written
        // while h is read by workgroups that start later
        need(apart(d_x, D * 4, d_h, uint64_t(H) * D * 4) && apart(d_x, D * 4, d_mix, 32) &&
                 (!d_norm_w_or_null || apart(d_x, D * 4, d_norm_w_or_null, D * 4)) &&
                 apart(d_out, D * 4, d_h, uint64_t(H) * D * 4) && apart(d_out, D * 4, d_x, D * 4),
             XL_E_ARG, "pre-norm layer: x or out overlaps an input");
        hipStream_t s = pick_stream(ctx, stream);
        Ordered ord(ctx, s);
        if (H == 1 && enqueue_layer_prenorm(ctx, layer, d_ids, d_w, k, d_h, d_mix, d_norm_w_or_null, eps, d_x,
                                            d_shared_or_null, d_out, s, ord.stop())) {
            ord.carried_by_launch(true);
            return;
        }
        hip_check(xl::dev::launch_hc_pre_norm(d_h, d_mix, d_norm_w_or_null, int(D), H, 1, eps, d_x, s, nullptr),
                  "hc_pre_norm launch");
        ord.carried_by_launch(enqueue_layer(ctx, layer, d_ids, d_w, k, d_x, d_shared_or_null, d_out, s, nullptr,
                                            nullptr, ord.stop()));
    });
}

int32_t xl_layer_forward_post_async(xl_context* ctx, int32_t layer, const int32_t* d_ids, const float* d_w,
                                    int32_t k, const float* d_x, const float* d_shared_or_null, float* d_out,
                                    const float* d_res, const float* d_post, const float* d_comb, int32_t H,
                                    float* d_post_out, void* stream, xl_error* err) {
    return guarded(ctx, err, [&] {
        ready(ctx, true);
        check_layer(ctx, layer);
        need(k >= 1 && k <= ctx->cfg.max_picks, XL_E_ARG, "pick count outside 1..max_picks");
        need(d_ids && d_w && d_x && d_out && d_res && d_post && d_comb && d_post_out, XL_E_ARG, "null device pointer");
        need(H >= 1 && H <= 4, XL_E_ARG, "hc geometry: H in 1..4");
        const uint64_t D = uint64_t(ctx->cfg.dim), ob = uint64_t(H) * D * 4;
        // post_out: res itself (in place) or apart from every input and from out; out
        // apart from what hc_post reads (other workgroups read those columns later)
        need(d_post_out == d_res || apart(d_post_out, ob, d_res, ob), XL_E_ARG, "hc output overlaps the residual streams");
        need(apart(d_post_out, ob, d_out, D * 4) && apart(d_post_out, ob, d_x, D * 4) &&
                 (!d_shared_or_null || apart(d_post_out, ob, d_shared_or_null, D * 4)) &&
                 apart(d_post_out, ob, d_post, 32) && apart(d_post_out, ob, d_comb, 256) &&
                 apart(d_post_out, ob, d_ids, uint64_t(k) * 4) && apart(d_post_out, ob, d_w, uint64_t(k) * 4),
             XL_E_ARG, "hc output overlaps an input");
        need(apart(d_out, D * 4, d_res, ob) && apart(d_out, D * 4, d_post, 32) && apart(d_out, D * 4, d_comb, 256),
             XL_E_ARG, "layer output overlaps an hc_post input");
        hipStream_t s = pick_stream(ctx, stream);
        Ordered ord(ctx, s);
        if (enqueue_layer_post(ctx, layer, d_ids, d_w, k, d_x, d_shared_or_null, d_out, d_res, d_post, d_comb, H,
                               d_post_out, s, ord.stop())) {
            ord.carried_by_launch(true);
            return;
        }
        enqueue_layer(ctx, layer, d_ids, d_w, k, d_x, d_shared_or_null, d_out, s);
        hip_check(xl::dev::launch_hc_post(d_out, d_res, d_post, d_comb, int(D), H, 1, d_post_out, s, ord.stop()),
                  "hc_post launch");
        ord.carried_by_launch(true);
    });
}

int32_t xl_layer_trace_async(xl_context* ctx, int32_t layer, const int32_t* d_ids, const float* d_w, int32_t k,
                             const float* d_x, const float* d_shared_or_null, float* d_out, void* d_q8x, void* d_q8h,
                             float* d_h, int32_t* d_ints, float* d_y, int32_t* kernel_out, void* stream,
                             xl_error* err) {
    return guarded(ctx, err, [&] {
        ready(ctx, true);
        check_layer(ctx, layer);
        need(k >= 1 && k <= ctx->cfg.max_picks, XL_E_ARG, "pick count outside 1..max_picks");
        need(d_ids && d_w && d_x && d_out, XL_E_ARG, "null device pointer");
        need(d_q8x || d_q8h || d_h || d_ints || d_y, XL_E_ARG, "trace: no output requested");
        LayerTrace tr;
        tr.q8x = static_cast<uint8_t*>(d_q8x);
        tr.q8h = static_cast<uint8_t*>(d_q8h);
        tr.h = d_h;
        tr.ints = d_ints;
        tr.y = d_y;
        hipStream_t s = pick_stream(ctx, stream);
        Ordered ord(ctx, s);
        ord.carried_by_launch(
            enqueue_layer(ctx, layer, d_ids, d_w, k, d_x, d_shared_or_null, d_out, s, nullptr, nullptr, ord.stop(), &tr));
        if (kernel_out) *kernel_out = tr.kernel;
    });
}

int32_t xl_grouped_trace_async(xl_context* ctx, int32_t layer, int32_t T, int32_t k, const int32_t* d_ids,
                               const float* d_w, const float* d_x, const float* d_shared_or_null, float* d_out,
                               void* d_q8x, void* d_q8h, float* d_h, int32_t* d_ints, float* d_y, void* stream,
                               xl_error* err) {
    return guarded(ctx, err, [&] {
        ready(ctx, true);
        check_layer(ctx, layer);
        check_grouped(ctx, T, k);
        need(d_ids && d_w && d_x && d_out, XL_E_ARG, "null device pointer");
        need(d_q8x || d_q8h || d_h || d_ints || d_y, XL_E_ARG, "trace: no output requested");
        LayerTrace tr;
        tr.q8x = static_cast<uint8_t*>(d_q8x);
        tr.q8h = static_cast<uint8_t*>(d_q8h);
        tr.h = d_h;
        tr.ints = d_ints;
        tr.y = d_y;
        hipStream_t s = pick_stream(ctx, stream);
        Ordered ord(ctx, s);
        enqueue_grouped(ctx, layer, T, k, d_ids, d_w, d_x, d_shared_or_null, d_out, s, &tr);
    });
}

int32_t xl_combine_async(xl_context* ctx, const int32_t* d_ids, const float* d_w, int32_t k, const float* d_rows,
                         int32_t dim, const float* d_shared_or_null, float* d_out, void* stream, xl_error* err) {
    return guarded(ctx, err, [&] {
        ready(ctx, false);
        need(k >= 1 && k <= 16, XL_E_ARG, "pick count outside 1..16");
        need(dim >= 1 && dim <= (1 << 24), XL_E_ARG, "dim outside 1..2^24");
        need(d_ids && d_w && d_rows && d_out, XL_E_ARG, "null device pointer");
        hipStream_t s = pick_stream(ctx, stream);
        Ordered ord(ctx, s);
        hip_check(xl::dev::launch_combine(d_ids, d_w, k, d_rows, dim, d_shared_or_null, d_out, s), "combine");
    });
}

int32_t xl_layer_forward_per32(xl_context* ctx, int32_t layer, const int32_t* ids, const float* w, int32_t k,
                               const float* x, const float* shared_or_null, float* y_or_null, float* out_or_null,
                               xl_error* err) {
    return guarded(ctx, err, [&] {
        ready(ctx, true);
        check_layer(ctx, layer);
        check_ids(ctx, ids, k);
        check_finite(x, size_t(ctx->cfg.dim), "input vector");
        need(y_or_null || out_or_null, XL_E_ARG, "neither per-pick outputs nor a combined output requested");
        if (out_or_null) check_finite(w, size_t(k), "route weights");
        if (out_or_null && shared_or_null) check_finite(shared_or_null, size_t(ctx->cfg.dim), "shared vector");
        hipStream_t s = ctx->stream;
        Ordered ord(ctx, s);
        const int dim = ctx->cfg.dim;
        hip_check(hipMemcpyAsync(ctx->ids, ids, sizeof(int32_t) * k, hipMemcpyHostToDevice, s), "ids upload");
        if (out_or_null) hip_check(hipMemcpyAsync(ctx->w, w, sizeof(float) * k, hipMemcpyHostToDevice, s), "weights upload");
        hip_check(hipMemcpyAsync(ctx->x, x, sizeof(float) * dim, hipMemcpyHostToDevice, s), "x upload");
        const bool sh = out_or_null && shared_or_null;
        if (sh)
            hip_check(hipMemcpyAsync(ctx->shared, shared_or_null, sizeof(float) * dim, hipMemcpyHostToDevice, s),
                      "shared upload");
        enqueue_per32(ctx, layer, ctx->ids, ctx->w, k, ctx->x, sh ? ctx->shared : nullptr, ctx->y,
                      out_or_null ? ctx->out : nullptr, s);
        if (y_or_null)
            hip_check(hipMemcpyAsync(y_or_null, ctx->y, sizeof(float) * size_t(k) * dim, hipMemcpyDeviceToHost, s),
                      "per-pick output download");
        if (out_or_null)
            hip_check(hipMemcpyAsync(out_or_null, ctx->out, sizeof(float) * dim, hipMemcpyDeviceToHost, s),
                      "output download");
        drain(ctx, s);
    });
}

int32_t xl_layer_forward_per32_async(xl_context* ctx, int32_t layer, const int32_t* d_ids, const float* d_w, int32_t k,
                                     const float* d_x, const float* d_shared_or_null, float* d_y,
                                     float* d_out_or_null, void* stream, xl_error* err) {
    return guarded(ctx, err, [&] {
        ready(ctx, true);
        check_layer(ctx, layer);
        need(k >= 1 && k <= ctx->cfg.max_picks, XL_E_ARG, "pick count outside 1..max_picks");
        need(d_ids && d_x && d_y, XL_E_ARG, "null device pointer");
        need(!d_out_or_null || d_w, XL_E_ARG, "a combined output needs route weights");
        hipStream_t s = pick_stream(ctx, stream);
        Ordered ord(ctx, s);
        enqueue_per32(ctx, layer, d_ids, d_w, k, d_x, d_shared_or_null, d_y, d_out_or_null, s);
    });
}

int32_t xl_quantize_per32_async(xl_context* ctx, const float* d_x, int32_t rows, int32_t k, int8_t* d_q, float* d_d,
                                void* stream, xl_error* err) {
    return guarded(ctx, err, [&] {
        ready(ctx, false);
        need(d_x && d_q && d_d, XL_E_ARG, "null device pointer");
        need(rows >= 1 && k >= 32 && k % 32 == 0, XL_E_ARG, "rows >= 1 and k a positive multiple of 32");
        need(int64_t(rows) * k <= int64_t(1) << 30, XL_E_ARG, "more than 2^30 values");
        hipStream_t s = pick_stream(ctx, stream);
        Ordered ord(ctx, s);
        hip_check(xl::dev::launch_quant32(d_x, rows, k, d_q, d_d, ctx->err_flag, s),
                  "quant32 launch");
    });
}

int32_t xl_matvec_per32_async(xl_context* ctx, int32_t type, const void* d_planar, int32_t n, int32_t k,
                              const int8_t* d_q, const float* d_d, float* d_y, void* stream, xl_error* err) {
    return guarded(ctx, err, [&] {
        ready(ctx, false);
        need(xl::supported_type(type) || xl::dense_type(type), XL_E_ARG, "unsupported block type");
        need(d_planar && d_q && d_d && d_y, XL_E_ARG, "null device pointer");
        need(reinterpret_cast<uintptr_t>(d_q) % 16 == 0, XL_E_ARG, "quants not 16-byte aligned");
        need(n >= 1 && n <= (1 << 24) && k >= 256 && k % 256 == 0 && k <= (1 << 20), XL_E_ARG,
             "n in 1..2^24 and k a multiple of 256 up to 2^20");
        const xl::MatRef m = per32_matrix(type, d_planar, n, k);
        hipStream_t s = pick_stream(ctx, stream);
        Ordered ord(ctx, s);
        hip_check(xl::dev::launch_mv32(nullptr, nullptr, m, m, 1, 0, 0, 1, n, k, d_q, 0, d_d, 0, d_y, nullptr, 0,
                                       ctx->tables, ctx->err_flag, s),
                  "per32 matvec launch");
    });
}

uint64_t xl_shared_work_bytes(int32_t dim, int32_t ff, int32_t T) {
    if (dim < 256 || ff < 256 || dim % 256 || ff % 256 || dim > (1 << 16) || ff > (1 << 16) || T < 1 || T > 8192)
        return 0;
    return shared_work(dim, ff, T).bytes;
}

namespace {

void check_shared(const xl_context* ctx, int32_t type_gate, const void* d_gate, int32_t type_up, const void* d_up,
                  int32_t type_down, const void* d_down, int32_t ff, int32_t T, const float* d_x, const float* d_out) {
    need(d_gate && d_up && d_down && d_x && d_out, XL_E_ARG, "null device pointer");
    need(ff >= 256 && ff % 256 == 0 && ff <= (1 << 16), XL_E_ARG, "shared ff a multiple of 256 up to 65536");
    need(T >= 1 && T <= 8192, XL_E_ARG, "T outside 1..8192");
    for (const int32_t t : {type_gate, type_up, type_down})
        need(xl::supported_type(t) || xl::dense_type(t), XL_E_ARG, "unsupported shared-expert block type");
    (void)ctx;
}

// hip_backend.cpp:664-666: mv(gate, up), swiglu, mv(down), T tokens per launch,
// the intermediates carved from `base` (256-byte aligned, w.bytes long).
void enqueue_shared(xl_context* ctx, int32_t type_gate, const void* d_gate, int32_t type_up, const void* d_up,
                    int32_t type_down, const void* d_down, int32_t ff, int32_t T, const float* d_x, float* d_out,
                    uint8_t* base, const SharedWork& w, hipStream_t s) {
    const int dim = ctx->cfg.dim;
    float* g = reinterpret_cast<float*>(base + w.g);
    float* u = reinterpret_cast<float*>(base + w.u);
    int8_t* xq = reinterpret_cast<int8_t*>(base + w.xq);
    int8_t* hq = reinterpret_cast<int8_t*>(base + w.hq);
    float* xd = reinterpret_cast<float*>(base + w.xd);
    float* hd = reinterpret_cast<float*>(base + w.hd);
    const xl::MatRef mg = per32_matrix(type_gate, d_gate, ff, dim), mu = per32_matrix(type_up, d_up, ff, dim);
    const xl::MatRef md = per32_matrix(type_down, d_down, dim, ff);
    hip_check(xl::dev::launch_quant32(d_x, T, dim, xq, xd, ctx->err_flag, s), "quant32(x) launch");
    hip_check(xl::dev::launch_mv32(nullptr, nullptr, mg, mu, T, 0, 0, 2, ff, dim, xq, size_t(dim), xd,
                                   size_t(dim / 32), g, u, size_t(ff), ctx->tables, ctx->err_flag, s),
              "shared gate/up launch");
    hip_check(xl::dev::launch_swiglu_quant32(g, u, T, ff, ctx->cfg.swiglu_limit, hq, hd, s),
              "shared SwiGLU + quant32(h) launch");
    hip_check(xl::dev::launch_mv32(nullptr, nullptr, md, md, T, 0, 0, 1, dim, ff, hq, size_t(ff), hd,
                                   size_t(ff / 32), d_out, nullptr, size_t(dim), ctx->tables, ctx->err_flag, s),
              "shared down launch");
}

}  // namespace

int32_t xl_shared_forward_async(xl_context* ctx, int32_t type_gate, const void* d_gate, int32_t type_up,
                                const void* d_up, int32_t type_down, const void* d_down, int32_t ff, int32_t T,
                                const float* d_x, float* d_out, void* d_work, uint64_t work_bytes, void* stream,
                                xl_error* err) {
    return guarded(ctx, err, [&] {
        ready(ctx, false);
        check_shared(ctx, type_gate, d_gate, type_up, d_up, type_down, d_down, ff, T, d_x, d_out);
        need(d_work != nullptr, XL_E_ARG, "null workspace");
        const SharedWork w = shared_work(ctx->cfg.dim, ff, T);
        need(work_bytes >= w.bytes, XL_E_ARG, "workspace smaller than xl_shared_work_bytes(dim, ff)");
        need(reinterpret_cast<uintptr_t>(d_work) % 256 == 0, XL_E_ARG, "workspace not 256-byte aligned");
        hipStream_t s = pick_stream(ctx, stream);
        Ordered ord(ctx, s);
        enqueue_shared(ctx, type_gate, d_gate, type_up, d_up, type_down, d_down, ff, T, d_x, d_out,
                       static_cast<uint8_t*>(d_work), w, s);
    });
}

int32_t xl_shared_forward_noalloc(xl_context* ctx, int32_t type_gate, const void* d_gate, int32_t type_up,
                                  const void* d_up, int32_t type_down, const void* d_down, int32_t ff, int32_t T,
                                  const float* d_x, float* d_out, void* stream, xl_error* err) {
    return guarded(ctx, err, [&] {
        ready(ctx, false);
        check_shared(ctx, type_gate, d_gate, type_up, d_up, type_down, d_down, ff, T, d_x, d_out);
        const SharedWork w = shared_work(ctx->cfg.dim, ff, T);
        if (w.bytes > xl::kNoAllocScratchBytes)
            fail(XL_E_ARG, "xl_shared_forward_noalloc: %llu bytes of intermediates for T = %d exceed the %llu-byte "
                           "static scratch (xl_shared_work_bytes gives the need; use xl_shared_forward_async)",
                 (unsigned long long)w.bytes, T, (unsigned long long)xl::kNoAllocScratchBytes);
        void* scratch = nullptr;   // this device's copy (found once, at xl_open)
        hip_check(xl::dev::noalloc_scratch(ctx->cfg.device, &scratch), "no-allocation scratch address");
        hipStream_t s = pick_stream(ctx, stream);
        Ordered ord(ctx, s);
        // Every intermediate is written before it is read (quant32 fills xq/xd, the
        // gate/up rows fill g/u, the SwiGLU fills hq/hd): nothing to clear.
        enqueue_shared(ctx, type_gate, d_gate, type_up, d_up, type_down, d_down, ff, T, d_x, d_out,
                       static_cast<uint8_t*>(scratch), w, s);
    });
}

int32_t xl_moe_block_async(xl_context* ctx, int32_t layer, const int32_t* d_ids, const float* d_w, int32_t k,
                           const float* d_x, int32_t type_gate, const void* d_gate, int32_t type_up, const void* d_up,
                           int32_t type_down, const void* d_down, int32_t ff, void* d_work, uint64_t work_bytes,
                           const float* d_res, const float* d_post, const float* d_comb, int32_t H, float* d_out,
                           float* d_post_out, void* stream, xl_error* err) {
    return guarded(ctx, err, [&] {
        ready(ctx, true);
        check_layer(ctx, layer);
        need(k >= 1 && k <= ctx->cfg.max_picks, XL_E_ARG, "pick count outside 1..max_picks");
        check_shared(ctx, type_gate, d_gate, type_up, d_up, type_down, d_down, ff, 1, d_x, d_out);
        need(d_ids && d_w && d_res && d_post && d_comb && d_post_out && d_work, XL_E_ARG, "null device pointer");
        need(H >= 1 && H <= 4, XL_E_ARG, "hc geometry: H in 1..4");
        const int dim = ctx->cfg.dim;
        const SharedWork w = shared_work(dim, ff, 1);
        need(work_bytes >= w.bytes, XL_E_ARG, "workspace smaller than xl_shared_work_bytes(dim, ff, 1)");
        need(reinterpret_cast<uintptr_t>(d_work) % 256 == 0, XL_E_ARG, "workspace not 256-byte aligned");
        const uint64_t D = uint64_t(dim), ob = uint64_t(H) * D * 4;
        // the workspace, out and post_out each apart from everything the block reads or
        // writes (post_out may be res itself)
        const std::pair<const void*, uint64_t> ins[] = {{d_x, D * 4}, {d_ids, uint64_t(k) * 4}, {d_w, uint64_t(k) * 4},
                                                        {d_post, 32}, {d_comb, 256}, {d_res, ob}};
        for (const auto& [p, b] : ins) {
            need(apart(d_work, w.bytes, p, b), XL_E_ARG, "workspace overlaps an input");
            need(apart(d_out, D * 4, p, b), XL_E_ARG, "block output overlaps an input");
            need(p == d_res || apart(d_post_out, ob, p, b), XL_E_ARG, "hc output overlaps an input");
        }
        need(d_post_out == d_res || apart(d_post_out, ob, d_res, ob), XL_E_ARG, "hc output overlaps the residual streams");
        need(apart(d_work, w.bytes, d_out, D * 4) && apart(d_work, w.bytes, d_post_out, ob) &&
                 apart(d_out, D * 4, d_post_out, ob),
             XL_E_ARG, "workspace, block output and hc output overlap");
        uint8_t* base = static_cast<uint8_t*>(d_work);
        float* g = reinterpret_cast<float*>(base + w.g);
        float* u = reinterpret_cast<float*>(base + w.u);
        int8_t* xq = reinterpret_cast<int8_t*>(base + w.xq);
        int8_t* hq = reinterpret_cast<int8_t*>(base + w.hq);
        float* xd = reinterpret_cast<float*>(base + w.xd);
        float* hd = reinterpret_cast<float*>(base + w.hd);
        hipStream_t s = pick_stream(ctx, stream);
        Ordered ord(ctx, s);
        // the routed layer (no shared row): out = its fixed-order combine; the
        // streaming launch also writes x per 32
        bool fused = false;
        if ((ctx->path == 1 || ctx->path == 4) && !ctx->prof.on) {
            xl::Layer3Args a = layer3_args(ctx, layer, d_ids, d_w, k, d_x, nullptr, d_out, s, nullptr);
            a.p32_q = xq;
            a.p32_d = xd;
            const hipError_t e = xl::dev::launch_stream(a, ctx->gu_mask[size_t(layer)], ctx->dn_mask[size_t(layer)],
                                                        ctx->cus, s, nullptr);
            if (e == hipSuccess) {
                fused = true;
                ++ctx->launches[XL_LAUNCH_BLOCK];
            } else if (e != hipErrorNotSupported) {
                hip_check(e, "streaming layer with quant32(x)");
            }
            (void)hipGetLastError();
        }
        if (!fused) {
            hip_check(xl::dev::launch_quant32(d_x, 1, dim, xq, xd, ctx->err_flag, s), "quant32(x) launch");
            enqueue_layer(ctx, layer, d_ids, d_w, k, d_x, nullptr, d_out, s);
        }
        // the shared expert: gate/up rows, SwiGLU + quant32(h), then its down rows
        // added to the routed output (out = routed + shared) and hc_post of the sum
        const xl::MatRef mg = per32_matrix(type_gate, d_gate, ff, dim), mu = per32_matrix(type_up, d_up, ff, dim);
        const xl::MatRef md = per32_matrix(type_down, d_down, dim, ff);
        hip_check(xl::dev::launch_mv32(nullptr, nullptr, mg, mu, 1, 0, 0, 2, ff, dim, xq, size_t(dim), xd,
                                       size_t(dim / 32), g, u, size_t(ff), ctx->tables, ctx->err_flag, s),
                  "shared gate/up launch");
        hip_check(xl::dev::launch_swiglu_quant32(g, u, 1, ff, ctx->cfg.swiglu_limit, hq, hd, s),
                  "shared SwiGLU + quant32(h) launch");
        const xl::dev::Mv32Post ep{d_out, d_res, d_post, d_comb, d_post_out, H};
        hip_check(xl::dev::launch_mv32(nullptr, nullptr, md, md, 1, 0, 0, 1, dim, ff, hq, size_t(ff), hd,
                                       size_t(ff / 32), d_out, nullptr, size_t(dim), ctx->tables, ctx->err_flag, s, &ep),
                  "shared down + hc_post launch");
    });
}

int32_t xl_hc_pre_norm_async(xl_context* ctx, const float* d_h, const float* d_mix, const float* d_w_or_null,
                             int32_t D, int32_t H, int32_t T, float eps, float* d_x, void* stream, xl_error* err) {
    return guarded(ctx, err, [&] {
        ready(ctx, false);
        // hc.cpp:5-7,89-92: geometry, a finite positive epsilon, no null input,
        // x neither h itself nor overlapping h, mix or w
        need(d_h && d_mix && d_x, XL_E_ARG, "null device pointer");
        need(D >= 1 && D <= 32768 && H >= 1 && H <= 4 && T >= 1 && T <= 8192, XL_E_ARG,
             "hc geometry: D in 1..32768, H in 1..4, T in 1..8192");
        need(std::isfinite(eps) && eps > 0.0f, XL_E_ARG, "hc epsilon must be finite and positive");
        const uint64_t xb = uint64_t(T) * D * 4;
        const auto overlaps = [&](const void* p, uint64_t bytes) {
            const uintptr_t a = reinterpret_cast<uintptr_t>(d_x), b = reinterpret_cast<uintptr_t>(p);
            return a <= b ? b - a < xb : a - b < bytes;
        };
        need(!overlaps(d_h, uint64_t(T) * H * D * 4) && !overlaps(d_mix, uint64_t(T) * 32) &&
                 (!d_w_or_null || !overlaps(d_w_or_null, uint64_t(D) * 4)),
             XL_E_ARG, "hc output overlaps an input");
        hipStream_t s = pick_stream(ctx, stream);
        Ordered ord(ctx, s);
        hip_check(xl::dev::launch_hc_pre_norm(d_h, d_mix, d_w_or_null, D, H, T, eps, d_x, s, ord.stop()),
                  "hc_pre_norm launch");
        ord.carried_by_launch(true);   // the launch records the ordering event itself
    });
}

int32_t xl_hc_post_async(xl_context* ctx, const float* d_y, const float* d_res, const float* d_post,
                         const float* d_comb, int32_t D, int32_t H, int32_t T, float* d_out, void* stream,
                         xl_error* err) {
    return guarded(ctx, err, [&] {
        ready(ctx, false);
        need(d_y && d_res && d_post && d_comb && d_out, XL_E_ARG, "null device pointer");
        need(D >= 1 && D <= 32768 && H >= 1 && H <= 4 && T >= 1 && T <= 8192, XL_E_ARG,
             "hc geometry: D in 1..32768, H in 1..4, T in 1..8192");
        const uint64_t ob = uint64_t(T) * H * D * 4;
        const auto overlaps = [&](const void* p, uint64_t bytes) {
            const uintptr_t a = reinterpret_cast<uintptr_t>(d_out), b = reinterpret_cast<uintptr_t>(p);
            return a <= b ? b - a < ob : a - b < bytes;
        };
        // hc.cpp:108-109,113-114: out may be res itself (in place), never a
        // partial overlap with res nor any overlap with y, post or comb.
        need(d_out == d_res || !overlaps(d_res, ob), XL_E_ARG, "hc output overlaps the residual streams");
        need(!overlaps(d_y, uint64_t(T) * D * 4) && !overlaps(d_post, uint64_t(T) * 32) &&
                 !overlaps(d_comb, uint64_t(T) * 256),
             XL_E_ARG, "hc output overlaps an input");
        hipStream_t s = pick_stream(ctx, stream);
        Ordered ord(ctx, s);
        hip_check(xl::dev::launch_hc_post(d_y, d_res, d_post, d_comb, D, H, T, d_out, s, ord.stop()), "hc_post launch");
        ord.carried_by_launch(true);   // the launch records the ordering event itself
    });
}

int32_t xl_sync(xl_context* ctx, void* stream, xl_error* err) {
    return guarded(ctx, err, [&] {
        need(ctx != nullptr, XL_E_ARG, "null context");
        hip_check(hipSetDevice(ctx->cfg.device), "hipSetDevice");
        // the context's last call first (it may have run on another stream), then the named stream
        if (ctx->has_last) hip_check(hipEventSynchronize(ctx->done), "last call synchronize");
        drain(ctx, pick_stream(ctx, stream));
    });
}

int32_t xl_quantize_q8k_async(xl_context* ctx, const float* d_x, int32_t rows, int32_t k, void* d_q8k, void* stream,
                              xl_error* err) {
    return guarded(ctx, err, [&] {
        ready(ctx, false);
        need(d_x && d_q8k, XL_E_ARG, "null device pointer");
        need(rows >= 1 && k >= 256 && k % 256 == 0, XL_E_ARG, "rows >= 1 and k a positive multiple of 256");
        const uint64_t nblocks = uint64_t(rows) * uint64_t(k / 256);
        need(nblocks <= uint64_t(ctx->act_max / 256), XL_E_ARG, "more blocks than the activation workspace holds");
        hipStream_t s = pick_stream(ctx, stream);
        Ordered ord(ctx, s);
        hip_check(xl::dev::launch_q8k(d_x, int(nblocks), ctx->xq, ctx->xd, static_cast<uint8_t*>(d_q8k), ctx->err_flag, s),
                  "Q8_K launch");
    });
}

int32_t xl_swiglu_async(xl_context* ctx, const float* d_g, const float* d_u, int32_t n, float limit, float* d_h,
                        void* stream, xl_error* err) {
    return guarded(ctx, err, [&] {
        ready(ctx, false);
        need(d_g && d_u && d_h, XL_E_ARG, "null device pointer");
        need(n >= 1 && n <= (1 << 28), XL_E_ARG, "n outside 1..2^28");
        need(std::isfinite(limit), XL_E_ARG, "limit not finite");
        hipStream_t s = pick_stream(ctx, stream);
        Ordered ord(ctx, s);
        hip_check(xl::dev::launch_swiglu(d_g, d_u, n, limit, d_h, s), "SwiGLU launch");
    });
}

int32_t xl_matvec_async(xl_context* ctx, int32_t type, const void* d_planar, int32_t n, int32_t k, const float* d_x,
                        float* d_y, int32_t* d_partials, void* stream, xl_error* err) {
    return guarded(ctx, err, [&] {
        ready(ctx, false);
        need(xl::supported_type(type), XL_E_ARG, "unsupported block type");
        need(d_planar && d_x && d_y, XL_E_ARG, "null device pointer");
        int lpr, ppl;
        need(n >= 1 && xl::row_shape(k, lpr, ppl), XL_E_ARG, "unsupported matvec shape");
        need(k <= ctx->act_max, XL_E_ARG, "k exceeds the activation workspace");
        hipStream_t s = pick_stream(ctx, stream);
        Ordered ord(ctx, s);
        hip_check(xl::dev::launch_q8k(d_x, k / 256, ctx->xq, ctx->xd, nullptr, ctx->err_flag, s), "Q8_K launch");
        const auto P = xl::plane_layout(type, matrix_blocks(n, k));
        xl::MatRef m{};
        m.base = static_cast<const uint8_t*>(d_planar);
        m.off1 = P.off[1];
        m.off2 = P.off[2];
        m.type = type;
        m.nb = k / 256;
        hip_check(xl::dev::launch_matvec(m, n, k, ctx->xq, ctx->xd, ctx->codes, d_y, d_partials, ctx->err_flag, s),
                  "matvec launch");
    });
}

int32_t xl_profile_begin(xl_context* ctx, int32_t max_calls, xl_error* err) {
    return guarded(ctx, err, [&] {
        ready(ctx, false);
        need(!ctx->prof.on, XL_E_STATE, "profiling already active");
        need(max_calls >= 1 && max_calls <= 1 << 16, XL_E_ARG, "max_calls outside 1..65536");
        auto& P = ctx->prof;
        P = xl_context::Prof{};
        P.ev.resize(size_t(max_calls) * (kMaxStages + 1), nullptr);
        for (auto& e : P.ev) hip_check(hipEventCreate(&e), "hipEventCreate");
        P.max_calls = max_calls;
        P.on = true;
    });
}

int32_t xl_profile_end(xl_context* ctx, float* stage_ms, int32_t max_stages, int32_t* n_stages, int32_t* n_calls,
                       char* names, int32_t names_bytes, xl_error* err) {
    return guarded(ctx, err, [&] {
        need(ctx != nullptr && ctx->prof.on, XL_E_STATE, "profiling not active");
        auto& P = ctx->prof;
        struct Free {
            xl_context::Prof& p;
            ~Free() { for (auto& e : p.ev) if (e) (void)hipEventDestroy(e); p = xl_context::Prof{}; }
        } release{P};
        hip_check(hipSetDevice(ctx->cfg.device), "hipSetDevice");
        const int S = std::min(P.stages, std::max(0, int(max_stages)));
        for (int i = 0; i < S; ++i) stage_ms[i] = 0.0f;
        for (int c = 0; c < P.calls; ++c) {
            hip_check(hipEventSynchronize(P.ev[size_t(c) * (kMaxStages + 1) + S]), "event synchronize");
            for (int i = 0; i < S; ++i) {
                float ms = 0.0f;
                hip_check(hipEventElapsedTime(&ms, P.ev[size_t(c) * (kMaxStages + 1) + i],
                                              P.ev[size_t(c) * (kMaxStages + 1) + i + 1]), "event elapsed");
                stage_ms[i] += ms;
            }
        }
        if (n_stages) *n_stages = S;
        if (n_calls) *n_calls = P.calls;
        if (names && names_bytes > 0) {
            std::string all;
            for (int i = 0; i < S && i < int(P.names.size()); ++i) { if (i) all += ','; all += P.names[i]; }
            std::snprintf(names, size_t(names_bytes), "%s", all.c_str());
        }
    });
}

int32_t xl_debug_set_launch_count(xl_context* ctx, uint32_t launches, xl_error* err) {
    return guarded(ctx, err, [&] {
        ready(ctx, false);
        hipStream_t s = ctx->stream;
        Ordered ord(ctx, s);
        // ctl[0]: the all-types kernel's epoch, ctl[2]: the streaming kernel's launch
        // count (its parity); the arrival counters ctl[1], ctl[3] are zero between launches.
        const uint32_t w[4] = {launches, 0u, launches, 0u};
        hip_check(hipMemcpyAsync(ctx->ctl, w, sizeof w, hipMemcpyHostToDevice, s), "launch count upload");
        // The exchange state back to its state at xl_open, so that any count is
        // safe: the streaming kernel reads the h buffer of parity (count + 1) & 1
        // and expects it to hold the sentinel only (each launch refills the other
        // one), and the all-types kernel's tags of an epoch set back to one already
        // used would otherwise read as ready.
        const int P = ctx->cfg.max_picks, ff = ctx->cfg.ff;
        hip_check(hipMemsetAsync(ctx->hbuf, 0xff, size_t(2) * xl::kHBufWords * 4, s), "h exchange fill");
        hip_check(hipMemsetAsync(ctx->htag, 0, size_t(P) * ff * 8, s), "tag clear");
        hip_check(hipMemsetAsync(ctx->hdtag, 0, size_t(P) * (ff / 256) * 8, s), "tag clear");
        hip_check(hipMemsetAsync(ctx->hqtag, 0, size_t(P) * ff * 2, s), "tag clear");
        hip_check(hipStreamSynchronize(s), "launch count drain");
    });
}

int32_t xl_debug_launch_counts(xl_context* ctx, int64_t* counts, int32_t n, xl_error* err) {
    return guarded(ctx, err, [&] {
        need(counts != nullptr && n >= 0, XL_E_ARG, "null output");
        for (int i = 0; i < n; ++i) counts[i] = i < XL_LAUNCH_KINDS ? ctx->launches[i] : 0;
    });
}

int32_t xl_profile_timeline(xl_context* ctx, uint64_t* out, int32_t max_words, int32_t* n_words, xl_error* err) {
    return guarded(ctx, err, [&] {
        ready(ctx, false);
        need(out != nullptr && n_words != nullptr && max_words >= 0, XL_E_ARG, "null output");
        const uint64_t n = std::min<uint64_t>(ctx->timeline_words, uint64_t(max_words));
        hip_check(hipStreamSynchronize(ctx->stream), "stream synchronize");
        hip_check(hipDeviceSynchronize(), "device synchronize");
        if (n) hip_check(hipMemcpy(out, ctx->timeline, n * 8, hipMemcpyDeviceToHost), "timeline download");
        *n_words = int32_t(n);
    });
}

uint64_t xl_planar_bytes(int32_t type, int32_t n, int32_t k) {
    if (!xl::supported_type(type) || n <= 0 || k <= 0 || k % 256) return 0;
    return xl::plane_layout(type, matrix_blocks(n, k)).bytes;
}

int32_t xl_repack(int32_t type, int32_t n, int32_t k, const void* aos, void* planar) {
    if (!xl::supported_type(type) || n <= 0 || k <= 0 || k % 256 || !aos || !planar) return XL_E_ARG;
    const uint64_t nblk = matrix_blocks(n, k);
    const auto P = xl::plane_layout(type, nblk);
    std::memset(planar, 0, P.bytes);
    for (uint64_t b = 0; b < nblk; ++b)
        xl::block_to_planes(type, static_cast<const uint8_t*>(aos) + b * xl::block_bytes(type),
                            static_cast<uint8_t*>(planar), P, b);
    return XL_OK;
}

int32_t xl_restore(int32_t type, int32_t n, int32_t k, const void* planar, void* aos) {
    if (!xl::supported_type(type) || n <= 0 || k <= 0 || k % 256 || !aos || !planar) return XL_E_ARG;
    const uint64_t nblk = matrix_blocks(n, k);
    const auto P = xl::plane_layout(type, nblk);
    for (uint64_t b = 0; b < nblk; ++b)
        xl::planes_to_block(type, static_cast<const uint8_t*>(planar), P, b,
                            static_cast<uint8_t*>(aos) + b * xl::block_bytes(type));
    return XL_OK;
}

int32_t xl_generate_host(int32_t type, uint64_t seed, int32_t layer, int32_t expert, int32_t role, int32_t n, int32_t k,
                         void* aos) {
    if (!xl::supported_type(type) || n <= 0 || k <= 0 || k % 256 || !aos || layer < 0 || expert < 0 || role < 0 ||
        role > 2)
        return XL_E_ARG;
    const uint64_t key = xl::gen_key(seed, uint32_t(layer), uint32_t(expert), uint32_t(role));
    const uint64_t nblk = matrix_blocks(n, k);
    for (uint64_t b = 0; b < nblk; ++b) xl::gen_block(type, key, b, static_cast<uint8_t*>(aos) + b * xl::block_bytes(type));
    return XL_OK;
}

int32_t xl_codebook(int32_t which, uint64_t* out) {
    if (!out || which < 0 || which > 3) return XL_E_ARG;
    try {
        const auto t = device_tables();
        if (which == 0) std::copy(t.begin(), t.begin() + 256, out);
        else if (which == 1) std::copy(t.begin() + 256, t.begin() + 768, out);
        else if (which == 2) std::copy(t.begin() + 768, t.begin() + 2816, out);
        else for (int i = 0; i < 128; ++i) out[i] = ksigns(i);
        return XL_OK;
    } catch (...) {
        return XL_E_STATE;
    }
}

}  // extern "C"
