// ds3_hip.cpp -- host runtime of the MI355X MoE-FFN backend (C ABI in
// include/ds3_hip.h).  One device context, one stream, opaque buffers, a
// growable device workspace, and the entry points that validate arguments
// like the reference's Metal host (src/ds3_metal.m:373-449, 1841-1862,
// 2172-2828) and enqueue the gfx950 kernels.
#include "ds3_hip.h"
#include "kernels/launch.h"

#include <hip/hip_runtime.h>

#include <algorithm>
#include <chrono>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <string>
#include <unistd.h>
#include <vector>

struct ds3_hip_buffer {
    uint8_t *base;      // device allocation (shared by views)
    size_t bytes;       // bytes visible through this handle
    size_t offset;      // byte offset of this handle inside base
    bool owner;         // frees base on ds3_hip_buffer_free
    bool readonly;      // from_mmap buffers refuse writes
};

using namespace ds3k;

// Scratch of the allocation-free entry point ds3_hip_moe_ffn_batch_noalloc:
// every buffer a call of that entry point needs beyond its inputs and outputs
// (routing rows, bucketing lists, h, y) is carved from this array.  Each GPU
// the library runs on holds its own copy until the process ends.  Host code
// never passes `scratch` itself to a kernel (on the host the name is only a
// stand-in): ds3_hip_init looks up its device address once per device and the
// entry point passes that.
constexpr size_t kScratchBytes = (size_t)64 << 20;
static __device__ __align__(256) uint8_t scratch[kScratchBytes];

namespace {

constexpr int kDefaultPrefillMin = 17;     // grouped path from this many tokens (decode kernels up to 16)
constexpr int kDefaultDenseMfmaMin = 64;   // matmul_quantized_batch: fp16 MFMA path from this many rows of A
constexpr int kTickets = 32;             // router token-group tickets (zero between launches)
constexpr int kCertMaxTokens = 16;       // automatic mode: certified router up to this many tokens
#ifndef DS3_FUSE_SELECT_MAX_T
#define DS3_FUSE_SELECT_MAX_T 1          // decode: certified selection inside the gate/up kernel up to this T
#endif
constexpr int kFuseSelMaxTokens = DS3_FUSE_SELECT_MAX_T;
#ifndef DS3_FUSED_NB
#define DS3_FUSED_NB 4                   // repair batch rows of the fused selection at T <= 2
#endif
constexpr size_t kAllocPad = 256;        // slack after every allocation: kernels read whole dwords
constexpr int kMaxDevices = 64;

struct KRec {
    const char *name;
    int e0, e1;
};

struct State {
    bool inited = false;
    hipStream_t stream = nullptr;
    bool batch = false;
    bool capturing = false;          // between ds3_hip_graph_begin and ds3_hip_graph_end
    bool no_alloc = false;           // inside ds3_hip_moe_ffn_batch_noalloc: nothing may allocate
    uint8_t *ws = nullptr;
    size_t ws_bytes = 0;
    std::vector<void *> graphs;      // live executable graphs (graph_end .. graph_destroy)
    std::vector<uint8_t *> retired;  // workspace blocks outgrown while a live graph may address them
    std::vector<ds3_hip_buffer_t *> deferred_free;   // buffers freed during a capture
    int device = 0;                  // the device the context runs on
    uint8_t *scratch_dev[kMaxDevices] = {};   // device address of `scratch` per device, from ds3_hip_init
    int32_t *zero_idx = nullptr;     // device {0}
    int32_t *tickets = nullptr;      // kTickets router tickets (zero between launches)
    int router_mode = 0;             // ds3_hip_set_router_mode
    unsigned long long *cert_stats = nullptr;   // device {certified, repaired} token counts
    float *one_f = nullptr;          // device {1.0f}
    int prefill_min = kDefaultPrefillMin;
    int dense_mfma_min = kDefaultDenseMfmaMin;
    // reference-style profiling (src/ds3_metal.m:2868-2885)
    bool profile = false;
    int cb_count = 0;
    double gpu_ms = 0.0, cpu_ms = 0.0;
    hipEvent_t bev0 = nullptr, bev1 = nullptr;
    // per-kernel timing
    bool ktiming = false;
    std::string ktiming_only;          // empty: every kernel
    std::vector<hipEvent_t> pool;
    int pool_used = 0;
    std::vector<KRec> recs;
    std::vector<std::string> stat_names;
    std::vector<int64_t> stat_count;
    std::vector<double> stat_ms;
    bool stats_dirty = true;
    hipEvent_t t0 = nullptr, t1 = nullptr;
    // FP32 copies of non-F32 routers held in read-only buffers (see
    // router_f32_rows), kept until the owning buffer is freed.
    struct RouterF32 {
        const uint8_t *rows;     // the router rows as passed
        const uint8_t *alloc;    // the allocation holding them (its free drops the copy)
        int rtype;
        uint32_t E, K;
        uint64_t stride;
        float *f32;              // [E][K]
    };
    std::vector<RouterF32> router_f32;
    // The bucketing lists of the last chunk of the last grouped-path call
    // (device pointers into that call's workspace), for
    // ds3_hip_debug_grouped_lists; cleared when the workspace moves.
    struct {
        bool valid = false;
        ds3k::BucketOut bo{};
        int t0 = 0, tc = 0, k = 0, E = 0;
        bool marked = false;
    } lists;
};

State g;

void *dptr(const ds3_hip_buffer_t *b) { return b ? (void *)(b->base + b->offset) : nullptr; }
const uint8_t *cptr(const ds3_hip_buffer_t *b) { return b ? b->base + b->offset : nullptr; }
float *fptr(const ds3_hip_buffer_t *b) { return (float *)dptr(b); }

bool ensure_init()
{
    if (g.inited) return true;
    return ds3_hip_init() == 0;
}

int report(hipError_t e, const char *what)
{
    if (e == hipSuccess) return 0;
    fprintf(stderr, "ds3_hip: %s failed: %s\n", what, hipGetErrorString(e));
    return -1;
}

// Complete an entry point: surface launch errors, and outside a batch wait
// for the stream (calls are synchronous there, as in the reference).
int finish(hipError_t e, const char *what)
{
    if (report(e, what) != 0) return -1;
    if (!g.batch) return report(hipStreamSynchronize(g.stream), what);
    return 0;
}

// Refuse an entry point that would synchronise, copy from the host or
// allocate while a graph capture is open on the library stream: any of those
// would break the capture or record a node that replays stale host data.
bool refuse_in_capture(const char *what)
{
    if (!g.capturing) return false;
    fprintf(stderr, "ds3_hip: %s is not allowed during graph capture (ds3_hip_graph_begin .. ds3_hip_graph_end)\n",
            what);
    return true;
}

// Device workspace, grown on demand.  Growing waits for queued work that may
// still use the old block.  While an executable graph is alive the old block
// is retired instead of freed (the graph's kernels address it); retired blocks
// are freed once the last live graph is destroyed.
uint8_t *ws_get(size_t bytes)
{
    if (bytes <= g.ws_bytes) return g.ws;
    if (g.capturing) {
        fprintf(stderr, "ds3_hip: a captured call needs %zu workspace bytes (have %zu): make the same call once "
                        "before ds3_hip_graph_begin\n", bytes, g.ws_bytes);
        return nullptr;
    }
    g.lists.valid = false;
    if (g.ws) {
        (void)hipStreamSynchronize(g.stream);
        if (g.graphs.empty()) (void)hipFree(g.ws);
        else g.retired.push_back(g.ws);
        g.ws = nullptr;
        g.ws_bytes = 0;
    }
    const size_t want = bytes + bytes / 4 + (1u << 20);
    if (hipMalloc((void **)&g.ws, want) != hipSuccess) {
        fprintf(stderr, "ds3_hip: workspace allocation of %zu bytes failed\n", want);
        g.ws = nullptr;
        return nullptr;
    }
    g.ws_bytes = want;
    return g.ws;
}

// Buffers whose ds3_hip_buffer_free came during the capture that just ended.
void free_deferred()
{
    std::vector<ds3_hip_buffer_t *> v;
    v.swap(g.deferred_free);
    for (ds3_hip_buffer_t *b : v) ds3_hip_buffer_free(b);
}

// Workspace blocks retired while graphs were alive, once none is left.
void free_retired()
{
    if (!g.graphs.empty() || g.retired.empty()) return;
    (void)hipStreamSynchronize(g.stream);
    for (uint8_t *p : g.retired) (void)hipFree(p);
    g.retired.clear();
}

bool graph_live(void *graph) { return std::find(g.graphs.begin(), g.graphs.end(), graph) != g.graphs.end(); }



struct Bump {
    size_t off = 0;
    size_t take(size_t bytes)
    {
        const size_t o = off;
        off = (off + bytes + 255) & ~(size_t)255;
        return o;
    }
};

// RAII event pair around one launcher call while kernel timing is on
// (timing-only events: no system-scope fence when recorded).
struct KScope {
    int e0 = -1;
    const char *name;
    explicit KScope(const char *n) : name(n)
    {
        if (g.ktiming && g.pool_used + 2 <= (int)g.pool.size() && (g.ktiming_only.empty() || g.ktiming_only == n)) {
            e0 = g.pool_used;
            g.pool_used += 2;
            (void)hipEventRecord(g.pool[e0], g.stream);
        }
    }
    ~KScope()
    {
        if (e0 >= 0) {
            (void)hipEventRecord(g.pool[e0 + 1], g.stream);
            g.recs.push_back({ name, e0, e0 + 1 });
            g.stats_dirty = true;
        }
    }
};

// The FP32 rows of a non-F32 router held in a read-only buffer (the engine's
// mmap'd weights, ds3_hip_buffer_from_mmap), expanded once and kept until that
// buffer is freed: its bytes cannot change (buffer_write refuses it), so every
// later call skips the per-call expansion.  nullptr: the caller expands per
// call (an F32 router, a writable buffer, or no copy yet during a capture or
// an allocation-free call).
const float *router_f32_rows(const ds3_hip_buffer_t *router, int rtype, uint32_t E, uint32_t K, uint64_t stride)
{
    if (rtype == T_F32 || !router->readonly) return nullptr;
    const uint8_t *rows = cptr(router);
    for (const State::RouterF32 &r : g.router_f32)
        if (r.rows == rows && r.rtype == rtype && r.E == E && r.K == K && r.stride == stride) return r.f32;
    if (g.capturing || g.no_alloc || !router_seq_type_ok(rtype, (int)K)) return nullptr;
    float *f = nullptr;
    if (hipMalloc((void **)&f, (size_t)E * K * 4 + kAllocPad) != hipSuccess) return nullptr;
    hipError_t e;
    {
        KScope ks("router_rows");
        e = launch_router_rows(rtype, rows, stride, (int)E, (int)K, f, g.stream);
    }
    if (e != hipSuccess) {
        (void)hipStreamSynchronize(g.stream);
        (void)hipFree(f);
        return nullptr;
    }
    g.router_f32.push_back({ rows, router->base, rtype, E, K, stride, f });
    return f;
}

// Drop the router copies made from the allocation at base, which is being
// freed; while a live graph may read a copy it is retired, not freed.
void drop_router_f32(const uint8_t *base)
{
    auto &v = g.router_f32;
    for (size_t i = 0; i < v.size();) {
        if (v[i].alloc != base) {
            i++;
            continue;
        }
        if (g.graphs.empty()) (void)hipFree(v[i].f32);
        else g.retired.push_back((uint8_t *)v[i].f32);
        v.erase(v.begin() + (std::ptrdiff_t)i);
    }
}

bool is_quant(int t) { return t == T_Q4_K || t == T_Q6_K || t == T_Q8_0; }

// Bytes of one row of n values of a weight type (0 for an unknown type).
size_t row_bytes(int type, uint32_t n)
{
    switch (type) {
    case T_F32: return (size_t)n * 4;
    case T_F16: return (size_t)n * 2;
    case T_Q8_0: return (size_t)n / 32 * 34;
    case T_Q4_K: return (size_t)n / 256 * 144;
    case T_Q6_K: return (size_t)n / 256 * 210;
    default: return 0;
    }
}

// reference src/ds3_metal.m:1841-1862
bool quant_type_ok_for_moe(int type, uint32_t in_dim, const char *name)
{
    if (type == T_F32) {
        if (in_dim % 32 != 0) {
            fprintf(stderr, "ds3_hip: %s F32 requires in_dim=%u multiple of 32\n", name, in_dim);
            return false;
        }
        return true;
    }
    if (type == T_Q4_K || type == T_Q6_K) {
        if (in_dim % 256 != 0) {
            fprintf(stderr, "ds3_hip: %s type=%d requires in_dim=%u multiple of 256\n", name, type, in_dim);
            return false;
        }
        return true;
    }
    if (type == T_Q8_0) {
        if (in_dim % 32 != 0) {
            fprintf(stderr, "ds3_hip: %s type=%d requires in_dim=%u multiple of 32\n", name, type, in_dim);
            return false;
        }
        return true;
    }
    fprintf(stderr, "ds3_hip: unsupported %s type %d\n", name, type);
    return false;
}

bool fits(const ds3_hip_buffer_t *b, size_t need, const char *what)
{
    if (!b) return true;
    if (b->bytes < need) {
        fprintf(stderr, "ds3_hip: buffer %s holds %zu bytes, needs %zu\n", what, b->bytes, need);
        return false;
    }
    return true;
}

// Bytes a [rows] x row_bytes matrix with rows `stride` bytes apart spans.
uint64_t span_bytes(uint64_t rows, uint64_t stride, uint64_t row_b)
{
    return rows == 0 ? 0 : (rows - 1) * stride + row_b;
}

// The router and the routed experts' tensors hold what a MoE call reads on
// the device: row strides of at least one row's bytes, n_expert router rows,
// n_expert experts per tensor (expert e at e * rows * stride when no offset
// table is given) and, with a table, its n_expert x 3 u64 entries.  The
// table's offsets themselves live in device memory and are the caller's, as
// the engine builds them (src/ds3_engine.c:1747-1773).
bool moe_weights_fit(const ds3_hip_buffer_t *router, uint64_t rstride, int rtype, const ds3_hip_buffer_t *wg,
                     const ds3_hip_buffer_t *wu, const ds3_hip_buffer_t *wd, int gt, int ut, int dt, uint64_t gs,
                     uint64_t us, uint64_t ds, const ds3_hip_buffer_t *table, uint32_t n_embd, uint32_t n_expert,
                     uint32_t n_ff)
{
    const uint64_t rb_r = row_bytes(rtype, n_embd), rb_g = row_bytes(gt, n_embd), rb_u = row_bytes(ut, n_embd),
                   rb_d = row_bytes(dt, n_ff);
    struct { const char *name; uint64_t stride, need; } st[4] = {
        { "router_row_stride", rstride, rb_r }, { "gate_row_stride", gs, rb_g },
        { "up_row_stride", us, rb_u }, { "down_row_stride", ds, rb_d } };
    for (const auto &s : st)
        if (s.need == 0 || s.stride < s.need) {
            fprintf(stderr, "ds3_hip: %s=%llu is shorter than one row (%llu bytes)\n", s.name,
                    (unsigned long long)s.stride, (unsigned long long)s.need);
            return false;
        }
    if (!fits(router, span_bytes(n_expert, rstride, rb_r), "router (n_expert rows)")) return false;
    if (table) return fits(table, (size_t)n_expert * 3 * sizeof(uint64_t), "expert_offsets (n_expert x 3 u64)");
    return fits(wg, span_bytes((uint64_t)n_expert * n_ff, gs, rb_g), "gate experts (n_expert x n_ff rows)") &&
           fits(wu, span_bytes((uint64_t)n_expert * n_ff, us, rb_u), "up experts (n_expert x n_ff rows)") &&
           fits(wd, span_bytes((uint64_t)n_expert * n_embd, ds, rb_d), "down experts (n_expert x n_embd rows)");
}

// A certified selection left to the decode gate/up kernel's prologue
// (launch_decode_gate_up_sel): set by route_tokens when the caller allows it.
struct DeferredSel {
    bool on = false;
    CertSel cs{};
    RouteArgs ra{};
};

// Per-token expert products for `slots` routed slots of T tokens:
// h = swiglu(gate, up) then out (+)= sum_k w_k * down(h_k).
// With xt (tokens routed by the certified router's selection launch), the
// gate/up launch also recomputes their weights from exact logits.
int run_experts_decode(const float *x, int64_t ldx, const int32_t *idx, const float *wts, int T, int n_used,
                       const ExpertWeights &ew, uint32_t n_embd, uint32_t n_ff, float *out, const float *residual,
                       bool accumulate, float *h, float *tmp_up, const DeferredSel *sel = nullptr,
                       const ExactTail *xt = nullptr)
{
    const int slots = T * n_used;
    hipError_t e;
    if (sel != nullptr && sel->on) {
        // route_tokens defers only where this kernel applies (same gate/up
        // types, rows n_embd floats apart)
        KScope ks("moe_decode_gate_up_sel");
        e = launch_decode_gate_up_sel(x, T, n_used, ew, (int)n_embd, (int)n_ff, h, sel->cs, sel->ra, g.stream);
    } else if (ew.gate_type == ew.up_type) {
        KScope ks("moe_decode_gate_up");
        e = launch_decode_gate_up(x, ldx, idx, slots, n_used, ew, (int)n_embd, (int)n_ff, h, g.stream, xt);
    } else {
        // Mismatched gate/up types: two projections, then silu_mul
        // (the reference's unfused fallback, src/ds3_metal.m:2107-2140).
        ExpertWeights eg = ew, eu = ew;
        eg.up = ew.gate; eg.up_type = ew.gate_type; eg.up_stride = ew.gate_stride;
        eu.gate = ew.up; eu.gate_type = ew.up_type; eu.gate_stride = ew.up_stride;
        KScope ks("moe_decode_proj");
        e = launch_decode_proj(x, ldx, idx, slots, n_used, eg, 0, (int)n_embd, (int)n_ff, h, g.stream, xt);
        if (e == hipSuccess)
            e = launch_decode_proj(x, ldx, idx, slots, n_used, eu, 1, (int)n_embd, (int)n_ff, tmp_up, g.stream);
        if (e == hipSuccess) e = launch_silu_mul(h, tmp_up, h, (int64_t)slots * n_ff, g.stream);
    }
    if (e != hipSuccess) return report(e, "decode gate/up");
    KScope ks("moe_decode_down");
    e = launch_decode_down(h, idx, wts, T, n_used, ew, (int)n_embd, (int)n_ff, out, n_embd, residual, accumulate,
                           g.stream);
    return report(e, "decode down");
}

}  // namespace

// ===========================================================================
// Lifecycle
// ===========================================================================

extern "C" int ds3_hip_init(void)
{
    if (g.inited) return 0;
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || n <= 0) {
        fprintf(stderr, "ds3_hip: no HIP device available\n");
        return -1;
    }
    if (hipSetDevice(0) != hipSuccess) return -1;
    g.device = 0;
    if (hipStreamCreateWithFlags(&g.stream, hipStreamNonBlocking) != hipSuccess) {
        fprintf(stderr, "ds3_hip: stream creation failed\n");
        return -1;
    }
    if (g.scratch_dev[g.device] == nullptr) {
        // with the device current: this device's copy of the scratch array
        void *sp = nullptr;
        const hipError_t es = hipGetSymbolAddress(&sp, HIP_SYMBOL(scratch));
        if (es != hipSuccess || sp == nullptr) {
            fprintf(stderr, "ds3_hip: scratch array lookup failed: %s\n", hipGetErrorString(es));
            return -1;
        }
        g.scratch_dev[g.device] = (uint8_t *)sp;
    }
    void *consts = nullptr;
    if (hipMalloc(&consts, 128 + (size_t)kTickets * 4 + 16) != hipSuccess) return -1;
    g.zero_idx = (int32_t *)consts;
    g.one_f = (float *)((uint8_t *)consts + 64);
    g.tickets = (int32_t *)((uint8_t *)consts + 128);   // router token-group tickets, kept at zero between launches
    g.cert_stats = (unsigned long long *)((uint8_t *)consts + 128 + (size_t)kTickets * 4);
    if (hipMemsetAsync(g.tickets, 0, (size_t)kTickets * 4 + 16, g.stream) != hipSuccess ||
        hipStreamSynchronize(g.stream) != hipSuccess)
        return -1;
    const int32_t zi = 0;
    const float one = 1.0f;
    (void)hipMemcpy(g.zero_idx, &zi, sizeof zi, hipMemcpyHostToDevice);
    (void)hipMemcpy(g.one_f, &one, sizeof one, hipMemcpyHostToDevice);
    (void)hipEventCreate(&g.bev0);
    (void)hipEventCreate(&g.bev1);
    (void)hipEventCreate(&g.t0);
    (void)hipEventCreate(&g.t1);
    const char *p = getenv("DS3_HIP_PROFILE");
    g.profile = p && *p && *p != '0';
    g.inited = true;
    return 0;
}

extern "C" void ds3_hip_shutdown(void)
{
    if (!g.inited) return;
    if (g.capturing) {                       // abandon an open capture
        hipGraph_t gr = nullptr;
        if (hipStreamEndCapture(g.stream, &gr) == hipSuccess && gr) (void)hipGraphDestroy(gr);
        g.capturing = false;
        g.batch = false;
        free_deferred();
    }
    (void)hipStreamSynchronize(g.stream);
    // graphs address the workspace freed below: they end with the context
    for (void *gr : g.graphs) (void)hipGraphExecDestroy((hipGraphExec_t)gr);
    g.graphs.clear();
    for (uint8_t *p : g.retired) (void)hipFree(p);
    g.retired.clear();
    for (hipEvent_t e : g.pool) (void)hipEventDestroy(e);
    g.pool.clear();
    g.recs.clear();
    (void)hipEventDestroy(g.bev0);
    (void)hipEventDestroy(g.bev1);
    (void)hipEventDestroy(g.t0);
    (void)hipEventDestroy(g.t1);
    if (g.ws) (void)hipFree(g.ws);
    for (const State::RouterF32 &r : g.router_f32) (void)hipFree(r.f32);
    (void)hipFree(g.zero_idx);
    (void)hipStreamDestroy(g.stream);
    uint8_t *sd[kMaxDevices];
    std::copy(g.scratch_dev, g.scratch_dev + kMaxDevices, sd);
    g = State();
    std::copy(sd, sd + kMaxDevices, g.scratch_dev);      // the arrays outlive the context
}

// ===========================================================================
// Buffers (reference src/ds3_metal.m:373-449)
// ===========================================================================

extern "C" ds3_hip_buffer_t *ds3_hip_buffer_alloc(size_t bytes)
{
    if (bytes == 0 || refuse_in_capture("buffer_alloc") || !ensure_init()) return nullptr;
    void *p = nullptr;
    const size_t padded = ((bytes + 255) & ~(size_t)255) + kAllocPad;
    if (hipMalloc(&p, padded) != hipSuccess) return nullptr;
    // Zero on the library stream and wait: the stream is non-blocking, so a
    // null-stream memset could still be running when a later kernel on the
    // library stream writes the buffer, and then overwrite its output.
    if (hipMemsetAsync(p, 0, padded, g.stream) != hipSuccess || hipStreamSynchronize(g.stream) != hipSuccess) {
        (void)hipFree(p);
        return nullptr;
    }
    auto *b = (ds3_hip_buffer_t *)calloc(1, sizeof(ds3_hip_buffer_t));
    if (!b) {
        (void)hipFree(p);
        return nullptr;
    }
    *b = { (uint8_t *)p, bytes, 0, true, false };
    return b;
}

extern "C" ds3_hip_buffer_t *ds3_hip_buffer_from_mmap(const void *base, size_t bytes)
{
    if (!base || bytes == 0 || refuse_in_capture("buffer_from_mmap")) return nullptr;
    long ps = sysconf(_SC_PAGESIZE);
    if (ps <= 0) ps = 4096;
    if (((uintptr_t)base) & ((uintptr_t)ps - 1)) {
        fprintf(stderr, "ds3_hip: mmap base %p is not page-aligned\n", base);
        return nullptr;
    }
    ds3_hip_buffer_t *b = ds3_hip_buffer_alloc(bytes);
    if (!b) return nullptr;
    if (hipMemcpy(b->base, base, bytes, hipMemcpyHostToDevice) != hipSuccess) {
        ds3_hip_buffer_free(b);
        return nullptr;
    }
    b->readonly = true;
    return b;
}

extern "C" ds3_hip_buffer_t *ds3_hip_buffer_view(const ds3_hip_buffer_t *base, size_t offset, size_t bytes)
{
    if (!base || !base->base || offset > base->bytes || bytes == 0 || offset + bytes > base->bytes) return nullptr;
    auto *v = (ds3_hip_buffer_t *)calloc(1, sizeof(ds3_hip_buffer_t));
    if (!v) return nullptr;
    *v = { base->base, bytes, base->offset + offset, false, base->readonly };
    return v;
}

extern "C" void ds3_hip_buffer_free(ds3_hip_buffer_t *buf)
{
    if (!buf) return;
    if (g.capturing) {
        // freeing waits for the stream, which a capture forbids: free it when the capture ends
        g.deferred_free.push_back(buf);
        return;
    }
    if (buf->owner && buf->base) {
        if (g.inited) (void)hipStreamSynchronize(g.stream);
        drop_router_f32(buf->base);
        (void)hipFree(buf->base);
    }
    free(buf);
}

extern "C" int ds3_hip_buffer_write(ds3_hip_buffer_t *buf, size_t offset, const void *src, size_t bytes)
{
    if (!buf || !src || offset + bytes > buf->bytes || refuse_in_capture("buffer_write")) return -1;
    if (buf->readonly) {
        fprintf(stderr, "ds3_hip: buffer_write into a buffer imported with buffer_from_mmap is refused\n");
        return -1;
    }
    if (bytes == 0) return 0;
    hipError_t e = hipMemcpyAsync(buf->base + buf->offset + offset, src, bytes, hipMemcpyHostToDevice, g.stream);
    if (e == hipSuccess) e = hipStreamSynchronize(g.stream);
    return report(e, "buffer_write");
}

extern "C" int ds3_hip_buffer_read(ds3_hip_buffer_t *buf, size_t offset, void *dst, size_t bytes)
{
    if (!buf || !dst || offset + bytes > buf->bytes || refuse_in_capture("buffer_read")) return -1;
    if (bytes == 0) return 0;
    hipError_t e = hipMemcpyAsync(dst, buf->base + buf->offset + offset, bytes, hipMemcpyDeviceToHost, g.stream);
    if (e == hipSuccess) e = hipStreamSynchronize(g.stream);
    return report(e, "buffer_read");
}

// ===========================================================================
// Products
// ===========================================================================

static int vec_matmul_typed(const ds3_hip_buffer_t *x, const ds3_hip_buffer_t *W, ds3_hip_buffer_t *y,
                            uint32_t in_dim, uint32_t out_dim, uint64_t row_stride, int type, const char *what)
{
    if (!x || !W || !y || !ensure_init()) return -1;
    if (!gemv_type_ok(type, (int)in_dim)) {
        fprintf(stderr, "ds3_hip: %s type=%d in_dim=%u unsupported\n", what, type, in_dim);
        return -1;
    }
    if (!fits(x, (size_t)in_dim * 4, "x") || !fits(y, (size_t)out_dim * 4, "y") ||
        !fits(W, (size_t)(out_dim - 1) * row_stride + (size_t)row_stride, "W"))
        return -1;
    KScope ks(gemv1_path(type, cptr(W), row_stride, 1, (int)in_dim) ? "gemv1" : "gemv");
    return finish(launch_gemv(type, (const float *)dptr(x), in_dim, cptr(W), row_stride, fptr(y), out_dim, 1,
                              (int)out_dim, (int)in_dim, nullptr, g.stream),
                  what);
}

extern "C" int ds3_hip_vec_matmul_f32(const ds3_hip_buffer_t *x, const ds3_hip_buffer_t *W, ds3_hip_buffer_t *y,
                                      uint32_t in_dim, uint32_t out_dim, uint64_t row_stride)
{
    if (row_stride < (uint64_t)in_dim * 4) {
        fprintf(stderr, "ds3_hip: vec_matmul_f32 row_stride=%llu < in_dim*4\n", (unsigned long long)row_stride);
        return -1;
    }
    return vec_matmul_typed(x, W, y, in_dim, out_dim, row_stride, T_F32, "vec_matmul_f32");
}

extern "C" int ds3_hip_vec_matmul_quantized(const ds3_hip_buffer_t *x, const ds3_hip_buffer_t *W, ds3_hip_buffer_t *y,
                                            uint32_t in_dim, uint32_t out_dim, uint64_t row_stride,
                                            ds3_hip_type_t type)
{
    if (!x || !W || !y) return -1;
    if (type == T_Q4_K || type == T_Q6_K) {
        if (in_dim % 256 != 0) {
            fprintf(stderr, "ds3_hip: type %d in_dim=%u must be a multiple of 256\n", type, in_dim);
            return -1;
        }
    } else if (type == T_Q8_0) {
        if (in_dim % 32 != 0) {
            fprintf(stderr, "ds3_hip: Q8_0 in_dim=%u must be a multiple of 32\n", in_dim);
            return -1;
        }
    } else {
        fprintf(stderr, "ds3_hip: unsupported quantized matmul type %d\n", type);
        return -1;
    }
    return vec_matmul_typed(x, W, y, in_dim, out_dim, row_stride, type, "vec_matmul_quantized");
}

// reference src/ds3_metal.h:142-146 (metal matmul_vec_q4k_half): x holds
// fp16 values; they are widened exactly to fp32 and the Q4_K product runs as
// for an fp32 x.
extern "C" int ds3_hip_vec_matmul_q4k_half(const ds3_hip_buffer_t *x, const ds3_hip_buffer_t *W, ds3_hip_buffer_t *y,
                                           uint32_t in_dim, uint32_t out_dim, uint64_t row_stride)
{
    if (!x || !W || !y || in_dim == 0 || !ensure_init()) return -1;
    if (in_dim % 256 != 0) {
        fprintf(stderr, "ds3_hip: vec_matmul_q4k_half in_dim=%u must be a multiple of 256\n", in_dim);
        return -1;
    }
    if (!fits(x, (size_t)in_dim * 2, "x (fp16)")) return -1;
    if (row_stride < row_bytes(T_Q4_K, in_dim)) {
        fprintf(stderr, "ds3_hip: vec_matmul_q4k_half row_stride=%llu < one row\n", (unsigned long long)row_stride);
        return -1;
    }
    if (!fits(y, (size_t)out_dim * 4, "y") || !fits(W, span_bytes(out_dim, row_stride, row_bytes(T_Q4_K, in_dim)), "W"))
        return -1;
    uint8_t *ws = ws_get((size_t)in_dim * 4);
    if (!ws) return -1;
    hipError_t e;
    {
        KScope ks("to_f32");
        e = launch_to_f32((const _Float16 *)dptr(x), (float *)ws, in_dim, g.stream);
    }
    if (e == hipSuccess) {
        KScope ks(gemv1_path(T_Q4_K, cptr(W), row_stride, 1, (int)in_dim) ? "gemv1" : "gemv");
        e = launch_gemv(T_Q4_K, (const float *)ws, in_dim, cptr(W), row_stride, fptr(y), out_dim, 1, (int)out_dim,
                        (int)in_dim, nullptr, g.stream);
    }
    return finish(e, "vec_matmul_q4k_half");
}

extern "C" int ds3_hip_vec_matmul_f32_simd(const ds3_hip_buffer_t *x, const ds3_hip_buffer_t *W, ds3_hip_buffer_t *y,
                                           uint32_t in_dim, uint32_t out_dim, uint64_t row_stride)
{
    return ds3_hip_vec_matmul_f32(x, W, y, in_dim, out_dim, row_stride);
}

extern "C" int ds3_hip_vec_matmul_q8_0_simd(const ds3_hip_buffer_t *x, const ds3_hip_buffer_t *W, ds3_hip_buffer_t *y,
                                            uint32_t in_dim, uint32_t out_dim, uint64_t row_stride)
{
    return ds3_hip_vec_matmul_quantized(x, W, y, in_dim, out_dim, row_stride, T_Q8_0);
}

extern "C" int ds3_hip_vec_matmul_q4k_simd(const ds3_hip_buffer_t *x, const ds3_hip_buffer_t *W, ds3_hip_buffer_t *y,
                                           uint32_t in_dim, uint32_t out_dim, uint64_t row_stride)
{
    return ds3_hip_vec_matmul_quantized(x, W, y, in_dim, out_dim, row_stride, T_Q4_K);
}

extern "C" int ds3_hip_vec_matmul_q6k_simd(const ds3_hip_buffer_t *x, const ds3_hip_buffer_t *W, ds3_hip_buffer_t *y,
                                           uint32_t in_dim, uint32_t out_dim, uint64_t row_stride)
{
    return ds3_hip_vec_matmul_quantized(x, W, y, in_dim, out_dim, row_stride, T_Q6_K);
}

// reference src/ds3_metal.m:2741-2828
extern "C" int ds3_hip_matmul_quantized_batch(const ds3_hip_buffer_t *A, const ds3_hip_buffer_t *W,
                                              ds3_hip_buffer_t *C, uint32_t M, uint32_t N, uint32_t K,
                                              uint64_t weight_row_stride, uint64_t weight_offset,
                                              ds3_hip_type_t type)
{
    if (!A || !W || !C || !ensure_init()) return -1;
    if (type == T_Q4_K || type == T_Q6_K) {
        if (K % 256 != 0) {
            fprintf(stderr, "ds3_hip: type %d batch K=%u must be a multiple of 256\n", type, K);
            return -1;
        }
    } else if (type == T_Q8_0) {
        if (K % 32 != 0) {
            fprintf(stderr, "ds3_hip: Q8_0 batch K=%u must be a multiple of 32\n", K);
            return -1;
        }
    } else {
        fprintf(stderr, "ds3_hip: unsupported quantized batch matmul type %d\n", type);
        return -1;
    }
    if (M == 0 || N == 0) return 0;
    if (!fits(A, (size_t)M * K * 4, "A") || !fits(C, (size_t)M * N * 4, "C") ||
        !fits(W, weight_offset + (size_t)N * weight_row_stride, "W"))
        return -1;
    if (weight_row_stride < row_bytes(type, K)) {
        fprintf(stderr, "ds3_hip: matmul_quantized_batch weight_row_stride=%llu < one row\n",
                (unsigned long long)weight_row_stride);
        return -1;
    }
    if ((int64_t)M >= g.dense_mfma_min && dense_mfma_shape_ok(type, (int)N, (int)K) && M <= 65535) {
        // fp16 MFMA path: A in fp16, the weights decoded to fp16, fp32
        // accumulate, on the grouped gate_up kernel as one expert that holds
        // every row of A (the bucketing lists of M zero expert indices)
        const int rpi_gu = dense_runs_per_tile((int)N);         // gate_up's run list only: no down
        const int max_tiles = (int)((M + 63) / 64) + 1;
        Bump bp;
        const size_t o_x16 = bp.take((size_t)M * K * 2), o_cnt = bp.take(16), o_off = bp.take(16),
                     o_ids = bp.take((size_t)M * 4), o_wts = bp.take((size_t)M * 4), o_pos = bp.take((size_t)M * 4),
                     o_tiles = bp.take((size_t)max_tiles * 4), o_nt = bp.take(16),
                     o_rg = bp.take((size_t)max_tiles * rpi_gu * 4), o_dg = bp.take((size_t)max_tiles * rpi_gu * 8);
        uint8_t *ws = ws_get(bp.off);
        if (!ws) return -1;
        BucketOut bo{ (int32_t *)(ws + o_cnt), (int32_t *)(ws + o_off), (int32_t *)(ws + o_ids), (float *)(ws + o_wts),
                      (int32_t *)(ws + o_pos), (int32_t *)(ws + o_tiles), (int32_t *)(ws + o_nt), max_tiles, 64,
                      (int32_t *)(ws + o_rg), nullptr, (int32_t *)(ws + o_nt) + 1, rpi_gu, 0, (int2 *)(ws + o_dg),
                      nullptr };
        hipError_t e = launch_to_f16(fptr(A), (_Float16 *)(ws + o_x16), (int64_t)M * K, g.stream);
        if (e == hipSuccess) {
            KScope ks("dense_lists");
            e = launch_dense_lists((int)M, bo, g.stream);           // one expert holding every row, in order
        }
        if (e == hipSuccess) {
            KScope ks("dense_mfma");
            e = launch_dense_mfma((const _Float16 *)(ws + o_x16), (int)K, cptr(W) + weight_offset, weight_row_stride,
                                  type, (int)N, bo, fptr(C), g.stream);
        }
        return finish(e, "matmul_quantized_batch");
    }
    KScope ks(gemv1_path(type, cptr(W) + weight_offset, weight_row_stride, (int)M, (int)K) ? "gemv1" : "gemv");
    return finish(launch_gemv(type, fptr(A), K, cptr(W) + weight_offset, weight_row_stride, fptr(C), N, (int)M,
                              (int)N, (int)K, nullptr, g.stream),
                  "matmul_quantized_batch");
}

// ===========================================================================
// Elementwise (reference src/ds3_metal.m:994-1103)
// ===========================================================================

extern "C" int ds3_hip_buffer_copy_f32(const ds3_hip_buffer_t *src, ds3_hip_buffer_t *dst, size_t bytes)
{
    if (!src || !dst || bytes == 0 || !ensure_init()) return -1;
    if (bytes % sizeof(float) != 0) {
        fprintf(stderr, "ds3_hip: buffer_copy_f32 bytes=%zu must be a multiple of %zu\n", bytes, sizeof(float));
        return -1;
    }
    if (!fits(src, bytes, "src") || !fits(dst, bytes, "dst")) return -1;
    KScope ks("copy");
    return finish(launch_copy(fptr(src), fptr(dst), (int64_t)(bytes / 4), g.stream), "buffer_copy_f32");
}

extern "C" int ds3_hip_buffer_zero_f32(ds3_hip_buffer_t *buf, size_t bytes)
{
    if (!buf || bytes == 0 || !ensure_init()) return -1;
    if (bytes % sizeof(float) != 0) {
        fprintf(stderr, "ds3_hip: buffer_zero_f32 bytes=%zu must be a multiple of %zu\n", bytes, sizeof(float));
        return -1;
    }
    if (!fits(buf, bytes, "buf")) return -1;
    KScope ks("zero");
    return finish(launch_fill_zero(fptr(buf), (int64_t)(bytes / 4), g.stream), "buffer_zero_f32");
}

extern "C" int ds3_hip_vec_add_inplace(ds3_hip_buffer_t *acc, const ds3_hip_buffer_t *addend, uint32_t n)
{
    if (!acc || !addend || !ensure_init()) return -1;
    if (n == 0) return 0;
    if (!fits(acc, (size_t)n * 4, "acc") || !fits(addend, (size_t)n * 4, "addend")) return -1;
    KScope ks("add");
    return finish(launch_add(fptr(acc), fptr(addend), fptr(acc), n, g.stream), "vec_add_inplace");
}

extern "C" int ds3_hip_vec_add(const ds3_hip_buffer_t *a, const ds3_hip_buffer_t *b, ds3_hip_buffer_t *c, uint32_t n)
{
    if (!a || !b || !c || !ensure_init()) return -1;
    if (n == 0) return 0;
    if (!fits(a, (size_t)n * 4, "a") || !fits(b, (size_t)n * 4, "b") || !fits(c, (size_t)n * 4, "c")) return -1;
    KScope ks("add");
    return finish(launch_add(fptr(a), fptr(b), fptr(c), n, g.stream), "vec_add");
}

extern "C" int ds3_hip_gather_rows_f32(const ds3_hip_buffer_t *src, const ds3_hip_buffer_t *ids, ds3_hip_buffer_t *dst,
                                       uint32_t n_cols, uint32_t count, uint32_t offset)
{
    if (!src || !ids || !dst || n_cols == 0 || count == 0 || !ensure_init()) return -1;
    if (!fits(ids, ((size_t)offset + count) * 4, "ids") || !fits(dst, (size_t)count * n_cols * 4, "dst")) return -1;
    KScope ks("gather_rows");
    return finish(launch_gather_rows(fptr(src), (const int32_t *)dptr(ids) + offset, fptr(dst), (int)n_cols,
                                     (int)count, (int64_t)(src->bytes / ((size_t)n_cols * 4)), g.stream),
                  "gather_rows_f32");
}

extern "C" int ds3_hip_scatter_add_weighted_f32(const ds3_hip_buffer_t *src, const ds3_hip_buffer_t *scores,
                                                const ds3_hip_buffer_t *ids, ds3_hip_buffer_t *dst, uint32_t n_cols,
                                                uint32_t count, uint32_t offset)
{
    if (!src || !scores || !ids || !dst || n_cols == 0 || count == 0 || !ensure_init()) return -1;
    if (!fits(ids, ((size_t)offset + count) * 4, "ids") || !fits(scores, ((size_t)offset + count) * 4, "scores") ||
        !fits(src, (size_t)count * n_cols * 4, "src"))
        return -1;
    KScope ks("scatter_add");
    return finish(launch_scatter_add(fptr(src), fptr(scores) + offset, (const int32_t *)dptr(ids) + offset,
                                     fptr(dst), (int)n_cols, (int)count, (int64_t)(dst->bytes / ((size_t)n_cols * 4)),
                                     g.stream),
                  "scatter_add_weighted_f32");
}

extern "C" int ds3_hip_silu_mul_f32(const ds3_hip_buffer_t *gate, const ds3_hip_buffer_t *up, ds3_hip_buffer_t *out,
                                    uint32_t n)
{
    if (!gate || !up || !out || !ensure_init()) return -1;
    if (n == 0) return 0;
    if (!fits(gate, (size_t)n * 4, "gate") || !fits(up, (size_t)n * 4, "up") || !fits(out, (size_t)n * 4, "out"))
        return -1;
    KScope ks("silu_mul");
    return finish(launch_silu_mul(fptr(gate), fptr(up), fptr(out), n, g.stream), "silu_mul_f32");
}

// reference src/ds3_metal.h:48-57 (metal/rms_norm.metal; CPU src/ds3_reference.c:329-342)
extern "C" int ds3_hip_rms_norm(const ds3_hip_buffer_t *x, const ds3_hip_buffer_t *weight, ds3_hip_buffer_t *out,
                                uint32_t n, uint32_t n_rows, float eps)
{
    if (!x || !weight || !out || n == 0 || n_rows == 0 || !(eps >= 0.0f) || !ensure_init()) return -1;
    const size_t bytes = (size_t)n * n_rows * 4;
    if (!fits(x, bytes, "x") || !fits(weight, (size_t)n * 4, "weight") || !fits(out, bytes, "out")) return -1;
    KScope ks("rms_norm");
    return finish(launch_rms_norm(fptr(x), fptr(weight), fptr(out), (int)n, (int)n_rows, eps, n, n, g.stream),
                  "rms_norm");
}

// ===========================================================================
// MoE
// ===========================================================================

namespace {

ExpertWeights make_ew(const ds3_hip_buffer_t *wg, const ds3_hip_buffer_t *wu, const ds3_hip_buffer_t *wd, int gt,
                      int ut, int dt, uint64_t gs, uint64_t us, uint64_t ds, const ds3_hip_buffer_t *table)
{
    ExpertWeights ew;
    ew.gate = cptr(wg);
    ew.up = cptr(wu);
    ew.down = cptr(wd);
    ew.gate_stride = gs;
    ew.up_stride = us;
    ew.down_stride = ds;
    ew.gate_type = gt;
    ew.up_type = ut;
    ew.down_type = dt;
    ew.table = table ? (const uint64_t *)dptr(table) : nullptr;
    return ew;
}

// Shared expert, weight 1, accumulated into out (reference src/ds3_metal.m:2227-2243).
int run_shared(const float *x, const ds3_hip_buffer_t *sg, const ds3_hip_buffer_t *su, const ds3_hip_buffer_t *sd,
               int sgt, int sut, int sdt, uint64_t sgs, uint64_t sus, uint64_t sds, uint32_t n_embd,
               uint32_t n_ff_shared, float *out, float *h, float *tmp)
{
    ExpertWeights ew = make_ew(sg, su, sd, sgt, sut, sdt, sgs, sus, sds, nullptr);
    return run_experts_decode(x, n_embd, g.zero_idx, g.one_f, 1, 1, ew, n_embd, n_ff_shared, out, nullptr, true, h,
                              tmp);
}

bool moe_limits_ok(uint32_t n_expert, uint32_t n_used)
{
    if (n_expert > 256 || n_used > 16) {
        fprintf(stderr, "ds3_hip: n_expert=%u (max 256) / n_used=%u (max 16) out of range\n", n_expert, n_used);
        return false;
    }
    return true;
}

}  // namespace

namespace {

struct RouteBufs {
    float *logits;       // [T][E] router logits (output)
    int32_t *idx;
    float *scores;
    float *wf32;         // [E][n_embd] FP32 copy of router rows stored in another type
    _Float16 *x16;       // optional [T][n_embd] fp16 copy of x, written by the router
    void *cert;          // certified router scratch (router_cert_scratch bytes)
};

// Scratch of route_tokens beyond the output buffers, laid out from `base`.
struct RouteScratch {
    size_t o_wf32, o_cert, bytes;
};

RouteScratch route_scratch(int T, uint32_t n_embd, uint32_t n_expert)
{
    Bump b;
    RouteScratch r;
    r.o_wf32 = b.take((size_t)n_expert * n_embd * 4);
    r.o_cert = b.take(router_cert_scratch(T, (int)n_expert));
    r.bytes = b.off;
    return r;
}

RouteBufs route_bufs(uint8_t *base, const RouteScratch &r, float *logits, int32_t *idx, float *scores,
                     _Float16 *x16)
{
    return RouteBufs{ logits, idx, scores, (float *)(base + r.o_wf32), x16, base + r.o_cert };
}

// Whether the certified router serves this call: entry points that only need
// the routing (allow) take it for few tokens, or always under router mode 2;
// mode 1 keeps the sequential-order router everywhere.
bool use_cert(const float *x, int T, uint32_t n_embd, uint32_t n_expert, uint32_t n_used, bool allow)
{
    if (g.router_mode == 1 || !router_cert_ok((int)n_embd, (int)n_expert, (int)n_used)) return false;
    if (((uintptr_t)x & 15) != 0) return false;
    if (g.router_mode == 2) return true;
    return allow && T <= kCertMaxTokens;
}

// Router logits + softmax/top-k/renorm for T tokens.  Sets *x16_done when the
// router also wrote rb.x16.  With defer, a certified selection may be left to
// the decode gate/up kernel (defer->on): the routing outputs are then written
// by that kernel.  With np (certified router only), x holds raw rows and the
// router's sums kernel normalises them, writing np->xn, which the rest of the
// routing reads.  allow_cert: the caller runs the decode gate/up kernels next
// and passes them `exact`, which is set (exact->w != nullptr) when the
// certified selection launch routed the tokens: those kernels then replace
// its weights with ones from the exact logits of the selected experts.
int route_tokens(const float *x, const ds3_hip_buffer_t *router, uint64_t rstride, int rtype, int T, uint32_t n_embd,
                 uint32_t n_expert, uint32_t n_used, bool norm, const RouteBufs &rb, bool *x16_done = nullptr,
                 bool allow_cert = false, DeferredSel *defer = nullptr, const NormPro *np = nullptr,
                 ExactTail *exact = nullptr, uint8_t *masks = nullptr, bool *marked = nullptr)
{
    if (exact) *exact = ExactTail{};
    if (marked) *marked = false;
    RouteArgs ra{};
    ra.logits = rb.logits;
    ra.idx = rb.idx;
    ra.scores = rb.scores;
    ra.T = T;
    ra.E = (int)n_expert;
    ra.k = (int)n_used;
    ra.logit_stride = n_expert;
    ra.out_stride = n_used;
    ra.norm = norm;
    // a read-only router's FP32 copy, made once: the routing then reads F32 rows
    const float *rf = router_f32_rows(router, rtype, n_expert, n_embd, rstride);
    const uint8_t *rw = rf ? (const uint8_t *)rf : cptr(router);
    if (rf) {
        rtype = T_F32;
        rstride = (uint64_t)n_embd * 4;
    }
    hipError_t e;
    if (use_cert(x, T, n_embd, n_expert, n_used, allow_cert)) {
        {
            KScope ks("router_sums");
            e = launch_router_cert(x, T, (int)n_embd, (int)n_expert, rtype, rw, rstride, rb.wf32,
                                   rb.logits, n_expert, rb.x16, ra, rb.cert, g.cert_stats, 1, g.stream, np);
        }
        if (np != nullptr) x = np->xn;
        if (e == hipSuccess && defer != nullptr && T <= kFuseSelMaxTokens) {
            // repair batch of the fused kernel: 4 candidate rows (~32 KiB of
            // LDS at K = 2048) keep 3 of its workgroups per CU at T <= 2
            const int rowb = ((int)n_embd + 4) * 4;
            const int nb = std::max(1, std::min(T <= 2 ? DS3_FUSED_NB : 2, 33792 / rowb));
            e = router_cert_sel(T, (int)n_embd, (int)n_expert, (int)n_used, rtype, rw, rstride, rb.wf32,
                                rb.cert, g.cert_stats, nb, &defer->cs);
            if (e == hipSuccess) {
                defer->on = true;
                defer->ra = ra;
            }
        } else if (e == hipSuccess) {
            {
                KScope ks("router_select");
                e = launch_router_cert(x, T, (int)n_embd, (int)n_expert, rtype, rw, rstride, rb.wf32,
                                       rb.logits, n_expert, rb.x16, ra, rb.cert, g.cert_stats, 2, g.stream);
            }
            CertSel cs{};
            if (e == hipSuccess && exact != nullptr &&
                router_cert_sel(T, (int)n_embd, (int)n_expert, (int)n_used, rtype, rw, rstride, rb.wf32,
                                rb.cert, g.cert_stats, 1, &cs) == hipSuccess)
                *exact = ExactTail{ cs.w, cs.wstride, ra };
        }
        if (x16_done) *x16_done = rb.x16 != nullptr;
        return report(e, "router (certified)");
    }
    if (np != nullptr) return report(hipErrorInvalidValue, "router: fused norm needs the certified router");
    bool topk_done = false;
    {
        KScope ks("router_logits");
        e = launch_router_seq(x, T, (int)n_embd, (int)n_expert, rtype, rw, rstride, rb.wf32, rb.logits,
                              n_expert, rb.x16, &ra, g.tickets, &topk_done, g.stream);
    }
    if (e != hipSuccess) return report(e, "router logits");
    if (x16_done) *x16_done = rb.x16 != nullptr;
    if (topk_done) return 0;                    // the router kernel also selected the experts
    KScope ks("router_topk");
    if (masks != nullptr) {
        // also the 4-token bitmaps the grouped path's placement reads
        e = launch_route_mark(ra, masks, g.stream);
        if (e == hipSuccess && marked) *marked = true;
        return report(e, "router topk");
    }
    return report(launch_route(ra, g.stream), "router topk");
}

// Largest token chunk whose bucketing bitmaps fit in LDS.
int prefill_chunk(uint32_t n_expert)
{
    int c = (int)(61440 / (6 * n_expert)) * 32;
    if (c > 2048) c = 2048;
    if (c < 32) c = 32;
    return c;
}

}  // namespace

// reference src/ds3_metal.m:2415-2661
extern "C" int ds3_hip_moe_ffn(
    const ds3_hip_buffer_t *input, const ds3_hip_buffer_t *w_gate_inp, const ds3_hip_buffer_t *w_gate_exps,
    const ds3_hip_buffer_t *w_up_exps, const ds3_hip_buffer_t *w_down_exps, ds3_hip_type_t gate_type,
    ds3_hip_type_t up_type, ds3_hip_type_t down_type, uint64_t gate_row_stride, uint64_t up_row_stride,
    uint64_t down_row_stride, const ds3_hip_buffer_t *w_shared_gate, const ds3_hip_buffer_t *w_shared_up,
    const ds3_hip_buffer_t *w_shared_down, ds3_hip_type_t shared_gate_type, ds3_hip_type_t shared_up_type,
    ds3_hip_type_t shared_down_type, uint64_t shared_gate_row_stride, uint64_t shared_up_row_stride,
    uint64_t shared_down_row_stride, ds3_hip_buffer_t *output, ds3_hip_buffer_t *gate_logits,
    const ds3_hip_buffer_t *expert_offsets, ds3_hip_buffer_t *hidden, ds3_hip_buffer_t *expert_up,
    ds3_hip_buffer_t *expert_down, uint32_t n_embd, uint32_t n_expert, uint32_t n_used, uint32_t n_ff_exp,
    uint32_t n_ff_shared, uint64_t router_row_stride, ds3_hip_type_t router_type, bool norm_topk_prob)
{
    const bool has_shared = w_shared_gate && w_shared_up && w_shared_down;
    if (!input || !w_gate_inp || !w_gate_exps || !w_up_exps || !w_down_exps || !output || !gate_logits || !hidden)
        return -1;
    if (!quant_type_ok_for_moe(gate_type, n_embd, "gate") || !quant_type_ok_for_moe(up_type, n_embd, "up") ||
        !quant_type_ok_for_moe(down_type, n_ff_exp, "down"))
        return -1;
    if (has_shared && (!quant_type_ok_for_moe(shared_gate_type, n_embd, "shared_gate") ||
                       !quant_type_ok_for_moe(shared_up_type, n_embd, "shared_up") ||
                       !quant_type_ok_for_moe(shared_down_type, n_ff_shared, "shared_down")))
        return -1;
    const bool routed_q = is_quant(gate_type) || is_quant(up_type) || is_quant(down_type);
    const bool shared_q =
        has_shared && (is_quant(shared_gate_type) || is_quant(shared_up_type) || is_quant(shared_down_type));
    if ((routed_q || shared_q) && (!expert_up || !expert_down)) {
        fprintf(stderr, "ds3_hip: quantized MoE path requires expert_up/expert_down scratch buffers\n");
        return -1;
    }
    if (n_embd == 0 || n_expert == 0 || n_used == 0 || n_ff_exp == 0) return -1;
    if (n_used > n_expert) return -1;
    if (!moe_limits_ok(n_expert, n_used) || !router_seq_type_ok(router_type, (int)n_embd) || !ensure_init()) {
        if (!router_seq_type_ok(router_type, (int)n_embd))
            fprintf(stderr, "ds3_hip: router type %d unsupported\n", router_type);
        return -1;
    }
    if (!fits(input, (size_t)n_embd * 4, "input") || !fits(output, (size_t)n_embd * 4, "output") ||
        !fits(gate_logits, (size_t)n_expert * 4, "gate_logits"))
        return -1;
    if (!moe_weights_fit(w_gate_inp, router_row_stride, router_type, w_gate_exps, w_up_exps, w_down_exps, gate_type,
                         up_type, down_type, gate_row_stride, up_row_stride, down_row_stride, expert_offsets, n_embd,
                         n_expert, n_ff_exp))
        return -1;
    if (has_shared &&
        (!fits(w_shared_gate, span_bytes(n_ff_shared, shared_gate_row_stride, row_bytes(shared_gate_type, n_embd)),
               "shared_gate") ||
         !fits(w_shared_up, span_bytes(n_ff_shared, shared_up_row_stride, row_bytes(shared_up_type, n_embd)),
               "shared_up") ||
         !fits(w_shared_down, span_bytes(n_embd, shared_down_row_stride, row_bytes(shared_down_type, n_ff_shared)),
               "shared_down") ||
         shared_gate_row_stride < row_bytes(shared_gate_type, n_embd) ||
         shared_up_row_stride < row_bytes(shared_up_type, n_embd) ||
         shared_down_row_stride < row_bytes(shared_down_type, n_ff_shared))) {
        fprintf(stderr, "ds3_hip: moe_ffn: shared expert weights smaller than their shapes\n");
        return -1;
    }

    const uint32_t ff_max = has_shared && n_ff_shared > n_ff_exp ? n_ff_shared : n_ff_exp;
    Bump bp;
    const size_t o_idx = bp.take((size_t)n_used * 4), o_sc = bp.take((size_t)n_used * 4);
    const RouteScratch rs = route_scratch(1, n_embd, n_expert);
    const size_t o_r = bp.take(rs.bytes);
    const size_t o_h = bp.take((size_t)n_used * ff_max * 4), o_t = bp.take((size_t)n_used * ff_max * 4);
    uint8_t *ws = ws_get(bp.off);
    if (!ws) return -1;
    int32_t *idx = (int32_t *)(ws + o_idx);
    float *sc = (float *)(ws + o_sc), *h = (float *)(ws + o_h), *tmp = (float *)(ws + o_t);
    const float *x = fptr(input);
    const RouteBufs rb = route_bufs(ws + o_r, rs, fptr(gate_logits), idx, sc, nullptr);
    DeferredSel sel;
    ExactTail xt{};
    if (route_tokens(x, w_gate_inp, router_row_stride, router_type, 1, n_embd, n_expert, n_used, norm_topk_prob,
                     rb, nullptr, true, gate_type == up_type ? &sel : nullptr, nullptr, &xt) != 0)
        return -1;
    if (has_shared &&
        run_shared(x, w_shared_gate, w_shared_up, w_shared_down, shared_gate_type, shared_up_type, shared_down_type,
                   shared_gate_row_stride, shared_up_row_stride, shared_down_row_stride, n_embd, n_ff_shared,
                   fptr(output), h, tmp) != 0)
        return -1;
    ExpertWeights ew = make_ew(w_gate_exps, w_up_exps, w_down_exps, gate_type, up_type, down_type, gate_row_stride,
                               up_row_stride, down_row_stride, expert_offsets);
    if (run_experts_decode(x, n_embd, idx, sc, 1, (int)n_used, ew, n_embd, n_ff_exp, fptr(output), nullptr, true, h,
                           tmp, &sel, xt.w ? &xt : nullptr) != 0)
        return -1;
    return finish(hipSuccess, "moe_ffn");
}

extern "C" int ds3_hip_moe_ffn_router(const ds3_hip_buffer_t *input, const ds3_hip_buffer_t *w_gate_inp,
                                      ds3_hip_buffer_t *gate_logits, uint32_t n_embd, uint32_t n_expert,
                                      uint64_t router_row_stride, ds3_hip_type_t router_type)
{
    // the logits of the reference's sequential fp32 sums, bit for bit
    if (!input || !w_gate_inp || !gate_logits || n_embd == 0 || n_expert == 0 || n_expert > 256 ||
        !router_seq_type_ok(router_type, (int)n_embd) || !ensure_init())
        return -1;
    if (!fits(input, (size_t)n_embd * 4, "input") || !fits(gate_logits, (size_t)n_expert * 4, "gate_logits") ||
        !fits(w_gate_inp, (size_t)n_expert * router_row_stride, "router"))
        return -1;
    const RouteScratch rs = route_scratch(1, n_embd, n_expert);
    uint8_t *ws = ws_get(rs.bytes);
    if (!ws) return -1;
    KScope ks("router_logits");
    return finish(launch_router_seq(fptr(input), 1, (int)n_embd, (int)n_expert, router_type, cptr(w_gate_inp),
                                    router_row_stride, (float *)(ws + rs.o_wf32), fptr(gate_logits), n_expert,
                                    nullptr, nullptr, nullptr, nullptr, g.stream),
                  "moe_ffn_router");
}

// reference src/ds3_metal.m:2172-2290
extern "C" int ds3_hip_moe_ffn_experts(
    const ds3_hip_buffer_t *input, const ds3_hip_buffer_t *w_gate_exps, const ds3_hip_buffer_t *w_up_exps,
    const ds3_hip_buffer_t *w_down_exps, ds3_hip_type_t gate_type, ds3_hip_type_t up_type, ds3_hip_type_t down_type,
    uint64_t gate_row_stride, uint64_t up_row_stride, uint64_t down_row_stride, const ds3_hip_buffer_t *w_shared_gate,
    const ds3_hip_buffer_t *w_shared_up, const ds3_hip_buffer_t *w_shared_down, ds3_hip_type_t shared_gate_type,
    ds3_hip_type_t shared_up_type, ds3_hip_type_t shared_down_type, uint64_t shared_gate_row_stride,
    uint64_t shared_up_row_stride, uint64_t shared_down_row_stride, ds3_hip_buffer_t *output, ds3_hip_buffer_t *hidden,
    ds3_hip_buffer_t *expert_up, ds3_hip_buffer_t *expert_down, uint32_t n_embd, uint32_t n_used, uint32_t n_ff_exp,
    uint32_t n_ff_shared, const int32_t *indices_host, const float *scores_host)
{
    (void)hidden;
    (void)expert_up;
    (void)expert_down;
    if (!input || !w_gate_exps || !w_up_exps || !w_down_exps || !output || !indices_host || !scores_host) return -1;
    if (n_embd == 0 || n_used == 0 || n_ff_exp == 0) return -1;
    const bool has_shared = w_shared_gate && w_shared_up && w_shared_down;
    if (!quant_type_ok_for_moe(gate_type, n_embd, "gate") || !quant_type_ok_for_moe(up_type, n_embd, "up") ||
        !quant_type_ok_for_moe(down_type, n_ff_exp, "down"))
        return -1;
    if (has_shared && (!quant_type_ok_for_moe(shared_gate_type, n_embd, "shared_gate") ||
                       !quant_type_ok_for_moe(shared_up_type, n_embd, "shared_up") ||
                       !quant_type_ok_for_moe(shared_down_type, n_ff_shared, "shared_down")))
        return -1;
    if (n_used > 16 || refuse_in_capture("moe_ffn_experts (copies the host's indices and scores)") || !ensure_init())
        return -1;
    if (!fits(input, (size_t)n_embd * 4, "input") || !fits(output, (size_t)n_embd * 4, "output")) return -1;
    if (has_shared) {
        const int sgt = shared_gate_type, sut = shared_up_type, sdt = shared_down_type;
        if (!fits(w_shared_gate, (size_t)n_ff_shared * shared_gate_row_stride, "shared_gate") ||
            !fits(w_shared_up, (size_t)n_ff_shared * shared_up_row_stride, "shared_up") ||
            !fits(w_shared_down, (size_t)n_embd * shared_down_row_stride, "shared_down") ||
            shared_gate_row_stride < (uint64_t)row_bytes(sgt, n_embd) ||
            shared_up_row_stride < (uint64_t)row_bytes(sut, n_embd) ||
            shared_down_row_stride < (uint64_t)row_bytes(sdt, n_ff_shared)) {
            fprintf(stderr, "ds3_hip: moe_ffn_experts: shared expert weights smaller than their shapes\n");
            return -1;
        }
    }
    // Host-selected expert ids must address rows inside every expert tensor.
    {
        const uint64_t ne_g = gate_row_stride ? w_gate_exps->bytes / ((uint64_t)n_ff_exp * gate_row_stride) : 0;
        const uint64_t ne_u = up_row_stride ? w_up_exps->bytes / ((uint64_t)n_ff_exp * up_row_stride) : 0;
        const uint64_t ne_d = down_row_stride ? w_down_exps->bytes / ((uint64_t)n_embd * down_row_stride) : 0;
        const uint64_t ne = ne_g < ne_u ? (ne_g < ne_d ? ne_g : ne_d) : (ne_u < ne_d ? ne_u : ne_d);
        for (uint32_t i = 0; i < n_used; i++) {
            if (indices_host[i] < 0 || (uint64_t)indices_host[i] >= ne) {
                fprintf(stderr, "ds3_hip: moe_ffn_experts: expert id %d outside the %llu experts the weights hold\n",
                        indices_host[i], (unsigned long long)ne);
                return -1;
            }
        }
    }
    const uint32_t ff_max = has_shared && n_ff_shared > n_ff_exp ? n_ff_shared : n_ff_exp;
    Bump bp;
    const size_t o_idx = bp.take((size_t)n_used * 4), o_sc = bp.take((size_t)n_used * 4);
    const size_t o_h = bp.take((size_t)n_used * ff_max * 4), o_t = bp.take((size_t)n_used * ff_max * 4);
    uint8_t *ws = ws_get(bp.off);
    if (!ws) return -1;
    int32_t *idx = (int32_t *)(ws + o_idx);
    float *sc = (float *)(ws + o_sc), *h = (float *)(ws + o_h), *tmp = (float *)(ws + o_t);
    if (hipMemcpyAsync(idx, indices_host, (size_t)n_used * 4, hipMemcpyHostToDevice, g.stream) != hipSuccess ||
        hipMemcpyAsync(sc, scores_host, (size_t)n_used * 4, hipMemcpyHostToDevice, g.stream) != hipSuccess)
        return -1;
    const float *x = fptr(input);
    if (has_shared &&
        run_shared(x, w_shared_gate, w_shared_up, w_shared_down, shared_gate_type, shared_up_type, shared_down_type,
                   shared_gate_row_stride, shared_up_row_stride, shared_down_row_stride, n_embd, n_ff_shared,
                   fptr(output), h, tmp) != 0)
        return -1;
    ExpertWeights ew = make_ew(w_gate_exps, w_up_exps, w_down_exps, gate_type, up_type, down_type, gate_row_stride,
                               up_row_stride, down_row_stride, nullptr);
    if (run_experts_decode(x, n_embd, idx, sc, 1, (int)n_used, ew, n_embd, n_ff_exp, fptr(output), nullptr, true, h,
                           tmp) != 0)
        return -1;
    return finish(hipSuccess, "moe_ffn_experts");
}

static int topk_rows(const ds3_hip_buffer_t *logits, ds3_hip_buffer_t *indices, ds3_hip_buffer_t *scores, uint32_t rows,
                     uint32_t n_expert, uint32_t n_used, bool norm, const char *what)
{
    if (!logits || !indices || !scores || rows == 0 || n_expert == 0 || n_used == 0) return -1;
    if (n_used > n_expert || n_expert > 256 || n_used > 32 || !ensure_init()) return -1;
    if (!fits(logits, (size_t)rows * n_expert * 4, "logits") || !fits(indices, (size_t)rows * n_used * 4, "indices") ||
        !fits(scores, (size_t)rows * n_used * 4, "scores"))
        return -1;
    RouteArgs ra{};
    ra.logits = fptr(logits);
    ra.idx = (int32_t *)dptr(indices);
    ra.scores = fptr(scores);
    ra.T = (int)rows;
    ra.E = (int)n_expert;
    ra.k = (int)n_used;
    ra.logit_stride = n_expert;
    ra.out_stride = n_used;
    ra.norm = norm;
    KScope ks("router_topk");
    return finish(launch_route(ra, g.stream), what);
}

extern "C" int ds3_hip_moe_router_topk_batch(const ds3_hip_buffer_t *logits, ds3_hip_buffer_t *indices,
                                             ds3_hip_buffer_t *scores, uint32_t n_layers, uint32_t n_expert,
                                             uint32_t n_used, bool norm_topk_prob)
{
    return topk_rows(logits, indices, scores, n_layers, n_expert, n_used, norm_topk_prob, "moe_router_topk_batch");
}

extern "C" int ds3_hip_moe_router_topk_batch_tokens(const ds3_hip_buffer_t *logits, ds3_hip_buffer_t *indices,
                                                    ds3_hip_buffer_t *scores, uint32_t n_layers, uint32_t n_tokens,
                                                    uint32_t n_expert, uint32_t n_used, bool norm_topk_prob)
{
    if (n_tokens == 0) return -1;
    return topk_rows(logits, indices, scores, n_layers * n_tokens, n_expert, n_used, norm_topk_prob,
                     "moe_router_topk_batch_tokens");
}

// ===========================================================================
// Device-routed extensions
// ===========================================================================


extern "C" int ds3_hip_moe_route(const ds3_hip_buffer_t *input, const ds3_hip_buffer_t *w_gate_inp,
                                 ds3_hip_buffer_t *gate_logits, ds3_hip_buffer_t *indices, ds3_hip_buffer_t *scores,
                                 uint32_t n_tokens, uint32_t n_embd, uint32_t n_expert, uint32_t n_used,
                                 uint64_t router_row_stride, ds3_hip_type_t router_type, bool norm_topk_prob)
{
    if (!input || !w_gate_inp || !indices || !scores || n_tokens == 0 || n_embd == 0 || n_expert == 0 ||
        n_used == 0 || n_used > n_expert || !ensure_init())
        return -1;
    if (!moe_limits_ok(n_expert, n_used) || !router_seq_type_ok(router_type, (int)n_embd)) return -1;
    const size_t T = n_tokens;
    if (!fits(input, T * n_embd * 4, "input") || !fits(indices, T * n_used * 4, "indices") ||
        !fits(scores, T * n_used * 4, "scores") || !fits(gate_logits, T * n_expert * 4, "gate_logits"))
        return -1;
    Bump bp;
    const RouteScratch rs = route_scratch((int)T, n_embd, n_expert);
    const size_t o_l = bp.take(T * n_expert * 4), o_r = bp.take(rs.bytes);
    uint8_t *ws = ws_get(bp.off);
    if (!ws) return -1;
    const RouteBufs rb = route_bufs(ws + o_r, rs, gate_logits ? fptr(gate_logits) : (float *)(ws + o_l),
                                    (int32_t *)dptr(indices), fptr(scores), nullptr);
    if (route_tokens(fptr(input), w_gate_inp, router_row_stride, router_type, (int)T, n_embd, n_expert, n_used,
                     norm_topk_prob, rb) != 0)
        return -1;
    return finish(hipSuccess, "moe_route");
}

extern "C" int ds3_hip_moe_bucket(const ds3_hip_buffer_t *indices, const ds3_hip_buffer_t *scores, uint32_t n_tokens,
                                  uint32_t n_used, uint32_t n_expert, ds3_hip_buffer_t *counts,
                                  ds3_hip_buffer_t *offsets, ds3_hip_buffer_t *ids, ds3_hip_buffer_t *wts,
                                  ds3_hip_buffer_t *slot_pos)
{
    if (!indices || !scores || !counts || !offsets || !ids || !wts || !slot_pos || n_tokens == 0 || n_used == 0 ||
        n_expert == 0 || !ensure_init())
        return -1;
    const size_t S = (size_t)n_tokens * n_used;
    if (!fits(indices, S * 4, "indices") || !fits(scores, S * 4, "scores") || !fits(counts, n_expert * 4, "counts") ||
        !fits(offsets, ((size_t)n_expert + 1) * 4, "offsets") || !fits(ids, S * 4, "ids") ||
        !fits(wts, S * 4, "wts") || !fits(slot_pos, S * 4, "slot_pos"))
        return -1;
    const int max_tiles = (int)((S + 63) / 64) + (int)n_expert;
    Bump bp;
    const size_t o_t = bp.take((size_t)max_tiles * 4), o_n = bp.take(4);
    uint8_t *ws = ws_get(bp.off);
    if (!ws) return -1;
    BucketOut bo{ (int32_t *)dptr(counts), (int32_t *)dptr(offsets), (int32_t *)dptr(ids), fptr(wts),
                  (int32_t *)dptr(slot_pos), (int32_t *)(ws + o_t), (int32_t *)(ws + o_n), max_tiles, 64 };
    KScope ks("bucket");
    return finish(launch_bucket((const int32_t *)dptr(indices), fptr(scores), (int)n_tokens, (int)n_used,
                                (int)n_expert, bo, g.stream),
                  "moe_bucket");
}

namespace {

// Optional RMSNorm prologue of moe_batch: the input rows are the hidden state,
// and the MoE runs on rms_norm(hidden) * weight, written to xn (or workspace).
struct NormIn {
    const float *weight;
    float eps;
    float *xn;
};

// A caller-fixed workspace (the allocation-free entry point's scratch array):
// moe_batch uses it instead of growing the library workspace.
struct WsFixed {
    uint8_t *base;
    size_t cap;
};

// The batch MoE of ds3_hip_moe_ffn_batch / ds3_hip_moe_block on raw device
// rows: input x_in [T][n_embd]; out (+)= result (+ residual res); the routing
// outputs (logits, indices, scores) are optional.  With `fixed`, the call's
// workspace is fixed->base and a call that needs more fails.
int moe_batch(const float *x_in, const NormIn *norm, const ds3_hip_buffer_t *w_gate_inp,
              const ds3_hip_buffer_t *w_gate_exps, const ds3_hip_buffer_t *w_up_exps,
              const ds3_hip_buffer_t *w_down_exps, ds3_hip_type_t gate_type, ds3_hip_type_t up_type,
              ds3_hip_type_t down_type, uint64_t gate_row_stride, uint64_t up_row_stride, uint64_t down_row_stride,
              const ds3_hip_buffer_t *expert_offsets, float *out, const float *res, float *logits_out,
              int32_t *idx_out, float *scores_out, uint32_t n_tokens, uint32_t n_embd, uint32_t n_expert,
              uint32_t n_used, uint32_t n_ff_exp, uint64_t router_row_stride, ds3_hip_type_t router_type,
              bool norm_topk_prob, const char *what, const WsFixed *fixed = nullptr)
{
    if (!w_gate_inp || !w_gate_exps || !w_up_exps || !w_down_exps) return -1;
    if (n_tokens == 0 || n_embd == 0 || n_expert == 0 || n_used == 0 || n_ff_exp == 0 || n_used > n_expert)
        return -1;
    if (!quant_type_ok_for_moe(gate_type, n_embd, "gate") || !quant_type_ok_for_moe(up_type, n_embd, "up") ||
        !quant_type_ok_for_moe(down_type, n_ff_exp, "down"))
        return -1;
    if (!moe_limits_ok(n_expert, n_used) || !ensure_init()) return -1;
    if (!router_seq_type_ok(router_type, (int)n_embd)) {
        fprintf(stderr, "ds3_hip: router type %d unsupported\n", router_type);
        return -1;
    }
    if (!moe_weights_fit(w_gate_inp, router_row_stride, router_type, w_gate_exps, w_up_exps, w_down_exps, gate_type,
                         up_type, down_type, gate_row_stride, up_row_stride, down_row_stride, expert_offsets, n_embd,
                         n_expert, n_ff_exp))
        return -1;
    const size_t T = n_tokens;

    const bool grouped_ok = gate_type == up_type && grouped_type_ok(gate_type, (int)n_embd) &&
                            grouped_type_ok(down_type, (int)n_ff_exp) && grouped_shape_ok((int)n_embd, (int)n_ff_exp);
    const bool use_grouped = grouped_ok && (int)n_tokens >= g.prefill_min;
    const int chunk = use_grouped ? prefill_chunk(n_expert) : (int)n_tokens;
    const size_t Tc = (size_t)(chunk < (int)n_tokens ? chunk : (int)n_tokens);
    const size_t S = Tc * n_used;
    const int max_tiles = (int)((S + 63) / 64) + (int)n_expert;
    // routing writes the placement's bitmaps (4-token rows).  A call of more
    // than one chunk places chunk by chunk: the chunk must then be a multiple
    // of 32 tokens, and every chunk's slice of the bitmaps must start on 16
    // bytes, as the placement loads them.
    const bool mark = use_grouped && n_expert <= 256 && n_used <= 32 && Tc <= 2048 && max_tiles <= 1280 &&
                      (T <= Tc || (Tc % 32 == 0 && (Tc / 4 * n_expert) % 16 == 0));

    Bump bp;
    const size_t o_xn = norm && !norm->xn ? bp.take(T * n_embd * 4) : 0;
    const size_t o_l = bp.take(T * n_expert * 4), o_i = bp.take(T * n_used * 4), o_s = bp.take(T * n_used * 4);
    const RouteScratch rs = route_scratch((int)T, n_embd, n_expert);
    const size_t o_w = bp.take(rs.bytes);
    size_t o_h = 0, o_t = 0, o_x16 = 0, o_cnt = 0, o_off = 0, o_ids = 0, o_wts = 0, o_pos = 0, o_tiles = 0, o_nt = 0,
           o_h16 = 0, o_y = 0, o_rg = 0, o_rd = 0, o_dg = 0, o_dd = 0, o_mask = 0;
    int rpi_gu = 0, rpi_dn = 0;
    if (use_grouped) {
        grouped_runs_per_tile((int)n_embd, (int)n_ff_exp, (int)S, (int)n_expert, rpi_gu, rpi_dn);
        o_x16 = bp.take(T * n_embd * 2);
        o_cnt = bp.take((size_t)n_expert * 4);
        o_off = bp.take(((size_t)n_expert + 1) * 4);
        o_ids = bp.take(S * 4);
        o_wts = bp.take(S * 4);
        o_pos = bp.take(S * 4);
        o_tiles = bp.take((size_t)max_tiles * 4);
        o_nt = bp.take(16);                          // n_tiles, then the two run counts
        o_rg = bp.take((size_t)max_tiles * rpi_gu * 4);
        o_rd = bp.take((size_t)max_tiles * rpi_dn * 4);
        o_dg = bp.take((size_t)max_tiles * rpi_gu * 8);
        o_dd = bp.take((size_t)max_tiles * rpi_dn * 8);
        o_h16 = bp.take(S * n_ff_exp * 2);
        o_y = bp.take(S * n_embd * 2);
        if (mark) o_mask = bp.take((T + 3) / 4 * n_expert);
    } else {
        o_h = bp.take(T * n_used * n_ff_exp * 4);
        o_t = bp.take(T * n_used * n_ff_exp * 4);
    }
    uint8_t *ws = nullptr;
    if (fixed) {
        if (bp.off > fixed->cap) {
            fprintf(stderr, "ds3_hip: %s: %u tokens need %zu scratch bytes, more than the %zu the allocation-free "
                            "entry point holds (split the call into fewer tokens)\n",
                    what, n_tokens, bp.off, fixed->cap);
            return -1;
        }
        ws = fixed->base;
    } else {
        ws = ws_get(bp.off);
    }
    if (!ws) return -1;
    const RouteBufs rb = route_bufs(ws + o_w, rs, logits_out ? logits_out : (float *)(ws + o_l),
                                    idx_out ? idx_out : (int32_t *)(ws + o_i), scores_out ? scores_out : (float *)(ws + o_s),
                                    use_grouped ? (_Float16 *)(ws + o_x16) : nullptr);
    // The norm: fused into the certified router's sums kernel where that
    // router serves the call, else its own launch before the router.
    const float *x = x_in;
    NormPro np{};
    bool fuse_norm = false;
    if (norm) {
        float *xn = norm->xn ? norm->xn : (float *)(ws + o_xn);
        np = NormPro{ norm->weight, norm->eps, xn };
        fuse_norm = use_cert(x_in, (int)T, n_embd, n_expert, n_used, !use_grouped) &&
                    ((uintptr_t)norm->weight & 15) == 0 && ((uintptr_t)xn & 15) == 0;
        if (!fuse_norm) {
            KScope ks("rms_norm");
            const hipError_t e = launch_rms_norm(x_in, norm->weight, xn, (int)n_embd, (int)T, norm->eps, n_embd,
                                                 n_embd, g.stream);
            if (e != hipSuccess) return report(e, what);
            x = xn;
        }
    }
    // the certified router only ahead of the decode kernels, which make its
    // weights exact (ExactTail / the fused selection)
    bool x16_done = false, marked = false;
    DeferredSel sel;
    ExactTail xt{};
    uint8_t *masks = mark ? ws + o_mask : nullptr;
    if (route_tokens(x, w_gate_inp, router_row_stride, router_type, (int)T, n_embd, n_expert, n_used, norm_topk_prob,
                     rb, &x16_done, !use_grouped, !use_grouped && gate_type == up_type ? &sel : nullptr,
                     fuse_norm ? &np : nullptr, &xt, masks, &marked) != 0)
        return -1;
    if (fuse_norm) x = np.xn;
    if (use_grouped && xt.w != nullptr) {
        // certified routing on the grouped path (router mode 2): the weights
        // from the exact logits of the selected experts, as the decode path's
        // gate/up launch computes them
        KScope ks("exact_weights");
        const hipError_t e = launch_exact_weights(x, n_embd, xt, (int)n_embd, g.stream);
        if (e != hipSuccess) return report(e, what);
    }
    ExpertWeights ew = make_ew(w_gate_exps, w_up_exps, w_down_exps, gate_type, up_type, down_type, gate_row_stride,
                               up_row_stride, down_row_stride, expert_offsets);
    if (!use_grouped) {
        if (run_experts_decode(x, n_embd, rb.idx, rb.scores, (int)T, (int)n_used, ew, n_embd, n_ff_exp, out, res, true,
                               (float *)(ws + o_h), (float *)(ws + o_t), &sel, xt.w ? &xt : nullptr) != 0)
            return -1;
        return finish(hipSuccess, what);
    }
    BucketOut bo{ (int32_t *)(ws + o_cnt), (int32_t *)(ws + o_off), (int32_t *)(ws + o_ids), (float *)(ws + o_wts),
                  (int32_t *)(ws + o_pos), (int32_t *)(ws + o_tiles), (int32_t *)(ws + o_nt), max_tiles, 64,
                  (int32_t *)(ws + o_rg), (int32_t *)(ws + o_rd), (int32_t *)(ws + o_nt) + 1, rpi_gu, rpi_dn,
                  (int2 *)(ws + o_dg), (int2 *)(ws + o_dd) };
    _Float16 *x16_all = (_Float16 *)(ws + o_x16), *h16 = (_Float16 *)(ws + o_h16);
    _Float16 *y = (_Float16 *)(ws + o_y);
    if (!x16_done) {
        KScope ks("to_f16");
        const hipError_t e = launch_to_f16(x, x16_all, (int64_t)T * n_embd, g.stream);
        if (e != hipSuccess) return report(e, what);
    }
    for (size_t t0 = 0; t0 < T; t0 += Tc) {
        const int tc = (int)((T - t0) < Tc ? (T - t0) : Tc);
        const _Float16 *x16 = x16_all + t0 * n_embd;
        hipError_t e = hipSuccess;
        {
            KScope ks("bucket");
            if (marked)
                e = launch_bucket_place(rb.idx + t0 * n_used, rb.scores + t0 * n_used, masks + t0 / 4 * n_expert, tc,
                                        (int)n_used, (int)n_expert, bo, g.stream);
            else
                e = launch_bucket(rb.idx + t0 * n_used, rb.scores + t0 * n_used, tc, (int)n_used, (int)n_expert, bo,
                                  g.stream);
        }
        if (e == hipSuccess) {
            g.lists.valid = true;
            g.lists.bo = bo;
            g.lists.t0 = (int)t0;
            g.lists.tc = tc;
            g.lists.k = (int)n_used;
            g.lists.E = (int)n_expert;
            g.lists.marked = marked;
        }
        if (e == hipSuccess) {
            KScope ks("moe_grouped_gate_up");
            e = launch_grouped_gate_up(x16, (int)n_embd, ew, (int)n_ff_exp, bo, h16, g.stream);
        }
        if (e == hipSuccess) {
            KScope ks("moe_grouped_down");
            e = launch_grouped_down(h16, (int)n_ff_exp, ew, (int)n_embd, bo, y, g.stream);
        }
        if (e == hipSuccess) {
            KScope ks("moe_combine");
            e = launch_combine(y, bo.slot_pos, rb.scores + t0 * n_used, tc, (int)n_used, (int)n_embd,
                               out + t0 * n_embd, n_embd, res ? res + t0 * n_embd : nullptr, true, g.stream);
        }
        if (e != hipSuccess) return report(e, what);
    }
    return finish(hipSuccess, what);
}

}  // namespace

extern "C" int ds3_hip_moe_ffn_batch(
    const ds3_hip_buffer_t *input, const ds3_hip_buffer_t *w_gate_inp, const ds3_hip_buffer_t *w_gate_exps,
    const ds3_hip_buffer_t *w_up_exps, const ds3_hip_buffer_t *w_down_exps, ds3_hip_type_t gate_type,
    ds3_hip_type_t up_type, ds3_hip_type_t down_type, uint64_t gate_row_stride, uint64_t up_row_stride,
    uint64_t down_row_stride, const ds3_hip_buffer_t *expert_offsets, ds3_hip_buffer_t *output,
    const ds3_hip_buffer_t *residual, ds3_hip_buffer_t *gate_logits, ds3_hip_buffer_t *indices,
    ds3_hip_buffer_t *scores, uint32_t n_tokens, uint32_t n_embd, uint32_t n_expert, uint32_t n_used,
    uint32_t n_ff_exp, uint64_t router_row_stride, ds3_hip_type_t router_type, bool norm_topk_prob)
{
    if (!input || !output) return -1;
    const size_t T = n_tokens;
    if (!fits(input, T * n_embd * 4, "input") || !fits(output, T * n_embd * 4, "output") ||
        !fits(residual, T * n_embd * 4, "residual") || !fits(gate_logits, T * n_expert * 4, "gate_logits") ||
        !fits(indices, T * n_used * 4, "indices") || !fits(scores, T * n_used * 4, "scores"))
        return -1;
    return moe_batch(fptr(input), nullptr, w_gate_inp, w_gate_exps, w_up_exps, w_down_exps, gate_type, up_type,
                     down_type, gate_row_stride, up_row_stride, down_row_stride, expert_offsets, fptr(output),
                     residual ? fptr(residual) : nullptr, gate_logits ? fptr(gate_logits) : nullptr,
                     indices ? (int32_t *)dptr(indices) : nullptr, scores ? fptr(scores) : nullptr, n_tokens, n_embd,
                     n_expert, n_used, n_ff_exp, router_row_stride, router_type, norm_topk_prob, "moe_ffn_batch");
}

// ds3_hip_moe_ffn_batch with every intermediate in the library's `scratch`
// array: no allocation of any kind.  No reference counterpart.
extern "C" int ds3_hip_moe_ffn_batch_noalloc(
    const ds3_hip_buffer_t *input, const ds3_hip_buffer_t *w_gate_inp, const ds3_hip_buffer_t *w_gate_exps,
    const ds3_hip_buffer_t *w_up_exps, const ds3_hip_buffer_t *w_down_exps, ds3_hip_type_t gate_type,
    ds3_hip_type_t up_type, ds3_hip_type_t down_type, uint64_t gate_row_stride, uint64_t up_row_stride,
    uint64_t down_row_stride, const ds3_hip_buffer_t *expert_offsets, ds3_hip_buffer_t *output,
    const ds3_hip_buffer_t *residual, ds3_hip_buffer_t *gate_logits, ds3_hip_buffer_t *indices,
    ds3_hip_buffer_t *scores, uint32_t n_tokens, uint32_t n_embd, uint32_t n_expert, uint32_t n_used,
    uint32_t n_ff_exp, uint64_t router_row_stride, ds3_hip_type_t router_type, bool norm_topk_prob)
{
    if (!input || !output) return -1;
    if (!g.inited) {
        // initialising allocates (stream, constants): callers that cannot allocate initialise first
        fprintf(stderr, "ds3_hip: moe_ffn_batch_noalloc needs ds3_hip_init first\n");
        return -1;
    }
    const size_t T = n_tokens;
    if (!fits(input, T * n_embd * 4, "input") || !fits(output, T * n_embd * 4, "output") ||
        !fits(residual, T * n_embd * 4, "residual") || !fits(gate_logits, T * n_expert * 4, "gate_logits") ||
        !fits(indices, T * n_used * 4, "indices") || !fits(scores, T * n_used * 4, "scores"))
        return -1;
    const WsFixed fx{ g.scratch_dev[g.device], kScratchBytes };
    g.no_alloc = true;
    const int rc = moe_batch(fptr(input), nullptr, w_gate_inp, w_gate_exps, w_up_exps, w_down_exps, gate_type,
                             up_type, down_type, gate_row_stride, up_row_stride, down_row_stride, expert_offsets,
                             fptr(output), residual ? fptr(residual) : nullptr,
                             gate_logits ? fptr(gate_logits) : nullptr, indices ? (int32_t *)dptr(indices) : nullptr,
                             scores ? fptr(scores) : nullptr, n_tokens, n_embd, n_expert, n_used, n_ff_exp,
                             router_row_stride, router_type, norm_topk_prob, "moe_ffn_batch_noalloc", &fx);
    g.no_alloc = false;
    return rc;
}

extern "C" size_t ds3_hip_noalloc_scratch_bytes(void) { return kScratchBytes; }

// reference src/ds3_engine.c:519-527, 675-720 (rms_norm, zero, moe_ffn, vec_add around the MoE)
extern "C" int ds3_hip_moe_block(
    ds3_hip_buffer_t *hidden, const ds3_hip_buffer_t *ffn_norm, float eps, const ds3_hip_buffer_t *w_gate_inp,
    const ds3_hip_buffer_t *w_gate_exps, const ds3_hip_buffer_t *w_up_exps, const ds3_hip_buffer_t *w_down_exps,
    ds3_hip_type_t gate_type, ds3_hip_type_t up_type, ds3_hip_type_t down_type, uint64_t gate_row_stride,
    uint64_t up_row_stride, uint64_t down_row_stride, const ds3_hip_buffer_t *expert_offsets,
    ds3_hip_buffer_t *x_norm, ds3_hip_buffer_t *gate_logits, ds3_hip_buffer_t *indices, ds3_hip_buffer_t *scores,
    uint32_t n_tokens, uint32_t n_embd, uint32_t n_expert, uint32_t n_used, uint32_t n_ff_exp,
    uint64_t router_row_stride, ds3_hip_type_t router_type, bool norm_topk_prob)
{
    if (!hidden || !ffn_norm || !(eps >= 0.0f)) return -1;
    const size_t T = n_tokens;
    if (!fits(hidden, T * n_embd * 4, "hidden") || !fits(ffn_norm, (size_t)n_embd * 4, "ffn_norm") ||
        !fits(x_norm, T * n_embd * 4, "x_norm") || !fits(gate_logits, T * n_expert * 4, "gate_logits") ||
        !fits(indices, T * n_used * 4, "indices") || !fits(scores, T * n_used * 4, "scores"))
        return -1;
    if (x_norm) {                                                     // the normalised rows must not overlap hidden
        const uint8_t *a = cptr(x_norm), *h = cptr(hidden);
        if (a < h + T * n_embd * 4 && h < a + T * n_embd * 4) return -1;
    }
    const NormIn norm{ fptr(ffn_norm), eps, x_norm ? fptr(x_norm) : nullptr };
    return moe_batch(fptr(hidden), &norm, w_gate_inp, w_gate_exps, w_up_exps, w_down_exps, gate_type, up_type,
                     down_type, gate_row_stride, up_row_stride, down_row_stride, expert_offsets, fptr(hidden), nullptr,
                     gate_logits ? fptr(gate_logits) : nullptr, indices ? (int32_t *)dptr(indices) : nullptr,
                     scores ? fptr(scores) : nullptr, n_tokens, n_embd, n_expert, n_used, n_ff_exp, router_row_stride,
                     router_type, norm_topk_prob, "moe_block");
}

extern "C" int ds3_hip_dequantize(const ds3_hip_buffer_t *src, uint64_t src_offset, ds3_hip_type_t type, uint64_t n,
                                  ds3_hip_buffer_t *dst)
{
    if (!src || !dst || n == 0 || !ensure_init()) return -1;
    int64_t blk = 0, bytes = 0;
    switch (type) {
    case T_F32: blk = 1; bytes = 4; break;
    case T_F16: blk = 1; bytes = 2; break;
    case T_Q8_0: blk = 32; bytes = 34; break;
    case T_Q4_K: blk = 256; bytes = 144; break;
    case T_Q6_K: blk = 256; bytes = 210; break;
    default: fprintf(stderr, "ds3_hip: dequantize: unsupported type %d\n", type); return -1;
    }
    if (n % (uint64_t)blk != 0) {
        fprintf(stderr, "ds3_hip: dequantize: n=%llu not a multiple of %lld\n", (unsigned long long)n, (long long)blk);
        return -1;
    }
    if ((type == T_Q6_K || type == T_Q8_0 || type == T_F16) && (src_offset & 1)) return -1;
    if ((type == T_Q4_K) && (src_offset & 15)) {
        fprintf(stderr, "ds3_hip: dequantize: Q4_K source offset must be 16-byte aligned\n");
        return -1;
    }
    if (type == T_F32 && (src_offset & 3)) return -1;
    if (!fits(src, src_offset + n / blk * bytes, "src") || !fits(dst, n * 4, "dst")) return -1;
    KScope ks("dequant");
    return finish(launch_dequant(type, cptr(src) + src_offset, fptr(dst), (int64_t)n, g.stream), "dequantize");
}

extern "C" int ds3_hip_debug_grouped_lists(int32_t *meta, int32_t *counts, int32_t *offsets, int32_t *ids,
                                           float *wts, int32_t *slot_pos, int32_t *tiles, int32_t *runs_gu,
                                           int32_t *runs_dn)
{
    if (!meta || refuse_in_capture("debug_grouped_lists") || !ensure_init()) return -1;
    if (!g.lists.valid) {
        fprintf(stderr, "ds3_hip: debug_grouped_lists: no grouped-path call since the workspace last moved\n");
        return -1;
    }
    const BucketOut &o = g.lists.bo;
    int32_t n[3] = { 0, 0, 0 };
    if (hipStreamSynchronize(g.stream) != hipSuccess ||
        hipMemcpy(&n[0], o.n_tiles, 4, hipMemcpyDeviceToHost) != hipSuccess ||
        hipMemcpy(&n[1], o.n_runs, 8, hipMemcpyDeviceToHost) != hipSuccess)
        return -1;
    const int E = g.lists.E, S = g.lists.tc * g.lists.k;
    const int32_t m[DS3_HIP_LISTS_META] = { g.lists.t0, g.lists.tc, g.lists.k, E, n[0], n[1], n[2],
                                            g.lists.marked ? 1 : 0, o.rpi_gu, o.rpi_dn, o.max_tiles, o.tile_m };
    memcpy(meta, m, sizeof m);
    struct { void *dst; const void *src; size_t bytes; } cp[] = {
        { counts, o.counts, (size_t)E * 4 }, { offsets, o.offsets, ((size_t)E + 1) * 4 },
        { ids, o.ids, (size_t)S * 4 }, { wts, o.wts, (size_t)S * 4 }, { slot_pos, o.slot_pos, (size_t)S * 4 },
        { tiles, o.tiles, (size_t)n[0] * 4 }, { runs_gu, o.runs_gu, (size_t)n[1] * 4 },
        { runs_dn, o.runs_dn, (size_t)n[2] * 4 } };
    for (const auto &c : cp)
        if (c.dst && c.bytes && hipMemcpy(c.dst, c.src, c.bytes, hipMemcpyDeviceToHost) != hipSuccess) return -1;
    return 0;
}

extern "C" int ds3_hip_debug_grouped_descs(int32_t *desc_gu, int32_t *desc_dn)
{
    if (refuse_in_capture("debug_grouped_descs") || !ensure_init()) return -1;
    if (!g.lists.valid || g.lists.bo.desc_gu == nullptr || g.lists.bo.desc_dn == nullptr) {
        fprintf(stderr, "ds3_hip: debug_grouped_descs: no grouped-path call since the workspace last moved\n");
        return -1;
    }
    const BucketOut &o = g.lists.bo;
    int32_t n[2] = { 0, 0 };
    if (hipStreamSynchronize(g.stream) != hipSuccess ||
        hipMemcpy(n, o.n_runs, 8, hipMemcpyDeviceToHost) != hipSuccess)
        return -1;
    if (desc_gu && n[0] > 0 && hipMemcpy(desc_gu, o.desc_gu, (size_t)n[0] * 8, hipMemcpyDeviceToHost) != hipSuccess)
        return -1;
    if (desc_dn && n[1] > 0 && hipMemcpy(desc_dn, o.desc_dn, (size_t)n[1] * 8, hipMemcpyDeviceToHost) != hipSuccess)
        return -1;
    return 0;
}

extern "C" int ds3_hip_router_stats(uint64_t *certified, uint64_t *repaired, int reset)
{
    if (refuse_in_capture("router_stats") || !ensure_init()) return -1;
    unsigned long long v[2] = { 0, 0 };
    if (hipStreamSynchronize(g.stream) != hipSuccess ||
        hipMemcpy(v, g.cert_stats, sizeof v, hipMemcpyDeviceToHost) != hipSuccess)
        return -1;
    if (certified) *certified = v[0];
    if (repaired) *repaired = v[1];
    if (reset && (launch_fill_zero((float *)g.cert_stats, 4, g.stream) != hipSuccess ||
                  hipStreamSynchronize(g.stream) != hipSuccess))
        return -1;
    return 0;
}

extern "C" int ds3_hip_set_router_mode(int mode)
{
    const int prev = g.router_mode;
    g.router_mode = (mode >= 0 && mode <= 2) ? mode : 0;
    return prev;
}

extern "C" int ds3_hip_set_dense_mfma_min_rows(int min_rows)
{
    const int prev = g.dense_mfma_min;
    g.dense_mfma_min = min_rows > 0 ? min_rows : kDefaultDenseMfmaMin;
    return prev;
}

extern "C" int ds3_hip_set_prefill_min_tokens(int min_tokens)
{
    const int prev = g.prefill_min;
    g.prefill_min = min_tokens > 0 ? min_tokens : kDefaultPrefillMin;
    return prev;
}

// ===========================================================================
// Batching and profiling (reference src/ds3_metal.m:2830-2900)
// ===========================================================================

extern "C" int ds3_hip_begin_batch(void)
{
    if (!ensure_init()) return -1;
    if (g.batch) {
        fprintf(stderr, "ds3_hip: begin_batch called while already in batch mode\n");
        return -1;
    }
    g.batch = true;
    if (g.profile) (void)hipEventRecord(g.bev0, g.stream);
    return 0;
}

extern "C" void ds3_hip_end_batch(void)
{
    if (!g.batch || refuse_in_capture("end_batch")) return;
    if (g.profile) (void)hipEventRecord(g.bev1, g.stream);
    const auto c0 = std::chrono::steady_clock::now();
    (void)hipStreamSynchronize(g.stream);
    const auto c1 = std::chrono::steady_clock::now();
    if (g.profile) {
        float ms = 0.f;
        (void)hipEventElapsedTime(&ms, g.bev0, g.bev1);
        g.gpu_ms += ms;
        g.cpu_ms += std::chrono::duration<double, std::milli>(c1 - c0).count();
        g.cb_count++;
    }
    g.batch = false;
}

// ===========================================================================
// HIP graphs (no ds3_metal.h counterpart): stream capture of library calls
// ===========================================================================

extern "C" int ds3_hip_graph_begin(void)
{
    if (!ensure_init()) return -1;
    if (g.batch || g.capturing) {
        fprintf(stderr, "ds3_hip: graph_begin inside batch mode or another capture\n");
        return -1;
    }
    if (g.ktiming) {
        fprintf(stderr, "ds3_hip: graph_begin with kernel timing on\n");
        return -1;
    }
    if (report(hipStreamBeginCapture(g.stream, hipStreamCaptureModeThreadLocal), "graph_begin") != 0) return -1;
    g.capturing = true;
    g.batch = true;                  // calls enqueue without waiting
    return 0;
}


extern "C" int ds3_hip_graph_end(void **graph)
{
    if (!g.capturing) return -1;
    hipGraph_t gr = nullptr;
    const hipError_t e = hipStreamEndCapture(g.stream, &gr);
    g.capturing = false;
    g.batch = false;
    free_deferred();
    if (report(e, "graph_end") != 0 || gr == nullptr) return -1;
    hipGraphExec_t ex = nullptr;
    const hipError_t ei = hipGraphInstantiate(&ex, gr, nullptr, nullptr, 0);
    (void)hipGraphDestroy(gr);
    if (report(ei, "graph_end (instantiate)") != 0) return -1;
    if (graph) {
        *graph = (void *)ex;
        g.graphs.push_back((void *)ex);          // pins the workspace block its kernels address
    } else {
        (void)hipGraphExecDestroy(ex);
    }
    return 0;
}

extern "C" int ds3_hip_debug_simulate_capture(int on)
{
    // only without a device context, where no real capture can be open
    if (g.inited) return -1;
    g.capturing = on != 0;
    return 0;
}

extern "C" int ds3_hip_graph_launch(void *graph)
{
    if (!graph || refuse_in_capture("graph_launch") || !ensure_init()) return -1;
    if (!graph_live(graph)) {
        fprintf(stderr, "ds3_hip: graph_launch of a graph that graph_end did not return or that was destroyed\n");
        return -1;
    }
    return finish(hipGraphLaunch((hipGraphExec_t)graph, g.stream), "graph_launch");
}

extern "C" void ds3_hip_graph_destroy(void *graph)
{
    if (!graph || !graph_live(graph)) return;
    if (g.inited) (void)hipStreamSynchronize(g.stream);     // a replay may still be running
    (void)hipGraphExecDestroy((hipGraphExec_t)graph);
    g.graphs.erase(std::find(g.graphs.begin(), g.graphs.end(), graph));
    free_retired();
}

extern "C" void ds3_hip_synchronize(void)
{
    if (g.inited && !refuse_in_capture("synchronize")) (void)hipStreamSynchronize(g.stream);
}

extern "C" void ds3_hip_profile_reset(void)
{
    g.cb_count = 0;
    g.gpu_ms = 0.0;
    g.cpu_ms = 0.0;
}

extern "C" void ds3_hip_profile_print(const char *label)
{
    if (!g.profile) return;
    fprintf(stderr, "[profile %s] cb_count=%d total_gpu_ms=%.3f total_cpu_wait_ms=%.3f\n", label ? label : "",
            g.cb_count, g.gpu_ms, g.cpu_ms);
}

extern "C" void ds3_hip_kernel_timing(int enable)
{
    if (!ensure_init()) return;
    if (enable && g.capturing) {
        fprintf(stderr, "ds3_hip: kernel timing cannot start during graph capture\n");
        return;
    }
    if (enable && g.pool.empty()) {
        // timing-only events: no system-scope fence (and its L2 writeback)
        // when recorded, which would otherwise add several microseconds to
        // every bracketed kernel
        g.pool.resize(16384);
        for (auto &e : g.pool) (void)hipEventCreateWithFlags(&e, hipEventDisableSystemFence);
    }
    g.ktiming = enable != 0;
}

extern "C" void ds3_hip_kernel_timing_only(const char *name)
{
    g.ktiming_only = name ? name : "";
}

extern "C" void ds3_hip_kernel_timing_reset(void)
{
    if (refuse_in_capture("kernel_timing_reset")) return;
    if (g.inited) (void)hipStreamSynchronize(g.stream);
    g.recs.clear();
    g.pool_used = 0;
    g.stat_names.clear();
    g.stat_count.clear();
    g.stat_ms.clear();
    g.stats_dirty = true;
}

extern "C" int ds3_hip_kernel_stats(int i, char *name, size_t name_len, int64_t *count, double *total_ms)
{
    if (!g.inited || refuse_in_capture("kernel_stats")) return -1;
    if (g.stats_dirty) {
        (void)hipStreamSynchronize(g.stream);
        g.stat_names.clear();
        g.stat_count.clear();
        g.stat_ms.clear();
        for (const KRec &r : g.recs) {
            float ms = 0.f;
            (void)hipEventElapsedTime(&ms, g.pool[r.e0], g.pool[r.e1]);
            size_t j = 0;
            while (j < g.stat_names.size() && g.stat_names[j] != r.name) j++;
            if (j == g.stat_names.size()) {
                g.stat_names.emplace_back(r.name);
                g.stat_count.push_back(0);
                g.stat_ms.push_back(0.0);
            }
            g.stat_count[j]++;
            g.stat_ms[j] += ms;
        }
        g.stats_dirty = false;
    }
    if (i < 0 || i >= (int)g.stat_names.size()) return -1;
    if (name && name_len) {
        strncpy(name, g.stat_names[i].c_str(), name_len - 1);
        name[name_len - 1] = 0;
    }
    if (count) *count = g.stat_count[i];
    if (total_ms) *total_ms = g.stat_ms[i];
    return 0;
}

extern "C" int ds3_hip_timer_start(void)
{
    if (refuse_in_capture("timer_start") || !ensure_init()) return -1;
    return report(hipEventRecord(g.t0, g.stream), "timer_start");
}

extern "C" double ds3_hip_timer_stop_ms(void)
{
    if (!g.inited || refuse_in_capture("timer_stop_ms")) return -1.0;
    (void)hipEventRecord(g.t1, g.stream);
    (void)hipEventSynchronize(g.t1);
    float ms = 0.f;
    (void)hipEventElapsedTime(&ms, g.t0, g.t1);
    return ms;
}

extern "C" int ds3_hip_hold_stream(double us)
{
    if (refuse_in_capture("hold_stream") || !ensure_init()) return -1;
    return report(ds3k::launch_hold(us, g.stream), "hold_stream");
}

extern "C" int ds3_hip_device_info(char *arch, size_t arch_len, int *n_cu, uint64_t *hbm_bytes)
{
    if (refuse_in_capture("device_info") || !ensure_init()) return -1;
    hipDeviceProp_t p;
    if (hipGetDeviceProperties(&p, 0) != hipSuccess) return -1;
    if (arch && arch_len) {
        strncpy(arch, p.gcnArchName, arch_len - 1);
        arch[arch_len - 1] = 0;
    }
    if (n_cu) *n_cu = p.multiProcessorCount;
    if (hbm_bytes) *hbm_bytes = p.totalGlobalMem;
    return 0;
}
