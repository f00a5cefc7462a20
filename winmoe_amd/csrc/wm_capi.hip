// wm_capi.hip -- the extern "C" surface of libwinmoe_hip.so (include/winmoe_hip.h):
// argument validation, the fixed workspace layout, stream-ordered
// orchestration of the expert kernels, and the gpu_* shims of
// engine/runtime/gpu_offload.h.  Host code only.
#include <hip/hip_runtime.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <algorithm>
#include <mutex>
#include <vector>

#include "../../include/winmoe_hip.h"
#include "wm_decode.h"
#include "wm_host.h"
#include "wm_launch.h"
#include "wm_prefill.h"
#include "wm_quant.h"
#include "wm_wave.h"

using namespace wm;

static inline hipStream_t S(void* s) { return (hipStream_t)s; }
static inline bool al(const void* p, uintptr_t a) { return ((uintptr_t)p % a) == 0; }
static inline int64_t up256(int64_t v) { return (v + 255) & ~(int64_t)255; }

static bool g_dev_ready = false;

// ------------------------------------------------------------------ phase profiler
namespace {
enum Phase { PH_ROUTER = 0, PH_TOPK, PH_SHGATE, PH_GATEUP, PH_SWIGLU, PH_DOWN, PH_COMBINE, PH_STEP };
const char* kPhaseNames[WM_PROF_NPHASE] = {"router_logits", "topk", "shared_gate", "gate_up_swiglu",
                                           "swiglu", "down", "combine", "step"};
struct Prof {
    bool on = false;
    std::vector<hipEvent_t> pool;                 // free events
    std::vector<std::pair<int, std::pair<hipEvent_t, hipEvent_t>>> pending;
    double ms[WM_PROF_NPHASE] = {0};
    int64_t cnt[WM_PROF_NPHASE] = {0};
};
Prof P;

hipEvent_t prof_event() {
    if (!P.pool.empty()) {
        hipEvent_t e = P.pool.back();
        P.pool.pop_back();
        return e;
    }
    hipEvent_t e = nullptr;
    if (hipEventCreate(&e) != hipSuccess) return nullptr;
    return e;
}

// Brackets one phase on stream s when profiling is on.
struct PhaseTimer {
    int ph;
    hipStream_t s;
    hipEvent_t a = nullptr, b = nullptr;
    PhaseTimer(int phase, hipStream_t st) : ph(phase), s(st) {
        if (!P.on) return;
        a = prof_event();
        b = prof_event();
        if (a && b) (void)hipEventRecord(a, s);
    }
    ~PhaseTimer() {
        if (!a || !b) return;
        (void)hipEventRecord(b, s);
        P.pending.push_back({ph, {a, b}});
    }
};
}  // namespace

extern "C" int wm_profile_enable(int on) {
    P.on = on != 0;
    return WM_OK;
}

extern "C" int wm_profile_read(double* ms, int64_t* count, int nphase) {
    WM_CHECK_ARG(nphase >= 0 && nphase <= WM_PROF_NPHASE);
    for (auto& p : P.pending) {
        float t = 0.0f;
        WM_FAIL_HIP(hipEventSynchronize(p.second.second));
        WM_FAIL_HIP(hipEventElapsedTime(&t, p.second.first, p.second.second));
        P.ms[p.first] += t;
        P.cnt[p.first] += 1;
        P.pool.push_back(p.second.first);
        P.pool.push_back(p.second.second);
    }
    P.pending.clear();
    for (int i = 0; i < nphase; i++) {
        if (ms) ms[i] = P.ms[i];
        if (count) count[i] = P.cnt[i];
        P.ms[i] = 0.0;
        P.cnt[i] = 0;
    }
    return WM_OK;
}

extern "C" const char* wm_profile_phase_name(int phase) {
    return (phase >= 0 && phase < WM_PROF_NPHASE) ? kPhaseNames[phase] : "";
}

extern "C" int wm_init(void) {
    if (g_dev_ready) return WM_OK;
    int n = 0;
    WM_FAIL_HIP(hipGetDeviceCount(&n));
    if (n <= 0) {
        fprintf(stderr, "winmoe_hip: no HIP device\n");
        return WM_ERR;
    }
    g_dev_ready = true;
    return WM_OK;
}

extern "C" const char* wm_version(void) { return "winmoe_hip 0.1 (gfx950)"; }
extern "C" int wm_block_bytes(int t) { return block_bytes(t); }
extern "C" int wm_block_elems(int t) { return block_elems(t); }

// ------------------------------------------------------------------ simple entry points

extern "C" int wm_dequant(int t, const void* blocks, int64_t nblocks, float* out, void* stream) {
    WM_CHECK_ARG(supported(t));
    WM_CHECK_ARG(nblocks >= 0);
    if (nblocks == 0) return WM_OK;
    WM_CHECK_ARG(blocks && out && al(blocks, 4) && al(out, 4));
    if (wm_init()) return WM_ERR;
    WM_FAIL_HIP(launch_dequant(t, blocks, nblocks, out, S(stream)));
    return WM_OK;
}

extern "C" int wm_quantize(int t, const float* x, int64_t n, void* blocks, void* stream) {
    WM_CHECK_ARG(supported(t));
    WM_CHECK_ARG(n >= 0 && n % block_elems(t) == 0);
    if (n == 0) return WM_OK;
    WM_CHECK_ARG(x && blocks);
    if (wm_init()) return WM_ERR;
    WM_FAIL_HIP(launch_quantize(t, x, n / block_elems(t), blocks, S(stream)));
    return WM_OK;
}

extern "C" int wm_quantize_host(int t, const float* x, int64_t n, void* blocks) {
    WM_CHECK_ARG(supported(t));
    WM_CHECK_ARG(n >= 0 && n % block_elems(t) == 0);
    WM_CHECK_ARG(n == 0 || (x && blocks));
    int64_t nb = n / block_elems(t);
    for (int64_t b = 0; b < nb; b++)
        quant_block(t, x + b * block_elems(t), (uint8_t*)blocks + b * block_bytes(t));
    return WM_OK;
}

static int check_matrix(int t, const void* W, int in) {
    if (!gemv_shape_ok(t, in)) {
        fprintf(stderr, "winmoe_hip: unsupported matrix shape: type %d, in %d (in must be 64..4096, a power-of-two "
                        "multiple of 64 and of the block size)\n", t, in);
        return WM_EINVAL;
    }
    if (!al(W, 16)) {
        fprintf(stderr, "winmoe_hip: expert tensor base must be 16-byte aligned\n");
        return WM_EINVAL;
    }
    return WM_OK;
}

static int64_t xop_bytes(int in) { return (int64_t)(in / SEG) * XOP_DW * 4; }

// Input vectors are read as b128 vectors: one that is not 16-byte aligned is
// first copied to an aligned workspace buffer of at least n floats.
static int aligned_input(const float*& x, int64_t n, float* scratch, hipStream_t s) {
    if (al(x, 16)) return WM_OK;
    WM_FAIL_HIP(hipMemcpyAsync(scratch, x, (size_t)n * 4, hipMemcpyDeviceToDevice, s));
    x = scratch;
    return WM_OK;
}

extern "C" int wm_quant_matvec(int t, const void* W, const float* x, int rows, int in, float* y, void* ws,
                               int64_t ws_bytes, void* stream) {
    WM_CHECK_ARG(supported(t) && W && x && y && rows >= 0);
    if (int rc = check_matrix(t, W, in)) return rc;
    WM_CHECK_ARG(ws && al(ws, 256) && ws_bytes >= xop_bytes(in));
    if (rows == 0) return WM_OK;
    if (wm_init()) return WM_ERR;
    hipStream_t s = S(stream);
    if (int rc = aligned_input(x, in, (float*)ws, s)) return rc;
    GemvArgs g = {};
    g.m = MatSet{(const uint8_t*)W, 0, nullptr, 1, 1, nullptr};
    g.slot0 = 0;
    g.rows = rows;
    g.in = in;
    g.x = x;
    g.y = y;
    WM_FAIL_HIP(launch_gemv(t, g, 1, s));
    return WM_OK;
}

extern "C" int64_t wm_router_workspace_size(int E) { return E > 0 ? up256((int64_t)E * 4) + 256 : WM_EINVAL; }

extern "C" int wm_router_logits(const float* x, const float* W, int H, int E, float* logits, void* stream) {
    WM_CHECK_ARG(x && W && logits && H > 0 && E > 0);
    WM_CHECK_ARG(router_rows_per_wg(H, false) > 0);
    if (wm_init()) return WM_ERR;
    WM_FAIL_HIP(launch_router_logits(x, W, H, E, logits, S(stream)));
    return WM_OK;
}

extern "C" int wm_router_topk(const float* x, const float* W, int H, int E, int K, int32_t* ids, float* w, void* ws,
                              int64_t ws_bytes, void* stream) {
    WM_CHECK_ARG(x && W && ids && w && H > 0 && E > 0 && E <= 1024 && K >= 1 && K <= 16 && K <= E);
    WM_CHECK_ARG(router_rows_per_wg(H, false) > 0);
    WM_CHECK_ARG(ws && al(ws, 256) && ws_bytes >= wm_router_workspace_size(E));
    if (wm_init()) return WM_ERR;
    hipStream_t s = S(stream);
    float* logits = (float*)ws;
    int32_t* status = (int32_t*)((uint8_t*)ws + up256((int64_t)E * 4));
    WM_FAIL_HIP(launch_router_logits(x, W, H, E, logits, s));
    WM_FAIL_HIP(launch_topk(logits, E, K, ids, w, nullptr, status, s));
    return WM_OK;
}

// ------------------------------------------------------------------ layer descriptor + workspace

struct WsLayout {
    int64_t status, ctr, logits, tr_ids, tr_w, hits, shgate, xin, gbuf, ubuf, act, ypart, tlog, hello, pctr, tact,
        tx, timeline, total;
    int K1, Imax, Is;
};

static int Ishared(const wm_layer_desc* d) { return d->inter_shared > 0 ? d->inter_shared : d->inter; }
static bool has_shared(const wm_layer_desc* d) { return d->sh_gate && d->sh_up && d->sh_down; }

static int validate_desc(const wm_layer_desc* d, bool need_router) {
    WM_CHECK_ARG(d);
    WM_CHECK_ARG(d->hidden > 0 && d->inter > 0 && d->n_experts > 0 && d->n_experts <= 1024);
    WM_CHECK_ARG(d->top_k >= 1 && d->top_k <= 16 && d->top_k <= d->n_experts);
    WM_CHECK_ARG(d->gate_exps && d->up_exps && d->down_exps);
    if (int rc = check_matrix(d->gate_type, d->gate_exps, d->hidden)) return rc;
    if (int rc = check_matrix(d->up_type, d->up_exps, d->hidden)) return rc;
    if (int rc = check_matrix(d->down_type, d->down_exps, d->inter)) return rc;
    WM_CHECK_ARG(d->gate_stride >= 0 && d->up_stride >= 0 && d->down_stride >= 0);
    WM_CHECK_ARG(d->gate_stride % 16 == 0 && d->up_stride % 16 == 0 && d->down_stride % 16 == 0);
    if (need_router) {
        WM_CHECK_ARG(d->router != nullptr);
        WM_CHECK_ARG(router_rows_per_wg(d->hidden, false) > 0);
    }
    if (has_shared(d)) {
        int Is = Ishared(d);
        if (int rc = check_matrix(d->sh_gate_type, d->sh_gate, d->hidden)) return rc;
        if (int rc = check_matrix(d->sh_up_type, d->sh_up, d->hidden)) return rc;
        if (int rc = check_matrix(d->sh_down_type, d->sh_down, Is)) return rc;
    } else {
        WM_CHECK_ARG(!d->sh_gate && !d->sh_up && !d->sh_down);
    }
    return WM_OK;
}

static WsLayout layout(const wm_layer_desc* d, int max_tokens) {
    WsLayout L;
    int K = d->top_k, E = d->n_experts, H = d->hidden;
    L.K1 = K + 1;
    L.Is = Ishared(d);
    L.Imax = std::max(d->inter, L.Is);
    int64_t o = 0;
    L.status = o; o += 256;
    L.ctr = o; o += (int64_t)C_TOTAL * CTR_STRIDE * 4;
    L.logits = o; o += up256((int64_t)E * 4);
    L.tr_ids = o; o += up256((int64_t)max_tokens * K * 4);
    L.tr_w = o; o += up256((int64_t)max_tokens * K * 4);
    L.hits = o; o += up256((int64_t)E * 4);
    L.shgate = o; o += 256;
    L.xin = o; o += up256((int64_t)H * 4);
    L.gbuf = o; o += up256((int64_t)L.K1 * L.Imax * 4);
    L.ubuf = o; o += up256((int64_t)L.K1 * L.Imax * 4);
    L.act = o; o += up256((int64_t)L.K1 * L.Imax * 4);
    L.ypart = o; o += up256((int64_t)L.K1 * H * 4);
    // persistent step: tagged logits, per-workgroup start tags, epoch line,
    // tagged SwiGLU outputs
    L.tlog = o; o += up256((int64_t)P_REP * E * 8);
    L.hello = o; o += up256((int64_t)P_MAX_WG * 4);
    L.pctr = o; o += (int64_t)CTR_STRIDE * 4;
    L.tact = o; o += up256((int64_t)L.K1 * P_AREP * ((L.Imax + 1) / 2) * 8);
    // the layer's output as tagged words for the next layer of a chained launch
    L.tx = o; o += up256((int64_t)P_XREP * H * 8);
    L.timeline = o;
    if (d->flags & WM_FLAG_TIMELINE) o += up256((int64_t)TIMELINE_CAP * 8 * 8);
    L.total = o;
    return L;
}

extern "C" int64_t wm_workspace_size(const wm_layer_desc* d, int max_tokens) {
    if (!d || max_tokens <= 0 || d->top_k <= 0 || d->n_experts <= 0 || d->hidden <= 0 || d->inter <= 0) return WM_EINVAL;
    return layout(d, max_tokens).total;
}

extern "C" int wm_workspace_trace(const wm_layer_desc* d, int max_tokens, int64_t* ids_off, int64_t* w_off,
                                  int64_t* hits_off) {
    WM_CHECK_ARG(d && max_tokens > 0 && d->top_k > 0 && d->n_experts > 0);
    WsLayout L = layout(d, max_tokens);
    if (ids_off) *ids_off = L.tr_ids;
    if (w_off) *w_off = L.tr_w;
    if (hits_off) *hits_off = L.hits;
    return WM_OK;
}

extern "C" int wm_workspace_reset(const wm_layer_desc* d, int max_tokens, void* ws, int64_t ws_bytes, void* stream) {
    WM_CHECK_ARG(d && ws && max_tokens > 0 && al(ws, 256));
    int64_t total = wm_workspace_size(d, max_tokens);
    WM_CHECK_ARG(total > 0 && ws_bytes >= total);
    if (wm_init()) return WM_ERR;
    WM_FAIL_HIP(launch_fill_i32((int32_t*)ws, 0, total / 4, S(stream)));
    return WM_OK;
}

extern "C" int wm_workspace_timeline(const wm_layer_desc* d, int max_tokens, int64_t* offset, int64_t* capacity) {
    WM_CHECK_ARG(d && max_tokens > 0 && d->top_k > 0 && d->n_experts > 0 && (d->flags & WM_FLAG_TIMELINE));
    WsLayout L = layout(d, max_tokens);
    if (offset) *offset = L.timeline;
    if (capacity) *capacity = TIMELINE_CAP;
    return WM_OK;
}

extern "C" int64_t wm_device_clock_khz(void) {
    if (wm_init()) return WM_ERR;
    int dev = 0, khz = 0;
    WM_FAIL_HIP(hipGetDevice(&dev));
    WM_FAIL_HIP(hipDeviceGetAttribute(&khz, hipDeviceAttributeWallClockRate, dev));
    return khz;
}

extern "C" int wm_workspace_status(void* ws, int64_t ws_bytes, int32_t* status_out) {
    WM_CHECK_ARG(ws && status_out && ws_bytes >= 4);
    if (wm_init()) return WM_ERR;
    WM_FAIL_HIP(hipDeviceSynchronize());
    WM_FAIL_HIP(hipMemcpy(status_out, ws, 4, hipMemcpyDeviceToHost));
    return WM_OK;
}

// The expert part of one decode token, given routing already in the trace
// entry (ids_d / w_d): gate/up + SwiGLU, down, combine.
static int run_experts(const wm_layer_desc* d, const WsLayout& L, uint8_t* ws, const float* x, const int32_t* ids_d,
                       const float* w_d, float* out, hipStream_t s) {
    const int H = d->hidden, I = d->inter, K = d->top_k, E = d->n_experts, Is = L.Is;
    const bool sh = has_shared(d);
    int32_t* status = (int32_t*)(ws + L.status);
    float* act = (float*)(ws + L.act);
    float* gbuf = (float*)(ws + L.gbuf);
    float* ubuf = (float*)(ws + L.ubuf);
    float* ypart = (float*)(ws + L.ypart);
    const int64_t act_stride = L.Imax;
    if (int rc = aligned_input(x, H, (float*)(ws + L.xin), s)) return rc;
    if (sh && d->sh_gate_inp) {
        PhaseTimer pt(PH_SHGATE, s);
        WM_FAIL_HIP(launch_shgate(x, d->sh_gate_inp, H, (float*)(ws + L.shgate), s));
    }

    MatSet mg = {(const uint8_t*)d->gate_exps, d->gate_stride ? d->gate_stride : matrix_bytes(d->gate_type, I, H),
                 ids_d, K, E, (const uint8_t*)d->sh_gate};
    MatSet mu = {(const uint8_t*)d->up_exps, d->up_stride ? d->up_stride : matrix_bytes(d->up_type, I, H), ids_d, K,
                 E, (const uint8_t*)d->sh_up};
    MatSet md = {(const uint8_t*)d->down_exps, d->down_stride ? d->down_stride : matrix_bytes(d->down_type, H, I),
                 ids_d, K, E, (const uint8_t*)d->sh_down};

    // gate/up (+ SwiGLU) for slots [slot0, slot0 + nslots): one fused launch
    // when gate and up share a type, else two GEMVs and an elementwise SwiGLU
    auto gate_up = [&](int slot0, int nslots, int gt, int ut, int rows) -> int {
        if (gt == ut) {
            GateUpArgs a = {};
            a.gate = mg; a.up = mu;
            a.slot0 = slot0; a.rows = rows; a.in = H;
            a.x = x;
            a.act = act; a.act_slot_stride = act_stride; a.status = status;
            return launch_gateup(gt, a, nslots, s);
        }
        GemvArgs a = {};
        a.slot0 = slot0; a.rows = rows; a.in = H; a.status = status;
        a.m = mg; a.x = x; a.y = gbuf; a.y_slot_stride = act_stride;
        if (int e = launch_gemv(gt, a, nslots, s)) return e;
        a.m = mu; a.y = ubuf;
        if (int e = launch_gemv(ut, a, nslots, s)) return e;
        PhaseTimer pt(PH_SWIGLU, s);
        return launch_swiglu(gbuf + slot0 * act_stride, ubuf + slot0 * act_stride, act + slot0 * act_stride, rows,
                             nslots, act_stride, s);
    };
    auto down = [&](int slot0, int nslots, int dt, int in) -> int {
        GemvArgs a = {};
        a.m = md; a.slot0 = slot0; a.rows = H; a.in = in; a.status = status;
        a.x = act; a.x_slot_stride = act_stride; a.y = ypart; a.y_slot_stride = H;
        return launch_gemv(dt, a, nslots, s);
    };

    const bool merge = sh && d->sh_gate_type == d->gate_type && d->sh_up_type == d->up_type &&
                       d->sh_down_type == d->down_type && Is == I;
    const int n_main = merge ? K + 1 : K;
    {
        PhaseTimer pt(PH_GATEUP, s);
        WM_FAIL_HIP(gate_up(0, n_main, d->gate_type, d->up_type, I));
        if (sh && !merge) WM_FAIL_HIP(gate_up(K, 1, d->sh_gate_type, d->sh_up_type, Is));
    }
    {
        PhaseTimer pt(PH_DOWN, s);
        WM_FAIL_HIP(down(0, n_main, d->down_type, I));
        if (sh && !merge) WM_FAIL_HIP(down(K, 1, d->sh_down_type, Is));
    }

    CombineArgs c = {};
    c.ypart = ypart; c.y_stride = H; c.w = w_d; c.ids = ids_d; c.K = K; c.E = E; c.H = H;
    c.has_shared = sh ? 1 : 0;
    c.sh_gate = (sh && d->sh_gate_inp) ? (const float*)(ws + L.shgate) : nullptr;
    c.out = out;
    PhaseTimer pt(PH_COMBINE, s);
    WM_FAIL_HIP(launch_combine(c, s));
    return WM_OK;
}

static int rpt_of(int t, int in) { return geometry(t, in).rpt; }

// CUs of the current device (cached per device).
static int cu_count() {
    static int cached[64] = {0};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
    if (!cached[dev]) {
        int cus = 0;
        if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0) cus = 256;
        cached[dev] = cus;
    }
    return cached[dev];
}

// Workgroups of the fused step resident on the current device at once: two
// per CU (each holds a 64 KB LDS ring set).
static int resident_slots() { return 2 * cu_count(); }

// Dynamic LDS one workgroup may use on the current device (cached per device).
static int max_lds_per_wg() {
    static int cached[64] = {0};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 65536;
    if (!cached[dev]) {
        // the opt-in limit (what hipFuncAttributeMaxDynamicSharedMemorySize may
        // raise a kernel to: 160 KB on gfx950), else the default per-block limit
        int v = 0, opt = 0;
        if (hipDeviceGetAttribute(&v, hipDeviceAttributeMaxSharedMemoryPerBlock, dev) != hipSuccess || v <= 0) v = 65536;
        if (hipDeviceGetAttribute(&opt, hipDeviceAttributeSharedMemPerBlockOptin, dev) == hipSuccess && opt > v) v = opt;
        cached[dev] = v;
    }
    return cached[dev];
}

// Persistent launches on different streams must not overlap: each needs one
// workgroup on every CU at once, and two sharing the CUs would each wait for
// workgroups that cannot start.  Per device, the stream of the last
// persistent launch.  While every launch comes on one stream, stream order
// is enough and nothing is added.  The first launch on a second stream waits
// for the device to drain once (no other stream's handle is touched: it may
// be gone); from then on an event is recorded after every persistent launch
// and a launch on another stream than the last waits for it on the device.
struct PersistOrder {
    hipStream_t last = nullptr;
    bool used = false, multi = false, recorded = false;
    hipEvent_t ev = nullptr;
};
static std::mutex g_persist_mu;
static PersistOrder g_persist_order[64];

static bool capturing(hipStream_t s) {
    hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
    return hipStreamIsCapturing(s, &cap) == hipSuccess && cap != hipStreamCaptureStatusNone;
}

// The current device's ordering event, created ahead of time so that no
// later launch has to create it (wm_moe_decode_noalloc's set-up calls this).
int wm::persist_order_prepare() {
    int dev = 0;
    WM_FAIL_HIP(hipGetDevice(&dev));
    if (dev < 0 || dev >= 64) return WM_OK;
    std::lock_guard<std::mutex> lock(g_persist_mu);
    PersistOrder& po = g_persist_order[dev];
    if (!po.ev) WM_FAIL_HIP(hipEventCreateWithFlags(&po.ev, hipEventDisableTiming));
    return WM_OK;
}

// Launches `launch` on s after the last persistent launch of another stream.
template <typename F> static int persistent_ordered(hipStream_t s, F&& launch) {
    int dev = 0;
    WM_FAIL_HIP(hipGetDevice(&dev));
    if (dev < 0 || dev >= 64 || capturing(s)) return launch();
    std::lock_guard<std::mutex> lock(g_persist_mu);
    PersistOrder& po = g_persist_order[dev];
    if (po.used && po.last != s) {
        if (!po.multi) {
            if (!po.ev) WM_FAIL_HIP(hipEventCreateWithFlags(&po.ev, hipEventDisableTiming));
            WM_FAIL_HIP(hipDeviceSynchronize());
            po.multi = true;
        } else if (po.recorded) {
            WM_FAIL_HIP(hipStreamWaitEvent(s, po.ev, 0));
        }
    }
    if (int rc = launch()) return rc;
    if (po.multi) {
        WM_FAIL_HIP(hipEventRecord(po.ev, s));
        po.recorded = true;
    }
    po.last = s;
    po.used = true;
    return WM_OK;
}

// One launch of the persistent step kernel (wm_persist.hip); returns 1 when
// the layer does not fit it (the caller then uses the work-item-list kernel).
// prep_persist fills the kernel's arguments, LDS bytes and instance types
// (stage: a layer of a chained launch that takes its input from the previous
// layer, which needs LDS for the staged tagged input).
struct PersistPlan {
    PersistArgs a;
    int lds;
    int gut, dt, sgut, sdt;
};
static int prep_persist(const wm_layer_desc* d, const WsLayout& L, uint8_t* ws, const float* x, float* out,
                        const int32_t* forced_ids, const float* forced_w, int32_t* ids, float* w, bool stage,
                        hipStream_t s, PersistPlan& plan) {
    const bool sh = has_shared(d);
    if (d->gate_type != d->up_type || (sh && d->sh_gate_type != d->sh_up_type)) return 1;
    const int gut = d->gate_type, dt = d->down_type;
    const int sgut = sh ? d->sh_gate_type : gut, sdt = sh ? d->sh_down_type : dt;
    if (!persist_supported(gut, dt, sgut, sdt)) return 1;
    const int H = d->hidden, I = d->inter, K = d->top_k, E = d->n_experts;
    const bool forced = forced_ids != nullptr;
    if (sh && L.Is != I) return 1;
    if (!gemv_shape_ok(gut, H) || !gemv_shape_ok(sgut, H) || !gemv_shape_ok(dt, I) || !gemv_shape_ok(sdt, I)) return 1;
    if (!forced && !al(d->router, 16)) return 1;
    const int nwg = cu_count();
    if (nwg > P_MAX_WG) return 1;
    const int rr = forced ? 0 : (E + nwg - 1) / nwg;
    if (rr > 4) return 1;
    PersistArgs a = {};
    a.H = H; a.I = I; a.E = E; a.K = K; a.has_shared = sh ? 1 : 0; a.forced = forced ? 1 : 0;
    a.nwg = nwg; a.rr = rr;
    const int rpt_gu = rpt_of(gut, H), rpt_dn = rpt_of(dt, I);
    a.gu_tiles = (I + rpt_gu - 1) / rpt_gu;
    a.dn_tiles = (H + rpt_dn - 1) / rpt_dn;
    // a hand-off word carries two SwiGLU outputs, so a workgroup's gate/up
    // rows come in pairs: one-row tiles are split in units of two
    a.gu_step = rpt_gu == 1 ? 2 : 1;
    if (a.gu_tiles % a.gu_step || (rpt_gu * a.gu_step) % 2) return 1;
    a.gu_cap = (a.gu_tiles / a.gu_step + nwg - 1) / nwg * a.gu_step * rpt_gu;
    a.y_cap = (a.dn_tiles + nwg - 1) / nwg * rpt_dn;
    a.ring_buf = std::max(std::max(ring_tile_bytes_rt(gut), ring_tile_bytes_rt(dt)),
                          std::max(ring_tile_bytes_rt(sgut), ring_tile_bytes_rt(sdt)));
    // LDS: control block | SwiGLU operand records | x operand records |
    // gate/up row sums | down row sums | tile descriptors | the streaming
    // waves' buffers | x and the router rows (or those in the first buffers)
    int o = (int)((sizeof(PersistCtl) + 255) / 256 * 256);
    a.x_region = (H * 4 + 1023) / 1024 * 1024;
    // x (normalised in place when the layer has an RMSNorm), then the router rows
    const int router_bytes = (1 + (forced ? 0 : rr)) * a.x_region;
    a.n_rwaves = (router_bytes + PRING * a.ring_buf - 1) / (PRING * a.ring_buf);
    const int rec = XOP_DW * 4;
    a.o_reg = o; o += (K + 1) * (I / SEG) * rec;
    a.o_xop = o; o += (H / SEG) * rec;
    a.o_xop2 = a.o_xop;
    if (sh && sgut != gut) { a.o_xop2 = o; o += (H / SEG) * rec; }
    // the RMSNorm weights share the operand records' space: they are read
    // before x is in, and every record is written after that
    a.o_norm = a.o_reg;
    if (d->norm_w) o = std::max(o, a.o_norm + a.x_region);
    a.o_gu = o; o += 2 * (K + 1) * a.gu_cap * 4;
    a.o_y = o; o += (K + 1) * a.y_cap * 4;
    // act tiles: the SwiGLU outputs of a slot come into the streaming waves'
    // buffers in tiles of aseg 64-value segments (4 B per value: two to a
    // tagged 8-byte word; whole K-quant super-blocks, so every tile is a
    // contiguous column range).  One wave builds a tile's records, 8
    // segments at a time: with few slots a slot's down tiles wait for them,
    // and 8-segment tiles let two waves share a slot; with many, the act
    // tiles run well ahead and 16-segment tiles halve their number.
    a.aseg = (K + (sh ? 1 : 0) >= 8 && a.ring_buf >= 16 * SEG * 4) ? 16 : 8;
    a.nact = (I / SEG + a.aseg - 1) / a.aseg;
    if (a.nact > PMAXACT || a.aseg * SEG * 4 > a.ring_buf) return 1;
    // the tile list's descriptor table, 16 bytes an entry, for the longest
    // list of any workgroup: per slot 2 * (gate/up tiles) + act tiles + down tiles
    {
        const int gu_units = a.gu_tiles / a.gu_step;
        const int ngu_max = a.gu_step * ((gu_units + nwg - 1) / nwg), ndn_max = (a.dn_tiles + nwg - 1) / nwg;
        a.n_desc = (K + (sh ? 1 : 0)) * (2 * ngu_max + a.nact + ndn_max);
        a.o_desc = o;
        o += a.n_desc * 16;
    }
    o = (o + 255) / 256 * 256;
    // the streaming waves' rings take what is left, up to PW of them; x and
    // the router rows get a region of their own when it fits, else they sit
    // in the first rings until the router helpers are done with them
    a.o_ring = o;
    a.nstream = std::min(PW, (max_lds_per_wg() - o) / (PRING * a.ring_buf));
    a.o_router = o;
    if (o + a.nstream * PRING * a.ring_buf + router_bytes <= max_lds_per_wg()) {
        a.o_router = o + a.nstream * PRING * a.ring_buf;
        o += router_bytes;
        a.n_rwaves = 0;
    }
    // a chained layer's input: the previous layer's tagged words (8 bytes a
    // value, whole kilobytes) after the router region, which must have its
    // own space
    a.o_stage = 0;
    if (stage) {
        const int st = (H * 8 + 1023) / 1024 * 1024;
        if (a.n_rwaves || a.o_router + router_bytes + st > max_lds_per_wg()) return 1;
        a.o_stage = a.o_router + router_bytes;
        o += st;
    }
    if (a.nstream < a.n_rwaves + 1 || a.nstream < 4) return 1;
    // (and more than half of a CU's LDS, so that each CU holds one workgroup)
    const int lds = std::max((o + a.nstream * PRING * a.ring_buf + 255) / 256 * 256,
                             (max_lds_per_wg() / 2 + 256) / 256 * 256);
    if (d->norm_w && !al(d->norm_w, 16)) return 1;      // (its weights are read as 16-byte vectors)
    if (int rc = aligned_input(x, H, (float*)(ws + L.xin), s)) return rc;
    a.x = x; a.out = out; a.router = d->router;
    a.norm_w = d->norm_w; a.norm_eps = d->norm_eps; a.add_res = d->norm_w && d->add_residual ? 1 : 0;
    a.gate = (const uint8_t*)d->gate_exps; a.up = (const uint8_t*)d->up_exps; a.down = (const uint8_t*)d->down_exps;
    a.gstride = d->gate_stride ? d->gate_stride : matrix_bytes(gut, I, H);
    a.ustride = d->up_stride ? d->up_stride : matrix_bytes(gut, I, H);
    a.dstride = d->down_stride ? d->down_stride : matrix_bytes(dt, H, I);
    a.sh_gate = (const uint8_t*)d->sh_gate; a.sh_up = (const uint8_t*)d->sh_up; a.sh_down = (const uint8_t*)d->sh_down;
    a.sh_gate_inp = sh ? d->sh_gate_inp : nullptr;
    a.forced_ids = forced_ids; a.forced_w = forced_w;
    a.ids = ids; a.w = w;
    a.hits = (uint32_t*)(ws + L.hits); a.status = (int32_t*)(ws + L.status);
    a.tlogits = (uint64_t*)(ws + L.tlog);
    a.hello = (uint32_t*)(ws + L.hello);
    a.epoch = (uint32_t*)(ws + L.pctr);
    a.tact = (uint64_t*)(ws + L.tact);
    if (d->flags & WM_FLAG_TIMELINE) a.timeline = (uint64_t*)(ws + L.timeline);
    a.probe = (d->flags & WM_FLAG_SPIN_PROBE) ? 1u : 0u;
    plan.a = a;
    plan.lds = lds;
    plan.gut = gut; plan.dt = dt; plan.sgut = sgut; plan.sdt = sdt;
    return WM_OK;
}

static int run_persist(const wm_layer_desc* d, const WsLayout& L, uint8_t* ws, const float* x, float* out,
                       const int32_t* forced_ids, const float* forced_w, int32_t* ids, float* w, hipStream_t s) {
    PersistPlan plan;
    if (int rc = prep_persist(d, L, ws, x, out, forced_ids, forced_w, ids, w, false, s, plan)) return rc;
    PhaseTimer pt(PH_STEP, s);
    return persistent_ordered(s, [&]() -> int {
        WM_FAIL_HIP(launch_persist(plan.a, (size_t)plan.lds, plan.gut, plan.dt, plan.sgut, plan.sdt, s));
        return WM_OK;
    });
}

// One launch of the fused step kernel; returns 1 when the type combination has
// no fused instantiation (the caller then runs the per-phase kernels).
static int run_fused(const wm_layer_desc* d, const WsLayout& L, uint8_t* ws, const float* x, float* out,
                     const int32_t* forced_ids, const float* forced_w, int32_t* ids, float* w, hipStream_t s) {
    if (!(d->flags & WM_FLAG_ITEM_KERNEL)) {
        const int rc = run_persist(d, L, ws, x, out, forced_ids, forced_w, ids, w, s);
        if (rc <= 0) return rc;
    }
    const bool sh = has_shared(d);
    if (d->gate_type != d->up_type || (sh && d->sh_gate_type != d->sh_up_type)) return 1;
    const int gut = d->gate_type, dt = d->down_type;
    const int sgut = sh ? d->sh_gate_type : gut, sdt = sh ? d->sh_down_type : dt;
    if (!decode_step_supported(gut, dt, sgut, sdt)) return 1;
    const int H = d->hidden, I = d->inter, Is = L.Is, K = d->top_k, E = d->n_experts;
    DecodeArgs a = {};
    a.H = H; a.I = I; a.Is = Is; a.E = E; a.K = K; a.has_shared = sh ? 1 : 0;
    a.forced = forced_ids ? 1 : 0;
    if (int rc = aligned_input(x, H, (float*)(ws + L.xin), s)) return rc;
    {
        const bool aligned = (H % 4 == 0) && al(x, 16) && al(d->router, 16);
        // two rows per item: with the shared gate/up items the router
        // items fill the device at the start
        a.rr = std::min(2, router_rows_per_wg(H, aligned));
        a.router_region = router_region(H, aligned);
        if (a.rr <= 0) return 1;
    }
    a.x = x; a.out = out; a.router = d->router;
    a.gate = (const uint8_t*)d->gate_exps; a.up = (const uint8_t*)d->up_exps; a.down = (const uint8_t*)d->down_exps;
    a.gstride = d->gate_stride ? d->gate_stride : matrix_bytes(gut, I, H);
    a.ustride = d->up_stride ? d->up_stride : matrix_bytes(gut, I, H);
    a.dstride = d->down_stride ? d->down_stride : matrix_bytes(dt, H, I);
    a.sh_gate = (const uint8_t*)d->sh_gate; a.sh_up = (const uint8_t*)d->sh_up; a.sh_down = (const uint8_t*)d->sh_down;
    a.sh_gate_inp = sh ? d->sh_gate_inp : nullptr;
    a.forced_ids = forced_ids; a.forced_w = forced_w;
    a.logits = (float*)(ws + L.logits); a.ids = ids; a.w = w;
    a.hits = (uint32_t*)(ws + L.hits); a.status = (int32_t*)(ws + L.status);
    a.act = (float*)(ws + L.act); a.act_stride = L.Imax;
    a.ypart = (float*)(ws + L.ypart); a.shgate = (float*)(ws + L.shgate); a.ctr = (uint32_t*)(ws + L.ctr);
    // Work split.  The device holds `slots` decode-step workgroups at once
    // (2 per CU by LDS); items are sized so that each phase fits one wave of
    // them: the shared gate/up next to the router items, all routed gate/up
    // items together, all down items together.  Gate/up items are 2 x tpw
    // tiles of gate and of up (at most GU_ROWS_MAX rows); down items are
    // rows_dn_item rows, a whole number of tiles per wave for the routed and
    // the shared down type alike.
    const int slots = resident_slots();
    const int rpt_gu = rpt_of(gut, H);
    auto gu_tpw = [&](int rows, int items) {
        const int per = (rows + std::max(items, 1) - 1) / std::max(items, 1);
        return std::max(1, std::min((per + 2 * rpt_gu - 1) / (2 * rpt_gu), GU_ROWS_MAX / (2 * rpt_gu)));
    };
    int unit = WAVES * rpt_of(dt, I);
    if (sh) unit = std::max(unit, WAVES * rpt_of(sdt, Is));      // powers of two: the max is the lcm
    const int K1 = K + (sh ? 1 : 0);
    const int ranges_want = std::max(1, slots / K1);
    int rows_dn = ((H + ranges_want - 1) / ranges_want + unit - 1) / unit * unit;
    while ((H + rows_dn - 1) / rows_dn > C_MAX_RANGES) rows_dn *= 2;
    a.rows_dn_item = rows_dn;
    a.n_dn_slot = (H + rows_dn - 1) / rows_dn;
    a.n_router = a.forced ? 0 : (E + a.rr - 1) / a.rr;
    a.tpw_sgu = sh ? gu_tpw(Is, slots - 1 - a.n_router) : 1;
    a.n_sgu = sh ? (Is + 2 * a.tpw_sgu * rpt_gu - 1) / (2 * a.tpw_sgu * rpt_gu) : 0;
    a.tpw_gu = gu_tpw(I, (slots - (sh ? a.n_dn_slot : 0)) / K);
    a.n_gu_slot = (I + 2 * a.tpw_gu * rpt_gu - 1) / (2 * a.tpw_gu * rpt_gu);
    a.it_router = 1;
    a.n_rgroups = (a.n_router + RGROUP - 1) / RGROUP;
    if (a.n_rgroups > C_MAX_RGROUPS) return 1;
    // Item order: routers, routed gate/up, shared gate/up, shared down, routed
    // down.  The routed gate/up items that get a workgroup slot at launch only
    // wait for the routing, so the router's rows have the memory system to
    // themselves; the shared expert's items take the slots the routers free
    // and stream while the routing completes.
    a.it_gu = a.it_router + a.n_router;
    a.it_sgu = a.it_gu + K * a.n_gu_slot;
    a.it_sdn = a.it_sgu + a.n_sgu;
    a.it_dn = a.it_sdn + (sh ? a.n_dn_slot : 0);
    a.n_items = a.it_dn + K * a.n_dn_slot;
    if (d->flags & WM_FLAG_TIMELINE) {
        a.timeline = (uint64_t*)(ws + L.timeline);
        a.timeline_cap = TIMELINE_CAP;
    }
    PhaseTimer pt(PH_STEP, s);
    WM_FAIL_HIP(launch_decode_step(a, gut, dt, sgut, sdt, s));
    return WM_OK;
}

extern "C" int wm_moe_decode(const wm_layer_desc* d, const float* x, float* out, void* ws, int64_t ws_bytes,
                             int max_tokens, int step, void* stream) {
    if (int rc = validate_desc(d, true)) return rc;
    WM_CHECK_ARG(x && out && ws && al(ws, 256) && max_tokens > 0 && step >= 0);
    WsLayout L = layout(d, max_tokens);
    WM_CHECK_ARG(ws_bytes >= L.total);
    if (wm_init()) return WM_ERR;
    hipStream_t s = S(stream);
    uint8_t* w8 = (uint8_t*)ws;
    int slot = step % max_tokens;
    int32_t* ids = (int32_t*)(w8 + L.tr_ids) + (int64_t)slot * d->top_k;
    float* wts = (float*)(w8 + L.tr_w) + (int64_t)slot * d->top_k;
    float* logits = (float*)(w8 + L.logits);
    if (d->norm_w) {      // RMSNorm in, residual out: the persistent kernel only
        WM_CHECK_ARG(!(d->flags & (WM_FLAG_MULTI_KERNEL | WM_FLAG_ITEM_KERNEL)));
        const int rc = run_persist(d, L, w8, x, out, nullptr, nullptr, ids, wts, s);
        return rc == 1 ? WM_EINVAL : rc;
    }
    WM_CHECK_ARG(!d->add_residual);
    if (!(d->flags & WM_FLAG_MULTI_KERNEL)) {
        int rc = run_fused(d, L, w8, x, out, nullptr, nullptr, ids, wts, s);
        if (rc <= 0) return rc;
    }
    PhaseTimer step_timer(PH_STEP, s);
    {
        PhaseTimer pt(PH_ROUTER, s);
        WM_FAIL_HIP(launch_router_logits(x, d->router, d->hidden, d->n_experts, logits, s));
    }
    {
        PhaseTimer pt(PH_TOPK, s);
        WM_FAIL_HIP(launch_topk(logits, d->n_experts, d->top_k, ids, wts, (uint32_t*)(w8 + L.hits),
                                (int32_t*)(w8 + L.status), s));
    }
    return run_experts(d, L, w8, x, ids, wts, out, s);
}

extern "C" int wm_moe_decode_forced(const wm_layer_desc* d, const float* x, const int32_t* ids_in, const float* w_in,
                                    float* out, void* ws, int64_t ws_bytes, int max_tokens, int step, void* stream) {
    if (int rc = validate_desc(d, false)) return rc;
    WM_CHECK_ARG(x && out && ids_in && w_in && ws && al(ws, 256) && max_tokens > 0 && step >= 0);
    WsLayout L = layout(d, max_tokens);
    WM_CHECK_ARG(ws_bytes >= L.total);
    if (wm_init()) return WM_ERR;
    hipStream_t s = S(stream);
    uint8_t* w8 = (uint8_t*)ws;
    int slot = step % max_tokens;
    int32_t* ids = (int32_t*)(w8 + L.tr_ids) + (int64_t)slot * d->top_k;
    float* wts = (float*)(w8 + L.tr_w) + (int64_t)slot * d->top_k;
    if (d->norm_w) {      // RMSNorm in, residual out: the persistent kernel only
        WM_CHECK_ARG(!(d->flags & (WM_FLAG_MULTI_KERNEL | WM_FLAG_ITEM_KERNEL)));
        const int rc = run_persist(d, L, w8, x, out, ids_in, w_in, ids, wts, s);
        return rc == 1 ? WM_EINVAL : rc;
    }
    WM_CHECK_ARG(!d->add_residual);
    if (!(d->flags & WM_FLAG_MULTI_KERNEL)) {
        int rc = run_fused(d, L, w8, x, out, ids_in, w_in, ids, wts, s);
        if (rc <= 0) return rc;
    }
    PhaseTimer step_timer(PH_STEP, s);
    WM_FAIL_HIP(hipMemcpyAsync(ids, ids_in, (size_t)d->top_k * 4, hipMemcpyDeviceToDevice, s));
    WM_FAIL_HIP(hipMemcpyAsync(wts, w_in, (size_t)d->top_k * 4, hipMemcpyDeviceToDevice, s));
    WM_FAIL_HIP(launch_count_hits(ids, d->top_k, d->n_experts, (uint32_t*)(w8 + L.hits), (int32_t*)(w8 + L.status), s));
    return run_experts(d, L, w8, x, ids, wts, out, s);
}

extern "C" int wm_moe_decode_stack(int n_layers, const wm_layer_desc* const* d, void* const* ws, const int64_t* ws_bytes,
                                   const float* x, float* out, const int32_t* const* ids_in, const float* const* w_in,
                                   int max_tokens, int step, void* stream) {
    WM_CHECK_ARG(n_layers >= 1 && d && ws && ws_bytes && x && out && max_tokens > 0 && step >= 0);
    WM_CHECK_ARG(!ids_in == !w_in);
    for (int l = 0; l < n_layers; l++) {
        const bool forced = ids_in && ids_in[l];
        if (int rc = validate_desc(d[l], !forced)) return rc;
        WM_CHECK_ARG(!forced || w_in[l]);
        WM_CHECK_ARG(ws[l] && al(ws[l], 256) && ws_bytes[l] >= layout(d[l], max_tokens).total);
        WM_CHECK_ARG(d[l]->hidden == d[0]->hidden);
        WM_CHECK_ARG(!d[l]->add_residual || d[l]->norm_w);
    }
    if (wm_init()) return WM_ERR;
    hipStream_t s = S(stream);
    const int H = d[0]->hidden;
    const int slot = step % max_tokens;
    // one layer the usual way (input xl, output ol)
    auto one = [&](int l, const float* xl, float* ol) -> int {
        const bool forced = ids_in && ids_in[l];
        return forced ? wm_moe_decode_forced(d[l], xl, ids_in[l], w_in[l], ol, ws[l], ws_bytes[l], max_tokens, step, stream)
                      : wm_moe_decode(d[l], xl, ol, ws[l], ws_bytes[l], max_tokens, step, stream);
    };
    const float* xin = x;
    for (int l0 = 0; l0 < n_layers;) {
        const int cnt = std::min(P_STACK, n_layers - l0);
        StackArgs sa = {};
        int lds = 0, gut = 0, dt = 0, sgut = 0, sdt = 0;
        bool ok = cnt > 1;
        for (int k = 0; ok && k < cnt; k++) {
            const int l = l0 + k;
            const wm_layer_desc* dl = d[l];
            if (dl->flags & (WM_FLAG_MULTI_KERNEL | WM_FLAG_ITEM_KERNEL)) { ok = false; break; }
            // layers of one launch need workspaces of their own (each holds
            // the layer's launch tag and tagged hand-off words); layers that
            // share one run one launch each, in order
            for (int q = l0; ok && q < l; q++) {
                const uint8_t *a0 = (const uint8_t*)ws[q], *b0 = (const uint8_t*)ws[l];
                if (a0 < b0 + ws_bytes[l] && b0 < a0 + ws_bytes[q]) ok = false;
            }
            if (!ok) break;
            const WsLayout L = layout(dl, max_tokens);
            uint8_t* w8 = (uint8_t*)ws[l];
            int32_t* tid = (int32_t*)(w8 + L.tr_ids) + (int64_t)slot * dl->top_k;
            float* tw = (float*)(w8 + L.tr_w) + (int64_t)slot * dl->top_k;
            const bool forced = ids_in && ids_in[l];
            PersistPlan plan;
            const int rc = prep_persist(dl, L, w8, k == 0 ? xin : out + (int64_t)(l - 1) * H, out + (int64_t)l * H,
                                        forced ? ids_in[l] : nullptr, forced ? w_in[l] : nullptr, tid, tw, k > 0, s, plan);
            if (rc < 0) return rc;
            if (rc > 0) { ok = false; break; }
            if (k == 0) {
                gut = plan.gut; dt = plan.dt; sgut = plan.sgut; sdt = plan.sdt;
                if (!stack_supported(gut, dt, sgut, sdt)) { ok = false; break; }
            } else if (plan.gut != gut || plan.dt != dt || plan.sgut != sgut || plan.sdt != sdt ||
                       plan.a.nwg != sa.L[0].nwg) {
                ok = false;
                break;
            }
            plan.a.tx_out = k + 1 < cnt ? (uint64_t*)(w8 + L.tx) : nullptr;
            plan.a.tx_in = k > 0 ? sa.L[k - 1].tx_out : nullptr;
            sa.L[k] = plan.a;
            lds = std::max(lds, plan.lds);
        }
        if (ok) {
            sa.n = cnt;
            PhaseTimer pt(PH_STEP, s);
            const int rc = persistent_ordered(s, [&]() -> int {
                WM_FAIL_HIP(launch_stack(sa, (size_t)lds, gut, dt, sgut, sdt, s));
                return WM_OK;
            });
            if (rc) return rc;
        } else {
            for (int k = 0; k < cnt; k++) {
                const int l = l0 + k;
                if (int rc = one(l, k == 0 ? xin : out + (int64_t)(l - 1) * H, out + (int64_t)l * H)) return rc;
            }
        }
        xin = out + (int64_t)(l0 + cnt - 1) * H;
        l0 += cnt;
    }
    return WM_OK;
}

extern "C" int64_t wm_expert_workspace_size(int H, int I) {
    if (H <= 0 || I <= 0) return WM_EINVAL;
    return 256 + 2 * up256(xop_bytes(H)) + 3 * up256((int64_t)I * 4) + up256(xop_bytes(I));
}

extern "C" int wm_expert_ffn(const void* gate, int gt, const void* up, int ut, const void* down, int dt, const float* x,
                             int H, int I, float* out, void* ws, int64_t ws_bytes, void* stream) {
    WM_CHECK_ARG(gate && up && down && x && out && ws && al(ws, 256));
    if (int rc = check_matrix(gt, gate, H)) return rc;
    if (int rc = check_matrix(ut, up, H)) return rc;
    if (int rc = check_matrix(dt, down, I)) return rc;
    WM_CHECK_ARG(ws_bytes >= wm_expert_workspace_size(H, I));
    if (wm_init()) return WM_ERR;
    hipStream_t s = S(stream);
    uint8_t* w8 = (uint8_t*)ws;
    int32_t* status = (int32_t*)w8;
    int64_t o = 256;
    float* xin = (float*)(w8 + o); o += 2 * up256(xop_bytes(H));
    float* gb = (float*)(w8 + o); o += up256((int64_t)I * 4);
    float* ub = (float*)(w8 + o); o += up256((int64_t)I * 4);
    float* act = (float*)(w8 + o);
    if (int rc = aligned_input(x, H, xin, s)) return rc;
    MatSet mg = {(const uint8_t*)gate, 0, nullptr, 1, 1, nullptr};
    MatSet mu = {(const uint8_t*)up, 0, nullptr, 1, 1, nullptr};
    MatSet md = {(const uint8_t*)down, 0, nullptr, 1, 1, nullptr};
    if (gt == ut) {
        GateUpArgs a = {};
        a.gate = mg; a.up = mu; a.rows = I; a.in = H; a.x = x; a.act = act; a.status = status;
        WM_FAIL_HIP(launch_gateup(gt, a, 1, s));
    } else {
        GemvArgs a = {};
        a.m = mg; a.rows = I; a.in = H; a.x = x; a.y = gb; a.status = status;
        WM_FAIL_HIP(launch_gemv(gt, a, 1, s));
        a.m = mu; a.y = ub;
        WM_FAIL_HIP(launch_gemv(ut, a, 1, s));
        WM_FAIL_HIP(launch_swiglu(gb, ub, act, I, 1, 0, s));
    }
    GemvArgs dn = {};
    dn.m = md; dn.rows = H; dn.in = I; dn.x = act; dn.y = out; dn.status = status;
    WM_FAIL_HIP(launch_gemv(dt, dn, 1, s));
    return WM_OK;
}

// ------------------------------------------------------------------ prefill

struct PfLayout {
    int64_t status, ids, w, logits, hits, offsets, sorted, passes, pass_count, sg, x16, xexp, act_hi, act_lo, act_sc, y,
        total;
    int64_t act_stride;
};

static PfLayout pf_layout(const wm_layer_desc* d, int max_tokens) {
    PfLayout L = {};
    const int64_t T = max_tokens, K = d->top_k, E = d->n_experts, H = d->hidden;
    const bool sh = has_shared(d);
    const int64_t Imax = std::max<int64_t>(d->inter, sh ? Ishared(d) : 0);
    const int64_t pairs = T * K + (sh ? T : 0);
    int64_t o = 0;
    L.status = o; o += 256;
    L.ids = o; o += up256(T * K * 4);
    L.w = o; o += up256(T * K * 4);
    L.logits = o; o += up256(T * E * 4);
    L.hits = o; o += up256(E * 4);
    L.offsets = o; o += up256((E + 2) * 4);
    L.sorted = o; o += up256(pairs * 4);
    L.passes = o; o += up256(prefill_max_passes(T, K, E) * 256);
    L.pass_count = o; o += 256;
    L.sg = o; o += up256(T * 4);
    L.x16 = o; o += up256(T * H * 2);
    L.xexp = o; o += up256(T * 4);
    L.act_stride = (Imax + 255) / 256 * 256;
    L.act_hi = o; o += up256(pairs * L.act_stride * 2);
    L.act_lo = o; o += up256(pairs * L.act_stride * 2);
    L.act_sc = o; o += up256(pairs * (L.act_stride / 128) * 4);
    L.y = o; o += up256(pairs * H * 4);
    L.total = o;
    return L;
}

extern "C" int64_t wm_prefill_workspace_size(const wm_layer_desc* d, int max_tokens) {
    if (!d || max_tokens <= 0 || d->top_k <= 0 || d->n_experts <= 0 || d->hidden <= 0 || d->inter <= 0) return WM_EINVAL;
    return pf_layout(d, max_tokens).total;
}

extern "C" int wm_prefill_workspace_routing(const wm_layer_desc* d, int max_tokens, int64_t* ids_off, int64_t* w_off,
                                            int64_t* hits_off) {
    WM_CHECK_ARG(d && max_tokens > 0 && d->top_k > 0 && d->n_experts > 0);
    PfLayout L = pf_layout(d, max_tokens);
    if (ids_off) *ids_off = L.ids;
    if (w_off) *w_off = L.w;
    if (hits_off) *hits_off = L.hits;
    return WM_OK;
}

static int run_prefill(const wm_layer_desc* d, const uint16_t* x, int T, const int32_t* fids, const float* fw,
                       float* out, void* ws, int64_t ws_bytes, int max_tokens, void* stream) {
    if (int rc = validate_desc(d, fids == nullptr)) return rc;
    WM_CHECK_ARG(!d->norm_w && !d->add_residual);     // the fused RMSNorm is a decode-step feature
    WM_CHECK_ARG(x && out && ws && al(ws, 256) && al(x, 16) && al(out, 16) && T > 0 && T <= max_tokens);
    PfLayout L = pf_layout(d, max_tokens);
    WM_CHECK_ARG(ws_bytes >= L.total);
    const bool sh = has_shared(d);
    const bool types = d->gate_type == d->up_type && prefill_type(d->gate_type) && prefill_type(d->down_type) &&
                       (!sh || (d->sh_gate_type == d->sh_up_type && prefill_type(d->sh_gate_type) &&
                                prefill_type(d->sh_down_type)));
    const bool shapes = d->hidden % 256 == 0 && d->inter % 256 == 0 && (!sh || Ishared(d) % 256 == 0);
    if (!types || !shapes) {
        fprintf(stderr, "winmoe_hip: prefill needs quantised expert matrices (Q8_0, Q2_K .. Q6_K) with gate and up "
                        "of one format, and H, I multiples of 256\n");
        return WM_EINVAL;
    }
    if (wm_init()) return WM_ERR;
    hipStream_t s = S(stream);
    uint8_t* w8 = (uint8_t*)ws;
    PrefillArgs a = {};
    a.H = d->hidden; a.I = d->inter; a.Is = Ishared(d); a.E = d->n_experts; a.K = d->top_k; a.T = T;
    a.has_shared = sh ? 1 : 0;
    a.gt = d->gate_type; a.dt = d->down_type;
    a.sgt = sh ? d->sh_gate_type : a.gt; a.sdt = sh ? d->sh_down_type : a.dt;
    a.x = x; a.router = d->router;
    a.gate = (const uint8_t*)d->gate_exps; a.up = (const uint8_t*)d->up_exps; a.down = (const uint8_t*)d->down_exps;
    a.gstride = d->gate_stride ? d->gate_stride : matrix_bytes(d->gate_type, d->inter, d->hidden);
    a.ustride = d->up_stride ? d->up_stride : matrix_bytes(d->up_type, d->inter, d->hidden);
    a.dstride = d->down_stride ? d->down_stride : matrix_bytes(d->down_type, d->hidden, d->inter);
    a.sh_gate = (const uint8_t*)d->sh_gate; a.sh_up = (const uint8_t*)d->sh_up; a.sh_down = (const uint8_t*)d->sh_down;
    a.sh_gate_inp = sh ? d->sh_gate_inp : nullptr;
    a.ids = (int32_t*)(w8 + L.ids); a.w = (float*)(w8 + L.w); a.logits = (float*)(w8 + L.logits);
    a.hits = (uint32_t*)(w8 + L.hits); a.status = (int32_t*)(w8 + L.status);
    a.offsets = (int32_t*)(w8 + L.offsets); a.sorted = (int32_t*)(w8 + L.sorted); a.sg = (float*)(w8 + L.sg);
    a.passes = (int32_t*)(w8 + L.passes); a.pass_count = (int32_t*)(w8 + L.pass_count);
    a.x16 = (uint16_t*)(w8 + L.x16); a.xexp = (int32_t*)(w8 + L.xexp);
    a.act_hi = (uint16_t*)(w8 + L.act_hi); a.act_lo = (uint16_t*)(w8 + L.act_lo); a.act_sc = (float*)(w8 + L.act_sc);
    a.act_stride = L.act_stride; a.y = (float*)(w8 + L.y); a.out = out;
    a.n_wg = cu_count();
    WM_CHECK_ARG((d->flags & (WM_FLAG_PREFILL_PASS16 | WM_FLAG_PREFILL_PASS32)) !=
                 (WM_FLAG_PREFILL_PASS16 | WM_FLAG_PREFILL_PASS32));
    a.pass_m = (d->flags & WM_FLAG_PREFILL_PASS16)   ? 16
               : (d->flags & WM_FLAG_PREFILL_PASS32) ? 32
                                                     : prefill_pass_size(T, a.K, a.E, a.gt);
    // the expert GEMMs read 16-byte granules from row starts
    WM_CHECK_ARG(al(a.gate, 16) && al(a.up, 16) && al(a.down, 16) && a.gstride % 16 == 0 && a.ustride % 16 == 0 &&
                 a.dstride % 16 == 0 && (!sh || (al(a.sh_gate, 16) && al(a.sh_up, 16) && al(a.sh_down, 16))));
    PhaseTimer step_timer(PH_STEP, s);
    {
        PhaseTimer pt(PH_ROUTER, s);
        WM_FAIL_HIP(launch_prefill_route(a, fids, fw, s));
    }
    {
        PhaseTimer pt(PH_GATEUP, s);
        WM_FAIL_HIP(launch_prefill_gateup(a, s));
    }
    {
        PhaseTimer pt(PH_DOWN, s);
        WM_FAIL_HIP(launch_prefill_down(a, s));
    }
    PhaseTimer pt(PH_COMBINE, s);
    WM_FAIL_HIP(launch_prefill_combine(a, s));
    return WM_OK;
}

extern "C" int wm_moe_prefill(const wm_layer_desc* d, const uint16_t* x_bf16, int T, float* out, void* ws,
                              int64_t ws_bytes, int max_tokens, void* stream) {
    return run_prefill(d, x_bf16, T, nullptr, nullptr, out, ws, ws_bytes, max_tokens, stream);
}

extern "C" int wm_moe_prefill_forced(const wm_layer_desc* d, const uint16_t* x_bf16, int T, const int32_t* ids,
                                     const float* w, float* out, void* ws, int64_t ws_bytes, int max_tokens,
                                     void* stream) {
    WM_CHECK_ARG(ids && w);
    return run_prefill(d, x_bf16, T, ids, w, out, ws, ws_bytes, max_tokens, stream);
}
