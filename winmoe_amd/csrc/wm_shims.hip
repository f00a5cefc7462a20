// wm_shims.hip -- the expert subset of the reference's GPU offload ABI
// (engine/runtime/gpu_offload.h:15-100) on top of libwinmoe_hip's device API.
// Host code only.
//
// What a caller of the reference sees is kept: the function names and
// argument meaning, 0 / -1 returns (-1 also for "not cached" and "refused"),
// caller-owned host buffers, every call that returns data blocking until it
// is in the caller's buffer, a bounded table of cached experts addressed by
// slot number with an O(1) (layer, expert) lookup, round-robin recycling of
// slots once the table is full, and refusal of an expert that would pass the
// memory budget.
//
// What is built differently: a cached expert is one HBM allocation holding
// its [gate | up | down] blocks back to back (the expert slot layout of
// winmoe_inference.c:1764-1786), each part starting on a 256-byte boundary;
// any supported quant type may back a part (recorded by
// gpu_cache_expert_typed, or inferred from the byte count); the budget is a
// fraction of this device's HBM and counts the bytes a recycled slot gives
// back; the arithmetic is the library's own expert kernels.
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdio.h>

#include <algorithm>
#include <vector>

#include "../../include/winmoe_hip.h"
#include "wm_format.h"
#include "wm_host.h"
#include "wm_launch.h"
#include "wm_wave.h"

using namespace wm;

namespace {

// (layer, expert) ids a cached expert may carry: the lookup table the
// reference allocates on first use covers 80 layers x 1024 experts
// (gpu_offload.cu:596-601); ids outside it are refused.
constexpr int kIdLayers = 80, kIdExperts = 1024;
// Initial table capacity: the reference's MAX_GPU_EXPERTS (gpu_offload.cu:540).
constexpr int kDefaultCapacity = 300;
// Largest capacity gpu_set_expert_limit accepts here.  The reference caps it
// at 300 because of an 8 GB card; 288 GB of HBM holds tens of thousands of
// experts of the supported shapes.
constexpr int kCapacityCeiling = 16384;
// Router tables uploaded by gpu_upload_router (one per layer below this).
constexpr int kRouterLayers = 64;
// Share of the device's HBM the shims may fill with cached experts and routers.
constexpr double kBudgetShare = 0.9;

struct CachedExpert {
    int layer = -1, expert = -1;
    uint8_t* mem = nullptr;              // [gate | up | down]
    int64_t off[3] = {0, 0, 0};          // byte offset of each part in mem
    int bytes[3] = {0, 0, 0};
    int qtype[3] = {-1, -1, -1};         // ggml type, -1: inferred from bytes when used
    int64_t footprint() const { return mem ? off[2] + bytes[2] : 0; }
    const void* part(int k) const { return mem + off[k]; }
};

// Quant type of part k (rows x in weights) of a cached expert: the recorded
// one, else the supported type whose packing of that shape has exactly the
// part's byte count (bytes per weight differ for every supported type).
int part_type(const CachedExpert& ce, int k, int rows, int in) {
    if (ce.qtype[k] >= 0) return ce.qtype[k];
    for (int t : {Q8_0, Q2_K, Q3_K, Q4_K, Q5_K, Q6_K})
        if (in % block_elems(t) == 0 && matrix_bytes(t, rows, in) == (int64_t)ce.bytes[k]) return t;
    return -1;
}

class ExpertTable {
  public:
    void open(int64_t budget) {
        slots_.clear();
        where_.assign((size_t)kIdLayers * kIdExperts, -1);
        capacity_ = kDefaultCapacity;
        cursor_ = 0;
        held_ = 0;
        budget_ = budget;
        budget_noted_ = false;
    }
    // Every slot's memory back to the device (the caller has drained the stream).
    void close() {
        for (CachedExpert& ce : slots_)
            if (ce.mem) (void)hipFree(ce.mem);
        slots_.clear();
        where_.clear();
        held_ = 0;
    }
    int count() const { return (int)slots_.size(); }
    int64_t held() const { return held_; }

    int find(int layer, int expert) const {
        if (!valid_id(layer, expert) || where_.empty()) return -1;
        return where_[(size_t)layer * kIdExperts + expert];
    }
    const CachedExpert* get(int slot) const {
        if (slot < 0 || slot >= count() || !slots_[slot].mem) return nullptr;
        return &slots_[slot];
    }
    // The recycling cursor is left as it is: as in gpu_offload.cu:582-623,
    // the next recycle of a full table takes the slot under it (which may lie
    // past a lowered capacity) and only then wraps it modulo the capacity.
    void set_capacity(int n) {
        capacity_ = std::min(std::max(n, 1), kCapacityCeiling);
        fprintf(stderr, "winmoe_hip: expert table capacity now %d slots (ceiling %d)\n", capacity_,
                kCapacityCeiling);
    }

    // Copies one expert's three parts into a slot; returns the slot, or -1
    // when the ids are out of range, an input is empty, the budget would be
    // passed or HIP fails.  A full table recycles the slot under the cursor.
    int admit(int layer, int expert, const void* const src[3], const int bytes[3], const int qtype[3],
              hipStream_t s) {
        if (!valid_id(layer, expert)) return -1;
        for (int k = 0; k < 3; k++)
            if (!src[k] || bytes[k] <= 0) return -1;
        int64_t off[3];
        off[0] = 0;
        off[1] = round_up256(bytes[0]);
        off[2] = off[1] + round_up256(bytes[1]);
        const int64_t need = off[2] + bytes[2];
        const bool grow = count() < capacity_;
        const int slot = grow ? count() : cursor_;
        const int64_t returned = grow ? 0 : slots_[slot].footprint();
        if (held_ - returned + need > budget_) {
            if (!budget_noted_) {
                fprintf(stderr,
                        "winmoe_hip: not caching expert %d of layer %d: %.1f MiB would bring the expert table to "
                        "%.1f MiB, over its budget of %.1f MiB (reported once)\n",
                        expert, layer, need / 1048576.0, (held_ - returned + need) / 1048576.0, budget_ / 1048576.0);
                budget_noted_ = true;
            }
            return -1;
        }
        if (grow) {
            slots_.emplace_back();
        } else {
            cursor_ = (cursor_ + 1) % capacity_;
            if (hipStreamSynchronize(s) != hipSuccess) return -1;   // kernels may still read the old bytes
            recycle(slot);
        }
        CachedExpert& ce = slots_[slot];
        if (hipMalloc((void**)&ce.mem, (size_t)need) != hipSuccess) {
            ce = CachedExpert();
            fprintf(stderr, "winmoe_hip: hipMalloc of %lld bytes for an expert slot failed\n", (long long)need);
            return -1;
        }
        for (int k = 0; k < 3; k++)
            if (hipMemcpyAsync(ce.mem + off[k], src[k], (size_t)bytes[k], hipMemcpyHostToDevice, s) != hipSuccess) {
                (void)hipStreamSynchronize(s);
                recycle(slot);
                return -1;
            }
        if (hipStreamSynchronize(s) != hipSuccess) return -1;      // the caller may reuse its buffers now
        for (int k = 0; k < 3; k++) {
            ce.off[k] = off[k];
            ce.bytes[k] = bytes[k];
            ce.qtype[k] = qtype[k];
        }
        ce.layer = layer;
        ce.expert = expert;
        where_[(size_t)layer * kIdExperts + expert] = slot;
        held_ += need;
        return slot;
    }

  private:
    static bool valid_id(int layer, int expert) {
        return layer >= 0 && expert >= 0 && layer < kIdLayers && expert < kIdExperts;
    }
    // Empties a slot: its lookup entry (if it still points here) and memory.
    void recycle(int slot) {
        CachedExpert& ce = slots_[slot];
        if (ce.layer >= 0) {
            int32_t& w = where_[(size_t)ce.layer * kIdExperts + ce.expert];
            if (w == slot) w = -1;
        }
        held_ -= ce.footprint();
        if (ce.mem) (void)hipFree(ce.mem);
        ce = CachedExpert();
    }

    std::vector<CachedExpert> slots_;
    std::vector<int32_t> where_;     // [layer][expert] -> slot or -1
    int capacity_ = kDefaultCapacity;
    int cursor_ = 0;                 // the slot a full table recycles next
    int64_t held_ = 0, budget_ = 0;
    bool budget_noted_ = false;
};

// Device side of the shims: one stream, the expert kernels' workspace, a
// staging area of four float vectors (input, output, gate, up), the batch
// accumulator and the uploaded routers.
struct ShimDevice {
    bool ready = false;
    hipStream_t stream = nullptr;
    ExpertTable experts;
    void* ws = nullptr;
    int64_t ws_bytes = 0;
    float* io = nullptr;             // 4 vectors of io_len floats
    int64_t io_len = 0;
    bool batch_open = false;         // io's input vector holds a batch's x
    float* acc = nullptr;            // batch accumulator
    int acc_len = 0;
    float* router[kRouterLayers] = {};
    int router_h[kRouterLayers] = {}, router_e[kRouterLayers] = {};
    int64_t router_bytes = 0;

    enum { IN = 0, OUT = 1, GATE = 2, UP = 3 };
    float* vec(int which) { return io + which * io_len; }

    // Workspace and staging for an expert of hidden H and intermediate I.
    // The staging vectors are at least 16384 floats and only grow outside a
    // batch (a batch's uploaded x must survive every batch_add).
    int reserve(int H, int I) {
        const int64_t need_ws = wm_expert_workspace_size(H, I);
        if (need_ws < 0) return WM_EINVAL;
        if (need_ws > ws_bytes) {
            if (ws) (void)hipFree(ws);
            ws = nullptr;
            ws_bytes = 0;
            WM_FAIL_HIP(hipMalloc(&ws, (size_t)need_ws));
            ws_bytes = need_ws;
        }
        const int64_t len = round_up256(std::max<int64_t>(std::max(H, I), 16384));
        if (len > io_len) {
            if (batch_open) return WM_EINVAL;
            if (io) (void)hipFree(io);
            io = nullptr;
            io_len = 0;
            WM_FAIL_HIP(hipMalloc((void**)&io, (size_t)(4 * len) * sizeof(float)));
            io_len = len;
        }
        return WM_OK;
    }
    void release() {
        if (stream) (void)hipStreamSynchronize(stream);
        experts.close();
        for (float*& r : router)
            if (r) { (void)hipFree(r); r = nullptr; }
        if (ws) (void)hipFree(ws);
        if (io) (void)hipFree(io);
        if (acc) (void)hipFree(acc);
        if (stream) (void)hipStreamDestroy(stream);
        *this = ShimDevice();
    }
};
ShimDevice D;

// Runs the cached expert on the staged input (vec(IN), H floats) into dst (H floats).
int run_cached(const CachedExpert& ce, int H, int I, float* dst) {
    const int gt = part_type(ce, 0, I, H), ut = part_type(ce, 1, I, H), dt = part_type(ce, 2, H, I);
    if (gt < 0 || ut < 0 || dt < 0) {
        fprintf(stderr, "winmoe_hip: cached expert's byte counts fit no supported type at hidden %d, intermediate %d\n",
                H, I);
        return -1;
    }
    return wm_expert_ffn(ce.part(0), gt, ce.part(1), ut, ce.part(2), dt, D.vec(ShimDevice::IN), H, I, dst, D.ws,
                         D.ws_bytes, D.stream) == WM_OK ? 0 : -1;
}

int cache_one(int layer, int expert, const void* g, int gb, int gt, const void* u, int ub, int ut, const void* dn,
              int db, int dt) {
    if (!D.ready && gpu_init()) return -1;
    const void* src[3] = {g, u, dn};
    const int bytes[3] = {gb, ub, db}, types[3] = {gt, ut, dt};
    return D.experts.admit(layer, expert, src, bytes, types, D.stream);
}

}  // namespace

// ------------------------------------------------------------------ lifecycle

extern "C" int gpu_init(void) {
    if (D.ready) return 0;
    if (wm_init() != WM_OK) return -1;
    WM_FAIL_HIP(hipStreamCreateWithFlags(&D.stream, hipStreamNonBlocking));
    size_t free_b = 0, total_b = 0;
    WM_FAIL_HIP(hipMemGetInfo(&free_b, &total_b));
    D.experts.open((int64_t)(kBudgetShare * (double)total_b));
    D.ready = true;
    return 0;
}

extern "C" void gpu_shutdown(void) {
    if (D.ready) D.release();
}

extern "C" int gpu_is_initialized(void) { return D.ready ? 1 : 0; }

extern "C" float gpu_vram_used_mb(void) {
    return (float)((double)(D.experts.held() + D.router_bytes) / (1024.0 * 1024.0));
}

extern "C" int gpu_expert_cache_count(void) { return D.experts.count(); }

extern "C" void gpu_set_expert_limit(int limit) { D.experts.set_capacity(limit); }

// ------------------------------------------------------------------ router

extern "C" int gpu_upload_router(int layer, const float* weights, int hidden_dim, int num_experts) {
    if (!D.ready && gpu_init()) return -1;
    if (layer < 0 || layer >= kRouterLayers || !weights || hidden_dim <= 0 || num_experts <= 0) return -1;
    const size_t bytes = (size_t)hidden_dim * (size_t)num_experts * sizeof(float);
    if (D.router[layer]) {
        (void)hipStreamSynchronize(D.stream);
        (void)hipFree(D.router[layer]);
        D.router_bytes -= (int64_t)D.router_h[layer] * D.router_e[layer] * 4;
        D.router[layer] = nullptr;
    }
    if (hipMalloc((void**)&D.router[layer], bytes) != hipSuccess) return -1;
    if (hipMemcpy(D.router[layer], weights, bytes, hipMemcpyHostToDevice) != hipSuccess) return -1;
    D.router_h[layer] = hidden_dim;
    D.router_e[layer] = num_experts;
    D.router_bytes += (int64_t)bytes;
    return 0;
}

extern "C" int gpu_router(int layer, const float* normed, int hidden_dim, float* logits_out, int num_experts) {
    if (!D.ready || layer < 0 || layer >= kRouterLayers || !D.router[layer] || !normed || !logits_out) return -1;
    if (D.router_h[layer] != hidden_dim || D.router_e[layer] != num_experts) return -1;
    if (router_rows_per_wg(hidden_dim, false) <= 0) return -1;
    if (D.reserve(hidden_dim, std::max(num_experts, 64)) != WM_OK) return -1;
    float* dx = D.vec(ShimDevice::IN);
    float* dl = D.vec(ShimDevice::OUT);
    WM_FAIL_HIP(hipMemcpyAsync(dx, normed, (size_t)hidden_dim * sizeof(float), hipMemcpyHostToDevice, D.stream));
    WM_FAIL_HIP(launch_router_logits(dx, D.router[layer], hidden_dim, num_experts, dl, D.stream));
    WM_FAIL_HIP(hipMemcpyAsync(logits_out, dl, (size_t)num_experts * sizeof(float), hipMemcpyDeviceToHost, D.stream));
    WM_FAIL_HIP(hipStreamSynchronize(D.stream));
    return 0;
}

// ------------------------------------------------------------------ expert table

extern "C" int gpu_cache_expert(int layer, int expert_id, const void* gate_data, int gate_size, const void* up_data,
                                int up_size, const void* down_data, int down_size) {
    return cache_one(layer, expert_id, gate_data, gate_size, -1, up_data, up_size, -1, down_data, down_size, -1);
}

extern "C" int gpu_cache_expert_typed(int layer, int expert_id, const void* gate_data, int gate_size, int gate_type,
                                      const void* up_data, int up_size, int up_type, const void* down_data,
                                      int down_size, int down_type) {
    if (!supported(gate_type) || !supported(up_type) || !supported(down_type)) return -1;
    return cache_one(layer, expert_id, gate_data, gate_size, gate_type, up_data, up_size, up_type, down_data,
                     down_size, down_type);
}

extern "C" int gpu_find_cached_expert(int layer, int expert_id) {
    return D.ready ? D.experts.find(layer, expert_id) : -1;
}

// ------------------------------------------------------------------ expert compute (blocking, host buffers)

extern "C" int gpu_expert_ffn_fused(int cache_idx, const float* input, int hidden_dim, int intermediate,
                                    float* expert_out) {
    const CachedExpert* ce = D.ready ? D.experts.get(cache_idx) : nullptr;
    if (!ce || !input || !expert_out) return -1;
    if (D.reserve(hidden_dim, intermediate) != WM_OK) return -1;
    WM_FAIL_HIP(hipMemcpyAsync(D.vec(ShimDevice::IN), input, (size_t)hidden_dim * sizeof(float),
                               hipMemcpyHostToDevice, D.stream));
    if (run_cached(*ce, hidden_dim, intermediate, D.vec(ShimDevice::OUT))) return -1;
    WM_FAIL_HIP(hipMemcpyAsync(expert_out, D.vec(ShimDevice::OUT), (size_t)hidden_dim * sizeof(float),
                               hipMemcpyDeviceToHost, D.stream));
    WM_FAIL_HIP(hipStreamSynchronize(D.stream));
    return 0;
}

// Gate and up projections (before SwiGLU) to the host; expert_out is left
// alone and the type arguments are not used (the slot knows its types), as
// in gpu_offload.cu:675-698.
extern "C" int gpu_expert_ffn(int cache_idx, const float* input, int hidden_dim, int intermediate, float* gate_out,
                              float* up_out, float* expert_out, int gate_type, int down_type) {
    (void)expert_out;
    (void)gate_type;
    (void)down_type;
    const CachedExpert* ce = D.ready ? D.experts.get(cache_idx) : nullptr;
    if (!ce || !input || !gate_out || !up_out) return -1;
    const int H = hidden_dim, I = intermediate;
    const int gt = part_type(*ce, 0, I, H), ut = part_type(*ce, 1, I, H);
    if (gt < 0 || ut < 0 || D.reserve(H, I) != WM_OK) return -1;
    float *x = D.vec(ShimDevice::IN), *g = D.vec(ShimDevice::GATE), *u = D.vec(ShimDevice::UP);
    WM_FAIL_HIP(hipMemcpyAsync(x, input, (size_t)H * sizeof(float), hipMemcpyHostToDevice, D.stream));
    if (wm_quant_matvec(gt, ce->part(0), x, I, H, g, D.ws, D.ws_bytes, D.stream) != WM_OK) return -1;
    if (wm_quant_matvec(ut, ce->part(1), x, I, H, u, D.ws, D.ws_bytes, D.stream) != WM_OK) return -1;
    WM_FAIL_HIP(hipMemcpyAsync(gate_out, g, (size_t)I * sizeof(float), hipMemcpyDeviceToHost, D.stream));
    WM_FAIL_HIP(hipMemcpyAsync(up_out, u, (size_t)I * sizeof(float), hipMemcpyDeviceToHost, D.stream));
    WM_FAIL_HIP(hipStreamSynchronize(D.stream));
    return 0;
}

// Down projection of a host activation vector (gpu_offload.cu:700-712).
extern "C" int gpu_expert_down(int cache_idx, const float* act, int intermediate, float* output, int hidden_dim) {
    const CachedExpert* ce = D.ready ? D.experts.get(cache_idx) : nullptr;
    if (!ce || !act || !output) return -1;
    const int H = hidden_dim, I = intermediate;
    const int dt = part_type(*ce, 2, H, I);
    if (dt < 0 || D.reserve(H, I) != WM_OK) return -1;
    float *a = D.vec(ShimDevice::IN), *y = D.vec(ShimDevice::OUT);
    WM_FAIL_HIP(hipMemcpyAsync(a, act, (size_t)I * sizeof(float), hipMemcpyHostToDevice, D.stream));
    if (wm_quant_matvec(dt, ce->part(2), a, H, I, y, D.ws, D.ws_bytes, D.stream) != WM_OK) return -1;
    WM_FAIL_HIP(hipMemcpyAsync(output, y, (size_t)H * sizeof(float), hipMemcpyDeviceToHost, D.stream));
    WM_FAIL_HIP(hipStreamSynchronize(D.stream));
    return 0;
}

// ------------------------------------------------------------------ batched experts (gpu_offload.cu:757-809)
// start uploads x and zeroes the accumulator; add queues one expert and
// acc += w * y on the stream (no host wait); finish copies acc to the host.

extern "C" int gpu_expert_batch_start(const float* normed, int hidden_dim) {
    if (!D.ready || !normed || hidden_dim <= 0) return -1;
    D.batch_open = false;
    if (D.reserve(hidden_dim, 64) != WM_OK) return -1;
    if (D.acc_len < hidden_dim) {
        (void)hipStreamSynchronize(D.stream);
        if (D.acc) (void)hipFree(D.acc);
        D.acc = nullptr;
        D.acc_len = 0;
        WM_FAIL_HIP(hipMalloc((void**)&D.acc, (size_t)hidden_dim * sizeof(float)));
        D.acc_len = hidden_dim;
    }
    WM_FAIL_HIP(hipMemcpyAsync(D.vec(ShimDevice::IN), normed, (size_t)hidden_dim * sizeof(float),
                               hipMemcpyHostToDevice, D.stream));
    WM_FAIL_HIP(launch_fill_i32((int32_t*)D.acc, 0, hidden_dim, D.stream));
    D.batch_open = true;
    return 0;
}

extern "C" int gpu_expert_batch_add(int cache_idx, int hidden_dim, int intermediate, float weight) {
    const CachedExpert* ce = D.ready ? D.experts.get(cache_idx) : nullptr;
    if (!ce || !D.batch_open || hidden_dim > D.acc_len) return -1;
    if (D.reserve(hidden_dim, intermediate) != WM_OK) return -1;     // never moves the uploaded x
    if (run_cached(*ce, hidden_dim, intermediate, D.vec(ShimDevice::OUT))) return -1;
    WM_FAIL_HIP(launch_axpy(D.acc, D.vec(ShimDevice::OUT), weight, hidden_dim, D.stream));
    return 0;
}

extern "C" int gpu_expert_batch_finish(float* moe_out, int hidden_dim) {
    if (!D.ready || !D.acc || !moe_out || hidden_dim > D.acc_len) return -1;
    WM_FAIL_HIP(hipMemcpyAsync(moe_out, D.acc, (size_t)hidden_dim * sizeof(float), hipMemcpyDeviceToHost, D.stream));
    WM_FAIL_HIP(hipStreamSynchronize(D.stream));
    D.batch_open = false;      // the staging vectors may grow again
    return 0;
}
