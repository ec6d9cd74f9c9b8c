// C ABI of libllmp_hip.so: context, memory helpers, device KV cache manager, RoPE tables,
// per-layer configuration, decode attention entry point and profiling hooks.
// Declarations and reference citations: include/llmp_hip.h.
#include "llmp_hip.h"
#include "llmp_internal.h"
#include "prefill_kernels.h"
#include "gemv_kernels.h"
#include "proj_tok_kernels.h"

#include <algorithm>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <map>
#include <memory>
#include <mutex>
#include <string>
#include <utility>
#include <vector>

namespace llmp {
namespace {

thread_local std::string t_last_error;

int fail(int code, const char* fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    t_last_error = buf;
    return code;
}

#define LLMP_HIP_CHECK(call, what)                                                         \
    do {                                                                                   \
        hipError_t e_ = (call);                                                            \
        if (e_ != hipSuccess)                                                              \
            return fail(LLMP_ERR_HIP, "HIP error in %s: %s (%d)", what, hipGetErrorString(e_), \
                        (int)e_);                                                          \
    } while (0)

// A projection weight or fp32 vector of a layer (llmp_layer_weight), repacked into planes.
struct DevWeight {
    int type = -1;
    int rows = 0, cols = 0;
    void* mem = nullptr;
    gk::WPlanes planes{};
    // The token-batched projections split fp32 and bf16 weights into fp16 parts: false when
    // some weight reaches fp16's largest magnitude, 65504, or for a type proj_tok_supported
    // rejects (llmp_attn_block_batch then runs the tokens one by one, on the fp32 single-token
    // kernels).
    bool tok_ok = true;
};

struct LayerCfg {
    bool configured = false;
    int n_heads = 0;
    int kgroup = 0;             // query heads per workgroup's KV head (kernel_group)
    int krep = 1;               // virtual KV heads per cached KV head: n_heads / (Hkv * kgroup)
    int rope_type = 0;
    int rope_sel = LLMP_ROPE_SEL_GLOBAL;
    int window = 0;
    int is_global = 1;
    float scale = 0.0f;
    float softcap = 0.0f;
    float eps = 0.0f;
    float* d_qnw = nullptr;
    float* d_knw = nullptr;
    float* d_sinks = nullptr;   // [n_heads] sink logits times log2(e) (llmp_layer_sinks)
    int norm_mode = 0;          // LLMP_NORM_* bits (llmp_layer_norm_mode)
    DevWeight w[LLMP_W_SLOTS];  // attention-block weights (llmp_layer_weight)
};

struct RopeTable {
    float* d_cos = nullptr;
    float* d_sin = nullptr;
    int max_seq = 0;
    int half = 0;
};

struct ProfPair {
    hipEvent_t begin, end;
};

struct KvHandle {
    int n_layers = 0, max_seq = 0, n_kv_heads = 0, head_dim = 0, dtype = 0;
    float* pool = nullptr;
    size_t plane_floats = 0;  // floats of one K or V plane of one layer
    RopeTable rope[2];
    std::vector<LayerCfg> layers;
    void* prefill_ws = nullptr;   // prefill tile images (grown on demand)
    size_t prefill_ws_bytes = 0;
    float* prefill_part = nullptr;   // prefill split-K partials (grown on demand)
    size_t prefill_part_bytes = 0;
    float* part_o = nullptr;
    float* part_ml = nullptr;
    int* done = nullptr;             // per virtual KV head: the decode split counters (zero between calls)
    int blk_dim = 0;                 // llmp_block_config: embedding length
    float blk_rscale = 0.0f;         // Granite residual scale, 0 = off
    int blk_input = LLMP_INPUT_F32;  // llmp_block_input_mode
    float* blk_buf = nullptr;        // block scratch: q|k|v, attention output, Wo output
    size_t blk_floats = 0;
    void* blkb_buf = nullptr;        // token-batched block scratch (llmp_attn_block_batch)
    size_t blkb_bytes = 0;
    size_t part_slots = 0;    // (split, query head) slots the workspace holds
    bool prof_on = false;
    std::vector<ProfPair> prof_pending[LLMP_PROF_KINDS];
    std::vector<hipEvent_t> prof_free;
    double prof_ms[LLMP_PROF_KINDS] = {};
    long long prof_count[LLMP_PROF_KINDS] = {};

    // fp32 pool: [layer][K|V][kv_head][pos][D].
    float* k_plane(int layer) const { return pool + (size_t)(2 * layer) * plane_floats; }
    float* v_plane(int layer) const { return pool + (size_t)(2 * layer + 1) * plane_floats; }
    // Q8_0 pool, per layer: K quants, K scales, V quants, V scales, each section padded to
    // 256 bytes so every quant row is 16-byte aligned for the wide loads.
    bool q8() const { return dtype == LLMP_KV_Q8_0 || dtype == LLMP_KV_Q8_0_TRUNC; }
    static size_t pad256(size_t b) { return (b + 255) & ~(size_t)255; }
    size_t q8_quant_bytes() const { return pad256(plane_floats); }
    size_t q8_scale_bytes() const { return pad256(plane_floats / 32 * sizeof(float)); }
    size_t q8_layer_bytes() const { return 2 * (q8_quant_bytes() + q8_scale_bytes()); }
    char* q8_layer(int layer) const {
        return reinterpret_cast<char*>(pool) + (size_t)layer * q8_layer_bytes();
    }
    signed char* kq(int layer) const { return reinterpret_cast<signed char*>(q8_layer(layer)); }
    float* ks(int layer) const {
        return reinterpret_cast<float*>(q8_layer(layer) + q8_quant_bytes());
    }
    signed char* vq(int layer) const {
        return reinterpret_cast<signed char*>(q8_layer(layer) + q8_quant_bytes() + q8_scale_bytes());
    }
    float* vs(int layer) const {
        return reinterpret_cast<float*>(q8_layer(layer) + 2 * q8_quant_bytes() + q8_scale_bytes());
    }
    size_t rows_bytes() const {
        return q8() ? (size_t)n_layers * q8_layer_bytes()
                    : 2 * (size_t)n_layers * plane_floats * sizeof(float);
    }
    // Range exponents of the stored rows (dk::note_range), [layer][kv_head][K, V] int32, after
    // the rows in the same allocation: zeroed with them, raised by every append and by
    // llmp_kv_write / llmp_kv_write_q8.
    int* range(int layer) const {
        return reinterpret_cast<int*>(reinterpret_cast<char*>(pool) + rows_bytes()) +
               (size_t)layer * 2 * (size_t)n_kv_heads;
    }
    size_t pool_bytes() const {
        return rows_bytes() + pad256((size_t)n_layers * 2 * (size_t)n_kv_heads * sizeof(int));
    }
};

// Workspace of llmp_attn_prefill_f32_static, the entry point that allocates nothing: a
// file-scope device array each GPU holds from module load to process end.  Host code never
// uses its name as an address (on the host it is only a stand-in symbol); llmp_init resolves
// the device address once with hipGetSymbolAddress and every use goes through
// Global::scratch.
static __device__ __align__(256) unsigned char scratch[LLMP_PREFILL_STATIC_BYTES];

struct Global {
    std::mutex mu;
    bool init = false;
    int device = -1;
    int n_cu = 0;
    void* scratch = nullptr;   // device address of `scratch` on `device` (llmp_init)
    hipStream_t stream = nullptr;
    std::string arch;
    uint64_t next_handle = 1;
    std::map<uint64_t, std::unique_ptr<KvHandle>> handles;
};

Global& G() {
    static Global g;
    return g;
}

int ensure_init() {
    Global& g = G();
    if (!g.init) return fail(LLMP_ERR_NOT_INIT, "llmp_init has not been called");
    hipError_t e = hipSetDevice(g.device);
    if (e != hipSuccess)
        return fail(LLMP_ERR_HIP, "HIP error in hipSetDevice: %s", hipGetErrorString(e));
    return LLMP_OK;
}

hipStream_t pick_stream(uint64_t s) {
    return s ? reinterpret_cast<hipStream_t>(s) : G().stream;
}

// The handle table is shared by every thread: lookups take the same lock as create and
// destroy.  (Calls on one handle must not overlap; different handles may be used, created and
// destroyed from different threads.)
KvHandle* find_handle(uint64_t h) {
    std::lock_guard<std::mutex> lk(G().mu);
    auto it = G().handles.find(h);
    return it == G().handles.end() ? nullptr : it->second.get();
}

#define LLMP_GET_HANDLE(var, h)                                                   \
    KvHandle* var = find_handle(h);                                               \
    if (!var) return fail(LLMP_ERR_BAD_HANDLE, "unknown KV handle %llu", (unsigned long long)(h))

void free_handle(KvHandle* kv) {
    if (kv->pool) (void)hipFree(kv->pool);
    for (auto& t : kv->rope) {
        if (t.d_cos) (void)hipFree(t.d_cos);
        if (t.d_sin) (void)hipFree(t.d_sin);
    }
    for (auto& l : kv->layers) {
        if (l.d_qnw) (void)hipFree(l.d_qnw);
        if (l.d_knw) (void)hipFree(l.d_knw);
        if (l.d_sinks) (void)hipFree(l.d_sinks);
        for (auto& w : l.w)
            if (w.mem) (void)hipFree(w.mem);
    }
    if (kv->blk_buf) (void)hipFree(kv->blk_buf);
    if (kv->blkb_buf) (void)hipFree(kv->blkb_buf);
    if (kv->part_o) (void)hipFree(kv->part_o);
    if (kv->part_ml) (void)hipFree(kv->part_ml);
    if (kv->done) (void)hipFree(kv->done);
    if (kv->prefill_ws) (void)hipFree(kv->prefill_ws);
    if (kv->prefill_part) (void)hipFree(kv->prefill_part);
    for (auto& v : kv->prof_pending)
        for (auto& p : v) {
            (void)hipEventDestroy(p.begin);
            (void)hipEventDestroy(p.end);
        }
    for (auto e : kv->prof_free) (void)hipEventDestroy(e);
}

int prof_event(KvHandle* kv, hipEvent_t* ev) {
    if (!kv->prof_free.empty()) {
        *ev = kv->prof_free.back();
        kv->prof_free.pop_back();
        return LLMP_OK;
    }
    LLMP_HIP_CHECK(hipEventCreate(ev), "hipEventCreate");
    return LLMP_OK;
}

// Folds completed event pairs of one kind into the totals (waits for them).
int prof_fold(KvHandle* kv, int kind) {
    for (auto& p : kv->prof_pending[kind]) {
        LLMP_HIP_CHECK(hipEventSynchronize(p.end), "hipEventSynchronize");
        float ms = 0.0f;
        LLMP_HIP_CHECK(hipEventElapsedTime(&ms, p.begin, p.end), "hipEventElapsedTime");
        kv->prof_ms[kind] += ms;
        kv->prof_count[kind] += 1;
        kv->prof_free.push_back(p.begin);
        kv->prof_free.push_back(p.end);
    }
    kv->prof_pending[kind].clear();
    return LLMP_OK;
}

// Default launch shape of a decode step over n attended rows (default_splits, from sweeps over
// the BASELINE shapes on MI355X, 256 CUs in 8 XCDs):
//  - fp32 cache: about one workgroup per CU (below 32 rows per split the per-workgroup prologue
//    and merge dominate); very long splits (>= 1024 rows) run 8-wave workgroups on 3/4 as many
//    splits: fewer concurrent KV streams, each read by more waves, keep HBM closer to its peak.
//  - Q8_0 cache: its rows are 3.6x shorter and its math per byte higher, so the kernel is
//    bound by issue and latency: 4-wave workgroups, as many per CU as stay resident at once
//    (one full round over the chip, no tail), at least 160 rows per split (measured on MI355X
//    at the Llama-3.2-3B shape: 96 splits best at 32k rows, 24 at 4k).
void auto_launch(int n, int n_kv_heads, int n_cu, int head_dim, int group, bool q8, int* splits,
                 int* waves) {
    const int per_cu = q8 ? decode_split_blocks_per_cu(head_dim, group, 4, true) : 1;
    bool wide = false;
    *splits = default_splits(n, n_kv_heads, n_cu, per_cu, q8, &wide);
    // head_dim 64 splits of at most 32 rows: 2-wave workgroups (one 16-row trip per wave)
    const bool small = !q8 && !wide && head_dim == 64 && (n + *splits - 1) / *splits <= 32;
    *waves = decode_split_waves(head_dim, group, wide ? 8 : (small ? 2 : 4), q8);
}

struct Plan {
    int start;           // first attended position
    int n;               // attended rows
    int splits;          // split-K partitions per KV head
    int rows_per_split;
    int waves;           // waves per workgroup
};

// Attention window of a layer (Attention.java:330-335): local layers attend to the last
// `window` rows, global layers to all of them.
int layer_window(const LayerCfg& c) { return (c.window > 0 && !c.is_global) ? c.window : 0; }

// Launch plan of one decode call at `position`: splits and workgroup size (auto_launch unless
// the caller fixed the splits), then the kernels' own step plan (plan_step).
Plan make_plan(const KvHandle* kv, const LayerCfg& c, int position, int splits_req) {
    const int window = layer_window(c);
    const StepPlan full = plan_step(position, window, 1);
    const int D = kv->head_dim, Hkv = kv->n_kv_heads * c.krep, group = c.kgroup;
    const bool q8 = kv->q8();
    int s = splits_req, waves = 4;
    if (s <= 0)
        auto_launch(full.n, Hkv, G().n_cu, D, group, q8, &s, &waves);
    else
        waves = decode_split_waves(D, group, (!q8 && full.n / s >= 1024) ? 8 : 4, q8);
    const StepPlan sp = plan_step(position, window, s);
    return Plan{sp.start, sp.n, sp.splits, sp.rows_per_split, waves};
}

// Enqueues one decode layer-call.  With d_pos == nullptr the step runs at `position`;
// otherwise the kernels read the position from device memory when they run, and the launch
// is planned for the longest step the layer can take (position = max_seq - 1).
//
// src_layer >= 0 is a shared-KV layer (Gemma 4): it attends to src_layer's cache rows with its
// own configuration and appends nothing (row `position` must already be cached); k and v are
// not read.  src_layer < 0: the layer's own cache, with the append.
int enqueue_decode(KvHandle* kv, int layer, int src_layer, int position, const int* d_pos,
                   uint64_t q, uint64_t k, uint64_t v, uint64_t gate, uint64_t out, int splits,
                   uint64_t stream) {
    if (layer < 0 || layer >= kv->n_layers)
        return fail(LLMP_ERR_OUT_OF_RANGE, "layer %d outside [0, %d)", layer, kv->n_layers);
    if (src_layer >= kv->n_layers)
        return fail(LLMP_ERR_OUT_OF_RANGE, "source layer %d outside [0, %d)", src_layer,
                    kv->n_layers);
    const bool shared = src_layer >= 0;
    const int kv_layer = shared ? src_layer : layer;
    if (position < 0 || position >= kv->max_seq)
        return fail(LLMP_ERR_OUT_OF_RANGE, "position %d outside [0, %d)", position, kv->max_seq);
    const LayerCfg& c = kv->layers[(size_t)layer];
    if (!c.configured)
        return fail(LLMP_ERR_INVALID_ARG, "layer %d was never configured (llmp_layer_config)", layer);
    if (!q || !out || (!shared && (!k || !v)))
        return fail(LLMP_ERR_INVALID_ARG, "decode: null buffer");
    if ((q | k | v | out) & 15)
        return fail(LLMP_ERR_INVALID_ARG, "decode: q/k/v/out must be 16-byte aligned");
    if (gate & 3) return fail(LLMP_ERR_INVALID_ARG, "decode: gate must be 4-byte aligned");
    if (splits > kMaxSplits)
        return fail(LLMP_ERR_INVALID_ARG, "splits=%d above the maximum %d", splits, kMaxSplits);

    // The grid runs over virtual KV heads: krep per cached KV head, kgroup query heads each.
    const int D = kv->head_dim, Hkv = kv->n_kv_heads * c.krep, group = c.kgroup;
    const Plan plan = make_plan(kv, c, position, splits);
    DecodeArgs a{};
    a.kv_rep = c.krep;
    a.q = reinterpret_cast<const float*>(q);
    a.k = reinterpret_cast<const float*>(k);
    a.v = reinterpret_cast<const float*>(v);
    if (kv->q8()) {
        a.kq = kv->kq(kv_layer);
        a.ks = kv->ks(kv_layer);
        a.vq = kv->vq(kv_layer);
        a.vs = kv->vs(kv_layer);
        a.q8_trunc = kv->dtype == LLMP_KV_Q8_0_TRUNC;
    } else {
        a.kc = kv->k_plane(kv_layer);
        a.vc = kv->v_plane(kv_layer);
    }
    if (c.rope_sel != LLMP_ROPE_SEL_NONE) {
        const RopeTable& t = kv->rope[c.rope_sel];
        if (!t.d_cos)
            return fail(LLMP_ERR_INVALID_ARG, "layer %d selects a RoPE table never uploaded", layer);
        a.cos_t = t.d_cos;
        a.sin_t = t.d_sin;
        a.half_rope = t.half;
    }
    a.norm_seq = (c.norm_mode & LLMP_NORM_SEQUENTIAL) != 0;
    a.v_norm = (c.norm_mode & LLMP_NORM_V) != 0;
    a.no_append = shared;
    a.qnw = c.d_qnw;
    a.knw = c.d_knw;
    a.sinks = c.d_sinks;
    a.gate = reinterpret_cast<const float*>(gate);
    a.out = reinterpret_cast<float*>(out);
    a.part_o = kv->part_o;
    a.part_ml = kv->part_ml;
    a.done = kv->done;
    a.fused = decode_fused_merge(D, group, plan.waves, plan.splits) ? 1 : 0;
    a.d_pos = d_pos;
    a.range = kv->range(kv_layer);
    a.head_stride = (long long)kv->max_seq * D;
    a.pos = position;
    a.max_seq = kv->max_seq;
    a.window = layer_window(c);
    a.splits = plan.splits;
    a.rope_type = c.rope_type;
    a.eps = c.eps;
    const float scale = c.scale > 0.0f ? c.scale : (float)(1.0 / std::sqrt((double)D));
    const float log2e = 1.4426950408889634f;
    if (c.softcap > 0.0f) {
        a.qk_scale = scale;
        a.softcap = c.softcap;
        a.softcap_log2e = c.softcap * log2e;
        a.inv_softcap = 1.0f / c.softcap;
    } else {
        a.qk_scale = scale * log2e;
    }

    hipStream_t st = pick_stream(stream);
    hipEvent_t e0 = nullptr, e1 = nullptr;
    if (kv->prof_on) {
        if (int rc = prof_event(kv, &e0)) return rc;
        if (int rc = prof_event(kv, &e1)) return rc;
        LLMP_HIP_CHECK(hipEventRecord(e0, st), "hipEventRecord");
    }
    LLMP_HIP_CHECK(launch_decode_split(a, D, group, Hkv, plan.waves, kv->q8(), st),
                   "decode split-K launch");
    if (kv->prof_on) {
        LLMP_HIP_CHECK(hipEventRecord(e1, st), "hipEventRecord");
        kv->prof_pending[LLMP_PROF_DECODE_SPLIT].push_back({e0, e1});
    }
    // Several splits: merged by the split kernel's last workgroup per KV head when that is one
    // round of loads (a.fused), else by the combine kernel.
    if (plan.splits > 1 && !a.fused) {
        hipEvent_t e2 = nullptr, e3 = nullptr;
        if (kv->prof_on) {
            if (int rc = prof_event(kv, &e2)) return rc;
            if (int rc = prof_event(kv, &e3)) return rc;
            LLMP_HIP_CHECK(hipEventRecord(e2, st), "hipEventRecord");
        }
        LLMP_HIP_CHECK(launch_decode_reduce(a, D, group, c.n_heads, st), "decode reduce launch");
        if (kv->prof_on) {
            LLMP_HIP_CHECK(hipEventRecord(e3, st), "hipEventRecord");
            kv->prof_pending[LLMP_PROF_DECODE_REDUCE].push_back({e2, e3});
        }
    }
    if (kv->prof_on && kv->prof_pending[LLMP_PROF_DECODE_SPLIT].size() >= 4096) {
        for (int kind = 0; kind < LLMP_PROF_KINDS; ++kind)
            if (int rc = prof_fold(kv, kind)) return rc;
    }
    return LLMP_OK;
}

}  // namespace
}  // namespace llmp

using namespace llmp;

extern "C" {

int llmp_init(int device) {
    Global& g = G();
    std::lock_guard<std::mutex> lk(g.mu);
    if (g.init) {
        if (g.device == device) return LLMP_OK;
        return fail(LLMP_ERR_INVALID_ARG, "already initialised on device %d", g.device);
    }
    int count = 0;
    if (hipGetDeviceCount(&count) != hipSuccess || count <= 0)
        return fail(LLMP_ERR_NO_DEVICE, "no HIP device visible");
    if (device < 0 || device >= count)
        return fail(LLMP_ERR_NO_DEVICE, "device %d out of range (%d devices)", device, count);
    LLMP_HIP_CHECK(hipSetDevice(device), "hipSetDevice");
    hipDeviceProp_t prop;
    LLMP_HIP_CHECK(hipGetDeviceProperties(&prop, device), "hipGetDeviceProperties");
    std::string arch = prop.gcnArchName;
    if (arch.rfind("gfx950", 0) != 0)
        return fail(LLMP_ERR_NO_DEVICE, "device %d is %s; this library is built for gfx950",
                    device, arch.c_str());
    void* sp = nullptr;
    LLMP_HIP_CHECK(hipGetSymbolAddress(&sp, HIP_SYMBOL(scratch)), "hipGetSymbolAddress(scratch)");
    if (!sp) return fail(LLMP_ERR_HIP, "hipGetSymbolAddress(scratch) returned a null address");
    hipStream_t s = nullptr;
    LLMP_HIP_CHECK(hipStreamCreateWithFlags(&s, hipStreamNonBlocking), "hipStreamCreate");
    g.scratch = sp;
    g.device = device;
    g.n_cu = prop.multiProcessorCount;
    g.arch = arch;
    g.stream = s;
    g.init = true;
    return LLMP_OK;
}

int llmp_shutdown(void) {
    Global& g = G();
    std::lock_guard<std::mutex> lk(g.mu);
    if (!g.init) return LLMP_OK;
    (void)hipSetDevice(g.device);
    (void)hipDeviceSynchronize();
    for (auto& kv : g.handles) free_handle(kv.second.get());
    g.handles.clear();
    (void)hipStreamDestroy(g.stream);
    g.stream = nullptr;
    g.scratch = nullptr;
    g.init = false;
    return LLMP_OK;
}

int llmp_device_info(int* n_cu, int64_t* hbm_total, int64_t* hbm_free, char* name, int name_len) {
    if (int rc = ensure_init()) return rc;
    size_t fr = 0, tot = 0;
    LLMP_HIP_CHECK(hipMemGetInfo(&fr, &tot), "hipMemGetInfo");
    if (n_cu) *n_cu = G().n_cu;
    if (hbm_total) *hbm_total = (int64_t)tot;
    if (hbm_free) *hbm_free = (int64_t)fr;
    if (name && name_len > 0) {
        std::strncpy(name, G().arch.c_str(), (size_t)name_len - 1);
        name[name_len - 1] = 0;
    }
    return LLMP_OK;
}

int llmp_last_error(char* buf, int len) {
    if (!buf || len <= 0) return LLMP_ERR_INVALID_ARG;
    std::strncpy(buf, t_last_error.c_str(), (size_t)len - 1);
    buf[len - 1] = 0;
    return LLMP_OK;
}

// ---- memory, streams, events --------------------------------------------------------------
int llmp_malloc(uint64_t* dptr, uint64_t bytes) {
    if (int rc = ensure_init()) return rc;
    if (!dptr || bytes == 0) return fail(LLMP_ERR_INVALID_ARG, "llmp_malloc: bad arguments");
    void* p = nullptr;
    hipError_t e = hipMalloc(&p, bytes);
    if (e == hipErrorOutOfMemory)
        return fail(LLMP_ERR_OUT_OF_MEMORY, "llmp_malloc: %llu bytes do not fit",
                    (unsigned long long)bytes);
    LLMP_HIP_CHECK(e, "hipMalloc");
    *dptr = reinterpret_cast<uint64_t>(p);
    return LLMP_OK;
}

int llmp_free(uint64_t dptr) {
    if (int rc = ensure_init()) return rc;
    LLMP_HIP_CHECK(hipFree(reinterpret_cast<void*>(dptr)), "hipFree");
    return LLMP_OK;
}

int llmp_memcpy_htod(uint64_t dst, const void* src, uint64_t bytes, uint64_t stream) {
    if (int rc = ensure_init()) return rc;
    hipStream_t s = pick_stream(stream);
    LLMP_HIP_CHECK(hipMemcpyAsync(reinterpret_cast<void*>(dst), src, bytes, hipMemcpyHostToDevice, s),
                   "hipMemcpyAsync(HtoD)");
    LLMP_HIP_CHECK(hipStreamSynchronize(s), "hipStreamSynchronize");
    return LLMP_OK;
}

int llmp_memcpy_dtoh(void* dst, uint64_t src, uint64_t bytes, uint64_t stream) {
    if (int rc = ensure_init()) return rc;
    hipStream_t s = pick_stream(stream);
    LLMP_HIP_CHECK(hipMemcpyAsync(dst, reinterpret_cast<const void*>(src), bytes, hipMemcpyDeviceToHost, s),
                   "hipMemcpyAsync(DtoH)");
    LLMP_HIP_CHECK(hipStreamSynchronize(s), "hipStreamSynchronize");
    return LLMP_OK;
}

int llmp_memcpy_dtod(uint64_t dst, uint64_t src, uint64_t bytes, uint64_t stream) {
    if (int rc = ensure_init()) return rc;
    LLMP_HIP_CHECK(hipMemcpyAsync(reinterpret_cast<void*>(dst), reinterpret_cast<const void*>(src),
                                  bytes, hipMemcpyDeviceToDevice, pick_stream(stream)),
                   "hipMemcpyAsync(DtoD)");
    return LLMP_OK;
}

int llmp_memset_zero(uint64_t dst, uint64_t bytes, uint64_t stream) {
    if (int rc = ensure_init()) return rc;
    LLMP_HIP_CHECK(hipMemsetAsync(reinterpret_cast<void*>(dst), 0, bytes, pick_stream(stream)),
                   "hipMemsetAsync");
    return LLMP_OK;
}

int llmp_stream_create(uint64_t* stream) {
    if (int rc = ensure_init()) return rc;
    if (!stream) return fail(LLMP_ERR_INVALID_ARG, "llmp_stream_create: null out");
    hipStream_t s = nullptr;
    LLMP_HIP_CHECK(hipStreamCreateWithFlags(&s, hipStreamNonBlocking), "hipStreamCreate");
    *stream = reinterpret_cast<uint64_t>(s);
    return LLMP_OK;
}

int llmp_stream_destroy(uint64_t stream) {
    if (int rc = ensure_init()) return rc;
    if (!stream) return fail(LLMP_ERR_INVALID_ARG, "llmp_stream_destroy: the library stream is not destroyable");
    LLMP_HIP_CHECK(hipStreamDestroy(reinterpret_cast<hipStream_t>(stream)), "hipStreamDestroy");
    return LLMP_OK;
}

int llmp_stream_sync(uint64_t stream) {
    if (int rc = ensure_init()) return rc;
    LLMP_HIP_CHECK(hipStreamSynchronize(pick_stream(stream)), "hipStreamSynchronize");
    return LLMP_OK;
}

int llmp_event_create(uint64_t* event) {
    if (int rc = ensure_init()) return rc;
    if (!event) return fail(LLMP_ERR_INVALID_ARG, "llmp_event_create: null out");
    hipEvent_t e = nullptr;
    LLMP_HIP_CHECK(hipEventCreate(&e), "hipEventCreate");
    *event = reinterpret_cast<uint64_t>(e);
    return LLMP_OK;
}

int llmp_event_destroy(uint64_t event) {
    if (int rc = ensure_init()) return rc;
    LLMP_HIP_CHECK(hipEventDestroy(reinterpret_cast<hipEvent_t>(event)), "hipEventDestroy");
    return LLMP_OK;
}

int llmp_event_record(uint64_t event, uint64_t stream) {
    if (int rc = ensure_init()) return rc;
    LLMP_HIP_CHECK(hipEventRecord(reinterpret_cast<hipEvent_t>(event), pick_stream(stream)),
                   "hipEventRecord");
    return LLMP_OK;
}

int llmp_event_sync(uint64_t event) {
    if (int rc = ensure_init()) return rc;
    LLMP_HIP_CHECK(hipEventSynchronize(reinterpret_cast<hipEvent_t>(event)), "hipEventSynchronize");
    return LLMP_OK;
}

int llmp_event_elapsed_ms(float* ms, uint64_t start, uint64_t end) {
    if (int rc = ensure_init()) return rc;
    if (!ms) return fail(LLMP_ERR_INVALID_ARG, "llmp_event_elapsed_ms: null out");
    LLMP_HIP_CHECK(hipEventElapsedTime(ms, reinterpret_cast<hipEvent_t>(start),
                                       reinterpret_cast<hipEvent_t>(end)),
                   "hipEventElapsedTime");
    return LLMP_OK;
}

// ---- KV cache manager ------------------------------------------------------------------------
int llmp_kv_create(int n_layers, int max_seq, int n_kv_heads, int head_dim, int dtype,
                   uint64_t* handle) {
    if (int rc = ensure_init()) return rc;
    if (!handle) return fail(LLMP_ERR_INVALID_ARG, "llmp_kv_create: null handle out");
    if (n_layers <= 0 || max_seq <= 0 || n_kv_heads <= 0)
        return fail(LLMP_ERR_INVALID_ARG, "llmp_kv_create: n_layers=%d max_seq=%d n_kv_heads=%d",
                    n_layers, max_seq, n_kv_heads);
    if (head_dim != 64 && head_dim != 80 && head_dim != 96 && head_dim != 128 && head_dim != 256 &&
        head_dim != 512)
        return fail(LLMP_ERR_UNSUPPORTED,
                    "llmp_kv_create: head_dim %d (supported: 64, 80, 96, 128, 256, 512)", head_dim);
    if (dtype != LLMP_KV_F32 && dtype != LLMP_KV_Q8_0 && dtype != LLMP_KV_Q8_0_TRUNC)
        return fail(LLMP_ERR_UNSUPPORTED,
                    "llmp_kv_create: dtype %d (LLMP_KV_F32, LLMP_KV_Q8_0 or LLMP_KV_Q8_0_TRUNC)",
                    dtype);
    if ((head_dim == 512 || head_dim == 80 || head_dim == 96) && dtype != LLMP_KV_F32)
        return fail(LLMP_ERR_UNSUPPORTED, "llmp_kv_create: head_dim %d needs an fp32 cache", head_dim);
    if ((long long)max_seq * head_dim >= (1LL << 31))
        return fail(LLMP_ERR_INVALID_ARG, "llmp_kv_create: max_seq*head_dim exceeds 2^31");
    auto kv = std::make_unique<KvHandle>();
    kv->n_layers = n_layers;
    kv->max_seq = max_seq;
    kv->n_kv_heads = n_kv_heads;
    kv->head_dim = head_dim;
    kv->dtype = dtype;
    kv->plane_floats = (size_t)n_kv_heads * (size_t)max_seq * (size_t)head_dim;
    const size_t bytes = kv->pool_bytes();
    size_t fr = 0, tot = 0;
    LLMP_HIP_CHECK(hipMemGetInfo(&fr, &tot), "hipMemGetInfo");
    if (bytes > fr)
        return fail(LLMP_ERR_OUT_OF_MEMORY,
                    "llmp_kv_create: %zu bytes requested, %zu free of %zu HBM bytes", bytes, fr, tot);
    void* p = nullptr;
    hipError_t e = hipMalloc(&p, bytes);
    if (e == hipErrorOutOfMemory)
        return fail(LLMP_ERR_OUT_OF_MEMORY, "llmp_kv_create: hipMalloc(%zu) out of memory", bytes);
    LLMP_HIP_CHECK(e, "hipMalloc(kv pool)");
    kv->pool = static_cast<float*>(p);
    kv->layers.resize((size_t)n_layers);
    // Split workspace for every layer configuration the handle can take (kMaxSplits slots per
    // query head, at most kMaxGroup query heads per KV head), allocated once so that its
    // address never changes under a captured graph.
    const size_t slots = (size_t)kMaxSplits * (size_t)kMaxGroup * (size_t)n_kv_heads;
    hipError_t ea = hipMalloc(&kv->part_o, slots * (size_t)head_dim * sizeof(float));
    if (ea == hipSuccess) ea = hipMalloc(&kv->part_ml, slots * 2 * sizeof(float));
    // one split counter per query head bounds the virtual KV heads of any layer configuration
    if (ea == hipSuccess) ea = hipMalloc(&kv->done, slots / kMaxSplits * sizeof(int));
    if (ea != hipSuccess) {
        free_handle(kv.get());
        return fail(ea == hipErrorOutOfMemory ? LLMP_ERR_OUT_OF_MEMORY : LLMP_ERR_HIP,
                    "llmp_kv_create: split workspace: %s", hipGetErrorString(ea));
    }
    kv->part_slots = slots;
    hipError_t z = hipMemsetAsync(p, 0, bytes, G().stream);
    if (z == hipSuccess) z = hipMemsetAsync(kv->done, 0, slots / kMaxSplits * sizeof(int), G().stream);
    if (z == hipSuccess) z = hipStreamSynchronize(G().stream);
    if (z != hipSuccess) {
        free_handle(kv.get());
        return fail(LLMP_ERR_HIP, "HIP error in hipMemset(kv pool): %s", hipGetErrorString(z));
    }
    std::lock_guard<std::mutex> lk(G().mu);
    const uint64_t id = G().next_handle++;
    G().handles[id] = std::move(kv);
    *handle = id;
    return LLMP_OK;
}

int llmp_kv_destroy(uint64_t handle) {
    if (int rc = ensure_init()) return rc;
    std::lock_guard<std::mutex> lk(G().mu);
    auto it = G().handles.find(handle);
    if (it == G().handles.end())
        return fail(LLMP_ERR_BAD_HANDLE, "unknown KV handle %llu", (unsigned long long)handle);
    // Work on the handle's memory may sit on any stream the caller used, not only the
    // library's: wait for the whole device before freeing.
    (void)hipDeviceSynchronize();
    free_handle(it->second.get());
    G().handles.erase(it);
    return LLMP_OK;
}

static int check_rows(const KvHandle* kv, int layer, int pos0, int n) {
    if (layer < 0 || layer >= kv->n_layers)
        return fail(LLMP_ERR_OUT_OF_RANGE, "layer %d outside [0, %d)", layer, kv->n_layers);
    if (pos0 < 0 || n < 0 || (long long)pos0 + n > kv->max_seq)
        return fail(LLMP_ERR_OUT_OF_RANGE, "rows [%d, %lld) outside [0, %d)", pos0,
                    (long long)pos0 + n, kv->max_seq);
    return LLMP_OK;
}

// Copies between rows [pos0, pos0+n) of one head-major device plane (per KV head, rows of
// `row` bytes) and a host array in the reference layout [pos][n_kv_heads * row bytes].  The
// host side is re-laid out through a head-major staging buffer so that each head moves as one
// contiguous copy (narrow pitched copies, e.g. the 16-byte scale rows of a Q8_0 cache, are
// otherwise moved row by row).
static int copy_plane(KvHandle* kv, void* dev_plane, size_t row, int pos0, int n, void* host,
                      bool to_host) {
    const size_t H = (size_t)kv->n_kv_heads, span = row * (size_t)n;
    std::vector<char> stage(span * H);
    if (!to_host) rows_to_heads(host, stage.data(), H, (size_t)n, row);
    for (size_t h = 0; h < H; ++h) {
        char* dev = static_cast<char*>(dev_plane) + (h * (size_t)kv->max_seq + (size_t)pos0) * row;
        hipError_t e = to_host ? hipMemcpyAsync(stage.data() + h * span, dev, span,
                                                hipMemcpyDeviceToHost, G().stream)
                               : hipMemcpyAsync(dev, stage.data() + h * span, span,
                                                hipMemcpyHostToDevice, G().stream);
        LLMP_HIP_CHECK(e, "hipMemcpyAsync(kv plane)");
    }
    // The staging buffer is released on return: every copy from or into it must be done.
    LLMP_HIP_CHECK(hipStreamSynchronize(G().stream), "hipStreamSynchronize");
    if (to_host) heads_to_rows(stage.data(), host, H, (size_t)n, row);
    return LLMP_OK;
}

int llmp_kv_read(uint64_t handle, int layer, int pos0, int n, float* host_k, float* host_v) {
    if (int rc = ensure_init()) return rc;
    LLMP_GET_HANDLE(kv, handle);
    if (kv->q8()) return fail(LLMP_ERR_UNSUPPORTED, "llmp_kv_read: Q8_0 cache (use llmp_kv_read_q8)");
    if (int rc = check_rows(kv, layer, pos0, n)) return rc;
    if (n == 0) return LLMP_OK;
    const size_t row = (size_t)kv->head_dim * sizeof(float);
    if (host_k) if (int rc = copy_plane(kv, kv->k_plane(layer), row, pos0, n, host_k, true)) return rc;
    if (host_v) if (int rc = copy_plane(kv, kv->v_plane(layer), row, pos0, n, host_v, true)) return rc;
    return LLMP_OK;
}

// Raises the layer's range exponents to those of rows written from the host (ek / ev: one
// per KV head): a read, a maximum and a write of the layer's 2 * n_kv_heads words.
static int raise_range(KvHandle* kv, int layer, const std::vector<int>& ek, const std::vector<int>& ev) {
    const size_t H = (size_t)kv->n_kv_heads;
    bool any = false;
    for (size_t h = 0; h < H; ++h) any = any || ek[h] > 0 || ev[h] > 0;
    if (!any) return LLMP_OK;
    std::vector<int> cur(2 * H);
    LLMP_HIP_CHECK(hipMemcpyAsync(cur.data(), kv->range(layer), cur.size() * sizeof(int),
                                  hipMemcpyDeviceToHost, G().stream), "hipMemcpyAsync(range)");
    LLMP_HIP_CHECK(hipStreamSynchronize(G().stream), "hipStreamSynchronize");
    for (size_t h = 0; h < H; ++h) {
        cur[2 * h] = std::max(cur[2 * h], ek[h]);
        cur[2 * h + 1] = std::max(cur[2 * h + 1], ev[h]);
    }
    LLMP_HIP_CHECK(hipMemcpyAsync(kv->range(layer), cur.data(), cur.size() * sizeof(int),
                                  hipMemcpyHostToDevice, G().stream), "hipMemcpyAsync(range)");
    LLMP_HIP_CHECK(hipStreamSynchronize(G().stream), "hipStreamSynchronize");
    return LLMP_OK;
}

int llmp_kv_write(uint64_t handle, int layer, int pos0, int n, const float* host_k,
                  const float* host_v) {
    if (int rc = ensure_init()) return rc;
    LLMP_GET_HANDLE(kv, handle);
    if (kv->q8()) return fail(LLMP_ERR_UNSUPPORTED, "llmp_kv_write: Q8_0 cache (use llmp_kv_write_q8)");
    if (int rc = check_rows(kv, layer, pos0, n)) return rc;
    if (n == 0) return LLMP_OK;
    {
        std::vector<int> ek((size_t)kv->n_kv_heads, 0), ev((size_t)kv->n_kv_heads, 0);
        range_exp_rows(host_k, host_v, (size_t)kv->n_kv_heads, (size_t)n, (size_t)kv->head_dim,
                       ek.data(), ev.data());
        if (int rc = raise_range(kv, layer, ek, ev)) return rc;
    }
    const size_t row = (size_t)kv->head_dim * sizeof(float);
    if (host_k)
        if (int rc = copy_plane(kv, kv->k_plane(layer), row, pos0, n, const_cast<float*>(host_k), false))
            return rc;
    if (host_v)
        if (int rc = copy_plane(kv, kv->v_plane(layer), row, pos0, n, const_cast<float*>(host_v), false))
            return rc;
    return LLMP_OK;
}

int llmp_kv_read_q8(uint64_t handle, int layer, int pos0, int n, int8_t* k_quants,
                    float* k_scales, int8_t* v_quants, float* v_scales) {
    if (int rc = ensure_init()) return rc;
    LLMP_GET_HANDLE(kv, handle);
    if (!kv->q8()) return fail(LLMP_ERR_UNSUPPORTED, "llmp_kv_read_q8: not a Q8_0 cache");
    if (int rc = check_rows(kv, layer, pos0, n)) return rc;
    if (n == 0) return LLMP_OK;
    const size_t qrow = (size_t)kv->head_dim, srow = (size_t)kv->head_dim / 32 * sizeof(float);
    if (k_quants) if (int rc = copy_plane(kv, kv->kq(layer), qrow, pos0, n, k_quants, true)) return rc;
    if (k_scales) if (int rc = copy_plane(kv, kv->ks(layer), srow, pos0, n, k_scales, true)) return rc;
    if (v_quants) if (int rc = copy_plane(kv, kv->vq(layer), qrow, pos0, n, v_quants, true)) return rc;
    if (v_scales) if (int rc = copy_plane(kv, kv->vs(layer), srow, pos0, n, v_scales, true)) return rc;
    return LLMP_OK;
}

int llmp_kv_write_q8(uint64_t handle, int layer, int pos0, int n, const int8_t* k_quants,
                     const float* k_scales, const int8_t* v_quants, const float* v_scales) {
    if (int rc = ensure_init()) return rc;
    LLMP_GET_HANDLE(kv, handle);
    if (!kv->q8()) return fail(LLMP_ERR_UNSUPPORTED, "llmp_kv_write_q8: not a Q8_0 cache");
    if (int rc = check_rows(kv, layer, pos0, n)) return rc;
    if (n == 0) return LLMP_OK;
    const size_t qrow = (size_t)kv->head_dim, srow = (size_t)kv->head_dim / 32 * sizeof(float);
    auto cp = [&](void* plane, size_t row, const void* host) {
        return copy_plane(kv, plane, row, pos0, n, const_cast<void*>(host), false);
    };
    if (k_quants) if (int rc = cp(kv->kq(layer), qrow, k_quants)) return rc;
    if (k_scales) if (int rc = cp(kv->ks(layer), srow, k_scales)) return rc;
    if (v_quants) if (int rc = cp(kv->vq(layer), qrow, v_quants)) return rc;
    if (v_scales) if (int rc = cp(kv->vs(layer), srow, v_scales)) return rc;
    // Range exponents of the values the kernels now dequantise from these rows (quant * scale),
    // read back whole so that a write of quants or scales alone is bounded too.
    const size_t H = (size_t)kv->n_kv_heads;
    std::vector<int> ek(H, 0), ev(H, 0);
    std::vector<int8_t> qb((size_t)n * H * qrow);
    std::vector<float> sb((size_t)n * H * qrow / 32);
    for (int which = 0; which < 2; ++which) {
        const bool k_side = which == 0;
        if (k_side ? !(k_quants || k_scales) : !(v_quants || v_scales)) continue;
        if (int rc = copy_plane(kv, k_side ? (void*)kv->kq(layer) : (void*)kv->vq(layer), qrow, pos0, n,
                                qb.data(), true))
            return rc;
        if (int rc = copy_plane(kv, k_side ? (void*)kv->ks(layer) : (void*)kv->vs(layer), srow, pos0, n,
                                sb.data(), true))
            return rc;
        range_exp_rows_q8(qb.data(), sb.data(), H, (size_t)n, qrow, k_side ? ek.data() : ev.data());
    }
    return raise_range(kv, layer, ek, ev);
}

int llmp_kv_layer_ptrs(uint64_t handle, int layer, uint64_t* k_plane, uint64_t* v_plane) {
    if (int rc = ensure_init()) return rc;
    LLMP_GET_HANDLE(kv, handle);
    if (layer < 0 || layer >= kv->n_layers)
        return fail(LLMP_ERR_OUT_OF_RANGE, "layer %d outside [0, %d)", layer, kv->n_layers);
    if (k_plane)
        *k_plane = kv->q8() ? reinterpret_cast<uint64_t>(kv->kq(layer))
                            : reinterpret_cast<uint64_t>(kv->k_plane(layer));
    if (v_plane)
        *v_plane = kv->q8() ? reinterpret_cast<uint64_t>(kv->vq(layer))
                            : reinterpret_cast<uint64_t>(kv->v_plane(layer));
    return LLMP_OK;
}

int llmp_kv_clear(uint64_t handle, uint64_t stream) {
    if (int rc = ensure_init()) return rc;
    LLMP_GET_HANDLE(kv, handle);
    LLMP_HIP_CHECK(hipMemsetAsync(kv->pool, 0, kv->pool_bytes(), pick_stream(stream)),
                   "hipMemsetAsync(kv)");
    return LLMP_OK;
}

// ---- RoPE ------------------------------------------------------------------------------------
int llmp_rope_table(int rope_dim, int max_seq, float theta, float linear_freq_scale,
                    const float* freq_factors, int n_freq_factors, float* cos_out,
                    float* sin_out) {
    if (rope_dim <= 0 || (rope_dim & 1) || max_seq <= 0 || !cos_out || !sin_out)
        return fail(LLMP_ERR_INVALID_ARG, "llmp_rope_table: rope_dim=%d max_seq=%d", rope_dim,
                    max_seq);
    const int half = rope_dim / 2;
    const float freq_scale = linear_freq_scale > 1.0f ? 1.0f / linear_freq_scale : 1.0f;
    std::vector<float> freq((size_t)half);
    for (int i = 0; i < half; ++i) {
        const double ex = 2.0 * (double)i / (double)rope_dim;
        float base = (float)(1.0 / std::pow((double)theta, ex));
        if (freq_factors && i < n_freq_factors) base = base / freq_factors[i];
        freq[(size_t)i] = base * freq_scale;
    }
    for (int pos = 0; pos < max_seq; ++pos) {
        for (int i = 0; i < half; ++i) {
            const float angle = (float)pos * freq[(size_t)i];
            cos_out[(size_t)pos * half + i] = (float)std::cos((double)angle);
            sin_out[(size_t)pos * half + i] = (float)std::sin((double)angle);
        }
    }
    return LLMP_OK;
}

int llmp_rope_table_yarn(int rope_dim, int max_seq, float theta, const float* freq_factors,
                         int n_freq_factors, float scaling_factor, int orig_ctx, float beta_fast,
                         float beta_slow, float yarn_log_mul, float* cos_out, float* sin_out,
                         float* mscale) {
    if (!(scaling_factor > 1.0f)) {   // RoPE.java:59: no YaRN, no linear scale
        if (mscale) *mscale = 1.0f;
        return llmp_rope_table(rope_dim, max_seq, theta, 1.0f, freq_factors, n_freq_factors, cos_out,
                               sin_out);
    }
    if (rope_dim <= 0 || (rope_dim & 1) || max_seq <= 0 || !cos_out || !sin_out || orig_ctx <= 0 ||
        !(beta_fast > 0.0f) || !(beta_slow > 0.0f))
        return fail(LLMP_ERR_INVALID_ARG, "llmp_rope_table_yarn: rope_dim=%d max_seq=%d orig_ctx=%d",
                    rope_dim, max_seq, orig_ctx);
    const int half = rope_dim / 2;
    const float freq_scale = 1.0f / scaling_factor;
    const double pi = 3.141592653589793;
    // RoPE.yarnCorrDim (RoPE.java:107-110) for both betas, floored / ceiled into [0, R/2 - 1]
    auto corr_dim = [&](float beta) {
        return (float)rope_dim * (float)std::log((double)orig_ctx / ((double)beta * 2.0 * pi)) /
               (2.0f * (float)std::log((double)theta));
    };
    const float fl = (float)std::floor((double)corr_dim(beta_fast));
    const float low = fl > 0.0f ? fl : 0.0f;
    const float ce = (float)std::ceil((double)corr_dim(beta_slow));
    const float lim = (float)rope_dim / 2.0f - 1.0f;
    const float high = lim < ce ? lim : ce;
    float attn_factor = 1.0f;
    if (yarn_log_mul > 0.0f)
        attn_factor = 0.1f * yarn_log_mul * (float)std::log((double)scaling_factor) + 1.0f;
    if (mscale) *mscale = attn_factor * (1.0f + 0.1f * (float)std::log((double)(1.0f / freq_scale)));
    std::vector<float> freq((size_t)half);
    for (int i = 0; i < half; ++i) {
        const double ex = 2.0 * (double)i / (double)rope_dim;
        float base = (float)(1.0 / std::pow((double)theta, ex));
        if (freq_factors && i < n_freq_factors) base = base / freq_factors[i];
        // NTK-by-parts blend (RoPE.java:89-93, yarnRamp :113-117)
        const float span = high - low;
        const float y = ((float)i - low) / (span > 0.001f ? span : 0.001f);
        const float cl = y < 0.0f ? 0.0f : (y < 1.0f ? y : 1.0f);
        const float ramp = 1.0f - cl;
        const float interp = freq_scale * base;
        const float a = interp * (1.0f - ramp);
        const float b = base * ramp;
        freq[(size_t)i] = a + b;
    }
    for (int pos = 0; pos < max_seq; ++pos) {
        for (int i = 0; i < half; ++i) {
            const float angle = (float)pos * freq[(size_t)i];
            cos_out[(size_t)pos * half + i] = (float)std::cos((double)angle);
            sin_out[(size_t)pos * half + i] = (float)std::sin((double)angle);
        }
    }
    return LLMP_OK;
}

int llmp_rope_upload(uint64_t handle, int which, const float* cos_t, const float* sin_t,
                     int max_seq, int half_rope) {
    if (int rc = ensure_init()) return rc;
    LLMP_GET_HANDLE(kv, handle);
    if (which != LLMP_ROPE_SEL_GLOBAL && which != LLMP_ROPE_SEL_LOCAL)
        return fail(LLMP_ERR_INVALID_ARG, "llmp_rope_upload: which=%d", which);
    if (!cos_t || !sin_t || half_rope <= 0 || 2 * half_rope > kv->head_dim || max_seq < kv->max_seq)
        return fail(LLMP_ERR_INVALID_ARG,
                    "llmp_rope_upload: need >= %d rows of <= %d pairs (got max_seq=%d half=%d)",
                    kv->max_seq, kv->head_dim / 2, max_seq, half_rope);
    RopeTable& t = kv->rope[which];
    const size_t bytes = (size_t)kv->max_seq * half_rope * sizeof(float);
    if (t.d_cos && (t.half != half_rope)) {
        (void)hipFree(t.d_cos);
        (void)hipFree(t.d_sin);
        t.d_cos = t.d_sin = nullptr;
    }
    if (!t.d_cos) {
        LLMP_HIP_CHECK(hipMalloc(&t.d_cos, bytes), "hipMalloc(rope cos)");
        LLMP_HIP_CHECK(hipMalloc(&t.d_sin, bytes), "hipMalloc(rope sin)");
    }
    LLMP_HIP_CHECK(hipMemcpy(t.d_cos, cos_t, bytes, hipMemcpyHostToDevice), "hipMemcpy(rope cos)");
    LLMP_HIP_CHECK(hipMemcpy(t.d_sin, sin_t, bytes, hipMemcpyHostToDevice), "hipMemcpy(rope sin)");
    t.max_seq = kv->max_seq;
    t.half = half_rope;
    return LLMP_OK;
}

// ---- layer configuration -------------------------------------------------------------------
int llmp_layer_config(uint64_t handle, int layer, int n_heads, int n_kv_heads, int head_dim,
                      int rope_type, int rope_sel, int window, int is_global, float scale,
                      float softcap, float eps, const float* qnorm_w, const float* knorm_w) {
    if (int rc = ensure_init()) return rc;
    LLMP_GET_HANDLE(kv, handle);
    if (layer < 0 || layer >= kv->n_layers)
        return fail(LLMP_ERR_OUT_OF_RANGE, "layer %d outside [0, %d)", layer, kv->n_layers);
    if (n_kv_heads != kv->n_kv_heads || head_dim != kv->head_dim)
        return fail(LLMP_ERR_INVALID_ARG,
                    "layer %d: n_kv_heads=%d head_dim=%d differ from the cache's %d/%d", layer,
                    n_kv_heads, head_dim, kv->n_kv_heads, kv->head_dim);
    if (n_heads <= 0 || n_heads % n_kv_heads != 0)
        return fail(LLMP_ERR_INVALID_ARG, "layer %d: n_heads=%d not a multiple of n_kv_heads=%d",
                    layer, n_heads, n_kv_heads);
    const int group = n_heads / n_kv_heads;
    const int kgroup = kernel_group(head_dim, group);
    if (kgroup == 0)
        return fail(LLMP_ERR_UNSUPPORTED, "layer %d: no decode kernel for head_dim=%d group=%d",
                    layer, head_dim, group);
    if (rope_type != LLMP_ROPE_NORMAL && rope_type != LLMP_ROPE_NEOX)
        return fail(LLMP_ERR_INVALID_ARG, "layer %d: rope_type=%d", layer, rope_type);
    if (rope_sel != LLMP_ROPE_SEL_NONE && rope_sel != LLMP_ROPE_SEL_GLOBAL &&
        rope_sel != LLMP_ROPE_SEL_LOCAL)
        return fail(LLMP_ERR_INVALID_ARG, "layer %d: rope_sel=%d", layer, rope_sel);
    if (window < 0 || softcap < 0.0f || !std::isfinite(scale) || !std::isfinite(softcap) ||
        !std::isfinite(eps))
        return fail(LLMP_ERR_INVALID_ARG, "layer %d: window=%d softcap=%g", layer, window,
                    (double)softcap);
    if ((qnorm_w == nullptr) != (knorm_w == nullptr))
        return fail(LLMP_ERR_INVALID_ARG, "layer %d: QK-norm needs both weights or neither", layer);

    if ((size_t)kMaxSplits * (size_t)n_heads > kv->part_slots) {
        // More query heads than llmp_kv_create sized the split workspace for (groups above
        // kMaxGroup): it grows here, at set-up, so graphs captured before must be captured again.
        const size_t slots = (size_t)kMaxSplits * (size_t)n_heads;
        LLMP_HIP_CHECK(hipDeviceSynchronize(), "hipDeviceSynchronize");
        (void)hipFree(kv->part_o);
        (void)hipFree(kv->part_ml);
        (void)hipFree(kv->done);
        kv->part_o = kv->part_ml = nullptr;
        kv->done = nullptr;
        kv->part_slots = 0;
        hipError_t ea = hipMalloc(&kv->part_o, slots * (size_t)head_dim * sizeof(float));
        if (ea == hipSuccess) ea = hipMalloc(&kv->part_ml, slots * 2 * sizeof(float));
        if (ea == hipSuccess) ea = hipMalloc(&kv->done, (size_t)n_heads * sizeof(int));
        if (ea == hipSuccess) ea = hipMemset(kv->done, 0, (size_t)n_heads * sizeof(int));
        if (ea != hipSuccess)
            return fail(ea == hipErrorOutOfMemory ? LLMP_ERR_OUT_OF_MEMORY : LLMP_ERR_HIP,
                        "layer %d: split workspace for %d query heads: %s", layer, n_heads,
                        hipGetErrorString(ea));
        kv->part_slots = slots;
    }
    LayerCfg& c = kv->layers[(size_t)layer];
    const size_t wbytes = (size_t)head_dim * sizeof(float);
    if (qnorm_w) {
        if (!c.d_qnw) LLMP_HIP_CHECK(hipMalloc(&c.d_qnw, wbytes), "hipMalloc(qnorm)");
        if (!c.d_knw) LLMP_HIP_CHECK(hipMalloc(&c.d_knw, wbytes), "hipMalloc(knorm)");
        LLMP_HIP_CHECK(hipMemcpy(c.d_qnw, qnorm_w, wbytes, hipMemcpyHostToDevice), "hipMemcpy(qnorm)");
        LLMP_HIP_CHECK(hipMemcpy(c.d_knw, knorm_w, wbytes, hipMemcpyHostToDevice), "hipMemcpy(knorm)");
    } else {
        if (c.d_qnw) (void)hipFree(c.d_qnw);
        if (c.d_knw) (void)hipFree(c.d_knw);
        c.d_qnw = c.d_knw = nullptr;
    }
    if (c.d_sinks && c.n_heads != n_heads) {   // sinks are per query head: a new count drops them
        (void)hipFree(c.d_sinks);
        c.d_sinks = nullptr;
    }
    c.n_heads = n_heads;
    c.kgroup = kgroup;
    c.krep = group / kgroup;
    c.rope_type = rope_type;
    c.rope_sel = rope_sel;
    c.window = window;
    c.is_global = is_global;
    c.scale = scale;
    c.softcap = softcap;
    c.eps = eps;
    c.configured = true;
    return LLMP_OK;
}

// ---- decode attention --------------------------------------------------------------------------
int llmp_attn_decode(uint64_t handle, int layer, int position, uint64_t q, uint64_t k, uint64_t v,
                     uint64_t out, int splits, uint64_t stream) {
    if (int rc = ensure_init()) return rc;
    LLMP_GET_HANDLE(kv, handle);
    return enqueue_decode(kv, layer, -1, position, nullptr, q, k, v, 0, out, splits, stream);
}

int llmp_attn_decode_devpos(uint64_t handle, int layer, uint64_t d_position, uint64_t q,
                            uint64_t k, uint64_t v, uint64_t out, int splits, uint64_t stream) {
    if (int rc = ensure_init()) return rc;
    LLMP_GET_HANDLE(kv, handle);
    if (!d_position || (d_position & 3))
        return fail(LLMP_ERR_INVALID_ARG, "llmp_attn_decode_devpos: null or misaligned position word");
    return enqueue_decode(kv, layer, -1, kv->max_seq - 1, reinterpret_cast<const int*>(d_position), q,
                          k, v, 0, out, splits, stream);
}

int llmp_attn_decode_ex(uint64_t handle, int layer, int position, uint64_t d_position,
                        uint64_t q, uint64_t k, uint64_t v, uint64_t gate, uint64_t out,
                        int splits, uint64_t stream) {
    if (int rc = ensure_init()) return rc;
    LLMP_GET_HANDLE(kv, handle);
    if (d_position & 3)
        return fail(LLMP_ERR_INVALID_ARG, "llmp_attn_decode_ex: misaligned position word");
    if (d_position)
        return enqueue_decode(kv, layer, -1, kv->max_seq - 1, reinterpret_cast<const int*>(d_position),
                              q, k, v, gate, out, splits, stream);
    return enqueue_decode(kv, layer, -1, position, nullptr, q, k, v, gate, out, splits, stream);
}

int llmp_attn_decode_shared(uint64_t handle, int layer, int src_layer, int position,
                            uint64_t d_position, uint64_t q, uint64_t gate, uint64_t out,
                            int splits, uint64_t stream) {
    if (int rc = ensure_init()) return rc;
    LLMP_GET_HANDLE(kv, handle);
    if (src_layer < 0)
        return fail(LLMP_ERR_OUT_OF_RANGE, "llmp_attn_decode_shared: source layer %d", src_layer);
    if (d_position & 3)
        return fail(LLMP_ERR_INVALID_ARG, "llmp_attn_decode_shared: misaligned position word");
    if (d_position)
        return enqueue_decode(kv, layer, src_layer, kv->max_seq - 1,
                              reinterpret_cast<const int*>(d_position), q, 0, 0, gate, out, splits,
                              stream);
    return enqueue_decode(kv, layer, src_layer, position, nullptr, q, 0, 0, gate, out, splits,
                          stream);
}

int llmp_layer_norm_mode(uint64_t handle, int layer, int mode) {
    if (int rc = ensure_init()) return rc;
    LLMP_GET_HANDLE(kv, handle);
    if (layer < 0 || layer >= kv->n_layers)
        return fail(LLMP_ERR_OUT_OF_RANGE, "layer %d outside [0, %d)", layer, kv->n_layers);
    if (mode & ~(LLMP_NORM_SEQUENTIAL | LLMP_NORM_V))
        return fail(LLMP_ERR_INVALID_ARG, "llmp_layer_norm_mode: unknown mode bits 0x%x", mode);
    kv->layers[(size_t)layer].norm_mode = mode;
    return LLMP_OK;
}

// ---- attention block: projections around the attention core ------------------------------
// Byte offsets of the token-batched block scratch: q, k, v, the attention output and the
// output projection of kTokBatch tokens (each region 256-byte aligned).
struct BatchLayout {
    size_t q, k, v, attn, o, sc, q8b, q8d, q8s, total;
};
static BatchLayout batch_layout(const KvHandle* kv, int qd, int kvd) {
    auto al = [](size_t b) { return (b + 255) & ~(size_t)255; };
    const int dim = kv->blk_dim;
    BatchLayout L;
    L.q = 0;
    L.k = L.q + al((size_t)kTokBatch * qd * sizeof(float));
    L.v = L.k + al((size_t)kTokBatch * kvd * sizeof(float));
    L.attn = L.v + al((size_t)kTokBatch * kvd * sizeof(float));
    L.o = L.attn + al((size_t)kTokBatch * qd * sizeof(float));
    L.sc = L.o + al((size_t)kTokBatch * dim * sizeof(float));
    // the Q8_1 staging of the widest projection input (dim for Q/K/V, q_dim for Wo)
    const size_t groups = (size_t)(dim > qd ? dim : qd) / 32;
    L.q8b = L.sc + al((size_t)kTokBatch * 2 * sizeof(float));
    L.q8d = L.q8b + al(groups * 64 * 16);
    L.q8s = L.q8d + al(groups * kTokBatch * sizeof(float));
    L.total = L.q8s + al(groups * kTokBatch * sizeof(float));
    return L;
}

int llmp_block_config(uint64_t handle, int dim, float residual_scale) {
    if (int rc = ensure_init()) return rc;
    LLMP_GET_HANDLE(kv, handle);
    if (dim <= 0 || dim > gk::kMaxGemvCols || dim % 32)
        return fail(LLMP_ERR_INVALID_ARG, "llmp_block_config: dim %d (a multiple of 32 up to %d)",
                    dim, gk::kMaxGemvCols);
    if (!(residual_scale >= 0.0f) || !std::isfinite(residual_scale))
        return fail(LLMP_ERR_INVALID_ARG, "llmp_block_config: residual scale %g", (double)residual_scale);
    if (kv->blk_dim != 0 && kv->blk_dim != dim)
        for (auto& l : kv->layers)
            for (auto& w : l.w)
                if (w.mem) return fail(LLMP_ERR_INVALID_ARG, "llmp_block_config: weights uploaded for dim %d",
                                       kv->blk_dim);
    kv->blk_dim = dim;
    kv->blk_rscale = residual_scale;
    return LLMP_OK;
}

int llmp_block_input_mode(uint64_t handle, int mode) {
    if (int rc = ensure_init()) return rc;
    LLMP_GET_HANDLE(kv, handle);
    if (mode != LLMP_INPUT_F32 && mode != LLMP_INPUT_Q8_1)
        return fail(LLMP_ERR_INVALID_ARG, "llmp_block_input_mode: mode %d", mode);
    kv->blk_input = mode;
    return LLMP_OK;
}

int llmp_layer_weight(uint64_t handle, int layer, int slot, int ggml_type, int rows, int cols,
                      const void* data, uint64_t nbytes) {
    if (int rc = ensure_init()) return rc;
    LLMP_GET_HANDLE(kv, handle);
    if (layer < 0 || layer >= kv->n_layers)
        return fail(LLMP_ERR_OUT_OF_RANGE, "layer %d outside [0, %d)", layer, kv->n_layers);
    if (slot < 0 || slot >= LLMP_W_SLOTS)
        return fail(LLMP_ERR_INVALID_ARG, "llmp_layer_weight: slot %d", slot);
    LayerCfg& c = kv->layers[(size_t)layer];
    if (!c.configured)
        return fail(LLMP_ERR_INVALID_ARG, "layer %d was never configured (llmp_layer_config)", layer);
    if (kv->blk_dim == 0)
        return fail(LLMP_ERR_INVALID_ARG, "llmp_layer_weight: call llmp_block_config first");
    DevWeight& w = c.w[slot];
    if (w.mem) (void)hipFree(w.mem);
    w = DevWeight{};
    if (data == nullptr) return LLMP_OK;   // slot removed
    const int D = kv->head_dim, qd = c.n_heads * D, kvd = kv->n_kv_heads * D, dim = kv->blk_dim;
    int want_rows = 1, want_cols = 0;
    bool vec = false;
    switch (slot) {
    case LLMP_W_ATTN_NORM: case LLMP_W_POST_ATTN_NORM: case LLMP_W_O_BIAS:
        vec = true; want_cols = dim; break;
    case LLMP_W_Q_BIAS: vec = true; want_cols = qd; break;
    case LLMP_W_K_BIAS: case LLMP_W_V_BIAS: vec = true; want_cols = kvd; break;
    case LLMP_W_Q: want_rows = qd; want_cols = dim; break;
    case LLMP_W_K: case LLMP_W_V: want_rows = kvd; want_cols = dim; break;
    case LLMP_W_QKV: want_rows = qd + 2 * kvd; want_cols = dim; break;
    case LLMP_W_O: want_rows = dim; want_cols = qd; break;
    }
    if (rows != want_rows || cols != want_cols)
        return fail(LLMP_ERR_INVALID_ARG, "llmp_layer_weight: slot %d is [%d][%d], got [%d][%d]", slot,
                    want_rows, want_cols, rows, cols);
    if (vec && ggml_type != LLMP_GGML_F32)
        return fail(LLMP_ERR_INVALID_ARG, "llmp_layer_weight: slot %d takes fp32 values", slot);
    const int unit = vec ? 1 : gemv_unit(ggml_type);
    const size_t rb = ggml_row_bytes(ggml_type, cols);
    if (unit == 0 || rb == 0)
        return fail(LLMP_ERR_UNSUPPORTED, "llmp_layer_weight: GGML type %d has no kernel", ggml_type);
    if (cols % unit || (!vec && cols > gk::kMaxGemvCols))
        return fail(LLMP_ERR_UNSUPPORTED, "llmp_layer_weight: %d columns for GGML type %d", cols, ggml_type);
    if (nbytes != (uint64_t)rb * (uint64_t)rows)
        return fail(LLMP_ERR_INVALID_ARG, "llmp_layer_weight: %llu bytes, expected %llu",
                    (unsigned long long)nbytes, (unsigned long long)rb * rows);
    std::vector<uint8_t> packed;
    size_t off[4] = {0, 0, 0, 0}, pitch[4] = {0, 0, 0, 0};
    const int np = repack_weight(ggml_type, rows, cols, static_cast<const uint8_t*>(data), packed, off, pitch);
    if (np == 0)
        return fail(LLMP_ERR_UNSUPPORTED, "llmp_layer_weight: %d columns for GGML type %d", cols, ggml_type);
    hipError_t e = hipMalloc(&w.mem, packed.size());
    if (e == hipErrorOutOfMemory)
        return fail(LLMP_ERR_OUT_OF_MEMORY, "llmp_layer_weight: %zu bytes", packed.size());
    LLMP_HIP_CHECK(e, "hipMalloc(weight)");
    LLMP_HIP_CHECK(hipMemcpy(w.mem, packed.data(), packed.size(), hipMemcpyHostToDevice), "hipMemcpy(weight)");
    w.tok_ok = vec || proj_tok_supported(ggml_type);
    if (!vec && (ggml_type == LLMP_GGML_F32 || ggml_type == LLMP_GGML_BF16)) {
        const size_t n = (size_t)rows * cols;
        for (size_t i = 0; i < n && w.tok_ok; ++i) {
            float f;
            if (ggml_type == LLMP_GGML_F32) {
                std::memcpy(&f, static_cast<const char*>(data) + 4 * i, 4);
            } else {
                uint16_t b;
                std::memcpy(&b, static_cast<const char*>(data) + 2 * i, 2);
                const uint32_t u = (uint32_t)b << 16;
                std::memcpy(&f, &u, 4);
            }
            if (!(std::fabs(f) < 65504.0f)) w.tok_ok = false;
        }
    }
    w.type = ggml_type;
    w.rows = rows;
    w.cols = cols;
    for (int i = 0; i < np; ++i) {
        w.planes.p[i] = static_cast<const unsigned char*>(w.mem) + off[i];
        w.planes.pitch[i] = (long long)pitch[i];
    }
    // Block scratch: q | k | v, the attention output and the Wo output (kept per handle).
    const size_t need = (size_t)(qd + 2 * kvd) + (size_t)qd + (size_t)dim + 64;
    if (need > kv->blk_floats) {
        LLMP_HIP_CHECK(hipDeviceSynchronize(), "hipDeviceSynchronize");
        if (kv->blk_buf) (void)hipFree(kv->blk_buf);
        kv->blk_buf = nullptr;
        kv->blk_floats = 0;
        LLMP_HIP_CHECK(hipMalloc(&kv->blk_buf, need * sizeof(float)), "hipMalloc(block scratch)");
        kv->blk_floats = need;
    }
    // Token-batched block scratch: q, k, v, the attention output and the output projection of
    // 16 tokens.
    const size_t needb = batch_layout(kv, qd, kvd).total;
    if (needb > kv->blkb_bytes) {
        LLMP_HIP_CHECK(hipDeviceSynchronize(), "hipDeviceSynchronize");
        if (kv->blkb_buf) (void)hipFree(kv->blkb_buf);
        kv->blkb_buf = nullptr;
        kv->blkb_bytes = 0;
        LLMP_HIP_CHECK(hipMalloc(&kv->blkb_buf, needb), "hipMalloc(batched block scratch)");
        kv->blkb_bytes = needb;
    }
    return LLMP_OK;
}

static int enqueue_block(KvHandle* kv, int layer, int position, uint64_t d_position, uint64_t x,
                         int splits, uint64_t stream);

int llmp_attn_block(uint64_t handle, int layer, int position, uint64_t d_position, uint64_t x,
                    int splits, uint64_t stream) {
    if (int rc = ensure_init()) return rc;
    LLMP_GET_HANDLE(kv, handle);
    return enqueue_block(kv, layer, position, d_position, x, splits, stream);
}

// One token's attention half (llmp_attn_block).
static int enqueue_block(KvHandle* kv, int layer, int position, uint64_t d_position, uint64_t x,
                         int splits, uint64_t stream) {
    if (layer < 0 || layer >= kv->n_layers)
        return fail(LLMP_ERR_OUT_OF_RANGE, "layer %d outside [0, %d)", layer, kv->n_layers);
    const LayerCfg& c = kv->layers[(size_t)layer];
    if (!c.configured)
        return fail(LLMP_ERR_INVALID_ARG, "layer %d was never configured (llmp_layer_config)", layer);
    const DevWeight* W = c.w;
    const bool merged = W[LLMP_W_QKV].mem != nullptr;
    if (kv->blk_dim == 0 || !W[LLMP_W_O].mem ||
        (!merged && (!W[LLMP_W_Q].mem || !W[LLMP_W_K].mem || !W[LLMP_W_V].mem)))
        return fail(LLMP_ERR_INVALID_ARG, "llmp_attn_block: layer %d lacks projection weights", layer);
    if (!x || (x & 3)) return fail(LLMP_ERR_INVALID_ARG, "llmp_attn_block: null or misaligned x");
    if (d_position & 3) return fail(LLMP_ERR_INVALID_ARG, "llmp_attn_block: misaligned position word");
    const int D = kv->head_dim, qd = c.n_heads * D, kvd = kv->n_kv_heads * D, dim = kv->blk_dim;
    float* q = kv->blk_buf;
    float* attn = q + qd + 2 * kvd;
    float* o = attn + qd;
    float* xp = reinterpret_cast<float*>(x);
    hipStream_t st = pick_stream(stream);
    const bool q8in = kv->blk_input == LLMP_INPUT_Q8_1;
    auto vecp = [&](int slot) -> const float* {
        return static_cast<const float*>(W[slot].mem);
    };

    // 1-2. Pre-norm (fused into the projections' input staging; absent: x as is, the copy
    //      TransformerBlock makes for OLMo2) and the Q/K/V projections with their biases.
    gk::GemvSeg segs[3];
    int types[3];
    const int seg_rows[3] = {qd, kvd, kvd}, seg_off[3] = {0, qd, qd + kvd};
    const int bias_slot[3] = {LLMP_W_Q_BIAS, LLMP_W_K_BIAS, LLMP_W_V_BIAS};
    for (int i = 0; i < 3; ++i) {
        const DevWeight& dw = merged ? W[LLMP_W_QKV] : W[LLMP_W_Q + i];
        segs[i].w = dw.planes;
        if (merged)   // rows seg_off[i].. of the merged matrix
            for (int p = 0; p < 4; ++p)
                if (dw.planes.p[p]) segs[i].w.p[p] = dw.planes.p[p] + (long long)seg_off[i] * dw.planes.pitch[p];
        segs[i].rows = seg_rows[i];
        segs[i].out_off = seg_off[i];
        segs[i].bias = vecp(bias_slot[i]);
        segs[i].fmt = 0;
        types[i] = dw.type;
    }
    // One launch for the three projections when they share a type or form a supported mix
    // of two (a Q4_K_M layer: q, k Q4_K and v Q6_K; GemvSeg::fmt tells each row's format);
    // otherwise one launch per run of consecutive segments with the same type (their rows are
    // contiguous in the q|k|v output).
    int t1 = types[0], t2 = -1;
    for (int i = 1; i < 3; ++i)
        if (types[i] != t1) {
            if (t2 < 0) t2 = types[i];
            else if (types[i] != t2) t2 = -2;
        }
    if (t2 >= 0 && !gemv_pair_supported(t1, t2) && gemv_pair_supported(t2, t1)) std::swap(t1, t2);
    if (t2 >= 0 && gemv_pair_supported(t1, t2)) {
        gk::GemvArgs g{};
        for (int k = 0; k < 3; ++k) {
            g.seg[k] = segs[k];
            g.seg[k].fmt = types[k] == t1 ? 0 : 1;
        }
        g.nseg = 3;
        g.rows_total = qd + 2 * kvd;
        g.cols = dim;
        g.x = xp;
        g.norm_w = vecp(LLMP_W_ATTN_NORM);
        g.eps = c.eps;
        g.out = q;
        LLMP_HIP_CHECK(launch_gemv_pair(g, t1, t2, q8in, st), "block Q/K/V projection launch");
    } else {
        for (int i = 0; i < 3;) {
            int n = 1;
            while (i + n < 3 && types[i + n] == types[i]) ++n;
            gk::GemvArgs g{};
            for (int k = 0; k < n; ++k) {
                g.seg[k] = segs[i + k];
                g.seg[k].out_off = segs[i + k].out_off - segs[i].out_off;
            }
            g.nseg = n;
            g.rows_total = 0;
            for (int k = 0; k < n; ++k) g.rows_total += segs[i + k].rows;
            g.cols = dim;
            g.x = xp;
            g.norm_w = vecp(LLMP_W_ATTN_NORM);
            g.eps = c.eps;
            g.out = q + segs[i].out_off;
            LLMP_HIP_CHECK(launch_gemv(g, types[i], q8in, st), "block Q/K/V projection launch");
            i += n;
        }
    }
    // 3-5. The attention core (QK-norm, RoPE, append, attention) into `attn`.
    const int* dpos = reinterpret_cast<const int*>(d_position);
    if (int rc = enqueue_decode(kv, layer, -1, d_position ? kv->max_seq - 1 : position, dpos,
                                reinterpret_cast<uint64_t>(q), reinterpret_cast<uint64_t>(q + qd),
                                reinterpret_cast<uint64_t>(q + qd + kvd), 0,
                                reinterpret_cast<uint64_t>(attn), splits, stream))
        return rc;
    // 6. Output projection (+ bias), post-norm, residual scale and residual add.
    gk::GemvArgs g{};
    g.seg[0].w = W[LLMP_W_O].planes;
    g.seg[0].rows = dim;
    g.seg[0].bias = vecp(LLMP_W_O_BIAS);
    g.nseg = 1;
    g.rows_total = dim;
    g.cols = qd;
    g.x = attn;
    const float* post = vecp(LLMP_W_POST_ATTN_NORM);
    if (post) {
        g.out = o;
        LLMP_HIP_CHECK(launch_gemv(g, W[LLMP_W_O].type, q8in, st), "block output projection launch");
        LLMP_HIP_CHECK(launch_post_norm_residual(o, post, c.eps, kv->blk_rscale, xp, dim, 1, st),
                       "block post-norm launch");
    } else {
        g.resid = xp;
        g.rscale = kv->blk_rscale;
        LLMP_HIP_CHECK(launch_gemv(g, W[LLMP_W_O].type, q8in, st), "block output projection launch");
    }
    return LLMP_OK;
}

static int enqueue_prefill(KvHandle* kv, int layer, int src_layer, int pos0, int n_tokens,
                           bool in_f32, uint64_t q, uint64_t k, uint64_t v, uint64_t gate,
                           uint64_t out, uint64_t stream, bool use_static);

// The attention half of n_tokens tokens at positions pos0 .. pos0+n_tokens-1 over the rows
// x[t][dim] (LLMEngine.forwardBatch's per-token forwards, LLMEngine.java:1019-1033, with the
// projections batched as speculative-decoding.md:120-140 plans): per group of up to kTokBatch
// tokens, the Q/K/V projections of all of them on the matrix cores (each weight row read once),
// the multi-token attention on fp32 projections (the rows appended exactly as the single-token
// decode appends them), the output projection with its residual epilogue, and the post-norm.
// In the Q8_1 input mode the tokens run one llmp_attn_block call each (that contract's int8 dot
// products have no batched kernel).
int llmp_attn_block_batch(uint64_t handle, int layer, int pos0, int n_tokens, uint64_t x,
                          uint64_t stream) {
    if (int rc = ensure_init()) return rc;
    LLMP_GET_HANDLE(kv, handle);
    if (layer < 0 || layer >= kv->n_layers)
        return fail(LLMP_ERR_OUT_OF_RANGE, "layer %d outside [0, %d)", layer, kv->n_layers);
    if (n_tokens <= 0 || pos0 < 0 || (long long)pos0 + n_tokens > kv->max_seq)
        return fail(LLMP_ERR_OUT_OF_RANGE, "llmp_attn_block_batch: rows [%d, %lld) outside [0, %d)",
                    pos0, (long long)pos0 + n_tokens, kv->max_seq);
    const LayerCfg& c = kv->layers[(size_t)layer];
    if (!c.configured)
        return fail(LLMP_ERR_INVALID_ARG, "layer %d was never configured (llmp_layer_config)", layer);
    const DevWeight* W = c.w;
    const bool merged = W[LLMP_W_QKV].mem != nullptr;
    if (kv->blk_dim == 0 || !W[LLMP_W_O].mem ||
        (!merged && (!W[LLMP_W_Q].mem || !W[LLMP_W_K].mem || !W[LLMP_W_V].mem)))
        return fail(LLMP_ERR_INVALID_ARG, "llmp_attn_block_batch: layer %d lacks projection weights", layer);
    if (!x || (x & 15)) return fail(LLMP_ERR_INVALID_ARG, "llmp_attn_block_batch: null or misaligned x");
    const int D = kv->head_dim, qd = c.n_heads * D, kvd = kv->n_kv_heads * D, dim = kv->blk_dim;
    const bool w_ok = W[LLMP_W_O].tok_ok && (merged ? W[LLMP_W_QKV].tok_ok
                                                     : W[LLMP_W_Q].tok_ok && W[LLMP_W_K].tok_ok &&
                                                           W[LLMP_W_V].tok_ok);
    const bool q8 = kv->blk_input == LLMP_INPUT_Q8_1;
    if (prefill_tile_keys(D) <= 0 || !w_ok) {
        // a head size with decode kernels only, fp32 / bf16 weights beyond fp16's range, or a
        // type without a token-batched kernel
        for (int t = 0; t < n_tokens; ++t)
            if (int rc = enqueue_block(kv, layer, pos0 + t, 0, x + (uint64_t)t * dim * sizeof(float), 0,
                                       stream))
                return rc;
        return LLMP_OK;
    }
    for (int i = 0; i < 3; ++i) {
        const DevWeight& dw = merged ? W[LLMP_W_QKV] : W[LLMP_W_Q + i];
        if (!proj_tok_supported(dw.type))
            return fail(LLMP_ERR_UNSUPPORTED, "llmp_attn_block_batch: GGML type %d", dw.type);
    }
    if (!proj_tok_supported(W[LLMP_W_O].type))
        return fail(LLMP_ERR_UNSUPPORTED, "llmp_attn_block_batch: GGML type %d", W[LLMP_W_O].type);
    const BatchLayout L = batch_layout(kv, qd, kvd);
    if (!kv->blkb_buf || L.total > kv->blkb_bytes)
        return fail(LLMP_ERR_INVALID_ARG, "llmp_attn_block_batch: layer %d weights not uploaded", layer);
    char* base = static_cast<char*>(kv->blkb_buf);
    float* qb = reinterpret_cast<float*>(base + L.q);
    float* kb = reinterpret_cast<float*>(base + L.k);
    float* vb = reinterpret_cast<float*>(base + L.v);
    float* attn = reinterpret_cast<float*>(base + L.attn);
    float* ob = reinterpret_cast<float*>(base + L.o);
    float* sc = reinterpret_cast<float*>(base + L.sc);
    void* q8b = base + L.q8b;
    float* q8d = reinterpret_cast<float*>(base + L.q8d);
    float* q8s = reinterpret_cast<float*>(base + L.q8s);
    hipStream_t st = pick_stream(stream);
    auto vecp = [&](int slot) -> const float* { return static_cast<const float*>(W[slot].mem); };

    // Q/K/V segments: outputs q [K][qd], k [K][kvd], v [K][kvd].
    tk::TokSeg segs[3];
    int types[3];
    const int seg_rows[3] = {qd, kvd, kvd}, seg_off[3] = {0, qd, qd + kvd};
    const int bias_slot[3] = {LLMP_W_Q_BIAS, LLMP_W_K_BIAS, LLMP_W_V_BIAS};
    float* seg_out[3] = {qb, kb, vb};
    for (int i = 0; i < 3; ++i) {
        const DevWeight& dw = merged ? W[LLMP_W_QKV] : W[LLMP_W_Q + i];
        segs[i].w = dw.planes;
        if (merged)
            for (int p = 0; p < 4; ++p)
                if (dw.planes.p[p]) segs[i].w.p[p] = dw.planes.p[p] + (long long)seg_off[i] * dw.planes.pitch[p];
        segs[i].rows = seg_rows[i];
        segs[i].out_off = seg_off[i];
        segs[i].fmt = 0;
        segs[i].bias = vecp(bias_slot[i]);
        segs[i].out = seg_out[i];
        segs[i].out_pitch = seg_rows[i];
        types[i] = dw.type;
    }
    // One launch when the three share a type or form a supported pair (the Q4_K_M mix);
    // otherwise one per run of segments of one type.
    int t1 = types[0], t2 = -1;
    for (int i = 1; i < 3; ++i)
        if (types[i] != t1) {
            if (t2 < 0) t2 = types[i];
            else if (types[i] != t2) t2 = -2;
        }
    if (t2 >= 0 && !proj_tok_pair_supported(t1, t2) && proj_tok_pair_supported(t2, t1)) std::swap(t1, t2);
    const bool paired = t2 >= 0 && proj_tok_pair_supported(t1, t2);
    float* xp = reinterpret_cast<float*>(x);
    for (int t0 = 0; t0 < n_tokens; t0 += kTokBatch) {
        const int K = n_tokens - t0 < kTokBatch ? n_tokens - t0 : kTokBatch;
        float* xc = xp + (size_t)t0 * dim;
        if (K == 1) {   // one token: the single-token launches are faster (27 against 49 µs at C3)
            if (int rc = enqueue_block(kv, layer, pos0 + t0, 0, reinterpret_cast<uint64_t>(xc), 0, stream))
                return rc;
            continue;
        }
        // 1-2. The tokens' pre-norm factors and input range exponents, then the Q/K/V
        //      projections of the normalised inputs.
        // In the Q8_1 mode the tokens' quantised inputs come with the same factors.
        if (q8)
            LLMP_HIP_CHECK(launch_tok_q8(xc, dim, dim, vecp(LLMP_W_ATTN_NORM), c.eps, K, q8b, q8d, q8s, sc, st),
                           "batched block Q8_1 input launch");
        else
            LLMP_HIP_CHECK(launch_tok_prep(xc, dim, dim, vecp(LLMP_W_ATTN_NORM), c.eps, sc, K, st),
                           "batched block input prep launch");
        if (paired || t2 == -1) {
            tk::ProjTokArgs g{};
            for (int k = 0; k < 3; ++k) {
                g.seg[k] = segs[k];
                g.seg[k].fmt = types[k] == t1 ? 0 : 1;
            }
            g.nseg = 3;
            g.rows_total = qd + 2 * kvd;
            g.cols = dim;
            g.K = K;
            g.x = xc;
            g.x_pitch = dim;
            g.norm_w = vecp(LLMP_W_ATTN_NORM);
            g.tok_sc = sc;
            g.eps = c.eps;
            g.q8b = static_cast<const uint4*>(q8b);
            g.q8d = q8d;
            g.q8s = q8s;
            LLMP_HIP_CHECK(launch_proj_tok(g, t1, paired ? t2 : -1, q8, st), "batched block Q/K/V projection launch");
        } else {
            for (int i = 0; i < 3;) {
                int n = 1;
                while (i + n < 3 && types[i + n] == types[i]) ++n;
                tk::ProjTokArgs g{};
                int off = 0;
                for (int k = 0; k < n; ++k) {
                    g.seg[k] = segs[i + k];
                    g.seg[k].out_off = off;
                    off += segs[i + k].rows;
                }
                g.nseg = n;
                g.rows_total = off;
                g.cols = dim;
                g.K = K;
                g.x = xc;
                g.x_pitch = dim;
                g.norm_w = vecp(LLMP_W_ATTN_NORM);
                g.tok_sc = sc;
                g.eps = c.eps;
                g.q8b = static_cast<const uint4*>(q8b);
                g.q8d = q8d;
                g.q8s = q8s;
                LLMP_HIP_CHECK(launch_proj_tok(g, types[i], -1, q8, st), "batched block Q/K/V projection launch");
                i += n;
            }
        }
        // 3-5. Attention of the K tokens (QK-norm, RoPE, exact appends, causal over the cache).
        if (int rc = enqueue_prefill(kv, layer, -1, pos0 + t0, K, true, reinterpret_cast<uint64_t>(qb),
                                     reinterpret_cast<uint64_t>(kb), reinterpret_cast<uint64_t>(vb), 0,
                                     reinterpret_cast<uint64_t>(attn), stream, false))
            return rc;
        // 6. Output projection (+ bias), post-norm, residual scale and residual add.
        tk::ProjTokArgs g{};
        g.seg[0].w = W[LLMP_W_O].planes;
        g.seg[0].rows = dim;
        g.seg[0].bias = vecp(LLMP_W_O_BIAS);
        g.nseg = 1;
        g.rows_total = dim;
        g.cols = qd;
        g.K = K;
        g.x = attn;
        g.x_pitch = qd;
        g.in_range = kv->range(layer);   // |attention output| <= the largest stored |V|
        g.in_range_n = kv->n_kv_heads;
        const bool wo_q8 = q8 && proj_tok_q8_routed(W[LLMP_W_O].type);
        if (wo_q8) {   // the attention output quantised, as the single-token kernel does
            LLMP_HIP_CHECK(launch_tok_q8(attn, qd, qd, nullptr, 0.0f, K, q8b, q8d, q8s, nullptr, st),
                           "batched block Q8_1 attention-output launch");
            g.q8b = static_cast<const uint4*>(q8b);
            g.q8d = q8d;
            g.q8s = q8s;
        }
        const float* post = vecp(LLMP_W_POST_ATTN_NORM);
        if (post) {
            g.seg[0].out = ob;
            g.seg[0].out_pitch = dim;
            LLMP_HIP_CHECK(launch_proj_tok(g, W[LLMP_W_O].type, -1, wo_q8, st), "batched block output projection launch");
            LLMP_HIP_CHECK(launch_post_norm_residual(ob, post, c.eps, kv->blk_rscale, xc, dim, K, st),
                           "batched block post-norm launch");
        } else {
            g.resid = xc;
            g.resid_pitch = dim;
            g.rscale = kv->blk_rscale;
            LLMP_HIP_CHECK(launch_proj_tok(g, W[LLMP_W_O].type, -1, wo_q8, st), "batched block output projection launch");
        }
    }
    return LLMP_OK;
}

int llmp_layer_sinks(uint64_t handle, int layer, const float* sinks) {
    if (int rc = ensure_init()) return rc;
    LLMP_GET_HANDLE(kv, handle);
    if (layer < 0 || layer >= kv->n_layers)
        return fail(LLMP_ERR_OUT_OF_RANGE, "layer %d outside [0, %d)", layer, kv->n_layers);
    LayerCfg& c = kv->layers[(size_t)layer];
    if (!c.configured)
        return fail(LLMP_ERR_INVALID_ARG, "layer %d was never configured (llmp_layer_config)", layer);
    if (!sinks) {
        if (c.d_sinks) (void)hipFree(c.d_sinks);
        c.d_sinks = nullptr;
        return LLMP_OK;
    }
    // The kernels keep scores in the log2 domain (scale folded with log2(e)): so do the sinks.
    std::vector<float> l2((size_t)c.n_heads);
    for (int h = 0; h < c.n_heads; ++h) {
        if (!std::isfinite(sinks[h]))
            return fail(LLMP_ERR_INVALID_ARG, "layer %d: sink %d is not finite", layer, h);
        l2[(size_t)h] = (float)((double)sinks[h] * 1.4426950408889634);
    }
    if (!c.d_sinks)
        LLMP_HIP_CHECK(hipMalloc(&c.d_sinks, l2.size() * sizeof(float)), "hipMalloc(sinks)");
    LLMP_HIP_CHECK(hipMemcpy(c.d_sinks, l2.data(), l2.size() * sizeof(float), hipMemcpyHostToDevice),
                   "hipMemcpy(sinks)");
    return LLMP_OK;
}

int llmp_decode_plan(uint64_t handle, int layer, int position, int splits, int* out_splits,
                     int* out_waves, int* out_rows_per_split, int* out_start) {
    if (int rc = ensure_init()) return rc;
    LLMP_GET_HANDLE(kv, handle);
    if (layer < 0 || layer >= kv->n_layers)
        return fail(LLMP_ERR_OUT_OF_RANGE, "layer %d outside [0, %d)", layer, kv->n_layers);
    if (position < 0 || position >= kv->max_seq)
        return fail(LLMP_ERR_OUT_OF_RANGE, "position %d outside [0, %d)", position, kv->max_seq);
    const LayerCfg& c = kv->layers[(size_t)layer];
    if (!c.configured)
        return fail(LLMP_ERR_INVALID_ARG, "layer %d was never configured (llmp_layer_config)", layer);
    if (splits > kMaxSplits)
        return fail(LLMP_ERR_INVALID_ARG, "splits=%d above the maximum %d", splits, kMaxSplits);
    const Plan p = make_plan(kv, c, position, splits);
    if (out_splits) *out_splits = p.splits;
    if (out_waves) *out_waves = p.waves;
    if (out_rows_per_split) *out_rows_per_split = p.rows_per_split;
    if (out_start) *out_start = p.start;
    return LLMP_OK;
}

// ---- prefill attention -------------------------------------------------------------------------
static int enqueue_prefill(KvHandle* kv, int layer, int src_layer, int pos0, int n_tokens,
                           bool in_f32, uint64_t q, uint64_t k, uint64_t v, uint64_t gate,
                           uint64_t out, uint64_t stream, bool use_static = false);

int llmp_attn_prefill(uint64_t handle, int layer, int pos0, int n_tokens, uint64_t q, uint64_t k,
                      uint64_t v, uint64_t out, uint64_t stream) {
    if (int rc = ensure_init()) return rc;
    LLMP_GET_HANDLE(kv, handle);
    return enqueue_prefill(kv, layer, -1, pos0, n_tokens, false, q, k, v, 0, out, stream);
}

int llmp_attn_prefill_ex(uint64_t handle, int layer, int pos0, int n_tokens, uint64_t q,
                         uint64_t k, uint64_t v, uint64_t gate, uint64_t out, uint64_t stream) {
    if (int rc = ensure_init()) return rc;
    LLMP_GET_HANDLE(kv, handle);
    return enqueue_prefill(kv, layer, -1, pos0, n_tokens, false, q, k, v, gate, out, stream);
}

int llmp_attn_prefill_f32(uint64_t handle, int layer, int pos0, int n_tokens, uint64_t q,
                          uint64_t k, uint64_t v, uint64_t gate, uint64_t out, uint64_t stream) {
    if (int rc = ensure_init()) return rc;
    LLMP_GET_HANDLE(kv, handle);
    return enqueue_prefill(kv, layer, -1, pos0, n_tokens, true, q, k, v, gate, out, stream);
}

int llmp_attn_prefill_f32_static(uint64_t handle, int layer, int pos0, int n_tokens,
                                 uint64_t q, uint64_t k, uint64_t v, uint64_t gate, uint64_t out,
                                 uint64_t stream) {
    if (int rc = ensure_init()) return rc;
    LLMP_GET_HANDLE(kv, handle);
    return enqueue_prefill(kv, layer, -1, pos0, n_tokens, true, q, k, v, gate, out, stream, true);
}

int llmp_attn_prefill_shared(uint64_t handle, int layer, int src_layer, int pos0, int n_tokens,
                             uint64_t q, uint64_t gate, uint64_t out, uint64_t stream) {
    if (int rc = ensure_init()) return rc;
    LLMP_GET_HANDLE(kv, handle);
    if (src_layer < 0)
        return fail(LLMP_ERR_OUT_OF_RANGE, "llmp_attn_prefill_shared: source layer %d", src_layer);
    return enqueue_prefill(kv, layer, src_layer, pos0, n_tokens, false, q, 0, 0, gate, out, stream);
}

int llmp_attn_prefill_shared_f32(uint64_t handle, int layer, int src_layer, int pos0,
                                 int n_tokens, uint64_t q, uint64_t gate, uint64_t out,
                                 uint64_t stream) {
    if (int rc = ensure_init()) return rc;
    LLMP_GET_HANDLE(kv, handle);
    if (src_layer < 0)
        return fail(LLMP_ERR_OUT_OF_RANGE, "llmp_attn_prefill_shared_f32: source layer %d",
                    src_layer);
    return enqueue_prefill(kv, layer, src_layer, pos0, n_tokens, true, q, 0, 0, gate, out, stream);
}

// src_layer >= 0: shared-KV layer (as in enqueue_decode): attention over src_layer's rows,
// which must already hold the prompt's rows; no append.  in_f32: q/k/v are fp32 (the CPU
// path's projections), else bf16 bits.
static int enqueue_prefill(KvHandle* kv, int layer, int src_layer, int pos0, int n_tokens,
                           bool in_f32, uint64_t q, uint64_t k, uint64_t v, uint64_t gate,
                           uint64_t out, uint64_t stream, bool use_static) {
    if (layer < 0 || layer >= kv->n_layers)
        return fail(LLMP_ERR_OUT_OF_RANGE, "layer %d outside [0, %d)", layer, kv->n_layers);
    if (src_layer >= kv->n_layers)
        return fail(LLMP_ERR_OUT_OF_RANGE, "source layer %d outside [0, %d)", src_layer,
                    kv->n_layers);
    const bool shared = src_layer >= 0;
    const int kv_layer = shared ? src_layer : layer;
    if (n_tokens <= 0 || pos0 < 0 || (long long)pos0 + n_tokens > kv->max_seq)
        return fail(LLMP_ERR_OUT_OF_RANGE, "prefill rows [%d, %lld) outside [0, %d)", pos0,
                    (long long)pos0 + n_tokens, kv->max_seq);
    const LayerCfg& c = kv->layers[(size_t)layer];
    if (!c.configured)
        return fail(LLMP_ERR_INVALID_ARG, "layer %d was never configured (llmp_layer_config)", layer);
    if (!q || !out || (!shared && (!k || !v)))
        return fail(LLMP_ERR_INVALID_ARG, "llmp_attn_prefill: null buffer");
    if (prefill_tile_keys(kv->head_dim) <= 0)
        return fail(LLMP_ERR_UNSUPPORTED, "llmp_attn_prefill: head_dim %d (decode only)",
                    kv->head_dim);
    if ((q | k | v) & (in_f32 ? 3 : 1) || out & 15 || gate & 3)
        return fail(LLMP_ERR_INVALID_ARG,
                    "llmp_attn_prefill: misaligned q/k/v (%d B), gate (4 B) or out (16 B)",
                    in_f32 ? 4 : 2);
    const int D = kv->head_dim, Hkv = kv->n_kv_heads, group = c.kgroup;
    pk::PrefillArgs a{};
    a.kv_rep = c.krep;
    a.q = reinterpret_cast<const void*>(q);
    a.k = reinterpret_cast<const void*>(k);
    a.v = reinterpret_cast<const void*>(v);
    a.in_f32 = in_f32 ? 1 : 0;
    if (kv->q8()) {
        a.kq = kv->kq(kv_layer);
        a.ks = kv->ks(kv_layer);
        a.vq = kv->vq(kv_layer);
        a.vs = kv->vs(kv_layer);
        a.q8_trunc = kv->dtype == LLMP_KV_Q8_0_TRUNC;
    } else {
        a.kc = kv->k_plane(kv_layer);
        a.vc = kv->v_plane(kv_layer);
    }
    a.norm_seq = (c.norm_mode & LLMP_NORM_SEQUENTIAL) != 0;
    a.v_norm = (c.norm_mode & LLMP_NORM_V) != 0;
    a.head_stride = (long long)kv->max_seq * D;
    a.range = kv->range(kv_layer);
    if (c.rope_sel != LLMP_ROPE_SEL_NONE) {
        const RopeTable& t = kv->rope[c.rope_sel];
        if (!t.d_cos)
            return fail(LLMP_ERR_INVALID_ARG, "layer %d selects a RoPE table never uploaded", layer);
        a.cos_t = t.d_cos;
        a.sin_t = t.d_sin;
        a.half_rope = t.half;
    }
    a.qnw = c.d_qnw;
    a.knw = c.d_knw;
    a.sinks = c.d_sinks;
    a.gate = reinterpret_cast<const float*>(gate);
    a.out = reinterpret_cast<float*>(out);
    a.pos0 = pos0;
    a.P = n_tokens;
    a.Hq = c.n_heads;
    a.Hkv = Hkv;
    a.rope_type = c.rope_type;
    a.window = (c.window > 0 && !c.is_global) ? c.window : 0;
    a.eps = c.eps;
    const float scale = c.scale > 0.0f ? c.scale : (float)(1.0 / std::sqrt((double)D));
    const float log2e = 1.4426950408889634f;
    if (c.softcap > 0.0f) {
        a.qk_scale = scale;
        a.softcap = c.softcap;
        a.softcap_log2e = c.softcap * log2e;
        a.inv_softcap = 1.0f / c.softcap;
    } else {
        a.qk_scale = scale * log2e;
    }
    hipStream_t st = pick_stream(stream);
    // Key tiles any query of this call attends: from the first query's window start (or 0) to
    // the last prompt row.  Their images live in the handle's workspace, grown when a call
    // needs more (a growth synchronises the device; the size only depends on the row range).
    const int TK = prefill_tile_keys(D);
    const int kbeg_min = a.window > 0 ? std::max(0, pos0 - a.window + 1) : 0;
    const int tile0 = kbeg_min / TK, tile_last = (pos0 + n_tokens - 1) / TK;
    const int n_tiles = tile_last - tile0 + 1;
    const int ksplit = prefill_key_splits(n_tokens, pos0, a.window, Hkv * c.krep, group, D, G().n_cu);
    const size_t ws_bytes =
        ksplit == 1 ? (size_t)Hkv * (size_t)n_tiles * prefill_tile_bytes(D) : 0;
    const size_t part_bytes =
        ksplit > 1
            ? (size_t)ksplit * (size_t)n_tokens * (size_t)c.n_heads * (size_t)(D + 2) * sizeof(float)
            : 0;
    void* ws = nullptr;
    if (use_static) {
        // The whole workspace (tile images, or split-K partials) in the static array: no
        // allocation, no profiling events.
        const size_t need = ksplit > 1 ? part_bytes : ws_bytes;
        if (need > (size_t)LLMP_PREFILL_STATIC_BYTES)
            return fail(LLMP_ERR_INVALID_ARG,
                        "llmp_attn_prefill_f32_static: the call needs %zu bytes of workspace; the "
                        "static scratch holds %u (fewer tokens per call, or llmp_attn_prefill_f32)",
                        need, (unsigned)LLMP_PREFILL_STATIC_BYTES);
        void* sp = G().scratch;
        if (!sp) return fail(LLMP_ERR_NOT_INIT, "llmp_attn_prefill_f32_static: no scratch address");
        if (ksplit > 1) {
            a.part_o = static_cast<float*>(sp);
            a.part_ml = a.part_o + (size_t)ksplit * n_tokens * c.n_heads * D;
        } else {
            ws = sp;
        }
        if (!shared) LLMP_HIP_CHECK(launch_prefill_append(a, D, st), "prefill append launch");
        if (ksplit == 1)
            LLMP_HIP_CHECK(launch_prefill_tiles(a, D, ws, tile0, n_tiles, pos0 + n_tokens, st),
                           "prefill tile launch");
        LLMP_HIP_CHECK(launch_prefill_attn(a, D, group, ws, tile0, n_tiles, G().n_cu, ksplit, st),
                       "prefill attention launch");
        return LLMP_OK;
    }
    if (ws_bytes > kv->prefill_ws_bytes) {
        if (kv->prefill_ws) {
            LLMP_HIP_CHECK(hipStreamSynchronize(st), "hipStreamSynchronize");
            (void)hipFree(kv->prefill_ws);
            kv->prefill_ws = nullptr;
            kv->prefill_ws_bytes = 0;
        }
        hipError_t e = hipMalloc(&kv->prefill_ws, ws_bytes);
        if (e == hipErrorOutOfMemory)
            return fail(LLMP_ERR_OUT_OF_MEMORY, "llmp_attn_prefill: %zu-byte tile workspace", ws_bytes);
        LLMP_HIP_CHECK(e, "hipMalloc(prefill workspace)");
        kv->prefill_ws_bytes = ws_bytes;
    }
    // Key splits (short prompts after a long prefix) and their partials buffer.
    if (ksplit > 1) {
        if (part_bytes > kv->prefill_part_bytes) {
            if (kv->prefill_part) {
                LLMP_HIP_CHECK(hipStreamSynchronize(st), "hipStreamSynchronize");
                (void)hipFree(kv->prefill_part);
                kv->prefill_part = nullptr;
                kv->prefill_part_bytes = 0;
            }
            hipError_t e = hipMalloc(&kv->prefill_part, part_bytes);
            if (e == hipErrorOutOfMemory)
                return fail(LLMP_ERR_OUT_OF_MEMORY, "llmp_attn_prefill: %zu-byte split workspace",
                            part_bytes);
            LLMP_HIP_CHECK(e, "hipMalloc(prefill partials)");
            kv->prefill_part_bytes = part_bytes;
        }
        a.part_o = kv->prefill_part;
        a.part_ml = kv->prefill_part + (size_t)ksplit * n_tokens * c.n_heads * D;
    }
    hipEvent_t e0 = nullptr, e1 = nullptr, e2 = nullptr, e3 = nullptr;
    if (kv->prof_on) {
        for (hipEvent_t* e : {&e0, &e1, &e2, &e3})
            if (int rc = prof_event(kv, e)) return rc;
        LLMP_HIP_CHECK(hipEventRecord(e0, st), "hipEventRecord");
    }
    if (!shared) LLMP_HIP_CHECK(launch_prefill_append(a, D, st), "prefill append launch");
    if (kv->prof_on) {
        LLMP_HIP_CHECK(hipEventRecord(e1, st), "hipEventRecord");
        kv->prof_pending[LLMP_PROF_PREFILL_APPEND].push_back({e0, e1});
        LLMP_HIP_CHECK(hipEventRecord(e2, st), "hipEventRecord");
    }
    if (ksplit == 1)   // split launches stage straight from the cache (no images)
        LLMP_HIP_CHECK(launch_prefill_tiles(a, D, kv->prefill_ws, tile0, n_tiles, pos0 + n_tokens, st),
                       "prefill tile launch");
    LLMP_HIP_CHECK(launch_prefill_attn(a, D, group, kv->prefill_ws, tile0, n_tiles, G().n_cu,
                                       ksplit, st),
                   "prefill attention launch");
    if (kv->prof_on) {
        LLMP_HIP_CHECK(hipEventRecord(e3, st), "hipEventRecord");
        kv->prof_pending[LLMP_PROF_PREFILL_ATTN].push_back({e2, e3});
    }
    return LLMP_OK;
}

// ---- graph capture ---------------------------------------------------------------------------------
int llmp_graph_begin(uint64_t stream) {
    if (int rc = ensure_init()) return rc;
    {
        std::lock_guard<std::mutex> lk(G().mu);
        for (auto& kv : G().handles)
            if (kv.second->prof_on)
                return fail(LLMP_ERR_INVALID_ARG, "llmp_graph_begin: turn profiling off before capturing");
    }
    LLMP_HIP_CHECK(hipStreamBeginCapture(pick_stream(stream), hipStreamCaptureModeThreadLocal),
                   "hipStreamBeginCapture");
    return LLMP_OK;
}

int llmp_graph_end(uint64_t stream, uint64_t* graph) {
    if (int rc = ensure_init()) return rc;
    if (!graph) return fail(LLMP_ERR_INVALID_ARG, "llmp_graph_end: null out");
    hipGraph_t g = nullptr;
    LLMP_HIP_CHECK(hipStreamEndCapture(pick_stream(stream), &g), "hipStreamEndCapture");
    hipGraphExec_t ge = nullptr;
    hipError_t e = hipGraphInstantiate(&ge, g, nullptr, nullptr, 0);
    (void)hipGraphDestroy(g);
    LLMP_HIP_CHECK(e, "hipGraphInstantiate");
    *graph = reinterpret_cast<uint64_t>(ge);
    return LLMP_OK;
}

int llmp_graph_launch(uint64_t graph, uint64_t stream) {
    if (int rc = ensure_init()) return rc;
    if (!graph) return fail(LLMP_ERR_INVALID_ARG, "llmp_graph_launch: null graph");
    LLMP_HIP_CHECK(hipGraphLaunch(reinterpret_cast<hipGraphExec_t>(graph), pick_stream(stream)),
                   "hipGraphLaunch");
    return LLMP_OK;
}

int llmp_graph_destroy(uint64_t graph) {
    if (int rc = ensure_init()) return rc;
    if (!graph) return fail(LLMP_ERR_INVALID_ARG, "llmp_graph_destroy: null graph");
    LLMP_HIP_CHECK(hipGraphExecDestroy(reinterpret_cast<hipGraphExec_t>(graph)), "hipGraphExecDestroy");
    return LLMP_OK;
}

// ---- profiling ---------------------------------------------------------------------------------
int llmp_profile_enable(uint64_t handle, int on) {
    if (int rc = ensure_init()) return rc;
    LLMP_GET_HANDLE(kv, handle);
    kv->prof_on = on != 0;
    return LLMP_OK;
}

int llmp_profile_read(uint64_t handle, int kind, int* count, double* total_ms) {
    if (int rc = ensure_init()) return rc;
    LLMP_GET_HANDLE(kv, handle);
    if (kind < 0 || kind >= LLMP_PROF_KINDS)
        return fail(LLMP_ERR_INVALID_ARG, "llmp_profile_read: kind %d", kind);
    if (int rc = prof_fold(kv, kind)) return rc;
    if (count) *count = (int)kv->prof_count[kind];
    if (total_ms) *total_ms = kv->prof_ms[kind];
    return LLMP_OK;
}

int llmp_profile_reset(uint64_t handle) {
    if (int rc = ensure_init()) return rc;
    LLMP_GET_HANDLE(kv, handle);
    for (int kind = 0; kind < LLMP_PROF_KINDS; ++kind) {
        if (int rc = prof_fold(kv, kind)) return rc;
        kv->prof_ms[kind] = 0.0;
        kv->prof_count[kind] = 0;
    }
    return LLMP_OK;
}

// ---- utilities -----------------------------------------------------------------------------------
int llmp_copy_kernel(uint64_t dst, uint64_t src, uint64_t bytes, uint64_t stream) {
    if (int rc = ensure_init()) return rc;
    if (!dst || !src || bytes % 16 != 0)
        return fail(LLMP_ERR_INVALID_ARG, "llmp_copy_kernel: needs non-null 16-byte multiples");
    LLMP_HIP_CHECK(launch_copy(reinterpret_cast<void*>(dst), reinterpret_cast<const void*>(src),
                               (size_t)bytes, pick_stream(stream)),
                   "copy kernel launch");
    return LLMP_OK;
}

}  // extern "C"
