// colizig_hip.hip - libcolizig_hip.so: colizig's block-FP8 MoE expert path on
// MI355X (gfx950), behind colizig's src/backend C-ABI (include/colizig_hip.h).
//
// One global context (as the CUDA DLL, colizig_cuda.cu:80-106), one HIP
// stream at default priority.  Every entry point saves/restores the host
// MXCSR (colizig_cuda.cu:22-29): the GPU runtime must not leak FTZ/DAZ into
// the engine's CPU float math.
#include "cz_grouped.h"
#include "cz_fused.h"
#include "cz_lru.h"
#include "cz_sched.h"
#include "cz_plan.h"
#include "colizig_hip.h"

#include <xmmintrin.h>

#include <algorithm>
#include <cstdio>
#include <cstring>
#include <mutex>
#include <string>
#include <type_traits>
#include <unordered_map>
#include <vector>

namespace {

struct CsrGuard {
    unsigned saved;
    CsrGuard() : saved(_mm_getcsr()) {}
    ~CsrGuard() { _mm_setcsr(saved); }
};

inline uint32_t nblk(uint32_t x) { return (x + CZ_BLOCK - 1) / CZ_BLOCK; }

// ---- keyed HBM weight cache for the per-matmul ABI (colizig_cuda.cu:80-169)
struct Slot {
    uint64_t key = 0;  // 0 = free
    void *w = nullptr;
    size_t wcap = 0;
    void *s = nullptr;
    size_t scap = 0;
    uint64_t clock = 0;
    int I = 0, O = 0;  // the resident matrix's shape
    int bf16 = 0;      // 1: BF16 rows (no scales), 0: block-FP8
};
constexpr size_t kMaxSlots = 4096;

// ---- one registered MoE layer
struct LayerHost {
    colizig_dims d{};
    float *router = nullptr;
    uint8_t *ew = nullptr;
    float *es = nullptr;
    uint8_t *sw = nullptr;
    float *ss = nullptr;
    float *shg = nullptr;
    float *rbias = nullptr;  // optional router bias [E]
    unsigned long long *usage = nullptr;  // [E] routed-selection counters (ExpertUsage row)
    uint16_t *router_bf16 = nullptr;      // BF16 router [E][H] (NativeMatrix bf16); `router` is then null
    // a NativeMatrix shared expert (f32 or BF16 rows, moe.zig:300-303,
    // 467-479), evaluated by its own GEMVs after the routed experts
    int shn_dtype = -1;                   // 0 f32, 1 bf16, -1 none (FP8 or no shared expert)
    void *shn_gate = nullptr, *shn_up = nullptr, *shn_down = nullptr;
    // streamed from host memory: experts live in pinned host memory (two
    // slabs in the ew/es layout, or one packed slab of [weights | scales] per
    // expert) and in slots of the HBM expert pool while cached
    const uint8_t *host_ew = nullptr;
    const float *host_es = nullptr;
    const uint8_t *host_packed = nullptr;
    uint64_t pool_ew_stride = 0, pool_es_stride = 0;  // a pool slot, in bytes / floats
    int32_t *slot_map_dev = nullptr;   // [E] device copy of slot_map
    int32_t *slot_map_stage = nullptr; // [E] pinned staging of the upload
    std::vector<int32_t> slot_map;     // [E] pool slot or -1
    std::vector<uint8_t> loaded;
    uint32_t nloaded = 0;
    bool shared_set = false;
    // changes whenever a device buffer the kernels take as an argument is
    // replaced (re-registration, router bias added or removed, streaming):
    // a HIP graph captured before then holds stale pointers
    uint64_t gen = 0;

    uint64_t ew_stride() const { return 3ull * d.inter * d.hidden; }
    uint64_t es_stride() const { return 3ull * nblk(d.inter) * nblk(d.hidden); }
    uint64_t sw_bytes() const { return 3ull * d.shared_inter * d.hidden; }
    uint64_t ss_floats() const { return 3ull * nblk(d.shared_inter) * nblk(d.hidden); }
    bool streamed() const { return host_ew != nullptr || host_packed != nullptr; }
    bool ready() const { return (streamed() || nloaded == d.experts) && (d.shared_inter == 0 || shared_set); }
    LayerDev dev() const {
        LayerDev L{};
        L.H = d.hidden;
        L.E = d.experts;
        L.K = d.topk;
        L.I = d.inter;
        L.SI = d.shared_inter;
        L.norm_topk = d.norm_topk;
        L.nbH = nblk(d.hidden);
        L.nbI = nblk(d.inter);
        L.nbSI = nblk(d.shared_inter);
        L.router = router;
        L.ew = ew;
        L.es = es;
        L.ew_stride = streamed() ? pool_ew_stride : ew_stride();
        L.es_stride = streamed() ? pool_es_stride : es_stride();
        L.sw = sw;
        L.ss = ss;
        L.sh_gate = shg;
        L.router_bias = rbias;
        L.slot_map = slot_map_dev;
        L.usage = usage;
        L.router_bf16 = router_bf16;
        if (shn_dtype >= 0) {  // the routed-expert kernels see no shared expert
            L.SI = 0;
            L.nbSI = 0;
            L.sw = nullptr;
            L.ss = nullptr;
            L.sh_gate = nullptr;
        }
        return L;
    }
};

// ---- device scratch of a forward (grow-only; retired buffers live until
// shutdown so a captured graph never points at freed memory)
struct Work {
    float *xin = nullptr, *out = nullptr, *xn = nullptr, *logits = nullptr, *gates = nullptr, *sgate = nullptr;
    float *h = nullptr, *hs = nullptr;
    float *ng = nullptr, *nu = nullptr, *no = nullptr, *nsg = nullptr;  // NativeMatrix shared expert
    size_t cap_ng = 0, cap_nu = 0, cap_no = 0, cap_nsg = 0;
    uint32_t *idx = nullptr;
    size_t cap_xin = 0, cap_out = 0, cap_xn = 0, cap_logits = 0, cap_idx = 0, cap_gates = 0, cap_sgate = 0,
           cap_h = 0, cap_hs = 0;
    // grouped regime
    uint32_t *counts = nullptr, *offsets = nullptr, *sorted_slot = nullptr, *slot_pos = nullptr,
             *tok_order = nullptr, *tile_expert = nullptr, *tile_row0 = nullptr, *ntiles = nullptr;
    float *o = nullptr, *os = nullptr;
    uint8_t *xq = nullptr, *xe = nullptr, *hq = nullptr, *he = nullptr, *hsq = nullptr, *hse = nullptr;
    size_t cap_xq = 0, cap_xe = 0, cap_hq = 0, cap_he = 0, cap_hsq = 0, cap_hse = 0;
    _Float16 *xh = nullptr, *xl = nullptr, *hh = nullptr, *hl = nullptr, *hsh = nullptr, *hsl = nullptr;
    size_t cap_counts = 0, cap_offsets = 0, cap_sorted = 0, cap_slot_pos = 0, cap_tok_order = 0, cap_tiles = 0,
           cap_tiles2 = 0, cap_ntiles = 0, cap_o = 0, cap_os = 0, cap_xh = 0, cap_xl = 0, cap_hh = 0, cap_hl = 0,
           cap_hsh = 0, cap_hsl = 0;
};

// ---- HBM expert pool of the streaming tier: fixed-size slots (one expert's
// gate|up|down weights and scales each), a global LRU over (layer, expert)
// keys, a side stream for the host->HBM fills.  ExpertCache (moe.zig:121-249)
// redesigned for one pool shared by every streamed layer.
constexpr size_t kSchedCapacity = 64;  // queued prefetches at most (io.zig:62-63 bounded queue)
constexpr int kCopyStreams = 3;        // copy (prefetch), copy_hi (demand), copy2 (prefetch)

struct StreamPool {
    bool on = false;
    colizig_dims d{};
    uint64_t w_slot = 0, s_slot = 0;  // bytes of an expert's weights / floats of its scales
    uint64_t slot_bytes = 0;          // one slot: [weights | scales], a multiple of 16 bytes
    uint8_t *base = nullptr;          // nslots slots
    uint32_t nslots = 0;
    std::vector<uint64_t> key;         // 1 + (layer << 32 | expert), 0 = free
    std::vector<uint64_t> used;        // LRU clock of the last use (or fill)
    std::vector<uint32_t> prefetched;  // stats epoch + 1 of a prefetch fill not used since (0: none)
    uint32_t stats_epoch = 0;          // colizig_hip_stream_stats_reset opens a new one
    std::vector<uint32_t> pin_epoch;   // slot is needed by the layer in flight
    std::unordered_map<uint64_t, uint32_t> where;
    uint64_t clock = 0;
    uint32_t epoch = 0;
    hipStream_t copy = nullptr;
    hipEvent_t ev_idx = nullptr, ev_copy = nullptr, ev_copy_hi = nullptr, ev_copy2 = nullptr;
    uint32_t *h_idx = nullptr;         // pinned routing read-back (host-coherent)
    size_t h_idx_cap = 0;
    uint32_t *h_flag = nullptr;        // host-coherent: sequence number of the last one-token routing written
    uint32_t seq = 0;
    // routing prediction (one token), bit 0: the next streamed layer's from
    // the current layer's router input; bit 1: every later streamed layer's
    // from the chain's first router input; bit 2 (with bit 1): those later
    // layers in speculative runs (run_spec_layers).  Device scratch of the predicted
    // routing, the picks in host-coherent memory and their sequence numbers.
    int predict_mode = 6;
    float *pred_logits = nullptr, *pred_gates = nullptr, *pred_sgate = nullptr;
    uint32_t *pred_idx = nullptr, *pred_tord = nullptr;
    uint32_t *route_count = nullptr;  // the router kernel's block counter (one-token routing), kept at zero
    uint32_t *h_pred = nullptr, *h_pflag = nullptr;
    uint32_t pseq = 0;
    std::unordered_map<uint32_t, std::vector<uint32_t>> pred_ids;  // layer -> its next-layer prediction
    cz::PredStats next_stats;          // next-layer prediction accuracy
    float *tok_logits = nullptr, *tok_gates = nullptr;
    uint32_t *tok_idx = nullptr, *tok_tord = nullptr;
    size_t tok_cap = 0;                // rows (layers) of the token-level buffers
    const float **tok_ptr_stage = nullptr;  // pinned [2][rows]: routers, biases
    const float **tok_ptr_dev = nullptr;
    uint32_t *h_tok = nullptr, *h_tflag = nullptr;
    uint32_t tseq = 0;
    std::unordered_map<uint32_t, std::vector<uint32_t>> tok_ids;   // layer -> its token-level prediction
    cz::PredStats tok_stats;
    // Fills go on three copy streams: prefetches alternate between copy and
    // copy2 (a fill starts while the one before it on the other stream
    // finishes, so the link does not idle between fills), demand fills (a
    // layer's misses) go on copy_hi, so a miss does not queue behind the
    // prefetches.  Per slot: the event recorded after its latest fill, that
    // fill's sequence number and its stream.  The compute stream has waited
    // for every fill of copy stream s up to waited[s] (each stream is in
    // order).
    hipStream_t copy_hi = nullptr, copy2 = nullptr;
    std::vector<hipEvent_t> slot_ev;
    std::vector<uint64_t> fill_seq;
    std::vector<uint8_t> fill_sid;
    uint64_t fill_counter = 0, waited[kCopyStreams] = {0, 0, 0};
    uint32_t prefetch_rr = 0;  // the stream of the next prefetch fill
    hipStream_t copy_stream(uint8_t sid) const { return sid == 1 ? copy_hi : sid == 2 ? copy2 : copy; }
    void all_waited() {
        for (uint64_t &w : waited) w = fill_counter;
    }
    cz::LastTokenPredictor last_pred{8};
    cz::Scheduler sched{kSchedCapacity};
    cz::SlotLru lru;                   // held slots in order of last use, and the free ones
    bool log_on = false;
    std::vector<uint32_t> log;         // policy ops, 4 words each (op, layer, expert, result)
    // counters (CacheStats, moe.zig:121-139)
    uint64_t hits = 0, misses = 0, loads = 0, evictions = 0, prefetch_issued = 0, prefetch_hits = 0,
             prefetch_wasted = 0, bytes_h2d = 0;
    // routing prediction bit 2 (with bit 1): the later layers of a token run
    // with the host off their path (run_spec_layers).  Device stop word, the
    // run's picks ([layers][K]) and their pinned read-back (stop word first)
    uint32_t *stop_dev = nullptr, *spec_idx_dev = nullptr, *h_spec = nullptr;
    size_t spec_cap = 0;               // picks the buffers hold
    int32_t *spec_tab_dev = nullptr, *h_spec_tab = nullptr;  // the run's slot maps [layers][E], one upload
    size_t spec_tab_cap = 0;
    uint64_t spec_layers = 0, spec_stops = 0;  // layers run that way; runs a missing slot stopped
};

// ---- one-launch-per-layer batch-1 decode (cz_fused.h): its device state.
// Grow-only like Work: captured graphs hold these pointers.
struct FusedState {
    bool enabled = true;             // colizig_hip_set_fused_decode
    int cus = 0;                     // compute units of the device
    float *r = nullptr;              // [2][H] residual stream (layer inputs), ping-pong
    float *p = nullptr;              // [2][8][H] per-XCD partial outputs, ping-pong
    float *zero = nullptr;           // [8][H] zeros: the first layer's partials
    unsigned long long *lgx = nullptr;  // [8][E] tagged logits
    unsigned long long *hx = nullptr;   // [K*I] tagged gated products
    uint32_t *pred = nullptr;        // [2][64] predicted experts of the next layer, ping-pong
    unsigned long long *lgpx = nullptr;  // [E] tagged next-layer logits
    unsigned long long *pstat = nullptr;  // [2] slots predicted, predictions picked
    unsigned long long *spec_pstat = nullptr;  // [2] the same for the streaming tier's speculative runs
    int predict = 1;                 // colizig_hip_set_fused_predict
    uint32_t *run = nullptr;         // chain-run counter
    uint32_t *err_host = nullptr;    // host-coherent error word
    uint32_t *err_dev = nullptr;     // its device address
    size_t cap_h = 0, cap_e = 0, cap_ki = 0;
    bool placement_ok = false;       // the init census found the workgroup placement the kernel needs
    int fault_pos = -1;              // test hook: the chain position whose polls never match
};

struct Ctx {
    int inited = 0;
    char name[192] = {0};
    hipStream_t stream = nullptr;
    // per-matmul ABI buffers
    void *d_x = nullptr, *d_y = nullptr, *d_w = nullptr, *d_s = nullptr;
    size_t d_x_cap = 0, d_y_cap = 0, d_w_cap = 0, d_s_cap = 0;
    void *h_stage = nullptr;  // pinned staging for x / y
    size_t h_stage_cap = 0;
    // keyed cache
    uint64_t budget = 0, used = 0, lru = 0;
    std::vector<Slot> slots;
    std::unordered_map<uint64_t, int> by_key;
    uint64_t hits = 0, misses = 0, uploaded = 0;
    // MoE layers
    std::unordered_map<uint32_t, LayerHost> layers;
    Work work;
    std::vector<void *> retired;
    std::unordered_map<int64_t, hipGraphExec_t> graphs;
    std::unordered_map<int64_t, hipGraph_t> graph_defs;
    // (layer, generation) of every layer a graph captured
    std::unordered_map<int64_t, std::vector<std::pair<uint32_t, uint64_t>>> graph_layers;
    uint64_t layer_gen = 0;
    std::unordered_map<int64_t, hipEvent_t> events;
    int64_t next_handle = 1;
    StreamPool pool;
    FusedState fused;
    bool prefill_fp8 = true;   // grouped GEMMs on FP8 MFMA (k_gg8), else f16 (k_gg)
};

Ctx g;
std::recursive_mutex g_mu;
char g_err[512] = {0};

#define CZ_CHECK(call, rc)                                                   \
    do {                                                                     \
        hipError_t e_ = (call);                                              \
        if (e_ != hipSuccess) {                                              \
            snprintf(g_err, sizeof g_err, "%s: %s", #call, hipGetErrorString(e_)); \
            return (rc);                                                     \
        }                                                                    \
    } while (0)

int ensure_dev(void **p, size_t *cap, size_t need) {
    if (*cap >= need) return 0;
    if (*p) {
        if (hipFree(*p) != hipSuccess) {}
    }
    *p = nullptr;
    *cap = 0;
    if (hipMalloc(p, need) != hipSuccess) {
        *p = nullptr;
        return -1;
    }
    *cap = need;
    return 0;
}

int ensure_host(size_t need) {
    if (g.h_stage_cap >= need) return 0;
    if (g.h_stage) (void)hipHostFree(g.h_stage);
    g.h_stage = nullptr;
    g.h_stage_cap = 0;
    if (hipHostMalloc(&g.h_stage, need, hipHostMallocDefault) != hipSuccess) {
        g.h_stage = nullptr;
        return -1;
    }
    g.h_stage_cap = need;
    return 0;
}

template <typename T>
int grow(T **p, size_t *cap, size_t need) {
    if (*cap >= need) return 0;
    if (*p) g.retired.push_back((void *)*p);
    *p = nullptr;
    *cap = 0;
    void *q = nullptr;
    if (hipMalloc(&q, need * sizeof(T)) != hipSuccess) return -1;
    *p = (T *)q;
    *cap = need;
    return 0;
}

// Scratch for S tokens of a layer with dims d (max over callers).
int ensure_work(const colizig_dims &d, int S) {
    Work &w = g.work;
    const size_t s = (size_t)S;
    if (grow(&w.xin, &w.cap_xin, s * d.hidden) || grow(&w.out, &w.cap_out, s * d.hidden) ||
        grow(&w.xn, &w.cap_xn, s * d.hidden) || grow(&w.logits, &w.cap_logits, s * d.experts) ||
        grow(&w.idx, &w.cap_idx, s * d.topk) || grow(&w.gates, &w.cap_gates, s * d.topk) ||
        grow(&w.sgate, &w.cap_sgate, s) || grow(&w.h, &w.cap_h, s * d.topk * (size_t)d.inter) ||
        grow(&w.hs, &w.cap_hs, std::max<size_t>(1, s * d.shared_inter)) ||
        (d.shared_inter && (grow(&w.ng, &w.cap_ng, s * d.shared_inter) || grow(&w.nu, &w.cap_nu, s * d.shared_inter) ||
                            grow(&w.no, &w.cap_no, s * d.hidden) || grow(&w.nsg, &w.cap_nsg, s)))) {
        snprintf(g_err, sizeof g_err, "scratch allocation failed (S=%d)", S);
        return -2;
    }
    return 0;
}

// The grouped (dispatch + MFMA) regime serves S >= kGroupedMinTokens when the
// shapes tile by 128 and the slots fit the dispatch workgroup.
constexpr int kGroupedMinTokens = 16;

// Upper bound on the M-tiles of the grouped GEMMs: sum_e ceil(n_e/32) <=
// S*K/32 + min(E, S*K).
uint32_t grouped_max_tiles(const colizig_dims &d, int S) {
    const uint32_t sk = (uint32_t)S * d.topk;
    return sk / CZ_GG_M + std::min(d.experts, sk) + 1;
}

int ensure_work_grouped(const colizig_dims &d, int S) {
    Work &w = g.work;
    const size_t s = (size_t)S, sk = s * d.topk, mt = grouped_max_tiles(d, S);
    if (grow(&w.counts, &w.cap_counts, (size_t)d.experts) || grow(&w.offsets, &w.cap_offsets, (size_t)d.experts + 1) ||
        grow(&w.sorted_slot, &w.cap_sorted, sk) || grow(&w.slot_pos, &w.cap_slot_pos, sk) ||
        grow(&w.tok_order, &w.cap_tok_order, sk) || grow(&w.tile_expert, &w.cap_tiles, mt) ||
        grow(&w.tile_row0, &w.cap_tiles2, mt) || grow(&w.ntiles, &w.cap_ntiles, (size_t)1) ||
        grow(&w.o, &w.cap_o, sk * d.hidden) || grow(&w.os, &w.cap_os, std::max<size_t>(1, s * d.hidden)) ||
        // the GEMM operands of the active mode only: f16 hi + lo splits, or
        // three E4M3 terms and their exponents
        (!g.prefill_fp8 &&
         (grow(&w.xh, &w.cap_xh, s * d.hidden) || grow(&w.xl, &w.cap_xl, s * d.hidden) ||
          grow(&w.hh, &w.cap_hh, sk * d.inter) || grow(&w.hl, &w.cap_hl, sk * d.inter) ||
          grow(&w.hsh, &w.cap_hsh, std::max<size_t>(1, s * d.shared_inter)) ||
          grow(&w.hsl, &w.cap_hsl, std::max<size_t>(1, s * d.shared_inter)))) ||
        (g.prefill_fp8 &&
         (grow(&w.xq, &w.cap_xq, 3 * s * d.hidden) || grow(&w.xe, &w.cap_xe, 3 * s * d.hidden / 32) ||
          grow(&w.hq, &w.cap_hq, 3 * sk * d.inter) || grow(&w.he, &w.cap_he, 3 * sk * d.inter / 32) ||
          grow(&w.hsq, &w.cap_hsq, std::max<size_t>(1, 3 * s * d.shared_inter)) ||
          grow(&w.hse, &w.cap_hse, std::max<size_t>(1, 3 * s * d.shared_inter / 32))))) {
        snprintf(g_err, sizeof g_err, "grouped scratch allocation failed (S=%d)", S);
        return -2;
    }
    return 0;
}


bool grouped_ok(const colizig_dims &d, int S) {
    return S >= kGroupedMinTokens && d.hidden % 256 == 0 && d.inter % 128 == 0 && d.shared_inter % 128 == 0 &&
           (size_t)S * d.topk <= CZ_DISPATCH_MAX;
}

void free_layer(LayerHost &L) {
    if (!L.streamed())
        for (void *p : {(void *)L.ew, (void *)L.es})
            if (p) (void)hipFree(p);
    for (void *p : {(void *)L.router, (void *)L.sw, (void *)L.ss, (void *)L.shg, (void *)L.rbias,
                    (void *)L.slot_map_dev, (void *)L.usage, (void *)L.router_bf16, L.shn_gate, L.shn_up,
                    L.shn_down})
        if (p) (void)hipFree(p);
    if (L.slot_map_stage) (void)hipHostFree(L.slot_map_stage);
    L = LayerHost{};
}

hipStream_t pick_stream(void *s) { return s ? (hipStream_t)s : g.stream; }

// Device activations are read and written as float4: x_dev / out_dev must be
// 16-byte aligned (hipMalloc'ed buffers always are).
bool dev_aligned(const void *a, const void *b = nullptr) {
    if ((((uintptr_t)a) | ((uintptr_t)b)) & 15u) {
        snprintf(g_err, sizeof g_err, "device activation buffers must be 16-byte aligned");
        return false;
    }
    return true;
}

// ---- launches of one layer ------------------------------------------------
// Router token tile: tt tokens of H floats staged in LDS, kept <= 32 KiB.
int router_tokens_per_tile(uint32_t H) {
    return (int)std::min<uint32_t>(CZ_ROUTER_TT, std::max<uint32_t>(1u, 8192u / std::max<uint32_t>(H, 1u)));
}

// rows of each of gate/up per wave: 1, or 2 when that still leaves at least
// kUpRows2Blocks workgroups (each workgroup stages the token's x once, so two
// rows per wave halve those reads; with fewer workgroups the grid is too thin)
constexpr uint32_t kUpRows2Blocks = 1024;
constexpr int kDownKC = 8;    // experts per load batch of the down kernel

enum Which { kRouter = 1, kUp = 2, kDown = 4, kAll = 7 };

// The RMS rows kernel that launch_router runs for these arguments also forms
// the shared-expert gate (the workgroup-per-row form, with a shared expert).
// Whether the RMS rows of S tokens go through k_rms_rows_wg (launch_router's
// choice), which can also write xn's FP8-MFMA terms.
bool rms_rows_wg(const LayerHost &Lh, int S) {
    const colizig_dims &d = Lh.d;
    const uint32_t q = (d.hidden / 4 + 255) / 256;
    if (Lh.router_bf16) return d.hidden % 256 == 0 && (q == 1 || q == 2 || q == 4 || q == 8);
    return S >= kGroupedMinTokens && d.hidden % 256 == 0 && q <= 8;
}

bool rms_rows_write_sgate(const StepArgs &A) {
    const LayerDev &L = A.L;
    return A.rms && A.S >= kGroupedMinTokens && L.H % 256 == 0 && L.SI != 0 && (L.H / 4 + 255) / 256 <= 8;
}

// y[S][O] = x[S][I] . W^T for NativeMatrix rows (f32: dotF32; BF16: dotBf16,
// tensors.zig:114-119), bit for bit.
template <typename T>
void launch_gemv_native(float *y, const float *x, const T *w, int S, int I, int O, hipStream_t st) {
    constexpr int WPB = 8;
    const dim3 grid((O + 2 * WPB - 1) / (2 * WPB)), blk(64 * WPB);
    switch ((I % 32) ? 0 : I / 32) {
        case 8: k_gemv_native<8, WPB, T><<<grid, blk, 0, st>>>(y, x, w, (uint32_t)S, (uint32_t)O); return;
        case 16: k_gemv_native<16, WPB, T><<<grid, blk, 0, st>>>(y, x, w, (uint32_t)S, (uint32_t)O); return;
        case 32: k_gemv_native<32, WPB, T><<<grid, blk, 0, st>>>(y, x, w, (uint32_t)S, (uint32_t)O); return;
        case 64: k_gemv_native<64, WPB, T><<<grid, blk, 0, st>>>(y, x, w, (uint32_t)S, (uint32_t)O); return;
        case 96: k_gemv_native<96, WPB, T><<<grid, blk, 0, st>>>(y, x, w, (uint32_t)S, (uint32_t)O); return;
        case 128: k_gemv_native<128, WPB, T><<<grid, blk, 0, st>>>(y, x, w, (uint32_t)S, (uint32_t)O); return;
        default:
            k_gemv_native_any<T><<<(O + 1) / 2, 64, 0, st>>>(y, x, w, (uint32_t)S, (uint32_t)I, (uint32_t)O);
            return;
    }
}

// A BF16 router (NativeMatrix bf16, tensors.zig:114-119): rms rows first when
// asked (the same bits as the f32 router kernels' staging), then dotBf16 rows
// and the bias add.
void launch_router_bf16(const StepArgs &A, hipStream_t st) {
    const LayerDev &L = A.L;
    const float *xin = A.x;
    if (A.rms) {
        switch (L.H % 256 ? 0u : (L.H / 4 + 255) / 256) {
            case 1: k_rms_rows_wg<1><<<A.S, 256, 0, st>>>(A); break;
            case 2: k_rms_rows_wg<2><<<A.S, 256, 0, st>>>(A); break;
            case 4: k_rms_rows_wg<4><<<A.S, 256, 0, st>>>(A); break;
            case 8: k_rms_rows_wg<8><<<A.S, 256, 0, st>>>(A); break;
            default: k_rms_rows<<<(A.S + 3) / 4, 256, 0, st>>>(A); break;
        }
        xin = A.xn;
    }
    launch_gemv_native<uint16_t>(A.logits, xin, L.router_bf16, A.S, (int)L.H, (int)L.E, st);
    if (L.router_bias) {
        const uint64_t n = (uint64_t)A.S * L.E;
        k_add_bias<<<(uint32_t)((n + 255) / 256), 256, 0, st>>>(A.logits, L.router_bias, (uint32_t)A.S, L.E);
    }
}

void launch_router(const StepArgs &A, hipStream_t st) {
    const LayerDev &L = A.L;
    if (L.router_bf16) {
        launch_router_bf16(A, st);
        return;
    }
    if (A.S >= kGroupedMinTokens && L.H % 256 == 0) {  // many tokens: RMS rows, then 16 x 16 tiles
        if (A.rms && !A.rms_ready) {
            switch ((L.H / 4 + 255) / 256) {  // 128-bit words per thread
                case 1: k_rms_rows_wg<1><<<A.S, 256, 0, st>>>(A); break;
                case 2: k_rms_rows_wg<2><<<A.S, 256, 0, st>>>(A); break;
                case 3: k_rms_rows_wg<3><<<A.S, 256, 0, st>>>(A); break;
                case 4: k_rms_rows_wg<4><<<A.S, 256, 0, st>>>(A); break;
                case 5: k_rms_rows_wg<5><<<A.S, 256, 0, st>>>(A); break;
                case 6: k_rms_rows_wg<6><<<A.S, 256, 0, st>>>(A); break;
                case 7: k_rms_rows_wg<7><<<A.S, 256, 0, st>>>(A); break;
                case 8: k_rms_rows_wg<8><<<A.S, 256, 0, st>>>(A); break;
                default: k_rms_rows<<<(A.S + 3) / 4, 256, 0, st>>>(A); break;
            }
        }
        // tokens per workgroup: the most that still gives 256 workgroups
        const uint32_t ge = (L.E + CZ_RT_EXP - 1) / CZ_RT_EXP;
        const uint32_t S = (uint32_t)A.S;
        auto launch = [&](auto TOKc) {
            constexpr int TOK = decltype(TOKc)::value;
            const uint32_t tiles = (S + TOK - 1) / TOK;
            if (S > L.E)  // more input rows than router rows: token tiles across the XCDs
                k_router_tiled<TOK, true><<<dim3(tiles, ge), 256 * CZ_RT_TG, 0, st>>>(A);
            else
                k_router_tiled<TOK, false><<<dim3(ge, tiles), 256 * CZ_RT_TG, 0, st>>>(A);
        };
        if (ge * ((S + 15) / 16) >= 256)
            launch(std::integral_constant<int, 16>{});
        else if (ge * ((S + 7) / 8) >= 256)
            launch(std::integral_constant<int, 8>{});
        else
            launch(std::integral_constant<int, 4>{});
        return;
    }
    const dim3 grid((L.E + 1) / 2, (A.S + A.tt - 1) / A.tt);
    const size_t lds = (size_t)A.tt * L.H * sizeof(float);
    switch ((L.H % 32) ? 0u : L.H / 32) {
        case 8: k_router_fast<8><<<grid, 64, lds, st>>>(A); return;
        case 16: k_router_fast<16><<<grid, 64, lds, st>>>(A); return;
        case 32: k_router_fast<32><<<grid, 64, lds, st>>>(A); return;
        case 64: k_router_fast<64><<<grid, 64, lds, st>>>(A); return;
        case 96: k_router_fast<96><<<grid, 64, lds, st>>>(A); return;
        case 128: k_router_fast<128><<<grid, 64, lds, st>>>(A); return;
        default: k_router_generic<<<grid, 64, lds, st>>>(A); return;
    }
}

template <int NB, int M>
void launch_up_nm(const StepArgs &A, hipStream_t st) {
    const LayerDev &L = A.L;
    if constexpr (NB == 0) {
        const uint32_t blocks = (uint32_t)A.S * L.K * ((L.I + 3) / 4) + (L.SI ? (uint32_t)A.S * ((L.SI + 3) / 4) : 0u);
        k_up_generic<M><<<blocks, 256, 0, st>>>(A);
    } else {
        auto blocks_for = [&](uint32_t rows_wg) {
            return (uint32_t)A.S * L.K * ((L.I + rows_wg - 1) / rows_wg) +
                   (L.SI ? (uint32_t)A.S * ((L.SI + rows_wg - 1) / rows_wg) : 0u);
        };
        if constexpr (NB >= 32) {
            if (blocks_for(8) >= kUpRows2Blocks) {
                k_up_fast<NB, 2, M><<<blocks_for(8), 256, 0, st>>>(A);
                return;
            }
        }
        k_up_fast<NB, 1, M><<<blocks_for(4), 256, 0, st>>>(A);
    }
}

template <int NB>
void launch_up_n(const StepArgs &A, hipStream_t st) {
    switch (cz_route_groups(A.L.E)) {
        case 1: launch_up_nm<NB, 1>(A, st); return;
        case 2: launch_up_nm<NB, 2>(A, st); return;
        case 4: launch_up_nm<NB, 4>(A, st); return;
        case 8: launch_up_nm<NB, 8>(A, st); return;
        default: launch_up_nm<NB, 16>(A, st); return;
    }
}

// fast path for H = 64 * {4, 8, 16, 32, 48, 64}, generic kernel otherwise
void launch_up(const StepArgs &A, hipStream_t st) {
    const LayerDev &L = A.L;
    switch ((L.H % 64) ? 0u : L.H / 64) {
        case 4: launch_up_n<4>(A, st); return;
        case 8: launch_up_n<8>(A, st); return;
        case 16: launch_up_n<16>(A, st); return;
        case 32: launch_up_n<32>(A, st); return;
        case 48: launch_up_n<48>(A, st); return;
        case 64: launch_up_n<64>(A, st); return;
        default: launch_up_n<0>(A, st); return;
    }
}

template <int NJ, int NJS>
void launch_down_t(const StepArgs &A, hipStream_t st) {
    const uint32_t blocks = (uint32_t)A.S * ((A.L.H + 3) / 4);
    if (A.L.K > kDownKC && A.L.K % 5 == 0 && A.L.K <= 20)  // e.g. top-10: two batches of 5
        k_down_fast<NJ, NJS, 5><<<blocks, 256, 0, st>>>(A);
    else
        k_down_fast<NJ, NJS, kDownKC><<<blocks, 256, 0, st>>>(A);
}

template <int NJ>
bool launch_down_s(const StepArgs &A, hipStream_t st) {
    const LayerDev &L = A.L;
    if (L.SI == 0) { launch_down_t<NJ, 0>(A, st); return true; }
    switch ((L.SI % 256) ? 0u : L.SI / 256) {
        case 1: launch_down_t<NJ, 1>(A, st); return true;
        case 2: launch_down_t<NJ, 2>(A, st); return true;
        case 4: launch_down_t<NJ, 4>(A, st); return true;
        case 8: launch_down_t<NJ, 8>(A, st); return true;
        case 16: launch_down_t<NJ, 16>(A, st); return true;
        default: return false;
    }
}

// output rows per wave of the multi-row down kernel
constexpr int kDownRows = 2;

template <int BPL, int NQ, int KM>
void launch_down_rows(const StepArgs &A, hipStream_t st) {
    const uint32_t tiles = (A.L.H + 4 * kDownRows - 1) / (4 * kDownRows);
    k_down_rows<BPL, NQ, KM, kDownRows><<<(uint32_t)A.S * tiles, 256, 0, st>>>(A);
}

// multi-row kernel for the Qwen4-Exp shape (I 512, top-10, shared 4096:
// there the h reads of one row per wave dominate; for the Qwen3-30B-A3B shape
// one row per wave measured faster); fast path for I = 256 * {1, 2, 3, 4} and
// SI = 256 * {0, 1, 2, 4, 8, 16}, generic kernel otherwise
void launch_down(const StepArgs &A, hipStream_t st) {
    const LayerDev &L = A.L;
    if (L.I == 512 && L.SI == 4096 && L.K == 10) { launch_down_rows<8, 4, 10>(A, st); return; }
    bool ok = false;
    switch ((L.I % 256) ? 0u : L.I / 256) {
        case 1: ok = launch_down_s<1>(A, st); break;
        case 2: ok = launch_down_s<2>(A, st); break;
        case 3: ok = launch_down_s<3>(A, st); break;
        case 4: ok = launch_down_s<4>(A, st); break;
        default: break;
    }
    if (!ok) {
        const uint32_t blocks = (uint32_t)A.S * ((L.H + 3) / 4);
        k_down_generic<<<blocks, 256, 0, st>>>(A);
    }
}

// x: router input (rms=0) or residual (rms=1); out may alias xres.
StepArgs step_args(const LayerHost &Lh, const float *x, int S, float *out, int rms, float eps, const float *xres,
                   float *xn_trace, uint32_t *idx_trace, float *gates_trace) {
    Work &w = g.work;
    StepArgs A{};
    A.L = Lh.dev();
    A.x = x;
    A.xn = w.xn;
    A.logits = w.logits;
    A.idx = w.idx;
    A.gates = w.gates;
    A.sgate = w.sgate;
    A.h = w.h;
    A.hs = w.hs;
    A.xres = xres;
    A.out = out;
    A.idx_trace = idx_trace;
    A.gates_trace = gates_trace;
    A.xn_trace = xn_trace;
    A.S = S;
    A.tt = router_tokens_per_tile(Lh.d.hidden);
    A.rms = rms;
    A.eps = eps;
    return A;
}

int launch_step(const StepArgs &A, hipStream_t st, int which = kAll) {
    if (which & kRouter) launch_router(A, st);
    if (which & kUp) launch_up(A, st);
    if (which & kDown) launch_down(A, st);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) {
        snprintf(g_err, sizeof g_err, "kernel launch: %s", hipGetErrorString(e));
        return -4;
    }
    return 0;
}

// Grouped regime: router logits (as in decode), per-token routing, dispatch,
// grouped gate/up and down GEMMs (routed experts, then the shared expert as
// a dense problem), combine.
// grid of a grouped GEMM: M-tiles rounded up to whole groups of 8 (one per
// XCD) times the N-tiles; workgroups past the real M-tiles exit
// grid of a grouped GEMM: 8 x ceil(items / 8) workgroups for at most mtiles
// M-tiles x (N / cols) column tiles
uint32_t gg_blocks(uint32_t mtiles, uint32_t N, uint32_t cols) { return (mtiles * (N / cols) + 7) / 8 * 8; }

template <int M>
void launch_route_tokens(const GroupArgs &G, hipStream_t st) {
    k_route_tokens<M><<<(G.S + 3) / 4, 256, 0, st>>>(G);
}

// A NativeMatrix shared expert (moe.zig:467-479): from the MoE input xn,
// before the routed kernels (which may write over x): gate and up rows (f32
// or BF16, dotF32 / dotBf16 order), h = silu(g) * u, the down rows and the
// sigmoid gate, kept in scratch; then, after the routed experts' combine,
// out += sgate * shared.
int launch_shared_native_pre(const LayerHost &Lh, const float *xn, int S, hipStream_t st) {
    Work &w = g.work;
    const int H = (int)Lh.d.hidden, SI = (int)Lh.d.shared_inter;
    if (Lh.shn_dtype == 1) {
        launch_gemv_native<uint16_t>(w.ng, xn, (const uint16_t *)Lh.shn_gate, S, H, SI, st);
        launch_gemv_native<uint16_t>(w.nu, xn, (const uint16_t *)Lh.shn_up, S, H, SI, st);
    } else {
        launch_gemv_native<float>(w.ng, xn, (const float *)Lh.shn_gate, S, H, SI, st);
        launch_gemv_native<float>(w.nu, xn, (const float *)Lh.shn_up, S, H, SI, st);
    }
    const uint64_t n = (uint64_t)S * SI;
    k_swiglu_native<<<(uint32_t)((n + 255) / 256), 256, 0, st>>>(w.ng, w.nu, n);
    if (Lh.shn_dtype == 1)
        launch_gemv_native<uint16_t>(w.no, w.ng, (const uint16_t *)Lh.shn_down, S, SI, H, st);
    else
        launch_gemv_native<float>(w.no, w.ng, (const float *)Lh.shn_down, S, SI, H, st);
    k_shared_gate_native<<<S, 64, 0, st>>>(w.nsg, xn, Lh.shg, (uint32_t)H);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) {
        snprintf(g_err, sizeof g_err, "shared expert launch: %s", hipGetErrorString(e));
        return -4;
    }
    return 0;
}

int launch_shared_native_add(const LayerHost &Lh, float *out, int S, hipStream_t st) {
    const uint64_t n = (uint64_t)S * Lh.d.hidden;
    k_shared_add_native<<<(uint32_t)((n + 255) / 256), 256, 0, st>>>(out, g.work.no, g.work.nsg, (uint32_t)S,
                                                                    Lh.d.hidden);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) {
        snprintf(g_err, sizeof g_err, "shared expert launch: %s", hipGetErrorString(e));
        return -4;
    }
    return 0;
}

// A grouped layer's step arguments: with rms, the RMS rows also write xn's
// f16 split (f16 GEMMs) or its three E4M3 terms (FP8 GEMMs).
StepArgs grouped_args(const LayerHost &Lh, const float *x, int S, float *out, int rms, float eps, const float *xres,
                      float *xn_trace, uint32_t *idx_trace, float *gates_trace) {
    StepArgs A = step_args(Lh, x, S, out, rms, eps, xres, xn_trace, idx_trace, gates_trace);
    Work &w = g.work;
    if (rms && !g.prefill_fp8) {
        A.xh = w.xh;
        A.xl = w.xl;
    }
    if (rms && g.prefill_fp8 && rms_rows_wg(Lh, S)) {
        A.xq = w.xq;
        A.xe = w.xe;
    }
    return A;
}

// Whether the combine of grouped layer Lh can form the RMS rows of the chain's
// next layer Ln (k_combine_rms): f32 routers, no NativeMatrix shared expert
// (whose output is added after the combine), one hidden size, and enough
// tokens to fill the GPU with one workgroup per token (at 32 tokens the
// combine's four workgroups per token were faster: 11.93 against 12.10 ms
// per c4 step).
constexpr int kCombineRmsMinTokens = 256;
bool combine_rms_ok(const LayerHost &Lh, const LayerHost &Ln, int S) {
    const uint32_t q = (Lh.d.hidden / 4 + 255) / 256;
    return S >= kCombineRmsMinTokens && grouped_ok(Lh.d, S) && grouped_ok(Ln.d, S) && Ln.d.hidden == Lh.d.hidden &&
           !Ln.router_bf16 &&
           Lh.shn_dtype < 0 && Ln.shn_dtype < 0 && rms_rows_wg(Ln, S) && q >= 1 && q <= 8;
}

// rms_ready: the previous layer's combine wrote this layer's RMS rows; next
// (nullable, combine_rms_ok): this layer's combine writes the next layer's.
int launch_grouped(const LayerHost &Lh, const float *x, int S, float *out, int rms, float eps, const float *xres,
                   float *xn_trace, uint32_t *idx_trace, float *gates_trace, hipStream_t st, bool rms_ready = false,
                   const LayerHost *next = nullptr, float *next_xn_trace = nullptr) {
    StepArgs A = grouped_args(Lh, x, S, out, rms, eps, xres, xn_trace, idx_trace, gates_trace);
    A.rms_ready = rms_ready ? 1u : 0u;
    const LayerDev &L = A.L;
    Work &w = g.work;
    const bool f8 = g.prefill_fp8;
    const bool xq_rms = A.xq != nullptr;
    launch_router(A, st);
    if (Lh.shn_dtype >= 0) {
        if (int rc = launch_shared_native_pre(Lh, rms ? w.xn : x, S, st)) return rc;
    }
    GroupArgs G{};
    G.L = L;
    G.S = S;
    G.xn = rms ? w.xn : x;
    G.logits = w.logits;
    G.idx = w.idx;
    G.gates = w.gates;
    G.sgate = w.sgate;
    G.sgate_ready = rms_rows_write_sgate(A) ? 1u : 0u;
    G.usage = nullptr;  // k_dispatch counts the round's picks per expert
    G.idx_trace = idx_trace;
    G.gates_trace = gates_trace;
    G.counts = w.counts;
    G.offsets = w.offsets;
    G.sorted_slot = w.sorted_slot;
    G.slot_pos = w.slot_pos;
    G.tok_order = w.tok_order;
    G.tile_expert = w.tile_expert;
    G.tile_row0 = w.tile_row0;
    G.ntiles = w.ntiles;
    G.max_tiles = grouped_max_tiles(Lh.d, S);
    G.xh = rms || f8 ? nullptr : w.xh;  // no RMS rows kernel: the routing kernel splits x
    G.xl = rms || f8 ? nullptr : w.xl;
    G.hh = w.hh;
    G.hl = w.hl;
    G.hsh = w.hsh;
    G.hsl = w.hsl;
    G.o = w.o;
    G.os = w.os;
    G.xres = xres;
    G.out = out;
    switch (cz_route_groups(L.E)) {
        case 1: launch_route_tokens<1>(G, st); break;
        case 2: launch_route_tokens<2>(G, st); break;
        case 4: launch_route_tokens<4>(G, st); break;
        case 8: launch_route_tokens<8>(G, st); break;
        default: launch_route_tokens<16>(G, st); break;
    }
    G.usage = L.usage;
    k_dispatch<<<1, 1024, 0, st>>>(G);
    const uint32_t mts = (uint32_t)(S + CZ_GG_M - 1) / CZ_GG_M;
    const uint64_t sk = (uint64_t)S * L.K;
    auto quant3 = [&](const float *src, uint64_t rows, uint32_t K, uint8_t *q, uint8_t *e) {
        const uint64_t n = rows * K / 4;  // one float4 per thread
        k_quant3<<<(uint32_t)((n + 255) / 256), 256, 0, st>>>(src, (uint32_t)rows, K, q, rows * K, e, rows * K / 32);
    };
    if (f8 && !xq_rms) quant3(G.xn, (uint64_t)S, L.H, w.xq, w.xe);  // no RMS rows kernel splits x
    // gate/up
    GGProblem P{};
    P.w0 = L.ew;
    P.s0 = L.es;
    P.w_stride = L.ew_stride;
    P.s_stride = L.es_stride;
    P.w1_off = (uint64_t)L.I * L.H;
    P.s1_off = (uint64_t)L.nbI * L.nbH;
    P.N = L.I;
    P.Kd = L.H;
    P.nbK = L.nbH;
    P.a_hi = w.xh;
    P.a_lo = w.xl;
    P.c_hi = w.hh;
    P.c_lo = w.hl;
    P.routed = 1;
    if (f8) {
        P.aq = w.xq;
        P.ae = w.xe;
        P.aq_plane = (uint64_t)S * L.H;
        P.ae_plane = (uint64_t)S * L.H / 32;
        P.cq = w.hq;  // the gate/up GEMM writes h as the down GEMM's three terms
        P.ce = w.he;
        P.cq_plane = sk * L.I;
        P.ce_plane = sk * L.I / 32;
    }
    constexpr uint32_t cu = cz_gg_cols<GG_GATEUP>(), cd = cz_gg_cols<GG_DOWN>();
    // the shared expert's items run in the same launches as the routed ones
    GGProblem Q{};
    if (L.SI) {
        Q = P;
        Q.w0 = L.sw;
        Q.s0 = L.ss;
        Q.w_stride = 0;
        Q.s_stride = 0;
        Q.w1_off = (uint64_t)L.SI * L.H;
        Q.s1_off = (uint64_t)L.nbSI * L.nbH;
        Q.N = L.SI;
        Q.c_hi = w.hsh;
        Q.c_lo = w.hsl;
        Q.cq = w.hsq;
        Q.ce = w.hse;
        Q.cq_plane = (uint64_t)S * L.SI;
        Q.ce_plane = (uint64_t)S * L.SI / 32;
        Q.routed = 0;
        Q.rows_total = (uint32_t)S;
    }
    const uint32_t qu = L.SI ? (mts * (L.SI / cu) + 7) / 8 * 8 : 0u;
    if (f8)
        k_gg8<GG_GATEUP><<<qu + gg_blocks(G.max_tiles, L.I, cu), 256, 0, st>>>(G, P, Q);
    else
        k_gg<GG_GATEUP><<<qu + gg_blocks(G.max_tiles, L.I, cu), 256, 0, st>>>(G, P, Q);

    // down
    GGProblem D{};
    D.w0 = L.ew + 2ull * L.I * L.H;
    D.s0 = L.es + 2ull * L.nbI * L.nbH;
    D.w_stride = L.ew_stride;
    D.s_stride = L.es_stride;
    D.N = L.H;
    D.Kd = L.I;
    D.nbK = L.nbI;
    D.a_hi = w.hh;
    D.a_lo = w.hl;
    D.c = w.o;
    D.routed = 1;
    D.aq = w.hq;
    D.ae = w.he;
    D.aq_plane = sk * L.I;
    D.ae_plane = sk * L.I / 32;
    GGProblem QD{};
    if (L.SI) {
        QD = D;
        QD.w0 = L.sw + 2ull * L.SI * L.H;
        QD.s0 = L.ss + 2ull * L.nbSI * L.nbH;
        QD.w_stride = 0;
        QD.s_stride = 0;
        QD.Kd = L.SI;
        QD.nbK = L.nbSI;
        QD.a_hi = w.hsh;
        QD.a_lo = w.hsl;
        QD.c = w.os;
        QD.routed = 0;
        QD.rows_total = (uint32_t)S;
        QD.aq = w.hsq;
        QD.ae = w.hse;
        QD.aq_plane = (uint64_t)S * L.SI;
        QD.ae_plane = (uint64_t)S * L.SI / 32;
    }
    const uint32_t qd = L.SI ? (mts * (L.H / cd) + 7) / 8 * 8 : 0u;
    if (f8)
        k_gg8<GG_DOWN><<<qd + gg_blocks(G.max_tiles, L.H, cd), 256, 0, st>>>(G, D, QD);
    else
        k_gg<GG_DOWN><<<qd + gg_blocks(G.max_tiles, L.H, cd), 256, 0, st>>>(G, D, QD);
    if (next) {
        const StepArgs An = grouped_args(*next, out, S, out, 1, eps, out, next_xn_trace, nullptr, nullptr);
        switch ((L.H / 4 + 255) / 256) {
            case 1: k_combine_rms<1><<<S, 256, 0, st>>>(G, An); break;
            case 2: k_combine_rms<2><<<S, 256, 0, st>>>(G, An); break;
            case 3: k_combine_rms<3><<<S, 256, 0, st>>>(G, An); break;
            case 4: k_combine_rms<4><<<S, 256, 0, st>>>(G, An); break;
            case 5: k_combine_rms<5><<<S, 256, 0, st>>>(G, An); break;
            case 6: k_combine_rms<6><<<S, 256, 0, st>>>(G, An); break;
            case 7: k_combine_rms<7><<<S, 256, 0, st>>>(G, An); break;
            default: k_combine_rms<8><<<S, 256, 0, st>>>(G, An); break;
        }
    } else {
        k_combine<<<dim3((L.H + CZ_COMBINE_COLS - 1) / CZ_COMBINE_COLS, S), 256, 0, st>>>(G);
    }
    if (Lh.shn_dtype >= 0) {
        if (int rc = launch_shared_native_add(Lh, out, S, st)) return rc;
    }
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) {
        snprintf(g_err, sizeof g_err, "grouped launch: %s", hipGetErrorString(e));
        return -4;
    }
    return 0;
}

LayerHost *find_layer(uint32_t layer);

// The one-launch decode serves batch 1 on a device of 8 XCDs x 32 CUs for
// resident layers without a shared expert with H in {512, 1024, 2048},
// E <= 128, K <= 32, I a multiple of 128 and K*I/1024 in {1, 2, 4, 6, 8}.
// The one-launch decode's shape and device conditions; a streamed layer
// runs it only inside a speculative run (slot maps on the device).
bool fused_shape_ok(const LayerHost &L, int S) {
    const colizig_dims &d = L.d;
    if (!g.fused.enabled || S != 1 || g.fused.cus != CZ_FWG || !g.fused.placement_ok) return false;
    if (d.shared_inter != 0 || d.experts > 128 || d.topk > 32 || d.inter % CZ_BLOCK || L.router_bf16)
        return false;
    if (d.hidden != 512 && d.hidden != 1024 && d.hidden != 2048) return false;
    const uint64_t ki = (uint64_t)d.topk * d.inter;
    if (ki % 1024) return false;
    const uint64_t rw = ki / 1024;
    return rw == 1 || rw == 2 || rw == 4 || rw == 6 || rw == 8;
}

bool fused_ok(const LayerHost &L, int S) { return !L.streamed() && fused_shape_ok(L, S); }

int ensure_fused(const colizig_dims &d) {
    FusedState &F = g.fused;
    const size_t ki = (size_t)d.topk * d.inter;
    if (!F.run) {
        if (hipMalloc(&F.run, 256) != hipSuccess) return -2;
        if (hipMemset(F.run, 0, 256) != hipSuccess) return -2;
        F.pstat = reinterpret_cast<unsigned long long *>(F.run) + 16;       // bytes 128..143 of the same block
        F.spec_pstat = reinterpret_cast<unsigned long long *>(F.run) + 18;  // bytes 144..159
        if (hipMalloc(&F.pred, 2 * 64 * sizeof(uint32_t)) != hipSuccess) return -2;
        if (hipMemset(F.pred, 0, 2 * 64 * sizeof(uint32_t)) != hipSuccess) return -2;
        if (hipHostMalloc(&F.err_host, 64, hipHostMallocCoherent | hipHostMallocMapped) != hipSuccess) return -2;
        __atomic_store_n(F.err_host, 0u, __ATOMIC_RELEASE);
        if (hipHostGetDevicePointer((void **)&F.err_dev, F.err_host, 0) != hipSuccess) return -2;
    }
    if (F.cap_h < d.hidden) {
        size_t cap_r = 0, cap_p = 0, cap_z = 0;
        for (float *q : {F.r, F.p, F.zero})
            if (q) g.retired.push_back(q);
        F.r = F.p = F.zero = nullptr;
        if (grow(&F.r, &cap_r, 2ull * d.hidden) || grow(&F.p, &cap_p, 2ull * CZ_NXCD * d.hidden) ||
            grow(&F.zero, &cap_z, (size_t)CZ_NXCD * d.hidden))
            return -2;
        if (hipMemset(F.zero, 0, cap_z * sizeof(float)) != hipSuccess) return -2;
        F.cap_h = d.hidden;
    }
    if (F.cap_e < d.experts) {
        size_t cap = 0, cap_p = 0;
        if (F.lgx) g.retired.push_back(F.lgx);
        if (F.lgpx) g.retired.push_back(F.lgpx);
        F.lgx = nullptr;
        F.lgpx = nullptr;
        if (grow(&F.lgx, &cap, (size_t)CZ_NXCD * d.experts) || grow(&F.lgpx, &cap_p, (size_t)d.experts)) return -2;
        if (hipMemset(F.lgx, 0, cap * sizeof(unsigned long long)) != hipSuccess) return -2;
        if (hipMemset(F.lgpx, 0, cap_p * sizeof(unsigned long long)) != hipSuccess) return -2;
        F.cap_e = d.experts;
    }
    if (F.cap_ki < ki) {
        size_t cap = 0;
        if (F.hx) g.retired.push_back(F.hx);
        F.hx = nullptr;
        if (grow(&F.hx, &cap, ki)) return -2;
        if (hipMemset(F.hx, 0, cap * sizeof(unsigned long long)) != hipSuccess) return -2;
        F.cap_ki = ki;
    }
    return 0;
}

template <int NB, bool SPEC, bool STOP>
void launch_fused_spec(const FusedArgs &A, uint32_t rw, hipStream_t st) {
    switch (rw) {
        case 1: k_layer_fused<NB, 1, SPEC, STOP><<<CZ_FWG, 512, 0, st>>>(A); return;
        case 2: k_layer_fused<NB, 2, SPEC, STOP><<<CZ_FWG, 512, 0, st>>>(A); return;
        case 4: k_layer_fused<NB, 4, SPEC, STOP><<<CZ_FWG, 512, 0, st>>>(A); return;
        case 6: k_layer_fused<NB, 6, SPEC, STOP><<<CZ_FWG, 512, 0, st>>>(A); return;
        default: k_layer_fused<NB, 8, SPEC, STOP><<<CZ_FWG, 512, 0, st>>>(A); return;
    }
}

// A speculative run's layers (A.stop set, with their slot maps and the
// token-level prediction) take the kernels built with STOP.
template <int NB>
void launch_fused_nb(const FusedArgs &A, uint32_t rw, hipStream_t st) {
    if (A.stop && A.pred_in && A.L.slot_map)
        launch_fused_spec<NB, true, true>(A, rw, st);
    else if (A.pred_in)
        launch_fused_spec<NB, true, false>(A, rw, st);
    else
        launch_fused_spec<NB, false, false>(A, rw, st);
}

// The layers [layer0, layer0 + n) (all fused_ok, one hidden size) as n
// layer launches and the final residual add.  Residual / partial buffers:
// layer p reads x_p's parts (x_dev for p <= 1, else r[(p-1) % 2], plus the
// partials p[(p-1) % 2] for p >= 1), keeps x_p in r[p % 2] (p >= 1) and
// writes its partials to p[p % 2]; the final kernel writes x_dev.
int chain_enqueue_fused(uint32_t layer0, uint32_t n, float *x_dev, float eps, float *xn_trace,
                        uint32_t *idx_trace, float *gates_trace, hipStream_t st) {
    FusedState &F = g.fused;
    const uint32_t H = find_layer(layer0)->d.hidden;
    for (uint32_t p = 0; p < n; ++p) {
        const LayerHost &L = *find_layer(layer0 + p);
        FusedArgs A{};
        A.L = L.dev();
        A.rin = p <= 1 ? x_dev : F.r + (uint64_t)((p - 1) % 2) * H;
        A.pin = p == 0 ? F.zero : F.p + (uint64_t)((p - 1) % 2) * CZ_NXCD * H;
        A.has_pin = p == 0 ? 0u : 1u;
        A.rout = p == 0 ? nullptr : F.r + (uint64_t)(p % 2) * H;
        A.pout = F.p + (uint64_t)(p % 2) * CZ_NXCD * H;
        A.lgx = F.lgx;
        A.hx = F.hx;
        A.run = F.run;
        A.err = F.err_dev;
        A.xn_trace = xn_trace ? xn_trace + (uint64_t)p * H : nullptr;
        A.idx_trace = idx_trace ? idx_trace + (uint64_t)p * L.d.topk : nullptr;
        A.gates_trace = gates_trace ? gates_trace + (uint64_t)p * L.d.topk : nullptr;
        A.pos = p;
        A.eps = eps;
        // predicted experts: layer p + 1's top-k on layer p's router input
        // (same expert count and top-k), in F.pred[(p + 1) % 2]
        const LayerHost *Ln = p + 1 < n ? find_layer(layer0 + p + 1) : nullptr;
        const LayerHost *Lp = p > 0 ? find_layer(layer0 + p - 1) : nullptr;
        if (F.predict && Lp && Lp->d.experts == L.d.experts && Lp->d.topk == L.d.topk)
            A.pred_in = F.pred + (uint64_t)(p % 2) * 64;
        if (F.predict && Ln && Ln->d.experts == L.d.experts && Ln->d.topk == L.d.topk) {
            A.pred_out = F.pred + (uint64_t)((p + 1) % 2) * 64;
            A.rnext = Ln->router;
            A.rbias_next = Ln->rbias;
        }
        A.lgpx = F.lgpx;
        A.pred_mode = F.predict >= 2 ? (uint32_t)(F.predict - 1) : 0u;
        A.pstat = F.pstat;
        A.poll_mask = (int)p == F.fault_pos ? ~1023u : ~0u;
        const uint32_t rw = (uint32_t)((uint64_t)L.d.topk * L.d.inter / 1024);
        switch (H) {
            case 512: launch_fused_nb<8>(A, rw, st); break;
            case 1024: launch_fused_nb<16>(A, rw, st); break;
            default: launch_fused_nb<32>(A, rw, st); break;
        }
    }
    const float *rin_f = n == 1 ? x_dev : F.r + (uint64_t)((n - 1) % 2) * H;
    k_chain_final<<<(H + 255) / 256, 256, 0, st>>>(x_dev, rin_f, F.p + (uint64_t)((n - 1) % 2) * CZ_NXCD * H, H,
                                                   F.run);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) {
        snprintf(g_err, sizeof g_err, "fused decode launch: %s", hipGetErrorString(e));
        return -4;
    }
    return 0;
}

// Whether a chain of n layers from layer0 at S tokens runs the one-launch
// decode (every layer eligible, one hidden size, < 1023 layers), preparing
// its buffers; <0 on an allocation failure.
int chain_fused_prepare(uint32_t layer0, uint32_t n, int S) {
    if (n >= 1023) return 0;
    const LayerHost *L0 = find_layer(layer0);
    if (!L0) return 0;
    for (uint32_t l = 0; l < n; ++l) {
        const LayerHost *L = find_layer(layer0 + l);
        if (!L || !fused_ok(*L, S) || L->d.hidden != L0->d.hidden) return 0;
    }
    for (uint32_t l = 0; l < n; ++l) {
        const int rc = ensure_fused(find_layer(layer0 + l)->d);
        if (rc) return rc;
    }
    return 1;
}

int launch_layer(const LayerHost &Lh, const float *x, int S, float *out, int rms, float eps, const float *xres,
                 float *xn_trace, uint32_t *idx_trace, float *gates_trace, hipStream_t st, bool rms_ready = false,
                 const LayerHost *next = nullptr, float *next_xn_trace = nullptr) {
    if (grouped_ok(Lh.d, S))
        return launch_grouped(Lh, x, S, out, rms, eps, xres, xn_trace, idx_trace, gates_trace, st, rms_ready, next,
                              next_xn_trace);
    const StepArgs A = step_args(Lh, x, S, out, rms, eps, xres, xn_trace, idx_trace, gates_trace);
    if (Lh.shn_dtype < 0) return launch_step(A, st);
    int rc = launch_step(A, st, kRouter);
    if (!rc) rc = launch_shared_native_pre(Lh, rms ? g.work.xn : x, S, st);
    if (!rc) rc = launch_step(A, st, kUp | kDown);
    if (!rc) rc = launch_shared_native_add(Lh, out, S, st);
    return rc;
}

void pool_drop_layer(uint32_t layer);
int ensure_h_idx(int S);
struct LayerHost;
int run_streamed_layer(LayerHost &L, uint32_t layer, const float *x, int S, float *out, int rms, float eps,
                       const float *xres, LayerHost *next, uint32_t next_layer, hipStream_t st,
                       const std::vector<uint32_t> *later);

LayerHost *find_layer(uint32_t layer) {
    auto it = g.layers.find(layer);
    return it == g.layers.end() ? nullptr : &it->second;
}

int check_layer_ready(LayerHost *L, uint32_t layer) {
    if (!L) {
        snprintf(g_err, sizeof g_err, "layer %u not registered", layer);
        return -6;
    }
    if (!L->ready()) {
        snprintf(g_err, sizeof g_err, "layer %u: %u of %u experts loaded%s", layer, L->nloaded, L->d.experts,
                 (L->d.shared_inter && !L->shared_set) ? ", shared expert missing" : "");
        return -6;
    }
    if (L->d.experts > CZ_MAX_E || L->d.topk > CZ_MAX_K || L->d.topk == 0 || L->d.topk > L->d.experts) {
        snprintf(g_err, sizeof g_err, "layer %u: experts %u / topk %u outside the supported range", layer,
                 L->d.experts, L->d.topk);
        return -1;
    }
    if (L->d.hidden > 8192) {
        snprintf(g_err, sizeof g_err, "layer %u: hidden %u > 8192", layer, L->d.hidden);
        return -1;
    }
    return 0;
}

// The one-launch decode's error word (set by its kernels when a poll ran
// out): reported once as -5, then cleared.
int fused_check_error() {
    if (!g.fused.err_host) return 0;
    const uint32_t e = __atomic_exchange_n(g.fused.err_host, 0u, __ATOMIC_ACQ_REL);
    if (!e) return 0;
    snprintf(g_err, sizeof g_err, "one-launch decode: an exchange between the workgroups of an XCD timed out "
             "(error word %#x); the step's results are invalid", e);
    return -5;
}

uint8_t *noalloc_scratch();

// The one-launch decode's placement census (k_xcd_census): true when each of
// the 8 XCDs received exactly one workgroup of each rank 0 .. 31 of a
// CZ_FWG-wide launch, the layout k_layer_fused's exchanges assume.  Anything
// else (another XCD count, another dispatch order, a failed launch) keeps
// the layers on the three-kernel path.
bool fused_placement_census() {
    uint32_t *d = nullptr;
    uint32_t h[CZ_FWG];
    bool ok = hipMalloc(&d, sizeof h) == hipSuccess;
    if (ok) {
        k_xcd_census<<<CZ_FWG, 64, 0, g.stream>>>(d);
        ok = hipGetLastError() == hipSuccess && hipStreamSynchronize(g.stream) == hipSuccess &&
             hipMemcpy(h, d, sizeof h, hipMemcpyDeviceToHost) == hipSuccess;
    }
    if (d) (void)hipFree(d);
    if (!ok) return false;
    uint32_t seen[CZ_NXCD] = {0};  // bit w: rank w seen on that XCD
    for (uint32_t b = 0; b < CZ_FWG; ++b) {
        if (h[b] >= CZ_NXCD) return false;
        const uint32_t bit = 1u << (b / CZ_NXCD);
        if (seen[h[b]] & bit) return false;
        seen[h[b]] |= bit;
    }
    for (uint32_t x = 0; x < CZ_NXCD; ++x)
        if (seen[x] != 0xffffffffu) return false;
    return true;
}

uint64_t mix64(uint64_t z) {
    z += 0x9e3779b97f4a7c15ull;
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
    return z ^ (z >> 31);
}

}  // namespace

// synthetic generator over one role of every expert of a layer
__global__ __launch_bounds__(256) void k_synth_fp8_experts(uint8_t *ew, float *es, uint64_t ew_stride,
                                                           uint64_t es_stride, uint64_t w_off, uint64_t s_off,
                                                           uint32_t rows, uint32_t cols, uint64_t seed, float stdv);

// ===========================================================================
// 1. the existing backend ABI
// ===========================================================================
extern "C" int colizig_cuda_init(void) {
    CsrGuard csr;
    std::lock_guard<std::recursive_mutex> lk(g_mu);
    if (g.inited) return 0;
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || n < 1) {
        snprintf(g_err, sizeof g_err, "no HIP device");
        return -1;
    }
    if (hipSetDevice(0) != hipSuccess) return -2;
    hipDeviceProp_t prop;
    if (hipGetDeviceProperties(&prop, 0) != hipSuccess) return -3;
    snprintf(g.name, sizeof g.name, "%s (%s, %zu MiB)", prop.name, prop.gcnArchName,
             (size_t)(prop.totalGlobalMem >> 20));
    g.fused.cus = prop.multiProcessorCount;
    if (hipStreamCreateWithFlags(&g.stream, hipStreamNonBlocking) != hipSuccess) return -4;
    g.fused.placement_ok = g.fused.cus == CZ_FWG && fused_placement_census();
    // the no-alloc forward's scratch address on this device; a failure is
    // reported by that entry point, which tries again
    if (!noalloc_scratch()) g_err[0] = 0;
    g.budget = 0;  // keyed cache off until set (colizig_cuda.cu:185)
    g.inited = 1;
    return 0;
}

extern "C" const char *colizig_cuda_device_name(void) { return g.inited ? g.name : ""; }

extern "C" void colizig_cuda_set_vram_budget(uint64_t bytes) {
    CsrGuard csr;
    std::lock_guard<std::recursive_mutex> lk(g_mu);
    if (!g.inited) return;
    size_t freeb = 0, totalb = 0;
    if (hipMemGetInfo(&freeb, &totalb) == hipSuccess && bytes > freeb - (freeb / 8)) bytes = freeb - (freeb / 8);
    g.budget = bytes;
}

extern "C" void colizig_cuda_stats(uint64_t *hits, uint64_t *misses, uint64_t *uploaded_mib, uint64_t *resident) {
    if (hits) *hits = g.hits;
    if (misses) *misses = g.misses;
    if (uploaded_mib) *uploaded_mib = g.uploaded >> 20;
    if (resident) *resident = (uint64_t)g.slots.size();
}

extern "C" void colizig_cuda_shutdown(void) {
    CsrGuard csr;
    std::lock_guard<std::recursive_mutex> lk(g_mu);
    if (!g.inited) return;
    (void)hipStreamSynchronize(g.stream);
    for (auto &kv : g.graphs) (void)hipGraphExecDestroy(kv.second);
    for (auto &kv : g.graph_defs) (void)hipGraphDestroy(kv.second);
    for (auto &kv : g.events) (void)hipEventDestroy(kv.second);
    for (auto &kv : g.layers) free_layer(kv.second);
    for (Slot &s : g.slots) {
        if (s.w) (void)hipFree(s.w);
        if (s.s) (void)hipFree(s.s);
    }
    for (void *p : {g.d_x, g.d_y, g.d_w, g.d_s}) if (p) (void)hipFree(p);
    if (g.h_stage) (void)hipHostFree(g.h_stage);
    Work &w = g.work;
    for (void *p : {(void *)w.xin, (void *)w.out, (void *)w.xn, (void *)w.logits, (void *)w.gates,
                    (void *)w.sgate, (void *)w.h, (void *)w.hs, (void *)w.idx, (void *)w.counts, (void *)w.offsets,
                    (void *)w.sorted_slot, (void *)w.slot_pos, (void *)w.tok_order, (void *)w.tile_expert,
                    (void *)w.tile_row0, (void *)w.ntiles, (void *)w.o, (void *)w.os, (void *)w.xh, (void *)w.xl,
                    (void *)w.hh, (void *)w.hl, (void *)w.hsh, (void *)w.hsl, (void *)w.ng, (void *)w.nu,
                    (void *)w.no, (void *)w.nsg, (void *)w.xq, (void *)w.xe, (void *)w.hq, (void *)w.he,
                    (void *)w.hsq, (void *)w.hse})
        if (p) (void)hipFree(p);
    for (void *p : g.retired) (void)hipFree(p);
    for (void *p : {(void *)g.fused.r, (void *)g.fused.p, (void *)g.fused.zero, (void *)g.fused.lgx,
                    (void *)g.fused.hx, (void *)g.fused.run, (void *)g.fused.pred, (void *)g.fused.lgpx})
        if (p) (void)hipFree(p);
    if (g.fused.err_host) (void)hipHostFree(g.fused.err_host);
    StreamPool &P = g.pool;
    if (P.copy) (void)hipStreamSynchronize(P.copy);
    if (P.copy_hi) (void)hipStreamSynchronize(P.copy_hi);
    if (P.copy2) (void)hipStreamSynchronize(P.copy2);
    for (void *p : {(void *)P.base, (void *)P.pred_logits, (void *)P.pred_gates, (void *)P.pred_sgate,
                    (void *)P.pred_idx, (void *)P.pred_tord, (void *)P.route_count, (void *)P.tok_logits, (void *)P.tok_gates,
                    (void *)P.tok_idx, (void *)P.tok_tord, (void *)P.tok_ptr_dev, (void *)P.stop_dev,
                    (void *)P.spec_idx_dev, (void *)P.spec_tab_dev})
        if (p) (void)hipFree(p);
    for (void *p : {(void *)P.h_idx, (void *)P.h_flag, (void *)P.h_pred, (void *)P.h_pflag, (void *)P.h_tok,
                    (void *)P.h_tflag, (void *)P.tok_ptr_stage, (void *)P.h_spec, (void *)P.h_spec_tab})
        if (p) (void)hipHostFree(p);
    for (hipEvent_t e : P.slot_ev) (void)hipEventDestroy(e);
    if (P.ev_idx) (void)hipEventDestroy(P.ev_idx);
    if (P.ev_copy) (void)hipEventDestroy(P.ev_copy);
    if (P.ev_copy_hi) (void)hipEventDestroy(P.ev_copy_hi);
    if (P.ev_copy2) (void)hipEventDestroy(P.ev_copy2);
    if (P.copy) (void)hipStreamDestroy(P.copy);
    if (P.copy_hi) (void)hipStreamDestroy(P.copy_hi);
    if (P.copy2) (void)hipStreamDestroy(P.copy2);
    (void)hipStreamDestroy(g.stream);
    g.~Ctx();
    new (&g) Ctx();
}

// Slot for `key` (hit), or a slot to fill (colizig_cuda.cu:132-169 policy:
// fresh slot within budget, else the LRU slot whose buffers fit, else grow
// the globally LRU slot).  -1 when nothing can be allocated.
static int cache_slot_for(uint64_t key, size_t wb, size_t sb) {
    auto it = g.by_key.find(key);
    if (it != g.by_key.end()) return it->second;
    if (g.slots.size() < kMaxSlots && g.used + wb + sb <= g.budget) {
        Slot s;
        if (ensure_dev(&s.w, &s.wcap, wb) || ensure_dev(&s.s, &s.scap, sb)) {
            if (s.w) (void)hipFree(s.w);
            if (s.s) (void)hipFree(s.s);
            return -1;
        }
        g.used += s.wcap + s.scap;
        g.slots.push_back(s);
        return (int)g.slots.size() - 1;
    }
    int victim = -1;
    uint64_t best = ~0ull;
    for (size_t i = 0; i < g.slots.size(); ++i)
        if (g.slots[i].wcap >= wb && g.slots[i].scap >= sb && g.slots[i].clock < best) {
            best = g.slots[i].clock;
            victim = (int)i;
        }
    if (victim < 0) {
        for (size_t i = 0; i < g.slots.size(); ++i)
            if (g.slots[i].clock < best) {
                best = g.slots[i].clock;
                victim = (int)i;
            }
        if (victim < 0) return -1;
        Slot &s = g.slots[victim];
        g.used -= s.wcap + s.scap;
        if (ensure_dev(&s.w, &s.wcap, wb) || ensure_dev(&s.s, &s.scap, sb)) return -1;
        g.used += s.wcap + s.scap;
    }
    if (g.slots[victim].key) g.by_key.erase(g.slots[victim].key);
    g.slots[victim].key = 0;
    return victim;
}

void launch_matmul_fp8(float *y, const float *x, const uint8_t *w, const float *s, int S, int I, int O,
                       hipStream_t st);

extern "C" int colizig_cuda_matmul_fp8(float *y, const float *x, const unsigned char *w, const float *scales, int S,
                                       int I, int O, uint64_t key) {
    CsrGuard csr;
    std::lock_guard<std::recursive_mutex> lk(g_mu);
    if (!g.inited || S < 1 || I < 1 || O < 1 || !y || !x || !w || !scales) return -1;
    const size_t nbi = nblk((uint32_t)I), nbo = nblk((uint32_t)O);
    const size_t xb = (size_t)S * I * sizeof(float), wb = (size_t)O * I, sb = nbo * nbi * sizeof(float),
                 yb = (size_t)S * O * sizeof(float);
    if (ensure_dev(&g.d_x, &g.d_x_cap, xb) || ensure_dev(&g.d_y, &g.d_y_cap, yb)) return -2;
    if (ensure_host(std::max(xb, yb))) return -2;
    memcpy(g.h_stage, x, xb);
    if (hipMemcpyAsync(g.d_x, g.h_stage, xb, hipMemcpyHostToDevice, g.stream) != hipSuccess) return -3;
    const void *wdev = nullptr, *sdev = nullptr;
    if (key != 0 && g.budget != 0) {
        int i = cache_slot_for(key, wb, sb);
        // a hit is used only when the resident matrix is this call's: FP8 rows
        // of the same shape.  Otherwise the slot is refilled when its buffers
        // hold this matrix, else the call takes the uncached path.
        bool same = false;
        if (i >= 0 && g.slots[i].key == key) {
            const Slot &sl = g.slots[i];
            same = sl.bf16 == 0 && sl.I == I && sl.O == O;
            if (!same && (sl.wcap < wb || sl.scap < sb)) i = -1;
        }
        if (i < 0) {
            key = 0;  // cache full of bigger blocks, or the key holds another matrix: uncached path
        } else if (same) {
            g.hits++;
            g.slots[i].clock = ++g.lru;
            wdev = g.slots[i].w;
            sdev = g.slots[i].s;
        } else {
            g.misses++;
            if (hipMemcpyAsync(g.slots[i].w, w, wb, hipMemcpyHostToDevice, g.stream) != hipSuccess) return -3;
            if (hipMemcpyAsync(g.slots[i].s, scales, sb, hipMemcpyHostToDevice, g.stream) != hipSuccess) return -3;
            g.uploaded += wb + sb;
            g.slots[i].key = key;
            g.slots[i].I = I;
            g.slots[i].O = O;
            g.slots[i].bf16 = 0;
            g.by_key[key] = i;
            g.slots[i].clock = ++g.lru;
            wdev = g.slots[i].w;
            sdev = g.slots[i].s;
        }
    }
    if (key == 0 || g.budget == 0) {
        if (ensure_dev(&g.d_w, &g.d_w_cap, wb) || ensure_dev(&g.d_s, &g.d_s_cap, sb)) return -2;
        if (hipMemcpyAsync(g.d_w, w, wb, hipMemcpyHostToDevice, g.stream) != hipSuccess) return -3;
        if (hipMemcpyAsync(g.d_s, scales, sb, hipMemcpyHostToDevice, g.stream) != hipSuccess) return -3;
        g.uploaded += wb + sb;
        wdev = g.d_w;
        sdev = g.d_s;
    }
    launch_matmul_fp8((float *)g.d_y, (const float *)g.d_x, (const uint8_t *)wdev, (const float *)sdev, S, I, O,
                      g.stream);
    if (hipGetLastError() != hipSuccess) return -4;
    if (hipMemcpyAsync(g.h_stage, g.d_y, yb, hipMemcpyDeviceToHost, g.stream) != hipSuccess) return -5;
    if (hipStreamSynchronize(g.stream) != hipSuccess) return -5;
    memcpy(y, g.h_stage, yb);
    return 0;
}

// Keyed FP8 GEMV on device pointers: the matrix under `key` must be resident
// in the keyed HBM cache (colizig_hip_matrix_load, or an earlier
// colizig_cuda_matmul_fp8 with the same key).
// rows per wave: 2 when that still leaves kGemvRows2Blocks workgroups
constexpr int kGemvRows2Blocks = 256;

template <int NB>
void launch_gemv_fp8(float *y, const float *x, const uint8_t *w, const float *s, int S, int O, hipStream_t st) {
    constexpr int ST = NB >= 32 ? 128 / NB : 4;  // tokens staged per pass: at most 32 KiB of LDS
    if ((O + 7) / 8 >= kGemvRows2Blocks)
        k_gemv_fp8<NB, ST, 2><<<(O + 7) / 8, 256, 0, st>>>(y, x, w, s, (uint32_t)S, (uint32_t)O);
    else
        k_gemv_fp8<NB, ST, 1><<<(O + 3) / 4, 256, 0, st>>>(y, x, w, s, (uint32_t)S, (uint32_t)O);
}

// y[S][O] = x[S][I] . dequant(W)^T on device pointers (matmulFp8's
// contract, fp8.zig:215-257): the row-parallel GEMV for I = 64 x {4, 8, 16,
// 32, 48, 64} (rows 16-byte aligned), else the generic kernel.
void launch_matmul_fp8(float *y, const float *x, const uint8_t *w, const float *s, int S, int I, int O,
                       hipStream_t st) {
    switch ((I % 64) ? 0 : I / 64) {
        case 4: launch_gemv_fp8<4>(y, x, w, s, S, O, st); return;
        case 8: launch_gemv_fp8<8>(y, x, w, s, S, O, st); return;
        case 16: launch_gemv_fp8<16>(y, x, w, s, S, O, st); return;
        case 32: launch_gemv_fp8<32>(y, x, w, s, S, O, st); return;
        case 48: launch_gemv_fp8<48>(y, x, w, s, S, O, st); return;
        case 64: launch_gemv_fp8<64>(y, x, w, s, S, O, st); return;
        default: k_gemm_fp8_generic<<<(O + 3) / 4, 256, 0, st>>>(y, x, w, s, S, I, O); return;
    }
}

template <int NB>
void launch_gemv_fp8_multi(GemvMulti G, const float *x, int S, hipStream_t st) {
    constexpr int ST = NB >= 32 ? 128 / NB : 4;
    uint32_t b8 = 0;
    for (uint32_t m = 0; m < G.n; ++m) b8 += (G.O[m] + 7) / 8;
    const int rw = b8 >= (uint32_t)kGemvRows2Blocks ? 2 : 1;
    uint32_t b = 0;
    for (uint32_t m = 0; m < G.n; ++m) {
        G.blk0[m] = b;
        b += (G.O[m] + 4 * rw - 1) / (4 * rw);
    }
    G.blk0[G.n] = b;
    if (rw == 2)
        k_gemv_fp8_multi<NB, ST, 2><<<b, 256, 0, st>>>(G, x, (uint32_t)S);
    else
        k_gemv_fp8_multi<NB, ST, 1><<<b, 256, 0, st>>>(G, x, (uint32_t)S);
}

extern "C" int colizig_hip_matrix_load(uint64_t key, const unsigned char *w, const float *scales, int I, int O) {
    CsrGuard csr;
    std::lock_guard<std::recursive_mutex> lk(g_mu);
    if (!g.inited || key == 0 || I < 1 || O < 1 || !w || !scales) return -1;
    if (g.budget == 0) {
        snprintf(g_err, sizeof g_err, "matrix_load: no HBM cache budget (colizig_cuda_set_vram_budget)");
        return -8;
    }
    const size_t wb = (size_t)O * I, sb = (size_t)nblk((uint32_t)O) * nblk((uint32_t)I) * sizeof(float);
    const int i = cache_slot_for(key, wb, sb);
    if (i < 0) {
        snprintf(g_err, sizeof g_err, "matrix_load: no cache slot for %zu bytes", wb + sb);
        return -2;
    }
    Slot &sl = g.slots[i];
    if (sl.wcap < wb || sl.scap < sb) {  // the key was resident with a smaller matrix
        snprintf(g_err, sizeof g_err, "matrix_load: key resident with another shape");
        return -1;
    }
    CZ_CHECK(hipMemcpyAsync(sl.w, w, wb, hipMemcpyHostToDevice, g.stream), -3);
    CZ_CHECK(hipMemcpyAsync(sl.s, scales, sb, hipMemcpyHostToDevice, g.stream), -3);
    CZ_CHECK(hipStreamSynchronize(g.stream), -3);
    g.uploaded += wb + sb;
    if (sl.key != key) g.misses++;
    sl.key = key;
    sl.I = I;
    sl.O = O;
    sl.bf16 = 0;
    g.by_key[key] = i;
    sl.clock = ++g.lru;
    return 0;
}

extern "C" int colizig_hip_matrix_load_bf16(uint64_t key, const uint16_t *w, int I, int O) {
    CsrGuard csr;
    std::lock_guard<std::recursive_mutex> lk(g_mu);
    if (!g.inited || key == 0 || I < 1 || O < 1 || !w) return -1;
    if (g.budget == 0) {
        snprintf(g_err, sizeof g_err, "matrix_load_bf16: no HBM cache budget (colizig_cuda_set_vram_budget)");
        return -8;
    }
    const size_t wb = (size_t)O * I * sizeof(uint16_t);
    const int i = cache_slot_for(key, wb, 16);
    if (i < 0) {
        snprintf(g_err, sizeof g_err, "matrix_load_bf16: no cache slot for %zu bytes", wb);
        return -2;
    }
    Slot &sl = g.slots[i];
    if (sl.wcap < wb) {
        snprintf(g_err, sizeof g_err, "matrix_load_bf16: key resident with another shape");
        return -1;
    }
    CZ_CHECK(hipMemcpyAsync(sl.w, w, wb, hipMemcpyHostToDevice, g.stream), -3);
    CZ_CHECK(hipStreamSynchronize(g.stream), -3);
    g.uploaded += wb;
    if (sl.key != key) g.misses++;
    sl.key = key;
    sl.I = I;
    sl.O = O;
    sl.bf16 = 1;
    g.by_key[key] = i;
    sl.clock = ++g.lru;
    return 0;
}

extern "C" int colizig_hip_matmul_bf16_dev(float *y_dev, const float *x_dev, int S, int I, int O, uint64_t key,
                                           void *stream) {
    CsrGuard csr;
    std::lock_guard<std::recursive_mutex> lk(g_mu);
    if (!g.inited || S < 1 || I < 1 || O < 1 || !y_dev || !x_dev || !dev_aligned(x_dev, y_dev)) return -1;
    const auto it = g.by_key.find(key);
    if (key == 0 || it == g.by_key.end()) {
        snprintf(g_err, sizeof g_err, "matmul_bf16_dev: key %llu not resident", (unsigned long long)key);
        return -7;
    }
    Slot &sl = g.slots[it->second];
    if (!sl.bf16 || sl.I != I || sl.O != O) {
        snprintf(g_err, sizeof g_err, "matmul_bf16_dev: key resident as %s %d x %d, called as BF16 %d x %d",
                 sl.bf16 ? "BF16" : "FP8", sl.O, sl.I, O, I);
        return -1;
    }
    sl.clock = ++g.lru;
    g.hits++;
    const hipStream_t st = pick_stream(stream);
    launch_gemv_native<uint16_t>(y_dev, x_dev, (const uint16_t *)sl.w, S, I, O, st);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) {
        snprintf(g_err, sizeof g_err, "matmul_bf16_dev launch: %s", hipGetErrorString(e));
        return -4;
    }
    return 0;
}

extern "C" int colizig_hip_matmul_fp8_dev(float *y_dev, const float *x_dev, int S, int I, int O, uint64_t key,
                                          void *stream) {
    CsrGuard csr;
    std::lock_guard<std::recursive_mutex> lk(g_mu);
    if (!g.inited || S < 1 || I < 1 || O < 1 || !y_dev || !x_dev || !dev_aligned(x_dev, y_dev)) return -1;
    const auto it = g.by_key.find(key);
    if (key == 0 || it == g.by_key.end()) {
        snprintf(g_err, sizeof g_err, "matmul_fp8_dev: key %llu not resident", (unsigned long long)key);
        return -7;
    }
    Slot &sl = g.slots[it->second];
    if (sl.bf16 || sl.I != I || sl.O != O) {
        snprintf(g_err, sizeof g_err, "matmul_fp8_dev: key resident as %s %d x %d, called as FP8 %d x %d",
                 sl.bf16 ? "BF16" : "FP8", sl.O, sl.I, O, I);
        return -1;
    }
    sl.clock = ++g.lru;
    g.hits++;
    const hipStream_t st = pick_stream(stream);
    launch_matmul_fp8(y_dev, x_dev, (const uint8_t *)sl.w, (const float *)sl.s, S, I, O, st);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) {
        snprintf(g_err, sizeof g_err, "matmul_fp8_dev launch: %s", hipGetErrorString(e));
        return -4;
    }
    return 0;
}

// Several keyed FP8 matrices of one row width on the same input rows in one
// launch: y_devs[m][S][Os[m]] = x . dequant(W_keys[m])^T, each bit-identical
// to colizig_hip_matmul_fp8_dev of that key alone (the same per-row kernel
// body).  For a caller that has the q, k and v projections of a layer
// together (attn.zig:206-208 makes them three matmulFp8Keyed calls): one
// launch instead of three.  n in 1..4; every key resident as FP8 [Os[m]][I].
extern "C" int colizig_hip_matmul_fp8_dev_multi(int n, float *const *y_devs, const uint64_t *keys, const int *Os,
                                                const float *x_dev, int S, int I, void *stream) {
    CsrGuard csr;
    std::lock_guard<std::recursive_mutex> lk(g_mu);
    if (!g.inited || n < 1 || n > CZ_GEMV_MULTI || !y_devs || !keys || !Os || !x_dev || S < 1 || I < 1) return -1;
    GemvMulti G{};
    G.n = (uint32_t)n;
    for (int m = 0; m < n; ++m) {
        if (!y_devs[m] || Os[m] < 1 || !dev_aligned(x_dev, y_devs[m])) return -1;
        const auto it = g.by_key.find(keys[m]);
        if (keys[m] == 0 || it == g.by_key.end()) {
            snprintf(g_err, sizeof g_err, "matmul_fp8_dev_multi: key %llu not resident", (unsigned long long)keys[m]);
            return -7;
        }
        Slot &sl = g.slots[it->second];
        if (sl.bf16 || sl.I != I || sl.O != Os[m]) {
            snprintf(g_err, sizeof g_err, "matmul_fp8_dev_multi: key resident as %s %d x %d, called as FP8 %d x %d",
                     sl.bf16 ? "BF16" : "FP8", sl.O, sl.I, Os[m], I);
            return -1;
        }
        sl.clock = ++g.lru;
        g.hits++;
        G.y[m] = y_devs[m];
        G.w[m] = (const uint8_t *)sl.w;
        G.s[m] = (const float *)sl.s;
        G.O[m] = (uint32_t)Os[m];
    }
    const hipStream_t st = pick_stream(stream);
    switch ((I % 64) ? 0 : I / 64) {
        case 4: launch_gemv_fp8_multi<4>(G, x_dev, S, st); break;
        case 8: launch_gemv_fp8_multi<8>(G, x_dev, S, st); break;
        case 16: launch_gemv_fp8_multi<16>(G, x_dev, S, st); break;
        case 32: launch_gemv_fp8_multi<32>(G, x_dev, S, st); break;
        case 48: launch_gemv_fp8_multi<48>(G, x_dev, S, st); break;
        case 64: launch_gemv_fp8_multi<64>(G, x_dev, S, st); break;
        default:  // another row width: one launch per matrix
            for (int m = 0; m < n; ++m) launch_matmul_fp8(G.y[m], x_dev, G.w[m], G.s[m], S, I, Os[m], st);
    }
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) {
        snprintf(g_err, sizeof g_err, "matmul_fp8_dev_multi launch: %s", hipGetErrorString(e));
        return -4;
    }
    return 0;
}

// ===========================================================================
// 2. MoE-level extensions
// ===========================================================================
extern "C" int colizig_hip_dequant_fp8(float *out, const unsigned char *w, const float *scales, int rows, int cols) {
    CsrGuard csr;
    std::lock_guard<std::recursive_mutex> lk(g_mu);
    if (!g.inited || rows < 1 || cols < 1 || !out || !w || !scales) return -1;
    const size_t n = (size_t)rows * cols, sb = (size_t)nblk(rows) * nblk(cols) * sizeof(float);
    void *dw = nullptr, *ds = nullptr, *dout = nullptr;
    int rc = 0;
    if (hipMalloc(&dw, (n + 3) & ~(size_t)3) != hipSuccess || hipMalloc(&ds, sb) != hipSuccess ||
        hipMalloc(&dout, n * sizeof(float)) != hipSuccess) {
        rc = -2;
        goto done;
    }
    if (hipMemcpy(dw, w, n, hipMemcpyHostToDevice) != hipSuccess ||
        hipMemcpy(ds, scales, sb, hipMemcpyHostToDevice) != hipSuccess) {
        rc = -3;
        goto done;
    }
    {
        const uint64_t work = (cols % 4 == 0) ? n / 4 : n;
        const uint32_t blocks = (uint32_t)std::min<uint64_t>((work + 255) / 256, 65536);
        k_dequant_fp8<<<blocks, 256, 0, g.stream>>>((float *)dout, (const uint8_t *)dw, (const float *)ds,
                                                    (uint32_t)rows, (uint32_t)cols, nblk(cols));
        if (hipGetLastError() != hipSuccess) {
            rc = -4;
            goto done;
        }
        if (hipStreamSynchronize(g.stream) != hipSuccess ||
            hipMemcpy(out, dout, n * sizeof(float), hipMemcpyDeviceToHost) != hipSuccess)
            rc = -5;
    }
done:
    if (dw) (void)hipFree(dw);
    if (ds) (void)hipFree(ds);
    if (dout) (void)hipFree(dout);
    return rc;
}

extern "C" int colizig_hip_layer_init(uint32_t layer, const colizig_dims *dims, const float *router) {
    CsrGuard csr;
    std::lock_guard<std::recursive_mutex> lk(g_mu);
    if (!g.inited || !dims) return -1;
    const colizig_dims d = *dims;
    if (d.hidden == 0 || d.experts == 0 || d.topk == 0 || d.inter == 0 || d.topk > d.experts ||
        d.experts > CZ_MAX_E || d.topk > CZ_MAX_K || d.hidden > 8192) {
        snprintf(g_err, sizeof g_err, "unsupported dims H=%u E=%u K=%u I=%u", d.hidden, d.experts, d.topk, d.inter);
        return -1;
    }
    (void)hipStreamSynchronize(g.stream);
    if (g.pool.copy) (void)hipStreamSynchronize(g.pool.copy);
    pool_drop_layer(layer);
    auto it = g.layers.find(layer);
    if (it != g.layers.end()) free_layer(it->second);
    LayerHost &L = g.layers[layer];
    L.d = d;
    L.gen = ++g.layer_gen;
    if (hipMalloc(&L.router, (size_t)d.experts * d.hidden * sizeof(float)) != hipSuccess ||
        hipMalloc(&L.ew, L.ew_stride() * d.experts) != hipSuccess ||
        hipMalloc(&L.es, L.es_stride() * d.experts * sizeof(float)) != hipSuccess ||
        hipMalloc(&L.usage, (size_t)d.experts * sizeof(unsigned long long)) != hipSuccess ||
        hipMemset(L.usage, 0, (size_t)d.experts * sizeof(unsigned long long)) != hipSuccess) {
        free_layer(L);
        g.layers.erase(layer);
        snprintf(g_err, sizeof g_err, "layer %u: HBM allocation failed", layer);
        return -2;
    }
    if (d.shared_inter) {
        if (hipMalloc(&L.sw, L.sw_bytes()) != hipSuccess || hipMalloc(&L.ss, L.ss_floats() * sizeof(float)) != hipSuccess ||
            hipMalloc(&L.shg, (size_t)d.hidden * sizeof(float)) != hipSuccess) {
            free_layer(L);
            g.layers.erase(layer);
            return -2;
        }
    }
    L.loaded.assign(d.experts, 0);
    if (router) {
        if (hipMemcpy(L.router, router, (size_t)d.experts * d.hidden * sizeof(float), hipMemcpyHostToDevice) !=
            hipSuccess)
            return -3;
    }
    return 0;
}

extern "C" int colizig_hip_expert_load(uint32_t layer, uint32_t expert, const unsigned char *gate_w,
                                       const float *gate_s, const unsigned char *up_w, const float *up_s,
                                       const unsigned char *down_w, const float *down_s) {
    CsrGuard csr;
    std::lock_guard<std::recursive_mutex> lk(g_mu);
    LayerHost *L = find_layer(layer);
    if (!g.inited || !L || expert >= L->d.experts || !gate_w || !gate_s || !up_w || !up_s || !down_w || !down_s)
        return -1;
    const uint64_t mb = (uint64_t)L->d.inter * L->d.hidden;
    const uint64_t nsc = (uint64_t)nblk(L->d.inter) * nblk(L->d.hidden);
    uint8_t *wb = L->ew + expert * L->ew_stride();
    float *sb = L->es + expert * L->es_stride();
    CZ_CHECK(hipMemcpyAsync(wb, gate_w, mb, hipMemcpyHostToDevice, g.stream), -3);
    CZ_CHECK(hipMemcpyAsync(wb + mb, up_w, mb, hipMemcpyHostToDevice, g.stream), -3);
    CZ_CHECK(hipMemcpyAsync(wb + 2 * mb, down_w, mb, hipMemcpyHostToDevice, g.stream), -3);
    CZ_CHECK(hipMemcpyAsync(sb, gate_s, nsc * 4, hipMemcpyHostToDevice, g.stream), -3);
    CZ_CHECK(hipMemcpyAsync(sb + nsc, up_s, nsc * 4, hipMemcpyHostToDevice, g.stream), -3);
    CZ_CHECK(hipMemcpyAsync(sb + 2 * nsc, down_s, nsc * 4, hipMemcpyHostToDevice, g.stream), -3);
    CZ_CHECK(hipStreamSynchronize(g.stream), -3);
    if (!L->loaded[expert]) {
        L->loaded[expert] = 1;
        L->nloaded++;
    }
    return 0;
}

extern "C" int colizig_hip_layer_set_shared(uint32_t layer, const unsigned char *gate_w, const float *gate_s,
                                            const unsigned char *up_w, const float *up_s,
                                            const unsigned char *down_w, const float *down_s,
                                            const float *sh_gate) {
    CsrGuard csr;
    std::lock_guard<std::recursive_mutex> lk(g_mu);
    LayerHost *L = find_layer(layer);
    if (!g.inited || !L || L->d.shared_inter == 0 || !gate_w || !gate_s || !up_w || !up_s || !down_w || !down_s ||
        !sh_gate)
        return -1;
    const uint64_t mb = (uint64_t)L->d.shared_inter * L->d.hidden;
    const uint64_t nsc = (uint64_t)nblk(L->d.shared_inter) * nblk(L->d.hidden);
    (void)hipStreamSynchronize(g.stream);
    if (L->shn_dtype >= 0) {  // a NativeMatrix shared expert is replaced
        for (void *p : {L->shn_gate, L->shn_up, L->shn_down})
            if (p) (void)hipFree(p);
        L->shn_gate = L->shn_up = L->shn_down = nullptr;
        L->shn_dtype = -1;
        L->gen = ++g.layer_gen;
    }
    if (!L->sw && (hipMalloc(&L->sw, L->sw_bytes()) != hipSuccess ||
                   hipMalloc(&L->ss, L->ss_floats() * sizeof(float)) != hipSuccess))
        return -2;
    CZ_CHECK(hipMemcpyAsync(L->sw, gate_w, mb, hipMemcpyHostToDevice, g.stream), -3);
    CZ_CHECK(hipMemcpyAsync(L->sw + mb, up_w, mb, hipMemcpyHostToDevice, g.stream), -3);
    CZ_CHECK(hipMemcpyAsync(L->sw + 2 * mb, down_w, mb, hipMemcpyHostToDevice, g.stream), -3);
    CZ_CHECK(hipMemcpyAsync(L->ss, gate_s, nsc * 4, hipMemcpyHostToDevice, g.stream), -3);
    CZ_CHECK(hipMemcpyAsync(L->ss + nsc, up_s, nsc * 4, hipMemcpyHostToDevice, g.stream), -3);
    CZ_CHECK(hipMemcpyAsync(L->ss + 2 * nsc, down_s, nsc * 4, hipMemcpyHostToDevice, g.stream), -3);
    CZ_CHECK(hipMemcpyAsync(L->shg, sh_gate, (size_t)L->d.hidden * 4, hipMemcpyHostToDevice, g.stream), -3);
    CZ_CHECK(hipStreamSynchronize(g.stream), -3);
    L->shared_set = true;
    return 0;
}

// A NativeMatrix shared expert (moe.zig:300-303, 316-325: the reference keeps
// shared_expert.{gate,up,down}_proj as f32 or BF16 rows and evaluates them
// with dotF32 / dotBf16): gate, up [SI][H], down [H][SI], dtype 0 f32, 1 BF16
// (raw bits); sh_gate [H] f32.  Replaces a block-FP8 shared expert.
extern "C" int colizig_hip_layer_set_shared_native(uint32_t layer, int dtype, const void *gate, const void *up,
                                                   const void *down, const float *sh_gate) {
    CsrGuard csr;
    std::lock_guard<std::recursive_mutex> lk(g_mu);
    LayerHost *L = find_layer(layer);
    if (!g.inited || !L || L->d.shared_inter == 0 || (dtype != 0 && dtype != 1) || !gate || !up || !down ||
        !sh_gate)
        return -1;
    const size_t es = dtype == 1 ? 2 : 4, mb = (size_t)L->d.shared_inter * L->d.hidden * es;
    (void)hipStreamSynchronize(g.stream);
    for (void *p : {L->shn_gate, L->shn_up, L->shn_down, (void *)L->sw, (void *)L->ss})
        if (p) (void)hipFree(p);
    L->shn_gate = L->shn_up = L->shn_down = nullptr;
    L->sw = nullptr;
    L->ss = nullptr;
    L->shn_dtype = -1;
    L->shared_set = false;
    L->gen = ++g.layer_gen;
    if (hipMalloc(&L->shn_gate, mb) != hipSuccess || hipMalloc(&L->shn_up, mb) != hipSuccess ||
        hipMalloc(&L->shn_down, mb) != hipSuccess) {
        snprintf(g_err, sizeof g_err, "layer %u: shared expert allocation failed", layer);
        return -2;
    }
    CZ_CHECK(hipMemcpy(L->shn_gate, gate, mb, hipMemcpyHostToDevice), -3);
    CZ_CHECK(hipMemcpy(L->shn_up, up, mb, hipMemcpyHostToDevice), -3);
    CZ_CHECK(hipMemcpy(L->shn_down, down, mb, hipMemcpyHostToDevice), -3);
    CZ_CHECK(hipMemcpy(L->shg, sh_gate, (size_t)L->d.hidden * 4, hipMemcpyHostToDevice), -3);
    L->shn_dtype = dtype;
    L->shared_set = true;
    return 0;
}

// A BF16 router (NativeMatrix bf16, tensors.zig:114-119; raw bits [E][H])
// in place of the f32 one: logits in dotBf16's order (matmul.zig:84-110).
extern "C" int colizig_hip_layer_set_router_bf16(uint32_t layer, const uint16_t *router) {
    CsrGuard csr;
    std::lock_guard<std::recursive_mutex> lk(g_mu);
    LayerHost *L = find_layer(layer);
    if (!g.inited || !L || !router) return -1;
    if (L->streamed() && g.pool.on) (void)hipStreamSynchronize(g.pool.copy);
    (void)hipStreamSynchronize(g.stream);
    const size_t n = (size_t)L->d.experts * L->d.hidden;
    if (!L->router_bf16 && hipMalloc(&L->router_bf16, n * 2) != hipSuccess) {
        L->router_bf16 = nullptr;
        return -2;
    }
    CZ_CHECK(hipMemcpy(L->router_bf16, router, n * 2, hipMemcpyHostToDevice), -3);
    if (L->router) (void)hipFree(L->router);
    L->router = nullptr;
    L->gen = ++g.layer_gen;
    return 0;
}

extern "C" int colizig_hip_layer_set_router_bias(uint32_t layer, const float *bias) {
    CsrGuard csr;
    std::lock_guard<std::recursive_mutex> lk(g_mu);
    LayerHost *L = find_layer(layer);
    if (!g.inited || !L) return -1;
    (void)hipStreamSynchronize(g.stream);
    if (!bias) {
        if (L->rbias) {
            (void)hipFree(L->rbias);
            L->gen = ++g.layer_gen;
        }
        L->rbias = nullptr;
        return 0;
    }
    if (!L->rbias) {
        L->gen = ++g.layer_gen;
        if (hipMalloc(&L->rbias, (size_t)L->d.experts * sizeof(float)) != hipSuccess) {
            L->rbias = nullptr;
            return -2;
        }
    }
    CZ_CHECK(hipMemcpy(L->rbias, bias, (size_t)L->d.experts * sizeof(float), hipMemcpyHostToDevice), -3);
    return 0;
}

extern "C" int colizig_hip_moe_forward_dev(uint32_t layer, const float *x_dev, int S, float *out_dev,
                                           uint32_t *idx_dev, float *gates_dev, void *stream) {
    CsrGuard csr;
    std::lock_guard<std::recursive_mutex> lk(g_mu);
    if (!g.inited || S < 1 || !x_dev || !out_dev || !dev_aligned(x_dev, out_dev)) return -1;
    LayerHost *L = find_layer(layer);
    int rc = check_layer_ready(L, layer);
    if (rc) return rc;
    if ((rc = ensure_work(L->d, S))) return rc;
    if (grouped_ok(L->d, S) && (rc = ensure_work_grouped(L->d, S))) return rc;
    if (L->streamed()) {
        if ((rc = ensure_work_grouped(L->d, S)) || (rc = ensure_h_idx(S))) return rc ? rc : -2;
        rc = run_streamed_layer(*L, layer, x_dev, S, out_dev, 0, 0.0f, nullptr, nullptr, 0, pick_stream(stream),
                                nullptr);
        if (rc) return rc;
        const size_t kb = (size_t)S * L->d.topk * sizeof(float);
        if (idx_dev) CZ_CHECK(hipMemcpyAsync(idx_dev, g.work.idx, kb, hipMemcpyDeviceToDevice, pick_stream(stream)), -4);
        if (gates_dev) CZ_CHECK(hipMemcpyAsync(gates_dev, g.work.gates, kb, hipMemcpyDeviceToDevice, pick_stream(stream)), -4);
        return 0;
    }
    return launch_layer(*L, x_dev, S, out_dev, 0, 0.0f, nullptr, nullptr, idx_dev, gates_dev, pick_stream(stream));
}

// ---- scratch of colizig_hip_moe_forward_dev_noalloc: one array per GPU,
// held until the process ends.  In host code `scratch` names a host-side
// stand-in, never the device memory: kernels and copies take the address
// hipGetSymbolAddress returns for the current device (noalloc_scratch).
constexpr size_t kNoAllocScratchBytes = 4u << 20;
static __device__ __align__(256) uint8_t scratch[kNoAllocScratchBytes];

namespace {
constexpr int kNoAllocMaxDevices = 64;
uint8_t *g_scratch_dev[kNoAllocMaxDevices] = {};

// Device address of the current device's `scratch`, resolved once per device.
uint8_t *noalloc_scratch() {
    int dev = -1;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kNoAllocMaxDevices) {
        snprintf(g_err, sizeof g_err, "no-alloc forward: no usable current device (%d)", dev);
        return nullptr;
    }
    if (!g_scratch_dev[dev]) {
        void *p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !p) {
            snprintf(g_err, sizeof g_err, "no-alloc forward: hipGetSymbolAddress(scratch) on device %d: %s", dev,
                     hipGetErrorString(e));
            return nullptr;
        }
        g_scratch_dev[dev] = (uint8_t *)p;
    }
    return g_scratch_dev[dev];
}

// Bytes of scratch a decode-regime forward of S tokens needs; each buffer
// starts on a 256-byte boundary.
size_t noalloc_bytes(const colizig_dims &d, int S, size_t off[7]) {
    const size_t s = (size_t)S;
    const size_t n[7] = {s * d.hidden * 4,  s * d.experts * 4, s * d.topk * 4, s * d.topk * 4, s * 4,
                         s * d.topk * (size_t)d.inter * 4, std::max<size_t>(1, s * d.shared_inter) * 4};
    size_t at = 0;
    for (int i = 0; i < 7; ++i) {
        off[i] = at;
        at += (n[i] + 255) & ~(size_t)255;
    }
    return at;
}
}  // namespace

extern "C" int colizig_hip_moe_forward_dev_noalloc(uint32_t layer, const float *x_dev, int S, float *out_dev,
                                                   uint32_t *idx_dev, float *gates_dev, void *stream) {
    CsrGuard csr;
    std::lock_guard<std::recursive_mutex> lk(g_mu);
    if (!g.inited || S < 1 || !x_dev || !out_dev || !dev_aligned(x_dev, out_dev)) return -1;
    LayerHost *L = find_layer(layer);
    int rc = check_layer_ready(L, layer);
    if (rc) return rc;
    if (L->streamed()) {
        snprintf(g_err, sizeof g_err, "no-alloc forward: layer %u is streamed; only resident layers are served",
                 layer);
        return -1;
    }
    if (grouped_ok(L->d, S)) {
        snprintf(g_err, sizeof g_err, "no-alloc forward: S=%d takes the grouped regime (S >= %d), which this "
                 "entry point does not serve", S, kGroupedMinTokens);
        return -1;
    }
    if (L->shn_dtype >= 0) {
        snprintf(g_err, sizeof g_err, "no-alloc forward: layer %u has a NativeMatrix shared expert, which this "
                 "entry point does not serve", layer);
        return -1;
    }
    size_t off[7];
    const size_t need = noalloc_bytes(L->d, S, off);
    if (need > kNoAllocScratchBytes) {
        snprintf(g_err, sizeof g_err, "no-alloc forward: S=%d needs %zu bytes of scratch, more than the %zu "
                 "available", S, need, kNoAllocScratchBytes);
        return -1;
    }
    uint8_t *base = noalloc_scratch();
    if (!base) return -2;
    StepArgs A{};
    A.L = L->dev();
    A.x = x_dev;
    A.xn = (float *)(base + off[0]);
    A.logits = (float *)(base + off[1]);
    A.idx = (uint32_t *)(base + off[2]);
    A.gates = (float *)(base + off[3]);
    A.sgate = (float *)(base + off[4]);
    A.h = (float *)(base + off[5]);
    A.hs = (float *)(base + off[6]);
    A.out = out_dev;
    A.idx_trace = idx_dev;
    A.gates_trace = gates_dev;
    A.S = S;
    A.tt = router_tokens_per_tile(L->d.hidden);
    return launch_step(A, pick_stream(stream));
}

extern "C" int colizig_hip_moe_forward(uint32_t layer, const float *x, int S, float *out, uint32_t *routed_idx,
                                       float *routed_gates) {
    CsrGuard csr;
    std::lock_guard<std::recursive_mutex> lk(g_mu);
    if (!g.inited || S < 1 || !x || !out) return -1;
    LayerHost *L = find_layer(layer);
    int rc = check_layer_ready(L, layer);
    if (rc) return rc;
    if ((rc = ensure_work(L->d, S))) return rc;
    if (grouped_ok(L->d, S) && (rc = ensure_work_grouped(L->d, S))) return rc;
    const size_t xb = (size_t)S * L->d.hidden * sizeof(float);
    const size_t kb = (size_t)S * L->d.topk * sizeof(float);
    if (ensure_host(xb + 2 * kb)) return -2;
    memcpy(g.h_stage, x, xb);
    CZ_CHECK(hipMemcpyAsync(g.work.xin, g.h_stage, xb, hipMemcpyHostToDevice, g.stream), -3);
    if (L->streamed()) {
        if ((rc = ensure_work_grouped(L->d, S)) || (rc = ensure_h_idx(S))) return rc ? rc : -2;
        rc = run_streamed_layer(*L, layer, g.work.xin, S, g.work.out, 0, 0.0f, nullptr, nullptr, 0, g.stream,
                                nullptr);
    } else {
        rc = launch_layer(*L, g.work.xin, S, g.work.out, 0, 0.0f, nullptr, nullptr, nullptr, nullptr, g.stream);
    }
    if (rc) return rc;
    char *hs = (char *)g.h_stage;
    CZ_CHECK(hipMemcpyAsync(hs, g.work.out, xb, hipMemcpyDeviceToHost, g.stream), -5);
    CZ_CHECK(hipMemcpyAsync(hs + xb, g.work.idx, kb, hipMemcpyDeviceToHost, g.stream), -5);
    CZ_CHECK(hipMemcpyAsync(hs + xb + kb, g.work.gates, kb, hipMemcpyDeviceToHost, g.stream), -5);
    CZ_CHECK(hipStreamSynchronize(g.stream), -5);
    memcpy(out, hs, xb);
    if (routed_idx) memcpy(routed_idx, hs + xb, kb);
    if (routed_gates) memcpy(routed_gates, hs + xb + kb, kb);
    return 0;
}

static int chain_enqueue(uint32_t layer0, uint32_t nlayers, float *x_dev, int S, float eps, float *xn_trace,
                         uint32_t *idx_trace, float *gates_trace, hipStream_t st) {
    for (uint32_t l = 0; l < nlayers; ++l) {
        LayerHost *L = find_layer(layer0 + l);
        int rc = check_layer_ready(L, layer0 + l);
        if (rc) return rc;
        if (L->streamed()) {
            snprintf(g_err, sizeof g_err, "layer %u streams from host memory: use colizig_hip_stream_decode",
                     layer0 + l);
            return -1;
        }
        if ((rc = ensure_work(L->d, S))) return rc;
        if (grouped_ok(L->d, S) && (rc = ensure_work_grouped(L->d, S))) return rc;
    }
    const int fz = chain_fused_prepare(layer0, nlayers, S);
    if (fz < 0) return fz;
    if (fz) return chain_enqueue_fused(layer0, nlayers, x_dev, eps, xn_trace, idx_trace, gates_trace, st);
    // grouped layers: each layer's combine forms the next layer's RMS rows
    bool ready = false;
    for (uint32_t l = 0; l < nlayers; ++l) {
        LayerHost *L = find_layer(layer0 + l);
        const LayerHost *N = l + 1 < nlayers ? find_layer(layer0 + l + 1) : nullptr;
        if (N && !combine_rms_ok(*L, *N, S)) N = nullptr;
        const size_t sh = (size_t)S * L->d.hidden, sk = (size_t)S * L->d.topk;
        const int rc = launch_layer(*L, x_dev, S, x_dev, 1, eps, x_dev, xn_trace ? xn_trace + l * sh : nullptr,
                                    idx_trace ? idx_trace + l * sk : nullptr,
                                    gates_trace ? gates_trace + l * sk : nullptr, st, ready, N,
                                    N && xn_trace ? xn_trace + (l + 1) * sh : nullptr);
        if (rc) return rc;
        ready = N != nullptr;
    }
    return 0;
}

extern "C" int colizig_hip_chain_decode(uint32_t layer0, uint32_t nlayers, float *x_dev, int S, float eps,
                                        float *xn_trace, uint32_t *idx_trace, float *gates_trace, void *stream) {
    CsrGuard csr;
    std::lock_guard<std::recursive_mutex> lk(g_mu);
    if (!g.inited || S < 1 || !x_dev || nlayers == 0 || !dev_aligned(x_dev)) return -1;
    return chain_enqueue(layer0, nlayers, x_dev, S, eps, xn_trace, idx_trace, gates_trace, pick_stream(stream));
}

extern "C" int64_t colizig_hip_chain_graph_create(uint32_t layer0, uint32_t nlayers, float *x_dev, int S,
                                                  float eps) {
    CsrGuard csr;
    std::lock_guard<std::recursive_mutex> lk(g_mu);
    if (!g.inited || S < 1 || !x_dev || nlayers == 0 || !dev_aligned(x_dev)) return -1;
    // allocate scratch before capture (no allocation inside a capture)
    for (uint32_t l = 0; l < nlayers; ++l) {
        LayerHost *L = find_layer(layer0 + l);
        int rc = check_layer_ready(L, layer0 + l);
        if (rc) return rc;
        if ((rc = ensure_work(L->d, S))) return rc;
        if (grouped_ok(L->d, S) && (rc = ensure_work_grouped(L->d, S))) return rc;
    }
    if (const int fz = chain_fused_prepare(layer0, nlayers, S); fz < 0) return fz;
    CZ_CHECK(hipStreamSynchronize(g.stream), -4);
    hipGraph_t graph = nullptr;
    CZ_CHECK(hipStreamBeginCapture(g.stream, hipStreamCaptureModeThreadLocal), -4);
    const int rc = chain_enqueue(layer0, nlayers, x_dev, S, eps, nullptr, nullptr, nullptr, g.stream);
    const hipError_t ec = hipStreamEndCapture(g.stream, &graph);
    if (rc) {
        if (graph) (void)hipGraphDestroy(graph);
        return rc;
    }
    if (ec != hipSuccess) {
        snprintf(g_err, sizeof g_err, "hipStreamEndCapture: %s", hipGetErrorString(ec));
        return -4;
    }
    hipGraphExec_t exec = nullptr;
    if (hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0) != hipSuccess) {
        (void)hipGraphDestroy(graph);
        return -4;
    }
    const int64_t h = g.next_handle++;
    g.graphs[h] = exec;
    g.graph_defs[h] = graph;
    auto &gl = g.graph_layers[h];
    for (uint32_t l = 0; l < nlayers; ++l) gl.emplace_back(layer0 + l, find_layer(layer0 + l)->gen);
    return h;
}

extern "C" int colizig_hip_graph_launch(int64_t handle, void *stream) {
    CsrGuard csr;
    std::lock_guard<std::recursive_mutex> lk(g_mu);
    auto it = g.graphs.find(handle);
    if (!g.inited || it == g.graphs.end()) return -1;
    // a layer re-registered (or its router bias or expert source changed)
    // since the capture: the graph's kernel arguments point at freed buffers
    for (const auto &lg : g.graph_layers[handle]) {
        const LayerHost *L = find_layer(lg.first);
        if (!L || L->gen != lg.second) {
            snprintf(g_err, sizeof g_err, "graph %lld: layer %u changed since capture; create the graph again",
                     (long long)handle, lg.first);
            return -1;
        }
    }
    CZ_CHECK(hipGraphLaunch(it->second, pick_stream(stream)), -4);
    return 0;
}

extern "C" void colizig_hip_graph_destroy(int64_t handle) {
    std::lock_guard<std::recursive_mutex> lk(g_mu);
    auto it = g.graphs.find(handle);
    if (it == g.graphs.end()) return;
    (void)hipStreamSynchronize(g.stream);
    (void)hipGraphExecDestroy(it->second);
    g.graphs.erase(it);
    auto jt = g.graph_defs.find(handle);
    if (jt != g.graph_defs.end()) {
        (void)hipGraphDestroy(jt->second);
        g.graph_defs.erase(jt);
    }
    g.graph_layers.erase(handle);
}

// ---- synthetic weights -----------------------------------------------------
__global__ __launch_bounds__(256) void k_synth_fp8_experts(uint8_t *ew, float *es, uint64_t ew_stride,
                                                           uint64_t es_stride, uint64_t w_off, uint64_t s_off,
                                                           uint32_t rows, uint32_t cols, uint64_t seed, float stdv) {
    const uint32_t e = blockIdx.y;
    uint8_t *w = ew + (uint64_t)e * ew_stride + w_off;
    float *sc = es + (uint64_t)e * es_stride + s_off;
    const uint32_t nbc = (cols + CZ_BLOCK - 1) / CZ_BLOCK;
    const uint32_t br = blockIdx.x / nbc, bc = blockIdx.x - br * nbc;
    const uint32_t r_lo = br * CZ_BLOCK, c_lo = bc * CZ_BLOCK;
    const uint32_t nr = min((uint32_t)CZ_BLOCK, rows - r_lo), nc = min((uint32_t)CZ_BLOCK, cols - c_lo);
    const uint32_t rr = threadIdx.x >> 1, ch = (threadIdx.x & 1) * 64;
    const uint64_t mseed = cz_mix64(seed ^ cz_mix64(0x5eedull + e));
    float v[64];
    float amax = 0.0f;
#pragma unroll
    for (int c = 0; c < 64; ++c) {
        const uint32_t col = ch + c;
        float val = 0.0f;
        if (rr < nr && col < nc) val = stdv * cz_normal(mseed, (uint64_t)(r_lo + rr) * cols + (c_lo + col));
        v[c] = val;
        amax = fmaxf(amax, fabsf(val));
    }
    amax = cz_wave_max(amax);
    __shared__ float wmax[4];
    if ((threadIdx.x & 63) == 0) wmax[threadIdx.x >> 6] = amax;
    __syncthreads();
    amax = fmaxf(fmaxf(wmax[0], wmax[1]), fmaxf(wmax[2], wmax[3]));
    const float scale = amax > 0.0f ? amax / 448.0f : 1.0f;
    if (threadIdx.x == 0) sc[blockIdx.x] = scale;
    if (rr < nr) {
        uint8_t *row = w + (uint64_t)(r_lo + rr) * cols + c_lo;
#pragma unroll
        for (int c = 0; c < 64; c += 2) {
            float a = fminf(fmaxf(v[c] / scale, -448.0f), 448.0f);
            float b = fminf(fmaxf(v[c + 1] / scale, -448.0f), 448.0f);
            const int packed = __builtin_amdgcn_cvt_pk_fp8_f32(a, b, 0, false);
            const uint32_t col = ch + c;
            if (col < nc) row[col] = (uint8_t)(packed & 0xff);
            if (col + 1 < nc) row[col + 1] = (uint8_t)((packed >> 8) & 0xff);
        }
    }
}

extern "C" int colizig_hip_layer_synth(uint32_t layer, uint64_t seed, float std_w, float std_router) {
    CsrGuard csr;
    std::lock_guard<std::recursive_mutex> lk(g_mu);
    LayerHost *L = find_layer(layer);
    if (!g.inited || !L) return -1;
    if (L->streamed() || !L->router || L->shn_dtype >= 0 || (L->d.shared_inter && !L->sw)) {
        snprintf(g_err, sizeof g_err, "layer %u streams from host memory or holds NativeMatrix weights: synthesis "
                 "writes the f32 router and block-FP8 experts of a resident layer", layer);
        return -1;
    }
    const colizig_dims &d = L->d;
    const uint64_t ls = mix64(seed ^ mix64(0xC011716ull + layer));
    const uint64_t rn = (uint64_t)d.experts * d.hidden;
    k_synth_f32<<<(uint32_t)std::min<uint64_t>((rn + 255) / 256, 16384), 256, 0, g.stream>>>(L->router, rn,
                                                                                             mix64(ls + 1), std_router);
    const uint32_t nbH = nblk(d.hidden), nbI = nblk(d.inter);
    const uint64_t mb = (uint64_t)d.inter * d.hidden, nsc = (uint64_t)nbI * nbH;
    // gate, up: [I][H]; down: [H][I]
    const struct { uint64_t woff, soff; uint32_t rows, cols; } roles[3] = {
        {0, 0, d.inter, d.hidden}, {mb, nsc, d.inter, d.hidden}, {2 * mb, 2 * nsc, d.hidden, d.inter}};
    for (int r = 0; r < 3; ++r) {
        const dim3 grid(nblk(roles[r].rows) * nblk(roles[r].cols), d.experts);
        k_synth_fp8_experts<<<grid, 256, 0, g.stream>>>(L->ew, L->es, L->ew_stride(), L->es_stride(), roles[r].woff,
                                                        roles[r].soff, roles[r].rows, roles[r].cols,
                                                        mix64(ls + 10 + r), std_w);
    }
    if (d.shared_inter) {
        const uint64_t smb = (uint64_t)d.shared_inter * d.hidden, snsc = (uint64_t)nblk(d.shared_inter) * nbH;
        const struct { uint64_t woff, soff; uint32_t rows, cols; } sroles[3] = {
            {0, 0, d.shared_inter, d.hidden}, {smb, snsc, d.shared_inter, d.hidden},
            {2 * smb, 2 * snsc, d.hidden, d.shared_inter}};
        for (int r = 0; r < 3; ++r) {
            const dim3 grid(nblk(sroles[r].rows) * nblk(sroles[r].cols), 1);
            k_synth_fp8_experts<<<grid, 256, 0, g.stream>>>(L->sw, L->ss, 0, 0, sroles[r].woff, sroles[r].soff,
                                                            sroles[r].rows, sroles[r].cols, mix64(ls + 20 + r),
                                                            std_w);
        }
        k_synth_f32<<<(d.hidden + 255) / 256, 256, 0, g.stream>>>(L->shg, d.hidden, mix64(ls + 30), std_router);
        L->shared_set = true;
    }
    if (hipGetLastError() != hipSuccess) return -4;
    CZ_CHECK(hipStreamSynchronize(g.stream), -5);
    std::fill(L->loaded.begin(), L->loaded.end(), 1);
    L->nloaded = d.experts;
    return 0;
}

extern "C" int colizig_hip_expert_read(uint32_t layer, uint32_t expert, unsigned char *gate_w, float *gate_s,
                                       unsigned char *up_w, float *up_s, unsigned char *down_w, float *down_s) {
    CsrGuard csr;
    std::lock_guard<std::recursive_mutex> lk(g_mu);
    LayerHost *L = find_layer(layer);
    if (!g.inited || !L || expert >= L->d.experts) return -1;
    if (L->streamed()) {
        snprintf(g_err, sizeof g_err, "layer %u streams from host memory", layer);
        return -1;
    }
    const uint64_t mb = (uint64_t)L->d.inter * L->d.hidden;
    const uint64_t nsc = (uint64_t)nblk(L->d.inter) * nblk(L->d.hidden);
    const uint8_t *wb = L->ew + expert * L->ew_stride();
    const float *sb = L->es + expert * L->es_stride();
    CZ_CHECK(hipStreamSynchronize(g.stream), -5);
    if (gate_w) CZ_CHECK(hipMemcpy(gate_w, wb, mb, hipMemcpyDeviceToHost), -5);
    if (up_w) CZ_CHECK(hipMemcpy(up_w, wb + mb, mb, hipMemcpyDeviceToHost), -5);
    if (down_w) CZ_CHECK(hipMemcpy(down_w, wb + 2 * mb, mb, hipMemcpyDeviceToHost), -5);
    if (gate_s) CZ_CHECK(hipMemcpy(gate_s, sb, nsc * 4, hipMemcpyDeviceToHost), -5);
    if (up_s) CZ_CHECK(hipMemcpy(up_s, sb + nsc, nsc * 4, hipMemcpyDeviceToHost), -5);
    if (down_s) CZ_CHECK(hipMemcpy(down_s, sb + 2 * nsc, nsc * 4, hipMemcpyDeviceToHost), -5);
    return 0;
}

extern "C" int colizig_hip_router_read(uint32_t layer, float *router) {
    CsrGuard csr;
    std::lock_guard<std::recursive_mutex> lk(g_mu);
    LayerHost *L = find_layer(layer);
    if (!g.inited || !L || !router) return -1;
    CZ_CHECK(hipStreamSynchronize(g.stream), -5);
    const size_t n = (size_t)L->d.experts * L->d.hidden;
    if (L->router_bf16) {  // widened (exact)
        std::vector<uint16_t> b(n);
        CZ_CHECK(hipMemcpy(b.data(), L->router_bf16, n * 2, hipMemcpyDeviceToHost), -5);
        for (size_t i = 0; i < n; ++i) {
            const uint32_t u = (uint32_t)b[i] << 16;
            memcpy(router + i, &u, 4);
        }
        return 0;
    }
    CZ_CHECK(hipMemcpy(router, L->router, n * 4, hipMemcpyDeviceToHost), -5);
    return 0;
}

extern "C" int colizig_hip_shared_read(uint32_t layer, unsigned char *gate_w, float *gate_s, unsigned char *up_w,
                                       float *up_s, unsigned char *down_w, float *down_s, float *sh_gate) {
    CsrGuard csr;
    std::lock_guard<std::recursive_mutex> lk(g_mu);
    LayerHost *L = find_layer(layer);
    if (!g.inited || !L || L->d.shared_inter == 0 || !L->sw) return -1;  // none, or NativeMatrix rows
    const uint64_t mb = (uint64_t)L->d.shared_inter * L->d.hidden;
    const uint64_t nsc = (uint64_t)nblk(L->d.shared_inter) * nblk(L->d.hidden);
    CZ_CHECK(hipStreamSynchronize(g.stream), -5);
    if (gate_w) CZ_CHECK(hipMemcpy(gate_w, L->sw, mb, hipMemcpyDeviceToHost), -5);
    if (up_w) CZ_CHECK(hipMemcpy(up_w, L->sw + mb, mb, hipMemcpyDeviceToHost), -5);
    if (down_w) CZ_CHECK(hipMemcpy(down_w, L->sw + 2 * mb, mb, hipMemcpyDeviceToHost), -5);
    if (gate_s) CZ_CHECK(hipMemcpy(gate_s, L->ss, nsc * 4, hipMemcpyDeviceToHost), -5);
    if (up_s) CZ_CHECK(hipMemcpy(up_s, L->ss + nsc, nsc * 4, hipMemcpyDeviceToHost), -5);
    if (down_s) CZ_CHECK(hipMemcpy(down_s, L->ss + 2 * nsc, nsc * 4, hipMemcpyDeviceToHost), -5);
    if (sh_gate) CZ_CHECK(hipMemcpy(sh_gate, L->shg, (size_t)L->d.hidden * 4, hipMemcpyDeviceToHost), -5);
    return 0;
}

// ---- per-kernel timing pass --------------------------------------------------
// One eager chain step leaves valid routing/scratch state; then, per kernel
// kind, a HIP graph of `reps` passes over the layers launching only that
// kernel (same arguments as in the chain; the down kernel writes to scratch so
// x is left as the chain step made it) is replayed between two events.
extern "C" int colizig_hip_chain_kernel_times(uint32_t layer0, uint32_t nlayers, float *x_dev, int S, float eps,
                                              int reps, float *us_out) {
    CsrGuard csr;
    std::lock_guard<std::recursive_mutex> lk(g_mu);
    if (!g.inited || S < 1 || !x_dev || nlayers == 0 || reps < 1 || !us_out || !dev_aligned(x_dev)) return -1;
    for (uint32_t l = 0; l < nlayers; ++l) {
        LayerHost *L = find_layer(layer0 + l);
        int rc = check_layer_ready(L, layer0 + l);
        if (rc) return rc;
        if (L->streamed()) return -1;
        if ((rc = ensure_work(L->d, S))) return rc;
        if (grouped_ok(L->d, S) && (rc = ensure_work_grouped(L->d, S))) return rc;
    }
    std::vector<StepArgs> args;
    for (uint32_t l = 0; l < nlayers; ++l) {
        const LayerHost &L = *find_layer(layer0 + l);
        args.push_back(step_args(L, x_dev, S, x_dev, 1, eps, x_dev, nullptr, nullptr, nullptr));
    }
    for (const StepArgs &A : args) {
        const int rc = launch_step(A, g.stream);
        if (rc) return rc;
    }
    CZ_CHECK(hipStreamSynchronize(g.stream), -5);
    hipEvent_t e0 = nullptr, e1 = nullptr;
    CZ_CHECK(hipEventCreate(&e0), -2);
    CZ_CHECK(hipEventCreate(&e1), -2);
    const int kinds[3] = {kRouter, kUp, kDown};
    int rc = 0;
    for (int k = 0; k < 3 && rc == 0; ++k) {
        hipGraph_t graph = nullptr;
        hipGraphExec_t exec = nullptr;
        if (hipStreamBeginCapture(g.stream, hipStreamCaptureModeThreadLocal) != hipSuccess) { rc = -4; break; }
        for (int r = 0; r < reps && rc == 0; ++r)
            for (StepArgs A : args) {
                if (kinds[k] == kDown) A.out = g.work.out;  // leave x untouched
                rc = launch_step(A, g.stream, kinds[k]);
                if (rc) break;
            }
        const hipError_t ec = hipStreamEndCapture(g.stream, &graph);
        if (rc == 0 && ec != hipSuccess) rc = -4;
        if (rc == 0 && hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0) != hipSuccess) rc = -4;
        if (rc == 0 && hipGraphLaunch(exec, g.stream) != hipSuccess) rc = -4;  // warm
        if (rc == 0 && (hipEventRecord(e0, g.stream) != hipSuccess || hipGraphLaunch(exec, g.stream) != hipSuccess ||
                        hipEventRecord(e1, g.stream) != hipSuccess || hipEventSynchronize(e1) != hipSuccess))
            rc = -5;
        float ms = 0.0f;
        if (rc == 0 && hipEventElapsedTime(&ms, e0, e1) != hipSuccess) rc = -5;
        if (rc == 0) us_out[k] = (float)(1000.0 * ms / ((double)reps * nlayers));
        if (exec) (void)hipGraphExecDestroy(exec);
        if (graph) (void)hipGraphDestroy(graph);
    }
    (void)hipEventDestroy(e0);
    (void)hipEventDestroy(e1);
    if (rc && !g_err[0]) snprintf(g_err, sizeof g_err, "kernel timing pass failed (%d)", rc);
    return rc;
}

// One-launch decode timing: a HIP graph of `reps` chain steps (n layer
// launches + the final residual add each) and one of `reps` final kernels
// alone, each replayed between two events on the library stream; us_out[0] =
// mean time per layer launch ((chains - finals) / (reps * n)), us_out[1] =
// mean time of the final kernel.  x_dev advances reps + 1 steps.
extern "C" int colizig_hip_chain_fused_times(uint32_t layer0, uint32_t nlayers, float *x_dev, float eps, int reps,
                                             float *us_out) {
    CsrGuard csr;
    std::lock_guard<std::recursive_mutex> lk(g_mu);
    if (!g.inited || !x_dev || nlayers == 0 || reps < 1 || !us_out || !dev_aligned(x_dev)) return -1;
    for (uint32_t l = 0; l < nlayers; ++l) {
        LayerHost *L = find_layer(layer0 + l);
        int rc = check_layer_ready(L, layer0 + l);
        if (rc) return rc;
        if ((rc = ensure_work(L->d, 1))) return rc;
    }
    const int fz = chain_fused_prepare(layer0, nlayers, 1);
    if (fz <= 0) {
        if (fz == 0) snprintf(g_err, sizeof g_err, "chain is not served by the one-launch decode");
        return fz < 0 ? fz : -1;
    }
    int rc = chain_enqueue_fused(layer0, nlayers, x_dev, eps, nullptr, nullptr, nullptr, g.stream);
    if (rc) return rc;
    CZ_CHECK(hipStreamSynchronize(g.stream), -5);
    const uint32_t H = find_layer(layer0)->d.hidden;
    const FusedState &F = g.fused;
    hipEvent_t e0 = nullptr, e1 = nullptr;
    CZ_CHECK(hipEventCreate(&e0), -2);
    CZ_CHECK(hipEventCreate(&e1), -2);
    float ms[2] = {0.0f, 0.0f};
    for (int k = 0; k < 2 && rc == 0; ++k) {
        hipGraph_t graph = nullptr;
        hipGraphExec_t exec = nullptr;
        if (hipStreamBeginCapture(g.stream, hipStreamCaptureModeThreadLocal) != hipSuccess) { rc = -4; break; }
        for (int r = 0; r < reps && rc == 0; ++r) {
            if (k == 0) {
                rc = chain_enqueue_fused(layer0, nlayers, x_dev, eps, nullptr, nullptr, nullptr, g.stream);
            } else {
                k_chain_final<<<(H + 255) / 256, 256, 0, g.stream>>>(x_dev, F.r, F.p, H, F.run);
                if (hipGetLastError() != hipSuccess) rc = -4;
            }
        }
        const hipError_t ec = hipStreamEndCapture(g.stream, &graph);
        if (rc == 0 && ec != hipSuccess) rc = -4;
        if (rc == 0 && hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0) != hipSuccess) rc = -4;
        if (rc == 0 && hipGraphLaunch(exec, g.stream) != hipSuccess) rc = -4;  // warm
        if (rc == 0 && (hipEventRecord(e0, g.stream) != hipSuccess || hipGraphLaunch(exec, g.stream) != hipSuccess ||
                        hipEventRecord(e1, g.stream) != hipSuccess || hipEventSynchronize(e1) != hipSuccess))
            rc = -5;
        if (rc == 0 && hipEventElapsedTime(&ms[k], e0, e1) != hipSuccess) rc = -5;
        if (exec) (void)hipGraphExecDestroy(exec);
        if (graph) (void)hipGraphDestroy(graph);
    }
    (void)hipEventDestroy(e0);
    (void)hipEventDestroy(e1);
    if (rc == 0) {
        us_out[0] = (float)(1000.0 * (ms[0] - ms[1]) / ((double)reps * nlayers));
        us_out[1] = (float)(1000.0 * ms[1] / reps);
        rc = fused_check_error();
    }
    return rc;
}

extern "C" int colizig_hip_expert_slab_read(uint32_t layer, unsigned char *ew, float *es) {
    CsrGuard csr;
    std::lock_guard<std::recursive_mutex> lk(g_mu);
    LayerHost *L = find_layer(layer);
    if (!g.inited || !L || !ew || !es) return -1;
    if (L->streamed()) {
        snprintf(g_err, sizeof g_err, "layer %u streams from host memory", layer);
        return -1;
    }
    CZ_CHECK(hipStreamSynchronize(g.stream), -5);
    CZ_CHECK(hipMemcpy(ew, L->ew, L->ew_stride() * L->d.experts, hipMemcpyDeviceToHost), -5);
    CZ_CHECK(hipMemcpy(es, L->es, L->es_stride() * L->d.experts * sizeof(float), hipMemcpyDeviceToHost), -5);
    return 0;
}

// ---- streaming tier --------------------------------------------------------------
namespace {

uint64_t pool_key(uint32_t layer, uint32_t e) { return 1ull + (((uint64_t)layer << 32) | e); }

// Op log of the pool's policy decisions (4 words per op: op, layer, expert,
// result), replayed by the oracle's LRU restatement in the tests.
enum PoolOp : uint32_t { kOpEpoch = 0, kOpGet = 1, kOpPrefetch = 2, kOpWarm = 3, kOpClear = 4 };
constexpr uint32_t kLogHit = 0x80000000u;       // GET result: slot | kLogHit on a hit
constexpr uint32_t kLogResident = 0xfffffffeu;  // PREFETCH of a resident expert (no-op)
constexpr uint32_t kLogNoSlot = 0xffffffffu;    // PREFETCH with every slot pinned (dropped)

void pool_log(uint32_t op, uint32_t layer, uint32_t e, uint32_t result) {
    StreamPool &P = g.pool;
    if (!P.log_on) return;
    P.log.insert(P.log.end(), {op, layer, e, result});
}

uint8_t *slot_w(uint32_t i) { return g.pool.base + (uint64_t)i * g.pool.slot_bytes; }

// A slot for a new entry: the first free one, else the least recently used
// slot not pinned by the layer in flight (victimSlot, moe.zig:183-197, over
// one pool for every streamed layer), from the pool's use-ordered list
// (cz_lru.h) instead of a scan of every slot's clock (5.8 us per fill at
// 3,390 slots).  Returns nslots when every slot is pinned.
uint32_t pool_victim() {
    StreamPool &P = g.pool;
    return P.lru.victim([&](uint32_t i) { return P.epoch != 0 && P.pin_epoch[i] == P.epoch; });
}

// Forgets every pool entry of `layer` (re-registration).
void pool_drop_layer(uint32_t layer) {
    StreamPool &P = g.pool;
    for (uint32_t i = 0; i < P.nslots; ++i)
        if (P.key[i] && ((P.key[i] - 1) >> 32) == layer) {
            P.where.erase(P.key[i]);
            P.key[i] = 0;
            P.lru.release(i);
            P.prefetched[i] = 0;
        }
}

// Copies expert e of streamed layer L into slot i on the copy stream (fill,
// moe.zig:199-217): one copy from a packed host slab, else weights and
// scales separately.
int pool_fill(LayerHost &L, uint32_t layer, uint32_t e, uint32_t i, bool prefetch) {
    StreamPool &P = g.pool;
    if (P.key[i] != 0) {
        P.where.erase(P.key[i]);
        const uint64_t ok = P.key[i] - 1;  // the evicted (layer, expert): no slot any more
        if (LayerHost *Lo = find_layer((uint32_t)(ok >> 32)))
            if ((uint32_t)ok < Lo->slot_map.size() && Lo->slot_map[(uint32_t)ok] == (int32_t)i)
                Lo->slot_map[(uint32_t)ok] = -1;
        P.evictions++;
        if (P.prefetched[i] == P.stats_epoch + 1) P.prefetch_wasted++;  // issued in this stats window
    }
    uint8_t *dst = slot_w(i);
    const uint8_t sid = prefetch ? ((P.prefetch_rr++ & 1u) ? 2 : 0) : 1;
    hipStream_t cs = P.copy_stream(sid);
    // the slot's previous fill went through another copy stream: this one
    // waits for it, so two copies never overlap in one slot
    if (P.fill_seq[i] && P.fill_sid[i] != sid && P.fill_seq[i] > P.waited[P.fill_sid[i]])
        CZ_CHECK(hipStreamWaitEvent(cs, P.slot_ev[i], 0), -4);
    if (L.host_packed) {
        CZ_CHECK(hipMemcpyAsync(dst, L.host_packed + (uint64_t)e * P.slot_bytes, P.slot_bytes, hipMemcpyHostToDevice,
                                cs), -3);
    } else {
        CZ_CHECK(hipMemcpyAsync(dst, L.host_ew + (uint64_t)e * P.w_slot, P.w_slot, hipMemcpyHostToDevice, cs), -3);
        CZ_CHECK(hipMemcpyAsync(dst + P.w_slot, L.host_es + (uint64_t)e * P.s_slot, P.s_slot * sizeof(float),
                                hipMemcpyHostToDevice, cs), -3);
    }
    CZ_CHECK(hipEventRecord(P.slot_ev[i], cs), -4);
    P.fill_seq[i] = ++P.fill_counter;
    P.fill_sid[i] = sid;
    P.bytes_h2d += P.w_slot + P.s_slot * sizeof(float);
    P.loads++;
    P.key[i] = pool_key(layer, e);
    P.where[P.key[i]] = i;
    L.slot_map[e] = (int32_t)i;  // a layer's slot map holds every resident expert of it
    P.used[i] = ++P.clock;
    P.lru.touch(i);
    P.prefetched[i] = prefetch ? P.stats_epoch + 1 : 0;
    if (prefetch) P.prefetch_issued++;
    return 0;
}

// Makes the experts `sel` of streamed layer `layer` resident (get,
// moe.zig:221-240: hits touch the LRU, misses are filled on the copy stream)
// and pins them for the layer in flight.  With `Ld` (at most CZ_SEL_ARGS
// experts, slots and ids below 2^16) their slots go into Ld's argument table
// and the compute stream waits for the copy stream only if fills are in
// flight; otherwise the layer's slot map is uploaded on the copy stream and
// the compute stream waits for all of it.
// Stream st waits for the latest fill of each copy stream among `slots`.
int wait_fills(hipStream_t st, const uint32_t *slots, size_t n) {
    StreamPool &P = g.pool;
    uint64_t need[kCopyStreams] = {P.waited[0], P.waited[1], P.waited[2]};
    uint32_t at[kCopyStreams] = {0, 0, 0};
    for (size_t k = 0; k < n; ++k) {
        const uint32_t i = slots[k];
        const uint8_t s = P.fill_sid[i];
        if (P.fill_seq[i] > need[s]) {
            need[s] = P.fill_seq[i];
            at[s] = i;
        }
    }
    for (int s = 0; s < kCopyStreams; ++s)
        if (need[s] > P.waited[s]) {
            CZ_CHECK(hipStreamWaitEvent(st, P.slot_ev[at[s]], 0), -4);
            P.waited[s] = need[s];
        }
    return 0;
}

int stream_resident(LayerHost &L, uint32_t layer, const std::vector<uint32_t> &sel, hipStream_t st,
                    LayerDev *Ld = nullptr) {
    StreamPool &P = g.pool;
    P.epoch++;
    pool_log(kOpEpoch, layer, 0, 0);
    for (uint32_t e : sel) {
        P.sched.cancel(cz::ExpertKey{layer, e});  // demand-served (io.zig:127-137)
        auto it = P.where.find(pool_key(layer, e));
        if (it != P.where.end()) {
            const uint32_t i = it->second;
            P.hits++;
            if (P.prefetched[i]) {
                if (P.prefetched[i] == P.stats_epoch + 1) P.prefetch_hits++;  // issued in this stats window
                P.prefetched[i] = 0;
            }
            P.used[i] = ++P.clock;
            P.lru.touch(i);
            P.pin_epoch[i] = P.epoch;
            L.slot_map[e] = (int32_t)i;
            pool_log(kOpGet, layer, e, i | kLogHit);
            continue;
        }
        P.misses++;
        const uint32_t i = pool_victim();
        if (i == P.nslots) {
            snprintf(g_err, sizeof g_err, "expert pool of %u slots cannot hold one layer's selection", P.nslots);
            return -2;
        }
        int rc = pool_fill(L, layer, e, i, false);
        if (rc) return rc;
        P.pin_epoch[i] = P.epoch;
        L.slot_map[e] = (int32_t)i;
        pool_log(kOpGet, layer, e, i);
    }
    if (Ld && sel.size() <= CZ_SEL_ARGS && P.nslots <= 0x10000u && L.d.experts <= 0x10000u) {
        Ld->sel_n = (uint32_t)sel.size();
        for (size_t k = 0; k < sel.size(); ++k) Ld->sel[k] = sel[k] | ((uint32_t)L.slot_map[sel[k]] << 16);
        // the compute stream waits for the latest fill of these slots on
        // each copy stream only (each is in order: that covers the earlier
        // ones); later prefetches keep filling underneath
        std::vector<uint32_t> slots;
        for (uint32_t e : sel) slots.push_back((uint32_t)L.slot_map[e]);
        if (int rc = wait_fills(st, slots.data(), slots.size())) return rc;
    } else {
        // the slot map of this layer: only its selected entries matter (others
        // may be stale and are never read by this layer's kernels); uploaded
        // behind every fill so far, which the compute stream then waits for
        memcpy(L.slot_map_stage, L.slot_map.data(), L.slot_map.size() * sizeof(int32_t));
        CZ_CHECK(hipEventRecord(P.ev_copy_hi, P.copy_hi), -4);  // behind the demand fills too
        CZ_CHECK(hipStreamWaitEvent(P.copy, P.ev_copy_hi, 0), -4);
        CZ_CHECK(hipEventRecord(P.ev_copy2, P.copy2), -4);  // and the other prefetch stream's
        CZ_CHECK(hipStreamWaitEvent(P.copy, P.ev_copy2, 0), -4);
        CZ_CHECK(hipMemcpyAsync(L.slot_map_dev, L.slot_map_stage, L.slot_map.size() * sizeof(int32_t),
                                hipMemcpyHostToDevice, P.copy), -3);
        CZ_CHECK(hipEventRecord(P.ev_copy, P.copy), -4);
        CZ_CHECK(hipStreamWaitEvent(st, P.ev_copy, 0), -4);
        P.all_waited();
    }
    return 0;
}

// Services the scheduler's queue (prefetch, moe.zig:244-248): each key not
// yet resident is filled into a slot the layer in flight does not pin; a key
// of a layer that is not streamed is dropped; with every slot pinned the
// rest of the queue is dropped.
int pool_service() {
    StreamPool &P = g.pool;
    cz::ExpertKey k;
    while (P.sched.next(&k)) {
        LayerHost *L = find_layer(k.layer);
        if (!L || !L->streamed() || k.id >= L->d.experts) continue;
        if (P.where.count(pool_key(k.layer, k.id))) {
            pool_log(kOpPrefetch, k.layer, k.id, kLogResident);
            continue;
        }
        const uint32_t i = pool_victim();
        if (i == P.nslots) {
            pool_log(kOpPrefetch, k.layer, k.id, kLogNoSlot);
            P.sched.clear();
            return 0;
        }
        const int rc = pool_fill(*L, k.layer, k.id, i, true);
        if (rc) return rc;
        pool_log(kOpPrefetch, k.layer, k.id, i);
    }
    return 0;
}

int ensure_h_idx(int S) {
    StreamPool &P = g.pool;
    const size_t kmax = (size_t)S * CZ_MAX_K;
    if (!P.h_flag) {
        if (hipHostMalloc(&P.h_flag, 64, hipHostMallocCoherent) != hipSuccess ||
            hipHostMalloc(&P.h_pflag, 64, hipHostMallocCoherent) != hipSuccess ||
            hipHostMalloc(&P.h_pred, CZ_MAX_K * sizeof(uint32_t), hipHostMallocCoherent) != hipSuccess)
            return -2;
        __atomic_store_n(P.h_flag, 0u, __ATOMIC_RELEASE);
        __atomic_store_n(P.h_pflag, 0u, __ATOMIC_RELEASE);
        P.seq = P.pseq = 0;
    }
    if (P.h_idx_cap >= kmax) return 0;
    if (P.h_idx) (void)hipHostFree(P.h_idx);
    P.h_idx = nullptr;
    P.h_idx_cap = 0;
    if (hipHostMalloc(&P.h_idx, kmax * sizeof(uint32_t), hipHostMallocCoherent) != hipSuccess) return -2;
    P.h_idx_cap = kmax;
    return 0;
}

// Waits for a routing kernel's host-memory sequence number; now and then
// checks that the stream is still working (a failed kernel never sets it).
int wait_host_seq(const uint32_t *flag, uint32_t seq, hipStream_t st, const char *what) {
    for (uint32_t n = 1;; ++n) {
        if (__atomic_load_n(flag, __ATOMIC_ACQUIRE) == seq) return 0;
        if ((n & 4095u) == 0) {
            const hipError_t q = hipStreamQuery(st);
            if (q == hipSuccess && __atomic_load_n(flag, __ATOMIC_ACQUIRE) != seq) {
                snprintf(g_err, sizeof g_err, "%s: the routing kernel ended without its flag", what);
                return -5;
            }
            if (q != hipSuccess && q != hipErrorNotReady) {
                snprintf(g_err, sizeof g_err, "%s: %s", what, hipGetErrorString(q));
                return -5;
            }
        }
    }
}

// Scratch of the token-level prediction for n later layers of E experts.
int ensure_tok_pred(size_t n, uint32_t E) {
    StreamPool &P = g.pool;
    if (!P.h_tflag) {
        if (hipHostMalloc(&P.h_tflag, 64, hipHostMallocCoherent) != hipSuccess) return -2;
        __atomic_store_n(P.h_tflag, 0u, __ATOMIC_RELEASE);
        P.tseq = 0;
    }
    if (P.tok_cap >= n) return 0;
    for (void *p : {(void *)P.tok_logits, (void *)P.tok_gates, (void *)P.tok_idx, (void *)P.tok_tord,
                    (void *)P.tok_ptr_dev})
        if (p) (void)hipFree(p);
    for (void *p : {(void *)P.h_tok, (void *)P.tok_ptr_stage})
        if (p) (void)hipHostFree(p);
    P.tok_logits = P.tok_gates = nullptr;
    P.tok_idx = P.tok_tord = P.h_tok = nullptr;
    P.tok_ptr_dev = P.tok_ptr_stage = nullptr;
    P.tok_cap = 0;
    if (hipMalloc(&P.tok_logits, n * CZ_MAX_E * sizeof(float)) != hipSuccess ||
        hipMalloc(&P.tok_gates, n * CZ_MAX_K * sizeof(float)) != hipSuccess ||
        hipMalloc(&P.tok_idx, n * CZ_MAX_K * sizeof(uint32_t)) != hipSuccess ||
        hipMalloc(&P.tok_tord, n * CZ_MAX_K * sizeof(uint32_t)) != hipSuccess ||
        hipMalloc(&P.tok_ptr_dev, 2 * n * sizeof(float *)) != hipSuccess ||
        hipHostMalloc(&P.h_tok, n * CZ_MAX_K * sizeof(uint32_t), hipHostMallocCoherent) != hipSuccess ||
        hipHostMalloc(&P.tok_ptr_stage, 2 * n * sizeof(float *), hipHostMallocDefault) != hipSuccess)
        return -2;
    (void)E;
    P.tok_cap = n;
    return 0;
}

template <typename F>
void for_route_groups(uint32_t E, F &&f) {
    switch (cz_route_groups(E)) {
        case 1: f(std::integral_constant<int, 1>{}); break;
        case 2: f(std::integral_constant<int, 2>{}); break;
        case 4: f(std::integral_constant<int, 4>{}); break;
        case 8: f(std::integral_constant<int, 8>{}); break;
        default: f(std::integral_constant<int, 16>{}); break;
    }
}

// One streamed layer.  On the compute stream: router and routing, and at
// one token the next streamed layer's routing predicted from this layer's
// router input (that layer's router on this layer's rms(x): the residual
// stream changes little from one layer to the next).  Once this layer's
// picks are on the host (every earlier kernel has then finished): hits,
// demand fills of the misses (HIGH) and the layer's expert kernels, after
// its fills; then the next layer's predicted experts (MEDIUM) and the ones
// it routed for the previous token (LOW, LastTokenPredictor) go through the
// scheduler and fill on the copy stream while this layer's kernels run,
// sparing the slots they read.  Scratch (ensure_work + ensure_work_grouped)
// and the host read-back buffers must be in place.
int run_streamed_layer(LayerHost &L, uint32_t layer, const float *x, int S, float *out, int rms, float eps,
                       const float *xres, LayerHost *next, uint32_t next_layer, hipStream_t st,
                       const std::vector<uint32_t> *later) {
    StreamPool &P = g.pool;
    Work &w = g.work;
    const StepArgs A = step_args(L, x, S, out, rms, eps, xres, nullptr, nullptr, nullptr);
    // one token: the picks go into host memory, then a sequence number; the
    // host waits on that (no copy, no event).  The router kernel's last block
    // routes where the router is k_router_fast and E <= 128; otherwise a
    // routing launch follows the router.
    const bool direct = S == 1;
    const uint32_t hw = L.d.hidden % 32 ? 0u : L.d.hidden / 32;
    const bool route_in_router = direct && !L.router_bf16 && L.d.experts <= 128 &&
                                 (hw == 8 || hw == 16 || hw == 32 || hw == 64 || hw == 96 || hw == 128);
    void *h_idx_dev = nullptr, *h_flag_dev = nullptr;
    if (direct) {
        CZ_CHECK(hipHostGetDevicePointer(&h_idx_dev, P.h_idx, 0), -4);
        CZ_CHECK(hipHostGetDevicePointer(&h_flag_dev, P.h_flag, 0), -4);
    }
    if (route_in_router) {
        StepArgs Ar = A;
        Ar.route_count = P.route_count;
        Ar.host_idx = (uint32_t *)h_idx_dev;
        Ar.host_flag = (uint32_t *)h_flag_dev;
        Ar.host_seq = ++P.seq;
        launch_router(Ar, st);
    } else {
        launch_router(A, st);
    }
    GroupArgs G{};
    G.L = A.L;
    G.S = S;
    G.xn = rms ? w.xn : x;
    G.logits = w.logits;
    G.idx = w.idx;
    G.gates = w.gates;
    G.sgate = w.sgate;
    G.sgate_ready = rms_rows_write_sgate(A) ? 1u : 0u;
    G.tok_order = w.tok_order;
    G.usage = nullptr;  // the expert kernels below route again and count
    G.xh = nullptr;  // routing only: the grouped regime below splits x itself
    G.xl = nullptr;
    if (!route_in_router) {
        if (direct) {
            G.host_idx = (uint32_t *)h_idx_dev;
            G.host_flag = (uint32_t *)h_flag_dev;
            G.host_seq = ++P.seq;
        }
        for_route_groups(A.L.E, [&](auto m) { launch_route_tokens<decltype(m)::value>(G, st); });
    }
    const bool predict = direct && (P.predict_mode & 1) && next && next->streamed() && next->ready() &&
                         next->d.hidden == L.d.hidden && next->d.topk <= CZ_MAX_K;
    if (predict) {
        StepArgs Pn = step_args(*next, G.xn, 1, nullptr, 0, eps, nullptr, nullptr, nullptr, nullptr);
        Pn.logits = P.pred_logits;
        launch_router(Pn, st);
        GroupArgs G2{};
        G2.L = Pn.L;
        G2.S = 1;
        G2.xn = G.xn;
        G2.logits = P.pred_logits;
        G2.idx = P.pred_idx;
        G2.gates = P.pred_gates;
        G2.sgate = P.pred_sgate;
        G2.sgate_ready = 1;
        G2.tok_order = P.pred_tord;
        G2.usage = nullptr;
        void *di = nullptr, *df = nullptr;
        CZ_CHECK(hipHostGetDevicePointer(&di, P.h_pred, 0), -4);
        CZ_CHECK(hipHostGetDevicePointer(&df, P.h_pflag, 0), -4);
        G2.host_idx = (uint32_t *)di;
        G2.host_flag = (uint32_t *)df;
        G2.host_seq = ++P.pseq;
        for_route_groups(next->d.experts, [&](auto m) { launch_route_tokens<decltype(m)::value>(G2, st); });
    }
    // every later streamed layer's routing from this router input (the
    // chain's first): one router launch over the layers, one routing launch
    // with a row per layer, then the host flag
    const bool tok_predict = direct && (P.predict_mode & 2) && later && !later->empty() && L.d.hidden % 32 == 0;
    uint32_t tok_k = 0;
    if (tok_predict) {
        const size_t n = later->size();
        const LayerHost &F0 = *find_layer((*later)[0]);
        const uint32_t E2 = F0.d.experts;
        tok_k = F0.d.topk;
        if (int rc = ensure_tok_pred(n, E2)) return rc;
        for (size_t i = 0; i < n; ++i) {
            const LayerHost *Lj = find_layer((*later)[i]);
            P.tok_ptr_stage[i] = Lj->router;
            P.tok_ptr_stage[n + i] = Lj->rbias;
        }
        CZ_CHECK(hipMemcpyAsync(P.tok_ptr_dev, P.tok_ptr_stage, 2 * n * sizeof(float *), hipMemcpyHostToDevice, st),
                 -3);
        RouterLayersArgs R{};
        R.router = P.tok_ptr_dev;
        R.bias = P.tok_ptr_dev + n;
        R.x = G.xn;
        R.logits = P.tok_logits;
        R.E = E2;
        R.H = F0.d.hidden;
        k_router_layers<<<dim3((E2 + 1) / 2, (uint32_t)n), 64, 0, st>>>(R);
        GroupArgs G3{};
        G3.L = F0.dev();
        G3.S = (int)n;
        G3.xn = G.xn;
        G3.logits = P.tok_logits;
        G3.idx = P.tok_idx;
        G3.gates = P.tok_gates;
        G3.sgate = P.pred_sgate;
        G3.sgate_ready = 1;
        G3.tok_order = P.tok_tord;
        G3.usage = nullptr;
        void *di = nullptr, *df = nullptr;
        CZ_CHECK(hipHostGetDevicePointer(&di, P.h_tok, 0), -4);
        CZ_CHECK(hipHostGetDevicePointer(&df, P.h_tflag, 0), -4);
        G3.host_idx = (uint32_t *)di;
        G3.host_flag = nullptr;  // published below, once every row is written
        for_route_groups(E2, [&](auto m) { launch_route_tokens<decltype(m)::value>(G3, st); });
        k_host_signal<<<1, 64, 0, st>>>((uint32_t *)df, ++P.tseq);
    }
    const size_t nk = (size_t)S * L.d.topk;
    CZ_CHECK(hipGetLastError(), -4);
    if (direct) {
        if (int rc = wait_host_seq(P.h_flag, P.seq, st, "routing read-back")) return rc;
    } else {
        CZ_CHECK(hipMemcpyAsync(P.h_idx, w.idx, nk * sizeof(uint32_t), hipMemcpyDeviceToHost, st), -5);
        CZ_CHECK(hipEventRecord(P.ev_idx, st), -4);
        // the routing is on the critical path: poll for it rather than block
        for (;;) {
            const hipError_t q = hipEventQuery(P.ev_idx);
            if (q == hipSuccess) break;
            if (q != hipErrorNotReady) {
                snprintf(g_err, sizeof g_err, "routing read-back: %s", hipGetErrorString(q));
                return -5;
            }
        }
    }
    std::vector<uint32_t> sel;
    for (size_t k = 0; k < nk; ++k) {
        const uint32_t e = std::min(P.h_idx[k], L.d.experts - 1);
        if (std::find(sel.begin(), sel.end(), e) == sel.end()) sel.push_back(e);
    }
    if (direct) {  // score the predictions of this layer's routing (predict.zig:74-90)
        const auto it = P.pred_ids.find(layer);
        if (it != P.pred_ids.end()) {
            P.next_stats.score(it->second, P.h_idx, nk);
            P.pred_ids.erase(it);
        }
        const auto jt = P.tok_ids.find(layer);
        if (jt != P.tok_ids.end()) {
            P.tok_stats.score(jt->second, P.h_idx, nk);
            P.tok_ids.erase(jt);
        }
        P.last_pred.record(layer, P.h_idx, nk);
    }
    const bool grouped = grouped_ok(L.d, S);
    StepArgs A2 = A;  // the decode kernels can take the slots in their arguments
    int rc = stream_resident(L, layer, sel, st, grouped ? nullptr : &A2.L);
    if (rc) return rc;
    if (grouped) {
        rc = launch_grouped(L, x, S, out, rms, eps, xres, nullptr, nullptr, nullptr, st);
    } else {
        if (L.shn_dtype >= 0 && (rc = launch_shared_native_pre(L, G.xn, S, st))) return rc;
        rc = launch_step(A2, st, kUp | kDown);
        if (!rc && L.shn_dtype >= 0) rc = launch_shared_native_add(L, out, S, st);
    }
    if (rc) return rc;
    if (!next || !next->streamed()) return 0;
    if (predict) {
        if ((rc = wait_host_seq(P.h_pflag, P.pseq, st, "predicted routing read-back"))) return rc;
        std::vector<uint32_t> &pred = P.pred_ids[next_layer];
        pred.clear();
        for (uint32_t k = 0; k < next->d.topk; ++k) {
            const uint32_t e = std::min(P.h_pred[k], next->d.experts - 1);
            if (std::find(pred.begin(), pred.end(), e) == pred.end()) pred.push_back(e);
        }
        for (uint32_t e : pred) P.sched.submit(cz::ExpertKey{next_layer, e}, cz::kMedium);
    }
    for (uint32_t e : P.last_pred.predict(next_layer)) P.sched.submit(cz::ExpertKey{next_layer, e}, cz::kLow);
    if ((rc = pool_service())) return rc;
    if (tok_predict) {  // the later layers' predicted experts, layer by layer
        if ((rc = wait_host_seq(P.h_tflag, P.tseq, st, "token-level predicted routing read-back"))) return rc;
        for (size_t i = 0; i < later->size(); ++i) {
            const uint32_t lj = (*later)[i];
            const LayerHost *Lj = find_layer(lj);
            std::vector<uint32_t> &pred = P.tok_ids[lj];
            pred.clear();
            for (uint32_t k = 0; k < tok_k; ++k) {
                const uint32_t e = std::min(P.h_tok[i * tok_k + k], Lj->d.experts - 1);
                if (std::find(pred.begin(), pred.end(), e) == pred.end()) pred.push_back(e);
            }
            for (uint32_t e : pred) P.sched.submit(cz::ExpertKey{lj, e}, cz::kMedium);
            if ((rc = pool_service())) return rc;
        }
    }
    return 0;
}

// Buffers of a run of n later layers of E experts and K picks each.
int ensure_spec(size_t n, uint32_t E, uint32_t K) {
    StreamPool &P = g.pool;
    if (!P.stop_dev && hipMalloc(&P.stop_dev, sizeof(uint32_t)) != hipSuccess) return -2;
    if (P.spec_tab_cap < n * E) {
        if (P.spec_tab_dev) (void)hipFree(P.spec_tab_dev);
        if (P.h_spec_tab) (void)hipHostFree(P.h_spec_tab);
        P.spec_tab_dev = P.h_spec_tab = nullptr;
        P.spec_tab_cap = 0;
        if (hipMalloc(&P.spec_tab_dev, n * E * sizeof(int32_t)) != hipSuccess ||
            hipHostMalloc(&P.h_spec_tab, n * E * sizeof(int32_t), hipHostMallocDefault) != hipSuccess)
            return -2;
        P.spec_tab_cap = n * E;
    }
    const size_t need = n * K;
    if (P.spec_cap >= need) return 0;
    if (P.spec_idx_dev) (void)hipFree(P.spec_idx_dev);
    if (P.h_spec) (void)hipHostFree(P.h_spec);
    P.spec_idx_dev = P.h_spec = nullptr;
    P.spec_cap = 0;
    if (hipMalloc(&P.spec_idx_dev, need * sizeof(uint32_t)) != hipSuccess ||
        hipHostMalloc(&P.h_spec, (1 + need) * sizeof(uint32_t), hipHostMallocDefault) != hipSuccess)
        return -2;
    P.spec_cap = need;
    return 0;
}

// The host's side of a layer that ran in a speculative run, once its picks
// are back: the routing-prediction scores and the last-token record, as the
// per-layer path makes them, then the layer's gets in pick order (repeats
// dropped).  Every pick had a slot (else the layer would have stopped the
// run) and no fill ran since the slot maps were taken, so each get is a hit:
// the LRU touch, the pin and the op log entry of a hit.
int spec_account(uint32_t layer, const uint32_t *picks, uint32_t K) {
    StreamPool &P = g.pool;
    LayerHost &L = *find_layer(layer);
    const auto it = P.tok_ids.find(layer);
    if (it != P.tok_ids.end()) {
        P.tok_stats.score(it->second, picks, K);
        P.tok_ids.erase(it);
    }
    P.pred_ids.erase(layer);
    P.last_pred.record(layer, picks, K);
    std::vector<uint32_t> sel;
    for (uint32_t k = 0; k < K; ++k) {
        const uint32_t e = std::min(picks[k], L.d.experts - 1);
        if (std::find(sel.begin(), sel.end(), e) == sel.end()) sel.push_back(e);
    }
    P.epoch++;
    pool_log(kOpEpoch, layer, 0, 0);
    for (uint32_t e : sel) {
        P.sched.cancel(cz::ExpertKey{layer, e});
        const auto w = P.where.find(pool_key(layer, e));
        if (w == P.where.end()) {
            snprintf(g_err, sizeof g_err, "layer %u ran on expert %u without a pool slot", layer, e);
            return -5;
        }
        const uint32_t i = w->second;
        P.hits++;
        if (P.prefetched[i]) {
            if (P.prefetched[i] == P.stats_epoch + 1) P.prefetch_hits++;
            P.prefetched[i] = 0;
        }
        P.used[i] = ++P.clock;
        P.lru.touch(i);
        P.pin_epoch[i] = P.epoch;
        pool_log(kOpGet, layer, e, i | kLogHit);
    }
    return 0;
}

// The later streamed layers of a one-token chain with the host off their
// path.  The prefetches queued so far are serviced first; then every
// layer's slot map (every resident expert of it: no fill runs until the run
// is over) goes to the device in one copy on the compute stream, and each
// layer's three kernels follow, after a wait for the latest fill of any slot
// in its map, all enqueued at once.  A layer whose routing picks an expert without a slot
// sets the stop word and every later kernel does nothing; x is then the
// output of the last layer that ran.  One read-back after the run; the
// layers that ran are accounted in order.  *done: how many layers ran.
int run_spec_layers(const std::vector<uint32_t> &layers, size_t j0, float *x, float eps, hipStream_t st,
                    size_t *done) {
    StreamPool &P = g.pool;
    const size_t n = layers.size() - j0;
    const uint32_t K = find_layer(layers[j0])->d.topk, E = find_layer(layers[j0])->d.experts;
    *done = 0;
    if (int rc = pool_service()) return rc;
    if (int rc = ensure_spec(n, E, K)) return rc;
    for (size_t j = 0; j < n; ++j)
        memcpy(P.h_spec_tab + j * E, find_layer(layers[j0 + j])->slot_map.data(), E * sizeof(int32_t));
    CZ_CHECK(hipMemcpyAsync(P.spec_tab_dev, P.h_spec_tab, n * E * sizeof(int32_t), hipMemcpyHostToDevice, st), -3);
    CZ_CHECK(hipMemsetAsync(P.stop_dev, 0, sizeof(uint32_t), st), -4);
    // the one-launch decode where every layer of the run has its shape: one
    // launch per layer, its predicted experts the token-level prediction
    // (k_layer_fused with slot maps and the stop word), then k_spec_final
    const LayerHost &F0 = *find_layer(layers[j0]);
    const uint32_t H = F0.d.hidden;
    bool fused = P.tok_idx != nullptr && P.tok_cap >= layers.size() && n < 1023;
    for (size_t j = 0; fused && j < n; ++j) {
        const LayerHost &L = *find_layer(layers[j0 + j]);
        fused = fused_shape_ok(L, 1) && L.d.hidden == H && L.d.experts == E && L.d.topk == K;
    }
    for (size_t j = 0; fused && j < n; ++j)
        if (int rc = ensure_fused(find_layer(layers[j0 + j])->d)) return rc;
    FusedState &F = g.fused;
    for (size_t j = 0; j < n; ++j) {
        LayerHost &L = *find_layer(layers[j0 + j]);
        std::vector<uint32_t> slots;
        for (uint32_t e = 0; e < E; ++e)
            if (L.slot_map[e] >= 0) slots.push_back((uint32_t)L.slot_map[e]);
        if (int rc = wait_fills(st, slots.data(), slots.size())) return rc;
        if (fused) {
            FusedArgs A{};
            A.L = L.dev();
            A.L.slot_map = P.spec_tab_dev + j * E;  // this run's map of the layer
            A.rin = j <= 1 ? x : F.r + (uint64_t)((j - 1) % 2) * H;
            A.pin = j == 0 ? F.zero : F.p + (uint64_t)((j - 1) % 2) * CZ_NXCD * H;
            A.has_pin = j == 0 ? 0u : 1u;
            A.rout = j == 0 ? nullptr : F.r + (uint64_t)(j % 2) * H;
            A.pout = F.p + (uint64_t)(j % 2) * CZ_NXCD * H;
            A.lgx = F.lgx;
            A.hx = F.hx;
            A.run = F.run;
            A.err = F.err_dev;
            A.idx_trace = P.spec_idx_dev + j * K;
            A.pos = (uint32_t)j;
            A.eps = eps;
            A.pred_in = P.tok_idx + (j0 + j) * K;  // the token-level prediction of this layer
            A.lgpx = F.lgpx;
            A.pstat = F.spec_pstat;
            A.poll_mask = ~0u;
            A.stop = P.stop_dev;
            A.stop_code = (uint32_t)j + 1;
            const uint32_t rw = (uint32_t)((uint64_t)K * L.d.inter / 1024);
            switch (H) {
                case 512: launch_fused_nb<8>(A, rw, st); break;
                case 1024: launch_fused_nb<16>(A, rw, st); break;
                default: launch_fused_nb<32>(A, rw, st); break;
            }
        } else {
            StepArgs A = step_args(L, x, 1, x, 1, eps, x, nullptr, P.spec_idx_dev + j * K, nullptr);
            A.L.slot_map = P.spec_tab_dev + j * E;  // this run's map of the layer
            A.stop = P.stop_dev;
            A.stop_code = (uint32_t)j + 1;
            if (int rc = launch_step(A, st)) return rc;
        }
    }
    if (fused) {
        k_spec_final<<<(H + 255) / 256, 256, 0, st>>>(x, F.r, F.p, H, (uint32_t)n, P.stop_dev, F.run);
        const hipError_t e = hipGetLastError();
        if (e != hipSuccess) {
            snprintf(g_err, sizeof g_err, "speculative run launch: %s", hipGetErrorString(e));
            return -4;
        }
    }
    CZ_CHECK(hipMemcpyAsync(P.h_spec, P.stop_dev, sizeof(uint32_t), hipMemcpyDeviceToHost, st), -5);
    CZ_CHECK(hipMemcpyAsync(P.h_spec + 1, P.spec_idx_dev, n * K * sizeof(uint32_t), hipMemcpyDeviceToHost, st), -5);
    CZ_CHECK(hipEventRecord(P.ev_idx, st), -4);
    for (;;) {
        const hipError_t q = hipEventQuery(P.ev_idx);
        if (q == hipSuccess) break;
        if (q != hipErrorNotReady) {
            snprintf(g_err, sizeof g_err, "speculative run read-back: %s", hipGetErrorString(q));
            return -5;
        }
    }
    const uint32_t stop = P.h_spec[0];
    const size_t ran = stop ? std::min((size_t)stop - 1, n) : n;
    for (size_t j = 0; j < ran; ++j)
        if (int rc = spec_account(layers[j0 + j], P.h_spec + 1 + j * K, K)) return rc;
    P.spec_layers += ran;
    if (stop) P.spec_stops++;
    *done = ran;
    return 0;
}

}  // namespace

// The pool's configured shape is fixed until colizig_hip_stream_pool_free.
extern "C" int colizig_hip_stream_pool_init(const colizig_dims *dims, uint64_t cap_bytes) {
    CsrGuard csr;
    std::lock_guard<std::recursive_mutex> lk(g_mu);
    if (!g.inited || !dims) return -1;
    StreamPool &P = g.pool;
    if (P.on) {
        snprintf(g_err, sizeof g_err, "expert pool already configured");
        return -1;
    }
    const colizig_dims d = *dims;
    if (d.hidden == 0 || d.inter == 0 || d.experts == 0 || d.experts > CZ_MAX_E || d.topk == 0 ||
        d.topk > CZ_MAX_K) {
        snprintf(g_err, sizeof g_err, "unsupported pool dims");
        return -1;
    }
    const uint64_t w_slot = 3ull * d.inter * d.hidden, s_slot = 3ull * nblk(d.inter) * nblk(d.hidden);
    const uint64_t slot_bytes = (w_slot + s_slot * sizeof(float) + 15) / 16 * 16;
    const uint32_t n = (uint32_t)std::min<uint64_t>(cap_bytes / slot_bytes, 1u << 24);
    if (n < d.topk) {
        snprintf(g_err, sizeof g_err, "pool of %llu bytes holds %u experts < top-k %u", (unsigned long long)cap_bytes,
                 n, d.topk);
        return -1;
    }
    if (hipMalloc(&P.base, slot_bytes * n) != hipSuccess) {
        P.base = nullptr;
        snprintf(g_err, sizeof g_err, "expert pool allocation of %u slots failed", n);
        return -2;
    }
    if (!P.pred_logits &&
        (hipMalloc(&P.pred_logits, CZ_MAX_E * sizeof(float)) != hipSuccess ||
         hipMalloc(&P.pred_idx, CZ_MAX_K * sizeof(uint32_t)) != hipSuccess ||
         hipMalloc(&P.pred_gates, CZ_MAX_K * sizeof(float)) != hipSuccess ||
         hipMalloc(&P.pred_sgate, 64) != hipSuccess ||
         hipMalloc(&P.pred_tord, CZ_MAX_K * sizeof(uint32_t)) != hipSuccess ||
         hipMalloc(&P.route_count, sizeof(uint32_t)) != hipSuccess || hipMemset(P.route_count, 0, 4) != hipSuccess))
        return -2;
    if (!P.copy) {
        CZ_CHECK(hipStreamCreateWithFlags(&P.copy, hipStreamNonBlocking), -4);
        CZ_CHECK(hipStreamCreateWithFlags(&P.copy_hi, hipStreamNonBlocking), -4);
        CZ_CHECK(hipStreamCreateWithFlags(&P.copy2, hipStreamNonBlocking), -4);
        CZ_CHECK(hipEventCreateWithFlags(&P.ev_idx, hipEventDisableTiming), -4);
        CZ_CHECK(hipEventCreateWithFlags(&P.ev_copy, hipEventDisableTiming), -4);
        CZ_CHECK(hipEventCreateWithFlags(&P.ev_copy_hi, hipEventDisableTiming), -4);
        CZ_CHECK(hipEventCreateWithFlags(&P.ev_copy2, hipEventDisableTiming), -4);
    }
    P.d = d;
    P.w_slot = w_slot;
    P.s_slot = s_slot;
    P.slot_bytes = slot_bytes;
    P.nslots = n;
    while (P.slot_ev.size() < n) {
        hipEvent_t e = nullptr;
        CZ_CHECK(hipEventCreateWithFlags(&e, hipEventDisableTiming), -4);
        P.slot_ev.push_back(e);
    }
    P.fill_seq.assign(n, 0);
    P.fill_sid.assign(n, 0);
    P.fill_counter = 0;
    P.all_waited();
    P.key.assign(n, 0);
    P.used.assign(n, 0);
    P.lru.reset(n);
    P.prefetched.assign(n, 0);
    P.pin_epoch.assign(n, 0);
    P.where.clear();
    P.clock = 0;
    P.epoch = 0;
    P.last_pred.set_topk(d.topk);
    P.on = true;
    return 0;
}

// Frees the pool: every streamed layer is unregistered first (its host slabs
// stay the caller's), the counters start again from zero.
extern "C" int colizig_hip_stream_pool_free(void) {
    CsrGuard csr;
    std::lock_guard<std::recursive_mutex> lk(g_mu);
    StreamPool &P = g.pool;
    if (!g.inited || !P.on) return -1;
    CZ_CHECK(hipStreamSynchronize(g.stream), -5);
    CZ_CHECK(hipStreamSynchronize(P.copy), -5);
    CZ_CHECK(hipStreamSynchronize(P.copy_hi), -5);
    CZ_CHECK(hipStreamSynchronize(P.copy2), -5);
    for (auto it = g.layers.begin(); it != g.layers.end();) {
        if (it->second.streamed()) {
            free_layer(it->second);
            it = g.layers.erase(it);
        } else {
            ++it;
        }
    }
    (void)hipFree(P.base);
    P.base = nullptr;
    P.on = false;
    P.nslots = 0;
    P.key.clear();
    P.used.clear();
    P.prefetched.clear();
    P.pin_epoch.clear();
    P.where.clear();
    P.sched = cz::Scheduler(kSchedCapacity);
    P.last_pred.reset();
    P.pred_ids.clear();
    P.next_stats = cz::PredStats{};
    P.tok_ids.clear();
    P.tok_stats = cz::PredStats{};
    P.fill_counter = 0;
    P.all_waited();
    P.hits = P.misses = P.loads = P.evictions = P.prefetch_issued = P.prefetch_hits = P.prefetch_wasted =
        P.bytes_h2d = P.spec_layers = P.spec_stops = 0;
    P.log.clear();
    return 0;
}

namespace {
// Points a registered layer at the pool (its experts now live in host memory).
int stream_layer_setup(LayerHost *L, uint32_t layer) {
    StreamPool &P = g.pool;
    const colizig_dims &d = L->d;
    if (d.hidden != P.d.hidden || d.inter != P.d.inter) {
        snprintf(g_err, sizeof g_err, "layer %u shape differs from the expert pool's", layer);
        return -1;
    }
    (void)hipStreamSynchronize(g.stream);
    (void)hipStreamSynchronize(P.copy);
    (void)hipStreamSynchronize(P.copy_hi);
    (void)hipStreamSynchronize(P.copy2);
    if (!L->streamed()) {
        if (L->ew) (void)hipFree(L->ew);
        if (L->es) (void)hipFree(L->es);
    }
    L->ew = P.base;
    L->es = reinterpret_cast<float *>(P.base + P.w_slot);
    L->pool_ew_stride = P.slot_bytes;
    L->pool_es_stride = P.slot_bytes / sizeof(float);
    L->gen = ++g.layer_gen;
    L->slot_map.assign(d.experts, -1);
    if (!L->slot_map_dev && hipMalloc(&L->slot_map_dev, d.experts * sizeof(int32_t)) != hipSuccess) return -2;
    CZ_CHECK(hipMemset(L->slot_map_dev, 0xff, d.experts * sizeof(int32_t)), -4);  // all -1
    if (!L->slot_map_stage && hipHostMalloc(&L->slot_map_stage, d.experts * sizeof(int32_t), hipHostMallocDefault) !=
                                  hipSuccess)
        return -2;
    pool_drop_layer(layer);
    return 0;
}
}  // namespace

extern "C" int colizig_hip_layer_stream_from_host(uint32_t layer, const unsigned char *host_ew,
                                                  const float *host_es) {
    CsrGuard csr;
    std::lock_guard<std::recursive_mutex> lk(g_mu);
    LayerHost *L = find_layer(layer);
    if (!g.inited || !L || !host_ew || !host_es || !g.pool.on) return -1;
    const int rc = stream_layer_setup(L, layer);
    if (rc) return rc;
    L->host_ew = host_ew;
    L->host_es = host_es;
    L->host_packed = nullptr;
    return 0;
}

extern "C" int colizig_hip_layer_stream_from_host_packed(uint32_t layer, const unsigned char *host_slab) {
    CsrGuard csr;
    std::lock_guard<std::recursive_mutex> lk(g_mu);
    LayerHost *L = find_layer(layer);
    StreamPool &P = g.pool;
    if (!g.inited || !L || !host_slab || !P.on) return -1;
    if (P.slot_bytes != P.w_slot + P.s_slot * sizeof(float)) {
        snprintf(g_err, sizeof g_err, "packed expert stride %llu is not a multiple of 16 bytes",
                 (unsigned long long)(P.w_slot + P.s_slot * sizeof(float)));
        return -1;
    }
    const int rc = stream_layer_setup(L, layer);
    if (rc) return rc;
    L->host_ew = nullptr;
    L->host_es = nullptr;
    L->host_packed = host_slab;
    return 0;
}

extern "C" int colizig_hip_stream_decode(uint32_t layer0, uint32_t nlayers, float *x_dev, int S, float eps) {
    CsrGuard csr;
    std::lock_guard<std::recursive_mutex> lk(g_mu);
    StreamPool &P = g.pool;
    if (!g.inited || !P.on || S < 1 || !x_dev || nlayers == 0 || !dev_aligned(x_dev)) return -1;
    for (uint32_t l = 0; l < nlayers; ++l) {
        LayerHost *L = find_layer(layer0 + l);
        int rc = check_layer_ready(L, layer0 + l);
        if (rc) return rc;
        if ((rc = ensure_work(L->d, S))) return rc;
        if ((rc = ensure_work_grouped(L->d, S))) return rc;
    }
    if (ensure_h_idx(S)) return -2;
    hipStream_t st = g.stream;
    // the streamed layers after the first one, whose routing the first one
    // predicts (one token; the same experts, top-k and hidden size)
    uint32_t first = nlayers;
    std::vector<uint32_t> later;
    for (uint32_t l = 0; l < nlayers; ++l) {
        const LayerHost &L = *find_layer(layer0 + l);
        if (!L.streamed()) continue;
        if (first == nlayers) {
            first = l;
            continue;
        }
        const LayerHost &F = *find_layer(layer0 + first);
        if (S == 1 && !L.router_bf16 && L.d.hidden == F.d.hidden && L.d.experts <= CZ_MAX_E &&
            L.d.topk <= CZ_MAX_K &&
            (later.empty() || (L.d.experts == find_layer(later[0])->d.experts &&
                               L.d.topk == find_layer(later[0])->d.topk &&
                               L.d.norm_topk == find_layer(later[0])->d.norm_topk)))
            later.push_back(layer0 + l);
    }
    // speculative runs (prediction bits 1 and 2): every layer after the
    // first is a predicted streamed one, with an f32 router and no NativeMatrix
    // shared expert
    bool spec = S == 1 && (P.predict_mode & 6) == 6 && first == 0 && later.size() + 1 == nlayers;
    for (size_t j = 0; spec && j < later.size(); ++j) {
        const LayerHost &Lj = *find_layer(later[j]);
        spec = later[j] == layer0 + 1 + j && Lj.shn_dtype < 0 && !Lj.router_bf16;
    }
    for (uint32_t l = 0; l < nlayers; ++l) {
        LayerHost &L = *find_layer(layer0 + l);
        LayerHost *next = l + 1 < nlayers ? find_layer(layer0 + l + 1) : nullptr;
        const int rc = L.streamed() ? run_streamed_layer(L, layer0 + l, x_dev, S, x_dev, 1, eps, x_dev, next,
                                                         layer0 + l + 1, st, l == first ? &later : nullptr)
                                    : launch_layer(L, x_dev, S, x_dev, 1, eps, x_dev, nullptr, nullptr, nullptr, st);
        if (rc) return rc;
        if (spec && l + 1 < nlayers) {
            // the layers from l + 1 in one run; the layer that stopped it goes
            // through the per-layer path, then the next run starts after it
            size_t ran = 0;
            if (int rc2 = run_spec_layers(later, l, x_dev, eps, st, &ran)) return rc2;
            l += (uint32_t)ran;
        }
    }
    return 0;
}
// Routed-selection counts of every registered layer (ExpertUsage.bump,
// expert_usage.zig:39-45, fed by bumpUsage, moe.zig:428-432): each routing
// kernel adds one per pick of each token; rows of unregistered layers, or
// of layers with another expert count, read as zeros.  Waits for the
// library stream.
extern "C" int colizig_hip_usage_read(uint32_t layer0, uint32_t nlayers, uint32_t experts, uint64_t *counts) {
    CsrGuard csr;
    std::lock_guard<std::recursive_mutex> lk(g_mu);
    if (!g.inited || !counts || experts == 0) return -1;
    CZ_CHECK(hipStreamSynchronize(g.stream), -5);
    for (uint32_t l = 0; l < nlayers; ++l) {
        uint64_t *row = counts + (uint64_t)l * experts;
        const LayerHost *L = find_layer(layer0 + l);
        if (!L || !L->usage || L->d.experts != experts) {
            memset(row, 0, experts * sizeof(uint64_t));
            continue;
        }
        CZ_CHECK(hipMemcpy(row, L->usage, experts * sizeof(uint64_t), hipMemcpyDeviceToHost), -5);
    }
    return 0;
}

// Zeroes every registered layer's routed-selection counters.
extern "C" int colizig_hip_usage_reset(void) {
    CsrGuard csr;
    std::lock_guard<std::recursive_mutex> lk(g_mu);
    if (!g.inited) return -1;
    CZ_CHECK(hipStreamSynchronize(g.stream), -5);
    for (auto &kv : g.layers)
        if (kv.second.usage)
            CZ_CHECK(hipMemset(kv.second.usage, 0, kv.second.d.experts * sizeof(unsigned long long)), -4);
    CZ_CHECK(hipDeviceSynchronize(), -5);
    return 0;
}

// The streamed layers' counts: the same counters (kept for callers of the
// streaming tier's priors).
extern "C" int colizig_hip_stream_usage(uint32_t layer0, uint32_t nlayers, uint32_t experts, uint64_t *counts) {
    return colizig_hip_usage_read(layer0, nlayers, experts, counts);
}

// Pre-warms the HBM pool from learned priors (warmCaches, expert_usage.zig:
// 137-160): the streamed (layer, expert) pairs with a non-zero count, hottest
// first (ties: lower layer, then lower expert), into the pool's free slots
// only, so a warmed expert never displaces a hotter one.  The pool is one
// budget across layers, where the reference warms one cache per layer with
// its top entries.  Fills run on the copy stream and are complete on return;
// they count as prefetches.  Returns the number of experts warmed.
extern "C" int colizig_hip_stream_warm(uint32_t layer0, uint32_t nlayers, uint32_t experts, const uint64_t *counts) {
    CsrGuard csr;
    std::lock_guard<std::recursive_mutex> lk(g_mu);
    StreamPool &P = g.pool;
    if (!g.inited || !P.on || !counts || experts == 0) return -1;
    struct Cand { uint64_t c; uint32_t l, e; };
    std::vector<Cand> cand;
    for (uint32_t l = 0; l < nlayers; ++l) {
        LayerHost *L = find_layer(layer0 + l);
        if (!L || !L->streamed() || L->d.experts != experts) continue;
        for (uint32_t e = 0; e < experts; ++e) {
            const uint64_t c = counts[(uint64_t)l * experts + e];
            if (c) cand.push_back({c, layer0 + l, e});
        }
    }
    std::stable_sort(cand.begin(), cand.end(), [](const Cand &a, const Cand &b) { return a.c > b.c; });
    uint32_t next_free = 0, warmed = 0;
    for (const Cand &k : cand) {
        if (P.where.count(pool_key(k.l, k.e))) continue;
        while (next_free < P.nslots && P.key[next_free] != 0) ++next_free;
        if (next_free == P.nslots) break;
        const int rc = pool_fill(*find_layer(k.l), k.l, k.e, next_free, true);
        if (rc) return rc;
        pool_log(kOpWarm, k.l, k.e, next_free);
        ++warmed;
    }
    CZ_CHECK(hipStreamSynchronize(P.copy), -3);
    CZ_CHECK(hipStreamSynchronize(P.copy_hi), -3);
    CZ_CHECK(hipStreamSynchronize(P.copy2), -3);
    P.all_waited();  // every fill is complete
    return (int)warmed;
}

// Empties the pool (every slot free; counters and usage kept): the state of a
// fresh run, for priors measured in the same process.
extern "C" int colizig_hip_stream_evict_all(void) {
    CsrGuard csr;
    std::lock_guard<std::recursive_mutex> lk(g_mu);
    StreamPool &P = g.pool;
    if (!g.inited || !P.on) return -1;
    CZ_CHECK(hipStreamSynchronize(P.copy), -3);
    CZ_CHECK(hipStreamSynchronize(P.copy_hi), -3);
    CZ_CHECK(hipStreamSynchronize(P.copy2), -3);
    CZ_CHECK(hipStreamSynchronize(g.stream), -3);
    for (uint32_t i = 0; i < P.nslots; ++i) {
        P.key[i] = 0;
        P.prefetched[i] = 0;
    }
    P.lru.reset(P.nslots);
    P.where.clear();
    P.all_waited();  // every fill is complete
    P.sched.clear();
    P.pred_ids.clear();
    P.tok_ids.clear();
    P.last_pred.reset();
    pool_log(kOpClear, 0, 0, 0);
    for (auto &kv : g.layers)
        if (kv.second.streamed()) std::fill(kv.second.slot_map.begin(), kv.second.slot_map.end(), -1);
    return 0;
}

// Opens a new statistics window: every counter of colizig_hip_stream_stats
// restarts at 0 (the scheduler's queue peak at the queue's current length),
// and a prefetch counts as a hit or as wasted only in the window that issued
// it.  The pool's contents, LRU order and predictions are kept.  0, or -1
// without a pool.
extern "C" int colizig_hip_stream_stats_reset(void) {
    CsrGuard csr;
    std::lock_guard<std::recursive_mutex> lk(g_mu);
    StreamPool &P = g.pool;
    if (!g.inited || !P.on) return -1;
    P.stats_epoch++;
    P.hits = P.misses = P.loads = P.evictions = P.prefetch_issued = P.prefetch_hits = P.prefetch_wasted =
        P.bytes_h2d = 0;
    P.next_stats = cz::PredStats{};
    P.tok_stats = cz::PredStats{};
    P.spec_layers = P.spec_stops = 0;
    P.last_pred.reset_stats();
    P.sched.reset_stats();
    return 0;
}

extern "C" int colizig_hip_stream_stats(uint64_t *out, int n) {
    CsrGuard csr;
    std::lock_guard<std::recursive_mutex> lk(g_mu);
    const StreamPool &P = g.pool;
    const cz::SchedStats &s = P.sched.stats();
    const cz::PredStats &lt = P.last_pred.stats();
    const uint64_t v[27] = {P.hits, P.misses, P.loads, P.evictions, P.prefetch_issued, P.prefetch_hits,
                            P.prefetch_wasted, P.bytes_h2d, P.nslots, (uint64_t)P.where.size(),
                            P.next_stats.predicted, P.next_stats.correct, lt.predicted, lt.correct,
                            s.submitted, s.deduped, s.upgraded, s.rejected_full, s.serviced[0], s.serviced[1],
                            s.serviced[2], s.cancelled, s.queue_peak, P.tok_stats.predicted, P.tok_stats.correct,
                            P.spec_layers, P.spec_stops};
    if (!out || n < 1) return -1;
    for (int i = 0; i < n && i < 27; ++i) out[i] = v[i];
    return 0;
}

// Routing prediction mode (bit 0 next layer, bit 1 every later layer from
// the chain's first router input); returns the previous mode.
extern "C" int colizig_hip_stream_set_predict(int mode) {
    CsrGuard csr;
    std::lock_guard<std::recursive_mutex> lk(g_mu);
    if (mode < 0 || mode > 7) return -1;
    const int prev = g.pool.predict_mode;
    g.pool.predict_mode = mode;
    return prev;
}

// The pool's op log: enable != 0 clears it and starts recording; 0 stops.
extern "C" int colizig_hip_stream_log(int enable) {
    CsrGuard csr;
    std::lock_guard<std::recursive_mutex> lk(g_mu);
    g.pool.log.clear();
    g.pool.log_on = enable != 0;
    return 0;
}

// Copies up to max_ops recorded ops (4 words each) and returns how many the
// log holds.
extern "C" int64_t colizig_hip_stream_log_read(uint32_t *out, uint64_t max_ops) {
    CsrGuard csr;
    std::lock_guard<std::recursive_mutex> lk(g_mu);
    const std::vector<uint32_t> &lg = g.pool.log;
    const uint64_t n = lg.size() / 4;
    if (out) memcpy(out, lg.data(), std::min<uint64_t>(n, max_ops) * 4 * sizeof(uint32_t));
    return (int64_t)n;
}

// ---- the scheduler and the last-token predictor on their own (host only;
// no device or init needed): the interfaces of io.zig and predict.zig.
namespace {
std::mutex g_obj_mu;
std::unordered_map<int64_t, cz::Scheduler> g_scheds;
std::unordered_map<int64_t, cz::LastTokenPredictor> g_preds;
int64_t g_next_obj = 1;
}  // namespace

extern "C" int64_t colizig_hip_sched_create(uint32_t capacity) {
    std::lock_guard<std::mutex> lk(g_obj_mu);
    const int64_t h = g_next_obj++;
    g_scheds.emplace(h, cz::Scheduler(capacity));
    return h;
}

extern "C" void colizig_hip_sched_destroy(int64_t h) {
    std::lock_guard<std::mutex> lk(g_obj_mu);
    g_scheds.erase(h);
}

extern "C" int colizig_hip_sched_submit(int64_t h, uint32_t layer, uint32_t id, int prio) {
    std::lock_guard<std::mutex> lk(g_obj_mu);
    const auto it = g_scheds.find(h);
    if (it == g_scheds.end() || prio < 0 || prio > 2) return -1;
    return it->second.submit(cz::ExpertKey{layer, id}, (cz::Prio)prio) ? 1 : 0;
}

extern "C" int colizig_hip_sched_next(int64_t h, uint32_t *layer, uint32_t *id) {
    std::lock_guard<std::mutex> lk(g_obj_mu);
    const auto it = g_scheds.find(h);
    if (it == g_scheds.end() || !layer || !id) return -1;
    cz::ExpertKey k;
    if (!it->second.next(&k)) return 0;
    *layer = k.layer;
    *id = k.id;
    return 1;
}

extern "C" int colizig_hip_sched_cancel(int64_t h, uint32_t layer, uint32_t id) {
    std::lock_guard<std::mutex> lk(g_obj_mu);
    const auto it = g_scheds.find(h);
    if (it == g_scheds.end()) return -1;
    return it->second.cancel(cz::ExpertKey{layer, id}) ? 1 : 0;
}

extern "C" int colizig_hip_sched_has(int64_t h, uint32_t layer, uint32_t id) {
    std::lock_guard<std::mutex> lk(g_obj_mu);
    const auto it = g_scheds.find(h);
    if (it == g_scheds.end()) return -1;
    return it->second.has(cz::ExpertKey{layer, id}) ? 1 : 0;
}

extern "C" int colizig_hip_sched_stats(int64_t h, uint64_t *out, int n) {
    std::lock_guard<std::mutex> lk(g_obj_mu);
    const auto it = g_scheds.find(h);
    if (it == g_scheds.end() || !out) return -1;
    const cz::SchedStats &s = it->second.stats();
    const uint64_t v[10] = {s.submitted, s.deduped, s.upgraded, s.rejected_full, s.serviced[0], s.serviced[1],
                            s.serviced[2], s.cancelled, s.queue_peak, it->second.len()};
    for (int i = 0; i < n && i < 10; ++i) out[i] = v[i];
    return 0;
}

extern "C" int64_t colizig_hip_predictor_create(uint32_t topk) {
    std::lock_guard<std::mutex> lk(g_obj_mu);
    const int64_t h = g_next_obj++;
    g_preds.emplace(h, cz::LastTokenPredictor(topk));
    return h;
}

extern "C" void colizig_hip_predictor_destroy(int64_t h) {
    std::lock_guard<std::mutex> lk(g_obj_mu);
    g_preds.erase(h);
}

extern "C" int colizig_hip_predictor_record(int64_t h, uint32_t layer, const uint32_t *ids, uint32_t n) {
    std::lock_guard<std::mutex> lk(g_obj_mu);
    const auto it = g_preds.find(h);
    if (it == g_preds.end() || (n && !ids)) return -1;
    it->second.record(layer, ids, n);
    return 0;
}

extern "C" int colizig_hip_predictor_predict(int64_t h, uint32_t layer, uint32_t *out, uint32_t max) {
    std::lock_guard<std::mutex> lk(g_obj_mu);
    const auto it = g_preds.find(h);
    if (it == g_preds.end()) return -1;
    const std::vector<uint32_t> &p = it->second.predict(layer);
    const uint32_t n = (uint32_t)std::min<size_t>(p.size(), max);
    if (n && !out) return -1;
    std::copy(p.begin(), p.begin() + n, out);
    return (int)n;
}

extern "C" int colizig_hip_predictor_predict_scored(int64_t h, uint32_t layer, colizig_prefetch_prediction *out,
                                                    uint32_t max) {
    static_assert(sizeof(colizig_prefetch_prediction) == sizeof(cz::PrefetchPrediction), "row layout");
    std::lock_guard<std::mutex> lk(g_obj_mu);
    const auto it = g_preds.find(h);
    if (it == g_preds.end() || (max && !out)) return -1;
    cz::PrefetchPrediction rows[64];
    const size_t n = it->second.predict_scored(layer, rows, std::min<uint32_t>(max, 64));
    for (size_t i = 0; i < n; ++i)
        out[i] = colizig_prefetch_prediction{rows[i].layer, rows[i].expert, rows[i].confidence,
                                             rows[i].expected_use_distance};
    return (int)n;
}

extern "C" int colizig_hip_predictor_stats(int64_t h, uint64_t *predicted, uint64_t *correct) {
    std::lock_guard<std::mutex> lk(g_obj_mu);
    const auto it = g_preds.find(h);
    if (it == g_preds.end()) return -1;
    if (predicted) *predicted = it->second.stats().predicted;
    if (correct) *correct = it->second.stats().correct;
    return 0;
}

// ---- HBM plan (budget.plan, budget.zig:184-264, for one GPU's HBM): cz_plan.h
static_assert(cz::kPlanTileRows == CZ_GG_M && cz::kPlanGroupedMinTokens == (uint32_t)kGroupedMinTokens,
              "the plan's scratch count follows the forward's regimes");

extern "C" int colizig_hip_plan_hbm(const colizig_dims *dims, uint32_t layers, uint64_t hbm_budget,
                                    uint32_t max_tokens, colizig_hbm_plan *out) {
    CsrGuard csr;
    if (!dims || !out || layers == 0 || dims->experts == 0 || dims->topk == 0 || dims->hidden == 0 ||
        dims->inter == 0)
        return -1;
    if (hbm_budget == 0) {
        std::lock_guard<std::recursive_mutex> lk(g_mu);
        size_t freeb = 0, totalb = 0;
        if (!g.inited || hipMemGetInfo(&freeb, &totalb) != hipSuccess) return -1;
        hbm_budget = freeb - freeb / 8;
    }
    *out = cz::plan_hbm(*dims, layers, hbm_budget, max_tokens, g.prefill_fp8);
    return 0;
}

// Bytes the forward's scratch (Work) holds now: the capacities of its
// buffers (grow-only; buffers retired by a growth are not counted).
extern "C" int colizig_hip_work_bytes(uint64_t *out) {
    std::lock_guard<std::recursive_mutex> lk(g_mu);
    if (!g.inited || !out) return -1;
    const Work &w = g.work;
    *out = 4 * (w.cap_xin + w.cap_out + w.cap_xn + w.cap_logits + w.cap_idx + w.cap_gates + w.cap_sgate + w.cap_h +
                w.cap_hs + w.cap_ng + w.cap_nu + w.cap_no + w.cap_nsg + w.cap_counts + w.cap_offsets +
                w.cap_sorted + w.cap_slot_pos + w.cap_tok_order + w.cap_tiles + w.cap_tiles2 + w.cap_ntiles +
                w.cap_o + w.cap_os) +
           2 * (w.cap_xh + w.cap_xl + w.cap_hh + w.cap_hl + w.cap_hsh + w.cap_hsl) +
           (w.cap_xq + w.cap_xe + w.cap_hq + w.cap_he + w.cap_hsq + w.cap_hse);
    return 0;
}

extern "C" void *colizig_hip_host_alloc(uint64_t bytes) {
    CsrGuard csr;
    void *p = nullptr;
    if (!g.inited || bytes == 0 || hipHostMalloc(&p, bytes, hipHostMallocDefault) != hipSuccess) return nullptr;
    return p;
}

extern "C" void colizig_hip_host_free(void *p) {
    CsrGuard csr;
    if (g.inited && p) (void)hipHostFree(p);
}

// ---- exp test hooks -------------------------------------------------------------
__global__ void k_expf(const float *in, float *out, int n) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) out[i] = cz_expf(in[i]);
}

extern "C" int colizig_hip_expf_dev(const float *in, float *out, int n) {
    CsrGuard csr;
    std::lock_guard<std::recursive_mutex> lk(g_mu);
    if (!g.inited || n < 1 || !in || !out) return -1;
    float *di = nullptr, *dout = nullptr;
    int rc = 0;
    if (hipMalloc(&di, (size_t)n * 4) != hipSuccess || hipMalloc(&dout, (size_t)n * 4) != hipSuccess) {
        rc = -2;
    } else if (hipMemcpy(di, in, (size_t)n * 4, hipMemcpyHostToDevice) != hipSuccess) {
        rc = -3;
    } else {
        k_expf<<<(n + 255) / 256, 256, 0, g.stream>>>(di, dout, n);
        if (hipGetLastError() != hipSuccess) rc = -4;
        else if (hipStreamSynchronize(g.stream) != hipSuccess ||
                 hipMemcpy(out, dout, (size_t)n * 4, hipMemcpyDeviceToHost) != hipSuccess)
            rc = -5;
    }
    if (di) (void)hipFree(di);
    if (dout) (void)hipFree(dout);
    return rc;
}

extern "C" float colizig_hip_expf_host(float x) { return cz_expf(x); }

// ---- device memory / stream / event helpers -------------------------------------
extern "C" void *colizig_hip_malloc(uint64_t bytes) {
    CsrGuard csr;
    void *p = nullptr;
    if (!g.inited || bytes == 0 || hipMalloc(&p, bytes) != hipSuccess) return nullptr;
    return p;
}
extern "C" void colizig_hip_free(void *p) {
    CsrGuard csr;
    if (g.inited && p) (void)hipFree(p);
}
extern "C" int colizig_hip_memcpy_htod(void *dst, const void *src, uint64_t bytes) {
    CsrGuard csr;
    if (!g.inited) return -1;
    CZ_CHECK(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, g.stream), -3);
    CZ_CHECK(hipStreamSynchronize(g.stream), -3);
    return 0;
}
extern "C" int colizig_hip_memcpy_dtoh(void *dst, const void *src, uint64_t bytes) {
    CsrGuard csr;
    if (!g.inited) return -1;
    CZ_CHECK(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, g.stream), -5);
    CZ_CHECK(hipStreamSynchronize(g.stream), -5);
    return 0;
}
extern "C" int colizig_hip_memset(void *dst, int value, uint64_t bytes) {
    CsrGuard csr;
    if (!g.inited) return -1;
    CZ_CHECK(hipMemsetAsync(dst, value, bytes, g.stream), -4);
    CZ_CHECK(hipStreamSynchronize(g.stream), -4);
    return 0;
}
extern "C" void *colizig_hip_stream(void) { return g.inited ? (void *)g.stream : nullptr; }

// The prefill's grouped GEMMs on FP8 MFMA (1) or f16 MFMA (0); returns the
// previous setting.
extern "C" int colizig_hip_set_prefill_fp8(int enable) {
    CsrGuard csr;
    std::lock_guard<std::recursive_mutex> lk(g_mu);
    const int prev = g.prefill_fp8 ? 1 : 0;
    g.prefill_fp8 = enable != 0;
    return prev;
}

extern "C" int colizig_hip_set_fused_decode(int enable) {
    std::lock_guard<std::recursive_mutex> lk(g_mu);
    const int prev = g.fused.enabled ? 1 : 0;
    g.fused.enabled = enable != 0;
    return prev;
}

// Predicted experts in the one-launch decode: 0 off, 1 on, 2 and 3 on with
// the prediction spoiled on purpose (no slot keeps its prediction; slot 0
// does not) so that every slot, or one, loads after the routing.  Returns
// the previous setting, or -1 for another value.
extern "C" int colizig_hip_set_fused_predict(int mode) {
    std::lock_guard<std::recursive_mutex> lk(g_mu);
    if (mode < 0 || mode > 3) return -1;
    const int prev = g.fused.predict;
    g.fused.predict = mode;
    return prev;
}

// Counts of the predicted experts since the last call: out[0] slots that had
// a prediction, out[1] slots whose predicted expert was picked; then zeroes
// them.  0, or -1 before any one-launch decode.
extern "C" int colizig_hip_fused_predict_stats(uint64_t *out) {
    CsrGuard csr;
    std::lock_guard<std::recursive_mutex> lk(g_mu);
    if (!g.inited || !g.fused.pstat || !out) return -1;
    CZ_CHECK(hipStreamSynchronize(g.stream), -5);
    CZ_CHECK(hipMemcpy(out, g.fused.pstat, 2 * sizeof(uint64_t), hipMemcpyDeviceToHost), -5);
    CZ_CHECK(hipMemset(g.fused.pstat, 0, 2 * sizeof(uint64_t)), -5);
    return 0;
}

// Test hook: from the next chain on, the layer at chain position pos polls
// for a tag no layer writes, so its bounded waits give up after 20 ms, the
// kernel finishes with what it read and colizig_hip_sync reports -5 (-1:
// off).  Returns the previous position.
extern "C" int colizig_hip_set_fused_fault(int pos) {
    std::lock_guard<std::recursive_mutex> lk(g_mu);
    const int prev = g.fused.fault_pos;
    g.fused.fault_pos = pos < 0 ? -1 : pos;
    return prev;
}

// 1 when the init census found the workgroup placement the one-launch decode
// needs (8 XCDs, one workgroup of each rank per XCD), 0 otherwise, -1 before
// init.
extern "C" int colizig_hip_fused_placement(void) {
    std::lock_guard<std::recursive_mutex> lk(g_mu);
    if (!g.inited) return -1;
    return g.fused.placement_ok ? 1 : 0;
}

extern "C" int colizig_hip_fused_decode_active(uint32_t layer0, uint32_t nlayers, int S) {
    std::lock_guard<std::recursive_mutex> lk(g_mu);
    if (!g.inited || nlayers == 0 || nlayers >= 1023) return 0;
    const LayerHost *L0 = find_layer(layer0);
    if (!L0) return 0;
    for (uint32_t l = 0; l < nlayers; ++l) {
        const LayerHost *L = find_layer(layer0 + l);
        if (!L || !L->ready() || !fused_ok(*L, S) || L->d.hidden != L0->d.hidden) return 0;
    }
    return 1;
}
extern "C" int colizig_hip_sync(void) {
    CsrGuard csr;
    if (!g.inited) return -1;
    CZ_CHECK(hipStreamSynchronize(g.stream), -5);
    return fused_check_error();
}
extern "C" int64_t colizig_hip_event_create(void) {
    CsrGuard csr;
    std::lock_guard<std::recursive_mutex> lk(g_mu);
    if (!g.inited) return -1;
    hipEvent_t e;
    if (hipEventCreate(&e) != hipSuccess) return -2;
    const int64_t h = g.next_handle++;
    g.events[h] = e;
    return h;
}
extern "C" int colizig_hip_event_record(int64_t ev, void *stream) {
    CsrGuard csr;
    std::lock_guard<std::recursive_mutex> lk(g_mu);
    auto it = g.events.find(ev);
    if (!g.inited || it == g.events.end()) return -1;
    CZ_CHECK(hipEventRecord(it->second, pick_stream(stream)), -4);
    return 0;
}
extern "C" float colizig_hip_event_elapsed_ms(int64_t a, int64_t b) {
    CsrGuard csr;
    std::lock_guard<std::recursive_mutex> lk(g_mu);
    auto ia = g.events.find(a), ib = g.events.find(b);
    if (!g.inited || ia == g.events.end() || ib == g.events.end()) return -1.0f;
    if (hipEventSynchronize(ib->second) != hipSuccess) return -1.0f;
    float ms = -1.0f;
    if (hipEventElapsedTime(&ms, ia->second, ib->second) != hipSuccess) return -1.0f;
    return ms;
}
extern "C" void colizig_hip_event_destroy(int64_t ev) {
    std::lock_guard<std::recursive_mutex> lk(g_mu);
    auto it = g.events.find(ev);
    if (it == g.events.end()) return;
    (void)hipEventDestroy(it->second);
    g.events.erase(it);
}
extern "C" const char *colizig_hip_last_error(void) { return g_err; }
