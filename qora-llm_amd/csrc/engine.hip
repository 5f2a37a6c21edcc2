// C ABI of the MI355X decode path: context, weights, device-resident model,
// KV cache, captured decode step, and kernel-level entry points.
#include "../../include/qora_hip.h"
#include "launch.hpp"

#include <algorithm>
#include <atomic>
#include <chrono>
#include <mutex>
#include <cstdlib>
#include <cstring>
#include <cstdio>
#include <string>
#include <unordered_map>
#include <initializer_list>
#include <vector>

using namespace qora;

constexpr uint32_t kDefaultKvCapacity = 65536;   // kv_capacity 0 for a model without RoPE layers

// Scratch of the allocation-free GEMV entry (qora_hip_gemv_q4_noalloc): its
// fixed-point accumulator, one copy on every device the library runs on,
// held until the process ends. Host code never passes the array's name to
// a kernel or a copy: it uses the device address that hipGetSymbolAddress
// returns for the current device (noalloc_scratch below).
constexpr uint64_t kNoAllocMaxN = 65536;   // outputs; int64 words of the array (512 KiB)
static __device__ __align__(256) long long scratch[kNoAllocMaxN];

namespace {

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};
hipError_t g_scratch_err[kMaxDevices] = {};
bool g_scratch_done[kMaxDevices] = {};

// The device address of `scratch` on `device`, looked up once per device
// with that device current (the caller's set-up, qora_hip_create).
hipError_t noalloc_scratch_setup(int device) {
    if (device < 0 || device >= kMaxDevices) return hipErrorInvalidDevice;
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    if (!g_scratch_done[device]) {
        void* ptr = nullptr;
        const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
        g_scratch_err[device] = e;
        g_scratch_ptr[device] = e == hipSuccess ? ptr : nullptr;
        if (e != hipSuccess) (void)hipGetLastError();
        g_scratch_done[device] = true;
    }
    return g_scratch_err[device];
}

long long* noalloc_scratch(int device) {
    if (device < 0 || device >= kMaxDevices) return nullptr;
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    return static_cast<long long*>(g_scratch_ptr[device]);
}

}  // namespace

namespace {

struct DevWeight {
    int fmt = 0;            // FMT_Q4 / FMT_F16
    uint64_t k = 0, n = 0;
    void* w = nullptr;      // packed bytes or f16 words
    void* scales = nullptr; // Q4 only
    bool alive = false;
};

struct ModelState {
    bool ready = false;
    uint32_t L = 0, vocab = 0, hidden = 0, inter = 0, H = 0, KVH = 0, hd = 0, groups = 0, half = 0, fmt = 0;
    uint32_t cap = 0;
    int kv_f16 = 0;
    uint64_t rope_positions = 0;
    bool any_rope = false;
    std::vector<uint32_t> wids;
    uint32_t embed_wid = 0;
    std::vector<void*> allocs;           // every device allocation of the model
    uint16_t* d_norms = nullptr;         // [L][2][hidden]
    uint16_t* d_final = nullptr;
    float* d_cos = nullptr;
    float* d_sin = nullptr;
    void* d_k = nullptr;                 // [L][cap][kvd]
    void* d_v = nullptr;
    long long* d_xacc = nullptr;         // residual stream, fixed point [hidden]
    long long* d_qkv_acc = nullptr;      // q|k|v sums [qd + 2 kvd]
    long long* d_gu_acc = nullptr;       // gate|up sums [2 inter]
    float* d_attn_part = nullptr;        // attention split partials
    float* d_ss = nullptr;               // [L][2][64] sums of squares per K slice (RMSNorm)
    int* d_range = nullptr;              // set by the kernels when a fixed-point value leaves its range
    bool range_bad = false;              // a step reported it: refused until the cache is reset
    float* d_logits = nullptr;
    int32_t* d_token = nullptr;
    int32_t* d_pos = nullptr;
    int32_t* d_gen = nullptr;
    int32_t* d_prompt = nullptr;
    float* d_argv = nullptr;
    uint32_t* d_argi = nullptr;
    GemvPlan pl_qkv, pl_o, pl_gu, pl_down;
    uint32_t lm_blocks = 0;              // argmax partials of the lm_head launch
    bool lm_mfma = false;                // Q4 lm_head on the matrix cores (else the VALU row-dot)
    uint32_t attn_chunk = 0, attn_s_max = 0;
    std::vector<GemvParams> p_qkv, p_o, p_gu, p_down;
    std::vector<AttnParams> p_attn;
    // short contexts: attention inside the o GEMV (gemv_q4m_attn_kernel) for
    // steps that append a position below attn_o_max
    std::vector<AttnOParams> p_ao;
    uint32_t attn_o_max = 0;
    // steps that append a position in [attn_o_max, attn_ch_max) run the
    // chunked step (gemv_q4m_attn_kernel with CH); ch_np_max passes at most
    uint32_t attn_ch_max = 0, ch_np_max = 0;
    RowdotParams p_lm{};
    LmHeadParams p_lmq{};
    ArgmaxFinishParams p_fin{};
    EmbedParams p_emb_tok{}, p_emb_prompt{};
    hipGraphExec_t g_step = nullptr;
    hipGraphExec_t g_prefill = nullptr;
    // split steps that append a position below split_short_max run the
    // one-subgroup split attention (p_attn_ss) although the capacity's split
    // length would pick the long-context kernel (0: no separate variant)
    uint32_t split_short_max = 0;
    std::vector<AttnParams> p_attn_ss;
    hipGraphExec_t g_step_ss = nullptr;
    hipGraphExec_t g_prefill_ss = nullptr;
    // the same steps with the fused attention + o kernel, one per pass count
    // (index np - 1: contexts of 32 (np - 1) < L <= 32 np positions)
    hipGraphExec_t g_step_ao[kFusedMaxPasses] = {};
    hipGraphExec_t g_prefill_ao[kFusedMaxPasses] = {};
    hipGraphExec_t g_step_ch[kFusedMaxPasses] = {};
    hipGraphExec_t g_prefill_ch[kFusedMaxPasses] = {};
    uint64_t host_pos = 0;
    // token id that d_token holds once the queued work is done (-1: not known):
    // a decode call passing that id skips the upload
    int64_t dev_token = -1;
    // batched prefill (prefill.hpp), set up on first use
    bool pf_ready = false;
    uint32_t pf_tc = 0;                  // tokens per chunk
    float* d_pf_x = nullptr;             // residual rows [tc][hidden]
    float* d_pf_qkv = nullptr;           // q|k|v rows [tc][qd + 2 kvd]
    float* d_pf_q = nullptr;             // rotated q [tc][qd]
    float* d_pf_ao = nullptr;            // attention output [tc][qd]
    float* d_pf_gu = nullptr;            // gate|up rows [tc][2 inter]
    float* d_pf_xn = nullptr;            // final-normed last row [hidden]
    uint16_t* d_pf_xh = nullptr;         // split GEMM operand [tc][max k]
    uint16_t* d_pf_xl = nullptr;
    int32_t* d_pf_xe = nullptr;          // [tc]
    uint32_t* d_pf_ids = nullptr;        // [cap]
    float* d_pf_part = nullptr;          // split-K partials of the GEMMs
    uint64_t pf_part_bytes = 0;          // its size (the largest split set at set-up)
    float* d_pf_apart = nullptr;         // key-chunk partials of the prefill attention
    std::vector<int8_t*> pf_wf;          // [L][7] Q4 group exponents
    // Q4 weights packed for pf_gemm2_kernel ([L][7]), when every projection
    // has k % 32 == 0 and n % 128 == 0; else the prefill runs pf_gemm_kernel
    bool pf2 = false;
    std::vector<uint2*> pf_wq;
    std::vector<uint16_t*> pf_sc;
    LmHeadParams p_lmq_pf{};
    RowdotParams p_lm_pf{};
    ArgmaxFinishParams p_fin_pf{};
};

}  // namespace

// A kernel-level GEMV bound to uploaded weights in tile layout.
struct PreparedGemv {
    bool alive = false;
    int fmt = 0;
    bool paired = false;
    uint64_t k = 0, n = 0;
    GemvPlan plan;
    GemvParams p{};
    void* tw = nullptr;
    void* ts = nullptr;
    void* te = nullptr;
    // lm_head (qora_hip_lm_head_prepare): k = rows, n = cols
    bool lm_head = false;
    LmHeadParams lp{};
    uint32_t lm_blocks = 0;
    void* part_val = nullptr;
    void* part_idx = nullptr;
};

struct qora_hip_ctx {
    int device = 0;
    hipStream_t stream = nullptr;
    int cus = 0;
    std::string err;
    std::vector<DevWeight> weights;
    long long* ws_acc = nullptr;         // kernel-level fixed-point accumulator
    uint64_t ws_acc_n = 0;
    // on-device sampling scratch (grown to the largest vocab seen)
    float* smp_work = nullptr;
    unsigned long long* smp_cand = nullptr;
    unsigned long long* smp_rng = nullptr;
    int32_t* smp_tok = nullptr;
    SamplePenalty* smp_pen = nullptr;
    SamplePenalty* h_pen = nullptr;      // pinned staging of the penalty list
    uint64_t h_pen_n = 0;
    uint32_t smp_vocab = 0;
    void* smp_sort = nullptr;            // full-sort path: two key buffers and the probabilities
    uint64_t smp_sort_bytes = 0;
    uint64_t smp_pen_n = 0;
    void* ws_pf = nullptr;               // kernel-level GEMM: split operand and group exponents
    uint64_t ws_pf_bytes = 0;
    float* ws_attn_part = nullptr;
    uint64_t ws_attn_part_n = 0;
    int32_t* h_pin = nullptr;            // pinned staging: [0] token in, [1] token out, [2] pos
    // The step's argmax, stored by argmax_finish_kernel straight into mapped,
    // coherent pinned memory: reading it back takes the stream sync only, not
    // a copy (null if that allocation failed: then a copy is used).
    int32_t* h_tok = nullptr;
    int32_t* d_h_tok = nullptr;
    bool capturing = false;
    bool tok_armed = false;              // h_tok[0] set to kTokPending for the step in flight
    std::vector<PreparedGemv> gemvs;
    ModelState m;
};

namespace {

int fail(qora_hip_ctx* c, int code, const std::string& msg) {
    if (c) c->err = msg;
    return code;
}

bool force_fail(const char* what) {
    const char* v = std::getenv("QORA_HIP_FORCE_FAIL");
    return v && std::strcmp(v, what) == 0;
}

#define HIP_TRY(ctx, expr)                                                                      \
    do {                                                                                        \
        hipError_t e_ = (expr);                                                                 \
        if (e_ != hipSuccess)                                                                   \
            return fail((ctx), QORA_HIP_E_DEVICE, std::string(#expr) + ": " + hipGetErrorString(e_)); \
    } while (0)

int dalloc(qora_hip_ctx* c, size_t bytes, void** p) {
    *p = nullptr;
    if (force_fail("alloc")) return fail(c, QORA_HIP_E_NOMEM, "forced allocation failure (QORA_HIP_FORCE_FAIL=alloc)");
    if (bytes == 0) bytes = 16;
    const hipError_t e = hipMalloc(p, bytes);
    if (e != hipSuccess) {
        *p = nullptr;
        (void)hipGetLastError();
        return fail(c, QORA_HIP_E_NOMEM, "hipMalloc(" + std::to_string(bytes) + "): " + hipGetErrorString(e));
    }
    return QORA_HIP_OK;
}

hipStream_t pick_stream(qora_hip_ctx* c, void* s) { return s ? reinterpret_cast<hipStream_t>(s) : c->stream; }

// Grow the kernel-level scratch (fixed-point accumulator, attention partials).
int ensure_acc_ws(qora_hip_ctx* c, uint64_t n) {
    if (n <= c->ws_acc_n) return QORA_HIP_OK;
    if (c->capturing) return fail(c, QORA_HIP_E_STATE, "scratch must be sized by an eager call before capture");
    HIP_TRY(c, hipStreamSynchronize(c->stream));
    if (c->ws_acc) (void)hipFree(c->ws_acc);
    c->ws_acc = nullptr;
    c->ws_acc_n = 0;
    void* p;
    const uint64_t nn = n < 65536 ? 65536 : n;
    if (int rc = dalloc(c, nn * sizeof(long long), &p)) return rc;
    c->ws_acc = (long long*)p;
    c->ws_acc_n = nn;
    return QORA_HIP_OK;
}

int ensure_attn_ws(qora_hip_ctx* c, uint64_t part_floats) {
    if (part_floats <= c->ws_attn_part_n) return QORA_HIP_OK;
    if (c->capturing) return fail(c, QORA_HIP_E_STATE, "scratch must be sized by an eager call before capture");
    HIP_TRY(c, hipStreamSynchronize(c->stream));
    if (c->ws_attn_part) (void)hipFree(c->ws_attn_part);
    c->ws_attn_part = nullptr;
    c->ws_attn_part_n = 0;
    void* p;
    if (int rc = dalloc(c, part_floats * sizeof(float), &p)) return rc;
    c->ws_attn_part = (float*)p;
    c->ws_attn_part_n = part_floats;
    return QORA_HIP_OK;
}

int ensure_pf_ws(qora_hip_ctx* c, uint64_t bytes) {
    if (bytes <= c->ws_pf_bytes) return QORA_HIP_OK;
    if (c->capturing) return fail(c, QORA_HIP_E_STATE, "scratch must be sized by an eager call before capture");
    HIP_TRY(c, hipStreamSynchronize(c->stream));
    if (c->ws_pf) (void)hipFree(c->ws_pf);
    c->ws_pf = nullptr;
    c->ws_pf_bytes = 0;
    void* p;
    if (int rc = dalloc(c, bytes, &p)) return rc;
    c->ws_pf = p;
    c->ws_pf_bytes = bytes;
    return QORA_HIP_OK;
}

void free_model(qora_hip_ctx* c) {
    ModelState& m = c->m;
    // a greedy step without logits returns while its graph may still run
    (void)hipStreamSynchronize(c->stream);
    if (m.g_step) (void)hipGraphExecDestroy(m.g_step);
    if (m.g_prefill) (void)hipGraphExecDestroy(m.g_prefill);
    if (m.g_step_ss) (void)hipGraphExecDestroy(m.g_step_ss);
    if (m.g_prefill_ss) (void)hipGraphExecDestroy(m.g_prefill_ss);
    for (hipGraphExec_t g : m.g_step_ao)
        if (g) (void)hipGraphExecDestroy(g);
    for (hipGraphExec_t g : m.g_prefill_ao)
        if (g) (void)hipGraphExecDestroy(g);
    for (hipGraphExec_t g : m.g_step_ch)
        if (g) (void)hipGraphExecDestroy(g);
    for (hipGraphExec_t g : m.g_prefill_ch)
        if (g) (void)hipGraphExecDestroy(g);
    for (void* p : m.allocs) (void)hipFree(p);
    m = ModelState();
}

int model_alloc(qora_hip_ctx* c, size_t bytes, void** p) {
    if (int rc = dalloc(c, bytes, p)) return rc;
    c->m.allocs.push_back(*p);
    return QORA_HIP_OK;
}

const DevWeight* get_weight(qora_hip_ctx* c, uint32_t wid) {
    if (wid >= c->weights.size() || !c->weights[wid].alive) return nullptr;
    return &c->weights[wid];
}

// Launch plan of a decode-step GEMV: Q4 runs on the matrix cores
// (gemv_q4m_kernel), F16 on the VALU kernel.
bool plan_model_gemv(int fmt, uint32_t k, const uint32_t* seg_groups, int nseg, bool paired, int cus, GemvPlan* pl,
                     uint32_t row_align = 1) {
    return fmt == FMT_Q4 ? plan_gemv_q4m(k, seg_groups, nseg, paired, cus, pl, row_align)
                         : plan_gemv(fmt, k, seg_groups, nseg, paired, cus, pl, row_align);
}

// Allocates the tile layout of a planned GEMV (model-owned) and packs the
// reference-layout segments of *p into it.
int pack_model_gemv(qora_hip_ctx* c, int fmt, const GemvPlan& pl, GemvParams* p) {
    uint64_t wb = 0, sb = 0, eb = 0;
    gemv_tile_bytes(fmt, pl, &wb, &sb, &eb);
    void* tw = nullptr;
    void* ts = nullptr;
    void* te = nullptr;
    if (int rc = model_alloc(c, wb, &tw)) return rc;
    if (sb)
        if (int rc = model_alloc(c, sb, &ts)) return rc;
    if (eb)
        if (int rc = model_alloc(c, eb, &te)) return rc;
    HIP_TRY(c, launch_gemv_tile(fmt, pl, *p, (uint8_t*)tw, (uint16_t*)ts, (int8_t*)te, c->stream));
    p->tw = (const uint8_t*)tw;
    p->ts = (const uint16_t*)ts;
    p->tes = (const int8_t*)te;
    return QORA_HIP_OK;
}

// np > 0: attention inside the o GEMV for contexts of at most 32 np
// positions (short contexts, see attn_o_max), or with chunked, the chunked
// step whose column tiles take 32 np positions each; np = 0: split attention
int record_step(qora_hip_ctx* c, bool with_lm_head, uint32_t np, bool chunked = false, bool split_short = false) {
    ModelState& m = c->m;
    const hipStream_t s = c->stream;
    HIP_TRY(c, launch_embed(with_lm_head ? m.p_emb_tok : m.p_emb_prompt, s));
    for (uint32_t l = 0; l < m.L; ++l) {
        HIP_TRY(c, launch_gemv(m.fmt, m.pl_qkv, m.p_qkv[l], s));
        if (np) {
            HIP_TRY(c, launch_attn_o(m.pl_o, m.p_ao[l], np, chunked, s));
        } else {
            HIP_TRY(c, launch_attn(split_short ? m.p_attn_ss[l] : m.p_attn[l], s));
            HIP_TRY(c, launch_gemv(m.fmt, m.pl_o, m.p_o[l], s));
        }
        HIP_TRY(c, launch_gemv(m.fmt, m.pl_gu, m.p_gu[l], s));
        HIP_TRY(c, launch_gemv(m.fmt, m.pl_down, m.p_down[l], s));
    }
    if (with_lm_head) {
        if (m.lm_mfma) HIP_TRY(c, launch_lmhead(m.lm_blocks, m.p_lmq, s));
        else HIP_TRY(c, launch_rowdot(m.fmt, m.lm_blocks, m.p_lm, s));
        HIP_TRY(c, launch_argmax_finish(m.p_fin, s));
    } else {
        HIP_TRY(c, launch_advance_pos(m.d_pos, s));
    }
    return QORA_HIP_OK;
}

// QORA_HIP_EAGER=1 launches the decode step kernel by kernel instead of
// replaying the captured graph (for profilers that do not follow graphs).
// Attention subgroups per block (1 or 4): by default 4 when a split can hold
// more than one 32-position pass; QORA_HIP_ATTN_NSG overrides.
constexpr uint32_t kSplitShortMax = 4096;   // see split_short_max

uint32_t attn_nsg(uint32_t max_chunk) {
    const char* v = tuning_env("QORA_HIP_ATTN_NSG");
    if (v && *v) return std::atoi(v) > 1 ? 4u : 1u;
    return max_chunk > (uint32_t)kAttnSub ? 4u : 1u;
}

// Steps that append a position below this bound run attention inside the o
// GEMV (gemv_q4m_attn_kernel): every workgroup reads its head's whole
// context, so the fused step pays off only while the context is short; the
// kernel takes at most kFusedMaxPasses passes of 32 positions. QORA_HIP_ATTN_O
// lowers the bound (0: never fused).
constexpr uint32_t kAttnODefaultMax = kFusedPass * kFusedMaxPasses;

uint32_t attn_o_limit(const ModelState& m) {
    if (m.fmt != FMT_Q4 || !attn_o_supported(m.pl_o, m.hd, m.H, m.groups)) return 0;
    const char* v = std::getenv("QORA_HIP_ATTN_O");
    const long n = (v && *v) ? std::atol(v) : (long)kAttnODefaultMax;
    return n <= 0 ? 0u : (uint32_t)std::min<long>(std::min<long>(n, (long)kAttnODefaultMax), (long)m.cap);
}

// Steps that append a position in [attn_o_max, this bound) run the chunked
// step: the column tiles of a head each attend over a chunk of 32 np
// positions (tiles * 32 np >= the context) and exchange their states, so a
// layer's attention and o projection stay one launch without each workgroup
// reading the whole context. The exchange costs a few microseconds of
// device-coherent stores, polls and loads, and every query head re-reads its
// KV head's rows, so the step beats the split attention only while each
// column tile holds few positions: by default up to kChunkDefaultPerTile per
// tile (measured on SmolLM3-3B against the split attention: +2.2% at 280-340
// positions, even at 480-540, -2.1% at 680-740 and at 900-960).
// QORA_HIP_ATTN_CHUNK sets the bound (0: never chunked), up to
// kFusedMaxPasses passes a tile.
constexpr uint32_t kChunkDefaultPerTile = 32;

uint32_t attn_ch_limit(const ModelState& m, int cus) {
    if (m.fmt != FMT_Q4 || !attn_chunk_supported(m.pl_o, m.hd, m.H, m.groups, m.attn_s_max, cus)) return 0;
    const uint64_t top = std::min<uint64_t>((uint64_t)kFusedPass * kFusedMaxPasses * m.pl_o.tiles, m.cap);
    const char* v = std::getenv("QORA_HIP_ATTN_CHUNK");
    const long long n = (v && *v) ? std::atoll(v) : (long long)kChunkDefaultPerTile * m.pl_o.tiles;
    const uint64_t lim = n <= 0 ? 0u : std::min<uint64_t>((uint64_t)n, top);
    return lim > m.attn_o_max ? (uint32_t)lim : 0u;
}

// Attention of the step that appends `pos` (its context is pos + 1
// positions): the fused kernel's pass count, or the chunked step's passes per
// chunk (chunked), or np = 0 for the split attention.
struct StepAttn {
    uint32_t np;
    bool chunked;
    bool split_short;           // np = 0: the one-subgroup split attention (p_attn_ss)
};

StepAttn step_attn(const ModelState& m, uint64_t pos) {
    if (pos < (uint64_t)m.attn_o_max) return {(uint32_t)(pos / kFusedPass) + 1u, false, false};
    if (pos < (uint64_t)m.attn_ch_max) return {(uint32_t)(pos / ((uint64_t)kFusedPass * m.pl_o.tiles)) + 1u, true, false};
    return {0u, false, pos < (uint64_t)m.split_short_max};
}

bool eager_mode() {
    const char* v = std::getenv("QORA_HIP_EAGER");
    return v && *v && *v != '0';
}

// pos: the position the step appends (its context length is pos + 1).
int launch_step(qora_hip_ctx* c, bool with_lm_head, uint64_t pos) {
    ModelState& m = c->m;
    const StepAttn sa = step_attn(m, pos);
    if (eager_mode()) return record_step(c, with_lm_head, sa.np, sa.chunked, sa.split_short);
    hipGraphExec_t g = !sa.np ? (sa.split_short ? (with_lm_head ? m.g_step_ss : m.g_prefill_ss)
                                                : (with_lm_head ? m.g_step : m.g_prefill))
                       : sa.chunked ? (with_lm_head ? m.g_step_ch[sa.np - 1] : m.g_prefill_ch[sa.np - 1])
                                    : (with_lm_head ? m.g_step_ao[sa.np - 1] : m.g_prefill_ao[sa.np - 1]);
    HIP_TRY(c, hipGraphLaunch(g, c->stream));
    return QORA_HIP_OK;
}

int capture_step(qora_hip_ctx* c, bool with_lm_head, uint32_t np, hipGraphExec_t* out, bool chunked = false,
                 bool split_short = false) {
    HIP_TRY(c, hipStreamBeginCapture(c->stream, hipStreamCaptureModeThreadLocal));
    const int rc = record_step(c, with_lm_head, np, chunked, split_short);
    hipGraph_t g = nullptr;
    const hipError_t e = hipStreamEndCapture(c->stream, &g);
    if (rc) {
        if (g) (void)hipGraphDestroy(g);
        return rc;
    }
    if (e != hipSuccess) return fail(c, QORA_HIP_E_DEVICE, std::string("hipStreamEndCapture: ") + hipGetErrorString(e));
    const hipError_t e2 = hipGraphInstantiate(out, g, nullptr, nullptr, 0);
    (void)hipGraphDestroy(g);
    if (e2 != hipSuccess) return fail(c, QORA_HIP_E_DEVICE, std::string("hipGraphInstantiate: ") + hipGetErrorString(e2));
    return QORA_HIP_OK;
}

}  // namespace

// ===========================================================================
// context
// ===========================================================================

extern "C" int qora_hip_create(int device, qora_hip_ctx** out) {
    if (!out) return QORA_HIP_E_INVALID;
    *out = nullptr;
    if (force_fail("init")) return QORA_HIP_E_DEVICE;
    int count = 0;
    if (hipGetDeviceCount(&count) != hipSuccess || count <= 0) {
        (void)hipGetLastError();
        return QORA_HIP_E_DEVICE;
    }
    if (device < 0 || device >= count) return QORA_HIP_E_INVALID;
    qora_hip_ctx* c = new qora_hip_ctx();
    c->device = device;
    if (hipSetDevice(device) != hipSuccess || hipStreamCreateWithFlags(&c->stream, hipStreamNonBlocking) != hipSuccess) {
        delete c;
        return QORA_HIP_E_DEVICE;
    }
    int cus = 0;
    (void)hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, device);
    c->cus = cus > 0 ? cus : 256;
    // the allocation-free entry's scratch address on this device (an error
    // here only disables that entry, which then reports it)
    (void)noalloc_scratch_setup(device);
    if (hipHostMalloc((void**)&c->h_pin, 128, hipHostMallocDefault) != hipSuccess) {
        (void)hipStreamDestroy(c->stream);
        delete c;
        return QORA_HIP_E_DEVICE;
    }
    if (hipHostMalloc((void**)&c->h_tok, 64, hipHostMallocMapped | hipHostMallocCoherent) == hipSuccess) {
        std::memset(c->h_tok, 0, 64);   // [0] argmax token
        if (hipHostGetDevicePointer((void**)&c->d_h_tok, c->h_tok, 0) != hipSuccess) c->d_h_tok = nullptr;
    } else {
        c->h_tok = nullptr;
    }
    *out = c;
    return QORA_HIP_OK;
}

extern "C" int qora_hip_destroy(qora_hip_ctx* c) {
    if (!c) return QORA_HIP_E_INVALID;
    (void)hipSetDevice(c->device);
    (void)hipStreamSynchronize(c->stream);
    free_model(c);
    for (PreparedGemv& g : c->gemvs)
        for (void* q : {g.tw, g.ts, g.te, g.part_val, g.part_idx})
            if (q) (void)hipFree(q);
    for (DevWeight& w : c->weights) {
        if (w.w) (void)hipFree(w.w);
        if (w.scales) (void)hipFree(w.scales);
    }
    for (void* p : {(void*)c->ws_acc, (void*)c->ws_attn_part, c->ws_pf, (void*)c->smp_work, (void*)c->smp_cand,
                    (void*)c->smp_rng, (void*)c->smp_pen, c->smp_sort})
        if (p) (void)hipFree(p);
    if (c->h_pin) (void)hipHostFree(c->h_pin);
    if (c->h_pen) (void)hipHostFree(c->h_pen);
    if (c->h_tok) (void)hipHostFree(c->h_tok);
    (void)hipStreamDestroy(c->stream);
    delete c;
    return QORA_HIP_OK;
}

extern "C" const char* qora_hip_last_error(const qora_hip_ctx* c) {
    return c ? c->err.c_str() : "null context";
}

extern "C" int qora_hip_device_cus(const qora_hip_ctx* c) { return c ? c->cus : 0; }

// ===========================================================================
// weights
// ===========================================================================

extern "C" int qora_hip_upload_q4(qora_hip_ctx* c, const uint8_t* packed, size_t packed_len,
                                  const uint16_t* scales, size_t n_scales, uint64_t k, uint64_t n, uint32_t* wid) {
    if (!c || !packed || !scales || !wid) return fail(c, QORA_HIP_E_INVALID, "null argument");
    if (k == 0 || n == 0 || n % 32 != 0) return fail(c, QORA_HIP_E_INVALID, "Q4 weight needs k > 0 and n % 32 == 0");
    if (packed_len != k * n / 2 || n_scales != k * n / 32)
        return fail(c, QORA_HIP_E_INVALID, "Q4 buffer lengths do not match k*n/2 and k*n/32");
    DevWeight w;
    w.fmt = FMT_Q4;
    w.k = k;
    w.n = n;
    if (int rc = dalloc(c, packed_len, &w.w)) return rc;
    if (int rc = dalloc(c, n_scales * 2, &w.scales)) { (void)hipFree(w.w); return rc; }
    HIP_TRY(c, hipMemcpy(w.w, packed, packed_len, hipMemcpyHostToDevice));
    HIP_TRY(c, hipMemcpy(w.scales, scales, n_scales * 2, hipMemcpyHostToDevice));
    w.alive = true;
    *wid = (uint32_t)c->weights.size();
    c->weights.push_back(w);
    return QORA_HIP_OK;
}

extern "C" int qora_hip_upload_f16(qora_hip_ctx* c, const uint16_t* data, size_t len, uint64_t k, uint64_t n,
                                   uint32_t* wid) {
    if (!c || !data || !wid) return fail(c, QORA_HIP_E_INVALID, "null argument");
    if (k == 0 || n == 0 || n % 32 != 0) return fail(c, QORA_HIP_E_INVALID, "F16 weight needs k > 0 and n % 32 == 0");
    if (len != k * n) return fail(c, QORA_HIP_E_INVALID, "F16 buffer length does not match k*n");
    DevWeight w;
    w.fmt = FMT_F16;
    w.k = k;
    w.n = n;
    if (int rc = dalloc(c, len * 2, &w.w)) return rc;
    HIP_TRY(c, hipMemcpy(w.w, data, len * 2, hipMemcpyHostToDevice));
    w.alive = true;
    *wid = (uint32_t)c->weights.size();
    c->weights.push_back(w);
    return QORA_HIP_OK;
}

extern "C" int qora_hip_release_weight(qora_hip_ctx* c, uint32_t wid) {
    if (!c) return QORA_HIP_E_INVALID;
    if (!get_weight(c, wid)) return fail(c, QORA_HIP_E_INVALID, "unknown weight id");
    if (c->capturing) return fail(c, QORA_HIP_E_STATE, "release_weight frees: not allowed during capture");
    const ModelState& m = c->m;
    if (m.ready && (wid == m.embed_wid || std::find(m.wids.begin(), m.wids.end(), wid) != m.wids.end()))
        return fail(c, QORA_HIP_E_STATE, "weight is part of the initialised model");
    HIP_TRY(c, hipStreamSynchronize(c->stream));
    DevWeight& w = c->weights[wid];
    if (w.w) (void)hipFree(w.w);
    if (w.scales) (void)hipFree(w.scales);
    w = DevWeight();
    return QORA_HIP_OK;
}

extern "C" int qora_hip_weight_ptrs(qora_hip_ctx* c, uint32_t wid, void** data, void** scales) {
    if (!c) return QORA_HIP_E_INVALID;
    const DevWeight* w = get_weight(c, wid);
    if (!w) return fail(c, QORA_HIP_E_INVALID, "unknown weight id");
    if (data) *data = w->w;
    if (scales) *scales = w->scales;
    return QORA_HIP_OK;
}

// ===========================================================================
// model
// ===========================================================================

extern "C" int qora_hip_model_init(qora_hip_ctx* c, const qora_model_desc* d) {
    if (!c || !d) return fail(c, QORA_HIP_E_INVALID, "null argument");
    if (c->capturing) return fail(c, QORA_HIP_E_STATE, "model_init allocates: not allowed during capture");
    HIP_TRY(c, hipSetDevice(c->device));
    free_model(c);
    if (d->num_layers == 0 || d->vocab == 0 || d->hidden == 0 || d->intermediate == 0 || d->num_heads == 0 ||
        d->num_kv_heads == 0 || d->head_dim == 0)
        return fail(c, QORA_HIP_E_INVALID, "zero-sized model dimension");
    if (d->format > 1) return fail(c, QORA_HIP_E_INVALID, "format must be 0 (F16) or 1 (Q4)");
    if (d->num_heads % d->num_kv_heads != 0 || d->num_kv_groups != d->num_heads / d->num_kv_heads)
        return fail(c, QORA_HIP_E_INVALID, "num_kv_groups must equal num_heads / num_kv_heads");
    if (d->num_kv_groups > (uint32_t)kAttnMaxGroups || d->head_dim > (uint32_t)kAttnMaxHd)
        return fail(c, QORA_HIP_E_INVALID, "attention kernel supports head_dim <= 128 and <= 4 query heads per KV head");
    if (d->head_dim < 32 || d->head_dim % 8 != 0)
        return fail(c, QORA_HIP_E_INVALID, "head_dim must be a multiple of 8 and at least 32");
    if (2 * d->rope_half_dim > d->head_dim) return fail(c, QORA_HIP_E_INVALID, "rope_half_dim exceeds head_dim / 2");
    if (d->hidden % 32 != 0 || 64 % (d->hidden / 32) != 0 || d->intermediate % 32 != 0)
        return fail(c, QORA_HIP_E_INVALID, "hidden/32 must divide 64 and intermediate must be a multiple of 32");
    if (!d->layer_wids || !d->input_norm || !d->post_attn_norm || !d->final_norm || !d->use_rope)
        return fail(c, QORA_HIP_E_INVALID, "null model pointer");
    bool any_rope = false;
    for (uint32_t l = 0; l < d->num_layers; ++l) any_rope |= d->use_rope[l] != 0;
    // kv_capacity 0: as many positions as the model can place, i.e. the
    // RoPE table length (65536 for SmolLM3-3B), or kDefaultKvCapacity for a
    // model without RoPE layers, so a caller never runs out of cache where
    // the reference's growing RawKvCache would go on
    const uint64_t cap = d->kv_capacity ? d->kv_capacity
                                        : (any_rope ? std::min<uint64_t>(d->rope_positions, 0x7FFFFFFFull)
                                                    : (uint64_t)kDefaultKvCapacity);
    if (cap == 0) return fail(c, QORA_HIP_E_INVALID, "zero-sized KV cache (empty RoPE tables)");
    if (any_rope && (!d->rope_cos || !d->rope_sin || d->rope_half_dim == 0 || d->rope_positions < cap))
        return fail(c, QORA_HIP_E_INVALID, "RoPE tables must cover kv_capacity positions");

    ModelState& m = c->m;
    m.L = d->num_layers;
    m.vocab = d->vocab;
    m.hidden = d->hidden;
    m.inter = d->intermediate;
    m.H = d->num_heads;
    m.KVH = d->num_kv_heads;
    m.hd = d->head_dim;
    m.groups = d->num_kv_groups;
    m.half = d->rope_half_dim;
    m.fmt = d->format;
    m.cap = (uint32_t)cap;
    m.kv_f16 = d->kv_dtype == 1;
    m.rope_positions = d->rope_positions;
    m.any_rope = any_rope;
    const uint32_t qd = m.H * m.hd, kvd = m.KVH * m.hd;

    // shape and format checks of every weight (LayerWeights, gemv.rs:177-191)
    const uint64_t shapes[7][2] = {{m.hidden, qd}, {m.hidden, kvd}, {m.hidden, kvd}, {qd, m.hidden},
                                   {m.hidden, m.inter}, {m.hidden, m.inter}, {m.inter, m.hidden}};
    m.wids.assign(d->layer_wids, d->layer_wids + (size_t)m.L * 7);
    for (uint32_t l = 0; l < m.L; ++l)
        for (int j = 0; j < 7; ++j) {
            const DevWeight* w = get_weight(c, m.wids[l * 7 + j]);
            if (!w) { free_model(c); return fail(c, QORA_HIP_E_INVALID, "unknown weight id in layer_wids"); }
            if (w->fmt != (int)d->format || w->k != shapes[j][0] || w->n != shapes[j][1]) {
                free_model(c);
                return fail(c, QORA_HIP_E_INVALID, "layer " + std::to_string(l) + " weight " + std::to_string(j) +
                                                       " has the wrong format or shape");
            }
        }
    const DevWeight* emb = get_weight(c, d->embed_wid);
    if (!emb || emb->fmt != (int)d->format || emb->k != m.vocab || emb->n != m.hidden) {
        free_model(c);
        return fail(c, QORA_HIP_E_INVALID, "embedding weight has the wrong format or shape");
    }
    m.embed_wid = d->embed_wid;

    // launch plans
    const uint32_t gq = qd / 32, gkv = kvd / 32, gh = m.hidden / 32, gi = m.inter / 32;
    const uint32_t qkv_groups[3] = {gq, gkv, gkv};
    const uint32_t gu_groups[2] = {gi, gi};
    // Q4 o projection: K slices of exactly one head (64 or 128 rows), the
    // work items of the fused short-context step (gemv_q4m_attn_kernel)
    const bool o_by_head = m.fmt == FMT_Q4 && (m.hd == 64 || m.hd == 128);
    if (!plan_model_gemv(m.fmt, m.hidden, qkv_groups, 3, false, c->cus, &m.pl_qkv) ||
        !(o_by_head ? plan_gemv_q4m(qd, &gh, 1, false, c->cus, &m.pl_o, m.hd, m.hd)
                    : plan_model_gemv(m.fmt, qd, &gh, 1, false, c->cus, &m.pl_o, m.hd)) ||
        !plan_model_gemv(m.fmt, m.hidden, gu_groups, 2, true, c->cus, &m.pl_gu) ||
        !plan_model_gemv(m.fmt, m.inter, &gh, 1, false, c->cus, &m.pl_down)) {
        free_model(c);
        return fail(c, QORA_HIP_E_INVALID, "unsupported GEMV shape");
    }
    if (m.pl_qkv.splits > (uint32_t)kAttnMaxSplits || m.pl_gu.splits > (uint32_t)kAttnMaxSplits) {
        free_model(c);
        return fail(c, QORA_HIP_E_INVALID, "RMSNorm input split into more than 64 K slices");
    }
    // The fixed-point range guard (params.hpp) holds while an accumulator
    // takes at most kFixMaxTerms terms between two reads: the residual takes
    // the o or the down projection's split-K terms, the other accumulators
    // start from zero.
    for (const GemvPlan* pl : {&m.pl_qkv, &m.pl_o, &m.pl_gu, &m.pl_down})
        if (pl->splits > kFixMaxTerms) {
            free_model(c);
            return fail(c, QORA_HIP_E_INVALID, "a projection's contraction is split into more than " +
                                                   std::to_string(kFixMaxTerms) + " K slices");
        }
    m.lm_mfma = m.fmt == FMT_Q4 && lmhead_supported(m.hidden) && !tuning_env("QORA_HIP_LM_ROWDOT");
    m.lm_blocks = m.lm_mfma ? lmhead_blocks(m.vocab, c->cus) : rowdot_blocks(m.vocab, m.hidden, c->cus);
    attn_geometry(m.cap, &m.attn_chunk, &m.attn_s_max);
    // The step's split length follows the live context (attn_chunk_for(L):
    // 32 positions up to L = 2048), so a context shorter than the capacity
    // can need more splits than the capacity's own geometry has: launch
    // enough for every L <= cap (splits past L exit at once).
    m.attn_s_max = std::min<uint32_t>((uint32_t)kAttnMaxSplits, (m.cap + kAttnSub - 1) / kAttnSub);

    // device buffers
    void* p = nullptr;
    const size_t kvb = m.kv_f16 ? 2 : 4;
    const size_t qkv_n = (size_t)qd + 2 * kvd;
#define MALLOC(field, bytes)                                   \
    do {                                                       \
        if (int rc_ = model_alloc(c, (bytes), &p)) { free_model(c); return rc_; } \
        m.field = (decltype(m.field))p;                        \
    } while (0)
    MALLOC(d_norms, (size_t)m.L * 2 * m.hidden * 2);
    MALLOC(d_final, (size_t)m.hidden * 2);
    if (any_rope) {
        MALLOC(d_cos, (size_t)m.rope_positions * m.half * 4);
        MALLOC(d_sin, (size_t)m.rope_positions * m.half * 4);
    }
    MALLOC(d_k, (size_t)m.L * m.cap * kvd * kvb);
    MALLOC(d_v, (size_t)m.L * m.cap * kvd * kvb);
    MALLOC(d_xacc, (size_t)m.hidden * 8);
    // q|k|v sums, then the chunked step's per-head counters (cleared with them)
    MALLOC(d_qkv_acc, (qkv_n + kChunkCountWords) * 8);
    MALLOC(d_gu_acc, (size_t)2 * m.inter * 8);
    MALLOC(d_attn_part, (size_t)m.KVH * m.attn_s_max * m.groups * (m.hd + 2) * 4);
    MALLOC(d_ss, (size_t)m.L * 2 * kAttnMaxSplits * 4);
    MALLOC(d_range, 64);
    MALLOC(d_logits, (size_t)m.vocab * 4);
    MALLOC(d_token, 64);
    MALLOC(d_pos, 64);
    MALLOC(d_gen, (size_t)m.cap * 4 + 64);
    MALLOC(d_prompt, (size_t)m.cap * 4 + 64);
    MALLOC(d_argv, (size_t)m.lm_blocks * 4);
    MALLOC(d_argi, (size_t)m.lm_blocks * 4);
#undef MALLOC
    {
        // Cache slots past the current length are read (and skipped) by the
        // attention kernel; they start as zeros, or as NaN bit patterns with
        // QORA_HIP_KV_FILL=nan (a test of that skipping).
        const char* fill = tuning_env("QORA_HIP_KV_FILL");
        const int byte = (fill && std::strcmp(fill, "nan") == 0) ? 0xFF : 0;
        HIP_TRY(c, hipMemset(m.d_k, byte, (size_t)m.L * m.cap * kvd * kvb));
        HIP_TRY(c, hipMemset(m.d_v, byte, (size_t)m.L * m.cap * kvd * kvb));
    }
    HIP_TRY(c, hipMemset(m.d_xacc, 0, (size_t)m.hidden * 8));
    HIP_TRY(c, hipMemset(m.d_qkv_acc, 0, (qkv_n + kChunkCountWords) * 8));
    HIP_TRY(c, hipMemset(m.d_gu_acc, 0, (size_t)2 * m.inter * 8));
    HIP_TRY(c, hipMemset(m.d_pos, 0, 64));
    HIP_TRY(c, hipMemset(m.d_range, 0, 64));
    HIP_TRY(c, hipMemset(m.d_token, 0, 64));
    HIP_TRY(c, hipMemset(m.d_gen, 0, (size_t)m.cap * 4 + 64));
    HIP_TRY(c, hipMemset(m.d_prompt, 0, (size_t)m.cap * 4 + 64));
    for (uint32_t l = 0; l < m.L; ++l) {
        HIP_TRY(c, hipMemcpy(m.d_norms + ((size_t)l * 2 + 0) * m.hidden, d->input_norm[l], (size_t)m.hidden * 2,
                             hipMemcpyHostToDevice));
        HIP_TRY(c, hipMemcpy(m.d_norms + ((size_t)l * 2 + 1) * m.hidden, d->post_attn_norm[l], (size_t)m.hidden * 2,
                             hipMemcpyHostToDevice));
    }
    HIP_TRY(c, hipMemcpy(m.d_final, d->final_norm, (size_t)m.hidden * 2, hipMemcpyHostToDevice));
    if (any_rope) {
        HIP_TRY(c, hipMemcpy(m.d_cos, d->rope_cos, (size_t)m.rope_positions * m.half * 4, hipMemcpyHostToDevice));
        HIP_TRY(c, hipMemcpy(m.d_sin, d->rope_sin, (size_t)m.rope_positions * m.half * 4, hipMemcpyHostToDevice));
    }

    // Per-layer launch parameters. Data flow of one layer (each arrow is a
    // kernel boundary; accumulators are fixed point, see params.hpp):
    //   xacc --RMSNorm+q|k|v GEMV--> qkv_acc --attention(RoPE, K/V append)-->
    //   partials --merge+o GEMV--> xacc (+=) --RMSNorm+gate|up GEMV--> gu_acc
    //   --silu*up+down GEMV--> xacc (+=)
    // qkv_acc (with the chunked step's counters behind it) is cleared by the
    // gate|up kernel and gu_acc by the o kernel (the waves it has left over),
    // each after its last reader has finished and before its next writer
    // starts. Below attn_ch_max positions attention and the o GEMV run as one
    // kernel (gemv_q4m_attn_kernel) that reads qkv_acc itself: below
    // attn_o_max every workgroup over the whole context, above it each over
    // its chunk (the chunked step).
    m.p_qkv.resize(m.L);
    m.p_o.resize(m.L);
    m.p_gu.resize(m.L);
    m.p_down.resize(m.L);
    m.p_attn.resize(m.L);
    m.attn_o_max = attn_o_limit(m);
    m.attn_ch_max = attn_ch_limit(m, c->cus);
    m.ch_np_max = m.attn_ch_max ? (uint32_t)((m.attn_ch_max - 1u) / ((uint64_t)kFusedPass * m.pl_o.tiles)) + 1u : 0u;
    if (m.attn_o_max || m.attn_ch_max) m.p_ao.resize(m.L);
    for (uint32_t l = 0; l < m.L; ++l) {
        const DevWeight* W[7];
        for (int j = 0; j < 7; ++j) W[j] = get_weight(c, m.wids[l * 7 + j]);
        uint8_t* kl = (uint8_t*)m.d_k + (size_t)l * m.cap * kvd * kvb;
        uint8_t* vl = (uint8_t*)m.d_v + (size_t)l * m.cap * kvd * kvb;

        GemvParams& q = m.p_qkv[l];
        q = GemvParams{};
        for (int j = 0; j < 3; ++j)
            q.seg[j] = GemvSeg{(const uint8_t*)W[j]->w, (const uint16_t*)W[j]->scales, (uint32_t)(W[j]->n / 32), 0, 0, 0};
        q.nseg = 3;
        q.k = m.hidden;
        q.pro = PRO_GAMMA_FIXED;
        q.xacc = m.d_xacc;
        q.gamma = m.d_norms + ((size_t)l * 2 + 0) * m.hidden;
        q.ss_out = m.d_ss + ((size_t)l * 2 + 0) * kAttnMaxSplits;
        q.acc = m.d_qkv_acc;
        q.range_flag = m.d_range;
        apply_plan(m.pl_qkv, &q);
        if (int rc = pack_model_gemv(c, (int)m.fmt, m.pl_qkv, &q)) { free_model(c); return rc; }

        AttnParams& a = m.p_attn[l];
        a = AttnParams{};
        a.qkv_acc = m.d_qkv_acc;
        a.ss_in = m.d_ss + ((size_t)l * 2 + 0) * kAttnMaxSplits;
        a.ss_n = m.pl_qkv.splits;
        a.norm_n = m.hidden;
        a.rope_cos = m.d_cos;
        a.rope_sin = m.d_sin;
        a.use_rope = d->use_rope[l] ? 1 : 0;
        a.half = m.half;
        a.kc = kl;
        a.vc = vl;
        a.kv_f16 = m.kv_f16;
        a.pos = m.d_pos;
        a.H = m.H;
        a.KVH = m.KVH;
        a.hd = m.hd;
        a.groups = m.groups;
        a.scale = 1.0f / sqrtf((float)m.hd);
        a.chunk = 0;                       // split length follows the live context length
        a.part = m.d_attn_part;
        a.s_max = m.attn_s_max;
        a.nsg = attn_nsg(m.attn_chunk);
        a.kv_ps = m.hd;                  // head-major cache: [KVH][cap][hd] per layer
        a.kv_hs = (uint64_t)m.cap * m.hd;

        GemvParams& o = m.p_o[l];
        o = GemvParams{};
        o.seg[0] = GemvSeg{(const uint8_t*)W[3]->w, (const uint16_t*)W[3]->scales, gh, 0, 0, 0};
        o.nseg = 1;
        o.k = qd;
        o.pro = PRO_ATTN;
        o.attn_part = m.d_attn_part;
        o.attn_s_max = m.attn_s_max;
        o.attn_chunk = 0;
        o.head_dim = m.hd;
        o.groups = m.groups;
        o.pos = m.d_pos;
        o.acc = m.d_xacc;
        o.range_flag = m.d_range;
        o.zero_ptr = m.d_gu_acc;      // cleared by the attention + o launch's idle waves
        o.zero_n = 2 * m.inter;
        apply_plan(m.pl_o, &o);
        if (int rc = pack_model_gemv(c, (int)m.fmt, m.pl_o, &o)) { free_model(c); return rc; }
        if (m.attn_o_max || m.attn_ch_max) {
            // the chunked step's bounded wait; QORA_HIP_CHUNK_SPIN (a test
            // hook) shortens it, 0 forcing the timeout path
            const char* spin = tuning_env("QORA_HIP_CHUNK_SPIN");
            m.p_ao[l] = AttnOParams{o, a, reinterpret_cast<uint32_t*>(m.d_qkv_acc + qkv_n),
                                    spin ? (uint32_t)std::strtoul(spin, nullptr, 10) : kChunkSpin};
        }

        GemvParams& g = m.p_gu[l];
        g = GemvParams{};
        g.seg[0] = GemvSeg{(const uint8_t*)W[4]->w, (const uint16_t*)W[4]->scales, gi, 0, 0, 0};
        g.seg[1] = GemvSeg{(const uint8_t*)W[5]->w, (const uint16_t*)W[5]->scales, gi, 0, 0, 0};
        g.nseg = 2;
        g.paired = 1;
        g.k = m.hidden;
        g.pro = PRO_GAMMA_FIXED;
        g.xacc = m.d_xacc;
        g.gamma = m.d_norms + ((size_t)l * 2 + 1) * m.hidden;
        g.ss_out = m.d_ss + ((size_t)l * 2 + 1) * kAttnMaxSplits;
        g.acc = m.d_gu_acc;
        g.zero_ptr = m.d_qkv_acc;
        g.range_flag = m.d_range;
        g.zero_n = (uint32_t)(qkv_n + kChunkCountWords);   // with the chunked step's counters
        apply_plan(m.pl_gu, &g);
        if (int rc = pack_model_gemv(c, (int)m.fmt, m.pl_gu, &g)) { free_model(c); return rc; }

        GemvParams& dn = m.p_down[l];
        dn = GemvParams{};
        dn.seg[0] = GemvSeg{(const uint8_t*)W[6]->w, (const uint16_t*)W[6]->scales, gh, 0, 0, 0};
        dn.nseg = 1;
        dn.k = m.inter;
        dn.pro = PRO_SILU_FIXED;
        dn.xacc = m.d_gu_acc;
        dn.ss_in = m.d_ss + ((size_t)l * 2 + 1) * kAttnMaxSplits;
        dn.ss_n = m.pl_gu.splits;
        dn.norm_n = m.hidden;
        dn.acc = m.d_xacc;
        dn.range_flag = m.d_range;
        apply_plan(m.pl_down, &dn);
        if (int rc = pack_model_gemv(c, (int)m.fmt, m.pl_down, &dn)) { free_model(c); return rc; }
    }
    // A capacity whose split length exceeds one 32-position pass gives every
    // split step the long-context attention (four subgroups a split, or the
    // direct kernel for an f16 cache), built for splits of many passes. Below
    // kSplitShortMax positions (splits of at most two passes) the
    // one-subgroup split attention is faster (SmolLM3-3B, f16 cache of 32768
    // positions: 1106 against 984 tok/s at ~1000 positions, 972 against 963 at
    // ~4000; the long kernels win from ~8000 on): those steps take their own
    // graph.
    if (!m.p_attn.empty() && m.p_attn[0].nsg > 1 && !tuning_env("QORA_HIP_ATTN_NSG")) {
        m.split_short_max = std::min<uint32_t>(kSplitShortMax, m.cap);
        m.p_attn_ss = m.p_attn;
        for (AttnParams& a : m.p_attn_ss) a.nsg = 1;
    }
    m.p_lm = RowdotParams{};
    m.p_lm.w = (const uint8_t*)emb->w;
    m.p_lm.scales = (const uint16_t*)emb->scales;
    m.p_lm.rows = m.vocab;
    m.p_lm.cols = m.hidden;
    m.p_lm.xacc = m.d_xacc;
    m.p_lm.gamma = m.d_final;
    m.p_lm.y = m.d_logits;
    m.p_lm.do_argmax = 1;
    m.p_lm.part_val = m.d_argv;
    m.p_lm.part_idx = m.d_argi;
    m.p_lm.range_flag = m.d_range;
    if (m.lm_mfma) {
        uint64_t wb = 0, sb = 0;
        lmhead_tile_bytes(m.vocab, m.hidden, &wb, &sb);
        void* tw = nullptr;
        void* ts = nullptr;
        if (int rc = model_alloc(c, wb, &tw)) { free_model(c); return rc; }
        if (int rc = model_alloc(c, sb, &ts)) { free_model(c); return rc; }
        HIP_TRY(c, launch_lmhead_pack((const uint8_t*)emb->w, (const uint16_t*)emb->scales, m.vocab, m.hidden,
                                      (uint8_t*)tw, (uint32_t*)ts, c->stream));
        m.p_lmq = LmHeadParams{};
        m.p_lmq.tw = (const uint8_t*)tw;
        m.p_lmq.ts = (const uint32_t*)ts;
        m.p_lmq.rows = m.vocab;
        m.p_lmq.cols = m.hidden;
        m.p_lmq.tiles = lmhead_tiles(m.vocab);
        m.p_lmq.xacc = m.d_xacc;
        m.p_lmq.gamma = m.d_final;
        m.p_lmq.y = m.d_logits;
        m.p_lmq.do_argmax = 1;
        m.p_lmq.part_val = m.d_argv;
        m.p_lmq.part_idx = m.d_argi;
        m.p_lmq.range_flag = m.d_range;
    }
    m.p_fin = ArgmaxFinishParams{m.d_argv, m.d_argi, m.lm_blocks, m.d_token, m.d_pos, m.d_gen, c->d_h_tok, m.d_range};
    m.p_emb_tok = EmbedParams{(const uint8_t*)emb->w, (const uint16_t*)emb->scales, (int)m.fmt, m.hidden,
                              m.vocab, m.d_token, nullptr, m.d_xacc};
    m.p_emb_prompt = EmbedParams{(const uint8_t*)emb->w, (const uint16_t*)emb->scales, (int)m.fmt, m.hidden,
                                 m.vocab, m.d_prompt, m.d_pos, m.d_xacc};

    HIP_TRY(c, hipDeviceSynchronize());
    if (int rc = capture_step(c, true, 0, &m.g_step)) { free_model(c); return rc; }
    if (int rc = capture_step(c, false, 0, &m.g_prefill)) { free_model(c); return rc; }
    if (m.split_short_max) {
        if (int rc = capture_step(c, true, 0, &m.g_step_ss, false, true)) { free_model(c); return rc; }
        if (int rc = capture_step(c, false, 0, &m.g_prefill_ss, false, true)) { free_model(c); return rc; }
    }
    // one fused variant per pass count a step below attn_o_max can need
    for (uint32_t np = 1; m.attn_o_max && np <= (m.attn_o_max - 1) / kFusedPass + 1; ++np) {
        if (int rc = capture_step(c, true, np, &m.g_step_ao[np - 1])) { free_model(c); return rc; }
        if (int rc = capture_step(c, false, np, &m.g_prefill_ao[np - 1])) { free_model(c); return rc; }
    }
    // one chunked variant per passes-per-chunk count
    for (uint32_t np = 1; np <= m.ch_np_max; ++np) {
        if (int rc = capture_step(c, true, np, &m.g_step_ch[np - 1], true)) { free_model(c); return rc; }
        if (int rc = capture_step(c, false, np, &m.g_prefill_ch[np - 1], true)) { free_model(c); return rc; }
    }
    m.host_pos = 0;
    m.ready = true;
    return QORA_HIP_OK;
}

namespace {

// Sets the device position; a new cache state also clears the range flag.
int set_device_pos(qora_hip_ctx* c, uint64_t pos) {
    c->h_pin[2] = (int32_t)pos;
    HIP_TRY(c, hipMemcpyAsync(c->m.d_pos, &c->h_pin[2], 4, hipMemcpyHostToDevice, c->stream));
    HIP_TRY(c, hipMemsetAsync(c->m.d_range, 0, 4, c->stream));
    HIP_TRY(c, hipStreamSynchronize(c->stream));
    if (c->h_tok) reinterpret_cast<volatile int32_t*>(c->h_tok)[1] = 0;
    c->m.range_bad = false;
    return QORA_HIP_OK;
}

// The error of a step whose fixed-point values left their range (the flag
// reached the host with the token); later steps are refused until the cache
// is reset, re-filled by a prefill or uploaded.
int range_error(qora_hip_ctx* c) {
    c->m.range_bad = true;
    return fail(c, QORA_HIP_E_RANGE,
                "fixed-point range exceeded (a residual value of 2^25 or more, or a projection term of 2^20 or "
                "more): the step's results are not valid; reset the KV cache");
}

int check_step_room(qora_hip_ctx* c, uint64_t steps) {
    ModelState& m = c->m;
    if (!m.ready) return fail(c, QORA_HIP_E_STATE, "model not initialised");
    if (c->capturing) return fail(c, QORA_HIP_E_STATE, "decode and prefill steps are not allowed during capture");
    if (m.range_bad) return range_error(c);
    if (m.host_pos + steps > m.cap)
        return fail(c, QORA_HIP_E_STATE, "KV cache full (capacity " + std::to_string(m.cap) + ")");
    if (m.any_rope && m.host_pos + steps > m.rope_positions)
        return fail(c, QORA_HIP_E_STATE, "position beyond the RoPE tables");
    return QORA_HIP_OK;
}

// h_tok[0] while a step's token is outstanding (argmax_finish_kernel stores
// the token there, a vocabulary index, never this value)
constexpr int32_t kTokPending = INT32_MIN;

int finish_step(qora_hip_ctx* c, float* logits, uint32_t* argmax) {
    ModelState& m = c->m;
    const bool mapped = c->d_h_tok != nullptr;   // argmax_finish_kernel stored the token in h_tok
    if (mapped && c->tok_armed && !logits) {
        // Greedy step without logits: the token is read from the mapped word as
        // soon as the device has stored it, without waiting for the stream's
        // completion signal. Stream order keeps the next step's work behind
        // this one. After 200 ms without a token (a failed launch, a fault)
        // the stream is synchronised and its error reported.
        c->tok_armed = false;
        volatile int32_t* ht = c->h_tok;
        const auto t0 = std::chrono::steady_clock::now();
        for (uint32_t i = 1;; ++i) {
            const int32_t tok = ht[0];
            if (tok != kTokPending) {
                if (ht[1] != 0) return range_error(c);
                m.dev_token = tok;
                if (argmax) *argmax = (uint32_t)tok;
                return QORA_HIP_OK;
            }
            if ((i & 1023u) == 0 && std::chrono::steady_clock::now() - t0 > std::chrono::milliseconds(200)) break;
        }
    }
    c->tok_armed = false;
    if (!mapped) {
        HIP_TRY(c, hipMemcpyAsync(&c->h_pin[16], m.d_token, 4, hipMemcpyDeviceToHost, c->stream));
        HIP_TRY(c, hipMemcpyAsync(&c->h_pin[17], m.d_range, 4, hipMemcpyDeviceToHost, c->stream));
    }
    if (logits) HIP_TRY(c, hipMemcpyAsync(logits, m.d_logits, (size_t)m.vocab * 4, hipMemcpyDeviceToHost, c->stream));
    HIP_TRY(c, hipStreamSynchronize(c->stream));
    if ((mapped ? reinterpret_cast<volatile int32_t*>(c->h_tok)[1] : c->h_pin[17]) != 0) return range_error(c);
    const int32_t tok = mapped ? *reinterpret_cast<volatile int32_t*>(c->h_tok) : c->h_pin[16];
    m.dev_token = tok;
    if (argmax) *argmax = (uint32_t)tok;
    return QORA_HIP_OK;
}

// Uploads the step's input token unless d_token already holds it (the previous
// step's argmax, the usual greedy case). The known value is dropped until the
// new step's result has been read back.
int put_token(qora_hip_ctx* c, uint32_t token) {
    ModelState& m = c->m;
    const bool known = m.dev_token == (int64_t)token;
    m.dev_token = -1;
    if (known) return QORA_HIP_OK;
    c->h_pin[0] = (int32_t)token;
    HIP_TRY(c, hipMemcpyAsync(m.d_token, &c->h_pin[0], 4, hipMemcpyHostToDevice, c->stream));
    return QORA_HIP_OK;
}

}  // namespace

extern "C" int qora_hip_decode(qora_hip_ctx* c, uint32_t token, float* logits, uint32_t* argmax) {
    if (!c) return QORA_HIP_E_INVALID;
    if (int rc = check_step_room(c, 1)) return rc;
    ModelState& m = c->m;
    if (token >= m.vocab) return fail(c, QORA_HIP_E_INVALID, "token id out of range");
    if (force_fail("launch")) return fail(c, QORA_HIP_E_DEVICE, "forced launch failure (QORA_HIP_FORCE_FAIL=launch)");
    if (int rc = put_token(c, token)) return rc;
    if (c->h_tok) {
        reinterpret_cast<volatile int32_t*>(c->h_tok)[0] = kTokPending;
        std::atomic_thread_fence(std::memory_order_seq_cst);
        c->tok_armed = true;
    }
    if (int rc = launch_step(c, true, m.host_pos)) {
        c->tok_armed = false;
        return rc;
    }
    if (int rc = finish_step(c, logits, argmax)) return rc;
    m.host_pos += 1;
    return QORA_HIP_OK;
}

extern "C" int qora_hip_generate_greedy(qora_hip_ctx* c, uint32_t token, uint32_t steps, uint32_t* out) {
    if (!c || (!out && steps)) return fail(c, QORA_HIP_E_INVALID, "null argument");
    if (int rc = check_step_room(c, steps)) return rc;
    ModelState& m = c->m;
    if (token >= m.vocab) return fail(c, QORA_HIP_E_INVALID, "token id out of range");
    if (steps == 0) return QORA_HIP_OK;
    if (force_fail("launch")) return fail(c, QORA_HIP_E_DEVICE, "forced launch failure (QORA_HIP_FORCE_FAIL=launch)");
    if (int rc = put_token(c, token)) return rc;
    for (uint32_t i = 0; i < steps; ++i)
        if (int rc = launch_step(c, true, m.host_pos + i)) return rc;
    HIP_TRY(c, hipMemcpyAsync(out, m.d_gen + m.host_pos, (size_t)steps * 4, hipMemcpyDeviceToHost, c->stream));
    HIP_TRY(c, hipMemcpyAsync(&c->h_pin[17], m.d_range, 4, hipMemcpyDeviceToHost, c->stream));
    HIP_TRY(c, hipStreamSynchronize(c->stream));
    if (c->h_pin[17] != 0) return range_error(c);
    m.dev_token = out[steps - 1];   // the last step's argmax stays in d_token
    m.host_pos += steps;
    return QORA_HIP_OK;
}

namespace {

// Batched prefill unless QORA_HIP_PREFILL=seq (one decode step per prompt
// position) or a contraction length is not a multiple of 32.
bool pf_batched(const ModelState& m) {
    const char* v = std::getenv("QORA_HIP_PREFILL");
    if (v && std::strcmp(v, "seq") == 0) return false;
    return pf_gemm_supported(m.hidden, 2) && pf_gemm_supported(m.H * m.hd, 2) && pf_gemm_supported(m.inter, 2);
}

constexpr uint32_t kPfAttnChunks = 8;   // key chunks per query block of the prefill attention

int pf_setup(qora_hip_ctx* c) {
    ModelState& m = c->m;
    if (m.pf_ready) return QORA_HIP_OK;
    if (c->capturing) return fail(c, QORA_HIP_E_STATE, "prefill set-up allocates: not allowed during capture");
    const uint32_t qd = m.H * m.hd, kvd = m.KVH * m.hd;
    const uint32_t tc = std::min<uint32_t>(512, m.cap);
    const uint32_t kmax = std::max(std::max(m.hidden, qd), m.inter);
    void* ptr = nullptr;
#define PF_ALLOC(field, bytes)                                                     \
    do {                                                                           \
        if (int rc_ = model_alloc(c, (bytes), &ptr)) return rc_;                   \
        m.field = reinterpret_cast<decltype(m.field)>(ptr);                        \
    } while (0)
    PF_ALLOC(d_pf_x, (size_t)tc * m.hidden * 4);
    PF_ALLOC(d_pf_qkv, (size_t)tc * (qd + 2 * kvd) * 4);
    PF_ALLOC(d_pf_q, (size_t)tc * qd * 4);
    PF_ALLOC(d_pf_ao, (size_t)tc * qd * 4);
    PF_ALLOC(d_pf_gu, (size_t)tc * 2 * m.inter * 4);
    PF_ALLOC(d_pf_xn, (size_t)m.hidden * 4);
    PF_ALLOC(d_pf_xh, (size_t)tc * kmax * 2);
    PF_ALLOC(d_pf_xl, (size_t)tc * kmax * 2);
    PF_ALLOC(d_pf_xe, (size_t)tc * 4);
    PF_ALLOC(d_pf_ids, (size_t)m.cap * 4);
    // attention key chunks: up to kPfAttnChunks per query block of >= 16 rows,
    // 64 rows (4 waves x 16) of hd values plus (m, l) per block
    PF_ALLOC(d_pf_apart, (size_t)((tc + 15) / 16) * kPfAttnChunks * m.KVH * 64 * (m.hd + 2) * 4);
    {
        // the largest split-K partial set over every chunk length (the 7 shapes
        // repeat in every layer)
        uint64_t pb = 4;
        for (int j = 0; j < 7; ++j) {
            const DevWeight* w = get_weight(c, m.wids[(size_t)j]);
            if (!w) return fail(c, QORA_HIP_E_STATE, "model weight released");
            for (uint32_t t = 1; t <= tc; ++t) {
                const PfGemmShape sh = pf_gemm_shape(t, (uint32_t)w->k, (uint32_t)w->n, c->cus);
                if (sh.splits > 1) pb = std::max<uint64_t>(pb, (uint64_t)sh.splits * t * w->n * 4);
            }
        }
        // the fused launches of the packed-weight GEMM: q|k|v, o, gate|up, down
        m.pf2 = m.fmt == FMT_Q4 && pf_gemm2_supported(m.hidden, qd) && pf_gemm2_supported(m.hidden, kvd) &&
                pf_gemm2_supported(qd, m.hidden) && pf_gemm2_supported(m.hidden, m.inter) &&
                pf_gemm2_supported(m.inter, m.hidden);
        if (m.pf2) {
            const uint32_t shapes[4][2] = {{m.hidden, qd + 2 * kvd}, {qd, m.hidden}, {m.hidden, 2 * m.inter},
                                           {m.inter, m.hidden}};
            for (const auto& kn : shapes)
                for (uint32_t t = 1; t <= tc; ++t) {
                    const PfGemm2Shape sh = pf_gemm2_shape(t, kn[0], kn[1], c->cus);
                    if (sh.splits > 1) pb = std::max<uint64_t>(pb, (uint64_t)sh.splits * t * kn[1] * 4);
                }
        }
        PF_ALLOC(d_pf_part, pb);
        m.pf_part_bytes = pb;
    }
#undef PF_ALLOC
    m.pf_wf.assign((size_t)m.L * 7, nullptr);
    if (m.fmt == FMT_Q4) {
        uint64_t sb = 0;
        for (uint32_t l = 0; l < m.L; ++l)
            for (int j = 0; j < 7; ++j) {
                const DevWeight* w = get_weight(c, m.wids[(size_t)l * 7 + j]);
                if (!w) return fail(c, QORA_HIP_E_STATE, "model weight released");
                sb = std::max(sb, pf_weight_exp_scratch((uint32_t)w->k, (uint32_t)(w->n / 32)));
            }
        if (int rc = model_alloc(c, sb, &ptr)) return rc;
        uint32_t* scratch = (uint32_t*)ptr;
        for (uint32_t l = 0; l < m.L; ++l)
            for (int j = 0; j < 7; ++j) {
                const DevWeight* w = get_weight(c, m.wids[(size_t)l * 7 + j]);
                if (!w) return fail(c, QORA_HIP_E_STATE, "model weight released");
                const uint32_t groups = (uint32_t)(w->n / 32);
                if (int rc = model_alloc(c, groups, &ptr)) return rc;
                m.pf_wf[(size_t)l * 7 + j] = (int8_t*)ptr;
                HIP_TRY(c, launch_pf_weight_exp((const uint16_t*)w->scales, (uint32_t)w->k, groups, (int8_t*)ptr,
                                                scratch, c->stream));
            }
    }
    if (m.pf2) {
        m.pf_wq.assign((size_t)m.L * 7, nullptr);
        m.pf_sc.assign((size_t)m.L * 7, nullptr);
        for (uint32_t l = 0; l < m.L; ++l)
            for (int j = 0; j < 7; ++j) {
                const DevWeight* w = get_weight(c, m.wids[(size_t)l * 7 + j]);
                if (!w) return fail(c, QORA_HIP_E_STATE, "model weight released");
                if (int rc = model_alloc(c, w->k * w->n / 2, &ptr)) return rc;
                m.pf_wq[(size_t)l * 7 + j] = (uint2*)ptr;
                if (int rc = model_alloc(c, w->k * w->n / 16, &ptr)) return rc;
                m.pf_sc[(size_t)l * 7 + j] = (uint16_t*)ptr;
                HIP_TRY(c, launch_pf_pack_q4((const uint8_t*)w->w, (const uint16_t*)w->scales,
                                             m.pf_wf[(size_t)l * 7 + j], (uint32_t)w->k, (uint32_t)w->n,
                                             m.pf_wq[(size_t)l * 7 + j], m.pf_sc[(size_t)l * 7 + j], c->stream));
            }
    }
    // the lm_head of the last prompt row reads the final-normed fp32 row
    m.p_lmq_pf = m.p_lmq;
    m.p_lmq_pf.x = m.d_pf_xn;
    m.p_lmq_pf.xacc = nullptr;
    m.p_lmq_pf.gamma = nullptr;
    m.p_lm_pf = m.p_lm;
    m.p_lm_pf.x = m.d_pf_xn;
    m.p_lm_pf.xacc = nullptr;
    m.p_lm_pf.gamma = nullptr;
    m.p_fin_pf = ArgmaxFinishParams{m.d_argv, m.d_argi, m.lm_blocks, m.d_token, nullptr, nullptr, c->d_h_tok};
    m.pf_tc = tc;
    m.pf_ready = true;
    return QORA_HIP_OK;
}

int pf_gemm(qora_hip_ctx* c, uint32_t l, int j, uint32_t T, float* y, uint32_t ldy, bool accumulate) {
    ModelState& m = c->m;
    const DevWeight* w = get_weight(c, m.wids[(size_t)l * 7 + j]);
    if (!w) return fail(c, QORA_HIP_E_STATE, "model weight released");
    PrefillGemmParams g{};
    g.xh = m.d_pf_xh;
    g.xl = m.d_pf_xl;
    g.xe = m.d_pf_xe;
    g.T = T;
    g.k = (uint32_t)w->k;
    g.n = (uint32_t)w->n;
    g.w = (const uint8_t*)w->w;
    g.scales = (const uint16_t*)w->scales;
    g.wf = m.pf_wf[(size_t)l * 7 + j];
    g.y = y;
    g.ldy = ldy;
    g.accumulate = accumulate ? 1 : 0;
    PfGemmShape sh = pf_gemm_shape(T, g.k, g.n, c->cus);
    if (sh.splits > 1 && (uint64_t)sh.splits * T * g.n * 4 > m.pf_part_bytes) {
        sh.splits = 1;   // (as in pf_gemm2 below)
        sh.kper = g.k;
    }
    g.nt = sh.nt;
    g.splits = sh.splits;
    g.kper = sh.kper;
    g.part = m.d_pf_part;
    HIP_TRY(c, launch_pf_gemm(w->fmt, g, c->stream));
    return QORA_HIP_OK;
}

// One launch of the packed-weight GEMM over the projections js of layer l
// (their columns side by side), each written to its own rows ys[i] (row
// stride ldy) or added to them.
// Split-K partials left for the next row kernel (the residual add of an o or
// down GEMM summed by the norm that follows it); part == nullptr: none.
struct PfDeferred {
    const float* part = nullptr;
    uint32_t splits = 0;
    uint64_t stride = 0;
};

// defer: when set and the launch splits K, with the segments' rows side by
// side in one output (row stride ldy == ntot), the partials are left for the
// caller, who sums them in split order (and adds them when accumulating)
// swiglu: when set (gate, up: two segments of equal width, not accumulated)
// and the launch runs K unsplit, the GEMM writes h = SiLU(gate) * up to
// ys[0] (row stride n) instead of gate and up, and *swiglu stays true;
// otherwise it is cleared and gate and up are written as usual.
int pf_gemm2(qora_hip_ctx* c, uint32_t l, std::initializer_list<int> js, uint32_t T, std::initializer_list<float*> ys,
             uint32_t ldy, bool accumulate, PfDeferred* defer = nullptr, bool* swiglu = nullptr) {
    ModelState& m = c->m;
    PfGemm2Params g{};
    g.xh = m.d_pf_xh;
    g.xl = m.d_pf_xl;
    g.xe = m.d_pf_xe;
    g.T = T;
    auto yi = ys.begin();
    for (int j : js) {
        const size_t wi = (size_t)l * 7 + (size_t)j;
        const DevWeight* w = get_weight(c, m.wids[wi]);
        if (!w) return fail(c, QORA_HIP_E_STATE, "model weight released");
        PfGemm2Seg& sg = g.seg[g.nseg++];
        sg.wq = m.pf_wq[wi];
        sg.sc = m.pf_sc[wi];
        sg.wf = m.pf_wf[wi];
        sg.n = (uint32_t)w->n;
        sg.nb0 = g.ntot / 128u;
        sg.y = *yi++;
        sg.ldy = ldy;
        sg.accumulate = accumulate ? 1 : 0;
        g.k = (uint32_t)w->k;
        g.ntot += (uint32_t)w->n;
    }
    PfGemm2Shape sh = pf_gemm2_shape(T, g.k, g.ntot, c->cus);
    // (a split set larger than the buffer sized at set-up, as the tuning
    // variables read at each call could ask for, runs unsplit)
    if (sh.splits > 1 && (uint64_t)sh.splits * T * g.ntot * 4 > m.pf_part_bytes) {
        sh.splits = 1;
        sh.kper = g.k;
    }
    g.splits = sh.splits;
    g.kper = sh.kper;
    g.part = m.d_pf_part;
    if (swiglu) {
        *swiglu = *swiglu && g.nseg == 2 && g.seg[0].n == g.seg[1].n && g.splits == 1 && !accumulate;
        if (*swiglu) {
            g.swiglu = 1;
            g.seg[0].ldy = g.seg[0].n;
        }
    }
    bool side = ldy == g.ntot;
    for (int i = 0; i < g.nseg; ++i) side = side && g.seg[i].y == g.seg[0].y + (size_t)g.seg[i].nb0 * 128u;
    const bool leave = defer && g.splits > 1 && side;
    HIP_TRY(c, launch_pf_gemm2(sh.bm, g, c->stream, !leave));
    if (defer) *defer = leave ? PfDeferred{g.part, g.splits, (uint64_t)T * g.ntot} : PfDeferred{};
    return QORA_HIP_OK;
}

// raw_prefill (gemv.rs:1027-1190) over the prompt in chunks of pf_tc tokens:
// every layer runs on the whole chunk (GEMMs on the matrix cores, causal
// attention over the cache rows written so far), then the last row's final
// norm and lm_head give the logits and the greedy token.
int prefill_batched(qora_hip_ctx* c, size_t n, float* logits, uint32_t* argmax) {
    ModelState& m = c->m;
    if (int rc = pf_setup(c)) return rc;
    const hipStream_t s = c->stream;
    const uint32_t qd = m.H * m.hd, kvd = m.KVH * m.hd, qkvn = qd + 2 * kvd;
    const size_t kvb = m.kv_f16 ? 2 : 4;
    const DevWeight* emb = get_weight(c, m.embed_wid);
    if (!emb) return fail(c, QORA_HIP_E_STATE, "embedding weight released");
    uint32_t T = 0;
    for (size_t c0 = 0; c0 < n; c0 += m.pf_tc) {
        T = (uint32_t)std::min<size_t>(m.pf_tc, n - c0);
        PrefillRowParams r{};
        r.ids = m.d_pf_ids + c0;
        r.vocab = m.vocab;
        r.fmt = (int)m.fmt;
        r.emb_w = (const uint8_t*)emb->w;
        r.emb_s = (const uint16_t*)emb->scales;
        r.x = m.d_pf_x;
        r.n = m.hidden;
        HIP_TRY(c, launch_pf_rows(PF_ROW_EMBED, r, T, s));
        PfDeferred pend;   // the previous layer's down partials, summed by this layer's first norm
        for (uint32_t l = 0; l < m.L; ++l) {
            PrefillRowParams nr{};
            nr.x = m.d_pf_x;
            nr.n = m.hidden;
            nr.gamma = m.d_norms + ((size_t)l * 2 + 0) * m.hidden;
            nr.xh = m.d_pf_xh;
            nr.xl = m.d_pf_xl;
            nr.xe = m.d_pf_xe;
            nr.part = pend.part;
            nr.splits = pend.splits;
            nr.part_stride = pend.stride;
            HIP_TRY(c, launch_pf_rows(PF_ROW_RMSNORM, nr, T, s));
            PfDeferred qd_def;   // the q|k|v GEMM's partials, summed by the RoPE / cache kernel
            if (m.pf2) {
                if (int rc = pf_gemm2(c, l, {0, 1, 2}, T, {m.d_pf_qkv, m.d_pf_qkv + qd, m.d_pf_qkv + qd + kvd},
                                      qkvn, false, qkvn <= kPfRopeRowMax ? &qd_def : nullptr))
                    return rc;
            } else {
                if (int rc = pf_gemm(c, l, 0, T, m.d_pf_qkv, qkvn, false)) return rc;
                if (int rc = pf_gemm(c, l, 1, T, m.d_pf_qkv + qd, qkvn, false)) return rc;
                if (int rc = pf_gemm(c, l, 2, T, m.d_pf_qkv + qd + kvd, qkvn, false)) return rc;
            }
            PrefillAttnParams a{};
            a.qkv = m.d_pf_qkv;
            a.q = m.d_pf_q;
            a.kc = (uint8_t*)m.d_k + (size_t)l * m.cap * kvd * kvb;
            a.vc = (uint8_t*)m.d_v + (size_t)l * m.cap * kvd * kvb;
            a.kv_f16 = m.kv_f16;
            a.rope_cos = m.d_cos;
            a.rope_sin = m.d_sin;
            a.use_rope = m.p_attn[l].use_rope;
            a.half = m.half;
            a.pos0 = (uint32_t)c0;
            a.T = T;
            a.H = m.H;
            a.KVH = m.KVH;
            a.hd = m.hd;
            a.scale = 1.0f / sqrtf((float)m.hd);
            a.out = m.d_pf_ao;
            a.kv_ps = m.hd;
            a.kv_hs = (uint64_t)m.cap * m.hd;
            a.part = m.d_pf_apart;
            a.part_nc = kPfAttnChunks;
            a.qkv_part = qd_def.part;
            a.qkv_splits = qd_def.splits;
            a.qkv_part_stride = qd_def.stride;
            HIP_TRY(c, launch_pf_rope_cache(a, s));
            a.qkv_part = nullptr;
            // the attention output comes back split for the o GEMM
            a.xh = m.d_pf_xh;
            a.xl = m.d_pf_xl;
            a.xe = m.d_pf_xe;
            HIP_TRY(c, launch_pf_attn(a, s));
            PfDeferred od;     // the o GEMM's partials, summed by the second norm
            if (int rc = m.pf2 ? pf_gemm2(c, l, {3}, T, {m.d_pf_x}, m.hidden, true, &od)
                               : pf_gemm(c, l, 3, T, m.d_pf_x, m.hidden, true))
                return rc;
            nr.gamma = m.d_norms + ((size_t)l * 2 + 1) * m.hidden;
            nr.part = od.part;
            nr.splits = od.splits;
            nr.part_stride = od.stride;
            HIP_TRY(c, launch_pf_rows(PF_ROW_RMSNORM, nr, T, s));
            bool swiglu = m.pf2;           // SiLU(g) * u formed by the gate|up GEMM when it runs unsplit
            if (m.pf2) {
                if (int rc = pf_gemm2(c, l, {4, 5}, T, {m.d_pf_gu, m.d_pf_gu + m.inter}, 2 * m.inter, false, nullptr,
                                      &swiglu))
                    return rc;
            } else {
                if (int rc = pf_gemm(c, l, 4, T, m.d_pf_gu, 2 * m.inter, false)) return rc;
                if (int rc = pf_gemm(c, l, 5, T, m.d_pf_gu + m.inter, 2 * m.inter, false)) return rc;
            }
            PrefillRowParams gr{};
            gr.x = m.d_pf_gu;
            gr.u = swiglu ? nullptr : m.d_pf_gu + m.inter;
            gr.ld = swiglu ? m.inter : 2 * m.inter;
            gr.n = m.inter;
            gr.xh = m.d_pf_xh;
            gr.xl = m.d_pf_xl;
            gr.xe = m.d_pf_xe;
            HIP_TRY(c, launch_pf_rows(PF_ROW_SILU, gr, T, s));
            // the last layer's down GEMM is reduced in place: the final norm
            // reads the residual rows
            pend = PfDeferred{};
            if (int rc = m.pf2 ? pf_gemm2(c, l, {6}, T, {m.d_pf_x}, m.hidden, true, l + 1 < m.L ? &pend : nullptr)
                               : pf_gemm(c, l, 6, T, m.d_pf_x, m.hidden, true))
                return rc;
        }
    }
    HIP_TRY(c, launch_rmsnorm(m.d_pf_x + (size_t)(T - 1) * m.hidden, m.d_final, m.hidden, m.d_pf_xn, s));
    if (m.lm_mfma) HIP_TRY(c, launch_lmhead(m.lm_blocks, m.p_lmq_pf, s));
    else HIP_TRY(c, launch_rowdot(m.fmt, m.lm_blocks, m.p_lm_pf, s));
    HIP_TRY(c, launch_argmax_finish(m.p_fin_pf, s));
    if (int rc = set_device_pos(c, n)) return rc;
    return finish_step(c, logits, argmax);
}

}  // namespace

extern "C" int qora_hip_prefill(qora_hip_ctx* c, const uint32_t* ids, size_t n, float* logits, uint32_t* argmax) {
    if (!c || !ids) return fail(c, QORA_HIP_E_INVALID, "null argument");
    ModelState& m = c->m;
    if (!m.ready) return fail(c, QORA_HIP_E_STATE, "model not initialised");
    if (c->capturing) return fail(c, QORA_HIP_E_STATE, "decode and prefill steps are not allowed during capture");
    if (n == 0) return fail(c, QORA_HIP_E_INVALID, "empty prompt");
    for (size_t i = 0; i < n; ++i)
        if (ids[i] >= m.vocab) return fail(c, QORA_HIP_E_INVALID, "token id out of range");
    m.host_pos = 0;
    m.dev_token = -1;
    if (int rc = set_device_pos(c, 0)) return rc;
    if (int rc = check_step_room(c, n)) return rc;
    if (force_fail("launch")) return fail(c, QORA_HIP_E_DEVICE, "forced launch failure (QORA_HIP_FORCE_FAIL=launch)");
    if (pf_batched(m) && n > 1) {
        if (int rc = pf_setup(c)) return rc;
        HIP_TRY(c, hipMemcpy(m.d_pf_ids, ids, n * 4, hipMemcpyHostToDevice));
        if (int rc = prefill_batched(c, n, logits, argmax)) return rc;
        m.host_pos = n;
        return QORA_HIP_OK;
    }
    HIP_TRY(c, hipMemcpy(m.d_prompt, ids, n * 4, hipMemcpyHostToDevice));
    for (size_t i = 0; i + 1 < n; ++i)
        if (int rc = launch_step(c, false, i)) return rc;
    if (int rc = put_token(c, ids[n - 1])) return rc;
    if (int rc = launch_step(c, true, n - 1)) return rc;
    if (int rc = finish_step(c, logits, argmax)) return rc;
    m.host_pos = n;
    return QORA_HIP_OK;
}

extern "C" uint32_t qora_hip_attn_o_limit(const qora_hip_ctx* c) {
    if (!c || !c->m.ready) return 0;
    return c->m.attn_o_max;
}

extern "C" uint32_t qora_hip_attn_chunk_limit(const qora_hip_ctx* c) {
    if (!c || !c->m.ready) return 0;
    return c->m.attn_ch_max;
}

extern "C" int qora_hip_kv_len(qora_hip_ctx* c, uint64_t* len) {
    if (!c || !len) return QORA_HIP_E_INVALID;
    if (!c->m.ready) return fail(c, QORA_HIP_E_STATE, "model not initialised");
    *len = c->m.host_pos;
    return QORA_HIP_OK;
}

extern "C" int qora_hip_kv_reset(qora_hip_ctx* c) {
    if (!c) return QORA_HIP_E_INVALID;
    if (!c->m.ready) return fail(c, QORA_HIP_E_STATE, "model not initialised");
    if (c->capturing) return fail(c, QORA_HIP_E_STATE, "kv_reset is not allowed during capture");
    c->m.host_pos = 0;
    return set_device_pos(c, 0);
}

extern "C" int qora_hip_kv_upload(qora_hip_ctx* c, uint32_t layer, const float* k, const float* v, uint64_t len) {
    if (!c) return QORA_HIP_E_INVALID;
    ModelState& m = c->m;
    if (!m.ready) return fail(c, QORA_HIP_E_STATE, "model not initialised");
    if (layer >= m.L) return fail(c, QORA_HIP_E_INVALID, "layer out of range");
    if (len > m.cap) return fail(c, QORA_HIP_E_INVALID, "len beyond the KV capacity");
    if (m.any_rope && len > m.rope_positions) return fail(c, QORA_HIP_E_INVALID, "len beyond the RoPE tables");
    if (len && (!k || !v)) return fail(c, QORA_HIP_E_INVALID, "null argument");
    if (c->capturing) return fail(c, QORA_HIP_E_STATE, "kv_upload is not allowed during capture");
    const size_t kvd = (size_t)m.KVH * m.hd;
    const size_t count = (size_t)len * kvd;
    if (count) {
        // host: token-major [len][KVH][hd] f32, copied up in one piece; a kernel moves it into
        // the head-major [KVH][cap][hd] cache (binary16 for an f16 cache)
        void* tmp = nullptr;
        if (int rc = dalloc(c, count * 4, &tmp)) return rc;
        const float* src[2] = {k, v};
        const size_t eb = m.kv_f16 ? 2 : 4;
        hipError_t e = hipSuccess;
        for (int which = 0; which < 2 && e == hipSuccess; ++which) {
            uint8_t* base = (uint8_t*)(which ? m.d_v : m.d_k) + (size_t)layer * m.cap * kvd * eb;
            e = hipMemcpyAsync(tmp, src[which], count * 4, hipMemcpyHostToDevice, c->stream);
            if (e == hipSuccess)
                e = launch_kv_move(true, m.kv_f16 != 0, (float*)tmp, base, (uint32_t)len, m.KVH, m.hd, m.cap, c->stream);
            if (e == hipSuccess) e = hipStreamSynchronize(c->stream);
        }
        (void)hipFree(tmp);
        if (e != hipSuccess) return fail(c, QORA_HIP_E_DEVICE, std::string("kv_upload: ") + hipGetErrorString(e));
    }
    m.host_pos = len;
    return set_device_pos(c, len);
}

extern "C" int qora_hip_kv_download(qora_hip_ctx* c, uint32_t layer, float* k, float* v) {
    if (!c || !k || !v) return fail(c, QORA_HIP_E_INVALID, "null argument");
    ModelState& m = c->m;
    if (!m.ready) return fail(c, QORA_HIP_E_STATE, "model not initialised");
    if (layer >= m.L) return fail(c, QORA_HIP_E_INVALID, "layer out of range");
    if (c->capturing) return fail(c, QORA_HIP_E_STATE, "kv_download is not allowed during capture");
    const size_t kvd = (size_t)m.KVH * m.hd;
    const size_t n = (size_t)m.host_pos;
    HIP_TRY(c, hipStreamSynchronize(c->stream));
    if (n == 0) return QORA_HIP_OK;
    // device: head-major [KVH][cap][hd]; host: the reference's token-major [len][KVH][hd] f32,
    // gathered on the device and copied down in one piece
    void* tmp = nullptr;
    if (int rc = dalloc(c, n * kvd * 4, &tmp)) return rc;
    const size_t eb = m.kv_f16 ? 2 : 4;
    hipError_t e = hipSuccess;
    for (int which = 0; which < 2 && e == hipSuccess; ++which) {
        uint8_t* base = (uint8_t*)(which ? m.d_v : m.d_k) + (size_t)layer * m.cap * kvd * eb;
        e = launch_kv_move(false, m.kv_f16 != 0, (float*)tmp, base, (uint32_t)n, m.KVH, m.hd, m.cap, c->stream);
        if (e == hipSuccess) e = hipMemcpyAsync(which ? v : k, tmp, n * kvd * 4, hipMemcpyDeviceToHost, c->stream);
        if (e == hipSuccess) e = hipStreamSynchronize(c->stream);
    }
    (void)hipFree(tmp);
    if (e != hipSuccess) return fail(c, QORA_HIP_E_DEVICE, std::string("kv_download: ") + hipGetErrorString(e));
    return QORA_HIP_OK;
}

// ===========================================================================
// memory / graph plumbing
// ===========================================================================

extern "C" int qora_hip_malloc(qora_hip_ctx* c, size_t bytes, void** dptr) {
    if (!c || !dptr) return QORA_HIP_E_INVALID;
    return dalloc(c, bytes, dptr);
}

extern "C" int qora_hip_free(qora_hip_ctx* c, void* dptr) {
    if (!c) return QORA_HIP_E_INVALID;
    if (dptr) HIP_TRY(c, hipFree(dptr));
    return QORA_HIP_OK;
}

extern "C" int qora_hip_memcpy_h2d(qora_hip_ctx* c, void* dst, const void* src, size_t bytes) {
    if (!c || (!dst && bytes) || (!src && bytes)) return QORA_HIP_E_INVALID;
    HIP_TRY(c, hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, c->stream));
    HIP_TRY(c, hipStreamSynchronize(c->stream));
    return QORA_HIP_OK;
}

extern "C" int qora_hip_memcpy_d2h(qora_hip_ctx* c, void* dst, const void* src, size_t bytes) {
    if (!c || (!dst && bytes) || (!src && bytes)) return QORA_HIP_E_INVALID;
    HIP_TRY(c, hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, c->stream));
    HIP_TRY(c, hipStreamSynchronize(c->stream));
    return QORA_HIP_OK;
}

extern "C" int qora_hip_synchronize(qora_hip_ctx* c) {
    if (!c) return QORA_HIP_E_INVALID;
    HIP_TRY(c, hipStreamSynchronize(c->stream));
    return QORA_HIP_OK;
}

extern "C" void* qora_hip_stream(qora_hip_ctx* c) { return c ? (void*)c->stream : nullptr; }

extern "C" int qora_hip_capture_begin(qora_hip_ctx* c) {
    if (!c || c->capturing) return QORA_HIP_E_STATE;
    HIP_TRY(c, hipStreamBeginCapture(c->stream, hipStreamCaptureModeThreadLocal));
    c->capturing = true;
    return QORA_HIP_OK;
}

extern "C" int qora_hip_capture_end(qora_hip_ctx* c, void** graph_exec) {
    if (!c || !c->capturing || !graph_exec) return QORA_HIP_E_STATE;
    c->capturing = false;
    hipGraph_t g = nullptr;
    HIP_TRY(c, hipStreamEndCapture(c->stream, &g));
    hipGraphExec_t ge = nullptr;
    const hipError_t e = hipGraphInstantiate(&ge, g, nullptr, nullptr, 0);
    (void)hipGraphDestroy(g);
    if (e != hipSuccess) return fail(c, QORA_HIP_E_DEVICE, std::string("hipGraphInstantiate: ") + hipGetErrorString(e));
    *graph_exec = (void*)ge;
    return QORA_HIP_OK;
}

extern "C" int qora_hip_graph_launch(qora_hip_ctx* c, void* graph_exec, uint32_t count) {
    if (!c || !graph_exec) return QORA_HIP_E_INVALID;
    for (uint32_t i = 0; i < count; ++i) HIP_TRY(c, hipGraphLaunch((hipGraphExec_t)graph_exec, c->stream));
    return QORA_HIP_OK;
}

extern "C" int qora_hip_graph_destroy(qora_hip_ctx* c, void* graph_exec) {
    if (!c || !graph_exec) return QORA_HIP_E_INVALID;
    HIP_TRY(c, hipGraphExecDestroy((hipGraphExec_t)graph_exec));
    return QORA_HIP_OK;
}

// ===========================================================================
// kernel-level entry points
// ===========================================================================

namespace {

// Argument checks and launch plan of acc[0:n] (+ acc[n:2n] when paired) +=
// W x; nothing is launched, so a refused call leaves the device untouched.
int gemv_acc_prepare(qora_hip_ctx* c, int fmt, const void* w0, const void* s0, const void* w1, const void* s1,
                     const float* x, long long* acc, uint64_t k, uint64_t n, bool paired, GemvPlan* plan,
                     GemvParams* params) {
    if (!c) return QORA_HIP_E_INVALID;
    if (!w0 || !x || !acc || (fmt == FMT_Q4 && !s0) || (paired && (!w1 || (fmt == FMT_Q4 && !s1))))
        return fail(c, QORA_HIP_E_INVALID, "null argument");
    if (k == 0 || n == 0 || n % 32 != 0 || k > 0xFFFFFFFFull || n / 32 > 0xFFFFFFFFull)
        return fail(c, QORA_HIP_E_INVALID, "GEMV needs k > 0 and n % 32 == 0");
    const uint32_t G = (uint32_t)(n / 32);
    const uint32_t groups[2] = {G, G};
    GemvPlan pl;
    if (!plan_gemv(fmt, (uint32_t)k, groups, paired ? 2 : 1, paired, c->cus, &pl))
        return fail(c, QORA_HIP_E_INVALID, "unsupported GEMV shape");
    GemvParams p{};
    p.seg[0] = GemvSeg{(const uint8_t*)w0, (const uint16_t*)s0, G, 0, 0, 0};
    p.nseg = 1;
    if (paired) {
        p.seg[1] = GemvSeg{(const uint8_t*)w1, (const uint16_t*)s1, G, 0, 0, 0};
        p.nseg = 2;
        p.paired = 1;
    }
    p.k = (uint32_t)k;
    p.pro = PRO_PLAIN;
    p.x = x;
    p.acc = acc;
    apply_plan(pl, &p);
    *plan = pl;
    *params = p;
    return QORA_HIP_OK;
}

// acc[0:n] (+ acc[n:2n] when paired) += W x, one launch of the model's GEMV
// kernel with the plain-vector prologue.
int gemv_acc_entry(qora_hip_ctx* c, int fmt, const void* w0, const void* s0, const void* w1, const void* s1,
                   const float* x, long long* acc, uint64_t k, uint64_t n, bool paired, void* stream) {
    GemvPlan pl;
    GemvParams p{};
    if (int rc = gemv_acc_prepare(c, fmt, w0, s0, w1, s1, x, acc, k, n, paired, &pl, &p)) return rc;
    HIP_TRY(c, launch_gemv(fmt, pl, p, pick_stream(c, stream)));
    return QORA_HIP_OK;
}

// y = W x (paired: y = silu(Wg x) * (Wu x)) through the context accumulator:
// clear, accumulate, convert.
int gemv_entry(qora_hip_ctx* c, int fmt, const void* w0, const void* s0, const void* w1, const void* s1,
               const float* x, float* y, uint64_t k, uint64_t n, bool paired, void* stream) {
    if (!c) return QORA_HIP_E_INVALID;
    if (!y) return fail(c, QORA_HIP_E_INVALID, "null argument");
    if (n == 0 || n > 0x7FFFFFFFull) return fail(c, QORA_HIP_E_INVALID, "GEMV needs 0 < n < 2^31");
    const uint64_t accn = paired ? 2 * n : n;
    if (int rc = ensure_acc_ws(c, accn)) return rc;
    const hipStream_t s = pick_stream(c, stream);
    HIP_TRY(c, launch_fill_zero(c->ws_acc, accn, s));
    if (int rc = gemv_acc_entry(c, fmt, w0, s0, w1, s1, x, c->ws_acc, k, n, paired, stream)) return rc;
    HIP_TRY(c, launch_acc_to_f32(c->ws_acc, (uint32_t)n, paired ? 1 : 0, y, s));
    return QORA_HIP_OK;
}

int rowdot_entry(qora_hip_ctx* c, int fmt, const void* w, const void* s, const float* x, float* y, uint64_t rows,
                 uint64_t cols, void* stream) {
    if (!c) return QORA_HIP_E_INVALID;
    if (!w || !x || !y || (fmt == FMT_Q4 && !s)) return fail(c, QORA_HIP_E_INVALID, "null argument");
    if (rows == 0 || rows > 0xFFFFFFFFull || cols == 0 || cols % 32 != 0 || cols / 32 > 64 || 64 % (cols / 32) != 0)
        return fail(c, QORA_HIP_E_INVALID, "row-dot GEMV needs cols % 32 == 0 and cols/32 dividing 64");
    RowdotParams p{};
    p.w = (const uint8_t*)w;
    p.scales = (const uint16_t*)s;
    p.rows = (uint32_t)rows;
    p.cols = (uint32_t)cols;
    p.x = x;
    p.y = y;
    HIP_TRY(c, launch_rowdot(fmt, rowdot_blocks(p.rows, p.cols, c->cus), p, pick_stream(c, stream)));
    return QORA_HIP_OK;
}

}  // namespace

extern "C" int qora_hip_gemv_q4(qora_hip_ctx* c, const void* packed, const void* scales, const float* x, float* y,
                                uint64_t k, uint64_t n, void* stream) {
    return gemv_entry(c, FMT_Q4, packed, scales, nullptr, nullptr, x, y, k, n, false, stream);
}

extern "C" int qora_hip_gemv_q4_noalloc(qora_hip_ctx* c, const void* packed, const void* scales, const float* x,
                                        float* y, uint64_t k, uint64_t n, void* stream) {
    if (!c) return QORA_HIP_E_INVALID;
    if (!y) return fail(c, QORA_HIP_E_INVALID, "null argument");
    if (n == 0 || n > kNoAllocMaxN)
        return fail(c, QORA_HIP_E_INVALID, "gemv_q4_noalloc takes 0 < n <= " + std::to_string(kNoAllocMaxN));
    long long* acc = noalloc_scratch(c->device);
    if (!acc) return fail(c, QORA_HIP_E_DEVICE, "gemv_q4_noalloc: no scratch address on this device");
    // the same kernels as qora_hip_gemv_q4, on the device's static scratch
    // instead of the context's grown accumulator: clear (a kernel, not a
    // memset), accumulate, convert
    // every argument is checked before the first launch: a refused call
    // writes nothing to the device-wide scratch
    GemvPlan pl;
    GemvParams p{};
    if (int rc = gemv_acc_prepare(c, FMT_Q4, packed, scales, nullptr, nullptr, x, acc, k, n, false, &pl, &p))
        return rc;
    const hipStream_t s = pick_stream(c, stream);
    HIP_TRY(c, launch_fill_zero(acc, n, s));
    HIP_TRY(c, launch_gemv(FMT_Q4, pl, p, s));
    HIP_TRY(c, launch_acc_to_f32(acc, (uint32_t)n, 0, y, s));
    return QORA_HIP_OK;
}

extern "C" int qora_hip_gemv_f16(qora_hip_ctx* c, const void* w, const float* x, float* y, uint64_t k, uint64_t n,
                                 void* stream) {
    return gemv_entry(c, FMT_F16, w, nullptr, nullptr, nullptr, x, y, k, n, false, stream);
}

extern "C" int qora_hip_gate_up_q4(qora_hip_ctx* c, const void* gp, const void* gs, const void* up, const void* us,
                                   const float* x, float* out, uint64_t k, uint64_t n, void* stream) {
    return gemv_entry(c, FMT_Q4, gp, gs, up, us, x, out, k, n, true, stream);
}

extern "C" int qora_hip_gate_up_f16(qora_hip_ctx* c, const void* gw, const void* uw, const float* x, float* out,
                                    uint64_t k, uint64_t n, void* stream) {
    return gemv_entry(c, FMT_F16, gw, nullptr, uw, nullptr, x, out, k, n, true, stream);
}

extern "C" int qora_hip_gemv_q4_accumulate(qora_hip_ctx* c, const void* packed, const void* scales,
                                           const float* x, long long* acc, uint64_t k, uint64_t n, void* stream) {
    return gemv_acc_entry(c, FMT_Q4, packed, scales, nullptr, nullptr, x, acc, k, n, false, stream);
}

extern "C" int qora_hip_gate_up_q4_accumulate(qora_hip_ctx* c, const void* gp, const void* gs, const void* up,
                                              const void* us, const float* x, long long* acc, uint64_t k,
                                              uint64_t n, void* stream) {
    return gemv_acc_entry(c, FMT_Q4, gp, gs, up, us, x, acc, k, n, true, stream);
}

extern "C" int qora_hip_gemv_prepare(qora_hip_ctx* c, uint32_t wid, uint32_t wid_up, int paired, uint32_t* gemv_id) {
    if (!c) return QORA_HIP_E_INVALID;
    if (!gemv_id) return fail(c, QORA_HIP_E_INVALID, "null argument");
    if (c->capturing) return fail(c, QORA_HIP_E_STATE, "gemv_prepare allocates: not allowed during capture");
    const DevWeight* w0 = get_weight(c, wid);
    const DevWeight* w1 = paired ? get_weight(c, wid_up) : nullptr;
    if (!w0 || (paired && !w1)) return fail(c, QORA_HIP_E_INVALID, "unknown weight id");
    if (paired && (w1->fmt != w0->fmt || w1->k != w0->k || w1->n != w0->n))
        return fail(c, QORA_HIP_E_INVALID, "gate and up weights differ in format or shape");
    if (w0->k > 0xFFFFFFFFull || w0->n / 32 > 0xFFFFFFFFull)
        return fail(c, QORA_HIP_E_INVALID, "GEMV shape too large");
    PreparedGemv g;
    g.fmt = w0->fmt;
    g.paired = paired != 0;
    g.k = w0->k;
    g.n = w0->n;
    const uint32_t G = (uint32_t)(w0->n / 32);
    const uint32_t groups[2] = {G, G};
    if (!plan_model_gemv(g.fmt, (uint32_t)g.k, groups, g.paired ? 2 : 1, g.paired, c->cus, &g.plan))
        return fail(c, QORA_HIP_E_INVALID, "unsupported GEMV shape");
    g.p.seg[0] = GemvSeg{(const uint8_t*)w0->w, (const uint16_t*)w0->scales, G, 0, 0, 0};
    g.p.nseg = 1;
    if (g.paired) {
        g.p.seg[1] = GemvSeg{(const uint8_t*)w1->w, (const uint16_t*)w1->scales, G, 0, 0, 0};
        g.p.nseg = 2;
        g.p.paired = 1;
    }
    g.p.k = (uint32_t)g.k;
    g.p.pro = PRO_PLAIN;
    apply_plan(g.plan, &g.p);
    uint64_t wb = 0, sb = 0, eb = 0;
    gemv_tile_bytes(g.fmt, g.plan, &wb, &sb, &eb);
    auto release = [&]() {
        for (void* q : {g.tw, g.ts, g.te})
            if (q) (void)hipFree(q);
    };
    if (int rc = dalloc(c, wb, &g.tw)) return rc;
    if (sb)
        if (int rc = dalloc(c, sb, &g.ts)) { release(); return rc; }
    if (eb)
        if (int rc = dalloc(c, eb, &g.te)) { release(); return rc; }
    const hipError_t e =
        launch_gemv_tile(g.fmt, g.plan, g.p, (uint8_t*)g.tw, (uint16_t*)g.ts, (int8_t*)g.te, c->stream);
    const hipError_t e2 = e == hipSuccess ? hipStreamSynchronize(c->stream) : e;
    if (e2 != hipSuccess) {
        release();
        return fail(c, QORA_HIP_E_DEVICE, std::string("gemv tile packing: ") + hipGetErrorString(e2));
    }
    g.p.tw = (const uint8_t*)g.tw;
    g.p.ts = (const uint16_t*)g.ts;
    g.p.tes = (const int8_t*)g.te;
    g.alive = true;
    *gemv_id = (uint32_t)c->gemvs.size();
    c->gemvs.push_back(g);
    return QORA_HIP_OK;
}

extern "C" int qora_hip_gemv_run(qora_hip_ctx* c, uint32_t gemv_id, const float* x, long long* acc, void* stream) {
    if (!c) return QORA_HIP_E_INVALID;
    if (gemv_id >= c->gemvs.size() || !c->gemvs[gemv_id].alive) return fail(c, QORA_HIP_E_INVALID, "unknown GEMV id");
    if (!x || !acc) return fail(c, QORA_HIP_E_INVALID, "null argument");
    const PreparedGemv& g = c->gemvs[gemv_id];
    if (g.lm_head) return fail(c, QORA_HIP_E_INVALID, "id was prepared by lm_head_prepare: use lm_head_run");
    GemvParams p = g.p;
    p.x = x;
    p.acc = acc;
    HIP_TRY(c, launch_gemv(g.fmt, g.plan, p, pick_stream(c, stream)));
    return QORA_HIP_OK;
}

extern "C" int qora_hip_gemv_release(qora_hip_ctx* c, uint32_t gemv_id) {
    if (!c) return QORA_HIP_E_INVALID;
    if (gemv_id >= c->gemvs.size() || !c->gemvs[gemv_id].alive) return fail(c, QORA_HIP_E_INVALID, "unknown GEMV id");
    if (c->capturing) return fail(c, QORA_HIP_E_STATE, "gemv_release frees: not allowed during capture");
    HIP_TRY(c, hipStreamSynchronize(c->stream));
    PreparedGemv& g = c->gemvs[gemv_id];
    for (void* q : {g.tw, g.ts, g.te, g.part_val, g.part_idx})
        if (q) (void)hipFree(q);
    g = PreparedGemv();
    return QORA_HIP_OK;
}

extern "C" int qora_hip_lm_head_prepare(qora_hip_ctx* c, uint32_t wid, uint32_t* lm_id) {
    if (!c) return QORA_HIP_E_INVALID;
    if (!lm_id) return fail(c, QORA_HIP_E_INVALID, "null argument");
    if (c->capturing) return fail(c, QORA_HIP_E_STATE, "lm_head_prepare allocates: not allowed during capture");
    const DevWeight* w = get_weight(c, wid);
    if (!w) return fail(c, QORA_HIP_E_INVALID, "unknown weight id");
    if (w->fmt != FMT_Q4) return fail(c, QORA_HIP_E_INVALID, "lm_head_prepare takes a Q4 weight");
    if (w->k == 0 || w->k > 0x7FFFFFF0ull || w->n > 0xFFFFFFFFull || !lmhead_supported((uint32_t)w->n))
        return fail(c, QORA_HIP_E_INVALID, "lm_head shape: cols must be 128, 256, 512, 1024 or 2048");
    PreparedGemv g;
    g.fmt = FMT_Q4;
    g.lm_head = true;
    g.k = w->k;
    g.n = w->n;
    const uint32_t rows = (uint32_t)w->k, cols = (uint32_t)w->n;
    g.lm_blocks = lmhead_blocks(rows, c->cus);
    uint64_t wb = 0, sb = 0;
    lmhead_tile_bytes(rows, cols, &wb, &sb);
    auto release = [&]() {
        for (void* q : {g.tw, g.ts, g.part_val, g.part_idx})
            if (q) (void)hipFree(q);
    };
    if (int rc = dalloc(c, wb, &g.tw)) return rc;
    if (int rc = dalloc(c, sb, &g.ts)) { release(); return rc; }
    if (int rc = dalloc(c, (size_t)g.lm_blocks * 4, &g.part_val)) { release(); return rc; }
    if (int rc = dalloc(c, (size_t)g.lm_blocks * 4, &g.part_idx)) { release(); return rc; }
    const hipError_t e = launch_lmhead_pack((const uint8_t*)w->w, (const uint16_t*)w->scales, rows, cols,
                                            (uint8_t*)g.tw, (uint32_t*)g.ts, c->stream);
    const hipError_t e2 = e == hipSuccess ? hipStreamSynchronize(c->stream) : e;
    if (e2 != hipSuccess) {
        release();
        return fail(c, QORA_HIP_E_DEVICE, std::string("lm_head tile packing: ") + hipGetErrorString(e2));
    }
    g.lp.tw = (const uint8_t*)g.tw;
    g.lp.ts = (const uint32_t*)g.ts;
    g.lp.rows = rows;
    g.lp.cols = cols;
    g.lp.tiles = lmhead_tiles(rows);
    g.lp.part_val = (float*)g.part_val;
    g.lp.part_idx = (uint32_t*)g.part_idx;
    g.alive = true;
    *lm_id = (uint32_t)c->gemvs.size();
    c->gemvs.push_back(g);
    return QORA_HIP_OK;
}

extern "C" int qora_hip_lm_head_run(qora_hip_ctx* c, uint32_t lm_id, const float* x, float* logits,
                                    int32_t* argmax_device, void* stream) {
    if (!c) return QORA_HIP_E_INVALID;
    if (lm_id >= c->gemvs.size() || !c->gemvs[lm_id].alive) return fail(c, QORA_HIP_E_INVALID, "unknown lm_head id");
    if (!x || !logits) return fail(c, QORA_HIP_E_INVALID, "null argument");
    const PreparedGemv& g = c->gemvs[lm_id];
    if (!g.lm_head) return fail(c, QORA_HIP_E_INVALID, "id was prepared by gemv_prepare: use gemv_run");
    LmHeadParams p = g.lp;
    p.x = x;
    p.y = logits;
    p.do_argmax = argmax_device != nullptr;
    const hipStream_t s = pick_stream(c, stream);
    HIP_TRY(c, launch_lmhead(g.lm_blocks, p, s));
    if (argmax_device) {
        const ArgmaxFinishParams f{p.part_val, p.part_idx, g.lm_blocks, argmax_device, nullptr, nullptr};
        HIP_TRY(c, launch_argmax_finish(f, s));
    }
    return QORA_HIP_OK;
}

extern "C" int qora_hip_acc_to_f32(qora_hip_ctx* c, const long long* acc, uint64_t n, int paired, float* y,
                                   void* stream) {
    if (!c) return QORA_HIP_E_INVALID;
    if (!acc || !y) return fail(c, QORA_HIP_E_INVALID, "null argument");
    if (n == 0 || n > 0x7FFFFFFFull) return fail(c, QORA_HIP_E_INVALID, "bad length");
    HIP_TRY(c, launch_acc_to_f32(acc, (uint32_t)n, paired ? 1 : 0, y, pick_stream(c, stream)));
    return QORA_HIP_OK;
}

extern "C" int qora_hip_gemv_q4_rowdot(qora_hip_ctx* c, const void* packed, const void* scales, const float* x,
                                       float* y, uint64_t rows, uint64_t cols, void* stream) {
    return rowdot_entry(c, FMT_Q4, packed, scales, x, y, rows, cols, stream);
}

extern "C" int qora_hip_gemv_f16_rowdot(qora_hip_ctx* c, const void* w, const float* x, float* y, uint64_t rows,
                                        uint64_t cols, void* stream) {
    return rowdot_entry(c, FMT_F16, w, nullptr, x, y, rows, cols, stream);
}

extern "C" int qora_hip_dequant_q4(qora_hip_ctx* c, const void* packed, const void* scales, uint64_t k, uint64_t n,
                                   float* out, void* stream) {
    if (!c) return QORA_HIP_E_INVALID;
    if (!packed || !scales || !out) return fail(c, QORA_HIP_E_INVALID, "null argument");
    if (k == 0 || n == 0 || n % 32 != 0) return fail(c, QORA_HIP_E_INVALID, "dequant needs n % 32 == 0");
    HIP_TRY(c, launch_dequant_q4((const uint8_t*)packed, (const uint16_t*)scales, k, n, out, pick_stream(c, stream)));
    return QORA_HIP_OK;
}

extern "C" int qora_hip_rmsnorm(qora_hip_ctx* c, const float* x, const void* gamma, uint64_t n, float* out,
                                void* stream) {
    if (!c) return QORA_HIP_E_INVALID;
    if (!x || !gamma || !out) return fail(c, QORA_HIP_E_INVALID, "null argument");
    if (n == 0 || n > 0xFFFFFFFFull) return fail(c, QORA_HIP_E_INVALID, "bad length");
    HIP_TRY(c, launch_rmsnorm(x, (const uint16_t*)gamma, (uint32_t)n, out, pick_stream(c, stream)));
    return QORA_HIP_OK;
}

extern "C" int qora_hip_rope(qora_hip_ctx* c, float* data, uint32_t num_heads, uint32_t head_dim, const float* cos_t,
                             const float* sin_t, uint32_t half_dim, uint32_t position, void* stream) {
    if (!c) return QORA_HIP_E_INVALID;
    if (!data || !cos_t || !sin_t) return fail(c, QORA_HIP_E_INVALID, "null argument");
    if (num_heads == 0 || half_dim == 0 || 2 * half_dim > head_dim)
        return fail(c, QORA_HIP_E_INVALID, "need 0 < 2*half_dim <= head_dim");
    HIP_TRY(c, launch_rope(data, num_heads, head_dim, cos_t, sin_t, half_dim, position, pick_stream(c, stream)));
    return QORA_HIP_OK;
}

extern "C" int qora_hip_attn_decode(qora_hip_ctx* c, const float* q, const void* kc, const void* vc, int kv_f16,
                                    uint32_t L, uint32_t H, uint32_t KVH, uint32_t hd, float* out, void* stream) {
    if (!c) return QORA_HIP_E_INVALID;
    if (!q || !kc || !vc || !out) return fail(c, QORA_HIP_E_INVALID, "null argument");
    if (L == 0 || H == 0 || KVH == 0 || H % KVH != 0 || H / KVH > (uint32_t)kAttnMaxGroups || hd == 0 ||
        hd > (uint32_t)kAttnMaxHd || hd % 8 != 0)
        return fail(c, QORA_HIP_E_INVALID,
                    "attention needs L > 0, H % KVH == 0, H/KVH <= 4, head_dim <= 128 and a multiple of 8");
    AttnParams a{};
    a.q = q;
    a.kc = const_cast<void*>(kc);
    a.vc = const_cast<void*>(vc);
    a.kv_f16 = kv_f16 ? 1 : 0;
    a.L = L;
    a.H = H;
    a.KVH = KVH;
    a.hd = hd;
    a.groups = H / KVH;
    a.scale = 1.0f / sqrtf((float)hd);
    attn_geometry(L, &a.chunk, &a.s_max);
    a.nsg = attn_nsg(a.chunk);
    if (int rc = ensure_attn_ws(c, (uint64_t)KVH * a.s_max * a.groups * (hd + 2))) return rc;
    a.part = c->ws_attn_part;
    const hipStream_t s = pick_stream(c, stream);
    HIP_TRY(c, launch_attn(a, s));
    AttnCombineParams cp{a.part, nullptr, L, H, KVH, hd, a.groups, a.chunk, a.s_max, out};
    HIP_TRY(c, launch_attn_combine(cp, s));
    return QORA_HIP_OK;
}

extern "C" int qora_hip_gemm(qora_hip_ctx* c, uint32_t wid, const float* x, float* y, uint64_t T, void* stream) {
    if (!c) return QORA_HIP_E_INVALID;
    if (!x || !y) return fail(c, QORA_HIP_E_INVALID, "null argument");
    const DevWeight* w = get_weight(c, wid);
    if (!w) return fail(c, QORA_HIP_E_INVALID, "unknown weight id");
    if (T == 0 || T > 0x7FFFFFFFull) return fail(c, QORA_HIP_E_INVALID, "bad row count");
    if (!pf_gemm_supported((uint32_t)w->k, (uint32_t)w->n)) return fail(c, QORA_HIP_E_INVALID, "k must be a multiple of 32");
    const uint32_t K = (uint32_t)w->k, N = (uint32_t)w->n;
    // Q4 with n % 128 == 0 runs the prefill's packed-weight GEMM (the weight
    // packed into the workspace for this call), anything else pf_gemm_kernel
    const bool packed = w->fmt == FMT_Q4 && pf_gemm2_supported(K, N);
    // scratch: xh, xl [T][k] binary16, xe [T], wf [n/32], exponent partials,
    // then the packed weight (wq, sc) or nothing, then the split-K partials
    // (each part 256-byte aligned)
    auto al = [](uint64_t b) { return (b + 255) & ~uint64_t(255); };
    const uint64_t bx = al(T * K * 2), be = al(T * 4), bf = al(N / 32 + 1);
    const uint64_t bs = al(pf_weight_exp_scratch(K, N / 32));
    const uint64_t bq = packed ? al((uint64_t)K * N / 2) : 0, bc = packed ? al((uint64_t)K * N / 16) : 0;
    const PfGemmShape sh = pf_gemm_shape((uint32_t)T, K, N, c->cus);
    const PfGemm2Shape s2 = packed ? pf_gemm2_shape((uint32_t)T, K, N, c->cus) : PfGemm2Shape{};
    const uint32_t splits = packed ? s2.splits : sh.splits;
    const uint64_t bp = splits > 1 ? al((uint64_t)splits * T * N * 4) : 0;
    if (int rc = ensure_pf_ws(c, 2 * bx + be + bf + bs + bq + bc + bp)) return rc;
    uint8_t* base = (uint8_t*)c->ws_pf;
    uint8_t* wq = base + 2 * bx + be + bf + bs;
    float* part = splits > 1 ? (float*)(wq + bq + bc) : nullptr;
    const hipStream_t s = pick_stream(c, stream);
    PrefillRowParams r{};
    r.x = const_cast<float*>(x);
    r.n = K;
    r.xh = (uint16_t*)base;
    r.xl = (uint16_t*)(base + bx);
    r.xe = (int32_t*)(base + 2 * bx);
    HIP_TRY(c, launch_pf_rows(PF_ROW_SPLIT, r, (uint32_t)T, s));
    int8_t* wf = (int8_t*)(base + 2 * bx + be);
    if (w->fmt == FMT_Q4)
        HIP_TRY(c, launch_pf_weight_exp((const uint16_t*)w->scales, K, N / 32, wf, (uint32_t*)(base + 2 * bx + be + bf), s));
    if (packed) {
        HIP_TRY(c, launch_pf_pack_q4((const uint8_t*)w->w, (const uint16_t*)w->scales, wf, K, N, (uint2*)wq,
                                     (uint16_t*)(wq + bq), s));
        PfGemm2Params h{};
        h.xh = r.xh;
        h.xl = r.xl;
        h.xe = r.xe;
        h.T = (uint32_t)T;
        h.k = K;
        h.nseg = 1;
        h.ntot = N;
        h.seg[0] = PfGemm2Seg{(const uint2*)wq, (const uint16_t*)(wq + bq), wf, N, 0, y, N, 0};
        h.splits = s2.splits;
        h.kper = s2.kper;
        h.part = part;
        HIP_TRY(c, launch_pf_gemm2(s2.bm, h, s));
        return QORA_HIP_OK;
    }
    PrefillGemmParams g{};
    g.xh = r.xh;
    g.xl = r.xl;
    g.xe = r.xe;
    g.T = (uint32_t)T;
    g.k = K;
    g.n = N;
    g.w = (const uint8_t*)w->w;
    g.scales = (const uint16_t*)w->scales;
    g.wf = w->fmt == FMT_Q4 ? wf : nullptr;
    g.y = y;
    g.ldy = N;
    g.nt = sh.nt;
    g.splits = sh.splits;
    g.kper = sh.kper;
    g.part = part;
    HIP_TRY(c, launch_pf_gemm(w->fmt, g, s));
    return QORA_HIP_OK;
}

extern "C" int qora_hip_attn_prefill(qora_hip_ctx* c, const float* q, const void* kc, const void* vc, int kv_f16,
                                     uint32_t pos0, uint32_t T, uint32_t H, uint32_t KVH, uint32_t hd, float* out,
                                     void* stream) {
    if (!c) return QORA_HIP_E_INVALID;
    if (!q || !kc || !vc || !out) return fail(c, QORA_HIP_E_INVALID, "null argument");
    if (T == 0 || H == 0 || KVH == 0 || H % KVH != 0 || hd == 0 || hd > (uint32_t)kAttnMaxHd || hd % 8 != 0)
        return fail(c, QORA_HIP_E_INVALID, "attention needs T > 0, H % KVH == 0, head_dim <= 128 and a multiple of 8");
    PrefillAttnParams a{};
    a.q = const_cast<float*>(q);
    a.kc = const_cast<void*>(kc);
    a.vc = const_cast<void*>(vc);
    a.kv_f16 = kv_f16 ? 1 : 0;
    a.pos0 = pos0;
    a.T = T;
    a.H = H;
    a.KVH = KVH;
    a.hd = hd;
    a.scale = 1.0f / sqrtf((float)hd);
    a.out = out;
    HIP_TRY(c, launch_pf_attn(a, pick_stream(c, stream)));
    return QORA_HIP_OK;
}

namespace {

// Argument checks of a sampling call, made before anything is launched.
int sample_check(qora_hip_ctx* c, bool have_logits, uint64_t vocab, const uint32_t* history, uint64_t n_history,
                 const qora_sample_params* sp, const uint64_t* rng_state, const uint32_t* token) {
    if (!have_logits || !sp || !rng_state || !token || (n_history && !history))
        return fail(c, QORA_HIP_E_INVALID, "null argument");
    if (vocab == 0 || vocab > 0xFFFFFFFFull || !smp_sort_supported((uint32_t)vocab))
        return fail(c, QORA_HIP_E_INVALID, "sampling supports vocabularies of 1 .. 4194304 tokens");
    if (c->capturing) return fail(c, QORA_HIP_E_STATE, "sampling copies to the host: not allowed during capture");
    return QORA_HIP_OK;
}

// Penalty list and device scratch for one sampling call, then the kernels;
// the token and the advanced rng state come back to the host. top_k 1..64
// on a vocabulary of up to 131072 keeps each block's best 64 keys; any other
// top_k (0 = the whole vocabulary, sample_token_top_k's k, generate.rs:357-363)
// or a larger vocabulary sorts every key.

// dev_token (optional): the token is also stored there on the device (a
// decode step's input slot). With mapped host memory the token and state are
// read from it as soon as the kernel has stored them, without waiting for the
// stream (as a greedy step's token is); the list's copy and the kernels have
// then finished reading their inputs.
int sample_device(qora_hip_ctx* c, const float* logits, uint64_t vocab, const uint32_t* history, uint64_t n_history,
                  const qora_sample_params* sp, uint64_t* rng_state, uint32_t* token, hipStream_t s,
                  int32_t* dev_token = nullptr) {
    if (int rc = sample_check(c, logits != nullptr, vocab, history, n_history, sp, rng_state, token)) return rc;
    const bool greedy = !(sp->temperature > 0.0f);
    const bool rep = !greedy && sp->repetition_penalty > 1.0f;
    const bool pres = !greedy && sp->presence_penalty > 0.0f;
    // distinct history tokens with their penalties (apply_repetition_penalty walks the last 64
    // tokens, apply_presence_penalty every token; ids >= vocab are skipped, generate.rs:68, 85)
    std::vector<SamplePenalty> pen;
    {
        std::unordered_map<uint32_t, size_t> at;
        auto entry = [&](uint32_t t) -> SamplePenalty& {
            auto it = at.find(t);
            if (it != at.end()) return pen[it->second];
            at.emplace(t, pen.size());
            pen.push_back(SamplePenalty{t, 0, 0, 0});
            return pen.back();
        };
        if (rep)
            for (uint64_t i = n_history - std::min<uint64_t>(64, n_history); i < n_history; ++i)
                if (history[i] < vocab) entry(history[i]).rep_count += 1;
        if (pres)
            for (uint64_t i = 0; i < n_history; ++i)
                if (history[i] < vocab) entry(history[i]).seen = 1;
    }
    const uint32_t V = (uint32_t)vocab, blocks = smp_blocks(V);
    if (V > c->smp_vocab || !c->smp_rng) {
        HIP_TRY(c, hipStreamSynchronize(c->stream));
        for (void* q : {(void*)c->smp_work, (void*)c->smp_cand, (void*)c->smp_rng})   // smp_tok lies in smp_rng
            if (q) (void)hipFree(q);
        c->smp_work = nullptr;
        c->smp_cand = nullptr;
        c->smp_rng = nullptr;
        c->smp_tok = nullptr;
        c->smp_vocab = 0;
        void* q = nullptr;
        if (int rc = dalloc(c, (size_t)V * 4, &q)) return rc;
        c->smp_work = (float*)q;
        if (int rc = dalloc(c, (size_t)blocks * 64 * 8, &q)) return rc;
        c->smp_cand = (unsigned long long*)q;
        if (int rc = dalloc(c, 256, &q)) return rc;
        c->smp_rng = (unsigned long long*)q;
        c->smp_tok = (int32_t*)((uint8_t*)q + 64);
        c->smp_vocab = V;
    }
    if (pen.size() > c->smp_pen_n) {
        HIP_TRY(c, hipStreamSynchronize(c->stream));
        if (c->smp_pen) (void)hipFree(c->smp_pen);
        c->smp_pen = nullptr;
        c->smp_pen_n = 0;
        void* q = nullptr;
        const uint64_t n = std::max<uint64_t>(pen.size(), 1024);
        if (int rc = dalloc(c, n * sizeof(SamplePenalty), &q)) return rc;
        c->smp_pen = (SamplePenalty*)q;
        c->smp_pen_n = n;
    }
    if (pen.size() > c->h_pen_n) {
        HIP_TRY(c, hipStreamSynchronize(s));
        if (c->h_pen) (void)hipHostFree(c->h_pen);
        c->h_pen = nullptr;
        c->h_pen_n = 0;
        const uint64_t n = std::max<uint64_t>(pen.size(), 1024);
        if (hipHostMalloc((void**)&c->h_pen, n * sizeof(SamplePenalty), hipHostMallocDefault) != hipSuccess) {
            c->h_pen = nullptr;
            return fail(c, QORA_HIP_E_NOMEM, "pinned penalty buffer");
        }
        c->h_pen_n = n;
    }
    if (!pen.empty()) {
        // through pinned memory: the copy may run after this call returns
        std::memcpy(c->h_pen, pen.data(), pen.size() * sizeof(SamplePenalty));
        HIP_TRY(c, hipMemcpyAsync(c->smp_pen, c->h_pen, pen.size() * sizeof(SamplePenalty), hipMemcpyHostToDevice, s));
    }
    volatile int32_t* ho = c->d_h_tok ? c->h_tok + 4 : nullptr;   // [0] token, [2..3] state
    if (ho) {
        ho[0] = kTokPending;
        std::atomic_thread_fence(std::memory_order_seq_cst);
    }
    SampleParams p{};
    p.rng_in = *rng_state;
    p.host_out = ho ? c->d_h_tok + 4 : nullptr;
    p.dev_token = dev_token;
    p.work = c->smp_work;
    p.vocab = V;
    p.pen = c->smp_pen;
    p.n_pen = (uint32_t)pen.size();
    p.repetition = sp->repetition_penalty;
    p.presence = sp->presence_penalty;
    p.cand = c->smp_cand;
    p.blocks = blocks;
    p.temperature = sp->temperature;
    p.top_p = sp->top_p;
    p.top_k = sp->top_k;
    p.rng = c->smp_rng;
    p.token_out = c->smp_tok;
    const bool few = sp->top_k >= 1 && sp->top_k <= 64 && smp_supported(V);
    if (few) {
        HIP_TRY(c, launch_sample(logits, p, s));
    } else {
        const uint32_t k = sp->top_k > 0 ? std::min<uint32_t>(sp->top_k, V) : V;
        const uint32_t ns = smp_sort_keys(V);
        const uint64_t bytes = (uint64_t)ns * 16 + (uint64_t)V * 4;
        if (bytes > c->smp_sort_bytes) {
            HIP_TRY(c, hipStreamSynchronize(c->stream));
            if (c->smp_sort) (void)hipFree(c->smp_sort);
            c->smp_sort = nullptr;
            c->smp_sort_bytes = 0;
            if (int rc = dalloc(c, bytes, &c->smp_sort)) return rc;
            c->smp_sort_bytes = bytes;
        }
        p.sort_a = (unsigned long long*)c->smp_sort;
        p.sort_b = p.sort_a + ns;
        p.n_sort = ns;
        p.probs = (float*)(p.sort_b + ns);
        HIP_TRY(c, launch_sample_sorted(logits, p, k, s));
    }
    if (ho) {
        // the token word, stored last by the kernel; after 200 ms without it
        // (a failed launch, a fault) the stream is synchronised and its error
        // reported
        const auto t0 = std::chrono::steady_clock::now();
        bool seen = false;
        for (uint32_t i = 1; !seen; ++i) {
            seen = ho[0] != kTokPending;
            if (!seen && (i & 1023u) == 0 && std::chrono::steady_clock::now() - t0 > std::chrono::milliseconds(200))
                break;
        }
        if (!seen) {
            HIP_TRY(c, hipStreamSynchronize(s));
            if (ho[0] == kTokPending) return fail(c, QORA_HIP_E_DEVICE, "sampling kernel did not store its token");
        }
        *token = (uint32_t)ho[0];
        *rng_state = (uint64_t)(uint32_t)ho[2] | ((uint64_t)(uint32_t)ho[3] << 32);
        return QORA_HIP_OK;
    }
    HIP_TRY(c, hipMemcpyAsync(&c->h_pin[20], c->smp_tok, 4, hipMemcpyDeviceToHost, s));
    HIP_TRY(c, hipMemcpyAsync(&c->h_pin[22], c->smp_rng, 8, hipMemcpyDeviceToHost, s));
    HIP_TRY(c, hipStreamSynchronize(s));
    *token = (uint32_t)c->h_pin[20];
    std::memcpy(rng_state, &c->h_pin[22], 8);
    return QORA_HIP_OK;
}

}  // namespace

extern "C" int qora_hip_sample(qora_hip_ctx* c, const float* logits, uint64_t vocab, const uint32_t* history,
                               uint64_t n_history, const qora_sample_params* params, uint64_t* rng_state,
                               uint32_t* token, void* stream) {
    if (!c) return QORA_HIP_E_INVALID;
    return sample_device(c, logits, vocab, history, n_history, params, rng_state, token, pick_stream(c, stream));
}

extern "C" int qora_hip_decode_sample(qora_hip_ctx* c, uint32_t token, const uint32_t* history, uint64_t n_history,
                                      const qora_sample_params* params, uint64_t* rng_state, float* logits,
                                      uint32_t* token_out) {
    if (!c) return QORA_HIP_E_INVALID;
    if (int rc = check_step_room(c, 1)) return rc;
    ModelState& m = c->m;
    if (token >= m.vocab) return fail(c, QORA_HIP_E_INVALID, "token id out of range");
    // every argument is checked before the step is launched, so a refused call
    // leaves the cache and the stream as they were
    if (int rc = sample_check(c, true, m.vocab, history, n_history, params, rng_state, token_out)) return rc;
    if (force_fail("launch")) return fail(c, QORA_HIP_E_DEVICE, "forced launch failure (QORA_HIP_FORCE_FAIL=launch)");
    if (int rc = put_token(c, token)) return rc;
    if (int rc = launch_step(c, true, m.host_pos)) {
        (void)hipStreamSynchronize(c->stream);
        return rc;
    }
    if (logits) {
        uint32_t greedy = 0;
        if (int rc = finish_step(c, logits, &greedy)) return rc;
    } else {
        // no wait here: the sampling kernels follow the step on the stream, and
        // the host builds the penalty list while the step runs
        m.dev_token = -1;
    }
    m.host_pos += 1;
    const int rc =
        sample_device(c, m.d_logits, m.vocab, history, n_history, params, rng_state, token_out, c->stream, m.d_token);
    if (rc) {
        // nothing of this call stays in flight behind an error
        (void)hipStreamSynchronize(c->stream);
        m.dev_token = -1;
        return rc;
    }
    m.dev_token = (int64_t)*token_out;   // the sampling kernel stored it as the next step's input
    if (!logits) {
        // The step's range flag (finish_step reads it when logits are asked
        // for). The sampling kernels ran after the step's argmax_finish_kernel,
        // which stored the flag to the mapped word before them (system-scope
        // fence), so the flag is in place once the sampled token is.
        int32_t bad;
        if (c->d_h_tok) {
            bad = reinterpret_cast<volatile int32_t*>(c->h_tok)[1];
        } else {
            HIP_TRY(c, hipMemcpyAsync(&c->h_pin[17], m.d_range, 4, hipMemcpyDeviceToHost, c->stream));
            HIP_TRY(c, hipStreamSynchronize(c->stream));
            bad = c->h_pin[17];
        }
        if (bad) return range_error(c);
    }
    return QORA_HIP_OK;
}

extern "C" int qora_hip_argmax(qora_hip_ctx* c, const float* logits, uint64_t n, int32_t* out, void* stream) {
    if (!c) return QORA_HIP_E_INVALID;
    if (!logits || !out) return fail(c, QORA_HIP_E_INVALID, "null argument");
    if (n == 0 || n > 0x7FFFFFFFull) return fail(c, QORA_HIP_E_INVALID, "bad length");
    HIP_TRY(c, launch_argmax(logits, (uint32_t)n, out, pick_stream(c, stream)));
    return QORA_HIP_OK;
}
