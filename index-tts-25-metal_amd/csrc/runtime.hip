// Host runtime of the GPT semantic-token loop and its C ABI (include/itts_gpt.h).
//
// One itts_gpt handle = resident weights + KV cache slots + one HIP stream.
//   * weights: Conv1D matrices [in][out] are transposed on the device into one slab,
//     row-major [out][in], in consumption order (per layer: c_attn, c_proj, c_fc,
//     mlp.c_proj; then mel_head), fp32 or bf16 (gpt.cpp:24-37 does this on the host);
//   * KV cache: [slot][layer][K|V][head][row][64] fp32, `kv_capacity` rows per slot
//     (gptKvCacheCreate, metal_context.mm:5675-5700, uses [layer][K|V][row][1280]);
//   * decode: the 24-layer step (5 kernels per layer + head, + sampler) is captured once
//     per batch bucket as a hipGraph and replayed per token.  Token, position and KV
//     length live in device SeqState; the sampler advances them, so generate() replays
//     the graph with no per-token host work (the reference blocks per token:
//     gpt.cpp:123 / metal_context.mm:4613-4630).
#include <algorithm>
#include <atomic>
#include <chrono>
#include <cmath>
#include <cstdlib>
#include <cstring>
#include <map>
#include <memory>
#include <mutex>
#include <stdexcept>
#include <string>
#include <thread>
#include <tuple>
#include <unordered_map>
#include <vector>

#include "itts_gpt.h"
#include "kernels.h"

namespace itts {
namespace {

thread_local std::string g_create_error;

#define HIP_CHECK(x)                                                                                         \
    do {                                                                                                     \
        const hipError_t e_ = (x);                                                                           \
        if (e_ != hipSuccess) throw std::runtime_error(std::string("HIP error ") + hipGetErrorString(e_) + " in " #x); \
    } while (0)

// Every device or pinned allocation and every graph instantiation this file makes, counted
// process-wide (itts_gpt_alloc_events): the check that an entry point allocates nothing.
std::atomic<uint64_t> g_alloc_events{0};

template <class T>
struct DevBuf {
    T* p = nullptr;
    size_t n = 0;
    DevBuf() = default;
    DevBuf(const DevBuf&) = delete;
    DevBuf& operator=(const DevBuf&) = delete;
    ~DevBuf() { reset(); }
    void reset() {
        if (p) (void)hipFree(p);
        p = nullptr;
        n = 0;
    }
    void alloc(size_t count) {
        reset();
        if (count) {
            g_alloc_events.fetch_add(1, std::memory_order_relaxed);
            HIP_CHECK(hipMalloc(&p, count * sizeof(T)));
        }
        n = count;
    }
    void ensure(size_t count) {
        if (count > n) alloc(count);
    }
};

struct HostTensor {
    const float* data;
    std::vector<int64_t> shape;
};

// Status codes written by the sampler (sampler.hip).
const char* sampler_message(uint32_t s) {
    switch (s) {
        case 1: return "GPT top_p filtering removed all logits";
        case 2: return "GPT sampling probability mass is zero";
        case 3: return "GPT sampling received no finite logits";
        case 4: return "GPT generated invalid semantic code";
        default: return "GPT sampler failed";
    }
}

struct Snapshot {
    uint32_t tokens = 0;
    DevBuf<float> kv;
};

// A persistent step grid takes one workgroup slot on every CU and needs all of its
// workgroups resident together.  Two such grids running at once on one GPU (decoders of
// this process on different streams) could each hold CUs the other is waiting for, so
// while more than one decoder on a device can launch them, the launches are chained: each
// waits for the previous one, whichever decoder made it.  With one such decoder the chain
// is skipped (its marker packets cost about 3 us per token).  A decoder that registers as
// the second one drains the device first, so no unchained grid is still running when
// chained launches begin; a decoder drains its own stream before it unregisters.
// The chain is process-wide and never freed.
std::mutex g_step_mu;
std::unordered_map<int, int> g_step_users;          // device -> decoders that launch persistent grids
std::unordered_map<int, hipEvent_t> g_step_last;    // device -> recorded after its latest chained launch

void register_step_user(int dev) {
    int users = 0;
    {
        std::lock_guard<std::mutex> lock(g_step_mu);
        users = ++g_step_users[dev];
    }
    if (users == 2) HIP_CHECK(hipDeviceSynchronize());
}
void unregister_step_user(int dev) {
    std::lock_guard<std::mutex> lock(g_step_mu);
    --g_step_users[dev];
}

hipError_t launch_step_serialized(const StepArgs& a, int nseq, int grid, bool bf16, int dev, hipStream_t s) {
    std::lock_guard<std::mutex> lock(g_step_mu);
    if (g_step_users[dev] <= 1) return nseq == 1 ? launch_step(a, grid, bf16, s) : launch_step_batch(a, nseq, grid, s);
    auto& last = g_step_last;
    auto it = last.find(dev);
    if (it == last.end()) {
        hipEvent_t e = nullptr;
        const hipError_t err = hipEventCreateWithFlags(&e, hipEventDisableTiming);
        if (err != hipSuccess) return err;
        it = last.emplace(dev, e).first;
    } else {
        const hipError_t err = hipStreamWaitEvent(s, it->second, 0);
        if (err != hipSuccess) return err;
    }
    const hipError_t err = nseq == 1 ? launch_step(a, grid, bf16, s) : launch_step_batch(a, nseq, grid, s);
    if (err != hipSuccess) return err;
    return hipEventRecord(it->second, s);
}

// ---------------------------------------------------------------- scratch of generate_noalloc
// itts_gpt_generate_noalloc takes the prefill's activations (which itts_gpt_generate grows
// with hipMalloc as prefixes get longer) from this file-scope device array instead, so the
// call allocates nothing.  Layout for M <= kNoAllocRows prefix rows, every part 256-B aligned:
//   x, xn, q, att [kNoAllocRows][1280] f32; ff [kNoAllocRows][5120] f32;
//   row_slot, row_pos [kNoAllocRows] u32; last_rows [64] u32; the split-K GEMM workspace
//   (kGemmWsFloats f32).
// Each GPU holds its own copy (28 MiB) until the process ends.  Host code never passes the
// array's name to a kernel: it is a host-side stand-in there.  The device address, per
// device, comes from hipGetSymbolAddress at decoder creation (scratch_address below).
constexpr uint32_t kNoAllocRows = 512;
constexpr size_t kScratchActBytes = size_t(kNoAllocRows) * kWidth * 4;
constexpr size_t kScratchOffX = 0;
constexpr size_t kScratchOffXn = kScratchOffX + kScratchActBytes;
constexpr size_t kScratchOffQ = kScratchOffXn + kScratchActBytes;
constexpr size_t kScratchOffAtt = kScratchOffQ + kScratchActBytes;
constexpr size_t kScratchOffFf = kScratchOffAtt + kScratchActBytes;
constexpr size_t kScratchOffSlot = kScratchOffFf + size_t(kNoAllocRows) * kFfn * 4;
constexpr size_t kScratchOffPos = kScratchOffSlot + size_t(kNoAllocRows) * 4;
constexpr size_t kScratchOffLast = kScratchOffPos + size_t(kNoAllocRows) * 4;
constexpr size_t kScratchOffWs = kScratchOffLast + 64 * 4;
constexpr size_t kScratchBytes = kScratchOffWs + kGemmWsFloats * 4;
static_assert(kScratchOffXn % 256 == 0 && kScratchOffFf % 256 == 0 && kScratchOffSlot % 256 == 0 &&
                  kScratchOffPos % 256 == 0 && kScratchOffLast % 256 == 0 && kScratchOffWs % 256 == 0 && kMaxBatch <= 64,
              "scratch parts must stay 256-B aligned");

static __device__ __align__(256) uint8_t scratch[kScratchBytes];

// Per device: the address of `scratch` there, and a lock that serialises the no-alloc calls
// of this process on that device (they share the one array).  Filled once per device.
struct ScratchEntry {
    uint8_t* ptr = nullptr;
    std::string error;
    std::unique_ptr<std::mutex> lock;
};
std::mutex g_scratch_mu;
std::unordered_map<int, ScratchEntry> g_scratch;

// Looks `scratch` up on device `dev`, which must be current.  A failure is recorded, not
// thrown: only itts_gpt_generate_noalloc needs the address, and it reports the error.
ScratchEntry* scratch_entry(int dev) {
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    auto it = g_scratch.find(dev);
    if (it != g_scratch.end()) return &it->second;
    ScratchEntry e;
    void* p = nullptr;
    const hipError_t err = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (err != hipSuccess || !p)
        e.error = std::string("hipGetSymbolAddress(scratch) failed: ") + hipGetErrorString(err);
    else
        e.ptr = static_cast<uint8_t*>(p);
    e.lock = std::make_unique<std::mutex>();
    return &g_scratch.emplace(dev, std::move(e)).first->second;
}

}  // namespace

// Device buffers of one prefill (enqueue_prefill_layers).
struct PrefillBufs {
    float *x, *xn, *q, *att, *ff;
    uint32_t *row_slot, *row_pos, *last_rows;
    float* ws;  // split-K workspace, kGemmWsFloats
};

struct Engine {
    // ---------------------------------------------------------------- model
    int layers = 0;
    uint32_t text_vocab = 0, text_pos_rows = 0, lang_vocab = 0, mel_pos_rows = 0;
    bool bf16 = false;
    uint32_t cap = 4096, max_batch = 1;
    DevBuf<uint8_t> slab;  // GEMV weights
    size_t elt = 4;
    std::vector<size_t> off_qkv, off_proj, off_fc, off_fc2;  // element offsets
    size_t off_head = 0;
    DevBuf<float> params, head_params, text_emb, text_pos, lang_emb, mel_emb, mel_pos, spk_w, spk_b;
    bool has_speaker = false;

    // ---------------------------------------------------------------- sequences
    hipStream_t stream = nullptr;
    DevBuf<float> kv;
    size_t kv_slot_stride = 0, kv_layer_stride = 0, kv_v_off = 0;
    DevBuf<float> h, hmid, q, attn, ff, logits, partial;
    DevBuf<float> xn;  // LayerNorm'd GEMV inputs of a batched step, [kMaxBatch][1280]
    DevBuf<uint32_t> codes, status, d_parent;
    DevBuf<SeqState> state;  // kMaxBatch + 1 entries; the last one serves the processor/sampler API
    DevBuf<uint8_t> seen, seen_tmp, table, table_tmp;
    DevBuf<float> seg_cond;     // conditioning rows shared by a request's segments
    DevBuf<uint32_t> seg_ids;   // the segments' wrapped text ids
    DevBuf<double> probs;
    // prefill scratch
    DevBuf<float> px, pxn, pq, patt, pff, pws;
    DevBuf<uint32_t> row_slot, row_pos, last_rows;
    // beam search scratch
    DevBuf<float> beam_scores, all_scores;
    DevBuf<uint32_t> beam_list, d_token;
    DevBuf<double> beam_probs;
    DevBuf<BeamCand> cand;
    DevBuf<uint64_t> beam_rng;
    DevBuf<uint32_t> beam_np;    // the step's parent count, advanced by beam_advance_kernel
    DevBuf<SeqState> beam_tmpl;  // decode state of a child, before its n, position and token
    // Candidates and statuses of a queued beam step, written into pinned memory by
    // beam_select_kernel; the host runs up to kBeamLag steps behind the device.
    struct BeamSlot {
        BeamCand cand[kMaxBeamTake];
        uint32_t status[1 + kMaxBatch];
    };
    static constexpr uint32_t kBeamRing = 4, kBeamLag = 2;
    BeamSlot* beam_ring = nullptr;
    BeamSlot* beam_ring_dev = nullptr;  // beam_ring as the device addresses it
    hipEvent_t bev[kBeamRing] = {};
    // API scratch
    DevBuf<float> api_out;
    DevBuf<uint32_t> api_tokens;
    uint32_t* pinned = nullptr;  // host pinned staging (flags)
    SeqState* pinned_state = nullptr;
    int splits = 16;
    bool use_graphs = true;  // ITTS_GPT_GRAPHS=0: launch the same kernels eagerly (profilers)
    // Persistent single-sequence step (step.hip): one launch per token for batch-1 decode
    // (bitwise the same logits as the multi-kernel path, which ITTS_GPT_PERSISTENT=0 selects).
    bool step_ok = false;
    bool step_batch_ok[kStepBatchMax + 1] = {};  // persistent batch step available for this many sequences
    uint32_t beam_slots = 0;                     // slots the beam row-owner table may name (this search's beams)
    int step_grid = 0;
    int step_dev = 0;
    size_t per_layer = 0;       // weight elements per layer block
    DevBuf<uint64_t> xch;       // tagged exchange slots
    DevBuf<uint32_t> step_err;  // hand-off timeout flag
    // ITTS_GPT_FUSED_SAMPLER=1: batch-1 decode steps sample the next token in the step
    // kernel's fused tail (one launch per token).  Off by default: the tail runs the sampler on
    // the step kernel's 512 threads, and a separate 1024-thread sampler launch measured faster
    // (1526 against 1509 tokens/s on the 600-code workload), the same codes either way.
    bool fused_sampling = false;
    DevBuf<uint32_t> step_tail;  // workgroups past their mel_head rows in the running step (0 between)
    uint32_t epoch = 8;         // tag base of the next launch
    std::map<std::tuple<int, int, bool, bool>, hipGraphExec_t> graphs;
    hipEvent_t ev[4] = {};
    uint32_t cached = 0;
    itts_gpt_timing timing{};
    std::string last_error;
    // itts_gpt_generate_noalloc: this device's `scratch` entry (address or lookup error), and
    // whether the call in progress must not allocate (no graph capture, no buffer growth).
    ScratchEntry* scratch_dev = nullptr;
    bool no_alloc_call = false;

    ~Engine() {
        // Queued work may still write this handle's buffers (a beam search that raised with
        // later steps in flight copies into the pinned ring), and no persistent grid of this
        // decoder may outlive its registration: drain the stream before anything is freed.
        if (stream) (void)hipStreamSynchronize(stream);
        if (step_ok) unregister_step_user(step_dev);
        for (auto& kvp : graphs) (void)hipGraphExecDestroy(kvp.second);
        for (auto& e : ev)
            if (e) (void)hipEventDestroy(e);
        for (auto& e : bev)
            if (e) (void)hipEventDestroy(e);
        if (beam_ring) (void)hipHostFree(beam_ring);
        if (pinned) (void)hipHostFree(pinned);
        if (pinned_state) (void)hipHostFree(pinned_state);
        if (stream) (void)hipStreamDestroy(stream);
    }

    void* w_ptr(size_t off) const { return slab.p + off * elt; }
    size_t kv_layer_off(int l) const { return static_cast<size_t>(l) * kv_layer_stride; }

    // ---------------------------------------------------------------- construction
    // Stream, events and the sampler/processor buffers (all a sampler-only handle needs).
    void init_common() {
        HIP_CHECK(hipStreamCreateWithFlags(&stream, hipStreamNonBlocking));
        for (auto& e : ev) HIP_CHECK(hipEventCreate(&e));
        g_alloc_events.fetch_add(2, std::memory_order_relaxed);
        HIP_CHECK(hipHostMalloc(&pinned, 64 * sizeof(uint32_t), hipHostMallocDefault));
        HIP_CHECK(hipHostMalloc(&pinned_state, (kMaxBatch + 1) * sizeof(SeqState), hipHostMallocDefault));
        const size_t B = kMaxBatch;
        logits.alloc((B + 1) * kMelVocab);
        status.alloc(B + 1);
        state.alloc(B + 1);
        HIP_CHECK(hipMemsetAsync(state.p, 0, state.n * sizeof(SeqState), stream));
        seen.alloc((B + 1) * kMelVocab);
        probs.alloc((B + 1) * kMelVocab);
        api_out.alloc(kMelVocab);
        api_tokens.alloc(1 << 16);
        HIP_CHECK(hipStreamSynchronize(stream));
    }

    void create(const itts_tensor* tensors, int32_t count, const itts_gpt_config* cfg) {
        if (const char* g = std::getenv("ITTS_GPT_GRAPHS")) use_graphs = std::strcmp(g, "0") != 0;
        init_common();
        if (count == 0) return;  // sampler-only handle
        std::unordered_map<std::string, HostTensor> by;
        for (int32_t i = 0; i < count; ++i)
            by[tensors[i].name] = HostTensor{tensors[i].data, std::vector<int64_t>(tensors[i].shape, tensors[i].shape + tensors[i].ndim)};
        auto info = [&](const std::string& name) -> const HostTensor& {
            auto it = by.find(name);
            if (it == by.end()) throw std::runtime_error("Missing tensor: " + name);
            return it->second;
        };
        // gpt.cpp:9-11: shape checks; vocabulary/position table sizes come from the tensors.
        auto check = [&](const std::string& name, const std::vector<int64_t>& shape) -> const float* {
            const auto& t = info(name);
            if (t.shape != shape) throw std::runtime_error("Unsupported 2.5 GPT shape: " + name);
            return t.data;
        };
        auto rows_of = [&](const std::string& name) -> uint32_t {
            const auto& t = info(name);
            if (t.shape.size() != 2 || t.shape[1] != kWidth || t.shape[0] <= 0)
                throw std::runtime_error("Unsupported 2.5 GPT shape: " + name);
            return static_cast<uint32_t>(t.shape[0]);
        };
        cap = cfg && cfg->kv_capacity ? cfg->kv_capacity : 4096;
        max_batch = cfg && cfg->max_batch ? cfg->max_batch : 1;
        bf16 = cfg && cfg->weight_dtype == ITTS_WEIGHTS_BF16;
        if (cfg && cfg->weight_dtype > ITTS_WEIGHTS_BF16) throw std::invalid_argument("Unknown weight dtype");
        if (max_batch > static_cast<uint32_t>(kMaxBatch)) throw std::invalid_argument("max_batch exceeds 10");
        if (cap < 2 || cap > 65536) throw std::invalid_argument("Invalid KV capacity");
        elt = bf16 ? 2 : 4;

        text_vocab = rows_of("gpt.text_embedding.weight");
        text_pos_rows = rows_of("gpt.text_pos_embedding.emb.weight");
        lang_vocab = rows_of("gpt.lang_embedding.weight");
        mel_pos_rows = rows_of("gpt.mel_pos_embedding.emb.weight");
        check("gpt.mel_embedding.weight", {kMelVocab, kWidth});
        has_speaker = by.count("gpt.spk_emb_proj.weight") != 0;
        if (has_speaker) check("gpt.spk_emb_proj.weight", {kWidth, 192});
        while (by.count("gpt.gpt.h." + std::to_string(layers) + ".attn.c_attn.weight")) ++layers;
        if (!layers) throw std::runtime_error("Missing tensor: gpt.gpt.h.0.attn.c_attn.weight");

        // Weight slab.
        per_layer = static_cast<size_t>(kQkv) * kWidth + static_cast<size_t>(kWidth) * kWidth + 2 * static_cast<size_t>(kFfn) * kWidth;
        const size_t total = per_layer * layers + static_cast<size_t>(kMelVocab) * kWidth;
        slab.alloc(total * elt);
        DevBuf<float> staging;
        staging.alloc(static_cast<size_t>(kMelVocab) * kWidth);
        auto upload = [&](const float* src, size_t n, float* dst) {
            HIP_CHECK(hipMemcpyAsync(dst, src, n * 4, hipMemcpyHostToDevice, stream));
        };
        auto put_conv = [&](const std::string& name, int in, int out, size_t off) {
            const float* src = check(name, {in, out});
            upload(src, static_cast<size_t>(in) * out, staging.p);
            HIP_CHECK(launch_transpose(staging.p, w_ptr(off), in, out, bf16, stream));
            HIP_CHECK(hipStreamSynchronize(stream));  // staging is reused
        };
        params.alloc(static_cast<size_t>(layers) * kParLayer);
        std::vector<float> par(static_cast<size_t>(layers) * kParLayer);
        size_t off = 0;
        for (int l = 0; l < layers; ++l) {
            const std::string p = "gpt.gpt.h." + std::to_string(l);
            off_qkv.push_back(off);
            put_conv(p + ".attn.c_attn.weight", kWidth, kQkv, off);
            off += static_cast<size_t>(kQkv) * kWidth;
            off_proj.push_back(off);
            put_conv(p + ".attn.c_proj.weight", kWidth, kWidth, off);
            off += static_cast<size_t>(kWidth) * kWidth;
            off_fc.push_back(off);
            put_conv(p + ".mlp.c_fc.weight", kWidth, kFfn, off);
            off += static_cast<size_t>(kFfn) * kWidth;
            off_fc2.push_back(off);
            put_conv(p + ".mlp.c_proj.weight", kFfn, kWidth, off);
            off += static_cast<size_t>(kFfn) * kWidth;
            float* dst = &par[static_cast<size_t>(l) * kParLayer];
            auto cp = [&](const std::string& name, int n, int at) { std::memcpy(dst + at, check(name, {n}), n * 4); };
            cp(p + ".ln_1.weight", kWidth, kParLn1W);
            cp(p + ".ln_1.bias", kWidth, kParLn1B);
            cp(p + ".attn.c_attn.bias", kQkv, kParQkvB);
            cp(p + ".attn.c_proj.bias", kWidth, kParProjB);
            cp(p + ".ln_2.weight", kWidth, kParLn2W);
            cp(p + ".ln_2.bias", kWidth, kParLn2B);
            cp(p + ".mlp.c_fc.bias", kFfn, kParFcB);
            cp(p + ".mlp.c_proj.bias", kWidth, kParFc2B);
        }
        off_head = off;
        upload(check("gpt.mel_head.weight", {kMelVocab, kWidth}), static_cast<size_t>(kMelVocab) * kWidth, staging.p);
        HIP_CHECK(launch_convert(staging.p, w_ptr(off_head), static_cast<size_t>(kMelVocab) * kWidth, bf16, stream));
        HIP_CHECK(hipStreamSynchronize(stream));
        upload(par.data(), par.size(), params.p);
        std::vector<float> hp(kHeadPar);
        std::memcpy(&hp[kHeadLnfW], check("gpt.gpt.ln_f.weight", {kWidth}), kWidth * 4);
        std::memcpy(&hp[kHeadLnfB], check("gpt.gpt.ln_f.bias", {kWidth}), kWidth * 4);
        std::memcpy(&hp[kHeadFnW], check("gpt.final_norm.weight", {kWidth}), kWidth * 4);
        std::memcpy(&hp[kHeadFnB], check("gpt.final_norm.bias", {kWidth}), kWidth * 4);
        std::memcpy(&hp[kHeadBias], check("gpt.mel_head.bias", {kMelVocab}), kMelVocab * 4);
        head_params.alloc(kHeadPar);
        upload(hp.data(), hp.size(), head_params.p);
        auto table_up = [&](DevBuf<float>& d, const std::string& name, uint32_t rows) {
            d.alloc(static_cast<size_t>(rows) * kWidth);
            upload(info(name).data, d.n, d.p);
        };
        table_up(text_emb, "gpt.text_embedding.weight", text_vocab);
        table_up(text_pos, "gpt.text_pos_embedding.emb.weight", text_pos_rows);
        table_up(lang_emb, "gpt.lang_embedding.weight", lang_vocab);
        table_up(mel_emb, "gpt.mel_embedding.weight", kMelVocab);
        table_up(mel_pos, "gpt.mel_pos_embedding.emb.weight", mel_pos_rows);
        if (has_speaker) {
            spk_w.alloc(static_cast<size_t>(kWidth) * 192);
            upload(info("gpt.spk_emb_proj.weight").data, spk_w.n, spk_w.p);
            spk_b.alloc(kWidth);
            upload(check("gpt.spk_emb_proj.bias", {kWidth}), kWidth, spk_b.p);
        }

        // KV cache and decode buffers.
        kv_layer_stride = 2ull * kHeads * cap * kHeadDim;
        kv_v_off = static_cast<size_t>(kHeads) * cap * kHeadDim;
        kv_slot_stride = kv_layer_stride * layers;
        kv.alloc(kv_slot_stride * max_batch);
        const size_t B = kMaxBatch;
        h.alloc(B * kWidth);
        hmid.alloc(B * kWidth);
        q.alloc(B * kWidth);
        attn.alloc(B * kWidth);
        ff.alloc(B * kFfn);
        xn.alloc(B * kWidth);
        // Enough splits that no split exceeds kAttnMaxChunk rows at full capacity.
        splits = std::max<int>((cap + kAttnSplitRows - 1) / kAttnSplitRows, (cap + kAttnMaxChunk - 1) / kAttnMaxChunk);
        splits = std::min(splits, kAttnMaxSplits);
        if (static_cast<uint32_t>(splits) * kAttnMaxChunk < cap) throw std::invalid_argument("KV capacity exceeds attention splits");
        partial.alloc(B * kHeads * splits * 68);
        codes.alloc((B + 1) * cap);
        d_parent.alloc(B);
        seen_tmp.alloc((B + 1) * kMelVocab);
        table.alloc(B * cap);
        table_tmp.alloc(B * cap);
        init_step();
        int dev = 0;
        HIP_CHECK(hipGetDevice(&dev));
        scratch_dev = scratch_entry(dev);
        HIP_CHECK(hipStreamSynchronize(stream));
    }

    // The persistent step runs when one 512-thread workgroup fits per CU (the grid is one
    // workgroup per CU, all resident together), there is a workgroup per attention head
    // (step_fits: head h's merge runs on workgroup h), weights are FP32 and the cache holds
    // at most 4096 rows (at most 32 splits, kAttnMaxChunk rows each).
    void init_step() {
        const char* pe = std::getenv("ITTS_GPT_PERSISTENT");
        if ((pe && std::strcmp(pe, "0") == 0) || bf16 || cap > 4096) return;
        int dev = 0, cus = 0, occ = 0;
        HIP_CHECK(hipGetDevice(&dev));
        step_dev = dev;
        HIP_CHECK(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev));
        HIP_CHECK(step_occupancy(false, &occ));
        if (occ < 1 || !step_fits(cus)) return;
        // Batches and beams of 2..4 sequences in one launch (step_batch.hip) only when
        // ITTS_GPT_PERSISTENT_BATCH=1: the multi-kernel path's batched GEMVs (five-wave
        // workgroups, LayerNorms formed in the GEMV) measure as fast at 2 sequences and faster
        // from 3 on (3: 932 against 1015 us per step, 4: 1036 against 1207; beam-3 3070
        // against 2824 beam tokens/s), with bitwise the same logits.
        const char* pb = std::getenv("ITTS_GPT_PERSISTENT_BATCH");
        const bool batch = max_batch >= 2 && pb && std::strcmp(pb, "1") == 0;
        for (int nb = 2; batch && nb <= kStepBatchMax; ++nb) {
            int bocc = 0;
            HIP_CHECK(step_batch_occupancy(nb, &bocc));
            step_batch_ok[nb] = bocc >= 1 && step_batch_fits(cus, nb);
        }
        xch.alloc(kStepExchangeTotal * (batch ? kStepBatchMax : 1));
        HIP_CHECK(hipMemsetAsync(xch.p, 0, xch.n * sizeof(uint64_t), stream));
        step_err.alloc(1);
        HIP_CHECK(hipMemsetAsync(step_err.p, 0, sizeof(uint32_t), stream));
        step_tail.alloc(1);
        HIP_CHECK(hipMemsetAsync(step_tail.p, 0, sizeof(uint32_t), stream));
        const char* fs = std::getenv("ITTS_GPT_FUSED_SAMPLER");
        fused_sampling = fs && std::strcmp(fs, "1") == 0;
        step_grid = cus;
        register_step_user(dev);
        step_ok = true;
    }

    // Arguments of one persistent step launch for sequences q0 .. q0 + nq - 1 (slots, states and
    // logits rows from q0; each launch takes its own range of tags).
    StepArgs step_args(int q0 = 0, int nq = 1) {
        // Each launch takes a fresh range of 8*(layers+1) tags; before the 32-bit counter
        // wraps, the exchange is cleared and numbering restarts.
        const uint32_t span = 8u * static_cast<uint32_t>(layers + 1);
        if (epoch > 0xF0000000u - span) {
            HIP_CHECK(hipMemsetAsync(xch.p, 0, xch.n * sizeof(uint64_t), stream));
            epoch = 8;
        }
        StepArgs s{};
        s.w = slab.p;
        s.layer_stride = per_layer;
        s.off_head = off_head;
        s.params = params.p;
        s.head = head_params.p;
        s.mel_emb = mel_emb.p;
        s.mel_pos = mel_pos.p;
        s.kv = kv.p + static_cast<size_t>(q0) * kv_slot_stride;
        s.kv_layer_stride = kv_layer_stride;
        s.kv_v_off = kv_v_off;
        s.kv_cap = cap;
        s.layers = layers;
        s.splits = splits;
        s.state = state.p + q0;
        s.xch = xch.p;
        s.logits = logits.p + static_cast<size_t>(q0) * kMelVocab;
        s.epoch = epoch;
        s.err = step_err.p;
        s.nseq = nq;
        s.kv_slot_stride = kv_slot_stride;
        s.logit_stride = kMelVocab;
        epoch += span;
        return s;
    }

    // Raises (and clears) a hand-off timeout reported by the persistent step; call after a sync.
    void check_step_error() {
        if (!step_ok) return;
        uint32_t e = 0;
        HIP_CHECK(hipMemcpy(&e, step_err.p, sizeof(e), hipMemcpyDeviceToHost));
        if (e) {
            HIP_CHECK(hipMemset(step_err.p, 0, sizeof(uint32_t)));
            throw std::runtime_error("GPT decode step: a workgroup hand-off timed out");
        }
    }
    // The persistent path takes one sequence (step.hip) or, when enabled (init_step),
    // 2..kStepBatchMax in one launch (step_batch.hip; with the beam row-owner table when every
    // slot it may name is below kStepBatchMax).  Other batches take the multi-kernel path,
    // whose batched GEMVs read the weights once for all of them.
    bool persistent(int nseq, bool use_table) const {
        if (!step_ok || nseq < 1 || nseq > kStepBatchMax) return false;
        if (use_table) return nseq >= 2 && step_batch_ok[nseq] && beam_slots <= static_cast<uint32_t>(kStepBatchMax);
        return nseq == 1 || step_batch_ok[nseq];
    }
    // fuse_sampler: the single-sequence step kernel also samples the next token (its tail).
    void launch_persistent(int nseq, bool use_table, bool fuse_sampler = false) {
        StepArgs s = step_args(0, nseq);
        s.table = use_table ? table.p : nullptr;
        if (fuse_sampler) {
            s.tail = step_tail.p;
            s.sample = sample_base(kModeDecode);
        }
        HIP_CHECK(launch_step_serialized(s, nseq, step_grid, bf16, step_dev, stream));
    }

    // ---------------------------------------------------------------- forward pieces
    GemvArgs gemv_base(int nseq) const {
        GemvArgs a{};
        a.state = state.p;
        a.nseq = nseq;
        a.kv = kv.p;
        a.kv_slot_stride = kv_slot_stride;
        a.kv_v_off = kv_v_off;
        a.kv_cap = cap;
        a.xn = xn.p;
        return a;
    }

    // One decode step for sequences 0..nseq-1 (state-driven), padded to batch bucket nb.
    void enqueue_forward(int nseq, int nb, bool use_table) {
        for (int l = 0; l < layers; ++l) {
            const float* par = params.p + static_cast<size_t>(l) * kParLayer;
            GemvArgs a = gemv_base(nseq);
            a.w = w_ptr(off_qkv[l]);
            a.bias = par + kParQkvB;
            a.rows = kQkv;
            a.x = h.p;
            a.x_stride = kWidth;
            a.ln_w = par + kParLn1W;
            a.ln_b = par + kParLn1B;
            a.q = q.p;
            a.kv_layer_off = kv_layer_off(l);
            a.mel_emb = mel_emb.p;
            a.mel_pos = mel_pos.p;
            a.h_out = h.p;
            HIP_CHECK(launch_gemv_qkv(a, nb, bf16, l == 0, stream));

            AttnArgs t{};
            t.q = q.p;
            t.kv = kv.p;
            t.kv_slot_stride = kv_slot_stride;
            t.kv_layer_off = kv_layer_off(l);
            t.kv_v_off = kv_v_off;
            t.kv_cap = cap;
            t.table = use_table ? table.p : nullptr;
            t.partial = partial.p;
                        t.out = attn.p;
            t.state = state.p;
            t.nseq = nseq;
            t.splits = splits;
            HIP_CHECK(launch_attention(t, nb, stream));

            GemvArgs p = gemv_base(nseq);
            p.w = w_ptr(off_proj[l]);
            p.bias = par + kParProjB;
            p.rows = kWidth;
            p.x = attn.p;
            p.x_stride = kWidth;
            p.resid = h.p;
            p.out = hmid.p;
            p.out_stride = kWidth;
            HIP_CHECK(launch_gemv_proj(p, nb, bf16, stream));

            GemvArgs f = gemv_base(nseq);
            f.w = w_ptr(off_fc[l]);
            f.bias = par + kParFcB;
            f.rows = kFfn;
            f.x = hmid.p;
            f.x_stride = kWidth;
            f.ln_w = par + kParLn2W;
            f.ln_b = par + kParLn2B;
            f.out = ff.p;
            f.out_stride = kFfn;
            HIP_CHECK(launch_gemv_fc(f, nb, bf16, stream));

            GemvArgs g = gemv_base(nseq);
            g.w = w_ptr(off_fc2[l]);
            g.bias = par + kParFc2B;
            g.rows = kWidth;
            g.x = ff.p;
            g.x_stride = kFfn;
            g.resid = hmid.p;
            g.out = h.p;
            g.out_stride = kWidth;
            HIP_CHECK(launch_gemv_fc2(g, nb, bf16, stream));
        }
        enqueue_head(nseq, nb);
    }

    void enqueue_head(int nseq, int nb) {
        GemvArgs a = gemv_base(nseq);
        a.w = w_ptr(off_head);
        a.bias = head_params.p + kHeadBias;
        a.rows = kMelVocab;
        a.x = h.p;
        a.x_stride = kWidth;
        a.ln_w = head_params.p + kHeadLnfW;
        a.ln_b = head_params.p + kHeadLnfB;
        a.ln2_w = head_params.p + kHeadFnW;
        a.ln2_b = head_params.p + kHeadFnB;
        a.out = logits.p;
        a.out_stride = kMelVocab;
        HIP_CHECK(launch_gemv_head(a, nb, bf16, stream));
    }

    SampleArgs sample_base(int mode) {
        SampleArgs s{};
        s.logits = logits.p;
        s.logit_stride = kMelVocab;
        s.state = state.p;
        s.seen = seen.p;
        s.codes = codes.p;
        s.code_stride = static_cast<int>(cap);
        s.probs = probs.p;
        s.status = status.p;
        s.mode = mode;
        return s;
    }

    // Runs one step (forward [+ sampler]) as a replay of its captured graph, or eagerly.
    void run_step(int nseq, int nb, bool sampler, bool use_table) {
        if (persistent(nseq, use_table)) {
            timing.decode_path = ITTS_PATH_STEP;
            const bool fuse = sampler && nseq == 1 && fused_sampling;
            launch_persistent(nseq, use_table, fuse);
            if (sampler && !fuse) HIP_CHECK(launch_sampler(sample_base(kModeDecode), nseq, stream));
            return;
        }
        timing.decode_path = ITTS_PATH_MULTI;
        // A call that must not allocate replays a graph only if it was captured earlier
        // (capture and instantiation allocate); otherwise it launches the same kernels eagerly.
        if (use_graphs && (!no_alloc_call || graphs.count(std::make_tuple(nseq, nb, sampler, use_table)))) {
            HIP_CHECK(hipGraphLaunch(graph(nseq, nb, sampler, use_table), stream));
            return;
        }
        enqueue_forward(nseq, nb, use_table);
        if (sampler) HIP_CHECK(launch_sampler(sample_base(kModeDecode), nseq, stream));
    }

    hipGraphExec_t graph(int nseq, int nb, bool sampler, bool use_table) {
        const auto key = std::make_tuple(nseq, nb, sampler, use_table);
        auto it = graphs.find(key);
        if (it != graphs.end()) return it->second;
        hipGraph_t g = nullptr;
        HIP_CHECK(hipStreamBeginCapture(stream, hipStreamCaptureModeThreadLocal));
        try {
            enqueue_forward(nseq, nb, use_table);
            if (sampler) HIP_CHECK(launch_sampler(sample_base(kModeDecode), nseq, stream));
        } catch (...) {
            (void)hipStreamEndCapture(stream, &g);
            if (g) (void)hipGraphDestroy(g);
            throw;
        }
        HIP_CHECK(hipStreamEndCapture(stream, &g));
        hipGraphExec_t exec = nullptr;
        g_alloc_events.fetch_add(1, std::memory_order_relaxed);
        const hipError_t e = hipGraphInstantiate(&exec, g, nullptr, nullptr, 0);
        (void)hipGraphDestroy(g);
        HIP_CHECK(e);
        graphs[key] = exec;
        return exec;
    }

    // ---------------------------------------------------------------- prefill
    // Stacked prefill of several sequences (slot b <- prefixes[b], rows[b] rows each).
    void enqueue_prefill(const std::vector<const float*>& prefixes, const std::vector<uint32_t>& rows) {
        const int nseq = static_cast<int>(prefixes.size());
        uint32_t M = 0;
        for (auto r : rows) M += r;
        px.ensure(static_cast<size_t>(M) * kWidth);
        pxn.ensure(static_cast<size_t>(M) * kWidth);
        pq.ensure(static_cast<size_t>(M) * kWidth);
        patt.ensure(static_cast<size_t>(M) * kWidth);
        pff.ensure(static_cast<size_t>(M) * kFfn);
        row_slot.ensure(M);
        row_pos.ensure(M);
        last_rows.ensure(kMaxBatch);
        pws.ensure(kGemmWsFloats);
        std::vector<uint32_t> slot(M), pos(M), last(kMaxBatch, 0);
        uint32_t m = 0;
        for (int b = 0; b < nseq; ++b) {
            // a null prefix: its rows were staged in px on the device (generate_segments)
            if (prefixes[b])
                HIP_CHECK(hipMemcpyAsync(px.p + static_cast<size_t>(m) * kWidth, prefixes[b], static_cast<size_t>(rows[b]) * kWidth * 4,
                                         hipMemcpyHostToDevice, stream));
            for (uint32_t r = 0; r < rows[b]; ++r) {
                slot[m + r] = static_cast<uint32_t>(b);
                pos[m + r] = r;
            }
            m += rows[b];
            last[b] = m - 1;
        }
        HIP_CHECK(hipMemcpyAsync(row_slot.p, slot.data(), M * 4, hipMemcpyHostToDevice, stream));
        HIP_CHECK(hipMemcpyAsync(row_pos.p, pos.data(), M * 4, hipMemcpyHostToDevice, stream));
        HIP_CHECK(hipMemcpyAsync(last_rows.p, last.data(), kMaxBatch * 4, hipMemcpyHostToDevice, stream));
        // Host vectors above must outlive the async copies.
        HIP_CHECK(hipStreamSynchronize(stream));
        enqueue_prefill_layers(PrefillBufs{px.p, pxn.p, pq.p, patt.p, pff.p, row_slot.p, row_pos.p, last_rows.p, pws.p}, nseq, M);
    }

    // The prefill forward over M stacked rows whose inputs are in b.x, with each row's
    // sequence slot and position in b.row_slot / b.row_pos and each sequence's last row in
    // b.last_rows; leaves the last rows' logits in logits[0..nseq).
    void enqueue_prefill_layers(const PrefillBufs& b, int nseq, uint32_t M) {
        float *px_ = b.x, *pxn_ = b.xn, *pq_ = b.q, *patt_ = b.att, *pff_ = b.ff;
        for (int l = 0; l < layers; ++l) {
            const float* par = params.p + static_cast<size_t>(l) * kParLayer;
            // layers after the first get ln_1 from the previous layer's mlp.c_proj launch
            if (l == 0) HIP_CHECK(launch_ln_rows(LnRowsArgs{px_, pxn_, par + kParLn1W, par + kParLn1B, static_cast<int>(M)}, stream));
            GemmArgs g{};
            g.a = pxn_;
            g.w = w_ptr(off_qkv[l]);
            g.bias = par + kParQkvB;
            g.M = static_cast<int>(M);
            g.N = kQkv;
            g.K = kWidth;
            g.splits = gemm_splits(static_cast<int>(M), kQkv, kWidth);
            g.ws = b.ws;
            g.c = pq_;
            g.kv = kv.p;
            g.kv_slot_stride = kv_slot_stride;
            g.kv_layer_off = kv_layer_off(l);
            g.kv_v_off = kv_v_off;
            g.kv_cap = cap;
            g.row_slot = b.row_slot;
            g.row_pos = b.row_pos;
            HIP_CHECK(launch_gemm(g, kGemmQkv, bf16, stream));
            CausalArgs c{};
            c.q = pq_;
            c.kv = kv.p;
            c.kv_slot_stride = kv_slot_stride;
            c.kv_layer_off = kv_layer_off(l);
            c.kv_v_off = kv_v_off;
            c.kv_cap = cap;
            c.row_slot = b.row_slot;
            c.row_pos = b.row_pos;
            c.out = patt_;
            c.M = static_cast<int>(M);
            HIP_CHECK(launch_causal_attention(c, stream));
            GemmArgs p{};
            p.a = patt_;
            p.w = w_ptr(off_proj[l]);
            p.bias = par + kParProjB;
            p.M = static_cast<int>(M);
            p.N = kWidth;
            p.K = kWidth;
            p.splits = gemm_splits(static_cast<int>(M), kWidth, kWidth);
            p.ws = b.ws;
            p.c = px_;
            p.ln_w = par + kParLn2W;  // ln_2 of the new residual rows
            p.ln_b = par + kParLn2B;
            p.ln_out = pxn_;
            HIP_CHECK(launch_gemm(p, kGemmResid, bf16, stream));
            GemmArgs f{};
            f.a = pxn_;
            f.w = w_ptr(off_fc[l]);
            f.bias = par + kParFcB;
            f.M = static_cast<int>(M);
            f.N = kFfn;
            f.K = kWidth;
            f.splits = gemm_splits(static_cast<int>(M), kFfn, kWidth);
            f.ws = b.ws;
            f.c = pff_;
            HIP_CHECK(launch_gemm(f, kGemmGelu, bf16, stream));
            GemmArgs f2{};
            f2.a = pff_;
            f2.w = w_ptr(off_fc2[l]);
            f2.bias = par + kParFc2B;
            f2.M = static_cast<int>(M);
            f2.N = kWidth;
            f2.K = kFfn;
            f2.splits = gemm_splits(static_cast<int>(M), kWidth, kFfn);
            f2.ws = b.ws;
            f2.c = px_;
            if (l + 1 < layers) {  // ln_1 of the next layer
                f2.ln_w = par + kParLayer + kParLn1W;
                f2.ln_b = par + kParLayer + kParLn1B;
                f2.ln_out = pxn_;
            }
            HIP_CHECK(launch_gemm(f2, kGemmResid, bf16, stream));
        }
        HIP_CHECK(launch_gather_rows(px_, b.last_rows, h.p, nseq, stream));
        enqueue_head(nseq, gemv_batch_bucket(nseq));
    }

    void upload_states(int n) {
        HIP_CHECK(hipMemcpyAsync(state.p, pinned_state, n * sizeof(SeqState), hipMemcpyHostToDevice, stream));
    }

    static SeqState make_state(const itts_gen_options& o, uint32_t prefix_rows, uint32_t max_tokens) {
        SeqState s{};
        s.n = prefix_rows;
        s.active = 1;
        s.max_tokens = max_tokens;
        s.prefix_rows = prefix_rows;
        s.do_sample = o.do_sample ? 1u : 0u;
        s.top_k = o.top_k;
        s.num_beams = o.num_beams;
        s.temperature = o.temperature;
        s.top_p = o.top_p;
        s.penalty = o.repetition_penalty;
        s.suppress_stop = o.suppress_stop;
        s.rng = o.seed;
        return s;
    }

    // ---------------------------------------------------------------- API operations
    void check_prefix(uint32_t rows) const {
        if (rows == 0 || rows > 1024 || rows > cap) throw std::invalid_argument("Invalid GPT prefill dimensions");
    }

    void prefill(const float* prefix, uint32_t rows, float* out_logits) {
        check_prefix(rows);
        itts_gen_options o;
        itts_gen_options_default(&o);
        pinned_state[0] = make_state(o, rows, 1);
        upload_states(1);
        HIP_CHECK(hipEventRecord(ev[0], stream));
        enqueue_prefill({prefix}, {rows});
        HIP_CHECK(hipEventRecord(ev[1], stream));
        HIP_CHECK(hipMemcpyAsync(out_logits, logits.p, kMelVocab * 4, hipMemcpyDeviceToHost, stream));
        HIP_CHECK(hipStreamSynchronize(stream));
        HIP_CHECK(hipEventElapsedTime(&timing.prefill_ms, ev[0], ev[1]));
        cached = rows;
    }

    void step(uint32_t code, uint32_t position, float* out_logits) {
        if (!cached || cached >= cap || code >= static_cast<uint32_t>(kMelVocab) || position >= mel_pos_rows)
            throw std::invalid_argument("GPT step requires valid cache, code and position");
        itts_gen_options o;
        itts_gen_options_default(&o);
        SeqState s = make_state(o, cached, 1);
        s.n = cached;
        s.token = code;
        s.position = position;
        pinned_state[0] = s;
        upload_states(1);
        run_step(1, 1, false, false);
        HIP_CHECK(hipMemcpyAsync(out_logits, logits.p, kMelVocab * 4, hipMemcpyDeviceToHost, stream));
        HIP_CHECK(hipStreamSynchronize(stream));
        check_step_error();
        cached++;
    }

    static void validate_generation(itts_gen_options& c, uint32_t maximum, uint32_t prefix_rows, uint32_t mel_rows, uint32_t cap) {
        // gpt_sampling.cpp:169-173 (the reference's literal 1280 and 4096 are width and capacity).
        if (!maximum || maximum + 1 >= mel_rows || prefix_rows + maximum >= cap)
            throw std::invalid_argument("GPT generation capacity exceeded");
        if (!c.do_sample) {
            c.temperature = 1;
            c.top_k = 0;
            c.top_p = 1;
        }
        if (!std::isfinite(c.temperature) || !std::isfinite(c.top_p) || !std::isfinite(c.repetition_penalty) || c.temperature <= 0 ||
            c.top_p <= 0 || c.top_p > 1 || c.repetition_penalty <= 0)
            throw std::invalid_argument("Invalid GPT generation parameters");
        if (!c.num_beams || c.num_beams > 10 || !std::isfinite(c.length_penalty))
            throw std::invalid_argument("Invalid beam search configuration");
    }

    // Repetition sets of sequences 0..nseq-1 = the history {1, 8192} (gpt_sampling.cpp:176).
    void reset_seen(int nseq) { HIP_CHECK(launch_seen_reset(seen.p, nseq, stream)); }

    // Device-driven decode loop for nseq independent sequences whose prefill logits
    // are in logits[0..nseq): sampler, then (forward + sampler) graph replays.
    void decode_loop(int nseq, uint32_t max_tokens) {
        const int nb = gemv_batch_bucket(nseq);
        if (use_graphs && !no_alloc_call && !persistent(nseq, false)) (void)graph(nseq, nb, true, false);  // captured before any work is queued
        HIP_CHECK(launch_sampler(sample_base(kModeDecode), nseq, stream));
        constexpr uint32_t kChunk = 16;
        uint32_t launched = 0;
        int k = 0;
        while (launched + 1 < max_tokens) {
            const uint32_t n = std::min(kChunk, max_tokens - 1 - launched);
            for (uint32_t i = 0; i < n; ++i) run_step(nseq, nb, true, false);
            launched += n;
            HIP_CHECK(hipMemcpyAsync(pinned + 16 * (k & 1), &state.p[0].active, 4, hipMemcpyDeviceToHost, stream));
            for (int b = 1; b < nseq; ++b)
                HIP_CHECK(hipMemcpyAsync(pinned + 16 * (k & 1) + b, &state.p[b].active, 4, hipMemcpyDeviceToHost, stream));
            HIP_CHECK(hipEventRecord(ev[2 + (k & 1)], stream));
            if (k >= 1) {
                HIP_CHECK(hipEventSynchronize(ev[2 + ((k - 1) & 1)]));
                bool any = false;
                for (int b = 0; b < nseq; ++b) any |= pinned[16 * ((k - 1) & 1) + b] != 0;
                if (!any) break;
            }
            ++k;
        }
    }

    void generate_batch(const std::vector<const float*>& prefixes, const std::vector<uint32_t>& rows,
                        const std::vector<itts_gen_options>& opts_in, uint32_t max_tokens, uint32_t* codes_out,
                        uint32_t* n_codes, int32_t* stopped) {
        const int nseq = static_cast<int>(prefixes.size());
        if (nseq < 1 || static_cast<uint32_t>(nseq) > max_batch) throw std::invalid_argument("Invalid batch size");
        std::vector<itts_gen_options> opts = opts_in;
        for (int b = 0; b < nseq; ++b) {
            check_prefix(rows[b]);
            validate_generation(opts[b], max_tokens, rows[b], mel_pos_rows, cap);
            if (opts[b].num_beams > 1) throw std::invalid_argument("Beam search is decoded one request at a time");
        }
        for (int b = 0; b < nseq; ++b) pinned_state[b] = make_state(opts[b], rows[b], max_tokens);
        upload_states(nseq);
        reset_seen(nseq);
        HIP_CHECK(hipEventRecord(ev[0], stream));
        enqueue_prefill(prefixes, rows);
        HIP_CHECK(hipEventRecord(ev[1], stream));
        decode_loop(nseq, max_tokens);
        finish_generation(nseq, max_tokens, codes_out, n_codes, stopped);
    }

    // After decode_loop: timings, errors and the codes of sequences 0..nseq-1 (statuses are
    // staged in pinned[32..32+nseq); decode_loop uses pinned[0..32)).
    void finish_generation(int nseq, uint32_t max_tokens, uint32_t* codes_out, uint32_t* n_codes, int32_t* stopped) {
        HIP_CHECK(hipEventRecord(ev[2], stream));
        HIP_CHECK(hipMemcpyAsync(pinned_state, state.p, nseq * sizeof(SeqState), hipMemcpyDeviceToHost, stream));
        uint32_t* st = pinned + 32;
        HIP_CHECK(hipMemcpyAsync(st, status.p, nseq * 4, hipMemcpyDeviceToHost, stream));
        HIP_CHECK(hipStreamSynchronize(stream));
        HIP_CHECK(hipEventElapsedTime(&timing.prefill_ms, ev[0], ev[1]));
        HIP_CHECK(hipEventElapsedTime(&timing.decode_ms, ev[1], ev[2]));
        check_step_error();
        uint32_t steps = 0;
        for (int b = 0; b < nseq; ++b) {
            const SeqState& s = pinned_state[b];
            if (s.error) throw std::runtime_error(sampler_message(st[b]));
            steps = std::max(steps, s.count);
            HIP_CHECK(hipMemcpy(codes_out + static_cast<size_t>(b) * max_tokens, codes.p + static_cast<size_t>(b) * cap,
                                s.count * 4, hipMemcpyDeviceToHost));
            n_codes[b] = s.count;
            stopped[b] = s.stopped ? 1 : 0;
        }
        timing.decode_steps = steps;
        const SeqState& s0 = pinned_state[0];
        cached = s0.prefix_rows + (s0.stopped ? s0.count : (s0.count ? s0.count - 1 : 0));
    }

    // generate() for one sequence (num_beams 1) without allocating: the prefill activations
    // live in this device's `scratch` array (prefixes up to kNoAllocRows rows), the decode
    // loop uses the buffers allocated at creation, and a decode graph not captured yet is
    // replaced by eager launches of the same kernels.  Same kernels, same codes as generate().
    void generate_noalloc(const float* prefix, uint32_t rows, const itts_gen_options& opt, uint32_t max_tokens,
                          uint32_t* codes_out, uint32_t* n_codes, int32_t* stopped) {
        itts_gen_options c = opt;
        check_prefix(rows);
        validate_generation(c, max_tokens, rows, mel_pos_rows, cap);
        if (c.num_beams != 1)
            throw std::invalid_argument("itts_gpt_generate_noalloc decodes one sequence without beams (num_beams 1)");
        if (rows > kNoAllocRows)
            throw std::invalid_argument("itts_gpt_generate_noalloc: the prefix exceeds the 512-row scratch");
        if (!scratch_dev || !scratch_dev->ptr)
            throw std::runtime_error("itts_gpt_generate_noalloc: no scratch on this device" +
                                     (scratch_dev ? ": " + scratch_dev->error : std::string()));
        std::lock_guard<std::mutex> lock(*scratch_dev->lock);
        struct Drain {  // destroyed before `lock`: on every exit, errors included, the work this
                        // call queued on the shared scratch has finished before the lock is released
            hipStream_t s;
            ~Drain() { (void)hipStreamSynchronize(s); }
        } drain{stream};
        uint8_t* base = scratch_dev->ptr;
        const PrefillBufs b{reinterpret_cast<float*>(base + kScratchOffX),      reinterpret_cast<float*>(base + kScratchOffXn),
                            reinterpret_cast<float*>(base + kScratchOffQ),      reinterpret_cast<float*>(base + kScratchOffAtt),
                            reinterpret_cast<float*>(base + kScratchOffFf),     reinterpret_cast<uint32_t*>(base + kScratchOffSlot),
                            reinterpret_cast<uint32_t*>(base + kScratchOffPos), reinterpret_cast<uint32_t*>(base + kScratchOffLast),
                            reinterpret_cast<float*>(base + kScratchOffWs)};
        struct Flag {  // cleared on every exit, errors included
            bool& f;
            explicit Flag(bool& x) : f(x) { f = true; }
            ~Flag() { f = false; }
        } flag(no_alloc_call);
        pinned_state[0] = make_state(c, rows, max_tokens);
        upload_states(1);
        reset_seen(1);
        HIP_CHECK(hipEventRecord(ev[0], stream));
        HIP_CHECK(hipMemcpyAsync(b.x, prefix, static_cast<size_t>(rows) * kWidth * 4, hipMemcpyHostToDevice, stream));
        HIP_CHECK(launch_prefill_rows_one(b.row_slot, b.row_pos, b.last_rows, rows, stream));
        enqueue_prefill_layers(b, 1, rows);
        HIP_CHECK(hipEventRecord(ev[1], stream));
        decode_loop(1, max_tokens);
        finish_generation(1, max_tokens, codes_out, n_codes, stopped);
    }

    void generate(const float* prefix, uint32_t rows, const itts_gen_options& opt, uint32_t max_tokens, uint32_t* codes_out,
                  uint32_t* n_codes, int32_t* stopped);
    void generate_segments(const float* cond, uint32_t n_cond, const float* speaker, const float* emotion, const uint32_t* ids,
                           const uint32_t* id_counts, uint32_t nseg, uint32_t language, const itts_gen_options& options,
                           uint32_t max_tokens, uint32_t* codes_out, uint32_t* n_codes, int32_t* stopped);

    // ---------------------------------------------------------------- processors / sampler API
    void apply_processors(const float* in, uint32_t vocab, const uint32_t* history, uint32_t n_history,
                          const itts_gen_options& o, float* out) {
        if (vocab != static_cast<uint32_t>(kMelVocab)) throw std::invalid_argument("Processors run on the 8194-entry mel vocabulary");
        // Argument checks in the reference's order (gpt_sampling.cpp:33-35, 50-52, 69-71).
        if (o.repetition_penalty != 1.0f && o.repetition_penalty <= 0.0f)
            throw std::runtime_error("GPT repetition penalty must be positive");
        if (o.temperature <= 0.0f) throw std::runtime_error("GPT sampling temperature must be positive");
        if (o.top_p < 1.0f && o.top_p <= 0.0f) throw std::runtime_error("GPT top_p must be in (0, 1]");
        const int slot = kMaxBatch;
        std::vector<uint8_t> sn(kMelVocab, 0);
        for (uint32_t i = 0; i < n_history; ++i)
            if (history[i] < vocab) sn[history[i]] = 1;
        SeqState s = make_state(o, 0, 0);
        pinned_state[slot] = s;
        HIP_CHECK(hipMemcpyAsync(state.p + slot, pinned_state + slot, sizeof(SeqState), hipMemcpyHostToDevice, stream));
        HIP_CHECK(hipMemcpyAsync(seen.p + static_cast<size_t>(slot) * kMelVocab, sn.data(), kMelVocab, hipMemcpyHostToDevice, stream));
        HIP_CHECK(hipMemcpyAsync(logits.p + static_cast<size_t>(slot) * kMelVocab, in, kMelVocab * 4, hipMemcpyHostToDevice, stream));
        SampleArgs a = sample_base(kModeProcessors);
        a.logits = logits.p + static_cast<size_t>(slot) * kMelVocab;
        a.state = state.p + slot;
        a.seen = seen.p + static_cast<size_t>(slot) * kMelVocab;
        a.probs = probs.p + static_cast<size_t>(slot) * kMelVocab;
        a.status = status.p + slot;
        a.out_scores = api_out.p;
        HIP_CHECK(launch_sampler(a, 1, stream));
        uint32_t st = 0;
        HIP_CHECK(hipMemcpyAsync(out, api_out.p, kMelVocab * 4, hipMemcpyDeviceToHost, stream));
        HIP_CHECK(hipMemcpyAsync(&st, status.p + slot, 4, hipMemcpyDeviceToHost, stream));
        HIP_CHECK(hipStreamSynchronize(stream));
        if (st) throw std::runtime_error(sampler_message(st));
    }

    void sample(const float* processed, uint32_t vocab, uint64_t* rng, uint32_t draws, uint32_t* tokens) {
        if (vocab != static_cast<uint32_t>(kMelVocab)) throw std::invalid_argument("Sampler runs on the 8194-entry mel vocabulary");
        if (draws == 0 || draws > api_tokens.n) throw std::invalid_argument("Invalid draw count");
        const int slot = kMaxBatch;
        itts_gen_options o;
        itts_gen_options_default(&o);
        SeqState s = make_state(o, 0, 0);
        s.rng = *rng;
        pinned_state[slot] = s;
        HIP_CHECK(hipMemcpyAsync(state.p + slot, pinned_state + slot, sizeof(SeqState), hipMemcpyHostToDevice, stream));
        HIP_CHECK(hipMemcpyAsync(logits.p + static_cast<size_t>(slot) * kMelVocab, processed, kMelVocab * 4, hipMemcpyHostToDevice, stream));
        SampleArgs a = sample_base(kModeDraw);
        a.logits = logits.p + static_cast<size_t>(slot) * kMelVocab;
        a.state = state.p + slot;
        a.seen = seen.p + static_cast<size_t>(slot) * kMelVocab;
        a.probs = probs.p + static_cast<size_t>(slot) * kMelVocab;
        a.status = status.p + slot;
        a.out_tokens = api_tokens.p;
        a.draws = static_cast<int>(draws);
        HIP_CHECK(launch_sampler(a, 1, stream));
        uint32_t st = 0;
        HIP_CHECK(hipMemcpyAsync(tokens, api_tokens.p, draws * 4, hipMemcpyDeviceToHost, stream));
        HIP_CHECK(hipMemcpyAsync(&st, status.p + slot, 4, hipMemcpyDeviceToHost, stream));
        HIP_CHECK(hipMemcpyAsync(pinned_state + slot, state.p + slot, sizeof(SeqState), hipMemcpyDeviceToHost, stream));
        HIP_CHECK(hipStreamSynchronize(stream));
        if (st) throw std::runtime_error(sampler_message(st));
        *rng = pinned_state[slot].rng;
    }

    // ---------------------------------------------------------------- checkpoint / restore
    Snapshot* checkpoint() {
        if (!cached || cached > cap) throw std::invalid_argument("Invalid KV snapshot");
        auto s = std::make_unique<Snapshot>();
        s->tokens = cached;
        const size_t blocks = static_cast<size_t>(layers) * 2 * kHeads;
        s->kv.alloc(blocks * cached * kHeadDim);
        HIP_CHECK(hipMemcpy2DAsync(s->kv.p, static_cast<size_t>(cached) * kHeadDim * 4, kv.p, static_cast<size_t>(cap) * kHeadDim * 4,
                                   static_cast<size_t>(cached) * kHeadDim * 4, blocks, hipMemcpyDeviceToDevice, stream));
        HIP_CHECK(hipStreamSynchronize(stream));
        return s.release();
    }
    void restore(const Snapshot& s) {
        if (!s.tokens || s.tokens > cap) throw std::invalid_argument("Invalid KV restore");
        const size_t blocks = static_cast<size_t>(layers) * 2 * kHeads;
        HIP_CHECK(hipMemcpy2DAsync(kv.p, static_cast<size_t>(cap) * kHeadDim * 4, s.kv.p, static_cast<size_t>(s.tokens) * kHeadDim * 4,
                                   static_cast<size_t>(s.tokens) * kHeadDim * 4, blocks, hipMemcpyDeviceToDevice, stream));
        HIP_CHECK(hipStreamSynchronize(stream));
        cached = s.tokens;
    }

    // ---------------------------------------------------------------- prefix
    void prepare_tail(const uint32_t* text, uint32_t n_text, uint32_t language, std::vector<uint32_t>& ids) {
        if (language >= lang_vocab) throw std::invalid_argument("Invalid GPT conditioning dimensions");
        ids.assign(1, 0u);
        for (uint32_t i = 0; i < n_text; ++i) {
            if (text[i] >= text_vocab) throw std::invalid_argument("Text token is outside 2.5 vocabulary");
            if (text[i] != 0 && text[i] != 1) ids.push_back(text[i]);
        }
        ids.push_back(1);
        if (ids.size() > text_pos_rows) throw std::invalid_argument("Text segment exceeds GPT position capacity");
    }
    void build_prefix(const float* cond_host, uint32_t n_cond, const float* speaker, const float* emotion, const uint32_t* text,
                      uint32_t n_text, uint32_t language, float* out, uint32_t capacity_rows, uint32_t* rows) {
        std::vector<uint32_t> ids;
        prepare_tail(text, n_text, language, ids);
        const uint32_t total = n_cond + static_cast<uint32_t>(ids.size()) + 1;
        if (total > capacity_rows) throw std::invalid_argument("Prefix output buffer too small");
        DevBuf<float> d;
        d.alloc(static_cast<size_t>(total) * kWidth);
        DevBuf<uint32_t> did;
        did.alloc(ids.size());
        HIP_CHECK(hipMemcpyAsync(did.p, ids.data(), ids.size() * 4, hipMemcpyHostToDevice, stream));
        if (cond_host) {
            HIP_CHECK(hipMemcpyAsync(d.p, cond_host, static_cast<size_t>(n_cond) * kWidth * 4, hipMemcpyHostToDevice, stream));
        } else {
            DevBuf<float> sp, em;
            sp.alloc(192);
            em.alloc(kWidth);
            HIP_CHECK(hipMemcpyAsync(sp.p, speaker, 192 * 4, hipMemcpyHostToDevice, stream));
            HIP_CHECK(hipMemcpyAsync(em.p, emotion, kWidth * 4, hipMemcpyHostToDevice, stream));
            HIP_CHECK(hipMemsetAsync(d.p, 0, 3ull * kWidth * 4, stream));
            HIP_CHECK(launch_speaker_row(spk_w.p, spk_b.p, sp.p, em.p, d.p, stream));
            HIP_CHECK(hipStreamSynchronize(stream));
        }
        HIP_CHECK(launch_text_rows(text_emb.p, text_pos.p, lang_emb.p, mel_emb.p, mel_pos.p, did.p, static_cast<int>(ids.size()),
                                   language, d.p + static_cast<size_t>(n_cond) * kWidth, stream));
        HIP_CHECK(hipMemcpyAsync(out, d.p, d.n * 4, hipMemcpyDeviceToHost, stream));
        HIP_CHECK(hipStreamSynchronize(stream));
        *rows = total;
    }

    // ---------------------------------------------------------------- measurement
    // Launches one decode kernel kind `iters` times (layer l = i % layers, so consecutive
    // launches stream different weights) between two HIP events on the handle's stream.
    void bench_kernel(int which, int batch, uint32_t cached_rows, int iters, float* avg_ms, double* bytes) {
        const bool one_layer = (which & ITTS_BENCH_ONE_LAYER) != 0;  // every launch on layer 0's weights
        which &= ~ITTS_BENCH_ONE_LAYER;
        if (!layers || which < 0 || which > 7 || iters < 1 || batch < 1 || batch > static_cast<int>(max_batch))
            throw std::invalid_argument("Invalid kernel benchmark request");
        if (which == 6 && !persistent(batch, false)) throw std::invalid_argument("The persistent step kernel is not available on this decoder");
        if (!cached_rows) cached_rows = 752;
        if (cached_rows + 1 >= cap) throw std::invalid_argument("Invalid kernel benchmark request");
        if (which == 7) {
            bench_copy(iters, avg_ms, bytes);
            return;
        }
        const int nb = gemv_batch_bucket(batch);
        std::vector<SeqState> st(batch);
        for (int b = 0; b < batch; ++b) {
            itts_gen_options o;
            itts_gen_options_default(&o);
            st[b] = make_state(o, cached_rows, 2);
            st[b].token = 1;
            st[b].position = 2;
        }
        std::copy(st.begin(), st.end(), pinned_state);
        upload_states(batch);
        HIP_CHECK(hipStreamSynchronize(stream));
        auto launch = [&](int l) {
            const float* par = params.p + static_cast<size_t>(l) * kParLayer;
            GemvArgs a = gemv_base(batch);
            a.x_stride = kWidth;
            a.out_stride = kWidth;
            switch (which) {
                case 0:
                    a.w = w_ptr(off_qkv[l]); a.bias = par + kParQkvB; a.rows = kQkv; a.x = h.p; a.ln_w = par + kParLn1W;
                    a.ln_b = par + kParLn1B; a.q = q.p; a.kv_layer_off = kv_layer_off(l);
                    HIP_CHECK(launch_gemv_qkv(a, nb, bf16, false, stream));
                    break;
                case 1:
                    a.w = w_ptr(off_proj[l]); a.bias = par + kParProjB; a.rows = kWidth; a.x = attn.p; a.resid = h.p; a.out = hmid.p;
                    HIP_CHECK(launch_gemv_proj(a, nb, bf16, stream));
                    break;
                case 2:
                    a.w = w_ptr(off_fc[l]); a.bias = par + kParFcB; a.rows = kFfn; a.x = hmid.p; a.ln_w = par + kParLn2W;
                    a.ln_b = par + kParLn2B; a.out = ff.p; a.out_stride = kFfn;
                    HIP_CHECK(launch_gemv_fc(a, nb, bf16, stream));
                    break;
                case 3:
                    a.w = w_ptr(off_fc2[l]); a.bias = par + kParFc2B; a.rows = kWidth; a.x = ff.p; a.x_stride = kFfn; a.resid = hmid.p;
                    a.out = h.p;
                    HIP_CHECK(launch_gemv_fc2(a, nb, bf16, stream));
                    break;
                case 4:
                    enqueue_head(batch, nb);
                    break;
                case 6:
                    launch_persistent(batch, false);
                    break;
                default: {
                    AttnArgs t{};
                    t.q = q.p; t.kv = kv.p; t.kv_slot_stride = kv_slot_stride; t.kv_layer_off = kv_layer_off(l); t.kv_v_off = kv_v_off;
                    t.kv_cap = cap; t.partial = partial.p; t.out = attn.p; t.state = state.p; t.nseq = batch; t.splits = splits;
                    HIP_CHECK(launch_attention(t, nb, stream));
                }
            }
        };
        for (int i = 0; i < std::min(iters, layers); ++i) launch(one_layer ? 0 : i % layers);  // warm-up
        HIP_CHECK(hipEventRecord(ev[0], stream));
        for (int i = 0; i < iters; ++i) launch(one_layer ? 0 : i % layers);
        HIP_CHECK(hipEventRecord(ev[1], stream));
        HIP_CHECK(hipEventSynchronize(ev[1]));
        float ms = 0;
        HIP_CHECK(hipEventElapsedTime(&ms, ev[0], ev[1]));
        *avg_ms = ms / iters;
        const double e = static_cast<double>(elt);
        const double rows[5] = {kQkv, kWidth, kFfn, kWidth, kMelVocab};
        const double cols[5] = {kWidth, kWidth, kWidth, kFfn, kWidth};
        if (which == 6) {
            // the whole forward: every weight byte once, then per sequence its embedding rows and
            // K/V rows read and the new row written
            const double weights = static_cast<double>(slab.n) + 4.0 * (params.n + head_params.n);
            *bytes = weights + batch * (2.0 * kWidth * 4 + static_cast<double>(layers) * 2.0 * (st[0].n + 1) * kWidth * 4.0);
            check_step_error();
        } else if (which < 5) {
            // weights + bias + input rows (+ LayerNorm params) + outputs, per launch
            *bytes = rows[which] * cols[which] * e + rows[which] * 4.0 + batch * cols[which] * 4.0 + batch * rows[which] * 4.0 +
                     ((which == 0 || which == 2) ? 2.0 * kWidth * 4 : 0.0) + (which == 4 ? 4.0 * kWidth * 4 : 0.0) +
                     ((which == 1 || which == 3) ? batch * rows[which] * 4.0 : 0.0);
        } else {
            *bytes = static_cast<double>(batch) * 2.0 * (st[0].n + 1) * kWidth * 4.0;  // K and V rows read
        }
    }

    // Device-to-device copy of 256 MiB of the weight slab (a plain copy kernel of known
    // size, the reference point for HBM traffic counters): bytes = read + written.
    // Phases of the persistent step (batch 1) or batch step (nseq 2-4 sequences, each at
    // `cached_rows` cached rows) from the kernel's own clock stamps (100 MHz): T_k(l) = the
    // latest workgroup's end of phase k of layer l; the phase's share of the step is
    // T_k - T_{k-1} (T_0 = the latest layer start).  out[0] mean layer time, out[1..6] mean
    // phase shares (c_attn, attention tiles, merge, attn.c_proj, mlp.c_fc, mlp.c_proj), out[7]
    // the head (ln_f, final_norm, mel_head), all in us.
    void step_phases(uint32_t cached_rows, int iters, float* out, int nseq = 1) {
        if (!layers || iters < 1 || nseq < 1 || nseq > static_cast<int>(max_batch) || !persistent(nseq, false))
            throw std::invalid_argument("The persistent step kernel is not available on this decoder");
        if (!cached_rows) cached_rows = 752;
        if (cached_rows + 1 >= cap) throw std::invalid_argument("Invalid kernel benchmark request");
        itts_gen_options o;
        itts_gen_options_default(&o);
        SeqState st = make_state(o, cached_rows, 2);
        st.token = 1;
        st.position = 2;
        for (int q = 0; q < nseq; ++q) pinned_state[q] = st;
        upload_states(nseq);
        const size_t per = static_cast<size_t>(layers + 1) * kStepStampsPerLayer;
        DevBuf<uint64_t> stamps;
        stamps.alloc(static_cast<size_t>(step_grid) * per);
        std::vector<uint64_t> host(stamps.n);
        std::vector<double> sum(8, 0.0);
        for (int it = 0; it <= iters; ++it) {  // launch 0 warms up
            HIP_CHECK(hipMemsetAsync(stamps.p, 0, stamps.n * 8, stream));
            StepArgs a = step_args(0, nseq);
            a.stamps = stamps.p;
            HIP_CHECK(launch_step_serialized(a, nseq, step_grid, bf16, step_dev, stream));
            HIP_CHECK(hipMemcpyAsync(host.data(), stamps.p, stamps.n * 8, hipMemcpyDeviceToHost, stream));
            HIP_CHECK(hipStreamSynchronize(stream));
            check_step_error();
            if (it == 0) continue;
            auto T = [&](int l, int k) {
                uint64_t m = 0;
                for (int b = 0; b < step_grid; ++b) m = std::max(m, host[b * per + static_cast<size_t>(l) * kStepStampsPerLayer + k]);
                return static_cast<double>(m);
            };
            for (int l = 0; l < layers; ++l) {
                sum[0] += T(l, 6) - T(l, 0);
                for (int k = 1; k <= 6; ++k) sum[k] += T(l, k) - T(l, k - 1);
            }
            sum[7] += T(layers, 6) - T(layers, 0);
        }
        for (int k = 0; k < 7; ++k) out[k] = static_cast<float>(sum[k] / (static_cast<double>(iters) * layers) * 0.01);  // 10 ns ticks
        out[7] = static_cast<float>(sum[7] / iters * 0.01);
    }

    void bench_copy(int iters, float* avg_ms, double* bytes) {
        const size_t n = std::min<size_t>(slab.n, size_t(256) << 20);
        DevBuf<uint8_t> dst;
        dst.alloc(n);
        HIP_CHECK(hipMemcpyAsync(dst.p, slab.p, n, hipMemcpyDeviceToDevice, stream));
        HIP_CHECK(hipEventRecord(ev[0], stream));
        for (int i = 0; i < iters; ++i) HIP_CHECK(hipMemcpyAsync(dst.p, slab.p, n, hipMemcpyDeviceToDevice, stream));
        HIP_CHECK(hipEventRecord(ev[1], stream));
        HIP_CHECK(hipEventSynchronize(ev[1]));
        float ms = 0;
        HIP_CHECK(hipEventElapsedTime(&ms, ev[0], ev[1]));
        *avg_ms = ms / iters;
        *bytes = 2.0 * static_cast<double>(n);
    }

    // ---------------------------------------------------------------- beams
    void generate_beams(const float* prefix, uint32_t rows, const itts_gen_options& config, uint32_t maximum,
                        std::vector<uint32_t>& result, bool& eos);
};

void Engine::generate(const float* prefix, uint32_t rows, const itts_gen_options& opt, uint32_t max_tokens, uint32_t* codes_out,
                      uint32_t* n_codes, int32_t* stopped) {
    itts_gen_options c = opt;
    check_prefix(rows);
    validate_generation(c, max_tokens, rows, mel_pos_rows, cap);
    if (c.num_beams > 1) {
        std::vector<uint32_t> out;
        bool eos = false;
        generate_beams(prefix, rows, c, max_tokens, out, eos);
        std::copy(out.begin(), out.end(), codes_out);
        *n_codes = static_cast<uint32_t>(out.size());
        *stopped = eos ? 1 : 0;
        return;
    }
    generate_batch({prefix}, {rows}, {c}, max_tokens, codes_out, n_codes, stopped);
}

// NativeRuntime::synthesize's GPT loop (native_runtime.cpp:98-99): segment i's prefix is
// prepare(conditioning, ids_i, language) (gpt.cpp:42-71) and its codes are
// generate(prefix, options with seed + i, max_tokens).  Every segment is checked, in order,
// before any work is queued.  The prefixes are built on the device straight into the
// prefill input (no host copy of the rows), and the segments are decoded together,
// max_batch at a time; each gets the codes it gets alone (the batched forward gives every
// row its batch-1 result).  Beam search decodes one segment at a time, as generate() does.
void Engine::generate_segments(const float* cond, uint32_t n_cond, const float* speaker, const float* emotion, const uint32_t* ids,
                               const uint32_t* id_counts, uint32_t nseg, uint32_t language, const itts_gen_options& options,
                               uint32_t max_tokens, uint32_t* codes_out, uint32_t* n_codes, int32_t* stopped) {
    if (!nseg) throw std::invalid_argument("Invalid segment count");
    std::vector<std::vector<uint32_t>> tails(nseg);
    std::vector<uint32_t> rows(nseg);
    std::vector<itts_gen_options> opts(nseg, options);
    size_t off = 0;
    for (uint32_t i = 0; i < nseg; ++i) {
        prepare_tail(ids + off, id_counts[i], language, tails[i]);
        off += id_counts[i];
        rows[i] = n_cond + static_cast<uint32_t>(tails[i].size()) + 1;
        check_prefix(rows[i]);
        opts[i].seed = options.seed + i;  // native_runtime.cpp:98 (opts.seed += index)
        validate_generation(opts[i], max_tokens, rows[i], mel_pos_rows, cap);
    }
    // The conditioning rows, once for all segments.
    seg_cond.ensure(static_cast<size_t>(n_cond) * kWidth);
    if (cond) {
        HIP_CHECK(hipMemcpyAsync(seg_cond.p, cond, static_cast<size_t>(n_cond) * kWidth * 4, hipMemcpyHostToDevice, stream));
    } else {
        DevBuf<float> sp, em;
        sp.alloc(192);
        em.alloc(kWidth);
        HIP_CHECK(hipMemcpyAsync(sp.p, speaker, 192 * 4, hipMemcpyHostToDevice, stream));
        HIP_CHECK(hipMemcpyAsync(em.p, emotion, kWidth * 4, hipMemcpyHostToDevice, stream));
        HIP_CHECK(hipMemsetAsync(seg_cond.p, 0, static_cast<size_t>(n_cond) * kWidth * 4, stream));
        HIP_CHECK(launch_speaker_row(spk_w.p, spk_b.p, sp.p, em.p, seg_cond.p, stream));
        HIP_CHECK(hipStreamSynchronize(stream));  // sp and em are freed at the end of this block
    }
    // Segments i0 .. i0 + n - 1: their prefixes staged back to back in px.
    auto stage = [&](uint32_t i0, uint32_t n) {
        size_t m = 0, nid = 0;
        for (uint32_t i = i0; i < i0 + n; ++i) {
            m += rows[i];
            nid += tails[i].size();
        }
        px.ensure(m * kWidth);
        seg_ids.ensure(nid);
        std::vector<uint32_t> flat;
        flat.reserve(nid);
        for (uint32_t i = i0; i < i0 + n; ++i) flat.insert(flat.end(), tails[i].begin(), tails[i].end());
        HIP_CHECK(hipMemcpyAsync(seg_ids.p, flat.data(), nid * 4, hipMemcpyHostToDevice, stream));
        size_t r = 0, k = 0;
        for (uint32_t i = i0; i < i0 + n; ++i) {
            float* dst = px.p + r * kWidth;
            HIP_CHECK(hipMemcpyAsync(dst, seg_cond.p, static_cast<size_t>(n_cond) * kWidth * 4, hipMemcpyDeviceToDevice, stream));
            HIP_CHECK(launch_text_rows(text_emb.p, text_pos.p, lang_emb.p, mel_emb.p, mel_pos.p, seg_ids.p + k,
                                       static_cast<int>(tails[i].size()), language, dst + static_cast<size_t>(n_cond) * kWidth, stream));
            r += rows[i];
            k += tails[i].size();
        }
        HIP_CHECK(hipStreamSynchronize(stream));  // `flat` is read by the copy above
    };
    float prefill_ms = 0, decode_ms = 0;
    uint32_t steps = 0;
    const uint32_t group = options.num_beams > 1 ? 1u : max_batch;
    for (uint32_t i0 = 0; i0 < nseg; i0 += group) {
        const uint32_t n = std::min(group, nseg - i0);
        stage(i0, n);
        uint32_t* out = codes_out + static_cast<size_t>(i0) * max_tokens;
        if (options.num_beams > 1) {
            generate(nullptr, rows[i0], opts[i0], max_tokens, out, n_codes + i0, stopped + i0);
        } else {
            const std::vector<const float*> staged(n, nullptr);
            generate_batch(staged, std::vector<uint32_t>(rows.begin() + i0, rows.begin() + i0 + n),
                           std::vector<itts_gen_options>(opts.begin() + i0, opts.begin() + i0 + n), max_tokens, out, n_codes + i0,
                           stopped + i0);
        }
        prefill_ms += timing.prefill_ms;
        decode_ms += timing.decode_ms;
        steps += timing.decode_steps;
    }
    timing.prefill_ms = prefill_ms;
    timing.decode_ms = decode_ms;
    timing.decode_steps = steps;
}

// gpt_sampling.cpp:190-245.  Scores, processors and candidate selection run on the device
// (beam.hip); so does the choice of children (beam_advance_kernel applies the rule of
// :229-236 to the ranked candidates), so every step (scores, selection, children, KV
// reorder, forward) is queued without waiting for the host.  The host reads each step's
// candidates (written into pinned memory by the selection) a step or two later and runs
// the reference's child/finish bookkeeping
// on them, with the same rule, so its beams are the device's children.  When the search
// ends (early stop, no children, an error), up to kBeamLag queued steps are discarded.
// Beam KV is not snapshotted: child c lives in slot c and inherits its parent's rows
// through the row-owner table (one byte per row), which the attention kernels gather
// through.  Every forward runs num_beams rows; slots without a child are inactive.
void Engine::generate_beams(const float* prefix, uint32_t rows, const itts_gen_options& config, uint32_t maximum,
                            std::vector<uint32_t>& result, bool& eos) {
    const uint32_t nbeam = config.num_beams;
    if (nbeam > max_batch) throw std::invalid_argument("num_beams exceeds the decoder's max_batch");
    struct Beam {
        std::vector<uint32_t> codes;
        float score = 0;
    };
    struct Finished {
        std::vector<uint32_t> codes;
        double score;
        bool eos;
    };
    std::vector<Finished> finished;
    const uint32_t take = 2 * nbeam;
    beam_slots = nbeam;
    beam_scores.ensure(kMaxBatch);
    all_scores.ensure(static_cast<size_t>(kMaxBatch) * kMelVocab);
    beam_list.ensure(static_cast<size_t>(kMaxBatch) * kMelVocab);
    beam_probs.ensure(static_cast<size_t>(kMaxBatch) * kMelVocab);
    cand.ensure(kMaxBeamTake);
    d_token.ensure(kMaxBatch);
    beam_rng.ensure(1);
    beam_np.ensure(1);
    beam_tmpl.ensure(1);
    if (!beam_ring) {
        g_alloc_events.fetch_add(1, std::memory_order_relaxed);
        HIP_CHECK(hipHostMalloc(&beam_ring, kBeamRing * sizeof(BeamSlot), hipHostMallocDefault));
        HIP_CHECK(hipHostGetDevicePointer(reinterpret_cast<void**>(&beam_ring_dev), beam_ring, 0));
        for (auto& e : bev) HIP_CHECK(hipEventCreateWithFlags(&e, hipEventDisableTiming));
    }
    const int nb = gemv_batch_bucket(static_cast<int>(nbeam));
    if (use_graphs && !persistent(static_cast<int>(nbeam), true)) (void)graph(static_cast<int>(nbeam), nb, false, true);

    pinned_state[0] = make_state(config, rows, maximum);
    upload_states(1);
    HIP_CHECK(hipEventRecord(ev[0], stream));
    enqueue_prefill({prefix}, {rows});
    for (uint32_t b = 1; b < nbeam; ++b)
        HIP_CHECK(hipMemcpyAsync(logits.p + static_cast<size_t>(b) * kMelVocab, logits.p, kMelVocab * 4, hipMemcpyDeviceToDevice, stream));
    HIP_CHECK(hipMemsetAsync(table.p, 0, static_cast<size_t>(nbeam) * cap, stream));  // prefix rows live in slot 0
    HIP_CHECK(hipEventRecord(ev[1], stream));
    reset_seen(static_cast<int>(nbeam));
    // The initial beams (gpt_sampling.cpp:196-198): nbeam parents sharing the prefill logits,
    // scores 0, -1e9, ...; the search's RNG; the children's state template.
    uint64_t* prng = reinterpret_cast<uint64_t*>(pinned + 62);
    *prng = config.seed;
    float* pscore = reinterpret_cast<float*>(pinned + 32);
    for (uint32_t p = 0; p < nbeam; ++p) pscore[p] = p ? -1e9f : 0.0f;
    pinned[48] = nbeam;
    HIP_CHECK(hipMemcpyAsync(beam_rng.p, prng, 8, hipMemcpyHostToDevice, stream));
    HIP_CHECK(hipMemcpyAsync(beam_scores.p, pscore, nbeam * 4, hipMemcpyHostToDevice, stream));
    HIP_CHECK(hipMemcpyAsync(beam_np.p, pinned + 48, 4, hipMemcpyHostToDevice, stream));
    HIP_CHECK(hipMemcpyAsync(beam_tmpl.p, pinned_state, sizeof(SeqState), hipMemcpyHostToDevice, stream));

    // Step k: scores and selection over the current parents, the candidates read back into
    // ring slot k, then (unless it is the last step) the children, their KV rows and repetition
    // sets, and their forward.
    auto enqueue = [&](uint32_t k) {
        BeamArgs a{};
        a.logits = logits.p;
        a.seen = seen.p;
        a.beam_score = beam_scores.p;
        a.all_scores = all_scores.p;
        a.probs = beam_probs.p;
        a.list = beam_list.p;
        a.status = status.p;
        a.rng = beam_rng.p;
        a.cand = cand.p;
        a.parents = static_cast<int>(nbeam);
        a.parents_dev = beam_np.p;
        a.take = static_cast<int>(take);
        a.do_sample = config.do_sample ? 1 : 0;
        a.suppress_stop = config.suppress_stop ? 1 : 0;
        a.temperature = config.temperature;
        a.top_p = config.top_p;
        a.penalty = config.repetition_penalty;
        a.top_k = config.top_k;
        a.num_beams = nbeam;
        BeamSlot& slot = beam_ring_dev[k % kBeamRing];
        a.host_cand = slot.cand;
        a.host_status = slot.status;
        HIP_CHECK(launch_beam_scores(a, stream));
        HIP_CHECK(launch_beam_select(a, stream));
        if (k + 1 < maximum) {
            BeamAdvanceArgs v{};
            v.cand = cand.p;
            v.take = static_cast<int>(take);
            v.beams = static_cast<int>(nbeam);
            v.parents_dev = beam_np.p;
            v.parent = d_parent.p;
            v.token = d_token.p;
            v.score = beam_scores.p;
            v.state = state.p;
            v.tmpl = beam_tmpl.p;
            v.n = rows + k;  // rows cached before this forward, equal for every beam
            v.position = k + 2;
            v.cap = cap;
            v.table = table.p;
            v.table_tmp = table_tmp.p;
            v.seen = seen.p;
            v.seen_tmp = seen_tmp.p;
            HIP_CHECK(launch_beam_advance(v, stream));
            run_step(static_cast<int>(nbeam), nb, false, true);
        }
        HIP_CHECK(hipEventRecord(bev[k % kBeamRing], stream));
    };

    std::vector<Beam> beams(nbeam);
    for (uint32_t i = 1; i < beams.size(); ++i) beams[i].score = -1e9f;
    auto finish = [&](const Beam& beam, float score, uint32_t length, bool e) {
        finished.push_back({beam.codes, score / std::pow(static_cast<double>(std::max(length, 1u)), config.length_penalty), e});
        std::stable_sort(finished.begin(), finished.end(), [](const auto& x, const auto& y) { return x.score > y.score; });
        if (finished.size() > nbeam) finished.resize(nbeam);
    };
    uint32_t last_rows = rows, steps = 0, queued = 0;
    std::vector<BeamCand> cands(take);
    for (uint32_t step_index = 0; step_index < maximum; ++step_index) {
        while (queued < maximum && queued <= step_index + kBeamLag) enqueue(queued++);
        HIP_CHECK(hipEventSynchronize(bev[step_index % kBeamRing]));
        const BeamSlot& slot = beam_ring[step_index % kBeamRing];
        const uint32_t P = static_cast<uint32_t>(beams.size());
        for (uint32_t i = 0; i <= P; ++i)
            if (slot.status[i]) throw std::runtime_error(sampler_message(slot.status[i]));
        std::copy(slot.cand, slot.cand + take, cands.begin());
        std::vector<Beam> next;
        for (uint32_t rank = 0; rank < take; ++rank) {
            const BeamCand c = cands[rank];
            const Beam& parent = beams[c.parent];
            if (c.token == static_cast<uint32_t>(kMelStop)) {
                if (rank < nbeam) finish(parent, c.score, step_index + 1, true);
                continue;
            }
            if (c.token >= static_cast<uint32_t>(kMelStart)) throw std::runtime_error("Beam generated invalid semantic code");
            Beam child;
            child.codes = parent.codes;
            child.codes.push_back(c.token);
            child.score = c.score;
            next.push_back(std::move(child));
            if (next.size() == nbeam) break;
        }
        if (next.empty()) break;
        if (step_index + 1 < maximum) {  // this step's forward (queued with the step) counts
            last_rows = rows + step_index + 1;
            ++steps;
        }
        beams = std::move(next);
        if (finished.size() == nbeam &&
            finished.back().score >= cands[0].score / std::pow(static_cast<double>(step_index + 1), config.length_penalty)) {
            beams.clear();
            break;
        }
    }
    HIP_CHECK(hipEventRecord(ev[2], stream));
    HIP_CHECK(hipStreamSynchronize(stream));
    HIP_CHECK(hipEventElapsedTime(&timing.prefill_ms, ev[0], ev[1]));
    HIP_CHECK(hipEventElapsedTime(&timing.decode_ms, ev[1], ev[2]));
    timing.decode_steps = steps;
    check_step_error();
    for (const auto& beam : beams) finish(beam, beam.score, static_cast<uint32_t>(beam.codes.size()), false);
    if (finished.empty()) throw std::runtime_error("Beam search produced no hypotheses");
    result = std::move(finished[0].codes);
    eos = finished[0].eos;
    cached = last_rows;
}

}  // namespace itts

// ==================================================================== C ABI

struct itts_gpt {
    itts::Engine e;
};
struct itts_gpt_state {
    std::unique_ptr<itts::Snapshot> s;
};

namespace {
template <class F>
int guarded(itts_gpt* h, F&& f) {
    try {
        f();
        return ITTS_OK;
    } catch (const std::invalid_argument& e) {
        if (h) h->e.last_error = e.what();
        return ITTS_EINVAL;
    } catch (const std::runtime_error& e) {
        if (h) h->e.last_error = e.what();
        return ITTS_ERUNTIME;
    } catch (const std::exception& e) {
        if (h) h->e.last_error = e.what();
        return ITTS_ELOGIC;
    }
}
}  // namespace

extern "C" {

uint64_t itts_gpt_alloc_events(void) { return itts::g_alloc_events.load(std::memory_order_relaxed); }

void itts_gen_options_default(itts_gen_options* o) {
    std::memset(o, 0, sizeof(*o));
    o->do_sample = 1;
    o->seed = 20261002ull;
    o->temperature = 0.8f;
    o->top_k = 30;
    o->top_p = 0.8f;
    o->repetition_penalty = 10.0f;
    o->num_beams = 1;
    o->length_penalty = 0.0f;
}

int itts_gpt_create(const itts_tensor* tensors, int32_t count, const itts_gpt_config* cfg, itts_gpt** out) {
    if (!out) return ITTS_EINVAL;
    *out = nullptr;
    auto h = std::make_unique<itts_gpt>();
    try {
        h->e.create(tensors, count, cfg);
    } catch (const std::invalid_argument& e) {
        itts::g_create_error = e.what();
        return ITTS_EINVAL;
    } catch (const std::exception& e) {
        itts::g_create_error = e.what();
        return ITTS_ERUNTIME;
    }
    *out = h.release();
    return ITTS_OK;
}

// GptDecoder(Weights&, ...) over a MIT2 bundle: the GPT tensors by the reference's names
// (include/itts25/gpt.hpp collect list; gpt.cpp:8-23), zero-copy from the mapping.
int itts_gpt_create_from_bundle(const itts_bundle* b, const itts_gpt_config* cfg, itts_gpt** out) {
    if (!out) return ITTS_EINVAL;
    *out = nullptr;
    static const char* const kGlobal[] = {"gpt.spk_emb_proj.weight", "gpt.spk_emb_proj.bias", "gpt.text_embedding.weight",
                                          "gpt.text_pos_embedding.emb.weight", "gpt.lang_embedding.weight",
                                          "gpt.mel_embedding.weight", "gpt.mel_pos_embedding.emb.weight", "gpt.gpt.ln_f.weight",
                                          "gpt.gpt.ln_f.bias", "gpt.final_norm.weight", "gpt.final_norm.bias",
                                          "gpt.mel_head.weight", "gpt.mel_head.bias"};
    static const char* const kLayer[] = {".ln_1.weight", ".ln_1.bias", ".attn.c_attn.weight", ".attn.c_attn.bias",
                                         ".attn.c_proj.weight", ".attn.c_proj.bias", ".ln_2.weight", ".ln_2.bias",
                                         ".mlp.c_fc.weight", ".mlp.c_fc.bias", ".mlp.c_proj.weight", ".mlp.c_proj.bias"};
    std::vector<std::string> names;
    std::vector<itts_tensor> list;
    try {
        if (!b) throw std::invalid_argument("Invalid bundle");
        for (const char* n : kGlobal) names.emplace_back(n);
        itts_bundle_tensor t{};
        for (int i = 0;; ++i) {  // layers gpt.gpt.h.0 ... while the bundle has them (24 in IndexTTS 2.5)
            const std::string p = "gpt.gpt.h." + std::to_string(i);
            if (itts_bundle_find(b, (p + ".ln_1.weight").c_str(), &t) != ITTS_OK) break;
            for (const char* s : kLayer) names.push_back(p + s);
        }
        for (const auto& n : names) {
            if (itts_bundle_find(b, n.c_str(), &t) != ITTS_OK) throw std::runtime_error("Missing tensor: " + n);
            if (t.dtype != ITTS_DTYPE_F32) throw std::runtime_error("Expected float32: " + n);
            if (t.ndim > 4) throw std::invalid_argument("Invalid GPT tensor rank: " + n);
            itts_tensor x{};
            x.name = t.name;
            x.data = static_cast<const float*>(t.data);
            x.ndim = t.ndim;
            for (int d = 0; d < t.ndim; ++d) x.shape[d] = t.shape[d];
            list.push_back(x);
        }
    } catch (const std::invalid_argument& e) {
        itts::g_create_error = e.what();
        return ITTS_EINVAL;
    } catch (const std::exception& e) {
        itts::g_create_error = e.what();
        return ITTS_ERUNTIME;
    }
    return itts_gpt_create(list.data(), static_cast<int32_t>(list.size()), cfg, out);
}

void itts_gpt_destroy(itts_gpt* h) { delete h; }

const char* itts_gpt_last_error(const itts_gpt* h) { return h ? h->e.last_error.c_str() : itts::g_create_error.c_str(); }

int itts_gpt_prepare(itts_gpt* h, const float* speaker, const float* emotion, const uint32_t* text, uint32_t n_text,
                     uint32_t language, float* prefix_out, uint32_t capacity_rows, uint32_t* rows) {
    return guarded(h, [&] {
        if (!h->e.has_speaker || !speaker || !emotion) throw std::invalid_argument("Invalid GPT conditioning dimensions");
        h->e.build_prefix(nullptr, 3, speaker, emotion, text, n_text, language, prefix_out, capacity_rows, rows);
    });
}

int itts_gpt_prepare_cond(itts_gpt* h, const float* cond, uint32_t n_cond, const uint32_t* text, uint32_t n_text,
                          uint32_t language, float* prefix_out, uint32_t capacity_rows, uint32_t* rows) {
    return guarded(h, [&] {
        if (!cond || !n_cond) throw std::invalid_argument("Invalid GPT conditioning dimensions");
        h->e.build_prefix(cond, n_cond, nullptr, nullptr, text, n_text, language, prefix_out, capacity_rows, rows);
    });
}

int itts_gpt_prefill(itts_gpt* h, const float* prefix, uint32_t rows, float* logits) {
    return guarded(h, [&] {
        if (!prefix) throw std::invalid_argument("Invalid GPT prefill dimensions");
        h->e.prefill(prefix, rows, logits);
    });
}

int itts_gpt_step(itts_gpt* h, uint32_t code, uint32_t position, float* logits) {
    return guarded(h, [&] { h->e.step(code, position, logits); });
}

uint32_t itts_gpt_cached_tokens(const itts_gpt* h) { return h->e.cached; }

int itts_gpt_checkpoint(itts_gpt* h, itts_gpt_state** out) {
    return guarded(h, [&] {
        auto s = std::make_unique<itts_gpt_state>();
        s->s.reset(h->e.checkpoint());
        *out = s.release();
    });
}

int itts_gpt_restore(itts_gpt* h, const itts_gpt_state* state) {
    return guarded(h, [&] {
        if (!state || !state->s) throw std::invalid_argument("Invalid KV restore");
        h->e.restore(*state->s);
    });
}

uint32_t itts_gpt_state_tokens(const itts_gpt_state* state) { return state && state->s ? state->s->tokens : 0; }
void itts_gpt_state_release(itts_gpt_state* state) { delete state; }

int itts_gpt_generate(itts_gpt* h, const float* prefix, uint32_t rows, const itts_gen_options* options, uint32_t max_tokens,
                      uint32_t* codes_out, uint32_t* n_codes, int32_t* stopped) {
    return guarded(h, [&] {
        if (!prefix) throw std::invalid_argument("Invalid GPT prefill dimensions");
        h->e.generate(prefix, rows, *options, max_tokens, codes_out, n_codes, stopped);
    });
}

int itts_gpt_generate_noalloc(itts_gpt* h, const float* prefix, uint32_t rows, const itts_gen_options* options,
                              uint32_t max_tokens, uint32_t* codes_out, uint32_t* n_codes, int32_t* stopped) {
    return guarded(h, [&] {
        if (!prefix || !options || !codes_out || !n_codes || !stopped) throw std::invalid_argument("Invalid GPT prefill dimensions");
        h->e.generate_noalloc(prefix, rows, *options, max_tokens, codes_out, n_codes, stopped);
    });
}

int itts_gpt_generate_batch(itts_gpt* h, uint32_t batch, const float* const* prefixes, const uint32_t* rows,
                            const itts_gen_options* options, uint32_t max_tokens, uint32_t* codes_out, uint32_t* n_codes,
                            int32_t* stopped) {
    return guarded(h, [&] {
        std::vector<const float*> p(prefixes, prefixes + batch);
        for (const float* x : p)
            if (!x) throw std::invalid_argument("Invalid GPT prefill dimensions");
        std::vector<uint32_t> r(rows, rows + batch);
        std::vector<itts_gen_options> o(options, options + batch);
        h->e.generate_batch(p, r, o, max_tokens, codes_out, n_codes, stopped);
    });
}

int itts_gpt_generate_segments(itts_gpt* h, const float* speaker, const float* emotion, const uint32_t* ids,
                               const uint32_t* id_counts, uint32_t n_segments, uint32_t language, const itts_gen_options* options,
                               uint32_t max_tokens, uint32_t* codes_out, uint32_t* n_codes, int32_t* stopped) {
    return guarded(h, [&] {
        if (!h->e.has_speaker || !speaker || !emotion) throw std::invalid_argument("Invalid GPT conditioning dimensions");
        h->e.generate_segments(nullptr, 3, speaker, emotion, ids, id_counts, n_segments, language, *options, max_tokens, codes_out,
                               n_codes, stopped);
    });
}

int itts_gpt_generate_segments_cond(itts_gpt* h, const float* cond, uint32_t n_cond, const uint32_t* ids, const uint32_t* id_counts,
                                    uint32_t n_segments, uint32_t language, const itts_gen_options* options, uint32_t max_tokens,
                                    uint32_t* codes_out, uint32_t* n_codes, int32_t* stopped) {
    return guarded(h, [&] {
        if (!cond || !n_cond) throw std::invalid_argument("Invalid GPT conditioning dimensions");
        h->e.generate_segments(cond, n_cond, nullptr, nullptr, ids, id_counts, n_segments, language, *options, max_tokens, codes_out,
                               n_codes, stopped);
    });
}

int itts_gpt_apply_processors(itts_gpt* h, const float* logits, uint32_t vocab, const uint32_t* history, uint32_t n_history,
                              const itts_gen_options* options, float* out) {
    return guarded(h, [&] { h->e.apply_processors(logits, vocab, history, n_history, *options, out); });
}

int itts_gpt_sample(itts_gpt* h, const float* processed, uint32_t vocab, uint64_t* rng_state, uint32_t draws, uint32_t* tokens) {
    return guarded(h, [&] { h->e.sample(processed, vocab, rng_state, draws, tokens); });
}

int itts_gpt_bench_kernel(itts_gpt* h, int32_t which, uint32_t batch, uint32_t cached_rows, uint32_t iters, float* avg_ms,
                          double* bytes_per_launch) {
    return guarded(h, [&] {
        h->e.bench_kernel(which, static_cast<int>(batch), cached_rows, static_cast<int>(iters), avg_ms, bytes_per_launch);
    });
}

int itts_gpt_step_phases(itts_gpt* h, uint32_t cached_rows, uint32_t iters, float* phase_us) {
    return guarded(h, [&] {
        if (!phase_us) throw std::invalid_argument("Invalid kernel benchmark request");
        h->e.step_phases(cached_rows, static_cast<int>(iters), phase_us);
    });
}

int itts_gpt_step_phases_batch(itts_gpt* h, uint32_t nseq, uint32_t cached_rows, uint32_t iters, float* phase_us) {
    return guarded(h, [&] {
        if (!phase_us || nseq < 2 || nseq > static_cast<uint32_t>(itts::kStepBatchMax)) throw std::invalid_argument("Invalid kernel benchmark request");
        h->e.step_phases(cached_rows, static_cast<int>(iters), phase_us, static_cast<int>(nseq));
    });
}

int itts_gpt_last_timing(const itts_gpt* h, itts_gpt_timing* out) {
    if (!h || !out) return ITTS_EINVAL;
    *out = h->e.timing;
    return ITTS_OK;
}

void itts_synthetic_normal(float* out, size_t n, uint64_t seed, float mean, float stddev) {
    auto mix = [](uint64_t z) {
        z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
        z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
        return z ^ (z >> 31);
    };
    const unsigned threads = std::max(1u, std::min(16u, std::thread::hardware_concurrency()));
    std::vector<std::thread> pool;
    for (unsigned t = 0; t < threads; ++t) {
        pool.emplace_back([=] {
            const size_t lo = n * t / threads, hi = n * (t + 1) / threads;
            for (size_t i = lo; i < hi; ++i) {
                // SplitMix64 outputs 2i and 2i+1 of the stream seeded with `seed`.
                const uint64_t a = mix(seed + (2 * i + 1) * 0x9E3779B97F4A7C15ull);
                const uint64_t b = mix(seed + (2 * i + 2) * 0x9E3779B97F4A7C15ull);
                const double u1 = (static_cast<double>(a >> 11) + 1.0) * (1.0 / 9007199254740992.0);
                const double u2 = static_cast<double>(b >> 11) * (1.0 / 9007199254740992.0);
                const double z = std::sqrt(-2.0 * std::log(u1)) * std::cos(6.283185307179586 * u2);
                out[i] = static_cast<float>(mean + stddev * z);
            }
        });
    }
    for (auto& th : pool) th.join();
}

}  // extern "C"
