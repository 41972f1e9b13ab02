// Qwen2 decoder step over the paged KV cache. Per layer, for the T new tokens
// of a step (hf Qwen2DecoderLayer order):
//   h = rms_norm(x) ; qkv = h Wqkv^T ; q,k = rope(q+bq, k+bk), v+bv
//   k,v written into the layer's pages (same kernel) ; a = paged_attention(q)
//   x += a Wo^T                      (residual folded into the GEMM)
//   h = rms_norm(x) ; gu = h [Wg;Wu]^T ; act = up * silu(gate)
//   x += act Wd^T
// then, for each sequence's last token: logits = rms_norm(x) Wlm^T, argmax.
#include "qwen2.hpp"

#include "../common.hpp"
#include "../core/core.hpp"
#include "../kernels/launch.hpp"
#include "../device/hip_check.hpp"
#include "../ops/ops.hpp"

#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdlib>
#include <cstring>

namespace llaisys::models {

namespace K = llaisys::kernels;

namespace {

// KV pages handed out in the block manager's scattered order unless
// LLAISYS_KV_SCATTER=0.
bool scatterBlocks() {
    const char *e = std::getenv("LLAISYS_KV_SCATTER");
    return !(e && e[0] == '0');
}

// Steps with at most this many token rows use the folded-norm projections.
constexpr size_t kFoldMaxRows = 512;
bool takesDecodeGemm(const tensor_t &packed, int M, int N, int K);

tensor_t dev(std::vector<size_t> shape, llaisysDataType_t dt, int id) {
    return Tensor::create(shape, dt, LLAISYS_DEVICE_AMD, id);
}
uint16_t *u16(const tensor_t &t) { return reinterpret_cast<uint16_t *>(t->data()); }
int64_t *i64(const tensor_t &t) { return reinterpret_cast<int64_t *>(t->data()); }
int32_t *i32(const tensor_t &t) { return reinterpret_cast<int32_t *>(t->data()); }
tensor_t rows(const tensor_t &t, size_t n) { return t->slice(0, 0, n); }

// Stream-ordered error-flag snapshots around one model call: slot 0 (taken
// on construction) holds the bits earlier calls raised, slot 1 (end()) this
// call's; collect() reads both after the call's own stream sync. If the call
// throws in between, the destructor waits for the stream and keeps whatever
// was snapshotted for llaisysGetDeviceErrorFlags, as the device word would
// have.
class FlagSnapshots {
public:
    explicit FlagSnapshots(core::Runtime &rt) : rt_(rt) { rt_.flagSnapshotAsync(0); }
    void end() {
        rt_.flagSnapshotAsync(1);
        ended_ = true;
    }
    int collect() {
        rt_.addPendingErrorFlags(rt_.flagSnapshot(0));
        collected_ = true;
        return rt_.flagSnapshot(1);
    }
    ~FlagSnapshots() {
        if (collected_) return;
        try {
            rt_.api()->stream_synchronize(rt_.stream());
            rt_.addPendingErrorFlags(rt_.flagSnapshot(0) | (ended_ ? rt_.flagSnapshot(1) : 0));
        } catch (...) {
        }
    }

private:
    core::Runtime &rt_;
    bool ended_ = false, collected_ = false;
};

// Y[M, N] = X W^T (+ bias) (+ Y) through the MFMA GEMM over row-major W.
void gemm(const tensor_t &y, const tensor_t &x, const tensor_t &w, const tensor_t &bias, int M, int N, int K,
          bool accumulate, void *s) {
    void *ws = core::context().runtime().scratch(K::linearWorkspaceBytes(K::ElemType::BF16, M, N, K));
    K::linear(y->data(), x->data(), w->data(), bias ? bias->data() : nullptr, K::ElemType::BF16, M, N, K, s,
              accumulate, ws);
}

} // namespace

Qwen2Model::Qwen2Model(const Qwen2Config &cfg, int device_id, size_t num_blocks)
    : cfg_(cfg), dev_(device_id), num_blocks_(num_blocks), blocks_(int(num_blocks), scatterBlocks()) {
    LLAISYS_CHECK(cfg.dtype == LLAISYS_DTYPE_BF16, "qwen2: the paged KV path runs bf16 models (meta.dtype)");
    LLAISYS_CHECK(cfg.dh == size_t(K::kHeadDim), "qwen2: head dim must be " << K::kHeadDim << ", got " << cfg.dh);
    LLAISYS_CHECK(cfg.nlayer > 0 && cfg.hs > 0 && cfg.nh > 0 && cfg.nkvh > 0 && cfg.di > 0 && cfg.voc > 0,
                  "qwen2: meta sizes must be positive");
    LLAISYS_CHECK(cfg.nh % cfg.nkvh == 0 && cfg.nh / cfg.nkvh <= 16, "qwen2: need nh % nkvh == 0, nh / nkvh <= 16");
    LLAISYS_CHECK(cfg.di % 8 == 0 && cfg.hs % 8 == 0, "qwen2: hs and di must be multiples of 8");
    LLAISYS_CHECK(num_blocks > 0 && num_blocks < (size_t(1) << 31), "qwen2: bad KV block count " << num_blocks);
    core::context().setDevice(LLAISYS_DEVICE_AMD, dev_);
    if (const char *e = std::getenv("LLAISYS_QWEN2_GRAPHS")) use_graphs_ = e[0] != '0';
    if (const char *e = std::getenv("LLAISYS_QWEN2_FOLD_NORM")) fold_norm_ = e[0] != '0';
    if (const char *e = std::getenv("LLAISYS_DECODE_GEMM")) decode_gemm_ = e[0] != '0';
    if (const char *e = std::getenv("LLAISYS_DECODE_UNITS")) unit_decode_allowed_ = e[0] != '0';
    unit_rope_ = K::decodeUnitsRopeSupported(int(cfg.nh), int(cfg.nkvh), int(cfg.dh));
    if (const char *e = std::getenv("LLAISYS_DECODE_UNIT_ROPE")) unit_rope_ = unit_rope_ && e[0] != '0';
    if (const char *e = std::getenv("LLAISYS_PACKED_X")) packed_x_ = e[0] != '0';
    if (const char *e = std::getenv("LLAISYS_QKV_GEMM_EPILOGUE")) qkv_gemm_epilogue_ = e[0] != '0';
    if (const char *e = std::getenv("LLAISYS_SPLITK_PACKED")) splitk_packed_ = e[0] != '0';
    if (const char *e = std::getenv("LLAISYS_GEMM_SWIGLU")) gemm_swiglu_ = e[0] != '0';
    gemm_swiglu_ = gemm_swiglu_ && K::linearSwigluSupported(K::ElemType::BF16, 1, int(cfg.di), int(cfg.hs));
    const auto dt = cfg.dtype;
    const size_t q = cfg.nh * cfg.dh, kv = cfg.nkvh * cfg.dh;
    in_embed_ = dev({cfg.voc, cfg.hs}, dt, dev_);
    out_embed_ = dev({cfg.voc, cfg.hs}, dt, dev_);
    out_norm_ = dev({cfg.hs}, dt, dev_);
    layers_.resize(cfg.nlayer);
    for (auto &L : layers_) {
        L.attn_norm = dev({cfg.hs}, dt, dev_);
        L.qkv_w = dev({q + 2 * kv, cfg.hs}, dt, dev_);
        L.qkv_b = dev({q + 2 * kv}, dt, dev_);
        L.o_w = dev({cfg.hs, q}, dt, dev_);
        L.mlp_norm = dev({cfg.hs}, dt, dev_);
        L.gate_up_w = dev({2 * cfg.di, cfg.hs}, dt, dev_);
        L.down_w = dev({cfg.hs, cfg.di}, dt, dev_);
        L.q_w = L.qkv_w->slice(0, 0, q);
        L.k_w = L.qkv_w->slice(0, q, q + kv);
        L.v_w = L.qkv_w->slice(0, q + kv, q + 2 * kv);
        L.q_b = L.qkv_b->slice(0, 0, q);
        L.k_b = L.qkv_b->slice(0, q, q + kv);
        L.v_b = L.qkv_b->slice(0, q + kv, q + 2 * kv);
        L.gate_w = L.gate_up_w->slice(0, 0, cfg.di);
        L.up_w = L.gate_up_w->slice(0, cfg.di, 2 * cfg.di);
        if (fold_norm_) {
            L.qkv_wf = dev({q + 2 * kv, cfg.hs}, dt, dev_);
            L.gate_up_wf = dev({2 * cfg.di, cfg.hs}, dt, dev_);
        }
        if (decode_gemm_ && fold_norm_ && K::decodeGemmSupported(1, int(q + 2 * kv), int(cfg.hs)) &&
            K::decodeGemmSupported(1, int(2 * cfg.di), int(cfg.hs))) {
            L.qkv_wfp = dev({q + 2 * kv, cfg.hs}, dt, dev_);
            L.gate_up_wfp = dev({2 * cfg.di, cfg.hs}, dt, dev_);
        }
        if (gemm_swiglu_) L.gate_up_wi = dev({2 * cfg.di, cfg.hs}, dt, dev_);
        if (decode_gemm_ && K::decodeGemmSupported(1, int(cfg.hs), int(q))) L.o_wp = dev({cfg.hs, q}, dt, dev_);
        if (decode_gemm_ && K::splitKGemmSupported(1, int(cfg.hs), int(cfg.di)))
            L.down_wp = dev({cfg.hs, cfg.di}, dt, dev_);
    }
    if (decode_gemm_ && K::decodeGemmSupported(1, int(cfg.voc), int(cfg.hs))) out_embed_p_ = dev({cfg.voc, cfg.hs}, dt, dev_);
    for (size_t l = 0; l < cfg.nlayer; ++l) {
        k_pool_.push_back(dev({num_blocks, cfg.nkvh, size_t(K::kPageTokens), cfg.dh}, LLAISYS_DTYPE_BF16, dev_));
        v_pool_.push_back(dev({num_blocks, cfg.nkvh, size_t(K::kPageTokens), cfg.dh}, LLAISYS_DTYPE_BF16, dev_));
    }
}

Qwen2Model::~Qwen2Model() {
    for (auto *m : {&graphs_, &multi_graphs_})
        for (auto &kv : *m)
            if (kv.second.exec) (void)hipGraphExecDestroy(static_cast<hipGraphExec_t>(kv.second.exec));
}

// Decode steps of one batch size replay a captured graph of forward(): same
// kernels, same arguments, the per-step indices read from the same device
// buffers. A graph is (re)captured when the table width, any workspace buffer
// or the runtime's split workspace moved; the step that captures runs eagerly
// first (so workspace growth happens outside the capture) and its results are the eager ones.
Qwen2Model::DecodeGraph Qwen2Model::capture(const std::function<void()> &work, size_t width) {
    auto &rt = core::context().runtime();
    auto s = static_cast<hipStream_t>(rt.stream());
    hipGraph_t graph = nullptr;
    HIP_CHECK(hipStreamBeginCapture(s, hipStreamCaptureModeThreadLocal));
    try {
        work();
    } catch (...) {
        (void)hipStreamEndCapture(s, &graph);
        if (graph) (void)hipGraphDestroy(graph);
        throw;
    }
    HIP_CHECK(hipStreamEndCapture(s, &graph));
    hipGraphExec_t exec = nullptr;
    const hipError_t e = hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0);
    (void)hipGraphDestroy(graph);
    HIP_CHECK(e);
    DecodeGraph g;
    g.exec = exec;
    g.width = width;
    g.gen = ws_gen_;
    g.ws = rt.workspaceGeneration();
    g.unit = unit_decode_;
    return g;
}

// Decode steps (B > 0) of at least kUnitDecodeMinUnits units whose lengths
// stay within 2x: every unit's workgroup then finishes at about the same
// time, and the one-launch kernel saves the stream-K kernel's length scan,
// split records and combine launch. Other batches (mixed lengths, few
// sequences, prefill) keep the stream-K kernel.
static constexpr size_t kUnitDecodeMinUnits = 128;

void Qwen2Model::chooseDecodeAttention(size_t B, int32_t min_ctx, int32_t max_ctx) {
    unit_decode_ = unit_decode_allowed_ && B > 0 && B * cfg_.nkvh >= kUnitDecodeMinUnits && min_ctx >= 1 &&
                   max_ctx <= 2 * min_ctx;
}

void Qwen2Model::decodeGraph(size_t B, size_t width) {
    auto &rt = core::context().runtime();
    auto s = static_cast<hipStream_t>(rt.stream());
    DecodeGraph &g = graphs_[B];
    if (g.exec && g.width == width && g.gen == ws_gen_ && g.ws == rt.workspaceGeneration() && g.unit == unit_decode_) {
        HIP_CHECK(hipGraphLaunch(static_cast<hipGraphExec_t>(g.exec), s));
        return;
    }
    if (g.exec) {
        HIP_CHECK(hipGraphExecDestroy(static_cast<hipGraphExec_t>(g.exec)));
        g.exec = nullptr;
    }
    forward(B, B, true);
    g = capture([&] { forward(B, B, true); }, width);
}

void Qwen2Model::ensureWorkspace(size_t T, size_t B, size_t ints32, size_t ints64) {
    auto &rt = core::context().runtime();
    const auto dt = cfg_.dtype;
    if (T > cap_T_) {
        const size_t cap = std::max(T, cap_T_ * 2);
        const size_t q = cfg_.nh * cfg_.dh, kv = cfg_.nkvh * cfg_.dh;
        rt.api()->device_synchronize();
        x_ = dev({cap, cfg_.hs}, dt, dev_);
        h_ = dev({cap, cfg_.hs}, dt, dev_);
        qkv_ = dev({cap, q + 2 * kv}, dt, dev_);
        q_ = dev({cap, cfg_.nh, cfg_.dh}, dt, dev_);
        attn_ = dev({cap, cfg_.nh, cfg_.dh}, dt, dev_);
        xp_ = dev({K::packedRowsElems(int(cap), int(cfg_.hs))}, dt, dev_);
        ap_ = dev({K::packedRowsElems(int(cap), int(q))}, dt, dev_);
        actp_ = dev({K::packedRowsElems(int(cap), int(cfg_.di))}, dt, dev_);
        gu_ = dev({cap, 2 * cfg_.di}, dt, dev_);
        act_ = dev({cap, cfg_.di}, dt, dev_);
        cap_T_ = cap;
        ++ws_gen_;
    }
    if (B > cap_B_) {
        const size_t cap = std::max(B, cap_B_ * 2);
        rt.api()->device_synchronize();
        hl_ = dev({cap, cfg_.hs}, dt, dev_);
        logits_ = dev({cap, cfg_.voc}, dt, dev_);
        next_ = dev({cap}, LLAISYS_DTYPE_I64, dev_);
        cap_B_ = cap;
        ++ws_gen_;
    }
    if (ints32 > cap_i32_) {
        const size_t cap = std::max(ints32, cap_i32_ * 2);
        rt.api()->device_synchronize();
        dev_i32_ = dev({cap}, LLAISYS_DTYPE_I32, dev_);
        host32_ = rt.allocateHostStorage(cap * sizeof(int32_t));
        cap_i32_ = cap;
        ++ws_gen_;
    }
    if (ints64 + B > cap_i64_) {
        const size_t cap = std::max(ints64 + B, cap_i64_ * 2);
        rt.api()->device_synchronize();
        dev_i64_ = dev({cap}, LLAISYS_DTYPE_I64, dev_);
        host64_ = rt.allocateHostStorage(cap * sizeof(int64_t));
        cap_i64_ = cap;
        ++ws_gen_;
    }
}

// Map the pages positions [len, len + n_i) of each sequence land in; returns
// the copy-on-write (src, dst) block pairs to copy before writing, and the
// lengths before. If a reservation fails, copies already decided are made.
std::vector<int32_t> Qwen2Model::reserveAll(const int64_t *ids, size_t B, const size_t *n, std::vector<int32_t> &before) {
    auto &rt = core::context().runtime();
    std::vector<int32_t> cow;
    try {
        for (size_t i = 0; i < B; ++i) {
            before[i] = blocks_.length(ids[i]);
            int32_t pair[2];
            if (blocks_.reserve(ids[i], int(n[i]), pair, 1) == 1) cow.insert(cow.end(), pair, pair + 2);
        }
    } catch (...) {
        // A sequence already switched to its private copy of a shared block
        // must get that copy's contents even though this call fails.
        if (!cow.empty()) {
            auto pairs = Tensor::create({cow.size() / 2, 2}, LLAISYS_DTYPE_I32, LLAISYS_DEVICE_AMD, dev_);
            pairs->load(cow.data());
            for (size_t l = 0; l < cfg_.nlayer; ++l) ops::pagedKVCopyBlocks(k_pool_[l], v_pool_[l], pairs);
            rt.api()->stream_synchronize(rt.stream());
        }
        throw;
    }
    return cow;
}

void Qwen2Model::step(const int64_t *ids, size_t nseq, const int64_t *tokens, const size_t *ntokens, int64_t *next) {
    LLAISYS_CHECK(nseq > 0, "qwen2 step: no sequences");
    LLAISYS_CHECK(ids && tokens && ntokens && next, "qwen2 step: null argument");
    core::context().setDevice(LLAISYS_DEVICE_AMD, dev_);
    ensureFolded();
    auto &rt = core::context().runtime();
    // Earlier calls' bits stay for llaisysGetDeviceErrorFlags: snapshot (and
    // clear) the device word in stream order, read after the step's one sync.
    FlagSnapshots flag_snaps(rt);
    const size_t B = nseq;
    size_t T = 0;
    for (size_t i = 0; i < B; ++i) {
        LLAISYS_CHECK(ntokens[i] >= 1, "qwen2 step: sequence " << ids[i] << " appends no token");
        LLAISYS_CHECK(size_t(blocks_.length(ids[i])) + ntokens[i] <= cfg_.maxseq,
                      "qwen2 step: sequence " << ids[i] << " would exceed maxseq " << cfg_.maxseq);
        for (size_t j = 0; j < i; ++j) LLAISYS_CHECK(ids[j] != ids[i], "qwen2 step: sequence " << ids[i] << " listed twice");
        T += ntokens[i];
    }
    for (size_t i = 0; i < T; ++i)
        LLAISYS_CHECK(tokens[i] >= 0 && size_t(tokens[i]) < cfg_.voc, "qwen2 step: token id " << tokens[i] << " out of vocabulary");

    std::vector<int32_t> before(B);
    const std::vector<int32_t> cow = reserveAll(ids, B, ntokens, before);
    // Table width rounded up to 32 pages, so it (and a captured decode graph)
    // changes once per 512 tokens of the longest sequence, not every page.
    const size_t used_pages = size_t(std::max(1, blocks_.buildTable(ids, B, nullptr, 0, nullptr)));
    const size_t max_pages = (used_pages + 31) / 32 * 32;
    const size_t ncow = cow.size() / 2;
    const size_t n32 = B * max_pages + 3 * B + 1 + cow.size();
    const size_t n64 = T + B;
    ensureWorkspace(T, B, n32, n64);

    // int32 staging: table | ctx_before | ctx_after | cu | cow pairs
    int32_t *h32 = reinterpret_cast<int32_t *>(host32_->memory());
    std::vector<int32_t> ctx_scratch(B);
    blocks_.buildTable(ids, B, h32, max_pages, ctx_scratch.data());
    int32_t *cb = h32 + B * max_pages, *ca = cb + B, *cu = ca + B;
    cu[0] = 0;
    for (size_t i = 0; i < B; ++i) {
        cb[i] = before[i];
        ca[i] = before[i] + int32_t(ntokens[i]);
        cu[i + 1] = cu[i] + int32_t(ntokens[i]);
    }
    std::copy(cow.begin(), cow.end(), cu + B + 1);
    chooseDecodeAttention(T == B ? B : 0, *std::min_element(ca, ca + B), *std::max_element(ca, ca + B));
    // int64 staging: tokens | last row of each sequence
    int64_t *h64 = reinterpret_cast<int64_t *>(host64_->memory());
    std::memcpy(h64, tokens, T * sizeof(int64_t));
    for (size_t i = 0; i < B; ++i) h64[T + i] = cu[i + 1] - 1;
    auto *api = rt.api();
    api->memcpy_async(dev_i32_->data(), h32, n32 * sizeof(int32_t), LLAISYS_MEMCPY_H2D, rt.stream());
    api->memcpy_async(dev_i64_->data(), h64, n64 * sizeof(int64_t), LLAISYS_MEMCPY_H2D, rt.stream());

    table_ = dev_i32_->slice(0, 0, B * max_pages)->view({B, max_pages});
    ctx_before_ = dev_i32_->slice(0, B * max_pages, B * max_pages + B);
    ctx_after_ = dev_i32_->slice(0, B * max_pages + B, B * max_pages + 2 * B);
    cu_ = dev_i32_->slice(0, B * max_pages + 2 * B, B * max_pages + 3 * B + 1);
    cow_ = ncow ? dev_i32_->slice(0, B * max_pages + 3 * B + 1, n32)->view({ncow, 2}) : nullptr;
    tok_ = dev_i64_->slice(0, 0, T);
    last_ = dev_i64_->slice(0, T, T + B);

    if (cow_)
        for (size_t l = 0; l < cfg_.nlayer; ++l) ops::pagedKVCopyBlocks(k_pool_[l], v_pool_[l], cow_);
    const bool decode_only = T == B;
    if (decode_only && use_graphs_) {
        decodeGraph(B, max_pages);
    } else {
        forward(T, B, decode_only);
    }

    // next tokens back to the host; the staging buffers are free after this.
    int64_t *hnext = h64 + n64;
    flag_snaps.end(); // this call's kernels only
    api->memcpy_async(hnext, next_->data(), B * sizeof(int64_t), LLAISYS_MEMCPY_D2H, rt.stream());
    api->stream_synchronize(rt.stream());
    const int flags = flag_snaps.collect();
    LLAISYS_CHECK(flags == 0, "qwen2 step: kernels reported error flags " << flags);
    std::memcpy(next, hnext, B * sizeof(int64_t));
    last_B_ = B;
    for (size_t i = 0; i < B; ++i) blocks_.commit(ids[i], int(ntokens[i]), tokens + cu[i]);
}


// Multi-step greedy decode: nsteps single-token steps of the batch with the
// next token fed back on the device. Pages for all steps are reserved up
// front and the table is uploaded once; each step is decodeAdvance (the
// previous step's argmax into the history, lengths and tokens from a device
// step counter, counter + 1) and forward() - one captured graph replayed
// nsteps times - and one decodeRecordLast after the last step.
void Qwen2Model::decode(const int64_t *ids, size_t nseq, const int64_t *first, size_t nsteps, int64_t *out) {
    LLAISYS_CHECK(nseq > 0 && nsteps > 0, "qwen2 decode: no sequences or no steps");
    LLAISYS_CHECK(ids && first && out, "qwen2 decode: null argument");
    core::context().setDevice(LLAISYS_DEVICE_AMD, dev_);
    ensureFolded();
    auto &rt = core::context().runtime();
    FlagSnapshots flag_snaps(rt); // earlier calls' bits, read after the call's one sync
    const size_t B = nseq;
    for (size_t i = 0; i < B; ++i) {
        LLAISYS_CHECK(size_t(blocks_.length(ids[i])) + nsteps <= cfg_.maxseq,
                      "qwen2 decode: sequence " << ids[i] << " would exceed maxseq " << cfg_.maxseq);
        for (size_t j = 0; j < i; ++j)
            LLAISYS_CHECK(ids[j] != ids[i], "qwen2 decode: sequence " << ids[i] << " listed twice");
        LLAISYS_CHECK(first[i] >= 0 && size_t(first[i]) < cfg_.voc,
                      "qwen2 decode: token id " << first[i] << " out of vocabulary");
    }
    std::vector<int32_t> before(B);
    const std::vector<size_t> counts(B, nsteps);
    const std::vector<int32_t> cow = reserveAll(ids, B, counts.data(), before);
    const size_t used_pages = size_t(std::max(1, blocks_.buildTable(ids, B, nullptr, 0, nullptr)));
    const size_t width = (used_pages + 31) / 32 * 32;
    const size_t ncow = cow.size() / 2;
    // int32: table | ctx_before | ctx_after | cu | base | counter | cow ; int64: tok | last | first | history
    const size_t o_cb = B * width, o_ca = o_cb + B, o_cu = o_ca + B, o_base = o_cu + B + 1, o_cnt = o_base + B;
    const size_t n32 = o_cnt + 1 + cow.size();
    const size_t n64 = 3 * B + nsteps * B;
    ensureWorkspace(B, B, n32, n64);
    int32_t *h32 = reinterpret_cast<int32_t *>(host32_->memory());
    std::vector<int32_t> ctx_scratch(B);
    blocks_.buildTable(ids, B, h32, width, ctx_scratch.data());
    for (size_t i = 0; i < B; ++i) {
        h32[o_cb + i] = before[i];
        h32[o_ca + i] = before[i] + 1;
        h32[o_cu + i] = int32_t(i);
        h32[o_base + i] = before[i];
    }
    h32[o_cu + B] = int32_t(B);
    h32[o_cnt] = 0;
    // Every step of the call runs one captured graph: choose for the range
    // of lengths the call spans.
    chooseDecodeAttention(B, *std::min_element(before.begin(), before.end()) + 1,
                          *std::max_element(before.begin(), before.end()) + int32_t(nsteps));
    std::copy(cow.begin(), cow.end(), h32 + o_cnt + 1);
    int64_t *h64 = reinterpret_cast<int64_t *>(host64_->memory());
    for (size_t i = 0; i < B; ++i) {
        h64[i] = first[i];
        h64[B + i] = int64_t(i);
        h64[2 * B + i] = first[i];
    }
    auto *api = rt.api();
    api->memcpy_async(dev_i32_->data(), h32, n32 * sizeof(int32_t), LLAISYS_MEMCPY_H2D, rt.stream());
    api->memcpy_async(dev_i64_->data(), h64, 3 * B * sizeof(int64_t), LLAISYS_MEMCPY_H2D, rt.stream());

    table_ = dev_i32_->slice(0, 0, B * width)->view({B, width});
    ctx_before_ = dev_i32_->slice(0, o_cb, o_cb + B);
    ctx_after_ = dev_i32_->slice(0, o_ca, o_ca + B);
    cu_ = dev_i32_->slice(0, o_cu, o_cu + B + 1);
    cow_ = ncow ? dev_i32_->slice(0, o_cnt + 1, n32)->view({ncow, 2}) : nullptr;
    tok_ = dev_i64_->slice(0, 0, B);
    last_ = dev_i64_->slice(0, B, 2 * B);
    auto *base = reinterpret_cast<int32_t *>(dev_i32_->data()) + o_base;
    auto *counter = reinterpret_cast<int32_t *>(dev_i32_->data()) + o_cnt;
    auto *first_d = reinterpret_cast<int64_t *>(dev_i64_->data()) + 2 * B;
    auto *history = reinterpret_cast<int64_t *>(dev_i64_->data()) + 3 * B;
    if (cow_)
        for (size_t l = 0; l < cfg_.nlayer; ++l) ops::pagedKVCopyBlocks(k_pool_[l], v_pool_[l], cow_);

    void *s = rt.stream();
    auto oneStep = [&] {
        K::decodeAdvance(i32(ctx_before_), i32(ctx_after_), i64(tok_), history, base, first_d, i64(next_), counter,
                         int(B), s);
        forward(B, B, true);
    };
    size_t done = 0;
    if (use_graphs_) {
        DecodeGraph &g = multi_graphs_[B];
        const bool valid = g.exec && g.width == width && g.gen == ws_gen_ && g.ws == rt.workspaceGeneration() &&
                           g.unit == unit_decode_;
        if (!valid) {
            if (g.exec) HIP_CHECK(hipGraphExecDestroy(static_cast<hipGraphExec_t>(g.exec)));
            g.exec = nullptr;
            oneStep(); // eager: workspace growth stays outside the capture
            done = 1;
            g = capture(oneStep, width);
        }
        for (; done < nsteps; ++done) HIP_CHECK(hipGraphLaunch(static_cast<hipGraphExec_t>(g.exec), static_cast<hipStream_t>(s)));
    } else {
        for (; done < nsteps; ++done) oneStep();
    }
    K::decodeRecordLast(history, i64(next_), counter, int(B), s);

    int64_t *hout = h64 + 3 * B;
    flag_snaps.end(); // this call's kernels only
    api->memcpy_async(hout, history, nsteps * B * sizeof(int64_t), LLAISYS_MEMCPY_D2H, s);
    api->stream_synchronize(s);
    const int flags = flag_snaps.collect();
    LLAISYS_CHECK(flags == 0, "qwen2 decode: kernels reported error flags " << flags);
    std::memcpy(out, hout, nsteps * B * sizeof(int64_t));
    last_B_ = B;
    std::vector<int64_t> fed(nsteps);
    for (size_t i = 0; i < B; ++i) {
        fed[0] = first[i];
        for (size_t t = 1; t < nsteps; ++t) fed[t] = out[(t - 1) * B + i];
        blocks_.commit(ids[i], int(nsteps), fed.data());
    }
}

void Qwen2Model::ensureFolded() {
    void *s = core::context().runtime().stream();
    // Packed copies for the decode GEMM: o_w and the LM head from their own
    // versions, the folded projections whenever they are refolded below.
    if (out_embed_p_ && out_embed_->version() != out_embed_packed_from_) {
        K::packWeight(u16(out_embed_p_), u16(out_embed_), nullptr, int(cfg_.voc), int(cfg_.hs), s);
        out_embed_packed_from_ = out_embed_->version();
    }
    for (auto &L : layers_) {
        if (L.o_wp && L.o_w->version() != L.o_packed_from) {
            K::packWeight(u16(L.o_wp), u16(L.o_w), nullptr, int(L.o_w->shape()[0]), int(L.o_w->shape()[1]), s);
            L.o_packed_from = L.o_w->version();
        }
        if (L.down_wp && L.down_w->version() != L.down_packed_from) {
            K::packWeight(u16(L.down_wp), u16(L.down_w), nullptr, int(L.down_w->shape()[0]),
                          int(L.down_w->shape()[1]), s);
            L.down_packed_from = L.down_w->version();
        }
        if (L.gate_up_wi && L.gate_up_w->version() != L.interleaved_from) {
            K::swigluInterleave(u16(L.gate_up_wi), u16(L.gate_up_w), int(cfg_.di), int(cfg_.hs), s);
            L.interleaved_from = L.gate_up_w->version();
        }
    }
    if (!fold_norm_) return;
    for (auto &L : layers_) {
        const uint64_t v[4] = {L.qkv_w->version(), L.attn_norm->version(), L.gate_up_w->version(),
                               L.mlp_norm->version()};
        if (v[0] != L.folded_from[0] || v[1] != L.folded_from[1]) {
            K::foldNormColumns(u16(L.qkv_wf), u16(L.qkv_w), u16(L.attn_norm), L.qkv_w->shape()[0], int(cfg_.hs), s);
            if (L.qkv_wfp)
                K::packWeight(u16(L.qkv_wfp), u16(L.qkv_wf), nullptr, int(L.qkv_w->shape()[0]), int(cfg_.hs), s);
            L.folded_from[0] = v[0];
            L.folded_from[1] = v[1];
        }
        if (v[2] != L.folded_from[2] || v[3] != L.folded_from[3]) {
            K::foldNormColumns(u16(L.gate_up_wf), u16(L.gate_up_w), u16(L.mlp_norm), L.gate_up_w->shape()[0],
                               int(cfg_.hs), s);
            // Gate and up rows interleaved per 16-row block, so that each
            // block of the product finishes its own SwiGLU columns.
            if (L.gate_up_wfp) K::packWeightGateUp(u16(L.gate_up_wfp), u16(L.gate_up_wf), int(cfg_.di), int(cfg_.hs), s);
            L.folded_from[2] = v[2];
            L.folded_from[3] = v[3];
        }
    }
}

void Qwen2Model::forward(size_t T, size_t B, bool decode_only) {
    auto &rt = core::context().runtime();
    void *s = rt.stream();
    const auto et = K::ElemType::BF16;
    const int hs = int(cfg_.hs), di = int(cfg_.di);
    const int q = int(cfg_.nh * cfg_.dh), kv = int(cfg_.nkvh * cfg_.dh);
    const int M = int(T);
    const float scale = 1.f / std::sqrt(float(cfg_.dh));

    // Packed-operand decode path: qkv and o read x and the attention output
    // in MFMA operand order, written beside their rows by the embedding, the
    // down projection's split-K reduce and the attention itself.
    // Batches of unequal lengths (stream-K attention, not one workgroup per
    // unit) take it too when the QKV epilogue runs in the projection: the
    // stream-K kernels then write their rows packed as well.
    const auto &L0 = layers_[0];
    const bool qkv_epi_ok = qkv_gemm_epilogue_ && K::qkvRopeGemmSupported(M, int(cfg_.nh), int(cfg_.nkvh), hs);
    const bool px = packed_x_ && decode_only && ((unit_decode_ && unit_rope_) || qkv_epi_ok) && fold_norm_ &&
                    T <= kFoldMaxRows && cfg_.dtype == LLAISYS_DTYPE_BF16 && L0.qkv_wfp && L0.o_wp && L0.down_wp &&
                    K::packedXGemmSupported(M, q + 2 * kv, hs) && K::packedXGemmSupported(M, hs, q) &&
                    K::splitKGemmSupported(M, hs, di);
    // On that path the gate-up projection, the row's 1/rms and the SwiGLU
    // run as one kernel over the packed x the o projection leaves.
    const bool fused_mlp = px && L0.gate_up_wfp && K::gateUpSwigluSupported(M, di, hs);
    // and the QKV epilogue runs in the QKV projection's epilogue.
    const bool qkv_epi = px && qkv_epi_ok;
    // and the down projection reads the SwiGLU output packed.
    const bool down_px = fused_mlp && splitk_packed_ && K::splitKPackedSupported(M, hs, di) && di % 32 == 0;
    if (px)
        K::embedRowsPacked(u16(x_), u16(xp_), i64(tok_), u16(in_embed_), M, int64_t(cfg_.voc), hs, rt.errorWord(),
                           s);
    else
        K::embedding(x_->data(), i64(tok_), in_embed_->data(), et, T, int64_t(cfg_.voc), hs, rt.errorWord(), s);
    const tensor_t q3 = rows(q_, T), a3 = rows(attn_, T);
    for (size_t l = 0; l < cfg_.nlayer; ++l) {
        const auto &L = layers_[l];
        // Folded norms (decode-sized steps): the projections read the residual
        // x itself and the next kernel applies each row's 1/rms (see
        // foldNormColumns). Every wave of those kernels reduces its row again,
        // which costs more than one rms_norm launch once a step holds
        // thousands of rows, so long prefill steps keep the separate launch.
        const bool fold = fold_norm_ && T <= kFoldMaxRows;
        const uint16_t *xr = fold ? u16(x_) : nullptr;
        if (!fold) K::rmsNormRows(u16(h_), u16(x_), nullptr, u16(L.attn_norm), T, hs, cfg_.epsilon, s);
        if (qkv_epi) {
            // QKV epilogue (bias, 1/rms, RoPE, k/v append) in the projection's
            // own epilogue, then the attention reading q.
            K::qkvRopeGemm(u16(q_), u16(k_pool_[l]), u16(v_pool_[l]), u16(xp_), u16(L.qkv_wfp), u16(L.qkv_b),
                           i32(table_), i32(ctx_before_), M, int(cfg_.nh), int(cfg_.nkvh), hs,
                           int(table_->shape()[1]), int(num_blocks_), cfg_.epsilon, cfg_.theta, rt.errorWord(), s);
            if (unit_decode_) {
                K::pagedDecodeUnits(a3->data(), false, u16(q3), u16(k_pool_[l]), u16(v_pool_[l]), i32(table_),
                                    i32(ctx_after_), int(B), int(cfg_.nh), int(cfg_.nkvh), int(table_->shape()[1]),
                                    int(num_blocks_), scale, rt.errorWord(), s, u16(ap_));
            } else {
                const int max_pages = int(table_->shape()[1]);
                const auto plan = K::planDecode(int(B), int(cfg_.nkvh), int(cfg_.nh / cfg_.nkvh), max_pages);
                auto *records = static_cast<float *>(rt.scratch(plan.record_bytes));
                K::pagedDecode(a3->data(), false, u16(q3), u16(k_pool_[l]), u16(v_pool_[l]), i32(table_),
                               i32(ctx_after_), nullptr, int(B), int(B), int(cfg_.nh), int(cfg_.nkvh), max_pages,
                               int(num_blocks_), scale, plan, records, rt.errorWord(),
                               plan.slot_headers ? rt.decodeSlotHeaders(plan.slot_headers) : nullptr,
                               plan.slot_headers ? rt.decodeSlotRecords(plan.slot_record_bytes) : nullptr, s,
                               u16(ap_));
            }
        } else if (px)
            K::packedXGemm(u16(qkv_), u16(xp_), u16(L.qkv_wfp), M, q + 2 * kv, hs, false, s);
        else
            project(qkv_, fold ? x_ : h_, fold ? L.qkv_wf : L.qkv_w, fold ? L.qkv_wfp : nullptr, M, q + 2 * kv, hs,
                    false, s);
        if (!qkv_epi && decode_only && unit_decode_ && unit_rope_) {
            // QKV epilogue (bias, 1/rms, RoPE, k/v append) inside the attention
            // launch: one kernel fewer per layer.
            K::pagedDecodeUnitsRope(a3->data(), false, u16(k_pool_[l]), u16(v_pool_[l]), u16(qkv_), u16(L.qkv_b), xr,
                                    hs, cfg_.epsilon, cfg_.theta, i32(table_), i32(ctx_after_), int(B),
                                    int(cfg_.nh), int(cfg_.nkvh), int(table_->shape()[1]), int(num_blocks_), scale,
                                    rt.errorWord(), s, px ? u16(ap_) : nullptr);
        } else if (!qkv_epi) {
            K::qkvRopeAppend(u16(q_), u16(k_pool_[l]), u16(v_pool_[l]), u16(qkv_), u16(L.qkv_b), i32(table_),
                             i32(ctx_before_), decode_only ? nullptr : i32(cu_), M, int(B), int(cfg_.nh),
                             int(cfg_.nkvh), int(cfg_.dh), int(table_->shape()[1]), int(num_blocks_), cfg_.theta,
                             rt.errorWord(), xr, hs, cfg_.epsilon, s);
            if (decode_only && unit_decode_)
                K::pagedDecodeUnits(a3->data(), false, u16(q3), u16(k_pool_[l]), u16(v_pool_[l]), i32(table_),
                                    i32(ctx_after_), int(B), int(cfg_.nh), int(cfg_.nkvh), int(table_->shape()[1]),
                                    int(num_blocks_), scale, rt.errorWord(), s);
            else
                ops::pagedAttention(a3, q3, k_pool_[l], v_pool_[l], table_, ctx_after_, decode_only ? nullptr : cu_,
                                    scale);
        }
        if (px)
            K::packedXGemm(u16(x_), u16(ap_), u16(L.o_wp), M, hs, q, true, s, fused_mlp ? u16(xp_) : nullptr);
        else
            project(x_, attn_, L.o_w, L.o_wp, M, hs, q, true, s);
        if (fused_mlp) {
            K::gateUpSwiglu(down_px ? u16(actp_) : u16(act_), u16(xp_), u16(L.gate_up_wfp), M, di, hs, cfg_.epsilon, s,
                            down_px);
        } else {
            if (!fold) K::rmsNormRows(u16(h_), u16(x_), nullptr, u16(L.mlp_norm), T, hs, cfg_.epsilon, s);
            if (!fold && L.gate_up_wi) {
                // The general GEMM with the SwiGLU in its epilogue.
                K::linearSwiglu(act_->data(), h_->data(), L.gate_up_wi->data(), K::ElemType::BF16, M, di, hs, s);
            } else {
                const tensor_t gup = fold ? L.gate_up_wfp : tensor_t();
                project(gu_, fold ? x_ : h_, fold ? L.gate_up_wf : L.gate_up_w, gup, M, 2 * di, hs, false, s);
                // The decode GEMM over the interleaved packed copy leaves gate
                // and up columns interleaved as well.
                K::swigluRows(u16(act_), u16(gu_), xr, T, di, hs, cfg_.epsilon, s,
                              takesDecodeGemm(gup, M, 2 * di, hs));
            }
        }
        if (down_px) {
            auto *part = static_cast<float *>(rt.scratch(K::splitKPackedWorkspaceBytes(M, hs, di)));
            K::splitKPackedGemm(u16(x_), u16(actp_), u16(L.down_wp), M, hs, di, true, part, s, u16(xp_));
        } else {
            project(x_, act_, L.down_w, L.down_wp, M, hs, di, true, s, px ? u16(xp_) : nullptr);
        }
    }
    K::rmsNormRows(u16(hl_), u16(x_), i64(last_), u16(out_norm_), B, hs, cfg_.epsilon, s);
    const int voc = int(cfg_.voc);
    if (takesDecodeGemm(out_embed_p_, int(B), voc, hs) && (B <= 64 || voc >= 8192)) {
        // The LM head's workgroups leave each row's argmax over their columns
        // (no second pass over the logits).
        const int chunks = K::decodeGemmKeyChunks(voc);
        auto *keys = static_cast<uint64_t *>(rt.scratch(B * size_t(chunks) * sizeof(uint64_t)));
        K::decodeGemm(u16(logits_), u16(hl_), u16(out_embed_p_), int(B), voc, hs, false, s, keys);
        K::argmaxFinishKeys(i64(next_), keys, B, chunks, s);
    } else {
        project(logits_, hl_, out_embed_, out_embed_p_, int(B), voc, hs, false, s);
        K::argmax(i64(next_), nullptr, logits_->data(), et, B, int64_t(cfg_.voc),
                  rt.scratch(K::argmaxWorkspaceBytes(B, int64_t(cfg_.voc))), s);
    }
}

// Largest M at which the decode GEMM over packed weights takes a projection
// of N rows (K = 1536) instead of the general MFMA GEMM (linear): the LM head
// (N = 151936) at every M <= 128, gate-up (N = 17920) up to 96, qkv and o
// (N = 2048, 1536) up to 64. The limits were measured on MI355X with weights
// cold in HBM; config-5 decode steps (M = 128) take the packed-operand
// kernels instead (packedXGemm, qkvRopeGemm, gateUpSwiglu).
namespace {
int decodeGemmMaxM(int N) { return N >= 65536 ? 128 : N >= 8192 ? 96 : 64; }

// Whether project() runs the decode GEMM over `packed` for this shape.
bool takesDecodeGemm(const tensor_t &packed, int M, int N, int K) {
    return packed && M <= decodeGemmMaxM(N) && K::decodeGemmSupported(M, N, K);
}
} // namespace

void Qwen2Model::project(const tensor_t &y, const tensor_t &x, const tensor_t &w, const tensor_t &packed, int M,
                         int N, int K, bool accumulate, void *s, uint16_t *y_packed) const {
    if (!y_packed && takesDecodeGemm(packed, M, N, K)) {
        K::decodeGemm(u16(y), u16(x), u16(packed), M, N, K, accumulate, s);
        return;
    }
    // Long K (the down projection): the split-K kernel over packed weights at
    // every M <= 128 (weights cold, MI355X: 11.5 us at M = 1, 19.5 us at
    // M = 128, GEMM + reduce).
    if (packed && K::splitKGemmSupported(M, N, K)) {
        auto *part = static_cast<float *>(core::context().runtime().scratch(K::splitKWorkspaceBytes(M, N, K)));
        K::splitKGemm(u16(y), u16(x), u16(packed), M, N, K, accumulate, part, s, y_packed);
        return;
    }
    LLAISYS_CHECK(!y_packed, "qwen2: a packed copy of the output needs the split-K projection");
    gemm(y, x, w, nullptr, M, N, K, accumulate, s);
}

tensor_t Qwen2Model::lastLogits() const {
    LLAISYS_CHECK(last_B_ > 0, "qwen2: no step has run yet");
    return rows(logits_, last_B_);
}

int64_t Qwen2Model::infer(const int64_t *token_ids, size_t ntoken) {
    LLAISYS_CHECK(token_ids && ntoken > 0, "qwen2 infer: no tokens");
    const bool extends = have0_ && hist0_.size() < ntoken &&
                         std::equal(hist0_.begin(), hist0_.end(), token_ids);
    size_t start = hist0_.size();
    if (!extends) {
        if (have0_) blocks_.release(0);
        have0_ = false;
        hist0_.clear();
        start = size_t(blocks_.create(0, token_ids, ntoken));
        have0_ = true;
        hist0_.assign(token_ids, token_ids + start);
    }
    const int64_t id = 0;
    const size_t n = ntoken - start;
    int64_t next = -1;
    try {
        step(&id, 1, token_ids + start, &n, &next);
    } catch (...) {
        // The sequence may hold reserved, uncommitted pages: start over next time.
        blocks_.release(0);
        have0_ = false;
        hist0_.clear();
        throw;
    }
    hist0_.assign(token_ids, token_ids + ntoken);
    return next;
}

int64_t Qwen2Model::seqCreate(const int64_t *tokens, size_t ntokens, size_t *reused) {
    const int64_t id = next_id_++;
    const int r = blocks_.create(id, tokens, tokens ? ntokens : 0);
    if (reused) *reused = size_t(r);
    return id;
}

int64_t Qwen2Model::seqFork(int64_t parent) {
    LLAISYS_CHECK(parent != 0, "qwen2: sequence 0 belongs to Infer");
    const int64_t id = next_id_++;
    blocks_.fork(parent, id);
    return id;
}

void Qwen2Model::seqFree(int64_t id) {
    LLAISYS_CHECK(id != 0, "qwen2: sequence 0 belongs to Infer");
    blocks_.release(id);
}

size_t Qwen2Model::seqLength(int64_t id) const { return size_t(blocks_.length(id)); }

} // namespace llaisys::models
