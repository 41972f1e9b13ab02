// Batched paged decode attention for gfx950: flash-decoding over a dynamic
// queue of page-pair chunks.
//
// Work = every (sequence b, kv head h) unit's page pairs, laid end to end:
// unit u = b*nkvh + h owns npairs(b) = ceil(ceil(ctx_b/16)/2) consecutive
// pair indices; chunk c is pairs [c*kChunk, (c+1)*kChunk). A persistent grid
// of single-wave workgroups (about one per SIMD) takes chunks from a global
// atomic counter, so waves on faster XCDs simply take more chunks. Each wave
// streams its chunks through a ring of NSTAGE page pairs in flight; the next
// chunk's id is taken two chunks ahead and its block ids one chunk ahead, so
// the ring never drains between chunks. Every wave does the same small prefix
// scan of ctx into LDS to map pair indices to (b, h, page), so no host-side
// knowledge of the lengths and no planning kernel is needed.
//
// A unit whose pairs all fall in one chunk is finished there (normalised
// output). Otherwise each chunk holding part of it writes a record
// (unnormalised O, running max m, sum l) into slot 0 (the chunk's first unit)
// or slot 1 (its last unit), and the combine kernel, launched next on the same
// stream, merges the records with log-sum-exp weights and resets the queue
// counter. The kernel boundary orders records before the merge: no wave ever
// waits on another, and no cache-maintaining fences are issued.
//
// Per pair the wave reads 16 KiB of K/V plus the unit's query rows (1 KiB per
// 16 columns, from L2) and issues 24 MFMAs (mfma_common.hpp has the layout).
#include "mfma_common.hpp"

#include "../device/hip_check.hpp"

#include <algorithm>
#include <cstdlib>
#include <mutex>
#include <vector>

namespace llaisys::kernels {

namespace {

using namespace mfma;

constexpr int kChunk = 4; // page pairs per queue entry

struct DecodeArgs {
    const uint16_t *q;
    void *out;
    const uint16_t *k_pool;
    const uint16_t *v_pool;
    const int32_t *table;
    const int32_t *ctx;
    float *records;
    int *counters;
    int *err;
    int B, nh, nkvh, G, max_pages, num_blocks, W;
    float scale_log2;
};

// Exclusive prefix (over b) of nkvh * npairs(b) into S[0..B], lengths into C.
// Invalid lengths (< 1 or beyond the block table) count as empty and raise
// kErrTooLong when `report`. Returns the total pair count N. Run by the first
// wave of the workgroup only; the caller synchronises before reading S/C.
__device__ int scanPairs(const DecodeArgs &a, int *S, int *C, bool report) {
    const int lane = threadIdx.x;
    int carry = 0;
    for (int base = 0; base < a.B; base += 64) {
        const int bb = base + lane;
        int c = 0;
        if (bb < a.B) {
            c = a.ctx[bb];
            if (c < 1 || c > a.max_pages * 16) {
                if (report) atomicOr(a.err, kErrTooLong);
                c = 0;
            }
        }
        const int mine = ((((c + 15) >> 4) + 1) >> 1) * a.nkvh;
        int incl = mine;
#pragma unroll
        for (int off = 1; off < 64; off <<= 1) {
            const int y = __shfl_up(incl, off);
            if (lane >= off) incl += y;
        }
        if (bb < a.B) {
            S[bb] = carry + incl - mine;
            C[bb] = c;
        }
        carry += __shfl(incl, 63);
    }
    if (lane == 0) S[a.B] = carry;
    return carry;
}

template <int NSTAGE> struct Ring {
    PagePair pp[NSTAGE];
    u32x4 q[NSTAGE][4];
};

// Lane i < kChunk describes pair chunk*kChunk + i (clamped into the chunk and
// below N): sequence, kv head, pair index within the unit, block ids.
struct Window {
    int b, h, j, bidA, bidB;
};

__device__ Window loadWindow(const DecodeArgs &a, const int *S, const int *C, int chunk, int N) {
    const int lane = threadIdx.x;
    const int g = min(chunk * kChunk + min(lane, kChunk - 1), N - 1);
    int lo = 0, hi = a.B - 1;
    while (lo < hi) {
        const int mid = (lo + hi + 1) >> 1;
        if (S[mid] <= g)
            lo = mid;
        else
            hi = mid - 1;
    }
    Window w;
    w.b = lo;
    const int np = (C[lo] + 15) >> 4;
    const int npr = (np + 1) >> 1;
    const int rem = g - S[lo];
    w.h = rem / npr;
    w.j = rem - w.h * npr;
    const int pa = 2 * w.j;
    const int pb = min(pa + 1, np - 1);
    const int32_t *row = a.table + size_t(lo) * a.max_pages;
    // Range-checked where used (issue): checking here would wait on the load.
    w.bidA = row[pa];
    w.bidB = row[pb];
    return w;
}

template <bool OUT_F32, int NSTAGE>
__global__ void __launch_bounds__(64) decodeKernel(DecodeArgs a) {
    static_assert(kChunk % NSTAGE == 0, "ring slots must line up across chunks");
    extern __shared__ int lds[];
    int *S = lds;
    int *C = lds + a.B + 1;
    const int lane = threadIdx.x;
    const int n = lane & 15;
    const int grp = lane >> 4;
    const int G = a.G;
    int *queue = a.counters;

    const int N = scanPairs(a, S, C, blockIdx.x == 0);
    __syncthreads();
    const int NC = (N + kChunk - 1) / kChunk;
    // Chunks w and W + w are this wave's by construction; later ones come from
    // the queue, which hands out 2W, 2W+1, ... (all waves hitting one counter
    // at kernel start would serialise on it). A queue value stays in lane 0 of
    // a vector register until read (chunkOf): reading it forces a wait on the
    // atomic, and with in-order load counters that wait would drain the load
    // ring, so every id is taken a full chunk before it is read.
    const int W = gridDim.x;
    auto grab = [&]() {
        int c = 0;
        if (lane == 0) c = atomicAdd(queue, 1);
        return c;
    };
    auto chunkOf = [&](int raw) { return 2 * W + __builtin_amdgcn_readfirstlane(raw); };
    int c_cur = blockIdx.x;
    if (c_cur >= NC) return;
    int c_nxt = W + blockIdx.x;
    Window cur = loadWindow(a, S, C, c_cur, N);
    Window nxt = loadWindow(a, S, C, min(c_nxt, NC - 1), N);
    int raw_after = grab();

    const u32x4 *kp = reinterpret_cast<const u32x4 *>(a.k_pool) + lane;
    const u32x4 *vp = reinterpret_cast<const u32x4 *>(a.v_pool) + lane;
    const int ncol = min(n, G - 1); // columns past G read a valid row and are masked later

    Ring<NSTAGE> ring;
    // Load page pair (window `use_nxt ? nxt : cur`, lane k) into ring slot st.
    // The window choice is a uniform select, never a branch around the loads,
    // so the compiler can keep counting the loads in flight.
    bool bad_block = false;
    auto issue = [&](int st, bool use_nxt, int k) {
        int bA = use_nxt ? __builtin_amdgcn_readlane(nxt.bidA, k) : __builtin_amdgcn_readlane(cur.bidA, k);
        int bB = use_nxt ? __builtin_amdgcn_readlane(nxt.bidB, k) : __builtin_amdgcn_readlane(cur.bidB, k);
        const bool bad = unsigned(bA) >= unsigned(a.num_blocks) || unsigned(bB) >= unsigned(a.num_blocks);
        bad_block |= bad;
        bA = bad ? 0 : bA;
        bB = bad ? 0 : bB;
        const int b = use_nxt ? __builtin_amdgcn_readlane(nxt.b, k) : __builtin_amdgcn_readlane(cur.b, k);
        const int h = use_nxt ? __builtin_amdgcn_readlane(nxt.h, k) : __builtin_amdgcn_readlane(cur.h, k);
        loadPair(ring.pp[st], kp, vp, (size_t(bA) * a.nkvh + h) * 256, (size_t(bB) * a.nkvh + h) * 256);
        const uint16_t *qrow = a.q + (size_t(b) * a.nh + h * G + ncol) * kHeadDim + grp * 8;
#pragma unroll
        for (int t = 0; t < 4; ++t) ring.q[st][t] = *reinterpret_cast<const u32x4 *>(qrow + 32 * t);
    };

    Acc acc;
    acc.reset();
    int cur_b = -1, cur_h = 0;
    int chunk_lo = 0, chunk_hi = 0; // pair range of the chunk being consumed

    auto finish = [&]() {
        float lt = acc.l + __shfl_xor(acc.l, 16);
        lt += __shfl_xor(lt, 32);
        const int np = (C[cur_b] + 15) >> 4;
        const int npr = (np + 1) >> 1;
        const int first = S[cur_b] + cur_h * npr;
        if (first >= chunk_lo && first + npr <= chunk_hi) {
            if (n < G) {
                const float inv = 1.f / lt;
                const size_t row = (size_t(cur_b) * a.nh + cur_h * G + n) * kHeadDim;
#pragma unroll
                for (int i = 0; i < 8; ++i) storeOut<OUT_F32>(a.out, row, i, grp, acc.o[i] * inv);
            }
        } else if (n < G) {
            const int slot = first <= chunk_lo ? 0 : 1;
            float *rec = a.records + size_t(2 * (chunk_lo / kChunk) + slot) * size_t(G * (kHeadDim + 2));
#pragma unroll
            for (int i = 0; i < 8; ++i) *reinterpret_cast<f32x4 *>(rec + n * kHeadDim + i * 16 + grp * 4) = acc.o[i];
            if (grp == 0) {
                rec[G * kHeadDim + 2 * n] = acc.m;
                rec[G * kHeadDim + 2 * n + 1] = lt;
            }
        }
    };

    int len_cur = min(kChunk, N - c_cur * kChunk);
#pragma unroll
    for (int st = 0; st < NSTAGE; ++st) issue(st, false, min(st, len_cur - 1));
    while (true) {
        const bool more = c_nxt < NC;
        const int len_nxt = more ? min(kChunk, N - c_nxt * kChunk) : 0;
        chunk_lo = c_cur * kChunk;
        chunk_hi = chunk_lo + len_cur;
#pragma unroll
        for (int p = 0; p < kChunk; ++p) {
            const int st = p % NSTAGE;
            if (p < len_cur) {
                const int b = __builtin_amdgcn_readlane(cur.b, p);
                const int h = __builtin_amdgcn_readlane(cur.h, p);
                const int j = __builtin_amdgcn_readlane(cur.j, p);
                if (b != cur_b || h != cur_h) {
                    if (cur_b >= 0) finish();
                    acc.reset();
                    cur_b = b;
                    cur_h = h;
                }
                const int c = C[b];
                const bool hasB = 2 * j + 1 < ((c + 15) >> 4);
                u32x4 qop[4];
#pragma unroll
                for (int t = 0; t < 4; ++t) qop[t] = n < G ? ring.q[st][t] : u32x4{0, 0, 0, 0};
                consumePair(acc, ring.pp[st], qop, 32 * j, c - 1, c, hasB, grp, a.scale_log2);
            }
            // Refill this slot with the pair NSTAGE ahead (from the next chunk
            // near the end; past the last chunk it re-reads a pair, an L2 hit).
            const int q = p + NSTAGE;
            if (q < kChunk)
                issue(st, false, min(q, len_cur - 1));
            else
                issue(st, more, more ? min(q - kChunk, len_nxt - 1) : len_cur - 1);
        }
        finish();
        cur_b = -1;
        if (!more) break;
        c_cur = c_nxt;
        cur = nxt;
        len_cur = len_nxt;
        c_nxt = chunkOf(raw_after);
        nxt = loadWindow(a, S, C, min(c_nxt, NC - 1), N);
        raw_after = grab();
    }
    if (bad_block && lane == 0) atomicOr(a.err, kErrBadBlock);
}

// Merge the records of every unit that spans more than one chunk.
// 256 threads = 4 waves per unit. Wave 0 scans the lengths into LDS; then
// wave v takes every 4th batch of the unit's records, with all loads of a
// batch in flight, and merges them online (O = sum 2^(m_r - M) O_r, l
// likewise); the four partial states meet in LDS and wave 0 writes the
// output. Block 0 also resets the chunk queue for the next launch.
constexpr int kCombineWaves = 4;
constexpr int kMergeBatch = 4;

template <bool OUT_F32> __global__ void __launch_bounds__(64 * kCombineWaves) decodeCombineKernel(DecodeArgs a) {
    extern __shared__ int lds[];
    int *S = lds;
    int *C = lds + a.B + 1;
    __shared__ float part_o[kCombineWaves - 1][8][64][4];
    __shared__ float part_ml[kCombineWaves - 1][2][64];
    const int wave = threadIdx.x >> 6;
    const int lane = threadIdx.x & 63;
    const int n = lane & 15;
    const int grp = lane >> 4;
    const int G = a.G;
    if (blockIdx.x == 0 && threadIdx.x == 0) a.counters[0] = 0;
    if (wave == 0) scanPairs(a, S, C, false);
    __syncthreads();
    const int u = blockIdx.x;
    const int b = u / a.nkvh;
    const int h = u - b * a.nkvh;
    const int np = (C[b] + 15) >> 4;
    const int npr = (np + 1) >> 1;
    if (npr == 0) return;
    const int first = S[b] + h * npr;
    const int c0 = first / kChunk;
    const int c1 = (first + npr - 1) / kChunk;
    if (c0 == c1) return;
    const int nrec = c1 - c0 + 1;
    const size_t stride = size_t(G) * (kHeadDim + 2);
    const int col = min(n, G - 1);
    // Record k of the unit: chunk c0 + k, slot 1 for chunk c0 unless the unit starts it.
    auto recordOf = [&](int k) {
        const int c = c0 + k;
        return a.records + size_t(2 * c + ((k == 0 && first % kChunk != 0) ? 1 : 0)) * stride;
    };

    float M = -INFINITY, L = 0.f;
    f32x4 o[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) o[i] = f32x4{0.f, 0.f, 0.f, 0.f};
    for (int k0 = wave * kMergeBatch; k0 < nrec; k0 += kCombineWaves * kMergeBatch) {
        float mr[kMergeBatch], lr[kMergeBatch];
        f32x4 orr[kMergeBatch][8];
#pragma unroll
        for (int t = 0; t < kMergeBatch; ++t) {
            const float *rec = recordOf(min(k0 + t, nrec - 1));
            mr[t] = rec[G * kHeadDim + 2 * col];
            lr[t] = rec[G * kHeadDim + 2 * col + 1];
#pragma unroll
            for (int i = 0; i < 8; ++i)
                orr[t][i] = *reinterpret_cast<const f32x4 *>(rec + col * kHeadDim + i * 16 + grp * 4);
            if (k0 + t >= nrec) mr[t] = -INFINITY; // weight 0
        }
#pragma unroll
        for (int t = 0; t < kMergeBatch; ++t) {
            if (mr[t] == -INFINITY) continue;
            const float Mn = fmaxf(M, mr[t]);
            const float sa = exp2Fast(M - Mn);
            const float sb = exp2Fast(mr[t] - Mn);
            L = L * sa + lr[t] * sb;
#pragma unroll
            for (int i = 0; i < 8; ++i) o[i] = o[i] * sa + orr[t][i] * sb;
            M = Mn;
        }
    }
    if (wave > 0) {
#pragma unroll
        for (int i = 0; i < 8; ++i)
#pragma unroll
            for (int c = 0; c < 4; ++c) part_o[wave - 1][i][lane][c] = o[i][c];
        part_ml[wave - 1][0][lane] = M;
        part_ml[wave - 1][1][lane] = L;
    }
    __syncthreads();
    if (wave > 0 || n >= G) return;
#pragma unroll
    for (int v = 0; v < kCombineWaves - 1; ++v) {
        const float mv = part_ml[v][0][lane];
        if (mv == -INFINITY) continue;
        const float Mn = fmaxf(M, mv);
        const float sa = exp2Fast(M - Mn);
        const float sb = exp2Fast(mv - Mn);
        L = L * sa + part_ml[v][1][lane] * sb;
#pragma unroll
        for (int i = 0; i < 8; ++i)
#pragma unroll
            for (int c = 0; c < 4; ++c) o[i][c] = o[i][c] * sa + part_o[v][i][lane][c] * sb;
        M = Mn;
    }
    const float inv = 1.f / L;
    const size_t row = (size_t(b) * a.nh + h * G + n) * kHeadDim;
#pragma unroll
    for (int i = 0; i < 8; ++i) storeOut<OUT_F32>(a.out, row, i, grp, o[i] * inv);
}

int envInt(const char *name, int fallback) {
    const char *v = std::getenv(name);
    return (v && *v) ? std::atoi(v) : fallback;
}

int computeUnits() {
    static std::mutex mu;
    static std::vector<int> cache;
    int dev = 0;
    HIP_CHECK(hipGetDevice(&dev));
    std::lock_guard<std::mutex> lock(mu);
    if (size_t(dev) >= cache.size()) cache.resize(dev + 1, 0);
    if (!cache[dev]) HIP_CHECK(hipDeviceGetAttribute(&cache[dev], hipDeviceAttributeMultiprocessorCount, dev));
    return cache[dev];
}

} // namespace

DecodePlan planDecode(int B, int nkvh, int group, int max_pages) {
    DecodePlan p{};
    const long long max_pairs = (long long)B * nkvh * ((max_pages + 1) / 2);
    const long long max_chunks = (max_pairs + kChunk - 1) / kChunk;
    p.waves = std::max(1, envInt("LLAISYS_DECODE_WAVES", 4 * computeUnits()));
    p.record_bytes = size_t(2) * size_t(std::max(1LL, max_chunks)) * group * (kHeadDim + 2) * sizeof(float);
    p.lds_bytes = size_t(2 * B + 1) * sizeof(int);
    p.stages = envInt("LLAISYS_DECODE_STAGES", 2) >= 4 ? 4 : 2;
    return p;
}

void pagedDecode(void *out, bool out_f32, const uint16_t *q, const uint16_t *k_pool, const uint16_t *v_pool,
                 const int32_t *block_table, const int32_t *ctx_len, int B, int nh, int nkvh, int max_pages,
                 int num_blocks, float scale, const DecodePlan &plan, float *records, int *counters, int *err,
                 void *stream) {
    if (B == 0) return;
    DecodeArgs a;
    a.q = q;
    a.out = out;
    a.k_pool = k_pool;
    a.v_pool = v_pool;
    a.table = block_table;
    a.ctx = ctx_len;
    a.records = records;
    a.counters = counters;
    a.err = err;
    a.B = B;
    a.nh = nh;
    a.nkvh = nkvh;
    a.G = nh / nkvh;
    a.max_pages = max_pages;
    a.num_blocks = num_blocks;
    a.W = plan.waves;
    a.scale_log2 = scale * 1.4426950408889634f;
    auto s = static_cast<hipStream_t>(stream);
    const unsigned lds = unsigned(plan.lds_bytes);
    const dim3 grid(plan.waves), comb(B * nkvh);
    const dim3 one(64), four(64 * kCombineWaves);
    if (out_f32) {
        if (plan.stages == 4)
            hipLaunchKernelGGL((decodeKernel<true, 4>), grid, one, lds, s, a);
        else
            hipLaunchKernelGGL((decodeKernel<true, 2>), grid, one, lds, s, a);
        hipLaunchKernelGGL((decodeCombineKernel<true>), comb, four, lds, s, a);
    } else {
        if (plan.stages == 4)
            hipLaunchKernelGGL((decodeKernel<false, 4>), grid, one, lds, s, a);
        else
            hipLaunchKernelGGL((decodeKernel<false, 2>), grid, one, lds, s, a);
        hipLaunchKernelGGL((decodeCombineKernel<false>), comb, four, lds, s, a);
    }
    HIP_CHECK(hipGetLastError());
}

} // namespace llaisys::kernels
