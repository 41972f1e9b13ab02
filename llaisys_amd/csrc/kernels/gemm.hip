// Y[M, N] (+)= X[M, K] . W[N, K]^T (+ bias[N]) for any M, N, K: the
// reference's linear (README.md:181-198, stub src/ops/linear/op.cpp:4-6) as a
// hand-written MFMA GEMM for gfx950, in f32, f16 and bf16 with fp32
// accumulation and one rounding of (old Y +) sum (+ bias) to the output type.
//
// Both operands are K-contiguous rows ("NT"), so one 16 B piece of a row is a
// whole MFMA operand fragment per lane:
//  * 16-bit types: v_mfma_f32_16x16x32_{bf16,f16}; lane l holds row l % 16,
//    k 8 (l / 16) .. + 7 of a 32-k step.
//  * f32: v_mfma_f32_16x16x4_f32 four times per 16 B piece; lane l holds row
//    l % 16, k 4 (l / 16) .. + 3 of a 16-k step, and MFMA e takes element e
//    of every lane (k 4 g + e, g = 0..3): the same k order on both operands,
//    so the sum is over the same products.
//
// A workgroup of 4 or 8 waves (2 x 2, 2 x 4 or 4 x 2) owns a BM x BN tile
// of Y; each wave one sub-tile of it (64 x 48 to 128 x 64). K advances in
// tiles of 128 B per row (64 16-bit elements; f32: 64 B, 16 elements)
// through an LDS ring of two stages (f32: four): each wave moves whole 1 KiB
// blocks of X and W rows straight from global memory into LDS by 16 B
// global_load_lds (buffer loads: out-of-range rows and k come back as zeros,
// so edge tiles need no other guard), and one barrier per stage both
// publishes a stage and frees the slot the next issue refills. Each wave
// reads the next fragments from LDS while the current MFMAs run (two
// register sets, reads spread between the MFMAs). In LDS, piece c of row r
// sits at a slot swizzled by r, so a fragment read is free of bank
// conflicts. Shapes that leave CUs idle split K over workgroups into fp32
// partials that a second kernel sums in split order (deterministic) before
// the single rounding.
//
// W is the MFMA's A operand and X its B operand, so a lane's accumulator
// holds 4 consecutive columns n of one row m of Y. 16-bit tiles leave
// through the idle LDS ring as whole rows (16 B per lane); otherwise one 8 B
// or 16 B store per lane and fragment.
//
// Workgroups go to the XCDs round-robin by id; the tile order puts each
// XCD's workgroups on one contiguous run of tiles, walked m-fastest in groups
// of kGroupN column tiles, so the workgroups resident on one XCD share both
// their W columns and their X rows in that XCD's L2.
#include "launch.hpp"

#include "../common.hpp"
#include "../device/hip_check.hpp"

#include <hip/hip_fp16.h>

#include <algorithm>
#include <cstdlib>
#include <mutex>
#include <type_traits>
#include <vector>

namespace llaisys::kernels {

namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int kXcds = 8;
constexpr int kGroupN = 4;             // column tiles per m-fastest group
constexpr int kRowBytes = 64;          // bytes of one row per k tile (one 32-k MFMA step of 16-bit data)
constexpr int kThreads = 256;
constexpr uint32_t kRsrcWord3 = 0x00020000u; // raw buffer, 32-bit dwords (gfx9 family)
constexpr uint32_t kMasked = 0x80000000u;    // an offset past any buffer: the load returns 0

template <ElemType T> struct Elem;
template <> struct Elem<ElemType::BF16> { using type = __bf16; static constexpr int size = 2; };
template <> struct Elem<ElemType::F16> { using type = _Float16; static constexpr int size = 2; };
template <> struct Elem<ElemType::F32> { using type = float; static constexpr int size = 4; };

// acc += A . B for one 16 B piece per lane (one 32-k step for 16-bit types,
// one 16-k step for f32).
template <ElemType T> __device__ __forceinline__ f32x4 mfmaPiece(u32x4 a, u32x4 b, f32x4 acc) {
    if constexpr (T == ElemType::BF16) {
        return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b),
                                                       acc, 0, 0, 0);
    } else if constexpr (T == ElemType::F16) {
        return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), acc,
                                                      0, 0, 0);
    } else {
#pragma unroll
        for (int e = 0; e < 4; ++e)
            acc = __builtin_amdgcn_mfma_f32_16x16x4f32(__uint_as_float(a[e]), __uint_as_float(b[e]), acc, 0, 0, 0);
        return acc;
    }
}

template <ElemType T> __device__ __forceinline__ float loadElem(const void *p, size_t i) {
    using E = typename Elem<T>::type;
    return float(static_cast<const E *>(p)[i]);
}

template <ElemType T> __device__ __forceinline__ void storeElem(void *p, size_t i, float v) {
    using E = typename Elem<T>::type;
    static_cast<E *>(p)[i] = E(v);
}

// Four consecutive elements (one 8 B or 16 B access), widened to fp32.
template <ElemType T> __device__ __forceinline__ f32x4 load4(const void *p, size_t i) {
    if constexpr (T == ElemType::F32) {
        return *reinterpret_cast<const f32x4 *>(static_cast<const float *>(p) + i);
    } else {
        using E = typename Elem<T>::type;
        typedef E e4 __attribute__((ext_vector_type(4)));
        const e4 v = *reinterpret_cast<const e4 *>(static_cast<const E *>(p) + i);
        return f32x4{float(v[0]), float(v[1]), float(v[2]), float(v[3])};
    }
}

template <ElemType T> __device__ __forceinline__ void store4(void *p, size_t i, f32x4 v) {
    if constexpr (T == ElemType::F32) {
        *reinterpret_cast<f32x4 *>(static_cast<float *>(p) + i) = v;
    } else {
        using E = typename Elem<T>::type;
        typedef E e4 __attribute__((ext_vector_type(4)));
        *reinterpret_cast<e4 *>(static_cast<E *>(p) + i) = e4{E(v[0]), E(v[1]), E(v[2]), E(v[3])};
    }
}

struct GemmParams {
    void *y;
    const void *x, *w, *bias;
    int M, N, K;
    int accumulate;
    int mtiles, ntiles;
    uint32_t x_bytes, w_bytes; // buffer extents (range checks)
    int splits;                // > 1: K split over workgroups, fp32 partials part[split][M][N]
    float *part;
    int swiglu; // y = act[M][N / 2]: W rows are gate and up blocks of 16 in turn (swigluInterleave)
    int staged; // 16-bit output, no split, N % 8 == 0, 16 B aligned rows: the tile leaves through LDS
    int ldy;    // elements between rows of y (N, or N / 2 for swiglu, unless y is a column range of a wider
                // matrix); split partials and the reduce keep ldy == N
};

// Bytes per row of a tile staged in LDS for the store: BN 16-bit values and
// 32 B of padding, so that the 16 rows one fragment write touches start 8
// banks apart.
template <int BN> constexpr int stagePitch() { return BN * 2 + 32; }
template <int BM, int BN> constexpr size_t stageBytes() { return size_t(BM) * stagePitch<BN>(); }

// 1 KiB blocks of one ring stage: the tile's X blocks, then its W blocks
// rounded up to whole blocks per wave (a BN / 16 that is not a multiple of the
// wave count leaves some waves one masked load into the spare blocks, so
// every wave issues the same number of loads and waits on the same counts).
template <int BM, int BN, int NW, int RB = 64> constexpr int stageBlocks() {
    return BM / (1024 / RB) + (BN / (1024 / RB) + NW - 1) / NW * NW;
}

// Tile index of workgroup b: XCD b % 8 takes tiles [(b % 8) T / 8, ...) in
// order b / 8 (T = tiles; when T % 8 != 0 the plain order is kept).
__device__ __forceinline__ void tileOf(const GemmParams &p, int b, int &mt, int &nt) {
    const int tiles = p.mtiles * p.ntiles;
    int t = b;
    if (tiles % kXcds == 0) t = (t % kXcds) * (tiles / kXcds) + t / kXcds;
    // m-fastest within groups of kGroupN column tiles
    const int per_group = kGroupN * p.mtiles;
    const int g = t / per_group, r = t % per_group;
    const int gn = min(kGroupN, p.ntiles - g * kGroupN);
    mt = r / gn;
    nt = g * kGroupN + r % gn;
}

typedef __attribute__((address_space(3))) void lds_void;

// 64 B k tiles (f32, and 16-bit types with LLAISYS_GEMM_WIDE_K=0):
// one k tile of an operand is ROWS rows x 64 B (4 pieces of 16 B), kept in
// LDS as blocks of 16 rows x 64 B: one 64-lane global_load_lds instruction
// fills one block, lane i writing bytes 16 i .. 16 i + 15 of it (row i / 4,
// slot i % 4). Piece c of row r sits at slot c ^ key(r). A fragment read
// (lane l: row l % 16, piece l / 16) serves 8 lanes per LDS cycle with 32
// banks of 4 B (16 with 64): rows r and r + 2 start on the same banks, so
// the key must differ across the rows of one parity within every 8 rows and
// across the rows of one residue mod 4 within the 16: bit 1 = r2 ^ r3,
// bit 0 = r1 ^ r3 does both. (The key (r / 4) % 4 left half of all LDS
// cycles as bank conflicts: SQ_LDS_BANK_CONFLICT / SQ_LDS_IDX_ACTIVE 0.50.)
// Lane i therefore fetches piece (i % 4) ^ key(i / 4).
__device__ __forceinline__ int rowKey(int r) { return ((((r >> 2) ^ (r >> 3)) & 1) << 1) | (((r >> 1) ^ (r >> 3)) & 1); }
__device__ __forceinline__ int slotOf(int r, int c) { return c ^ rowKey(r); }

// Stages of the LDS ring, also when the fragments of the next k tile are
// read from LDS while the current tile's MFMAs run (PIPE): 4 (PIPE with 5
// stages was 3-5 % slower, 3 stages slower again: 8192 x 17920 x 1536 486
// against 503 and 497 us; more loads in flight per CU than it can stream).
template <bool PIPE, int RB = 64, int WS = 2> constexpr int ringStages() { return RB == 128 ? WS : 4; }

// Stages of the wide ring: two for the 8-wave tiles (256 x 256 and 256 x 192
// fit no more; 128 x 256 and 256 x 128 ran 1-6 % slower with three), four
// for the 4-wave ones, whose short k loops wait on their loads more: 1024 x
// 2048 x 1536 16.9 -> 14.1 us, 1024 x 1536 x 8960 47.6 -> 37.4 us, 2048 x 1536
// x 1536 17.1 -> 14.8 us (LLAISYS_GEMM_WIDE_DEEP=0: two everywhere).
template <int BM, int BN, int NW> constexpr int wideStages() {
    constexpr int n = 163840 / (((BM / 8) + (BN / 8 + NW - 1) / NW * NW) * 1024);
    return NW > 4 ? 2 : n > 4 ? 4 : n < 2 ? 2 : n;
}

// Wide k tiles (RB = 128: 64 16-bit k per row and stage). A 64 B row piece
// per load instruction made every L1 -> L2 request 64 B, half a cache line:
// at 256 x 256 x 1536 the kernel sent 54 M requests where hipBLASLt's
// 128 B pieces send 28 M for the same bytes, and a CU's requests in flight
// (~62 at ~290 cycles each) then bound the k loop. With 128 B per row a
// block of one instruction is 8 rows x 128 B, piece c of row r sits at slot
// c ^ (r % 8) (the 8 lanes one LDS cycle serves read 8 rows of one piece:
// 8 distinct slots), and a stage is twice the bytes, so the ring holds two
// stages: the next stage's loads go out right after the barrier that frees
// its slot and have the current stage's two MFMA steps to land; the second
// step's fragments are read under the first step's MFMAs.
// WGM x WGN waves, wave (wm, wn) owning the (BM / WGM) x (BN / WGN) sub-tile.
template <ElemType T, int BM, int BN, int WGM = 2, int WGN = 2, bool PIPE = false, int RB = 64, int WS = 2>
__global__ void __launch_bounds__(64 * WGM * WGN) gemmKernel(GemmParams p) {
    static_assert(RB == 64 || RB == 128, "k tiles of 64 or 128 B per row");
    constexpr bool WIDE = RB == 128;
    constexpr int NS = ringStages<PIPE, RB, WS>();
    constexpr int NW = WGM * WGN;
    constexpr int ES = Elem<T>::size;
    constexpr int KT = RB / ES;                     // elements per k tile
    constexpr int PPR = RB / 16;                    // 16 B pieces per row and k tile
    constexpr int RPB = 64 / PPR;                   // rows per 1 KiB block (one load instruction)
    constexpr int TM = BM / (16 * WGM), TN = BN / (16 * WGN); // 16-row fragments per wave
    constexpr int XB = BM / RPB, WB = BN / RPB;     // 1 KiB blocks per operand per k tile
    constexpr int XW = XB / NW, WW = (WB + NW - 1) / NW; // ... issued by each wave
    constexpr int STAGE = stageBlocks<BM, BN, NW, RB>() * 64; // u32x4 per stage
    constexpr int kLoadsPerStage = XW + WW;          // per wave
    static_assert(XB % NW == 0, "each wave issues whole X blocks");
    extern __shared__ u32x4 lds[];                   // [NS][X blocks | W blocks]

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave % WGM, wn = wave / WGM;
    // Workgroup b: split b / tiles over k tiles [s nk / S, (s + 1) nk / S)
    // of tile b % tiles.
    const int tiles = p.mtiles * p.ntiles;
    const int split = int(blockIdx.x) / tiles;
    int mt, nt;
    tileOf(p, int(blockIdx.x) % tiles, mt, nt);
    const int m0 = mt * BM, n0 = nt * BN;

    const __amdgpu_buffer_rsrc_t xr =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(p.x), (short)0, int(p.x_bytes), kRsrcWord3);
    const __amdgpu_buffer_rsrc_t wr =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(p.w), (short)0, int(p.w_bytes), kRsrcWord3);
    const uint32_t row_bytes = uint32_t(p.K) * ES;

    // Lane's piece of a block: row lr = lane / PPR of the block, global piece lc.
    const int lr = lane / PPR, lc = WIDE ? (lane % PPR) ^ lr : (lane & 3) ^ rowKey(lr);
    // Block b of the wave is block wave + NW b of the operand (rows RPB (wave + NW b) ..).
    const uint32_t xbase = uint32_t(m0 + RPB * wave + lr) * row_bytes + 16 * lc;
    const uint32_t wbase = uint32_t(n0 + RPB * wave + lr) * row_bytes + 16 * lc;
    const uint32_t bstride = uint32_t(RPB) * NW * row_bytes; // NW blocks of RPB rows
    const int nk_all = (p.K + KT - 1) / KT;
    const int kt0 = split * nk_all / p.splits;
    const int nk = (split + 1) * nk_all / p.splits - kt0;
    auto issue = [&](int kt) {
        u32x4 *st = lds + (kt % NS) * STAGE;
        const uint32_t kb = uint32_t(kt0 + kt) * RB;
        const bool in_k = kt < nk && kb + 16 * lc < row_bytes;
#pragma unroll
        for (int b = 0; b < XW; ++b)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(xr, (lds_void *)(st + (wave + NW * b) * 64), 16,
                                                     int(in_k ? xbase + kb + b * bstride : kMasked), 0, 0, 0);
#pragma unroll
        for (int b = 0; b < WW; ++b)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(
                wr, (lds_void *)(st + (XB + wave + NW * b) * 64), 16,
                int(in_k && (WB % NW == 0 || wave + NW * b < WB) ? wbase + kb + b * bstride : kMasked), 0, 0, 0);
    };

    f32x4 acc[TN][TM];
#pragma unroll
    for (int i = 0; i < TN; ++i)
#pragma unroll
        for (int j = 0; j < TM; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

#pragma unroll
    for (int s = 0; s < (WIDE ? NS : NS - 1); ++s) issue(s);
    // Fragment reads: lane reads row l % 16 of a 16-row block, piece l / 16.
    const int fr = lane & 15, fslot = slotOf(fr, lane >> 4);
    const int xblk0 = wm * TM, wblk0 = XB + wn * TN;
    auto readFrags = [&](int kt, u32x4 (&a)[TN], u32x4 (&b)[TM]) {
        const u32x4 *st = lds + (kt % NS) * STAGE;
#pragma unroll
        for (int i = 0; i < TN; ++i) a[i] = st[(wblk0 + i) * 64 + fr * 4 + fslot];
#pragma unroll
        for (int j = 0; j < TM; ++j) b[j] = st[(xblk0 + j) * 64 + fr * 4 + fslot];
    };
    auto mfmaTile = [&](const u32x4 (&a)[TN], const u32x4 (&b)[TM]) {
        if constexpr (T == ElemType::F32) {
            // element e of every piece, all tiles, then e + 1: dependent
            // MFMAs on one accumulator are TN x TM instructions apart
#pragma unroll
            for (int e = 0; e < 4; ++e)
#pragma unroll
                for (int i = 0; i < TN; ++i)
#pragma unroll
                    for (int j = 0; j < TM; ++j)
                        acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(__uint_as_float(a[i][e]),
                                                                         __uint_as_float(b[j][e]), acc[i][j], 0, 0, 0);
        } else {
#pragma unroll
            for (int i = 0; i < TN; ++i)
#pragma unroll
                for (int j = 0; j < TM; ++j) acc[i][j] = mfmaPiece<T>(a[i], b[j], acc[i][j]);
        }
    };
    // (The compiler does not count global_load_lds against LDS reads, so
    // the waits for the ring are explicit; the barrier after each makes
    // every wave's part of a stage visible.)
    if constexpr (WIDE) {
        // Row R of the stage (X rows, then W rows) at R * 8 + (piece ^ (R % 8)).
        auto readHalf = [&](int kt, int half, u32x4 (&a)[TN], u32x4 (&b)[TM]) {
            const u32x4 *st = lds + (kt % NS) * STAGE;
            const int slot = ((lane >> 4) + 4 * half) ^ (fr & 7);
#pragma unroll
            for (int i = 0; i < TN; ++i) a[i] = st[(BM + 16 * (wn * TN + i) + fr) * PPR + slot];
#pragma unroll
            for (int j = 0; j < TM; ++j) b[j] = st[(16 * (wm * TM + j) + fr) * PPR + slot];
        };
        constexpr int kReads = TN + TM;
        constexpr int kMfmas = TN * TM * (T == ElemType::F32 ? 4 : 1);
        constexpr int kPer = kMfmas / kReads > 0 ? kMfmas / kReads : 1;
        // The reads of one half between the MFMAs of the other.
        auto interleave = [&]() {
#pragma unroll
            for (int g = 0; g < kReads; ++g) {
                __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);    // one LDS read
                __builtin_amdgcn_sched_group_barrier(0x008, kPer, 0); // then MFMAs
            }
        };
        // Stage 0 has landed once only stages 1 .. NS - 1 are in flight.
        asm volatile("s_waitcnt vmcnt(%0)\n\ts_barrier" ::"n"((NS - 1) * kLoadsPerStage) : "memory");
        u32x4 a0[TN], b0[TM], a1[TN], b1[TM];
        readHalf(0, 0, a0, b0);
        for (int kt = 0; kt < nk; ++kt) {
            readHalf(kt, 1, a1, b1);
            mfmaTile(a0, b0);
            interleave();
            // Stage kt + 1 has landed (this wave's loads; the barrier: every
            // wave's) and every wave has read all of stage kt, whose slot
            // stage kt + NS takes.
            asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)\n\ts_barrier" ::"n"((NS - 2) * kLoadsPerStage) : "memory");
            issue(kt + NS);
            readHalf(kt + 1, 0, a0, b0); // past the end: the zero-filled stage
            mfmaTile(a1, b1);
            interleave();
        }
    } else if constexpr (PIPE) {
        // Stage 0 has landed once at most NS - 2 stages are in flight.
        asm volatile("s_waitcnt vmcnt(%0)\n\ts_barrier" ::"n"((NS - 2) * kLoadsPerStage) : "memory");
        // One k tile: wait for stage kt + 1, refill the slot of stage kt - 1,
        // read stage kt + 1's fragments into (an, bn) while the MFMAs of
        // stage kt run from (a, b). Two sets alternate (the loop below runs
        // two steps per turn), so no fragment is copied between registers.
        auto step = [&](int kt, const u32x4 (&a)[TN], const u32x4 (&b)[TM], u32x4 (&an)[TN], u32x4 (&bn)[TM]) {
            // Stage kt + 1 has landed once at most NS - 3 stages are in
            // flight; this wave's fragments of stage kt are in registers.
            asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)\n\ts_barrier" ::"n"((NS - 3) * kLoadsPerStage) : "memory");
            // Slot (kt - 1) % NS was last read (fragments of stage kt - 1)
            // before the previous barrier.
            issue(kt + NS - 1);
            readFrags(kt + 1, an, bn); // past the end: the zero-filled stages
            mfmaTile(a, b);
            // Spread the LDS reads over the MFMAs (left to itself the
            // scheduler puts them all after the MFMAs, right before the
            // next barrier, where nothing hides their latency).
            constexpr int kReads = TN + TM;
            constexpr int kMfmas = TN * TM * (T == ElemType::F32 ? 4 : 1);
            constexpr int kPer = kMfmas / kReads > 0 ? kMfmas / kReads : 1;
#pragma unroll
            for (int g = 0; g < kReads; ++g) {
                __builtin_amdgcn_sched_group_barrier(0x100, 1, 0); // one LDS read
                __builtin_amdgcn_sched_group_barrier(0x008, kPer, 0); // then MFMAs
            }
            __builtin_amdgcn_sched_group_barrier(0x008, kMfmas - kPer * kReads > 0 ? kMfmas - kPer * kReads : 0, 0);
        };
        u32x4 a0[TN], b0[TM], a1[TN], b1[TM];
        readFrags(0, a0, b0);
        for (int kt = 0; kt < nk; kt += 2) {
            step(kt, a0, b0, a1, b1);
            if (kt + 1 < nk) step(kt + 1, a1, b1, a0, b0);
        }
    } else {
        for (int kt = 0; kt < nk; ++kt) {
            // Stage kt has landed once at most NS - 2 stages of this wave's
            // loads are still in flight; the barrier then covers every wave's.
            asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)\n\ts_barrier" ::"n"((NS - 2) * kLoadsPerStage) : "memory");
            // Slot (kt - 1) % NS was read by every wave before this barrier.
            issue(kt + NS - 1);
            u32x4 a[TN], b[TM];
            readFrags(kt, a, b);
            mfmaTile(a, b);
        }
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); // the trailing (zero) stages

    // Epilogue: lane holds Y[m][n .. n + 3], m = row l % 16 of X fragment j,
    // n = 4 (l / 16) of W fragment i; (old Y +) sum (+ bias), rounded once;
    // or, split, the fp32 partial for the reduce.
    const int fg = lane >> 4;
    const bool vec = (p.N & 3) == 0;
    if (p.splits > 1) {
        float *part = p.part + size_t(split) * p.M * p.N;
#pragma unroll
        for (int j = 0; j < TM; ++j) {
            const int m = m0 + wm * (BM / WGM) + 16 * j + fr;
            if (m >= p.M) continue;
#pragma unroll
            for (int i = 0; i < TN; ++i) {
                const int n = n0 + wn * (BN / WGN) + 16 * i + 4 * fg;
                if (n >= p.N) continue;
                const size_t base = size_t(m) * p.N + n;
                if (vec) {
                    *reinterpret_cast<f32x4 *>(part + base) = acc[i][j];
                } else {
#pragma unroll
                    for (int r = 0; r < 4; ++r)
                        if (n + r < p.N) part[base + r] = acc[i][j][r];
                }
            }
        }
        return;
    }
    if constexpr (ES == 2) {
        if (p.staged) {
            // The tile leaves through LDS (the ring is idle now): every lane
            // writes its 8 B pieces to a row-major copy, then each lane stores
            // 16 B of a row, so one store instruction writes whole 128 B lines
            // (the fragment layout writes 32 B of 16 rows each, and the stores
            // then took a fifth of a 256 x 256 x 1536 tile's time).
            using E = typename Elem<T>::type;
            typedef E e4 __attribute__((ext_vector_type(4)));
            constexpr int PITCH = stagePitch<BN>();
            char *stage = reinterpret_cast<char *>(lds);
            __syncthreads(); // every wave is done with the ring
            if constexpr (T == ElemType::BF16 && TN % 2 == 0) {
                if (p.swiglu) {
#pragma unroll
                    for (int j = 0; j < TM; ++j) {
                        const int ml = wm * (BM / WGM) + 16 * j + fr;
#pragma unroll
                        for (int t = 0; t < TN / 2; ++t) {
                            const int nl = (wn * (BN / WGN) + 32 * t) / 2 + 4 * fg; // act column in the tile
                            uint32_t w2[2];
#pragma unroll
                            for (int h = 0; h < 2; ++h) {
                                uint32_t pk = 0;
#pragma unroll
                                for (int e = 0; e < 2; ++e) {
                                    const float g = float(__bf16(acc[2 * t][j][2 * h + e]));
                                    const float u = float(__bf16(acc[2 * t + 1][j][2 * h + e]));
                                    pk |= uint32_t(__builtin_bit_cast(uint16_t, __bf16(u * g / (1.f + expf(-g)))))
                                          << (16 * e);
                                }
                                w2[h] = pk;
                            }
                            *reinterpret_cast<uint2 *>(stage + ml * PITCH + nl * 2) = make_uint2(w2[0], w2[1]);
                        }
                    }
                }
            }
            if (!p.swiglu) {
#pragma unroll
                for (int j = 0; j < TM; ++j) {
                    const int ml = wm * (BM / WGM) + 16 * j + fr, m = m0 + ml;
#pragma unroll
                    for (int i = 0; i < TN; ++i) {
                        const int nl = wn * (BN / WGN) + 16 * i + 4 * fg, n = n0 + nl;
                        f32x4 v = acc[i][j];
                        if (m < p.M && n < p.N) {
                            if (p.accumulate) v = load4<T>(p.y, size_t(m) * p.ldy + n) + v;
                            if (p.bias) v += load4<T>(p.bias, n);
                        }
                        *reinterpret_cast<e4 *>(stage + ml * PITCH + nl * 2) = e4{E(v[0]), E(v[1]), E(v[2]), E(v[3])};
                    }
                }
            }
            __syncthreads();
            // Rows out, 16 B (8 values) per lane.
            auto storeRows = [&](auto cpr_tag) {
                constexpr int CPR = decltype(cpr_tag)::value; // 16 B chunks per tile row
                const int n_out = p.swiglu ? p.N / 2 : p.N, c0 = p.swiglu ? n0 / 2 : n0;
#pragma unroll 4
                for (int q = tid; q < BM * CPR; q += 64 * NW) {
                    const int row = q / CPR, c = q % CPR;
                    const int m = m0 + row, col = c0 + 8 * c;
                    if (m < p.M && col < n_out)
                        *reinterpret_cast<u32x4 *>(static_cast<E *>(p.y) + size_t(m) * p.ldy + col) =
                            *reinterpret_cast<const u32x4 *>(stage + row * PITCH + c * 16);
                }
            };
            if (p.swiglu)
                storeRows(std::integral_constant<int, BN / 16>{});
            else
                storeRows(std::integral_constant<int, BN / 8>{});
            return;
        }
    }
    if constexpr (T == ElemType::BF16 && TN % 2 == 0) {
        if (p.swiglu) {
            // W fragments 2t and 2t + 1 of the wave are a gate block and its up
            // block (the wave's columns start at a multiple of 32): the lane
            // holds gate and up of the same four act columns. Both are rounded
            // to bf16 first, as the GEMM output swigluRows would read.
            const int da = p.ldy;
#pragma unroll
            for (int j = 0; j < TM; ++j) {
                const int m = m0 + wm * (BM / WGM) + 16 * j + fr;
                if (m >= p.M) continue;
#pragma unroll
                for (int t = 0; t < TN / 2; ++t) {
                    const int ng = n0 + wn * (BN / WGN) + 32 * t; // gate block 2 (ng / 32)
                    if (ng >= p.N) continue;
                    const int col = ng / 2 + 4 * fg;
                    uint32_t w2[2];
#pragma unroll
                    for (int h = 0; h < 2; ++h) {
                        uint32_t pk = 0;
#pragma unroll
                        for (int e = 0; e < 2; ++e) {
                            const float g = float(__bf16(acc[2 * t][j][2 * h + e]));
                            const float u = float(__bf16(acc[2 * t + 1][j][2 * h + e]));
                            pk |= uint32_t(__builtin_bit_cast(uint16_t, __bf16(u * g / (1.f + expf(-g))))) << (16 * e);
                        }
                        w2[h] = pk;
                    }
                    *reinterpret_cast<uint2 *>(static_cast<uint16_t *>(p.y) + size_t(m) * da + col) =
                        make_uint2(w2[0], w2[1]);
                }
            }
            return;
        }
    }
#pragma unroll
    for (int j = 0; j < TM; ++j) {
        const int m = m0 + wm * (BM / WGM) + 16 * j + fr;
        if (m >= p.M) continue;
#pragma unroll
        for (int i = 0; i < TN; ++i) {
            const int n = n0 + wn * (BN / WGN) + 16 * i + 4 * fg;
            if (n >= p.N) continue;
            const size_t base = size_t(m) * p.ldy + n;
            f32x4 v = acc[i][j];
            if (vec) {
                if (p.accumulate) v = load4<T>(p.y, base) + v;
                if (p.bias) v += load4<T>(p.bias, n);
                store4<T>(p.y, base, v);
            } else {
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    if (n + r >= p.N) break;
                    float e = v[r];
                    if (p.accumulate) e = loadElem<T>(p.y, base + r) + e;
                    if (p.bias) e += loadElem<T>(p.bias, n + r);
                    storeElem<T>(p.y, base + r, e);
                }
            }
        }
    }
}

// Shapes whose rows are not whole 16 B pieces (K * element size % 16 != 0,
// e.g. the reference test's K = 4): one thread per output, fp32 sum in k
// order, the same epilogue.
template <ElemType T>
__global__ void __launch_bounds__(256) gemmRowsKernel(void *y, const void *x, const void *w, const void *bias, int M,
                                                      int N, int K, int accumulate) {
    const size_t idx = size_t(blockIdx.x) * blockDim.x + threadIdx.x;
    if (idx >= size_t(M) * N) return;
    const int m = int(idx / N), n = int(idx % N);
    float sum = 0.f;
    for (int k = 0; k < K; ++k) sum = fmaf(loadElem<T>(x, size_t(m) * K + k), loadElem<T>(w, size_t(n) * K + k), sum);
    if (accumulate) sum = loadElem<T>(y, idx) + sum;
    if (bias) sum += loadElem<T>(bias, n);
    storeElem<T>(y, idx, sum);
}

// Y[m, n] = (old Y +) sum over s of part[s][m][n] (+ bias[n]), in split
// order, rounded once; one thread per 4 columns (N % 4 == 0) or per element.
template <ElemType T>
__global__ void __launch_bounds__(256) gemmReduceKernel(void *y, const float *part, const void *bias, int M, int N,
                                                        int S, int accumulate) {
    const size_t idx = size_t(blockIdx.x) * blockDim.x + threadIdx.x;
    const size_t stride = size_t(M) * N;
    if ((N & 3) == 0) {
        if (idx >= stride / 4) return;
        const size_t base = 4 * idx;
        f32x4 v = *reinterpret_cast<const f32x4 *>(part + base);
        for (int s = 1; s < S; ++s) v += *reinterpret_cast<const f32x4 *>(part + s * stride + base);
        if (accumulate) v = load4<T>(y, base) + v;
        if (bias) v += load4<T>(bias, base % N);
        store4<T>(y, base, v);
    } else {
        if (idx >= stride) return;
        float v = part[idx];
        for (int s = 1; s < S; ++s) v += part[s * stride + idx];
        if (accumulate) v = loadElem<T>(y, idx) + v;
        if (bias) v += loadElem<T>(bias, idx % N);
        storeElem<T>(y, idx, v);
    }
}

int cusOf() {
    static std::mutex mu;
    static std::vector<int> cache;
    int dev = 0;
    HIP_CHECK(hipGetDevice(&dev));
    std::lock_guard<std::mutex> lock(mu);
    if (size_t(dev) >= cache.size()) cache.resize(dev + 1, 0);
    if (!cache[dev]) HIP_CHECK(hipDeviceGetAttribute(&cache[dev], hipDeviceAttributeMultiprocessorCount, dev));
    return cache[dev];
}

template <ElemType T, int BM, int BN, int WGM, int WGN, bool PIPE, int RB = 64, int WS = 2>
void launchTileAs(GemmParams p, hipStream_t s) {
    const size_t lds = std::max(size_t(ringStages<PIPE, RB, WS>()) * stageBlocks<BM, BN, WGM * WGN, RB>() * 1024,
                                Elem<T>::size == 2 ? stageBytes<BM, BN>() : size_t(0));
    // The LDS limit is raised once per device the kernel runs on.
    static std::mutex mu;
    static std::vector<bool> raised;
    int dev = 0;
    HIP_CHECK(hipGetDevice(&dev));
    {
        std::lock_guard<std::mutex> lock(mu);
        if (size_t(dev) >= raised.size()) raised.resize(dev + 1, false);
        if (!raised[dev]) {
            HIP_CHECK(hipFuncSetAttribute(reinterpret_cast<const void *>(&gemmKernel<T, BM, BN, WGM, WGN, PIPE, RB, WS>),
                                          hipFuncAttributeMaxDynamicSharedMemorySize, int(lds)));
            raised[dev] = true;
        }
    }
    hipLaunchKernelGGL((gemmKernel<T, BM, BN, WGM, WGN, PIPE, RB, WS>), dim3(unsigned(p.mtiles * p.ntiles * p.splits)),
                       dim3(64 * WGM * WGN), lds, s, p);
}

// LLAISYS_GEMM_PIPE=0: the 4-stage ring whose waves read a stage's
// fragments only after its barrier.
bool pipelined() {
    static const bool v = [] { const char *e = std::getenv("LLAISYS_GEMM_PIPE"); return !(e && e[0] == '0'); }();
    return v;
}

// 16-bit tiles move k in 128 B row pieces (two stages) unless
// LLAISYS_GEMM_WIDE_K=0 (64 B pieces, four stages).
bool wideK() {
    static const bool v = [] { const char *e = std::getenv("LLAISYS_GEMM_WIDE_K"); return !(e && e[0] == '0'); }();
    return v;
}

template <ElemType T, int BM, int BN, int WGM = 2, int WGN = 2> void launchTile(GemmParams p, hipStream_t s) {
    if constexpr (Elem<T>::size == 2) {
        if (wideK()) {
            static const bool deep = [] { const char *e = std::getenv("LLAISYS_GEMM_WIDE_DEEP"); return !(e && e[0] == '0'); }();
            if (deep)
                launchTileAs<T, BM, BN, WGM, WGN, true, 128, wideStages<BM, BN, WGM * WGN>()>(p, s);
            else
                launchTileAs<T, BM, BN, WGM, WGN, true, 128, 2>(p, s);
            return;
        }
    }
    if (pipelined())
        launchTileAs<T, BM, BN, WGM, WGN, true>(p, s);
    else
        launchTileAs<T, BM, BN, WGM, WGN, false>(p, s);
}

// The (tile, K split) with the least estimated time. A launch runs
// ceil(workgroups / CUs) rounds; a round costs a fixed kFixedUs (first loads,
// epilogue) plus the tile's k loop, bm x bn x (K / split) at the tile's
// relative MFMA rate eff (bigger wave tiles read less LDS per MFMA); a split
// adds the reduce kernel, priced by its bytes (fp32 partials written and read
// back, the output written). Fitted to timings of the kernel on MI355X
// (bf16, M = 2048 / 8192 by the Qwen2 projection widths): e.g. 2048 x 2048 x
// 1536 runs 21.0 us on 128 x 128 tiles against 29 us on 128 x 256 tiles split
// in two, and 2048 x 1536 x 8960 85.8 us split in two against 93.5 us not.
struct Plan {
    int tile = 0; // index into kTiles
    int mtiles = 0, ntiles = 0, splits = 1;
    double est = 0; // the model's time, us
};
// narrow: waves 48 columns wide. 256 x 192 (8 waves of 128 x 48) and
// 128 x 96 (4 waves of 64 x 48) fill the 256 CUs where the tiles twice their
// size leave a quarter idle (8192 x 1536 x 1536: 256 tiles against 192, 44.6
// -> 40.2 us; 2048 x 1536 x 8960 split in 4: 76 -> 69.5 us). They run only
// where one round holds all their workgroups: over several (2048 x 17920 x
// 1536: 3 rounds, 128-131 us) 256 x 256 tiles with the column split below run
// faster (123-125 us) than the model prices them. Their wave columns are not
// whole SwiGLU block pairs, so the fused gate-up skips them.
struct TileShape { int bm, bn; double eff; bool narrow; };
constexpr TileShape kTiles[] = {{128, 256, 1.0, false}, {256, 128, 1.0, false}, {128, 128, 0.8, false},
                                {64, 64, 0.45, false},  {256, 256, 1.2, false}, {256, 192, 1.1, true},
                                {128, 96, 0.7, true}};
constexpr int kTile192 = 5, kTile96 = 6;
constexpr int kMinSplitTiles = 8;            // k tiles per split at least
constexpr double kFixedUs = 6.0;             // per round of workgroups
constexpr double kMacsPerUs = 2.1e6;         // bm * bn * k per us at eff 1 (bf16)
constexpr double kReduceBytesPerUs = 5.0e6;  // HBM rate of the reduce kernel
constexpr double kReduceLaunchUs = 2.0;

Plan planGemm(ElemType t, int M, int N, int K, bool no_split = false, bool swiglu = false) {
    const long cus = cusOf();
    const int es = t == ElemType::F32 ? 4 : 2;
    const int nk = (K * es + kRowBytes - 1) / kRowBytes;
    Plan best;
    double best_t = 1e300;
    // LLAISYS_GEMM_BIG=0 leaves out the 256 x 256 tile (8 waves of 128 x 64),
    // LLAISYS_GEMM_NARROW=0 the narrow ones.
    static const bool big = [] { const char *e = std::getenv("LLAISYS_GEMM_BIG"); return !(e && e[0] == '0'); }();
    static const bool narrow = [] { const char *e = std::getenv("LLAISYS_GEMM_NARROW"); return !(e && e[0] == '0'); }();
    for (int i = 0; i < int(sizeof(kTiles) / sizeof(kTiles[0])); ++i) {
        if (t == ElemType::F32 && i >= 4) break; // f32: 128 accumulators at most
        if ((i == 4 && !big) || (kTiles[i].narrow && (!narrow || swiglu))) continue;
        const TileShape &c = kTiles[i];
        const long mt = (M + c.bm - 1) / c.bm, nt = (N + c.bn - 1) / c.bn;
        for (int sp = 1; sp <= 8; sp *= 2) {
            if (sp > 1 && (no_split || nk / sp < kMinSplitTiles)) break;
            const long rounds = (mt * nt * sp + cus - 1) / cus;
            if (c.narrow && rounds > 1) continue;
            double tm = double(rounds) * (kFixedUs + double(c.bm) * c.bn * (double(K) / sp) / (c.eff * kMacsPerUs));
            if (sp > 1)
                tm += kReduceLaunchUs + (2.0 * sp * 4.0 + es) * double(M) * N / kReduceBytesPerUs;
            if (tm < best_t) {
                best_t = tm;
                best.tile = i;
                best.mtiles = int(mt);
                best.ntiles = int(nt);
                best.splits = sp;
                best.est = tm;
            }
        }
    }
    return best;
}

// A plan whose last round of workgroups leaves most CUs idle (2048 x 17920:
// 560 tiles of 256 x 256 in three rounds on 256 CUs, the last under a fifth
// full) runs as two launches instead: columns [0, na) on the plan's tiles in
// whole rounds, the rest on their own (smaller) tiles, when the model prices
// the two below the one. Splits of K are left alone. na is a multiple of the
// tile width (so of 64: whole SwiGLU pairs, 16 B aligned rows).
constexpr double kSecondLaunchUs = 3.0;
struct ColumnSplit {
    int na = 0; // 0: one launch
    Plan a, b;
};
ColumnSplit splitColumns(ElemType t, int M, int N, int K, const Plan &one, bool swiglu = false) {
    ColumnSplit cs;
    static const bool on = [] { const char *e = std::getenv("LLAISYS_GEMM_COLUMN_SPLIT"); return !(e && e[0] == '0'); }();
    if (!on || one.splits != 1 || N % 8 != 0) return cs; // (vector stores need rows of whole 16 B)
    const long cus = cusOf();
    const long tiles = long(one.mtiles) * one.ntiles, rounds = (tiles + cus - 1) / cus;
    if (rounds < 2 || tiles % cus == 0) return cs;
    const int nta = int((rounds - 1) * cus / one.mtiles); // column tiles that fill rounds - 1 rounds
    if (nta <= 0 || nta >= one.ntiles) return cs;
    const int na = nta * kTiles[one.tile].bn;
    const Plan a = planGemm(t, M, na, K, true, swiglu), b = planGemm(t, M, N - na, K, true, swiglu);
    if (a.est + b.est + kSecondLaunchUs < 0.95 * one.est) {
        cs.na = na;
        cs.a = a;
        cs.b = b;
    }
    return cs;
}

// LLAISYS_GEMM_STAGED=0: 16-bit tiles stored straight from the fragments.
bool stagedStores() {
    static const bool v = [] { const char *e = std::getenv("LLAISYS_GEMM_STAGED"); return !(e && e[0] == '0'); }();
    return v;
}

// 128 x 256 and 256 x 128 tiles with 8 waves (two per SIMD, 64 x 64 each)
// unless LLAISYS_GEMM_W8=0 (4 waves of 64 x 128): the second wave of a SIMD
// runs its MFMAs while the first waits on its fragment reads.
bool w8() {
    static const bool v = [] { const char *e = std::getenv("LLAISYS_GEMM_W8"); return !(e && e[0] == '0'); }();
    return v;
}

template <ElemType T> void launchGemm(GemmParams p, const Plan &plan, hipStream_t s) {
    p.mtiles = plan.mtiles;
    p.ntiles = plan.ntiles;
    p.splits = plan.splits;
    switch (plan.tile) {
    case 0:
        if (w8()) launchTile<T, 128, 256, 2, 4>(p, s);
        else launchTile<T, 128, 256>(p, s);
        break;
    case 1:
        if (w8()) launchTile<T, 256, 128, 4, 2>(p, s);
        else launchTile<T, 256, 128>(p, s);
        break;
    case 2: launchTile<T, 128, 128>(p, s); break;
    case 4:
        if constexpr (T != ElemType::F32) {
            launchTile<T, 256, 256, 2, 4>(p, s);
            break;
        }
        [[fallthrough]];
    case kTile192:
        if constexpr (T != ElemType::F32) {
            launchTile<T, 256, 192, 2, 4>(p, s);
            break;
        }
        [[fallthrough]];
    case kTile96:
        if constexpr (T != ElemType::F32) {
            launchTile<T, 128, 96>(p, s);
            break;
        }
        [[fallthrough]];
    default: launchTile<T, 64, 64>(p, s); break;
    }
    HIP_CHECK(hipGetLastError());
    if (plan.splits > 1) {
        const size_t n = (p.N & 3) == 0 ? size_t(p.M) * p.N / 4 : size_t(p.M) * p.N;
        hipLaunchKernelGGL(gemmReduceKernel<T>, dim3(unsigned((n + 255) / 256)), dim3(256), 0, s, p.y, p.part, p.bias,
                           p.M, p.N, plan.splits, p.accumulate);
        HIP_CHECK(hipGetLastError());
    }
}

// Rows of X per launch so that one launch's X stays inside a buffer's
// 32-bit range. (A tile overhangs the last row by < 256 rows: with rows
// under 8 MiB the byte offsets stay below 2^32.)
constexpr size_t kMaxBufferBytes = size_t(1) << 31;
constexpr size_t kMaxRowBytes = size_t(1) << 23;

bool tiled(ElemType t, int K) { return K > 0 && (size_t(K) * (t == ElemType::F32 ? 4 : 2)) % 16 == 0; }

int rowsPerLaunch(ElemType t, int M, int K) {
    const size_t row_bytes = size_t(K) * (t == ElemType::F32 ? 4 : 2);
    return int(std::min<size_t>(size_t(M), (kMaxBufferBytes - 1) / row_bytes));
}

} // namespace

// The fp32 partials of the largest launch: rows go out in launches of
// rowsPerLaunch rows and a last, shorter one, whose plan may split K where
// the full launches' does not.
size_t linearWorkspaceBytes(ElemType t, int M, int N, int K) {
    if (M <= 0 || N <= 0 || !tiled(t, K)) return 0;
    const int rpl = rowsPerLaunch(t, M, K);
    size_t need = 0;
    for (const int m : {rpl, M % rpl}) {
        if (m <= 0) continue;
        const Plan plan = planGemm(t, m, N, K);
        if (plan.splits > 1) need = std::max(need, size_t(plan.splits) * size_t(m) * N * sizeof(float));
    }
    return need;
}

void linear(void *y, const void *x, const void *w, const void *bias, ElemType t, int M, int N, int K, void *stream,
            bool accumulate, void *workspace) {
    if (M <= 0 || N <= 0) return;
    auto s = static_cast<hipStream_t>(stream);
    if (!tiled(t, K)) {
        const size_t n = size_t(M) * N;
        const dim3 grid(unsigned((n + 255) / 256));
        const int acc = accumulate ? 1 : 0, k = std::max(K, 0);
        switch (t) {
        case ElemType::BF16:
            hipLaunchKernelGGL(gemmRowsKernel<ElemType::BF16>, grid, dim3(256), 0, s, y, x, w, bias, M, N, k, acc);
            break;
        case ElemType::F16:
            hipLaunchKernelGGL(gemmRowsKernel<ElemType::F16>, grid, dim3(256), 0, s, y, x, w, bias, M, N, k, acc);
            break;
        case ElemType::F32:
            hipLaunchKernelGGL(gemmRowsKernel<ElemType::F32>, grid, dim3(256), 0, s, y, x, w, bias, M, N, k, acc);
            break;
        }
        HIP_CHECK(hipGetLastError());
        return;
    }
    const size_t es = t == ElemType::F32 ? 4 : 2;
    const size_t row_bytes = size_t(K) * es;
    LLAISYS_CHECK(size_t(N) * row_bytes < kMaxBufferBytes && row_bytes < kMaxRowBytes,
                  "linear: the weight (" << N << " x " << K << ") must be under 2 GiB, its rows under 8 MiB");
    const int rows_per_launch = rowsPerLaunch(t, M, K);
    for (int r0 = 0; r0 < M; r0 += rows_per_launch) {
        const int m = std::min(rows_per_launch, M - r0);
        const Plan plan = planGemm(t, m, N, K);
        LLAISYS_CHECK(plan.splits == 1 || workspace, "linear: this shape needs linearWorkspaceBytes() of workspace");
        // Columns [c0, c1) of this launch's rows on `pl` (y keeps its row stride N).
        auto run = [&](int c0, int c1, const Plan &pl) {
            GemmParams p{};
            p.y = static_cast<char *>(y) + (size_t(r0) * N + c0) * es;
            p.x = static_cast<const char *>(x) + size_t(r0) * row_bytes;
            p.w = static_cast<const char *>(w) + size_t(c0) * row_bytes;
            p.bias = bias ? static_cast<const char *>(bias) + size_t(c0) * es : nullptr;
            p.M = m;
            p.N = c1 - c0;
            p.K = K;
            p.ldy = N;
            p.accumulate = accumulate ? 1 : 0;
            p.x_bytes = uint32_t(size_t(m) * row_bytes);
            p.w_bytes = uint32_t(size_t(c1 - c0) * row_bytes);
            p.part = static_cast<float *>(workspace);
            p.staged = es == 2 && pl.splits == 1 && N % 8 == 0 && (c1 - c0) % 8 == 0 &&
                       reinterpret_cast<uintptr_t>(p.y) % 16 == 0 && stagedStores();
            switch (t) {
            case ElemType::BF16: launchGemm<ElemType::BF16>(p, pl, s); break;
            case ElemType::F16: launchGemm<ElemType::F16>(p, pl, s); break;
            case ElemType::F32: launchGemm<ElemType::F32>(p, pl, s); break;
            }
        };
        const ColumnSplit cs = splitColumns(t, m, N, K, plan);
        if (cs.na) {
            run(0, cs.na, cs.a);
            run(cs.na, N, cs.b);
        } else {
            run(0, N, plan);
        }
    }
}

bool linearSwigluSupported(ElemType t, int M, int di, int K) {
    return t == ElemType::BF16 && M > 0 && di > 0 && di % 16 == 0 && tiled(t, K) &&
           size_t(2 * di) * size_t(K) * 2 < kMaxBufferBytes && size_t(K) * 2 < kMaxRowBytes;
}

void linearSwiglu(void *act, const void *x, const void *w_interleaved, ElemType t, int M, int di, int K,
                  void *stream) {
    LLAISYS_CHECK(linearSwigluSupported(t, M, di, K),
                  "linearSwiglu: needs bf16, di % 16 == 0 and whole 16 B rows (M=" << M << " di=" << di << " K=" << K
                                                                                   << ")");
    auto s = static_cast<hipStream_t>(stream);
    const int N = 2 * di;
    const size_t row_bytes = size_t(K) * 2;
    const int rows_per_launch = rowsPerLaunch(t, M, K);
    for (int r0 = 0; r0 < M; r0 += rows_per_launch) {
        const int m = std::min(rows_per_launch, M - r0);
        const Plan plan = planGemm(t, m, N, K, true, true);
        // Columns [c0, c1) of the gate-up product, act columns [c0 / 2, c1 / 2).
        auto run = [&](int c0, int c1, const Plan &pl) {
            GemmParams p{};
            p.y = static_cast<uint16_t *>(act) + size_t(r0) * di + c0 / 2;
            p.x = static_cast<const char *>(x) + size_t(r0) * row_bytes;
            p.w = static_cast<const char *>(w_interleaved) + size_t(c0) * row_bytes;
            p.M = m;
            p.N = c1 - c0;
            p.K = K;
            p.ldy = di;
            p.x_bytes = uint32_t(size_t(m) * row_bytes);
            p.w_bytes = uint32_t(size_t(c1 - c0) * row_bytes);
            p.swiglu = 1;
            p.staged = di % 8 == 0 && ((c1 - c0) / 2) % 8 == 0 && reinterpret_cast<uintptr_t>(p.y) % 16 == 0 &&
                       stagedStores();
            launchGemm<ElemType::BF16>(p, pl, s);
        };
        const ColumnSplit cs = splitColumns(t, m, N, K, plan, true);
        if (cs.na) {
            run(0, cs.na, cs.a);
            run(cs.na, N, cs.b);
        } else {
            run(0, N, plan);
        }
    }
}

} // namespace llaisys::kernels
