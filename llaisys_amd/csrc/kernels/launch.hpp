// Host-side launchers for the HIP kernels. Plain pointers and sizes only; the
// op layer (ops/attention.cpp) validates tensors and calls these.
#pragma once

#include <cstddef>
#include <cstdint>

namespace llaisys::kernels {

// Page geometry fixed by the MI355X page format.
constexpr int kPageTokens = 16;
constexpr int kHeadDim = 128;
constexpr int kPageElems = kPageTokens * kHeadDim; // bf16 elements per (block, kv head) page

enum class ElemType { F32, F16, BF16 };

// Contiguous causal GQA attention (the reference's self_attention op).
// Small grids (few query rows x heads) split the keys over workgroups into
// fp32 partials in `workspace` (selfAttentionWorkspaceBytes; 0: none needed).
size_t selfAttentionWorkspaceBytes(int L, int S, int nh, int dv);
void selfAttention(void *out, const void *q, const void *k, const void *v, ElemType type, int L, int S, int nh,
                   int nkvh, int d, int dv, float scale, void *stream, void *workspace);

// Paged KV append; cu_new may be null (one token per sequence, T == B).
void pagedAppend(uint16_t *k_pool, uint16_t *v_pool, const uint16_t *k_new, const uint16_t *v_new,
                 const int32_t *block_table, const int32_t *ctx_len, const int32_t *cu_new, int T, int B, int nkvh,
                 int max_pages, int num_blocks, int *err, void *stream);

void pagedGather(uint16_t *k_out, uint16_t *v_out, const uint16_t *k_pool, const uint16_t *v_pool,
                 const int32_t *block_table, const int32_t *cu_seqlens, int T, int B, int nkvh, int max_pages,
                 int num_blocks, int *err, void *stream);

// Append of one token per sequence (k_new/v_new [B, nkvh, 128]) fused into the
// gather of the contexts including it (cu_seqlens[b+1] - cu_seqlens[b] must be
// ctx_len[b] + 1).
void pagedAppendGather(uint16_t *k_out, uint16_t *v_out, uint16_t *k_pool, uint16_t *v_pool, const uint16_t *k_new,
                       const uint16_t *v_new, const int32_t *block_table, const int32_t *ctx_len,
                       const int32_t *cu_seqlens, int T, int B, int nkvh, int max_pages, int num_blocks, int *err,
                       void *stream);

// Batched decode: stream-K over all page pairs, then a combine kernel for
// sequences split across waves. cu_q == nullptr: sequence b's query is row b
// (T == B); else its row is cu_q[b] and sequences with cu_q[b+1]-cu_q[b] != 1
// are skipped (left to pagedPrefill). out_packed (bf16 only): the rows go
// there in operand order (packedRowIndex over nh * 128 columns) instead of to
// out, for a packed-X projection after it.
struct DecodePlan {
    int waves;           // grid of single-wave workgroups
    int stages;          // page pairs in flight per wave
    size_t record_bytes; // workspace for split records
    size_t lds_bytes;    // per-workgroup LDS (length prefix)
    size_t slot_headers;      // per-unit record slot headers (int32; 0: per-wave records only)
    size_t slot_record_bytes; // per-unit record slots
};
constexpr int kDecodeMaxBatch = 4096; // sequences per launch (LDS-resident prefix)
DecodePlan planDecode(int B, int nkvh, int group, int max_pages);
void pagedDecode(void *out, bool out_f32, const uint16_t *q, const uint16_t *k_pool, const uint16_t *v_pool,
                 const int32_t *block_table, const int32_t *ctx_len, const int32_t *cu_q, int B, int T, int nh,
                 int nkvh, int max_pages, int num_blocks, float scale, const DecodePlan &plan, float *records,
                 int *err, int *slot_headers, void *slot_records, void *stream, uint16_t *out_packed = nullptr);

// The same attention (cu_q null: query row b is sequence b) with one
// workgroup of 4 waves per (sequence, kv head), merging in LDS: no records,
// one launch. For batches whose contexts are of similar length (the waves
// of a long sequence's workgroup would otherwise finish last). out_packed
// (bf16 only): the output rows in operand order (packedRowIndex) there
// instead of in out.
void pagedDecodeUnits(void *out, bool out_f32, const uint16_t *q, const uint16_t *k_pool, const uint16_t *v_pool,
                      const int32_t *block_table, const int32_t *ctx_len, int B, int nh, int nkvh, int max_pages,
                      int num_blocks, float scale, int *err, void *stream, uint16_t *out_packed = nullptr);

// pagedDecodeUnits with the decode step's QKV epilogue fused in (one token per
// sequence): from qkv [B, (nh + 2 nkvh) * 128] (projection rows before bias)
// each workgroup forms its unit's query heads and k/v head as qkvRopeAppend
// does (x: residual rows whose RMSNorm is folded into the projection, or
// null; position ctx_len[b] - 1), stores k/v into their page slot and attends
// with q straight from LDS. Needs nh / nkvh <= 6 and head dim 128
// (decodeUnitsRopeSupported). out_packed (bf16 only): write the [B, nh * 128]
// output rows in operand order (packedRowIndex) there instead of to out.
bool decodeUnitsRopeSupported(int nh, int nkvh, int d);
void pagedDecodeUnitsRope(void *out, bool out_f32, uint16_t *k_pool, uint16_t *v_pool, const uint16_t *qkv,
                          const uint16_t *bias, const uint16_t *x, int hs, float eps, float theta,
                          const int32_t *block_table, const int32_t *ctx_len, int B, int nh, int nkvh, int max_pages,
                          int num_blocks, float scale, int *err, void *stream, uint16_t *out_packed = nullptr);

// The decode above with its split records in a fixed per-GPU device array
// (noAllocScratchBytes() bytes) instead of runtime workspace: no device
// allocation per call. noAllocInit() looks the array's address up for the
// current device (once per device; the runtime's set-up calls it). Calls that
// overlap on one GPU share the array and race.
void noAllocInit();
size_t noAllocScratchBytes();
void pagedDecodeNoAlloc(void *out, bool out_f32, const uint16_t *q, const uint16_t *k_pool, const uint16_t *v_pool,
                        const int32_t *block_table, const int32_t *ctx_len, int B, int nh, int nkvh, int max_pages,
                        int num_blocks, float scale, int *err, void *stream);

// Chunked prefill: the sequences of a varlen batch with >= 2 queries, as
// (16-column query tile, kv head) units split over pages, then a combine kernel.
// Copy whole blocks (all kv heads, K and V): pairs[P][2] = (src, dst).
void pagedCopyBlocks(uint16_t *k_pool, uint16_t *v_pool, const int32_t *pairs, int P, int nkvh, int num_blocks,
                     int *err, void *stream);

struct PagedAttentionPlan {
    int units;           // (query group, kv head) record units (upper bound)
    int units_padded;    // same (kept for callers sizing by it)
    int block_units;     // (block of groups, kv head) workgroup units (upper bound)
    int block_units_padded; // rounded up to a multiple of the XCD count
    int max_splits;      // split-KV partitions per unit
    int pages_per_split;
    size_t partial_bytes; // workspace for split records
};
PagedAttentionPlan planPrefill(int B, int T, int nkvh, int group, int max_pages);
// Whether pagedPrefill runs its persistent kernel (the work-queue counters
// given, the batch's tables fit its LDS) and, then, whether that kernel also
// takes the batch's single-query sequences (T != B), in which case the
// caller runs no pagedDecode for them.
bool prefillQueueUsable(int B, const PagedAttentionPlan &plan, const int *queue);
bool prefillTakesDecode(int B, int T, const PagedAttentionPlan &plan, const int *queue);
// queue: two zeroed int32 counters that persist between calls (the
// persistent kernel's work queue, left zero when it ends), or null for one
// workgroup per (block, split) slot.
void pagedPrefill(void *out, bool out_f32, const uint16_t *q, const uint16_t *k_pool, const uint16_t *v_pool,
                  const int32_t *block_table, const int32_t *ctx_len, const int32_t *cu_q, int B, int T, int nh,
                  int nkvh, int max_pages, int num_blocks, float scale, const PagedAttentionPlan &plan,
                  float *records, int *err, int *queue, void *stream);

// ---- model ops (model_ops.hip, linear.cpp)
constexpr int kMaxDims = 8;
void add(void *c, const void *a, const void *b, ElemType t, size_t n, void *stream);
void swiglu(void *out, const void *gate, const void *up, ElemType t, size_t n, void *stream);
void addBias(void *x, const void *bias, ElemType t, size_t rows, size_t cols, void *stream);
// x[r, c] = row[c] for every row r.
void fillRows(void *x, const void *row, ElemType t, size_t rows, size_t cols, void *stream);
void rmsNorm(void *out, const void *x, const void *w, ElemType t, size_t rows, int d, float eps, void *stream);
void rope(void *out, const void *in, const int64_t *pos, ElemType t, size_t ntok, int nhead, int d, float theta,
          void *stream);
void embedding(void *out, const int64_t *idx, const void *weight, ElemType t, size_t rows, int64_t vocab, int d,
               int *err, void *stream);
// Row-wise argmax over the last dim: idx[rows] (first maximum; NaN counts as
// the largest value), val[rows] (may be null); workspace of argmaxWorkspaceBytes().
size_t argmaxWorkspaceBytes(size_t rows, int64_t n);
// idx[r] = the column of the maximum of keys[r * chunks .. + chunks) (argmaxKey).
void argmaxFinishKeys(int64_t *idx, const uint64_t *keys, size_t rows, int chunks, void *stream);
void argmax(int64_t *idx, void *val, const void *vals, ElemType t, size_t rows, int64_t n, void *workspace,
            void *stream);
void rearrange(void *out, const void *in, size_t esz, int ndim, const int64_t *shape, const int64_t *out_strides,
               const int64_t *in_strides, void *stream);
// Y[M, N] = X[M, K] . W[N, K]^T (+ bias[N]), row-major, fp32 accumulation
// (gemm.hip's MFMA GEMM). accumulate: Y += X . W^T (+ bias) instead (a
// residual add folded into the GEMM). Shapes that leave CUs idle split K
// into fp32 partials in `workspace` (linearWorkspaceBytes; 0 = none needed).
size_t linearWorkspaceBytes(ElemType t, int M, int N, int K);
void linear(void *y, const void *x, const void *w, const void *bias, ElemType t, int M, int N, int K, void *stream,
            bool accumulate, void *workspace);
// act[M, di] = up * silu(gate) of X[M, K] . W^T, one launch: the same GEMM with
// W = swigluInterleave's row order of a [gate (di) | up (di)] weight, gate and
// up rounded to bf16 before the SwiGLU (bit for bit linear() + swigluRows()).
// bf16, di % 16 == 0, K * 2 % 16 == 0; K is never split.
bool linearSwigluSupported(ElemType t, int M, int di, int K);
void linearSwiglu(void *act, const void *x, const void *w_interleaved, ElemType t, int M, int di, int K,
                  void *stream);

// ---- decode-sized projections (decode_gemm.hip), bf16
// Y[M, N] (+)= X[M, K] . W[N, K]^T for M <= kDecodeGemmMaxM, K == kDecodeGemmK,
// N % 16 == 0, with W pre-packed by packWeight (N * K elements, MFMA operand
// order; fold_g, if given, multiplies column k by fold_g[k] before the one
// rounding to bf16). accumulate adds the old Y before the one rounding (a
// bias enters that way: preset Y's rows to it).
constexpr int kDecodeGemmMaxM = 128;
constexpr int kDecodeGemmK = 1536;
bool decodeGemmSupported(int M, int N, int K);
size_t packedWeightElems(int N, int K);
void packWeight(uint16_t *packed, const uint16_t *w, const uint16_t *fold_g, int N, int K, void *stream);
// packWeight of a fused [gate; up] weight (2 di rows) with the halves
// interleaved: 16-row block b holds gate rows 8b .. 8b + 7, then up rows
// 8b .. 8b + 7 (di % 8 == 0). A product over it has gate columns 8b + e at
// 16b + e and up columns at 16b + 8 + e (swigluRows' interleaved layout).
void packWeightGateUp(uint16_t *packed, const uint16_t *w, int di, int K, void *stream);
void decodeGemm(uint16_t *y, const uint16_t *x, const uint16_t *packed, int M, int N, int K, bool accumulate,
                void *stream, uint64_t *argmax_keys = nullptr);
// argmax_keys (M <= 64 or N >= 8192): each workgroup also leaves, per row,
// the argmax key of the bf16 values it stored (argmaxKey), at
// argmax_keys[m * decodeGemmKeyChunks(N) + workgroup]; argmaxFinishKeys
// turns them into the rows' first maximum.
int decodeGemmKeyChunks(int N);
// The same product for long K (kDecodeGemmK < K <= kSplitKMaxK, K % 32 == 0,
// N % 128 == 0, M <= kDecodeGemmMaxM), same packed W: K splits over
// workgroups into fp32 partials (splitKWorkspaceBytes of device memory),
// summed in a fixed order by a second kernel that also adds the old Y
// (accumulate) and rounds once.
constexpr int kSplitKMaxK = 16384;
bool splitKGemmSupported(int M, int N, int K);
size_t splitKWorkspaceBytes(int M, int N, int K);
void splitKGemm(uint16_t *y, const uint16_t *x, const uint16_t *packed, int M, int N, int K, bool accumulate,
                float *partials, void *stream, uint16_t *y_packed = nullptr);
// Rows in operand order: element (m, k) of an [M, K] matrix (K % 32 == 0)
// kept the way packWeight keeps a weight, 16-row blocks of 1 KiB tiles, so
// one 64-lane x 16 B load is an MFMA operand as loaded. Producers that write
// a packed copy beside (or instead of) the row-major rows use this index;
// a buffer holds ceil(M / 16) whole blocks (rows past M are never read back
// into an output).
__host__ __device__ inline size_t packedRowIndex(int m, int k, int K) {
    return ((size_t(m >> 4) * size_t(K >> 5) + size_t(k >> 5)) * 64 + size_t(m & 15) + 16 * ((k >> 3) & 3)) * 8 +
           size_t(k & 7);
}
inline size_t packedRowsElems(int M, int K) { return size_t((M + 15) / 16) * 16 * size_t(K); }
// Y[M, N] (+)= X . W^T with X given packed (packedRowIndex) as well as W
// (packWeight), for M <= kDecodeGemmMaxM, K == kDecodeGemmK, N % 32 == 0:
// one workgroup per 32 x 32 tile of Y, its 4 waves splitting K, every operand
// load issued before the first MFMA.
bool packedXGemmSupported(int M, int N, int K);
void packedXGemm(uint16_t *y, const uint16_t *x_packed, const uint16_t *w_packed, int M, int N, int K,
                 bool accumulate, void *stream, uint16_t *y_packed = nullptr);
// act[M, di] = up * silu(gate) of r * (x [gate; up]^T), r = 1/sqrt(mean(x^2)
// + eps) per row, for x given packed ([M, K], K == kDecodeGemmK, M <=
// kDecodeGemmMaxM) and the gate/up weight packed by packWeightGateUp (its
// RMSNorm weight folded in): the gate-up projection, the row's 1/rms and the
// SwiGLU in one kernel, from fp32 sums (no bf16 gate/up rows in between).
// The QKV projection of a decode step (one token per row: row m is sequence
// m at position ctx[m]) with qkvRopeAppend's epilogue in the GEMM: y = r *
// (x W^T) + bias (r: the row's 1/rms, W with the RMSNorm weight folded in),
// q and k heads rotated, q to q [M, nh, 128], k and v stored into their page
// slot (block table [M, max_pages]; err bits as qkvRopeAppend). x packed,
// W packed (packWeight), K == kDecodeGemmK, M <= kDecodeGemmMaxM.
bool qkvRopeGemmSupported(int M, int nh, int nkvh, int K);
void qkvRopeGemm(uint16_t *q, uint16_t *k_pool, uint16_t *v_pool, const uint16_t *x_packed, const uint16_t *w_packed,
                 const uint16_t *bias, const int32_t *table, const int32_t *ctx, int M, int nh, int nkvh, int K,
                 int max_pages, int num_blocks, float eps, float theta, int *err, void *stream);
bool gateUpSwigluSupported(int M, int di, int K);
void gateUpSwiglu(uint16_t *act, const uint16_t *x_packed, const uint16_t *w_packed, int M, int di, int K, float eps,
                  void *stream, bool act_packed = false); // act_packed: act written in operand order
// The split-K product over packed X (K > kDecodeGemmK, N % 64 == 0, M <=
// kDecodeGemmMaxM; W packed by packWeight): X streams through registers
// beside W instead of being staged in LDS, so each workgroup covers a longer
// k range and the fp32 partials (splitKPackedWorkspaceBytes) are fewer; the
// reduce adds the old Y (accumulate), rounds once and, given y_packed, also
// writes Y in operand order.
bool splitKPackedSupported(int M, int N, int K);
size_t splitKPackedWorkspaceBytes(int M, int N, int K);
void splitKPackedGemm(uint16_t *y, const uint16_t *x_packed, const uint16_t *w_packed, int M, int N, int K,
                      bool accumulate, float *partials, void *stream, uint16_t *y_packed = nullptr);

// ---- Qwen2 step glue (qwen2_step.hip), bf16
// qkv [T, (nh + 2 nkvh) d] + bias -> q [T, nh, d] rotated by position, and k
// (rotated) and v written
// into the paged pool at each token's position (decode: cu == null, T == B;
// else row r belongs to the sequence b with cu[b] <= r < cu[b+1]);
// ctx = lengths before the append. Error bits 1 (bad block), 2 (past table).
// x (may be null): residual rows [T, hs] whose RMSNorm weight was folded into
// the QKV weights; qkv is then scaled by each row's 1/rms before the bias.
void qkvRopeAppend(uint16_t *q, uint16_t *k_pool, uint16_t *v_pool, const uint16_t *qkv, const uint16_t *bias,
                   const int32_t *table, const int32_t *ctx, const int32_t *cu, int T, int B, int nh, int nkvh, int d,
                   int max_pages, int num_blocks, float theta, int *err, const uint16_t *x, int hs, float eps,
                   void *stream);
// act [T, di] = up * silu(gate) with gate_up rows [gate (di) | up (di)]; di % 8 == 0.
// x (may be null): as for qkvRopeAppend, gate and up scaled by the row's 1/rms.
// interleaved: rows in packWeightGateUp's column order instead (gate columns
// 8b + e at 16b + e, up columns at 16b + 8 + e).
void swigluRows(uint16_t *act, const uint16_t *gate_up, const uint16_t *x, size_t T, int di, int hs, float eps,
                void *stream, bool interleaved = false);
// out[r, c] = w[r, c] * g[c] (bf16, one rounding): an RMSNorm weight folded
// into the columns of the projection that consumes the normalised rows.
void foldNormColumns(uint16_t *out, const uint16_t *w, const uint16_t *g, size_t rows, int cols, void *stream);
// out = the rows of w [gate (di) | up (di)] as 16-row blocks gate 0, up 0,
// gate 1, up 1, ... (linearSwiglu's weight order); di % 16 == 0.
void swigluInterleave(uint16_t *out, const uint16_t *w, int di, int cols, void *stream);
// Multi-step decode bookkeeping on the device (s = *counter, the steps
// started): before step s, history[s - 1][:] = next (s > 0), ctx_before =
// base + s, ctx_after = base + s + 1, tok = s ? next : first, *counter = s + 1;
// after the last step, decodeRecordLast sets history[*counter - 1][:] = next.
void decodeAdvance(int32_t *ctx_before, int32_t *ctx_after, int64_t *tok, int64_t *history, const int32_t *base,
                   const int64_t *first, const int64_t *next, int32_t *counter, int B, void *stream);
void decodeRecordLast(int64_t *history, const int64_t *next, const int32_t *counter, int B, void *stream);
// x[r] = weight[idx[r]] for r < T (bf16 rows of d, d % 32 == 0; an index
// outside [0, vocab) sets bit 4 of err and leaves the row), also written in
// operand order to x_packed (packedRowIndex over d columns).
void embedRowsPacked(uint16_t *x, uint16_t *x_packed, const int64_t *idx, const uint16_t *weight, int T,
                     int64_t vocab, int d, int *err, void *stream);
// out [R, d] = rms_norm(x[rows ? rows[r] : r]) * w; d % 8 == 0.
void rmsNormRows(uint16_t *out, const uint16_t *x, const int64_t *rows, const uint16_t *w, size_t R, int d, float eps,
                 void *stream);

} // namespace llaisys::kernels
