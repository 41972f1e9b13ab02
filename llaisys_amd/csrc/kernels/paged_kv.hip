// Paged KV append (scatter) and gather kernels for gfx950.
//
// Page format (one (block, kv head) page = 16 tokens x 128 dims bf16 = 4 KiB):
//   K: index(t, d) = (d/8)*128 + t*8 + d%8
//   V: index(t, d) = (d/32)*512 + (t/4)*128 + (d%16)*8 + ((d/16)%2)*4 + t%4
// Each 1 KiB quarter of a page is what one wave's 64 lanes x 16 B load hands
// to an MFMA operand in the attention kernel.
#include "launch.hpp"

#include "../device/hip_check.hpp"

namespace llaisys::kernels {

namespace {

constexpr int kErrBadBlock = 1;
constexpr int kErrTooLong = 2;

__device__ __forceinline__ int kIndex(int t, int d) { return (d >> 3) * 128 + t * 8 + (d & 7); }
__device__ __forceinline__ int vIndex(int t, int d) {
    return (d >> 5) * 512 + (t >> 2) * 128 + (d & 15) * 8 + ((d >> 4) & 1) * 4 + (t & 3);
}

// Sequence owning row r: largest b with cu[b] <= r (cu non-decreasing, cu[0] = 0).
__device__ int owningSequence(const int32_t *cu, int B, int r) {
    int lo = 0, hi = B - 1;
    while (lo < hi) {
        int mid = (lo + hi + 1) >> 1;
        if (cu[mid] <= r)
            lo = mid;
        else
            hi = mid - 1;
    }
    return lo;
}

// One 64-lane block per new token row; each lane moves 16 B chunks (8 dims).
// The row's own loads do not depend on the position or the block table, so
// each lane's first chunk is loaded before those lookups.
__global__ void __launch_bounds__(64) appendKernel(uint16_t *__restrict__ k_pool, uint16_t *__restrict__ v_pool,
                                                   const uint16_t *__restrict__ k_new,
                                                   const uint16_t *__restrict__ v_new,
                                                   const int32_t *__restrict__ table, const int32_t *__restrict__ ctx,
                                                   const int32_t *__restrict__ cu, int B, int nkvh, int max_pages,
                                                   int num_blocks, int *err) {
    const int r = blockIdx.x;
    const int chunks = nkvh * 16; // 16 chunks of 8 dims per kv head
    const size_t row = size_t(r) * nkvh * kHeadDim;
    uint4 k0 = {}, v0 = {};
    if (int(threadIdx.x) < chunks) {
        k0 = *reinterpret_cast<const uint4 *>(k_new + row + threadIdx.x * 8);
        v0 = *reinterpret_cast<const uint4 *>(v_new + row + threadIdx.x * 8);
    }
    int b, pos;
    if (cu) {
        b = owningSequence(cu, B, r);
        pos = ctx[b] + (r - cu[b]);
    } else {
        b = r;
        pos = ctx[b];
    }
    const int page = pos >> 4;
    const int t = pos & 15;
    if (pos < 0 || page >= max_pages) {
        if (threadIdx.x == 0) atomicOr(err, kErrTooLong);
        return;
    }
    const int blk = table[size_t(b) * max_pages + page];
    if (blk < 0 || blk >= num_blocks) {
        if (threadIdx.x == 0) atomicOr(err, kErrBadBlock);
        return;
    }
    for (int c = threadIdx.x; c < chunks; c += 64) {
        const int h = c >> 4;
        const int d0 = (c & 15) * 8;
        const uint4 kv = c < 64 ? k0 : *reinterpret_cast<const uint4 *>(k_new + row + c * 8);
        const uint4 vv = c < 64 ? v0 : *reinterpret_cast<const uint4 *>(v_new + row + c * 8);
        const size_t page_base = (size_t(blk) * nkvh + h) * kPageElems;
        // K: 8 consecutive dims are contiguous in the page -> one 16 B store.
        *reinterpret_cast<uint4 *>(k_pool + page_base + kIndex(t, d0)) = kv;
        // V: 8 consecutive dims land 8 elements apart.
        const uint32_t w[4] = {vv.x, vv.y, vv.z, vv.w};
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const uint16_t val = uint16_t(w[e >> 1] >> ((e & 1) * 16));
            v_pool[page_base + vIndex(t, d0 + e)] = val;
        }
    }
}

// One 256-thread block per (page, sequence, kv head). The K and V pages are
// staged through LDS in page format and written out row-major, each token row
// (256 B) by 16 consecutive threads.
__global__ void __launch_bounds__(256) gatherKernel(uint16_t *__restrict__ k_out, uint16_t *__restrict__ v_out,
                                                    const uint16_t *__restrict__ k_pool,
                                                    const uint16_t *__restrict__ v_pool,
                                                    const int32_t *__restrict__ table, const int32_t *__restrict__ cu,
                                                    int T, int nkvh, int max_pages, int num_blocks, int *err) {
    __shared__ uint4 ks[256];
    __shared__ uint16_t vs[kPageElems];
    const int page = blockIdx.x;
    const int b = blockIdx.y;
    const int h = blockIdx.z;
    // The table entry does not depend on the lengths: both loads go out together.
    const int blk = table[size_t(b) * max_pages + page];
    const int row0 = cu[b];
    const int len = cu[b + 1] - row0;
    if (page * 16 >= len) return;
    if (row0 < 0 || cu[b + 1] > T) { // rows outside k_out/v_out: refuse the sequence
        if (threadIdx.x == 0) atomicOr(err, kErrTooLong);
        return;
    }
    if (page == max_pages - 1 && len > max_pages * 16 && threadIdx.x == 0) atomicOr(err, kErrTooLong);
    if (blk < 0 || blk >= num_blocks) {
        if (threadIdx.x == 0) atomicOr(err, kErrBadBlock);
        return;
    }
    const size_t page_base = (size_t(blk) * nkvh + h) * kPageElems;
    const int tid = threadIdx.x;
    ks[tid] = reinterpret_cast<const uint4 *>(k_pool + page_base)[tid];
    reinterpret_cast<uint4 *>(vs)[tid] = reinterpret_cast<const uint4 *>(v_pool + page_base)[tid];
    __syncthreads();
    const int t = tid >> 4;
    const int c = tid & 15;
    if (page * 16 + t >= len) return;
    const size_t dst = (size_t(row0 + page * 16 + t) * nkvh + h) * kHeadDim + c * 8;
    // K chunk c of token t sits at page index c*128 + t*8, i.e. uint4 slot c*16 + t.
    *reinterpret_cast<uint4 *>(k_out + dst) = ks[c * 16 + t];
    uint32_t w[4];
#pragma unroll
    for (int e = 0; e < 8; e += 2) {
        const uint32_t lo = vs[vIndex(t, c * 8 + e)];
        const uint32_t hi = vs[vIndex(t, c * 8 + e + 1)];
        w[e >> 1] = lo | (hi << 16);
    }
    *reinterpret_cast<uint4 *>(v_out + dst) = make_uint4(w[0], w[1], w[2], w[3]);
}

// Append then gather in one launch, for one new token per sequence: the
// gather grid of gatherKernel, where the block holding page ctx[b] / 16 of
// sequence b also writes the new token's K/V (k_new/v_new row b) into slot
// ctx[b] % 16 of that page, in the pool and in its LDS copy, before the rows
// go out. Output rows of sequence b: [cu[b], cu[b+1]) with cu[b+1] - cu[b]
// == ctx[b] + 1 (other sequences raise kErrTooLong and are skipped). Same
// bytes as appendKernel followed by gatherKernel; the append's own chain of
// lookups no longer runs ahead of the gather.
__global__ void __launch_bounds__(256) appendGatherKernel(
    uint16_t *__restrict__ k_out, uint16_t *__restrict__ v_out, uint16_t *__restrict__ k_pool,
    uint16_t *__restrict__ v_pool, const uint16_t *__restrict__ k_new, const uint16_t *__restrict__ v_new,
    const int32_t *__restrict__ table, const int32_t *__restrict__ ctx, const int32_t *__restrict__ cu, int T,
    int nkvh, int max_pages, int num_blocks, int *err) {
    __shared__ uint4 ks[256];
    __shared__ uint16_t vs[kPageElems];
    const int page = blockIdx.x;
    const int b = blockIdx.y;
    const int h = blockIdx.z;
    const int tid = threadIdx.x;
    // None of these loads depends on another: all go out together.
    const int blk = table[size_t(b) * max_pages + page];
    const int c = ctx[b];
    const int row0 = cu[b];
    const int len = cu[b + 1] - row0;
    // The new row does not depend on the lookups either.
    const size_t new_row = (size_t(b) * nkvh + h) * kHeadDim;
    uint4 kv = {};
    uint16_t vv = 0;
    if (tid < 16)
        kv = reinterpret_cast<const uint4 *>(k_new + new_row)[tid];
    else if (tid < 16 + kHeadDim)
        vv = v_new[new_row + tid - 16];
    if (c < 0 || len != c + 1) { // output rows must hold the context plus the new token
        if (page == 0 && h == 0 && tid == 0) atomicOr(err, kErrTooLong);
        return;
    }
    if (page * 16 >= len) return;
    if (row0 < 0 || cu[b + 1] > T) {
        if (tid == 0) atomicOr(err, kErrTooLong);
        return;
    }
    if (page == max_pages - 1 && len > max_pages * 16 && tid == 0) atomicOr(err, kErrTooLong);
    if (blk < 0 || blk >= num_blocks) {
        if (tid == 0) atomicOr(err, kErrBadBlock);
        return;
    }
    const size_t page_base = (size_t(blk) * nkvh + h) * kPageElems;
    ks[tid] = reinterpret_cast<const uint4 *>(k_pool + page_base)[tid];
    reinterpret_cast<uint4 *>(vs)[tid] = reinterpret_cast<const uint4 *>(v_pool + page_base)[tid];
    if (page == (c >> 4)) { // block-uniform: this block's page receives the new token
        const int slot = c & 15;
        __syncthreads(); // the page is in LDS before its slot is overwritten
        if (tid < 16) {
            ks[tid * 16 + slot] = kv; // K chunk tid of token `slot`
            *reinterpret_cast<uint4 *>(k_pool + page_base + kIndex(slot, tid * 8)) = kv;
        } else if (tid < 16 + kHeadDim) {
            const int d = tid - 16;
            vs[vIndex(slot, d)] = vv;
            v_pool[page_base + vIndex(slot, d)] = vv;
        }
    }
    __syncthreads();
    const int t = tid >> 4;
    const int cc = tid & 15;
    if (page * 16 + t >= len) return;
    const size_t dst = (size_t(row0 + page * 16 + t) * nkvh + h) * kHeadDim + cc * 8;
    *reinterpret_cast<uint4 *>(k_out + dst) = ks[cc * 16 + t];
    uint32_t w[4];
#pragma unroll
    for (int e = 0; e < 8; e += 2) {
        const uint32_t lo = vs[vIndex(t, cc * 8 + e)];
        const uint32_t hi = vs[vIndex(t, cc * 8 + e + 1)];
        w[e >> 1] = lo | (hi << 16);
    }
    *reinterpret_cast<uint4 *>(v_out + dst) = make_uint4(w[0], w[1], w[2], w[3]);
}

// One 256-thread block per (pair, pool): 16 B per thread per 4 KiB page,
// looping over the kv heads of the block.
__global__ void __launch_bounds__(256) copyBlocksKernel(uint16_t *__restrict__ k_pool, uint16_t *__restrict__ v_pool,
                                                        const int32_t *__restrict__ pairs, int nkvh, int num_blocks,
                                                        int *err) {
    const int src = pairs[2 * blockIdx.x];
    const int dst = pairs[2 * blockIdx.x + 1];
    if (src < 0 || src >= num_blocks || dst < 0 || dst >= num_blocks) {
        if (threadIdx.x == 0) atomicOr(err, kErrBadBlock);
        return;
    }
    uint4 *pool = reinterpret_cast<uint4 *>(blockIdx.y == 0 ? k_pool : v_pool);
    const size_t per_block = size_t(nkvh) * kPageElems / 8; // uint4 per block
    for (size_t i = threadIdx.x; i < per_block; i += 256) pool[dst * per_block + i] = pool[src * per_block + i];
}

} // namespace

void pagedCopyBlocks(uint16_t *k_pool, uint16_t *v_pool, const int32_t *pairs, int P, int nkvh, int num_blocks,
                     int *err, void *stream) {
    if (P == 0) return;
    hipLaunchKernelGGL(copyBlocksKernel, dim3(P, 2), dim3(256), 0, static_cast<hipStream_t>(stream), k_pool, v_pool,
                       pairs, nkvh, num_blocks, err);
    HIP_CHECK(hipGetLastError());
}

void pagedAppend(uint16_t *k_pool, uint16_t *v_pool, const uint16_t *k_new, const uint16_t *v_new,
                 const int32_t *block_table, const int32_t *ctx_len, const int32_t *cu_new, int T, int B, int nkvh,
                 int max_pages, int num_blocks, int *err, void *stream) {
    if (T == 0) return;
    hipLaunchKernelGGL(appendKernel, dim3(T), dim3(64), 0, static_cast<hipStream_t>(stream), k_pool, v_pool, k_new,
                       v_new, block_table, ctx_len, cu_new, B, nkvh, max_pages, num_blocks, err);
    HIP_CHECK(hipGetLastError());
}

void pagedGather(uint16_t *k_out, uint16_t *v_out, const uint16_t *k_pool, const uint16_t *v_pool,
                 const int32_t *block_table, const int32_t *cu_seqlens, int T, int B, int nkvh, int max_pages,
                 int num_blocks, int *err, void *stream) {
    if (B == 0 || max_pages == 0) return;
    // One block per possible page; blocks past a sequence's length exit at once.
    hipLaunchKernelGGL(gatherKernel, dim3(max_pages, B, nkvh), dim3(256), 0, static_cast<hipStream_t>(stream), k_out,
                       v_out, k_pool, v_pool, block_table, cu_seqlens, T, nkvh, max_pages, num_blocks, err);
    HIP_CHECK(hipGetLastError());
}

void pagedAppendGather(uint16_t *k_out, uint16_t *v_out, uint16_t *k_pool, uint16_t *v_pool, const uint16_t *k_new,
                       const uint16_t *v_new, const int32_t *block_table, const int32_t *ctx_len,
                       const int32_t *cu_seqlens, int T, int B, int nkvh, int max_pages, int num_blocks, int *err,
                       void *stream) {
    if (B == 0 || max_pages == 0) return;
    hipLaunchKernelGGL(appendGatherKernel, dim3(max_pages, B, nkvh), dim3(256), 0, static_cast<hipStream_t>(stream),
                       k_out, v_out, k_pool, v_pool, k_new, v_new, block_table, ctx_len, cu_seqlens, T, nkvh,
                       max_pages, num_blocks, err);
    HIP_CHECK(hipGetLastError());
}

} // namespace llaisys::kernels
