// Device-side tree metadata for gfx950: per-node ancestor bitmasks built from the
// parent arrays, and the reference's additive f32 bias derived from them.
//
// The reference ships a request-local f32 matrix qq_bias[T x T] (0 = ancestor or self,
// -inf = hidden) from the host every round (packed_metadata.py:93-100,185-195): T^2
// floats per request, 1 MiB for a 512-node chunk.  Here the host uploads the parent
// array (4 bytes per node) and the device derives:
//   ancestor_words_kernel   words[q * W + w] bit b = node 64w + b is q's ancestor or q
//   bias_from_words_kernel  qq_bias in the reference's layout, for callers that read it
//
// ancestor_words_kernel: one workgroup per request, pointer doubling in LDS.  With
// M(i) the mask of node i and J(i) an ancestor of i, start from M(i) = {i},
// J(i) = parent(i); each round sets M(i) |= M(J(i)) and then J(i) = J(J(i)).  After
// round r, M(i) holds every ancestor closer than 2^(r+1) and J(i) is the ancestor at
// distance 2^(r+1), so ceil(log2(T)) rounds cover any depth (a 512-node causal chunk
// takes 9 rounds, not 511).  Masks only gain bits, and every bit OR-ed in is an
// ancestor of an ancestor, so reading a mask that another lane is updating in the same
// round (old or new bits, even a torn 64-bit read) can only add true ancestors early;
// the jump pointers are double-buffered so each round moves them exactly 2^r further.
#include <stdint.h>

#include "tv_internal.h"

namespace tv {
namespace {

constexpr int kMetaThreads = 256;

__global__ void __launch_bounds__(kMetaThreads)
ancestor_words_kernel(const int32_t* __restrict__ parents, const int32_t* __restrict__ cu, int32_t words_per_row,
                      int32_t max_nodes, uint64_t* __restrict__ words, int32_t* status) {
    extern __shared__ __attribute__((aligned(16))) char smem[];
    const int r = blockIdx.x;
    const int lo = cu[r], n = cu[r + 1] - lo;
    const int W = words_per_row;
    if (n < 1 || n > max_nodes || n > 64 * W) {
        if (threadIdx.x == 0) set_status(status, TV_STATUS_BAD_REQUEST);
        return;
    }
    uint64_t* mask = reinterpret_cast<uint64_t*>(smem);
    int32_t* jump = reinterpret_cast<int32_t*>(smem + static_cast<size_t>(max_nodes) * W * 8);
    int32_t* jump_next = jump + max_nodes;
    for (int e = threadIdx.x; e < n * W; e += kMetaThreads) {
        const int i = e / W, w = e - i * W;
        mask[e] = (i >> 6) == w ? (1ull << (i & 63)) : 0ull;
    }
    bool bad = false;
    for (int i = threadIdx.x; i < n; i += kMetaThreads) {
        int p = parents[lo + i];
        // Parents precede their children and the root has none; anything else is
        // reported and treated as a root so the walk below stays inside the request.
        if ((i == 0 && p != -1) || (i > 0 && (p < 0 || p >= i))) {
            bad = true;
            p = -1;
        }
        jump[i] = p;
    }
    if (bad) set_status(status, TV_STATUS_BAD_REQUEST);
    __syncthreads();
    for (int span = 1; span < n; span <<= 1) {
        for (int e = threadIdx.x; e < n * W; e += kMetaThreads) {
            const int i = e / W, w = e - i * W;
            const int j = jump[i];
            if (j >= 0) mask[e] |= mask[j * W + w];
        }
        __syncthreads();
        for (int i = threadIdx.x; i < n; i += kMetaThreads) {
            const int j = jump[i];
            jump_next[i] = j >= 0 ? jump[j] : -1;
        }
        __syncthreads();
        int32_t* t = jump;
        jump = jump_next;
        jump_next = t;
    }
    for (int e = threadIdx.x; e < n * W; e += kMetaThreads) {
        words[static_cast<int64_t>(lo) * W + e] = mask[e];
    }
}

// One workgroup per packed row q (request r, local row i): writes the row's n floats of
// the reference bias, 0 where node m is visible to i and -inf elsewhere.
__global__ void __launch_bounds__(kMetaThreads)
bias_from_words_kernel(const uint64_t* __restrict__ words, int32_t words_per_row, const int32_t* __restrict__ q2r,
                       const int32_t* __restrict__ local, const int32_t* __restrict__ counts,
                       const int64_t* __restrict__ bias_off, float* __restrict__ bias) {
    const int64_t q = blockIdx.x;
    const int r = q2r[q], i = local[q], n = counts[r];
    const uint64_t* row = words + q * words_per_row;
    float* out = bias + bias_off[r] + static_cast<int64_t>(i) * n;
    for (int m = threadIdx.x; m < n; m += kMetaThreads) {
        out[m] = (row[m >> 6] >> (m & 63)) & 1ull ? 0.0f : -INFINITY;
    }
}

}  // namespace
}  // namespace tv

using namespace tv;

extern "C" int tv_ancestor_words_from_parents(const int32_t* parents, const int32_t* cu_seqlens,
                                              int32_t num_requests, int32_t max_nodes, int32_t words_per_row,
                                              uint64_t* words, int32_t* status, void* stream) {
    clear_error();
    if (num_requests < 0 || max_nodes < 1 || max_nodes > 1024 || words_per_row < (max_nodes + 63) / 64 ||
        words_per_row > 16) {
        return fail(TV_ERR_INVALID, "ancestor_words_from_parents: invalid sizes (max_nodes %d, words_per_row %d)",
                    max_nodes, words_per_row);
    }
    if (num_requests == 0) return TV_OK;
    if (!parents || !cu_seqlens || !words) return fail(TV_ERR_INVALID, "ancestor_words_from_parents: null pointer");
    const size_t lds = static_cast<size_t>(max_nodes) * words_per_row * 8 + 2 * static_cast<size_t>(max_nodes) * 4;
    if (lds > 64 * 1024) {
        // 1024 nodes need 136 KiB of gfx950's 160 KiB; allow more than the default 64 KiB.
        const hipError_t err = hipFuncSetAttribute(reinterpret_cast<const void*>(&ancestor_words_kernel),
                                                   hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(lds));
        if (err != hipSuccess) {
            return fail(TV_ERR_LAUNCH, "ancestor_words_from_parents: %s", hipGetErrorString(err));
        }
    }
    hipLaunchKernelGGL(ancestor_words_kernel, dim3(num_requests), dim3(kMetaThreads), lds, as_stream(stream), parents,
                       cu_seqlens, words_per_row, max_nodes, words, status);
    return check_launch("ancestor_words_from_parents");
}

extern "C" int tv_bias_from_ancestor_words(const uint64_t* words, int32_t words_per_row,
                                           const int32_t* query_to_request, const int32_t* query_local_row,
                                           const int32_t* node_counts, const int64_t* qq_bias_offsets,
                                           int32_t total_queries, float* qq_bias, void* stream) {
    clear_error();
    if (total_queries < 0 || words_per_row < 1) return fail(TV_ERR_INVALID, "bias_from_ancestor_words: invalid sizes");
    if (total_queries == 0) return TV_OK;
    if (!words || !query_to_request || !query_local_row || !node_counts || !qq_bias_offsets || !qq_bias) {
        return fail(TV_ERR_INVALID, "bias_from_ancestor_words: null pointer");
    }
    hipLaunchKernelGGL(bias_from_words_kernel, dim3(total_queries), dim3(kMetaThreads), 0, as_stream(stream), words,
                       words_per_row, query_to_request, query_local_row, node_counts, qq_bias_offsets, qq_bias);
    return check_launch("bias_from_ancestor_words");
}
