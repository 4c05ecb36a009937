// Greedy tree acceptance on the device, for gfx950: the per-row argmax of the target
// logits and the per-request walk down the draft tree (serving_ops.py:55-90).
//
// argmax_rows_kernel: one 256-thread workgroup per logits row, 16-byte loads, each
// thread scanning its elements in increasing index order, then a wave and a workgroup
// reduction.  The order is torch.argmax's (ATen's GreaterOrNan): a NaN beats every
// number, and between equal values (or two NaNs) the lower index wins.  The kernel is
// HBM-bound: rows x vocab x element bytes, read once.
//
// tree_accept_kernel: one wave per request.  From the root, the next node is the child
// of the current node whose token equals the current node's argmax; among duplicate
// sibling tokens the last child wins (the child_maps rule, serving_ops.py:58-59).  The
// walk stops at a miss or after max_depth + 1 nodes, and every node on the path must
// sit at the depth equal to its path index (serving_ops.py:84-85), else the request is
// flagged.  The 64 lanes scan the request's nodes for the matching child in parallel.
#include <math.h>
#include <stdint.h>

#include "tv_internal.h"

namespace tv {
namespace {

constexpr int kArgmaxThreads = 256;

// a beats b under torch's ordering (GreaterOrNan).
__device__ __forceinline__ bool beats(float a, int64_t ia, float b, int64_t ib) {
    const bool na = a != a, nb = b != b;
    if (na) return nb ? ia < ib : true;
    if (nb) return false;
    return a == b ? ia < ib : a > b;
}

__device__ __forceinline__ float elem_value(const uint16_t* p, int64_t i) {
    return __uint_as_float(static_cast<uint32_t>(p[i]) << 16);
}
__device__ __forceinline__ float elem_value(const float* p, int64_t i) { return p[i]; }

// Unit: 8 bf16 or 4 fp32 per 16-byte load (Vec > 1), or one element.  Each thread
// visits its elements in increasing index order, so within a thread a later element
// replaces the best one only if it is larger, or a NaN replacing a number: equal
// values and later NaNs keep the earlier index.  Four loads are issued per iteration
// so that each wave keeps several in flight.  The logits are read once, so the vector
// loads are non-temporal (0.210 -> 0.185 ms for 4096 x 151936 bf16 rows, 5.9 -> 6.7 TB/s).
//
// The vector scan tracks units, not elements: per unit only its maximum and whether it
// holds a NaN, and a unit replaces the thread's best unit when its maximum is larger,
// or when it holds a NaN and the best unit does not (the first such unit, since a later
// unit must beat it strictly).  The best unit's raw bits are kept, and at the end its
// elements are visited in order, which gives the first element of the thread's largest
// value (or its first NaN): the element an element-by-element scan keeps, with about a
// third of its VALU work per element (0.225 -> 0.210 ms on the same rows).
template <typename S, int VEC>
__global__ void __launch_bounds__(kArgmaxThreads)
argmax_rows_kernel(const S* __restrict__ logits, int64_t row_stride, int64_t vocab, int64_t* __restrict__ out) {
    constexpr int kUnroll = 4;
    const int64_t row = blockIdx.x;
    const S* base = logits + row * row_stride;
    float best = -INFINITY;
    int64_t best_i = INT64_MAX;
    bool any = false;
    auto visit = [&](float v, int64_t i) {
        const bool take = !any || v > best || (v != v && best == best);
        best = take ? v : best;
        best_i = take ? i : best_i;
        any = true;
    };
    // Full vector units first (VEC elements each), then the scalar tail.
    const int64_t units = VEC > 1 ? vocab / VEC : 0;
    if constexpr (VEC > 1) {
        static_assert(VEC * sizeof(S) == sizeof(u32x4), "a vector unit is one 16-byte load");
        float unit_max = -INFINITY;   // the best unit's maximum (NaN once a unit holding a NaN is taken)
        int64_t unit = -1;            // the best unit
        u32x4 unit_raw = {0u, 0u, 0u, 0u};
        for (int64_t u0 = threadIdx.x; u0 < units; u0 += kUnroll * kArgmaxThreads) {
            u32x4 raw[kUnroll];
#pragma unroll
            for (int k = 0; k < kUnroll; ++k) {
                const int64_t u = u0 + k * kArgmaxThreads;
                if (u < units) raw[k] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(base + u * VEC));
            }
#pragma unroll
            for (int k = 0; k < kUnroll; ++k) {
                const int64_t u = u0 + k * kArgmaxThreads;
                if (u < units) {
                    S vals[VEC];
                    __builtin_memcpy(vals, &raw[k], sizeof(vals));
                    // NaN-propagating maximum (v_maximum3_f32): NaN when the unit holds one.
                    // Its -0 < +0 order is harmless: the maximum is only compared with > and ==.
                    float m = elem_value(vals, 0);
#pragma unroll
                    for (int e = 1; e < VEC; ++e) m = __builtin_elementwise_maximum(m, elem_value(vals, e));
                    const bool take = unit < 0 || m > unit_max || (m != m && unit_max == unit_max);
                    unit_max = take ? m : unit_max;
                    unit = take ? u : unit;
                    unit_raw = take ? raw[k] : unit_raw;
                }
            }
        }
        if (unit >= 0) {
            S vals[VEC];
            __builtin_memcpy(vals, &unit_raw, sizeof(vals));
#pragma unroll
            for (int e = 0; e < VEC; ++e) visit(elem_value(vals, e), unit * VEC + e);
        }
    }
    for (int64_t i = units * VEC + threadIdx.x; i < vocab; i += kArgmaxThreads) visit(elem_value(base, i), i);
    // Wave reduction (64 lanes), then across the 4 waves through LDS.
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
        const float ov = __shfl_xor(best, off);
        const int64_t oi = __shfl_xor(best_i, off);
        const bool oany = __shfl_xor(static_cast<int>(any), off) != 0;
        if (oany && (!any || beats(ov, oi, best, best_i))) {
            best = ov;
            best_i = oi;
            any = true;
        }
    }
    __shared__ float wave_best[kArgmaxThreads / 64];
    __shared__ int64_t wave_idx[kArgmaxThreads / 64];
    __shared__ int wave_any[kArgmaxThreads / 64];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    if (lane == 0) {
        wave_best[wave] = best;
        wave_idx[wave] = best_i;
        wave_any[wave] = any;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        float b = wave_best[0];
        int64_t bi = wave_idx[0];
        bool ba = wave_any[0] != 0;
        for (int w = 1; w < kArgmaxThreads / 64; ++w) {
            if (wave_any[w] && (!ba || beats(wave_best[w], wave_idx[w], b, bi))) {
                b = wave_best[w];
                bi = wave_idx[w];
                ba = true;
            }
        }
        out[row] = ba ? bi : 0;
    }
}

template <typename I>
__device__ __forceinline__ int64_t load_index(const void* p, int64_t i) {
    return static_cast<int64_t>(static_cast<const I*>(p)[i]);
}

__device__ __forceinline__ int64_t load_int(const void* p, int is64, int64_t i) {
    return is64 ? load_index<int64_t>(p, i) : load_index<int32_t>(p, i);
}

struct AcceptParams {
    const int64_t* greedy;     // [Q] argmax per packed row
    const void* tokens;        // [Q] draft token of each node
    const void* parents;       // [Q] request-local parent (-1 at the root)
    const void* depths;        // [Q] depth of each node
    int32_t tokens64, parents64, depths64;
    const int32_t* cu;         // [R + 1] packed row offsets
    int32_t num_requests, max_depth;
    int32_t* paths;            // [R, max_depth + 1] root-inclusive path, -1 padded
    int32_t* lengths;          // [R] accepted draft length = path nodes - 1
    int64_t* corrections;      // [R] greedy token at the last path node
    int32_t* status;
};

__global__ void __launch_bounds__(64)
tree_accept_kernel(const AcceptParams p) {
    const int r = blockIdx.x;
    const int lane = threadIdx.x;
    const int lo = p.cu[r], hi = p.cu[r + 1];
    const int n = hi - lo;
    const int width = p.max_depth + 1;
    int32_t* path = p.paths + static_cast<int64_t>(r) * width;
    for (int i = lane; i < width; i += 64) path[i] = -1;
    if (n < 1) {
        if (lane == 0) {
            set_status(p.status, TV_STATUS_BAD_REQUEST);
            p.lengths[r] = -1;
            p.corrections[r] = -1;
        }
        return;
    }
    int node = 0, count = 1;
    bool depth_ok = load_int(p.depths, p.depths64, lo) == 0;
    if (lane == 0) path[0] = 0;
    while (count <= p.max_depth) {
        const int64_t want = p.greedy[lo + node];
        int found = -1;
        for (int m = 1 + lane; m < n; m += 64) {
            if (load_int(p.parents, p.parents64, lo + m) == node && load_int(p.tokens, p.tokens64, lo + m) == want) {
                found = m;   // increasing m per lane: the lane keeps its last match
            }
        }
#pragma unroll
        for (int off = 32; off > 0; off >>= 1) found = max(found, __shfl_xor(found, off));
        if (found < 0) break;
        node = found;
        if (lane == 0) path[count] = node;
        depth_ok = depth_ok && load_int(p.depths, p.depths64, lo + node) == count;
        ++count;
    }
    if (lane == 0) {
        p.lengths[r] = count - 1;
        p.corrections[r] = p.greedy[lo + node];
        if (!depth_ok) set_status(p.status, TV_STATUS_BAD_DEPTH);
    }
}

}  // namespace
}  // namespace tv

using namespace tv;

extern "C" int tv_argmax_rows(const void* logits, int64_t rows, int64_t vocab, int64_t row_stride, int32_t dtype,
                              int64_t* out, void* stream) {
    clear_error();
    if (rows < 0 || vocab < 1 || row_stride < vocab) return fail(TV_ERR_INVALID, "argmax_rows: invalid sizes");
    if (dtype != TV_BF16 && dtype != TV_F32) return fail(TV_ERR_UNSUPPORTED, "argmax_rows: logits must be bf16 or fp32");
    if (rows == 0) return TV_OK;
    if (rows > 0x7fffffff) return fail(TV_ERR_UNSUPPORTED, "argmax_rows: too many rows");
    if (!logits || !out) return fail(TV_ERR_INVALID, "argmax_rows: null pointer");
    const int64_t elem = dtype == TV_F32 ? 4 : 2;
    const bool vec = aligned(logits, 16) && (row_stride * elem) % 16 == 0;
    hipStream_t s = as_stream(stream);
    if (dtype == TV_BF16) {
        if (vec) {
            hipLaunchKernelGGL((argmax_rows_kernel<uint16_t, 8>), dim3(rows), dim3(kArgmaxThreads), 0, s,
                               static_cast<const uint16_t*>(logits), row_stride, vocab, out);
        } else {
            hipLaunchKernelGGL((argmax_rows_kernel<uint16_t, 1>), dim3(rows), dim3(kArgmaxThreads), 0, s,
                               static_cast<const uint16_t*>(logits), row_stride, vocab, out);
        }
    } else {
        if (vec) {
            hipLaunchKernelGGL((argmax_rows_kernel<float, 4>), dim3(rows), dim3(kArgmaxThreads), 0, s,
                               static_cast<const float*>(logits), row_stride, vocab, out);
        } else {
            hipLaunchKernelGGL((argmax_rows_kernel<float, 1>), dim3(rows), dim3(kArgmaxThreads), 0, s,
                               static_cast<const float*>(logits), row_stride, vocab, out);
        }
    }
    return check_launch("argmax_rows");
}

extern "C" int tv_tree_accept(const int64_t* greedy, const void* token_ids, int32_t tokens_is_int64,
                              const void* parents, int32_t parents_is_int64, const void* depths,
                              int32_t depths_is_int64, const int32_t* cu_seqlens, int32_t num_requests,
                              int32_t max_depth, int32_t* paths, int32_t* lengths, int64_t* corrections,
                              int32_t* status, void* stream) {
    clear_error();
    if (num_requests < 0 || max_depth < 0 || max_depth > 4096) {
        return fail(TV_ERR_INVALID, "tree_accept: invalid request count or max_depth");
    }
    if (num_requests == 0) return TV_OK;
    if (!greedy || !token_ids || !parents || !depths || !cu_seqlens || !paths || !lengths || !corrections) {
        return fail(TV_ERR_INVALID, "tree_accept: null pointer");
    }
    AcceptParams p;
    p.greedy = greedy;
    p.tokens = token_ids;
    p.parents = parents;
    p.depths = depths;
    p.tokens64 = tokens_is_int64 != 0;
    p.parents64 = parents_is_int64 != 0;
    p.depths64 = depths_is_int64 != 0;
    p.cu = cu_seqlens;
    p.num_requests = num_requests;
    p.max_depth = max_depth;
    p.paths = paths;
    p.lengths = lengths;
    p.corrections = corrections;
    p.status = status;
    hipLaunchKernelGGL(tree_accept_kernel, dim3(num_requests), dim3(64), 0, as_stream(stream), p);
    return check_launch("tree_accept");
}

// ------------------------------------------------------------ accepted-path truncation
// batch_runtime.py:636-655 cuts each request's accepted outputs before it commits them:
// values = tokens along the path after the root, then the correction; limit =
// min(len(values), max_new_tokens - len(output_ids)); unless ignore_eos, the first EOS
// among values[:limit] ends them (limit = its index + 1); the request emits
// values[:limit] and caches path[:limit], which leaves its last emitted token uncached.
// One workgroup walks the batch in chunks of kTruncThreads requests, one thread per
// request, and a block scan of the limits lays the cut paths out back to back (the
// packed form tv_commit_slots takes).
namespace tv {
namespace {
constexpr int kTruncThreads = 1024;

__global__ void __launch_bounds__(kTruncThreads)
truncate_accepted_kernel(const int32_t* __restrict__ paths, int32_t stride, const int32_t* __restrict__ lengths,
                         const int64_t* __restrict__ corrections, const void* __restrict__ tokens, int tokens64,
                         const int32_t* __restrict__ cu, int32_t num_requests, const int32_t* __restrict__ budgets,
                         const uint8_t* __restrict__ ignore_eos, const int64_t* __restrict__ eos, int32_t num_eos,
                         int32_t* __restrict__ limits, int64_t* __restrict__ emitted,
                         int32_t* __restrict__ commit_paths, int32_t* __restrict__ commit_offsets, int32_t* status) {
    __shared__ int32_t scan[kTruncThreads];
    __shared__ int32_t carry;
    const int t = threadIdx.x;
    if (t == 0) carry = 0;
    __syncthreads();
    for (int32_t base = 0; base < num_requests; base += kTruncThreads) {
        const int32_t r = base + t;
        int32_t limit = 0;
        if (r < num_requests) {
            const int32_t len = lengths[r];
            const int32_t q0 = cu[r], nodes = cu[r + 1] - q0;
            const int32_t* path = paths + static_cast<int64_t>(r) * stride;
            bool ok = len >= 0 && len < stride && budgets[r] >= 1 && nodes >= 1;
            for (int32_t j = 0; ok && j <= len; ++j) ok = path[j] >= 0 && path[j] < nodes;
            auto value = [&](int32_t j) -> int64_t {
                if (j == len) return corrections[r];
                const int64_t row = q0 + path[j + 1];
                return tokens64 ? static_cast<const int64_t*>(tokens)[row]
                                : static_cast<int64_t>(static_cast<const int32_t*>(tokens)[row]);
            };
            if (!ok) {
                set_status(status, TV_STATUS_BAD_REQUEST);
            } else {
                limit = min(len + 1, budgets[r]);
                if (!ignore_eos[r]) {
                    for (int32_t j = 0; j < limit; ++j) {
                        const int64_t v = value(j);
                        bool hit = false;
                        for (int32_t e = 0; e < num_eos; ++e) hit = hit || v == eos[e];
                        if (hit) {
                            limit = j + 1;
                            break;
                        }
                    }
                }
            }
            limits[r] = limit;
            for (int32_t j = 0; j < stride; ++j) emitted[static_cast<int64_t>(r) * stride + j] = j < limit ? value(j) : -1;
        }
        scan[t] = limit;
        __syncthreads();
        for (int off = 1; off < kTruncThreads; off <<= 1) {
            const int32_t add = t >= off ? scan[t - off] : 0;
            __syncthreads();
            scan[t] += add;
            __syncthreads();
        }
        const int32_t start = carry + scan[t] - limit;
        if (r < num_requests) {
            commit_offsets[r] = start;
            const int32_t* path = paths + static_cast<int64_t>(r) * stride;
            for (int32_t j = 0; j < limit; ++j) commit_paths[start + j] = path[j];
        }
        __syncthreads();
        if (t == kTruncThreads - 1) carry += scan[t];
        __syncthreads();
    }
    if (t == 0) commit_offsets[num_requests] = carry;
}
}  // namespace
}  // namespace tv

extern "C" int tv_truncate_accepted(const int32_t* paths, int32_t path_stride, const int32_t* lengths,
                                    const int64_t* corrections, const void* token_ids, int32_t tokens_is_int64,
                                    const int32_t* cu_seqlens, int32_t num_requests, const int32_t* budgets,
                                    const uint8_t* ignore_eos, const int64_t* eos_token_ids, int32_t num_eos,
                                    int32_t* limits, int64_t* emitted, int32_t* commit_paths,
                                    int32_t* commit_offsets, int32_t* status, void* stream) {
    using namespace tv;
    clear_error();
    if (num_requests < 0 || path_stride < 1 || num_eos < 0) {
        return fail(TV_ERR_INVALID, "truncate_accepted: invalid request count, path stride or EOS count");
    }
    if (num_requests == 0) return TV_OK;
    if (static_cast<int64_t>(num_requests) * path_stride > 0x7fffffff) {
        return fail(TV_ERR_UNSUPPORTED, "truncate_accepted: too many path entries");
    }
    if (!paths || !lengths || !corrections || !token_ids || !cu_seqlens || !budgets || !ignore_eos || !limits ||
        !emitted || !commit_paths || !commit_offsets || (num_eos > 0 && !eos_token_ids)) {
        return fail(TV_ERR_INVALID, "truncate_accepted: null pointer");
    }
    hipLaunchKernelGGL(truncate_accepted_kernel, dim3(1), dim3(kTruncThreads), 0, as_stream(stream), paths,
                       path_stride, lengths, corrections, token_ids, tokens_is_int64 != 0 ? 1 : 0, cu_seqlens,
                       num_requests, budgets, ignore_eos, eos_token_ids, num_eos, limits, emitted, commit_paths,
                       commit_offsets, status);
    return check_launch("truncate_accepted");
}
