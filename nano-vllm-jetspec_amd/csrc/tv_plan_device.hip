// Device-side work planner for the packed tree-verify attention, for gfx950.
//
// Produces the same items and merge groups as the host planner (tv_plan.cpp), item for
// item, but from the prefix lengths and node counts in device memory.  A launch sequence
// that reads its plan from the device keeps fixed grid sizes while the prefix lengths
// change, which is what a captured HIP graph replays: the attention and merge kernels
// are launched with a capacity grid and their surplus workgroups exit on the counts
// this planner writes.
//
// One 1024-thread workgroup:
//   1. per request: KV heads per group, node blocks, cost; the total cost (reduction);
//   2. per request: prefix chunk length and count (the host formulas), item / group /
//      slot counts, and their exclusive prefix sums (one scan);
//   3. every item gets a 64-bit sort key = (~cost, request, head group, chunk, block),
//      the host's comparator; a bitonic sort in LDS orders them longest first;
//   4. the XCD placement of the host (64-item windows, multi-block groups first,
//      column-major), then the items and groups are written out.
// Capacity overflow writes zero counts and an error flag instead of writing past the
// caller's arrays.
#include <math.h>
#include <stdint.h>

#include <algorithm>

#include "tv_internal.h"

namespace tv {
namespace {

constexpr int kPlanThreads = 1024;
constexpr int kMaxSortItems = 8192;      // LDS sort capacity (64 KiB of keys)
constexpr int kMaxPlanRequests = 2048;
constexpr int kMaxPlanNodes = 2048;     // tree nodes of one request (the attention kernel's page-mode cache)
constexpr int kMinChunkKeys = 64;
constexpr int kMaxChunkPages = 512;
constexpr int kXcds = 8;
constexpr int64_t kFillRounds = 4;

struct PlanArgs {
    const int32_t* prefix_lens;
    const int32_t* node_counts;
    int32_t num_requests, num_kv_heads, qpk, block_size, compute_units, chunk_keys;
    int32_t item_capacity, group_capacity, slot_capacity;
    int32_t* items;      // [item_capacity, 8]
    int32_t* groups;     // [group_capacity, 8]
    int32_t* counts;     // [4]: items, groups, partial slots, error
};

// Nodes of one KV head per work item and the two-head rule of the host planner (tv_plan.cpp).
__host__ __device__ __forceinline__ int nodes_per_item(int hpw, int qpk) { return (8 / hpw) * (32 / qpk); }

__device__ __forceinline__ int heads_per_group(int nodes, int kv_heads, int qpk) {
    int h = nodes <= nodes_per_item(2, qpk) ? 2 : 1;
    while (h > 1 && h > kv_heads) h >>= 1;
    return h;
}

__device__ __forceinline__ int64_t round_up(int64_t x, int64_t m) { return (x + m - 1) / m * m; }

// Cost of one key of a work item in quarter key-steps of a one-head item: a two-head
// tile costs ~1.25x a one-head tile (each wave still runs one head's MFMAs).  The host
// planner uses the same weights.
__device__ __forceinline__ int64_t cost_weight(int hpw) { return hpw == 2 ? 5 : 4; }

constexpr int kPlanWaves = kPlanThreads / 64;
constexpr int kProbeWaves = 4;   // waves that probe chunk targets in the refit (one per SIMD)

// Block-wide exclusive scan of three int64 values per thread (kPlanThreads threads): each
// thread's prefixes of v[0..2] are returned in v, the totals written to total[0..2].  A scan
// within each wave (lane shuffles), then the wave totals through LDS: two barriers.
__device__ void block_scan3(int64_t (&v)[3], int64_t* scratch, int64_t* total) {
    const int t = threadIdx.x, lane = t & 63, w = t >> 6;
    int64_t x[3] = {v[0], v[1], v[2]};
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
#pragma unroll
        for (int j = 0; j < 3; ++j) {
            const int64_t y = __shfl_up(x[j], off);
            if (lane >= off) x[j] += y;
        }
    }
    if (lane == 63) {
#pragma unroll
        for (int j = 0; j < 3; ++j) scratch[3 * w + j] = x[j];
    }
    __syncthreads();
#pragma unroll
    for (int j = 0; j < 3; ++j) {
        int64_t before = 0, all = 0;
#pragma unroll
        for (int k = 0; k < kPlanWaves; ++k) {
            const int64_t s = scratch[3 * k + j];
            before += k < w ? s : 0;
            all += s;
        }
        if (t == 0) total[j] = all;
        v[j] = before + x[j] - v[j];
    }
    __syncthreads();   // the totals are visible, and every thread has read `scratch`
}

// Sum over one wave (returned to every lane).
__device__ __forceinline__ int64_t wave_sum(int64_t v) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off);
    return v;
}

// Block-wide sum of one int64 per thread (kPlanThreads threads), returned to all.
__device__ int64_t block_sum(int64_t v, int64_t* scratch) {
    v = wave_sum(v);
    const int t = threadIdx.x;
    __syncthreads();
    if ((t & 63) == 0) scratch[t >> 6] = v;
    __syncthreads();
    int64_t total = 0;
#pragma unroll
    for (int w = 0; w < kPlanWaves; ++w) total += scratch[w];
    __syncthreads();   // every thread has read `scratch` before anyone reuses it
    return total;
}

// One request's geometry from its (clamped) node count: KV heads per item, nodes per item,
// head groups and node blocks (heads_per_group and nodes_per_item with nw = 32 / qpk nodes
// per wave taken once per thread, so only the node-block count divides).
struct ReqShape {
    int hpw, npw, G, NB;
};
__device__ __forceinline__ ReqShape req_shape(int n, int kv_heads, int nw) {
    ReqShape s;
    s.hpw = (n <= 4 * nw && kv_heads >= 2) ? 2 : 1;
    s.npw = (8 / s.hpw) * nw;
    s.G = s.hpw == 2 ? (kv_heads + 1) >> 1 : kv_heads;
    s.NB = (n + s.npw - 1) / s.npw;
    return s;
}

// The host planner's chunk length (tv_plan.cpp, chunk_for) for a prefix of p keys, with
// q = tau / cost_weight(hpw) precomputed: min(round_up(max(64, q), 32), max_chunk), then
// equalised over the chunks.  Every quantity after the first min is below 2^32.
__device__ __forceinline__ uint32_t chunk_of(uint32_t p, int64_t q, int64_t max_chunk) {
    const int64_t c0 = min(round_up(max(static_cast<int64_t>(kMinChunkKeys), min(q, max_chunk)), 32), max_chunk);
    const uint32_t c = static_cast<uint32_t>(c0);
    const uint32_t nchunks = p > 0 ? (p + c - 1) / c : 1;
    const uint32_t chunk = ((p + nchunks - 1) / nchunks + 31) / 32 * 32;
    return chunk < 32 ? 32 : chunk;
}

// Plans in one 1024-thread workgroup.  The prefix lengths and node counts are read once into
// LDS; every later per-request quantity comes from there.
__global__ void __launch_bounds__(kPlanThreads)
plan_device_kernel(const PlanArgs a) {
    __shared__ uint64_t keys[kMaxSortItems];
    __shared__ int32_t stream_id[kMaxSortItems];   // (request, head group, chunk) of each sorted item
    __shared__ int32_t req_p[kMaxPlanRequests], req_n[kMaxPlanRequests];
    __shared__ int32_t req_chunk[kMaxPlanRequests], req_nchunks[kMaxPlanRequests];
    __shared__ int32_t req_item_off[kMaxPlanRequests], req_group_off[kMaxPlanRequests], req_slot_off[kMaxPlanRequests];
    __shared__ int64_t scan[3 * kPlanWaves];
    __shared__ int64_t totals[4];
    __shared__ int shared_flag;
    __shared__ int32_t probe_fits[kPlanWaves];
    __shared__ int64_t probe_val[kPlanWaves];
    const int t = threadIdx.x;
    const int R = a.num_requests;
    const int B = a.block_size;
    const int KV = a.num_kv_heads, QPK = a.qpk, NW = 32 / a.qpk;

    // 1. Prefix lengths and node counts into LDS (clamped; a value outside the planner's
    // range fails the plan), costs and their total.
    if (t == 0) shared_flag = 0;
    bool bad = false;
    int64_t my_cost = 0;
    for (int r = t; r < R; r += kPlanThreads) {
        const int p = a.prefix_lens[r], n = a.node_counts[r];
        bad |= p < 0 || n < 1 || n > kMaxPlanNodes;
        const int pc = max(0, p), nc = max(1, min(kMaxPlanNodes, n));
        req_p[r] = pc;
        req_n[r] = nc;
        const ReqShape s = req_shape(nc, KV, NW);
        my_cost += static_cast<int64_t>(s.G) * s.NB * cost_weight(s.hpw) * (static_cast<int64_t>(pc) + nc);
    }
    __syncthreads();   // shared_flag is cleared before anyone sets it
    if (bad) atomicOr(&shared_flag, 1);
    const int64_t total_cost = block_sum(my_cost, scan);   // its barriers also publish req_p / req_n
    const int64_t target = max(static_cast<int64_t>(kMinChunkKeys), total_cost / a.compute_units);
    const int64_t max_chunk = min((static_cast<int64_t>(kMaxChunkPages - 1) * B) / 32 * 32, int64_t{1} << 31);

    // 1b. The host's refit of the chunk target when the items leave the last of at most
    // kFillRounds rounds part-empty: the smallest target whose item count fits the same
    // rounds.  The count falls as the target grows, so any search finds the host's
    // bisection result; here one wave per SIMD probes one target per round (a 5-way
    // search, two barriers per round; more probing waves would share the SIMDs and make
    // every round as much longer).
    auto request_items = [&](int r, int64_t q4, int64_t q5) -> int64_t {
        const uint32_t p = static_cast<uint32_t>(req_p[r]);
        const ReqShape s = req_shape(req_n[r], KV, NW);
        const uint32_t chunk = chunk_of(p, s.hpw == 2 ? q5 : q4, max_chunk);
        return static_cast<int64_t>(s.G) * s.NB * (p > 0 ? (p + chunk - 1) / chunk : 1u);
    };
    int64_t tau = target;
    if (a.chunk_keys == 0) {
        int64_t now = 0;
        for (int r = t; r < R; r += kPlanThreads) now += request_items(r, target / 4, target / 5);
        now = block_sum(now, scan);
        const int64_t rounds = (now + a.compute_units - 1) / a.compute_units;
        if (now > a.compute_units && rounds <= kFillRounds) {
            const int64_t limit = rounds * a.compute_units;
            const int lane = t & 63, w = t >> 6;
            int64_t lo = 1, hi = target;   // items(hi) <= limit; the answer is in [lo, hi]
            while (lo < hi) {
                const int64_t span = hi - lo;
                if (w < kProbeWaves) {
                    const int64_t probe = lo + span * (w + 1) / (kProbeWaves + 1);   // in [lo, hi)
                    const int64_t q4 = probe / 4, q5 = probe / 5;
                    int64_t n = 0;
                    for (int r = lane; r < R; r += 64) n += request_items(r, q4, q5);
                    n = wave_sum(n);
                    if (lane == 0) {
                        probe_fits[w] = n <= limit ? 1 : 0;
                        probe_val[w] = probe;
                    }
                }
                __syncthreads();
                int64_t new_lo = lo, new_hi = hi;
#pragma unroll
                for (int k = 0; k < kProbeWaves; ++k) {
                    const int64_t pk = probe_val[k];
                    if (probe_fits[k]) new_hi = min(new_hi, pk); else new_lo = max(new_lo, pk + 1);
                }
                __syncthreads();   // every thread has read probe_fits
                lo = new_lo;
                hi = new_hi;
            }
            tau = lo;
        }
    }

    // 2. Chunking and per-request counts.  Requests are handled in contiguous runs per
    // thread so that one scan yields request-ordered offsets.
    const int per_thread = (R + kPlanThreads - 1) / kPlanThreads;
    const int r0 = min(R, t * per_thread), r1 = min(R, r0 + per_thread);
    int64_t mine[3] = {0, 0, 0};   // items, groups, slots
    {
        const int64_t q4 = tau / 4, q5 = tau / 5;
        for (int r = r0; r < r1; ++r) {
            const uint32_t p = static_cast<uint32_t>(req_p[r]);
            const ReqShape s = req_shape(req_n[r], KV, NW);
            const uint32_t chunk = a.chunk_keys > 0 ? static_cast<uint32_t>(a.chunk_keys)
                                                    : chunk_of(p, s.hpw == 2 ? q5 : q4, max_chunk);
            const uint32_t nchunks = p > 0 ? (p + chunk - 1) / chunk : 1u;
            req_chunk[r] = static_cast<int32_t>(chunk);
            req_nchunks[r] = static_cast<int32_t>(nchunks);
            const int64_t units = static_cast<int64_t>(s.G) * s.NB;
            mine[0] += units * nchunks;
            if (nchunks > 1) {
                mine[1] += units;
                mine[2] += units * nchunks;
            }
        }
    }
    int64_t base[3] = {mine[0], mine[1], mine[2]};
    block_scan3(base, scan, &totals[1]);
    for (int r = r0; r < r1; ++r) {
        const ReqShape s = req_shape(req_n[r], KV, NW);
        const int64_t units = static_cast<int64_t>(s.G) * s.NB, nc = req_nchunks[r];
        req_item_off[r] = static_cast<int32_t>(base[0]);
        req_group_off[r] = static_cast<int32_t>(base[1]);
        req_slot_off[r] = static_cast<int32_t>(base[2]);
        base[0] += units * nc;
        if (nc > 1) {
            base[1] += units;
            base[2] += units * nc;
        }
    }
    __syncthreads();
    const int64_t num_items = totals[1], num_groups = totals[2], num_slots = totals[3];
    const bool overflow = shared_flag || num_items > a.item_capacity || num_items > kMaxSortItems ||
                          num_groups > a.group_capacity || num_slots > a.slot_capacity || R > kMaxPlanRequests;
    if (overflow) {
        if (t == 0) {
            a.counts[0] = 0;
            a.counts[1] = 0;
            a.counts[2] = 0;
            a.counts[3] = 1;
        }
        return;
    }
    const int nitems = static_cast<int>(num_items);

    // The request of item enumeration index idx (the last request whose first item is at or
    // before it; every request has at least one item).
    auto request_of = [&](int idx) -> int {
        int lo = 0, hi = R - 1;
        while (lo < hi) {
            const int mid = (lo + hi + 1) >> 1;
            if (req_item_off[mid] <= idx) lo = mid; else hi = mid - 1;
        }
        return lo;
    };

    // 3. Sort keys, one thread per item: (~cost, request, head group, chunk, block), the
    // enumeration index idx = item offset + (hg * nchunks + c) * NB + nb being the tie order.
    int npow = 1;
    while (npow < nitems) npow <<= 1;
    for (int e = t; e < npow; e += kPlanThreads) {
        uint64_t key = ~0ull;
        if (e < nitems) {
            const int r = request_of(e);
            const ReqShape s = req_shape(req_n[r], KV, NW);
            const int nc = req_nchunks[r];
            const int local = e - req_item_off[r];
            const int c = (local / s.NB) % nc;
            const int64_t p = req_p[r], chunk = req_chunk[r];
            const int64_t kb = min(p, c * chunk), ke = min(p, (c + 1) * chunk);
            const int64_t cost = cost_weight(s.hpw) * ((ke - kb) + (c == nc - 1 ? req_n[r] : 0));
            key = (static_cast<uint64_t>(0x7fffffffu - static_cast<uint32_t>(cost)) << 32) | static_cast<uint32_t>(e);
        }
        keys[e] = key;
    }
    __syncthreads();
    // Bitonic sort of npow keys, longest first.  Thread t owns elements t + k * kPlanThreads;
    // a stride below 64 pairs two elements of one wave with the same k, so those stages run
    // on registers with lane shuffles (the keys are loaded once per run of such stages, and
    // waves that own no element skip them), and the stages of larger strides exchange
    // through LDS with a barrier each.  `in_regs` depends only on the loop position, so every
    // wave takes the same barriers.
    constexpr int kPer = kMaxSortItems / kPlanThreads;
    const bool owns = t - (t & 63) < npow;   // wave-uniform
    uint64_t x[kPer];
    bool in_regs = false;
    for (int size = 2; size <= npow; size <<= 1) {
        for (int stride = size >> 1; stride > 0; stride >>= 1) {
            if (stride >= 64) {
                if (in_regs) {
                    if (owns) {
#pragma unroll
                        for (int k = 0; k < kPer; ++k) {
                            const int e = t + k * kPlanThreads;
                            if (e < npow) keys[e] = x[k];
                        }
                    }
                    __syncthreads();
                    in_regs = false;
                }
                for (int e = t; e < npow; e += kPlanThreads) {
                    const int partner = e ^ stride;
                    if (partner > e) {
                        const bool ascending = (e & size) == 0;
                        const uint64_t u = keys[e], v = keys[partner];
                        if ((u > v) == ascending) {
                            keys[e] = v;
                            keys[partner] = u;
                        }
                    }
                }
                __syncthreads();
                continue;
            }
            if (!in_regs) {
                if (owns) {
#pragma unroll
                    for (int k = 0; k < kPer; ++k) {
                        const int e = t + k * kPlanThreads;
                        x[k] = e < npow ? keys[e] : ~0ull;
                    }
                }
                in_regs = true;
            }
            if (owns) {
                const bool lower = (t & stride) == 0;
#pragma unroll
                for (int k = 0; k < kPer; ++k) {
                    const int e = t + k * kPlanThreads;
                    if (k * kPlanThreads < npow) {   // wave-uniform: the wave's elements of row k exist
                        const uint32_t lo32 = __shfl_xor(static_cast<uint32_t>(x[k]), stride);
                        const uint32_t hi32 = __shfl_xor(static_cast<uint32_t>(x[k] >> 32), stride);
                        const uint64_t y = (static_cast<uint64_t>(hi32) << 32) | lo32;
                        const bool ascending = (e & size) == 0;
                        x[k] = (lower == ascending) ? min(x[k], y) : max(x[k], y);
                    }
                }
            }
        }
    }
    if (in_regs && owns) {
#pragma unroll
        for (int k = 0; k < kPer; ++k) {
            const int e = t + k * kPlanThreads;
            if (e < npow) keys[e] = x[k];
        }
    }
    __syncthreads();

    // Decode a sorted key back into its item.
    auto decode = [&](int sorted_pos, int32_t* out) {
        const int idx = static_cast<int>(keys[sorted_pos] & 0xffffffffull);
        const int r = request_of(idx);
        const ReqShape s = req_shape(req_n[r], KV, NW);
        const int nc = req_nchunks[r];
        const int local = idx - req_item_off[r];
        const int nb = local % s.NB;
        const int hc = local / s.NB;
        const int c = hc % nc;
        const int hg = hc / nc;
        const int64_t p = req_p[r], chunk = req_chunk[r];
        out[0] = r;
        out[1] = hg * s.hpw;
        out[2] = nb * s.npw;
        out[3] = static_cast<int32_t>(min(p, c * chunk));
        out[4] = static_cast<int32_t>(min(p, (c + 1) * chunk));
        out[5] = (c == nc - 1 ? kItemLastChunk : 0) | (nb == s.NB - 1 ? kItemLastBlock : 0) | (QPK << kItemGroupShift);
        out[6] = nc > 1 ? req_slot_off[r] + (hg * s.NB + nb) * nc + c : -1;
        out[7] = s.hpw;
    };

    // 4. XCD placement (tv_plan.cpp::place_for_xcds) and output.  Stream identity (request,
    // head group, chunk) of each sorted position.
    for (int i = t; i < nitems; i += kPlanThreads) {
        const int idx = static_cast<int>(keys[i] & 0xffffffffull);
        const int r = request_of(idx);
        const ReqShape s = req_shape(req_n[r], KV, NW);
        stream_id[i] = r * kMaxSortItems + (idx - req_item_off[r]) / s.NB;
    }
    if (t == 0) shared_flag = 0;
    __syncthreads();
    // Bit 0: some stream has several items; bit 1: some stream's item count (its
    // request's node blocks) is not a multiple of 8.
    for (int i = 1 + t; i < nitems; i += kPlanThreads) {
        if (stream_id[i] == stream_id[i - 1]) atomicOr(&shared_flag, 1);
    }
    for (int r = t; r < R; r += kPlanThreads) {
        const ReqShape s = req_shape(req_n[r], KV, NW);
        if (s.NB > 1 && s.NB % kXcds) atomicOr(&shared_flag, 2);
    }
    __syncthreads();
    const bool shared = (shared_flag & 1) != 0;
    const bool aligned = (shared_flag & 2) == 0;
    constexpr int kWindow = kXcds * kXcds;
    const int full = shared ? (nitems / kWindow) * kWindow : 0;
    auto position_of = [&](int rank) {
        if (rank >= full) return rank;
        const int w = rank - rank % kWindow;
        const int k = rank - w;
        const int column = (w / kWindow) % 2 ? kXcds - 1 - k / kXcds : k / kXcds;   // odd windows mirrored
        return w + kXcds * (k % kXcds) + column;
    };
    if (shared && aligned) {
        // Groups ahead of the at most 7 singles before them since the last multiple of
        // 8: ranks from the number of single items before each sorted position.
        const int i0 = t * kPer;
        uint32_t single_bits = 0;
        int64_t counted[3] = {0, 0, 0};
        for (int e = 0; e < kPer; ++e) {
            const int i = i0 + e;
            if (i >= nitems) break;
            const int32_t sid = stream_id[i];
            const bool single = !((i > 0 && stream_id[i - 1] == sid) || (i + 1 < nitems && stream_id[i + 1] == sid));
            single_bits |= static_cast<uint32_t>(single) << e;
            counted[0] += single;
        }
        block_scan3(counted, scan, &totals[0]);   // syncs: stream_id reads are done
        const int singles_total = static_cast<int>(totals[0]);
        int run = static_cast<int>(counted[0]);
        for (int e = 0; e < kPer; ++e) {
            const int i = i0 + e;
            if (i >= nitems) break;
            stream_id[i] = run;                 // now: singles before position i
            run += (single_bits >> e) & 1u;
        }
        __syncthreads();
        auto singles_before = [&](int q) -> int { return q < nitems ? stream_id[q] : singles_total; };
        // Ranks and output, one item per thread (position i is single iff the count steps there).
        for (int i = t; i < nitems; i += kPlanThreads) {
            const int sb = stream_id[i];
            int rank;
            if (singles_before(i + 1) == sb) {
                rank = (i - sb) + sb / kXcds * kXcds;
            } else {
                int lo = i + 1, hi = nitems;   // first q with floor8(singles before q) > sb
                while (lo < hi) {
                    const int mid = (lo + hi) >> 1;
                    if (singles_before(mid) / kXcds * kXcds > sb) hi = mid; else lo = mid + 1;
                }
                rank = sb + (lo - singles_before(lo));
            }
            decode(i, a.items + static_cast<int64_t>(position_of(rank)) * 8);
        }
    } else {
        for (int i = t; i < nitems; i += kPlanThreads) {
            int rank = i;
            if (i < full) {
                const int w = i - i % kWindow;
                const int k = i - w;
                // Rank of item k in the window's "grouped first" order.
                auto grouped = [&](int j) {
                    const int32_t s = stream_id[w + j];
                    return (j + 1 < kWindow && stream_id[w + j + 1] == s) || (j > 0 && stream_id[w + j - 1] == s);
                };
                const bool mine_grouped = grouped(k);
                int within = 0;
                for (int j = 0; j < kWindow; ++j) {
                    if (j == k) continue;
                    const bool g = grouped(j);
                    if (mine_grouped ? (g && j < k) : (g || j < k)) ++within;
                }
                rank = w + within;
            }
            decode(i, a.items + static_cast<int64_t>(position_of(rank)) * 8);
        }
    }
    // Merge groups in (request, head group, block) order with their first partial slot.
    for (int r = r0; r < r1; ++r) {
        const int nc = req_nchunks[r];
        if (nc < 2) continue;
        const ReqShape s = req_shape(req_n[r], KV, NW);
        for (int hg = 0; hg < s.G; ++hg) {
            for (int nb = 0; nb < s.NB; ++nb) {
                int32_t* gr = a.groups + static_cast<int64_t>(req_group_off[r] + hg * s.NB + nb) * 8;
                gr[0] = r;
                gr[1] = hg * s.hpw;
                gr[2] = nb * s.npw;
                gr[3] = s.hpw;
                gr[4] = req_slot_off[r] + (hg * s.NB + nb) * nc;
                gr[5] = nc;
                gr[6] = QPK;   // the grouping the slots' rows are laid out for
                gr[7] = 0;
            }
        }
    }
    if (t == 0) {
        a.counts[0] = static_cast<int32_t>(num_items);
        a.counts[1] = static_cast<int32_t>(num_groups);
        a.counts[2] = static_cast<int32_t>(num_slots);
        a.counts[3] = 0;
    }
}

}  // namespace
}  // namespace tv

using namespace tv;

namespace tv {
namespace {

// Capacities of a device-planned launch from the node-block total of the batch:
// items <= 2 * CUs + blocks * (1 + ceil(P_max / longest chunk)).  A chunk is at least
// total/CUs keys per unit of cost unless it is capped by the LDS page cache, and the
// round-filling refit keeps the item count within the rounds that count needed, so it
// adds at most CUs - 1 items.  A forced chunk length gives every node-block group
// ceil(P_max / chunk) items.
int fill_capacity(int64_t blocks, int32_t max_nodes, int32_t block_size, int32_t num_compute_units,
                  int32_t chunk_keys, int64_t max_prefix, tv_attention_plan_info* info) {
    const int64_t max_chunk = (static_cast<int64_t>(kMaxChunkPages - 1) * block_size) / 32 * 32;
    const int64_t capped = (max_prefix + max_chunk - 1) / max_chunk;
    const int64_t items = chunk_keys > 0 ? blocks * std::max<int64_t>(1, (max_prefix + chunk_keys - 1) / chunk_keys)
                                         : 2 * static_cast<int64_t>(num_compute_units) + blocks * (1 + capped);
    if (items > kMaxSortItems) {
        return fail(TV_ERR_UNSUPPORTED, "plan_capacity: %lld items exceed the device planner's %d",
                    static_cast<long long>(items), kMaxSortItems);
    }
    info->num_items = static_cast<int32_t>(items);
    info->num_groups = static_cast<int32_t>(blocks);
    info->num_partial_slots = static_cast<int32_t>(items);
    info->ancestor_words_per_row = (max_nodes + 63) / 64;
    info->workspace_bytes = (items * 256 * 128 * 4 + 255) / 256 * 256 + (items * 256 * 8 + 255) / 256 * 256;
    return TV_OK;
}

bool supported_group(int32_t qpk) { return (qpk >= 1 && qpk <= 8) || qpk == 16; }

bool capacity_args_ok(int32_t num_requests, int32_t num_kv_heads, int32_t qpk, int32_t block_size,
                      int32_t num_compute_units, int32_t chunk_keys, int64_t max_prefix) {
    return num_requests >= 1 && num_kv_heads >= 1 && supported_group(qpk) && block_size >= 32 &&
           block_size % 32 == 0 && num_compute_units >= 1 && max_prefix >= 0 && chunk_keys >= 0 && chunk_keys % 32 == 0;
}

}  // namespace
}  // namespace tv

extern "C" int tv_tree_attention_plan_capacity(const int32_t* node_counts_host, int32_t num_requests,
                                               int32_t num_kv_heads, int32_t queries_per_kv, int32_t block_size,
                                               int32_t num_compute_units, int32_t chunk_keys, int64_t max_prefix,
                                               tv_attention_plan_info* info) {
    clear_error();
    const int32_t qpk = queries_per_kv;
    if (!node_counts_host || !info ||
        !capacity_args_ok(num_requests, num_kv_heads, qpk, block_size, num_compute_units, chunk_keys, max_prefix)) {
        return fail(TV_ERR_INVALID, "plan_capacity: invalid arguments");
    }
    if (num_requests > kMaxPlanRequests) {
        return fail(TV_ERR_UNSUPPORTED, "plan_capacity: at most %d requests", kMaxPlanRequests);
    }
    int64_t blocks = 0;
    int32_t max_nodes = 1;
    for (int32_t r = 0; r < num_requests; ++r) {
        const int32_t n = node_counts_host[r];
        if (n < 1 || n > kMaxPlanNodes) {
            return fail(TV_ERR_UNSUPPORTED, "plan_capacity: request %d has %d nodes", r, n);
        }
        max_nodes = n > max_nodes ? n : max_nodes;
        const int hpw = n <= nodes_per_item(2, qpk) && num_kv_heads >= 2 ? 2 : 1;
        const int npw = nodes_per_item(hpw, qpk);
        blocks += static_cast<int64_t>((num_kv_heads + hpw - 1) / hpw) * ((n + npw - 1) / npw);
    }
    return fill_capacity(blocks, max_nodes, block_size, num_compute_units, chunk_keys, max_prefix, info);
}

extern "C" int tv_tree_attention_plan_capacity_packed(int32_t total_queries, int32_t num_requests,
                                                      int64_t sum_node_squares, int32_t num_kv_heads,
                                                      int32_t queries_per_kv, int32_t block_size,
                                                      int32_t num_compute_units, int32_t chunk_keys,
                                                      int64_t max_prefix, tv_attention_plan_info* info) {
    clear_error();
    const int32_t qpk = queries_per_kv;
    if (!info || total_queries < num_requests ||
        !capacity_args_ok(num_requests, num_kv_heads, qpk, block_size, num_compute_units, chunk_keys, max_prefix)) {
        return fail(TV_ERR_INVALID, "plan_capacity_packed: invalid arguments");
    }
    if (num_requests > kMaxPlanRequests) {
        return fail(TV_ERR_UNSUPPORTED, "plan_capacity_packed: at most %d requests", kMaxPlanRequests);
    }
    // Largest node count: every other request has at least one node, and when the sum of
    // squares is given, max_r T_r^2 <= sum_r T_r^2.
    int64_t max_nodes = static_cast<int64_t>(total_queries) - (num_requests - 1);
    if (sum_node_squares > 0) {
        int64_t root = static_cast<int64_t>(sqrt(static_cast<double>(sum_node_squares)));
        while (root * root > sum_node_squares) --root;
        while ((root + 1) * (root + 1) <= sum_node_squares) ++root;
        max_nodes = std::min(max_nodes, root);
    }
    max_nodes = std::min<int64_t>(max_nodes, kMaxPlanNodes);
    // With N = nodes_per_item(1, qpk) nodes per one-head item (64 at qpk 4), a request of T
    // nodes has at most num_kv_heads * ceil(T / N) node blocks (two-head groups of smaller
    // trees have fewer), and sum_r ceil(T_r / N) is at most (Q + (N - 1) R) / N and at most
    // R * ceil(max T / N).
    const int64_t npw1 = nodes_per_item(1, qpk);
    const int64_t per_head = std::min<int64_t>((static_cast<int64_t>(total_queries) + (npw1 - 1) * num_requests) / npw1,
                                               static_cast<int64_t>(num_requests) * ((max_nodes + npw1 - 1) / npw1));
    const int64_t blocks = static_cast<int64_t>(num_kv_heads) * per_head;
    return fill_capacity(blocks, static_cast<int32_t>(max_nodes), block_size, num_compute_units, chunk_keys,
                         max_prefix, info);
}

extern "C" int tv_stream_capture_info(void* stream, int32_t* capturing, uint64_t* capture_id) {
    clear_error();
    if (!capturing || !capture_id) return fail(TV_ERR_INVALID, "stream_capture_info: null output");
    hipStreamCaptureStatus status = hipStreamCaptureStatusNone;
    unsigned long long id = 0;
    const hipError_t err = hipStreamGetCaptureInfo(as_stream(stream), &status, &id);
    if (err != hipSuccess) {
        return fail(TV_ERR_LAUNCH, "stream_capture_info: %s", hipGetErrorString(err));
    }
    *capturing = status == hipStreamCaptureStatusActive ? 1 : (status == hipStreamCaptureStatusNone ? 0 : -1);
    *capture_id = status == hipStreamCaptureStatusNone ? 0 : static_cast<uint64_t>(id);
    return TV_OK;
}

extern "C" int tv_tree_attention_plan_device(const int32_t* prefix_lens, const int32_t* node_counts,
                                             int32_t num_requests, int32_t num_kv_heads, int32_t queries_per_kv,
                                             int32_t block_size,
                                             int32_t num_compute_units, int32_t chunk_keys, int32_t item_capacity,
                                             int32_t group_capacity, int32_t slot_capacity, int32_t* items,
                                             int32_t* groups, int32_t* counts, void* stream) {
    clear_error();
    if (num_requests < 1 || num_requests > kMaxPlanRequests || num_kv_heads < 1 || !supported_group(queries_per_kv) ||
        block_size < 32 ||
        block_size % 32 || num_compute_units < 1 || chunk_keys < 0 || chunk_keys % 32 || item_capacity < 1 ||
        item_capacity > kMaxSortItems || group_capacity < 0 || slot_capacity < 0) {
        return fail(TV_ERR_INVALID, "plan_device: invalid arguments");
    }
    if (!prefix_lens || !node_counts || !items || !counts || (group_capacity > 0 && !groups)) {
        return fail(TV_ERR_INVALID, "plan_device: null pointer");
    }
    PlanArgs a{prefix_lens, node_counts, num_requests, num_kv_heads, queries_per_kv, block_size, num_compute_units,
               chunk_keys, item_capacity, group_capacity, slot_capacity, items, groups, counts};
    hipLaunchKernelGGL(plan_device_kernel, dim3(1), dim3(kPlanThreads), 0, as_stream(stream), a);
    return check_launch("plan_device");
}
