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

// Block-wide exclusive scan of one int per thread (kPlanThreads threads); returns the
// thread's prefix and writes the total to *total.  A scan within each wave (lane
// shuffles), then the wave totals through LDS: two barriers.
__device__ int64_t block_scan(int64_t v, int64_t* scratch, int64_t* total) {
    const int t = threadIdx.x, lane = t & 63, w = t >> 6;
    int64_t x = v;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
        const int64_t y = __shfl_up(x, off);
        if (lane >= off) x += y;
    }
    if (lane == 63) scratch[w] = x;
    __syncthreads();
    int64_t before = 0, all = 0;
#pragma unroll
    for (int k = 0; k < kPlanWaves; ++k) {
        const int64_t s = scratch[k];
        before += k < w ? s : 0;
        all += s;
    }
    if (t == 0) *total = all;
    __syncthreads();   // *total is visible, and every thread has read `scratch`
    return before + x - v;
}

// Sum over one wave (returned to every lane).
__device__ __forceinline__ int64_t wave_sum(int64_t v) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off);
    return v;
}

// Block-wide sum of one int64 per thread (kPlanThreads threads), returned to all.
__device__ int64_t block_sum(int64_t v, int64_t* scratch) {
    for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off);
    const int t = threadIdx.x;
    __syncthreads();
    if ((t & 63) == 0) scratch[t >> 6] = v;
    __syncthreads();
    int64_t total = 0;
    for (int w = 0; w < kPlanThreads / 64; ++w) total += scratch[w];
    __syncthreads();   // every thread has read `scratch` before anyone reuses it
    return total;
}

// The host planner's chunk length for a prefix of p keys and chunk target tau.
__device__ __forceinline__ int64_t chunk_for(int64_t p, int hpw, int64_t tau, int64_t max_chunk) {
    int64_t chunk = min(round_up(max(static_cast<int64_t>(kMinChunkKeys), tau / cost_weight(hpw)), 32), max_chunk);
    const int64_t nchunks = p > 0 ? (p + chunk - 1) / chunk : 1;
    chunk = round_up((p + nchunks - 1) / max<int64_t>(nchunks, 1), 32);
    return chunk < 32 ? 32 : chunk;
}

__global__ void __launch_bounds__(kPlanThreads)
plan_device_kernel(const PlanArgs a) {
    __shared__ uint64_t keys[kMaxSortItems];
    __shared__ int64_t scan[kPlanThreads];
    __shared__ int64_t totals[4];
    __shared__ int32_t req_chunk[kMaxPlanRequests], req_nchunks[kMaxPlanRequests];
    __shared__ int32_t req_item_off[kMaxPlanRequests], req_group_off[kMaxPlanRequests], req_slot_off[kMaxPlanRequests];
    __shared__ int32_t stream_id[kMaxSortItems];   // (request, head group, chunk) of each sorted item
    __shared__ int shared_flag;
    __shared__ int32_t probe_fits[kPlanWaves];
    const int t = threadIdx.x;
    const int R = a.num_requests;
    const int B = a.block_size;

    // 1. Costs and their total.
    int64_t my_cost = 0;
    bool bad = false;
    for (int r = t; r < R; r += kPlanThreads) {
        const int p = a.prefix_lens[r], n = a.node_counts[r];
        if (p < 0 || n < 1 || n > 1024) {
            bad = true;
            continue;
        }
        const int hpw = heads_per_group(n, a.num_kv_heads, a.qpk);
        const int npw = nodes_per_item(hpw, a.qpk);
        const int64_t groups = (a.num_kv_heads + hpw - 1) / hpw;
        const int64_t blocks = (n + npw - 1) / npw;
        my_cost += groups * blocks * cost_weight(hpw) * (static_cast<int64_t>(p) + n);
    }
    if (t == 0) shared_flag = 0;
    __syncthreads();
    if (bad) atomicOr(&shared_flag, 1);
    const int64_t cost_before = block_scan(my_cost, scan, &totals[0]);
    (void)cost_before;
    const int64_t total_cost = totals[0];
    const int64_t target = max(static_cast<int64_t>(kMinChunkKeys), total_cost / a.compute_units);
    const int64_t max_chunk = (static_cast<int64_t>(kMaxChunkPages - 1) * B) / 32 * 32;

    // 1b. The host's refit of the chunk target when the items leave the last of at most
    // kFillRounds rounds part-empty: the smallest target whose item count fits the same
    // rounds.  The count falls as the target grows, so any search finds the host's
    // bisection result; here each of the 16 waves probes one target per round (a
    // 17-way search, one barrier per round).
    auto request_items = [&](int r, int64_t tau) -> int64_t {
        const int64_t p = max(0, a.prefix_lens[r]);
        const int nodes = max(1, min(1024, a.node_counts[r]));
        const int hpw = heads_per_group(nodes, a.num_kv_heads, a.qpk);
        const int npw = nodes_per_item(hpw, a.qpk);
        const int64_t units = static_cast<int64_t>((a.num_kv_heads + hpw - 1) / hpw) * ((nodes + npw - 1) / npw);
        const int64_t chunk = chunk_for(p, hpw, tau, max_chunk);
        return units * (p > 0 ? (p + chunk - 1) / chunk : 1);
    };
    int64_t tau = target;
    if (a.chunk_keys == 0) {
        int64_t now = 0;
        for (int r = t; r < R; r += kPlanThreads) now += request_items(r, target);
        now = block_sum(now, scan);
        const int64_t rounds = (now + a.compute_units - 1) / a.compute_units;
        if (now > a.compute_units && rounds <= kFillRounds) {
            const int64_t limit = rounds * a.compute_units;
            const int lane = t & 63, w = t >> 6;
            int64_t lo = 1, hi = target;   // items(hi) <= limit; the answer is in [lo, hi]
            while (lo < hi) {
                const int64_t span = hi - lo;
                const int64_t probe = lo + span * (w + 1) / (kPlanWaves + 1);   // in [lo, hi)
                int64_t n = 0;
                for (int r = lane; r < R; r += 64) n += request_items(r, probe);
                n = wave_sum(n);
                if (lane == 0) probe_fits[w] = n <= limit ? 1 : 0;
                __syncthreads();
                int64_t new_lo = lo, new_hi = hi;
#pragma unroll
                for (int k = 0; k < kPlanWaves; ++k) {
                    const int64_t pk = lo + span * (k + 1) / (kPlanWaves + 1);
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
    int64_t my_items = 0, my_groups = 0, my_slots = 0;
    for (int r = r0; r < r1; ++r) {
        const int p = max(0, a.prefix_lens[r]);
        const int n = max(1, min(1024, a.node_counts[r]));
        const int hpw = heads_per_group(n, a.num_kv_heads, a.qpk);
        const int npw = nodes_per_item(hpw, a.qpk);
        const int64_t G = (a.num_kv_heads + hpw - 1) / hpw;
        const int64_t NB = (n + npw - 1) / npw;
        const int64_t chunk = a.chunk_keys > 0 ? a.chunk_keys : chunk_for(p, hpw, tau, max_chunk);
        const int64_t nchunks = p > 0 ? (p + chunk - 1) / chunk : 1;
        req_chunk[r] = static_cast<int32_t>(chunk);
        req_nchunks[r] = static_cast<int32_t>(nchunks);
        my_items += G * NB * nchunks;
        if (nchunks > 1) {
            my_groups += G * NB;
            my_slots += G * NB * nchunks;
        }
    }
    int64_t item_base = block_scan(my_items, scan, &totals[1]);
    int64_t group_base = block_scan(my_groups, scan, &totals[2]);
    int64_t slot_base = block_scan(my_slots, scan, &totals[3]);
    for (int r = r0; r < r1; ++r) {
        const int n = max(1, min(1024, a.node_counts[r]));
        const int hpw = heads_per_group(n, a.num_kv_heads, a.qpk);
        const int64_t G = (a.num_kv_heads + hpw - 1) / hpw;
        const int64_t NB = (n + nodes_per_item(hpw, a.qpk) - 1) / nodes_per_item(hpw, a.qpk);
        req_item_off[r] = static_cast<int32_t>(item_base);
        req_group_off[r] = static_cast<int32_t>(group_base);
        req_slot_off[r] = static_cast<int32_t>(slot_base);
        item_base += G * NB * req_nchunks[r];
        if (req_nchunks[r] > 1) {
            group_base += G * NB;
            slot_base += G * NB * req_nchunks[r];
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

    // 3. Sort keys: (~cost, request, head group, chunk, block), each item's secondary
    // index being its rank in that (request, head group, chunk, block) enumeration.
    int npow = 1;
    while (npow < num_items) npow <<= 1;
    for (int e = t; e < npow; e += kPlanThreads) keys[e] = ~0ull;
    __syncthreads();
    for (int r = r0; r < r1; ++r) {
        const int p = max(0, a.prefix_lens[r]);
        const int n = max(1, min(1024, a.node_counts[r]));
        const int hpw = heads_per_group(n, a.num_kv_heads, a.qpk);
        const int G = (a.num_kv_heads + hpw - 1) / hpw;
        const int NB = (n + nodes_per_item(hpw, a.qpk) - 1) / nodes_per_item(hpw, a.qpk);
        const int nc = req_nchunks[r];
        const int64_t chunk = req_chunk[r];
        for (int hg = 0; hg < G; ++hg) {
            for (int c = 0; c < nc; ++c) {
                const int64_t kb = min(static_cast<int64_t>(p), c * chunk), ke = min(static_cast<int64_t>(p), (c + 1) * chunk);
                const int64_t cost = cost_weight(hpw) * ((ke - kb) + (c == nc - 1 ? n : 0));
                for (int nb = 0; nb < NB; ++nb) {
                    const int64_t idx = req_item_off[r] + (static_cast<int64_t>(hg) * nc + c) * NB + nb;
                    keys[idx] = (static_cast<uint64_t>(0x7fffffffu - static_cast<uint32_t>(cost)) << 32) |
                                static_cast<uint32_t>(idx);
                }
            }
        }
    }
    __syncthreads();
    for (int size = 2; size <= npow; size <<= 1) {
        for (int stride = size >> 1; stride > 0; stride >>= 1) {
            for (int e = t; e < npow; e += kPlanThreads) {
                const int partner = e ^ stride;
                if (partner > e) {
                    const bool ascending = (e & size) == 0;
                    const uint64_t x = keys[e], y = keys[partner];
                    if ((x > y) == ascending) {
                        keys[e] = y;
                        keys[partner] = x;
                    }
                }
            }
            // A stride below 64 pairs elements that one wave owns (e and e ^ stride differ
            // only in bits below 64, and thread t owns e = t + k * kPlanThreads).  Between
            // two such stages the wave's own LDS ordering is enough; a workgroup barrier
            // precedes and follows every stage whose pairs cross waves, and the last stage.
            const int next_stride = stride > 1 ? stride >> 1 : size;
            if (stride < 64 && next_stride < 64 && size < npow) {
                __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
                __builtin_amdgcn_wave_barrier();
                __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
            } else {
                __syncthreads();
            }
        }
    }

    // Decode a sorted key back into its item (request found by the offsets).
    auto decode = [&](int64_t sorted_pos, int32_t* out) {
        const int64_t idx = static_cast<int64_t>(keys[sorted_pos] & 0xffffffffull);
        int lo = 0, hi = R - 1;
        while (lo < hi) {      // last request whose item offset is <= idx
            const int mid = (lo + hi + 1) >> 1;
            if (req_item_off[mid] <= idx) lo = mid; else hi = mid - 1;
        }
        const int r = lo;
        const int p = max(0, a.prefix_lens[r]);
        const int n = max(1, min(1024, a.node_counts[r]));
        const int hpw = heads_per_group(n, a.num_kv_heads, a.qpk);
        const int NB = (n + nodes_per_item(hpw, a.qpk) - 1) / nodes_per_item(hpw, a.qpk);
        const int nc = req_nchunks[r];
        const int64_t local = idx - req_item_off[r];
        const int nb = static_cast<int>(local % NB);
        const int64_t hc = local / NB;
        const int c = static_cast<int>(hc % nc);
        const int hg = static_cast<int>(hc / nc);
        const int64_t chunk = req_chunk[r];
        out[0] = r;
        out[1] = hg * hpw;
        out[2] = nb * nodes_per_item(hpw, a.qpk);
        out[3] = static_cast<int32_t>(min(static_cast<int64_t>(p), c * chunk));
        out[4] = static_cast<int32_t>(min(static_cast<int64_t>(p), (c + 1) * chunk));
        out[5] = (c == nc - 1 ? kItemLastChunk : 0) | (nb == NB - 1 ? kItemLastBlock : 0) | (a.qpk << kItemGroupShift);
        out[6] = nc > 1 ? req_slot_off[r] + (hg * NB + nb) * nc + c : -1;
        out[7] = hpw;
    };
    // Stream identity (request, head group, chunk) of a sorted position.
    auto stream_of = [&](int64_t sorted_pos) -> int64_t {
        const int64_t idx = static_cast<int64_t>(keys[sorted_pos] & 0xffffffffull);
        int lo = 0, hi = R - 1;
        while (lo < hi) {
            const int mid = (lo + hi + 1) >> 1;
            if (req_item_off[mid] <= idx) lo = mid; else hi = mid - 1;
        }
        const int n = max(1, min(1024, a.node_counts[lo]));
        const int hpw = heads_per_group(n, a.num_kv_heads, a.qpk);
        const int NB = (n + nodes_per_item(hpw, a.qpk) - 1) / nodes_per_item(hpw, a.qpk);
        return (static_cast<int64_t>(lo) << 32) | ((idx - req_item_off[lo]) / NB);
    };

    // 4. XCD placement (tv_plan.cpp::place_for_xcds) and output.
    for (int64_t i = t; i < num_items; i += kPlanThreads) {
        const int64_t s = stream_of(i);
        stream_id[i] = static_cast<int32_t>((s >> 32) * kMaxSortItems + (s & 0xffffffff));
    }
    if (t == 0) shared_flag = 0;
    __syncthreads();
    // Bit 0: some stream has several items; bit 1: some stream's item count (its
    // request's node blocks) is not a multiple of 8.
    for (int64_t i = 1 + t; i < num_items; i += kPlanThreads) {
        if (stream_id[i] == stream_id[i - 1]) atomicOr(&shared_flag, 1);
    }
    for (int r = t; r < R; r += kPlanThreads) {
        const int n = max(1, min(1024, a.node_counts[r]));
        const int hpw = heads_per_group(n, a.num_kv_heads, a.qpk);
        const int NB = (n + nodes_per_item(hpw, a.qpk) - 1) / nodes_per_item(hpw, a.qpk);
        if (NB > 1 && NB % kXcds) atomicOr(&shared_flag, 2);
    }
    __syncthreads();
    const bool shared = (shared_flag & 1) != 0;
    const bool aligned = (shared_flag & 2) == 0;
    constexpr int kWindow = kXcds * kXcds;
    const int64_t full = shared ? (num_items / kWindow) * kWindow : 0;
    auto position_of = [&](int64_t rank) {
        if (rank >= full) return rank;
        const int64_t w = rank - rank % kWindow;
        const int k = static_cast<int>(rank - w);
        const int column = (w / kWindow) % 2 ? kXcds - 1 - k / kXcds : k / kXcds;   // odd windows mirrored
        return w + kXcds * (k % kXcds) + column;
    };
    if (shared && aligned) {
        // Groups ahead of the at most 7 singles before them since the last multiple of
        // 8: ranks from the number of single items before each sorted position.
        constexpr int kPer = kMaxSortItems / kPlanThreads;
        const int64_t i0 = static_cast<int64_t>(t) * kPer;
        uint32_t single_bits = 0;
        int64_t mine = 0;
        for (int e = 0; e < kPer; ++e) {
            const int64_t i = i0 + e;
            if (i >= num_items) break;
            const int32_t sid = stream_id[i];
            const bool single = !((i > 0 && stream_id[i - 1] == sid) || (i + 1 < num_items && stream_id[i + 1] == sid));
            single_bits |= static_cast<uint32_t>(single) << e;
            mine += single;
        }
        const int64_t before = block_scan(mine, scan, &totals[0]);   // syncs: stream_id reads are done
        const int64_t singles_total = totals[0];
        int64_t run = before;
        for (int e = 0; e < kPer; ++e) {
            const int64_t i = i0 + e;
            if (i >= num_items) break;
            stream_id[i] = static_cast<int32_t>(run);                 // now: singles before position i
            run += (single_bits >> e) & 1u;
        }
        __syncthreads();
        auto singles_before = [&](int64_t q) -> int64_t { return q < num_items ? stream_id[q] : singles_total; };
        for (int e = 0; e < kPer; ++e) {
            const int64_t i = i0 + e;
            if (i >= num_items) break;
            const int64_t sb = stream_id[i];
            int64_t rank;
            if (!((single_bits >> e) & 1u)) {
                rank = (i - sb) + sb / kXcds * kXcds;
            } else {
                int64_t lo = i + 1, hi = num_items;   // first q with floor8(singles before q) > sb
                while (lo < hi) {
                    const int64_t mid = (lo + hi) >> 1;
                    if (singles_before(mid) / kXcds * kXcds > sb) hi = mid; else lo = mid + 1;
                }
                rank = sb + (lo - singles_before(lo));
            }
            decode(i, a.items + position_of(rank) * 8);
        }
    } else {
        for (int64_t i = t; i < num_items; i += kPlanThreads) {
            int64_t rank = i;
            if (i < full) {
                const int64_t w = i - i % kWindow;
                const int k = static_cast<int>(i - w);
                // Rank of item k in the window's "grouped first" order.
                auto grouped = [&](int j) {
                    const int32_t s = stream_id[w + j];
                    return (j + 1 < kWindow && stream_id[w + j + 1] == s) || (j > 0 && stream_id[w + j - 1] == s);
                };
                const bool mine = grouped(k);
                int within = 0;
                for (int j = 0; j < kWindow; ++j) {
                    if (j == k) continue;
                    const bool g = grouped(j);
                    if (mine ? (g && j < k) : (g || j < k)) ++within;
                }
                rank = w + within;
            }
            decode(i, a.items + position_of(rank) * 8);
        }
    }
    // Merge groups in (request, head group, block) order with their first partial slot.
    for (int r = r0; r < r1; ++r) {
        const int nc = req_nchunks[r];
        if (nc < 2) continue;
        const int n = max(1, min(1024, a.node_counts[r]));
        const int hpw = heads_per_group(n, a.num_kv_heads, a.qpk);
        const int G = (a.num_kv_heads + hpw - 1) / hpw;
        const int NB = (n + nodes_per_item(hpw, a.qpk) - 1) / nodes_per_item(hpw, a.qpk);
        for (int hg = 0; hg < G; ++hg) {
            for (int nb = 0; nb < NB; ++nb) {
                int32_t* gr = a.groups + static_cast<int64_t>(req_group_off[r] + hg * NB + nb) * 8;
                gr[0] = r;
                gr[1] = hg * hpw;
                gr[2] = nb * nodes_per_item(hpw, a.qpk);
                gr[3] = hpw;
                gr[4] = req_slot_off[r] + (hg * NB + nb) * nc;
                gr[5] = nc;
                gr[6] = a.qpk;   // the grouping the slots' rows are laid out for
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
        if (n < 1 || n > 1024) return fail(TV_ERR_UNSUPPORTED, "plan_capacity: request %d has %d nodes", r, n);
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
    max_nodes = std::min<int64_t>(max_nodes, 1024);
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
