// Device-side work planner for the packed tree-verify attention, for gfx950.
//
// Produces the same items and merge groups as the host planner (tv_plan.cpp), item for
// item, but from the prefix lengths and node counts in device memory.  A launch sequence
// that reads its plan from the device keeps fixed grid sizes while the prefix lengths
// change, which is what a captured HIP graph replays: the attention and merge kernels
// are launched with a capacity grid and their surplus workgroups exit on the counts
// this planner writes.
//
// One 1024-thread workgroup (steps 1 and 2 in wave 0 alone, one request per lane and no
// barrier, for batches of at most 64 requests):
//   1. per request: KV heads per group, node blocks, cost; the total cost (reduction);
//   2. per request: prefix chunk length and count (the host formulas), item / group /
//      slot counts, and their exclusive prefix sums (one scan); the host's refit of the
//      chunk target when the last round of items is part-empty;
//   3. the items in the host comparator's order, (~cost, request, head group, chunk,
//      block), longest first: up to 128 requests by ranking each request's two cost
//      classes (its chunks before the last, its last chunk) and placing every item at its
//      class's offset; larger batches by a bitonic sort of 64-bit keys in LDS;
//   4. the XCD placement of the host (64-item windows, multi-block groups first,
//      column-major), then the items and groups are written out; the cost-class path
//      writes the items of plans whose placement needs no window ranking directly.
// Capacity overflow writes zero counts and an error flag instead of writing past the
// caller's arrays.
#include <math.h>
#include <stdint.h>

#include <algorithm>

#include "tv_internal.h"

namespace tv {
namespace {

constexpr int kPlanThreads = 1024;
constexpr int kMaxSortItems = 8192;      // items of one plan (64 KiB of sorted keys in LDS)
constexpr int kMaxPlanRequests = 2048;
// A sorted position holds (request in bits 32-47, enumeration index in bits 0-31); the
// XCD placement may park a 16-bit position in bits 48-63.
static_assert(kMaxPlanRequests <= 65536 && kMaxSortItems <= 65536, "sorted keys pack 16-bit fields");
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

__device__ __forceinline__ int64_t round_up(int64_t x, int64_t m) { return (x + m - 1) / m * m; }

// Cost of one key of a work item in quarter key-steps of a one-head item: a two-head
// tile costs ~1.25x a one-head tile (each wave still runs one head's MFMAs).  The host
// planner uses the same weights.
__device__ __forceinline__ int64_t cost_weight(int hpw) { return hpw == 2 ? 5 : 4; }

constexpr int kPlanWaves = kPlanThreads / 64;
constexpr int kPer = kMaxSortItems / kPlanThreads;   // sorted positions per thread
constexpr int kProbeWaves = 4;   // waves that probe chunk targets in the refit (one per SIMD)

// One lane move of a wave scan (gfx9 DPP, on both halves of an int64): `kCtrl` is row_shr:n
// (0x110 + n) or a row broadcast, `kRowMask` the rows that receive; a lane with no source, or
// in a row that does not receive, reads 0.  Every lane of the wave must be active.
template <int kCtrl, int kRowMask = 0xf>
__device__ __forceinline__ int64_t dpp_move(int64_t v) {
    const int lo = __builtin_amdgcn_update_dpp(0, static_cast<int>(v), kCtrl, kRowMask, 0xf, false);
    const int hi = __builtin_amdgcn_update_dpp(0, static_cast<int>(v >> 32), kCtrl, kRowMask, 0xf, false);
    return static_cast<int64_t>((static_cast<uint64_t>(static_cast<uint32_t>(hi)) << 32) | static_cast<uint32_t>(lo));
}

// Inclusive prefix sum over the 64 lanes: shifts by 1, 2, 4 and 8 within each row of 16
// lanes, then row 0's last lane into rows 1 and 3 and lane 31 into rows 2 and 3.  DPP moves
// instead of LDS permutes: a few cycles per step.
__device__ __forceinline__ int64_t wave_inclusive_sum(int64_t x) {
    x += dpp_move<0x111>(x);
    x += dpp_move<0x112>(x);
    x += dpp_move<0x114>(x);
    x += dpp_move<0x118>(x);
    x += dpp_move<0x142, 0xa>(x);   // row_bcast:15
    x += dpp_move<0x143, 0xc>(x);   // row_bcast:31
    return x;
}

// Lane `lane`'s value (wave-uniform `lane`), to every lane.
__device__ __forceinline__ int64_t lane_value(int64_t x, int lane) {
    const uint32_t lo = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(x), lane));
    const uint32_t hi = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(x >> 32), lane));
    return static_cast<int64_t>((static_cast<uint64_t>(hi) << 32) | lo);
}

// Block-wide exclusive scan of three int64 values per thread over the first `waves` waves
// (wave-uniform, at least 1; every thread of a later wave must hold zeros, and gets no
// prefixes back): each such thread's prefixes of v[0..2] are returned in v, the totals
// written to total[0..2].  A scan within each of those waves, then their totals through LDS,
// one per lane, scanned again.  Sixteen waves share the CU's four SIMDs, so a wave with
// nothing to add skips its scans instead of repeating them.  Every thread takes both barriers.
__device__ void block_scan3(int64_t (&v)[3], int waves, int64_t* scratch, int64_t* total) {
    const int t = threadIdx.x, lane = t & 63;
    const int w = __builtin_amdgcn_readfirstlane(t >> 6);
    int64_t x[3] = {0, 0, 0};
    if (w < waves) {
#pragma unroll
        for (int j = 0; j < 3; ++j) x[j] = wave_inclusive_sum(v[j]);
        if (lane == 63) {
#pragma unroll
            for (int j = 0; j < 3; ++j) scratch[3 * w + j] = x[j];
        }
    }
    __syncthreads();
    if (w < waves) {
#pragma unroll
        for (int j = 0; j < 3; ++j) {
            const int64_t sums = wave_inclusive_sum(lane < waves ? scratch[3 * lane + j] : 0);
            const int64_t before = w > 0 ? lane_value(sums, w - 1) : 0;
            if (t == 0) total[j] = lane_value(sums, waves - 1);
            v[j] = before + x[j] - v[j];
        }
    }
    __syncthreads();   // the totals are visible, and every thread has read `scratch`
}

// Sum over one wave (returned to every lane).
__device__ __forceinline__ int64_t wave_sum(int64_t v) { return lane_value(wave_inclusive_sum(v), 63); }

// Block-wide sum of one int64 per thread, returned to all; as for block_scan3, only the
// first `waves` waves (wave-uniform, at least 1) may hold nonzero values.
__device__ int64_t block_sum(int64_t v, int waves, int64_t* scratch) {
    const int t = threadIdx.x, lane = t & 63;
    const int w = __builtin_amdgcn_readfirstlane(t >> 6);
    if (w < waves) v = wave_sum(v);
    __syncthreads();
    if (w < waves && lane == 0) scratch[w] = v;
    __syncthreads();
    const int64_t total = wave_sum(lane < waves ? scratch[lane] : 0);
    __syncthreads();   // every thread has read `scratch` before anyone reuses it
    return total;
}

// One request's geometry from its (clamped) node count: KV heads per item, nodes per item,
// head groups and node blocks (the host planner's heads_per_group and nodes_per_item, with
// nw = 32 / qpk nodes per wave taken once per thread, so only the node-block count divides).
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

// q = a / b and rem = a % b for 0 <= a < 2^20 and b >= 1: a float reciprocal estimate is
// within 1/4 of a / b, so its truncation is off by at most one, which the remainder fixes.
// Item and block indices here stay below 2^13; a generic 32-bit division costs ~35 VALU
// instructions, which the per-item loops of sixteen waves on four SIMDs feel.
__device__ __forceinline__ int div_small(int a, int b, int& rem) {
    int q = static_cast<int>(static_cast<float>(a) * __builtin_amdgcn_rcpf(static_cast<float>(b)));
    int r = a - q * b;
    if (r >= b) {
        ++q;
        r -= b;
    } else if (r < 0) {
        --q;
        r += b;
    }
    rem = r;
    return q;
}

// The host planner's chunk length (tv_plan.cpp, chunk_for) for a prefix of p keys before
// a tree of n nodes, with q = tau / cost_weight(hpw) precomputed: the chunk count from
// min(round_up(max(64, q), 32), max_chunk), then the prefix and the tree's weight shared
// evenly over the chunks as far as the count and the cap allow.  Every quantity after the
// first min is below 2^32.
constexpr uint32_t kTreeKeyWeight = 2;   // prefix keys a tree node costs (tv_plan.cpp)

__device__ __forceinline__ uint32_t chunk_of(uint32_t p, uint32_t n, int64_t q, int64_t max_chunk) {
    const int64_t c0 = min(round_up(max(static_cast<int64_t>(kMinChunkKeys), min(q, max_chunk)), 32), max_chunk);
    const uint32_t c = static_cast<uint32_t>(c0);
    const uint32_t nchunks = p > 0 ? (p + c - 1) / c : 1;
    uint32_t chunk = ((p + nchunks - 1) / nchunks + 31) / 32 * 32;
    if (nchunks > 1) {
        const uint32_t even = ((p + kTreeKeyWeight * n + nchunks - 1) / nchunks + 31) / 32 * 32;
        const uint32_t keep = min((p - 1) / (nchunks - 1) / 32 * 32, static_cast<uint32_t>(max_chunk));
        chunk = max(chunk, min(even, keep));
    }
    return chunk < 32 ? 32 : chunk;
}

// Plans in one 1024-thread workgroup.  The prefix lengths and node counts are read once into
// LDS; every later per-request quantity comes from there.
__global__ void __launch_bounds__(kPlanThreads)
plan_device_kernel(const PlanArgs a) {
    __shared__ uint64_t keys[kMaxSortItems];
    // The cost classes of step 3, then per sorted position the data of step 4's placement.
    __shared__ __align__(16) int32_t stream_id[kMaxSortItems];
    __shared__ int32_t req_p[kMaxPlanRequests], req_n[kMaxPlanRequests];
    __shared__ int32_t req_chunk[kMaxPlanRequests], req_nchunks[kMaxPlanRequests];
    __shared__ int32_t req_item_off[kMaxPlanRequests], req_group_off[kMaxPlanRequests], req_slot_off[kMaxPlanRequests];
    __shared__ int64_t scan[3 * kPlanWaves];
    __shared__ int64_t totals[4];
    // Per request: node blocks (bits 0-11), its chunks all cost the same (bit 14, set by the
    // cost-class ranking), two KV heads per item (bit 15).
    __shared__ uint16_t req_bits[kMaxPlanRequests];
    __shared__ int shared_flag;
    __shared__ int shape_flag;   // bit 0: some request has several node blocks; bit 1: one not a multiple of 8
    __shared__ int class_singles;   // single items of a cost-class plan
    __shared__ int32_t probe_fits[kPlanWaves];
    __shared__ int64_t probe_val[kPlanWaves];
    const int t = threadIdx.x;
    const int lane = t & 63;
    const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
    const int R = a.num_requests;
    const int B = a.block_size;
    const int KV = a.num_kv_heads, QPK = a.qpk, NW = 32 / a.qpk;
    // Batches of at most 64 requests run steps 1 and 2 (and the cost classes of step 3) in wave
    // 0 alone, one request per lane, with wave reductions and no barrier; the other waves wait
    // at the barrier after them.  Larger batches spread the requests over the block.
    const bool one_wave = R <= 64;
    const int64_t max_chunk = min((static_cast<int64_t>(kMaxChunkPages - 1) * B) / 32 * 32, int64_t{1} << 31);
    // A request's geometry from req_bits (req_shape's result, without its division).
    auto shape_at = [&](int r) -> ReqShape {
        const int bits = req_bits[r];
        ReqShape s;
        s.hpw = (bits >> 15) + 1;
        s.npw = s.hpw == 2 ? 4 * NW : 8 * NW;
        s.G = s.hpw == 2 ? (KV + 1) >> 1 : KV;
        s.NB = bits & 0xfff;
        return s;
    };
    // Items of request r at chunk target tau (q4 = tau / 4, q5 = tau / 5).
    auto request_items = [&](int r, int64_t q4, int64_t q5) -> int64_t {
        const uint32_t p = static_cast<uint32_t>(req_p[r]);
        const ReqShape s = shape_at(r);
        const uint32_t chunk = chunk_of(p, static_cast<uint32_t>(req_n[r]), s.hpw == 2 ? q5 : q4, max_chunk);
        return static_cast<int64_t>(s.G) * s.NB * (p > 0 ? (p + chunk - 1) / chunk : 1u);
    };

    // Step 3's cost classes (ranked there) in stream_id, which the placement overwrites later.
    // Class 0: the chunks before the last (the whole request when both costs are equal), class
    // 1: the last chunk.  An absent class has no items and a cost field above every real one,
    // so the present classes rank first and every key stays distinct.
    constexpr int kClassRankMax = 256;
    uint64_t* ckey = reinterpret_cast<uint64_t*>(stream_id);   // [2R]: (~cost, request, class)
    int32_t* ccount = stream_id + 2 * kClassRankMax;            // [2R] items per class
    int32_t* crank = ccount + kClassRankMax;                     // [2R] rank of each class
    int32_t* cstart = crank + kClassRankMax;                     // [rank] first position of that class
    int32_t* sstart = cstart + kClassRankMax;                    // [rank] single items before that class
    auto write_classes = [&](int r) {
        auto class_key = [&](int64_t cost, int cls) {
            return (static_cast<uint64_t>(0x7fffffffu - static_cast<uint32_t>(cost)) << 32) |
                   static_cast<uint32_t>(2 * r + cls);
        };
        auto absent_key = [&](int cls) { return (uint64_t{0xffffffffu} << 32) | static_cast<uint32_t>(2 * r + cls); };
        const ReqShape sh = shape_at(r);
        const int nc = req_nchunks[r];
        const int64_t p = req_p[r], chunk = req_chunk[r], w = cost_weight(sh.hpw);
        const int64_t units = static_cast<int64_t>(sh.G) * sh.NB;
        const int64_t last = w * ((p - min(p, (nc - 1) * chunk)) + req_n[r]);
        const int64_t mid = w * chunk;
        if (nc == 1) {
            ckey[2 * r] = absent_key(0);
            ccount[2 * r] = 0;
            ckey[2 * r + 1] = class_key(last, 1);
            ccount[2 * r + 1] = static_cast<int32_t>(units);
        } else if (mid == last) {
            ckey[2 * r] = class_key(mid, 0);
            ccount[2 * r] = static_cast<int32_t>(units * nc);
            ckey[2 * r + 1] = absent_key(1);
            ccount[2 * r + 1] = 0;
            req_bits[r] |= 0x4000;
        } else {
            ckey[2 * r] = class_key(mid, 0);
            ccount[2 * r] = static_cast<int32_t>(units * (nc - 1));
            ckey[2 * r + 1] = class_key(last, 1);
            ccount[2 * r + 1] = static_cast<int32_t>(units);
        }
    };

    if (!one_wave || wave == 0) {   // wave-uniform; with one_wave nothing below takes a barrier
        // 1. Prefix lengths and node counts into LDS (clamped; a value outside the planner's
        // range fails the plan), request shapes, costs and their total.
        if (t == 0) {
            shared_flag = 0;
            shape_flag = 0;
        }
        bool bad = false;
        int my_shapes = 0;
        int64_t my_cost = 0;
        for (int r = t; r < R; r += kPlanThreads) {
            const int p = a.prefix_lens[r], n = a.node_counts[r];
            bad |= p < 0 || n < 1 || n > kMaxPlanNodes;
            const int pc = max(0, p), nc = max(1, min(kMaxPlanNodes, n));
            req_p[r] = pc;
            req_n[r] = nc;
            const ReqShape s = req_shape(nc, KV, NW);
            req_bits[r] = static_cast<uint16_t>(s.NB | (s.hpw == 2 ? 0x8000 : 0));
            my_shapes |= (s.NB > 1 ? 1 : 0) | (s.NB > 1 && s.NB % kXcds ? 2 : 0);
            my_cost += static_cast<int64_t>(s.G) * s.NB * cost_weight(s.hpw) * (static_cast<int64_t>(pc) + nc);
        }
        if (!one_wave) __syncthreads();   // the flags are cleared before anyone sets them
        if (bad) atomicOr(&shared_flag, 1);
        if (my_shapes) atomicOr(&shape_flag, my_shapes);
        // The block sum's barriers also publish req_p, req_n, req_bits and the flags.
        const int64_t total_cost = one_wave ? wave_sum(my_cost)
                                            : block_sum(my_cost, (min(R, kPlanThreads) + 63) / 64, scan);
        const int64_t target = max(static_cast<int64_t>(kMinChunkKeys), total_cost / a.compute_units);

        // 2. Chunking and per-request counts at chunk target tau (or the forced chunk length):
        // chunk lengths and counts per request, their exclusive prefix sums (one scan) and the
        // totals, in totals[1..3] and in tot[] of every thread taking part.  Requests are
        // handled in contiguous runs per thread so that one scan yields request-ordered offsets.
        const int per_thread = (R + kPlanThreads - 1) / kPlanThreads;
        const int r0 = min(R, t * per_thread), r1 = min(R, r0 + per_thread);
        int64_t tot[3];
        auto chunking = [&](int64_t tau) {
            int64_t base[3] = {0, 0, 0};   // items, groups, slots
            const int64_t q4 = tau / 4, q5 = tau / 5;
            for (int r = r0; r < r1; ++r) {
                const uint32_t p = static_cast<uint32_t>(req_p[r]);
                const ReqShape s = shape_at(r);
                const uint32_t chunk = a.chunk_keys > 0 ? static_cast<uint32_t>(a.chunk_keys)
                                                        : chunk_of(p, static_cast<uint32_t>(req_n[r]),
                                                                   s.hpw == 2 ? q5 : q4, max_chunk);
                const uint32_t nchunks = p > 0 ? (p + chunk - 1) / chunk : 1u;
                req_chunk[r] = static_cast<int32_t>(chunk);
                req_nchunks[r] = static_cast<int32_t>(nchunks);
                const int64_t units = static_cast<int64_t>(s.G) * s.NB;
                base[0] += units * nchunks;
                if (nchunks > 1) {
                    base[1] += units;
                    base[2] += units * nchunks;
                }
            }
            if (one_wave) {
#pragma unroll
                for (int j = 0; j < 3; ++j) {
                    const int64_t incl = wave_inclusive_sum(base[j]);
                    tot[j] = lane_value(incl, 63);
                    base[j] = incl - base[j];
                }
                if (t == 0) {
                    totals[1] = tot[0];
                    totals[2] = tot[1];
                    totals[3] = tot[2];
                }
            } else {
                block_scan3(base, ((R + per_thread - 1) / per_thread + 63) / 64, scan, &totals[1]);
                tot[0] = totals[1];
                tot[1] = totals[2];
                tot[2] = totals[3];
            }
            for (int r = r0; r < r1; ++r) {
                const ReqShape s = shape_at(r);
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
            if (!one_wave) __syncthreads();
        };
        chunking(target);

        // 2b. The host's refit of the chunk target when the items leave the last of at most
        // kFillRounds rounds part-empty: the smallest target whose item count fits the same
        // rounds, then the chunking again at it.  When the rounds are already full, every
        // smaller target that keeps the item count keeps every request's chunk count (each is
        // non-increasing in the target), so the plan stands.  The count falls as the target
        // grows, so any search finds the host's bisection result: wave 0 alone bisects; the
        // block has one wave per SIMD probe one target per round (a 5-way search, two
        // barriers per round; more probing waves would share the SIMDs and make every round
        // as much longer).
        if (a.chunk_keys == 0) {
            const int64_t now = tot[0];
            const int64_t rounds = (now + a.compute_units - 1) / a.compute_units;
            if (now > a.compute_units && rounds <= kFillRounds && now < rounds * a.compute_units) {
                const int64_t limit = rounds * a.compute_units;
                int64_t lo = 1, hi = target;   // items(hi) <= limit; the answer is in [lo, hi]
                if (one_wave) {
                    while (lo < hi) {
                        const int64_t mid = lo + (hi - lo) / 2;
                        const int64_t n = wave_sum(lane < R ? request_items(lane, mid / 4, mid / 5) : 0);
                        if (n <= limit) hi = mid; else lo = mid + 1;
                    }
                } else {
                    while (lo < hi) {
                        const int64_t span = hi - lo;
                        if (wave < kProbeWaves) {
                            const int64_t probe = lo + span * (wave + 1) / (kProbeWaves + 1);   // in [lo, hi)
                            const int64_t q4 = probe / 4, q5 = probe / 5;
                            int64_t n = 0;
                            for (int r = lane; r < R; r += 64) n += request_items(r, q4, q5);
                            n = wave_sum(n);
                            if (lane == 0) {
                                probe_fits[wave] = n <= limit ? 1 : 0;
                                probe_val[wave] = probe;
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
                }
                if (lo != target) chunking(lo);
            }
        }
        if (one_wave && lane < R) write_classes(lane);
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

    // The XCD placement (tv_plan.cpp::place_for_xcds) in step 4.  A stream (request, head
    // group, chunk) holds its request's NB node blocks, adjacent in the sorted order (equal
    // costs, consecutive enumeration indices), so some stream has several items iff some
    // request has NB > 1, and every such run is a multiple of 8 iff every such NB is.  Without
    // such a stream every item's rank is its output row.
    const bool shared = (shape_flag & 1) != 0;
    const bool aligned = (shape_flag & 2) == 0;
    constexpr int kWindow = kXcds * kXcds;
    const int full = shared ? (nitems / kWindow) * kWindow : 0;
    auto position_of = [&](int rank) {
        if (rank >= full) return rank;
        const int w = rank - rank % kWindow;
        const int k = rank - w;
        const int column = (w / kWindow) % 2 ? kXcds - 1 - k / kXcds : k / kXcds;   // odd windows mirrored
        return w + kXcds * (k % kXcds) + column;
    };
    // Rows of 8 int32 go out as two 16-byte stores when both arrays allow it.
    const bool vec_rows = ((reinterpret_cast<uintptr_t>(a.items) | reinterpret_cast<uintptr_t>(a.groups)) & 15) == 0;
    auto store_row = [&](int32_t* dst, const int32_t (&v)[8]) {
        if (vec_rows) {
            reinterpret_cast<int4*>(dst)[0] = make_int4(v[0], v[1], v[2], v[3]);
            reinterpret_cast<int4*>(dst)[1] = make_int4(v[4], v[5], v[6], v[7]);
        } else {
#pragma unroll
            for (int k = 0; k < 8; ++k) dst[k] = v[k];
        }
    };
    // Item (request r, head group hg, chunk c, node block nb) at output row `row`.
    auto write_item = [&](int r, const ReqShape& s, int nc, int hg, int c, int nb, int row) {
        const int64_t p = req_p[r], chunk = req_chunk[r];
        const int32_t out[8] = {
            r,
            hg * s.hpw,
            nb * s.npw,
            static_cast<int32_t>(min(p, c * chunk)),
            static_cast<int32_t>(min(p, (c + 1) * chunk)),
            (c == nc - 1 ? kItemLastChunk : 0) | (nb == s.NB - 1 ? kItemLastBlock : 0) | (QPK << kItemGroupShift),
            nc > 1 ? req_slot_off[r] + (hg * s.NB + nb) * nc + c : -1,
            s.hpw};
        store_row(a.items + static_cast<int64_t>(row) * 8, out);
    };
    // Decode a sorted (request, idx) back into its item and write it at output row `row`.
    auto decode = [&](int sorted_pos, int row) {
        const uint64_t key = keys[sorted_pos];
        const int idx = static_cast<int>(key & 0xffffffffull);
        const int r = static_cast<int>((key >> 32) & 0xffffu);
        const ReqShape s = shape_at(r);
        const int nc = req_nchunks[r];
        int nb, c;
        const int hg = div_small(div_small(idx - req_item_off[r], s.NB, nb), nc, c);
        write_item(r, s, nc, hg, c, nb, row);
    };

    // 3. The items longest first, ties in enumeration order: the host comparator's
    // (~cost, request, head group, chunk, block), the enumeration index
    // idx = item offset + (hg * nchunks + c) * NB + nb being the tie order.  keys[rank] ends
    // up holding (request, idx).
    //
    // A request's items take at most two costs, w * chunk for every chunk but the last and
    // w * (last chunk keys + nodes) for the last, so with at most kClassRankMax / 2 requests
    // the planner ranks those cost classes (2 per request) by counting and writes every item
    // at its class's offset plus its place in the class, in enumeration order: no item sort.
    // Larger batches sort the items' 64-bit keys (bitonic, in LDS and registers).
    const bool class_ranked = 2 * R <= kClassRankMax;
    if (class_ranked) {
        if (!one_wave) {
            for (int r = t; r < R; r += kPlanThreads) write_classes(r);
            __syncthreads();
        }
        // Rank of class c = classes with a smaller key (keys are distinct), counted by
        // `lanes` lanes per class: the largest power of two up to a wave that fits the block.
        const int C = 2 * R;
        int lane_bits = 6;
        while ((C << lane_bits) > kPlanThreads) --lane_bits;
        {
            const int lanes = 1 << lane_bits;
            const int c = t >> lane_bits, q = t & (lanes - 1);
            int below = 0;
            if (c < C) {
                const uint64_t mine = ckey[c];
#pragma unroll 8
                for (int j = q; j < C; j += lanes) below += ckey[j] < mine ? 1 : 0;
            }
            for (int off = 1; off < lanes; off <<= 1) below += __shfl_xor(below, off);
            if (c < C && q == 0) {
                crank[c] = below;
                cstart[below] = ccount[c];
                // A class is single (its items are streams of one item) iff its request has one
                // node block.
                sstart[below] = (req_bits[c >> 1] & 0xfff) == 1 ? ccount[c] : 0;
            }
        }
        __syncthreads();
        // Exclusive scans of the class sizes and single counts in rank order, in wave 0 (four
        // per lane).
        if (t < 64) {
            int v[4], u[4], sum = 0, usum = 0;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                v[i] = 4 * t + i < C ? cstart[4 * t + i] : 0;
                u[i] = 4 * t + i < C ? sstart[4 * t + i] : 0;
                sum += v[i];
                usum += u[i];
            }
            int run = static_cast<int>(wave_inclusive_sum(sum)) - sum;
            const int64_t uincl = wave_inclusive_sum(usum);
            int urun = static_cast<int>(uincl) - usum;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                if (4 * t + i < C) {
                    cstart[4 * t + i] = run;
                    sstart[4 * t + i] = urun;
                }
                run += v[i];
                urun += u[i];
            }
            if (t == 0) class_singles = static_cast<int>(lane_value(uincl, 63));
        }
        __syncthreads();
        const int singles_total = class_singles;
        // The aligned XCD placement of sorted position i (step 4, from the number sb of single
        // items before it and whether it is single): a group item goes ahead of the at most 7
        // singles since the last multiple of 8; single number sb goes after the group items
        // before q, the first position whose singles count rounded down to 8 exceeds sb: q is
        // one past single m - 1, m the next multiple of 8 above sb, or the end when there are
        // not m singles.  Single j lies in the last class (rank order) whose singles start at or
        // below j.
        auto aligned_rank = [&](int i, int sb, bool single) -> int {
            if (!single) return (i - sb) + sb / kXcds * kXcds;
            const int m = (sb / kXcds + 1) * kXcds;
            if (m > singles_total) return sb + (nitems - singles_total);
            const int j = m - 1;
            int lo = 0, hi = C - 1;
            while (lo < hi) {
                const int mid = (lo + hi + 1) >> 1;
                if (sstart[mid] <= j) lo = mid; else hi = mid - 1;
            }
            const int at = cstart[lo] + (j - sstart[lo]);
            return sb + (at + 1 - m);
        };
        // Every item at its class's first position plus its place in the class.
        for (int e = t; e < nitems; e += kPlanThreads) {
            const int r = request_of(e);
            const ReqShape sh = shape_at(r);
            const int nc = req_nchunks[r];
            const int local = e - req_item_off[r];
            int nb, c;
            const int hc = div_small(local, sh.NB, nb);
            const int hg = div_small(hc, nc, c);
            const bool merged = (req_bits[r] & 0x4000) != 0;
            int cls, pos;
            if (nc == 1 || (!merged && c == nc - 1)) {
                cls = 1;
                pos = hg * sh.NB + nb;
            } else if (merged) {
                cls = 0;
                pos = local;
            } else {
                cls = 0;
                pos = (hg * (nc - 1) + c) * sh.NB + nb;
            }
            const int k = crank[2 * r + cls];
            const int i = cstart[k] + pos;   // sorted position
            if (!shared) {
                write_item(r, sh, nc, hg, c, nb, i);
            } else if (aligned) {
                const bool single = sh.NB == 1;
                write_item(r, sh, nc, hg, c, nb, position_of(aligned_rank(i, sstart[k] + (single ? pos : 0), single)));
            } else {
                keys[i] = (static_cast<uint64_t>(r) << 32) | static_cast<uint32_t>(e);
            }
        }
        // Only the windowed placement reads the keys; the other plans are written.
        if (shared && !aligned) __syncthreads();
    } else {
        // 3. Sort keys, one thread per item: (~cost, request, head group, chunk, block), the
        // enumeration index idx = item offset + (hg * nchunks + c) * NB + nb being the tie order.
        int npow = 1;
        while (npow < nitems) npow <<= 1;
        for (int e = t; e < npow; e += kPlanThreads) {
            uint64_t key = ~0ull;
            if (e < nitems) {
                const int r = request_of(e);
                const ReqShape s = shape_at(r);
                const int nc = req_nchunks[r];
                const int local = e - req_item_off[r];
                int nb, c;
                div_small(div_small(local, s.NB, nb), nc, c);
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
        // (~cost, idx) -> (request, idx); each thread rewrites the positions it reads.
        for (int e = t; e < nitems; e += kPlanThreads) {
            const int idx = static_cast<int>(keys[e] & 0xffffffffull);
            keys[e] = (static_cast<uint64_t>(request_of(idx)) << 32) | static_cast<uint32_t>(idx);
        }
        __syncthreads();
    }

    // 4. XCD placement (tv_plan.cpp::place_for_xcds) and output.  The cost-class path wrote
    // the unshared and aligned plans already.
    if (!shared) {
        // Every rank is its position.
        if (!class_ranked) {
            for (int i = t; i < nitems; i += kPlanThreads) decode(i, i);
        }
    } else if (aligned) {
        if (!class_ranked) {
            // Groups ahead of the at most 7 singles before them since the last multiple of
            // 8: ranks from the number of single items (those of one-block requests) before each
            // sorted position, and the position of every single (in the keys' top 16 bits, which
            // decode ignores).  Positions go in 64-position chunks, chunk ch to wave ch % 16: a
            // ballot marks a chunk's singles, every wave scans the chunk counts (at most 128, two
            // per lane), and a single's number is its chunk's prefix plus the singles below it.
            static_assert(kMaxSortItems / 64 <= 128, "two chunk counts per lane");
            uint16_t* single_at = reinterpret_cast<uint16_t*>(keys) + 3;   // [j * 4]: position of single j
            int32_t* chunk_singles = stream_id;                            // [nchunks]
            const int lane = t & 63;
            const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
            const int nchunks = (nitems + 63) / 64;
            const uint64_t below = (uint64_t{1} << lane) - 1;
            uint64_t marks[kPer];
#pragma unroll
            for (int e = 0; e < kPer; ++e) {
                const int ch = wave + e * kPlanWaves;
                marks[e] = 0;
                if (ch < nchunks) {   // wave-uniform
                    const int i = ch * 64 + lane;
                    bool single = false;
                    if (i < nitems) single = (req_bits[static_cast<int>((keys[i] >> 32) & 0xffffu)] & 0xfff) == 1;
                    marks[e] = __ballot(single);
                    if (lane == 0) chunk_singles[ch] = __popcll(marks[e]);
                }
            }
            __syncthreads();
            const int c0 = 2 * lane < nchunks ? chunk_singles[2 * lane] : 0;
            const int c1 = 2 * lane + 1 < nchunks ? chunk_singles[2 * lane + 1] : 0;
            const int64_t pair_end = wave_inclusive_sum(c0 + c1);
            const int singles_total = static_cast<int>(lane_value(pair_end, 63));
            int sbs[kPer];
#pragma unroll
            for (int e = 0; e < kPer; ++e) {
                const int ch = wave + e * kPlanWaves;
                sbs[e] = 0;
                if (ch < nchunks) {   // wave-uniform
                    const int i = ch * 64 + lane;
                    const int owner = ch >> 1;
                    int prefix = static_cast<int>(lane_value(pair_end, owner)) - __builtin_amdgcn_readlane(c0 + c1, owner);
                    if (ch & 1) prefix += __builtin_amdgcn_readlane(c0, owner);
                    sbs[e] = prefix + __popcll(marks[e] & below);
                    if (i < nitems && ((marks[e] >> lane) & 1)) single_at[4 * sbs[e]] = static_cast<uint16_t>(i);
                }
            }
            __syncthreads();
            // Ranks and output.  Single number sb goes after the group items before q, the first
            // position whose singles count rounded down to 8 exceeds sb: q is one past single
            // m - 1, m the next multiple of 8 above sb, or the end when there are not m singles.
#pragma unroll
            for (int e = 0; e < kPer; ++e) {
                const int ch = wave + e * kPlanWaves;
                const int i = ch * 64 + lane;
                if (ch < nchunks && i < nitems) {
                    const int sb = sbs[e];
                    int rank;
                    if (!((marks[e] >> lane) & 1)) {
                        rank = (i - sb) + sb / kXcds * kXcds;
                    } else {
                        const int m = (sb / kXcds + 1) * kXcds;
                        rank = m <= singles_total ? sb + (single_at[4 * (m - 1)] + 1 - m) : sb + (nitems - singles_total);
                    }
                    decode(i, position_of(rank));
                }
            }
        }
    } else {
        // A window is one wave's 64 positions (kWindow == 64, kPlanThreads a multiple of it),
        // so the loop runs per wave and each window ranks by one ballot of its grouped items
        // (those next to an item of the same stream within the window; the neighbours' stream
        // ids come by DPP wave shifts, -1 past the window's ends): a grouped item follows the
        // grouped ones before it, a single one follows every grouped item and the singles
        // before it.
        static_assert(kWindow == 64 && kPlanThreads % kWindow == 0, "one window per wave");
        const int k = t & 63;
        for (int w = t - k; w < nitems; w += kPlanThreads) {   // wave-uniform
            const int i = w + k;
            int rank = i;
            if (w < full) {   // wave-uniform: the whole window lies below full <= nitems
                const uint64_t key = keys[i];
                const int r = static_cast<int>((key >> 32) & 0xffffu);
                int nb;
                const int sid = r * kMaxSortItems +
                                div_small(static_cast<int>(key & 0xffffffffull) - req_item_off[r], req_bits[r] & 0xfff, nb);
                const int prev = __builtin_amdgcn_update_dpp(-1, sid, 0x138, 0xf, 0xf, false);   // wave_shr:1
                const int next = __builtin_amdgcn_update_dpp(-1, sid, 0x130, 0xf, 0xf, false);   // wave_shl:1
                const bool g = prev == sid || next == sid;
                const uint64_t grouped = __ballot(g);
                const uint64_t before = (uint64_t{1} << k) - 1;
                rank = w + (g ? __popcll(grouped & before) : __popcll(grouped) + __popcll(~grouped & before));
            }
            if (i < nitems) decode(i, position_of(rank));
        }
    }
    // Merge groups in (request, head group, block) order with their first partial slot, one
    // per thread (the request: the last one whose first group is at or before it; requests
    // without groups share their successor's offset).
    for (int gi = t; gi < num_groups; gi += kPlanThreads) {
        int lo = 0, hi = R - 1;
        while (lo < hi) {
            const int mid = (lo + hi + 1) >> 1;
            if (req_group_off[mid] <= gi) lo = mid; else hi = mid - 1;
        }
        const int r = lo;
        const ReqShape s = shape_at(r);
        const int nc = req_nchunks[r];
        const int unit = gi - req_group_off[r];   // hg * NB + nb
        int nb;
        const int hg = div_small(unit, s.NB, nb);
        const int32_t out[8] = {r, hg * s.hpw, nb * s.npw, s.hpw, req_slot_off[r] + unit * nc, nc,
                                QPK,   // the grouping the slots' rows are laid out for
                                0};
        store_row(a.groups + static_cast<int64_t>(gi) * 8, out);
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
// adds at most CUs - 1 items.  The chunk count is also ceil(p / c0) with c0 >= 64 keys,
// so items <= blocks * ceil(P_max / 64) as well, which is the smaller bound for short
// prefixes (every surplus workgroup of a capacity grid still takes a CU's LDS for a
// moment).  A forced chunk length gives every node-block group ceil(P_max / chunk) items.
int fill_capacity(int64_t blocks, int32_t max_nodes, int32_t block_size, int32_t num_compute_units,
                  int32_t chunk_keys, int64_t max_prefix, tv_attention_plan_info* info) {
    const int64_t max_chunk = (static_cast<int64_t>(kMaxChunkPages - 1) * block_size) / 32 * 32;
    const int64_t capped = (max_prefix + max_chunk - 1) / max_chunk;
    const int64_t shortest = blocks * std::max<int64_t>(1, (max_prefix + kMinChunkKeys - 1) / kMinChunkKeys);
    const int64_t items = chunk_keys > 0 ? blocks * std::max<int64_t>(1, (max_prefix + chunk_keys - 1) / chunk_keys)
                                         : std::min(2 * static_cast<int64_t>(num_compute_units) + blocks * (1 + capped),
                                                    shortest);
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
