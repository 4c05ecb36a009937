// Host-side work planner for the packed tree-verify attention kernel.
//
// The reference launches one program per (packed query, query head)
// (paged_backend.py:290) or per (4-node block, KV head) (tree_gqa.py:130), and every
// program walks its request's whole prefix.  On MI355X the kernel instead gives a
// 512-thread workgroup 256 score rows that share one K/V stream:
//   NPW (nodes per workgroup)    = (8 / HPW) * (32 / G) for G query heads per KV head,
//   HPW (KV heads per workgroup) = 2 for trees that fit NPW(2) nodes (32 at G = 4), else 1,
// so a KV tile staged in LDS is reused by every (node, query head) row of its group.
// Long prefixes are cut into chunks (split-K) only as far as needed to give every
// compute unit work; items are ordered longest first so the hardware dispatcher's
// greedy assignment balances ragged contexts (an LPT schedule).  When that chunking
// leaves a few rounds of items with the last round part-empty (more items than compute
// units, at most kFillRounds rounds), the chunk target is lowered to the smallest
// value whose item count still fits the same number of full rounds, so the rounds
// fill with smaller, more even chunks.
#include <stdint.h>

#include <algorithm>
#include <vector>

#include "tv_internal.h"

namespace tv {
namespace {

constexpr int kItemInts = 8;
constexpr int kRowsPerItem = 256;   // score rows of one workgroup
constexpr int kHeadDim = 128;
constexpr int kMinChunkKeys = 64;   // shortest prefix chunk worth a partial result
constexpr int kMaxChunkPages = 512; // page numbers a workgroup caches in LDS
constexpr int kMaxSlotChunk = 2048; // prefix slots a workgroup caches in LDS (slot addressing)
constexpr int kMaxTreeNodes = 2048; // tree slots a workgroup caches in LDS (page-table prefixes)
constexpr int kMaxTreeNodesSlots = 1024;   // ... beside a slot-addressed prefix chunk
constexpr int64_t kFillRounds = 4;  // item rounds the chunk target is refitted for

struct Item {
    int32_t r, h0, n0, kbeg, kend, flags, slot, hpw;
    int64_t cost;
    int32_t hg, chunk, nb;
};

// A wave owns 32 score rows = floor(32 / qpk) nodes x qpk query heads (plus padding rows
// when qpk does not divide 32), so a workgroup of 8 waves holds (8 / hpw) * floor(32 / qpk)
// nodes of each of its hpw KV heads; trees that fit the two-head form (<= 32 nodes at
// qpk 4) take it.
int nodes_per_item(int hpw, int32_t qpk) { return (8 / hpw) * (32 / qpk); }

bool supported_group(int32_t qpk) { return (qpk >= 1 && qpk <= 8) || qpk == 16; }

int heads_per_group(int32_t nodes, int32_t kv_heads, int32_t qpk) {
    int h = nodes <= nodes_per_item(2, qpk) ? 2 : 1;
    while (h > 1 && h > kv_heads) h >>= 1;
    return h;
}

int64_t round_up(int64_t x, int64_t m) { return (x + m - 1) / m * m; }

// Cost of one key of a work item in quarter key-steps of a one-head item.  A two-head
// item stages both heads' K/V but every wave still runs one head's 16 MFMAs per tile,
// so a tile costs it ~1.25x a one-head tile, not 2x (per-workgroup timestamps: 1.30 vs
// 1.03 us per tile on the mixed batch of config 5).  Weighting by the head count left
// two-head chunks at half the length of one-head chunks of the same cost.
int64_t cost_weight(int hpw) { return hpw == 2 ? 5 : 4; }

// A tree tile takes the general loop (ancestor masks, per-key slot addresses) and costs
// about two prefix tiles (per-workgroup timestamps on config 2: 16.3 us for the last-chunk
// items of 64-node trees, 11 prefix tiles + 2 tree tiles, against 13.2 us for 12 prefix
// tiles).  The chunk lengths of a split prefix are set so that the last chunk, which also
// walks the tree, ends level with the others: the prefix is cut as if it held this many
// keys per tree node more, within the same number of chunks.
constexpr int64_t kTreeKeyWeight = 2;

// MI355X dispatches workgroup i of a launch to XCD i % 8, and each XCD has its own L2.
// The node blocks of one (request, head group, prefix chunk) stream the same K/V, and
// in longest-first order they sit next to each other, so they would land on different
// XCDs and each XCD would pull that K/V from HBM.  Items are therefore given ranks in
// which such groups are whole blocks of 8, and every window of 64 ranks is laid out
// column-major (rank i -> position 8 * (i % 8) + i / 8), so 8 consecutive ranks share an
// XCD and are dispatched together; a partial last window keeps its ranks as positions.
// Odd windows mirror the columns (rank i -> XCD 7 - i / 8): the first column of a window
// holds its longest items, and always giving it to XCD 0 overloaded XCD 0 by a few
// percent over a launch.
//   * When every group has a multiple of 8 items (trees of 512 or 1024 nodes among
//     one-block trees), each group moves ahead of the at most 7 single items that
//     precede it since the last multiple of 8: group items get rank (group items
//     before) + 8 * floor(singles before / 8), and the j-th single moves behind every
//     group so moved, which makes every group a run of whole 8-rank blocks.
//   * Otherwise, within every window of 64 items the items of multi-block groups are
//     taken first (keeping their order); a group that straddles two windows is split.
// Batches without multi-block groups keep the plain longest-first order.
constexpr int kXcds = 8;

void place_for_xcds(std::vector<Item>& items) {
    constexpr size_t kWindow = kXcds * kXcds;
    const size_t n = items.size();
    auto same_stream = [&](size_t i, size_t j) {
        return items[i].r == items[j].r && items[i].hg == items[j].hg && items[i].chunk == items[j].chunk;
    };
    bool shared = false, aligned = true;
    for (size_t i = 0; i < n;) {
        size_t j = i + 1;
        while (j < n && same_stream(i, j)) ++j;
        if (j - i > 1) {
            shared = true;
            aligned = aligned && (j - i) % kXcds == 0;
        }
        i = j;
    }
    if (!shared) return;
    std::vector<Item> ranked(n);
    if (aligned) {
        std::vector<int64_t> singles_before(n + 1, 0);
        std::vector<char> single(n);
        for (size_t i = 0; i < n; ++i) {
            single[i] = !((i > 0 && same_stream(i - 1, i)) || (i + 1 < n && same_stream(i, i + 1)));
            singles_before[i + 1] = singles_before[i] + single[i];
        }
        auto floor8 = [](int64_t x) { return x / kXcds * kXcds; };
        for (size_t i = 0; i < n; ++i) {
            const int64_t sb = singles_before[i];
            int64_t rank;
            if (!single[i]) {
                rank = (static_cast<int64_t>(i) - sb) + floor8(sb);
            } else {
                // p = first position whose rounded singles count exceeds this single's index;
                // the group items before p are exactly the ones moved ahead of it.
                size_t lo = i + 1, hi = n;
                while (lo < hi) {
                    const size_t mid = (lo + hi) / 2;
                    if (floor8(singles_before[mid]) > sb) hi = mid; else lo = mid + 1;
                }
                rank = sb + (static_cast<int64_t>(lo) - singles_before[lo]);
            }
            ranked[static_cast<size_t>(rank)] = items[i];
        }
    } else {
        ranked = items;
        std::vector<Item> window;
        for (size_t w = 0; w + kWindow <= n; w += kWindow) {
            window.assign(items.begin() + w, items.begin() + w + kWindow);
            auto in_group = [&](size_t i) {
                const Item& x = window[i];
                auto same = [&](size_t j) {
                    return j < kWindow && window[j].r == x.r && window[j].hg == x.hg && window[j].chunk == x.chunk;
                };
                return same(i + 1) || (i > 0 && same(i - 1));
            };
            size_t k = w;
            for (size_t i = 0; i < kWindow; ++i) {
                if (in_group(i)) ranked[k++] = window[i];
            }
            for (size_t i = 0; i < kWindow; ++i) {
                if (!in_group(i)) ranked[k++] = window[i];
            }
        }
    }
    const size_t full = n / kWindow * kWindow;
    for (size_t i = 0; i < n; ++i) {
        const size_t w = i - i % kWindow, k = i - w;
        const size_t column = (w / kWindow) % 2 ? kXcds - 1 - k / kXcds : k / kXcds;
        items[i < full ? w + kXcds * (k % kXcds) + column : i] = ranked[i];
    }
}

// The plan for chunks of at most max_chunk keys (a multiple of 32).
int plan(const int32_t* prefix_lens_host, const int32_t* node_counts_host, int32_t num_requests,
         int32_t num_kv_heads, int32_t qpk, int32_t num_compute_units, int32_t chunk_keys, int64_t max_chunk,
         int32_t max_tree_nodes, int32_t* items_host, int32_t* groups_host, tv_attention_plan_info* info) {
    if (!info || !prefix_lens_host || !node_counts_host) return fail(TV_ERR_INVALID, "plan: null argument");
    if (num_requests < 1) return fail(TV_ERR_INVALID, "plan: at least one request is required");
    if (num_kv_heads < 1) return fail(TV_ERR_INVALID, "plan: num_kv_heads must be positive");
    if (!supported_group(qpk)) {
        return fail(TV_ERR_UNSUPPORTED, "plan: %d query heads per KV head (implemented: 1 to 8 or 16)", qpk);
    }
    if (num_compute_units < 1) return fail(TV_ERR_INVALID, "plan: num_compute_units must be positive");
    if (chunk_keys < 0 || chunk_keys % 32) {
        return fail(TV_ERR_INVALID, "plan: chunk_keys %d must be a non-negative multiple of 32", chunk_keys);
    }
    int32_t max_nodes = 1;
    int64_t total_cost = 0;
    for (int32_t r = 0; r < num_requests; ++r) {
        const int32_t p = prefix_lens_host[r], t = node_counts_host[r];
        if (p < 0) return fail(TV_ERR_INVALID, "plan: negative prefix length for request %d", r);
        if (t < 1) return fail(TV_ERR_INVALID, "plan: request %d has no tree nodes", r);
        if (t > max_tree_nodes) {
            return fail(TV_ERR_UNSUPPORTED, "plan: request %d has %d tree nodes (at most %d per request)", r, t,
                        max_tree_nodes);
        }
        max_nodes = std::max(max_nodes, t);
        const int hpw = heads_per_group(t, num_kv_heads, qpk);
        const int npw = nodes_per_item(hpw, qpk);
        const int64_t groups = (num_kv_heads + hpw - 1) / hpw;
        const int64_t blocks = (t + npw - 1) / npw;
        total_cost += groups * blocks * cost_weight(hpw) * (static_cast<int64_t>(p) + t);
    }
    const int64_t target = std::max<int64_t>(kMinChunkKeys, total_cost / num_compute_units);
    if (chunk_keys > max_chunk) {
        return fail(TV_ERR_INVALID, "plan: chunk_keys %d exceeds %lld", chunk_keys, (long long)max_chunk);
    }

    // Chunk length of a prefix of p keys before a tree of t nodes (hpw heads per item) for
    // chunk target `tau` (in cost units): the longest multiple of 32 keys whose cost is not
    // above tau gives the chunk count; the chunks then share the prefix and the tree's
    // weight (kTreeKeyWeight keys a node) evenly, in multiples of 32 keys, as far as that
    // keeps the chunk count (the chunks before the last stay below the prefix) and the cap.
    auto chunk_for = [&](int64_t p, int64_t t, int hpw, int64_t tau) -> int64_t {
        int64_t chunk = std::min(round_up(std::max<int64_t>(kMinChunkKeys, tau / cost_weight(hpw)), 32), max_chunk);
        const int64_t nchunks = p > 0 ? (p + chunk - 1) / chunk : 1;
        chunk = round_up((p + nchunks - 1) / std::max<int64_t>(nchunks, 1), 32);
        if (nchunks > 1) {
            const int64_t even = round_up((p + kTreeKeyWeight * t + nchunks - 1) / nchunks, 32);
            const int64_t keep = std::min((p - 1) / (nchunks - 1) / 32 * 32, max_chunk);
            chunk = std::max(chunk, std::min(even, keep));
        }
        return chunk < 32 ? 32 : chunk;
    };
    auto items_for = [&](int64_t tau) -> int64_t {
        int64_t n = 0;
        for (int32_t r = 0; r < num_requests; ++r) {
            const int64_t p = prefix_lens_host[r];
            const int hpw = heads_per_group(node_counts_host[r], num_kv_heads, qpk);
            const int npw = nodes_per_item(hpw, qpk);
            const int64_t units = static_cast<int64_t>((num_kv_heads + hpw - 1) / hpw) * ((node_counts_host[r] + npw - 1) / npw);
            const int64_t chunk = chunk_for(p, node_counts_host[r], hpw, tau);
            n += units * (p > 0 ? (p + chunk - 1) / chunk : 1);
        }
        return n;
    };
    int64_t tau = target;
    if (chunk_keys == 0) {
        const int64_t now = items_for(target);
        const int64_t rounds = (now + num_compute_units - 1) / num_compute_units;
        // Rounds already full: every smaller target that keeps the item count keeps every
        // request's chunk count (each is non-increasing in the target), so the plan is this one.
        if (now > num_compute_units && rounds <= kFillRounds && now < rounds * num_compute_units) {
            int64_t lo = 1, hi = target;   // items_for(hi) fits `rounds` full rounds
            while (lo < hi) {
                const int64_t mid = lo + (hi - lo) / 2;
                if (items_for(mid) <= rounds * num_compute_units) hi = mid; else lo = mid + 1;
            }
            tau = lo;
        }
    }

    std::vector<Item> items;
    int32_t num_slots = 0, num_groups = 0;
    for (int32_t r = 0; r < num_requests; ++r) {
        const int32_t p = prefix_lens_host[r], t = node_counts_host[r];
        const int hpw = heads_per_group(t, num_kv_heads, qpk);
        const int npw = nodes_per_item(hpw, qpk);
        const int32_t groups = (num_kv_heads + hpw - 1) / hpw;
        const int32_t blocks = (t + npw - 1) / npw;
        const int64_t chunk = chunk_keys > 0 ? chunk_keys : chunk_for(p, t, hpw, tau);
        const int32_t nchunks = p > 0 ? static_cast<int32_t>((p + chunk - 1) / chunk) : 1;
        for (int32_t hg = 0; hg < groups; ++hg) {
            for (int32_t nb = 0; nb < blocks; ++nb) {
                const int32_t first_slot = nchunks > 1 ? num_slots : -1;
                for (int32_t c = 0; c < nchunks; ++c) {
                    Item it;
                    it.r = r;
                    it.h0 = hg * hpw;
                    it.n0 = nb * npw;
                    it.kbeg = static_cast<int32_t>(std::min<int64_t>(p, c * chunk));
                    it.kend = static_cast<int32_t>(std::min<int64_t>(p, (c + 1) * chunk));
                    it.flags = ((c == nchunks - 1) ? kItemLastChunk : 0) | ((nb == blocks - 1) ? kItemLastBlock : 0) |
                               (qpk << kItemGroupShift);
                    it.slot = nchunks > 1 ? first_slot + c : -1;
                    it.hpw = hpw;
                    // Node blocks of one (request, head group, chunk) share their K/V
                    // stream, so they get equal cost and stay adjacent after sorting.
                    it.cost = cost_weight(hpw) * ((it.kend - it.kbeg) + ((it.flags & kItemLastChunk) ? t : 0));
                    it.hg = hg;
                    it.chunk = c;
                    it.nb = nb;
                    items.push_back(it);
                }
                if (nchunks > 1) {
                    if (groups_host) {
                        int32_t* gr = groups_host + kItemInts * num_groups;
                        gr[0] = r;
                        gr[1] = hg * hpw;
                        gr[2] = nb * npw;
                        gr[3] = hpw;
                        gr[4] = first_slot;
                        gr[5] = nchunks;
                        gr[6] = qpk;   // the grouping the slots' rows are laid out for
                        gr[7] = 0;
                    }
                    num_slots += nchunks;
                    ++num_groups;
                }
            }
        }
    }
    std::stable_sort(items.begin(), items.end(), [](const Item& a, const Item& b) {
        if (a.cost != b.cost) return a.cost > b.cost;
        if (a.r != b.r) return a.r < b.r;
        if (a.hg != b.hg) return a.hg < b.hg;
        if (a.chunk != b.chunk) return a.chunk < b.chunk;
        return a.nb < b.nb;
    });
    place_for_xcds(items);
    if (items_host) {
        for (size_t i = 0; i < items.size(); ++i) {
            int32_t* o = items_host + kItemInts * i;
            o[0] = items[i].r;
            o[1] = items[i].h0;
            o[2] = items[i].n0;
            o[3] = items[i].kbeg;
            o[4] = items[i].kend;
            o[5] = items[i].flags;
            o[6] = items[i].slot;
            o[7] = items[i].hpw;
        }
    }
    info->num_items = static_cast<int32_t>(items.size());
    info->num_groups = num_groups;
    info->num_partial_slots = num_slots;
    info->ancestor_words_per_row = (max_nodes + 63) / 64;
    const int64_t o_bytes = static_cast<int64_t>(num_slots) * kRowsPerItem * kHeadDim * 4;
    const int64_t ml_bytes = static_cast<int64_t>(num_slots) * kRowsPerItem * 8;
    info->workspace_bytes = num_slots ? round_up(o_bytes, 256) + round_up(ml_bytes, 256) : 0;
    return TV_OK;
}

}  // namespace
}  // namespace tv

using namespace tv;

extern "C" int tv_tree_attention_plan(const int32_t* prefix_lens_host, const int32_t* node_counts_host,
                                      int32_t num_requests, int32_t num_kv_heads, int32_t queries_per_kv,
                                      int32_t block_size,
                                      int32_t num_compute_units, int32_t chunk_keys, int32_t* items_host,
                                      int32_t* groups_host, tv_attention_plan_info* info) {
    clear_error();
    if (block_size < 32 || block_size % 32) {
        return fail(TV_ERR_UNSUPPORTED, "plan: block_size %d is not a positive multiple of 32", block_size);
    }
    // Longest chunk whose pages fit the LDS page cache wherever it starts.
    const int64_t max_chunk = (static_cast<int64_t>(kMaxChunkPages - 1) * block_size) / 32 * 32;
    return plan(prefix_lens_host, node_counts_host, num_requests, num_kv_heads, queries_per_kv, num_compute_units,
                chunk_keys, max_chunk, kMaxTreeNodes, items_host, groups_host, info);
}

extern "C" int tv_tree_attention_plan_slots(const int32_t* prefix_lens_host, const int32_t* node_counts_host,
                                            int32_t num_requests, int32_t num_kv_heads, int32_t queries_per_kv,
                                            int32_t num_compute_units,
                                            int32_t chunk_keys, int32_t* items_host, int32_t* groups_host,
                                            tv_attention_plan_info* info) {
    clear_error();
    return plan(prefix_lens_host, node_counts_host, num_requests, num_kv_heads, queries_per_kv, num_compute_units,
                chunk_keys, kMaxSlotChunk, kMaxTreeNodesSlots, items_host, groups_host, info);
}
