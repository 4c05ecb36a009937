// Tree attention entry points (include/treeverify.h): argument checks, the merge of
// split-prefix partials, the ancestor-word packing, and the allocation-free variant.
// The attention kernel itself lives in tv_attention_kernel.h (instantiated per query
// group size in tv_attention_g<G>.hip).
#include <math.h>
#include <stdint.h>

#include <algorithm>
#include <mutex>

#include "tv_attention.h"

namespace tv {
namespace {

// Combines the split-K partials of one (request, head group, node block).  Grid
// (groups, 32): workgroup y takes score rows 8y..8y+7 of the group, one thread per
// (row, 16-byte quad of the head dimension), so the partial loads of all rows are in
// flight at once.  Each partial holds O unnormalised against its own reference
// maximum m_s with sum l_s: the result is sum_s w_s O_s / sum_s w_s l_s with
// w_s = 2^((m_s - max m) * c).
template <typename T>
__device__ __forceinline__ void merge_group(const AttnParams& p, int group) {
    const int32_t* gr = p.groups + 8 * static_cast<int64_t>(group);
    // The group record is the same for the whole workgroup: scalar registers.
    const int r = __builtin_amdgcn_readfirstlane(gr[0]), h0 = __builtin_amdgcn_readfirstlane(gr[1]);
    const int n0 = __builtin_amdgcn_readfirstlane(gr[2]), hpw = __builtin_amdgcn_readfirstlane(gr[3]);
    const int first = __builtin_amdgcn_readfirstlane(gr[4]), ns = __builtin_amdgcn_readfirstlane(gr[5]);
    if (r < 0 || r >= p.num_requests || h0 < 0 || n0 < 0 || (hpw != 1 && hpw != 2) || first < 0 || ns < 1 ||
        first > p.num_slots - ns || gr[6] != p.qpk) {
        if (blockIdx.y == 0 && threadIdx.x == 0) set_status(p.status, TV_STATUS_BAD_REQUEST);
        return;
    }
    const int wph = 8 / hpw;
    const int G = p.qpk, nw = 32 / G;   // query heads per KV head, nodes per wave (floor)
    const int wr = 8 * blockIdx.y + (threadIdx.x >> 5), quad = threadIdx.x & 31;
    const int wave = wr >> 5, c = wr & 31;
    const int hl = wave / wph;
    const int head = h0 + hl;
    const int node = n0 + nw * (wave - hl * wph) + c / G;
    const int qh = head * G + c % G;
    // Every partial of a row is loaded together, 8 partials at a time, with the running
    // maximum rescaled between batches.  Up to 8 partials this is the plain maximum-then-sum.
    // Partial s of this thread's row sits at the group's base plus s partial strides plus
    // the row's own offset: the bases are wave-uniform (scalar registers) and the row
    // offsets 32-bit, so the addresses of the 8 partials in flight cost few vector
    // registers.  With a 64-bit vector address per partial the merge took 125 registers,
    // 4 waves per SIMD (config 2: 10.1 us); this form takes 79 and 6 waves (9.1 us).
    const int D = p.head_dim;
    const uint64_t ml_step = static_cast<uint64_t>(kRowsPerItem) * sizeof(float2);
    const uint64_t o_step = static_cast<uint64_t>(kRowsPerItem) * D * sizeof(float);
    const char* ml_base = reinterpret_cast<const char*>(p.ws_ml) + static_cast<uint64_t>(first) * ml_step;
    const char* o_base = reinterpret_cast<const char*>(p.ws_o) + static_cast<uint64_t>(first) * o_step;
    const uint32_t ml_off = static_cast<uint32_t>(wr) * sizeof(float2);
    const uint32_t o_row = static_cast<uint32_t>(wr * D) * sizeof(float);
    const int tn = __builtin_amdgcn_readfirstlane(p.cnt[r]), qbase = __builtin_amdgcn_readfirstlane(p.cu[r]);
    if (qbase < 0 || tn < 0 || tn > p.total_queries - qbase) {   // rows outside the packed batch
        if (blockIdx.y == 0 && threadIdx.x == 0) set_status(p.status, TV_STATUS_BAD_REQUEST);
        return;
    }
    const bool row_ok = head < p.num_kv_heads && node < tn && c < nw * G;   // c >= nw * G: padding row
    // Rows past the tree (or padding) were never written and are not stored: no loads.  A
    // 16-node tree leaves 3 of every 4 rows of its 64-node block empty.
    if (!row_ok) return;
    // Partial rows are D floats apart.  A thread merges dims 4*quad..4*quad+3 and, at head
    // size 256, the same 128 dims further; quads past D / 4 (head size 64) have none.
#pragma unroll 1
    for (int d4 = 4 * quad; d4 < D; d4 += 128) {
        const uint32_t po_off = o_row + static_cast<uint32_t>(d4) * sizeof(float);
        float m = -INFINITY, l = 0.f;
        f32x4 o = {0.f, 0.f, 0.f, 0.f};
        for (int s0 = 0; s0 < ns; s0 += 8) {
            float2 part[8];
            f32x4 po4[8];
#pragma unroll
            for (int k = 0; k < 8; ++k) {
                if (s0 + k < ns) {
                    const uint64_t s = static_cast<uint64_t>(s0 + k);
                    part[k] = *reinterpret_cast<const float2*>(ml_base + s * ml_step + ml_off);
                    po4[k] = *reinterpret_cast<const f32x4*>(o_base + s * o_step + po_off);
                } else {
                    part[k] = make_float2(-INFINITY, 0.f);
                    po4[k] = f32x4{0.f, 0.f, 0.f, 0.f};
                }
            }
            float mb = m;
#pragma unroll
            for (int k = 0; k < 8; ++k) mb = fmaxf(mb, part[k].x);
            const float mc = (mb == -INFINITY ? 0.f : mb) * p.c;
            if (m != -INFINITY) {
                const float keep = __builtin_amdgcn_exp2f(m * p.c - mc);
                l *= keep;
                o *= keep;
            }
#pragma unroll
            for (int k = 0; k < 8; ++k) {
                if (s0 + k < ns) {
                    const float w = __builtin_amdgcn_exp2f(part[k].x * p.c - mc);
                    l += part[k].y * w;
                    o += po4[k] * w;
                }
            }
            m = mb;
        }
        store_out4<T>(p, qbase + node, qh, d4, o * (1.f / l));
    }
}

// Grid (groups, 32) for a host plan.  A device-built plan (graph capture) launches at most
// kMergeGridCap workgroup columns and the columns loop over the live group count, so a
// signature-wide group capacity costs no flood of empty workgroups.
constexpr int kMergeGridCap = 128;

template <typename T>
__global__ void __launch_bounds__(256)
merge_partials_kernel(const AttnParams p) {
    const int count = p.counts ? p.counts[1] : static_cast<int>(gridDim.x);
    for (int group = blockIdx.x; group < count; group += gridDim.x) merge_group<T>(p, group);
}

// One wave per row of the ancestor bits.  Row i of a tree of tn nodes carries bits for its
// elements m <= i; word w is the ballot of the zeros among elements 64w..64w+63, which the
// wave's lanes read with one coalesced 256-byte load (indices clamped into the row's first
// i + 1 elements, so nothing past the node is read).  A wave issues the loads of up to
// kPackBatch words before their ballots and writes every word of its row, zeros past the
// node.  Any element at or before the node that is neither 0 nor -inf sets
// TV_STATUS_BAD_BIAS.  (One wave per word made as many waves as words, each waiting out its
// own chain of dependent loads; one thread per word read 64 scattered rows per load.)
constexpr int kPackWaves = 4;   // rows per 256-thread workgroup
constexpr int kPackBatch = 8;   // words whose loads a wave issues together

__global__ void __launch_bounds__(64 * kPackWaves)
pack_ancestor_kernel(const float* __restrict__ bias, const int64_t* __restrict__ bias_off,
                     const int32_t* __restrict__ q2r, const int32_t* __restrict__ local,
                     const int32_t* __restrict__ counts, int32_t total_q, int32_t num_requests, int32_t words,
                     uint64_t* __restrict__ out, int32_t* status) {
    const int lane = threadIdx.x & 63;
    const int64_t q = static_cast<int64_t>(blockIdx.x) * kPackWaves + (threadIdx.x >> 6);   // wave-uniform
    if (q >= total_q) return;
    const int r = q2r[q];
    int lim = 0;   // elements of the row that carry bits
    const float* row = bias;
    if (r < 0 || r >= num_requests) {
        if (lane == 0) set_status(status, TV_STATUS_BAD_REQUEST);
    } else {
        const int i = local[q];
        const int tn = counts[r];
        if (i >= 0 && i < tn) {
            lim = i + 1;
            row = bias + bias_off[r] + static_cast<int64_t>(i) * tn;
        } else if (lane == 0) {
            set_status(status, TV_STATUS_BAD_REQUEST);
        }
    }
    const int used = (lim + 63) / 64;   // words with an element that carries a bit
    uint64_t* row_out = out + q * words;
    bool other = false;   // a value bits cannot carry
    for (int w0 = 0; w0 < words; w0 += kPackBatch) {
        float x[kPackBatch];
#pragma unroll
        for (int k = 0; k < kPackBatch; ++k) {
            x[k] = w0 + k < used ? row[min(64 * (w0 + k) + lane, lim - 1)] : -INFINITY;
        }
        uint64_t mine = 0;   // lane k keeps word w0 + k
#pragma unroll
        for (int k = 0; k < kPackBatch; ++k) {
            const bool in = 64 * (w0 + k) + lane < lim;
            const uint64_t bits = __ballot(in && x[k] == 0.f);
            other |= in && x[k] != 0.f && x[k] != -INFINITY;
            if (lane == k) mine = bits;
        }
        if (lane < kPackBatch && w0 + lane < words) row_out[w0 + lane] = mine;
    }
    if (__ballot(other) && lane == 0) set_status(status, TV_STATUS_BAD_BIAS);
}

}  // namespace
}  // namespace tv

using namespace tv;

extern "C" int tv_pack_ancestor_words(const float* qq_bias, const int64_t* qq_bias_offsets,
                                      const int32_t* query_to_request, const int32_t* query_local_row,
                                      const int32_t* node_counts, int32_t total_queries, int32_t num_requests,
                                      int32_t words_per_row, uint64_t* words, int32_t* status, void* stream) {
    clear_error();
    if (total_queries < 0 || num_requests < 1 || words_per_row < 1) {
        return fail(TV_ERR_INVALID, "pack_ancestor_words: invalid sizes");
    }
    if (total_queries == 0) return TV_OK;
    if (!qq_bias || !qq_bias_offsets || !query_to_request || !query_local_row || !node_counts || !words) {
        return fail(TV_ERR_INVALID, "pack_ancestor_words: null pointer");
    }
    const int64_t blocks = (static_cast<int64_t>(total_queries) + kPackWaves - 1) / kPackWaves;
    hipLaunchKernelGGL(pack_ancestor_kernel, dim3(static_cast<uint32_t>(blocks)), dim3(64 * kPackWaves), 0,
                       as_stream(stream), qq_bias,
                       qq_bias_offsets, query_to_request, query_local_row, node_counts, total_queries,
                       num_requests, words_per_row, words, status);
    return check_launch("pack_ancestor_words");
}

// Scratch of the allocation-free entry (tv_tree_attention_noalloc): one array per device,
// held until the process ends.  Its host-side name is only a stand-in; the device address
// comes from hipGetSymbolAddress, taken once per device with that device current.
constexpr int64_t kScratchBytes = int64_t{64} << 20;
static __device__ __align__(256) char scratch[kScratchBytes];

namespace {

// Split-K workspace of `slots` partial slots: partial O (256 rows of max(D, 128) floats per
// slot, so head sizes up to 128 share one size), then (max, sum) per row.
int64_t partial_o_span(int64_t slots, int32_t head_dim) {
    const int64_t row = head_dim > kHeadDim ? head_dim : kHeadDim;
    return slots > 0 ? (slots * kRowsPerItem * row * 4 + 255) / 256 * 256 : 0;
}
int64_t workspace_need(int64_t slots, int32_t head_dim) {
    if (slots <= 0) return 0;
    return partial_o_span(slots, head_dim) + (slots * kRowsPerItem * 8 + 255) / 256 * 256;
}

// Validates `a` and enqueues the attention (and the merge of split prefixes) with the
// partial-result workspace that `a` names.
int launch_tree_attention(const tv_tree_attention_args* a, void* stream) {
    if (!a) return fail(TV_ERR_INVALID, "tree_attention: null args");
    const int32_t qpk = a->num_kv_heads >= 1 && a->num_q_heads % a->num_kv_heads == 0
                            ? a->num_q_heads / a->num_kv_heads : 0;
    if (!((qpk >= 1 && qpk <= 8) || qpk == 16)) {
        return fail(TV_ERR_UNSUPPORTED,
                    "tree_attention: %d query heads over %d KV heads (implemented: 1 to 8 or 16 per KV head)",
                    a->num_q_heads, a->num_kv_heads);
    }
    const bool pow2_group = (qpk & (qpk - 1)) == 0;
    if (!(a->head_dim == 128 || ((a->head_dim == 64 || a->head_dim == 256) && pow2_group))) {
        return fail(TV_ERR_UNSUPPORTED,
                    "tree_attention: head_dim %d with %d query heads per KV head (implemented: 128, or 64 and 256 "
                    "with 1, 2, 4, 8 or 16)", a->head_dim, qpk);
    }
    if (a->prefix_slots ? a->block_size < 1 : (a->block_size < 32 || a->block_size % 32)) {
        return fail(TV_ERR_UNSUPPORTED, "tree_attention: block_size %d is not a multiple of 32", a->block_size);
    }
    if (a->prefix_slots && a->prefix_slots_stride < 0) {
        return fail(TV_ERR_INVALID, "tree_attention: negative prefix slot stride");
    }
    if (a->prefix_slots && !a->exact_probabilities) {
        return fail(TV_ERR_UNSUPPORTED, "tree_attention: slot-addressed prefixes run with exact probabilities");
    }
    // The online softmax orders scores by their value times the scale.
    if (!(a->scale > 0.f) || !isfinite(a->scale)) {
        return fail(TV_ERR_UNSUPPORTED, "tree_attention: softmax scale must be positive and finite");
    }
    if (a->in_dtype != TV_BF16 && a->in_dtype != TV_F16) {
        return fail(TV_ERR_UNSUPPORTED, "tree_attention: operands must be bf16 or f16");
    }
    if (a->out_dtype != a->in_dtype && a->out_dtype != TV_F32) {
        return fail(TV_ERR_INVALID, "tree_attention: output dtype must match the operands or be f32");
    }
    if (a->k_stride[3] != 1 || a->v_stride[3] != 1) {
        return fail(TV_ERR_UNSUPPORTED, "tree_attention: K/V head dim must be contiguous");
    }
    const int64_t* ks = a->k_stride;
    const int64_t* vs = a->v_stride;
    if ((ks[0] | ks[1] | ks[2] | vs[0] | vs[1] | vs[2]) % 8 || (a->q_stride_row | a->q_stride_head) % 8 ||
        !aligned(a->q, 16) || !aligned(a->k_pool, 16) || !aligned(a->v_pool, 16)) {
        return fail(TV_ERR_UNSUPPORTED, "tree_attention: Q/K/V rows must be 16-byte aligned");
    }
    // Tiles are addressed as page base + per-lane byte offset of up to 31 key rows, with
    // 32-bit page and key-row byte strides; the streaming loop also adds the step to the
    // group's second KV head to that 32-bit lane offset.
    if (ks[0] < 0 || vs[0] < 0 || ks[1] < 0 || vs[1] < 0 || ks[2] < 0 || vs[2] < 0 ||
        ks[0] * 2 >= (int64_t{1} << 32) || vs[0] * 2 >= (int64_t{1} << 32) ||
        ks[1] * 2 * kTileKeys >= (int64_t{1} << 31) || vs[1] * 2 * kTileKeys >= (int64_t{1} << 31) ||
        ks[2] * 2 >= (int64_t{1} << 31) || vs[2] * 2 >= (int64_t{1} << 31)) {
        return fail(TV_ERR_UNSUPPORTED, "tree_attention: K/V strides out of range");
    }
    if (a->ancestor_words_per_row < 1 || a->ancestor_words_per_row > kMaxTreeNodes / 64) {
        return fail(TV_ERR_INVALID, "tree_attention: ancestor_words_per_row %d out of range",
                    a->ancestor_words_per_row);
    }
    const int out_elem = a->out_dtype == TV_F32 ? 4 : 2;
    if ((a->out_stride_row | a->out_stride_head) % (16 / out_elem) || !aligned(a->out, 16)) {
        return fail(TV_ERR_UNSUPPORTED, "tree_attention: output rows must be 16-byte aligned");
    }
    if (a->num_requests < 1 || a->total_queries < 0 || a->num_items < 0 || a->num_groups < 0 ||
        a->num_partial_slots < 0) {
        return fail(TV_ERR_INVALID, "tree_attention: invalid counts");
    }
    // Tree slots are cached as 32-bit values.
    if (a->num_blocks < 0 || a->num_blocks * a->block_size >= (int64_t{1} << 31)) {
        return fail(TV_ERR_UNSUPPORTED, "tree_attention: %lld pool pages of %d slots (at most 2^31 slots)",
                    (long long)a->num_blocks, a->block_size);
    }
    if (a->num_items == 0) return TV_OK;
    if (!a->q || !a->k_pool || !a->v_pool || !a->out || !a->cu_seqlens_q || !a->prefix_lens || !a->node_counts ||
        !a->block_tables || !a->tree_slots || !a->ancestor_words || !a->items) {
        return fail(TV_ERR_INVALID, "tree_attention: null pointer");
    }
    const int64_t o_span = partial_o_span(a->num_partial_slots, a->head_dim);
    const int64_t need = workspace_need(a->num_partial_slots, a->head_dim);
    if ((a->num_groups > 0 && !a->groups) || (a->num_partial_slots > 0 && !a->workspace)) {
        return fail(TV_ERR_INVALID, "tree_attention: split plan without groups/workspace");
    }
    if (a->workspace_bytes < need) {
        return fail(TV_ERR_CAPACITY, "tree_attention: workspace %lld < %lld bytes", (long long)a->workspace_bytes,
                    (long long)need);
    }
    AttnParams p;
    p.q = a->q;
    p.q_s0 = a->q_stride_row;
    p.q_s1 = a->q_stride_head;
    p.k = a->k_pool;
    p.v = a->v_pool;
    p.k_s0 = ks[0];
    p.k_s1 = ks[1];
    p.k_s2 = ks[2];
    p.v_s0 = vs[0];
    p.v_s1 = vs[1];
    p.v_s2 = vs[2];
    p.num_blocks = a->num_blocks;
    p.out = a->out;
    p.o_s0 = a->out_stride_row;
    p.o_s1 = a->out_stride_head;
    p.out_f32 = a->out_dtype == TV_F32;
    p.cu = a->cu_seqlens_q;
    p.plen = a->prefix_lens;
    p.cnt = a->node_counts;
    p.tables = a->block_tables;
    p.t_s0 = a->block_table_stride;
    p.tree_slots = a->tree_slots;
    p.pslots = a->prefix_slots;
    p.ps_s0 = a->prefix_slots_stride;
    p.ps_i64 = a->prefix_slots_is_int64 != 0;
    p.anc = a->ancestor_words;
    p.words = a->ancestor_words_per_row;
    p.num_requests = a->num_requests;
    p.total_queries = a->total_queries;
    p.num_kv_heads = a->num_kv_heads;
    p.qpk = qpk;
    p.head_dim = a->head_dim;
    p.num_items = a->num_items;
    p.block_size = a->block_size;
    p.c = a->scale * kLog2e;
    p.items = a->items;
    p.groups = a->groups;
    p.counts = a->device_counts;
    p.ws_o = static_cast<float*>(a->workspace);
    p.ws_ml = a->workspace ? reinterpret_cast<float2*>(static_cast<char*>(a->workspace) + o_span) : nullptr;
    p.num_slots = a->workspace ? a->num_partial_slots : 0;
    p.status = a->status;
    hipStream_t s = as_stream(stream);
    const bool exact = a->exact_probabilities != 0;
    const bool bf16 = a->in_dtype == TV_BF16;
    if (a->head_dim == 256) {
        switch (qpk) {
            case 1: launch_tree_attention_d256_g1(p, a->num_items, bf16, exact, s); break;
            case 2: launch_tree_attention_d256_g2(p, a->num_items, bf16, exact, s); break;
            case 4: launch_tree_attention_d256_g4(p, a->num_items, bf16, exact, s); break;
            case 8: launch_tree_attention_d256_g8(p, a->num_items, bf16, exact, s); break;
            default: launch_tree_attention_d256_g16(p, a->num_items, bf16, exact, s); break;
        }
    } else if (a->head_dim == 64) {
        switch (qpk) {
            case 1: launch_tree_attention_d64_g1(p, a->num_items, bf16, exact, s); break;
            case 2: launch_tree_attention_d64_g2(p, a->num_items, bf16, exact, s); break;
            case 4: launch_tree_attention_d64_g4(p, a->num_items, bf16, exact, s); break;
            case 8: launch_tree_attention_d64_g8(p, a->num_items, bf16, exact, s); break;
            default: launch_tree_attention_d64_g16(p, a->num_items, bf16, exact, s); break;
        }
    } else {
        switch (qpk) {
            case 1: launch_tree_attention_g1(p, a->num_items, bf16, exact, s); break;
            case 2: launch_tree_attention_g2(p, a->num_items, bf16, exact, s); break;
            case 3: launch_tree_attention_g3(p, a->num_items, bf16, exact, s); break;
            case 4: launch_tree_attention_g4(p, a->num_items, bf16, exact, s); break;
            case 5: launch_tree_attention_g5(p, a->num_items, bf16, exact, s); break;
            case 6: launch_tree_attention_g6(p, a->num_items, bf16, exact, s); break;
            case 7: launch_tree_attention_g7(p, a->num_items, bf16, exact, s); break;
            case 8: launch_tree_attention_g8(p, a->num_items, bf16, exact, s); break;
            default: launch_tree_attention_g16(p, a->num_items, bf16, exact, s); break;
        }
    }
    if (a->num_groups > 0) {
        const int columns = a->device_counts ? std::min(a->num_groups, kMergeGridCap) : a->num_groups;
        if (bf16) {
            hipLaunchKernelGGL(merge_partials_kernel<__bf16>, dim3(columns, kRowsPerItem / 8), dim3(256), 0, s, p);
        } else {
            hipLaunchKernelGGL(merge_partials_kernel<_Float16>, dim3(columns, kRowsPerItem / 8), dim3(256), 0, s, p);
        }
    }
    return check_launch("tree_attention");
}


constexpr int kMaxDevices = 64;
std::mutex g_scratch_lock;
void* g_scratch_ptr[kMaxDevices] = {};

// The scratch address of the device that `stream` belongs to (the thread's current device
// for the null stream), resolved once per device with that device current.
int scratch_for_stream_device(hipStream_t stream, void** out) {
    int device = -1;
    hipError_t err = stream ? hipStreamGetDevice(stream, &device) : hipGetDevice(&device);
    if (err != hipSuccess) {
        return fail(TV_ERR_LAUNCH, "tree_attention_noalloc: device of the stream: %s", hipGetErrorString(err));
    }
    if (device < 0 || device >= kMaxDevices) {
        return fail(TV_ERR_UNSUPPORTED, "tree_attention_noalloc: device %d beyond %d", device, kMaxDevices);
    }
    std::lock_guard<std::mutex> guard(g_scratch_lock);
    if (!g_scratch_ptr[device]) {
        int current = -1;
        err = hipGetDevice(&current);
        if (err == hipSuccess && current != device) err = hipSetDevice(device);
        void* ptr = nullptr;
        if (err == hipSuccess) err = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
        if (current >= 0 && current != device) {
            const hipError_t restore = hipSetDevice(current);
            if (err == hipSuccess) err = restore;
        }
        if (err != hipSuccess || !ptr) {
            return fail(TV_ERR_LAUNCH, "tree_attention_noalloc: hipGetSymbolAddress: %s", hipGetErrorString(err));
        }
        g_scratch_ptr[device] = ptr;
    }
    *out = g_scratch_ptr[device];
    return TV_OK;
}

}  // namespace

extern "C" int tv_tree_attention(const tv_tree_attention_args* a, void* stream) {
    clear_error();
    return launch_tree_attention(a, stream);
}

extern "C" int64_t tv_tree_attention_noalloc_max_workspace(void) { return kScratchBytes; }

extern "C" int64_t tv_tree_attention_workspace_bytes(int32_t num_partial_slots, int32_t head_dim) {
    return workspace_need(num_partial_slots, head_dim);
}

extern "C" int tv_tree_attention_noalloc(const tv_tree_attention_args* a, void* stream) {
    clear_error();
    if (!a) return fail(TV_ERR_INVALID, "tree_attention_noalloc: null args");
    if (a->num_partial_slots < 0) return fail(TV_ERR_INVALID, "tree_attention_noalloc: invalid counts");
    const int64_t need = workspace_need(a->num_partial_slots, a->head_dim);
    if (need > kScratchBytes) {
        return fail(TV_ERR_CAPACITY,
                    "tree_attention_noalloc: the plan's %d partial slots need %lld workspace bytes, above the "
                    "%lld-byte built-in scratch; use tv_tree_attention with a caller workspace",
                    a->num_partial_slots, (long long)need, (long long)kScratchBytes);
    }
    tv_tree_attention_args local = *a;
    local.workspace = nullptr;
    local.workspace_bytes = 0;
    if (need > 0) {
        const int code = scratch_for_stream_device(as_stream(stream), &local.workspace);
        if (code != TV_OK) return code;
        local.workspace_bytes = kScratchBytes;
    }
    return launch_tree_attention(&local, stream);
}
