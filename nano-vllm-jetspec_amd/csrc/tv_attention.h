// Declarations shared by the tree-attention translation units: the kernel parameter
// block, one launcher per query-heads-per-KV-head group size G (each group size is its
// own translation unit, tv_attention_g<G>.hip, so the instantiations compile in
// parallel), and the device helpers both the attention and the merge kernels use.
#pragma once

#include <math.h>
#include <stdint.h>

#include "tv_internal.h"

namespace tv {

struct AttnParams {
    const void* q;
    int64_t q_s0, q_s1;
    const void* k;
    const void* v;
    int64_t k_s0, k_s1, k_s2;
    int64_t v_s0, v_s1, v_s2;
    int64_t num_blocks;
    void* out;
    int64_t o_s0, o_s1;
    int32_t out_f32;
    const int32_t* cu;
    const int32_t* plen;
    const int32_t* cnt;
    const int32_t* tables;
    int64_t t_s0;
    const int64_t* tree_slots;
    // Slot addressing of the prefix (the legacy single-request form, paged_backend.py:20-113):
    // prefix key k of request r lives at slot pslots[r * ps_s0 + k] instead of its page-table
    // position.  Null for page-table addressing.
    const void* pslots;
    int64_t ps_s0;
    int32_t ps_i64;
    const uint64_t* anc;
    int32_t words;
    int32_t num_requests;
    int32_t total_queries;   // packed rows of Q and O: every request's rows must lie below it
    int32_t num_kv_heads;
    int32_t block_size;
    float c;  // softmax scale * log2(e)
    const int32_t* items;
    const int32_t* groups;
    const int32_t* counts;   // device {items, groups, ...} of a device-built plan, or null
    float* ws_o;
    float2* ws_ml;
    int32_t num_slots;       // partial-result slots the workspace holds (items' and groups' slot bound)
    int32_t* status;
    int32_t qpk;             // query heads per KV head (G; the merge kernel reads it)
    int32_t head_dim;        // D: 128, 64 or 256 (the d64/d256 instances); partial rows are D floats apart
    int32_t num_items;       // items of a host plan (the D = 256 grid covers whole windows of 8)
};

// Enqueue tree_attention_kernel<operand type, exact probabilities, G> on a grid of
// num_items workgroups (bf16 operands if `bf16`, else f16); the caller checks the
// launch status with check_launch.
int launch_tree_attention_g1(const AttnParams& p, int32_t num_items, bool bf16, bool exact, hipStream_t s);
int launch_tree_attention_g2(const AttnParams& p, int32_t num_items, bool bf16, bool exact, hipStream_t s);
int launch_tree_attention_g3(const AttnParams& p, int32_t num_items, bool bf16, bool exact, hipStream_t s);
int launch_tree_attention_g4(const AttnParams& p, int32_t num_items, bool bf16, bool exact, hipStream_t s);
int launch_tree_attention_g5(const AttnParams& p, int32_t num_items, bool bf16, bool exact, hipStream_t s);
int launch_tree_attention_g6(const AttnParams& p, int32_t num_items, bool bf16, bool exact, hipStream_t s);
int launch_tree_attention_g7(const AttnParams& p, int32_t num_items, bool bf16, bool exact, hipStream_t s);
int launch_tree_attention_g8(const AttnParams& p, int32_t num_items, bool bf16, bool exact, hipStream_t s);
int launch_tree_attention_g16(const AttnParams& p, int32_t num_items, bool bf16, bool exact, hipStream_t s);
// Head size 64 (tv_attention_d64_g<G>.hip), for the power-of-two groups the reference's grouped
// kernel takes (tree_gqa.py:124-126); other groups at head size 64 run the FP32 kernel.
int launch_tree_attention_d64_g1(const AttnParams& p, int32_t num_items, bool bf16, bool exact, hipStream_t s);
int launch_tree_attention_d64_g2(const AttnParams& p, int32_t num_items, bool bf16, bool exact, hipStream_t s);
int launch_tree_attention_d64_g4(const AttnParams& p, int32_t num_items, bool bf16, bool exact, hipStream_t s);
int launch_tree_attention_d64_g8(const AttnParams& p, int32_t num_items, bool bf16, bool exact, hipStream_t s);
int launch_tree_attention_d64_g16(const AttnParams& p, int32_t num_items, bool bf16, bool exact, hipStream_t s);
// Head size 256 (tv_attention_d256_g<G>.hip), the same groups; two 4-wave workgroups per item.
int launch_tree_attention_d256_g1(const AttnParams& p, int32_t num_items, bool bf16, bool exact, hipStream_t s);
int launch_tree_attention_d256_g2(const AttnParams& p, int32_t num_items, bool bf16, bool exact, hipStream_t s);
int launch_tree_attention_d256_g4(const AttnParams& p, int32_t num_items, bool bf16, bool exact, hipStream_t s);
int launch_tree_attention_d256_g8(const AttnParams& p, int32_t num_items, bool bf16, bool exact, hipStream_t s);
int launch_tree_attention_d256_g16(const AttnParams& p, int32_t num_items, bool bf16, bool exact, hipStream_t s);

namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef short i16x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) i16x4 lds_i16x4;

constexpr int kHeadDim = 128;
constexpr int kThreads = 512;       // 8 waves
constexpr int kRowsPerItem = 256;
constexpr int kTileKeys = 32;
constexpr int kRowBytes = kHeadDim * 2;               // one K or V row of one head (bf16/f16)
constexpr int kTileBytes = kTileKeys * kRowBytes;     // 8 KiB: K (or V) of one head, one tile
constexpr int kMaskBytes = 8 * 64 * 4;                // per stage: each wave's 64 ancestor words
// Tile stages: 8 of one head (HPW 1) or 4 of two heads (HPW 2); the larger is 144 KiB.
constexpr int kRingBytes = 8 * (2 * kTileBytes + kMaskBytes);
constexpr int kMaxPages = 512;                        // page numbers of one prefix chunk
constexpr int kMaxSlotChunk = 2048;                   // prefix keys of one chunk in slot addressing
constexpr int kMaxTreeSlots = 1024;                   // tree slots cached per work item (slot-addressed prefix)
constexpr int kMaxTreeNodes = 2048;                   // ... with a page-table prefix
constexpr int kPagesOffset = kRingBytes;              // page numbers, or the chunk's prefix slots
constexpr int kSlotsOffset = kPagesOffset + kMaxSlotChunk * 4;
constexpr int kLdsBytes = kSlotsOffset + kMaxTreeSlots * 4;   // 159744 of gfx950's 160 KiB
// With a page-table prefix only kMaxPages page numbers occupy the prefix region, so the tree
// slots start right after them and run on through the slot region: kMaxTreeNodes of them.
constexpr int kTreeSlotsPageOffset = kPagesOffset + kMaxPages * 4;
static_assert(kTreeSlotsPageOffset + kMaxTreeNodes * 4 <= kLdsBytes, "page-mode tree slots exceed the LDS");
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kMaxTileSum = 256.f;                  // per lane half, against the reference

template <typename T>
__device__ __forceinline__ void store_out4(const AttnParams& p, int64_t row, int qh, int dim, f32x4 v) {
    if (p.out_f32) {
        float* o = static_cast<float*>(p.out) + row * p.o_s0 + static_cast<int64_t>(qh) * p.o_s1 + dim;
        *reinterpret_cast<f32x4*>(o) = v;
    } else {
        T* o = static_cast<T*>(p.out) + row * p.o_s0 + static_cast<int64_t>(qh) * p.o_s1 + dim;
        T h[4] = {static_cast<T>(v[0]), static_cast<T>(v[1]), static_cast<T>(v[2]), static_cast<T>(v[3])};
        *reinterpret_cast<u32x2*>(o) = __builtin_bit_cast(u32x2, h);
    }
}

}  // namespace
}  // namespace tv
