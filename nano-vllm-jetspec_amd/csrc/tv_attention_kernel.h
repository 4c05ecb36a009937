// Ragged packed tree-verify attention over a paged KV pool, written for gfx950.
//
// Semantics (paged_backend.py:116-213): packed query row q of request r, query head
// h, attends to every committed prefix position of r (page table addressed) and to
// the tree nodes of r whose ancestor bit is set (scratch slot addressed), with an
// fp32 online softmax.  GQA: query head h reads KV head h / G (G query heads per KV
// head; 4 for Qwen3-8B).
//
// Work decomposition (tv_plan.cpp): one 512-thread workgroup = 8 waves owns 256
// score rows = HPW KV heads x NPW nodes x G query heads, and a key range of the
// request (a prefix chunk, plus the tree on the last chunk).  Each wave owns 32
// score rows (32 / G nodes x G query heads of one KV head; 8 x 4 at G = 4).
//
// Data path per 32-key tile:
//   HBM -> VGPR   every thread loads one 16-byte chunk of K and of V per head; the
//                 loads of the next PF tiles are in flight while a tile is computed
//                 (PF * HPW = 4 tiles of 16 KiB per workgroup), and no address
//                 depends on a load inside the loop: the chunk's page numbers and the
//                 tree's slots are read into LDS once per work item.
//   VGPR -> LDS   natural [key][dim] rows of 256 B with the 16-byte chunks XOR-
//                 swizzled per key (K: chunk ^ key%16, V: chunk ^ 4*(key%4)), which
//                 makes both operand reads below bank-conflict free.
//   LDS -> MFMA   S^T[32 keys x 32 rows]  = K . Q^T   (8 x v_mfma_f32_32x32x16_bf16)
//                 O^T[128 dims x 32 rows] += V^T . P^T (8 x v_mfma_f32_32x32x16_bf16)
//                 K operands are ds_read_b128; V^T operands come from ds_read_b64_tr_b16
//                 transposing reads, so V is never transposed in registers.
// Writing the products transposed keeps every per-row quantity (running max, sum,
// rescale factor) in the two lanes (c, c+32) that own row c: the MFMA C layout puts
// column c in lanes c and c+32, so the softmax needs one cross-lane exchange per
// reduction and the O^T rescale none.
//
// MFMA 32x32x16 register layouts (gfx950):
//   A (32 x 16): lane l holds row l%32, k-slots 8*(l/32)+0..7
//   B (16 x 32): lane l holds col l%32, k-slots 8*(l/32)+0..7
//   C (32 x 32): lane l, register v holds row 8*(v/4) + 4*(l/32) + v%4, col l%32
// The P^T operand is taken straight from the S^T registers, so the k-slot order of
// the P.V product is a permutation of the tile's keys:
//   k-slot t of lane half g in product kk  <->  key 16*kk + 8*(t/4) + 4*g + t%4.
// ds_read_b64_tr_b16 (per 16-lane group, result lane 4a+b receives element b of
// source lanes a, a+4, a+8, a+12) delivers exactly those keys when source lane s of
// group G reads key 16*kk + 8*h + 4*(G/2) + s/4, dims 32*db + 16*(G%2) + 4*(s%4) + 0..3.
//
// Softmax: scores are scaled by softmax_scale*log2(e) inside one FMA before exp2.
// The running maximum is raised only when a tile's maximum exceeds it by more than
// 2^8 in probability units (then O and the sum are rescaled); between raises the
// probabilities are bounded by 2^8, which fp32 and bf16 hold exactly as well as
// values <= 1, so the result is the same online softmax with fewer rescales.
//
// This header holds the kernel templates; tv_attention_g<G>.hip instantiates them for one
// group size G (query heads per KV head: 1-8 or 16).  A wave's 32 score rows are
// NW = floor(32 / G) nodes x G query heads of one KV head; when G does not divide 32 the
// last 32 - NW * G rows are padding (zero Q, never stored).
#pragma once

#include <utility>

#include "tv_attention.h"

namespace tv {
namespace {

template <typename T>
struct Mfma;
template <>
struct Mfma<__bf16> {
    typedef bf16x8_t vec;
    typedef bf16x2_t pair;
    static __device__ __forceinline__ f32x16 run(vec a, vec b, f32x16 c) {
        return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
    }
    // acc + a.x + a.y in fp32 (one v_dot2 against (1, 1)).
    static __device__ __forceinline__ float dot2(pair a, float acc) {
        const pair one = {static_cast<__bf16>(1.f), static_cast<__bf16>(1.f)};
        return __builtin_amdgcn_fdot2_f32_bf16(a, one, acc, false);
    }
};
template <>
struct Mfma<_Float16> {
    typedef f16x8_t vec;
    typedef f16x2_t pair;
    static __device__ __forceinline__ f32x16 run(vec a, vec b, f32x16 c) {
        return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
    }
    static __device__ __forceinline__ float dot2(pair a, float acc) {
        const pair one = {static_cast<_Float16>(1.f), static_cast<_Float16>(1.f)};
        return __builtin_amdgcn_fdot2(a, one, acc, false);
    }
};

// Head-dimension geometry, D = 128 (Qwen3), 64 or 256.  A 32-key tile of one head is held in
// LDS as kParts parts of 32 rows x kPartRow bytes: D = 128 one part of 256-byte rows, D = 64
// one part of 128-byte rows, D = 256 four parts of 128-byte rows (dims 64p..64p+63 in part
// p), each 16-byte chunk XOR-swizzled per key within its row.  gfx950 LDS serves 256 B per
// clock from 64 banks (16 sixteen-byte bank groups):
//   K operand reads (ds_read_b128): 16 keys at one chunk per clock must land in 16 distinct
//     bank groups.  256-byte rows (every row starts at group 0): chunk ^ key%16.  128-byte
//     rows (odd rows start at group 8): chunk ^ (key/2)%8 makes the 8 keys of each row
//     parity take 8 distinct groups.
//   V^T reads (ds_read_b64_tr_b16, 32 lanes per clock): 4 keys x 4 chunks.  256-byte rows:
//     chunk ^ 4*(key%4) spreads the 4 keys over the four 4-group blocks.  128-byte rows: odd
//     keys start 8 groups over, so chunk ^ 4*((key/2)%2) separates keys of equal parity.
// Both measured 0 SQ_LDS_BANK_CONFLICT.  The 128-byte parts let one DMA lane keep one key for
// all of a tile's loads at D = 256 (8 lanes per key, one load per part).
// D = 256 doubles a wave's Q operands and O accumulators (64 + 128 registers per lane), which
// two waves per SIMD cannot hold: its workgroups have 4 waves (one per SIMD, up to 512
// registers) and a work item's 256 score rows take two of them (kHalves).
template <int D>
struct HeadDim {
    static_assert(D == 64 || D == 128 || D == 256, "head dimension of the MFMA kernel");
    static constexpr int kSteps = D / 16;          // QK^T MFMAs per tile (16 dims each)
    static constexpr int kBlocks = D / 32;         // P.V output blocks (32 dims each)
    static constexpr int kRow = 2 * D;             // bytes of one K or V row (bf16/f16)
    static constexpr int kTile = kTileKeys * kRow; // one head's K (or V) tile
    static constexpr int kSlots = 2 * kSteps;      // MFMA slots of the tile step (QK^T and P.V alternate)
    static constexpr int kPartRow = D == 128 ? 256 : 128;        // LDS row of one part
    static constexpr int kParts = kRow / kPartRow;               // parts per tile
    static constexpr int kPartBytes = kTileKeys * kPartRow;
    static constexpr int kPartChunks = kPartRow / 16;            // 16-byte chunks per part row
    static constexpr int kWaves = D == 256 ? 4 : 8;              // waves per workgroup
    static constexpr int kThreads = 64 * kWaves;
    static constexpr int kHalves = 8 / kWaves;                   // workgroups per work item
    static __device__ __forceinline__ int k_swizzle(int key) { return D == 128 ? (key & 15) : ((key >> 1) & 7); }
    static __device__ __forceinline__ int v_swizzle(int key) { return D == 128 ? 4 * (key & 3) : 4 * ((key >> 1) & 1); }
};


// s_waitcnt immediate that waits for vmcnt <= n and leaves expcnt/lgkmcnt alone.
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 0xF) | ((N >> 4) << 14) | (0x7 << 4) | (0xF << 8));
}

// Global -> LDS DMA of 16 (or 4) bytes per lane into LDS at `lds_addr` + 16 * lane
// (+ 4 * lane).  Issued from inline asm so the compiler's wait-count pass does not
// treat every later LDS read as dependent on the DMA (it would wait for vmcnt(0));
// the kernel orders the DMA explicitly with wait_vmcnt + a workgroup barrier.
// M0 is otherwise unused by this kernel (no LDS DMA builtins, GWS or indexed VGPR
// moves are emitted), so clobbering it here is safe; the kernel's ISA is checked for
// other M0 writes when it is built (nano-vllm-jetspec_amd/build.py).
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
__device__ __forceinline__ void dma_b128(const void* src, uint32_t lds_addr) {
    asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, off"
                 :
                 : "s"(lds_addr), "v"(src)
                 : "memory", "m0");
}
// Scalar-base forms: address = 64-bit SGPR base + 32-bit per-lane VGPR byte offset.
__device__ __forceinline__ void dma_b128_s(uint32_t lane_offset, const void* base, uint32_t lds_addr) {
    asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, %2"
                 :
                 : "s"(lds_addr), "v"(lane_offset), "s"(base)
                 : "memory", "m0");
}
__device__ __forceinline__ void dma_b128_s_nt(uint32_t lane_offset, const void* base, uint32_t lds_addr) {
    asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, %2 nt"
                 :
                 : "s"(lds_addr), "v"(lane_offset), "s"(base)
                 : "memory", "m0");
}
// Compile-time choice of the streaming DMA's cache policy (non-temporal or not).
template <bool B>
struct NtTag {
    static constexpr bool value = B;
};
// A compile-time integer argument (a tile part).
template <int N>
struct IntTag {
    static constexpr int value = N;
};
// f(0), f(1), ..., f(N - 1), each call with a constant argument.
template <typename F, int... I>
__device__ __forceinline__ void unrolled_seq(F&& f, std::integer_sequence<int, I...>) {
    (f(I), ...);
}
template <int N, typename F>
__device__ __forceinline__ void unrolled(F&& f) {
    unrolled_seq(f, std::make_integer_sequence<int, N>{});
}
// Forms with an immediate byte offset (D = 256: the tile part).  The instruction adds its
// immediate offset to the LDS address as well as to the global one, so M0 is set to the LDS
// destination minus the offset.
template <int OFS>
__device__ __forceinline__ void dma_b128_o(const void* src, uint32_t lds_addr) {
    asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, off offset:%2"
                 :
                 : "s"(lds_addr - OFS), "v"(src), "i"(OFS)
                 : "memory", "m0");
}
template <int OFS>
__device__ __forceinline__ void dma_b128_s_o(uint32_t lane_offset, const void* base, uint32_t lds_addr) {
    asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, %2 offset:%3"
                 :
                 : "s"(lds_addr - OFS), "v"(lane_offset), "s"(base), "i"(OFS)
                 : "memory", "m0");
}
template <int OFS>
__device__ __forceinline__ void dma_b128_s_nt_o(uint32_t lane_offset, const void* base, uint32_t lds_addr) {
    asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, %2 offset:%3 nt"
                 :
                 : "s"(lds_addr - OFS), "v"(lane_offset), "s"(base), "i"(OFS)
                 : "memory", "m0");
}
__device__ __forceinline__ void dma_b32_s(uint32_t lane_offset, const void* base, uint32_t lds_addr) {
    asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dword %1, %2"
                 :
                 : "s"(lds_addr), "v"(lane_offset), "s"(base)
                 : "memory", "m0");
}

#pragma clang diagnostic pop

struct Item {
    int r, h0, n0, kbeg, kend, flags, slot, hpw;
};

// A pointer the caller knows to be wave-uniform, moved to SGPRs.
__device__ __forceinline__ const void* uniform_ptr(const void* ptr) {
    const uint64_t v = reinterpret_cast<uint64_t>(ptr);
    const uint32_t lo = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(v));
    const uint32_t hi = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(v >> 32));
    return reinterpret_cast<const void*>((static_cast<uint64_t>(hi) << 32) | lo);
}

// Keeps the compiler from moving instructions across this point, so the hand-made
// MFMA / LDS / VALU interleave of the tile step survives scheduling.
__device__ __forceinline__ void order_point() { __builtin_amdgcn_sched_barrier(0); }

// An empty use of a VGPR value: emits nothing, but keeps the computation of `x` in
// the basic block where it is written, so code sinking cannot move VALU work out of
// its slot (the tile step has a branchy scalar section in its middle).
__device__ __forceinline__ void pin(float x) { asm volatile("" : : "v"(x)); }

// LDS operands are read this many MFMA slots ahead of their use (4 measured 1 % faster than
// 2 on the long-context batches, 3 no faster than 2).
constexpr int kReadAhead = 4;

// One work item with HPW KV heads per workgroup.  EXACT keeps every probability to about
// 2^-17 relative in the P.V product: it is split into a rounded operand-type part and the
// operand-type rounding of the remainder, and both are multiplied into O (two MFMAs), with
// the row sums taken in fp32; otherwise the probability is rounded to the operand type once.
template <typename T, int HPW, bool EXACT, int G, int D>
__device__ __forceinline__ void run_item(const AttnParams& p, char* smem, const Item& it, const int half) {
    typedef HeadDim<D> HD;
    typedef typename Mfma<T>::vec V8;
    typedef typename Mfma<T>::pair V2;
    typedef __attribute__((address_space(3))) char lds_char;
    constexpr int THREADS = HD::kThreads;
    constexpr int WPH = 8 / HPW;                        // waves per KV head (of the item's 8)
    constexpr int NW = 32 / G;                          // nodes per wave (G query heads each)
    constexpr int NPW = NW * WPH;                       // nodes per work item
    static_assert(G >= 1 && G <= 16, "query heads per KV head");
    // KV heads this workgroup stages: the item's HPW, or one per 4-wave half at D = 256 (a
    // two-head item's halves are its two heads; a one-head item's halves share its head).
    constexpr int HPWL = D == 256 ? 1 : HPW;
    // LDS ring of NS stages.  K tiles, V tiles and ancestor words live in three regions
    // so every operand address is a per-lane constant plus a compile-time stage offset.
    // 32 KiB tile sets (two heads at D = 128, one at D = 256) leave room for 4 stages.
    constexpr int NS = (D == 256 || (D == 128 && HPWL == 2)) ? 4 : 8;
    constexpr int TILE_SET = HPWL * HD::kTile;          // K (or V) of the staged heads, one stage
    constexpr int V_REGION = NS * TILE_SET;
    constexpr int M_REGION = 2 * NS * TILE_SET;
    // DMA loads per tile per wave, at least: a K and a V load per head at D = 128 (each wave
    // moves 4 keys, 16 lanes per key); at D = 64 waves 0-3 move K and waves 4-7 V, 8 keys each;
    // at D = 256 each wave moves 8 keys of K and of V, one load per part.
    constexpr int LPT = D == 128 ? 2 * HPW : (D == 64 ? HPW : 2 * HD::kParts);
    static_assert(M_REGION + NS * kMaskBytes <= kRingBytes, "ring exceeds its LDS region");
    // At D = 256 the 4-stage ring stages K one tile further ahead than V (SPLIT): in step t, K
    // of tile t+3 goes into the stage of tile t-1, whose K was last read in step t-2 (its V is
    // still read in step t), and V (with the ancestor words) of tile t+2 into the stage of tile
    // t-2.  K then has two steps to arrive and V three, and each step waits only for the loads
    // issued two steps back: two tile sets in flight per workgroup instead of one (cfg4 at
    // D = 256: 3.71 -> 3.19 ms).  The two-head items of D = 128, whose streams are short, ran
    // 4-6 % slower that way (cfg1, cfg2) and keep the one-ahead ring.
    constexpr bool SPLIT = NS == 4 && D == 256;
    constexpr int LPTK = D == 256 ? HD::kParts : HPW;   // K loads per tile and wave (SPLIT)
    constexpr int WAIT_STEP = SPLIT ? LPT : (NS - 4) * LPT;   // loads a step may leave in flight

    // `wave` is the same in all lanes; readfirstlane lets the compiler see that, so
    // every per-wave quantity below lives in SGPRs and per-wave branches are scalar.
    // `vw` is the wave's place among the item's 8 (the workgroup's half at D = 256).
    const int tid = threadIdx.x, lane = tid & 63, c = lane & 31, g = lane >> 5;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int vw = D == 256 ? HD::kWaves * half + wave : wave;
    const int hl = vw / WPH;
    const int head = it.h0 + hl;
    const int hs = D == 256 ? 0 : hl;                   // the head's place in the staged set
    const int nsub = vw - hl * WPH;
    const int r = it.r;
    const int tn = p.cnt[r], qbase = p.cu[r], plen = p.plen[r];
    const int node = it.n0 + NW * nsub + c / G;
    const int qh = head * G + c % G;
    const bool head_ok = head < p.num_kv_heads;
    const bool wave_active = head_ok && (it.n0 + NW * nsub) < tn;
    if constexpr (D == 256) {
        // A half with no rows to compute (past the tree or the last head) stages nothing.
        const int vw0 = HD::kWaves * half, hl0 = vw0 / WPH;
        if (!(it.h0 + hl0 < p.num_kv_heads && it.n0 + NW * (vw0 - hl0 * WPH) < tn)) return;
    }
    // Rows past NW * G (G not dividing 32) are padding: they load no Q and store nothing.
    const bool row_ok = head_ok && c < NW * G && node < tn;
    const int tree_end = (it.flags & kItemLastChunk) ? min(tn, it.n0 + NPW) : 0;
    const int ntp = (it.kend - it.kbeg + kTileKeys - 1) / kTileKeys;
    const int nt = ntp + (tree_end + kTileKeys - 1) / kTileKeys;
    const int B = p.block_size;
    const int64_t pool_slots = p.num_blocks * B;
    // Slot addressing is compiled into the EXACT instance only (the legacy entry's mode).
    const bool slot_mode = EXACT && p.pslots != nullptr;
    const int page0 = it.kbeg / B;
    const int nkeys = it.kend - it.kbeg;
    const int npages = slot_mode ? 0 : (nkeys > 0 ? (it.kend - 1) / B - page0 + 1 : 0);
    // The planner keeps every item within the LDS page/slot caches, non-empty, inside its
    // request's prefix and inside the workspace; an item that is not (a plan made for other
    // metadata) is reported and skipped rather than read past the request's table row.
    if (nt == 0 || npages > kMaxPages || tree_end > (slot_mode ? kMaxTreeSlots : kMaxTreeNodes) ||
        (slot_mode && nkeys > kMaxSlotChunk) ||
        it.h0 < 0 || it.n0 < 0 || it.kbeg < 0 || it.kend < it.kbeg || it.kend > plen || it.slot >= p.num_slots) {
        if (tid == 0) set_status(p.status, TV_STATUS_BAD_REQUEST);
        return;
    }

    // Page numbers of the prefix chunk and slots of the tree, validated, into LDS, and
    // this lane's Q rows into registers.  All of them are loaded before any is used
    // (at most one page and two tree slots per thread, four at D = 256), so the three
    // lookups cost one round trip, not three.
    constexpr int PPT = (kMaxPages + THREADS - 1) / THREADS;       // page loads per thread
    constexpr int TPT = (kMaxTreeSlots + THREADS - 1) / THREADS;   // tree slot loads per thread (first 1024)
    constexpr int XPT = (kMaxTreeNodes - kMaxTreeSlots + THREADS - 1) / THREADS;   // ... beyond them
    constexpr int SPT = (kMaxSlotChunk + THREADS - 1) / THREADS;   // prefix slot loads per thread
    int32_t* pages = reinterpret_cast<int32_t*>(smem + kPagesOffset);
    int32_t* tslots = reinterpret_cast<int32_t*>(smem + (slot_mode ? kSlotsOffset : kTreeSlotsPageOffset));
    int32_t pg[PPT];
    int64_t sl[TPT];
    int64_t ps[SPT];
#pragma unroll
    for (int k = 0; k < PPT; ++k) {
        pg[k] = 0;
        if (tid + k * THREADS < npages) pg[k] = p.tables[static_cast<int64_t>(r) * p.t_s0 + page0 + tid + k * THREADS];
    }
#pragma unroll
    for (int k = 0; k < SPT; ++k) ps[k] = 0;
    if (slot_mode) {
        const int64_t base = static_cast<int64_t>(r) * p.ps_s0 + it.kbeg;
#pragma unroll
        for (int k = 0; k < SPT; ++k) {
            const int i = tid + k * THREADS;
            if (i < nkeys) {
                ps[k] = p.ps_i64 ? static_cast<const int64_t*>(p.pslots)[base + i]
                                 : static_cast<int64_t>(static_cast<const int32_t*>(p.pslots)[base + i]);
            }
        }
    }
#pragma unroll
    for (int k = 0; k < TPT; ++k) {
        sl[k] = 0;
        if (tid + k * THREADS < tree_end) sl[k] = p.tree_slots[qbase + tid + k * THREADS];
    }
    // Q^T operand: lane (c, g) holds score row c, dims 16*st + 8*g + 0..7.
    V8 qb[HD::kSteps];
    {
        const T* qrow = static_cast<const T*>(p.q) + static_cast<int64_t>(qbase + node) * p.q_s0 +
                        static_cast<int64_t>(qh) * p.q_s1 + 8 * g;
#pragma unroll
        for (int st = 0; st < HD::kSteps; ++st) {
            u32x4 raw = {0u, 0u, 0u, 0u};
            if (row_ok) raw = *reinterpret_cast<const u32x4*>(qrow + 16 * st);
            qb[st] = __builtin_bit_cast(V8, raw);
        }
    }
#pragma unroll
    for (int k = 0; k < PPT; ++k) {
        if (tid + k * THREADS < npages) {
            int32_t v = pg[k];
            if (v < 0 || v >= p.num_blocks) {
                set_status(p.status, TV_STATUS_BAD_PAGE);
                v = 0;
            }
            pages[tid + k * THREADS] = v;
        }
    }
    if (slot_mode) {
#pragma unroll
        for (int k = 0; k < SPT; ++k) {
            const int i = tid + k * THREADS;
            if (i < nkeys) {
                int64_t v = ps[k];
                if (v < 0 || v >= pool_slots) {
                    set_status(p.status, TV_STATUS_BAD_PAGE);
                    v = 0;
                }
                pages[i] = static_cast<int32_t>(v);
            }
        }
    }
#pragma unroll
    for (int k = 0; k < TPT; ++k) {
        const int i = tid + k * THREADS;
        if (i < tree_end) {
            int64_t v = sl[k];
            if (v < 0 || v >= pool_slots) {
                set_status(p.status, TV_STATUS_BAD_PAGE);
                v = 0;
            }
            tslots[i] = static_cast<int32_t>(v);
        }
    }
    // Trees above 1024 nodes (page-table prefixes only): their further slots in a second round
    // trip, so the common prologue keeps its one.
    if (tree_end > kMaxTreeSlots) {
#pragma unroll
        for (int k = 0; k < XPT; ++k) {
            const int i = kMaxTreeSlots + tid + k * THREADS;
            if (i < tree_end) {
                int64_t v = p.tree_slots[qbase + i];
                if (v < 0 || v >= pool_slots) {
                    set_status(p.status, TV_STATUS_BAD_PAGE);
                    v = 0;
                }
                tslots[i] = static_cast<int32_t>(v);
            }
        }
    }
    // Retire the Q loads here: the tile loop then contains no compiler-tracked vector
    // load, so the only vmcnt waits in it are the explicit per-tile ones below.
    wait_vmcnt<0>();
    __syncthreads();  // page and slot lists visible

    lds_char* lds = (lds_char*)(smem);
    // Per-lane LDS operand offsets (stage 0).
    //   K, MFMA step st: key c, chunk 2*st+g at position (2*st+g) ^ swizzle(c), in part
    //   st / (steps per part).
    //   V, output block db: key vk (+16*kk+8*h), chunk 4*db+vc at position ^ swizzle(vk), in
    //   part db / (blocks per part).
    constexpr int SPP = HD::kSteps / HD::kParts, BPP = HD::kBlocks / HD::kParts;
    uint32_t k_ofs[HD::kSteps];
#pragma unroll
    for (int st = 0; st < HD::kSteps; ++st) {
        k_ofs[st] = hs * HD::kTile + (st / SPP) * HD::kPartBytes + c * HD::kPartRow +
                    (((2 * (st % SPP) + g) ^ HD::k_swizzle(c)) & (HD::kPartChunks - 1)) * 16;
    }
    const int grp = lane >> 4, src = lane & 15;
    const int vk = 4 * (grp >> 1) + (src >> 2);
    const int vc = 2 * (grp & 1) + ((src & 3) >> 1);
    uint32_t v_ofs[HD::kBlocks];
#pragma unroll
    for (int db = 0; db < HD::kBlocks; ++db) {
        v_ofs[db] = V_REGION + hs * HD::kTile + (db / BPP) * HD::kPartBytes + vk * HD::kPartRow +
                    (((4 * (db % BPP) + vc) ^ HD::v_swizzle(vk)) & (HD::kPartChunks - 1)) * 16 + (src & 1) * 8;
    }
    const uint32_t m_ofs = M_REGION + wave * 256 + 4 * (c / G);

    // Staging: global -> LDS DMA (global_load_lds_dwordx4 writes lane L's 16 bytes at
    // the wave's LDS base + 16*L).  Wave w moves keys 4w..4w+3 of every tile: lane L
    // loads key 4w + L/16 and the 16-byte chunk that belongs at LDS position L%16 of
    // that key's row, i.e. global chunk (L%16) ^ swizzle(key).  Every load takes a
    // per-lane 64-bit address: for a prefix tile the tile's page base (scalar
    // arithmetic) plus a per-lane byte offset, for a tree tile the lane's own slot.
    // At D = 128 wave w moves keys 4w..4w+3 of every tile (16 lanes per key); at D = 64 wave w
    // moves keys 8(w%4)..8(w%4)+7 (8 lanes per key) of K (w < 4) or V (w >= 4); at D = 256
    // (4 waves) wave w moves keys 8w..8w+7 of K and of V, one load per part (8 lanes per key,
    // the part's 8 chunks; part p adds 128p bytes to the global address and 4 KiB in LDS).
    const int s_key = D == 128 ? (tid >> 4) : 8 * (wave & 3) + (lane >> 3);
    const int k_chunk = (lane & (HD::kPartChunks - 1)) ^ HD::k_swizzle(s_key);
    const int v_chunk = (lane & (HD::kPartChunks - 1)) ^ HD::v_swizzle(s_key);
    const bool k_wave = D != 64 || wave < 4;    // D = 64: this wave's DMA moves K (else V)
    const uint32_t k_chunk_b = 16u * k_chunk, v_chunk_b = 16u * v_chunk;
    // Byte strides; the host checks that a page stride fits 32 bits and 32 key rows 31.
    const uint32_t k_page_b = static_cast<uint32_t>(p.k_s0 * static_cast<int64_t>(sizeof(T)));
    const uint32_t v_page_b = static_cast<uint32_t>(p.v_s0 * static_cast<int64_t>(sizeof(T)));
    const uint32_t k_key_b = static_cast<uint32_t>(p.k_s1 * static_cast<int64_t>(sizeof(T)));
    const uint32_t v_key_b = static_cast<uint32_t>(p.v_s1 * static_cast<int64_t>(sizeof(T)));
    const uint32_t k_lane_b = s_key * k_key_b + k_chunk_b;
    const uint32_t v_lane_b = s_key * v_key_b + v_chunk_b;
    // First staged head (h0 of the group; at D = 256 the half's head), and the byte step to
    // staged head j (clamped to the last head).
    const int hfirst = D == 256 && HPW == 2 ? it.h0 + half : it.h0;
    const int h0c = min(hfirst, p.num_kv_heads - 1);
    const uint64_t k_head_b = reinterpret_cast<uint64_t>(p.k) + static_cast<uint64_t>(h0c * p.k_s2 * sizeof(T));
    const uint64_t v_head_b = reinterpret_cast<uint64_t>(p.v) + static_cast<uint64_t>(h0c * p.v_s2 * sizeof(T));
    int64_t k_hstep_b[HPWL], v_hstep_b[HPWL];
#pragma unroll
    for (int j = 0; j < HPWL; ++j) {
        const int64_t dh = min(hfirst + j, p.num_kv_heads - 1) - h0c;
        k_hstep_b[j] = dh * p.k_s2 * static_cast<int64_t>(sizeof(T));
        v_hstep_b[j] = dh * p.v_s2 * static_cast<int64_t>(sizeof(T));
    }
    const bool pow2 = (B & (B - 1)) == 0;
    const int bshift = __builtin_ctz(B);

    // Ancestor bits: lane L of wave w fetches the word of node n0 + NW*nsub + L%NW (the
    // wave's own NW nodes; rows past the tree read the last node's word).
    const int mask_node = min(it.n0 + NW * nsub + lane % NW, tn - 1);
    const uint32_t m_lane_b = static_cast<uint32_t>(mask_node * p.words * 8);
    const char* anc_req = reinterpret_cast<const char*>(p.anc + static_cast<int64_t>(qbase) * p.words);

    // A tile's DMA is issued in steps spread over a tile step of the pipeline (so the
    // eight waves do not all queue on the scalar unit and the load path at once):
    //   fetch(t)           one iteration ahead: the LDS-cached page number (prefix
    //                      tile) or this lane's tree slot (tree tile);
    //   describe(t, f)     the per-lane K and V addresses of tile t (head h0);
    //   issue_k/v/mask     the loads into a stage (ancestor words for tree tiles only).
    // Keys past the item's range, and tiles past the last one, read the tile's first
    // key (finite data, masked later; cache hits), so every load is in bounds and each
    // wave issues at least 2*HPW loads per tile (the count the waits are based on).
    auto fetch = [&](int t) -> int {
        const int tt = t < nt ? t : nt - 1;
        if (tt < ntp && slot_mode) {
            const int m0 = kTileKeys * tt;
            int m = m0 + s_key;
            if (m >= nkeys) m = m0;
            return pages[m];
        }
        if (tt < ntp) {
            const uint32_t tile_pos = static_cast<uint32_t>(it.kbeg + kTileKeys * tt);
            const uint32_t page_abs = pow2 ? (tile_pos >> bshift) : (tile_pos / static_cast<uint32_t>(B));
            return pages[page_abs - page0];
        }
        const int m0 = kTileKeys * (tt - ntp);
        int m = m0 + s_key;
        if (m >= tree_end) m = m0;
        return tslots[m];
    };
    uint64_t dk = 0, dv = 0;   // this lane's K and V chunk addresses of the described tile
    bool dtree = false;        // described tile is a tree tile
    uint32_t dmask = 0;        // its ancestor word offset (bytes)
    auto describe = [&](int t, int fetched) {
        const int tt = t < nt ? t : nt - 1;
        if (tt < ntp && slot_mode) {
            const uint32_t slot = static_cast<uint32_t>(fetched);
            const uint32_t pg = pow2 ? (slot >> bshift) : (slot / static_cast<uint32_t>(B));
            const uint32_t off = slot - pg * static_cast<uint32_t>(B);
            dk = k_head_b + static_cast<uint64_t>(pg) * k_page_b + static_cast<uint64_t>(off) * k_key_b + k_chunk_b;
            dv = v_head_b + static_cast<uint64_t>(pg) * v_page_b + static_cast<uint64_t>(off) * v_key_b + v_chunk_b;
            dtree = false;
        } else if (tt < ntp) {
            const uint32_t tile_pos = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(it.kbeg + kTileKeys * tt));
            const uint32_t page_abs = pow2 ? (tile_pos >> bshift) : (tile_pos / static_cast<uint32_t>(B));
            const uint32_t off0 = tile_pos - page_abs * static_cast<uint32_t>(B);
            const uint32_t page = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(fetched));
            const uint64_t kb = k_head_b + static_cast<uint64_t>(page) * k_page_b + static_cast<uint64_t>(off0) * k_key_b;
            const uint64_t vb = v_head_b + static_cast<uint64_t>(page) * v_page_b + static_cast<uint64_t>(off0) * v_key_b;
            uint32_t kl = k_lane_b, vl = v_lane_b;
            if (static_cast<int>(tile_pos) + kTileKeys > it.kend) {
                const bool in = static_cast<int>(tile_pos) + s_key < it.kend;
                kl = in ? kl : k_chunk_b;
                vl = in ? vl : v_chunk_b;
            }
            dk = kb + kl;
            dv = vb + vl;
            dtree = false;
        } else {
            const uint32_t slot = static_cast<uint32_t>(fetched);
            const uint32_t pg = pow2 ? (slot >> bshift) : (slot / static_cast<uint32_t>(B));
            const uint32_t off = slot - pg * static_cast<uint32_t>(B);
            dk = k_head_b + static_cast<uint64_t>(pg) * k_page_b + static_cast<uint64_t>(off) * k_key_b + k_chunk_b;
            dv = v_head_b + static_cast<uint64_t>(pg) * v_page_b + static_cast<uint64_t>(off) * v_key_b + v_chunk_b;
            dtree = true;
            dmask = static_cast<uint32_t>(tt - ntp) * 4;
        }
    };
    // LDS destination of a DMA: this wave's part of the ring (one SGPR for tiles, one
    // for ancestor words) plus a compile-time stage offset.  The empty asm makes the
    // base opaque at each use, so the compiler emits one scalar add per DMA instead of
    // keeping every stage address live (and spilled).
    const uint32_t lds_base = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(reinterpret_cast<uintptr_t>(lds)));
    // Each wave's DMA fills 1 KB of a tile (4 keys at D = 128, 8 at D = 64); at D = 64 the V
    // waves' part lies in the V region.
    const uint32_t wave_tile_lds = lds_base + (D == 128 ? wave : (wave & 3)) * 1024 + (k_wave ? 0 : V_REGION);
    const uint32_t wave_mask_lds = lds_base + M_REGION + wave * 256;
    auto tile_dst = [&](int offset) {
        uint32_t base = wave_tile_lds;
        asm volatile("" : "+s"(base));
        return base + static_cast<uint32_t>(offset);
    };
    auto mask_dst = [&](int offset) {
        uint32_t base = wave_mask_lds;
        asm volatile("" : "+s"(base));
        return base + static_cast<uint32_t>(offset);
    };
    auto issue_k = [&](int stage, int j) {
        dma_b128(reinterpret_cast<const void*>(dk + k_hstep_b[j]), tile_dst(stage * TILE_SET + j * HD::kTile));
    };
    auto issue_v = [&](int stage, int j) {
        dma_b128(reinterpret_cast<const void*>(dv + v_hstep_b[j]),
                 tile_dst(V_REGION + stage * TILE_SET + j * HD::kTile));
    };
    // D = 64: this wave's one load per head and tile, K or V (wave_tile_lds holds the region).
    auto issue_kv = [&](int stage, int j) {
        const uint64_t src = k_wave ? dk + k_hstep_b[j] : dv + v_hstep_b[j];
        dma_b128(reinterpret_cast<const void*>(src), tile_dst(stage * TILE_SET + j * HD::kTile));
    };
    // D = 256: part P of this wave's K (or V) keys of the staged head.
    auto issue_k_part = [&](auto part, int stage) {
        constexpr int P = decltype(part)::value;
        dma_b128_o<128 * P>(reinterpret_cast<const void*>(dk), tile_dst(stage * TILE_SET + P * HD::kPartBytes));
    };
    auto issue_v_part = [&](auto part, int stage) {
        constexpr int P = decltype(part)::value;
        dma_b128_o<128 * P>(reinterpret_cast<const void*>(dv),
                            tile_dst(V_REGION + stage * TILE_SET + P * HD::kPartBytes));
    };
    auto issue_mask = [&](int stage) {
        if (dtree) dma_b32_s(m_lane_b, uniform_ptr(anc_req + dmask), mask_dst(stage * kMaskBytes));
    };
    auto issue_all = [&](int stage) {
        if constexpr (D == 256) {
            issue_k_part(IntTag<0>{}, stage);
            issue_k_part(IntTag<1>{}, stage);
            issue_k_part(IntTag<2>{}, stage);
            issue_k_part(IntTag<3>{}, stage);
            issue_v_part(IntTag<0>{}, stage);
            issue_v_part(IntTag<1>{}, stage);
            issue_v_part(IntTag<2>{}, stage);
            issue_v_part(IntTag<3>{}, stage);
        } else if constexpr (D == 128) {
#pragma unroll
            for (int j = 0; j < HPW; ++j) issue_k(stage, j);
#pragma unroll
            for (int j = 0; j < HPW; ++j) issue_v(stage, j);
        } else {
#pragma unroll
            for (int j = 0; j < HPW; ++j) issue_kv(stage, j);
        }
        issue_mask(stage);
    };
    // SPLIT rings (D = 128 two-head items, D = 256): the K or the V loads of a described tile.
    auto issue_k_set = [&](int stage) {
        if constexpr (D == 256) {
            issue_k_part(IntTag<0>{}, stage);
            issue_k_part(IntTag<1>{}, stage);
            issue_k_part(IntTag<2>{}, stage);
            issue_k_part(IntTag<3>{}, stage);
        } else {
#pragma unroll
            for (int j = 0; j < HPW; ++j) issue_k(stage, j);
        }
    };
    f32x16 acc[HD::kBlocks];
#pragma unroll
    for (int db = 0; db < HD::kBlocks; ++db) acc[db] = f32x16{};
    // Per row: reference maximum m_run (score units), -m_run*cs, and this lane's half
    // of the running sum.
    float m_run = -INFINITY, nmc = 0.f, l_run = 0.f;
    const float cs = p.c;
    // Tiles [0, nfull) are whole prefix tiles that need no mask.
    const int nfull = (it.kend - it.kbeg) / kTileKeys;

    // Masks tile tt's scores in place (partial prefix tile and tree tiles only).
    auto mask_tile = [&](f32x16& s, int stage, int tt) {
        // Visibility of the 16 keys this lane holds: key index 8*(v/4) + 4*g + v%4.
        if (tt < ntp) {
            const int nvalid = it.kend - (it.kbeg + kTileKeys * tt);
#pragma unroll
            for (int v = 0; v < 16; ++v) {
                if (8 * (v >> 2) + 4 * g + (v & 3) >= nvalid) s[v] = -INFINITY;
            }
        } else {
            const uint32_t tree_bits =
                row_ok ? *(const __attribute__((address_space(3))) uint32_t*)(lds + m_ofs + stage * kMaskBytes) : 0u;
            const uint32_t half_bits = tree_bits >> (4 * g);
#pragma unroll
            for (int v = 0; v < 16; ++v) {
                if (!((half_bits >> (8 * (v >> 2) + (v & 3))) & 1u)) s[v] = -INFINITY;
            }
        }
    };
    // Raises the reference maximum of each row that asks for it (`need` in either lane
    // half) to the maximum of tile scores `s` where that is larger, rescaling O and
    // the sum (which then hold every earlier tile).  Both lane halves of a row take the
    // decision on the full row, so they share one reference; rows that do not ask keep
    // theirs, so a row's result never depends on other rows' scores.
    auto raise_max = [&](const f32x16& s, bool need) {
        float mx = fmaxf(fmaxf(s[0], s[1]), s[2]);
#pragma unroll
        for (int v = 3; v < 15; v += 2) mx = fmaxf(fmaxf(mx, s[v]), s[v + 1]);
        mx = fmaxf(mx, s[15]);
        const float row_max = fmaxf(mx, __shfl_xor(mx, 32));
        // Both halves must see the exchange: no short-circuit, which would make the
        // lane exchange divergent and leave the two halves of a row disagreeing.
        const int partner_need = __shfl_xor(static_cast<int>(need), 32);
        const bool row_need = need | (partner_need != 0);
        if (row_need && row_max > m_run) {
            const float alpha = __builtin_amdgcn_exp2f((m_run - row_max) * cs);
            l_run *= alpha;
#pragma unroll
            for (int db = 0; db < HD::kBlocks; ++db) acc[db] *= alpha;
            m_run = row_max;
            nmc = -row_max * cs;
        }
    };
    // Probabilities of tile scores `s` against the current reference, packed as the
    // P^T operand, and this lane's sum of the packed values.
    auto probabilities = [&](const f32x16& s, V8 (&pb)[2], V8 (&pl)[2]) -> float {
        float l0 = 0.f, l1 = 0.f;
#pragma unroll
        for (int kk = 0; kk < 2; ++kk) {
#pragma unroll
            for (int t8 = 0; t8 < 8; ++t8) {
                const float pr = __builtin_amdgcn_exp2f(fmaf(s[8 * kk + t8], cs, nmc));
                pb[kk][t8] = static_cast<T>(pr);
                if constexpr (EXACT) {
                    pl[kk][t8] = static_cast<T>(pr - static_cast<float>(pb[kk][t8]));
                    if (t8 & 1) l1 += pr; else l0 += pr;
                }
            }
            if constexpr (!EXACT) {
#pragma unroll
                for (int q2 = 0; q2 < 4; ++q2) {
                    const V2 two = {pb[kk][2 * q2], pb[kk][2 * q2 + 1]};
                    if (q2 & 1) l1 = Mfma<T>::dot2(two, l1); else l0 = Mfma<T>::dot2(two, l0);
                }
            }
        }
        return l0 + l1;
    };

    // One tile step of the pipeline, in a fixed issue order: MFMA slots alternate
    // between the 8 QK^T steps of tile t+1 and the 8 P.V steps of tile t-1 (whose
    // probabilities were packed in the previous step), every LDS operand is read
    // kReadAhead slots ahead of its use, and the softmax VALU work of tile t (16 exp2, the bf16
    // packing, the row sums) runs as one block halfway through the step's MFMA slots (before
    // slot 8 of 16 at D = 128; slots 2, 4, 6, 10, 12 or after 16 measured slower).  No MFMA of the
    // step waits for a VALU result of the same step.  The block, rather than one exp2
    // per slot, keeps each wave's MFMAs back to back while the other wave of its SIMD
    // fills the matrix core; it measured 3-3.5 % faster on the long-context batches.
    // piece(slot) adds the DMA issue of a later tile, a step at a time.
    auto step = [&](const f32x16& s, f32x16& sn, const V8 (&pb_prev)[2], V8 (&pb)[2], const V8 (&pl_prev)[2],
                    V8 (&pl)[2], const int kst,
                    const int vst, auto&& piece) -> float {
        V8 ka[HD::kSteps];
        i16x4 vlo[HD::kSteps], vhi[HD::kSteps];
        float pr[16];
        float l0 = 0.f, l1 = 0.f;
        auto kread = [&](int i) {
            ka[i] = __builtin_bit_cast(V8, *(const __attribute__((address_space(3))) u32x4*)(lds + k_ofs[i] + kst));
        };
        // P.V step j: k half kk = j / 4, output block db = j % 4.
        auto vread = [&](int j) {
            const int kk = j / HD::kBlocks, db = j % HD::kBlocks;
            vlo[j] = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                (lds_i16x4*)(lds + v_ofs[db] + vst + (16 * kk) * HD::kPartRow));
            vhi[j] = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                (lds_i16x4*)(lds + v_ofs[db] + vst + (16 * kk + 8) * HD::kPartRow));
        };
        auto slot_mfma = [&](int sl) {
            if ((sl & 1) == 0) {
                const int i = sl >> 1;
                sn = Mfma<T>::run(ka[i], qb[i], i == 0 ? f32x16{} : sn);
            } else {
                const int j = sl >> 1, kk = j / HD::kBlocks, db = j % HD::kBlocks;
                const V8 a = __builtin_bit_cast(V8, __builtin_shufflevector(vlo[j], vhi[j], 0, 1, 2, 3, 4, 5, 6, 7));
                acc[db] = Mfma<T>::run(a, pb_prev[kk], acc[db]);
                if constexpr (EXACT) acc[db] = Mfma<T>::run(a, pl_prev[kk], acc[db]);
            }
        };
        auto slot_read = [&](int sl) {
            if ((sl & 1) == 0) kread(sl >> 1); else vread(sl >> 1);
        };
        auto ex = [&](int e) {
            pr[e] = __builtin_amdgcn_exp2f(fmaf(s[e], cs, nmc));
            pin(pr[e]);
        };
        auto pack = [&](int q) {  // probabilities 2q, 2q+1
            pb[q >> 2][2 * (q & 3)] = static_cast<T>(pr[2 * q]);
            pb[q >> 2][2 * (q & 3) + 1] = static_cast<T>(pr[2 * q + 1]);
            if constexpr (EXACT) {
                pl[q >> 2][2 * (q & 3)] = static_cast<T>(pr[2 * q] - static_cast<float>(pb[q >> 2][2 * (q & 3)]));
                pl[q >> 2][2 * (q & 3) + 1] =
                    static_cast<T>(pr[2 * q + 1] - static_cast<float>(pb[q >> 2][2 * (q & 3) + 1]));
            }
        };
        auto rsum = [&](int q) {
            if constexpr (EXACT) {
                if (q & 1) l1 += pr[2 * q] + pr[2 * q + 1]; else l0 += pr[2 * q] + pr[2 * q + 1];
                return;
            }
            const V2 two = {pb[q >> 2][2 * (q & 3)], pb[q >> 2][2 * (q & 3) + 1]};
            if (q & 1) {
                l1 = Mfma<T>::dot2(two, l1);
                pin(l1);
            } else {
                l0 = Mfma<T>::dot2(two, l0);
                pin(l0);
            }
        };
#pragma unroll
        for (int sl = 0; sl < kReadAhead; ++sl) slot_read(sl);
        order_point();
        auto slot = [&](int sl) {
            if (sl == HD::kSlots / 2) {
#pragma unroll
                for (int e = 0; e < 16; ++e) ex(e);
#pragma unroll
                for (int q = 0; q < 8; ++q) pack(q);
#pragma unroll
                for (int q = 0; q < 8; ++q) rsum(q);
                order_point();
            }
            slot_mfma(sl);
            if (sl + kReadAhead < HD::kSlots) slot_read(sl + kReadAhead);
            order_point();
            piece(sl);
            order_point();
        };
        if constexpr (D == 256) {
            // 32 slots exceed the unroller's size limit for a pragma; a fold over the slot
            // indices unrolls them at compile time.
            unrolled<HD::kSlots>(slot);
        } else {
#pragma unroll
            for (int sl = 0; sl < HD::kSlots; ++sl) slot(sl);
        }
        return l0 + l1;
    };

    // Software pipeline over the tiles, three deep: iteration t waits for tile t+1 and
    // barriers (publishing every wave's DMA of tile t+1 and retiring stage (t-2)%NS,
    // last read by P.V of tile t-2 in iteration t-1), masks tile t if needed, and runs
    // the step (S of tile t+1, P.V of tile t-1, softmax of tile t) with the DMA of tile
    // t+NS-2 into the retired stage.  The reference maximum comes from tile 0 exactly;
    // later tiles use it as it stands, and only when a tile's probabilities sum past
    // 2^8 (a score above the reference by more than log2 of that, or a non-finite sum)
    // is the maximum raised and the tile recomputed, before its P.V is issued.  The
    // loop is unrolled NS times so every stage offset is a compile-time constant.
    {
        // P.V of "tile -1" (iteration 0) multiplies zero probabilities into stage NS-1;
        // make that stage's V finite.
        typedef __attribute__((address_space(3))) u32x4 lds_u32x4;
#pragma unroll
        for (int i = tid; i < TILE_SET / 16; i += THREADS) {
            *(lds_u32x4*)(lds + V_REGION + (NS - 1) * TILE_SET + 16 * i) = u32x4{0u, 0u, 0u, 0u};
        }
    }
#pragma unroll
    for (int b = 0; b < NS - 2; ++b) {
        describe(b, fetch(b));
        issue_all(b);
    }
    if constexpr (SPLIT) {
        describe(NS - 2, fetch(NS - 2));
        issue_k_set(NS - 2);
    }

    // Streaming DMA of whole prefix tiles.  Steps t < t_fast need no mask and stage a
    // whole prefix tile t+NS-2, so their loads come from wave-uniform K and V tile
    // bases (SGPRs) that advance by one tile per step, plus each lane's fixed byte
    // offset; a new page is read from the LDS page list, prefetched one page ahead,
    // when the current one is used up.  Pages hold whole tiles when B is a multiple
    // of the tile (the item's first key is).
    const int t_fast = (B % kTileKeys == 0 && !slot_mode) ? max(0, nfull - (SPLIT ? NS - 1 : NS - 2)) : 0;
    uint64_t fk = 0, fv = 0;     // K and V base of the next streamed tile (head h0)
    uint64_t fv_prev = 0;        // SPLIT: V base of the tile before it (V runs one tile behind K)
    int f_left = 0, f_pidx = 0;  // tiles left in its page; the page's index in `pages`
    int32_t f_next = 0;          // page number at f_pidx + 1
    const uint32_t k_tile_b = kTileKeys * k_key_b, v_tile_b = kTileKeys * v_key_b;
    const uint64_t k_head_u = reinterpret_cast<uint64_t>(uniform_ptr(reinterpret_cast<const void*>(k_head_b)));
    const uint64_t v_head_u = reinterpret_cast<uint64_t>(uniform_ptr(reinterpret_cast<const void*>(v_head_b)));
    uint32_t k_lane_h[HPWL], v_lane_h[HPWL], kv_lane_h[HPWL];
#pragma unroll
    for (int j = 0; j < HPWL; ++j) {
        k_lane_h[j] = k_lane_b + static_cast<uint32_t>(k_hstep_b[j]);
        v_lane_h[j] = v_lane_b + static_cast<uint32_t>(v_hstep_b[j]);
        kv_lane_h[j] = k_wave ? k_lane_h[j] : v_lane_h[j];
    }
    if (t_fast > 0) {
        const uint32_t tile_pos = static_cast<uint32_t>(it.kbeg + kTileKeys * (NS - 2));
        const uint32_t page_abs = pow2 ? (tile_pos >> bshift) : (tile_pos / static_cast<uint32_t>(B));
        const uint32_t off0 = tile_pos - page_abs * static_cast<uint32_t>(B);
        f_pidx = static_cast<int>(page_abs) - page0;
        f_left = static_cast<int>((static_cast<uint32_t>(B) - off0) / kTileKeys);
        const uint32_t page = static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(pages[f_pidx]));
        fk = k_head_u + static_cast<uint64_t>(page) * k_page_b + static_cast<uint64_t>(off0) * k_key_b;
        fv = v_head_u + static_cast<uint64_t>(page) * v_page_b + static_cast<uint64_t>(off0) * v_key_b;
        f_next = pages[min(f_pidx + 1, npages - 1)];
    }
    auto fast_issue_k = [&](auto nt, int stage, int j) {
        if constexpr (decltype(nt)::value) {
            dma_b128_s_nt(k_lane_h[j], reinterpret_cast<const void*>(fk), tile_dst(stage * TILE_SET + j * HD::kTile));
        } else {
            dma_b128_s(k_lane_h[j], reinterpret_cast<const void*>(fk), tile_dst(stage * TILE_SET + j * HD::kTile));
        }
    };
    auto fast_issue_v = [&](auto nt, int stage, int j) {
        const void* base = reinterpret_cast<const void*>(SPLIT ? fv_prev : fv);
        if constexpr (decltype(nt)::value) {
            dma_b128_s_nt(v_lane_h[j], base, tile_dst(V_REGION + stage * TILE_SET + j * HD::kTile));
        } else {
            dma_b128_s(v_lane_h[j], base, tile_dst(V_REGION + stage * TILE_SET + j * HD::kTile));
        }
    };
    // D = 256: part P of this wave's streamed K (or V) keys.
    auto fast_issue_k_part = [&](auto nt, auto part, int stage) {
        constexpr int P = decltype(part)::value;
        if constexpr (decltype(nt)::value) {
            dma_b128_s_nt_o<128 * P>(k_lane_h[0], reinterpret_cast<const void*>(fk),
                                     tile_dst(stage * TILE_SET + P * HD::kPartBytes));
        } else {
            dma_b128_s_o<128 * P>(k_lane_h[0], reinterpret_cast<const void*>(fk),
                                  tile_dst(stage * TILE_SET + P * HD::kPartBytes));
        }
    };
    auto fast_issue_v_part = [&](auto nt, auto part, int stage) {
        constexpr int P = decltype(part)::value;
        const void* base = reinterpret_cast<const void*>(SPLIT ? fv_prev : fv);
        if constexpr (decltype(nt)::value) {
            dma_b128_s_nt_o<128 * P>(v_lane_h[0], base, tile_dst(V_REGION + stage * TILE_SET + P * HD::kPartBytes));
        } else {
            dma_b128_s_o<128 * P>(v_lane_h[0], base, tile_dst(V_REGION + stage * TILE_SET + P * HD::kPartBytes));
        }
    };
    // D = 64: this wave's one streamed load per head and tile, K or V.
    auto fast_issue_kv = [&](auto nt, int stage, int j) {
        const void* base = reinterpret_cast<const void*>(k_wave ? fk : fv);
        if constexpr (decltype(nt)::value) {
            dma_b128_s_nt(kv_lane_h[j], base, tile_dst(stage * TILE_SET + j * HD::kTile));
        } else {
            dma_b128_s(kv_lane_h[j], base, tile_dst(stage * TILE_SET + j * HD::kTile));
        }
    };
    auto fast_advance = [&]() {
        fk += k_tile_b;
        fv += v_tile_b;
        if (--f_left == 0) {
            const uint32_t page = static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(f_next));
            ++f_pidx;
            f_next = pages[min(f_pidx + 1, npages - 1)];
            fk = k_head_u + static_cast<uint64_t>(page) * k_page_b;
            fv = v_head_u + static_cast<uint64_t>(page) * v_page_b;
            f_left = B / kTileKeys;
        }
    };
    // SPLIT: a streamed step stages V of the tile behind the walker and K of the walker's tile,
    // then moves both on; the walker starts at tile NS-1 (the first streamed K).
    auto fast_shift = [&]() {
        fv_prev = fv;
        fast_advance();
    };
    if (SPLIT && t_fast > 0) fast_shift();
    wait_vmcnt<SPLIT ? (NS - 3) * LPT + LPTK : (NS - 3) * LPT>();   // tile 0 staged
    __syncthreads();
    f32x16 s = f32x16{};
    V8 pb_prev[2], pl_prev[2];
    pb_prev[0] = V8{};
    pb_prev[1] = V8{};
    pl_prev[0] = V8{};
    pl_prev[1] = V8{};
    if (wave_active) {
#pragma unroll
        for (int st = 0; st < HD::kSteps; ++st) {
            const V8 a = __builtin_bit_cast(V8, *(const __attribute__((address_space(3))) u32x4*)(lds + k_ofs[st]));
            s = Mfma<T>::run(a, qb[st], s);
        }
        if (nfull == 0) mask_tile(s, 0, 0);
        raise_max(s, true);
    }
    // Fast steps.  Active waves alternate two register sets for the scores and the
    // probabilities (and, for EXACT, the probabilities' remainders) by tile parity (NS is
    // even, so the parity of t is that of b), so no copies between steps; inactive waves
    // only stage their share of the tiles.
    // Long streams that no other item reads (the request's tree fits one node block, and at
    // least 64 streamed tiles) use non-temporal loads: 2 % faster on the long-context batches,
    // whose K/V is read once.  Streams shared with other node blocks stay cacheable in L2
    // for them (non-temporal loads made those 4 % slower), and short streams, which are
    // latency-bound, measured slightly slower non-temporal too.  The exact instance keeps one
    // form (a second one would not fit its registers).
    auto fast_steps = [&](auto nt) {
        if (wave_active) {
            f32x16 sc[2];
            V8 pp[2][2], pq[2][2];
            auto& pr_sets = [&]() -> V8 (&)[2][2] {
                if constexpr (EXACT) return pq; else return pp;
            }();
            sc[0] = s;
            pp[0][0] = pb_prev[0];
            pp[0][1] = pb_prev[1];
            if constexpr (EXACT) {
                pq[0][0] = pl_prev[0];
                pq[0][1] = pl_prev[1];
            }
            for (int t0 = 0; t0 < t_fast; t0 += NS) {
#pragma unroll
                for (int b = 0; b < NS; ++b) {
                    const int t = t0 + b;
                    if (t >= t_fast) break;
                    wait_vmcnt<WAIT_STEP>();
                    __syncthreads();
                    const int ds = (b + NS - 2) % NS;
                    const int dks = SPLIT ? (b + NS - 1) % NS : ds;   // stage of the streamed K
                    auto piece = [&](int sl) {
                        if constexpr (D == 256) {
                            if (sl == 2) fast_issue_v_part(nt, IntTag<0>{}, ds);
                            if (sl == 4) fast_issue_v_part(nt, IntTag<1>{}, ds);
                            if (sl == 6) fast_issue_v_part(nt, IntTag<2>{}, ds);
                            if (sl == 8) fast_issue_v_part(nt, IntTag<3>{}, ds);
                            if (sl == 10) fast_issue_k_part(nt, IntTag<0>{}, dks);
                            if (sl == 12) fast_issue_k_part(nt, IntTag<1>{}, dks);
                            if (sl == 14) fast_issue_k_part(nt, IntTag<2>{}, dks);
                            if (sl == 18) fast_issue_k_part(nt, IntTag<3>{}, dks);
                            if (sl == 24) fast_shift();
                        } else if constexpr (D == 128) {
                            if (HPW == 1) {
                                if (sl == 4) fast_issue_k(nt, ds, 0);
                                if (sl == 8) fast_issue_v(nt, ds, 0);
                            } else {
                                if (sl == 3 || sl == 5) fast_issue_k(nt, ds, (sl - 3) >> 1);
                                if (sl == 7 || sl == 9) fast_issue_v(nt, ds, (sl - 7) >> 1);
                            }
                            if (sl == 12) fast_advance();
                        } else {
                            if (sl == 2 || (HPW == 2 && sl == 4)) fast_issue_kv(nt, ds, (sl - 2) >> 1);
                            if (sl == 6) fast_advance();
                        }
                    };
                    f32x16& s_cur = sc[b & 1];
                    float lt = step(s_cur, sc[(b + 1) & 1], pp[b & 1], pp[(b + 1) & 1], pr_sets[b & 1],
                                    pr_sets[(b + 1) & 1], ((b + 1) % NS) * TILE_SET, ((b + NS - 1) % NS) * TILE_SET,
                                    piece);
                    const bool need = !(lt <= kMaxTileSum);
                    if (__any(need)) {
                        raise_max(s_cur, need);
                        lt = probabilities(s_cur, pp[(b + 1) & 1], pr_sets[(b + 1) & 1]);
                    }
                    l_run += lt;
                }
            }
            const bool odd = t_fast & 1;
            s = odd ? sc[1] : sc[0];
            pb_prev[0] = odd ? pp[1][0] : pp[0][0];
            pb_prev[1] = odd ? pp[1][1] : pp[0][1];
            if constexpr (EXACT) {
                pl_prev[0] = odd ? pq[1][0] : pq[0][0];
                pl_prev[1] = odd ? pq[1][1] : pq[0][1];
            }
        } else {
            for (int t0 = 0; t0 < t_fast; t0 += NS) {
#pragma unroll
                for (int b = 0; b < NS; ++b) {
                    const int t = t0 + b;
                    if (t >= t_fast) break;
                    wait_vmcnt<WAIT_STEP>();
                    __syncthreads();
                    const int ds = (b + NS - 2) % NS;
                    const int dks = SPLIT ? (b + NS - 1) % NS : ds;
                    if constexpr (D == 256) {
                        fast_issue_v_part(nt, IntTag<0>{}, ds);
                        fast_issue_v_part(nt, IntTag<1>{}, ds);
                        fast_issue_v_part(nt, IntTag<2>{}, ds);
                        fast_issue_v_part(nt, IntTag<3>{}, ds);
                        fast_issue_k_part(nt, IntTag<0>{}, dks);
                        fast_issue_k_part(nt, IntTag<1>{}, dks);
                        fast_issue_k_part(nt, IntTag<2>{}, dks);
                        fast_issue_k_part(nt, IntTag<3>{}, dks);
                    } else if constexpr (D == 128) {
#pragma unroll
                        for (int j = 0; j < HPW; ++j) fast_issue_k(nt, dks, j);
#pragma unroll
                        for (int j = 0; j < HPW; ++j) fast_issue_v(nt, ds, j);
                    } else {
#pragma unroll
                        for (int j = 0; j < HPW; ++j) fast_issue_kv(nt, ds, j);
                    }
                    if constexpr (SPLIT) fast_shift(); else fast_advance();
                }
            }
        }
    };
    // D = 256 keeps the cacheable form only: a one-head item's two halves read one K/V stream,
    // and two forms of its loop do not fit the registers.
    if (!EXACT && D != 256 && tn <= NPW && t_fast >= 64) {
        fast_steps(NtTag<!EXACT && D != 256>{});
    } else {
        fast_steps(NtTag<false>{});
    }
    // The remaining steps: masks, partial and tree tiles, general DMA.  SPLIT: the first
    // step stages V of tile t_fast + NS - 2 (its K is staged), so that tile is described here.
    if constexpr (SPLIT) describe(t_fast + NS - 2, fetch(t_fast + NS - 2));
    int pf = fetch(t_fast + (SPLIT ? NS - 1 : NS - 2));
    for (int t0 = t_fast - t_fast % NS; t0 < nt; t0 += NS) {
#pragma unroll
        for (int b = 0; b < NS; ++b) {
            const int t = t0 + b;
            if (t < t_fast) continue;
            if (t >= nt) break;
            wait_vmcnt<WAIT_STEP>();
            __syncthreads();
            // DMA of tile t+NS-2 into the retired stage, spread over the step's slots.  SPLIT
            // (D = 256): V and ancestor words of tile t+NS-2 (described in the previous step) into
            // the stage retired by P.V of tile t-2, then K of tile t+NS-1 into the stage of tile t-1.
            const int ds = (b + NS - 2) % NS;
            const int dks = (b + NS - 1) % NS;
            auto piece = [&](int sl) {
                if constexpr (D == 256) {
                    if (sl == 1) issue_v_part(IntTag<0>{}, ds);
                    if (sl == 3) issue_v_part(IntTag<1>{}, ds);
                    if (sl == 5) issue_v_part(IntTag<2>{}, ds);
                    if (sl == 7) issue_v_part(IntTag<3>{}, ds);
                    if (sl == 8) issue_mask(ds);
                    if (sl == 9) describe(t + NS - 1, pf);
                    if (sl == 11) issue_k_part(IntTag<0>{}, dks);
                    if (sl == 13) issue_k_part(IntTag<1>{}, dks);
                    if (sl == 15) issue_k_part(IntTag<2>{}, dks);
                    if (sl == 17) issue_k_part(IntTag<3>{}, dks);
                    if (sl == 22) pf = fetch(t + NS);
                } else if constexpr (D == 128) {
                    if (sl == 1) describe(t + NS - 2, pf);
                    if (HPW == 1) {
                        if (sl == 4) issue_k(ds, 0);
                        if (sl == 8) issue_v(ds, 0);
                    } else {
                        if (sl == 3 || sl == 5) issue_k(ds, (sl - 3) >> 1);
                        if (sl == 7 || sl == 9) issue_v(ds, (sl - 7) >> 1);
                    }
                    if (sl == 12) issue_mask(ds);
                    if (sl == 13) pf = fetch(t + NS - 1);
                } else {
                    if (sl == 1) describe(t + NS - 2, pf);
                    if (sl == 2 || (HPW == 2 && sl == 4)) issue_kv(ds, (sl - 2) >> 1);
                    if (sl == 5) issue_mask(ds);
                    if (sl == 6) pf = fetch(t + NS - 1);
                }
            };
            if (wave_active) {
                if (t >= nfull && t > 0) mask_tile(s, b, t);
                f32x16 sn;
                V8 pb[2], pl[2];
                float lt = step(s, sn, pb_prev, pb, pl_prev, pl, ((b + 1) % NS) * TILE_SET,
                                ((b + NS - 1) % NS) * TILE_SET, piece);
                const bool need = !(lt <= kMaxTileSum);
                if (__any(need)) {
                    raise_max(s, need);
                    lt = probabilities(s, pb, pl);
                }
                l_run += lt;
                pb_prev[0] = pb[0];
                pb_prev[1] = pb[1];
                if constexpr (EXACT) {
                    pl_prev[0] = pl[0];
                    pl_prev[1] = pl[1];
                }
                s = sn;
            } else {
#pragma unroll
                for (int sl = 0; sl < HD::kSlots; ++sl) piece(sl);
            }
        }
    }
    if (wave_active) {
        // P.V of the last tile.
        const uint32_t vst = static_cast<uint32_t>((nt - 1) % NS) * TILE_SET;
#pragma unroll
        for (int kk = 0; kk < 2; ++kk) {
#pragma unroll
            for (int db = 0; db < HD::kBlocks; ++db) {
                const i16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                    (lds_i16x4*)(lds + v_ofs[db] + vst + (16 * kk) * HD::kPartRow));
                const i16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                    (lds_i16x4*)(lds + v_ofs[db] + vst + (16 * kk + 8) * HD::kPartRow));
                const V8 a = __builtin_bit_cast(V8, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
                acc[db] = Mfma<T>::run(a, pb_prev[kk], acc[db]);
                if constexpr (EXACT) acc[db] = Mfma<T>::run(a, pl_prev[kk], acc[db]);
            }
        }
    }
    wait_vmcnt<0>();  // retire the padding loads before the workgroup ends

    if (!wave_active) return;
    l_run += __shfl_xor(l_run, 32);  // both halves of the row
    if (!row_ok) return;
    const int wr = vw * 32 + c;  // score row within the item
    if (it.slot < 0) {
        const float inv = 1.f / l_run;
        const int64_t row = qbase + node;
#pragma unroll
        for (int db = 0; db < HD::kBlocks; ++db) {
#pragma unroll
            for (int i4 = 0; i4 < 4; ++i4) {
                const f32x4 o = {acc[db][4 * i4] * inv, acc[db][4 * i4 + 1] * inv, acc[db][4 * i4 + 2] * inv,
                                 acc[db][4 * i4 + 3] * inv};
                store_out4<T>(p, row, qh, 32 * db + 8 * i4 + 4 * g, o);
            }
        }
    } else {
        // Partial rows are D floats apart (the merge reads them with the same stride).
        float* wo = p.ws_o + (static_cast<int64_t>(it.slot) * kRowsPerItem + wr) * D;
#pragma unroll
        for (int db = 0; db < HD::kBlocks; ++db) {
#pragma unroll
            for (int i4 = 0; i4 < 4; ++i4) {
                const f32x4 o = {acc[db][4 * i4], acc[db][4 * i4 + 1], acc[db][4 * i4 + 2], acc[db][4 * i4 + 3]};
                *reinterpret_cast<f32x4*>(wo + 32 * db + 8 * i4 + 4 * g) = o;
            }
        }
        if (g == 0) p.ws_ml[static_cast<int64_t>(it.slot) * kRowsPerItem + wr] = make_float2(m_run, l_run);
    }
}

template <typename T, bool EXACT, int G, int D>
__global__ void __launch_bounds__(HeadDim<D>::kThreads)
tree_attention_kernel(const AttnParams p) {
    __shared__ __attribute__((aligned(16))) char smem[kLdsBytes];
    // D = 256: two 4-wave workgroups per work item.  Item i's halves are workgroups
    // 16 * (i / 8) + i % 8 and that + 8: both on XCD i % 8 (workgroup w runs on XCD w % 8),
    // where the planner placed the item, and dispatched close together, so a one-head item's
    // halves share its K/V stream in that XCD's L2.
    int item = static_cast<int>(blockIdx.x), half = 0;
    if constexpr (D == 256) {
        item = (item >> 4) * 8 + (item & 7);
        half = (static_cast<int>(blockIdx.x) >> 3) & 1;
    }
    // A device-built plan launches a capacity grid; workgroups past its item count exit.
    // A plan that overflowed its capacities has no items and reports it here.
    if (p.counts) {
        if (p.counts[3] != 0 && blockIdx.x == 0 && threadIdx.x == 0) set_status(p.status, TV_STATUS_BAD_REQUEST);
        if (item >= p.counts[0]) return;
    } else if (D == 256 && item >= p.num_items) {
        return;
    }
    const int32_t* d = p.items + 8 * static_cast<int64_t>(item);
    const Item it{d[0], d[1], d[2], d[3], d[4], d[5], d[6], d[7]};
    if (it.r < 0 || it.r >= p.num_requests) {
        if (threadIdx.x == 0) set_status(p.status, TV_STATUS_BAD_REQUEST);
        return;
    }
    // The item against the live metadata.  Refused (reported and skipped): an item laid out
    // for another query grouping, a request whose rows fall outside the packed batch, and a
    // chunk past a shrunk prefix (also a stale plan).  Reported only: a plan made before the
    // request grew (host plans read the metadata's host copies), whose last chunk ends before
    // the live prefix length or whose last node block ends before the live node count; the
    // planned keys and rows are still computed, every address in bounds.
    {
        const int tn = p.cnt[it.r], qbase = p.cu[it.r], plen = p.plen[it.r];
        const int npw = (it.hpw == 2 ? 4 : 8) * (32 / G);
        const bool foreign = ((it.flags >> kItemGroupShift) & 0xff) != G || qbase < 0 || tn > p.total_queries - qbase;
        const bool shrunk = it.kend > plen;
        const bool grown = ((it.flags & kItemLastChunk) && it.kend < plen) ||
                           ((it.flags & kItemLastBlock) && it.n0 + npw < tn);
        if (foreign || shrunk || grown) {
            if (threadIdx.x == 0) {
                set_status(p.status, (foreign || shrunk ? TV_STATUS_BAD_REQUEST : 0) |
                                     (shrunk || grown ? TV_STATUS_STALE_PLAN : 0));
            }
            if (foreign || shrunk) return;
        }
    }
    switch (it.hpw) {
        case 1: run_item<T, 1, EXACT, G, D>(p, smem, it, half); break;
        case 2: run_item<T, 2, EXACT, G, D>(p, smem, it, half); break;
        default:
            if (threadIdx.x == 0) set_status(p.status, TV_STATUS_BAD_REQUEST);
            break;
    }
}

template <int G, int D = 128>
int launch_group(const AttnParams& p, int32_t num_items, bool bf16, bool exact, hipStream_t s) {
    typedef HeadDim<D> HD;
    // D = 256: both halves of every item, on a grid of whole 16-workgroup windows.
    const uint32_t grid = D == 256 ? static_cast<uint32_t>((num_items + 7) / 8) * 16u : static_cast<uint32_t>(num_items);
    if (bf16) {
        if (exact) {
            hipLaunchKernelGGL((tree_attention_kernel<__bf16, true, G, D>), dim3(grid), dim3(HD::kThreads), 0, s, p);
        } else {
            hipLaunchKernelGGL((tree_attention_kernel<__bf16, false, G, D>), dim3(grid), dim3(HD::kThreads), 0, s, p);
        }
    } else {
        if (exact) {
            hipLaunchKernelGGL((tree_attention_kernel<_Float16, true, G, D>), dim3(grid), dim3(HD::kThreads), 0, s, p);
        } else {
            hipLaunchKernelGGL((tree_attention_kernel<_Float16, false, G, D>), dim3(grid), dim3(HD::kThreads), 0, s, p);
        }
    }
    return TV_OK;   // the caller reads the launch status (check_launch)
}

}  // namespace
}  // namespace tv
