// Slot-mapped KV append and accepted-only KV commit for gfx950.
//
// Both operations are pure byte movement of 2 KiB slot rows (8 KV heads x 128 dims
// x bf16 at the served geometry), so the kernels are written for HBM efficiency:
// 16-byte vector loads and stores, every load of a row issued before its stores,
// and no arithmetic beyond address generation.  Bit-exactness is by construction.
#include <stdint.h>

#include "tv_internal.h"

namespace tv {
namespace {

// ------------------------------------------------------------------ store_kvcache
// layers/attention.py:15-35: program idx copies key/value row idx to cache row
// slot_mapping[idx] unless the slot is -1.  Here one workgroup handles one row
// per iteration; its threads cover the row in `Unit`-byte pieces.
template <typename Unit>
__global__ void __launch_bounds__(256)
store_kvcache_kernel(const char* __restrict__ key, int64_t key_stride_b,
                     const char* __restrict__ value, int64_t value_stride_b,
                     char* __restrict__ k_cache, char* __restrict__ v_cache,
                     int64_t num_slots, const void* __restrict__ slots, int slot_is_int64,
                     int64_t num_rows, int32_t units_per_row, int32_t* status) {
    const int64_t row_bytes = static_cast<int64_t>(units_per_row) * sizeof(Unit);
    for (int64_t row = blockIdx.x; row < num_rows; row += gridDim.x) {
        const char* ksrc = key + row * key_stride_b;
        const char* vsrc = value + row * value_stride_b;
        // The row's first piece is loaded together with its slot (the key/value rows do
        // not depend on it), so the slot lookup is not a round trip of its own.
        const int32_t u0 = threadIdx.x;
        Unit kv0{}, vv0{};
        if (u0 < units_per_row) {
            kv0 = reinterpret_cast<const Unit*>(ksrc)[u0];
            vv0 = reinterpret_cast<const Unit*>(vsrc)[u0];
        }
        const int64_t slot = slot_is_int64 ? static_cast<const int64_t*>(slots)[row]
                                           : static_cast<int64_t>(static_cast<const int32_t*>(slots)[row]);
        if (slot == -1) continue;
        if (slot < 0 || slot >= num_slots) {
            if (threadIdx.x == 0) set_status(status, TV_STATUS_BAD_SLOT);
            continue;
        }
        char* kdst = k_cache + slot * row_bytes;
        char* vdst = v_cache + slot * row_bytes;
        if (u0 < units_per_row) {
            reinterpret_cast<Unit*>(kdst)[u0] = kv0;
            reinterpret_cast<Unit*>(vdst)[u0] = vv0;
        }
        for (int32_t u = u0 + blockDim.x; u < units_per_row; u += blockDim.x) {
            const Unit kv = reinterpret_cast<const Unit*>(ksrc)[u];
            const Unit vv = reinterpret_cast<const Unit*>(vsrc)[u];
            reinterpret_cast<Unit*>(kdst)[u] = kv;
            reinterpret_cast<Unit*>(vdst)[u] = vv;
        }
    }
}

// --------------------------------------------------------------- copy_accepted_kv
// state.py:80-85 gathers pool[:, :, src] into a temporary and then scatters it to
// pool[:, :, dst], so an overlap between the two slot sets is well defined.  The
// served callers never overlap (scratch arena pages vs owned/pending pages,
// state.py:687-688), so the fast path copies rows directly and only an actual
// overlap takes the staged path:
//   1. commit_check:   per 256 destinations, OR of {overlap with any source,
//                      out-of-range slot}; one flag word per workgroup, always
//                      written, so the workspace needs no clearing.  Sources go
//                      into a hash set in LDS (up to 8192 slots), else tiles of
//                      them are scanned.
//   2. commit_move:    no flag -> every workgroup copies its rows of two (K/V,
//                      layer) planes directly, up to 16 of a thread's loads in
//                      flight before its stores; overlap alone -> workgroup 0 gathers
//                      every row into the workspace, synchronises, and scatters
//                      them (the reference's order; never taken by the served
//                      callers); an invalid slot -> nothing is written.
// Up to kFusedMaxSlots slots (typical served rounds) take one launch instead,
// commit_fused_kernel, which does the same per row without the flag pass.

constexpr int kCheckThreads = 256;
constexpr int kSrcTile = 1024;
constexpr int kFlagOverlap = 1;
constexpr int kFlagInvalid = 2;

__global__ void __launch_bounds__(kCheckThreads)
commit_check_kernel(const int64_t* __restrict__ src, const int64_t* __restrict__ dst,
                    int64_t n, int64_t pool_slots, int32_t* __restrict__ flags,
                    int32_t* status) {
    __shared__ int64_t tile[kSrcTile];
    __shared__ int32_t block_flag;
    if (threadIdx.x == 0) block_flag = 0;
    const int64_t j = static_cast<int64_t>(blockIdx.x) * kCheckThreads + threadIdx.x;
    int32_t flag = 0;
    int64_t d = -1;
    if (j < n) {
        d = dst[j];
        const int64_t s = src[j];
        if (d < 0 || d >= pool_slots || s < 0 || s >= pool_slots) flag |= kFlagInvalid;
    }
    for (int64_t base = 0; base < n; base += kSrcTile) {
        const int64_t count = (n - base < kSrcTile) ? (n - base) : kSrcTile;
        __syncthreads();
        for (int64_t k = threadIdx.x; k < count; k += kCheckThreads) tile[k] = src[base + k];
        __syncthreads();
        if (j < n) {
            for (int64_t k = 0; k < count; ++k) {
                if (tile[k] == d) flag |= kFlagOverlap;
            }
        }
    }
    if (flag) atomicOr(&block_flag, flag);
    __syncthreads();
    if (threadIdx.x == 0) {
        flags[blockIdx.x] = block_flag;
        if (block_flag & kFlagInvalid) set_status(status, TV_STATUS_BAD_SLOT);
    }
}

// The same flags in O(n) per workgroup for up to kCheckHashMax slots of a pool of fewer than
// 2^31 slots: every workgroup puts all sources into an open-addressing set in LDS and probes
// its 256 destinations (the tiled scan above compares each destination with every source,
// n compares per thread: about 25 us at 4096 slots).
constexpr int kCheckHash = 16384;                  // set entries (64 KB of LDS), load <= 1/2
constexpr int64_t kCheckHashMax = kCheckHash / 2;

__device__ __forceinline__ uint32_t check_hash(int32_t v) {
    return (static_cast<uint32_t>(v) * 2654435761u) >> (32 - 14);   // 14 bits: kCheckHash entries
}
static_assert(kCheckHash == 1 << 14, "check_hash takes 14 bits");

__global__ void __launch_bounds__(kCheckThreads)
commit_check_hash_kernel(const int64_t* __restrict__ src, const int64_t* __restrict__ dst, int64_t n,
                         int64_t pool_slots, int32_t* __restrict__ flags, int32_t* status) {
    __shared__ int32_t table[kCheckHash];
    __shared__ int32_t block_flag;
    if (threadIdx.x == 0) block_flag = 0;
    for (int k = threadIdx.x; k < kCheckHash; k += kCheckThreads) table[k] = -1;
    const int64_t j = static_cast<int64_t>(blockIdx.x) * kCheckThreads + threadIdx.x;
    int32_t flag = 0;
    int64_t d = -1;
    if (j < n) {
        d = dst[j];
        const int64_t s = src[j];
        if (d < 0 || d >= pool_slots || s < 0 || s >= pool_slots) flag |= kFlagInvalid;
    }
    __syncthreads();
    for (int64_t k = threadIdx.x; k < n; k += kCheckThreads) {
        const int64_t v = src[k];
        if (v < 0 || v >= pool_slots) continue;   // reported by its own workgroup
        uint32_t h = check_hash(static_cast<int32_t>(v));
        while (true) {
            const int32_t prev = atomicCAS(&table[h], -1, static_cast<int32_t>(v));
            if (prev == -1 || prev == static_cast<int32_t>(v)) break;
            h = (h + 1) & (kCheckHash - 1);
        }
    }
    __syncthreads();
    if (j < n && !(flag & kFlagInvalid)) {
        uint32_t h = check_hash(static_cast<int32_t>(d));
        while (true) {
            const int32_t e = table[h];
            if (e == static_cast<int32_t>(d)) {
                flag |= kFlagOverlap;
                break;
            }
            if (e == -1) break;
            h = (h + 1) & (kCheckHash - 1);
        }
    }
    if (flag) atomicOr(&block_flag, flag);
    __syncthreads();
    if (threadIdx.x == 0) {
        flags[blockIdx.x] = block_flag;
        if (block_flag & kFlagInvalid) set_status(status, TV_STATUS_BAD_SLOT);
    }
}

__device__ __forceinline__ int32_t read_flags(const int32_t* flags, int32_t num_flags) {
    __shared__ int32_t combined;
    if (threadIdx.x == 0) combined = 0;
    __syncthreads();
    int32_t f = 0;
    for (int32_t k = threadIdx.x; k < num_flags; k += blockDim.x) f |= flags[k];
    if (f) atomicOr(&combined, f);
    __syncthreads();
    return combined;
}

struct PoolGeom {
    char* base;
    int64_t s_kv, s_layer, s_block, s_off;  // bytes
    int64_t layers, block_size, n;
    int32_t units_per_row;
};

__device__ __forceinline__ char* slot_row(const PoolGeom& g, int64_t kv, int64_t layer, int64_t slot) {
    const int64_t block = slot / g.block_size;
    const int64_t off = slot - block * g.block_size;
    return g.base + kv * g.s_kv + layer * g.s_layer + block * g.s_block + off * g.s_off;
}

constexpr int kMoveRows = 8;        // slot rows per workgroup
// (K/V, layer) planes per move workgroup, copied back to back: 2 measured fastest above 512
// slots (cold caches: 4096 slots 289 -> 244 us, 1848 slots 129 -> 113 us, against 1 plane;
// 8 and 16 planes 244-248 and 116-120 us).
constexpr int kMovePlanes = 2;
constexpr int kMoveThreads = 256;
constexpr int kMoveUnroll = 16;     // units a thread keeps in flight (16 B each at most)

// Byte offset of `slot`'s row within a (K/V, layer) plane.
__device__ __forceinline__ int64_t slot_offset(const PoolGeom& g, int64_t slot) {
    const int64_t block = slot / g.block_size;
    const int64_t off = slot - block * g.block_size;
    return block * g.s_block + off * g.s_off;
}

// Direct copy of up to kMoveRows rows whose byte offsets within a plane are in LDS, in
// planes plane0 .. plane0 + nplanes - 1; rows whose bit is set in `skip` are left alone.
// Every thread issues up to kMoveUnroll loads before its stores, and one workgroup's rows
// of several planes share the slot lookups, so a plane's rows cost no round trip of their
// own.
// One plane's rows (the one-launch commit's copiers): the plane base once, 8 loads in flight
// per thread.  A separate form from copy_rows keeps these small workgroups at 58 VGPRs (8 waves
// per SIMD); the multi-plane form takes 76 here and measured 2-3 us slower on config 3.
template <typename Unit>
__device__ __forceinline__ void copy_plane_rows(const PoolGeom& g, int32_t plane, const int64_t* row_src,
                                                const int64_t* row_dst, int32_t nrows, uint32_t skip) {
    constexpr int kUnroll = 8;
    char* base = g.base + (plane / g.layers) * g.s_kv + (plane % g.layers) * g.s_layer;
    const int32_t upr = g.units_per_row;
    const int32_t total = nrows * upr;
    for (int32_t u0 = 0; u0 < total; u0 += kMoveThreads * kUnroll) {
        Unit v[kUnroll];
#pragma unroll
        for (int k = 0; k < kUnroll; ++k) {
            const int32_t u = u0 + k * kMoveThreads + threadIdx.x;
            if (u < total) {
                const int32_t r = u / upr, c = u - r * upr;
                if (!((skip >> r) & 1u)) v[k] = reinterpret_cast<const Unit*>(base + row_src[r])[c];
            }
        }
#pragma unroll
        for (int k = 0; k < kUnroll; ++k) {
            const int32_t u = u0 + k * kMoveThreads + threadIdx.x;
            if (u < total) {
                const int32_t r = u / upr, c = u - r * upr;
                if (!((skip >> r) & 1u)) reinterpret_cast<Unit*>(base + row_dst[r])[c] = v[k];
            }
        }
    }
}

template <typename Unit, int UNROLL, int MAXP>
__device__ __forceinline__ void copy_rows(const PoolGeom& g, int32_t plane0, int32_t nplanes, const int64_t* row_src,
                                          const int64_t* row_dst, int32_t nrows, uint32_t skip) {
    // Plane bases once per workgroup (a plane is (K/V, layer)); the unit loop divides only
    // 32-bit unit indices.
    char* pbase[MAXP];
#pragma unroll
    for (int q = 0; q < MAXP; ++q) {
        const int64_t plane = plane0 + (q < nplanes ? q : nplanes - 1);
        pbase[q] = g.base + (plane / g.layers) * g.s_kv + (plane % g.layers) * g.s_layer;
    }
    const uint32_t upr = static_cast<uint32_t>(g.units_per_row);
    const uint32_t per_plane = static_cast<uint32_t>(nrows) * upr;
    const uint32_t total = per_plane * static_cast<uint32_t>(nplanes);
    auto unit_at = [&](uint32_t u, uint32_t& r, uint32_t& c) -> char* {
        const uint32_t pl = MAXP == 1 ? 0u : u / per_plane;
        const uint32_t w = u - pl * per_plane;
        r = w / upr;
        c = w - r * upr;
        char* base = pbase[0];
#pragma unroll
        for (int q = 1; q < MAXP; ++q) base = pl == static_cast<uint32_t>(q) ? pbase[q] : base;
        return base;
    };
    for (uint32_t u0 = 0; u0 < total; u0 += kMoveThreads * UNROLL) {
        Unit v[UNROLL];
#pragma unroll
        for (int k = 0; k < UNROLL; ++k) {
            const uint32_t u = u0 + k * kMoveThreads + threadIdx.x;
            if (u < total) {
                uint32_t r, c;
                const char* base = unit_at(u, r, c);
                if (!((skip >> r) & 1u)) v[k] = reinterpret_cast<const Unit*>(base + row_src[r])[c];
            }
        }
#pragma unroll
        for (int k = 0; k < UNROLL; ++k) {
            const uint32_t u = u0 + k * kMoveThreads + threadIdx.x;
            if (u < total) {
                uint32_t r, c;
                char* base = unit_at(u, r, c);
                if (!((skip >> r) & 1u)) reinterpret_cast<Unit*>(base + row_dst[r])[c] = v[k];
            }
        }
    }
}

// Grid (ceil(n / kMoveRows), ceil(2 * layers / kMovePlanes)).  Runs after commit_check on
// the same stream.
template <typename Unit>
__global__ void __launch_bounds__(kMoveThreads)
commit_move_kernel(PoolGeom g, const int64_t* __restrict__ src, const int64_t* __restrict__ dst,
                   const int32_t* __restrict__ flags, int32_t num_flags, Unit* __restrict__ staging) {
    // This workgroup's row slots are loaded together with the flag words (one round trip
    // before the copy, not two).
    const int64_t i0 = static_cast<int64_t>(blockIdx.x) * kMoveRows;
    const int32_t nrows = static_cast<int32_t>(g.n - i0 < kMoveRows ? g.n - i0 : kMoveRows);
    int64_t my_src = 0, my_dst = 0;
    if (threadIdx.x < nrows) {
        my_src = src[i0 + threadIdx.x];
        my_dst = dst[i0 + threadIdx.x];
    }
    const int32_t f = read_flags(flags, num_flags);
    if (f & kFlagInvalid) return;
    const int32_t upr = g.units_per_row;
    if (f == kFlagOverlap) {
        // Gather every row into the workspace, then scatter: one workgroup, so the
        // barrier orders all reads before all writes.
        if (blockIdx.x != 0 || blockIdx.y != 0) return;
        const int64_t rows = 2 * g.layers * g.n;
        for (int64_t u = threadIdx.x; u < rows * upr; u += kMoveThreads) {
            const int64_t row = u / upr, i = row % g.n, plane = row / g.n;
            const char* base = g.base + (plane / g.layers) * g.s_kv + (plane % g.layers) * g.s_layer;
            staging[u] = reinterpret_cast<const Unit*>(base + slot_offset(g, src[i]))[u % upr];
        }
        __syncthreads();
        for (int64_t u = threadIdx.x; u < rows * upr; u += kMoveThreads) {
            const int64_t row = u / upr, i = row % g.n, plane = row / g.n;
            char* base = g.base + (plane / g.layers) * g.s_kv + (plane % g.layers) * g.s_layer;
            reinterpret_cast<Unit*>(base + slot_offset(g, dst[i]))[u % upr] = staging[u];
        }
        return;
    }
    __shared__ int64_t row_src[kMoveRows], row_dst[kMoveRows];
    const int32_t plane0 = blockIdx.y * kMovePlanes;
    const int32_t nplanes = static_cast<int32_t>(2 * g.layers - plane0 < kMovePlanes ? 2 * g.layers - plane0 : kMovePlanes);
    if (threadIdx.x < nrows) {
        row_src[threadIdx.x] = slot_offset(g, my_src);
        row_dst[threadIdx.x] = slot_offset(g, my_dst);
    }
    __syncthreads();
    copy_rows<Unit, kMoveUnroll, kMovePlanes>(g, plane0, nplanes, row_src, row_dst, nrows, 0u);
}

// One-launch commit for up to kFusedMaxSlots slots.  Row i is "dirty" when its
// source is some row's destination or its destination some row's source; a clean
// row's source is never written and its destination never read by any row, so it
// can be copied directly whatever the other rows do.  Workgroups (x >= 1, y) copy
// the clean rows among rows R(x-1)..R(x-1)+R-1 of plane y (R = kFusedRows); workgroup
// (0, 0) finds the dirty rows and moves them through the workspace (gather all,
// barrier, scatter all), the reference's order.  Every workgroup validates every slot
// first, so an invalid map writes nothing anywhere.  Each copy workgroup tests its R rows
// against every slot (R n compares, its share of the n slots loaded once), so the one-launch form
// is kept to n <= 512, where that costs less than a second launch; larger batches take
// commit_check + commit_move.
constexpr int64_t kFusedMaxSlots = 512;
// Slot rows of one plane per copier workgroup: 4 (more, smaller workgroups) measured 20.1 us
// against 22.7 us at 8 and 24.3 us at 16 for config 3 with the caches evicted first, and the
// same 15.8 us warm.
constexpr int kFusedRows = 4;
// One (K/V, layer) plane per copier workgroup: 4 and 8 planes per workgroup measured 3.5 and
// 5.8 us slower on config 3 with the caches evicted (fewer, longer workgroups).
constexpr int kFusedHash = 2 * kFusedMaxSlots;   // open-addressing slots per hash set (load <= 1/2)

// Open-addressing set of non-negative 32-bit slots in LDS (empty entries are -1),
// for the dirty-row test in O(n): insert every slot of one list, then probe.
__device__ __forceinline__ uint32_t slot_hash(int32_t v) {
    return (static_cast<uint32_t>(v) * 2654435761u) >> (32 - 10);   // 10 bits: kFusedHash entries
}
static_assert(kFusedHash == 1024, "slot_hash takes 10 bits");

__device__ __forceinline__ void hash_insert(int32_t* table, int32_t v) {
    uint32_t h = slot_hash(v);
    while (true) {
        const int32_t prev = atomicCAS(&table[h], -1, v);
        if (prev == -1 || prev == v) return;
        h = (h + 1) & (kFusedHash - 1);
    }
}

__device__ __forceinline__ bool hash_contains(const int32_t* table, int32_t v) {
    uint32_t h = slot_hash(v);
    while (true) {
        const int32_t e = table[h];
        if (e == v) return true;
        if (e == -1) return false;
        h = (h + 1) & (kFusedHash - 1);
    }
}

template <typename Unit>
__global__ void __launch_bounds__(kMoveThreads)
commit_fused_kernel(PoolGeom g, const int64_t* __restrict__ src, const int64_t* __restrict__ dst,
                    int64_t pool_slots, Unit* __restrict__ staging, int32_t* status) {
    if (blockIdx.x == 0 && blockIdx.y != 0) return;
    const int32_t n = static_cast<int32_t>(g.n);
    if (blockIdx.x == 0) {
        // The dirty-row mover.  The slot lists go to LDS as 32-bit values (the host takes
        // this path only for pools of fewer than 2^31 slots) and into two hash sets, so
        // the dirty test is O(n): row i is dirty iff src[i] is in the destination set or
        // dst[i] in the source set.  About 10 KB of LDS per workgroup still lets a CU
        // hold 8 of them.
        __shared__ int32_t s_src[kFusedMaxSlots], s_dst[kFusedMaxSlots];
        __shared__ int32_t h_src[kFusedHash], h_dst[kFusedHash];
        __shared__ uint8_t dirty[kFusedMaxSlots];
        for (int32_t k = threadIdx.x; k < kFusedHash; k += kMoveThreads) {
            h_src[k] = -1;
            h_dst[k] = -1;
        }
        int bad = 0;
        for (int32_t k = threadIdx.x; k < n; k += kMoveThreads) {
            const int64_t a = src[k], b = dst[k];
            bad |= (a < 0 || a >= pool_slots || b < 0 || b >= pool_slots);
            s_src[k] = static_cast<int32_t>(a);
            s_dst[k] = static_cast<int32_t>(b);
        }
        if (__syncthreads_or(bad)) {
            if (threadIdx.x == 0) set_status(status, TV_STATUS_BAD_SLOT);
            return;
        }
        for (int32_t k = threadIdx.x; k < n; k += kMoveThreads) {
            hash_insert(h_src, s_src[k]);
            hash_insert(h_dst, s_dst[k]);
        }
        __syncthreads();
        int any = 0;
        for (int32_t i = threadIdx.x; i < n; i += kMoveThreads) {
            const int d = hash_contains(h_dst, s_src[i]) || hash_contains(h_src, s_dst[i]);
            dirty[i] = static_cast<uint8_t>(d);
            any |= d;
        }
        if (!__syncthreads_or(any)) return;
        const int32_t upr = g.units_per_row;
        const int64_t rows = 2 * g.layers * g.n;
        for (int64_t u = threadIdx.x; u < rows * upr; u += kMoveThreads) {
            const int64_t row = u / upr, i = row % g.n, plane = row / g.n;
            if (!dirty[i]) continue;
            const char* base = g.base + (plane / g.layers) * g.s_kv + (plane % g.layers) * g.s_layer;
            staging[u] = reinterpret_cast<const Unit*>(base + slot_offset(g, src[i]))[u % upr];
        }
        __syncthreads();
        for (int64_t u = threadIdx.x; u < rows * upr; u += kMoveThreads) {
            const int64_t row = u / upr, i = row % g.n, plane = row / g.n;
            if (!dirty[i]) continue;
            char* base = g.base + (plane / g.layers) * g.s_kv + (plane % g.layers) * g.s_layer;
            reinterpret_cast<Unit*>(base + slot_offset(g, dst[i]))[u % upr] = staging[u];
        }
        return;
    }
    // Clean-row copier for rows i0..i0+nrows-1 of plane blockIdx.y.  Its own rows'
    // slots and this thread's share of all slots are loaded together, so validity and
    // dirtiness cost one round trip before the copy.
    __shared__ int64_t row_src[kFusedRows], row_dst[kFusedRows];
    __shared__ uint32_t skip;
    const int32_t i0 = (blockIdx.x - 1) * kFusedRows;
    const int32_t nrows = n - i0 < kFusedRows ? n - i0 : kFusedRows;
    int64_t my_s[kFusedRows], my_d[kFusedRows];
#pragma unroll
    for (int r = 0; r < kFusedRows; ++r) {
        my_s[r] = r < nrows ? src[i0 + r] : -1;
        my_d[r] = r < nrows ? dst[i0 + r] : -1;
    }
    if (threadIdx.x == 0) skip = 0u;
    int bad = 0;
    uint32_t mine = 0u;
    for (int32_t k = threadIdx.x; k < n; k += kMoveThreads) {
        const int64_t a = src[k], b = dst[k];
        bad |= (a < 0 || a >= pool_slots || b < 0 || b >= pool_slots);
#pragma unroll
        for (int r = 0; r < kFusedRows; ++r) {
            if (r < nrows && (my_s[r] == b || my_d[r] == a)) mine |= 1u << r;
        }
    }
    if (threadIdx.x < nrows) {
        row_src[threadIdx.x] = slot_offset(g, my_s[threadIdx.x]);
        row_dst[threadIdx.x] = slot_offset(g, my_d[threadIdx.x]);
    }
    __syncthreads();
    if (mine) atomicOr(&skip, mine);
    if (__syncthreads_or(bad)) return;
    copy_plane_rows<Unit>(g, blockIdx.y, row_src, row_dst, nrows, skip);
}

template <typename Unit>
int launch_commit(const PoolGeom& g, const int64_t* src, const int64_t* dst, int32_t* flags,
                  int32_t num_flags, void* staging, hipStream_t stream) {
    const int64_t groups = (g.n + kMoveRows - 1) / kMoveRows;
    const int64_t planes = (2 * g.layers + kMovePlanes - 1) / kMovePlanes;
    if (groups > 0x7fffffff || planes > 65535) {
        return fail(TV_ERR_UNSUPPORTED, "copy_accepted_kv: %lld slots x %lld layers exceed the launch grid",
                    (long long)g.n, (long long)g.layers);
    }
    hipLaunchKernelGGL((commit_move_kernel<Unit>), dim3(static_cast<uint32_t>(groups), static_cast<uint32_t>(planes)),
                       dim3(kMoveThreads), 0, stream, g, src, dst, flags, num_flags, static_cast<Unit*>(staging));
    return check_launch("copy_accepted_kv");
}

int unit_for(int64_t alignment_bytes) {
    if (alignment_bytes % 16 == 0) return 16;
    if (alignment_bytes % 8 == 0) return 8;
    if (alignment_bytes % 4 == 0) return 4;
    if (alignment_bytes % 2 == 0) return 2;
    return 1;
}

int64_t gcd64(int64_t a, int64_t b) {
    a = a < 0 ? -a : a;
    b = b < 0 ? -b : b;
    while (b) {
        const int64_t t = a % b;
        a = b;
        b = t;
    }
    return a;
}

int64_t num_flag_words(int64_t n) { return (n + kCheckThreads - 1) / kCheckThreads; }

// ------------------------------------------------------------------ commit slots
// state.py:746-798 builds each request's commit maps on the host: the sources are its
// accepted tree nodes' scratch slots (nodes.index_select(0, path), :780) and the
// destinations the next len(path) canonical slots after cache_len through its owned +
// pending pages (_slots_for_blocks, :54-61, :782-785), one host-to-device copy per
// request.  Here one 64-lane wave per request builds both for the whole batch.  A path
// that is empty, does not start at the root, repeats a node or names a node outside its tree, or
// a destination beyond the request's table row or outside the pool, marks the request
// bad: its rows get -1 (copy_accepted_kv then writes nothing) and a status bit is set.
constexpr int kSlotWaves = 4;

__global__ void __launch_bounds__(64 * kSlotWaves)
commit_slots_kernel(const int64_t* __restrict__ tree_slots, const int32_t* __restrict__ cu,
                    const int32_t* __restrict__ paths, const int32_t* __restrict__ path_off,
                    const int32_t* __restrict__ tables, int64_t table_stride, int32_t table_width,
                    const int32_t* __restrict__ cache_lens, int32_t num_requests, int32_t block_size,
                    int64_t num_blocks, int64_t* __restrict__ src, int64_t* __restrict__ dst, int32_t* status) {
    const int r = blockIdx.x * kSlotWaves + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (r >= num_requests) return;
    const int32_t begin = path_off[r], end = path_off[r + 1];
    const int32_t q0 = cu[r], nodes = cu[r + 1] - q0;
    const int64_t cache_len = cache_lens[r];
    bool bad = begin >= end || nodes < 1 || cache_len < 0;
    if (!bad && paths[begin] != 0) bad = true;
    for (int32_t i = begin + lane; !bad && i < end; i += 64) {
        const int32_t node = paths[i];
        bool b = node < 0 || node >= nodes;
        for (int32_t j = begin; j < i && !b; ++j) b = paths[j] == node;
        const int64_t pos = cache_len + (i - begin);
        const int64_t page_index = pos / block_size;
        if (page_index >= table_width) {
            b = true;
        } else {
            const int64_t page = tables[static_cast<int64_t>(r) * table_stride + page_index];
            b = b || page < 0 || page >= num_blocks;
        }
        bad = bad || b;
    }
    bad = __any(bad);
    if (bad && lane == 0) set_status(status, TV_STATUS_BAD_SLOT);
    for (int32_t i = begin + lane; i < end; i += 64) {
        if (bad) {
            src[i] = -1;
            dst[i] = -1;
            continue;
        }
        const int64_t pos = cache_len + (i - begin);
        const int64_t page = tables[static_cast<int64_t>(r) * table_stride + pos / block_size];
        src[i] = tree_slots[q0 + paths[i]];
        dst[i] = page * block_size + pos % block_size;
    }
}

}  // namespace
}  // namespace tv

using namespace tv;

extern "C" int tv_store_kvcache(const void* key, int64_t key_row_stride, const void* value,
                                int64_t value_row_stride, void* k_cache, void* v_cache,
                                int64_t num_cache_slots, const void* slot_mapping,
                                int32_t slot_is_int64, int64_t num_rows, int64_t row_elems,
                                int32_t elem_bytes, int32_t* status, void* stream) {
    clear_error();
    if (num_rows < 0 || row_elems <= 0 || num_cache_slots < 0) {
        return fail(TV_ERR_INVALID, "store_kvcache: invalid sizes rows=%lld row_elems=%lld",
                    (long long)num_rows, (long long)row_elems);
    }
    if (elem_bytes != 1 && elem_bytes != 2 && elem_bytes != 4 && elem_bytes != 8) {
        return fail(TV_ERR_INVALID, "store_kvcache: element size %d", elem_bytes);
    }
    if (num_rows == 0) return TV_OK;
    if (!key || !value || !k_cache || !v_cache || !slot_mapping) {
        return fail(TV_ERR_INVALID, "store_kvcache: null pointer");
    }
    const int64_t row_bytes = row_elems * elem_bytes;
    int64_t align = gcd64(row_bytes, gcd64(key_row_stride * elem_bytes, value_row_stride * elem_bytes));
    align = gcd64(align, static_cast<int64_t>(reinterpret_cast<uintptr_t>(key) | reinterpret_cast<uintptr_t>(value) |
                                              reinterpret_cast<uintptr_t>(k_cache) |
                                              reinterpret_cast<uintptr_t>(v_cache)) | 16);
    if (align == 0) align = 16;
    const int unit = unit_for(align);
    const int32_t units = static_cast<int32_t>(row_bytes / unit);
    int threads = 64;
    while (threads < units && threads < 256) threads *= 2;
    int64_t blocks = num_rows < 65536 ? num_rows : 65536;
    hipStream_t s = as_stream(stream);
    const char* k = static_cast<const char*>(key);
    const char* v = static_cast<const char*>(value);
    char* kc = static_cast<char*>(k_cache);
    char* vc = static_cast<char*>(v_cache);
    const int64_t ks = key_row_stride * elem_bytes, vs = value_row_stride * elem_bytes;
    switch (unit) {
        case 16:
            hipLaunchKernelGGL(store_kvcache_kernel<u32x4>, dim3(blocks), dim3(threads), 0, s, k, ks, v, vs,
                               kc, vc, num_cache_slots, slot_mapping, slot_is_int64, num_rows, units, status);
            break;
        case 8:
            hipLaunchKernelGGL(store_kvcache_kernel<u32x2>, dim3(blocks), dim3(threads), 0, s, k, ks, v, vs,
                               kc, vc, num_cache_slots, slot_mapping, slot_is_int64, num_rows, units, status);
            break;
        case 4:
            hipLaunchKernelGGL(store_kvcache_kernel<uint32_t>, dim3(blocks), dim3(threads), 0, s, k, ks, v, vs,
                               kc, vc, num_cache_slots, slot_mapping, slot_is_int64, num_rows, units, status);
            break;
        case 2:
            hipLaunchKernelGGL(store_kvcache_kernel<uint16_t>, dim3(blocks), dim3(threads), 0, s, k, ks, v, vs,
                               kc, vc, num_cache_slots, slot_mapping, slot_is_int64, num_rows, units, status);
            break;
        default:
            hipLaunchKernelGGL(store_kvcache_kernel<uint8_t>, dim3(blocks), dim3(threads), 0, s, k, ks, v, vs,
                               kc, vc, num_cache_slots, slot_mapping, slot_is_int64, num_rows, units, status);
            break;
    }
    return check_launch("store_kvcache");
}

extern "C" int64_t tv_copy_accepted_kv_workspace_bytes(int64_t num_slots, int64_t num_layers,
                                                       int64_t row_elems, int32_t elem_bytes) {
    if (num_slots <= 0 || num_layers <= 0 || row_elems <= 0 || elem_bytes <= 0) return 0;
    const int64_t flag_bytes = ((num_flag_words(num_slots) * 4 + 255) / 256) * 256;
    return flag_bytes + 2 * num_layers * num_slots * row_elems * elem_bytes;
}

extern "C" int tv_copy_accepted_kv(void* kv_pool, const int64_t pool_shape[6], const int64_t pool_stride[6],
                                   int32_t elem_bytes, const int64_t* source_slots,
                                   const int64_t* destination_slots, int64_t num_slots, void* workspace,
                                   int64_t workspace_bytes, int64_t* payload_bytes_host, int32_t* status,
                                   void* stream) {
    clear_error();
    if (!pool_shape || !pool_stride) return fail(TV_ERR_INVALID, "copy_accepted_kv: null geometry");
    if (pool_shape[0] != 2) return fail(TV_ERR_INVALID, "copy_accepted_kv: pool axis 0 must be 2 (K, V)");
    for (int d = 0; d < 6; ++d) {
        if (pool_shape[d] <= 0) return fail(TV_ERR_INVALID, "copy_accepted_kv: empty pool axis %d", d);
        if (pool_stride[d] < 0) return fail(TV_ERR_INVALID, "copy_accepted_kv: negative stride %d", d);
    }
    if (pool_stride[5] != 1 || pool_stride[4] != pool_shape[5]) {
        return fail(TV_ERR_UNSUPPORTED, "copy_accepted_kv: a slot row [heads, dim] must be dense");
    }
    if (num_slots < 0) return fail(TV_ERR_INVALID, "copy_accepted_kv: negative slot count");
    const int64_t layers = pool_shape[1];
    const int64_t row_elems = pool_shape[4] * pool_shape[5];
    const int64_t payload = 2 * layers * num_slots * row_elems * elem_bytes;
    if (num_slots == 0) {
        if (payload_bytes_host) *payload_bytes_host = 0;
        return TV_OK;
    }
    if (!kv_pool || !source_slots || !destination_slots || !workspace) {
        return fail(TV_ERR_INVALID, "copy_accepted_kv: null pointer");
    }
    const int64_t need = tv_copy_accepted_kv_workspace_bytes(num_slots, layers, row_elems, elem_bytes);
    if (workspace_bytes < need) {
        return fail(TV_ERR_CAPACITY, "copy_accepted_kv: workspace %lld < %lld bytes", (long long)workspace_bytes,
                    (long long)need);
    }
    PoolGeom g;
    g.base = static_cast<char*>(kv_pool);
    g.s_kv = pool_stride[0] * elem_bytes;
    g.s_layer = pool_stride[1] * elem_bytes;
    g.s_block = pool_stride[2] * elem_bytes;
    g.s_off = pool_stride[3] * elem_bytes;
    g.layers = layers;
    g.block_size = pool_shape[3];
    g.n = num_slots;
    const int64_t row_bytes = row_elems * elem_bytes;
    int64_t align = gcd64(row_bytes, gcd64(g.s_kv, gcd64(g.s_layer, gcd64(g.s_block, g.s_off))));
    align = gcd64(align, static_cast<int64_t>(reinterpret_cast<uintptr_t>(kv_pool) | 16));
    const int unit = unit_for(align);
    g.units_per_row = static_cast<int32_t>(row_bytes / unit);
    const int64_t pool_slots = pool_shape[2] * pool_shape[3];
    const int32_t nflags = static_cast<int32_t>(num_flag_words(num_slots));
    int32_t* flags = static_cast<int32_t*>(workspace);
    const int64_t flag_bytes = ((static_cast<int64_t>(nflags) * 4 + 255) / 256) * 256;
    void* staging = static_cast<char*>(workspace) + flag_bytes;
    hipStream_t s = as_stream(stream);
    int rc;
    if (num_slots <= kFusedMaxSlots && 2 * layers <= 65535 && pool_slots < (int64_t{1} << 31)) {
        const dim3 grid(static_cast<uint32_t>((num_slots + kFusedRows - 1) / kFusedRows + 1),
                        static_cast<uint32_t>(2 * layers));
        switch (unit) {
            case 16: hipLaunchKernelGGL(commit_fused_kernel<u32x4>, grid, dim3(kMoveThreads), 0, s, g, source_slots,
                                        destination_slots, pool_slots, static_cast<u32x4*>(staging), status); break;
            case 8: hipLaunchKernelGGL(commit_fused_kernel<u32x2>, grid, dim3(kMoveThreads), 0, s, g, source_slots,
                                       destination_slots, pool_slots, static_cast<u32x2*>(staging), status); break;
            case 4: hipLaunchKernelGGL(commit_fused_kernel<uint32_t>, grid, dim3(kMoveThreads), 0, s, g, source_slots,
                                       destination_slots, pool_slots, static_cast<uint32_t*>(staging), status); break;
            case 2: hipLaunchKernelGGL(commit_fused_kernel<uint16_t>, grid, dim3(kMoveThreads), 0, s, g, source_slots,
                                       destination_slots, pool_slots, static_cast<uint16_t*>(staging), status); break;
            default: hipLaunchKernelGGL(commit_fused_kernel<uint8_t>, grid, dim3(kMoveThreads), 0, s, g, source_slots,
                                        destination_slots, pool_slots, static_cast<uint8_t*>(staging), status); break;
        }
        rc = check_launch("copy_accepted_kv");
        if (rc != TV_OK) return rc;
        if (payload_bytes_host) *payload_bytes_host = payload;
        return TV_OK;
    }
    if (num_slots <= kCheckHashMax && pool_slots < (int64_t{1} << 31)) {
        hipLaunchKernelGGL(commit_check_hash_kernel, dim3(nflags), dim3(kCheckThreads), 0, s, source_slots,
                           destination_slots, num_slots, pool_slots, flags, status);
    } else {
        hipLaunchKernelGGL(commit_check_kernel, dim3(nflags), dim3(kCheckThreads), 0, s, source_slots,
                           destination_slots, num_slots, pool_slots, flags, status);
    }
    switch (unit) {
        case 16: rc = launch_commit<u32x4>(g, source_slots, destination_slots, flags, nflags, staging, s); break;
        case 8: rc = launch_commit<u32x2>(g, source_slots, destination_slots, flags, nflags, staging, s); break;
        case 4: rc = launch_commit<uint32_t>(g, source_slots, destination_slots, flags, nflags, staging, s); break;
        case 2: rc = launch_commit<uint16_t>(g, source_slots, destination_slots, flags, nflags, staging, s); break;
        default: rc = launch_commit<uint8_t>(g, source_slots, destination_slots, flags, nflags, staging, s); break;
    }
    if (rc != TV_OK) return rc;
    if (payload_bytes_host) *payload_bytes_host = payload;
    return TV_OK;
}

extern "C" int tv_commit_slots(const int64_t* tree_slots, const int32_t* cu_seqlens, const int32_t* paths,
                               const int32_t* path_offsets, const int32_t* block_tables, int64_t table_stride,
                               int32_t table_width, const int32_t* cache_lens, int32_t num_requests,
                               int32_t block_size, int64_t num_blocks, int64_t* source_slots,
                               int64_t* destination_slots, int32_t* status, void* stream) {
    clear_error();
    if (num_requests < 0 || block_size < 1 || num_blocks < 1 || table_width < 0 || table_stride < table_width) {
        return fail(TV_ERR_INVALID, "commit_slots: invalid sizes");
    }
    if (num_requests == 0) return TV_OK;
    if (!tree_slots || !cu_seqlens || !paths || !path_offsets || !cache_lens || !source_slots ||
        !destination_slots || (table_width > 0 && !block_tables)) {
        return fail(TV_ERR_INVALID, "commit_slots: null pointer");
    }
    const int64_t blocks = (static_cast<int64_t>(num_requests) + kSlotWaves - 1) / kSlotWaves;
    hipLaunchKernelGGL(commit_slots_kernel, dim3(static_cast<uint32_t>(blocks)), dim3(64 * kSlotWaves), 0,
                       as_stream(stream), tree_slots, cu_seqlens, paths, path_offsets, block_tables, table_stride,
                       table_width, cache_lens, num_requests, block_size, num_blocks, source_slots,
                       destination_slots, status);
    return check_launch("commit_slots");
}
