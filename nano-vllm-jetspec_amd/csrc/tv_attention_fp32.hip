// FP32 tree attention for every geometry (include/treeverify.h: tv_tree_attention_fp32).
//
// The MI355X form of the reference's scalar FP32 kernel (paged_backend.py:116-213) and
// of its legacy slot-addressed form (paged_backend.py:20-113): the path for batches the
// MFMA kernel does not take (f32 operands, head sizes other than 128, query groups the
// MFMA kernel is not built for, page sizes that are not multiples of 32, trees above
// 1024 nodes, finite qq_bias values).  The reference runs one program per (packed row,
// query head).  Here a workgroup of four waves owns four consecutive rows of one request
// and one KV head with its G query heads, so every K/V row it loads serves 4 x G rows.
//
// Per tile of TK keys (64 up to head_dim 128) of the group's visible range:
//   the first TK threads resolve the keys' slots (page table, prefix slot vector or tree
//   slot); all threads stage the K and V rows into LDS as float (coalesced loads, rows
//   padded to an odd pitch);
//   each wave, for its own row: lane k scores key k against the row's G query vectors
//   (LDS broadcast reads), adds the tree key's bias, runs each head's online softmax as
//   wave reductions (max, then sum) in fp32, and for P.V the lanes own head dimensions
//   (lane + 64 j) and walk the tile's keys.
// Accumulators: G_pass x DJ floats per lane with DJ = ceil(D / 64) and G_pass the smallest
// power of two >= G up to min(16, 64 / DJ); query heads beyond G_pass take further passes
// over the keys.
#include <math.h>
#include <stdint.h>

#include "tv_internal.h"

namespace tv {
namespace {

struct Fp32Params {
    const void* q;
    int64_t q_s0, q_s1;
    const void* k;
    const void* v;
    int64_t k_s0, k_s1, k_s2, k_s3;
    int64_t v_s0, v_s1, v_s2, v_s3;
    int64_t num_blocks;
    void* out;
    int64_t o_s0, o_s1;
    int32_t out_dtype;
    const int32_t* cu;
    const int32_t* q2r;
    const int32_t* local;
    const int32_t* plen;
    const int32_t* cnt;
    const int32_t* tables;
    int64_t t_s0;
    const int64_t* tree_slots;
    const float* bias;
    const int64_t* bias_off;
    const void* pslots;
    int64_t ps_s0;
    int32_t ps_i64;
    int32_t num_requests;
    int32_t total_queries;
    int32_t groups;       // query heads per KV head
    int32_t head_dim;
    int32_t block_size;
    float scale;
    int32_t* status;
};

constexpr int kWave = 64;

__device__ __forceinline__ float to_float(float x) { return x; }
__device__ __forceinline__ float to_float(__bf16 x) { return static_cast<float>(x); }
__device__ __forceinline__ float to_float(_Float16 x) { return static_cast<float>(x); }

__device__ __forceinline__ float wave_max(float x) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) x = fmaxf(x, __shfl_xor(x, off));
    return x;
}
__device__ __forceinline__ float wave_sum(float x) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) x += __shfl_xor(x, off);
    return x;
}

__device__ __forceinline__ void store_value(const Fp32Params& p, int64_t index, float x) {
    if (p.out_dtype == TV_F32) {
        static_cast<float*>(p.out)[index] = x;
    } else if (p.out_dtype == TV_BF16) {
        static_cast<__bf16*>(p.out)[index] = static_cast<__bf16>(x);
    } else {
        static_cast<_Float16*>(p.out)[index] = static_cast<_Float16>(x);
    }
}

constexpr int kRowsPerGroup = 4;    // waves per workgroup: consecutive rows of one request
constexpr int kThreadsFp32 = kWave * kRowsPerGroup;

// The launch numbers the row groups of request r from start(r) = cu[r] / 4 + r on: the
// ranges are disjoint and increasing (start(r + 1) - start(r) >= ceil(T_r / 4)), so a grid
// of Q / 4 + R + 1 workgroups covers every group with at most one idle workgroup per
// request, and consecutive workgroups (spread over the XCDs) all have work.
__device__ __forceinline__ int64_t group_start(const int32_t* cu, int r) {
    return static_cast<int64_t>(cu[r] / kRowsPerGroup) + r;
}

// The request whose group range holds workgroup b: the last r with start(r) <= b, by a
// 64-way search of the wave (two rounds of loads up to 4096 requests).
__device__ int request_of_group(const int32_t* cu, int num_requests, int64_t b) {
    const int lane = threadIdx.x & (kWave - 1);
    int lo = 0, hi = num_requests;   // start(lo) <= b; the answer is in [lo, hi)
    while (hi - lo > 1) {
        const int step = (hi - lo + kWave - 1) / kWave;
        const int r = lo + lane * step;
        const bool le = r < hi && group_start(cu, r) <= b;
        const uint64_t mask = __ballot(le);   // lanes 0 .. k set: start() increases with r
        const int last = 63 - __builtin_clzll(mask | 1ull);
        lo += last * step;
        hi = min(hi, lo + step);
    }
    return lo;
}

// Keys per LDS tile: 64 up to head_dim 128, fewer above (the K and V tiles stay near 66 KiB).
template <int DJ>
struct TileShape {
    static constexpr int TK = DJ <= 2 ? 64 : 64 * 2 / DJ;
    static constexpr int PITCH = kWave * DJ;          // LDS row of one query head (floats)
    // K/V rows padded by 4 floats: 16-byte aligned, and a lane-per-key 16-byte read of 16
    // lanes covers the 64 banks once.
    static constexpr int KV_PITCH = kWave * DJ + 4;
    static constexpr int KPW = TK / kRowsPerGroup;    // keys each wave stages per tile
};

// A score more than this far above a row's reference maximum (natural-log units) raises
// the maximum; below it probabilities stay <= e^8, which fp32 holds with its full
// relative precision, so the result is the same online softmax with rare rescales.
constexpr float kRaiseMargin = 8.f;

// T: operand type; DJ: head dimensions per lane (D <= 64 * DJ); GP: query heads per pass
// (the launch picks the smallest power of two >= G, at most 16 and at most 64 / DJ, so
// G_pass x DJ accumulators fit).  Workgroup: rows local0 .. local0 + 3 of one request and
// one KV head.  Software pipeline over tiles of TK keys: while tile t is computed, the K/V
// loads of tile t + 1 (slots resolved one iteration earlier) and the slot lookups of
// tile t + 2 are in flight; tile t's K/V rows, staged in LDS as float, serve all four
// rows.  Each wave runs its own row: lane k scores key k against the row's G query
// vectors, the row's reference maximum is raised only when a score exceeds it by
// kRaiseMargin (a ballot; the wave reduction runs then), probabilities and per-lane sums
// use it, and for P.V the lanes own head dimensions.
template <typename T, int DJ, int GP>
__global__ void __launch_bounds__(kThreadsFp32)
tree_attention_fp32_kernel(const Fp32Params p) {
    typedef TileShape<DJ> S;
    constexpr int TK = S::TK, PITCH = S::PITCH, KV_PITCH = S::KV_PITCH, KPW = S::KPW;
    static_assert(GP * DJ <= 64, "accumulators per lane");
    static_assert(TK <= kThreadsFp32 && TK % 4 == 0, "one slot lookup per thread, 4-key P.V steps");
    __shared__ __attribute__((aligned(16))) float q_lds[kRowsPerGroup][GP * PITCH];
    __shared__ __attribute__((aligned(16))) float p_lds[kRowsPerGroup][GP * TK];
    __shared__ __attribute__((aligned(16))) float k_lds[TK * KV_PITCH];
    __shared__ __attribute__((aligned(16))) float v_lds[TK * KV_PITCH];
    __shared__ int64_t kbase_lds[2][TK], vbase_lds[2][TK];   // element offsets of the rows, -1: missing

    const int tid = threadIdx.x, lane = tid & (kWave - 1);
    const int wave = __builtin_amdgcn_readfirstlane(tid / kWave);
    const int kvh = blockIdx.y;
    const int r = __builtin_amdgcn_readfirstlane(request_of_group(p.cu, p.num_requests, blockIdx.x));
    const int local0 = static_cast<int>(blockIdx.x - group_start(p.cu, r)) * kRowsPerGroup;
    const int P = p.plen[r], nodes = p.cnt[r];
    if (local0 >= nodes) return;   // the gap after request r's groups
    if (P < 0) {
        if (tid == 0) set_status(p.status, TV_STATUS_BAD_REQUEST);
        return;
    }
    const int64_t leader = static_cast<int64_t>(p.cu[r]) + local0;
    const int rows = min(kRowsPerGroup, nodes - local0);
    if (leader < 0 || leader + rows > p.total_queries) {
        if (tid == 0) set_status(p.status, TV_STATUS_BAD_REQUEST);
        return;
    }
    // This wave's row; the metadata must place a request's rows consecutively.
    const int64_t row = leader + wave;
    const int local = local0 + wave;
    bool row_ok = wave < rows;
    if (row_ok && (p.q2r[row] != r || p.local[row] != local)) {
        if (lane == 0) set_status(p.status, TV_STATUS_BAD_REQUEST);
        row_ok = false;
    }
    const int D = p.head_dim, B = p.block_size, G = p.groups;
    const int64_t tree0 = p.cu[r];
    const int64_t bias_row = p.bias_off[r] + static_cast<int64_t>(local) * nodes;
    const int seq = P + local0 + rows;    // keys any row of the group can see
    const int ntiles = (seq + TK - 1) / TK;
    const int my_end = P + local + 1;     // this row's visible range
    const int64_t pool_slots = p.num_blocks * B;
    const T* q = static_cast<const T*>(p.q);
    const T* k = static_cast<const T*>(p.k);
    const T* v = static_cast<const T*>(p.v);

    // Slot of key t0 + tid (threads < TK): the load, then the row offsets.
    auto slot_load = [&](int t0) -> int64_t {
        const int pos = t0 + tid;
        if (tid >= TK || pos >= seq) return -1;
        if (pos >= P) return p.tree_slots[tree0 + (pos - P)];
        if (p.pslots) {
            const int64_t at = static_cast<int64_t>(r) * p.ps_s0 + pos;
            return p.ps_i64 ? static_cast<const int64_t*>(p.pslots)[at]
                            : static_cast<int64_t>(static_cast<const int32_t*>(p.pslots)[at]);
        }
        const int64_t page = p.tables[static_cast<int64_t>(r) * p.t_s0 + pos / B];
        return (page >= 0 && page < p.num_blocks) ? page * B + pos % B : -2;
    };
    auto slot_store = [&](int t0, int64_t slot, int buf) {
        const int pos = t0 + tid;
        if (tid >= TK) return;
        int64_t kb = -1, vb = -1;
        if (pos < seq) {
            if (slot < 0 || slot >= pool_slots) {
                set_status(p.status, TV_STATUS_BAD_PAGE);
            } else {
                const int64_t blk = slot / B, off = slot - blk * B;
                kb = blk * p.k_s0 + off * p.k_s1 + static_cast<int64_t>(kvh) * p.k_s2;
                vb = blk * p.v_s0 + off * p.v_s1 + static_cast<int64_t>(kvh) * p.v_s2;
            }
        }
        kbase_lds[buf][tid] = kb;
        vbase_lds[buf][tid] = vb;
    };
    // This thread's share of a tile's K and V: wave w stages keys w, w + 4, ..., its lanes
    // along the head dimension (coalesced); every load is issued before any is used.
    float kx[KPW][DJ], vx[KPW][DJ];
    auto kv_load = [&](int buf) {
#pragma unroll
        for (int i = 0; i < KPW; ++i) {
            const int key = wave + kRowsPerGroup * i;
            const int64_t kb = kbase_lds[buf][key], vb = vbase_lds[buf][key];
#pragma unroll
            for (int j = 0; j < DJ; ++j) {
                const int d = lane + kWave * j;
                const bool ok = kb >= 0 && d < D;
                kx[i][j] = ok ? to_float(k[kb + d * p.k_s3]) : 0.f;
                vx[i][j] = ok ? to_float(v[vb + d * p.v_s3]) : 0.f;
            }
        }
    };
    auto kv_store = [&]() {
#pragma unroll
        for (int i = 0; i < KPW; ++i) {
            const int key = wave + kRowsPerGroup * i;
#pragma unroll
            for (int j = 0; j < DJ; ++j) {
                const int d = lane + kWave * j;
                k_lds[key * KV_PITCH + d] = kx[i][j];
                v_lds[key * KV_PITCH + d] = vx[i][j];
            }
        }
    };

    for (int g0 = 0; g0 < G; g0 += GP) {
        const int gn = min(GP, G - g0);
        const int head0 = kvh * G + g0;
        for (int i = lane; i < GP * PITCH; i += kWave) {
            const int g = i / PITCH, d = i - g * PITCH;
            float x = 0.f;
            if (row_ok && g < gn && d < D) x = to_float(q[row * p.q_s0 + static_cast<int64_t>(head0 + g) * p.q_s1 + d]);
            q_lds[wave][i] = x;
        }
        float m[GP], l[GP], acc[GP][DJ];
#pragma unroll
        for (int g = 0; g < GP; ++g) {
            m[g] = -INFINITY;
            l[g] = 0.f;
#pragma unroll
            for (int j = 0; j < DJ; ++j) acc[g][j] = 0.f;
        }
        // Pipeline prologue: slots of tiles 0 and 1, K/V loads of tile 0.
        __syncthreads();   // the previous pass's LDS reads are done
        slot_store(0, slot_load(0), 0);
        __syncthreads();
        kv_load(0);
        if (ntiles > 1) slot_store(TK, slot_load(TK), 1);
        int64_t next_slot = -1;   // slot of key (t + 1) * TK + tid, loaded during iteration t - 1
        for (int t = 0; t < ntiles; ++t) {
            const int t0 = t * TK;
            __syncthreads();   // every wave is done with tile t - 1 (its K/V rows and its slot buffer)
            // Tile t + 1's slots go into the buffer tile t - 1 used: only after the barrier, since
            // every wave reads its tile's slot buffer in its own compute (the visibility test).
            if (t >= 1 && t + 1 < ntiles) slot_store(t0 + TK, next_slot, (t + 1) & 1);
            kv_store();
            __syncthreads();   // tile t is staged; tile t + 1's slots are in LDS
            if (t + 1 < ntiles) kv_load((t + 1) & 1);
            next_slot = t + 2 < ntiles ? slot_load(t0 + 2 * TK) : -1;
            if (row_ok) {
                const int pos = t0 + lane;
                bool visible = lane < TK && pos < my_end && kbase_lds[t & 1][lane < TK ? lane : 0] >= 0;
                float bias = 0.f;
                if (visible && pos >= P) {
                    bias = p.bias[bias_row + (pos - P)];
                    if (bias == -INFINITY) visible = false;
                }
                float sc[GP];
#pragma unroll
                for (int g = 0; g < GP; ++g) sc[g] = 0.f;
                if (visible) {
                    const float* kr = k_lds + (lane < TK ? lane : 0) * KV_PITCH;
#pragma unroll 2
                    for (int d = 0; d < D; d += 4) {
                        const float4 kv4 = *reinterpret_cast<const float4*>(kr + d);
#pragma unroll
                        for (int g = 0; g < GP; ++g) {
                            const float4 qv = *reinterpret_cast<const float4*>(&q_lds[wave][g * PITCH + d]);
                            sc[g] = fmaf(qv.x, kv4.x, sc[g]);
                            sc[g] = fmaf(qv.y, kv4.y, sc[g]);
                            sc[g] = fmaf(qv.z, kv4.z, sc[g]);
                            sc[g] = fmaf(qv.w, kv4.w, sc[g]);
                        }
                    }
                }
#pragma unroll
                for (int g = 0; g < GP; ++g) {
                    const float score = visible ? fmaf(sc[g], p.scale, bias) : -INFINITY;
                    if (__ballot(score > m[g] + kRaiseMargin)) {   // rare after the first tile
                        const float m_new = fmaxf(m[g], wave_max(score));
                        const float alpha = expf(m[g] - m_new);   // 0 while m[g] is -inf
                        l[g] *= alpha;
#pragma unroll
                        for (int j = 0; j < DJ; ++j) acc[g][j] *= alpha;
                        m[g] = m_new;
                    }
                    const float pr = score == -INFINITY ? 0.f : expf(score - m[g]);
                    l[g] += pr;
                    if (lane < TK) p_lds[wave][g * TK + lane] = pr;
                }
                // P.V over the tile's keys (the wave reads only its own probabilities).
                __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
                __builtin_amdgcn_wave_barrier();
                __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
                const int keys = min(TK, my_end - t0);
                for (int kk = 0; kk < keys; kk += 4) {
                    float vv[4][DJ];
#pragma unroll
                    for (int u = 0; u < 4; ++u) {
#pragma unroll
                        for (int j = 0; j < DJ; ++j) vv[u][j] = v_lds[(kk + u) * KV_PITCH + lane + kWave * j];
                    }
#pragma unroll
                    for (int g = 0; g < GP; ++g) {
                        const float4 pg = *reinterpret_cast<const float4*>(&p_lds[wave][g * TK + kk]);
#pragma unroll
                        for (int j = 0; j < DJ; ++j) {
                            acc[g][j] = fmaf(pg.x, vv[0][j], acc[g][j]);
                            acc[g][j] = fmaf(pg.y, vv[1][j], acc[g][j]);
                            acc[g][j] = fmaf(pg.z, vv[2][j], acc[g][j]);
                            acc[g][j] = fmaf(pg.w, vv[3][j], acc[g][j]);
                        }
                    }
                }
            }
        }
        if (row_ok) {
#pragma unroll
            for (int g = 0; g < GP; ++g) {
                const float inv = 1.f / wave_sum(l[g]);
                const int64_t base = row * p.o_s0 + static_cast<int64_t>(head0 + g) * p.o_s1;
#pragma unroll
                for (int j = 0; j < DJ; ++j) {
                    const int d = lane + kWave * j;
                    if (g < gn && d < D) store_value(p, base + d, acc[g][j] * inv);
                }
            }
        }
    }
}

template <typename T, int DJ>
void launch_for_dims(const Fp32Params& p, const dim3& grid, hipStream_t s) {
    constexpr int kMaxPass = 64 / DJ < 16 ? 64 / DJ : 16;
    int gp = 2;
    while (gp < p.groups && gp < kMaxPass) gp *= 2;
    switch (gp) {
        case 2: hipLaunchKernelGGL((tree_attention_fp32_kernel<T, DJ, 2>), grid, dim3(kThreadsFp32), 0, s, p); break;
        case 4: hipLaunchKernelGGL((tree_attention_fp32_kernel<T, DJ, 4>), grid, dim3(kThreadsFp32), 0, s, p); break;
        case 8: hipLaunchKernelGGL((tree_attention_fp32_kernel<T, DJ, 8>), grid, dim3(kThreadsFp32), 0, s, p); break;
        default:
            hipLaunchKernelGGL((tree_attention_fp32_kernel<T, DJ, kMaxPass>), grid, dim3(kThreadsFp32), 0, s, p);
            break;
    }
}

template <typename T>
void launch_for_type(const Fp32Params& p, int32_t kv_heads, hipStream_t s) {
    // One workgroup per group of four rows of a request (group_start); the grid depends
    // only on the packed row and request counts, which a captured graph keeps fixed.
    const int64_t groups = static_cast<int64_t>(p.total_queries) / kRowsPerGroup + p.num_requests + 1;
    const dim3 grid(static_cast<uint32_t>(groups), static_cast<uint32_t>(kv_heads));
    if (p.head_dim <= 64) {
        launch_for_dims<T, 1>(p, grid, s);
    } else if (p.head_dim <= 128) {
        launch_for_dims<T, 2>(p, grid, s);
    } else if (p.head_dim <= 256) {
        launch_for_dims<T, 4>(p, grid, s);
    } else {
        launch_for_dims<T, 8>(p, grid, s);
    }
}

bool valid_dtype(int32_t code) { return code == TV_F32 || code == TV_BF16 || code == TV_F16; }

}  // namespace
}  // namespace tv

using namespace tv;

extern "C" int64_t tv_sizeof_tree_attention_fp32_args(void) { return sizeof(tv_tree_attention_fp32_args); }

extern "C" int tv_tree_attention_fp32(const tv_tree_attention_fp32_args* a, void* stream) {
    clear_error();
    if (!a) return fail(TV_ERR_INVALID, "tree_attention_fp32: null args");
    if (a->num_requests < 1 || a->total_queries < 0) return fail(TV_ERR_INVALID, "tree_attention_fp32: invalid counts");
    if (a->num_kv_heads < 1 || a->num_q_heads < a->num_kv_heads || a->num_q_heads % a->num_kv_heads) {
        return fail(TV_ERR_INVALID, "tree_attention_fp32: %d query heads over %d KV heads", a->num_q_heads,
                    a->num_kv_heads);
    }
    if (a->num_kv_heads > 65535) return fail(TV_ERR_UNSUPPORTED, "tree_attention_fp32: more than 65535 KV heads");
    if (a->head_dim < 1 || a->head_dim > 512) {
        return fail(TV_ERR_UNSUPPORTED, "tree_attention_fp32: head_dim %d (implemented: 1..512)", a->head_dim);
    }
    if (a->block_size < 1 || a->num_blocks < 0 || a->num_blocks > (int64_t{1} << 62) / a->block_size) {
        return fail(TV_ERR_INVALID, "tree_attention_fp32: invalid pool geometry");
    }
    if (!valid_dtype(a->in_dtype) || !valid_dtype(a->out_dtype)) {
        return fail(TV_ERR_INVALID, "tree_attention_fp32: dtypes must be TV_F32, TV_BF16 or TV_F16");
    }
    if (!isfinite(a->scale)) return fail(TV_ERR_INVALID, "tree_attention_fp32: softmax scale must be finite");
    if (a->prefix_slots && a->prefix_slots_stride < 0) {
        return fail(TV_ERR_INVALID, "tree_attention_fp32: negative prefix slot stride");
    }
    if (a->total_queries == 0) return TV_OK;
    if (!a->q || !a->k_pool || !a->v_pool || !a->out || !a->cu_seqlens_q || !a->query_to_request ||
        !a->query_local_row || !a->prefix_lens || !a->node_counts || !a->tree_slots || !a->qq_bias ||
        !a->qq_bias_offsets || (!a->prefix_slots && !a->block_tables)) {
        return fail(TV_ERR_INVALID, "tree_attention_fp32: null pointer");
    }
    Fp32Params p;
    p.q = a->q;
    p.q_s0 = a->q_stride_row;
    p.q_s1 = a->q_stride_head;
    p.k = a->k_pool;
    p.v = a->v_pool;
    p.k_s0 = a->k_stride[0];
    p.k_s1 = a->k_stride[1];
    p.k_s2 = a->k_stride[2];
    p.k_s3 = a->k_stride[3];
    p.v_s0 = a->v_stride[0];
    p.v_s1 = a->v_stride[1];
    p.v_s2 = a->v_stride[2];
    p.v_s3 = a->v_stride[3];
    p.num_blocks = a->num_blocks;
    p.out = a->out;
    p.o_s0 = a->out_stride_row;
    p.o_s1 = a->out_stride_head;
    p.out_dtype = a->out_dtype;
    p.cu = a->cu_seqlens_q;
    p.q2r = a->query_to_request;
    p.local = a->query_local_row;
    p.plen = a->prefix_lens;
    p.cnt = a->node_counts;
    p.tables = a->block_tables;
    p.t_s0 = a->block_table_stride;
    p.tree_slots = a->tree_slots;
    p.bias = a->qq_bias;
    p.bias_off = a->qq_bias_offsets;
    p.pslots = a->prefix_slots;
    p.ps_s0 = a->prefix_slots_stride;
    p.ps_i64 = a->prefix_slots_is_int64 != 0;
    p.num_requests = a->num_requests;
    p.total_queries = a->total_queries;
    p.groups = a->num_q_heads / a->num_kv_heads;
    p.head_dim = a->head_dim;
    p.block_size = a->block_size;
    p.scale = a->scale;
    p.status = a->status;
    hipStream_t s = as_stream(stream);
    if (a->in_dtype == TV_F32) {
        launch_for_type<float>(p, a->num_kv_heads, s);
    } else if (a->in_dtype == TV_BF16) {
        launch_for_type<__bf16>(p, a->num_kv_heads, s);
    } else {
        launch_for_type<_Float16>(p, a->num_kv_heads, s);
    }
    return check_launch("tree_attention_fp32");
}
