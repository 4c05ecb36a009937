// FP32 tree attention for every geometry (include/treeverify.h: tv_tree_attention_fp32).
//
// The MI355X form of the reference's scalar FP32 kernel (paged_backend.py:116-213) and
// of its legacy slot-addressed form (paged_backend.py:20-113): the path for batches the
// MFMA kernel does not take (f32 operands, head sizes other than 128, query groups
// other than 1/2/4/8/16, page sizes that are not multiples of 32, trees above 1024
// nodes, finite qq_bias values).  The reference runs one program per (packed row,
// query head); here one wave owns a (packed row, KV head) and its G query heads, so
// every K/V row it loads serves all G heads.
//
// Per 64-key tile of the visible range [0, P + local]:
//   lane k resolves key k's slot (page table, prefix slot vector or tree slot) and its
//   bias, and computes the G scores q_g . K[key] from its own K row against the wave's
//   Q rows in LDS (broadcast reads);
//   each head's online softmax runs as wave reductions (max, then sum), in fp32;
//   for P.V the lanes own head dimensions (lane + 64 j) and walk the tile's keys:
//   coalesced V row loads, probabilities read from LDS.
// Accumulators: G_pass x DJ floats per lane with DJ = ceil(D / 64); query heads beyond
// G_pass = min(16, 64 / DJ) take further passes over the keys.
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

// T: operand type; DJ: head dimensions per lane (D <= 64 * DJ).
template <typename T, int DJ>
__global__ void __launch_bounds__(kWave)
tree_attention_fp32_kernel(const Fp32Params p) {
    constexpr int GP = (kWave / DJ < 16) ? kWave / DJ : 16;   // query heads per pass
    constexpr int PITCH = kWave * DJ;                          // LDS row of one query head
    __shared__ __attribute__((aligned(16))) float q_lds[GP * PITCH];
    __shared__ float p_lds[GP * kWave];
    __shared__ int64_t slot_lds[kWave];

    const int lane = threadIdx.x;
    const int64_t row = blockIdx.x;
    const int kvh = blockIdx.y;
    const int r = p.q2r[row];
    if (r < 0 || r >= p.num_requests) {
        if (lane == 0) set_status(p.status, TV_STATUS_BAD_REQUEST);
        return;
    }
    const int local = p.local[row];
    const int P = p.plen[r], nodes = p.cnt[r];
    if (local < 0 || local >= nodes || P < 0) {
        if (lane == 0) set_status(p.status, TV_STATUS_BAD_REQUEST);
        return;
    }
    const int D = p.head_dim, B = p.block_size, G = p.groups;
    const int64_t tree0 = p.cu[r];
    const int64_t bias_row = p.bias_off[r] + static_cast<int64_t>(local) * nodes;
    const int seq = P + local + 1;   // positions past P + local are never visible
    const int64_t pool_slots = p.num_blocks * B;
    const T* q = static_cast<const T*>(p.q);
    const T* k = static_cast<const T*>(p.k);
    const T* v = static_cast<const T*>(p.v);

    for (int g0 = 0; g0 < G; g0 += GP) {
        const int gn = min(GP, G - g0);
        const int head0 = kvh * G + g0;
        for (int i = lane; i < GP * PITCH; i += kWave) {
            const int g = i / PITCH, d = i - g * PITCH;
            float x = 0.f;
            if (g < gn && d < D) x = to_float(q[row * p.q_s0 + static_cast<int64_t>(head0 + g) * p.q_s1 + d]);
            q_lds[i] = x;
        }
        __syncthreads();
        float m[GP], l[GP], acc[GP][DJ];
#pragma unroll
        for (int g = 0; g < GP; ++g) {
            m[g] = -INFINITY;
            l[g] = 0.f;
#pragma unroll
            for (int j = 0; j < DJ; ++j) acc[g][j] = 0.f;
        }
        for (int t0 = 0; t0 < seq; t0 += kWave) {
            // This lane's key: slot, bias and visibility.
            const int pos = t0 + lane;
            int64_t slot = -1;
            float bias = 0.f;
            bool visible = pos < seq;
            if (visible) {
                if (pos < P) {
                    if (p.pslots) {
                        const int64_t at = static_cast<int64_t>(r) * p.ps_s0 + pos;
                        slot = p.ps_i64 ? static_cast<const int64_t*>(p.pslots)[at]
                                        : static_cast<int64_t>(static_cast<const int32_t*>(p.pslots)[at]);
                    } else {
                        const int64_t page = p.tables[static_cast<int64_t>(r) * p.t_s0 + pos / B];
                        slot = (page >= 0 && page < p.num_blocks) ? page * B + pos % B : -1;
                    }
                } else {
                    slot = p.tree_slots[tree0 + (pos - P)];
                    bias = p.bias[bias_row + (pos - P)];
                }
                if (slot < 0 || slot >= pool_slots) {
                    set_status(p.status, TV_STATUS_BAD_PAGE);
                    visible = false;
                } else if (bias == -INFINITY) {
                    visible = false;
                }
            }
            slot_lds[lane] = visible ? slot : -1;
            float s[GP];
#pragma unroll
            for (int g = 0; g < GP; ++g) s[g] = 0.f;
            if (visible) {
                const T* kr = k + (slot / B) * p.k_s0 + (slot % B) * p.k_s1 + static_cast<int64_t>(kvh) * p.k_s2;
                for (int d = 0; d < D; d += 4) {
                    float kx[4];
#pragma unroll
                    for (int i = 0; i < 4; ++i) kx[i] = d + i < D ? to_float(kr[(d + i) * p.k_s3]) : 0.f;
#pragma unroll
                    for (int g = 0; g < GP; ++g) {
                        const float4 qv = *reinterpret_cast<const float4*>(&q_lds[g * PITCH + d]);
                        s[g] = fmaf(qv.x, kx[0], s[g]);
                        s[g] = fmaf(qv.y, kx[1], s[g]);
                        s[g] = fmaf(qv.z, kx[2], s[g]);
                        s[g] = fmaf(qv.w, kx[3], s[g]);
                    }
                }
            }
            // Online softmax per query head; a tile with no visible key leaves a head as it was.
#pragma unroll
            for (int g = 0; g < GP; ++g) {
                const float score = visible ? fmaf(s[g], p.scale, bias) : -INFINITY;
                const float m_new = fmaxf(m[g], wave_max(score));
                const float m_ref = m_new == -INFINITY ? 0.f : m_new;
                const float alpha = expf(m[g] - m_ref);
                const float pr = expf(score - m_ref);
                l[g] = l[g] * alpha + wave_sum(pr);
#pragma unroll
                for (int j = 0; j < DJ; ++j) acc[g][j] *= alpha;
                m[g] = m_new;
                p_lds[g * kWave + lane] = pr;
            }
            __syncthreads();
            const int keys = min(kWave, seq - t0);
            for (int kk = 0; kk < keys; ++kk) {
                const int64_t sl = slot_lds[kk];
                if (sl < 0) continue;
                const T* vr = v + (sl / B) * p.v_s0 + (sl % B) * p.v_s1 + static_cast<int64_t>(kvh) * p.v_s2;
                float vx[DJ];
#pragma unroll
                for (int j = 0; j < DJ; ++j) {
                    const int d = lane + kWave * j;
                    vx[j] = d < D ? to_float(vr[d * p.v_s3]) : 0.f;
                }
#pragma unroll
                for (int g = 0; g < GP; ++g) {
                    const float pg = p_lds[g * kWave + kk];
#pragma unroll
                    for (int j = 0; j < DJ; ++j) acc[g][j] = fmaf(pg, vx[j], acc[g][j]);
                }
            }
            __syncthreads();   // slot_lds and p_lds are rewritten by the next tile
        }
#pragma unroll
        for (int g = 0; g < GP; ++g) {
            if (g >= gn) break;
            const float inv = 1.f / l[g];
            const int64_t base = row * p.o_s0 + static_cast<int64_t>(head0 + g) * p.o_s1;
#pragma unroll
            for (int j = 0; j < DJ; ++j) {
                const int d = lane + kWave * j;
                if (d < D) store_value(p, base + d, acc[g][j] * inv);
            }
        }
        __syncthreads();   // q_lds is rewritten by the next pass
    }
}

template <typename T>
void launch_for_type(const Fp32Params& p, int32_t kv_heads, hipStream_t s) {
    const dim3 grid(static_cast<uint32_t>(p.total_queries), static_cast<uint32_t>(kv_heads));
    if (p.head_dim <= 64) {
        hipLaunchKernelGGL((tree_attention_fp32_kernel<T, 1>), grid, dim3(kWave), 0, s, p);
    } else if (p.head_dim <= 128) {
        hipLaunchKernelGGL((tree_attention_fp32_kernel<T, 2>), grid, dim3(kWave), 0, s, p);
    } else if (p.head_dim <= 256) {
        hipLaunchKernelGGL((tree_attention_fp32_kernel<T, 4>), grid, dim3(kWave), 0, s, p);
    } else {
        hipLaunchKernelGGL((tree_attention_fp32_kernel<T, 8>), grid, dim3(kWave), 0, s, p);
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
