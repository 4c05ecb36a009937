// HF-order RoPE of the tree Q/K fused with the scatter of the tree K/V into their
// scratch slots, for gfx950.
//
// Semantics (tree_fusion.py:20-82, and the eager path it replaces,
// models/qwen3.py:241-258): row i, head h, halves x1 = x[:D/2], x2 = x[D/2:] and the
// cache row [cos | sin] at positions[i]:
//     y1 = round(round(x1*cos) - round(x2*sin)),  y2 = round(round(x2*cos) + round(x1*sin))
// where round() is bf16 round-to-nearest-even for bf16 operands (cos/sin are rounded
// to bf16 first, the products of two bf16 values are exact in fp32) and the identity
// for fp32 operands, whose products and sums are then separate fp32 operations (no
// fused multiply-add: the kernel is compiled with contraction off).  Q goes to `out`,
// rotated K and the raw V go to page slot / page_size, offset slot % page_size.
//
// The operation moves ~12 B per element and computes a handful of flops, so it is
// HBM-bound: one 256-thread workgroup per row, which stages the row's cos/sin in LDS
// once (in the operand dtype) for all of its heads; each thread owns `Vec` consecutive
// dims of one head's first half and the matching dims of its second half, loaded and
// stored as 16-byte vectors where strides and alignment allow it.  Each K/V row has
// exactly one writer (the KV-head work items of its own row).
#include <stdint.h>

#include "tv_internal.h"

namespace tv {
namespace {

// float -> bf16 bits, round to nearest even, any NaN -> 0x7FC0 (the rounding PyTorch
// applies when an eager bf16 op stores its fp32 result).
__device__ __forceinline__ uint32_t bf16_bits(float f) {
    const uint32_t u = __float_as_uint(f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return 0x7fc0u;
    return (u + 0x7fffu + ((u >> 16) & 1u)) >> 16;
}

__device__ __forceinline__ float bf16_value(uint32_t bits) { return __uint_as_float(bits << 16); }

struct Bf16Ops {
    typedef uint16_t storage;
    static __device__ __forceinline__ float load(storage s) { return bf16_value(s); }
    static __device__ __forceinline__ float round(float x) { return bf16_value(bf16_bits(x)); }
    static __device__ __forceinline__ storage store(float x) { return static_cast<storage>(bf16_bits(x)); }
};

struct F32Ops {
    typedef float storage;
    static __device__ __forceinline__ float load(storage s) { return s; }
    static __device__ __forceinline__ float round(float x) { return x; }
    static __device__ __forceinline__ storage store(float x) { return x; }
};

struct RopeParams {
    const void* q;
    int64_t q_s0, q_s1, q_s2;
    const void* k;
    int64_t k_s0, k_s1, k_s2;
    const void* v;
    int64_t v_s0, v_s1, v_s2;
    const void* positions;
    int64_t pos_s;
    int32_t pos64;
    const void* cache;
    int64_t cache_rows, cache_s0, cache_s1;
    int32_t cache_f32;
    void* kp;
    int64_t kp_s0, kp_s1, kp_s2, kp_s3;
    void* vp;
    int64_t vp_s0, vp_s1, vp_s2, vp_s3;
    int64_t pool_pages, page_size;
    const void* slots;
    int64_t slot_s;
    int32_t slot64;
    void* out;
    int64_t o_s0, o_s1, o_s2;
    int32_t q_heads, kv_heads, head_dim;
    int32_t* status;
};

// VEC consecutive elements at `p` with element stride `s` (one 16-byte access when
// VEC > 1: the host only picks that path for unit strides and 16-byte alignment).
template <typename S, int VEC>
__device__ __forceinline__ void load_elems(const S* p, int64_t s, S (&out)[VEC]) {
    if constexpr (VEC > 1) {
        static_assert(VEC * sizeof(S) == 16, "vector path moves 16 bytes");
        const u32x4 raw = *reinterpret_cast<const u32x4*>(p);
        __builtin_memcpy(out, &raw, 16);
    } else {
        out[0] = p[0];
    }
}

template <typename S, int VEC>
__device__ __forceinline__ void store_elems(S* p, int64_t s, const S (&in)[VEC]) {
    if constexpr (VEC > 1) {
        u32x4 raw;
        __builtin_memcpy(&raw, in, 16);
        *reinterpret_cast<u32x4*>(p) = raw;
    } else {
        p[0] = in[0];
    }
}

template <class Ops, int VEC>
__global__ void __launch_bounds__(256)
rope_scatter_kernel(const RopeParams p) {
#pragma clang fp contract(off)
    typedef typename Ops::storage S;
    const int64_t row = blockIdx.x;
    const int64_t pos = p.pos64 ? static_cast<const int64_t*>(p.positions)[row * p.pos_s]
                                : static_cast<int64_t>(static_cast<const int32_t*>(p.positions)[row * p.pos_s]);
    const int64_t slot = p.slot64 ? static_cast<const int64_t*>(p.slots)[row * p.slot_s]
                                  : static_cast<int64_t>(static_cast<const int32_t*>(p.slots)[row * p.slot_s]);
    if (pos < 0 || pos >= p.cache_rows) {
        if (threadIdx.x == 0) set_status(p.status, TV_STATUS_BAD_POSITION);
        return;
    }
    const bool slot_ok = slot >= 0 && slot < p.pool_pages * p.page_size;
    if (!slot_ok) {
        if (threadIdx.x == 0) set_status(p.status, TV_STATUS_BAD_SLOT);
        return;
    }
    const int64_t page = slot / p.page_size, offset = slot - page * p.page_size;
    const int half = p.head_dim >> 1;
    const int per_half = half / VEC;              // work items per head half
    const int per_row = p.head_dim / VEC;         // V copy items per head
    const int nq = p.q_heads * per_half;
    const int nk = p.kv_heads * per_half;
    const int nv = p.kv_heads * per_row;
    // The row's cos/sin, in the operand dtype, staged once in LDS for all its heads.
    __shared__ __attribute__((aligned(16))) float lds_cos[128], lds_sin[128];
    const char* cache_row = static_cast<const char*>(p.cache) + pos * p.cache_s0 * (p.cache_f32 ? 4 : 2);
    for (int e = threadIdx.x; e < half; e += blockDim.x) {
        const int64_t ci = static_cast<int64_t>(e) * p.cache_s1;
        const int64_t si = static_cast<int64_t>(half + e) * p.cache_s1;
        float c, s;
        if (p.cache_f32) {
            c = reinterpret_cast<const float*>(cache_row)[ci];
            s = reinterpret_cast<const float*>(cache_row)[si];
        } else {
            c = bf16_value(reinterpret_cast<const uint16_t*>(cache_row)[ci]);
            s = bf16_value(reinterpret_cast<const uint16_t*>(cache_row)[si]);
        }
        lds_cos[e] = Ops::round(c);
        lds_sin[e] = Ops::round(s);
    }
    __syncthreads();

    for (int u = threadIdx.x; u < nq + nk + nv; u += blockDim.x) {
        if (u < nq + nk) {
            const bool is_q = u < nq;
            const int w = is_q ? u : u - nq;
            const int h = w / per_half;
            const int j = (w - h * per_half) * VEC;
            float cs[VEC], sn[VEC];
#pragma unroll
            for (int e = 0; e < VEC; ++e) {
                cs[e] = lds_cos[j + e];
                sn[e] = lds_sin[j + e];
            }
            const S* src;
            int64_t s2;
            S* dst;
            int64_t d2;
            if (is_q) {
                src = static_cast<const S*>(p.q) + row * p.q_s0 + h * p.q_s1;
                s2 = p.q_s2;
                dst = static_cast<S*>(p.out) + row * p.o_s0 + h * p.o_s1;
                d2 = p.o_s2;
            } else {
                src = static_cast<const S*>(p.k) + row * p.k_s0 + h * p.k_s1;
                s2 = p.k_s2;
                dst = static_cast<S*>(p.kp) + page * p.kp_s0 + offset * p.kp_s1 + h * p.kp_s2;
                d2 = p.kp_s3;
            }
            S a[VEC], b[VEC], y1[VEC], y2[VEC];
            load_elems<S, VEC>(src + j * s2, s2, a);
            load_elems<S, VEC>(src + (half + j) * s2, s2, b);
#pragma unroll
            for (int e = 0; e < VEC; ++e) {
                const float x1 = Ops::load(a[e]), x2 = Ops::load(b[e]);
                const float t0 = Ops::round(x1 * cs[e]);
                const float t1 = Ops::round(x2 * sn[e]);
                const float t2 = Ops::round(x2 * cs[e]);
                const float t3 = Ops::round(x1 * sn[e]);
                y1[e] = Ops::store(t0 - t1);
                y2[e] = Ops::store(t2 + t3);
            }
            store_elems<S, VEC>(dst + j * d2, d2, y1);
            store_elems<S, VEC>(dst + (half + j) * d2, d2, y2);
        } else {
            const int w = u - nq - nk;
            const int h = w / per_row;
            const int j = (w - h * per_row) * VEC;
            const S* src = static_cast<const S*>(p.v) + row * p.v_s0 + h * p.v_s1 + j * p.v_s2;
            S* dst = static_cast<S*>(p.vp) + page * p.vp_s0 + offset * p.vp_s1 + h * p.vp_s2 + j * p.vp_s3;
            S x[VEC];
            load_elems<S, VEC>(src, p.v_s2, x);
            store_elems<S, VEC>(dst, p.vp_s3, x);
        }
    }
}

// Scalar fallback: element strides, one element (and its partner in the other half)
// per work item.  The vector path is the Vec = 16 / sizeof(element) instance.
template <class Ops>
void launch(const RopeParams& p, int64_t rows, bool vec, hipStream_t stream) {
    constexpr int kVec = 16 / sizeof(typename Ops::storage);
    if (vec) {
        hipLaunchKernelGGL((rope_scatter_kernel<Ops, kVec>), dim3(rows), dim3(256), 0, stream, p);
    } else {
        hipLaunchKernelGGL((rope_scatter_kernel<Ops, 1>), dim3(rows), dim3(256), 0, stream, p);
    }
}

}  // namespace
}  // namespace tv

using namespace tv;

extern "C" int64_t tv_sizeof_rope_scatter_args(void) { return static_cast<int64_t>(sizeof(tv_rope_scatter_args)); }

extern "C" int tv_rope_scatter(const tv_rope_scatter_args* a, void* stream) {
    clear_error();
    if (!a) return fail(TV_ERR_INVALID, "rope_scatter: null args");
    if (a->rows < 0 || a->q_heads < 1 || a->kv_heads < 1 || a->q_heads % a->kv_heads) {
        return fail(TV_ERR_INVALID, "rope_scatter: invalid GQA geometry (%d query heads, %d KV heads)", a->q_heads,
                    a->kv_heads);
    }
    if (a->head_dim < 2 || a->head_dim % 2 || a->head_dim > 256) {
        return fail(TV_ERR_INVALID, "rope_scatter: head_dim %d must be even and in [2, 256]", a->head_dim);
    }
    if (a->dtype != TV_BF16 && a->dtype != TV_F32) {
        return fail(TV_ERR_UNSUPPORTED, "rope_scatter: operands must be bf16 or fp32");
    }
    if (a->cache_dtype != TV_BF16 && a->cache_dtype != TV_F32) {
        return fail(TV_ERR_UNSUPPORTED, "rope_scatter: cos/sin cache must be bf16 or fp32");
    }
    if (a->rows == 0) return TV_OK;
    if (a->rows > 0x7fffffff) return fail(TV_ERR_UNSUPPORTED, "rope_scatter: too many rows");
    if (!a->q || !a->k || !a->v || !a->positions || !a->cache || !a->k_pool || !a->v_pool || !a->node_slots ||
        !a->out) {
        return fail(TV_ERR_INVALID, "rope_scatter: null pointer");
    }
    if (a->cache_rows < 1 || a->pool_pages < 1 || a->page_size < 1) {
        return fail(TV_ERR_INVALID, "rope_scatter: empty cos/sin cache or KV pool");
    }
    const int64_t* strides[] = {a->q_stride, a->k_stride, a->v_stride, a->out_stride};
    for (const int64_t* s : strides) {
        if (s[0] <= 0 || s[1] <= 0 || s[2] <= 0) return fail(TV_ERR_INVALID, "rope_scatter: strides must be positive");
    }
    for (int i = 0; i < 4; ++i) {
        if (a->k_pool_stride[i] <= 0 || a->v_pool_stride[i] <= 0) {
            return fail(TV_ERR_INVALID, "rope_scatter: pool strides must be positive");
        }
    }
    if (a->positions_stride <= 0 || a->slots_stride <= 0 || a->cache_stride_row <= 0 || a->cache_stride_elem <= 0) {
        return fail(TV_ERR_INVALID, "rope_scatter: strides must be positive");
    }
    const int64_t elem = a->dtype == TV_F32 ? 4 : 2;
    const int64_t half_b = (a->head_dim / 2) * elem;
    bool vec = half_b % 16 == 0 && a->q_stride[2] == 1 && a->k_stride[2] == 1 && a->v_stride[2] == 1 &&
               a->out_stride[2] == 1 && a->k_pool_stride[3] == 1 && a->v_pool_stride[3] == 1;
    const void* ptrs[] = {a->q, a->k, a->v, a->out, a->k_pool, a->v_pool};
    for (const void* ptr : ptrs) vec = vec && aligned(ptr, 16);
    const int64_t outer[] = {a->q_stride[0], a->q_stride[1], a->k_stride[0], a->k_stride[1], a->v_stride[0],
                             a->v_stride[1], a->out_stride[0], a->out_stride[1], a->k_pool_stride[0],
                             a->k_pool_stride[1], a->k_pool_stride[2], a->v_pool_stride[0], a->v_pool_stride[1],
                             a->v_pool_stride[2]};
    for (int64_t s : outer) vec = vec && (s * elem) % 16 == 0;

    RopeParams p;
    p.q = a->q;
    p.q_s0 = a->q_stride[0];
    p.q_s1 = a->q_stride[1];
    p.q_s2 = a->q_stride[2];
    p.k = a->k;
    p.k_s0 = a->k_stride[0];
    p.k_s1 = a->k_stride[1];
    p.k_s2 = a->k_stride[2];
    p.v = a->v;
    p.v_s0 = a->v_stride[0];
    p.v_s1 = a->v_stride[1];
    p.v_s2 = a->v_stride[2];
    p.positions = a->positions;
    p.pos_s = a->positions_stride;
    p.pos64 = a->positions_is_int64 != 0;
    p.cache = a->cache;
    p.cache_rows = a->cache_rows;
    p.cache_s0 = a->cache_stride_row;
    p.cache_s1 = a->cache_stride_elem;
    p.cache_f32 = a->cache_dtype == TV_F32;
    p.kp = a->k_pool;
    p.kp_s0 = a->k_pool_stride[0];
    p.kp_s1 = a->k_pool_stride[1];
    p.kp_s2 = a->k_pool_stride[2];
    p.kp_s3 = a->k_pool_stride[3];
    p.vp = a->v_pool;
    p.vp_s0 = a->v_pool_stride[0];
    p.vp_s1 = a->v_pool_stride[1];
    p.vp_s2 = a->v_pool_stride[2];
    p.vp_s3 = a->v_pool_stride[3];
    p.pool_pages = a->pool_pages;
    p.page_size = a->page_size;
    p.slots = a->node_slots;
    p.slot_s = a->slots_stride;
    p.slot64 = a->slots_is_int64 != 0;
    p.out = a->out;
    p.o_s0 = a->out_stride[0];
    p.o_s1 = a->out_stride[1];
    p.o_s2 = a->out_stride[2];
    p.q_heads = a->q_heads;
    p.kv_heads = a->kv_heads;
    p.head_dim = a->head_dim;
    p.status = a->status;
    if (a->dtype == TV_BF16) {
        launch<Bf16Ops>(p, a->rows, vec, as_stream(stream));
    } else {
        launch<F32Ops>(p, a->rows, vec, as_stream(stream));
    }
    return check_launch("rope_scatter");
}
