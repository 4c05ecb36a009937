// Ragged packed tree-verify attention over a paged KV pool, written for gfx950.
//
// Semantics (paged_backend.py:116-213): packed query row q of request r, query head
// h, attends to every committed prefix position of r (page table addressed) and to
// the tree nodes of r whose ancestor bit is set (scratch slot addressed), with an
// fp32 online softmax.  GQA: query head h reads KV head h / 4.
//
// Work decomposition (see tv_plan.cpp): one 512-thread workgroup = 8 waves owns
// 256 score rows = HPW KV heads x NPW nodes x 4 query heads, and a key range of the
// request (a prefix chunk, plus the tree on the last chunk).  Each wave owns 32
// score rows (8 nodes x 4 query heads of one KV head).
//
// Per 32-key tile the workgroup stages K and V of its HPW heads in LDS once, and
// every wave of a head reads them from LDS:
//   S^T[32 keys x 32 rows]  = K  . Q^T   (8 x v_mfma_f32_32x32x16_bf16)
//   O^T[128 dims x 32 rows] += V^T . P^T  (8 x v_mfma_f32_32x32x16_bf16)
// Writing the products transposed keeps every per-row quantity (running max, sum,
// rescale factor) in the two lanes (c, c+32) that own row c: the MFMA C layout puts
// column c in lanes c and c+32, so the softmax needs one cross-lane exchange per
// reduction and the O^T rescale needs none.
//
// MFMA 32x32x16 register layouts (gfx950):
//   A (32 x 16): lane l holds row l%32, k-slots 8*(l/32)+0..7
//   B (16 x 32): lane l holds col l%32, k-slots 8*(l/32)+0..7
//   C (32 x 32): lane l, register v holds row 8*(v/4) + 4*(l/32) + v%4, col l%32
// The P^T operand is taken straight from the S^T registers, so the k-slot order of
// the P.V product is a permutation of the tile's keys:
//   k-slot t of lane half g in product kk  <->  key 16*kk + 8*(t/4) + 4*g + t%4.
// V is stored in LDS transposed ([dim][key], keys in that permuted order), so each
// V^T operand is one 16-byte LDS read.
#include <math.h>
#include <stdint.h>

#include "tv_internal.h"

namespace tv {
namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int kHeadDim = 128;
constexpr int kGroups = 4;          // query heads per KV head
constexpr int kThreads = 512;       // 8 waves
constexpr int kRowsPerItem = 256;
constexpr int kTileKeys = 32;
constexpr int kKRow = kHeadDim + 8;                   // bf16 per LDS K row (272 B: conflict-free reads)
constexpr int kVRow = kTileKeys + 8;                  // bf16 per LDS V^T row (80 B: conflict-free reads)
constexpr int kKHeadBytes = kTileKeys * kKRow * 2;    // 8704
constexpr int kVHeadBytes = kHeadDim * kVRow * 2;     // 10240
constexpr int kMaxHpw = 4;
constexpr int kStageBytes = kMaxHpw * (kKHeadBytes + kVHeadBytes);  // 75776
constexpr int kLdsBytes = 2 * kStageBytes;                          // 151552 of gfx950's 160 KiB
constexpr float kLog2e = 1.4426950408889634f;

template <typename T>
struct Mfma;
template <>
struct Mfma<__bf16> {
    typedef bf16x8_t vec;
    static __device__ __forceinline__ f32x16 run(vec a, vec b, f32x16 c) {
        return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
    }
};
template <>
struct Mfma<_Float16> {
    typedef f16x8_t vec;
    static __device__ __forceinline__ f32x16 run(vec a, vec b, f32x16 c) {
        return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
    }
};

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
    const uint64_t* anc;
    int32_t words;
    int32_t num_requests;
    int32_t num_kv_heads;
    int32_t block_size;
    float c;  // softmax scale * log2(e)
    const int32_t* items;
    const int32_t* groups;
    float* ws_o;
    float2* ws_ml;
    int32_t* status;
};

// Element offset of key `key` of tile `t` within its page row, for K and V.
// Returns false (and reports) when the key is outside the item's range or its
// page lies outside the pool; such keys are neither loaded nor visible.
struct KeyRow {
    int64_t k_off, v_off;
    bool valid;
};

__device__ __forceinline__ KeyRow key_row(const AttnParams& p, int r, int qbase, int kbeg, int kend, int ntp,
                                          int tree_end, int t, int key) {
    KeyRow out{0, 0, false};
    int64_t page, off;
    if (t < ntp) {
        const int pos = kbeg + kTileKeys * t + key;
        if (pos >= kend) return out;
        page = p.tables[static_cast<int64_t>(r) * p.t_s0 + pos / p.block_size];
        off = pos % p.block_size;
    } else {
        const int m = kTileKeys * (t - ntp) + key;
        if (m >= tree_end) return out;
        const int64_t slot = p.tree_slots[qbase + m];
        if (slot < 0) {
            set_status(p.status, TV_STATUS_BAD_PAGE);
            return out;
        }
        page = slot / p.block_size;
        off = slot - page * p.block_size;
    }
    if (page < 0 || page >= p.num_blocks) {
        set_status(p.status, TV_STATUS_BAD_PAGE);
        return out;
    }
    out.k_off = page * p.k_s0 + off * p.k_s1;
    out.v_off = page * p.v_s0 + off * p.v_s1;
    out.valid = true;
    return out;
}

__device__ __forceinline__ uint32_t pack_lo(uint32_t a, uint32_t b) { return (a & 0xffffu) | (b << 16); }
__device__ __forceinline__ uint32_t pack_hi(uint32_t a, uint32_t b) { return (a >> 16) | (b & 0xffff0000u); }

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

template <typename T>
__global__ void __launch_bounds__(kThreads)
tree_attention_kernel(const AttnParams p) {
    typedef typename Mfma<T>::vec V8;
    __shared__ __attribute__((aligned(16))) char smem[kLdsBytes];

    const int32_t* it = p.items + 8 * blockIdx.x;
    const int r = it[0], h0 = it[1], n0 = it[2], kbeg = it[3], kend = it[4];
    const int flags = it[5], slot = it[6], hpw = it[7];
    if (r < 0 || r >= p.num_requests) {
        if (threadIdx.x == 0) set_status(p.status, TV_STATUS_BAD_REQUEST);
        return;
    }
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, c = lane & 31, g = lane >> 5;
    const int wph = 8 / hpw;  // waves per KV head
    const int npw = 8 * wph;  // nodes per workgroup
    const int hl = wave / wph;
    const int head = h0 + hl;
    const int nsub = wave - hl * wph;
    const int P = p.plen[r], tn = p.cnt[r], qbase = p.cu[r];
    const int node = n0 + 8 * nsub + (c >> 2);
    const int qh = head * kGroups + (c & 3);
    const bool head_ok = head < p.num_kv_heads;
    const bool wave_active = head_ok && (n0 + 8 * nsub) < tn;  // uniform per wave
    const bool row_ok = head_ok && node < tn;
    const int tree_end = (flags & 1) ? min(tn, n0 + npw) : 0;
    const int ntp = (kend - kbeg + kTileKeys - 1) / kTileKeys;
    const int nt = ntp + (tree_end + kTileKeys - 1) / kTileKeys;

    // Q^T operand: lane (c, g) holds score row c, dims 16*st + 8*g + 0..7.
    V8 qb[8];
    {
        const T* qrow = static_cast<const T*>(p.q) + static_cast<int64_t>(qbase + node) * p.q_s0 +
                        static_cast<int64_t>(qh) * p.q_s1 + 8 * g;
#pragma unroll
        for (int st = 0; st < 8; ++st) {
            u32x4 raw = {0u, 0u, 0u, 0u};
            if (row_ok) raw = *reinterpret_cast<const u32x4*>(qrow + 16 * st);
            qb[st] = __builtin_bit_cast(V8, raw);
        }
    }

    // Staging assignment.  K: thread -> (key, 16-byte dim chunk), one per head.
    // V: unit -> (key quad a, dim quad u, head); 4 keys x 4 dims per unit.
    const int k_key = tid >> 4, k_chunk = tid & 15;
    const int v_units = 256 * hpw;
    const T* kbase = static_cast<const T*>(p.k);
    const T* vbase = static_cast<const T*>(p.v);
    u32x4 kreg[kMaxHpw];
    u32x2 vreg[2][4];

    auto gload = [&](int t) {
        const KeyRow kr = key_row(p, r, qbase, kbeg, kend, ntp, tree_end, t, k_key);
#pragma unroll
        for (int j = 0; j < kMaxHpw; ++j) {
            u32x4 x = {0u, 0u, 0u, 0u};
            if (j < hpw && kr.valid && h0 + j < p.num_kv_heads) {
                x = *reinterpret_cast<const u32x4*>(kbase + kr.k_off + static_cast<int64_t>(h0 + j) * p.k_s2 +
                                                    8 * k_chunk);
            }
            kreg[j] = x;
        }
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const int id = tid + kThreads * j;
            const int a = id & 7, u = (id >> 3) & 31, vh = id >> 8;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                u32x2 x = {0u, 0u};
                if (id < v_units && h0 + vh < p.num_kv_heads) {
                    const KeyRow vr = key_row(p, r, qbase, kbeg, kend, ntp, tree_end, t, 4 * a + i);
                    if (vr.valid) {
                        x = *reinterpret_cast<const u32x2*>(vbase + vr.v_off + static_cast<int64_t>(h0 + vh) * p.v_s2 +
                                                            4 * u);
                    }
                }
                vreg[j][i] = x;
            }
        }
    };

    auto sstore = [&](int stage) {
        char* base = smem + stage * kStageBytes;
#pragma unroll
        for (int j = 0; j < kMaxHpw; ++j) {
            if (j < hpw) {
                *reinterpret_cast<u32x4*>(base + j * kKHeadBytes + (k_key * kKRow + 8 * k_chunk) * 2) = kreg[j];
            }
        }
        char* vt = base + hpw * kKHeadBytes;
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const int id = tid + kThreads * j;
            if (id < v_units) {
                const int a = id & 7, u = (id >> 3) & 31, vh = id >> 8;
                const int p0 = 16 * (a >> 2) + 8 * (a & 1) + 4 * ((a >> 1) & 1);
                char* dst = vt + vh * kVHeadBytes + ((4 * u) * kVRow + p0) * 2;
                const u32x2* k4 = vreg[j];
                const u32x2 d0 = {pack_lo(k4[0].x, k4[1].x), pack_lo(k4[2].x, k4[3].x)};
                const u32x2 d1 = {pack_hi(k4[0].x, k4[1].x), pack_hi(k4[2].x, k4[3].x)};
                const u32x2 d2 = {pack_lo(k4[0].y, k4[1].y), pack_lo(k4[2].y, k4[3].y)};
                const u32x2 d3 = {pack_hi(k4[0].y, k4[1].y), pack_hi(k4[2].y, k4[3].y)};
                *reinterpret_cast<u32x2*>(dst + 0 * kVRow * 2) = d0;
                *reinterpret_cast<u32x2*>(dst + 1 * kVRow * 2) = d1;
                *reinterpret_cast<u32x2*>(dst + 2 * kVRow * 2) = d2;
                *reinterpret_cast<u32x2*>(dst + 3 * kVRow * 2) = d3;
            }
        }
    };

    f32x16 acc[4];
#pragma unroll
    for (int db = 0; db < 4; ++db) acc[db] = f32x16{};
    float m_run = -INFINITY, l_run = 0.f;
    const float cs = p.c;

    auto compute = [&](int stage, int t) {
        const char* kh = smem + stage * kStageBytes + hl * kKHeadBytes;
        f32x16 s = f32x16{};
#pragma unroll
        for (int st = 0; st < 8; ++st) {
            const V8 a = __builtin_bit_cast(V8, *reinterpret_cast<const u32x4*>(kh + (c * kKRow + 16 * st + 8 * g) * 2));
            s = Mfma<T>::run(a, qb[st], s);
        }
        // Visibility of the 16 keys this lane holds: key index 8*(v/4) + 4*g + v%4.
        if (t < ntp) {
            const int nvalid = kend - (kbeg + kTileKeys * t);
            if (nvalid < kTileKeys) {
#pragma unroll
                for (int v = 0; v < 16; ++v) {
                    const int key = 8 * (v >> 2) + 4 * g + (v & 3);
                    if (key >= nvalid) s[v] = -INFINITY;
                }
            }
        } else {
            const int m0 = kTileKeys * (t - ntp);
            uint32_t bits = 0;
            if (row_ok) {
                bits = static_cast<uint32_t>(p.anc[static_cast<int64_t>(qbase + node) * p.words + (m0 >> 6)] >>
                                             (m0 & 32));
            }
#pragma unroll
            for (int v = 0; v < 16; ++v) {
                const int key = 8 * (v >> 2) + 4 * g + (v & 3);
                if (!((bits >> key) & 1u)) s[v] = -INFINITY;
            }
        }
        float mx = s[0];
#pragma unroll
        for (int v = 1; v < 16; ++v) mx = fmaxf(mx, s[v]);
        mx = fmaxf(mx, __shfl_xor(mx, 32));
        const float m_new = fmaxf(m_run, mx);
        const float m_use = (m_new == -INFINITY) ? 0.f : m_new;
        const float mc = m_use * cs;
        const float alpha = __builtin_amdgcn_exp2f(m_run * cs - mc);
        float pr[16];
        float ps = 0.f;
#pragma unroll
        for (int v = 0; v < 16; ++v) {
            pr[v] = __builtin_amdgcn_exp2f(fmaf(s[v], cs, -mc));
            ps += pr[v];
        }
        ps += __shfl_xor(ps, 32);
        l_run = l_run * alpha + ps;
        m_run = m_new;
#pragma unroll
        for (int db = 0; db < 4; ++db) acc[db] *= alpha;
        V8 pb[2];
#pragma unroll
        for (int kk = 0; kk < 2; ++kk) {
#pragma unroll
            for (int t8 = 0; t8 < 8; ++t8) pb[kk][t8] = static_cast<T>(pr[8 * kk + t8]);
        }
        const char* vh = smem + stage * kStageBytes + hpw * kKHeadBytes + hl * kVHeadBytes;
#pragma unroll
        for (int db = 0; db < 4; ++db) {
#pragma unroll
            for (int kk = 0; kk < 2; ++kk) {
                const V8 a = __builtin_bit_cast(
                    V8, *reinterpret_cast<const u32x4*>(vh + ((32 * db + c) * kVRow + 16 * kk + 8 * g) * 2));
                acc[db] = Mfma<T>::run(a, pb[kk], acc[db]);
            }
        }
    };

    if (nt > 0) {
        gload(0);
        sstore(0);
    }
    if (nt > 1) gload(1);
    __syncthreads();
    for (int t = 0; t < nt; ++t) {
        if (wave_active) compute(t & 1, t);
        if (t + 1 < nt) sstore((t + 1) & 1);
        if (t + 2 < nt) gload(t + 2);
        __syncthreads();
    }

    if (!wave_active || !row_ok) return;
    const int wr = wave * 32 + c;  // score row within the item
    if (slot < 0) {
        const float inv = 1.f / l_run;
        const int64_t row = qbase + node;
#pragma unroll
        for (int db = 0; db < 4; ++db) {
#pragma unroll
            for (int i4 = 0; i4 < 4; ++i4) {
                const f32x4 o = {acc[db][4 * i4] * inv, acc[db][4 * i4 + 1] * inv, acc[db][4 * i4 + 2] * inv,
                                 acc[db][4 * i4 + 3] * inv};
                store_out4<T>(p, row, qh, 32 * db + 8 * i4 + 4 * g, o);
            }
        }
    } else {
        float* wo = p.ws_o + (static_cast<int64_t>(slot) * kRowsPerItem + wr) * kHeadDim;
#pragma unroll
        for (int db = 0; db < 4; ++db) {
#pragma unroll
            for (int i4 = 0; i4 < 4; ++i4) {
                const f32x4 o = {acc[db][4 * i4], acc[db][4 * i4 + 1], acc[db][4 * i4 + 2], acc[db][4 * i4 + 3]};
                *reinterpret_cast<f32x4*>(wo + 32 * db + 8 * i4 + 4 * g) = o;
            }
        }
        if (g == 0) p.ws_ml[static_cast<int64_t>(slot) * kRowsPerItem + wr] = make_float2(m_run, l_run);
    }
}

// Combines the split-K partials of one (request, head group, node block).
template <typename T>
__global__ void __launch_bounds__(256)
merge_partials_kernel(const AttnParams p) {
    const int32_t* gr = p.groups + 8 * blockIdx.x;
    const int r = gr[0], h0 = gr[1], n0 = gr[2], hpw = gr[3], first = gr[4], ns = gr[5];
    if (r < 0 || r >= p.num_requests) return;
    const int wph = 8 / hpw;
    const int tn = p.cnt[r], qbase = p.cu[r];
    for (int idx = threadIdx.x; idx < kRowsPerItem * 32; idx += blockDim.x) {
        const int wr = idx >> 5, quad = idx & 31;
        const int wave = wr >> 5, c = wr & 31;
        const int hl = wave / wph;
        const int head = h0 + hl;
        const int node = n0 + 8 * (wave - hl * wph) + (c >> 2);
        if (head >= p.num_kv_heads || node >= tn) continue;
        const int qh = head * kGroups + (c & 3);
        float m = -INFINITY;
        for (int s = 0; s < ns; ++s) m = fmaxf(m, p.ws_ml[static_cast<int64_t>(first + s) * kRowsPerItem + wr].x);
        const float mc = (m == -INFINITY ? 0.f : m) * p.c;
        float l = 0.f;
        f32x4 o = {0.f, 0.f, 0.f, 0.f};
        for (int s = 0; s < ns; ++s) {
            const int64_t pr = static_cast<int64_t>(first + s) * kRowsPerItem + wr;
            const float2 ml = p.ws_ml[pr];
            const float w = __builtin_amdgcn_exp2f(ml.x * p.c - mc);
            l += ml.y * w;
            o += *reinterpret_cast<const f32x4*>(p.ws_o + pr * kHeadDim + 4 * quad) * w;
        }
        const float inv = 1.f / l;
        store_out4<T>(p, qbase + node, qh, 4 * quad, o * inv);
    }
}

__global__ void __launch_bounds__(256)
pack_ancestor_kernel(const float* __restrict__ bias, const int64_t* __restrict__ bias_off,
                     const int32_t* __restrict__ q2r, const int32_t* __restrict__ local,
                     const int32_t* __restrict__ counts, int32_t total_q, int32_t num_requests, int32_t words,
                     uint64_t* __restrict__ out, int32_t* status) {
    const int64_t idx = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (idx >= static_cast<int64_t>(total_q) * words) return;
    const int64_t q = idx / words;
    const int w = static_cast<int>(idx - q * words);
    const int r = q2r[q];
    uint64_t word = 0;
    if (r < 0 || r >= num_requests) {
        set_status(status, TV_STATUS_BAD_REQUEST);
    } else {
        const int i = local[q];
        const int tn = counts[r];
        if (i >= 0 && i < tn) {
            const float* row = bias + bias_off[r] + static_cast<int64_t>(i) * tn;
            for (int b = 0; b < 64; ++b) {
                const int m = 64 * w + b;
                if (m < tn && m <= i && row[m] == 0.f) word |= 1ull << b;
            }
        } else {
            set_status(status, TV_STATUS_BAD_REQUEST);
        }
    }
    out[idx] = word;
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
    const int64_t n = static_cast<int64_t>(total_queries) * words_per_row;
    const int64_t blocks = (n + 255) / 256;
    hipLaunchKernelGGL(pack_ancestor_kernel, dim3(blocks), dim3(256), 0, as_stream(stream), qq_bias,
                       qq_bias_offsets, query_to_request, query_local_row, node_counts, total_queries,
                       num_requests, words_per_row, words, status);
    return check_launch("pack_ancestor_words");
}

extern "C" int tv_tree_attention(const tv_tree_attention_args* a, void* stream) {
    clear_error();
    if (!a) return fail(TV_ERR_INVALID, "tree_attention: null args");
    if (a->head_dim != kHeadDim) {
        return fail(TV_ERR_UNSUPPORTED, "tree_attention: head_dim %d (implemented: 128)", a->head_dim);
    }
    if (a->num_kv_heads < 1 || a->num_q_heads != kGroups * a->num_kv_heads) {
        return fail(TV_ERR_UNSUPPORTED, "tree_attention: %d query heads over %d KV heads (implemented: 4 per KV head)",
                    a->num_q_heads, a->num_kv_heads);
    }
    if (a->block_size < 32 || a->block_size % 32) {
        return fail(TV_ERR_UNSUPPORTED, "tree_attention: block_size %d is not a multiple of 32", a->block_size);
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
    const int out_elem = a->out_dtype == TV_F32 ? 4 : 2;
    if ((a->out_stride_row | a->out_stride_head) % (16 / out_elem) || !aligned(a->out, 16)) {
        return fail(TV_ERR_UNSUPPORTED, "tree_attention: output rows must be 16-byte aligned");
    }
    if (a->num_requests < 1 || a->total_queries < 0 || a->num_items < 0 || a->num_groups < 0) {
        return fail(TV_ERR_INVALID, "tree_attention: invalid counts");
    }
    if (a->num_items == 0) return TV_OK;
    if (!a->q || !a->k_pool || !a->v_pool || !a->out || !a->cu_seqlens_q || !a->prefix_lens || !a->node_counts ||
        !a->block_tables || !a->tree_slots || !a->ancestor_words || !a->items) {
        return fail(TV_ERR_INVALID, "tree_attention: null pointer");
    }
    const int64_t o_bytes = static_cast<int64_t>(a->num_partial_slots) * kRowsPerItem * kHeadDim * 4;
    const int64_t o_span = (o_bytes + 255) / 256 * 256;
    const int64_t need = a->num_partial_slots ? o_span + (static_cast<int64_t>(a->num_partial_slots) * kRowsPerItem * 8 + 255) / 256 * 256 : 0;
    if (a->num_groups > 0 && (!a->groups || !a->workspace)) {
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
    p.anc = a->ancestor_words;
    p.words = a->ancestor_words_per_row;
    p.num_requests = a->num_requests;
    p.num_kv_heads = a->num_kv_heads;
    p.block_size = a->block_size;
    p.c = a->scale * kLog2e;
    p.items = a->items;
    p.groups = a->groups;
    p.ws_o = static_cast<float*>(a->workspace);
    p.ws_ml = a->workspace ? reinterpret_cast<float2*>(static_cast<char*>(a->workspace) + o_span) : nullptr;
    p.status = a->status;
    hipStream_t s = as_stream(stream);
    if (a->in_dtype == TV_BF16) {
        hipLaunchKernelGGL(tree_attention_kernel<__bf16>, dim3(a->num_items), dim3(kThreads), 0, s, p);
        if (a->num_groups > 0) {
            hipLaunchKernelGGL(merge_partials_kernel<__bf16>, dim3(a->num_groups), dim3(256), 0, s, p);
        }
    } else {
        hipLaunchKernelGGL(tree_attention_kernel<_Float16>, dim3(a->num_items), dim3(kThreads), 0, s, p);
        if (a->num_groups > 0) {
            hipLaunchKernelGGL(merge_partials_kernel<_Float16>, dim3(a->num_groups), dim3(256), 0, s, p);
        }
    }
    return check_launch("tree_attention");
}
