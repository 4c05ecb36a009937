/*
 * verify_round.c - one tree-verification round through the C ABI alone (no Python, no torch).
 *
 * A caller that owns its own device buffers (a C/C++ serving engine, or the reference's
 * runner binding the library through ctypes) makes these calls per layer and round:
 *
 *   1. tv_store_kvcache        append the round's tree K/V rows into their scratch slots
 *   2. tv_pack_ancestor_words  the tree visibility bits from the 0 / -inf qq_bias
 *   3. tv_tree_attention_plan  the host work plan (once per metadata), copied to the device
 *   4. tv_tree_attention       the packed ragged tree attention over the paged pool
 *   5. tv_copy_accepted_kv     commit one accepted path from scratch into the request's pages
 *
 * The program builds a small two-request batch with shuffled pages (prefixes of 300 and 70
 * tokens, trees of 16 and 9 nodes, 8 query heads over 2 KV heads, head_dim 128, pages of
 * 64 keys, every unused pool row NaN), runs the five calls, and checks them on the host:
 * the append and the commit byte for byte against the expected pool, the attention
 * against a double-precision softmax over each row's visible keys (the tolerance of the
 * bf16 path: max-abs 2e-2, mean-abs 2e-3).  It prints one line and exits 0 when every
 * check holds.
 *
 * Build (from the repository root; nano-vllm-jetspec_amd/build.py does this):
 *   gcc -O2 -std=c11 -D__HIP_PLATFORM_AMD__ -I/opt/rocm/include -Iinclude \
 *       nano-vllm-jetspec_amd/examples/verify_round.c \
 *       -Lnano-vllm-jetspec_amd/jetspec_amd -ltreeverify -L/opt/rocm/lib -lamdhip64 -lm \
 *       -Wl,-rpath,'$ORIGIN/../jetspec_amd' -Wl,-rpath,/opt/rocm/lib \
 *       -o nano-vllm-jetspec_amd/examples/verify_round
 */
#include <hip/hip_runtime_api.h>
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "treeverify.h"

enum { R = 2, HKV = 2, G = 4, HQ = HKV * G, D = 128, B = 64, PAGES = 12, LAYERS = 1 };
static const int kPrefix[R] = {300, 70};
static const int kNodes[R] = {16, 9};

#define ROW (HKV * D)                 /* elements of one pool slot row (all KV heads) */
#define SLOTS (PAGES * B)
#define CHECK_HIP(x)                                                                        \
    do {                                                                                    \
        hipError_t e_ = (x);                                                                \
        if (e_ != hipSuccess) {                                                             \
            fprintf(stderr, "verify_round: %s failed: %s\n", #x, hipGetErrorString(e_));    \
            return 2;                                                                       \
        }                                                                                   \
    } while (0)
#define CHECK_TV(x)                                                                         \
    do {                                                                                    \
        int c_ = (x);                                                                       \
        if (c_ != TV_OK) {                                                                  \
            fprintf(stderr, "verify_round: %s returned %d: %s\n", #x, c_, tv_last_error()); \
            return 2;                                                                       \
        }                                                                                   \
    } while (0)

/* bf16 <-> float, round to nearest even. */
static uint16_t to_bf16(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    if ((u & 0x7fffffffu) > 0x7f800000u) return 0x7fc0u;
    return (uint16_t)((u + 0x7fffu + ((u >> 16) & 1u)) >> 16);
}
static double from_bf16(uint16_t h) {
    uint32_t u = (uint32_t)h << 16;
    float f;
    memcpy(&f, &u, 4);
    return f;
}

/* Deterministic N(0,1)-ish values: a 64-bit LCG through the sum of four uniforms. */
static uint64_t rng_state = 0x9e3779b97f4a7c15ull;
static double uniform(void) {
    rng_state = rng_state * 6364136223846793005ull + 1442695040888963407ull;
    return (double)(rng_state >> 11) / 9007199254740992.0;
}
static uint16_t random_bf16(void) {
    double s = uniform() + uniform() + uniform() + uniform() - 2.0;
    return to_bf16((float)(s * 1.7320508));
}

int main(void) {
    int device_count = 0;
    if (hipGetDeviceCount(&device_count) != hipSuccess || device_count < 1) {
        fprintf(stderr, "verify_round: no GPU\n");
        return 2;
    }
    if (tv_abi_version() != TV_ABI_VERSION) {
        fprintf(stderr, "verify_round: library ABI %d, header %d\n", tv_abi_version(), TV_ABI_VERSION);
        return 2;
    }
    int cus = 0;
    CHECK_HIP(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, 0));

    /* Pages: a shuffled pool; request r owns ceil(P_r / B) pages, the trees share one
     * scratch page that no prefix uses. */
    int order[PAGES];
    for (int i = 0; i < PAGES; ++i) order[i] = i;
    for (int i = PAGES - 1; i > 0; --i) {
        int j = (int)(uniform() * (i + 1));
        int t = order[i];
        order[i] = order[j];
        order[j] = t;
    }
    int table_width = 0, cursor = 0, table[R][8];
    for (int r = 0; r < R; ++r) {
        int n = (kPrefix[r] + B - 1) / B;
        if (n > table_width) table_width = n;
        for (int i = 0; i < 8; ++i) table[r][i] = i < n ? order[cursor + i] : -1;
        cursor += n;
    }
    const int scratch_page = order[cursor];

    /* Packed rows and trees: request 0 a heap (parent (i-1)/2), request 1 a chain. */
    int cu[R + 1] = {0}, total = 0;
    for (int r = 0; r < R; ++r) cu[r + 1] = cu[r] + kNodes[r];
    total = cu[R];
    int parent[64], q2r[64], local[64];
    int64_t tree_slot[64], bias_off[R + 1] = {0};
    for (int r = 0; r < R; ++r) {
        for (int i = 0; i < kNodes[r]; ++i) {
            int q = cu[r] + i;
            parent[q] = i == 0 ? -1 : (r == 0 ? (i - 1) / 2 : i - 1);
            q2r[q] = r;
            local[q] = i;
            tree_slot[q] = (int64_t)scratch_page * B + (int64_t)((q * 37) % B);  /* scattered, unique */
        }
        bias_off[r + 1] = bias_off[r] + (int64_t)kNodes[r] * kNodes[r];
    }
    float* bias = malloc(sizeof(float) * (size_t)bias_off[R]);
    for (int r = 0; r < R; ++r) {
        int n = kNodes[r];
        for (int i = 0; i < n; ++i) {
            for (int m = 0; m < n; ++m) bias[bias_off[r] + (int64_t)i * n + m] = -INFINITY;
            for (int a = i; a >= 0; a = parent[cu[r] + a]) bias[bias_off[r] + (int64_t)i * n + a] = 0.f;
        }
    }

    /* Host pool [2][LAYERS][PAGES][B][HKV][D]: prefix rows random, everything else NaN. */
    const size_t plane = (size_t)SLOTS * ROW;
    uint16_t* pool = malloc(sizeof(uint16_t) * 2 * plane);
    for (size_t i = 0; i < 2 * plane; ++i) pool[i] = 0x7fc0u;
    for (int r = 0; r < R; ++r) {
        for (int pos = 0; pos < kPrefix[r]; ++pos) {
            size_t slot = (size_t)table[r][pos / B] * B + pos % B;
            for (int kv = 0; kv < 2; ++kv)
                for (int e = 0; e < ROW; ++e) pool[kv * plane + slot * ROW + e] = random_bf16();
        }
    }
    uint16_t* new_kv = malloc(sizeof(uint16_t) * 2 * (size_t)total * ROW);   /* [2][Q][HKV][D] */
    for (size_t i = 0; i < 2 * (size_t)total * ROW; ++i) new_kv[i] = random_bf16();
    uint16_t* q = malloc(sizeof(uint16_t) * (size_t)total * HQ * D);
    for (size_t i = 0; i < (size_t)total * HQ * D; ++i) q[i] = random_bf16();
    int32_t tables_i32[R * 8];
    for (int r = 0; r < R; ++r)
        for (int i = 0; i < table_width; ++i) tables_i32[r * table_width + i] = table[r][i];

    /* Device buffers. */
    void *d_pool, *d_new, *d_q, *d_out, *d_bias, *d_cu, *d_plen, *d_cnt, *d_tab, *d_slots, *d_q2r, *d_loc,
        *d_boff, *d_words, *d_status;
    CHECK_HIP(hipMalloc(&d_pool, sizeof(uint16_t) * 2 * plane));
    CHECK_HIP(hipMalloc(&d_new, sizeof(uint16_t) * 2 * (size_t)total * ROW));
    CHECK_HIP(hipMalloc(&d_q, sizeof(uint16_t) * (size_t)total * HQ * D));
    CHECK_HIP(hipMalloc(&d_out, sizeof(uint16_t) * (size_t)total * HQ * D));
    CHECK_HIP(hipMalloc(&d_bias, sizeof(float) * (size_t)bias_off[R]));
    CHECK_HIP(hipMalloc(&d_cu, sizeof(cu)));
    CHECK_HIP(hipMalloc(&d_plen, sizeof(kPrefix)));
    CHECK_HIP(hipMalloc(&d_cnt, sizeof(kNodes)));
    CHECK_HIP(hipMalloc(&d_tab, sizeof(int32_t) * R * table_width));
    CHECK_HIP(hipMalloc(&d_slots, sizeof(int64_t) * total));
    CHECK_HIP(hipMalloc(&d_q2r, sizeof(int32_t) * total));
    CHECK_HIP(hipMalloc(&d_loc, sizeof(int32_t) * total));
    CHECK_HIP(hipMalloc(&d_boff, sizeof(bias_off)));
    CHECK_HIP(hipMalloc(&d_words, sizeof(uint64_t) * total));
    CHECK_HIP(hipMalloc(&d_status, sizeof(int32_t)));
    CHECK_HIP(hipMemcpy(d_pool, pool, sizeof(uint16_t) * 2 * plane, hipMemcpyHostToDevice));
    CHECK_HIP(hipMemcpy(d_new, new_kv, sizeof(uint16_t) * 2 * (size_t)total * ROW, hipMemcpyHostToDevice));
    CHECK_HIP(hipMemcpy(d_q, q, sizeof(uint16_t) * (size_t)total * HQ * D, hipMemcpyHostToDevice));
    CHECK_HIP(hipMemcpy(d_bias, bias, sizeof(float) * (size_t)bias_off[R], hipMemcpyHostToDevice));
    CHECK_HIP(hipMemcpy(d_cu, cu, sizeof(cu), hipMemcpyHostToDevice));
    CHECK_HIP(hipMemcpy(d_plen, kPrefix, sizeof(kPrefix), hipMemcpyHostToDevice));
    CHECK_HIP(hipMemcpy(d_cnt, kNodes, sizeof(kNodes), hipMemcpyHostToDevice));
    CHECK_HIP(hipMemcpy(d_tab, tables_i32, sizeof(int32_t) * R * table_width, hipMemcpyHostToDevice));
    CHECK_HIP(hipMemcpy(d_slots, tree_slot, sizeof(int64_t) * total, hipMemcpyHostToDevice));
    int32_t q2r32[64], loc32[64];
    for (int i = 0; i < total; ++i) {
        q2r32[i] = q2r[i];
        loc32[i] = local[i];
    }
    CHECK_HIP(hipMemcpy(d_q2r, q2r32, sizeof(int32_t) * total, hipMemcpyHostToDevice));
    CHECK_HIP(hipMemcpy(d_loc, loc32, sizeof(int32_t) * total, hipMemcpyHostToDevice));
    CHECK_HIP(hipMemcpy(d_boff, bias_off, sizeof(bias_off), hipMemcpyHostToDevice));
    CHECK_HIP(hipMemset(d_status, 0, sizeof(int32_t)));
    uint16_t* d_k = (uint16_t*)d_pool;            /* pool[0, 0] */
    uint16_t* d_v = (uint16_t*)d_pool + plane;    /* pool[1, 0] */

    /* 1. Append the tree K/V rows into their scratch slots. */
    CHECK_TV(tv_store_kvcache(d_new, ROW, (uint16_t*)d_new + (size_t)total * ROW, ROW, d_k, d_v, SLOTS, d_slots, 1,
                              total, ROW, 2, (int32_t*)d_status, NULL));
    for (int i = 0; i < total; ++i)
        for (int kv = 0; kv < 2; ++kv)
            memcpy(pool + kv * plane + (size_t)tree_slot[i] * ROW, new_kv + ((size_t)kv * total + i) * ROW,
                   sizeof(uint16_t) * ROW);

    /* 2. Visibility bits (one 64-bit word per row: trees of at most 64 nodes). */
    CHECK_TV(tv_pack_ancestor_words((const float*)d_bias, (const int64_t*)d_boff, (const int32_t*)d_q2r,
                                    (const int32_t*)d_loc, (const int32_t*)d_cnt, total, R, 1, (uint64_t*)d_words,
                                    (int32_t*)d_status, NULL));

    /* 3. The work plan, then its device copy and the split-K workspace. */
    tv_attention_plan_info info;
    CHECK_TV(tv_tree_attention_plan(kPrefix, kNodes, R, HKV, G, B, cus, 0, NULL, NULL, &info));
    int32_t* items = calloc((size_t)info.num_items * 8 + 8, sizeof(int32_t));
    int32_t* groups = calloc((size_t)info.num_groups * 8 + 8, sizeof(int32_t));
    CHECK_TV(tv_tree_attention_plan(kPrefix, kNodes, R, HKV, G, B, cus, 0, items, groups, &info));
    void *d_items, *d_groups, *d_ws = NULL;
    CHECK_HIP(hipMalloc(&d_items, sizeof(int32_t) * ((size_t)info.num_items * 8 + 8)));
    CHECK_HIP(hipMalloc(&d_groups, sizeof(int32_t) * ((size_t)info.num_groups * 8 + 8)));
    CHECK_HIP(hipMemcpy(d_items, items, sizeof(int32_t) * (size_t)info.num_items * 8, hipMemcpyHostToDevice));
    if (info.num_groups)
        CHECK_HIP(hipMemcpy(d_groups, groups, sizeof(int32_t) * (size_t)info.num_groups * 8, hipMemcpyHostToDevice));
    if (info.workspace_bytes) CHECK_HIP(hipMalloc(&d_ws, (size_t)info.workspace_bytes));

    /* 4. Attention. */
    tv_tree_attention_args a;
    memset(&a, 0, sizeof(a));
    if (tv_sizeof_tree_attention_args() != (int64_t)sizeof(a)) {
        fprintf(stderr, "verify_round: argument struct layout differs from the library's\n");
        return 2;
    }
    a.q = d_q;
    a.q_stride_row = HQ * D;
    a.q_stride_head = D;
    a.k_pool = d_k;
    a.v_pool = d_v;
    const int64_t pool_stride[4] = {(int64_t)B * ROW, ROW, D, 1};   /* [PAGES, B, HKV, D] */
    memcpy(a.k_stride, pool_stride, sizeof(pool_stride));
    memcpy(a.v_stride, pool_stride, sizeof(pool_stride));
    a.num_blocks = PAGES;
    a.in_dtype = TV_BF16;
    a.out = d_out;
    a.out_stride_row = HQ * D;
    a.out_stride_head = D;
    a.out_dtype = TV_BF16;
    a.cu_seqlens_q = (const int32_t*)d_cu;
    a.prefix_lens = (const int32_t*)d_plen;
    a.node_counts = (const int32_t*)d_cnt;
    a.block_tables = (const int32_t*)d_tab;
    a.block_table_stride = table_width;
    a.tree_slots = (const int64_t*)d_slots;
    a.ancestor_words = (const uint64_t*)d_words;
    a.ancestor_words_per_row = 1;
    a.num_requests = R;
    a.total_queries = total;
    a.num_q_heads = HQ;
    a.num_kv_heads = HKV;
    a.head_dim = D;
    a.block_size = B;
    a.scale = (float)(1.0 / sqrt((double)D));
    a.items = (const int32_t*)d_items;
    a.num_items = info.num_items;
    a.groups = info.num_groups ? (const int32_t*)d_groups : NULL;
    a.num_groups = info.num_groups;
    a.num_partial_slots = info.num_partial_slots;
    a.workspace = d_ws;
    a.workspace_bytes = info.workspace_bytes;
    a.status = (int32_t*)d_status;
    CHECK_TV(tv_tree_attention(&a, NULL));

    /* 5. Commit request 0's accepted path 0 -> 1 -> 3 into positions P0, P0+1, P0+2. */
    const int path[3] = {0, 1, 3};
    int64_t src[3], dst[3];
    for (int i = 0; i < 3; ++i) {
        int pos = kPrefix[0] + i;
        src[i] = tree_slot[cu[0] + path[i]];
        dst[i] = (int64_t)table[0][pos / B] * B + pos % B;
    }
    void *d_src, *d_dst, *d_cws = NULL;
    CHECK_HIP(hipMalloc(&d_src, sizeof(src)));
    CHECK_HIP(hipMalloc(&d_dst, sizeof(dst)));
    CHECK_HIP(hipMemcpy(d_src, src, sizeof(src), hipMemcpyHostToDevice));
    CHECK_HIP(hipMemcpy(d_dst, dst, sizeof(dst), hipMemcpyHostToDevice));
    const int64_t shape6[6] = {2, LAYERS, PAGES, B, HKV, D};
    const int64_t stride6[6] = {(int64_t)LAYERS * plane, (int64_t)plane, (int64_t)B * ROW, ROW, D, 1};
    int64_t cws = tv_copy_accepted_kv_workspace_bytes(3, LAYERS, ROW, 2);
    if (cws > 0) CHECK_HIP(hipMalloc(&d_cws, (size_t)cws));
    int64_t payload = 0;
    /* The commit runs after the attention on the same stream, as in the runner's round. */
    CHECK_TV(tv_copy_accepted_kv(d_pool, shape6, stride6, 2, (const int64_t*)d_src, (const int64_t*)d_dst, 3,
                                 d_cws, cws, &payload, (int32_t*)d_status, NULL));
    for (int i = 0; i < 3; ++i)
        for (int kv = 0; kv < 2; ++kv)
            memcpy(pool + kv * plane + (size_t)dst[i] * ROW, pool + kv * plane + (size_t)src[i] * ROW,
                   sizeof(uint16_t) * ROW);
    CHECK_HIP(hipDeviceSynchronize());

    /* Checks. */
    int failures = 0;
    int32_t status = 0;
    CHECK_HIP(hipMemcpy(&status, d_status, sizeof(status), hipMemcpyDeviceToHost));
    if (status != 0) {
        fprintf(stderr, "verify_round: status bits %d\n", status);
        ++failures;
    }
    if (payload != 2LL * LAYERS * 3 * ROW * 2) {
        fprintf(stderr, "verify_round: commit payload %lld\n", (long long)payload);
        ++failures;
    }
    uint16_t* pool_after = malloc(sizeof(uint16_t) * 2 * plane);
    CHECK_HIP(hipMemcpy(pool_after, d_pool, sizeof(uint16_t) * 2 * plane, hipMemcpyDeviceToHost));
    size_t differing = 0;
    for (size_t i = 0; i < 2 * plane; ++i) differing += pool_after[i] != pool[i];
    if (differing) {
        fprintf(stderr, "verify_round: %zu pool elements differ from the expected append + commit\n", differing);
        ++failures;
    }
    uint16_t* out = malloc(sizeof(uint16_t) * (size_t)total * HQ * D);
    CHECK_HIP(hipMemcpy(out, d_out, sizeof(uint16_t) * (size_t)total * HQ * D, hipMemcpyDeviceToHost));

    /* Double-precision reference: row (r, i), head h sees prefix keys 0..P_r-1 and the tree
     * nodes on its root path; K/V from the host pool as it stood before the commit (the
     * commit only writes positions past every prefix, which no row of this round sees). */
    const double scale = 1.0 / sqrt((double)D);
    double max_abs = 0.0, sum_abs = 0.0;
    double scores[512], acc[D];
    size_t slots[512];
    for (int qi = 0; qi < total; ++qi) {
        const int r = q2r[qi], i = local[qi];
        for (int h = 0; h < HQ; ++h) {
            const int kvh = h / G;
            int n = 0;
            for (int k = 0; k < kPrefix[r]; ++k) slots[n++] = (size_t)table[r][k / B] * B + k % B;
            for (int m = 0; m < kNodes[r]; ++m)
                if (bias[bias_off[r] + (int64_t)i * kNodes[r] + m] == 0.f) slots[n++] = (size_t)tree_slot[cu[r] + m];
            double top = -INFINITY;
            for (int k = 0; k < n; ++k) {
                const uint16_t* key = pool + slots[k] * ROW + (size_t)kvh * D;
                const uint16_t* query = q + ((size_t)qi * HQ + h) * D;
                double dot = 0.0;
                for (int e = 0; e < D; ++e) dot += from_bf16(query[e]) * from_bf16(key[e]);
                scores[k] = dot * scale;
                if (scores[k] > top) top = scores[k];
            }
            double denominator = 0.0;
            for (int e = 0; e < D; ++e) acc[e] = 0.0;
            for (int k = 0; k < n; ++k) {
                const double w = exp(scores[k] - top);
                const uint16_t* value = pool + plane + slots[k] * ROW + (size_t)kvh * D;
                denominator += w;
                for (int e = 0; e < D; ++e) acc[e] += w * from_bf16(value[e]);
            }
            for (int e = 0; e < D; ++e) {
                const double err = fabs(from_bf16(out[((size_t)qi * HQ + h) * D + e]) - acc[e] / denominator);
                if (!(err <= max_abs)) max_abs = err;   /* a NaN output becomes the maximum */
                sum_abs += err;
            }
        }
    }
    const double mean_abs = sum_abs / ((double)total * HQ * D);
    if (!(max_abs <= 2e-2) || !(mean_abs <= 2e-3)) {
        fprintf(stderr, "verify_round: attention max-abs %.3e mean-abs %.3e outside the bf16 gate\n", max_abs,
                mean_abs);
        ++failures;
    }
    printf("verify_round: %d requests, %d tree rows, %d work items; attention max-abs %.2e mean-abs %.2e; "
           "append + commit byte-exact: %s\n", R, total, info.num_items, max_abs, mean_abs, differing ? "no" : "yes");
    printf("verify_round: %s\n", failures ? "FAILED" : "OK");

    void* device_buffers[] = {d_pool, d_new, d_q, d_out, d_bias, d_cu, d_plen, d_cnt, d_tab, d_slots, d_q2r,
                              d_loc, d_boff, d_words, d_status, d_items, d_groups, d_ws, d_src, d_dst, d_cws};
    for (size_t i = 0; i < sizeof(device_buffers) / sizeof(device_buffers[0]); ++i)
        if (device_buffers[i]) CHECK_HIP(hipFree(device_buffers[i]));
    free(out);
    free(pool_after);
    free(items);
    free(groups);
    free(q);
    free(new_kv);
    free(pool);
    free(bias);
    return failures ? 1 : 0;
}
