/*
 * tv_oracle.c - CPU restatement of the reference's tree-verify hot path.
 *
 * TEST INFRASTRUCTURE ONLY.  Nothing in the product (nano-vllm-jetspec_amd/) links,
 * loads or calls this code; only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg use it, as the checker.
 *
 * Each function restates one reference algorithm (file:line under the reference
 * repository) literally, in double precision where arithmetic is involved:
 *   oracle_store_kvcache      layers/attention.py:15-45
 *   oracle_copy_accepted_kv   speculative/jetspec/state.py:64-86
 *   oracle_tree_attention     speculative/jetspec/paged_backend.py:116-213
 * Pinning (tests/test_oracle_pins.py): reference KATs, an independent parent-chain
 * brute force, closed forms, and planted-mistake checks.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

/*
 * layers/attention.py:15-35 - program idx: slot = slot_mapping[idx]; if slot == -1
 * return; copy D elements of key/value row idx to cache offset slot * D.
 * Rows are handled as bytes (row_bytes = D * element size).
 */
void oracle_store_kvcache(const uint8_t* key, int64_t key_row_stride_bytes, const uint8_t* value,
                          int64_t value_row_stride_bytes, uint8_t* k_cache, uint8_t* v_cache,
                          const int64_t* slot_mapping, int64_t num_rows, int64_t row_bytes) {
    for (int64_t i = 0; i < num_rows; ++i) {
        const int64_t slot = slot_mapping[i];
        if (slot == -1) continue;
        memcpy(k_cache + slot * row_bytes, key + i * key_row_stride_bytes, (size_t)row_bytes);
        memcpy(v_cache + slot * row_bytes, value + i * value_row_stride_bytes, (size_t)row_bytes);
    }
}

/*
 * speculative/jetspec/state.py:76-86 - accepted = pool[:, :, src // B, src % B]
 * (a materialised gather), then pool[:, :, dst // B, dst % B] = accepted.
 * Dense pool [2][layers][blocks][block_size][row_bytes].  `staging` holds
 * 2 * layers * n rows.  Returns the payload byte count (accepted.numel() * size).
 */
int64_t oracle_copy_accepted_kv(uint8_t* pool, int64_t layers, int64_t blocks, int64_t block_size,
                                int64_t row_bytes, const int64_t* src, const int64_t* dst, int64_t n,
                                uint8_t* staging) {
    const int64_t layer_bytes = blocks * block_size * row_bytes;
    for (int64_t kv = 0; kv < 2; ++kv) {
        for (int64_t l = 0; l < layers; ++l) {
            const uint8_t* base = pool + (kv * layers + l) * layer_bytes;
            for (int64_t i = 0; i < n; ++i) {
                const int64_t b = src[i] / block_size, o = src[i] % block_size;
                memcpy(staging + ((kv * layers + l) * n + i) * row_bytes, base + (b * block_size + o) * row_bytes,
                       (size_t)row_bytes);
            }
        }
    }
    for (int64_t kv = 0; kv < 2; ++kv) {
        for (int64_t l = 0; l < layers; ++l) {
            uint8_t* base = pool + (kv * layers + l) * layer_bytes;
            for (int64_t i = 0; i < n; ++i) {
                const int64_t b = dst[i] / block_size, o = dst[i] % block_size;
                memcpy(base + (b * block_size + o) * row_bytes, staging + ((kv * layers + l) * n + i) * row_bytes,
                       (size_t)row_bytes);
            }
        }
    }
    return 2 * layers * n * row_bytes;
}

/*
 * speculative/jetspec/paged_backend.py:116-213 - one (packed query, query head):
 *   request = query_to_request[q], local = query_local_row[q], P = prefix_lens[r],
 *   T = node_counts[r], seq = P + T, kv_head = head / groups;
 *   key position pos in [0, seq):
 *     pos <  P: slot = block_tables[r, pos // B] * B + pos % B          (:161-171)
 *     pos >= P: slot = tree_slots[cu[r] + pos - P]
 *   score = scale * q . k[slot] (+ qq_bias[bias_off[r] + local * T + pos - P] for tree keys)
 *   visible iff pos <= P + local; softmax over visible keys; out = sum p * v[slot].
 * Inputs are fp32 copies of the operands (bf16 converts exactly); arithmetic is
 * double.  Pools are dense [blocks][block_size][kv_heads][head_dim].
 * row_select (may be NULL) limits the work to rows with a nonzero entry.
 * Returns 0, or -1 if an address lies outside the pool (the row is then NaN).
 */
int oracle_tree_attention(const float* q, const float* k, const float* v, int64_t num_blocks, int32_t block_size,
                          int32_t q_heads, int32_t kv_heads, int32_t head_dim, const int32_t* cu_seqlens_q,
                          const int32_t* query_to_request, const int32_t* query_local_row,
                          const int32_t* prefix_lens, const int32_t* block_tables, int64_t table_stride,
                          const int64_t* tree_slots, const float* qq_bias, const int64_t* bias_offsets,
                          const int32_t* node_counts, int32_t total_queries, double scale,
                          const uint8_t* row_select, double* out) {
    const int32_t groups = q_heads / kv_heads;
    const int64_t slot_elems = (int64_t)kv_heads * head_dim;
    const int64_t pool_slots = num_blocks * block_size;
    int status = 0;
#pragma omp parallel for schedule(dynamic, 1) reduction(min : status)
    for (int32_t qi = 0; qi < total_queries; ++qi) {
        if (row_select && !row_select[qi]) continue;
        const int32_t r = query_to_request[qi];
        const int32_t local = query_local_row[qi];
        const int32_t prefix = prefix_lens[r];
        const int32_t nodes = node_counts[r];
        const int32_t seq = prefix + nodes;
        int64_t* slots = (int64_t*)malloc(sizeof(int64_t) * (size_t)(seq > 0 ? seq : 1));
        double* score = (double*)malloc(sizeof(double) * (size_t)(seq > 0 ? seq : 1));
        int bad = 0;
        for (int32_t pos = 0; pos < seq; ++pos) {
            int64_t slot;
            if (pos < prefix) {
                const int64_t page = block_tables[(int64_t)r * table_stride + pos / block_size];
                slot = page * block_size + pos % block_size;
            } else {
                slot = tree_slots[cu_seqlens_q[r] + (pos - prefix)];
            }
            if (slot < 0 || slot >= pool_slots) bad = 1;
            slots[pos] = slot;
        }
        for (int32_t h = 0; h < q_heads; ++h) {
            const int32_t kvh = h / groups;
            const float* qv = q + ((int64_t)qi * q_heads + h) * head_dim;
            double* o = out + ((int64_t)qi * q_heads + h) * head_dim;
            if (bad) {
                for (int32_t x = 0; x < head_dim; ++x) o[x] = NAN;
                continue;
            }
            double m = -INFINITY;
            for (int32_t pos = 0; pos < seq; ++pos) {
                if (pos > prefix + local) {
                    score[pos] = -INFINITY;
                    continue;
                }
                const float* kv = k + slots[pos] * slot_elems + (int64_t)kvh * head_dim;
                double dot = 0.0;
                for (int32_t x = 0; x < head_dim; ++x) dot += (double)qv[x] * (double)kv[x];
                double s = dot * scale;
                if (pos >= prefix) s += (double)qq_bias[bias_offsets[r] + (int64_t)local * nodes + (pos - prefix)];
                score[pos] = s;
                if (s > m) m = s;
            }
            double total = 0.0;
            for (int32_t x = 0; x < head_dim; ++x) o[x] = 0.0;
            for (int32_t pos = 0; pos < seq; ++pos) {
                if (score[pos] == -INFINITY) continue;
                const double p = exp(score[pos] - m);
                total += p;
                const float* vv = v + slots[pos] * slot_elems + (int64_t)kvh * head_dim;
                for (int32_t x = 0; x < head_dim; ++x) o[x] += p * (double)vv[x];
            }
            for (int32_t x = 0; x < head_dim; ++x) o[x] /= total;
        }
        if (bad && status > -1) status = -1;
        free(slots);
        free(score);
    }
    return status;
}
