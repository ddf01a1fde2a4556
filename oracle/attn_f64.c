/* Float64 brute-force restatement of the attention hot path -- test infrastructure.
 *
 * This file is the independent check of the numpy oracle (attention.py): a
 * different language, explicit loops, double precision, natural-base exp, and
 * page gathering by direct index arithmetic instead of fancy indexing.  It is
 * built into oracle/_build/libattn_f64.so and loaded by tests only.
 *
 * attention:     sonhoang/flash-attention-from-scratch attnkernels/reference.py:9-18
 *                (softmax(scale*QK^T + causal mask j > i) V)
 * paged decode:  attnkernels/reference.py:54-70 with the gather of
 *                paged_decode.cu:95-96 (token t of sequence b lives in page
 *                block_tables[b][t / bs] at offset t % bs; query head h reads
 *                kv head h / G).
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>

/* q, k, v: float32 [bh, n, d] contiguous; out: float64 [bh, n, d]. */
int oracle_attention_f64(const float *q, const float *k, const float *v, double *out,
                         int64_t bh, int64_t n, int64_t d, int causal, double scale) {
    double *s = (double *)malloc((size_t)(n > 0 ? n : 1) * sizeof(double));
    if (!s) return -1;
    for (int64_t b = 0; b < bh; ++b) {
        const float *qb = q + b * n * d, *kb = k + b * n * d, *vb = v + b * n * d;
        double *ob = out + b * n * d;
        for (int64_t i = 0; i < n; ++i) {
            const int64_t jend = causal ? i + 1 : n;
            double mx = -INFINITY;
            for (int64_t j = 0; j < jend; ++j) {
                double dot = 0.0;
                for (int64_t c = 0; c < d; ++c) dot += (double)qb[i * d + c] * (double)kb[j * d + c];
                s[j] = dot * scale;
                if (s[j] > mx) mx = s[j];
            }
            double den = 0.0;
            for (int64_t j = 0; j < jend; ++j) {
                s[j] = exp(s[j] - mx);
                den += s[j];
            }
            for (int64_t c = 0; c < d; ++c) {
                double acc = 0.0;
                for (int64_t j = 0; j < jend; ++j) acc += s[j] * (double)vb[j * d + c];
                ob[i * d + c] = acc / den;
            }
        }
    }
    free(s);
    return 0;
}

/* q: float32 [B, hq, d]; k_cache, v_cache: float32 [num_blocks, hkv, bs, d];
 * block_tables: int32 [B, max_blocks]; context_lens: int32 [B];
 * out: float64 [B, hq, d].  Returns -1 on an out-of-range page id or length. */
int oracle_paged_decode_f64(const float *q, const float *k_cache, const float *v_cache,
                            const int32_t *block_tables, const int32_t *context_lens,
                            double *out, int64_t B, int64_t hq, int64_t hkv, int64_t d,
                            int64_t num_blocks, int64_t bs, int64_t max_blocks, double scale) {
    const int64_t G = hq / hkv;
    int64_t max_ctx = 0;
    for (int64_t b = 0; b < B; ++b)
        if (context_lens[b] > max_ctx) max_ctx = context_lens[b];
    double *s = (double *)malloc((size_t)(max_ctx > 0 ? max_ctx : 1) * sizeof(double));
    if (!s) return -1;
    int rc = 0;
    for (int64_t b = 0; b < B && rc == 0; ++b) {
        const int64_t ctx = context_lens[b];
        if (ctx < 1 || ctx > max_blocks * bs) { rc = -1; break; }
        for (int64_t h = 0; h < hq && rc == 0; ++h) {
            const int64_t kvh = h / G;
            const float *qh = q + (b * hq + h) * d;
            double mx = -INFINITY;
            for (int64_t t = 0; t < ctx; ++t) {
                const int64_t page = block_tables[b * max_blocks + t / bs];
                if (page < 0 || page >= num_blocks) { rc = -1; break; }
                const float *kr = k_cache + ((page * hkv + kvh) * bs + t % bs) * d;
                double dot = 0.0;
                for (int64_t c = 0; c < d; ++c) dot += (double)qh[c] * (double)kr[c];
                s[t] = dot * scale;
                if (s[t] > mx) mx = s[t];
            }
            if (rc) break;
            double den = 0.0;
            for (int64_t t = 0; t < ctx; ++t) {
                s[t] = exp(s[t] - mx);
                den += s[t];
            }
            double *oh = out + (b * hq + h) * d;
            for (int64_t c = 0; c < d; ++c) oh[c] = 0.0;
            for (int64_t t = 0; t < ctx; ++t) {
                const int64_t page = block_tables[b * max_blocks + t / bs];
                const float *vr = v_cache + ((page * hkv + kvh) * bs + t % bs) * d;
                for (int64_t c = 0; c < d; ++c) oh[c] += s[t] * (double)vr[c];
            }
            for (int64_t c = 0; c < d; ++c) oh[c] /= den;
        }
    }
    free(s);
    return rc;
}
