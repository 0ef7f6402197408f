/*
 * oracle.c — CPU restatement of the swiftllm decode hot-path contract.
 *
 * TEST INFRASTRUCTURE ONLY. tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py load it as the checker and as the timed CPU
 * baseline. The product library never links, loads or calls it.
 *
 * Reference text followed (crates/swiftllm-cuda/kernels/paged_attention.cu,
 * "cu:" below); the reference kernel's output stage is a stub (cu:131-135),
 * so the attention itself is the textbook softmax(q.K^T * scale).V that the
 * kernel's comments and indexing describe:
 *   cu:50-52   one (sequence, query head); kv head = head / (H / Hkv)
 *   cu:57-58   context length, ceil(L / BS) blocks
 *   cu:67      query row q[s, h, :] (stride H * D)
 *   cu:80-87   physical block = block_tables[s * MB + j]; K tile address
 *   cu:92-96   logit = (sum_d q[d] * K[d * BS + t]) * scale
 *   cu:114-123 V tile address, V[d * BS + t]
 *   cu:131-135 output row out[s, h, :] (stride H * D)
 *   cu:167-199 reshape_and_cache: K[slot / BS, h, d, slot % BS] = key[t, h, d]
 * A context length <= 0 yields zeros (the reference divides 0 by 0 there).
 *
 * Which independent checks pin each function is listed in the test files
 * (tests/test_oracle_*.py).
 */
#include <immintrin.h>
#include <math.h>
#include <stddef.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

/* IEEE binary16 -> binary32, exact (F16C). */
static inline float h2f(uint16_t h) { return _cvtsh_ss(h); }

/* Element (b, h, d, t) of a cache laid out [NB, Hkv, D, BS] (cu:39-40). */
static inline size_t kv_index(int64_t b, int h, int d, int t, int Hkv, int D, int BS) {
    return (((size_t)b * (size_t)Hkv + (size_t)h) * (size_t)D + (size_t)d) * (size_t)BS + (size_t)t;
}

int oracle_max_threads(void) {
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}

void oracle_set_threads(int n) {
#ifdef _OPENMP
    if (n > 0) omp_set_num_threads(n);
#else
    (void)n;
#endif
}

/*
 * Textbook decode in double precision: two passes (max, then exp / sum /
 * weighted V) per (sequence, query head). out is double [S, H, D].
 */
void oracle_decode_f64(const uint16_t* q, const uint16_t* kc, const uint16_t* vc,
                       const int32_t* bt, const int32_t* ctx, double scale, int S, int H,
                       int Hkv, int D, int BS, int MB, double* out) {
    const int G = H / Hkv;
#pragma omp parallel
    {
        double* logit = NULL;
        size_t cap = 0;
        double* acc = (double*)malloc(sizeof(double) * (size_t)D);
#pragma omp for collapse(2) schedule(dynamic)
        for (int s = 0; s < S; ++s) {
            for (int h = 0; h < H; ++h) {
                const int kvh = h / G; /* cu:52 */
                int L = ctx[s] < 0 ? 0 : ctx[s];
                double* o = out + ((size_t)s * H + h) * D;
                if (L == 0) {
                    for (int d = 0; d < D; ++d) o[d] = 0.0;
                    continue;
                }
                if ((size_t)L > cap) {
                    free(logit);
                    cap = (size_t)L;
                    logit = (double*)malloc(sizeof(double) * cap);
                }
                const uint16_t* qv = q + ((size_t)s * H + h) * D; /* cu:67 */
                double m = -INFINITY;
                for (int j = 0; j < L; ++j) {
                    const int64_t b = bt[(size_t)s * MB + j / BS]; /* cu:80 */
                    const int t = j % BS;
                    double dot = 0.0;
                    for (int d = 0; d < D; ++d) {
                        dot += (double)h2f(qv[d]) * (double)h2f(kc[kv_index(b, kvh, d, t, Hkv, D, BS)]);
                    }
                    logit[j] = dot * scale; /* cu:96: scale after the dot */
                    if (logit[j] > m) m = logit[j];
                }
                double l = 0.0;
                for (int j = 0; j < L; ++j) {
                    logit[j] = exp(logit[j] - m);
                    l += logit[j];
                }
                for (int d = 0; d < D; ++d) acc[d] = 0.0;
                for (int j = 0; j < L; ++j) {
                    const int64_t b = bt[(size_t)s * MB + j / BS];
                    const int t = j % BS;
                    const double p = logit[j];
                    for (int d = 0; d < D; ++d) {
                        acc[d] += p * (double)h2f(vc[kv_index(b, kvh, d, t, Hkv, D, BS)]);
                    }
                }
                for (int d = 0; d < D; ++d) o[d] = acc[d] / l;
            }
        }
        free(logit);
        free(acc);
    }
}

/*
 * The same contract in fp32 arithmetic, organised for the CPU: one task per
 * (sequence, kv head) serving its G query heads, inner loops over the 16
 * tokens of a block (vectorised by the compiler). This is the timed CPU
 * baseline. out is float [S, H, D].
 */
void oracle_decode_f32(const uint16_t* q, const uint16_t* kc, const uint16_t* vc,
                       const int32_t* bt, const int32_t* ctx, float scale, int S, int H,
                       int Hkv, int D, int BS, int MB, float* out) {
    const int G = H / Hkv;
#pragma omp parallel
    {
        float* logit = NULL; /* [G][L] */
        size_t cap = 0;
        float* qf = (float*)malloc(sizeof(float) * (size_t)G * D);
        float* pv = (float*)malloc(sizeof(float) * (size_t)G * D * BS); /* [G][D][BS] */
        float* row = (float*)malloc(sizeof(float) * (size_t)BS);
        float* lsum = (float*)malloc(sizeof(float) * (size_t)G);
#pragma omp for collapse(2) schedule(dynamic)
        for (int s = 0; s < S; ++s) {
            for (int kvh = 0; kvh < Hkv; ++kvh) {
                const int L = ctx[s] < 0 ? 0 : ctx[s];
                const int h0 = kvh * G;
                if (L == 0) {
                    for (int g = 0; g < G; ++g) {
                        float* o = out + ((size_t)s * H + h0 + g) * D;
                        for (int d = 0; d < D; ++d) o[d] = 0.0f;
                    }
                    continue;
                }
                const int nblk = (L + BS - 1) / BS;
                const size_t need = (size_t)G * nblk * BS;
                if (need > cap) {
                    free(logit);
                    cap = need;
                    logit = (float*)malloc(sizeof(float) * cap);
                }
                const size_t lstride = (size_t)nblk * BS;
                for (int g = 0; g < G; ++g) {
                    const uint16_t* qv = q + ((size_t)s * H + h0 + g) * D;
                    for (int d = 0; d < D; ++d) qf[(size_t)g * D + d] = h2f(qv[d]);
                }
                memset(logit, 0, sizeof(float) * (size_t)G * lstride);
                for (int j = 0; j < nblk; ++j) {
                    const int64_t b = bt[(size_t)s * MB + j];
                    const uint16_t* tile = kc + kv_index(b, kvh, 0, 0, Hkv, D, BS);
                    for (int d = 0; d < D; ++d) {
                        for (int t = 0; t < BS; ++t) row[t] = h2f(tile[(size_t)d * BS + t]);
                        for (int g = 0; g < G; ++g) {
                            const float qd = qf[(size_t)g * D + d];
                            float* lg = logit + (size_t)g * lstride + (size_t)j * BS;
                            for (int t = 0; t < BS; ++t) lg[t] += qd * row[t];
                        }
                    }
                }
                for (int g = 0; g < G; ++g) {
                    float* lg = logit + (size_t)g * lstride;
                    float m = -INFINITY;
                    for (int j = 0; j < L; ++j) {
                        lg[j] *= scale;
                        if (lg[j] > m) m = lg[j];
                    }
                    float l = 0.0f;
                    for (int j = 0; j < L; ++j) {
                        lg[j] = expf(lg[j] - m);
                        l += lg[j];
                    }
                    for (size_t j = (size_t)L; j < lstride; ++j) lg[j] = 0.0f;
                    lsum[g] = l;
                }
                memset(pv, 0, sizeof(float) * (size_t)G * D * BS);
                for (int j = 0; j < nblk; ++j) {
                    const int64_t b = bt[(size_t)s * MB + j];
                    const uint16_t* tile = vc + kv_index(b, kvh, 0, 0, Hkv, D, BS);
                    const int nv = (L - j * BS) < BS ? (L - j * BS) : BS;
                    for (int d = 0; d < D; ++d) {
                        for (int t = 0; t < BS; ++t) row[t] = (t < nv) ? h2f(tile[(size_t)d * BS + t]) : 0.0f;
                        for (int g = 0; g < G; ++g) {
                            const float* p = logit + (size_t)g * lstride + (size_t)j * BS;
                            float* acc = pv + ((size_t)g * D + d) * BS;
                            for (int t = 0; t < BS; ++t) acc[t] += p[t] * row[t];
                        }
                    }
                }
                for (int g = 0; g < G; ++g) {
                    float* o = out + ((size_t)s * H + h0 + g) * D;
                    for (int d = 0; d < D; ++d) {
                        const float* acc = pv + ((size_t)g * D + d) * BS;
                        float sum = 0.0f;
                        for (int t = 0; t < BS; ++t) sum += acc[t];
                        o[d] = sum / lsum[g];
                    }
                }
            }
        }
        free(logit);
        free(qf);
        free(pv);
        free(row);
        free(lsum);
    }
}

/*
 * reshape_and_cache (cu:167-199): bit copies into the [NB, Hkv, D, BS]
 * caches. A negative slot is skipped (padding); the reference text would
 * write out of bounds there.
 */
void oracle_reshape_and_cache(const uint16_t* key, const uint16_t* value, uint16_t* kc,
                              uint16_t* vc, const int32_t* slot_mapping, int T, int Hkv, int D,
                              int BS) {
    for (int t = 0; t < T; ++t) {
        const int slot = slot_mapping[t];
        if (slot < 0) continue;
        const int b = slot / BS; /* cu:185 */
        const int o = slot % BS; /* cu:186 */
        for (int h = 0; h < Hkv; ++h) {
            for (int d = 0; d < D; ++d) {
                const size_t src = (size_t)t * Hkv * D + (size_t)h * D + d; /* cu:190, stride Hkv*D */
                kc[kv_index(b, h, d, o, Hkv, D, BS)] = key[src];
                vc[kv_index(b, h, d, o, Hkv, D, BS)] = value[src];
            }
        }
    }
}

/*
 * MoE routing and dispatch on one thread: the CPU baseline of the MoE row
 * (MoeMlp::forward steps 1-2, crates/swiftllm-models/src/layers/mlp.rs:
 * 240-246, whose reference body returns zeros) with the sampling
 * conventions of crates/swiftllm-core/src/sampling/mod.rs:366-385:
 *   - fp32 softmax with the row max subtracted (:380-385);
 *   - top-k by k argmax passes over the logits, ties to the lower expert
 *     index (the stable descending sort of :367-377), weights = the selected
 *     probabilities renormalised to sum 1;
 *   - a serial counting sort of the (t, k) entries by expert: histogram,
 *     exclusive prefix, then placement in (t asc, k asc) order, which is
 *     stable; x_perm[row] = x[t] (row copy), inverse[t, k] = row,
 *     sorted_token_ids[row] = t.
 * K <= 8 and E <= 256, as the device path accepts.
 */
void oracle_moe_route_dispatch_serial(const float* logits, const uint16_t* x, int T, int E, int K,
                                      int hidden, int32_t* ids, float* weights, int32_t* counts,
                                      int32_t* offsets, uint16_t* x_perm, int32_t* inverse,
                                      int32_t* sorted_token_ids) {
    for (int t = 0; t < T; ++t) {
        const float* row = logits + (size_t)t * E;
        float mx = row[0];
        for (int e = 1; e < E; ++e) mx = row[e] > mx ? row[e] : mx;
        float sum = 0.0f;
        for (int e = 0; e < E; ++e) sum += expf(row[e] - mx);
        unsigned char taken[256] = {0};
        float psel[8];
        float psum = 0.0f;
        for (int k = 0; k < K; ++k) {
            int best = -1;
            for (int e = 0; e < E; ++e) {
                if (!taken[e] && (best < 0 || row[e] > row[best])) best = e;
            }
            taken[best] = 1;
            ids[(size_t)t * K + k] = best;
            psel[k] = expf(row[best] - mx) / sum;
            psum += psel[k];
        }
        for (int k = 0; k < K; ++k) weights[(size_t)t * K + k] = psel[k] / psum;
    }
    for (int e = 0; e < E; ++e) counts[e] = 0;
    for (size_t i = 0; i < (size_t)T * K; ++i) counts[ids[i]] += 1;
    offsets[0] = 0;
    for (int e = 0; e < E; ++e) offsets[e + 1] = offsets[e] + counts[e];
    int32_t fill[256];
    for (int e = 0; e < E; ++e) fill[e] = offsets[e];
    for (int t = 0; t < T; ++t) {
        for (int k = 0; k < K; ++k) {
            const int e = ids[(size_t)t * K + k];
            const int r = fill[e]++;
            inverse[(size_t)t * K + k] = r;
            sorted_token_ids[r] = t;
            memcpy(x_perm + (size_t)r * hidden, x + (size_t)t * hidden, sizeof(uint16_t) * hidden);
        }
    }
}
