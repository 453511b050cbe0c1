/*
 * fgqa_oracle.c -- CPU restatement of the reference's flash-GQA attention.
 *
 * TEST INFRASTRUCTURE: a parity checker and the timed CPU baseline, never the
 * product.  Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline
 * leg may load it.  Built with -ffp-contract=off so that every a*b+c rounds
 * twice, as the reference's host compiler does on baseline x86-64, and the
 * results do not depend on the host CPU.
 */
#include "fgqa_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

#ifdef _OPENMP
#include <omp.h>
#endif

#define ORACLE_MAX_D 512

uint16_t fgqa_oracle_f32_to_bf16(float x) {
    uint32_t u;
    memcpy(&u, &x, sizeof(u));
    if ((u & 0x7fffffffu) > 0x7f800000u) {
        /* NaN: keep sign and payload top bits, force quiet. */
        return (uint16_t)((u >> 16) | 0x0040u);
    }
    /* Round to nearest, ties to even, on the 16 discarded bits. */
    u += 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

float fgqa_oracle_bf16_to_f32(uint16_t h) {
    uint32_t u = (uint32_t)h << 16;
    float f;
    memcpy(&f, &u, sizeof(f));
    return f;
}

void fgqa_oracle_f32_to_bf16_array(const float* src, uint16_t* dst, size_t n) {
    for (size_t i = 0; i < n; ++i) dst[i] = fgqa_oracle_f32_to_bf16(src[i]);
}

void fgqa_oracle_bf16_to_f32_array(const uint16_t* src, float* dst, size_t n) {
    for (size_t i = 0; i < n; ++i) dst[i] = fgqa_oracle_bf16_to_f32(src[i]);
}

static inline float bf(uint16_t h) { return fgqa_oracle_bf16_to_f32(h); }

static void set_threads(int nthreads) {
#ifdef _OPENMP
    if (nthreads > 0) omp_set_num_threads(nthreads);
#else
    (void)nthreads;
#endif
}

/*
 * Decode.  Per (batch, query head) the loop below follows
 * examples/cplusplus/test_decode_flash_gqa.cu:186-252 step by step:
 *   :193-201  qk = sum_d q[d]*k[t][d]            (fp32, d ascending)
 *   :202-208  m_new = max(m, qk*scale)
 *   :209-215  l_tile = sum_t expf(qk*scale - m_new)
 *   :216-223  P = bf16(expf(qk*scale - m_new))   (p_bf16 = 1; with p_bf16 = 0
 *             P stays fp32, which is the torch tiled decode reference
 *             examples/python/Triton/test_decode_flash_gqa_kernel.py:56-73)
 *   :225-233  o_tile[d] = sum_t P*V[t][d]         (fp32, t ascending)
 *   :234-241  O = (first tile) ? o_tile : O*expf(m - m_new) + o_tile
 *   :243-244  l = l*expf(m - m_new) + l_tile; m = m_new
 *   :247-251  out = bf16(O / l)
 * The reference parallelises over batch only (:185); here (batch, head) pairs
 * are independent work items, which changes no arithmetic.
 */
int fgqa_oracle_decode_bf16(const uint16_t* q, const uint16_t* k, const uint16_t* v,
                            float scale, uint16_t* o, float* lse,
                            int batch, int s_max, int hq, int hkv, int d,
                            const int32_t* seqlens, int tile, int p_bf16, int nthreads) {
    if (!q || !k || !v || !o) return -1;
    if (batch < 0 || s_max < 0 || hq <= 0 || hkv <= 0 || d <= 0 || d > ORACLE_MAX_D) return -1;
    if (hq % hkv != 0 || tile <= 0) return -1;
    if (seqlens) {
        for (int b = 0; b < batch; ++b)
            if (seqlens[b] < 0 || seqlens[b] > s_max) return -1;
    }
    const int group = hq / hkv;
    set_threads(nthreads);

#pragma omp parallel
    {
        float* s = (float*)malloc(sizeof(float) * (size_t)tile);
        float* p = (float*)malloc(sizeof(float) * (size_t)tile);
        float acc[ORACLE_MAX_D];
        float otile[ORACLE_MAX_D];
#pragma omp for collapse(2) schedule(dynamic)
        for (int b = 0; b < batch; ++b) {
            for (int h = 0; h < hq; ++h) {
                const int len = seqlens ? seqlens[b] : s_max;
                const int kvh = h / group;
                const uint16_t* qrow = q + ((size_t)b * hq + h) * d;
                float m = -INFINITY;
                float l = 0.f;
                for (int x = 0; x < d; ++x) acc[x] = 0.f;
                for (int t0 = 0; t0 < len; t0 += tile) {
                    const int n = (len - t0 < tile) ? (len - t0) : tile;
                    for (int j = 0; j < n; ++j) {
                        const uint16_t* krow = k + (((size_t)b * s_max + (t0 + j)) * hkv + kvh) * d;
                        float qk = 0.f;
                        for (int x = 0; x < d; ++x) qk += bf(qrow[x]) * bf(krow[x]);
                        s[j] = qk;
                    }
                    float m_new = m;
                    for (int j = 0; j < n; ++j) m_new = fmaxf(m_new, s[j] * scale);
                    float l_tile = 0.f;
                    for (int j = 0; j < n; ++j) l_tile += expf(s[j] * scale - m_new);
                    for (int j = 0; j < n; ++j) {
                        const float e = expf(s[j] * scale - m_new);
                        p[j] = p_bf16 ? bf(fgqa_oracle_f32_to_bf16(e)) : e;
                    }
                    /* o_tile[x] accumulates over t ascending for each x (same order as
                     * the reference's inner token loop). */
                    for (int x = 0; x < d; ++x) otile[x] = 0.f;
                    for (int j = 0; j < n; ++j) {
                        const uint16_t* vrow = v + (((size_t)b * s_max + (t0 + j)) * hkv + kvh) * d;
                        const float pj = p[j];
                        for (int x = 0; x < d; ++x) otile[x] += pj * bf(vrow[x]);
                    }
                    const float corr = expf(m - m_new);
                    if (t0 == 0) {
                        for (int x = 0; x < d; ++x) acc[x] = otile[x];
                    } else {
                        for (int x = 0; x < d; ++x) acc[x] = acc[x] * corr + otile[x];
                    }
                    l = l * corr + l_tile;
                    m = m_new;
                }
                uint16_t* orow = o + ((size_t)b * hq + h) * d;
                if (len == 0) {
                    for (int x = 0; x < d; ++x) orow[x] = 0;
                    if (lse) lse[(size_t)b * hq + h] = -INFINITY;
                } else {
                    for (int x = 0; x < d; ++x) orow[x] = fgqa_oracle_f32_to_bf16(acc[x] / l);
                    if (lse) lse[(size_t)b * hq + h] = m + logf(l);
                }
            }
        }
        free(s);
        free(p);
    }
    return 0;
}

/*
 * Prefill.  Per (batch, query head, query row) this follows the torch
 * reference examples/python/Triton/test_flash_gqa_kernel.py:60-90:
 *   :81     scores = (q . k) * scale                 (fp32)
 *   :69-82  causal: scores[j] = -inf for j > i        (triu(diagonal=1))
 *   :83-86  row_max; e = exp(scores - row_max); probs = e / sum(e);
 *           lse = log(sum(e)) + row_max
 *   :88     out = probs . v (fp32), then cast to bf16 (:93)
 */
int fgqa_oracle_prefill_bf16(const uint16_t* q, const uint16_t* k, const uint16_t* v,
                             float scale, uint16_t* o, float* lse,
                             int batch, int sq, int skv, int hq, int hkv, int d,
                             const int64_t* qs, const int64_t* ks,
                             const int64_t* vs, const int64_t* os,
                             int causal, int q_offset, int nthreads) {
    if (!q || !k || !v || !o || !qs || !ks || !vs || !os) return -1;
    if (batch < 0 || sq < 0 || skv < 0 || hq <= 0 || hkv <= 0 || d <= 0 || d > ORACLE_MAX_D) return -1;
    if (hq % hkv != 0) return -1;
    const int group = hq / hkv;
    set_threads(nthreads);

#pragma omp parallel
    {
        float* sc = (float*)malloc(sizeof(float) * (size_t)(skv > 0 ? skv : 1));
        float out[ORACLE_MAX_D];
#pragma omp for collapse(3) schedule(dynamic, 4)
        for (int b = 0; b < batch; ++b) {
            for (int h = 0; h < hq; ++h) {
                for (int i = 0; i < sq; ++i) {
                    const int kvh = h / group;
                    const uint16_t* qrow = q + b * qs[0] + (int64_t)i * qs[1] + h * qs[2];
                    uint16_t* orow = o + b * os[0] + (int64_t)i * os[1] + h * os[2];
                    int nvis = skv;
                    if (causal) {
                        const long lim = (long)i + q_offset + 1;
                        if (lim < nvis) nvis = lim < 0 ? 0 : (int)lim;
                    }
                    float rmax = -INFINITY;
                    for (int j = 0; j < nvis; ++j) {
                        const uint16_t* krow = k + b * ks[0] + (int64_t)j * ks[1] + kvh * ks[2];
                        float acc = 0.f;
                        for (int x = 0; x < d; ++x) acc += bf(qrow[x]) * bf(krow[x]);
                        sc[j] = acc * scale;
                        rmax = fmaxf(rmax, sc[j]);
                    }
                    if (nvis == 0) {
                        for (int x = 0; x < d; ++x) orow[x] = 0;
                        if (lse) lse[((size_t)b * hq + h) * sq + i] = -INFINITY;
                        continue;
                    }
                    float sum = 0.f;
                    for (int j = 0; j < nvis; ++j) {
                        sc[j] = expf(sc[j] - rmax);
                        sum += sc[j];
                    }
                    for (int x = 0; x < d; ++x) out[x] = 0.f;
                    for (int j = 0; j < nvis; ++j) {
                        const uint16_t* vrow = v + b * vs[0] + (int64_t)j * vs[1] + kvh * vs[2];
                        const float pj = sc[j] / sum;
                        for (int x = 0; x < d; ++x) out[x] += pj * bf(vrow[x]);
                    }
                    for (int x = 0; x < d; ++x) orow[x] = fgqa_oracle_f32_to_bf16(out[x]);
                    if (lse) lse[((size_t)b * hq + h) * sq + i] = logf(sum) + rmax;
                }
            }
        }
        free(sc);
    }
    return 0;
}

/* Softmax attention in double: the exact answer both fp32 paths approximate. */
int fgqa_oracle_attention_f64(const uint16_t* q, const uint16_t* k, const uint16_t* v,
                              double scale, double* o, double* lse,
                              int batch, int sq, int skv, int hq, int hkv, int d,
                              const int64_t* qs, const int64_t* ks,
                              const int64_t* vs, const int32_t* seqlens,
                              int causal, int causal_offset, int nthreads) {
    if (!q || !k || !v || !o || !qs || !ks || !vs) return -1;
    if (batch < 0 || sq < 0 || skv < 0 || hq <= 0 || hkv <= 0 || d <= 0) return -1;
    if (hq % hkv != 0) return -1;
    const int group = hq / hkv;
    set_threads(nthreads);

#pragma omp parallel
    {
        double* sc = (double*)malloc(sizeof(double) * (size_t)(skv > 0 ? skv : 1));
#pragma omp for collapse(3) schedule(dynamic, 4)
        for (int b = 0; b < batch; ++b) {
            for (int h = 0; h < hq; ++h) {
                for (int i = 0; i < sq; ++i) {
                    const int kvh = h / group;
                    int len = seqlens ? seqlens[b] : skv;
                    if (len > skv) len = skv;
                    int nvis = len;
                    if (causal) {
                        const long lim = (long)i + causal_offset + 1;
                        if (lim < nvis) nvis = lim < 0 ? 0 : (int)lim;
                    }
                    const uint16_t* qrow = q + b * qs[0] + (int64_t)i * qs[1] + h * qs[2];
                    double* orow = o + (((size_t)b * sq + i) * hq + h) * d;
                    double rmax = -INFINITY;
                    for (int j = 0; j < nvis; ++j) {
                        const uint16_t* krow = k + b * ks[0] + (int64_t)j * ks[1] + kvh * ks[2];
                        double acc = 0.0;
                        for (int x = 0; x < d; ++x) acc += (double)bf(qrow[x]) * (double)bf(krow[x]);
                        sc[j] = acc * scale;
                        if (sc[j] > rmax) rmax = sc[j];
                    }
                    for (int x = 0; x < d; ++x) orow[x] = 0.0;
                    if (nvis == 0) {
                        if (lse) lse[((size_t)b * hq + h) * sq + i] = -INFINITY;
                        continue;
                    }
                    double sum = 0.0;
                    for (int j = 0; j < nvis; ++j) {
                        sc[j] = exp(sc[j] - rmax);
                        sum += sc[j];
                    }
                    for (int j = 0; j < nvis; ++j) {
                        const uint16_t* vrow = v + b * vs[0] + (int64_t)j * vs[1] + kvh * vs[2];
                        const double pj = sc[j] / sum;
                        for (int x = 0; x < d; ++x) orow[x] += pj * (double)bf(vrow[x]);
                    }
                    if (lse) lse[((size_t)b * hq + h) * sq + i] = log(sum) + rmax;
                }
            }
        }
        free(sc);
    }
    return 0;
}
