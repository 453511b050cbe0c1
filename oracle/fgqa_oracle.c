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

float fgqa_oracle_fp8e4m3_to_f32(uint8_t c) {
    const int sgn = (c >> 7) & 1, e = (c >> 3) & 15, m = c & 7;
    if (e == 15 && m == 7) return NAN;
    const float v = (e == 0) ? ldexpf((float)m, -9) : ldexpf(1.0f + (float)m / 8.0f, e - 7);
    return sgn ? -v : v;
}

/* Row `t` of sequence b, kv head kvh, decoded to float. */
static void paged_row(const void* cache, int kv_fp8, const int32_t* bt, int64_t bt_stride, int page_size,
                      const int64_t* st, int b, int t, int kvh, int d, float* out) {
    const int64_t page = bt[(int64_t)b * bt_stride + t / page_size];
    const int64_t off = page * st[0] + (int64_t)(t % page_size) * st[1] + (int64_t)kvh * st[2];
    if (kv_fp8) {
        const uint8_t* r = (const uint8_t*)cache + off;
        for (int x = 0; x < d; ++x) out[x] = fgqa_oracle_fp8e4m3_to_f32(r[x]);
    } else {
        const uint16_t* r = (const uint16_t*)cache + off;
        for (int x = 0; x < d; ++x) out[x] = bf(r[x]);
    }
}

int fgqa_oracle_decode_paged(const uint16_t* q, const void* k_cache, const void* v_cache, int kv_fp8,
                             const int32_t* block_table, int64_t bt_stride, int page_size,
                             const int64_t* ks, const int64_t* vs,
                             float scale, float k_scale, float v_scale, uint16_t* o, float* lse,
                             int batch, int hq, int hkv, int d, const int32_t* seqlens, int tile,
                             int nthreads) {
    if (!q || !k_cache || !v_cache || !block_table || !ks || !vs || !o || !seqlens) return -1;
    if (batch < 0 || hq <= 0 || hkv <= 0 || d <= 0 || d > ORACLE_MAX_D || page_size <= 0) return -1;
    if (hq % hkv != 0 || tile <= 0) return -1;
    for (int b = 0; b < batch; ++b)
        if (seqlens[b] < 0 || (int64_t)seqlens[b] > bt_stride * page_size) return -1;
    const int group = hq / hkv;
    const float sc = scale * k_scale;
    set_threads(nthreads);

#pragma omp parallel
    {
        float* s = (float*)malloc(sizeof(float) * (size_t)tile);
        float* p = (float*)malloc(sizeof(float) * (size_t)tile);
        float acc[ORACLE_MAX_D];
        float otile[ORACLE_MAX_D];
        float row[ORACLE_MAX_D];
#pragma omp for collapse(2) schedule(dynamic)
        for (int b = 0; b < batch; ++b) {
            for (int h = 0; h < hq; ++h) {
                const int len = seqlens[b];
                const int kvh = h / group;
                const uint16_t* qrow = q + ((size_t)b * hq + h) * d;
                float m = -INFINITY;
                float l = 0.f;
                for (int x = 0; x < d; ++x) acc[x] = 0.f;
                for (int t0 = 0; t0 < len; t0 += tile) {
                    const int n = (len - t0 < tile) ? (len - t0) : tile;
                    for (int j = 0; j < n; ++j) {
                        paged_row(k_cache, kv_fp8, block_table, bt_stride, page_size, ks, b, t0 + j, kvh, d, row);
                        float qk = 0.f;
                        for (int x = 0; x < d; ++x) qk += bf(qrow[x]) * row[x];
                        s[j] = qk;
                    }
                    float m_new = m;
                    for (int j = 0; j < n; ++j) m_new = fmaxf(m_new, s[j] * sc);
                    float l_tile = 0.f;
                    for (int j = 0; j < n; ++j) l_tile += expf(s[j] * sc - m_new);
                    for (int j = 0; j < n; ++j) p[j] = bf(fgqa_oracle_f32_to_bf16(expf(s[j] * sc - m_new)));
                    for (int x = 0; x < d; ++x) otile[x] = 0.f;
                    for (int j = 0; j < n; ++j) {
                        paged_row(v_cache, kv_fp8, block_table, bt_stride, page_size, vs, b, t0 + j, kvh, d, row);
                        const float pj = p[j];
                        for (int x = 0; x < d; ++x) otile[x] += pj * row[x];
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
                    for (int x = 0; x < d; ++x) orow[x] = fgqa_oracle_f32_to_bf16((acc[x] / l) * v_scale);
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
static int prefill_core(const uint16_t* q, const uint16_t* k, const uint16_t* v,
                        float scale, uint16_t* o, float* lse,
                        int batch, int sq, int skv, int hq, int hkv, int d, int dv,
                        const int64_t* qs, const int64_t* ks,
                        const int64_t* vs, const int64_t* os,
                        int causal, int q_offset, int nthreads) {
    if (!q || !k || !v || !o || !qs || !ks || !vs || !os) return -1;
    if (batch < 0 || sq < 0 || skv < 0 || hq <= 0 || hkv <= 0 || d <= 0 || d > ORACLE_MAX_D) return -1;
    if (dv <= 0 || dv > ORACLE_MAX_D) return -1;
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
                        for (int x = 0; x < dv; ++x) orow[x] = 0;
                        if (lse) lse[((size_t)b * hq + h) * sq + i] = -INFINITY;
                        continue;
                    }
                    float sum = 0.f;
                    for (int j = 0; j < nvis; ++j) {
                        sc[j] = expf(sc[j] - rmax);
                        sum += sc[j];
                    }
                    for (int x = 0; x < dv; ++x) out[x] = 0.f;
                    for (int j = 0; j < nvis; ++j) {
                        const uint16_t* vrow = v + b * vs[0] + (int64_t)j * vs[1] + kvh * vs[2];
                        const float pj = sc[j] / sum;
                        for (int x = 0; x < dv; ++x) out[x] += pj * bf(vrow[x]);
                    }
                    for (int x = 0; x < dv; ++x) orow[x] = fgqa_oracle_f32_to_bf16(out[x]);
                    if (lse) lse[((size_t)b * hq + h) * sq + i] = logf(sum) + rmax;
                }
            }
        }
        free(sc);
    }
    return 0;
}

int fgqa_oracle_prefill_bf16(const uint16_t* q, const uint16_t* k, const uint16_t* v,
                             float scale, uint16_t* o, float* lse,
                             int batch, int sq, int skv, int hq, int hkv, int d,
                             const int64_t* qs, const int64_t* ks,
                             const int64_t* vs, const int64_t* os,
                             int causal, int q_offset, int nthreads) {
    return prefill_core(q, k, v, scale, o, lse, batch, sq, skv, hq, hkv, d, d, qs, ks, vs, os,
                        causal, q_offset, nthreads);
}

/*
 * MLA prefill: the same loop with separate Q/K and V/O head dims.  It restates
 * examples/python/Triton/test_flash_mla_kernel.py:27-95 (fp32 scores over
 * head_dim_qk, triu(diagonal=1) causal mask at :69-72, full softmax and
 * lse at :82-86, fp32 probs . v over head_dim_v at :88, cast to bf16 at :93).
 */
int fgqa_oracle_prefill_mla_bf16(const uint16_t* q, const uint16_t* k, const uint16_t* v,
                                 float scale, uint16_t* o, float* lse,
                                 int batch, int sq, int skv, int hq, int hkv, int dqk, int dv,
                                 const int64_t* qs, const int64_t* ks,
                                 const int64_t* vs, const int64_t* os,
                                 int causal, int q_offset, int nthreads) {
    return prefill_core(q, k, v, scale, o, lse, batch, sq, skv, hq, hkv, dqk, dv, qs, ks, vs, os,
                        causal, q_offset, nthreads);
}

/* Sliding-window + sink prefill (see the header for the reference lines). */
int fgqa_oracle_prefill_swa_bf16(const uint16_t* q, const uint16_t* k, const uint16_t* v,
                                 float scale, uint16_t* o, float* lse,
                                 int batch, int sq, int skv, int hq, int hkv, int d,
                                 const int64_t* qs, const int64_t* ks,
                                 const int64_t* vs, const int64_t* os,
                                 int window, const float* sink, int q_offset, int nthreads) {
    if (!q || !k || !v || !o || !qs || !ks || !vs || !os) return -1;
    if (batch < 0 || sq < 0 || skv < 0 || hq <= 0 || hkv <= 0 || d <= 0 || d > ORACLE_MAX_D) return -1;
    if (hq % hkv != 0 || window <= 0) return -1;
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
                    const long pos = (long)i + q_offset;        /* keys j <= pos, j > pos - window */
                    const int j1 = (pos + 1 < skv) ? (int)(pos + 1) : skv;
                    const int j0 = (pos - window + 1 > 0) ? (int)(pos - window + 1) : 0;
                    const float sk = sink ? sink[h] : 0.f;
                    if (j0 >= j1) {
                        for (int x = 0; x < d; ++x) orow[x] = 0;
                        if (lse) lse[((size_t)b * hq + h) * sq + i] = sink ? logf(fmaxf(sk, 1.0e-9f)) : -INFINITY;
                        continue;
                    }
                    float rmax = -INFINITY;
                    for (int j = j0; j < j1; ++j) {
                        const uint16_t* krow = k + b * ks[0] + (int64_t)j * ks[1] + kvh * ks[2];
                        float acc = 0.f;
                        for (int x = 0; x < d; ++x) acc += bf(qrow[x]) * bf(krow[x]);
                        sc[j] = acc * scale;
                        rmax = fmaxf(rmax, sc[j]);
                    }
                    float sum = 0.f;
                    for (int j = j0; j < j1; ++j) {
                        sc[j] = expf(sc[j] - rmax);
                        sum += sc[j];
                    }
                    if (sink) sum = sum + sk * expf(-rmax);
                    for (int x = 0; x < d; ++x) out[x] = 0.f;
                    for (int j = j0; j < j1; ++j) {
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

/*
 * Prefill backward (reference src/python/Triton/flash_gqa_backward_kernel.py).
 * p and dS of a (row, key) pair are recomputed by bwd_pair() with the same
 * operation order wherever they are needed, so the dQ pass (parallel over
 * rows) and the dK/dV pass (parallel over keys) see identical values.
 */
typedef struct {
    const uint16_t *q, *k, *v, *grad_o;
    const float *lse, *delta;
    const int64_t *qs, *ks, *vs, *dos;
    float scale;
    int sq, hq, d, dv, group;   /* d: Q/K row length, dv: V/O row length */
} bwd_ctx;

/* :253-285 for query row i of head h and key j of batch b: returns p (fp32)
 * and stores dS (rounded to bf16, as a float) in *ds. */
static float bwd_pair(const bwd_ctx* c, int b, int h, int i, int j, float* ds) {
    const int kvh = h / c->group;
    const uint16_t* qrow = c->q + b * c->qs[0] + (int64_t)i * c->qs[1] + h * c->qs[2];
    const uint16_t* krow = c->k + b * c->ks[0] + (int64_t)j * c->ks[1] + kvh * c->ks[2];
    const uint16_t* vrow = c->v + b * c->vs[0] + (int64_t)j * c->vs[1] + kvh * c->vs[2];
    const uint16_t* dorow = c->grad_o + b * c->dos[0] + (int64_t)i * c->dos[1] + h * c->dos[2];
    float s = 0.f, dp = 0.f;
    for (int x = 0; x < c->d; ++x) s += bf(qrow[x]) * bf(krow[x]);
    for (int x = 0; x < c->dv; ++x) dp += bf(dorow[x]) * bf(vrow[x]);
    const size_t r = ((size_t)b * c->hq + h) * c->sq + i;
    const float p = expf(s * c->scale - c->lse[r]);
    *ds = bf(fgqa_oracle_f32_to_bf16(p * (dp - c->delta[r]) * c->scale));
    return p;
}

/* d: Q/K row length; dvd: V/O/dO row length (the MLA backward has d = 192,
 * dvd = 128; the GQA backward d = dvd).  dq, dk have d-element rows, dv
 * dvd-element rows. */
static int backward_core(const uint16_t* q, const uint16_t* k, const uint16_t* v,
                         const uint16_t* o, const float* lse, const uint16_t* grad_o,
                         float scale, float* dq, float* dk, float* dv,
                         int batch, int sq, int skv, int hq, int hkv, int d, int dvd,
                         const int64_t* qs, const int64_t* ks,
                         const int64_t* vs, const int64_t* os,
                         const int64_t* dos, int causal, int window,
                         const int* rows, const int* keys, int nthreads) {
    if (!q || !k || !v || !o || !lse || !grad_o || !qs || !ks || !vs || !os || !dos) return -1;
    if (batch < 0 || sq < 0 || skv < 0 || hq <= 0 || hkv <= 0 || d <= 0 || d > ORACLE_MAX_D) return -1;
    if (dvd <= 0 || dvd > ORACLE_MAX_D) return -1;
    if (hq % hkv != 0 || window < 0 || (window > 0 && !causal)) return -1;
    const int group = hq / hkv;
    const int r0 = rows ? rows[0] : 0, r1 = rows ? rows[1] : sq;
    const int k0 = keys ? keys[0] : 0, k1 = keys ? keys[1] : skv;
    if (r0 < 0 || r1 > sq || k0 < 0 || k1 > skv) return -1;
    set_threads(nthreads);

    /* :16-50 delta for every row (the dK/dV pass needs all of them) */
    const size_t nrows = (size_t)batch * hq * sq;
    float* delta = (float*)malloc(sizeof(float) * (nrows > 0 ? nrows : 1));
    if (!delta) return -1;
#pragma omp parallel for collapse(3) schedule(static)
    for (int b = 0; b < batch; ++b)
        for (int h = 0; h < hq; ++h)
            for (int i = 0; i < sq; ++i) {
                const uint16_t* orow = o + b * os[0] + (int64_t)i * os[1] + h * os[2];
                const uint16_t* dorow = grad_o + b * dos[0] + (int64_t)i * dos[1] + h * dos[2];
                float acc = 0.f;
                for (int x = 0; x < dvd; ++x) acc += bf(orow[x]) * bf(dorow[x]);
                delta[((size_t)b * hq + h) * sq + i] = acc;
            }

    bwd_ctx c = {q, k, v, grad_o, lse, delta, qs, ks, vs, dos, scale, sq, hq, d, dvd, group};

    /* :292-293 dQ_i = sum_j dS_ij k_j over the keys row i sees */
    if (dq) {
#pragma omp parallel for collapse(3) schedule(dynamic, 4)
        for (int b = 0; b < batch; ++b)
            for (int h = 0; h < hq; ++h)
                for (int i = r0; i < r1; ++i) {
                    const int kvh = h / group;
                    float acc[ORACLE_MAX_D];
                    for (int x = 0; x < d; ++x) acc[x] = 0.f;
                    const int jend = causal ? (i + 1 < skv ? i + 1 : skv) : skv;
                    const int jbeg = (window > 0 && i - window + 1 > 0) ? i - window + 1 : 0;
                    for (int j = jbeg; j < jend; ++j) {
                        float ds;
                        (void)bwd_pair(&c, b, h, i, j, &ds);
                        const uint16_t* krow = k + b * ks[0] + (int64_t)j * ks[1] + kvh * ks[2];
                        for (int x = 0; x < d; ++x) acc[x] += ds * bf(krow[x]);
                    }
                    float* out = dq + (((size_t)b * sq + i) * hq + h) * d;
                    for (int x = 0; x < d; ++x) out[x] = acc[x];
                }
    }

    /* :271-272, :287 dV_j = sum p_bf16 dO_i, dK_j = sum dS_ij q_i over the
     * G heads of kv head kvh and the rows that see key j */
    if (dk || dv) {
#pragma omp parallel for collapse(3) schedule(dynamic, 4)
        for (int b = 0; b < batch; ++b)
            for (int kvh = 0; kvh < hkv; ++kvh)
                for (int j = k0; j < k1; ++j) {
                    float ak[ORACLE_MAX_D], av[ORACLE_MAX_D];
                    for (int x = 0; x < d; ++x) ak[x] = 0.f;
                    for (int x = 0; x < dvd; ++x) av[x] = 0.f;
                    const int ibeg = causal ? j : 0;
                    const int iend = (window > 0 && j + window < sq) ? j + window : sq;
                    for (int h = kvh * group; h < (kvh + 1) * group; ++h)
                        for (int i = ibeg; i < iend; ++i) {
                            float ds;
                            const float pb = bf(fgqa_oracle_f32_to_bf16(bwd_pair(&c, b, h, i, j, &ds)));
                            const uint16_t* qrow = q + b * qs[0] + (int64_t)i * qs[1] + h * qs[2];
                            const uint16_t* dorow = grad_o + b * dos[0] + (int64_t)i * dos[1] + h * dos[2];
                            for (int x = 0; x < d; ++x) ak[x] += ds * bf(qrow[x]);
                            for (int x = 0; x < dvd; ++x) av[x] += pb * bf(dorow[x]);
                        }
                    const size_t row = ((size_t)b * skv + j) * hkv + kvh;
                    if (dk)
                        for (int x = 0; x < d; ++x) dk[row * d + x] = ak[x];
                    if (dv)
                        for (int x = 0; x < dvd; ++x) dv[row * dvd + x] = av[x];
                }
    }
    free(delta);
    return 0;
}

int fgqa_oracle_prefill_backward_bf16(const uint16_t* q, const uint16_t* k, const uint16_t* v,
                                      const uint16_t* o, const float* lse, const uint16_t* grad_o,
                                      float scale, float* dq, float* dk, float* dv,
                                      int batch, int sq, int skv, int hq, int hkv, int d,
                                      const int64_t* qs, const int64_t* ks,
                                      const int64_t* vs, const int64_t* os,
                                      const int64_t* dos, int causal,
                                      const int* rows, const int* keys, int nthreads) {
    return backward_core(q, k, v, o, lse, grad_o, scale, dq, dk, dv, batch, sq, skv, hq, hkv, d, d, qs, ks, vs, os,
                         dos, causal, 0, rows, keys, nthreads);
}

/*
 * MLA backward (Q/K rows of dqk, V/O/dO rows of dv), restating
 * src/python/Triton/flash_mla_backward_kernel.py: the steps of the GQA
 * backward above with the scores over dqk (:366-372) and dP, delta over dv
 * (:388, :16-50).  dq, dk: dqk-element rows; dv: dv-element rows.
 */
int fgqa_oracle_prefill_mla_backward_bf16(const uint16_t* q, const uint16_t* k, const uint16_t* v,
                                          const uint16_t* o, const float* lse, const uint16_t* grad_o,
                                          float scale, float* dq, float* dk, float* dv,
                                          int batch, int sq, int skv, int hq, int hkv, int dqk, int dvd,
                                          const int64_t* qs, const int64_t* ks,
                                          const int64_t* vs, const int64_t* os,
                                          const int64_t* dos, int causal,
                                          const int* rows, const int* keys, int nthreads) {
    return backward_core(q, k, v, o, lse, grad_o, scale, dq, dk, dv, batch, sq, skv, hq, hkv, dqk, dvd, qs, ks, vs,
                         os, dos, causal, 0, rows, keys, nthreads);
}

/*
 * Sliding-window backward: the same steps with the window mask of
 * src/python/Triton/SWA/flash_swa_backward_kernel.py:278-282 (key j used by
 * row i when i - window < j <= i).  The sink enters only through the given
 * LSE, which the forward computed with it (:252-253 of the same file).
 */
int fgqa_oracle_prefill_swa_backward_bf16(const uint16_t* q, const uint16_t* k, const uint16_t* v,
                                          const uint16_t* o, const float* lse, const uint16_t* grad_o,
                                          float scale, float* dq, float* dk, float* dv,
                                          int batch, int sq, int skv, int hq, int hkv, int d,
                                          const int64_t* qs, const int64_t* ks,
                                          const int64_t* vs, const int64_t* os,
                                          const int64_t* dos, int window,
                                          const int* rows, const int* keys, int nthreads) {
    if (window <= 0) return -1;
    return backward_core(q, k, v, o, lse, grad_o, scale, dq, dk, dv, batch, sq, skv, hq, hkv, d, d, qs, ks, vs, os,
                         dos, 1, window, rows, keys, nthreads);
}

/* Exact gradient of softmax attention in double (see the header); window > 0
 * limits row i to keys (i - window, i], sink (nullable, per query head) adds
 * sink[h] to the softmax denominator. */
static int attention_backward_f64_core(const uint16_t* q, const uint16_t* k, const uint16_t* v,
                                       const uint16_t* o, const uint16_t* grad_o, double scale,
                                       double* dq, double* dk, double* dv,
                                       int batch, int sq, int skv, int hq, int hkv, int d, int dvd,
                                       const int64_t* qs, const int64_t* ks,
                                       const int64_t* vs, const int64_t* os,
                                       const int64_t* dos, int causal, int window, const float* sink,
                                       int nthreads) {
    if (!q || !k || !v || !grad_o || !dq || !dk || !dv || !qs || !ks || !vs || !dos) return -1;
    if (o && !os) return -1;
    if (batch < 0 || sq < 0 || skv < 0 || hq <= 0 || hkv <= 0 || d <= 0 || dvd <= 0) return -1;
    if (hq % hkv != 0 || window < 0 || (window > 0 && !causal)) return -1;
    const int group = hq / hkv;
    set_threads(nthreads);
    memset(dq, 0, sizeof(double) * (size_t)batch * sq * hq * d);
    memset(dk, 0, sizeof(double) * (size_t)batch * skv * hkv * d);
    memset(dv, 0, sizeof(double) * (size_t)batch * skv * hkv * dvd);

    /* One (batch, kv head) per task: its dK/dV rows are private to it. */
#pragma omp parallel for collapse(2) schedule(dynamic, 1)
    for (int b = 0; b < batch; ++b)
        for (int kvh = 0; kvh < hkv; ++kvh) {
            double* p = (double*)malloc(sizeof(double) * (size_t)(skv > 0 ? skv : 1));
            double* dp = (double*)malloc(sizeof(double) * (size_t)(skv > 0 ? skv : 1));
            for (int h = kvh * group; h < (kvh + 1) * group; ++h)
                for (int i = 0; i < sq; ++i) {
                    const uint16_t* qrow = q + b * qs[0] + (int64_t)i * qs[1] + h * qs[2];
                    const uint16_t* dorow = grad_o + b * dos[0] + (int64_t)i * dos[1] + h * dos[2];
                    const int nvis = causal ? (i + 1 < skv ? i + 1 : skv) : skv;
                    const int j0 = (window > 0 && i - window + 1 > 0) ? i - window + 1 : 0;
                    if (nvis <= j0) continue;
                    double rmax = -INFINITY;
                    for (int j = j0; j < nvis; ++j) {
                        const uint16_t* krow = k + b * ks[0] + (int64_t)j * ks[1] + kvh * ks[2];
                        double acc = 0.0;
                        for (int x = 0; x < d; ++x) acc += (double)bf(qrow[x]) * (double)bf(krow[x]);
                        p[j] = acc * scale;
                        if (p[j] > rmax) rmax = p[j];
                    }
                    double sum = 0.0;
                    for (int j = j0; j < nvis; ++j) {
                        p[j] = exp(p[j] - rmax);
                        sum += p[j];
                    }
                    if (sink) sum += (double)sink[h] * exp(-rmax);
                    double delta = 0.0;
                    for (int j = j0; j < nvis; ++j) {
                        p[j] /= sum;
                        const uint16_t* vrow = v + b * vs[0] + (int64_t)j * vs[1] + kvh * vs[2];
                        double acc = 0.0;
                        for (int x = 0; x < dvd; ++x) acc += (double)bf(dorow[x]) * (double)bf(vrow[x]);
                        dp[j] = acc;
                        delta += p[j] * acc;
                    }
                    if (o) {
                        const uint16_t* orow = o + b * os[0] + (int64_t)i * os[1] + h * os[2];
                        delta = 0.0;
                        for (int x = 0; x < dvd; ++x) delta += (double)bf(orow[x]) * (double)bf(dorow[x]);
                    }
                    double* dqrow = dq + (((size_t)b * sq + i) * hq + h) * d;
                    for (int j = j0; j < nvis; ++j) {
                        const double ds = p[j] * (dp[j] - delta) * scale;
                        const uint16_t* krow = k + b * ks[0] + (int64_t)j * ks[1] + kvh * ks[2];
                        double* dkrow = dk + (((size_t)b * skv + j) * hkv + kvh) * d;
                        double* dvrow = dv + (((size_t)b * skv + j) * hkv + kvh) * dvd;
                        for (int x = 0; x < d; ++x) {
                            dqrow[x] += ds * (double)bf(krow[x]);
                            dkrow[x] += ds * (double)bf(qrow[x]);
                        }
                        for (int x = 0; x < dvd; ++x) dvrow[x] += p[j] * (double)bf(dorow[x]);
                    }
                }
            free(p);
            free(dp);
        }
    return 0;
}

int fgqa_oracle_attention_backward_f64(const uint16_t* q, const uint16_t* k, const uint16_t* v,
                                       const uint16_t* o, const uint16_t* grad_o, double scale,
                                       double* dq, double* dk, double* dv,
                                       int batch, int sq, int skv, int hq, int hkv, int d,
                                       const int64_t* qs, const int64_t* ks,
                                       const int64_t* vs, const int64_t* os,
                                       const int64_t* dos, int causal, int nthreads) {
    return attention_backward_f64_core(q, k, v, o, grad_o, scale, dq, dk, dv, batch, sq, skv, hq, hkv, d, d, qs, ks,
                                       vs, os, dos, causal, 0, NULL, nthreads);
}

int fgqa_oracle_attention_mla_backward_f64(const uint16_t* q, const uint16_t* k, const uint16_t* v,
                                           const uint16_t* o, const uint16_t* grad_o, double scale,
                                           double* dq, double* dk, double* dv,
                                           int batch, int sq, int skv, int hq, int hkv, int dqk, int dvd,
                                           const int64_t* qs, const int64_t* ks,
                                           const int64_t* vs, const int64_t* os,
                                           const int64_t* dos, int causal, int nthreads) {
    return attention_backward_f64_core(q, k, v, o, grad_o, scale, dq, dk, dv, batch, sq, skv, hq, hkv, dqk, dvd, qs,
                                       ks, vs, os, dos, causal, 0, NULL, nthreads);
}

int fgqa_oracle_attention_swa_backward_f64(const uint16_t* q, const uint16_t* k, const uint16_t* v,
                                           const uint16_t* o, const uint16_t* grad_o, double scale,
                                           double* dq, double* dk, double* dv,
                                           int batch, int sq, int skv, int hq, int hkv, int d,
                                           const int64_t* qs, const int64_t* ks,
                                           const int64_t* vs, const int64_t* os,
                                           const int64_t* dos, int window, const float* sink, int nthreads) {
    if (window <= 0) return -1;
    return attention_backward_f64_core(q, k, v, o, grad_o, scale, dq, dk, dv, batch, sq, skv, hq, hkv, d, d, qs, ks,
                                       vs, os, dos, 1, window, sink, nthreads);
}

/*
 * Sparse-index prefill.  Per (batch, query head h, query row i) this follows
 * the torch reference examples/python/Triton/test_flash_sgqa_kernel.py:97-222:
 *   :185-188  slot s of row i holds key index j = idx[b][h / G][i][s]; it is
 *             valid when 0 <= j < Skv and, if causal, j <= the row's position
 *   :194-195  scores = (q . k_j) * scale over every slot (fp32), -inf if invalid
 *   :197-201  row_max; e = exp(scores - row_max), 0 where invalid; denom = sum(e);
 *             probs = e / denom (0 when denom == 0)
 *   :203-208  out = probs . v_j (fp32), lse = log(denom) + row_max, or -inf when
 *             denom == 0; out cast to bf16 (:212)
 * Slots are visited in order, so a key listed twice counts twice.
 */
int fgqa_oracle_sparse_prefill_bf16(const uint16_t* q, const uint16_t* k, const uint16_t* v,
                                    float scale, uint16_t* o, float* lse,
                                    int batch, int sq, int skv, int hq, int hkv, int d,
                                    const int64_t* qs, const int64_t* ks,
                                    const int64_t* vs, const int64_t* os,
                                    const int32_t* idx, const int64_t* is, int nsparse,
                                    int causal, int q_offset, int nthreads) {
    if (!q || !k || !v || !o || !qs || !ks || !vs || !os || !idx || !is) return -1;
    if (batch < 0 || sq < 0 || skv < 0 || hq <= 0 || hkv <= 0 || d <= 0 || d > ORACLE_MAX_D) return -1;
    if (hq % hkv != 0 || nsparse < 1) return -1;
    const int group = hq / hkv;
    set_threads(nthreads);

#pragma omp parallel
    {
        float* sc = (float*)malloc(sizeof(float) * (size_t)nsparse);
        int* kj = (int*)malloc(sizeof(int) * (size_t)nsparse);
        float out[ORACLE_MAX_D];
#pragma omp for collapse(3) schedule(dynamic, 4)
        for (int b = 0; b < batch; ++b) {
            for (int h = 0; h < hq; ++h) {
                for (int i = 0; i < sq; ++i) {
                    const int kvh = h / group;
                    const uint16_t* qrow = q + b * qs[0] + (int64_t)i * qs[1] + h * qs[2];
                    uint16_t* orow = o + b * os[0] + (int64_t)i * os[1] + h * os[2];
                    const int32_t* list = idx + b * is[0] + kvh * is[1] + (int64_t)i * is[2];
                    const long pos = (long)i + q_offset;
                    int nvis = 0;
                    float rmax = -INFINITY;
                    for (int s = 0; s < nsparse; ++s) {
                        const int j = list[s];
                        if (j < 0 || j >= skv || (causal && j > pos)) continue;
                        const uint16_t* krow = k + b * ks[0] + (int64_t)j * ks[1] + kvh * ks[2];
                        float acc = 0.f;
                        for (int x = 0; x < d; ++x) acc += bf(qrow[x]) * bf(krow[x]);
                        kj[nvis] = j;
                        sc[nvis] = acc * scale;
                        rmax = fmaxf(rmax, sc[nvis]);
                        ++nvis;
                    }
                    if (nvis == 0) {
                        for (int x = 0; x < d; ++x) orow[x] = 0;
                        if (lse) lse[((size_t)b * hq + h) * sq + i] = -INFINITY;
                        continue;
                    }
                    float sum = 0.f;
                    for (int t = 0; t < nvis; ++t) {
                        sc[t] = expf(sc[t] - rmax);
                        sum += sc[t];
                    }
                    for (int x = 0; x < d; ++x) out[x] = 0.f;
                    for (int t = 0; t < nvis; ++t) {
                        const uint16_t* vrow = v + b * vs[0] + (int64_t)kj[t] * vs[1] + kvh * vs[2];
                        const float pj = sc[t] / sum;
                        for (int x = 0; x < d; ++x) out[x] += pj * bf(vrow[x]);
                    }
                    for (int x = 0; x < d; ++x) orow[x] = fgqa_oracle_f32_to_bf16(out[x]);
                    if (lse) lse[((size_t)b * hq + h) * sq + i] = logf(sum) + rmax;
                }
            }
        }
        free(kj);
        free(sc);
    }
    return 0;
}
