// Causal GQA prefill forward for gfx950.
//
// Stands in for the reference's Triton-only flash_gqa_forward_bf16_kernel
// (src/python/Triton/flash_gqa_kernel.py:15-138).  Same maths: S = Q.K^T*scale
// in fp32, top-left causal mask (q_idx >= kv_idx, :113-117), online softmax,
// P rounded to bf16 before P.V with the rowsum kept from the fp32 P (:122-129),
// O /= rowsum and lse = max + log(rowsum) (:131-138).
//
// One workgroup = 4 waves = 128 query rows: HB heads of one KV group x
// (128/HB) consecutive query positions, so the 4 waves share every K/V tile
// staged in LDS (HB = 4 when G % 4 == 0, else 2 or 1).  Per wave, 32 rows:
//   S^T[t][q] = K[t][:] . Q[q][:]       v_mfma_f32_32x32x16_bf16 (K from LDS,
//                                       Q^T held in registers for the whole loop)
//   O^T[d][q] += V^T[d][t] . P^T[t][q]  v_mfma_f32_32x32x16_bf16; P^T is the
//                                       S^T accumulator itself, converted in
//                                       registers, V^T staged transposed in LDS
// K/V tiles of 64 tokens are double buffered in LDS: tile j+1 is fetched into
// registers while tile j is multiplied.  Causal tile skipping: a workgroup
// stops at its last query row, and heavy (late) query blocks are launched
// first so the light ones fill the tail.
#include <math.h>

#include "fgqa_device.h"
#include "fgqa_internal.h"

namespace fgqa {

struct PrefillParams {
    const __bf16* q;
    const __bf16* k;
    const __bf16* v;
    __bf16* o;
    float* lse;
    int64_t q_sb, q_ss, q_sh;
    int64_t k_sb, k_ss, k_sh;
    int64_t v_sb, v_ss, v_sh;
    int64_t o_sb, o_ss, o_sh;
    int batch, sq, skv, hq, hkv, group, causal;
    int hb;         // heads per workgroup
    int n_hgroups;  // group / hb
    int n_qblocks;  // ceil(sq / (128 / hb))
    float scale_log2;
};

constexpr int kPfThreads = 256;
constexpr int kPfTile = 64;        // KV tokens per tile
constexpr int kPfKStride = 136;    // K tile row stride in LDS (elements): conflict-free b128 reads
constexpr int kPfVtStride = 68;    // V^T tile row stride in LDS (elements): conflict-free b64 reads
constexpr int kPfKBytes = kPfTile * kPfKStride * 2;
constexpr int kPfVtBytes = kHeadDim * kPfVtStride * 2;
constexpr int kPfBufBytes = kPfKBytes + kPfVtBytes;
constexpr int kPfSmemBytes = 2 * kPfBufBytes;

__global__ __launch_bounds__(kPfThreads) void prefill_kernel(PrefillParams p) {
    extern __shared__ __attribute__((aligned(16))) unsigned char smem[];

    // Block index -> (query block, head group, kv head, batch); late query
    // blocks (most KV tiles under a causal mask) come first.
    int idx = blockIdx.x;
    const int per_q = p.n_hgroups * p.hkv * p.batch;
    int qb = idx / per_q;
    int rem = idx - qb * per_q;
    if (p.causal) qb = p.n_qblocks - 1 - qb;
    const int hg = rem % p.n_hgroups;
    rem /= p.n_hgroups;
    const int kvh = rem % p.hkv;
    const int b = rem / p.hkv;

    const int tid = threadIdx.x;
    const int lane = tid & (kWave - 1);
    const int wave = tid / kWave;
    const int l32 = lane & 31;
    const int g2 = lane >> 5;
    const int qrows = 128 / p.hb;
    const int q_wg0 = qb * qrows;
    const int h = kvh * p.group + hg * p.hb + (wave % p.hb);
    const int q0w = q_wg0 + (wave / p.hb) * 32;

    // KV extent of the workgroup and of this wave.
    int kv_end = p.skv;
    if (p.causal) kv_end = min(kv_end, min(q_wg0 + qrows, p.sq));
    int kv_end_w = p.skv;
    if (p.causal) kv_end_w = min(kv_end_w, q0w + 32);
    const int n_tiles = (kv_end + kPfTile - 1) / kPfTile;

    // Q^T as the B operand: lane holds Q[q0w + l32][16*kk + 8*g2 .. +7]; rows >= sq read as 0.
    const uint32_t qss = (uint32_t)(p.q_ss * 2);
    const __amdgpu_buffer_rsrc_t qrs =
        make_rsrc(p.q + b * p.q_sb + h * p.q_sh, (uint32_t)(p.sq - 1) * qss + kHeadDim * 2);
    bf16x8_t qop[8];
#pragma unroll
    for (int kk = 0; kk < 8; ++kk)
        qop[kk] = as_bf16x8(buf_load16(qrs, (uint32_t)(q0w + l32) * qss + (kk * 16 + g2 * 8) * 2));

    // Tile loader: thread (c = tid % 16, r0 = tid / 16) moves the 16-byte chunk c
    // of token rows r0 + 16*i, i = 0..3.
    const int c = tid & 15;
    const int r0 = tid >> 4;
    const uint32_t kss = (uint32_t)(p.k_ss * 2);
    const uint32_t vss = (uint32_t)(p.v_ss * 2);
    const uint32_t kv_last = (uint32_t)(p.skv > 0 ? p.skv - 1 : 0);
    const __amdgpu_buffer_rsrc_t krs = make_rsrc(p.k + b * p.k_sb + kvh * p.k_sh, kv_last * kss + kHeadDim * 2);
    const __amdgpu_buffer_rsrc_t vrs = make_rsrc(p.v + b * p.v_sb + kvh * p.v_sh, kv_last * vss + kHeadDim * 2);
    u32x4_t kr[4], vr[4];
    auto load_tile = [&](int j) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint32_t tok = (uint32_t)(j * kPfTile + r0 + 16 * i);
            kr[i] = buf_load16(krs, tok * kss + c * 16);
            vr[i] = buf_load16(vrs, tok * vss + c * 16);
        }
    };
    auto store_tile = [&](int buf) {
        __bf16* kl = reinterpret_cast<__bf16*>(smem + buf * kPfBufBytes);
        __bf16* vt = reinterpret_cast<__bf16*>(smem + buf * kPfBufBytes + kPfKBytes);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int row = r0 + 16 * i;
            *reinterpret_cast<u32x4_t*>(kl + row * kPfKStride + c * 8) = kr[i];
            const bf16x8_t vv = as_bf16x8(vr[i]);
#pragma unroll
            for (int e = 0; e < 8; ++e) vt[(c * 8 + e) * kPfVtStride + row] = vv[e];
        }
    };

    float m_run = -INFINITY;
    float l_run = 0.f;
    f32x16_t oacc[4];
#pragma unroll
    for (int db = 0; db < 4; ++db)
#pragma unroll
        for (int i = 0; i < 16; ++i) oacc[db][i] = 0.f;

    if (n_tiles > 0) {
        load_tile(0);
        store_tile(0);
    }
    const int qrow = q0w + l32;
    for (int j = 0; j < n_tiles; ++j) {
        __syncthreads();
        const int buf = j & 1;
        if (j + 1 < n_tiles) load_tile(j + 1);
        const int kv0 = j * kPfTile;
        if (kv0 < kv_end_w) {
            const __bf16* kl = reinterpret_cast<const __bf16*>(smem + buf * kPfBufBytes);
            const __bf16* vt = reinterpret_cast<const __bf16*>(smem + buf * kPfBufBytes + kPfKBytes);
            f32x16_t s[2];
#pragma unroll
            for (int tb = 0; tb < 2; ++tb) {
#pragma unroll
                for (int i = 0; i < 16; ++i) s[tb][i] = 0.f;
#pragma unroll
                for (int kk = 0; kk < 8; ++kk) {
                    const bf16x8_t ka =
                        *reinterpret_cast<const bf16x8_t*>(kl + (tb * 32 + l32) * kPfKStride + kk * 16 + g2 * 8);
                    s[tb] = mfma32(ka, qop[kk], s[tb]);
                }
            }
            // Online softmax for query row qrow over tokens kv0 + 32*tb + 8*(i/4) + 4*g2 + i%4.
            const bool need_mask = (kv0 + kPfTile > p.skv) || (p.causal && kv0 + kPfTile - 1 > q0w);
            float tmax = -INFINITY;
#pragma unroll
            for (int tb = 0; tb < 2; ++tb)
#pragma unroll
                for (int i = 0; i < 16; ++i) {
                    float val = s[tb][i] * p.scale_log2;
                    if (need_mask) {
                        const int tok = kv0 + tb * 32 + (i >> 2) * 8 + g2 * 4 + (i & 3);
                        if (tok >= p.skv || (p.causal && tok > qrow)) val = -INFINITY;
                    }
                    s[tb][i] = val;
                    tmax = fmaxf(tmax, val);
                }
            tmax = xor_max(tmax, 32);
            const float m_new = fmaxf(m_run, tmax);
            const float m_use = (m_new == -INFINITY) ? 0.f : m_new;
            const float alpha = fast_exp2(m_run - m_use);
            float psum = 0.f;
#pragma unroll
            for (int tb = 0; tb < 2; ++tb)
#pragma unroll
                for (int i = 0; i < 16; ++i) {
                    const float pv = fast_exp2(s[tb][i] - m_use);
                    s[tb][i] = pv;
                    psum += pv;
                }
            l_run = l_run * alpha + psum;
            m_run = m_new;
#pragma unroll
            for (int db = 0; db < 4; ++db) oacc[db] *= alpha;

            // P.V over four 16-token k-blocks: slots 8*g2 + e map to tokens
            // tA + e (e < 4) and tA + 8 + (e - 4), tA = 32*tb + 16*kh + 4*g2,
            // exactly the S^T registers 8*kh .. 8*kh + 7 of this lane.
#pragma unroll
            for (int tb = 0; tb < 2; ++tb)
#pragma unroll
                for (int kh = 0; kh < 2; ++kh) {
                    bf16x8_t pb;
#pragma unroll
                    for (int e = 0; e < 8; ++e) pb[e] = (__bf16)s[tb][kh * 8 + e];
                    const int tA = tb * 32 + kh * 16 + g2 * 4;
#pragma unroll
                    for (int db = 0; db < 4; ++db) {
                        const __bf16* vrow = vt + (db * 32 + l32) * kPfVtStride;
                        const bf16x4_t lo = *reinterpret_cast<const bf16x4_t*>(vrow + tA);
                        const bf16x4_t hi = *reinterpret_cast<const bf16x4_t*>(vrow + tA + 8);
                        const bf16x8_t va = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
                        oacc[db] = mfma32(va, pb, oacc[db]);
                    }
                }
        }
        if (j + 1 < n_tiles) store_tile(buf ^ 1);
    }

    l_run = xor_sum(l_run, 32);
    if (qrow < p.sq) {
        const float inv = (l_run > 0.f) ? 1.f / l_run : 0.f;
        __bf16* orow = p.o + b * p.o_sb + (int64_t)qrow * p.o_ss + h * p.o_sh;
#pragma unroll
        for (int db = 0; db < 4; ++db)
#pragma unroll
            for (int i4 = 0; i4 < 4; ++i4) {
                bf16x4_t w;
#pragma unroll
                for (int e = 0; e < 4; ++e) w[e] = (__bf16)(oacc[db][i4 * 4 + e] * inv);
                *reinterpret_cast<bf16x4_t*>(orow + db * 32 + i4 * 8 + g2 * 4) = w;
            }
        if (p.lse != nullptr && g2 == 0)
            p.lse[((int64_t)b * p.hq + h) * p.sq + qrow] = (l_run > 0.f) ? m_run * kLn2 + logf(l_run) : -INFINITY;
    }
}

namespace {

int validate_prefill(const fgqa_prefill_args* a) {
    if (a == nullptr) return FGQA_ERR_INVALID_ARGUMENT;
    if (a->batch < 0 || a->seqlen_q < 0 || a->seqlen_kv < 0 || a->num_q_heads <= 0 ||
        a->num_kv_heads <= 0 || a->head_dim <= 0)
        return FGQA_ERR_INVALID_ARGUMENT;
    if (a->num_q_heads % a->num_kv_heads != 0) return FGQA_ERR_INVALID_ARGUMENT;
    if (!isfinite(a->scale)) return FGQA_ERR_INVALID_ARGUMENT;
    for (int i = 0; i < 3; ++i)
        if (a->q_stride[i] < 0 || a->k_stride[i] < 0 || a->v_stride[i] < 0 || a->o_stride[i] < 0)
            return FGQA_ERR_INVALID_ARGUMENT;
    if (a->head_dim != kHeadDim) return FGQA_ERR_UNSUPPORTED;
    const int64_t lim = (int64_t)1 << 31;
    if ((int64_t)(a->seqlen_q + 128) * a->q_stride[1] * 2 >= lim ||
        (int64_t)(a->seqlen_kv + 128) * a->k_stride[1] * 2 >= lim ||
        (int64_t)(a->seqlen_kv + 128) * a->v_stride[1] * 2 >= lim)
        return FGQA_ERR_UNSUPPORTED;
    if (a->batch == 0 || a->seqlen_q == 0) return FGQA_OK;
    if (a->q == nullptr || a->k == nullptr || a->v == nullptr || a->o == nullptr)
        return FGQA_ERR_INVALID_ARGUMENT;
    if (!aligned16(a->q) || !aligned16(a->k) || !aligned16(a->v) || !aligned16(a->o))
        return FGQA_ERR_UNSUPPORTED;
    for (int i = 0; i < 3; ++i)
        if ((a->q_stride[i] & 7) || (a->k_stride[i] & 7) || (a->v_stride[i] & 7) || (a->o_stride[i] & 3))
            return FGQA_ERR_UNSUPPORTED;
    return FGQA_OK;
}

}  // namespace
}  // namespace fgqa

using namespace fgqa;

extern "C" int fgqa_prefill_bf16(const fgqa_prefill_args* a, void* stream) {
    int st = validate_prefill(a);
    if (st != FGQA_OK) return st;
    if (a->batch == 0 || a->seqlen_q == 0) return FGQA_OK;

    PrefillParams p;
    p.q = static_cast<const __bf16*>(a->q);
    p.k = static_cast<const __bf16*>(a->k);
    p.v = static_cast<const __bf16*>(a->v);
    p.o = static_cast<__bf16*>(a->o);
    p.lse = a->lse;
    p.q_sb = a->q_stride[0];
    p.q_ss = a->q_stride[1];
    p.q_sh = a->q_stride[2];
    p.k_sb = a->k_stride[0];
    p.k_ss = a->k_stride[1];
    p.k_sh = a->k_stride[2];
    p.v_sb = a->v_stride[0];
    p.v_ss = a->v_stride[1];
    p.v_sh = a->v_stride[2];
    p.o_sb = a->o_stride[0];
    p.o_ss = a->o_stride[1];
    p.o_sh = a->o_stride[2];
    p.batch = a->batch;
    p.sq = a->seqlen_q;
    p.skv = a->seqlen_kv;
    p.hq = a->num_q_heads;
    p.hkv = a->num_kv_heads;
    p.group = a->num_q_heads / a->num_kv_heads;
    p.causal = a->causal ? 1 : 0;
    p.hb = (p.group % 4 == 0) ? 4 : (p.group % 2 == 0) ? 2 : 1;
    p.n_hgroups = p.group / p.hb;
    p.n_qblocks = (int)ceil_div(p.sq, 128 / p.hb);
    p.scale_log2 = a->scale * kLog2e;

    const int64_t nblocks = (int64_t)p.n_qblocks * p.n_hgroups * p.hkv * p.batch;
    if (nblocks >= ((int64_t)1 << 31)) return FGQA_ERR_UNSUPPORTED;

    static bool smem_set = false;
    if (!smem_set) {
        if (hipFuncSetAttribute(reinterpret_cast<const void*>(prefill_kernel),
                                hipFuncAttributeMaxDynamicSharedMemorySize, kPfSmemBytes) != hipSuccess)
            return FGQA_ERR_HIP;
        smem_set = true;
    }
    hipLaunchKernelGGL(prefill_kernel, dim3((unsigned)nblocks), dim3(kPfThreads), kPfSmemBytes,
                       static_cast<hipStream_t>(stream), p);
    if (hipGetLastError() != hipSuccess) return FGQA_ERR_HIP;
    return FGQA_OK;
}
