// Split-KV (flash-decoding) GQA decode for gfx950.
//
// Replaces the reference's decode_flash_gqa_bf16_kernel
// (src/cplusplus/FlashGQA/decode_flash_gqa_kernel.cu:119-389), which walks the
// whole sequence serially per (kv head, batch) workgroup.  Here:
//   pass 1 (decode_split_kernel): 4 waves per (split of the KV sequence,
//     kv head, batch), two such items (adjacent kv heads) per 8-wave
//     workgroup when the kv heads pair up.  Each wave streams 32-token steps;
//     every K/V byte is read once from HBM and serves all G query heads of
//     the group.
//       K and V rows stream in with coalesced 16-byte non-temporal loads
//       (a quarter-wave reads one 256-byte row) and are staged in LDS
//       S^T[t][h] = K[t][:] . Q[h][:]        v_mfma_f32_16x16x32_bf16
//       online softmax in fp32 (exp2 with log2(e) folded into the scale), P
//       rounded to bf16 before P.V and the rowsum kept from the fp32 P, as the
//       reference does (decode_flash_gqa_kernel.cu:266-278)
//       O^T[d][h] += V^T[d][t] . P^T[t][h]   v_mfma_f32_16x16x32_bf16, V^T
//                                            read transposed from the staged
//                                            rows (ds_read_b64_tr_b16)
//     The 4 waves merge their (max, sum, O) in LDS; with one split the
//     workgroup writes the normalised bf16 output directly, otherwise it
//     writes an fp32 partial (O, max, sum) to the workspace.
//   pass 2 (decode_combine_kernel): log-sum-exp merge of the partials.
//
// Paged KV cache (fgqa_decode_paged): the same kernels read K/V rows through a
// block table (token t of sequence b lives in page block_table[b][t / page],
// slot t % page), in bf16 or in OCP fp8 e4m3 with per-tensor scales.  fp8 rows
// are widened to bf16 exactly (v_cvt_scalef32_pk_bf16_fp8, scale 1) as they are
// staged in LDS; the K scale is folded into the softmax scale and the V scale
// into the output, so the arithmetic after staging is the bf16 path's.  Pages
// of at least one load instruction's rows (4 bf16 rows, 8 fp8 rows) are read
// by page segment (min(page, 32) rows of a step): one buffer resource per
// segment, the wave's pages taken from one vector load of the block table per
// 64 segments; smaller pages, and caches whose page bytes reach 2^31, look up
// each row's page and form its 64-bit address.
#include <math.h>

#include "fgqa_device.h"
#include "fgqa_internal.h"

namespace fgqa {

struct DecodeParams {
    const __bf16* q;
    const __bf16* k;
    const __bf16* v;
    __bf16* o;
    float* lse;
    const int32_t* seqlens;
    float* part_o;   // [B, Hkv, nsplit, G, 128]
    float* part_ml;  // [B, Hkv, nsplit, G, 2]  (max in log2 units, sum)
    int64_t q_sb, q_sh;
    int64_t k_sb, k_ss, k_sh;
    int64_t v_sb, v_ss, v_sh;
    int64_t o_sb, o_sh;
    const int32_t* work;   // ragged work list: [0] = entries, then (b << 16 | split) per entry
    int batch, max_seqlen, hq, hkv, group;
    int nsplit, chunk;
    float scale_log2;
    // paged KV: k/v are the page caches, strides {page, slot, head} in elements
    // of the cache type; page of token t = block_table[b * bt_stride + (t >> page_shift)]
    const int32_t* block_table;
    int64_t bt_stride;
    int page_shift;
    int num_pages;      // page indices are clamped to [0, num_pages)
    float v_scale;      // multiplies O (the fp8 V scale; 1 otherwise)
};

// Cache layouts the decode items read.
enum DecKv { kKvContig = 0, kKvPagedBf16 = 1, kKvPagedFp8 = 2 };

// 16 OCP fp8 e4m3 values -> 16 bf16 (exact: every e4m3 value is a bf16 value).
__device__ __forceinline__ void fp8x16_to_bf16(u32x4_t in, u32x4_t* lo, u32x4_t* hi) {
    uint32_t w[8];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        w[2 * i] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(in[i], 1.0f, false));
        w[2 * i + 1] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(in[i], 1.0f, true));
    }
    *lo = u32x4_t{w[0], w[1], w[2], w[3]};
    *hi = u32x4_t{w[4], w[5], w[6], w[7]};
}

constexpr int kDecThreads = 256;
constexpr int kDecWaves = kDecThreads / kWave;
constexpr int kDecStep = 32;        // tokens per wave step (two 16-token MFMA blocks)
constexpr int kDecRowStride = 136;  // LDS row stride (elements) of a staged K or V row: 272 B
                                    // spreads 16 rows over all 64 banks for b128 reads
constexpr int kDecTileElems = kDecStep * kDecRowStride;
constexpr int kDecSmemBytes = kDecWaves * 2 * kDecTileElems * 2;  // per wave: K tile + V tile
static_assert(kDecWaves * 16 * kHeadDim * 4 + kDecWaves * 16 * 2 * 4 <= kDecSmemBytes,
              "wave merge buffers must fit in the staging area");

__device__ __forceinline__ int clamp_len(const DecodeParams& p, int b) {
    int len = p.seqlens ? p.seqlens[b] : p.max_seqlen;
    return min(max(len, 0), p.max_seqlen);
}

// One (split, kv head, batch) item of pass 1, run by 4 waves (tid: the
// thread's index among them, smem: their kDecSmemBytes of LDS).  kSeg (paged
// caches, 0 or a power of two from one load instruction's rows up to 32): the
// rows of a 32-token step fall into page segments of kSeg rows
// (kSeg = min(page, 32)), each read through one buffer resource; 0 is the
// general form, with a page lookup and a 64-bit address per row.
// The only workgroup barriers are the two of the wave merge (none when the
// split is empty), so two items of one split can share a workgroup.
template <int kKv, int kSeg = 0>
__device__ __forceinline__ void dec_item(const DecodeParams& p, unsigned char* smem, int split, int kvh, int b,
                                         int tid) {
    const int len = clamp_len(p, b);
    const int t_begin = split * p.chunk;
    if (t_begin >= len) {
        // Empty split: the combine never reads it.  Without a combine pass an
        // empty sequence still needs its O = 0, lse = -inf written here.
        if (p.nsplit == 1 && (tid >> 4) < p.group) {
            const int qh = kvh * p.group + (tid >> 4);
            bf16x8_t z;
#pragma unroll
            for (int j = 0; j < 8; ++j) z[j] = (__bf16)0.f;
            *reinterpret_cast<bf16x8_t*>(p.o + b * p.o_sb + qh * p.o_sh + (tid & 15) * 8) = z;
            if (p.lse != nullptr && (tid & 15) == 0) p.lse[(int64_t)b * p.hq + qh] = -INFINITY;
        }
        return;
    }
    const int t_end = min(t_begin + p.chunk, len);

    const int lane = tid & (kWave - 1);
    constexpr bool kUni = kSeg > 0;
    const int wave = kUni ? __builtin_amdgcn_readfirstlane(tid / kWave) : tid / kWave;
    const int l16 = lane & 15;
    const int g4 = lane >> 4;

    __bf16* kl = reinterpret_cast<__bf16*>(smem) + wave * 2 * kDecTileElems;
    __bf16* vl = kl + kDecTileElems;

    // Q^T as the B operand: lane holds Q[h = l16][32*kk + 8*g4 .. +7]; heads >= G are zero.
    bf16x8_t qop[4];
    {
        const bool hv = l16 < p.group;
        const __bf16* qrow = p.q + b * p.q_sb + (int64_t)(kvh * p.group + (hv ? l16 : 0)) * p.q_sh;
        const u32x4_t zero = {0u, 0u, 0u, 0u};
#pragma unroll
        for (int kk = 0; kk < 4; ++kk) {
            u32x4_t t = *reinterpret_cast<const u32x4_t*>(qrow + kk * 32 + g4 * 8);
            qop[kk] = as_bf16x8(hv ? t : zero);
        }
    }

    float m_run = -INFINITY;
    float l_run = 0.f;  // this lane's share of the rowsum of head l16
    f32x4_t oacc[8];
#pragma unroll
    for (int db = 0; db < 8; ++db) oacc[db] = f32x4_t{0.f, 0.f, 0.f, 0.f};

    const int n_steps = (t_end - t_begin + kDecStep - 1) / kDecStep;
    // One step = 32 token rows of K and of V.  bf16: load r (0..7) of a lane
    // covers row 4*r + g4, 16-byte chunk l16, so each quarter-wave reads one
    // whole 256-byte row (the coalesced pattern).  fp8: rows are 128 bytes;
    // load r (0..3) covers row 8*r + lane/8, chunk lane%8.
    constexpr int kRows = (kKv == kKvPagedFp8) ? 4 : 8;
    const int fp8_row = lane >> 3;
    const int fp8_chunk = lane & 7;
    auto row_of = [&](int r) { return (kKv == kKvPagedFp8) ? 8 * r + fp8_row : 4 * r + g4; };
    u32x4_t kreg[kRows];
    u32x4_t vreg[kRows];

    // Contiguous cache: buffer resources end at the split's last valid token,
    // so later tokens read as zero.
    const uint32_t kss = (uint32_t)(p.k_ss * 2);
    const uint32_t vss = (uint32_t)(p.v_ss * 2);
    __amdgpu_buffer_rsrc_t krs, vrs;
    if constexpr (kKv == kKvContig) {
        krs = make_rsrc(p.k + b * p.k_sb + kvh * p.k_sh, (uint32_t)(t_end - 1) * kss + kHeadDim * 2);
        vrs = make_rsrc(p.v + b * p.v_sb + kvh * p.v_sh, (uint32_t)(t_end - 1) * vss + kHeadDim * 2);
    }
    // Paged cache: each row's page comes from the block table one step ahead
    // of its load.  Tokens past the split's end reuse its last token (their
    // scores are masked; the row only has to be finite).
    constexpr int kElemBytes = (kKv == kKvPagedFp8) ? 1 : 2;
    const unsigned char* kbase = reinterpret_cast<const unsigned char*>(p.k) + kvh * p.k_sh * kElemBytes;
    const unsigned char* vbase = reinterpret_cast<const unsigned char*>(p.v) + kvh * p.v_sh * kElemBytes;
    const int32_t* bt = p.block_table + (int64_t)b * p.bt_stride;
    const int pmask = (1 << p.page_shift) - 1;
    int pg[kRows];
    // kSeg > 0: segment g of a step (rows kSeg*g .. +kSeg-1, one page) is
    // read through one buffer resource per cache, starting at the segment's
    // first row and ending at the split's last token (rows past it read as
    // zeros).  The wave's segment pages come 64 at a time from one vector
    // load of the block table (lane l: the wave's segment pt_first + l, its
    // segments numbered n * kSegs + g for its n-th step) and are taken out
    // with v_readlane (a scalar load would share its wait counter with the
    // LDS traffic).  Load instruction i
    // of a segment reads its rows kR*i .. kR*i + kR - 1 at a per-lane offset
    // that is the same in every segment and step.  The host picks kSeg only
    // when a page's bytes stay below 2^31.
    constexpr int kR = (kKv == kKvPagedFp8) ? 8 : 4;           // rows per load instruction
    constexpr int kSegs = kUni ? kDecStep / kSeg : 1;          // segments per step
    constexpr int kPerSeg = kRows / kSegs;                     // load instructions per segment
    static_assert(!kUni || (kSeg >= kR && kSeg <= kDecStep && kPerSeg * kSegs == kRows), "page segment");
    constexpr uint32_t kRowBytes = kHeadDim * kElemBytes;
    const uint32_t kss_e = (uint32_t)(p.k_ss * kElemBytes);
    const uint32_t vss_e = (uint32_t)(p.v_ss * kElemBytes);
    const int64_t ksb_e = p.k_sb * kElemBytes;
    const int64_t vsb_e = p.v_sb * kElemBytes;
    const int t_end_u = kUni ? __builtin_amdgcn_readfirstlane(t_end) : t_end;
    [[maybe_unused]] uint32_t kvoff[kPerSeg], vvoff[kPerSeg];
    if constexpr (kUni) {
        const int lr = (kKv == kKvPagedFp8) ? fp8_row : g4;             // the lane's row in an instruction
        const int cb = (kKv == kKvPagedFp8) ? fp8_chunk * 16 : l16 * 16;
#pragma unroll
        for (int i = 0; i < kPerSeg; ++i) {
            kvoff[i] = (uint32_t)(kR * i + lr) * kss_e + cb;
            vvoff[i] = (uint32_t)(kR * i + lr) * vss_e + cb;
        }
    }
    [[maybe_unused]] int pt_lane = 0;       // block table entry of segment pt_first + lane
    [[maybe_unused]] int pt_first = -kWave;
    [[maybe_unused]] auto pt_load = [&](int first) {
        const int n = first + lane;
        const int tok = min(t_begin + (wave + kDecWaves * (n / kSegs)) * kDecStep + kSeg * (n % kSegs), t_end_u - 1);
        pt_lane = bt[tok >> p.page_shift];
        pt_first = first;
    };
    if constexpr (kUni) pt_load(0);
    auto fetch_pages = [&](int s) {
        if constexpr (kUni) {
            (void)s;   // the pages are taken out in load_step
        } else if constexpr (kKv != kKvContig) {
            // Raw entries: they are clamped where load_step uses them.  A
            // clamp here would make the wave wait for the table loads at once,
            // and vector loads complete in order, so that wait would also take
            // the K/V loads issued just before, leaving none in flight while
            // the step computes.
#pragma unroll
            for (int r = 0; r < kRows; ++r) {
                const int tok = min(t_begin + s * kDecStep + row_of(r), t_end - 1);
                pg[r] = bt[tok >> p.page_shift];
            }
        }
    };
    auto load_step = [&](int s) {
        const int t0 = t_begin + s * kDecStep;
        if constexpr (kUni) {
            const int n0 = ((s - wave) / kDecWaves) * kSegs;   // the wave's first segment of step s
            if (n0 + kSegs > pt_first + kWave) pt_load(n0);
#pragma unroll
            for (int g = 0; g < kSegs; ++g) {
                pg[g] = min(max(__builtin_amdgcn_readlane(pt_lane, n0 - pt_first + g), 0), p.num_pages - 1);
            }
#pragma unroll
            for (int g = 0; g < kSegs; ++g) {
                const int tok = t0 + kSeg * g;
                const int nv = min(kSeg, t_end_u - tok);   // rows before the split's end
                const uint32_t slot = (uint32_t)(tok & pmask);
                const __amdgpu_buffer_rsrc_t kr = make_rsrc(kbase + pg[g] * ksb_e + slot * kss_e,
                                                            nv > 0 ? (uint32_t)(nv - 1) * kss_e + kRowBytes : 0u);
                const __amdgpu_buffer_rsrc_t vr = make_rsrc(vbase + pg[g] * vsb_e + slot * vss_e,
                                                            nv > 0 ? (uint32_t)(nv - 1) * vss_e + kRowBytes : 0u);
#pragma unroll
                for (int i = 0; i < kPerSeg; ++i) {
                    kreg[g * kPerSeg + i] = buf_load16_nt(kr, kvoff[i]);
                    vreg[g * kPerSeg + i] = buf_load16_nt(vr, vvoff[i]);
                }
            }
        } else if constexpr (kKv == kKvContig) {
#pragma unroll
            for (int r = 0; r < 8; ++r) kreg[r] = buf_load16_nt(krs, (uint32_t)(t0 + r * 4 + g4) * kss + l16 * 16);
#pragma unroll
            for (int r = 0; r < 8; ++r) vreg[r] = buf_load16_nt(vrs, (uint32_t)(t0 + r * 4 + g4) * vss + l16 * 16);
        } else {
            const int cb = (kKv == kKvPagedFp8) ? fp8_chunk * 16 : l16 * 16;
#pragma unroll
            for (int r = 0; r < kRows; ++r) {
                const int slot = min(t0 + row_of(r), t_end - 1) & pmask;
                const int page = min(max(pg[r], 0), p.num_pages - 1);
                const int64_t ko = ((int64_t)page * p.k_sb + (int64_t)slot * p.k_ss) * kElemBytes + cb;
                const int64_t vo = ((int64_t)page * p.v_sb + (int64_t)slot * p.v_ss) * kElemBytes + cb;
                kreg[r] = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(kbase + ko));
                vreg[r] = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(vbase + vo));
            }
        }
    };

    int st = wave;
    if (st < n_steps) {
        fetch_pages(st);
        load_step(st);
    }
    if (st + kDecWaves < n_steps) fetch_pages(st + kDecWaves);
    for (; st < n_steps; st += kDecWaves) {
        // Stage this step's rows (fp8 widened to bf16), then put the next
        // step's loads and the page lookups of the step after in flight.
        if constexpr (kKv == kKvPagedFp8) {
#pragma unroll
            for (int r = 0; r < kRows; ++r) {
                u32x4_t lo, hi;
                __bf16* kd = kl + row_of(r) * kDecRowStride + fp8_chunk * 16;
                __bf16* vd = vl + row_of(r) * kDecRowStride + fp8_chunk * 16;
                fp8x16_to_bf16(kreg[r], &lo, &hi);
                *reinterpret_cast<u32x4_t*>(kd) = lo;
                *reinterpret_cast<u32x4_t*>(kd + 8) = hi;
                fp8x16_to_bf16(vreg[r], &lo, &hi);
                *reinterpret_cast<u32x4_t*>(vd) = lo;
                *reinterpret_cast<u32x4_t*>(vd + 8) = hi;
            }
        } else {
#pragma unroll
            for (int r = 0; r < 8; ++r) {
                *reinterpret_cast<u32x4_t*>(kl + (r * 4 + g4) * kDecRowStride + l16 * 8) = kreg[r];
                *reinterpret_cast<u32x4_t*>(vl + (r * 4 + g4) * kDecRowStride + l16 * 8) = vreg[r];
            }
        }
        if (st + kDecWaves < n_steps) load_step(st + kDecWaves);
        if (st + 2 * kDecWaves < n_steps) fetch_pages(st + 2 * kDecWaves);
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");

        // S^T = K Q^T; K as the A operand: lane holds K[16*tb + l16][32*kk + 8*g4 .. +7].
        const int t0 = t_begin + st * kDecStep;
        f32x4_t s[2];
#pragma unroll
        for (int tb = 0; tb < 2; ++tb) {
            s[tb] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int kk = 0; kk < 4; ++kk) {
                const bf16x8_t ka =
                    *reinterpret_cast<const bf16x8_t*>(kl + (tb * 16 + l16) * kDecRowStride + kk * 32 + g4 * 8);
                s[tb] = mfma16(ka, qop[kk], s[tb]);
            }
        }

        // Online softmax for head l16 over tokens t0 + 16*tb + 4*g4 + i.
        float x[8];
        float tmax = -INFINITY;
#pragma unroll
        for (int tb = 0; tb < 2; ++tb)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int tok = t0 + tb * 16 + g4 * 4 + i;
                const float val = (tok < t_end) ? s[tb][i] * p.scale_log2 : -INFINITY;
                x[tb * 4 + i] = val;
                tmax = fmaxf(tmax, val);
            }
        tmax = xor_max(xor_max(tmax, 16), 32);
        const float m_new = fmaxf(m_run, tmax);  // finite: every step holds a valid token
        const float alpha = fast_exp2(m_run - m_new);
        float psum = 0.f;
        bf16x8_t pop;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const float pv = fast_exp2(x[j] - m_new);
            psum += pv;
            pop[j] = (__bf16)pv;
        }
        l_run = l_run * alpha + psum;
        m_run = m_new;
#pragma unroll
        for (int db = 0; db < 8; ++db) oacc[db] *= alpha;

        // V^T as the A operand: lane holds V[token(slot)][16*db + l16] for the
        // 8 slots of group g4: tokens 4*g4 + {0..3} and 16 + 4*g4 + {0..3},
        // the same tokens whose P this lane already holds.  Two transposed
        // reads (ds_read_b64_tr_b16) per column block: source lane l16 of the
        // group points at row 4*g4 + l16/4 (+16), columns 16*db + 4*(l16%4) .. +3.
        const __bf16* vsrc = vl + (4 * g4 + (l16 >> 2)) * kDecRowStride + 4 * (l16 & 3);
#pragma unroll
        for (int db = 0; db < 8; ++db) {
            const bf16x4_t lo = lds_read_tr16(vsrc + db * 16);
            const bf16x4_t hi = lds_read_tr16(vsrc + 16 * kDecRowStride + db * 16);
            oacc[db] = mfma16(__builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7), pop, oacc[db]);
        }

        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    }

    l_run = xor_sum(xor_sum(l_run, 16), 32);

    // Merge the 4 waves in LDS (reusing the staging area).
    __syncthreads();
    float* ow = reinterpret_cast<float*>(smem);        // [wave][16][128]
    float* mlw = ow + kDecWaves * 16 * kHeadDim;       // [wave][16][2]
#pragma unroll
    for (int db = 0; db < 8; ++db)
#pragma unroll
        for (int i = 0; i < 4; ++i) ow[(wave * 16 + l16) * kHeadDim + db * 16 + g4 * 4 + i] = oacc[db][i];
    if (g4 == 0) {
        mlw[(wave * 16 + l16) * 2 + 0] = m_run;
        mlw[(wave * 16 + l16) * 2 + 1] = l_run;
    }
    __syncthreads();

    const int h = tid >> 4;
    const int d0 = (tid & 15) * 8;
    if (h >= p.group) return;
    float mw[kDecWaves];
    float M = -INFINITY;
#pragma unroll
    for (int w = 0; w < kDecWaves; ++w) {
        mw[w] = mlw[(w * 16 + h) * 2];
        M = fmaxf(M, mw[w]);
    }
    float L = 0.f;
    float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int w = 0; w < kDecWaves; ++w) {
        const float c = (mw[w] == -INFINITY) ? 0.f : fast_exp2(mw[w] - M);
        L += c * mlw[(w * 16 + h) * 2 + 1];
        const float* src = ow + (w * 16 + h) * kHeadDim + d0;
#pragma unroll
        for (int j = 0; j < 8; ++j) acc[j] += c * src[j];
    }
    const int qh = kvh * p.group + h;
    if (p.nsplit == 1) {
        const float inv = p.v_scale / L;
        bf16x8_t out;
#pragma unroll
        for (int j = 0; j < 8; ++j) out[j] = (__bf16)(acc[j] * inv);
        *reinterpret_cast<bf16x8_t*>(p.o + b * p.o_sb + qh * p.o_sh + d0) = out;
        if (p.lse != nullptr && (tid & 15) == 0) p.lse[(int64_t)b * p.hq + qh] = M * kLn2 + logf(L);
    } else {
        const int64_t slot = (((int64_t)b * p.hkv + kvh) * p.nsplit + split) * p.group + h;
        float* po = p.part_o + slot * kHeadDim + d0;
        const float vs = p.v_scale;
        *reinterpret_cast<f32x4_t*>(po) = f32x4_t{acc[0] * vs, acc[1] * vs, acc[2] * vs, acc[3] * vs};
        *reinterpret_cast<f32x4_t*>(po + 4) = f32x4_t{acc[4] * vs, acc[5] * vs, acc[6] * vs, acc[7] * vs};
        if ((tid & 15) == 0) {
            p.part_ml[slot * 2 + 0] = M;
            p.part_ml[slot * 2 + 1] = L;
        }
    }
}

// Pass 1 over the full (split, kv head, batch) grid.  kPair (an even number
// of kv heads): 8-wave workgroups over (split, kv head pair, batch), waves 0-3
// on kv head 2j and waves 4-7 on kv head 2j + 1, so that the two 256-byte
// pieces of a token's cache row that lie side by side are read together (at
// 480 four-wave workgroups 159.5 us, 240 eight-wave ones
// 145.4 us, outputs bit-identical).
template <bool kPair>
__global__ __launch_bounds__(kPair ? 2 * kDecThreads : kDecThreads) void decode_split_kernel(DecodeParams p) {
    __shared__ __attribute__((aligned(16))) unsigned char smem[(kPair ? 2 : 1) * kDecSmemBytes];
    const int half = kPair ? __builtin_amdgcn_readfirstlane((int)(threadIdx.x / kDecThreads)) : 0;
    dec_item<kKvContig>(p, smem + half * kDecSmemBytes, blockIdx.x, kPair ? 2 * (int)blockIdx.y + half : blockIdx.y,
                        blockIdx.z, (int)threadIdx.x - half * kDecThreads);
}

// Ragged batches: build the work list of non-empty splits, full-length splits
// first and the partial last split of each sequence after them, longest first
// (batch order beyond kPlanSortMax sequences), so that equal work fills the
// GPU and the short items form the tail.  One workgroup; entry =
// (b << 16) | split, so batch < 2^15 and splits < 2^16 (checked on the host).
constexpr int kPlanThreads = 256;
constexpr int kPlanSortMax = 1024;   // remainders kept in LDS and length-sorted up to this batch size

// Exclusive prefix sum of one int per thread over the workgroup (256 threads).
__device__ __forceinline__ int block_exclusive_scan(int v, int* s_wave, int* total) {
    const int lane = threadIdx.x & (kWave - 1);
    const int wave = threadIdx.x / kWave;
    int incl = v;
#pragma unroll
    for (int d = 1; d < kWave; d <<= 1) {
        const int t = __shfl_up(incl, d, kWave);
        if (lane >= d) incl += t;
    }
    if (lane == kWave - 1) s_wave[wave] = incl;
    __syncthreads();
    int base = 0, all = 0;
#pragma unroll
    for (int w = 0; w < kPlanThreads / kWave; ++w) {
        base += (w < wave) ? s_wave[w] : 0;
        all += s_wave[w];
    }
    __syncthreads();   // s_wave is reused by the next scan
    *total = all;
    return base + incl - v;
}

__global__ __launch_bounds__(kPlanThreads) void decode_plan_kernel(DecodeParams p, int32_t* work) {
    __shared__ int s_wave[kPlanThreads / kWave];
    __shared__ int s_rem[kPlanSortMax];   // len % chunk per sequence (batch <= kPlanSortMax)
    const int tid = threadIdx.x;
    const bool sort = p.batch <= kPlanSortMax;
    // sequences b = tid, tid + 256, ... belong to this thread
    int nf = 0, np = 0;
    for (int b = tid; b < p.batch; b += kPlanThreads) {
        const int len = clamp_len(p, b);
        nf += len / p.chunk;
        np += (len % p.chunk) != 0;
        if (sort) s_rem[b] = len % p.chunk;
    }
    int n_full, n_part;
    int pos_f = block_exclusive_scan(nf, s_wave, &n_full);
    int pos_p = block_exclusive_scan(np, s_wave, &n_part);   // also publishes s_rem (barriers inside)
    if (tid == 0) work[0] = n_full + n_part;
    for (int b = tid; b < p.batch; b += kPlanThreads) {
        const int len = clamp_len(p, b);
        const int full = len / p.chunk;
        for (int sp = 0; sp < full; ++sp) work[1 + pos_f + sp] = (b << 16) | sp;
        pos_f += full;
        const int rem = len % p.chunk;
        if (rem == 0) continue;
        int rank = pos_p;   // batch order
        if (sort) {
            rank = 0;       // longest remainder first, ties by batch
            for (int o = 0; o < p.batch; ++o) {
                const int ro = s_rem[o];
                rank += (ro > rem) || (ro == rem && o < b);
            }
        }
        work[1 + n_full + rank] = (b << 16) | full;
        ++pos_p;
    }
    // Without a combine pass, empty sequences (no list entry) still need
    // O = 0 and lse = -inf.
    if (p.nsplit == 1) {
        for (int b = 0; b < p.batch; ++b) {
            if (clamp_len(p, b) != 0) continue;
            for (int i = tid; i < p.hq * 16; i += kPlanThreads) {
                const int qh = i >> 4;
                bf16x8_t z;
#pragma unroll
                for (int j = 0; j < 8; ++j) z[j] = (__bf16)0.f;
                *reinterpret_cast<bf16x8_t*>(p.o + b * p.o_sb + qh * p.o_sh + (i & 15) * 8) = z;
                if (p.lse != nullptr && (i & 15) == 0) p.lse[(int64_t)b * p.hq + qh] = -INFINITY;
            }
        }
    }
}

// Pass 1 over the ragged work list: a fixed grid walks the entries, each
// entry once per kv head (kv head fastest, so heads of one split run together).
// kPair (an even number of kv heads): 8-wave workgroups, waves 0-3 on kv head
// 2j and waves 4-7 on kv head 2j + 1 of the same split.  Each half reads its
// own head's rows, but the two halves' loads of one token arrive together, so
// the 2 x 128-byte (fp8) or 2 x 256-byte (bf16) pieces of a cache row that lie
// side by side in memory are read at the same time: a streaming read of
// config 3's fp8 page pattern ran at 5.84 TB/s with one head per workgroup and
// 6.45 TB/s with head pairs.  Both halves of a workgroup hold the same split
// of the same sequence, so they pass the same workgroup barriers.
template <int kKv, int kSeg = 0, bool kPair = false>
__global__ __launch_bounds__(kPair ? 2 * kDecThreads : kDecThreads) void decode_list_kernel(DecodeParams p) {
    __shared__ __attribute__((aligned(16))) unsigned char smem[(kPair ? 2 : 1) * kDecSmemBytes];
    // wave-uniform (readfirstlane), so the buffer resources built from the
    // head stay scalar
    const int half = kPair ? __builtin_amdgcn_readfirstlane((int)(threadIdx.x / kDecThreads)) : 0;
    const int per_entry = kPair ? p.hkv / 2 : p.hkv;
    const int total = p.work[0] * per_entry;
    for (int item = blockIdx.x; item < total; item += gridDim.x) {
        const int e = p.work[1 + item / per_entry];
        const int kvh = kPair ? 2 * (item % per_entry) + half : item % per_entry;
        __syncthreads();   // the previous item's merge buffers alias the staging area
        dec_item<kKv, kSeg>(p, smem + half * kDecSmemBytes, e & 0xffff, kvh, e >> 16,
                            (int)threadIdx.x - half * kDecThreads);
    }
}

// Launches pass 1 over the work list: the head-pair form (one 8-wave
// workgroup per CU) when the kv heads pair up, else two 4-wave workgroups per
// CU.  Persistent: the grid never exceeds what the CUs hold at once.
template <int kKv, int kSeg>
static void launch_list(const DecodeParams& p, int nsplit, int cus, hipStream_t s) {
    const bool pair = (p.hkv % 2) == 0;
    const int64_t items = (int64_t)p.batch * nsplit * (pair ? p.hkv / 2 : p.hkv);   // most the list can hold
    const int64_t slots = (int64_t)(pair ? 1 : 2) * cus;
    const int grid = (int)(items < slots ? items : slots);
    if (pair)
        hipLaunchKernelGGL((decode_list_kernel<kKv, kSeg, true>), dim3(grid), dim3(2 * kDecThreads), 0, s, p);
    else
        hipLaunchKernelGGL((decode_list_kernel<kKv, kSeg, false>), dim3(grid), dim3(kDecThreads), 0, s, p);
}

// Log-sum-exp merge of the per-split partials of one (kv head, batch).
__global__ __launch_bounds__(kDecThreads) void decode_combine_kernel(DecodeParams p) {
    const int kvh = blockIdx.x;
    const int b = blockIdx.y;
    const int tid = threadIdx.x;
    const int h = tid >> 4;
    const int d0 = (tid & 15) * 8;
    if (h >= p.group) return;
    const int len = clamp_len(p, b);
    const int nvalid = (len + p.chunk - 1) / p.chunk;
    const int qh = kvh * p.group + h;
    __bf16* orow = p.o + b * p.o_sb + qh * p.o_sh + d0;
    if (nvalid == 0) {
        bf16x8_t z;
#pragma unroll
        for (int j = 0; j < 8; ++j) z[j] = (__bf16)0.f;
        *reinterpret_cast<bf16x8_t*>(orow) = z;
        if (p.lse != nullptr && (tid & 15) == 0) p.lse[(int64_t)b * p.hq + qh] = -INFINITY;
        return;
    }
    const int64_t base = ((int64_t)b * p.hkv + kvh) * p.nsplit;
    // Splits in batches of kCombineBatch whose loads are all issued before any
    // is used (slots past the last valid split re-read it and are masked), so
    // a batch costs one memory round trip; the sums run in split order.
    constexpr int kCombineBatch = 8;
    float M = -INFINITY;
    for (int s0 = 0; s0 < nvalid; s0 += kCombineBatch) {
        float mv[kCombineBatch];
#pragma unroll
        for (int i = 0; i < kCombineBatch; ++i)
            mv[i] = p.part_ml[((base + min(s0 + i, nvalid - 1)) * p.group + h) * 2];
#pragma unroll
        for (int i = 0; i < kCombineBatch; ++i) M = fmaxf(M, mv[i]);
    }
    float L = 0.f;
    float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    for (int s0 = 0; s0 < nvalid; s0 += kCombineBatch) {
        float ms[kCombineBatch], ls[kCombineBatch];
        f32x4_t a[kCombineBatch], bb[kCombineBatch];
#pragma unroll
        for (int i = 0; i < kCombineBatch; ++i) {
            const int64_t slot = (base + min(s0 + i, nvalid - 1)) * p.group + h;
            ms[i] = p.part_ml[slot * 2];
            ls[i] = p.part_ml[slot * 2 + 1];
            a[i] = *reinterpret_cast<const f32x4_t*>(p.part_o + slot * kHeadDim + d0);
            bb[i] = *reinterpret_cast<const f32x4_t*>(p.part_o + slot * kHeadDim + d0 + 4);
        }
        // selects, not a branch, so the loads above stay ahead of every use
#pragma unroll
        for (int i = 0; i < kCombineBatch; ++i) {
            const bool valid = s0 + i < nvalid;
            const float c = (ms[i] == -INFINITY) ? 0.f : fast_exp2(ms[i] - M);
            L = valid ? L + c * ls[i] : L;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                acc[j] = valid ? acc[j] + c * a[i][j] : acc[j];
                acc[4 + j] = valid ? acc[4 + j] + c * bb[i][j] : acc[4 + j];
            }
        }
    }
    const float inv = 1.f / L;
    bf16x8_t out;
#pragma unroll
    for (int j = 0; j < 8; ++j) out[j] = (__bf16)(acc[j] * inv);
    *reinterpret_cast<bf16x8_t*>(orow) = out;
    if (p.lse != nullptr && (tid & 15) == 0) p.lse[(int64_t)b * p.hq + qh] = M * kLn2 + logf(L);
}

// One pass of the 4 decode waves covers the planner's split rounding.
static_assert(kDecWaves * kDecStep == plan::kDecodeStepRound, "decode split rounding");

namespace {
using plan::DecodePlan;
using plan::DecodeShape;

// The split plan of a validated call on the current device.
int plan_on_device(const DecodeShape& shape, DecodePlan* pl) {
    const int cus = plan::decode_needs_cus(shape) ? device_cu_count() : 0;
    return plan::plan_decode(shape, cus, pl);
}
}  // namespace
}  // namespace fgqa

using namespace fgqa;

extern "C" int fgqa_decode_workspace_bytes(const fgqa_decode_args* a, size_t* bytes) {
    if (bytes == nullptr) return FGQA_ERR_INVALID_ARGUMENT;
    int st = plan::validate_decode(a);
    if (st != FGQA_OK) return st;
    DecodePlan plan;
    st = plan_on_device(plan::decode_shape(a), &plan);
    if (st != FGQA_OK) return st;
    *bytes = plan.ws_bytes;
    return FGQA_OK;
}

// Device scratch of fgqa_decode_bf16_noalloc: the split partials and the
// ragged work list of one call (FGQA_DECODE_NOALLOC_SCRATCH_BYTES, held by
// every device the library runs on until the process ends).  In host code the
// name `scratch` is a host-side stand-in, not a device address: the address is
// looked up once per device (hipGetSymbolAddress, with that device current)
// and only that pointer is passed to kernels.
namespace fgqa {
namespace {
constexpr size_t kNoAllocScratchBytes = FGQA_DECODE_NOALLOC_SCRATCH_BYTES;
static __device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];
constexpr int kScratchDevices = 64;
std::mutex g_scratch_mutex;
void* g_scratch_ptr[kScratchDevices] = {nullptr};

// The current device's copy of `scratch` (its address is looked up on the
// first call on that device).  Returns nullptr and sets *status on failure.
void* noalloc_scratch(int* status) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kScratchDevices) {
        *status = FGQA_ERR_HIP;
        return nullptr;
    }
    std::lock_guard<std::mutex> lock(g_scratch_mutex);
    if (g_scratch_ptr[dev] == nullptr) {
        void* ptr = nullptr;
        if (hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)) != hipSuccess || ptr == nullptr) {
            *status = FGQA_ERR_HIP;
            return nullptr;
        }
        g_scratch_ptr[dev] = ptr;
    }
    *status = FGQA_OK;
    return g_scratch_ptr[dev];
}

// The decode call; `noalloc`: the workspace is the device scratch above
// (the caller passes none), never the caller's or the library's buffer.
int decode_run(const fgqa_decode_args* a, void* stream, bool noalloc) {
    int st = plan::validate_decode(a);
    if (st != FGQA_OK) return st;
    st = plan::validate_decode_pointers(a);
    if (st != FGQA_OK) return st;
    if (a->batch == 0) return FGQA_OK;
    DecodePlan plan;
    st = plan_on_device(plan::decode_shape(a), &plan);
    if (st != FGQA_OK) return st;

    DecodeParams p;
    p.block_table = nullptr;
    p.bt_stride = 0;
    p.page_shift = 0;
    p.num_pages = 0;
    p.v_scale = 1.f;
    p.q = static_cast<const __bf16*>(a->q);
    p.k = static_cast<const __bf16*>(a->k);
    p.v = static_cast<const __bf16*>(a->v);
    p.o = static_cast<__bf16*>(a->o);
    p.lse = a->lse;
    p.seqlens = a->seqlens;
    p.part_o = nullptr;
    p.part_ml = nullptr;
    p.q_sb = a->q_stride[0];
    p.q_sh = a->q_stride[1];
    p.k_sb = a->k_stride[0];
    p.k_ss = a->k_stride[1];
    p.k_sh = a->k_stride[2];
    p.v_sb = a->v_stride[0];
    p.v_ss = a->v_stride[1];
    p.v_sh = a->v_stride[2];
    p.o_sb = a->o_stride[0];
    p.o_sh = a->o_stride[1];
    p.batch = a->batch;
    p.max_seqlen = a->max_seqlen;
    p.hq = a->num_q_heads;
    p.hkv = a->num_kv_heads;
    p.group = a->num_q_heads / a->num_kv_heads;
    p.nsplit = plan.nsplit;
    p.chunk = plan.chunk;
    p.scale_log2 = a->scale * kLog2e;

    int32_t* work = nullptr;
    std::unique_lock<std::mutex> ws_lock;   // held through the launches when the library's buffer is used
    if (plan.ws_bytes > 0) {
        void* ws = a->workspace;
        if (noalloc) {
            // the partials and the list are written before they are read, so
            // the previous call's contents need no clearing
            if (plan.ws_bytes > kNoAllocScratchBytes) return FGQA_ERR_WORKSPACE;
            ws = noalloc_scratch(&st);
            if (ws == nullptr) return st;
        } else if (ws == nullptr && a->workspace_bytes == 0) {
            ws_lock = workspace_lock();
            ws = internal_workspace(plan.ws_bytes, &st);
            if (st != FGQA_OK) return st;
        } else if (ws == nullptr || a->workspace_bytes < plan.ws_bytes) {
            return FGQA_ERR_WORKSPACE;
        } else if (!aligned16(ws)) {
            return FGQA_ERR_UNSUPPORTED;
        }
        char* w = static_cast<char*>(ws);
        if (plan.nsplit > 1) {
            p.part_o = reinterpret_cast<float*>(w);
            p.part_ml = reinterpret_cast<float*>(w + plan.part_o_bytes);
        }
        if (plan.list) work = reinterpret_cast<int32_t*>(w + plan.part_o_bytes + plan.part_ml_bytes);
    }
    p.work = work;

    hipStream_t s = static_cast<hipStream_t>(stream);
    if (a->max_seqlen == 0) {
        // Every sequence is empty: the combine writes O = 0, lse = -inf.
        p.nsplit = 1;
        hipLaunchKernelGGL(decode_combine_kernel, dim3(p.hkv, p.batch), dim3(kDecThreads), 0, s, p);
    } else if (plan.list) {
        const int cus = device_cu_count();
        if (cus <= 0) return FGQA_ERR_HIP;
        hipLaunchKernelGGL(decode_plan_kernel, dim3(1), dim3(kPlanThreads), 0, s, p, work);
        launch_list<kKvContig, 0>(p, plan.nsplit, cus, s);
        if (plan.nsplit > 1)
            hipLaunchKernelGGL(decode_combine_kernel, dim3(p.hkv, p.batch), dim3(kDecThreads), 0, s, p);
    } else {
        // Head pairs once the grid holds at least one item per CU; smaller
        // grids are latency-bound and keep one item per workgroup (BASELINE
        // config 1's 16 items: 9.9 us paired, 9.4 us not).
        const int cus = device_cu_count();
        if (cus <= 0) return FGQA_ERR_HIP;
        const bool pair = p.hkv % 2 == 0 && (int64_t)p.nsplit * p.hkv * p.batch >= cus;
        if (pair)
            hipLaunchKernelGGL(decode_split_kernel<true>, dim3(p.nsplit, p.hkv / 2, p.batch), dim3(2 * kDecThreads), 0,
                               s, p);
        else
            hipLaunchKernelGGL(decode_split_kernel<false>, dim3(p.nsplit, p.hkv, p.batch), dim3(kDecThreads), 0, s, p);
        if (plan.nsplit > 1)
            hipLaunchKernelGGL(decode_combine_kernel, dim3(p.hkv, p.batch), dim3(kDecThreads), 0, s, p);
    }
    if (hipGetLastError() != hipSuccess) return FGQA_ERR_HIP;
    return FGQA_OK;
}

}  // namespace
}  // namespace fgqa

extern "C" int fgqa_decode_bf16(const fgqa_decode_args* a, void* stream) { return decode_run(a, stream, false); }

extern "C" int fgqa_decode_bf16_noalloc(const fgqa_decode_args* a, void* stream) {
    if (a != nullptr && (a->workspace != nullptr || a->workspace_bytes != 0)) return FGQA_ERR_INVALID_ARGUMENT;
    return decode_run(a, stream, true);
}

// ---------------------------------------------------------------- paged KV cache
extern "C" int fgqa_decode_paged_workspace_bytes(const fgqa_decode_paged_args* a, size_t* bytes) {
    if (bytes == nullptr) return FGQA_ERR_INVALID_ARGUMENT;
    int st = plan::validate_paged(a);
    if (st != FGQA_OK) return st;
    DecodePlan plan;
    st = plan::plan_paged(a, &plan);
    if (st != FGQA_OK) return st;
    *bytes = plan.ws_bytes;
    return FGQA_OK;
}

extern "C" int fgqa_decode_paged(const fgqa_decode_paged_args* a, void* stream) {
    int st = plan::validate_paged(a);
    if (st != FGQA_OK) return st;
    st = plan::validate_paged_pointers(a);
    if (st != FGQA_OK) return st;
    if (a->batch == 0) return FGQA_OK;
    DecodePlan plan;
    st = plan::plan_paged(a, &plan);
    if (st != FGQA_OK) return st;

    DecodeParams p;
    p.q = static_cast<const __bf16*>(a->q);
    p.k = static_cast<const __bf16*>(a->k_cache);
    p.v = static_cast<const __bf16*>(a->v_cache);
    p.o = static_cast<__bf16*>(a->o);
    p.lse = a->lse;
    p.seqlens = a->seqlens;
    p.part_o = nullptr;
    p.part_ml = nullptr;
    p.q_sb = a->q_stride[0];
    p.q_sh = a->q_stride[1];
    p.k_sb = a->k_stride[0];
    p.k_ss = a->k_stride[1];
    p.k_sh = a->k_stride[2];
    p.v_sb = a->v_stride[0];
    p.v_ss = a->v_stride[1];
    p.v_sh = a->v_stride[2];
    p.o_sb = a->o_stride[0];
    p.o_sh = a->o_stride[1];
    p.batch = a->batch;
    p.max_seqlen = a->max_seqlen;
    p.hq = a->num_q_heads;
    p.hkv = a->num_kv_heads;
    p.group = a->num_q_heads / a->num_kv_heads;
    p.nsplit = plan.nsplit;
    p.chunk = plan.chunk;
    p.scale_log2 = a->scale * a->k_scale * kLog2e;
    p.block_table = a->block_table;
    p.bt_stride = a->block_table_stride;
    int shift = 0;
    while ((1 << shift) < a->page_size) ++shift;
    p.page_shift = shift;
    p.num_pages = a->num_pages;
    p.v_scale = a->v_scale;

    int32_t* work = nullptr;
    std::unique_lock<std::mutex> ws_lock;   // held through the launches when the library's buffer is used
    if (plan.ws_bytes > 0) {
        void* ws = a->workspace;
        if (ws == nullptr && a->workspace_bytes == 0) {
            ws_lock = workspace_lock();
            ws = internal_workspace(plan.ws_bytes, &st);
            if (st != FGQA_OK) return st;
        } else if (ws == nullptr || a->workspace_bytes < plan.ws_bytes) {
            return FGQA_ERR_WORKSPACE;
        } else if (!aligned16(ws)) {
            return FGQA_ERR_UNSUPPORTED;
        }
        char* w = static_cast<char*>(ws);
        if (plan.nsplit > 1) {
            p.part_o = reinterpret_cast<float*>(w);
            p.part_ml = reinterpret_cast<float*>(w + plan.part_o_bytes);
        }
        if (plan.list) work = reinterpret_cast<int32_t*>(w + plan.part_o_bytes + plan.part_ml_bytes);
    }
    p.work = work;

    hipStream_t s = static_cast<hipStream_t>(stream);
    if (a->max_seqlen == 0) {
        p.nsplit = 1;
        hipLaunchKernelGGL(decode_combine_kernel, dim3(p.hkv, p.batch), dim3(kDecThreads), 0, s, p);
    } else {
        const int cus = device_cu_count();
        if (cus <= 0) return FGQA_ERR_HIP;
        hipLaunchKernelGGL(decode_plan_kernel, dim3(1), dim3(kPlanThreads), 0, s, p, work);
        // Pages of at least one load instruction's rows (4 bf16, 8 fp8) whose
        // bytes stay below 2^31: page segments of min(page, 32) rows, each
        // read through one buffer resource (at BASELINE config 3's lengths
        // with 16- and 64-token pages: bf16 -4 %, fp8 with head pairs -1 to
        // -2 % against the per-row form).
        const bool fp8 = a->kv_dtype == FGQA_KV_FP8_E4M3;
        const bool small_pages = (int64_t)a->page_size * a->k_stride[1] * 2 < ((int64_t)1 << 31) &&
                                 (int64_t)a->page_size * a->v_stride[1] * 2 < ((int64_t)1 << 31);
        const int seg = !small_pages ? 0 : a->page_size >= 32 ? 32 : a->page_size >= 4 ? a->page_size : 0;
        if (fp8) {
            switch (seg >= 8 ? seg : 0) {
                case 32: launch_list<kKvPagedFp8, 32>(p, plan.nsplit, cus, s); break;
                case 16: launch_list<kKvPagedFp8, 16>(p, plan.nsplit, cus, s); break;
                case 8: launch_list<kKvPagedFp8, 8>(p, plan.nsplit, cus, s); break;
                default: launch_list<kKvPagedFp8, 0>(p, plan.nsplit, cus, s); break;
            }
        } else {
            switch (seg) {
                case 32: launch_list<kKvPagedBf16, 32>(p, plan.nsplit, cus, s); break;
                case 16: launch_list<kKvPagedBf16, 16>(p, plan.nsplit, cus, s); break;
                case 8: launch_list<kKvPagedBf16, 8>(p, plan.nsplit, cus, s); break;
                case 4: launch_list<kKvPagedBf16, 4>(p, plan.nsplit, cus, s); break;
                default: launch_list<kKvPagedBf16, 0>(p, plan.nsplit, cus, s); break;
            }
        }
        if (plan.nsplit > 1)
            hipLaunchKernelGGL(decode_combine_kernel, dim3(p.hkv, p.batch), dim3(kDecThreads), 0, s, p);
    }
    if (hipGetLastError() != hipSuccess) return FGQA_ERR_HIP;
    return FGQA_OK;
}
