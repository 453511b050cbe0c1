// Causal (or full) GQA prefill forward for gfx950 with 64 query rows per wave.
//
// Same maths as the other prefill kernels and the reference's Triton
// flash_gqa_forward_bf16_kernel (src/python/Triton/flash_gqa_kernel.py:15-138):
// S = Q.K^T*scale in fp32, top-left causal mask (:113-117), online softmax,
// P rounded to bf16 before P.V with the row sum kept from the fp32 P
// (:122-129), O /= row sum and lse = max + log(row sum) (:131-138).
//
// Work unit: 256 query rows (up to 8 heads of one KV group x 256/heads
// positions) on one workgroup of 4 waves, one wave per SIMD.  Each wave owns
// 64 rows as two 32-row halves, so every K or V operand it reads from LDS
// feeds two v_mfma_f32_32x32x16_bf16 (one per half): half the LDS operand
// bytes per MFMA of the 32-row-per-wave kernels.  Per 64-key tile j a wave
// runs two phases, each a single instruction stream of 32 MFMAs with the
// softmax of one half interleaved:
//   phase A: S(j+1) = K(j+1).Q^T for both halves     || exp2, sums, bf16 P of half 1, tile j
//   phase B: O += V(j).P(j) for both halves          || exp2, sums, bf16 P of half 0, tile j+1
// so each half's softmax overlaps the other's MFMAs, as two waves of a SIMD
// would, with the operand reuse of one.  The registers this needs (O: 128,
// Q: 64, S: up to 96, P: 48 per lane) exceed 256, so O and Q live in AGPRs:
// Q is only ever an MFMA source, and O is only written by MFMAs (inline asm
// with AGPR accumulators) and read at the end or on a rare rescale.  S and P
// stay in VGPRs (this file is compiled with MFMAs in their VGPR form).
//
// The running max moves (and O is rescaled) only when a lane's share of a
// tile's row sum, computed against the current max, passes 2^16 or a row has
// no max yet; P then stays below 2^16 and O far inside fp32 range.
//
// Two grids:
//   prefill_tall_pairs_kernel       unit pairs (heaviest with lightest) on two
//                                   workgroups of one XCD, the heavy unit's
//                                   KV range split between them and merged
//                                   through device memory (grids whose pairs
//                                   fill the CUs);
//   prefill_tall_persistent_kernel  whole units, one workgroup per CU, ranks
//                                   in snake order (larger grids).
#include <math.h>
#include <stdint.h>

#include "fgqa_device.h"
#include "fgqa_internal.h"
#include "prefill_common.h"
#include "prefill_tall.h"

namespace fgqa {

namespace {

constexpr int kTlWaves = 4;
constexpr int kTlThreads = kTlWaves * kWave;
constexpr int kTlRowBytes = kHeadDim * 2;                     // one K, V, Q or O row
constexpr int kTlTileBytes = kPfTile * kTlRowBytes;           // 16 KB: one K or V tile
constexpr int kTlVBuf = 3 * kTlTileBytes;                     // K0, K1, K2, then V0, V1
constexpr int kTlStage = 5 * kTlTileBytes;                    // after the tile buffers
constexpr int kTlWaveStage = 64 * kTlRowBytes;                // 16 KB: a wave's 64 Q (later O) rows
constexpr int kTlWords = kTlStage + kTlWaves * kTlWaveStage;  // 3 words that broadcast counter reads
constexpr int kTlLaneFloats = 132;                            // partial per lane: 128 of O, 2 max, 2 sums
static_assert(kTlWaves * kTlLaneFloats * kWave == kPfPartFloats, "merge slot size");

}  // namespace

const int kTallSmemBytes = kTlWords + 16;

namespace {

// Fences the instruction order: nothing moves across it.
#define TL_FENCE() __builtin_amdgcn_sched_barrier(0)

// O^T += V^T . P^T on an accumulator held in AGPRs.  The compiler counts no
// wait states around inline asm, and its register allocator may copy the
// accumulators between AGPRs before or after any asm statement, so each MFMA
// waits 2 states first (a VALU write, such as such a copy, before an MFMA
// reads the register; the wave usually waits for the MFMA pipe then anyway),
// and each phase of them ends with o_drain.  A copy of an accumulator between
// two MFMAs of a phase would still need o_drain's wait states after the MFMA
// that wrote it: tests/test_tall_isa.py checks the built code for that.
__device__ __forceinline__ void mfma_o(f32x16_t& acc, bf16x8_t a, bf16x8_t b) {
    asm volatile("s_nop 1\n\tv_mfma_f32_32x32x16_bf16 %0, %1, %2, %0" : "+a"(acc) : "v"(a), "v"(b));
}
// 24 wait states after a phase's last mfma_o, before any VALU access to the
// accumulators (copies included).
__device__ __forceinline__ void o_drain(f32x16_t (&o)[2][4]) {
    asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7"
                 : "+a"(o[0][0]), "+a"(o[0][1]), "+a"(o[0][2]), "+a"(o[0][3]), "+a"(o[1][0]), "+a"(o[1][1]),
                   "+a"(o[1][2]), "+a"(o[1][3]));
}
// The hardware does not hold a VALU read of an MFMA result until the MFMA has
// written it, and the compiler counts no wait states across inline asm: the
// accumulators mfma_o wrote are read only after this.
__device__ __forceinline__ void o_settle(f32x16_t (&o)[4]) {
    asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7" : "+a"(o[0]), "+a"(o[1]), "+a"(o[2]), "+a"(o[3]));
}
// o *= alpha, one accumulator at a time (16 VGPRs of room instead of 64),
// each back in AGPRs with the wait states the next mfma_o needs after a VALU
// write.  Call after o_settle.
__device__ __forceinline__ void o_scale(f32x16_t (&o)[4], float alpha) {
#pragma unroll
    for (int db = 0; db < 4; ++db) {
        asm volatile("" : "+a"(o[db]));
        f32x16_t t = o[db];
        t *= alpha;
        o[db] = t;
        asm volatile("s_nop 3" : "+a"(o[db]));
    }
}

// buffer_load_dwordx4 ... lds: 16 bytes per lane straight into LDS at
// M0 + 16 * lane, M0 = base + kOff.  Inline asm, so that the compiler does not
// make later LDS reads wait for these writes; they are awaited explicitly
// before the barrier that publishes the tile.
template <int kOff>
__device__ __forceinline__ void tl_dma(uint32_t base, uint32_t voffset, uint32_t soffset, __amdgpu_buffer_rsrc_t rsrc) {
    asm volatile("s_add_u32 m0, %0, %4\n\tbuffer_load_dwordx4 %1, %2, %3 offen lds"
                 :: "s"(base), "v"(voffset), "s"(rsrc), "s"(soffset), "i"(kOff) : "memory", "scc");
}

// One segment (tiles [seg.lo, seg.hi) of the KV range) of 256-row unit
// (qb, hg, kvh, b).
__device__ __forceinline__ void tall_unit(const PrefillParams& p, unsigned char* smem, int qb, int hg, int kvh,
                                          int b, const PfSeg& seg) {
    const int tid = threadIdx.x;
    const int lane = tid & (kWave - 1);
    const int wave = __builtin_amdgcn_readfirstlane(tid / kWave);
    const int l32 = lane & 31;
    const int l16 = lane & 15;
    const int g2 = lane >> 5;
    const int qrows = 256 >> p.hb_log2;
    const int q_wg0 = qb * qrows;
    // half h of the wave: unit slot 2*wave + h, 32 rows of head hd[h] at positions q0[h]..+31
    int hd[2], q0[2];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        const int s = 2 * wave + h;
        hd[h] = kvh * p.group + hg * p.hb + (s & (p.hb - 1));
        q0[h] = q_wg0 + (s >> p.hb_log2) * 32;
    }
    int kv_end = p.skv;
    if (p.causal) kv_end = min(kv_end, min(q_wg0 + qrows, p.sq));
    const int t_first = seg.lo;
    const int n_tiles = seg.hi - seg.lo;
    const int kv_hi = min(kv_end, (t_first + n_tiles) * kPfTile);   // keys this segment may use

    const uint32_t qss = (uint32_t)(p.q_ss * 2);
    const uint32_t kss = (uint32_t)(p.k_ss * 2);
    const uint32_t vss = (uint32_t)(p.v_ss * 2);
    const int kv_last = p.skv > 0 ? p.skv - 1 : 0;
    const __bf16* kbase = p.k + b * p.k_sb + kvh * p.k_sh;
    const __bf16* vbase = p.v + b * p.v_sb + kvh * p.v_sh;
    const uint32_t lds_base = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) unsigned char*)smem;

    // Tile loads.  Instruction i of this wave fills the 1 KB at slot
    // 64*(wave + 4*i) of a tile; lane l writes slot 64*(wave + 4*i) + l.
    //   K: row r = slot / 16, chunk c of the row sits in slot c ^ (r % 16)
    //   V: row r = 4*(wave + 4*i) + lane/16, chunk c in slot c ^ 4*(r % 4)
    // so 16 rows read at one chunk (K, b128) and 4 rows x 4 chunks (V,
    // transposed b64) hit distinct banks.  The per-lane offsets are relative
    // to the tile's first row, and each tile gets a buffer resource that
    // starts there and ends at the last key: rows past it read as zeros
    // (their scores are masked, so they only need to be finite), and a tile
    // wholly past it reads nothing.
    uint32_t kvo[4], vvo[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int kr = 4 * (wave + 4 * i) + (lane >> 4);
        kvo[i] = (uint32_t)kr * kss + (uint32_t)((l16 ^ (kr & 15)) << 4);
        vvo[i] = (uint32_t)kr * vss + (uint32_t)((l16 ^ (4 * (kr & 3))) << 4);
    }
    auto tile_rsrc = [&](const __bf16* base, uint32_t ss, int j) {
        const int t0 = (t_first + j) * kPfTile;
        const int d = kv_last - t0;   // (the host bounds (skv + 128) * stride below 2^31 bytes)
        return make_rsrc(reinterpret_cast<const unsigned char*>(base) + (uint32_t)t0 * ss,
                         d >= 0 ? (uint32_t)d * ss + kTlRowBytes : 0u);
    };
    __amdgpu_buffer_rsrc_t krs_t, vrs_t;   // the next K and V tile loads
    // instruction i of tile krs_t into the K buffer at byte kbuf, of vrs_t
    // into V buffer vb (instruction i of wave w writes the 1 KB at
    // 1 KB * w + 4 KB * i of the tile)
    auto dma_k = [&](auto ic, uint32_t kbuf) {
        constexpr int i = decltype(ic)::value;
        tl_dma<4096 * i>(lds_base + kbuf + 1024 * wave, kvo[i], 0u, krs_t);
    };
    auto dma_v = [&](auto ic, auto vb) {
        constexpr int i = decltype(ic)::value;
        tl_dma<4096 * i>(lds_base + kTlVBuf + decltype(vb)::value * kTlTileBytes + 1024 * wave, vvo[i], 0u, vrs_t);
    };
    using C0 = std::integral_constant<int, 0>;
    using C1 = std::integral_constant<int, 1>;

    // K operand (tb, kk) of S^T = K.Q^T: rows 32*tb + l32, chunk 2*kk + g2.
    int koff[8];
#pragma unroll
    for (int kk = 0; kk < 8; ++kk) koff[kk] = l32 * kTlRowBytes + (((2 * kk + g2) ^ (l32 & 15)) << 4);
    // V^T operand (kb, db) through two transposed reads: lane i of a 16-lane
    // group supplies row 16*kb + 4*g2 + i/4 (+8), columns 32*db +
    // 16*((lane/16)%2) + 4*(i%4) .. +3: chunk 4*db + 2*((lane/16)%2) + (i%4)/2,
    // half i%2 of the swizzled row.
    int voff[4];
    {
        const int q4 = l16 >> 2;
        const int dh = (lane >> 4) & 1;
#pragma unroll
        for (int db = 0; db < 4; ++db)
            voff[db] = (4 * g2 + q4) * kTlRowBytes + ((4 * (db ^ q4) + 2 * dh + ((l16 >> 1) & 1)) << 4) + 8 * (l16 & 1);
    }

    // ---- prologue: Q rows and the first tiles -------------------------------
    // The wave's 64 Q rows go to its 16 KB stage area (half h at +8 KB * h,
    // row r at 256 * r, chunk c in slot c ^ (r % 16)), 4 whole rows per load.
    const uint32_t stage = lds_base + kTlStage + wave * kTlWaveStage;
    __syncthreads();   // the previous unit may still read the tiles and the stage area
    [[maybe_unused]] uint32_t my_xcc1 = 0;
    if (seg.part != nullptr) {
        uint32_t hw;
        asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(hw));
        my_xcc1 = (hw & 15u) + 1u;
        if (tid == 0) __hip_atomic_store(seg.ctr + 1 + seg.slot, my_xcc1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        const __amdgpu_buffer_rsrc_t qrs =
            make_rsrc(p.q + b * p.q_sb + hd[h] * p.q_sh, (uint32_t)(p.sq - 1) * qss + kTlRowBytes);
        static_for<8>([&](auto ic) {
            constexpr int i = decltype(ic)::value;
            const int slot = 64 * i + lane;
            const int r = slot >> 4;
            const uint32_t vo = (uint32_t)(q0[h] + r) * qss + ((uint32_t)((slot & 15) ^ (r & 15)) << 4);
            tl_dma<1024 * i>(stage + h * 8192, vo, 0u, qrs);
        });
    }
    // K(0..2) (tiles past the segment read as zeros or as keys it does not
    // use) and V(0)
    if (n_tiles > 0) {
#pragma unroll
        for (int t = 0; t < 3; ++t) {
            krs_t = tile_rsrc(kbase, kss, t);
            static_for<4>([&](auto ic) { dma_k(ic, (uint32_t)(t * kTlTileBytes)); });
        }
        vrs_t = tile_rsrc(vbase, vss, 0);
        static_for<4>([&](auto ic) { dma_v(ic, C0{}); });
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    bf16x8_t qop[2][8];
    {
        const unsigned char* ql = smem + kTlStage + wave * kTlWaveStage + l32 * kTlRowBytes;
#pragma unroll
        for (int h = 0; h < 2; ++h)
#pragma unroll
            for (int kk = 0; kk < 8; ++kk) {
                u32x4_t t = *reinterpret_cast<const u32x4_t*>(ql + h * 8192 + (((2 * kk + g2) ^ (l32 & 15)) << 4));
                t ^= p.q_sign;
                qop[h][kk] = as_bf16x8(t);
                asm volatile("" : "+a"(qop[h][kk]));   // Q lives in AGPRs
            }
    }

    const float c = p.scale_log2;
    float m_run[2] = {-INFINITY, -INFINITY};   // running max (log2 units) of this lane's row
    float m_use[2] = {0.f, 0.f};               // m_run, or 0 while m_run is -inf
    float l_run[2] = {0.f, 0.f};               // this lane's share of the row sum
    f32x16_t oacc[2][4];
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int db = 0; db < 4; ++db) {
#pragma unroll
            for (int i = 0; i < 16; ++i) oacc[h][db][i] = 0.f;
            asm volatile("" : "+a"(oacc[h][db]));
        }

    // Causal / tail mask of half h's S of tile j, in place (tiles that cross
    // the diagonal or the segment's last key only).
    auto mask = [&](f32x16_t (&s)[2], int h, int j) {
        const int kv0 = (t_first + j) * kPfTile;
        if ((kv0 + kPfTile > kv_hi) || (p.causal && kv0 + kPfTile - 1 > q0[h])) {
            const int row = q0[h] + l32;
            const int row_lim = p.causal ? min(row + 1, kv_hi) : kv_hi;
            const int lim = row_lim - (kv0 + g2 * 4);   // tokens at or past lim are masked
#pragma unroll
            for (int tb = 0; tb < 2; ++tb)
#pragma unroll
                for (int i = 0; i < 16; ++i)
                    if (tb * 32 + (i >> 2) * 8 + (i & 3) >= lim) s[tb][i] = -INFINITY;
        }
    };
    // exp2(S*scale - max) of elements 2*ch, 2*ch + 1 of the lane's 32 into
    // the bf16 P operands; ps[t]: sums of the 8 elements of operand t.  In
    // two halves (sm_lo: element 2*ch into *plo; sm_hi: element 2*ch + 1, the
    // sum and the bf16 pair), so each can follow one MFMA: the wave issues in
    // order, so the VALU work after an MFMA must fit the MFMA pipe's time for
    // the next one not to wait.
    auto sm_lo = [&](const f32x16_t (&s)[2], float* plo, float mu, int ch) {
        const int t = ch >> 2;
        const int e = (ch & 3) * 2;
        *plo = fast_exp2(__builtin_fmaf(s[t >> 1][(t & 1) * 8 + e], c, -mu));
    };
    auto sm_hi = [&](const f32x16_t (&s)[2], bf16x8_t (&pp)[4], float (&ps)[4], float plo, float mu, int ch) {
        const int t = ch >> 2;
        const int e = (ch & 3) * 2;
        const float p1 = fast_exp2(__builtin_fmaf(s[t >> 1][(t & 1) * 8 + e + 1], c, -mu));
        ps[t] = (e == 0) ? plo + p1 : ps[t] + (plo + p1);
        pp[t][e] = (__bf16)plo;
        pp[t][e + 1] = (__bf16)p1;
        // the operand is complete: convert here, not where phase B uses it
        if (e == 6) asm volatile("" : "+v"(pp[t]));
    };
    auto softmax_all = [&](const f32x16_t (&s)[2], bf16x8_t (&pp)[4], float mu) {
        float ps[4];
#pragma unroll
        for (int ch = 0; ch < 16; ++ch) {
            float plo;
            sm_lo(s, &plo, mu, ch);
            sm_hi(s, pp, ps, plo, mu, ch);
        }
        return (ps[0] + ps[1]) + (ps[2] + ps[3]);
    };
    // Slow path of half h after P was computed against the current max: the
    // row max of the tile, a move of the running max (rescaling O and the
    // sum) when some row's exceeds it by more than 2^8, and P again.
    // the row max of a half's S tile (log2 units), over both lanes of a row
    auto row_max = [&](const f32x16_t (&s)[2]) {
        float pm[4];
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            pm[t] = s[t >> 1][(t & 1) * 8];
#pragma unroll
            for (int i = 1; i < 8; ++i) pm[t] = fmaxf(pm[t], s[t >> 1][(t & 1) * 8 + i]);
        }
        return half_max(fmaxf(fmaxf(pm[0], pm[1]), fmaxf(pm[2], pm[3]))) * c;
    };
    auto slow = [&](const f32x16_t (&s)[2], bf16x8_t (&pp)[4], auto hc) -> float {
        constexpr int h = decltype(hc)::value;
        const float tmax = row_max(s);
        if (__builtin_amdgcn_ballot_w64(tmax > m_run[h] + 8.f) != 0) {
            const float m_new = fmaxf(m_run[h], tmax);
            const float m_new_use = (m_new == -INFINITY) ? 0.f : m_new;
            // 0 while the row had no max (O and the sum are still 0)
            const float alpha = (m_run[h] == -INFINITY) ? 0.f : fast_exp2(m_use[h] - m_new_use);
            l_run[h] *= alpha;
            if (__builtin_amdgcn_ballot_w64(m_run[h] != -INFINITY) != 0) {
                o_settle(oacc[h]);
                o_scale(oacc[h], alpha);
            }
            m_run[h] = m_new;
            m_use[h] = m_new_use;
        }
        return softmax_all(s, pp, m_use[h]);
    };
    auto need_slow = [&](int h, float lt) {
        return __builtin_amdgcn_ballot_w64(m_run[h] == -INFINITY || !(lt <= 65536.f)) != 0;
    };

    // operand i of the K tile at byte kbuf: (kk, tb) = (i / 2, i % 2);
    // operand i of V buffer vb: (kb, db) = (i / 4, i % 4)
    auto kfetch = [&](uint32_t kbuf, int i) -> bf16x8_t {
        return *reinterpret_cast<const bf16x8_t*>(smem + kbuf + (i & 1) * 32 * kTlRowBytes + koff[i >> 1]);
    };
    auto vfetch = [&](auto vb, int i) -> bf16x8_t {
        const unsigned char* base =
            smem + kTlVBuf + decltype(vb)::value * kTlTileBytes + 16 * (i >> 2) * kTlRowBytes + voff[i & 3];
        const bf16x4_t lo = lds_read_tr16(reinterpret_cast<const __bf16*>(base));
        const bf16x4_t hi = lds_read_tr16(reinterpret_cast<const __bf16*>(base + 8 * kTlRowBytes));
        return __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
    };

    bf16x8_t pop[2][4];    // P(j) operands of both halves
    f32x16_t s0[2], s1[2];  // S of half 0 (tile j+1 after phase A) and half 1 (tile j)
    // The operands of a wave's MFMAs come from LDS as one stream, each read
    // four MFMA pairs ahead into a ring of 4 registers, across the phases:
    // phase A's last groups read phase B's first V operands, phase B's last
    // groups the next phase A's first K operands (its tile is three buffers
    // deep, so it is in LDS before the barrier that ends the iteration).
    bf16x8_t ring[4];
    if (n_tiles > 0) {
        // S(0) of both halves, their row max, P of half 0
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const bf16x8_t ka = kfetch(0u, i);
            s0[i & 1] = mfma32(ka, qop[0][i >> 1], i < 2 ? f32x16_t{} : s0[i & 1]);
            s1[i & 1] = mfma32(ka, qop[1][i >> 1], i < 2 ? f32x16_t{} : s1[i & 1]);
        }
        mask(s0, 0, 0);
        mask(s1, 1, 0);
        m_run[0] = row_max(s0);
        m_run[1] = row_max(s1);
#pragma unroll
        for (int h = 0; h < 2; ++h) m_use[h] = (m_run[h] == -INFINITY) ? 0.f : m_run[h];
        float lt = softmax_all(s0, pop[0], m_use[0]);
        if (need_slow(0, lt)) lt = slow(s0, pop[0], C0{});
        l_run[0] += lt;
#pragma unroll
        for (int i = 0; i < 4; ++i) ring[i] = kfetch((uint32_t)kTlTileBytes, i);   // K(1)
    }
    __syncthreads();   // every wave has read K(0): iteration 0 refills its buffer
    // K buffers of iteration j: ka holds K(j+1) (phase A), kp K(j+2) (its
    // first operands read in phase B), kd receives K(j+3)
    uint32_t ka = kTlTileBytes, kp = 2 * kTlTileBytes, kd = 0;

    // ---- the tile loop ------------------------------------------------------
    // Iteration j (P = j & 1 a constant, so every V offset is an immediate):
    // on entry S_1(j) (masked) and P_0(j) are in registers, ring holds K(j+1)'s
    // first operands, K(j+1), K(j+2) and V(j) are in LDS; K(j+3) and V(j+1)
    // load during the iteration into the buffers iteration j-1 finished with.
    auto iter = [&](int j, auto par, auto full) {
        constexpr int P = decltype(par)::value;
        constexpr bool kFull = decltype(full)::value;   // false: the last tile (no S(j+1))
        using CP = std::integral_constant<int, P>;
        using CQ = std::integral_constant<int, 1 - P>;
        // (tiles past the segment load as zeros or as keys it does not use,
        // into buffers nothing reads again)
        if constexpr (kFull) {
            krs_t = tile_rsrc(kbase, kss, j + 3);
            vrs_t = tile_rsrc(vbase, vss, j + 1);
        }
        // phase A
        {
            float ps[4];
            if constexpr (kFull) {
                f32x16_t n0[2], n1[2];
                TL_FENCE();
                // per K operand: its MFMA for half 0, half of a softmax
                // chunk, its MFMA for half 1, the other half
                static_for<16>([&](auto ic) {
                    constexpr int i = decltype(ic)::value;
                    const bf16x8_t a = ring[i % 4];
                    float plo;
                    n0[i % 2] = mfma32(a, qop[0][i / 2], i < 2 ? f32x16_t{} : n0[i % 2]);
                    TL_FENCE();
                    sm_lo(s1, &plo, m_use[1], i);
                    if constexpr (i % 4 == 1) dma_k(std::integral_constant<int, i / 4>{}, kd);
                    TL_FENCE();
                    n1[i % 2] = mfma32(a, qop[1][i / 2], i < 2 ? f32x16_t{} : n1[i % 2]);
                    TL_FENCE();
                    ring[i % 4] = i + 4 < 16 ? kfetch(ka, i + 4) : vfetch(CP{}, i - 12);
                    sm_hi(s1, pop[1], ps, plo, m_use[1], i);
                    TL_FENCE();
                });
                float lt = (ps[0] + ps[1]) + (ps[2] + ps[3]);
                if (need_slow(1, lt)) lt = slow(s1, pop[1], C1{});
                l_run[1] += lt;
#pragma unroll
                for (int tb = 0; tb < 2; ++tb) {
                    s0[tb] = n0[tb];
                    s1[tb] = n1[tb];
                }
                mask(s0, 0, j + 1);
                mask(s1, 1, j + 1);
            } else {
                float lt = softmax_all(s1, pop[1], m_use[1]);
                if (need_slow(1, lt)) lt = slow(s1, pop[1], C1{});
                l_run[1] += lt;
#pragma unroll
                for (int i = 0; i < 4; ++i) ring[i] = vfetch(CP{}, i);
            }
        }
        // phase B
        {
            float ps[4];
            bf16x8_t pn[4];
            TL_FENCE();
            static_for<16>([&](auto ic) {
                constexpr int i = decltype(ic)::value;
                const bf16x8_t a = ring[i % 4];
                float plo;
                mfma_o(oacc[0][i % 4], a, pop[0][i / 4]);
                TL_FENCE();
                if constexpr (kFull) {
                    sm_lo(s0, &plo, m_use[0], i);
                    if constexpr (i % 4 == 1) dma_v(std::integral_constant<int, i / 4>{}, CQ{});
                }
                TL_FENCE();
                mfma_o(oacc[1][i % 4], a, pop[1][i / 4]);
                TL_FENCE();
                if constexpr (i + 4 < 16) ring[i % 4] = vfetch(CP{}, i + 4);
                else if constexpr (kFull) ring[i % 4] = kfetch(kp, i - 12);
                if constexpr (kFull) sm_hi(s0, pn, ps, plo, m_use[0], i);
                TL_FENCE();
            });
            o_drain(oacc);
            if constexpr (kFull) {
                float lt = (ps[0] + ps[1]) + (ps[2] + ps[3]);
                if (need_slow(0, lt)) lt = slow(s0, pn, C0{});
                l_run[0] += lt;
#pragma unroll
                for (int t = 0; t < 4; ++t) pop[0][t] = pn[t];
            }
        }
        if constexpr (kFull) {
            asm volatile("s_waitcnt vmcnt(0)" ::: "memory");   // this wave's K(j+3), V(j+1)
            __syncthreads();
            const uint32_t k0 = ka;
            ka = kp;
            kp = kd;
            kd = k0;
        }
    };
    {
        int j = 0;
        for (; j + 2 < n_tiles; j += 2) {
            iter(j, C0{}, std::true_type{});
            iter(j + 1, C1{}, std::true_type{});
        }
        if (j + 1 < n_tiles) {
            iter(j, C0{}, std::true_type{});
            ++j;
        }
        if (n_tiles > 0) {
            if (j & 1) iter(j, C1{}, std::false_type{});
            else iter(j, C0{}, std::false_type{});
        }
    }
    o_settle(oacc[0]);
    o_settle(oacc[1]);

    // ---- a split unit's two partial results ---------------------------------
    bool merging = false;
    if (seg.part != nullptr) {
        // The first of the unit's two segments to finish publishes its
        // partial (O, max, sum of every lane) in its slot and counts its
        // arrival; the second merges that with its own and writes the output.
        // A segment that finds no arrival publishes, and merges anyway if the
        // other one arrived meanwhile.  The merger sets the unit's words back
        // to 0 for the next launch.  Words of the unit: ctr[0] counts arrivals
        // as 1 + the publisher's XCD, ctr[1 + slot] holds 1 + the XCD of the
        // segment in that slot (written at its start).  Every wave waits for
        // its own partial stores (they are then in its XCD's L2: the L1 writes
        // through) before the barrier after which thread 0 counts the
        // arrival.  When the other segment runs on the same XCD (it does for
        // blocks w and w + 8) the two share that L2, the arrival is counted
        // with a relaxed atomic and the reader only invalidates its L1;
        // otherwise the count is a device-scope release and the reader's
        // waves acquire at device scope.
        unsigned* word = reinterpret_cast<unsigned*>(smem + kTlWords);
        const int woff = wave * kTlLaneFloats * kWave;
        float* own = seg.part + seg.slot * kPfPartFloats + woff;
        if (tid == 0) {
            word[0] = __hip_atomic_load(seg.ctr, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            word[1] = __hip_atomic_load(seg.ctr + 2 - seg.slot, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        __syncthreads();
        unsigned arrived = word[0];
        bool merge = arrived != 0u;
        if (!merge) {
            const bool near = word[1] == my_xcc1;   // the reader shares this XCD's L2
            f32x4_t* o4 = reinterpret_cast<f32x4_t*>(own) + lane;
#pragma unroll
            for (int h = 0; h < 2; ++h)
#pragma unroll
                for (int db = 0; db < 4; ++db)
#pragma unroll
                    for (int i4 = 0; i4 < 4; ++i4)
                        o4[(h * 16 + db * 4 + i4) * kWave] =
                            f32x4_t{oacc[h][db][4 * i4], oacc[h][db][4 * i4 + 1], oacc[h][db][4 * i4 + 2],
                                    oacc[h][db][4 * i4 + 3]};
            own[128 * kWave + lane] = m_run[0];
            own[129 * kWave + lane] = m_run[1];
            own[130 * kWave + lane] = l_run[0];
            own[131 * kWave + lane] = l_run[1];
            asm volatile("s_waitcnt vmcnt(0)" ::: "memory");   // this wave's partial is in L2
            __syncthreads();
            if (tid == 0)
                word[2] = near ? __hip_atomic_fetch_add(seg.ctr, my_xcc1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)
                               : __hip_atomic_fetch_add(seg.ctr, my_xcc1, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_AGENT);
            __syncthreads();
            arrived = word[2];
            merge = arrived != 0u;
            if (!merge) return;   // the other segment merges
        }
        // every wave acquires the other partial
        if (arrived == my_xcc1) asm volatile("buffer_inv sc0" ::: "memory");
        else __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
        if (tid == 0) {
            __hip_atomic_store(seg.ctr, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_store(seg.ctr + 1, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_store(seg.ctr + 2, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        merging = true;
    }

    // ---- epilogue: O / sum through the stage area, and the LSE --------------
    // (merging: each element is the two partials' sum, slot 0's term first
    // whichever segment merges, so the output does not depend on the order
    // of arrival.)  8-byte pieces into (row 32*h + l32, chunk 4*db + i4, half
    // g2), chunk c of row r in slot c ^ (r % 16); then whole 256-byte rows, 4
    // per store.
    unsigned char* ol = smem + kTlStage + wave * kTlWaveStage;
    auto stage_out = [&](auto mc) {
        constexpr bool kMerge = decltype(mc)::value;
        const bool first = seg.slot == 0;
        const float* other = kMerge ? seg.part + (1 - seg.slot) * kPfPartFloats + wave * kTlLaneFloats * kWave : nullptr;
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            float wa = 1.f, wb = 0.f;   // weights of slot 0's and slot 1's partial
            if constexpr (kMerge) {
                const float m_o = other[(128 + h) * kWave + lane];
                const float l_o = other[(130 + h) * kWave + lane];
                const float mA = first ? m_run[h] : m_o, lA = first ? l_run[h] : l_o;
                const float mB = first ? m_o : m_run[h], lB = first ? l_o : l_run[h];
                const float m = fmaxf(mA, mB);
                const float mu = (m == -INFINITY) ? 0.f : m;
                wa = (mA == -INFINITY) ? 0.f : fast_exp2(mA - mu);   // 0 when a segment saw no key
                wb = (mB == -INFINITY) ? 0.f : fast_exp2(mB - mu);
                l_run[h] = __builtin_fmaf(lA, wa, lB * wb);
                m_run[h] = m;
            }
            const float lsum = half_sum(l_run[h]);
            const float inv = (lsum > 0.f) ? 1.f / lsum : 0.f;
#pragma unroll
            for (int db = 0; db < 4; ++db)
#pragma unroll
                for (int i4 = 0; i4 < 4; ++i4) {
                    f32x4_t ot = {};
                    if constexpr (kMerge) ot = reinterpret_cast<const f32x4_t*>(other)[(h * 16 + db * 4 + i4) * kWave + lane];
                    bf16x4_t w;
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        float val = oacc[h][db][i4 * 4 + e];
                        if constexpr (kMerge) val = first ? __builtin_fmaf(val, wa, ot[e] * wb) : __builtin_fmaf(ot[e], wa, val * wb);
                        w[e] = (__bf16)(val * inv);
                    }
                    *reinterpret_cast<bf16x4_t*>(ol + (32 * h + l32) * kTlRowBytes + (((4 * db + i4) ^ (l32 & 15)) << 4) +
                                                 g2 * 8) = w;
                }
            const int row = q0[h] + l32;
            if (row < p.sq && p.lse != nullptr && g2 == 0)
                p.lse[((int64_t)b * p.hq + hd[h]) * p.sq + row] =
                    (lsum > 0.f) ? m_run[h] * kLn2 + logf(lsum) : -INFINITY;
        }
    };
    if (merging) stage_out(std::true_type{});
    else stage_out(std::false_type{});
    // this wave's LDS writes complete before its reads (no other wave uses the area)
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        const int r = 4 * i + (lane >> 4);   // row of the wave's 64: half r / 32, row r % 32
        const u32x4_t v = *reinterpret_cast<const u32x4_t*>(ol + r * kTlRowBytes + (l16 << 4));
        const int h = r >> 5;
        const int row = q0[h] + (r & 31);
        if (row < p.sq) {
            __bf16* orow = p.o + b * p.o_sb + (int64_t)row * p.o_ss + hd[h] * p.o_sh;
            *reinterpret_cast<u32x4_t*>(orow + ((l16 ^ (r & 15)) << 3)) = v;
        }
    }
}

// Pairs: blocks w and w + 8 of each 16 (one XCD) run unit pair
// pf_pair_of_block(w): ranks r (heavy) and units - 1 - r (light).  Role 0 runs
// the heavy unit's first `a` tiles, role 1 the rest of it and then the light
// unit; a = min(n_heavy, ceil((n_heavy + n_light + bias) / 2)), the bias
// paying for role 1's extra unit start.
__global__ __launch_bounds__(kTlThreads, 1) void prefill_tall_pairs_kernel(PrefillParams p0) {
    extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
    const int w = blockIdx.x;
    const int role = pf_role_of_block(w);
    const int pair = pf_pair_of_block(w);
    const int units = p0.n_qblocks * p0.n_streams;
    if (pair >= (units + 1) / 2) return;
#pragma nounroll
    for (int sgi = 0; sgi < 2; ++sgi) {
        const PrefillParams p = pf_params_reread(p0);
        const int qrows = 256 >> p.hb_log2;
        const int rh = pair, rl = units - 1 - pair;   // rl == rh: the middle unit of an odd count
        int qb, hg, kvh, b;
        pf_rank_unit(p, rh, &qb, &hg, &kvh, &b);
        const int nh = pf_unit_tiles(p, qb, qrows);
        int nl = 0;
        if (rl != rh) {
            int qb2, hg2, kvh2, b2;
            pf_rank_unit(p, rl, &qb2, &hg2, &kvh2, &b2);
            nl = pf_unit_tiles(p, qb2, qrows);
        }
        const int a = min(nh, (nh + nl + p.wide_bias + 1) >> 1);
        const bool split = a < nh;
        PfSeg seg{0, a, role, nullptr, p.wide_ctr + 4 * pair};
        if (role == 0) {
            if (sgi > 0) break;
            if (split) seg.part = p.wide_part + (size_t)pair * 2 * kPfPartFloats;
        } else if (sgi == 0) {
            if (!split) continue;
            seg.lo = a;
            seg.hi = nh;
            seg.part = p.wide_part + (size_t)pair * 2 * kPfPartFloats;
        } else {
            if (rl == rh) break;
            pf_rank_unit(p, rl, &qb, &hg, &kvh, &b);
            seg.lo = 0;
            seg.hi = nl;
        }
        tall_unit(p, smem, qb, hg, kvh, b, seg);
    }
}

// Whole units on a persistent grid: workgroup w runs ranks w, 2G-1-w, 2G+w,
// ... (G = gridDim.x) of the heaviest-first order, so each lap goes the other
// way and every CU's units add up to about the same number of tiles.
__global__ __launch_bounds__(kTlThreads, 1) void prefill_tall_persistent_kernel(PrefillParams p0) {
    extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
    const int units = p0.n_qblocks * p0.n_streams;
    const int g = gridDim.x;
    const int w = blockIdx.x;
#pragma nounroll
    for (int lap = 0;; ++lap) {
        const int r = (lap & 1) ? (lap + 1) * g - 1 - w : lap * g + w;
        if (r >= units) break;   // later laps hold only higher ranks
        const PrefillParams p = pf_params_reread(p0);
        int qb, hg, kvh, b;
        pf_rank_unit(p, r, &qb, &hg, &kvh, &b);
        const PfSeg seg{0, pf_unit_tiles(p, qb, 256 >> p.hb_log2), 0, nullptr, nullptr};
        tall_unit(p, smem, qb, hg, kvh, b, seg);
    }
}

}  // namespace

int launch_prefill_tall(const PrefillParams& p, bool pairs, int cus, hipStream_t s) {
    const void* fn = pairs ? reinterpret_cast<const void*>(prefill_tall_pairs_kernel)
                           : reinterpret_cast<const void*>(prefill_tall_persistent_kernel);
    // attribute slots 20, 21: the tall kernels
    if (const int e = set_kernel_smem_once(pairs ? 20 : 21, fn, kTallSmemBytes); e != FGQA_OK) return e;
    const int64_t units = (int64_t)p.n_qblocks * p.n_streams;
    if (pairs) {
        const int64_t npairs = (units + 1) / 2;
        const dim3 grid((unsigned)(16 * ceil_div(npairs, 8)));
        hipLaunchKernelGGL(prefill_tall_pairs_kernel, grid, dim3(kTlThreads), kTallSmemBytes, s, p);
    } else {
        const dim3 grid((unsigned)(units < cus ? units : cus));
        hipLaunchKernelGGL(prefill_tall_persistent_kernel, grid, dim3(kTlThreads), kTallSmemBytes, s, p);
    }
    return hipGetLastError() == hipSuccess ? FGQA_OK : FGQA_ERR_HIP;
}

}  // namespace fgqa
