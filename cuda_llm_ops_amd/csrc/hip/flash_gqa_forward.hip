// Causal GQA prefill forward for gfx950.
//
// Stands in for the reference's Triton-only flash_gqa_forward_bf16_kernel
// (src/python/Triton/flash_gqa_kernel.py:15-138).  Same maths: S = Q.K^T*scale
// in fp32, top-left causal mask (q_idx >= kv_idx, :113-117), online softmax,
// P rounded to bf16 before P.V with the rowsum kept from the fp32 P (:122-129),
// O /= rowsum and lse = max + log(rowsum) (:131-138).
//
// Work unit = 128 query rows: HB heads of one KV group x (128/HB) consecutive
// query positions (HB = 4 when G % 4 == 0, else 2 or 1), one wave per 32 rows,
// so the waves of a unit share every K/V tile staged in LDS.  Two shapes:
//   prefill_kernel        4 waves run a unit over its whole KV range; two
//                         workgroups share a CU (2 waves per SIMD).
//   prefill_split_kernel  8 waves: two groups of 4 run the two halves of the
//                         unit's KV range side by side (2 waves per SIMD) and
//                         merge their partial (max, sum, O) through LDS.  Used
//                         when there are too few units to keep every CU busy
//                         with two workgroups until the end.  Persistent: one
//                         workgroup per CU runs its share of the units in a
//                         fixed order that balances their tile counts.  The groups run
//                         ping-pong: while one wave of a SIMD issues the MFMAs
//                         of a tile, the other runs the softmax of its own.
//                         With head dim 128 it stages the unit's Q tile (once
//                         for both groups) and its O tile through 32 KB of LDS,
//                         so those global loads and stores move whole rows;
//                         the two groups then merge and store half of O each.
//   prefill_wide_kernel   8 waves on a 256-row unit: the two groups take 128
//                         rows each and share every K/V tile (half the tile
//                         loads per row).  Units pair heaviest with lightest;
//                         a pair runs on two workgroups of one XCD, the first
//                         taking the heavy unit's first tiles, the second the
//                         rest of it and then the light unit; the heavy unit's
//                         two partial results merge through device memory.
//                         Used when the pairs fill the CUs (BASELINE-size
//                         causal grids such as S=4096, Hq=16, Hkv=1).
//
// Per wave (32 rows) and 64-token K/V tile j, software pipelined one tile ahead:
//   phase A: S^T(j+1) = K(j+1) . Q^T          v_mfma_f32_32x32x16_bf16, K from LDS,
//                                              Q^T in registers for the whole unit
//            || exp2 / row sums / bf16 cast of S(j)
//   phase B: O^T += V^T(j) . P^T(j)          v_mfma_f32_32x32x16_bf16; V^T read from
//                                              the row-major V tile with ds_read_b64_tr_b16,
//                                              P^T is the S^T accumulator converted in place
//            || masks / row max / scale of S(j+1)
// The running max only moves (and O is rescaled) when a row's new max exceeds
// it by more than 2^8, so P <= 256 and O stays far inside fp32 range.  The
// split kernel does not even compute the row max per tile: it checks the
// tile's row sums against 2^16 after the exps, and takes the max (and
// recomputes P) only when that check fails or a row has no max yet.
// K(j+2) and V(j+1) stream straight into LDS (buffer_load ... lds) while tile
// j is computed.
//
// The MLA prefill (src/python/Triton/flash_mla_kernel.py:16-270: Q/K head dim
// 192, V/O head dim 128, same maths) is the same kernel instantiated with
// kDk = 192: Q^T holds 12 k-steps in registers, K rows are 384 bytes, phase A
// issues 24 MFMAs per tile instead of 16, and a group's LDS grows from 64 KB
// to 80 KB (two workgroups still share a CU's 160 KB).
#include <math.h>
#include <stdint.h>

#include <mutex>
#include <type_traits>

#include "fgqa_device.h"
#include "fgqa_internal.h"
#include "prefill_common.h"
#include "prefill_tall.h"


namespace fgqa {

constexpr int kPfWaves = 4;                            // waves per group (one unit's rows)
constexpr int kPfThreads = kPfWaves * kWave;
constexpr int kPfVRowBytes = kHeadDim * 2;             // one V row (V/O head dim 128)
constexpr int kPfVTileBytes = kPfTile * kPfVRowBytes;  // 16 KB
constexpr float kPfRescaleSlack = 8.f;                 // log2 units: P <= 2^8 between rescales
// merge area of the split kernel: per wave, 64 O values + max + sum per lane
constexpr int kPfMergeFloats = 66;
// Q tile of a unit staged in LDS by the split kernel (head dim 128): 4 waves x
// 32 rows x 256 bytes, after the two groups' tile buffers (2 x 64 KB + 32 KB =
// the CU's 160 KB).
constexpr int kPfQStageBytes = kPfWaves * 32 * kHeadDim * 2;
// Wide kernel (head dim 128): both wave groups work on one set of tile
// buffers (K0, K1, V0, V1: 64 KB), followed by the 256-row unit's Q tile
// (64 KB, later its O tile) and one word that broadcasts the arrival count.
// A split unit's partial result: 66 floats per lane (64 of O, max, sum) of
// each of the 8 waves.
constexpr int kPwTileBytes = 4 * kPfVTileBytes;
constexpr int kPwQBytes = 2 * kPfQStageBytes;
constexpr int kPwSmemBytes = kPwTileBytes + kPwQBytes + 16;   // + 3 words that broadcast counter reads
// With the MLA head dim (192) the wide kernel loads Q straight into registers
// (a 256-row Q tile does not fit beside the 80 KB of tiles) and stages O in
// the tile buffers, idle after the loop.
constexpr int pw_smem_bytes(int dk) { return dk == kHeadDim ? kPwSmemBytes : 2 * (64 * 384) + 2 * kPfVTileBytes + 16; }
static_assert(kPfPartFloats == 2 * kPfWaves * kPfMergeFloats * kWave, "merge slot size");

// Sizes that depend on the Q/K head dim kDk (128; 192 for MLA; 256, which
// only the whole-range kernel is built for).
template <int kDk>
struct PfDims {
    static_assert(kDk == 128 || kDk == 192 || kDk == 256, "Q/K head dim");
    static constexpr int kRowBytes = kDk * 2;                         // one K row
    static constexpr int kChunks = kDk / 8;                           // 16-byte chunks per K row
    static constexpr int kKTileBytes = kPfTile * kRowBytes;           // 16, 24 or 32 KB
    static constexpr int kGroupBytes = 2 * kKTileBytes + 2 * kPfVTileBytes;   // K0, K1, V0, V1
    static constexpr int kSteps = kDk / 16;                           // MFMA k-steps over the head dim
    static constexpr int kDmaK = kDk / 32;                            // K-tile DMA instructions per wave
    // Per-lane K read offsets: k-steps kk and kk + kKoffRegs read chunks
    // 2 * kKoffRegs apart, which the swizzle keeps 32 * kKoffRegs bytes apart.
    static constexpr int kKoffRegs = kDk == 192 ? 4 : 8;
    // K swizzle: chunk c of row r sits in slot c ^ kswz(r).  16 consecutive
    // rows read at one chunk hit 16 distinct 16-byte bank groups: 256- and
    // 512-byte rows all start at bank 0 (XOR with r % 16, which keeps c inside
    // its aligned block of 16); 384-byte rows start at bank 0 or 32 by row
    // parity, so an XOR with (r / 2) % 8 (which keeps c inside its aligned
    // block of 8) spreads each parity class over 8 groups.
    static __device__ __forceinline__ int kswz(int r) { return kDk == 192 ? ((r >> 1) & 7) : (r & 15); }
    static_assert(kPfWaves * kPfMergeFloats * kWave * 4 <= 2 * kGroupBytes, "merge area must fit in the tile buffers");
};

// LDS tiles hold unpadded rows whose 16-byte chunks are permuted (XOR
// swizzle) so that both read patterns are free of bank conflicts:
//   K: chunk c of row r sits in slot c ^ kswz(r)       (16 rows, one chunk each: b128 reads)
//   V: chunk c of row r sits in slot c ^ 4*(r % 4)     (4 rows x 4 chunks: transposed b64 reads)
// Tiles are filled by buffer_load ... lds (16 bytes per lane straight into
// LDS): one instruction writes 1 KB, lane l taking the l-th 16-byte slot of
// it, so each lane fetches the chunk that belongs in its slot.

// One unit (query block qb of head group hg, kv head kvh, batch b).  With
// kGroups == 2, group `grp` covers tiles [grp*half, grp*half + half) of the
// unit's KV range; tiles past the range are fully masked and add nothing.
// kSwa: sliding window and/or sink (a separate instantiation, so the plain
// causal kernels carry none of its work).
// kWide (with kGroups == 2, head dim 128): a 256-row unit whose two groups
// take 128 rows each and share every K/V tile; the call runs segment `seg` of
// the unit's KV range.
template <int kGroups, bool kSwa, int kDk, bool kWide = false>
__device__ __forceinline__ void pf_unit(const PrefillParams& p, unsigned char* smem_all, int qb, int hg, int kvh,
                                        int b, PfSeg seg = PfSeg{0, 0, 0, nullptr, nullptr}) {
    using D = PfDims<kDk>;
    static_assert(!kWide || kGroups == 2, "wide units: two groups");
    // wide: the tile buffers, then (head dim 128) the Q/O area, then 3 broadcast words
    [[maybe_unused]] constexpr int kWWords = D::kGroupBytes + (kDk == kHeadDim ? kPwQBytes : 0);
    // opaque in the split kernel: its loop over units recomputes what depends
    // on the thread index inside each unit instead of holding it in
    // registers across the loop
    int tid = threadIdx.x;
    if constexpr (kGroups == 2) asm volatile("" : "+v"(tid));
    const int lane = tid & (kWave - 1);
    const int wave_wg = __builtin_amdgcn_readfirstlane(tid / kWave);   // wave-uniform
    const int grp = wave_wg / kPfWaves;
    const int wave = wave_wg % kPfWaves;
    unsigned char* smem = kWide ? smem_all : smem_all + grp * D::kGroupBytes;
    const int l32 = lane & 31;
    const int l16 = lane & 15;
    const int g2 = lane >> 5;
    // the wave's 32 rows: slot `wslot` of the unit (a wide unit has 8 slots)
    const int wslot = kWide ? wave_wg : wave;
    const int qrows = (kWide ? 256 : 128) >> p.hb_log2;
    const int q_wg0 = qb * qrows;
    const int h = kvh * p.group + hg * p.hb + (wslot & (p.hb - 1));
    const int q0w = q_wg0 + (wslot >> p.hb_log2) * 32;
    const int qrow = q0w + l32;

    int kv_end = p.skv;
    if (p.causal) kv_end = min(kv_end, min(q_wg0 + qrows, p.sq));
    // a sliding window starts the unit at the tile holding its first row's first key
    const int t_lo = (kSwa && p.window > 0) ? max(0, q_wg0 - p.window + 1) / kPfTile : 0;
    const int unit_tiles = max(0, (kv_end + kPfTile - 1) / kPfTile - t_lo);
    // loop trips, same for both groups, and this group's first tile
    const int n_tiles = kWide ? seg.hi - seg.lo : kGroups == 1 ? unit_tiles : (unit_tiles + 1) / 2;
    const int t_first = kWide ? t_lo + seg.lo : t_lo + grp * n_tiles;
    (void)unit_tiles;
    // keys this group may use: the unit's range, cut at the group's last tile
    const int kv_hi = min(kv_end, (t_first + n_tiles) * kPfTile);

    // Q^T as the B operand: lane holds Q[q0w + l32][16*kk + 8*g2 .. +7]; rows >= sq read as 0.
    // The split kernel (head dim 128) stages the unit's Q tile in LDS first
    // (kStageQ below): a direct load puts 32 rows 4 KB apart (BSHD) into
    // one instruction, 32 bytes each, and both groups would load the same rows.
    constexpr bool kStageQ = kGroups == 2 && kDk == kHeadDim;
    const uint32_t qss = (uint32_t)(p.q_ss * 2);
    const __amdgpu_buffer_rsrc_t qrs =
        make_rsrc(p.q + b * p.q_sb + h * p.q_sh, (uint32_t)(p.sq - 1) * qss + D::kRowBytes);
    bf16x8_t qop[D::kSteps];
    if constexpr (!kStageQ) {
#pragma unroll
        for (int kk = 0; kk < D::kSteps; ++kk) {
            u32x4_t t = buf_load16(qrs, (uint32_t)qrow * qss + (kk * 16 + g2 * 8) * 2);
            t ^= p.q_sign;
            qop[kk] = as_bf16x8(t);
        }
    }

    // Direct K/V tile loads.  Rows past the last key are clamped to it (their
    // scores are masked, so they only need to be finite).
    const uint32_t kss = (uint32_t)(p.k_ss * 2);
    const uint32_t vss = (uint32_t)(p.v_ss * 2);
    const int kv_last = p.skv > 0 ? p.skv - 1 : 0;
    const __amdgpu_buffer_rsrc_t krs =
        make_rsrc(p.k + b * p.k_sb + kvh * p.k_sh, (uint32_t)kv_last * kss + D::kRowBytes);
    const __amdgpu_buffer_rsrc_t vrs =
        make_rsrc(p.v + b * p.v_sb + kvh * p.v_sh, (uint32_t)kv_last * vss + kHeadDim * 2);
    // K(t_first + j) -> K buffer kb (skipped when kb < 0), V(t_first + j) -> V buffer vb.
    // Written as inline asm so that the compiler does not treat every later
    // LDS read as dependent on these writes (it would wait for them to land
    // before reading the other buffer); their completion is awaited
    // explicitly (wait_vmem) before the barrier that publishes the tile.
    const uint32_t lds_base = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) unsigned char*)smem;
    // Instruction i writes 4096*i bytes past the wave's first KB of the tile.
    // The destination goes to M0 as base + literal inside the asm, so only
    // one SGPR per tile buffer stays live (one SGPR per instruction made the
    // compiler spill them and reload each with v_readlane in the loop).
    auto dma16 = [](auto ic, uint32_t base, uint32_t voffset, uint32_t soffset, __amdgpu_buffer_rsrc_t rsrc) {
        constexpr int kOff = decltype(ic)::value * 4096;
        asm volatile("s_add_u32 m0, %0, %4\n\tbuffer_load_dwordx4 %1, %2, %3 offen lds"
                     :: "s"(base), "v"(voffset), "s"(rsrc), "s"(soffset), "i"(kOff) : "memory", "scc");
    };
    // Instruction i of this wave fills the 1 KB at slot 64*(wave + 4*i) of a
    // tile; lane l writes slot 64*(wave + 4*i) + l, i.e. row r = slot / chunks,
    // swizzled position slot % chunks, which holds chunk (slot % chunks) ^ swz(r).
    // Per-lane byte offsets of those chunks within a tile; the tile's start
    // goes in the scalar offset.
    int krow_dma[D::kDmaK];
    uint32_t kcol_dma[D::kDmaK], koff_dma[D::kDmaK], voff_dma[4];
#pragma unroll
    for (int i = 0; i < D::kDmaK; ++i) {
        const int slot = 64 * (wave + 4 * i) + lane;
        const int r = slot / D::kChunks;
        krow_dma[i] = r;
        kcol_dma[i] = (uint32_t)(((slot % D::kChunks) ^ D::kswz(r)) << 4);
        koff_dma[i] = (uint32_t)r * kss + kcol_dma[i];
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int r = 4 * (wave + 4 * i) + (lane >> 4);
        voff_dma[i] = (uint32_t)r * vss + ((l16 ^ (4 * (r & 3))) << 4);
    }
    // kb / vb: an int, or (split kernel loop) a std::integral_constant, so that
    // every LDS address folds into the instructions' offset fields
    auto issue_tile = [&](int j, auto kb, auto vb) {
        const int t0 = (t_first + j) * kPfTile;
        const uint32_t kdst = lds_base + kb * D::kKTileBytes + 1024 * wave;
        const uint32_t vdst = lds_base + 2 * D::kKTileBytes + vb * kPfVTileBytes + 1024 * wave;
        // K and V instructions interleaved, K first
        if (t0 + kPfTile - 1 <= kv_last) {   // whole tile in range
            static_for<D::kDmaK>([&](auto ic) {
                constexpr int i = decltype(ic)::value;
                if (kb >= 0) dma16(ic, kdst, koff_dma[i], (uint32_t)t0 * kss, krs);
                if constexpr (i < 4)
                    if (vb >= 0) dma16(ic, vdst, voff_dma[i], (uint32_t)t0 * vss, vrs);
            });
        } else {   // last tile: rows past the last key are clamped to it
            static_for<D::kDmaK>([&](auto ic) {
                constexpr int i = decltype(ic)::value;
                if (kb >= 0) {
                    const uint32_t tok = (uint32_t)min(t0 + krow_dma[i], kv_last);
                    dma16(ic, kdst, tok * kss + kcol_dma[i], 0u, krs);
                }
                if (vb >= 0 && i < 4) {
                    const int r = 4 * (wave + 4 * i) + (lane >> 4);
                    const uint32_t tok = (uint32_t)min(t0 + r, kv_last);
                    dma16(ic, vdst, tok * vss + ((l16 ^ (4 * (r & 3))) << 4), 0u, vrs);
                }
            });
        }
    };

    // S^T(tile j) = K(j) . Q^T: lane holds column q = l32, tokens 32*tb + 8*(i/4) + 4*g2 + i%4.
    // K operand of (tb, kk): row 32*tb + l32, chunk 2*kk + g2.  The swizzle of
    // rows 32*tb + l32 does not depend on tb; with 384-byte rows it only
    // permutes within aligned blocks of 8 chunks, so k-steps kk and kk + 4 sit
    // 128 bytes apart and share one offset register.
    int koff[D::kKoffRegs];
#pragma unroll
    for (int kk = 0; kk < D::kKoffRegs; ++kk)
        koff[kk] = l32 * D::kRowBytes + (((2 * kk + g2) ^ D::kswz(l32)) << 4);
    auto qk = [&](f32x16_t (&s)[2], auto buf) {
        const unsigned char* kl = smem + buf * D::kKTileBytes;
#pragma unroll
        for (int tb = 0; tb < 2; ++tb)
#pragma unroll
            for (int i = 0; i < 16; ++i) s[tb][i] = 0.f;
#pragma unroll
        for (int kk = 0; kk < D::kSteps; ++kk)
#pragma unroll
            for (int tb = 0; tb < 2; ++tb) {
                const int off = tb * 32 * D::kRowBytes + koff[kk % D::kKoffRegs] + (kk / D::kKoffRegs) * (D::kKoffRegs * 32);
                const bf16x8_t ka = *reinterpret_cast<const bf16x8_t*>(kl + off);
                s[tb] = mfma32(ka, qop[kk], s[tb]);
            }
    };

    const float c = p.scale_log2;
    // this lane's row sees keys [0, row_lim)
    const int row_lim = p.causal ? min(p.skv, qrow + 1) : p.skv;
    float m_run = -INFINITY;   // running max (log2 units) of this lane's row
    float m_use = 0.f;         // m_run, or 0 while m_run is -inf
    float l_run = 0.f;         // this lane's share of the row sum
    f32x16_t oacc[4];
#pragma unroll
    for (int db = 0; db < 4; ++db)
#pragma unroll
        for (int i = 0; i < 16; ++i) oacc[db][i] = 0.f;

    // Causal / window / tail mask of S(j), in place (only tiles that cross a boundary).
    auto mask = [&](f32x16_t (&s)[2], int j) {
        const int kv0 = (t_first + j) * kPfTile;
        bool need_mask = (kv0 + kPfTile > kv_hi) || (p.causal && kv0 + kPfTile - 1 > q0w);
        if constexpr (kSwa) need_mask = need_mask || (p.window > 0 && kv0 < q0w + 32 - p.window);
        if (need_mask) {
            // tokens at or past `lim`, or (window) before `lo`, relative to
            // this lane's first token, are masked
            const int lim = min(row_lim, kv_hi) - (kv0 + g2 * 4);
            const int lo = (kSwa && p.window > 0) ? qrow - p.window + 1 - (kv0 + g2 * 4) : -kPfTile;
#pragma unroll
            for (int tb = 0; tb < 2; ++tb)
#pragma unroll
                for (int i = 0; i < 16; ++i) {
                    const int idx = tb * 32 + (i >> 2) * 8 + (i & 3);
                    if (idx >= lim || (kSwa && idx < lo)) s[tb][i] = -INFINITY;
                }
        }
    };
    // Row max of S(j) (log2 units) across both wave halves.
    // The split kernel's softmax phase runs on a SIMD whose other wave issues
    // MFMAs, so its reductions use four independent chains (the serial chain
    // costs the latency of each step); the whole-range kernel keeps one chain,
    // which needs fewer registers.
    auto rowmax = [&](f32x16_t (&s)[2]) {
        float tmax;
        if constexpr (kGroups == 2) {
            float pm[4];
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                pm[t] = s[t >> 1][(t & 1) * 8];
#pragma unroll
                for (int i = 1; i < 8; ++i) pm[t] = fmaxf(pm[t], s[t >> 1][(t & 1) * 8 + i]);
            }
            tmax = fmaxf(fmaxf(pm[0], pm[1]), fmaxf(pm[2], pm[3]));
        } else {
            tmax = s[0][0];
#pragma unroll
            for (int tb = 0; tb < 2; ++tb)
#pragma unroll
                for (int i = 0; i < 16; ++i)
                    if (tb != 0 || i != 0) tmax = fmaxf(tmax, s[tb][i]);
        }
        return half_max(tmax) * c;
    };
    // Move the running max when some row's tile max exceeds it by more than
    // the slack (rare after the first tiles): rescale O and the row sum.
    auto update_max = [&](float tmax) {
        if (__builtin_amdgcn_ballot_w64(tmax > m_run + kPfRescaleSlack) != 0) {
            const float m_new = fmaxf(m_run, tmax);
            const float m_new_use = (m_new == -INFINITY) ? 0.f : m_new;
            const float alpha = fast_exp2(m_use - m_new_use);   // 0 on the first tile
            l_run *= alpha;
#pragma unroll
            for (int db = 0; db < 4; ++db) oacc[db] *= alpha;
            m_run = m_new;
            m_use = m_new_use;
        }
    };

    // exp2(S*scale - max) and the bf16 P^T operands of S(j); returns this
    // lane's share of the tile's row sum.
    bf16x8_t pop[4];
    auto softmax_p = [&](f32x16_t (&s)[2]) {
        if constexpr (kGroups == 2) {
            float ps[4];
#pragma unroll
            for (int t = 0; t < 4; ++t) {
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    const float pv = fast_exp2(__builtin_fmaf(s[t >> 1][(t & 1) * 8 + e], c, -m_use));
                    ps[t] = e == 0 ? pv : ps[t] + pv;
                    pop[t][e] = (__bf16)pv;
                }
            }
            return (ps[0] + ps[1]) + (ps[2] + ps[3]);
        } else {
            float psum = 0.f;
#pragma unroll
            for (int tb = 0; tb < 2; ++tb)
#pragma unroll
                for (int kh = 0; kh < 2; ++kh)
#pragma unroll
                    for (int e = 0; e < 8; ++e) {
                        const float pv = fast_exp2(__builtin_fmaf(s[tb][kh * 8 + e], c, -m_use));
                        psum += pv;
                        pop[tb * 2 + kh][e] = (__bf16)pv;
                    }
            return psum;
        }
    };

    // O^T += V^T(j) . P^T(j) over four 16-token k-blocks.  Slots 0..3 of lane
    // (l32, g2) hold tokens 16*kb + 4*g2 + 0..3, slots 4..7 tokens 16*kb + 8 + 4*g2 + 0..3:
    // the S^T registers 8*(kb%2) .. +7 of block kb/2, and the two transposed
    // V reads below.  Lane i of a 16-lane group supplies row 16*kb + 4*g2 + i/4
    // (+8), columns 32*db + 16*((lane/16)%2) + 4*(i%4) .. +3, which is chunk
    // 4*db + 2*((lane/16)%2) + (i%4)/2, half i%2 of the swizzled row.
    int voff[4];
    {
        const int q4 = l16 >> 2;
        const int dh = (lane >> 4) & 1;
#pragma unroll
        for (int db = 0; db < 4; ++db)
            voff[db] = (4 * g2 + q4) * kPfVRowBytes + ((4 * (db ^ q4) + 2 * dh + ((l16 >> 1) & 1)) << 4) + 8 * (l16 & 1);
    }
    auto pv = [&](auto buf) {
        const unsigned char* vl = smem + 2 * D::kKTileBytes + buf * kPfVTileBytes;
#pragma unroll
        for (int kb = 0; kb < 4; ++kb)
#pragma unroll
            for (int db = 0; db < 4; ++db) {
                const unsigned char* base = vl + 16 * kb * kPfVRowBytes + voff[db];
                const bf16x4_t lo = lds_read_tr16(reinterpret_cast<const __bf16*>(base));
                const bf16x4_t hi = lds_read_tr16(reinterpret_cast<const __bf16*>(base + 8 * kPfVRowBytes));
                const bf16x8_t va = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
                oacc[db] = mfma32(va, pop[kb], oacc[db]);
            }
    };

    // this wave's direct LDS loads have landed (then a barrier publishes them)
    auto wait_vmem = [] { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); };
    // every load of this wave but the newest n has landed (loads complete in
    // order); n is a multiple of 4 up to 8 (the split kernel's K and V tiles
    // at head dim 128 take 4 instructions per wave each)
    [[maybe_unused]] auto wait_vmem_but = [](int n) {
        if (n >= 8) asm volatile("s_waitcnt vmcnt(8)" ::: "memory");
        else if (n >= 4) asm volatile("s_waitcnt vmcnt(4)" ::: "memory");
        else asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    };

    // K runs one tile ahead of V: iteration j reads K(j+1) and V(j) while
    // K(j+2) and V(j+1) land in the buffers freed by iteration j-1.  No
    // branch touches the accumulators (a branch costs register copies), and
    // S(j+1) is computed even on the last step (its tile is fully masked).
    __syncthreads();  // the previous unit may still read the buffers
    // wide split segment: this workgroup's XCD, for the other segment of the unit
    [[maybe_unused]] uint32_t my_xcc1 = 0;
    if constexpr (kWide) {
        if (seg.part != nullptr) {
            uint32_t hw;
            asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(hw));
            my_xcc1 = (hw & 15u) + 1u;
            if (tid == 0) __hip_atomic_store(seg.ctr + 1 + seg.slot, my_xcc1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    }
    // Staged Q: wave slot w's 32 rows fill 8 KB at kPfQStageBytes/4 * w past
    // the tile buffers, row r at 256*r with chunk c in slot c ^ (r % 16) (the
    // K layout).  One load instruction fills 1 KB = 4 whole rows; the wave of
    // slot w in group g issues instructions 4g .. 4g+3 of its slot's 8, so
    // each row is fetched once for both groups.
    [[maybe_unused]] const uint32_t q_lds =
        kWide ? lds_base + kPwTileBytes + wave_wg * (kPfQStageBytes / kPfWaves)
              : lds_base + (2 - grp) * D::kGroupBytes + wave * (kPfQStageBytes / kPfWaves);
    if constexpr (kWide) {
        // a wide unit's waves have rows of their own: each loads its 8 KB
        // (head dim 192: Q came straight into registers above)
        if constexpr (kStageQ) {
            auto dmaq = [](auto ic, uint32_t base, uint32_t voffset, __amdgpu_buffer_rsrc_t rsrc) {
                constexpr int kOff = decltype(ic)::value * 1024;
                asm volatile("s_add_u32 m0, %0, %3\n\tbuffer_load_dwordx4 %1, %2, 0 offen lds"
                             :: "s"(base), "v"(voffset), "s"(rsrc), "i"(kOff) : "memory", "scc");
            };
            static_for<8>([&](auto ic) {
                const int slot = 64 * decltype(ic)::value + lane;
                const int r = slot >> 4;
                const uint32_t voff = (uint32_t)(q0w + r) * qss + ((uint32_t)((slot & 15) ^ (r & 15)) << 4);
                dmaq(ic, q_lds, voff, qrs);
            });
        }
        // group 0 loads K(0); group 1 loads V(0) and K(1), awaited by the end
        // of its S(0) phase (group 0's first MFMA phase comes after that)
        if (grp == 0) {
            if (n_tiles > 0) issue_tile(0, 0, -1);
            wait_vmem();
        } else {
            if (n_tiles > 0) issue_tile(0, -1, 0);
            if (n_tiles > 1) issue_tile(1, 1, -1);
            wait_vmem_but((n_tiles > 0 ? 4 : 0) + (n_tiles > 1 ? D::kDmaK : 0));
        }
    } else if constexpr (kStageQ) {
        auto dmaq = [](auto ic, uint32_t base, uint32_t voffset, __amdgpu_buffer_rsrc_t rsrc) {
            constexpr int kOff = decltype(ic)::value * 1024;
            asm volatile("s_add_u32 m0, %0, %3\n\tbuffer_load_dwordx4 %1, %2, 0 offen lds"
                         :: "s"(base), "v"(voffset), "s"(rsrc), "i"(kOff) : "memory", "scc");
        };
        static_for<4>([&](auto ic) {
            const int slot = 64 * (4 * grp + decltype(ic)::value) + lane;
            const int r = slot >> 4;
            const uint32_t voff = (uint32_t)(q0w + r) * qss + ((uint32_t)((slot & 15) ^ (r & 15)) << 4);
            dmaq(ic, q_lds + grp * 4096, voff, qrs);
        });
    }
    if constexpr (kWide) {
    } else if constexpr (kStageQ) {
        // the first barrier needs Q and K(0) only: V(0) and K(1) are waited
        // for by the first softmax phase
        static_assert(D::kDmaK == 4, "wait_vmem_but counts 4 loads per tile");
        if (n_tiles > 0) issue_tile(0, 0, -1);
        if (n_tiles > 0) issue_tile(0, -1, 0);
        if (n_tiles > 1) issue_tile(1, 1, -1);
        wait_vmem_but((n_tiles > 0 ? 4 : 0) + (n_tiles > 1 ? 4 : 0));
    } else {
        if (n_tiles > 0) issue_tile(0, 0, 0);
        if (n_tiles > 1) issue_tile(1, 1, -1);
        wait_vmem();
    }
    __syncthreads();
    if constexpr (kStageQ) {
        const unsigned char* ql = reinterpret_cast<const unsigned char*>(smem_all) +
                                  (kWide ? kPwTileBytes + wave_wg * (kPfQStageBytes / kPfWaves)
                                         : 2 * D::kGroupBytes + wave * (kPfQStageBytes / kPfWaves)) +
                                  l32 * D::kRowBytes;
#pragma unroll
        for (int kk = 0; kk < D::kSteps; ++kk) {
            u32x4_t t = *reinterpret_cast<const u32x4_t*>(ql + (((2 * kk + g2) ^ (l32 & 15)) << 4));
            t ^= p.q_sign;
            qop[kk] = as_bf16x8(t);
        }
    }

    // One pipelined step.  On entry sc holds the masked S(j) and the running
    // max covers it; on exit sn holds the masked S(j+1), likewise.
    auto step = [&](f32x16_t (&sc)[2], f32x16_t (&sn)[2], int j) {
        if (j + 2 < n_tiles) issue_tile(j + 2, j & 1, -1);
        if (j + 1 < n_tiles) issue_tile(j + 1, -1, (j + 1) & 1);
        // phase A: S(j+1) on the MFMA pipe while exp2 / sums / bf16 P of S(j)
        // run on the VALU: each MFMA is followed by its K read for a later
        // MFMA and a slice of the softmax.
        qk(sn, (j + 1) & 1);
        l_run += softmax_p(sc);
        // keep P here: otherwise the compiler sinks the softmax to its use in phase B
#pragma unroll
        for (int kb = 0; kb < 4; ++kb) asm volatile("" : "+v"(pop[kb]));
        asm volatile("" : "+v"(l_run));
        // The scheduler's small-GEMM interleave (LLVM's IGLP strategy 0)
        // places the K reads and the softmax's ~96 VALU ops among the
        // phase's 16 (or 24) MFMAs: 4.9 % faster at the reference's
        // sliding-window shape than pinning one K read 4 MFMAs ahead and
        // 96 / 16 VALU ops after each MFMA (strategies 2 and 3, the MFMA /
        // exp interleaves, were no faster than the pinning).
        __builtin_amdgcn_iglp_opt(0);
        mask(sn, j + 1);
        // phase B: P(j).V(j) on the MFMA pipe while the row max of S(j+1)
        // runs on the VALU.
        pv(j & 1);
        const float tmax = rowmax(sn);
        // V reads run 3 MFMAs ahead of their use
        __builtin_amdgcn_sched_group_barrier(0x100, 6, 0);       // DS reads
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);   // MFMA
            __builtin_amdgcn_sched_group_barrier(0x002, 2, 0);   // VALU
            if (i < 13) __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);   // DS reads
        }
        update_max(tmax);
        wait_vmem();
        __syncthreads();
    };
    if constexpr (kGroups == 2) {
        // Ping-pong: the two waves of a SIMD (one per group) alternate an
        // MFMA phase (S(j+1) = K(j+1).Q^T and O += V(j).P(j), with their LDS
        // reads) and a VALU phase (mask, row max, exp2, sums and bf16 P of
        // S(j+1), then the tile loads for the MFMA phase after next), group 1
        // one phase behind group 0, with a workgroup barrier between phases.
        // Both groups pass the same number of barriers: group 1 computes S(0)
        // in an extra leading phase, group 0 ends with an empty one.
        f32x16_t s[2];
        if (grp == 0 && n_tiles > 0) qk(s, 0);
        __syncthreads();
        if (grp == 1) {
            if (n_tiles > 0) qk(s, 0);
            if constexpr (kWide) wait_vmem();   // V(0), K(1)
            __syncthreads();              // both groups' S(0) phases are past: K(0) is free
        }
        // S(j+1) -> P(j+1); then K(j+3) and V(j+2) go into the buffers that
        // the MFMA phase j has just finished reading.
        // The running max only keeps P and O inside fp32 range (O / sum does
        // not depend on it), so this phase computes P against the current
        // max first and takes the row max only when it must: when a row has
        // no max yet (its first visible keys), or when a lane's share of the
        // tile's row sum passes 2^16 (some P above 2^11: the tile's max beat
        // the running max by more than the rescale slack).  Then it moves the
        // max, rescales O and the sum, and recomputes P, which ends at most
        // 2^8 per element.  Otherwise every P stays below 2^16 and the row
        // max is never computed (it is the softmax phase's costliest
        // reduction, and this phase sets the pace).
        // j: the MFMA phase this softmax phase follows (-1 for the first one);
        // par = j & 1 as a constant.
        auto vphase = [&](int j, auto par) {
            constexpr int P = decltype(par)::value;
            using CK = std::integral_constant<int, 1 - P>;   // K buffer of tile j + 3
            using CV = std::integral_constant<int, P>;       // V buffer of tile j + 2
            using CN = std::integral_constant<int, -1>;
            // the softmax phase sets the pace: its wave wins issue ties
            // against the MFMA wave of the same SIMD
            __builtin_amdgcn_s_setprio(1);
            // Head dim 128: the next tiles go in first, under the softmax (the
            // MFMA phase j before this one's barrier has finished with K
            // buffer (j+1)&1 and V buffer j&1); the loads of the previous
            // softmax phase are awaited at the end.  Issuing a tile's loads
            // stalls the issuing wave for a few hundred cycles, which the
            // softmax then no longer waits behind.
            [[maybe_unused]] int n_new = 0;
            if constexpr (kWide) {
                // wide units share the tiles: group 1 alone loads them, into
                // the buffers both groups' MFMA phases j have finished with,
                // and awaits them at the end of its next MFMA phase
                if (grp == 1) {
                    if (j + 3 < n_tiles) issue_tile(j + 3, CK{}, CN{});
                    if (j + 2 < n_tiles) issue_tile(j + 2, CN{}, CV{});
                }
            } else if constexpr (kStageQ) {
                if (j + 3 < n_tiles) {
                    issue_tile(j + 3, CK{}, CN{});
                    n_new += D::kDmaK;
                }
                if (j + 2 < n_tiles) {
                    issue_tile(j + 2, CN{}, CV{});
                    n_new += 4;
                }
            }
            mask(s, j + 1);
            float lt = softmax_p(s);
            if (__builtin_amdgcn_ballot_w64(m_run == -INFINITY || !(lt <= 65536.f)) != 0) {
                update_max(rowmax(s));
                lt = softmax_p(s);
            }
            l_run += lt;
#pragma unroll
            for (int kb = 0; kb < 4; ++kb) asm volatile("" : "+v"(pop[kb]));
            asm volatile("" : "+v"(l_run));
            if constexpr (kWide) {
            } else if constexpr (kStageQ) {
                wait_vmem_but(n_new);         // K(j+2), V(j+1), issued one softmax phase ago
            } else {
                wait_vmem();                  // K(j+2), V(j+1), issued one softmax phase ago
                if (j + 3 < n_tiles) issue_tile(j + 3, CK{}, CN{});
                if (j + 2 < n_tiles) issue_tile(j + 2, CN{}, CV{});
            }
            __builtin_amdgcn_s_setprio(0);
            __syncthreads();
        };
        // S(j+1) (unless this is the last tile) and O += V(j).P(j): K reads
        // run 4 MFMAs ahead, V reads 4 ahead at 2 per MFMA.
        // par = j & 1 as a constant: the buffer offsets are then instruction
        // immediates, and the phase issues nothing but LDS reads and MFMAs.
        // The operand reads are written in the order they should issue: the
        // phase's 16 (or 24) K operands and then its 16 V operands form one
        // stream, each read 4 MFMAs ahead of its use into a ring of 4
        // registers.  So even a schedule that keeps source order (which the
        // compiler falls back to when it judges a region's register pressure
        // too high) keeps the reads ahead of the MFMAs.
        auto mphase = [&](auto with_qk, int j, auto par) {
            constexpr int kA = decltype(with_qk)::value ? 2 * D::kSteps : 0;
            constexpr int P = decltype(par)::value;
            constexpr int kOps = kA + 16;
            (void)j;
            const unsigned char* kl = smem + (1 - P) * D::kKTileBytes;
            const unsigned char* vl = smem + 2 * D::kKTileBytes + P * kPfVTileBytes;
            // operand i: K operand (kk, tb) = (i / 2, i % 2) for i < kA, else V
            // operand (kb, db) = ((i - kA) / 4, (i - kA) % 4)
            auto fetch = [&](auto ic) -> bf16x8_t {
                constexpr int i = decltype(ic)::value;
                if constexpr (i < kA) {
                    constexpr int kk = i / 2, tb = i % 2;
                    const int off = tb * 32 * D::kRowBytes + koff[kk % D::kKoffRegs] + (kk / D::kKoffRegs) * (D::kKoffRegs * 32);
                    return *reinterpret_cast<const bf16x8_t*>(kl + off);
                } else {
                    constexpr int kb = (i - kA) / 4, db = (i - kA) % 4;
                    const unsigned char* base = vl + 16 * kb * kPfVRowBytes + voff[db];
                    const bf16x4_t lo = lds_read_tr16(reinterpret_cast<const __bf16*>(base));
                    const bf16x4_t hi = lds_read_tr16(reinterpret_cast<const __bf16*>(base + 8 * kPfVRowBytes));
                    return __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
                }
            };
            bf16x8_t ring[4];
            static_for<4>([&](auto ic) { ring[decltype(ic)::value] = fetch(ic); });
            if constexpr (kA > 0) {
#pragma unroll
                for (int tb = 0; tb < 2; ++tb)
#pragma unroll
                    for (int i = 0; i < 16; ++i) s[tb][i] = 0.f;
            }
            static_for<kOps>([&](auto ic) {
                constexpr int i = decltype(ic)::value;
                const bf16x8_t a = ring[i % 4];
                if constexpr (i < kA) {
                    s[i % 2] = mfma32(a, qop[i / 2], s[i % 2]);
                } else {
                    constexpr int kb = (i - kA) / 4, db = (i - kA) % 4;
                    oacc[db] = mfma32(a, pop[kb], oacc[db]);
                }
                if constexpr (i + 4 < kOps) ring[i % 4] = fetch(std::integral_constant<int, i + 4>{});
            });
            if constexpr (kA > 0) {
                __builtin_amdgcn_sched_group_barrier(0x100, 4, 0);   // DS read
#pragma unroll
                for (int i = 0; i < kA - 4; ++i) {
                    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);   // MFMA
                    __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
                }
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                    __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
                }
            } else {
                __builtin_amdgcn_sched_group_barrier(0x100, 8, 0);
            }
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                if (i < 12) __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
            }
            // all of the phase's MFMAs before its barrier (the scheduler would
            // otherwise sink the last ones into the softmax phase)
            __builtin_amdgcn_sched_barrier(0);
            if constexpr (kWide) {
                if (grp == 1) wait_vmem();   // the tiles its last softmax phase loaded
            }
            __syncthreads();
        };
        // the loop runs two tiles per trip, so that every buffer index is a constant
        using C0 = std::integral_constant<int, 0>;
        using C1 = std::integral_constant<int, 1>;
        vphase(-1, C1{});
        int j = 0;
        for (; j + 2 < n_tiles; j += 2) {
            mphase(std::true_type{}, j, C0{});
            vphase(j, C0{});
            mphase(std::true_type{}, j + 1, C1{});
            vphase(j + 1, C1{});
        }
        if (j + 1 < n_tiles) {
            mphase(std::true_type{}, j, C0{});
            vphase(j, C0{});
            ++j;
        }
        if (n_tiles > 0) {
            if (j & 1) mphase(std::false_type{}, j, C1{});
            else mphase(std::false_type{}, j, C0{});
        }
        if (grp == 0) __syncthreads();
    } else {
        f32x16_t sa[2], sb[2];
        if (n_tiles > 0) {
            qk(sa, 0);
            mask(sa, 0);
            update_max(rowmax(sa));
        }
        __syncthreads();   // every wave has read K(0) before step 0 refills its buffer
        for (int j = 0; j < n_tiles; j += 2) {
            step(sa, sb, j);
            if (j + 1 < n_tiles) step(sb, sa, j + 1);
        }
    }

    if constexpr (kWide) {
        if (seg.part != nullptr) {
            // Split unit: the first of its two segments to finish publishes
            // its partial (O, max, sum of every lane) in its slot and counts
            // its arrival; the second merges that with its own and writes the
            // output.  A segment that finds no arrival publishes, and merges
            // anyway if the other one arrived in the meantime.  The merger
            // sets the unit's words back to 0 for the next launch.
            // Words of the unit: ctr[0] counts arrivals as 1 + the publisher's
            // XCD, ctr[1 + slot] holds 1 + the XCD of the segment in that slot
            // (written at its start).  Ordering: every wave waits for its own
            // partial stores (they are then in its XCD's L2: the L1 writes
            // through) before the barrier after which thread 0 counts the
            // arrival.  When the other segment runs on the same XCD (blocks w
            // and w + 8 do: blocks go round-robin over the XCDs) the two share
            // that L2, and the reader only invalidates its L1 (the compiler's
            // own acquire for workgroups spread over CUs of one L2); otherwise
            // thread 0 counts with a device-scope release (one L2 write-back
            // for the workgroup) and the reader's waves acquire at device
            // scope.
            unsigned* word = reinterpret_cast<unsigned*>(smem_all + kWWords);
            const int woff = wave_wg * kPfMergeFloats * kWave;
            float* own = seg.part + seg.slot * kPfPartFloats + woff;
            const float* other = seg.part + (1 - seg.slot) * kPfPartFloats + woff;
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
                for (int db = 0; db < 4; ++db)
#pragma unroll
                    for (int i4 = 0; i4 < 4; ++i4)
                        o4[(db * 4 + i4) * kWave] = f32x4_t{oacc[db][4 * i4], oacc[db][4 * i4 + 1],
                                                            oacc[db][4 * i4 + 2], oacc[db][4 * i4 + 3]};
                own[64 * kWave + lane] = m_run;
                own[65 * kWave + lane] = l_run;
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
            // slot 0's terms first whichever merges, so the output does not
            // depend on the order of arrival
            const bool first = seg.slot == 0;
            const float m_o = other[64 * kWave + lane];
            const float l_o = other[65 * kWave + lane];
            const float mA = first ? m_run : m_o, lA = first ? l_run : l_o;
            const float mB = first ? m_o : m_run, lB = first ? l_o : l_run;
            const float m = fmaxf(mA, mB);
            const float mu = (m == -INFINITY) ? 0.f : m;
            const float aA = fast_exp2(mA - mu);   // 0 when a segment saw no key
            const float aB = fast_exp2(mB - mu);
            const f32x4_t* r4 = reinterpret_cast<const f32x4_t*>(other) + lane;
#pragma unroll
            for (int db = 0; db < 4; ++db)
#pragma unroll
                for (int i4 = 0; i4 < 4; ++i4) {
                    const f32x4_t ot = r4[(db * 4 + i4) * kWave];
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        const float mine = oacc[db][4 * i4 + e];
                        const float oa = first ? mine : ot[e], ob = first ? ot[e] : mine;
                        oacc[db][4 * i4 + e] = __builtin_fmaf(oa, aA, ob * aB);
                    }
                }
            l_run = __builtin_fmaf(lA, aA, lB * aB);
            m_run = m;
            m_use = mu;
        }
    } else if constexpr (kGroups == 2 && kStageQ) {
        // Head dim 128: each group keeps O columns 64*grp .. +63 (blocks
        // 2*grp, 2*grp + 1) and hands the other half, with its max and sum, to
        // the same wave slot of the other group through its own tile
        // buffers (idle since the loop's last barrier): 8 blocks of [lane][4]
        // floats, then [lane] max and [lane] sum.  Both groups then merge and
        // store their half, so neither waits for the other to store all of O.
        // Both merge in one form, group 0's terms first, so the two halves of
        // a row share bit-identical max, sum and weights.
        float* mine = reinterpret_cast<float*>(smem_all + grp * D::kGroupBytes) + wave * 34 * kWave;
        const float* theirs = reinterpret_cast<const float*>(smem_all + (1 - grp) * D::kGroupBytes) + wave * 34 * kWave;
        f32x4_t* mw = reinterpret_cast<f32x4_t*>(mine) + lane;
        const f32x4_t* mr = reinterpret_cast<const f32x4_t*>(theirs) + lane;
        auto handoff = [&](auto od) {
            constexpr int o = decltype(od)::value;
#pragma unroll
            for (int k = 0; k < 2; ++k)
#pragma unroll
                for (int i4 = 0; i4 < 4; ++i4)
                    mw[(k * 4 + i4) * kWave] = f32x4_t{oacc[o + k][4 * i4], oacc[o + k][4 * i4 + 1],
                                                       oacc[o + k][4 * i4 + 2], oacc[o + k][4 * i4 + 3]};
        };
        if (grp == 0) handoff(std::integral_constant<int, 2>{});
        else handoff(std::integral_constant<int, 0>{});
        mine[32 * kWave + lane] = m_run;
        mine[33 * kWave + lane] = l_run;
        __syncthreads();
        const float m_o = theirs[32 * kWave + lane];
        const float l_o = theirs[33 * kWave + lane];
        const float mA = grp == 0 ? m_run : m_o, lA = grp == 0 ? l_run : l_o;   // group 0's
        const float mB = grp == 0 ? m_o : m_run, lB = grp == 0 ? l_o : l_run;   // group 1's
        const float m = fmaxf(mA, mB);
        const float mu = (m == -INFINITY) ? 0.f : m;
        const float aA = fast_exp2(mA - mu);   // 0 when a group saw no key
        const float aB = fast_exp2(mB - mu);
        auto merge_half = [&](auto kd) {
            constexpr int o = decltype(kd)::value;
#pragma unroll
            for (int k = 0; k < 2; ++k)
#pragma unroll
                for (int i4 = 0; i4 < 4; ++i4) {
                    const f32x4_t other = mr[(k * 4 + i4) * kWave];
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        const float own = oacc[o + k][4 * i4 + e];
                        const float oa = grp == 0 ? own : other[e], ob = grp == 0 ? other[e] : own;
                        oacc[o + k][4 * i4 + e] = __builtin_fmaf(oa, aA, ob * aB);
                    }
                }
        };
        if (grp == 0) merge_half(std::integral_constant<int, 0>{});
        else merge_half(std::integral_constant<int, 2>{});
        l_run = __builtin_fmaf(lA, aA, lB * aB);
        m_run = m;
        m_use = mu;
    } else if constexpr (kGroups == 2) {
        // Group 1 hands its partial state to group 0 (same wave slot, same lane)
        // through the tile buffers, idle since the loop's last barrier: per
        // wave, 16 blocks of [lane][4] O values (one 16-byte access per lane
        // and block), then [lane] max and [lane] sum.
        float* mg = reinterpret_cast<float*>(smem_all) + wave * kPfMergeFloats * kWave;
        f32x4_t* mo = reinterpret_cast<f32x4_t*>(mg) + lane;
        if (grp == 1) {
#pragma unroll
            for (int db = 0; db < 4; ++db)
#pragma unroll
                for (int i4 = 0; i4 < 4; ++i4)
                    mo[(db * 4 + i4) * kWave] = f32x4_t{oacc[db][4 * i4], oacc[db][4 * i4 + 1],
                                                        oacc[db][4 * i4 + 2], oacc[db][4 * i4 + 3]};
            mg[64 * kWave + lane] = m_run;
            mg[65 * kWave + lane] = l_run;
        }
        __syncthreads();
        if (grp == 1) return;
        const float m1 = mg[64 * kWave + lane];
        const float l1 = mg[65 * kWave + lane];
        const float m = fmaxf(m_run, m1);
        const float mu = (m == -INFINITY) ? 0.f : m;
        const float a0 = fast_exp2(m_run - mu);   // 0 when a group saw no key
        const float a1 = fast_exp2(m1 - mu);
#pragma unroll
        for (int db = 0; db < 4; ++db)
#pragma unroll
            for (int i4 = 0; i4 < 4; ++i4) {
                const f32x4_t o1 = mo[(db * 4 + i4) * kWave];
#pragma unroll
                for (int e = 0; e < 4; ++e) oacc[db][4 * i4 + e] = oacc[db][4 * i4 + e] * a0 + o1[e] * a1;
            }
        l_run = l_run * a0 + l1 * a1;
        m_run = m;
        m_use = mu;   // O and the sum are now relative to mu (the sink term uses it)
    }

    l_run = half_sum(l_run);
    // the sink joins the denominator relative to the same reference max:
    // sum exp(x - m) + sink * exp(-m)  (flash_swa_kernel.py:142-147)
    const bool has_sink = kSwa && p.sink != nullptr;
    const float sink = has_sink ? p.sink[h] : 0.f;
    const float denom = (l_run > 0.f && has_sink) ? l_run + sink * fast_exp2(-m_use) : l_run;
    const float inv = (l_run > 0.f) ? 1.f / denom : 0.f;
    if constexpr (kGroups == 2 && kStageQ && !kWide) {
        // this group's 64 columns of the wave's 32 rows go out through 4 KB of
        // the (idle) Q area: 8-byte pieces into 128-byte half rows, chunk c of
        // row r in slot c ^ (r % 8), then 8 half rows per store instruction
        unsigned char* ol = smem_all + 2 * D::kGroupBytes + (grp * kPfWaves + wave) * 4096;
        auto stage = [&](auto kd) {
            constexpr int o = decltype(kd)::value;
#pragma unroll
            for (int k = 0; k < 2; ++k)
#pragma unroll
                for (int i4 = 0; i4 < 4; ++i4) {
                    bf16x4_t w;
#pragma unroll
                    for (int e = 0; e < 4; ++e) w[e] = (__bf16)(oacc[o + k][i4 * 4 + e] * inv);
                    *reinterpret_cast<bf16x4_t*>(ol + l32 * 128 + (((4 * k + i4) ^ (l32 & 7)) << 4) + g2 * 8) = w;
                }
        };
        if (grp == 0) stage(std::integral_constant<int, 0>{});
        else stage(std::integral_constant<int, 2>{});
        // this wave's LDS writes complete before its reads (no other wave uses the area)
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int r = 8 * i + (lane >> 3);
            const int cc = lane & 7;
            const u32x4_t v = *reinterpret_cast<const u32x4_t*>(ol + r * 128 + ((cc ^ (r & 7)) << 4));
            if (q0w + r < p.sq) {
                __bf16* orow = p.o + b * p.o_sb + (int64_t)(q0w + r) * p.o_ss + h * p.o_sh;
                *reinterpret_cast<u32x4_t*>(orow + 64 * grp + 8 * cc) = v;
            }
        }
        if (grp == 1) return;   // group 0 writes the LSE
    } else {
        // O goes out through 8 KB of idle LDS per wave (the split kernel: the
        // wave's Q area, or with head dim 192 group 1's tile buffers, past the
        // merge area; the whole-range kernel: its tile buffers, which every
        // wave has finished reading at the loop's last barrier):
        // 8-byte pieces in (row l32, chunk 4*db + i4, half g2), then whole
        // 256-byte rows, 4 per store instruction (the accumulator layout would
        // give each store 32 rows 16 bytes each).
        static_assert(kGroups == 1 || kStageQ || kPfWaves * kPfMergeFloats * kWave * 4 <= D::kGroupBytes,
                      "O staging in group 1's buffers must not overlap the merge area");
        unsigned char* ol = kWide ? smem_all + (kStageQ ? kPwTileBytes : 0) + wave_wg * (kPfQStageBytes / kPfWaves)
                                  : smem_all + (kGroups == 1 ? 0 : kStageQ ? 2 : 1) * D::kGroupBytes +
                                        wave * (kPfQStageBytes / kPfWaves);
#pragma unroll
        for (int db = 0; db < 4; ++db)
#pragma unroll
            for (int i4 = 0; i4 < 4; ++i4) {
                bf16x4_t w;
#pragma unroll
                for (int e = 0; e < 4; ++e) w[e] = (__bf16)(oacc[db][i4 * 4 + e] * inv);
                *reinterpret_cast<bf16x4_t*>(ol + l32 * kPfVRowBytes + (((4 * db + i4) ^ (l32 & 15)) << 4) + g2 * 8) = w;
            }
        // this wave's LDS writes complete before its reads (no other wave uses the area)
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const int r = 4 * i + (lane >> 4);
            const u32x4_t v = *reinterpret_cast<const u32x4_t*>(ol + r * kPfVRowBytes + (l16 << 4));
            if (q0w + r < p.sq) {
                __bf16* orow = p.o + b * p.o_sb + (int64_t)(q0w + r) * p.o_ss + h * p.o_sh;
                *reinterpret_cast<u32x4_t*>(orow + ((l16 ^ (r & 15)) << 3)) = v;
            }
        }
    }
    if (qrow < p.sq) {
        if (p.lse != nullptr && g2 == 0)
            p.lse[((int64_t)b * p.hq + h) * p.sq + qrow] =
                (l_run > 0.f) ? m_run * kLn2 + logf(denom)
                              : (has_sink ? logf(fmaxf(sink, 1.0e-9f)) : -INFINITY);
    }
}

// (Q/K head dim 256: 96 KB of tile buffers, one workgroup per CU, so each
// wave may hold up to 512 registers.)
template <bool kSwa, int kDk>
__global__ __launch_bounds__(kPfThreads, kDk == 256 ? 1 : 2) void prefill_kernel(PrefillParams p) {
    extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
    int qb, hg, kvh, b;
    pf_rank_unit(p, blockIdx.x, &qb, &hg, &kvh, &b);
    pf_unit<1, kSwa, kDk>(p, smem, qb, hg, kvh, b);
}

// Persistent: gridDim.x = min(units, CUs) workgroups, one per CU.  Workgroup
// w runs ranks w, 2G-1-w, 2G+w, 4G-1-w, ... (G = gridDim.x): each lap over
// the heaviest-first ranks goes the other way, so every CU's units add up to
// about the same number of tiles (under a causal mask a rank-r unit plus a
// rank 2G-1-r unit hold as many tiles as any other such pair), and a CU moves
// to its next unit without a round trip through the dispatcher.
template <int kDk>
__global__ __launch_bounds__(2 * kPfThreads, 1) void prefill_split_kernel(PrefillParams p0) {
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
        pf_unit<2, false, kDk>(p, smem, qb, hg, kvh, b);
    }
}

// Wide kernel (head dim 128, no window or sink): 256-row units whose two wave
// groups take 128 rows each and share every K/V tile, so a CU loads half the
// tile bytes per row of the split kernel.  There are half as many units as
// the split kernel's, too few to balance whole units over the CUs: units pair
// heaviest with lightest (rank r with rank units - 1 - r), and a pair runs on
// two workgroups of one XCD (blocks w and w + 8; blocks go round-robin over
// the 8 XCDs).  The first runs the heavy unit's first tiles; the second the
// rest of the heavy unit and then the light unit.  The first keeps wide_bias
// tiles beyond half the pair's tiles, which pays for the second's extra unit
// start.  The heavy unit's two partial results merge through device memory
// (pf_unit: whichever segment finishes second merges).
template <bool kSwa, int kDk>
__global__ __launch_bounds__(2 * kPfThreads, 1) void prefill_wide_kernel(PrefillParams p0) {
    extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
    const int w = blockIdx.x;
    const int role = (w >> 3) & 1;
    const int pair = ((w >> 4) << 3) | (w & 7);
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
        // the first workgroup's share of the heavy unit
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
        pf_unit<2, kSwa, kDk, true>(p, smem, qb, hg, kvh, b, seg);
    }
}

// Wide kernel for grids with more unit pairs than the split form holds:
// persistent, one workgroup per CU; workgroup w runs ranks w, 2G-1-w, 2G+w,
// ... (G = gridDim.x) of the heaviest-first order as whole units, so each
// lap goes the other way and every CU's units add up to about the same
// number of tiles.
template <bool kSwa, int kDk>
__global__ __launch_bounds__(2 * kPfThreads, 1) void prefill_wide_persistent_kernel(PrefillParams p0) {
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
        pf_unit<2, kSwa, kDk, true>(p, smem, qb, hg, kvh, b, seg);
    }
}

// Merge scratch of the kernels that split a unit's KV range over two
// workgroups, in the layout of a caller workspace: the arrival counters (4
// words per unit pair) in the first FGQA_PREFILL_WORKSPACE_ZERO_BYTES, then
// two partial-result slots per pair (plan::merge_scratch_bytes_for).

// The library's merge scratch for calls that pass no workspace (kPwMaxSplit
// pairs; held by every device the library runs on until the process ends; the
// counters start at 0 and each launch leaves them at 0).  In host code the
// name is a host-side stand-in, not a device address: the address is looked
// up once per device (hipGetSymbolAddress, with that device current) and only
// that pointer is passed to kernels.  Launches that overlap on one device
// share it and would race: such callers pass workspaces of their own.
static __device__ __align__(256) unsigned char pw_scratch_mem[plan::merge_scratch_bytes_for(kPwMaxSplit)];

namespace {

constexpr int kPwDevices = 64;
std::mutex g_pw_mutex;
unsigned char* g_pw_scratch[kPwDevices] = {nullptr};

// The current device's copy of pw_scratch_mem.
int pw_scratch(unsigned char** mem) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kPwDevices) return FGQA_ERR_HIP;
    std::lock_guard<std::mutex> lock(g_pw_mutex);
    if (g_pw_scratch[dev] == nullptr) {
        void* pp = nullptr;
        if (hipGetSymbolAddress(&pp, HIP_SYMBOL(pw_scratch_mem)) != hipSuccess || pp == nullptr)
            return FGQA_ERR_HIP;
        g_pw_scratch[dev] = static_cast<unsigned char*>(pp);
    }
    *mem = g_pw_scratch[dev];
    return FGQA_OK;
}

using plan::tall_on_pairs;
using plan::wide_on_pairs;
using plan::wide_pairs;

}  // namespace

// Head dims the kernels are not built for: rows of D elements (at b/s/h
// strides) -> contiguous zero-padded rows of 8 << wlog2 elements (128, 192
// or 256: pieces per row 16, 24 or 32, `ppr`).  A thread per 16-byte piece
// of a padded row (grid-stride); 2-byte reads, so the source needs no
// alignment.
__global__ __launch_bounds__(256) void pad_rows_kernel(const __bf16* src, int64_t sb, int64_t ss, int64_t sh, int S,
                                                       int H, int D, int ppr, __bf16* dst, int64_t pieces) {
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < pieces; i += (int64_t)gridDim.x * blockDim.x) {
        const int64_t row = i / ppr;
        const int c = (int)(i - row * ppr) * 8;
        const int h = (int)(row % H);
        const int64_t t = row / H;
        const __bf16* r = src + (t / S) * sb + (t % S) * ss + h * sh;
        bf16x8_t v;
#pragma unroll
        for (int j = 0; j < 8; ++j) v[j] = (c + j < D) ? r[c + j] : (__bf16)0.f;
        *reinterpret_cast<bf16x8_t*>(dst + row * (8 * ppr) + c) = v;
    }
}

// The first D columns of contiguous rows of 8 * ppr elements -> rows at
// b/s/h strides.
__global__ __launch_bounds__(256) void unpad_rows_kernel(const __bf16* src, int ppr, __bf16* dst, int64_t db,
                                                         int64_t ds, int64_t dh, int S, int H, int D, int64_t pieces) {
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < pieces; i += (int64_t)gridDim.x * blockDim.x) {
        const int64_t row = i / ppr;
        const int c = (int)(i - row * ppr) * 8;
        if (c >= D) continue;
        const int h = (int)(row % H);
        const int64_t t = row / H;
        __bf16* r = dst + (t / S) * db + (t % S) * ds + h * dh;
        const bf16x8_t v = *reinterpret_cast<const bf16x8_t*>(src + row * (8 * ppr) + c);
#pragma unroll
        for (int j = 0; j < 8; ++j)
            if (c + j < D) r[c + j] = v[j];
    }
}

// Grid of the copy kernels: a thread per piece, at most 2^16 workgroups.
inline unsigned copy_grid(int64_t pieces) { return (unsigned)(ceil_div(pieces, 256) < 65536 ? ceil_div(pieces, 256) : 65536); }

void launch_pad_rows(const void* src, const int64_t* st, int B, int S, int H, int D, int width, void* dst,
                     hipStream_t s) {
    const int64_t pieces = (int64_t)B * S * H * (width / 8);
    if (pieces == 0) return;
    hipLaunchKernelGGL(pad_rows_kernel, dim3(copy_grid(pieces)), dim3(256), 0, s, static_cast<const __bf16*>(src),
                       st[0], st[1], st[2], S, H, D, width / 8, static_cast<__bf16*>(dst), pieces);
}

void launch_unpad_rows(const void* src, int width, void* dst, const int64_t* st, int B, int S, int H, int D,
                       hipStream_t s) {
    const int64_t pieces = (int64_t)B * S * H * (width / 8);
    if (pieces == 0) return;
    hipLaunchKernelGGL(unpad_rows_kernel, dim3(copy_grid(pieces)), dim3(256), 0, s, static_cast<const __bf16*>(src),
                       width / 8, static_cast<__bf16*>(dst), st[0], st[1], st[2], S, H, D, pieces);
}

namespace {

// The launches of a validated (128, 128) or MLA call.
int prefill_launch(const fgqa_prefill_args* a, hipStream_t s);

// Head dims the kernels are not built for (plan::prefill_padded): pad, run
// the built kernels on the copies (once per 128 columns of V), unpad O.  The
// copies live in the caller's workspace after the merge scratch, or with
// none in the library's cached buffer (the merge scratch then being the
// library's per-device one).
int prefill_padded_launch(const fgqa_prefill_args* a, hipStream_t s) {
    const int cus = device_cu_count();
    if (cus <= 0) return FGQA_ERR_HIP;
    fgqa_prefill_args pa = plan::padded_args(a);
    const size_t merge = plan::merge_scratch_bytes(&pa, plan::prefill_choice(&pa, cus), cus);
    const plan::PadLayout L = plan::pad_layout(a, merge);
    std::unique_lock<std::mutex> lock;
    unsigned char* base = nullptr;   // the copies: base + L.q .. base + L.total
    unsigned char* ws = static_cast<unsigned char*>(a->workspace);
    if (ws == nullptr && a->workspace_bytes == 0) {
        lock = workspace_lock();
        int st = FGQA_OK;
        unsigned char* buf = static_cast<unsigned char*>(internal_workspace(L.total - L.q, &st));
        if (st != FGQA_OK) return st;
        base = buf - L.q;
    } else if (ws == nullptr || a->workspace_bytes < L.total) {
        return FGQA_ERR_WORKSPACE;
    } else if ((reinterpret_cast<uintptr_t>(ws) & 255u) != 0) {
        return FGQA_ERR_UNSUPPORTED;
    } else {
        base = ws;
        if (merge > 0) {
            pa.workspace = ws;
            pa.workspace_bytes = merge;
        }
    }
    __bf16* qp = reinterpret_cast<__bf16*>(base + L.q);
    __bf16* kp = reinterpret_cast<__bf16*>(base + L.k);
    __bf16* vp = reinterpret_cast<__bf16*>(base + L.v);
    __bf16* op = reinterpret_cast<__bf16*>(base + L.o);
    const int dv = a->head_dim_v == 0 ? a->head_dim : a->head_dim_v;
    const int dkp = plan::padded_dk(a), dvp = plan::padded_dv(a);
    launch_pad_rows(a->q, a->q_stride, a->batch, a->seqlen_q, a->num_q_heads, a->head_dim, dkp, qp, s);
    launch_pad_rows(a->k, a->k_stride, a->batch, a->seqlen_kv, a->num_kv_heads, a->head_dim, dkp, kp, s);
    launch_pad_rows(a->v, a->v_stride, a->batch, a->seqlen_kv, a->num_kv_heads, dv, dvp, vp, s);
    if (hipGetLastError() != hipSuccess) return FGQA_ERR_HIP;
    pa.q = qp;
    pa.k = kp;
    // V / O rows of 256: a launch per 128 columns (each recomputes the
    // scores and writes the same LSE)
    for (int c0 = 0; c0 < dvp; c0 += kHeadDim) {
        pa.v = vp + c0;
        pa.o = op + c0;
        if (const int st = prefill_launch(&pa, s); st != FGQA_OK) return st;
    }
    launch_unpad_rows(op, dvp, a->o, a->o_stride, a->batch, a->seqlen_q, a->num_q_heads, dv, s);
    if (hipGetLastError() != hipSuccess) return FGQA_ERR_HIP;
    return FGQA_OK;
}

}  // namespace
}  // namespace fgqa

using namespace fgqa;

extern "C" int fgqa_prefill_kernel_choice(const fgqa_prefill_args* a, int32_t* kernel) {
    int st = plan::validate_prefill(a);
    if (st != FGQA_OK) return st;
    if (kernel == nullptr) return FGQA_ERR_INVALID_ARGUMENT;
    const int cus = device_cu_count();
    if (cus <= 0) return FGQA_ERR_HIP;
    const fgqa_prefill_args pa = plan::prefill_padded(a) ? plan::padded_args(a) : *a;
    *kernel = plan::prefill_choice(&pa, cus);
    return FGQA_OK;
}

extern "C" int fgqa_prefill_kernel_name(const fgqa_prefill_args* a, const char** name) {
    int st = plan::validate_prefill(a);
    if (st != FGQA_OK) return st;
    if (name == nullptr) return FGQA_ERR_INVALID_ARGUMENT;
    const int cus = device_cu_count();
    if (cus <= 0) return FGQA_ERR_HIP;
    const fgqa_prefill_args pa = plan::prefill_padded(a) ? plan::padded_args(a) : *a;
    *name = plan::prefill_kernel_name(&pa, cus);
    return FGQA_OK;
}

extern "C" int fgqa_prefill_workspace_bytes(const fgqa_prefill_args* a, size_t* bytes) {
    int st = plan::validate_prefill(a);
    if (st != FGQA_OK) return st;
    if (bytes == nullptr) return FGQA_ERR_INVALID_ARGUMENT;
    const int cus = device_cu_count();
    if (cus <= 0) return FGQA_ERR_HIP;
    *bytes = plan::prefill_workspace_bytes(a, cus);
    return FGQA_OK;
}

extern "C" int fgqa_prefill_bf16(const fgqa_prefill_args* a, void* stream) {
    int st = plan::validate_prefill(a);
    if (st != FGQA_OK) return st;
    if (a->batch == 0 || a->seqlen_q == 0) return FGQA_OK;
    const hipStream_t s = static_cast<hipStream_t>(stream);
    return plan::prefill_padded(a) ? prefill_padded_launch(a, s) : prefill_launch(a, s);
}

namespace fgqa {
namespace {

int prefill_launch(const fgqa_prefill_args* a, hipStream_t s) {
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
    p.hb_log2 = p.hb == 4 ? 2 : p.hb == 2 ? 1 : 0;
    p.n_hgroups = p.group / p.hb;
    p.n_qblocks = (int)ceil_div(p.sq, 128 / p.hb);
    p.n_streams = p.n_hgroups * p.hkv * p.batch;
    p.div_streams = make_fast_div(p.n_streams);
    p.div_hgroups = make_fast_div(p.n_hgroups);
    p.div_hkv = make_fast_div(p.hkv);
    p.scale_log2 = fabsf(a->scale) * kLog2e;
    p.q_sign = (a->scale < 0.f) ? 0x80008000u : 0u;
    p.window = a->window_size;
    p.sink = a->sink;
    p.wide_bias = 0;
    p.wide_part = nullptr;
    p.wide_ctr = nullptr;

    const int64_t units = (int64_t)p.n_qblocks * p.n_streams;
    if (units >= ((int64_t)1 << 31)) return FGQA_ERR_UNSUPPORTED;
    const int cus = device_cu_count();
    if (cus <= 0) return FGQA_ERR_HIP;
    const int choice = plan::prefill_choice(a, cus);
    // merge scratch: the caller's workspace, or with none the library's
    if (const size_t need = plan::merge_scratch_bytes(a, choice, cus); need > 0) {
        unsigned char* ws = static_cast<unsigned char*>(a->workspace);
        if (ws == nullptr && a->workspace_bytes == 0) {
            if (const int e = pw_scratch(&ws); e != FGQA_OK) return e;
        } else if (ws == nullptr || a->workspace_bytes < need) {
            return FGQA_ERR_WORKSPACE;
        } else if ((reinterpret_cast<uintptr_t>(ws) & 255u) != 0) {
            return FGQA_ERR_UNSUPPORTED;
        }
        p.wide_ctr = reinterpret_cast<unsigned*>(ws);
        p.wide_part = reinterpret_cast<float*>(ws + FGQA_PREFILL_WORKSPACE_ZERO_BYTES);
    }
    const bool swa = p.window > 0 || p.sink != nullptr;
    const bool mla = a->head_dim == 192;
    const bool split = choice == FGQA_KERNEL_SPLIT;
    if (a->head_dim == 256) {
        // Q/K head dim 256: the whole-range kernel (the plan refuses the
        // other shapes); attribute slots 22, 23
        const int sm = PfDims<256>::kGroupBytes;
        const void* fn = swa ? reinterpret_cast<const void*>(prefill_kernel<true, 256>)
                             : reinterpret_cast<const void*>(prefill_kernel<false, 256>);
        if (const int e = set_kernel_smem_once(swa ? 23 : 22, fn, sm); e != FGQA_OK) return e;
        if (swa) hipLaunchKernelGGL((prefill_kernel<true, 256>), dim3((unsigned)units), dim3(kPfThreads), sm, s, p);
        else hipLaunchKernelGGL((prefill_kernel<false, 256>), dim3((unsigned)units), dim3(kPfThreads), sm, s, p);
        if (hipGetLastError() != hipSuccess) return FGQA_ERR_HIP;
        return FGQA_OK;
    }
    if (choice == FGQA_KERNEL_WIDE || choice == FGQA_KERNEL_TALL) {
        // 256-row units: up to 8 heads of a KV group
        const int hbw = (p.group % 8 == 0) ? 8 : p.hb;
        p.hb = hbw;
        p.hb_log2 = hbw == 8 ? 3 : hbw == 4 ? 2 : hbw == 2 ? 1 : 0;
        p.n_hgroups = p.group / hbw;
        p.n_qblocks = (int)ceil_div(p.sq, 256 / hbw);
        p.n_streams = p.n_hgroups * p.hkv * p.batch;
        p.div_streams = make_fast_div(p.n_streams);
        p.div_hgroups = make_fast_div(p.n_hgroups);
        p.wide_bias = 3;
        if (choice == FGQA_KERNEL_TALL) return launch_prefill_tall(p, tall_on_pairs(a, cus), cus, s);
        if (!wide_on_pairs(a, cus)) {
            // more pairs than one per two CUs: whole units on a persistent grid
            // attribute slots 7, 8, 9: the persistent wide kernels (plain, window, MLA)
            const int slot = mla ? 9 : swa ? 8 : 7;
            const void* pfn = mla   ? reinterpret_cast<const void*>(prefill_wide_persistent_kernel<false, 192>)
                              : swa ? reinterpret_cast<const void*>(prefill_wide_persistent_kernel<true, kHeadDim>)
                                    : reinterpret_cast<const void*>(prefill_wide_persistent_kernel<false, kHeadDim>);
            const int sm = pw_smem_bytes(a->head_dim);
            if (const int e = set_kernel_smem_once(slot, pfn, sm); e != FGQA_OK) return e;
            const int64_t units_w = (int64_t)p.n_qblocks * p.n_streams;
            const dim3 grid((unsigned)(units_w < cus ? units_w : cus));
            if (mla) hipLaunchKernelGGL((prefill_wide_persistent_kernel<false, 192>), grid, dim3(2 * kPfThreads), sm, s, p);
            else if (swa) hipLaunchKernelGGL((prefill_wide_persistent_kernel<true, kHeadDim>), grid, dim3(2 * kPfThreads), sm, s, p);
            else hipLaunchKernelGGL((prefill_wide_persistent_kernel<false, kHeadDim>), grid, dim3(2 * kPfThreads), sm, s, p);
            if (hipGetLastError() != hipSuccess) return FGQA_ERR_HIP;
            return FGQA_OK;
        }
        // attribute slots 5, 6: the wide kernels
        // attribute slots 5, 6, 18: the wide kernels (plain, window, MLA)
        const int wslot = mla ? 18 : swa ? 6 : 5;
        const void* wfn = mla   ? reinterpret_cast<const void*>(prefill_wide_kernel<false, 192>)
                          : swa ? reinterpret_cast<const void*>(prefill_wide_kernel<true, kHeadDim>)
                                : reinterpret_cast<const void*>(prefill_wide_kernel<false, kHeadDim>);
        const int wsm = pw_smem_bytes(a->head_dim);
        if (const int e = set_kernel_smem_once(wslot, wfn, wsm); e != FGQA_OK) return e;
        // blocks w and w + 8 of each 16 run one pair
        const dim3 grid((unsigned)(16 * ceil_div(wide_pairs(a), 8)));
        if (mla) hipLaunchKernelGGL((prefill_wide_kernel<false, 192>), grid, dim3(2 * kPfThreads), wsm, s, p);
        else if (swa) hipLaunchKernelGGL((prefill_wide_kernel<true, kHeadDim>), grid, dim3(2 * kPfThreads), wsm, s, p);
        else hipLaunchKernelGGL((prefill_wide_kernel<false, kHeadDim>), grid, dim3(2 * kPfThreads), wsm, s, p);
        if (hipGetLastError() != hipSuccess) return FGQA_ERR_HIP;
        return FGQA_OK;
    }

    const int group_bytes = mla ? PfDims<192>::kGroupBytes : PfDims<128>::kGroupBytes;
    // the split kernel with head dim 128 also stages the Q tile in LDS
    const int smem_bytes = (split ? 2 : 1) * group_bytes + (split && !mla ? kPfQStageBytes : 0);
    // kernel table: plain, window / sink, split, MLA, MLA split
    const int which = mla ? (split ? 4 : 3) : (split ? 2 : (swa ? 1 : 0));
    const void* fns[5] = {reinterpret_cast<const void*>(prefill_kernel<false, 128>),
                          reinterpret_cast<const void*>(prefill_kernel<true, 128>),
                          reinterpret_cast<const void*>(prefill_split_kernel<128>),
                          reinterpret_cast<const void*>(prefill_kernel<false, 192>),
                          reinterpret_cast<const void*>(prefill_split_kernel<192>)};
    // attribute slots 0..4: the prefill kernels
    if (const int e = set_kernel_smem_once(which, fns[which], smem_bytes); e != FGQA_OK) return e;
    // the split kernel is persistent: at most one workgroup per CU
    const dim3 grid((unsigned)(split && units > cus ? cus : units));
    switch (which) {
        case 0: hipLaunchKernelGGL((prefill_kernel<false, 128>), grid, dim3(kPfThreads), smem_bytes, s, p); break;
        case 1: hipLaunchKernelGGL((prefill_kernel<true, 128>), grid, dim3(kPfThreads), smem_bytes, s, p); break;
        case 2: hipLaunchKernelGGL(prefill_split_kernel<128>, grid, dim3(2 * kPfThreads), smem_bytes, s, p); break;
        case 3: hipLaunchKernelGGL((prefill_kernel<false, 192>), grid, dim3(kPfThreads), smem_bytes, s, p); break;
        default: hipLaunchKernelGGL(prefill_split_kernel<192>, grid, dim3(2 * kPfThreads), smem_bytes, s, p); break;
    }
    if (hipGetLastError() != hipSuccess) return FGQA_ERR_HIP;
    return FGQA_OK;
}

}  // namespace
}  // namespace fgqa
