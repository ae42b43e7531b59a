// Flash attention (forward and backward) for gfx950 with bf16 MFMA.
//
// Operand layouts and the transposed LDS reads are described in fx_mfma.h.
// Accumulator tiles are reused as the next product's operand without any shuffle:
// the 16 values a lane holds for one column are packed as the operand's 8 K-values
// of two 16-wide K chunks, and the other operand's K order is permuted to match
// (positions j < 4 -> 4*g + j, j >= 4 -> 8 + 4*g + j - 4, g = l/32).
//
// Forward: "transposed" scores S^T = K Q^T so each lane owns one query column and the
// row softmax is 15 in-lane steps plus one exchange with lane l^32.
// Backward: per query tile, S^T, dP^T and dQ^T = K^T dS^T (Delta computed in the same
// kernel); per key tile, S = Q K^T, dP = dO V^T, dV^T += dO^T P, dK^T += Q^T dS.
// The softmax scale of dS is applied once to dQ / dK at the end.
// Semantics follow ml/fxlm/kernels/attention.hip:103-534 (mask key <= query, lse =
// m + log l or -inf, Delta from the bf16 output, dS = P (dP - Delta) scale).
//
// Each tile's MFMA operands are read from LDS up front and the independent
// accumulator chains are interleaved, so LDS latency and MFMA dependencies overlap.
// K/V (Q/dO) tiles are double-buffered in LDS and filled by direct global -> LDS
// loads that are in flight during the previous tile's math (one barrier per tile).
#include <math.h>

#include "fx_mfma.h"

namespace fx {

constexpr int kAttWaves = 4;
constexpr int kAttThreads = 64 * kAttWaves;
constexpr int kBM = 32 * kAttWaves;  // queries per workgroup (forward, dQ)
constexpr int kBN = 64;              // keys per streamed tile (forward, dQ)
constexpr int kBK = 32 * kAttWaves;  // keys per workgroup (dK/dV)
constexpr int kBQ = 64;              // queries per streamed tile (dK/dV)
constexpr float kNegInfA = -__builtin_huge_valf();

// Lazy rescaling (forward): the running max only moves when a row's new max exceeds
// it by more than this (log2 units), so P stays <= 2^8 and most tiles skip the O rescale.
constexpr float kLazyRescale = 8.f;

__device__ __forceinline__ bf16x8 as_bf16x8(const uint4& v) { return __builtin_bit_cast(bf16x8, v); }

// v with every bit cleared unless keep is all ones (a per-lane zeroing by bitwise and: a
// select between two vectors can become a select between their addresses, which puts
// the vectors in scratch memory)
__device__ __forceinline__ uint4 mask16(const uint4& v, uint32_t keep) {
    return make_uint4(v.x & keep, v.y & keep, v.z & keep, v.w & keep);
}

// 8 fp32 accumulator values (elements 8h..8h+7) -> bf16x8 operand
__device__ __forceinline__ bf16x8 pack_op(const f32x16& c, int h) {
    const f32x8 v = h == 0 ? __builtin_shufflevector(c, c, 0, 1, 2, 3, 4, 5, 6, 7)
                           : __builtin_shufflevector(c, c, 8, 9, 10, 11, 12, 13, 14, 15);
    return __builtin_convertvector(v, bf16x8);
}

// row index (within a 32-row accumulator tile) of accumulator element i of lane l is
// acc_c(i) + 4 * (l / 32), acc_c(i) a compile-time constant once i is unrolled
__device__ __forceinline__ constexpr int acc_c(int i) { return 8 * (i >> 2) + (i & 3); }

// -inf into the elements whose row offset acc_c(i) lies outside [lo, hi] (one compare
// pair and one select per element; lo / hi already hold the lane's 4 * (l / 32) shift)
__device__ __forceinline__ void mask_rows(f32x16& x, int lo, int hi) {
#pragma unroll
    for (int i = 0; i < 16; ++i)
        if (acc_c(i) < lo || acc_c(i) > hi) x[i] = kNegInfA;
}

// 1-D grid over (tile rank, bh), rank-major: all heads' rank-0 tiles are dispatched
// first, so with ranks ordered by decreasing causal work the longest workgroups start
// first and the short ones fill the tail (bh-major order left heavy tiles of the last
// heads for the end: 63 -> 50 us at [16,12,1024,64] causal forward).  Workgroups are
// dealt round-robin to the 8 XCDs, so with nbh % 8 == 0 every tile of one head runs
// on the same XCD and shares its L2.
__device__ __forceinline__ void grid_map(int ntiles, int nbh, int& bh, int& tile) {
    (void)ntiles;
    const int x = blockIdx.x;
    tile = x / nbh;
    bh = x - tile * nbh;
}

// Store a wave's 32 x D output block held in the transposed accumulator layout
// (lane l: output row l % 32; elements 4r..4r+3 of tile dt are columns
// 32 dt + 8 r + 4 (l / 32) + 0..3), scaled by `mul` (per lane), to rows
// first + i * rs (i < nvalid).  The block goes through the wave's private LDS
// region `tmp` (32 x (D + 8) bf16) so that each lane then writes 16 contiguous bytes
// and eight lanes cover a 128-byte row; storing 8 bytes per lane straight from the
// accumulators spreads every instruction over 32 rows.  LDS operations of one wave
// complete in order, so no barrier is needed between the writes and the reads.
template <int D>
__device__ __forceinline__ void store_rows(const f32x16 (&acc)[D / 32], float mul, uint16_t* tmp,
                                           uint16_t* first, int64_t rs, int nvalid, int lane) {
    constexpr int LDT = D + 8;
    constexpr int CPR = D / 8;  // 16-byte chunks per row
    const int g = lane >> 5, ln = lane & 31;
#pragma unroll
    for (int dt = 0; dt < D / 32; ++dt)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            uint2 u;
            u.x = pack_bf16x2(acc[dt][4 * r + 0] * mul, acc[dt][4 * r + 1] * mul);
            u.y = pack_bf16x2(acc[dt][4 * r + 2] * mul, acc[dt][4 * r + 3] * mul);
            *reinterpret_cast<uint2*>(tmp + ln * LDT + 32 * dt + 8 * r + 4 * g) = u;
        }
#pragma unroll
    for (int c = 0; c < 32 * CPR / 64; ++c) {
        const int ch = c * 64 + lane;
        const int row = ch / CPR, col = (ch - row * CPR) * 8;
        if (row < nvalid) st16(first + row * rs + col, *reinterpret_cast<const uint4*>(tmp + row * LDT + col));
    }
}

// ---------------------------------------------------------------------------
// LDS layout of a streamed R x D tile.
//
// D = 64: unpadded 128-byte rows whose eight 16-byte chunks are permuted per row: logical
// chunk c of row r sits at chunk c ^ swz(r), swz(r) = bits 1, 2, 3 of r reversed.  Rows
// r and r + 1 differ in bank half, so among any 16 consecutive rows the 8 even ones (and
// the 8 odd ones) cover all 8 chunk positions: a row read (16 lanes, 16 consecutive rows,
// one chunk) is conflict-free; bit 2 of swz follows bit 1 of r, so the 4 rows of a
// transposed read (4 rows x 4 chunks per 32 lanes) fall in disjoint banks as well.
// Against the padded layout this drops one slot in nine from every tile load (the loads'
// cost grows faster than their byte count: half the loads measured a third of their cost)
// and the 2-way conflicts of the transposed reads.
// D = 128: row stride D + 8 elements (the pad keeps the operand reads conflict-free).
template <int D, bool SW>
struct TileLayout {
    static constexpr int LD = D + 8;       // row stride (elements)
    static constexpr int SPR = D / 8 + 1;  // 16-byte slots per row, the last one padding
    __device__ __forceinline__ static int off(int row, int col) { return row * LD + col; }
    // logical chunk held by slot `slot` of row `row` (the pad slot: any in-row chunk)
    __device__ __forceinline__ static int chunk(int row, int slot) { return slot == SPR - 1 ? SPR - 2 : slot; }
};
template <>
struct TileLayout<64, true> {
    static constexpr int LD = 64;
    static constexpr int SPR = 8;
    __device__ __forceinline__ static int swz(int row) {
        return (((row >> 1) & 1) << 2) | (((row >> 2) & 1) << 1) | ((row >> 3) & 1);
    }
    __device__ __forceinline__ static int off(int row, int col) {
        return row * 64 + ((((col >> 3) ^ swz(row)) << 3) | (col & 7));
    }
    __device__ __forceinline__ static int chunk(int row, int slot) { return slot ^ swz(row); }
};

// MFMA operands from a tile in this layout (see fx_mfma.h for the lane mappings): K along a
// row (8 contiguous elements of row r0 + l%32 at column c0 + 8 (l/32)), or K down the rows
// (two ds_read_b64_tr_b16; a lane's 4 columns never cross a 16-byte chunk).  The kernels
// only read at r0, k0 multiples of 16 (which leave swz unchanged) and c0, m0 multiples of
// 16 and 32, so for D = 64 each lane's offsets are a per-lane table plus a compile-time
// row offset (a per-lane swizzle computed at every read cost 10 VGPRs in the forward).
template <int D, bool SW>
struct TileLane {
    __device__ __forceinline__ void init(int) {}
    __device__ __forceinline__ int row(int r0, int c0, int lane) const {
        return TileLayout<D, SW>::off(r0 + (lane & 31), c0 + 8 * (lane >> 5));
    }
    __device__ __forceinline__ int tr(int k0, int m0, int h, int lane) const {
        const int grp = lane >> 4, s = lane & 15;
        return TileLayout<D, SW>::off(k0 + 4 * (grp >> 1) + (s >> 2) + 8 * h, m0 + 16 * (grp & 1) + 4 * (s & 3));
    }
};
template <>
struct TileLane<64, true> {
    int ro[4];     // row reads at c0 = 16 c, rows 0..31
    int to[2][2];  // transposed reads at m0 = 32 m, rows 0..7 (h = 0) or 8..15 (h = 1)
    __device__ __forceinline__ void init(int lane) {
        const int g = lane >> 5, l32 = lane & 31;
        const int p = g ^ TileLayout<64, true>::swz(l32);
#pragma unroll
        for (int c = 0; c < 4; ++c) ro[c] = l32 * 64 + (((2 * c) ^ p) << 3);
        const int grp = lane >> 4, s = lane & 15;
        const int rb = 4 * (grp >> 1) + (s >> 2);
        const int cl = 2 * (grp & 1) + ((s & 3) >> 1);
#pragma unroll
        for (int m = 0; m < 2; ++m)
#pragma unroll
            for (int h = 0; h < 2; ++h)
                to[m][h] = (rb + 8 * h) * 64 + ((((4 * m) ^ cl ^ TileLayout<64, true>::swz(rb) ^ h)) << 3) + 4 * (s & 1);
    }
    __device__ __forceinline__ int row(int r0, int c0, int) const { return r0 * 64 + ro[c0 >> 4]; }
    __device__ __forceinline__ int tr(int k0, int m0, int h, int) const { return k0 * 64 + to[m0 >> 5][h]; }
};
template <int D, bool SW>
__device__ __forceinline__ bf16x8 tile_op_row(const TileLane<D, SW>& tl, const uint16_t* tile, int r0, int c0, int lane) {
    if constexpr (SW) return *reinterpret_cast<const bf16x8*>(tile + tl.row(r0, c0, lane));
    else return lds_op_row(tile, TileLayout<D, SW>::LD, r0, c0, lane);
}
template <int D, bool SW>
__device__ __forceinline__ bf16x8 tile_op_t(const TileLane<D, SW>& tl, const uint16_t* tile, int k0, int m0, int lane) {
    if constexpr (SW) return cat8(lds_tr16(tile + tl.tr(k0, m0, 0, lane)), lds_tr16(tile + tl.tr(k0, m0, 1, lane)));
    else return lds_op_t(tile, TileLayout<D, SW>::LD, k0, m0, lane);
}

// ---------------------------------------------------------------------------
// Tile staging by direct global -> LDS loads (global_load_lds_dwordx4).
//
// A wave-wide global_load_lds writes 64 consecutive 16-byte LDS slots (lane i -> slot
// base + i), so a tile is covered slot by slot: slot s is slot s % SPR of row s / SPR and
// holds that row's logical chunk TileLayout::chunk(row, slot); rows past the end of the
// sequence read a zero line.  The loads need no registers and no LDS stores; they are
// complete once the issuing wave's vmcnt drains, and visible to the other waves after
// the following barrier.

// Two R x D tiles (K and V, or Q and dO) staged together: 2 * R * SPR / 64 wave
// instructions dealt round-robin to the workgroup's waves.
template <int D, int R, bool SW>
struct TileDma2 {
    static constexpr int SPR = TileLayout<D, SW>::SPR;
    static constexpr int NI = R * SPR / 64;  // wave instructions per tile
    static_assert(R * SPR % 64 == 0, "tile must be a whole number of wave loads");
    static constexpr int PW = (2 * NI + kAttWaves - 1) / kAttWaves;  // per wave, at most
    static_assert(4 * kAttWaves <= 2 * NI, "every wave issues at least four loads per tile pair");
    uint32_t off[PW];  // byte offset of this lane's chunk from the tile's first row
    int wave;
    // tile row and in-row chunk of this lane's slot in wave instruction i
    __device__ __forceinline__ static void slot(int i, int lane, int& r, int& c) {
        const int s = (i % NI) * 64 + lane;
        r = s / SPR;
        c = TileLayout<D, SW>::chunk(r, s - r * SPR);
    }
    __device__ __forceinline__ void init(int64_t rs0, int64_t rs1) {
        wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
        const int lane = threadIdx.x & 63;
#pragma unroll
        for (int k = 0; k < PW; ++k) {
            const int i = wave + k * kAttWaves;
            int r, c;
            slot(i, lane, r, c);
            off[k] = (uint32_t)(r * (i < NI ? rs0 : rs1) + c * 8) * 2u;
        }
    }
    // the source base and LDS destination of this wave's load k (wave-uniform)
    __device__ __forceinline__ void target(int k, const uint16_t* first0, const uint16_t* first1,
                                           const uint16_t* lds0, const uint16_t* lds1, const uint16_t*& base,
                                           uint32_t& dst) const {
        const int i = wave + k * kAttWaves;
        const bool second = i >= NI;
        base = second ? first1 : first0;
        dst = lds_addr((second ? lds1 : lds0) + (i - (second ? NI : 0)) * 64 * 8);
    }
    // first0/first1: the tiles' first rows in global memory; rows >= valid read zeros
    __device__ __forceinline__ void issue(const uint16_t* first0, const uint16_t* first1, int valid,
                                          const uint16_t* lds0, const uint16_t* lds1) const {
        const bool full = valid >= R;  // wave-uniform: every row of the tile exists
        if (full) {
            // straight-line: the first four loads of every wave exist (4 kAttWaves <= 2 NI)
            const uint16_t *b0, *b1, *b2, *b3;
            uint32_t d0, d1, d2, d3;
            target(0, first0, first1, lds0, lds1, b0, d0);
            target(1, first0, first1, lds0, lds1, b1, d1);
            target(2, first0, first1, lds0, lds1, b2, d2);
            target(3, first0, first1, lds0, lds1, b3, d3);
            dma16_so_x4(b0, off[0], d0, b1, off[1], d1, b2, off[2], d2, b3, off[3], d3);
#pragma unroll
            for (int k = 4; k < PW; ++k) {
                if (wave + k * kAttWaves < 2 * NI) {
                    const uint16_t* b;
                    uint32_t d;
                    target(k, first0, first1, lds0, lds1, b, d);
                    dma16_so(b, off[k], d);
                }
            }
            return;
        }
#pragma unroll
        for (int k = 0; k < PW; ++k) {
            const int i = wave + k * kAttWaves;
            if (i < 2 * NI) {
                const bool second = i >= NI;
                const uint16_t* base = second ? first1 : first0;
                const uint32_t dst = lds_addr((second ? lds1 : lds0) + (i - (second ? NI : 0)) * 64 * 8);
                if (full) {
                    dma16_so(base, off[k], dst);
                } else {
                    int r, c;
                    slot(i, threadIdx.x & 63, r, c);
                    const void* p = r < valid ? (const void*)((const char*)base + off[k])
                                              : (const void*)g_zero_line;
                    dma16(p, dst);
                }
            }
        }
    }
};

// ---------------------------------------------------------------------------
// forward

// max / sum over the two lanes l and l ^ 32 that hold the same query column: one
// v_permlane32_swap hands every lane both values (same operand order in both lanes,
// so both end with the same bits)
__device__ __forceinline__ float pair_max(float x) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float pair_sum(float x) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

template <int D>
__global__ void __launch_bounds__(kAttThreads) attn_fwd_kernel(fxAttnArgs a) {
    // padded tiles: the swizzle's per-lane offset table would take the forward past 128
    // VGPRs (3 waves per SIMD instead of 4), and its tile loads cost it little
    constexpr bool SW = false;
    constexpr int LD = TileLayout<D, SW>::LD;
    constexpr int DC = D / 16;  // K chunks of Q.K
    constexpr int DT = D / 32;  // 32-row tiles of O^T
    __shared__ __attribute__((aligned(16))) uint16_t sk0[kBN * LD], sk1[kBN * LD];
    __shared__ __attribute__((aligned(16))) uint16_t sv0[kBN * LD], sv1[kBN * LD];
    static_assert(32 * (D + 8) <= kBN * LD, "a stage buffer holds one wave's output staging");

    const int T = a.T;
    const int nqt = (T + kBM - 1) / kBM;
    int bh, qt;
    grid_map(nqt, a.B * a.H, bh, qt);
    qt = nqt - 1 - qt;  // longest causal tiles first
    const int b = bh / a.H, h = bh - b * a.H;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int g = lane >> 5, ln = lane & 31;
    TileLane<D, SW> tl;
    tl.init(lane);
    const int q0 = qt * kBM;
    const int q0w = q0 + 32 * wave;
    const int qi = q0w + ln;

    const uint16_t* kbase = a.k + b * a.ksb + h * a.ksh;
    const uint16_t* vbase = a.v + b * a.vsb + h * a.vsh;
    const int kend = a.causal ? min(T, q0 + kBM) : T;
    const int nblk = (kend + kBN - 1) / kBN;

    TileDma2<D, kBN, SW> dma;
    dma.init(a.kst, a.vst);
    dma.issue(kbase, vbase, T, sk0, sv0);
    // the next tile's first K and V rows, advanced by one tile per step
    const int64_t kstep = (int64_t)kBN * a.kst, vstep = (int64_t)kBN * a.vst;
    const uint16_t* kn = kbase;
    const uint16_t* vn = vbase;

    bf16x8 qop[DC];
    {
        const uint16_t* qrow = a.q + b * a.qsb + h * a.qsh + (int64_t)(qi < T ? qi : 0) * a.qst;
#pragma unroll
        for (int c = 0; c < DC; ++c) {
            uint4 v = make_uint4(0u, 0u, 0u, 0u);
            if (qi < T) v = ld16(qrow + 16 * c + 8 * g);
            qop[c] = as_bf16x8(v);
        }
    }

    const float sl2 = a.scale * kLog2e;
    float m_run = kNegInfA, l_run = 0.f;
    f32x16 acc[DT];
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) acc[dt] = f32x16{};

    // one 64-key tile: K/V in (K, V); the next tile's loads go to (nK, nV)
    auto step = [&](int j, const uint16_t* K, const uint16_t* V, uint16_t* nK, uint16_t* nV) {
        const int kb = j * kBN;
        tile_arrive();
        kn += kstep;
        vn += vstep;
        if (j + 1 < nblk) dma.issue(kn, vn, T - kb - kBN, nK, nV);
#pragma unroll
        for (int hh = 0; hh < 2; ++hh) {
            const int kh = kb + 32 * hh;  // first key of this half
            if (kh >= T || (a.causal && kh > q0w + 31)) continue;  // every key masked for this wave
            bf16x8 kop[DC];
#pragma unroll
            for (int c = 0; c < DC; ++c) kop[c] = tile_op_row(tl, K, 32 * hh, 16 * c, lane);
            f32x16 sc = f32x16{};
#pragma unroll
            for (int c = 0; c < DC; ++c) sc = mfma32(kop[c], qop[c], sc);
            bf16x8 vop[DT][2];
#pragma unroll
            for (int dt = 0; dt < DT; ++dt)
#pragma unroll
                for (int kc = 0; kc < 2; ++kc) vop[dt][kc] = tile_op_t(tl, V, 32 * hh + 16 * kc, 32 * dt, lane);
            if ((kh + 32 > T) || (a.causal && kh + 31 > q0w))  // keys past T or after the query
                mask_rows(sc, 0, (a.causal ? min(qi, T - 1) : T - 1) - kh - 4 * g);
            float mloc = sc[0];
#pragma unroll
            for (int i = 1; i < 16; ++i) mloc = fmaxf(mloc, sc[i]);
            mloc = pair_max(mloc);
            const float m_new = fmaxf(m_run, mloc * sl2);
            const bool need = m_new > m_run + kLazyRescale;
            // wave-uniform: the rescale (its exp, the l and O multiplies) only runs in the
            // rare tiles where some row's max moved
            const bool any_need = __ballot(need) != 0;
            float alpha = 1.f;
            if (any_need && need) {
                alpha = exp2_fast(m_run - m_new);
                m_run = m_new;
            }
            const float mu = (m_run == kNegInfA) ? 0.f : m_run;
            // row sum in four partial sums, each started from its first term (no adds of 0)
            float r4[4];
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                const float p = exp2_fast(fmaf(sc[i], sl2, -mu));
                sc[i] = p;
                if (i < 4) r4[i] = p;
                else r4[i & 3] += p;
            }
            const float rs = (r4[0] + r4[1]) + (r4[2] + r4[3]);
            if (any_need) {
                l_run = l_run * alpha + rs;
#pragma unroll
                for (int dt = 0; dt < DT; ++dt)
#pragma unroll
                    for (int i = 0; i < 16; ++i) acc[dt][i] *= alpha;
            } else {
                l_run += rs;
            }
            const bf16x8 p0 = pack_op(sc, 0), p1 = pack_op(sc, 1);
#pragma unroll
            for (int dt = 0; dt < DT; ++dt) {
                acc[dt] = mfma32(vop[dt][0], p0, acc[dt]);
                acc[dt] = mfma32(vop[dt][1], p1, acc[dt]);
            }
        }
    };
    // stages alternate with the tile parity; unrolled by two so that each LDS access
    // names its stage array
    for (int j = 0; j < nblk; j += 2) {
        step(j, sk0, sv0, sk1, sv1);
        if (j + 1 < nblk) step(j + 1, sk1, sv1, sk0, sv0);
    }

    const float l_tot = pair_sum(l_run);
    if (qi < T && g == 0)
        a.lse_out[(int64_t)bh * T + qi] = l_tot > 0.f ? (m_run + log2_fast(l_tot)) * kLn2 : kNegInfA;
    __syncthreads();  // every wave is done with the K/V stages: they become store scratch
    store_rows<D>(acc, l_tot > 0.f ? 1.f / l_tot : 0.f, (wave < 2 ? sk0 : sk1) + (wave & 1) * 32 * LD,
                  a.o_out + (((int64_t)b * T + q0w) * a.H + h) * D, (int64_t)a.H * D, T - q0w, lane);
}

// ---------------------------------------------------------------------------
// backward, query side: Delta and dQ

template <int D>
__global__ void __launch_bounds__(kAttThreads, D == 64 ? 2 : 1) attn_bwd_dq_kernel(fxAttnArgs a) {
    constexpr bool SW = D == 64;  // swizzled tiles: 9 % fewer tile loads, no transposed-read conflicts
    constexpr int LD = TileLayout<D, SW>::LD;
    constexpr int DC = D / 16;
    constexpr int DT = D / 32;
    __shared__ __attribute__((aligned(16))) uint16_t sk0[kBN * LD], sk1[kBN * LD];
    __shared__ __attribute__((aligned(16))) uint16_t sv0[kBN * LD], sv1[kBN * LD];
    static_assert(32 * (D + 8) <= kBN * LD, "a stage buffer holds one wave's output staging");

    const int T = a.T;
    const int nqt = (T + kBM - 1) / kBM;
    int bh, qt;
    grid_map(nqt, a.B * a.H, bh, qt);
    qt = nqt - 1 - qt;
    const int b = bh / a.H, h = bh - b * a.H;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int g = lane >> 5, ln = lane & 31;
    TileLane<D, SW> tl;
    tl.init(lane);
    const int q0 = qt * kBM;
    const int q0w = q0 + 32 * wave;
    const int qi = q0w + ln;
    const bool qok = qi < T;

    const uint16_t* kbase = a.k + b * a.ksb + h * a.ksh;
    const uint16_t* vbase = a.v + b * a.vsb + h * a.vsh;
    const int kend = a.causal ? min(T, q0 + kBM) : T;
    const int nblk = (kend + kBN - 1) / kBN;
    TileDma2<D, kBN, SW> dma;
    dma.init(a.kst, a.vst);
    dma.issue(kbase, vbase, T, sk0, sv0);
    // the next tile's first K and V rows, advanced by one tile per step
    const int64_t kstep = (int64_t)kBN * a.kst, vstep = (int64_t)kBN * a.vst;
    const uint16_t* kn = kbase;
    const uint16_t* vn = vbase;

    // This lane's lse (read before the Delta store below: a load after a store to another
    // fp32 array may not be moved above it), Q^T and dO^T operands and O row: every load is
    // issued before any is used, and the lse is scaled only after Delta, so the wave makes
    // one memory round trip here.  Rows past T read row 0 and are zeroed after.
    const float lse_raw = qok ? a.lse[(int64_t)bh * T + qi] : 0.f;
    bf16x8 qop[DC], dop[DC];
    float delta = 0.f;
    {
        const uint16_t* qrow = a.q + b * a.qsb + h * a.qsh + (int64_t)(qok ? qi : 0) * a.qst;
        const int64_t orow = (((int64_t)b * T + (qok ? qi : 0)) * a.H + h) * D;
        uint4 qv[DC], dv[DC], ov[DC];
#pragma unroll
        for (int c = 0; c < DC; ++c) {
            qv[c] = ld16(qrow + 16 * c + 8 * g);
            dv[c] = ld16(a.dout + orow + 16 * c + 8 * g);
            ov[c] = ld16(a.o + orow + 16 * c + 8 * g);
        }
        const uint32_t keep = qok ? ~0u : 0u;
#pragma unroll
        for (int c = 0; c < DC; ++c) {
            const uint4 d = mask16(dv[c], keep), o = mask16(ov[c], keep);
            qop[c] = as_bf16x8(mask16(qv[c], keep));
            dop[c] = as_bf16x8(d);
            float fd[8], fo[8];
            unpack8(d, fd);
            unpack8(o, fo);
#pragma unroll
            for (int j = 0; j < 8; ++j) delta += fd[j] * fo[j];
        }
        delta = pair_sum(delta);
        if (qok && g == 0) a.delta[(int64_t)bh * T + qi] = delta;
    }
    float lse_l = lse_raw;
    __asm__ volatile("" : "+v"(lse_l));  // scaled here, after Delta, not where it is loaded
    const float lse2 = lse_l * kLog2e;
    const float sl2 = a.scale * kLog2e;

    f32x16 acc[DT];
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) acc[dt] = f32x16{};

    auto step = [&](int j, const uint16_t* K, const uint16_t* V, uint16_t* nK, uint16_t* nV) {
        const int kb = j * kBN;
        tile_arrive();
        kn += kstep;
        vn += vstep;
        if (j + 1 < nblk) dma.issue(kn, vn, T - kb - kBN, nK, nV);
#pragma unroll
        for (int hh = 0; hh < 2; ++hh) {
            const int kh = kb + 32 * hh;
            if (kh >= T || (a.causal && kh > q0w + 31)) continue;
            // S^T = K Q^T and dP^T = V dO^T, operands read chunk by chunk (few live registers)
            f32x16 s = f32x16{}, dp = f32x16{};
#pragma unroll
            for (int c = 0; c < DC; ++c) {
                const bf16x8 kop = tile_op_row(tl, K, 32 * hh, 16 * c, lane);
                const bf16x8 vop = tile_op_row(tl, V, 32 * hh, 16 * c, lane);
                s = mfma32(kop, qop[c], s);
                dp = mfma32(vop, dop[c], dp);
            }
            if ((kh + 32 > T) || (a.causal && kh + 31 > q0w))  // masked scores give P = 0
                mask_rows(s, 0, (a.causal ? min(qi, T - 1) : T - 1) - kh - 4 * g);
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                const float p = exp2_fast(fmaf(s[i], sl2, -lse2));
                s[i] = p * (dp[i] - delta);  // dS^T / scale
            }
            const bf16x8 d0 = pack_op(s, 0), d1 = pack_op(s, 1);
#pragma unroll
            for (int dt = 0; dt < DT; ++dt) {
                const bf16x8 k0t = tile_op_t(tl, K, 32 * hh, 32 * dt, lane);
                const bf16x8 k1t = tile_op_t(tl, K, 32 * hh + 16, 32 * dt, lane);
                acc[dt] = mfma32(k0t, d0, acc[dt]);
                acc[dt] = mfma32(k1t, d1, acc[dt]);
            }
        }
    };
    for (int j = 0; j < nblk; j += 2) {
        step(j, sk0, sv0, sk1, sv1);
        if (j + 1 < nblk) step(j + 1, sk1, sv1, sk0, sv0);
    }

    __syncthreads();  // every wave is done with the K/V stages: they become store scratch
    store_rows<D>(acc, a.scale, wave == 0 ? sk0 : wave == 1 ? sk1 : wave == 2 ? sv0 : sv1,
                  a.dq + b * a.dqb + h * a.dqh + (int64_t)q0w * a.dqt, a.dqt, T - q0w, lane);
}

// ---------------------------------------------------------------------------
// backward, key side: dK and dV

template <int D>
__global__ void __launch_bounds__(kAttThreads, D == 64 ? 2 : 1) attn_bwd_dkv_kernel(fxAttnArgs a) {
    constexpr bool SW = D == 64;
    constexpr int LD = TileLayout<D, SW>::LD;
    constexpr int DC = D / 16;
    constexpr int DT = D / 32;
    __shared__ __attribute__((aligned(16))) uint16_t sq0[kBQ * LD], sq1[kBQ * LD];
    __shared__ __attribute__((aligned(16))) uint16_t sdo0[kBQ * LD], sdo1[kBQ * LD];
    static_assert(32 * (D + 8) <= kBQ * LD, "a stage buffer holds one wave's output staging");
    __shared__ __attribute__((aligned(16))) float slse[2][kBQ];
    __shared__ __attribute__((aligned(16))) float sdelta[2][kBQ];

    const int T = a.T;
    const int nkt = (T + kBK - 1) / kBK;
    int bh, kt;
    grid_map(nkt, a.B * a.H, bh, kt);  // key tile 0 (most causal work) first
    const int b = bh / a.H, h = bh - b * a.H;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int g = lane >> 5, ln = lane & 31;
    TileLane<D, SW> tl;
    tl.init(lane);
    const int k0 = kt * kBK;
    const int k0w = k0 + 32 * wave;
    const int ki = k0w + ln;
    const bool kok = ki < T;

    const uint16_t* qbase = a.q + b * a.qsb + h * a.qsh;
    const uint16_t* dobase = a.dout + (int64_t)b * T * a.H * D + (int64_t)h * D;
    const int64_t dors = (int64_t)a.H * D;
    const float* lse_bh = a.lse + (int64_t)bh * T;
    const float* del_bh = a.delta + (int64_t)bh * T;
    const int qstart = a.causal ? k0 : 0;  // k0 is a multiple of kBQ
    const int nblk = (T - qstart + kBQ - 1) / kBQ;

    // Q / dO tiles by DMA; the tile's lse and Delta through one register each
    // (threads 0..63), stored to LDS once they have arrived.  The lse is kept raw until
    // then: scaling it where it is loaded makes the wave wait for that load, and with it
    // for the tile loads issued just before (memory loads complete in order), at every
    // tile.
    TileDma2<D, kBQ, SW> dma;
    dma.init(a.qst, dors);
    float rl = 0.f, rdl = 0.f;
    // the next tile's first Q and dO rows, advanced by one tile per issue
    const int64_t qstep = (int64_t)kBQ * a.qst, dostep = (int64_t)kBQ * dors;
    const uint16_t* qn = qbase + (int64_t)qstart * a.qst;
    const uint16_t* don = dobase + (int64_t)qstart * dors;
    auto issue = [&](int qb, const uint16_t* nQ, const uint16_t* nDO) {
        dma.issue(qn, don, T - qb, nQ, nDO);
        qn += qstep;
        don += dostep;
        if (threadIdx.x < kBQ) {
            const int q = qb + threadIdx.x;
            rl = q < T ? lse_bh[q] : 0.f;
            rdl = q < T ? del_bh[q] : 0.f;
        }
    };
    if (nblk > 0) issue(qstart, sq0, sdo0);

    // K and V rows of this lane's key: every load issued before any is used (rows past T
    // read row 0 and are zeroed after)
    bf16x8 kop[DC], vop[DC];
    {
        const uint16_t* krow = a.k + b * a.ksb + h * a.ksh + (int64_t)(kok ? ki : 0) * a.kst;
        const uint16_t* vrow = a.v + b * a.vsb + h * a.vsh + (int64_t)(kok ? ki : 0) * a.vst;
        uint4 kv[DC], vv[DC];
#pragma unroll
        for (int c = 0; c < DC; ++c) {
            kv[c] = ld16(krow + 16 * c + 8 * g);
            vv[c] = ld16(vrow + 16 * c + 8 * g);
        }
        const uint32_t keep = kok ? ~0u : 0u;
#pragma unroll
        for (int c = 0; c < DC; ++c) {
            kop[c] = as_bf16x8(mask16(kv[c], keep));
            vop[c] = as_bf16x8(mask16(vv[c], keep));
        }
    }
    const float sl2 = a.scale * kLog2e;

    f32x16 adv[DT], adk[DT];
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) {
        adv[dt] = f32x16{};
        adk[dt] = f32x16{};
    }

    auto step = [&](int j, const uint16_t* Q, const uint16_t* DO, uint16_t* nQ, uint16_t* nDO) {
        const int qb = qstart + j * kBQ;
        const int st = j & 1;
        __builtin_amdgcn_s_waitcnt(0x0f70);  // vmcnt(0): this wave's tile loads and rl / rdl
        if (threadIdx.x < kBQ) {
            slse[st][threadIdx.x] = rl * kLog2e;
            sdelta[st][threadIdx.x] = rdl;
        }
        __syncthreads();
        if (j + 1 < nblk) issue(qb + kBQ, nQ, nDO);
#pragma unroll
        for (int hh = 0; hh < 2; ++hh) {
            const int qh = qb + 32 * hh;  // first query of this half
            if (qh >= T || (a.causal && qh + 31 < k0w)) continue;  // all of this wave's keys follow these queries
            // S = Q K^T and dP = dO V^T, operands read chunk by chunk (few live registers)
            f32x16 s = f32x16{}, dp = f32x16{};
#pragma unroll
            for (int c = 0; c < DC; ++c) {
                const bf16x8 qa = tile_op_row(tl, Q, 32 * hh, 16 * c, lane);
                const bf16x8 da = tile_op_row(tl, DO, 32 * hh, 16 * c, lane);
                s = mfma32(qa, kop[c], s);
                dp = mfma32(da, vop[c], dp);
            }
            if ((qh + 32 > T) || (a.causal && qh < k0w + 31))  // queries past T or before the key
                mask_rows(s, a.causal ? ki - qh - 4 * g : INT32_MIN, T - 1 - qh - 4 * g);
            // P and dS / scale in fp32, four rows (queries) at a time with their lse and
            // Delta, then packed: only the bf16 operands stay live for the products
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int qr = 32 * hh + 8 * r + 4 * g;  // 4 consecutive queries of this lane
                const float4 l4 = *reinterpret_cast<const float4*>(&slse[st][qr]);
                const float4 d4 = *reinterpret_cast<const float4*>(&sdelta[st][qr]);
                const float lv[4] = {l4.x, l4.y, l4.z, l4.w};
                const float dv[4] = {d4.x, d4.y, d4.z, d4.w};
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const int i = 4 * r + e;
                    const float p = exp2_fast(fmaf(s[i], sl2, -lv[e]));
                    s[i] = p;                          // P
                    dp[i] = p * (dp[i] - dv[e]);       // dS / scale
                }
            }
            const bf16x8 p0 = pack_op(s, 0), p1 = pack_op(s, 1);
            const bf16x8 d0 = pack_op(dp, 0), d1 = pack_op(dp, 1);
#pragma unroll
            for (int dt = 0; dt < DT; ++dt) {
                const bf16x8 o0 = tile_op_t(tl, DO, 32 * hh, 32 * dt, lane);
                const bf16x8 o1 = tile_op_t(tl, DO, 32 * hh + 16, 32 * dt, lane);
                const bf16x8 q0t = tile_op_t(tl, Q, 32 * hh, 32 * dt, lane);
                const bf16x8 q1t = tile_op_t(tl, Q, 32 * hh + 16, 32 * dt, lane);
                adv[dt] = mfma32(o0, p0, adv[dt]);
                adk[dt] = mfma32(q0t, d0, adk[dt]);
                adv[dt] = mfma32(o1, p1, adv[dt]);
                adk[dt] = mfma32(q1t, d1, adk[dt]);
            }
        }
    };
    for (int j = 0; j < nblk; j += 2) {
        step(j, sq0, sdo0, sq1, sdo1);
        if (j + 1 < nblk) step(j + 1, sq1, sdo1, sq0, sdo0);
    }

    __syncthreads();  // every wave is done with the Q/dO stages: they become store scratch
    uint16_t* tmp = wave == 0 ? sq0 : wave == 1 ? sq1 : wave == 2 ? sdo0 : sdo1;
    store_rows<D>(adk, a.scale, tmp, a.dk + b * a.dkb + h * a.dkh + (int64_t)k0w * a.dkt, a.dkt, T - k0w, lane);
    store_rows<D>(adv, 1.f, tmp, a.dv + b * a.dvb + h * a.dvh + (int64_t)k0w * a.dvt, a.dvt, T - k0w, lane);
}

}  // namespace fx

using namespace fx;

static int attn_check(const fxAttnArgs* p, bool bwd) {
    FX_REQUIRE(p != nullptr, "fx_attn: null args");
    const fxAttnArgs& a = *p;
    FX_REQUIRE(a.D == 64 || a.D == 128, "fx_attn: head_dim %d not supported (64 or 128)", a.D);
    FX_REQUIRE(a.B >= 1 && a.T >= 1 && a.H >= 1, "fx_attn: bad shape B=%d T=%d H=%d", a.B, a.T, a.H);
    FX_REQUIRE((int64_t)a.B * a.H * ((a.T + kBM - 1) / kBM) < 0x7fffffff, "fx_attn: grid too large");
    FX_REQUIRE(a.q && a.k && a.v, "fx_attn: null q/k/v");
    // masked scores are -inf before the scale is applied: the scale must be positive
    FX_REQUIRE(a.scale > 0.f && a.scale < __builtin_huge_valf(), "fx_attn: scale %g must be positive and finite",
               (double)a.scale);
    const int64_t s[] = {a.qsb, a.qst, a.qsh, a.ksb, a.kst, a.ksh, a.vsb, a.vst, a.vsh};
    for (int64_t x : s) FX_REQUIRE(x % 8 == 0, "fx_attn: q/k/v strides must be multiples of 8 elements");
    FX_REQUIRE((((uintptr_t)a.q | (uintptr_t)a.k | (uintptr_t)a.v) & 15) == 0,
               "fx_attn: q/k/v must be 16-byte aligned");
    // tile offsets row * stride are 32-bit inside the kernels
    const int64_t mx = (int64_t)64 * (a.qst > a.kst ? (a.qst > a.vst ? a.qst : a.vst) : (a.kst > a.vst ? a.kst : a.vst));
    FX_REQUIRE(mx < ((int64_t)1 << 30) && (int64_t)64 * a.H * a.D < ((int64_t)1 << 30),
               "fx_attn: row strides too large");
    if (!bwd) {
        FX_REQUIRE(a.o_out && a.lse_out, "fx_attn_fwd: null output");
        FX_REQUIRE(((uintptr_t)a.o_out & 15) == 0, "fx_attn_fwd: o must be 16-byte aligned");
    } else {
        FX_REQUIRE(a.o && a.dout && a.lse && a.delta && a.dq && a.dk && a.dv, "fx_attn_bwd: null pointer");
        FX_REQUIRE((((uintptr_t)a.o | (uintptr_t)a.dout) & 15) == 0, "fx_attn_bwd: o/dout must be 16-byte aligned");
        FX_REQUIRE((((uintptr_t)a.dq | (uintptr_t)a.dk | (uintptr_t)a.dv) & 15) == 0,
                   "fx_attn_bwd: dq/dk/dv must be 16-byte aligned");
        const int64_t t[] = {a.dqb, a.dqt, a.dqh, a.dkb, a.dkt, a.dkh, a.dvb, a.dvt, a.dvh};
        for (int64_t x : t) FX_REQUIRE(x % 8 == 0, "fx_attn_bwd: dq/dk/dv strides must be multiples of 8");
    }
    return 0;
}

extern "C" int fx_attn_fwd(const fxAttnArgs* args, void* stream) {
    if (int e = attn_check(args, false)) return e;
    const fxAttnArgs& a = *args;
    const dim3 grid((unsigned)(a.B * a.H * ((a.T + kBM - 1) / kBM)));
    hipStream_t s = (hipStream_t)stream;
    if (a.D == 64)
        hipLaunchKernelGGL(attn_fwd_kernel<64>, grid, dim3(kAttThreads), 0, s, a);
    else
        hipLaunchKernelGGL(attn_fwd_kernel<128>, grid, dim3(kAttThreads), 0, s, a);
    return check_launch("attn_fwd");
}

extern "C" int fx_attn_bwd(const fxAttnArgs* args, void* stream) {
    if (int e = attn_check(args, true)) return e;
    const fxAttnArgs& a = *args;
    hipStream_t s = (hipStream_t)stream;
    const dim3 gq((unsigned)(a.B * a.H * ((a.T + kBM - 1) / kBM)));
    const dim3 gk((unsigned)(a.B * a.H * ((a.T + kBK - 1) / kBK)));
    if (a.D == 64) {
        hipLaunchKernelGGL(attn_bwd_dq_kernel<64>, gq, dim3(kAttThreads), 0, s, a);
        if (int e = check_launch("attn_bwd_dq")) return e;
        hipLaunchKernelGGL(attn_bwd_dkv_kernel<64>, gk, dim3(kAttThreads), 0, s, a);
    } else {
        hipLaunchKernelGGL(attn_bwd_dq_kernel<128>, gq, dim3(kAttThreads), 0, s, a);
        if (int e = check_launch("attn_bwd_dq")) return e;
        hipLaunchKernelGGL(attn_bwd_dkv_kernel<128>, gk, dim3(kAttThreads), 0, s, a);
    }
    return check_launch("attn_bwd_dkv");
}
