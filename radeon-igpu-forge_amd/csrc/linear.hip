// Fused (gather) linear layer for gfx950: C = act(A W^T + bias) with bf16 MFMA.
//
// A rows are either dense (row m at A + m*lda) or gathered: row m is the
// window of W consecutive rows of X starting at idx[m], i.e. the contiguous
// slice X + idx[m]*F .. + K (K = W*F), which is exactly the window-major
// flattening Xg[m, w*F + f] = X[idx[m] + w, f] of ml/fxgpu/gather_gemm.hip:175-206.
// So gathering costs nothing beyond a per-row base pointer, and the gathered
// rows can be written out (Xg) by the first column of tiles for the backward.
//
// Tiling: 256 x 256 output tile per workgroup (128 FLOP per byte of tile loads: a
// 128 x 128 tile measured L2-bandwidth bound), 16 waves in 4 x 4, each wave
// 64 x 64 = 2 x 2 tiles of v_mfma_f32_32x32x16_bf16 (128 VGPRs: 4 waves per SIMD,
// which hide the LDS operand latency that left 8 waves of 128 x 64 at half speed).
// K advances 64 per stage through two LDS stages (row stride 72 elements,
// conflict-free row reads) filled by direct global -> LDS loads that are in flight
// during the previous stage's MFMAs (147 KB of LDS: one persistent workgroup per CU
// walking tiles, with the stage pipeline running on from one tile into the next).
// Epilogue: + bias, optional GELU-tanh, optional pre-activation output, stored
// from the MFMA layout so each half-wave writes 64 contiguous bytes of a row (a
// transposed layout with 8-byte stores scattered over 32 rows measured 1.6x slower).
// Tiles sharing an A row panel are dealt to one XCD (shared L2).
#include <math.h>
#include <stdlib.h>

#include "fx_mfma.h"
#include "gemm_asm.h"

namespace fx {

constexpr int kGBM = 256, kGBN = 256, kGBK = 64;
constexpr int kGLD = kGBK + 8;              // LDS row stride (elements)
constexpr int kGSPR = kGBK / 8 + 1;         // 16-byte LDS slots per row (the last is padding)
constexpr int kGNI = kGBM * kGSPR / 64;     // wave loads per 256-row tile
constexpr int kGThreads = 1024;
constexpr int kGWaves = kGThreads / 64;
constexpr int kGWM = 64, kGWN = 64;         // wave tile: 16 waves in 4 (M) x 4 (N)
constexpr int kGTI = kGWM / 32, kGTJ = kGWN / 32;  // 32 x 32 MFMA tiles per wave
static_assert(kGBM == kGBN && kGBM * kGSPR % 64 == 0, "tile shape");
static_assert((kGBM / kGWM) * (kGBN / kGWN) == kGWaves, "wave layout");
// The general forward kernel: 8 waves of 64 x 128 in 4 (M) x 2 (N), two waves per SIMD.
// Its epilogue variants (bias, GELU, pre-activation H, residual) kept 16 waves of 64 x 64
// past the 128 registers of four waves per SIMD and into scratch; 128 accumulators of 256
// registers leave them room.
constexpr int kFThreads = 512;
constexpr int kFWaves = kFThreads / 64;
constexpr int kFPW = (2 * kGNI + kFWaves - 1) / kFWaves;  // wave loads per wave per stage (A and W)
constexpr int kFWM = 64, kFWN = 128;
constexpr int kFTI = kFWM / 32, kFTJ = kFWN / 32;
static_assert((kGBM / kFWM) * (kGBN / kFWN) == kFWaves, "forward wave layout");

struct GemmArgs {
    const uint16_t* A;
    int64_t lda;
    const int32_t* idx;
    int64_t F;
    int64_t R;  // rows of X when gathering
    const uint16_t* B;
    int64_t ldb;
    const uint16_t* bias;
    uint16_t* C;
    int64_t ldc;
    uint16_t* H;
    int64_t ldh;
    uint16_t* Xg;
    int64_t ldxg;
    int M, N, K;
    int act;   // 0: identity, 1: GELU (tanh approximation)
    const uint16_t* res;  // residual (M, N) added to the output after the activation, or null
    int64_t ldres;
    const uint16_t* nw;  // RMSNorm weight (K,) applied to the A rows first (few-row kernel), or null
    float eps;
    bool vec_c, vec_h;   // C / H rows start 16-byte aligned (16-byte epilogue stores)
    bool vec_r;          // residual rows start 16-byte aligned (16-byte epilogue loads)
};

// tile t -> (row panel, column tile).  Workgroups are dealt round-robin to the 8 XCDs, so
// tiles with t % 8 == x run on XCD x.  With a multiple of 8 row panels, XCD x owns panels
// x, x + 8, ... and walks them in groups of (up to) 4 panels, the column tiles outer: the
// 32 tiles an XCD runs at once then share 4 A row panels and 8 W column panels in its L2
// (one A panel and 32 W panels with the panels outer: measured 7 % slower at the cfg5 fc).
__device__ __forceinline__ void gemm_tile(int t, int nm, int nn, int& m0, int& n0, int& nt) {
    int mt;
    if ((nm & 7) == 0) {
        const int x = t & 7, sq = t >> 3;
        const int per = nm >> 3;
        const int gm = per < 4 ? per : 4;
        const int grp = sq / (gm * nn), w = sq - grp * (gm * nn);
        const int rows = min(gm, per - grp * gm);  // panels in this (possibly last, smaller) group
        mt = (grp * gm + w % rows) * 8 + x;
        nt = w / rows;
    } else {
        mt = t / nn;
        nt = t - mt * nn;
    }
    m0 = mt * kGBM;
    n0 = nt * kGBN;
}

// A 32 x 32 bf16 block of C leaves through the wave's LDS region `tmp`: lane l writes its
// row (l%32) 4 columns at a time (epi_put: columns 8 q + 4 g + 0..3, g = l/32), then
// epi_flush sends 16-byte row chunks out, two per lane (rows r = ch / 4, columns 8 (ch % 4)).
// `vec`: every row start of `out` is 16-byte aligned (ld % 8 == 0, aligned base), so a
// chunk is one store; otherwise element by element.  LDS operations of one wave complete
// in order: the next block's writes cannot overtake these reads.
constexpr int kEpiLD = 40;  // LDS row stride of the staging block (elements)
static_assert((kGWaves / 2) * 32 * kEpiLD <= kGBM * kGLD, "eight waves' staging blocks fill one operand stage");
__device__ __forceinline__ void epi_put(uint16_t* tmp, int q, const float (&v)[4], int lane) {
    *reinterpret_cast<uint2*>(tmp + (lane & 31) * kEpiLD + 8 * q + 4 * (lane >> 5)) =
        make_uint2(pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3]));
}
// The 32 x 32 bf16 block of `src` at (mb, nb) into `tmp`, in the layout epi_flush reads (rows
// r = ch / 4, 16-byte chunks 8 (ch % 4)); elements past M or N are not read (their outputs
// are not stored).
__device__ __forceinline__ void epi_load(uint16_t* tmp, const uint16_t* src, int64_t ld, int mb, int nb, int M, int N,
                                         bool vec, int lane) {
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        const int ch = h * 64 + lane;
        const int r = ch >> 2, c = (ch & 3) * 8;
        const int m = mb + r, n = nb + c;
        if (m >= M || n >= N) continue;
        const uint16_t* p = src + (int64_t)m * ld + n;
        uint4 u;
        if (vec && n + 8 <= N) {
            u = ld16(p);
        } else {
            uint32_t w[4] = {0u, 0u, 0u, 0u};
            for (int e = 0; e < 8 && n + e < N; ++e) w[e >> 1] |= (uint32_t)p[e] << (16 * (e & 1));
            u = make_uint4(w[0], w[1], w[2], w[3]);
        }
        *reinterpret_cast<uint4*>(tmp + r * kEpiLD + c) = u;
    }
}
__device__ __forceinline__ void epi_flush(const uint16_t* tmp, uint16_t* out, int64_t ld, int mb, int nb, int M,
                                          int N, bool vec, int lane) {
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        const int ch = h * 64 + lane;
        const int r = ch >> 2, c = (ch & 3) * 8;
        const uint4 u = *reinterpret_cast<const uint4*>(tmp + r * kEpiLD + c);
        const int m = mb + r, n = nb + c;
        if (m >= M || n >= N) continue;
        uint16_t* o = out + (int64_t)m * ld + n;
        if (vec && n + 8 <= N) {
            st16(o, u);
        } else {
            const uint32_t w[4] = {u.x, u.y, u.z, u.w};
            for (int e = 0; e < 8 && n + e < N; ++e) o[e] = (uint16_t)(w[e >> 1] >> (16 * (e & 1)));
        }
    }
}

// Persistent: each workgroup walks tiles blockIdx.x, blockIdx.x + gridDim.x, ...; the
// stage pipeline runs on across tiles, so the next tile's first K stage loads during
// the current tile's last MFMAs and epilogue.
// EPI selects the epilogue at compile time (fewer live registers than runtime switches):
// bit 0 GELU, bit 1 pre-activation H out, bit 2 bias, bit 3 residual, bit 4 (with bits 0
// and 1) H receives the GELU derivative at the pre-activation instead
template <int EPI>
__global__ void __launch_bounds__(kFThreads, 1) gemm_bias_act_kernel(GemmArgs a) {
    constexpr bool kGelu = EPI & 1, kH = EPI & 2, kBias = EPI & 4, kRes = EPI & 8, kDeriv = EPI & 16;
    static_assert(!kDeriv || (kGelu && kH), "the derivative goes to H, of a GELU layer");
    __shared__ __attribute__((aligned(16))) uint16_t sa[2][kGBM * kGLD];
    __shared__ __attribute__((aligned(16))) uint16_t sb[2][kGBN * kGLD];
    // the bias of the current tile's columns (0 past N), read by the epilogue at
    // compile-time offsets from one per-lane address: per-element global loads of the bias
    // made the compiler keep 16 64-bit column offsets live across the tile and spill them
    __shared__ __attribute__((aligned(16))) uint16_t sbias[kBias ? kGBN : 1];

    const int nm = (a.M + kGBM - 1) / kGBM, nn = (a.N + kGBN - 1) / kGBN;
    const int ntiles = nm * nn;
    int t = blockIdx.x;
    if (t >= ntiles) return;
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = (wave / (kGBN / kFWN)) * kFWM, wn = (wave % (kGBN / kFWN)) * kFWN;
    const int g = lane >> 5;
    const int nk = (a.K + kGBK - 1) / kGBK;

    // this wave's slot loads: instruction i = wave + 16k covers 64 slots of the A tile
    // (i < kGNI) or the W tile; per lane a row pointer (null: row past M / N, or a
    // gathered window that leaves X, read as zeros) and the slot's column
    const uint16_t* src[kFPW];
    int kcol[kFPW], trow[kFPW];
#pragma unroll
    for (int k = 0; k < kFPW; ++k) {
        const int i = wave + kFWaves * k;
        const int sl = (i % kGNI) * 64 + lane;
        const int r = sl / kGSPR;
        int c = sl - r * kGSPR;
        if (c == kGSPR - 1) c = kGSPR - 2;  // pad slot: any in-row chunk
        kcol[k] = c * 8;
        trow[k] = r;
    }
    auto set_rows = [&](int m0, int n0) {
#pragma unroll
        for (int k = 0; k < kFPW; ++k) {
            const int i = wave + kFWaves * k;
            const uint16_t* row = nullptr;
            if (i < kGNI) {
                const int m = m0 + trow[k];
                if (m < a.M) {
                    if (a.idx) {
                        const int64_t st = a.idx[m];
                        if (st >= 0 && st * a.F + a.K <= a.R * a.F) row = a.A + st * a.F;
                    } else {
                        row = a.A + (int64_t)m * a.lda;
                    }
                }
            } else {
                const int n = n0 + trow[k];
                if (n < a.N) row = a.B + (int64_t)n * a.ldb;
            }
            src[k] = row ? row + kcol[k] : nullptr;
        }
    };
    auto issue = [&](int kt, int st) {
        const int k0 = kt * kGBK;
        const bool full = k0 + kGBK <= a.K;
#pragma unroll
        for (int k = 0; k < kFPW; ++k) {
            const int i = wave + kFWaves * k;
            if (i >= 2 * kGNI) break;
            const uint16_t* tile = (i < kGNI) ? sa[st] : sb[st];
            const uint32_t dst = lds_addr(tile + (i % kGNI) * 64 * 8);
            const bool ok = src[k] != nullptr && (full || k0 + kcol[k] < a.K);
            dma16(ok ? (const void*)(src[k] + k0) : (const void*)g_zero_line, dst);
        }
    };

    int m0, n0, nt;
    gemm_tile(t, nm, nn, m0, n0, nt);
    set_rows(m0, n0);
    issue(0, 0);
    int st = 0;  // stage of the next K step to consume
    for (; t < ntiles; t += gridDim.x) {
        f32x16 acc[kFTJ][kFTI];  // [j: 32 columns of W][i: 32 rows of A]
#pragma unroll
        for (int j = 0; j < kFTJ; ++j)
#pragma unroll
            for (int i = 0; i < kFTI; ++i) acc[j][i] = f32x16{};
        const bool write_xg = a.Xg != nullptr && nt == 0;
        const int cm0 = m0, cn0 = n0;
        for (int kt = 0; kt < nk; ++kt, st ^= 1) {
            tile_arrive();
            if (kt + 1 < nk) {
                issue(kt + 1, st ^ 1);
            } else if (t + (int)gridDim.x < ntiles) {  // first stage of this workgroup's next tile
                gemm_tile(t + gridDim.x, nm, nn, m0, n0, nt);
                set_rows(m0, n0);
                issue(0, st ^ 1);
            }
            const uint16_t* A = sa[st];
            const uint16_t* Bt = sb[st];
            if (write_xg) {
                // the gathered rows of this K stage, from LDS to Xg (first column of tiles)
#pragma unroll
                for (int q = 0; q < kGBM * (kGBK / 8) / kFThreads; ++q) {
                    const int v = tid + kFThreads * q;
                    const int r = v / (kGBK / 8), c = v - r * (kGBK / 8);
                    const int m = cm0 + r, k = kt * kGBK + c * 8;
                    if (m < a.M && k < a.K)
                        st16(a.Xg + (int64_t)m * a.ldxg + k, *reinterpret_cast<const uint4*>(A + r * kGLD + c * 8));
                }
            }
#pragma unroll
            for (int c = 0; c < kGBK / 16; ++c) {
                bf16x8 av[kFTI], bv[kFTJ];
#pragma unroll
                for (int i = 0; i < kFTI; ++i)
                    av[i] = *reinterpret_cast<const bf16x8*>(A + (wm + 32 * i + (lane & 31)) * kGLD + 16 * c + 8 * g);
#pragma unroll
                for (int j = 0; j < kFTJ; ++j)
                    bv[j] = *reinterpret_cast<const bf16x8*>(Bt + (wn + 32 * j + (lane & 31)) * kGLD + 16 * c + 8 * g);
#pragma unroll
                for (int j = 0; j < kFTJ; ++j)
#pragma unroll
                    for (int i = 0; i < kFTI; ++i) acc[j][i] = mfma32(bv[j], av[i], acc[j][i]);
            }
        }

        // epilogue.  The accumulators hold C^T: lane l has row m = cm0 + wm + 32 i + l%32 and,
        // for q = 0..3, the columns cn0 + wn + 32 j + 8 q + 4 g + 0..3 (g = l/32).  Bias,
        // activation and residual are applied in fp32 in registers; each 32 x 32 block then
        // goes through the wave's private 32 x kEpiLD LDS region (8-byte writes) and leaves
        // as 16-byte row chunks, 8 columns per lane (2-byte stores straight from the
        // accumulators measured 8 % slower).  `st` now names the next tile's first stage
        // (its loads are in flight): the stage just consumed, st ^ 1, is the scratch once
        // every wave is done reading it.
        if constexpr (kBias) {
            if (tid < kGBN) sbias[tid] = cn0 + tid < a.N ? a.bias[cn0 + tid] : (uint16_t)0;
        }
        __syncthreads();
        uint16_t* tmp = (wave < 8 ? sa[st ^ 1] : sb[st ^ 1]) + (wave & 7) * (32 * kEpiLD);
#pragma unroll
        for (int j = 0; j < kFTJ; ++j) {
            const int nb = cn0 + wn + 32 * j;  // first column of the block
            const uint16_t* bcol = sbias + wn + 32 * j + 4 * g;  // bias of columns nb + 4 g + ...
#pragma unroll
            for (int i = 0; i < kFTI; ++i) {
                const int mb = cm0 + wm + 32 * i;  // first row of the block
                const int m = mb + (lane & 31);
                (void)m;
                // pre-activation h = acc + bias (H, when wanted), then y = act(h) (+ residual).
                // The residual block is staged in tmp by coalesced row loads; each lane reads
                // its 4 values of a q group back from the position it then writes.
#pragma unroll
                for (int pass = 0; pass < 2; ++pass) {
                    if (pass == 0 && !kH) continue;
                    if (pass == 1 && kRes) epi_load(tmp, a.res, a.ldres, mb, nb, a.M, a.N, a.vec_r, lane);
#pragma unroll
                    for (int q = 0; q < 4; ++q) {
                        float rv[4] = {0.f, 0.f, 0.f, 0.f};
                        if (pass == 1 && kRes) {
                            const uint2 u = *reinterpret_cast<const uint2*>(tmp + (lane & 31) * kEpiLD + 8 * q + 4 * g);
                            rv[0] = bf16_to_f32((uint16_t)u.x);
                            rv[1] = bf16_to_f32((uint16_t)(u.x >> 16));
                            rv[2] = bf16_to_f32((uint16_t)u.y);
                            rv[3] = bf16_to_f32((uint16_t)(u.y >> 16));
                        }
                        float v[4];
#pragma unroll
                        for (int e = 0; e < 4; ++e) {
                            float h = acc[j][i][4 * q + e];
                            if (kBias) h += bf16_to_f32(bcol[8 * q + e]);
                            if (pass == 1) {
                                if (kGelu) h = gelu_tanh(h);
                                if (kRes) h += rv[e];
                            } else if (kDeriv) {
                                float c;
                                gelu_tanh_and_grad(h, c, h);
                            }
                            v[e] = h;
                        }
                        epi_put(tmp, q, v, lane);
                    }
                    if (pass == 0)
                        epi_flush(tmp, a.H, a.ldh, mb, nb, a.M, a.N, a.vec_h, lane);
                    else
                        epi_flush(tmp, a.C, a.ldc, mb, nb, a.M, a.N, a.vec_c, lane);
                    // one block at a time: interleaving the blocks' loads and stores raised
                    // the register pressure of the widest epilogues past the budget
                    __builtin_amdgcn_sched_barrier(0);
                }
            }
        }
    }
}

// ---------------------------------------------------------------------------
// Whole-tile kernels: the forward product above, the input gradient dX = dY W and the
// weight gradient below, on tiles that divide the output (M % 256 == 0, N % (64 NJ) == 0)
// and K steps of 32 (K % 32 == 0, K >= 128).  4 waves of 128 x (32 NJ), one workgroup per
// 256 x (64 NJ) tile, the K loop a single generated inline-asm statement (gemm_asm.h, from
// gemm_asm_gen.py, which documents the schedule and checks it on the CPU).  With the
// accumulators in AGPRs (one wave per SIMD) and the LDS operand reads interleaved with the
// MFMAs by hand, the loop runs at the MFMA rate the compiler-scheduled kernels do not
// reach.  The products are the same MFMAs on the same operands in the same K order as the
// general kernels', and the epilogues round the same way, so the results are bit-identical.
// NJ = 4: 256 x 256 tiles; NJ = 3: 256 x 192 tiles (N = 768 is 4 of them: 256 tiles for
// M = 16384, one per CU, where 256 x 256 tiles would leave a quarter of the CUs idle).
__device__ __forceinline__ void raw_barrier() { asm volatile("s_barrier" ::: "memory"); }

constexpr int kAsmStages = FX_FWD_NJ4_STAGES;  // K-step stages of every generated loop
static_assert(kAsmStages == FX_WGRAD_STAGES && kAsmStages == FX_DGRAD_NJ4_STAGES, "one stage count");

// One operand tile of a whole-tile kernel as its loads see it.  The stages live in LDS
// buffers of ks K steps of 32 (ks = 2 for the loops with a row operand, 1 for the weight
// gradient's).  base: the tile's element (0, 0) at the buffer's first K step.  Row operand
// (K along the rows, `rows` tile rows): LDS rows of 4 ks + 1 16-byte slots, the ks steps'
// 64-byte segments side by side (with ks = 2 one 128-byte run of the row, a whole cache
// line) and a padding slot loading the last chunk again.  Col operand (K down the rows,
// `cols` tile columns): 32 ks LDS rows of cols / 8 + 4 slots, the last 4 (padding) loading
// the row's first chunks again.  step: bytes from one buffer's K steps to the next's.
struct TileSrc {
    const uint16_t* base;
    int64_t ld;
    bool col;
    int cols;
    uint64_t step;
    int rmax = 1 << 30;  // row operand: tile rows past this one load this row (a ragged last tile)
    int cmax = 1 << 30;  // col operand: 8-column chunks past this one load this chunk (a ragged last tile)
    int ks = 1;          // K steps per buffer
};

__device__ __forceinline__ const uint16_t* slot_addr(const TileSrc& t, int s) {
    if (!t.col) {
        const int spr = 4 * t.ks + 1;
        const int r = s / spr;
        return t.base + (int64_t)min(r, t.rmax) * t.ld + 8 * min(s - spr * r, 4 * t.ks - 1);
    }
    const int spr = t.cols / 8 + 4;
    const int r = s / spr;
    int c = s - spr * r;
    if (c >= t.cols / 8) c -= t.cols / 8;
    return t.base + (int64_t)r * t.ld + 8 * min(c, t.cmax);
}

// whether slot s of a buffer holds the buffer's first K step (a row's first 4 chunks, or the
// first 32 K rows of a col operand)
__device__ __forceinline__ bool slot_first_step(const TileSrc& t, int s) {
    if (!t.col) {
        const int spr = 4 * t.ks + 1;
        return s - spr * (s / spr) < 4;
    }
    return s / (t.cols / 8 + 4) < 32;
}

// K steps a loop of KS-step buffers runs for K: an odd count of steps of two-step buffers
// gets a leading step of zeros (the "lead", which adds exact zeros to the accumulators).
template <int KS>
__device__ __forceinline__ int asm_gemm_steps(int K, bool& lead) {
    const int n = K / 32;
    lead = KS == 2 && (n & 1);
    return n + (lead ? 1 : 0);
}

// Load pointers, their strides and the prologue: wave-instruction q = wave + 4 t of a buffer
// covers 64 slots of the M-side tile (q < MI), the N-side tile (q < MI + NI) or a pad after
// them that is never read (loading the N tile's first slot); its LDS slots start at q KiB.
// Steps 0..3 go to stages phase + 0..3 (mod 4), the buffers of KS steps each; the pointers
// are left at step 4.  With the lead, the pointers start one step before K = 0 and the first
// buffer's lead-step slots load the zero line.
template <int L, int MI, int NI, int KS>
__device__ __forceinline__ void asm_gemm_prologue(const TileSrc& ms, const TileSrc& ns, int wave, int lane, int phase,
                                                  bool lead, uint32_t base, int buf_bytes, uint64_t (&P)[L],
                                                  uint64_t (&S)[L]) {
    static_assert(MI + NI <= 4 * L && MI + NI > 4 * (L - 1), "load count");
    constexpr int kBufs = kAsmStages / KS;
    bool zero[L];
#pragma unroll
    for (int t = 0; t < L; ++t) {
        const int q = wave + 4 * t;
        const TileSrc& src = q < MI ? ms : ns;
        const int s = q < MI ? q * 64 + lane : q < MI + NI ? (q - MI) * 64 + lane : 0;
        // one K step back: 32 elements along a row, 32 rows down a column
        const int64_t back = lead ? (src.col ? 32 * src.ld : 32) : 0;
        P[t] = (uint64_t)(uintptr_t)slot_addr(src, s) - (uint64_t)(back * 2);
        S[t] = src.step;
        zero[t] = lead && slot_first_step(src, s);
    }
#pragma unroll
    for (int g = 0; g < kBufs; ++g) {
        const int buf = ((g * KS + phase) % kAsmStages) / KS;
#pragma unroll
        for (int t = 0; t < L; ++t) {
            const void* src = g == 0 && zero[t] ? (const void*)g_zero_line : (const void*)(uintptr_t)(P[t] + g * S[t]);
            dma16(src, base + buf * buf_bytes + (wave + 4 * t) * 1024);
        }
    }
#pragma unroll
    for (int t = 0; t < L; ++t) P[t] += kBufs * S[t];
}

// LDS address of stage s (K step s mod 4 of the loop) in buffers of KS steps: the buffer, then
// `sub` bytes per step inside it (a row operand's 64-byte segment, a col operand's 32 rows)
template <int KS>
__device__ __forceinline__ uint32_t stage_addr(uint32_t base, int s, int buf_bytes, int sub) {
    return base + (s / KS) * buf_bytes + (s % KS) * sub;
}

// Per-lane LDS read address of a wave's operand blocks relative to a stage's base
// (stage_addr).  Row side (row_bytes per LDS row): row w0 + l%32, 16 bytes per l/32.  Col
// side (row_bytes per K row):
// the transposed reads' lane pattern, K rows 8 (g'/2) + l%16 / 4 (natural order: the second
// read 4 rows on) or 4 (g'/2) + l%16 / 4 (lds_op_t's order: 8 rows on), columns
// w0 + 16 (g' % 2) + 4 (l % 4), g' = l / 16.
__device__ __forceinline__ uint32_t read_addr(bool col, bool natural, int row_bytes, int w0, int lane) {
    if (!col) return (w0 + (lane & 31)) * row_bytes + 16 * (lane >> 5);
    const int grp = lane >> 4, s16 = lane & 15;
    const int k = (natural ? 8 : 4) * (grp >> 1) + (s16 >> 2);
    return k * row_bytes + (w0 + 16 * (grp & 1) + 4 * (s16 & 3)) * 2;
}

// phase and loop iterations for n >= 4 K steps (the loop body is 4 steps; the last 4 are its
// tail)
__device__ __forceinline__ void asm_gemm_schedule(int nsteps, uint32_t& phase, uint32_t& iters) {
    phase = __builtin_amdgcn_readfirstlane((kAsmStages - nsteps % kAsmStages) % kAsmStages);
    iters = __builtin_amdgcn_readfirstlane((nsteps - kAsmStages + (int)phase) / kAsmStages);
}

// C^T-layout epilogue of the forward and input-gradient kernels: acc[4 j + i] holds rows
// m0 + wm + 32 i + l%32, columns n0 + wn + 32 j + 8 q + 4 g + 0..3 (g = l/32).  Each 32-row
// block leaves through the wave's LDS share `stg` (free once every wave is done with the
// stages): 8-byte writes from the MFMA layout, read back and stored as 16-byte row chunks,
// 32 NJ columns contiguous.  value(i, j, q, a, v) turns the 4 accumulators a into the
// 4 outputs v.  nt: non-temporal stores, for an output that no kernel reads soon.
constexpr int kStgExtra = 8;  // staging row padding (elements)
template <int NJ, class Value>
__device__ __forceinline__ void ct_store_block(uint16_t* stg, int lane, int i, uint16_t* out, int64_t ld, int64_t row0,
                                               int col0, const f32x16 (&acc)[4 * NJ], Value&& value, int nrows = 32, bool nt = false) {
    constexpr int LDE = 32 * NJ + kStgExtra;
    const int g = lane >> 5;
#pragma unroll
    for (int j = 0; j < NJ; ++j)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const float a[4] = {acc[4 * j + i][4 * q], acc[4 * j + i][4 * q + 1], acc[4 * j + i][4 * q + 2],
                                acc[4 * j + i][4 * q + 3]};
            float v[4];
            value(j, q, a, v);
            *reinterpret_cast<uint2*>(stg + (lane & 31) * LDE + 32 * j + 8 * q + 4 * g) =
                make_uint2(pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3]));
        }
#pragma unroll
    for (int k = 0; k < 2 * NJ; ++k) {
        const int idx = lane + 64 * k;
        const int r = idx / (4 * NJ), c = idx - r * (4 * NJ);
        if (r < nrows) {
            const uint4 v = *reinterpret_cast<const uint4*>(stg + r * LDE + 8 * c);
            if (nt)
                st16_nt(out + (row0 + r) * ld + col0 + 8 * c, v);
            else
                st16(out + (row0 + r) * ld + col0 + 8 * c, v);
        }
    }
}

// Two outputs of block i from one evaluation: value(j, q, acc4, o, o2) gives the 4 values of
// `out` (ordinary stores) and of `out2` (non-temporal stores) at the positions ct_store_block
// describes, staged in stg and stg2 (two disjoint 32-row staging blocks of the wave).
template <int NJ, typename Value>
__device__ __forceinline__ void ct_store_block2(uint16_t* stg, uint16_t* stg2, int lane, int i, uint16_t* out,
                                                int64_t ld, uint16_t* out2, int64_t ld2, int64_t row0, int col0,
                                                const f32x16 (&acc)[4 * NJ], Value&& value) {
    constexpr int LDE = 32 * NJ + kStgExtra;
    const int g = lane >> 5;
#pragma unroll
    for (int j = 0; j < NJ; ++j)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const float a[4] = {acc[4 * j + i][4 * q], acc[4 * j + i][4 * q + 1], acc[4 * j + i][4 * q + 2],
                                acc[4 * j + i][4 * q + 3]};
            float v[4], w[4];
            value(j, q, a, v, w);
            const int off = (lane & 31) * LDE + 32 * j + 8 * q + 4 * g;
            *reinterpret_cast<uint2*>(stg + off) = make_uint2(pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3]));
            *reinterpret_cast<uint2*>(stg2 + off) = make_uint2(pack_bf16x2(w[0], w[1]), pack_bf16x2(w[2], w[3]));
        }
#pragma unroll
    for (int k = 0; k < 2 * NJ; ++k) {
        const int idx = lane + 64 * k;
        const int r = idx / (4 * NJ), c = idx - r * (4 * NJ);
        st16(out + (row0 + r) * ld + col0 + 8 * c, *reinterpret_cast<const uint4*>(stg + r * LDE + 8 * c));
        st16_nt(out2 + (row0 + r) * ld2 + col0 + 8 * c, *reinterpret_cast<const uint4*>(stg2 + r * LDE + 8 * c));
    }
}

template <int NJ>
struct FastGemm {
    static constexpr int kStage = NJ == 4 ? FX_FWD_NJ4_STAGE : FX_FWD_NJ3_STAGE;  // bytes of one LDS buffer
    static constexpr int kBufs = NJ == 4 ? FX_FWD_NJ4_BUFS : FX_FWD_NJ3_BUFS;
    static constexpr int kKs = NJ == 4 ? FX_FWD_NJ4_KSTEPS : FX_FWD_NJ3_KSTEPS;
    static constexpr int kRowB = NJ == 4 ? FX_FWD_NJ4_ROW : FX_FWD_NJ3_ROW;      // LDS bytes per operand row
    static constexpr int kLds = kBufs * kStage;
    static constexpr int kLoads = NJ == 4 ? FX_FWD_NJ4_LOADS : FX_FWD_NJ3_LOADS;
    static constexpr int kTN = 64 * NJ;
    static constexpr int kWaveLds = kLds / 4;
    static_assert(2 * 32 * (32 * NJ + kStgExtra) * 2 <= kWaveLds && kWaveLds % 16 == 0,
                  "two staging blocks fit a wave's share");
};

// The product of one 256 x (64 NJ) tile: acc = A[m0.., :] B[n0.., :]^T over K (A rows past
// m0 + rmax read row m0 + rmax), in the C^T layout ct_store_block describes.  Every wave is
// done with the LDS stages when it returns.
template <int NJ>
__device__ __forceinline__ void fast_tile_product(const uint16_t* A, int64_t lda, const uint16_t* B, int64_t ldb, int K,
                                                  int m0, int n0, int rmax, unsigned char* lds, int wave, int lane,
                                                  f32x16 (&acc)[4 * NJ]) {
    using G = FastGemm<NJ>;
    constexpr int L = G::kLoads;
    const int wm = (wave >> 1) * 128, wn = (wave & 1) * 32 * NJ;
    const uint32_t base = __builtin_amdgcn_readfirstlane(lds_addr(lds));
    uint32_t phase, iters;
    bool lead;
    asm_gemm_schedule(asm_gemm_steps<G::kKs>(K, lead), phase, iters);
    TileSrc ms{A + (int64_t)m0 * lda, lda, false, 0, 64 * G::kKs};
    ms.rmax = rmax;
    ms.ks = G::kKs;
    TileSrc ns{B + (int64_t)n0 * ldb, ldb, false, 0, 64 * G::kKs};
    ns.ks = G::kKs;
    uint64_t P[L], S[L];
    if constexpr (NJ == 4)
        asm_gemm_prologue<L, FX_FWD_NJ4_M_INS, FX_FWD_NJ4_N_INS, G::kKs>(ms, ns, wave, lane, phase, lead, base,
                                                                        G::kStage, P, S);
    else
        asm_gemm_prologue<L, FX_FWD_NJ3_M_INS, FX_FWD_NJ3_N_INS, G::kKs>(ms, ns, wave, lane, phase, lead, base,
                                                                        G::kStage, P, S);
    constexpr int kNOff = NJ == 4 ? FX_FWD_NJ4_N_OFF : FX_FWD_NJ3_N_OFF;
    uint32_t vM[kAsmStages], vN[kAsmStages];
#pragma unroll
    for (int s = 0; s < kAsmStages; ++s) {
        vM[s] = stage_addr<G::kKs>(base, s, G::kStage, 64) + read_addr(false, true, G::kRowB, wm, lane);
        vN[s] = stage_addr<G::kKs>(base, s, G::kStage, 64) + kNOff + read_addr(false, true, G::kRowB, wn, lane);
    }
    const uint32_t sbase = base + wave * 1024;
    uint32_t m0save;
#pragma unroll
    for (int k = 0; k < 4 * NJ; ++k) acc[k] = f32x16{};
    if constexpr (NJ == 4)
        asm volatile(FX_FWD_NJ4_KLOOP : FX_FWD_NJ4_OUTS : FX_FWD_NJ4_INS : FX_FWD_NJ4_CLOBBERS);
    else
        asm volatile(FX_FWD_NJ3_KLOOP : FX_FWD_NJ3_OUTS : FX_FWD_NJ3_INS : FX_FWD_NJ3_CLOBBERS);
    (void)m0save;
    raw_barrier();  // every wave is done reading the stages (the loop ends with no load in flight)
}

// Forward: C = act(X W^T + bias), with the pre-activation H.  EPI: bit 0 GELU, bit 1 H out,
// bit 2 bias, bit 3 (with bits 0 and 1) H receives the GELU derivative at the pre-activation
// instead (no residual, gather or Xg)
template <int NJ, int EPI>
__global__ void __launch_bounds__(256, 1) gemm_fast_kernel(GemmArgs a) {
    using G = FastGemm<NJ>;
    constexpr bool kGelu = EPI & 1, kH = EPI & 2, kBias = EPI & 4, kDeriv = EPI & 8;
    static_assert(!kDeriv || (kGelu && kH), "the derivative goes to H, of a GELU layer");
    __shared__ __attribute__((aligned(16))) unsigned char lds[G::kLds];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int g = lane >> 5;
    const int wm = (wave >> 1) * 128, wn = (wave & 1) * 32 * NJ;
    int m0, n0, nt;
    gemm_tile(blockIdx.x, a.M / 256, a.N / G::kTN, m0, n0, nt);
    n0 = nt * G::kTN;
    f32x16 acc[4 * NJ];
    fast_tile_product<NJ>(a.A, a.lda, a.B, a.ldb, a.K, m0, n0, 1 << 30, lds, wave, lane, acc);

    // epilogue: h = acc + bias (H, when wanted), then C = act(h), rounded as
    // gemm_bias_act_kernel rounds them.  H (the pre-activation, which only the backward's GELU
    // derivative reads) leaves with non-temporal stores: in the cfg5 training step that kept
    // the caches for the data the next kernels read, 0.10-0.14 ms per step in in-process
    // A/Bs on three boxes (C, which fc2 reads next, measured slower that way)
    uint16_t* stg = reinterpret_cast<uint16_t*>(lds + wave * G::kWaveLds);
    float bias[NJ][4][4];
#pragma unroll
    for (int j = 0; j < NJ; ++j)
#pragma unroll
        for (int q = 0; q < 4; ++q)
#pragma unroll
            for (int e = 0; e < 4; ++e)
                bias[j][q][e] = kBias ? bf16_to_f32(a.bias[n0 + wn + 32 * j + 8 * q + 4 * g + e]) : 0.f;
    if constexpr (kDeriv) {
        // C and H = gelu'(h) from one exponential and reciprocal per value (the two-pass
        // form below would evaluate them twice: 24 us more per cfg5 fc product)
        uint16_t* stg2 = stg + 32 * (32 * NJ + kStgExtra);
#pragma unroll
        for (int i = 0; i < 4; ++i)
            ct_store_block2<NJ>(stg, stg2, lane, i, a.C, a.ldc, a.H, a.ldh, m0 + wm + 32 * i, n0 + wn, acc,
                                [&](int j, int q, const float (&v)[4], float (&o)[4], float (&d)[4]) {
#pragma unroll
                                    for (int e = 0; e < 4; ++e)
                                        gelu_tanh_and_grad(kBias ? v[e] + bias[j][q][e] : v[e], o[e], d[e]);
                                });
        return;
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int64_t row0 = m0 + wm + 32 * i;
        if constexpr (kH)
            ct_store_block<NJ>(stg, lane, i, a.H, a.ldh, row0, n0 + wn, acc,
                               [&](int j, int q, const float (&v)[4], float (&o)[4]) {
#pragma unroll
                                   for (int e = 0; e < 4; ++e) o[e] = kBias ? v[e] + bias[j][q][e] : v[e];
                               }, 32, true);
        ct_store_block<NJ>(stg, lane, i, a.C, a.ldc, row0, n0 + wn, acc,
                           [&](int j, int q, const float (&v)[4], float (&o)[4]) {
#pragma unroll
                               for (int e = 0; e < 4; ++e) {
                                   float h = kBias ? v[e] + bias[j][q][e] : v[e];
                                   o[e] = kGelu ? gelu_tanh(h) : h;
                               }
                           });
    }
}

// ---------------------------------------------------------------------------
// Linear cross-entropy on the whole-tile product: the logits X E^T (E the (V, K) head
// weight) exist only in the accumulators of one 256 x (64 NJ) tile.  Each logit is rounded
// to bf16, as the unfused path stores it, and then used in fp32 exactly as ce_row_kernel
// uses a stored one:
//   lce_stats_kernel: per row and column tile, (max, sum exp(x - max)) into part[tile][row]
//     (the two waves of a row block merged in LDS), and the target's logit into xt[row]
//     from the one lane that holds it;
//   lce_combine_kernel: per row, the tiles' pairs merged in a fixed order into (M, Z), and
//     the row loss M + log Z - x_t (0 for ignored rows);
//   lce_grad_kernel: the product again, and dl = exp(x - M) (mul / Z) - mul [col == t]
//     stored as bf16, zero rows for ignored targets: the dlogits of ce_row_kernel without
//     the logits ever reaching memory.
// Semantics: the chunk loop of ml/fxlm/cross_entropy.py:107-149 (mm, then ce_fwd_grad)
// with the target rules of ml/fxlm/kernels/ce.hip:32-116 (valid = t != ignore_index and
// 0 <= t < V; out-of-range targets give no loss and a zero gradient row).
struct LceArgs {
    const uint16_t* X;   // (M, K), row stride ldx
    int64_t ldx;
    const uint16_t* E;   // (V, K), contiguous
    const int64_t* target;
    int64_t ignore_index;
    float2* part;        // stats: (V / (64 NJ), M)
    float* xt;           // stats: (M,)
    float2* stat;        // combine: out, grad: in; (M,) pairs (M, Z)
    const float* mul;    // grad: device scalar
    uint16_t* dl;        // grad: (M, V), row stride ldd
    int64_t ldd;
    int M, V, K;
};

// (max, sum of exp(x - max)) pairs: merge (m2, s2) into (m, s); -inf sides carry s == 0
__device__ __forceinline__ void lce_merge(float& m, float& s, float m2, float s2) {
    const float mn = fmaxf(m, m2);
    const float ea = (m == mn) ? 1.f : exp2_fast((m - mn) * kLog2e);
    const float eb = (m2 == mn) ? 1.f : exp2_fast((m2 - mn) * kLog2e);
    s = s * ea + s2 * eb;
    m = mn;
}

// the value lanes l and l ^ 32 hold for one row, combined (same operand order in both
// lanes, so both end with the same bits)
__device__ __forceinline__ float lce_pair_max(float x) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float lce_pair_sum(float x) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// bf16 rounding of a pair (round-to-nearest-even, as the unfused path stores the logits)
__device__ __forceinline__ void round2(float& x, float& y) {
    const uint32_t w = pack_bf16x2(x, y);
    x = bf16_lo(w);
    y = bf16_hi(w);
}

// Where the target column t of a row lies among a lane's accumulators: lane l holds columns
// c0 + 32 j + 8 q + 4 (l / 32) + e of its row (c0 = the wave's first column).  Returns
// 16 j + 4 q + e, or -1 when another lane (or tile) holds it.
template <int NJ>
__device__ __forceinline__ int lce_target_slot(int64_t t, int64_t c0, int g) {
    const int64_t o = t - c0;
    if (o < 0 || o >= 32 * NJ || ((o >> 2) & 1) != g) return -1;
    return (int)(((o >> 5) << 4) | (((o >> 3) & 3) << 2) | (o & 3));
}

template <int NJ>
__global__ void __launch_bounds__(256, 1) lce_stats_kernel(LceArgs a) {
    using G = FastGemm<NJ>;
    __shared__ __attribute__((aligned(16))) unsigned char lds[G::kLds];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int g = lane >> 5, ln = lane & 31;
    const int wm = (wave >> 1) * 128, wn = (wave & 1) * 32 * NJ;
    int m0, n0, nt;
    gemm_tile(blockIdx.x, (a.M + 255) / 256, a.V / G::kTN, m0, n0, nt);
    n0 = nt * G::kTN;
    f32x16 acc[4 * NJ];
    fast_tile_product<NJ>(a.X, a.ldx, a.E, a.K, a.K, m0, n0, a.M - 1 - m0, lds, wave, lane, acc);

    float2* red = reinterpret_cast<float2*>(lds);  // [wave][128 rows] (the stages are free)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int row = m0 + wm + 32 * i + ln;
        // the rounded maximum is the maximum of the rounded logits (rounding is monotonic)
        float m = acc[i][0];
#pragma unroll
        for (int j = 0; j < NJ; ++j)
#pragma unroll
            for (int e = 0; e < 16; ++e) m = fmaxf(m, acc[4 * j + i][e]);
        m = bf16_to_f32(f32_to_bf16(m));
        m = lce_pair_max(m);
        const float ml = m * kLog2e;
        float s4[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int j = 0; j < NJ; ++j)
#pragma unroll
            for (int e = 0; e < 16; e += 2) {
                float x = acc[4 * j + i][e], y = acc[4 * j + i][e + 1];
                round2(x, y);
                s4[e & 3] += exp2_fast(fmaf(x, kLog2e, -ml));
                s4[(e + 1) & 3] += exp2_fast(fmaf(y, kLog2e, -ml));
            }
        const float s = lce_pair_sum((s4[0] + s4[1]) + (s4[2] + s4[3]));
        if (g == 0) red[wave * 128 + 32 * i + ln] = make_float2(m, s);
        // the target's logit, from the lane that holds it
        const int64_t t = row < a.M ? a.target[row] : -1;
        const bool valid = t != a.ignore_index && t >= 0 && t < a.V;
        const int k = valid ? lce_target_slot<NJ>(t, (int64_t)n0 + wn, g) : -1;
        if (__builtin_amdgcn_ballot_w64(k >= 0)) {
            float xv = 0.f;
#pragma unroll
            for (int j = 0; j < NJ; ++j)
#pragma unroll
                for (int e = 0; e < 16; ++e)
                    if (k == 16 * j + e) xv = acc[4 * j + i][e];
            if (k >= 0) a.xt[row] = bf16_to_f32(f32_to_bf16(xv));
        }
    }
    __syncthreads();
    // thread r: tile row r, the pairs of its two waves merged (left columns first)
    const int r = tid, wp = (r >> 7) * 2;
    float m = red[wp * 128 + (r & 127)].x, s = red[wp * 128 + (r & 127)].y;
    const float2 o = red[(wp + 1) * 128 + (r & 127)];
    lce_merge(m, s, o.x, o.y);
    if (m0 + r < a.M) a.part[(int64_t)nt * a.M + m0 + r] = make_float2(m, s);
}

// One workgroup per 16 rows: thread (slice, row) merges the pairs of tiles slice,
// slice + 16, ... in order, then the 16 slices merge in order: a fixed summation order.
__global__ void __launch_bounds__(256) lce_combine_kernel(LceArgs a, int ntiles, float* row_loss) {
    __shared__ float2 sh[16][16];
    const int rr = threadIdx.x & 15, slice = threadIdx.x >> 4;
    const int row = blockIdx.x * 16 + rr;
    float m = -__builtin_huge_valf(), s = 0.f;
    if (row < a.M) {
        int p = slice;
        for (; p + 48 < ntiles; p += 64) {  // four loads in flight
            const float2 v0 = a.part[(int64_t)p * a.M + row], v1 = a.part[(int64_t)(p + 16) * a.M + row];
            const float2 v2 = a.part[(int64_t)(p + 32) * a.M + row], v3 = a.part[(int64_t)(p + 48) * a.M + row];
            lce_merge(m, s, v0.x, v0.y);
            lce_merge(m, s, v1.x, v1.y);
            lce_merge(m, s, v2.x, v2.y);
            lce_merge(m, s, v3.x, v3.y);
        }
        for (; p < ntiles; p += 16) {
            const float2 v = a.part[(int64_t)p * a.M + row];
            lce_merge(m, s, v.x, v.y);
        }
    }
    sh[slice][rr] = make_float2(m, s);
    __syncthreads();
    if (slice == 0 && row < a.M) {
#pragma unroll
        for (int k = 1; k < 16; ++k) lce_merge(m, s, sh[k][rr].x, sh[k][rr].y);
        const int64_t t = a.target[row];
        const bool valid = t != a.ignore_index && t >= 0 && t < a.V;
        a.stat[row] = make_float2(m, s);
        row_loss[row] = valid ? m + logf(s) - a.xt[row] : 0.f;
    }
}

template <int NJ>
__global__ void __launch_bounds__(256, 1) lce_grad_kernel(LceArgs a) {
    using G = FastGemm<NJ>;
    __shared__ __attribute__((aligned(16))) unsigned char lds[G::kLds];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int g = lane >> 5, ln = lane & 31;
    const int wm = (wave >> 1) * 128, wn = (wave & 1) * 32 * NJ;
    int m0, n0, nt;
    gemm_tile(blockIdx.x, (a.M + 255) / 256, a.V / G::kTN, m0, n0, nt);
    n0 = nt * G::kTN;
    f32x16 acc[4 * NJ];
    fast_tile_product<NJ>(a.X, a.ldx, a.E, a.K, a.K, m0, n0, a.M - 1 - m0, lds, wave, lane, acc);

    uint16_t* stg = reinterpret_cast<uint16_t*>(lds + wave * G::kWaveLds);
    const float mul = *a.mul;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int64_t row0 = m0 + wm + 32 * i;
        const int row = (int)row0 + ln;
        const int64_t t = row < a.M ? a.target[row] : -1;
        const bool valid = t != a.ignore_index && t >= 0 && t < a.V;
        const float2 st = valid ? a.stat[row] : make_float2(0.f, 1.f);
        // ignored rows: exp2(-inf) = 0 everywhere and no target column
        const float ml = valid ? st.x * kLog2e : __builtin_huge_valf();
        const float sc = valid ? mul / st.y : 0.f;
        const int k = valid ? lce_target_slot<NJ>(t, (int64_t)n0 + wn, g) : -1;
        ct_store_block<NJ>(stg, lane, i, a.dl, a.ldd, row0, n0 + wn, acc,
                           [&](int j, int q, const float (&v)[4], float (&o)[4]) {
                               float x[4] = {v[0], v[1], v[2], v[3]};
                               round2(x[0], x[1]);
                               round2(x[2], x[3]);
#pragma unroll
                               for (int e = 0; e < 4; ++e) {
                                   o[e] = exp2_fast(fmaf(x[e], kLog2e, -ml)) * sc;
                                   if (k == 16 * j + 4 * q + e) o[e] -= mul;
                               }
                           },
                           (int)min<int64_t>(32, a.M - row0));
    }
}

// Input gradient dX (M x N) = dY (M x K) W (K x N), W row-major with K down its rows (the
// layer's weight, N its input features); EPI 1: dX = (dY W) gelu'(H), H (M x N) the
// pre-activation at dX's layout: the GELU backward of the layer below, which the unfused
// path computes as bf16(bf16(dY W) gelu'(H)), rounded the same way here.
struct DgradArgs {
    const uint16_t* dY;
    int64_t ldy;
    const uint16_t* W;
    int64_t ldw;
    const uint16_t* H;
    uint16_t* dX;
    int64_t ldx;
    int M, N, K;
};

template <int NJ>
struct DgradGemm {
    static constexpr int kStage = NJ == 4 ? FX_DGRAD_NJ4_STAGE : FX_DGRAD_NJ3_STAGE;  // bytes of one LDS buffer
    static constexpr int kBufs = NJ == 4 ? FX_DGRAD_NJ4_BUFS : FX_DGRAD_NJ3_BUFS;
    static constexpr int kKs = NJ == 4 ? FX_DGRAD_NJ4_KSTEPS : FX_DGRAD_NJ3_KSTEPS;
    static constexpr int kRowB = NJ == 4 ? FX_DGRAD_NJ4_ROW : FX_DGRAD_NJ3_ROW;  // LDS bytes per dY row
    static constexpr int kLds = kBufs * kStage;
    static constexpr int kLoads = NJ == 4 ? FX_DGRAD_NJ4_LOADS : FX_DGRAD_NJ3_LOADS;
    static constexpr int kNOff = NJ == 4 ? FX_DGRAD_NJ4_N_OFF : FX_DGRAD_NJ3_N_OFF;
    static constexpr int kRow = (64 * NJ + 32) * 2;  // LDS bytes per K row of the W tile
    static constexpr int kTN = 64 * NJ;
    static constexpr int kWaveLds = kLds / 4;
    static_assert(32 * (32 * NJ + kStgExtra) * 2 <= kWaveLds && kWaveLds % 16 == 0, "staging fits a wave's share");
};

template <int NJ, int EPI>
__global__ void __launch_bounds__(256, 1) gemm_dgrad_fast_kernel(DgradArgs a) {
    using G = DgradGemm<NJ>;
    constexpr int L = G::kLoads;
    __shared__ __attribute__((aligned(16))) unsigned char lds[G::kLds];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int g = lane >> 5;
    const int wm = (wave >> 1) * 128, wn = (wave & 1) * 32 * NJ;
    int m0, n0, nt;
    gemm_tile(blockIdx.x, a.M / 256, a.N / G::kTN, m0, n0, nt);
    n0 = nt * G::kTN;
    const uint32_t base = __builtin_amdgcn_readfirstlane(lds_addr(lds));
    uint32_t phase, iters;
    bool lead;
    asm_gemm_schedule(asm_gemm_steps<G::kKs>(a.K, lead), phase, iters);
    TileSrc ms{a.dY + (int64_t)m0 * a.ldy, a.ldy, false, 0, 64 * G::kKs};
    ms.ks = G::kKs;
    TileSrc ns{a.W + n0, a.ldw, true, G::kTN, (uint64_t)a.ldw * 64 * G::kKs};
    ns.ks = G::kKs;
    uint64_t P[L], S[L];
    if constexpr (NJ == 4)
        asm_gemm_prologue<L, FX_DGRAD_NJ4_M_INS, FX_DGRAD_NJ4_N_INS, G::kKs>(ms, ns, wave, lane, phase, lead, base,
                                                                            G::kStage, P, S);
    else
        asm_gemm_prologue<L, FX_DGRAD_NJ3_M_INS, FX_DGRAD_NJ3_N_INS, G::kKs>(ms, ns, wave, lane, phase, lead, base,
                                                                            G::kStage, P, S);
    uint32_t vM[kAsmStages], vN[kAsmStages];
#pragma unroll
    for (int s = 0; s < kAsmStages; ++s) {
        vM[s] = stage_addr<G::kKs>(base, s, G::kStage, 64) + read_addr(false, true, G::kRowB, wm, lane);
        vN[s] = stage_addr<G::kKs>(base, s, G::kStage, 32 * G::kRow) + G::kNOff +
                read_addr(true, true, G::kRow, wn, lane);
    }
    const uint32_t sbase = base + wave * 1024;
    uint32_t m0save;
    f32x16 acc[4 * NJ];
#pragma unroll
    for (int k = 0; k < 4 * NJ; ++k) acc[k] = f32x16{};
    // EPI 1: the pre-activation of each 32-row block (EPI 2: the GELU derivative there),
    // loaded one block ahead (the first before the K loop: older than the loop's loads, so
    // its waits only get stricter) as whole 16-byte row chunks, then staged in the wave's
    // second LDS block, from which each lane reads its 4 columns per (j, q).  Loading each
    // lane's 8 bytes per (j, q) directly spread every load over 32 rows and touched each
    // line four times (the cfg5 step 0.09 ms slower)
    constexpr int LDE = 32 * NJ + kStgExtra;
    static_assert(2 * 32 * LDE * 2 <= G::kWaveLds, "two staging blocks fit a wave's share");
    uint4 hb[2][2 * NJ];
    // chunk k of a lane: row (lane + 64 k) / (4 NJ), 16-byte column chunk (lane + 64 k) % (4 NJ);
    // with NJ = 4 the chunk is the lane's own in every row it loads (rows lane / 16 + 4 k)
    auto load_h = [&](int i, uint4 (&d)[2 * NJ]) {
        const int64_t row0 = m0 + wm + 32 * i;
        if constexpr (NJ == 4) {
            const uint16_t* p = a.H + (row0 + (lane >> 4)) * a.ldx + n0 + wn + 8 * (lane & 15);
            const int64_t step = 4 * a.ldx;
#pragma unroll
            for (int k = 0; k < 2 * NJ; ++k) d[k] = ld16(p + k * step);
        } else {
#pragma unroll
            for (int k = 0; k < 2 * NJ; ++k) {
                const int idx = lane + 64 * k;
                const int r = idx / (4 * NJ), c = idx - r * (4 * NJ);
                d[k] = ld16(a.H + (row0 + r) * a.ldx + n0 + wn + 8 * c);
            }
        }
    };
    if constexpr (EPI != 0) load_h(0, hb[0]);
    if constexpr (NJ == 4)
        asm volatile(FX_DGRAD_NJ4_KLOOP : FX_DGRAD_NJ4_OUTS : FX_DGRAD_NJ4_INS : FX_DGRAD_NJ4_CLOBBERS);
    else
        asm volatile(FX_DGRAD_NJ3_KLOOP : FX_DGRAD_NJ3_OUTS : FX_DGRAD_NJ3_INS : FX_DGRAD_NJ3_CLOBBERS);
    (void)m0save;

    raw_barrier();
    uint16_t* stg = reinterpret_cast<uint16_t*>(lds + wave * G::kWaveLds);
    uint16_t* stg2 = stg + 32 * LDE;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int64_t row0 = m0 + wm + 32 * i;
        if constexpr (EPI != 0) {
#pragma unroll
            for (int k = 0; k < 2 * NJ; ++k) {
                const int idx = lane + 64 * k;
                const int r = idx / (4 * NJ), c = idx - r * (4 * NJ);
                *reinterpret_cast<uint4*>(stg2 + r * LDE + 8 * c) = hb[i & 1][k];
            }
            if (i + 1 < 4) load_h(i + 1, hb[(i + 1) & 1]);
        }
        ct_store_block<NJ>(stg, lane, i, a.dX, a.ldx, row0, n0 + wn, acc,
                           [&](int j, int q, const float (&v)[4], float (&o)[4]) {
                               if constexpr (EPI != 0) {
                                   const uint2 hh =
                                       *reinterpret_cast<const uint2*>(stg2 + (lane & 31) * LDE + 32 * j + 8 * q + 4 * g);
                                   const float h[4] = {bf16_to_f32((uint16_t)hh.x), bf16_to_f32((uint16_t)(hh.x >> 16)),
                                                       bf16_to_f32((uint16_t)hh.y), bf16_to_f32((uint16_t)(hh.y >> 16))};
#pragma unroll
                                   for (int e = 0; e < 4; ++e)
                                       o[e] = bf16_to_f32(f32_to_bf16(v[e])) * (EPI == 1 ? gelu_tanh_grad(h[e]) : h[e]);
                               } else {
#pragma unroll
                                   for (int e = 0; e < 4; ++e) o[e] = v[e];
                               }
                           });
    }
}

// FX_GEMM_GENERAL in the environment routes products to the general kernels
// (gemm_bias_act_kernel, gemm_wgrad_kernel): "1" all of them, a value containing 'f' the
// forwards, one containing 'w' the weight gradients.  A diagnostic switch, read on every
// call, that lets a test or a benchmark compare the whole-tile kernels with them.
static bool whole_tile_kernels_enabled(char kind) {
    const char* v = getenv("FX_GEMM_GENERAL");
    if (!v) return true;
    if (v[0] == '1') return false;
    for (; *v; ++v)
        if (*v == kind) return false;
    return true;
}

// 4 or 3 (the tile width in 64-column units) when gemm_fast_kernel takes the product, else 0:
// of the tile widths that divide N, the one with the fewest MFMA rounds per CU
static int fast_gemm_nj(const GemmArgs& a) {
    if (a.idx || a.res || a.nw || a.Xg || !whole_tile_kernels_enabled('f')) return 0;
    if (a.M % 256 || a.K % 32 || a.K < 32 * kAsmStages || a.lda % 8 || a.ldb % 8 || !a.vec_c || (a.H && !a.vec_h))
        return 0;
    const int64_t cus = device_cus();
    int64_t best = 0, nj = 0;
    for (int w : {4, 3}) {
        if (a.N % (64 * w)) continue;
        const int64_t tiles = (int64_t)(a.M / 256) * (a.N / (64 * w));
        const int64_t cost = (tiles + cus - 1) / cus * w;
        if (nj == 0 || cost < best) best = cost, nj = w;
    }
    return (int)nj;
}

// ---------------------------------------------------------------------------
// Weight gradient of a linear layer: C (M x N) = A^T B, A (K x M) = dY and B (K x N) =
// X, both row-major with the contraction (tokens) down the rows, so dW = dY^T X.
// The long K (16384 tokens at cfg5) and the small output (768 x 3072 is 36 tiles of
// 256 x 256) leave most CUs idle without splitting K: the grid is tiles x slices
// workgroups, slice s covering an even share of the K steps, and each slice writes an
// fp32 partial tile that one reduce kernel sums in slice order (deterministic).  With
// a single slice the tile is written as bf16 directly.
// Both operands are staged K-major (64 token rows x 256 columns per stage, row stride
// 288 elements = 144 dwords = 16 banks mod 64, so the four rows of a transposed read
// fall in disjoint banks) and fed to the MFMAs with ds_read_b64_tr_b16; the wave
// layout, MFMA tiles and the two-stage direct global -> LDS pipeline are those of the
// forward GEMM above.
constexpr int kWBK = 64;                          // K (token) rows per stage
constexpr int kWLD = kGBM + 32;                   // LDS row stride (elements)
constexpr int kWSPR = kWLD / 8;                   // 16-byte slots per LDS row; the last 4 are padding
constexpr int kWNI = kWBK * kWSPR / 64;           // wave loads per operand tile
constexpr int kWPW = (2 * kWNI + kGWaves - 1) / kGWaves;  // wave loads per wave per stage
static_assert(kWBK * kWSPR % 64 == 0 && kGBM == kGBN, "wgrad tile shape");

struct WgradArgs {
    const uint16_t* A;  // dY (K x M)
    int64_t lda;
    const uint16_t* B;  // X (K x N)
    int64_t ldb;
    uint16_t* C;        // dW (M x N), written when slices == 1 and by the reduce
    int64_t ldc;
    float* part;        // slices x M x N fp32 partials (slices > 1)
    int M, N, K, slices;
};

// Work item of workgroup b in a grid of `total` over (slice, tile) items numbered slice-major,
// tiles row-panel-major.  Workgroups are dealt round-robin to the 8 XCDs (b % 8), each with
// its own L2, so the items are dealt to XCDs in contiguous runs instead: XCD x takes items
// x * (total / 8) + min(x, total % 8) onward, in order.  The tiles of one slice that share a
// token slice of dY (one row panel, every column tile) or of X then run under one L2, and the
// operand panels are fetched from memory about once (with b itself as the item, the column
// tiles of a row panel ran on four different XCDs and every panel was fetched by each).  Only
// which workgroup computes an item changes: the items, and so the results, are the same.
__device__ __forceinline__ int wgrad_item(int b, int total) {
    const int x = b & 7, q = total >> 3, r = total & 7;
    return x * q + min(x, r) + (b >> 3);
}

__global__ void __launch_bounds__(kGThreads, 1) gemm_wgrad_kernel(WgradArgs a) {
    __shared__ __attribute__((aligned(16))) uint16_t sa[2][kWBK * kWLD];
    __shared__ __attribute__((aligned(16))) uint16_t sb[2][kWBK * kWLD];

    const int nn = (a.N + kGBN - 1) / kGBN;
    // slice-major items, dealt to the XCDs in contiguous runs (wgrad_item)
    const int ntiles = ((a.M + kGBM - 1) / kGBM) * nn;
    const int item = wgrad_item(blockIdx.x, ntiles * a.slices);
    const int sl = item / ntiles, t = item - sl * ntiles;
    const int m0 = (t / nn) * kGBM, n0 = (t - (t / nn) * nn) * kGBN;
    const int nk = (a.K + kWBK - 1) / kWBK;
    const int kb = (int)((int64_t)nk * sl / a.slices), ke = (int)((int64_t)nk * (sl + 1) / a.slices);

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = (wave / (kGBN / kGWN)) * kGWM, wn = (wave % (kGBN / kGWN)) * kGWN;
    const int g = lane >> 5;

    // this wave's slot loads: instruction i = wave + 16 k covers 64 slots of the A tile
    // (i < kWNI) or the B tile; per lane the column chunk's address at token row 0 (null:
    // columns past M / N, read as zeros) and the slot's token row
    const uint16_t* src[kWPW];
    int trow[kWPW];
#pragma unroll
    for (int k = 0; k < kWPW; ++k) {
        const int i = wave + kGWaves * k;
        const int slot = (i % kWNI) * 64 + lane;
        const int r = slot / kWSPR;
        int c = slot - r * kWSPR;
        if (c >= kGBM / 8) c -= kGBM / 8;  // pad slot: any in-row chunk
        trow[k] = r;
        src[k] = nullptr;
        if (i < kWNI) {
            if (m0 + 8 * c < a.M) src[k] = a.A + (int64_t)r * a.lda + m0 + 8 * c;
        } else if (i < 2 * kWNI) {
            if (n0 + 8 * c < a.N) src[k] = a.B + (int64_t)r * a.ldb + n0 + 8 * c;
        }
    }
    auto issue = [&](int kt, int st) {
        const int k0 = kt * kWBK;
#pragma unroll
        for (int k = 0; k < kWPW; ++k) {
            const int i = wave + kGWaves * k;
            if (i >= 2 * kWNI) break;
            const bool isa = i < kWNI;
            const uint16_t* tile = isa ? sa[st] : sb[st];
            const uint32_t dst = lds_addr(tile + (i % kWNI) * 64 * 8);
            const bool ok = src[k] != nullptr && k0 + trow[k] < a.K;
            dma16(ok ? (const void*)(src[k] + (int64_t)k0 * (isa ? a.lda : a.ldb)) : (const void*)g_zero_line, dst);
        }
    };

    f32x16 acc[kGTJ][kGTI];  // [j: 32 columns of B][i: 32 columns of A]
#pragma unroll
    for (int j = 0; j < kGTJ; ++j)
#pragma unroll
        for (int i = 0; i < kGTI; ++i) acc[j][i] = f32x16{};
    if (kb < ke) issue(kb, 0);
    int st = 0;
    for (int kt = kb; kt < ke; ++kt, st ^= 1) {
        tile_arrive();
        if (kt + 1 < ke) issue(kt + 1, st ^ 1);
        const uint16_t* At = sa[st];
        const uint16_t* Bt = sb[st];
#pragma unroll
        for (int c = 0; c < kWBK / 16; ++c) {
            bf16x8 av[kGTI], bv[kGTJ];
#pragma unroll
            for (int i = 0; i < kGTI; ++i) av[i] = lds_op_t(At, kWLD, 16 * c, wm + 32 * i, lane);
#pragma unroll
            for (int j = 0; j < kGTJ; ++j) bv[j] = lds_op_t(Bt, kWLD, 16 * c, wn + 32 * j, lane);
#pragma unroll
            for (int j = 0; j < kGTJ; ++j)
#pragma unroll
                for (int i = 0; i < kGTI; ++i) acc[j][i] = mfma32(av[i], bv[j], acc[j][i]);
        }
    }

    // lane holds column n = n0 + wn + 32 j + lane%32 and rows m0 + wm + 32 i + 8 (e/4) + 4 g
    // + e%4; a half-wave stores 32 consecutive columns of a row
    float* part = a.slices > 1 ? a.part + (int64_t)sl * a.M * a.N : nullptr;
#pragma unroll
    for (int j = 0; j < kGTJ; ++j) {
        const int n = n0 + wn + 32 * j + (lane & 31);
        if (n >= a.N) continue;
#pragma unroll
        for (int i = 0; i < kGTI; ++i)
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                const int m = m0 + wm + 32 * i + 8 * (e >> 2) + 4 * g + (e & 3);
                if (m < a.M) {
                    if (part)
                        part[(int64_t)m * a.N + n] = acc[j][i][e];
                    else
                        a.C[(int64_t)m * a.ldc + n] = f32_to_bf16(acc[j][i][e]);
                }
            }
    }
}

// The same product on whole tiles (M % 256 == 0, N % 256 == 0, K % 32 == 0) with the
// generated K loop (gemm_asm.h's WGRAD): 4 waves of 128 x 128, accumulators in AGPRs,
// 32-token steps in 4 LDS stages loaded three steps ahead.  The slices, their token ranges,
// the transposed operand reads (lds_op_t's K permutation) and the MFMA order over K are
// those of gemm_wgrad_kernel, so its partial tiles, and the reduced result, are
// bit-identical.
template <int NJ>
struct WgradGemm {
    static constexpr int kStage = NJ == 4 ? FX_WGRAD_STAGE : FX_WGRAD_NJ3_STAGE;
    static constexpr int kLoads = NJ == 4 ? FX_WGRAD_LOADS : FX_WGRAD_NJ3_LOADS;
    static constexpr int kNOff = NJ == 4 ? FX_WGRAD_N_OFF : FX_WGRAD_NJ3_N_OFF;
    static constexpr int kRowM = (256 + 32) * 2, kRowN = (64 * NJ + 32) * 2;  // LDS bytes per token row
    static_assert(kNOff == 32 * kRowM, "stage layout");
    static_assert((NJ == 4 ? FX_WGRAD_KSTEPS : FX_WGRAD_NJ3_KSTEPS) == 1, "one K step per buffer");
    static constexpr int kLds = kAsmStages * kStage;
};

template <int NJ>
__global__ void __launch_bounds__(256, 1) gemm_wgrad_fast_kernel(WgradArgs a) {
    using G = WgradGemm<NJ>;
    constexpr int L = G::kLoads;
    __shared__ __attribute__((aligned(16))) unsigned char lds[G::kLds];
    const int nn = a.N / (64 * NJ);
    const int ntiles = ((a.M + 255) / 256) * nn;  // the last row panel may be partial (M % 256 != 0)
    const int item = wgrad_item(blockIdx.x, ntiles * a.slices);
    const int sl = item / ntiles, t = item - sl * ntiles;
    const int m0 = (t / nn) * 256, n0 = (t - (t / nn) * nn) * 64 * NJ;
    const int nk64 = (a.K + 63) / 64;
    const int kb = (int)((int64_t)nk64 * sl / a.slices), ke = (int)((int64_t)nk64 * (sl + 1) / a.slices);
    const int t0 = 64 * kb, nsteps = (min(64 * ke, a.K) - t0) / 32;  // >= 4: the host checks
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = (wave >> 1) * 128, wn = (wave & 1) * 32 * NJ;
    const uint32_t base = __builtin_amdgcn_readfirstlane(lds_addr(lds));
    uint32_t phase, iters;
    asm_gemm_schedule(nsteps, phase, iters);
    TileSrc ms{a.A + (int64_t)t0 * a.lda + m0, a.lda, true, 256, (uint64_t)a.lda * 64};
    ms.cmax = (min(256, a.M - m0) >> 3) - 1;  // columns past M load the last chunk (never stored)
    const TileSrc ns{a.B + (int64_t)t0 * a.ldb + n0, a.ldb, true, 64 * NJ, (uint64_t)a.ldb * 64};
    uint64_t P[L], S[L];
    if constexpr (NJ == 4)
        asm_gemm_prologue<L, FX_WGRAD_M_INS, FX_WGRAD_N_INS, 1>(ms, ns, wave, lane, phase, false, base, G::kStage, P, S);
    else
        asm_gemm_prologue<L, FX_WGRAD_NJ3_M_INS, FX_WGRAD_NJ3_N_INS, 1>(ms, ns, wave, lane, phase, false, base,
                                                                       G::kStage, P, S);
    uint32_t vM[kAsmStages], vN[kAsmStages];
#pragma unroll
    for (int s = 0; s < kAsmStages; ++s) {
        vM[s] = base + s * G::kStage + read_addr(true, false, G::kRowM, wm, lane);
        vN[s] = base + s * G::kStage + G::kNOff + read_addr(true, false, G::kRowN, wn, lane);
    }
    const uint32_t sbase = base + wave * 1024;
    uint32_t m0save;
    f32x16 acc[4 * NJ];
#pragma unroll
    for (int k = 0; k < 4 * NJ; ++k) acc[k] = f32x16{};
    if constexpr (NJ == 4)
        asm volatile(FX_WGRAD_KLOOP : FX_WGRAD_OUTS : FX_WGRAD_INS : FX_WGRAD_CLOBBERS);
    else
        asm volatile(FX_WGRAD_NJ3_KLOOP : FX_WGRAD_NJ3_OUTS : FX_WGRAD_NJ3_INS : FX_WGRAD_NJ3_CLOBBERS);
    (void)m0save;

    // Epilogue through LDS (the stages are free once every wave is past its loop): lane
    // holds column n0 + wn + 32 j + lane%32 and rows m0 + wm + 32 i + 8 (e/4) + 4 g + e%4 of
    // acc[4 j + i].  Per 32-row block i the wave writes these fp32 values into a 32 x (32 NJ)
    // block of its own LDS region (row stride kWStg floats, so the half-waves' rows, 4 apart,
    // fall in disjoint banks), then reads the block back along its rows and stores 16-byte
    // chunks: 4 fp32 partials or 8 bf16 outputs per lane and store, rather than one element.
    // One block at a time, so the accumulators are read block by block (read all at once
    // they spill).  A wave's LDS operations complete in order, so a block's writes do not
    // overtake the previous block's reads.
    raw_barrier();
    const int g = lane >> 5;
    constexpr int kWStg = 32 * NJ + 8;  // 4 kWStg = 32 (mod 64): rows r and r + 4 in disjoint banks
    static_assert(4 * 32 * kWStg * 4 <= kAsmStages * G::kStage, "staging fits the stages");
    float* stg = reinterpret_cast<float*>(lds) + wave * 32 * kWStg;
    auto store = [&](auto* out, int64_t ldo) {
        constexpr bool kF32 = sizeof(*out) == 4;
        constexpr int kCh = kF32 ? 8 * NJ : 4 * NJ;  // 16-byte chunks per output row of the block
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int64_t row0 = m0 + wm + 32 * i;
#pragma unroll
            for (int j = 0; j < NJ; ++j) {
#pragma unroll
                for (int e = 0; e < 16; ++e)
                    stg[(8 * (e >> 2) + 4 * g + (e & 3)) * kWStg + 32 * j + (lane & 31)] = acc[4 * j + i][e];
                __builtin_amdgcn_sched_barrier(0);
            }
#pragma unroll
            for (int k = 0; k < kCh / 2; ++k) {
                const int idx = lane + 64 * k;
                const int r = idx / kCh, c = idx - r * kCh;
                if (row0 + r >= a.M) continue;  // past a ragged last panel
                auto* o = out + (row0 + r) * ldo + n0 + wn;
                const float* src = stg + r * kWStg;
                if constexpr (kF32) {
                    st16(o + 4 * c, *reinterpret_cast<const uint4*>(src + 4 * c));
                } else {
                    const float4 lo = *reinterpret_cast<const float4*>(src + 8 * c);
                    const float4 hi = *reinterpret_cast<const float4*>(src + 8 * c + 4);
                    st16(o + 8 * c, make_uint4(pack_bf16x2(lo.x, lo.y), pack_bf16x2(lo.z, lo.w),
                                               pack_bf16x2(hi.x, hi.y), pack_bf16x2(hi.z, hi.w)));
                }
            }
            __builtin_amdgcn_sched_barrier(0);
        }
    };
    if (a.slices > 1)
        store(a.part + (int64_t)sl * a.M * a.N, (int64_t)a.N);
    else
        store(a.C, a.ldc);
}

// C = bf16(sum over slices of the fp32 partials), slice 0 first; 8 consecutive
// elements (one 16-byte store) per thread and step, N % 8 == 0
__global__ void __launch_bounds__(256)
wgrad_reduce_kernel(const float* __restrict__ part, int slices, int64_t MN, int N, uint16_t* __restrict__ C,
                    int64_t ldc) {
    const int64_t stride = (int64_t)gridDim.x * 256;
    for (int64_t v = (int64_t)blockIdx.x * 256 + threadIdx.x; v < MN / 8; v += stride) {
        float s[8];
        const float4* p = reinterpret_cast<const float4*>(part + v * 8);
        float4 lo = p[0], hi = p[1];
        s[0] = lo.x; s[1] = lo.y; s[2] = lo.z; s[3] = lo.w;
        s[4] = hi.x; s[5] = hi.y; s[6] = hi.z; s[7] = hi.w;
        for (int k = 1; k < slices; ++k) {
            const float4* q = reinterpret_cast<const float4*>(part + (int64_t)k * MN + v * 8);
            lo = q[0];
            hi = q[1];
            s[0] += lo.x; s[1] += lo.y; s[2] += lo.z; s[3] += lo.w;
            s[4] += hi.x; s[5] += hi.y; s[6] += hi.z; s[7] += hi.w;
        }
        const int64_t e = v * 8;
        const int64_t m = e / N, n = e - m * N;
        st16(C + m * ldc + n, pack8(s));
    }
}

// ---------------------------------------------------------------------------
// Few-row forward (M <= 64: decoding, small batches).  The GEMM is then a stream
// over W (N K bf16 read once), so the kernel is shaped for loads in flight, not for
// operand reuse.  It computes the transpose, C^T (N x M) = W X^T, with
// v_mfma_f32_16x16x32_bf16: A = 16 W rows, B = 16 X rows, both read straight from
// global memory in 16-byte row chunks (lane l takes row l%16 and k = k0 + 8(l/16) +
// 0..7 in both operands: the K order inside one instruction is the same for the two,
// so the product is the plain contraction); the accumulator lane l holds column
// (X row) l%16 and rows (W rows) 4(l/16) + 0..3.  A workgroup owns 16 NT rows of W and
// its sw waves split the K steps of 32; each wave keeps NT x MT accumulator tiles.
// The partial tiles meet in LDS and are summed in wave order (deterministic), then
// + bias, activation and the stores.  Gathered rows work as in the tiled kernel; the
// first workgroup writes them out (Xg) while it streams them.
constexpr int kSKMaxM = 64;
constexpr int kSKMaxTiles = 16;  // sw * NT * MT: 1 KB of LDS per accumulator tile

__device__ __forceinline__ f32x4 mfma16(const uint4& a, const uint4& b, const f32x4& c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c,
                                                   0, 0, 0);
}

// row m of A (dense or gathered; null for a window that leaves X)
__device__ __forceinline__ const uint16_t* xrow_base(const GemmArgs& a, int m) {
    if (a.idx) {
        const int64_t st = a.idx[m];
        return (st >= 0 && st * a.F + a.K <= a.R * a.F) ? a.A + st * a.F : nullptr;
    }
    return a.A + (int64_t)m * a.lda;
}

template <int NT, int MT, bool NORM>
__global__ void __launch_bounds__(1024) gemm_skinny_kernel(GemmArgs a, int sw) {
    constexpr int U = NT * MT >= 4 ? 2 : 4;  // K steps per load batch
    __shared__ __attribute__((aligned(16))) float red[kSKMaxTiles * 256];
    const int lane = threadIdx.x & 63;
    const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int r = lane & 15, kg = lane >> 4;
    const int n0 = blockIdx.x * 16 * NT;
    const int ks = (a.K + 31) / 32;
    const int kb = w * ks / sw, ke = (w + 1) * ks / sw;

    const uint16_t* wrow[NT];
#pragma unroll
    for (int i = 0; i < NT; ++i) {
        const int n = n0 + 16 * i + r;
        wrow[i] = n < a.N ? a.B + (int64_t)n * a.ldb + 8 * kg : nullptr;
    }
    const uint16_t* xrow[MT];
#pragma unroll
    for (int j = 0; j < MT; ++j) {
        const int m = 16 * j + r;
        const uint16_t* row = m < a.M ? xrow_base(a, m) : nullptr;
        xrow[j] = row ? row + 8 * kg : nullptr;
    }
    const bool wxg = a.Xg != nullptr && blockIdx.x == 0;

    // NORM: A rows are RMS-normalised on the fly, x * rstd[m] * nw[k] rounded to bf16 as
    // the norm kernel writes them.  Each workgroup first computes rstd of every row: wave
    // v sums rows v, v + sw, ... (lane partials, then a butterfly: a fixed order).
    __shared__ float srstd[kSKMaxM];
    float rs[MT];
    if constexpr (NORM) {
        for (int m = w; m < a.M; m += sw) {
            const uint16_t* row = xrow_base(a, m);
            float q = 0.f;
            if (row)
                for (int c = lane; c < a.K / 8; c += 64) {
                    float f[8];
                    unpack8(ld16(row + c * 8), f);
#pragma unroll
                    for (int e = 0; e < 8; ++e) q = fmaf(f[e], f[e], q);
                }
            q = group_sum<64>(q);
            if (lane == 0) srstd[m] = 1.f / sqrtf(q / (float)a.K + a.eps);
        }
        __syncthreads();
#pragma unroll
        for (int j = 0; j < MT; ++j) rs[j] = 16 * j + r < a.M ? srstd[16 * j + r] : 0.f;
    }

    f32x4 acc[NT][MT];
#pragma unroll
    for (int i = 0; i < NT; ++i)
#pragma unroll
        for (int j = 0; j < MT; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
    const uint4 zero = make_uint4(0u, 0u, 0u, 0u);
    for (int s0 = kb; s0 < ke; s0 += U) {
        uint4 wv[U][NT], xv[U][MT];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int s = s0 + u;
            const bool ok = s < ke && s * 32 + 8 * kg < a.K;
#pragma unroll
            for (int i = 0; i < NT; ++i) wv[u][i] = ok && wrow[i] ? ld16(wrow[i] + s * 32) : zero;
#pragma unroll
            for (int j = 0; j < MT; ++j) xv[u][j] = ok && xrow[j] ? ld16(xrow[j] + s * 32) : zero;
            if constexpr (NORM) {
                const uint4 wn = ok ? ld16(a.nw + s * 32 + 8 * kg) : zero;
                float fw[8];
                unpack8(wn, fw);
#pragma unroll
                for (int j = 0; j < MT; ++j) {
                    float f[8];
                    unpack8(xv[u][j], f);
#pragma unroll
                    for (int e = 0; e < 8; ++e) f[e] = f[e] * rs[j] * fw[e];
                    xv[u][j] = pack8(f);
                }
            }
        }
        if (wxg) {
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const int s = s0 + u;
                if (s >= ke || s * 32 + 8 * kg >= a.K) continue;
#pragma unroll
                for (int j = 0; j < MT; ++j) {
                    const int m = 16 * j + r;
                    if (m < a.M) st16(a.Xg + (int64_t)m * a.ldxg + s * 32 + 8 * kg, xv[u][j]);
                }
            }
        }
#pragma unroll
        for (int u = 0; u < U; ++u)
#pragma unroll
            for (int i = 0; i < NT; ++i)
#pragma unroll
                for (int j = 0; j < MT; ++j) acc[i][j] = mfma16(wv[u][i], xv[u][j], acc[i][j]);
    }
#pragma unroll
    for (int i = 0; i < NT; ++i)
#pragma unroll
        for (int j = 0; j < MT; ++j)
            *reinterpret_cast<f32x4*>(&red[((w * NT + i) * MT + j) * 256 + lane * 4]) = acc[i][j];
    __syncthreads();
    // value (tile, m_local, n_local), n_local fastest so neighbouring threads store
    // neighbouring columns; in the accumulator layout it sits at lane m_local +
    // 16 (n_local / 4), element n_local % 4
    constexpr int kVals = NT * MT * 256;
    for (int v = threadIdx.x; v < kVals; v += blockDim.x) {
        const int tile = v >> 8, ml = (v >> 4) & 15, nl = v & 15;
        const int off = tile * 256 + (ml + 16 * (nl >> 2)) * 4 + (nl & 3);
        float sum = 0.f;
        for (int ww = 0; ww < sw; ++ww) sum += red[ww * kVals + off];
        const int n = n0 + 16 * (tile / MT) + nl, m = 16 * (tile % MT) + ml;
        if (n < a.N && m < a.M) {
            const float h = sum + (a.bias ? bf16_to_f32(a.bias[n]) : 0.f);
            float y = h;
            if (a.act == 2) {
                float d;
                gelu_tanh_and_grad(h, y, d);
                if (a.H) a.H[(int64_t)m * a.ldh + n] = f32_to_bf16(d);
            } else {
                if (a.H) a.H[(int64_t)m * a.ldh + n] = f32_to_bf16(h);
                if (a.act == 1) y = gelu_tanh(h);
            }
            if (a.res) y += bf16_to_f32(a.res[(int64_t)m * a.ldres + n]);
            a.C[(int64_t)m * a.ldc + n] = f32_to_bf16(y);
        }
    }
}

template <int NT, bool NORM>
static int skinny_launch(const GemmArgs& a, hipStream_t st) {
    const int mt = (a.M + 15) / 16;
    const int64_t nblk = ((int64_t)a.N + 16 * NT - 1) / (16 * NT);
    const int64_t ks = (a.K + 31) / 32;
    const int64_t target = 4LL * device_cus();  // waves
    int sw = 1;
    while (sw < 16 && nblk * sw < target && 2 * sw <= ks && 2 * sw * NT * mt <= kSKMaxTiles) sw *= 2;
    const dim3 grid((unsigned)nblk), block(64 * sw);
    switch (mt) {
        case 1: hipLaunchKernelGGL((gemm_skinny_kernel<NT, 1, NORM>), grid, block, 0, st, a, sw); break;
        case 2: hipLaunchKernelGGL((gemm_skinny_kernel<NT, 2, NORM>), grid, block, 0, st, a, sw); break;
        case 3: hipLaunchKernelGGL((gemm_skinny_kernel<NT, 3, NORM>), grid, block, 0, st, a, sw); break;
        default: hipLaunchKernelGGL((gemm_skinny_kernel<NT, 4, NORM>), grid, block, 0, st, a, sw); break;
    }
    return check_launch("gemm_skinny");
}

// two W row tiles per workgroup once there are enough workgroups (fewer re-reads of X)
static int linear_skinny(const GemmArgs& a, hipStream_t st) {
    const bool two = (a.N + 31) / 32 >= 2LL * device_cus();
    if (a.nw) return two ? skinny_launch<2, true>(a, st) : skinny_launch<1, true>(a, st);
    return two ? skinny_launch<2, false>(a, st) : skinny_launch<1, false>(a, st);
}

__global__ void __launch_bounds__(256)
gelu_bwd_kernel(const uint16_t* __restrict__ dy, const uint16_t* __restrict__ h, uint16_t* __restrict__ dh,
                int64_t n) {
    const int64_t stride = (int64_t)gridDim.x * 256;
    const int64_t n8 = n >> 3;
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n8; i += stride) {
        float fd[8], fh[8], o[8];
        unpack8(ld16_nt(dy + i * 8), fd);
        unpack8(ld16_nt(h + i * 8), fh);
#pragma unroll
        for (int j = 0; j < 8; ++j) o[j] = fd[j] * gelu_tanh_grad(fh[j]);
        st16_nt(dh + i * 8, pack8(o));
    }
    for (int64_t i = n8 * 8 + (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += stride)
        dh[i] = f32_to_bf16(bf16_to_f32(dy[i]) * gelu_tanh_grad(bf16_to_f32(h[i])));
}

// dh = dy * g elementwise (g the GELU derivative the forward stored), rounded to bf16
__global__ void __launch_bounds__(256)
gate_mul_kernel(const uint16_t* __restrict__ dy, const uint16_t* __restrict__ g, uint16_t* __restrict__ dh,
                int64_t n) {
    const int64_t stride = (int64_t)gridDim.x * 256;
    const int64_t n8 = n >> 3;
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n8; i += stride) {
        float fd[8], fg[8], o[8];
        unpack8(ld16_nt(dy + i * 8), fd);
        unpack8(ld16_nt(g + i * 8), fg);
#pragma unroll
        for (int j = 0; j < 8; ++j) o[j] = fd[j] * fg[j];
        st16_nt(dh + i * 8, pack8(o));
    }
    for (int64_t i = n8 * 8 + (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += stride)
        dh[i] = f32_to_bf16(bf16_to_f32(dy[i]) * bf16_to_f32(g[i]));
}

// the few-row kernel for M <= kSKMaxM, else the persistent tiled kernel
static int linear_fwd(GemmArgs a, hipStream_t stream) {
    if (a.M <= kSKMaxM) return linear_skinny(a, stream);
    a.vec_c = a.ldc % 8 == 0 && ((uintptr_t)a.C & 15) == 0;
    a.vec_h = a.H && a.ldh % 8 == 0 && ((uintptr_t)a.H & 15) == 0;
    a.vec_r = a.res && a.ldres % 8 == 0 && ((uintptr_t)a.res & 15) == 0;
    const int64_t tiles = ((int64_t)(a.M + kGBM - 1) / kGBM) * ((a.N + kGBN - 1) / kGBN);
    FX_REQUIRE(tiles < 0x7fffffffLL, "fx_linear_fwd: too many tiles");
    if (const int nj = fast_gemm_nj(a)) {
        const int64_t ft = (int64_t)(a.M / 256) * (a.N / (64 * nj));
        const int fe = (a.act != 0 ? 1 : 0) | (a.H ? 2 : 0) | (a.bias ? 4 : 0) | (a.act == 2 && a.H ? 8 : 0);
#define FX_FAST_EPI(J, E) \
    case E: hipLaunchKernelGGL((gemm_fast_kernel<J, E>), dim3((unsigned)ft), dim3(256), 0, stream, a); break;
        if (nj == 4) {
            switch (fe) { FX_FAST_EPI(4, 0) FX_FAST_EPI(4, 1) FX_FAST_EPI(4, 2) FX_FAST_EPI(4, 3)
                          FX_FAST_EPI(4, 4) FX_FAST_EPI(4, 5) FX_FAST_EPI(4, 6) FX_FAST_EPI(4, 7)
                          FX_FAST_EPI(4, 11) FX_FAST_EPI(4, 15)
                          default: return set_error(FX_EINVAL, "fx_linear_fwd: epilogue %d", fe); }
        } else {
            switch (fe) { FX_FAST_EPI(3, 0) FX_FAST_EPI(3, 1) FX_FAST_EPI(3, 2) FX_FAST_EPI(3, 3)
                          FX_FAST_EPI(3, 4) FX_FAST_EPI(3, 5) FX_FAST_EPI(3, 6) FX_FAST_EPI(3, 7)
                          FX_FAST_EPI(3, 11) FX_FAST_EPI(3, 15)
                          default: return set_error(FX_EINVAL, "fx_linear_fwd: epilogue %d", fe); }
        }
#undef FX_FAST_EPI
        return check_launch("gemm_fast");
    }
    // persistent grid: one workgroup per CU (the LDS of one is 147 KB)
    const int64_t cus = device_cus();
    const int64_t grid = tiles < cus ? tiles : cus;
    const int epi = (a.act != 0 ? 1 : 0) | (a.H ? 2 : 0) | (a.bias ? 4 : 0) | (a.res ? 8 : 0) |
                    (a.act == 2 && a.H ? 16 : 0);
#define FX_GEMM_EPI(E) \
    case E: hipLaunchKernelGGL(gemm_bias_act_kernel<E>, dim3((unsigned)grid), dim3(kFThreads), 0, stream, a); break;
    switch (epi) {
        FX_GEMM_EPI(0) FX_GEMM_EPI(1) FX_GEMM_EPI(2) FX_GEMM_EPI(3) FX_GEMM_EPI(4) FX_GEMM_EPI(5) FX_GEMM_EPI(6)
        FX_GEMM_EPI(7) FX_GEMM_EPI(8) FX_GEMM_EPI(9) FX_GEMM_EPI(10) FX_GEMM_EPI(11) FX_GEMM_EPI(12)
        FX_GEMM_EPI(13) FX_GEMM_EPI(14) FX_GEMM_EPI(15) FX_GEMM_EPI(19) FX_GEMM_EPI(23)
        default: return set_error(FX_EINVAL, "fx_linear_fwd: epilogue %d", epi);
    }
#undef FX_GEMM_EPI
    return check_launch("gemm_bias_act");
}

}  // namespace fx

using namespace fx;

extern "C" int fx_linear_fwd(const uint16_t* X, int64_t ldx, const int32_t* idx, int64_t F,
                             int64_t R, const uint16_t* W, const uint16_t* bias, uint16_t* Y, uint16_t* H,
                             uint16_t* Xg, int64_t M, int64_t N, int64_t K, int32_t act, void* stream) {
    FX_REQUIRE(X && W && Y, "fx_linear_fwd: null pointer");
    FX_REQUIRE(M >= 0 && N >= 1 && K >= 8, "fx_linear_fwd: bad shape M=%lld N=%lld K=%lld", (long long)M,
               (long long)N, (long long)K);
    FX_REQUIRE(K % 8 == 0, "fx_linear_fwd: K=%lld must be a multiple of 8", (long long)K);
    FX_REQUIRE(M < 0x7fffffffLL && N < 0x7fffffffLL && K < 0x7fffffffLL, "fx_linear_fwd: size too large");
    FX_REQUIRE(act >= 0 && act <= 2, "fx_linear_fwd: act=%d (0 identity, 1 gelu_tanh, 2 gelu_tanh with its derivative in H)",
               act);
    if (idx) {
        FX_REQUIRE(F >= 8 && F % 8 == 0 && K % F == 0, "fx_linear_fwd: gather needs F%%8==0 and K%%F==0 (F=%lld)",
                   (long long)F);
        FX_REQUIRE(R >= 0, "fx_linear_fwd: R=%lld", (long long)R);
    } else {
        FX_REQUIRE(ldx >= K && ldx % 8 == 0, "fx_linear_fwd: ldx=%lld", (long long)ldx);
    }
    FX_REQUIRE(((((uintptr_t)X) | ((uintptr_t)W) | ((uintptr_t)Xg)) & 15) == 0,
               "fx_linear_fwd: X, W, Xg must be 16-byte aligned");
    if (M == 0) return 0;
    GemmArgs a{};
    a.A = X;
    a.lda = ldx;
    a.idx = idx;
    a.F = F;
    a.R = R;
    a.B = W;
    a.ldb = K;
    a.bias = bias;
    a.C = Y;
    a.ldc = N;
    a.H = H;
    a.ldh = N;
    a.Xg = Xg;
    a.ldxg = K;
    a.M = (int)M;
    a.N = (int)N;
    a.K = (int)K;
    a.act = act;
    return linear_fwd(a, (hipStream_t)stream);
}

extern "C" int fx_linear_fwd_ex(const fxLinearArgs* args, void* stream) {
    FX_REQUIRE(args != nullptr, "fx_linear_fwd_ex: null args");
    const fxLinearArgs& p = *args;
    FX_REQUIRE(p.X && p.W && p.Y, "fx_linear_fwd_ex: null pointer");
    FX_REQUIRE(p.M >= 0 && p.N >= 1 && p.K >= 8 && p.K % 8 == 0,
               "fx_linear_fwd_ex: bad shape M=%lld N=%lld K=%lld (K a multiple of 8)", (long long)p.M,
               (long long)p.N, (long long)p.K);
    FX_REQUIRE(p.M < 0x7fffffffLL && p.N < 0x7fffffffLL && p.K < 0x7fffffffLL, "fx_linear_fwd_ex: size too large");
    FX_REQUIRE(p.act == 0 || p.act == 1, "fx_linear_fwd_ex: act=%d (0 identity, 1 gelu_tanh)", p.act);
    FX_REQUIRE(p.ldx >= p.K && p.ldx % 8 == 0, "fx_linear_fwd_ex: ldx=%lld", (long long)p.ldx);
    FX_REQUIRE(p.res == nullptr || p.ldres >= p.N, "fx_linear_fwd_ex: ldres=%lld < N", (long long)p.ldres);
    FX_REQUIRE(p.norm_w == nullptr || p.M <= kSKMaxM,
               "fx_linear_fwd_ex: the input RMSNorm needs M <= %d rows (M=%lld)", kSKMaxM, (long long)p.M);
    FX_REQUIRE(p.norm_w == nullptr || (p.eps >= 0.f && p.eps < __builtin_huge_valf()),
               "fx_linear_fwd_ex: eps %g", (double)p.eps);
    FX_REQUIRE(((((uintptr_t)p.X) | ((uintptr_t)p.W) | ((uintptr_t)p.norm_w)) & 15) == 0,
               "fx_linear_fwd_ex: X, W and norm_w must be 16-byte aligned");
    if (p.M == 0) return 0;
    GemmArgs a{};
    a.A = p.X;
    a.lda = p.ldx;
    a.B = p.W;
    a.ldb = p.K;
    a.bias = p.bias;
    a.C = p.Y;
    a.ldc = p.N;
    a.H = p.H;
    a.ldh = p.N;
    a.M = (int)p.M;
    a.N = (int)p.N;
    a.K = (int)p.K;
    a.act = p.act;
    a.res = p.res;
    a.ldres = p.ldres;
    a.nw = p.norm_w;
    a.eps = p.eps;
    return linear_fwd(a, (hipStream_t)stream);
}

// The weight gradient's plan: the tile width (0: the general kernel's 256 x 256 tiles, or
// the whole-tile kernel's 256 x 64 NJ) and the K split.  Slices: at least 4 K steps of 64
// tokens each, at most 32, and no more workgroups than CUs (one workgroup per CU).  The
// whole-tile kernel takes N % (64 NJ) == 0, K % 32 == 0, K >= 128 (any M, a partial last
// 256-row panel clamped on load and masked on store).  With
// FX_GEMM_GENERAL selecting the general kernel the slices stay those of the whole-tile plan,
// so the two produce the same partials.  256 x 192 tiles wherever N % 192 == 0: more tiles,
// hence fewer slices and less fp32 partial traffic (5 slices instead of 7 at the cfg5 fc
// shapes); measured 67.9 / 43.1 / 80.4 / 78.5 µs against 80.3 / 47.6 / 92.9 / 81.9 for
// 256 x 256 tiles (qkv / proj / fc / fc2 weight gradients, reduce included) and 18.05
// against 18.47 ms per cfg5 step.  FX_WGRAD_TILE=256 keeps 256 x 256 tiles (comparisons).
// How fx_linear_wgrad divides a product.  Outputs with fewer whole tiles than CUs split K
// into `slices` (fp32 partials, then a reduce in slice order).  Outputs with more tiles
// than CUs run one slice, except that a last, partly filled round of tiles (the tied head's
// (50304, 768) gradient is 788 tiles: three rounds of 256 and 20 tiles in a fourth, which
// would take as long as a full one) is split off: the rows from split_rows on (whole row
// panels) run as a second product in tail_slices slices, one round.  The same plan drives the
// general kernel (FX_GEMM_GENERAL), so the two agree bit for bit.
struct WgradPlan {
    int nj, slices;
    bool fast;
    int64_t split_rows;  // 0: one product
    int tail_slices;
};
static WgradPlan wgrad_plan(int64_t M, int64_t N, int64_t K) {
    WgradPlan p{0, 1, false, 0, 1};
    const char* tw = getenv("FX_WGRAD_TILE");
    const bool want4 = tw && tw[0] == '2' && tw[1] == '5' && tw[2] == '6';
    // M need not divide into whole 256-row panels: the last panel's loads are clamped and its
    // rows past M are not stored (the tied head's (50304, 768) gradient has a half panel)
    if (K % 32 == 0 && K >= 32 * kAsmStages) {
        if (!want4 && N % 192 == 0) p.nj = 3;
        else if (N % 256 == 0) p.nj = 4;
    }
    const int64_t tiles = p.nj ? ((M + 255) / 256) * (N / (64 * p.nj))
                               : ((M + kGBM - 1) / kGBM) * ((N + kGBN - 1) / kGBN);
    const int64_t nk = (K + kWBK - 1) / kWBK;
    const int64_t cus = device_cus();
    auto slices_for = [&](int64_t t) {
        int64_t sl = cus / t;
        if (sl > nk / 4) sl = nk / 4;
        if (sl > 32) sl = 32;
        return sl < 1 ? 1 : (int)sl;
    };
    p.slices = slices_for(tiles);
    p.fast = p.nj != 0 && whole_tile_kernels_enabled('w');
    if (p.nj && p.slices == 1 && tiles > cus) {
        const int64_t nn = N / (64 * p.nj), panels = (M + 255) / 256;
        const int64_t full = (tiles / cus) * cus / nn;  // row panels that fill whole rounds
        if (full > 0 && full < panels) {
            const int tail = slices_for((panels - full) * nn);
            if (tail >= 2) {
                p.split_rows = 256 * full;
                p.tail_slices = tail;
            }
        }
    }
    return p;
}

extern "C" int64_t fx_linear_wgrad_workspace(int64_t M, int64_t N, int64_t K) {
    if (M <= 0 || N <= 0 || K <= 0) return 0;
    const WgradPlan p = wgrad_plan(M, N, K);
    if (p.split_rows) return (int64_t)p.tail_slices * (M - p.split_rows) * N * (int64_t)sizeof(float);
    return p.slices > 1 ? (int64_t)p.slices * M * N * (int64_t)sizeof(float) : 0;
}

extern "C" int fx_linear_wgrad(const uint16_t* dY, int64_t ldy, const uint16_t* X, int64_t ldx, uint16_t* dW,
                               int64_t ldw, float* work, int64_t M, int64_t N, int64_t K, void* stream) {
    FX_REQUIRE(dW && (K == 0 || (dY && X)), "fx_linear_wgrad: null pointer");
    FX_REQUIRE(M >= 8 && N >= 8 && K >= 0 && M % 8 == 0 && N % 8 == 0,
               "fx_linear_wgrad: bad shape M=%lld N=%lld K=%lld (M, N multiples of 8)", (long long)M,
               (long long)N, (long long)K);
    FX_REQUIRE(M < 0x7fffffffLL && N < 0x7fffffffLL && K < 0x7fffffffLL && M * N < 0x7fffffffLL * 8,
               "fx_linear_wgrad: size too large");
    FX_REQUIRE(ldy >= M && ldx >= N && ldw >= N && ldy % 8 == 0 && ldx % 8 == 0 && ldw % 8 == 0,
               "fx_linear_wgrad: bad leading dimension (ldy=%lld ldx=%lld ldw=%lld)", (long long)ldy,
               (long long)ldx, (long long)ldw);
    FX_REQUIRE(((((uintptr_t)dY) | ((uintptr_t)X) | ((uintptr_t)dW) | ((uintptr_t)work)) & 15) == 0,
               "fx_linear_wgrad: dY, X, dW and work must be 16-byte aligned");
    const WgradPlan plan = K > 0 ? wgrad_plan(M, N, K) : WgradPlan{0, 1, false, 0, 1};
    FX_REQUIRE((plan.slices == 1 && !plan.split_rows) || work != nullptr,
               "fx_linear_wgrad: null workspace (%d slices)", plan.split_rows ? plan.tail_slices : plan.slices);
    hipStream_t s = (hipStream_t)stream;
    // rows [r0, r0 + rows) of dW in `slices` slices
    auto product = [&](int64_t r0, int64_t rows, int slices) -> int {
        WgradArgs a;
        a.A = dY + r0;
        a.lda = ldy;
        a.B = X;
        a.ldb = ldx;
        a.C = dW + r0 * ldw;
        a.ldc = ldw;
        a.part = work;
        a.M = (int)rows;
        a.N = (int)N;
        a.K = (int)K;
        a.slices = slices;
        // whole tiles and 32-token steps, every slice at least 4 steps: the generated loop (with
        // several slices each spans at least 4 64-token steps, the last perhaps 32 tokens short)
        if (plan.fast) {
            const int64_t tiles = ((rows + 255) / 256) * (N / (64 * plan.nj));
            if (plan.nj == 4)
                hipLaunchKernelGGL(gemm_wgrad_fast_kernel<4>, dim3((unsigned)(tiles * slices)), dim3(256), 0, s, a);
            else
                hipLaunchKernelGGL(gemm_wgrad_fast_kernel<3>, dim3((unsigned)(tiles * slices)), dim3(256), 0, s, a);
        } else {
            const int64_t tiles = ((rows + kGBM - 1) / kGBM) * ((N + kGBN - 1) / kGBN);
            hipLaunchKernelGGL(gemm_wgrad_kernel, dim3((unsigned)(tiles * slices)), dim3(kGThreads), 0, s, a);
        }
        if (int e = check_launch("gemm_wgrad")) return e;
        if (slices == 1) return 0;
        int64_t blocks = (rows * N / 8 + 255) / 256;
        if (blocks > 4096) blocks = 4096;
        hipLaunchKernelGGL(wgrad_reduce_kernel, dim3((unsigned)blocks), dim3(256), 0, s, (const float*)work, slices,
                           rows * N, (int)N, a.C, ldw);
        return check_launch("wgrad_reduce");
    };
    if (!plan.split_rows) return product(0, M, plan.slices);
    if (int e = product(0, plan.split_rows, 1)) return e;
    return product(plan.split_rows, M - plan.split_rows, plan.tail_slices);
}

// the tile width (in 64-column units) of gemm_dgrad_fast_kernel for N columns: of the widths
// that divide N, the one with the fewest MFMA rounds per CU; 0 if none divides it
static int dgrad_nj(int64_t M, int64_t N) {
    const int64_t cus = device_cus();
    int64_t best = 0, nj = 0;
    for (int w : {4, 3}) {
        if (N % (64 * w)) continue;
        const int64_t cost = ((M / 256) * (N / (64 * w)) + cus - 1) / cus * w;
        if (nj == 0 || cost < best) best = cost, nj = w;
    }
    return (int)nj;
}

// EPI 0: dX = dY W; 1: H the pre-activation of a GELU layer, dX = bf16(dY W) gelu'(H);
// 2: H the GELU derivative itself, dX = bf16(dY W) H
static int dgrad_run(const char* fn, const uint16_t* dY, int64_t ldy, const uint16_t* W, int64_t ldw,
                     const uint16_t* H, int epi, uint16_t* dX, int64_t ldx, int64_t M, int64_t N, int64_t K,
                     void* stream) {
    FX_REQUIRE(dY && W && dX && (epi == 0 || H), "%s: null pointer", fn);
    FX_REQUIRE(M >= 0 && N >= 1 && K >= 1, "%s: bad shape M=%lld N=%lld K=%lld", fn, (long long)M, (long long)N,
               (long long)K);
    FX_REQUIRE(M < 0x7fffffffLL && N < 0x7fffffffLL && K < 0x7fffffffLL, "%s: size too large", fn);
    const int nj = dgrad_nj(M, N);
    FX_REQUIRE(M % 256 == 0 && nj != 0 && K % 32 == 0 && K >= 32 * kAsmStages,
               "%s: whole tiles only (M %% 256, N %% 256 or %% 192, K %% 32 == 0, K >= 128): "
               "M=%lld N=%lld K=%lld", fn, (long long)M, (long long)N, (long long)K);
    FX_REQUIRE(ldy >= K && ldw >= N && ldx >= N && ldy % 8 == 0 && ldw % 8 == 0 && ldx % 8 == 0,
               "%s: bad leading dimension (ldy=%lld ldw=%lld ldx=%lld)", fn, (long long)ldy, (long long)ldw,
               (long long)ldx);
    FX_REQUIRE(((((uintptr_t)dY) | ((uintptr_t)W) | ((uintptr_t)H) | ((uintptr_t)dX)) & 15) == 0,
               "%s: dY, W, H and dX must be 16-byte aligned", fn);
    if (M == 0) return 0;
    DgradArgs a{dY, ldy, W, ldw, H, dX, ldx, (int)M, (int)N, (int)K};
    const unsigned tiles = (unsigned)((M / 256) * (N / (64 * nj)));
    hipStream_t s = (hipStream_t)stream;
#define FX_DGRAD(J, E) hipLaunchKernelGGL((gemm_dgrad_fast_kernel<J, E>), dim3(tiles), dim3(256), 0, s, a)
    if (nj == 4) {
        if (epi == 2) FX_DGRAD(4, 2);
        else if (epi == 1) FX_DGRAD(4, 1);
        else FX_DGRAD(4, 0);
    } else {
        if (epi == 2) FX_DGRAD(3, 2);
        else if (epi == 1) FX_DGRAD(3, 1);
        else FX_DGRAD(3, 0);
    }
#undef FX_DGRAD
    return check_launch("gemm_dgrad");
}

extern "C" int fx_linear_dgrad(const uint16_t* dY, int64_t ldy, const uint16_t* W, int64_t ldw, const uint16_t* H,
                               uint16_t* dX, int64_t ldx, int64_t M, int64_t N, int64_t K, void* stream) {
    return dgrad_run("fx_linear_dgrad", dY, ldy, W, ldw, H, H ? 1 : 0, dX, ldx, M, N, K, stream);
}

extern "C" int fx_linear_dgrad_gate(const uint16_t* dY, int64_t ldy, const uint16_t* W, int64_t ldw,
                                    const uint16_t* G, uint16_t* dX, int64_t ldx, int64_t M, int64_t N, int64_t K,
                                    void* stream) {
    return dgrad_run("fx_linear_dgrad_gate", dY, ldy, W, ldw, G, 2, dX, ldx, M, N, K, stream);
}

extern "C" int fx_gelu_bwd(const uint16_t* dy, const uint16_t* h, uint16_t* dh, int64_t n, void* stream) {
    FX_REQUIRE(n >= 0 && (n == 0 || (dy && h && dh)), "fx_gelu_bwd: null pointer");
    FX_REQUIRE(((((uintptr_t)dy) | ((uintptr_t)h) | ((uintptr_t)dh)) & 15) == 0,
               "fx_gelu_bwd: buffers must be 16-byte aligned");
    if (n == 0) return 0;
    int64_t blocks = (n / 8 + 255) / 256;
    if (blocks > 16384) blocks = 16384;
    if (blocks < 1) blocks = 1;
    hipLaunchKernelGGL(gelu_bwd_kernel, dim3((unsigned)blocks), dim3(256), 0, (hipStream_t)stream, dy, h, dh, n);
    return check_launch("gelu_bwd");
}

extern "C" int fx_gelu_bwd_gate(const uint16_t* dy, const uint16_t* g, uint16_t* dh, int64_t n, void* stream) {
    FX_REQUIRE(n >= 0 && (n == 0 || (dy && g && dh)), "fx_gelu_bwd_gate: null pointer");
    FX_REQUIRE(((((uintptr_t)dy) | ((uintptr_t)g) | ((uintptr_t)dh)) & 15) == 0,
               "fx_gelu_bwd_gate: buffers must be 16-byte aligned");
    if (n == 0) return 0;
    int64_t blocks = (n / 8 + 255) / 256;
    if (blocks > 16384) blocks = 16384;
    if (blocks < 1) blocks = 1;
    hipLaunchKernelGGL(gate_mul_kernel, dim3((unsigned)blocks), dim3(256), 0, (hipStream_t)stream, dy, g, dh, n);
    return check_launch("gate_mul");
}

// ---------------------------------------------------------------------------
// fused linear cross-entropy

// the tile width (64-column units) of the linear-CE kernels for V columns, or 0 when the
// shape is not theirs (V a multiple of 256 or 192, K % 32 == 0, K >= 128)
static int lce_nj(int64_t M, int64_t V, int64_t K) {
    if (M < 1 || V < 1 || K % 32 || K < 32 * kAsmStages) return 0;
    if (M >= 0x7fffffffLL || V >= 0x7fffffffLL || K >= 0x7fffffffLL) return 0;
    const int64_t cus = device_cus();
    int64_t best = 0, nj = 0;
    for (int w : {4, 3}) {
        if (V % (64 * w)) continue;
        const int64_t tiles = ((M + 255) / 256) * (V / (64 * w));
        if (tiles >= 0x7fffffffLL) continue;
        const int64_t cost = (tiles + cus - 1) / cus * w;
        if (nj == 0 || cost < best) best = cost, nj = w;
    }
    return (int)nj;
}

static int64_t lce_part_bytes(int64_t M, int64_t V, int nj) { return ((V / (64 * nj)) * M * 8 + 255) / 256 * 256; }

extern "C" int64_t fx_lce_workspace(int64_t M, int64_t V, int64_t K) {
    const int nj = lce_nj(M, V, K);
    return nj ? lce_part_bytes(M, V, nj) + (M * 4 + 255) / 256 * 256 : 0;
}

static int lce_check(const char* fn, const uint16_t* X, int64_t ldx, const uint16_t* E, const int64_t* target,
                     int64_t M, int64_t V, int64_t K, int& nj) {
    FX_REQUIRE(X && E && target, "%s: null pointer", fn);
    FX_REQUIRE(M >= 0 && V >= 1 && K >= 1, "%s: bad shape M=%lld V=%lld K=%lld", fn, (long long)M, (long long)V,
               (long long)K);
    nj = M == 0 ? 0 : lce_nj(M, V, K);
    FX_REQUIRE(M == 0 || nj != 0,
               "%s: V %% 256 or %% 192 == 0, K %% 32 == 0 and K >= 128 only: M=%lld V=%lld K=%lld", fn, (long long)M,
               (long long)V, (long long)K);
    FX_REQUIRE(ldx >= K && ldx % 8 == 0, "%s: ldx=%lld", fn, (long long)ldx);
    FX_REQUIRE(((((uintptr_t)X) | ((uintptr_t)E)) & 15) == 0, "%s: X and E must be 16-byte aligned", fn);
    return 0;
}

extern "C" int fx_lce_fwd(const uint16_t* X, int64_t ldx, const uint16_t* E, const int64_t* target,
                          int64_t ignore_index, void* work, float* stat, float* row_loss, int64_t M, int64_t V,
                          int64_t K, void* stream) {
    int nj;
    if (int e = lce_check("fx_lce_fwd", X, ldx, E, target, M, V, K, nj)) return e;
    if (M == 0) return 0;
    FX_REQUIRE(work && stat && row_loss, "fx_lce_fwd: null workspace or output");
    FX_REQUIRE(((((uintptr_t)work) | ((uintptr_t)stat)) & 15) == 0, "fx_lce_fwd: work and stat must be 16-byte aligned");
    LceArgs a{};
    a.X = X, a.ldx = ldx, a.E = E, a.target = target, a.ignore_index = ignore_index;
    a.part = reinterpret_cast<float2*>(work);
    a.xt = reinterpret_cast<float*>((char*)work + lce_part_bytes(M, V, nj));
    a.stat = reinterpret_cast<float2*>(stat);
    a.M = (int)M, a.V = (int)V, a.K = (int)K;
    const int ntiles = (int)(V / (64 * nj));
    const unsigned tiles = (unsigned)(((M + 255) / 256) * ntiles);
    hipStream_t s = (hipStream_t)stream;
    if (nj == 4) hipLaunchKernelGGL(lce_stats_kernel<4>, dim3(tiles), dim3(256), 0, s, a);
    else hipLaunchKernelGGL(lce_stats_kernel<3>, dim3(tiles), dim3(256), 0, s, a);
    if (int e = check_launch("lce_stats")) return e;
    hipLaunchKernelGGL(lce_combine_kernel, dim3((unsigned)((M + 15) / 16)), dim3(256), 0, s, a, ntiles, row_loss);
    return check_launch("lce_combine");
}

extern "C" int fx_lce_grad(const uint16_t* X, int64_t ldx, const uint16_t* E, const int64_t* target,
                           int64_t ignore_index, const float* stat, const float* mul, uint16_t* dl, int64_t ldd,
                           int64_t M, int64_t V, int64_t K, void* stream) {
    int nj;
    if (int e = lce_check("fx_lce_grad", X, ldx, E, target, M, V, K, nj)) return e;
    if (M == 0) return 0;
    FX_REQUIRE(stat && mul && dl, "fx_lce_grad: null stat, mul or dl");
    FX_REQUIRE(ldd >= V && ldd % 8 == 0 && ((uintptr_t)dl & 15) == 0 && ((uintptr_t)stat & 7) == 0,
               "fx_lce_grad: dl needs a row stride >= V, a multiple of 8, and 16-byte alignment (ldd=%lld)",
               (long long)ldd);
    LceArgs a{};
    a.X = X, a.ldx = ldx, a.E = E, a.target = target, a.ignore_index = ignore_index;
    a.stat = const_cast<float2*>(reinterpret_cast<const float2*>(stat));
    a.mul = mul, a.dl = dl, a.ldd = ldd;
    a.M = (int)M, a.V = (int)V, a.K = (int)K;
    const unsigned tiles = (unsigned)(((M + 255) / 256) * (V / (64 * nj)));
    hipStream_t s = (hipStream_t)stream;
    if (nj == 4) hipLaunchKernelGGL(lce_grad_kernel<4>, dim3(tiles), dim3(256), 0, s, a);
    else hipLaunchKernelGGL(lce_grad_kernel<3>, dim3(tiles), dim3(256), 0, s, a);
    return check_launch("lce_grad");
}
