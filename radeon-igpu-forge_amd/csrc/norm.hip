// RMSNorm forward / backward for gfx950.
//
// Row layout shared by both kernels: a "row group" of LPR consecutive lanes owns one
// row.  Lane j of the group holds the 16-byte vectors j, j+LPR, ..., j+(NV-1)*LPR of
// the row (8 bf16 each), so every load and store is a coalesced 128-bit access and
// the row statistics are a butterfly reduction inside the group (no LDS, no barrier).
// LPR divides 64, so a group never straddles two waves.
//
// Semantics follow ml/fxlm/kernels/norm.hip:32-127 (fp32 math, bf16 I/O here):
//   rstd = rsqrt(mean(x^2) + eps); y = (x * rstd) * w
//   dx = rstd * w * dy - x * (rstd^3 * sum(x*w*dy) / D)
//   dw = sum_rows x * rstd * dy
#include "fx_device.h"

namespace fx {

// ADD: the row is x + radd instead (fp32 sum rounded to bf16, as a bf16 tensor add
// rounds it), written to xsum and normalised from those rounded values.
template <int LPR, int NV, bool ADD = false>
__global__ void __launch_bounds__(256)
rms_fwd_kernel(const uint16_t* __restrict__ x, const uint16_t* __restrict__ w,
               uint16_t* __restrict__ y, float* __restrict__ rstd, int64_t N, int D, float eps,
               const uint16_t* __restrict__ radd, uint16_t* __restrict__ xsum) {
    constexpr int G = 256 / LPR;
    const int lane = threadIdx.x % LPR;
    const int64_t row = (int64_t)blockIdx.x * G + threadIdx.x / LPR;
    if (row >= N) return;  // uniform per group: partners of the shuffles below stay active
    const int V8 = D >> 3;
    const uint16_t* xr = x + row * D;

    uint4 xv[NV];
    float ss = 0.f;
    if constexpr (ADD) {
        const uint16_t* rr = radd + row * D;
        uint16_t* sr = xsum + row * D;
        uint4 rv[NV];
#pragma unroll
        for (int i = 0; i < NV; ++i) {
            const int c = i * LPR + lane;
            xv[i] = make_uint4(0u, 0u, 0u, 0u);
            rv[i] = xv[i];
            if (c < V8) {
                xv[i] = ld16_nt(xr + (int64_t)c * 8);
                rv[i] = ld16_nt(rr + (int64_t)c * 8);
            }
        }
#pragma unroll
        for (int i = 0; i < NV; ++i) {
            const int c = i * LPR + lane;
            if (c < V8) {
                float f[8], q[8];
                unpack8(xv[i], f);
                unpack8(rv[i], q);
#pragma unroll
                for (int j = 0; j < 8; ++j) f[j] += q[j];
                xv[i] = pack8(f);
                st16_nt(sr + (int64_t)c * 8, xv[i]);
            }
            float f[8];
            unpack8(xv[i], f);
#pragma unroll
            for (int j = 0; j < 8; ++j) ss += f[j] * f[j];
        }
    } else {
#pragma unroll
        for (int i = 0; i < NV; ++i) {
            const int c = i * LPR + lane;
            xv[i] = make_uint4(0u, 0u, 0u, 0u);
            if (c < V8) xv[i] = ld16_nt(xr + (int64_t)c * 8);
            float f[8];
            unpack8(xv[i], f);
#pragma unroll
            for (int j = 0; j < 8; ++j) ss += f[j] * f[j];
        }
    }
    ss = group_sum<LPR>(ss);
    const float r = rsqrtf(ss / (float)D + eps);
    if (lane == 0) rstd[row] = r;

    uint16_t* yr = y + row * D;
#pragma unroll
    for (int i = 0; i < NV; ++i) {
        const int c = i * LPR + lane;
        if (c < V8) {
            float f[8], g[8], o[8];
            unpack8(xv[i], f);
            unpack8(ld16(w + c * 8), g);
#pragma unroll
            for (int j = 0; j < 8; ++j) o[j] = (f[j] * r) * g[j];
            st16_nt(yr + (int64_t)c * 8, pack8(o));
        }
    }
}

// dx for the rows dealt to this block, plus the block's partial dw (fp32, one row of
// `part` per block).  Rows are dealt round-robin over the whole grid, so all blocks
// stream one window of consecutive rows at a time (DRAM pages stay open, as in a
// plain copy); per-block strips of consecutive rows measured about 10% slower.
// The row groups of a wave fold their dw partials with lane exchanges and the waves
// then fold through LDS in a fixed order (deterministic).
constexpr int kNormBwdThreads = 512;

template <int LPR, int NV>
struct NormBwdRow {
    uint4 xv[NV], dv[NV], rv[NV];  // x, dy and (dres != null) the residual gradient
    float r;
    __device__ __forceinline__ void load(const uint16_t* __restrict__ x, const uint16_t* __restrict__ dy,
                                         const uint16_t* __restrict__ dres, const float* __restrict__ rstd,
                                         int64_t row, int64_t n, int D, int lane) {
        if (row >= n) return;  // past the last row: nothing is read (uniform per row group)
        const uint16_t* xr = x + row * D;
        const uint16_t* dr = dy + row * D;
        const int V8 = D >> 3;
#pragma unroll
        for (int i = 0; i < NV; ++i) {
            const int c = i * LPR + lane;
            xv[i] = make_uint4(0u, 0u, 0u, 0u);
            dv[i] = make_uint4(0u, 0u, 0u, 0u);
            rv[i] = make_uint4(0u, 0u, 0u, 0u);
            if (c < V8) {
                xv[i] = ld16_nt(xr + (int64_t)c * 8);
                dv[i] = ld16_nt(dr + (int64_t)c * 8);
                if (dres) rv[i] = ld16_nt(dres + row * D + (int64_t)c * 8);
            }
        }
        r = rstd[row];
    }
};

// `wv`: this lane's vectors of w (zero past D), loaded once per block; `res`: add the
// residual gradient row b.rv to dx
template <int LPR, int NV>
__device__ __forceinline__ void norm_bwd_row(const NormBwdRow<LPR, NV>& b, const uint4 (&wv)[NV],
                                             uint16_t* __restrict__ dxr, float (&acc)[NV][8], int D,
                                             float invD, int lane, bool res) {
    const int V8 = D >> 3;
    float t = 0.f;
#pragma unroll
    for (int i = 0; i < NV; ++i) {
        float fx_[8], fd[8], fw[8];
        unpack8(b.xv[i], fx_);
        unpack8(b.dv[i], fd);
        unpack8(wv[i], fw);
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            t = fmaf(fx_[j] * fw[j], fd[j], t);
            acc[i][j] = fmaf(fx_[j] * b.r, fd[j], acc[i][j]);
        }
    }
    t = group_sum<LPR>(t);
    const float corr = b.r * b.r * b.r * t * invD;
#pragma unroll
    for (int i = 0; i < NV; ++i) {
        const int c = i * LPR + lane;
        if (c < V8) {
            float fx_[8], fd[8], fw[8], o[8];
            unpack8(b.xv[i], fx_);
            unpack8(b.dv[i], fd);
            unpack8(wv[i], fw);
#pragma unroll
            for (int j = 0; j < 8; ++j) o[j] = fmaf(b.r * fw[j], fd[j], -fx_[j] * corr);
            if (res) {
                float fr[8];
                unpack8(b.rv[i], fr);
#pragma unroll
                for (int j = 0; j < 8; ++j) o[j] += fr[j];
            }
            st16_nt(dxr + (int64_t)c * 8, pack8(o));
        }
    }
}

// waves per SIMD to budget registers for (two 512-thread blocks per CU up to 3
// vectors per lane)
template <int NV>
constexpr int norm_bwd_min_waves() { return NV <= 3 ? 4 : 2; }

// One row per row group per iteration: loading two rows before reducing either needs
// the registers of a wave per SIMD (5.5 % slower at [65536, 768]); occupancy hides the loads.
template <int LPR, int NV, int NT = kNormBwdThreads, int MW = norm_bwd_min_waves<NV>()>
__global__ void __launch_bounds__(NT, MW)
rms_bwd_kernel(const uint16_t* __restrict__ x, const uint16_t* __restrict__ dy,
               const uint16_t* __restrict__ w, const float* __restrict__ rstd,
               const uint16_t* __restrict__ dres, uint16_t* __restrict__ dx, float* __restrict__ part, int64_t N,
               int D) {
    constexpr int G = NT / LPR;
    constexpr int NW = NT / 64;
    extern __shared__ float red[];  // NW x D floats
    const int lane = threadIdx.x % LPR;
    const int grp = threadIdx.x / LPR;
    const int V8 = D >> 3;
    const float invD = 1.f / (float)D;

    float acc[NV][8];
#pragma unroll
    for (int i = 0; i < NV; ++i)
#pragma unroll
        for (int j = 0; j < 8; ++j) acc[i][j] = 0.f;

    // rows are dealt to the blocks' row groups round-robin (row = (k * P + block) * G +
    // group), so at any moment the whole grid streams one window of consecutive rows
    const int64_t stride = (int64_t)gridDim.x * G;
    const int64_t first = (int64_t)blockIdx.x * G + grp;
    uint4 wv[NV];
#pragma unroll
    for (int i = 0; i < NV; ++i) {
        const int c = i * LPR + lane;
        wv[i] = c < V8 ? ld16(w + c * 8) : make_uint4(0u, 0u, 0u, 0u);
    }
    NormBwdRow<LPR, NV> b;
    for (int64_t row = first; row < N; row += stride) {
        b.load(x, dy, dres, rstd, row, N, D, lane);
        norm_bwd_row<LPR, NV>(b, wv, dx + row * D, acc, D, invD, lane, dres != nullptr);
    }

    // row groups sharing a wave: butterfly over the group index
#pragma unroll
    for (int off = LPR; off < 64; off <<= 1)
#pragma unroll
        for (int i = 0; i < NV; ++i)
#pragma unroll
            for (int j = 0; j < 8; ++j) acc[i][j] += __shfl_xor(acc[i][j], off, 64);
    // waves: each writes its partial row to LDS, one barrier, then every column is summed
    // over the waves in order (1 us faster at [65536, 768] than a wave-by-wave fold with a
    // barrier per wave)
    const int wave = threadIdx.x >> 6;
    float* pr = part + (int64_t)blockIdx.x * D;
    if ((threadIdx.x & 63) < LPR) {
#pragma unroll
        for (int i = 0; i < NV; ++i) {
            const int c = i * LPR + lane;
            if (c < V8) {
                float4* r = reinterpret_cast<float4*>(red + wave * D + c * 8);
                r[0] = make_float4(acc[i][0], acc[i][1], acc[i][2], acc[i][3]);
                r[1] = make_float4(acc[i][4], acc[i][5], acc[i][6], acc[i][7]);
            }
        }
    }
    __syncthreads();
    for (int c = threadIdx.x; c < D; c += NT) {
        float sum = red[c];
        for (int k = 1; k < NW; ++k) sum += red[k * D + c];
        pr[c] = sum;
    }
}

// Backward for D > 1536: the whole 512-thread block owns one row at a time (thread t holds
// the row's 16-byte vectors t and t + 512, so NV <= 2 covers D <= 8192) and loads the
// block's next row while it computes the current one.  The row sum of x * w * dy is a lane
// butterfly per wave and then the 8 wave sums in a fixed order through LDS (double-buffered
// by row parity: one barrier per row).  Each column's dw partial belongs to one thread, so
// the block's partial row is written without a reduction.  The register kernel above held
// up to 16 vectors of x, dy and dw per lane at these widths and spilled up to 1.7 KB per
// lane; here a lane holds at most 2 of each.
template <int NV>
struct WideRow {
    uint4 xv[NV], dv[NV], rv[NV];
    float r;
    __device__ __forceinline__ void load(const uint16_t* __restrict__ x, const uint16_t* __restrict__ dy,
                                         const uint16_t* __restrict__ dres, const float* __restrict__ rstd,
                                         int64_t row, int64_t n, int V8) {
        if (row >= n) return;  // uniform per block
#pragma unroll
        for (int i = 0; i < NV; ++i) {
            const int c = i * kNormBwdThreads + (int)threadIdx.x;
            xv[i] = make_uint4(0u, 0u, 0u, 0u);
            dv[i] = xv[i];
            rv[i] = xv[i];
            if (c < V8) {
                xv[i] = ld16_nt(x + row * V8 * 8 + (int64_t)c * 8);
                dv[i] = ld16_nt(dy + row * V8 * 8 + (int64_t)c * 8);
                if (dres) rv[i] = ld16_nt(dres + row * V8 * 8 + (int64_t)c * 8);
            }
        }
        r = rstd[row];
    }
};

template <int NV>
__global__ void __launch_bounds__(kNormBwdThreads)
rms_bwd_wide_kernel(const uint16_t* __restrict__ x, const uint16_t* __restrict__ dy,
                    const uint16_t* __restrict__ w, const float* __restrict__ rstd,
                    const uint16_t* __restrict__ dres, uint16_t* __restrict__ dx, float* __restrict__ part,
                    int64_t N, int D) {
    constexpr int NW = kNormBwdThreads / 64;
    __shared__ float red[2][NW];
    const int V8 = D >> 3;
    const int wave = threadIdx.x >> 6;
    const float invD = 1.f / (float)D;
    float acc[NV][8];
    uint4 wv[NV];
#pragma unroll
    for (int i = 0; i < NV; ++i) {
        const int c = i * kNormBwdThreads + (int)threadIdx.x;
        wv[i] = c < V8 ? ld16(w + c * 8) : make_uint4(0u, 0u, 0u, 0u);
#pragma unroll
        for (int j = 0; j < 8; ++j) acc[i][j] = 0.f;
    }
    WideRow<NV> cur, nxt;
    int par = 0;
    for (int64_t row = blockIdx.x; row < N; row += gridDim.x, par ^= 1) {
        if (row == blockIdx.x) cur.load(x, dy, dres, rstd, row, N, V8);
        nxt.load(x, dy, dres, rstd, row + gridDim.x, N, V8);
        float t = 0.f;
#pragma unroll
        for (int i = 0; i < NV; ++i) {
            float fx_[8], fd[8], fw[8];
            unpack8(cur.xv[i], fx_);
            unpack8(cur.dv[i], fd);
            unpack8(wv[i], fw);
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                t = fmaf(fx_[j] * fw[j], fd[j], t);
                acc[i][j] = fmaf(fx_[j] * cur.r, fd[j], acc[i][j]);
            }
        }
        t = group_sum<64>(t);
        if ((threadIdx.x & 63) == 0) red[par][wave] = t;
        __syncthreads();
        float tot = red[par][0];
#pragma unroll
        for (int k = 1; k < NW; ++k) tot += red[par][k];
        const float corr = cur.r * cur.r * cur.r * tot * invD;
#pragma unroll
        for (int i = 0; i < NV; ++i) {
            const int c = i * kNormBwdThreads + (int)threadIdx.x;
            if (c < V8) {
                float fx_[8], fd[8], fw[8], o[8];
                unpack8(cur.xv[i], fx_);
                unpack8(cur.dv[i], fd);
                unpack8(wv[i], fw);
#pragma unroll
                for (int j = 0; j < 8; ++j) o[j] = fmaf(cur.r * fw[j], fd[j], -fx_[j] * corr);
                if (dres) {
                    float fr[8];
                    unpack8(cur.rv[i], fr);
#pragma unroll
                    for (int j = 0; j < 8; ++j) o[j] += fr[j];
                }
                st16_nt(dx + row * D + (int64_t)c * 8, pack8(o));
            }
        }
        cur = nxt;
    }
    float* pr = part + (int64_t)blockIdx.x * D;
#pragma unroll
    for (int i = 0; i < NV; ++i) {
        const int c = i * kNormBwdThreads + (int)threadIdx.x;
        if (c < V8) {
            float4* o = reinterpret_cast<float4*>(pr + c * 8);
            o[0] = make_float4(acc[i][0], acc[i][1], acc[i][2], acc[i][3]);
            o[1] = make_float4(acc[i][4], acc[i][5], acc[i][6], acc[i][7]);
        }
    }
}

// Backward for 512 <= D <= 1536 with the rows prefetched into LDS.  Each wave owns one
// row per step (64 lanes, lane j holding 16-byte vectors j, j + 64, ...) and keeps the
// next S - 1 rows in flight in a private ring of S slots, each slot the row's x, dy and
// (T == 3) dres plus its rstd, filled by global_load_lds (no registers held for the
// prefetch, which the register kernel above cannot afford: loading the next row into
// registers spilled).  One 512-thread block per CU (256 blocks): at [65536, 768] 50.2 us
// against 54.3 us for the register kernel (75 % against 70 % of HBM), with dres 64.6
// against 74.3 us; dx is bit for bit the register kernel's, dw the same sum over half as
// many partial rows.
//
// Waits: every prefetched row is GOPS = T * NV + 1 vector-memory instructions (a masked
// instruction still counts) and every computed row NV stores; completion is in issue
// order, so row k has landed once at most (S - 1) * GOPS + min(k, S - 1) * NV
// instructions are outstanding (the loads of rows k + 1 .. k + S - 1 and the stores of
// the rows before k issued after row k's loads).  The last S - 1 rows wait for all.
constexpr int kNormLdsBlocks = 256;  // one per CU

template <int NV, int T, int S>
__global__ void __launch_bounds__(kNormBwdThreads, 2)
rms_bwd_lds_kernel(const uint16_t* __restrict__ x, const uint16_t* __restrict__ dy,
                   const uint16_t* __restrict__ dres, const uint16_t* __restrict__ w,
                   const float* __restrict__ rstd, uint16_t* __restrict__ dx, float* __restrict__ part,
                   int64_t N, int D) {
    constexpr int NT = kNormBwdThreads, NW = NT / 64, LPR = 64;
    constexpr int GOPS = T * NV + 1;
    extern __shared__ __attribute__((aligned(16))) unsigned char ring_mem[];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int V8 = D >> 3;
    const int RB = D * 2;          // bytes of one bf16 row
    const int SB = T * RB + 16;    // bytes of one slot: T rows, then rstd
    unsigned char* ring = ring_mem + wave * S * SB;
    const uint32_t ring_lds = __builtin_amdgcn_readfirstlane(lds_addr(ring));
    // rows first, first + stride, ... (the register kernel's assignment for 64-lane rows)
    const int64_t stride = (int64_t)gridDim.x * NW;
    const int64_t first = (int64_t)blockIdx.x * NW + wave;
    const int nrows = first < N ? (int)((N - 1 - first) / stride + 1) : 0;
    const float invD = 1.f / (float)D;

    float acc[NV][8];
#pragma unroll
    for (int i = 0; i < NV; ++i)
#pragma unroll
        for (int j = 0; j < 8; ++j) acc[i][j] = 0.f;
    uint4 wv[NV];
#pragma unroll
    for (int i = 0; i < NV; ++i) {
        const int c = i * LPR + lane;
        wv[i] = c < V8 ? ld16(w + c * 8) : make_uint4(0u, 0u, 0u, 0u);
    }
    // row k of this wave into slot s: NV instructions per tensor (the last one with the
    // lanes c < V8, at least one), then rstd by lane 0
    auto prefetch = [&](int k, int s) {
        const int64_t row = first + (int64_t)k * stride;
        const uint32_t slot = ring_lds + s * SB;
#pragma unroll
        for (int t = 0; t < T; ++t) {
            const uint16_t* src = (t == 0 ? x : t == 1 ? dy : dres) + row * D;
#pragma unroll
            for (int i = 0; i < NV; ++i) {
                const int c = i * LPR + lane;
                if (c < V8) dma16(src + c * 8, slot + t * RB + i * 1024);
            }
        }
        if (lane == 0) dma4(rstd + row, slot + T * RB);
    };
#pragma unroll
    for (int s = 0; s < S - 1; ++s)
        if (s < nrows) prefetch(s, s);
    for (int k0 = 0; k0 < nrows; k0 += S) {
#pragma unroll
        for (int s = 0; s < S; ++s) {
            const int k = k0 + s;
            if (k >= nrows) break;
            if (k + S - 1 < nrows) {
                prefetch(k + S - 1, (s + S - 1) % S);
                if (k0 == 0) wait_vmcnt_folded(GOPS * (S - 1) + NV * s);
                else wait_vmcnt_folded((GOPS + NV) * (S - 1));
            } else {
                wait_vmcnt<0>();
            }
            const unsigned char* sl = ring + s * SB;
            NormBwdRow<LPR, NV> b;
#pragma unroll
            for (int i = 0; i < NV; ++i) {
                const int c = i * LPR + lane;
                b.xv[i] = b.dv[i] = b.rv[i] = make_uint4(0u, 0u, 0u, 0u);
                if (c < V8) {
                    b.xv[i] = *reinterpret_cast<const uint4*>(sl + c * 16);
                    b.dv[i] = *reinterpret_cast<const uint4*>(sl + RB + c * 16);
                    if (T == 3) b.rv[i] = *reinterpret_cast<const uint4*>(sl + 2 * RB + c * 16);
                }
            }
            b.r = *reinterpret_cast<const float*>(sl + T * RB);
            norm_bwd_row<LPR, NV>(b, wv, dx + (first + (int64_t)k * stride) * D, acc, D, invD, lane, T == 3);
            asm volatile("" ::: "memory");  // the slot's reads stay before its next prefetch
        }
    }

    // dw partial of the block: as the register kernel's per-wave fold, in the ring's LDS
    __syncthreads();  // every wave is done with its ring
    float* red = reinterpret_cast<float*>(ring_mem);
#pragma unroll
    for (int i = 0; i < NV; ++i) {
        const int c = i * LPR + lane;
        if (c < V8) {
            float4* r = reinterpret_cast<float4*>(red + wave * D + c * 8);
            r[0] = make_float4(acc[i][0], acc[i][1], acc[i][2], acc[i][3]);
            r[1] = make_float4(acc[i][4], acc[i][5], acc[i][6], acc[i][7]);
        }
    }
    __syncthreads();
    float* pr = part + (int64_t)blockIdx.x * D;
    for (int c = threadIdx.x; c < D; c += NT) {
        float sum = red[c];
        for (int k = 1; k < NW; ++k) sum += red[k * D + c];
        pr[c] = sum;
    }
}

// dw[c] = sum_p part[p][c] in a fixed order.  A block owns 8 columns (2 float4 lanes)
// and 128 partial-row lanes (32 per wave): each thread sums every 128th partial row of
// its 4 columns with its loads in flight, the row lanes of a wave fold with a butterfly
// (every lane ends with the same bits) and the 4 waves through LDS.  96 blocks at D = 768
// (16-column blocks with 64 row lanes: 0.3 us slower).
__global__ void __launch_bounds__(256)
rms_dw_reduce_kernel(const float* __restrict__ part, int64_t P, int D, float* __restrict__ dw_f32,
                     uint16_t* __restrict__ dw) {
    __shared__ float4 red[4][2];
    const int cg = threadIdx.x & 1, rl = threadIdx.x >> 1;
    const int col = blockIdx.x * 8 + cg * 4;
    float4 s = make_float4(0.f, 0.f, 0.f, 0.f);
    if (col < D) {
#pragma unroll 8
        for (int64_t p = rl; p < P; p += 128) {
            const float4 v = *reinterpret_cast<const float4*>(part + p * D + col);
            s.x += v.x; s.y += v.y; s.z += v.z; s.w += v.w;
        }
    }
#pragma unroll
    for (int off = 2; off < 64; off <<= 1) {
        s.x += __shfl_xor(s.x, off, 64);
        s.y += __shfl_xor(s.y, off, 64);
        s.z += __shfl_xor(s.z, off, 64);
        s.w += __shfl_xor(s.w, off, 64);
    }
    const int wave = threadIdx.x >> 6;
    if ((threadIdx.x & 63) < 2) red[wave][cg] = s;
    __syncthreads();
    if (threadIdx.x < 2 && col < D) {
        float4 t = red[0][cg];
#pragma unroll
        for (int k = 1; k < 4; ++k) {
            const float4 v = red[k][cg];
            t.x += v.x; t.y += v.y; t.z += v.z; t.w += v.w;
        }
        *reinterpret_cast<float4*>(dw_f32 + col) = t;
        if (dw) {
            uint2 u;
            u.x = pack_bf16x2(t.x, t.y);
            u.y = pack_bf16x2(t.z, t.w);
            *reinterpret_cast<uint2*>(dw + col) = u;
        }
    }
}

// ---------------------------------------------------------------------------
// host dispatch

struct RowShape {
    int lpr, nv;
};

// Pick the (LPR, NV) instantiation covering D/8 vectors with the fewest idle slots,
// preferring wider groups on ties.
static RowShape pick_shape(int D) {
    static const int lprs[] = {64, 32, 16, 8};
    static const int nvs[] = {1, 2, 3, 4, 6, 8, 12, 16};
    const int v8 = D / 8;
    RowShape best{0, 0};
    int best_waste = 1 << 30;
    for (int l : lprs)
        for (int n : nvs)
            if (l * n >= v8 && l * n - v8 < best_waste) {
                best_waste = l * n - v8;
                best = {l, n};
            }
    return best;
}

// Backward, register kernel (D < 512, below the LDS-ring kernel's range): one vector per
// lane, the narrowest row group that covers the row.
constexpr int kNormRegMaxD = 1536;  // wider rows: rms_bwd_wide_kernel
static RowShape pick_bwd_shape(int D) {
    static const int lprs[] = {8, 16, 32, 64};
    const int v8 = D / 8;
    for (int l : lprs)
        if (l >= v8) return {l, 1};
    return {64, 1};
}

#define FX_NORM_NV_CASES(LPR, CALL) \
    case 1: CALL(LPR, 1); break;    \
    case 2: CALL(LPR, 2); break;    \
    case 3: CALL(LPR, 3); break;    \
    case 4: CALL(LPR, 4); break;    \
    case 6: CALL(LPR, 6); break;    \
    case 8: CALL(LPR, 8); break;    \
    case 12: CALL(LPR, 12); break;  \
    case 16: CALL(LPR, 16); break;

#define FX_NORM_DISPATCH(shape, CALL)                                           \
    switch (shape.lpr) {                                                        \
        case 64: switch (shape.nv) { FX_NORM_NV_CASES(64, CALL) } break;        \
        case 32: switch (shape.nv) { FX_NORM_NV_CASES(32, CALL) } break;        \
        case 16: switch (shape.nv) { FX_NORM_NV_CASES(16, CALL) } break;        \
        case 8: switch (shape.nv) { FX_NORM_NV_CASES(8, CALL) } break;          \
    }

// blocks of the backward (one dw partial each) for `ngroups` row groups of work:
// two per CU on a 256-CU part, never more than there are row groups
static int64_t bwd_blocks(int64_t ngroups) {
    const int64_t target = 512;
    return ngroups < target ? (ngroups > 0 ? ngroups : 1) : target;
}

// The LDS-ring backward takes 512 <= D <= 1536 (1 to 3 vectors per lane), whether or not
// dres is given, so that fx_rms_norm_bwd and fx_rms_norm_bwd_add produce the same dw bits;
// its ring depth is the largest S <= 3 whose 8 waves' slots fit the CU's 160 KB of LDS
// (S >= 2 for every such D, with dres too).
constexpr int kNormLdsBytes = 160 * 1024;
static bool bwd_lds_fits(int D) { return D >= 512 && D <= 1536; }
static int bwd_lds_depth(int D, int T) {
    const int slot = T * D * 2 + 16;
    const int s = kNormLdsBytes / ((kNormBwdThreads / 64) * slot);
    return s < 3 ? s : 3;
}

}  // namespace fx

using namespace fx;

// x and w are read as 16-byte vectors: both must be 16-byte aligned
static int norm_check(const void* x, const void* w, int64_t N, int32_t D, const char* who) {
    FX_REQUIRE((N == 0 || x != nullptr) && w != nullptr, "%s: null pointer", who);
    FX_REQUIRE(N >= 0, "%s: N=%lld < 0", who, (long long)N);
    FX_REQUIRE(D >= 8 && D <= 8192 && D % 8 == 0, "%s: D=%d needs D%%8==0 and 8<=D<=8192", who, D);
    FX_REQUIRE(((((uintptr_t)x) | ((uintptr_t)w)) & 15) == 0, "%s: x and w must be 16-byte aligned", who);
    return 0;
}

extern "C" int fx_rms_norm_fwd(const uint16_t* x, const uint16_t* w, uint16_t* y, float* rstd,
                               int64_t N, int32_t D, float eps, void* stream) {
    if (int e = norm_check(x, w, N, D, "fx_rms_norm_fwd")) return e;
    if (N == 0) return 0;
    FX_REQUIRE(y != nullptr && rstd != nullptr, "fx_rms_norm_fwd: null output");
    FX_REQUIRE(((uintptr_t)y & 15) == 0, "fx_rms_norm_fwd: y must be 16-byte aligned");
    const RowShape s = pick_shape(D);
    const int G = 256 / s.lpr;
    const int64_t blocks = (N + G - 1) / G;
    FX_REQUIRE(blocks <= 0x7fffffff, "fx_rms_norm_fwd: N=%lld too large", (long long)N);
#define FX_CALL(L, V)                                                                       \
    hipLaunchKernelGGL((rms_fwd_kernel<L, V>), dim3((unsigned)blocks), dim3(256), 0,        \
                       (hipStream_t)stream, x, w, y, rstd, N, (int)D, eps, nullptr, nullptr)
    FX_NORM_DISPATCH(s, FX_CALL)
#undef FX_CALL
    return check_launch("rms_norm_fwd");
}

extern "C" int fx_rms_norm_fwd_add(const uint16_t* x, const uint16_t* r, const uint16_t* w, uint16_t* xsum,
                                   uint16_t* y, float* rstd, int64_t N, int32_t D, float eps, void* stream) {
    if (int e = norm_check(x, w, N, D, "fx_rms_norm_fwd_add")) return e;
    if (N == 0) return 0;
    FX_REQUIRE(r != nullptr && xsum != nullptr && y != nullptr && rstd != nullptr,
               "fx_rms_norm_fwd_add: null pointer");
    FX_REQUIRE(((((uintptr_t)x) | ((uintptr_t)r) | ((uintptr_t)xsum) | ((uintptr_t)y)) & 15) == 0,
               "fx_rms_norm_fwd_add: x, r, xsum and y must be 16-byte aligned");
    const RowShape s = pick_shape(D);
    const int G = 256 / s.lpr;
    const int64_t blocks = (N + G - 1) / G;
    FX_REQUIRE(blocks <= 0x7fffffff, "fx_rms_norm_fwd_add: N=%lld too large", (long long)N);
#define FX_CALL(L, V)                                                                       \
    hipLaunchKernelGGL((rms_fwd_kernel<L, V, true>), dim3((unsigned)blocks), dim3(256), 0,  \
                       (hipStream_t)stream, x, w, y, rstd, N, (int)D, eps, r, xsum)
    FX_NORM_DISPATCH(s, FX_CALL)
#undef FX_CALL
    return check_launch("rms_norm_fwd_add");
}

extern "C" int64_t fx_rms_norm_bwd_workspace(int64_t N, int32_t D) {
    if (N <= 0 || D <= 0) return 0;
    return bwd_blocks(N) * (int64_t)D * (int64_t)sizeof(float);  // >= the blocks any D uses
}

static int rms_norm_bwd(const uint16_t* x, const uint16_t* dy, const uint16_t* dres, const uint16_t* w,
                        const float* rstd, uint16_t* dx, float* dw_f32, uint16_t* dw, float* work, int64_t N,
                        int32_t D, void* stream, const char* who) {
    if (int e = norm_check(x, w, N, D, who)) return e;
    FX_REQUIRE(dw_f32 != nullptr, "%s: null dw", who);
    FX_REQUIRE(((uintptr_t)dw_f32 & 15) == 0 && ((uintptr_t)dw & 7) == 0 && ((uintptr_t)work & 15) == 0,
               "%s: dw_f32 and work must be 16-byte aligned, dw 8-byte aligned", who);
    FX_REQUIRE(N == 0 || (dy != nullptr && rstd != nullptr && dx != nullptr),
               "%s: null pointer", who);
    FX_REQUIRE(((((uintptr_t)dy) | ((uintptr_t)dx) | ((uintptr_t)dres)) & 15) == 0,
               "%s: dy, dx and dres must be 16-byte aligned", who);
    if (N == 0) {
        // dw of an empty batch is zero
        hipLaunchKernelGGL(rms_dw_reduce_kernel, dim3((D + 7) / 8), dim3(256), 0,
                           (hipStream_t)stream, (const float*)nullptr, (int64_t)0, (int)D, dw_f32, dw);
        return check_launch("rms_dw_reduce");
    }
    FX_REQUIRE(work != nullptr, "%s: null workspace", who);
    if (bwd_lds_fits(D)) {
        const int NV = (D / 8 + 63) / 64, T = dres ? 3 : 2, S = bwd_lds_depth(D, T);
        const int64_t rows_per_block = kNormBwdThreads / 64;
        const int64_t P = std::min<int64_t>(kNormLdsBlocks, (N + rows_per_block - 1) / rows_per_block);
        const size_t lds = (size_t)(kNormBwdThreads / 64) * S * (T * D * 2 + 16);
        bool launched = false;
#define FX_LDS(NV_, T_, S_)                                                                            \
    if (NV == NV_ && T == T_ && S == S_) {                                                             \
        hipLaunchKernelGGL((rms_bwd_lds_kernel<NV_, T_, S_>), dim3((unsigned)P), dim3(kNormBwdThreads), \
                           lds, (hipStream_t)stream, x, dy, dres, w, rstd, dx, work, N, (int)D);       \
        launched = true;                                                                               \
    }
        // the (vectors, tensors, depth) triples 512 <= D <= 1536 gives
        FX_LDS(1, 2, 3) FX_LDS(2, 2, 3) FX_LDS(3, 2, 3)
        FX_LDS(1, 3, 3) FX_LDS(2, 3, 3) FX_LDS(3, 3, 3) FX_LDS(3, 3, 2)
#undef FX_LDS
        FX_REQUIRE(launched, "%s: no LDS backward for D=%d", who, D);
        if (int e = check_launch("rms_norm_bwd")) return e;
        hipLaunchKernelGGL(rms_dw_reduce_kernel, dim3((D + 7) / 8), dim3(256), 0, (hipStream_t)stream,
                           (const float*)work, P, (int)D, dw_f32, dw);
        return check_launch("rms_dw_reduce");
    }
    if (D > kNormRegMaxD) {
        const int64_t P = bwd_blocks(N);  // one row per block at a time
        if (D <= 8 * kNormBwdThreads)
            hipLaunchKernelGGL((rms_bwd_wide_kernel<1>), dim3((unsigned)P), dim3(kNormBwdThreads), 0,
                               (hipStream_t)stream, x, dy, w, rstd, dres, dx, work, N, (int)D);
        else
            hipLaunchKernelGGL((rms_bwd_wide_kernel<2>), dim3((unsigned)P), dim3(kNormBwdThreads), 0,
                               (hipStream_t)stream, x, dy, w, rstd, dres, dx, work, N, (int)D);
        if (int e = check_launch("rms_norm_bwd")) return e;
        hipLaunchKernelGGL(rms_dw_reduce_kernel, dim3((D + 7) / 8), dim3(256), 0, (hipStream_t)stream,
                           (const float*)work, P, (int)D, dw_f32, dw);
        return check_launch("rms_dw_reduce");
    }
    const RowShape s = pick_bwd_shape(D);
    const int G = kNormBwdThreads / s.lpr;
    const int64_t P = bwd_blocks((N + G - 1) / G);  // every block gets a row group's worth
    // one LDS partial row per wave (D < 512: 16 KB at most)
    const size_t lds = (size_t)(kNormBwdThreads / 64) * D * sizeof(float);
#define FX_CALL(L)                                                                               \
    hipLaunchKernelGGL((rms_bwd_kernel<L, 1>), dim3((unsigned)P), dim3(kNormBwdThreads), lds,     \
                       (hipStream_t)stream, x, dy, w, rstd, dres, dx, work, N, (int)D)
    switch (s.lpr) {
        case 64: FX_CALL(64); break;
        case 32: FX_CALL(32); break;
        case 16: FX_CALL(16); break;
        default: FX_CALL(8); break;
    }
#undef FX_CALL
    if (int e = check_launch("rms_norm_bwd")) return e;
    hipLaunchKernelGGL(rms_dw_reduce_kernel, dim3((D + 7) / 8), dim3(256), 0, (hipStream_t)stream,
                       (const float*)work, P, (int)D, dw_f32, dw);
    return check_launch("rms_dw_reduce");
}

extern "C" int fx_rms_norm_bwd(const uint16_t* x, const uint16_t* dy, const uint16_t* w,
                               const float* rstd, uint16_t* dx, float* dw_f32, uint16_t* dw,
                               float* work, int64_t N, int32_t D, void* stream) {
    return rms_norm_bwd(x, dy, nullptr, w, rstd, dx, dw_f32, dw, work, N, D, stream, "fx_rms_norm_bwd");
}

extern "C" int fx_rms_norm_bwd_add(const uint16_t* x, const uint16_t* dy, const uint16_t* dres,
                                   const uint16_t* w, const float* rstd, uint16_t* dx, float* dw_f32,
                                   uint16_t* dw, float* work, int64_t N, int32_t D, void* stream) {
    FX_REQUIRE(N == 0 || dres != nullptr, "fx_rms_norm_bwd_add: null dres");
    return rms_norm_bwd(x, dy, dres, w, rstd, dx, dw_f32, dw, work, N, D, stream, "fx_rms_norm_bwd_add");
}
