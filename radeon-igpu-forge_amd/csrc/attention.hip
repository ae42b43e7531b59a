// Flash attention (forward and backward) for gfx950 with bf16 MFMA.
//
// Matrix-core layouts (v_mfma_f32_32x32x16_bf16, wave64):
//   A (32 x 16): lane l supplies row l%32, k = 8*(l/32) + 0..7
//   B (16 x 32): lane l supplies column l%32, k = 8*(l/32) + 0..7
//   C (32 x 32): lane l holds column l%32, rows 8*(i/4) + 4*(l/32) + i%4, i = 0..15
// A product whose K dimension is strided in LDS (V in P.V, K in dS.K, Q / dO in the
// key-side products) is fed with ds_read_b64_tr_b16: within a group of 16 lanes,
// lane s points at row k0 + s/4, column m0 + 4*(s%4) of a row-major tile and lane i
// receives column m0 + i of rows k0..k0+3.  Two such reads give the 8 K-values.
// Accumulator tiles are reused as the next product's operand without any shuffle:
// the 16 values a lane holds for one column are packed as the operand's 8 K-values
// of two 16-wide K chunks, and the other operand's K order is permuted to match
// (positions j < 4 -> 4*g + j, j >= 4 -> 8 + 4*g + j - 4, g = l/32).
//
// Forward: "transposed" scores S^T = K Q^T so each lane owns one query column and the
// row softmax is 15 in-lane steps plus one exchange with lane l^32.
// Backward: per query tile, S^T, dP^T and dQ^T = K^T dS^T (Delta computed in the same
// kernel); per key tile, S = Q K^T, dP = dO V^T, dV^T += dO^T P, dK^T += Q^T dS.
// Semantics follow ml/fxlm/kernels/attention.hip:103-534 (mask key <= query, lse =
// m + log l or -inf, Delta from the bf16 output, dS = P (dP - Delta) scale).
#include <math.h>

#include "fx_device.h"

namespace fx {

constexpr int kAttWaves = 4;
constexpr int kAttThreads = 64 * kAttWaves;
constexpr int kBM = 32 * kAttWaves;  // queries per workgroup (forward, dQ)
constexpr int kBN = 64;              // keys per streamed tile (forward, dQ)
constexpr int kBK = 32 * kAttWaves;  // keys per workgroup (dK/dV)
constexpr int kBQ = 64;              // queries per streamed tile (dK/dV)
constexpr float kNegInfA = -__builtin_huge_valf();

typedef __attribute__((address_space(3))) bf16x4 lds_bf16x4;

__device__ __forceinline__ f32x16 mfma32(const bf16x8& a, const bf16x8& b, const f32x16& c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ bf16x4 lds_tr16(const uint16_t* p) {
    return __builtin_amdgcn_ds_read_tr16_b64_v4bf16(
        (lds_bf16x4*)(__attribute__((address_space(3))) void*)(p));
}

__device__ __forceinline__ bf16x8 cat8(const bf16x4& lo, const bf16x4& hi) {
    return __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
}

__device__ __forceinline__ bf16x8 as_bf16x8(const uint4& v) {
    return __builtin_bit_cast(bf16x8, v);
}

// 8 fp32 accumulator values -> bf16x8 operand
__device__ __forceinline__ bf16x8 pack_op(const f32x16& c, int base) {
    uint4 u;
    u.x = pack_bf16x2(c[base + 0], c[base + 1]);
    u.y = pack_bf16x2(c[base + 2], c[base + 3]);
    u.z = pack_bf16x2(c[base + 4], c[base + 5]);
    u.w = pack_bf16x2(c[base + 6], c[base + 7]);
    return as_bf16x8(u);
}

// A operand whose K dimension runs down the rows of a row-major LDS tile with row
// stride `ld` (elements): rows k0.. (8 K-values at the permuted positions), columns
// m0 + 0..31 (lane l -> column m0 + l%32).  k0 is the 16-row chunk base.
__device__ __forceinline__ bf16x8 lds_op_t(const uint16_t* tile, int ld, int k0, int m0, int lane) {
    const int grp = lane >> 4, s = lane & 15;
    const int row = k0 + 4 * (grp >> 1) + (s >> 2);
    const int col = m0 + 16 * (grp & 1) + 4 * (s & 3);
    const uint16_t* p = tile + row * ld + col;
    return cat8(lds_tr16(p), lds_tr16(p + 8 * ld));
}

// Operand whose K dimension runs along a row: lane l reads 8 contiguous elements of
// row r0 + l%32 starting at column c0 + 8*(l/32).
__device__ __forceinline__ bf16x8 lds_op_row(const uint16_t* tile, int ld, int r0, int c0, int lane) {
    return *reinterpret_cast<const bf16x8*>(tile + (r0 + (lane & 31)) * ld + c0 + 8 * (lane >> 5));
}

// row index (within a 32-row accumulator tile) of accumulator element i of lane l
__device__ __forceinline__ int acc_row(int i, int lane) { return 8 * (i >> 2) + 4 * (lane >> 5) + (i & 3); }

// Stage rows [r0, r0+R) of a (rows, D) bf16 matrix with row stride `rs` into an LDS
// tile of row stride D+8; rows >= nrows are zero.
template <int D, int R>
__device__ __forceinline__ void stage_tile(uint16_t* tile, const uint16_t* src, int64_t rs, int r0, int nrows) {
    constexpr int VPR = D / 8;  // 16-byte vectors per row
    constexpr int LD = D + 8;
#pragma unroll
    for (int it = 0; it < (R * VPR + kAttThreads - 1) / kAttThreads; ++it) {
        const int idx = it * kAttThreads + threadIdx.x;
        if (idx < R * VPR) {
            const int r = idx / VPR, cv = idx % VPR;
            uint4 v = make_uint4(0u, 0u, 0u, 0u);
            if (r0 + r < nrows) v = ld16(src + (int64_t)(r0 + r) * rs + cv * 8);
            *reinterpret_cast<uint4*>(tile + r * LD + cv * 8) = v;
        }
    }
}

// 1-D grid over (bh, tile): consecutive tiles of one (b, h) land on one XCD
// (workgroups are dealt round-robin to the 8 XCDs), so they share its L2.
__device__ __forceinline__ void grid_map(int ntiles, int nbh, int& bh, int& tile) {
    const int G = ntiles * nbh;
    int x = blockIdx.x;
    if ((G & 7) == 0) x = (x & 7) * (G >> 3) + (x >> 3);
    bh = x / ntiles;
    tile = x - bh * ntiles;
}

// ---------------------------------------------------------------------------
// forward

template <int D>
__global__ void __launch_bounds__(kAttThreads) attn_fwd_kernel(fxAttnArgs a) {
    constexpr int LD = D + 8;
    constexpr int DC = D / 16;  // K chunks of Q.K
    constexpr int DT = D / 32;  // 32-row tiles of O^T
    __shared__ __attribute__((aligned(16))) uint16_t sk[kBN * LD];
    __shared__ __attribute__((aligned(16))) uint16_t sv[kBN * LD];

    const int T = a.T;
    const int nqt = (T + kBM - 1) / kBM;
    int bh, qt;
    grid_map(nqt, a.B * a.H, bh, qt);
    qt = nqt - 1 - qt;  // longest causal tiles first
    const int b = bh / a.H, h = bh - b * a.H;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int g = lane >> 5, ln = lane & 31;
    const int q0 = qt * kBM;
    const int q0w = q0 + 32 * wave;
    const int qi = q0w + ln;

    const uint16_t* kbase = a.k + b * a.ksb + h * a.ksh;
    const uint16_t* vbase = a.v + b * a.vsb + h * a.vsh;

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

    const int kend = a.causal ? min(T, q0 + kBM) : T;
    for (int kb = 0; kb < kend; kb += kBN) {
        __syncthreads();
        stage_tile<D, kBN>(sk, kbase, a.kst, kb, T);
        stage_tile<D, kBN>(sv, vbase, a.vst, kb, T);
        __syncthreads();
        if (a.causal && kb > q0w + 31) continue;  // every key of the tile is masked for this wave

        f32x16 s[2];
#pragma unroll
        for (int t = 0; t < 2; ++t) {
            s[t] = f32x16{};
#pragma unroll
            for (int c = 0; c < DC; ++c)
                s[t] = mfma32(lds_op_row(sk, LD, 32 * t, 16 * c, lane), qop[c], s[t]);
        }
        const bool need_mask = (kb + kBN > T) || (a.causal && kb + kBN - 1 > q0w);
        float mloc = kNegInfA;
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                float v = s[t][i] * sl2;
                if (need_mask) {
                    const int key = kb + 32 * t + acc_row(i, lane);
                    if (key >= T || (a.causal && key > qi)) v = kNegInfA;
                }
                s[t][i] = v;
                mloc = fmaxf(mloc, v);
            }
        mloc = fmaxf(mloc, __shfl_xor(mloc, 32, 64));
        const float m_new = fmaxf(m_run, mloc);
        const float m_use = (m_new == kNegInfA) ? 0.f : m_new;
        const float alpha = exp2_fast(m_run - m_use);
        float rs = 0.f;
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                const float p = exp2_fast(s[t][i] - m_use);
                s[t][i] = p;
                rs += p;
            }
        l_run = l_run * alpha + rs;
        m_run = m_new;
#pragma unroll
        for (int dt = 0; dt < DT; ++dt)
#pragma unroll
            for (int i = 0; i < 16; ++i) acc[dt][i] *= alpha;

        bf16x8 pop[4];
#pragma unroll
        for (int kc = 0; kc < 4; ++kc) pop[kc] = pack_op(s[kc >> 1], 8 * (kc & 1));
#pragma unroll
        for (int dt = 0; dt < DT; ++dt)
#pragma unroll
            for (int kc = 0; kc < 4; ++kc)
                acc[dt] = mfma32(lds_op_t(sv, LD, 16 * kc, 32 * dt, lane), pop[kc], acc[dt]);
    }

    const float l_tot = l_run + __shfl_xor(l_run, 32, 64);
    if (qi < T) {
        const float inv = l_tot > 0.f ? 1.f / l_tot : 0.f;
        uint16_t* orow = a.o_out + (((int64_t)b * T + qi) * a.H + h) * D;
#pragma unroll
        for (int dt = 0; dt < DT; ++dt)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int d = 32 * dt + 8 * r + 4 * g;
                uint2 u;
                u.x = pack_bf16x2(acc[dt][4 * r + 0] * inv, acc[dt][4 * r + 1] * inv);
                u.y = pack_bf16x2(acc[dt][4 * r + 2] * inv, acc[dt][4 * r + 3] * inv);
                *reinterpret_cast<uint2*>(orow + d) = u;
            }
        if (g == 0)
            a.lse_out[(int64_t)bh * T + qi] = l_tot > 0.f ? (m_run + log2_fast(l_tot)) * kLn2 : kNegInfA;
    }
}

// ---------------------------------------------------------------------------
// backward, query side: Delta and dQ

template <int D>
__global__ void __launch_bounds__(kAttThreads) attn_bwd_dq_kernel(fxAttnArgs a) {
    constexpr int LD = D + 8;
    constexpr int DC = D / 16;
    constexpr int DT = D / 32;
    __shared__ __attribute__((aligned(16))) uint16_t sk[kBN * LD];
    __shared__ __attribute__((aligned(16))) uint16_t sv[kBN * LD];

    const int T = a.T;
    const int nqt = (T + kBM - 1) / kBM;
    int bh, qt;
    grid_map(nqt, a.B * a.H, bh, qt);
    qt = nqt - 1 - qt;
    const int b = bh / a.H, h = bh - b * a.H;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int g = lane >> 5, ln = lane & 31;
    const int q0 = qt * kBM;
    const int q0w = q0 + 32 * wave;
    const int qi = q0w + ln;
    const bool qok = qi < T;

    // Q^T and dO^T operands, Delta = rowsum(dO * O) for this lane's query
    bf16x8 qop[DC], dop[DC];
    float delta = 0.f;
    {
        const uint16_t* qrow = a.q + b * a.qsb + h * a.qsh + (int64_t)(qok ? qi : 0) * a.qst;
        const int64_t orow = (((int64_t)b * T + (qok ? qi : 0)) * a.H + h) * D;
#pragma unroll
        for (int c = 0; c < DC; ++c) {
            uint4 qv = make_uint4(0u, 0u, 0u, 0u), dv = qv, ov = qv;
            if (qok) {
                qv = ld16(qrow + 16 * c + 8 * g);
                dv = ld16(a.dout + orow + 16 * c + 8 * g);
                ov = ld16(a.o + orow + 16 * c + 8 * g);
            }
            qop[c] = as_bf16x8(qv);
            dop[c] = as_bf16x8(dv);
            float fd[8], fo[8];
            unpack8(dv, fd);
            unpack8(ov, fo);
#pragma unroll
            for (int j = 0; j < 8; ++j) delta += fd[j] * fo[j];
        }
        delta += __shfl_xor(delta, 32, 64);
        if (qok && g == 0) a.delta[(int64_t)bh * T + qi] = delta;
    }
    const float lse2 = qok ? a.lse[(int64_t)bh * T + qi] * kLog2e : 0.f;
    const float sl2 = a.scale * kLog2e;
    const uint16_t* kbase = a.k + b * a.ksb + h * a.ksh;
    const uint16_t* vbase = a.v + b * a.vsb + h * a.vsh;

    f32x16 acc[DT];
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) acc[dt] = f32x16{};

    const int kend = a.causal ? min(T, q0 + kBM) : T;
    for (int kb = 0; kb < kend; kb += kBN) {
        __syncthreads();
        stage_tile<D, kBN>(sk, kbase, a.kst, kb, T);
        stage_tile<D, kBN>(sv, vbase, a.vst, kb, T);
        __syncthreads();
        if (a.causal && kb > q0w + 31) continue;

        f32x16 s[2], dp[2];
#pragma unroll
        for (int t = 0; t < 2; ++t) {
            s[t] = f32x16{};
            dp[t] = f32x16{};
#pragma unroll
            for (int c = 0; c < DC; ++c) {
                s[t] = mfma32(lds_op_row(sk, LD, 32 * t, 16 * c, lane), qop[c], s[t]);
                dp[t] = mfma32(lds_op_row(sv, LD, 32 * t, 16 * c, lane), dop[c], dp[t]);
            }
        }
        const bool need_mask = (kb + kBN > T) || (a.causal && kb + kBN - 1 > q0w);
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                float p = exp2_fast(s[t][i] * sl2 - lse2);
                if (need_mask) {
                    const int key = kb + 32 * t + acc_row(i, lane);
                    if (key >= T || (a.causal && key > qi)) p = 0.f;
                }
                s[t][i] = p * (dp[t][i] - delta) * a.scale;  // dS^T
            }
        bf16x8 dsop[4];
#pragma unroll
        for (int kc = 0; kc < 4; ++kc) dsop[kc] = pack_op(s[kc >> 1], 8 * (kc & 1));
#pragma unroll
        for (int dt = 0; dt < DT; ++dt)
#pragma unroll
            for (int kc = 0; kc < 4; ++kc)
                acc[dt] = mfma32(lds_op_t(sk, LD, 16 * kc, 32 * dt, lane), dsop[kc], acc[dt]);
    }

    if (qok) {
        uint16_t* dqrow = a.dq + b * a.dqb + h * a.dqh + (int64_t)qi * a.dqt;
#pragma unroll
        for (int dt = 0; dt < DT; ++dt)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int d = 32 * dt + 8 * r + 4 * g;
                uint2 u;
                u.x = pack_bf16x2(acc[dt][4 * r + 0], acc[dt][4 * r + 1]);
                u.y = pack_bf16x2(acc[dt][4 * r + 2], acc[dt][4 * r + 3]);
                *reinterpret_cast<uint2*>(dqrow + d) = u;
            }
    }
}

// ---------------------------------------------------------------------------
// backward, key side: dK and dV

template <int D>
__global__ void __launch_bounds__(kAttThreads) attn_bwd_dkv_kernel(fxAttnArgs a) {
    constexpr int LD = D + 8;
    constexpr int DC = D / 16;
    constexpr int DT = D / 32;
    __shared__ __attribute__((aligned(16))) uint16_t sq[kBQ * LD];
    __shared__ __attribute__((aligned(16))) uint16_t sdo[kBQ * LD];
    __shared__ __attribute__((aligned(16))) float slse[kBQ];
    __shared__ __attribute__((aligned(16))) float sdelta[kBQ];

    const int T = a.T;
    const int nkt = (T + kBK - 1) / kBK;
    int bh, kt;
    grid_map(nkt, a.B * a.H, bh, kt);  // key tile 0 (most causal work) first
    const int b = bh / a.H, h = bh - b * a.H;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int g = lane >> 5, ln = lane & 31;
    const int k0 = kt * kBK;
    const int k0w = k0 + 32 * wave;
    const int ki = k0w + ln;
    const bool kok = ki < T;

    bf16x8 kop[DC], vop[DC];
    {
        const uint16_t* krow = a.k + b * a.ksb + h * a.ksh + (int64_t)(kok ? ki : 0) * a.kst;
        const uint16_t* vrow = a.v + b * a.vsb + h * a.vsh + (int64_t)(kok ? ki : 0) * a.vst;
#pragma unroll
        for (int c = 0; c < DC; ++c) {
            uint4 kv = make_uint4(0u, 0u, 0u, 0u), vv = kv;
            if (kok) {
                kv = ld16(krow + 16 * c + 8 * g);
                vv = ld16(vrow + 16 * c + 8 * g);
            }
            kop[c] = as_bf16x8(kv);
            vop[c] = as_bf16x8(vv);
        }
    }
    const float sl2 = a.scale * kLog2e;
    const uint16_t* qbase = a.q + b * a.qsb + h * a.qsh;
    const uint16_t* dobase = a.dout + (int64_t)b * T * a.H * D + (int64_t)h * D;
    const int64_t dors = (int64_t)a.H * D;

    f32x16 adv[DT], adk[DT];
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) {
        adv[dt] = f32x16{};
        adk[dt] = f32x16{};
    }

    const int qstart = a.causal ? k0 : 0;  // k0 is a multiple of kBQ
    for (int qb = qstart; qb < T; qb += kBQ) {
        __syncthreads();
        stage_tile<D, kBQ>(sq, qbase, a.qst, qb, T);
        stage_tile<D, kBQ>(sdo, dobase, dors, qb, T);
        if (threadIdx.x < kBQ) {
            const int q = qb + threadIdx.x;
            slse[threadIdx.x] = q < T ? a.lse[(int64_t)bh * T + q] * kLog2e : 0.f;
            sdelta[threadIdx.x] = q < T ? a.delta[(int64_t)bh * T + q] : 0.f;
        }
        __syncthreads();
        if (a.causal && qb + kBQ - 1 < k0w) continue;  // all of this wave's keys are after these queries

        f32x16 s[2], dp[2];
#pragma unroll
        for (int t = 0; t < 2; ++t) {
            s[t] = f32x16{};
            dp[t] = f32x16{};
#pragma unroll
            for (int c = 0; c < DC; ++c) {
                s[t] = mfma32(lds_op_row(sq, LD, 32 * t, 16 * c, lane), kop[c], s[t]);
                dp[t] = mfma32(lds_op_row(sdo, LD, 32 * t, 16 * c, lane), vop[c], dp[t]);
            }
        }
        const bool need_mask = (qb + kBQ > T) || (a.causal && qb < k0w + 31);
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int qr = 32 * t + 8 * r + 4 * g;  // 4 consecutive queries of this lane
                const float4 l4 = *reinterpret_cast<const float4*>(slse + qr);
                const float4 d4 = *reinterpret_cast<const float4*>(sdelta + qr);
                const float lv[4] = {l4.x, l4.y, l4.z, l4.w};
                const float dv[4] = {d4.x, d4.y, d4.z, d4.w};
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const int i = 4 * r + e;
                    float p = exp2_fast(s[t][i] * sl2 - lv[e]);
                    if (need_mask) {
                        const int q = qb + qr + e;
                        if (q >= T || (a.causal && ki > q)) p = 0.f;
                    }
                    s[t][i] = p;                                      // P
                    dp[t][i] = p * (dp[t][i] - dv[e]) * a.scale;      // dS
                }
            }
        bf16x8 pop[4], dsop[4];
#pragma unroll
        for (int kc = 0; kc < 4; ++kc) {
            pop[kc] = pack_op(s[kc >> 1], 8 * (kc & 1));
            dsop[kc] = pack_op(dp[kc >> 1], 8 * (kc & 1));
        }
#pragma unroll
        for (int dt = 0; dt < DT; ++dt)
#pragma unroll
            for (int kc = 0; kc < 4; ++kc) {
                adv[dt] = mfma32(lds_op_t(sdo, LD, 16 * kc, 32 * dt, lane), pop[kc], adv[dt]);
                adk[dt] = mfma32(lds_op_t(sq, LD, 16 * kc, 32 * dt, lane), dsop[kc], adk[dt]);
            }
    }

    if (kok) {
        uint16_t* dkrow = a.dk + b * a.dkb + h * a.dkh + (int64_t)ki * a.dkt;
        uint16_t* dvrow = a.dv + b * a.dvb + h * a.dvh + (int64_t)ki * a.dvt;
#pragma unroll
        for (int dt = 0; dt < DT; ++dt)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int d = 32 * dt + 8 * r + 4 * g;
                uint2 u;
                u.x = pack_bf16x2(adk[dt][4 * r + 0], adk[dt][4 * r + 1]);
                u.y = pack_bf16x2(adk[dt][4 * r + 2], adk[dt][4 * r + 3]);
                *reinterpret_cast<uint2*>(dkrow + d) = u;
                u.x = pack_bf16x2(adv[dt][4 * r + 0], adv[dt][4 * r + 1]);
                u.y = pack_bf16x2(adv[dt][4 * r + 2], adv[dt][4 * r + 3]);
                *reinterpret_cast<uint2*>(dvrow + d) = u;
            }
    }
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
    const int64_t s[] = {a.qsb, a.qst, a.qsh, a.ksb, a.kst, a.ksh, a.vsb, a.vst, a.vsh};
    for (int64_t x : s) FX_REQUIRE(x % 8 == 0, "fx_attn: q/k/v strides must be multiples of 8 elements");
    FX_REQUIRE((((uintptr_t)a.q | (uintptr_t)a.k | (uintptr_t)a.v) & 15) == 0,
               "fx_attn: q/k/v must be 16-byte aligned");
    if (!bwd) {
        FX_REQUIRE(a.o_out && a.lse_out, "fx_attn_fwd: null output");
        FX_REQUIRE(((uintptr_t)a.o_out & 15) == 0, "fx_attn_fwd: o must be 16-byte aligned");
    } else {
        FX_REQUIRE(a.o && a.dout && a.lse && a.delta && a.dq && a.dk && a.dv, "fx_attn_bwd: null pointer");
        FX_REQUIRE((((uintptr_t)a.o | (uintptr_t)a.dout) & 15) == 0, "fx_attn_bwd: o/dout must be 16-byte aligned");
        FX_REQUIRE((((uintptr_t)a.dq | (uintptr_t)a.dk | (uintptr_t)a.dv) & 7) == 0,
                   "fx_attn_bwd: dq/dk/dv must be 8-byte aligned");
        const int64_t t[] = {a.dqb, a.dqt, a.dqh, a.dkb, a.dkt, a.dkh, a.dvb, a.dvt, a.dvh};
        for (int64_t x : t) FX_REQUIRE(x % 4 == 0, "fx_attn_bwd: dq/dk/dv strides must be multiples of 4");
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
