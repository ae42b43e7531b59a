// Fused (gather) linear layer for gfx950: C = act(A W^T + bias) with bf16 MFMA.
//
// A rows are either dense (row m at A + m*lda) or gathered: row m is the
// window of W consecutive rows of X starting at idx[m], i.e. the contiguous
// slice X + idx[m]*F .. + K (K = W*F), which is exactly the window-major
// flattening Xg[m, w*F + f] = X[idx[m] + w, f] of ml/fxgpu/gather_gemm.hip:175-206.
// So gathering costs nothing beyond a per-row base pointer, and the gathered
// rows can be written out (Xg) by the first column of tiles for the backward.
//
// Tiling: 128 x 128 output tile per workgroup, 4 waves in 2 x 2, each wave
// 64 x 64 = 2 x 2 tiles of v_mfma_f32_32x32x16_bf16; K advances 32 per stage
// through double-buffered LDS (row stride 40 elements) with the next stage's
// global loads in flight during the MFMAs.  Epilogue: + bias, optional
// GELU-tanh, optional pre-activation output.
#include <math.h>

#include "fx_device.h"

namespace fx {

constexpr int kGBM = 128, kGBN = 128, kGBK = 32;
constexpr int kGLD = kGBK + 8;  // LDS row stride (elements)
constexpr int kGThreads = 256;

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
    int act;  // 0: identity, 1: GELU (tanh approximation)
};

__device__ __forceinline__ f32x16 mfma32g(const bf16x8& a, const bf16x8& b, const f32x16& c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ float gelu_tanh(float h) {
    // 0.5 h (1 + tanh(u)), u = sqrt(2/pi) (h + 0.044715 h^3); tanh(u) = 1 - 2 / (e^{2u} + 1)
    const float u = 0.7978845608028654f * (h + 0.044715f * h * h * h);
    const float e = exp2_fast(2.f * kLog2e * u);
    const float th = 1.f - 2.f / (e + 1.f);
    return 0.5f * h * (1.f + th);
}

__device__ __forceinline__ float gelu_tanh_grad(float h) {
    const float u = 0.7978845608028654f * (h + 0.044715f * h * h * h);
    const float e = exp2_fast(2.f * kLog2e * u);
    const float th = 1.f - 2.f / (e + 1.f);
    return 0.5f * (1.f + th) +
           0.5f * h * (1.f - th * th) * 0.7978845608028654f * (1.f + 3.f * 0.044715f * h * h);
}

// Grid: x over N tiles, y over M tiles (a row of tiles shares its A rows in L2).
__global__ void __launch_bounds__(kGThreads) gemm_bias_act_kernel(GemmArgs a) {
    __shared__ __attribute__((aligned(16))) uint16_t sa[2][kGBM * kGLD];
    __shared__ __attribute__((aligned(16))) uint16_t sb[2][kGBN * kGLD];

    const int n0 = blockIdx.x * kGBN, m0 = blockIdx.y * kGBM;
    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const int wm = (wave >> 1) * 64, wn = (wave & 1) * 64;
    const int g = lane >> 5;
    const bool write_xg = (a.Xg != nullptr) && blockIdx.x == 0;

    // each thread moves 2 x 16 B of A and 2 x 16 B of B per stage:
    // vector v = tid + 256*r (r = 0, 1) -> row v / 4, k-vector v % 4
    const uint16_t* arow[2];
    const uint16_t* brow[2];
    int vrow[2], vk[2];
#pragma unroll
    for (int r = 0; r < 2; ++r) {
        const int v = tid + kGThreads * r;
        vrow[r] = v >> 2;
        vk[r] = (v & 3) * 8;
        const int m = m0 + vrow[r];
        const int n = n0 + vrow[r];
        arow[r] = nullptr;
        if (m < a.M) {
            if (a.idx) {
                // a window that leaves X reads as zeros instead of faulting
                const int64_t s = a.idx[m];
                if (s >= 0 && s * a.F + a.K <= a.R * a.F) arow[r] = a.A + s * a.F;
            } else {
                arow[r] = a.A + (int64_t)m * a.lda;
            }
        }
        brow[r] = (n < a.N) ? a.B + (int64_t)n * a.ldb : nullptr;
    }
    const int nk = (a.K + kGBK - 1) / kGBK;
    uint4 ra[2], rb[2];
    auto gload = [&](int kt) {
#pragma unroll
        for (int r = 0; r < 2; ++r) {
            const int k = kt * kGBK + vk[r];
            ra[r] = make_uint4(0u, 0u, 0u, 0u);
            rb[r] = make_uint4(0u, 0u, 0u, 0u);
            if (arow[r] && k < a.K) ra[r] = ld16(arow[r] + k);
            if (brow[r] && k < a.K) rb[r] = ld16(brow[r] + k);
            if (write_xg && m0 + vrow[r] < a.M && k < a.K)
                st16(a.Xg + (int64_t)(m0 + vrow[r]) * a.ldxg + k, ra[r]);
        }
    };
    auto sstore = [&](int buf) {
#pragma unroll
        for (int r = 0; r < 2; ++r) {
            *reinterpret_cast<uint4*>(&sa[buf][vrow[r] * kGLD + vk[r]]) = ra[r];
            *reinterpret_cast<uint4*>(&sb[buf][vrow[r] * kGLD + vk[r]]) = rb[r];
        }
    };

    f32x16 acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) acc[i][j] = f32x16{};

    gload(0);
    sstore(0);
    __syncthreads();
    for (int kt = 0; kt < nk; ++kt) {
        const int buf = kt & 1;
        if (kt + 1 < nk) gload(kt + 1);
#pragma unroll
        for (int c = 0; c < kGBK / 16; ++c) {
            bf16x8 av[2], bv[2];
#pragma unroll
            for (int i = 0; i < 2; ++i)
                av[i] = *reinterpret_cast<const bf16x8*>(&sa[buf][(wm + 32 * i + (lane & 31)) * kGLD + 16 * c + 8 * g]);
#pragma unroll
            for (int j = 0; j < 2; ++j)
                bv[j] = *reinterpret_cast<const bf16x8*>(&sb[buf][(wn + 32 * j + (lane & 31)) * kGLD + 16 * c + 8 * g]);
#pragma unroll
            for (int i = 0; i < 2; ++i)
#pragma unroll
                for (int j = 0; j < 2; ++j) acc[i][j] = mfma32g(av[i], bv[j], acc[i][j]);
        }
        if (kt + 1 < nk) sstore(buf ^ 1);
        __syncthreads();
    }

    // epilogue: lane holds column n = n0 + wn + 32 j + lane%32, rows 8*(e/4) + 4 g + e%4
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        const int n = n0 + wn + 32 * j + (lane & 31);
        if (n >= a.N) continue;
        const float bn = a.bias ? bf16_to_f32(a.bias[n]) : 0.f;
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                const int m = m0 + wm + 32 * i + 8 * (e >> 2) + 4 * g + (e & 3);
                if (m < a.M) {
                    const float h = acc[i][j][e] + bn;
                    if (a.H) a.H[(int64_t)m * a.ldh + n] = f32_to_bf16(h);
                    a.C[(int64_t)m * a.ldc + n] = f32_to_bf16(a.act == 1 ? gelu_tanh(h) : h);
                }
            }
    }
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
    FX_REQUIRE(act == 0 || act == 1, "fx_linear_fwd: act=%d (0 identity, 1 gelu_tanh)", act);
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
    GemmArgs a;
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
    const dim3 grid((unsigned)((N + kGBN - 1) / kGBN), (unsigned)((M + kGBM - 1) / kGBM));
    FX_REQUIRE(grid.y <= 65535u * 16u, "fx_linear_fwd: M too large");
    hipLaunchKernelGGL(gemm_bias_act_kernel, grid, dim3(kGThreads), 0, (hipStream_t)stream, a);
    return check_launch("gemm_bias_act");
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
