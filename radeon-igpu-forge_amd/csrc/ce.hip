// Fused softmax cross-entropy for gfx950.
//
// One workgroup per row.  The row is read from HBM exactly once into registers
// (NV 16-byte vectors per lane, coalesced), the max and the sum of exponentials are
// block reductions over those registers, and the gradient row is written once:
// 1 read + 1 write of the logits per row, against 2 reads + 1 write when the row
// does not fit a cache (ml/fxlm/kernels/ce.hip:45-50, :99-108).
//
// Semantics (ml/fxlm/kernels/ce.hip:32-116): valid = t != ignore && 0 <= t < V;
// loss_r = m + log Z - x_t for valid rows; grad = (softmax - onehot(t)) * mul for
// valid rows and 0 for the others.
#include <math.h>

#include "fx_device.h"

namespace fx {

constexpr float kNegInf = -__builtin_huge_valf();

// (max, sum of exp(x - max)) pairs: merge b into a
__device__ __forceinline__ void ms_merge(float& m, float& s, float m2, float s2) {
    const float mn = fmaxf(m, m2);
    // a side whose max equals the new max keeps its sum; -inf sides carry s == 0
    const float ea = (m == mn) ? 1.f : exp2_fast((m - mn) * kLog2e);
    const float eb = (m2 == mn) ? 1.f : exp2_fast((m2 - mn) * kLog2e);
    s = s * ea + s2 * eb;
    m = mn;
}

// Register-resident row: needs V % 8 == 0, ld % 8 == 0, ldg % 8 == 0 and 16-byte
// aligned bases (checked by the host); V <= 8 * NT * NV.
// Each thread reduces its own vectors to (max, sum exp(x - max)) without any
// barrier; one block-wide merge of those pairs gives (M, Z); the gradient pass
// then rereads the registers.  The target's gradient element is fixed up by the one
// thread that holds it.
template <int NT, int NV>
__global__ void __launch_bounds__(NT) ce_row_kernel(fxCEArgs a) {
    constexpr int NW = NT / 64;
    __shared__ float shm[NW], shs[NW];
    const int64_t row = blockIdx.x;
    const uint16_t* lr = a.logits + row * a.ld;
    const int64_t t = a.target[row];
    const bool valid = (t != a.ignore_index) && (t >= 0) && (t < a.V);
    const int V8 = (int)(a.V >> 3);
    const int tid = threadIdx.x;
    // x_t is read before the barrier: with grad == logits (in place) other threads
    // overwrite the row once the reduction is done.
    const float xt = (tid == 0 && valid) ? bf16_to_f32(lr[t]) : 0.f;
    uint16_t* gr = a.grad != nullptr ? a.grad + row * a.ldg : nullptr;
    if (!valid) {  // no loss and a zero gradient row: the logits are not read
        if (tid == 0) a.row_loss[row] = 0.f;
        if (gr != nullptr) {
#pragma unroll
            for (int i = 0; i < NV; ++i) {
                const int c = i * NT + tid;
                if (c < V8) st16_nt(gr + (int64_t)c * 8, make_uint4(0u, 0u, 0u, 0u));
            }
        }
        return;
    }

    uint4 xv[NV];
#pragma unroll
    for (int i = 0; i < NV; ++i) {
        const int c = i * NT + tid;
        xv[i] = make_uint4(0u, 0u, 0u, 0u);
        if (c < V8) xv[i] = ld16_nt(lr + (int64_t)c * 8);
    }
    float m = kNegInf;
#pragma unroll
    for (int i = 0; i < NV; ++i) {
        if (i * NT + tid < V8) {
            float f[8];
            unpack8(xv[i], f);
#pragma unroll
            for (int j = 0; j < 8; ++j) m = fmaxf(m, f[j]);
        }
    }
    float s = 0.f;
    {
        const float ml = (m == kNegInf) ? 0.f : m * kLog2e;
#pragma unroll
        for (int i = 0; i < NV; ++i) {
            if (i * NT + tid < V8) {
                float f[8];
                unpack8(xv[i], f);
#pragma unroll
                for (int j = 0; j < 8; ++j) s += exp2_fast(fmaf(f[j], kLog2e, -ml));
            }
        }
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) ms_merge(m, s, __shfl_xor(m, off, 64), __shfl_xor(s, off, 64));
    if (NW > 1) {
        if ((tid & 63) == 0) {
            shm[tid >> 6] = m;
            shs[tid >> 6] = s;
        }
        __syncthreads();
        m = shm[0];
        s = shs[0];
#pragma unroll
        for (int w = 1; w < NW; ++w) ms_merge(m, s, shm[w], shs[w]);
    }

    if (tid == 0) a.row_loss[row] = m + logf(s) - xt;
    if (gr == nullptr) return;

    const float gmul = *a.mul;
    const float scale = gmul / s;  // softmax * mul = exp(x - M) * (mul / Z)
    const float ml = m * kLog2e;
    const int tc = (int)(t >> 3);
#pragma unroll
    for (int i = 0; i < NV; ++i) {
        const int c = i * NT + tid;
        if (c < V8) {
            float f[8];
            unpack8(xv[i], f);
#pragma unroll
            for (int j = 0; j < 8; ++j) f[j] = exp2_fast(fmaf(f[j], kLog2e, -ml)) * scale;
            if (c == tc) {
                const int tj = (int)(t & 7);
#pragma unroll
                for (int j = 0; j < 8; ++j)
                    if (j == tj) f[j] -= gmul;
            }
            st16_nt(gr + (int64_t)c * 8, pack8(f));
        }
    }
}

// Any V / stride / alignment: two passes over the row from global memory with an
// online (max, sum) per thread merged across the block.
__global__ void __launch_bounds__(256) ce_row_generic_kernel(fxCEArgs a) {
    __shared__ float shm[4], shl[4];
    const int64_t row = blockIdx.x;
    const uint16_t* lr = a.logits + row * a.ld;
    const int64_t t = a.target[row];
    const bool valid = (t != a.ignore_index) && (t >= 0) && (t < a.V);
    const float xt = (threadIdx.x == 0 && valid) ? bf16_to_f32(lr[t]) : 0.f;
    float m = kNegInf, l = 0.f;
    for (int64_t d = threadIdx.x; d < a.V; d += 256) {
        const float f = bf16_to_f32(lr[d]);
        if (f > m) {
            l = l * exp2_fast((m - f) * kLog2e) + 1.f;
            m = f;
        } else {
            l += exp2_fast((f - m) * kLog2e);
        }
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
        const float m2 = __shfl_xor(m, off, 64), l2 = __shfl_xor(l, off, 64);
        const float mn = fmaxf(m, m2);
        const float ea = (m > kNegInf) ? exp2_fast((m - mn) * kLog2e) : 0.f;
        const float eb = (m2 > kNegInf) ? exp2_fast((m2 - mn) * kLog2e) : 0.f;
        l = l * ea + l2 * eb;
        m = mn;
    }
    if ((threadIdx.x & 63) == 0) {
        shm[threadIdx.x >> 6] = m;
        shl[threadIdx.x >> 6] = l;
    }
    __syncthreads();
    float M = shm[0];
    for (int i = 1; i < 4; ++i) M = fmaxf(M, shm[i]);
    float Z = 0.f;
    for (int i = 0; i < 4; ++i) Z += (shm[i] > kNegInf) ? shl[i] * exp2_fast((shm[i] - M) * kLog2e) : 0.f;
    if (threadIdx.x == 0) a.row_loss[row] = valid ? M + logf(Z) - xt : 0.f;
    if (a.grad == nullptr) return;
    const float gmul = valid ? *a.mul : 0.f;
    const float scale = gmul / Z;
    uint16_t* gr = a.grad + row * a.ldg;
    for (int64_t d = threadIdx.x; d < a.V; d += 256) {
        float p = exp2_fast((bf16_to_f32(lr[d]) - M) * kLog2e) * scale;
        if (d == t) p -= gmul;
        gr[d] = f32_to_bf16(valid ? p : 0.f);
    }
}

__global__ void __launch_bounds__(1024)
ce_inv_nvalid_kernel(const int64_t* __restrict__ target, int64_t N, int64_t ignore,
                     const float* __restrict__ gs, float gsv, float* __restrict__ inv_n,
                     float* __restrict__ mul) {
    __shared__ int sh[16];
    int cnt = 0;
#pragma unroll 8
    for (int64_t i = threadIdx.x; i < N; i += 1024) cnt += (target[i] != ignore) ? 1 : 0;
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) cnt += __shfl_xor(cnt, off, 64);
    if ((threadIdx.x & 63) == 0) sh[threadIdx.x >> 6] = cnt;
    __syncthreads();
    if (threadIdx.x == 0) {
        long long tot = 0;
        for (int i = 0; i < 16; ++i) tot += sh[i];
        const float nv = (float)tot;
        const float inv = nv > 0.f ? 1.f / nv : 0.f;
        *inv_n = inv;
        if (mul) *mul = inv * (gs ? *gs : gsv);
    }
}

__global__ void __launch_bounds__(1024)
ce_loss_finalize_kernel(const float* __restrict__ row_loss, int64_t N,
                        const float* __restrict__ inv_n, float* __restrict__ loss) {
    __shared__ float sh[16];
    float s = 0.f;
#pragma unroll 8
    for (int64_t i = threadIdx.x; i < N; i += 1024) s += row_loss[i];
    s = group_sum<64>(s);
    if ((threadIdx.x & 63) == 0) sh[threadIdx.x >> 6] = s;
    __syncthreads();
    if (threadIdx.x == 0) {
        float tot = 0.f;
        for (int i = 0; i < 16; ++i) tot += sh[i];
        *loss = tot * (*inv_n);
    }
}

__global__ void __launch_bounds__(256)
ce_scale_grad_kernel(uint16_t* __restrict__ grad, int64_t numel, const float* __restrict__ g,
                     float* __restrict__ applied, int src) {
    const float gv = *g;
    const float f = gv / (src < 0 ? 1.f : applied[src]);
    if (blockIdx.x == 0 && threadIdx.x == 0) applied[src == 1 ? 0 : 1] = gv;  // no block reads this slot
    if (f == 1.f) return;
    const int64_t stride = (int64_t)gridDim.x * 256;
    const int64_t n8 = numel >> 3;
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n8; i += stride) {
        float v[8];
        unpack8(ld16(grad + i * 8), v);
#pragma unroll
        for (int j = 0; j < 8; ++j) v[j] *= f;
        st16(grad + i * 8, pack8(v));
    }
    for (int64_t i = n8 * 8 + (int64_t)blockIdx.x * 256 + threadIdx.x; i < numel; i += stride)
        grad[i] = f32_to_bf16(bf16_to_f32(grad[i]) * f);
}

// Linear-CE backward scaling: s = (*g) * (gs ? 1 / *gs : inv_value) (the reciprocal and
// the product rounded as the separate fp32 operations round them), then
// dw_out = bf16(dw * s) over nw fp32 elements and dx_out = bf16(dx * bf16(s)) over nx bf16
// elements, 8 per thread and step with an element-wise tail.
// WT: the weight gradient's element type, float or bf16 (uint16_t, exact in fp32)
template <typename WT>
__global__ void __launch_bounds__(256)
ce_lin_grad_scale_kernel(const WT* __restrict__ dw, int64_t nw, const uint16_t* __restrict__ dx, int64_t nx,
                         const float* __restrict__ g, const float* __restrict__ gs, float inv_value,
                         uint16_t* __restrict__ dw_out, uint16_t* __restrict__ dx_out) {
    const float inv = gs != nullptr ? 1.f / *gs : inv_value;
    const float sc = *g * inv;
    // dx's product takes the factor as bf16: a bf16 tensor times a 0-dim fp32 tensor has
    // bf16 as its common dtype, so the factor is rounded to bf16 first
    const float sx = bf16_to_f32(f32_to_bf16(sc));
    const int64_t stride = (int64_t)gridDim.x * 256;
    const int64_t t0 = (int64_t)blockIdx.x * 256 + threadIdx.x;
    for (int64_t v = t0; v < nw / 8; v += stride) {
        float f[8];
        if constexpr (sizeof(WT) == 4) {
            const float4* p = reinterpret_cast<const float4*>(dw + v * 8);
            const float4 lo = p[0], hi = p[1];
            f[0] = lo.x; f[1] = lo.y; f[2] = lo.z; f[3] = lo.w;
            f[4] = hi.x; f[5] = hi.y; f[6] = hi.z; f[7] = hi.w;
        } else {
            unpack8(ld16(dw + v * 8), f);
        }
#pragma unroll
        for (int j = 0; j < 8; ++j) f[j] *= sc;
        st16(dw_out + v * 8, pack8(f));
    }
    for (int64_t v = t0; v < nx / 8; v += stride) {
        float f[8];
        unpack8(ld16(dx + v * 8), f);
#pragma unroll
        for (int j = 0; j < 8; ++j) f[j] *= sx;
        st16(dx_out + v * 8, pack8(f));
    }
    if (t0 == 0) {
        for (int64_t i = nw / 8 * 8; i < nw; ++i) {
            float w;
            if constexpr (sizeof(WT) == 4) w = dw[i]; else w = bf16_to_f32(dw[i]);
            dw_out[i] = f32_to_bf16(w * sc);
        }
        for (int64_t i = nx / 8 * 8; i < nx; ++i) dx_out[i] = f32_to_bf16(bf16_to_f32(dx[i]) * sx);
    }
}

// ce_lin_grad_scale_kernel for a bf16 dw, in place: dw = bf16(dw * s), dx = bf16(dx * bf16(s)),
// the same roundings.  s == 1 changes no value (x * 1 is exact), so then the whole grid
// returns without touching memory.
__global__ void __launch_bounds__(256)
ce_lin_grad_scale_inplace_kernel(uint16_t* dw, int64_t nw, uint16_t* dx, int64_t nx, const float* __restrict__ g,
                                 const float* __restrict__ gs, float inv_value) {
    const float inv = gs != nullptr ? 1.f / *gs : inv_value;
    const float sc = *g * inv;
    if (sc == 1.f) return;
    const float sx = bf16_to_f32(f32_to_bf16(sc));
    const int64_t stride = (int64_t)gridDim.x * 256;
    const int64_t t0 = (int64_t)blockIdx.x * 256 + threadIdx.x;
    for (int64_t v = t0; v < nw / 8; v += stride) {
        float f[8];
        unpack8(ld16(dw + v * 8), f);
#pragma unroll
        for (int j = 0; j < 8; ++j) f[j] *= sc;
        st16(dw + v * 8, pack8(f));
    }
    for (int64_t v = t0; v < nx / 8; v += stride) {
        float f[8];
        unpack8(ld16(dx + v * 8), f);
#pragma unroll
        for (int j = 0; j < 8; ++j) f[j] *= sx;
        st16(dx + v * 8, pack8(f));
    }
    if (t0 == 0) {
        for (int64_t i = nw / 8 * 8; i < nw; ++i) dw[i] = f32_to_bf16(bf16_to_f32(dw[i]) * sc);
        for (int64_t i = nx / 8 * 8; i < nx; ++i) dx[i] = f32_to_bf16(bf16_to_f32(dx[i]) * sx);
    }
}

}  // namespace fx

using namespace fx;

#define FX_CE_NV_CASES(NT, CALL)                                                            \
    case 1: CALL(NT, 1); break;   case 2: CALL(NT, 2); break;   case 3: CALL(NT, 3); break;   \
    case 4: CALL(NT, 4); break;   case 5: CALL(NT, 5); break;   case 6: CALL(NT, 6); break;   \
    case 7: CALL(NT, 7); break;   case 8: CALL(NT, 8); break;   case 9: CALL(NT, 9); break;   \
    case 10: CALL(NT, 10); break; case 11: CALL(NT, 11); break; case 12: CALL(NT, 12); break; \
    case 13: CALL(NT, 13); break; case 14: CALL(NT, 14); break; case 15: CALL(NT, 15); break; \
    case 16: CALL(NT, 16); break;
#define FX_CE_NV_CASES10(NT, CALL)                                                          \
    case 1: CALL(NT, 1); break;   case 2: CALL(NT, 2); break;   case 3: CALL(NT, 3); break;   \
    case 4: CALL(NT, 4); break;   case 5: CALL(NT, 5); break;   case 6: CALL(NT, 6); break;   \
    case 7: CALL(NT, 7); break;   case 8: CALL(NT, 8); break;   case 9: CALL(NT, 9); break;   \
    case 10: CALL(NT, 10); break;

extern "C" int fx_ce_inv_nvalid(const int64_t* target, int64_t N, int64_t ignore_index,
                                const float* grad_scale, float grad_scale_value, float* inv_n,
                                float* mul, void* stream) {
    FX_REQUIRE(inv_n != nullptr, "fx_ce_inv_nvalid: null inv_n");
    FX_REQUIRE(N >= 0 && (N == 0 || target != nullptr), "fx_ce_inv_nvalid: bad target");
    hipLaunchKernelGGL(ce_inv_nvalid_kernel, dim3(1), dim3(1024), 0, (hipStream_t)stream, target, N,
                       ignore_index, grad_scale, grad_scale_value, inv_n, mul);
    return check_launch("ce_inv_nvalid");
}

extern "C" int fx_ce_fwd_grad(const fxCEArgs* args, void* stream) {
    FX_REQUIRE(args != nullptr, "fx_ce_fwd_grad: null args");
    const fxCEArgs& a = *args;
    FX_REQUIRE(a.N >= 0 && a.V >= 1, "fx_ce_fwd_grad: bad shape N=%lld V=%lld", (long long)a.N,
               (long long)a.V);
    FX_REQUIRE(a.N <= 0x7fffffff, "fx_ce_fwd_grad: N=%lld too large", (long long)a.N);
    FX_REQUIRE(a.ld >= a.V && (a.grad == nullptr || a.ldg >= a.V), "fx_ce_fwd_grad: bad row stride");
    FX_REQUIRE(a.N == 0 || (a.logits && a.target && a.row_loss), "fx_ce_fwd_grad: null pointer");
    FX_REQUIRE(a.grad == nullptr || a.mul != nullptr, "fx_ce_fwd_grad: grad needs mul");
    if (a.N == 0) return 0;
    const bool vec = (a.V % 8 == 0) && (a.ld % 8 == 0) && (((uintptr_t)a.logits & 15) == 0) &&
                     (a.grad == nullptr || ((a.ldg % 8 == 0) && (((uintptr_t)a.grad & 15) == 0)));
    const int64_t V8 = a.V / 8;
    // block size: the first of 64, 256, 512, 768, 1024 threads that holds the row in at
    // most 8 vectors per lane, else the first of 64, 256, 512, 1024 with at most 16.  Fewer
    // vectors per lane shorten the phase in which a row's block computes instead of
    // loading: at [16384, 50304] 1024 x 7 ran 548 us against 560 us for 768 x 9 and 576 us
    // for 512 x 13 (one process, medians), and a plain copy with the same access pattern
    // 582 us.
    int nt = 0, nv = 0;
    if (vec) {
        static const int nts8[] = {64, 256, 512, 768, 1024};
        static const int nts16[] = {64, 256, 512, 1024};
        for (int cand : nts8) {
            const int64_t need = (V8 + cand - 1) / cand;
            if (need <= 8) {
                nt = cand;
                nv = (int)need;
                break;
            }
        }
        for (int k = 0; nt == 0 && k < 4; ++k) {
            const int64_t need = (V8 + nts16[k] - 1) / nts16[k];
            if (need <= 16) {
                nt = nts16[k];
                nv = (int)need;
            }
        }
    }
    const dim3 grid((unsigned)a.N);
    hipStream_t s = (hipStream_t)stream;
    if (nt == 0) {
        hipLaunchKernelGGL(ce_row_generic_kernel, grid, dim3(256), 0, s, a);
        return check_launch("ce_row_generic");
    }
#define FX_CALL(NT, NV) hipLaunchKernelGGL((ce_row_kernel<NT, NV>), grid, dim3(NT), 0, s, a)
    switch (nt) {
        case 64: switch (nv) { FX_CE_NV_CASES(64, FX_CALL) } break;
        case 256: switch (nv) { FX_CE_NV_CASES(256, FX_CALL) } break;
        case 512: switch (nv) { FX_CE_NV_CASES(512, FX_CALL) } break;
        case 768: switch (nv) { FX_CE_NV_CASES10(768, FX_CALL) } break;
        case 1024: switch (nv) { FX_CE_NV_CASES(1024, FX_CALL) } break;
    }
#undef FX_CALL
    return check_launch("ce_row");
}

extern "C" int fx_ce_loss_finalize(const float* row_loss, int64_t N, const float* inv_n, float* loss,
                                   void* stream) {
    FX_REQUIRE(inv_n != nullptr && loss != nullptr, "fx_ce_loss_finalize: null pointer");
    FX_REQUIRE(N >= 0 && (N == 0 || row_loss != nullptr), "fx_ce_loss_finalize: bad row_loss");
    hipLaunchKernelGGL(ce_loss_finalize_kernel, dim3(1), dim3(1024), 0, (hipStream_t)stream, row_loss,
                       N, inv_n, loss);
    return check_launch("ce_loss_finalize");
}

extern "C" int fx_ce_scale_grad(uint16_t* grad, int64_t numel, const float* g, float* applied,
                                int32_t src, void* stream) {
    FX_REQUIRE(g != nullptr && applied != nullptr, "fx_ce_scale_grad: null scalar");
    FX_REQUIRE(src >= -1 && src <= 1, "fx_ce_scale_grad: src=%d must be -1, 0 or 1", src);
    FX_REQUIRE(numel >= 0 && (numel == 0 || grad != nullptr), "fx_ce_scale_grad: bad grad");
    FX_REQUIRE(((uintptr_t)grad & 15) == 0, "fx_ce_scale_grad: grad not 16-byte aligned");
    // one launch whatever the ratio (the kernel writes applied[1 - src]); a grid-stride
    // grid of 4 blocks per CU streams the scaling and exits cheaply when it is a no-op
    int64_t blocks = (numel / 8 + 255) / 256;
    if (blocks > 1024) blocks = 1024;
    if (blocks < 1) blocks = 1;
    hipLaunchKernelGGL(ce_scale_grad_kernel, dim3((unsigned)blocks), dim3(256), 0, (hipStream_t)stream, grad,
                       numel, g, applied, (int)src);
    return check_launch("ce_scale_grad");
}

template <typename WT>
static int lin_grad_scale(const WT* dw, int64_t nw, const uint16_t* dx, int64_t nx, const float* g, const float* gs,
                          float inv_value, uint16_t* dw_out, uint16_t* dx_out, void* stream, const char* who) {
    FX_REQUIRE(nw >= 0 && nx >= 0 && g != nullptr, "%s: bad arguments", who);
    FX_REQUIRE((nw == 0 || (dw && dw_out)) && (nx == 0 || (dx && dx_out)), "%s: null pointer", who);
    FX_REQUIRE(((((uintptr_t)dw) | ((uintptr_t)dx) | ((uintptr_t)dw_out) | ((uintptr_t)dx_out)) & 15) == 0,
               "%s: buffers must be 16-byte aligned", who);
    if (nw == 0 && nx == 0) return 0;
    const int64_t groups = (nw > nx ? nw : nx) / 8 + 1;
    int64_t blocks = (groups + 255) / 256;
    if (blocks > 8192) blocks = 8192;
    hipLaunchKernelGGL(ce_lin_grad_scale_kernel<WT>, dim3((unsigned)blocks), dim3(256), 0, (hipStream_t)stream, dw,
                       nw, dx, nx, g, gs, inv_value, dw_out, dx_out);
    return check_launch("ce_lin_grad_scale");
}

extern "C" int fx_ce_lin_grad_scale(const float* dw, int64_t nw, const uint16_t* dx, int64_t nx, const float* g,
                                    const float* gs, float inv_value, uint16_t* dw_out, uint16_t* dx_out,
                                    void* stream) {
    return lin_grad_scale(dw, nw, dx, nx, g, gs, inv_value, dw_out, dx_out, stream, "fx_ce_lin_grad_scale");
}

extern "C" int fx_ce_lin_grad_scale_bf16w(const uint16_t* dw, int64_t nw, const uint16_t* dx, int64_t nx,
                                          const float* g, const float* gs, float inv_value, uint16_t* dw_out,
                                          uint16_t* dx_out, void* stream) {
    return lin_grad_scale(dw, nw, dx, nx, g, gs, inv_value, dw_out, dx_out, stream, "fx_ce_lin_grad_scale_bf16w");
}

extern "C" int fx_ce_lin_grad_scale_inplace(uint16_t* dw, int64_t nw, uint16_t* dx, int64_t nx, const float* g,
                                            const float* gs, float inv_value, void* stream) {
    FX_REQUIRE(nw >= 0 && nx >= 0 && g != nullptr, "fx_ce_lin_grad_scale_inplace: bad arguments");
    FX_REQUIRE((nw == 0 || dw) && (nx == 0 || dx), "fx_ce_lin_grad_scale_inplace: null pointer");
    FX_REQUIRE(((((uintptr_t)dw) | ((uintptr_t)dx)) & 15) == 0,
               "fx_ce_lin_grad_scale_inplace: buffers must be 16-byte aligned");
    if (nw == 0 && nx == 0) return 0;
    const int64_t groups = (nw > nx ? nw : nx) / 8 + 1;
    int64_t blocks = (groups + 255) / 256;
    if (blocks > 8192) blocks = 8192;
    hipLaunchKernelGGL(ce_lin_grad_scale_inplace_kernel, dim3((unsigned)blocks), dim3(256), 0, (hipStream_t)stream, dw,
                       nw, dx, nx, g, gs, inv_value);
    return check_launch("ce_lin_grad_scale_inplace");
}
