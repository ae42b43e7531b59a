// FlatAdamW step for gfx950: three launches, no host synchronisation.
//
//   adamw_sumsq   one fp32 partial sum of g^2 per chunk of kChunk elements
//   adamw_final   one block: fixed-order fp64 sum of the partials, found_inf, grad
//                 norm, clip coefficient, step counter and the loss-scale update
//   adamw_update  the elementwise AdamW update over the flat master/m/v buffers,
//                 writing the bf16 parameter copy
//
// Work is split into equal chunks across all tensors of a list (a chunk never spans
// two tensors), so small tensors do not pay for the grid of the largest one.
// A non-finite gradient makes its chunk's partial non-finite (squares are >= 0, inf
// or nan), so the final sum alone tells whether the step must be skipped, as the
// reference's separate flag word did (ml/fxlm/kernels/optim.hip:44-51, :85-91).
#include <math.h>

#include <mutex>

#include "fx_device.h"

namespace fx {

constexpr int kOptThreads = 256;
constexpr int kOptVec = 4;                                   // 16-byte vectors per thread
constexpr int64_t kChunk = (int64_t)kOptThreads * 8 * kOptVec;  // 8192 elements

struct ChunkList {
    const uint16_t* g[FX_ADAMW_MAX_TENSORS];
    int64_t off[FX_ADAMW_MAX_TENSORS];
    int64_t n[FX_ADAMW_MAX_TENSORS];
    int32_t wd[FX_ADAMW_MAX_TENSORS];
    int32_t cstart[FX_ADAMW_MAX_TENSORS + 1];  // first chunk of each tensor
    int32_t count;
    int32_t pbase;                              // index of this list's first partial
};

__device__ __forceinline__ int find_tensor(const ChunkList& L, int b) {
    int t = 0;
    while (t + 1 < L.count && L.cstart[t + 1] <= b) ++t;
    return t;
}

// work layout (fp32): [0] = clip/scale, [1] = skip flag, [2] = 1/(1-beta1^step),
// [3] = 1/(1-beta2^step), [4..] partials
constexpr int kWorkHead = 4;

__global__ void __launch_bounds__(kOptThreads) adamw_sumsq_kernel(ChunkList L, float* __restrict__ work) {
    __shared__ float sh[kOptThreads / 64];
    const int b = blockIdx.x;
    const int t = find_tensor(L, b);
    const uint16_t* g = L.g[t];
    const int64_t n = L.n[t];
    const int64_t base = (int64_t)(b - L.cstart[t]) * kChunk;
    float ss = 0.f;
    uint4 gv[kOptVec];
#pragma unroll
    for (int u = 0; u < kOptVec; ++u) {
        const int64_t e = base + ((int64_t)u * kOptThreads + threadIdx.x) * 8;
        gv[u] = make_uint4(0u, 0u, 0u, 0u);
        if (e + 8 <= n) {
            gv[u] = ld16(g + e);  // cached: the update kernel re-reads it
        } else if (e < n) {
            uint16_t tmp[8] = {0, 0, 0, 0, 0, 0, 0, 0};
            for (int j = 0; j < 8 && e + j < n; ++j) tmp[j] = g[e + j];
            gv[u] = *reinterpret_cast<uint4*>(tmp);
        }
    }
#pragma unroll
    for (int u = 0; u < kOptVec; ++u) {
        float f[8];
        unpack8(gv[u], f);
#pragma unroll
        for (int j = 0; j < 8; ++j) ss += f[j] * f[j];
    }
    ss = group_sum<64>(ss);
    if ((threadIdx.x & 63) == 0) sh[threadIdx.x >> 6] = ss;
    __syncthreads();
    if (threadIdx.x == 0) {
        float s = 0.f;
#pragma unroll
        for (int i = 0; i < kOptThreads / 64; ++i) s += sh[i];
        work[kWorkHead + L.pbase + b] = s;
    }
}

__global__ void __launch_bounds__(1024)
adamw_final_kernel(float* __restrict__ work, int64_t nparts, int32_t* __restrict__ step,
                   float* __restrict__ found_inf, float* __restrict__ grad_norm,
                   float* __restrict__ scale, int32_t* __restrict__ growth, float max_norm,
                   float growth_factor, float backoff_factor, int32_t growth_interval, float beta1,
                   float beta2) {
    __shared__ double sh[16];
    double s = 0.0;
#pragma unroll 16
    for (int64_t i = threadIdx.x; i < nparts; i += 1024) s += (double)work[kWorkHead + i];
    s = group_sum_d<64>(s);
    if ((threadIdx.x & 63) == 0) sh[threadIdx.x >> 6] = s;
    __syncthreads();
    if (threadIdx.x != 0) return;
    double tot = 0.0;
    for (int i = 0; i < 16; ++i) tot += sh[i];
    const float sumsq = (float)tot;
    const bool bad = !isfinite(sumsq);
    const float sc = *scale;
    const float norm = sqrtf(sumsq) / sc;
    const float clip = bad ? 0.f : fminf(1.f, max_norm / (norm + 1e-6f));
    *found_inf = bad ? 1.f : 0.f;
    *grad_norm = norm;
    work[0] = clip / sc;
    work[1] = bad ? 1.f : 0.f;
    if (!bad) {
        const int32_t st = *step + 1;
        *step = st;
        work[2] = 1.f / (1.f - powf(beta1, (float)st));  // bias corrections of this step
        work[3] = 1.f / (1.f - powf(beta2, (float)st));
    }
    // loss-scale update (semantics of torch._amp_update_scale_)
    if (bad) {
        *scale = sc * backoff_factor;
        *growth = 0;
    } else {
        const int32_t ok = *growth + 1;
        if (ok == growth_interval) {
            const float ns = sc * growth_factor;
            if (isfinite(ns)) *scale = ns;
            *growth = 0;
        } else {
            *growth = ok;
        }
    }
}

__device__ __forceinline__ void adamw_elem(float g, float& w, float& m, float& v, float lr, float lrwd,
                                           float b1, float b2, float b1c, float b2c, float ibc1,
                                           float ibc2, float eps, bool wd_on) {
    if (wd_on) w -= lrwd * w;
    m = m * b1 + b1c * g;
    v = v * b2 + b2c * g * g;
    w -= lr * (m * ibc1) / (sqrtf(v * ibc2) + eps);
}

// One block per quarter chunk (kChunk / kOptVec = 2048 elements, 512 per wave).
// Lane l of a wave updates elements 4l..4l+3 and 256+4l..256+4l+3 of the wave's
// 512, so every load and store instruction covers one contiguous span (1 KB of
// fp32, 512 B of bf16).  The block's g/master/m/v loads are issued before the
// step's scalars (clip factor, skip flag, bias corrections) are read, so no block
// waits on them before its data is in flight.
// Cache policy: master, m and v are loaded and stored non-temporally, while the
// gradient (read just before by adamw_sumsq with ordinary loads) is loaded normally.
// The bf16 gradient of a 124M-parameter model (249 MB) then stays in the GPU's 256 MB
// memory-side cache between the two passes instead of being evicted by the 3 GB fp32
// stream, and its second read is served from there: 699 -> 627-639 us per step at
// 124,373,760 parameters, bitwise-identical results.
__global__ void __launch_bounds__(kOptThreads)
adamw_update_kernel(ChunkList L, const float* __restrict__ work, float* __restrict__ master,
                    float* __restrict__ mom, float* __restrict__ var, uint16_t* __restrict__ p16,
                    float lr, float b1, float b2, float eps, float wd) {
    const int b = blockIdx.x / kOptVec;
    const int u = blockIdx.x - b * kOptVec;
    const int t = find_tensor(L, b);
    const uint16_t* g = L.g[t];
    const int64_t n = L.n[t];
    const int64_t off = L.off[t];
    const bool wd_on = L.wd[t] != 0;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int64_t e0 = (int64_t)(b - L.cstart[t]) * kChunk + (int64_t)u * (kChunk / kOptVec) + wave * 512 + 4 * lane;
    const float b1c = 1.f - b1, b2c = 1.f - b2, lrwd = lr * wd;
    if (e0 + 256 + 4 <= n) {
        uint2 gq[2];
        float4 w[2], m[2], v[2];
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const int64_t e = e0 + 256 * h;
            gq[h] = *reinterpret_cast<const uint2*>(g + e);
            w[h] = ldf4_nt(master + off + e);
            m[h] = ldf4_nt(mom + off + e);
            v[h] = ldf4_nt(var + off + e);
        }
        const float4 sc = *reinterpret_cast<const float4*>(work);  // clip/scale, skip, 1/bc1, 1/bc2
        if (sc.y != 0.f) return;  // non-finite gradients: skip the step
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const int64_t e = e0 + 256 * h;
            const float gf[4] = {bf16_lo(gq[h].x), bf16_hi(gq[h].x), bf16_lo(gq[h].y), bf16_hi(gq[h].y)};
            float wf[4] = {w[h].x, w[h].y, w[h].z, w[h].w};
            float mf[4] = {m[h].x, m[h].y, m[h].z, m[h].w};
            float vf[4] = {v[h].x, v[h].y, v[h].z, v[h].w};
#pragma unroll
            for (int j = 0; j < 4; ++j)
                adamw_elem(gf[j] * sc.x, wf[j], mf[j], vf[j], lr, lrwd, b1, b2, b1c, b2c, sc.z, sc.w, eps, wd_on);
            stf4_nt(master + off + e, make_float4(wf[0], wf[1], wf[2], wf[3]));
            stf4_nt(mom + off + e, make_float4(mf[0], mf[1], mf[2], mf[3]));
            stf4_nt(var + off + e, make_float4(vf[0], vf[1], vf[2], vf[3]));
            uint2 o;
            o.x = pack_bf16x2(wf[0], wf[1]);
            o.y = pack_bf16x2(wf[2], wf[3]);
            *reinterpret_cast<uint2*>(p16 + off + e) = o;
        }
    } else if (e0 < n) {
        // tail of a tensor: this lane's two spans element by element
        const float4 sc = *reinterpret_cast<const float4*>(work);
        if (sc.y != 0.f) return;
        for (int h = 0; h < 2; ++h)
            for (int64_t i = e0 + 256 * h; i < e0 + 256 * h + 4 && i < n; ++i) {
                float w = master[off + i], m = mom[off + i], v = var[off + i];
                adamw_elem(bf16_to_f32(g[i]) * sc.x, w, m, v, lr, lrwd, b1, b2, b1c, b2c, sc.z, sc.w, eps,
                           wd_on);
                master[off + i] = w;
                mom[off + i] = m;
                var[off + i] = v;
                p16[off + i] = f32_to_bf16(w);
            }
    }
}

static int build_chunks(const fxTensorList& in, int32_t pbase, ChunkList& out, int64_t& nchunks) {
    FX_REQUIRE(in.count >= 0 && in.count <= FX_ADAMW_MAX_TENSORS, "fx_adamw: list count %d out of range",
               in.count);
    out.count = in.count;
    out.pbase = pbase;
    int64_t c = 0;
    for (int t = 0; t < in.count; ++t) {
        FX_REQUIRE(in.n[t] >= 0, "fx_adamw: tensor %d has n=%lld", t, (long long)in.n[t]);
        FX_REQUIRE(in.off[t] % 8 == 0, "fx_adamw: tensor %d offset %lld not a multiple of 8", t,
                   (long long)in.off[t]);
        FX_REQUIRE(in.n[t] == 0 || in.g[t] != nullptr, "fx_adamw: tensor %d has a null gradient", t);
        FX_REQUIRE(((uintptr_t)in.g[t] & 15) == 0, "fx_adamw: gradient %d not 16-byte aligned", t);
        out.g[t] = in.g[t];
        out.off[t] = in.off[t];
        out.n[t] = in.n[t];
        out.wd[t] = in.wd[t];
        out.cstart[t] = (int32_t)c;
        c += (in.n[t] + kChunk - 1) / kChunk;
        FX_REQUIRE(c * kOptVec < 0x7fffffff, "fx_adamw: too many chunks");
    }
    out.cstart[in.count] = (int32_t)c;
    nchunks = c;
    return 0;
}

// Workspace of fx_adamw_step_noalloc: a file-scope device array (one copy per GPU, held
// until the process ends).  In host code `scratch` names a host-side stand-in, not device
// memory: the kernels get the device address hipGetSymbolAddress returns for the
// current device, looked up once per device and kept.  The step writes every word it
// reads (the sum-of-squares kernel writes each chunk's partial, the final kernel the
// header) before reading it, so nothing needs clearing between calls.
static __device__ __align__(256) float scratch[FX_ADAMW_NOALLOC_SCRATCH_BYTES / sizeof(float)];

constexpr int kMaxDevices = 64;
static std::mutex g_scratch_mu;
static float* g_scratch[kMaxDevices];

static int scratch_ptr(float** out, const char* who) {
    int dev = -1;
    const hipError_t e = hipGetDevice(&dev);
    FX_REQUIRE(e == hipSuccess, "%s: hipGetDevice failed (%s)", who, hipGetErrorString(e));
    FX_REQUIRE(dev >= 0 && dev < kMaxDevices, "%s: device %d beyond the %d supported", who, dev, kMaxDevices);
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (g_scratch[dev] == nullptr) {
        void* p = nullptr;
        const hipError_t r = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (r != hipSuccess || p == nullptr)
            return set_error(r != hipSuccess ? (int)r : FX_EINVAL,
                             "%s: hipGetSymbolAddress(scratch) failed on device %d (%s)", who, dev,
                             hipGetErrorString(r));
        g_scratch[dev] = static_cast<float*>(p);
    }
    *out = g_scratch[dev];
    return 0;
}

}  // namespace fx

using namespace fx;

extern "C" int64_t fx_adamw_workspace(const fxTensorList* lists, int32_t nlists) {
    int64_t parts = 0;
    for (int i = 0; lists != nullptr && i < nlists; ++i)
        for (int t = 0; t < lists[i].count && t < FX_ADAMW_MAX_TENSORS; ++t)
            if (lists[i].n[t] > 0) parts += (lists[i].n[t] + kChunk - 1) / kChunk;
    return (kWorkHead + parts) * (int64_t)sizeof(float);
}

// The step's launches with `work` as the workspace (null: the per-device scratch below,
// whose size is checked against the lists first).
static int adamw_step(const fxAdamWState* st, const fxTensorList* lists, int32_t nlists, float* work,
                      void* stream, const char* who) {
    FX_REQUIRE(st != nullptr, "%s: null state", who);
    FX_REQUIRE(nlists >= 0 && (nlists == 0 || lists != nullptr), "%s: bad lists", who);
    FX_REQUIRE(st->master && st->m && st->v && st->p16 && st->step && st->found_inf && st->grad_norm &&
                   st->scale && st->growth,
               "%s: null state pointer", who);
    FX_REQUIRE(((uintptr_t)st->master & 31) == 0 && ((uintptr_t)st->m & 31) == 0 &&
                   ((uintptr_t)st->v & 31) == 0 && ((uintptr_t)st->p16 & 15) == 0,
               "%s: flat buffers must be 32-byte (fp32) / 16-byte (bf16) aligned", who);
    hipStream_t s = (hipStream_t)stream;
    // At most a few lists: keep their chunk tables on the host stack.
    FX_REQUIRE(nlists <= 64, "%s: %d lists (max 64)", who, nlists);
    ChunkList cl[64];
    int64_t nch[64];
    int64_t total = 0;
    for (int i = 0; i < nlists; ++i) {
        if (int e = build_chunks(lists[i], (int32_t)total, cl[i], nch[i])) return e;
        total += nch[i];
        FX_REQUIRE(total * kOptVec < 0x7fffffff, "%s: too many chunks over the lists", who);
    }
    if (work == nullptr) {
        const int64_t need = (kWorkHead + total) * (int64_t)sizeof(float);
        FX_REQUIRE(need <= FX_ADAMW_NOALLOC_SCRATCH_BYTES,
                   "%s: %lld chunks of %lld elements need %lld bytes of scratch, more than its %lld "
                   "(at most %lld parameters)", who, (long long)total, (long long)kChunk, (long long)need,
                   (long long)FX_ADAMW_NOALLOC_SCRATCH_BYTES,
                   (long long)((FX_ADAMW_NOALLOC_SCRATCH_BYTES / (int64_t)sizeof(float) - kWorkHead) * kChunk));
        if (int e = scratch_ptr(&work, who)) return e;
    }
    FX_REQUIRE(((uintptr_t)work & 15) == 0, "%s: work must be 16-byte aligned", who);
    for (int i = 0; i < nlists; ++i) {
        if (nch[i] == 0) continue;
        hipLaunchKernelGGL(adamw_sumsq_kernel, dim3((unsigned)nch[i]), dim3(kOptThreads), 0, s, cl[i], work);
        if (int e = check_launch("adamw_sumsq")) return e;
    }
    hipLaunchKernelGGL(adamw_final_kernel, dim3(1), dim3(1024), 0, s, work, total, st->step,
                       st->found_inf, st->grad_norm, st->scale, st->growth, st->max_grad_norm,
                       st->growth_factor, st->backoff_factor, st->growth_interval, st->beta1, st->beta2);
    if (int e = check_launch("adamw_final")) return e;
    for (int i = 0; i < nlists; ++i) {
        if (nch[i] == 0) continue;
        hipLaunchKernelGGL(adamw_update_kernel, dim3((unsigned)(nch[i] * kOptVec)), dim3(kOptThreads), 0, s,
                           cl[i], (const float*)work, st->master, st->m, st->v, st->p16, st->lr,
                           st->beta1, st->beta2, st->eps, st->weight_decay);
        if (int e = check_launch("adamw_update")) return e;
    }
    return 0;
}

extern "C" int fx_adamw_step(const fxAdamWState* st, const fxTensorList* lists, int32_t nlists,
                             void* stream) {
    FX_REQUIRE(st != nullptr && st->work != nullptr, "fx_adamw_step: null state or workspace");
    return adamw_step(st, lists, nlists, st->work, stream, "fx_adamw_step");
}

extern "C" int fx_adamw_step_noalloc(const fxAdamWState* st, const fxTensorList* lists, int32_t nlists,
                                     void* stream) {
    return adamw_step(st, lists, nlists, nullptr, stream, "fx_adamw_step_noalloc");
}
