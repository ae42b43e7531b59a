// Decode attention for gfx950: one new query per (sequence, head) against a KV cache.
//
// o[b, h] = softmax(scale * q[b, h] . K[b, :len_b, h]) V[b, :len_b, h]: the last row of
// causal attention over the cached keys, which is what the reference's sampler
// recomputes from the whole context for every token (ml/fxlm/sample.py:62-73).
//
// HBM-bound (each cached key and value is read once per step, 4 D bytes per key and
// head), so the work is split over the keys: one wave per (sequence, head, chunk of CH
// keys), CH = 256, 128 or 64, the largest that still gives kDecWaves waves (enough
// loads in flight to cover HBM latency).  A key row is read by D/8 lanes, 16 bytes each, so one load instruction
// covers 64 / (D/8) whole rows.  Pass 1 keeps all of the chunk's scores in registers
// (log2 domain, q pre-scaled), then one max / exp pass; pass 2 accumulates P V with
// each lane owning 8 of the D outputs; the partial (max, sum, o) of every chunk is
// merged by the second kernel with the same rule as the forward's lse.  Chunks that
// start at or past the sequence's length do nothing and the merge reads only the
// chunks below it.  With a single chunk the first kernel writes the result itself.
#include <math.h>

#include "fx_device.h"

namespace fx {

constexpr int kDecBatch = 8;      // key loads in flight per lane
constexpr int kDecWaves = 2048;   // grid size the chunk choice aims for
constexpr float kDecNegInf = -__builtin_huge_valf();

template <int D, int CH>
__global__ void __launch_bounds__(64) attn_decode_kernel(fxAttnDecodeArgs a, int nchunks) {
    constexpr int LPK = D / 8;       // lanes per key row
    constexpr int KPI = 64 / LPK;    // key rows per load instruction
    constexpr int NS = CH / KPI;     // load steps per chunk
    static_assert(NS % kDecBatch == 0, "chunk");
    const int lane = threadIdx.x;
    const int kg = lane / LPK, dl = lane % LPK;  // key group and 8-element slice of D
    const int c = blockIdx.x % nchunks;
    const int bh = blockIdx.x / nchunks;
    const int b = bh / a.H, h = bh - b * a.H;
    int len = a.lens[b];
    len = len < 0 ? 0 : (len > a.Tmax ? a.Tmax : len);
    const int j0 = c * CH;
    if (nchunks > 1 && j0 >= len) return;  // the merge skips this chunk

    float qf[8];
    {
        const float s = a.scale * kLog2e;
        unpack8(ld16(a.q + b * a.qsb + h * a.qsh + dl * 8), qf);
#pragma unroll
        for (int e = 0; e < 8; ++e) qf[e] *= s;
    }
    const uint16_t* kb = a.k + b * a.ksb + h * a.ksh + dl * 8;
    const uint16_t* vb = a.v + b * a.vsb + h * a.vsh + dl * 8;

    // pass 1: scores of keys j0 + s KPI + kg, s < NS
    float sc[NS];
    float m = kDecNegInf;
#pragma unroll
    for (int s0 = 0; s0 < NS; s0 += kDecBatch) {
        uint4 kv[kDecBatch];
#pragma unroll
        for (int u = 0; u < kDecBatch; ++u) {
            const int j = j0 + (s0 + u) * KPI + kg;
            kv[u] = j < len ? ld16(kb + (int64_t)j * a.kst) : make_uint4(0u, 0u, 0u, 0u);
        }
#pragma unroll
        for (int u = 0; u < kDecBatch; ++u) {
            float kf[8];
            unpack8(kv[u], kf);
            float t = 0.f;
#pragma unroll
            for (int e = 0; e < 8; ++e) t = fmaf(qf[e], kf[e], t);
            t = group_sum<LPK>(t);
            const int j = j0 + (s0 + u) * KPI + kg;
            sc[s0 + u] = j < len ? t : kDecNegInf;
            m = fmaxf(m, sc[s0 + u]);
        }
    }
    // chunk max over the key groups (lanes with equal dl hold equal values already)
#pragma unroll
    for (int off = LPK; off < 64; off <<= 1) m = fmaxf(m, __shfl_xor(m, off, 64));
    const float mu = m == kDecNegInf ? 0.f : m;
    float l = 0.f;
#pragma unroll
    for (int s = 0; s < NS; ++s) {
        sc[s] = exp2_fast(sc[s] - mu);  // exp2(-inf) = 0
        l += sc[s];
    }
    // pass 2: o = sum_j p_j v_j over this lane's key group, 8 outputs per lane
    float o[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s0 = 0; s0 < NS; s0 += kDecBatch) {
        uint4 vv[kDecBatch];
#pragma unroll
        for (int u = 0; u < kDecBatch; ++u) {
            const int j = j0 + (s0 + u) * KPI + kg;
            vv[u] = j < len ? ld16(vb + (int64_t)j * a.vst) : make_uint4(0u, 0u, 0u, 0u);
        }
#pragma unroll
        for (int u = 0; u < kDecBatch; ++u) {
            float vf[8];
            unpack8(vv[u], vf);
#pragma unroll
            for (int e = 0; e < 8; ++e) o[e] = fmaf(sc[s0 + u], vf[e], o[e]);
        }
    }
    // sum over the key groups: every lane of slice dl ends with the chunk's o slice
#pragma unroll
    for (int off = LPK; off < 64; off <<= 1) {
        l += __shfl_xor(l, off, 64);
#pragma unroll
        for (int e = 0; e < 8; ++e) o[e] += __shfl_xor(o[e], off, 64);
    }
    if (kg != 0) return;
    if (nchunks == 1) {  // the only chunk: final output
        const float inv = l > 0.f ? 1.f / l : 0.f;
#pragma unroll
        for (int e = 0; e < 8; ++e) o[e] *= inv;
        st16(a.o + (int64_t)bh * D + dl * 8, pack8(o));
        if (a.lse && dl == 0) a.lse[bh] = l > 0.f ? (m + log2_fast(l)) * kLn2 : kDecNegInf;
        return;
    }
    // partial of chunk c: (max, sum, o[D]) at work + (bh * nchunks + c) * (D + 4)
    float* w = a.work + ((int64_t)bh * nchunks + c) * (D + 4);
    *reinterpret_cast<float4*>(w + 4 + dl * 8) = make_float4(o[0], o[1], o[2], o[3]);
    *reinterpret_cast<float4*>(w + 8 + dl * 8) = make_float4(o[4], o[5], o[6], o[7]);
    if (dl == 0) *reinterpret_cast<float2*>(w) = make_float2(m, l);
}

// merge the chunk partials of one (sequence, head) per wave, over the chunks that hold
// keys (c CH < len): M = max m_c, L = sum l_c 2^(m_c - M), o = sum o_c 2^(m_c - M) / L,
// lse = (M + log2 L) ln 2
template <int D, int CH>
__global__ void __launch_bounds__(64) attn_decode_merge_kernel(fxAttnDecodeArgs a, int nchunks) {
    constexpr int EPL = D / 64;  // outputs per lane
    const int lane = threadIdx.x;
    const int bh = blockIdx.x;
    int len = a.lens[bh / a.H];
    len = len < 0 ? 0 : (len > a.Tmax ? a.Tmax : len);
    const int nc = (len + CH - 1) / CH;  // <= nchunks
    const float* w = a.work + (int64_t)bh * nchunks * (D + 4);
    float M = kDecNegInf;
    for (int c = 0; c < nc; ++c) M = fmaxf(M, w[(int64_t)c * (D + 4)]);
    const float mu = M == kDecNegInf ? 0.f : M;
    float L = 0.f, o[EPL];
#pragma unroll
    for (int e = 0; e < EPL; ++e) o[e] = 0.f;
    for (int c = 0; c < nc; ++c) {
        const float* p = w + (int64_t)c * (D + 4);
        const float f = exp2_fast(p[0] - mu);
        L += p[1] * f;
#pragma unroll
        for (int e = 0; e < EPL; ++e) o[e] += p[4 + lane * EPL + e] * f;
    }
    const float inv = L > 0.f ? 1.f / L : 0.f;
    uint16_t* out = a.o + (int64_t)bh * D + lane * EPL;
#pragma unroll
    for (int e = 0; e < EPL; ++e) out[e] = f32_to_bf16(o[e] * inv);
    if (a.lse && lane == 0) a.lse[bh] = L > 0.f ? (M + log2_fast(L)) * kLn2 : kDecNegInf;
}

// keys per chunk: the largest of 256, 128, 64 whose grid reaches kDecWaves waves
static int decode_chunk(int32_t B, int32_t H, int32_t Tmax) {
    for (int ch = 256; ch > 64; ch >>= 1)
        if ((int64_t)B * H * ((Tmax + ch - 1) / ch) >= kDecWaves) return ch;
    return 64;
}
static int decode_chunks(int32_t B, int32_t H, int32_t Tmax) {
    const int ch = decode_chunk(B, H, Tmax);
    return (Tmax + ch - 1) / ch;
}

template <int D, int CH>
static int decode_launch(const fxAttnDecodeArgs& a, int nc, hipStream_t st) {
    const unsigned nbh = (unsigned)(a.B * a.H);
    hipLaunchKernelGGL((attn_decode_kernel<D, CH>), dim3(nbh * nc), dim3(64), 0, st, a, nc);
    if (int e = check_launch("attn_decode")) return e;
    if (nc == 1) return 0;
    hipLaunchKernelGGL((attn_decode_merge_kernel<D, CH>), dim3(nbh), dim3(64), 0, st, a, nc);
    return check_launch("attn_decode_merge");
}

}  // namespace fx

using namespace fx;

extern "C" int64_t fx_attn_decode_workspace(int32_t B, int32_t H, int32_t Tmax, int32_t D) {
    if (B <= 0 || H <= 0 || Tmax <= 0 || D <= 0) return 0;
    const int nc = decode_chunks(B, H, Tmax);
    return nc > 1 ? (int64_t)B * H * nc * (D + 4) * (int64_t)sizeof(float) : 0;
}

extern "C" int fx_attn_decode(const fxAttnDecodeArgs* args, void* stream) {
    FX_REQUIRE(args != nullptr, "fx_attn_decode: null args");
    const fxAttnDecodeArgs& a = *args;
    FX_REQUIRE(a.D == 64 || a.D == 128, "fx_attn_decode: head_dim %d not supported (64 or 128)", a.D);
    FX_REQUIRE(a.B >= 1 && a.H >= 1 && a.Tmax >= 1, "fx_attn_decode: bad shape B=%d H=%d Tmax=%d", a.B, a.H,
               a.Tmax);
    FX_REQUIRE((int64_t)a.B * a.H * ((a.Tmax + 63) / 64) < 0x7fffffffLL, "fx_attn_decode: grid too large");
    FX_REQUIRE(a.q && a.k && a.v && a.lens && a.o, "fx_attn_decode: null pointer");
    FX_REQUIRE(a.scale > 0.f && a.scale < __builtin_huge_valf(), "fx_attn_decode: scale %g must be positive and finite",
               (double)a.scale);
    const int64_t s[] = {a.qsb, a.qsh, a.ksb, a.kst, a.ksh, a.vsb, a.vst, a.vsh};
    for (int64_t x : s) FX_REQUIRE(x % 8 == 0, "fx_attn_decode: strides must be multiples of 8 elements");
    FX_REQUIRE((((uintptr_t)a.q | (uintptr_t)a.k | (uintptr_t)a.v | (uintptr_t)a.o | (uintptr_t)a.work) & 15) == 0,
               "fx_attn_decode: q, k, v, o and work must be 16-byte aligned");
    const int ch = decode_chunk(a.B, a.H, a.Tmax);
    const int nc = (a.Tmax + ch - 1) / ch;
    FX_REQUIRE(nc == 1 || a.work != nullptr, "fx_attn_decode: null workspace (%d chunks)", nc);
    hipStream_t st = (hipStream_t)stream;
    if (a.D == 64)
        return ch == 256 ? decode_launch<64, 256>(a, nc, st)
             : ch == 128 ? decode_launch<64, 128>(a, nc, st)
                         : decode_launch<64, 64>(a, nc, st);
    return ch == 256 ? decode_launch<128, 256>(a, nc, st)
         : ch == 128 ? decode_launch<128, 128>(a, nc, st)
                     : decode_launch<128, 64>(a, nc, st);
}
