// Decode attention for gfx950: one new query per (sequence, head) against a KV cache.
//
// o[b, h] = softmax(scale * q[b, h] . K[b, :len_b, h]) V[b, :len_b, h]: the last row of
// causal attention over the cached keys, which is what the reference's sampler
// recomputes from the whole context for every token (ml/fxlm/sample.py:62-73).
//
// HBM-bound: each cached key and value is read once per step (4 D bytes per key and
// head).  One workgroup per (sequence, head) -- or per (sequence, head, segment of the
// keys) when there are fewer (sequence, head) pairs than half the CUs -- of up to 16
// waves.  Wave w streams sub-chunks w, w + nw, ... of CH keys (64 at D = 64, 32 at
// D = 128); a key row is read by D/8 lanes, 16 bytes each, and a sub-chunk's K and V
// rows are all loaded at once (one memory round trip per sub-chunk).  Every lane keeps
// an online softmax (max, sum, o for its 8 of the D outputs) over the keys of its key
// group; the key groups of a wave combine with lane exchanges at the end, the waves
// through LDS in wave order.  With one segment the workgroup writes the output; with
// several it writes (max, sum, o) per segment and a second kernel merges them by the
// forward's lse rule, reading only the segments below the sequence's length.  Given
// the new token's key and value (knew / vnew), the wave that reaches key len - 1 reads
// it from there and writes it into the caches: the step needs no separate cache write.
#include <math.h>

#include "fx_device.h"

namespace fx {

constexpr int kDecMaxWaves = 16;
constexpr float kDecNegInf = -__builtin_huge_valf();

// (m, l, o[8]) <- (m, l, o) merged with (m2, l2, o2): max-rescaled sums in the exp2 domain
__device__ __forceinline__ void dec_merge(float& m, float& l, float (&o)[8], float m2, float l2,
                                          const float (&o2)[8]) {
    const float M = fmaxf(m, m2);
    const float mu = M == kDecNegInf ? 0.f : M;
    const float f1 = exp2_fast(m - mu), f2 = exp2_fast(m2 - mu);  // 0 for an empty side
    l = l * f1 + l2 * f2;
#pragma unroll
    for (int e = 0; e < 8; ++e) o[e] = o[e] * f1 + o2[e] * f2;
    m = M;
}

template <int D, int CH>
__global__ void __launch_bounds__(64 * kDecMaxWaves) attn_decode_kernel(fxAttnDecodeArgs a, int nseg,
                                                                        int seglen) {
    constexpr int LPK = D / 8;       // lanes per key row
    constexpr int KPI = 64 / LPK;    // key rows per load instruction
    constexpr int NS = CH / KPI;     // load steps per sub-chunk
    __shared__ float red[kDecMaxWaves][D + 2];
    const int lane = threadIdx.x & 63;
    const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int nw = blockDim.x >> 6;
    const int kg = lane / LPK, dl = lane % LPK;  // key group and 8-element slice of D
    const int seg = blockIdx.x % nseg;
    const int bh = blockIdx.x / nseg;
    const int b = bh / a.H, h = bh - b * a.H;
    int len = a.lens[b];
    len = len < 0 ? 0 : (len > a.Tmax ? a.Tmax : len);
    const int k0 = seg * seglen;
    if (nseg > 1 && k0 >= len) return;  // the merge skips this segment (uniform per block)
    const int k1 = min(k0 + seglen, len);

    float qf[8];
    {
        const float s = a.scale * kLog2e;
        unpack8(ld16(a.q + b * a.qsb + h * a.qsh + dl * 8), qf);
#pragma unroll
        for (int e = 0; e < 8; ++e) qf[e] *= s;
    }
    const uint16_t* kb = a.k + b * a.ksb + h * a.ksh + dl * 8;
    const uint16_t* vb = a.v + b * a.vsb + h * a.vsh + dl * 8;
    // the new token's key / value (row len - 1) when given: read from knew / vnew and
    // stored into the caches by the lanes that load it (no other lane reads that row)
    const int jnew = a.knew ? len - 1 : -1;
    const uint16_t* kn = a.knew ? a.knew + b * a.knb + h * a.knh + dl * 8 : nullptr;
    const uint16_t* vn = a.vnew ? a.vnew + b * a.vnb + h * a.vnh + dl * 8 : nullptr;

    float m = kDecNegInf, l = 0.f;
    float o[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    for (int j0 = k0 + w * CH; j0 < k1; j0 += nw * CH) {
        uint4 kv[NS], vv[NS];
#pragma unroll
        for (int s = 0; s < NS; ++s) {
            const int j = j0 + s * KPI + kg;
            const bool ok = j < k1;
            if (j == jnew) {
                kv[s] = ld16(kn);
                vv[s] = ld16(vn);
                st16(const_cast<uint16_t*>(kb) + (int64_t)j * a.kst, kv[s]);
                st16(const_cast<uint16_t*>(vb) + (int64_t)j * a.vst, vv[s]);
            } else {
                kv[s] = ok ? ld16(kb + (int64_t)j * a.kst) : make_uint4(0u, 0u, 0u, 0u);
                vv[s] = ok ? ld16(vb + (int64_t)j * a.vst) : make_uint4(0u, 0u, 0u, 0u);
            }
        }
        float sc[NS];
        float mc = kDecNegInf;
#pragma unroll
        for (int s = 0; s < NS; ++s) {
            float kf[8];
            unpack8(kv[s], kf);
            float t = 0.f;
#pragma unroll
            for (int e = 0; e < 8; ++e) t = fmaf(qf[e], kf[e], t);
            t = group_sum<LPK>(t);
            sc[s] = (j0 + s * KPI + kg) < k1 ? t : kDecNegInf;
            mc = fmaxf(mc, sc[s]);
        }
        // online softmax over this lane's key group (lanes of one group hold equal scores)
        const float mn = fmaxf(m, mc);
        const float mu = mn == kDecNegInf ? 0.f : mn;
        const float alpha = exp2_fast(m - mu);
        l *= alpha;
#pragma unroll
        for (int e = 0; e < 8; ++e) o[e] *= alpha;
        m = mn;
#pragma unroll
        for (int s = 0; s < NS; ++s) {
            const float p = exp2_fast(sc[s] - mu);  // exp2(-inf) = 0
            l += p;
            float vf[8];
            unpack8(vv[s], vf);
#pragma unroll
            for (int e = 0; e < 8; ++e) o[e] = fmaf(p, vf[e], o[e]);
        }
    }
    // key groups of the wave: lanes kg and kg ^ (off / LPK) merge, every lane of slice dl
    // ends with the wave's (m, l, o)
#pragma unroll
    for (int off = LPK; off < 64; off <<= 1) {
        float o2[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) o2[e] = __shfl_xor(o[e], off, 64);
        const float m2 = __shfl_xor(m, off, 64), l2 = __shfl_xor(l, off, 64);
        dec_merge(m, l, o, m2, l2, o2);
    }
    if (kg == 0) {
#pragma unroll
        for (int e = 0; e < 8; ++e) red[w][dl * 8 + e] = o[e];
        if (dl == 0) {
            red[w][D] = m;
            red[w][D + 1] = l;
        }
    }
    __syncthreads();
    // waves in order: one thread per output dimension
    for (int t = threadIdx.x; t < D; t += blockDim.x) {
        float M = kDecNegInf;
        for (int v = 0; v < nw; ++v) M = fmaxf(M, red[v][D]);
        const float mu = M == kDecNegInf ? 0.f : M;
        float L = 0.f, O = 0.f;
        for (int v = 0; v < nw; ++v) {
            const float f = exp2_fast(red[v][D] - mu);
            L += red[v][D + 1] * f;
            O += red[v][t] * f;
        }
        if (nseg == 1) {
            a.o[(int64_t)bh * D + t] = f32_to_bf16(L > 0.f ? O / L : 0.f);
            if (a.lse && t == 0) a.lse[bh] = L > 0.f ? (M + log2_fast(L)) * kLn2 : kDecNegInf;
        } else {
            // segment partial (max, sum, o[D]) at work + (bh * nseg + seg) * (D + 4)
            float* pw = a.work + ((int64_t)bh * nseg + seg) * (D + 4);
            pw[4 + t] = O;
            if (t == 0) {
                pw[0] = M;
                pw[1] = L;
            }
        }
    }
}

// merge the segment partials of one (sequence, head) per wave, over the segments that
// hold keys (s * seglen < len): M = max m_s, L = sum l_s 2^(m_s - M),
// o = sum o_s 2^(m_s - M) / L, lse = (M + log2 L) ln 2
template <int D>
__global__ void __launch_bounds__(64) attn_decode_merge_kernel(fxAttnDecodeArgs a, int nseg, int seglen) {
    constexpr int EPL = D / 64;  // outputs per lane
    const int lane = threadIdx.x;
    const int bh = blockIdx.x;
    int len = a.lens[bh / a.H];
    len = len < 0 ? 0 : (len > a.Tmax ? a.Tmax : len);
    const int ns = (len + seglen - 1) / seglen;  // <= nseg
    const float* w = a.work + (int64_t)bh * nseg * (D + 4);
    float M = kDecNegInf;
    for (int c = 0; c < ns; ++c) M = fmaxf(M, w[(int64_t)c * (D + 4)]);
    const float mu = M == kDecNegInf ? 0.f : M;
    float L = 0.f, o[EPL];
#pragma unroll
    for (int e = 0; e < EPL; ++e) o[e] = 0.f;
    for (int c = 0; c < ns; ++c) {
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

// Launch shape: segments, waves per workgroup and keys per segment.  One segment per
// (sequence, head) once those fill half the CUs; else enough segments for about one
// workgroup per CU, each at least two sub-chunks long.
struct DecodeShape {
    int nseg, nw, seglen;
};

static DecodeShape decode_shape(int32_t B, int32_t H, int32_t Tmax, int32_t D) {
    const int ch = D == 64 ? 64 : 32;
    const int64_t nbh = (int64_t)B * H;
    const int nsub = (Tmax + ch - 1) / ch;
    const int64_t cus = device_cus();
    int nseg = 1;
    if (nbh < cus / 2) {
        const int64_t want = (cus + nbh - 1) / nbh;
        const int64_t most = (nsub + 1) / 2;
        nseg = (int)(want < most ? want : most);
        if (nseg < 1) nseg = 1;
    }
    const int per = (nsub + nseg - 1) / nseg;  // sub-chunks per segment
    nseg = (nsub + per - 1) / per;             // no empty trailing segment
    return {nseg, per < kDecMaxWaves ? per : kDecMaxWaves, per * ch};
}

template <int D>
static int decode_launch(const fxAttnDecodeArgs& a, const DecodeShape& s, hipStream_t st) {
    constexpr int CH = D == 64 ? 64 : 32;
    const unsigned nbh = (unsigned)(a.B * a.H);
    hipLaunchKernelGGL((attn_decode_kernel<D, CH>), dim3(nbh * s.nseg), dim3(64 * s.nw), 0, st, a, s.nseg,
                       s.seglen);
    if (int e = check_launch("attn_decode")) return e;
    if (s.nseg == 1) return 0;
    hipLaunchKernelGGL((attn_decode_merge_kernel<D>), dim3(nbh), dim3(64), 0, st, a, s.nseg, s.seglen);
    return check_launch("attn_decode_merge");
}

}  // namespace fx

using namespace fx;

extern "C" int64_t fx_attn_decode_workspace(int32_t B, int32_t H, int32_t Tmax, int32_t D) {
    if (B <= 0 || H <= 0 || Tmax <= 0 || (D != 64 && D != 128)) return 0;
    const DecodeShape s = decode_shape(B, H, Tmax, D);
    return s.nseg > 1 ? (int64_t)B * H * s.nseg * (D + 4) * (int64_t)sizeof(float) : 0;
}

extern "C" int fx_attn_decode(const fxAttnDecodeArgs* args, void* stream) {
    FX_REQUIRE(args != nullptr, "fx_attn_decode: null args");
    const fxAttnDecodeArgs& a = *args;
    FX_REQUIRE(a.D == 64 || a.D == 128, "fx_attn_decode: head_dim %d not supported (64 or 128)", a.D);
    FX_REQUIRE(a.B >= 1 && a.H >= 1 && a.Tmax >= 1, "fx_attn_decode: bad shape B=%d H=%d Tmax=%d", a.B, a.H,
               a.Tmax);
    FX_REQUIRE((int64_t)a.B * a.H * ((a.Tmax + 31) / 32) < 0x7fffffffLL, "fx_attn_decode: grid too large");
    FX_REQUIRE(a.q && a.k && a.v && a.lens && a.o, "fx_attn_decode: null pointer");
    FX_REQUIRE(a.scale > 0.f && a.scale < __builtin_huge_valf(), "fx_attn_decode: scale %g must be positive and finite",
               (double)a.scale);
    const int64_t s[] = {a.qsb, a.qsh, a.ksb, a.kst, a.ksh, a.vsb, a.vst, a.vsh, a.knb, a.knh, a.vnb, a.vnh};
    for (int64_t x : s) FX_REQUIRE(x % 8 == 0, "fx_attn_decode: strides must be multiples of 8 elements");
    FX_REQUIRE((a.knew == nullptr) == (a.vnew == nullptr), "fx_attn_decode: knew and vnew go together");
    FX_REQUIRE((((uintptr_t)a.q | (uintptr_t)a.k | (uintptr_t)a.v | (uintptr_t)a.o | (uintptr_t)a.work |
                 (uintptr_t)a.knew | (uintptr_t)a.vnew) & 15) == 0,
               "fx_attn_decode: q, k, v, o, work, knew and vnew must be 16-byte aligned");
    const DecodeShape sh = decode_shape(a.B, a.H, a.Tmax, a.D);
    FX_REQUIRE(sh.nseg == 1 || a.work != nullptr, "fx_attn_decode: null workspace (%d segments)", sh.nseg);
    hipStream_t st = (hipStream_t)stream;
    return a.D == 64 ? decode_launch<64>(a, sh, st) : decode_launch<128>(a, sh, st);
}
