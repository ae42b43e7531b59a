// Shared device helpers for the gfx950 kernels: bf16 packing, 16-byte vector
// access, wave64 reductions and the host-side error plumbing of the C ABI.
#pragma once

#include <hip/hip_runtime.h>
#include <hip/hip_bf16.h>
#include <stdint.h>

#include "../../include/fx_abi.h"

// ---------------------------------------------------------------------------
// host side: error string of the last failed call (per host thread)

namespace fx {

int set_error(int code, const char* fmt, ...);
int check_launch(const char* what);   // hipGetLastError -> return code
// compute units of the current device (queried once per process; 256 if the query fails)
int device_cus();

}  // namespace fx

#define FX_REQUIRE(cond, ...)                                   \
    do {                                                        \
        if (!(cond)) return ::fx::set_error(FX_EINVAL, __VA_ARGS__); \
    } while (0)

// ---------------------------------------------------------------------------
// device side

namespace fx {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

// bf16 bit pattern -> fp32 (exact)
__device__ __forceinline__ float bf16_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }
__device__ __forceinline__ float bf16_to_f32(uint16_t h) { return __uint_as_float((uint32_t)h << 16); }

typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef float f32x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));

// two fp32 -> packed bf16 pair, round-to-nearest-even (one v_cvt_pk_bf16_f32)
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
    return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2){lo, hi}, bf16x2));
}
__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
    return (uint16_t)(pack_bf16x2(f, 0.f) & 0xffffu);
}

// 8 bf16 in a uint4 <-> 8 fp32
__device__ __forceinline__ void unpack8(const uint4& v, float* f) {
    f[0] = bf16_lo(v.x); f[1] = bf16_hi(v.x);
    f[2] = bf16_lo(v.y); f[3] = bf16_hi(v.y);
    f[4] = bf16_lo(v.z); f[5] = bf16_hi(v.z);
    f[6] = bf16_lo(v.w); f[7] = bf16_hi(v.w);
}
__device__ __forceinline__ uint4 pack8(const float* f) {
    const f32x8 v = {f[0], f[1], f[2], f[3], f[4], f[5], f[6], f[7]};
    return __builtin_bit_cast(uint4, __builtin_convertvector(v, bf16x8));
}

__device__ __forceinline__ uint4 ld16(const void* p) { return *reinterpret_cast<const uint4*>(p); }
__device__ __forceinline__ void st16(void* p, const uint4& v) { *reinterpret_cast<uint4*>(p) = v; }

// streaming (non-temporal) variants for data touched exactly once
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ uint4 ld16_nt(const void* p) {
    u32x4 r = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
    return make_uint4(r.x, r.y, r.z, r.w);
}
__device__ __forceinline__ void st16_nt(void* p, const uint4& v) {
    u32x4 r = {v.x, v.y, v.z, v.w};
    __builtin_nontemporal_store(r, reinterpret_cast<u32x4*>(p));
}
__device__ __forceinline__ float4 ldf4_nt(const float* p) {
    const f32x4 r = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(p));
    return make_float4(r.x, r.y, r.z, r.w);
}
__device__ __forceinline__ void stf4_nt(float* p, const float4& v) {
    const f32x4 r = {v.x, v.y, v.z, v.w};
    __builtin_nontemporal_store(r, reinterpret_cast<f32x4*>(p));
}

// butterfly reductions over groups of W consecutive lanes (W a power of two <= 64)
template <int W>
__device__ __forceinline__ float group_sum(float v) {
#pragma unroll
    for (int off = W / 2; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
    return v;
}
template <int W>
__device__ __forceinline__ float group_max(float v) {
#pragma unroll
    for (int off = W / 2; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, 64));
    return v;
}
template <int W>
__device__ __forceinline__ double group_sum_d(double v) {
#pragma unroll
    for (int off = W / 2; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
    return v;
}

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;

// 2^x on the transcendental unit (v_exp_f32)
__device__ __forceinline__ float exp2_fast(float x) { return __builtin_amdgcn_exp2f(x); }
// log2(x) on the transcendental unit (v_log_f32)
__device__ __forceinline__ float log2_fast(float x) { return __builtin_amdgcn_logf(x); }

// GELU, tanh approximation: 0.5 h (1 + tanh(u)), u = sqrt(2/pi) (h + 0.044715 h^3),
// evaluated as h / (1 + e) with e = exp(-2u) (= h * sigmoid(2u)): e = 2^(h (k0 + k1 h^2)),
// the constants -2 log2(e) sqrt(2/pi) (1, 0.044715) folded, so three multiplies / fmas,
// v_exp_f32, one add, v_rcp_f32 (1 ulp, not a correctly rounded division, a
// ten-instruction sequence) and one multiply.  e = 0 gives h, e = inf gives h * 0 (-0 for
// negative h, as 0.5 h (1 + tanh(u)) gives); h = +inf gives +inf.
__device__ __forceinline__ float gelu_tanh(float h) {
    constexpr float k0 = -2.f * 1.4426950408889634f * 0.7978845608028654f;
    constexpr float k1 = k0 * 0.044715f;
    const float e = exp2_fast(h * fmaf(h * h, k1, k0));
    return h * __builtin_amdgcn_rcpf(e + 1.f);
}

// GELU and its derivative from the one v_exp_f32 and v_rcp_f32 of gelu_tanh: with
// s = 1 / (1 + e) = sigmoid(2u), GELU = h s (c here is gelu_tanh(h) bit for bit) and
// d/dh (h s) = s + h s (1 - s) 2 u'(h) = s (1 + h (1 - s) (2c0 + 6 c0 0.044715 h^2)),
// c0 = sqrt(2/pi), which equals gelu_tanh_grad's 0.5 (1 + t) + 0.5 h (1 - t^2) u' since
// 1 + t = 2 s and 1 - t^2 = 4 s (1 - s).  Four more VALU operations than the GELU alone.
__device__ __forceinline__ void gelu_tanh_and_grad(float h, float& c, float& d) {
    constexpr float k0 = -2.f * 1.4426950408889634f * 0.7978845608028654f;
    constexpr float k1 = k0 * 0.044715f;
    constexpr float c2 = 2.f * 0.7978845608028654f, c6 = 6.f * 0.7978845608028654f * 0.044715f;
    const float h2 = h * h;
    const float s = __builtin_amdgcn_rcpf(exp2_fast(h * fmaf(h2, k1, k0)) + 1.f);
    c = h * s;
    d = s * fmaf(fmaf(-h, s, h), fmaf(h2, c6, c2), 1.f);  // explicit fmas: the same bits in every kernel
}

// d/dh of the above: 0.5 (1 + t) + 0.5 h (1 - t^2) u'(h), t = tanh(u) = 1 - 2 / (e + 1)
__device__ __forceinline__ float gelu_tanh_grad(float h) {
    const float u = 0.7978845608028654f * fmaf(0.044715f * h, h * h, h);
    const float e = exp2_fast(2.f * kLog2e * u);
    const float th = 1.f - 2.f * __builtin_amdgcn_rcpf(e + 1.f);
    return 0.5f * (1.f + th) +
           0.5f * h * (1.f - th * th) * 0.7978845608028654f * (1.f + 3.f * 0.044715f * h * h);
}

// ---------------------------------------------------------------------------
// Direct global -> LDS loads (global_load_lds_dwordx4, gfx950): a wave-wide load
// writes 64 consecutive 16-byte LDS slots, lane i -> slot base + i, from per-lane
// global addresses.  No registers and no LDS store instructions; complete once the
// issuing wave's vmcnt drains, visible to the other waves after the following barrier.

// 16 zero bytes in global memory (one copy per code object): the source of tile
// slots past the end of a tensor
static __device__ __attribute__((aligned(16))) uint32_t g_zero_line[4];

typedef __attribute__((address_space(3))) void lds_void;

// global_load_lds_dwordx4 to LDS slots lds + 16 * lane, from per-lane address `src`
// (dma16) or from the wave-uniform base `sbase` plus a per-lane 32-bit byte offset
// (dma16_so: no 64-bit address arithmetic per lane).  Issued as inline asm so that the
// compiler's wait-count pass does not treat every later LDS read as possibly
// depending on it (it would insert vmcnt(0) before the reads of the other stage and
// serialise the prefetch); the protocol waits for the loads itself (tile_arrive).
// vmcnt completes in order, so loads the compiler does not know about only make its
// own waits stricter.  `lds` must be wave-uniform.  M0 (the LDS base the instruction
// reads) is saved and restored inside the statement, so whatever the compiler keeps
// in it survives.
__device__ __forceinline__ void dma16(const void* src, uint32_t lds) {
    uint32_t saved;
    asm volatile(
        "s_mov_b32 %0, m0\n\t"
        "s_mov_b32 m0, %2\n\t"
        "s_nop 0\n\t"
        "global_load_lds_dwordx4 %1, off\n\t"
        "s_nop 0\n\t"
        "s_mov_b32 m0, %0"
        : "=&s"(saved)
        : "v"(src), "s"(lds)
        : "memory");
}
__device__ __forceinline__ void dma16_so(const void* sbase, uint32_t voff, uint32_t lds) {
    uint32_t saved;
    asm volatile(
        "s_mov_b32 %0, m0\n\t"
        "s_mov_b32 m0, %3\n\t"
        "s_nop 0\n\t"
        "global_load_lds_dwordx4 %1, %2\n\t"
        "s_nop 0\n\t"
        "s_mov_b32 m0, %0"
        : "=&s"(saved)
        : "v"(voff), "s"(sbase), "s"(lds)
        : "memory");
}
// Four dma16_so loads in one statement, M0 saved and restored once (one statement per load
// spends two more M0 moves per load on saving and restoring it).
__device__ __forceinline__ void dma16_so_x4(const void* b0, uint32_t o0, uint32_t l0, const void* b1, uint32_t o1,
                                            uint32_t l1, const void* b2, uint32_t o2, uint32_t l2, const void* b3,
                                            uint32_t o3, uint32_t l3) {
    uint32_t saved;
    asm volatile(
        "s_mov_b32 %0, m0\n\t"
        "s_mov_b32 m0, %3\n\t"
        "s_nop 0\n\t"
        "global_load_lds_dwordx4 %1, %2\n\t"
        "s_nop 0\n\t"
        "s_mov_b32 m0, %6\n\t"
        "s_nop 0\n\t"
        "global_load_lds_dwordx4 %4, %5\n\t"
        "s_nop 0\n\t"
        "s_mov_b32 m0, %9\n\t"
        "s_nop 0\n\t"
        "global_load_lds_dwordx4 %7, %8\n\t"
        "s_nop 0\n\t"
        "s_mov_b32 m0, %12\n\t"
        "s_nop 0\n\t"
        "global_load_lds_dwordx4 %10, %11\n\t"
        "s_nop 0\n\t"
        "s_mov_b32 m0, %0"
        : "=&s"(saved)
        : "v"(o0), "s"(b0), "s"(l0), "v"(o1), "s"(b1), "s"(l1), "v"(o2), "s"(b2), "s"(l2), "v"(o3), "s"(b3),
          "s"(l3)
        : "memory");
}
// global_load_lds_dword: 4 bytes per active lane to lds + 4 * lane (same protocol as dma16)
__device__ __forceinline__ void dma4(const void* src, uint32_t lds) {
    uint32_t saved;
    asm volatile(
        "s_mov_b32 %0, m0\n\t"
        "s_mov_b32 m0, %2\n\t"
        "s_nop 0\n\t"
        "global_load_lds_dword %1, off\n\t"
        "s_nop 0\n\t"
        "s_mov_b32 m0, %0"
        : "=&s"(saved)
        : "v"(src), "s"(lds)
        : "memory");
}
__device__ __forceinline__ uint32_t lds_addr(const void* p) {
    return (uint32_t)(uintptr_t)(lds_void*)p;
}

// Wait until at most N of this wave's vector-memory instructions (loads, stores and the
// LDS loads above, completing in issue order) are outstanding.  The memory clobber keeps
// the compiler from moving LDS reads of the awaited data above the wait.
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
    static_assert(N >= 0 && N < 64, "vmcnt is a 6-bit count");
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}
// the same for a count that is a compile-time constant only after loop unrolling
__device__ __forceinline__ void wait_vmcnt_folded(int n) {
    switch (n) {
#define FX_WC(i) case i: wait_vmcnt<i>(); break;
        FX_WC(1) FX_WC(2) FX_WC(3) FX_WC(4) FX_WC(5) FX_WC(6) FX_WC(7) FX_WC(8) FX_WC(9) FX_WC(10)
        FX_WC(11) FX_WC(12) FX_WC(13) FX_WC(14) FX_WC(15) FX_WC(16) FX_WC(17) FX_WC(18) FX_WC(19)
        FX_WC(20) FX_WC(21) FX_WC(22) FX_WC(23) FX_WC(24) FX_WC(25) FX_WC(26) FX_WC(27) FX_WC(28)
        FX_WC(29) FX_WC(30) FX_WC(31) FX_WC(32)
#undef FX_WC
        default: wait_vmcnt<0>();  // stricter than asked: always safe
    }
}

// Wait for this wave's outstanding vector-memory operations (including its tile
// loads), then barrier: afterwards every wave's loads of the tile are visible.
__device__ __forceinline__ void tile_arrive() {
    __builtin_amdgcn_s_waitcnt(0x0f70);  // vmcnt(0)
    __syncthreads();
}

}  // namespace fx
