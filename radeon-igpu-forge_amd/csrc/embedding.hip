// Token-embedding gradient for gfx950: grad[v] = the sum, in increasing t, of dy[t] over the
// positions t with idx[t] == v (fp32 accumulation, one bf16 rounding); vocabulary rows that no
// position selects are zero, and ids outside [0, V) select nothing.
//
// The reference's GPT takes this from torch's nn.Embedding backward (tok_emb(idx),
// ml/fxlm/model.py:114-117), which sorts the ids and sums segments with launch sizes it reads
// from the device.  Here every launch size follows from n and V alone, and nothing uses
// atomics, so the result is deterministic.  A stable counting sort groups the positions by id:
//   emb_rank     one 1024-thread workgroup per chunk of 1024 positions: the keys
//                (id << 10 | position in the chunk) sorted in the workgroup (bitonic), so that
//                equal ids sit together in position order; a position's rank is its distance
//                from the start of its id's run, and the run's last entry writes the chunk's
//                count of the id into the chunk's row of cnt (zeroed first by the workgroup);
//   emb_colscan  per id, the chunk counts turned into each chunk's first slot (an exclusive
//                scan down the chunks), the id's total, and the totals' exclusive scan within
//                each block of 256 ids, with the block's sum;
//   emb_offsets  per block of 256 ids, the sum of the earlier blocks added: offs[v] is the first
//                slot of id v, offs[V] the count of valid positions;
//   emb_scatter  position t to slot offs[id] + its chunk's first slot + its rank, and the id
//                of every slot into sid;
//   emb_part     one wave per segment of kEmbSeg consecutive slots, for the runs that cross
//                its edges: the run entering from the previous segment leaves the fp32 sum of
//                its rows here (in slot order, i.e. increasing t) as a "head" partial row, the
//                run continuing into the next segment a "tail" partial row;
//   emb_final    one wave per id: zeros when the id has no position; a run inside one segment
//                summed in slot order; a longer run its first segment's tail partial plus the
//                later segments' head partials, in segment order; rounded once.
// So no wave sums more than kEmbSeg rows, whatever the ids: one id holding 15 % of the
// positions (the space byte of byte-level text) is 77 segments summed side by side and one
// combine of 77 partial rows, where one wave per id would walk its 2,500 rows one by one.
#include "fx_device.h"

namespace fx {

constexpr int kEmbChunk = 1024;  // positions per emb_rank workgroup (the key keeps 10 bits of it)
constexpr int kEmbBlock = 256;   // ids per emb_colscan / emb_offsets workgroup
constexpr int kEmbSeg = 32;      // slots per emb_part wave

__global__ void __launch_bounds__(256) emb_zero_kernel(uint32_t* __restrict__ p, int64_t n) {
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) p[i] = 0u;
}

__device__ inline uint64_t emb_xor64(uint64_t x, int j) {
    const int lo = __shfl_xor((int)(uint32_t)x, j), hi = __shfl_xor((int)(uint32_t)(x >> 32), j);
    return ((uint64_t)(uint32_t)hi << 32) | (uint32_t)lo;
}

__global__ void __launch_bounds__(kEmbChunk) emb_rank_kernel(const int64_t* __restrict__ idx, int64_t n, int64_t V,
                                                            int32_t* __restrict__ cnt, int32_t* __restrict__ rank) {
    __shared__ uint64_t sk[kEmbChunk];
    __shared__ int32_t wmax[kEmbChunk / 64];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int64_t t0 = (int64_t)blockIdx.x * kEmbChunk;
    int32_t* row = cnt + (int64_t)blockIdx.x * V;
    for (int64_t i = tid; i < V; i += kEmbChunk) row[i] = 0;
    // V: an id outside [0, V) (rank -1); V + 1: past the end of the positions (nothing written)
    uint64_t v = (uint64_t)V + 1;
    if (t0 + tid < n) {
        const int64_t x = idx[t0 + tid];
        v = (x >= 0 && x < V) ? (uint64_t)x : (uint64_t)V;
    }
    uint64_t key = (v << 10) | (uint64_t)tid;
    for (int k = 2; k <= kEmbChunk; k <<= 1) {
        for (int j = k >> 1; j > 0; j >>= 1) {
            uint64_t other;
            if (j >= 64) {
                sk[tid] = key;
                __syncthreads();
                other = sk[tid ^ j];
                __syncthreads();
            } else {
                other = emb_xor64(key, j);
            }
            // ascending where (tid & k) == 0: the lower index of the pair keeps the smaller key
            const bool keep_min = ((tid & k) == 0) == ((tid & j) == 0);
            key = keep_min ? (key < other ? key : other) : (key < other ? other : key);
        }
    }
    sk[tid] = key;
    __syncthreads();  // also orders the row's zeros before the counts below
    const uint64_t vk = key >> 10;
    const bool head = tid == 0 || (sk[tid - 1] >> 10) != vk;
    const bool last = tid == kEmbChunk - 1 || (sk[tid + 1] >> 10) != vk;
    int st = head ? tid : 0;  // the run's first index: an inclusive max-scan of the heads
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
        const int y = __shfl_up(st, d);
        if (lane >= d && y > st) st = y;
    }
    if (lane == 63) wmax[wave] = st;
    __syncthreads();
    for (int w = 0; w < wave; ++w) st = wmax[w] > st ? wmax[w] : st;
    const int r = tid - st;
    const int64_t t = t0 + (int64_t)(key & (kEmbChunk - 1));
    if (vk < (uint64_t)V) {
        rank[t] = r;
        if (last) row[vk] = r + 1;
    } else if (vk == (uint64_t)V) {
        rank[t] = -1;
    }
}

// Wave-then-workgroup inclusive scan of x over a 256-thread workgroup; *tot = the sum.
__device__ inline int32_t emb_block_scan(int32_t x, int32_t* ws, int32_t* tot) {
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    int32_t inc = x;
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
        const int32_t y = __shfl_up(inc, d);
        if (lane >= d) inc += y;
    }
    if (lane == 63) ws[wave] = inc;
    __syncthreads();
    int32_t woff = 0, s = 0;
#pragma unroll
    for (int w = 0; w < kEmbBlock / 64; ++w) {
        const int32_t y = ws[w];
        if (w < wave) woff += y;
        s += y;
    }
    *tot = s;
    return woff + inc;
}

__global__ void __launch_bounds__(kEmbBlock) emb_colscan_kernel(int32_t* __restrict__ cnt, int nch, int64_t V,
                                                               int32_t* __restrict__ offs, int32_t* __restrict__ bsum) {
    __shared__ int32_t ws[kEmbBlock / 64];
    const int64_t v = (int64_t)blockIdx.x * kEmbBlock + threadIdx.x;
    int32_t run = 0;
    if (v < V) {
        for (int c0 = 0; c0 < nch; c0 += 8) {  // eight loads in flight, then their stores
            int32_t x[8];
#pragma unroll
            for (int k = 0; k < 8; ++k) x[k] = c0 + k < nch ? cnt[(int64_t)(c0 + k) * V + v] : 0;
#pragma unroll
            for (int k = 0; k < 8; ++k) {
                if (c0 + k < nch) cnt[(int64_t)(c0 + k) * V + v] = run;
                run += x[k];
            }
        }
    }
    int32_t tot;
    const int32_t inc = emb_block_scan(run, ws, &tot);
    if (v < V) offs[v] = inc - run;
    if (threadIdx.x == 0) bsum[blockIdx.x] = tot;
}

__global__ void __launch_bounds__(kEmbBlock) emb_offsets_kernel(int32_t* __restrict__ offs,
                                                               const int32_t* __restrict__ bsum, int64_t V) {
    __shared__ int32_t ws[kEmbBlock / 64];
    const int64_t b = blockIdx.x;
    int32_t s = 0;
    for (int64_t i = threadIdx.x; i < b; i += kEmbBlock) s += bsum[i];
    int32_t pre;
    emb_block_scan(s, ws, &pre);
    const int64_t v = b * kEmbBlock + threadIdx.x;
    if (v < V) offs[v] += pre;
    if (b == (int64_t)gridDim.x - 1 && threadIdx.x == 0) offs[V] = pre + bsum[b];
}

__global__ void __launch_bounds__(256) emb_scatter_kernel(const int64_t* __restrict__ idx, int64_t n, int64_t V,
                                                         const int32_t* __restrict__ cnt,
                                                         const int32_t* __restrict__ offs,
                                                         const int32_t* __restrict__ rank, int32_t* __restrict__ order,
                                                         int32_t* __restrict__ sid) {
    const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= n) return;
    const int32_t r = rank[t];
    if (r < 0) return;
    const int64_t v = idx[t];
    const int64_t pos = (int64_t)offs[v] + cnt[(t / kEmbChunk) * V + v] + r;
    if (pos >= 0 && pos < n) {
        order[pos] = (int32_t)t;
        sid[pos] = (int32_t)v;
    }
}

// acc (this lane's 16-byte vector ch of a row, 8 fp32) += the rows of slots b .. e - 1 in slot
// order; `tl` holds slot j's position in lane j (0 <= b < e <= 64).  Batches of 8 rows: a batch's
// loads are issued before its adds.
__device__ __forceinline__ void emb_sum_slots(float (&acc)[8], const uint16_t* __restrict__ dy, int64_t ldy,
                                              int32_t tl, int b, int e, int64_t ch) {
    for (int q = b; q < e; q += 8) {
        uint4 r[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            const int32_t t = __builtin_amdgcn_readlane(tl, q + u < e ? q + u : q);
            if (q + u < e) r[u] = ld16(dy + (int64_t)t * ldy + 8 * ch);
        }
#pragma unroll
        for (int u = 0; u < 8; ++u)
            if (q + u < e) {
                float f[8];
                unpack8(r[u], f);
#pragma unroll
                for (int k = 0; k < 8; ++k) acc[k] += f[k];
            }
    }
}

// One wave per segment c of kEmbSeg slots: the partial sums of the (at most two) runs that
// cross the segment's edges.  The first run, if its id also holds slot s0 - 1, leaves its rows'
// sum in head row 2c; the last run, if its id also holds slot s0 + kEmbSeg and it did not start
// before s0, leaves its sum in tail row 2c + 1.  Runs inside the segment are emb_final's.
__global__ void __launch_bounds__(256) emb_part_kernel(const uint16_t* __restrict__ dy, int64_t ldy,
                                                      const int32_t* __restrict__ order,
                                                      const int32_t* __restrict__ sid,
                                                      const int32_t* __restrict__ offs, int64_t n, int64_t nseg,
                                                      float* __restrict__ part, int64_t V, int64_t D) {
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int64_t c = (int64_t)blockIdx.x * 4 + wave;
    if (c >= nseg) return;
    const int64_t s0 = c * kEmbSeg;
    int64_t nvalid = offs[V];
    if (nvalid > n) nvalid = n;
    const int ns = (int)(nvalid - s0 < kEmbSeg ? nvalid - s0 : kEmbSeg);  // slots of this segment
    if (ns <= 0) return;
    // lane u < ns: slot s0 + u's position and id; lane ns: the id of the slot after the segment
    // (-1 past the last); lane 63: the id of the slot before it (-1 for the first segment)
    int32_t tl = 0, vl = -1;
    if (lane < ns) {
        tl = order[s0 + lane];
        vl = sid[s0 + lane];
    } else if (lane == ns && s0 + ns < nvalid) {
        vl = sid[s0 + ns];
    } else if (lane == 63 && s0 > 0) {
        vl = sid[s0 - 1];
    }
    const int v0 = __builtin_amdgcn_readlane(vl, 0), vlast = __builtin_amdgcn_readlane(vl, ns - 1);
    const bool head = s0 > 0 && __builtin_amdgcn_readlane(vl, 63) == v0;
    const bool tail = __builtin_amdgcn_readlane(vl, ns) == vlast && !(head && vlast == v0);
    if (!head && !tail) return;
    int e0 = 1;  // the first run: slots 0 .. e0 - 1
    while (e0 < ns && __builtin_amdgcn_readlane(vl, e0) == v0) ++e0;
    int b1 = ns - 1;  // the last run: slots b1 .. ns - 1
    while (b1 > 0 && __builtin_amdgcn_readlane(vl, b1 - 1) == vlast) --b1;
    for (int64_t ch = lane; ch < D / 8; ch += 64) {
        if (head) {
            float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
            emb_sum_slots(acc, dy, ldy, tl, 0, e0, ch);
            float4* o = reinterpret_cast<float4*>(part + 2 * c * D + 8 * ch);
            o[0] = make_float4(acc[0], acc[1], acc[2], acc[3]);
            o[1] = make_float4(acc[4], acc[5], acc[6], acc[7]);
        }
        if (tail) {
            float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
            emb_sum_slots(acc, dy, ldy, tl, b1, ns, ch);
            float4* o = reinterpret_cast<float4*>(part + (2 * c + 1) * D + 8 * ch);
            o[0] = make_float4(acc[0], acc[1], acc[2], acc[3]);
            o[1] = make_float4(acc[4], acc[5], acc[6], acc[7]);
        }
    }
}

// One wave per id v, run = slots offs[v] .. offs[v + 1] - 1: zeros when empty; a run inside one
// segment summed here in slot order (at most kEmbSeg rows); a longer one is its first segment's
// tail partial plus the later segments' head partials, in segment order.  One bf16 rounding.
__global__ void __launch_bounds__(256) emb_final_kernel(const uint16_t* __restrict__ dy, int64_t ldy,
                                                       const int32_t* __restrict__ order,
                                                       const int32_t* __restrict__ offs, int64_t n,
                                                       const float* __restrict__ part, uint16_t* __restrict__ grad,
                                                       int64_t V, int64_t D) {
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int64_t v = (int64_t)blockIdx.x * 4 + wave;
    if (v >= V) return;
    int64_t beg = offs[v], end = offs[v + 1];
    if (beg < 0) beg = 0;
    if (end > n) end = n;
    uint16_t* out = grad + v * D;
    if (end <= beg) {  // no position has this id
        for (int64_t ch = lane; ch < D / 8; ch += 64) st16(out + 8 * ch, make_uint4(0u, 0u, 0u, 0u));
        return;
    }
    const int64_t c0 = beg / kEmbSeg, c1 = (end - 1) / kEmbSeg;
    if (c0 == c1) {  // inside one segment: at most kEmbSeg rows
        const int len = (int)(end - beg);
        const int32_t tl = lane < len ? order[beg + lane] : 0;
        for (int64_t ch = lane; ch < D / 8; ch += 64) {
            float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
            emb_sum_slots(acc, dy, ldy, tl, 0, len, ch);
            st16(out + 8 * ch, pack8(acc));
        }
        return;
    }
    for (int64_t ch = lane; ch < D / 8; ch += 64) {
        const float4* t0 = reinterpret_cast<const float4*>(part + (2 * c0 + 1) * D + 8 * ch);
        float acc[8];
        {
            const float4 a = t0[0], b = t0[1];
            acc[0] = a.x; acc[1] = a.y; acc[2] = a.z; acc[3] = a.w;
            acc[4] = b.x; acc[5] = b.y; acc[6] = b.z; acc[7] = b.w;
        }
        for (int64_t c = c0 + 1; c <= c1; c += 8) {
            float4 h[8][2];
#pragma unroll
            for (int u = 0; u < 8; ++u)
                if (c + u <= c1) {
                    const float4* p = reinterpret_cast<const float4*>(part + 2 * (c + u) * D + 8 * ch);
                    h[u][0] = p[0];
                    h[u][1] = p[1];
                }
#pragma unroll
            for (int u = 0; u < 8; ++u)
                if (c + u <= c1) {
                    acc[0] += h[u][0].x; acc[1] += h[u][0].y; acc[2] += h[u][0].z; acc[3] += h[u][0].w;
                    acc[4] += h[u][1].x; acc[5] += h[u][1].y; acc[6] += h[u][1].z; acc[7] += h[u][1].w;
                }
        }
        st16(out + 8 * ch, pack8(acc));
    }
}

static int64_t emb_align16(int64_t b) { return (b + 15) / 16 * 16; }

}  // namespace fx

using namespace fx;

extern "C" int64_t fx_embedding_bwd_workspace(int64_t n, int64_t V, int64_t D) {
    if (n <= 0 || V <= 0 || D <= 0) return 0;
    const int64_t nch = (n + kEmbChunk - 1) / kEmbChunk, nb = (V + kEmbBlock - 1) / kEmbBlock;
    const int64_t nseg = (n + kEmbSeg - 1) / kEmbSeg;
    return emb_align16(nch * V * 4) + emb_align16((V + 1) * 4) + emb_align16(nb * 4) + 3 * emb_align16(n * 4) +
           emb_align16(2 * nseg * D * 4);
}

extern "C" int fx_embedding_bwd(const int64_t* idx, int64_t n, const uint16_t* dy, int64_t ldy, uint16_t* grad,
                                int64_t V, int64_t D, void* work, void* stream) {
    FX_REQUIRE(V >= 1 && V < ((int64_t)1 << 31) - 1, "fx_embedding_bwd: bad vocabulary size V=%lld", (long long)V);
    FX_REQUIRE(D >= 8 && D % 8 == 0 && D < ((int64_t)1 << 24),
               "fx_embedding_bwd: D=%lld must be a positive multiple of 8", (long long)D);
    FX_REQUIRE(n >= 0 && n < ((int64_t)1 << 31) - kEmbChunk, "fx_embedding_bwd: bad position count n=%lld",
               (long long)n);
    FX_REQUIRE(grad != nullptr && ((uintptr_t)grad & 15) == 0, "fx_embedding_bwd: grad must be 16-byte aligned");
    FX_REQUIRE(n == 0 || (idx && dy && work), "fx_embedding_bwd: null pointer");
    FX_REQUIRE(n == 0 || (ldy >= D && ldy % 8 == 0 && ((uintptr_t)dy & 15) == 0 && ((uintptr_t)work & 15) == 0),
               "fx_embedding_bwd: dy rows and work must be 16-byte aligned (ldy=%lld)", (long long)ldy);
    FX_REQUIRE(((uintptr_t)idx & 7) == 0, "fx_embedding_bwd: idx must be 8-byte aligned");
    hipStream_t s = (hipStream_t)stream;
    if (n == 0) {  // every row zero
        const int64_t words = V * D / 2;
        hipLaunchKernelGGL(emb_zero_kernel, dim3((unsigned)(words < 4096 * 256 ? (words + 255) / 256 : 4096)), dim3(256),
                           0, s, reinterpret_cast<uint32_t*>(grad), words);
        return check_launch("emb_zero");
    }
    const int64_t nch = (n + kEmbChunk - 1) / kEmbChunk, nb = (V + kEmbBlock - 1) / kEmbBlock;
    char* w = static_cast<char*>(work);
    int32_t* cnt = reinterpret_cast<int32_t*>(w);
    w += emb_align16(nch * V * 4);
    int32_t* offs = reinterpret_cast<int32_t*>(w);
    w += emb_align16((V + 1) * 4);
    int32_t* bsum = reinterpret_cast<int32_t*>(w);
    w += emb_align16(nb * 4);
    int32_t* rank = reinterpret_cast<int32_t*>(w);
    w += emb_align16(n * 4);
    int32_t* order = reinterpret_cast<int32_t*>(w);
    w += emb_align16(n * 4);
    int32_t* sid = reinterpret_cast<int32_t*>(w);
    w += emb_align16(n * 4);
    float* part = reinterpret_cast<float*>(w);  // per segment: head row, then tail row
    const int64_t nseg = (n + kEmbSeg - 1) / kEmbSeg;
    hipLaunchKernelGGL(emb_rank_kernel, dim3((unsigned)nch), dim3(kEmbChunk), 0, s, idx, n, V, cnt, rank);
    if (int e = check_launch("emb_rank")) return e;
    hipLaunchKernelGGL(emb_colscan_kernel, dim3((unsigned)nb), dim3(kEmbBlock), 0, s, cnt, (int)nch, V, offs, bsum);
    if (int e = check_launch("emb_colscan")) return e;
    hipLaunchKernelGGL(emb_offsets_kernel, dim3((unsigned)nb), dim3(kEmbBlock), 0, s, offs, bsum, V);
    if (int e = check_launch("emb_offsets")) return e;
    hipLaunchKernelGGL(emb_scatter_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, idx, n, V, cnt, offs,
                       rank, order, sid);
    if (int e = check_launch("emb_scatter")) return e;
    hipLaunchKernelGGL(emb_part_kernel, dim3((unsigned)((nseg + 3) / 4)), dim3(256), 0, s, dy, ldy, order, sid, offs, n,
                       nseg, part, V, D);
    if (int e = check_launch("emb_part")) return e;
    hipLaunchKernelGGL(emb_final_kernel, dim3((unsigned)((V + 3) / 4)), dim3(256), 0, s, dy, ldy, order, offs, n, part,
                       grad, V, D);
    return check_launch("emb_final");
}
