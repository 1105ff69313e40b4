// vq2_sorted.hpp -- device pieces shared by the kernels over the code-sorted
// layout (vq2_sorted.hip: dense matrices; vq2_sorted_moe.hip: expert pools).
//
// Layout recap (built by vq2_sorted_pack / vq2_sorted_pack_pool): a matrix
// is cut into chunks of R rows; every code of a chunk is one uint32 entry
// (code << 16) | (row << gbits) | group, sorted by code and dealt into
// 64-entry instructions with no row twice in a 32-lane half; 4 instructions
// form a 1 KiB iteration, lane l reading the 16-byte word l of it; padding
// entries add code 0 into the dummy row R.
#pragma once

#include "vq2_gemv_kernel.hpp"

namespace vq2 {

constexpr int SG_THREADS = 1024;
constexpr int SG_WAVES = SG_THREADS / 64;
constexpr int SG_ITER = 256;  // entries per iteration (64 lanes x 4)
constexpr int SG_MAX_R = 255;
constexpr int SG_PARTS = 2;                   // accumulator arrays per wave
constexpr int SG_PART_LANES = 64 / SG_PARTS;  // lanes sharing one array
constexpr int SG_MAX_SHM = 96 * 1024;         // dynamic LDS: activation (+ stage) + accumulators

inline int sorted_gbits(int64_t ng)
{
    int b = 0;
    while ((int64_t(1) << b) < ng) b++;
    return b;
}

// Rows are cut into ceil(rows / R) chunks of as equal a height as possible:
// the first rows % chunks chunks hold rows / chunks + 1 rows, the others
// rows / chunks, so no chunk is much shorter than the rest (all chunks are
// padded to one iteration count, and padding is not free).  Chunk c starts
// at row c * rb + min(c, nbig) and holds rb + (c < nbig) rows.
struct ChunkSplit {
    int64_t n_chunks, rb, nbig;
};
__host__ __device__ inline ChunkSplit chunk_split(int64_t rows, int64_t R)
{
    ChunkSplit k;
    k.n_chunks = (rows + R - 1) / R;
    k.rb = k.n_chunks > 0 ? rows / k.n_chunks : 0;
    k.nbig = k.n_chunks > 0 ? rows % k.n_chunks : 0;
    return k;
}

// Largest chunk height for ng groups: row R is the dummy row, so
// (R << gbits) | group must fit 16 bits; at most SG_MAX_R.
inline int64_t sorted_max_rows(int64_t ng)
{
    const int gb = sorted_gbits(ng);
    if (ng < 1 || gb > 15) return 0;
    const int64_t rmax = (int64_t(1) << (16 - gb)) - 1;
    return rmax < SG_MAX_R ? rmax : SG_MAX_R;
}

// The activation in LDS as the loop reads it (fp32, "split" layout): the
// first 4 values of group g at float offset 4 g, the last 4 at SG_XB + 4 g.
// A 16-byte stride puts the reads of random groups at 16 bank positions
// (g mod 16) instead of the 8 of a 32-byte stride (g mod 8), so the lanes
// the LDS serves together collide less, and both halves come from one
// address register with an immediate offset.  Needs n <= 2 SG_XB.
constexpr int SG_XB = 4096;
constexpr int SG_X_SPLIT = 2 * SG_XB;  // floats of the split activation

__device__ __forceinline__ void x_store_group(float* s_split, int64_t g, const float (&v)[8])
{
    u32x4 w0, w1;
#pragma unroll
    for (int k = 0; k < 4; k++) {
        w0[k] = __float_as_uint(v[k]);
        w1[k] = __float_as_uint(v[4 + k]);
    }
    *(u32x4*)(s_split + 4 * g) = w0;
    *(u32x4*)(s_split + SG_XB + 4 * g) = w1;
}

// s_split = s_nat (the rotated activation in natural order, fp32, visible
// after a barrier) times `scale`, one thread per group.  The two regions
// must not overlap; a barrier must follow.
__device__ __forceinline__ void x_finalize(const float* s_nat, float* s_split, int64_t n, float scale)
{
    for (int64_t g = threadIdx.x; g < n / 8; g += blockDim.x) {
        const u32x4 a = *(const u32x4*)(s_nat + g * 8), b = *(const u32x4*)(s_nat + g * 8 + 4);
        float v[8];
#pragma unroll
        for (int k = 0; k < 4; k++) {
            v[k] = __uint_as_float(a[k]) * scale;
            v[4 + k] = __uint_as_float(b[k]) * scale;
        }
        x_store_group(s_split, g, v);
    }
}

// 8-term dot product of one centroid (fp16 or bf16, 16 bytes) with group g
// of the split activation in LDS, fp32.
template <int CBT>
__device__ __forceinline__ float centroid_dot(const u32x4 c, const float* s_x, uint32_t g)
{
    const float* p = s_x + 4 * g;
    const u32x4 x0 = *(const u32x4*)p, x1 = *(const u32x4*)(p + SG_XB);
    float xv[8];
#pragma unroll
    for (int k = 0; k < 4; k++) {
        xv[k] = __uint_as_float(x0[k]);
        xv[4 + k] = __uint_as_float(x1[k]);
    }
    float d = 0.0f;
#pragma unroll
    for (int w = 0; w < 4; w++) {
        float lo, hi;
        if constexpr (CBT == VQ2_DT_F16) {
            lo = f16_bits_to_f32((uint16_t)(c[w] & 0xFFFFu));
            hi = f16_bits_to_f32((uint16_t)(c[w] >> 16));
        } else {
            lo = __uint_as_float(c[w] << 16);
            hi = __uint_as_float(c[w] & 0xFFFF0000u);
        }
        d = fmaf(lo, xv[2 * w], d);
        d = fmaf(hi, xv[2 * w + 1], d);
    }
    return d;
}

// One wave's pass over iterations [s0, s1) of a chunk (stride SG_WAVES,
// starting at s0 + wave), stage-2 entries from c_mid on.  load_entries()
// issues the first three iterations' entry words and gathers() the first
// GD iterations' centroid gathers (clamped in-bounds addresses when the wave
// has fewer), so a caller can put a prologue between them, or before both.
// run() keeps entry words three iterations ahead and gathers GD ahead of
// the arithmetic (GD 2: about 8K codes in flight per CU at 16 waves, 64
// VGPRs of entry words and centroids; GD 1 saves 16 of them, for kernels
// held to 64 VGPRs that share the CU with a second workgroup).  Loads
// complete in issue order and no branch separates them, so each wait covers
// exactly the values it needs.
template <int CBT, int GD = 2>
struct SortedPipe {
    static_assert(GD == 1 || GD == 2, "gather depth 1 or 2");
    const u32x4* ent;
    const u32x4* cb0;
    const u32x4* cb1;
    int c_beg, c_mid, s1, lane;
    int it, i2;
    u32x4 e0, e1, e2;
    u32x4 c0[4], c1[4];

    __device__ __forceinline__ int clampit(int i) const { return i < s1 ? i : c_beg; }
    __device__ __forceinline__ u32x4 load_e(int i) const
    {
        return __builtin_nontemporal_load(ent + (int64_t)i * 64 + lane);
    }
    __device__ __forceinline__ void gather(int i, const u32x4& e, u32x4 (&c)[4]) const
    {
        const u32x4* cb = i < c_mid ? cb0 : cb1;
#pragma unroll
        for (int q = 0; q < 4; q++) c[q] = cb[e[q] >> 16];
    }
    // a missing stage-2 codebook is never selected for a real entry; cb0
    // stands in so that no gather can use a null base
    __device__ __forceinline__ void load_entries(const u32x4* ent_, const void* cb0_, const void* cb1_, int c_beg_,
                                                 int c_mid_, int s0, int s1_, int wave, int lane_)
    {
        ent = ent_;
        cb0 = (const u32x4*)cb0_;
        cb1 = (const u32x4*)(cb1_ ? cb1_ : cb0_);
        c_beg = c_beg_;
        c_mid = c_mid_;
        s1 = s1_;
        lane = lane_;
        it = s0 + wave;
        i2 = clampit(it + 2 * SG_WAVES);
        e0 = load_e(clampit(it));
        e1 = load_e(clampit(it + SG_WAVES));
        e2 = load_e(i2);
    }
    __device__ __forceinline__ void gathers()
    {
        gather(clampit(it), e0, c0);
        if constexpr (GD == 2) gather(clampit(it + SG_WAVES), e1, c1);
    }
    __device__ __forceinline__ void start(const u32x4* ent_, const void* cb0_, const void* cb1_, int c_beg_,
                                          int c_mid_, int s0, int s1_, int wave, int lane_)
    {
        load_entries(ent_, cb0_, cb1_, c_beg_, c_mid_, s0, s1_, wave, lane_);
        gathers();
    }
    // acc: this lane's accumulator array (R + 1 floats), x: the activation
    __device__ __forceinline__ void run(float* acc, const float* x, int gbits, int64_t ng, int R)
    {
        const uint32_t gmask = (1u << gbits) - 1u;
        const uint32_t gmax = (uint32_t)(ng - 1);
        for (; it < s1; it += SG_WAVES) {
            const int i3 = clampit(it + 3 * SG_WAVES);
            const u32x4 e3 = load_e(i3);
            u32x4 cn[4];  // the gathers GD iterations ahead
            if constexpr (GD == 2) gather(i2, e2, cn);
            else gather(clampit(it + SG_WAVES), e1, cn);
#pragma unroll
            for (int q = 0; q < 4; q++) {
                const uint32_t pos = e0[q] & 0xFFFFu;
                const uint32_t r = min(pos >> gbits, (uint32_t)R);
                const uint32_t g = min(pos & gmask, gmax);
                const float d = centroid_dot<CBT>(c0[q], x, g);
                acc[r] += d;
            }
            e0 = e1;
            e1 = e2;
            e2 = e3;
            i2 = i3;
#pragma unroll
            for (int q = 0; q < 4; q++) {
                if constexpr (GD == 2) {
                    c0[q] = c1[q];
                    c1[q] = cn[q];
                } else {
                    c0[q] = cn[q];
                }
            }
        }
    }
};

// This lane's accumulator array: 2 per wave, one per 32-lane half.
__device__ __forceinline__ float* sorted_acc(float* s_acc, int wave, int lane, int R)
{
    return s_acc + (wave * SG_PARTS + lane / SG_PART_LANES) * (R + 1);
}

__device__ __forceinline__ void sorted_acc_zero(float* acc, int lane, int R)
{
    for (int i = lane % SG_PART_LANES; i <= R; i += SG_PART_LANES) acc[i] = 0.0f;
}

// Row sums of the SG_WAVES x SG_PARTS accumulator arrays (after a barrier):
// thread (p, r) adds a quarter of the arrays of row r, then the four
// partials are added in p order (a fixed order: deterministic).  The result
// is meaningful for threads with threadIdx.x < R (row threadIdx.x); ends with
// a barrier-free read, after the barrier between the two halves.
__device__ __forceinline__ float sorted_row_sums(const float* s_acc, int R, float (*s_red)[256])
{
    const int rr = threadIdx.x & 255, pp = threadIdx.x >> 8;
    if (rr < R) {
        float part = 0.0f;
        constexpr int NA = SG_WAVES * SG_PARTS / 4;
#pragma unroll 4
        for (int w = NA * pp; w < NA * pp + NA; w++) part += s_acc[w * (R + 1) + rr];
        s_red[pp][rr] = part;
    }
    __syncthreads();
    return (pp == 0 && rr < R) ? ((s_red[0][rr] + s_red[1][rr]) + s_red[2][rr]) + s_red[3][rr] : 0.0f;
}

}  // namespace vq2
