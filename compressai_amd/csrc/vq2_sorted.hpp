// vq2_sorted.hpp -- device pieces shared by the kernels over the code-sorted
// layout (vq2_sorted.hip: dense matrices; vq2_sorted_batch.hip: batch 2-4;
// vq2_sorted_moe.hip: expert pools).
//
// Layout recap (built by vq2_sorted_pack / vq2_sorted_pack_pool): a matrix
// is cut into chunks of R rows; the codes of a chunk are sorted by value and
// dealt into 64-lane instructions with no row twice in a 32-lane half.
// Lane 63 of an instruction holds no code: it carries the instruction's base
// code (its smallest).  Every other lane holds a 24-bit field
//     F = (code - base) << P | row << gbits | group,   P = gbits + bitlen(R),
// so P <= 17 and the code offset has 24 - P >= 7 bits (the packer closes an
// instruction early rather than exceed it; P = 17 only for the taller
// chunks of very tall matrices, sorted_rows_per_chunk).  Four instructions form an
// iteration of 768 bytes: lane l reads the 12 bytes at 12 l, three words
//     w0 = lo16(F0) | lo16(F1) << 16,  w1 = lo16(F2) | lo16(F3) << 16,
//     w2 = hi8(F0) | hi8(F1) << 8 | hi8(F2) << 16 | hi8(F3) << 24,
// and lane 63's w0 / w1 are the four base codes in the same places (w2 = 0).
// Padding fields add code `base` into the dummy row R (group 0).  3 bytes
// per code against 2 in the reference planes (4 in the first version of
// this format, which stored every code in full).
#pragma once

#include "vq2_gemv_kernel.hpp"

namespace vq2 {

constexpr int SG_THREADS = 1024;
constexpr int SG_WAVES = SG_THREADS / 64;
constexpr int SG_ITER = 256;        // entry slots per iteration (64 lanes x 4 instructions)
constexpr int SG_LANE_WORDS = 3;    // uint32 words per lane and iteration
constexpr int SG_ITER_WORDS = 64 * SG_LANE_WORDS;  // 768 bytes per iteration
constexpr int SG_BASE_LANE = 63;    // the lane that carries the instructions' base codes
constexpr int SG_MAX_R = 511;
constexpr int SG_PARTS = 2;                   // accumulator arrays per wave
constexpr int SG_PART_LANES = 64 / SG_PARTS;  // lanes sharing one array
// Dense matrices packed in chunks of at most SG_QUAD_R rows take four
// arrays per wave (16 lanes each): a 32-lane half can hold only R distinct
// rows, so their instructions would run partly empty (2048 x 2048 in
// 16-row chunks: 41 iterations per chunk with two arrays, 22 with four; 32
// rows: 51 and 33).  Taller chunks keep two (their halves fill; four would
// double the accumulators' LDS), and so do expert pools.
constexpr int SG_QUAD_R = 32;
constexpr int SG_MAX_PARTS = 4;
__host__ __device__ constexpr int sorted_parts(int64_t R) { return R <= SG_QUAD_R ? SG_MAX_PARTS : SG_PARTS; }
constexpr int SG_MAX_SHM = 150 * 1024;        // dynamic LDS: activation (+ stage) + accumulators
constexpr int SG_MAX_SEG = 4;                 // matrices per launch

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

// Bits of a field's position part: gbits + bitlen(R) (rows 0..R, R the
// dummy row); at most 17 when R <= sorted_max_rows(ng).
__host__ __device__ inline int sorted_pbits(int gbits, int R)
{
    return gbits + (32 - __builtin_clz((unsigned)R));
}

// Largest chunk height for ng groups: row R is the dummy row, so
// (R << gbits) | group must fit `pbits` bits (17: what a field holds with a
// 7-bit code offset; 16: the default chunking's limit); at most SG_MAX_R.
inline int64_t sorted_max_rows(int64_t ng, int pbits = 17)
{
    const int gb = sorted_gbits(ng);
    if (ng < 1 || gb > 15) return 0;
    const int64_t rmax = (int64_t(1) << (pbits - gb)) - 1;
    return rmax < SG_MAX_R ? rmax : SG_MAX_R;
}

// The activation in LDS as the loop reads it (fp32, "split" layout): the
// first 4 values of group g at float offset 4 g, the last 4 at xb + 4 g.
// A 16-byte stride puts the reads of random groups at 16 bank positions
// (g mod 16) instead of the 8 of a 32-byte stride (g mod 8), so the lanes
// the LDS serves together collide less.  The dense kernels take xb = n / 2
// (the layout fills n floats: the LM head's workgroups stay small enough for
// two per CU); the MoE kernels the fixed SG_XB (n <= 2 SG_XB).
constexpr int SG_XB = 4096;
constexpr int SG_X_SPLIT = 2 * SG_XB;  // floats of the split activation at xb = SG_XB

__device__ __forceinline__ void x_store_group(float* s_split, int64_t g, const float (&v)[8], int xb)
{
    u32x4 w0, w1;
#pragma unroll
    for (int k = 0; k < 4; k++) {
        w0[k] = __float_as_uint(v[k]);
        w1[k] = __float_as_uint(v[4 + k]);
    }
    *(u32x4*)(s_split + 4 * g) = w0;
    *(u32x4*)(s_split + xb + 4 * g) = w1;
}

// s_split = s_nat (the rotated activation in natural order, fp32, visible
// after a barrier) times `scale`, one thread per group.  The two regions
// must not overlap; a barrier must follow.
__device__ __forceinline__ void x_finalize(const float* s_nat, float* s_split, int64_t n, float scale, int xb)
{
    for (int64_t g = threadIdx.x; g < n / 8; g += blockDim.x) {
        const u32x4 a = *(const u32x4*)(s_nat + g * 8), b = *(const u32x4*)(s_nat + g * 8 + 4);
        float v[8];
#pragma unroll
        for (int k = 0; k < 4; k++) {
            v[k] = __uint_as_float(a[k]) * scale;
            v[4 + k] = __uint_as_float(b[k]) * scale;
        }
        x_store_group(s_split, g, v, xb);
    }
}

// ---- RHT of one activation row in 2048-point blocks, by all 1024 threads
// (n = k * 2048, 1 <= k <= 4, hb = 2048): y = FWHT_2048(sign * x[perm]) per
// block, times `scale`, into the split layout.  The prologue of the gather
// kernels (stage_x / build_x: 8 consecutive values per thread) keeps only
// n / 8 threads busy, a quarter of the workgroup at n = 2048, and runs
// latency-bound on one wave per SIMD; here every thread holds, for each
// block b, the two values b * 2048 + 2 t + j (j = 0, 1), so value bit 0 is
// j, bits 1-6 the lane and bits 7-10 the wave, and four waves per SIMD
// share the work:
//   bit 0 in registers; bits 1-6 across lanes (DPP quad permutes for lane
//   ^ 1 and ^ 2, row shifts for ^ 4, row rotate for ^ 8, ds_swizzle for
//   ^ 16, ds_bpermute for ^ 32); bits 7-8 and 9-10 as two radix-4 passes
//   through LDS, the second one scaling and storing the split layout.
// The stages and their operands are those of the blockwise Walsh-Hadamard
// transform (stages commute; rounding differs from other stage orders only
// at fp32 accumulation level).  A permutation entry outside [0, n) poisons
// its value with NaN, as the gather kernels' prologue does.
constexpr int RHT2K = 2048;
constexpr int RHT2K_MAXB = 4;

struct Rht2kLoad {
    u32x2 p[RHT2K_MAXB];     // the two permutation entries of each block
    uint32_t s[RHT2K_MAXB];  // the two sign bytes (low 16 bits)
    u32x2 x[RHT2K_MAXB];     // the two raw activation values (fp32: two words; fp16 / bf16: both in x[b][0])
};

// Loads of the thread's values, issued early (nothing waits for them here).
template <int XT>
__device__ __forceinline__ void rht2k_load(const void* x, const int32_t* perm, const int8_t* sign, int k, int64_t xrow,
                                           Rht2kLoad& L)
{
    typedef const __attribute__((address_space(1))) u32x2* gp2;
    typedef const __attribute__((address_space(1))) uint16_t* gp16;
    typedef const __attribute__((address_space(1))) uint32_t* gp32;
#pragma unroll
    for (int b = 0; b < RHT2K_MAXB; b++) {
        if (b < k) {
            const int64_t e = (int64_t)b * RHT2K + 2 * threadIdx.x;
            L.p[b] = *(gp2)(perm ? perm + e : g_perm_iota.v + e);
            L.s[b] = *(gp16)(sign ? sign + e : g_sign_ones.v + e);
            if constexpr (XT == VQ2_DT_F32) L.x[b] = *(gp2)((const float*)x + xrow + e);
            else L.x[b][0] = *(gp32)((const uint16_t*)x + xrow + e);
        }
    }
}
template <int XT>
__device__ __forceinline__ void rht2k_load(const GemvArgs& a, int k, int64_t xrow, Rht2kLoad& L)
{
    rht2k_load<XT>(a.x, a.perm, a.sign, k, xrow, L);
}

template <int M>
__device__ __forceinline__ float lane_xor(float v, int lane)
{
    const int vi = __float_as_int(v);
    if constexpr (M == 1) return __int_as_float(__builtin_amdgcn_mov_dpp(vi, 0xB1, 0xF, 0xF, true));  // quad_perm [1,0,3,2]
    else if constexpr (M == 2) return __int_as_float(__builtin_amdgcn_mov_dpp(vi, 0x4E, 0xF, 0xF, true));  // quad_perm [2,3,0,1]
    else if constexpr (M == 4) {
        const int up = __builtin_amdgcn_mov_dpp(vi, 0x104, 0xF, 0xF, true);  // row_shl:4 (lane + 4)
        const int dn = __builtin_amdgcn_mov_dpp(vi, 0x114, 0xF, 0xF, true);  // row_shr:4 (lane - 4)
        return __int_as_float((lane & 4) ? dn : up);
    } else if constexpr (M == 8) return __int_as_float(__builtin_amdgcn_mov_dpp(vi, 0x128, 0xF, 0xF, true));  // row_ror:8
    else if constexpr (M == 16) return __int_as_float(__builtin_amdgcn_ds_swizzle(vi, 0x401F));  // lane ^ 16 within 32
    else return __int_as_float(__builtin_amdgcn_ds_bpermute((lane ^ 32) << 2, vi));
}

// One butterfly stage across lanes: v' = p + v on the lane whose bit M is
// clear, p - v on its partner (p: the partner's value), written as
// p + (v with its sign flipped on the upper lane) -- the same sums, and the
// single-row DPP moves then fold into the adds (v_add_f32 with a DPP source).
template <int M>
__device__ __forceinline__ void lane_stage(float& v0, float& v1, int lane)
{
    const uint32_t flip = (uint32_t)(lane & M) << (31 - __builtin_ctz(M));
    const float t0 = __uint_as_float(__float_as_uint(v0) ^ flip);
    const float t1 = __uint_as_float(__float_as_uint(v1) ^ flip);
    if constexpr (M == 4) {
        // lane ^ 4 as two row shifts into one register: lane + 4 written
        // into banks 0 and 2 of each row (lanes with bit 2 clear), lane - 4
        // into banks 1 and 3
        auto x4 = [](float v) {
            const int vi = __float_as_int(v);
            const int lo = __builtin_amdgcn_update_dpp(vi, vi, 0x104, 0xF, 0x5, false);  // row_shl:4
            return __int_as_float(__builtin_amdgcn_update_dpp(lo, vi, 0x114, 0xF, 0xA, false));  // row_shr:4
        };
        v0 = x4(v0) + t0;
        v1 = x4(v1) + t1;
    } else {
        v0 = lane_xor<M>(v0, lane) + t0;
        v1 = lane_xor<M>(v1, lane) + t1;
    }
}

__device__ __forceinline__ void radix4(float (&v)[4])
{
    const float a = v[0] + v[1], b = v[0] - v[1], c = v[2] + v[3], d = v[2] - v[3];
    v[0] = a + c;
    v[1] = b + d;
    v[2] = a - c;
    v[3] = b - d;
}

// Part 1: the raw values into s_stage (n values, natural order); ends with
// a barrier.
template <int XT>
__device__ __forceinline__ void rht2k_stage(int k, const Rht2kLoad& L, void* s_stage)
{
#pragma unroll
    for (int b = 0; b < RHT2K_MAXB; b++) {
        if (b < k) {
            const int64_t e = (int64_t)b * RHT2K + 2 * threadIdx.x;
            if constexpr (XT == VQ2_DT_F32) *(u32x2*)((float*)s_stage + e) = L.x[b];
            else *(uint32_t*)((uint16_t*)s_stage + e) = L.x[b][0];
        }
    }
    __syncthreads();
}

// Part 2, the transform: s_nat: n floats; s_split: the split layout (may
// overlap s_stage, not s_nat).  mid() runs after the register and lane
// stages, before the two LDS passes (a caller issues its first centroid
// gathers there: their latency then overlaps the LDS passes).  A barrier
// must follow.
struct NoMid {
    __device__ void operator()() const {}
};
template <int XT, class M = NoMid>
__device__ __forceinline__ void rht2k_transform(int k, int64_t n, const Rht2kLoad& L, const void* s_stage,
                                                float* s_nat, float* s_split, float scale, int xb, M mid = M())
{
    const int t = threadIdx.x, lane = t & 63;
    // permuted values, signs, bit 0, bits 1-6
#pragma unroll
    for (int b = 0; b < RHT2K_MAXB; b++) {
        if (b < k) {
            float v[2];
#pragma unroll
            for (int j = 0; j < 2; j++) {
                const uint32_t pj = L.p[b][j];
                const bool bad = pj >= (uint32_t)n;
                const uint32_t src = bad ? 0u : pj;
                float xv;
                if constexpr (XT == VQ2_DT_F32) xv = ((const float*)s_stage)[src];
                else if constexpr (XT == VQ2_DT_F16) xv = f16_bits_to_f32(((const uint16_t*)s_stage)[src]);
                else xv = bf16_bits_to_f32(((const uint16_t*)s_stage)[src]);
                const float sg = (float)(int8_t)((L.s[b] >> (8 * j)) & 0xFFu);
                v[j] = bad ? __builtin_nanf("") : xv * sg;
            }
            float v0 = v[0] + v[1], v1 = v[0] - v[1];
            lane_stage<1>(v0, v1, lane);
            lane_stage<2>(v0, v1, lane);
            lane_stage<4>(v0, v1, lane);
            lane_stage<8>(v0, v1, lane);
            lane_stage<16>(v0, v1, lane);
            lane_stage<32>(v0, v1, lane);
            u32x2 w;
            w[0] = __float_as_uint(v0);
            w[1] = __float_as_uint(v1);
            *(u32x2*)(s_nat + (int64_t)b * RHT2K + 2 * t) = w;
        }
    }
    __syncthreads();
    mid();
    // bits 7-8: values base + 128 i
    for (int u = t; u < 512 * k; u += SG_THREADS) {
        const int64_t base = (int64_t)(u >> 9) * RHT2K + ((u & 511) >> 7 << 9) + (u & 127);
        float v[4];
#pragma unroll
        for (int i = 0; i < 4; i++) v[i] = s_nat[base + 128 * i];
        radix4(v);
#pragma unroll
        for (int i = 0; i < 4; i++) s_nat[base + 128 * i] = v[i];
    }
    __syncthreads();
    // bits 9-10: values base + 512 i, scaled, into the split layout
    for (int u = t; u < 512 * k; u += SG_THREADS) {
        const int64_t base = (int64_t)(u >> 9) * RHT2K + (u & 511);
        float v[4];
#pragma unroll
        for (int i = 0; i < 4; i++) v[i] = s_nat[base + 512 * i];
        radix4(v);
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int64_t e = base + 512 * i;
            s_split[((e >> 2) & 1) * xb + 4 * (e >> 3) + (e & 3)] = v[i] * scale;
        }
    }
}

template <int XT, class M = NoMid>
__device__ __forceinline__ void rht2k_build(int k, int64_t n, const Rht2kLoad& L, void* s_stage, float* s_nat,
                                            float* s_split, float scale, int xb, M mid = M())
{
    rht2k_stage<XT>(k, L, s_stage);
    rht2k_transform<XT>(k, n, L, s_stage, s_nat, s_split, scale, xb, mid);
}

// One 512-point block by the same all-threads scheme (the MoE down
// projection's rotation): thread t < 256 holds the permuted, signed values
// 2 t + j read through `val` (natural order, index < 512), bit 0 in
// registers, bits 1-6 across lanes, bits 7-8 as one radix-4 pass through
// LDS (s_nat: 512 floats that `val` does not read) that scales and stores
// the split layout (halves xb floats apart).  A barrier must follow.
struct RhtPairLoad {
    u32x2 p;     // permutation entries 2 t, 2 t + 1
    uint32_t s;  // their two sign bytes (low 16 bits)
};

constexpr int RHT512 = 512;

__device__ __forceinline__ void rht512_load(const GemvArgs& a, RhtPairLoad& L)
{
    typedef const __attribute__((address_space(1))) u32x2* gp2;
    typedef const __attribute__((address_space(1))) uint16_t* gp16;
    const int64_t e = 2 * (int64_t)(threadIdx.x < RHT512 / 2 ? threadIdx.x : 0);
    L.p = *(gp2)(a.perm ? a.perm + e : g_perm_iota.v + e);
    L.s = *(gp16)(a.sign ? a.sign + e : g_sign_ones.v + e);
}

template <typename F>
__device__ __forceinline__ void rht512_transform(const RhtPairLoad& L, F val, float* s_nat, float* s_split, float scale,
                                                 int xb)
{
    const int t = threadIdx.x, lane = t & 63;
    if (t < RHT512 / 2) {
        float v[2];
#pragma unroll
        for (int j = 0; j < 2; j++) {
            const uint32_t pj = L.p[j];
            const bool bad = pj >= (uint32_t)RHT512;
            const float sg = (float)(int8_t)((L.s >> (8 * j)) & 0xFFu);
            const float xv = val(bad ? 0u : pj);
            v[j] = bad ? __builtin_nanf("") : xv * sg;
        }
        float v0 = v[0] + v[1], v1 = v[0] - v[1];
        lane_stage<1>(v0, v1, lane);
        lane_stage<2>(v0, v1, lane);
        lane_stage<4>(v0, v1, lane);
        lane_stage<8>(v0, v1, lane);
        lane_stage<16>(v0, v1, lane);
        lane_stage<32>(v0, v1, lane);
        u32x2 w;
        w[0] = __float_as_uint(v0);
        w[1] = __float_as_uint(v1);
        *(u32x2*)(s_nat + 2 * t) = w;
    }
    __syncthreads();
    // bits 7-8: values t + 128 i, scaled, into the split layout
    if (t < 128) {
        float v[4];
#pragma unroll
        for (int i = 0; i < 4; i++) v[i] = s_nat[t + 128 * i];
        radix4(v);
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int e = t + 128 * i;
            s_split[((e >> 2) & 1) * xb + 4 * (e >> 3) + (e & 3)] = v[i] * scale;
        }
    }
}

// 8-term dot product of one centroid (fp16 or bf16, 16 bytes) with group g
// of the split activation in LDS, fp32.
template <int CBT>
__device__ __forceinline__ float centroid_dot(const u32x4 c, const float* s_x, uint32_t g, int xb)
{
    const float* p = s_x + 4 * g;
    const u32x4 x0 = *(const u32x4*)p, x1 = *(const u32x4*)(p + xb);
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

// One lane's entry words of an iteration (SG_LANE_WORDS = 3; a 3-element
// vector type would be read as 16 bytes).
struct Ent3 {
    uint32_t w[SG_LANE_WORDS];
};

// One wave's pass over iterations [s0, s1) of a chunk (stride W, the waves of
// the workgroup, starting at s0 + wave), stage-2 entries from c_mid on.
// load_entries() issues the first three (GD 3: four) iterations' entry words
// and gathers() the first GD iterations' centroid gathers (iterations at or
// past s1 are clamped to the chunk's first, whose lines are cached), so a
// caller can put a prologue between them, or before both.  run() keeps entry
// words that far ahead and gathers GD ahead of the arithmetic until the last
// GD iterations, which it finishes from the gathers already in flight (no
// loads past the range).  Loads complete in issue order and no branch
// separates them, so each wait covers exactly the values it needs.
// A gather reads the iteration's four base codes from lane SG_BASE_LANE
// (v_readlane: scalar registers, no memory access) and adds each lane's
// offset; a code is masked to its codebook's size (65536 rows, or 256 for
// the uint8 stage 2 of (16,8)), so no entry word can address outside it.
// TALL: chunks whose positions may take 17 bits (bit 16 in the field's high
// byte); the others read a position from its field's low 16 bits alone
// (the full decode measured 0.24 us slower per dense step).
template <int CBT, int GD = 2, int W = SG_WAVES, bool TALL = false>
struct SortedPipe {
    static_assert(GD >= 1 && GD <= 3, "gather depth 1 to 3");
    static constexpr int NE = GD + 1 > 3 ? GD + 1 : 3;  // entry words held: iterations it .. it + (NE - 1) W
    const uint32_t* ent;
    const u32x4* cb0;
    const u32x4* cb1;
    int c_beg, c_mid, s1, lane;
    int it;
    uint32_t pb;     // position bits P of a field
    uint32_t dummy;  // the dummy row's position, R << gbits
    uint32_t mask1;  // stage-2 code mask: 0xFFFF, or 0xFF for a 256-row codebook
    int ie[NE];      // the (clamped) iterations of the entry words
    Ent3 e[NE];
    u32x4 c[GD][4];  // centroids of iterations it .. it + (GD - 1) W

    __device__ __forceinline__ int clampit(int i) const { return i < s1 ? i : c_beg; }
    __device__ __forceinline__ Ent3 load_e(int i) const
    {
        typedef const __attribute__((address_space(1))) uint32_t* gp;
        const gp p = (gp)(ent + ((int64_t)i * 64 + lane) * SG_LANE_WORDS);
        Ent3 v;
#pragma unroll
        for (int k = 0; k < SG_LANE_WORDS; k++) v.w[k] = __builtin_nontemporal_load(p + k);
        return v;
    }
    // the low 16 bits of field q (its position, and for P < 16 the low bits
    // of its code offset) and the whole 24-bit field
    static __device__ __forceinline__ uint32_t lo16(const Ent3& ew, int q)
    {
        const uint32_t d = ew.w[q >> 1];
        return (q & 1) ? d >> 16 : d & 0xFFFFu;
    }
    static __device__ __forceinline__ uint32_t field(const Ent3& ew, int q)
    {
        return lo16(ew, q) | (((ew.w[2] >> (8 * q)) & 0xFFu) << 16);
    }
    __device__ __forceinline__ void gather(int i, const Ent3& ew, u32x4 (&cw)[4]) const
    {
        const u32x4* cb = i < c_mid ? cb0 : cb1;
        const uint32_t cmask = i < c_mid ? 0xFFFFu : mask1;
        const uint32_t b01 = (uint32_t)__builtin_amdgcn_readlane((int)ew.w[0], SG_BASE_LANE);
        const uint32_t b23 = (uint32_t)__builtin_amdgcn_readlane((int)ew.w[1], SG_BASE_LANE);
#pragma unroll
        for (int q = 0; q < 4; q++) {
            const uint32_t bw = q < 2 ? b01 : b23;
            const uint32_t base = (q & 1) ? bw >> 16 : bw & 0xFFFFu;
            cw[q] = cb[(base + (field(ew, q) >> pb)) & cmask];
        }
    }
    // the four positions (row << gbits | group) of this lane's entries;
    // the base lane's are the dummy row's
    __device__ __forceinline__ u32x4 positions(const Ent3& ew) const
    {
        const uint32_t pmask = (1u << pb) - 1u;
        u32x4 p;
#pragma unroll
        for (int q = 0; q < 4; q++) p[q] = lane == SG_BASE_LANE ? dummy : (TALL ? field(ew, q) : lo16(ew, q)) & pmask;
        return p;
    }
    // a missing stage-2 codebook is never selected for a real entry; cb0
    // stands in so that no gather can use a null base
    __device__ __forceinline__ void load_entries(const uint32_t* ent_, const void* cb0_, const void* cb1_, int c_beg_,
                                                 int c_mid_, int s0, int s1_, int wave, int lane_, int gbits, int R,
                                                 uint32_t mask1_ = 0xFFFFu)
    {
        mask1 = mask1_;
        ent = ent_;
        cb0 = (const u32x4*)cb0_;
        cb1 = (const u32x4*)(cb1_ ? cb1_ : cb0_);
        c_beg = c_beg_;
        c_mid = c_mid_;
        s1 = s1_;
        lane = lane_;
        pb = (uint32_t)sorted_pbits(gbits, R);
        dummy = (uint32_t)R << gbits;
        it = s0 + wave;
#pragma unroll
        for (int d = 0; d < NE; d++) {
            ie[d] = clampit(it + d * W);
            e[d] = load_e(ie[d]);
        }
    }
    // the stage-2 start and the position fields, set after load_entries
    // (whose loads need neither)
    __device__ __forceinline__ void set_fields(int c_mid_, int gbits, int R)
    {
        c_mid = c_mid_;
        pb = (uint32_t)sorted_pbits(gbits, R);
        dummy = (uint32_t)R << gbits;
    }
    __device__ __forceinline__ void gathers()
    {
#pragma unroll
        for (int d = 0; d < GD; d++) gather(ie[d], e[d], c[d]);
    }
    __device__ __forceinline__ void start(const uint32_t* ent_, const void* cb0_, const void* cb1_, int c_beg_,
                                          int c_mid_, int s0, int s1_, int wave, int lane_, int gbits, int R,
                                          uint32_t mask1_ = 0xFFFFu)
    {
        load_entries(ent_, cb0_, cb1_, c_beg_, c_mid_, s0, s1_, wave, lane_, gbits, R, mask1_);
        gathers();
    }
    __device__ __forceinline__ void shift(const Ent3& enew, int inew)
    {
#pragma unroll
        for (int d = 0; d + 1 < NE; d++) {
            e[d] = e[d + 1];
            ie[d] = ie[d + 1];
        }
        e[NE - 1] = enew;
        ie[NE - 1] = inew;
    }
    __device__ __forceinline__ void accumulate(float* acc, const float* x, uint32_t gbits, uint32_t gmax, uint32_t R,
                                               int xb)
    {
        const uint32_t gmask = (1u << gbits) - 1u;
        const u32x4 pos = positions(e[0]);
#pragma unroll
        for (int q = 0; q < 4; q++) {
            const uint32_t r = min(pos[q] >> gbits, R);
            const uint32_t g = min(pos[q] & gmask, gmax);
            acc[r] += centroid_dot<CBT>(c[0][q], x, g, xb);
        }
    }
    // acc: this lane's accumulator array (R + 1 floats), x: the activation
    // (split layout, halves xb floats apart)
    __device__ __forceinline__ void run(float* acc, const float* x, int gbits, int64_t ng, int R, int xb)
    {
        const uint32_t gmax = (uint32_t)(ng - 1);
        // iterations whose gathers GD ahead are real
        for (; it + GD * W < s1; it += W) {
            const int inew = clampit(it + NE * W);
            const Ent3 enew = load_e(inew);
            u32x4 cn[4];  // the gathers GD iterations ahead
            gather(ie[GD], e[GD], cn);
            accumulate(acc, x, (uint32_t)gbits, gmax, (uint32_t)R, xb);
            shift(enew, inew);
#pragma unroll
            for (int d = 0; d + 1 < GD; d++)
#pragma unroll
                for (int q = 0; q < 4; q++) c[d][q] = c[d + 1][q];
#pragma unroll
            for (int q = 0; q < 4; q++) c[GD - 1][q] = cn[q];
        }
        // the last (at most GD) iterations: their gathers are in flight
#pragma unroll
        for (int k = 0; k < GD; k++) {
            if (it >= s1) break;
            accumulate(acc, x, (uint32_t)gbits, gmax, (uint32_t)R, xb);
            shift(e[NE - 1], ie[NE - 1]);
#pragma unroll
            for (int d = 0; d + 1 < GD; d++)
#pragma unroll
                for (int q = 0; q < 4; q++) c[d][q] = c[d + 1][q];
            it += W;
        }
    }
    // run() with the arithmetic of an iteration given by the caller:
    // f(the four positions of this lane's entries, their four centroids)
    template <class F>
    __device__ __forceinline__ void run_each(F&& f)
    {
        for (; it + GD * W < s1; it += W) {
            const int inew = clampit(it + NE * W);
            const Ent3 enew = load_e(inew);
            u32x4 cn[4];
            gather(ie[GD], e[GD], cn);
            f(positions(e[0]), c[0]);
            shift(enew, inew);
#pragma unroll
            for (int d = 0; d + 1 < GD; d++)
#pragma unroll
                for (int q = 0; q < 4; q++) c[d][q] = c[d + 1][q];
#pragma unroll
            for (int q = 0; q < 4; q++) c[GD - 1][q] = cn[q];
        }
#pragma unroll
        for (int k = 0; k < GD; k++) {
            if (it >= s1) break;
            f(positions(e[0]), c[0]);
            shift(e[NE - 1], ie[NE - 1]);
#pragma unroll
            for (int d = 0; d + 1 < GD; d++)
#pragma unroll
                for (int q = 0; q < 4; q++) c[d][q] = c[d + 1][q];
            it += W;
        }
    }
};

// This lane's accumulator array: `parts` per wave (2 or 4), one per
// 64 / parts consecutive lanes.
__device__ __forceinline__ float* sorted_acc(float* s_acc, int wave, int lane, int R, int parts = SG_PARTS)
{
    return s_acc + (wave * parts + (lane >> (parts == SG_MAX_PARTS ? 4 : 5))) * (R + 1);
}

__device__ __forceinline__ void sorted_acc_zero(float* acc, int lane, int R, int parts = SG_PARTS)
{
    const int pl = 64 / parts;
    for (int i = lane & (pl - 1); i <= R; i += pl) acc[i] = 0.0f;
}

// Row sums of the SG_WAVES x parts accumulator arrays (after a barrier):
// thread (p, r) adds a quarter of the arrays of row r, then the four
// partials are added in p order (a fixed order: deterministic); chunks of
// 256 rows or more (TALL instantiations), half of them and then the two
// halves.  The result is meaningful for threads with threadIdx.x < R (row
// threadIdx.x); ends with a barrier-free read, after the barrier between
// the two halves.
template <bool TALL = false>
__device__ __forceinline__ float sorted_row_sums(const float* s_acc, int R, float (*s_red)[256], int parts = SG_PARTS)
{
    if (TALL && R >= 256) {
        float* sr = &s_red[0][0];  // [2][512]
        const int rr = threadIdx.x & 511, pp = threadIdx.x >> 9;
        if (rr < R) {
            float part = 0.0f;
            const int NA = SG_WAVES * parts / 2;
#pragma unroll 4
            for (int w = NA * pp; w < NA * pp + NA; w++) part += s_acc[w * (R + 1) + rr];
            sr[pp * 512 + rr] = part;
        }
        __syncthreads();
        return (pp == 0 && rr < R) ? sr[rr] + sr[512 + rr] : 0.0f;
    }
    const int rr = threadIdx.x & 255, pp = threadIdx.x >> 8;
    if (rr < R) {
        float part = 0.0f;
        const int NA = SG_WAVES * parts / 4;
#pragma unroll 4
        for (int w = NA * pp; w < NA * pp + NA; w++) part += s_acc[w * (R + 1) + rr];
        s_red[pp][rr] = part;
    }
    __syncthreads();
    return (pp == 0 && rr < R) ? ((s_red[0][rr] + s_red[1][rr]) + s_red[2][rr]) + s_red[3][rr] : 0.0f;
}

}  // namespace vq2
