// vq2_gemv_kernel.hpp -- vector-quantized GEMV kernel body for gfx950 (CDNA4, wave64).
//
// One kernel body serves three call shapes of the decode path:
//   dense    y[b, r]    = VQ(W) x_b                                     (P = 1, no ids)
//   grouped  y[k, r]    = VQ(W_{ids[k]}) x_k                            (P = 1, ids)
//   combine  out[t, r]  = sum_j w[t*P+j] * VQ(W_{ids[t*P+j]}) x_{t*P+j}   (P > 1)
// with VQ(W)[r, 8g+j] = (cb0[i0[r,g]] [+ cb1[i1[r,g]]])[j] and the row scale
// and rs applied after fp32 accumulation: y = (acc * s[r]) * rs.
//
// Reference semantics: vq2/kernels.py:32-78 (_vq_gemv_16_8, _vq_gemv_16) and
// vq2/kernels.py:117-176 (_parallel_moe_gate_up/_down_kernel); the weighted
// combine is vq2/paged_runtime.py:510.
//
// Work decomposition (the MI355X layout, not the reference's Triton tiling):
//   * each lane owns GPL consecutive groups of one K-chunk; its slice of the
//     activation (GPL*8 values per batch column) lives in VGPRs as fp32;
//   * LPR lanes cover one row of a K-chunk (KC = LPR*GPL groups), so a wave
//     streams 64/LPR rows per index load: consecutive lanes read consecutive
//     index words -> fully coalesced, non-temporal index streams;
//   * every index triggers one 16-byte centroid gather (the 1 MiB codebook is
//     L2-resident); the (16,8) stage-2 codebook (256 x 8) is staged in LDS;
//   * a row block's work items (expert pair x K-chunk) are spread over WI
//     waves, the other waves split the rows; item partials are scaled per
//     pair and reduced through LDS in a fixed order (deterministic split-K
//     and weighted combine inside the workgroup);
//   * row partials are reduced across the LPR lanes with DPP/swizzle.
// Shapes whose index rows or activations cannot be read with vector loads
// (n/8 not a multiple of GPL, misaligned planes or rows) take vq_gemv_generic.
#pragma once
#include <type_traits>

#include "vq2_common.hpp"
#include "vq2_internal.hpp"
#include "vq2_router.hpp"

namespace vq2 {

// One matrix of a launch.  Dense launches may carry up to VQ2_MAX_SEG
// matrices that share the activation (q/k/v, gate/up); grouped launches have
// one segment whose pointers are the expert pool's base.
struct GemvSeg {
    const int16_t* idx0;
    const void* idx1;
    const void* scale;
    void* y;
    int64_t out_rows;
    int64_t y_bstride;  // elements between batch columns of y
    int64_t rb_start;   // first row block of this segment in the launch
};

constexpr int VQ2_MAX_SEG = 4;

struct GemvArgs {
    const void* x;
    int x_dt;
    int64_t x_bstride;  // elements between batch columns
    int64_t x_pstride;  // elements between x blocks
    int x_pdiv;         // pair p reads x block p / x_pdiv
    const void* cb0;
    const void* cb1;
    int s_dt;
    int64_t e_istride;  // elements between experts in the index planes
    int64_t e_sstride;  // elements between experts in the scale array
    const void* ids;
    int ids_i64;
    int64_t n_experts;
    const float* pair_w;  // per-pair combine weights, may be null
    int y_acc;            // XM 2: add the combine to y instead of overwriting it
    int P;                // pairs per output group
    int y_dt;
    int64_t y_ostride;
    int64_t ng;
    int batch;
    float rs;
    int lpr;  // lanes per row (power of two <= 32)
    int wi;   // waves along work items (pair x chunk)
    int nch;  // K chunks of lpr * GPL groups per row
    int64_t n_rowblocks;
    int nseg;
    GemvSeg seg[VQ2_MAX_SEG];
    // activation prologue (XM != 0): the workgroup builds the rotated
    // activation in LDS: XM 1: RHT(x) of each batch column; XM 2: RHT of
    // silu(gate) * up for each pair of the output group (x holds the pairs'
    // [gate | up] rows, stride x_pstride, width 2 * n).
    const int32_t* perm;
    const int8_t* sign;
    int hb_log2;
    float xscale;
    // fused router (XM 3: the gate_up launch, one pair per output group): output group
    // og is slot og % r_pairs of token og / r_pairs; slots < r_k take the
    // token's top-k routed experts from its logits, slot r_k the shared
    // expert r_shared.  Workgroup 0 of each group writes the pair's expert id
    // and combine weight to r_ids / r_w.
    const void* r_logits;
    int r_ldt;
    int64_t r_ne;
    int r_k;
    int r_pairs;
    int64_t r_shared;
    const void* r_gate;
    int r_gdt;
    int32_t* r_ids;
    float* r_w;
    uint64_t* cand;  // EP 1: [gridDim.x][batch] best top-1 keys
};

template <int CBT>
struct Centroid;

// fp16 codebook: one 16-byte gather, converted inside the FMA (v_fma_mix).
template <>
struct Centroid<VQ2_DT_F16> {
    half8_t h;
    __device__ __forceinline__ void load(const void* cb, uint32_t code) { h = *((const half8_t*)cb + code); }
    __device__ __forceinline__ float get(int j) const { return (float)h[j]; }
};

template <>
struct Centroid<VQ2_DT_BF16> {
    u32x4 u;
    __device__ __forceinline__ void load(const void* cb, uint32_t code) { u = *((const u32x4*)cb + code); }
    __device__ __forceinline__ float get(int j) const
    {
        const uint32_t w = u[j >> 1];
        return (j & 1) ? __uint_as_float(w & 0xFFFF0000u) : __uint_as_float(w << 16);
    }
};

template <>
struct Centroid<VQ2_DT_F32> {
    u32x4 a, b;
    __device__ __forceinline__ void load(const void* cb, uint32_t code)
    {
        const u32x4* p = (const u32x4*)cb + 2 * (size_t)code;
        a = p[0];
        b = p[1];
    }
    __device__ __forceinline__ float get(int j) const { return __uint_as_float(j < 4 ? a[j] : b[j - 4]); }
};

// Stage-2 centroid from the LDS copy of a 256-row codebook.
template <int CBT>
__device__ __forceinline__ Centroid<CBT> lds_centroid(const u32x4* s_cb1, uint32_t code)
{
    Centroid<CBT> c;
    if constexpr (CBT == VQ2_DT_F32) {
        c.a = s_cb1[2 * code];
        c.b = s_cb1[2 * code + 1];
    } else if constexpr (CBT == VQ2_DT_F16) {
        c.h = __builtin_bit_cast(half8_t, s_cb1[code]);
    } else {
        c.u = s_cb1[code];
    }
    return c;
}

// Raw index words of one lane for IT rows of GPL groups, as loaded: uint16
// codes (stage 1, and stage 2 of (16,16)) two per dword, uint8 codes (stage 2
// of (16,8)) four per dword.  Codes are unpacked where the gathers use them:
// unpacking right after the load would make the compiler wait for the
// (HBM-latency) load there, and the next row block's index prefetch would
// overlap nothing.
template <int S2, int GPL, int IT>
struct Codes {
    static constexpr int W0 = (GPL + 1) / 2;
    static constexpr int W1 = S2 == VQ2_S2_U8 ? (GPL + 3) / 4 : (S2 == VQ2_S2_U16 ? W0 : 1);
    uint32_t w0[IT][W0];
    uint32_t w1[IT][W1];
    // the row scale's raw 16-bit halves (fp32: low, high; fp16 / bf16: the
    // value twice), fetched with the index words so the epilogue has it
    uint32_t s0[IT], s1[IT];
    __device__ __forceinline__ uint32_t c0(int it, int q) const { return (w0[it][q >> 1] >> (16 * (q & 1))) & 0xFFFFu; }
    __device__ __forceinline__ float scale(int it, int dt) const
    {
        return dt == VQ2_DT_F32 ? __uint_as_float((s1[it] << 16) | s0[it])
                                : (dt == VQ2_DT_F16 ? f16_bits_to_f32((uint16_t)s0[it]) : bf16_bits_to_f32(s0[it]));
    }
    __device__ __forceinline__ uint32_t c1(int it, int q) const
    {
        if constexpr (S2 == VQ2_S2_U8) return (w1[it][q >> 2] >> (8 * (q & 3))) & 0xFFu;
        else return (w1[it][q >> 1] >> (16 * (q & 1))) & 0xFFFFu;
    }
};

// GPL uint16 codes (int16 storage) starting at element off; one vector load.
template <int GPL>
__device__ __forceinline__ void load_raw16(const int16_t* p, int64_t off, uint32_t (&w)[(GPL + 1) / 2])
{
    const int16_t* q = p + off;
    if constexpr (GPL == 8) {
        const u32x4 v = __builtin_nontemporal_load((const u32x4*)q);
#pragma unroll
        for (int i = 0; i < 4; i++) w[i] = v[i];
    } else if constexpr (GPL == 4) {
        const u32x2 v = __builtin_nontemporal_load((const u32x2*)q);
        w[0] = v.x;
        w[1] = v.y;
    } else if constexpr (GPL == 2) {
        w[0] = __builtin_nontemporal_load((const uint32_t*)q);
    } else {
        w[0] = (uint32_t)__builtin_nontemporal_load((const uint16_t*)q);
    }
}

// GPL uint8 codes starting at element off; one load.
template <int GPL>
__device__ __forceinline__ void load_raw8(const uint8_t* p, int64_t off, uint32_t (&w)[(GPL + 3) / 4])
{
    const uint8_t* q = p + off;
    if constexpr (GPL == 8) {
        const u32x2 v = __builtin_nontemporal_load((const u32x2*)q);
        w[0] = v.x;
        w[1] = v.y;
    } else if constexpr (GPL == 4) {
        w[0] = __builtin_nontemporal_load((const uint32_t*)q);
    } else if constexpr (GPL == 2) {
        w[0] = (uint32_t)__builtin_nontemporal_load((const uint16_t*)q);
    } else {
        w[0] = (uint32_t)__builtin_nontemporal_load(q);
    }
}

// Row scale element idx of a scale array of dtype dt, as two 16-bit loads at
// addresses chosen by the dtype (no branch around a load: the compiler would
// then wait for every outstanding load where the paths merge).
template <int S2, int GPL, int IT>
__device__ __forceinline__ void load_scale(const void* sp, int dt, int64_t idx, int it, Codes<S2, GPL, IT>& cd)
{
    const uint16_t* p = (const uint16_t*)sp;
    const bool f32 = dt == VQ2_DT_F32;
    cd.s0[it] = p[f32 ? 2 * idx : idx];
    cd.s1[it] = p[f32 ? 2 * idx + 1 : idx];
}

// The index words of one lane for every plane of a row at element offset off.
template <int S2, int GPL, int IT>
__device__ __forceinline__ void load_codes(const int16_t* i0, const void* i1, int64_t off, int it, Codes<S2, GPL, IT>& cd)
{
    load_raw16<GPL>(i0, off, cd.w0[it]);
    if constexpr (S2 == VQ2_S2_U8) load_raw8<GPL>((const uint8_t*)i1, off, cd.w1[it]);
    if constexpr (S2 == VQ2_S2_U16) load_raw16<GPL>((const int16_t*)i1, off, cd.w1[it]);
}

// This lane's activation slice: groups [g0, g0+GPL) for nb batch columns,
// as fp32.  Loads are unconditional from a clamped (always valid) address;
// idle lanes and columns >= nb are zeroed afterwards.
template <int GPL, int BT, int XT>
__device__ __forceinline__ void load_x_t(const GemvArgs& a, const void* xb, int64_t g0, bool lane_ok, int nb,
                                         float (&xs)[BT][GPL * 8])
{
#pragma unroll
    for (int b = 0; b < BT; b++) {
        const bool ok = lane_ok && b < nb;
        const int64_t base = ok ? (int64_t)b * a.x_bstride + g0 * 8 : 0;
        const float keep = ok ? 1.0f : 0.0f;
        if constexpr (XT == VQ2_DT_F32) {
            const u32x4* p = (const u32x4*)((const float*)xb + base);
#pragma unroll
            for (int i = 0; i < GPL * 2; i++) {
                const u32x4 v = p[i];
#pragma unroll
                for (int k = 0; k < 4; k++) xs[b][4 * i + k] = __uint_as_float(v[k]) * keep;
            }
        } else {
            const u32x4* p = (const u32x4*)((const uint16_t*)xb + base);
#pragma unroll
            for (int i = 0; i < GPL; i++) {
                const u32x4 v = p[i];
#pragma unroll
                for (int k = 0; k < 4; k++) {
                    if constexpr (XT == VQ2_DT_BF16) {
                        xs[b][8 * i + 2 * k] = __uint_as_float(v[k] << 16) * keep;
                        xs[b][8 * i + 2 * k + 1] = __uint_as_float(v[k] & 0xFFFF0000u) * keep;
                    } else {
                        xs[b][8 * i + 2 * k] = f16_bits_to_f32((uint16_t)(v[k] & 0xFFFFu)) * keep;
                        xs[b][8 * i + 2 * k + 1] = f16_bits_to_f32((uint16_t)(v[k] >> 16)) * keep;
                    }
                }
            }
        }
    }
}

template <int GPL, int BT>
__device__ __forceinline__ void load_x(const GemvArgs& a, const void* xb, int64_t g0, bool lane_ok, int nb,
                                       float (&xs)[BT][GPL * 8])
{
    if (a.x_dt == VQ2_DT_F32)
        load_x_t<GPL, BT, VQ2_DT_F32>(a, xb, g0, lane_ok, nb, xs);
    else if (a.x_dt == VQ2_DT_F16)
        load_x_t<GPL, BT, VQ2_DT_F16>(a, xb, g0, lane_ok, nb, xs);
    else
        load_x_t<GPL, BT, VQ2_DT_BF16>(a, xb, g0, lane_ok, nb, xs);
}

// Element i of a wave-uniform read-only array, read through the scalar cache
// (the constant address space).  Scalar loads count on their own counter, so
// waiting for one does not wait for the vector loads issued before it (the
// prologue's activation loads).  The arrays read this way (expert ids,
// combine weights) are inputs the kernel never writes.
template <typename T>
__device__ __forceinline__ T uniform_load(const void* p, int64_t i)
{
    return ((const __attribute__((address_space(4))) T*)p)[i];
}

__device__ __forceinline__ int64_t pair_expert(const GemvArgs& a, int64_t pair, bool& bad, int64_t e_rt = -1)
{
    if (e_rt >= 0) {
        bad = false;
        return e_rt;
    }
    int64_t e = 0;
    if (a.ids) e = a.ids_i64 ? uniform_load<int64_t>(a.ids, pair) : (int64_t)uniform_load<int32_t>(a.ids, pair);
    bad = a.ids && (e < 0 || e >= a.n_experts);
    return bad ? 0 : e;
}

// Expert of output group og under the fused router (uniform per wave; every
// wave of the group computes it, workgroup 0 / wave 0 also publishes it).
__device__ __forceinline__ int64_t route_pair(const GemvArgs& a, int og, int lane, int wave)
{
    const int64_t t = og / a.r_pairs;
    const int p = og - (int)t * a.r_pairs;
    const bool writer = blockIdx.x == 0 && wave == 0;
    if (p < a.r_k) {
        float mine, tot;
        int my_id;
        if (a.r_ne <= 256)
            router_select<4>(a.r_logits, a.r_ldt, t, a.r_ne, a.r_k, lane, mine, my_id, tot);
        else
            router_select<ROUTER_MAX_E / 64>(a.r_logits, a.r_ldt, t, a.r_ne, a.r_k, lane, mine, my_id, tot);
        if (writer && lane == p) {
            a.r_ids[og] = my_id;
            a.r_w[og] = mine / tot;
        }
        return __builtin_amdgcn_readlane(my_id, p);
    }
    if (writer) {
        const float sw = router_shared_weight(a.r_gate, a.r_gdt, a.x, a.x_dt, t, a.ng * 8, lane);
        if (lane == 0) {
            a.r_ids[og] = (int32_t)a.r_shared;
            a.r_w[og] = sw;
        }
    }
    return a.r_shared;
}

// In-place blockwise Walsh-Hadamard transform of v[0, total) over
// 2^L-point blocks (natural / Sylvester order) by all threads of the block:
// radix-8 passes, each thread butterflies whole groups in registers, one
// barrier per pass.
template <int W>
__device__ __forceinline__ void fwht_pass(float* v, int64_t total, int lo)
{
    const int64_t groups = total >> W;
    for (int64_t g = threadIdx.x; g < groups; g += blockDim.x) {
        const int64_t base = ((g >> lo) << (lo + W)) | (g & ((1LL << lo) - 1));
        float r[1 << W];
#pragma unroll
        for (int k = 0; k < (1 << W); k++) r[k] = v[base + ((int64_t)k << lo)];
#pragma unroll
        for (int h = 1; h < (1 << W); h <<= 1)
#pragma unroll
            for (int k = 0; k < (1 << W); k++)
                if ((k & h) == 0) {
                    const float x0 = r[k], x1 = r[k | h];
                    r[k] = x0 + x1;
                    r[k | h] = x0 - x1;
                }
#pragma unroll
        for (int k = 0; k < (1 << W); k++) v[base + ((int64_t)k << lo)] = r[k];
    }
}

__device__ __forceinline__ void block_fwht(float* v, int64_t total, int L, int lo0 = 0)
{
    for (int lo = lo0; lo < L; lo += 3) {
        const int w = L - lo < 3 ? L - lo : 3;
        if (w == 3) fwht_pass<3>(v, total, lo);
        else if (w == 2) fwht_pass<2>(v, total, lo);
        else fwht_pass<1>(v, total, lo);
        __syncthreads();
    }
}

// The stages of bits 0-5 of the 2^L-point blockwise FWHT for the 8
// consecutive elements [8u, 8u + 8) that thread u holds: bits 0-2 inside the
// thread, bits 3-5 with lanes u ^ 1, u ^ 2, u ^ 4 -- the stages, their order
// and their operands as block_fwht's first two passes, so the values are the
// same, without those passes' strided (bank-conflicting) LDS traffic and
// barriers.  Every 2^L block whose element the thread holds lies entirely
// inside [0, total) with total a multiple of 2^L, so partner lanes are active.
__device__ __forceinline__ void fwht_head(float (&v)[8], int L)
{
#pragma unroll
    for (int b = 0; b < 3; b++) {
        const int h = 1 << b;
        if (b < L) {
#pragma unroll
            for (int k = 0; k < 8; k++)
                if ((k & h) == 0) {
                    const float x0 = v[k], x1 = v[k | h];
                    v[k] = x0 + x1;
                    v[k | h] = x0 - x1;
                }
        }
    }
    const int lane = threadIdx.x & 63;
#pragma unroll
    for (int b = 3; b < 6; b++) {
        const int m = 1 << (b - 3);
        if (b < L) {
            const bool hi = (lane & m) != 0;
#pragma unroll
            for (int k = 0; k < 8; k++) {
                // DPP moves instead of LDS-pipe permutes: lane ^ 1 and
                // lane ^ 2 by quad_perm ([1,0,3,2] = 0xB1, [2,3,0,1] = 0x4E),
                // lane ^ 4 by row_shl:4 (lane + 4, 0x104) where bit 2 is clear
                // and row_shr:4 (lane - 4, 0x114) where it is set
                float p;
                const int vi = __float_as_int(v[k]);
                if (m == 1)
                    p = __int_as_float(__builtin_amdgcn_mov_dpp(vi, 0xB1, 0xF, 0xF, true));
                else if (m == 2)
                    p = __int_as_float(__builtin_amdgcn_mov_dpp(vi, 0x4E, 0xF, 0xF, true));
                else {
                    const int up = __builtin_amdgcn_mov_dpp(vi, 0x104, 0xF, 0xF, true);
                    const int dn = __builtin_amdgcn_mov_dpp(vi, 0x114, 0xF, 0xF, true);
                    p = __int_as_float(hi ? dn : up);
                }
                v[k] = hi ? p - v[k] : v[k] + p;
            }
        }
    }
}

// Prologue of XM 1 / 2: s_x[r * n + i] = sign[i] * f(row r)[perm[i]] for the
// rows r of this workgroup (batch columns for XM 1, pairs for XM 2), then the
// blockwise FWHT.  The RHT scale is applied when lanes read their slices.
// Each thread takes 8 consecutive elements per iteration: perm and sign are
// read with vector loads.  n % 8 == 0; perm 16-byte and sign 8-byte aligned
// (checked on the host).
//
// The permutation is applied in LDS: a thread loads the activation elements
// of its own 8 slots (contiguous, coalesced) together with the slots'
// permutation and sign words, so no global load waits for another.  The
// workgroup stages the raw block in LDS (stage_x), and after a barrier each
// thread reads its permuted elements from there (xpro_permute) and does the
// arithmetic (xpro_finish).  The kernel issues the first iteration's loads
// before its first index load: loads complete in issue order, so the RHT
// arithmetic then waits only for these L2-resident values, not for the index
// words coming from HBM.
struct XProLoad {
    uint32_t g[8];  // the slots' own activation bits (gate half for XM 2), then the permuted staged values
    uint32_t u[8];  // the slots' up-half bits (XM 2)
    u32x4 p0, p1;   // the slots' permutation entries (identity-table entries without a permutation)
    u32x2 sv;       // 8 sign bytes
    bool bad[8];    // permutation entry outside [0, n): the value is poisoned
};

template <int XT>
__device__ __forceinline__ float raw_to_f32(uint32_t r)
{
    if constexpr (XT == VQ2_DT_F32) return __uint_as_float(r);
    else if constexpr (XT == VQ2_DT_F16) return f16_bits_to_f32((uint16_t)r);
    else return bf16_bits_to_f32(r);
}

// +1 signs and identity entries for a rotation without a sign table or a
// permutation: the prologue then loads its words from here (a select of
// pointers, no branch around the load).  The tables repeat every 8192
// elements: the identity entry of element i is i & 8191, and the prologue
// adds i & ~8191.
constexpr int VQ2_ONES = 8192;
struct OnesTable {
    int8_t v[VQ2_ONES];
    constexpr OnesTable() : v() { for (int i = 0; i < VQ2_ONES; i++) v[i] = 1; }
};
static __device__ const OnesTable g_sign_ones = OnesTable();
struct IotaTable {
    int32_t v[VQ2_ONES];
    constexpr IotaTable() : v() { for (int i = 0; i < VQ2_ONES; i++) v[i] = i; }
};
static __device__ const __align__(16) IotaTable g_perm_iota = IotaTable();

// Activation row of slot row r.
template <int XM>
__device__ __forceinline__ int64_t x_row(const GemvArgs& a, int r, int og, int bt0)
{
    if constexpr (XM == 1) return (int64_t)(og / a.x_pdiv) * a.x_pstride + (int64_t)(bt0 + r) * a.x_bstride;
    else return ((int64_t)og * a.P + r) / a.x_pdiv * a.x_pstride;
}

// Activation loads of the 8 slots starting at element t0 of the nrows x n
// block (t0 < total; callers clamp idle threads to t0 = 0): contiguous
// elements, activation dtype XT a template value (no branch around a load).
template <int XM, int XT>
__device__ __forceinline__ void xpro_xload(const GemvArgs& a, int64_t t0, int64_t n, int og, int bt0, XProLoad& L)
{
    const int r = (int)(t0 / n);
    const int64_t i0 = t0 - (int64_t)r * n;
    const int64_t row = x_row<XM>(a, r, og, bt0) + i0;
    if constexpr (XT == VQ2_DT_F32) {
        const uint32_t* x = (const uint32_t*)a.x + row;
#pragma unroll
        for (int k = 0; k < 8; k++) L.g[k] = x[k];
        if constexpr (XM == 2)
#pragma unroll
            for (int k = 0; k < 8; k++) L.u[k] = x[n + k];
    } else {
        const uint16_t* x = (const uint16_t*)a.x + row;
#pragma unroll
        for (int k = 0; k < 8; k++) L.g[k] = x[k];
        if constexpr (XM == 2)
#pragma unroll
            for (int k = 0; k < 8; k++) L.u[k] = x[n + k];
    }
}

// Permutation and sign words of the same slots.  Both tables are global
// memory; said explicitly, or the selected pointer is generic and the load
// becomes a flat load, which the compiler's memory-counter waits cannot
// order against the global loads.
__device__ __forceinline__ void xpro_tables(const GemvArgs& a, int64_t t0, int64_t n, XProLoad& L)
{
    const int r = (int)(t0 / n);
    const int64_t i0 = t0 - (int64_t)r * n;
    const int32_t* pp = a.perm ? a.perm + i0 : g_perm_iota.v + (i0 & (VQ2_ONES - 1));
    const __attribute__((address_space(1))) u32x4* pg = (const __attribute__((address_space(1))) u32x4*)pp;
    L.p0 = pg[0];
    L.p1 = pg[1];
    const int8_t* sgn = a.sign ? a.sign + i0 : g_sign_ones.v + (i0 & (VQ2_ONES - 1));
    L.sv = *(const __attribute__((address_space(1))) u32x2*)sgn;
}

// All loads of an iteration; no loaded value is used here.
template <int XM, int XT>
__device__ __forceinline__ void xpro_load(const GemvArgs& a, int64_t t0, int64_t n, int og, int bt0, XProLoad& L)
{
    xpro_tables(a, t0, n, L);
    xpro_xload<XM, XT>(a, t0, n, og, bt0, L);
}

// Staged block in LDS, [nrows x n]: XM 1 the raw elements in the
// activation's own width; XM 2 silu(gate) * up as fp32 (the activation is
// elementwise, so it is taken before the permutation).
template <int XM, int XT>
__device__ __forceinline__ void stage_store(void* s_stage, int64_t t0, const XProLoad& L)
{
    if constexpr (XM == 2 || XT == VQ2_DT_F32) {
        uint32_t w[8];
#pragma unroll
        for (int k = 0; k < 8; k++)
            w[k] = XM == 2 ? __float_as_uint(silu_f32(raw_to_f32<XT>(L.g[k])) * raw_to_f32<XT>(L.u[k])) : L.g[k];
        u32x4 w0, w1;
#pragma unroll
        for (int k = 0; k < 4; k++) { w0[k] = w[k]; w1[k] = w[4 + k]; }
        uint32_t* st = (uint32_t*)s_stage;
        *(u32x4*)(st + t0) = w0;
        *(u32x4*)(st + t0 + 4) = w1;
    } else {
        u32x4 w;
#pragma unroll
        for (int k = 0; k < 4; k++) w[k] = (L.g[2 * k] & 0xFFFFu) | (L.g[2 * k + 1] << 16);
        *(u32x4*)((uint16_t*)s_stage + t0) = w;
    }
}

// The slots' permuted elements, read from the staged block (same row).
template <int XM, int XT>
__device__ __forceinline__ void xpro_permute(const GemvArgs& a, const void* s_stage, int64_t t0, int64_t n,
                                             XProLoad& L)
{
    const int r = (int)(t0 / n);
    const int64_t rbase = (int64_t)r * n;
    // identity-table entries repeat every VQ2_ONES elements
    const int64_t pbase = a.perm ? 0 : ((t0 - rbase) & ~(int64_t)(VQ2_ONES - 1));
    int64_t src[8];
#pragma unroll
    for (int k = 0; k < 4; k++) {
        src[k] = pbase + (int32_t)L.p0[k];
        src[4 + k] = pbase + (int32_t)L.p1[k];
    }
#pragma unroll
    for (int k = 0; k < 8; k++) {
        L.bad[k] = (uint64_t)src[k] >= (uint64_t)n;  // not a permutation of [0, n): poison the value
        src[k] = rbase + (L.bad[k] ? 0 : src[k]);
    }
    if constexpr (XM == 2 || XT == VQ2_DT_F32) {
        const uint32_t* st = (const uint32_t*)s_stage;
#pragma unroll
        for (int k = 0; k < 8; k++) L.g[k] = st[src[k]];
    } else {
        const uint16_t* st = (const uint16_t*)s_stage;
#pragma unroll
        for (int k = 0; k < 8; k++) L.g[k] = st[src[k]];
    }
}

// Arithmetic of one iteration: activation (silu(gate) * up for XM 2), sign,
// FWHT bits 0-5 (fwht_head), 16-byte LDS stores.
template <int XM, int XT>
__device__ __forceinline__ void xpro_finish(const GemvArgs& a, float* s_x, int64_t t0, const XProLoad& L)
{
    float v[8];
#pragma unroll
    for (int k = 0; k < 8; k++) {
        if constexpr (XM == 2) v[k] = __uint_as_float(L.g[k]);  // silu(gate) * up, taken when staged
        else v[k] = raw_to_f32<XT>(L.g[k]);
        const float sg = (float)(int8_t)((L.sv[k >> 2] >> (8 * (k & 3))) & 0xFFu);
        v[k] = L.bad[k] ? __builtin_nanf("") : v[k] * sg;
    }
    fwht_head(v, a.hb_log2);
    u32x4 o0, o1;
#pragma unroll
    for (int k = 0; k < 4; k++) {
        o0[k] = __float_as_uint(v[k]);
        o1[k] = __float_as_uint(v[4 + k]);
    }
    *(u32x4*)(s_x + t0) = o0;
    *(u32x4*)(s_x + t0 + 4) = o1;
}

// Prologue, part 1: every slot's raw elements into the LDS stage, given the
// first iteration's loads (issued by the caller at t0 = threadIdx.x * 8,
// clamped to 0 past the block); ends with the barrier after which any
// element may be read.
template <int XM, int XT>
__device__ __forceinline__ void stage_x(const GemvArgs& a, void* s_stage, int nrows, int64_t n, int og, int bt0,
                                        const XProLoad& first)
{
    const int64_t total = (int64_t)nrows * n;
    int64_t t0 = (int64_t)threadIdx.x * 8;
    if (t0 < total) stage_store<XM, XT>(s_stage, t0, first);
    for (t0 += (int64_t)blockDim.x * 8; t0 < total; t0 += (int64_t)blockDim.x * 8) {
        XProLoad L;
        xpro_xload<XM, XT>(a, t0, n, og, bt0, L);
        stage_store<XM, XT>(s_stage, t0, L);
    }
    __syncthreads();
}

// Prologue, part 2: permuted reads, arithmetic, then the blockwise FWHT.
template <int XM, int XT>
__device__ __forceinline__ void build_x(const GemvArgs& a, float* s_x, const void* s_stage, int nrows, int64_t n,
                                        XProLoad& first)
{
    const int64_t total = (int64_t)nrows * n;
    int64_t t0 = (int64_t)threadIdx.x * 8;
    if (t0 < total) {
        xpro_permute<XM, XT>(a, s_stage, t0, n, first);
        xpro_finish<XM, XT>(a, s_x, t0, first);
    }
    for (t0 += (int64_t)blockDim.x * 8; t0 < total; t0 += (int64_t)blockDim.x * 8) {
        XProLoad L;
        xpro_tables(a, t0, n, L);
        xpro_permute<XM, XT>(a, s_stage, t0, n, L);
        xpro_finish<XM, XT>(a, s_x, t0, L);
    }
    __syncthreads();
    block_fwht(s_x, total, a.hb_log2, 6);  // bits 0-5 done by fwht_head
}

// A lane's activation slice from the LDS activation block.
template <int GPL, int BT>
__device__ __forceinline__ void load_x_lds(const float* s_x, int64_t row0, int64_t rstride, int64_t g0, bool lane_ok,
                                           int nb, float scale, float (&xs)[BT][GPL * 8])
{
#pragma unroll
    for (int b = 0; b < BT; b++) {
        const bool ok = lane_ok && b < nb;
        const u32x4* p = (const u32x4*)(s_x + (ok ? (row0 + b) * rstride + g0 * 8 : 0));
        const float keep = ok ? scale : 0.0f;
#pragma unroll
        for (int i = 0; i < GPL * 2; i++) {
            const u32x4 v = p[i];
#pragma unroll
            for (int k = 0; k < 4; k++) xs[b][4 * i + k] = __uint_as_float(v[k]) * keep;
        }
    }
}

// Segment of row block rb: a sum of independent comparisons (unused slots
// start at INT64_MAX), so the segment starts load together, with no
// dependent loop.
__device__ __forceinline__ int seg_of(const GemvArgs& a, int64_t rb)
{
    int si = 0;
#pragma unroll
    for (int s = 1; s < VQ2_MAX_SEG; s++) si += rb >= a.seg[s].rb_start ? 1 : 0;
    return si;
}

// Index words of row block rb for this lane; valid = false past the end,
// for idle lanes and for rows beyond their segment.  Past the last row block
// (uniform over the workgroup) nothing is loaded; inside it the loads do not
// depend on the lane: an invalid row reads its plane's first word (every
// segment has at least one row), whose codes index the codebooks in bounds,
// and its partial is zeroed after the dot product.  IN_RANGE: the caller
// knows rb < n_rowblocks (a workgroup's first row block: the persistent grid
// never exceeds the row-block count), so no branch is needed around the
// loads -- where a path with loads and one without merge, the compiler waits
// for every outstanding load at the next use of an earlier one.
template <int S2, int GPL, int IT, bool IN_RANGE = false, bool ZERO_PAST = false>
__device__ __forceinline__ void fetch_codes(const GemvArgs& a, int64_t rb, int rows_per_block, int wr, int wr_id,
                                            int rpw, int sub, int64_t g0, bool lane_ok, int64_t e,
                                            Codes<S2, GPL, IT>& cd, bool (&valid)[IT])
{
    const int si = seg_of(a, rb);
    const GemvSeg& sg = a.seg[si];
    const int64_t row_base = (rb - sg.rb_start) * rows_per_block;
    const bool in_range = IN_RANGE || rb < a.n_rowblocks;
#pragma unroll
    for (int it = 0; it < IT; it++) {
        const int64_t row = row_base + (int64_t)(it * wr + wr_id) * rpw + sub;
        valid[it] = in_range && row < sg.out_rows && lane_ok;
    }
    if (!in_range) {
        // nothing to load; ZERO_PAST: zero codes keep a gather issued ahead
        // for this task inside the codebooks
        if constexpr (ZERO_PAST) {
#pragma unroll
            for (int it = 0; it < IT; it++) {
#pragma unroll
                for (int q = 0; q < Codes<S2, GPL, IT>::W0; q++) cd.w0[it][q] = 0;
#pragma unroll
                for (int q = 0; q < Codes<S2, GPL, IT>::W1; q++) cd.w1[it][q] = 0;
                cd.s0[it] = cd.s1[it] = 0;
            }
        }
        return;
    }
#pragma unroll
    for (int it = 0; it < IT; it++) {
        const int64_t row = row_base + (int64_t)(it * wr + wr_id) * rpw + sub;
        const int64_t off = valid[it] ? row * a.ng + g0 : 0;
        load_codes<S2, GPL, IT>(sg.idx0 + e * a.e_istride,
                                S2 == VQ2_S2_U8 ? (const void*)((const uint8_t*)sg.idx1 + e * a.e_istride)
                                                : (const void*)((const int16_t*)sg.idx1 + e * a.e_istride),
                                off, it, cd);
    }
#pragma unroll
    for (int it = 0; it < IT; it++) {
        const int64_t row = row_base + (int64_t)(it * wr + wr_id) * rpw + sub;
        load_scale<S2, GPL, IT>(sg.scale, a.s_dt, row < sg.out_rows ? e * a.e_sstride + row : 0, it, cd);
    }
}

// Codes of task (row block rb, item) for this lane: item = pair * nch + chunk.
template <int S2, int GPL, int IT, bool IN_RANGE = false, bool ZERO_PAST = false>
__device__ __forceinline__ void task_codes(const GemvArgs& a, int64_t rb, int item, int nch, int64_t kc, int og,
                                           int rows_per_block, int wr, int wr_id, int rpw, int sub, int col,
                                           Codes<S2, GPL, IT>& cd, bool (&valid)[IT], int64_t e_rt)
{
    const int pj = item / nch, c = item - (item / nch) * nch;
    bool bad;
    const int64_t e = pair_expert(a, (int64_t)og * a.P + pj, bad, e_rt);
    const int64_t g0 = c * kc + (int64_t)col * GPL;
    fetch_codes<S2, GPL, IT, IN_RANGE, ZERO_PAST>(a, rb, rows_per_block, wr, wr_id, rpw, sub, g0, g0 < a.ng && !bad, e, cd,
                                       valid);
}

// The centroids of one row block for this lane (global gathers; the (16,8)
// stage-2 centroids come from LDS inside dot_block).
template <int CBT, int S2, int GPL, int IT>
struct Cens {
    Centroid<CBT> c0[IT][GPL];
    Centroid<CBT> c1[IT][S2 == VQ2_S2_U16 ? GPL : 1];
};

// ST0 / ST1: gather the stage-1 / the (16,16) stage-2 centroids
template <int CBT, int S2, int GPL, int IT, bool ST0 = true, bool ST1 = true>
__device__ __forceinline__ void gather_block(const GemvArgs& a, const Codes<S2, GPL, IT>& cd, Cens<CBT, S2, GPL, IT>& ce)
{
#pragma unroll
    for (int it = 0; it < IT; it++) {
        if constexpr (ST0)
#pragma unroll
            for (int q = 0; q < GPL; q++) ce.c0[it][q].load(a.cb0, cd.c0(it, q));
        if constexpr (S2 == VQ2_S2_U16 && ST1)
#pragma unroll
            for (int q = 0; q < GPL; q++) ce.c1[it][q].load(a.cb1, cd.c1(it, q));
    }
}

// acc[it][b] = sum over this lane's GPL groups of VQ(W)[row_it] . x_b, from
// gathered centroids
template <int CBT, int S2, int GPL, int BT, int IT>
__device__ __forceinline__ void dot_block(const u32x4* s_cb1, const Codes<S2, GPL, IT>& cd,
                                          const Cens<CBT, S2, GPL, IT>& ce, const bool (&valid)[IT],
                                          const float (&xs)[BT][GPL * 8], float (&acc)[IT][BT])
{
#pragma unroll
    for (int it = 0; it < IT; it++) {
#pragma unroll
        for (int b = 0; b < BT; b++) acc[it][b] = 0.0f;
        if constexpr (S2 == VQ2_S2_U16) {
#pragma unroll
            for (int q = 0; q < GPL; q++)
#pragma unroll
                for (int j = 0; j < 8; j++) {
                    const float w = ce.c0[it][q].get(j) + ce.c1[it][q].get(j);
#pragma unroll
                    for (int b = 0; b < BT; b++) acc[it][b] = fmaf(w, xs[b][q * 8 + j], acc[it][b]);
                }
        } else if constexpr (S2 == VQ2_S2_U8) {
#pragma unroll
            for (int q = 0; q < GPL; q++) {
                const Centroid<CBT> c2 = lds_centroid<CBT>(s_cb1, cd.c1(it, q));
#pragma unroll
                for (int j = 0; j < 8; j++) {
                    const float w = ce.c0[it][q].get(j) + c2.get(j);
#pragma unroll
                    for (int b = 0; b < BT; b++) acc[it][b] = fmaf(w, xs[b][q * 8 + j], acc[it][b]);
                }
            }
        } else {
#pragma unroll
            for (int q = 0; q < GPL; q++)
#pragma unroll
                for (int j = 0; j < 8; j++)
#pragma unroll
                    for (int b = 0; b < BT; b++) acc[it][b] = fmaf(ce.c0[it][q].get(j), xs[b][q * 8 + j], acc[it][b]);
        }
        if (!valid[it]) {
#pragma unroll
            for (int b = 0; b < BT; b++) acc[it][b] = 0.0f;
        }
    }
}

template <int CBT, int S2, int GPL, int BT, int IT>
__device__ __forceinline__ void block_dot(const GemvArgs& a, const u32x4* s_cb1, const Codes<S2, GPL, IT>& cd,
                                          const bool (&valid)[IT], const float (&xs)[BT][GPL * 8],
                                          float (&acc)[IT][BT])
{
    Cens<CBT, S2, GPL, IT> ce;
    gather_block<CBT, S2, GPL, IT>(a, cd, ce);
    dot_block<CBT, S2, GPL, BT, IT>(s_cb1, cd, ce, valid, xs, acc);
}

// EP 0: store y; EP 1 (pre-rotated x, one item per wave): no y -- every
// workgroup keeps the best (value, row) key of each batch column over its
// row blocks and writes it to a.cand[blockIdx.x * batch + column] (the fused
// top-1 of the LM head).
// Workgroup size limit.  The expert epilogue (XM 2: SwiGLU + RHT + down +
// combine over the P pairs of a token) runs one pair per wave, so it takes
// up to 12 waves (2 bpw, fp16 codebook; <= 170 VGPRs at 3 waves per SIMD)
// or 8 (the rest; <= 256 VGPRs), which those instantiations fit without
// spilling.  Every other kernel keeps 4 waves: a wider bound changes their
// register allocation, and the dense launches measured slower with it.
// XM 4 (the RHT prologue of XM 1 for activations wider than 256 threads x 8
// values, e.g. the 6144-input down projection) takes up to 12 waves, so its
// single prologue pass covers n = 6144 per batch column -- up to 8 with bf16
// or fp32 (16,16) codebooks, whose centroid words would spill at 12.
constexpr int gemv_max_threads(int s2, int cbt, int xm)
{
    return xm == 4 ? (cbt != VQ2_DT_F16 && s2 == VQ2_S2_U16 ? 512 : 768)
                   : (xm != 2 ? 256 : (s2 == VQ2_S2_NONE && cbt == VQ2_DT_F16 ? 768 : 512));
}

// XT: activation dtype of the prologue kernels (XM != 0); unused for XM 0.
template <int CBT, int S2, int GPL, int BT, int IT, int XM, int EP = 0, int XT = VQ2_DT_F32>
// The plan fields the first index load needs come first as 9 dwords of
// scalar kernel arguments: with -amdgpu-kernarg-preload-count the wave
// starts with them in SGPRs (the preload covers 14 dwords).  k_plan packs
// lpr (bits 0-5), wi (6-9), wr (10-13; waves along rows, so blockDim, an
// implicit-argument load, is not on that path) and "fast" (bit 14: one
// segment and no expert ids, so the first fetch uses k_idx0 / k_idx1 /
// k_rows0 directly); k_nchp packs nch (bits 0-15) and P (16-31).
__global__ void __launch_bounds__(gemv_max_threads(S2, CBT, XM))
    vq_gemv_kernel(const int k_ng, const int k_nrb, const uint32_t k_plan, const uint32_t k_nchp,
                   const int16_t* const k_idx0, const void* const k_idx1, const int k_rows0, const GemvArgs a)
{
    // stage-2 (uint8) codebook in LDS: 256 rows x 16 B (x2 for fp32)
    __shared__ u32x4 s_cb1[S2 == VQ2_S2_U8 ? (CBT == VQ2_DT_F32 ? 512 : 256) : 1];
    // 16-byte aligned: the activation block is written and read with 16-byte LDS accesses
    // [activation block (XM != 0)] [item partials | raw activation stage (XM != 0, prologue only)]
    extern __shared__ __align__(16) float s_dyn[];
    // XM 3 is XM 1 (rotate x in the prologue) with the router built in; XM 4
    // is XM 1 in wide workgroups
    constexpr int XP = (XM == 3 || XM == 4) ? 1 : XM;

    const int og = blockIdx.y;
    const int bt0 = blockIdx.z * BT;
    const int k_P = (int)(k_nchp >> 16);
    const int64_t n = (int64_t)k_ng * 8;
    float* s_x = s_dyn;
    float* s_part = s_dyn + (XP == 0 ? 0 : (XP == 2 ? k_P : BT) * n);
    void* const s_stage = s_part;  // the partials are first written after the prologue's last barrier

    const int lane = threadIdx.x & 63;
    // wave-uniform (an SGPR value), so per-wave work items, expert ids and
    // their loads stay scalar
    const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    const int lpr = (int)(k_plan & 63u), wi = (int)((k_plan >> 6) & 15u);
    const int wr = (int)((k_plan >> 10) & 15u);
    const int wi_id = wave % wi, wr_id = wave / wi;
    const int rpw = 64 / lpr;
    const int sub = lane / lpr, col = lane % lpr;
    const int64_t kc = (int64_t)lpr * GPL;
    const int nch = (int)(k_nchp & 0xFFFFu);
    const int items = k_P * nch;
    const int rows_per_block = IT * rpw * wr;

    // Load order: the prologue's first-iteration loads (permutation and sign
    // words, the thread's own activation elements; L2-resident), then the
    // first task's index words (HBM).  The index latency overlaps the
    // prologue, whose LDS staging waits only for its own loads.
    XProLoad xpl;
    int x_rows = 0;
    if constexpr (XP != 0) {
        x_rows = XP == 2 ? k_P : min(BT, a.batch - bt0);
        const int64_t t0 = (int64_t)threadIdx.x * 8;
        xpro_load<XP, XT>(a, t0 < (int64_t)x_rows * n ? t0 : 0, n, og, bt0, xpl);
    }
    // fused router: this group's expert, before its first index words.  The
    // router reads a chain of argument fields (pairs, k, experts, logits):
    // the argument lines are fetched first so every link hits.
    int64_t e_rt = -1;
    if constexpr (XM == 3) {
        touch_kernargs(a);
        e_rt = route_pair(a, og, lane, wave);
    }
    Codes<S2, GPL, IT> cd;
    bool valid[IT];
    if (XP == 0 && ((k_plan >> 14) & 1u) && items == 1) {
        // the common pre-rotated dense case: its first index load needs only
        // the scalar arguments (no segment lookup, no expert id, no argument
        // load).  Prologue kernels take the general path below: their
        // activation loads already wait for the argument lines, and a single
        // path lets the compiler count the loads after them exactly (where two
        // paths with different loads merge, it waits for all of them).
        const int64_t g0 = (int64_t)col * GPL;
        const int64_t rb = blockIdx.x;
#pragma unroll
        for (int it = 0; it < IT; it++) {
            const int64_t row = rb * rows_per_block + (int64_t)(it * wr + wr_id) * rpw + sub;
            valid[it] = rb < k_nrb && row < k_rows0 && g0 < k_ng;
            load_codes<S2, GPL, IT>(k_idx0, k_idx1, valid[it] ? row * k_ng + g0 : 0, it, cd);
        }
        touch_kernargs(a);  // the argument lines the rest of the kernel reads
#pragma unroll
        for (int it = 0; it < IT; it++) {
            const int64_t row = rb * rows_per_block + (int64_t)(it * wr + wr_id) * rpw + sub;
            load_scale<S2, GPL, IT>(a.seg[0].scale, a.s_dt, row < k_rows0 ? row : 0, it, cd);
        }
    } else {
        // the lookup chain below reads several argument lines: fetch them all first
        touch_kernargs(a);
        task_codes<S2, GPL, IT, true>(a, blockIdx.x, wi_id, nch, kc, og, rows_per_block, wr, wr_id, rpw, sub, col,
                                      cd, valid, e_rt);
    }
    const int nb = min(BT, a.batch - bt0);

    // The unpermuted activation block goes to LDS as soon as its loads
    // arrive (the index words, issued after them, may still be in flight).
    if constexpr (XP != 0) stage_x<XP, XT>(a, s_stage, x_rows, n, og, bt0, xpl);
    // Prologue kernels (PRE): the first task's gathers are issued as soon as
    // its index words arrive, before the prologue's arithmetic.  The
    // prologue's first iteration loads nothing more (its loads went out
    // before the index words), so its LDS reads, barriers and passes run
    // while the gathers are in flight.  Unconditional: a branch around them
    // would leave the compiler unsure which loads are outstanding, and it
    // would then wait for the gathers inside the prologue.
    // (The 12-wave XM 4 kernel has at most 168 registers: it holds only the
    // stage-1 centroids through the prologue, and only of fp16 codebooks --
    // more would spill, and a spill reload waits for every gather.)
    constexpr bool PRE = XP != 0 && !(XM == 4 && CBT != VQ2_DT_F16);
    constexpr bool PRE_ST1 = !(XM == 4 && S2 == VQ2_S2_U16);
    Cens<CBT, S2, GPL, IT> ce0;
    if constexpr (PRE) gather_block<CBT, S2, GPL, IT, true, PRE_ST1>(a, cd, ce0);

    if constexpr (S2 == VQ2_S2_U8) {
        const int nent = CBT == VQ2_DT_F32 ? 512 : 256;
        for (int i = threadIdx.x; i < nent; i += blockDim.x) s_cb1[i] = ((const u32x4*)a.cb1)[i];
    }
    if constexpr (XP != 0) build_x<XP, XT>(a, s_x, s_stage, x_rows, n, xpl);
    if constexpr (S2 == VQ2_S2_U8 || XM != 0) __syncthreads();

    float xs[BT][GPL * 8];
    int cur_item = -1;

    if (items == 1 && a.pair_w == nullptr) {
        // One work item (pair og, the whole K range) per wave: the activation
        // slice is loaded once, and the next row block's codes are fetched
        // before the current block's gathers so the HBM latency of the index
        // stream overlaps the codebook gathers.
        const int64_t pair = og;
        bool bad;
        const int64_t e = pair_expert(a, pair, bad, e_rt);
        const int64_t g0 = (int64_t)col * GPL;
        const bool lane_ok = g0 < a.ng;
        if constexpr (XM == 0) {
            const int64_t xoff = (pair / a.x_pdiv) * a.x_pstride + (int64_t)bt0 * a.x_bstride;
            const void* xb = a.x_dt == VQ2_DT_F32 ? (const void*)((const float*)a.x + xoff)
                                                  : (const void*)((const uint16_t*)a.x + xoff);
            load_x<GPL, BT>(a, xb, g0, lane_ok, nb, xs);
        } else {
            load_x_lds<GPL, BT>(s_x, 0, n, g0, lane_ok, nb, a.xscale, xs);
        }
        int64_t rb = blockIdx.x;
        uint64_t bkey[BT];
#pragma unroll
        for (int b = 0; b < BT; b++) bkey[b] = 0;
        // one row block; PRE: its centroids were gathered before the prologue
        auto step = [&](auto pre) {
            const int64_t rbn = rb + gridDim.x;
            Codes<S2, GPL, IT> nx;
            bool nvalid[IT];
            fetch_codes<S2, GPL, IT>(a, rbn, rows_per_block, wr, wr_id, rpw, sub, g0, lane_ok && !bad, e, nx, nvalid);
            float acc[IT][BT];
            if constexpr (decltype(pre)::value) {
                if constexpr (!PRE_ST1) gather_block<CBT, S2, GPL, IT, false, true>(a, cd, ce0);
                dot_block<CBT, S2, GPL, BT, IT>(s_cb1, cd, ce0, valid, xs, acc);
            } else {
                block_dot<CBT, S2, GPL, BT, IT>(a, s_cb1, cd, valid, xs, acc);
            }
#pragma unroll
            for (int it = 0; it < IT; it++)
#pragma unroll
                for (int b = 0; b < BT; b++) acc[it][b] = group_sum(acc[it][b], lpr);
            const int si = seg_of(a, rb);
            const GemvSeg& sg = a.seg[si];
            const int64_t row_base = (rb - sg.rb_start) * rows_per_block;
            if (col == 0) {
#pragma unroll
                for (int it = 0; it < IT; it++) {
                    const int64_t row = row_base + (int64_t)(it * wr + wr_id) * rpw + sub;
                    if (row >= sg.out_rows) continue;
                    const float sc = cd.scale(it, a.s_dt);
#pragma unroll
                    for (int b = 0; b < BT; b++) {
                        float v = (acc[it][b] * sc) * a.rs;
                        if (bad) v = __builtin_nanf("");
                        if constexpr (EP == 1) {
                            const uint64_t k = argmax_key(v, row);
                            bkey[b] = k > bkey[b] ? k : bkey[b];
                        } else if (b < nb) {
                            store_from_f32(sg.y, a.y_dt, (int64_t)og * a.y_ostride + (int64_t)(bt0 + b) * sg.y_bstride + row,
                                           v);
                        }
                    }
                }
            }
#pragma unroll
            for (int it = 0; it < IT; it++) valid[it] = nvalid[it];
            cd = nx;
            rb = rbn;
        };
        // prologue kernels pre-gathered the first block (rb < n_rowblocks:
        // the persistent grid never exceeds the row-block count)
        if constexpr (PRE) step(std::true_type{});
        while (rb < a.n_rowblocks) step(std::false_type{});
        if constexpr (EP == 1) {
            // best key of the workgroup per batch column: wave, then waves
            __shared__ uint64_t s_key[4][BT];
#pragma unroll
            for (int b = 0; b < BT; b++) {
                uint64_t k = bkey[b];
                for (int off = 32; off > 0; off >>= 1) {
                    const uint64_t o = __shfl_xor(k, off);
                    k = o > k ? o : k;
                }
                if (lane == 0) s_key[wave][b] = k;
            }
            __syncthreads();
            if (threadIdx.x < BT && (int)threadIdx.x < nb) {
                uint64_t k = s_key[0][threadIdx.x];
                for (int w = 1; w < (int)(blockDim.x >> 6); w++) k = s_key[w][threadIdx.x] > k ? s_key[w][threadIdx.x] : k;
                a.cand[(int64_t)blockIdx.x * a.batch + bt0 + threadIdx.x] = k;
            }
        }
        return;
    }

    // Several items (expert pairs x K-chunks) per row block: wave wi_id runs
    // its tasks (row block, item) in order and fetches the next task's codes
    // before the current task's gathers; the WI waves' row partials are
    // reduced through LDS in a fixed order once per row block.  AHEAD: the
    // next task's gathers are issued right after the current task's dot
    // product, before the row block's reduction, so the barriers of that
    // reduction do not drain the gathers in flight (not for the 12-wave XM 4
    // kernel or batch tiles above 2, whose registers would spill).
    constexpr bool AHEAD = XM != 4 && BT <= 2;
    int64_t rbg = blockIdx.x;
    int item = wi_id;
    float fin[IT][BT];
#pragma unroll
    for (int it = 0; it < IT; it++)
#pragma unroll
        for (int b = 0; b < BT; b++) fin[it][b] = 0.0f;
    // AHEAD: the first task's centroids (PRE: gathered before the prologue;
    // rbg < n_rowblocks and item < items hold for it)
    if constexpr (AHEAD && !PRE) gather_block<CBT, S2, GPL, IT, true, true>(a, cd, ce0);
    else if constexpr (AHEAD && !PRE_ST1) gather_block<CBT, S2, GPL, IT, false, true>(a, cd, ce0);
    // one task; AHEAD: its centroids are in ce0, and it leaves the next
    // task's there; PRE: the first task, whose centroids were gathered before
    // the prologue
    auto mstep = [&](auto pre) {
        int nitem = item + wi;
        int64_t nrbg = rbg;
        if (nitem >= items) {
            nitem = wi_id;
            nrbg = rbg + gridDim.x;
        }
        Codes<S2, GPL, IT> nx;
        bool nvalid[IT];
        task_codes<S2, GPL, IT, false, AHEAD>(a, nrbg, nitem, nch, kc, og, rows_per_block, wr, wr_id, rpw, sub, col,
                                              nx, nvalid, e_rt);

        const int pj = item / nch, c = item - (item / nch) * nch;
        const int64_t pair = (int64_t)og * a.P + pj;
        bool bad;
        const int64_t e = pair_expert(a, pair, bad, e_rt);
        const int64_t g0 = c * kc + (int64_t)col * GPL;
        const bool lane_ok = g0 < a.ng;
        if (item != cur_item) {
            if constexpr (XM == 0) {
                const int64_t xoff = (pair / a.x_pdiv) * a.x_pstride + (int64_t)bt0 * a.x_bstride;
                const void* xb = a.x_dt == VQ2_DT_F32 ? (const void*)((const float*)a.x + xoff)
                                                      : (const void*)((const uint16_t*)a.x + xoff);
                load_x<GPL, BT>(a, xb, g0, lane_ok, nb, xs);
            } else {
                load_x_lds<GPL, BT>(s_x, XP == 2 ? pj : 0, n, g0, lane_ok, nb, a.xscale, xs);
            }
            cur_item = item;
        }
        float acc[IT][BT];
        if constexpr (AHEAD) {
            dot_block<CBT, S2, GPL, BT, IT>(s_cb1, cd, ce0, valid, xs, acc);
            // the next task's gathers (zero codes past the last row block)
            gather_block<CBT, S2, GPL, IT, true, true>(a, nx, ce0);
        } else if constexpr (decltype(pre)::value) {
            if constexpr (!PRE_ST1) gather_block<CBT, S2, GPL, IT, false, true>(a, cd, ce0);
            dot_block<CBT, S2, GPL, BT, IT>(s_cb1, cd, ce0, valid, xs, acc);
        } else {
            block_dot<CBT, S2, GPL, BT, IT>(a, s_cb1, cd, valid, xs, acc);
        }
#pragma unroll
        for (int it = 0; it < IT; it++)
#pragma unroll
            for (int b = 0; b < BT; b++) acc[it][b] = group_sum(acc[it][b], lpr);

        const int si = seg_of(a, rbg);
        const GemvSeg& sg = a.seg[si];
        const int64_t row_base = (rbg - sg.rb_start) * rows_per_block;
        const float pw = a.pair_w ? uniform_load<float>(a.pair_w, pair) : 1.0f;
#pragma unroll
        for (int it = 0; it < IT; it++) {
            const int64_t row = row_base + (int64_t)(it * wr + wr_id) * rpw + sub;
            const float sc = row < sg.out_rows ? cd.scale(it, a.s_dt) : 0.0f;
#pragma unroll
            for (int b = 0; b < BT; b++) {
                float v = (acc[it][b] * sc) * a.rs;
                if (bad) v = __builtin_nanf("");
                fin[it][b] = fmaf(pw, v, fin[it][b]);
            }
        }

        if (nitem == wi_id) {
            // the wave's last item of this row block: reduce and store
            if (wi == 1) {
                if (col == 0) {
#pragma unroll
                    for (int it = 0; it < IT; it++) {
                        const int64_t row = row_base + (int64_t)(it * wr + wr_id) * rpw + sub;
                        if (row >= sg.out_rows) continue;
#pragma unroll
                        for (int b = 0; b < BT; b++)
                            if (b < nb) {
                                const int64_t yi = (int64_t)og * a.y_ostride + (int64_t)(bt0 + b) * sg.y_bstride + row;
                                float v = fin[it][b];
                                if constexpr (XM == 2)
                                    if (a.y_acc) v = load_as_f32(sg.y, a.y_dt, yi) + v;
                                store_from_f32(sg.y, a.y_dt, yi, v);
                            }
                    }
                }
            } else {
                if (col == 0) {
#pragma unroll
                    for (int it = 0; it < IT; it++) {
                        const int lr = (it * wr + wr_id) * rpw + sub;
#pragma unroll
                        for (int b = 0; b < BT; b++) s_part[(wi_id * rows_per_block + lr) * BT + b] = fin[it][b];
                    }
                }
                __syncthreads();
                for (int t = threadIdx.x; t < rows_per_block * BT; t += blockDim.x) {
                    const int lr = t / BT, b = t % BT;
                    const int64_t row = row_base + lr;
                    float sum = s_part[lr * BT + b];
                    for (int w = 1; w < wi; w++) sum += s_part[(w * rows_per_block + lr) * BT + b];
                    if (row < sg.out_rows && b < nb) {
                        const int64_t yi = (int64_t)og * a.y_ostride + (int64_t)(bt0 + b) * sg.y_bstride + row;
                        if constexpr (XM == 2)
                            if (a.y_acc) sum = load_as_f32(sg.y, a.y_dt, yi) + sum;
                        store_from_f32(sg.y, a.y_dt, yi, sum);
                    }
                }
                __syncthreads();
            }
#pragma unroll
            for (int it = 0; it < IT; it++)
#pragma unroll
                for (int b = 0; b < BT; b++) fin[it][b] = 0.0f;
        }
#pragma unroll
        for (int it = 0; it < IT; it++) valid[it] = nvalid[it];
        cd = nx;
        item = nitem;
        rbg = nrbg;
    };
    if constexpr (PRE && !AHEAD) mstep(std::true_type{});
    while (rbg < a.n_rowblocks) mstep(std::false_type{});
}

// Generic path for shapes the vector kernel does not take (activations are
// pre-rotated, XM 0 only): one thread per (output group, batch column, row)
// of one segment, scalar loads, same arithmetic.
template <int CBT>
__global__ void __launch_bounds__(256) vq_gemv_generic(const GemvArgs a, int s2, int si)
{
    const GemvSeg& sg = a.seg[si];
    for (int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; t < a.batch * sg.out_rows;
         t += (int64_t)gridDim.x * blockDim.x) {
        const int64_t og = blockIdx.y;
        const int64_t b = t / sg.out_rows, row = t - (t / sg.out_rows) * sg.out_rows;
        float out = 0.0f;
        for (int pj = 0; pj < a.P; pj++) {
            const int64_t pair = og * a.P + pj;
            bool bad;
            const int64_t e = pair_expert(a, pair, bad);
            const int64_t xoff = (pair / a.x_pdiv) * a.x_pstride + b * a.x_bstride;
            float acc = 0.0f;
            if (!bad) {
                for (int64_t g = 0; g < a.ng; g++) {
                    const int64_t i = e * a.e_istride + row * a.ng + g;
                    const uint32_t c0 = (uint16_t)sg.idx0[i];
                    uint32_t c1 = 0;
                    if (s2 == VQ2_S2_U8) c1 = ((const uint8_t*)sg.idx1)[i];
                    if (s2 == VQ2_S2_U16) c1 = (uint16_t)((const int16_t*)sg.idx1)[i];
                    for (int j = 0; j < 8; j++) {
                        float w = load_as_f32(a.cb0, CBT, (int64_t)c0 * 8 + j);
                        if (s2 != VQ2_S2_NONE) w += load_as_f32(a.cb1, CBT, (int64_t)c1 * 8 + j);
                        acc = fmaf(w, load_as_f32(a.x, a.x_dt, xoff + g * 8 + j), acc);
                    }
                }
            }
            const float s = load_as_f32(sg.scale, a.s_dt, e * a.e_sstride + row);
            float v = (acc * s) * a.rs;
            if (bad) v = __builtin_nanf("");
            const float pw = a.pair_w ? uniform_load<float>(a.pair_w, pair) : 1.0f;
            out = (a.P == 1) ? v : fmaf(pw, v, out);
        }
        store_from_f32(sg.y, a.y_dt, og * a.y_ostride + b * sg.y_bstride + row, out);
    }
}

// ------------------------------------------------------------------- host
struct GemvPlan {
    int gpl, bt, lpr, wi, wr, it, xm, num_cu;
    double occ_scale;  // multiplier on the resident-workgroup count
    int64_t rows_per_block, n_rowblocks;
    int threads;
    int ep;                 // epilogue (0 store, 1 fused top-1)
    unsigned* grid_x_out;   // receives the launched grid.x (may be null)
};

// Resident workgroups per CU of a kernel at a block size / LDS size (cached).
int resident_blocks_per_cu(const void* fn, int threads, size_t shm);

// Persistent grid: as many row-block workers as stay resident on the GPU
// (rounded down over the grid.y * grid.z output groups: a workgroup beyond
// the resident count would start only when another ends, a whole row block
// late).
inline dim3 persistent_grid(const void* fn, const GemvPlan& p, dim3 grid, size_t shm)
{
    const int64_t resident = (int64_t)resident_blocks_per_cu(fn, p.threads, shm) * p.num_cu * p.occ_scale;
    const int64_t per_x = resident / ((int64_t)grid.y * grid.z);
    int64_t gx = per_x < 1 ? 1 : per_x;
    if (gx > p.n_rowblocks) gx = p.n_rowblocks;
    grid.x = (unsigned)gx;
    return grid;
}

template <int CBT, int S2, int GPL, int BT, int IT, int XM, int EP = 0, int XT = VQ2_DT_F32>
inline hipError_t launch_one(const GemvArgs& a, const GemvPlan& p, dim3 grid, size_t shm, hipStream_t st)
{
    const void* fn = (const void*)vq_gemv_kernel<CBT, S2, GPL, BT, IT, XM, EP, XT>;
    grid = persistent_grid(fn, p, grid, shm);
    if (p.grid_x_out) *p.grid_x_out = grid.x;
    // packed scalar arguments (ranges checked by gemv_launch)
    const uint32_t fast = a.nseg == 1 && a.ids == nullptr ? 1u : 0u;
    const uint32_t plan = (uint32_t)a.lpr | ((uint32_t)a.wi << 6) | ((uint32_t)p.wr << 10) | (fast << 14);
    const uint32_t nchp = (uint32_t)a.nch | ((uint32_t)a.P << 16);
    hipLaunchKernelGGL((vq_gemv_kernel<CBT, S2, GPL, BT, IT, XM, EP, XT>), grid, dim3(p.threads), shm, st, (int)a.ng,
                       (int)a.n_rowblocks, plan, nchp, a.seg[0].idx0, a.seg[0].idx1, (int)a.seg[0].out_rows, a);
    return hipGetLastError();
}

// prologue kernels, one instantiation per activation dtype
template <int CBT, int S2, int GPL, int BT, int IT, int XM>
inline hipError_t launch_xt(const GemvArgs& a, const GemvPlan& p, dim3 grid, size_t shm, hipStream_t st)
{
    switch (a.x_dt) {
    case VQ2_DT_F16: return launch_one<CBT, S2, GPL, BT, IT, XM, 0, VQ2_DT_F16>(a, p, grid, shm, st);
    case VQ2_DT_BF16: return launch_one<CBT, S2, GPL, BT, IT, XM, 0, VQ2_DT_BF16>(a, p, grid, shm, st);
    default: return launch_one<CBT, S2, GPL, BT, IT, XM, 0, VQ2_DT_F32>(a, p, grid, shm, st);
    }
}

template <int CBT, int S2, int GPL, int BT, int IT>
inline hipError_t launch_xm(const GemvArgs& a, const GemvPlan& p, dim3 grid, size_t shm, hipStream_t st)
{
    switch (p.xm) {
    case 1:
        if constexpr (BT <= 2) return launch_xt<CBT, S2, GPL, BT, IT, 1>(a, p, grid, shm, st);
        else return hipErrorInvalidValue;
    case 2:
        if constexpr (S2 != VQ2_S2_U16 && BT == 1) return launch_xt<CBT, S2, GPL, BT, IT, 2>(a, p, grid, shm, st);
        else return hipErrorInvalidValue;
    case 3:
        if constexpr (S2 == VQ2_S2_NONE && BT == 1) return launch_xt<CBT, S2, GPL, BT, IT, 3>(a, p, grid, shm, st);
        else return hipErrorInvalidValue;
    case 4:
        if constexpr (BT <= 2) return launch_xt<CBT, S2, GPL, BT, IT, 4>(a, p, grid, shm, st);
        else return hipErrorInvalidValue;
    default:
        if (p.ep == 1) {
            if constexpr (BT == 1 && IT == 1) return launch_one<CBT, S2, GPL, BT, IT, 0, 1>(a, p, grid, shm, st);
            else return hipErrorInvalidValue;
        }
        return launch_one<CBT, S2, GPL, BT, IT, 0>(a, p, grid, shm, st);
    }
}

// rows per lane: 2 for the 8-column batch tile (its lanes hold one code per
// row), else 1 -- measured on MI355X over the decode shapes
template <int BT>
constexpr int gemv_it() { return BT == 8 ? 2 : 1; }

template <int CBT, int S2, int GPL, int BT>
inline hipError_t launch_it(const GemvArgs& a, const GemvPlan& p, dim3 grid, size_t shm, hipStream_t st)
{
    if (p.it != gemv_it<BT>()) return hipErrorInvalidValue;
    return launch_xm<CBT, S2, GPL, BT, gemv_it<BT>()>(a, p, grid, shm, st);
}

template <int CBT, int S2>
inline hipError_t launch_bt(const GemvArgs& a, const GemvPlan& p, dim3 grid, size_t shm, hipStream_t st)
{
    switch (p.bt) {
    case 1: return launch_it<CBT, S2, 8, 1>(a, p, grid, shm, st);
    case 2: return launch_it<CBT, S2, 4, 2>(a, p, grid, shm, st);
    case 4: return launch_it<CBT, S2, 2, 4>(a, p, grid, shm, st);
    default: return launch_it<CBT, S2, 1, 8>(a, p, grid, shm, st);
    }
}

template <int CBT>
inline hipError_t launch_s2(int s2, const GemvArgs& a, const GemvPlan& p, dim3 grid, size_t shm, hipStream_t st)
{
    switch (s2) {
    case VQ2_S2_U8: return launch_bt<CBT, VQ2_S2_U8>(a, p, grid, shm, st);
    case VQ2_S2_U16: return launch_bt<CBT, VQ2_S2_U16>(a, p, grid, shm, st);
    default: return launch_bt<CBT, VQ2_S2_NONE>(a, p, grid, shm, st);
    }
}

template <int CBT>
inline hipError_t launch_generic(int s2, int si, const GemvArgs& a, dim3 grid, hipStream_t st)
{
    hipLaunchKernelGGL((vq_gemv_generic<CBT>), grid, dim3(256), 0, st, a, s2, si);
    return hipGetLastError();
}

// per-codebook-dtype dispatchers (one translation unit each)
hipError_t gemv_dispatch_f16(int s2, const GemvArgs& a, const GemvPlan& p, dim3 grid, size_t shm, hipStream_t st);
hipError_t gemv_dispatch_bf16(int s2, const GemvArgs& a, const GemvPlan& p, dim3 grid, size_t shm, hipStream_t st);
hipError_t gemv_dispatch_f32(int s2, const GemvArgs& a, const GemvPlan& p, dim3 grid, size_t shm, hipStream_t st);
hipError_t gemv_generic_dispatch(int cb_dt, int s2, int si, const GemvArgs& a, dim3 grid, hipStream_t st);

}  // namespace vq2
