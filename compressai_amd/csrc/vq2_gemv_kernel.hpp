// vq2_gemv_kernel.hpp -- vector-quantized GEMV kernel body for gfx950 (CDNA4, wave64).
//
// One kernel body serves three call shapes of the decode path:
//   dense    y[b, r]      = VQ(W) x_b                                   (P = 1, no ids)
//   grouped  y[k, r]      = VQ(W_{ids[k]}) x_k                          (P = 1, ids)
//   combine  out[t, r]    = sum_j w[t*P+j] * VQ(W_{ids[t*P+j]}) x_{t*P+j} (P > 1)
// with VQ(W)[r, 8g+j] = (cb0[i0[r,g]] [+ cb1[i1[r,g]]])[j], the row scale and
// rs applied after fp32 accumulation: y = (acc * s[r]) * rs.
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
//     16-byte index words -> fully coalesced, non-temporal index streams;
//   * every index triggers one 16-byte centroid gather (the 1 MiB codebook is
//     L2-resident); the (16,8) stage-2 codebook (256 x 8) is staged in LDS;
//   * WK waves split K (one K-chunk each) and reduce through LDS in a fixed
//     order (deterministic split-K inside the workgroup);
//   * row partials are reduced across the LPR lanes with DPP/swizzle.
#pragma once
#include "vq2_common.hpp"
#include "vq2_internal.hpp"

namespace vq2 {

struct GemvArgs {
    const void* x;
    int x_dt;
    int x_vec;          // 1: x rows are 16-byte aligned -> vector loads
    int64_t x_bstride;  // elements between batch columns
    int64_t x_pstride;  // elements between x blocks of consecutive pair groups
    int x_pdiv;         // pair p uses x block p / x_pdiv
    const int16_t* idx0;
    const void* idx1;
    const void* cb0;
    const void* cb1;
    const void* scale;
    int s_dt;
    int64_t e_istride;  // elements between experts in the index planes
    int64_t e_sstride;  // elements between experts in the scale array
    const void* ids;
    int ids_i64;
    int64_t n_experts;
    const float* pair_w;  // per-pair combine weights (P > 1), may be null
    int P;                // pairs per output group
    void* y;
    int y_dt;
    int64_t y_bstride;
    int64_t y_ostride;
    int64_t out_rows;
    int64_t ng;
    int batch;
    float rs;
    int lpr;  // lanes per row (power of two <= 32)
    int wk;   // waves along K
    int vec_ok;  // index planes allow GPL-wide vector loads
    int64_t n_rowblocks;
};

template <int CBT>
struct Centroid;

// fp16 codebook: one 16-byte gather, converted inside the FMA (v_fma_mix).
template <>
struct Centroid<VQ2_DT_F16> {
    half8_t h;
    __device__ __forceinline__ void load(const void* cb, uint32_t code)
    {
        h = *((const half8_t*)cb + code);
    }
    __device__ __forceinline__ float get(int j) const { return (float)h[j]; }
};

template <>
struct Centroid<VQ2_DT_BF16> {
    uint4 u;
    __device__ __forceinline__ void load(const void* cb, uint32_t code) { u = *((const uint4*)cb + code); }
    __device__ __forceinline__ float get(int j) const
    {
        uint32_t w = (j >> 1) == 0 ? u.x : (j >> 1) == 1 ? u.y : (j >> 1) == 2 ? u.z : u.w;
        return (j & 1) ? __uint_as_float(w & 0xFFFF0000u) : __uint_as_float(w << 16);
    }
};

template <>
struct Centroid<VQ2_DT_F32> {
    float4 a, b;
    __device__ __forceinline__ void load(const void* cb, uint32_t code)
    {
        const float4* p = (const float4*)cb + 2 * (size_t)code;
        a = p[0];
        b = p[1];
    }
    __device__ __forceinline__ float get(int j) const
    {
        switch (j) {
        case 0: return a.x;
        case 1: return a.y;
        case 2: return a.z;
        case 3: return a.w;
        case 4: return b.x;
        case 5: return b.y;
        case 6: return b.z;
        default: return b.w;
        }
    }
};

// Stage-2 centroid from the LDS copy of a 256-row codebook.
template <int CBT>
__device__ __forceinline__ Centroid<CBT> lds_centroid(const uint4* s_cb1, uint32_t code)
{
    Centroid<CBT> c;
    if constexpr (CBT == VQ2_DT_F32) {
        uint4 a = s_cb1[2 * code], b = s_cb1[2 * code + 1];
        c.a = make_float4(__uint_as_float(a.x), __uint_as_float(a.y), __uint_as_float(a.z), __uint_as_float(a.w));
        c.b = make_float4(__uint_as_float(b.x), __uint_as_float(b.y), __uint_as_float(b.z), __uint_as_float(b.w));
    } else if constexpr (CBT == VQ2_DT_F16) {
        uint4 a = s_cb1[code];
        c.h = __builtin_bit_cast(half8_t, a);
    } else {
        c.u = s_cb1[code];
    }
    return c;
}

// Load GPL uint16 codes of plane 0 (int16 storage) starting at element off.
template <int GPL>
__device__ __forceinline__ void load_codes16(const int16_t* p, int64_t off, uint32_t (&c)[GPL])
{
    const int16_t* q = p + off;
    if constexpr (GPL == 8) {
        u32x4 v = __builtin_nontemporal_load((const u32x4*)q);
        c[0] = v.x & 0xFFFFu; c[1] = v.x >> 16; c[2] = v.y & 0xFFFFu; c[3] = v.y >> 16;
        c[4] = v.z & 0xFFFFu; c[5] = v.z >> 16; c[6] = v.w & 0xFFFFu; c[7] = v.w >> 16;
    } else if constexpr (GPL == 4) {
        u32x2 v = __builtin_nontemporal_load((const u32x2*)q);
        c[0] = v.x & 0xFFFFu; c[1] = v.x >> 16; c[2] = v.y & 0xFFFFu; c[3] = v.y >> 16;
    } else if constexpr (GPL == 2) {
        uint32_t v = __builtin_nontemporal_load((const uint32_t*)q);
        c[0] = v & 0xFFFFu; c[1] = v >> 16;
    } else {
        c[0] = (uint32_t)(uint16_t)__builtin_nontemporal_load(q);
    }
}

template <int GPL>
__device__ __forceinline__ void load_codes8(const uint8_t* p, int64_t off, uint32_t (&c)[GPL])
{
    const uint8_t* q = p + off;
    if constexpr (GPL == 8) {
        u32x2 v = __builtin_nontemporal_load((const u32x2*)q);
#pragma unroll
        for (int i = 0; i < 4; i++) {
            c[i] = (v.x >> (8 * i)) & 0xFFu;
            c[4 + i] = (v.y >> (8 * i)) & 0xFFu;
        }
    } else if constexpr (GPL == 4) {
        uint32_t v = __builtin_nontemporal_load((const uint32_t*)q);
#pragma unroll
        for (int i = 0; i < 4; i++) c[i] = (v >> (8 * i)) & 0xFFu;
    } else {
#pragma unroll
        for (int i = 0; i < GPL; i++) c[i] = q[i];
    }
}

// Load this lane's activation slice: groups [g0, g0+GPL) for nb batch
// columns, as fp32.  Groups at or beyond ng read as zero.
template <int GPL, int BT>
__device__ __forceinline__ void load_x(const GemvArgs& a, const void* xb, int64_t g0, int nb, float (&xs)[BT][GPL * 8])
{
#pragma unroll
    for (int b = 0; b < BT; b++) {
        if (b < nb) {
            const int64_t base = (int64_t)b * a.x_bstride + g0 * 8;
            if (a.x_vec && g0 + GPL <= a.ng) {
                if (a.x_dt == VQ2_DT_F32) {
                    const float4* p = (const float4*)((const float*)xb + base);
#pragma unroll
                    for (int i = 0; i < GPL * 2; i++) {
                        float4 v = p[i];
                        xs[b][4 * i] = v.x; xs[b][4 * i + 1] = v.y; xs[b][4 * i + 2] = v.z; xs[b][4 * i + 3] = v.w;
                    }
                } else {
                    const uint4* p = (const uint4*)((const uint16_t*)xb + base);
                    const bool bf = a.x_dt == VQ2_DT_BF16;
#pragma unroll
                    for (int i = 0; i < GPL; i++) {
                        uint4 v = p[i];
                        uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
                        for (int k = 0; k < 4; k++) {
                            if (bf) {
                                xs[b][8 * i + 2 * k] = __uint_as_float(w[k] << 16);
                                xs[b][8 * i + 2 * k + 1] = __uint_as_float(w[k] & 0xFFFF0000u);
                            } else {
                                xs[b][8 * i + 2 * k] = f16_bits_to_f32((uint16_t)(w[k] & 0xFFFFu));
                                xs[b][8 * i + 2 * k + 1] = f16_bits_to_f32((uint16_t)(w[k] >> 16));
                            }
                        }
                    }
                }
            } else {
#pragma unroll
                for (int i = 0; i < GPL * 8; i++) {
                    const int64_t g = g0 + i / 8;
                    xs[b][i] = g < a.ng ? load_as_f32(xb, a.x_dt, base + i) : 0.0f;
                }
            }
        } else {
#pragma unroll
            for (int i = 0; i < GPL * 8; i++) xs[b][i] = 0.0f;
        }
    }
}

template <int CBT, int S2, int GPL, int BT, int IT>
__global__ void __launch_bounds__(256) vq_gemv_kernel(const GemvArgs a)
{
    // stage-2 (uint8) codebook in LDS: 256 rows x 16 B (x2 for fp32)
    __shared__ uint4 s_cb1[S2 == VQ2_S2_U8 ? (CBT == VQ2_DT_F32 ? 512 : 256) : 1];
    extern __shared__ float s_part[];

    if constexpr (S2 == VQ2_S2_U8) {
        const int nent = CBT == VQ2_DT_F32 ? 512 : 256;
        for (int i = threadIdx.x; i < nent; i += blockDim.x) s_cb1[i] = ((const uint4*)a.cb1)[i];
        __syncthreads();
    }

    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int lpr = a.lpr, wk = a.wk;
    const int wr = (blockDim.x >> 6) / wk;
    const int wk_id = wave % wk, wr_id = wave / wk;
    const int rpw = 64 / lpr;
    const int sub = lane / lpr, col = lane % lpr;
    const int64_t kc = (int64_t)lpr * GPL;
    const int64_t nch = (a.ng + kc - 1) / kc;
    const int rows_per_iter = IT * rpw * wr;
    const int og = blockIdx.y;
    const int bt0 = blockIdx.z * BT;
    const int nb = min(BT, a.batch - bt0);
    const bool use_lds = (wk > 1) || (a.P > 1);
    const int nfin = rows_per_iter * BT;  // finalize slots, <= blockDim.x (host-checked)

    // x stays resident across row blocks when a wave owns exactly one chunk
    // of one pair's activation.
    const bool x_resident = (a.P == 1) && (nch <= wk);

    float xs[BT][GPL * 8];
    int64_t x_c = -1;  // chunk currently in xs
    int x_pair = -1;

    for (int64_t rb = blockIdx.x; rb < a.n_rowblocks; rb += gridDim.x) {
        const int64_t row_base = rb * rows_per_iter;
        float fin = 0.0f;  // combine accumulator of finalize slot threadIdx.x

        for (int pj = 0; pj < a.P; pj++) {
            const int64_t pair = (int64_t)og * a.P + pj;
            int64_t e = 0;
            if (a.ids) e = a.ids_i64 ? ((const int64_t*)a.ids)[pair] : (int64_t)((const int32_t*)a.ids)[pair];
            const bool bad = a.ids && (e < 0 || e >= a.n_experts);
            if (bad) e = 0;
            const int16_t* I0 = a.idx0 + e * a.e_istride;
            const void* I1 = nullptr;
            if constexpr (S2 == VQ2_S2_U8) I1 = (const uint8_t*)a.idx1 + e * a.e_istride;
            if constexpr (S2 == VQ2_S2_U16) I1 = (const int16_t*)a.idx1 + e * a.e_istride;
            const int64_t xoff = (pair / a.x_pdiv) * a.x_pstride + (int64_t)bt0 * a.x_bstride;
            const void* xb = a.x_dt == VQ2_DT_F32 ? (const void*)((const float*)a.x + xoff)
                                                  : (const void*)((const uint16_t*)a.x + xoff);

            float acc[IT][BT];
#pragma unroll
            for (int it = 0; it < IT; it++)
#pragma unroll
                for (int b = 0; b < BT; b++) acc[it][b] = 0.0f;

            for (int64_t c = wk_id; c < nch; c += wk) {
                const int64_t g0 = c * kc + (int64_t)col * GPL;
                if (!(x_resident && x_c == c && x_pair == (int)pair)) {
                    load_x<GPL, BT>(a, xb, g0, nb, xs);
                    x_c = c;
                    x_pair = (int)pair;
                }
                if (bad) continue;
                const bool full = a.vec_ok && (g0 + GPL <= a.ng);

                uint32_t c0[IT][GPL], c1[IT][GPL];
                bool valid[IT];
#pragma unroll
                for (int it = 0; it < IT; it++) {
                    const int64_t row = row_base + (int64_t)(it * wr + wr_id) * rpw + sub;
                    valid[it] = row < a.out_rows && g0 < a.ng;
                    const int64_t off = row * a.ng + g0;
#pragma unroll
                    for (int q = 0; q < GPL; q++) { c0[it][q] = 0; c1[it][q] = 0; }
                    if (valid[it]) {
                        if (full) {
                            load_codes16<GPL>(I0, off, c0[it]);
                            if constexpr (S2 == VQ2_S2_U8) load_codes8<GPL>((const uint8_t*)I1, off, c1[it]);
                            if constexpr (S2 == VQ2_S2_U16) load_codes16<GPL>((const int16_t*)I1, off, c1[it]);
                        } else {
#pragma unroll
                            for (int q = 0; q < GPL; q++) {
                                if (g0 + q < a.ng) {
                                    c0[it][q] = (uint16_t)I0[off + q];
                                    if constexpr (S2 == VQ2_S2_U8) c1[it][q] = ((const uint8_t*)I1)[off + q];
                                    if constexpr (S2 == VQ2_S2_U16) c1[it][q] = (uint16_t)((const int16_t*)I1)[off + q];
                                }
                            }
                        }
                    }
                }

#pragma unroll
                for (int it = 0; it < IT; it++) {
                    if (!valid[it]) continue;
                    Centroid<CBT> cen[GPL];
#pragma unroll
                    for (int q = 0; q < GPL; q++) cen[q].load(a.cb0, c0[it][q]);
                    if constexpr (S2 == VQ2_S2_U16) {
                        Centroid<CBT> cen1[GPL];
#pragma unroll
                        for (int q = 0; q < GPL; q++) cen1[q].load(a.cb1, c1[it][q]);
#pragma unroll
                        for (int q = 0; q < GPL; q++) {
                            if (!full && g0 + q >= a.ng) continue;
#pragma unroll
                            for (int j = 0; j < 8; j++) {
                                const float w = cen[q].get(j) + cen1[q].get(j);
#pragma unroll
                                for (int b = 0; b < BT; b++) acc[it][b] = fmaf(w, xs[b][q * 8 + j], acc[it][b]);
                            }
                        }
                    } else if constexpr (S2 == VQ2_S2_U8) {
#pragma unroll
                        for (int q = 0; q < GPL; q++) {
                            if (!full && g0 + q >= a.ng) continue;
                            const Centroid<CBT> c2 = lds_centroid<CBT>(s_cb1, c1[it][q]);
#pragma unroll
                            for (int j = 0; j < 8; j++) {
                                const float w = cen[q].get(j) + c2.get(j);
#pragma unroll
                                for (int b = 0; b < BT; b++) acc[it][b] = fmaf(w, xs[b][q * 8 + j], acc[it][b]);
                            }
                        }
                    } else {
#pragma unroll
                        for (int q = 0; q < GPL; q++) {
                            if (!full && g0 + q >= a.ng) continue;
#pragma unroll
                            for (int j = 0; j < 8; j++) {
                                const float w = cen[q].get(j);
#pragma unroll
                                for (int b = 0; b < BT; b++) acc[it][b] = fmaf(w, xs[b][q * 8 + j], acc[it][b]);
                            }
                        }
                    }
                }
            }

            // reduce row partials over the LPR lanes of each row
#pragma unroll
            for (int it = 0; it < IT; it++)
#pragma unroll
                for (int b = 0; b < BT; b++) acc[it][b] = group_sum(acc[it][b], lpr);

            const float pw = a.pair_w ? a.pair_w[pair] : 1.0f;
            if (!use_lds) {
                if (col == 0) {
#pragma unroll
                    for (int it = 0; it < IT; it++) {
                        const int64_t row = row_base + (int64_t)(it * wr + wr_id) * rpw + sub;
                        if (row >= a.out_rows) continue;
                        const float s = load_as_f32(a.scale, a.s_dt, e * a.e_sstride + row);
#pragma unroll
                        for (int b = 0; b < BT; b++) {
                            if (b >= nb) continue;
                            float v = (acc[it][b] * s) * a.rs;
                            if (bad) v = __builtin_nanf("");
                            store_from_f32(a.y, a.y_dt, (int64_t)og * a.y_ostride + (int64_t)(bt0 + b) * a.y_bstride + row, v);
                        }
                    }
                }
            } else {
                // partials: s_part[wk_id][local_row][b]
                if (col == 0) {
#pragma unroll
                    for (int it = 0; it < IT; it++) {
                        const int lr = (it * wr + wr_id) * rpw + sub;
#pragma unroll
                        for (int b = 0; b < BT; b++) s_part[(wk_id * rows_per_iter + lr) * BT + b] = acc[it][b];
                    }
                }
                __syncthreads();
                if ((int)threadIdx.x < nfin) {
                    const int lr = threadIdx.x / BT, b = threadIdx.x % BT;
                    const int64_t row = row_base + lr;
                    float sum = 0.0f;
                    for (int w = 0; w < wk; w++) sum += s_part[(w * rows_per_iter + lr) * BT + b];
                    if (row < a.out_rows) {
                        const float s = load_as_f32(a.scale, a.s_dt, e * a.e_sstride + row);
                        float v = (sum * s) * a.rs;
                        if (bad) v = __builtin_nanf("");
                        fin = (pj == 0) ? pw * v : fmaf(pw, v, fin);
                    }
                }
                __syncthreads();
            }
        }

        if (use_lds && (int)threadIdx.x < nfin) {
            const int lr = threadIdx.x / BT, b = threadIdx.x % BT;
            const int64_t row = row_base + lr;
            if (row < a.out_rows && b < nb) {
                // P == 1 keeps the plain (acc * s) * rs value (pw == 1)
                store_from_f32(a.y, a.y_dt, (int64_t)og * a.y_ostride + (int64_t)(bt0 + b) * a.y_bstride + row, fin);
            }
        }
    }
}

// ------------------------------------------------------------------- host
struct GemvPlan {
    int gpl, bt, lpr, wk, wr, it;
    int64_t rows_per_iter, n_rowblocks;
    int threads;
};

template <int CBT, int S2, int GPL, int BT>
inline hipError_t launch_it(const GemvArgs& a, const GemvPlan& p, dim3 grid, size_t shm, hipStream_t st)
{
    switch (p.it) {
    case 4: hipLaunchKernelGGL((vq_gemv_kernel<CBT, S2, GPL, BT, 4>), grid, dim3(p.threads), shm, st, a); break;
    case 2: hipLaunchKernelGGL((vq_gemv_kernel<CBT, S2, GPL, BT, 2>), grid, dim3(p.threads), shm, st, a); break;
    default: hipLaunchKernelGGL((vq_gemv_kernel<CBT, S2, GPL, BT, 1>), grid, dim3(p.threads), shm, st, a); break;
    }
    return hipGetLastError();
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

// per-codebook-dtype dispatchers (one translation unit each)
hipError_t gemv_dispatch_f16(int s2, const GemvArgs& a, const GemvPlan& p, dim3 grid, size_t shm, hipStream_t st);
hipError_t gemv_dispatch_bf16(int s2, const GemvArgs& a, const GemvPlan& p, dim3 grid, size_t shm, hipStream_t st);
hipError_t gemv_dispatch_f32(int s2, const GemvArgs& a, const GemvPlan& p, dim3 grid, size_t shm, hipStream_t st);

}  // namespace vq2
