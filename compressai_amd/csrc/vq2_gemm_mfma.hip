// vq2_gemm_mfma.hip -- small-M batched VQ GEMM on the gfx950 matrix cores.
//
//   y[b, r] = (sum_k x[b, k] * W[r, k]) * s[r] * rs,   b < M (1..64),
//   W[r, 8g + j] = cb0[i0[r, g]][j] (+ cb1[i1[r, g]][j]),  x already rotated.
//
// The batched GEMV gathers every centroid once per 8-column batch tile, so at
// M = 64 each code costs eight L2 gathers.  Here each centroid is gathered
// once and fed as fp16 to v_mfma_f32_16x16x32_f16 for all M rows:
//
//  * Operand layout of v_mfma_f32_16x16x32_f16: lane l holds 8 consecutive k
//    of row (l % 16) of A and of column (l % 16) of B, k block l / 16; the
//    result D[i][j] sits in lane j + 16 * (i / 4), element i % 4.  A VQ
//    centroid is exactly 8 consecutive k of one weight row, so a lane's B
//    operand is one 16-byte gather, with no shuffles.
//  * Inside a tile the k <-> group assignment is free (A and B only have to
//    agree), so lane (n = l % 16, q = l / 16) takes the 8 consecutive groups
//    [8q, 8q + 8) of its row with one 16-byte index load (4 lanes x 16 B =
//    64 contiguous bytes per row), and k-step t uses group 8q + t.
//  * A is the activation, staged in LDS as fp16 with a power-of-two scale per
//    (row, split): fp16 then holds any fp32 range at full fp16 precision, and
//    the scale is divided out of the fp32 partial exactly (fp16 activations
//    are copied as they are).  fp16 codebooks
//    are used as they are; bf16 / fp32 centroids are rounded to fp16.  The
//    accumulation is fp32.
//  * A workgroup is 4 waves x 16 output rows over one K split; the split
//    count is chosen so that the grid fills the device.  With more than one
//    split the raw partials go to a workspace and a second launch sums them in
//    split order (deterministic) and applies s * rs.
//
// Semantics: the PackedLinear fallback for batch > 1, dequantize then
// F.linear (vq2/runtime.py:82-89, 105-110), for the (16,), (16,8) and (16,16)
// index configurations.
#include <stdlib.h>

#include <mutex>

#include "vq2_gemv_kernel.hpp"

namespace vq2 {

typedef float f32x4_t __attribute__((ext_vector_type(4)));

constexpr int MM_WAVES = 4;
constexpr int MM_THREADS = 64 * MM_WAVES;
constexpr int MM_ROWS = 16 * MM_WAVES;  // output rows per workgroup
constexpr int MM_TILE_G = 32;           // groups per index tile: 4 k blocks x 8 codes per lane
constexpr int MM_STAGE = 8;             // activation groups staged per thread
constexpr int MM_MAX_XG = MM_STAGE * MM_THREADS;  // M_pad * kcg groups per workgroup
constexpr int MM_MAX_M = 64;

struct GemmArgs {
    const void* x;
    int x_dt;
    int64_t x_stride;
    int m;
    const int16_t* idx0;
    const void* idx1;
    const void* cb0;
    const void* cb1;
    const void* scale;
    int s_dt;
    void* y;
    int y_dt;
    int64_t y_stride;
    int64_t out_rows;
    int64_t ng;
    float rs;
    int kcg;     // groups per K split (multiple of 32)
    int splits;  // K splits (grid.y)
    float* part; // [splits][m][out_rows] raw partials when splits > 1 or to_part
    int to_part;     // write raw partials even with one split (fused top-1)
    uint64_t* cand;  // fused top-1: [gridDim.x of the reduce][m] best keys
};

// One centroid as 8 fp16 values (the MFMA B operand).
template <int CBT>
__device__ __forceinline__ half8_t centroid_h8(const void* cb, uint32_t code)
{
    if constexpr (CBT == VQ2_DT_F16) {
        return *((const half8_t*)cb + code);
    } else if constexpr (CBT == VQ2_DT_BF16) {
        const u32x4 u = *((const u32x4*)cb + code);
        half8_t h;
#pragma unroll
        for (int k = 0; k < 4; k++) {
            h[2 * k] = (_Float16)__uint_as_float(u[k] << 16);
            h[2 * k + 1] = (_Float16)__uint_as_float(u[k] & 0xFFFF0000u);
        }
        return h;
    } else {
        const u32x4* p = (const u32x4*)cb + 2 * (size_t)code;
        const u32x4 lo = p[0], hi = p[1];
        half8_t h;
#pragma unroll
        for (int k = 0; k < 4; k++) {
            h[k] = (_Float16)__uint_as_float(lo[k]);
            h[4 + k] = (_Float16)__uint_as_float(hi[k]);
        }
        return h;
    }
}

// 8 consecutive activation values (16- or 32-byte aligned) as fp32.
__device__ __forceinline__ void load8_f32(const void* p, int dt, int64_t off, float (&v)[8])
{
    if (dt == VQ2_DT_F32) {
        const u32x4* q = (const u32x4*)((const float*)p + off);
        const u32x4 a = q[0], b = q[1];
#pragma unroll
        for (int k = 0; k < 4; k++) { v[k] = __uint_as_float(a[k]); v[4 + k] = __uint_as_float(b[k]); }
    } else {
        const u32x4 a = *(const u32x4*)((const uint16_t*)p + off);
#pragma unroll
        for (int k = 0; k < 4; k++) {
            if (dt == VQ2_DT_BF16) {
                v[2 * k] = __uint_as_float(a[k] << 16);
                v[2 * k + 1] = __uint_as_float(a[k] & 0xFFFF0000u);
            } else {
                v[2 * k] = f16_bits_to_f32((uint16_t)(a[k] & 0xFFFFu));
                v[2 * k + 1] = f16_bits_to_f32((uint16_t)(a[k] >> 16));
            }
        }
    }
}

template <int CBT, int S2, int MT>
__global__ void __launch_bounds__(MM_THREADS) vq_gemm_mfma_kernel(const GemmArgs a)
{
    touch_kernargs(a);
    constexpr int MP = MT * 16;
    extern __shared__ half8_t s_xh[];  // [MP][kcg + 1] activation groups (fp16, scaled)
    __shared__ uint32_t s_amax[MP];
    __shared__ int s_e[MP];
    __shared__ half8_t s_c1[S2 == VQ2_S2_U8 ? 256 : 1];

    const int tid = threadIdx.x;
    const int64_t g_begin = (int64_t)blockIdx.y * a.kcg;
    const int gcount = (int)(a.ng - g_begin < a.kcg ? a.ng - g_begin : a.kcg);  // multiple of 8
    const int xsg = a.kcg + 1;  // LDS row stride in groups (odd: rows start in different banks)

    if (tid < MP) s_amax[tid] = 0u;
    if constexpr (S2 == VQ2_S2_U8)
        for (int i = tid; i < 256; i += MM_THREADS) s_c1[i] = centroid_h8<CBT>(a.cb1, (uint32_t)i);
    __syncthreads();

    // stage this split's activation: thread owns groups tid + j * MM_THREADS
    // of the [MP][gcount] chunk (rows >= m are zero)
    const int tot = MP * gcount;
    if (a.x_dt == VQ2_DT_F16) {
        // fp16 activations are exact in fp16: copied as they are, scale 1
        const half8_t zero8 = {0, 0, 0, 0, 0, 0, 0, 0};
        for (int t = tid; t < tot; t += MM_THREADS) {
            const int mr = t / gcount, g = t - mr * gcount;
            s_xh[mr * xsg + g] =
                mr < a.m ? *(const half8_t*)((const _Float16*)a.x + (int64_t)mr * a.x_stride + (g_begin + g) * 8)
                         : zero8;
        }
        if (tid < MP) s_e[tid] = 0;
    } else {
    float v[MM_STAGE][8];
#pragma unroll
    for (int j = 0; j < MM_STAGE; j++) {
        const int t = tid + j * MM_THREADS;
        const int mr = t / gcount, g = t - mr * gcount;
        const bool ok = t < tot && mr < a.m;
        if (ok) {
            load8_f32(a.x, a.x_dt, (int64_t)mr * a.x_stride + (g_begin + g) * 8, v[j]);
            float am = 0.0f;
#pragma unroll
            for (int k = 0; k < 8; k++) am = fmaxf(am, fabsf(v[j][k]));
            // fmaxf skips NaN (it still reaches its output row through the
            // product); an infinite row keeps scale 1
            if (__float_as_uint(am) != 0u) atomicMax(&s_amax[mr], __float_as_uint(am));
        } else {
#pragma unroll
            for (int k = 0; k < 8; k++) v[j][k] = 0.0f;
        }
    }
    __syncthreads();
    if (tid < MP) {
        const uint32_t am = s_amax[tid];
        // scale so that the row maximum lands in [2^14, 2^15): exact, far below fp16's 65504
        s_e[tid] = (am != 0u && am < 0x7F800000u) ? 14 - ilogbf(__uint_as_float(am)) : 0;
    }
    __syncthreads();
#pragma unroll
    for (int j = 0; j < MM_STAGE; j++) {
        const int t = tid + j * MM_THREADS;
        if (t < tot) {
            const int mr = t / gcount, g = t - mr * gcount;
            const int e = s_e[mr];
            half8_t h;
#pragma unroll
            for (int k = 0; k < 8; k++) h[k] = (_Float16)ldexpf(v[j][k], e);
            s_xh[mr * xsg + g] = h;
        }
    }
    }
    __syncthreads();

    const int lane = tid & 63, wave = tid >> 6;
    const int nl = lane & 15, q = lane >> 4;
    const int64_t row = (int64_t)blockIdx.x * MM_ROWS + wave * 16 + nl;
    const bool row_ok = row < a.out_rows;
    const int64_t rowc = row_ok ? row : 0;
    const half8_t zero8 = {0, 0, 0, 0, 0, 0, 0, 0};

    f32x4_t acc[MT];
#pragma unroll
    for (int mt = 0; mt < MT; mt++) acc[mt] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};

    for (int gt = 0; gt < gcount; gt += MM_TILE_G) {
        const int gl = gt + q * 8;
        const bool g_ok = gl < gcount;
        const bool w_ok = g_ok && row_ok;
        const int64_t off = rowc * a.ng + g_begin + (g_ok ? gl : 0);
        Codes<S2, 8, 1> cd;
        load_codes<S2, 8, 1>(a.idx0, a.idx1, off, 0, cd);
        half8_t b0[8], b1[8];
#pragma unroll
        for (int t = 0; t < 8; t++) {
            b0[t] = centroid_h8<CBT>(a.cb0, cd.c0(0, t));
            if constexpr (S2 == VQ2_S2_U16) b1[t] = centroid_h8<CBT>(a.cb1, cd.c1(0, t));
            if constexpr (S2 == VQ2_S2_U8) b1[t] = s_c1[cd.c1(0, t)];
        }
#pragma unroll
        for (int t = 0; t < 8; t++) {
            const half8_t bb0 = w_ok ? b0[t] : zero8;
#pragma unroll
            for (int mt = 0; mt < MT; mt++) {
                const half8_t av = g_ok ? s_xh[(mt * 16 + nl) * xsg + gl + t] : zero8;
                acc[mt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(av, bb0, acc[mt], 0, 0, 0);
                if constexpr (S2 != VQ2_S2_NONE) {
                    const half8_t bb1 = w_ok ? b1[t] : zero8;
                    acc[mt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(av, bb1, acc[mt], 0, 0, 0);
                }
            }
        }
    }

    // D[i][j]: activation row mt * 16 + 4q + e, output row `row`
    if (!row_ok) return;
    const bool direct = a.splits == 1 && !a.to_part;
    const float s = direct ? load_as_f32(a.scale, a.s_dt, row) : 0.0f;
#pragma unroll
    for (int mt = 0; mt < MT; mt++) {
#pragma unroll
        for (int e = 0; e < 4; e++) {
            const int m = mt * 16 + q * 4 + e;
            if (m >= a.m) continue;
            const float p = ldexpf(acc[mt][e], -s_e[m]);
            if (direct)
                store_from_f32(a.y, a.y_dt, (int64_t)m * a.y_stride + row, (p * s) * a.rs);
            else
                a.part[((int64_t)blockIdx.y * a.m + m) * a.out_rows + row] = p;
        }
    }
}

// Sum of the splits' partials at element t in split order.  The loads go out
// eight at a time (indices clamped to the last split, so the loads need no
// branch) before the adds: a plain loop over a run-time split count issues
// them a few at a time, one memory round trip apart.
__device__ __forceinline__ float split_sum(const GemmArgs& a, int64_t t, int64_t pstride)
{
    float sum = 0.0f;
    for (int sp0 = 0; sp0 < a.splits; sp0 += 8) {
        float v[8];
#pragma unroll
        for (int k = 0; k < 8; k++) {
            const int sp = sp0 + k < a.splits ? sp0 + k : a.splits - 1;
            v[k] = __builtin_nontemporal_load(&a.part[sp * pstride + t]);
        }
#pragma unroll
        for (int k = 0; k < 8; k++)
            if (sp0 + k < a.splits) sum += v[k];
    }
    return sum;
}

// y[b, r] = (partials summed in split order) * s[r] * rs
__global__ void __launch_bounds__(256) vq_gemm_reduce_kernel(const GemmArgs a)
{
    const int64_t tot = (int64_t)a.m * a.out_rows;
    const int64_t pstride = (int64_t)a.m * a.out_rows;
    for (int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; t < tot; t += (int64_t)gridDim.x * blockDim.x) {
        const int64_t m = t / a.out_rows, row = t - m * a.out_rows;
        const float sum = split_sum(a, t, pstride);
        const float s = load_as_f32(a.scale, a.s_dt, row);
        store_from_f32(a.y, a.y_dt, m * a.y_stride + row, (sum * s) * a.rs);
    }
}

// Fused top-1 of every activation row m = blockIdx.y: the same split-order
// sum and (sum * s) * rs as vq_gemm_reduce_kernel, so the keys are those of
// the fp32 logits; each block keeps the best (value, row) key and writes it
// to cand[blockIdx.x * m_total + m] for argmax_final_kernel.  No logits are
// written.
__global__ void __launch_bounds__(256) vq_gemm_reduce_top1_kernel(const GemmArgs a)
{
    const int m = blockIdx.y;
    const int64_t pstride = (int64_t)a.m * a.out_rows;
    uint64_t best = 0;
    for (int64_t row = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; row < a.out_rows;
         row += (int64_t)gridDim.x * blockDim.x) {
        const int64_t t = (int64_t)m * a.out_rows + row;
        const float sum = split_sum(a, t, pstride);
        const float s = load_as_f32(a.scale, a.s_dt, row);
        const uint64_t k = argmax_key((sum * s) * a.rs, row);
        best = k > best ? k : best;
    }
    for (int off = 32; off > 0; off >>= 1) {
        const uint64_t o = __shfl_xor(best, off);
        best = o > best ? o : best;
    }
    __shared__ uint64_t s_best[4];
    if ((threadIdx.x & 63) == 0) s_best[threadIdx.x >> 6] = best;
    __syncthreads();
    if (threadIdx.x == 0) {
        uint64_t b = s_best[0];
        for (int w = 1; w < (int)(blockDim.x >> 6); w++) b = s_best[w] > b ? s_best[w] : b;
        a.cand[(int64_t)blockIdx.x * a.m + m] = b;
    }
}

// reduce blocks per activation row of the fused top-1 (bounds its candidates)
constexpr int64_t MM_TOP1_BLOCKS = 1024;

struct GemmPlan {
    int mt;
    int kcg;
    int splits;
    int64_t rowtiles;
};

// LDS a workgroup may take for its activation chunk: four stay resident per
// CU (measured: a single-split 65 KiB plan halves occupancy and slows the
// batch-4 LM head by 4 %; larger K splits win on some shapes and lose on
// others, so the plan keeps at least two workgroups' worth of splits per CU)
constexpr int MM_LDS_BUDGET = 40 * 1024;

// x_f16: fp16 activations are copied straight to LDS, so only LDS bounds the
// K split; other dtypes are staged through MM_STAGE registers per thread.
static GemmPlan plan_gemm(int64_t m, int64_t out_rows, int64_t ng, int num_cu, bool x_f16)
{
    GemmPlan p;
    p.mt = (int)((m + 15) / 16);
    const int mp = p.mt * 16;
    const int k_lds = (MM_LDS_BUDGET / (mp * (int)sizeof(half8_t)) - 1) / MM_TILE_G * MM_TILE_G;
    const int k_reg = MM_MAX_XG / mp / MM_TILE_G * MM_TILE_G;
    int kmax = x_f16 ? k_lds : (k_reg < k_lds ? k_reg : k_lds);
    if (kmax < MM_TILE_G) kmax = MM_TILE_G;
    const int64_t ng_t = (ng + MM_TILE_G - 1) / MM_TILE_G * MM_TILE_G;
    int kcg = (int)(ng_t < kmax ? ng_t : kmax);
    p.rowtiles = (out_rows + MM_ROWS - 1) / MM_ROWS;
    // smallest split count whose grid covers the device `fill` times over
    static const double fill = [] {
        const char* e = getenv("VQ2_MM_FILL");
        return e ? atof(e) : 2.0;
    }();
    const int64_t target = (int64_t)(fill * num_cu);
    while (kcg > MM_TILE_G && p.rowtiles * ((ng + kcg - 1) / kcg) < target) kcg -= MM_TILE_G;
    p.kcg = kcg;
    p.splits = (int)((ng + kcg - 1) / kcg);
    return p;
}

static int64_t top1_blocks(int64_t out_rows)
{
    const int64_t b = (out_rows + 255) / 256;
    return b < MM_TOP1_BLOCKS ? b : MM_TOP1_BLOCKS;
}

// partials of every split (one at least), 256-byte aligned, then the keys
static size_t top1_part_bytes(int64_t m, int64_t out_rows, int splits)
{
    return ((size_t)(splits > 1 ? splits : 1) * m * out_rows * sizeof(float) + 255) / 256 * 256;
}

size_t gemm_small_m_top1_workspace_bytes(int64_t m, int64_t out_rows, int64_t ng)
{
    if (m < 1 || out_rows < 1 || ng < 1) return 0;
    const GemmPlan p = plan_gemm(m, out_rows, ng, device_cu_count(), false);
    return top1_part_bytes(m, out_rows, p.splits) + (size_t)top1_blocks(out_rows) * m * sizeof(uint64_t);
}

size_t gemm_small_m_workspace_bytes(int64_t m, int64_t out_rows, int64_t ng)
{
    if (m < 1 || out_rows < 1 || ng < 1) return 0;
    // the register-staged plan has the most K splits: enough for any dtype
    const GemmPlan p = plan_gemm(m, out_rows, ng, device_cu_count(), false);
    return p.splits > 1 ? (size_t)p.splits * m * out_rows * sizeof(float) : 0;
}

template <int CBT, int S2, int MT>
static hipError_t launch_mm(const GemmArgs& a, dim3 grid, size_t shm, hipStream_t st)
{
    // opt in to more than 64 KiB of dynamic LDS, once per instantiation
    static std::once_flag once;
    static hipError_t attr = hipSuccess;
    std::call_once(once, [] {
        attr = hipFuncSetAttribute((const void*)vq_gemm_mfma_kernel<CBT, S2, MT>,
                                   hipFuncAttributeMaxDynamicSharedMemorySize, MM_LDS_BUDGET);
    });
    if (attr != hipSuccess) return attr;
    hipLaunchKernelGGL((vq_gemm_mfma_kernel<CBT, S2, MT>), grid, dim3(MM_THREADS), shm, st, a);
    return hipGetLastError();
}

template <int CBT, int S2>
static hipError_t launch_mm_mt(int mt, const GemmArgs& a, dim3 grid, size_t shm, hipStream_t st)
{
    switch (mt) {
    case 1: return launch_mm<CBT, S2, 1>(a, grid, shm, st);
    case 2: return launch_mm<CBT, S2, 2>(a, grid, shm, st);
    case 3: return launch_mm<CBT, S2, 3>(a, grid, shm, st);
    default: return launch_mm<CBT, S2, 4>(a, grid, shm, st);
    }
}

template <int CBT>
static hipError_t launch_mm_s2(int s2, int mt, const GemmArgs& a, dim3 grid, size_t shm, hipStream_t st)
{
    switch (s2) {
    case VQ2_S2_U8: return launch_mm_mt<CBT, VQ2_S2_U8>(mt, a, grid, shm, st);
    case VQ2_S2_U16: return launch_mm_mt<CBT, VQ2_S2_U16>(mt, a, grid, shm, st);
    default: return launch_mm_mt<CBT, VQ2_S2_NONE>(mt, a, grid, shm, st);
    }
}

static int gemm_launch(const GemmCall& c, int64_t* top1_idx, float* top1_val)
{
    const bool top1 = top1_idx != nullptr;
    if (c.m < 1 || c.m > MM_MAX_M) return set_error(VQ2_ERR_UNSUPPORTED, "vq2 small-M GEMM: batch must be 1..%d", MM_MAX_M);
    if (c.out_rows == 0) return VQ2_OK;
    if (c.ng % 8) return set_error(VQ2_ERR_UNSUPPORTED, "vq2 small-M GEMM: n must be a multiple of 64");
    const uintptr_t al = (uintptr_t)c.idx0 | (c.s2 == VQ2_S2_U16 ? (uintptr_t)c.idx1 : 0);
    if (al % 16 || (c.s2 == VQ2_S2_U8 && (uintptr_t)c.idx1 % 8))
        return set_error(VQ2_ERR_UNSUPPORTED, "vq2 small-M GEMM: index planes must be 16-byte aligned");
    const int64_t esz = dt_size(c.x_dt);
    if ((uintptr_t)c.x % 16 || (c.x_stride * esz) % 16)
        return set_error(VQ2_ERR_UNSUPPORTED, "vq2 small-M GEMM: activation rows must be 16-byte aligned");
    const GemmPlan p = plan_gemm(c.m, c.out_rows, c.ng, device_cu_count(), c.x_dt == VQ2_DT_F16);
    if (p.rowtiles > 0x7FFFFFFF || p.splits > 65535)
        return set_error(VQ2_ERR_UNSUPPORTED, "vq2 small-M GEMM: shape too large");
    GemmArgs a{};
    a.x = c.x;
    a.x_dt = c.x_dt;
    a.x_stride = c.x_stride;
    a.m = (int)c.m;
    a.idx0 = c.idx0;
    a.idx1 = c.idx1;
    a.cb0 = c.cb0;
    a.cb1 = c.cb1;
    a.scale = c.scale;
    a.s_dt = c.s_dt;
    a.y = c.y;
    a.y_dt = c.y_dt;
    a.y_stride = c.y_stride;
    a.out_rows = c.out_rows;
    a.ng = c.ng;
    a.rs = c.rs;
    a.kcg = p.kcg;
    a.splits = p.splits;
    a.part = (float*)c.workspace;
    a.to_part = top1 ? 1 : 0;
    const int64_t t1_blocks = top1_blocks(c.out_rows);
    if (p.splits > 1 || top1) {
        const size_t need = top1 ? top1_part_bytes(c.m, c.out_rows, p.splits) + (size_t)t1_blocks * c.m * sizeof(uint64_t)
                                 : (size_t)p.splits * c.m * c.out_rows * sizeof(float);
        if (!c.workspace || c.ws_bytes < need)
            return set_error(VQ2_ERR_ARG, "vq2 small-M GEMM: workspace of %zu bytes needed (got %zu)", need, c.ws_bytes);
        if ((uintptr_t)c.workspace % 16) return set_error(VQ2_ERR_ARG, "vq2 small-M GEMM: workspace must be 16-byte aligned");
    }
    if (top1) a.cand = (uint64_t*)((char*)c.workspace + top1_part_bytes(c.m, c.out_rows, p.splits));
    const size_t shm = (size_t)p.mt * 16 * (p.kcg + 1) * sizeof(half8_t);
    hipStream_t st = (hipStream_t)c.stream;
    const dim3 grid((unsigned)p.rowtiles, (unsigned)p.splits);
    hipError_t err;
    switch (c.cb_dt) {
    case VQ2_DT_F16: err = launch_mm_s2<VQ2_DT_F16>(c.s2, p.mt, a, grid, shm, st); break;
    case VQ2_DT_BF16: err = launch_mm_s2<VQ2_DT_BF16>(c.s2, p.mt, a, grid, shm, st); break;
    default: err = launch_mm_s2<VQ2_DT_F32>(c.s2, p.mt, a, grid, shm, st); break;
    }
    if (err != hipSuccess) return set_hip_error(err, "vq2 small-M GEMM launch");
    if (top1) {
        hipLaunchKernelGGL(vq_gemm_reduce_top1_kernel, dim3((unsigned)t1_blocks, (unsigned)c.m), dim3(256), 0, st, a);
        err = hipGetLastError();
        if (err != hipSuccess) return set_hip_error(err, "vq2 small-M GEMM top-1 reduce launch");
        return argmax_final_launch(a.cand, (unsigned)t1_blocks, c.m, top1_idx, top1_val, c.stream);
    }
    if (p.splits > 1) {
        const int64_t tot = c.m * c.out_rows;
        int64_t blocks = (tot + 255) / 256;
        if (blocks > 8192) blocks = 8192;
        hipLaunchKernelGGL(vq_gemm_reduce_kernel, dim3((unsigned)blocks), dim3(256), 0, st, a);
        err = hipGetLastError();
        if (err != hipSuccess) return set_hip_error(err, "vq2 small-M GEMM reduce launch");
    }
    return VQ2_OK;
}

int gemm_small_m_launch(const GemmCall& c) { return gemm_launch(c, nullptr, nullptr); }

// ------------------------------------------------- no-allocation variant
// The split-K partials of vq2_gemm_small_m_noalloc live in this file-scope
// device array instead of a caller workspace: every GPU the library runs on
// holds its own copy, at its own address, until the process ends.  In host
// code `scratch` names a host-side stand-in, never the device memory: the
// device address comes from hipGetSymbolAddress, once per device, with that
// device current, and only that address reaches the kernels.  The GEMM
// writes every partial before the reduce reads it, so nothing needs zeroing
// between calls.
static __device__ __align__(256) unsigned char scratch[MM_NOALLOC_SCRATCH_BYTES];

constexpr int MM_MAX_DEVICES = 64;

// device address of `scratch` on the current device (nullptr + error set on failure)
static void* scratch_on_current_device()
{
    int dev = -1;
    hipError_t err = hipGetDevice(&dev);
    if (err != hipSuccess) {
        set_hip_error(err, "vq2_gemm_small_m_noalloc: hipGetDevice");
        return nullptr;
    }
    if (dev < 0 || dev >= MM_MAX_DEVICES) {
        set_error(VQ2_ERR_UNSUPPORTED, "vq2_gemm_small_m_noalloc: device %d beyond the %d the library tracks", dev,
                  MM_MAX_DEVICES);
        return nullptr;
    }
    static std::mutex mu;
    static void* ptr[MM_MAX_DEVICES] = {};
    std::lock_guard<std::mutex> lock(mu);
    if (!ptr[dev]) {
        void* p = nullptr;
        err = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (err != hipSuccess || !p) {
            set_hip_error(err != hipSuccess ? err : hipErrorInvalidSymbol,
                          "vq2_gemm_small_m_noalloc: hipGetSymbolAddress(scratch)");
            return nullptr;
        }
        ptr[dev] = p;
    }
    return ptr[dev];
}

int gemm_small_m_noalloc_launch(GemmCall c)
{
    if (c.m >= 1 && c.m <= MM_MAX_M && c.out_rows > 0 && c.ng > 0) {
        const GemmPlan p = plan_gemm(c.m, c.out_rows, c.ng, device_cu_count(), c.x_dt == VQ2_DT_F16);
        const size_t need = p.splits > 1 ? (size_t)p.splits * c.m * c.out_rows * sizeof(float) : 0;
        if (need > MM_NOALLOC_SCRATCH_BYTES)
            return set_error(VQ2_ERR_UNSUPPORTED,
                             "vq2_gemm_small_m_noalloc: this shape needs %zu bytes of split-K partials, more than the "
                             "%zu-byte device scratch of the no-allocation entry (use vq2_gemm_small_m with a workspace)",
                             need, (size_t)MM_NOALLOC_SCRATCH_BYTES);
        if (need > 0) {
            void* p_scratch = scratch_on_current_device();
            if (!p_scratch) return VQ2_ERR_HIP;
            c.workspace = p_scratch;
            c.ws_bytes = MM_NOALLOC_SCRATCH_BYTES;
        }
    }
    return gemm_launch(c, nullptr, nullptr);
}

int gemm_small_m_top1_launch(const GemmCall& c, int64_t* out_idx, float* out_val)
{
    if (!out_idx) return set_error(VQ2_ERR_ARG, "vq2 small-M GEMM top-1: NULL out_idx");
    return gemm_launch(c, out_idx, out_val);
}

}  // namespace vq2
