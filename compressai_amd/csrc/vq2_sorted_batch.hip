// vq2_sorted_batch.hip -- VQ GEMM of 2 to 4 activation rows over the
// code-sorted layout (gfx950).
//
//   y[b][r] = (sum_g cb0[i0[r, g]] . x[b]_g  [+ sum_g cb1[i1[r, g]] . x[b]_g]) * s[r] * rs,
//   b < batch <= 4
//
// Why: at batch 2-4 the other paths gather every code at random (the
// batched gather kernel once per 8 activation rows, the matrix-core small-M
// GEMM once for all of them) and are capped by the L2 request rate, like the
// batch-1 gather kernel.  Over the code-sorted layout (vq2_sorted.hip: the
// same packed entries, chunks, slices and iteration order) a wave's 64 lanes
// share codebook lines, and one centroid gather serves every activation row.
//
// Kernel: one workgroup of 8 waves per (chunk, slice), two per CU.  LDS
// holds the activation as fp16, group-major with the NB (2 or 4) rows of a
// group side by side (16 * NB bytes per group), and every wave owns two
// accumulator arrays of NB floats per row of the chunk (one per 32-lane
// half, as the packing guarantees distinct rows per half; four, one per 16
// lanes, for chunks of at most 32 rows).  Per entry a lane
// reads its group's NB activation vectors, forms NB 8-term dot products in
// fp32 (v_dot2_f32_f16 for fp16 codebooks) and adds them to its row with one
// 8- or 16-byte read-add-write.
//
// Precision: x is stored in fp16 with a power-of-two scale per activation
// row (the row maximum lands in [2^14, 2^15); fp16 activations are copied
// as they are), which the epilogue divides out exactly; the centroids and
// all sums stay fp32 -- the same activation rounding as the matrix-core
// small-M GEMM this path replaces at batch 3-4 (~1e-4 of max |y|).  Sums over
// the waves' arrays and the slices run in a fixed order: deterministic.
//
// Semantics: the PackedLinear batch > 1 fallback (dequant + F.linear,
// vq2/runtime.py:82-89, 105-110) for the (16,) and (16,16) configurations,
// and with the fused top-1 PackedLMHead at batch > 1 (vq2/runtime.py:136-144)
// + torch.argmax (legion/engine.py:288).
#include <algorithm>
#include <mutex>

#include "vq2_sorted.hpp"

namespace vq2 {

constexpr int SB_THREADS = 512;
constexpr int SB_WAVES = SB_THREADS / 64;
constexpr int SB_MAX_SHM = 150 * 1024;          // two workgroups per CU up to 80 KiB (chunks of <= 255 rows)

typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
template <int NB>
struct AccVec;
template <>
struct AccVec<2> {
    typedef f32x2 type;
};
template <>
struct AccVec<4> {
    typedef f32x4 type;
};

struct SortedBatchSeg {
    const uint32_t* ent;
    int32_t ipc, ipc1;
    const void* scale;
    void* y;        // [batch][out_rows]
    float* part;    // slices > 1: [slices][NB][out_rows] row sums (activation scale divided out)
    uint32_t* cnt;  // slices > 1: arrival counter per chunk
    int64_t out_rows;
    int32_t chunk_start;
    int32_t sq, sr;
    int32_t R, rb, nbig;
};

struct SortedBatchArgs {
    const void* x;  // [batch][x_stride], rotated
    int64_t x_stride;
    int batch;
    const void* cb0;
    const void* cb1;
    uint32_t c1mask;  // stage-2 code mask (0xFF: the 256-row codebook of (16,8))
    int s_dt;
    int y_dt;
    int64_t ng;
    int gbits;
    int slices;
    float rs;
    int nseg;
    int nc;
    int x_floats;  // floats of LDS before the accumulators (activation, later the row-sum stage)
    int rg_wgs;    // > 0: workgroups [g * rg_wgs, (g + 1) * rg_wgs) take rows NB g .. NB g + NB - 1
    SortedBatchSeg seg[SG_MAX_SEG];
    uint64_t* cand;  // EP 1: [workgroup][batch] best top-1 keys
};

// Eight activation values of row b, group g (16-byte aligned: x and its row
// stride are checked on the host).
template <int XT>
__device__ __forceinline__ void sb_load8(const SortedBatchArgs& a, const void* x, int b, int64_t g, float (&v)[8])
{
    const int64_t off = (int64_t)b * a.x_stride + g * 8;
    if constexpr (XT == VQ2_DT_F32) {
        const u32x4* q = (const u32x4*)((const float*)x + off);
        const u32x4 p0 = q[0], p1 = q[1];
#pragma unroll
        for (int k = 0; k < 4; k++) {
            v[k] = __uint_as_float(p0[k]);
            v[4 + k] = __uint_as_float(p1[k]);
        }
    } else {
        const u32x4 p = *(const u32x4*)((const uint16_t*)a.x + off);
#pragma unroll
        for (int k = 0; k < 4; k++) {
            v[2 * k] = __uint_as_float(p[k] << 16);  // bf16
            v[2 * k + 1] = __uint_as_float(p[k] & 0xFFFF0000u);
        }
    }
}

// The NB dot products of one centroid with group g's activation vectors.
template <int CBT, int NB>
__device__ __forceinline__ void sb_dots(const u32x4 c, const _Float16* s_xh, uint32_t g, float (&d)[NB])
{
    const u32x4* xp = (const u32x4*)(s_xh + (size_t)g * (NB * 8));
    if constexpr (CBT == VQ2_DT_F16) {
        half2_t ch[4];
#pragma unroll
        for (int w = 0; w < 4; w++) {
            const uint32_t cw = c[w];  // a scalar copy: a bit cast of the vector element itself misreads it
            ch[w] = __builtin_bit_cast(half2_t, cw);
        }
#pragma unroll
        for (int b = 0; b < NB; b++) {
            const u32x4 xv = xp[b];
            float s = 0.0f;
#pragma unroll
            for (int w = 0; w < 4; w++) {
                const uint32_t xw = xv[w];
                s = __builtin_amdgcn_fdot2(ch[w], __builtin_bit_cast(half2_t, xw), s, false);
            }
            d[b] = s;
        }
    } else {
        float cf[8];
#pragma unroll
        for (int w = 0; w < 4; w++) {
            cf[2 * w] = __uint_as_float(c[w] << 16);
            cf[2 * w + 1] = __uint_as_float(c[w] & 0xFFFF0000u);
        }
#pragma unroll
        for (int b = 0; b < NB; b++) {
            const u32x4 xv = xp[b];
            float s = 0.0f;
#pragma unroll
            for (int w = 0; w < 4; w++) {
                const uint32_t xw = xv[w];
                const half2_t xh = __builtin_bit_cast(half2_t, xw);
                s = fmaf(cf[2 * w], (float)xh[0], s);
                s = fmaf(cf[2 * w + 1], (float)xh[1], s);
            }
            d[b] = s;
        }
    }
}

// XT: activation dtype; EP 0: y (or slice partials), EP 1: fused top-1 keys.
// TALL: chunks of 256 rows or more or 17-bit positions (the row sums and
// the position decode for them; the other instantiations keep the short
// ones).
template <int CBT, int NB, int XT, int EP, bool TALL>
__global__ void __launch_bounds__(SB_THREADS, 2) vq_sorted_batch_kernel(const SortedBatchArgs a)
{
    typedef typename AccVec<NB>::type accv;
    extern __shared__ __align__(16) float smem[];
    __shared__ uint32_t s_amax[NB];
    __shared__ int s_e[NB];
    touch_kernargs(a);
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    _Float16* s_xh = (_Float16*)smem;             // [ng][NB][8]
    accv* s_acc = (accv*)(smem + a.x_floats);     // SB_WAVES x sorted_parts(R) x (R + 1)

    // row group (rg_wgs > 0): this workgroup's rows are brow .. brow + nbat - 1
    const int rg = a.rg_wgs ? (int)blockIdx.x / a.rg_wgs : 0;
    const int pos = (int)blockIdx.x - rg * a.rg_wgs;
    const int brow = NB * rg, nbat = min(NB, a.batch - brow);
    const void* xg = (const char*)a.x + (int64_t)brow * a.x_stride * (XT == VQ2_DT_F32 ? 4 : 2);
    const int slice = pos / a.nc, gchunk = pos - slice * a.nc;
    int si = 0;
#pragma unroll
    for (int s = 1; s < SG_MAX_SEG; s++) si += (s < a.nseg && gchunk >= a.seg[s].chunk_start) ? 1 : 0;
    const SortedBatchSeg& sg = a.seg[si];
    const int R = sg.R;
    const int chunk = gchunk - sg.chunk_start;
    const int c_beg = chunk * sg.ipc;
    const int c_mid = c_beg + sg.ipc1;
    const int s0 = c_beg + slice * sg.sq + min(slice, sg.sr);
    const int s1 = s0 + sg.sq + (slice < sg.sr ? 1 : 0);

    // entry words and the first gathers go out first; the activation comes
    // from L2 meanwhile.  Gathers one iteration ahead (measured, LM head at
    // batch 2 / 4: 67.9 / 144.6 us; two ahead 68.8 / 144.9, three 70.9 / 154.8)
    SortedPipe<CBT, 1, SB_WAVES, TALL> pipe;
    pipe.start(sg.ent, a.cb0, a.cb1, c_beg, c_mid, s0, s1, wave, lane, a.gbits, R, a.c1mask);

    const int parts = sorted_parts(R), pl = 64 / parts;
    accv* acc = s_acc + (wave * parts + (lane >> (parts == SG_MAX_PARTS ? 4 : 5))) * (R + 1);
    for (int i = lane & (pl - 1); i <= R; i += pl) acc[i] = (accv)0.0f;

    // the activation: group-major fp16, rows >= batch zero
    const int64_t groups = a.ng * NB;
    if constexpr (XT == VQ2_DT_F16) {
        if (threadIdx.x < NB) s_e[threadIdx.x] = 0;
        for (int64_t t = threadIdx.x; t < groups; t += SB_THREADS) {
            const int64_t g = t / NB;
            const int b = (int)(t - g * NB);
            u32x4 v = {0u, 0u, 0u, 0u};
            if (b < nbat) v = *(const u32x4*)((const uint16_t*)xg + (int64_t)b * a.x_stride + g * 8);
            *(u32x4*)(s_xh + t * 8) = v;
        }
    } else {
        if (threadIdx.x < NB) s_amax[threadIdx.x] = 0u;
        __syncthreads();
        for (int64_t t = threadIdx.x; t < groups; t += SB_THREADS) {
            const int64_t g = t / NB;
            const int b = (int)(t - g * NB);
            if (b < nbat) {
                float v[8];
                sb_load8<XT>(a, xg, b, g, v);
                float am = 0.0f;
#pragma unroll
                for (int k = 0; k < 8; k++) am = fmaxf(am, fabsf(v[k]));
                // fmaxf skips NaN (it still reaches its row through the
                // products); an infinite row keeps scale 1
                if (__float_as_uint(am) != 0u) atomicMax(&s_amax[b], __float_as_uint(am));
            }
        }
        __syncthreads();
        if (threadIdx.x < NB) {
            const uint32_t am = s_amax[threadIdx.x];
            // the row maximum lands in [2^14, 2^15): exact, far below fp16's 65504
            s_e[threadIdx.x] = (am != 0u && am < 0x7F800000u) ? 14 - ilogbf(__uint_as_float(am)) : 0;
        }
        __syncthreads();
        for (int64_t t = threadIdx.x; t < groups; t += SB_THREADS) {
            const int64_t g = t / NB;
            const int b = (int)(t - g * NB);
            half8_t h = {0, 0, 0, 0, 0, 0, 0, 0};
            if (b < nbat) {
                float v[8];
                sb_load8<XT>(a, xg, b, g, v);  // an L2 hit: loaded above
                const int e = s_e[b];
#pragma unroll
                for (int k = 0; k < 8; k++) h[k] = (_Float16)ldexpf(v[k], e);
            }
            *(half8_t*)(s_xh + t * 8) = h;
        }
    }
    __syncthreads();

    const uint32_t gmask = (1u << a.gbits) - 1u, gmax = (uint32_t)(a.ng - 1);
    pipe.run_each([&](const u32x4& pos, const u32x4 (&cw)[4]) {
#pragma unroll
        for (int q = 0; q < 4; q++) {
            const uint32_t p = pos[q];
            const uint32_t r = min(p >> a.gbits, (uint32_t)R);
            const uint32_t g = min(p & gmask, gmax);
            float d[NB];
            sb_dots<CBT, NB>(cw[q], s_xh, g, d);
            accv v = acc[r];
#pragma unroll
            for (int b = 0; b < NB; b++) v[b] += d[b];
            acc[r] = v;
        }
    });
    __syncthreads();

    // row sums: thread (pp, rr) adds half the arrays of row rr, then the two
    // halves in order (the activation's LDS is free by now); chunks of 256
    // rows or more: thread rr adds both halves itself (the same order)
    const int NA = SB_WAVES * parts / 2;
    const bool tall = TALL && R >= 256;
    const int rr = tall ? (int)threadIdx.x : (int)(threadIdx.x & 255), pp = tall ? 0 : (int)(threadIdx.x >> 8);
    accv tsum = (accv)0.0f;
    if (tall) {
        if (rr <= R) {
            accv p0 = (accv)0.0f, p1 = (accv)0.0f;
#pragma unroll 4
            for (int w = 0; w < NA; w++) p0 += s_acc[w * (R + 1) + rr];
#pragma unroll 4
            for (int w = NA; w < 2 * NA; w++) p1 += s_acc[w * (R + 1) + rr];
            tsum = p0 + p1;
        }
    } else {
        accv* s_red = (accv*)smem;  // [2][256]
        if (rr <= R) {
            accv part = (accv)0.0f;
#pragma unroll 4
            for (int w = NA * pp; w < NA * pp + NA; w++) part += s_acc[w * (R + 1) + rr];
            s_red[pp * 256 + rr] = part;
        }
        __syncthreads();
        if (pp == 0 && rr <= R) tsum = s_red[rr] + s_red[256 + rr];
    }
    const bool own = pp == 0 && rr < sg.rb + (chunk < sg.nbig ? 1 : 0);
    const int64_t row = (int64_t)chunk * sg.rb + min(chunk, sg.nbig) + rr;
    float sum[NB];
    if (pp == 0 && rr <= R) {
        const accv t = tsum;
#pragma unroll
        for (int b = 0; b < NB; b++) sum[b] = ldexpf(t[b], -s_e[b]);
    } else {
#pragma unroll
        for (int b = 0; b < NB; b++) sum[b] = 0.0f;
    }
    if constexpr (EP == 1) {
        const float sc = own ? load_as_f32(sg.scale, a.s_dt, row) : 0.0f;
        __shared__ uint64_t s_key[SB_WAVES][NB];
#pragma unroll
        for (int b = 0; b < NB; b++) {
            uint64_t best = own ? argmax_key((sum[b] * sc) * a.rs, row) : 0;
            for (int off = 32; off > 0; off >>= 1) {
                const uint64_t o = __shfl_xor(best, off);
                best = o > best ? o : best;
            }
            if (lane == 0) s_key[wave][b] = best;  // 0 from waves with no row of their own
        }
        __syncthreads();
        if (threadIdx.x < NB && (int)threadIdx.x < nbat) {
            const int b = threadIdx.x;
            uint64_t best = s_key[0][b];
            for (int w = 1; w < SB_WAVES; w++) best = s_key[w][b] > best ? s_key[w][b] : best;
            a.cand[(int64_t)pos * a.batch + brow + b] = best;
        }
    } else if (a.slices == 1) {
        if (own) {
            const float sc = load_as_f32(sg.scale, a.s_dt, row);
#pragma unroll
            for (int b = 0; b < NB; b++)
                if (b < nbat) store_from_f32(sg.y, a.y_dt, (int64_t)(brow + b) * sg.out_rows + row, (sum[b] * sc) * a.rs);
        }
    } else {
        // several slices: the last of the chunk's workgroups to finish adds
        // the slices' row sums in slice order
        if (own)
#pragma unroll
            for (int b = 0; b < NB; b++)
                if (b < nbat) share_store(sg.part + ((int64_t)slice * NB + b) * sg.out_rows + row, sum[b]);
        if (arrive_last(sg.cnt + chunk, (uint32_t)a.slices) && own) {
            const float sc = load_as_f32(sg.scale, a.s_dt, row);
#pragma unroll
            for (int b = 0; b < NB; b++) {
                if (b >= nbat) break;
                float tot = 0.0f;
                for (int j0 = 0; j0 < a.slices; j0 += 8) {
                    float v[8];
#pragma unroll
                    for (int j = 0; j < 8; j++) {
                        const int s = j0 + j < a.slices ? j0 + j : slice;
                        v[j] = s == slice ? sum[b] : share_load(sg.part + ((int64_t)s * NB + b) * sg.out_rows + row);
                    }
#pragma unroll
                    for (int j = 0; j < 8; j++)
                        if (j0 + j < a.slices) tot += v[j];
                }
                store_from_f32(sg.y, a.y_dt, (int64_t)(brow + b) * sg.out_rows + row, (tot * sc) * a.rs);
            }
        }
    }
}

// ------------------------------------------------------------------ launch
template <int CBT, int NB, int XT, int EP, bool TALL>
static hipError_t launch_batch(const SortedBatchArgs& a, unsigned grid, size_t shm, hipStream_t st)
{
    static std::once_flag once;
    static hipError_t attr = hipSuccess;
    std::call_once(once, [] {
        attr = hipFuncSetAttribute((const void*)vq_sorted_batch_kernel<CBT, NB, XT, EP, TALL>,
                                   hipFuncAttributeMaxDynamicSharedMemorySize, SB_MAX_SHM);
    });
    if (attr != hipSuccess) return attr;
    hipLaunchKernelGGL((vq_sorted_batch_kernel<CBT, NB, XT, EP, TALL>), dim3(grid), dim3(SB_THREADS), shm, st, a);
    return hipGetLastError();
}

template <int NB, int EP, bool TALL>
static hipError_t launch_batch_t(int cb_dt, int x_dt, const SortedBatchArgs& a, unsigned grid, size_t shm,
                                 hipStream_t st)
{
    if (cb_dt == VQ2_DT_F16) {
        switch (x_dt) {
        case VQ2_DT_F16: return launch_batch<VQ2_DT_F16, NB, VQ2_DT_F16, EP, TALL>(a, grid, shm, st);
        case VQ2_DT_BF16: return launch_batch<VQ2_DT_F16, NB, VQ2_DT_BF16, EP, TALL>(a, grid, shm, st);
        default: return launch_batch<VQ2_DT_F16, NB, VQ2_DT_F32, EP, TALL>(a, grid, shm, st);
        }
    }
    switch (x_dt) {
    case VQ2_DT_F16: return launch_batch<VQ2_DT_BF16, NB, VQ2_DT_F16, EP, TALL>(a, grid, shm, st);
    case VQ2_DT_BF16: return launch_batch<VQ2_DT_BF16, NB, VQ2_DT_BF16, EP, TALL>(a, grid, shm, st);
    default: return launch_batch<VQ2_DT_BF16, NB, VQ2_DT_F32, EP, TALL>(a, grid, shm, st);
    }
}

template <int NB, int EP>
static hipError_t launch_batch_nb(int cb_dt, int x_dt, bool tall, const SortedBatchArgs& a, unsigned grid,
                                  size_t shm, hipStream_t st)
{
    return tall ? launch_batch_t<NB, EP, true>(cb_dt, x_dt, a, grid, shm, st)
                : launch_batch_t<NB, EP, false>(cb_dt, x_dt, a, grid, shm, st);
}

static int batch_slots(int64_t batch) { return batch <= 2 ? 2 : 4; }

// LDS of a workgroup that still lets two share a CU (160 KiB per CU)
constexpr size_t SB_PAIR_SHM = 80 * 1024;

// Workspace with several slices: VQ2_SORTED_WS_HEADER bytes of arrival
// counters (zero between launches), then per matrix [slices][slots][rows]
// row sums.
size_t sorted_batch_workspace_bytes(const SortedCall& c)
{
    if (c.slices <= 1) return 0;
    size_t b = VQ2_SORTED_WS_HEADER;
    for (int s = 0; s < c.nseg; s++)
        b += (size_t)c.slices * batch_slots(c.batch) * c.seg[s].out_rows * sizeof(float);
    return b;
}

size_t sorted_batch_top1_workspace_bytes(int64_t out_rows, int64_t rows_per_chunk, int64_t batch)
{
    if (rows_per_chunk < 1 || out_rows < 1 || batch < 1) return 0;
    return (size_t)((out_rows + rows_per_chunk - 1) / rows_per_chunk) * batch * sizeof(uint64_t);
}

int sorted_batch_launch(const SortedCall& c, int64_t* top1_idx, float* top1_val)
{
    const bool top1 = top1_idx != nullptr;
    if (c.batch < 1 || c.batch > 4) return set_error(VQ2_ERR_ARG, "vq2 sorted GEMM: batch=%lld outside 1..4", (long long)c.batch);
    int64_t rmax = 0;
    if (int r = sorted_check_call(c, top1, "vq2 sorted GEMM", &rmax)) return r;
    const int64_t n = c.ng * 8;
    if (c.x_stride < n || c.x_stride % 8 || (uintptr_t)c.x % 16)
        return set_error(VQ2_ERR_ARG, "vq2 sorted GEMM: x must be 16-byte aligned with a row stride >= n, a multiple "
                         "of 8 (got %lld)", (long long)c.x_stride);
    int nb = batch_slots(c.batch), groups = 1;
    // chunks of 256 rows or more, or 17-bit positions: the TALL kernels
    const bool tall = rmax >= 256 || sorted_pbits(sorted_gbits(c.ng), (int)rmax) > 16;
    // activation (fp16, nb rows) or the row-sum stage, whichever is larger, then the accumulators
    const auto shm_of = [&](int rows) {
        return (size_t)(std::max<int64_t>(n * rows / 2, 2 * 256 * rows) + (int64_t)SB_WAVES * sorted_acc_arrays(c) * rows) *
               sizeof(float);
    };
    if (nb == 4 && shm_of(4) > SB_PAIR_SHM && c.slices == 1) {
        // 4-row workgroups this large run one per CU (8 waves): 2-row
        // workgroups instead, several per CU, one launch over both row
        // pairs (rows 2 g, 2 g + 1 in workgroups [g * wg, (g + 1) * wg))
        // and one final top-1; a row group's workgroups start as the other's
        // finish (the LM head 151936 x 2048 in 297-row chunks: top-1 at
        // batch 4 148.9 us as 4-row workgroups, 129.8 as two 2-row launches,
        // 121.6 as one; batch 3 147.7 / 120.5; logits at batch 4 145.3 /
        // 116.9)
        nb = 2;
        groups = (int)((c.batch + 1) / 2);
    }
    const int64_t x_floats = std::max<int64_t>(n * nb / 2, 2 * 256 * nb);
    const size_t shm = shm_of(nb);
    if (nb == 4 && shm > SB_PAIR_SHM) {
        // the same with several slices (whose counters and partials are per
        // chunk): rows 0-1, then the rest, as two launches that reuse the
        // workspace in stream order (gate + up, 79.6 KiB at batch 4, stays one
        // launch: 37.2 us against 38.4 split)
        SortedCall lo = c, hi = c;
        lo.batch = 2;
        hi.batch = c.batch - 2;
        hi.x = (const char*)c.x + 2 * c.x_stride * dt_size(c.x_dt);
        for (int s = 0; s < c.nseg; s++)
            hi.seg[s].y = c.seg[s].y ? (char*)c.seg[s].y + 2 * c.seg[s].out_rows * dt_size(c.y_dt) : nullptr;
        if (int r = sorted_batch_launch(lo, top1_idx, top1_val)) return r;
        return sorted_batch_launch(hi, top1 ? top1_idx + 2 : nullptr, top1 ? top1_val + 2 : nullptr);
    }
    if (shm > SB_MAX_SHM)
        return set_error(VQ2_ERR_UNSUPPORTED, "vq2 sorted GEMM: n=%lld with %lld-row chunks needs %zu bytes of LDS "
                         "(at most %d)", (long long)n, (long long)rmax, shm, SB_MAX_SHM);
    SortedBatchArgs a{};
    a.x = c.x;
    a.x_stride = c.x_stride;
    a.batch = (int)c.batch;
    a.cb0 = c.cb0;
    a.cb1 = c.cb1;
    a.c1mask = c.cb1_rows == 256 ? 0xFFu : 0xFFFFu;
    a.s_dt = c.s_dt;
    a.y_dt = c.y_dt;
    a.ng = c.ng;
    a.gbits = sorted_gbits(c.ng);
    a.slices = c.slices;
    a.rs = c.rs;
    a.nseg = c.nseg;
    a.x_floats = (int)x_floats;
    uint32_t* cnt = (uint32_t*)c.workspace;
    float* part = (float*)((char*)c.workspace + VQ2_SORTED_WS_HEADER);
    if (top1) {
        const size_t need = sorted_batch_top1_workspace_bytes(c.seg[0].out_rows, c.seg[0].rows_per_chunk, c.batch);
        if (!c.workspace || c.ws_bytes < need || (uintptr_t)c.workspace % 8)
            return set_error(VQ2_ERR_ARG, "vq2 sorted GEMM top-1: workspace of %zu bytes (8-byte aligned) needed, got "
                             "%zu", need, c.ws_bytes);
        a.cand = (uint64_t*)c.workspace;
    } else if (c.slices > 1) {
        const size_t need = sorted_batch_workspace_bytes(c);
        if (!c.workspace || c.ws_bytes < need || (uintptr_t)c.workspace % 16)
            return set_error(VQ2_ERR_ARG, "vq2 sorted GEMM: workspace of %zu bytes (16-byte aligned) needed, got %zu",
                             need, c.ws_bytes);
    }
    int64_t wg = 0, n_cnt = 0, nc = 0;
    for (int s = 0; s < c.nseg; s++) {
        const SortedSegCall& sc = c.seg[s];
        ChunkSplit ks;
        if (int r = sorted_check_seg(c, s, "vq2 sorted GEMM", &ks)) return r;
        const int64_t n_chunks = ks.n_chunks;
        SortedBatchSeg& d = a.seg[s];
        d.ent = sc.entries;
        d.ipc = (int32_t)sc.iters_per_chunk;
        d.ipc1 = (int32_t)sc.stage1_iters;
        d.scale = sc.scale;
        d.y = sc.y;
        d.out_rows = sc.out_rows;
        d.chunk_start = (int32_t)nc;
        d.sq = (int32_t)(sc.iters_per_chunk / c.slices);
        d.sr = (int32_t)(sc.iters_per_chunk % c.slices);
        d.R = (int32_t)sc.rows_per_chunk;
        d.rb = (int32_t)ks.rb;
        d.nbig = (int32_t)ks.nbig;
        d.part = part;
        d.cnt = cnt + n_cnt;
        if (!top1 && c.slices > 1) {
            part += (int64_t)c.slices * nb * sc.out_rows;
            n_cnt += n_chunks;
        }
        wg += n_chunks * c.slices;
        nc += n_chunks;
    }
    if (n_cnt > VQ2_SORTED_MAX_COUNTERS)
        return set_error(VQ2_ERR_UNSUPPORTED, "vq2 sorted GEMM: %lld chunks with several slices (at most %d)",
                         (long long)n_cnt, VQ2_SORTED_MAX_COUNTERS);
    if (wg == 0) return VQ2_OK;
    if (wg * groups > 0x7FFFFFFF) return set_error(VQ2_ERR_UNSUPPORTED, "vq2 sorted GEMM: grid too large");
    a.nc = (int)nc;
    a.rg_wgs = groups > 1 ? (int)wg : 0;
    const unsigned grid = (unsigned)(wg * groups);
    hipStream_t st = (hipStream_t)c.stream;
    hipError_t err;
    if (top1) {
        // keys [workgroup of a group][batch]: one final pass over wg keys per row
        err = nb == 2 ? launch_batch_nb<2, 1>(c.cb_dt, c.x_dt, tall, a, grid, shm, st)
                      : launch_batch_nb<4, 1>(c.cb_dt, c.x_dt, tall, a, grid, shm, st);
        if (err != hipSuccess) return set_hip_error(err, "vq2 sorted GEMM launch");
        return argmax_final_launch(a.cand, wg, c.batch, top1_idx, top1_val, c.stream);
    }
    err = nb == 2 ? launch_batch_nb<2, 0>(c.cb_dt, c.x_dt, tall, a, grid, shm, st)
                  : launch_batch_nb<4, 0>(c.cb_dt, c.x_dt, tall, a, grid, shm, st);
    if (err != hipSuccess) return set_hip_error(err, "vq2 sorted GEMM launch");
    return VQ2_OK;
}

}  // namespace vq2
