// vq2_rht.hip -- randomised Hadamard transform (sign flip + FWHT) for gfx950.
//
// Reference semantics: Rot.fwd / Rot.inv (vq2/vq.py:74-87) with the
// Sylvester Hadamard of vq2/vq.py:22-27, blockwise over hb-point blocks;
// FastRot (vq2/runtime.py:57-63) is the scale = 1 case.
//
// Design: one workgroup per (hb-block, vector).  T threads each hold
// V = hb / T values in VGPRs.  The log2(hb) butterfly stages are split into
// passes of at most log2(V) stages; inside a pass every stage is an
// in-register butterfly, and between passes the block is transposed through
// LDS so that the next pass's index bits become register bits.  For
// hb = 2048 that is T = 64 (one wave), V = 32 and 3 passes (4+4+3 stages),
// i.e. two LDS round trips and no cross-lane shuffles.  The permutation
// gather, the sign flip, the optional SwiGLU of the MoE epilogue, the scale
// and the dtype conversion are fused into the first and last passes.
#include "vq2_common.hpp"
#include "vq2_internal.hpp"

namespace vq2 {

struct RhtArgs {
    const void* x;
    int x_dt;
    int64_t x_stride;
    void* y;
    int y_dt;
    int64_t y_stride;
    const int32_t* perm;
    const int8_t* sign;
    float scale;
    int inverse;
    int swiglu;     // x holds [gate | up] of width 2*inter; transform silu(gate)*up
    int64_t inter;  // n of the transform in swiglu mode
    int64_t n;      // transform length (bounds of perm entries)
    int stage;      // forward with a permutation: the row is staged in LDS (dynamic, n elements)
};

template <int L>
struct RhtShape {
    static constexpr int HB = 1 << L;
    // threads per block: 64 for hb <= 1024, up to 256 for the largest blocks
    static constexpr int T = HB / 16 > 256 ? 256 : (HB / 16 > (HB / 2 < 64 ? HB / 2 : 64) ? HB / 16 : (HB / 2 < 64 ? HB / 2 : 64));
    static constexpr int V = HB / T;
    static constexpr int VB = V == 2 ? 1 : V == 4 ? 2 : V == 8 ? 3 : V == 16 ? 4 : 5;
    static constexpr int NP = (L + VB - 1) / VB;
    static constexpr int width(int p) { return L / NP + (p < L % NP ? 1 : 0); }
    static constexpr int lo(int p)
    {
        int s = 0;
        for (int i = 0; i < p; i++) s += width(i);
        return s;
    }
    static_assert(T * V == HB && (1 << VB) == V, "bad RHT shape");
};

// element index of register i of thread tid in the layout whose butterfly
// bits are [lo, lo + W)
template <int VB, int W, int LO>
__device__ __forceinline__ int elem_of(int tid, int i)
{
    const int k = i & ((1 << W) - 1);
    const int s = i >> W;
    const int rest = (tid << (VB - W)) | s;
    return ((rest >> LO) << (LO + W)) | (k << LO) | (rest & ((1 << LO) - 1));
}

template <int V, int W>
__device__ __forceinline__ void butterflies(float (&v)[V])
{
#pragma unroll
    for (int h = 1; h < (1 << W); h <<= 1) {
#pragma unroll
        for (int i = 0; i < V; i++) {
            if ((i & h) == 0) {
                const float a = v[i], b = v[i | h];
                v[i] = a + b;
                v[i | h] = a - b;
            }
        }
    }
}

template <int L, int P>
__device__ __forceinline__ void rht_passes(float (&v)[RhtShape<L>::V], float* lds, int tid)
{
    using S = RhtShape<L>;
    if constexpr (P < S::NP) {
        constexpr int W = S::width(P);
        constexpr int LO = S::lo(P);
        if constexpr (P > 0) {
            constexpr int WP = S::width(P - 1);
            constexpr int LOP = S::lo(P - 1);
#pragma unroll
            for (int i = 0; i < S::V; i++) lds[elem_of<S::VB, WP, LOP>(tid, i)] = v[i];
            __syncthreads();
#pragma unroll
            for (int i = 0; i < S::V; i++) v[i] = lds[elem_of<S::VB, W, LO>(tid, i)];
            __syncthreads();
        }
        butterflies<S::V, W>(v);
        rht_passes<L, P + 1>(v, lds, tid);
    }
}

template <int XT>
__device__ __forceinline__ float ld_elem(const void* p, int64_t i)
{
    if constexpr (XT == VQ2_DT_F32) return ((const float*)p)[i];
    else if constexpr (XT == VQ2_DT_F16) return f16_bits_to_f32(((const uint16_t*)p)[i]);
    else return bf16_bits_to_f32(((const uint16_t*)p)[i]);
}

// Pass-0 load: thread tid holds elements tid*V + i.  Every address is
// computed first and all loads are issued before any value is used.
template <int V, int XT>
__device__ __forceinline__ void rht_load(const RhtArgs& a, int64_t b, int64_t e0, float (&v)[V])
{
    const char* xrow = (const char*)a.x + (size_t)(b * a.x_stride) * (XT == VQ2_DT_F32 ? 4 : 2);
    if (a.inverse || (!a.perm && !a.swiglu)) {
        float raw[V];
#pragma unroll
        for (int i = 0; i < V; i++) raw[i] = ld_elem<XT>(xrow, e0 + i);
        int8_t sg[V];
#pragma unroll
        for (int i = 0; i < V; i++) sg[i] = (!a.inverse && a.sign) ? a.sign[e0 + i] : (int8_t)1;
#pragma unroll
        for (int i = 0; i < V; i++) v[i] = raw[i] * (float)sg[i];
        return;
    }
    int64_t src[V];
    bool bad[V];
#pragma unroll
    for (int i = 0; i < V; i++) {
        const int64_t s0 = a.perm ? (int64_t)a.perm[e0 + i] : e0 + i;
        bad[i] = (uint64_t)s0 >= (uint64_t)a.n;  // not a permutation of [0, n): poison, never read out of bounds
        src[i] = bad[i] ? 0 : s0;
    }
    float g[V], u[V];
#pragma unroll
    for (int i = 0; i < V; i++) g[i] = ld_elem<XT>(xrow, src[i]);
    if (a.swiglu) {
#pragma unroll
        for (int i = 0; i < V; i++) u[i] = ld_elem<XT>(xrow, a.inter + src[i]);
    }
    int8_t sg[V];
#pragma unroll
    for (int i = 0; i < V; i++) sg[i] = a.sign ? a.sign[e0 + i] : (int8_t)1;
#pragma unroll
    for (int i = 0; i < V; i++) {
        float val = a.swiglu ? silu_f32(g[i]) * u[i] : g[i];
        val *= (float)sg[i];
        v[i] = bad[i] ? __builtin_nanf("") : val;
    }
}

// +1 bytes standing in for a missing sign table (repeats every RHT_ONES elements)
constexpr int RHT_ONES = 8192;
struct RhtOnes {
    int8_t v[RHT_ONES];
    constexpr RhtOnes() : v() { for (int i = 0; i < RHT_ONES; i++) v[i] = 1; }
};
static __device__ const __align__(16) RhtOnes g_rht_ones = RhtOnes();

// Pass-0 load with the permutation applied in LDS (forward, no SwiGLU): the
// thread's permutation and sign words and the whole unpermuted row (16-byte
// chunks, contiguous) are loaded together, so no global load waits for
// another; after a barrier the permuted elements are read from LDS.  The row
// is 16-byte aligned and n * element size a multiple of 16 (checked on the
// host).
template <int T, int V, int XT>
__device__ __forceinline__ void rht_load_staged(const RhtArgs& a, int64_t b, int64_t e0, float (&v)[V], u32x4* s_row,
                                                int tid)
{
    constexpr int ESZ = XT == VQ2_DT_F32 ? 4 : 2;
    // permutation and sign words with 16-byte loads where V allows (both
    // tables 16-byte aligned, checked on the host)
    int32_t pw[V];
    if constexpr (V % 4 == 0) {
#pragma unroll
        for (int q = 0; q < V / 4; q++) {
            const u32x4 w = *((const u32x4*)(a.perm + e0) + q);
#pragma unroll
            for (int k = 0; k < 4; k++) pw[4 * q + k] = (int32_t)w[k];
        }
    } else {
#pragma unroll
        for (int i = 0; i < V; i++) pw[i] = a.perm[e0 + i];
    }
    int8_t sg[V];
    if constexpr (V % 16 == 0) {
        // a missing sign table reads +1 bytes (a pointer select, not a branch around the load)
        const int8_t* sp = a.sign ? a.sign + e0 : g_rht_ones.v + (e0 & (RHT_ONES - 1));
#pragma unroll
        for (int q = 0; q < V / 16; q++) {
            const u32x4 w = *((const __attribute__((address_space(1))) u32x4*)sp + q);
#pragma unroll
            for (int k = 0; k < 16; k++) sg[16 * q + k] = (int8_t)((w[k >> 2] >> (8 * (k & 3))) & 0xFFu);
        }
    } else {
#pragma unroll
        for (int i = 0; i < V; i++) sg[i] = a.sign ? a.sign[e0 + i] : (int8_t)1;
    }
    const u32x4* xr = (const u32x4*)((const char*)a.x + (size_t)(b * a.x_stride) * ESZ);
    const int64_t nch = a.n * ESZ / 16;
    // 8 chunks per thread and round, loaded before any is stored (clamped
    // index: every load is unconditional, only the store is guarded)
    for (int64_t c0 = tid; c0 < nch; c0 += 8 * T) {
        u32x4 r[8];
#pragma unroll
        for (int j = 0; j < 8; j++) {
            const int64_t c = c0 + (int64_t)j * T;
            r[j] = xr[c < nch ? c : nch - 1];
        }
#pragma unroll
        for (int j = 0; j < 8; j++) {
            const int64_t c = c0 + (int64_t)j * T;
            if (c < nch) s_row[c] = r[j];
        }
    }
    __syncthreads();
#pragma unroll
    for (int i = 0; i < V; i++) {
        const bool bad = (uint32_t)pw[i] >= (uint64_t)a.n;  // not a permutation of [0, n): poison
        const int src = bad ? 0 : pw[i];
        float val;
        if constexpr (XT == VQ2_DT_F32) val = ((const float*)s_row)[src];
        else if constexpr (XT == VQ2_DT_F16) val = f16_bits_to_f32(((const uint16_t*)s_row)[src]);
        else val = bf16_bits_to_f32(((const uint16_t*)s_row)[src]);
        v[i] = bad ? __builtin_nanf("") : val * (float)sg[i];
    }
}

template <int L>
__global__ void __launch_bounds__(256) rht_kernel(const RhtArgs a)
{
    touch_kernargs(a);
    using S = RhtShape<L>;
    __shared__ float lds[S::NP > 1 ? S::HB : 1];
    extern __shared__ __align__(16) u32x4 s_row[];  // the staged row (a.stage)
    const int tid = threadIdx.x;
    const int64_t base = (int64_t)blockIdx.x * S::HB;
    const int64_t b = blockIdx.y;
    float v[S::V];

    const int64_t e0 = base + (int64_t)tid * S::V;
    if (a.stage) {
        if (a.x_dt == VQ2_DT_F32)
            rht_load_staged<S::T, S::V, VQ2_DT_F32>(a, b, e0, v, s_row, tid);
        else if (a.x_dt == VQ2_DT_F16)
            rht_load_staged<S::T, S::V, VQ2_DT_F16>(a, b, e0, v, s_row, tid);
        else
            rht_load_staged<S::T, S::V, VQ2_DT_BF16>(a, b, e0, v, s_row, tid);
    } else if (a.x_dt == VQ2_DT_F32)
        rht_load<S::V, VQ2_DT_F32>(a, b, e0, v);
    else if (a.x_dt == VQ2_DT_F16)
        rht_load<S::V, VQ2_DT_F16>(a, b, e0, v);
    else
        rht_load<S::V, VQ2_DT_BF16>(a, b, e0, v);

    rht_passes<L, 0>(v, lds, tid);

    constexpr int WL = S::width(S::NP - 1);
    constexpr int LOL = S::lo(S::NP - 1);
    int64_t dst[S::V];
    float val[S::V];
#pragma unroll
    for (int i = 0; i < S::V; i++) {
        dst[i] = base + elem_of<S::VB, WL, LOL>(tid, i);
        val[i] = v[i] * a.scale;
    }
    if (a.inverse) {
        // z[i] *= sign[i]; y[perm[i]] = z[i]  (loads first, then the scatter)
        int8_t sg[S::V];
        int64_t pd[S::V];
#pragma unroll
        for (int i = 0; i < S::V; i++) {
            sg[i] = a.sign ? a.sign[dst[i]] : (int8_t)1;
            pd[i] = a.perm ? (int64_t)a.perm[dst[i]] : dst[i];
        }
#pragma unroll
        for (int i = 0; i < S::V; i++) {
            val[i] *= (float)sg[i];
            dst[i] = (uint64_t)pd[i] < (uint64_t)a.n ? pd[i] : -1;  // bad permutation entry: drop the store
        }
    }
    const int64_t yrow = b * a.y_stride;
    if (a.y_dt == VQ2_DT_F32) {
#pragma unroll
        for (int i = 0; i < S::V; i++)
            if (dst[i] >= 0) ((float*)a.y)[yrow + dst[i]] = val[i];
    } else if (a.y_dt == VQ2_DT_F16) {
#pragma unroll
        for (int i = 0; i < S::V; i++)
            if (dst[i] >= 0) ((uint16_t*)a.y)[yrow + dst[i]] = f32_to_f16_bits(val[i]);
    } else {
#pragma unroll
        for (int i = 0; i < S::V; i++)
            if (dst[i] >= 0) ((uint16_t*)a.y)[yrow + dst[i]] = f32_to_bf16_bits(val[i]);
    }
}

template <int L>
static void launch_rht_l(const RhtArgs& a, int64_t nblk, int64_t batch, size_t shm, hipStream_t st)
{
    hipLaunchKernelGGL((rht_kernel<L>), dim3((unsigned)nblk, (unsigned)batch), dim3(RhtShape<L>::T), shm, st, a);
}

// largest row staged in LDS by the forward permuted transform
constexpr int64_t RHT_STAGE_BYTES = 32 * 1024;

int rht_launch(const void* x, int x_dt, int64_t x_stride, void* y, int y_dt, int64_t y_stride, const int32_t* perm,
               const int8_t* sign, int64_t n, int64_t hb, int64_t batch, float scale, int inverse, int swiglu,
               int64_t inter, void* stream)
{
    if (batch == 0 || n == 0) return VQ2_OK;
    int L = 0;
    while ((1LL << L) < hb) L++;
    if (L < 1 || L > 13 || (1LL << L) != hb)
        return set_error(VQ2_ERR_ARG, "vq2 rht: hb=%lld must be a power of two in [2, 8192]", (long long)hb);
    if (n % hb) return set_error(VQ2_ERR_ARG, "vq2 rht: n=%lld is not a multiple of hb=%lld", (long long)n, (long long)hb);
    if (batch > 65535 || n / hb > 0x7FFFFFFF) return set_error(VQ2_ERR_UNSUPPORTED, "vq2 rht: grid too large");
    const int64_t esz = dt_size(x_dt);
    const bool stage = !inverse && !swiglu && perm && (uintptr_t)x % 16 == 0 && (x_stride * esz) % 16 == 0 &&
                       (n * esz) % 16 == 0 && n * esz <= RHT_STAGE_BYTES && (uintptr_t)perm % 16 == 0 &&
                       (uintptr_t)sign % 16 == 0;
    RhtArgs a{x, x_dt, x_stride, y, y_dt, y_stride, perm, sign, scale, inverse, swiglu, inter, n, stage ? 1 : 0};
    hipStream_t st = (hipStream_t)stream;
    const int64_t nblk = n / hb;
    const size_t shm = stage ? (size_t)(n * esz) : 0;
    switch (L) {
    case 1: launch_rht_l<1>(a, nblk, batch, shm, st); break;
    case 2: launch_rht_l<2>(a, nblk, batch, shm, st); break;
    case 3: launch_rht_l<3>(a, nblk, batch, shm, st); break;
    case 4: launch_rht_l<4>(a, nblk, batch, shm, st); break;
    case 5: launch_rht_l<5>(a, nblk, batch, shm, st); break;
    case 6: launch_rht_l<6>(a, nblk, batch, shm, st); break;
    case 7: launch_rht_l<7>(a, nblk, batch, shm, st); break;
    case 8: launch_rht_l<8>(a, nblk, batch, shm, st); break;
    case 9: launch_rht_l<9>(a, nblk, batch, shm, st); break;
    case 10: launch_rht_l<10>(a, nblk, batch, shm, st); break;
    case 11: launch_rht_l<11>(a, nblk, batch, shm, st); break;
    case 12: launch_rht_l<12>(a, nblk, batch, shm, st); break;
    default: launch_rht_l<13>(a, nblk, batch, shm, st); break;
    }
    hipError_t err = hipGetLastError();
    if (err != hipSuccess) return set_hip_error(err, "vq2 rht launch");
    return VQ2_OK;
}

}  // namespace vq2
