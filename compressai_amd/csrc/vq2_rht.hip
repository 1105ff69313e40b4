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
};

template <int L>
struct RhtShape {
    static constexpr int HB = 1 << L;
    static constexpr int V = HB <= 128 ? 2 : (HB / 64 < 32 ? HB / 64 : 32);
    static constexpr int VB = V == 2 ? 1 : V == 4 ? 2 : V == 8 ? 3 : V == 16 ? 4 : 5;
    static constexpr int T = HB / V;
    static constexpr int NP = (L + VB - 1) / VB;
    static constexpr int width(int p) { return L / NP + (p < L % NP ? 1 : 0); }
    static constexpr int lo(int p)
    {
        int s = 0;
        for (int i = 0; i < p; i++) s += width(i);
        return s;
    }
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

template <int L>
__global__ void __launch_bounds__(256) rht_kernel(const RhtArgs a)
{
    using S = RhtShape<L>;
    __shared__ float lds[S::NP > 1 ? S::HB : 1];
    const int tid = threadIdx.x;
    const int64_t base = (int64_t)blockIdx.x * S::HB;
    const int64_t b = blockIdx.y;
    float v[S::V];

    // pass-0 layout: thread tid holds elements tid*V + i
#pragma unroll
    for (int i = 0; i < S::V; i++) {
        const int64_t gi = base + tid * S::V + i;
        float val;
        if (a.inverse) {
            val = load_as_f32(a.x, a.x_dt, b * a.x_stride + gi);
        } else {
            const int64_t src = a.perm ? (int64_t)a.perm[gi] : gi;
            if ((uint64_t)src >= (uint64_t)a.n) {
                val = __builtin_nanf("");  // not a permutation of [0, n): poison, never read out of bounds
            } else if (a.swiglu) {
                const float g = load_as_f32(a.x, a.x_dt, b * a.x_stride + src);
                const float u = load_as_f32(a.x, a.x_dt, b * a.x_stride + a.inter + src);
                val = silu_f32(g) * u;
            } else {
                val = load_as_f32(a.x, a.x_dt, b * a.x_stride + src);
            }
            if (a.sign) val *= (float)a.sign[gi];
        }
        v[i] = val;
    }

    rht_passes<L, 0>(v, lds, tid);

    constexpr int WL = S::width(S::NP - 1);
    constexpr int LOL = S::lo(S::NP - 1);
#pragma unroll
    for (int i = 0; i < S::V; i++) {
        const int64_t gi = base + elem_of<S::VB, WL, LOL>(tid, i);
        float val = v[i] * a.scale;
        int64_t dst = gi;
        if (a.inverse) {
            if (a.sign) val *= (float)a.sign[gi];
            if (a.perm) dst = a.perm[gi];
            if ((uint64_t)dst >= (uint64_t)a.n) continue;  // bad permutation entry: drop the store
        }
        store_from_f32(a.y, a.y_dt, b * a.y_stride + dst, val);
    }
}

template <int L>
static void launch_rht_l(const RhtArgs& a, int64_t nblk, int64_t batch, hipStream_t st)
{
    hipLaunchKernelGGL((rht_kernel<L>), dim3((unsigned)nblk, (unsigned)batch), dim3(RhtShape<L>::T), 0, st, a);
}

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
    RhtArgs a{x, x_dt, x_stride, y, y_dt, y_stride, perm, sign, scale, inverse, swiglu, inter, n};
    hipStream_t st = (hipStream_t)stream;
    const int64_t nblk = n / hb;
    switch (L) {
    case 1: launch_rht_l<1>(a, nblk, batch, st); break;
    case 2: launch_rht_l<2>(a, nblk, batch, st); break;
    case 3: launch_rht_l<3>(a, nblk, batch, st); break;
    case 4: launch_rht_l<4>(a, nblk, batch, st); break;
    case 5: launch_rht_l<5>(a, nblk, batch, st); break;
    case 6: launch_rht_l<6>(a, nblk, batch, st); break;
    case 7: launch_rht_l<7>(a, nblk, batch, st); break;
    case 8: launch_rht_l<8>(a, nblk, batch, st); break;
    case 9: launch_rht_l<9>(a, nblk, batch, st); break;
    case 10: launch_rht_l<10>(a, nblk, batch, st); break;
    case 11: launch_rht_l<11>(a, nblk, batch, st); break;
    case 12: launch_rht_l<12>(a, nblk, batch, st); break;
    default: launch_rht_l<13>(a, nblk, batch, st); break;
    }
    hipError_t err = hipGetLastError();
    if (err != hipSuccess) return set_hip_error(err, "vq2 rht launch");
    return VQ2_OK;
}

}  // namespace vq2
