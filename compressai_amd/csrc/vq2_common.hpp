// vq2_common.hpp -- device helpers shared by the VQ2 decode-path kernels
// (gfx950 / CDNA4, wave64).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "vq2_amd.h"

namespace vq2 {

typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef _Float16 half4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

// ------------------------------------------------------------ conversions
__device__ __forceinline__ float bf16_bits_to_f32(uint32_t b16) { return __uint_as_float(b16 << 16); }

__device__ __forceinline__ float f16_bits_to_f32(uint16_t h) { return (float)__builtin_bit_cast(_Float16, h); }

// fp32 -> bf16 bits, round to nearest even, quiet NaN.
__device__ __forceinline__ uint16_t f32_to_bf16_bits(float f)
{
    uint32_t u = __float_as_uint(f);
    if ((u & 0x7F800000u) == 0x7F800000u && (u & 0x7FFFFFu)) return (uint16_t)((u >> 16) | 0x40u);
    u += 0x7FFFu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

__device__ __forceinline__ uint16_t f32_to_f16_bits(float f) { return __builtin_bit_cast(uint16_t, (_Float16)f); }

// Load element i of a float array of runtime dtype dt as fp32.
__device__ __forceinline__ float load_as_f32(const void* p, int dt, int64_t i)
{
    if (dt == VQ2_DT_F16) return f16_bits_to_f32(((const uint16_t*)p)[i]);
    if (dt == VQ2_DT_BF16) return bf16_bits_to_f32(((const uint16_t*)p)[i]);
    return ((const float*)p)[i];
}

// Bits of element i of an array of runtime dtype dt (fp32: the word; fp16 /
// bf16: the half in the low bits); raw_as_f32 converts them.  Kept apart so
// that a load can be issued early and waited for at its first use (a
// conversion inside the dtype branch makes the wait come at once).
__device__ __forceinline__ uint32_t load_raw(const void* p, int dt, int64_t i)
{
    return dt == VQ2_DT_F32 ? ((const uint32_t*)p)[i] : (uint32_t)((const uint16_t*)p)[i];
}

__device__ __forceinline__ float raw_as_f32(uint32_t r, int dt)
{
    if (dt == VQ2_DT_F16) return f16_bits_to_f32((uint16_t)r);
    if (dt == VQ2_DT_BF16) return bf16_bits_to_f32(r);
    return __uint_as_float(r);
}

// Store fp32 v into element i of an array of runtime dtype dt.
__device__ __forceinline__ void store_from_f32(void* p, int dt, int64_t i, float v)
{
    if (dt == VQ2_DT_F16)
        ((uint16_t*)p)[i] = f32_to_f16_bits(v);
    else if (dt == VQ2_DT_BF16)
        ((uint16_t*)p)[i] = f32_to_bf16_bits(v);
    else
        ((float*)p)[i] = v;
}

// ------------------------------------------------------- wave reductions
// Sum over aligned groups of `width` lanes (width a power of two <= 64);
// every lane of the group ends with the group sum.  Uses DPP row ops for the
// in-row steps and ds_swizzle / permlane32 for the cross-row ones.
__device__ __forceinline__ float dpp_xor1(float v)
{
    return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0xB1, 0xF, 0xF, true)); // quad_perm [1,0,3,2]
}
__device__ __forceinline__ float dpp_xor2(float v)
{
    return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x4E, 0xF, 0xF, true)); // quad_perm [2,3,0,1]
}
// row_half_mirror: lane i <- lane (i ^ 7) within each 8-lane half row
__device__ __forceinline__ float dpp_half_mirror(float v)
{
    return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x141, 0xF, 0xF, true));
}
// row_mirror: lane i <- lane (i ^ 15) within each 16-lane row
__device__ __forceinline__ float dpp_row_mirror(float v)
{
    return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x140, 0xF, 0xF, true));
}
// lane i <- lane i ^ 16 (ds_swizzle bit mode, and=0x1F, xor=0x10)
__device__ __forceinline__ float swz_xor16(float v)
{
    return __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(v), 0x401F));
}
// lane i <- lane i ^ 32
__device__ __forceinline__ float xor32(float v)
{
    return __int_as_float(__builtin_amdgcn_ds_bpermute((int)((threadIdx.x ^ 32) & 63) << 2, __float_as_int(v)));
}

// Group sum over `width` lanes.  After the xor1/xor2 steps every lane holds
// its quad sum, so mirrored partners (i^7, i^15) add the other half.
__device__ __forceinline__ float group_sum(float v, int width)
{
    if (width >= 2) v += dpp_xor1(v);
    if (width >= 4) v += dpp_xor2(v);
    if (width >= 8) v += dpp_half_mirror(v);
    if (width >= 16) v += dpp_row_mirror(v);
    if (width >= 32) v += swz_xor16(v);
    if (width >= 64) v += xor32(v);
    return v;
}

// Full-wave reductions that end uniform in every lane: DPP inside each row
// of 16, ds_swizzle across the rows of a 32-lane half, then the two halves
// combined through readlane.  Any pairing is valid for these commutative,
// associative operators.
template <int CTRL>
__device__ __forceinline__ int dpp_mov(int v)
{
    return __builtin_amdgcn_mov_dpp(v, CTRL, 0xF, 0xF, true);
}

__device__ __forceinline__ float wave_sum_all(float v)
{
    v += __int_as_float(dpp_mov<0xB1>(__float_as_int(v)));
    v += __int_as_float(dpp_mov<0x4E>(__float_as_int(v)));
    v += __int_as_float(dpp_mov<0x141>(__float_as_int(v)));
    v += __int_as_float(dpp_mov<0x140>(__float_as_int(v)));
    v += swz_xor16(v);
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0)) +
           __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32));
}

__device__ __forceinline__ float wave_max_all(float v)
{
    v = fmaxf(v, __int_as_float(dpp_mov<0xB1>(__float_as_int(v))));
    v = fmaxf(v, __int_as_float(dpp_mov<0x4E>(__float_as_int(v))));
    v = fmaxf(v, __int_as_float(dpp_mov<0x141>(__float_as_int(v))));
    v = fmaxf(v, __int_as_float(dpp_mov<0x140>(__float_as_int(v))));
    v = fmaxf(v, swz_xor16(v));
    return fmaxf(__int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0)),
                 __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32)));
}

// (value, index) maximum with ties to the lower index
__device__ __forceinline__ void argmax_step(float& v, int& i, float ov, int oi)
{
    if (ov > v || (ov == v && oi < i)) { v = ov; i = oi; }
}

template <int CTRL>
__device__ __forceinline__ void argmax_dpp(float& v, int& i)
{
    const float ov = __int_as_float(dpp_mov<CTRL>(__float_as_int(v)));
    const int oi = dpp_mov<CTRL>(i);
    argmax_step(v, i, ov, oi);
}

__device__ __forceinline__ void wave_argmax_all(float& v, int& i)
{
    argmax_dpp<0xB1>(v, i);
    argmax_dpp<0x4E>(v, i);
    argmax_dpp<0x141>(v, i);
    argmax_dpp<0x140>(v, i);
    argmax_step(v, i, swz_xor16(v), __builtin_amdgcn_ds_swizzle(i, 0x401F));
    const float v0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0));
    const int i0 = __builtin_amdgcn_readlane(i, 0);
    const float v1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32));
    const int i1 = __builtin_amdgcn_readlane(i, 32);
    v = v0;
    i = i0;
    argmax_step(v, i, v1, i1);
}

// Order-preserving 64-bit key: high word = float bits mapped to an unsigned
// order, low word = 0xFFFFFFFF - column, so an unsigned max picks the largest
// value and, among equal values, the smallest column (torch.argmax's first
// maximum).  NaN-free rows are assumed, as for the reference's logits.
__device__ __forceinline__ uint64_t argmax_key(float v, int64_t col)
{
    uint32_t u = __float_as_uint(v);
    u = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
    return ((uint64_t)u << 32) | (uint64_t)(0xFFFFFFFFu - (uint32_t)col);
}

// The column and value an argmax_key encodes.
__device__ __forceinline__ void argmax_key_decode(uint64_t key, int64_t* idx, float* val)
{
    const uint32_t lo = (uint32_t)(key & 0xFFFFFFFFu);
    uint32_t u = (uint32_t)(key >> 32);
    u = (u & 0x80000000u) ? (u & 0x7FFFFFFFu) : ~u;
    if (val) *val = __uint_as_float(u);
    *idx = (int64_t)(0xFFFFFFFFu - lo);
}

__device__ __forceinline__ float silu_f32(float v) { return v / (1.0f + __expf(-v)); }

// Touch every 64-byte line of the kernel arguments with independent scalar
// loads at entry.  The fields the kernel reads before its first index load
// (plan, segment, expert ids) come in a chain of dependent scalar loads with
// a wait after each; with the lines already in the scalar cache every link
// is a hit (measured on MI355X: first index load issued 0.4-0.5 us sooner).
template <typename T>
__device__ __forceinline__ void touch_kernargs(const T& a)
{
    const uint32_t* w = (const uint32_t*)&a;
    uint32_t h = 0;
#pragma unroll
    for (int i = 0; i < (int)(sizeof(T) / 4); i += 16) h ^= w[i];
    // an empty asm that takes the value keeps the loads.  (A never-taken
    // store to a sink compiled to a flat store, after which the compiler's
    // memory-counter waits fall back to waiting for every outstanding load.)
    asm volatile("; kernarg lines touched %0" ::"s"(h));
}

// ------------------------------------------- in-kernel split reductions
// A reduction split over workgroups is finished by the workgroup that
// arrives last, instead of by a second launch.  Each workgroup writes its
// share with agent-scope atomic stores (written through the XCD-private L2
// to the device's coherence point), waits until they are complete, and
// counts itself in; the one whose increment completes the count reads every
// share with agent-scope atomic loads (which do not hit stale L2 lines of
// another XCD's data) and puts the counter back to 0 for the next launch.
// Every location involved is only ever accessed through agent-scope atomics,
// so no agent-scope fence is needed (on gfx950 a release fence writes the
// whole L2 back and an acquire fence invalidates it: the codebook lines the
// other workgroups of that XCD are reading would be fetched again).
__device__ __forceinline__ void share_store(float* p, float v)
{
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float share_load(const float* p)
{
    return __hip_atomic_load((float*)p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Called by every thread of the workgroup after its share_store()s; true in
// every thread of the workgroup whose arrival is number `expected` at cnt.
// The counter must be 0 before the launch's first arrival; the last arrival
// leaves it 0.
__device__ __forceinline__ bool arrive_last(uint32_t* cnt, uint32_t expected)
{
    __shared__ int s_last;
    // this wave's share stores are complete (acknowledged at the coherence
    // point) before the barrier, so all of the workgroup's are before the
    // increment
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    if (threadIdx.x == 0) {
        const uint32_t old = __hip_atomic_fetch_add(cnt, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        const int last = old + 1u == expected;
        if (last) __hip_atomic_store(cnt, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        s_last = last;
    }
    __syncthreads();
    return s_last != 0;
}

}  // namespace vq2
