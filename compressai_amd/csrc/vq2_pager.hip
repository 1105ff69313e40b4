// vq2_pager.hip -- device-resident expert pager for the paged MoE pool
// (gfx950).
//
// The reference pages experts on the host: every step it reads the routed
// ids back, walks an LRU dict and copies each missing expert synchronously
// (vq2/paged_runtime.py:415-437, 491-500).  Here the slot tables live on the
// device and two small launches do the paging, so a step needs no host
// synchronisation and can be captured in a HIP graph:
//  * pager_kernel (one workgroup): loads the tables into LDS, stamps the
//    slots of resident experts used by the step with the step clock, picks
//    the least recently stamped slots not used by the step for the missing
//    experts (distinct experts, in pair order; ties to the lower slot),
//    updates the tables, and writes the slot of every pair plus the list of
//    (expert, slot) copies;
//  * pager_copy_kernel: copies the listed experts' container records from a
//    pinned host mirror of the layer (read from the .vq2m file at load time)
//    into their slots over PCIe, the fp16 row scales converted to the pool's
//    scale dtype (round to nearest even, as torch's copy_ rounds them).
// A pair whose expert id is outside [0, n_experts), or whose expert could
// not get a slot (more distinct experts than slots), gets slot -1: the
// grouped GEMV kernels give NaN rows for it, and state[4] records why.
#include "vq2_common.hpp"
#include "vq2_internal.hpp"

namespace vq2 {

constexpr int PG_THREADS = 256;

struct PagerArgs {
    const void* ids;
    int ids_i64;
    int n_pairs;
    int n_experts;
    int capacity;
    int32_t* slot_of;    // [n_experts]: slot or -1
    int32_t* expert_of;  // [capacity]: expert or -1
    int32_t* stamp;      // [capacity]: step clock of the last use, -1 if never used
    int32_t* state;      // [0] clock, [1] copies of this step, [2] hits, [3] misses, [4] error bits
    int32_t* copy_list;  // [n_pairs][2]: (expert, slot)
    int32_t* pair_slot;  // [n_pairs]
};

__global__ void __launch_bounds__(PG_THREADS) pager_kernel(const PagerArgs a)
{
    extern __shared__ __align__(16) int lds[];
    const int E = a.n_experts, C = a.capacity, NP = a.n_pairs;
    const int C4 = (C + 3) & ~3;
    int* s_stamp = lds;            // [C4] (16-byte aligned; entries C.. hold the clock)
    int* s_slot = s_stamp + C4;    // [E]
    int* s_first = s_slot + E;     // [E]: lowest pair index of a missing expert
    int* s_exp = s_first + E;      // [C]
    int* s_pe = s_exp + C;         // [NP]: the pair's expert, -1 if invalid
    int* s_miss = s_pe + NP;       // [NP]: distinct missing experts in pair order
    int* s_vict = s_miss + NP;     // [NP]: victim slot of miss r
    __shared__ int s_nmiss, s_nelig, s_err, s_hits;
    const int tid = threadIdx.x;
    const int clock = a.state[0] + 1;
    for (int i = tid; i < E; i += PG_THREADS) {
        s_slot[i] = a.slot_of[i];
        s_first[i] = 0x7FFFFFFF;
    }
    for (int i = tid; i < C4; i += PG_THREADS) {
        if (i < C) s_exp[i] = a.expert_of[i];
        s_stamp[i] = i < C ? a.stamp[i] : clock;  // padding: "used this step", never a victim
    }
    int err = 0;
    for (int i = tid; i < NP; i += PG_THREADS) {
        const int64_t e = a.ids_i64 ? ((const int64_t*)a.ids)[i] : (int64_t)((const int32_t*)a.ids)[i];
        const bool ok = e >= 0 && e < E;
        s_pe[i] = ok ? (int)e : -1;
        err |= ok ? 0 : 1;
    }
    if (tid == 0) {
        s_nmiss = 0;
        s_nelig = 0;
        s_err = 0;
        s_hits = 0;
    }
    __syncthreads();
    if (err) atomicOr(&s_err, err);
    // resident experts used by this step: stamp their slots; missing ones:
    // remember their first pair
    int valid = 0;
    for (int i = tid; i < NP; i += PG_THREADS) {
        const int e = s_pe[i];
        if (e < 0) continue;
        valid++;
        const int sl = s_slot[e];
        if (sl >= 0) s_stamp[sl] = clock;
        else atomicMin(&s_first[e], i);
    }
    if (valid) atomicAdd(&s_hits, valid);  // valid pairs; the distinct misses are taken off below
    __syncthreads();
    // distinct missing experts in pair order: wave 0 compacts with ballots
    if (tid < 64) {
        int base = 0;
        for (int i0 = 0; i0 < NP; i0 += 64) {
            const int i = i0 + tid;
            const int e = i < NP ? s_pe[i] : -1;
            const bool own = e >= 0 && s_slot[e] < 0 && s_first[e] == i;
            const uint64_t m = __ballot(own);
            if (own) s_miss[base + __popcll(m & ((1ull << tid) - 1))] = e;
            base += __popcll(m);
        }
        if (tid == 0) s_nmiss = base;
    }
    __syncthreads();
    const int nmiss = s_nmiss;
    // victims: slots not used by this step, oldest stamp first (ties: lower
    // slot); the slot of rank r serves miss r.  A step with no misses skips
    // the ranking (uniform: nmiss is in LDS); the stamps are read four at a
    // time (all threads read the same words: LDS broadcasts)
    if (nmiss > 0) {
        for (int s = tid; s < C; s += PG_THREADS) {
            const int st = s_stamp[s];
            if (st == clock) continue;
            int rank = 0;
#pragma unroll 4
            for (int o = 0; o < C4; o += 4) {
                const int4 so = *(const int4*)(s_stamp + o);
                rank += (so.x != clock && (so.x < st || (so.x == st && o < s))) ? 1 : 0;
                rank += (so.y != clock && (so.y < st || (so.y == st && o + 1 < s))) ? 1 : 0;
                rank += (so.z != clock && (so.z < st || (so.z == st && o + 2 < s))) ? 1 : 0;
                rank += (so.w != clock && (so.w < st || (so.w == st && o + 3 < s))) ? 1 : 0;
            }
            if (rank < nmiss) s_vict[rank] = s;
            atomicAdd(&s_nelig, 1);
        }
        __syncthreads();
    }
    const int served = min(nmiss, s_nelig);
    if (tid == 0 && served < nmiss) atomicOr(&s_err, 2);
    for (int r = tid; r < served; r += PG_THREADS) {
        const int old = s_exp[s_vict[r]];
        if (old >= 0) s_slot[old] = -1;  // evicted (not used by this step)
    }
    __syncthreads();
    for (int r = tid; r < served; r += PG_THREADS) {
        const int e = s_miss[r], v = s_vict[r];
        s_slot[e] = v;
        s_exp[v] = e;
        s_stamp[v] = clock;
        a.copy_list[2 * r] = e;
        a.copy_list[2 * r + 1] = v;
    }
    __syncthreads();
    for (int i = tid; i < NP; i += PG_THREADS) {
        const int e = s_pe[i];
        a.pair_slot[i] = e >= 0 ? s_slot[e] : -1;
    }
    for (int i = tid; i < E; i += PG_THREADS) a.slot_of[i] = s_slot[i];
    for (int i = tid; i < C; i += PG_THREADS) {
        a.expert_of[i] = s_exp[i];
        a.stamp[i] = s_stamp[i];
    }
    if (tid == 0) {
        a.state[0] = clock;
        a.state[1] = served;
        a.state[2] += s_hits - nmiss;  // a repeated missing expert's later pairs are hits, as on the host
        a.state[3] += nmiss;
        a.state[4] |= s_err;
    }
}

constexpr int PG_CHUNK = 8192;  // bytes of a record per work item
constexpr int PG_COPY_WGS = 512;  // copy workgroups at most (each loops over work items)

struct PagerCopyArgs {
    const uint8_t* mirror;  // device address of the pinned host mirror [n_experts][record_bytes]
    int64_t record_bytes;
    const int32_t* copy_list;
    const int32_t* state;
    int64_t seg_bytes[4];   // gate_up index plane, its fp16 scales, down index plane, its fp16 scales
    int64_t seg_off[4];     // offsets in a record
    void* dst[4];           // the pool tensors
    int64_t dst_stride[4];  // bytes between slots
    int chunk0[5];          // first chunk of each segment (chunk0[4] = total)
    int scale_dt;
    int max_copies;         // entries of copy_list
};

// Work item i = (copy r, chunk c) = (i / chunks, i % chunks) of the
// state[1] copies this step; workgroup b takes items b, b + grid, ...  (a
// fixed grid of at most PG_COPY_WGS: a step with nothing to copy dispatches
// that many workgroups, not one per (copy slot, chunk) -- 1,192 for the
// sorted records of the 35B expert shape)
__global__ void __launch_bounds__(256) pager_copy_kernel(const PagerCopyArgs a)
{
    const int chunks = a.chunk0[4];
    const int items = min(max(a.state[1], 0), a.max_copies) * chunks;  // uniform
    for (int i = blockIdx.x; i < items; i += gridDim.x) {
        const int r = i / chunks, c = i - r * chunks;
        const int e = a.copy_list[2 * r], v = a.copy_list[2 * r + 1];
        int s = 0;
#pragma unroll
        for (int k = 1; k < 4; k++) s += c >= a.chunk0[k] ? 1 : 0;
        const int64_t b0 = (int64_t)(c - a.chunk0[s]) * PG_CHUNK;
        const int64_t b1 = min(b0 + PG_CHUNK, a.seg_bytes[s]);
        const uint8_t* src = a.mirror + (int64_t)e * a.record_bytes + a.seg_off[s];
        uint8_t* dst = (uint8_t*)a.dst[s] + (int64_t)v * a.dst_stride[s];
        if (s == 0 || s == 2) {
            for (int64_t b = b0 + (int64_t)threadIdx.x * 16; b < b1; b += 256 * 16)
                *(u32x4*)(dst + b) = *(const u32x4*)(src + b);
        } else {
            // 8 fp16 scales per thread and pass -> the pool's dtype
            for (int64_t b = b0 + (int64_t)threadIdx.x * 16; b < b1; b += 256 * 16) {
                const u32x4 w = *(const u32x4*)(src + b);
                const int64_t i0 = b / 2;
#pragma unroll
                for (int k = 0; k < 8; k++) {
                    const uint16_t h = (uint16_t)(w[k >> 1] >> (16 * (k & 1)));
                    store_from_f32(dst, a.scale_dt, i0 + k, f16_bits_to_f32(h));
                }
            }
        }
    }
}

size_t pager_lds_bytes(int64_t n_experts, int64_t capacity, int64_t n_pairs)
{
    return (size_t)(2 * n_experts + ((capacity + 3) & ~int64_t(3)) + capacity + 3 * n_pairs) * sizeof(int);
}

int pager_step_launch(const void* ids, int ids_i64, int64_t n_pairs, int64_t n_experts, int64_t capacity,
                      int32_t* slot_of, int32_t* expert_of, int32_t* stamp, int32_t* state, int32_t* copy_list,
                      int32_t* pair_slot, void* stream)
{
    const size_t shm = pager_lds_bytes(n_experts, capacity, n_pairs);
    if (shm > 64 * 1024)
        return set_error(VQ2_ERR_UNSUPPORTED, "vq2_pager_step: %lld experts, %lld slots, %lld pairs need %zu bytes of "
                         "LDS (at most 64 KiB)", (long long)n_experts, (long long)capacity, (long long)n_pairs, shm);
    PagerArgs a{ids, ids_i64, (int)n_pairs, (int)n_experts, (int)capacity, slot_of, expert_of, stamp, state,
                copy_list, pair_slot};
    hipLaunchKernelGGL(pager_kernel, dim3(1), dim3(PG_THREADS), shm, (hipStream_t)stream, a);
    const hipError_t err = hipGetLastError();
    return err == hipSuccess ? VQ2_OK : set_hip_error(err, "vq2_pager_step launch");
}

int pager_copy_launch(const void* mirror_host, int64_t record_bytes, const int64_t* seg_bytes, const int32_t* copy_list,
                      const int32_t* state, int64_t max_copies, void* const* dst, const int64_t* dst_stride,
                      int scale_dt, void* stream)
{
    PagerCopyArgs a{};
    void* dev = nullptr;
    hipError_t err = hipHostGetDevicePointer(&dev, const_cast<void*>(mirror_host), 0);
    if (err != hipSuccess || !dev)
        return set_hip_error(err == hipSuccess ? hipErrorInvalidValue : err,
                             "vq2_pager_copy: the mirror must be pinned host memory (hipHostMalloc / pin_memory)");
    if ((uintptr_t)dev % 16 || record_bytes % 16)
        return set_error(VQ2_ERR_ARG, "vq2_pager_copy: mirror and records must be 16-byte aligned");
    a.mirror = (const uint8_t*)dev;
    a.record_bytes = record_bytes;
    a.copy_list = copy_list;
    a.state = state;
    a.scale_dt = scale_dt;
    a.max_copies = (int)std::min<int64_t>(max_copies, 65535);
    int64_t off = 0, chunks = 0;
    for (int s = 0; s < 4; s++) {
        if (seg_bytes[s] < 16 || seg_bytes[s] % 16 || !dst[s] || (uintptr_t)dst[s] % 16 ||
            (s % 2 == 0 && dst_stride[s] % 16))
            return set_error(VQ2_ERR_ARG, "vq2_pager_copy: segment %d: sizes, strides and pointers must be 16-byte "
                             "aligned", s);
        a.seg_bytes[s] = seg_bytes[s];
        a.seg_off[s] = off;
        a.dst[s] = dst[s];
        a.dst_stride[s] = dst_stride[s];
        a.chunk0[s] = (int)chunks;
        off += seg_bytes[s];
        chunks += (seg_bytes[s] + PG_CHUNK - 1) / PG_CHUNK;
    }
    a.chunk0[4] = (int)chunks;
    if (off != record_bytes) return set_error(VQ2_ERR_ARG, "vq2_pager_copy: segments do not add up to the record");
    if (max_copies < 1 || max_copies > 65535 || chunks > 65535 || max_copies * chunks > 0x7FFFFFFF)
        return set_error(VQ2_ERR_UNSUPPORTED, "vq2_pager_copy: grid too large");
    const unsigned grid = (unsigned)std::min<int64_t>(max_copies * chunks, PG_COPY_WGS);
    hipLaunchKernelGGL(pager_copy_kernel, dim3(grid), dim3(256), 0, (hipStream_t)stream, a);
    err = hipGetLastError();
    return err == hipSuccess ? VQ2_OK : set_hip_error(err, "vq2_pager_copy launch");
}

}  // namespace vq2
