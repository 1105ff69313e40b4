// vq2_sorted_moe.hip -- the MoE expert path over code-sorted expert pools
// (gfx950).
//
// Per token t and pair k (expert e = ids[t, k], weight w[t, k]), as the
// reference's expert loop computes it (vq2/paged_runtime.py:495-510,
// vq2/load_and_test_full_35b.py:75-95):
//
//   gu    = VQ(gate_up[e]) . RHT_H(h_t)                       [2I]
//   act   = RHT_I(silu(gu[:I]) * gu[I:])                      [I]
//   out_t = sum_k w[t, k] * VQ(down[e]) . act                  [H]
//
// Both pools are in the code-sorted layout (vq2_sorted_pack_pool: every
// expert a matrix of C chunks of R rows, experts one after another), so a
// wave's 64 centroid gathers share a few codebook lines (vq2_sorted.hip
// explains the layout).  Three launches, no host synchronisation (for
// hidden 2048 / intermediate 512, parts 1 and 2 are one launch whose down
// workgroups wait, bounded, on per-pair counts: vq_sorted_moe_fused_kernel):
//  1. gate_up: one workgroup per (pair, chunk, slice).  The expert comes from
//     ids (MODE 0) or from the router built in (MODE 1: softmax over the
//     token's logits, top-k, renormalised; slot k is the shared expert with
//     sigmoid(gate . h_t); the (pair, chunk 0, slice 0) workgroup publishes
//     the pair's id and weight).  The workgroup builds RHT_H(h_t) in LDS and
//     writes the raw row sums of its slice (unscaled) to a workspace.
//  2. down (MODE 2): one workgroup per (pair, chunk, slice); its prologue adds
//     the gate_up slices of its pair in slice order, applies the gate_up row
//     scales, silu(gate) * up, and RHT_I in LDS, then the down slice.
//     Each down slice writes its share w[t, k] * (row sum * s[e][row]).
//  3. combine: out_t[row] = the sum of those shares over the token's pairs
//     and the slices, in a fixed order (deterministic).
// An expert id outside the pool gives NaN for its pair (never an
// out-of-bounds read), as the gather kernels do.
#include <algorithm>
#include <atomic>
#include <mutex>

#include "vq2_internal.hpp"
#include "vq2_router.hpp"
#include "vq2_sorted.hpp"

namespace vq2 {

struct SortedPoolArgs {
    const uint32_t* ent;
    const void* scale;  // [n_experts, rows]
    const void* cb1;    // stage-2 codebook (two-stage pools), else nullptr
    uint32_t c1mask;    // stage-2 code mask: 0xFFFF, or 0xFF for the 256-row codebook of (16,8)
    int32_t ipc1;       // stage-1 iterations of a chunk (the stage-2 ones follow)
    int32_t ipc;        // iterations per chunk (every chunk padded to it)
    int s_dt;
    int32_t n_iters;
    int R;     // rows per chunk at most (row R is the dummy row)
    int C;     // chunks per expert
    int rb;    // chunk c: rows [c * rb + min(c, nbig), + rb + (c < nbig))
    int nbig;
    int rows;  // rows per expert
    int ng;    // groups per row
    int gbits;
};

struct SortedMoeArgs {
    // prologue fields: x = h [tokens, H] (token stride x_pstride, x_pdiv 1),
    // the rotation (perm, sign, hb_log2, xscale) of this launch, and the
    // fused router (r_*) of MODE 1
    GemvArgs g;
    SortedPoolArgs pool;
    const void* cb;
    int64_t n_experts;
    int P;        // pairs per token
    int n_pairs;  // tokens * P
    int slices;
    int sq, sr;   // slice j of a chunk: sq + (j < sr) iterations, from j * sq + min(j, sr)
    int xmap;     // 1: XCD-ordered units (several slices, one round of workgroups)
    int xq, xr;   // workgroups / 8, workgroups % 8
    int wgs;      // workgroups of this part of the launch (more are padding)
    // one launch for gate_up and down (pair_cnt non-null): gate_up counts
    // its finished workgroups per pair; down waits for gu_arrivals of them
    uint32_t* pair_cnt;
    int gu_arrivals;
    int id_poll;     // down part of one launch with the router: the pair's (id, weight) is published in the launch
    int max_polls;   // bound of each wait (polls of ~640 clocks each)
    uint32_t* status;  // sticky wait-timeout bits (VQ2_MOE_WAIT_*), never cleared by the kernels
    const void* ids;  // MODE 0 / 2 and the combine: pair experts
    int ids_i64;
    float* part;  // gate_up: [slices][n_pairs][pool.rows] raw row sums; down: [n_pairs][slices][pool.rows] shares
    // MODE 2: the gate_up launch's partials and scales
    const float* gu_part;
    int gu_slices;
    int gu_rows;
    const void* gu_scale;
    int gu_s_dt;
    // combine
    const float* w;
    void* out;
    int out_dt;
};

// LDS floats between the natural-order activation and the accumulators:
// the stage, later the split activation (n), and after it the 512-point
// rotation's scratch of the down part (MODE 2) in the all-threads form.
__host__ __device__ constexpr int64_t moe_split_floats(int mode, int f2k, int64_t n)
{
    return mode == 2 && f2k != 0 ? n + RHT512 : n;
}

// The pair's expert id by a scalar load (p is wave-uniform): waiting for it
// does not wait for the vector loads issued before it.  In the down launch
// the ids come from the gate_up launch before it (the scalar cache starts
// every launch empty).
__device__ __forceinline__ int64_t pair_expert(const SortedMoeArgs& a, int p, bool& bad)
{
    const int64_t e = a.ids_i64 ? uniform_load<int64_t>(a.ids, p) : (int64_t)uniform_load<int32_t>(a.ids, p);
    bad = e < 0 || e >= a.n_experts;
    return bad ? 0 : e;
}

// The router's top-k by wave 0 alone.  Each lane turns its 4 probabilities
// (router_probs: the same arithmetic as router_select) into 64-bit keys
// (bits of p) << 32 | (0xFFFFFFFF - expert) -- p >= 0, so a larger key is a
// larger probability, or an equal one with a lower id: the order of
// router_select's k argmax rounds -- and sorts them, descending.  Each
// round takes the wave maximum of the lanes' first keys (DPP within rows,
// row broadcasts across rows: no LDS), and the winning lane shifts its
// keys.  Lane r < k ends with the rank-r key.
template <int DPP, int ROW_MASK>
__device__ __forceinline__ uint64_t dpp_max_u64(uint64_t v)
{
    const uint32_t lo = (uint32_t)v, hi = (uint32_t)(v >> 32);
    const uint32_t olo = (uint32_t)__builtin_amdgcn_update_dpp((int)lo, (int)lo, DPP, ROW_MASK, 0xF, false);
    const uint32_t ohi = (uint32_t)__builtin_amdgcn_update_dpp((int)hi, (int)hi, DPP, ROW_MASK, 0xF, false);
    const uint64_t o = ((uint64_t)ohi << 32) | olo;
    return o > v ? o : v;
}

__device__ __forceinline__ uint64_t route_topk_keys(const GemvArgs& g, int64_t t, int lane)
{
    float pr[4];
    router_probs<4>(g.r_logits, g.r_ldt, t, g.r_ne, lane, pr);
    uint64_t k0, k1, k2, k3;
    {
        uint64_t key[4];
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const uint32_t ex = (uint32_t)(j * 64 + lane);
            key[j] = ex < (uint32_t)g.r_ne ? ((uint64_t)__float_as_uint(pr[j]) << 32) | (0xFFFFFFFFu - ex) : 0;
        }
        auto cs = [](uint64_t& x, uint64_t& y) {  // x >= y afterwards
            const uint64_t hi = x > y ? x : y, lo = x > y ? y : x;
            x = hi;
            y = lo;
        };
        cs(key[0], key[1]);
        cs(key[2], key[3]);
        cs(key[0], key[2]);
        cs(key[1], key[3]);
        cs(key[1], key[2]);
        k0 = key[0], k1 = key[1], k2 = key[2], k3 = key[3];
    }
    uint64_t mine = 0;
    for (int r = 0; r < g.r_k; r++) {
        uint64_t m = k0;
        m = dpp_max_u64<0xB1, 0xF>(m);   // quad_perm [1,0,3,2]
        m = dpp_max_u64<0x4E, 0xF>(m);   // quad_perm [2,3,0,1]
        m = dpp_max_u64<0x141, 0xF>(m);  // row_half_mirror
        m = dpp_max_u64<0x140, 0xF>(m);  // row_mirror: every lane holds its row's maximum
        m = dpp_max_u64<0x142, 0xA>(m);  // row_bcast:15 into rows 1 and 3
        m = dpp_max_u64<0x143, 0xC>(m);  // row_bcast:31 into rows 2 and 3: lane 63 holds the maximum
        const uint64_t best = ((uint64_t)(uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(m >> 32), 63) << 32) |
                              (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)m, 63);
        if (lane == r) mine = best;
        if (k0 == best) {  // keys are distinct: one lane shifts
            k0 = k1;
            k1 = k2;
            k2 = k3;
            k3 = 0;
        }
    }
    return mine;
}

constexpr int SG_MAX_TOPK = 64;

// MODE 0: gate_up, ids given; MODE 1: gate_up with the router; MODE 2: down.
// XT: dtype of h (MODE 0 / 1).
//
// Order of the prologue: the activation (or gate_up partial) loads, then the
// expert's first entry words; the activation is staged and rotated in LDS
// while the entry words come from HBM; the first centroid gathers are issued
// after the prologue (the entry words have arrived by then).
// F2K (MODE 0 / 1): hidden = 2048 rotated as one 2048-point block, the
// all-threads prologue (rht2k_stage / rht2k_transform).  The block count is
// a constant there, so no load of the prologue sits behind a branch and the
// compiler's load counts stay exact across the router's branches (with a
// runtime block count the transform waited for the first entry words).
// FUSED: gate_up and down in one launch (vq_sorted_moe_fused_kernel).  The
// gate_up workgroups publish their row sums and the router's ids and
// weights with agent-scope stores and count themselves in per pair; each
// down workgroup waits (a bounded poll) until its pair's count is complete,
// then reads them with agent-scope loads.  Nothing else is shared, so no
// agent-scope fence is needed (see arrive_last).
// Each pair's count has a 128-byte line of its own, and a waiting thread
// polls every ~640 clocks: with the counts packed in one line and a poll
// every ~128 clocks the polls and the gate_up increments contended for it
// (measured, T = 1 layer: 25.8 us fused against 20.9 us in two launches;
// padded, 20.15 us; with no wait at all, wrong results, 19.45 us).
constexpr int MOE_CNT_STRIDE = 32;        // uint32 per pair count
// Each wait is bounded: after max_polls polls (each a sleep of 640 clocks,
// ~0.27 us at 2.4 GHz, plus the agent-scope load's round trip; the default
// 2^20 is at least ~0.3 s) the waiting workgroup gives up, ORs its bit
// (VQ2_MOE_WAIT_ID: the pair's published id; VQ2_MOE_WAIT_COUNT: the
// pair's gate_up count) into the status word of the workspace header, and
// its pair's shares turn NaN.  Forward progress relies on the dispatcher
// starting workgroups in index order on each XCD (every gate_up workgroup
// precedes every down workgroup of its XCD, and gate_up workgroups wait for
// nothing), so a give-up means the order was broken or the launch was fed
// an unreachable count; the host reads the bits (vq2_sorted_moe_status).

// The router's pair (expert id + 1, combine weight) as one 64-bit word in
// the pair's count line (words 2-3), so a down workgroup can load its entry
// words while the pair's gate_up workgroups still run; 0 = not yet.
__device__ __forceinline__ uint64_t* pair_word(const SortedMoeArgs& a, int p)
{
    return (uint64_t*)(a.pair_cnt + p * MOE_CNT_STRIDE + 2);
}
__device__ __forceinline__ void publish_pair(const SortedMoeArgs& a, int p, uint32_t ex, float w)
{
    __hip_atomic_store(pair_word(a, p), ((uint64_t)__float_as_uint(w) << 32) | (uint64_t)(ex + 1u), __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_AGENT);
}

template <int CBT, int MODE, int XT, int F2K, int FUSED>
__device__ __forceinline__ void moe_body(const SortedMoeArgs& a, int bid, float* smem)
{
    __shared__ float s_red[4][256];
    __shared__ int s_top[SG_MAX_TOPK];
    __shared__ float s_topv[SG_MAX_TOPK];
    __shared__ int32_t s_e;
    __shared__ float s_w;
    __shared__ int s_ok;
    if (bid >= a.wgs) return;  // padding of a fused launch (whole workgroup, before any barrier)
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    const SortedPoolArgs& pl = a.pool;
    const int64_t n = (int64_t)pl.ng * 8;
    // [natural-order activation: n][stage (n), later the split activation
    // (n floats, halves xb = n / 2 apart); the down part's 512-point
    // rotation also has its scratch there, n floats on][accumulators]
    const int xb = (int)(n / 2);
    float* s_x = smem;
    float* s_stage = smem + n;
    float* s_split = smem + n;
    float* s_acc = s_split + moe_split_floats(MODE, F2K, n);  // SG_WAVES x SG_PARTS x (R + 1)
    const int R = pl.R;
    // Workgroup b runs on XCD b % 8; with xmap each XCD takes a contiguous
    // run of the (slice, pair, chunk) units in slice-major order.  A slice is
    // a contiguous code range of every chunk (all experts share the
    // codebook), so an XCD's L2 holds one or two slices' share of it.  The
    // host sets xmap when there are several slices and the grid fits one
    // round of workgroups (measured: T = 1 layer 27.8 -> 25.4-25.9 us; with
    // two slices over 2.8 rounds, T = 8, the plain order was faster; the
    // dense sorted GEMV gained nothing from it).
    const int xcd = bid & 7;
    const int pos = a.xmap ? xcd * a.xq + min(xcd, a.xr) + (bid >> 3) : bid;
    const int units = a.n_pairs * pl.C;
    // xmap: slice-major (a slice's code range per XCD); else pair-major (a
    // pair's chunks and slices consecutive, so the pairs of a later round
    // are whole pairs and the earlier ones complete in the first)
    const int slice = a.xmap ? pos / units : pos % a.slices;
    const int unit = a.xmap ? pos - slice * units : pos / a.slices;
    const int p = unit / pl.C, chunk = unit - p * pl.C;
    const int t = p / a.P, kslot = p - t * a.P;

    // prologue loads first: the token's activation and the rotation tables
    // (MODE 0 / 1), or the tables alone (MODE 2)
    // F2K: the all-threads rotation (MODE 0 / 1: one 2048-point block of h;
    // MODE 2: one 512-point block), which stores the split layout itself
    constexpr bool FAST = F2K != 0 && MODE != 2;
    XProLoad first;
    Rht2kLoad first2k;
    RhtPairLoad first512;
    constexpr int k2k = 1;
    const int64_t t0 = (int64_t)threadIdx.x * 8;
    if constexpr (FAST) rht2k_load<XT>(a.g, k2k, (int64_t)t * a.g.x_pstride, first2k);
    else if constexpr (MODE != 2) xpro_load<1, XT>(a.g, t0 < n ? t0 : 0, n, t, 0, first);
    else if constexpr (F2K != 0) rht512_load(a.g, first512);
    else xpro_tables(a.g, t0 < n ? t0 : 0, n, first);

    // chunk `chunk` of expert ex: iterations [(ex * C + chunk) * ipc, + ipc)
    // (in the pool: ex < n_experts, chunk < C), this slice's share of them
    // gathers two iterations ahead in gate_up, one in down (measured, one
    // workgroup per CU: T = 1 layer 22.7 / 21.4 / 23.2 / 21.0 us for 1-1,
    // 2-2, 1-2, 2-1); one ahead in both parts of the one launch with fp16
    // codebooks, which runs two workgroups per CU (vq_sorted_moe_fused_kernel)
    SortedPipe<CBT, (MODE == 2 || (FUSED && CBT == VQ2_DT_F16)) ? 1 : 2> pipe;
    auto entries = [&](int64_t ex) {
        const int c_beg = (int)((ex * pl.C + chunk) * pl.ipc);
        const int s0 = c_beg + slice * a.sq + min(slice, a.sr);
        const int s1 = s0 + a.sq + (slice < a.sr ? 1 : 0);
        pipe.load_entries(pl.ent, a.cb, pl.cb1, c_beg, c_beg + pl.ipc1, s0, s1, wave, lane, pl.gbits, R,
                          pl.c1mask);
    };
    float* acc = sorted_acc(s_acc, wave, lane, R);
    bool bad = false;
    int64_t e = 0;
    float wp = 1.0f;    // MODE 2: the pair's combine weight
    uint32_t dsc = 0u;  // MODE 2: raw bits of the row's down scale

    if constexpr (MODE == 0) {
        e = pair_expert(a, p, bad);
        entries(e);
        sorted_acc_zero(acc, lane, R);
        if constexpr (FAST) {
            rht2k_build<XT>(k2k, n, first2k, s_stage, s_x, s_split, a.g.xscale, xb);
        } else {
            stage_x<1, XT>(a.g, s_stage, 1, n, t, 0, first);
            build_x<1, XT>(a.g, s_x, s_stage, 1, n, first);
        }
    } else if constexpr (MODE == 1) {
        // the router in wave 0 (route_topk_keys); the shared expert's pairs
        // know their expert at once
        const bool routed = kslot < a.g.r_k;
        const bool writer = chunk == 0 && slice == 0 && wave == 0;
        if (!routed) {
            e = a.g.r_shared;
            entries(e);
            if (writer) {
                const float sw = router_shared_weight(a.g.r_gate, a.g.r_gdt, a.g.x, a.g.x_dt, t, n, lane);
                if (lane == 0) {
                    __hip_atomic_store(a.g.r_ids + p, (int32_t)a.g.r_shared, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    share_store(a.g.r_w + p, sw);
                    if constexpr (FUSED) publish_pair(a, p, (uint32_t)a.g.r_shared, sw);
                }
            }
        } else if (wave == 0) {
            const uint64_t key = route_topk_keys(a.g, t, lane);
            const uint32_t exu = 0xFFFFFFFFu - (uint32_t)key;
            const int ex = exu < (uint32_t)a.g.r_ne ? (int)exu : 0;  // in bounds whatever the logits hold
            if (lane < a.g.r_k) {
                s_top[lane] = ex;
                s_topv[lane] = __uint_as_float((uint32_t)(key >> 32));
            }
            if (writer) {
                // weight = p / (sum of the k chosen p), summed as router_select
                // sums it (lane r holds rank r)
                const float mine = lane < a.g.r_k ? __uint_as_float((uint32_t)(key >> 32)) : 0.0f;
                const float tot = wave_sum_all(mine);
                if (lane == kslot) {
                    __hip_atomic_store(a.g.r_ids + p, (int32_t)ex, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    share_store(a.g.r_w + p, mine / tot);
                    if constexpr (FUSED) publish_pair(a, p, (uint32_t)ex, mine / tot);
                }
            }
        }
        sorted_acc_zero(acc, lane, R);
        // the staging ends with a barrier: s_top is visible
        if constexpr (FAST) rht2k_stage<XT>(k2k, first2k, s_stage);
        else stage_x<1, XT>(a.g, s_stage, 1, n, t, 0, first);
        if (routed) {
            e = s_top[kslot];
            entries(e);
        }
        if constexpr (FAST) rht2k_transform<XT>(k2k, n, first2k, s_stage, s_x, s_split, a.g.xscale, xb);
        else build_x<1, XT>(a.g, s_x, s_stage, 1, n, first);
    } else {
        // the pair's gate_up rows: slices added in order, row scale, then
        // silu(gate) * up (elementwise, so taken before the permutation).
        // Thread i < 2n takes value i of [gate | up]; its slice loads (from
        // other XCDs' writes: memory round trips) are issued together, before
        // the expert id and the entry words.
        const int64_t gstride = (int64_t)a.n_pairs * a.gu_rows;
        const float* gp = a.gu_part + (int64_t)p * a.gu_rows;
        if constexpr (FUSED) {
            // the pair's expert id and combine weight: given, or published
            // by the router's writer in this launch (a bounded poll)
            if (threadIdx.x == 0) {
                int64_t ev = -1;
                float wv = 0.0f;
                if (a.id_poll) {
                    for (int it = 0; it < a.max_polls; it++) {
                        const uint64_t v = __hip_atomic_load(pair_word(a, p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                        if ((uint32_t)v != 0u) {
                            ev = (int64_t)((uint32_t)v - 1u);
                            wv = __uint_as_float((uint32_t)(v >> 32));
                            break;
                        }
                        __builtin_amdgcn_s_sleep(10);
                    }
                    if (ev < 0)
                        __hip_atomic_fetch_or(a.status, (uint32_t)VQ2_MOE_WAIT_ID, __ATOMIC_RELAXED,
                                              __HIP_MEMORY_SCOPE_AGENT);
                } else {
                    ev = a.ids_i64 ? ((const int64_t*)a.ids)[p] : (int64_t)((const int32_t*)a.ids)[p];
                    wv = a.w[p];
                }
                s_e = (ev >= 0 && ev < a.n_experts) ? (int32_t)ev : -1;
                s_w = wv;
            }
            __syncthreads();
        }
        auto slice_loads = [&](int64_t i, int s0, float (&pv)[8]) {
#pragma unroll
            for (int s = 0; s < 8; s++) {
                const float* q = gp + (s0 + s < a.gu_slices ? s0 + s : 0) * gstride + i;
                pv[s] = FUSED ? share_load(q) : *q;
            }
        };
        auto finish = [&](int64_t i, const float (&pv)[8], float sc) {
            float v = 0.0f;
#pragma unroll
            for (int s = 0; s < 8; s++)
                if (s < a.gu_slices) v += pv[s];
            for (int s0 = 8; s0 < a.gu_slices; s0 += 8) {
                float pw[8];
                slice_loads(i, s0, pw);
#pragma unroll
                for (int s = 0; s < 8; s++)
                    if (s0 + s < a.gu_slices) v += pw[s];
            }
            smem[i] = v * sc;  // gate values land in s_x, up values in s_stage (= smem + n)
        };
        const int64_t i0 = threadIdx.x < 2 * n ? threadIdx.x : 0;
        float pv0[8];
        if constexpr (!FUSED) {
            slice_loads(i0, 0, pv0);  // needs only the pair, not its expert
            asm volatile("" ::: "memory");
            e = pair_expert(a, p, bad);
        } else {
            bad = s_e < 0;
            e = bad ? 0 : s_e;
        }
        const uint32_t sc0 = load_raw(a.gu_scale, a.gu_s_dt, e * a.gu_rows + i0);
        // the epilogue's combine weight and row scale, fetched now; both
        // scale loads sit in dtype branches, ahead of the entry words so
        // that the waits for them stay exact
        wp = FUSED ? s_w : uniform_load<float>(a.w, p);
        const bool own_e = (int)threadIdx.x < pl.rb + (chunk < pl.nbig ? 1 : 0);
        const int64_t row_e = (int64_t)chunk * pl.rb + min(chunk, pl.nbig) + (own_e ? threadIdx.x : 0);
        dsc = load_raw(pl.scale, pl.s_dt, e * pl.rows + row_e);
        entries(e);
        if constexpr (FUSED) {
            // the entry words come while the pair's gate_up workgroups
            // finish; then their row sums (a bounded poll of the count)
            if (threadIdx.x == 0) {
                bool ok = false;
                for (int it = 0; it < a.max_polls; it++) {
                    if (__hip_atomic_load(a.pair_cnt + p * MOE_CNT_STRIDE, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) >=
                        (uint32_t)a.gu_arrivals) {
                        ok = true;
                        break;
                    }
                    __builtin_amdgcn_s_sleep(10);
                }
                if (!ok)
                    __hip_atomic_fetch_or(a.status, (uint32_t)VQ2_MOE_WAIT_COUNT, __ATOMIC_RELAXED,
                                          __HIP_MEMORY_SCOPE_AGENT);
                s_ok = ok ? 1 : 0;
            }
            __syncthreads();
            bad = bad || s_ok == 0;
            slice_loads(i0, 0, pv0);
        }
        sorted_acc_zero(acc, lane, R);
        if (threadIdx.x < 2 * n) finish(threadIdx.x, pv0, raw_as_f32(sc0, a.gu_s_dt));
        for (int64_t i = threadIdx.x + SG_THREADS; i < 2 * n; i += SG_THREADS) {
            float pv[8];
            slice_loads(i, 0, pv);
            finish(i, pv, load_as_f32(a.gu_scale, a.gu_s_dt, e * a.gu_rows + i));
        }
        __syncthreads();
        if constexpr (F2K != 0) {
            // silu(gate) * up taken as the transform reads it; its natural-
            // order scratch follows the split activation
            rht512_transform(first512, [&](uint32_t i) { return silu_f32(s_x[i]) * s_stage[i]; }, s_split + n,
                             s_split, a.g.xscale, xb);
        } else {
            for (int64_t j = threadIdx.x; j < n; j += SG_THREADS) s_stage[j] = silu_f32(s_x[j]) * s_stage[j];
            __syncthreads();
            build_x<2, VQ2_DT_F32>(a.g, s_x, s_stage, 1, n, first);
        }
    }
    if constexpr (F2K == 0) x_finalize(s_x, s_split, n, a.g.xscale, xb);
    __syncthreads();
    pipe.gathers();
    pipe.run(acc, s_split, pl.gbits, pl.ng, R, xb);
    __syncthreads();

    const int rr = threadIdx.x;
    const int64_t row = (int64_t)chunk * pl.rb + min(chunk, pl.nbig) + rr;
    const bool own = rr < pl.rb + (chunk < pl.nbig ? 1 : 0);
    // MODE 2: each slice's share of the combine, w[p] * (sum * s[e][row])
    float f = 1.0f;
    if constexpr (MODE == 2) f = own ? wp * raw_as_f32(dsc, pl.s_dt) : 0.0f;
    // chunks of 256 rows or more (taller down pools) sum rows in 512-thread halves
    const float sum = sorted_row_sums<true>(s_acc, R, s_red);
    if (own) {
        float v = sum;
        if constexpr (MODE == 2) v = f * sum;
        // gate_up: [slice][pair][row]; down: [pair][slice][row] (the combine reads a token's shares in one run)
        const int64_t pi = MODE == 2 ? (int64_t)p * a.slices + slice : (int64_t)slice * a.n_pairs + p;
        const float o = bad ? __builtin_nanf("") : v;
        if (FUSED && MODE != 2) share_store(a.part + pi * pl.rows + row, o);
        else a.part[pi * pl.rows + row] = o;
    }
    if constexpr (FUSED && MODE != 2) {
        // the row sums (and the router's ids and weights) are complete at
        // the coherence point before the pair's count moves
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        __syncthreads();
        if (threadIdx.x == 0) __hip_atomic_fetch_add(a.pair_cnt + p * MOE_CNT_STRIDE, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
}

template <int CBT, int MODE, int XT, int F2K>
__global__ void __launch_bounds__(SG_THREADS) vq_sorted_moe_kernel(const SortedMoeArgs a)
{
    extern __shared__ __align__(16) float smem[];
    touch_kernargs(a);
    moe_body<CBT, MODE, XT, F2K, 0>(a, (int)blockIdx.x, smem);
}

// gate_up (MODE GU, hidden 2048) and down (intermediate 512) in one launch:
// the first ceil8(a.wgs) workgroups run gate_up (a multiple of 8, so a down
// workgroup's XCD is its own index mod 8), the rest down.  Workgroups are
// dispatched in index order and a gate_up workgroup waits for nothing, so
// every gate_up workgroup a down workgroup waits for is running or done.
// Two workgroups per CU (64 VGPRs, ~76 KiB of LDS each): down workgroups
// then start beside running gate_up ones, issue their loads and wait there,
// instead of starting only when a gate_up workgroup leaves its CU (stamps:
// at T = 1 the down workgroups started ~11.5 us into the launch, when the
// gate_up ones ended).  Measured with the one-ahead pipelines: T = 1
// 20.1 -> 19.8-20.0 us, T = 8 70.7 -> 66.8 us (64.5 with two gate_up
// slices); with the gate_up part's two-ahead pipeline the 64-VGPR bound
// spilled and T = 1 took 20.7 us.  bf16 codebooks (whose centroid
// conversion needs more registers: 9-12 spilled at 64) keep one workgroup
// per CU and the two-ahead gate_up pipeline.
template <int CBT, int GU, int XT>
__global__ void __launch_bounds__(SG_THREADS, CBT == VQ2_DT_F16 ? 8 : 1) vq_sorted_moe_fused_kernel(const SortedMoeArgs a, const SortedMoeArgs d)
{
    extern __shared__ __align__(16) float smem[];
    const int gu_blocks = (a.wgs + 7) & ~7;
    if ((int)blockIdx.x < gu_blocks) {
        touch_kernargs(a);
        moe_body<CBT, GU, XT, 1, 1>(a, (int)blockIdx.x, smem);
    } else {
        touch_kernargs(d);
        moe_body<CBT, 2, VQ2_DT_F32, 1, 1>(d, (int)blockIdx.x - gu_blocks, smem);
    }
}

// out[t][row] = the sum of the token's down shares
// part[pair][slice][row] = w[pair] * ((down row sum of the slice) * s[e][row])
// over its pairs and slices, which are consecutive blocks of rows values.
// Four threads per row: thread `part` adds shares part, part + 4, ... (all
// its loads in flight together: each is a memory round trip, the shares
// were written by other XCDs), then a fixed DPP tree adds the four partial
// sums (deterministic).  grid (ceil(rows / 64), tokens).
__global__ void __launch_bounds__(256) vq_sorted_moe_combine_kernel(const SortedMoeArgs a)
{
    // the fused launch's per-pair counts go back to 0 for the next layer
    if (a.pair_cnt && blockIdx.x == 0 && blockIdx.y == 0)
        for (int i = threadIdx.x; i < a.n_pairs; i += 256) {
            a.pair_cnt[i * MOE_CNT_STRIDE] = 0u;
            *pair_word(a, i) = 0ull;
        }
    const int t = blockIdx.y;
    const int rows = a.pool.rows;
    const int part = threadIdx.x & 3;
    const int64_t row0 = (int64_t)blockIdx.x * 64 + (threadIdx.x >> 2);
    const int64_t row = row0 < rows ? row0 : rows - 1;  // every lane takes part in the DPP sums
    const float* base = a.part + (int64_t)t * a.P * a.slices * rows + row;
    const int terms = a.P * a.slices;
    float fin = 0.0f;
    for (int j0 = part; j0 < terms; j0 += 32) {
        float v[8];
#pragma unroll
        for (int j = 0; j < 8; j++) v[j] = base[(int64_t)(j0 + 4 * j < terms ? j0 + 4 * j : 0) * rows];
#pragma unroll
        for (int j = 0; j < 8; j++)
            if (j0 + 4 * j < terms) fin += v[j];
    }
    fin += __int_as_float(dpp_mov<0xB1>(__float_as_int(fin)));  // quad_perm [1,0,3,2]
    fin += __int_as_float(dpp_mov<0x4E>(__float_as_int(fin)));  // quad_perm [2,3,0,1]
    if (part == 0 && row0 < rows) store_from_f32(a.out, a.out_dt, (int64_t)t * rows + row0, fin);
}

// ------------------------------------------------------------------ launch
template <int CBT, int MODE, int XT, int F2K>
static hipError_t launch_moe(const SortedMoeArgs& a, unsigned grid, size_t shm, hipStream_t st)
{
    static std::once_flag once;
    static hipError_t attr = hipSuccess;
    std::call_once(once, [] {
        attr = hipFuncSetAttribute((const void*)vq_sorted_moe_kernel<CBT, MODE, XT, F2K>,
                                   hipFuncAttributeMaxDynamicSharedMemorySize, SG_MAX_SHM);
    });
    if (attr != hipSuccess) return attr;
    hipLaunchKernelGGL((vq_sorted_moe_kernel<CBT, MODE, XT, F2K>), dim3(grid), dim3(SG_THREADS), shm, st, a);
    return hipGetLastError();
}

template <int MODE, int XT, int F2K>
static hipError_t launch_moe_cb(int cb_dt, const SortedMoeArgs& a, unsigned grid, size_t shm, hipStream_t st)
{
    return cb_dt == VQ2_DT_F16 ? launch_moe<VQ2_DT_F16, MODE, XT, F2K>(a, grid, shm, st)
                               : launch_moe<VQ2_DT_BF16, MODE, XT, F2K>(a, grid, shm, st);
}

template <int MODE>
static hipError_t launch_moe_x(int cb_dt, int x_dt, bool f2k, const SortedMoeArgs& a, unsigned grid, size_t shm,
                               hipStream_t st)
{
    if (f2k) {
        switch (x_dt) {
        case VQ2_DT_F16: return launch_moe_cb<MODE, VQ2_DT_F16, 1>(cb_dt, a, grid, shm, st);
        case VQ2_DT_BF16: return launch_moe_cb<MODE, VQ2_DT_BF16, 1>(cb_dt, a, grid, shm, st);
        default: return launch_moe_cb<MODE, VQ2_DT_F32, 1>(cb_dt, a, grid, shm, st);
        }
    }
    switch (x_dt) {
    case VQ2_DT_F16: return launch_moe_cb<MODE, VQ2_DT_F16, 0>(cb_dt, a, grid, shm, st);
    case VQ2_DT_BF16: return launch_moe_cb<MODE, VQ2_DT_BF16, 0>(cb_dt, a, grid, shm, st);
    default: return launch_moe_cb<MODE, VQ2_DT_F32, 0>(cb_dt, a, grid, shm, st);
    }
}

template <int CBT, int GU, int XT>
static hipError_t launch_fused_t(const SortedMoeArgs& a, const SortedMoeArgs& d, unsigned grid, size_t shm, hipStream_t st)
{
    static std::once_flag once;
    static hipError_t attr = hipSuccess;
    std::call_once(once, [] {
        attr = hipFuncSetAttribute((const void*)vq_sorted_moe_fused_kernel<CBT, GU, XT>,
                                   hipFuncAttributeMaxDynamicSharedMemorySize, SG_MAX_SHM);
    });
    if (attr != hipSuccess) return attr;
    hipLaunchKernelGGL((vq_sorted_moe_fused_kernel<CBT, GU, XT>), dim3(grid), dim3(SG_THREADS), shm, st, a, d);
    return hipGetLastError();
}

template <int GU>
static hipError_t launch_fused(int cb_dt, int x_dt, const SortedMoeArgs& a, const SortedMoeArgs& d, unsigned grid,
                               size_t shm, hipStream_t st)
{
    if (cb_dt == VQ2_DT_F16) {
        switch (x_dt) {
        case VQ2_DT_F16: return launch_fused_t<VQ2_DT_F16, GU, VQ2_DT_F16>(a, d, grid, shm, st);
        case VQ2_DT_BF16: return launch_fused_t<VQ2_DT_F16, GU, VQ2_DT_BF16>(a, d, grid, shm, st);
        default: return launch_fused_t<VQ2_DT_F16, GU, VQ2_DT_F32>(a, d, grid, shm, st);
        }
    }
    switch (x_dt) {
    case VQ2_DT_F16: return launch_fused_t<VQ2_DT_BF16, GU, VQ2_DT_F16>(a, d, grid, shm, st);
    case VQ2_DT_BF16: return launch_fused_t<VQ2_DT_BF16, GU, VQ2_DT_BF16>(a, d, grid, shm, st);
    default: return launch_fused_t<VQ2_DT_BF16, GU, VQ2_DT_F32>(a, d, grid, shm, st);
    }
}

static int pool_args(const SortedPoolCall& pc, const char* name, int64_t n_experts, int64_t rows, int64_t ng,
                     SortedPoolArgs& pa)
{
    // pools: 16-bit positions (chunks of up to 511 rows where they fit)
    const int64_t r_lim = sorted_max_rows(ng, 16);
    if (r_lim == 0) return set_error(VQ2_ERR_UNSUPPORTED, "vq2_sorted_moe: %s: ng=%lld unsupported", name, (long long)ng);
    if (pc.rows != rows || pc.ng != ng)
        return set_error(VQ2_ERR_ARG, "vq2_sorted_moe: %s pool holds [%lld rows, %lld groups], expected [%lld, %lld]",
                         name, (long long)pc.rows, (long long)pc.ng, (long long)rows, (long long)ng);
    if (pc.rows_per_chunk < 1 || pc.rows_per_chunk > r_lim)
        return set_error(VQ2_ERR_ARG, "vq2_sorted_moe: %s: rows_per_chunk=%lld outside 1..%lld", name,
                         (long long)pc.rows_per_chunk, (long long)r_lim);
    const ChunkSplit ks = chunk_split(rows, pc.rows_per_chunk);
    const int64_t C = ks.n_chunks;
    if (pc.iters_per_chunk < 1 || n_experts * C * pc.iters_per_chunk != pc.n_iters || pc.n_iters > 0x7FFFFFFF)
        return set_error(VQ2_ERR_ARG, "vq2_sorted_moe: %s pool: %lld iterations are not %lld experts x %lld chunks x "
                         "%lld", name, (long long)pc.n_iters, (long long)n_experts, (long long)C,
                         (long long)pc.iters_per_chunk);
    if (!pc.entries || (uintptr_t)pc.entries % 16 || !pc.scale)
        return set_error(VQ2_ERR_ARG, "vq2_sorted_moe: %s pool: entries (16-byte aligned) and scales are required",
                         name);
    if (!dt_ok(pc.scale_dt)) return set_error(VQ2_ERR_ARG, "vq2_sorted_moe: %s: bad scale dtype", name);
    if (pc.s2 < 0 || pc.s2 > 2 || pc.stage1_iters < 1 || pc.stage1_iters > pc.iters_per_chunk ||
        (pc.s2 == 0 && pc.stage1_iters != pc.iters_per_chunk))
        return set_error(VQ2_ERR_ARG, "vq2_sorted_moe: %s pool: %lld stage-1 iterations of %lld (stage-2 kind %d)",
                         name, (long long)pc.stage1_iters, (long long)pc.iters_per_chunk, pc.s2);
    if (pc.s2 && (!pc.cb1 || (uintptr_t)pc.cb1 % 16))
        return set_error(VQ2_ERR_ARG, "vq2_sorted_moe: %s pool: a stage-2 pool needs its codebook (16-byte aligned)",
                         name);
    pa.ent = pc.entries;
    pa.cb1 = pc.s2 ? pc.cb1 : nullptr;
    pa.c1mask = pc.s2 == 2 ? 0xFFu : 0xFFFFu;
    pa.ipc1 = (int32_t)pc.stage1_iters;
    pa.ipc = (int32_t)pc.iters_per_chunk;
    pa.scale = pc.scale;
    pa.s_dt = pc.scale_dt;
    pa.n_iters = (int32_t)pc.n_iters;
    pa.R = (int)pc.rows_per_chunk;
    pa.C = (int)C;
    pa.rb = (int)ks.rb;
    pa.nbig = (int)ks.nbig;
    pa.rows = (int)rows;
    pa.ng = (int)ng;
    pa.gbits = sorted_gbits(ng);
    return VQ2_OK;
}

// Bound of the one-launch waits and an arrival target offset (a test of the
// give-up path passes a target the gate_up part cannot reach); process-wide.
static std::atomic<int64_t> g_wait_polls{int64_t(1) << 20};
static std::atomic<int32_t> g_wait_extra{0};
MoeWait sorted_moe_wait()
{
    return MoeWait{(int)g_wait_polls.load(), (int)g_wait_extra.load()};
}
int sorted_moe_set_wait(int64_t max_polls, int32_t extra_arrivals)
{
    if (max_polls < 0 || max_polls > 0x7FFFFFFF || extra_arrivals < 0 || extra_arrivals > 1024)
        return set_error(VQ2_ERR_ARG, "vq2_sorted_moe_set_wait: max_polls 0..2^31-1, extra_arrivals 0..1024");
    g_wait_polls.store(max_polls);
    g_wait_extra.store(extra_arrivals);
    return VQ2_OK;
}

// Workspace: VQ2_SORTED_WS_HEADER bytes of per-pair counters (the fused
// launch; zero between calls), then the gate_up row sums and the down
// shares.
size_t sorted_moe_workspace_bytes(int64_t n_pairs, int64_t hidden, int64_t inter, int slices_gu, int slices_dn)
{
    return VQ2_SORTED_WS_HEADER +
           ((size_t)slices_gu * n_pairs * 2 * inter + (size_t)slices_dn * n_pairs * hidden) * sizeof(float);
}

static int rot_fields(GemvArgs& g, const SortedRot& r, int64_t n, const char* name)
{
    if (r.hb < 2 || r.hb > n || (r.hb & (r.hb - 1)) || n % r.hb)
        return set_error(VQ2_ERR_ARG, "vq2_sorted_moe: %s: hb=%lld must be a power of two dividing %lld", name,
                         (long long)r.hb, (long long)n);
    if ((uintptr_t)r.perm % 16 || (uintptr_t)r.sign % 8)
        return set_error(VQ2_ERR_ARG, "vq2_sorted_moe: %s: perm 16-byte, sign 8-byte aligned", name);
    g.perm = r.perm;
    g.sign = r.sign;
    int hl = 0;
    while ((int64_t(1) << hl) < r.hb) hl++;
    g.hb_log2 = hl;
    g.xscale = r.scale;
    return VQ2_OK;
}

int sorted_moe_launch(const SortedMoeCall& c)
{
    const int64_t H = c.hidden, I = c.inter, T = c.tokens;
    const bool router = c.logits != nullptr;
    if (T < 1 || c.P < 1) return set_error(VQ2_ERR_ARG, "vq2_sorted_moe: tokens and pairs per token must be >= 1");
    if (H % 64 || I % 64 || H < 64 || I < 64 || H > 8192 || I > 8192)
        return set_error(VQ2_ERR_UNSUPPORTED, "vq2_sorted_moe: hidden=%lld / inter=%lld must be multiples of 64 up to "
                         "8192", (long long)H, (long long)I);
    if (c.cb_dt != VQ2_DT_F16 && c.cb_dt != VQ2_DT_BF16)
        return set_error(VQ2_ERR_UNSUPPORTED, "vq2_sorted_moe: fp16 / bf16 codebooks only");
    if (!c.cb || (uintptr_t)c.cb % 16) return set_error(VQ2_ERR_ARG, "vq2_sorted_moe: codebook must be 16-byte aligned");
    if (!dt_ok(c.h_dt) || !dt_ok(c.out_dt)) return set_error(VQ2_ERR_ARG, "vq2_sorted_moe: bad h / out dtype");
    if (!c.h || (uintptr_t)c.h % 16 || !c.out) return set_error(VQ2_ERR_ARG, "vq2_sorted_moe: h (16-byte aligned) and out required");
    if (c.slices_gu < 1 || c.slices_gu > 64 || c.slices_dn < 1 || c.slices_dn > 64)
        return set_error(VQ2_ERR_ARG, "vq2_sorted_moe: slices must be 1..64");
    if (c.n_experts < 1) return set_error(VQ2_ERR_ARG, "vq2_sorted_moe: empty pool");
    const int64_t n_pairs = T * c.P;
    if (n_pairs > 1 << 20) return set_error(VQ2_ERR_UNSUPPORTED, "vq2_sorted_moe: too many pairs");
    if (router) {
        if (c.top_k < 1 || c.top_k > SG_MAX_TOPK || c.P != c.top_k + 1 || c.n_routed < c.top_k || c.n_routed > 256)
            return set_error(VQ2_ERR_ARG, "vq2_sorted_moe: router needs 1 <= top_k <= n_routed <= 256 and pairs per "
                             "token = top_k + 1 (the shared expert last)");
        if (c.shared_id < 0 || c.shared_id >= c.n_experts || c.n_routed > c.n_experts)
            return set_error(VQ2_ERR_ARG, "vq2_sorted_moe: shared expert / routed experts outside the pool");
        if (!c.shared_gate || !c.ids_out || !c.w_out || !dt_ok(c.l_dt) || !dt_ok(c.g_dt))
            return set_error(VQ2_ERR_ARG, "vq2_sorted_moe: router needs shared_gate, ids_out and w_out");
    } else if (!c.ids || !c.w) {
        return set_error(VQ2_ERR_ARG, "vq2_sorted_moe: ids and w are required without router logits");
    }
    SortedMoeArgs a{};
    int r = pool_args(c.gate_up, "gate_up", c.n_experts, 2 * I, H / 8, a.pool);
    if (r) return r;
    SortedMoeArgs d{};
    r = pool_args(c.down, "down", c.n_experts, H, I / 8, d.pool);
    if (r) return r;
    const size_t need = sorted_moe_workspace_bytes(n_pairs, H, I, c.slices_gu, c.slices_dn);
    if (!c.workspace || c.ws_bytes < need || (uintptr_t)c.workspace % 16)
        return set_error(VQ2_ERR_ARG, "vq2_sorted_moe: workspace of %zu bytes (16-byte aligned) needed, got %zu", need,
                         c.ws_bytes);
    uint32_t* pair_cnt = (uint32_t*)c.workspace;
    float* gu_part = (float*)((char*)c.workspace + VQ2_SORTED_WS_HEADER);
    float* dn_part = gu_part + (size_t)c.slices_gu * n_pairs * 2 * I;
    const void* ids = router ? (const void*)c.ids_out : c.ids;
    const int ids_i64 = router ? 0 : c.ids_i64;
    const float* w = router ? c.w_out : c.w;

    // gate_up
    a.g.x = c.h;
    a.g.x_dt = c.h_dt;
    a.g.x_bstride = H;
    a.g.x_pstride = H;
    a.g.x_pdiv = 1;
    a.g.P = 1;
    a.g.ng = H / 8;
    a.g.batch = 1;
    if ((r = rot_fields(a.g, c.rot_h, H, "rot_h"))) return r;
    if (router) {
        a.g.r_logits = c.logits;
        a.g.r_ldt = c.l_dt;
        a.g.r_ne = c.n_routed;
        a.g.r_k = c.top_k;
        a.g.r_pairs = c.P;
        a.g.r_shared = c.shared_id;
        a.g.r_gate = c.shared_gate;
        a.g.r_gdt = c.g_dt;
        a.g.r_ids = c.ids_out;
        a.g.r_w = c.w_out;
    }
    a.cb = c.cb;
    a.n_experts = c.n_experts;
    a.P = c.P;
    a.n_pairs = (int)n_pairs;
    a.slices = c.slices_gu;
    a.ids = ids;
    a.ids_i64 = ids_i64;
    a.part = gu_part;
    hipStream_t st = (hipStream_t)c.stream;
    const int64_t grid_gu = n_pairs * a.pool.C * c.slices_gu;
    const int64_t grid_dn = n_pairs * d.pool.C * c.slices_dn;
    if (grid_gu > 0x7FFFFFFF / 2 || grid_dn > 0x7FFFFFFF / 2)
        return set_error(VQ2_ERR_UNSUPPORTED, "vq2_sorted_moe: grid too large");
    a.wgs = (int)grid_gu;
    a.sq = a.pool.ipc / a.slices;
    a.sr = a.pool.ipc % a.slices;
    a.xmap = a.slices > 1 && grid_gu <= device_cu_count();
    a.xq = (int)(grid_gu / 8);
    a.xr = (int)(grid_gu % 8);
    // 2048-point blocks: the all-threads prologue
    const bool f2k = c.rot_h.hb == RHT2K && H == RHT2K;
    const size_t shm_gu =
        (size_t)(H + moe_split_floats(1, f2k, H) + SG_WAVES * SG_PARTS * (a.pool.R + 1)) * sizeof(float);
    if (shm_gu > SG_MAX_SHM)
        return set_error(VQ2_ERR_UNSUPPORTED, "vq2_sorted_moe: gate_up needs %zu bytes of LDS", shm_gu);

    // down: SwiGLU + RHT_I prologue from the gate_up slices
    d.g.ng = I / 8;
    d.g.batch = 1;
    d.g.P = 1;
    d.g.x_pdiv = 1;
    if ((r = rot_fields(d.g, c.rot_i, I, "rot_i"))) return r;
    d.cb = c.cb;
    d.n_experts = c.n_experts;
    d.P = c.P;
    d.n_pairs = (int)n_pairs;
    d.slices = c.slices_dn;
    d.wgs = (int)grid_dn;
    d.sq = d.pool.ipc / d.slices;
    d.sr = d.pool.ipc % d.slices;
    d.xmap = d.slices > 1 && grid_dn <= device_cu_count();
    d.xq = (int)(grid_dn / 8);
    d.xr = (int)(grid_dn % 8);
    d.ids = ids;
    d.ids_i64 = ids_i64;
    d.part = dn_part;
    d.gu_part = gu_part;
    d.gu_slices = c.slices_gu;
    d.gu_rows = (int)(2 * I);
    d.gu_scale = c.gate_up.scale;
    d.gu_s_dt = c.gate_up.scale_dt;
    d.w = w;
    // one 512-point rotation block: the all-threads prologue
    const bool f512 = c.rot_i.hb == RHT512 && I == RHT512;
    const size_t shm_dn =
        (size_t)(I + moe_split_floats(2, f512, I) + SG_WAVES * SG_PARTS * (d.pool.R + 1)) * sizeof(float);
    if (shm_dn > SG_MAX_SHM) return set_error(VQ2_ERR_UNSUPPORTED, "vq2_sorted_moe: down needs %zu bytes of LDS", shm_dn);

    hipError_t err;
    if (f2k && f512 && n_pairs <= VQ2_SORTED_MAX_COUNTERS / MOE_CNT_STRIDE) {
        static_assert(VQ2_SORTED_MAX_COUNTERS * 4 <= VQ2_SORTED_WS_STATUS, "counts below the status word");
        // gate_up and down in one launch, the down workgroups waiting for
        // their pair's gate_up workgroups (counts in the workspace header)
        a.pair_cnt = d.pair_cnt = pair_cnt;
        const MoeWait wt = sorted_moe_wait();
        d.gu_arrivals = (int)(a.pool.C * c.slices_gu) + wt.extra_arrivals;
        d.id_poll = router ? 1 : 0;
        d.max_polls = wt.max_polls;
        d.status = (uint32_t*)((char*)c.workspace + VQ2_SORTED_WS_STATUS);
        const unsigned grid = (unsigned)((grid_gu + 7) / 8 * 8 + grid_dn);
        err = router ? launch_fused<1>(c.cb_dt, c.h_dt, a, d, grid, std::max(shm_gu, shm_dn), st)
                     : launch_fused<0>(c.cb_dt, c.h_dt, a, d, grid, std::max(shm_gu, shm_dn), st);
        if (err != hipSuccess) return set_hip_error(err, "vq2_sorted_moe gate_up + down launch");
    } else {
        err = router ? launch_moe_x<1>(c.cb_dt, c.h_dt, f2k, a, (unsigned)grid_gu, shm_gu, st)
                     : launch_moe_x<0>(c.cb_dt, c.h_dt, f2k, a, (unsigned)grid_gu, shm_gu, st);
        if (err != hipSuccess) return set_hip_error(err, "vq2_sorted_moe gate_up launch");
        if (f512)
            err = c.cb_dt == VQ2_DT_F16 ? launch_moe<VQ2_DT_F16, 2, VQ2_DT_F32, 1>(d, (unsigned)grid_dn, shm_dn, st)
                                        : launch_moe<VQ2_DT_BF16, 2, VQ2_DT_F32, 1>(d, (unsigned)grid_dn, shm_dn, st);
        else
            err = c.cb_dt == VQ2_DT_F16 ? launch_moe<VQ2_DT_F16, 2, VQ2_DT_F32, 0>(d, (unsigned)grid_dn, shm_dn, st)
                                        : launch_moe<VQ2_DT_BF16, 2, VQ2_DT_F32, 0>(d, (unsigned)grid_dn, shm_dn, st);
        if (err != hipSuccess) return set_hip_error(err, "vq2_sorted_moe down launch");
    }

    // combine
    d.out = c.out;
    d.out_dt = c.out_dt;
    hipLaunchKernelGGL(vq_sorted_moe_combine_kernel, dim3((unsigned)((H + 63) / 64), (unsigned)T), dim3(256), 0, st, d);
    err = hipGetLastError();
    if (err != hipSuccess) return set_hip_error(err, "vq2_sorted_moe combine launch");
    return VQ2_OK;
}

}  // namespace vq2
