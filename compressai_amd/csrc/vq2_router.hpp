// vq2_router.hpp -- MoE router math shared by the standalone router kernel
// and the router prologue of the fused gate_up launch.
//
// transformers 5.15.0 Qwen3_5MoeTopKRouter.forward (HF:760-776): softmax
// over the routed experts in fp32, top-k (ties: lowest expert id), the k
// probabilities renormalised to sum 1; the shared expert
// (Qwen3_5MoeSparseMoeBlock, HF:787-798) gets sigmoid(shared_gate . h_t).
#pragma once

#include "vq2_common.hpp"

namespace vq2 {

constexpr int ROUTER_MAX_E = 1024;

template <int DT>
__device__ __forceinline__ float ld_t(const void* p, int64_t i)
{
    if constexpr (DT == VQ2_DT_F32) return ((const float*)p)[i];
    else if constexpr (DT == VQ2_DT_F16) return f16_bits_to_f32(((const uint16_t*)p)[i]);
    else return bf16_bits_to_f32(((const uint16_t*)p)[i]);
}

template <int LT, int RPL>
__device__ __forceinline__ void router_load_logits(const void* logits, int64_t t, int64_t n_e, int lane,
                                                   float (&p)[RPL])
{
#pragma unroll
    for (int j = 0; j < RPL; j++) {
        const int e = j * 64 + lane;
        p[j] = ld_t<LT>(logits, t * n_e + (e < n_e ? e : 0));
    }
#pragma unroll
    for (int j = 0; j < RPL; j++)
        if (j * 64 + lane >= n_e) p[j] = -INFINITY;
}

// gate . h_t: 16 gate and 16 h loads in flight per lane per chunk
template <int GT, int HT>
__device__ __forceinline__ float router_gate_dot(const void* gate, const void* h, int64_t t, int64_t hidden, int lane)
{
    float d = 0.0f;
    for (int64_t i0 = 0; i0 < hidden; i0 += 16 * 64) {
        float g[16], x[16];
#pragma unroll
        for (int u = 0; u < 16; u++) {
            const int64_t i = i0 + u * 64 + lane;
            const int64_t ic = i < hidden ? i : 0;
            g[u] = ld_t<GT>(gate, ic);
            x[u] = ld_t<HT>(h, t * hidden + ic);
        }
#pragma unroll
        for (int u = 0; u < 16; u++)
            if (i0 + u * 64 + lane < hidden) d = fmaf(g[u], x[u], d);
    }
    return d;
}

// sigmoid(gate . h_t), uniform over the wave
__device__ __forceinline__ float router_shared_weight(const void* gate, int g_dt, const void* h, int h_dt, int64_t t,
                                                      int64_t hidden, int lane)
{
    float d;
    if (g_dt == VQ2_DT_F16 && h_dt == VQ2_DT_F16) d = router_gate_dot<VQ2_DT_F16, VQ2_DT_F16>(gate, h, t, hidden, lane);
    else if (g_dt == VQ2_DT_BF16 && h_dt == VQ2_DT_BF16) d = router_gate_dot<VQ2_DT_BF16, VQ2_DT_BF16>(gate, h, t, hidden, lane);
    else if (g_dt == VQ2_DT_F32 && h_dt == VQ2_DT_F32) d = router_gate_dot<VQ2_DT_F32, VQ2_DT_F32>(gate, h, t, hidden, lane);
    else {
        d = 0.0f;
        for (int64_t i = lane; i < hidden; i += 64) d = fmaf(load_as_f32(gate, g_dt, i), load_as_f32(h, h_dt, t * hidden + i), d);
    }
    const float dd = wave_sum_all(d);
    return 1.0f / (1.0f + __expf(-dd));
}

// Routing probabilities of token t by one full wave (RPL * 64 >= n_e): p[j]
// of expert j * 64 + lane is softmax(logits)[e] in fp32, -1 past n_e.
template <int RPL>
__device__ __forceinline__ void router_probs(const void* logits, int l_dt, int64_t t, int64_t n_e, int lane,
                                             float (&p)[RPL])
{
    if (l_dt == VQ2_DT_F16)
        router_load_logits<VQ2_DT_F16, RPL>(logits, t, n_e, lane, p);
    else if (l_dt == VQ2_DT_BF16)
        router_load_logits<VQ2_DT_BF16, RPL>(logits, t, n_e, lane, p);
    else
        router_load_logits<VQ2_DT_F32, RPL>(logits, t, n_e, lane, p);

    float m = -INFINITY;
#pragma unroll
    for (int j = 0; j < RPL; j++) m = fmaxf(m, p[j]);
    m = wave_max_all(m);
    float sum = 0.0f;
#pragma unroll
    for (int j = 0; j < RPL; j++) {
        p[j] = (j * 64 + lane) < n_e ? __expf(p[j] - m) : 0.0f;
        sum += p[j];
    }
    sum = wave_sum_all(sum);
#pragma unroll
    for (int j = 0; j < RPL; j++) p[j] = (j * 64 + lane) < n_e ? p[j] / sum : -1.0f;
}

// Top-k of token t by one full wave (RPL * 64 >= n_e): lane r < k ends with
// the round-r choice (probability `mine`, expert `my_id`); `tot` (uniform) is
// the sum of the k chosen probabilities, so weight r = mine / tot.
template <int RPL>
__device__ __forceinline__ void router_select(const void* logits, int l_dt, int64_t t, int64_t n_e, int k, int lane,
                                              float& mine, int& my_id, float& tot)
{
    float p[RPL];
    router_probs<RPL>(logits, l_dt, t, n_e, lane, p);

    mine = 0.0f;
    my_id = 0;
    for (int r = 0; r < k; r++) {
        float bv = -1.0f;
        int bi = 0x7FFFFFFF;
#pragma unroll
        for (int j = 0; j < RPL; j++) {
            const int e = j * 64 + lane;
            if (p[j] > bv || (p[j] == bv && e < bi)) { bv = p[j]; bi = e; }
        }
        wave_argmax_all(bv, bi);
#pragma unroll
        for (int j = 0; j < RPL; j++)
            if (j * 64 + lane == bi) p[j] = -2.0f;  // never selected again
        if (lane == r) { mine = bv; my_id = bi; }
    }
    tot = wave_sum_all(lane < k ? mine : 0.0f);
}

}  // namespace vq2
