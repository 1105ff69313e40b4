// vq2_misc.hip -- small kernels of the decode path: top-1 over logits,
// top-k router with the shared-expert gate, rotated-space dequant and index
// decode (gfx950).
#include "vq2_common.hpp"
#include "vq2_router.hpp"
#include "vq2_internal.hpp"

namespace vq2 {

// ------------------------------------------------------------------ argmax
__global__ void argmax_init_kernel(uint64_t* keys, int64_t rows)
{
    const int64_t r = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (r < rows) keys[r] = 0;
}

constexpr int ARGMAX_CHUNK = 8192;

__global__ void __launch_bounds__(256) argmax_partial_kernel(const void* v, int v_dt, int64_t cols, uint64_t* keys)
{
    __shared__ uint64_t s_best[4];
    const int64_t r = blockIdx.y;
    const int64_t c0 = (int64_t)blockIdx.x * ARGMAX_CHUNK;
    const int64_t c1 = min(cols, c0 + ARGMAX_CHUNK);
    uint64_t best = 0;
    for (int64_t c = c0 + threadIdx.x; c < c1; c += blockDim.x) {
        const uint64_t k = argmax_key(load_as_f32(v, v_dt, r * cols + c), c);
        best = k > best ? k : best;
    }
    // wave reduction of the 64-bit key
    for (int off = 32; off > 0; off >>= 1) {
        const uint64_t o = __shfl_xor(best, off);
        best = o > best ? o : best;
    }
    if ((threadIdx.x & 63) == 0) s_best[threadIdx.x >> 6] = best;
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int w = 1; w < (int)(blockDim.x >> 6); w++) best = s_best[w] > best ? s_best[w] : best;
        atomicMax((unsigned long long*)&keys[r], (unsigned long long)best);
    }
}

__global__ void argmax_decode_kernel(int64_t* out_idx, float* out_val, int64_t rows)
{
    const int64_t r = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (r >= rows) return;
    const uint64_t k = ((const uint64_t*)out_idx)[r];
    const uint32_t lo = (uint32_t)(k & 0xFFFFFFFFu);
    uint32_t u = (uint32_t)(k >> 32);
    u = (u & 0x80000000u) ? (u & 0x7FFFFFFFu) : ~u;
    if (out_val) out_val[r] = __uint_as_float(u);
    out_idx[r] = (int64_t)(0xFFFFFFFFu - lo);
}

// One workgroup per batch column: the best of the per-workgroup candidate
// keys of the fused LM-head top-1, decoded as argmax_decode_kernel does.
__global__ void __launch_bounds__(256) argmax_final_kernel(const uint64_t* cand, int64_t n_cand, int64_t batch,
                                                           int64_t* out_idx, float* out_val)
{
    __shared__ uint64_t s_best[4];
    const int64_t b = blockIdx.x;
    uint64_t best = 0;
    for (int64_t g = threadIdx.x; g < n_cand; g += blockDim.x) {
        const uint64_t k = cand[g * batch + b];
        best = k > best ? k : best;
    }
    for (int off = 32; off > 0; off >>= 1) {
        const uint64_t o = __shfl_xor(best, off);
        best = o > best ? o : best;
    }
    if ((threadIdx.x & 63) == 0) s_best[threadIdx.x >> 6] = best;
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int w = 1; w < (int)(blockDim.x >> 6); w++) best = s_best[w] > best ? s_best[w] : best;
        argmax_key_decode(best, out_idx + b, out_val ? out_val + b : nullptr);
    }
}

int argmax_final_launch(const uint64_t* cand, int64_t n_cand, int64_t batch, int64_t* out_idx, float* out_val,
                        void* stream)
{
    if (batch <= 0) return VQ2_OK;
    if (batch > 65535) return set_error(VQ2_ERR_UNSUPPORTED, "vq2 argmax: batch too large");
    hipLaunchKernelGGL(argmax_final_kernel, dim3((unsigned)batch), dim3(256), 0, (hipStream_t)stream, cand, n_cand,
                       batch, out_idx, out_val);
    hipError_t err = hipGetLastError();
    if (err != hipSuccess) return set_hip_error(err, "vq2 argmax final launch");
    return VQ2_OK;
}

int argmax_launch(const void* v, int v_dt, int64_t rows, int64_t cols, int64_t* out_idx, float* out_val, void* stream)
{
    if (rows == 0) return VQ2_OK;
    if (cols <= 0 || cols > 0xFFFFFFFFLL) return set_error(VQ2_ERR_ARG, "vq2 argmax: cols=%lld out of range", (long long)cols);
    if (rows > 65535) return set_error(VQ2_ERR_UNSUPPORTED, "vq2 argmax: rows=%lld > 65535", (long long)rows);
    hipStream_t st = (hipStream_t)stream;
    uint64_t* keys = (uint64_t*)out_idx;  // the int64 output doubles as the key buffer
    hipLaunchKernelGGL(argmax_init_kernel, dim3((unsigned)((rows + 255) / 256)), dim3(256), 0, st, keys, rows);
    const int64_t nchunk = (cols + ARGMAX_CHUNK - 1) / ARGMAX_CHUNK;
    hipLaunchKernelGGL(argmax_partial_kernel, dim3((unsigned)nchunk, (unsigned)rows), dim3(256), 0, st, v, v_dt, cols,
                       keys);
    hipLaunchKernelGGL(argmax_decode_kernel, dim3((unsigned)((rows + 255) / 256)), dim3(256), 0, st, out_idx, out_val,
                       rows);
    hipError_t err = hipGetLastError();
    if (err != hipSuccess) return set_hip_error(err, "vq2 argmax launch");
    return VQ2_OK;
}

// ------------------------------------------------------------------ router
// One wave per token.  Logits live in registers (expert e = j*64 + lane),
// softmax in fp32, then k rounds of a wave-wide (max probability, lowest id)
// reduction; lane r keeps round r's probability for the renormalisation.
// The shared-expert gate dot product is loaded alongside the logits.
__global__ void __launch_bounds__(64) router_kernel(const void* logits, int l_dt, int64_t n_e, int k, const void* h,
                                                    int h_dt, int64_t hidden, const void* gate, int g_dt,
                                                    int64_t shared_id, int32_t* ids, float* w)
{
    const int64_t t = blockIdx.x;
    const int lane = threadIdx.x;
    const int row = k + (shared_id >= 0 ? 1 : 0);
    float mine, tot;
    int my_id;
    if (n_e <= 256)
        router_select<4>(logits, l_dt, t, n_e, k, lane, mine, my_id, tot);
    else
        router_select<ROUTER_MAX_E / 64>(logits, l_dt, t, n_e, k, lane, mine, my_id, tot);
    if (lane < k) {
        ids[t * row + lane] = my_id;
        w[t * row + lane] = mine / tot;
    }
    if (shared_id >= 0) {
        const float sw = router_shared_weight(gate, g_dt, h, h_dt, t, hidden, lane);
        if (lane == 0) {
            ids[t * row + k] = (int32_t)shared_id;
            w[t * row + k] = sw;
        }
    }
}

int router_launch(const void* logits, int l_dt, int64_t tokens, int64_t n_experts, int k, const void* h, int h_dt,
                  int64_t hidden, const void* gate, int g_dt, int64_t shared_id, int32_t* ids, float* w, void* stream)
{
    if (tokens == 0) return VQ2_OK;
    if (n_experts <= 0 || n_experts > ROUTER_MAX_E)
        return set_error(VQ2_ERR_UNSUPPORTED, "vq2 router: n_experts=%lld not in [1, %d]", (long long)n_experts, ROUTER_MAX_E);
    if (k <= 0 || k > 32 || k > n_experts) return set_error(VQ2_ERR_ARG, "vq2 router: k=%d out of range", k);
    if (tokens > 0x7FFFFFFF) return set_error(VQ2_ERR_UNSUPPORTED, "vq2 router: too many tokens");
    hipLaunchKernelGGL(router_kernel, dim3((unsigned)tokens), dim3(64), 0, (hipStream_t)stream, logits, l_dt,
                       n_experts, k, h, h_dt, hidden, gate, g_dt, shared_id, ids, w);
    hipError_t err = hipGetLastError();
    if (err != hipSuccess) return set_hip_error(err, "vq2 router launch");
    return VQ2_OK;
}

// ----------------------------------------------------------------- dequant
// W[r, 8g+j] = (f32(cb0[a0][j]) [+ f32(cb1[a1][j])]) * f32(s[r]); explicit
// round-to-nearest intrinsics keep the add and the multiply separate.
__global__ void dequant_kernel(const int16_t* idx0, const void* idx1, int s2, const void* cb0, const void* cb1,
                               int cb_dt, const void* scale, int s_dt, int64_t r0, int64_t rows, int64_t ng,
                               float* out)
{
    const int64_t total = rows * ng * 8;
    for (int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; t < total; t += (int64_t)gridDim.x * blockDim.x) {
        const int64_t lr = t / (ng * 8);
        const int64_t rem = t - lr * ng * 8;
        const int64_t g = rem >> 3;
        const int j = (int)(rem & 7);
        const int64_t r = r0 + lr;
        const int64_t i = r * ng + g;
        const uint32_t a0 = (uint16_t)idx0[i];
        float w = load_as_f32(cb0, cb_dt, (int64_t)a0 * 8 + j);
        if (s2 == VQ2_S2_U8) {
            const uint32_t a1 = ((const uint8_t*)idx1)[i];
            w = __fadd_rn(w, load_as_f32(cb1, cb_dt, (int64_t)a1 * 8 + j));
        } else if (s2 == VQ2_S2_U16) {
            const uint32_t a1 = (uint16_t)((const int16_t*)idx1)[i];
            w = __fadd_rn(w, load_as_f32(cb1, cb_dt, (int64_t)a1 * 8 + j));
        }
        out[t] = __fmul_rn(w, load_as_f32(scale, s_dt, r));
    }
}

int dequant_launch(const int16_t* idx0, const void* idx1, int s2, const void* cb0, const void* cb1, int cb_dt,
                   const void* scale, int s_dt, int64_t r0, int64_t r1, int64_t n, float* out, void* stream)
{
    const int64_t rows = r1 - r0;
    if (rows == 0) return VQ2_OK;
    const int64_t total = rows * n;
    int64_t blocks = (total + 255) / 256;
    if (blocks > 65536) blocks = 65536;
    hipLaunchKernelGGL(dequant_kernel, dim3((unsigned)blocks), dim3(256), 0, (hipStream_t)stream, idx0, idx1, s2, cb0,
                       cb1, cb_dt, scale, s_dt, r0, rows, n / 8, out);
    hipError_t err = hipGetLastError();
    if (err != hipSuccess) return set_hip_error(err, "vq2 dequant launch");
    return VQ2_OK;
}

// ------------------------------------------------------------------ decode
__global__ void decode_kernel(const void* in, int is_u8, int64_t count, int32_t* out)
{
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < count; i += (int64_t)gridDim.x * blockDim.x)
        out[i] = is_u8 ? (int32_t)((const uint8_t*)in)[i] : ((int32_t)((const int16_t*)in)[i] & 0xFFFF);
}

int decode_launch(const void* in, int is_u8, int64_t count, int32_t* out, void* stream)
{
    if (count == 0) return VQ2_OK;
    int64_t blocks = (count + 255) / 256;
    if (blocks > 65536) blocks = 65536;
    hipLaunchKernelGGL(decode_kernel, dim3((unsigned)blocks), dim3(256), 0, (hipStream_t)stream, in, is_u8, count, out);
    hipError_t err = hipGetLastError();
    if (err != hipSuccess) return set_hip_error(err, "vq2 decode launch");
    return VQ2_OK;
}

// ------------------------------------------------------------ unpack_fixed
// Fixed-width symbol streams (vq2/export.py:39-70: pack_fixed / unpack_fixed)
// into uint16 codes in int16 storage, the planes the GEMV reads.  The
// packings are little-endian bit streams (4-bit: low nibble first; 12-bit:
// pairs a | b << 12 in 3 bytes), so 8 symbols always fill `bits` bytes = a
// whole number of dwords: one thread turns such a unit into one 16-byte
// store.  Symbols past the last whole unit, and every symbol of a buffer that
// is not 4-byte aligned, are decoded one by one from the bytes they occupy.
template <int BITS>
__device__ __forceinline__ void unpack_unit(const uint32_t* w, uint32_t (&c)[8])
{
    if constexpr (BITS == 16) {
#pragma unroll
        for (int k = 0; k < 8; k++) c[k] = (w[k >> 1] >> (16 * (k & 1))) & 0xFFFFu;
    } else if constexpr (BITS == 8) {
#pragma unroll
        for (int k = 0; k < 8; k++) c[k] = (w[k >> 2] >> (8 * (k & 3))) & 0xFFu;
    } else if constexpr (BITS == 4) {
#pragma unroll
        for (int k = 0; k < 8; k++) c[k] = (w[0] >> (4 * k)) & 0xFu;
    } else {
        const uint64_t lo = (uint64_t)w[0] | ((uint64_t)w[1] << 32);
#pragma unroll
        for (int k = 0; k < 5; k++) c[k] = (uint32_t)(lo >> (12 * k)) & 0xFFFu;
        c[5] = (uint32_t)(lo >> 60) | ((w[2] & 0xFFu) << 4);
        c[6] = (w[2] >> 8) & 0xFFFu;
        c[7] = (w[2] >> 20) & 0xFFFu;
    }
}

__device__ __forceinline__ uint32_t unpack_one(const uint8_t* b, int bits, int64_t i)
{
    if (bits == 16) return (uint32_t)b[2 * i] | ((uint32_t)b[2 * i + 1] << 8);
    if (bits == 8) return b[i];
    if (bits == 4) return (b[i >> 1] >> (4 * (i & 1))) & 0xFu;
    const int64_t p = 3 * (i >> 1);  // 12-bit: pair i/2 at bytes 3p .. 3p+2
    if ((i & 1) == 0) return (uint32_t)b[p] | (((uint32_t)b[p + 1] & 0xFu) << 8);
    return ((uint32_t)b[p + 1] >> 4) | ((uint32_t)b[p + 2] << 4);
}

template <int BITS>
__global__ void __launch_bounds__(256) unpack_fixed_kernel(const uint8_t* buf, int64_t n, int64_t units, int16_t* out)
{
    constexpr int WORDS = BITS / 4;  // dwords per 8-symbol unit
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    for (int64_t u = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; u < units; u += stride) {
        const uint32_t* src = (const uint32_t*)buf + u * WORDS;
        uint32_t w[WORDS];
#pragma unroll
        for (int k = 0; k < WORDS; k++) w[k] = __builtin_nontemporal_load(src + k);
        uint32_t c[8];
        unpack_unit<BITS>(w, c);
        u32x4 o;
#pragma unroll
        for (int k = 0; k < 4; k++) o[k] = c[2 * k] | (c[2 * k + 1] << 16);
        __builtin_nontemporal_store(o, (u32x4*)(out + u * 8));
    }
    for (int64_t i = units * 8 + (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride)
        out[i] = (int16_t)(uint16_t)unpack_one(buf, BITS, i);
}

int unpack_fixed_launch(const uint8_t* buf, int64_t nbytes, int bits, int64_t n, int16_t* out, void* stream)
{
    if (bits != 4 && bits != 8 && bits != 12 && bits != 16)
        return set_error(VQ2_ERR_ARG, "vq2 unpack_fixed: bits=%d not in {4, 8, 12, 16}", bits);
    if (n < 0 || nbytes < 0) return set_error(VQ2_ERR_ARG, "vq2 unpack_fixed: negative size");
    const int64_t need = (n * bits + 7) / 8;
    if (nbytes < need)
        return set_error(VQ2_ERR_ARG, "vq2 unpack_fixed: %lld symbols of %d bits need %lld bytes, got %lld", (long long)n,
                         bits, (long long)need, (long long)nbytes);
    if (n == 0) return VQ2_OK;
    // whole units need a 4-byte aligned stream and a 16-byte aligned output
    const bool vec = (uintptr_t)buf % 4 == 0 && (uintptr_t)out % 16 == 0;
    const int64_t units = vec ? n / 8 : 0;
    const int64_t work = units > 0 ? units : n;
    int64_t blocks = (work + 255) / 256;
    const int64_t cap = 8LL * device_cu_count();
    if (blocks > cap) blocks = cap;
    if (blocks < 1) blocks = 1;
    hipStream_t st = (hipStream_t)stream;
    switch (bits) {
    case 4: hipLaunchKernelGGL(unpack_fixed_kernel<4>, dim3((unsigned)blocks), dim3(256), 0, st, buf, n, units, out); break;
    case 8: hipLaunchKernelGGL(unpack_fixed_kernel<8>, dim3((unsigned)blocks), dim3(256), 0, st, buf, n, units, out); break;
    case 12: hipLaunchKernelGGL(unpack_fixed_kernel<12>, dim3((unsigned)blocks), dim3(256), 0, st, buf, n, units, out); break;
    default: hipLaunchKernelGGL(unpack_fixed_kernel<16>, dim3((unsigned)blocks), dim3(256), 0, st, buf, n, units, out); break;
    }
    hipError_t err = hipGetLastError();
    if (err != hipSuccess) return set_hip_error(err, "vq2 unpack_fixed launch");
    return VQ2_OK;
}

}  // namespace vq2
