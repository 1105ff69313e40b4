// vq2_misc.hip -- small kernels of the decode path: top-1 over logits,
// top-k router with the shared-expert gate, rotated-space dequant and index
// decode (gfx950).
#include "vq2_common.hpp"
#include "vq2_router.hpp"
#include "vq2_internal.hpp"

namespace vq2 {

// ------------------------------------------------------------------ argmax
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

}  // namespace vq2
