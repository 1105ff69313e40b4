// bench_gather.hip -- gather-ceiling microbenchmark for the VQ GEMV roofline.
//
// Streams 64M uint16 codes (non-temporal 16-byte loads) and, per code,
// gathers one entry of a 1 MiB table -- the access pattern of a VQ GEMV at
// batch 1 with the reference layout (a 65536 x 8 fp16 codebook) -- in several
// load flavours (including gfx950's direct-to-LDS global_load_lds_dwordx4),
// plus a 128 KiB LDS-resident table for comparison.  Prints codes/s for each.
// Every index is masked into its table.
// Build: make -C compressai_amd/csrc bench_gather
#include <hip/hip_runtime.h>
#include <stdio.h>
#include <stdint.h>
#include <vector>
#include <stdlib.h>
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

#define CK(x) do { hipError_t e = (x); if (e != hipSuccess) { printf("HIP %s @%d\n", hipGetErrorString(e), __LINE__); exit(1);} } while (0)

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc((void*)base, (short)0, (int)bytes, 0x00020000);
}

template <int MODE>
__global__ void __launch_bounds__(256) kgather(const uint16_t* __restrict__ codes, int64_t n, const u32x4* __restrict__ tab, uint32_t* out) {
  extern __shared__ u32x4 lds[];
  __shared__ u32x4 lds_dma[MODE == 8 ? 4 * 8 * 64 : 1];  // per wave: 8 gathers x 64 lanes x 16 B
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  if constexpr (MODE == 5) {
    for (int i = threadIdx.x; i < 8192; i += blockDim.x) lds[i] = tab[i];
    __syncthreads();
  }
  __amdgpu_buffer_rsrc_t rs = make_rsrc(tab, 1 << 20);
  uint32_t acc = 0;
  const int64_t tid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t nth = (int64_t)gridDim.x * blockDim.x;
  // each thread consumes 8 codes (one 16-B word) per iteration
  for (int64_t w = tid; w * 8 < n; w += nth) {
    u32x4 v = __builtin_nontemporal_load((const u32x4*)(codes) + w);
    uint32_t c[8] = {v.x & 0xffff, v.x >> 16, v.y & 0xffff, v.y >> 16, v.z & 0xffff, v.z >> 16, v.w & 0xffff, v.w >> 16};
    if constexpr (MODE == 0) {
#pragma unroll
      for (int q = 0; q < 8; q++) acc += c[q];
    } else if constexpr (MODE == 1) {
      u32x4 g[8];
#pragma unroll
      for (int q = 0; q < 8; q++) g[q] = tab[c[q]];
#pragma unroll
      for (int q = 0; q < 8; q++) acc ^= g[q].x + g[q].y + g[q].z + g[q].w;
    } else if constexpr (MODE == 2 || MODE == 3 || MODE == 6) {
      constexpr int AUX = MODE == 2 ? 1 : MODE == 3 ? 2 : 3;
      u32x4 g[8];
#pragma unroll
      for (int q = 0; q < 8; q++) g[q] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rs, c[q] * 16, 0, AUX));
#pragma unroll
      for (int q = 0; q < 8; q++) acc ^= g[q].x + g[q].y + g[q].z + g[q].w;
    } else if constexpr (MODE == 4) {
      const u32x2* t2 = (const u32x2*)tab;
      u32x2 g[8];
#pragma unroll
      for (int q = 0; q < 8; q++) g[q] = t2[c[q]];
#pragma unroll
      for (int q = 0; q < 8; q++) acc ^= g[q].x + g[q].y;
    } else if constexpr (MODE == 5) {
      u32x4 g[8];
#pragma unroll
      for (int q = 0; q < 8; q++) g[q] = lds[c[q] & 8191];
#pragma unroll
      for (int q = 0; q < 8; q++) acc ^= g[q].x + g[q].y + g[q].z + g[q].w;
    } else if constexpr (MODE == 8) {
      // each lane's centroid lands in LDS at the wave's slot base + lane * 16
#pragma unroll
      for (int q = 0; q < 8; q++)
        __builtin_amdgcn_global_load_lds((__attribute__((address_space(1))) void*)(tab + c[q]),
                                         (__attribute__((address_space(3))) void*)(lds_dma + (wave * 8 + q) * 64), 16, 0, 0);
      __builtin_amdgcn_s_waitcnt(0);
#pragma unroll
      for (int q = 0; q < 8; q++) {
        const u32x4 g = lds_dma[(wave * 8 + q) * 64 + lane];
        acc ^= g.x + g.y + g.z + g.w;
      }
    } else if constexpr (MODE == 7) {
      const uint32_t* t1 = (const uint32_t*)tab;
      uint32_t g[8];
#pragma unroll
      for (int q = 0; q < 8; q++) g[q] = t1[c[q] * 4];
#pragma unroll
      for (int q = 0; q < 8; q++) acc ^= g[q];
    }
  }
  out[tid] = acc;
}

template <int MODE>
float run(const uint16_t* codes, int64_t n, const u32x4* tab, uint32_t* out, int blocks, size_t shm) {
  hipEvent_t a, b; CK(hipEventCreate(&a)); CK(hipEventCreate(&b));
  hipLaunchKernelGGL(kgather<MODE>, dim3(blocks), dim3(256), shm, 0, codes, n, tab, out);
  CK(hipDeviceSynchronize());
  CK(hipEventRecord(a));
  const int R = 5;
  for (int r = 0; r < R; r++) hipLaunchKernelGGL(kgather<MODE>, dim3(blocks), dim3(256), shm, 0, codes, n, tab, out);
  CK(hipEventRecord(b)); CK(hipEventSynchronize(b));
  float ms; CK(hipEventElapsedTime(&ms, a, b));
  CK(hipGetLastError());
  return ms / R;
}

int main() {
  const int64_t n = 1LL << 26;  // 64M codes = 128 MiB stream
  uint16_t* codes; u32x4* tab; uint32_t* out;
  CK(hipMalloc(&codes, n * 2)); CK(hipMalloc(&tab, 1 << 20));
  std::vector<uint16_t> h(1 << 24);
  uint32_t s = 12345;
  for (auto& v : h) { s = s * 1664525u + 1013904223u; v = (uint16_t)(s >> 16); }
  for (int64_t o = 0; o < n; o += h.size()) CK(hipMemcpy(codes + o, h.data(), h.size() * 2, hipMemcpyHostToDevice));
  CK(hipMemset(tab, 1, 1 << 20));
  int cu = 0; CK(hipDeviceGetAttribute(&cu, hipDeviceAttributeMultiprocessorCount, 0));
  int maxlds = 0; CK(hipDeviceGetAttribute(&maxlds, hipDeviceAttributeMaxSharedMemoryPerBlock, 0));
  printf("CUs %d, max LDS per block %d\n", cu, maxlds);
  for (int bpc : {4, 8, 16}) {
    const int blocks = cu * bpc;
    CK(hipMalloc(&out, (size_t)blocks * 256 * 4));
    const char* names[] = {"stream only", "gather b128 default", "gather b128 buffer aux=1(sc0)", "gather b128 buffer aux=2(sc1)", "gather b64 default", "gather LDS b128 (128KiB)", "gather b128 buffer aux=3", "gather b32 default", "gather b128 direct to LDS"};
    float t[9];
    t[0] = run<0>(codes, n, tab, out, blocks, 0);
    t[1] = run<1>(codes, n, tab, out, blocks, 0);
    t[2] = run<2>(codes, n, tab, out, blocks, 0);
    t[3] = run<3>(codes, n, tab, out, blocks, 0);
    t[4] = run<4>(codes, n, tab, out, blocks, 0);
    t[5] = (maxlds >= 131072 && bpc <= 4) ? run<5>(codes, n, tab, out, cu, 131072) : -1.f;
    t[6] = run<6>(codes, n, tab, out, blocks, 0);
    t[7] = run<7>(codes, n, tab, out, blocks, 0);
    t[8] = bpc <= 4 ? run<8>(codes, n, tab, out, blocks, 0) : -1.f;
    for (int m = 0; m < 9; m++) {
      if (t[m] < 0) continue;
      printf("blocks/CU %2d  %-32s %8.3f ms  %7.1f G codes/s  %6.1f GB/s of codes  %.3f codes/clk/CU@2.4GHz\n", bpc, names[m], t[m],
             n / (t[m] * 1e-3) / 1e9, n * 2 / (t[m] * 1e-3) / 1e9, n / (t[m] * 1e-3) / (cu * 2.4e9));
    }
    CK(hipFree(out));
  }
  return 0;
}
