// stream_probe -- how fast one 512-thread workgroup per CU streams 64 KB "stages" (8 x 16 bytes
// per thread, then a wait and a barrier, as the grouped kernel's k-loop does) with
//   vgpr:     buffer loads into registers,
//   dma:      buffer_load_dwordx4 ... lds straight into LDS (the k-loop's loads),
//   vgpr+lds: loads into registers, then ds_write_b128 into LDS,
// from a 2 MB buffer (L2-resident) and from a 1 GB one (HBM).  Prints TB/s over 256 CUs.
// Every global access stays inside buf (S bytes, a power of two); every LDS write inside 64 KB.
//   hipcc --offload-arch=gfx950 -O3 -Xclang -target-feature -Xclang -packed-fp32-ops \
//         grouped_gemm_gpu_kernel_amd/bench/stream_probe.hip -o grouped_gemm_gpu_kernel_amd/_build/bin/stream_probe
#include <hip/hip_runtime.h>
#include <stdio.h>
#include <stdint.h>
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

__device__ __forceinline__ void dma16(const void* base, uint32_t nrec, uint32_t lds, uint32_t voff) {
  const uint64_t b = reinterpret_cast<uint64_t>(base);
  const u32x4_t rsrc = {(uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)b),
                        (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)(b >> 32)) & 0xffffu,
                        (uint32_t)__builtin_amdgcn_readfirstlane(nrec), 0x00020000u};
  const uint32_t m0 = __builtin_amdgcn_readfirstlane(lds);
  asm volatile("s_nop 4\n\tbuffer_load_dwordx4 %1, %2, 0 offen lds" : : "{m0}"(m0), "v"(voff), "s"(rsrc) : "memory");
}

// MODE 0: VGPR loads, 1: LDS-DMA loads, 2: VGPR loads then ds_write_b128
template <int MODE, int N>
__global__ __launch_bounds__(512) void stream(const u32x4* __restrict__ buf, uint32_t mask16, int iters, uint32_t* out) {
  __shared__ __attribute__((aligned(16))) u32x4 lds[4096];  // 64 KB
  const int tid = threadIdx.x;
  const int wave = tid >> 6, lane = tid & 63;
  uint32_t acc = 0;
  uint32_t base = (blockIdx.x * 977u) * 4096u;
  for (int it = 0; it < iters; ++it) {
    if (MODE == 1) {
#pragma unroll
      for (int j = 0; j < N; ++j) {
        const uint32_t idx = (base + (uint32_t)it * (uint32_t)(N * 512) + (uint32_t)j * 512 + tid) & mask16;
        const uint32_t slot = (uint32_t)((j * 8 + wave) & 63);  // 1 KB slots, 64 of them
        dma16(buf, (mask16 + 1) * 16u, (uint32_t)(uintptr_t)(__attribute__((address_space(3))) void*)lds + slot * 1024u, idx * 16u);
      }
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
      __syncthreads();
      acc ^= lds[(tid * 7) & 4095].x;
    } else {
      u32x4 v[N];
#pragma unroll
      for (int j = 0; j < N; ++j) {
        const uint32_t idx = (base + (uint32_t)it * (uint32_t)(N * 512) + (uint32_t)j * 512 + tid) & mask16;
        v[j] = buf[idx];
      }
      if (MODE == 2) {
#pragma unroll
        for (int j = 0; j < N; ++j) lds[((j * 8 + wave) & 63) * 64 + lane] = v[j];
        __syncthreads();
        acc ^= lds[(tid * 7) & 4095].x;
      } else {
#pragma unroll
        for (int j = 0; j < N; ++j) acc ^= v[j].x ^ v[j].y ^ v[j].z ^ v[j].w;
        __syncthreads();
      }
    }
  }
  if (acc == 0x12345678u) out[blockIdx.x * 512 + tid] = acc;
}

template <int MODE, int N>
double run(const u32x4* buf, size_t S, int iters, uint32_t* out) {
  hipEvent_t a, b; (void)hipEventCreate(&a); (void)hipEventCreate(&b);
  const uint32_t mask16 = (uint32_t)(S / 16 - 1);
  hipLaunchKernelGGL((stream<MODE, N>), dim3(256), dim3(512), 0, 0, buf, mask16, iters, out);
  (void)hipEventRecord(a);
  hipLaunchKernelGGL((stream<MODE, N>), dim3(256), dim3(512), 0, 0, buf, mask16, iters, out);
  (void)hipEventRecord(b); (void)hipEventSynchronize(b);
  float ms; (void)hipEventElapsedTime(&ms, a, b);
  return 256.0 * 512 * N * 16.0 * iters / (ms * 1e-3) / 1e12;
}
int main() {
  const size_t maxS = 1ull << 30;
  u32x4* buf; (void)hipMalloc(&buf, maxS); (void)hipMemset(buf, 1, maxS);
  uint32_t* out; (void)hipMalloc(&out, 256 * 512 * 4);
  const int iters = 400;
  for (size_t S : {1ull << 21, 1ull << 30}) {
    printf("S=%zu MB (TB/s over 256 CUs)\n", S >> 20);
    printf("  vgpr     N=4 %.2f N=8 %.2f\n", run<0, 4>(buf, S, iters * 2, out), run<0, 8>(buf, S, iters, out));
    printf("  dma      N=4 %.2f N=8 %.2f\n", run<1, 4>(buf, S, iters * 2, out), run<1, 8>(buf, S, iters, out));
    printf("  vgpr+lds N=4 %.2f N=8 %.2f\n", run<2, 4>(buf, S, iters * 2, out), run<2, 8>(buf, S, iters, out));
    fflush(stdout);
  }
  printf("done\n");
  return 0;
}
