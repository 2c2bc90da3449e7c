// hbm_ceiling_probe.hip — a standalone measurement program, not part of libiekv.so.
// The HBM streaming rates this GPU reaches with the access shape of the kv_move
// kernels (256-thread workgroups, 16-byte non-temporal loads and stores, one 4 KiB or
// 8 KiB chunk per workgroup, chunks in address order): read-only, write-only and a
// contiguous copy of 8 GiB buffers, each on all-zero and on pseudo-random data.
// These are the practical ceilings the handoff kernels are compared with.
//   hipcc --offload-arch=gfx950 -O3 -std=c++17 -Xclang -target-feature \
//       -Xclang -packed-fp32-ops inference-engine_amd/csrc/hbm_ceiling_probe.hip -o /tmp/hbm_ceiling_probe
//   /tmp/hbm_ceiling_probe      # one JSON line per (data, pass, kind, chunk)
#include <hip/hip_runtime.h>
#include <cstdio>
#include <cstdint>
#include <cstdlib>

#define CK(x) do { hipError_t e = (x); if (e != hipSuccess) { printf("HIP %s at %d\n", hipGetErrorString(e), __LINE__); exit(1);} } while (0)
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
template <typename T> using gptr = __attribute__((address_space(1))) T*;

__device__ __forceinline__ uint32_t mix(uint64_t x) {
  x ^= x >> 33; x *= 0xff51afd7ed558ccdULL; x ^= x >> 33; x *= 0xc4ceb9fe1a85ec53ULL; x ^= x >> 33;
  return static_cast<uint32_t>(x);
}

__global__ void __launch_bounds__(256) fill(u32x4* p, int64_t n, int random) {
  for (int64_t i = blockIdx.x * 256ll + threadIdx.x; i < n; i += int64_t(gridDim.x) * 256) {
    u32x4 v = {0u, 0u, 0u, 0u};
    if (random) v = {mix(4 * i), mix(4 * i + 1), mix(4 * i + 2), mix(4 * i + 3)};
    p[i] = v;
  }
}

template <int U>
__global__ void __launch_bounds__(256) rd(const u32x4* src, uint32_t* out) {
  gptr<const u32x4> s = (gptr<const u32x4>)src + int64_t(blockIdx.x) * 256 * U;
  u32x4 acc = {0u, 0u, 0u, 0u};
  u32x4 x[U];
#pragma unroll
  for (int u = 0; u < U; ++u) x[u] = __builtin_nontemporal_load(s + threadIdx.x + u * 256);
#pragma unroll
  for (int u = 0; u < U; ++u) acc ^= x[u];
  const uint32_t r = acc.x ^ acc.y ^ acc.z ^ acc.w;
  if (r == 0x9e3779b9u) out[blockIdx.x & 1023] = r;   // keeps the loads; practically never taken
}

template <int U>
__global__ void __launch_bounds__(256) wr(u32x4* dst, int random) {
  gptr<u32x4> d = (gptr<u32x4>)dst + int64_t(blockIdx.x) * 256 * U;
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const int64_t i = int64_t(blockIdx.x) * 256 * U + threadIdx.x + u * 256;
    u32x4 v = {0u, 0u, 0u, 0u};
    if (random) v = {mix(4 * i), mix(4 * i + 1), mix(4 * i + 2), mix(4 * i + 3)};
    __builtin_nontemporal_store(v, d + threadIdx.x + u * 256);
  }
}

template <int U>
__global__ void __launch_bounds__(256) cp(const u32x4* src, u32x4* dst) {
  const int64_t base = int64_t(blockIdx.x) * 256 * U;
  gptr<const u32x4> s = (gptr<const u32x4>)src + base;
  gptr<u32x4> d = (gptr<u32x4>)dst + base;
  u32x4 x[U];
#pragma unroll
  for (int u = 0; u < U; ++u) x[u] = __builtin_nontemporal_load(s + threadIdx.x + u * 256);
#pragma unroll
  for (int u = 0; u < U; ++u) __builtin_nontemporal_store(x[u], d + threadIdx.x + u * 256);
}

int main() {
  const int64_t bytes = 8ll << 30;
  const int64_t vecs = bytes / 16;
  u32x4 *a, *b; uint32_t* out;
  CK(hipMalloc(&a, bytes)); CK(hipMalloc(&b, bytes)); CK(hipMalloc(&out, 4096));
  hipEvent_t e0, e1; CK(hipEventCreate(&e0)); CK(hipEventCreate(&e1));
  for (int random = 0; random <= 1; ++random) {
    for (int pass = 0; pass < 2; ++pass) {
      hipLaunchKernelGGL(fill, dim3(8192), dim3(256), 0, 0, a, vecs, random);
      hipLaunchKernelGGL(fill, dim3(8192), dim3(256), 0, 0, b, vecs, random);
      CK(hipDeviceSynchronize());
      for (int u : {1, 2}) {
        const uint32_t grid = static_cast<uint32_t>(vecs / (256 * u));
        for (int kind = 0; kind < 3; ++kind) {
          float best = 1e30f, sum = 0.f;
          const int reps = 6;
          for (int r = 0; r < reps + 1; ++r) {
            CK(hipEventRecord(e0, 0));
            if (kind == 0) { if (u == 1) hipLaunchKernelGGL(rd<1>, dim3(grid), dim3(256), 0, 0, a, out);
                             else hipLaunchKernelGGL(rd<2>, dim3(grid), dim3(256), 0, 0, a, out); }
            if (kind == 1) { if (u == 1) hipLaunchKernelGGL(wr<1>, dim3(grid), dim3(256), 0, 0, b, random);
                             else hipLaunchKernelGGL(wr<2>, dim3(grid), dim3(256), 0, 0, b, random); }
            if (kind == 2) { if (u == 1) hipLaunchKernelGGL(cp<1>, dim3(grid), dim3(256), 0, 0, a, b);
                             else hipLaunchKernelGGL(cp<2>, dim3(grid), dim3(256), 0, 0, a, b); }
            CK(hipEventRecord(e1, 0));
            CK(hipEventSynchronize(e1));
            float ms; CK(hipEventElapsedTime(&ms, e0, e1));
            if (r == 0) continue;
            best = ms < best ? ms : best; sum += ms;
          }
          const double moved = (kind == 2 ? 2.0 : 1.0) * bytes;
          printf("{\"data\": \"%s\", \"pass\": %d, \"kind\": \"%s\", \"chunk_KiB\": %d, \"TBps_mean\": %.3f, \"TBps_best\": %.3f}\n",
                 random ? "random" : "zeros", pass, kind == 0 ? "read" : kind == 1 ? "write" : "copy", 4 * u,
                 moved / (sum / reps * 1e-3) / 1e12, moved / (best * 1e-3) / 1e12);
          fflush(stdout);
        }
      }
    }
  }
  CK(hipFree(a)); CK(hipFree(b)); CK(hipFree(out));
  return 0;
}
