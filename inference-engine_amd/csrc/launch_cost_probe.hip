// launch_cost_probe.hip — a standalone measurement program, not part of libiekv.so.
// The host's cost of issuing one kernel launch against the size of the kernel's
// argument segment: empty kernels whose arguments are 0 B to 2.4 KiB of plain bytes
// (kv_move carries 384 B, 128 B of its own plus the runtime's 256-byte block of
// hidden arguments it reads gridDim from; kv_move_inline 2,416 B). Each size is
// issued 1,000 times back to back on one stream from one thread; the sizes take
// turns over five rounds, and the median round is printed.
//   hipcc --offload-arch=gfx950 -O3 -std=c++17 -Xclang -target-feature \
//       -Xclang -packed-fp32-ops inference-engine_amd/csrc/launch_cost_probe.hip -o /tmp/launch_cost_probe
//   /tmp/launch_cost_probe      # one line per size: median, min and max us per launch
#include <hip/hip_runtime.h>
#include <algorithm>
#include <chrono>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <functional>
#include <vector>

#define CK(x) do { hipError_t e = (x); if (e != hipSuccess) { printf("HIP %s at %d\n", hipGetErrorString(e), __LINE__); exit(1);} } while (0)

template <int N> struct Words { int32_t v[N]; };

__global__ void no_args() {}

// N words of arguments; the branch is never taken, it only keeps them alive.
template <int N>
__global__ void words(Words<N> w) {
  if (threadIdx.x == 0 && blockIdx.x == 0 && w.v[N - 1] == 12345) asm volatile("" ::: "memory");
}

// The same, reading gridDim.x, which adds the hidden-argument block to the segment.
template <int N>
__global__ void words_grid(Words<N> w, int32_t* out) {
  if (out && threadIdx.x == 0 && blockIdx.x == gridDim.x + 5 && w.v[N - 1] == 12345) out[0] = 1;
}

int main() {
  hipStream_t s;
  CK(hipStreamCreate(&s));
  const int launches = 1000, rounds = 5;
  const dim3 grid(64), block(256);
  struct Case {
    const char* name;
    std::function<void()> launch;
    std::vector<double> us;
  };
  std::vector<Case> cases;
  cases.push_back({"0 B (no arguments)", [&] { hipLaunchKernelGGL(no_args, grid, block, 0, s); }, {}});
#define WORDS(N, NAME) \
  cases.push_back({NAME, [&] { Words<N> w{}; hipLaunchKernelGGL(words<N>, grid, block, 0, s, w); }, {}});
  WORDS(2, "8 B")
  WORDS(8, "32 B")
  WORDS(32, "128 B")
  WORDS(96, "384 B")
  WORDS(256, "1,024 B")
  WORDS(604, "2,416 B")
  cases.push_back({"384 B (120 B + hidden block)", [&] {
                     Words<30> w{};
                     hipLaunchKernelGGL(words_grid<30>, grid, block, 0, s, w, (int32_t*)nullptr);
                   }, {}});
  for (auto& c : cases)
    for (int i = 0; i < 50; ++i) c.launch();
  CK(hipStreamSynchronize(s));
  for (int r = 0; r < rounds; ++r) {
    for (auto& c : cases) {
      const auto t0 = std::chrono::steady_clock::now();
      for (int i = 0; i < launches; ++i) c.launch();
      const auto t1 = std::chrono::steady_clock::now();
      CK(hipStreamSynchronize(s));
      c.us.push_back(std::chrono::duration<double, std::micro>(t1 - t0).count() / launches);
    }
  }
  CK(hipGetLastError());
  for (auto& c : cases) {
    std::sort(c.us.begin(), c.us.end());
    printf("%-30s median %.3f  min %.3f  max %.3f us per launch\n", c.name, c.us[rounds / 2],
           c.us.front(), c.us.back());
  }
  CK(hipStreamDestroy(s));
  return 0;
}
