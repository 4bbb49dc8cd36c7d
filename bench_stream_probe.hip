// Streaming-bandwidth reference points for bench.py --ceiling-probe (built by
// __graft_entry__.build() into ./bench_stream_probe): read-only, write-only and copy kernels over
// 2 GiB buffers with 16-byte accesses, plain and non-temporal, at several grid sizes, plus
// hipMemcpy device-to-device.  One JSON line per measurement (best grid), HIP-event timed,
// 20 repetitions after 3 warm-ups.
#include <hip/hip_runtime.h>

#include <cstdio>
#include <cstdlib>

typedef float float4_t __attribute__((ext_vector_type(4)));

#define CHECK(x)                                                                  \
  do {                                                                            \
    hipError_t e_ = (x);                                                          \
    if (e_ != hipSuccess) {                                                       \
      fprintf(stderr, "HIP error %s at line %d\n", hipGetErrorString(e_), __LINE__); \
      exit(1);                                                                    \
    }                                                                             \
  } while (0)

constexpr int kUnroll = 8;

template <bool NT>
__global__ __launch_bounds__(256) void k_read(const float4_t* __restrict__ a, size_t n, float* out) {
  float4_t s = {0, 0, 0, 0};
  const size_t stride = (size_t)gridDim.x * 256 * kUnroll;
  for (size_t base = (size_t)blockIdx.x * 256 * kUnroll + threadIdx.x; base < n; base += stride) {
    float4_t v[kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      const size_t i = base + (size_t)u * 256;
      v[u] = i < n ? (NT ? __builtin_nontemporal_load(a + i) : a[i]) : float4_t{0, 0, 0, 0};
    }
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) s += v[u];
  }
  if (s[0] + s[1] + s[2] + s[3] == 12345.f) out[0] = 1.f;   // keeps the loads; never true here
}

template <bool NT>
__global__ __launch_bounds__(256) void k_write(float4_t* __restrict__ a, size_t n) {
  const size_t stride = (size_t)gridDim.x * 256 * kUnroll;
  for (size_t base = (size_t)blockIdx.x * 256 * kUnroll + threadIdx.x; base < n; base += stride) {
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      const size_t i = base + (size_t)u * 256;
      if (i < n) {
        if (NT) __builtin_nontemporal_store(float4_t{1, 2, 3, 4}, a + i);
        else a[i] = float4_t{1, 2, 3, 4};
      }
    }
  }
}

template <bool NT>
__global__ __launch_bounds__(256) void k_copy(const float4_t* __restrict__ a, float4_t* __restrict__ b, size_t n) {
  const size_t stride = (size_t)gridDim.x * 256 * kUnroll;
  for (size_t base = (size_t)blockIdx.x * 256 * kUnroll + threadIdx.x; base < n; base += stride) {
    float4_t v[kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      const size_t i = base + (size_t)u * 256;
      v[u] = i < n ? (NT ? __builtin_nontemporal_load(a + i) : a[i]) : float4_t{0, 0, 0, 0};
    }
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      const size_t i = base + (size_t)u * 256;
      if (i < n) {
        if (NT) __builtin_nontemporal_store(v[u], b + i);
        else b[i] = v[u];
      }
    }
  }
}

template <class F>
float time_ms(F f) {
  hipEvent_t e0, e1;
  CHECK(hipEventCreate(&e0));
  CHECK(hipEventCreate(&e1));
  for (int i = 0; i < 3; ++i) f();
  CHECK(hipDeviceSynchronize());
  CHECK(hipEventRecord(e0));
  for (int i = 0; i < 20; ++i) f();
  CHECK(hipEventRecord(e1));
  CHECK(hipEventSynchronize(e1));
  float ms = 0.f;
  CHECK(hipEventElapsedTime(&ms, e0, e1));
  CHECK(hipEventDestroy(e0));
  CHECK(hipEventDestroy(e1));
  return ms / 20;
}

int main() {
  const size_t bytes = (size_t)2 << 30;
  const size_t n = bytes / sizeof(float4_t);
  float4_t *a = nullptr, *b = nullptr;
  float* out = nullptr;
  CHECK(hipMalloc(&a, bytes));
  CHECK(hipMalloc(&b, bytes));
  CHECK(hipMalloc(&out, 64));
  CHECK(hipMemset(a, 0, bytes));
  CHECK(hipMemset(b, 0, bytes));
  const float ms = time_ms([&] { CHECK(hipMemcpyAsync(b, a, bytes, hipMemcpyDeviceToDevice)); });
  printf("{\"probe\": \"hipMemcpy device-to-device 2 GiB\", \"ms\": %.4f, \"TB/s read+write\": %.3f}\n", ms,
         2.0 * bytes / ms / 1e9);
  struct Case {
    const char* name;
    double moved;   // bytes read + written per launch
  };
  const Case cases[6] = {{"read, 16-B loads", 1.0 * bytes},          {"read, 16-B non-temporal loads", 1.0 * bytes},
                         {"write, 16-B stores", 1.0 * bytes},        {"write, 16-B non-temporal stores", 1.0 * bytes},
                         {"copy, 16-B loads and stores", 2.0 * bytes}, {"copy, non-temporal", 2.0 * bytes}};
  for (int c = 0; c < 6; ++c) {
    float best = 1e30f;
    int best_grid = 0;
    for (int grid : {1024, 4096, 16384}) {
      float t = 0.f;
      switch (c) {
        case 0: t = time_ms([&] { hipLaunchKernelGGL(k_read<false>, dim3(grid), dim3(256), 0, 0, a, n, out); }); break;
        case 1: t = time_ms([&] { hipLaunchKernelGGL(k_read<true>, dim3(grid), dim3(256), 0, 0, a, n, out); }); break;
        case 2: t = time_ms([&] { hipLaunchKernelGGL(k_write<false>, dim3(grid), dim3(256), 0, 0, b, n); }); break;
        case 3: t = time_ms([&] { hipLaunchKernelGGL(k_write<true>, dim3(grid), dim3(256), 0, 0, b, n); }); break;
        case 4: t = time_ms([&] { hipLaunchKernelGGL(k_copy<false>, dim3(grid), dim3(256), 0, 0, a, b, n); }); break;
        default: t = time_ms([&] { hipLaunchKernelGGL(k_copy<true>, dim3(grid), dim3(256), 0, 0, a, b, n); }); break;
      }
      CHECK(hipGetLastError());
      if (t < best) {
        best = t;
        best_grid = grid;
      }
    }
    printf("{\"probe\": \"streaming %s, 2 GiB\", \"ms\": %.4f, \"TB/s\": %.3f, \"workgroups\": %d}\n", cases[c].name,
           best, cases[c].moved / best / 1e9, best_grid);
  }
  CHECK(hipFree(a));
  CHECK(hipFree(b));
  CHECK(hipFree(out));
  return 0;
}
