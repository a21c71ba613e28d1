// Shared definitions for the gfx950 Conformer-encoder kernels.
#pragma once

#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <string>

namespace bark {

typedef _Float16 half;
typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half4 __attribute__((ext_vector_type(4)));
typedef float floatx16 __attribute__((ext_vector_type(16)));
typedef float floatx4 __attribute__((ext_vector_type(4)));

constexpr int HIDDEN = 1024;
constexpr int HEADS = 8;
constexpr int HDIM = 128;
constexpr int FFN = 4096;
constexpr int SUB_CH = 256;
constexpr int MEL = 128;
constexpr int PROJ = 640;

// Error raised by host code; turned into a status code at the C ABI.
struct Error {
  std::string msg;
};

#define BARK_HIP_CHECK(expr)                                                          \
  do {                                                                                \
    hipError_t e_ = (expr);                                                           \
    if (e_ != hipSuccess)                                                             \
      throw ::bark::Error{std::string(#expr) + ": " + hipGetErrorString(e_)};         \
  } while (0)

#define BARK_REQUIRE(cond, text)                                                      \
  do {                                                                                \
    if (!(cond)) throw ::bark::Error{std::string(text)};                              \
  } while (0)

// Kernel timing for the per-op profiler. While `stop` is set, every launch
// goes through hipExtLaunchKernelGGL with the events attached to the dispatch
// itself (start on the op's first kernel, stop on each, so the last one wins):
// the events then hold the kernels' own begin and end times, without the
// dispatch gaps that separate marker events would add.
struct LaunchTiming {
  hipEvent_t start = nullptr, stop = nullptr;
  int launches = 0;
};
extern thread_local LaunchTiming g_launch_timing;

#define BARK_LAUNCH(kernel, grid, block, shmem, stream, ...)                                  \
  do {                                                                                        \
    ::bark::LaunchTiming& lt_ = ::bark::g_launch_timing;                                      \
    if (lt_.stop) {                                                                           \
      hipExtLaunchKernelGGL(kernel, grid, block, shmem, stream, lt_.launches++ ? nullptr : lt_.start, \
                            lt_.stop, 0, __VA_ARGS__);                                        \
    } else {                                                                                  \
      hipLaunchKernelGGL(kernel, grid, block, shmem, stream, __VA_ARGS__);                    \
    }                                                                                         \
  } while (0)

inline int ceil_div(int a, int b) { return (a + b - 1) / b; }
inline int round_up(int a, int b) { return ceil_div(a, b) * b; }

// Uniform-address load of 8 halves (16 bytes).
__device__ inline half8 ld_half8(const half* p) { return *reinterpret_cast<const half8*>(p); }
__device__ inline void st_half8(half* p, half8 v) { *reinterpret_cast<half8*>(p) = v; }


// Butterfly reductions across the 64 lanes of a wave.
__device__ inline float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

}  // namespace bark
