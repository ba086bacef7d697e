// Streaming-bandwidth ceiling for the HBM-bound kernels of the path: a plain
// grid-stride kernel that reads rd 16-byte chunks and writes wr chunks per
// group (16 B per lane, two groups of loads in flight per thread, nontemporal
// loads and stores), i.e. the fastest data movement of a given read/write
// mix and byte count on this device.  bench.py times it at the byte counts
// and read/write mixes of quant_pool and linear_states.  Measurement only:
// bench.py builds it into its own library (bench_stream_probe.so), apart
// from the product library.
#include <hip/hip_runtime.h>

#include <cstdint>

namespace {

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
constexpr int kU = 2;  // groups per thread per pass

template <int RD, int WR>
__global__ __launch_bounds__(256) void stream_kernel(const u32x4* __restrict__ src,
                                                     u32x4* __restrict__ dst, int64_t n_grp,
                                                     u32x4* __restrict__ sink) {
  const int64_t stride = (int64_t)gridDim.x * 256 * kU;
  u32x4 acc = {0u, 0u, 0u, 0u};
  for (int64_t base = (int64_t)blockIdx.x * 256 * kU + threadIdx.x; base < n_grp; base += stride) {
    u32x4 v[kU][RD];
#pragma unroll
    for (int u = 0; u < kU; ++u) {
      const int64_t i = base + (int64_t)u * 256;
#pragma unroll
      for (int r = 0; r < RD; ++r)
        v[u][r] = i < n_grp ? __builtin_nontemporal_load(src + i + r * n_grp) : u32x4{0u, 0u, 0u, 0u};
    }
#pragma unroll
    for (int u = 0; u < kU; ++u) {
      const int64_t i = base + (int64_t)u * 256;
      u32x4 x = v[u][0];
#pragma unroll
      for (int r = 1; r < RD; ++r) x ^= v[u][r];
      if (WR == 0) {
        acc ^= x;
      } else if (i < n_grp) {
#pragma unroll
        for (int w = 0; w < WR; ++w) __builtin_nontemporal_store(x + (unsigned)w, dst + i + w * n_grp);
      }
    }
  }
  // read-only mix: keep the loads live without a store per group
  if (WR == 0 && (acc.x & acc.y & acc.z & acc.w) == 0xffffffffu) sink[blockIdx.x] = acc;
}

}  // namespace

// src holds rd * n_grp chunks of 16 B, dst wr * n_grp chunks (sink: grid
// chunks, used by the read-only mix).  Mixes: (2,1) (1,1) (1,2) (1,0).
extern "C" int sla2h_probe_stream(const void* src, void* dst, void* sink, int64_t n_grp, int rd,
                                  int wr, int grid, void* stream) {
  if (!src || !sink || n_grp <= 0 || grid <= 0 || (wr > 0 && !dst)) return (int)hipErrorInvalidValue;
  auto s = static_cast<const u32x4*>(src);
  auto d = static_cast<u32x4*>(dst);
  auto k = static_cast<u32x4*>(sink);
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (rd == 2 && wr == 1)
    stream_kernel<2, 1><<<grid, 256, 0, st>>>(s, d, n_grp, k);
  else if (rd == 1 && wr == 1)
    stream_kernel<1, 1><<<grid, 256, 0, st>>>(s, d, n_grp, k);
  else if (rd == 1 && wr == 2)
    stream_kernel<1, 2><<<grid, 256, 0, st>>>(s, d, n_grp, k);
  else if (rd == 1 && wr == 0)
    stream_kernel<1, 0><<<grid, 256, 0, st>>>(s, d, n_grp, k);
  else
    return (int)hipErrorInvalidValue;
  return (int)hipGetLastError();
}
