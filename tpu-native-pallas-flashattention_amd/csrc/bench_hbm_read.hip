// Streaming-read probe for bench.py (not part of the attention C ABI): the
// HBM read rate a plain, fully coalesced read of a large buffer reaches on
// this device, the practical ceiling the bandwidth-bound decode and paged
// kernels are compared with besides the 8 TB/s specification.
//
// Each thread reads 16-byte chunks with non-temporal loads, UNROLL of them in
// flight, over a grid-stride loop, and folds them into one XOR; one value per
// workgroup is stored so the loads cannot be removed. Built into its own
// library (libpf_bench_probe.so) by the package Makefile.
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

template <int UNROLL>
__global__ __launch_bounds__(256) void pf_probe_read_kernel(const u32x4* __restrict__ src, int64_t n_chunks,
                                                            uint32_t* __restrict__ sink) {
  const int64_t stride = (int64_t)gridDim.x * 256;
  int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  uint32_t acc = 0;
  for (; i + (UNROLL - 1) * stride < n_chunks; i += UNROLL * stride) {
    u32x4 v[UNROLL];
#pragma unroll
    for (int u = 0; u < UNROLL; ++u) v[u] = __builtin_nontemporal_load(src + i + u * stride);
#pragma unroll
    for (int u = 0; u < UNROLL; ++u) acc ^= v[u][0] ^ v[u][1] ^ v[u][2] ^ v[u][3];
  }
  for (; i < n_chunks; i += stride) {
    const u32x4 v = __builtin_nontemporal_load(src + i);
    acc ^= v[0] ^ v[1] ^ v[2] ^ v[3];
  }
  // one word per workgroup: the XOR of its lanes' values
  __shared__ uint32_t red[256];
  red[threadIdx.x] = acc;
  __syncthreads();
  for (int o = 128; o > 0; o >>= 1) {
    if ((int)threadIdx.x < o) red[threadIdx.x] ^= red[threadIdx.x + o];
    __syncthreads();
  }
  if (threadIdx.x == 0) sink[blockIdx.x] = red[0];
}

}  // namespace

extern "C" {

// Read `bytes` (a multiple of 16) of device memory at `src` with `blocks`
// workgroups of 256 threads, `unroll` (4 or 8) loads in flight per thread;
// `sink` receives `blocks` words. Returns 0, or -1 for bad arguments / a
// launch error.
int pf_probe_stream_read(const void* src, size_t bytes, uint32_t* sink, int blocks, int unroll, void* stream) {
  if (!src || !sink || blocks < 1 || bytes % 16 != 0 || (unroll != 4 && unroll != 8)) return -1;
  const int64_t n = (int64_t)(bytes / 16);
  const hipStream_t st = (hipStream_t)stream;
  if (unroll == 8)
    hipLaunchKernelGGL(pf_probe_read_kernel<8>, dim3(blocks), dim3(256), 0, st, static_cast<const u32x4*>(src), n, sink);
  else
    hipLaunchKernelGGL(pf_probe_read_kernel<4>, dim3(blocks), dim3(256), 0, st, static_cast<const u32x4*>(src), n, sink);
  return hipGetLastError() == hipSuccess ? 0 : -1;
}

}  // extern "C"
