// Measurement probes for bench.py (not part of the attention C ABI), built
// into their own library (libpf_bench_probe.so) by the package Makefile:
//
//  * HBM read forms: the rate a plain, fully coalesced read of a large buffer
//    reaches on this device, with four load forms -- 16-byte non-temporal
//    loads into registers, 16-byte temporal (ordinary) loads into registers,
//    and direct global -> LDS loads (buffer_load_dwordx4 ... lds, the form the
//    streaming decode kernel uses), temporal and non-temporal. The best is
//    the practical ceiling the
//    bandwidth-bound decode and paged kernels are compared with, besides the
//    8 TB/s specification.
//  * MFMA stream: back-to-back v_mfma_f32_32x32x16_bf16 with four independent
//    accumulators per wave and register operands (no memory traffic), the
//    matrix-core rate this device sustains under a pure MFMA load (its clock
//    under that power draw included), the same-run reference the prefill
//    kernels' TFLOP/s are read against besides the 2.5 PFLOP/s specification.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "pf_common.hpp"

namespace {

using pf::u32x4;

// Register loads: each thread reads 16-byte chunks, UNROLL of them in flight,
// over a grid-stride loop, and folds them into one XOR; one value per
// workgroup is stored so the loads cannot be removed.
template <int UNROLL, bool NT>
__global__ __launch_bounds__(256) void pf_probe_read_kernel(const u32x4* __restrict__ src, int64_t n_chunks,
                                                            uint32_t* __restrict__ sink) {
  const int64_t stride = (int64_t)gridDim.x * 256;
  int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  auto ld = [&](int64_t at) -> u32x4 {
    if constexpr (NT) return __builtin_nontemporal_load(src + at);
    else return src[at];
  };
  uint32_t acc = 0;
  for (; i + (UNROLL - 1) * stride < n_chunks; i += UNROLL * stride) {
    u32x4 v[UNROLL];
#pragma unroll
    for (int u = 0; u < UNROLL; ++u) v[u] = ld(i + u * stride);
#pragma unroll
    for (int u = 0; u < UNROLL; ++u) acc ^= v[u][0] ^ v[u][1] ^ v[u][2] ^ v[u][3];
  }
  for (; i < n_chunks; i += stride) {
    const u32x4 v = ld(i);
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

// Direct global -> LDS loads: each wave moves 1 KB per instruction (64 lanes x
// 16 bytes) into a wave-private ring of UNROLL 1 KB slots, issuing a batch of
// UNROLL instructions and then waiting for the previous batch, so up to
// 2 x UNROLL are in flight. Wave-chunk c covers bytes [1024 c, 1024 c + 1024).
// The buffer descriptor spans the buffer (bytes < 2^32; offsets 32-bit).
template <int UNROLL, bool NT>
__global__ __launch_bounds__(256) void pf_probe_read_lds_kernel(const void* __restrict__ src, uint32_t bytes,
                                                                uint32_t* __restrict__ sink) {
  __shared__ __attribute__((aligned(16))) char ring[4][UNROLL][1024];
  const int w = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
  const int l = threadIdx.x & 63;
  const pf::i32x4 d = pf::make_desc(src, bytes);
  const int64_t n_wc = bytes / 1024;
  const int64_t wstride = (int64_t)gridDim.x * 4;
  int64_t c = (int64_t)blockIdx.x * 4 + w;
  for (; c + (UNROLL - 1) * wstride < n_wc; c += UNROLL * wstride) {
#pragma unroll
    for (int u = 0; u < UNROLL; ++u)
      pf::dma16<NT>(d, (uint32_t)((c + u * wstride) * 1024) + 16u * l, pf::lds_u32(&ring[w][u][0]));
    pf::wait_vm<UNROLL>();
  }
  for (; c < n_wc; c += wstride) pf::dma16<NT>(d, (uint32_t)(c * 1024) + 16u * l, pf::lds_u32(&ring[w][0][0]));
  pf::wait_vm<0>();
  __syncthreads();
  // one word per workgroup from what the loads delivered
  if (threadIdx.x == 0) sink[blockIdx.x] = *reinterpret_cast<const uint32_t*>(&ring[0][0][0]);
}

// MFMA stream: ITERS x 8 MFMAs per wave in four independent accumulator
// chains (each MFMA depends on the one four back, which has finished by then).
__global__ __launch_bounds__(256) void pf_probe_mfma_kernel(float* __restrict__ out, int iters) {
  typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
  typedef float f32x16 __attribute__((ext_vector_type(16)));
  f32x16 a0 = (f32x16)(0.f), a1 = a0, a2 = a0, a3 = a0;
  bf16x8 x, y;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    x[i] = (__bf16)(1e-3f * (float)(threadIdx.x + i));
    y[i] = (__bf16)(2e-3f * (float)i);
  }
  for (int it = 0; it < iters; ++it) {
#pragma unroll
    for (int r = 0; r < 2; ++r) {
      a0 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(x, y, a0, 0, 0, 0);
      a1 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(x, y, a1, 0, 0, 0);
      a2 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(x, y, a2, 0, 0, 0);
      a3 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(x, y, a3, 0, 0, 0);
    }
  }
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < 16; ++i) s += a0[i] + a1[i] + a2[i] + a3[i];
  out[(int64_t)blockIdx.x * 256 + threadIdx.x] = s;
}

}  // namespace

extern "C" {

// Read `bytes` (a multiple of 1024, below 2^32) of device memory at `src`
// with `blocks` workgroups of 256 threads. form 0: non-temporal register
// loads, 1: temporal register loads, 2: direct-to-LDS loads, 3: non-temporal
// direct-to-LDS loads; `unroll` (4 or 8) loads in flight per thread (per wave
// for forms 2 and 3, which keep up to twice that). `sink` receives `blocks` words. Returns 0, or -1 for bad arguments /
// a launch error.
int pf_probe_read(const void* src, size_t bytes, uint32_t* sink, int blocks, int unroll, int form,
                  void* stream) {
  if (!src || !sink || blocks < 1 || bytes % 1024 != 0 || bytes >= ((size_t)1 << 32) ||
      (unroll != 4 && unroll != 8) || form < 0 || form > 3)
    return -1;
  const int64_t n = (int64_t)(bytes / 16);
  const hipStream_t st = (hipStream_t)stream;
  const u32x4* s16 = static_cast<const u32x4*>(src);
  const dim3 grid(blocks), blk(256);
  if (form == 0) {
    if (unroll == 8) hipLaunchKernelGGL((pf_probe_read_kernel<8, true>), grid, blk, 0, st, s16, n, sink);
    else hipLaunchKernelGGL((pf_probe_read_kernel<4, true>), grid, blk, 0, st, s16, n, sink);
  } else if (form == 1) {
    if (unroll == 8) hipLaunchKernelGGL((pf_probe_read_kernel<8, false>), grid, blk, 0, st, s16, n, sink);
    else hipLaunchKernelGGL((pf_probe_read_kernel<4, false>), grid, blk, 0, st, s16, n, sink);
  } else if (form == 2) {
    if (unroll == 8) hipLaunchKernelGGL((pf_probe_read_lds_kernel<8, false>), grid, blk, 0, st, src, (uint32_t)bytes, sink);
    else hipLaunchKernelGGL((pf_probe_read_lds_kernel<4, false>), grid, blk, 0, st, src, (uint32_t)bytes, sink);
  } else {
    if (unroll == 8) hipLaunchKernelGGL((pf_probe_read_lds_kernel<8, true>), grid, blk, 0, st, src, (uint32_t)bytes, sink);
    else hipLaunchKernelGGL((pf_probe_read_lds_kernel<4, true>), grid, blk, 0, st, src, (uint32_t)bytes, sink);
  }
  return hipGetLastError() == hipSuccess ? 0 : -1;
}

// `blocks` workgroups of 256 threads, each wave issuing 8 x `iters`
// 32x32x16 bf16 MFMAs (32768 FLOP each); `out` receives blocks x 256 floats.
int pf_probe_mfma(float* out, int blocks, int iters, void* stream) {
  if (!out || blocks < 1 || iters < 1) return -1;
  hipLaunchKernelGGL(pf_probe_mfma_kernel, dim3(blocks), dim3(256), 0, (hipStream_t)stream, out, iters);
  return hipGetLastError() == hipSuccess ? 0 : -1;
}

}  // extern "C"
