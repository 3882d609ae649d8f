// KV-cache maintenance (gfx950).
//
// Replaces, on device, the cache updates of the reference's decode loop
// (src/pallas_flash/model.py):
//   _cache_write (:257-262) as prefill (:299), decode_step (:342) and
//   ring_decode_step (:487) call it;
//   the ring-buffer slot scatter of prefill_ring (:437, :447-448);
// and `write_to_paged_cache` (paged.py:205-223), batched over sequences.
// (The single-token write of the fused decode step happens inside the
// streaming decode kernel, decode_stream.hip.)
//
// Both kernels are bandwidth-trivial (a few rows per sequence): at the kernel
// head dims (64, 128 and, 16-bit, 256) one thread moves one 16-byte chunk of
// the first half of a row together with the chunk D/2 further, so a row is
// 2 * D * ES / 16 coalesced 16-byte accesses; any other row of whole 16-byte
// chunks (D = 0 instantiation: the row length p.dr read at run time) moves
// one chunk per thread.
// Positions come from device memory, so a caller can advance them on the
// GPU between replays of a captured step.
//
// Index rules (deliberately stricter than the reference's clamping
// dynamic_update_slice, which would move an out-of-range write onto a valid
// slot): a row whose target is out of range is not written at all.
//   contiguous, linear: row i of batch b -> slot pos_b + i, written iff
//     0 <= slot < cache_size;
//   contiguous, ring:   slot (pos_b + i) mod cache_size, written iff
//     pos_b + i >= 0 and i >= seq_len - cache_size (only the last cache_size
//     rows, as prefill_ring keeps: otherwise two rows would race for a slot);
//   paged: position p = pos_b + i -> logical page p / page_size, offset
//     p % page_size, physical page block_tables[b][p / page_size], written iff
//     p >= 0, the logical page < pages_per_seq and the physical page lies in
//     [0, num_pages).
#include "pf_common.hpp"
#include "pf_kernels.hpp"

namespace pf {

namespace {

// Target slot of row i of a contiguous (linear or ring) write; -1 = skip.
__device__ inline int64_t cache_slot(int64_t pos, int i, int seq_len, int cache_size, bool ring) {
  const int64_t p = pos + i;
  if (ring) {
    if (p < 0 || i < seq_len - cache_size) return -1;
    return p % cache_size;
  }
  return (p >= 0 && p < cache_size) ? p : -1;
}

// ---------------------------------------------------------------------------
// Contiguous / ring cache write: k, v [B, Hkv, L, D] -> caches [B, Hkv, C, D].
// ---------------------------------------------------------------------------
template <typename T, int D>
__global__ __launch_bounds__(256) void pf_kv_cache_write_kernel(KvWriteParams p, int64_t n_items) {
  constexpr int EPC = 16 / (int)sizeof(T);
  const int dr = D > 0 ? D : p.dr;
  const int HC = D > 0 ? D / 2 / EPC : p.dr / EPC;  // chunk pairs (D = 0: chunks) per row
  const int64_t item = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (item >= n_items) return;
  const int c = (int)(item % HC);
  int64_t r = item / HC;
  const int i = (int)(r % p.L);
  r /= p.L;
  const int which = (int)(r & 1);  // 0 = K, 1 = V
  const int64_t bh = r >> 1;       // b * Hkv + kvh
  const int b = (int)(bh / p.Hkv);
  const int64_t slot = cache_slot(p.positions[(int64_t)b * p.pos_stride], i, p.L, p.C, p.ring != 0);
  if (slot < 0) return;
  const T* src = static_cast<const T*>(which ? p.v : p.k) + (bh * p.L + i) * dr + c * EPC;
  T* dst = static_cast<T*>(which ? p.v_cache : p.k_cache) + (bh * p.C + slot) * dr + c * EPC;
  stg16_nt(dst, ldg16_nt(src));
  if constexpr (D > 0) stg16_nt(dst + D / 2, ldg16_nt(src + D / 2));
}

// ---------------------------------------------------------------------------
// Paged write: k, v [B, Hkv, L, D] -> pools [num_pages, Hkv, page_size, D].
// ---------------------------------------------------------------------------
template <typename T, int D>
__global__ __launch_bounds__(256) void pf_paged_cache_write_kernel(PagedWriteParams p, int64_t n_items) {
  constexpr int EPC = 16 / (int)sizeof(T);
  const int dr = D > 0 ? D : p.dr;
  const int HC = D > 0 ? D / 2 / EPC : p.dr / EPC;
  const int64_t item = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (item >= n_items) return;
  const int c = (int)(item % HC);
  int64_t r = item / HC;
  const int i = (int)(r % p.L);
  r /= p.L;
  const int which = (int)(r & 1);
  const int64_t bh = r >> 1;
  const int b = (int)(bh / p.Hkv), kvh = (int)(bh % p.Hkv);
  const int64_t pos = (int64_t)p.positions[(int64_t)b * p.pos_stride] + i;
  if (pos < 0) return;
  const int64_t lp = pos / p.page_size;
  if (lp >= p.pages_per_seq) return;
  const int page = p.block_tables[(int64_t)b * p.pages_per_seq + lp];
  if (page < 0 || page >= p.num_pages) return;
  const int off = (int)(pos - lp * p.page_size);
  const T* src = static_cast<const T*>(which ? p.v : p.k) + (bh * p.L + i) * dr + c * EPC;
  T* dst = static_cast<T*>(which ? p.v_pages : p.k_pages) +
           (((int64_t)page * p.Hkv + kvh) * p.page_size + off) * dr + c * EPC;
  stg16_nt(dst, ldg16_nt(src));
  if constexpr (D > 0) stg16_nt(dst + D / 2, ldg16_nt(src + D / 2));
}

template <typename T, int D>
hipError_t kv_write_typed(const KvWriteParams& p, hipStream_t st) {
  const int HC = D > 0 ? D / 2 / (16 / (int)sizeof(T)) : p.dr / (16 / (int)sizeof(T));
  const int64_t n = (int64_t)p.B * p.Hkv * 2 * p.L * HC;
  if (n == 0) return hipSuccess;
  hipLaunchKernelGGL((pf_kv_cache_write_kernel<T, D>), dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, p, n);
  return hipGetLastError();
}

template <typename T, int D>
hipError_t paged_write_typed(const PagedWriteParams& p, hipStream_t st) {
  const int HC = D > 0 ? D / 2 / (16 / (int)sizeof(T)) : p.dr / (16 / (int)sizeof(T));
  const int64_t n = (int64_t)p.B * p.Hkv * 2 * p.L * HC;
  if (n == 0) return hipSuccess;
  hipLaunchKernelGGL((pf_paged_cache_write_kernel<T, D>), dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st,
                     p, n);
  return hipGetLastError();
}

#define PF_DISPATCH_ALL(FN, ...)                                   \
  do {                                                             \
    if (head_dim == 128) {                                         \
      if (dtype == kF32) return FN<float, 128>(__VA_ARGS__);       \
      if (dtype == kBF16) return FN<bf16_t, 128>(__VA_ARGS__);     \
      if (dtype == kF16) return FN<f16_t, 128>(__VA_ARGS__);       \
    } else if (head_dim == 64) {                                   \
      if (dtype == kF32) return FN<float, 64>(__VA_ARGS__);        \
      if (dtype == kBF16) return FN<bf16_t, 64>(__VA_ARGS__);      \
      if (dtype == kF16) return FN<f16_t, 64>(__VA_ARGS__);        \
    } else if (head_dim == 256 && dtype != kF32) {                 \
      if (dtype == kBF16) return FN<bf16_t, 256>(__VA_ARGS__);     \
      if (dtype == kF16) return FN<f16_t, 256>(__VA_ARGS__);       \
    } else {                                                       \
      if (dtype == kF32) return FN<float, 0>(__VA_ARGS__);         \
      if (dtype == kBF16) return FN<bf16_t, 0>(__VA_ARGS__);       \
      if (dtype == kF16) return FN<f16_t, 0>(__VA_ARGS__);         \
    }                                                              \
    return hipErrorInvalidValue;                                   \
  } while (0)

}  // namespace

hipError_t launch_kv_cache_write(const KvWriteParams& p, int dtype, int head_dim, hipStream_t stream) {
  PF_DISPATCH_ALL(kv_write_typed, p, stream);
}

hipError_t launch_paged_cache_write(const PagedWriteParams& p, int dtype, int head_dim, hipStream_t stream) {
  PF_DISPATCH_ALL(paged_write_typed, p, stream);
}


}  // namespace pf
