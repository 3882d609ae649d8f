// KV-cache maintenance and the prologue of the fused decode step (gfx950).
//
// Replaces, on device, the cache updates and the single-row RoPE of the
// reference's decode loop (src/pallas_flash/model.py):
//   _cache_write (:257-262) as prefill (:299), decode_step (:342) and
//   ring_decode_step (:487) call it;
//   the ring-buffer slot scatter of prefill_ring (:437, :447-448) and the
//   ring slot / live length of ring_decode_step (:475-476);
//   apply_rope at the new token's position (:340-341, :485-486; rotation
//   model.py:54-67);
// and `write_to_paged_cache` (paged.py:205-223), batched over sequences.
//
// All three kernels are bandwidth-trivial (a few rows per sequence): one
// thread moves one 16-byte chunk of the first half of a row together with the
// chunk D/2 further (the rotate-half partner), so a row is 2 * D * ES / 16
// coalesced 16-byte accesses. Positions come from device memory, so a caller
// can advance them on the GPU between replays of a captured step.
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

// Rotate-half RoPE of one chunk pair: x[c] (first half) and x[c + D/2]
// (second half) at table row `pos`; float32, rounded once to T. Without a
// table (cs == nullptr) the chunks pass through unchanged.
template <typename T, int D>
__device__ inline void rope_pair(u32x4& lo, u32x4& hi, const float* cs, const float* sn, int pos, int c) {
  if (cs == nullptr) return;
  constexpr int EPC = 16 / (int)sizeof(T);
  float a[EPC], bb[EPC], ra[EPC], rb[EPC];
  chunk_to_f32<T>(lo, a);
  chunk_to_f32<T>(hi, bb);
  const float* cr = cs + (int64_t)pos * D + c * EPC;
  const float* sr = sn + (int64_t)pos * D + c * EPC;
#pragma unroll
  for (int e = 0; e < EPC; ++e) {
    ra[e] = a[e] * cr[e] - bb[e] * sr[e];                  // x1 cos - x2 sin
    rb[e] = bb[e] * cr[D / 2 + e] + a[e] * sr[D / 2 + e];  // x2 cos + x1 sin
  }
  lo = f32_to_chunk<T>(ra);
  hi = f32_to_chunk<T>(rb);
}

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
  constexpr int HC = D / 2 / EPC;  // chunk pairs per row
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
  const T* src = static_cast<const T*>(which ? p.v : p.k) + (bh * p.L + i) * D + c * EPC;
  T* dst = static_cast<T*>(which ? p.v_cache : p.k_cache) + (bh * p.C + slot) * D + c * EPC;
  stg16(dst, ldg16(src));
  stg16(dst + D / 2, ldg16(src + D / 2));
}

// ---------------------------------------------------------------------------
// Paged write: k, v [B, Hkv, L, D] -> pools [num_pages, Hkv, page_size, D].
// ---------------------------------------------------------------------------
template <typename T, int D>
__global__ __launch_bounds__(256) void pf_paged_cache_write_kernel(PagedWriteParams p, int64_t n_items) {
  constexpr int EPC = 16 / (int)sizeof(T);
  constexpr int HC = D / 2 / EPC;
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
  const T* src = static_cast<const T*>(which ? p.v : p.k) + (bh * p.L + i) * D + c * EPC;
  T* dst = static_cast<T*>(which ? p.v_pages : p.k_pages) +
           (((int64_t)page * p.Hkv + kvh) * p.page_size + off) * D + c * EPC;
  stg16(dst, ldg16(src));
  stg16(dst + D / 2, ldg16(src + D / 2));
}

// ---------------------------------------------------------------------------
// Decode-step prologue. Rows: for each batch b, Hq query rows (rotated into
// q_rot), Hkv key rows (rotated into the cache slot) and Hkv value rows
// (copied into the cache slot); thread 0 of each batch's first row also
// writes kv_len[b]. An invalid position writes nothing and kv_len 0 (the
// decode then outputs zeros for that batch, flash_attention.py:150-159).
//   linear: valid iff 0 <= pos < C; slot pos; kv_len pos + 1
//   ring:   valid iff pos >= 0;      slot pos % C; kv_len min(pos + 1, C)
// With RoPE, pos must also be < rope_len (the table rows).
// ---------------------------------------------------------------------------
template <typename T, int D>
__global__ __launch_bounds__(256) void pf_decode_step_prep_kernel(DecodeStepParams p, int64_t n_items) {
  constexpr int EPC = 16 / (int)sizeof(T);
  constexpr int HC = D / 2 / EPC;
  const int64_t item = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (item >= n_items) return;
  const int rows = p.Hq + 2 * p.Hkv;
  const int c = (int)(item % HC);
  const int64_t rr = item / HC;
  const int row = (int)(rr % rows);
  const int b = (int)(rr / rows);
  const int pos = p.positions[(int64_t)b * p.pos_stride];
  bool valid = pos >= 0 && (p.ring != 0 || pos < p.C) && (p.cos == nullptr || pos < p.rope_len);
  const int slot = valid ? (p.ring ? pos % p.C : pos) : 0;
  if (row == 0 && c == 0) p.kv_lens[b] = valid ? (p.ring ? min(pos + 1, p.C) : pos + 1) : 0;

  if (row < p.Hq) {  // query row -> q_rot (rotated even for an invalid position: unused then)
    const int64_t off = ((int64_t)b * p.Hq + row) * D + c * EPC;
    u32x4 lo = ldg16(static_cast<const T*>(p.q) + off), hi = ldg16(static_cast<const T*>(p.q) + off + D / 2);
    rope_pair<T, D>(lo, hi, p.cos, p.sin, valid ? pos : 0, c);
    stg16(static_cast<T*>(p.q_rot) + off, lo);
    stg16(static_cast<T*>(p.q_rot) + off + D / 2, hi);
    return;
  }
  if (!valid) return;
  const int kr = row - p.Hq;
  const bool is_v = kr >= p.Hkv;
  const int kvh = is_v ? kr - p.Hkv : kr;
  const int64_t src = ((int64_t)b * p.Hkv + kvh) * D + c * EPC;
  const int64_t dst = (((int64_t)b * p.Hkv + kvh) * p.C + slot) * D + c * EPC;
  const T* s = static_cast<const T*>(is_v ? p.v_new : p.k_new);
  u32x4 lo = ldg16(s + src), hi = ldg16(s + src + D / 2);
  if (!is_v) rope_pair<T, D>(lo, hi, p.cos, p.sin, pos, c);
  T* d = static_cast<T*>(is_v ? p.v_cache : p.k_cache);
  stg16(d + dst, lo);
  stg16(d + dst + D / 2, hi);
}

template <typename T, int D>
hipError_t kv_write_typed(const KvWriteParams& p, hipStream_t st) {
  constexpr int HC = D / 2 / (16 / (int)sizeof(T));
  const int64_t n = (int64_t)p.B * p.Hkv * 2 * p.L * HC;
  if (n == 0) return hipSuccess;
  hipLaunchKernelGGL((pf_kv_cache_write_kernel<T, D>), dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, p, n);
  return hipGetLastError();
}

template <typename T, int D>
hipError_t paged_write_typed(const PagedWriteParams& p, hipStream_t st) {
  constexpr int HC = D / 2 / (16 / (int)sizeof(T));
  const int64_t n = (int64_t)p.B * p.Hkv * 2 * p.L * HC;
  if (n == 0) return hipSuccess;
  hipLaunchKernelGGL((pf_paged_cache_write_kernel<T, D>), dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st,
                     p, n);
  return hipGetLastError();
}

template <typename T, int D>
hipError_t step_prep_typed(const DecodeStepParams& p, hipStream_t st) {
  constexpr int HC = D / 2 / (16 / (int)sizeof(T));
  const int64_t n = (int64_t)p.B * (p.Hq + 2 * p.Hkv) * HC;
  if (n == 0) return hipSuccess;
  hipLaunchKernelGGL((pf_decode_step_prep_kernel<T, D>), dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st,
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

hipError_t launch_decode_step_prep(const DecodeStepParams& p, int dtype, int head_dim, hipStream_t stream) {
  PF_DISPATCH_ALL(step_prep_typed, p, stream);
}

}  // namespace pf
