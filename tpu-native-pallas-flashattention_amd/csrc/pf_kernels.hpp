// Kernel parameter blocks and host-side launchers (internal to the library;
// the public interface is include/pallas_flash_amd.h).
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include "pf_common.hpp"

namespace pf {

// Dynamic tail of a prefill launch (forward, dQ). Workgroups are
// dispatched round-robin over the 8 XCDs, and each XCD starts its workgroups
// in blockIdx order as its CUs free up; XCDs run at somewhat different
// speeds, so with a fixed item per workgroup they finish apart (up to 5-8%
// of a launch). Workgroups [0, n_static) take work item blockIdx (each XCD's
// share, with the L2 locality the item order gives it); each of the
// n_tickets workgroups after them draws a ticket t from *tickets and takes
// item n_static + t (none when t >= n_work - n_static), so an XCD that runs
// ahead takes more of the remaining, lightest items. tickets null: every
// item static (grid = n_work).
struct WorkTail {
  unsigned int* tickets;
  int n_static;
  int n_tickets;
};

// The ticket counter of a dynamic-tail launch on `stream` (zero between
// launches; work_tickets.hip), or null: launch without a dynamic tail.
unsigned int* work_tickets(hipStream_t stream);

// The device address of a file-scope __device__ variable (HIP_SYMBOL(x)) on
// device `dev`: looked up with that device current (each device holds its
// own copy), with this thread's stream-capture mode relaxed for the lookup so
// that a first call made while a stream is recorded into a graph works too;
// the current device and capture mode are restored. Inline, so the lookup is
// compiled into the source file that defines the variable.
inline hipError_t symbol_address(int dev, const void* symbol, void** out) {
  int cur = -1;
  hipError_t e = hipGetDevice(&cur);
  if (e != hipSuccess) return e;
  if (cur != dev && (e = hipSetDevice(dev)) != hipSuccess) return e;
  hipStreamCaptureMode mode = hipStreamCaptureModeRelaxed;
  e = hipThreadExchangeStreamCaptureMode(&mode);
  if (e == hipSuccess) {
    e = hipGetSymbolAddress(out, symbol);
    const hipError_t e2 = hipThreadExchangeStreamCaptureMode(&mode);
    if (e == hipSuccess) e = e2;
  }
  if (cur != dev) {
    const hipError_t e3 = hipSetDevice(cur);
    if (e == hipSuccess) e = e3;
  }
  return e;
}

__host__ __device__ inline int work_tail_grid(const WorkTail& t, int n_work) {
  return t.tickets ? t.n_static + t.n_tickets : n_work;
}

// Work-item index of the calling workgroup (WorkTail). The workgroup that
// draws the last ticket sets the counter back to zero for the next launch on
// the stream. Returns -1 for a workgroup that finds no item left (it exits).
// Uniform over the workgroup. `lds` is any LDS word of the workgroup: a
// drawing workgroup passes the ticket through it between two barriers, so it
// is free again on return.
__device__ inline int work_tail_item(const WorkTail& w, int n_work, int* lds) {
  const int bid = blockIdx.x;
  if (w.tickets == nullptr || bid < w.n_static) return bid;
  if (threadIdx.x == 0) {
    const unsigned t = __hip_atomic_fetch_add(w.tickets, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (t == (unsigned)w.n_tickets - 1u) __hip_atomic_store(w.tickets, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    *lds = (int)t;
  }
  __syncthreads();
  const int t = *lds;
  __syncthreads();  // every wave has read the word before any reuses it
  return t < n_work - w.n_static ? w.n_static + t : -1;
}

// Forward prefill (optionally with fused RoPE).
struct FwdParams {
  const void* q;
  const void* k;
  const void* v;
  void* o;
  float* lse;  // may be null
  const float* q_cos;  // fused RoPE: [Sq, D] tables for Q (K arrives rotated)
  const float* q_sin;
  int B, Hq, Hkv, Sq, Sk, kv_len, g;
  float scale_log2;  // sm_scale * log2(e)
  int hpw;           // query heads per workgroup (1, 2 or 4; divides g)
  int rpw;           // query rows per head per workgroup (128 / hpw: 32 per wave)
  int n_qblk;        // ceil(Sq / rpw)
  int n_work;        // B * Hq / hpw * n_qblk
  int pair_group;    // > 0: (batch, kv head) pairs an XCD streams at a time (fwd_work_item)
  WorkTail tail;
};

// Work item of forward workgroup `bid`: (batch b, kv head kvh, head group hg
// of the GQA group, query block qblk). Workgroups are dispatched round-robin
// over the 8 XCDs (XCD = bid % 8), each with its own L2, and start on an XCD
// in bid order. Items are issued heavy (late, causal) query blocks first.
//  * When the (batch, kv head) pairs are a multiple of 8 and p.pair_group
//    (P) is set, each XCD owns pairs xcd, xcd + 8, ... and runs them P at a
//    time, the P pairs' items interleaved: the workgroups resident on an XCD
//    then stream P pairs' K/V, which the host sizes to fit its L2.
//  * Otherwise items run in (query block, batch, kv head, head group) order
//    with the head groups of one kv head on one XCD (xcd_remap).
// Both are bijections of [0, n_work).
__device__ inline void fwd_work_item(int bid, const FwdParams& p, int& b, int& kvh, int& hg, int& qblk) {
  const int n_hg = p.g / p.hpw;
  if (p.pair_group > 0) {
    const int per_pair = p.n_qblk * n_hg;
    const int P = p.pair_group;
    const int xcd = bid & 7, slot = bid >> 3;
    const int grp = slot / (P * per_pair), r = slot - grp * (P * per_pair);
    const int pair = (grp * P + r % P) * 8 + xcd;
    const int it = r / P;  // item within the pair
    hg = it % n_hg;
    qblk = p.n_qblk - 1 - it / n_hg;
    kvh = pair % p.Hkv;
    b = pair / p.Hkv;
    return;
  }
  const int w = xcd_remap(bid, p.n_work, n_hg);
  hg = w % n_hg;
  int rest = w / n_hg;
  kvh = rest % p.Hkv;
  rest /= p.Hkv;
  b = rest % p.B;
  qblk = p.n_qblk - 1 - rest / p.B;
}

hipError_t launch_attn_fwd(const FwdParams& p, int dtype, int head_dim, bool causal, bool rope,
                           hipStream_t stream);

// Rotate rows [0, kv_len) of every (batch, head) of a [B, H, Sk, D] tensor
// into k_out (same layout): x*cos + rotate_half(x)*sin with the [>= kv_len, D]
// float32 tables (row = position); inverse: x*cos - rotate_half(x)*sin.
hipError_t launch_rope_rotate_k(const void* k, void* k_out, const float* cos, const float* sin, int B,
                                int Hkv, int Sk, int kv_len, int dtype, int head_dim, hipStream_t stream,
                                bool inverse = false);

// Backward.
struct BwdParams {
  const void* q;
  const void* k;
  const void* v;
  const void* o;
  const void* dout;
  const float* lse;
  float* delta;
  void* dq;
  void* dk;
  void* dv;
  int B, Hq, Hkv, Sq, Sk, kv_len, g;
  float sm_scale;
  float scale_log2;
  WorkTail tail;  // of the dQ kernel (the dK/dV kernel runs without one)
};

// Work items of the dQ kernel (128 query rows of one head) and of the dK/dV
// kernel (128 keys of one kv head, all its query heads).
inline int bwd_dq_items(const BwdParams& p) { return p.B * p.Hq * ((p.Sq + 127) / 128); }
inline int bwd_dkv_items(const BwdParams& p) { return p.B * p.Hkv * ((p.Sk + 127) / 128); }

hipError_t launch_attn_bwd_delta(const BwdParams& p, int dtype, int head_dim, hipStream_t stream);
hipError_t launch_attn_bwd_dq(const BwdParams& p, int dtype, int head_dim, bool causal,
                              hipStream_t stream);
hipError_t launch_attn_bwd_dkv(const BwdParams& p, int dtype, int head_dim, bool causal,
                               hipStream_t stream);

// Split-KV single-query decode, contiguous cache or paged pool.
struct DecodeParams {
  const void* q;
  const void* k;  // contiguous cache base, or page pool base
  const void* v;
  void* o;
  const int32_t* block_tables;  // null for the contiguous cache
  const int32_t* context_lens;  // paged: [B] lengths; contiguous: null
  float* part_o;                // [B, Hq, n_split, D] partial (unnormalised) outputs
  float* part_ml;               // [B, Hq, n_split, 2] partial (max, sum)
  int B, Hq, Hkv, D;  // D: the compute head dim (64, 128 or, 16-bit, 256)
  // Stored head dim: the row length of q, the cache or pool and o (the
  // generic kernel reads rows of dr elements, dr <= D a multiple of one
  // 16-byte chunk, and treats columns [dr, D) as zeros; the streaming
  // kernel needs dr == D).
  int dr;
  int cache_size;     // contiguous: slots per (b, kvh); paged: unused
  int cache_len;      // contiguous: valid slots
  int num_pages, page_size, pages_per_seq;  // paged only
  int n_split;        // KV chunks per (b, kvh)
  int chunk;          // keys per chunk (multiple of 32)
  float scale_log2;
  int stages;         // streaming kernel: LDS ring depth (2..4)
  int n_waves;        // streaming kernel: persistent grid (one wave per workgroup)
  // Fused decode step (streaming kernel, positions != null): the new token of
  // batch b is at pos = positions[b * pos_stride]; its k (rotated with table
  // row pos) and v go to cache slot pos (ring: pos % cache_size) and it
  // attends pos + 1 (ring: min(pos + 1, cache_size)) slots; q is rotated with
  // row pos too. An invalid position (negative; linear: >= cache_size; past
  // rope_len with tables) attends nothing and writes nothing.
  const int32_t* positions;
  int pos_stride;
  int ring;
  const float* rope_cos;  // [rope_len, D] or null (no rotation)
  const float* rope_sin;
  int rope_len;
  const void* k_new;  // [B, Hkv, D]
  const void* v_new;
  void* k_out;        // the cache again, writable (= k, v)
  void* v_out;
};

// Split-KV partials + combine; picks the streaming kernel (decode_stream.hip)
// when decode_stream_supported() holds, else the generic one (decode.hip).
hipError_t launch_decode(const DecodeParams& p, int dtype, bool paged, hipStream_t stream);
hipError_t launch_decode_combine(const DecodeParams& p, int dtype, bool paged, hipStream_t stream);
bool decode_stream_supported(int dtype, int head_dim, bool paged, int page_size);
int decode_stream_waves(int stages, int group);  // resident one-wave workgroups on this device
int decode_stream_qrows(int group);               // query rows per partial slot
hipError_t launch_decode_stream(const DecodeParams& p, int dtype, bool paged, hipStream_t stream);

// Cache writes (cache_ops.hip). positions: device int32, read at
// b * pos_stride (pos_stride 0 = one position for the whole batch).
struct KvWriteParams {
  const void* k;  // [B, Hkv, L, D] rows to write
  const void* v;
  void* k_cache;  // [B, Hkv, C, D]
  void* v_cache;
  const int32_t* positions;
  int pos_stride;
  int B, Hkv, L, C;
  int ring;  // 0: slot pos + i; 1: slot (pos + i) % C, last C rows only
  int dr;    // row length in elements (the head_dim; whole 16-byte chunks)
};
hipError_t launch_kv_cache_write(const KvWriteParams& p, int dtype, int head_dim, hipStream_t stream);

struct PagedWriteParams {
  const void* k;  // [B, Hkv, L, D]
  const void* v;
  void* k_pages;  // [num_pages, Hkv, page_size, D]
  void* v_pages;
  const int32_t* block_tables;  // [B, pages_per_seq]
  const int32_t* positions;
  int pos_stride;
  int B, Hkv, L, num_pages, page_size, pages_per_seq;
  int dr;  // row length in elements (the head_dim; whole 16-byte chunks)
};
hipError_t launch_paged_cache_write(const PagedWriteParams& p, int dtype, int head_dim, hipStream_t stream);

}  // namespace pf
