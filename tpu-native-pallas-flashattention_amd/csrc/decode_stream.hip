// Streaming single-query decode for 16-bit K/V at head_dim 128 (gfx950).
//
// Replaces, for bf16/f16 caches with D = 128, the decode launch of
// `flash_attention_decode` (flash_attention.py:555-589: the forward
// pallas_call with block_q = 1, kv_len = cache_len) and the
// `paged_flash_attention` pallas_call (paged.py:151-192, kernel :45-99).
// Other dtypes / head dims use the generic kernel in decode.hip.
//
// The path is HBM-bound (about 4 FLOP per byte); the design keeps every CU's
// share of bytes in flight at all times with fully coalesced loads:
//  * Work list. A "sequence" is one (batch b, kv head, 16-head slice of the
//    GQA group); its keys [0, len_b) split into stages of 32 keys. All
//    sequences' stages, in order, form one global list of S stages. The grid
//    is persistent (as many one-wave workgroups as fit on the chip) and wave
//    w takes the contiguous range [start(w), start(w + 1)) of that list, an
//    equal share to within one stage whatever the (paged) lengths are.
//  * All query heads of a group ride as the N columns of 16x16x32 MFMAs, so
//    each K/V byte is read from HBM once (the reference grid runs per query
//    head and re-streams each KV head g times).
//  * K/V rows stream through a wave-private ring of NS LDS stages (8 KB of K
//    + 8 KB of V + the sequence's query rows). The ring runs across sequence
//    boundaries, so a wave never drains its pipeline until its range ends.
//    Each stage is 16 direct global->LDS loads (buffer_load_dwordx4 ... lds)
//    that each move 4 whole rows (1 KB contiguous in HBM). They are issued
//    from inline assembly, so the compiler does not insert its conservative
//    "wait for every LDS DMA" before each LDS read; explicit vmcnt waits
//    leave the NS - 2 younger stages in flight while a stage is consumed.
//  * Paged pool: each 4-row load lies inside one page (page_size % 4 == 0),
//    so its page is a wave-uniform scalar load of the block table and its
//    buffer resource spans exactly that page's valid rows.
//  * Rows at or past the valid length lie outside the load's buffer range
//    and arrive as zeros (hardware bounds check): a NaN tail, -1 table
//    padding (never looked up: lookups stop below ceil(len / page_size)) and
//    unused pages cannot leak (flash_attention.py:95-100; paged.py:73-80, :93).
//  * A sequence whose stages all fall in one wave is finished by that wave
//    (o = acc / l, l == 0 -> 0; flash_attention.py:150-159, paged.py:95-99).
//    A sequence cut by wave boundaries leaves one partial (max, sum, acc)
//    per piece in slot 2w (the piece that opens wave w's range) or 2w + 1
//    (the piece that closes it); pf_decode_stream_combine_kernel merges them.
//
// LDS stage layout: row-major 32 x 256 B tiles with the 16-byte chunks of row
// r permuted by chunk ^ sswz(r). Both read patterns are conflict-free:
//  * K as the A operand of S^T = K Q^T: the 16 lanes of a group read one
//    chunk index from 16 rows that differ in row bits {0, 1, 3, 4};
//  * V^T through ds_read_b64_tr_b16: a 16-lane group reads 2 chunks of 4
//    consecutive rows (row bits {0, 1} vary).
#include "pf_common.hpp"
#include "pf_kernels.hpp"

#include <mutex>

namespace pf {

namespace {

constexpr int kSK = 32;               // keys per stage
constexpr int kRowB = 256;            // bytes per K/V row (128 16-bit elements)
constexpr int kTileB = kSK * kRowB;   // 8 KB: one stage of K (or V)
// K/V stages are loaded non-temporal: each cache or pool byte is read once
// per call, and a read-once stream reaches a higher HBM rate that way
// (bench.py's read-form probe).
constexpr bool kKvNt = true;

typedef short i16x4 __attribute__((ext_vector_type(4)));

__device__ inline int sswz(int r) { return ((r >> 3) & 1) | ((r & 3) << 1) | (((r >> 4) & 1) << 3); }

// Wait for the oldest issued stage; `younger` later stages (at least 16
// loads each, loads complete in issue order) may stay in flight.
template <int NS>
__device__ inline void wait_stage(int64_t younger) {
  if constexpr (NS >= 4) {
    if (younger >= 2) { wait_vm<32>(); return; }
  }
  if constexpr (NS >= 3) {
    if (younger >= 1) { wait_vm<16>(); return; }
  }
  wait_vm<0>();
}

__device__ inline int uni(int x) { return __builtin_amdgcn_readfirstlane(x); }
__device__ inline int64_t uni64(int64_t x) {
  const uint32_t lo = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)x);
  const uint32_t hi = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)((uint64_t)x >> 32));
  return (int64_t)(((uint64_t)hi << 32) | lo);
}

// Scalar (wave-uniform) 32-bit load through the constant address space; the
// index is made provably uniform so the compiler emits s_load (the scalar
// counter), not a vector load whose wait would drain the LDS DMA queue.
__device__ inline int sload_i32(const int32_t* p, int64_t idx) {
  const __attribute__((address_space(4))) int32_t* cp = (const __attribute__((address_space(4))) int32_t*)p;
  return uni(cp[uni64(idx)]);
}

template <typename T>
struct Mfma16;
template <>
struct Mfma16<bf16_t> {
  typedef bf16x8 Frag;
  __device__ static inline f32x4 run(Frag a, Frag b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
  }
};
template <>
struct Mfma16<f16_t> {
  typedef f16x8 Frag;
  __device__ static inline f32x4 run(Frag a, Frag b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
  }
};

// Live keys of a decode step whose new token is at `pos` (0 for an invalid
// position: it attends nothing and writes nothing): linear cache pos + 1,
// ring min(pos + 1, cache_size) (model.py:475-476).
__device__ inline int step_len(const DecodeParams& p, int pos) {
  const bool valid = pos >= 0 && (p.ring != 0 || pos < p.cache_size) &&
                     (p.rope_cos == nullptr || pos < p.rope_len);
  if (!valid) return 0;
  return p.ring != 0 ? min(pos + 1, p.cache_size) : pos + 1;
}

// Valid keys of batch b: PG == 0 the one cache_len; PG == 1 (decode step)
// from b's position; paged: b's context length clamped to the table's reach.
// len_lane reads per lane (b may differ across lanes), seq_len with scalar
// loads (b wave-uniform).
template <int PG>
__device__ inline int len_lane(const DecodeParams& p, int b) {
  if constexpr (PG == 0) {
    return p.cache_len;
  } else if constexpr (PG == 1) {
    return step_len(p, p.positions[(int64_t)b * p.pos_stride]);
  } else {
    return min(max(p.context_lens[b], 0), p.pages_per_seq * p.page_size);
  }
}
template <int PG>
__device__ inline int seq_len(const DecodeParams& p, int b) {
  if constexpr (PG == 0) {
    return p.cache_len;
  } else if constexpr (PG == 1) {
    return step_len(p, sload_i32(p.positions, (int64_t)b * p.pos_stride));
  } else {
    return min(max(sload_i32(p.context_lens, b), 0), p.pages_per_seq * p.page_size);
  }
}

// Balanced partition of the S-stage list over the waves.
__device__ inline int64_t wave_start(int64_t S, int W, int w) {
  const int64_t q = S / W, rem = S % W;
  return (int64_t)w * q + min((int64_t)w, rem);
}
__device__ inline int wave_of(int64_t S, int W, int64_t s) {
  const int64_t q = S / W, rem = S % W;
  if (s < rem * (q + 1)) return (int)(s / (q + 1));
  return (int)(rem + (s - rem * (q + 1)) / q);
}

// Position in the stage list: batch b, sequence j = kv_head * n_hc + slice
// within the batch, stage st of nst = ceil(L / 32).
struct Cursor {
  int b, j, st, nst, L;
};

template <int PG>
__device__ inline void cursor_next(Cursor& c, const DecodeParams& p, int J) {
  if (++c.st < c.nst) return;
  c.st = 0;
  if (++c.j < J) return;
  c.j = 0;
  do {
    ++c.b;
    c.L = (c.b < p.B) ? seq_len<PG>(p, c.b) : 0;
  } while (c.b < p.B && c.L == 0);
  c.nst = (c.L + kSK - 1) / kSK;
}

// Stage totals: per batch b, T_b = ceil(L_b / 32) * J stages. With s < 0
// returns the total S; otherwise also fills *out with the cursor of global
// stage s (which must be < S).
template <int PG>
__device__ inline int64_t locate(const DecodeParams& p, int J, int64_t s, Cursor* out) {
  const int lane = threadIdx.x & 63;
  if constexpr (PG == 0) {
    const int nst = (p.cache_len + kSK - 1) / kSK;
    const int64_t per_b = (int64_t)nst * J;
    if (s >= 0) {
      const int64_t r = s % per_b;
      *out = Cursor{uni((int)(s / per_b)), uni((int)(r / nst)), uni((int)(r % nst)), uni(nst), uni(p.cache_len)};
    }
    return uni64(per_b * p.B);
  } else {
    int64_t base = 0;
    for (int b0 = 0; b0 < p.B; b0 += 64) {
      const int bb = b0 + lane;
      const int Lb = bb < p.B ? len_lane<PG>(p, bb) : 0;
      const int64_t t = (int64_t)((Lb + kSK - 1) / kSK) * J;
      int64_t incl = t;  // inclusive scan over the 64 lanes
#pragma unroll
      for (int o = 1; o < 64; o <<= 1) {
        const int64_t y = __shfl_up(incl, o);
        if (lane >= o) incl += y;
      }
      const int64_t tot = __shfl(incl, 63);
      if (s >= base && s < base + tot) {
        const uint64_t hit = __ballot(base + incl > s);
        const int ln = __builtin_ctzll(hit);
        const int64_t excl = __shfl(incl - t, ln);
        const int Lh = __shfl(Lb, ln);
        const int nst = (Lh + kSK - 1) / kSK;
        const int64_t r = s - base - excl;
        *out = Cursor{uni(b0 + ln), uni((int)(r / nst)), uni((int)(r % nst)), uni(nst), uni(Lh)};
        return -1;  // found (the total is not needed after the search)
      }
      base += tot;
    }
    return uni64(base);
  }
}

// With at most 64 batches one load of the per-batch lengths (a lane per
// batch) gives everything both kernels need: lane bb's stage count T_bb =
// ceil(L_bb / 32) * J, their inclusive scan `incl` and the total S. (More
// batches take the looped scans of locate.)
struct Lens64 {
  int L;         // this lane's batch length (0 past B)
  int64_t t;     // its stage count
  int64_t incl;  // stage counts of batches <= this lane's, summed
  int64_t tot;   // S, the total
};
template <int PG>
__device__ inline Lens64 lens64(const DecodeParams& p, int J) {
  const int lane = threadIdx.x & 63;
  Lens64 r;
  r.L = lane < p.B ? len_lane<PG>(p, lane) : 0;
  r.t = (int64_t)((r.L + kSK - 1) / kSK) * J;
  r.incl = r.t;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const int64_t y = __shfl_up(r.incl, o);
    if (lane >= o) r.incl += y;
  }
  r.tot = uni64(__shfl(r.incl, 63));
  return r;
}

// The stages of wave w of W: their count (returned) and, if any, the cursor
// of the first one.
template <int PG>
__device__ inline int64_t wave_plan(const DecodeParams& p, int J, int W, int w, Cursor* cc) {
  if (PG != 0 && p.B <= 64) {
    const Lens64 ls = lens64<PG>(p, J);
    const int64_t s0 = wave_start(ls.tot, W, w);
    const int64_t n = wave_start(ls.tot, W, w + 1) - s0;
    if (n > 0) {
      const uint64_t hit = __ballot(ls.incl > s0);
      const int ln = __builtin_ctzll(hit);
      const int64_t excl = __shfl(ls.incl - ls.t, ln);
      const int Lh = __shfl(ls.L, ln);
      const int nst = (Lh + kSK - 1) / kSK;
      const int64_t r = s0 - excl;
      *cc = Cursor{uni(ln), uni((int)(r / nst)), uni((int)(r % nst)), uni(nst), uni(Lh)};
    }
    return n;
  }
  const int64_t S = locate<PG>(p, J, -1, cc);
  const int64_t s0 = wave_start(S, W, w);
  const int64_t n = wave_start(S, W, w + 1) - s0;
  if (n > 0) locate<PG>(p, J, s0, cc);
  return n;
}

// PG: 0 = contiguous cache, one length (cache_len) for every batch; 1 = the
// fused decode step (contiguous cache, per-batch positions in device memory,
// see below); 32 = paged with page_size % 32 == 0 (one page per stage); 4 =
// paged with page_size % 4 == 0 (one page per 4-row load).
// QR: query rows staged per sequence (4 when the group has <= 4 heads, else 16).
//
// Decode step (PG == 1; model.py:340-347, :475-491): batch b's new token sits
// at pos = positions[b * pos_stride], its slot is pos (ring: pos % C) and the
// sequence is slots [0, step_len). At the start of each piece the wave reads
// pos, rotates its query fragments with table row pos (rotate-half, float32,
// rounded once to T: model.py:54-67) and prepares the new K row (rotated the
// same way) and V row in registers. The stage holding the slot is patched in
// LDS with those rows after its DMA lands -- the cache still holds the old
// slot contents, and no other stage holds that row -- and the wave that owns
// head slice 0 writes them to the cache slot. Every wave that reads the slot
// (one per head slice) patches its own copy, so no wave depends on another's
// global write within the launch.
template <typename T, int PG, int NS, int QR>
__global__ __launch_bounds__(64) void pf_decode_stream_kernel(DecodeParams p) {
  using MF = Mfma16<T>;
  using Frag = typename MF::Frag;
  constexpr int kQB = QR * kRowB;
  constexpr int kSlotB = 2 * kTileB + kQB;  // K, V, query rows
  __shared__ __attribute__((aligned(1024))) char smem[NS * kSlotB];

  const int lane = threadIdx.x;
  const int i16 = lane & 15;
  const int h = lane >> 4;
  const int g = p.Hq / p.Hkv;
  const int n_hc = (g + 15) >> 4;
  const int J = p.Hkv * n_hc;
  const int W = p.n_waves;
  const int w = blockIdx.x;

  Cursor cc;
  const int64_t n = wave_plan<PG>(p, J, W, w, &cc);  // stages of this wave
  if (n <= 0) return;

  const uint32_t lds0 = lds_u32(smem);
  const T* Kb = static_cast<const T*>(p.k);
  const T* Vb = static_cast<const T*>(p.v);
  const T* Qb = static_cast<const T*>(p.q);

  // Per-lane byte offset (within a 32-row stage) of the chunk this lane
  // fetches for load i of a tile: row 4i + lane/16, physical slot lane%16.
  uint32_t loff[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int row = 4 * i + h;
    loff[i] = (uint32_t)(row * kRowB + 16 * (i16 ^ sswz(row)));
  }

  // Issue the loads of the stage under cursor c into ring slot `slot`; with
  // `with_q`, first the query rows of c's head slice (rows past the group
  // arrive as zeros).
  auto issue = [&](const Cursor& c, int slot, bool with_q) {
    const uint32_t ldk = lds0 + (uint32_t)(slot * kSlotB);
    const uint32_t ldv = ldk + kTileB;
    const int kvh = c.j / n_hc, hc = c.j - kvh * n_hc;
    if (with_q) {
      const int q0 = hc * 16;
      const int nq = min(QR, g - q0);
      const i32x4 dq = make_desc(Qb + ((int64_t)c.b * p.Hq + (int64_t)kvh * g + q0) * 128,
                                 (uint32_t)(nq * kRowB));
#pragma unroll
      for (int i = 0; i < QR / 4; ++i) {
        const int row = 4 * i + h;
        dma16(dq, (uint32_t)(row * kRowB + 16 * (i16 ^ (row & 15))), ldv + kTileB + 1024 * i);
      }
    }
    const int kv0 = c.st * kSK;
    if constexpr (PG == 0 || PG == 1) {
      const int64_t seq = ((int64_t)c.b * p.Hkv + kvh) * (int64_t)p.cache_size * 128;
      const i32x4 dk = make_desc(Kb + seq, (uint32_t)c.L * kRowB);
      const i32x4 dv = make_desc(Vb + seq, (uint32_t)c.L * kRowB);
      const uint32_t rb = (uint32_t)kv0 * kRowB;
#pragma unroll
      for (int i = 0; i < 8; ++i) dma16<kKvNt>(dk, rb + loff[i], ldk + 1024 * i);
#pragma unroll
      for (int i = 0; i < 8; ++i) dma16<kKvNt>(dv, rb + loff[i], ldv + 1024 * i);
    } else {
      const int ps = p.page_size;
      const int64_t trow = (int64_t)c.b * p.pages_per_seq;
      constexpr int kGroups = (PG == 32) ? 1 : 8;  // page-uniform groups per stage
      constexpr int kPer = 8 / kGroups;
#pragma unroll
      for (int gi = 0; gi < kGroups; ++gi) {
        const int key0 = kv0 + gi * (kSK / kGroups);
        // Groups at or past L load nothing (zero range) and look nothing up:
        // table entries at logical pages >= ceil(L / page_size) may be -1 or
        // lie past the table row.
        const bool live = key0 < c.L;
        const int lp = live ? key0 / ps : 0;
        int page = live ? sload_i32(p.block_tables, trow + lp) : 0;
        page = min(max(page, 0), p.num_pages - 1);
        const int prow0 = live ? lp * ps : key0;
        const int nvalid = live ? min(ps, c.L - prow0) : 0;
        const int64_t pbase = ((int64_t)page * p.Hkv + kvh) * (int64_t)ps * 128;
        const i32x4 dk = make_desc(Kb + pbase, (uint32_t)(nvalid * kRowB));
        const i32x4 dv = make_desc(Vb + pbase, (uint32_t)(nvalid * kRowB));
        const uint32_t rb = (uint32_t)(kv0 - prow0) * kRowB;
#pragma unroll
        for (int j = 0; j < kPer; ++j) dma16<kKvNt>(dk, rb + loff[gi * kPer + j], ldk + 1024 * (gi * kPer + j));
#pragma unroll
        for (int j = 0; j < kPer; ++j) dma16<kKvNt>(dv, rb + loff[gi * kPer + j], ldv + 1024 * (gi * kPer + j));
      }
    }
  };

  // ---- decode step (PG == 1) --------------------------------------------
  // Per piece: the token's position, this lane's chunk of the new K row
  // (lanes 0-15, chunk i16, and its rotate-half partner i16 ^ 8) or V row
  // (lanes 16-31), and the table values the lane's rotations use (K: elements
  // 8 i16 .. +7; Q: 32 s + 8 h .. +7 for s = 0..3).
  struct StepData {
    int pos;
    u32x4 kv, kvp;
    f32x4 kc[2], ks[2];
    f32x4 qc[4][2], qs[4][2];
  };
  [[maybe_unused]] auto step_load = [&](const Cursor& c, StepData& d) {
    d.pos = sload_i32(p.positions, (int64_t)c.b * p.pos_stride);  // valid: the piece has keys
    const int kvh = c.j / n_hc;
    const int64_t src = ((int64_t)c.b * p.Hkv + kvh) * 128;
    if (lane < 32) {
      const T* nb = static_cast<const T*>(lane < 16 ? p.k_new : p.v_new) + src;
      d.kv = ldg16(nb + 8 * i16);
      d.kvp = ldg16(nb + 8 * (i16 ^ 8));
    }
    if (p.rope_cos != nullptr) {
      const float* cr = p.rope_cos + (int64_t)d.pos * 128;
      const float* sr = p.rope_sin + (int64_t)d.pos * 128;
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        d.kc[u] = *reinterpret_cast<const f32x4*>(cr + 8 * i16 + 4 * u);
        d.ks[u] = *reinterpret_cast<const f32x4*>(sr + 8 * i16 + 4 * u);
#pragma unroll
        for (int s4 = 0; s4 < 4; ++s4) {
          d.qc[s4][u] = *reinterpret_cast<const f32x4*>(cr + 32 * s4 + 8 * h + 4 * u);
          d.qs[s4][u] = *reinterpret_cast<const f32x4*>(sr + 32 * s4 + 8 * h + 4 * u);
        }
      }
    }
  };
  // Rotate-half RoPE of 8 consecutive elements d0 .. d0 + 7 of a 128-element
  // row whose partner elements (d +- 64) are in xp, with those elements'
  // table values: y = x cos - x' sin (first half), x cos + x' sin (second
  // half), float32, rounded once to T (model.py:54-67; fused_rope.py:43-50).
  auto rope8 = [&](const u32x4& x, const u32x4& xp, const f32x4* c, const f32x4* sn, bool first_half) -> u32x4 {
    float a[8], b2[8], y[8];
    chunk_to_f32<T>(x, a);
    chunk_to_f32<T>(xp, b2);
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float ce = c[e >> 2][e & 3], se = sn[e >> 2][e & 3];
      y[e] = first_half ? a[e] * ce - b2[e] * se : a[e] * ce + b2[e] * se;
    }
    return f32_to_chunk<T>(y);
  };
  // New piece: the token's slot, the rotated query fragments (lane holds
  // Q[head i16][32 s + 8 h + e]; the partner of s is s ^ 2) and this lane's
  // new K (rotated) or V row chunk.
  [[maybe_unused]] auto step_apply = [&](const StepData& d, Frag* q4, int& tslot, u32x4& row) {
    tslot = p.ring != 0 ? d.pos % p.cache_size : d.pos;
    row = d.kv;
    if (p.rope_cos != nullptr) {
      if (lane < 16) row = rope8(d.kv, d.kvp, d.kc, d.ks, i16 < 8);
      u32x4 qx[4];
#pragma unroll
      for (int s4 = 0; s4 < 4; ++s4) qx[s4] = __builtin_bit_cast(u32x4, q4[s4]);
#pragma unroll
      for (int s4 = 0; s4 < 4; ++s4)
        q4[s4] = __builtin_bit_cast(Frag, rope8(qx[s4], qx[s4 ^ 2], d.qc[s4], d.qs[s4], s4 < 2));
    }
  };
  // Stage holding the token's slot at row r: overwrite that row of the K and
  // V tiles (after the stage's DMA landed), and write it to the cache once
  // (head slice 0).
  [[maybe_unused]] auto step_patch = [&](const Cursor& c, char* tK, char* tV, int r, int tslot, const u32x4& row) {
    if (lane < 32) {
      char* t = lane < 16 ? tK : tV;
      sts16(t + r * kRowB + 16 * (i16 ^ sswz(r)), row);
      const int kvh = c.j / n_hc, hc = c.j - kvh * n_hc;
      if (hc == 0) {
        T* out = static_cast<T*>(lane < 16 ? p.k_out : p.v_out);
        stg16(out + (((int64_t)c.b * p.Hkv + kvh) * p.cache_size + tslot) * 128 + 8 * i16, row);
      }
    }
    // this wave's LDS accesses run in order; keep the compiler from moving
    // the tile reads above the stores
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  };

  [[maybe_unused]] StepData pend;  // NS == 2: the step data of the piece the next stage opens

  // Prologue: the first NS - 1 stages.
  Cursor pc = cc;
#pragma unroll
  for (int k = 0; k < NS - 1; ++k) {
    if (k < n) {
      issue(pc, k, k == 0 || pc.st == 0);
      if constexpr (PG == 1 && NS == 2) step_load(pc, pend);  // stage 0 opens a piece
      cursor_next<PG>(pc, p, J);
    }
  }

  // Per-lane LDS read offsets.
  // K (A operand, tile u, d step s): key row 8(i16/4) + 4u + i16%4, chunk 4s + h.
  uint32_t koff[2][4];
#pragma unroll
  for (int u = 0; u < 2; ++u) {
    const int row = 8 * (i16 >> 2) + 4 * u + (i16 & 3);
#pragma unroll
    for (int s = 0; s < 4; ++s) koff[u][s] = (uint32_t)(row * kRowB + 16 * ((4 * s + h) ^ sswz(row)));
  }
  // V^T (A operand via transposing reads, d tile dt, key half e): the lane
  // addresses row 8h + 4e + i16/4, columns 16dt + 4(i16%4) .. +3.
  uint32_t voff[8][2];
#pragma unroll
  for (int e = 0; e < 2; ++e) {
    const int row = 8 * h + 4 * e + (i16 >> 2);
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) {
      const int chunk = 2 * dt + ((i16 >> 1) & 1);
      voff[dt][e] = (uint32_t)(row * kRowB + 16 * (chunk ^ sswz(row)) + 8 * (i16 & 1));
    }
  }

  Frag qf[4];
  f32x4 acc[8];
  float m_run = kNegInf, l_run = 0.f;
  int piece_st0 = 0;       // first stage (within the sequence) of the current piece
  bool first_piece = true;  // the current piece opens this wave's range
  // Decode step: the current piece's token slot and its new K (lanes 0-15,
  // 16-byte chunk i16) / V (lanes 16-31) row chunk.
  [[maybe_unused]] int tok_slot = -1;
  [[maybe_unused]] u32x4 new_row = (u32x4){0u, 0u, 0u, 0u};

  for (int64_t k = 0; k < n; ++k) {
    wait_stage<NS>(min((int64_t)(NS - 2), n - 1 - k));
    const int slot = (int)(k % NS);
    char* const sK = smem + slot * kSlotB;
    char* const sV = sK + kTileB;
    if (k == 0 || cc.st == 0) {
      // New piece: query fragments (B operand of S^T: lane holds
      // Q[head i16][d = 32 s + 8 h + 0..7]) and a fresh softmax state.
      const char* sQ = sV + kTileB;
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        const u32x4 x = (i16 < QR) ? lds16(sQ + i16 * kRowB + 16 * ((4 * s + h) ^ i16)) : (u32x4){0u, 0u, 0u, 0u};
        qf[s] = __builtin_bit_cast(Frag, x);
      }
      if constexpr (PG == 1) {
        if constexpr (NS == 2) {
          step_apply(pend, qf, tok_slot, new_row);  // loaded with the stage's DMA
        } else {
          StepData d;
          step_load(cc, d);
          step_apply(d, qf, tok_slot, new_row);
        }
      }
#pragma unroll
      for (int dt = 0; dt < 8; ++dt) acc[dt] = (f32x4)(0.f);
      m_run = kNegInf;
      l_run = 0.f;
      piece_st0 = cc.st;
    }
    if constexpr (PG == 1) {
      // the stage holding the new token's slot: its row comes from registers
      const int r = tok_slot - cc.st * kSK;
      if (r >= 0 && r < kSK) step_patch(cc, sK, sV, r, tok_slot, new_row);
    }
    if (k + NS - 1 < n) {
      issue(pc, (int)((k + NS - 1) % NS), pc.st == 0);
      if constexpr (PG == 1 && NS == 2) {
        // the next stage opens a piece: its step data arrive with its tiles
        if (pc.st == 0) step_load(pc, pend);
      }
      cursor_next<PG>(pc, p, J);
    }

    const int kv0 = cc.st * kSK;
    // S^T (32 keys x 16 heads): lane holds keys kv0 + 8h + 4u + r, head i16.
    f32x4 s[2] = {(f32x4)(0.f), (f32x4)(0.f)};
#pragma unroll
    for (int st = 0; st < 4; ++st)
#pragma unroll
      for (int u = 0; u < 2; ++u)
        s[u] = MF::run(__builtin_bit_cast(Frag, lds16(sK + koff[u][st])), qf[st], s[u]);

    float x[8];
    float mx = kNegInf;
#pragma unroll
    for (int t = 0; t < 8; ++t) {
      const int key = kv0 + 8 * h + t;
      x[t] = key < cc.L ? s[t >> 2][t & 3] * p.scale_log2 : kNegInf;
      mx = fmaxf(mx, x[t]);
    }
    mx = fmaxf(mx, __shfl_xor(mx, 16));
    mx = fmaxf(mx, __shfl_xor(mx, 32));
    const float m_new = fmaxf(m_run, mx);
    const float m_use = (m_new == kNegInf) ? 0.f : m_new;
    const float alpha = exp2f(m_run - m_use);
    float rs = 0.f;
    Frag pf;
#pragma unroll
    for (int t = 0; t < 8; ++t) {
      const float e = exp2f(x[t] - m_use);
      rs += e;
      pf[t] = Elem<T>::from_f32(e);
    }
    l_run = l_run * alpha + rs;
    m_run = m_new;

    // O^T (128 d x 16 heads) += V^T . P^T
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) {
      const i16x4 v0 = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
          (__attribute__((address_space(3))) i16x4*)(sV + voff[dt][0]));
      const i16x4 v1 = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
          (__attribute__((address_space(3))) i16x4*)(sV + voff[dt][1]));
      const Frag a = __builtin_bit_cast(Frag, __builtin_shufflevector(v0, v1, 0, 1, 2, 3, 4, 5, 6, 7));
      acc[dt] = MF::run(a, pf, acc[dt] * alpha);
    }

    if (cc.st == cc.nst - 1 || k == n - 1) {
      // ---- end of a piece ---------------------------------------------------
      float l_tot = l_run + __shfl_xor(l_run, 16);
      l_tot += __shfl_xor(l_tot, 32);
      const int kvh = cc.j / n_hc, hc = cc.j - kvh * n_hc;
      const int qh = hc * 16 + i16;
      if (piece_st0 == 0 && cc.st == cc.nst - 1) {
        // The whole sequence: finish it here.
        if (qh < g) {
          const float inv = (l_tot == 0.f) ? 0.f : 1.f / l_tot;
          T* out = static_cast<T*>(p.o) + ((int64_t)cc.b * p.Hq + (int64_t)kvh * g + qh) * 128;
#pragma unroll
          for (int dt = 0; dt < 8; ++dt) {
            typedef T v4 __attribute__((ext_vector_type(4)));
            v4 y;
#pragma unroll
            for (int r = 0; r < 4; ++r) y[r] = Elem<T>::from_f32(acc[dt][r] * inv);
            *reinterpret_cast<v4*>(out + 16 * dt + 4 * h) = y;
          }
        }
      } else if (i16 < QR) {
        const int64_t pslot = 2 * (int64_t)w + (first_piece ? 0 : 1);
        float* po = p.part_o + (pslot * QR + i16) * 128;
#pragma unroll
        for (int dt = 0; dt < 8; ++dt) *reinterpret_cast<f32x4*>(po + 16 * dt + 4 * h) = acc[dt];
        if (h == 0) {
          p.part_ml[(pslot * QR + i16) * 2 + 0] = m_run;
          p.part_ml[(pslot * QR + i16) * 2 + 1] = l_tot;
        }
      }
      first_piece = false;
    }
    cursor_next<PG>(cc, p, J);
  }
}

// Merge the partial pieces of each (b, h) whose sequence was cut by wave
// boundaries: o = sum_i acc_i 2^(m_i - M) / sum_i l_i 2^(m_i - M); a batch
// with no valid key gives o = 0 (flash_attention.py:150-159; paged.py:95-99).
// Sequences that one wave covered were written by the main kernel.
template <typename T, int PG, int QR>
__global__ __launch_bounds__(256) void pf_decode_stream_combine_kernel(DecodeParams p) {
  const int lane = threadIdx.x & 63;
  const int bh = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (bh >= p.B * p.Hq) return;
  const int b = bh / p.Hq, hq = bh - b * p.Hq;
  const int g = p.Hq / p.Hkv;
  const int n_hc = (g + 15) >> 4;
  const int J = p.Hkv * n_hc;
  const int kvh = hq / g, qh = hq - kvh * g, hc = qh >> 4, qi = qh & 15;
  const int W = p.n_waves;

  // Global stage range [s0, s1) of this head's sequence.
  int64_t S, before = 0;  // all stages; stages of batches < b
  int L;
  if constexpr (PG == 0) {
    Cursor dummy;
    S = locate<PG>(p, J, -1, &dummy);
    L = p.cache_len;
    before = (int64_t)b * ((L + kSK - 1) / kSK) * J;
  } else if (p.B <= 64) {
    const Lens64 ls = lens64<PG>(p, J);
    S = ls.tot;
    before = uni64(__shfl(ls.incl - ls.t, b));
    L = __builtin_amdgcn_readfirstlane(__shfl(ls.L, b));
  } else {
    Cursor dummy;
    S = locate<PG>(p, J, -1, &dummy);
    for (int b0 = 0; b0 < b; b0 += 64) {
      const int bb = b0 + lane;
      const int Lb = bb < b ? len_lane<PG>(p, bb) : 0;
      int64_t t = (int64_t)((Lb + kSK - 1) / kSK) * J;
#pragma unroll
      for (int o = 32; o > 0; o >>= 1) t += __shfl_xor(t, o);
      before += t;
    }
    L = len_lane<PG>(p, b);
  }
  const int nst = (L + kSK - 1) / kSK;
  T* out = static_cast<T*>(p.o) + (int64_t)bh * 128 + 2 * lane;
  if (nst == 0) {
    out[0] = Elem<T>::from_f32(0.f);
    out[1] = Elem<T>::from_f32(0.f);
    return;
  }
  const int64_t s0 = before + (int64_t)(kvh * n_hc + hc) * nst, s1 = s0 + nst;
  const int wa = wave_of(S, W, s0), wb = wave_of(S, W, s1 - 1);
  if (wa == wb) return;  // finished by the main kernel

  float M = kNegInf;
  for (int w = wa; w <= wb; ++w) {
    const int64_t slot = 2 * (int64_t)w + (wave_start(S, W, w) < s0 ? 1 : 0);
    M = fmaxf(M, p.part_ml[(slot * QR + qi) * 2]);
  }
  const float Mu = (M == kNegInf) ? 0.f : M;
  float o0 = 0.f, o1 = 0.f, lsum = 0.f;
  for (int w = wa; w <= wb; ++w) {
    const int64_t slot = 2 * (int64_t)w + (wave_start(S, W, w) < s0 ? 1 : 0);
    const float wt = exp2f(p.part_ml[(slot * QR + qi) * 2] - Mu);
    lsum += p.part_ml[(slot * QR + qi) * 2 + 1] * wt;
    const f32x2 v = *reinterpret_cast<const f32x2*>(p.part_o + (slot * QR + qi) * 128 + 2 * lane);
    o0 += v[0] * wt;
    o1 += v[1] * wt;
  }
  const float inv = (lsum == 0.f) ? 0.f : 1.f / lsum;
  out[0] = Elem<T>::from_f32(o0 * inv);
  out[1] = Elem<T>::from_f32(o1 * inv);
}

template <typename T, int PG, int NS, int QR>
hipError_t launch_stream(const DecodeParams& p, hipStream_t st) {
  hipLaunchKernelGGL((pf_decode_stream_kernel<T, PG, NS, QR>), dim3((unsigned)p.n_waves), dim3(64), 0, st, p);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  const int64_t n_bh = (int64_t)p.B * p.Hq;
  hipLaunchKernelGGL((pf_decode_stream_combine_kernel<T, PG, QR>), dim3((unsigned)((n_bh + 3) / 4)), dim3(256),
                     0, st, p);
  return hipGetLastError();
}

template <typename T, int PG, int QR>
hipError_t launch_ns(const DecodeParams& p, hipStream_t st) {
  switch (p.stages) {
    case 3: return launch_stream<T, PG, 3, QR>(p, st);
    case 4: return launch_stream<T, PG, 4, QR>(p, st);
    default: return launch_stream<T, PG, 2, QR>(p, st);
  }
}

template <typename T, int PG>
hipError_t launch_qr(const DecodeParams& p, hipStream_t st) {
  return (p.Hq / p.Hkv <= 4) ? launch_ns<T, PG, 4>(p, st) : launch_ns<T, PG, 16>(p, st);
}

template <typename T>
hipError_t launch_pg(const DecodeParams& p, bool paged, hipStream_t st) {
  if (!paged) return p.positions != nullptr ? launch_qr<T, 1>(p, st) : launch_qr<T, 0>(p, st);
  if (p.page_size % 32 == 0) return launch_qr<T, 32>(p, st);
  return launch_qr<T, 4>(p, st);
}

template <int NS, int QR>
int blocks_per_cu() {
  int n = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, pf_decode_stream_kernel<bf16_t, 0, NS, QR>, 64, 0) !=
      hipSuccess)
    return 0;
  return n;
}

}  // namespace

bool decode_stream_supported(int dtype, int head_dim, bool paged, int page_size) {
  if (head_dim != 128 || (dtype != kBF16 && dtype != kF16)) return false;
  return !paged || (page_size % 4 == 0);
}

// Resident one-wave workgroups of the streaming kernel on the current device
// (the persistent grid size). The device's CU count and the kernel's
// occupancy for every (stages, query rows) variant are queried once per
// device (std::call_once) and cached; later calls cost one hipGetDevice.
// Without a usable device (a host-only query), MI355X's 256 CUs and the
// LDS-limited occupancy are assumed.
namespace {

constexpr int kMaxDevices = 64;

struct StreamOccupancy {
  std::once_flag once;
  int cus = 0;
  int per_cu[3][2] = {};  // [stages - 2][query rows 4 / 16]
};
StreamOccupancy g_occupancy[kMaxDevices];

void query_occupancy(StreamOccupancy* o, int dev) {
  int cus = 0;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0) return;
  o->cus = cus;
  o->per_cu[0][0] = blocks_per_cu<2, 4>();
  o->per_cu[0][1] = blocks_per_cu<2, 16>();
  o->per_cu[1][0] = blocks_per_cu<3, 4>();
  o->per_cu[1][1] = blocks_per_cu<3, 16>();
  o->per_cu[2][0] = blocks_per_cu<4, 4>();
  o->per_cu[2][1] = blocks_per_cu<4, 16>();
}

}  // namespace

int decode_stream_waves(int stages, int group) {
  const bool small = group <= 4;
  const int si = (stages >= 2 && stages <= 4) ? stages - 2 : 0;
  int per_cu = 0, cus = 0;
  int dev = 0;
  if (hipGetDevice(&dev) == hipSuccess && dev >= 0 && dev < kMaxDevices) {
    StreamOccupancy& o = g_occupancy[dev];
    std::call_once(o.once, query_occupancy, &o, dev);
    cus = o.cus;
    per_cu = o.per_cu[si][small ? 0 : 1];
  }
  if (cus <= 0) cus = 256;
  if (per_cu <= 0) {
    const int lds = (si + 2) * (2 * kTileB + (small ? 4 : 16) * kRowB);
    per_cu = 160 * 1024 / lds;
  }
  return cus * max(per_cu, 1);
}

int decode_stream_qrows(int group) { return group <= 4 ? 4 : 16; }

hipError_t launch_decode_stream(const DecodeParams& p, int dtype, bool paged, hipStream_t stream) {
  return (dtype == kBF16) ? launch_pg<bf16_t>(p, paged, stream) : launch_pg<f16_t>(p, paged, stream);
}

}  // namespace pf
