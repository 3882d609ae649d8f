// LDS tiles shared by the prefill-shaped kernels (forward, dQ, dK/dV).
//
// A tile is 64 consecutive rows of a row-major [rows, D] matrix of T, staged
// in LDS unpadded (row pitch D*sizeof(T)), with each row's 16-byte chunks
// XOR-swizzled by tile_swz(row). Two MFMA operand reads come out of the same
// copy:
//  * "natural" A operand (contraction over D): MFMA row R = lane%32 of 32-row
//    tile t reads tile row mfma_src_row(R, t), so that in the result lane half
//    hh's accumulator register reg holds tile row 32hh + 16t + reg -- exactly
//    the reduction slots that the next MFMA's B operand needs from that lane;
//  * "transposed" A operand (contraction over the 64 tile rows): for 16-bit T
//    the gfx950 transposing LDS load ds_read_b64_tr_b16 (within each 16-lane
//    group, lane i receives element [4t + i/4][i%4] of the 16 x 4 block the
//    group addressed; lane j pointing at row k0 + j/4, column d0 + 4(j%4)
//    hands lane i the values [k0 + t][d0 + i]); for float32, scalar reads.
// The swizzle makes both read kinds and the staging writes conflict-free:
// the 16 lanes of a natural read hit 16 distinct chunks, and a transposed read
// (4 consecutive rows x 4 consecutive chunks) hits 16 distinct chunks.
// Rows at or past a limit are loaded as zeros by the buffer descriptor.
#pragma once

#include "pf_common.hpp"

#include <type_traits>

namespace pf {

__device__ inline int mfma_src_row(int R, int t) {
  return 32 * ((R >> 2) & 1) + 16 * t + 4 * (R >> 3) + (R & 3);
}

template <int CPR>
__device__ inline int tile_swz(int row) {
  if constexpr (CPR >= 16) {
    return ((row & 3) << 2) | (((row >> 2) & 1) << 1) | ((row >> 5) & 1);
  } else {
    return (((row >> 1) & 1) << 2) | (((row >> 2) & 1) << 1) | ((row >> 5) & 1);
  }
}

template <typename T, int D>
struct Tile {
  static constexpr int ES = sizeof(T);
  static constexpr int EPC = 16 / ES;      // elements per 16-byte chunk
  static constexpr int CPR = D / EPC;      // chunks per row
  static constexpr int RB = D * ES;        // row bytes
  static constexpr int BYTES = 64 * RB;
  static constexpr bool TR = (ES == 2);
};

// Direct global -> LDS staging (dma16): lane l of a wave writes its 16 bytes
// at the instruction's LDS base + 16*l, so each lane fetches the global chunk
// that belongs at its slot of the swizzled tile. No registers hold the data
// and no LDS store instructions are issued; the issuing wave must wait for
// its loads (dma_wait) before the barrier that publishes the tile.
// NW = waves of the workgroup that share the staging (each lane issues
// PER_T = 64 * CPR / (64 * NW) loads per tile).
template <typename T, int D, int NW = 4>
struct TileDma {
  using G = Tile<T, D>;
  static constexpr int PER_T = G::CPR / NW;
  static_assert(PER_T >= 1 && G::CPR % NW == 0, "whole 16-byte slots per lane");
  uint32_t voff[PER_T];  // this lane's byte offset within the 64 rows
  uint32_t slot[PER_T];  // this wave's LDS byte offset within the tile (uniform)
  // Once per kernel: the lane offsets do not depend on the rows loaded.
  __device__ inline void init(int tid) {
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6), l = tid & 63;
#pragma unroll
    for (int u = 0; u < PER_T; ++u) {
      const int s = 64 * (NW * u + w) + l;  // 16-byte slot within the tile
      const int row = s / G::CPR, phys = s % G::CPR;
      const int chunk = phys ^ tile_swz<G::CPR>(row);
      voff[u] = (uint32_t)(row * D + chunk * G::EPC) * G::ES;
      slot[u] = 16 * 64 * (NW * u + w);
    }
  }
  // The descriptor of rows [row0, ...) of the buffer `desc` describes: base
  // moved forward and size shrunk (clamped at 0, so rows past the end still
  // load as zeros), with scalar arithmetic.
  __device__ static inline i32x4 at_row(const i32x4& desc, int row0) {
    const uint32_t off = (uint32_t)row0 * G::RB;
    const uint64_t base = (((uint64_t)(uint32_t)desc[1] << 32) | (uint32_t)desc[0]) + off;
    i32x4 d = desc;
    d[0] = (int)(uint32_t)base;
    d[1] = (int)(uint32_t)(base >> 32);
    d[2] = (uint32_t)desc[2] > off ? (int)((uint32_t)desc[2] - off) : 0;
    return d;
  }
  // The descriptor of rows [row0, ...) pinned for a burst of loads (dma_pin).
  __device__ static inline i32x4 pinned_at_row(const i32x4& desc, int row0) { return dma_pin(at_row(desc, row0)); }
  // Part u (of PER_T) of a tile load from a descriptor made by pinned_at_row:
  // callers that spread a tile's loads over a compute sequence issue the
  // parts one at a time.
  __device__ inline void load_part(const i32x4& d, int u, char* tile) const {
    dma16_pinned(d, voff[u], __builtin_amdgcn_readfirstlane(lds_u32(tile) + slot[u]));
  }
  // Rows [row0, row0 + 64) of the buffer `desc` describes.
  __device__ inline void load(const i32x4& desc, int row0, char* tile) const {
    const i32x4 d = pinned_at_row(desc, row0);
#pragma unroll
    for (int u = 0; u < PER_T; ++u) load_part(d, u, tile);
  }
};

// Wait for this wave's outstanding global loads (including LDS DMA). The
// builtin (vmcnt(0)), not inline assembly, so the compiler's wait tracking
// knows every earlier load has completed and adds no waits of its own later.
__device__ inline void dma_wait() { __builtin_amdgcn_s_waitcnt(0x0F70); }

// Natural A operand: s0/s1 (32x32 tiles t = 0, 1) += tile rows x B fragments,
// contracting over D (lane half hh owns columns [hh*D/2, (hh+1)*D/2)).
template <typename T, int D>
__device__ inline void mfma_nat(const char* tile, int l32, int hh, const typename Mfma32<T>::Frag* bf,
                                f32x16& s0, f32x16& s1) {
  using MF = Mfma32<T>;
  using G = Tile<T, D>;
  constexpr int FPC = frags_per_chunk<T>();
  const int r0 = mfma_src_row(l32, 0), r1 = mfma_src_row(l32, 1);
  const char* b0 = tile + r0 * G::RB;
  const char* b1 = tile + r1 * G::RB;
  const int sw0 = tile_swz<G::CPR>(r0), sw1 = tile_swz<G::CPR>(r1);
#pragma unroll
  for (int c = 0; c < G::CPR / 2; ++c) {
    const int ch = hh * (G::CPR / 2) + c;
    const u32x4 a0 = lds16(b0 + 16 * (ch ^ sw0));
    const u32x4 a1 = lds16(b1 + 16 * (ch ^ sw1));
#pragma unroll
    for (int f = 0; f < FPC; ++f) {
      s0 = MF::run(chunk_frag<T>(a0, f), bf[c * FPC + f], s0);
      s1 = MF::run(chunk_frag<T>(a1, f), bf[c * FPC + f], s1);
    }
  }
}

// Natural A operands of two tiles at once, one 32-row half t each:
// s += tile_a rows x bf_a and d += tile_b rows x bf_b (two independent MFMA
// chains, interleaved).
template <typename T, int D>
__device__ inline void mfma_nat_pair(const char* tile_a, const typename Mfma32<T>::Frag* bf_a,
                                     const char* tile_b, const typename Mfma32<T>::Frag* bf_b, int t,
                                     int l32, int hh, f32x16& s, f32x16& d) {
  using MF = Mfma32<T>;
  using G = Tile<T, D>;
  constexpr int FPC = frags_per_chunk<T>();
  const int r = mfma_src_row(l32, t);
  const int sw = tile_swz<G::CPR>(r);
  const char* ba = tile_a + r * G::RB;
  const char* bb = tile_b + r * G::RB;
#pragma unroll
  for (int c = 0; c < G::CPR / 2; ++c) {
    const int off = 16 * ((hh * (G::CPR / 2) + c) ^ sw);
    const u32x4 a = lds16(ba + off);
    const u32x4 b = lds16(bb + off);
#pragma unroll
    for (int f = 0; f < FPC; ++f) {
      s = MF::run(chunk_frag<T>(a, f), bf_a[c * FPC + f], s);
      d = MF::run(chunk_frag<T>(b, f), bf_b[c * FPC + f], d);
    }
  }
}

// Per-lane byte offsets for the transposed reads of a tile (16-bit types):
// off[dt][r] + (8c + 4r) * RB addresses the 8 bytes lane `lane` contributes to
// step c, half r of the 32-column block dt.
template <typename T, int D>
struct TrAddr {
  using G = Tile<T, D>;
  int off[D / 32][2];
  __device__ inline void init(int lane) {
    const int g = lane >> 4, j = lane & 15, hh = lane >> 5;
    const int a = j >> 2;                          // row within the 4-row group
    const int x = 2 * (g & 1) + ((j >> 1) & 1);    // chunk within the 4-chunk group
    const int q = G::CPR >= 16 ? 4 * a : 4 * (a >> 1);
#pragma unroll
    for (int dt = 0; dt < D / 32; ++dt)
#pragma unroll
      for (int r = 0; r < 2; ++r)
        off[dt][r] = (32 * hh + a) * G::RB + 8 * (j & 1) + 16 * (((4 * dt) ^ q) + (x ^ (2 * r + hh)));
  }
};

// 32x32x16 MFMA whose float32 accumulator lives in AGPRs (inline assembly:
// the "+a" constraint pins it there, where the allocator would otherwise copy
// it between the register files around every builtin MFMA once the VGPRs
// are full). Hazards the compiler cannot see inside the assembly, with the
// wait states this compiler's own gfx950 hazard model inserts for the
// builtins: a VALU write of an A/B operand needs 2 before the MFMA reads it
// -- the callers' operands are LDS reads and fragments packed several MFMA
// slots earlier, and a scan of the gfx950 assembly (tests/test_mfma_hazards.py)
// checks that no VALU write of an operand comes within 2 wait states, so no
// padding is issued; back-to-back MFMAs accumulating into the same
// registers need none; an LDS load of an operand is waited for by the
// compiler (it sees the operand). A VALU/memory read of the result needs 12
// after the last MFMA: agpr_fence() before the accumulator is read. The
// statement is not volatile (it touches no memory; data dependencies order
// it), so the compiler may still hoist LDS reads above it.
template <typename T>
struct MfmaAgpr;
template <>
struct MfmaAgpr<bf16_t> {
  __device__ static inline void run(f32x16& acc, bf16x8 a, bf16x8 b) {
    asm("v_mfma_f32_32x32x16_bf16 %0, %1, %2, %0" : "+a"(acc) : "v"(a), "v"(b));
  }
};
template <>
struct MfmaAgpr<f16_t> {
  __device__ static inline void run(f32x16& acc, f16x8 a, f16x8 b) {
    asm("v_mfma_f32_32x32x16_f16 %0, %1, %2, %0" : "+a"(acc) : "v"(a), "v"(b));
  }
};
// 16 wait states before the compiler may read an AGPR accumulator written by
// MfmaAgpr (tied to the accumulator so every read is ordered after it).
__device__ inline void agpr_fence(f32x16& acc) { asm volatile("s_nop 7\n\ts_nop 7" : "+a"(acc)); }

// Transposed A operand: acc[dt] += tile^T (rows = D columns of the tile,
// reduction over the tile's 64 rows) x B fragments. Lane half hh's B slots
// for step c are tile rows 32hh + 8c + [0, 8) (16-bit) or 32hh + s (f32).
// Steps [C0, C1) of 4 (16-bit: step c = tile rows 32hh + 8c + [0, 8); f32:
// rows 32hh + 8c .. 32hh + 8c + 7 as 8 single-row steps); bf is indexed by step.
// AGPR = true (16-bit T only): accumulate with MfmaAgpr. NA: the column
// blocks accumulated, the first NA of the tile (16-bit T may pass a tile
// pointer moved on by a multiple of 256 bytes for a later range of columns).
template <typename T, int D, int C0 = 0, int C1 = 4, bool AGPR = false, int NA = D / 32>
__device__ inline void mfma_trn(const char* tile, int lane, const TrAddr<T, D>& ta,
                                const typename Mfma32<T>::Frag* bf, f32x16* acc) {
  static_assert(NA >= 1 && NA <= D / 32, "column blocks of the tile");
  using MF = Mfma32<T>;
  using G = Tile<T, D>;
  using Frag = typename MF::Frag;
  if constexpr (G::TR) {
    typedef short v4i16 __attribute__((ext_vector_type(4)));
    // c outer, dt inner: consecutive MFMAs feed independent accumulators, so
    // none waits on the previous one's result.
#pragma unroll
    for (int c = C0; c < C1; ++c)
#pragma unroll
      for (int dt = 0; dt < NA; ++dt) {
        v4i16 part[2];
#pragma unroll
        for (int r = 0; r < 2; ++r)
          part[r] = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
              (__attribute__((address_space(3))) v4i16*)(tile + ta.off[dt][r] + (8 * c + 4 * r) * G::RB));
        const Frag af = __builtin_bit_cast(Frag, __builtin_shufflevector(part[0], part[1], 0, 1, 2, 3, 4, 5, 6, 7));
        if constexpr (AGPR) MfmaAgpr<T>::run(acc[dt], af, bf[c]);
        else acc[dt] = MF::run(af, bf[c], acc[dt]);
      }
  } else {
    const int l32 = lane & 31, hh = lane >> 5;
#pragma unroll
    for (int s = 8 * C0; s < 8 * C1; ++s) {
      const int row = 32 * hh + s;
#pragma unroll
      for (int dt = 0; dt < NA; ++dt) {
        const int d = 32 * dt + l32;
        const float a = *reinterpret_cast<const float*>(
            tile + row * G::RB + 16 * ((d >> 2) ^ tile_swz<G::CPR>(row)) + 4 * (d & 3));
        acc[dt] = MF::run(a, bf[s], acc[dt]);
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Interleaved (software-pipelined) MFMA sequences, 16-bit operands.
//
// The same products as mfma_nat / mfma_trn, issued together with a caller
// VALU stream: valu(i), i = 0 .. NV-1, runs beside the i-th MFMA (NV = number
// of MFMAs). Each fenced slot (sched_barrier) holds one or two MFMAs, their
// share of the VALU work and the LDS reads of the MFMAs LEAD slots ahead, so
// the MFMA pipe and the VALU stay busy together inside one wave and the LDS
// latency is hidden behind the MFMAs already issued. The VALU work must not
// depend on the MFMA results of the same sequence.
// ---------------------------------------------------------------------------

// s0/s1 += tile rows x bf (natural operand, as mfma_nat); NV = CPR (2 per chunk).
template <typename T, int D, int LEAD = 2, typename VF>
__device__ inline void mfma_nat_il(const char* tile, int l32, int hh, const typename Mfma32<T>::Frag* bf,
                                   f32x16& s0, f32x16& s1, VF&& valu) {
  using MF = Mfma32<T>;
  using G = Tile<T, D>;
  static_assert(sizeof(T) == 2, "16-bit operands");
  constexpr int NC = G::CPR / 2;
  const int r0 = mfma_src_row(l32, 0), r1 = mfma_src_row(l32, 1);
  const char* b0 = tile + r0 * G::RB;
  const char* b1 = tile + r1 * G::RB;
  const int sw0 = tile_swz<G::CPR>(r0), sw1 = tile_swz<G::CPR>(r1);
  u32x4 a0[NC], a1[NC];
#pragma unroll
  for (int c = 0; c < NC + LEAD; ++c) {
    if (c < NC) {
      const int ch = hh * NC + c;
      a0[c] = lds16(b0 + 16 * (ch ^ sw0));
      a1[c] = lds16(b1 + 16 * (ch ^ sw1));
    }
    if (c >= LEAD) {
      const int k = c - LEAD;
      s0 = MF::run(chunk_frag<T>(a0[k], 0), bf[k], s0);
      valu(2 * k);
      s1 = MF::run(chunk_frag<T>(a1[k], 0), bf[k], s1);
      valu(2 * k + 1);
    }
    __builtin_amdgcn_sched_barrier(0);
  }
}

// acc[dt] += tile^T x bf (transposed operand, as mfma_trn over all 4 steps);
// MFMA i = step c * NDT + dt, NV = 4 * NDT.
template <typename T, int D, int LEAD = 2, typename VF>
__device__ inline void mfma_trn_il(const char* tile, const TrAddr<T, D>& ta,
                                   const typename Mfma32<T>::Frag* bf, f32x16* acc, VF&& valu) {
  using MF = Mfma32<T>;
  using G = Tile<T, D>;
  using Frag = typename MF::Frag;
  static_assert(sizeof(T) == 2, "16-bit operands");
  typedef short v4i16 __attribute__((ext_vector_type(4)));
  constexpr int NDT = D / 32, NM = 4 * NDT;
  Frag af[NM];
#pragma unroll
  for (int i = 0; i < NM + LEAD; ++i) {
    if (i < NM) {
      const int c = i / NDT, dt = i % NDT;
      v4i16 part[2];
#pragma unroll
      for (int r = 0; r < 2; ++r)
        part[r] = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
            (__attribute__((address_space(3))) v4i16*)(tile + ta.off[dt][r] + (8 * c + 4 * r) * G::RB));
      af[i] = __builtin_bit_cast(Frag, __builtin_shufflevector(part[0], part[1], 0, 1, 2, 3, 4, 5, 6, 7));
    }
    if (i >= LEAD) {
      const int k = i - LEAD;
      acc[k % NDT] = MF::run(af[k], bf[k / NDT], acc[k % NDT]);
      valu(k);
    }
    __builtin_amdgcn_sched_barrier(0);
  }
}

// Two 16-bit values rounded from float32 (round to nearest even), packed low-first.
template <typename T>
__device__ inline uint32_t pack2(float a, float b) {
  typedef T v2 __attribute__((ext_vector_type(2)));
  const v2 x = {Elem<T>::from_f32(a), Elem<T>::from_f32(b)};
  return __builtin_bit_cast(uint32_t, x);
}

// Pack the 32 values a lane holds (tile t register r <-> reduction slot
// 16t + r of this lane half) into B-operand fragments.
template <typename T>
__device__ inline void pack_frags(const f32x16& s0, const f32x16& s1, typename Mfma32<T>::Frag* out) {
  using Frag = typename Mfma32<T>::Frag;
  if constexpr (sizeof(T) == 4) {
#pragma unroll
    for (int m = 0; m < 16; ++m) {
      out[m] = s0[m];
      out[16 + m] = s1[m];
    }
  } else {
#pragma unroll
    for (int f = 0; f < 4; ++f) {
      Frag x;
#pragma unroll
      for (int e = 0; e < 8; ++e) x[e] = Elem<T>::from_f32((f < 2 ? s0 : s1)[8 * (f & 1) + e]);
      out[f] = x;
    }
  }
}

// Load a lane's operand fragments for row `row` (lane half hh owns columns
// [hh*D/2, (hh+1)*D/2)); zeros when the row is out of range.
template <typename T, int D>
__device__ inline void load_row_frags(const T* src, int row, bool valid, int hh,
                                      typename Mfma32<T>::Frag* out) {
  constexpr int EPC = 16 / (int)sizeof(T);
  constexpr int FPC = frags_per_chunk<T>();
  const T* r = src + (int64_t)row * D + hh * (D / 2);
#pragma unroll
  for (int c = 0; c < D / 2 / EPC; ++c) {
    const u32x4 ch = valid ? ldg16(r + c * EPC) : (u32x4){0u, 0u, 0u, 0u};
#pragma unroll
    for (int f = 0; f < FPC; ++f) out[c * FPC + f] = chunk_frag<T>(ch, f);
  }
}

// Store a lane's accumulator column (32x32 tiles over D) scaled by `mul` to
// row `row` of a row-major [*, D] matrix of T.
template <typename T, int D>
__device__ inline void store_acc_row(T* dst_row, const f32x16* acc, float mul, int hh) {
#pragma unroll
  for (int dt = 0; dt < D / 32; ++dt)
#pragma unroll
    for (int r4 = 0; r4 < 4; ++r4) {
      const int d0 = 32 * dt + 8 * r4 + 4 * hh;
      float y[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) y[e] = acc[dt][4 * r4 + e] * mul;
      if constexpr (sizeof(T) == 4) {
        *reinterpret_cast<f32x4*>(dst_row + d0) = (f32x4){y[0], y[1], y[2], y[3]};
      } else {
        typedef T v4 __attribute__((ext_vector_type(4)));
        v4 x;
#pragma unroll
        for (int e = 0; e < 4; ++e) x[e] = Elem<T>::from_f32(y[e]);
        *reinterpret_cast<v4*>(dst_row + d0) = x;
      }
    }
}

}  // namespace pf
